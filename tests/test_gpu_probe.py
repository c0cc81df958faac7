"""The MFMA throughput probes bench.py uses (kat_probe_mfma_bf16 and
kat_probe_mfma_bf16_random)."""

import ctypes

import pytest
import torch

from fastalgebraictransformer_amd import _lib

pytestmark = pytest.mark.gpu


def test_probe_mfma_runs_and_counts_flops(gpu):
    lib = _lib.load()
    out = torch.empty(4 * 256, dtype=torch.float32, device="cuda")
    flops = ctypes.c_double(0.0)
    rc = lib.kat_probe_mfma_bf16(ctypes.c_void_p(out.data_ptr()), 4, 10, ctypes.byref(flops),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0
    # 4 blocks x 4 waves x 10 iterations x 16 MFMAs x (16 x 16 x 32 x 2) flops
    assert flops.value == 4 * 4 * 10 * 16 * 16 * 16 * 32 * 2
    assert bool(torch.isfinite(out).all())


def test_probe_random_operands_runs_and_counts_flops(gpu):
    lib = _lib.load()
    out = torch.full((4 * 512,), float("nan"), dtype=torch.float32, device="cuda")
    flops = ctypes.c_double(0.0)
    rc = lib.kat_probe_mfma_bf16_random(ctypes.c_void_p(out.data_ptr()), 4, 10, ctypes.byref(flops),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0
    # 4 blocks x 8 waves x 10 iterations x 16 MFMAs x (16 x 16 x 32 x 2) flops
    assert flops.value == 4 * 8 * 10 * 16 * 16 * 16 * 32 * 2
    assert bool(torch.isfinite(out).all())


def test_probe_rejects_bad_arguments():
    lib = _lib.load()
    flops = ctypes.c_double(0.0)
    assert lib.kat_probe_mfma_bf16(None, 4, 10, ctypes.byref(flops), None) != 0
    assert lib.kat_probe_mfma_bf16_random(None, 4, 10, ctypes.byref(flops), None) != 0


def test_launch_stream_is_the_current_torch_stream(gpu):
    # every libkat call is queued on torch's current stream of the tensor's
    # device (the raw-pointer query in _lib.stream), also inside a
    # torch.cuda.stream(...) block
    x = torch.empty(1, device="cuda")
    assert (_lib.stream(x).value or 0) == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert (_lib.stream(x).value or 0) == s.cuda_stream
    assert (_lib.stream(x).value or 0) == torch.cuda.current_stream().cuda_stream
