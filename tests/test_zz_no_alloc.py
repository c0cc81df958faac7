"""kat_attn_decode_noalloc (partials in the library's fixed device array)
against kat_attn_decode (partials in a caller workspace): same kernels, so
outputs and L must agree bit for bit, on consecutive calls of decreasing size
(the array keeps the previous call's contents, which must not leak), and an
oversized call must fail cleanly with KAT_EUNSUPPORTED before any launch."""

import ctypes
import math

import pytest
import torch

import fastalgebraictransformer_amd as F
from fastalgebraictransformer_amd import _lib

pytestmark = pytest.mark.gpu


def _case(B, H, T, D, dtype, seed, ragged):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g).to(dtype).cuda()
    # token-major caches [B, T, H, D], read through (b, h, t) strides
    kc = torch.randn(B, T, H, D, generator=g).to(dtype).cuda().permute(0, 2, 1, 3)
    vc = torch.randn(B, T, H, D, generator=g).to(dtype).cuda().permute(0, 2, 1, 3)
    lengths = None
    if ragged:
        lengths = torch.randint(0, T + 1, (B,), generator=g, dtype=torch.int32).cuda()
    return q, kc, vc, F.compute_alibi_slopes(H).cuda(), 1.0 / math.sqrt(D), lengths


def _call(noalloc, q, kc, vc, slopes, scale, lengths, raw=False):
    lib = _lib.load()
    B, H, D = q.shape
    T = kc.shape[2]
    out = torch.full((B, H, D), float("nan"), dtype=q.dtype, device="cuda")
    L = torch.full((B, H), float("nan"), dtype=torch.float32, device="cuda")
    code = _lib.dtype_code(q)
    strides = _lib.i64_array((q.stride(0), q.stride(1), kc.stride(0), kc.stride(1), kc.stride(2),
                              vc.stride(0), vc.stride(1), vc.stride(2), out.stride(0), out.stride(1)))
    lp = None if lengths is None else lengths.data_ptr()
    st = _lib.stream(q)
    if noalloc:
        rc = lib.kat_attn_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                         L.data_ptr(), slopes.data_ptr(), lp, B, H, T, D, strides,
                                         scale, 1e-6, code, st)
    else:
        nbytes = lib.kat_attn_decode_workspace_size(B, H, T, D, code)
        ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device="cuda")
        rc = lib.kat_attn_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                 L.data_ptr(), slopes.data_ptr(), lp, ws.data_ptr(), nbytes, B, H, T,
                                 D, strides, scale, 1e-6, code, st)
    if raw:
        return rc
    _lib.check(rc, "decode")
    torch.cuda.synchronize()
    return out, L


@pytest.mark.parametrize("first,second", [
    ((16, 16, 4096, 128, torch.bfloat16, False), (2, 4, 700, 64, torch.bfloat16, True)),
    ((4, 8, 3000, 256, torch.float16, True), (1, 2, 33, 32, torch.float32, False)),
])
def test_noalloc_decode_matches_workspace_decode(gpu, first, second):
    for i, (B, H, T, D, dt, ragged) in enumerate((first, second)):
        args = _case(B, H, T, D, dt, 100 + i, ragged)
        nbytes = _lib.load().kat_attn_decode_workspace_size(B, H, T, D, _lib.dtype_code(args[0]))
        assert 0 < nbytes <= 8 << 20
        o_ref, l_ref = _call(False, *args)
        o_na, l_na = _call(True, *args)
        assert torch.equal(o_na, o_ref), (i, B, H, T, D)
        assert torch.equal(l_na, l_ref), (i, B, H, T, D)
        assert bool(torch.isfinite(o_na).all())


def test_noalloc_decode_rejects_more_than_its_array(gpu):
    # B*H*splits*(D+1) floats beyond 8 MiB: 128 x 128 (b, h) pairs at D = 128
    # take one split each, 16384 x 129 x 4 bytes = 8.06 MiB
    B, H, T, D = 128, 128, 16, 128
    q, kc, vc, slopes, scale, _ = _case(B, H, T, D, torch.bfloat16, 7, False)
    assert _lib.load().kat_attn_decode_workspace_size(B, H, T, D, 1) > 8 << 20
    assert _call(True, q, kc, vc, slopes, scale, None, raw=True) == 2  # KAT_EUNSUPPORTED
    assert "scratch array" in _lib.load().kat_last_error().decode()
    with pytest.raises(RuntimeError, match="scratch array"):
        _call(True, q, kc, vc, slopes, scale, None)
    # and the workspace entry point still serves it
    o, L = _call(False, q, kc, vc, slopes, scale, None)
    assert bool(torch.isfinite(o).all())
