"""A seeded random sweep of attention shapes against the oracle: sequence
lengths that are not multiples of the kernels' tiles, head dims 32 / 64 / 128
(bf16 / fp16 and fp32 on the MFMA kernels), 1 to 16
heads, bf16 / fp16 / fp32, causal or with a padding mask or non-causal; and a
second sweep over head dims between the layout widths (multiples of 8 up to
256, which the MFMA kernels of the next width run with the columns past D
read as zeros and not stored), and one over fp32 head dims (multiples of 4
up to 256) pinned to the fp32 MFMA kernels. The draws are fixed (seeds below), so a
failure names a reproducible case. Bars as in test_gpu_attention.py: fp32 <=
1e-5 of max|ref|; bf16 / fp16 2e-2 + 1/2 ulp elementwise and relative L2 <=
5e-3."""

import math
import random

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import check_lowp, max_abs

pytestmark = pytest.mark.gpu
dev = "cuda"


def _draw(n, seed=2024, dims=(32, 64, 128), dtypes=("bf16", "bf16", "fp16", "fp32")):
    rnd = random.Random(seed)
    cases = []
    for i in range(n):
        dtype = rnd.choice(dtypes)
        D = rnd.choice(dims)
        H = rnd.choice([1, 3, 12, 16])
        B = rnd.choice([1, 2])
        T = rnd.randrange(1, 600)
        mode = rnd.choice(["causal", "causal", "masked", "noncausal"])
        cases.append((i, dtype, B, H, T, D, mode))
    return cases


@pytest.mark.parametrize("i,dtype,B,H,T,D,mode", _draw(24))
def test_random_shape(gpu, i, dtype, B, H, T, D, mode):
    _check_case(i, dtype, B, H, T, D, mode)


_PADDED_DIMS = (8, 16, 24, 40, 48, 56, 72, 80, 96, 104, 112, 120, 136, 160, 192, 200, 224, 248)


@pytest.mark.parametrize("i,dtype,B,H,T,D,mode",
                         _draw(20, seed=77, dims=_PADDED_DIMS, dtypes=("bf16", "fp16")))
def test_random_shape_padded_head_dim(gpu, i, dtype, B, H, T, D, mode, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")  # a fallback to the tiled kernels is an error
    _check_case(100 + i, dtype, B, H, T, D, mode)


_FP32_DIMS = (4, 12, 20, 32, 44, 64, 76, 96, 128, 140, 200, 256)


@pytest.mark.parametrize("i,dtype,B,H,T,D,mode", _draw(16, seed=303, dims=_FP32_DIMS, dtypes=("fp32",)))
def test_random_shape_fp32_mfma(gpu, i, dtype, B, H, T, D, mode, monkeypatch):
    # fp32 head dims (multiples of 4 up to 256) on the fp32 MFMA kernels
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    _check_case(200 + i, dtype, B, H, T, D, mode)


def _check_case(i, dtype, B, H, T, D, mode):
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    g = torch.Generator().manual_seed(1000 + i)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to(dt).to(dev) for _ in range(4))
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    km, causal = None, mode != "noncausal"
    if mode == "masked":
        km = (torch.rand(B, T, generator=g) > 0.25).to(torch.int32)
        km[:, 0] = 1
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    if mode == "causal":
        o = F.rational_attention(qq, kk, vv, slopes.to(dev), scale)
    else:
        o = F.rational_attention_masked(qq, kk, vv, slopes.to(dev), scale,
                                        key_mask=None if km is None else km.to(dev), causal=causal)
    o.backward(do)
    torch.cuda.synchronize()
    # the oracle in fp64 for fp32 inputs (a truth below both fp32
    # implementations' rounding), in fp32 for the 16-bit ones
    odt = torch.float64 if dt == torch.float32 else torch.float32
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=odt, causal=causal, key_mask=km)
    rq, rk, rv = O.attention_bwd(q, k, v, o, rL, do, slopes, scale, dtype=odt,
                                 causal=causal, key_mask=km)
    for name, got, ref in (("o", o, ro), ("dq", qq.grad, rq), ("dk", kk.grad, rk),
                           ("dv", vv.grad, rv)):
        if dt == torch.float32:
            assert max_abs(got, ref) <= 1e-5 * max(1e-30, float(ref.abs().max())), name
        else:
            check_lowp(got, ref, dt, name)
