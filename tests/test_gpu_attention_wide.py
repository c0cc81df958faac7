"""GPU parity of the tiled attention kernels beyond the MFMA path -- fp64
tensors and head dims above 256 (up to 1024) -- and of the MFMA kernels at
head dim 256.

The reference takes any float dtype -- its kernels load with
``.to(tl.float32)`` and store in the input dtype (forward.py:103,155) -- and
any head dim (BLOCK_D = next_pow2(D), forward.py:297-301). Here fp64 tensors
keep fp64 arithmetic (as the row ops do), so fp64 gradient checks hold; L is
fp32 as in the reference (forward.py:294).

Tolerances (written beside each check):
  * fp64: <= 1e-10 of max|ref| against the fp64 oracle on the same inputs,
    with the kernel's own (fp32) L passed to the oracle's backward. The C ABI
    takes scale and eps as fp32 (the reference hands them to its kernels as
    fp32 scalars too), so the oracle takes the same fp32-rounded scale;
  * fp32: <= 1e-5 of max|ref|, the fp32 bar of test_gpu_attention.py;
  * bf16: the low-precision bar (check_lowp: 2e-2 + 1/2 ulp elementwise,
    relative L2 <= 5e-3).
"""

import math

import numpy as np
import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import check_lowp, max_abs

pytestmark = pytest.mark.gpu
dev = "cuda"


def _inputs(seed, B, H, T, D, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(dtype).to(dev)
            for _ in range(4)]


def _scale32(D):
    # 1 / sqrt(D) as the fp32 scalar the kernels receive
    return float(np.float32(1.0 / math.sqrt(D)))


def _rel(got, ref):
    return max_abs(got, ref) / max(1e-300, float(ref.detach().abs().max()))


def _run(q, k, v, do, slopes, scale, key_mask=None, causal=True):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    if key_mask is None and causal:
        out = F.rational_attention(q, k, v, slopes, scale)
        o, L = F.rational_attention_forward(q.detach(), k.detach(), v.detach(), slopes, scale)
        assert torch.equal(out.detach(), o)
    else:
        out = F.rational_attention_masked(q, k, v, slopes, scale, key_mask=key_mask,
                                          causal=causal)
        o, L = None, None
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), L, q.grad, k.grad, v.grad


@pytest.mark.parametrize("B,H,T,D", [(2, 3, 97, 64), (1, 2, 130, 128), (1, 2, 70, 256)])
def test_fp64_matches_oracle(gpu, B, H, T, D):
    q, k, v, do = _inputs(7 + D, B, H, T, D, torch.float64)
    slopes = F.compute_alibi_slopes(H)
    scale = _scale32(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    assert o.dtype == torch.float64 and dq.dtype == torch.float64 and L.dtype == torch.float32
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float64)
    assert _rel(o, ro) <= 1e-10, _rel(o, ro)
    assert _rel(L, rL) <= 1e-7  # L is stored in fp32
    # the backward takes L as stored (fp32), as the reference's does
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float64)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert got.dtype == torch.float64
        assert _rel(got, ref) <= 1e-10, (name, _rel(got, ref))


def test_fp64_masked_noncausal_matches_oracle(gpu):
    B, H, T, D = 2, 2, 90, 48
    q, k, v, do = _inputs(31, B, H, T, D, torch.float64)
    slopes = F.compute_alibi_slopes(H)
    scale = _scale32(D)
    km = torch.ones(B, T, dtype=torch.int32)
    km[0, :17] = 0
    km[1, 3::4] = 0
    for causal in (True, False):
        o, _, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale, key_mask=km, causal=causal)
        ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float64, causal=causal,
                                 key_mask=km)
        assert _rel(o, ro) <= 1e-10, (causal, _rel(o, ro))
        # the oracle's backward on its own fp64 L: the kernel's L (fp32) moves
        # p by ~6e-8 relative, so this comparison takes 1e-6
        rq, rk, rv = O.attention_bwd(q, k, v, ro, rL, do, slopes, scale, dtype=torch.float64,
                                     causal=causal, key_mask=km)
        for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
            assert _rel(got, ref) <= 1e-6, (causal, name, _rel(got, ref))


def test_fp64_gradcheck(gpu):
    # finite differences of the fp64 forward against the analytic backward
    # (gradcheck's default tolerances; the fp32 L perturbs p by ~6e-8)
    B, H, T, D = 1, 2, 12, 8
    q, k, v, _ = _inputs(3, B, H, T, D, torch.float64)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = _scale32(D)
    assert torch.autograd.gradcheck(lambda a, b, c: F.rational_attention(a, b, c, slopes, scale),
                                    (q, k, v), eps=1e-6, atol=1e-6, rtol=1e-4)


@pytest.mark.parametrize("D", [257, 320, 512, 640, 1024])
def test_wide_head_dims_fp32(gpu, D):
    B, H, T = 1, 2, 75
    q, k, v, do = _inputs(D, B, H, T, D, torch.float32)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float64)
    assert _rel(o, ro) <= 1e-5 and _rel(L, rL) <= 1e-5, (_rel(o, ro), _rel(L, rL))
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float64)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert _rel(got, ref) <= 1e-5, (D, name, _rel(got, ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_head_dim_lowp(gpu, dtype):
    B, H, T, D = 1, 3, 140, 512
    q, k, v, do = _inputs(11, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    with pytest.warns(RuntimeWarning, match="head dim 512"):
        o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    assert o.dtype == dtype and dq.dtype == dtype
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
    check_lowp(o, ro, dtype, "o")
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        check_lowp(got, ref, dtype, name)


def test_wide_head_dim_masked_noncausal_fp32(gpu):
    B, H, T, D = 2, 2, 100, 384
    q, k, v, do = _inputs(5, B, H, T, D, torch.float32)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    km = torch.ones(B, T, dtype=torch.int32)
    km[0, 60:] = 0
    km[1, ::3] = 0
    for causal in (True, False):
        o, _, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale, key_mask=km, causal=causal)
        ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float64, causal=causal,
                                 key_mask=km)
        assert _rel(o, ro) <= 1e-5, (causal, _rel(o, ro))
        rq, rk, rv = O.attention_bwd(q, k, v, ro, rL, do, slopes, scale, dtype=torch.float64,
                                     causal=causal, key_mask=km)
        for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
            assert _rel(got, ref) <= 1e-5, (causal, name, _rel(got, ref))


def test_head_dim_above_1024_is_rejected(gpu):
    q = torch.zeros(1, 1, 4, 1040, device=dev)
    with pytest.raises(RuntimeError, match="head dim 1040 > 1024"):
        F.rational_attention_forward(q, q, q, torch.ones(1, device=dev), 1.0)


# ------------------------------------------------------ MFMA at D = 256 ----
# The MFMA kernels also cover D = 256: the forward in 8-wave blocks of
# 16-query waves, the backward with 16 keys per dK/dV wave pair and 32 queries
# per dQ wave (the backward's parity cases at D = 256 sit with the other head
# dims in test_gpu_attention.py). Bar: check_lowp on o and the gradients (the
# north-star 2e-2 max-abs + 1/2 ulp, relative L2 <= 5e-3), L within 1e-2.

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 77, 300, 1025])
def test_mfma_forward_d256(gpu, dtype, T, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")  # fail instead of falling back
    B, H, D = 2, 3, 256
    q, k, v, _ = _inputs(17 + T, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L = F.rational_attention_forward(q, k, v, slopes.to(dev), scale)
    torch.cuda.synchronize()
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
    check_lowp(o, ro, dtype, "o")
    assert _rel(L, rL) <= 1e-2, _rel(L, rL)


@pytest.mark.parametrize("causal", [True, False])
def test_mfma_forward_d256_masked(gpu, causal, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T, D = 2, 2, 333, 256
    q, k, v, _ = _inputs(23, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    km = torch.ones(B, T, dtype=torch.int32)
    km[0, 200:] = 0
    km[1, 5::7] = 0
    km[1, 64:128] = 0  # a whole key tile dropped
    with torch.no_grad():
        o = F.rational_attention_masked(q, k, v, slopes.to(dev), scale, key_mask=km, causal=causal)
    torch.cuda.synchronize()
    ro, _ = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32, causal=causal, key_mask=km)
    check_lowp(o, ro, torch.bfloat16, "o")


def test_mfma_forward_d256_long_matches_tiled(gpu, monkeypatch):
    # T = 4096 (the config-3 length): MFMA forward against the fp32 tiled
    # kernels on the same bf16 inputs
    B, H, T, D = 1, 2, 4096, 256
    q, k, v, _ = _inputs(29, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(8)[4:6].to(dev)
    scale = 1.0 / math.sqrt(D)
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    o_m, L_m = F.rational_attention_forward(q, k, v, slopes, scale)
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    o_t, L_t = F.rational_attention_forward(q.float(), k.float(), v.float(), slopes, scale)
    torch.cuda.synchronize()
    check_lowp(o_m, o_t, torch.bfloat16, "o")
    assert _rel(L_m, L_t) <= 1e-3


def test_d256_training_step_on_the_mfma_kernels(gpu, monkeypatch):
    # fwd + bwd through autograd at D = 256, both on the MFMA kernels (no
    # fallback warning); gradients against the oracle at the bf16 bar
    import warnings
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T, D = 1, 2, 200, 256
    q, k, v, do = _inputs(37, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        o, _, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
    check_lowp(o, ro, torch.bfloat16, "o")
    rq, rk, rv = O.attention_bwd(q, k, v, o, rL, do, slopes, scale, dtype=torch.float32)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        check_lowp(got, ref, torch.bfloat16, name)


@pytest.mark.parametrize("D", [256, 160, 96])
@pytest.mark.parametrize("causal", [True, False])
def test_mfma_backward_masked_wide_and_between(gpu, D, causal, monkeypatch):
    # padding mask (a whole key tile and a whole 16-key half dropped), causal
    # and not, against the oracle's masked backward: D = 256, and head dims
    # that run the layout widths 256 / 128 with narrower MFMA loops
    from fastalgebraictransformer_amd.backward import _attn_bwd_into
    from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T = 2, 2, 333
    q, k, v, do = _inputs(61, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    m = torch.ones(B, T, dtype=torch.int32)
    m[0, 200:] = 0
    m[1, 5::7] = 0
    m[1, 64:128] = 0
    m[1, 144:160] = 0
    km = _key_mask_arg(m, B, T, dev)
    o = torch.empty_like(q)
    L = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    _attn_fwd_into(q, k, v, o, L, slopes.to(dev), scale, causal, 1e-6, km, extended=True)
    g = [torch.full_like(q, float("nan")) for _ in range(3)]
    _attn_bwd_into(q, k, v, o, L, do, *g, slopes.to(dev), scale, causal, 1e-6, km, extended=True)
    torch.cuda.synchronize()
    ro, _ = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32, causal=causal, key_mask=m)
    check_lowp(o, ro, torch.bfloat16, "o")
    rg = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32, causal=causal,
                         key_mask=m)
    for name, got, ref in zip(("dq", "dk", "dv"), g, rg):
        check_lowp(got, ref, torch.bfloat16, name)


def test_mfma_backward_d256_long_matches_tiled(gpu, monkeypatch):
    # T = 4096: the MFMA backward against the fp32 tiled kernels on the same
    # bf16 inputs (an independent implementation), at the bf16 bar
    B, H, T, D = 1, 2, 4096, 256
    q, k, v, do = _inputs(67, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(8)[2:4].to(dev)
    scale = 1.0 / math.sqrt(D)
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    o, L = F.rational_attention_forward(q, k, v, slopes, scale)
    g_m = F.rational_attention_backward(q, k, v, o, L, do, slopes, scale)
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    f32 = [t.float() for t in (q, k, v, do)]
    g_t = F.rational_attention_backward(f32[0], f32[1], f32[2], o.float(), L, f32[3], slopes, scale)
    torch.cuda.synchronize()
    for name, x, y in zip(("dq", "dk", "dv"), g_m, g_t):
        check_lowp(x, y, torch.bfloat16, name)
