"""GPU parity of the fp32 attention forward and backward on the fp32 matrix
instruction (v_mfma_f32_16x16x4_f32; csrc/attn_mfma_f32.hip).

fp32 operands, products and sums, as the reference's fp32 kernel computes
(forward.py:103,126,146 load every operand .to(tl.float32)). Bar: the fp32 bar
of test_gpu_attention.py, <= 1e-5 of max|ref| on o and L against the fp64
oracle; and against the fp32 tiled kernels (an independent fp32
implementation) on the same inputs. KAT_ATTN_IMPL=mfma pins the MFMA kernels
(a fallback is an error).
"""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from test_gpu_attention import _rel_max

pytestmark = pytest.mark.gpu
dev = "cuda"


def _inputs(seed, B, H, T, D):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g).to(dev) for _ in range(3)]


def _mask(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    km = (torch.rand(B, T, generator=g) > 0.3).to(torch.int32)
    km[:, 0] = 1
    if B > 1 and T > 80:
        km[1, 16:80] = 0  # a whole 64-key tile (and its 32-key halves) dropped
    return km


def _fwd(q, k, v, slopes, scale, mode, km):
    if mode == "causal":
        return F.rational_attention_forward(q, k, v, slopes, scale)
    from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg
    B, H, T, D = q.shape
    o = torch.empty_like(q)
    L = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    _attn_fwd_into(q, k, v, o, L, slopes, scale, mode != "noncausal", 1e-6,
                   _key_mask_arg(km, B, T, dev) if mode != "noncausal" else None, extended=True)
    return o, L


@pytest.mark.parametrize("mode", ["causal", "masked", "noncausal"])
@pytest.mark.parametrize("B,H,T,D", [(2, 3, 77, 64), (1, 2, 512, 64), (2, 2, 1000, 128),
                                     (1, 3, 300, 32), (2, 2, 200, 96), (1, 2, 130, 20),
                                     (1, 1, 1, 64), (2, 2, 257, 4), (1, 2, 190, 48),
                                     (2, 2, 333, 256), (1, 2, 200, 160), (1, 1, 1, 256)])
def test_fp32_mfma_forward_matches_oracle(gpu, B, H, T, D, mode, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    q, k, v = _inputs(7 * T + D, B, H, T, D)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    km = _mask(B, T, T + D) if mode == "masked" else None
    with torch.no_grad():
        o, L = _fwd(q, k, v, slopes.to(dev), scale, mode, km)
    torch.cuda.synchronize()
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, causal=mode != "noncausal", key_mask=km)
    assert _rel_max(o, ro) <= 1e-5, ("o", _rel_max(o, ro))
    assert _rel_max(L, rL) <= 1e-5, ("L", _rel_max(L, rL))
    # the tiled fp32 kernels on the same inputs
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    with torch.no_grad():
        o_t, L_t = _fwd(q, k, v, slopes.to(dev), scale, mode, km)
    assert _rel_max(o, o_t) <= 1e-5 and _rel_max(L, L_t) <= 1e-5


def test_fp32_mfma_config1_and_long(gpu, monkeypatch):
    # config 1 (B=2, H=12, S=512, D=64, slopes 2^(-8(i+1)/12)) and T = 4096 at
    # D = 128 (64 heads' worth of tiles on 2 heads), against the fp64 oracle
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    for (B, H, T, D, seed) in ((2, 12, 512, 64, 1), (1, 2, 4096, 128, 3)):
        q, k, v = _inputs(seed, B, H, T, D)
        slopes = torch.tensor([2.0 ** (-8.0 * (i + 1) / H) for i in range(H)], dtype=torch.float32)
        scale = 1.0 / math.sqrt(D)
        o, L = F.rational_attention_forward(q, k, v, slopes.to(dev), scale)
        torch.cuda.synchronize()
        ro, rL = O.attention_fwd(q, k, v, slopes, scale)
        assert _rel_max(o, ro) <= 1e-5, (T, _rel_max(o, ro))
        assert _rel_max(L, rL) <= 1e-5, (T, _rel_max(L, rL))
        assert float((o.cpu().double() - ro).abs().max()) < 1e-3  # tests.py:210


def test_fp32_strided_views_and_fallbacks(gpu, monkeypatch):
    # (b, h, t)-strided views (token-major [B, T, H, D]) take the MFMA kernel
    # and match the contiguous call bit for bit; a view whose rows are not
    # 16-byte aligned falls back to the tiled kernels (an error under
    # KAT_ATTN_IMPL=mfma); a head dim that is not a multiple of 4, or above
    # 256, runs the tiled kernels
    B, T, H, D = 2, 150, 3, 64
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, T, 3, H, D, generator=g).to(dev)
    q, k, v = x.permute(2, 0, 3, 1, 4)
    slopes = F.compute_alibi_slopes(H).to(dev)
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    o_s, L_s = F.rational_attention_forward(q, k, v, slopes, 0.125)
    o_c, L_c = F.rational_attention_forward(q.contiguous(), k.contiguous(), v.contiguous(), slopes, 0.125)
    assert torch.equal(o_s, o_c) and torch.equal(L_s, L_c)
    y = torch.randn(B, H, T, D + 1, generator=g).to(dev)[..., 1:]  # rows start 4 bytes in
    with pytest.raises(RuntimeError, match="fp32 MFMA"):
        F.rational_attention_forward(y, y, y, slopes, 0.125)
    monkeypatch.delenv("KAT_ATTN_IMPL")
    o_u, _ = F.rational_attention_forward(y, y, y, slopes, 0.125)
    ro, _ = O.attention_fwd(y, y, y, slopes.cpu(), 0.125)
    assert _rel_max(o_u, ro) <= 1e-5
    for Dt in (18, 260):
        z = torch.randn(1, 2, 70, Dt, generator=g).to(dev)
        o_z, _ = F.rational_attention_forward(z, z, z, slopes[:2], 1.0 / math.sqrt(Dt))
        ro, _ = O.attention_fwd(z, z, z, slopes[:2].cpu(), 1.0 / math.sqrt(Dt))
        assert _rel_max(o_z, ro) <= 1e-5, Dt


def _bwd(q, k, v, o, L, do, slopes, scale, mode, km):
    from fastalgebraictransformer_amd.backward import _attn_bwd_into
    from fastalgebraictransformer_amd.forward import _key_mask_arg
    B, H, T, D = q.shape
    g = [torch.full_like(q, float("nan")) for _ in range(3)]
    kmd = _key_mask_arg(km, B, T, dev) if km is not None else None
    _attn_bwd_into(q, k, v, o, L, do, *g, slopes, scale, mode != "noncausal", 1e-6, kmd,
                   extended=mode != "causal")
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("mode", ["causal", "masked", "noncausal"])
@pytest.mark.parametrize("B,H,T,D", [(2, 3, 77, 64), (1, 2, 512, 64), (2, 2, 600, 128),
                                     (1, 3, 300, 32), (2, 2, 200, 96), (1, 2, 130, 20),
                                     (1, 1, 1, 64), (2, 2, 257, 4), (1, 2, 190, 48),
                                     (2, 2, 333, 256), (1, 2, 200, 160), (1, 1, 1, 256)])
def test_fp32_mfma_backward_matches_oracle(gpu, B, H, T, D, mode, monkeypatch):
    # dq, dk, dv against the fp64 oracle's backward on the kernel's own (o, L)
    # at 1e-5 of max|ref|, and against the tiled fp32 kernels on the same
    # inputs; a dropped key's gradients are exactly 0
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    q, k, v = _inputs(11 * T + D, B, H, T, D)
    g = torch.Generator().manual_seed(17 * T + D)
    do = torch.randn(B, H, T, D, generator=g).to(dev)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    km = _mask(B, T, T + D) if mode == "masked" else None
    with torch.no_grad():
        o, L = _fwd(q, k, v, slopes.to(dev), scale, mode, km)
    got = _bwd(q, k, v, o, L, do, slopes.to(dev), scale, mode, km)
    ref = O.attention_bwd(q, k, v, o, L, do, slopes, scale, causal=mode != "noncausal", key_mask=km)
    for name, x, r in zip(("dq", "dk", "dv"), got, ref):
        assert bool(torch.isfinite(x).all()), name
        if T == 1 and name != "dv":
            # one key: dP - Delta = dO.v (1 - p) cancels to eps-level, so dq and dk
            # are rounding noise around ~0 and a bar relative to their max is void
            assert float((x.cpu().double() - r).abs().max()) <= 1e-5, name
            continue
        assert _rel_max(x, r) <= 1e-5, (name, _rel_max(x, r))
    if km is not None:
        dropped = (km == 0).to(dev)[:, None, :, None].expand(B, H, T, D)
        assert int(torch.count_nonzero(got[1][dropped])) == 0
        assert int(torch.count_nonzero(got[2][dropped])) == 0
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    tiled = _bwd(q, k, v, o, L, do, slopes.to(dev), scale, mode, km)
    for name, x, t in zip(("dq", "dk", "dv"), got, tiled):
        if T > 1 or name == "dv":
            assert _rel_max(x, t) <= 1e-5, (name, _rel_max(x, t))


def test_fp32_mfma_training_step_config1(gpu, monkeypatch):
    # config 1's shape through autograd (fwd + bwd), both on the fp32 MFMA
    # kernels, against the fp64 oracle (tests.py:210-211 bars and 1e-5 of max)
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T, D = 2, 12, 512, 64
    q, k, v = _inputs(1, B, H, T, D)
    g = torch.Generator().manual_seed(2)
    do = torch.randn(B, H, T, D, generator=g).to(dev)
    slopes = torch.tensor([2.0 ** (-8.0 * (i + 1) / H) for i in range(H)], dtype=torch.float32)
    scale = 1.0 / math.sqrt(D)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = F.rational_attention(qq, kk, vv, slopes.to(dev), scale)
    o.backward(do)
    torch.cuda.synchronize()
    ro, rL = O.attention_fwd(q, k, v, slopes, scale)
    rq, rk, rv = O.attention_bwd(q, k, v, ro, rL, do, slopes, scale)
    assert _rel_max(o, ro) <= 1e-5
    for name, x, r in (("dq", qq.grad, rq), ("dk", kk.grad, rk), ("dv", vv.grad, rv)):
        assert _rel_max(x, r) <= 1e-5, (name, _rel_max(x, r))
        assert float((x.cpu().double() - r).abs().max()) < 1e-2  # tests.py:211
