"""GPU parity of rational attention (forward and backward) against the CPU
oracle. Tolerances (written next to each check):
  * fp32 (tiled fp32 kernels): <= 1e-5 of max|ref| on outputs and gradients;
    the reference bars (tests.py:210-211) are 1e-3 / 1e-2 max-abs;
  * bf16 / fp16 (MFMA kernels, fp32 accumulation): 2e-2 max-abs on o, dq,
    dk, dv on top of the output's own rounding:
    elementwise |got - ref| <= 2e-2 + 1/2 ulp(ref) of the output dtype (the
    outputs are stored in the input dtype, as the reference does, and for
    |x| >= 4 half a bf16 ulp alone is >= 1.6e-2), plus a relative L2 error
    <= 5e-3 per tensor (check_lowp). L (fp32) within 1e-2 relative.
"""

import math
import os

import numpy as np
import pytest
import torch

import fastalgebraictransformer_amd as F
from fastalgebraictransformer_amd import _lib
import oracle as O
from _util import check_lowp, golden, lowp_ulp, max_abs

pytestmark = pytest.mark.gpu
dev = "cuda"


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.asarray(a)).to(dev, dtype)


def _inputs(seed, B, H, T, D, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g).to(dtype).to(dev) for _ in range(4)]


def _run(q, k, v, do, slopes, scale):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o, L = F.rational_attention_forward(q, k, v, slopes, scale)
    out = F.rational_attention(q, k, v, slopes, scale)
    assert torch.equal(out, o)
    out.backward(do)
    torch.cuda.synchronize()
    return o, L, q.grad, k.grad, v.grad


def _rel_max(a, b):
    return max_abs(a, b) / max(1e-30, float(b.detach().abs().max()))


def _ulp(ref, dtype):
    return lowp_ulp(ref, dtype)


def assert_lowp(got, ref, dtype, name, bar=2e-2):
    """check_lowp: |got - ref| <= bar + 1/2 ulp_dtype(ref) elementwise, and
    relative L2 <= 5e-3."""
    return check_lowp(got, ref, dtype, name, bar=bar)


# ----------------------------------------------------------------- fp32 ----

def test_golden_fp32(gpu):
    z = golden("attn_f32")
    q, k, v, do = (_t(z[n]) for n in ("q", "k", "v", "do"))
    o, L, dq, dk, dv = _run(q, k, v, do, _t(z["slopes"]), float(z["scale"]))
    for name, got in (("o", o), ("L", L), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert _rel_max(got, torch.from_numpy(z[name])) <= 1e-5, name


def test_config1_fp32(gpu):
    # B=2, H=12, S=512, D=64 fp32; scale 1/8; slopes 2^(-8(i+1)/12)
    B, H, T, D = 2, 12, 512, 64
    q, k, v, do = _inputs(1, B, H, T, D, torch.float32)
    slopes = torch.tensor([2.0 ** (-8.0 * (i + 1) / H) for i in range(H)], dtype=torch.float32)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale)
    assert _rel_max(o, ro) <= 1e-5 and _rel_max(L, rL) <= 1e-5
    assert max_abs(o, ro) < 1e-3  # tests.py:210
    rq, rk, rv = O.attention_bwd(q, k, v, o.detach(), L, do, slopes, scale)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert max_abs(got, ref) < 1e-2, name  # tests.py:211
        assert _rel_max(got, ref) <= 1e-5, name


@pytest.mark.parametrize("B,H,T,D", [(1, 4, 32, 32), (2, 8, 64, 64), (1, 4, 128, 32),
                                     (1, 3, 33, 20), (1, 2, 300, 160)])
def test_reference_shapes_fp32(gpu, B, H, T, D):
    # tests.py:183 shapes (+ ragged T / odd D), slopes from compute_alibi_slopes
    q, k, v, do = _inputs(T + D, B, H, T, D, torch.float32)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale)
    rq, rk, rv = O.attention_bwd(q, k, v, o.detach(), L, do, slopes, scale)
    assert _rel_max(o, ro) <= 1e-5 and _rel_max(L, rL) <= 1e-5
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert _rel_max(got, ref) <= 1e-5, name


# ------------------------------------------------------------ bf16 / fp16 ----

def _check_lowp(o, L, dq, dk, dv, q, k, v, do, slopes, scale, sel=None, chunk=None):
    """Compare against the fp32-upcast oracle on the same (rounded) inputs;
    ``sel`` restricts the oracle to one (b, h) pair. Returns the achieved
    (max error, relative L2) per output."""
    if sel is not None:
        b, h = sel
        q, k, v, do = (t[b:b + 1, h:h + 1] for t in (q, k, v, do))
        o, L, dq, dk, dv = (t[b:b + 1, h:h + 1] for t in (o, L, dq, dk, dv))
        slopes = slopes[h:h + 1]
    dt = q.dtype
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32, chunk=chunk)
    res = {"o": assert_lowp(o, ro, dt, "o")}
    assert _rel_max(L, rL) <= 1e-2, ("L", _rel_max(L, rL))
    # backward from the GPU forward's own O and L, as the autograd path does
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32, chunk=chunk)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        res[name] = assert_lowp(got, ref, dt, name)
    return res


def _pin_mfma(monkeypatch, D):
    # bf16 / fp16 calls whose head dim the MFMA kernels cover (multiples of 8
    # up to 256) must run on them: with KAT_ATTN_IMPL=mfma a fallback to the
    # tiled kernels is an error
    if D % 8 == 0 and D <= 256:
        monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")


@pytest.mark.parametrize("name", ["attn_bf16_d64", "attn_bf16_d128"])
def test_golden_bf16(gpu, name, monkeypatch):
    z = golden(name)
    _pin_mfma(monkeypatch, z["q"].shape[-1])
    q, k, v, do = (_t(z[n], torch.bfloat16) for n in ("q", "k", "v", "do"))
    o, L, dq, dk, dv = _run(q, k, v, do, _t(z["slopes"]), float(z["scale"]))
    assert_lowp(o, torch.from_numpy(z["o"]), torch.bfloat16, "o (fixture)")
    _check_lowp(o, L, dq, dk, dv, q, k, v, do, _t(z["slopes"]).cpu(), float(z["scale"]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,T,D", [(1, 2, 64, 64), (1, 3, 200, 128), (2, 2, 333, 64),
                                     (1, 2, 257, 32), (2, 3, 1000, 32), (1, 1, 1, 32),
                                     (1, 1, 1, 128), (1, 2, 1000, 128), (1, 2, 200, 256),
                                     (2, 2, 333, 256), (1, 1, 1, 256), (1, 2, 1000, 256),
                                     (1, 3, 200, 96), (2, 2, 333, 80), (1, 2, 300, 48),
                                     (1, 2, 257, 192), (1, 1, 1, 96), (2, 2, 100, 24),
                                     (1, 2, 257, 120), (1, 2, 300, 160), (1, 2, 200, 224),
                                     (1, 2, 130, 248)])
def test_lowp_shapes(gpu, dtype, B, H, T, D, monkeypatch):
    _pin_mfma(monkeypatch, D)
    q, k, v, do = _inputs(7 * T + D, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    _check_lowp(o, L, dq, dk, dv, q, k, v, do, slopes, scale)


def test_config3_bf16_all_heads(gpu, monkeypatch):
    # B=4, H=16, S=4096, D=128 bf16; slopes 2^(-(i+1)/2): every (b, h) head
    # against the fp32 oracle (two heads per oracle pass bound its memory)
    B, H, T, D = 4, 16, 4096, 128
    _pin_mfma(monkeypatch, D)
    q, k, v, do = _inputs(3, B, H, T, D, torch.bfloat16)
    slopes = torch.tensor([2.0 ** (-(i + 1) / 2) for i in range(H)], dtype=torch.float32)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    for t in (o, L, dq, dk, dv):
        assert bool(torch.isfinite(t).all())
    res = _check_lowp(o, L, dq, dk, dv, q, k, v, do, slopes, scale, chunk=2)
    print("config 3, all 64 heads: " + ", ".join(
        f"{n} max err {e:.3e} relL2 {r:.3e}" for n, (e, r) in res.items()))


def test_mfma_matches_tiled_kernel(gpu, monkeypatch):
    # the two kernel families on identical inputs: forward on (q, k, v); the
    # backward on the same (q, k, v, O, L, dO). Both results are bf16, so the
    # bar is 2e-2 + 2 ulp (one rounding on each side).
    B, H, T, D = 1, 4, 384, 128
    q, k, v, do = _inputs(11, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H).to(dev)
    _pin_mfma(monkeypatch, D)
    o_m, L_m = F.rational_attention_forward(q, k, v, slopes, 0.09)
    g_m = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, 0.09)
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    o_t, L_t = F.rational_attention_forward(q, k, v, slopes, 0.09)
    g_t = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, 0.09)
    torch.cuda.synchronize()
    assert _rel_max(L_m, L_t) <= 1e-3
    for x, y, n in zip((o_m,) + tuple(g_m), (o_t,) + tuple(g_t), ("o", "dq", "dk", "dv")):
        err = (x.double() - y.double()).abs()
        bound = 2e-2 + 2 * _ulp(y.cpu(), torch.bfloat16).to(dev)
        assert bool((err <= bound).all()), (n, float(err.max()))


def test_strided_qkv_views_match_contiguous(gpu, monkeypatch):
    # the model's layout: one [B, T, 3, H, D] buffer permuted to three views
    B, T, H, D = 2, 150, 4, 64
    _pin_mfma(monkeypatch, D)
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, T, 3, H, D, generator=g).to(torch.bfloat16).to(dev)
    q, k, v = qkv.permute(2, 0, 3, 1, 4)
    do = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(dev)
    slopes = F.compute_alibi_slopes(H).to(dev)
    a = _run(q, k, v, do, slopes, 0.125)
    b = _run(q.contiguous(), k.contiguous(), v.contiguous(), do, slopes, 0.125)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_backward_is_deterministic(gpu, monkeypatch):
    _pin_mfma(monkeypatch, 128)
    q, k, v, do = _inputs(9, 1, 2, 512, 128, torch.bfloat16)
    slopes = F.compute_alibi_slopes(2).to(dev)
    a = _run(q, k, v, do, slopes, 0.088)
    b = _run(q, k, v, do, slopes, 0.088)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("masked", [False, True])
def test_mfma_backward_is_invariant_to_the_upstream_gradient_scale(gpu, D, masked, monkeypatch):
    # dQ, dK, dV are linear in dO. A training step's dO is ~1e-5 .. 1e-7 per
    # element, where an unscaled fp16 dS would lose its significant bits; the
    # kernels scale dS per query tile by a power of two, so dO * 2^-e must give
    # exactly 2^-e times the gradients of dO (bit for bit: every scaling is a
    # power of two and the outputs stay within bf16's exponent range)
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T = 2, 3, 300
    q, k, v, do = _inputs(31 + D, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    km = None
    if masked:
        km = torch.ones(B, T, dtype=torch.int32, device=dev)
        km[1, T // 2:] = 0

    def grads(dout):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        if masked:
            o = F.rational_attention_masked(qq, kk, vv, slopes, scale, key_mask=km)
        else:
            o = F.rational_attention(qq, kk, vv, slopes, scale)
        o.backward(dout)
        torch.cuda.synchronize()
        return qq.grad, kk.grad, vv.grad

    base = grads(do)
    for e in (12, 20, 28):
        got = grads(do * 2.0 ** -e)
        for name, gt, b in zip(("dq", "dk", "dv"), got, base):
            assert torch.equal(gt.float() * 2.0 ** e, b.float()), (name, e)
    if not masked:  # and the unscaled gradients still meet the oracle bar
        o, L = F.rational_attention_forward(q, k, v, slopes, scale)
        rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
        for name, gt, r in zip(("dq", "dk", "dv"), base, (rq, rk, rv)):
            assert_lowp(gt, r, torch.bfloat16, name)


# ------------------------------------------------- input magnitude range ----
# The MFMA backward rounds dS, and copies of Q and K, to fp16 (range 2^-14 ..
# 65504). Each copy carries a power-of-two scale chosen from the data (per
# 64-row tile for Q, per 32 keys for K, per 64-query tile for dS), so inputs far outside
# N(0, 1) must still meet the bar. Outputs scale with the inputs: each check
# divides got and ref by the known factor of that output and applies the
# unit-scale bar, 2e-2 + 1/2 ulp.

def _scaled_check(q, k, v, do, slopes, scale, factors):
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    for t in (o, L, dq, dk, dv):
        assert bool(torch.isfinite(t).all())
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
    assert _rel_max(L, rL) <= 1e-2
    for name, got, ref in (("o", o, ro), ("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        f = factors[name]
        got = got.detach().to("cpu", torch.float64) / f
        ref = ref.detach().to("cpu", torch.float64) / f
        err = (got - ref).abs()
        excess = float((err - (2e-2 + 0.5 * _ulp(ref, q.dtype))).max())
        print(f"{name}: max err (unit scale) {float(err.max()):.3e}, relL2 "
              f"{float((got - ref).norm() / ref.norm()):.3e}")
        assert excess <= 0, (name, float(err.max()), excess)


@pytest.mark.parametrize("D", [32, 64, 80, 128, 256])
@pytest.mark.parametrize("case", ["v1e4", "do1e-6", "q1e5_k1e-5", "qk1e-4", "combined", "v1e3_do1e2"])
def test_mfma_backward_input_range_bf16(gpu, D, case, monkeypatch):
    _pin_mfma(monkeypatch, D)
    B, H, T = 1, 2, 300
    q, k, v, do = (t.float() for t in _inputs(41 + D, B, H, T, D, torch.float32))
    fq, fk, fv, fd = {"v1e4": (1, 1, 1e4, 1), "do1e-6": (1, 1, 1, 1e-6),
                      "q1e5_k1e-5": (1e5, 1e-5, 1, 1), "qk1e-4": (1e-4, 1e-4, 1, 1),
                      "combined": (1e5, 1e-5, 1e4, 1e-6), "v1e3_do1e2": (1, 1, 1e3, 1e2)}[case]
    q, k, v, do = ((t * f).to(torch.bfloat16) for t, f in ((q, fq), (k, fk), (v, fv), (do, fd)))
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    # s = scale q.k changes only for qk1e-4 (where it shrinks to ~1e-9, the bias alone)
    factors = {"o": fv, "dq": fv * fd * fk, "dk": fv * fd * fq, "dv": fd}
    _scaled_check(q, k, v, do, slopes, scale, factors)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("width", [32, 16])
def test_mfma_backward_key_groups_of_different_magnitude(gpu, D, dtype, width, monkeypatch):
    # K's fp16 form carries one exponent per 32 keys, chosen by the dK/dV
    # kernel and reused by the dQ kernel, which rescales its accumulators
    # whenever the next 32 keys bring another exponent. Keys whose magnitude
    # cycles 2^s, 1, 2^-s from one group of `width` keys to the next give every
    # 32-key group a different exponent (also inside each 64-key tile): a wrong
    # exponent for any group would move that group's share of dq or dk by 2^s.
    # width 16: the two 16-key halves of a 32-key group differ (at D = 256 two
    # wave pairs own them and must agree on the group's exponent: one from
    # the smaller half would overflow the larger half's fp16 copy). At D = 64
    # one wave pair owns 64 keys, two groups with an exponent each.
    _pin_mfma(monkeypatch, D)
    B, H, T = 1, 2, 300
    q, k, v, do = (t.float() for t in _inputs(47 + D, B, H, T, D, torch.float32))
    sh = 12 if dtype == torch.float16 else 20
    gsc = torch.tensor([2.0 ** (sh * (1 - (j // width) % 3)) for j in range(T)])
    k = k * gsc.view(1, 1, T, 1).to(k.device)
    q, k, v, do = (t.to(dtype) for t in (q, k, v, do))
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
    assert _rel_max(L, rL) <= 1e-2
    for name, got, ref in (("o", o, ro), ("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        got = got.detach().to("cpu", torch.float64)
        ref = ref.detach().to("cpu", torch.float64)
        assert bool(torch.isfinite(got).all()), name
        rel = float((got - ref).norm() / ref.norm())
        print(f"{name}: max err / max |ref| {_rel_max(got, ref):.3e}, relL2 {rel:.3e}")
        assert _rel_max(got, ref) <= 2e-2 and rel <= 1e-2, (name, _rel_max(got, ref), rel)
        if name == "dv":
            # each group's rows against that group's own scale (dv = P^T dO
            # takes P from the S recomputed on the groups' fp16 keys; dk is
            # checked over the whole tensor only: the dS of the 2^s groups
            # lies so far below its query tile's largest that fp16 holds it in
            # its subnormal range -- dS has one exponent per query tile, none
            # per key, the documented limit)
            for j0 in range(0, T, width):
                gg, gr = got[:, :, j0:j0 + width], ref[:, :, j0:j0 + width]
                assert _rel_max(gg, gr) <= 2e-2, (name, j0, _rel_max(gg, gr))


@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_mfma_backward_input_range_fp16(gpu, D, monkeypatch):
    _pin_mfma(monkeypatch, D)
    B, H, T = 1, 2, 300
    q, k, v, do = _inputs(43 + D, B, H, T, D, torch.float32)
    fq, fk, fv, fd = 2.0 ** 6, 2.0 ** -6, 2.0 ** 8, 2.0 ** -12
    q, k, v, do = ((t * f).to(torch.float16) for t, f in ((q, fq), (k, fk), (v, fv), (do, fd)))
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    _scaled_check(q, k, v, do, slopes, scale,
                  {"o": fv, "dq": fv * fd * fk, "dk": fv * fd * fq, "dv": fd})


@pytest.mark.parametrize("D", [32, 64, 96, 128, 256])
def test_mfma_attention_is_exactly_equivariant_to_power_of_two_scales(gpu, D, monkeypatch):
    # inputs on a grid of 1/16 are exact in fp16 at every scale used below, so
    # the fp16 copies hold the same significands whatever their exponent: then
    # q 2^16, k 2^-16, v 2^13 and dO 2^-20 must give o 2^13, dq 2^-23, dk 2^9
    # and dv 2^-20 times the unit-scale results, bit for bit -- every scale the
    # kernels pick is a power of two that cancels exactly
    _pin_mfma(monkeypatch, D)
    B, H, T = 2, 3, 200
    g = torch.Generator().manual_seed(53 + D)
    base = [torch.round(torch.randn(B, H, T, D, generator=g) * 16) / 16 for _ in range(4)]
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    unit = _run(*(t.to(torch.bfloat16).to(dev) for t in base), slopes, scale)
    sf = (2.0 ** 16, 2.0 ** -16, 2.0 ** 13, 2.0 ** -20)
    scaled = _run(*((t * f).to(torch.bfloat16).to(dev) for t, f in zip(base, sf)), slopes, scale)
    for name, u, s_, f in zip(("o", "L", "dq", "dk", "dv"), unit, scaled,
                              (2.0 ** 13, 1.0, 2.0 ** -23, 2.0 ** 9, 2.0 ** -20)):
        assert torch.equal(s_.float(), u.float() * f), name


def test_tiled_fallback_warns_once(gpu):
    # a bf16 call outside the MFMA kernels' envelope (here D = 100, not a
    # multiple of 8) runs the fp32 tiled kernels; the wrapper says so, once
    # per reason
    import warnings
    from fastalgebraictransformer_amd import forward as fw
    fw._WARNED.clear()
    q, k, v, _ = _inputs(5, 1, 2, 40, 100, torch.bfloat16)
    slopes = F.compute_alibi_slopes(2).to(dev)
    with pytest.warns(RuntimeWarning, match="head dim 100"):
        F.rational_attention_forward(q, k, v, slopes, 0.17)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        F.rational_attention_forward(q, k, v, slopes, 0.17)
        q2, k2, v2, _ = _inputs(6, 1, 2, 40, 128, torch.bfloat16)
        F.rational_attention_forward(q2, k2, v2, slopes, 0.09)  # covered: no warning


@pytest.mark.parametrize("mode", ["plain", "masked", "noncausal"])
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64), (torch.bfloat16, 256)])
def test_mfma_backward_head_groups_are_bit_identical(gpu, mode, dtype, D, monkeypatch):
    # the backward keeps the dS^T tiles of one group of heads at a time in the
    # workspace (dK/dV stores them, dQ reads them back); a small cap
    # (KAT_ATTN_DS_CAP_BYTES) splits the heads into several groups, the last
    # one short. The arithmetic per head is the same, so the gradients must be
    # equal bit for bit to the one-group run.
    from fastalgebraictransformer_amd.backward import _attn_bwd_into
    from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg
    _pin_mfma(monkeypatch, D)
    B, H, T = 2, 5, 300
    q, k, v, do = _inputs(91 + D, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    km, causal, ext = None, True, False
    if mode != "plain":
        ext, causal = True, mode == "masked"
        m = torch.ones(B, T, dtype=torch.int32)
        m[0, :70] = 0
        m[1, 5::7] = 0
        km = _key_mask_arg(m, B, T, dev)
    o = torch.empty_like(q)
    L = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    _attn_fwd_into(q, k, v, o, L, slopes, scale, causal, 1e-6, km, extended=ext)
    runs = []
    nt = (T + 63) // 64
    # T < 512: one dQ block (8 query tiles) per head, 8 x nt dS tiles of 8 KB
    for cap in (None, 3 * 8 * nt * 8192):  # groups of 3, 3, 3, 1 heads
        if cap is None:
            monkeypatch.delenv("KAT_ATTN_DS_CAP_BYTES", raising=False)
        else:
            monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", str(cap))
        g = [torch.full_like(q, float("nan")) for _ in range(3)]
        _attn_bwd_into(q, k, v, o, L, do, *g, slopes, scale, causal, 1e-6, km, extended=ext)
        torch.cuda.synchronize()
        runs.append(g)
    for name, a, b in zip(("dq", "dk", "dv"), *runs):
        assert bool(torch.isfinite(a).all()), name
        assert torch.equal(a, b), name


@pytest.mark.parametrize("mode", ["plain", "masked", "noncausal"])
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64), (torch.bfloat16, 256)])
def test_mfma_backward_key_bands_are_bit_identical(gpu, mode, dtype, D, monkeypatch):
    # when one head's dS^T tiles exceed the cap, the backward runs dK/dV + dQ
    # per band of key tiles (multiples of 8 tiles = 512 keys), dQ keeping fp32
    # partial sums between the bands. The MFMA accumulation order is the one
    # of the single-band run and the partial sums are stored and reloaded
    # exactly, so the gradients must be equal bit for bit.
    from fastalgebraictransformer_amd.backward import _attn_bwd_into
    from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg
    _pin_mfma(monkeypatch, D)
    B, H, T = 2, 3, 1300  # 21 key tiles: bands of 8, 8 and 5 tiles
    q, k, v, do = _inputs(131 + D, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    km, causal, ext = None, True, False
    if mode != "plain":
        ext, causal = True, mode == "masked"
        m = torch.ones(B, T, dtype=torch.int32)
        m[0, :300] = 0
        m[1, 7::5] = 0
        m[1, 600:1100] = 0  # whole key tiles (and a whole band's worth) dropped
        km = _key_mask_arg(m, B, T, dev)
    o = torch.empty_like(q)
    L = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    _attn_fwd_into(q, k, v, o, L, slopes, scale, causal, 1e-6, km, extended=ext)
    lib = _lib.load()
    code = _lib.dtype_code(q)
    runs = []
    # 192 tiles of 8 KB: an 8-tile band of this T in every mode, not 16 tiles
    for cap in (None, 192 * 8192):
        if cap is None:
            monkeypatch.delenv("KAT_ATTN_DS_CAP_BYTES", raising=False)
        else:
            monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", str(cap))
        ws = lib.kat_attn_bwd_masked_workspace_size(B, H, T, D, code, int(causal))
        g = [torch.full_like(q, float("nan")) for _ in range(3)]
        _attn_bwd_into(q, k, v, o, L, do, *g, slopes, scale, causal, 1e-6, km, extended=ext)
        torch.cuda.synchronize()
        runs.append((g, ws))
    (g0, ws0), (g1, ws1) = runs
    assert ws1 < ws0
    for name, a, b in zip(("dq", "dk", "dv"), g0, g1):
        assert bool(torch.isfinite(a).all()), name
        assert torch.equal(a, b), name
    # and the banded result against the oracle at the bf16 / fp16 bar, on two
    # heads (batch 1's mask drops a band's worth of keys)
    for bs, hs in ((slice(0, 1), slice(0, 1)), (slice(1, 2), slice(2, 3))):
        kmb = None if km is None else km[bs].cpu()
        args = [t[bs, hs] for t in (q, k, v)]
        rq, rk, rv = O.attention_bwd(*args, o[bs, hs], L[bs, hs], do[bs, hs], slopes[hs].cpu(), scale,
                                     dtype=torch.float32, key_mask=kmb, causal=causal)
        for name, got, ref in (("dq", g1[0], rq), ("dk", g1[1], rk), ("dv", g1[2], rv)):
            assert_lowp(got[bs, hs], ref, dtype, name)


def test_mfma_backward_at_65536_in_bands_matches_fp32_tiled(gpu, monkeypatch):
    # T = 65536: one causal head's dS tiles (~4.3 GB) exceed the default 4 GiB
    # cap, so the default call already runs in two bands; a 512 MiB cap runs
    # ~12 bands and must give the same bits, with a workspace within the cap
    # plus O(T D). Against the fp32 tiled kernels (an independent
    # implementation, O(T) memory) on the same bf16-rounded inputs at the bf16
    # bar.
    B, H, T, D = 1, 1, 65536, 128
    q, k, v, do = _inputs(167, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(8)[5:6].to(dev)  # a mid-range slope, 2^-3
    scale = 1.0 / math.sqrt(D)
    _pin_mfma(monkeypatch, D)
    lib = _lib.load()
    ws_default = lib.kat_attn_bwd_workspace_size(B, H, T, D, 1)
    assert ws_default <= (4 << 30) + T * D * 16
    o_m, L_m = F.rational_attention_forward(q, k, v, slopes, scale)
    g_m = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, scale)
    cap = 512 << 20
    monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", str(cap))
    assert lib.kat_attn_bwd_workspace_size(B, H, T, D, 1) <= cap + T * D * 16
    g_c = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, scale)
    monkeypatch.delenv("KAT_ATTN_DS_CAP_BYTES")
    for a, b, n in zip(g_m, g_c, ("dq", "dk", "dv")):
        assert torch.equal(a, b), n
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    f32 = [t.float() for t in (q, k, v, do)]
    o_t, L_t = F.rational_attention_forward(f32[0], f32[1], f32[2], slopes, scale)
    g_t = F.rational_attention_backward(f32[0], f32[1], f32[2], o_m.float(), L_m, f32[3], slopes, scale)
    torch.cuda.synchronize()
    assert _rel_max(L_m, L_t) <= 1e-3
    errs = {"o": assert_lowp(o_m, o_t, torch.bfloat16, "o")}
    for n, x, y in zip(("dq", "dk", "dv"), g_m, g_t):
        errs[n] = assert_lowp(x, y, torch.bfloat16, n)
    print("T = 65536 in bands vs fp32 tiled: " + ", ".join(f"{n} {e:.3e} / {r:.3e}" for n, (e, r) in errs.items()))


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mfma_backward_query_tiles_of_different_magnitude(gpu, D, dtype, monkeypatch):
    # dS enters the fp16 products with one exponent per 64-query tile, chosen
    # from that tile's bound. Upstream gradients whose magnitude differs by
    # 2^30 (bf16; 2^12 in fp16, whose own range is narrower) from one 64-query
    # tile to the next give the small tiles' dS its own exponent: their dq
    # must hold to the bar relative to their own size. (With one exponent per
    # head their dS lay 2^30 below the head's largest, in fp16's subnormal
    # range.) dk and dv are sums over all queries, dominated by the large
    # tiles; they are checked over the whole tensor.
    _pin_mfma(monkeypatch, D)
    B, H, T = 1, 2, 512
    q, k, v, do = (t.float() for t in _inputs(59 + D, B, H, T, D, torch.float32))
    sh = 12 if dtype == torch.float16 else 30
    tsc = torch.tensor([2.0 ** (-sh * ((i // 64) % 2)) for i in range(T)])
    do = do * tsc.view(1, 1, T, 1).to(do.device)
    q, k, v, do = (t.to(dtype) for t in (q, k, v, do))
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale)
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        got = got.detach().to("cpu", torch.float64)
        ref = ref.detach().to("cpu", torch.float64)
        assert bool(torch.isfinite(got).all()), name
        rel = float((got - ref).norm() / ref.norm())
        assert _rel_max(got, ref) <= 2e-2 and rel <= 1e-2, (name, _rel_max(got, ref), rel)
        if name == "dq":
            for i0 in range(0, T, 64):
                gg, gr = got[:, :, i0:i0 + 64], ref[:, :, i0:i0 + 64]
                rel_t = float((gg - gr).norm() / gr.norm())
                print(f"dq tile {i0 // 64}: max err / max |ref| {_rel_max(gg, gr):.3e}, relL2 {rel_t:.3e}")
                assert _rel_max(gg, gr) <= 2e-2 and rel_t <= 1e-2, (name, i0, _rel_max(gg, gr), rel_t)


def test_mfma_long_sequence_matches_fp32_tiled(gpu, monkeypatch):
    # T = 16384: the backward's stored dS tiles grow as T^2 (33792 tiles
    # per head here); the MFMA path against the fp32 tiled kernels on the same
    # (bf16-rounded) inputs, an independent implementation, at the bf16 bar;
    # and one head per dS group (a 1-byte cap) must give the same bits
    B, H, T, D = 1, 2, 16384, 128
    q, k, v, do = _inputs(101, B, H, T, D, torch.bfloat16)
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    _pin_mfma(monkeypatch, D)
    o_m, L_m = F.rational_attention_forward(q, k, v, slopes, scale)
    g_m = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, scale)
    monkeypatch.setenv("KAT_ATTN_DS_CAP_BYTES", "1")
    g_1 = F.rational_attention_backward(q, k, v, o_m, L_m, do, slopes, scale)
    monkeypatch.delenv("KAT_ATTN_DS_CAP_BYTES")
    for a, b, n in zip(g_m, g_1, ("dq", "dk", "dv")):
        assert torch.equal(a, b), n
    monkeypatch.setenv("KAT_ATTN_IMPL", "tiled")
    f32 = [t.float() for t in (q, k, v, do)]
    o_t, L_t = F.rational_attention_forward(f32[0], f32[1], f32[2], slopes, scale)
    g_t = F.rational_attention_backward(f32[0], f32[1], f32[2], o_m.float(), L_m, f32[3], slopes, scale)
    torch.cuda.synchronize()
    assert _rel_max(L_m, L_t) <= 1e-3
    errs = {"o": assert_lowp(o_m, o_t, torch.bfloat16, "o")}
    for n, x, y in zip(("dq", "dk", "dv"), g_m, g_t):
        errs[n] = assert_lowp(x, y, torch.bfloat16, n)
    print("T = 16384 vs fp32 tiled: " + ", ".join(f"{n} {e:.3e} / {r:.3e}" for n, (e, r) in errs.items()))
