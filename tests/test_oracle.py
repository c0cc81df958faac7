"""Pins for the CPU oracle (CPU only).

Each check is chosen so that a plausible slip in the oracle (a dropped term, a
flipped sign or index, a transposed operand, eps in the wrong place) fails:
closed-form known answers, symmetries, an independent formulation (the
reference test harness, tests.py:44-65), a pure-Python loop, torch.autograd and
central finite differences.
"""

import math

import pytest
import torch

import oracle as O

f64 = torch.float64


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- sigma ----

def test_rsig_known_answers():
    x = torch.tensor([0.0, 1.0, -1.0, 3.0, -3.0], dtype=f64)
    assert torch.equal(O.rsig(x), torch.tensor([0.5, 0.75, 0.25, 0.875, 0.125], dtype=f64))
    d = O.rsig_deriv(torch.tensor([0.0, 1.0, -1.0], dtype=f64))
    assert torch.allclose(d, torch.tensor([0.5, 0.125, 0.125], dtype=f64), rtol=0, atol=0)


def test_rsig_symmetry_range_and_derivative():
    x = torch.randn(4096, generator=_g(0), dtype=f64) * 10
    s = O.rsig(x)
    assert torch.allclose(O.rsig(-x), 1 - s, atol=1e-15, rtol=0)
    assert bool(((s > 0) & (s < 1)).all())
    h = 1e-6
    fd = (O.rsig(x + h) - O.rsig(x - h)) / (2 * h)
    assert torch.allclose(O.rsig_deriv(x), fd, atol=1e-8, rtol=1e-6)


# -------------------------------------------------------------- softmax ----

def test_softmax_constant_row_known_answer():
    c, n, eps = 0.7, 33, 1e-6
    x = torch.full((2, n), c, dtype=f64)
    s = 0.5 * (c / (abs(c) + 1) + 1)
    expect = s ** 4 / (n * s ** 4 + eps)
    assert torch.allclose(O.rational_softmax_fwd(x, eps), torch.full((2, n), expect, dtype=f64),
                          rtol=1e-15, atol=0)


def test_softmax_row_sum_identity():
    x = torch.randn(8, 257, generator=_g(1), dtype=f64) * 2
    eps = 1e-6
    p = O.rational_softmax_fwd(x, eps)
    z = (O.rsig(x) ** 4).sum(-1)
    assert torch.allclose(p.sum(-1), z / (z + eps), rtol=1e-14, atol=0)
    # the reference bar (tests.py:87,97): |sum - 1| < 1e-5
    assert float((p.sum(-1) - 1).abs().max()) < 1e-5


def test_softmax_bwd_matches_autograd_and_finite_differences():
    eps = 1e-6
    x = (torch.randn(3, 40, generator=_g(2), dtype=f64) * 2).requires_grad_(True)
    dy = torch.randn(3, 40, generator=_g(3), dtype=f64)
    sig = 0.5 * (x / (x.abs() + 1) + 1)
    f = sig.pow(4)
    p = f / (f.sum(-1, keepdim=True) + eps)
    (gx,) = torch.autograd.grad(p, x, dy)
    ours = O.rational_softmax_bwd(dy, x.detach(), p.detach(), eps)
    # the kernel formula uses sigma + eps in g (fused_ops.py:184); relative
    # deviation from the exact derivative is <= eps / sigma
    assert torch.allclose(ours, gx, rtol=1e-4, atol=1e-9)
    # central differences of <dy, p(x)> in a few coordinates
    xd = x.detach()
    for (r, c) in [(0, 0), (1, 17), (2, 39)]:
        h = 1e-6
        xp, xm = xd.clone(), xd.clone()
        xp[r, c] += h
        xm[r, c] -= h
        fd = ((O.rational_softmax_fwd(xp, eps) - O.rational_softmax_fwd(xm, eps)) * dy).sum() / (2 * h)
        assert abs(float(fd) - float(ours[r, c])) < 1e-6 + 1e-4 * abs(float(fd))


# --------------------------------------------------------------- swiglu ----

def test_swiglu_known_answers():
    assert float(O.swiglu_fwd(torch.tensor(1.0), torch.tensor(2.0))) == 1.5
    v = torch.randn(16, generator=_g(4), dtype=f64)
    assert torch.equal(O.swiglu_fwd(torch.zeros(16, dtype=f64), v), torch.zeros(16, dtype=f64))
    dy = torch.randn(16, generator=_g(5), dtype=f64)
    dg, dv = O.swiglu_bwd(dy, torch.zeros(16, dtype=f64), v)
    assert torch.allclose(dg, 0.5 * v * dy, rtol=0, atol=0)
    assert torch.equal(dv, torch.zeros(16, dtype=f64))


def test_swiglu_bwd_matches_autograd():
    g = torch.randn(5, 64, generator=_g(6), dtype=f64).requires_grad_(True)
    v = torch.randn(5, 64, generator=_g(7), dtype=f64).requires_grad_(True)
    dy = torch.randn(5, 64, generator=_g(8), dtype=f64)
    out = g * (0.5 * (g / (g.abs() + 1) + 1)) * v
    gg, gv = torch.autograd.grad(out, (g, v), dy)
    dg, dv = O.swiglu_bwd(dy, g.detach(), v.detach())
    assert torch.allclose(dg, gg, rtol=1e-13, atol=1e-14)
    assert torch.allclose(dv, gv, rtol=1e-13, atol=1e-14)


# ----------------------------------------------------------------- norm ----

def test_norm_constant_row_known_answer_and_scale_invariance():
    eps = 1e-6
    c, n = -2.5, 10
    x = torch.full((3, n), c, dtype=f64)
    w = torch.linspace(0.5, 1.5, n, dtype=f64)
    y, mu = O.mean_error_norm_fwd(x, w, eps)
    assert torch.allclose(mu, torch.full((3,), abs(c), dtype=f64), rtol=0, atol=0)
    assert torch.allclose(y, (c / (abs(c) + eps)) * w.expand(3, n), rtol=1e-15, atol=0)
    xr = torch.randn(4, 128, generator=_g(9), dtype=f64)
    y1, _ = O.mean_error_norm_fwd(xr, w.repeat(13)[:128], 0.0)
    y2, _ = O.mean_error_norm_fwd(7.0 * xr, w.repeat(13)[:128], 0.0)
    assert torch.allclose(y1, y2, rtol=1e-13, atol=1e-13)


def test_norm_bwd_matches_autograd():
    eps = 1e-6
    x = torch.randn(6, 96, generator=_g(10), dtype=f64).requires_grad_(True)
    w = (1 + 0.02 * torch.randn(96, generator=_g(11), dtype=f64)).requires_grad_(True)
    dy = torch.randn(6, 96, generator=_g(12), dtype=f64)
    y = x / (x.abs().mean(-1, keepdim=True) + eps) * w
    gx, gw = torch.autograd.grad(y, (x, w), dy)
    _, mu = O.mean_error_norm_fwd(x.detach(), w.detach(), eps)
    dx, dw = O.mean_error_norm_bwd(dy, x.detach(), w.detach(), mu, eps)
    assert torch.allclose(dx, gx, rtol=1e-12, atol=1e-12)
    assert torch.allclose(dw, gw, rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------- slopes ----

def test_alibi_slopes_closed_forms():
    s16 = O.alibi_slopes(16)
    # float32 torch.pow is within a few ulp of the exact power
    assert torch.allclose(s16, torch.tensor([2 ** (-(i + 1) / 2) for i in range(16)]), rtol=5e-7, atol=0)
    s8 = O.alibi_slopes(8)
    assert torch.equal(s8, torch.tensor([2.0 ** -(i + 1) for i in range(8)]))
    s12 = O.alibi_slopes(12)
    expect = [2.0 ** -(i + 1) for i in range(8)] + [0.70710678, 0.35355339, 0.1767767, 0.088388348]
    assert torch.allclose(s12, torch.tensor(expect), rtol=1e-6, atol=0)
    assert O.alibi_slopes(1).tolist() == [2.0 ** -8]


# ------------------------------------------------------------ attention ----

def _attn_inputs(B, H, T, D, seed):
    g = _g(seed)
    q = torch.randn(B, H, T, D, generator=g, dtype=f64)
    k = torch.randn(B, H, T, D, generator=g, dtype=f64)
    v = torch.randn(B, H, T, D, generator=g, dtype=f64)
    do = torch.randn(B, H, T, D, generator=g, dtype=f64)
    return q, k, v, do


@pytest.mark.parametrize("B,H,T,D", [(1, 4, 32, 32), (2, 3, 19, 16), (1, 2, 64, 8)])
def test_attention_fwd_matches_reference_harness(B, H, T, D):
    q, k, v, _ = _attn_inputs(B, H, T, D, 20 + T)
    slopes = O.alibi_slopes(H)
    scale = 1 / math.sqrt(D)
    o, L = O.attention_fwd(q, k, v, slopes, scale)
    ref = O.harness_attention(q, k, v, slopes.double(), scale)
    # masked keys add sigma(-1e4)^4 ~ 6e-18 each in the harness only
    assert torch.allclose(o, ref, rtol=1e-12, atol=1e-12)
    # chunked evaluation is exact
    o2, L2 = O.attention_fwd(q, k, v, slopes, scale, chunk=1)
    assert torch.equal(o, o2) and torch.equal(L, L2)


def test_attention_fwd_matches_python_loop():
    q, k, v, _ = _attn_inputs(1, 2, 6, 3, 30)
    slopes = torch.tensor([0.5, 0.125])
    o, L = O.attention_fwd(q, k, v, slopes, 0.7)
    ol, Ll = O.loop_attention_fwd(q, k, v, slopes, 0.7)
    assert torch.allclose(o, ol, rtol=1e-13, atol=1e-14)
    assert torch.allclose(L, Ll, rtol=1e-13, atol=1e-14)


def test_attention_fwd_known_answers():
    eps = 1e-6
    # T = 1: o = f / (f + eps) * v with f = sigma(scale q.k)^4
    q, k, v, _ = _attn_inputs(1, 1, 1, 4, 31)
    o, L = O.attention_fwd(q, k, v, torch.tensor([0.3]), 0.5, eps)
    f = O.rsig((q * k).sum(-1) * 0.5) ** 4
    assert torch.allclose(L, f, rtol=1e-15, atol=0)
    assert torch.allclose(o, v * (f / (f + eps)).unsqueeze(-1), rtol=1e-14, atol=0)
    # q = 0, slopes = 0: every f = 0.5^4, so o_i is the prefix mean of v
    # shrunk by (i+1) / ((i+1) + 16 eps)
    T = 9
    _, k, v, _ = _attn_inputs(1, 1, T, 5, 32)
    o, L = O.attention_fwd(torch.zeros(1, 1, T, 5, dtype=f64), k, v, torch.zeros(1), 1.0, eps)
    n = torch.arange(1, T + 1, dtype=f64)
    pm = v.cumsum(-2) / n.view(1, 1, T, 1)
    assert torch.allclose(o, pm * (n / (n + 16 * eps)).view(1, 1, T, 1), rtol=1e-13, atol=1e-15)
    assert torch.allclose(L[0, 0], n / 16, rtol=1e-15, atol=0)


@pytest.mark.parametrize("eps,tol", [(0.0, 1e-11), (1e-6, 5e-5)])
@pytest.mark.parametrize("B,H,T,D", [(1, 4, 32, 32), (2, 2, 17, 8)])
def test_attention_bwd_matches_autograd_of_harness(B, H, T, D, eps, tol):
    q, k, v, do = _attn_inputs(B, H, T, D, 40 + T)
    slopes = O.alibi_slopes(H)
    scale = 1 / math.sqrt(D)
    o, L = O.attention_fwd(q, k, v, slopes, scale, eps)
    dq, dk, dv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, eps)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref = O.harness_attention(qr, kr, vr, slopes.double(), scale, eps)
    gq, gk, gv = torch.autograd.grad(ref, (qr, kr, vr), do)
    # with eps = 0 the kernel formula is the exact derivative; with eps > 0 it
    # keeps sigma + eps in g (backward.py:145), a relative change <= eps/sigma
    for ours, theirs in ((dq, gq), (dk, gk), (dv, gv)):
        err = float((ours - theirs).abs().max())
        assert err < tol * max(1.0, float(theirs.abs().max())), err


def test_attention_bwd_matches_finite_differences():
    eps = 1e-6
    q, k, v, do = _attn_inputs(1, 2, 7, 4, 50)
    slopes = torch.tensor([0.5, 0.0625])
    scale = 0.6
    o, L = O.attention_fwd(q, k, v, slopes, scale, eps)
    grads = O.attention_bwd(q, k, v, o, L, do, slopes, scale, eps)
    h = 1e-6
    for which, t in enumerate((q, k, v)):
        for idx in [(0, 0, 0, 0), (0, 1, 3, 2), (0, 0, 6, 3), (0, 1, 5, 1)]:
            tp, tm = t.clone(), t.clone()
            tp[idx] += h
            tm[idx] -= h
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = tp, tm
            op, _ = O.attention_fwd(*args_p, slopes, scale, eps)
            om, _ = O.attention_fwd(*args_m, slopes, scale, eps)
            fd = float(((op - om) * do).sum() / (2 * h))
            an = float(grads[which][idx])
            assert abs(fd - an) < 1e-6 + 1e-5 * abs(fd), (which, idx, fd, an)


# ------------------------------------------ padding mask / non-causal ----
# Extensions beyond the reference kernels (which are always causal and take no
# mask). The padding mask is pinned to the reference's own CPU attention
# (algebraic_model.py:112-136, restated by harness_attention: -1e4 fill where
# mask == 0); the non-causal mode to closed forms, a symmetry the causal mode
# lacks, the causal path at the last query, a pure-Python loop and autograd.

def _padding_mask(B, T, seed):
    g = _g(seed)
    m = (torch.rand(B, T, generator=g) > 0.3).to(torch.int64)
    m[0, : T // 3] = 0          # left padding, incl. queries that see no key
    if B > 1:
        m[1, -(T // 4):] = 0    # right padding
    return m


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,T,D", [(2, 3, 21, 8), (3, 2, 64, 16)])
def test_masked_attention_fwd_matches_reference_cpu_path(B, H, T, D, causal):
    q, k, v, _ = _attn_inputs(B, H, T, D, 60 + T)
    slopes = O.alibi_slopes(H)
    scale = 1 / math.sqrt(D)
    km = _padding_mask(B, T, T)
    o, L = O.attention_fwd(q, k, v, slopes, scale, causal=causal, key_mask=km)
    ref = O.harness_attention(q, k, v, slopes.double(), scale, causal=causal, key_mask=km)
    # the fill leaves ~6e-18 per dropped key; rows with no visible key are
    # 0 here and (count * 6e-18 * v) / 1e-6 ~ 1e-10 there
    assert torch.allclose(o, ref, rtol=1e-10, atol=1e-9)
    o2, L2 = O.attention_fwd(q, k, v, slopes, scale, chunk=1, causal=causal, key_mask=km)
    assert torch.equal(o, o2) and torch.equal(L, L2)
    # an all-ones mask is no mask
    o3, L3 = O.attention_fwd(q, k, v, slopes, scale, causal=causal,
                             key_mask=torch.ones(B, T, dtype=torch.int64))
    o4, L4 = O.attention_fwd(q, k, v, slopes, scale, causal=causal)
    assert torch.equal(o3, o4) and torch.equal(L3, L4)


def test_masked_attention_fwd_matches_python_loop():
    q, k, v, _ = _attn_inputs(2, 2, 7, 3, 61)
    slopes = torch.tensor([0.5, 0.125])
    km = torch.tensor([[1, 0, 1, 1, 0, 1, 0], [0, 0, 0, 1, 1, 1, 1]])
    for causal in (True, False):
        o, L = O.attention_fwd(q, k, v, slopes, 0.7, causal=causal, key_mask=km)
        ol, Ll = O.loop_attention_fwd(q, k, v, slopes, 0.7, causal=causal, key_mask=km)
        assert torch.allclose(o, ol, rtol=1e-13, atol=1e-14)
        assert torch.allclose(L, Ll, rtol=1e-13, atol=1e-14)
    # batch 1, causal: queries 0..2 see only masked keys -> L = 0, o = 0
    o, L = O.attention_fwd(q, k, v, slopes, 0.7, key_mask=km)
    assert torch.equal(L[1, :, :3], torch.zeros(2, 3, dtype=f64))
    assert torch.equal(o[1, :, :3], torch.zeros(2, 3, 3, dtype=f64))


def test_noncausal_known_answers_and_symmetry():
    eps = 1e-6
    T = 11
    _, k, v, _ = _attn_inputs(1, 1, T, 5, 62)
    # q = 0, slopes = 0: every f = 0.5^4 over all T keys -> o_i = mean(v) T / (T + 16 eps)
    o, L = O.attention_fwd(torch.zeros(1, 1, T, 5, dtype=f64), k, v, torch.zeros(1), 1.0, eps,
                           causal=False)
    mean = v.mean(-2, keepdim=True).expand_as(v)
    assert torch.allclose(o, mean * (T / (T + 16 * eps)), rtol=1e-13, atol=1e-15)
    assert torch.allclose(L, torch.full_like(L, T / 16), rtol=1e-15, atol=0)
    # ALiBi on |i - j| is symmetric: reversing the sequence reverses the output
    # (the causal mode, and a signed i - j, break this)
    q, k, v, _ = _attn_inputs(2, 3, 13, 4, 63)
    slopes = O.alibi_slopes(3)
    o, L = O.attention_fwd(q, k, v, slopes, 0.5, causal=False)
    fl = lambda t: t.flip(-2)
    orr, Lr = O.attention_fwd(fl(q), fl(k), fl(v), slopes, 0.5, causal=False)
    assert torch.allclose(fl(orr), o, rtol=1e-13, atol=1e-14)
    assert torch.allclose(Lr.flip(-1), L, rtol=1e-13, atol=0)
    # the last query sees every key in both modes
    oc, Lc = O.attention_fwd(q, k, v, slopes, 0.5)
    assert torch.allclose(oc[..., -1, :], o[..., -1, :], rtol=1e-14, atol=1e-15)
    assert not torch.allclose(oc[..., 0, :], o[..., 0, :])


@pytest.mark.parametrize("causal", [True, False])
def test_masked_attention_bwd_matches_autograd_of_harness(causal):
    B, H, T, D = 2, 3, 19, 8
    q, k, v, do = _attn_inputs(B, H, T, D, 64)
    slopes = O.alibi_slopes(H)
    scale = 1 / math.sqrt(D)
    # every query keeps at least one visible key here, so that the -1e4
    # fill's remainders stay negligible in the gradients as well
    km = torch.ones(B, T, dtype=torch.int64)
    km[0, 3:7] = 0
    km[1, -5:] = 0
    km[1, 1] = 0
    o, L = O.attention_fwd(q, k, v, slopes, scale, 0.0, causal=causal, key_mask=km)
    dq, dk, dv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, 0.0, causal=causal,
                                 key_mask=km)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref = O.harness_attention(qr, kr, vr, slopes.double(), scale, 0.0, causal=causal, key_mask=km)
    gq, gk, gv = torch.autograd.grad(ref, (qr, kr, vr), do)
    for ours, theirs in ((dq, gq), (dk, gk), (dv, gv)):
        err = float((ours - theirs).abs().max())
        assert err < 1e-10 * max(1.0, float(theirs.abs().max())), err
    # dropped keys get exactly zero dK, dV
    drop = (km == 0)[:, None, :, None].expand_as(dk)
    assert torch.equal(dk[drop], torch.zeros_like(dk[drop]))
    assert torch.equal(dv[drop], torch.zeros_like(dv[drop]))
