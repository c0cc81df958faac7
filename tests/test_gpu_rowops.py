"""GPU parity of the row ops (rational softmax, SwiGLU, mean-error norm)
against the CPU oracle. Tolerances are written next to each check:
  * fp32: <= 1e-5 relative (+ a 1e-6 * max|ref| floor for near-zero values),
    the reference bars (tests.py:96-98,132-133,167-168) are looser;
  * bf16: within 1 bf16 ulp of the oracle (kernels compute in fp32 and round
    once) -- plus a small absolute floor where the oracle value itself is the
    difference of two nearly equal terms.
"""

import math

import numpy as np
import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import assert_bf16_within_ulp, assert_rel, golden, max_abs

pytestmark = pytest.mark.gpu
dev = "cuda"


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.asarray(a)).to(dev, dtype)


def _seeded(seed, *shape, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ------------------------------------------------------------- fixtures ----

def test_golden_fp32(gpu):
    z = golden("softmax_f32")
    x = _t(z["x"]).requires_grad_(True)
    p = F.rational_softmax(x)
    assert_rel(p, torch.from_numpy(z["p"]), 1e-5, "softmax fwd f32")
    p.backward(_t(z["dy"]))
    assert_rel(x.grad, torch.from_numpy(z["dx"]), 1e-5, "softmax bwd f32", floor_frac=1e-5)

    z = golden("swiglu_f32")
    g, v = _t(z["gate"]).requires_grad_(True), _t(z["value"]).requires_grad_(True)
    out = F.rational_swiglu(g, v)
    assert_rel(out, torch.from_numpy(z["out"]), 1e-5, "swiglu fwd f32")
    out.backward(_t(z["dy"]))
    assert_rel(g.grad, torch.from_numpy(z["dgate"]), 1e-5, "swiglu dgate f32")
    assert_rel(v.grad, torch.from_numpy(z["dvalue"]), 1e-5, "swiglu dvalue f32")

    z = golden("norm_f32")
    x, w = _t(z["x"]).requires_grad_(True), _t(z["w"]).requires_grad_(True)
    y = F.mean_error_norm(x, w)
    assert_rel(y, torch.from_numpy(z["y"]), 1e-5, "norm fwd f32")
    y.backward(_t(z["dy"]))
    assert_rel(x.grad, torch.from_numpy(z["dx"]), 1e-5, "norm dx f32", floor_frac=1e-5)
    assert_rel(w.grad, torch.from_numpy(z["dw"]), 1e-5, "norm dw f32", floor_frac=1e-5)


def test_golden_bf16(gpu):
    bf = torch.bfloat16
    z = golden("softmax_bf16")
    x = _t(z["x"], bf).requires_grad_(True)
    p = F.rational_softmax(x)
    assert_bf16_within_ulp(p, torch.from_numpy(z["p"]), what="softmax fwd bf16")
    p.backward(_t(z["dy"], bf))
    # dx = p g (dy - <dy,p>): the oracle's own value cancels; floor 1e-3 max|dx|
    ref = torch.from_numpy(z["dx"])
    assert_bf16_within_ulp(x.grad, ref, abs_floor=1e-3 * float(ref.abs().max()),
                           what="softmax bwd bf16")

    z = golden("swiglu_bf16")
    g, v = _t(z["gate"], bf).requires_grad_(True), _t(z["value"], bf).requires_grad_(True)
    out = F.rational_swiglu(g, v)
    assert_bf16_within_ulp(out, torch.from_numpy(z["out"]), what="swiglu fwd bf16")
    out.backward(_t(z["dy"], bf))
    assert_bf16_within_ulp(g.grad, torch.from_numpy(z["dgate"]), what="swiglu dgate bf16")
    assert_bf16_within_ulp(v.grad, torch.from_numpy(z["dvalue"]), what="swiglu dvalue bf16")

    z = golden("norm_bf16")
    x = _t(z["x"], bf).requires_grad_(True)
    w = _t(z["w"]).requires_grad_(True)  # fp32 parameter, bf16 activations
    y = F.mean_error_norm(x, w)
    assert_bf16_within_ulp(y, torch.from_numpy(z["y"]), what="norm fwd bf16")
    y.backward(_t(z["dy"], bf))
    ref = torch.from_numpy(z["dx"])
    assert_bf16_within_ulp(x.grad, ref, abs_floor=1e-3 * float(ref.abs().max()), what="norm dx bf16")
    assert w.grad.dtype == torch.float32
    assert_rel(w.grad, torch.from_numpy(z["dw"]), 1e-5, "norm dw (fp32 from bf16)", floor_frac=1e-5)


# --------------------------------------------- reference test shapes ----

@pytest.mark.parametrize("shape", [(2, 8, 64, 64), (4, 12, 128, 128), (2, 16, 256, 256)])
def test_softmax_reference_shapes_f32(gpu, shape):
    # tests.py:78-98 shapes; seeded here
    x = _seeded(1, *shape).to(dev).requires_grad_(True)
    dy = _seeded(2, *shape).to(dev)
    p = F.rational_softmax(x)
    ref = O.rational_softmax_fwd(x)
    assert_rel(p, ref, 1e-5, "softmax fwd")
    assert float((p.detach().double().sum(-1) - 1).abs().max()) < 1e-5  # tests.py:87,97
    p.backward(dy)
    ref_dx = O.rational_softmax_bwd(dy, x, p.detach().double())
    assert max_abs(x.grad, ref_dx) < 1e-3  # tests.py:98
    assert_rel(x.grad, ref_dx, 1e-5, "softmax bwd", floor_frac=1e-5)


@pytest.mark.parametrize("shape", [(2, 512, 768), (4, 1024, 1024), (8, 2048, 2048)])
def test_swiglu_reference_shapes_f32(gpu, shape):
    g = _seeded(3, *shape).to(dev).requires_grad_(True)
    v = _seeded(4, *shape).to(dev).requires_grad_(True)
    dy = _seeded(5, *shape).to(dev)
    out = F.rational_swiglu(g, v)
    assert_rel(out, O.swiglu_fwd(g, v), 1e-5, "swiglu fwd")
    out.backward(dy)
    dg, dv = O.swiglu_bwd(dy, g, v)
    assert_rel(g.grad, dg, 1e-5, "swiglu dgate")
    assert_rel(v.grad, dv, 1e-5, "swiglu dvalue")


@pytest.mark.parametrize("shape", [(2, 512, 768), (4, 1024, 1024)])
def test_norm_reference_shapes_f32(gpu, shape):
    x = _seeded(6, *shape).to(dev).requires_grad_(True)
    w = _seeded(7, shape[-1]).to(dev).requires_grad_(True)  # tests.py:149: weight ~ N(0,1)
    dy = _seeded(8, *shape).to(dev)
    y = F.mean_error_norm(x, w)
    ref, mu = O.mean_error_norm_fwd(x, w)
    assert_rel(y, ref, 1e-5, "norm fwd")
    y.backward(dy)
    dx, dw = O.mean_error_norm_bwd(dy, x, w, mu.float())
    assert max(max_abs(x.grad, dx), max_abs(w.grad, dw) / max(1.0, float(dw.abs().max()))) < 1e-3
    assert_rel(x.grad, dx, 1e-5, "norm dx", floor_frac=1e-5)
    assert_rel(w.grad, dw, 1e-5, "norm dw", floor_frac=1e-5)


# ------------------------------------------------- config-2 full sizes ----

def _row_sample(n_rows, k=192, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(n_rows, generator=g)[:k].sort().values


def test_norm_config2_bf16(gpu):
    # x [16384, 4096] ~ N(0,1) bf16, gamma = 1 + 0.02 N(0,1) fp32, dy ~ N(0,1)
    N, C = 16384, 4096
    x = _seeded(10, N, C, dtype=torch.bfloat16).to(dev).requires_grad_(True)
    w = (1 + 0.02 * _seeded(11, C)).to(dev).requires_grad_(True)
    dy = _seeded(12, N, C, dtype=torch.bfloat16).to(dev)
    y = F.mean_error_norm(x, w)
    y.backward(dy)
    rows = _row_sample(N)
    xs = x.detach()[rows.to(dev)].cpu()
    ref, mu = O.mean_error_norm_fwd(xs, w.detach().cpu())
    assert_bf16_within_ulp(y.detach()[rows.to(dev)], ref, what="norm fwd rows")
    dx, _ = O.mean_error_norm_bwd(dy[rows.to(dev)].cpu(), xs, w.detach().cpu(), mu.float())
    assert_bf16_within_ulp(x.grad[rows.to(dev)], dx, abs_floor=1e-3 * float(dx.abs().max()),
                           what="norm dx rows")
    # dgamma sums over all rows: fp64 reduction over the full matrix, chunked
    _, mu_all = O.mean_error_norm_fwd(x.detach().cpu(), w.detach().cpu())
    dw = torch.zeros(C, dtype=torch.float64)
    for r0 in range(0, N, 2048):
        sl = slice(r0, r0 + 2048)
        dw += (dy[sl].cpu().double() * x.detach()[sl].cpu().double() /
               (mu_all[sl].float().double().unsqueeze(1) + 1e-6)).sum(0)
    assert_rel(w.grad, dw, 1e-4, "norm dgamma full", floor_frac=1e-4)


def test_swiglu_config2_bf16(gpu):
    N, C = 16384, 11008
    g = _seeded(20, N, C, dtype=torch.bfloat16).to(dev).requires_grad_(True)
    v = _seeded(21, N, C, dtype=torch.bfloat16).to(dev).requires_grad_(True)
    dy = _seeded(22, N, C, dtype=torch.bfloat16).to(dev)
    out = F.rational_swiglu(g, v)
    out.backward(dy)
    rows = _row_sample(N).to(dev)
    gs, vs, ys = g.detach()[rows].cpu(), v.detach()[rows].cpu(), dy[rows].cpu()
    assert_bf16_within_ulp(out.detach()[rows], O.swiglu_fwd(gs, vs), what="swiglu fwd rows")
    dg, dv = O.swiglu_bwd(ys, gs, vs)
    assert_bf16_within_ulp(g.grad[rows], dg, what="swiglu dgate rows")
    assert_bf16_within_ulp(v.grad[rows], dv, what="swiglu dvalue rows")


def test_softmax_config2_bf16(gpu):
    N, C = 4096, 4096
    x = (_seeded(30, N, C) * 2).to(torch.bfloat16).to(dev).requires_grad_(True)  # N(0, 4)
    dy = _seeded(31, N, C, dtype=torch.bfloat16).to(dev)
    p = F.rational_softmax(x)
    p.backward(dy)
    rows = _row_sample(N).to(dev)
    xs = x.detach()[rows].cpu()
    assert_bf16_within_ulp(p.detach()[rows], O.rational_softmax_fwd(xs), what="softmax fwd rows")
    ref = O.rational_softmax_bwd(dy[rows].cpu(), xs, p.detach()[rows].cpu())
    assert_bf16_within_ulp(x.grad[rows], ref, abs_floor=1e-3 * float(ref.abs().max()),
                           what="softmax bwd rows")


# ------------------------------------------------------- layouts, edges ----

@pytest.mark.parametrize("dtype,f", [(torch.bfloat16, 264), (torch.bfloat16, 2048),
                                     (torch.float32, 1024), (torch.float32, 36)])
def test_swiglu_on_packed_chunks_matches_contiguous(gpu, dtype, f):
    # strided halves (row-indexed kernels: a general row length, and power-of-two
    # lengths, which index by shifts) against the flat launch over contiguous
    # copies, forward and backward
    gv = _seeded(40 + f, 3, 50, 2 * f, dtype=dtype).to(dev)
    dy = _seeded(41 + f, 3, 50, f, dtype=dtype).to(dev)
    ga, va = (t.detach().requires_grad_(True) for t in gv.chunk(2, dim=-1))
    gb, vb = (t.detach().contiguous().requires_grad_(True) for t in gv.chunk(2, dim=-1))
    a = F.rational_swiglu(ga, va)
    b = F.rational_swiglu(gb, vb)
    assert torch.equal(a, b)
    a.backward(dy)
    b.backward(dy)
    assert torch.equal(ga.grad, gb.grad) and torch.equal(va.grad, vb.grad)


@pytest.mark.parametrize("dtype,f", [(torch.bfloat16, 263), (torch.float16, 5461),
                                     (torch.float32, 37)])
def test_swiglu_odd_packed_halves_match_oracle(gpu, dtype, f):
    # an odd d_ffn: the value half of the packed [rows, 2F] buffer is only
    # element-aligned, so the scalar kernels run (2D grid, rows past 65535
    # walked in a loop -- 70000 rows here), forward and backward
    rows = 70000 if f < 300 else 40
    gv = _seeded(70 + f, rows, 2 * f, dtype=dtype).to(dev)
    dy = _seeded(71 + f, rows, f, dtype=dtype).to(dev)
    gvr = gv.clone().requires_grad_(True)
    out = F.rational_swiglu_packed(gvr)
    out.backward(dy)
    g, v = gv.chunk(2, dim=-1)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert_rel(out, O.swiglu_fwd(g.cpu(), v.cpu()), tol, "swiglu odd fwd", floor_frac=tol)
    dg, dv = O.swiglu_bwd(dy.cpu(), g.cpu(), v.cpu())
    assert_rel(gvr.grad[..., :f], dg, tol, "swiglu odd dgate", floor_frac=tol)
    assert_rel(gvr.grad[..., f:], dv, tol, "swiglu odd dvalue", floor_frac=tol)


@pytest.mark.parametrize("cols", [1, 7, 13, 100, 1000, 9000, 20000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_odd_and_wide_rows(gpu, cols, dtype):
    rows = 5
    x = _seeded(50 + cols, rows, cols, dtype=dtype).to(dev).requires_grad_(True)
    dy = _seeded(51 + cols, rows, cols, dtype=dtype).to(dev)
    w = (1 + 0.1 * _seeded(52, cols)).to(dev)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    p = F.rational_softmax(x)
    assert_rel(p, O.rational_softmax_fwd(x), tol, f"softmax {cols}", floor_frac=tol)
    p.backward(dy)
    # dx = p g (dy - <dy,p>) cancels when a row has one dominant entry (e.g.
    # cols = 1, where 1 - p ~ eps / f): bound the error by the size of the
    # terms before cancellation, p g (|dy| + |<dy,p>|)
    pd, xd, yd = p.detach().cpu().double(), x.detach().cpu().double(), dy.cpu().double()
    den = xd.abs() + 1
    gg = 2 / (den * den * (0.5 * (xd / den + 1) + 1e-6))
    terms = pd * gg * (yd.abs() + (yd * pd).sum(-1, keepdim=True).abs())
    ref_dx = O.rational_softmax_bwd(dy, x, p.detach())
    err = (x.grad.cpu().double() - ref_dx).abs()
    # plus one ulp of the output dtype for the final rounding
    # (fp16 subnormals below 2^-14 have the fixed spacing 2^-24)
    mant, emin = {torch.float32: (23, -126), torch.bfloat16: (7, -126),
                  torch.float16: (10, -14)}[dtype]
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref_dx.abs().clamp_min(2.0 ** emin))) - mant)
    assert bool((err <= tol * terms + ulp).all()), f"softmax bwd {cols}: {float(err.max()):.3e}"
    y = F.mean_error_norm(x.detach(), w)
    assert_rel(y, O.mean_error_norm_fwd(x, w)[0], tol, f"norm {cols}", floor_frac=tol)
    s = F.rational_swiglu(x.detach(), dy)
    assert_rel(s, O.swiglu_fwd(x, dy), tol, f"swiglu {cols}", floor_frac=tol)


def test_empty_inputs(gpu):
    x = torch.empty(0, 64, device=dev, requires_grad=True)
    p = F.rational_softmax(x)
    p.sum().backward()
    assert p.shape == (0, 64) and x.grad.shape == (0, 64)
    w = torch.ones(64, device=dev, requires_grad=True)
    y = F.mean_error_norm(x, w)
    y.sum().backward()
    assert torch.equal(w.grad, torch.zeros(64, device=dev))


def test_norm_bwd_is_deterministic(gpu):
    x = _seeded(60, 4096, 2048).to(dev).requires_grad_(True)
    w = torch.ones(2048, device=dev, requires_grad=True)
    dy = _seeded(61, 4096, 2048).to(dev)
    grads = []
    for _ in range(2):
        x.grad = w.grad = None
        F.mean_error_norm(x, w).backward(dy)
        grads.append((x.grad.clone(), w.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


def test_fp64_gradcheck(gpu):
    # reference tests.py:219-272 (fp64 gradcheck; eps 1e-6, atol 1e-4, rtol 1e-3)
    g = torch.Generator().manual_seed(70)
    x = torch.randn(2, 4, 16, 16, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: F.RationalSoftmax.apply(t, 1e-6), (x,), eps=1e-6,
                                    atol=1e-4, rtol=1e-3)
    a = torch.randn(2, 16, 32, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    b = torch.randn(2, 16, 32, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(F.RationalSwiGLU.apply, (a, b), eps=1e-6, atol=1e-4,
                                    rtol=1e-3)
    x = torch.randn(2, 16, 32, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    w = torch.randn(32, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t, u: F.MeanErrorNorm.apply(t, u, 1e-6), (x, w),
                                    eps=1e-6, atol=1e-4, rtol=1e-3)


def test_native_library_is_loaded(gpu):
    import os
    maps = open("/proc/self/maps").read()
    assert "libkat.so" in maps
    hip = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len(hip) == 1, f"more than one HIP runtime mapped: {hip}"
    assert os.path.basename(F._lib.LIB_PATH) == "libkat.so"
