"""The model configurations of the benchmark on the GPU path, against the
reference formulation (BASELINE configs 4 and 5):

  * config 4, AlgebraicTransformerLM(32000, 768, 12, 12) at batch 16 x 2048
    under bf16 autocast: one AlgebraicBlock(768, 12, d_ffn 2048) at the real
    sequence length on a 2-row batch slice against the same block's fp32 CPU
    path (the reference's CPU attention with its -1e4 causal fill, torch norm
    and SwiGLU formulas: algebraic_model.py:26-62, 112-152), and the full
    training step (finite, loss at the uniform-prediction level);
  * config 5, AlgebraicTransformerLM(50000, 2048, 16, 24, d_ffn=5632) at
    2 x 8192: its packed attention [2, 8192, 3, 16, 128] on sampled heads
    against the fp32 oracle, its fused residual norm [16384, 2048] and packed
    SwiGLU [16384, 2 x 5632] against the oracle on sampled rows, and the full
    training step.

Bars: attention as test_gpu_attention.py (2e-2 + 1/2 ulp, relative L2 <=
5e-3); norm / SwiGLU outputs within 1 bf16 ulp of the oracle (fp32 residual
stream exact); the block under autocast (whose GEMMs round both operands to
bf16, 2^-9 relative each) within 2e-2 relative L2 of the fp32 block, on the
block's increment (output minus input) and every gradient."""

import copy
import math

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import assert_bf16_within_ulp, assert_rel, check_lowp

pytestmark = pytest.mark.gpu


def _seeded(seed, *shape, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def _rel_l2(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return float((got - ref).norm() / ref.norm())


def test_config4_block_autocast_vs_cpu_fp32(gpu):
    torch.manual_seed(4)
    blk = F.AlgebraicBlock(768, 12, 2048, dropout=0.0)
    x = _seeded(40, 2, 2048, 768)
    dy = _seeded(41, 2, 2048, 768)
    xc = x.clone().requires_grad_(True)
    yc = blk(xc)
    yc.backward(dy)
    gblk = copy.deepcopy(blk).cuda()
    gblk.zero_grad(set_to_none=True)
    xg = x.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yg = gblk(xg)
    yg.float().backward(dy.cuda())
    torch.cuda.synchronize()
    res = {"increment": _rel_l2(yg.float() - xg, yc - xc),
           "dx increment": _rel_l2(xg.grad - dy.cuda(), xc.grad - dy)}
    for (n, pc), (_, pg) in zip(blk.named_parameters(), gblk.named_parameters()):
        res[n] = _rel_l2(pg.grad, pc.grad)
    print("config-4 block, relative L2 vs fp32 CPU: " +
          ", ".join(f"{n} {v:.2e}" for n, v in res.items()))
    for n, v in res.items():
        assert v <= 2e-2, (n, v)


def _model_step(vocab, d, h, layers, d_ffn, B, S, seed):
    torch.manual_seed(seed)
    with torch.device("cuda"):
        m = F.AlgebraicTransformerLM(vocab, d, h, layers, d_ffn=d_ffn, block_size=S)
    m.train()
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (B, S), generator=g).cuda()
    labels = torch.randint(0, vocab, (B, S), generator=g).cuda()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = m(ids, labels)
    loss.backward()
    torch.cuda.synchronize()
    lv = float(loss)
    # random init (N(0, 0.02) weights): near-uniform predictions, loss ~ ln(vocab)
    assert math.isfinite(lv) and abs(lv - math.log(vocab)) < 1.0, lv
    for n, p in m.named_parameters():
        assert p.grad is not None and bool(torch.isfinite(p.grad).all()), n
    del m
    torch.cuda.empty_cache()
    return lv


def test_config4_full_training_step(gpu):
    _model_step(32000, 768, 12, 12, None, 16, 2048, 44)


def test_config5_full_training_step(gpu):
    _model_step(50000, 2048, 16, 24, 5632, 2, 8192, 55)


def test_config5_packed_attention_sampled_heads(gpu, monkeypatch):
    # the 1.3B model's attention call: qkv [2, 8192, 3, 16, 128] bf16 (its own
    # ALiBi slopes), fwd + bwd on the GPU, three (b, h) heads against the oracle
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, T, H, D = 2, 8192, 16, 128
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    qkv = _seeded(50, B, T, 3, H, D, dtype=torch.bfloat16).cuda().requires_grad_(True)
    dy = _seeded(51, B, T, H, D, dtype=torch.bfloat16).cuda()
    y = F.rational_attention_packed(qkv, slopes.cuda(), scale)
    y.backward(dy)
    torch.cuda.synchronize()
    q, k, v = qkv.detach().permute(2, 0, 3, 1, 4)
    o = y.detach().permute(0, 2, 1, 3)
    do = dy.permute(0, 2, 1, 3)
    gq, gk, gv = qkv.grad.permute(2, 0, 3, 1, 4)
    for b, h in ((0, 0), (1, 7), (1, 15)):
        sl = lambda t: t[b:b + 1, h:h + 1]  # noqa: E731
        ro, rL = O.attention_fwd(sl(q), sl(k), sl(v), slopes[h:h + 1], scale, dtype=torch.float32)
        res = {"o": check_lowp(sl(o), ro, torch.bfloat16, f"o ({b},{h})")}
        rq, rk, rv = O.attention_bwd(sl(q), sl(k), sl(v), sl(o), rL, sl(do), slopes[h:h + 1], scale,
                                     dtype=torch.float32)
        for n, got, ref in (("dq", gq, rq), ("dk", gk, rk), ("dv", gv, rv)):
            res[n] = check_lowp(sl(got), ref, torch.bfloat16, f"{n} ({b},{h})")
        print(f"config 5 head ({b},{h}): " + ", ".join(
            f"{n} max err {e:.3e} relL2 {r:.3e}" for n, (e, r) in res.items()))


def _rows(n, k=256, seed=0):
    return torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:k].sort().values


def test_config5_fused_norm(gpu):
    # the model's pre-norm under autocast: fp32 residual stream x plus a bf16
    # branch r, normed output in bf16 (add_mean_error_norm), [2 x 8192, 2048]
    N, C = 16384, 2048
    x = _seeded(52, N, C).cuda().requires_grad_(True)
    r = _seeded(53, N, C, dtype=torch.bfloat16).cuda().requires_grad_(True)
    w = (1 + 0.02 * _seeded(54, C)).cuda().requires_grad_(True)
    dh = _seeded(55, N, C).cuda()
    dy = _seeded(56, N, C, dtype=torch.bfloat16).cuda()
    h, y = F.add_mean_error_norm(x, r, w, 1e-6, torch.bfloat16)
    torch.autograd.backward([h, y], [dh, dy])
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and h.dtype == torch.float32
    rows = _rows(N).cuda()
    hs = (x.detach()[rows] + r.detach()[rows].float()).cpu()
    assert torch.equal(h.detach()[rows].cpu(), hs)
    ry, mu = O.mean_error_norm_fwd(hs, w.detach().cpu())
    assert_bf16_within_ulp(y.detach()[rows], ry, what="config-5 norm y")
    dx, _ = O.mean_error_norm_bwd(dy[rows].cpu(), hs, w.detach().cpu(), mu.float())
    dx = dx + dh[rows].cpu().double()
    assert_rel(x.grad[rows], dx, 1e-5, "config-5 norm dx", floor_frac=1e-5)
    # dr is dx rounded to bf16; where norm_bwd and dh cancel, dx keeps fp32's
    # absolute accuracy (~1e-7 of its terms), hence the same floor as dx
    assert_bf16_within_ulp(r.grad[rows], dx, abs_floor=1e-5 * float(dx.abs().max()),
                           what="config-5 norm dr")
    # dgamma over every row, fp64
    hf = (x.detach() + r.detach().float()).double()
    muf = hf.abs().mean(dim=1, keepdim=True).float().double()
    dw = (dy.double() * hf / (muf + 1e-6)).sum(0).cpu()
    assert_rel(w.grad, dw, 1e-4, "config-5 norm dgamma", floor_frac=1e-4)


def test_config5_packed_swiglu(gpu):
    N, Fd = 16384, 5632
    gv = _seeded(57, N, 2 * Fd, dtype=torch.bfloat16).cuda().requires_grad_(True)
    dy = _seeded(58, N, Fd, dtype=torch.bfloat16).cuda()
    out = F.rational_swiglu_packed(gv)
    out.backward(dy)
    torch.cuda.synchronize()
    rows = _rows(N, seed=1).cuda()
    g, v = gv.detach()[rows].chunk(2, dim=-1)
    g, v = g.cpu(), v.cpu()
    assert_bf16_within_ulp(out.detach()[rows], O.swiglu_fwd(g, v), what="config-5 swiglu")
    dg, dvv = O.swiglu_bwd(dy[rows].cpu(), g, v)
    assert_bf16_within_ulp(gv.grad[rows][:, :Fd], dg, what="config-5 swiglu dgate")
    assert_bf16_within_ulp(gv.grad[rows][:, Fd:], dvv, what="config-5 swiglu dvalue")
