"""GPU parity of attention with a key padding mask and a real non-causal mode
(rational_attention_masked -> kat_attn_fwd_masked / kat_attn_bwd_masked)
against the CPU oracle (oracle.attention_fwd / attention_bwd with key_mask /
causal, pinned in test_oracle.py to the reference model's CPU attention,
algebraic_model.py:112-136). Tolerances as in test_gpu_attention.py:
  * fp32 (tiled kernels): <= 1e-5 of max|ref| on o, L, dq, dk, dv;
  * bf16 / fp16: |got - ref| <= 2e-2 + 1/2 ulp(ref) elementwise and relative
    L2 <= 5e-3 on o, dq, dk, dv; L within 1e-2 relative.
Exact properties on top: dropped keys get dk = dv = 0, queries with no visible
key get o = 0, L = 0, dq = 0, and an all-ones mask reproduces the unmasked
call bit for bit."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import max_abs
from test_gpu_attention import _rel_max, assert_lowp

pytestmark = pytest.mark.gpu
dev = "cuda"


def _inputs(seed, B, H, T, D, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g).to(dtype).to(dev) for _ in range(4)]


def _mask(kind, B, T, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "none":
        return None
    m = torch.ones(B, T, dtype=torch.int32)
    if kind == "random":
        m = (torch.rand(B, T, generator=g) > 0.3).to(torch.int32)
        m[0, : T // 3] = 0                 # left padding: early queries see no key
    elif kind == "right":
        for b in range(B):                 # right padding of a different length per row
            m[b, T - (T * (b + 1)) // (B + 2):] = 0
    elif kind == "tiles":
        m[:, 64:192] = 0                   # whole 64-key tiles dropped, plus mixed tiles
        m[:, 5::7] = 0
    if B > 1 and kind != "right":
        m[B - 1, -(T // 4):] = 0
    return m.to(dev)


def _run(q, k, v, do, slopes, scale, km, causal):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = F.rational_attention_masked(q, k, v, slopes, scale, key_mask=km, causal=causal)
    o.backward(do)
    # L from the forward entry point itself (same kernels)
    from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg
    B, H, T, D = q.shape
    o2 = torch.empty_like(o)
    L = torch.empty(B, H, T, device=dev)
    _attn_fwd_into(q.detach(), k.detach(), v.detach(), o2, L, slopes, scale, causal, O.EPS,
                   _key_mask_arg(km, B, T, q.device), extended=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    return o.detach(), L, q.grad, k.grad, v.grad


def _exact_properties(o, L, dq, dk, dv, km, causal):
    if km is None:
        return
    kmc = km.cpu() != 0
    drop = ~kmc[:, None, :, None].expand(dk.shape)
    assert torch.equal(dk.cpu()[drop], torch.zeros_like(dk.cpu()[drop])), "dk of dropped keys"
    assert torch.equal(dv.cpu()[drop], torch.zeros_like(dv.cpu()[drop])), "dv of dropped keys"
    T = kmc.shape[1]
    seen = kmc.cumsum(1) > 0 if causal else kmc.any(1, keepdim=True).expand(-1, T)
    blind = ~seen[:, None, :].expand(L.shape)
    if bool(blind.any()):
        assert torch.equal(L.cpu()[blind], torch.zeros_like(L.cpu()[blind]))
        ob = blind[..., None].expand(o.shape)
        assert torch.equal(o.cpu()[ob], torch.zeros_like(o.cpu()[ob]))
        assert torch.equal(dq.cpu()[ob], torch.zeros_like(dq.cpu()[ob]))


KINDS = ["none", "random", "right", "tiles"]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("B,H,T,D", [(2, 3, 77, 32), (3, 2, 260, 64), (1, 2, 1, 20)])
def test_masked_fp32(gpu, B, H, T, D, kind, causal):
    q, k, v, do = _inputs(T + D, B, H, T, D, torch.float32)
    km = _mask(kind, B, T, T)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale, km, causal)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, causal=causal, key_mask=km)
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, causal=causal, key_mask=km)
    assert _rel_max(o, ro) <= 1e-5 and _rel_max(L, rL) <= 1e-5
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        # 1e-5 of max|ref|, with a 1e-6 absolute floor: at T = 1 the exact dq
        # is the cancellation dP - Delta = (dO.v) eps / (f + eps) ~ 1e-4, far
        # below the O(1) terms whose fp32 rounding (~1e-7) it inherits
        err = max_abs(got, ref)
        assert err <= 1e-5 * float(ref.abs().max()) + 1e-6, (name, err)
    _exact_properties(o, L, dq, dk, dv, km, causal)


@pytest.mark.parametrize("impl", ["mfma", "tiled"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype,B,H,T,D", [(torch.bfloat16, 2, 2, 333, 128),
                                           (torch.float16, 3, 2, 200, 64),
                                           (torch.bfloat16, 2, 1, 1, 64),
                                           (torch.bfloat16, 1, 2, 700, 64),
                                           (torch.float16, 2, 3, 300, 32)])
def test_masked_lowp(gpu, dtype, B, H, T, D, kind, causal, impl, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", impl)
    q, k, v, do = _inputs(5 * T + D, B, H, T, D, dtype)
    km = _mask(kind, B, T, T + 1)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L, dq, dk, dv = _run(q, k, v, do, slopes.to(dev), scale, km, causal)
    ro, rL = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32, causal=causal,
                             key_mask=km)
    assert_lowp(o, ro, dtype, "o")
    assert _rel_max(L, rL) <= 1e-2, ("L", _rel_max(L, rL))
    rq, rk, rv = O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32,
                                 causal=causal, key_mask=km)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert_lowp(got, ref, dtype, name)
    _exact_properties(o, L, dq, dk, dv, km, causal)


@pytest.mark.parametrize("impl", ["mfma", "tiled"])
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_unmasked_and_all_ones_match_reference_entry_point(gpu, dtype, D, impl, monkeypatch):
    # fp32 with impl "mfma": the fp32 MFMA kernels (forward and recompute backward)
    monkeypatch.setenv("KAT_ATTN_IMPL", impl)
    B, H, T = 2, 3, 190
    q, k, v, do = _inputs(9, B, H, T, D, dtype)
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    results = []
    ones = torch.ones(B, T, dtype=torch.bool, device=dev)
    for which in ("no mask", "all ones", "reference"):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        if which == "reference":
            o = F.rational_attention(qq, kk, vv, slopes, scale)
        else:
            km = ones if which == "all ones" else None
            o = F.rational_attention_masked(qq, kk, vv, slopes, scale, key_mask=km)
        o.backward(do)
        results.append((o, qq.grad, kk.grad, vv.grad))
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert torch.equal(a, b)


def test_packed_with_mask_matches_views(gpu, monkeypatch):
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, T, H, D = 2, 150, 4, 64
    g = torch.Generator().manual_seed(21)
    base = torch.randn(B, T, 3, H, D, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    km = _mask("random", B, T, 3)
    slopes = F.compute_alibi_slopes(H).to(dev)
    qkv_p = base.clone().requires_grad_(True)
    y_p = F.rational_attention_packed(qkv_p, slopes, 0.125, key_mask=km)
    y_p.backward(dy)
    qkv_r = base.clone().requires_grad_(True)
    q, k, v = qkv_r.permute(2, 0, 3, 1, 4)
    y_r = F.rational_attention_masked(q, k, v, slopes, 0.125, key_mask=km).transpose(1, 2)
    y_r.backward(dy)
    assert torch.equal(y_p, y_r)
    assert torch.equal(qkv_p.grad, qkv_r.grad)

