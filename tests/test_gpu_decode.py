"""Decode attention over a KV cache (kat_attn_decode via
rational_attention_decode) and the model's cached generate().

The decode result is, by definition, the last row of the causal attention over
the cached keys -- what the reference's generate() recomputes over the whole
prefix (algebraic_model.py:239-265) -- so it is checked against that row of the
oracle (pinned in test_oracle.py) and of the causal kernels. Tolerances:
fp32 <= 1e-5 of max|ref| on o (L 1e-5 relative); bf16 / fp16
|got - ref| <= 2e-2 + 1/2 ulp(ref) and relative L2 <= 5e-3 on o, L within
1e-4 relative (fp32 sums of the same rounded inputs)."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from test_gpu_attention import _rel_max, assert_lowp

pytestmark = pytest.mark.gpu
dev = "cuda"


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(dev)


def _oracle_last_row(q, kc, vc, slopes, scale, n):
    """Row n-1 of the oracle's causal attention over keys 0..n-1 with query q."""
    B, H, D = q.shape
    qfull = torch.zeros(B, H, n, D, dtype=torch.float64)
    qfull[:, :, n - 1] = q.double().cpu()
    o, L = O.attention_fwd(qfull, kc[:, :, :n], vc[:, :, :n], slopes, scale,
                           dtype=torch.float32 if q.dtype != torch.float32 else torch.float64)
    return o[:, :, n - 1], L[:, :, n - 1]


# the layout widths, and head dims between them (fp32: multiples of 4 up to
# 128; bf16 / fp16: multiples of 8 up to 256), whose columns past D are the
# next head's data in the token-major caches below
CASES = [(torch.float32, 32), (torch.float32, 64), (torch.float32, 128), (torch.bfloat16, 64),
         (torch.bfloat16, 128), (torch.bfloat16, 256), (torch.float16, 128), (torch.float32, 20),
         (torch.float32, 100), (torch.bfloat16, 8), (torch.bfloat16, 96), (torch.float16, 200)]


@pytest.mark.parametrize("n", [1, 5, 200, 1000])
@pytest.mark.parametrize("dtype,D", CASES)
def test_decode_matches_oracle_last_row(gpu, dtype, D, n):
    B, H, Tmax = 2, 3, 1030
    q = _rand((B, H, D), dtype, n + D)
    # token-major caches [B, Tmax, H, D], viewed as [B, H, n, D]
    kt = _rand((B, Tmax, H, D), dtype, n + D + 1)
    vt = _rand((B, Tmax, H, D), dtype, n + D + 2)
    kc, vc = kt[:, :n].permute(0, 2, 1, 3), vt[:, :n].permute(0, 2, 1, 3)
    slopes = F.compute_alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L = F.rational_attention_decode(q, kc, vc, slopes.to(dev), scale)
    torch.cuda.synchronize()
    ro, rL = _oracle_last_row(q, kc.cpu(), vc.cpu(), slopes, scale, n)
    if dtype == torch.float32:
        assert _rel_max(o, ro) <= 1e-5
        assert _rel_max(L, rL) <= 1e-5
    else:
        assert_lowp(o, ro, dtype, "o")
        assert _rel_max(L, rL) <= 1e-4


def test_decode_ragged_lengths(gpu):
    B, H, T, D = 4, 2, 300, 128
    dtype = torch.bfloat16
    q = _rand((B, H, D), dtype, 1)
    kc = _rand((B, H, T, D), dtype, 2)
    vc = _rand((B, H, T, D), dtype, 3)
    lengths = torch.tensor([300, 1, 0, 171], dtype=torch.int32, device=dev)
    slopes = F.compute_alibi_slopes(H)
    o, L = F.rational_attention_decode(q, kc, vc, slopes.to(dev), 0.09, lengths=lengths)
    torch.cuda.synchronize()
    for b, n in enumerate(lengths.tolist()):
        if n == 0:  # nothing cached: L = 0, o = 0
            assert torch.equal(L[b].cpu(), torch.zeros(H))
            assert torch.equal(o[b].float().cpu(), torch.zeros(H, D))
            continue
        ro, rL = _oracle_last_row(q[b:b + 1], kc[b:b + 1].cpu(), vc[b:b + 1].cpu(), slopes, 0.09, n)
        assert_lowp(o[b:b + 1], ro, dtype, f"o[{b}]")
        assert _rel_max(L[b:b + 1], rL) <= 1e-4


def test_decode_matches_causal_kernel_last_row(gpu, monkeypatch):
    # the MFMA causal kernel and the decode kernel on one sequence: row T-1
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, H, T, D = 2, 4, 777, 128
    q, k, v = (_rand((B, H, T, D), torch.bfloat16, s) for s in (4, 5, 6))
    slopes = F.compute_alibi_slopes(H).to(dev)
    o_full, L_full = F.rational_attention_forward(q, k, v, slopes, 0.088)
    o, L = F.rational_attention_decode(q[:, :, -1].contiguous(), k, v, slopes, 0.088)
    torch.cuda.synchronize()
    assert _rel_max(L, L_full[:, :, -1]) <= 1e-3
    err = (o.double() - o_full[:, :, -1].double()).abs()
    assert float(err.max()) <= 2e-2


def test_decode_is_deterministic(gpu):
    B, H, T, D = 1, 2, 4096, 128
    q = _rand((B, H, D), torch.bfloat16, 7)
    kc = _rand((B, H, T, D), torch.bfloat16, 8)
    vc = _rand((B, H, T, D), torch.bfloat16, 9)
    slopes = F.compute_alibi_slopes(H).to(dev)
    a = F.rational_attention_decode(q, kc, vc, slopes, 0.088)
    b = F.rational_attention_decode(q, kc, vc, slopes, 0.088)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ----------------------------------------------------------------- model ----

def _small_model(seed, **kw):
    torch.manual_seed(seed)
    return F.AlgebraicTransformerLM(vocab_size=500, d_model=128, n_head=2, n_layers=2,
                                    dropout=0.0, **kw).cuda().eval()


def test_cached_logits_match_full_forward(gpu):
    m = _small_model(0)
    ids = torch.randint(0, 500, (2, 40), device=dev)
    with torch.no_grad():
        full, _ = m(ids)
        caches = m.new_kv_caches(40)
        pre = m.forward_cached(ids[:, :25], caches, 0)
        rows = [pre] + [m.forward_cached(ids[:, i:i + 1], caches, i) for i in range(25, 40)]
    got = torch.cat(rows, dim=1)
    assert got.shape == full.shape
    err = float((got - full).abs().max())
    assert err <= 1e-4 * max(1.0, float(full.abs().max())), err


def test_cached_generate_matches_uncached_greedy(gpu):
    m = _small_model(1, block_size=64)
    prompt = torch.randint(0, 500, (2, 11), device=dev)
    torch.manual_seed(5)
    a = m.generate(prompt, 20, top_k=1)
    torch.manual_seed(5)
    b = m.generate(prompt, 20, top_k=1, use_cache=False)
    assert a.shape == (2, 31) and torch.equal(a, b)


def test_cached_generate_past_block_size(gpu):
    # the context outgrows block_size: the reference crops it from then on
    m = _small_model(2, block_size=16)
    prompt = torch.randint(0, 500, (1, 10), device=dev)
    torch.manual_seed(6)
    a = m.generate(prompt, 14, top_k=1)
    torch.manual_seed(6)
    b = m.generate(prompt, 14, top_k=1, use_cache=False)
    assert torch.equal(a, b)


def test_cached_generate_bf16_autocast_runs(gpu):
    m = _small_model(3)
    prompt = torch.randint(0, 500, (3, 9), device=dev)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = m.generate(prompt, 8, temperature=0.8, top_k=50)
    assert out.shape == (3, 17) and torch.equal(out[:, :9], prompt)
    assert int(out.min()) >= 0 and int(out.max()) < 500


def test_decode_graph_replays_match_eager_steps(gpu):
    # the captured one-token step against the same step run eagerly, position
    # by position, with unrelated eager work and synchronisations between the
    # replays (every replay checked)
    from fastalgebraictransformer_amd.algebraic_model import _DecodeStep
    m = _small_model(4)
    ids = torch.randint(0, 500, (3, 30), device=dev)
    with torch.no_grad():
        caches = m.new_kv_caches(30)
        m.forward_cached(ids[:, :20], caches, 0)
        eager = _DecodeStep(m, caches, 3, ids.device, use_graph=False)
        graph = _DecodeStep(m, caches, 3, ids.device, use_graph=True)
        for pos in range(20, 30):
            a = eager(ids[:, pos:pos + 1], pos).clone()
            torch.cuda.synchronize()
            junk = torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)
            b = graph(ids[:, pos:pos + 1], pos).clone()
            torch.cuda.synchronize()
            assert torch.equal(a, b), pos
            del junk
        full, _ = m(ids)
    assert float((b - full[:, -1]).abs().max()) <= 1e-4 * max(1.0, float(full.abs().max()))


@pytest.mark.parametrize("autocast", [False, True])
def test_generate_graph_matches_eager_cache(gpu, autocast):
    m = _small_model(5, block_size=48)
    prompt = torch.randint(0, 500, (2, 13), device=dev)
    outs = []
    for use_graph in (True, False):
        torch.manual_seed(9)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            outs.append(m.generate(prompt, 24, top_k=1, use_graph=use_graph))
    assert torch.equal(outs[0], outs[1])
    if not autocast:
        torch.manual_seed(9)
        ref = m.generate(prompt, 24, top_k=1, use_cache=False)
        assert torch.equal(outs[0], ref)
