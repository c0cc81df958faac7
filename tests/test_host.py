"""Host-side logic of the Python API (CPU only, no kernel launches)."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from fastalgebraictransformer_amd import _lib


def test_public_names_match_reference_surface():
    # reference __init__.py:39-63
    expected = {
        "rational_softmax", "rational_swiglu", "mean_error_norm", "RationalSoftmax",
        "RationalSwiGLU", "MeanErrorNorm", "EPS", "rational_attention_forward",
        "compute_alibi_slopes", "rational_attention", "rational_attention_backward",
        "RationalAttentionFunction", "AlgebraicTransformerLM", "RationalMR",
        "AlgebraicAttention", "AlgebraicBlock", "create_small_model", "create_medium_model",
        "create_large_model"}
    assert set(F.__all__) == expected
    for n in expected:
        assert hasattr(F, n)
    assert F.RationalSwiGLUModule is F.algebraic_model.RationalSwiGLU
    assert F.EPS == 1e-6 and F.fused_ops.NEG_INF == -1e4


def test_install_as_reference_name():
    F.install_as("kernels")
    from kernels.backward import rational_attention  # noqa: F401
    from kernels.fused_ops import rational_softmax
    assert rational_softmax is F.rational_softmax


def test_alibi_slopes_match_oracle_bitwise():
    for n in (1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 48):
        assert torch.equal(F.compute_alibi_slopes(n), O.alibi_slopes(n))
    assert F.compute_alibi_slopes(4, device="cpu").device.type == "cpu"


def test_autograd_functions_reject_cpu_tensors():
    x = torch.randn(2, 8)
    with pytest.raises(AssertionError):
        F.RationalSoftmax.apply(x, 1e-6)
    with pytest.raises(AssertionError):
        F.RationalSwiGLU.apply(x, x)
    with pytest.raises(AssertionError):
        F.MeanErrorNorm.apply(x, torch.ones(8), 1e-6)
    q = torch.randn(1, 2, 4, 8)
    with pytest.raises(AssertionError):
        F.rational_attention_forward(q, q, q, torch.ones(2), 0.3)
    with pytest.raises(AssertionError):
        F.rational_attention(q, q, q, torch.ones(2), 0.3)


def test_cpu_functional_paths_follow_reference_formulas():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 40, generator=g, dtype=torch.float64)
    v = torch.randn(3, 5, 40, generator=g, dtype=torch.float64)
    w = torch.randn(40, generator=g, dtype=torch.float64)
    assert torch.allclose(F.rational_softmax(x), O.rational_softmax_fwd(x), rtol=1e-14, atol=0)
    assert torch.allclose(F.rational_swiglu(x, v), O.swiglu_fwd(x, v), rtol=1e-14, atol=0)
    assert torch.allclose(F.mean_error_norm(x, w), O.mean_error_norm_fwd(x, w)[0], rtol=1e-14,
                          atol=0)


def test_rows2d_views_without_copy():
    gv = torch.randn(2, 7, 2 * 48)
    gate, value = gv.chunk(2, dim=-1)
    g2, ld = _lib.rows2d(gate)
    assert ld == 96 and g2.shape == (14, 48) and g2.data_ptr() == gate.data_ptr()
    v2, ldv = _lib.rows2d(value)
    assert ldv == 96 and v2.data_ptr() == value.data_ptr()
    t = torch.randn(6, 10).t()  # non-unit last-dim stride: copied
    t2, ldt = _lib.rows2d(t)
    assert ldt == 6 and t2.is_contiguous()
    e = torch.randn(1, 5).expand(4, 5)  # overlapping rows: copied
    e2, lde = _lib.rows2d(e)
    assert lde == 5 and e2.is_contiguous()
    s, lds = _lib.rows2d(torch.randn(9))
    assert s.shape == (1, 9) and lds == 9


def test_dtype_codes():
    assert _lib.dtype_code(torch.empty(1, dtype=torch.bfloat16)) == 1
    with pytest.raises(TypeError):
        _lib.dtype_code(torch.empty(1, dtype=torch.int32))


def test_model_cpu_path_matches_harness_attention():
    torch.manual_seed(0)
    m = F.AlgebraicTransformerLM(vocab_size=50, d_model=32, n_head=4, n_layers=2, dropout=0.0)
    ids = torch.randint(0, 50, (2, 9))
    logits, loss = m(ids, labels=ids)
    assert logits.shape == (2, 9, 50) and loss.ndim == 0 and math.isfinite(loss.item())
    loss.backward()
    assert all(p.grad is not None for p in m.parameters())
    # the attention module's CPU path is the reference harness formulation
    att = m.blocks[0].attn
    x = torch.randn(2, 9, 32)
    q, k, v = att.qkv(x).view(2, 9, 3, 4, 8).permute(2, 0, 3, 1, 4)
    ref = O.harness_attention(q, k, v, att.alibi_slopes, att.scale)
    got = att._cpu_attention(q, k, v, None)
    assert torch.allclose(got, ref.to(got.dtype), rtol=1e-5, atol=1e-6)


def test_model_state_dict_names_match_reference_layout():
    m = F.create_small_model(vocab_size=100)
    names = set(m.state_dict().keys())
    for n in ("embed.weight", "head.weight", "norm.weight", "blocks.0.attn.qkv.weight",
              "blocks.0.attn.out.weight", "blocks.0.attn.alibi_slopes",
              "blocks.0.ffn.w_gate_val.weight", "blocks.0.ffn.w_out.weight",
              "blocks.0.norm1.weight", "blocks.0.norm2.weight", "blocks.11.norm2.weight"):
        assert n in names, n
    assert m.embed.weight is m.head.weight
    assert m.blocks[0].ffn.w_gate_val.weight.shape == (2 * int(768 * 8 / 3), 768)


def test_model_residual_stream_matches_reference_block_structure():
    """The model carries the stream as (x, r) so that each residual add fuses
    into the next norm; on CPU that must equal the reference block
    `x = x + attn(norm1(x)); x = x + ffn(norm2(x))` (algebraic_model.py:149-152)
    followed by the final norm and head (:209-237) exactly."""
    torch.manual_seed(3)
    m = F.AlgebraicTransformerLM(vocab_size=40, d_model=32, n_head=4, n_layers=3, dropout=0.0)
    ids = torch.randint(0, 40, (2, 7))
    logits, _ = m(ids)
    x = m.embed(ids)
    for blk in m.blocks:
        x = x + blk.attn(blk.norm1(x))
        x = x + blk.ffn(blk.norm2(x))
    ref = m.head(m.norm(x))
    assert torch.equal(logits, ref)
    # a single block called directly keeps the reference's x -> x contract
    x0 = torch.randn(2, 7, 32)
    blk = m.blocks[1]
    h = x0 + blk.attn(blk.norm1(x0))
    assert torch.equal(blk(x0), h + blk.ffn(blk.norm2(h)))


def test_add_mean_error_norm_cpu_is_add_then_norm():
    x = torch.randn(5, 24)
    r = torch.randn(5, 24)
    w = torch.rand(24) + 0.5
    h, y = F.add_mean_error_norm(x, r, w)
    assert torch.equal(h, x + r)
    assert torch.equal(y, F.mean_error_norm(x + r, w))


def test_add_mean_error_norm_cpu_out_dtype_is_the_cast():
    x, r = torch.randn(4, 40), torch.randn(4, 40).to(torch.bfloat16)
    w = torch.rand(40) + 0.5
    h, y = F.add_mean_error_norm(x, r, w, out_dtype=torch.bfloat16)
    assert h.dtype == torch.float32 and y.dtype == torch.bfloat16
    assert torch.equal(y, F.mean_error_norm(x + r, w).to(torch.bfloat16))
    _, y32 = F.add_mean_error_norm(x, r, w, out_dtype=torch.float32)
    assert y32.dtype == torch.float32


def test_model_loss_matches_reference_shifted_cross_entropy():
    """The loss uses the full logits with the last position's target ignored;
    the reference slices logits[..., :-1, :] and labels[..., 1:]
    (algebraic_model.py:229-236). Same value (up to the order of the final
    mean) and the same gradient, including labels that are already -100."""
    torch.manual_seed(7)
    m = F.AlgebraicTransformerLM(vocab_size=37, d_model=16, n_head=2, n_layers=1, dropout=0.0)
    ids = torch.randint(0, 37, (3, 11))
    labels = ids.clone()
    labels[1, 4] = -100
    logits, loss = m(ids, labels=labels)
    lg = logits.detach().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(lg[..., :-1, :].contiguous().view(-1, 37),
                                            labels[..., 1:].contiguous().view(-1))
    assert math.isclose(loss.item(), ref.item(), rel_tol=1e-6)
    (g_ref,) = torch.autograd.grad(ref, lg)
    (g_got,) = torch.autograd.grad(loss, logits)
    assert torch.allclose(g_got, g_ref, rtol=1e-6, atol=1e-9)
    assert torch.equal(g_got[:, -1], torch.zeros_like(g_got[:, -1]))


def test_masked_attention_cpu_tensors_use_reference_cpu_formulation():
    # CPU tensors take the reference model's CPU attention (-1e4 fill)
    B, H, T, D = 2, 2, 9, 8
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(B, H, T, D, generator=g) for _ in range(3))
    km = torch.tensor([[1] * 9, [0, 1, 1, 0, 1, 1, 1, 1, 0]])
    slopes = F.compute_alibi_slopes(H)
    for causal in (True, False):
        got = F.rational_attention_masked(q, k, v, slopes, 0.3, key_mask=km, causal=causal)
        ref = O.harness_attention(q, k, v, slopes, 0.3, causal=causal, key_mask=km)
        assert torch.allclose(got, ref.to(got.dtype), rtol=1e-5, atol=1e-6)


def test_generate_cpu_follows_reference_loop():
    # CPU tensors take the reference loop (algebraic_model.py:239-265)
    torch.manual_seed(0)
    m = F.AlgebraicTransformerLM(vocab_size=30, d_model=16, n_head=2, n_layers=1, dropout=0.0,
                                 block_size=8).eval()
    prompt = torch.randint(0, 30, (2, 5))
    torch.manual_seed(1)
    out = m.generate(prompt, 6, temperature=0.7, top_k=5)
    torch.manual_seed(1)
    idx = prompt
    with torch.no_grad():
        for _ in range(6):
            ctx = idx if idx.size(1) <= 8 else idx[:, -8:]
            logits = m(ctx)[0][:, -1, :] / 0.7
            v, _ = torch.topk(logits, 5)
            logits[logits < v[:, [-1]]] = float("-inf")
            idx = torch.cat((idx, torch.multinomial(torch.softmax(logits, -1), 1)), dim=1)
    assert torch.equal(out, idx)


def test_tiled_fallback_reasons_mirror_the_mfma_limits():
    # the wrapper's warning predicts every fallback of a bf16 / fp16 call to
    # the tiled kernels: head dim, 16-byte rows, and 31-bit byte offsets
    # within a (b, h) slice (csrc/attn_mfma.hip offsets_ok: (T + 128) * row
    # stride * 2 bytes must stay below 2^31)
    from fastalgebraictransformer_amd.forward import _tiled_reason
    T, D = 4096, 128
    contiguous = [((16 * T * D, T * D, D), 0)]
    assert _tiled_reason(contiguous, D, T, 2) is None
    for Dm in (8, 48, 80, 96, 256):  # multiples of 8 up to 256
        assert _tiled_reason([((16 * T * Dm, T * Dm, Dm), 0)], Dm, T, 2) is None, Dm
    for Dt in (4, 100, 264, 512):
        assert f"head dim {Dt}" in _tiled_reason([((T * 512, T * 512, 512), 0)], Dt, T, 2), Dt
    # fp32 (4-byte elements): multiples of 4 up to 256
    for Dm in (4, 20, 100, 256):
        assert _tiled_reason([((16 * T * Dm, T * Dm, Dm), 0)], Dm, T, 4) is None, Dm
    for Dt in (2, 18, 260):
        assert f"head dim {Dt}" in _tiled_reason([((T * 512, T * 512, 512), 0)], Dt, T, 4), Dt
    assert "31-bit" in _tiled_reason([((T * 6144, 128, 6144), 0)], 128, 0x7FFFFFFF // (6144 * 4), 4)
    assert "16-byte" in _tiled_reason([((T * D, T * D, D), 8)], D, T, 2)
    assert "16-byte" in _tiled_reason([((T * D, T * D, D + 1), 0)], D, T, 2)
    # the model's packed qkv [B, T, 3, H, D] (H = 16, D = 128): row stride 6144
    st = 3 * 16 * 128
    packed = [((T * st, D, st), 0)]
    last_ok = (0x7FFFFFFF // (st * 2)) - 128
    assert _tiled_reason(packed, D, last_ok, 2) is None
    assert "31-bit" in _tiled_reason(packed, D, last_ok + 1, 2)
    # a row stride below D (overlapping rows) also leaves the MFMA kernels
    assert _tiled_reason([((T * D, T * D, 64), 0)], D, T, 2) is not None
