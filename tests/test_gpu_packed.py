"""The packed-layout entry points the model uses (attention on a [B, T, 3, H, D]
projection, SwiGLU on a [..., 2F] gate|value buffer) against the reference-API
calls on the corresponding views. Both run the same kernels on the same data,
so outputs and gradients must agree bit for bit."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F

pytestmark = pytest.mark.gpu


def _randn(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64), (torch.float32, 64),
                                     (torch.bfloat16, 96), (torch.float16, 40)])
@pytest.mark.parametrize("T", [1, 300])
def test_packed_attention_matches_views(gpu, dtype, D, T):
    B, H = 2, 3
    slopes = F.compute_alibi_slopes(H).cuda()
    scale = 1.0 / math.sqrt(D)
    base = _randn((B, T, 3, H, D), dtype, 5 + T + D)
    dy = _randn((B, T, H, D), dtype, 7 + T)

    qkv_p = base.clone().requires_grad_(True)
    y_p = F.rational_attention_packed(qkv_p, slopes, scale)
    assert y_p.shape == (B, T, H, D) and y_p.is_contiguous()
    y_p.backward(dy)

    qkv_r = base.clone().requires_grad_(True)
    q, k, v = qkv_r.permute(2, 0, 3, 1, 4)
    y_r = F.rational_attention(q, k, v, slopes, scale).transpose(1, 2)
    y_r.backward(dy)

    assert torch.equal(y_p, y_r)
    assert torch.equal(qkv_p.grad, qkv_r.grad)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,f", [(96, 2048), (33, 517)])
def test_packed_swiglu_matches_chunks(gpu, dtype, rows, f):
    base = _randn((rows, 2 * f), dtype, rows + f)
    dy = _randn((rows, f), dtype, rows * 3 + f)

    gv_p = base.clone().requires_grad_(True)
    out_p = F.rational_swiglu_packed(gv_p)
    out_p.backward(dy)

    gv_r = base.clone().requires_grad_(True)
    gate, value = gv_r.chunk(2, dim=-1)
    out_r = F.rational_swiglu(gate, value)
    out_r.backward(dy)

    assert torch.equal(out_p, out_r)
    assert torch.equal(gv_p.grad, gv_r.grad)


# ---------------------------------------------------- against the oracle ----
# The packed entry point is the model's attention path on the GPU; besides
# the bit-equality with the view-based calls above, it is checked directly
# against the fp32 oracle on its [B, T, 3, H, D] views, with and without a
# key padding mask, at the bar of test_gpu_attention.py (2e-2 + 1/2 ulp
# elementwise, relative L2 <= 5e-3).

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 96])
@pytest.mark.parametrize("masked", [False, True])
def test_packed_attention_vs_oracle(gpu, dtype, D, masked, monkeypatch):
    import oracle as O
    from _util import check_lowp
    monkeypatch.setenv("KAT_ATTN_IMPL", "mfma")
    B, T, H = 2, 333, 3
    slopes = F.compute_alibi_slopes(H).cuda()
    scale = 1.0 / math.sqrt(D)
    qkv = _randn((B, T, 3, H, D), dtype, 61 + D).requires_grad_(True)
    dy = _randn((B, T, H, D), dtype, 62 + D)
    km = None
    if masked:
        km = torch.ones(B, T, dtype=torch.int32)
        km[0, :40] = 0                      # left padding: the first queries see no key
        km[1, T - 90:] = 0                  # right padding
        km[1, 7::11] = 0
        km = km.cuda()
    y = F.rational_attention_packed(qkv, slopes, scale, key_mask=km)
    y.backward(dy)
    q, k, v = qkv.detach().permute(2, 0, 3, 1, 4)
    o = y.detach().permute(0, 2, 1, 3)
    do = dy.permute(0, 2, 1, 3)
    ro, rL = O.attention_fwd(q, k, v, slopes.cpu(), scale, dtype=torch.float32, key_mask=km)
    check_lowp(o, ro, dtype, "packed o")
    rq, rk, rv = O.attention_bwd(q, k, v, o, rL, do, slopes.cpu(), scale, dtype=torch.float32,
                                 key_mask=km)
    gq, gk, gv = qkv.grad.permute(2, 0, 3, 1, 4)
    for name, got, ref in (("dq", gq, rq), ("dk", gk, rk), ("dv", gv, rv)):
        check_lowp(got, ref, dtype, f"packed {name}")
