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


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64), (torch.float32, 64)])
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
