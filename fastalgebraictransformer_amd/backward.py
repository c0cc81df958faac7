"""Rational attention backward and autograd glue on MI355X.

Same Python API as the reference ``kernels.backward``
(SkyeGunasekaran/fastAlgebraicTransformer backward.py:273-341
``rational_attention_backward``, :348-383 ``RationalAttentionFunction``,
:386-396 ``rational_attention``). Gradients follow the reference derivation
(backward.py:7-46): with p = f / (L + eps) and g = 2 / ((|s|+1)^2 (sigma+eps)),
dS = p g (dO.v - Delta), dq = scale dS K, dk = scale dS^T Q, dv = P^T dO.
The launch goes to ``kat_attn_bwd`` in libkat.so (deterministic: no atomics).
"""

import torch

from . import _lib
from .fused_ops import EPS, NEG_INF  # noqa: F401
from .forward import (  # noqa: F401
    _attn_fwd_into,
    _bht_strides,
    _unit_d,
    compute_alibi_slopes,
    rational_attention_forward,
)


def _attn_bwd_into(q, k, v, output, L, grad_output, dq, dk, dv, alibi_slopes, scale, causal, eps):
    """Launch kat_attn_bwd; every [B,H,T,D] argument may have any (b, h, t)
    strides with a unit d-stride. The workspace comes from torch's allocator."""
    lib = _lib.load()
    B, H, T, D = q.shape
    slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    code = _lib.dtype_code(q)
    ws_bytes = lib.kat_attn_bwd_workspace_size(B, H, T, D, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    strides = _lib.i64_array(
        _bht_strides(q) + _bht_strides(k) + _bht_strides(v) + _bht_strides(output) +
        _bht_strides(grad_output) + _bht_strides(dq) + _bht_strides(dk) + _bht_strides(dv))
    lstr = _lib.i64_array(_bht_strides(L))
    _lib.check(lib.kat_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(),
                                L.data_ptr(), grad_output.data_ptr(), dq.data_ptr(),
                                dk.data_ptr(), dv.data_ptr(), slopes.data_ptr(), ws.data_ptr(),
                                ws_bytes, B, H, T, D, strides, lstr, float(scale), float(eps),
                                int(bool(causal)), code, _lib.stream(q)), "kat_attn_bwd")


def rational_attention_backward(q, k, v, output, L, grad_output, alibi_slopes, scale,
                                causal=True, eps=EPS):
    """Returns (dq, dk, dv), contiguous, in q's dtype."""
    assert q.is_cuda
    B, H, T, D = q.shape
    dt = q.dtype
    k, v, output, grad_output = (t.to(dt) for t in (k, v, output, grad_output))
    q, k, v, output, grad_output = (_unit_d(t) for t in (q, k, v, output, grad_output))
    L = L.to(torch.float32)
    dq = torch.empty((B, H, T, D), dtype=dt, device=q.device)
    dk = torch.empty((B, H, T, D), dtype=dt, device=q.device)
    dv = torch.empty((B, H, T, D), dtype=dt, device=q.device)
    _attn_bwd_into(q, k, v, output, L, grad_output, dq, dk, dv, alibi_slopes, scale, causal, eps)
    return dq, dk, dv


class RationalAttentionFunction(torch.autograd.Function):
    """Autograd Function: saves (q, k, v, output, L, alibi_slopes) like the
    reference (backward.py:364) and recomputes the attention weights in the
    backward kernels."""

    @staticmethod
    def forward(ctx, q, k, v, alibi_slopes, scale, causal, eps):
        output, L = rational_attention_forward(q, k, v, alibi_slopes, scale, causal, eps)
        ctx.save_for_backward(q, k, v, output, L, alibi_slopes)
        ctx.scale = scale
        ctx.causal = causal
        ctx.eps = eps
        return output

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, output, L, alibi_slopes = ctx.saved_tensors
        dq, dk, dv = rational_attention_backward(q, k, v, output, L, grad_output, alibi_slopes,
                                                 ctx.scale, ctx.causal, ctx.eps)
        return dq, dk, dv, None, None, None, None


def rational_attention(q, k, v, alibi_slopes, scale, causal=True, eps=EPS):
    """Causal ALiBi rational attention with a recompute backward."""
    return RationalAttentionFunction.apply(q, k, v, alibi_slopes, scale, causal, eps)


class PackedRationalAttention(torch.autograd.Function):
    """Attention on a packed projection ``qkv`` of shape [B, T, 3, H, D] (the
    model's single q/k/v linear layer). An extension beyond the reference API,
    used by the model's attention module. The kernels read q, k, v in place and
    write the output as [B, T, H, D] memory, so the caller's [B, T, H*D] view
    needs no transpose copy. The backward writes dq, dk, dv into one
    [B, T, 3, H, D] gradient buffer, so autograd neither stacks nor permutes
    three separate gradients. Same kernels and results as ``rational_attention``
    on the three views."""

    @staticmethod
    def forward(ctx, qkv, alibi_slopes, scale, eps):
        assert qkv.is_cuda and qkv.dim() == 5 and qkv.shape[2] == 3, "qkv must be [B, T, 3, H, D]"
        qkv = _unit_d(qkv)
        B, T, _, H, D = qkv.shape
        q, k, v = qkv.permute(2, 0, 3, 1, 4)
        y = torch.empty((B, T, H, D), dtype=qkv.dtype, device=qkv.device)
        L = torch.empty((B, H, T), dtype=torch.float32, device=qkv.device)
        _attn_fwd_into(q, k, v, y.permute(0, 2, 1, 3), L, alibi_slopes, scale, True, eps)
        ctx.save_for_backward(qkv, y, L, alibi_slopes)
        ctx.scale = scale
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, grad_y):
        qkv, y, L, alibi_slopes = ctx.saved_tensors
        q, k, v = qkv.permute(2, 0, 3, 1, 4)
        grad_o = _unit_d(grad_y.to(qkv.dtype).permute(0, 2, 1, 3))
        dqkv = torch.empty(qkv.shape, dtype=qkv.dtype, device=qkv.device)
        dq, dk, dv = dqkv.permute(2, 0, 3, 1, 4)
        _attn_bwd_into(q, k, v, y.permute(0, 2, 1, 3), L, grad_o, dq, dk, dv, alibi_slopes,
                       ctx.scale, True, ctx.eps)
        return dqkv, None, None, None


def rational_attention_packed(qkv, alibi_slopes, scale, eps=EPS):
    """Causal ALiBi rational attention on qkv [B, T, 3, H, D]; returns
    [B, T, H, D] (see PackedRationalAttention)."""
    return PackedRationalAttention.apply(qkv, alibi_slopes, scale, eps)
