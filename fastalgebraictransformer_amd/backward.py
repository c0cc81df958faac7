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
    _bht_strides,
    _unit_d,
    compute_alibi_slopes,
    rational_attention_forward,
)


def rational_attention_backward(q, k, v, output, L, grad_output, alibi_slopes, scale,
                                causal=True, eps=EPS):
    """Returns (dq, dk, dv), contiguous, in q's dtype."""
    assert q.is_cuda
    lib = _lib.load()
    B, H, T, D = q.shape
    dt = q.dtype
    k, v, output, grad_output = (t.to(dt) for t in (k, v, output, grad_output))
    q, k, v, output, grad_output = (_unit_d(t) for t in (q, k, v, output, grad_output))
    L = L.to(torch.float32)
    slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    dq = torch.empty((B, H, T, D), dtype=dt, device=q.device)
    dk = torch.empty((B, H, T, D), dtype=dt, device=q.device)
    dv = torch.empty((B, H, T, D), dtype=dt, device=q.device)
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
