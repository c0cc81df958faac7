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
    _key_mask_arg,
    _bht_strides,
    _unit_d,
    _warn_if_tiled,
    compute_alibi_slopes,
    rational_attention_forward,
)


def _attn_bwd_into(q, k, v, output, L, grad_output, dq, dk, dv, alibi_slopes, scale, causal, eps,
                   key_mask=None, extended=False):
    """Launch the attention backward; every [B,H,T,D] argument may have any
    (b, h, t) strides with a unit d-stride. The workspace comes from torch's
    allocator. ``extended``: kat_attn_bwd_masked (see _attn_fwd_into)."""
    lib = _lib.load()
    B, H, T, D = q.shape
    _warn_if_tiled((q, k, v, output, grad_output, dq, dk, dv), D, q.dtype,
                   mfma_inputs=(q, k, v, output, grad_output))
    slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    code = _lib.dtype_code(q)
    if extended:
        ws_bytes = lib.kat_attn_bwd_masked_workspace_size(B, H, T, D, code, int(bool(causal)))
    else:
        ws_bytes = lib.kat_attn_bwd_workspace_size(B, H, T, D, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    strides = _lib.i64_array(
        _bht_strides(q) + _bht_strides(k) + _bht_strides(v) + _bht_strides(output) +
        _bht_strides(grad_output) + _bht_strides(dq) + _bht_strides(dk) + _bht_strides(dv))
    lstr = _lib.i64_array(_bht_strides(L))
    if not extended:
        _lib.check(lib.kat_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(),
                                    L.data_ptr(), grad_output.data_ptr(), dq.data_ptr(),
                                    dk.data_ptr(), dv.data_ptr(), slopes.data_ptr(), ws.data_ptr(),
                                    ws_bytes, B, H, T, D, strides, lstr, float(scale), float(eps),
                                    int(bool(causal)), code, _lib.stream(q)), "kat_attn_bwd")
        return
    km_ptr = None if key_mask is None else key_mask.data_ptr()
    _lib.check(lib.kat_attn_bwd_masked(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       output.data_ptr(), L.data_ptr(), grad_output.data_ptr(),
                                       dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                       slopes.data_ptr(), km_ptr, T, ws.data_ptr(), ws_bytes, B,
                                       H, T, D, strides, lstr, float(scale), float(eps),
                                       int(bool(causal)), code, _lib.stream(q)),
               "kat_attn_bwd_masked")


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
    def forward(ctx, qkv, alibi_slopes, scale, eps, key_mask=None):
        assert qkv.is_cuda and qkv.dim() == 5 and qkv.shape[2] == 3, "qkv must be [B, T, 3, H, D]"
        qkv = _unit_d(qkv)
        B, T, _, H, D = qkv.shape
        km = _key_mask_arg(key_mask, B, T, qkv.device)
        q, k, v = qkv.permute(2, 0, 3, 1, 4)
        y = torch.empty((B, T, H, D), dtype=qkv.dtype, device=qkv.device)
        L = torch.empty((B, H, T), dtype=torch.float32, device=qkv.device)
        _attn_fwd_into(q, k, v, y.permute(0, 2, 1, 3), L, alibi_slopes, scale, True, eps, km,
                       extended=km is not None)
        ctx.save_for_backward(qkv, y, L, alibi_slopes, km)
        ctx.scale = scale
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, grad_y):
        qkv, y, L, alibi_slopes, km = ctx.saved_tensors
        q, k, v = qkv.permute(2, 0, 3, 1, 4)
        grad_o = _unit_d(grad_y.to(qkv.dtype).permute(0, 2, 1, 3))
        dqkv = torch.empty(qkv.shape, dtype=qkv.dtype, device=qkv.device)
        dq, dk, dv = dqkv.permute(2, 0, 3, 1, 4)
        _attn_bwd_into(q, k, v, y.permute(0, 2, 1, 3), L, grad_o, dq, dk, dv, alibi_slopes,
                       ctx.scale, True, ctx.eps, km, extended=km is not None)
        return dqkv, None, None, None, None


def rational_attention_packed(qkv, alibi_slopes, scale, eps=EPS, key_mask=None):
    """Causal ALiBi rational attention on qkv [B, T, 3, H, D]; returns
    [B, T, H, D] (see PackedRationalAttention). ``key_mask`` [B, T]: keys where
    it is 0 are dropped (see rational_attention_masked)."""
    return PackedRationalAttention.apply(qkv, alibi_slopes, scale, eps, key_mask)


class MaskedRationalAttentionFunction(torch.autograd.Function):
    """Attention with a key padding mask and a real non-causal mode (see
    rational_attention_masked); recompute backward as RationalAttentionFunction."""

    @staticmethod
    def forward(ctx, q, k, v, alibi_slopes, scale, key_mask, causal, eps):
        assert q.is_cuda and k.is_cuda and v.is_cuda
        assert q.shape == k.shape == v.shape
        B, H, T, D = q.shape
        km = _key_mask_arg(key_mask, B, T, q.device)
        k, v = k.to(q.dtype), v.to(q.dtype)
        q, k, v = _unit_d(q), _unit_d(k), _unit_d(v)
        out = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
        L = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
        _attn_fwd_into(q, k, v, out, L, alibi_slopes, scale, causal, eps, km, extended=True)
        ctx.save_for_backward(q, k, v, out, L, alibi_slopes, km)
        ctx.scale = scale
        ctx.causal = causal
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, out, L, alibi_slopes, km = ctx.saved_tensors
        B, H, T, D = q.shape
        go = _unit_d(grad_output.to(q.dtype))
        dq, dk, dv = (torch.empty((B, H, T, D), dtype=q.dtype, device=q.device) for _ in range(3))
        _attn_bwd_into(q, k, v, out, L, go, dq, dk, dv, alibi_slopes, ctx.scale, ctx.causal,
                       ctx.eps, km, extended=True)
        return dq, dk, dv, None, None, None, None, None


def attention_torch(q, k, v, alibi_slopes, scale, key_mask=None, causal=True, eps=EPS):
    """The reference model's CPU attention (algebraic_model.py:112-136): full
    score matrix, ALiBi -slope |i - j|, the -1e4 causal fill (``causal``) and
    -1e4 padding fill where ``key_mask`` == 0, rational softmax, P @ V."""
    from .fused_ops import rational_softmax
    B, H, T, D = q.shape
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    idx = torch.arange(T, device=q.device)
    dist = (idx[:, None] - idx[None, :]).abs().float()
    scores = scores + (-dist * alibi_slopes.to(q.device).view(1, H, 1, 1))
    if causal:
        future = torch.ones(T, T, device=q.device, dtype=torch.bool).triu(1)
        scores = scores.masked_fill(future[None, None], NEG_INF)
    if key_mask is not None:
        scores = scores.masked_fill((key_mask == 0)[:, None, None, :], NEG_INF)
    return torch.matmul(rational_softmax(scores, eps=eps), v)


def rational_attention_masked(q, k, v, alibi_slopes, scale, key_mask=None, causal=True, eps=EPS):
    """ALiBi rational attention with a key padding mask and a real non-causal
    mode -- an extension beyond the reference API, whose GPU path ignores both
    (forward.py:273) while its model's CPU path applies the padding mask
    (algebraic_model.py:129-131).

    key_mask: [B, T] (any dtype); key j of batch b is dropped where it is 0.
    causal=False: every key is visible, with ALiBi -slope |i - j| (the CPU
    path's form). A dropped key contributes exactly nothing (the CPU path's
    -1e4 fill leaves ~6e-18 per key), so a query with no visible key returns 0.
    CUDA tensors run the libkat kernels; CPU tensors the reference's torch
    formulation (attention_torch)."""
    if q.is_cuda:
        return MaskedRationalAttentionFunction.apply(q, k, v, alibi_slopes, scale, key_mask,
                                                     causal, eps)
    return attention_torch(q, k, v, alibi_slopes, scale, key_mask, causal, eps)
