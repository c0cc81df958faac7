"""Rational attention forward on MI355X.

Same Python API as the reference ``kernels.forward``
(SkyeGunasekaran/fastAlgebraicTransformer forward.py:21-42
``compute_alibi_slopes`` and forward.py:267-319 ``rational_attention_forward``).
The launch goes to ``kat_attn_fwd`` in libkat.so: a bf16/fp16 MFMA kernel for
head dims it covers, a tiled kernel otherwise (fp32 arithmetic; fp64 for fp64
tensors; any head dim up to 1024).
"""

import math
import os
import warnings

import torch

from . import _lib
from .fused_ops import EPS, NEG_INF  # noqa: F401  (re-exported like the reference)


def compute_alibi_slopes(n_heads, device=None):
    """ALiBi slopes as in the reference (forward.py:21-42): with p the largest
    power of two <= n_heads, head i < p gets b^(i+1) with b = 2^(-8/p); the
    remaining n_heads - p heads get b'^k, b' = 2^(-8/(2p)), k = 1, 3, 5, ...
    The powers are taken by torch.pow of a float base over integer exponents,
    which is how the reference forms them (float32 result), so the slopes
    match it bit for bit."""
    p = 1 << int(math.floor(math.log2(n_heads)))
    slopes = torch.pow(2.0 ** (-8.0 / p), torch.arange(1, p + 1))
    extra = min(p, n_heads - p)
    if extra > 0:
        odd = torch.arange(1, 2 * extra, 2)
        slopes = torch.cat([slopes, torch.pow(2.0 ** (-8.0 / (2 * p)), odd)])
    slopes = slopes.float()
    return slopes.to(device) if device is not None else slopes


def _bht_strides(t):
    return (t.stride(0), t.stride(1), t.stride(2))


def _unit_d(t):
    return t if t.stride(-1) == 1 or t.shape[-1] == 1 else t.contiguous()


_WARNED = set()

# per-(b, h) slice byte offsets the MFMA kernels address with 31-bit buffer
# offsets: a row stride s (elements) must satisfy (T + 128) * s * 2 < 2^31
# (csrc/attn_mfma.hip offsets_ok)
_MFMA_OFFSET_LIMIT = 0x7FFFFFFF
_MFMA_ROW_PAD = 128


def _mfma_head_dim(D, elem=2):
    """Head dims the MFMA kernels cover (forward and backward): 16-byte rows
    up to 256 columns -- multiples of 8 for bf16 / fp16 (``elem`` 2), of 4
    for fp32 (``elem`` 4) -- run in the kernels of the next layout width (32,
    64, 128 or 256 columns) with the columns past D read as zeros."""
    step = 16 // elem
    return step <= D <= 256 and D % step == 0


def _tiled_reason(shapes_strides_ptrs, D, T, elem):
    """Why a bf16 / fp16 / fp32 attention call would leave the MFMA kernels
    for the tiled ones (None if it takes them), from each operand's (b, h, t)
    strides and data pointer: the head dim, 16-byte row alignment, and the
    31-bit byte offsets the MFMA kernels use within one (b, h) slice."""
    if not _mfma_head_dim(D, elem):
        return f"head dim {D} (the MFMA kernels cover multiples of {16 // elem} up to 256)"
    for strides, ptr in shapes_strides_ptrs:
        if ptr % 16 or any((st * elem) % 16 for st in strides):
            return "rows not 16-byte aligned (a view with an odd offset or stride)"
    for strides, _ in shapes_strides_ptrs:
        st = strides[2]
        if st < D or (T + _MFMA_ROW_PAD) * st * elem > _MFMA_OFFSET_LIMIT:
            return (f"row stride {st} at T = {T}: a (b, h) slice spans 2^31 bytes or more "
                    "(the MFMA kernels address a slice with 31-bit offsets)")
    if elem == 2 and (T * D * 2 >= _MFMA_OFFSET_LIMIT or T * 8 >= _MFMA_OFFSET_LIMIT):
        return f"T = {T}: per-head workspace rows exceed 31-bit offsets"
    return None


def _warn_if_tiled(tensors, D, dtype, mfma_inputs=None):
    """bf16 / fp16 (fp32) attention runs on the MFMA kernels when the head dim
    is a multiple of 8 (4) up to 256, every [B, H, T, D] operand has 16-byte aligned rows and the
    inputs the kernels address by 31-bit offsets (q, k, v; and O, dO in the
    backward: ``mfma_inputs``) keep each (b, h) slice below 2^31 bytes;
    otherwise libkat falls back to the tiled kernels, which are correct but
    about an order of magnitude slower. Warn once per dtype and reason, so a model with
    another head dim, a misaligned view or a very long packed sequence does
    not lose that silently."""
    if dtype not in (torch.bfloat16, torch.float16, torch.float32) or \
            os.environ.get("KAT_ATTN_IMPL") == "tiled":
        return
    T = tensors[0].shape[2]
    elem = tensors[0].element_size()
    # the common case in a few attribute reads (it runs on every call): every
    # operand with the (b, h, t) strides of a contiguous [B, H, T, D] tensor
    # (multiples of D, row stride D) and a 16-byte aligned start
    H = tensors[0].shape[1]
    dense = (H * T * D, T * D, D)
    if _mfma_head_dim(D, elem) and (T + _MFMA_ROW_PAD) * D * elem <= _MFMA_OFFSET_LIMIT and \
            (elem != 2 or (T * D * 2 < _MFMA_OFFSET_LIMIT and T * 8 < _MFMA_OFFSET_LIMIT)) and \
            all(t.stride()[:3] == dense and t.data_ptr() % 16 == 0 for t in tensors):
        return
    align = [(t.stride()[:3], t.data_ptr()) for t in tensors]
    reason = _tiled_reason(align, D, T, elem)
    if reason is None and mfma_inputs is not None:
        reason = _tiled_reason([(t.stride()[:3], 0) for t in mfma_inputs], D, T, elem)
    if reason is None:
        return
    if (dtype, reason) not in _WARNED:
        _WARNED.add((dtype, reason))
        warnings.warn(f"rational attention in {dtype}: {reason}; running the tiled "
                      "kernels, about 10x slower than the MFMA path", RuntimeWarning, stacklevel=3)


def _key_mask_arg(key_mask, B, T, device):
    """The padding mask as a uint8 [B, T] device tensor (nonzero = attend), or None."""
    if key_mask is None:
        return None
    assert tuple(key_mask.shape) == (B, T), f"key_mask must be [B, T] = [{B}, {T}]"
    return (key_mask.to(device) != 0).to(torch.uint8).contiguous()


def _attn_fwd_into(q, k, v, out, L, alibi_slopes, scale, causal, eps, key_mask=None,
                   extended=False):
    """Launch the attention forward on [B,H,T,D] q, k, v and out (any (b, h, t)
    strides, unit d-stride) and L [B,H,T] fp32. ``extended`` selects
    kat_attn_fwd_masked, which applies ``key_mask`` (uint8 [B, T] or None) and
    honours ``causal``; otherwise kat_attn_fwd, always causal as the reference."""
    lib = _lib.load()
    B, H, T, D = q.shape
    _warn_if_tiled((q, k, v, out), D, q.dtype, mfma_inputs=(q, k, v))
    slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    assert slopes.numel() == H, "alibi_slopes must have n_heads entries"
    strides = _lib.i64_array(_bht_strides(q) + _bht_strides(k) + _bht_strides(v) +
                             _bht_strides(out))
    lstr = _lib.i64_array(_bht_strides(L))
    if not extended:
        _lib.check(lib.kat_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                    L.data_ptr(), slopes.data_ptr(), B, H, T, D, strides, lstr,
                                    float(scale), float(eps), int(bool(causal)),
                                    _lib.dtype_code(q), _lib.stream(q)), "kat_attn_fwd")
        return
    km_ptr = None if key_mask is None else key_mask.data_ptr()
    _lib.check(lib.kat_attn_fwd_masked(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                       L.data_ptr(), slopes.data_ptr(), km_ptr, T, B, H, T, D,
                                       strides, lstr, float(scale), float(eps), int(bool(causal)),
                                       _lib.dtype_code(q), _lib.stream(q)), "kat_attn_fwd_masked")


def rational_attention_forward(q, k, v, alibi_slopes, scale, causal=True, eps=EPS):
    """Returns (output [B,H,T,D] in q's dtype, L [B,H,T] fp32 without eps).

    Always causal, as the reference (``causal`` is accepted and ignored,
    forward.py:273,110). q, k, v may be strided views with a unit last-dim
    stride (no copies are made for them)."""
    assert q.is_cuda and k.is_cuda and v.is_cuda
    assert q.shape == k.shape == v.shape
    B, H, T, D = q.shape
    k = k.to(q.dtype)
    v = v.to(q.dtype)
    q, k, v = _unit_d(q), _unit_d(k), _unit_d(v)
    out = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
    L = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    _attn_fwd_into(q, k, v, out, L, alibi_slopes, scale, causal, eps)
    return out, L


def rational_attention_decode(q, k_cache, v_cache, alibi_slopes, scale, lengths=None, eps=EPS):
    """One query per (batch, head) against a KV cache: the last row of the
    causal attention over the cached keys, which the reference's generate()
    recomputes over the whole prefix for every new token
    (algebraic_model.py:239-265). An extension beyond the reference API.

    q: [B, H, D]; k_cache, v_cache: [B, H, T, D] (any (b, h, t) strides with a
    unit last-dim stride, e.g. permuted views of token-major [B, T, H, D]
    caches). ``lengths`` (int32 [B] on the device, optional): keys cached per
    batch row, default T; the query sits at position lengths[b] - 1.
    Returns (out [B, H, D] in q's dtype, L [B, H] fp32 without eps). Runs
    ``kat_attn_decode`` (split-KV, deterministic); CUDA tensors only."""
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    B, H, D = q.shape
    T = k_cache.shape[2]
    assert tuple(k_cache.shape) == (B, H, T, D) and tuple(v_cache.shape) == (B, H, T, D)
    lib = _lib.load()
    k_cache, v_cache = k_cache.to(q.dtype), v_cache.to(q.dtype)
    q, k_cache, v_cache = _unit_d(q), _unit_d(k_cache), _unit_d(v_cache)
    slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    assert slopes.numel() == H, "alibi_slopes must have n_heads entries"
    if lengths is not None:
        lengths = lengths.to(device=q.device, dtype=torch.int32).contiguous()
        assert lengths.numel() == B, "lengths must have B entries"
    out = torch.empty((B, H, D), dtype=q.dtype, device=q.device)
    L = torch.empty((B, H), dtype=torch.float32, device=q.device)
    code = _lib.dtype_code(q)
    ws_bytes = lib.kat_attn_decode_workspace_size(B, H, T, D, code)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=q.device)
    strides = _lib.i64_array((q.stride(0), q.stride(1)) + _bht_strides(k_cache) +
                             _bht_strides(v_cache) + (out.stride(0), out.stride(1)))
    _lib.check(lib.kat_attn_decode(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                   out.data_ptr(), L.data_ptr(), slopes.data_ptr(),
                                   None if lengths is None else lengths.data_ptr(), ws.data_ptr(),
                                   ws_bytes, B, H, T, D, strides, float(scale), float(eps), code,
                                   _lib.stream(q)), "kat_attn_decode")
    return out, L
