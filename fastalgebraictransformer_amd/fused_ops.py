"""Rational softmax, rational SwiGLU and mean-error norm on MI355X.

Same Python API as the reference ``kernels.fused_ops``
(SkyeGunasekaran/fastAlgebraicTransformer, fused_ops.py:20-21 constants,
:435-599 autograd Functions, :606-636 functional wrappers). CUDA (HIP) tensors
run the hand-written gfx950 kernels of libkat.so through its C ABI; there is no
other GPU path. CPU tensors keep the reference's own torch formulas
(fused_ops.py:610-615, 623-626, 634-636), as the reference does.

Differences from the reference launch wrappers, all layout-only:
  * inputs whose last dim is unit-stride are read in place (row stride passed
    to the kernel) instead of being copied by ``.contiguous()``;
  * the weight gradient of MeanErrorNorm comes out of the same kernel pass
    (deterministic column reduction) instead of extra torch ops.
"""

import torch

from . import _lib

# fused_ops.py:20-21
EPS = 1e-6
NEG_INF = -1e4


def _ptr(t):
    return torch.Tensor.data_ptr(t)


class RationalSoftmax(torch.autograd.Function):
    """p = sigma(x)^4 / (sum sigma(x)^4 + eps) over the last dim
    (reference fused_ops.py:435-487)."""

    @staticmethod
    def forward(ctx, x, eps=EPS):
        assert x.is_cuda, "Input must be on CUDA"
        lib = _lib.load()
        x2, ldx = _lib.rows2d(x)
        rows, cols = x2.shape
        out = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        _lib.check(lib.kat_rsoftmax_fwd(_ptr(x2), _ptr(out), rows, cols, ldx, cols, float(eps),
                                        _lib.dtype_code(x), _lib.stream(x)), "kat_rsoftmax_fwd")
        out = out.view(x.shape)
        ctx.save_for_backward(x, out)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, out = ctx.saved_tensors
        lib = _lib.load()
        x2, ldx = _lib.rows2d(x)
        p2, ldp = _lib.rows2d(out)
        g2, ldg = _lib.rows2d(grad_output.to(x.dtype))
        rows, cols = x2.shape
        dx = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        _lib.check(lib.kat_rsoftmax_bwd(_ptr(g2), _ptr(x2), _ptr(p2), _ptr(dx), rows, cols, ldg,
                                        ldx, ldp, cols, float(ctx.eps), _lib.dtype_code(x),
                                        _lib.stream(x)), "kat_rsoftmax_bwd")
        return dx.view(x.shape), None


class RationalSwiGLU(torch.autograd.Function):
    """out = gate * sigma(gate) * value (reference fused_ops.py:490-539)."""

    @staticmethod
    def forward(ctx, gate, value):
        assert gate.is_cuda and value.is_cuda, "Inputs must be on CUDA"
        assert gate.shape == value.shape, "gate and value must have the same shape"
        lib = _lib.load()
        value = value.to(gate.dtype)
        g2, ldg = _lib.rows2d(gate)
        v2, ldv = _lib.rows2d(value)
        rows, cols = g2.shape
        out = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
        _lib.check(lib.kat_rswiglu_fwd(_ptr(g2), _ptr(v2), _ptr(out), rows, cols, ldg, ldv, cols,
                                       _lib.dtype_code(gate), _lib.stream(gate)),
                   "kat_rswiglu_fwd")
        ctx.save_for_backward(gate, value)
        return out.view(gate.shape)

    @staticmethod
    def backward(ctx, grad_output):
        gate, value = ctx.saved_tensors
        lib = _lib.load()
        g2, ldg = _lib.rows2d(gate)
        v2, ldv = _lib.rows2d(value)
        y2, ldy = _lib.rows2d(grad_output.to(gate.dtype))
        rows, cols = g2.shape
        dgate = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
        dvalue = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
        _lib.check(lib.kat_rswiglu_bwd(_ptr(y2), _ptr(g2), _ptr(v2), _ptr(dgate), _ptr(dvalue),
                                       rows, cols, ldy, ldg, ldv, cols, cols,
                                       _lib.dtype_code(gate), _lib.stream(gate)),
                   "kat_rswiglu_bwd")
        return dgate.view(gate.shape), dvalue.view(gate.shape)


class PackedRationalSwiGLU(torch.autograd.Function):
    """SwiGLU on a packed [..., 2F] buffer whose halves are (gate | value): the
    model's single gate/value projection. An extension beyond the reference
    API, used by the model's FFN. The forward reads both halves in place; the
    backward writes d(gate | value) into one [..., 2F] gradient, so autograd
    does not concatenate two separate gradients (the reference's chunk path,
    algebraic_model.py:52-53 with fused_ops.py:498-499,522-528, copies both).
    Same kernels and results as RationalSwiGLU on the two halves."""

    @staticmethod
    def forward(ctx, gv):
        assert gv.is_cuda, "Input must be on CUDA"
        assert gv.shape[-1] % 2 == 0, "the last dim holds gate and value halves"
        lib = _lib.load()
        g2, ld = _lib.rows2d(gv)
        rows, two_f = g2.shape
        f = two_f // 2
        out = torch.empty((rows, f), dtype=gv.dtype, device=gv.device)
        vptr = _ptr(g2) + f * g2.element_size()
        _lib.check(lib.kat_rswiglu_fwd(_ptr(g2), vptr, _ptr(out), rows, f, ld, ld, f,
                                       _lib.dtype_code(gv), _lib.stream(gv)), "kat_rswiglu_fwd")
        ctx.save_for_backward(gv)
        return out.view(*gv.shape[:-1], f)

    @staticmethod
    def backward(ctx, grad_output):
        (gv,) = ctx.saved_tensors
        lib = _lib.load()
        g2, ld = _lib.rows2d(gv)
        rows, two_f = g2.shape
        f = two_f // 2
        y2, ldy = _lib.rows2d(grad_output.to(gv.dtype))
        dgv = torch.empty((rows, two_f), dtype=gv.dtype, device=gv.device)
        es = g2.element_size()
        _lib.check(lib.kat_rswiglu_bwd(_ptr(y2), _ptr(g2), _ptr(g2) + f * es, _ptr(dgv),
                                       _ptr(dgv) + f * es, rows, f, ldy, ld, ld, two_f, two_f,
                                       _lib.dtype_code(gv), _lib.stream(gv)), "kat_rswiglu_bwd")
        return dgv.view(gv.shape)


def _weight_for(x, weight):
    """The kernels take the weight as fp32 or in x's dtype, contiguous."""
    if weight.dtype != x.dtype and not (weight.dtype == torch.float32 and x.dtype != torch.float64):
        weight = weight.to(torch.float32 if x.dtype != torch.float64 else x.dtype)
    return weight.contiguous()


class MeanErrorNorm(torch.autograd.Function):
    """y = x / (mean|x| + eps) * weight (reference fused_ops.py:542-599)."""

    @staticmethod
    def forward(ctx, x, weight, eps=EPS):
        assert x.is_cuda, "Input must be on CUDA"
        lib = _lib.load()
        w = _weight_for(x, weight)
        assert w.numel() == x.shape[-1], "weight must have x.shape[-1] elements"
        x2, ldx = _lib.rows2d(x)
        rows, cols = x2.shape
        y = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        _lib.check(lib.kat_men_fwd(_ptr(x2), _ptr(w), _ptr(y), _ptr(mean), rows, cols, ldx, cols,
                                   float(eps), _lib.dtype_code(x), _lib.dtype_code(w),
                                   _lib.stream(x)), "kat_men_fwd")
        ctx.save_for_backward(x, w, mean)
        ctx.eps = eps
        ctx.weight_dtype = weight.dtype
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, grad_output):
        x, w, mean = ctx.saved_tensors
        lib = _lib.load()
        x2, ldx = _lib.rows2d(x)
        g2, ldg = _lib.rows2d(grad_output.to(x.dtype))
        rows, cols = x2.shape
        code = _lib.dtype_code(x)
        dx = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        acc = torch.float64 if x.dtype == torch.float64 else torch.float32
        dw = torch.empty(cols, dtype=acc, device=x.device)
        ws_bytes = lib.kat_men_bwd_workspace_size(rows, cols, code)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        _lib.check(lib.kat_men_bwd(_ptr(g2), _ptr(x2), _ptr(w), _ptr(mean), _ptr(dx), _ptr(dw),
                                   _ptr(ws), ws_bytes, rows, cols, ldg, ldx, cols, float(ctx.eps),
                                   code, _lib.dtype_code(w), _lib.stream(x)), "kat_men_bwd")
        # like the reference, the weight gradient is returned in fp32
        # (fused_ops.py:595-599); autograd casts it to the parameter's dtype
        return dx.view(x.shape), dw, None


class ResidualMeanErrorNorm(torch.autograd.Function):
    """(h, y) = (x + r, mean_error_norm(x + r, weight)) in one pass: the
    pre-norm block's residual add and the norm that reads it
    (reference algebraic_model.py:150-151 with fused_ops.py:542-599).

    ``r`` may be narrower than ``x`` (bf16/fp16 branch output beside an fp32
    residual stream, as under autocast); ``h`` has ``x``'s dtype exactly as
    torch's promoted add gives it. ``out_dtype`` (bf16/fp16 beside an fp32
    stream) stores ``y`` narrowed, as the cast in front of an autocast matmul
    would, and takes its gradient in that dtype. Outputs and gradients equal
    those of ``h = x + r; y = MeanErrorNorm.apply(h, weight, eps)`` (followed
    by ``y.to(out_dtype)``) bit for bit."""

    @staticmethod
    def forward(ctx, x, r, weight, eps=EPS, out_dtype=None):
        assert x.is_cuda and r.is_cuda, "Input must be on CUDA"
        assert r.shape == x.shape, "residual branch must have the stream's shape"
        lib = _lib.load()
        w = _weight_for(x, weight)
        assert w.numel() == x.shape[-1], "weight must have x.shape[-1] elements"
        x2, ldx = _lib.rows2d(x)
        r2, ldr = _lib.rows2d(r)
        rows, cols = x2.shape
        h = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        y = torch.empty((rows, cols), dtype=out_dtype or x.dtype, device=x.device)
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        _lib.check(lib.kat_add_men_fwd(_ptr(x2), _ptr(r2), _ptr(w), _ptr(h), _ptr(y), _ptr(mean),
                                       rows, cols, ldx, ldr, cols, cols, float(eps),
                                       _lib.dtype_code(x), _lib.dtype_code(r), _lib.dtype_code(y),
                                       _lib.dtype_code(w), _lib.stream(x)), "kat_add_men_fwd")
        ctx.save_for_backward(h, w, mean)
        ctx.eps = eps
        ctx.r_dtype = r.dtype
        ctx.y_dtype = y.dtype
        return h.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, grad_h, grad_y):
        h, w, mean = ctx.saved_tensors
        lib = _lib.load()
        rows, cols = h.shape
        g2, ldg = _lib.rows2d(grad_y.to(ctx.y_dtype))
        d2, ldd = _lib.rows2d(grad_h.to(h.dtype))
        code = _lib.dtype_code(h)
        dx = torch.empty((rows, cols), dtype=h.dtype, device=h.device)
        # a same-dtype branch gets the stream's gradient itself (as torch's add
        # backward gives both operands the one tensor); a narrower one its cast
        dr = None
        if ctx.r_dtype != h.dtype and ctx.needs_input_grad[1]:
            dr = torch.empty((rows, cols), dtype=ctx.r_dtype, device=h.device)
        acc = torch.float64 if h.dtype == torch.float64 else torch.float32
        dw = torch.empty(cols, dtype=acc, device=h.device)
        ws_bytes = lib.kat_men_bwd_workspace_size(rows, cols, code)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
        _lib.check(lib.kat_add_men_bwd(_ptr(g2), _ptr(d2), _ptr(h), _ptr(w), _ptr(mean), _ptr(dx),
                                       None if dr is None else _ptr(dr), _ptr(dw), _ptr(ws),
                                       ws_bytes, rows, cols, ldg, ldd, cols, cols, cols,
                                       float(ctx.eps), code,
                                       _lib.dtype_code(dr if dr is not None else h),
                                       _lib.dtype_code(g2), _lib.dtype_code(w), _lib.stream(h)),
                   "kat_add_men_bwd")
        shape = grad_y.shape
        dx = dx.view(shape)
        if not ctx.needs_input_grad[1]:
            d_r = None
        else:
            d_r = dx if dr is None else dr.view(shape)
        return dx, d_r, dw, None, None


def rational_softmax(x, eps=EPS):
    """Rational softmax over the last dim (reference fused_ops.py:606-615)."""
    if x.is_cuda:
        return RationalSoftmax.apply(x, eps)
    sig = 0.5 * (x / (x.abs() + 1.0) + 1.0)
    f = sig.pow(4)
    return f / (f.sum(dim=-1, keepdim=True) + eps)


def rational_swiglu(gate, value):
    """gate * sigma(gate) * value (reference fused_ops.py:618-626)."""
    if gate.is_cuda:
        return RationalSwiGLU.apply(gate, value)
    sig = 0.5 * (gate / (gate.abs() + 1.0) + 1.0)
    return gate * sig * value


def mean_error_norm(x, weight, eps=EPS):
    """x / (mean|x| + eps) * weight (reference fused_ops.py:629-636)."""
    if x.is_cuda:
        return MeanErrorNorm.apply(x, weight, eps)
    m = x.abs().mean(dim=-1, keepdim=True)
    return (x / (m + eps)) * weight


def add_mean_error_norm(x, r, weight, eps=EPS, out_dtype=None):
    """(x + r, mean_error_norm(x + r, weight, eps)) with the add fused into the
    norm on CUDA tensors (see ResidualMeanErrorNorm); CPU tensors use the
    reference formulas. ``out_dtype``: the normalised output's dtype when it
    feeds a narrower (autocast) matmul; default x's dtype."""
    if out_dtype == x.dtype:
        out_dtype = None
    if x.is_cuda:
        return ResidualMeanErrorNorm.apply(x, r, weight, eps, out_dtype)
    h = x + r
    y = mean_error_norm(h, weight, eps)
    return h, (y if out_dtype is None else y.to(out_dtype))


def rational_swiglu_packed(gv):
    """gate * sigma(gate) * value with gate, value = gv.chunk(2, dim=-1)
    (see PackedRationalSwiGLU); CPU tensors use the reference formula."""
    if gv.is_cuda:
        return PackedRationalSwiGLU.apply(gv)
    gate, value = gv.chunk(2, dim=-1)
    return rational_swiglu(gate, value)
