"""MI355X-native (gfx950) kernels for the algebraic transformer.

Drop-in for the reference ``kernels`` package of
SkyeGunasekaran/fastAlgebraicTransformer: the same public names
(reference __init__.py:7-63), backed by hand-written HIP kernels in
``libkat.so`` behind the C ABI of ``include/kat.h``.

To run code written against the reference unchanged, alias this package
under the reference's import name before importing it::

    import fastalgebraictransformer_amd
    fastalgebraictransformer_amd.install_as("kernels")
    from kernels.fused_ops import rational_softmax   # resolves here
"""

import sys as _sys

from .fused_ops import (
    EPS,
    MeanErrorNorm,
    RationalSoftmax,
    RationalSwiGLU,
    PackedRationalSwiGLU,
    ResidualMeanErrorNorm,
    add_mean_error_norm,
    mean_error_norm,
    rational_softmax,
    rational_swiglu,
    rational_swiglu_packed,
)
from .forward import compute_alibi_slopes, rational_attention_decode, rational_attention_forward
from .backward import (
    MaskedRationalAttentionFunction,
    PackedRationalAttention,
    RationalAttentionFunction,
    rational_attention,
    rational_attention_backward,
    rational_attention_masked,
    rational_attention_packed,
)
from .algebraic_model import (
    AlgebraicAttention,
    AlgebraicBlock,
    AlgebraicTransformerLM,
    RationalMR,
    RationalSwiGLU as RationalSwiGLUModule,
    create_large_model,
    create_medium_model,
    create_small_model,
)

__all__ = [
    "rational_softmax",
    "rational_swiglu",
    "mean_error_norm",
    "RationalSoftmax",
    "RationalSwiGLU",
    "MeanErrorNorm",
    "EPS",
    "rational_attention_forward",
    "compute_alibi_slopes",
    "rational_attention",
    "rational_attention_backward",
    "RationalAttentionFunction",
    "AlgebraicTransformerLM",
    "RationalMR",
    "AlgebraicAttention",
    "AlgebraicBlock",
    "create_small_model",
    "create_medium_model",
    "create_large_model",
]
# Importable extensions beyond the reference surface (kept out of __all__):
# rational_attention_packed / PackedRationalAttention on a packed [B, T, 3, H, D]
# projection and rational_swiglu_packed / PackedRationalSwiGLU on a packed
# [..., 2F] gate|value buffer -- the model's layouts, same kernels; and
# add_mean_error_norm / ResidualMeanErrorNorm, the residual add fused with the
# norm that reads it; rational_attention_masked / MaskedRationalAttentionFunction,
# attention with a key padding mask and a real non-causal mode;
# rational_attention_decode, one query against a KV cache (the model's
# generate() uses it).


def install_as(name="kernels"):
    """Register this package and its submodules under ``name`` (default the
    reference's package name ``kernels``) in ``sys.modules``."""
    pkg = _sys.modules[__name__]
    _sys.modules[name] = pkg
    for sub in ("fused_ops", "forward", "backward", "algebraic_model"):
        _sys.modules[f"{name}.{sub}"] = _sys.modules[f"{__name__}.{sub}"]
    return pkg
