"""CPU oracle for the rational-attention kernel path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline),
never as the thing measured on the GPU.

It restates, in plain PyTorch on the CPU, the arithmetic of the reference
``kernels`` package (SkyeGunasekaran/fastAlgebraicTransformer). Every function
cites the reference file:line it follows. Inputs are upcast to ``dtype``
(float64 by default, float32 for the CPU baseline) before any arithmetic, which
matches the reference kernels' ``.to(tl.float32)`` loads.

Parity pins (checked in ``tests/test_oracle.py``):
  * rsig / rsig_deriv: closed-form known answers and the symmetry
    sigma(-x) = 1 - sigma(x); the derivative against central differences.
  * rational_softmax fwd: constant-row known answer, row-sum identity
    sum(p) = Z / (Z + eps); bwd against torch.autograd of the fwd and against
    central differences.
  * rational_swiglu: known answers swiglu(1, 2) = 1.5, swiglu(0, v) = 0,
    d/dgate at gate = 0 is 0.5 * value * dy; bwd against torch.autograd.
  * mean_error_norm: constant-row known answer, positive scale invariance;
    dx and dgamma against torch.autograd of the fwd.
  * alibi_slopes: closed form 2^(-8(i+1)/n) for powers of two and the
    hand-computed H=12 list.
  * attention fwd: against the reference test harness formulation (full score
    matrix, ALiBi, -1e4 causal fill, rational softmax, P@V), against a
    pure-Python loop on tiny inputs, and the T=1 and prefix-mean known answers.
  * attention bwd: against torch.autograd of that full-matrix formulation and
    against central differences of attention_fwd.
"""

from .ops import (  # noqa: F401
    EPS,
    NEG_FILL,
    rsig,
    rsig_deriv,
    rational_softmax_fwd,
    rational_softmax_bwd,
    swiglu_fwd,
    swiglu_bwd,
    mean_error_norm_fwd,
    mean_error_norm_bwd,
    alibi_slopes,
    attention_fwd,
    attention_bwd,
    attention_delta,
    harness_attention,
    loop_attention_fwd,
)
