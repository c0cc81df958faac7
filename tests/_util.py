"""Shared helpers for the test suite."""

import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf16_ulp(ref):
    """Spacing of bf16 numbers at |ref| (8 significand bits)."""
    a = ref.abs().to(torch.float64).clamp_min(2.0 ** -126)
    e = torch.floor(torch.log2(a))
    return torch.pow(2.0, e - 7)


def assert_bf16_within_ulp(out, ref, n_ulp=1.0, abs_floor=0.0, what=""):
    """|out - ref| <= n_ulp * ulp_bf16(ref) + abs_floor, elementwise.

    ``out`` is the bf16 result of a kernel that computes in fp32 and rounds
    once; ``ref`` the fp64/fp32 oracle value."""
    out = out.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    err = (out - ref).abs()
    bound = n_ulp * bf16_ulp(ref) + abs_floor
    bad = err > bound
    if bool(bad.any()):
        i = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements beyond {n_ulp} bf16 ulp; first at "
            f"flat index {i}: out={out.flatten()[i].item()!r} ref={ref.flatten()[i].item()!r}")


def assert_rel(out, ref, rel, what="", floor_frac=1e-6):
    """max|out - ref| <= rel * |ref| + floor_frac * max|ref| elementwise."""
    out = out.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    err = (out - ref).abs()
    bound = rel * ref.abs() + floor_frac * float(ref.abs().max()) + 1e-30
    bad = err > bound
    if bool(bad.any()):
        i = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements beyond rel {rel}; max err "
            f"{float(err.max()):.3e}; first at {i}: out={out.flatten()[i].item()!r} "
            f"ref={ref.flatten()[i].item()!r}")


def max_abs(a, b):
    return float((a.detach().to("cpu", torch.float64) - b.detach().to("cpu", torch.float64)).abs().max())


def lowp_ulp(ref, dtype):
    """Spacing of ``dtype`` (bf16 or fp16) numbers at |ref|."""
    if dtype == torch.float16:
        a = ref.abs().to(torch.float64).clamp_min(2.0 ** -14)
        return torch.pow(2.0, torch.floor(torch.log2(a)) - 10)
    return bf16_ulp(ref)


def check_lowp(got, ref, dtype, name, bar=2e-2, n_ulp=0.5, rel_l2=5e-3):
    """Low-precision attention bar: elementwise |got - ref| <= bar +
    n_ulp * ulp_dtype(ref) (the north-star 2e-2 max-abs plus the output's own
    rounding to dtype), and, where the reference is not ~0 (rms > 1e-3), a
    relative L2 error ||got - ref|| / ||ref|| <= rel_l2, which a systematic
    error of a few tenths of a percent would break even where the elementwise
    bar is loose. Returns (max error, relative L2 error)."""
    got = got.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    err = (got - ref).abs()
    worst = float((err - (bar + n_ulp * lowp_ulp(ref, dtype))).max())
    rn = float(ref.norm())
    rl2 = float((got - ref).norm()) / max(rn, 1e-300)
    assert worst <= 0, (f"{name}: max err {float(err.max()):.3e} (max|ref| "
                        f"{float(ref.abs().max()):.3e}) exceeds {bar} + {n_ulp} ulp by {worst:.3e}")
    if rn > 1e-3 * ref.numel() ** 0.5:
        assert rl2 <= rel_l2, f"{name}: relative L2 error {rl2:.3e} > {rel_l2}"
    return float(err.max()), rl2
