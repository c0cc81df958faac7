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
