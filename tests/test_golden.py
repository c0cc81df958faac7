"""The CPU oracle reproduces the committed golden fixtures (CPU only)."""

import numpy as np
import pytest
import torch

import oracle as O
from _util import golden


def _t(a):
    return torch.from_numpy(np.asarray(a))


def _close(a, b, rtol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    tol = rtol * (np.abs(b) + np.abs(b).max() * 1e-6)
    assert np.all(np.abs(a - b) <= tol), float(np.abs(a - b).max())


@pytest.mark.parametrize("name", ["softmax_f32", "softmax_bf16"])
def test_softmax_golden(name):
    z = golden(name)
    rt = 1e-12 if "f32" in name else 1e-6
    p = O.rational_softmax_fwd(_t(z["x"]))
    _close(p, z["p"], rt)
    bf = "bf16" in name
    ps = p.to(torch.bfloat16).double() if bf else p.float().double()
    _close(O.rational_softmax_bwd(_t(z["dy"]), _t(z["x"]), ps), z["dx"], rt)


@pytest.mark.parametrize("name", ["swiglu_f32", "swiglu_bf16"])
def test_swiglu_golden(name):
    z = golden(name)
    rt = 1e-12 if "f32" in name else 1e-6
    _close(O.swiglu_fwd(_t(z["gate"]), _t(z["value"])), z["out"], rt)
    dg, dv = O.swiglu_bwd(_t(z["dy"]), _t(z["gate"]), _t(z["value"]))
    _close(dg, z["dgate"], rt)
    _close(dv, z["dvalue"], rt)


@pytest.mark.parametrize("name", ["norm_f32", "norm_bf16"])
def test_norm_golden(name):
    z = golden(name)
    rt = 1e-12 if "f32" in name else 1e-6
    y, mu = O.mean_error_norm_fwd(_t(z["x"]), _t(z["w"]))
    _close(y, z["y"], rt)
    _close(mu, z["mu"], rt)
    dx, dw = O.mean_error_norm_bwd(_t(z["dy"]), _t(z["x"]), _t(z["w"]), mu.float())
    _close(dx, z["dx"], rt)
    _close(dw, z["dw"], rt)


@pytest.mark.parametrize("name", ["attn_f32", "attn_bf16_d64", "attn_bf16_d128"])
def test_attention_golden(name):
    z = golden(name)
    rt = 1e-10 if "f32" in name else 1e-5
    q, k, v, do = (_t(z[n]) for n in ("q", "k", "v", "do"))
    slopes = _t(z["slopes"])
    assert torch.equal(slopes, O.alibi_slopes(q.shape[1]))
    o, L = O.attention_fwd(q, k, v, slopes, float(z["scale"]))
    _close(o, z["o"], rt)
    _close(L, z["L"], rt)
    dq, dk, dv = O.attention_bwd(q, k, v, o, L, do, slopes, float(z["scale"]))
    _close(dq, z["dq"], rt)
    _close(dk, z["dk"], rt)
    _close(dv, z["dv"], rt)
