"""Write the golden fixtures (tests/golden/*.npz) from the CPU oracle.

Inputs are drawn from fixed seeds in float32 (bf16 cases are rounded to
bf16 first and stored as their exact float32 values); expected outputs are
the oracle's float64 results on exactly those inputs. Run from the repo root:

    python tests/golden/make_golden.py
"""

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def _rand(g, *shape, scale=1.0, bf16=False):
    t = torch.randn(*shape, generator=g, dtype=torch.float32) * scale
    if bf16:
        t = t.to(torch.bfloat16).to(torch.float32)
    return t


def _np(t):
    return t.detach().cpu().numpy()


def softmax_case(seed, rows, cols, bf16):
    g = torch.Generator().manual_seed(seed)
    x = _rand(g, rows, cols, scale=2.0, bf16=bf16)
    dy = _rand(g, rows, cols, bf16=bf16)
    p = O.rational_softmax_fwd(x)
    # the backward consumes the saved forward output in the input dtype
    p_saved = p.to(torch.bfloat16).to(torch.float64) if bf16 else p.to(torch.float32).double()
    dx = O.rational_softmax_bwd(dy, x, p_saved)
    return dict(x=_np(x), dy=_np(dy), p=_np(p), dx=_np(dx))


def swiglu_case(seed, rows, cols, bf16):
    g = torch.Generator().manual_seed(seed)
    gate = _rand(g, rows, cols, bf16=bf16)
    value = _rand(g, rows, cols, bf16=bf16)
    dy = _rand(g, rows, cols, bf16=bf16)
    out = O.swiglu_fwd(gate, value)
    dg, dv = O.swiglu_bwd(dy, gate, value)
    return dict(gate=_np(gate), value=_np(value), dy=_np(dy), out=_np(out), dgate=_np(dg),
                dvalue=_np(dv))


def norm_case(seed, rows, cols, bf16):
    g = torch.Generator().manual_seed(seed)
    x = _rand(g, rows, cols, bf16=bf16)
    w = 1.0 + 0.02 * torch.randn(cols, generator=g, dtype=torch.float32)
    dy = _rand(g, rows, cols, bf16=bf16)
    y, mu = O.mean_error_norm_fwd(x, w)
    # the backward consumes the saved fp32 mean
    dx, dw = O.mean_error_norm_bwd(dy, x, w, mu.to(torch.float32))
    return dict(x=_np(x), w=_np(w), dy=_np(dy), y=_np(y), mu=_np(mu), dx=_np(dx), dw=_np(dw))


def attention_case(seed, B, H, T, D, bf16):
    g = torch.Generator().manual_seed(seed)
    q = _rand(g, B, H, T, D, bf16=bf16)
    k = _rand(g, B, H, T, D, bf16=bf16)
    v = _rand(g, B, H, T, D, bf16=bf16)
    do = _rand(g, B, H, T, D, bf16=bf16)
    slopes = O.alibi_slopes(H)
    scale = 1.0 / math.sqrt(D)
    o, L = O.attention_fwd(q, k, v, slopes, scale)
    # backward from the fp64 forward (the GPU test feeds its own O and L)
    dq, dk, dv = O.attention_bwd(q, k, v, o, L, do, slopes, scale)
    return dict(q=_np(q), k=_np(k), v=_np(v), do=_np(do), slopes=_np(slopes),
                scale=np.float64(scale), o=_np(o), L=_np(L), dq=_np(dq), dk=_np(dk), dv=_np(dv))


CASES = {
    "softmax_f32": lambda: softmax_case(101, 6, 200, False),
    "softmax_bf16": lambda: softmax_case(102, 5, 1024, True),
    "swiglu_f32": lambda: swiglu_case(201, 7, 96, False),
    "swiglu_bf16": lambda: swiglu_case(202, 3, 520, True),
    "norm_f32": lambda: norm_case(301, 9, 192, False),
    "norm_bf16": lambda: norm_case(302, 4, 4096, True),
    "attn_f32": lambda: attention_case(401, 1, 3, 40, 16, False),
    "attn_bf16_d64": lambda: attention_case(402, 1, 2, 130, 64, True),
    "attn_bf16_d128": lambda: attention_case(403, 1, 2, 160, 128, True),
}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.npz")
        arrs = fn()
        if "bf16" in name:  # bf16 bars are ~1e-2: float32 expected values suffice
            arrs = {k: (v.astype(np.float32) if isinstance(v, np.ndarray) else v)
                    for k, v in arrs.items()}
        np.savez_compressed(path, **arrs)
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
