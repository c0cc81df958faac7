"""The norm backward's weight gradient (per-block column partials, then a
fixed-order reduction launch) against the CPU oracle (reference
fused_ops.py:595-597) over grids of one block, a few blocks and a full chip,
fp32 / fp64 accumulators and a partial last column block; repeated calls are
bit-identical, and so are calls queued on two streams at once and graph
replays of a captured backward."""

import numpy as np
import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from fastalgebraictransformer_amd import _lib
from fastalgebraictransformer_amd.fused_ops import MeanErrorNorm

pytestmark = pytest.mark.gpu


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(dtype).cuda()
    w = (torch.rand(cols, generator=g) + 0.5).to(torch.float64 if dtype == torch.float64 else torch.float32).cuda()
    dy = torch.randn(rows, cols, generator=g).to(dtype).cuda()
    return x, w, dy


def _bwd(x, w, dy):
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y = MeanErrorNorm.apply(xr, wr)
    y.backward(dy)
    return xr.grad, wr.grad


CASES = [
    # (dtype, rows, cols): grid G = min(2 per CU, ceil(rows / 4)) blocks
    (torch.bfloat16, 16384, 4096),  # config 2: G = 512 partial rows
    (torch.float32, 1, 768),        # one block
    (torch.float32, 3, 64),
    (torch.bfloat16, 9, 4096),      # G = 3
    (torch.float16, 1000, 2048),    # G = 250
    (torch.bfloat16, 4096, 32768),  # the widest rows of the resident kernels
    (torch.float64, 513, 8192),     # fp64 partials
    (torch.float32, 2000, 100),     # 100 columns: a partial last block of 16
]


@pytest.mark.parametrize("dtype,rows,cols", CASES)
def test_weight_gradient_against_oracle(gpu, dtype, rows, cols):
    print(f"norm dw: {dtype} {rows}x{cols}", flush=True)
    x, w, dy = _inputs(rows, cols, dtype, rows + cols)
    dx1, dw1 = _bwd(x, w, dy)
    for _ in range(3):  # fixed reduction order: the same bits every call
        dx2, dw2 = _bwd(x, w, dy)
        assert torch.equal(dx1, dx2)
        assert torch.equal(dw1, dw2)
    if rows * cols <= 4 * 1024 * 1024:
        # the kernels keep the row mean in fp32: the oracle takes it rounded the same way
        xd, wd = x.double().cpu(), w.double().cpu()
        mu = O.mean_error_norm_fwd(xd, wd)[1].float().double()
        dw_ref = O.mean_error_norm_bwd(dy.double().cpu(), xd, wd, mu)[1].numpy()
        got = dw1.double().cpu().numpy()
        tol = 1e-12 if dtype == torch.float64 else 1e-5
        err = np.abs(got - dw_ref).max() / max(np.abs(dw_ref).max(), 1e-30)
        print(f"  dw max rel err vs oracle {err:.2e}")
        assert err <= tol


def test_two_streams_at_once(gpu):
    """Backwards queued on two streams overlap; every result equals the same
    call made alone."""
    shapes = [(4096, 4096), (2048, 2048)]
    inputs = [_inputs(r, c, torch.bfloat16, 40 + i) for i, (r, c) in enumerate(shapes)]
    alone = [_bwd(*t) for t in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for _ in range(8):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i].append(_bwd(*inputs[i]))
    torch.cuda.synchronize()
    for i in range(2):
        for dx, dw in outs[i]:
            assert torch.equal(dx, alone[i][0])
            assert torch.equal(dw, alone[i][1])


def test_graph_replays(gpu):
    """A captured backward (through the C ABI with static buffers) replays to
    the eager result every time, with eager norm calls between replays."""
    rows, cols = 4096, 2048
    x, w, dy = _inputs(rows, cols, torch.bfloat16, 77)
    lib = _lib.load()
    mean = torch.empty(rows, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    dw = torch.empty(cols, dtype=torch.float32, device="cuda")
    ws_bytes = lib.kat_men_bwd_workspace_size(rows, cols, _lib.dtype_code(x))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")

    def call():
        st = _lib.stream(x)
        _lib.check(lib.kat_men_fwd(x.data_ptr(), w.data_ptr(), y.data_ptr(), mean.data_ptr(), rows, cols,
                                   cols, cols, 1e-5, _lib.dtype_code(x), _lib.dtype_code(w), st), "fwd")
        _lib.check(lib.kat_men_bwd(dy.data_ptr(), x.data_ptr(), w.data_ptr(), mean.data_ptr(),
                                   dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws_bytes, rows, cols,
                                   cols, cols, cols, 1e-5, _lib.dtype_code(x), _lib.dtype_code(w), st),
                   "bwd")

    call()
    torch.cuda.synchronize()
    dx_ref, dw_ref = dx.clone(), dw.clone()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()  # warm-up on the capture stream, outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=s):
        call()
    other = _inputs(1024, 2048, torch.bfloat16, 78)
    for _ in range(4):
        dx.zero_()
        dw.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_ref)
        assert torch.equal(dw, dw_ref)
        _bwd(*other)  # eager calls between replays
        torch.cuda.synchronize()
