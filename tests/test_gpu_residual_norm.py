"""The residual add fused with the mean-error norm (kat_add_men_fwd/bwd via
add_mean_error_norm) against the unfused pair it replaces -- torch's add
followed by mean_error_norm, with autograd summing h's two gradients and
casting the branch gradient. Both sides round identically, so outputs and
gradients must agree bit for bit; for fp32 / fp64 streams y and every
gradient are also checked against the CPU oracle (<= 1e-5 / 1e-12 relative,
with a floor of 1e-5 of the tensor's largest value for the gradients, whose
row sums cancel)."""

import pytest
import torch

import fastalgebraictransformer_amd as F
import oracle as O
from _util import assert_rel

pytestmark = pytest.mark.gpu


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).cuda()


CASES = [
    # (stream dtype, branch dtype, weight dtype, rows, cols)
    (torch.float32, torch.bfloat16, torch.float32, 300, 768),   # the model under autocast
    (torch.float32, torch.float32, torch.float32, 257, 768),
    (torch.float32, torch.float16, torch.float32, 64, 5000),    # several chunks per lane
    (torch.bfloat16, torch.bfloat16, torch.float32, 96, 1024),
    (torch.float16, torch.float16, torch.float16, 40, 512),
    (torch.float64, torch.float64, torch.float64, 33, 256),
    (torch.float32, torch.bfloat16, torch.float32, 50, 517),    # odd width: multi-pass kernels
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, 6, 33000),  # wider than the resident path
    (torch.float32, torch.bfloat16, torch.float32, 256, 2048),  # whole chunk rounds: the
    (torch.bfloat16, torch.bfloat16, torch.float32, 128, 4096),  # predicate-free kernels
]


@pytest.mark.parametrize("xd,rd,wd,rows,cols", CASES)
def test_fused_matches_add_then_norm(gpu, xd, rd, wd, rows, cols):
    seed = rows + cols
    x0 = _rand((rows, cols), xd, seed)
    r0 = _rand((rows, cols), rd, seed + 1, 0.5)
    w0 = (torch.rand(cols, generator=torch.Generator().manual_seed(seed + 2)) + 0.5).to(wd).cuda()
    dh = _rand((rows, cols), xd, seed + 3)
    dy = _rand((rows, cols), xd, seed + 4)

    xf, rf, wf = (t.clone().requires_grad_(True) for t in (x0, r0, w0))
    hf, yf = F.add_mean_error_norm(xf, rf, wf)
    torch.autograd.backward([hf, yf], [dh, dy])

    xu, ru, wu = (t.clone().requires_grad_(True) for t in (x0, r0, w0))
    hu = xu + ru
    yu = F.mean_error_norm(hu, wu)
    torch.autograd.backward([hu, yu], [dh, dy])

    assert hf.dtype == hu.dtype == xd
    assert torch.equal(hf, hu)
    assert torch.equal(yf, yu)
    assert torch.equal(xf.grad, xu.grad)
    assert rf.grad.dtype == rd and torch.equal(rf.grad, ru.grad)
    assert torch.equal(wf.grad, wu.grad)

    if xd in (torch.float32, torch.float64):
        # forward and backward against the oracle directly (fp64): the stream
        # gradient is dh plus the norm's dx at h, the branch gradient the same
        # in the branch dtype, and the weight gradient the norm's
        tol = 1e-5 if xd == torch.float32 else 1e-12
        h_ref = x0.cpu().double() + r0.cpu().double()
        y_ref, mu_ref = O.mean_error_norm_fwd(h_ref, w0.cpu())
        assert_rel(yf, y_ref, tol, "fused norm fwd vs oracle")
        dx_ref, dw_ref = O.mean_error_norm_bwd(dy.cpu(), h_ref, w0.cpu(), mu_ref)
        g_ref = dh.cpu().double() + dx_ref
        assert_rel(xf.grad, g_ref, tol, "fused norm bwd: stream gradient vs oracle", floor_frac=1e-5)
        if rd in (torch.float32, torch.float64):
            assert_rel(rf.grad, g_ref, tol, "fused norm bwd: branch gradient vs oracle", floor_frac=1e-5)
        assert_rel(wf.grad, dw_ref, tol, "fused norm bwd: weight gradient vs oracle", floor_frac=1e-5)


def test_fused_branch_without_grad_and_3d(gpu):
    x = _rand((2, 65, 768), torch.float32, 11).requires_grad_(True)
    r = _rand((2, 65, 768), torch.bfloat16, 12)          # no grad wanted
    w = torch.ones(768, device="cuda", requires_grad=True)
    h, y = F.add_mean_error_norm(x, r, w)
    assert h.shape == y.shape == x.shape
    y.sum().backward()
    assert r.grad is None and x.grad is not None and w.grad is not None
    x2 = x.detach().clone().requires_grad_(True)
    F.mean_error_norm(x2 + r, w.detach()).sum().backward()
    assert torch.equal(x.grad, x2.grad)


def test_fused_empty_rows(gpu):
    x = torch.empty(0, 64, device="cuda", requires_grad=True)
    r = torch.empty(0, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w = torch.ones(64, device="cuda", requires_grad=True)
    h, y = F.add_mean_error_norm(x, r, w)
    (h.sum() + y.sum()).backward()
    assert h.shape == (0, 64) and torch.equal(w.grad, torch.zeros(64, device="cuda"))


@pytest.mark.parametrize("rd,yd,rows,cols", [(torch.bfloat16, torch.bfloat16, 300, 768),
                                             (torch.bfloat16, torch.bfloat16, 200, 4096),
                                             (torch.float16, torch.float16, 64, 5000),
                                             (torch.bfloat16, torch.float16, 50, 517),
                                             (torch.float32, torch.bfloat16, 6, 33000)])
def test_fused_narrow_output_matches_norm_then_cast(gpu, rd, yd, rows, cols):
    # an fp32 stream whose norm output feeds an autocast matmul: y written in
    # the narrow dtype equals the fp32 y cast to it, and its narrow gradient
    # flows back as through the cast
    seed = 3 * rows + cols
    x0 = _rand((rows, cols), torch.float32, seed)
    r0 = _rand((rows, cols), rd, seed + 1, 0.5)
    w0 = (torch.rand(cols, generator=torch.Generator().manual_seed(seed + 2)) + 0.5).cuda()
    dh = _rand((rows, cols), torch.float32, seed + 3)
    dy = _rand((rows, cols), yd, seed + 4)

    xf, rf, wf = (t.clone().requires_grad_(True) for t in (x0, r0, w0))
    hf, yf = F.add_mean_error_norm(xf, rf, wf, out_dtype=yd)
    torch.autograd.backward([hf, yf], [dh, dy])

    xu, ru, wu = (t.clone().requires_grad_(True) for t in (x0, r0, w0))
    hu = xu + ru
    yu = F.mean_error_norm(hu, wu).to(yd)
    torch.autograd.backward([hu, yu], [dh, dy])

    assert yf.dtype == yd and hf.dtype == torch.float32
    assert torch.equal(hf, hu) and torch.equal(yf, yu)
    assert torch.equal(xf.grad, xu.grad)
    assert rf.grad.dtype == rd and torch.equal(rf.grad, ru.grad)
    assert torch.equal(wf.grad, wu.grad)
