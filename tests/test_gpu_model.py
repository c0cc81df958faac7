"""AlgebraicTransformerLM on the GPU kernels against the same module's CPU
path (the reference's torch formulation, algebraic_model.py:112-136)."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F

pytestmark = pytest.mark.gpu


def test_model_gpu_matches_cpu_path_fp32(gpu):
    torch.manual_seed(0)
    m = F.AlgebraicTransformerLM(vocab_size=1000, d_model=256, n_head=4, n_layers=2, dropout=0.0)
    ids = torch.randint(0, 1000, (2, 64))
    logits_c, loss_c = m(ids, labels=ids)
    loss_c.backward()
    grads_c = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad(set_to_none=True)
    mg = m.cuda()
    logits_g, loss_g = mg(ids.cuda(), labels=ids.cuda())
    loss_g.backward()
    # fp32 throughout; the CPU path includes the -1e4-filled keys (~6e-18 each)
    assert abs(loss_g.item() - loss_c.item()) <= 1e-5 * abs(loss_c.item())
    assert torch.allclose(logits_g.cpu(), logits_c, rtol=1e-4, atol=1e-4)
    for n, p in mg.named_parameters():
        gc = grads_c[n]
        err = float((p.grad.cpu() - gc).abs().max())
        assert err <= 1e-4 * max(1.0, float(gc.abs().max())), (n, err)


def test_model_small_bf16_autocast_step(gpu):
    # the reference model smoke test (tests.py:275-306) under bf16 autocast
    torch.manual_seed(0)
    m = F.AlgebraicTransformerLM(vocab_size=1000, d_model=256, n_head=4, n_layers=2).cuda()
    ids = torch.randint(0, 1000, (2, 64), device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        logits, loss = m(ids, labels=ids)
    loss.backward()
    assert math.isfinite(loss.item()) and abs(loss.item() - math.log(1000)) < 1.0
    gn = math.sqrt(sum(float(p.grad.float().norm()) ** 2 for p in m.parameters()))
    assert math.isfinite(gn) and gn > 0


@pytest.mark.parametrize("ckpt", [False, True])
def test_model_autocast_narrow_norm_outputs_change_no_bits(gpu, monkeypatch, ckpt):
    # under autocast the fused norms write their outputs in bf16 directly;
    # with that switched off (fp32 outputs, cast by the matmuls) the step
    # must give the same logits, loss and gradients bit for bit
    from fastalgebraictransformer_amd import algebraic_model as AM
    torch.manual_seed(2)
    m = F.AlgebraicTransformerLM(vocab_size=700, d_model=256, n_head=4, n_layers=3,
                                 dropout=0.0, gradient_checkpointing=ckpt).cuda()
    ids = torch.randint(0, 700, (2, 96), device="cuda")
    runs = []
    for narrow in (True, False):
        if not narrow:
            monkeypatch.setattr(AM, "_narrow", lambda x: None)
        m.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits, loss = m(ids, labels=ids)
        loss.backward()
        runs.append((logits.detach().clone(), loss.detach().clone(),
                     [p.grad.clone() for p in m.parameters()]))
    (la, sa, ga), (lb, sb, gb) = runs
    assert torch.equal(la, lb) and torch.equal(sa, sb)
    for a, b in zip(ga, gb):
        assert torch.equal(a, b)


def test_model_gradient_checkpointing_matches(gpu):
    torch.manual_seed(1)
    m = F.AlgebraicTransformerLM(vocab_size=500, d_model=128, n_head=2, n_layers=2,
                                 dropout=0.0).cuda()
    ids = torch.randint(0, 500, (2, 48), device="cuda")
    _, l1 = m(ids, labels=ids)
    l1.backward()
    g1 = [p.grad.clone() for p in m.parameters()]
    m.zero_grad(set_to_none=True)
    m.gradient_checkpointing = True
    _, l2 = m(ids, labels=ids)
    l2.backward()
    assert torch.equal(l1, l2)
    for a, p in zip(g1, m.parameters()):
        assert torch.equal(a, p.grad)


def test_model_padding_mask_gpu_matches_cpu_path(gpu):
    # the GPU path now applies attention_mask as the reference CPU path does
    # (algebraic_model.py:129-131); dropped keys contribute exactly 0 here and
    # sigma(-1e4)^4 ~ 6e-18 there
    torch.manual_seed(2)
    m = F.AlgebraicTransformerLM(vocab_size=300, d_model=128, n_head=2, n_layers=2, dropout=0.0)
    ids = torch.randint(0, 300, (2, 70))
    mask = torch.ones(2, 70, dtype=torch.long)
    mask[0, :10] = 0
    mask[1, 50:] = 0
    logits_c, loss_c = m(ids, labels=ids, attention_mask=mask)
    loss_c.backward()
    grads_c = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad(set_to_none=True)
    mg = m.cuda()
    logits_g, loss_g = mg(ids.cuda(), labels=ids.cuda(), attention_mask=mask.cuda())
    loss_g.backward()
    assert abs(loss_g.item() - loss_c.item()) <= 1e-5 * abs(loss_c.item())
    assert torch.allclose(logits_g.cpu(), logits_c, rtol=1e-4, atol=1e-4)
    for n, p in mg.named_parameters():
        gc = grads_c[n]
        err = float((p.grad.cpu() - gc).abs().max())
        assert err <= 1e-4 * max(1.0, float(gc.abs().max())), (n, err)
    # and the mask matters: without it the logits differ
    with torch.no_grad():
        unmasked, _ = mg(ids.cuda())
    assert not torch.allclose(unmasked.cpu(), logits_c, rtol=1e-3, atol=1e-3)


def test_bf16_training_tracks_cpu_fp32(gpu):
    # end to end: 30 AdamW steps of a small model on one fixed batch, the GPU
    # under bf16 autocast (MFMA attention, fused norms, packed SwiGLU) against
    # the same model in fp32 on the CPU (the reference formulation); the loss
    # curves must agree within bf16 training noise and the loss must fall
    import copy
    torch.manual_seed(0)
    m_cpu = F.AlgebraicTransformerLM(vocab_size=128, d_model=128, n_head=2, n_layers=2,
                                     dropout=0.0, block_size=64)
    m_gpu = copy.deepcopy(m_cpu).cuda()
    ids = torch.randint(0, 128, (8, 64), generator=torch.Generator().manual_seed(1))
    opt_c = torch.optim.AdamW(m_cpu.parameters(), lr=2e-3)
    opt_g = torch.optim.AdamW(m_gpu.parameters(), lr=2e-3)
    lc, lg = [], []
    for _ in range(30):
        opt_c.zero_grad(set_to_none=True)
        _, loss = m_cpu(ids, labels=ids)
        loss.backward()
        opt_c.step()
        lc.append(loss.item())
        opt_g.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = m_gpu(ids.cuda(), labels=ids.cuda())
        loss.backward()
        opt_g.step()
        lg.append(loss.item())
    assert lg[-1] < 0.7 * lg[0], lg
    # The first steps track the fp32 run closely (measured < 0.3%), which a
    # wrong or missing gradient term would break at once. Later steps of this
    # memorise-one-batch run amplify bf16 rounding chaotically: over 8 seeds the
    # final losses differed from the fp32 run by -14% .. +7%, with random signs,
    # so they only have to stay within 20%.
    for i, (a, b) in enumerate(zip(lc, lg)):
        assert abs(a - b) <= (0.01 if i < 10 else 0.2) * a, (i, lc, lg)
