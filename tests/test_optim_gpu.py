"""FusedAdamW on the GPU against the reference's clipped torch.optim.AdamW step
(alodlm/train.py:42-56,138-148) recorded for the micro model: the same
parameters and gradients, global-norm clip at 1.0, the reference's two
weight-decay groups, one step."""

import numpy as np
import pytest
import torch

from tests.golden import load

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
NO_DECAY = ("bias", "LayerNorm.weight", "layer_norm.weight")


def golden_params(layout):
    """(name, param, grad) from the micro golden, as standalone tensors or as
    views into one flat buffer at odd element offsets (unaligned rows)."""
    g = load("step_micro")
    names = [str(n) for n in g["param_names"]]
    params, grads = [], []
    if layout == "standalone":
        for n in names:
            params.append(torch.nn.Parameter(torch.from_numpy(g["param_" + n]).float().to(DEV)))
            grads.append(torch.from_numpy(g["grad_" + n]).float().to(DEV))
    else:
        total = sum(g["param_" + n].size + 1 for n in names)
        flat = torch.empty(total, dtype=torch.float32, device=DEV)
        gflat = torch.empty(total, dtype=torch.float32, device=DEV)
        off = 1
        for n in names:
            a, ga = g["param_" + n], g["grad_" + n]
            view = flat[off:off + a.size].view(a.shape)
            view.copy_(torch.from_numpy(a).float())
            p = torch.nn.Parameter(view)
            gview = gflat[off:off + a.size].view(a.shape)
            gview.copy_(torch.from_numpy(ga).float())
            params.append(p)
            grads.append(gview)
            off += a.size + 1
    return g, names, params, grads


@pytest.mark.parametrize("layout", ["standalone", "offset views"])
def test_fused_adamw_matches_reference_step(layout):
    from alodlm_amd.optim import FusedAdamW
    g, names, params, grads = golden_params(layout)
    for p, gr in zip(params, grads):
        p.grad = gr
    groups = [
        {"params": [p for n, p in zip(names, params) if not any(s in n for s in NO_DECAY)],
         "weight_decay": 0.01},
        {"params": [p for n, p in zip(names, params) if any(s in n for s in NO_DECAY)],
         "weight_decay": 0.0},
    ]
    opt = FusedAdamW(groups, lr=float(g["lr"]), max_grad_norm=1.0)
    opt.step()
    torch.cuda.synchronize()
    assert float(opt.last_grad_norm) == pytest.approx(float(g["grad_total_norm"]), rel=1e-6)
    for n, p in zip(names, params):
        want = torch.from_numpy(g["updated_" + n]).double()
        torch.testing.assert_close(p.detach().cpu().double(), want, atol=2e-7, rtol=1e-6, msg=n)


def test_fused_adamw_bf16_parameters_keep_float32_masters():
    """bf16 parameters: the update runs on float32 masters initialised from
    them; the parameters are the masters rounded to bf16."""
    from alodlm_amd.optim import FusedAdamW
    g, names, params, grads = golden_params("standalone")
    bparams = [torch.nn.Parameter(p.detach().to(torch.bfloat16)) for p in params]
    for p, gr in zip(bparams, grads):
        p.grad = gr.to(torch.bfloat16)
    opt = FusedAdamW([{"params": bparams, "weight_decay": 0.01}], lr=float(g["lr"]),
                     max_grad_norm=1.0)
    opt.step()
    torch.cuda.synchronize()
    # the first step in closed form (float64): m_hat = g, v_hat = g^2, so the
    # update is -lr * g / (|g| + eps) after the decay w * (1 - lr * wd)
    lr = float(g["lr"])
    norm = float(torch.sqrt(sum((x.grad.double() ** 2).sum() for x in bparams)))
    clip = min(1.0, 1.0 / (norm + 1e-6))
    for p, q in zip(bparams, params):
        master = opt.state[p]["master"]
        assert master.dtype == torch.float32
        assert torch.equal(p.detach(), master.to(torch.bfloat16))
        w0 = q.detach().to(torch.bfloat16).double().cpu()
        gi = p.grad.double().cpu() * clip
        want = w0 * (1 - lr * 0.01) - lr * gi / (gi.abs() + 1e-8)
        torch.testing.assert_close(master.double().cpu(), want, atol=1e-6, rtol=1e-5)
