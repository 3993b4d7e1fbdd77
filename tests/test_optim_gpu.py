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


def _tiny_bf16(seed):
    from oracle import step as O
    from tests.helpers import make_model
    dims = O.Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768, vocab=1024,
                  layers=4, eps=1e-6, theta=1e6)
    obj = O.Objective(loop_start=1, loop_end=3, mask_token_id=3, block_size=32)
    params = O.init_params(dims, obj.gate_init_pi, seed=seed)
    g = torch.Generator().manual_seed(seed)
    params["exit_gate.net.weight"] = 0.02 * torch.randn(1, dims.hidden, generator=g)
    model = make_model(dims, obj, params, dtype=torch.bfloat16)
    ids = torch.randint(0, dims.vocab, (512,), generator=g)
    return model, obj, ids, torch.tensor([0, 128, 256, 384, 512])


def _step_inputs(obj, ids, bounds, seed):
    from tests.helpers import cpu_draws
    draws, uniforms = cpu_draws(ids, bounds, obj.block_size, seed, obj.max_depth)
    return dict(draws=draws, exit_uniforms=[u.to(DEV) for u in uniforms])


def test_fused_optimizer_reads_float32_gradients():
    """Over exactly a model's parameters FusedAdamW binds to the model: the
    backward leaves .grad unset and keeps float32 gradients whose bf16
    rounding equals the .grad an unbound model gets for the same step
    (materialize_grads fills .grad with them); two backward calls without
    zero_grad accumulate (to float32 rounding of the two separate
    gradients); the first AdamW step equals its closed form on those float32
    gradients."""
    from alodlm_amd.optim import FusedAdamW, param_groups
    plain, obj, ids, bounds = _tiny_bf16(seed=6)
    fused, _, _, _ = _tiny_bf16(seed=6)
    opt = FusedAdamW(param_groups(fused, 0.01), lr=1e-3, max_grad_norm=1.0)
    kw = _step_inputs(obj, ids, bounds, 6)
    loss_a, _ = plain(ids.to(DEV), ids.to(DEV), bounds, **kw)
    loss_a.backward()
    loss_b, _ = fused(ids.to(DEV), ids.to(DEV), bounds, **kw)
    loss_b.backward()
    assert loss_a.item() == loss_b.item()
    assert all(p.grad is None for p in fused.parameters())
    f32 = {k: v.clone() for k, v in fused.float32_grads().items()}
    for name, p in plain.named_parameters():
        assert torch.equal(f32[name].to(torch.bfloat16), p.grad), name
    fused.materialize_grads()
    for name, p in fused.named_parameters():
        assert torch.equal(p.grad, f32[name].to(torch.bfloat16)), name
    # the first AdamW step on the float32 gradients
    masters0 = {n: p.detach().float().clone() for n, p in fused.named_parameters()}
    opt.step()
    torch.cuda.synchronize()
    norm = float(torch.sqrt(sum((g.double() ** 2).sum() for g in f32.values())))
    assert float(opt.last_grad_norm) == pytest.approx(norm, rel=1e-5)
    clip = min(1.0, 1.0 / (norm + 1e-6))
    groups = {id(p): grp["weight_decay"] for grp in opt.param_groups for p in grp["params"]}
    for name, p in fused.named_parameters():
        gi = f32[name].double() * clip
        wd = groups[id(p)]
        want = masters0[name].double() * (1 - 1e-3 * wd) - 1e-3 * gi / (gi.abs() + 1e-8)
        torch.testing.assert_close(opt.state[p]["master"].double(), want, atol=2e-6, rtol=1e-5,
                                   msg=name)
    # accumulation: two halves of two steps without zero_grad
    opt.zero_grad(set_to_none=True)
    assert fused.float32_grads() is None
    kw2 = _step_inputs(obj, ids, bounds, 7)
    parts = []
    for k in (kw, kw2):
        loss, _ = fused(ids.to(DEV), ids.to(DEV), bounds, **k)
        (loss / 2).backward()
        parts.append({n: g.clone() for n, g in fused.float32_grads().items()})
        opt.zero_grad(set_to_none=True)
    for k in (kw, kw2):
        loss, _ = fused(ids.to(DEV), ids.to(DEV), bounds, **k)
        (loss / 2).backward()
    acc = fused.float32_grads()
    for name, g in acc.items():
        want = parts[0][name] + parts[1][name]
        torch.testing.assert_close(g, want, rtol=1e-5, atol=1e-5 * want.abs().max().item(),
                                   msg=name)


def test_model_zero_grad_clears_bound_float32_gradients():
    """With a bound FusedAdamW, ``model.zero_grad()`` (nn.Module's, the loop
    model.zero_grad(); loss.backward(); opt.step()) clears the float32
    gradients too: each backward after it gives the gradients of that step
    alone, bit for bit the gradients of a fresh model on the same step."""
    from alodlm_amd.optim import FusedAdamW, param_groups
    model, obj, ids, bounds = _tiny_bf16(seed=8)
    fresh, _, _, _ = _tiny_bf16(seed=8)
    FusedAdamW(param_groups(model, 0.01), lr=1e-3, max_grad_norm=1.0)
    FusedAdamW(param_groups(fresh, 0.01), lr=1e-3, max_grad_norm=1.0)
    for seed in (8, 9, 10):
        kw = _step_inputs(obj, ids, bounds, seed)
        model.zero_grad()
        loss, _ = model(ids.to(DEV), ids.to(DEV), bounds, **kw)
        loss.backward()
        if fresh._engine is not None:
            fresh._engine.grads_pending = False   # a fresh step: the arena is overwritten
        loss_f, _ = fresh(ids.to(DEV), ids.to(DEV), bounds, **kw)
        loss_f.backward()
        got, want = model.float32_grads(), fresh.float32_grads()
        for name in want:
            assert torch.equal(got[name], want[name]), (seed, name)
    model.zero_grad()
    assert model.float32_grads() is None


def test_moving_bound_parameters_is_refused():
    """After a FusedAdamW bound the model's parameters, re-homing a parameter
    (which would leave the optimizer's tables pointing at freed memory) makes
    the next step raise instead of silently building a new arena."""
    from alodlm_amd.optim import FusedAdamW, param_groups
    model, obj, ids, bounds = _tiny_bf16(seed=8)
    opt = FusedAdamW(param_groups(model, 0.01), lr=1e-3)
    kw = _step_inputs(obj, ids, bounds, 8)
    loss, _ = model(ids.to(DEV), ids.to(DEV), bounds, **kw)
    loss.backward()
    opt.step()
    w = model.exit_gate.net.weight
    w.data = w.data.clone()
    with pytest.raises(RuntimeError, match="moved"):
        model(ids.to(DEV), ids.to(DEV), bounds, **kw)


def test_unbound_optimizer_rebuilds_tables_when_parameters_move():
    """An optimizer over standalone tensors follows a parameter given new
    storage: the update lands in the parameter's current storage."""
    from alodlm_amd.optim import FusedAdamW
    p = torch.nn.Parameter(torch.ones(1000, device=DEV, dtype=torch.bfloat16))
    opt = FusedAdamW([{"params": [p], "weight_decay": 0.0}], lr=0.1)
    p.grad = torch.ones_like(p)
    opt.step()
    first = p.detach().clone()
    p.data = p.data.clone()
    p.grad = torch.ones_like(p)
    opt.step()
    torch.cuda.synchronize()
    assert not torch.equal(p.detach(), first)


def test_optimizer_created_after_backward_applies_grad():
    """A FusedAdamW created after the backward (which then filled .grad, as
    for any model without a bound optimizer) steps on those .grad values, as
    torch.optim.AdamW would; after zero_grad a step changes nothing; the next
    backward goes to the float32 arena the optimizer now reads."""
    from alodlm_amd.optim import FusedAdamW, param_groups
    model, obj, ids, bounds = _tiny_bf16(seed=8)
    kw = _step_inputs(obj, ids, bounds, 8)
    loss, _ = model(ids.to(DEV), ids.to(DEV), bounds, **kw)
    loss.backward()
    grads = {n: p.grad.float().clone() for n, p in model.named_parameters()}
    opt = FusedAdamW(param_groups(model, 0.01), lr=1e-3, max_grad_norm=1.0)
    masters0 = {n: p.detach().float().clone() for n, p in model.named_parameters()}
    opt.step()
    torch.cuda.synchronize()
    norm = float(torch.sqrt(sum((g.double() ** 2).sum() for g in grads.values())))
    assert float(opt.last_grad_norm) == pytest.approx(norm, rel=1e-5)
    clip = min(1.0, 1.0 / (norm + 1e-6))
    groups = {id(p): grp["weight_decay"] for grp in opt.param_groups for p in grp["params"]}
    for name, p in model.named_parameters():
        gi = grads[name].double() * clip
        want = masters0[name].double() * (1 - 1e-3 * groups[id(p)]) - 1e-3 * gi / (gi.abs() + 1e-8)
        torch.testing.assert_close(opt.state[p]["master"].double(), want, atol=2e-6, rtol=1e-5,
                                   msg=name)
    opt.zero_grad(set_to_none=True)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(p.detach(), before[n]) for n, p in model.named_parameters())
    loss, _ = model(ids.to(DEV), ids.to(DEV), bounds, **kw)
    loss.backward()
    assert all(p.grad is None for p in model.parameters())
    assert model.float32_grads() is not None
    opt.step()
    torch.cuda.synchronize()
    assert not torch.equal(model.exit_gate.net.weight.detach(), before["exit_gate.net.weight"])
