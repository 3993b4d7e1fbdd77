"""Full training-step parity on the GPU.

* micro (the reference's tests/helpers.tiny_model, float32): loss, metrics,
  gates, exits and every gradient against the reference's golden vectors.
* tiny training-step configuration (hidden 256, 4 layers 1/2/1, 4 x 128
  tokens), float32: against the reference's golden vectors and the oracle,
  loss within 1e-5 relative.
* the same configuration in bf16: loss within 1e-2 relative and gradient
  cosine >= 0.999 against the float64 oracle run on the same bf16 weights;
  masks and exits bit-exact.
The draws (masking uniforms and permutations, exit uniforms) are consumed from
the CPU generator in the reference's order and replayed on the GPU.
"""

import numpy as np
import pytest
import torch

from oracle import step as O
from tests import golden
from tests.helpers import (cosine, cpu_draws, log, make_model, oracle_draws, oracle_name)

pytestmark = pytest.mark.gpu

MICRO = (O.Dims(hidden=32, heads=4, kv_heads=2, head_dim=8, intermediate=64, vocab=64, layers=3,
                eps=1e-6, theta=1e4),
         O.Objective(loop_start=1, loop_end=2, mask_token_id=3, block_size=4))
TINY = (O.Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768, vocab=1024,
               layers=4, eps=1e-6, theta=1e6),
        O.Objective(loop_start=1, loop_end=3, mask_token_id=3, block_size=32))


def _golden_name(name):
    return name if name.startswith("exit_gate.") else "backbone." + name


def _run_engine(model, ids, labels, bounds, draws, uniforms):
    engine = model.engine()
    out, state = engine.forward(ids.cuda(), labels.cuda(), bounds, True,
                                exit_uniforms=[u.cuda() for u in uniforms], draws=draws)
    grads = engine.backward(state, 1.0)
    torch.cuda.synchronize()
    named = {n: engine.arena.view(grads, n).cpu() for n in engine.arena.names}
    return out.cpu().double(), state, named


def _check_batch(state, g):
    b = state["batch"]
    np.testing.assert_array_equal(b.ids.cpu().numpy(), g["ids"])
    np.testing.assert_array_equal(b.original.cpu().numpy(), g["original"])
    np.testing.assert_array_equal(b.positions.cpu().numpy(), g["positions"])
    np.testing.assert_array_equal(b.masked.cpu().numpy(), g["masked"])
    np.testing.assert_array_equal(b.mask_probability.cpu().numpy(), g["mask_probability"])
    np.testing.assert_array_equal(b.boundaries.cpu().numpy(), g["boundaries"])


METRICS = ["denoising", "actor", "sampled_mean_depth", "prediction_cost", "regularization_cost",
           "profile_mean_depth", "first_pass_halt_probability", "ar_loss"]


@pytest.mark.parametrize("case", ["step_micro", "step_micro_ragged"])
def test_micro_step_matches_reference_golden(case):
    log(f"micro step {case}")
    g = golden.load(case)
    dims, obj = MICRO
    params = {n: torch.as_tensor(g["param_" + _golden_name(n)]) for n in O.param_names(dims)}
    model = make_model(dims, obj, params)
    labels = torch.as_tensor(g["in_labels"])
    draws, uniforms = cpu_draws(labels, g["in_boundaries"], obj.block_size, int(g["seed"]),
                                obj.max_depth)
    out, state, grads = _run_engine(model, torch.as_tensor(g["in_ids"]), labels,
                                    torch.as_tensor(g["in_boundaries"]), draws, uniforms)
    _check_batch(state, g)
    np.testing.assert_array_equal(state["exits"].cpu().numpy(), g["exits"])
    torch.testing.assert_close(state["gates"].cpu(), torch.as_tensor(g["gates"]), rtol=1e-5,
                               atol=1e-6)
    assert abs(out[0] - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    for i, key in enumerate(METRICS, 1):
        ref = float(g["metric_" + key])
        assert abs(out[i] - ref) <= 1e-5 * max(1.0, abs(ref)), key
    for name in O.param_names(dims):
        ref = torch.as_tensor(g["grad_" + _golden_name(name)])
        torch.testing.assert_close(grads[_golden_name(name)], ref, rtol=1e-4, atol=1e-6,
                                   msg=name)


def test_micro_step_autograd_path_fills_grads():
    """model(**item) + loss.backward() (alodlm/train.py:135,138) gives the engine's grads."""
    log("micro step autograd")
    g = golden.load("step_micro")
    dims, obj = MICRO
    params = {n: torch.as_tensor(g["param_" + _golden_name(n)]) for n in O.param_names(dims)}
    model = make_model(dims, obj, params)
    labels = torch.as_tensor(g["in_labels"])
    draws, uniforms = cpu_draws(labels, g["in_boundaries"], obj.block_size, int(g["seed"]),
                                obj.max_depth)
    loss, metrics = model(torch.as_tensor(g["in_ids"]).cuda(), labels.cuda(),
                          torch.as_tensor(g["in_boundaries"]),
                          exit_uniforms=[u.cuda() for u in uniforms], draws=draws)
    loss.backward()
    assert abs(float(loss) - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    assert set(metrics) == set(METRICS) | {"loss"}
    for name, p in model.named_parameters():
        ref = torch.as_tensor(g["grad_" + name])
        torch.testing.assert_close(p.grad.cpu(), ref, rtol=1e-4, atol=1e-6, msg=name)
    # a non-unit upstream gradient scales every parameter gradient
    model.zero_grad(set_to_none=True)
    loss, _ = model(torch.as_tensor(g["in_ids"]).cuda(), labels.cuda(),
                    torch.as_tensor(g["in_boundaries"]),
                    exit_uniforms=[u.cuda() for u in uniforms], draws=draws)
    (loss * -2.5).backward()
    for name, p in model.named_parameters():
        ref = -2.5 * torch.as_tensor(g["grad_" + name])
        torch.testing.assert_close(p.grad.cpu(), ref, rtol=1e-4, atol=3e-6, msg=name)


def _tiny_inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, 1024, (512,), generator=g)
    return ids, ids.clone(), torch.tensor([0, 128, 256, 384, 512])


def test_tiny_fp32_step_matches_reference_golden_and_oracle():
    log("tiny fp32 step")
    g = golden.load("step_tiny")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=0)
    model = make_model(dims, obj, params)
    ids, labels, bounds = _tiny_inputs()
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, 0, obj.max_depth)
    out, state, grads = _run_engine(model, ids, labels, bounds, draws, uniforms)
    _check_batch(state, g)
    np.testing.assert_array_equal(state["exits"].cpu().numpy(), g["exits"])
    # per-pass gate logits, hence halting probabilities, of the reference run
    torch.testing.assert_close(state["gates"].cpu(), torch.as_tensor(g["gates"]), rtol=1e-5,
                               atol=1e-6)
    assert abs(out[0] - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    for i, key in enumerate(METRICS, 1):
        ref = float(g["metric_" + key])
        assert abs(out[i] - ref) <= 1e-5 * max(1.0, abs(ref)), key
    names = list(g["param_names"])
    for index, gname in enumerate(names):
        grad = grads[gname].double().flatten()
        ref_norm = float(g["gnorm_" + gname])
        assert abs(grad.norm().item() - ref_norm) <= 1e-4 * ref_norm + 1e-9, gname
        proj = (grad * golden.projection_vector(index, grad.numel())).sum().item()
        assert abs(proj - float(g["gproj_" + gname])) <= 1e-4 * ref_norm * grad.numel() ** 0.5 + 1e-9
    # and against the oracle's full gradients
    p = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    od = oracle_draws(draws, [int(v) for v in bounds], obj.block_size)
    loss, _, _ = O.step_loss(p, ids, labels, bounds, dims, obj, od, uniforms)
    loss.backward()
    for name in O.param_names(dims):
        mine, ref = grads[_golden_name(name)].double(), p[name].grad.double()
        scale = ref.abs().max().item() + 1e-12
        assert (mine - ref).abs().max().item() <= 1e-4 * scale, name


def test_tiny_bf16_step_matches_oracle():
    log("tiny bf16 step")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=0)
    params = {k: v.to(torch.bfloat16) for k, v in params.items()}
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()}, dtype=torch.bfloat16)
    ids, labels, bounds = _tiny_inputs()
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, 0, obj.max_depth)
    out, state, grads = _run_engine(model, ids, labels, bounds, draws, uniforms)
    od = oracle_draws(draws, [int(v) for v in bounds], obj.block_size)
    # float64 oracle on the same bf16 weights, with the reference's bf16 rounding of
    # the LM-head logits and per-token CE (the values the actor's credit differences)
    p = {k: v.double().requires_grad_(True) for k, v in params.items()}
    loss, metrics, extra = O.step_loss(p, ids, labels, bounds, dims, obj, od, uniforms,
                                       ce_dtype=torch.bfloat16)
    loss.backward()
    np.testing.assert_array_equal(state["exits"].cpu().numpy(), extra["exits"].numpy())
    np.testing.assert_array_equal(state["batch"].masked.cpu().numpy(), extra["batch"]["masked"])
    assert abs(out[0] - loss.item()) <= 1e-2 * abs(loss.item())
    for d, ref in enumerate(extra["gates"]):
        diff = (torch.sigmoid(state["gates"][d].cpu().double()) - torch.sigmoid(ref.detach())).abs()
        assert diff.max().item() <= 1e-2, (d, diff.max().item())
    worst = 1.0
    for name in O.param_names(dims):
        c = cosine(grads[_golden_name(name)], p[name].grad)
        worst = min(worst, c)
        assert c >= 0.999, f"{name}: cosine {c}"
    # for information: the same comparison without any bf16 rounding in the oracle
    q = {k: v.double().requires_grad_(True) for k, v in params.items()}
    exact, _, _ = O.step_loss(q, ids, labels, bounds, dims, obj, od, uniforms)
    exact.backward()
    worst_exact = min(cosine(grads[_golden_name(n)], q[n].grad) for n in O.param_names(dims))
    log(f"tiny bf16: loss {out[0]:.6f} vs {loss.item():.6f} (unrounded {exact.item():.6f}); "
        f"worst grad cosine {worst:.6f} (unrounded oracle {worst_exact:.6f})")
    _compare_bf16_golden(out, state, grads)


def _compare_bf16_golden(out, state, grads):
    """The HIP bf16 step against the reference's own bf16 run of the same
    model (tests/golden/step_tiny_bf16.npz): masks and exits bit-exact,
    per-pass halting probabilities to 1e-3, the denoising and AR terms to
    2e-3 relative, the loss to 2e-2 relative, and every gradient's norm
    within 5 % and its strided sample at cosine >= 0.99 (0.98 for the gate).

    The loss bound is wider than the terms': the reference rounds every
    per-token CE to bf16 (an ulp of 0.03 at CE ~ 7) and the actor term
    multiplies sums of those values' differences by per-sequence sums of
    log q (about -90 here), so two bf16 runs that round a few CE values the
    other way differ by 1-2 % in the loss - the reference's own bf16 run is
    1.0e-2 from the float64 value of the same step.  Against the float64
    oracle with the same bf16 rounding points (above) the loss agrees to
    1e-2 and the gradients at cosine >= 0.999."""
    g = golden.load("step_tiny_bf16")
    _check_batch(state, g)
    np.testing.assert_array_equal(state["exits"].cpu().numpy(), g["exits"])
    halt = torch.sigmoid(state["gates"].cpu().double())
    ref_halt = torch.sigmoid(torch.as_tensor(g["gates"]).double())
    assert (halt - ref_halt).abs().max().item() <= 1e-3
    rel = abs(out[0] - float(g["loss"])) / abs(float(g["loss"]))
    terms = {key: (out[i], float(g["metric_" + key])) for i, key in enumerate(METRICS, 1)}
    log(f"tiny bf16 vs reference bf16 run: loss {out[0]:.6f} vs {float(g['loss']):.6f} "
        f"(rel {rel:.2e}); " + ", ".join(f"{k} {a:.5f}/{b:.5f}" for k, (a, b) in terms.items()))
    assert rel <= 2e-2
    for key in ("denoising", "ar_loss"):
        mine, ref = terms[key]
        assert abs(mine - ref) <= 2e-3 * abs(ref), key
    for index, gname in enumerate(g["param_names"]):
        grad = grads[str(gname)].double().flatten()
        ref_norm = float(g["gnorm_" + gname])
        assert abs(grad.norm().item() - ref_norm) <= 0.05 * ref_norm + 1e-12, gname
        sample = grad[torch.as_tensor(golden.sample_indices(grad.numel()))]
        c = cosine(sample, torch.as_tensor(g["gsample_" + gname]))
        # the gate's gradients reach it through log q of the actor term alone,
        # so they carry that term's bf16 CE noise in full (the float64 oracle
        # with the reference's rounding points scores 0.985 on depth_bias too)
        assert c >= (0.98 if str(gname).startswith("exit_gate.") else 0.99), (gname, c)


@pytest.mark.parametrize("keep", [(True, False), (True, True)])
def test_kept_forward_outputs_match_recompute(keep):
    """The backward gives the same bits whether it reuses the rotary q/k and
    the norm outputs kept from the forward or recomputes them (the policy the
    engine picks from its memory budget)."""
    log(f"kept forward outputs {keep}")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=1)
    model = make_model(dims, obj, params, dtype=torch.bfloat16)
    ids, labels, bounds = _tiny_inputs()
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, 1, obj.max_depth)
    engine = model.engine()
    results = []
    for policy in ((False, False), keep):
        engine._keep, engine._keep_rows = policy, 2 * len(ids)
        out, _, grads = _run_engine(model, ids, labels, bounds, draws, uniforms)
        results.append((out, grads))
    assert torch.equal(results[0][0], results[1][0])
    for name, g in results[0][1].items():
        # the embedding's rows of repeated ids are summed in a fixed order too
        assert torch.equal(g, results[1][1][name]), name


def test_tiny_step_without_masked_rows_or_targets():
    """A pack whose labels are all ignored (-100): no block has a candidate, so
    M = 0 and there is no autoregressive target.  The reference returns
    ce.sum() + 0 * gates = 0 with zero metrics (alodlm/loss.py:43-48) and an
    AR loss of 0 (loss.py:31-32); every gradient is zero."""
    log("tiny step, M = 0, no AR targets")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=2)
    model = make_model(dims, obj, params)
    ids, _, bounds = _tiny_inputs(seed=2)
    labels = torch.full_like(ids, -100)
    engine = model.engine()
    # a step with loss-bearing rows first, so the gradient arena holds values
    # the M = 0 step must overwrite (its matrices are written, not zeroed)
    gen = torch.Generator(device="cuda").manual_seed(2)
    out, state = engine.forward(ids.cuda(), ids.cuda(), bounds, True, generator=gen)
    engine.backward(state, 1.0)
    assert float(engine.grads.abs().sum()) > 0
    out, state = engine.forward(ids.cuda(), labels.cuda(), bounds, True, generator=gen)
    grads = engine.backward(state, 1.0)
    torch.cuda.synchronize()
    assert int(state["batch"].masked.sum()) == 0
    assert torch.equal(out.cpu()[:9], torch.zeros(9))
    assert torch.equal(grads.cpu(), torch.zeros_like(grads.cpu()))


def test_nonfinite_logits_or_readout_make_the_loss_nan():
    """The reference adds 0 * sum(logits + gates) to the loss
    (alodlm/model.py:186), over the logits of every row, so one non-finite
    logit anywhere makes the loss NaN while the metrics keep their values.
    On a pack whose labels are all ignored (no row carries loss, so no logit
    is computed here and every metric is 0): a finite model gives loss 0; a
    -inf or NaN LM-head weight (a non-finite logits column in every row)
    gives NaN; so does an infinite embedding row (non-finite readout rows,
    hence non-finite gate logits).  With loss-bearing rows a -inf LM-head
    weight gives NaN as well."""
    log("tiny step, non-finite LM head / readout")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=4)
    model = make_model(dims, obj, params)
    ids, _, bounds = _tiny_inputs(seed=4)
    labels = torch.full_like(ids, -100)
    engine = model.engine()
    gen = torch.Generator(device="cuda").manual_seed(4)

    def run(lab):
        out, _ = engine.forward(ids.cuda(), lab.cuda(), bounds, False, generator=gen)
        return out.cpu()

    assert torch.equal(run(labels)[:9], torch.zeros(9))
    W = model.backbone.lm_head.weight
    E = model.backbone.model.embed_tokens.weight
    for bad in (float("-inf"), float("nan")):
        with torch.no_grad():
            keep = W[5, 7].item()
            W[5, 7] = bad
        out = run(labels)
        assert torch.isnan(out[0]), bad
        assert torch.equal(out[1:9], torch.zeros(8)), bad
        with torch.no_grad():
            W[5, 7] = keep
    assert torch.equal(run(labels)[:9], torch.zeros(9))
    with torch.no_grad():
        row = E[int(ids[0])].clone()
        E[int(ids[0])] = float("inf")
    assert torch.isnan(run(labels)[0])
    with torch.no_grad():
        E[int(ids[0])] = row
        W[5, 7] = float("-inf")
    assert torch.isnan(run(ids)[0])


def test_tiny_step_without_masked_rows_matches_oracle():
    """Masking draws that mask nothing (every block's count round(n * p) = 0):
    M = 0, so the objective is the autoregressive loss alone; loss and every
    gradient against the oracle."""
    log("tiny step, M = 0 with AR targets")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=3)
    model = make_model(dims, obj, params)
    ids, labels, bounds = _tiny_inputs(seed=3)
    nblocks = sum(-(-(int(b) - int(a)) // obj.block_size) for a, b in zip(bounds, bounds[1:]))
    draws = (np.full(nblocks, 1e-8, dtype=np.float32), np.zeros(nblocks, dtype=np.int32),
             [None] * nblocks)
    uniforms = [torch.rand(2 * len(ids), generator=torch.Generator().manual_seed(d))
                for d in range(obj.max_depth - 1)]
    out, state, grads = _run_engine(model, ids, labels, bounds, draws, uniforms)
    assert int(state["batch"].masked.sum()) == 0
    p = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    od = oracle_draws(draws, [int(v) for v in bounds], obj.block_size)
    loss, metrics, _ = O.step_loss(p, ids, labels, bounds, dims, obj, od, uniforms)
    loss.backward()
    assert abs(out[0] - loss.item()) <= 1e-5 * abs(loss.item())
    assert abs(out[8] - metrics["ar_loss"].item()) <= 1e-5 * abs(metrics["ar_loss"].item())
    assert torch.equal(out[1:8], torch.zeros(7, dtype=out.dtype))
    for name in O.param_names(dims):
        mine, ref = grads[_golden_name(name)].double(), p[name].grad.double()
        scale = ref.abs().max().item() + 1e-12
        assert (mine - ref).abs().max().item() <= 1e-4 * scale, name
