"""The training step at the benchmark configurations' real shapes (bf16,
head_dim 128, vocabulary 151936).

Parity against the float32 oracle on the same bf16 weights (CPU, seconds to
a minute):

* Qwen3-1.7B layer shapes (hidden 2048, 16/8 heads, intermediate 6144), two
  layers run as the recurrent core (loop 0-2), K = 4, one 2048-token segment:
  the head_dim-128 attention with the dK/dV pass split by query head, the
  register-resident 151936-wide cross-entropy, the LM head's split-K dX;
* Qwen3-8B layer shapes (hidden 4096, 32/8 heads, intermediate 12288),
  prelude / core / coda of one layer each, one 1024-token segment.

Masks and permutations are compared bit for bit with torch's own device
draws from the same generator state, exits bit for bit with the exit rule
applied to the step's own gates and uniforms, and the oracle then follows
the step's exits.  Every masked row's cross-entropy at every depth before its
exit within two bf16 steps (mean 0.03, half a step); denoising and autoregressive terms
within 1e-2 relative; the loss within 1e-2 of the size of its terms
((|denoising| + |actor| + |AR|) / 2: the actor is negative and cancels
part of the others) when the credit's gradient-free prediction cost uses
the step's cross-entropies (otherwise the bf16 rounding of those values
alone moves the actor term by about 4 % at one 2048-token segment); gate logits of sampled rows within one bf16 step of a
CPU recompute from the step's own readout; per-pass halting probabilities
within 5e-2 of the oracle's (mean 5e-3); dL/dgate equal to the oracle's
autograd of the objective on the step's own values (1e-4) and the gate's
parameter gradients equal to their sums over it; every other parameter
gradient at cosine >= 0.999 (the 4-element depth bias at 0.99: its
gradient is a zero-mean score-function sum that bf16 gate rounding shifts).

Properties at full size (the 1.7B step, 8 x 2048 tokens; the 8B step, 1 x
2048 tokens, 36 layers): masks and exits as above, the loss and metrics equal
to the oracle objective recomputed in float64 from the step's own
cross-entropies, gates, exits and masks (1e-4 relative), 64 sampled
cross-entropies equal to a float32 CPU recompute from the step's readout
rows (one bf16 rounding step), and finite gradients.
"""

import gc
import math

import numpy as np
import pytest
import torch

from oracle import step as O
from tests.helpers import cosine, draw_masking, log, make_model, oracle_draws

pytestmark = pytest.mark.gpu

VOCAB = 151936
MASK_ID = 151665
METRICS = ["denoising", "actor", "sampled_mean_depth", "prediction_cost", "regularization_cost",
           "profile_mean_depth", "first_pass_halt_probability", "ar_loss"]


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _dims(hidden, heads, kv_heads, intermediate, layers):
    return O.Dims(hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=128,
                  intermediate=intermediate, vocab=VOCAB, layers=layers, eps=1e-6, theta=1e6)


def _bf16_params(dims, obj, seed):
    """N(0, 0.02) backbone, norm weights 1 + N(0, 0.05) and a gate with
    N(0, 0.02) weights (so halting probabilities vary by row), in bf16."""
    params = O.init_params(dims, obj.gate_init_pi, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    for name, value in params.items():
        if name.endswith("norm.weight"):
            params[name] = 1 + 0.05 * torch.randn(value.shape, generator=g)
    params["exit_gate.net.weight"] = 0.02 * torch.randn(1, dims.hidden, generator=g)
    return {k: v.to(torch.bfloat16) for k, v in params.items()}


def _tokens(lengths, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, VOCAB, (sum(lengths),), generator=g)
    bounds = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int64)
    return ids, ids.clone(), bounds


def _run_step(model, ids, labels, bounds, seed):
    """One forward + backward drawing from a seeded CUDA generator, then the
    reference's own draws (alodlm/batch.py:50-60, alodlm/model.py:166) replayed
    from the same generator state."""
    engine, K = model.engine(), model.config.max_depth
    gen = torch.Generator(device="cuda").manual_seed(seed)
    start = gen.get_state()
    out, state = engine.forward(ids.cuda(), labels.cuda(), bounds, True, generator=gen)
    end = gen.get_offset()
    grads = engine.backward(state, 1.0)
    torch.cuda.synchronize()
    gen.set_state(start)
    offsets = [int(v) for v in bounds]
    draws = draw_masking(labels.numpy(), offsets, model.config.block_size, "cuda", gen)
    uniforms = [torch.rand(2 * len(ids), device="cuda", generator=gen) for _ in range(K - 1)]
    assert gen.get_offset() == end, "the step consumed a different amount of randomness"
    return out.cpu().double(), state, grads, draws, uniforms


def _check_batch(state, ids, labels, bounds, draws, cfg):
    offsets = [int(v) for v in bounds]
    ref = O.build_batch(ids, labels, bounds, cfg.block_size, cfg.mask_token_id,
                        oracle_draws(draws, offsets, cfg.block_size))
    b = state["batch"]
    for key, got in (("ids", b.ids), ("original", b.original), ("positions", b.positions),
                     ("masked", b.masked), ("mask_probability", b.mask_probability),
                     ("boundaries", b.boundaries)):
        np.testing.assert_array_equal(got.cpu().numpy(), ref[key], err_msg=key)
    return ref


def _check_exits(state, uniforms, K):
    """Exits equal the rule of alodlm/model.py:163-168 applied to the step's own
    gates and uniforms (rows whose uniform is within 1e-6 of the hazard may
    round either way and are not counted)."""
    gates, exits, masked = state["gates"], state["exits"].long(), state["batch"].masked
    expect = torch.full_like(exits, K)
    tie = torch.zeros_like(masked)
    for d in range(K - 1):
        hazard = torch.sigmoid(gates[d])
        tie |= masked & (expect == K) & ((uniforms[d] - hazard).abs() < 1e-6)
        chosen = (uniforms[d] < hazard) & masked & (expect == K)
        expect = torch.where(chosen, d + 1, expect)
    bad = (expect != exits) & ~tie
    assert int(bad.sum()) == 0, f"{int(bad.sum())} exits differ from the rule"
    assert int(tie.sum()) <= 2
    return exits.cpu()


def _replay_uniforms(exits, K):
    """Uniforms that make the oracle take exactly these exits: 0 at the depth a
    row exits (0 < hazard), 1 elsewhere (hazard < 1)."""
    return [torch.where(exits == d + 1, 0.0, 1.0) for d in range(K - 1)]


def _objective_from_step(state, cfg):
    """Loss and metrics of alodlm/model.py:176-187 recomputed in float64 by the
    oracle from the step's own cross-entropies, gates, exits and masks."""
    b = state["batch"]
    masked = b.masked.cpu()
    ce = state["ce"].cpu().double()
    gates = list(state["gates"].cpu().double())
    den_actor, metrics = O.outcome_loss(ce[:, masked], gates, state["exits"].cpu().long(), masked,
                                        b.mask_probability.cpu(), b.boundaries.cpu(), cfg)
    ar_rows = b.ar_target.cpu() >= 0
    ar = (ce[:, ar_rows].sum(1) / int(ar_rows.sum())).mean() if bool(ar_rows.any()) else 0.0
    metrics = {k: float(v) for k, v in metrics.items()}
    metrics["ar_loss"] = float(ar)
    return float((den_actor + ar) / 2), metrics


def _check_gates_from_readout(state, model, rows=256):
    """Gate logits of sampled rows recomputed on the CPU from the step's own
    bf16 readout: round(round(w . x + b) + depth_bias[d]) in bf16
    (alodlm/model.py:37-38, 162), within one bf16 step of the logit."""
    gate = model.exit_gate
    w = gate.net.weight.detach().float().cpu()[0]
    b = gate.net.bias.detach().float().cpu()[0]
    db = gate.depth_bias.detach().float().cpu()
    g = torch.Generator().manual_seed(0)
    for d, rec in enumerate(state["depths"]):
        idx = torch.randperm(rec["readout"].shape[0], generator=g)[:rows]
        x = rec["readout"][idx.cuda()].float().cpu()
        logit = ((x @ w + b).to(torch.bfloat16).float() + db[d]).to(torch.bfloat16).float()
        got = state["gates"][d].cpu()[idx]
        for v, r in zip(got.tolist(), logit.tolist()):
            assert abs(v - r) <= _bf16_ulp(r) + 1e-6, (d, v, r)


def _check_gate_gradients(state, named, cfg):
    """dL/dgate of the objective kernel against the oracle's autograd of
    alodlm/loss.py:35-90 on the step's own cross-entropies, gates and exits
    (float64), and the gate's parameter gradients against the sums they are
    (net.weight = sum_d dgate_d . readout_d, net.bias = sum dgate,
    depth_bias[d] = sum_rows dgate_d) over the step's own dL/dgate and bf16
    readout rows."""
    b = state["batch"]
    masked = b.masked.cpu()
    ce = state["ce"].cpu().double()[:, masked]
    gates = state["gates"].cpu().double().requires_grad_(True)
    den_actor, _ = O.outcome_loss(ce, list(gates), state["exits"].cpu().long(), masked,
                                  b.mask_probability.cpu(), b.boundaries.cpu(), cfg)
    (den_actor / 2).backward()
    ref = gates.grad
    got = state["dgate"].cpu().double()
    assert (got - ref).abs().max().item() <= 1e-4 * ref.abs().max().item() + 1e-9
    dgate = state["dgate"]
    dw = sum(dgate[d][None, :] @ rec["readout"].float() for d, rec in enumerate(state["depths"]))
    torch.testing.assert_close(named["exit_gate.net.weight"], dw.cpu(), rtol=1e-4,
                               atol=1e-4 * dw.abs().max().item())
    bias = dgate.sum()
    assert abs(named["exit_gate.net.bias"].item() - bias.item()) <= 1e-4 * abs(bias.item()) + 1e-7
    torch.testing.assert_close(named["exit_gate.depth_bias"], dgate.sum(1).cpu(), rtol=1e-4,
                               atol=1e-7)


def _bf16_ulp(v):
    return 2.0 ** (math.floor(math.log2(max(abs(v), 1e-30))) - 7)


def _check_sampled_ce(state, lm_head, count=64, seed=0):
    """Cross-entropies of sampled loss-bearing rows against a float32 CPU
    recompute from the step's readout rows: logits rounded to bf16 as the
    LM-head product stores them, CE = logsumexp - logit[target] rounded to
    bf16 (alodlm/model.py:180-181 in bf16); and their token entropies
    -sum p log p of the same logits (alodlm/inference.py:114-117) to 2e-3."""
    b = state["batch"]
    W = lm_head.detach().float().cpu()
    g = torch.Generator().manual_seed(seed)
    K = len(state["depths"])
    checked = 0
    for d, rec in enumerate(state["depths"]):
        R = rec["R"]
        if R == 0:
            continue
        pick = torch.randperm(R, generator=g)[:count // K]
        rows = rec["sel_rows"][:R].cpu()[pick].long()
        x = rec["readout"][rows.cuda()].float().cpu()
        logits = (x @ W.T).to(torch.bfloat16).float()
        masked = b.masked.cpu()[rows]
        target = torch.where(masked, b.original.cpu()[rows], b.ar_target.cpu()[rows].long())
        ref = (torch.logsumexp(logits, -1) - logits.gather(1, target[:, None]).squeeze(1))
        got = state["ce"][d].cpu()[rows]
        for r, v in zip(ref.tolist(), got.tolist()):
            assert abs(v - r) <= _bf16_ulp(r) + 2e-3, (d, v, r)
        logp = logits.log_softmax(-1)
        ent = -(logp.exp() * logp).sum(-1)
        got_ent = state["entropy"][d].cpu()[rows]
        assert bool(((got_ent - ent).abs() <= 2e-3).all()), (d, (got_ent - ent).abs().max())
        checked += len(rows)
    assert checked >= count // 2


def _compare_with_oracle(model, params, dims, obj, ids, labels, bounds, seed):
    log(f"real shapes: hidden {dims.hidden}, {dims.heads}/{dims.kv_heads} heads, "
        f"{dims.layers} layers, segments {bounds.tolist()}")
    K = obj.max_depth
    out, state, grads, draws, uniforms = _run_step(model, ids, labels, bounds, seed)
    engine = model.engine()
    named = {n: engine.arena.view(grads, n).cpu() for n in engine.arena.names}
    hip_gates = state["gates"].cpu()
    _check_gates_from_readout(state, model)
    _check_gate_gradients(state, named, obj)
    masked = state["batch"].masked.cpu()
    hip_ce = state["ce"].cpu()[:, masked].double()
    _check_batch(state, ids, labels, bounds, draws, obj)
    exits = _check_exits(state, uniforms, K)
    del state, grads
    gc.collect()
    torch.cuda.empty_cache()
    log("oracle (float32, CPU)")
    # The oracle follows the step's exits and rounds logits and cross-entropies
    # to bf16 as the reference's bf16 run does.  The credit's prediction cost
    # (a sampled cost without gradient, alodlm/loss.py:72-78) takes the step's
    # own cross-entropies: each is rounded to bf16 (steps of 1/16 near the
    # 151936-vocabulary entropy), and the actor multiplies their mean by the
    # sum of log q over the segment's masked rows (about -1.4 per row), so two
    # bf16 evaluations of the same step - the reference's included - differ
    # by about 1/32 * sqrt(M) * 1.4 in the loss from rounding alone.
    p = {k: v.float().requires_grad_(True) for k, v in params.items()}
    od = oracle_draws(draws, [int(v) for v in bounds], obj.block_size)
    loss, metrics, extra = O.step_loss(p, ids, labels, bounds, dims, obj, od,
                                       _replay_uniforms(exits, K), ce_dtype=torch.bfloat16,
                                       credit_ce=hip_ce)
    loss.backward()
    assert torch.equal(extra["exits"], exits)
    # per-token cross-entropies of every masked row at the depths before its exit
    z = exits[masked]
    live = torch.arange(K)[:, None] < z[None, :]
    ref_ce = extra["ce"].detach().double()
    diff = (hip_ce - ref_ce).abs()[live]
    ulp = torch.tensor([_bf16_ulp(v) for v in ref_ce[live].tolist()], dtype=torch.float64)
    # at most two bf16 steps anywhere, and less than half a step (1/32 near the
    # 151936-vocabulary entropy) on average: most rows round to the same value
    assert bool((diff <= 2 * ulp + 1e-3).all()), diff.max().item()
    assert diff.mean().item() <= 0.03, diff.mean().item()
    assert abs(out[1] - metrics["denoising"].item()) <= 1e-2 * abs(metrics["denoising"].item())
    assert abs(out[8] - metrics["ar_loss"].item()) <= 1e-2 * abs(metrics["ar_loss"].item())
    # The loss is (denoising + actor + AR) / 2, whose terms partly cancel (the
    # actor is negative): its error is taken relative to the terms' magnitude.
    terms = (abs(metrics["denoising"].item()) + abs(metrics["actor"].item())
             + abs(metrics["ar_loss"].item())) / 2
    log(f"terms (denoising, actor, AR): step {out[1]:.5f} {out[2]:.5f} {out[8]:.5f}; oracle "
        f"{metrics['denoising'].item():.5f} {metrics['actor'].item():.5f} "
        f"{metrics['ar_loss'].item():.5f}")
    assert abs(out[0] - loss.item()) <= 1e-2 * terms, (out[0], loss.item(), terms)
    # for information: the oracle's loss with its own cross-entropies in the credit
    plain, _ = O.outcome_loss(ref_ce, [g.detach().double() for g in extra["gates"]], exits,
                              masked, extra["batch"]["mask_probability"],
                              extra["batch"]["boundaries"], obj)
    plain = (plain + metrics["ar_loss"].double()) / 2
    # halting probabilities against the float32 oracle: the step's readout
    # carries bf16 rounding through every layer application (2 more per depth)
    # and the gate logit is rounded to bf16 twice, as the reference's bf16 gate
    # does, so the gap grows with depth
    gaps = []
    for d in range(K):
        got = torch.sigmoid(hip_gates[d].double())
        ref = torch.sigmoid(extra["gates"][d].detach().double())
        gap = (got - ref).abs()
        gaps.append((round(gap.mean().item(), 5), round(gap.max().item(), 5)))
    log(f"halting probability |diff| (mean, max) per depth: {gaps}")
    assert all(mean <= 5e-3 and top <= 5e-2 for mean, top in gaps), gaps
    # Every gradient against the float32 oracle at cosine >= 0.999, except the
    # 4-element depth bias: its gradient sums the score function dlog q/dg over
    # the masked rows, a sum of zero expectation (about sqrt(M) in size) whose
    # bf16-rounded gates shift it by about M times their rounding, so it is
    # held to 0.99 here and checked exactly against the step's own dL/dgate
    # above.
    worst, worst_name = 1.0, None
    for name in O.param_names(dims):
        key = name if name.startswith("exit_gate.") else "backbone." + name
        c = cosine(named[key], p[name].grad)
        if name == "exit_gate.depth_bias":
            assert c >= 0.99, f"{name}: cosine {c}"
            continue
        if c < worst:
            worst, worst_name = c, name
        assert c >= 0.999, f"{name}: cosine {c}"
    log(f"loss {out[0]:.5f} vs oracle {loss.item():.5f} (with its own cross-entropies in the "
        f"credit {plain.item():.5f}); CE |diff| mean {diff.mean().item():.4f} max "
        f"{diff.max().item():.4f}; worst gradient cosine {worst:.6f} ({worst_name})")


def test_1p7b_layer_shapes_match_oracle():
    dims = _dims(2048, 16, 8, 6144, layers=2)
    obj = O.Objective(loop_start=0, loop_end=2, mask_token_id=MASK_ID, block_size=32)
    params = _bf16_params(dims, obj, seed=11)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()},
                       dtype=torch.bfloat16)
    ids, labels, bounds = _tokens([2048], seed=11)
    _compare_with_oracle(model, params, dims, obj, ids, labels, bounds, seed=11)


def test_8b_layer_shapes_match_oracle():
    dims = _dims(4096, 32, 8, 12288, layers=3)
    obj = O.Objective(loop_start=1, loop_end=2, mask_token_id=MASK_ID, block_size=32)
    params = _bf16_params(dims, obj, seed=12)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()},
                       dtype=torch.bfloat16)
    ids, labels, bounds = _tokens([1024], seed=12)
    # one short segment: few key tiles per key-value head, so the dK/dV pass
    # is split by query head (its workspace holds the float32 partials)
    from alodlm_amd import _lib
    assert (_lib.query("alodlm_attention_bwd_workspace", 2048, 32, 8, 128, 16, 0)
            > 2 * 2048 * 32)
    _compare_with_oracle(model, params, dims, obj, ids, labels, bounds, seed=12)


def _full_size(name, seed):
    import bench
    spec = bench.MODELS[name]
    log(f"full-size {spec['name']} step")
    model = bench.build_model(spec, torch.device("cuda", 0), torch.bfloat16, seed=seed)
    ids, labels, bounds = _tokens(spec["segments"], seed)
    out, state, grads, draws, uniforms = _run_step(model, ids, labels, bounds, seed)
    cfg = model.config
    _check_batch(state, ids, labels, bounds, draws, cfg)
    _check_exits(state, uniforms, cfg.max_depth)
    total, metrics = _objective_from_step(state, cfg)
    assert abs(out[0] - total) <= 1e-4 * abs(total) + 1e-6, (out[0], total)
    for i, key in enumerate(METRICS, 1):
        assert abs(out[i] - metrics[key]) <= 1e-4 * max(1.0, abs(metrics[key])), key
    _check_sampled_ce(state, model.backbone.lm_head.weight, seed=seed)
    _check_gates_from_readout(state, model)
    assert bool(torch.isfinite(grads).all())
    engine = model.engine()
    for layer_name in engine.arena.names:
        if layer_name.endswith("_proj.weight"):
            assert engine.arena.view(grads, layer_name).norm().item() > 0, layer_name
    log(f"{spec['name']}: loss {out[0]:.5f} (objective from the step's own outputs "
        f"{total:.5f}); masked rows {int(state['batch'].masked.sum())}")
    return state


def test_full_1p7b_step_properties():
    _full_size("1.7b", seed=21)


def test_full_8b_step_properties():
    from alodlm_amd import _lib
    # one 2048-token sequence: 32 key tiles per key-value head, so the dK/dV
    # pass is split by query head
    assert _lib.query("alodlm_attention_bwd_workspace", 4096, 32, 8, 128, 32, 0) > 2 * 4096 * 32
    _full_size("8b", seed=22)


def _sample_cosines(named, g, prefix=""):
    """Cosine of each gradient's strided sample (tests/golden.sample_indices,
    4096 elements) against the golden's ``prefix + gsample_`` vectors, by
    golden parameter name."""
    from tests.golden import sample_indices
    out = {}
    for name in g["param_names"]:
        grad = named[name].double().flatten()
        mine = grad[torch.as_tensor(sample_indices(grad.numel(), 4096))]
        out[str(name)] = cosine(mine, torch.as_tensor(g[prefix + "gsample_" + name]))
    return out


def test_1p7b_layer_shapes_match_reference_bf16_run():
    """The reference's own bf16 step at Qwen3-1.7B layer shapes
    (tests/golden/step_1p7b_layers_bf16.npz: hidden 2048, 16 / 8 heads of 128,
    SwiGLU 6144, vocabulary 151936, two layers as the recurrent core, one
    2048-token segment; the reference loaded in bf16 as its training loads
    it), and its float32 step on the same weights with the same exits.

    Masks are bit-exact (the reference's CPU draws replayed); the step takes
    the reference run's exits (uniforms replayed to them) so that both runs
    score the same rows.  Against the reference's bf16 run: every live
    masked cross-entropy within two bf16 steps; the denoising and
    autoregressive terms within 1e-3; halting probabilities within 5e-2
    (mean 5e-3).  The loss and the gradients are held to the step's parity
    bounds (loss 1e-2, gradient-sample cosine 0.999, norms 3 %) or, where the
    reference's own bf16 run misses them against its float32 run (the actor
    term: bf16 cross-entropies times sums of log q), to twice that gap:
    measured on the fixture, the reference's loss moves 1.3e-2 and its gate
    weight, gate bias and depth-bias gradients reach cosine 0.9987, 1 and
    0.9957 with the gate bias's norm at 0.48 of the float32 one."""
    from tests import golden
    from tests.helpers import cpu_draws
    g = golden.load("step_1p7b_layers_bf16")
    seed = int(g["seed"])
    dims = _dims(2048, 16, 8, 6144, layers=2)
    obj = O.Objective(loop_start=0, loop_end=2, mask_token_id=MASK_ID, block_size=32)
    K = obj.max_depth
    params = _bf16_params(dims, obj, seed=seed)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()}, dtype=torch.bfloat16)
    ids, labels = torch.as_tensor(g["in_ids"]), torch.as_tensor(g["in_labels"])
    bounds = torch.as_tensor(g["in_boundaries"])
    draws, _ = cpu_draws(labels, bounds, obj.block_size, seed, K)
    ref_exits = torch.as_tensor(g["exits"])
    log("1.7B layer shapes against the reference's bf16 and float32 runs")
    engine = model.engine()
    out, state = engine.forward(ids.cuda(), labels.cuda(), bounds, True, draws=draws,
                                exit_uniforms=[u.cuda() for u in _replay_uniforms(ref_exits, K)])
    grads = engine.backward(state, 1.0)
    torch.cuda.synchronize()
    out = out.cpu().double()
    b = state["batch"]
    for key in ("ids", "original", "positions", "masked", "mask_probability", "boundaries"):
        np.testing.assert_array_equal(getattr(b, key).cpu().numpy(), g[key], err_msg=key)
    assert torch.equal(state["exits"].cpu().long(), ref_exits.long())
    masked = b.masked.cpu()
    live = torch.arange(K)[:, None] < ref_exits[masked][None, :]
    hip_ce = state["ce"].cpu()[:, masked].double()[live]
    ref_ce = torch.as_tensor(g["ce"]).double()[live]
    ulp = torch.tensor([_bf16_ulp(v) for v in ref_ce.tolist()], dtype=torch.float64)
    ce_diff = (hip_ce - ref_ce).abs()
    assert bool((ce_diff <= 2 * ulp + 1e-3).all()), ce_diff.max()
    hz = lambda x: torch.sigmoid(torch.as_tensor(x).double())
    gap = (hz(state["gates"].cpu()) - hz(g["gates"])).abs()
    assert gap.mean().item() <= 5e-3 and gap.max().item() <= 5e-2, (gap.mean(), gap.max())
    for i, key in ((1, "denoising"), (8, "ar_loss")):
        ref = float(g["metric_" + key])
        assert abs(out[i] - ref) <= 1e-3 * abs(ref), (key, out[i], ref)
    rel = lambda a, r: abs(a - r) / abs(r)
    loss_b, loss_f = float(g["loss"]), float(g["f32_loss"])
    ref_gap = rel(loss_b, loss_f)
    log(f"loss: hip {out[0]:.4f}, reference bf16 {loss_b:.4f}, reference fp32 {loss_f:.4f}; "
        f"rel-err hip vs bf16 {rel(out[0], loss_b):.2e}, hip vs fp32 {rel(out[0], loss_f):.2e}, "
        f"reference bf16 vs fp32 {ref_gap:.2e}; CE |diff| mean {ce_diff.mean().item():.4f}; "
        f"halting |diff| mean {gap.mean().item():.2e} max {gap.max().item():.2e}")
    assert rel(out[0], loss_b) <= max(1e-2, 2 * ref_gap)
    assert rel(out[0], loss_f) <= max(1e-2, 2 * ref_gap)
    named = {n: engine.arena.view(grads, n).cpu() for n in engine.arena.names}
    hip_cos, hip_f32_cos = _sample_cosines(named, g), _sample_cosines(named, g, prefix="f32_")
    worst = []
    for name in g["param_names"]:
        name = str(name)
        ref_cos = cosine(torch.as_tensor(g["gsample_" + name]),
                         torch.as_tensor(g["f32_gsample_" + name]))
        floor = min(0.999, 1 - 2 * (1 - ref_cos))
        norm = named[name].double().norm().item()
        norm_b, norm_f = float(g["gnorm_" + name]), float(g["f32_gnorm_" + name])
        norm_tol = max(3e-2, 2 * rel(norm_b, norm_f))
        worst.append((hip_cos[name], name, ref_cos))
        assert hip_cos[name] >= floor, (name, hip_cos[name], ref_cos)
        assert hip_f32_cos[name] >= floor, (name, hip_f32_cos[name], ref_cos)
        assert rel(norm, norm_b) <= norm_tol, (name, norm, norm_b, norm_f)
    worst.sort()
    log("lowest gradient-sample cosines (hip vs reference bf16, reference bf16 vs fp32): " +
        ", ".join(f"{n} {c:.5f} ({r:.5f})" for c, n, r in worst[:4]))
