"""The recurrent core block and the fused readout on their own, at their
benchmark shapes (bf16, head_dim 128, vocabulary 151936).

Parity against the float32 oracle on the same bf16 weights and inputs:

* core block: one Qwen3-8B layer (hidden 4096, 32/8 heads, intermediate
  12288) run 4 times with shared weights from N(0, 1) hidden states over one
  1024-token segment (2048 dual-stream rows), committed rows re-embedded from
  an N(0, 1) 151936 x 4096 table: every pass's output (cosine >= 0.999 and
  3e-2 relative norm error), halting probabilities, and - for fixed random
  cotangents of the outputs and gate logits - the gradients in x0, the layer
  weights, the carry norm, the table and the gate (cosine >= 0.999, the
  4-element depth bias at 0.99);
* readout: hidden 2048 x vocabulary 151936 over 2048 rows (two 1024-row
  sequences, masked with probability t ~ U(0, 1) per sequence), 4 passes:
  per-row cross-entropies within two bf16 steps, the loss within 1e-2 of
  the size of its terms (the credit's gradient-free prediction cost taking
  the kernel's cross-entropies), gradients in every pass's hidden states, the
  LM head, the final norm and the gate.

Properties at full size (core block: 4 x 2048 tokens, 16384 rows; readout:
8192 rows x 4 passes): exits equal the exit rule on the blocks' own gates and
uniforms, gate logits of sampled rows equal a CPU recompute from the blocks'
readout rows, the readout's loss equals the oracle objective recomputed from
its own cross-entropies (1e-4), sampled cross-entropies equal a CPU
recompute, and every output and gradient is finite.  The autograd wrappers
(recurrent_core, fused_readout) give the engine stages' gradients.
"""

import gc

import numpy as np
import pytest
import torch

from alodlm_amd.batch import build_batch
from alodlm_amd.core import fused_readout, readout_batch, recurrent_core
from oracle import step as O
from tests.helpers import cosine, log, make_model
from tests.test_shapes_gpu import (MASK_ID, VOCAB, _bf16_ulp, _check_exits, _check_sampled_ce,
                                   _dims, _objective_from_step, _replay_uniforms)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _stage_params(dims, obj, seed, table_std):
    """bf16 parameters: N(0, 0.02) layers, norm weights 1 + N(0, 0.05), a gate
    with N(0, 0.02) weights, and word embeddings N(0, table_std)."""
    params = O.init_params(dims, obj.gate_init_pi, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    for name, value in params.items():
        if name.endswith("norm.weight"):
            params[name] = 1 + 0.05 * torch.randn(value.shape, generator=g)
    params["exit_gate.net.weight"] = 0.02 * torch.randn(1, dims.hidden, generator=g)
    params["model.embed_tokens.weight"] *= table_std / 0.02
    return {k: v.to(torch.bfloat16) for k, v in params.items()}


def _oracle_batch(batch):
    return {"ids": batch.ids.cpu().numpy(), "original": batch.original.cpu().numpy(),
            "positions": batch.positions.cpu().numpy(), "masked": batch.masked.cpu().numpy(),
            "mask_probability": batch.mask_probability.cpu().numpy(),
            "boundaries": batch.boundaries.cpu().numpy()}


def _core_case(tokens, seed):
    dims = _dims(4096, 32, 8, 12288, layers=1)
    obj = O.Objective(loop_start=0, loop_end=1, mask_token_id=MASK_ID, block_size=32)
    params = _stage_params(dims, obj, seed, table_std=1.0)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()}, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, VOCAB, (sum(tokens),), generator=g)
    bounds = torch.tensor([0] + list(np.cumsum(tokens)))
    gen = torch.Generator(device=DEV).manual_seed(seed)
    batch = build_batch(ids.to(DEV), ids.clone().to(DEV), bounds, 32, MASK_ID, generator=gen)
    x0 = torch.randn(2 * sum(tokens), dims.hidden, generator=g).to(torch.bfloat16)
    return dims, obj, params, model, batch, x0, gen


def _run_core(model, batch, x0, gen, cot, gcot):
    engine = model.engine()
    start = gen.get_state()
    outs, gates, exits, state = engine.core_forward(x0.to(DEV), batch, True, generator=gen)
    dx0, grads = engine.core_backward(state, [c.to(DEV) for c in cot], gcot.to(DEV))
    torch.cuda.synchronize()
    gen.set_state(start)
    K = model.config.max_depth
    uniforms = [torch.rand(x0.shape[0], device=DEV, generator=gen) for _ in range(K - 1)]
    return outs, gates, exits, state, dx0, grads, uniforms


def test_core_block_matches_oracle():
    log("core block: Qwen3-8B layer x 4 passes, 2048 rows, against the oracle")
    dims, obj, params, model, batch, x0, gen = _core_case([1024], seed=31)
    K, N, H = obj.max_depth, x0.shape[0], dims.hidden
    g = torch.Generator().manual_seed(32)
    cot = [torch.randn(N, H, generator=g).to(torch.bfloat16) for _ in range(K)]
    gcot = torch.randn(K, N, generator=g)
    outs, gates, exits, state, dx0, grads, uniforms = _run_core(model, batch, x0, gen, cot, gcot)
    exits_host = _check_exits({"gates": gates, "exits": exits, "batch": batch}, uniforms, K)
    engine = model.engine()
    named = {n: engine.arena.view(grads, n).cpu() for n in engine.arena.names}
    got_outs = [o.float().cpu() for o in outs]
    got_gates, got_dx0 = gates.cpu(), dx0.float().cpu()
    del outs, state, grads, dx0
    gc.collect()
    torch.cuda.empty_cache()
    log("oracle (float32, CPU)")
    p = {k: v.float().requires_grad_(True) for k, v in params.items()}
    xr = x0.float().requires_grad_(True)
    trace = {}
    _, ref_gates, ref_exits = O.rollout(p, _oracle_batch(batch), dims, obj,
                                        _replay_uniforms(exits_host, K), x0=xr, trace=trace,
                                        lm_head=False)
    assert torch.equal(ref_exits, exits_host)
    loss = sum((o * c.float()).sum() for o, c in zip(trace["core_out"], cot))
    loss = loss + sum((gt * gcot[d]).sum() for d, gt in enumerate(ref_gates))
    loss.backward()
    # bf16 storage rounds the hidden states (2^-9 relative) at every layer
    # output and residual, and the error grows with the passes: cosine >= 0.999
    # corresponds to a relative norm error of up to about 4.5 %
    errs = []
    for d in range(K):
        ref = trace["core_out"][d].detach()
        rel = ((got_outs[d] - ref).norm() / ref.norm()).item()
        errs.append(round(rel, 5))
        assert cosine(got_outs[d], ref) >= 0.999 and rel <= 3e-2, (d, rel)
        gap = (torch.sigmoid(got_gates[d].double()) - torch.sigmoid(ref_gates[d].detach().double()))
        assert gap.abs().mean().item() <= 5e-3 and gap.abs().max().item() <= 5e-2, d
    c = cosine(got_dx0, xr.grad)
    assert c >= 0.999, f"x0: cosine {c}"
    worst = 1.0
    for name in O.param_names(dims):
        if name == "lm_head.weight":
            continue
        key = name if name.startswith("exit_gate.") else "backbone." + name
        c = cosine(named[key], p[name].grad)
        floor = 0.99 if name == "exit_gate.depth_bias" else 0.999
        assert c >= floor, f"{name}: cosine {c}"
        worst = min(worst, c) if name != "exit_gate.depth_bias" else worst
    log(f"core block: output relative error per pass {errs}; worst gradient cosine "
        f"{worst:.6f}; masked rows "
        f"{int(batch.masked.sum())}, exits {np.bincount(exits_host.numpy(), minlength=5)[1:]}")


def test_core_block_full_size_properties():
    log("core block full size: 4 x 2048 tokens (16384 rows)")
    dims, obj, params, model, batch, x0, gen = _core_case([2048] * 4, seed=33)
    K, N, H = obj.max_depth, x0.shape[0], dims.hidden
    g = torch.Generator().manual_seed(34)
    cot = [torch.randn(N, H, generator=g).to(torch.bfloat16) for _ in range(K)]
    gcot = torch.randn(K, N, generator=g)
    outs, gates, exits, state, dx0, grads, uniforms = _run_core(model, batch, x0, gen, cot, gcot)
    _check_exits({"gates": gates, "exits": exits, "batch": batch}, uniforms, K)
    gate = model.exit_gate
    w = gate.net.weight.detach().float().cpu()[0]
    bias, db = gate.net.bias.detach().float().cpu()[0], gate.depth_bias.detach().float().cpu()
    sel = torch.randperm(N, generator=g)[:256]
    for d, rec in enumerate(state["depths"]):
        x = rec["readout"][sel.to(DEV)].float().cpu()
        logit = ((x @ w + bias).to(torch.bfloat16).float() + db[d]).to(torch.bfloat16).float()
        for v, r in zip(gates[d].cpu()[sel].tolist(), logit.tolist()):
            assert abs(v - r) <= _bf16_ulp(r) + 1e-6
        assert bool(torch.isfinite(outs[d]).all())
    assert bool(torch.isfinite(dx0).all()) and bool(torch.isfinite(grads).all())
    engine = model.engine()
    for name in ("backbone.model.layers.0.self_attn.q_proj.weight",
                 "backbone.model.layers.0.mlp.down_proj.weight", "backbone.model.norm.weight",
                 "backbone.model.embed_tokens.weight", "exit_gate.net.weight"):
        assert engine.arena.view(grads, name).norm().item() > 0, name
    # the autograd wrapper gives the same input gradient bit for bit (every
    # kernel sums in a fixed order; the gate-logit cotangents, rounded to the
    # parameter dtype on this path, reach only the gate parameters)
    x = x0.to(DEV).requires_grad_(True)
    outs2, gates2, _ = recurrent_core(model, x, batch, exit_uniforms=uniforms)
    loss = sum((o.float() * c.to(DEV).float()).sum() for o, c in zip(outs2, cot))
    loss = loss + (gates2.float() * gcot.to(DEV)).sum()
    gx = torch.autograd.grad(loss, x)[0]
    assert torch.equal(gx, dx0)
    log(f"core block full size: masked rows {int(batch.masked.sum())}")


def _readout_case(rows_per_seq, nseq, seed):
    dims = _dims(2048, 16, 8, 6144, layers=1)
    obj = O.Objective(loop_start=0, loop_end=1, mask_token_id=MASK_ID, block_size=32)
    params = _stage_params(dims, obj, seed, table_std=0.02)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()}, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    N = rows_per_seq * nseq
    K = obj.max_depth
    finals = [torch.randn(N, dims.hidden, generator=g).to(torch.bfloat16) for _ in range(K)]
    targets = torch.randint(0, VOCAB, (N,), generator=g)
    t = torch.rand(nseq, generator=g).clamp_min(1e-8).repeat_interleave(rows_per_seq)
    masked = torch.rand(N, generator=g) < t
    prob = torch.where(masked, t, torch.zeros_like(t))
    bounds = torch.arange(nseq + 1) * rows_per_seq
    batch = readout_batch(targets.to(DEV), bounds.to(DEV), masked.to(DEV), prob.to(DEV))
    uniforms = [torch.rand(N, generator=g) for _ in range(K - 1)]
    host = {"masked": masked.numpy(), "original": targets.numpy(),
            "mask_probability": prob.numpy(), "boundaries": bounds.numpy()}
    return dims, obj, params, model, batch, finals, uniforms, host


def test_readout_matches_oracle():
    log("readout: 2048 x 2048 x 151936, 4 passes, against the oracle")
    dims, obj, params, model, batch, finals, uniforms, host = _readout_case(1024, 2, seed=41)
    K = obj.max_depth
    engine = model.engine()
    out, state = engine.readout_forward([f.to(DEV) for f in finals], batch, True,
                                        exit_uniforms=[u.to(DEV) for u in uniforms])
    dfinals, grads = engine.readout_backward(state, 1.0)
    torch.cuda.synchronize()
    out = out.cpu().double()
    masked = batch.masked.cpu()
    exits = _check_exits(state, [u.to(DEV) for u in uniforms], K)
    hip_ce = state["ce"].cpu()[:, masked].double()
    named = {n: engine.arena.view(grads, n).cpu() for n in engine.arena.names}
    got_df = [d.float().cpu() for d in dfinals]
    del state, grads, dfinals
    gc.collect()
    log("oracle (float32, CPU)")
    p = {k: v.float().requires_grad_(True) for k, v in params.items()}
    fr = [f.float().requires_grad_(True) for f in finals]
    loss, metrics, extra = O.readout_objective(p, fr, host, dims, obj, _replay_uniforms(exits, K),
                                               ce_dtype=torch.bfloat16, credit_ce=hip_ce)
    loss.backward()
    assert torch.equal(extra["exits"], exits)
    z = exits[masked]
    live = torch.arange(K)[:, None] < z[None, :]
    diff = (hip_ce - extra["ce"].detach().double()).abs()[live]
    ulp = torch.tensor([_bf16_ulp(v) for v in extra["ce"].detach()[live].tolist()],
                       dtype=torch.float64)
    assert bool((diff <= 2 * ulp + 1e-3).all()) and diff.mean().item() <= 0.03
    terms = (abs(metrics["denoising"].item()) + abs(metrics["actor"].item())) / 2
    assert abs(out[0] - loss.item()) <= 1e-2 * terms, (out[0], loss.item(), terms)
    assert abs(out[1] - metrics["denoising"].item()) <= 1e-2 * abs(metrics["denoising"].item())
    for d in range(K):
        c = cosine(got_df[d], fr[d].grad)
        assert c >= 0.999, f"d final_in[{d}]: cosine {c}"
    for name in ("lm_head.weight", "model.norm.weight", "exit_gate.net.weight",
                 "exit_gate.net.bias", "exit_gate.depth_bias"):
        key = name if name.startswith("exit_gate.") else "backbone." + name
        c = cosine(named[key], p[name].grad)
        floor = 0.99 if name == "exit_gate.depth_bias" else 0.999
        assert c >= floor, f"{name}: cosine {c}"
    log(f"readout: loss {out[0]:.5f} vs oracle {loss.item():.5f}; CE |diff| mean "
        f"{diff.mean().item():.4f}; masked rows {int(masked.sum())}")


def test_readout_full_size_properties():
    log("readout full size: 8192 x 2048 x 151936, 4 passes")
    dims, obj, params, model, batch, finals, uniforms, host = _readout_case(2048, 4, seed=43)
    K = obj.max_depth
    engine = model.engine()
    fd = [f.to(DEV) for f in finals]
    u = [x.to(DEV) for x in uniforms]
    out, state = engine.readout_forward(fd, batch, True, exit_uniforms=u)
    dfinals, grads = engine.readout_backward(state, 1.0)
    torch.cuda.synchronize()
    out = out.cpu().double()
    _check_exits(state, u, K)
    total, metrics = _objective_from_step(state, model.config)
    assert abs(out[0] - total) <= 1e-4 * abs(total) + 1e-6, (out[0], total)
    _check_sampled_ce(state, model.backbone.lm_head.weight, seed=43)
    assert all(bool(torch.isfinite(d).all()) for d in dfinals)
    assert bool(torch.isfinite(grads).all())
    assert engine.arena.view(grads, "backbone.lm_head.weight").norm().item() > 0
    # the autograd wrapper gives the same loss and hidden-state gradients
    xs = [f.clone().requires_grad_(True) for f in fd]
    loss, m = fused_readout(model, xs, batch, exit_uniforms=u)
    gx = torch.autograd.grad(loss, xs)
    assert loss.item() == float(out[0])
    for a, b in zip(gx, dfinals):
        assert torch.equal(a, b)
    log(f"readout full size: loss {out[0]:.5f}; masked rows {int(batch.masked.sum())}; "
        f"loss-bearing rows per pass {engine.last_rows}")
