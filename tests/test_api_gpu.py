"""The reference's public functions through the product API, on the GPU.

* credit, outcome_loss and autoregressive_loss on the reference's known
  answers (tests/test_objective.py:22-86), values and gradients;
* build_batch's mask and sparse_plan on the reference's attention cases
  (tests/test_objective.py:88-105);
* rotary against the reference formula evaluated by torch (bf16: the same
  three roundings, bit for bit), layer_forward / training_layer against the
  oracle's decoder layer (float32, value and every gradient) with each mask
  form, the decoding window against the full-sequence layer, sparse_attention
  against masked softmax attention;
* ALoDLM.rollout + outcome_loss + autoregressive_loss, composed as
  alodlm/model.py:176-187 composes them, against the fused step: same loss and
  gradients;
* the reference's end-to-end check that one optimizer step moves both the
  gate and the denoiser (tests/test_objective.py:106-121).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from alodlm_amd.attention import plan_to_device, sparse_attention, sparse_plan
from alodlm_amd.batch import build_batch
from alodlm_amd.config import ModelConfig
from alodlm_amd.credit import masked_sequence_ids, sequence_score_function
from alodlm_amd.model import layer_forward, rotary, training_layer
from alodlm_amd.loss import autoregressive_loss, outcome_loss
from oracle import step as O
from tests import golden
from tests.helpers import cpu_draws, log, make_model
from tests.test_oracle import _analytic_outcome

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_sequence_credit_known_answer():
    """tests/test_objective.py:22-30: value (3 * -0.5 + 4 * -0.7) / 3,
    gradient [1, 1, 4/3] in log q and none in the credit."""
    log("sequence_score_function known answer")
    credit = torch.tensor([1., 2., 4.], device=DEV, requires_grad=True)
    logp = torch.tensor([-.2, -.3, -.7], device=DEV, requires_grad=True)
    result = sequence_score_function(credit, logp, torch.tensor([0, 0, 1], device=DEV), 2)
    grad = torch.autograd.grad(result, (credit, logp), allow_unused=True)
    assert grad[0] is None
    torch.testing.assert_close(grad[1].cpu(), torch.tensor([1., 1., 4 / 3]))
    torch.testing.assert_close(result.detach().cpu(), torch.tensor((3 * -.5 + 4 * -.7) / 3))


def test_masked_sequence_ids_against_bucketize():
    masked = torch.tensor([True, False, True, True, False, True, True], device=DEV)
    bounds = torch.tensor([0, 2, 5, 5, 7], device=DEV)
    rows = torch.arange(7, device=DEV)
    expect = torch.bucketize(rows, bounds[1:], right=True)[masked]
    assert torch.equal(masked_sequence_ids(masked, bounds), expect)
    assert torch.equal(masked_sequence_ids(masked, bounds.to(torch.int32)), expect)
    big = torch.rand(5000, device=DEV, generator=torch.Generator(DEV).manual_seed(0)) < 0.5
    bb = torch.tensor([0, 1000, 1001, 3333, 5000], device=DEV)
    assert torch.equal(masked_sequence_ids(big, bb),
                       torch.bucketize(torch.arange(5000, device=DEV), bb[1:], right=True)[big])


@pytest.mark.parametrize("K,depths", [(3, [1, 2, 3, 2]), (4, [4, 1, 3, 2])])
def test_outcome_loss_matches_analytic_gradient(K, depths):
    """tests/test_objective.py:32-74 (K = 3 verbatim, and a K = 4 variant):
    value and the gradients in every gate and in ce."""
    log(f"outcome_loss analytic K={K}")
    cfg = ModelConfig(max_depth=K, gate_init_pi=(1 / K,) * K)
    base = [[3., 4., 5., 6.], [2., 3., 3., 4.], [1., 2., 2., 3.], [1.5, .5, 2.5, 1.]]
    ce = torch.tensor(base[:K], device=DEV, requires_grad=True)
    gates = [torch.tensor([-.4, .2, -.3, .7], device=DEV, requires_grad=True) for _ in range(K)]
    mp = torch.tensor([.2, .4, .5, .8])
    batch = SimpleNamespace(masked=torch.ones(4, dtype=torch.bool, device=DEV),
                            mask_probability=mp.to(DEV), boundaries=torch.tensor([0, 2, 4], device=DEV))
    actual, metrics = outcome_loss(ce, gates, torch.tensor(depths, device=DEV), batch, cfg)
    assert set(metrics) == {"denoising", "actor", "sampled_mean_depth", "prediction_cost",
                            "regularization_cost", "profile_mean_depth",
                            "first_pass_halt_probability"}
    ce64 = torch.tensor(base[:K], dtype=torch.float64, requires_grad=True)
    g64 = [torch.tensor([-.4, .2, -.3, .7], dtype=torch.float64, requires_grad=True)
           for _ in range(K)]
    expected = _analytic_outcome(ce64, g64, torch.tensor(depths), mp.double(), cfg, [0, 2, 4])
    assert abs(actual.item() - expected.item()) <= 1e-5 * abs(expected.item())
    ag = torch.autograd.grad(actual, gates + [ce])
    eg = torch.autograd.grad(expected, g64 + [ce64], allow_unused=True)
    for a, e in zip(ag, eg):
        e = e if e is not None else torch.zeros_like(a.cpu(), dtype=torch.float64)
        torch.testing.assert_close(a.cpu().double(), e, rtol=1e-5, atol=1e-6)
    assert abs(metrics["sampled_mean_depth"].item() - np.mean(depths)) <= 1e-6


def test_outcome_loss_without_masked_rows_is_zero():
    cfg = ModelConfig(max_depth=3, gate_init_pi=(1 / 3,) * 3)
    ce = torch.zeros(3, 0, device=DEV, requires_grad=True)
    gates = [torch.randn(4, device=DEV, requires_grad=True) for _ in range(3)]
    batch = SimpleNamespace(masked=torch.zeros(4, dtype=torch.bool, device=DEV),
                            mask_probability=torch.zeros(4, device=DEV),
                            boundaries=torch.tensor([0, 4], device=DEV))
    out, metrics = outcome_loss(ce, gates, torch.full((4,), 3, device=DEV), batch, cfg)
    assert out.item() == 0.0 and all(v.item() == 0.0 for v in metrics.values())
    out.backward()
    assert all(float(g.grad.abs().sum()) == 0.0 for g in gates)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_autoregressive_loss_known_answer(dtype):
    """tests/test_objective.py:76-86: the loss equals the cross-entropy of the
    clean rows [1, 2, 8, 9, 10] against labels [2, 3, 5, 6, 7], gradient too."""
    log(f"autoregressive_loss {dtype}")
    torch.manual_seed(3)
    logits = torch.randn(16, 16)
    labels = torch.arange(8)
    labels[1] = -100
    ref_logits = logits.to(dtype).float().requires_grad_(True)
    expected = F.cross_entropy(ref_logits[[1, 2, 8, 9, 10]], labels[[2, 3, 5, 6, 7]])
    eg = torch.autograd.grad(expected, ref_logits)[0]
    x = logits.to(dtype).to(DEV).requires_grad_(True)
    actual = autoregressive_loss(x, labels.to(DEV), torch.tensor([0, 8, 16], device=DEV))
    ag = torch.autograd.grad(actual, x)[0]
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert abs(actual.item() - expected.item()) <= tol * abs(expected.item())
    torch.testing.assert_close(ag.float().cpu(), eg, rtol=tol, atol=tol * 0.1)
    # no target: 0 with requires_grad (loss.py:31-32)
    none = autoregressive_loss(x, torch.full((8,), -100, device=DEV),
                               torch.tensor([0, 8, 16], device=DEV))
    assert none.item() == 0.0 and none.requires_grad


def test_packed_attention_does_not_cross_sequences():
    """tests/test_objective.py:88-95 on the product's build_batch."""
    ids = torch.arange(8, device=DEV)
    batch = build_batch(ids, ids.clone(), torch.tensor([0, 4, 8]), 2, 3)
    assert not bool(batch.attention_mask[:8, 8:].any())
    assert not bool(batch.attention_mask[8:, :8].any())
    assert not bool(batch.attention_mask[4, 2])
    assert bool(batch.attention_mask[6, 0])
    assert not bool(batch.attention_mask[0, 4])


def test_sparse_ranges_match_dense_attention():
    """tests/test_objective.py:97-105 on the product's build_batch and sparse_plan."""
    ids = torch.arange(11, device=DEV)
    batch = build_batch(ids, ids.clone(), torch.tensor([0, 4, 11]), 3, 3)
    plan = sparse_plan(batch.boundaries.tolist(), 3, "magi")
    materialized = torch.zeros_like(batch.attention_mask)
    for (qa, qb), (ka, kb), causal in zip(plan["q_ranges"], plan["k_ranges"],
                                          plan["attn_type_map"]):
        allowed = torch.ones(qb - qa, kb - ka, dtype=torch.bool, device=DEV)
        materialized[qa:qb, ka:kb] |= allowed.tril() if causal else allowed
    assert torch.equal(materialized, batch.attention_mask)


def _rotate_half(x):
    first, second = x.chunk(2, -1)
    return torch.cat((-second, first), -1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotary_matches_reference_formula(dtype):
    """rotary (alodlm/model.py:41-46): q * cos + rotate(q) * sin evaluated by
    torch in the same dtype - bit for bit (three roundings in bf16) - and the
    gradients torch's autograd gives for that expression."""
    log(f"rotary {dtype}")
    g = torch.Generator().manual_seed(0)
    N, nq, nkv, dh = 37, 4, 2, 64
    q = torch.randn(N, nq, dh, generator=g).to(dtype).to(DEV)
    k = torch.randn(N, nkv, dh, generator=g).to(dtype).to(DEV)
    cos, sin = O.rope_tables(torch.randint(0, 500, (N,), generator=g), dh, 1e6, dtype)
    cos, sin = cos.to(DEV), sin.to(DEV)
    dq_out = torch.randn(N, nq, dh, generator=g).to(dtype).to(DEV)
    dk_out = torch.randn(N, nkv, dh, generator=g).to(dtype).to(DEV)
    qa, ka = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    rq, rk = qa * c + _rotate_half(qa) * s, ka * c + _rotate_half(ka) * s
    eq, ek = torch.autograd.grad((rq, rk), (qa, ka), (dq_out, dk_out))
    qb, kb = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    oq, ok = rotary(qb, kb, cos, sin)
    gq, gk = torch.autograd.grad((oq, ok), (qb, kb), (dq_out, dk_out))
    assert torch.equal(oq, rq.detach()) and torch.equal(ok, rk.detach())
    assert torch.equal(gq, eq) and torch.equal(gk, ek)


TINY = (O.Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768, vocab=1024,
               layers=4, eps=1e-6, theta=1e6),
        O.Objective(loop_start=1, loop_end=3, mask_token_id=3, block_size=32))


def _layer_case(seed=5):
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=seed)
    g = torch.Generator().manual_seed(seed)
    for name in params:
        if name.endswith("norm.weight"):
            params[name] = 1 + 0.1 * torch.randn(params[name].shape, generator=g)
    model = make_model(dims, obj, params)
    ids = torch.randint(0, dims.vocab, (104,), generator=g)
    bounds = torch.tensor([0, 40, 104])
    draws, _ = cpu_draws(ids, bounds, 8, seed, obj.max_depth)
    batch = build_batch(ids.to(DEV), ids.clone().to(DEV), bounds, 8, obj.mask_token_id,
                        draws=draws)
    base = model.backbone.model
    hidden = torch.randn(batch.ids.numel(), dims.hidden, generator=g)
    cos, sin = base.rotary_emb(hidden.to(DEV)[None], batch.positions[None])
    return dims, params, model, batch, hidden, cos[0], sin[0]


@pytest.mark.parametrize("form", ["batch", "plan", "training_layer"])
def test_layer_forward_matches_oracle(form):
    """layer_forward (alodlm/model.py:49-76) on layer 1 of a float32 model
    against the oracle's decoder layer under the dense dual-stream mask of a
    two-segment pack: output, current-token k/v, and the gradients of the
    output (times a fixed random cotangent) in the hidden states and all 11
    layer parameters."""
    log(f"layer_forward vs oracle ({form})")
    dims, params, model, batch, hidden, cos, sin = _layer_case()
    layer = model.backbone.model.layers[1]
    pre = "model.layers.1."
    mask = batch.attention_mask
    if form == "plan":
        mask = plan_to_device(sparse_plan(batch.boundaries.tolist(), 8, "magi"), DEV)
    x = hidden.to(DEV).requires_grad_(True)
    cot = torch.randn(hidden.shape, generator=torch.Generator().manual_seed(9))
    if form == "training_layer":
        out = training_layer(layer, x, cos, sin, mask)
    else:
        out, (k, v) = layer_forward(layer, x, cos, sin, mask)
    names = [n for n in O.param_names(dims) if n.startswith(pre)]
    mods = dict(layer.named_parameters())
    got = torch.autograd.grad(out, [x] + [mods[n[len(pre):]] for n in names], cot.to(DEV))
    p = {n: params[n].clone().requires_grad_(True) for n in names}
    xr = hidden.clone().requires_grad_(True)
    dense = torch.as_tensor(O.packed_attention_mask(batch.boundaries.tolist(), 8))
    ref = O.layer_forward(p, pre, xr, cos.cpu(), sin.cpu(), dense, dims)
    exp = torch.autograd.grad(ref, [xr] + [p[n] for n in names], cot)
    torch.testing.assert_close(out.detach().cpu(), ref.detach(), rtol=1e-5, atol=1e-5)
    for name, a, e in zip(["hidden"] + names, got, exp):
        torch.testing.assert_close(a.cpu(), e, rtol=1e-4, atol=1e-4 * e.abs().max().item(),
                                   msg=name)
    if form != "training_layer":
        # current-token keys and values through the transformers modules
        attn = layer.self_attn
        with torch.no_grad():
            h = layer.input_layernorm(x)
            kk = attn.k_norm(attn.k_proj(h).view(-1, dims.kv_heads, dims.head_dim))
            kk = kk * cos.unsqueeze(1) + _rotate_half(kk) * sin.unsqueeze(1)
            vv = attn.v_proj(h).view(-1, dims.kv_heads, dims.head_dim)
        torch.testing.assert_close(k, kk, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(v, vv, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype,prefix", [(torch.float32, 37), (torch.bfloat16, 150)])
def test_layer_forward_window_matches_full_sequence(dtype, prefix):
    """The decoding form of layer_forward (alodlm/inference.py:71-90): the last
    W rows with the first P rows' k/v as prefix and the window mask give the
    full causal sequence's last W outputs and k/v."""
    log(f"layer_forward window {dtype} P={prefix}")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=7)
    model = make_model(dims, obj, {k: v.float() for k, v in params.items()}, dtype=dtype)
    layer = model.backbone.model.layers[2]
    W = 16
    total = prefix + W
    g = torch.Generator().manual_seed(7)
    x = torch.randn(total, dims.hidden, generator=g).to(dtype).to(DEV)
    pos = torch.arange(total, device=DEV)
    cos, sin = model.backbone.model.rotary_emb(x[None], pos[None])
    cos, sin = cos[0], sin[0]
    causal = torch.ones(total, total, dtype=torch.bool, device=DEV).tril()
    with torch.no_grad():
        full, (kf, vf) = layer_forward(layer, x, cos, sin, causal)
        window = torch.cat((torch.ones(W, prefix, dtype=torch.bool, device=DEV),
                            torch.ones(W, W, dtype=torch.bool, device=DEV).tril()), 1)
        out, (kw, vw) = layer_forward(layer, x[prefix:], cos[prefix:], sin[prefix:], window,
                                      prefix=(kf[:prefix], vf[:prefix]))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out.float(), full[prefix:].float(), rtol=tol, atol=tol)
    assert torch.equal(kw, kf[prefix:]) and torch.equal(vw, vf[prefix:])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_attention_matches_masked_softmax(dtype):
    """sparse_attention (alodlm/attention.py:44-66) against softmax attention
    under the plan's dense mask (torch float32), values and gradients in q, k,
    v; grouped-query heads (4 query heads per key-value head)."""
    log(f"sparse_attention {dtype}")
    offsets, B = [0, 130, 200, 456], 32
    bounds = [2 * v for v in offsets]
    N, nq, nkv, dh = bounds[-1], 8, 2, 128
    g = torch.Generator().manual_seed(3)
    q = torch.randn(N, nq, dh, generator=g).to(dtype)
    k = torch.randn(N, nkv, dh, generator=g).to(dtype)
    v = torch.randn(N, nkv, dh, generator=g).to(dtype)
    do = torch.randn(N, nq, dh, generator=g).to(dtype)
    plan = plan_to_device(sparse_plan(bounds, B, "magi"), DEV)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = sparse_attention(qd, kd, vd, plan)
    got = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    qr, kr, vr = (t.float().requires_grad_(True) for t in (q, k, v))
    mask = torch.as_tensor(O.packed_attention_mask(bounds, B))
    ke, ve = kr.repeat_interleave(nq // nkv, 1), vr.repeat_interleave(nq // nkv, 1)
    s = torch.einsum("qhd,khd->hqk", qr, ke) * dh ** -0.5
    ref = torch.einsum("hqk,khd->qhd", s.masked_fill(~mask, float("-inf")).softmax(-1), ve)
    exp = torch.autograd.grad(ref, (qr, kr, vr), do.float())
    tol = 2e-5 if dtype == torch.float32 else 3e-2
    torch.testing.assert_close(out.float().cpu(), ref.detach(), rtol=tol, atol=tol)
    for a, e in zip(got, exp):
        torch.testing.assert_close(a.float().cpu(), e, rtol=tol, atol=tol * e.abs().max().item())
    with pytest.raises(ValueError):
        sparse_attention(q, k, v, plan)  # CPU tensors


def test_rollout_composition_matches_fused_step():
    """alodlm/model.py:176-187 composed from the product's public pieces -
    rollout, per-depth cross-entropy of the masked rows, outcome_loss and the
    mean autoregressive_loss - equals the fused step's loss and every
    parameter gradient (float32 tiny configuration, same draws)."""
    log("rollout composition vs fused step")
    dims, obj = TINY
    params = O.init_params(dims, obj.gate_init_pi, seed=4)
    model = make_model(dims, obj, params)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, dims.vocab, (512,), generator=g)
    labels = ids.clone()
    labels[:40] = -100
    bounds = torch.tensor([0, 128, 256, 384, 512])
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, 4, obj.max_depth)
    u = [t.to(DEV) for t in uniforms]
    batch = build_batch(ids.to(DEV), labels.to(DEV), bounds, obj.block_size, obj.mask_token_id,
                        draws=draws)
    logits, gates, exits = model.rollout(batch, exit_uniforms=u)
    masked = batch.masked
    ce = torch.stack([F.cross_entropy(lg[masked], batch.original[masked], reduction="none")
                      for lg in logits])
    den_actor, metrics = outcome_loss(ce, gates, exits, batch, model.config)
    ar = torch.stack([autoregressive_loss(lg, labels.to(DEV), batch.boundaries)
                      for lg in logits]).mean()
    total = (den_actor + ar) / 2 + 0.0 * sum(t.sum() for t in logits + gates)
    total.backward()
    composed = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
    model.zero_grad(set_to_none=True)
    loss, fused_metrics = model(ids.to(DEV), labels.to(DEV), bounds, exit_uniforms=u, draws=draws)
    loss.backward()
    assert abs(total.item() - loss.item()) <= 1e-5 * abs(loss.item())
    for key, value in metrics.items():
        assert abs(value.item() - fused_metrics[key].item()) <= 1e-5 * max(1.0, abs(value.item()))
    for name, p in model.named_parameters():
        ref = p.grad.detach()
        scale = ref.abs().max().item() + 1e-12
        assert (composed[name] - ref).abs().max().item() <= 1e-4 * scale, name


def test_real_model_updates_both_gate_and_denoiser():
    """tests/test_objective.py:106-121 on the micro model: finite loss and
    gradients, and one AdamW step moves the gate and the word embedding."""
    log("micro model: gate and denoiser updated")
    g = golden.load("step_micro")
    dims = O.Dims(hidden=32, heads=4, kv_heads=2, head_dim=8, intermediate=64, vocab=64,
                  layers=3, eps=1e-6, theta=1e4)
    obj = O.Objective(loop_start=1, loop_end=2, mask_token_id=3, block_size=4)
    name = lambda n: n if n.startswith("exit_gate.") else "backbone." + n
    params = {n: torch.as_tensor(g["param_" + name(n)]) for n in O.param_names(dims)}
    model = make_model(dims, obj, params)
    ids = torch.tensor([4, 7, 9, 2, 5, 9, 12, 2])
    labels = ids.clone()
    labels[:4] = -100
    gate_before = model.exit_gate.net.weight.detach().clone()
    word_before = model.backbone.model.embed_tokens.weight.detach().clone()
    optimizer = torch.optim.AdamW(model.parameters(), lr=1e-3)
    # the reference test's randomness: torch.manual_seed(5), drawn on the CPU
    bounds = torch.tensor([0, 8])
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, 5, obj.max_depth)
    loss, metrics = model(ids.to(DEV), labels.to(DEV), bounds, draws=draws,
                          exit_uniforms=[u.to(DEV) for u in uniforms])
    assert int(np.sum(draws[1])) > 0
    loss.backward()
    assert bool(torch.isfinite(loss))
    assert all(bool(torch.isfinite(p.grad).all()) for p in model.parameters() if p.grad is not None)
    optimizer.step()
    assert not torch.equal(model.exit_gate.net.weight, gate_before)
    assert not torch.equal(model.backbone.model.embed_tokens.weight, word_before)
    assert "sampled_mean_depth" in metrics
