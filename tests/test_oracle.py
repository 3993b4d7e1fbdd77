"""Pin the CPU oracle against the reference's golden vectors and known answers.

Golden vectors come from tests/golden/make_golden.py (the reference run on the
CPU).  Known answers restate the reference's own tests
(tests/test_objective.py, tests/test_gate.py of the reference) as data.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import step as O
from tests import golden


torch.set_num_threads(min(8, torch.get_num_threads()))


def _batch_arrays_equal(mine, gold):
    for key in ("ids", "original", "positions", "masked", "boundaries"):
        np.testing.assert_array_equal(mine[key], gold[key], err_msg=key)
    np.testing.assert_array_equal(mine["mask_probability"], gold["mask_probability"])


@pytest.mark.parametrize("case", ["batch_ragged", "batch_block32", "batch_allmasked_labels"])
def test_build_batch_matches_reference_golden(case):
    g = golden.load(case)
    labels = torch.as_tensor(g["in_labels"])
    torch.manual_seed(int(g["seed"]))
    draws = O.draw_mask_randomness(labels, g["in_boundaries"], int(g["block_size"]))
    mine = O.build_batch(g["in_ids"], g["in_labels"], g["in_boundaries"], int(g["block_size"]),
                         int(g["mask_token_id"]), draws)
    _batch_arrays_equal(mine, g)
    mask = O.packed_attention_mask(mine["boundaries"], int(g["block_size"]))
    np.testing.assert_array_equal(mask, g["attention_mask"])


def test_batch_invariants():
    """Counts are round(n*p); observed rows precede masked rows inside a block;
    positions are a per-block permutation (alodlm/batch.py:43-60)."""
    g = golden.load("batch_block32")
    torch.manual_seed(3)
    labels = torch.as_tensor(g["in_labels"])
    draws = O.draw_mask_randomness(labels, g["in_boundaries"], 32)
    b = O.build_batch(g["in_ids"], g["in_labels"], g["in_boundaries"], 32, 3, draws)
    offsets = list(g["in_boundaries"])
    for s, (a, e) in enumerate(zip(offsets, offsets[1:])):
        L = e - a
        noisy = slice(2 * a + L, 2 * a + 2 * L)
        pos, masked = b["positions"][noisy], b["masked"][noisy]
        for blk, left in enumerate(range(0, L, 32)):
            right = min(left + 32, L)
            bp, bm = pos[left:right], masked[left:right]
            assert sorted(bp) == list(range(left, right))
            n = int((g["in_labels"][a + left:a + right] != -100).sum())
            assert bm.sum() == round(n * float(draws[0][s][blk]))
            assert not (bm[:-1] & ~bm[1:]).any(), "masked rows must follow observed rows"
            assert (np.diff(bp[~bm]) > 0).all() and (np.diff(bp[bm]) > 0).all()


def test_mask_known_answers_and_density():
    """Reference test_objective.py:88-95 plus the closed-form allowed-pair count."""
    torch.manual_seed(0)
    ids = torch.arange(8)
    draws = O.draw_mask_randomness(ids, [0, 4, 8], 2)
    b = O.build_batch(ids, ids.clone(), [0, 4, 8], 2, 3, draws)
    m = O.packed_attention_mask(b["boundaries"], 2)
    assert not m[:8, 8:].any() and not m[8:, :8].any()
    assert not m[4, 2] and m[6, 0] and not m[0, 4]
    # L=2048, B=32: clean L(L+1)/2 pairs + noisy 64 blocks x (528 causal + clean prefix)
    L, B = 2048, 32
    per = O.attention_mask(128, 32).sum()
    clean = 128 * 129 // 2
    noisy = sum(32 * 33 // 2 + 32 * (32 * b) for b in range(4))
    assert per == clean + noisy
    nb = L // B
    total = L * (L + 1) // 2 + sum(B * (B + 1) // 2 + B * B * b for b in range(nb))
    assert total == 4196352


def test_sparse_plan_materializes_dense_mask():
    """Reference test_objective.py:97-105."""
    torch.manual_seed(1)
    ids = torch.arange(11)
    draws = O.draw_mask_randomness(ids, [0, 4, 11], 3)
    b = O.build_batch(ids, ids.clone(), [0, 4, 11], 3, 3, draws)
    qr, kr, causal = O.sparse_plan(b["boundaries"], 3)
    mat = np.zeros((22, 22), dtype=bool)
    for (qa, qb), (ka, kb), c in zip(qr, kr, causal):
        allowed = np.ones((qb - qa, kb - ka), dtype=bool)
        mat[qa:qb, ka:kb] |= np.tril(allowed) if c else allowed
    np.testing.assert_array_equal(mat, O.packed_attention_mask(b["boundaries"], 3))


def test_sequence_credit_known_answer():
    """Reference test_objective.py:22-30: d/dlogp = [1, 1, 4/3]; value -1.4333."""
    credit = torch.tensor([1., 2., 4.], requires_grad=True)
    logp = torch.tensor([-.2, -.3, -.7], requires_grad=True)
    out = O.sequence_score_function(credit, logp, torch.tensor([0, 0, 1]), 2)
    g = torch.autograd.grad(out, (credit, logp), allow_unused=True)
    assert g[0] is None or torch.all(g[0] == 0)
    torch.testing.assert_close(g[1], torch.tensor([1., 1., 4 / 3]))
    torch.testing.assert_close(out, torch.tensor((3 * -0.5 + 4 * -0.7) / 3))
    with pytest.raises(ValueError):
        O.masked_sequence_ids(torch.tensor([True, False]), torch.tensor([0, 1]))


def _analytic_outcome(ce, gates, depths, mask_probability, cfg, seg_bounds):
    """Per-token restatement with products of hazards (reference test_objective.py:42-69)."""
    K = cfg.max_depth
    probs = torch.stack(gates).sigmoid()
    n = ce.shape[1]
    w = 1 / (mask_probability + 1e-8)
    w = w / w.sum()
    lm = ce.new_zeros(())
    logq, full = [], []
    for i in range(n):
        z = int(depths[i])
        surv = ce.new_tensor(1.)
        masses = []
        for d in range(K):
            masses.append(surv if d == K - 1 else surv * probs[d, i])
            surv = surv * (1 - probs[d, i])
        full.append(torch.stack(masses))
        logq.append(sum(F.logsigmoid(-gates[d][i]) for d in range(z - 1))
                    + (F.logsigmoid(gates[z - 1][i]) if z < K else 0))
        surv = ce.new_tensor(1.)
        for d in range(z):
            mass = surv if d == z - 1 else surv * probs[d, i]
            lm = lm + w[i] * mass.detach() * ce[d, i]
            surv = surv * (1 - probs[d, i])
    logq = torch.stack(logq)
    qbar = torch.stack(full, 1).mean(1).detach()
    prior = torch.softmax(-cfg.depth_prior_c * torch.arange(1, K + 1).to(ce.dtype), 0)
    sampled = ce[depths - 1, torch.arange(n)]
    cost = ((sampled - ce[0]).detach() + cfg.kl_beta_mi * (logq.detach() - qbar[depths - 1].log())
            + cfg.kl_beta_marg * (qbar[depths - 1].log() - prior[depths - 1].log()))
    actor = sum(cost[a:b].sum() * logq[a:b].sum() for a, b in zip(seg_bounds, seg_bounds[1:])) / n
    return lm + actor


@pytest.mark.parametrize("K,depths", [(3, [1, 2, 3, 2]), (4, [4, 1, 3, 2])])
def test_outcome_loss_matches_analytic_restatement(K, depths):
    """Reference test_objective.py:32-74 (K=3 case verbatim in data) and a K=4 variant."""
    cfg = O.Objective(max_depth=K, gate_init_pi=(1 / K,) * K)
    base = [[3., 4., 5., 6.], [2., 3., 3., 4.], [1., 2., 2., 3.], [1.5, .5, 2.5, 1.]]
    ce = torch.tensor(base[:K], requires_grad=True)
    gates = [torch.tensor([-.4, .2, -.3, .7], requires_grad=True) for _ in range(K)]
    depths = torch.tensor(depths)
    masked = torch.ones(4, dtype=torch.bool)
    mp = torch.tensor([.2, .4, .5, .8])
    actual, _ = O.outcome_loss(ce, gates, depths, masked, mp, torch.tensor([0, 2, 4]), cfg)
    expected = _analytic_outcome(ce, gates, depths, mp, cfg, [0, 2, 4])
    torch.testing.assert_close(actual, expected)
    ag = torch.autograd.grad(actual, gates + [ce], retain_graph=True)
    eg = torch.autograd.grad(expected, gates + [ce], allow_unused=True)
    for a, e in zip(ag, eg):
        torch.testing.assert_close(a, e if e is not None else torch.zeros_like(a))


def test_outcome_loss_credit_costs_from_outside_enter_only_the_credit():
    """credit_ce equal to ce changes nothing; another credit_ce changes the
    actor through the credit's prediction cost only: the denoising term and
    every gradient with respect to ce stay the same (the credit carries no
    gradient, alodlm/loss.py:72-78)."""
    K = 3
    cfg = O.Objective(max_depth=K, gate_init_pi=(1 / K,) * K)
    ce = torch.tensor([[3., 4., 5., 6.], [2., 3., 3., 4.], [1., 2., 2., 3.]], requires_grad=True)
    gates = [torch.tensor([-.4, .2, -.3, .7], requires_grad=True) for _ in range(K)]
    args = (torch.tensor([1, 3, 2, 3]), torch.ones(4, dtype=torch.bool),
            torch.tensor([.2, .4, .5, .8]), torch.tensor([0, 2, 4]), cfg)
    base, m0 = O.outcome_loss(ce, gates, *args)
    same, m1 = O.outcome_loss(ce, gates, *args, credit_ce=ce.detach().clone())
    torch.testing.assert_close(base, same)
    other, m2 = O.outcome_loss(ce, gates, *args, credit_ce=ce.detach() + torch.tensor(
        [[0.], [0.5], [1.0]]))
    assert float(m2["denoising"]) == float(m0["denoising"])
    assert float(m2["actor"]) != float(m0["actor"])
    g0 = torch.autograd.grad(base, ce, retain_graph=True)[0]
    g2 = torch.autograd.grad(other, ce)[0]
    torch.testing.assert_close(g0, g2)


def test_outcome_loss_no_masked_rows_is_zero():
    cfg = O.Objective(max_depth=3, gate_init_pi=(1 / 3,) * 3)
    ce = torch.zeros(3, 0, requires_grad=True)
    gates = [torch.randn(4, requires_grad=True) for _ in range(3)]
    out, metrics = O.outcome_loss(ce, gates, torch.full((4,), 3), torch.zeros(4, dtype=torch.bool),
                                  torch.zeros(4), torch.tensor([0, 4]), cfg)
    assert float(out) == 0.0 and all(float(v) == 0.0 for v in metrics.values())


def test_autoregressive_known_answer():
    """Reference test_objective.py:76-86."""
    torch.manual_seed(3)
    logits = torch.randn(16, 16, requires_grad=True)
    labels = torch.arange(8)
    labels[1] = -100
    actual = O.autoregressive_loss(logits, labels, torch.tensor([0, 8, 16]))
    expected = F.cross_entropy(logits[[1, 2, 8, 9, 10]], labels[[2, 3, 5, 6, 7]])
    torch.testing.assert_close(actual, expected)
    torch.testing.assert_close(torch.autograd.grad(actual, logits, retain_graph=True)[0],
                               torch.autograd.grad(expected, logits)[0])


def test_gate_init_uniform_masses():
    """Reference test_gate.py:18-30: exit masses exactly 1/4 with a fresh gate."""
    bias = torch.tensor(O.gate_depth_bias((0.25,) * 4))
    torch.testing.assert_close(bias[:3], torch.log(torch.tensor([1 / 3, 1 / 2, 1.0])))
    surv, masses = torch.ones(()), []
    for d in range(3):
        h = torch.sigmoid(bias[d])
        masses.append(surv * h)
        surv = surv * (1 - h)
    masses.append(surv)
    torch.testing.assert_close(torch.stack(masses), torch.full((4,), 0.25))


def test_attention_matches_torch_sdpa():
    """The per-head masked softmax equals torch SDPA with repeat_interleave GQA."""
    g = torch.Generator().manual_seed(4)
    dims = O.Dims(hidden=32, heads=4, kv_heads=2, head_dim=8, intermediate=48, vocab=40, layers=1)
    p = O.init_params(dims, (0.25,) * 4, seed=4, std=0.2)
    for name in p:
        if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
            p[name] = 1 + 0.1 * torch.randn(p[name].shape, generator=g)
    n = 24
    x = torch.randn(n, 32, generator=g)
    pos = torch.randint(0, 12, (n,), generator=g)
    cos, sin = O.rope_tables(pos, 8, 1e6)
    allowed = torch.as_tensor(O.packed_attention_mask([0, 10, 24], 3))
    out = O.layer_forward(p, "model.layers.0.", x, cos, sin, allowed, dims)
    pre = "model.layers.0."
    h = O.rmsnorm(x, p[pre + "input_layernorm.weight"], 1e-6)
    q = O.rmsnorm((h @ p[pre + "self_attn.q_proj.weight"].T).view(n, 4, 8), p[pre + "self_attn.q_norm.weight"], 1e-6)
    k = O.rmsnorm((h @ p[pre + "self_attn.k_proj.weight"].T).view(n, 2, 8), p[pre + "self_attn.k_norm.weight"], 1e-6)
    v = (h @ p[pre + "self_attn.v_proj.weight"].T).view(n, 2, 8)
    rot = lambda t: torch.cat((-t[..., 4:], t[..., :4]), -1)
    q = q * cos[:, None] + rot(q) * sin[:, None]
    k = k * cos[:, None] + rot(k) * sin[:, None]
    k, v = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    att = F.scaled_dot_product_attention(q.transpose(0, 1)[None], k.transpose(0, 1)[None],
                                         v.transpose(0, 1)[None], attn_mask=allowed,
                                         scale=8 ** -0.5)[0].transpose(0, 1).reshape(n, 32)
    y = x + att @ p[pre + "self_attn.o_proj.weight"].T
    h2 = O.rmsnorm(y, p[pre + "post_attention_layernorm.weight"], 1e-6)
    y = y + (F.silu(h2 @ p[pre + "mlp.gate_proj.weight"].T) * (h2 @ p[pre + "mlp.up_proj.weight"].T)) @ p[pre + "mlp.down_proj.weight"].T
    torch.testing.assert_close(out, y, rtol=1e-5, atol=1e-5)


def test_rope_is_rotation():
    """RoPE preserves norms and pairs (i, i+d/2) by the angle pos*theta^(-2i/d)."""
    pos = torch.arange(5)
    cos, sin = O.rope_tables(pos, 8, 1e4, torch.float64)
    assert torch.allclose(cos ** 2 + sin ** 2, torch.ones_like(cos))
    torch.testing.assert_close(cos[3, 1], torch.tensor(np.cos(3 * 1e4 ** (-2 / 8)), dtype=torch.float64))


def _oracle_step(g, dims, cfg, params, ce_dtype=None):
    labels = torch.as_tensor(g["in_labels"])
    torch.manual_seed(int(g["seed"]))
    draws = O.draw_mask_randomness(labels, g["in_boundaries"], cfg.block_size)
    n = 2 * len(labels)
    uniforms = [torch.rand(n) for _ in range(cfg.max_depth - 1)]
    p = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    loss, metrics, extra = O.step_loss(p, g["in_ids"], labels, g["in_boundaries"], dims, cfg,
                                       draws, uniforms, ce_dtype=ce_dtype)
    loss.backward()
    return p, loss, metrics, extra


MICRO = (O.Dims(hidden=32, heads=4, kv_heads=2, head_dim=8, intermediate=64, vocab=64, layers=3,
                eps=1e-6, theta=1e4),
         O.Objective(loop_start=1, loop_end=2, mask_token_id=3, block_size=4))
TINY = (O.Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768, vocab=1024,
               layers=4, eps=1e-6, theta=1e6),
        O.Objective(loop_start=1, loop_end=3, mask_token_id=3, block_size=32))


def _golden_name(name):
    return name if name.startswith("exit_gate.") else "backbone." + name


@pytest.mark.parametrize("case", ["step_micro", "step_micro_ragged"])
def test_full_step_matches_reference_micro(case):
    g = golden.load(case)
    dims, cfg = MICRO
    params = {n: torch.as_tensor(g["param_" + _golden_name(n)]) for n in O.param_names(dims)}
    p, loss, metrics, extra = _oracle_step(g, dims, cfg, params)
    _batch_arrays_equal(extra["batch"], g)
    np.testing.assert_array_equal(extra["exits"].numpy(), g["exits"])
    torch.testing.assert_close(torch.stack(extra["gates"]).detach(), torch.as_tensor(g["gates"]),
                               rtol=1e-5, atol=1e-6)
    assert abs(float(loss) - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    for key, value in metrics.items():
        assert abs(float(value) - float(g["metric_" + key])) <= 1e-5 * max(1.0, abs(float(value))), key
    for name in O.param_names(dims):
        torch.testing.assert_close(p[name].grad, torch.as_tensor(g["grad_" + _golden_name(name)]),
                                   rtol=1e-4, atol=1e-6, msg=name)


def test_full_step_matches_reference_tiny():
    g = golden.load("step_tiny")
    dims, cfg = TINY
    params = O.init_params(dims, cfg.gate_init_pi, seed=0)
    p, loss, metrics, extra = _oracle_step(g, dims, cfg, params)
    _batch_arrays_equal(extra["batch"], g)
    np.testing.assert_array_equal(extra["exits"].numpy(), g["exits"])
    assert abs(float(loss) - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    for key, value in metrics.items():
        assert abs(float(value) - float(g["metric_" + key])) <= 1e-5 * max(1.0, abs(float(value))), key
    names = list(g["param_names"])
    for index, gname in enumerate(names):
        name = gname[len("backbone."):] if gname.startswith("backbone.") else gname
        grad = p[name].grad.double().flatten()
        ref_norm = float(g["gnorm_" + gname])
        assert abs(grad.norm().item() - ref_norm) <= 1e-4 * ref_norm + 1e-9, gname
        proj = (grad * golden.projection_vector(index, grad.numel())).sum().item()
        assert abs(proj - float(g["gproj_" + gname])) <= 1e-4 * ref_norm * grad.numel() ** 0.5 + 1e-9, gname
        sample = grad[torch.as_tensor(golden.sample_indices(grad.numel()))]
        torch.testing.assert_close(sample, torch.as_tensor(g["gsample_" + gname]),
                                   rtol=1e-4, atol=1e-4 * ref_norm / max(1, grad.numel()) ** 0.5 + 1e-10)


def test_bf16_oracle_matches_reference_bf16_run():
    """The bf16 model of the oracle (bf16 weights, float64 arithmetic, LM-head
    logits and per-token CE rounded to bf16 where the reference's eager bf16
    run rounds them) against the reference's own bf16 run of the tiny step
    (step_tiny_bf16.npz).  Masks, exits and gate values are exact; the
    denoising and AR terms agree to 2e-3 and the loss to 2e-2 (measured:
    1.3e-2; the reference's layers run in bf16 and its per-token CE carries a
    bf16 ulp of 0.03 at CE ~ 7, which the actor term differences); gradient
    norms to 5 % and strided gradient samples at cosine >= 0.98.  A dropped
    term or a sign error moves these by far more."""
    g = golden.load("step_tiny_bf16")
    dims, cfg = TINY
    params = {k: v.to(torch.bfloat16).double()
              for k, v in O.init_params(dims, cfg.gate_init_pi, seed=0).items()}
    p, loss, metrics, extra = _oracle_step(g, dims, cfg, params, ce_dtype=torch.bfloat16)
    _batch_arrays_equal(extra["batch"], g)
    np.testing.assert_array_equal(extra["exits"].numpy(), g["exits"])
    gates = torch.stack([x.detach() for x in extra["gates"]])
    torch.testing.assert_close(gates, torch.as_tensor(g["gates"]).double(), rtol=0, atol=1e-6)
    assert abs(float(loss) - float(g["loss"])) <= 2e-2 * abs(float(g["loss"]))
    for key in ("denoising", "ar_loss"):
        ref = float(g["metric_" + key])
        assert abs(float(metrics[key]) - ref) <= 2e-3 * abs(ref), key
    for key in ("sampled_mean_depth", "profile_mean_depth", "first_pass_halt_probability",
                "regularization_cost"):
        ref = float(g["metric_" + key])
        assert abs(float(metrics[key]) - ref) <= 1e-6 * max(1.0, abs(ref)), key
    for gname in g["param_names"]:
        name = gname[len("backbone."):] if gname.startswith("backbone.") else str(gname)
        grad = p[name].grad.double().flatten()
        ref_norm = float(g["gnorm_" + gname])
        assert abs(grad.norm().item() - ref_norm) <= 0.05 * ref_norm + 1e-12, gname
        sample = grad[torch.as_tensor(golden.sample_indices(grad.numel()))]
        ref = torch.as_tensor(g["gsample_" + gname])
        cos = float((sample @ ref) / (sample.norm() * ref.norm() + 1e-300))
        assert cos >= 0.98, (gname, cos)


def test_clip_and_adamw_match_reference_micro():
    """One clipped AdamW step (alodlm/train.py:42-56,140-143) against the golden update."""
    g = golden.load("step_micro")
    dims, cfg = MICRO
    names = list(g["param_names"])
    grads = [torch.as_tensor(g["grad_" + n]).double() for n in names]
    total, coef = O.clip_coefficient(grads, 1.0)
    assert abs(total - float(g["grad_total_norm"])) <= 1e-5 * total
    for n, grad in zip(names, grads):
        param = torch.as_tensor(g["param_" + n]).double().clone()
        wd = 0.0 if any(s in n for s in ("bias", "LayerNorm.weight", "layer_norm.weight")) else 0.01
        O.adamw_update(param, grad * coef, torch.zeros_like(param), torch.zeros_like(param), 1,
                       float(g["lr"]), wd)
        torch.testing.assert_close(param.float(), torch.as_tensor(g["updated_" + n]),
                                   rtol=1e-5, atol=1e-7, msg=n)


def test_adamw_first_step_closed_form():
    """m_hat = g and v_hat = g^2 on step 1, so dp = -lr*g/(|g|+eps) - lr*wd*p."""
    p = torch.tensor([0.5, -1.0, 2.0], dtype=torch.float64)
    g = torch.tensor([0.1, -0.2, 0.0], dtype=torch.float64)
    out = O.adamw_update(p.clone(), g, torch.zeros(3, dtype=torch.float64),
                         torch.zeros(3, dtype=torch.float64), 1, 1e-3, 0.01)
    expected = p * (1 - 1e-3 * 0.01) - 1e-3 * g / (g.abs() + 1e-8)
    torch.testing.assert_close(out, expected)


def test_cosine_schedule_closed_form():
    assert O.cosine_lr_multiplier(0, 0, 1) == 1.0
    assert O.cosine_lr_multiplier(0, 3, 100) == 0.0
    assert O.cosine_lr_multiplier(2, 4, 100) == 0.5
    assert abs(O.cosine_lr_multiplier(52, 4, 100) - 0.5) < 1e-12
    assert O.cosine_lr_multiplier(100, 4, 100) == 0.0



def _micro_case():
    from tests import golden
    from tests.helpers import cpu_draws, oracle_draws
    g = golden.load("step_micro")
    dims = O.Dims(hidden=32, heads=4, kv_heads=2, head_dim=8, intermediate=64, vocab=64,
                  layers=3, eps=1e-6, theta=1e4)
    obj = O.Objective(loop_start=1, loop_end=2, mask_token_id=3, block_size=4)
    name = lambda n: n if n.startswith("exit_gate.") else "backbone." + n
    p = {n: torch.as_tensor(g["param_" + name(n)]).double() for n in O.param_names(dims)}
    labels = torch.as_tensor(g["in_labels"])
    bounds = torch.as_tensor(g["in_boundaries"])
    draws, uniforms = cpu_draws(labels, bounds, obj.block_size, int(g["seed"]), obj.max_depth)
    od = oracle_draws(draws, [int(v) for v in bounds], obj.block_size)
    batch = O.build_batch(g["in_ids"], labels, bounds, obj.block_size, obj.mask_token_id, od)
    return g, dims, obj, p, labels, bounds, od, uniforms, batch


def test_rollout_from_given_core_input_is_the_same_rollout():
    """The x0 entry of the oracle rollout (the core block alone) reproduces the
    golden-pinned rollout when given the first core input the rollout itself
    computed: same logits, gates, exits and traced core outputs."""
    g, dims, obj, p, labels, bounds, od, uniforms, batch = _micro_case()
    t1, t2 = {}, {}
    l1, g1, e1 = O.rollout(p, batch, dims, obj, uniforms, trace=t1)
    l2, g2, e2 = O.rollout(p, batch, dims, obj, uniforms, x0=t1["core_in"][0], trace=t2)
    assert torch.equal(e1, e2)
    for a, b in zip(l1 + g1 + t1["core_out"], l2 + g2 + t2["core_out"]):
        assert torch.equal(a, b)
    np.testing.assert_array_equal(e1.numpy(), g["exits"])


def test_readout_objective_from_traced_finals_is_the_step_loss():
    """readout_objective on the rollout's own final-norm inputs gives the
    golden-pinned step loss, metrics, gates and exits."""
    g, dims, obj, p, labels, bounds, od, uniforms, batch = _micro_case()
    q = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    total, metrics, extra = O.step_loss(q, g["in_ids"], labels, bounds, dims, obj, od, uniforms)
    trace = {}
    O.rollout(p, batch, dims, obj, uniforms, trace=trace)
    t2, m2, x2 = O.readout_objective(p, trace["final_in"], batch, dims, obj, uniforms,
                                     labels=labels)
    assert abs(float(t2) - float(total)) <= 1e-12 * abs(float(total))
    assert abs(float(t2) - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    assert torch.equal(x2["exits"], extra["exits"])
    for key in m2:
        assert abs(float(m2[key]) - float(metrics[key])) <= 1e-12 * max(1.0, abs(float(metrics[key])))
