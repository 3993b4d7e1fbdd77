"""CPU restatement of the ALoDLM training step (TEST INFRASTRUCTURE ONLY).

Not a runtime backend: nothing in the product package imports this module.
Tensors are float32 by default; pass ``dtype=torch.float64`` for a tighter
restatement.  Citations are into the reference (amazon-science/ALoDLM) and,
with the prefix ``[tf]``, into transformers' Qwen3 modules.
"""

from dataclasses import dataclass
import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "Dims", "Objective", "draw_mask_randomness", "build_batch", "attention_mask",
    "packed_attention_mask", "sparse_plan", "rope_tables", "rmsnorm", "layer_forward",
    "gate_depth_bias", "rollout", "readout_objective", "outcome_loss", "autoregressive_loss",
    "masked_sequence_ids", "sequence_score_function", "step_loss", "init_params",
    "param_names", "clip_coefficient", "adamw_update", "cosine_lr_multiplier",
]


@dataclass
class Dims:
    """Qwen3 backbone dimensions ([tf] configuration_qwen3.py:62-80)."""
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    layers: int
    eps: float = 1e-6
    theta: float = 1e6


@dataclass
class Objective:
    """The ModelConfig fields the step reads (alodlm/config.py:16-31)."""
    loop_start: int = 10
    loop_end: int = 26
    max_depth: int = 4
    depth_prior_c: float = 0.4
    kl_beta_mi: float = 0.1
    kl_beta_marg: float = 1.0
    gate_init_pi: tuple = (0.25, 0.25, 0.25, 0.25)
    mask_token_id: int = 151665
    block_size: int = 32


# ----------------------------------------------------------------------------
# Dual-stream batch (alodlm/batch.py)
# ----------------------------------------------------------------------------

def draw_mask_randomness(labels, boundaries, block_size, generator=None, device=None):
    """Consume the generator exactly as alodlm/batch.py:50-60 does.

    Per segment: one ``uniform_(0, 1)`` of ceil(L/B) floats clamped at 1e-8
    (batch.py:50-51); then, block by block, one ``randperm(n_candidates)`` for
    every block whose count round(n*p) is nonzero (batch.py:55-60).
    Returns (list of per-segment uniform tensors, list of per-block permutations
    or None) on ``device`` (default: the labels' device).
    """
    device = labels.device if device is None else device
    offsets = [int(v) for v in boundaries]
    lab = labels.detach().cpu().numpy()
    uniforms, perms = [], []
    for a, b in zip(offsets, offsets[1:]):
        length = b - a
        nblocks = (length + block_size - 1) // block_size
        u = torch.empty(nblocks, device=device).uniform_(0, 1, generator=generator).clamp_min(1e-8)
        uniforms.append(u)
        host = u.tolist()
        for blk in range(nblocks):
            left, right = blk * block_size, min(blk * block_size + block_size, length)
            n = int((lab[a + left:a + right] != -100).sum())
            count = round(n * host[blk])
            perms.append(torch.randperm(n, device=device, generator=generator) if count else None)
    return uniforms, perms


def build_batch(ids, labels, boundaries, block_size, mask_token_id, draws):
    """Integer restatement of alodlm/batch.py:34-85 in numpy, from explicit draws.

    Returns a dict of numpy arrays over the dual-stream rows: ids, original,
    positions (int64), masked (bool), mask_probability (float32), boundaries
    (int64, doubled offsets).
    """
    uniforms, perms = draws
    ids = np.asarray(torch.as_tensor(ids).cpu(), dtype=np.int64)
    labels = np.asarray(torch.as_tensor(labels).cpu(), dtype=np.int64)
    offsets = [int(v) for v in boundaries]
    if ids.ndim != 1 or ids.shape != labels.shape or ids.size == 0:
        raise ValueError("Expected nonempty flat input and label tensors")
    if offsets[0] != 0 or offsets[-1] != len(ids):
        raise ValueError("Boundaries must cover the packed tokens")
    if any(a >= b for a, b in zip(offsets, offsets[1:])):
        raise ValueError("Packed segments must be nonempty")
    out = {k: [] for k in ("ids", "original", "positions", "masked", "mask_probability")}
    new_offsets = [0]
    perm_iter = iter(perms)
    for s, (a, b) in enumerate(zip(offsets, offsets[1:])):
        seq, lab = ids[a:b], labels[a:b]
        length = b - a
        probs = np.asarray(torch.as_tensor(uniforms[s]).cpu(), dtype=np.float32)
        noisy, gold, pos, sel, prob = [], [], [], [], []
        for blk, left in enumerate(range(0, length, block_size)):
            right = min(left + block_size, length)
            cand = np.nonzero(lab[left:right] != -100)[0]
            p = float(probs[blk])
            count = round(len(cand) * p)
            perm = next(perm_iter)
            chosen = np.zeros(right - left, dtype=bool)
            if count:
                chosen[cand[np.asarray(perm.cpu())[:count]]] = True
            order = np.concatenate((np.nonzero(~chosen)[0], np.nonzero(chosen)[0]))
            tok = seq[left:right]
            noisy.append(np.where(chosen, mask_token_id, tok)[order])
            gold.append(tok[order])
            pos.append(np.arange(left, right)[order])
            sel.append(chosen[order])
            prob.append(np.where(chosen[order], np.float32(p), np.float32(0)).astype(np.float32))
        out["ids"].append(np.concatenate((seq, *noisy)))
        out["original"].append(np.concatenate((seq, *gold)))
        out["positions"].append(np.concatenate((np.arange(length), *pos)))
        out["masked"].append(np.concatenate((np.zeros(length, bool), *sel)))
        out["mask_probability"].append(np.concatenate((np.zeros(length, np.float32), *prob)))
        new_offsets.append(new_offsets[-1] + 2 * length)
    batch = {k: np.concatenate(v) for k, v in out.items()}
    batch["boundaries"] = np.asarray(new_offsets, dtype=np.int64)
    return batch


def attention_mask(length, block_size):
    """Closed-form dual-stream mask of one segment (alodlm/batch.py:23-31)."""
    q = np.arange(2 * length)[:, None]
    k = np.arange(2 * length)[None, :]
    q_noisy, k_noisy = q >= length, k >= length
    q_block = np.where(q_noisy, q - length, q) // block_size
    k_block = np.where(k_noisy, k - length, k) // block_size
    same = (q_block == k_block) & (q_noisy == k_noisy) & (k <= q)
    earlier_clean = (k_block < q_block) & ~k_noisy
    return same | earlier_clean


def packed_attention_mask(packed_boundaries, block_size):
    """Block-diagonal of the per-segment masks (alodlm/batch.py:64-65,83)."""
    offsets = [int(v) for v in packed_boundaries]
    n = offsets[-1]
    mask = np.zeros((n, n), dtype=bool)
    for a, b in zip(offsets, offsets[1:]):
        mask[a:b, a:b] = attention_mask((b - a) // 2, block_size)
    return mask


def sparse_plan(packed_boundaries, block_size):
    """Range-triple form of the same mask (alodlm/attention.py:12-30).

    Returns (q_ranges, k_ranges, causal) lists.
    """
    qr, kr, causal = [], [], []
    offsets = [int(v) for v in packed_boundaries]
    for start, end in zip(offsets, offsets[1:]):
        length = (end - start) // 2
        blocks = [(start + length + b, start + length + min(b + block_size, length))
                  for b in range(0, length, block_size)]
        for lo, hi in blocks:
            qr.append((lo, hi)); kr.append((lo, hi)); causal.append(1)
        for index, (lo, hi) in enumerate(blocks[1:], 1):
            qr.append((lo, hi)); kr.append((start, start + index * block_size)); causal.append(0)
        if length:
            qr.append((start, start + length)); kr.append((start, start + length)); causal.append(1)
    return qr, kr, causal


# ----------------------------------------------------------------------------
# Qwen3 layer arithmetic ([tf] modeling_qwen3.py) and alodlm/model.py
# ----------------------------------------------------------------------------

def rope_tables(positions, head_dim, theta, dtype=torch.float32):
    """cos/sin of [tf] modeling_qwen3.py:115-137 at the (permuted) positions."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.as_tensor(positions).float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rmsnorm(x, weight, eps):
    """[tf] modeling_qwen3.py:59-64 (upcast, normalize, cast back, then scale)."""
    x32 = x.to(torch.promote_types(x.dtype, torch.float32))
    y = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return weight * y.to(x.dtype)


def _rotate(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), -1)


def layer_forward(p, prefix, x, cos, sin, allowed, dims):
    """One pre-norm Qwen3 decoder layer (alodlm/model.py:49-76).

    ``p`` maps parameter names to tensors; ``prefix`` is e.g.
    ``"model.layers.3."``.  ``allowed`` is the bool [N, N] attention mask.
    """
    n = x.shape[0]
    nq, nkv, dh = dims.heads, dims.kv_heads, dims.head_dim
    h = rmsnorm(x, p[prefix + "input_layernorm.weight"], dims.eps)
    q = (h @ p[prefix + "self_attn.q_proj.weight"].T).view(n, nq, dh)
    k = (h @ p[prefix + "self_attn.k_proj.weight"].T).view(n, nkv, dh)
    v = (h @ p[prefix + "self_attn.v_proj.weight"].T).view(n, nkv, dh)
    q = rmsnorm(q, p[prefix + "self_attn.q_norm.weight"], dims.eps)
    k = rmsnorm(k, p[prefix + "self_attn.k_norm.weight"], dims.eps)
    c, s = cos[:, None, :], sin[:, None, :]
    q, k = q * c + _rotate(q) * s, k * c + _rotate(k) * s          # model.py:41-46
    rep = nq // nkv                                                  # model.py:65-67
    mask = torch.as_tensor(allowed)
    heads = []
    for head in range(nq):
        scores = (q[:, head] @ k[:, head // rep].T) * dh ** -0.5
        scores = scores.masked_fill(~mask, float("-inf"))
        heads.append(torch.softmax(scores, -1) @ v[:, head // rep])
    out = torch.stack(heads, 1).reshape(n, nq * dh)
    x = x + out @ p[prefix + "self_attn.o_proj.weight"].T               # model.py:74
    h2 = rmsnorm(x, p[prefix + "post_attention_layernorm.weight"], dims.eps)
    act = F.silu(h2 @ p[prefix + "mlp.gate_proj.weight"].T) * (h2 @ p[prefix + "mlp.up_proj.weight"].T)
    return x + act @ p[prefix + "mlp.down_proj.weight"].T              # model.py:75, [tf] :81-83


def gate_depth_bias(initial_mass):
    """Depth biases of a fresh gate (alodlm/model.py:25-35): logit of the
    conditional hazard mass/survival for every depth but the last, then 0."""
    bias, survival = [], 1.0
    for mass in initial_mass[:-1]:
        hazard = mass / survival
        bias.append(math.log(hazard / (1 - hazard)))
        survival *= 1 - hazard
    return bias + [0.0]


def _gate(p, readout, depth):
    """GateHead on the detached readout (alodlm/model.py:37-38,162)."""
    gate = (readout.detach() @ p["exit_gate.net.weight"].T).squeeze(-1) + p["exit_gate.net.bias"]
    return gate + p["exit_gate.depth_bias"][depth]


def _sample_exits(gate, uniforms, masked, exits, depth, K):
    """alodlm/model.py:163-167: rows still at K whose uniform falls under the
    hazard exit after pass depth + 1."""
    with torch.no_grad():
        hazard = torch.sigmoid(gate.float())
        chosen = (torch.as_tensor(uniforms) < hazard) & masked & (exits == K)
    return torch.where(chosen, depth + 1, exits)


def rollout(p, batch, dims, cfg, exit_uniforms, allowed=None, x0=None, trace=None,
            lm_head=True):
    """alodlm/model.py:130-169 with the K-1 exit uniforms given explicitly.

    Returns (logits list [N,V], gates list [N], exits [N] int64).  ``x0``
    replaces the embedding and the prelude as the first core input (the
    core block alone); ``trace`` (a dict) receives the per-pass core outputs
    ("core_out") and final-norm inputs ("final_in"); ``lm_head=False`` skips
    the logits.
    """
    K = cfg.max_depth
    emb = p["model.embed_tokens.weight"]
    ids = torch.as_tensor(batch["ids"])
    original = torch.as_tensor(batch["original"])
    masked = torch.as_tensor(batch["masked"])
    dtype = emb.dtype
    cos, sin = rope_tables(batch["positions"], dims.head_dim, dims.theta, dtype)
    if allowed is None:
        allowed = packed_attention_mask(batch["boundaries"], cfg.block_size)
    allowed = torch.as_tensor(allowed)
    trace = {} if trace is None else trace
    trace["core_in"], trace["core_out"], trace["final_in"] = [], [], []

    def layer(i, h):
        return layer_forward(p, f"model.layers.{i}.", h, cos, sin, allowed, dims)

    if x0 is None:
        hidden = emb[ids]
        for i in range(cfg.loop_start):
            hidden = layer(i, hidden)
    else:
        hidden = x0
    gold = emb[original]
    exits = torch.full_like(ids, K)
    logits, gates = [], []
    for depth in range(K):
        if depth:
            hidden = torch.where((exits <= depth)[:, None], gold, hidden)
        trace["core_in"].append(hidden)
        for i in range(cfg.loop_start, cfg.loop_end):
            hidden = layer(i, hidden)
        trace["core_out"].append(hidden)
        readout = hidden
        for i in range(cfg.loop_end, dims.layers):
            readout = layer(i, readout)
        trace["final_in"].append(readout)
        readout = rmsnorm(readout, p["model.norm.weight"], dims.eps)
        if lm_head:
            logits.append(readout @ p["lm_head.weight"].T)
        gates.append(_gate(p, readout, depth))
        if depth < K - 1:
            exits = _sample_exits(gates[-1], exit_uniforms[depth], masked, exits, depth, K)
            hidden = rmsnorm(hidden, p["model.norm.weight"], dims.eps)
    return logits, gates, exits


# ----------------------------------------------------------------------------
# Objective (alodlm/loss.py, alodlm/credit.py)
# ----------------------------------------------------------------------------

def masked_sequence_ids(masked, packed_boundaries):
    """Segment index of every masked row (alodlm/credit.py:7-21)."""
    masked = torch.as_tensor(masked)
    bounds = torch.as_tensor(packed_boundaries)
    if masked.ndim != 1 or masked.dtype != torch.bool:
        raise ValueError("masked_indices must be a one-dimensional boolean tensor")
    if bounds.ndim != 1 or bounds.numel() < 2:
        raise ValueError("Outcome credit requires packed sequence boundaries")
    if int(bounds[0]) != 0 or int(bounds[-1]) != masked.numel():
        raise ValueError("Sequence boundaries must cover the actual packed stream")
    if bool((bounds[1:] < bounds[:-1]).any()):
        raise ValueError("Sequence boundaries must be nondecreasing")
    rows = torch.arange(masked.numel())
    # The segment of a row is the number of segment ends at or before it.
    seg = (rows[:, None] >= bounds[1:][None, :]).sum(1)
    return seg[masked]


def sequence_score_function(credit, logq, seq_ids, count):
    """(1/M) sum_s (sum_{i in s} credit_i)(sum_{i in s} logq_i) (alodlm/credit.py:23-40)."""
    if credit.numel() == 0:
        return logq.sum() * 0
    returns = torch.zeros(count, dtype=credit.dtype).index_add_(0, seq_ids, credit.detach())
    scores = torch.zeros(count, dtype=logq.dtype).index_add_(0, seq_ids, logq)
    return (returns * scores).sum() / credit.numel()


_METRICS = ("denoising", "actor", "sampled_mean_depth", "prediction_cost",
            "regularization_cost", "profile_mean_depth", "first_pass_halt_probability")


def outcome_loss(ce, gates, exits, masked, mask_probability, packed_boundaries, cfg,
                 credit_ce=None):
    """NELBO denoising term plus the sequence score-function actor (alodlm/loss.py:35-90).

    ce: [K, M] masked-token cross-entropies; gates: list of K [N] gate logits;
    exits: [N] sampled exit depth in 1..K.  ``credit_ce`` ([K, M], optional)
    replaces ``ce`` inside the credit's prediction cost only, which is a
    sampled cost without gradient (loss.py:72-78): a test then compares two
    implementations with the same realisation of that cost.
    """
    masked = torch.as_tensor(masked)
    M = int(masked.sum())
    if M == 0:                                                          # loss.py:43-48
        zero = ce.sum() + sum(g.sum() * 0 for g in gates)
        return zero, {k: zero.detach() for k in _METRICS}
    K = cfg.max_depth
    z = torch.as_tensor(exits)[masked]
    g = torch.stack([gt[masked] for gt in gates])                       # [K, M]
    depth = torch.arange(K)[:, None]
    # log survival before depth d and log mass of exiting at d (loss.py:55-57, 64-67)
    log_surv = torch.cat((torch.zeros_like(g[:1]), torch.cumsum(-F.softplus(g), 0)[:-1]))
    log_exit = torch.where(depth == K - 1, log_surv, -F.softplus(-g) + log_surv)
    # truncated stick: survival at the sampled exit, exit mass before it (loss.py:57-58)
    stick = torch.where(depth == z - 1, log_surv, log_exit)
    stick = stick.masked_fill(depth >= z, float("-inf")).exp().detach()
    w = 1 / (torch.as_tensor(mask_probability)[masked].to(ce.dtype) + 1e-8)
    w = w / w.sum()
    denoising = (w * (stick * (ce * (depth < z))).sum(0)).sum()         # loss.py:59-61
    logq = log_exit.gather(0, (z - 1)[None]).squeeze(0)                 # loss.py:68
    with torch.no_grad():
        log_prior = torch.log_softmax(-cfg.depth_prior_c * torch.arange(1, K + 1, dtype=g.dtype), 0)
        qbar = log_exit.detach().exp().mean(1).clamp_min(1e-12)
        marginal = qbar.log()[z - 1]
        costs = (ce if credit_ce is None else torch.as_tensor(credit_ce).to(ce.dtype)).detach()
        prediction = costs.gather(0, (z - 1)[None]).squeeze(0) - costs[0]
        mi_cost = cfg.kl_beta_mi * (logq - marginal)
        budget_cost = cfg.kl_beta_marg * (marginal - log_prior[z - 1])
        credit = (prediction + mi_cost) + budget_cost                   # loss.py:75-78
    seq = masked_sequence_ids(masked, packed_boundaries)
    actor = sequence_score_function(credit, logq, seq, len(packed_boundaries) - 1)
    metrics = {
        "denoising": denoising.detach(),
        "actor": actor.detach(),
        "sampled_mean_depth": z.to(g.dtype).mean(),
        "prediction_cost": prediction.mean(),
        "regularization_cost": (mi_cost + budget_cost).mean(),
        "profile_mean_depth": (qbar * torch.arange(1, K + 1, dtype=g.dtype)).sum(),
        "first_pass_halt_probability": torch.sigmoid(g[0]).mean().detach(),
    }
    return denoising + actor, metrics


def _round_through(x, dtype):
    """Round values to `dtype` (gradient passes unchanged), as a CE evaluated in
    that dtype returns them (alodlm/model.py:180 and alodlm/loss.py:24 run
    F.cross_entropy in the parameter dtype)."""
    if dtype is None:
        return x
    return x + (x.to(dtype).to(x.dtype) - x).detach()


def autoregressive_loss(logits, labels, packed_boundaries, ce_dtype=None):
    """Count-weighted next-token CE on each segment's clean stream (alodlm/loss.py:12-32)."""
    labels = torch.as_tensor(labels)
    total = logits.new_zeros(())
    count = 0
    offsets = [int(v) for v in packed_boundaries]
    for start, end in zip(offsets, offsets[1:]):
        length = (end - start) // 2
        if length < 2:
            continue
        targets = labels[start // 2 + 1:start // 2 + length]
        n = int((targets != -100).sum())
        if n == 0:
            continue
        token = F.cross_entropy(logits[start:start + length - 1], targets,
                                reduction="none", ignore_index=-100)
        total = total + _round_through(token, ce_dtype).sum()
        count += n
    if count:
        return total / count
    return logits.new_zeros((), requires_grad=True)


def step_loss(p, ids, labels, boundaries, dims, cfg, draws, exit_uniforms, ce_dtype=None,
              credit_ce=None):
    """The full ALoDLM._forward_loss (alodlm/model.py:176-187) from explicit draws.

    ``ce_dtype`` (e.g. torch.bfloat16) rounds every per-token cross-entropy to
    that dtype, as the reference's bf16 run does; None keeps full precision.
    ``credit_ce`` is passed to ``outcome_loss``.
    Returns (total loss, metrics dict, extras dict with batch/gates/exits/ce).
    """
    batch = build_batch(ids, labels, boundaries, cfg.block_size, cfg.mask_token_id, draws)
    logits, gates, exits = rollout(p, batch, dims, cfg, exit_uniforms)
    logits = [_round_through(lg, ce_dtype) for lg in logits]  # bf16 LM-head output
    masked = torch.as_tensor(batch["masked"])
    original = torch.as_tensor(batch["original"])
    ce = torch.stack([_round_through(F.cross_entropy(lg[masked], original[masked],
                                                     reduction="none"), ce_dtype)
                      for lg in logits])
    den_actor, metrics = outcome_loss(ce, gates, exits, masked, batch["mask_probability"],
                                      batch["boundaries"], cfg, credit_ce)
    ar = torch.stack([autoregressive_loss(lg, labels, batch["boundaries"], ce_dtype)
                      for lg in logits]).mean()
    total = (den_actor + ar) / 2
    total = total + 0.0 * sum(t.sum() for t in logits + gates)
    metrics = {**metrics, "ar_loss": ar.detach(), "loss": total.detach()}
    return total, metrics, {"batch": batch, "gates": gates, "exits": exits, "ce": ce,
                            "logits": logits}


def readout_objective(p, finals, batch, dims, cfg, exit_uniforms, labels=None, ce_dtype=None,
                      credit_ce=None):
    """The readout and objective of alodlm/model.py:157-187 from given final
    hidden states (the inputs of the final norm), one per pass: final norm,
    LM head, gate, exit sampling, masked cross-entropy, outcome_loss and -
    with ``labels`` - the autoregressive loss; total = (outcome + AR) / 2.
    ``batch`` holds masked, original, mask_probability and boundaries (the
    segment offsets of the rows).  Returns (total, metrics, extras)."""
    K = cfg.max_depth
    masked = torch.as_tensor(batch["masked"])
    original = torch.as_tensor(batch["original"])
    exits = torch.full((masked.numel(),), K, dtype=torch.int64)
    logits, gates = [], []
    for depth in range(K):
        readout = rmsnorm(finals[depth], p["model.norm.weight"], dims.eps)
        logits.append(_round_through(readout @ p["lm_head.weight"].T, ce_dtype))
        gates.append(_gate(p, readout, depth))
        if depth < K - 1:
            exits = _sample_exits(gates[-1], exit_uniforms[depth], masked, exits, depth, K)
    ce = torch.stack([_round_through(F.cross_entropy(lg[masked], original[masked],
                                                     reduction="none"), ce_dtype)
                      for lg in logits])
    den_actor, metrics = outcome_loss(ce, gates, exits, masked, batch["mask_probability"],
                                      batch["boundaries"], cfg, credit_ce)
    if labels is None:
        ar = den_actor.new_zeros(())
    else:
        ar = torch.stack([autoregressive_loss(lg, labels, batch["boundaries"], ce_dtype)
                          for lg in logits]).mean()
    total = (den_actor + ar) / 2
    metrics = {**metrics, "ar_loss": ar.detach(), "loss": total.detach()}
    return total, metrics, {"gates": gates, "exits": exits, "ce": ce, "logits": logits}


# ----------------------------------------------------------------------------
# Parameters, clipping and AdamW
# ----------------------------------------------------------------------------

def param_names(dims):
    """Qwen3ForCausalLM + exit gate parameter names in registration order."""
    names = ["model.embed_tokens.weight"]
    for i in range(dims.layers):
        pre = f"model.layers.{i}."
        names += [pre + s for s in (
            "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
            "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
            "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
            "input_layernorm.weight", "post_attention_layernorm.weight")]
    names += ["model.norm.weight", "lm_head.weight",
              "exit_gate.net.weight", "exit_gate.net.bias", "exit_gate.depth_bias"]
    return names


def init_params(dims, gate_init_pi, seed=0, std=0.02, dtype=torch.float32):
    """Random backbone N(0, std) ([tf] configuration_qwen3.py:71), unit norms,
    and a fresh gate (alodlm/model.py:25-35), drawn from a seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    H, I, V = dims.hidden, dims.intermediate, dims.vocab
    qd, kd = dims.heads * dims.head_dim, dims.kv_heads * dims.head_dim
    shapes = {"self_attn.q_proj.weight": (qd, H), "self_attn.k_proj.weight": (kd, H),
              "self_attn.v_proj.weight": (kd, H), "self_attn.o_proj.weight": (H, qd),
              "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    out = {}
    for name in param_names(dims):
        if name.startswith("exit_gate."):
            continue
        if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
            size = dims.head_dim if ("q_norm" in name or "k_norm" in name) else H
            out[name] = torch.ones(size, dtype=dtype)
        elif name in ("model.embed_tokens.weight", "lm_head.weight"):
            out[name] = (torch.randn(V, H, generator=g) * std).to(dtype)
        else:
            out[name] = (torch.randn(*shapes[name.split(".", 3)[3]], generator=g) * std).to(dtype)
    out["exit_gate.net.weight"] = torch.zeros(1, H, dtype=dtype)
    out["exit_gate.net.bias"] = torch.zeros(1, dtype=dtype)
    out["exit_gate.depth_bias"] = torch.tensor(gate_depth_bias(gate_init_pi),
                                               dtype=torch.float32).to(dtype)
    return out


def clip_coefficient(grads, max_norm):
    """torch.nn.utils.clip_grad_norm_ with norm_type 2 (alodlm/train.py:140):
    total = ||(||g_i||)_i||, coefficient = min(1, max/(total + 1e-6))."""
    total = torch.stack([g.detach().double().norm() for g in grads]).norm()
    return float(total), min(1.0, max_norm / (float(total) + 1e-6))


def adamw_update(param, grad, m, v, step, lr, weight_decay, beta1=0.9, beta2=0.999, eps=1e-8):
    """One decoupled-weight-decay Adam update (torch.optim.AdamW as used at
    alodlm/train.py:49,143; defaults beta=(0.9, 0.999), eps=1e-8).  In place."""
    param.mul_(1 - lr * weight_decay)
    m.mul_(beta1).add_(grad, alpha=1 - beta1)
    v.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    denom = v.sqrt() / math.sqrt(bc2) + eps
    param.addcdiv_(m, denom, value=-lr / bc1)
    return param


def cosine_lr_multiplier(step, warmup, total, cycles=0.5):
    """[tf] optimization.py:134-140, used through get_cosine_schedule_with_warmup
    at alodlm/train.py:55-56."""
    if step < warmup:
        return step / max(1, warmup)
    progress = (step - warmup) / max(1, total - warmup)
    return max(0.0, 0.5 * (1.0 + math.cos(math.pi * cycles * 2.0 * progress)))
