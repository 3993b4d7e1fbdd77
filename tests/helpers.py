"""Shared test fixtures: model construction and replayable randomness."""

import sys

import numpy as np
import torch

from oracle import step as O


def log(msg):
    """Name the case before a GPU step so a failing run says what it was doing."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def gpu_available():
    return torch.cuda.is_available()


def hf_backbone(dims, dtype=torch.float32):
    """A Qwen3ForCausalLM of these dimensions with uninitialised parameters
    (built on the meta device, so large vocabularies cost no random init);
    callers load every parameter.  The rotary embedding's frequency buffer is
    computed as transformers computes it."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(
        hidden_size=dims.hidden, intermediate_size=dims.intermediate,
        num_hidden_layers=dims.layers, num_attention_heads=dims.heads,
        num_key_value_heads=dims.kv_heads, head_dim=dims.head_dim, vocab_size=dims.vocab,
        max_position_embeddings=4096, rms_norm_eps=dims.eps,
        rope_parameters={"rope_type": "default", "rope_theta": dims.theta},
        bos_token_id=1, eos_token_id=2, pad_token_id=0, tie_word_embeddings=False)
    with torch.device("meta"):
        model = Qwen3ForCausalLM(cfg)
    model = model.to_empty(device="cpu")
    model.model.rotary_emb = Qwen3RotaryEmbedding(config=cfg)
    return model.to(dtype)


def make_model(dims, objective, params, device="cuda", dtype=torch.float32):
    """An alodlm_amd ALoDLM holding `params` (oracle names), on `device`."""
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.model import ALoDLM
    backbone = hf_backbone(dims, dtype)
    state = {k: v for k, v in params.items() if not k.startswith("exit_gate.")}
    backbone.load_state_dict({k: v.to(dtype) for k, v in state.items()}, strict=True)
    cfg = ModelConfig(loop_start=objective.loop_start, loop_end=objective.loop_end,
                      max_depth=objective.max_depth, mask_token_id=objective.mask_token_id,
                      block_size=objective.block_size, gate_init_pi=objective.gate_init_pi,
                      depth_prior_c=objective.depth_prior_c, kl_beta_mi=objective.kl_beta_mi,
                      kl_beta_marg=objective.kl_beta_marg)
    model = ALoDLM(backbone.to(device), cfg)
    model.exit_gate.load_state_dict({
        "net.weight": params["exit_gate.net.weight"].to(dtype),
        "net.bias": params["exit_gate.net.bias"].to(dtype),
        "depth_bias": params["exit_gate.depth_bias"].to(dtype)})
    return model.to(device)


def draw_masking(labels_host, offsets, block_size, device, generator=None):
    """The masking draws made the way alodlm/batch.py:50-60 makes them: per
    segment one ``uniform_`` of the block ratios, then one ``randperm`` per
    block whose masked count round(n * p) is nonzero.  Returns per-block
    (p, count) host arrays and the permutations (None where count is 0)."""
    from alodlm_amd.batch import block_supervised_counts
    probs, counts, perms = [], [], []
    for (a, b), n in zip(zip(offsets, offsets[1:]),
                         block_supervised_counts(labels_host, offsets, block_size)):
        nblocks = (b - a + block_size - 1) // block_size
        u = torch.empty(nblocks, device=device).uniform_(0, 1, generator=generator).clamp_min(1e-8)
        p = u.cpu().numpy().astype(np.float64)
        count = np.array([round(int(k) * float(v)) for k, v in zip(n, p)], dtype=np.int64)
        probs.extend(p.tolist())
        counts.extend(count.tolist())
        for blk in range(nblocks):
            perms.append(torch.randperm(int(n[blk]), device=device, generator=generator)
                         if count[blk] else None)
    return np.asarray(probs, dtype=np.float32), np.asarray(counts, dtype=np.int32), perms


def cpu_draws(labels, boundaries, block_size, seed, max_depth):
    """Masking draws and exit uniforms consumed from the CPU default generator
    in the reference's order (alodlm/batch.py:50-60, alodlm/model.py:166)."""
    torch.manual_seed(seed)
    labels_host = torch.as_tensor(labels).numpy()
    offsets = [int(v) for v in boundaries]
    draws = draw_masking(labels_host, offsets, block_size, "cpu", None)
    n = 2 * len(labels_host)
    uniforms = [torch.rand(n) for _ in range(max_depth - 1)]
    return draws, uniforms


def oracle_draws(draws, offsets, block_size):
    """Convert (p, count, perms) per block into the oracle's (uniforms per
    segment, perms) form."""
    probs, counts, perms = draws
    uniforms, i = [], 0
    for a, b in zip(offsets, offsets[1:]):
        nb = (b - a + block_size - 1) // block_size
        uniforms.append(torch.from_numpy(np.asarray(probs[i:i + nb], dtype=np.float32)))
        i += nb
    return uniforms, [None if p is None else p.cpu() for p in perms]


def named_grads(model):
    return {n: p.grad for n, p in model.named_parameters()}


def oracle_name(name):
    return name[len("backbone."):] if name.startswith("backbone.") else name


def cosine(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    na, nb = a.norm(), b.norm()
    if na == 0 and nb == 0:
        return 1.0
    return float((a @ b) / (na * nb).clamp_min(1e-300))
