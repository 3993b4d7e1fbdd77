"""Write golden vectors for the ALoDLM training step from the reference.

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_golden.py --reference /root/reference

The reference package is imported from the given checkout on the CPU, in
float32, and only its inputs and outputs are stored (``*.npz`` written with
numpy, loadable with ``allow_pickle=False``).  Cases:

* ``batch_*``: ``alodlm.batch.build_batch`` under ``torch.manual_seed`` for
  ragged segments, ignored labels and several block sizes.
* ``step_micro*``: the ``tests/helpers.tiny_model`` model (hidden 32, 3
  layers, topology 1/2/1, vocab 64) - full ``ALoDLM.forward`` + backward,
  every gradient, and one ``torch.optim.AdamW`` step.
* ``step_tiny``: the tiny training-step configuration (hidden 256, 4 layers
  1/2/1, 4 q / 2 kv heads of 64, SwiGLU 768, vocab 1024, 4 x 128 tokens,
  seed 0) - loss, metrics, gates, exits, CE, and per-gradient summaries
  (norm, a fixed random projection, a strided sample).
* ``step_tiny_bf16``: the same model and inputs cast to bfloat16, as the
  reference runs with ``precision: bf16`` (its eager bf16 rounding sequence
  on the CPU): the same outputs, gates and gradient summaries as float64 of
  the bf16 values.
"""

import argparse
import json
from pathlib import Path
import sys

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.step import Dims, init_params  # noqa: E402  (parameter initialisation only)


from tests.golden import projection_vector, sample_indices  # noqa: E402


def batch_case(build_batch, seed, ids, labels, boundaries, block, mask_id):
    torch.manual_seed(seed)
    b = build_batch(ids, labels, boundaries, block, mask_id, "sdpa")
    return {
        "in_ids": ids.numpy(), "in_labels": labels.numpy(), "in_boundaries": boundaries.numpy(),
        "block_size": np.int64(block), "mask_token_id": np.int64(mask_id), "seed": np.int64(seed),
        "ids": b.ids.numpy(), "original": b.original.numpy(), "positions": b.positions.numpy(),
        "masked": b.masked.numpy(), "mask_probability": b.mask_probability.numpy(),
        "boundaries": b.boundaries.numpy(), "attention_mask": b.attention_mask.numpy(),
    }


def step_case(model, ids, labels, boundaries, seed, lr, full_grads, capture):
    """Run the reference forward+backward and an AdamW step; return arrays."""
    names = [n for n, _ in model.named_parameters()]
    state = {n: p.detach().clone() for n, p in model.named_parameters()}
    captured = {}
    original_rollout = type(model).rollout

    def rollout(self, batch):
        logits, gates, exits = original_rollout(self, batch)
        captured["batch"] = batch
        captured["gates"] = torch.stack([g.detach() for g in gates]).float()
        captured["exits"] = exits.clone()
        return logits, gates, exits

    type(model).rollout = rollout
    try:
        torch.manual_seed(seed)
        loss, metrics = model(ids, labels, boundaries)
    finally:
        type(model).rollout = original_rollout
    loss.backward()
    b = captured["batch"]
    out = {
        "in_ids": ids.numpy(), "in_labels": labels.numpy(), "in_boundaries": boundaries.numpy(),
        "seed": np.int64(seed), "lr": np.float64(lr),
        "loss": np.float64(loss.item()),
        "ids": b.ids.numpy(), "original": b.original.numpy(), "positions": b.positions.numpy(),
        "masked": b.masked.numpy(), "mask_probability": b.mask_probability.numpy(),
        "boundaries": b.boundaries.numpy(),
        "gates": captured["gates"].numpy(), "exits": captured["exits"].numpy(),
    }
    for key, value in metrics.items():
        out["metric_" + key] = np.float64(value.item())
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
    for index, name in enumerate(names):
        g = grads[name].double().flatten()
        if full_grads:
            out["param_" + name] = state[name].numpy()
            out["grad_" + name] = grads[name].numpy()
        else:
            out["gnorm_" + name] = np.float64(g.norm().item())
            out["gproj_" + name] = np.float64((g * projection_vector(index, g.numel())).sum().item())
            out["gsample_" + name] = g[torch.as_tensor(sample_indices(g.numel()))].numpy()
    # One clipped AdamW step exactly as alodlm/train.py:42-56,140-143 (horizon 1, no warmup).
    no_decay = ("bias", "LayerNorm.weight", "layer_norm.weight")
    groups = [
        {"params": [p for n, p in model.named_parameters() if not any(s in n for s in no_decay)],
         "weight_decay": 0.01},
        {"params": [p for n, p in model.named_parameters() if any(s in n for s in no_decay)],
         "weight_decay": 0.0},
    ]
    optimizer = torch.optim.AdamW(groups, lr=lr)
    norm = torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
    out["grad_total_norm"] = np.float64(norm.item())
    optimizer.step()
    for index, (name, p) in enumerate(model.named_parameters()):
        delta = (p.detach() - state[name]).double().flatten()
        if full_grads:
            out["updated_" + name] = p.detach().numpy()
        else:
            out["dnorm_" + name] = np.float64(delta.norm().item())
            out["dproj_" + name] = np.float64((delta * projection_vector(index, delta.numel())).sum().item())
    out["param_names"] = np.array(names)
    return out


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--reference", default="/root/reference")
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    sys.path.insert(0, str(Path(args.reference) / "tests"))
    torch.set_num_threads(1)
    from alodlm.batch import build_batch
    from alodlm.config import ModelConfig
    from alodlm.model import ALoDLM
    from helpers import tiny_model
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cases = {}
    # --- dual-stream batches --------------------------------------------------
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 50, (45,), generator=g)
    labels = ids.clone()
    labels[:6] = -100
    labels[20:23] = -100
    cases["batch_ragged"] = batch_case(build_batch, 11, ids, labels,
                                       torch.tensor([0, 13, 14, 31, 45]), 4, 3)
    ids = torch.randint(0, 1000, (300,), generator=g)
    labels = ids.clone()
    labels[::7] = -100
    cases["batch_block32"] = batch_case(build_batch, 12, ids, labels,
                                        torch.tensor([0, 100, 171, 300]), 32, 3)
    ids = torch.randint(0, 64, (16,), generator=g)
    cases["batch_allmasked_labels"] = batch_case(
        build_batch, 13, ids, torch.full_like(ids, -100), torch.tensor([0, 9, 16]), 3, 3)

    # --- micro step: the reference's own tiny_model -----------------------------
    model = tiny_model()
    ids = torch.tensor([4, 7, 9, 2, 5, 9, 12, 2])
    labels = ids.clone()
    labels[:4] = -100
    cases["step_micro"] = step_case(model, ids, labels, torch.tensor([0, 8]), 5, 1e-3, True, None)
    model = tiny_model()
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(4, 64, (23,), generator=g)
    labels = ids.clone()
    labels[:3] = -100
    labels[9:12] = -100
    cases["step_micro_ragged"] = step_case(model, ids, labels, torch.tensor([0, 9, 10, 23]), 6,
                                           1e-3, True, None)

    # --- tiny training-step configuration -------------------------------------
    dims = Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768, vocab=1024,
                layers=4, eps=1e-6, theta=1e6)
    cfg = ModelConfig(loop_start=1, loop_end=3, mask_token_id=3, block_size=32,
                      attention_backend="sdpa", compile_layers=False)
    backbone = Qwen3ForCausalLM(Qwen3Config(
        hidden_size=256, intermediate_size=768, num_hidden_layers=4, num_attention_heads=4,
        num_key_value_heads=2, head_dim=64, vocab_size=1024, max_position_embeddings=512,
        rms_norm_eps=1e-6, rope_parameters={"rope_type": "default", "rope_theta": 1e6},
        bos_token_id=1, eos_token_id=2, pad_token_id=0, tie_word_embeddings=False))
    model = ALoDLM(backbone, cfg)
    params = init_params(dims, cfg.gate_init_pi, seed=0)
    model.load_state_dict({(k if k.startswith("exit_gate.") else "backbone." + k): v
                           for k, v in params.items()}, strict=True)
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 1024, (512,), generator=g)
    cases["step_tiny"] = step_case(model, ids, ids.clone(), torch.tensor([0, 128, 256, 384, 512]),
                                   0, 1e-4, False, None)
    model = ALoDLM(Qwen3ForCausalLM(backbone.config), cfg)
    model.load_state_dict({(k if k.startswith("exit_gate.") else "backbone." + k): v
                           for k, v in params.items()}, strict=True)
    model = model.to(torch.bfloat16)
    cases["step_tiny_bf16"] = step_case(model, ids, ids.clone(),
                                        torch.tensor([0, 128, 256, 384, 512]), 0, 1e-4, False, None)

    meta = {"torch": torch.__version__}
    import transformers
    meta["transformers"] = transformers.__version__
    for name, arrays in cases.items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
    (HERE / "versions.json").write_text(json.dumps(meta, indent=2) + "\n")
    print(json.dumps({"written": sorted(cases), **meta}))


if __name__ == "__main__":
    main()
