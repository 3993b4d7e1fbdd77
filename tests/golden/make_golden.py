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
* ``step_1p7b_layers_bf16``: Qwen3-1.7B layer shapes (hidden 2048, 16 / 8
  heads of 128, SwiGLU 6144), vocabulary 151936, two layers run as the
  recurrent core (loop 0-2), K = 4, one 2048-token segment, the bf16 weights
  of tests/test_shapes_gpu.py (seed 31): the reference's bf16 step (loss,
  metrics, masks, gates, exits, every depth's masked cross-entropies,
  per-gradient norm, projection and a 4096-element strided sample) and, under
  ``f32_``, the reference's float32 step on the same (bf16-valued) weights
  with the bf16 run's exits - the reference's own bf16-vs-float32 gap at
  that shape.  ``--cases step_1p7b_layers_bf16`` writes this case alone
  (about ten minutes and 40 GB on 8 cores).
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


def real_shape_run(model, ids, labels, boundaries, seed, forced_exits=None, samples=4096):
    """The reference forward + backward at a real shape: loss, metrics, batch,
    gates, exits, the masked cross-entropies [K, M] and gradient summaries.
    ``forced_exits`` (a previous run's exits) replaces the rollout's exit
    uniforms by 0 at each row's exit depth and 1 elsewhere, so the run takes
    exactly those exits (alodlm/model.py:163-167 selects u < hazard)."""
    import alodlm.model as reference_model
    captured = {}
    original_rollout = type(model).rollout
    original_outcome = reference_model.outcome_loss
    original_rand_like = torch.rand_like
    K = model.config.max_depth
    depth = {"d": 0}

    def rollout(self, batch):
        logits, gates, exits = original_rollout(self, batch)
        captured["batch"] = batch
        captured["gates"] = torch.stack([g.detach() for g in gates]).float()
        captured["exits"] = exits.clone()
        return logits, gates, exits

    def outcome(ce, *args, **kwargs):
        captured["ce"] = ce.detach().float().clone()
        return original_outcome(ce, *args, **kwargs)

    def rand_like(t, *args, **kwargs):
        d = depth["d"]
        depth["d"] += 1
        return torch.where(forced_exits == d + 1, 0.0, 1.0).to(t.dtype)

    type(model).rollout = rollout
    reference_model.outcome_loss = outcome
    if forced_exits is not None:
        torch.rand_like = rand_like
    try:
        torch.manual_seed(seed)
        loss, metrics = model(ids, labels, boundaries)
    finally:
        type(model).rollout = original_rollout
        reference_model.outcome_loss = original_outcome
        torch.rand_like = original_rand_like
    if forced_exits is not None:
        assert depth["d"] == K - 1
    loss.backward()
    b = captured["batch"]
    out = {"loss": np.float64(loss.item()), "gates": captured["gates"].numpy(),
           "exits": captured["exits"].numpy(), "ce": captured["ce"].numpy(),
           "ids": b.ids.numpy(), "original": b.original.numpy(), "positions": b.positions.numpy(),
           "masked": b.masked.numpy(), "mask_probability": b.mask_probability.numpy(),
           "boundaries": b.boundaries.numpy()}
    for key, value in metrics.items():
        out["metric_" + key] = np.float64(value.item())
    names = [n for n, _ in model.named_parameters()]
    for index, (name, p) in enumerate(model.named_parameters()):
        g = p.grad.detach().double().flatten()
        out["gnorm_" + name] = np.float64(g.norm().item())
        out["gproj_" + name] = np.float64((g * projection_vector(index, g.numel())).sum().item())
        out["gsample_" + name] = g[torch.as_tensor(sample_indices(g.numel(), samples))].numpy()
    out["param_names"] = np.array(names)
    model.zero_grad(set_to_none=True)
    return out


def reference_bf16(ALoDLM, backbone, cfg, state):
    """The reference model in bfloat16 as its training loads one
    (alodlm/train.py:38-39 -> ALoDLM.from_pretrained(dir, config, bfloat16),
    model.py:95-114): the backbone saved and read back by transformers with
    that dtype, which keeps the rotary inverse frequencies in float32 (a
    ``.to(bfloat16)`` of the module would round them), then ``state`` (the
    parameters, gate included) loaded."""
    import tempfile
    with tempfile.TemporaryDirectory() as directory:
        backbone.save_pretrained(directory)
        model = ALoDLM.from_pretrained(directory, cfg, torch.bfloat16, require_gate=False)
    assert model.backbone.model.rotary_emb.inv_freq.dtype == torch.float32
    model.load_state_dict(state, strict=True)
    return model


def real_shape_case(ALoDLM, ModelConfig, Qwen3Config, Qwen3ForCausalLM, seed=31):
    from oracle.step import Objective
    from tests.test_shapes_gpu import MASK_ID, VOCAB, _bf16_params, _dims, _tokens
    dims = _dims(2048, 16, 8, 6144, layers=2)
    obj = Objective(loop_start=0, loop_end=2, mask_token_id=MASK_ID, block_size=32)
    params = _bf16_params(dims, obj, seed=seed)
    cfg = ModelConfig(loop_start=0, loop_end=2, mask_token_id=MASK_ID, block_size=32,
                      attention_backend="sdpa", compile_layers=False,
                      gradient_checkpointing=False)
    with torch.device("meta"):
        backbone = Qwen3ForCausalLM(Qwen3Config(
            hidden_size=2048, intermediate_size=6144, num_hidden_layers=2,
            num_attention_heads=16, num_key_value_heads=8, head_dim=128, vocab_size=VOCAB,
            max_position_embeddings=4096, rms_norm_eps=1e-6,
            rope_parameters={"rope_type": "default", "rope_theta": 1e6},
            bos_token_id=1, eos_token_id=2, pad_token_id=0, tie_word_embeddings=False))
    backbone = backbone.to_empty(device="cpu")
    model = reference_bf16(ALoDLM, backbone, cfg,
                           {(k if k.startswith("exit_gate.") else "backbone." + k): v
                            for k, v in params.items()})
    del backbone
    ids, labels, bounds = _tokens([2048], seed=seed)
    out = real_shape_run(model, ids, labels, bounds, seed)
    out.update({"in_ids": ids.numpy(), "in_labels": labels.numpy(),
                "in_boundaries": bounds.numpy(), "seed": np.int64(seed)})
    model = model.float()
    f32 = real_shape_run(model, ids, labels, bounds, seed,
                         forced_exits=torch.as_tensor(out["exits"]))
    assert np.array_equal(f32["masked"], out["masked"]) and np.array_equal(f32["exits"],
                                                                          out["exits"])
    for key in ("loss", "gates", "ce"):
        out["f32_" + key] = f32[key]
    for key, value in f32.items():
        if key.startswith(("metric_", "gnorm_", "gproj_", "gsample_")):
            out["f32_" + key] = value
    return out


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--reference", default="/root/reference")
    parser.add_argument("--cases", nargs="*", help="write only these cases")
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    sys.path.insert(0, str(Path(args.reference) / "tests"))
    torch.set_num_threads(1)
    from alodlm.batch import build_batch
    from alodlm.config import ModelConfig
    from alodlm.model import ALoDLM
    from helpers import tiny_model
    from transformers import Qwen3Config, Qwen3ForCausalLM

    if args.cases == ["step_1p7b_layers_bf16"]:
        torch.set_num_threads(8)
        arrays = real_shape_case(ALoDLM, ModelConfig, Qwen3Config, Qwen3ForCausalLM)
        np.savez_compressed(HERE / "step_1p7b_layers_bf16.npz", **arrays)
        print(json.dumps({"written": ["step_1p7b_layers_bf16"], "loss": float(arrays["loss"]),
                          "f32_loss": float(arrays["f32_loss"])}))
        return
    wanted = set(args.cases or [])
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
    model = reference_bf16(ALoDLM, Qwen3ForCausalLM(backbone.config), cfg,
                           {(k if k.startswith("exit_gate.") else "backbone." + k):
                            v.to(torch.bfloat16) for k, v in params.items()})
    cases["step_tiny_bf16"] = step_case(model, ids, ids.clone(),
                                        torch.tensor([0, 128, 256, 384, 512]), 0, 1e-4, False, None)

    meta = {"torch": torch.__version__}
    import transformers
    meta["transformers"] = transformers.__version__
    if wanted:
        cases = {k: v for k, v in cases.items() if k in wanted}
    for name, arrays in cases.items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
    (HERE / "versions.json").write_text(json.dumps(meta, indent=2) + "\n")
    print(json.dumps({"written": sorted(cases), **meta}))


if __name__ == "__main__":
    main()
