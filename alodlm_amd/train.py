"""Training loop (drop-in for alodlm/train.py).  Run: python -m alodlm_amd.train --config train.yaml

``train(config)`` follows alodlm/train.py:22-169 step for step on one GPU:
seeding, the packed cache, the two weight-decay groups, the cosine schedule
with warmup over ``horizon`` optimizer steps, gradient accumulation, the
global-norm clip, ``metrics.jsonl``, checkpoints every ``save_steps`` with
``save_total_limit`` pruning, and exact resumption from a checkpoint's
``trainer_state.json`` (same identity digest, the same pack order within the
interrupted epoch, every random generator restored).

What differs by design:

* one process on one GPU; no accelerate or DeepSpeed wrapper (``use_deepspeed``
  is accepted and only enters the run identity);
* the optimizer is ``FusedAdamW`` with float32 masters and moments whatever
  the parameter dtype; ``training_state/`` keeps accelerate's layout
  (``model.safetensors``, ``optimizer.bin`` as a torch AdamW state dict with
  the float32 masters as an extra per-parameter entry,
  ``custom_checkpoint_0.pkl`` for the scheduler, ``random_states_0.pkl``), so
  checkpoints resume across the two
  implementations; it is read back with ``torch.load(weights_only=True)``;
* the loss finiteness check reads the loss after the backward has been
  queued, so the GPU does not idle between forward and backward; a non-finite
  loss still raises ``FloatingPointError`` before any parameter changes.
"""

import argparse
import itertools
import json
import math
import random
import shutil
from pathlib import Path

import numpy as np
import torch
from torch.utils.data import DataLoader, RandomSampler, Sampler

from .config import TrainConfig
from .data import PackedDataset, load_tokenizer, one_pack, prepare_cache
from .model import ALoDLM
from .optim import FusedAdamW, param_groups

WORLD_SIZE = 1


def set_seed(seed):
    """Seed Python, NumPy, torch's CPU generator and every GPU generator."""
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)


def training_horizon(packs, gradient_accumulation_steps, epochs, max_steps,
                     world_size=WORLD_SIZE):
    """Optimizer steps of the run (alodlm/train.py:50-54)."""
    per_epoch = math.ceil(math.ceil(packs / world_size) / gradient_accumulation_steps)
    horizon = per_epoch * epochs
    return min(horizon, max_steps) if max_steps else horizon


def cosine_schedule(optimizer, horizon, warmup_ratio):
    """Linear warmup over int(horizon * warmup_ratio) steps, then a half cosine
    to zero at ``horizon`` (alodlm/train.py:55-56)."""
    from transformers import get_cosine_schedule_with_warmup
    return get_cosine_schedule_with_warmup(optimizer, int(horizon * warmup_ratio), horizon)


def run_identity(config, cache_identity, horizon, world_size=WORLD_SIZE):
    """What a resumed run must share with the run it resumes
    (alodlm/train.py:68-74): the configuration without paths, the data
    cache's identity, the process count and the horizon."""
    signature = config.to_dict()
    for key in ("model_dir", "train_file", "cache_file", "output_dir", "resume"):
        signature.pop(key)
    return json.loads(json.dumps({"config": signature, "cache_identity": cache_identity,
                                  "world_size": world_size, "horizon": horizon}))


def completed_checkpoints(output):
    """``checkpoint-<step>`` directories with a ``trainer_state.json``, oldest first."""
    found = []
    for path in Path(output).glob("checkpoint-*"):
        number = path.name[len("checkpoint-"):]
        if not path.is_symlink() and number.isdigit() and (path / "trainer_state.json").is_file():
            found.append((int(number), path))
    return [path for _, path in sorted(found)]


def prune_checkpoints(output, limit):
    """Delete all but the newest ``limit`` completed checkpoints."""
    for obsolete in completed_checkpoints(output)[:-limit]:
        shutil.rmtree(obsolete)


class _SkipFirst(Sampler):
    """A sampler without its first ``skip`` indices.  The wrapped sampler still
    draws its whole permutation, so the remaining order is unchanged."""

    def __init__(self, sampler, skip):
        self.sampler, self.skip = sampler, skip

    def __iter__(self):
        return itertools.islice(iter(self.sampler), self.skip, None)

    def __len__(self):
        return max(0, len(self.sampler) - self.skip)


def pack_loader(dataset, skip=0):
    """One shuffled pass over the packs, one pack per item.

    The order comes from ``RandomSampler`` without a generator of its own, as
    in the reference's ``DataLoader(shuffle=True)``: each pass draws its seed
    from torch's CPU generator when iteration starts.
    """
    sampler = RandomSampler(dataset)
    if skip:
        sampler = _SkipFirst(sampler, skip)
    return DataLoader(dataset, batch_size=1, sampler=sampler, collate_fn=one_pack,
                      num_workers=0, pin_memory=torch.cuda.is_available())


def _param_names(model):
    return {id(p): name for name, p in model.named_parameters()}


# torch.load of the training state's tensors and plain containers only; the
# NumPy generator state additionally needs these (accelerate allows the same)
_NUMPY_SAFE = ("numpy.core.multiarray._reconstruct", "numpy._core.multiarray._reconstruct",
               "numpy.ndarray", "numpy.dtype", "numpy.dtypes.UInt32DType")


def _safe_load(path):
    import importlib
    allowed = []
    for qualified in _NUMPY_SAFE:
        module, _, attr = qualified.rpartition(".")
        try:
            allowed.append(getattr(importlib.import_module(module), attr))
        except (ImportError, AttributeError):
            pass
    with torch.serialization.safe_globals(allowed):
        return torch.load(path, map_location="cpu", weights_only=True)


def _adamw_group_defaults(lr):
    """The parameter-group fields torch.optim.AdamW(groups, lr) records in its
    state dict (this torch version's), so that a torch AdamW restores them."""
    probe = torch.optim.AdamW([torch.zeros(1, requires_grad=True)], lr=lr)
    fields = dict(probe.param_groups[0])
    fields.pop("params")
    return fields


def save_training_state(directory, model, optimizer, scheduler, loader_position=0):
    """Write ``directory`` in the layout accelerate's ``save_state`` gives a
    one-process run without DeepSpeed (alodlm/train.py:94; accelerate
    checkpointing.save_accelerator_state):

    * ``model.safetensors``: the model's state dict;
    * ``optimizer.bin``: a ``torch.optim.AdamW`` state dict - per parameter
      index (groups in order) ``step`` (float tensor), ``exp_avg`` and
      ``exp_avg_sq``, plus ``master``, the float32 master weight, which a torch
      AdamW carries along unused; group fields as torch.optim.AdamW records,
      and ``initial_lr`` as the LR scheduler adds it;
    * ``custom_checkpoint_0.pkl``: the LR scheduler's state dict (the
      reference registers its scheduler for checkpointing,
      alodlm/train.py:58);
    * ``random_states_0.pkl``: Python, NumPy, torch CPU and GPU generator
      states and accelerate's step counter (micro-batches since the epoch
      started, ``loader_position``).
    """
    from safetensors.torch import save_file
    directory = Path(directory)
    directory.mkdir(parents=True)
    weights = {k: v.detach().to("cpu").contiguous() for k, v in model.state_dict().items()}
    save_file(weights, str(directory / "model.safetensors"), metadata={"format": "pt"})
    index = {}
    state, groups = {}, []
    for group in optimizer.param_groups:
        defaults = _adamw_group_defaults(group["lr"])
        # torch AdamW's own fields, plus the schedule's base rate that a
        # LambdaLR records in each group (the reference's saved groups carry
        # it, and a scheduler rebuilt with last_epoch >= 0 reads it)
        kept = set(defaults) | {"initial_lr"}
        fields = {**defaults, **{k: v for k, v in group.items() if k in kept}}
        ids = []
        for p in group["params"]:
            i = index.setdefault(id(p), len(index))
            ids.append(i)
            entry = optimizer.state.get(p)
            if not entry:
                continue
            state[i] = {"step": torch.tensor(float(entry["step"]))}
            for key in ("exp_avg", "exp_avg_sq", "master"):
                state[i][key] = entry[key].detach().to("cpu", copy=True)
        groups.append({**fields, "params": ids})
    torch.save({"state": state, "param_groups": groups}, directory / "optimizer.bin")
    torch.save(scheduler.state_dict(), directory / "custom_checkpoint_0.pkl")
    rng = {"step": int(loader_position), "random_state": random.getstate(),
           "numpy_random_seed": np.random.get_state(), "torch_manual_seed": torch.get_rng_state()}
    if torch.cuda.is_available():
        rng["torch_cuda_manual_seed"] = torch.cuda.get_rng_state_all()
    torch.save(rng, directory / "random_states_0.pkl")


def load_training_state(directory, model, optimizer, scheduler):
    """Restore a training state in accelerate's layout: one written by
    ``save_training_state`` or by the reference's ``accelerator.save_state``
    (float32 masters taken from the parameters when the state has none, as a
    torch AdamW keeps no master).  Returns accelerate's step counter."""
    from safetensors.torch import load_file
    directory = Path(directory)
    weights = load_file(str(directory / "model.safetensors"))
    with torch.no_grad():
        missing, unexpected = model.load_state_dict(weights, strict=False)
    if missing or unexpected:
        raise ValueError(f"training state does not fit the model (missing {missing[:3]}, "
                         f"unexpected {unexpected[:3]})")
    optimizer.load_state_dict(_safe_load(directory / "optimizer.bin"))
    scheduler.load_state_dict(_safe_load(directory / "custom_checkpoint_0.pkl"))
    rng = _safe_load(directory / "random_states_0.pkl")
    random.setstate(rng["random_state"])
    np.random.set_state(rng["numpy_random_seed"])
    torch.set_rng_state(rng["torch_manual_seed"])
    cuda = rng.get("torch_cuda_manual_seed")
    if cuda is not None and torch.cuda.is_available() and len(cuda) == torch.cuda.device_count():
        torch.cuda.set_rng_state_all(cuda)
    return int(rng.get("step", 0))


def load_checkpoint_weights(model, directory):
    """Copy a checkpoint's weights (HF safetensors, single file or sharded,
    plus ``exit_gate.pt``) into the model's parameters in place."""
    from safetensors.torch import load_file
    directory = Path(directory)
    index = directory / "model.safetensors.index.json"
    if index.is_file():
        files = sorted(set(json.loads(index.read_text())["weight_map"].values()))
    else:
        files = ["model.safetensors"]
    weights = {}
    for name in files:
        weights.update(load_file(str(directory / name)))
    gate = torch.load(directory / "exit_gate.pt", map_location="cpu", weights_only=True)
    with torch.no_grad():
        model.backbone.load_state_dict(weights, strict=True)
        model.exit_gate.load_state_dict(gate, strict=True)


def train(config):
    """Run (or resume) training; returns the number of optimizer steps taken."""
    if not torch.cuda.is_available():
        raise RuntimeError("alodlm_amd.train needs a GPU: the training step runs on HIP kernels")
    device = torch.device("cuda", torch.cuda.current_device())
    set_seed(config.seed)
    tokenizer = load_tokenizer(config.model_dir)
    cache = prepare_cache(config.train_file, tokenizer, config.cache_file,
                          config.max_seq_length, config.seed)
    dataset = PackedDataset(cache)
    dtype = torch.bfloat16 if config.precision == "bf16" else torch.float32
    model = ALoDLM.from_pretrained(config.model_dir, config.model, dtype, require_gate=False)
    if config.max_seq_length > model.backbone.config.max_position_embeddings:
        raise ValueError("Training sequence length exceeds the model context")
    model.to(device)
    model.engine()  # parameters move into the device arena before the optimizer binds them
    accumulation = config.gradient_accumulation_steps
    optimizer = FusedAdamW(param_groups(model, config.weight_decay), lr=config.learning_rate,
                           max_grad_norm=config.max_grad_norm)
    horizon = training_horizon(len(dataset), accumulation, config.epochs, config.max_steps)
    scheduler = cosine_schedule(optimizer, horizon, config.warmup_ratio)
    output = Path(config.output_dir)
    output.mkdir(parents=True, exist_ok=True)
    print(json.dumps({"global_batch_size": WORLD_SIZE * accumulation,
                      "training_steps": horizon}), flush=True)
    identity = run_identity(config, dataset.cache["identity"], horizon)
    step, start_epoch, skip_batches, epoch_rng = 0, 0, 0, None
    if config.resume:
        resume = Path(config.resume)
        state = json.loads((resume / "trainer_state.json").read_text())
        if state["identity"] != identity:
            raise ValueError("Resume requires the same objective, data, schedule, and process count")
        load_checkpoint_weights(model, resume)
        load_training_state(resume / "training_state", model, optimizer, scheduler)
        step, start_epoch, skip_batches = state["step"], state["epoch"], state["next_batch"]
        epoch_rng = state["epoch_rng"]

    def save(epoch, next_batch):
        destination = output / f"checkpoint-{step}"
        if destination.exists():
            raise FileExistsError("Checkpoint already exists")
        model.save_pretrained(destination)
        tokenizer.save_pretrained(destination)
        save_training_state(destination / "training_state", model, optimizer, scheduler,
                            next_batch)
        record = {"step": step, "epoch": epoch, "next_batch": next_batch,
                  "identity": identity, "epoch_rng": epoch_rng}
        # written last: its presence marks the checkpoint complete
        (destination / "trainer_state.json").write_text(json.dumps(record, indent=2) + "\n")
        prune_checkpoints(output, config.save_total_limit)

    optimizer.zero_grad()
    model.train()
    last_saved = step if config.resume else -1
    micro = 0
    last_index = len(dataset) - 1
    for epoch in range(start_epoch, config.epochs):
        loader = pack_loader(dataset, skip_batches)
        if skip_batches:
            # the interrupted epoch's order: its sampler seed is drawn again from
            # the CPU generator state the epoch started with, after which the
            # generator returns to the checkpoint's state
            checkpoint_cpu_rng = torch.get_rng_state()
            torch.set_rng_state(torch.tensor(epoch_rng["cpu"], dtype=torch.uint8))
            current = iter(loader)
            first = next(current, None)
            torch.set_rng_state(checkpoint_cpu_rng)
            current = itertools.chain(() if first is None else (first,), current)
        else:
            epoch_rng = {"cpu": torch.get_rng_state().tolist(), "sampler": None}
            current = loader
        first_batch, skip_batches = skip_batches, 0
        for batch_index, item in enumerate(current, first_batch):
            if step >= horizon:
                break
            micro += 1
            sync = micro == accumulation or batch_index == last_index
            loss, metrics = model(**item)
            (loss / accumulation if accumulation > 1 else loss).backward()
            norm = optimizer.grad_norm()[0] if sync else None
            if not torch.isfinite(loss):
                raise FloatingPointError("Nonfinite training loss")
            if not sync:
                continue
            if not torch.isfinite(norm):
                raise FloatingPointError("Nonfinite gradient norm")
            optimizer.step()
            scheduler.step()
            optimizer.zero_grad()
            micro = 0
            step += 1
            if step % config.logging_steps == 0 or step == 1:
                values = {key: float(value.detach().float()) for key, value in metrics.items()}
                record = {"step": step, "learning_rate": scheduler.get_last_lr()[0], **values}
                print(json.dumps(record), flush=True)
                with (output / "metrics.jsonl").open("a") as handle:
                    handle.write(json.dumps(record) + "\n")
            if step % config.save_steps == 0 or step == horizon:
                save(epoch, batch_index + 1)
                last_saved = step
            if step >= horizon:
                break
        if step >= horizon:
            break
    if last_saved != step:
        save(config.epochs, 0)
    return step


def main():
    parser = argparse.ArgumentParser(description="Train with sequence outcome credit on MI355X.")
    parser.add_argument("--config", required=True)
    args = parser.parse_args()
    train(TrainConfig.load(args.config))


if __name__ == "__main__":
    main()
