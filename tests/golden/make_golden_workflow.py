"""Write golden vectors for the packed-data path and the training loop.

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_golden_workflow.py --reference /root/reference

The reference package is imported from the given checkout on the CPU.  Only
inputs and outputs are stored, under ``tests/golden/workflow/``:

* ``fixture/``: the workflow fixture of the reference's tests (a random
  Qwen3 model with hidden 32, 3 layers, vocab 64, saved with its word-level
  tokenizer and chat template, and ``training.jsonl`` of 12 conversations).
* ``cache_fixture.npz`` / ``cache_varied.npz``: ``alodlm.data.prepare_cache``
  outputs (every tensor, the identity digest, the filtered count) for the
  fixture (max length 24, seed 17) and for ``varied.jsonl`` (250
  conversations of 0-40 words, some invalid or too long; max length 48,
  seed 5).
* ``train.json``: an ``alodlm.train.train`` run of the fixture configuration
  (fp32, 2 epochs capped at 4 steps, save every 2, log every step, seed 17)
  and of its resumption from ``checkpoint-2``, plus a run with gradient
  accumulation over 2 packs and no step cap (2 epochs): the printed header,
  the pack index each step consumed, every ``metrics.jsonl`` record, each
  checkpoint's ``trainer_state.json`` and file names.
* ``reference_checkpoint-2/``: the run's ``checkpoint-2`` as the reference
  wrote it, ``training_state/`` in accelerate's layout included.
"""

import argparse
import json
from pathlib import Path
import random
import shutil
import sys
import tempfile
from contextlib import redirect_stdout
import io

import numpy as np
import yaml

HERE = Path(__file__).resolve().parent
OUT = HERE / "workflow"


def cache_arrays(path, torch):
    cached = torch.load(path, weights_only=True)
    arrays = {k: cached[k].numpy() for k in ("input_ids", "labels", "batch_offsets",
                                              "cum_flat", "cum_offsets")}
    arrays["identity"] = np.array(cached["identity"])
    arrays["filtered_records"] = np.array(cached["filtered_records"])
    return arrays


def varied_records(seed=5, count=250):
    words = ["Return", "value", "one", "two", "three", "."] + [f"t{i}" for i in range(13, 64)]
    rng = random.Random(seed)
    lines = []
    for i in range(count):
        kind = rng.random()
        ask = " ".join(rng.choice(words) for _ in range(rng.randint(0, 20)))
        answer = " ".join(rng.choice(words) for _ in range(rng.randint(0, 20)))
        if kind < 0.05:
            record = []  # empty: dropped
        elif kind < 0.10:
            record = {"role": "user", "content": ask}  # not a list: invalid
        elif kind < 0.15:
            record = [{"role": "user", "content": ask}, {"role": "user", "content": answer}]
        elif kind < 0.25:
            record = [{"role": "user", "content": ask}]  # single message: unsupervised
        else:
            record = [{"role": "user", "content": ask}, {"role": "assistant", "content": answer}]
        lines.append(json.dumps(record))
    lines.insert(40, "")  # blank lines are skipped
    return "\n".join(lines) + "\n"


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", required=True)
    args = parser.parse_args()
    reference = Path(args.reference).resolve()
    sys.path.insert(0, str(reference))
    sys.path.insert(0, str(reference / "tests"))
    import torch
    import transformers
    from helpers import write_fixture
    import alodlm.train as ref_train
    from alodlm.config import TrainConfig
    from alodlm.data import PackedDataset, load_tokenizer, prepare_cache

    if OUT.exists():
        shutil.rmtree(OUT)
    (OUT / "fixture").mkdir(parents=True)
    with tempfile.TemporaryDirectory() as tmp:
        root = Path(tmp)
        config = write_fixture(root)
        shutil.copytree(root / "base", OUT / "fixture" / "base")
        shutil.copy(root / "training.jsonl", OUT / "fixture" / "training.jsonl")
        (OUT / "fixture" / "varied.jsonl").write_text(varied_records())
        tokenizer = load_tokenizer(config["model_dir"])

        path = prepare_cache(config["train_file"], tokenizer, root / "fixture_cache.pt", 24, 17)
        np.savez(OUT / "cache_fixture.npz", **cache_arrays(path, torch))
        path = prepare_cache(OUT / "fixture" / "varied.jsonl", tokenizer,
                             root / "varied_cache.pt", 48, 5)
        np.savez(OUT / "cache_varied.npz", **cache_arrays(path, torch))

        consumed = []
        original_getitem = PackedDataset.__getitem__

        def recording_getitem(self, index):
            consumed.append(int(index))
            return original_getitem(self, index)

        PackedDataset.__getitem__ = recording_getitem
        result = {"config": {k: v for k, v in config.items()
                             if k not in ("model_dir", "train_file", "output_dir", "cache_file")}}
        for name, resume, extra in (("run", None, {}), ("resumed", "run/checkpoint-2", {}),
                                    ("accumulated", None,
                                     {"gradient_accumulation_steps": 2, "max_steps": 0})):
            cfg = dict(config, output_dir=str(root / name), **extra)
            if resume:
                cfg["resume"] = str(root / resume)
            yaml_path = root / f"{name}.yaml"
            yaml_path.write_text(yaml.safe_dump(cfg))
            consumed.clear()
            stdout = io.StringIO()
            with redirect_stdout(stdout):
                steps = ref_train.train(TrainConfig.load(yaml_path))
            lines = [json.loads(line) for line in stdout.getvalue().splitlines()
                     if line.startswith("{")]
            output = root / name
            checkpoints = {}
            for ckpt in sorted(output.glob("checkpoint-*")):
                checkpoints[ckpt.name] = {
                    "trainer_state": json.loads((ckpt / "trainer_state.json").read_text()),
                    "files": sorted(p.name for p in ckpt.iterdir()),
                }
            if name == "run":
                # a complete reference checkpoint (weights, tokenizer,
                # accelerate training state, trainer state) to resume from
                shutil.copytree(output / "checkpoint-2", OUT / "reference_checkpoint-2")
            result[name] = {
                "steps": steps,
                "header": lines[0],
                "consumed": list(consumed),
                "metrics": [json.loads(line) for line in
                            (output / "metrics.jsonl").read_text().splitlines()],
                "checkpoints": checkpoints,
            }
        PackedDataset.__getitem__ = original_getitem
    result["versions"] = {"torch": torch.__version__, "transformers": transformers.__version__}
    (OUT / "train.json").write_text(json.dumps(result, indent=1) + "\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
