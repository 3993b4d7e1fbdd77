"""Write golden vectors for cached adaptive decoding (alodlm/inference.py).

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_golden_decode.py --reference /root/reference

The reference package is imported from the given checkout and run on the CPU
in float32.  Stored under ``tests/golden/decode/``:

* ``trained/``: the checkpoint a 4-step reference training run of the
  workflow fixture ends on (model files and exit gate), so that decoding is
  also checked with a gate that has learned;
* ``decode.json``: for the fixture's base model (fresh gate) and for the
  trained checkpoint, ``Decoder.generate`` results (token ids, exit depths,
  first-pass halt probabilities, step and pass counts, stop reason) for
  several prompts and decoding settings, plus one prefill window's committed
  K/V summary.
"""

import argparse
import json
from pathlib import Path
import shutil
import sys
import tempfile

import yaml

HERE = Path(__file__).resolve().parent
OUT = HERE / "decode"
FIXTURE = HERE / "workflow" / "fixture"

CASES = [
    # (prompt, DecodeConfig fields)
    ([4, 7, 9], dict(q=.5, tau=.1, max_new_tokens=8, window_size=4)),
    ([4, 7, 10, 11], dict(q=.9, max_new_tokens=7, mode="left1")),
    ([4, 7, 9], dict(q=0, tau=0, max_new_tokens=6, window_size=4)),
    ([4, 7, 9], dict(q=1, tau=0, max_new_tokens=6, window_size=4)),
    ([4, 7, 9], dict(q=0, mode="left1", max_new_tokens=8, window_size=4)),
    (list(range(13, 53)), dict(q=.5, tau=4.15, max_new_tokens=24, window_size=16)),
    ([5, 8, 12, 6, 20], dict(q=.7, tau=4.155, max_new_tokens=20, window_size=5,
                             position_penalty=0.01)),
]
KEYS = ("token_ids", "exit_depths", "first_pass_halt_probabilities", "outer_steps",
        "recurrent_passes", "loop_token_passes", "stop_reason", "generated_tokens",
        "prompt_tokens")


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", required=True)
    args = parser.parse_args()
    reference = Path(args.reference).resolve()
    sys.path.insert(0, str(reference))
    sys.path.insert(0, str(reference / "tests"))
    import torch
    import transformers
    from helpers import tiny_model, tiny_tokenizer, write_fixture
    import alodlm.train as ref_train
    from alodlm.config import TrainConfig
    from alodlm.inference import DecodeConfig, Decoder, PrefixCache
    from alodlm.model import ALoDLM

    torch.set_num_threads(1)
    if OUT.exists():
        shutil.rmtree(OUT)
    OUT.mkdir(parents=True)
    with tempfile.TemporaryDirectory() as tmp:
        root = Path(tmp)
        config = write_fixture(root)
        path = root / "train.yaml"
        path.write_text(yaml.safe_dump(config))
        ref_train.train(TrainConfig.load(path))
        final = root / "run" / "checkpoint-4"
        (OUT / "trained").mkdir()
        for name in ("config.json", "model.safetensors", "exit_gate.pt", "alodlm_config.json"):
            shutil.copy(final / name, OUT / "trained" / name)
        trained = ALoDLM.from_pretrained(final)

    result = {"versions": {"torch": torch.__version__, "transformers": transformers.__version__},
              "cases": [{"prompt": p, "config": c} for p, c in CASES]}
    tokenizer = tiny_tokenizer()
    for name, model in (("base", tiny_model()), ("trained", trained)):
        decoder = Decoder(model, tokenizer)
        runs = []
        for prompt, fields in CASES:
            out = decoder.generate(prompt, DecodeConfig(**fields))
            runs.append({k: out[k] for k in KEYS})
        # one prefill window: the cached prefix K/V of every key
        cache = PrefixCache(model.config)
        prompt = torch.tensor([4, 7, 9, 12, 5])
        empty = torch.empty(0, dtype=torch.long)
        with torch.inference_mode():
            window = decoder._window(prompt, torch.arange(5), cache, empty, DecodeConfig(), empty)[0]
            cache.append(window, torch.arange(5))
        kv = {f"{k[0]},{k[1]}": [cache.values[k][0].flatten().tolist(),
                                 cache.values[k][1].flatten().tolist()]
              for k in sorted(cache.values)}
        result[name] = {"runs": runs, "prefill_kv": kv}
    (OUT / "decode.json").write_text(json.dumps(result, indent=1) + "\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
