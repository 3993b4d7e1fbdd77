"""The training loop on the GPU (alodlm/train.py; tests/test_workflow.py:20-60):
a 4-step run of the workflow fixture compared with the reference's recorded
run, exact resumption, and the loop's error and pruning behaviour."""

import json
import shutil
import sys

import pytest
import torch

from tests.golden import HERE as GOLDEN

pytestmark = pytest.mark.gpu

RUN = json.loads((GOLDEN / "workflow" / "train.json").read_text())
FIXTURE = GOLDEN / "workflow" / "fixture"


def write_config(tmp_path, name, **overrides):
    import yaml
    values = dict(RUN["config"])
    values.update(model_dir=str(FIXTURE / "base"), train_file=str(tmp_path / "training.jsonl"),
                  output_dir=str(tmp_path / name), cache_file=str(tmp_path / "packed.pt"))
    values.update(overrides)
    path = tmp_path / f"{name}.yaml"
    path.write_text(yaml.safe_dump(values))
    return path


def run_train(path, consumed=None):
    from alodlm_amd.config import TrainConfig
    from alodlm_amd import data, train
    original = data.PackedDataset.__getitem__

    def recording(self, index):
        if consumed is not None:
            consumed.append(int(index))
        return original(self, index)

    data.PackedDataset.__getitem__ = recording
    try:
        return train.train(TrainConfig.load(path))
    finally:
        data.PackedDataset.__getitem__ = original


def state_of(directory):
    """A checkpoint's saved tensors, in their saved dtype."""
    from safetensors.torch import load_file
    state = {f"backbone.{k}": v for k, v in load_file(str(directory / "model.safetensors")).items()}
    gate = torch.load(directory / "exit_gate.pt", map_location="cpu", weights_only=True)
    state.update({f"exit_gate.{k}": v for k, v in gate.items()})
    return state


@pytest.fixture(scope="module")
def workflow(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("workflow")
    shutil.copy(FIXTURE / "training.jsonl", tmp / "training.jsonl")
    consumed = []
    print("[train] fixture run, 4 steps", file=sys.stderr, flush=True)
    steps = run_train(write_config(tmp, "run"), consumed)
    return tmp, steps, consumed


def test_run_matches_reference_loop(workflow):
    """Same horizon, pack order, learning rates, metric names, checkpoint
    steps, files and trainer state as the reference's run."""
    tmp, steps, consumed = workflow
    assert steps == RUN["run"]["steps"] == 4
    assert consumed == RUN["run"]["consumed"][:4]
    records = [json.loads(l) for l in (tmp / "run" / "metrics.jsonl").read_text().splitlines()]
    want = RUN["run"]["metrics"]
    assert [r["step"] for r in records] == [r["step"] for r in want]
    for got, ref in zip(records, want):
        assert list(got) == list(ref)
        assert got["learning_rate"] == pytest.approx(ref["learning_rate"], rel=1e-12, abs=1e-18)
        assert all(torch.isfinite(torch.tensor(v)) for v in got.values())
    for name, ref in RUN["run"]["checkpoints"].items():
        directory = tmp / "run" / name
        files = sorted(p.name for p in directory.iterdir())
        assert files == ref["files"], name
        state = json.loads((directory / "trainer_state.json").read_text())
        want_state = ref["trainer_state"]
        for key in ("step", "epoch", "next_batch", "identity"):
            assert state[key] == want_state[key], (name, key)
        # the CPU generator entered the epoch in the reference's state: model
        # loading consumed the same random numbers
        assert state["epoch_rng"] == want_state["epoch_rng"], name


def test_trained_checkpoint_loads(workflow):
    """tests/test_workflow.py:48-52: the final checkpoint loads, is finite and
    the gate has learned."""
    tmp, _, _ = workflow
    from alodlm_amd.model import ALoDLM
    saved = ALoDLM.from_pretrained(tmp / "run" / "checkpoint-4")
    assert all(torch.isfinite(t).all() for t in saved.state_dict().values())
    assert float(saved.exit_gate.net.weight.detach().norm()) > 0


def test_resume_is_exact(workflow):
    """tests/test_workflow.py:53-60: resuming from checkpoint-2 reproduces the
    final weights bit for bit, and the logged metrics of steps 3 and 4."""
    tmp, _, _ = workflow
    consumed = []
    print("[train] resume from checkpoint-2", file=sys.stderr, flush=True)
    run_train(write_config(tmp, "resumed", resume=str(tmp / "run" / "checkpoint-2")), consumed)
    assert consumed[:2] == RUN["resumed"]["consumed"][:2]
    original, resumed = state_of(tmp / "run" / "checkpoint-4"), state_of(tmp / "resumed" / "checkpoint-4")
    for key, value in resumed.items():
        torch.testing.assert_close(value, original[key], atol=0, rtol=0, msg=key)
    straight = (tmp / "run" / "metrics.jsonl").read_text().splitlines()[2:]
    again = (tmp / "resumed" / "metrics.jsonl").read_text().splitlines()
    assert again == straight


def test_resume_from_reference_checkpoint(tmp_path):
    """A checkpoint the reference wrote (its recorded run's checkpoint-2, with
    training_state/ saved by accelerate) resumes here: the interrupted epoch's
    remaining packs in the reference's order, the reference resumption's
    learning rates and metric names, and its final trainer state."""
    shutil.copy(FIXTURE / "training.jsonl", tmp_path / "training.jsonl")
    consumed = []
    print("[train] resume from the reference's checkpoint-2", file=sys.stderr, flush=True)
    steps = run_train(write_config(tmp_path, "resumed", resume=str(
        GOLDEN / "workflow" / "reference_checkpoint-2")), consumed)
    want = RUN["resumed"]
    assert steps == want["steps"]
    # the remaining packs of the interrupted epoch (later epochs draw their
    # order after this run's masks, which come from the GPU generator here)
    assert consumed[:2] == want["consumed"][:2]
    records = [json.loads(l) for l in (tmp_path / "resumed" / "metrics.jsonl").read_text().splitlines()]
    assert [r["step"] for r in records] == [r["step"] for r in want["metrics"]]
    for got, ref in zip(records, want["metrics"]):
        assert list(got) == list(ref)
        assert got["learning_rate"] == pytest.approx(ref["learning_rate"], rel=1e-12, abs=1e-18)
    for name, ref in want["checkpoints"].items():
        state = json.loads((tmp_path / "resumed" / name / "trainer_state.json").read_text())
        for key in ("step", "epoch", "next_batch", "identity"):
            assert state[key] == ref["trainer_state"][key], (name, key)


def test_resume_requires_same_identity(workflow):
    tmp, _, _ = workflow
    path = write_config(tmp, "mismatch", learning_rate=2e-5, resume=str(tmp / "run" / "checkpoint-2"))
    with pytest.raises(ValueError, match="Resume requires"):
        run_train(path)


def test_existing_checkpoint_is_not_overwritten(workflow):
    tmp, _, _ = workflow
    with pytest.raises(FileExistsError):
        run_train(write_config(tmp, "run"))


def test_bf16_resume_is_exact_and_prunes(tmp_path):
    """bf16 parameters with float32 masters: a resumed run ends on the same
    weights as the straight run; save_total_limit keeps the newest checkpoint."""
    shutil.copy(FIXTURE / "training.jsonl", tmp_path / "training.jsonl")
    print("[train] bf16 run", file=sys.stderr, flush=True)
    run_train(write_config(tmp_path, "run", precision="bf16", save_steps=1, max_steps=3))
    kept = sorted(p.name for p in (tmp_path / "run").glob("checkpoint-*"))
    assert kept == ["checkpoint-1", "checkpoint-2", "checkpoint-3"]
    print("[train] bf16 resume", file=sys.stderr, flush=True)
    run_train(write_config(tmp_path, "resumed", precision="bf16", save_steps=1, max_steps=3,
                           resume=str(tmp_path / "run" / "checkpoint-1")))
    a, b = state_of(tmp_path / "run" / "checkpoint-3"), state_of(tmp_path / "resumed" / "checkpoint-3")
    for key, value in b.items():
        assert value.dtype == torch.bfloat16, key
        torch.testing.assert_close(value, a[key], atol=0, rtol=0, msg=key)
    print("[train] bf16 pruning", file=sys.stderr, flush=True)
    run_train(write_config(tmp_path, "pruned", precision="bf16", save_steps=1, max_steps=3,
                           save_total_limit=1))
    assert sorted(p.name for p in (tmp_path / "pruned").glob("checkpoint-*")) == ["checkpoint-3"]


def test_gradient_accumulation_follows_reference_loop(tmp_path):
    """Accumulation over 2 packs, 2 epochs of 5 packs (alodlm/train.py:50-54,
    134-150): the horizon, the sync at the end of each epoch's loader (the odd
    last pack steps alone), learning rates, and each checkpoint's step, epoch
    and next batch equal the reference's.  The second epoch's order is not
    compared: on the CPU the reference's masking draws advance the CPU
    generator, on a GPU they use the device's."""
    ref = RUN["accumulated"]
    shutil.copy(FIXTURE / "training.jsonl", tmp_path / "training.jsonl")
    consumed = []
    print("[train] accumulation run", file=sys.stderr, flush=True)
    steps = run_train(write_config(tmp_path, "acc", gradient_accumulation_steps=2, max_steps=0),
                      consumed)
    assert steps == ref["steps"] == 6
    assert consumed[:5] == ref["consumed"][:5]
    assert len(consumed) == 10
    records = [json.loads(l) for l in (tmp_path / "acc" / "metrics.jsonl").read_text().splitlines()]
    assert [r["step"] for r in records] == [r["step"] for r in ref["metrics"]]
    for got, want in zip(records, ref["metrics"]):
        assert got["learning_rate"] == pytest.approx(want["learning_rate"], rel=1e-12, abs=1e-18)
    for name, want in ref["checkpoints"].items():
        state = json.loads((tmp_path / "acc" / name / "trainer_state.json").read_text())
        for key in ("step", "epoch", "next_batch", "identity"):
            assert state[key] == want["trainer_state"][key], (name, key)
    first = json.loads((tmp_path / "acc" / "checkpoint-2" / "trainer_state.json").read_text())
    assert first["epoch_rng"] == ref["checkpoints"]["checkpoint-2"]["trainer_state"]["epoch_rng"]
