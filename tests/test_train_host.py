"""Host side of the training loop (alodlm/train.py) without a GPU: horizon,
schedule, run identity, pack order, checkpoint pruning and the training-state
round trip, against a recorded run of the reference on the workflow fixture."""

import json
import random

import numpy as np
import pytest
import torch

from tests.golden import HERE as GOLDEN

# the schedule is stepped without optimizer steps here
pytestmark = pytest.mark.filterwarnings("ignore:Detected call of `lr_scheduler.step")

RUN = json.loads((GOLDEN / "workflow" / "train.json").read_text())
FIXTURE = GOLDEN / "workflow" / "fixture"


def fixture_config(tmp_path, **overrides):
    from alodlm_amd.config import ModelConfig, TrainConfig
    values = dict(RUN["config"])
    values.update(model_dir=str(FIXTURE / "base"), train_file=str(tmp_path / "training.jsonl"),
                  output_dir=str(tmp_path / "run"), cache_file=str(tmp_path / "packed.pt"))
    values.update(overrides)
    values["model"] = ModelConfig(**values["model"])
    return TrainConfig(**values)


def test_horizon():
    """steps = ceil(packs / gas) per epoch, times epochs, capped by max_steps
    (alodlm/train.py:50-54); the fixture run has 5 packs, 2 epochs, cap 4."""
    from alodlm_amd.train import training_horizon
    assert training_horizon(5, 1, 2, 4) == RUN["run"]["header"]["training_steps"] == 4
    assert training_horizon(5, 1, 2, 0) == 10
    assert training_horizon(5, 2, 2, 0) == 6
    assert training_horizon(7, 3, 1, 0) == 3
    assert training_horizon(7, 3, 1, 2) == 2


def test_schedule_matches_reference_run(tmp_path):
    """The learning rate logged after each step equals the reference's."""
    from alodlm_amd.optim import FusedAdamW
    from alodlm_amd.train import cosine_schedule
    cfg = fixture_config(tmp_path)
    p = torch.nn.Parameter(torch.zeros(4))
    opt = FusedAdamW([{"params": [p], "weight_decay": 0.0}], lr=cfg.learning_rate)
    sched = cosine_schedule(opt, 4, cfg.warmup_ratio)
    assert opt.param_groups[0]["lr"] == cfg.learning_rate
    for record in RUN["run"]["metrics"]:
        sched.step()
        assert sched.get_last_lr()[0] == pytest.approx(record["learning_rate"], rel=1e-12, abs=1e-18)
    # warmup: int(20 * 0.25) = 5 steps from 0
    opt2 = FusedAdamW([{"params": [p], "weight_decay": 0.0}], lr=1.0)
    sched2 = cosine_schedule(opt2, 20, 0.25)
    lrs = [opt2.param_groups[0]["lr"]]
    for _ in range(20):
        sched2.step()
        lrs.append(opt2.param_groups[0]["lr"])
    assert lrs[:6] == pytest.approx([0.0, 0.2, 0.4, 0.6, 0.8, 1.0])
    assert lrs[20] == pytest.approx(0.0, abs=1e-12)


def test_identity_matches_reference(tmp_path):
    """The resume identity equals the one the reference wrote."""
    from alodlm_amd.train import run_identity
    want = RUN["run"]["checkpoints"]["checkpoint-2"]["trainer_state"]["identity"]
    got = run_identity(fixture_config(tmp_path), want["cache_identity"], 4)
    assert got == want
    other = run_identity(fixture_config(tmp_path, learning_rate=2e-5), want["cache_identity"], 4)
    assert other != want
    # paths do not enter the identity
    moved = run_identity(fixture_config(tmp_path, output_dir="/elsewhere", resume="x"),
                         want["cache_identity"], 4)
    assert moved == want


def test_pack_order_matches_reference():
    """From the CPU generator state the reference recorded at the start of
    the epoch, the loader yields the reference's packs in its order, and the
    resumed loader (2 packs skipped) continues with the same order."""
    from alodlm_amd.train import pack_loader

    class Indices(torch.utils.data.Dataset):
        def __len__(self):
            return 5

        def __getitem__(self, i):
            return {"index": i}

    epoch_rng = RUN["run"]["checkpoints"]["checkpoint-2"]["trainer_state"]["epoch_rng"]
    assert epoch_rng["sampler"] is None
    state = torch.tensor(epoch_rng["cpu"], dtype=torch.uint8)
    saved = torch.get_rng_state()
    try:
        torch.set_rng_state(state)
        order = [item["index"] for item in pack_loader(Indices())]
        assert order[:4] == RUN["run"]["consumed"][:4]
        torch.set_rng_state(state)
        resumed = [item["index"] for item in pack_loader(Indices(), skip=2)]
        assert resumed == order[2:]
        assert resumed[:2] == RUN["resumed"]["consumed"][:2]
    finally:
        torch.set_rng_state(saved)


def test_prune_checkpoints(tmp_path):
    """Only completed checkpoint-<n> directories count; the newest are kept."""
    from alodlm_amd.train import completed_checkpoints, prune_checkpoints
    for n in (2, 10, 4, 6):
        d = tmp_path / f"checkpoint-{n}"
        d.mkdir()
        (d / "trainer_state.json").write_text("{}")
    (tmp_path / "checkpoint-8").mkdir()  # incomplete
    (tmp_path / "checkpoint-x").mkdir()
    (tmp_path / "checkpoint-12").symlink_to(tmp_path / "checkpoint-10")
    assert [p.name for p in completed_checkpoints(tmp_path)] == [
        "checkpoint-2", "checkpoint-4", "checkpoint-6", "checkpoint-10"]
    prune_checkpoints(tmp_path, 2)
    assert sorted(p.name for p in tmp_path.iterdir()) == [
        "checkpoint-10", "checkpoint-12", "checkpoint-6", "checkpoint-8", "checkpoint-x"]


def test_training_state_round_trip(tmp_path):
    """Optimizer masters and moments stay float32 for bf16 parameters, step
    counts, schedule and every generator are restored."""
    from alodlm_amd.optim import FusedAdamW
    from alodlm_amd.train import cosine_schedule, load_training_state, save_training_state

    def make():
        model = torch.nn.Module()
        model.a = torch.nn.Parameter(torch.randn(3, 5).to(torch.bfloat16))
        model.bias = torch.nn.Parameter(torch.randn(7).to(torch.bfloat16))
        opt = FusedAdamW([{"params": [model.a], "weight_decay": 0.01},
                          {"params": [model.bias], "weight_decay": 0.0}], lr=1e-3)
        return model, opt, cosine_schedule(opt, 10, 0.2)

    model, opt, sched = make()
    for p in (model.a, model.bias):
        opt.state[p] = {"step": 3, "master": torch.randn(p.shape, dtype=torch.float64).float(),
                        "exp_avg": torch.randn(p.shape), "exp_avg_sq": torch.rand(p.shape)}
    for _ in range(3):
        sched.step()
    random.seed(5)
    np.random.seed(6)
    torch.manual_seed(7)
    save_training_state(tmp_path / "state", model, opt, sched)
    expect = (random.random(), np.random.rand(), torch.rand(1).item())
    model2, opt2, sched2 = make()
    load_training_state(tmp_path / "state", model2, opt2, sched2)
    for p, q in ((model.a, model2.a), (model.bias, model2.bias)):
        for key in ("master", "exp_avg", "exp_avg_sq"):
            assert opt2.state[q][key].dtype == torch.float32
            assert torch.equal(opt2.state[q][key], opt.state[p][key])
        assert opt2.state[q]["step"] == 3
    assert opt2.param_groups[0]["lr"] == opt.param_groups[0]["lr"]
    assert opt2.param_groups[1]["weight_decay"] == 0.0
    assert opt2.param_groups[0]["betas"] == (0.9, 0.999)
    sched.step()
    sched2.step()
    assert sched2.get_last_lr() == sched.get_last_lr()
    assert (random.random(), np.random.rand(), torch.rand(1).item()) == expect
    files = sorted(p.name for p in (tmp_path / "state").iterdir())
    assert files == sorted(p.name for p in (REFERENCE_CHECKPOINT / "training_state").iterdir())


REFERENCE_CHECKPOINT = GOLDEN / "workflow" / "reference_checkpoint-2"


def _reference_side(model):
    """The reference's optimizer and scheduler over ``model``
    (alodlm/train.py:42-56): torch.optim.AdamW over the two decay groups and
    transformers' cosine schedule with warmup."""
    from transformers import get_cosine_schedule_with_warmup
    no_decay = ("bias", "LayerNorm.weight", "layer_norm.weight")
    groups = [
        {"params": [p for n, p in model.named_parameters() if not any(s in n for s in no_decay)],
         "weight_decay": 0.01},
        {"params": [p for n, p in model.named_parameters() if any(s in n for s in no_decay)],
         "weight_decay": 0.0},
    ]
    optimizer = torch.optim.AdamW(groups, lr=1e-5)
    return optimizer, get_cosine_schedule_with_warmup(optimizer, 0, 4)


def test_reference_training_state_loads():
    """A training state the reference wrote through accelerate (checkpoint-2
    of its recorded run) restores into this implementation: moments and step
    counts equal the reference's, float32 masters are the parameters, the
    schedule continues from the same learning rate, the generators and
    accelerate's step counter are the reference's."""
    from alodlm_amd.model import ALoDLM
    from alodlm_amd.optim import FusedAdamW, param_groups
    from alodlm_amd.train import _safe_load, cosine_schedule, load_training_state
    state_dir = REFERENCE_CHECKPOINT / "training_state"
    model = ALoDLM.from_pretrained(REFERENCE_CHECKPOINT)
    opt = FusedAdamW(param_groups(model, 0.01), lr=1e-5, max_grad_norm=1.0)
    sched = cosine_schedule(opt, RUN["run"]["steps"], 0.03)  # the fixture run's warmup ratio
    position = load_training_state(state_dir, model, opt, sched)
    ref = _safe_load(state_dir / "optimizer.bin")
    params = [p for g in opt.param_groups for p in g["params"]]
    assert len(params) == len(ref["state"])
    for index, p in enumerate(params):
        entry = ref["state"][index]
        assert opt.state[p]["step"] == int(entry["step"]) == 2
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(opt.state[p][key], entry[key].float())
        assert torch.equal(opt.state[p]["master"], p.detach().float())
    assert [g["lr"] for g in opt.param_groups] == [g["lr"] for g in ref["param_groups"]]
    assert sched.get_last_lr() == _safe_load(state_dir / "custom_checkpoint_0.pkl")["_last_lr"]
    rng = _safe_load(state_dir / "random_states_0.pkl")
    assert torch.equal(torch.get_rng_state(), rng["torch_manual_seed"])
    assert random.getstate() == rng["random_state"]
    assert position == 2


def test_training_state_restores_into_the_reference(tmp_path):
    """A training state written here restores through accelerate's own
    loaders into the reference's objects (model, torch.optim.AdamW, the
    registered scheduler): weights, moments, step counts, learning rates and
    generators."""
    from accelerate import PartialState
    from accelerate.checkpointing import load_accelerator_state, load_custom_state
    PartialState(cpu=True)  # accelerate's loaders log through its process state
    from alodlm_amd.model import ALoDLM
    from alodlm_amd.optim import FusedAdamW, param_groups
    from alodlm_amd.train import cosine_schedule, save_training_state
    model = ALoDLM.from_pretrained(REFERENCE_CHECKPOINT)
    opt = FusedAdamW(param_groups(model, 0.01), lr=1e-5, max_grad_norm=1.0)
    sched = cosine_schedule(opt, 4, 0.0)
    g = torch.Generator().manual_seed(3)
    for p in model.parameters():
        opt.state[p] = {"step": 2, "master": p.detach().float().clone(),
                        "exp_avg": torch.randn(p.shape, generator=g),
                        "exp_avg_sq": torch.rand(p.shape, generator=g)}
    for _ in range(2):
        sched.step()
    torch.manual_seed(11)
    save_training_state(tmp_path / "state", model, opt, sched, loader_position=2)
    expect = torch.rand(3)

    target = ALoDLM.from_pretrained(REFERENCE_CHECKPOINT)
    with torch.no_grad():
        for p in target.parameters():
            p.zero_()
    ref_opt, ref_sched = _reference_side(target)
    torch.manual_seed(0)
    load_accelerator_state(str(tmp_path / "state"), [target], [ref_opt], [], [], 0)
    load_custom_state(ref_sched, str(tmp_path / "state"), 0)
    for (name, p), q in zip(model.named_parameters(), target.parameters()):
        assert torch.equal(p.detach(), q.detach()), name
        entry = ref_opt.state[q]
        assert int(entry["step"]) == 2
        assert torch.equal(entry["exp_avg"], opt.state[p]["exp_avg"])
        assert torch.equal(entry["exp_avg_sq"], opt.state[p]["exp_avg_sq"])
    assert ref_sched.get_last_lr() == sched.get_last_lr()
    assert [g["lr"] for g in ref_opt.param_groups] == [g["lr"] for g in opt.param_groups]
    assert torch.equal(torch.rand(3), expect)
    # the saved groups carry the keys of the reference's own accelerate-saved
    # optimizer state (initial_lr included), so a scheduler built later with
    # last_epoch >= 0 finds its base rates
    ours = torch.load(tmp_path / "state" / "optimizer.bin", weights_only=True)["param_groups"]
    theirs = torch.load(REFERENCE_CHECKPOINT / "training_state" / "optimizer.bin",
                        weights_only=True)["param_groups"]
    assert [set(g) for g in ours] == [set(g) for g in theirs]
    assert [g["initial_lr"] for g in ref_opt.param_groups] == [1e-5, 1e-5]


def test_train_needs_gpu(tmp_path):
    from alodlm_amd.train import train
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="GPU"):
        train(fixture_config(tmp_path))


def test_config_errors(tmp_path):
    """TrainConfig.load rejects what the reference rejects (alodlm/config.py:82-102)."""
    import yaml
    from alodlm_amd.config import TrainConfig
    base = dict(RUN["config"], model_dir="m", train_file="t", output_dir="o", cache_file="c")
    path = tmp_path / "c.yaml"
    path.write_text(yaml.safe_dump(base))
    assert TrainConfig.load(path).max_steps == 4
    for change in ({"bogus": 1}, {"warmup_ratio": 1.0}, {"precision": "fp16"},
                   {"learning_rate": 0.0}, {"save_steps": 0}, {"max_steps": -1}):
        path.write_text(yaml.safe_dump(dict(base, **change)))
        with pytest.raises(ValueError):
            TrainConfig.load(path)


class _FakeProps:
    total_memory = 100 * 2**30


def _engine_for_keep(monkeypatch, alloc, peak, fused_state):
    """A StepEngine shell for the keep decision with mocked memory figures
    (GiB): `alloc` is what memory_allocated reports at each call, `peak` the
    first step's peak."""
    import types
    from alodlm_amd import engine as E
    e = E.StepEngine.__new__(E.StepEngine)
    e.dims = E.Dims(hidden=1024, heads=8, kv_heads=4, head_dim=128, intermediate=4096, vocab=1000,
                    layers=4, eps=1e-6, theta=1e6)
    e.cfg = types.SimpleNamespace(loop_start=0, max_depth=4)
    e.dtype, e.device = __import__("torch").bfloat16, "cuda:0"
    e.arena = types.SimpleNamespace(params=[types.SimpleNamespace(numel=lambda: 2**30)])
    e.grads = None
    e.fused_optimizer = (None if fused_state is None else
                         types.SimpleNamespace(state_bytes_to_come=lambda: fused_state * 2**30))
    e._keep, e._keep_rows, e._step_alloc, e._step_peak = None, 0, None, None
    values = iter(alloc)
    last = {"bytes": 0}

    def allocated(dev=None):
        last["bytes"] = next(values) * 2**30
        return last["bytes"]

    # a 100 GiB device that this process alone uses, with no cached blocks
    monkeypatch.setattr("torch.cuda.memory_allocated", allocated)
    monkeypatch.setattr("torch.cuda.memory_reserved", lambda dev=None: last["bytes"])
    monkeypatch.setattr("torch.cuda.mem_get_info",
                        lambda dev=None: (100 * 2**30 - last["bytes"], 100 * 2**30))
    monkeypatch.setattr("torch.cuda.max_memory_allocated", lambda dev=None: peak * 2**30)
    monkeypatch.setattr("torch.cuda.reset_peak_memory_stats", lambda dev=None: None)
    monkeypatch.setattr("torch.cuda.get_device_properties", lambda dev=None: _FakeProps())
    return e


def test_keep_decision_counts_optimizer_state_not_yet_allocated(monkeypatch):
    """The keep decision at the second forward of an accumulated step (before
    any optimizer step) adds the bound FusedAdamW's state still to come; a
    decision after the first optimizer step has none to add.  With N = 262144
    rows and 16 layer applications the rotary q/k take 12 GiB and the norm
    outputs 16 GiB; the budget is 94 GiB (a 6 % margin of the 100 GiB
    device)."""
    N = 262144
    # first forward: 20 GiB allocated; the step peaks at 50 GiB (growth 30)
    e = _engine_for_keep(monkeypatch, [20, 20], 50, fused_state=30)
    assert e._decide_keep(N) == (False, False)
    e._step_peak = 50 * 2**30
    # 30 GiB of optimizer state to come: 20 + 30 + 30 = 80, so q/k (92) fit
    # and the norm outputs (108) do not; without counting it both would
    assert e._decide_keep(N) == (True, False)
    # the same decision once the state exists: 50 GiB allocated, nothing to come
    e2 = _engine_for_keep(monkeypatch, [20, 50], 50, fused_state=0)
    e2._decide_keep(N)
    e2._step_peak = 50 * 2**30
    assert e2._decide_keep(N) == (True, False)
    # a smaller pack keeps both: 80 + 6 + 8 <= 94
    e3 = _engine_for_keep(monkeypatch, [20, 20], 50, fused_state=30)
    e3._decide_keep(N // 2)
    e3._step_peak = 50 * 2**30
    assert e3._decide_keep(N // 2) == (True, True)


def test_keep_decision_without_fused_optimizer_reserves_adam_state(monkeypatch):
    """With no FusedAdamW bound the decision reserves AdamW's float32 master and
    moments (12 bytes per parameter: 12 GiB for 2^30 parameters): 20 + 30 + 12
    = 62 GiB, so q/k (74) and the norm outputs (90) fit at N = 262144; at three
    times the rows q/k alone (98) do not."""
    e = _engine_for_keep(monkeypatch, [20, 20], 50, fused_state=None)
    e._decide_keep(262144)
    e._step_peak = 50 * 2**30
    assert e._decide_keep(262144) == (True, True)
    e = _engine_for_keep(monkeypatch, [20, 20], 50, fused_state=None)
    e._decide_keep(3 * 262144)
    e._step_peak = 50 * 2**30
    assert e._decide_keep(3 * 262144) == (False, False)
