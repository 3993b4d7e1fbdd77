"""Recurrent Qwen3 ALoDLM (drop-in for alodlm/model.py).

``ALoDLM(backbone, config)`` wraps a transformers ``Qwen3ForCausalLM`` exactly
like the reference (same submodule names, so ``state_dict`` keys and the
checkpoint layout are unchanged).  ``forward(ids, labels, boundaries)`` runs
the whole training step - batch building, rollout over the recurrent depths,
cross-entropies and the objective - on the gfx950 HIP kernels through
``StepEngine`` and returns ``(loss, metrics)``; ``loss.backward()`` runs the
hand-scheduled backward and fills every parameter's ``.grad``.
"""

import json
import math
import weakref
from dataclasses import asdict
from pathlib import Path

import torch
import torch.nn as nn

from . import _lib
from .config import ModelConfig, local_dir
from .engine import METRIC_NAMES, StepEngine


class GateHead(nn.Module):
    """Halting gate: a shared linear readout plus one bias per depth
    (alodlm/model.py:22-38).  A fresh gate has zero weights and depth biases
    equal to the logits of the conditional hazards mass/survival, the last
    depth being forced."""

    def __init__(self, hidden_size, initial_mass):
        super().__init__()
        self.net = nn.Linear(hidden_size, 1)
        nn.init.zeros_(self.net.weight)
        nn.init.zeros_(self.net.bias)
        biases, survival = [], 1.0
        for mass in initial_mass[:-1]:
            hazard = mass / survival
            biases.append(math.log(hazard / (1 - hazard)))
            survival *= 1 - hazard
        self.depth_bias = nn.Parameter(torch.tensor(biases + [0.0], dtype=torch.float32))

    def forward(self, features, depth):
        return self.net(features).squeeze(-1) + self.depth_bias[depth]


class _Step(torch.autograd.Function):
    """One autograd node for the whole step; inputs are the arena parameters.

    The backward fills the engine's float32 gradient arena.  With a bound
    FusedAdamW (``engine.fused_optimizer``) the parameters' ``.grad`` stay
    unset: the optimizer reads the float32 arena itself (no rounding to the
    parameter dtype, no second arena; ``ALoDLM.materialize_grads`` fills
    ``.grad`` on request) and consecutive backward calls accumulate there.
    Otherwise the gradients are handed to autograd in the parameter dtype."""

    @staticmethod
    def forward(ctx, engine, inputs, need_grad, *params):
        ids, labels, boundaries, extra = inputs
        out, state = engine.forward(ids, labels, boundaries, need_grad, **extra)
        ctx.engine = engine
        ctx.state = state if need_grad else None
        ctx.nparams = len(params)
        metrics = out[1:].clone()
        ctx.mark_non_differentiable(metrics)
        return out[0].clone(), metrics

    @staticmethod
    def backward(ctx, grad_loss, grad_metrics):
        engine, state = ctx.engine, ctx.state
        if state is None:
            raise RuntimeError("the step was run without gradient tracking")
        ctx.state = None
        if engine.fused_optimizer is not None:
            # the upstream gradient scales the LM head and gate products
            # (everything else is linear in them); one read of the scalar
            engine.backward(state, float(grad_loss), accumulate=engine.grads_pending)
            del state
            engine.grads_pending = True
            engine.note_step_peak()
            return (None, None, None, *([None] * ctx.nparams))
        # The backward is linear in the loss's upstream gradient: it runs for a
        # unit seed and the seed (a device scalar, never read on the host, so
        # the host does not wait for the forward here) scales the result while
        # it is cast to the parameter dtype.
        seed = grad_loss.detach().to(device=engine.device, dtype=torch.float32).reshape(1)
        grads = engine.backward(state, 1.0)
        del state
        flat = torch.empty(engine.arena.total, dtype=engine.dtype, device=engine.device)
        _lib.call("alodlm_cast_f32", _lib.ptr(grads), _lib.ptr(seed), _lib.ptr(flat),
                  grads.numel(), engine.code, _lib.stream_handle(engine.device))
        engine.note_step_peak()
        views = [engine.arena.view(flat, name) for name in engine.arena.names]
        return (None, None, None, *views)


_MODELS = weakref.WeakSet()


def model_of(params):
    """The ALoDLM whose parameters are exactly ``params`` (by identity), or None."""
    ids = {id(p) for p in params}
    for model in list(_MODELS):
        mine = list(model.parameters())
        if len(mine) == len(ids) and all(id(p) in ids for p in mine):
            return model
    return None


class ALoDLM(nn.Module):
    def __init__(self, backbone, config):
        super().__init__()
        config.validate(backbone)
        self.backbone = backbone
        self.config = config
        self.exit_gate = GateHead(backbone.config.hidden_size, config.gate_init_pi)
        self.exit_gate.to(dtype=backbone.dtype, device=backbone.device)
        self._engine = None
        self._fused_optimizer = None
        _MODELS.add(self)

    @classmethod
    def from_pretrained(cls, directory, config=None, dtype=torch.float32, require_gate=True):
        """Load a checkpoint directory (alodlm/model.py:94-114)."""
        from transformers import AutoModelForCausalLM
        path = local_dir(directory)
        metadata = path / "alodlm_config.json"
        if config is None:
            if not metadata.is_file():
                raise ValueError("Checkpoint requires alodlm_config.json or an explicit ModelConfig")
            config = ModelConfig(**json.loads(metadata.read_text()))
        backbone = AutoModelForCausalLM.from_pretrained(
            str(path), local_files_only=True, trust_remote_code=False, dtype=dtype,
            attn_implementation="eager")
        model = cls(backbone, config)
        gate_file = path / "exit_gate.pt"
        if gate_file.is_file():
            model.exit_gate.load_state_dict(
                torch.load(gate_file, map_location="cpu", weights_only=True), strict=True)
        elif require_gate:
            raise ValueError("Adaptive inference requires trained exit_gate.pt weights")
        return model

    def save_pretrained(self, directory, state_dict=None):
        """HF backbone files, exit_gate.pt and alodlm_config.json (alodlm/model.py:116-128)."""
        path = Path(directory)
        path.mkdir(parents=True, exist_ok=True)
        state = state_dict if state_dict is not None else self.state_dict()
        # Parameters are views of one device arena: each tensor is copied to
        # host memory of its own, so that neither safetensors nor torch.save
        # sees (or writes) the shared storage.
        state = {k: v.detach().to("cpu", copy=True) for k, v in state.items()}
        backbone = {k[len("backbone."):]: v for k, v in state.items() if k.startswith("backbone.")}
        gate = {k[len("exit_gate."):]: v for k, v in state.items() if k.startswith("exit_gate.")}
        self.backbone.config._name_or_path = ""
        self.backbone.save_pretrained(path, state_dict=backbone, safe_serialization=True)
        torch.save(gate, path / "exit_gate.pt")
        (path / "alodlm_config.json").write_text(json.dumps(asdict(self.config), indent=2) + "\n")

    def rollout(self, batch, generator=None, exit_uniforms=None):
        """Sample commitments and return per-depth logits, gates and exits
        (alodlm/model.py:130-169), each operation a differentiable kernel
        launch (see ``alodlm_amd.rollout``)."""
        from .rollout import rollout
        return rollout(self, batch, generator=generator, exit_uniforms=exit_uniforms)

    def engine(self):
        """The step engine bound to the current parameter storage."""
        if self._engine is not None and not self._engine.arena.valid():
            if self._fused_optimizer is not None:
                raise RuntimeError("the model's parameters were moved after a FusedAdamW was "
                                   "bound to them; build the optimizer after moving the model")
            self._engine = None
        if self._engine is None:
            self._engine = StepEngine(self)
            self._engine.fused_optimizer = self._fused_optimizer
        return self._engine

    def bind_optimizer(self, optimizer):
        """Let ``optimizer`` (a FusedAdamW over exactly this model's
        parameters) read the step's float32 gradients directly; called by
        FusedAdamW itself."""
        self._fused_optimizer = optimizer
        if self._engine is not None:
            self._engine.fused_optimizer = optimizer

    def float32_grads(self):
        """name -> float32 gradient of the last backward(s) since zero_grad when
        a FusedAdamW reads them from the step's arena, else None."""
        e = self._engine
        if e is None or e.fused_optimizer is None or not e.grads_pending:
            return None
        return {name: e.arena.view(e.grads, name) for name in e.arena.names}

    def materialize_grads(self):
        """Fill every parameter's ``.grad`` (parameter dtype) from the float32
        gradients a bound FusedAdamW reads, for code that inspects ``.grad``;
        a no-op when autograd already filled them."""
        grads = self.float32_grads()
        if grads is None:
            return
        named = dict(self.named_parameters())
        for name, g in grads.items():
            named[name].grad = g.to(named[name].dtype)

    def forward(self, ids, labels, boundaries, exit_uniforms=None, draws=None, generator=None):
        """The training step's forward (alodlm/model.py:171-187).

        Returns ``(loss, metrics)``; ``loss.backward()`` fills parameter grads.
        ``exit_uniforms`` / ``draws`` replay known randomness (tests);
        ``generator`` replaces the device's default generator.
        """
        engine = self.engine()
        params = engine.arena.params
        need_grad = torch.is_grad_enabled() and any(p.requires_grad for p in params)
        extra = {"exit_uniforms": exit_uniforms, "draws": draws, "generator": generator}
        loss, metrics = _Step.apply(engine, (ids, labels, boundaries, extra), need_grad, *params)
        values = dict(zip(METRIC_NAMES + ("ar_loss",), metrics[:8].unbind()))
        values["loss"] = loss.detach()
        return loss, values
