"""Recurrent Qwen3 ALoDLM (drop-in for alodlm/model.py).

``ALoDLM(backbone, config)`` wraps a transformers ``Qwen3ForCausalLM`` exactly
like the reference (same submodule names, so ``state_dict`` keys and the
checkpoint layout are unchanged).  ``forward(ids, labels, boundaries)`` runs
the whole training step - batch building, rollout over the recurrent depths,
cross-entropies and the objective - on the gfx950 HIP kernels through
``StepEngine`` and returns ``(loss, metrics)``; ``loss.backward()`` runs the
hand-scheduled backward and fills every parameter's ``.grad``.

The reference's layer functions are defined here as in alodlm/model.py:41-80:
``rotary``, ``layer_forward`` (also the decoder's layer call) and
``training_layer``, each on the layer kernels of ``alodlm_amd.layers``.
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
from .layers import (LayerWeights, Rope, WindowMask, WindowSlot, _LayerFunction, _Rotary,
                     _check_device, _kernel_mask, _kernels_for, table)


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


def rotary(q, k, cos, sin):
    """q * cos + rotate_half(q) * sin and the same for k (alodlm/model.py:41-46),
    one kernel launch per tensor.

    q [L, nq, dh] and k [L, nkv, dh] share rows, head_dim, dtype and device;
    cos, sin are [L, dh] (or [1, L, dh]) and are used in q's dtype.
    Differentiable in q and k.  Other shapes raise ValueError (the
    reference's broadcasting error)."""
    if q.ndim != 3 or k.ndim != 3:
        raise ValueError("rotary takes q [rows, heads, head_dim] and k [rows, kv_heads, head_dim]")
    L, _, dh = q.shape
    if k.shape[0] != L or k.shape[2] != dh:
        raise ValueError(f"k {tuple(k.shape)} must have q's rows and head_dim ({L}, {dh})")
    if k.dtype != q.dtype or k.device != q.device:
        raise ValueError("q and k must share dtype and device")
    if dh % 2:
        raise ValueError("head_dim must be even for the rotary embedding")
    cos, sin = table(cos, L, dh, q), table(sin, L, dh, q)
    _check_device(q, "rotary")
    return _Rotary.apply(q, k, cos, sin)


def layer_forward(layer, hidden, cos, sin, mask, prefix=None):
    """Apply one decoder layer and return ``(hidden, (k, v))`` with the current
    rows' rotated keys and values [L, kv_heads, head_dim] (alodlm/model.py:49-76).

    ``layer`` is a transformers Qwen3 decoder layer, ``hidden`` [L, H], cos/sin
    [L, head_dim], ``mask`` one of the forms ``alodlm_amd.layers`` lists.
    ``prefix`` = (k, v) of cached rows [P, kv_heads, head_dim] runs the decoding
    window, whose mask must then be the prefix + causal window mask; that
    form (also without a prefix: the causal mask) runs without autograd.
    ``prefix`` may also be a ``layers.WindowSlot`` (what the decoder passes):
    the window's keys and values are then written in place after the cached
    rows.  Under the dual-stream mask the output is differentiable in
    ``hidden`` and the layer's parameters; the returned k, v carry no autograd
    history."""
    if isinstance(prefix, WindowSlot):
        _check_device(hidden, "layer_forward")
        return prefix.run(layer, hidden, cos, sin)
    kernels = _kernels_for(layer, hidden)
    d = kernels.dims
    if hidden.ndim != 2 or hidden.shape[1] != layer.input_layernorm.weight.shape[0]:
        raise ValueError(f"hidden must be [rows, {layer.input_layernorm.weight.shape[0]}]")
    L = hidden.shape[0]
    rope = Rope(cos=table(cos, L, d.head_dim, hidden), sin=table(sin, L, d.head_dim, hidden))
    _check_device(hidden, "layer_forward")
    kind = _kernel_mask(mask, L, hidden.device)
    if prefix is None and not (isinstance(kind, tuple) and kind[0] == "window"):
        y, k, v = _LayerFunction.apply(kernels, kind, rope, hidden,
                                       *LayerWeights.module_tensors(layer))
        return y, (k, v)
    P = kind[1] if isinstance(kind, tuple) else None
    if P is None:
        raise ValueError("a prefix cache needs the prefix + causal window mask")
    if prefix is None:
        prefix_k = prefix_v = hidden.new_empty(0, d.kv_heads, d.head_dim)
    else:
        prefix_k, prefix_v = prefix
    if prefix_k.shape[0] != P or prefix_v.shape[0] != P:
        raise ValueError(f"the mask allows {P} prefix keys but the cache holds {prefix_k.shape[0]}")
    KD = d.kv_heads * d.head_dim
    if prefix_k.numel() != P * KD or prefix_v.numel() != P * KD:
        raise ValueError(f"cached keys and values must be [{P}, {d.kv_heads}, {d.head_dim}]")
    params = LayerWeights.module_tensors(layer)
    if torch.is_grad_enabled() and (hidden.requires_grad or any(p.requires_grad for p in params)):
        raise RuntimeError("layer_forward under the decoding window mask runs without autograd; "
                           "wrap the call in torch.no_grad() (training takes the dual-stream "
                           "mask)")
    kbuf = hidden.new_empty(P + L, KD)
    vbuf = hidden.new_empty(P + L, KD)
    kbuf[:P].copy_(prefix_k.reshape(P, KD))
    vbuf[:P].copy_(prefix_v.reshape(P, KD))
    tiled = hidden.dtype == torch.bfloat16 and d.head_dim in (64, 128)
    window = WindowMask(P, L, tiled, hidden.device)
    with torch.no_grad():
        w = LayerWeights.from_tensors(*params)
        y = kernels.layer_window(w, hidden.detach().contiguous(), rope, window, kbuf, vbuf)
    return y, (kbuf[P:].view(L, d.kv_heads, d.head_dim), vbuf[P:].view(L, d.kv_heads, d.head_dim))


def training_layer(layer, hidden, cos, sin, mask):
    """The layer output alone (alodlm/model.py:79-80)."""
    return layer_forward(layer, hidden, cos, sin, mask)[0]


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
            # the upstream gradient (a device scalar, never read on the host)
            # scales the LM head's and the gate's gradients and the readout
            # gradient that every other gradient is linear in
            engine.backward(state, grad_loss, accumulate=engine.grads_pending)
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

    def zero_grad(self, set_to_none=True):
        """Clear the gradients: every parameter's ``.grad`` and, with a bound
        FusedAdamW, the float32 gradients of the step's arena (the next
        backward writes them afresh instead of accumulating)."""
        super().zero_grad(set_to_none)
        if self._engine is not None:
            self._engine.grads_pending = False

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
