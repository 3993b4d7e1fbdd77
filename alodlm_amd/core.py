"""The shared recurrent core and the fused readout as blocks of their own.

Two stages of the training step that are benchmarked and checked on their
own (alodlm/model.py:147-187):

* ``recurrent_core(model, x0, batch)`` - the core layers [loop_start,
  loop_end) run ``max_depth`` times with shared weights from given hidden
  states, the gate on the final norm of each pass's output, exit sampling,
  and between passes the carry norm or the re-embedding of committed rows
  from the word embedding (the core-block workload: one Qwen3-8B layer, four
  passes).  Returns per-pass outputs, gate logits and exits; differentiable
  in x0 and every parameter the passes read.
* ``fused_readout(model, finals, batch)`` - from the final hidden states of
  each pass: final norm and gate, exit sampling, the LM head over the
  loss-bearing rows, the vocabulary cross-entropy and the objective (the
  readout workload).  Returns the loss and metrics; differentiable in the
  final hidden states and the LM head, final norm and gate.

Both run the step engine's own schedule (``StepEngine.core_forward`` /
``readout_forward``), so the kernels and their order are the fused step's.
"""

import torch

from .batch import Batch
from .engine import METRIC_NAMES


def _param_grads(engine, flat):
    return [engine.arena.view(flat, name).to(engine.dtype) for name in engine.arena.names]


class _RecurrentCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, engine, batch, exit_uniforms, generator, x0, *params):
        outs, gates, exits, state = engine.core_forward(x0, batch, True, exit_uniforms,
                                                        generator)
        ctx.engine, ctx.state, ctx.K = engine, state, len(outs)
        ctx.mark_non_differentiable(exits)
        return (*outs, gates.to(engine.dtype), exits)

    @staticmethod
    def backward(ctx, *grads):
        engine, K = ctx.engine, ctx.K
        douts = [g if g is not None else torch.zeros_like(ctx.state["depths"][i]["core_out"])
                 for i, g in enumerate(grads[:K])]
        dgates = grads[K]
        dx0, flat = engine.core_backward(ctx.state, douts, dgates)
        ctx.state = None
        return (None, None, None, None, dx0, *_param_grads(engine, flat))


def recurrent_core(model, x0, batch, exit_uniforms=None, generator=None):
    """Run the shared recurrent core from hidden states ``x0`` [N, H] (see the
    module docstring).  ``batch`` is a build_batch result over the same N
    dual-stream rows (masks, positions, original tokens).  Returns (outputs:
    max_depth tensors [N, H], gate logits [max_depth, N] in the parameter
    dtype, exits [N] int32)."""
    engine = model.engine()
    result = _RecurrentCore.apply(engine, batch, exit_uniforms, generator, x0,
                                  *engine.arena.params)
    K = model.config.max_depth
    return list(result[:K]), result[K], result[K + 1]


def readout_batch(targets, boundaries, masked, mask_probability):
    """A batch for ``fused_readout`` over N plain rows: ``targets`` int64 [N]
    (the token each masked row must predict), ``boundaries`` int64 [S+1]
    segment offsets over the rows, ``masked`` bool [N] and
    ``mask_probability`` float32 [N] (0 on unmasked rows).  Rows carry no
    autoregressive target."""
    n = targets.numel()
    dev = targets.device
    return Batch(ids=targets, original=targets.to(torch.int64).contiguous(), positions=None,
                 masked=masked.contiguous(),
                 mask_probability=mask_probability.to(torch.float32).contiguous(),
                 boundaries=boundaries.to(device=dev, dtype=torch.int64).contiguous(),
                 attention_mask=None,
                 ar_target=torch.full((n,), -1, dtype=torch.int32, device=dev), ar_count=0)


class _FusedReadout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, engine, batch, exit_uniforms, generator, nfinals, *tensors):
        finals = list(tensors[:nfinals])
        out, state = engine.readout_forward(finals, batch, True, exit_uniforms, generator)
        ctx.engine, ctx.state, ctx.nfinals = engine, state, nfinals
        metrics = out[1:10].clone()
        ctx.mark_non_differentiable(metrics)
        return out[0].clone(), metrics

    @staticmethod
    def backward(ctx, grad_loss, _grad_metrics):
        engine = ctx.engine
        dfinals, flat = engine.readout_backward(ctx.state, float(grad_loss))
        ctx.state = None
        return (None, None, None, None, None, *dfinals, *_param_grads(engine, flat))


def fused_readout(model, finals, batch, exit_uniforms=None, generator=None):
    """Readout and objective from the final hidden states ``finals`` (one
    [N, H] tensor per pass; see the module docstring).  Returns (loss,
    metrics) with the step's metric names and the masked-row count."""
    engine = model.engine()
    loss, metrics = _FusedReadout.apply(engine, batch, exit_uniforms, generator, len(finals),
                                        *finals, *engine.arena.params)
    names = METRIC_NAMES + ("ar_loss", "masked_rows")
    values = dict(zip(names, metrics.unbind()))
    values["loss"] = loss.detach()
    return loss, values
