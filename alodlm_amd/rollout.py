"""``ALoDLM.rollout`` composed from differentiable HIP operations (drop-in for
alodlm/model.py:130-169).

``rollout(model, batch)`` returns the reference's ``(logits, gates, exits)``:
per depth the [N, V] LM-head logits and the [N] gate logits (both in the
parameter dtype) and the sampled exits.  Every operation is an autograd node
over the kernels - embedding gather, the decoder layers
(``layers._LayerFunction``), the carry (norm of the core output, or the
embedding of the original token for committed rows), the final norm with the
gate on its detached output, the LM head - so losses built on the outputs
(``loss.outcome_loss``, ``loss.autoregressive_loss``) back-propagate through
the same kernels as the fused step.  ``ALoDLM.forward`` does not use this
path: it runs the fused schedule of ``engine.StepEngine``, which keeps only
the loss-bearing rows' logits.
"""

import torch

from . import _lib
from ._lib import EPI_ACCUM, call, ptr, query
from .layers import DualStreamMask, LayerWeights, Rope, _LayerFunction


def _f32_zeros(*shape, device):
    return torch.zeros(*shape, dtype=torch.float32, device=device)


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, kernels, ids, table):
        N, (V, H) = ids.numel(), table.shape
        out = kernels._empty(N, H)
        call("alodlm_embed_gather", ptr(table), ptr(ids), ptr(out), N, H, V, kernels.code,
             kernels._stream())
        ctx.kernels, ctx.ids, ctx.shape = kernels, ids, table.shape
        return out

    @staticmethod
    def backward(ctx, dout):
        k, (V, H) = ctx.kernels, ctx.shape
        dtable = _f32_zeros(V, H, device=k.device)
        k.embed_scatter(dout.contiguous(), k.embed_plan(ctx.ids), dtable)
        return None, None, dtable.to(k.dtype)


class _CarrySelect(torch.autograd.Function):
    """x_in(d) = exits <= d ? table[original] : norm(core_out(d - 1))
    (alodlm/model.py:150-151,168)."""

    @staticmethod
    def forward(ctx, kernels, depth, original, exits, core_out, wf, table):
        d = kernels.dims
        N, H = core_out.shape
        V = table.shape[0]
        out = kernels._empty(N, H)
        rstd = kernels._empty(N, dtype=torch.float32)
        call("alodlm_carry_select", ptr(core_out), ptr(wf), ptr(table), ptr(original), ptr(exits),
             depth, ptr(out), ptr(rstd), N, H, V, d.eps, kernels.code, kernels._stream())
        ctx.kernels, ctx.depth, ctx.original, ctx.exits = kernels, depth, original, exits
        ctx.save_for_backward(core_out, rstd, wf)
        ctx.vocab = V
        return out

    @staticmethod
    def backward(ctx, dy):
        k = ctx.kernels
        core_out, rstd, wf = ctx.saved_tensors
        N, H = core_out.shape
        V = ctx.vocab
        dx = k._empty(N, H)
        dwf = _f32_zeros(H, device=k.device)
        dtable = _f32_zeros(V, H, device=k.device)
        ws = k._workspace(query("alodlm_carry_select_bwd_workspace", N, H))
        call("alodlm_carry_select_bwd", ptr(dy.contiguous()), ptr(core_out), ptr(rstd), ptr(wf),
             ptr(ctx.exits), ctx.depth, ptr(k.embed_plan(ctx.original)), None, ptr(dx), ptr(dwf),
             ptr(dtable), ptr(ws), N, H, V, k.code, k._stream())
        return None, None, None, None, dx, dwf.to(k.dtype), dtable.to(k.dtype)


class _FinalNormGate(torch.autograd.Function):
    """readout = norm(x) (alodlm/model.py:160) and gate = net(readout.detach())
    + depth_bias[depth] (model.py:37-38,162), one launch; the gate's gradient
    reaches only the gate parameters."""

    @staticmethod
    def forward(ctx, kernels, depth, x, wf, gw, gb, db):
        d = kernels.dims
        N, H = x.shape
        readout = kernels._empty(N, H)
        rstd = kernels._empty(N, dtype=torch.float32)
        gate = kernels._empty(N, dtype=torch.float32)
        call("alodlm_final_norm_gate", ptr(x), ptr(wf), ptr(gw), ptr(gb), ptr(db), depth,
             ptr(readout), ptr(rstd), ptr(gate), N, H, d.eps, kernels.code, kernels._stream())
        ctx.kernels, ctx.depth, ctx.db_len = kernels, depth, db.numel()
        ctx.save_for_backward(x, rstd, wf, readout)
        return readout, gate.to(kernels.dtype)

    @staticmethod
    def backward(ctx, dreadout, dgate):
        k = ctx.kernels
        x, rstd, wf, readout = ctx.saved_tensors
        N, H = x.shape
        dx = dwf = None
        if dreadout is not None:
            dx = k._empty(N, H)
            acc = _f32_zeros(H, device=k.device)
            ws = k._workspace(query("alodlm_rmsnorm_bwd_workspace", N, H))
            call("alodlm_rmsnorm_bwd", ptr(dreadout.contiguous()), ptr(x), ptr(rstd), ptr(wf),
                 None, ptr(dx), ptr(acc), ptr(ws), N, H, k.code, k._stream())
            dwf = acc.to(k.dtype)
        dgw = dgb = ddb = None
        if dgate is not None:
            gw_acc = _f32_zeros(1, H, device=k.device)
            gb_acc = _f32_zeros(1, device=k.device)
            db_acc = _f32_zeros(ctx.db_len, device=k.device)
            g32 = dgate.to(torch.float32).contiguous()
            ws = k._workspace(query("alodlm_gate_bwd_workspace", N, H))
            call("alodlm_gate_bwd", ptr(g32), ptr(readout), 1.0, ptr(gw_acc), ptr(gb_acc),
                 ptr(db_acc), ctx.depth, N, H, ptr(ws), k.code, k._stream())
            dgw, dgb, ddb = gw_acc.to(k.dtype), gb_acc.to(k.dtype), db_acc.to(k.dtype)
        return None, None, dx, dwf, dgw, dgb, ddb


class _LMHead(torch.autograd.Function):
    """logits = x . W^T (alodlm/model.py:161)."""

    @staticmethod
    def forward(ctx, kernels, x, w):
        N, H = x.shape
        V = w.shape[0]
        y = kernels._empty(N, V)
        kernels._gemm(x, H, 1, w, H, 1, y, V, N, V, H)
        ctx.kernels = kernels
        ctx.save_for_backward(x, w)
        return y

    @staticmethod
    def backward(ctx, dy):
        k = ctx.kernels
        x, w = ctx.saved_tensors
        N, H = x.shape
        V = w.shape[0]
        dy = dy.contiguous()
        dx = k._empty(N, H)
        k._gemm(dy, V, 1, w, H, 0, dx, H, N, H, V)
        dw = _f32_zeros(V, H, device=k.device)
        k._gemm(dy, V, 0, x, H, 0, dw, H, V, H, N, epi=EPI_ACCUM)
        return None, dx, dw.to(k.dtype)


def _mask_of(batch, device):
    mask = getattr(batch, "kernel_mask", None)
    if mask is not None:
        return mask
    if isinstance(batch.attention_mask, DualStreamMask):
        return batch.attention_mask
    if isinstance(batch.attention_mask, dict):
        return DualStreamMask.from_plan(batch.attention_mask, device)
    raise ValueError("rollout needs the batch's dual-stream mask (build_batch output)")


def rollout(model, batch, generator=None, exit_uniforms=None):
    """Sample commitments and return per-depth logits, gates and exits
    (alodlm/model.py:130-169) on the kernels.  ``exit_uniforms`` (K - 1
    tensors [N]) replace the ``rand_like`` draws; otherwise they come from
    ``generator`` (default: the device's) in the reference's order."""
    e = model.engine()
    cfg, base = model.config, model.backbone.model
    K, N = cfg.max_depth, batch.ids.numel()
    mask = _mask_of(batch, e.device)
    rope = Rope(positions=batch.positions, inv_freq=e.inv_freq)

    def run(layer, h):
        return _LayerFunction.apply(e, mask, rope, h, *LayerWeights.module_tensors(layer))[0]

    embed = base.embed_tokens.weight
    hidden = _Embedding.apply(e, batch.ids, embed)
    for layer in base.layers[:cfg.loop_start]:
        hidden = run(layer, hidden)
    exits = torch.full((N,), K, dtype=torch.int32, device=e.device)
    masked = batch.masked.contiguous().view(torch.uint8)
    gate = model.exit_gate
    logits, gates = [], []
    core_out = None
    for depth in range(K):
        if depth:
            hidden = _CarrySelect.apply(e, depth, batch.original, exits.clone(), core_out,
                                        base.norm.weight, embed)
        for layer in base.layers[cfg.loop_start:cfg.loop_end]:
            hidden = run(layer, hidden)
        core_out = hidden
        readout = hidden
        for layer in base.layers[cfg.loop_end:]:
            readout = run(layer, readout)
        features, g = _FinalNormGate.apply(e, depth, readout, base.norm.weight, gate.net.weight,
                                           gate.net.bias, gate.depth_bias)
        logits.append(_LMHead.apply(e, features, model.backbone.lm_head.weight))
        gates.append(g)
        if depth < K - 1:
            if exit_uniforms is not None:
                u = exit_uniforms[depth].to(device=e.device, dtype=torch.float32).contiguous()
            else:
                u = torch.rand(N, device=e.device, generator=generator)
            g32 = g.detach().to(torch.float32).contiguous()
            call("alodlm_exit_update", ptr(g32), ptr(u), ptr(masked), ptr(exits), depth, K, N,
                 _lib.stream_handle(e.device))
    return logits, gates, exits.to(torch.int64)
