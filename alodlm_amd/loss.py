"""The training objective's public functions on the HIP kernels (drop-in for
alodlm/loss.py).

``outcome_loss(ce, gate_logits, depths, batch, config)`` returns the NELBO
denoising term plus the sequence score-function actor and the reference's
seven metrics (alodlm/loss.py:35-90); ``autoregressive_loss(logits, labels,
packed_boundaries)`` the count-weighted next-token cross-entropy of each
segment's clean stream (alodlm/loss.py:12-32).  Both are differentiable:
outcome_loss in ``ce`` (through the detached truncated stick) and in the gate
logits (through log q), autoregressive_loss in ``logits``.

The objective kernel accumulates in float32 where the reference's bf16 run
keeps the stick and the denoising sum in bf16; sums run in one workgroup in a
fixed order.
"""

import torch

from . import _lib
from ._lib import call, ptr, query
from .credit import _require_gpu, check_sequence_boundaries

METRIC_KEYS = ("denoising", "actor", "sampled_mean_depth", "prediction_cost",
               "regularization_cost", "profile_mean_depth", "first_pass_halt_probability")


class _OutcomeLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ce, gates, depths, masked, mask_probability, boundaries, config):
        K, N = gates.shape
        dev = gates.device
        rows = torch.nonzero(masked).flatten()
        ce_full = torch.zeros(K, N, dtype=torch.float32, device=dev)
        ce_full[:, rows] = ce.detach().to(torch.float32)
        g32 = gates.detach().to(torch.float32).contiguous()
        exits = depths.to(torch.int32).contiguous()
        mask = masked.contiguous().view(torch.uint8)
        prob = mask_probability.to(torch.float32).contiguous()
        bounds = boundaries.to(torch.int64).contiguous()
        S = bounds.numel() - 1
        out = torch.empty(10, dtype=torch.float32, device=dev)
        dgate = torch.empty(K, N, dtype=torch.float32, device=dev)
        dce = torch.empty(K, N, dtype=torch.float32, device=dev)
        ws = torch.empty(query("alodlm_objective_workspace", N, S, K), dtype=torch.float32,
                         device=dev)
        call("alodlm_outcome_loss", ptr(g32), ptr(exits), ptr(mask), ptr(prob), ptr(ce_full),
             ptr(bounds), S, N, K, float(config.depth_prior_c), float(config.kl_beta_mi),
             float(config.kl_beta_marg), ptr(out), ptr(dgate), ptr(dce), ptr(ws),
             _lib.stream_handle(dev))
        ctx.save_for_backward(dgate, dce[:, rows])
        ctx.dtypes = (ce.dtype, gates.dtype)
        metrics = out[1:8].clone()
        ctx.mark_non_differentiable(metrics)
        return out[1] + out[2], metrics

    @staticmethod
    def backward(ctx, grad, _grad_metrics):
        dgate, dce = ctx.saved_tensors
        g = grad.to(torch.float32)
        ce_dtype, gate_dtype = ctx.dtypes
        return (dce * g).to(ce_dtype), (dgate * g).to(gate_dtype), None, None, None, None, None


def outcome_loss(ce, gate_logits, depths, batch, config):
    """Denoising + actor loss and metrics (alodlm/loss.py:35-90).

    ce [K, M] masked-token cross-entropies, ``gate_logits`` K tensors [N],
    ``depths`` [N] sampled exits in 1..K, ``batch`` with ``masked``,
    ``mask_probability`` and ``boundaries``; ``config`` a ModelConfig."""
    selected = batch.masked
    count = int(selected.sum())
    if count == 0:
        zero = ce.sum() + sum(g.sum() * 0 for g in gate_logits)
        return zero, {key: zero.detach() for key in METRIC_KEYS}
    check_sequence_boundaries(selected, batch.boundaries)
    _require_gpu(ce, "outcome_loss")
    if ce.shape != (config.max_depth, count) or len(gate_logits) != config.max_depth:
        raise ValueError("ce must be [max_depth, masked rows] with one gate tensor per depth")
    loss, metrics = _OutcomeLoss.apply(ce, torch.stack(list(gate_logits)), depths, selected,
                                       batch.mask_probability, batch.boundaries, config)
    return loss, dict(zip(METRIC_KEYS, metrics.unbind()))


class _AutoregressiveLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, rows, targets):
        dev, (N, V) = logits.device, logits.shape
        R = rows.numel()
        code, st = _lib.dtype_code(logits.dtype), _lib.stream_handle(dev)
        sel = rows.to(torch.int32).contiguous()
        buf = torch.empty(R, V, dtype=logits.dtype, device=dev)
        src = logits.detach().contiguous()
        call("alodlm_gather_rows", ptr(src), ptr(sel), R, ptr(buf), V, code, st)
        coef = torch.full((R,), 1.0 / R, dtype=torch.float32, device=dev)
        n_rows = torch.full((1,), R, dtype=torch.int32, device=dev)
        ce = torch.empty(R, dtype=torch.float32, device=dev)
        tgt = targets.to(torch.int32).contiguous()
        # ce[r] = logsumexp - logit[target]; buf <- (softmax - onehot) / R
        call("alodlm_cross_entropy", ptr(buf), ptr(tgt), ptr(coef), ptr(n_rows), R, V, ptr(ce),
             None, code, st)
        ctx.save_for_backward(buf, sel)
        ctx.shape = (N, V)
        return ce.sum() / R

    @staticmethod
    def backward(ctx, grad):
        buf, sel = ctx.saved_tensors
        N, V = ctx.shape
        scaled = (buf * grad.to(buf.dtype)).contiguous()
        out = torch.zeros(N, V, dtype=buf.dtype, device=buf.device)
        call("alodlm_scatter_rows", ptr(scaled), ptr(sel), sel.numel(), ptr(out), N, V,
             _lib.dtype_code(buf.dtype), _lib.stream_handle(buf.device))
        return out, None, None


def autoregressive_loss(logits, labels, packed_boundaries):
    """Average next-token loss without crossing segments (alodlm/loss.py:12-32):
    clean row start + i of each dual-stream segment [start, end) predicts
    labels[start // 2 + 1 + i] (i < L - 1, L = (end - start) // 2); ignored
    labels (-100) do not count.  Returns a float32 scalar (0 with
    requires_grad when no target counts)."""
    _require_gpu(logits, "autoregressive_loss")
    N = logits.shape[0]
    bounds = packed_boundaries.to(device=logits.device, dtype=torch.int64).contiguous()
    lab = labels.to(device=logits.device, dtype=torch.int64).contiguous()
    target = torch.empty(N, dtype=torch.int32, device=logits.device)
    call("alodlm_ar_targets", ptr(lab), ptr(bounds), bounds.numel() - 1, N, ptr(target),
         _lib.stream_handle(logits.device))
    rows = torch.nonzero(target >= 0).flatten()
    if rows.numel() == 0:
        return torch.tensor(0.0, device=logits.device, requires_grad=True)
    return _AutoregressiveLoss.apply(logits, rows, target[rows])
