"""Sequence credit primitives on the HIP kernels (drop-in for alodlm/credit.py).

``masked_sequence_ids(masked_indices, cum_seqlens)`` gives the sequence of
every masked row; ``sequence_score_function(credit, log_prob, sequence_ids,
sequence_count)`` is the score-function surrogate (1/M) sum_s R_s Q_s, R_s and
Q_s the per-sequence sums of the detached credit and of log q.  Arguments are
validated with the reference's ValueError messages (alodlm/credit.py:8-35);
the sums run in one workgroup with a fixed order (float32), so results are
deterministic.
"""

import torch

from . import _lib
from ._lib import call, ptr


def _require_gpu(t, what):
    if t.device.type != "cuda":
        raise ValueError(f"{what} runs on the HIP kernels; move the tensors to a CUDA (ROCm) device")


def check_sequence_boundaries(masked_indices, cum_seqlens):
    """The argument checks of alodlm/credit.py:8-19."""
    if masked_indices.ndim != 1 or masked_indices.dtype != torch.bool:
        raise ValueError('masked_indices must be a one-dimensional boolean tensor')
    if cum_seqlens is None or cum_seqlens.ndim != 1 or cum_seqlens.numel() < 2:
        raise ValueError('Outcome credit requires packed sequence boundaries')
    if cum_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError('Sequence boundaries must use an integer dtype')
    if cum_seqlens.device != masked_indices.device:
        raise ValueError('Sequence boundaries and mask must share a device')
    bounds = cum_seqlens.tolist()
    if bounds[0] != 0 or bounds[-1] != masked_indices.numel():
        raise ValueError('Sequence boundaries must cover the actual packed stream')
    if any(b < a for a, b in zip(bounds, bounds[1:])):
        raise ValueError('Sequence boundaries must be nondecreasing')


def masked_sequence_ids(masked_indices, cum_seqlens):
    """Sequence index of every masked row, in row order (alodlm/credit.py:7-21:
    bucketize(arange(N), cum_seqlens[1:], right=True)[masked])."""
    check_sequence_boundaries(masked_indices, cum_seqlens)
    _require_gpu(masked_indices, "masked_sequence_ids")
    rows = masked_indices.numel()
    bounds = cum_seqlens.to(torch.int64).contiguous()
    out = torch.empty(rows, dtype=torch.int64, device=masked_indices.device)
    count = torch.empty(1, dtype=torch.int64, device=masked_indices.device)
    mask = masked_indices.contiguous().view(torch.uint8)
    call("alodlm_masked_sequence_ids", ptr(mask), ptr(bounds), bounds.numel() - 1, rows,
         ptr(out), ptr(count), _lib.stream_handle(masked_indices.device))
    return out[:int(count.item())]


class _SequenceScore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, credit, log_prob, sequence_ids, sequence_count):
        n = credit.numel()
        dev = credit.device
        value = torch.empty(1, dtype=torch.float32, device=dev)
        dlogq = torch.empty(n, dtype=torch.float32, device=dev)
        ws = torch.empty(2 * sequence_count, dtype=torch.float32, device=dev)
        c32 = credit.detach().to(torch.float32).contiguous()
        q32 = log_prob.detach().to(torch.float32).contiguous()
        ids = sequence_ids.contiguous()
        call("alodlm_sequence_score", ptr(c32), ptr(q32), ptr(ids), n, sequence_count,
             ptr(value), ptr(dlogq), ptr(ws), _lib.stream_handle(dev))
        ctx.save_for_backward(dlogq)
        ctx.dtype = log_prob.dtype
        return value[0].to(log_prob.dtype)

    @staticmethod
    def backward(ctx, grad):
        (dlogq,) = ctx.saved_tensors
        return None, (dlogq * grad.to(torch.float32)).to(ctx.dtype), None, None


def sequence_score_function(credit, log_prob, sequence_ids, sequence_count):
    """dot(segment_sum(credit.detach()), segment_sum(log_prob)) / len(credit)
    (alodlm/credit.py:23-40); differentiable in ``log_prob``."""
    if credit.ndim != 1 or log_prob.shape != credit.shape or sequence_ids.shape != credit.shape:
        raise ValueError('Credit, log probabilities, and sequence IDs must be equal-length vectors')
    if sequence_ids.dtype != torch.int64 or sequence_count < 1:
        raise ValueError('Sequence IDs must be int64 and sequence_count must be positive')
    if not credit.device == log_prob.device == sequence_ids.device:
        raise ValueError('Credit, log probabilities, and IDs must share a device')
    if credit.dtype != log_prob.dtype:
        raise ValueError('Credit and log probabilities must share a dtype')
    if credit.numel() == 0:
        return log_prob.sum() * 0
    if bool(((sequence_ids < 0) | (sequence_ids >= sequence_count)).any()):
        raise ValueError('Sequence IDs must be within the declared sequence count')
    _require_gpu(credit, "sequence_score_function")
    return _SequenceScore.apply(credit, log_prob, sequence_ids, int(sequence_count))
