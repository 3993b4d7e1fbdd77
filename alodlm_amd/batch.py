"""Dual-stream masking (drop-in for alodlm/batch.py).

``build_batch`` keeps the reference's random numbers exactly
(alodlm/batch.py:50-60: per segment one ``uniform_`` of ceil(L/B) floats, then
one ``randperm`` per block whose masked count round(n*p) is nonzero, all from
the default generator of the ids' device).  The HIP entry point
``alodlm_mask_draws`` evaluates that whole sequence from the generator's
(seed, offset) in two launches, the generator is advanced past it, and
``alodlm_batch_build`` writes every dual-stream row.  Masks and orders are
therefore bit-identical to the reference's for the same generator state.  The attention mask is never materialised on the GPU: the attention
kernels enumerate the closed-form mask from the segment boundaries.
"""

from dataclasses import dataclass
import ctypes
import functools
import math

import numpy as np
import torch

from . import _lib
from .attention import plan_to_device, sparse_plan
from .layers import DualStreamMask, allowed_pairs, attention_tiles  # noqa: F401 (re-exported)


@dataclass
class Batch:
    """Dual-stream rows of one pack (fields of alodlm/batch.py:12-20).

    ``attention_mask`` is a ``layers.DualStreamMask`` (the kernels derive the
    mask from the segment boundaries; ``.dense()`` builds the reference's
    boolean [N, N] block-diagonal mask) for the "sdpa" backend, or the range
    plan of ``attention.plan_to_device`` for the others.  ``kernel_mask`` is
    the DualStreamMask in either case.  ``row_segment`` and ``ar_target`` are
    the per-row segment index and next-token target the step kernels use.
    """
    ids: torch.Tensor
    original: torch.Tensor
    positions: torch.Tensor
    masked: torch.Tensor
    mask_probability: torch.Tensor
    boundaries: torch.Tensor
    attention_mask: object
    row_segment: torch.Tensor = None
    ar_target: torch.Tensor = None
    ar_count: int = 0
    pairs: int = 0
    tiles: torch.Tensor = None
    kernel_mask: DualStreamMask = None


def attention_mask(length, block_size, device):
    """Dense dual-stream mask of one segment (closed form of alodlm/batch.py:23-31)."""
    q = torch.arange(2 * length, device=device)[:, None]
    k = torch.arange(2 * length, device=device)[None, :]
    q_noisy, k_noisy = q >= length, k >= length
    q_block = torch.where(q_noisy, q - length, q) // block_size
    k_block = torch.where(k_noisy, k - length, k) // block_size
    return ((q_block == k_block) & (q_noisy == k_noisy) & (k <= q)) | ((k_block < q_block) & ~k_noisy)


_DRAW_STREAMS = {}


def _draw_stream(device):
    """Per-device side stream (default priority) for the masking draws.

    The draws read no device data, so they need not wait for the compute
    stream: on a stream of their own, the host reads the generator's end
    offset back without draining the previous step's queued work."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _DRAW_STREAMS.get(index)
    if stream is None:
        stream = _DRAW_STREAMS[index] = torch.cuda.Stream(device=torch.device("cuda", index))
    return stream


def block_supervised_counts(labels_host, offsets, block_size):
    """Per segment, the number of supervised labels (!= -100) of every block
    (the candidate count n of alodlm/batch.py:50-55)."""
    out = []
    for a, b in zip(offsets, offsets[1:]):
        valid = (labels_host[a:b] != -100).astype(np.int64)
        out.append(np.add.reduceat(valid, np.arange(0, b - a, block_size)))
    return out


_LOG_THRESHOLD_12 = math.log(0.9) * 12


def max_segment_blocks(device):
    """Most masking blocks one segment may have on ``device``: torch's
    ``uniform_`` gives element i the first draw of Philox subsequence i only
    while its grid (256-thread blocks, max_threads_per_multi_processor / 256
    of them per compute unit) covers every element, i.e. up to compute units
    x max threads per compute unit elements (524288 on a 256-CU MI355X)."""
    props = torch.cuda.get_device_properties(device)
    return props.multi_processor_count * props.max_threads_per_multi_processor


@functools.lru_cache(maxsize=None)
def key_bits(block_size):
    """Key width torch.randperm(n) sorts on, for n = 0..block_size: the fewest
    bits that keep the chance of any duplicate key under 10 % (the randperm
    note of ATen/native/cuda/Randperm.cuh), evaluated in double precision as
    torch's host code does."""
    bits = [0]
    for n in range(1, block_size + 1):
        nd = float(n)
        bits.append(min(64, math.ceil(math.log2(nd - (6 * nd * nd + 1) / _LOG_THRESHOLD_12))))
    return np.asarray(bits, dtype=np.int32)


def _device_draws(block_n, seg_block, block_size, device, generator):
    """The draws of alodlm/batch.py:50-60 from the generator's current state,
    by ``alodlm_mask_draws`` on the side stream; the generator is then
    advanced past every random number the reference's calls would consume.

    Returns device tensors (p, count, perm_offset, perms) for batch_build."""
    limit = max_segment_blocks(device)
    if max(b - a for a, b in zip(seg_block, seg_block[1:])) > limit:
        raise ValueError(f"a segment of more than {limit} masking blocks is not supported on "
                         "this device (torch's uniform_ would draw them from shared Philox "
                         "subsequences)")
    gen = _generator_of(device, generator)
    seed, offset = gen.initial_seed(), gen.get_offset()
    nblocks = len(block_n)
    side = _draw_stream(device)
    with torch.cuda.stream(side):
        n_t = _to_device(block_n.astype(np.int32), device)
        sb_t = _to_device(np.asarray(seg_block, dtype=np.int32), device)
        bits_t = _to_device(key_bits(block_size), device)
        p_t = torch.empty(nblocks, dtype=torch.float32, device=device)
        c_t = torch.empty(nblocks, dtype=torch.int32, device=device)
        bo_t = torch.empty(nblocks, dtype=torch.int64, device=device)
        po_t = torch.empty(nblocks, dtype=torch.int64, device=device)
        perms = torch.empty(nblocks * block_size, dtype=torch.int64, device=device)
        end_t = torch.empty(1, dtype=torch.int64, device=device)
        _lib.call("alodlm_mask_draws", ctypes.c_uint64(seed), ctypes.c_uint64(offset),
                  _lib.ptr(sb_t), len(seg_block) - 1, _lib.ptr(n_t), nblocks, block_size,
                  _lib.ptr(bits_t), _lib.ptr(p_t), _lib.ptr(c_t), _lib.ptr(bo_t), _lib.ptr(po_t),
                  _lib.ptr(perms), _lib.ptr(end_t), _lib.stream_handle(device))
        end_host = torch.empty(1, dtype=torch.int64, pin_memory=True)
        end_host.copy_(end_t, non_blocking=True)
        done = torch.cuda.Event()
        done.record(side)
    done.synchronize()
    gen.set_offset(int(end_host[0]))
    main = torch.cuda.current_stream(device)
    main.wait_stream(side)
    for t in (p_t, c_t, po_t, perms):
        t.record_stream(main)
    return p_t, c_t, po_t, perms


def _replayed_draws(draws, device):
    """Device tensors of given (p, count, perms) per block."""
    probs, counts, perms = draws
    perm_offset = np.zeros(len(perms), dtype=np.int64)
    chunks, total = [], 0
    for i, perm in enumerate(perms):
        perm_offset[i] = total
        if perm is not None:
            chunks.append(perm.to(device=device, dtype=torch.int64))
            total += perm.numel()
    perm_buf = (torch.cat(chunks) if chunks
                else torch.zeros(1, dtype=torch.int64, device=device))
    return (_to_device(np.asarray(probs, dtype=np.float32), device),
            _to_device(np.asarray(counts, dtype=np.int32), device),
            _to_device(perm_offset, device), perm_buf)


def _generator_of(device, generator):
    if generator is not None:
        return generator
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch.cuda.default_generators[index]


def _to_device(array, device):
    """Host array -> device tensor through pinned memory, without blocking:
    a copy from pageable memory would wait for all work queued on the stream."""
    return torch.from_numpy(np.ascontiguousarray(array)).pin_memory().to(device, non_blocking=True)


@torch.no_grad()
def build_batch(ids, labels, boundaries, block_size, mask_token_id, backend="sdpa",
                generator=None, draws=None, labels_host=None):
    """Dual-stream batch of one pack (alodlm/batch.py:34-85) on the GPU.

    ``backend`` is accepted for API compatibility; the attention kernels read the
    mask from the boundaries whatever its value.  ``draws`` (p, counts, perms)
    may be supplied to replay known randomness.  ``labels_host``, a host copy
    of ``labels``, saves reading them back from the device (which waits for
    the work queued before this call).
    """
    if ids.ndim != 1 or ids.shape != labels.shape or ids.numel() == 0:
        raise ValueError("Expected nonempty flat input and label tensors")
    offsets = [int(v) for v in boundaries.tolist()]
    if offsets[0] != 0 or offsets[-1] != len(ids):
        raise ValueError("Boundaries must cover the packed tokens")
    if any(a >= b for a, b in zip(offsets, offsets[1:])):
        raise ValueError("Packed segments must be nonempty")
    if block_size < 1 or block_size > 1024:
        raise ValueError("block_size must be in [1, 1024]")
    device = ids.device
    if device.type != "cuda":
        raise ValueError("build_batch runs on the GPU; move ids/labels to a CUDA device")
    nseg = len(offsets) - 1
    seg_block = [0]
    for a, b in zip(offsets, offsets[1:]):
        seg_block.append(seg_block[-1] + (b - a + block_size - 1) // block_size)
    nblocks = seg_block[-1]
    if labels_host is None:
        labels_host = labels.detach().cpu().numpy()
    if draws is None:
        block_n = np.concatenate(block_supervised_counts(labels_host, offsets, block_size))
        p_t, c_t, po_t, perm_buf = _device_draws(block_n, seg_block, block_size, device,
                                                 generator)
    else:
        p_t, c_t, po_t, perm_buf = _replayed_draws(draws, device)
    ids = ids.to(torch.int64).contiguous()
    labels = labels.to(torch.int64).contiguous()
    n = 2 * len(ids)
    seg_t = _to_device(np.asarray(offsets, dtype=np.int64), device)
    seg_block_t = _to_device(np.asarray(seg_block, dtype=np.int32), device)
    out = {
        "ids": torch.empty(n, dtype=torch.int64, device=device),
        "original": torch.empty(n, dtype=torch.int64, device=device),
        "positions": torch.empty(n, dtype=torch.int64, device=device),
        "masked": torch.empty(n, dtype=torch.bool, device=device),
        "prob": torch.empty(n, dtype=torch.float32, device=device),
        "row_segment": torch.empty(n, dtype=torch.int32, device=device),
        "ar_target": torch.empty(n, dtype=torch.int32, device=device),
        "bounds": torch.empty(nseg + 1, dtype=torch.int64, device=device),
    }
    _lib.call("alodlm_batch_build", _lib.ptr(ids), _lib.ptr(labels), _lib.ptr(seg_t),
              _lib.ptr(seg_block_t), nseg, nblocks, block_size, mask_token_id, _lib.ptr(p_t),
              _lib.ptr(c_t), _lib.ptr(po_t), _lib.ptr(perm_buf), _lib.ptr(out["ids"]),
              _lib.ptr(out["original"]), _lib.ptr(out["positions"]), _lib.ptr(out["masked"]),
              _lib.ptr(out["prob"]), _lib.ptr(out["row_segment"]), _lib.ptr(out["ar_target"]),
              _lib.ptr(out["bounds"]), _lib.stream_handle(device))
    # number of autoregressive targets (alodlm/loss.py:21-29), from the host labels
    ar_count = 0
    for a, b in zip(offsets, offsets[1:]):
        if b - a >= 2:
            ar_count += int((labels_host[a + 1:b] != -100).sum())
    kernel_mask = DualStreamMask(offsets, block_size, device, boundaries=out["bounds"],
                                 row_segment=out["row_segment"])
    if backend == "sdpa":
        mask = kernel_mask
    else:
        mask = plan_to_device(sparse_plan([2 * v for v in offsets], block_size, backend), device)
    return Batch(out["ids"], out["original"], out["positions"], out["masked"], out["prob"],
                 out["bounds"], mask, out["row_segment"], out["ar_target"], ar_count,
                 kernel_mask.pairs, kernel_mask.tiles, kernel_mask)
