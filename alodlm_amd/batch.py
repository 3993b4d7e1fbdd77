"""Dual-stream masking (drop-in for alodlm/batch.py).

``build_batch`` keeps the reference's random-number consumption exactly
(alodlm/batch.py:50-60: per segment one ``uniform_`` of ceil(L/B) floats, then
one ``randperm`` per block whose masked count round(n*p) is nonzero, all from
the default generator of the ids' device) and hands the draws to the HIP
kernel ``alodlm_batch_build``, which writes every dual-stream row.  Masks and
orders are therefore bit-identical to the reference's for the same generator
state.  The attention mask is never materialised on the GPU: the attention
kernels enumerate the closed-form mask from the segment boundaries.
"""

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .attention import plan_to_device, sparse_plan


@dataclass
class Batch:
    """Dual-stream rows of one pack (fields of alodlm/batch.py:12-20).

    ``attention_mask`` is the string ``"dual-stream"`` (the kernels derive the
    mask from ``boundaries``) unless a dense mask or a range plan was requested.
    ``row_segment`` and ``ar_target`` are the per-row segment index and
    next-token target the step kernels use.
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


def allowed_pairs(length, block_size):
    """Number of (query, key) pairs the dual-stream mask allows in one segment:
    the causal clean stream plus, per noisy block, its causal self-block and
    the clean rows of all earlier blocks."""
    total = length * (length + 1) // 2
    for left in range(0, length, block_size):
        width = min(block_size, length - left)
        total += width * (width + 1) // 2 + width * left
    return total


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
    stream: on a stream of their own, the host reads the per-segment mask
    ratios back without draining the previous step's queued work.  The
    generator's state advances on the host at launch time, so the values and
    their order are the same as on the compute stream."""
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


def full_block_counts(offsets, block_size):
    """Per segment, the block widths: the candidate counts when every label
    is supervised."""
    out = []
    for a, b in zip(offsets, offsets[1:]):
        starts = np.arange(0, b - a, block_size)
        out.append(np.minimum(block_size, (b - a) - starts).astype(np.int64))
    return out


def draw_masking(labels_host, offsets, block_size, device, generator=None):
    """Draw the masking randomness in the reference's order.

    Returns per-block arrays (p, count) on the host and the list of per-block
    permutations (tensors on ``device``, or None where count is zero).  On a
    GPU the draws are issued on the side stream of ``_draw_stream``; the
    caller orders its own stream after that one before reading them.
    """
    device = torch.device(device)
    counts = block_supervised_counts(labels_host, offsets, block_size)
    if device.type == "cuda":
        with torch.cuda.stream(_draw_stream(device)):
            return _draw(counts, offsets, block_size, device, generator)
    return _draw(counts, offsets, block_size, device, generator)


def _draw(block_counts, offsets, block_size, device, generator):
    """The draws of alodlm/batch.py:50-60 for given candidate counts n."""
    probs, counts, perms = [], [], []
    for (a, b), n in zip(zip(offsets, offsets[1:]), block_counts):
        nblocks = (b - a + block_size - 1) // block_size
        u = torch.empty(nblocks, device=device).uniform_(0, 1, generator=generator).clamp_min(1e-8)
        # p as the reference reads it (a float32 value widened to float64) and
        # round(n * p) rounded half to even in float64 like Python's round
        p = u.cpu().numpy().astype(np.float64)
        count = np.rint(n * p).astype(np.int64)
        probs.extend(p.tolist())
        counts.extend(count.tolist())
        for blk in range(nblocks):
            perms.append(torch.randperm(int(n[blk]), device=device, generator=generator)
                         if count[blk] else None)
    return np.asarray(probs, dtype=np.float32), np.asarray(counts, dtype=np.int32), perms


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
    side = _draw_stream(device)
    speculative = None
    if draws is None:
        # The draws depend on the labels only through the supervised count of
        # every block.  Draw first assuming every label is supervised: this
        # needs no labels on the host, so it overlaps the work still queued
        # on the compute stream.  If the labels then show an unsupervised
        # position, the generator is rewound and the draws are made again
        # with the true counts; either way the consumed random numbers are
        # exactly the reference's.
        gen = _generator_of(device, generator)
        state = gen.get_state()
        assumed = full_block_counts(offsets, block_size)
        with torch.cuda.stream(side):
            speculative = _draw(assumed, offsets, block_size, device, generator)
    if labels_host is None:
        labels_host = labels.detach().cpu().numpy()
    with torch.cuda.stream(side):
        if draws is None:
            actual = block_supervised_counts(labels_host, offsets, block_size)
            if all(np.array_equal(x, y) for x, y in zip(actual, assumed)):
                draws = speculative
            else:
                gen.set_state(state)
                draws = _draw(actual, offsets, block_size, device, generator)
        probs, counts, perms = draws
        perm_offset = np.zeros(nblocks, dtype=np.int64)
        chunks, total = [], 0
        for i, perm in enumerate(perms):
            perm_offset[i] = total
            if perm is not None:
                chunks.append(perm.to(device=device, dtype=torch.int64))
                total += perm.numel()
        perm_buf = (torch.cat(chunks) if chunks
                    else torch.zeros(1, dtype=torch.int64, device=device))
    main = torch.cuda.current_stream(device)
    main.wait_stream(side)
    perm_buf.record_stream(main)
    ids = ids.to(torch.int64).contiguous()
    labels = labels.to(torch.int64).contiguous()
    n = 2 * len(ids)
    seg_t = _to_device(np.asarray(offsets, dtype=np.int64), device)
    seg_block_t = _to_device(np.asarray(seg_block, dtype=np.int32), device)
    p_t = _to_device(probs, device)
    c_t = _to_device(counts, device)
    po_t = _to_device(perm_offset, device)
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
    if backend == "sdpa":
        mask = "dual-stream"
    else:
        mask = plan_to_device(sparse_plan([2 * v for v in offsets], block_size, backend), device)
    pairs = sum(allowed_pairs(b - a, block_size) for a, b in zip(offsets, offsets[1:]))
    tiles = _to_device(np.asarray(attention_tiles(offsets), dtype=np.int32), device).view(-1, 2)
    return Batch(out["ids"], out["original"], out["positions"], out["masked"], out["prob"],
                 out["bounds"], mask, out["row_segment"], out["ar_target"], ar_count, pairs,
                 tiles)


TILE_ROWS = 128


def attention_tiles(offsets):
    """(segment, in-segment start) of every 128-row tile of each segment's clean
    and noisy stream; tiles never cross a stream or a segment.

    Tiles are listed by decreasing start within their stream.  A query tile's
    key range grows with its start and a key tile's query range shrinks with
    it, so the forward/dQ kernels (which take the list in order) and the dK/dV
    kernel (which takes it in reverse) both dispatch their heaviest tiles
    first."""
    tiles = []
    for s, (a, b) in enumerate(zip(offsets, offsets[1:])):
        length = b - a
        for stream in (0, length):
            for start in range(0, length, TILE_ROWS):
                tiles.append((start, s, stream + start))
    tiles.sort(key=lambda t: -t[0])
    return [v for _, s, start in tiles for v in (s, start)]
