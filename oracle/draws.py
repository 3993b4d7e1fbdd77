"""CPU restatement of the masking draws on a Philox device generator (TEST
INFRASTRUCTURE ONLY).

alodlm/batch.py:50-60 draws, per segment, the block mask ratios with
``torch.empty(n, device=cuda).uniform_(0, 1).clamp_min(1e-8)`` and, per block
with a nonzero masked count, ``torch.randperm(n_cand, device=cuda)``.  On a GPU
both come from torch's Philox4x32-10 generator, whose (seed, offset) state
fixes every value.  This module evaluates those calls on the host from that
state, in plain Python integers (small packs only), following torch's
kernels:

* ``uniform_``: ATen/native/cuda/DistributionTemplates.h
  (``calc_execution_policy``, ``distribution_elementwise_grid_stride_kernel``,
  ``uniform_kernel``) with the rocRAND float mapping 2^-32 + v * 2^-32
  (rocrand_uniform.h);
* ``randperm``: the randperm note of ATen/native/cuda/Randperm.cuh (keys from
  ``random_(INT_MIN, INT_MAX)``, a stable sort on the low key bits, and
  ``randperm_handle_duplicate_keys``'s Fisher-Yates over runs of equal keys);
* Philox4x32-10: Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as
  easy as 1, 2, 3" (SC 2011), with the cuRAND/rocRAND stream convention
  (key = seed, counter = (offset / 4, subsequence)).

Pinning: ``philox4x32_10`` against the Random123 known-answer vectors
(tests/test_draws_host.py); the whole sequence against torch's own draws on a
GPU (tests/test_draws_gpu.py), which is the reference's exact call sequence.
"""

import math

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32_10(counter, key):
    """Ten Philox rounds on a 4-word counter with a 2-word key (SC 2011, the
    S-box-free 4x32 variant)."""
    c0, c1, c2, c3 = counter
    k0, k1 = key
    for _ in range(10):
        p0, p1 = M0 * c0, M1 * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & MASK32, p1 & MASK32, \
                         ((p0 >> 32) ^ c3 ^ k1) & MASK32, p0 & MASK32
        k0, k1 = (k0 + W0) & MASK32, (k1 + W1) & MASK32
    return c0, c1, c2, c3


def stream(seed, subsequence, offset):
    """Successive 32-bit outputs of Philox stream (seed, subsequence, offset);
    offset is a multiple of 4."""
    block = offset // 4
    key = (seed & MASK32, (seed >> 32) & MASK32)
    while True:
        counter = (block & MASK32, (block >> 32) & MASK32,
                   subsequence & MASK32, (subsequence >> 32) & MASK32)
        yield from philox4x32_10(counter, key)
        block += 1


def _first4(seed, subsequence, offset):
    g = stream(seed, subsequence, offset)
    return [next(g) for _ in range(4)]


def uniform01(v):
    """float32 (0, 1] value of a 32-bit draw: 2^-32 + v * 2^-32."""
    return np.float32(np.float32(v) * np.float32(2.0 ** -32) + np.float32(2.0 ** -32))


def uniform(n, seed, offset):
    """``torch.empty(n).uniform_(0, 1)`` on the device: (values, offset after)."""
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        u = uniform01(_first4(seed, i, offset)[0])
        out[i] = np.float32(0.0) if u == np.float32(1.0) else u
    return out, offset + 4


def key_bits(n):
    """Bits of the randperm sort key (the randperm note in Randperm.cuh)."""
    nd = float(n)
    return min(64, math.ceil(math.log2(nd - (6 * nd * nd + 1) / (math.log(0.9) * 12))))


def randperm(n, seed, offset):
    """``torch.randperm(n)`` on the device for small n: (perm, offset after)."""
    bits = key_bits(n)
    assert bits <= 32
    mask = (1 << bits) - 1
    keys = []
    for j in range(n):
        x, y = _first4(seed, j, offset)[:2]
        keys.append(((x << 32 | y) % 0xFFFFFFFF) & mask)
    order = sorted(range(n), key=lambda j: keys[j])  # stable
    skeys = [keys[j] for j in order]
    dup = offset + 4
    t = 0
    while t < n - 1:
        size = 1
        while t + size < n and skeys[t + size] == skeys[t]:
            size += 1
        if size > 1:
            g = stream(seed, t, dup)
            for i in range(size - 1, 0, -1):
                r = next(g) % (i + 1)
                order[t + i], order[t + r] = order[t + r], order[t + i]
        t += size
    return np.asarray(order, dtype=np.int64), offset + 4 + (n + 3) // 4 * 4


def mask_draws(block_n_per_segment, seed, offset):
    """The draws of alodlm/batch.py:50-60 for candidate counts n of every block
    of every segment: (p float32, count int32, perms list, offset after)."""
    probs, counts, perms = [], [], []
    for block_n in block_n_per_segment:
        u, offset = uniform(len(block_n), seed, offset)
        p = np.maximum(u, np.float32(1e-8))
        for n, pv in zip(block_n, p):
            count = round(int(n) * float(pv))
            probs.append(pv)
            counts.append(count)
            if count:
                perm, offset = randperm(int(n), seed, offset)
                perms.append(perm)
            else:
                perms.append(None)
    return (np.asarray(probs, dtype=np.float32), np.asarray(counts, dtype=np.int32), perms,
            offset)
