"""Masking-draw restatement on the host (oracle/draws.py): Philox4x32-10
against the Random123 known-answer vectors, and the shape of the randperm and
uniform_ restatements (permutations, ranges, consumed offsets)."""

import numpy as np
import pytest

from oracle import draws as D


@pytest.mark.parametrize("counter,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_known_answers(counter, key, expect):
    """Random123's kat_vectors for philox4x32 with 10 rounds."""
    assert D.philox4x32_10(counter, key) == expect


def test_stream_counter_layout():
    """offset/4 is the low counter half, the subsequence the high half."""
    seed = 0x0123456789ABCDEF
    key = (seed & 0xFFFFFFFF, seed >> 32)
    g = D.stream(seed, 5, 8)
    assert tuple(next(g) for _ in range(4)) == D.philox4x32_10((2, 0, 5, 0), key)
    assert tuple(next(g) for _ in range(4)) == D.philox4x32_10((3, 0, 5, 0), key)
    big = D.stream(seed, 1 << 33, (1 << 34) + 4)
    assert tuple(next(big) for _ in range(4)) == D.philox4x32_10((1, 1, 0, 2), key)


def test_uniform_range_and_offset():
    u, off = D.uniform(300, seed=7, offset=12)
    assert off == 16
    assert u.dtype == np.float32 and np.all(u >= 0) and np.all(u < 1)
    # the float mapping: 2^-32 + v 2^-32 rounds v to 24 bits, so v = 2^32 - 1 gives 1.0
    assert D.uniform01(0xFFFFFFFF) == np.float32(1.0)
    assert D.uniform01(0) == np.float32(2.0 ** -32)


@pytest.mark.parametrize("n", [1, 2, 3, 17, 32, 100, 1024])
def test_randperm_is_permutation(n):
    perm, off = D.randperm(n, seed=11, offset=40)
    assert sorted(perm.tolist()) == list(range(n))
    assert off == 40 + 4 + (n + 3) // 4 * 4


def test_key_bits_table_matches():
    """The product's table of sort-key widths is the restatement's formula."""
    from alodlm_amd.batch import key_bits
    table = key_bits(1024)
    assert table[0] == 0
    assert [int(v) for v in table[1:]] == [D.key_bits(n) for n in range(1, 1025)]
    assert D.key_bits(32) == 13 and D.key_bits(1) == 3


def test_mask_draws_offsets():
    """Each segment consumes 4 for its ratios plus, per masked block,
    4 + n rounded up to 4."""
    probs, counts, perms, end = D.mask_draws([np.array([5, 32, 0]), np.array([7])], 3, 0)
    expect = 8 + sum(4 + (n + 3) // 4 * 4 for n, c in zip([5, 32, 0, 7], counts) if c)
    assert end == expect
    assert all((p is None) == (c == 0) for p, c in zip(perms, counts))
    assert counts[2] == 0
