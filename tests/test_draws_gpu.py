"""Masking draws by ``alodlm_mask_draws`` against torch's own device draws in
the reference's order (alodlm/batch.py:50-60: uniform_ per segment, randperm
per masked block) and against the host restatement (oracle/draws.py): the
ratios bit for bit, the counts, every permutation and the generator state
left behind."""

import numpy as np
import pytest
import torch

from tests.helpers import draw_masking, log

pytestmark = pytest.mark.gpu

CASES = [
    # (segment lengths, block size, unsupervised fraction, seed, draws made before)
    ([2048] * 8, 32, 0.0, 0, 0),
    ([2048, 2048], 32, 0.3, 7, 3),
    ([100, 1, 232, 31, 33], 32, 0.1, 123, 1),
    ([4096], 7, 0.2, 2 ** 63 + 12345, 2),
    ([1500, 900], 100, 0.5, 99, 0),
    ([3000], 1024, 0.0, 5, 1),
    ([16384], 32, 0.05, 17, 0),
]


def _labels(lengths, frac, seed):
    g = torch.Generator().manual_seed(seed % (2 ** 31))
    total = sum(lengths)
    labels = torch.randint(0, 1000, (total,), generator=g)
    if frac:
        labels[torch.rand(total, generator=g) < frac] = -100
    return labels.numpy()


@pytest.mark.parametrize("lengths,block_size,frac,seed,before", CASES)
def test_mask_draws_match_torch(lengths, block_size, frac, seed, before):
    from alodlm_amd.batch import _device_draws, block_supervised_counts
    log(f"mask_draws lengths={lengths} B={block_size} frac={frac} seed={seed}")
    labels = _labels(lengths, frac, seed)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).tolist()
    seg_block = [0]
    for n in lengths:
        seg_block.append(seg_block[-1] + (n + block_size - 1) // block_size)
    torch.cuda.manual_seed(seed)
    for k in range(before):
        torch.rand(5 + 300 * k, device="cuda")
    start = torch.cuda.get_rng_state()
    probs, counts, perms = draw_masking(labels, offsets, block_size, "cuda")
    torch.cuda.synchronize()
    after_ref = torch.cuda.get_rng_state()

    torch.cuda.set_rng_state(start)
    block_n = np.concatenate(block_supervised_counts(labels, offsets, block_size))
    p_t, c_t, po_t, perm_buf = _device_draws(block_n, seg_block, block_size,
                                             torch.device("cuda"), None)
    torch.cuda.synchronize()
    assert torch.equal(torch.cuda.get_rng_state(), after_ref), "generator state differs"
    p = p_t.cpu().numpy()
    assert np.array_equal(p.view(np.uint32), probs.view(np.uint32)), "mask ratios differ"
    assert np.array_equal(c_t.cpu().numpy(), counts)
    po = po_t.cpu().numpy()
    buf = perm_buf.cpu().numpy()
    for b, perm in enumerate(perms):
        if perm is None:
            continue
        got = buf[po[b]:po[b] + int(block_n[b])]
        assert np.array_equal(got, perm.cpu().numpy()), f"block {b} n={block_n[b]}"


def test_mask_draws_match_restatement():
    """The host restatement of torch's Philox draws agrees with the kernel."""
    from oracle import draws as D
    from alodlm_amd.batch import _device_draws, block_supervised_counts
    lengths, block_size = [300, 77, 64], 16
    labels = _labels(lengths, 0.2, 3)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).tolist()
    seg_block = [0]
    for n in lengths:
        seg_block.append(seg_block[-1] + (n + block_size - 1) // block_size)
    per_seg = block_supervised_counts(labels, offsets, block_size)
    torch.cuda.manual_seed(2024)
    torch.rand(10, device="cuda")
    gen = torch.cuda.default_generators[torch.cuda.current_device()]
    seed, offset = gen.initial_seed(), gen.get_offset()
    probs, counts, perms, end = D.mask_draws(per_seg, seed, offset)
    p_t, c_t, po_t, perm_buf = _device_draws(np.concatenate(per_seg), seg_block, block_size,
                                             torch.device("cuda"), None)
    torch.cuda.synchronize()
    assert gen.get_offset() == end
    assert np.array_equal(p_t.cpu().numpy().view(np.uint32), probs.view(np.uint32))
    assert np.array_equal(c_t.cpu().numpy(), counts)
    buf, po = perm_buf.cpu().numpy(), po_t.cpu().numpy()
    block_n = np.concatenate(per_seg)
    for b, perm in enumerate(perms):
        if perm is not None:
            assert np.array_equal(buf[po[b]:po[b] + int(block_n[b])], perm), b


def test_mask_draws_with_own_generator():
    """build_batch's `generator` argument: the draws come from that CUDA
    generator (not the default one) and advance only it."""
    from alodlm_amd.batch import _device_draws, block_supervised_counts
    lengths, block_size = [700, 300], 32
    labels = _labels(lengths, 0.1, 4)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).tolist()
    seg_block = [0]
    for n in lengths:
        seg_block.append(seg_block[-1] + (n + block_size - 1) // block_size)
    default_before = torch.cuda.get_rng_state()
    ref_gen = torch.Generator(device="cuda").manual_seed(31)
    probs, counts, perms = draw_masking(labels, offsets, block_size, "cuda", ref_gen)
    gen = torch.Generator(device="cuda").manual_seed(31)
    block_n = np.concatenate(block_supervised_counts(labels, offsets, block_size))
    p_t, c_t, po_t, perm_buf = _device_draws(block_n, seg_block, block_size,
                                             torch.device("cuda"), gen)
    torch.cuda.synchronize()
    assert gen.get_offset() == ref_gen.get_offset()
    assert torch.equal(torch.cuda.get_rng_state(), default_before)
    assert np.array_equal(p_t.cpu().numpy().view(np.uint32), probs.view(np.uint32))
    assert np.array_equal(c_t.cpu().numpy(), counts)
    buf, po = perm_buf.cpu().numpy(), po_t.cpu().numpy()
    for b, perm in enumerate(perms):
        if perm is not None:
            assert np.array_equal(buf[po[b]:po[b] + int(block_n[b])], perm.cpu().numpy()), b
