"""Batch building on the GPU generator: the masking draws consume exactly the
random numbers of the reference's order (alodlm/batch.py:50-60), whether or
not every label is supervised, and give the same rows as those draws made by
torch's own calls."""

import numpy as np
import pytest
import torch

from tests.helpers import draw_masking, log

pytestmark = pytest.mark.gpu


def _batch(labels, bounds, seed, draws=None):
    from alodlm_amd.batch import build_batch
    torch.cuda.manual_seed(seed)
    ids = torch.arange(len(labels), dtype=torch.int64) % 97 + 5
    b = build_batch(ids.cuda(), labels.cuda(), torch.tensor(bounds), 32, 3, draws=draws)
    torch.cuda.synchronize()
    state = torch.cuda.get_rng_state()
    return b, state


@pytest.mark.parametrize("unsupervised", [False, True])
@pytest.mark.parametrize("bounds", [[0, 2048, 4096], [0, 100, 101, 333]])
def test_device_draws_match_direct_draws(unsupervised, bounds):
    log(f"batch draws bounds={bounds} unsupervised={unsupervised}")
    g = torch.Generator().manual_seed(len(bounds))
    labels = torch.randint(0, 1000, (bounds[-1],), generator=g)
    if unsupervised:
        labels[torch.rand(bounds[-1], generator=g) < 0.1] = -100
    b, state = _batch(labels, bounds, seed=7)
    # the same generator state, drawn directly in the reference's order
    torch.cuda.manual_seed(7)
    draws = draw_masking(labels.numpy(), bounds, 32, "cuda")
    torch.cuda.synchronize()
    direct_state = torch.cuda.get_rng_state()
    assert torch.equal(state, direct_state), "random numbers consumed differ"
    ref, _ = _batch(labels, bounds, seed=123, draws=draws)
    for name in ("ids", "original", "positions", "masked", "mask_probability"):
        assert torch.equal(getattr(b, name).cpu(), getattr(ref, name).cpu()), name
