"""Host-side batch logic (no GPU): the candidate counts that decide the
masking draws of alodlm/batch.py:50-60."""

import numpy as np


def test_block_candidate_counts():
    """Supervised counts per block of every segment (the last block ragged)."""
    from alodlm_amd.batch import block_supervised_counts
    labels = np.array([1, -100, 2, 3, -100, -100, 4, 5, 6, 7, 8], dtype=np.int64)
    offsets = [0, 4, 11]
    got = block_supervised_counts(labels, offsets, 3)
    assert [x.tolist() for x in got] == [[2, 1], [1, 3, 1]]
    full = block_supervised_counts(np.arange(11), offsets, 3)
    assert [x.tolist() for x in full] == [[3, 1], [3, 3, 1]]
