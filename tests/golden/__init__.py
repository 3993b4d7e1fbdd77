"""Golden vectors written from the reference by make_golden.py (data only)."""

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def load(name):
    """Load one golden case as a dict of numpy arrays (no pickle)."""
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def projection_vector(index, numel):
    """The fixed +-1 vector make_golden.py summarises gradients with."""
    import torch
    g = torch.Generator().manual_seed(1000 + index)
    return (torch.randint(0, 2, (numel,), generator=g) * 2 - 1).double()


def sample_indices(numel, count=256):
    """``count`` strided indices into a tensor of ``numel`` elements."""
    stride = max(1, numel // count)
    return np.arange(0, numel, stride)[:count]
