"""The C ABI: every entry point declared in include/alodlm_hip.h is exported by
the built library and bound in alodlm_amd._lib with the same arity (no GPU
work is launched here)."""

import ctypes
from pathlib import Path
import re

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "alodlm_hip.h"


def declarations():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"(int64_t|int|const char\*)\s+(alodlm_\w+)\(([^;]*?)\);", text):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_header_declares_entry_points():
    decls = declarations()
    assert len(decls) >= 30
    assert "alodlm_gemm" in decls and "alodlm_attention_fwd" in decls


def test_library_exports_every_declared_symbol():
    from alodlm_amd import _lib
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built (run python -m alodlm_amd.build)")
    lib = ctypes.CDLL(str(_lib.LIBRARY))
    for name in declarations():
        assert hasattr(lib, name), name


def test_bindings_match_header_arity():
    from alodlm_amd import _lib
    decls = declarations()
    assert set(decls) == set(_lib.SIGNATURES), set(decls) ^ set(_lib.SIGNATURES)
    for name, nargs in decls.items():
        assert len(_lib.SIGNATURES[name]) == nargs, name


def test_library_loads_and_reports_abi():
    from alodlm_amd import _lib
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    assert lib.alodlm_abi_version() == _lib.ABI_VERSION
    # argument validation runs on the host and returns ALODLM_EINVAL without a GPU
    with pytest.raises(ValueError):
        _lib.call("alodlm_objective", None, None, None, None, None, None, None, None, 1, 4, 99,
                  0.4, 0.1, 1.0, None, None, None, None, None)


def test_gemm_workspace_policy():
    """The GEMM workspace query (host only): long-K bf16-output products with
    few output tiles ask for split-K partials, products that fill the chip's
    rounds and float32 outputs do not, and dW products split when their tiles
    are few."""
    from alodlm_amd import _lib
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    q = lambda *a: _lib.query("alodlm_gemm_workspace", *a)
    STORE, ACCUM, BF16, F32 = 0, 2, 1, 0
    # LM head dX at 1.7B (21504 rows, hidden 2048, vocab 151936): 672 tiles, 3 splits
    assert q(21504, 2048, 151936, STORE, BF16) == 3 * 21504 * 2048
    # LM head dX at 8B (about 2700 rows, hidden 4096): 176 tiles, 7 splits
    assert q(2700, 4096, 151936, STORE, BF16) == 7 * 2700 * 4096
    # forward products of the 1.7B step: whole rounds, or K too short to split
    assert q(32768, 12288, 2048, STORE, BF16) == 0
    assert q(4096, 6144, 4096, STORE, BF16) == 0
    assert q(21504, 2048, 151936, STORE, F32) == 0
    # dW of the 1.7B QKV projection (4096 x 2048 over 32768 rows): 128 tiles, split 4
    assert q(4096, 2048, 32768, ACCUM, BF16) == 4 * 4096 * 2048


def test_no_alloc_rmsnorm_bwd_rejects_oversize_on_the_host():
    """The allocation-free RMSNorm backward checks its scratch limit before
    touching the device (32768 x 2048 fits the 4 Mi-float scratch, 65536 x 2048
    does not)."""
    from alodlm_amd import _lib
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    assert _lib.query("alodlm_rmsnorm_bwd_workspace", 32768, 2048) <= 4194304
    assert _lib.query("alodlm_rmsnorm_bwd_workspace", 65536, 2048) > 4194304
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("alodlm_rmsnorm_bwd_noalloc", None, None, None, None, None, None, None,
                  65536, 2048, _lib.BF16_CODE, None)


def test_embed_plan_limits_on_the_host():
    """The embedding plan and scatter reject row counts of 2^24 and more (one
    256-thread workgroup per chunk) before any launch; the plan and workspace
    sizes are linear in the rows."""
    from alodlm_amd import _lib
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    assert _lib.query("alodlm_embed_plan_size", 1000) == 8 + 13 * 1000
    assert _lib.query("alodlm_embed_scatter_workspace", 3200, 64) == (200 + 1) * 64
    with pytest.raises(ValueError, match="rows"):
        _lib.call("alodlm_embed_plan", None, 1 << 24, 151936, None, None)
    with pytest.raises(ValueError, match="shape"):
        _lib.call("alodlm_embed_scatter_add", None, None, None, 0, None, None, 1 << 24, 64,
                  151936, _lib.BF16_CODE, None)
    # zero rows is a no-op that touches nothing
    _lib.call("alodlm_embed_plan", None, 0, 151936, None, None)


def test_ds_block_table_matches_mask():
    """The stored-dS attention backward's block table (host only): the library's
    alodlm_attention_ds_blocks and layers.ds_block_base agree, and per segment
    the 32x32 (query tile, key tile) blocks holding an allowed pair of the
    dense dual-stream mask (alodlm/batch.py:23-31) are exactly T (T + 1),
    T = ceil(L / 32), numbered without gaps or repeats by the kernels'
    clean-first, row-by-row order."""
    import numpy as np
    import torch
    from alodlm_amd import _lib
    from alodlm_amd.batch import attention_mask
    from alodlm_amd.layers import ds_block_base
    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    offsets = np.asarray([0, 1, 33, 97, 225, 288, 640], dtype=np.int64)
    base = np.zeros(len(offsets), dtype=np.int64)
    total = _lib.query("alodlm_attention_ds_blocks", offsets.ctypes.data, len(offsets) - 1, 32,
                       base.ctypes.data)
    assert total == base[-1] and np.array_equal(base, ds_block_base(offsets))
    assert _lib.query("alodlm_attention_ds_blocks", offsets.ctypes.data, len(offsets) - 1, 16,
                      None) == 0
    for a, b in zip(offsets, offsets[1:]):
        L = int(b - a)
        T = (L + 31) // 32
        mask = attention_mask(L, 32, "cpu")
        seen = []
        for qs in (0, L):          # clean, noisy query stream
            for qt in range(T):
                for ks in (0, L):
                    for kt in range(T):
                        q = slice(qs + 32 * qt, min(qs + 32 * qt + 32, qs + L))
                        k = slice(ks + 32 * kt, min(ks + 32 * kt + 32, ks + L))
                        if bool(mask[q, k].any()):
                            seen.append((qs > 0, qt, ks > 0, kt))
        assert len(seen) == T * (T + 1) == base[list(offsets).index(b)] - base[list(offsets).index(a)]
        half = T * (T + 1) // 2
        index = sorted((half if qn else 0) + qt * (qt + 1) // 2 + (qt if kn else kt)
                       for qn, qt, kn, kt in seen)
        assert index == list(range(T * (T + 1)))
        # the clean stream never sees a noisy key; a noisy tile's only noisy
        # key tile is its own
        assert all(qn or not kn for qn, qt, kn, kt in seen)
        assert all(kt == qt for qn, qt, kn, kt in seen if kn)
