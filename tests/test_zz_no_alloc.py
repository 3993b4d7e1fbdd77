"""The allocation-free RMSNorm backward (alodlm_rmsnorm_bwd_noalloc) against
alodlm_rmsnorm_bwd with a caller workspace, through the C ABI: identical bits
for dx and the accumulated weight gradient, on two calls in a row (the second
smaller, so it runs over the first call's leftover scratch), float32 and bf16.
"""

import pytest
import torch

from alodlm_amd import _lib
from tests.helpers import log

pytestmark = pytest.mark.gpu


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    dy = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    dres = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, device="cuda", generator=g)).to(dtype)
    rstd = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-6).contiguous()
    dw0 = torch.randn(cols, device="cuda", generator=g)
    return x, dy, dres, w, rstd, dw0


def _with_workspace(x, dy, dres, w, rstd, dw, rows, cols, code):
    ws = torch.empty(_lib.query("alodlm_rmsnorm_bwd_workspace", rows, cols), device="cuda")
    dx = torch.empty_like(x)
    _lib.call("alodlm_rmsnorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(rstd), _lib.ptr(w),
              _lib.ptr(dres), _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(ws), rows, cols, code,
              _lib.stream_handle())
    return dx


def _no_alloc(x, dy, dres, w, rstd, dw, rows, cols, code):
    dx = torch.empty_like(x)
    _lib.call("alodlm_rmsnorm_bwd_noalloc", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(rstd),
              _lib.ptr(w), _lib.ptr(dres), _lib.ptr(dx), _lib.ptr(dw), rows, cols, code,
              _lib.stream_handle())
    return dx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_no_alloc_rmsnorm_bwd_matches_workspace_entry_point(dtype):
    code = _lib.dtype_code(dtype)
    for call, (rows, cols) in enumerate(((32768, 2048), (1000, 1024))):
        log(f"rmsnorm_bwd_noalloc {dtype} call {call}: {rows} x {cols}")
        x, dy, dres, w, rstd, dw0 = _inputs(rows, cols, dtype, seed=call)
        dw_ref, dw_new = dw0.clone(), dw0.clone()
        dx_ref = _with_workspace(x, dy, dres, w, rstd, dw_ref, rows, cols, code)
        dx_new = _no_alloc(x, dy, dres, w, rstd, dw_new, rows, cols, code)
        torch.cuda.synchronize()
        assert torch.equal(dx_new, dx_ref)
        assert torch.equal(dw_new, dw_ref)
        assert not torch.equal(dw_new, dw0)


def test_no_alloc_rejects_shapes_beyond_its_scratch():
    log("rmsnorm_bwd_noalloc oversize")
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("alodlm_rmsnorm_bwd_noalloc", None, None, None, None, None, None, None,
                  65536, 2048, _lib.BF16_CODE, _lib.stream_handle())
