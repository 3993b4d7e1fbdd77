"""Kernel-level parity of the HIP library against float64 references on the CPU.

Each test calls the C ABI through alodlm_amd._lib on seeded inputs and checks
the result against the oracle's arithmetic (or a torch float64 product for the
GEMM).  bf16 tolerances are stated per test.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import step as O
from tests.helpers import log

pytestmark = pytest.mark.gpu

DEV = "cuda"


def lib():
    from alodlm_amd import _lib
    _lib.load()
    return _lib


def st():
    return torch.cuda.current_stream().cuda_stream


GEMM_CASES = [
    # (M, N, K, a_kmajor, b_kmajor, dtype)
    (256, 256, 128, 1, 1, torch.bfloat16),
    (200, 136, 64, 1, 1, torch.bfloat16),
    (384, 128, 320, 1, 0, torch.bfloat16),
    (128, 264, 192, 0, 1, torch.bfloat16),
    (256, 512, 1000, 0, 0, torch.bfloat16),
    (1040, 256, 1001, 0, 0, torch.bfloat16),   # LM-head dW shape class: K = selected rows
    (768, 640, 320, 1, 0, torch.bfloat16),     # 256x256 tiles with ragged edges
    (520, 768, 256, 0, 1, torch.bfloat16),
    (256, 256, 32, 1, 1, torch.bfloat16),      # one 32-deep k stage
    (512, 264, 64, 0, 0, torch.bfloat16),
    (296, 512, 96, 1, 0, torch.bfloat16),
    (1024, 768, 2048, 0, 1, torch.bfloat16),
    (96, 80, 40, 1, 0, torch.bfloat16),
    (70, 33, 19, 0, 0, torch.float32),
    (130, 65, 48, 1, 1, torch.float32),
]


@pytest.mark.parametrize("M,N,K,ak,bk,dtype", GEMM_CASES)
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_layouts_and_epilogues(M, N, K, ak, bk, dtype, epi):
    L = lib()
    log(f"gemm M={M} N={N} K={K} ak={ak} bk={bk} {dtype} epi={epi}")
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(N, K, generator=g).to(dtype)
    Ad = (A if ak else A.T.contiguous()).to(DEV)
    Bd = (B if bk else B.T.contiguous()).to(DEV)
    lda = K if ak else M
    ldb = K if bk else N
    ref = A.double() @ B.double().T * 0.5
    R = torch.randn(M, N, generator=g).to(dtype)
    if epi == 2:
        C = torch.randn(M, N, generator=g).float().to(DEV)
        expected = C.cpu().double() + ref
        ws_n = L.query("alodlm_gemm_workspace", M, N, K, epi, L.dtype_code(dtype))
        ws = torch.empty(max(ws_n, 1), dtype=torch.float32, device=DEV)
    else:
        C = torch.empty(M, N, dtype=dtype, device=DEV)
        ws = None
        expected = ref if epi == 0 else R.double() + ref.to(dtype).double()
    Rd = R.to(DEV)
    L.call("alodlm_gemm", L.ptr(Ad), lda, ak, L.ptr(Bd), ldb, bk, L.ptr(C), N, L.ptr(Rd), N, M,
           N, K, 0.5, epi, L.dtype_code(dtype), L.ptr(ws), st())
    torch.cuda.synchronize()
    out = C.cpu().double()
    scale = ref.abs().max().item() + 1e-6
    tol = 1e-5 if (dtype == torch.float32 or epi == 2) else 8e-3
    err = (out - expected).abs().max().item() / scale
    assert err <= tol, f"max rel err {err}"


@pytest.mark.parametrize("M,N,K,ak,bk", [
    (4352, 4160, 64, 0, 1),    # 17 x 17 tiles (more than one per workgroup), ragged edges
    (4096, 4608, 96, 1, 0),    # 16 x 18 tiles, a multiple of 8 (per-XCD tile chunks)
    (4160, 4096, 96, 1, 1),
    (4096, 4352, 64, 1, 1),    # 64-deep kernel
    (4608, 4096, 32, 0, 0),
])
@pytest.mark.parametrize("epi,alpha", [(0, 1.0), (0, 0.5), (1, 1.0), (2, 0.5)])
def test_gemm_many_tiles(M, N, K, ak, bk, epi, alpha):
    L = lib()
    log(f"gemm many tiles M={M} N={N} K={K} ak={ak} bk={bk} epi={epi} alpha={alpha}")
    g = torch.Generator().manual_seed(M + N + K + epi)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = torch.randn(N, K, generator=g).to(torch.bfloat16)
    Ad = (A if ak else A.T.contiguous()).to(DEV)
    Bd = (B if bk else B.T.contiguous()).to(DEV)
    ref = (A.float() @ B.float().T).double() * alpha
    R = torch.randn(M, N, generator=g).to(torch.bfloat16)
    if epi == 2:
        C = torch.randn(M, N, generator=g).to(DEV)
        expected = C.cpu().double() + ref
        ws = torch.empty(max(L.query("alodlm_gemm_workspace", M, N, K, epi, 1), 1),
                         dtype=torch.float32, device=DEV)
    else:
        C = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        ws = None
        expected = ref if epi == 0 else R.double() + ref.to(torch.bfloat16).double()
    Rd = R.to(DEV)
    L.call("alodlm_gemm", L.ptr(Ad), K if ak else M, ak, L.ptr(Bd), K if bk else N, bk, L.ptr(C),
           N, L.ptr(Rd), N, M, N, K, alpha, epi, 1, L.ptr(ws), st())
    torch.cuda.synchronize()
    err = (C.cpu().double() - expected).abs().max().item() / (ref.abs().max().item() + 1e-6)
    assert err <= (1e-5 if epi == 2 else 8e-3), f"max rel err {err}"


@pytest.mark.parametrize("M,N", [(512, 512), (300, 260)])
def test_gemm_store_splitk_long_k(M, N):
    """A bf16-output product with few output tiles and a long K (the LM head's
    dX shape: dlogits [rows, V] times the head weight) is split over K; the
    float partials are summed in split order and rounded once."""
    L = lib()
    K = 20480
    log(f"gemm store splitk M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M + N)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    Bt = torch.randn(K, N, generator=g).to(torch.bfloat16)  # n-contiguous like the head weight
    ws_n = L.query("alodlm_gemm_workspace", M, N, K, 0, 1)
    assert ws_n >= 2 * M * N, "the long-K product should be split"
    ws = torch.empty(ws_n, dtype=torch.float32, device=DEV)
    Ad, Bd = A.to(DEV), Bt.to(DEV)
    C = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    L.call("alodlm_gemm", L.ptr(Ad), K, 1, L.ptr(Bd), N, 0, L.ptr(C), N, None, 0, M, N, K, 0.5,
           0, 1, L.ptr(ws), st())
    torch.cuda.synchronize()
    ref = (A.double() @ Bt.double()) * 0.5
    scale = ref.abs().max().item()
    err = (C.cpu().double() - ref).abs().max().item() / scale
    assert err <= 8e-3, f"max rel err {err}"
    # the same product without a workspace runs unsplit: equal within bf16 rounding
    C1 = torch.empty_like(C)
    L.call("alodlm_gemm", L.ptr(Ad), K, 1, L.ptr(Bd), N, 0, L.ptr(C1), N, None, 0, M, N, K, 0.5,
           0, 1, None, st())
    torch.cuda.synchronize()
    assert (C1.cpu().double() - C.cpu().double()).abs().max().item() <= 8e-3 * scale


@pytest.mark.parametrize("epi", [2, 3])
@pytest.mark.parametrize("M,N,K", [(256, 384, 8192), (512, 512, 16384)])
def test_gemm_splitk_accumulates_large_k(M, N, K, epi):
    """dW-shaped products (both operands m/n-contiguous, long K) use split-K:
    accumulated into a float32 C holding ones (ALODLM_EPI_ACCUM: split 0 adds
    into C itself, the others' partials are added after), or written over a
    C holding garbage (ALODLM_EPI_STORE_F32); the same bits on a second run."""
    L = lib()
    log(f"gemm splitk M={M} N={N} K={K} epi={epi}")
    g = torch.Generator().manual_seed(5)
    dY = torch.randn(K, M, generator=g).to(torch.bfloat16)
    X = torch.randn(K, N, generator=g).to(torch.bfloat16)
    need = L.query("alodlm_gemm_workspace", M, N, K, epi, 1)
    assert need >= 2 * M * N, "the product should be split"
    ws = torch.empty(need, dtype=torch.float32, device=DEV)
    dYd, Xd = dY.to(DEV), X.to(DEV)  # named: the pointers must outlive the call
    outs = []
    for _ in range(2):
        C = torch.full((M, N), 1.0 if epi == 2 else float("nan"), dtype=torch.float32,
                       device=DEV)
        L.call("alodlm_gemm", L.ptr(dYd), M, 0, L.ptr(Xd), N, 0, L.ptr(C), N, None, 0,
               M, N, K, 1.0, epi, 1, L.ptr(ws), st())
        torch.cuda.synchronize()
        outs.append(C.cpu())
    ref = (1.0 if epi == 2 else 0.0) + dY.double().T @ X.double()
    err = (outs[0].double() - ref).abs().max().item() / ref.abs().max().item()
    assert err < 1e-5
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (70, 130), (64, 64), (4096, 2048), (2048, 6144),
                                       (1000, 33), (72, 136), (8, 4096)])
def test_transpose(dtype, rows, cols):
    """Weight transposes (exact: a permutation of the elements)."""
    L = lib()
    log(f"transpose rows={rows} cols={cols} {dtype}")
    g = torch.Generator().manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype).to(DEV)
    y = torch.full((cols, rows), float("nan"), dtype=dtype, device=DEV)
    L.call("alodlm_transpose", L.ptr(x), L.ptr(y), rows, cols, L.dtype_code(dtype), st())
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.cpu().T)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,offset", [(1, 0), (1000, 0), (1000, 1), (4096 * 2048 + 5, 0),
                                      (151936 * 2048, 0)])
def test_check_finite(dtype, n, offset):
    """The LM-head finiteness scan: the flag is set by one inf or NaN anywhere
    (first, last, middle element, the unaligned tail), stays 0 on finite
    data (the largest finite values included) and is never cleared."""
    L = lib()
    log(f"check_finite n={n} offset={offset} {dtype}")
    code = L.dtype_code(dtype)
    buf = torch.zeros(n + offset, dtype=dtype, device=DEV)
    x = buf[offset:]
    x[::max(1, n // 7)] = torch.finfo(dtype).max
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)

    def scan():
        flag.zero_()
        L.call("alodlm_check_finite", L.ptr(x), n, code, L.ptr(flag), st())
        torch.cuda.synchronize()
        return int(flag.item())

    assert scan() == 0
    for pos in sorted({0, n // 2, n - 1}):
        for bad in (float("inf"), float("-inf"), float("nan")):
            x[pos] = bad
            assert scan() == 1, (pos, bad)
            x[pos] = 0
    assert scan() == 0
    flag.fill_(1)
    L.call("alodlm_check_finite", L.ptr(x), n, code, L.ptr(flag), st())
    torch.cuda.synchronize()
    assert int(flag.item()) == 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,offset", [(1, 0), (13, 0), (1000, 1), (4096 * 2048 + 5, 0),
                                      (4096 * 2048 + 5, 3)])
def test_scale_in_place(dtype, n, offset):
    """x *= s[0] in place, rounded to the storage type once, on 16-byte pieces
    and the element tail (and a start that is not 16-byte aligned)."""
    L = lib()
    log(f"scale n={n} offset={offset} {dtype}")
    g = torch.Generator().manual_seed(n + offset)
    x = torch.randn(n + offset, generator=g).to(dtype)
    k = torch.tensor([0.37], dtype=torch.float32)
    xd, kd = x.to(DEV), k.to(DEV)
    L.call("alodlm_scale", L.ptr(xd[offset:]), L.ptr(kd), n, L.dtype_code(dtype), st())
    torch.cuda.synchronize()
    expected = x.clone()
    expected[offset:] = (x[offset:].float() * k[0]).to(dtype)
    assert torch.equal(xd.cpu(), expected)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,H,n_sel", [(300, 2048, 123), (50, 13, 20), (70000, 8, 66000),
                                          (40, 151936, 7)])
def test_gather_scatter_rows(dtype, rows, H, n_sel):
    """Row gather (dst[j] = src[sel[j]]) and scatter (dst zeroed, then
    dst[sel[j]] = src[j]) against torch indexing: 16-byte row moves, the
    element path (rows of 13), more selected rows than one launch takes."""
    L = lib()
    log(f"gather/scatter rows={rows} H={H} n_sel={n_sel} {dtype}")
    g = torch.Generator().manual_seed(rows + H)
    src = torch.randn(rows, H, generator=g).to(dtype)
    sel = torch.randperm(rows, generator=g)[:n_sel].sort().values.to(torch.int32)
    src_d, sel_d = src.to(DEV), sel.to(DEV)
    code = L.dtype_code(dtype)
    out = torch.empty(n_sel, H, dtype=dtype, device=DEV)
    L.call("alodlm_gather_rows", L.ptr(src_d), L.ptr(sel_d), n_sel, L.ptr(out), H, code, st())
    back = torch.full((rows, H), 7.0, dtype=dtype, device=DEV)
    L.call("alodlm_scatter_rows", L.ptr(out), L.ptr(sel_d), n_sel, L.ptr(back), rows, H, code,
           st())
    torch.cuda.synchronize()
    idx = sel.long()
    assert torch.equal(out.cpu(), src[idx])
    expected = torch.zeros(rows, H, dtype=dtype)
    expected[idx] = src[idx]
    assert torch.equal(back.cpu(), expected)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,inter", [(3, 8), (37, 768), (5, 13),
                                        # two column blocks per row, the second ragged;
                                        # more rows than one launch takes (65535)
                                        (300, 2056), (70001, 16)])
def test_swiglu_fwd_bwd(dtype, rows, inter):
    """SwiGLU against torch float64 ([tf] modeling_qwen3.py:81-83 with the
    reference's roundings); the product written by the backward is
    bit-identical to the forward's."""
    L = lib()
    log(f"swiglu rows={rows} inter={inter} {dtype}")
    g = torch.Generator().manual_seed(rows + inter)
    gu = (2 * torch.randn(rows, 2 * inter, generator=g)).to(dtype)
    dact = torch.randn(rows, inter, generator=g).to(dtype)
    gud, dactd = gu.to(DEV), dact.to(DEV)
    code = L.dtype_code(dtype)
    act = torch.empty(rows, inter, dtype=dtype, device=DEV)
    L.call("alodlm_swiglu_fwd", L.ptr(gud), L.ptr(act), rows, inter, code, st())
    dgu = torch.empty(rows, 2 * inter, dtype=dtype, device=DEV)
    act2 = torch.empty(rows, inter, dtype=dtype, device=DEV)
    L.call("alodlm_swiglu_bwd", L.ptr(dactd), L.ptr(gud), L.ptr(dgu), L.ptr(act2), rows, inter,
           code, st())
    dgu_noact = torch.empty(rows, 2 * inter, dtype=dtype, device=DEV)
    L.call("alodlm_swiglu_bwd", L.ptr(dactd), L.ptr(gud), L.ptr(dgu_noact), None, rows, inter,
           code, st())
    torch.cuda.synchronize()
    assert torch.equal(act2.cpu(), act.cpu())
    assert torch.equal(dgu_noact.cpu(), dgu.cpu())
    gate = gu[:, :inter].double().requires_grad_(True)
    up = gu[:, inter:].double().requires_grad_(True)
    silu = F.silu(gate)
    ref = silu.to(dtype).double() * up if dtype != torch.float32 else silu * up
    dg, du = torch.autograd.grad(ref, (gate, up), dact.double())
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(act.cpu().double(), ref.detach(), rtol=tol, atol=tol)
    torch.testing.assert_close(dgu.cpu().double()[:, :inter], dg, rtol=tol, atol=tol)
    torch.testing.assert_close(dgu.cpu().double()[:, inter:], du, rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(37, 256), (64, 2048), (5, 100), (129, 4096), (1000, 2048),
                                       (140000, 64)])
def test_rmsnorm_fwd_bwd(dtype, rows, cols):
    L = lib()
    log(f"rmsnorm rows={rows} cols={cols} {dtype}")
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    dres = torch.randn(rows, cols, generator=g).to(dtype)
    xd, wd, dyd, dresd = (t.to(DEV) for t in (x, w, dy, dres))
    y = torch.empty_like(xd)
    rstd = torch.empty(rows, dtype=torch.float32, device=DEV)
    code = L.dtype_code(dtype)
    L.call("alodlm_rmsnorm_fwd", L.ptr(xd), L.ptr(wd), L.ptr(y), L.ptr(rstd), rows, cols, 1e-6,
           code, st())
    dx = torch.empty_like(xd)
    dw = torch.zeros(cols, dtype=torch.float32, device=DEV)
    ws = torch.empty(L.query("alodlm_rmsnorm_bwd_workspace", rows, cols), dtype=torch.float32,
                     device=DEV)
    L.call("alodlm_rmsnorm_bwd", L.ptr(dyd), L.ptr(xd), L.ptr(rstd), L.ptr(wd), L.ptr(dresd),
           L.ptr(dx), L.ptr(dw), L.ptr(ws), rows, cols, code, st())
    torch.cuda.synchronize()
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    yr = O.rmsnorm(xr, wr, 1e-6)
    gx, gw = torch.autograd.grad(yr, (xr, wr), dy.double())
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(y.cpu().double(), yr.detach(), rtol=tol, atol=tol)
    torch.testing.assert_close(dx.cpu().double(), gx + dres.double(), rtol=tol, atol=tol * 4)
    torch.testing.assert_close(dw.cpu().double(), gw, rtol=tol, atol=tol * math.sqrt(rows))


def _dual_stream(bounds_tokens, block, seed):
    """Random dual-stream positions for a pack (clean positions 0..L-1, noisy
    positions a per-block permutation)."""
    g = torch.Generator().manual_seed(seed)
    pos, seg = [], []
    for s, (a, b) in enumerate(zip(bounds_tokens, bounds_tokens[1:])):
        L = b - a
        pos.append(torch.arange(L))
        noisy = []
        for left in range(0, L, block):
            right = min(left + block, L)
            noisy.append(left + torch.randperm(right - left, generator=g))
        pos.append(torch.cat(noisy))
        seg += [s] * (2 * L)
    packed = [2 * v for v in bounds_tokens]
    return torch.cat(pos), torch.tensor(seg, dtype=torch.int32), torch.tensor(packed)


ATTN_CASES = [
    # (dtype, nq, nkv, dh, token bounds, block, path)
    (torch.float32, 4, 2, 64, [0, 40, 41, 100], 8, "ref"),
    (torch.float32, 2, 1, 128, [0, 64, 160], 32, "ref"),
    (torch.float32, 4, 4, 8, [0, 7, 20], 3, "ref"),
    (torch.bfloat16, 4, 2, 64, [0, 40, 41, 100], 8, "ref"),
    (torch.bfloat16, 2, 1, 128, [0, 64, 160], 32, "ref"),
    (torch.bfloat16, 4, 2, 64, [0, 40, 41, 100], 8, "mfma"),
    (torch.bfloat16, 2, 1, 128, [0, 64, 160], 32, "mfma"),
    (torch.bfloat16, 4, 1, 128, [0, 300, 333], 32, "mfma"),
    (torch.bfloat16, 2, 2, 64, [0, 200, 390], 24, "mfma"),
    (torch.bfloat16, 2, 1, 128, [0, 1024], 32, "mfma"),
    (torch.bfloat16, 4, 2, 128, [0, 512, 1000, 1001], 32, "mfma"),
    # 21 heads: the q/k-norm kernels load several groups of four heads per
    # pass (a partial last group, and more than one pass per row)
    (torch.bfloat16, 18, 3, 128, [0, 100, 133], 32, "mfma"),
    # head_dim 128 with the dQ pass that recomputes S, P and dP (no stored dS)
    (torch.bfloat16, 4, 1, 128, [0, 300, 333], 32, "mfma-recompute"),
    (torch.bfloat16, 4, 2, 128, [0, 512, 1000, 1001], 32, "mfma-recompute"),
]


def _ds_table(L, bounds, block):
    """(device ds_base, ds_blocks) of the stored-dS backward from the
    library's host helper (ds_blocks is 0 unless block is 32)."""
    import numpy as np
    offs = np.asarray(bounds, dtype=np.int64)
    base = np.zeros(len(bounds), dtype=np.int64)
    n = L.query("alodlm_attention_ds_blocks", offs.ctypes.data, len(bounds) - 1, block,
                base.ctypes.data)
    return (torch.from_numpy(base).to(DEV) if n else None), n


@pytest.mark.parametrize("dtype,nq,nkv,dh,bounds,block,path", ATTN_CASES)
def test_qknorm_rope_attention_fwd_bwd(dtype, nq, nkv, dh, bounds, block, path):
    """Attention (dual-stream mask) with q/k norm + rotary, forward and backward,
    against autograd through the oracle's restatement in float64.  `path`
    selects the reference kernels (no tile table) or the MFMA flash kernels
    (with block size 32 and head_dim 128 the dK/dV pass stores dS and dQ is
    one dS*K product; "mfma-recompute" runs the dQ pass that recomputes)."""
    from alodlm_amd.batch import attention_tiles
    L = lib()
    log(f"attention nq={nq} nkv={nkv} dh={dh} bounds={bounds} block={block} {dtype} {path}")
    tiles = torch.tensor(attention_tiles(bounds), dtype=torch.int32).view(-1, 2).to(DEV)
    tiles_ptr = L.ptr(tiles) if path.startswith("mfma") else None
    ds_base, ds_blocks = _ds_table(L, bounds, block) if path == "mfma" else (None, 0)
    g = torch.Generator().manual_seed(dh + nq)
    positions, row_seg, packed = _dual_stream(bounds, block, dh)
    N = len(positions)
    W = (nq + 2 * nkv) * dh
    qkv = torch.randn(N, W, generator=g).to(dtype)
    wq = (1 + 0.2 * torch.randn(dh, generator=g)).to(dtype)
    wk = (1 + 0.2 * torch.randn(dh, generator=g)).to(dtype)
    dout = torch.randn(N, nq * dh, generator=g).to(dtype)
    code = L.dtype_code(dtype)
    theta = 1e4
    inv = (1.0 / (theta ** (torch.arange(0, dh, 2, dtype=torch.float32) / dh))).to(DEV)
    qkv_d, wq_d, wk_d = qkv.to(DEV), wq.to(DEV), wk.to(DEV)
    pos_d, seg_d, bnd_d = positions.to(DEV), row_seg.to(DEV), packed.to(DEV)
    q = torch.empty(N, nq * dh, dtype=dtype, device=DEV)
    k = torch.empty(N, nkv * dh, dtype=dtype, device=DEV)
    L.call("alodlm_qknorm_rope_fwd", L.ptr(qkv_d), L.ptr(wq_d), L.ptr(wk_d), L.ptr(pos_d),
           L.ptr(inv), L.ptr(q), L.ptr(k), N, nq, nkv, dh, 1e-6, code, st())
    v = qkv_d[:, (nq + nkv) * dh:]
    o = torch.empty(N, nq * dh, dtype=dtype, device=DEV)
    lse = torch.empty(nq, N, dtype=torch.float32, device=DEV)
    L.call("alodlm_attention_fwd", L.ptr(q), L.ptr(k), L.ptr(v), W, L.ptr(bnd_d), L.ptr(seg_d),
           tiles_ptr, tiles.shape[0], L.ptr(o), L.ptr(lse), N, nq, nkv, dh, block, code, st())
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dqkv = torch.zeros(N, W, dtype=dtype, device=DEV)
    ws = torch.empty(L.query("alodlm_attention_bwd_workspace", N, nq, nkv, dh, tiles.shape[0],
                             ds_blocks),
                     dtype=torch.float32,
                     device=DEV)
    dout_d = dout.to(DEV)
    L.call("alodlm_attention_bwd", L.ptr(q), L.ptr(k), L.ptr(v), W, L.ptr(o), L.ptr(lse),
           L.ptr(dout_d), L.ptr(bnd_d), L.ptr(seg_d), tiles_ptr, tiles.shape[0], L.ptr(dq),
           L.ptr(dk), L.ptr(dqkv[:, (nq + nkv) * dh:]), W, L.ptr(ws), L.ptr(ds_base), ds_blocks,
           N, nq, nkv, dh, block, code, st())
    dwq = torch.zeros(dh, dtype=torch.float32, device=DEV)
    dwk = torch.zeros(dh, dtype=torch.float32, device=DEV)
    ws2 = torch.empty(L.query("alodlm_qknorm_rope_bwd_workspace", N, nq, nkv, dh) * 2 + 16,
                      dtype=torch.float32, device=DEV)
    L.call("alodlm_qknorm_rope_bwd", L.ptr(dq), L.ptr(dk), L.ptr(qkv_d), L.ptr(wq_d), L.ptr(wk_d),
           L.ptr(pos_d), L.ptr(inv), L.ptr(dqkv), L.ptr(dwq), L.ptr(dwk), L.ptr(ws2), N, nq, nkv,
           dh, 1e-6, code, st())
    torch.cuda.synchronize()
    # float64 reference through the oracle's formulas
    X = qkv.double().requires_grad_(True)
    WQ = wq.double().requires_grad_(True)
    WK = wk.double().requires_grad_(True)
    qr = O.rmsnorm(X[:, :nq * dh].reshape(N, nq, dh), WQ, 1e-6)
    kr = O.rmsnorm(X[:, nq * dh:(nq + nkv) * dh].reshape(N, nkv, dh), WK, 1e-6)
    cos, sin = O.rope_tables(positions, dh, theta, torch.float64)
    rot = lambda t: torch.cat((-t[..., dh // 2:], t[..., :dh // 2]), -1)
    qr = qr * cos[:, None] + rot(qr) * sin[:, None]
    kr = kr * cos[:, None] + rot(kr) * sin[:, None]
    vr = X[:, (nq + nkv) * dh:].reshape(N, nkv, dh)
    mask = torch.as_tensor(O.packed_attention_mask(packed, block))
    heads = []
    for h in range(nq):
        s = (qr[:, h] @ kr[:, h // (nq // nkv)].T) * dh ** -0.5
        heads.append(torch.softmax(s.masked_fill(~mask, float("-inf")), -1) @ vr[:, h // (nq // nkv)])
    ref_o = torch.stack(heads, 1).reshape(N, nq * dh)
    gX, gWQ, gWK = torch.autograd.grad(ref_o, (X, WQ, WK), dout.double())
    tol = 2e-5 if dtype == torch.float32 else 3e-2
    torch.testing.assert_close(q.cpu().double(), qr.detach().reshape(N, -1), rtol=tol, atol=tol)
    torch.testing.assert_close(o.cpu().double(), ref_o.detach(), rtol=tol, atol=tol)
    scale = gX.abs().max().item()
    assert (dqkv.cpu().double() - gX).abs().max().item() <= tol * 2 * scale
    sw = max(gWQ.abs().max().item(), gWK.abs().max().item())
    assert (dwq.cpu().double() - gWQ).abs().max().item() <= tol * 2 * sw
    assert (dwk.cpu().double() - gWK).abs().max().item() <= tol * 2 * sw


@pytest.mark.parametrize("dtype,V", [(torch.float32, 1000), (torch.bfloat16, 1000),
                                     (torch.bfloat16, 151936), (torch.bfloat16, 100000)])
def test_cross_entropy_rows(dtype, V):
    """Small vocabularies take the two-pass kernel; bf16 rows of 81921..155648
    logits the register-resident one (151936: Qwen3's vocabulary; 100000: a
    row that ends inside a thread's chunk)."""
    L = lib()
    R = 37
    log(f"cross_entropy R={R} V={V} {dtype}")
    g = torch.Generator().manual_seed(9)
    logits = (3 * torch.randn(R, V, generator=g)).to(dtype)
    target = torch.randint(0, V, (R,), generator=g, dtype=torch.int32)
    coef = torch.rand(R, generator=g)
    ld = logits.to(DEV).contiguous()
    count = torch.tensor([R - 3], dtype=torch.int32, device=DEV)
    ce = torch.zeros(R, dtype=torch.float32, device=DEV)
    ent = torch.zeros(R, dtype=torch.float32, device=DEV)
    target_d, coef_d = target.to(DEV), coef.to(DEV)
    L.call("alodlm_cross_entropy", L.ptr(ld), L.ptr(target_d), L.ptr(coef_d),
           L.ptr(count), R, V, L.ptr(ce), L.ptr(ent), L.dtype_code(dtype), st())
    torch.cuda.synchronize()
    x = logits.double()[:R - 3]
    ref_ce = F.cross_entropy(x, target[:R - 3].long(), reduction="none")
    p = torch.softmax(x, -1)
    ref_ent = -(p * torch.log_softmax(x, -1)).sum(-1)
    grad = coef[:R - 3, None].double() * (p - F.one_hot(target[:R - 3].long(), V).double())
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(ce.cpu()[:R - 3].double(), ref_ce, rtol=tol, atol=tol)
    torch.testing.assert_close(ent.cpu()[:R - 3].double(), ref_ent, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(ld.cpu()[:R - 3].double(), grad, rtol=tol, atol=tol * 0.01)
    torch.testing.assert_close(ld.cpu()[R - 3:], logits[R - 3:])  # rows past the count untouched


@pytest.mark.parametrize("K,depths", [(3, [1, 2, 3, 2]), (4, [4, 1, 3, 2])])
def test_objective_kernel_matches_oracle(K, depths):
    """The objective kernel against the oracle's outcome loss (itself pinned by
    the reference's analytic restatement, test_objective.py:32-74)."""
    L = lib()
    log(f"objective K={K}")
    cfg = O.Objective(max_depth=K, gate_init_pi=(1 / K,) * K)
    base = [[3., 4., 5., 6.], [2., 3., 3., 4.], [1., 2., 2., 3.], [1.5, .5, 2.5, 1.]]
    # embed the 4 masked rows in 9 rows with 3 segments; rows 0,1,5 are AR rows
    rows = 9
    masked = torch.zeros(rows, dtype=torch.bool)
    mrows = [2, 3, 6, 8]
    masked[mrows] = True
    ce_m = torch.tensor(base[:K], dtype=torch.float64, requires_grad=True)
    gates_m = torch.tensor([[-.4, .2, -.3, .7], [.1, -.6, .9, .0], [.3, .3, -.2, -.8],
                            [0., 0., 0., 0.]][:K], dtype=torch.float64, requires_grad=True)
    gates_full = torch.zeros(K, rows, dtype=torch.float64)
    gates_full[:, mrows] = gates_m.detach()
    gates_full[:, [0, 1]] = 0.3
    ce_full = torch.zeros(K, rows, dtype=torch.float64)
    ce_full[:, mrows] = ce_m.detach()
    ar_target = torch.full((rows,), -1, dtype=torch.int32)
    ar_target[[0, 1, 5]] = 7
    ce_full[:, [0, 1, 5]] = torch.tensor([[1.0, 2.0, 3.0]] * K, dtype=torch.float64)
    exits = torch.full((rows,), K, dtype=torch.int64)
    exits[mrows] = torch.tensor(depths)
    prob = torch.zeros(rows)
    prob[mrows] = torch.tensor([.2, .4, .5, .8])
    bounds = torch.tensor([0, 4, 7, 9])
    # oracle (float64)
    gate_list = [gates_full[d].clone() for d in range(K)]
    for d in range(K):
        gate_list[d] = gate_list[d].index_put((torch.tensor(mrows),), gates_m[d])
    ref, metrics = O.outcome_loss(ce_m, gate_list, exits, masked, prob.double(), bounds, cfg)
    ar = ce_full[:, [0, 1, 5]].sum() / (3 * K)
    total = (ref + ar) / 2
    dg = torch.autograd.grad(total, gates_m)[0]
    out = torch.zeros(10, dtype=torch.float32, device=DEV)
    dgate = torch.zeros(K, rows, dtype=torch.float32, device=DEV)
    ws = torch.empty(L.query("alodlm_objective_workspace", rows, 3, K), dtype=torch.float32,
                     device=DEV)
    cfd = ce_full.float().to(DEV)
    gd, ed, md, pd = (gates_full.float().to(DEV), exits.int().to(DEV), masked.to(DEV),
                      prob.to(DEV))
    ad, bd = ar_target.to(DEV), bounds.to(DEV)
    L.call("alodlm_objective", L.ptr(gd), L.ptr(ed), L.ptr(md), L.ptr(pd), L.ptr(cfd), L.ptr(cfd),
           L.ptr(ad), L.ptr(bd), 3, rows, K, cfg.depth_prior_c,
           cfg.kl_beta_mi, cfg.kl_beta_marg, None, L.ptr(out), L.ptr(dgate), L.ptr(ws), st())
    torch.cuda.synchronize()
    out = out.cpu().double()
    assert abs(out[0] - total.item()) < 1e-5 * max(1, abs(total.item()))
    names = ["denoising", "actor", "sampled_mean_depth", "prediction_cost",
             "regularization_cost", "profile_mean_depth", "first_pass_halt_probability"]
    for i, name in enumerate(names, 1):
        assert abs(out[i] - metrics[name].item()) < 1e-5 * max(1, abs(metrics[name].item())), name
    assert abs(out[8] - ar.item()) < 1e-6
    torch.testing.assert_close(dgate.cpu().double()[:, mrows], dg, rtol=1e-5, atol=1e-7)
    assert (dgate.cpu()[:, [0, 1, 4, 5, 7]] == 0).all()


def test_cast_covers_more_than_2_32_elements():
    """The float32 -> bf16 gradient cast sweeps arenas beyond 2^32 elements (the
    8B arena holds 8.2 G); a one-thread-per-element dispatch would cover only
    n mod 2^32 of them."""
    L = lib()
    n = (1 << 32) + 4096 * 3
    log(f"cast n={n}")
    src = torch.full((n,), 1.5, dtype=torch.float32, device=DEV)
    src[-8192:] = 2.5
    dst = torch.zeros(n, dtype=torch.bfloat16, device=DEV)
    seed = torch.tensor([2.0], dtype=torch.float32, device=DEV)
    L.call("alodlm_cast_f32", L.ptr(src), L.ptr(seed), L.ptr(dst), n, 1, st())
    torch.cuda.synchronize()
    assert float(dst[0]) == 3.0
    assert torch.equal(dst[(1 << 32) - 8:(1 << 32) + 8].float().cpu(), torch.full((16,), 3.0))
    assert torch.equal(dst[-8192:].float().cpu(), torch.full((8192,), 5.0))
    del src, dst
    torch.cuda.empty_cache()


@pytest.mark.parametrize("stored", [True, False])
@pytest.mark.parametrize("seg_len,n_seg", [(1024, 8), (2048, 1)])
def test_attention_fa128_large_packs_against_torch_fp32(seg_len, n_seg, stored):
    """head_dim-128 attention at the 1.7B head layout (16 q / 8 kv heads) on
    long packs: 8 x 1024 tokens keeps one dK/dV workgroup per (kv head, key
    tile); 1 x 2048 splits the dK/dV work by query head and reduces the float32
    partials; `stored`: dQ from the dS the dK/dV pass stores, else the dQ pass
    that recomputes.  Reference: torch float32 autograd per segment under the
    dual-stream mask (alodlm/batch.py:23-31), on the GPU."""
    from alodlm_amd.batch import attention_mask, attention_tiles
    L = lib()
    nq, nkv, dh, block = 16, 8, 128, 32
    log(f"attention fa128 large pack seg_len={seg_len} n_seg={n_seg} stored={stored}")
    bounds = [i * seg_len for i in range(n_seg + 1)]
    N = 2 * bounds[-1]
    tiles = torch.tensor(attention_tiles(bounds), dtype=torch.int32).view(-1, 2).to(DEV)
    packed = torch.tensor([2 * b for b in bounds], dtype=torch.int64, device=DEV)
    seg = torch.repeat_interleave(torch.arange(n_seg, dtype=torch.int32), 2 * seg_len).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(seg_len + n_seg)
    W = (nq + 2 * nkv) * dh
    qkv = torch.randn(N, W, device=DEV, generator=g).to(torch.bfloat16)
    q = qkv[:, :nq * dh].contiguous()
    k = qkv[:, nq * dh:(nq + nkv) * dh].contiguous()
    v = qkv[:, (nq + nkv) * dh:]
    dout = torch.randn(N, nq * dh, device=DEV, generator=g).to(torch.bfloat16)
    o = torch.empty(N, nq * dh, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(nq, N, dtype=torch.float32, device=DEV)
    L.call("alodlm_attention_fwd", L.ptr(q), L.ptr(k), L.ptr(v), W, L.ptr(packed), L.ptr(seg),
           L.ptr(tiles), tiles.shape[0], L.ptr(o), L.ptr(lse), N, nq, nkv, dh, block, 1, st())
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dqkv = torch.zeros(N, W, dtype=torch.bfloat16, device=DEV)
    ds_base, ds_blocks = _ds_table(L, bounds, block) if stored else (None, 0)
    assert not stored or ds_blocks == n_seg * (seg_len // 32) * (seg_len // 32 + 1)
    ws = torch.empty(L.query("alodlm_attention_bwd_workspace", N, nq, nkv, dh, tiles.shape[0],
                             ds_blocks),
                     dtype=torch.float32, device=DEV)
    L.call("alodlm_attention_bwd", L.ptr(q), L.ptr(k), L.ptr(v), W, L.ptr(o), L.ptr(lse),
           L.ptr(dout), L.ptr(packed), L.ptr(seg), L.ptr(tiles), tiles.shape[0], L.ptr(dq),
           L.ptr(dk), L.ptr(dqkv[:, (nq + nkv) * dh:]), W, L.ptr(ws), L.ptr(ds_base), ds_blocks,
           N, nq, nkv, dh, block, 1, st())
    torch.cuda.synchronize()
    dv = dqkv[:, (nq + nkv) * dh:]
    mask = attention_mask(seg_len, block, DEV)
    errs = {}
    for s in range(n_seg):
        rows = slice(2 * bounds[s], 2 * bounds[s + 1])
        qs = q[rows].float().view(-1, nq, dh).transpose(0, 1).contiguous().requires_grad_(True)
        ks = k[rows].float().view(-1, nkv, dh).transpose(0, 1).contiguous().requires_grad_(True)
        vs = v[rows].float().reshape(-1, nkv, dh).transpose(0, 1).contiguous().requires_grad_(True)
        kr = ks.repeat_interleave(nq // nkv, 0)
        vr = vs.repeat_interleave(nq // nkv, 0)
        sc = torch.matmul(qs, kr.transpose(1, 2).contiguous()) * dh ** -0.5
        p = torch.softmax(sc.masked_fill(~mask, float("-inf")), -1)
        ref = torch.matmul(p, vr)
        go = dout[rows].float().view(-1, nq, dh).transpose(0, 1).contiguous()
        gq, gk, gv = torch.autograd.grad(ref, (qs, ks, vs), go)
        pairs = {"o": (o[rows], ref.detach().transpose(0, 1).reshape(-1, nq * dh)),
                 "dq": (dq[rows], gq.transpose(0, 1).reshape(-1, nq * dh)),
                 "dk": (dk[rows], gk.transpose(0, 1).reshape(-1, nkv * dh)),
                 "dv": (dv[rows], gv.transpose(0, 1).reshape(-1, nkv * dh))}
        for name, (got, want) in pairs.items():
            e = ((got.float() - want).abs().max() / want.abs().max()).item()
            errs[name] = max(errs.get(name, 0.0), e)
    assert all(e <= 2e-2 for e in errs.values()), errs


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,offset,scaled", [(1003, 0, True), (1003, 1, False), (64, 0, False),
                                             (100000, 0, True)])
def test_cast_tail_and_alignment(dtype, n, offset, scaled):
    """float32 -> dtype cast, with and without the device scale, over lengths
    that leave a tail after the 8-wide pieces and over unaligned buffers."""
    L = lib()
    log(f"cast n={n} offset={offset} scaled={scaled} {dtype}")
    g = torch.Generator().manual_seed(n + offset)
    src_all = torch.randn(n + offset, generator=g).to(DEV)
    dst_all = torch.zeros(n + offset, dtype=dtype, device=DEV)
    src, dst = src_all[offset:], dst_all[offset:]
    seed = torch.tensor([-0.75], dtype=torch.float32, device=DEV) if scaled else None
    L.call("alodlm_cast_f32", L.ptr(src), L.ptr(seed), L.ptr(dst), n, L.dtype_code(dtype), st())
    torch.cuda.synchronize()
    want = (src * -0.75 if scaled else src).to(dtype)
    assert torch.equal(dst.cpu(), want.cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_grad_norm_chunks(dtype):
    """Global L2 norm over a tensor list whose sizes leave ragged chunk tails
    (torch.nn.utils.clip_grad_norm_'s total norm)."""
    from alodlm_amd.optim import CHUNK, _Table
    L = lib()
    g = torch.Generator().manual_seed(3)
    sizes = [1, 7, CHUNK + 3, 2 * CHUNK, 200001]
    tensors = [torch.randn(s, generator=g).to(dtype).to(DEV) for s in sizes]
    table = _Table(tensors, DEV)
    ptrs = _Table.pointers(tensors, DEV)
    partial = torch.empty(table.n_chunks, dtype=torch.float32, device=DEV)
    total = torch.empty(1, dtype=torch.float32, device=DEV)
    L.call("alodlm_grad_norm", L.ptr(ptrs), L.ptr(table.chunk_tensor), L.ptr(table.chunk_start),
           L.ptr(table.numels), table.n_chunks, CHUNK, L.dtype_code(dtype), L.ptr(partial),
           L.ptr(total), st())
    torch.cuda.synchronize()
    want = torch.cat([t.double().cpu() for t in tensors]).norm().item()
    assert abs(float(total) - want) <= 1e-5 * want


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", [(100, 32), (5000, 256), (4096, 4096), (300, 100)])
def test_gate_bwd(dtype, rows, hidden):
    """Gate head backward: gw += scale * sum_r dgate[r] * readout[r],
    gb and depth_bias[depth] += scale * sum_r dgate[r] (alodlm/model.py:22-38);
    rows with dgate 0 contribute nothing."""
    L = lib()
    log(f"gate_bwd rows={rows} hidden={hidden} {dtype}")
    g = torch.Generator().manual_seed(rows + hidden)
    dgate = torch.randn(rows, generator=g)
    dgate[torch.rand(rows, generator=g) < 0.5] = 0.0
    readout = torch.randn(rows, hidden, generator=g).to(dtype)
    gw = torch.full((hidden,), 0.5, device=DEV)
    gb = torch.full((1,), 0.25, device=DEV)
    gdb = torch.zeros(4, device=DEV)
    ws = torch.empty(L.query("alodlm_gate_bwd_workspace", rows, hidden), dtype=torch.float32,
                     device=DEV)
    dg, ro = dgate.to(DEV), readout.to(DEV)
    L.call("alodlm_gate_bwd", L.ptr(dg), L.ptr(ro), 0.5, L.ptr(gw), L.ptr(gb), L.ptr(gdb), 2,
           rows, hidden, L.ptr(ws), L.dtype_code(dtype), st())
    torch.cuda.synchronize()
    want_w = 0.5 + 0.5 * (dgate.double()[:, None] * readout.double()).sum(0)
    want_b = 0.5 * dgate.double().sum()
    torch.testing.assert_close(gw.cpu().double(), want_w, atol=1e-4, rtol=1e-5)
    assert abs(float(gb) - (0.25 + want_b)) < 1e-4
    assert abs(float(gdb[2]) - want_b) < 1e-4 and float(gdb[0]) == 0.0


def _embed_ids(rows, vocab, seed):
    """Token ids with runs of every length class the plan distinguishes: one
    row, exactly one chunk (32), just over (33), two full chunks (64), a long
    run (the mask token's), and ids outside [0, vocab)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (rows,), generator=g)
    perm = torch.randperm(rows, generator=g)
    start = 0
    for token, count in ((7, 32), (8, 33), (9, 64), (vocab - 1, rows // 10), (-1, 5), (vocab, 5)):
        ids[perm[start:start + count]] = token
        start += count
    return ids


def _embed_fixed_order(dout, ids, keep, table, vocab, chunk=32):
    """float32 sums in the kernels' fixed order: rows of one id in ascending
    row order, summed in chunks of 32 rows; a one-chunk run is added to the
    table row, a longer run's chunk sums are added up in chunk order first."""
    out = table.copy()
    for token in np.unique(ids):
        if token < 0 or token >= vocab:
            continue
        rows = np.nonzero(ids == token)[0]
        partial = []
        for lo in range(0, len(rows), chunk):
            acc = np.zeros(dout.shape[1], np.float32)
            used = False
            for r in rows[lo:lo + chunk]:
                if keep[r]:
                    acc = acc + dout[r]
                    used = True
            partial.append((acc, used))
        if len(partial) == 1:
            if partial[0][1]:
                out[token] = out[token] + partial[0][0]
        else:
            acc = np.zeros(dout.shape[1], np.float32)
            for p, _ in partial:
                acc = acc + p
            out[token] = out[token] + acc
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden,filtered", [(5000, 512, False), (3001, 264, True),
                                                  (40, 8, False)])
def test_embed_scatter_is_deterministic_and_exact(dtype, rows, hidden, filtered):
    """Embedding backward (alodlm/model.py:133,149-151 through nn.Embedding):
    dtable[id] += sum of dout over the rows with that id, ids outside [0, V)
    contributing nothing, rows with row_exits > max_exit skipped.  The plan
    is a stable sort of the rows by id; the sums are bit-identical to float32
    additions in the plan's fixed order and within float32 rounding of the
    float64 sums."""
    L = lib()
    vocab = 1000
    log(f"embed scatter rows={rows} hidden={hidden} {dtype} filtered={filtered}")
    ids = _embed_ids(rows, vocab, rows + hidden)
    g = torch.Generator().manual_seed(rows)
    dout = torch.randn(rows, hidden, generator=g).to(dtype)
    table = torch.randn(vocab, hidden, generator=g)
    exits = torch.randint(0, 4, (rows,), generator=g, dtype=torch.int32)
    max_exit = 1
    keep = (exits <= max_exit).numpy() if filtered else np.ones(rows, bool)
    ids_d = ids.to(DEV)
    plan = torch.empty(L.query("alodlm_embed_plan_size", rows), dtype=torch.int32, device=DEV)
    L.call("alodlm_embed_plan", L.ptr(ids_d), rows, vocab, L.ptr(plan), st())
    ws = torch.empty(L.query("alodlm_embed_scatter_workspace", rows, hidden), dtype=torch.float32,
                     device=DEV)
    exits_d = exits.to(DEV) if filtered else None
    results = []
    for _ in range(2):
        dt = table.to(DEV)
        L.call("alodlm_embed_scatter_add", L.ptr(dout.to(DEV)), L.ptr(plan), L.ptr(exits_d),
               max_exit, L.ptr(dt), L.ptr(ws), rows, hidden, vocab, L.dtype_code(dtype), st())
        results.append(dt.cpu())
    torch.cuda.synchronize()
    assert torch.equal(results[0], results[1])
    # the plan: keys sorted (out-of-range ids as V), rows stable within a key
    p = plan.cpu().numpy()
    key, row = p[8:8 + rows], p[8 + rows:8 + 2 * rows]
    want_key = np.where((ids.numpy() >= 0) & (ids.numpy() < vocab), ids.numpy(), vocab)
    order = np.argsort(want_key, kind="stable")
    np.testing.assert_array_equal(row, order)
    np.testing.assert_array_equal(key, want_key[order])
    runs = np.unique(want_key, return_counts=True)[1]
    chunks = (runs + 31) // 32
    assert p[0] == len(runs) and p[1] == chunks.sum()
    assert p[2] == chunks[runs > 32].sum() and p[3] == (runs > 32).sum()
    dout32 = dout.float().numpy()
    want = _embed_fixed_order(dout32, ids.numpy(), keep, table.numpy(), vocab)
    np.testing.assert_array_equal(results[0].numpy(), want)
    exact = table.double().numpy().copy()
    valid = (ids.numpy() >= 0) & (ids.numpy() < vocab) & keep
    np.add.at(exact, ids.numpy()[valid], dout32.astype(np.float64)[valid])
    np.testing.assert_allclose(results[0].numpy(), exact, rtol=0, atol=2e-4 * np.sqrt(rows / 10))


def test_embed_scatter_without_rows_is_a_no_op():
    L = lib()
    table = torch.ones(10, 8, device=DEV)
    L.call("alodlm_embed_plan", None, 0, 10, None, st())
    L.call("alodlm_embed_scatter_add", None, None, None, 0, L.ptr(table), None, 0, 8, 10,
           L.F32_CODE, st())
    torch.cuda.synchronize()
    assert torch.equal(table.cpu(), torch.ones(10, 8))
