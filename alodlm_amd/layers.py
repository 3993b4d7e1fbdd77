"""One Qwen3 decoder layer on the HIP kernels.

The forward and backward schedules of a layer application live here
(``Kernels.layer_fwd``, ``layer_bwd``, ``layer_window``) and are shared by the
fused training step (``engine.StepEngine``), the decoder and the reference's
public layer functions, which ``alodlm_amd.model`` defines where the
reference does (alodlm/model.py:41-80): ``rotary``, ``layer_forward`` and
``training_layer`` run on the autograd nodes and mask forms of this module.

The attention mask is one of

* ``DualStreamMask`` - the training mask of a pack (alodlm/batch.py:23-31),
  what ``build_batch`` puts in ``Batch.attention_mask``; the kernels evaluate
  it from the segment boundaries, nothing N x N is built;
* the range plan of ``attention.sparse_plan`` / ``plan_to_device`` for the same
  mask (alodlm/attention.py:12-41);
* a dense boolean [L, P + L] mask that allows every one of P prefix keys and
  is causal over the L current rows - the decoder's window mask
  (alodlm/inference.py:77-79); P = 0 is the causal mask.

Other dense masks are rejected with ValueError: the kernels take the interval
forms above, not arbitrary masks.
"""

import functools

import numpy as np
import torch

from . import _lib
from ._lib import EPI_ACCUM, EPI_RESIDUAL, EPI_STORE, EPI_STORE_F32, call, ptr, query

TILE_ROWS = 128


def allowed_pairs(length, block_size):
    """Number of (query, key) pairs the dual-stream mask allows in one segment:
    the causal clean stream plus, per noisy block, its causal self-block and
    the clean rows of all earlier blocks."""
    total = length * (length + 1) // 2
    for left in range(0, length, block_size):
        width = min(block_size, length - left)
        total += width * (width + 1) // 2 + width * left
    return total


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


def ds_block_base(offsets):
    """First 32x32 dS block of each segment, and the total, for the stored-dS
    attention backward: a segment of L tokens holds T (T + 1) blocks per query
    head, T = ceil(L / 32) (the allowed pairs of 32-row query and key tiles
    of its clean and noisy streams).  int64 [S + 1]."""
    lengths = np.diff(np.asarray(offsets, dtype=np.int64))
    tiles = (lengths + 31) // 32
    return np.concatenate([[0], np.cumsum(tiles * (tiles + 1))]).astype(np.int64)


def _to_device(array, device):
    """Host array -> device tensor through pinned memory, without blocking."""
    return torch.from_numpy(np.ascontiguousarray(array)).pin_memory().to(device, non_blocking=True)


class DualStreamMask:
    """The dual-stream training mask of one pack (alodlm/batch.py:23-31) in
    the form the attention kernels take.

    ``boundaries``: int64 [S+1] dual-stream row offsets (twice the token
    offsets); ``row_segment``: int32 [N]; ``tiles``: int32 [T, 2] 128-row
    query/key tiles; ``pairs``: number of allowed (query, key) pairs.
    """

    def __init__(self, token_offsets, block_size, device, boundaries=None, row_segment=None):
        offsets = [int(v) for v in token_offsets]
        self.offsets = offsets
        self.block_size = int(block_size)
        self.rows = 2 * offsets[-1]
        self.pairs = sum(allowed_pairs(b - a, self.block_size) for a, b in zip(offsets, offsets[1:]))
        if boundaries is None:
            boundaries = _to_device(np.asarray([2 * v for v in offsets], dtype=np.int64), device)
        if row_segment is None:
            seg = np.repeat(np.arange(len(offsets) - 1, dtype=np.int32),
                            [2 * (b - a) for a, b in zip(offsets, offsets[1:])])
            row_segment = _to_device(seg, device)
        self.boundaries = boundaries
        self.row_segment = row_segment
        self.tiles = _to_device(np.asarray(attention_tiles(offsets), dtype=np.int32),
                                device).view(-1, 2)
        # the stored-dS attention backward's block table (block size 32 only)
        base = ds_block_base(offsets)
        self.ds_blocks = int(base[-1]) if self.block_size == 32 else 0
        self.ds_base = _to_device(base, device) if self.ds_blocks else None

    @classmethod
    def from_plan(cls, plan, device):
        """The mask a range plan of ``sparse_plan`` describes.  Raises
        ValueError for any other plan."""
        offsets, block = plan_segments(plan)
        return cls(offsets, block, device)

    def dense(self):
        """The boolean [N, N] mask (block-diagonal over segments) the reference's
        build_batch materialises (alodlm/batch.py:64-65,83); built on demand
        and kept."""
        if getattr(self, "_dense", None) is None:
            from .batch import attention_mask
            device = self.boundaries.device
            mask = torch.zeros(self.rows, self.rows, dtype=torch.bool, device=device)
            for a, b in zip(self.offsets, self.offsets[1:]):
                mask[2 * a:2 * b, 2 * a:2 * b] = attention_mask(b - a, self.block_size, device)
            self._dense = mask
        return self._dense

    # Used as a tensor (indexed, or passed to a torch function), the mask acts
    # as its dense form, as the reference's Batch.attention_mask does.
    shape = property(lambda self: torch.Size((self.rows, self.rows)))
    dtype = torch.bool
    device = property(lambda self: self.boundaries.device)

    def __getitem__(self, index):
        return self.dense()[index]

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        from torch.utils._pytree import tree_map
        dense = lambda a: a.dense() if isinstance(a, DualStreamMask) else a
        return func(*tree_map(dense, args), **tree_map(dense, kwargs or {}))


def plan_segments(plan):
    """(token offsets, block size) of the packed segments a range plan of
    ``attention.sparse_plan`` describes (alodlm/attention.py:12-30); any other
    plan raises ValueError.  Each segment lists its noisy blocks first (causal
    self ranges, then full ranges into the clean prefix) and its clean
    stream, the causal range starting at the segment start, last."""
    from .attention import sparse_plan
    host = {k: (v.tolist() if torch.is_tensor(v) else v)
            for k, v in plan.items() if k in ("q_ranges", "k_ranges", "attn_type_map")}
    q = [tuple(r) for r in host["q_ranges"]]
    k = [tuple(r) for r in host["k_ranges"]]
    types = list(host["attn_type_map"])
    if not q or len(q) != len(k) or len(q) != len(types):
        raise ValueError("the plan is not a dual-stream training plan (sparse_plan)")
    bounds, i, block = [0], 0, None
    while i < len(q):
        start = bounds[-1]
        j = next((j for j in range(i, len(q)) if q[j][0] == start and q[j] == k[j]
                  and types[j] == 1), None)
        if j is None:
            raise ValueError("the plan is not a dual-stream training plan (sparse_plan)")
        if j > i:
            # a segment's first noisy block is min(block size, its length) long
            block = max(block or 0, q[i][1] - q[i][0])
        bounds.append(start + 2 * (q[j][1] - q[j][0]))
        i = j + 1
    block = block or max((b - a) // 2 for a, b in zip(bounds, bounds[1:]))
    expect = sparse_plan(bounds, block, plan.get("backend"))
    if ([list(r) for r in q] != expect["q_ranges"]
            or [list(r) for r in k] != expect["k_ranges"] or types != expect["attn_type_map"]):
        raise ValueError("the plan is not a dual-stream training plan (sparse_plan)")
    return [b // 2 for b in bounds], block


class WindowMask:
    """Every one of ``prefix`` cached keys plus causal attention over
    ``window`` current rows (alodlm/inference.py:77-79), run as the clean
    stream of one dual-stream segment of length P + W whose first P rows are
    the cache.

    The MFMA kernels take 128-row query tiles from ``base`` = floor(P / 128) *
    128, so the query buffer also holds rows [base, P) (zeros; their outputs
    are ignored); the generic kernels take any row, so ``base`` = P there.
    Segment row r is query-buffer row r - base and key/value row r (the
    key/value pointers are offset by ``base`` rows)."""

    def __init__(self, prefix, window, tiled, device, block_size=1):
        self.prefix, self.window = prefix, window
        L = prefix + window
        self.block_size = block_size
        self.base = (prefix // TILE_ROWS) * TILE_ROWS if tiled else prefix
        self.q_rows = L - self.base
        self.q_off = prefix - self.base
        self.boundaries = torch.tensor([-self.base, 2 * L - self.base], dtype=torch.int64,
                                       device=device)
        self.row_segment = torch.zeros(self.q_rows, dtype=torch.int32, device=device)
        if tiled:
            starts = list(range(self.base, L, TILE_ROWS))[::-1]
            self.tiles = torch.tensor([v for s in starts for v in (0, s)], dtype=torch.int32,
                                      device=device).view(-1, 2)
        else:
            self.tiles = None
        self.pairs = window * prefix + window * (window + 1) // 2


class Rope:
    """Where a layer's rotary angles come from: positions (int64 [N]) with the
    float32 inverse frequencies ([tf] modeling_qwen3.py:115-137, evaluated in
    the kernels), or caller tables cos/sin [N, head_dim] in the storage dtype
    (alodlm/model.py:41-46)."""

    def __init__(self, positions=None, inv_freq=None, cos=None, sin=None):
        self.positions, self.inv_freq = positions, inv_freq
        self.cos, self.sin = cos, sin

    @property
    def tables(self):
        return self.cos is not None


class LayerWeights:
    """One layer's weights as the kernels take them: q|k|v stacked [W, H],
    gate|up stacked [2I, H], o [H, nq*dh], down [H, I], the four norm weights,
    and optional out-contiguous copies (``*_t``, [in, out]) that a forward
    product reads instead of its [out, in] weight when given (the step gives
    them for all four: the products run faster that way).  ``from_layer`` takes an HF Qwen3 decoder layer:
    adjacent projection weights (the step's parameter arena) are used in
    place, separate ones are stacked into a copy."""

    def __init__(self, wqkv, wo, wgu, wd, ln1, ln2, qn, kn, wqkv_t=None, wo_t=None,
                 wgu_t=None, wd_t=None):
        self.wqkv, self.wo, self.wgu, self.wd = wqkv, wo, wgu, wd
        self.ln1, self.ln2, self.qn, self.kn = ln1, ln2, qn, kn
        self.wqkv_t, self.wo_t, self.wgu_t, self.wd_t = wqkv_t, wo_t, wgu_t, wd_t

    @staticmethod
    def module_tensors(layer):
        """The layer's 11 parameters in a fixed order (alodlm/model.py:52-58,74-75)."""
        attn, mlp = layer.self_attn, layer.mlp
        return (attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight, attn.o_proj.weight,
                mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight,
                layer.input_layernorm.weight, layer.post_attention_layernorm.weight,
                attn.q_norm.weight, attn.k_norm.weight)

    @classmethod
    def from_tensors(cls, wq, wk, wv, wo, wg, wu, wd, ln1, ln2, qn, kn):
        return cls(_stack_rows(wq, wk, wv), wo.contiguous(), _stack_rows(wg, wu),
                   wd.contiguous(), ln1.contiguous(), ln2.contiguous(), qn.contiguous(),
                   kn.contiguous())


def _stack_rows(*ts):
    """[sum rows, cols] view of row-stacked tensors when they are adjacent in
    memory, else a stacked copy."""
    ts = [t.detach() for t in ts]
    first = ts[0]
    storage = first.untyped_storage().data_ptr()
    adjacent = all(t.is_contiguous() and t.untyped_storage().data_ptr() == storage for t in ts)
    offset = first.data_ptr()
    for t in ts:
        adjacent = adjacent and t.data_ptr() == offset
        offset += t.numel() * t.element_size()
    if adjacent:
        rows = sum(t.shape[0] for t in ts)
        return first.as_strided((rows, first.shape[1]), (first.shape[1], 1))
    return torch.cat(ts, 0)


class LayerGrads:
    """float32 gradient views of one layer (same layout as LayerWeights)."""

    def __init__(self, wqkv, wo, wgu, wd, ln1, ln2, qn, kn):
        self.wqkv, self.wo, self.wgu, self.wd = wqkv, wo, wgu, wd
        self.ln1, self.ln2, self.qn, self.kn = ln1, ln2, qn, kn


class Kernels:
    """Launch helpers and the layer schedules for one model shape, dtype and
    device.  Work is enqueued on the current stream."""

    def __init__(self, dims, dtype, device):
        self.dims, self.dtype, self.device = dims, dtype, device
        self.code = _lib.dtype_code(dtype)
        _lib.load()
        self._ws = None

    # ------------------------------------------------------------------ helpers
    def _stream(self):
        return _lib.stream_handle(self.device)

    def _empty(self, *shape, dtype=None):
        return torch.empty(*shape, dtype=dtype or self.dtype, device=self.device)

    def _workspace(self, n):
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(max(n, 1), dtype=torch.float32, device=self.device)
        return self._ws

    def embed_plan(self, ids):
        """The sorted-row plan of the int64 token ids ``ids`` that the
        deterministic embedding scatters take (one per id array and step)."""
        n = ids.numel()
        plan = self._empty(query("alodlm_embed_plan_size", n), dtype=torch.int32)
        call("alodlm_embed_plan", ptr(ids), n, self.dims.vocab, ptr(plan), self._stream())
        return plan

    def embed_scatter(self, dout, plan, dtable, row_exits=None, max_exit=0):
        """dtable[ids[r]] += dout[r] (float32 table) over the rows of ``plan``
        (those with row_exits[r] <= max_exit when ``row_exits`` is given), in
        a fixed order."""
        N, H = dout.shape
        ws = self._workspace(query("alodlm_embed_scatter_workspace", N, H))
        call("alodlm_embed_scatter_add", ptr(dout), ptr(plan), ptr(row_exits), max_exit,
             ptr(dtable), ptr(ws), N, H, dtable.shape[0], self.code, self._stream())

    def _gemm(self, A, lda, a_k, B, ldb, b_k, C, ldc, M, N, K, alpha=1.0, epi=EPI_STORE, R=None,
              ldr=0):
        ws = None
        need = query("alodlm_gemm_workspace", M, N, K, epi, self.code)
        if need:
            ws = self._workspace(need)
        call("alodlm_gemm", ptr(A), lda, a_k, ptr(B), ldb, b_k, ptr(C), ldc, ptr(R), ldr, M, N, K,
             alpha, epi, self.code, ptr(ws), self._stream())

    def _product(self, x, ldx, w, w_t, y, M, N, K, epi=EPI_STORE, R=None, ldr=0):
        """y = x . w^T (+ R) with w [N, K]: through the out-contiguous copy w_t
        [K, N] when there is one."""
        if w_t is not None:
            self._gemm(x, ldx, 1, w_t, N, 0, y, N, M, N, K, epi=epi, R=R, ldr=ldr)
        else:
            self._gemm(x, ldx, 1, w, K, 1, y, N, M, N, K, epi=epi, R=R, ldr=ldr)

    def _attention_fwd(self, q, k, v, ldv, o, lse, mask):
        d = self.dims
        call("alodlm_attention_fwd", ptr(q), ptr(k), ptr(v), ldv, ptr(mask.boundaries),
             ptr(mask.row_segment), ptr(mask.tiles),
             0 if mask.tiles is None else mask.tiles.shape[0], ptr(o), ptr(lse), q.shape[0],
             d.heads, d.kv_heads, d.head_dim, mask.block_size, self.code, self._stream())

    def _attention_bwd(self, q, k, v, ldv, o, lse, do, dq, dk, dv, lddv, mask):
        d, N = self.dims, q.shape[0]
        n_tiles = 0 if mask.tiles is None else mask.tiles.shape[0]
        ds_blocks = getattr(mask, "ds_blocks", 0)
        ws = self._workspace(query("alodlm_attention_bwd_workspace", N, d.heads, d.kv_heads,
                                   d.head_dim, n_tiles, ds_blocks))
        call("alodlm_attention_bwd", ptr(q), ptr(k), ptr(v), ldv, ptr(o), ptr(lse), ptr(do),
             ptr(mask.boundaries), ptr(mask.row_segment), ptr(mask.tiles), n_tiles, ptr(dq),
             ptr(dk), ptr(dv), lddv, ptr(ws), ptr(getattr(mask, "ds_base", None)), ds_blocks,
             N, d.heads, d.kv_heads, d.head_dim, mask.block_size, self.code, self._stream())

    def _attention_fwd_flops(self, q, k, v, ldv, o, lse, mask):
        """Algorithmic forward FLOPs: 4*dh per allowed (q, k) pair and head."""
        return 4.0 * self.dims.head_dim * self.dims.heads * mask.pairs

    def _attention_bwd_flops(self, q, k, v, ldv, o, lse, do, dq, dk, dv, lddv, mask):
        """Algorithmic backward FLOPs: 8*dh per allowed pair and head."""
        return 8.0 * self.dims.head_dim * self.dims.heads * mask.pairs

    def _rope_fwd(self, qkv, w, rope, q, k):
        d, N = self.dims, qkv.shape[0]
        if rope.tables:
            call("alodlm_qknorm_rotary_fwd", ptr(qkv), ptr(w.qn), ptr(w.kn), ptr(rope.cos),
                 ptr(rope.sin), ptr(q), ptr(k), N, d.heads, d.kv_heads, d.head_dim, d.eps,
                 self.code, self._stream())
        else:
            call("alodlm_qknorm_rope_fwd", ptr(qkv), ptr(w.qn), ptr(w.kn), ptr(rope.positions),
                 ptr(rope.inv_freq), ptr(q), ptr(k), N, d.heads, d.kv_heads, d.head_dim, d.eps,
                 self.code, self._stream())

    def _rope_bwd(self, dq, dk, qkv, w, rope, dqkv, gw):
        d, N = self.dims, qkv.shape[0]
        ws = self._workspace(query("alodlm_qknorm_rope_bwd_workspace", N, d.heads, d.kv_heads,
                                   d.head_dim))
        if rope.tables:
            call("alodlm_qknorm_rotary_bwd", ptr(dq), ptr(dk), ptr(qkv), ptr(w.qn), ptr(w.kn),
                 ptr(rope.cos), ptr(rope.sin), ptr(dqkv), ptr(gw.qn), ptr(gw.kn), ptr(ws), N,
                 d.heads, d.kv_heads, d.head_dim, d.eps, self.code, self._stream())
        else:
            call("alodlm_qknorm_rope_bwd", ptr(dq), ptr(dk), ptr(qkv), ptr(w.qn), ptr(w.kn),
                 ptr(rope.positions), ptr(rope.inv_freq), ptr(dqkv), ptr(gw.qn), ptr(gw.kn),
                 ptr(ws), N, d.heads, d.kv_heads, d.head_dim, d.eps, self.code, self._stream())

    # ------------------------------------------------------------------ layer
    def layer_fwd(self, w, x, mask, rope, save=None, keep=(False, False), tag=None):
        """One layer application (alodlm/model.py:49-76) over x [N, H].

        With ``save`` (a list) the activations the backward needs are
        appended: the input, rstd of both norms, the q|k|v projections, the
        attention output and log-sum-exp, the post-attention residual and the
        gate|up projections; ``keep`` = (rotary q/k, norm outputs) also keeps
        those (else the backward recomputes them).  Returns y [N, H]; with
        ``keep[0]`` the rotated q/k stay in the saved tuple (indices 9, 10)."""
        d, N, st, c = self.dims, x.shape[0], self._stream(), self.code
        H, W, I = d.hidden, d.qkv_width, d.intermediate
        QD = d.heads * d.head_dim
        h1 = self._empty(N, H)
        rstd1 = self._empty(N, dtype=torch.float32)
        call("alodlm_rmsnorm_fwd", ptr(x), ptr(w.ln1), ptr(h1), ptr(rstd1), N, H, d.eps, c, st)
        qkv = self._empty(N, W)
        self._product(h1, H, w.wqkv, w.wqkv_t, qkv, N, W, H)
        keep_rot, keep_norm = keep if save is not None else (False, False)
        if not keep_norm:
            h1 = None
        q = self._empty(N, QD)
        k = self._empty(N, d.kv_heads * d.head_dim)
        self._rope_fwd(qkv, w, rope, q, k)
        o = self._empty(N, QD)
        lse = self._empty(d.heads, N, dtype=torch.float32)
        v = qkv[:, QD + d.kv_heads * d.head_dim:]
        self._attention_fwd(q, k, v, W, o, lse, mask)
        if not keep_rot:
            q = k = None
        x1 = self._empty(N, H)
        self._product(o, QD, w.wo, w.wo_t, x1, N, H, QD, epi=EPI_RESIDUAL, R=x, ldr=H)
        h2 = self._empty(N, H)
        rstd2 = self._empty(N, dtype=torch.float32)
        call("alodlm_rmsnorm_fwd", ptr(x1), ptr(w.ln2), ptr(h2), ptr(rstd2), N, H, d.eps, c, st)
        gu = self._empty(N, 2 * I)
        self._product(h2, H, w.wgu, w.wgu_t, gu, N, 2 * I, H)
        if not keep_norm:
            h2 = None
        act = self._empty(N, I)
        call("alodlm_swiglu_fwd", ptr(gu), ptr(act), N, I, c, st)
        y = self._empty(N, H)
        self._product(act, I, w.wd, w.wd_t, y, N, H, I, epi=EPI_RESIDUAL, R=x1, ldr=H)
        if save is not None:
            save.append((tag, x, rstd1, qkv, o, lse, x1, rstd2, gu, q, k, h1, h2))
        return y

    def layer_bwd(self, dy, saved, w, gw, mask, rope, first=False, defer=None):
        """Backward of ``layer_fwd`` from its saved tuple: returns dx and adds
        the weight gradients into the float32 views ``gw`` (``first``: the four
        projection matrices' gradients are written instead of added; the norm
        weights' are always added).  With a list ``defer`` the four projection
        products are not run: their operands (A, lda, B, ldb, C, ldc, M, N;
        k = the rows) are appended to it in the order down, gate/up, O, QKV,
        and the tensors stay alive through the list."""
        _, x, rstd1, qkv, o, lse, x1, rstd2, gu, q, k, h1, h2 = saved
        d, N, st, c = self.dims, x.shape[0], self._stream(), self.code
        wepi = EPI_STORE_F32 if first else EPI_ACCUM

        def dw(A, lda, B, ldb, C, ldc, M, Nc):  # C (+)= A^T B over the N rows
            if defer is None:
                self._gemm(A, lda, 0, B, ldb, 0, C, ldc, M, Nc, N, epi=wepi)
            else:
                defer.append((A, lda, B, ldb, C, ldc, M, Nc))
        H, W, I = d.hidden, d.qkv_width, d.intermediate
        QD = d.heads * d.head_dim
        # ---- MLP: y = x1 + act . Wd^T  (the SwiGLU backward also rewrites act)
        dact = self._empty(N, I)
        self._gemm(dy, H, 1, w.wd, I, 0, dact, I, N, I, H)
        act = self._empty(N, I)
        dgu = self._empty(N, 2 * I)
        call("alodlm_swiglu_bwd", ptr(dact), ptr(gu), ptr(dgu), ptr(act), N, I, c, st)
        del dact
        dw(dy, H, act, I, gw.wd, I, H, I)
        del act
        if h2 is None:
            h2 = self._empty(N, H)
            call("alodlm_rmsnorm_fwd", ptr(x1), ptr(w.ln2), ptr(h2), None, N, H, d.eps, c, st)
        dh2 = self._empty(N, H)
        self._gemm(dgu, 2 * I, 1, w.wgu, H, 0, dh2, H, N, H, 2 * I)
        dw(dgu, 2 * I, h2, H, gw.wgu, H, 2 * I, H)
        del dgu, h2
        dx1 = self._empty(N, H)
        ws = self._workspace(query("alodlm_rmsnorm_bwd_workspace", N, H))
        call("alodlm_rmsnorm_bwd", ptr(dh2), ptr(x1), ptr(rstd2), ptr(w.ln2), ptr(dy), ptr(dx1),
             ptr(gw.ln2), ptr(ws), N, H, c, st)
        del dh2
        # ---- attention: x1 = x + o . Wo^T
        do = self._empty(N, QD)
        self._gemm(dx1, H, 1, w.wo, QD, 0, do, QD, N, QD, H)
        dw(dx1, H, o, QD, gw.wo, QD, H, QD)
        if q is None:
            q = self._empty(N, QD)
            k = self._empty(N, d.kv_heads * d.head_dim)
            self._rope_fwd(qkv, w, rope, q, k)
        dq = self._empty(N, QD)
        dk = self._empty(N, d.kv_heads * d.head_dim)
        dqkv = self._empty(N, W)
        v = qkv[:, QD + d.kv_heads * d.head_dim:]
        dv = dqkv[:, QD + d.kv_heads * d.head_dim:]
        self._attention_bwd(q, k, v, W, o, lse, do, dq, dk, dv, W, mask)
        del q, k, do
        self._rope_bwd(dq, dk, qkv, w, rope, dqkv, gw)
        del dq, dk
        if h1 is None:
            h1 = self._empty(N, H)
            call("alodlm_rmsnorm_fwd", ptr(x), ptr(w.ln1), ptr(h1), None, N, H, d.eps, c, st)
        dh1 = self._empty(N, H)
        self._gemm(dqkv, W, 1, w.wqkv, H, 0, dh1, H, N, H, W)
        dw(dqkv, W, h1, H, gw.wqkv, H, W, H)
        del dqkv, h1
        dx = self._empty(N, H)
        ws = self._workspace(query("alodlm_rmsnorm_bwd_workspace", N, H))
        call("alodlm_rmsnorm_bwd", ptr(dh1), ptr(x), ptr(rstd1), ptr(w.ln1), ptr(dx1), ptr(dx),
             ptr(gw.ln1), ptr(ws), N, H, c, st)
        return dx

    def layer_window(self, w, x, rope, mask, kbuf, vbuf):
        """Forward of one layer over a decoding window (no autograd): the
        window's rotated keys and values are written into rows [P, P + W) of
        the key/value buffers kbuf/vbuf [capacity, kv_heads * head_dim], whose
        rows [0, P) hold the prefix; ``mask`` is a WindowMask."""
        d, st, c = self.dims, self._stream(), self.code
        Wn = x.shape[0]
        H, QW, I = d.hidden, d.qkv_width, d.intermediate
        QD, KD = d.heads * d.head_dim, d.kv_heads * d.head_dim
        esize = x.element_size()
        h1 = self._empty(Wn, H)
        call("alodlm_rmsnorm_fwd", ptr(x), ptr(w.ln1), ptr(h1), None, Wn, H, d.eps, c, st)
        qkv = self._empty(Wn, QW)
        self._product(h1, H, w.wqkv, w.wqkv_t, qkv, Wn, QW, H)
        q_all = self._empty(mask.q_rows, QD)
        if mask.q_off:
            q_all[:mask.q_off].zero_()
        q_view = q_all[mask.q_off:]
        k_view = kbuf.view(-1, KD)[mask.prefix:mask.prefix + Wn]
        self._rope_fwd(qkv, w, rope, q_view, k_view)
        vbuf.view(-1, KD)[mask.prefix:mask.prefix + Wn].copy_(qkv[:, QD + KD:])
        o_all = self._empty(mask.q_rows, QD)
        lse = self._empty(d.heads, mask.q_rows, dtype=torch.float32)
        shift = mask.base * KD * esize
        call("alodlm_attention_fwd", ptr(q_all), ptr(kbuf) + shift, ptr(vbuf) + shift, KD,
             ptr(mask.boundaries), ptr(mask.row_segment), ptr(mask.tiles),
             0 if mask.tiles is None else mask.tiles.shape[0], ptr(o_all), ptr(lse), mask.q_rows,
             d.heads, d.kv_heads, d.head_dim, mask.block_size, c, st)
        o = o_all[mask.q_off:]
        x1 = self._empty(Wn, H)
        self._product(o, QD, w.wo, w.wo_t, x1, Wn, H, QD, epi=EPI_RESIDUAL, R=x, ldr=H)
        h2 = self._empty(Wn, H)
        call("alodlm_rmsnorm_fwd", ptr(x1), ptr(w.ln2), ptr(h2), None, Wn, H, d.eps, c, st)
        gu = self._empty(Wn, 2 * I)
        self._product(h2, H, w.wgu, w.wgu_t, gu, Wn, 2 * I, H)
        act = self._empty(Wn, I)
        call("alodlm_swiglu_fwd", ptr(gu), ptr(act), Wn, I, c, st)
        y = self._empty(Wn, H)
        self._product(act, I, w.wd, w.wd_t, y, Wn, H, I, epi=EPI_RESIDUAL, R=x1, ldr=H)
        return y


# ----------------------------------------------------------------------------
# The reference's public layer functions
# ----------------------------------------------------------------------------

def _dims_of_layer(layer, hidden):
    from .engine import Dims
    attn, cfg = layer.self_attn, layer.self_attn.config
    return Dims(hidden=hidden.shape[-1], heads=cfg.num_attention_heads,
                kv_heads=cfg.num_key_value_heads, head_dim=attn.head_dim,
                intermediate=layer.mlp.gate_proj.weight.shape[0], vocab=0, layers=1,
                eps=float(layer.input_layernorm.variance_epsilon), theta=0.0)


@functools.lru_cache(maxsize=16)
def _kernels(dims_key, dtype, device):
    from .engine import Dims
    return Kernels(Dims(*dims_key), dtype, device)


def _kernels_for(layer, hidden):
    d = _dims_of_layer(layer, hidden)
    key = (d.hidden, d.heads, d.kv_heads, d.head_dim, d.intermediate, d.vocab, d.layers, d.eps,
           d.theta)
    return _kernels(key, hidden.dtype, hidden.device)


def _check_device(t, what):
    if t.device.type != "cuda":
        raise ValueError(f"{what} runs on the HIP kernels; move the tensors to a CUDA (ROCm) device")


def _kernel_mask(mask, rows, device):
    """The kernels' form of a layer_forward mask (see the module docstring)."""
    if isinstance(mask, (DualStreamMask, WindowMask)):
        return mask
    if isinstance(mask, dict):
        return DualStreamMask.from_plan(mask, device)
    if torch.is_tensor(mask) and mask.dtype == torch.bool and mask.ndim == 2:
        L, total = mask.shape
        P = total - L
        if L == rows and P >= 0:
            causal = torch.ones(L, L, dtype=torch.bool, device=mask.device).tril()
            if bool(mask[:, :P].all()) and torch.equal(mask[:, P:], causal):
                return ("window", P)
    raise ValueError("the HIP attention takes the dual-stream training mask (Batch.attention_mask "
                     "or its sparse_plan) or a prefix + causal window mask")


class _LayerFunction(torch.autograd.Function):
    """training_layer / layer_forward as one autograd node over the kernels."""

    @staticmethod
    def forward(ctx, kernels, mask, rope, hidden, *params):
        w = LayerWeights.from_tensors(*params)
        save = []
        y = kernels.layer_fwd(w, hidden.contiguous(), mask, rope, save, keep=(True, False))
        ctx.kernels, ctx.mask, ctx.rope, ctx.saved, ctx.w = kernels, mask, rope, save[0], w
        ctx.shapes = [(p.shape, p.dtype) for p in params]
        d = kernels.dims
        q, k = save[0][9], save[0][10]
        qkv = save[0][3]
        v = qkv[:, (d.heads + d.kv_heads) * d.head_dim:]
        k_out = k.view(-1, d.kv_heads, d.head_dim)
        v_out = v.contiguous().view(-1, d.kv_heads, d.head_dim)
        ctx.mark_non_differentiable(k_out, v_out)
        return y, k_out, v_out

    @staticmethod
    def backward(ctx, dy, _dk, _dv):
        kernels, w, d = ctx.kernels, ctx.w, ctx.kernels.dims
        H, W, I, QD = d.hidden, d.qkv_width, d.intermediate, d.heads * d.head_dim
        sizes = [W * H, H * QD, 2 * I * H, H * I, H, H, d.head_dim, d.head_dim]
        flat = torch.zeros(sum(sizes), dtype=torch.float32, device=kernels.device)
        views, off = [], 0
        for n in sizes:
            views.append(flat[off:off + n])
            off += n
        gw = LayerGrads(views[0].view(W, H), views[1].view(H, QD), views[2].view(2 * I, H),
                        views[3].view(H, I), *views[4:])
        dx = kernels.layer_bwd(dy.contiguous(), ctx.saved, w, gw, ctx.mask, ctx.rope)
        ctx.saved = None
        qd, kd = QD, d.kv_heads * d.head_dim
        parts = [gw.wqkv[:qd], gw.wqkv[qd:qd + kd], gw.wqkv[qd + kd:], gw.wo, gw.wgu[:I],
                 gw.wgu[I:], gw.wd, gw.ln1, gw.ln2, gw.qn, gw.kn]
        grads = [g.reshape(shape).to(dtype) for g, (shape, dtype) in zip(parts, ctx.shapes)]
        return (None, None, None, dx, *grads)


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin):
        code, st = _lib.dtype_code(q.dtype), _lib.stream_handle(q.device)
        outs = []
        for x in (q, k):
            x = x.contiguous()
            out = torch.empty_like(x)
            call("alodlm_rotary_fwd", ptr(x), ptr(cos), ptr(sin), ptr(out), x.shape[0],
                 x.shape[1], x.shape[2], code, st)
            outs.append(out)
        ctx.save_for_backward(cos, sin)
        return tuple(outs)

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        grads = []
        for g in (dq, dk):
            if g is None:
                grads.append(None)
                continue
            g = g.contiguous()
            out = torch.empty_like(g)
            call("alodlm_rotary_bwd", ptr(g), ptr(cos), ptr(sin), ptr(out), g.shape[0],
                 g.shape[1], g.shape[2], _lib.dtype_code(g.dtype), _lib.stream_handle(g.device))
            grads.append(out)
        return grads[0], grads[1], None, None


class WindowSlot:
    """A decoding window's place in a prefix cache, passed to
    ``layer_forward`` as its ``prefix``: the layer's key/value buffers
    ``k``/``v`` [capacity, kv_heads, head_dim] whose rows [0, P) hold the
    cached prefix, the window's mask (a ``WindowMask`` over P prefix rows),
    and the kernels and arena weights of the model the layer belongs to
    (``weights`` may carry the out-contiguous copies of its matrices, which the
    caller keeps current).  The layer writes the window's rotated keys and
    values straight into rows [P, P + L) and returns views of them."""

    def __init__(self, kernels, weights, k, v, mask):
        self.kernels, self.weights = kernels, weights
        self.k, self.v, self.mask = k, v, mask

    def run(self, layer, hidden, cos, sin):
        d = self.kernels.dims
        L, P = hidden.shape[0], self.mask.prefix
        if self.weights.wqkv.data_ptr() != layer.self_attn.q_proj.weight.data_ptr():
            raise ValueError("the window slot belongs to another layer")
        if self.k.shape[0] < P + L or self.v.shape[0] < P + L or L != self.mask.window:
            raise ValueError("the window does not fit the slot's cache rows")
        rope = Rope(cos=table(cos, L, d.head_dim, hidden), sin=table(sin, L, d.head_dim, hidden))
        y = self.kernels.layer_window(self.weights, hidden.contiguous(), rope, self.mask,
                                      self.k, self.v)
        return y, (self.k[P:P + L], self.v[P:P + L])


def table(t, rows, head_dim, like):
    """A rotary cos/sin table as the kernels read it: [rows, head_dim]
    contiguous in ``like``'s dtype, on its device.  A leading dimension of 1
    is dropped (the shape rotary embedding modules return); any other shape
    raises ValueError (the kernels read rows x head_dim values)."""
    if t.ndim == 3 and t.shape[0] == 1:
        t = t[0]
    if t.ndim != 2 or tuple(t.shape) != (rows, head_dim):
        raise ValueError(f"cos/sin must be [{rows}, {head_dim}] (rows x head_dim), "
                         f"got {tuple(t.shape)}")
    if t.device != like.device:
        raise ValueError("cos/sin must be on the device of the rows they rotate")
    return t.to(like.dtype).contiguous()
