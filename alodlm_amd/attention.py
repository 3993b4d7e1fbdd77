"""Range-plan form of the dual-stream mask and the attention over it (drop-in
for alodlm/attention.py).

The plan format (q_ranges, k_ranges, attn_type_map with 1 = causal) is kept
because external callers name it; the HIP attention kernels take the same
mask as intervals derived from the segment boundaries, so ``sparse_attention``
recovers those boundaries from the plan (any plan that ``sparse_plan`` did not
produce is rejected with ValueError).
"""

import torch


def sparse_plan(boundaries, block_size, backend):
    """Per segment: each noisy block attends causally to itself and fully to the
    clean prefix of earlier blocks; the clean stream is causal
    (alodlm/attention.py:12-30)."""
    q_ranges, k_ranges, types = [], [], []
    for start, end in zip(boundaries[:-1], boundaries[1:]):
        length = (end - start) // 2
        noisy = [(start + length + b, start + length + min(b + block_size, length))
                 for b in range(0, length, block_size)]
        for lo, hi in noisy:
            q_ranges.append([lo, hi]); k_ranges.append([lo, hi]); types.append(1)
        for index, (lo, hi) in enumerate(noisy[1:], 1):
            q_ranges.append([lo, hi]); k_ranges.append([start, start + index * block_size])
            types.append(0)
        if length:
            q_ranges.append([start, start + length]); k_ranges.append([start, start + length])
            types.append(1)
    return {"q_ranges": q_ranges, "k_ranges": k_ranges, "attn_type_map": types,
            "backend": backend}


def plan_to_device(plan, device):
    """int32 range tensors plus the longest q/k range (alodlm/attention.py:33-41)."""
    result = dict(plan)
    result["max_seqlen_q"] = max((b - a for a, b in plan["q_ranges"]), default=0)
    result["max_seqlen_k"] = max((b - a for a, b in plan["k_ranges"]), default=0)
    for name in ("q_ranges", "k_ranges", "attn_type_map"):
        result[name] = torch.tensor(result[name], dtype=torch.int32, device=device)
        if name.endswith("_ranges"):
            result[name] = result[name].reshape(-1, 2)
    return result


class _SparseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, mask):
        from . import _lib
        N, nq, dh = q.shape
        nkv = k.shape[1]
        code, st = _lib.dtype_code(q.dtype), _lib.stream_handle(q.device)
        qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
        o = torch.empty_like(qc)
        lse = torch.empty(nq, N, dtype=torch.float32, device=q.device)
        _lib.call("alodlm_attention_fwd", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), nkv * dh,
                  _lib.ptr(mask.boundaries), _lib.ptr(mask.row_segment), _lib.ptr(mask.tiles),
                  mask.tiles.shape[0], _lib.ptr(o), _lib.ptr(lse), N, nq, nkv, dh,
                  mask.block_size, code, st)
        ctx.save_for_backward(qc, kc, vc, o, lse)
        ctx.mask = mask
        return o

    @staticmethod
    def backward(ctx, do):
        from . import _lib
        q, k, v, o, lse = ctx.saved_tensors
        mask = ctx.mask
        N, nq, dh = q.shape
        nkv = k.shape[1]
        code, st = _lib.dtype_code(q.dtype), _lib.stream_handle(q.device)
        do = do.contiguous()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        n_tiles = mask.tiles.shape[0]
        ws = torch.empty(_lib.query("alodlm_attention_bwd_workspace", N, nq, nkv, dh, n_tiles,
                                    mask.ds_blocks),
                         dtype=torch.float32, device=q.device)
        _lib.call("alodlm_attention_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), nkv * dh,
                  _lib.ptr(o), _lib.ptr(lse), _lib.ptr(do), _lib.ptr(mask.boundaries),
                  _lib.ptr(mask.row_segment), _lib.ptr(mask.tiles), n_tiles, _lib.ptr(dq),
                  _lib.ptr(dk), _lib.ptr(dv), nkv * dh, _lib.ptr(ws), _lib.ptr(mask.ds_base),
                  mask.ds_blocks, N, nq, nkv, dh, mask.block_size, code, st)
        return dq, dk, dv, None


def sparse_attention(q, k, v, plan):
    """Softmax attention under a range plan (alodlm/attention.py:44-66) with
    scale head_dim^-0.5 and no softcap: q [N, nq, dh], k and v [N, nkv, dh]
    (grouped-query heads), result [N, nq, dh]; differentiable in q, k, v."""
    if q.device.type != "cuda":
        raise ValueError("Sparse attention requires CUDA; use sdpa for CPU")
    from .layers import DualStreamMask
    mask = DualStreamMask.from_plan(plan, q.device)
    if q.shape[0] != mask.rows or k.shape[0] != mask.rows or v.shape != k.shape:
        raise ValueError("q, k and v must have one row per position of the plan")
    return _SparseAttention.apply(q, k, v, mask)
