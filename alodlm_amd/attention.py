"""Range-plan form of the dual-stream mask (drop-in for alodlm/attention.py:12-41).

The plan format (q_ranges, k_ranges, attn_type_map with 1 = causal) is kept
because external callers and checkpoints name it; the HIP attention kernels do
not need it (they derive the same ranges from the segment boundaries).
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
