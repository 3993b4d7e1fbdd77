"""Host-side checks of the public API that mirrors the reference's modules
(no GPU work): the range plan and its parsing back into segments, the
argument validation of the credit primitives with the reference's messages,
and the attention-mask forms layer_forward accepts."""

import pytest
import torch

from alodlm_amd.attention import plan_to_device, sparse_plan
from alodlm_amd.credit import (check_sequence_boundaries, masked_sequence_ids,
                               sequence_score_function)
from alodlm_amd.layers import _kernel_mask, plan_segments
from oracle import step as O


def _dense_from_plan(plan, n):
    """The reference test's materialisation of a plan (tests/test_objective.py:97-105)."""
    mask = torch.zeros(n, n, dtype=torch.bool)
    for (qa, qb), (ka, kb), causal in zip(plan["q_ranges"], plan["k_ranges"],
                                          plan["attn_type_map"]):
        allowed = torch.ones(qb - qa, kb - ka, dtype=torch.bool)
        mask[qa:qb, ka:kb] |= allowed.tril() if causal else allowed
    return mask


@pytest.mark.parametrize("offsets,block", [([0, 4, 11], 3), ([0, 128, 256, 300, 512], 32),
                                           ([0, 5], 32), ([0, 1, 3], 32), ([0, 64, 65], 4)])
def test_sparse_plan_is_the_dense_dual_stream_mask(offsets, block):
    """The product's sparse_plan materialises to the closed-form mask of every
    segment (alodlm/batch.py:23-31), block-diagonal over the pack, and the plan
    parses back into its segments."""
    bounds = [2 * v for v in offsets]
    plan = sparse_plan(bounds, block, "magi")
    dense = torch.as_tensor(O.packed_attention_mask(bounds, block))
    assert torch.equal(_dense_from_plan(plan, bounds[-1]), dense)
    segs, b = plan_segments(plan)
    assert segs == offsets
    assert sparse_plan([2 * v for v in segs], b, "magi") == plan


def test_plan_to_device_keeps_the_plan_and_adds_lengths():
    plan = sparse_plan([0, 8, 22], 3, "magi")
    dev = plan_to_device(plan, "cpu")
    assert dev["q_ranges"].dtype == torch.int32 and dev["q_ranges"].shape == (len(plan["q_ranges"]), 2)
    assert dev["q_ranges"].tolist() == plan["q_ranges"]
    assert dev["k_ranges"].tolist() == plan["k_ranges"]
    assert dev["attn_type_map"].tolist() == plan["attn_type_map"]
    assert dev["max_seqlen_q"] == 7 and dev["max_seqlen_k"] == 7
    assert plan_segments(dev) == ([0, 4, 11], 3)


def test_other_plans_are_rejected():
    plan = sparse_plan([0, 256], 32, "magi")
    plan["k_ranges"][3][1] += 1
    with pytest.raises(ValueError, match="dual-stream"):
        plan_segments(plan)
    with pytest.raises(ValueError, match="dual-stream"):
        plan_segments({"q_ranges": [[0, 4]], "k_ranges": [[0, 3]], "attn_type_map": [1]})


def test_credit_validation_messages():
    """alodlm/credit.py:8-35, and the reference test's isolation case
    (tests/test_objective.py:28-29)."""
    with pytest.raises(ValueError, match="cover the actual packed stream"):
        masked_sequence_ids(torch.tensor([True, False]), torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="one-dimensional boolean"):
        check_sequence_boundaries(torch.tensor([1, 0]), torch.tensor([0, 2]))
    with pytest.raises(ValueError, match="packed sequence boundaries"):
        check_sequence_boundaries(torch.tensor([True]), torch.tensor([0]))
    with pytest.raises(ValueError, match="integer dtype"):
        check_sequence_boundaries(torch.tensor([True]), torch.tensor([0., 1.]))
    with pytest.raises(ValueError, match="nondecreasing"):
        check_sequence_boundaries(torch.tensor([True, True]), torch.tensor([0, 2, 1, 2]))
    with pytest.raises(ValueError, match="equal-length"):
        sequence_score_function(torch.ones(3), torch.ones(2), torch.zeros(3, dtype=torch.int64), 1)
    with pytest.raises(ValueError, match="int64"):
        sequence_score_function(torch.ones(2), torch.ones(2), torch.zeros(2, dtype=torch.int32), 1)
    with pytest.raises(ValueError, match="share a dtype"):
        sequence_score_function(torch.ones(2), torch.ones(2, dtype=torch.float64),
                                torch.zeros(2, dtype=torch.int64), 1)
    with pytest.raises(ValueError, match="within the declared"):
        sequence_score_function(torch.ones(2), torch.ones(2), torch.tensor([0, 2]), 2)
    # empty: log_prob.sum() * 0 (credit.py:36-37)
    out = sequence_score_function(torch.ones(0), torch.ones(0, requires_grad=True),
                                  torch.zeros(0, dtype=torch.int64), 1)
    assert float(out) == 0.0 and out.requires_grad


def test_layer_forward_mask_forms():
    """The window mask (every prefix key, causal over the window) and the causal
    mask are recognised; any other dense mask is rejected."""
    L, P = 5, 3
    window = torch.cat((torch.ones(L, P, dtype=torch.bool),
                        torch.ones(L, L, dtype=torch.bool).tril()), 1)
    assert _kernel_mask(window, L, "cpu") == ("window", P)
    assert _kernel_mask(torch.ones(L, L, dtype=torch.bool).tril(), L, "cpu") == ("window", 0)
    bad = window.clone()
    bad[2, 0] = False
    with pytest.raises(ValueError, match="dual-stream"):
        _kernel_mask(bad, L, "cpu")
    with pytest.raises(ValueError, match="dual-stream"):
        _kernel_mask(torch.ones(L, L, dtype=torch.bool), L, "cpu")


def test_rotary_rejects_mismatched_operands():
    """rotary (alodlm/model.py:41-46) checks its operands on the host before
    any launch: k shares q's rows, head_dim, dtype and device, and the
    cos/sin tables are [rows, head_dim] (the reference raises a broadcasting
    error for each of these)."""
    from alodlm_amd.model import rotary
    q, k = torch.zeros(6, 4, 8), torch.zeros(6, 2, 8)
    cos = sin = torch.zeros(6, 8)
    cases = [
        ((q, torch.zeros(5, 2, 8), cos, sin), "rows and head_dim"),
        ((q, torch.zeros(6, 2, 4), cos, sin), "rows and head_dim"),
        ((q, k.double(), cos, sin), "dtype"),
        ((q, k, torch.zeros(5, 8), sin), r"cos/sin must be \[6, 8\]"),
        ((q, k, cos, torch.zeros(6, 4)), r"cos/sin must be \[6, 8\]"),
        ((q, k, torch.zeros(2, 6, 8), sin), r"cos/sin must be \[6, 8\]"),
        ((torch.zeros(6, 4, 7), torch.zeros(6, 2, 7), torch.zeros(6, 7), torch.zeros(6, 7)),
         "even"),
        ((q.view(6, 32), k, cos, sin), "rows, heads, head_dim"),
    ]
    for args, message in cases:
        with pytest.raises(ValueError, match=message):
            rotary(*args)
    # well-formed operands pass the checks and stop at the device check
    with pytest.raises(ValueError, match="CUDA"):
        rotary(q, k, cos.unsqueeze(0), sin)


def test_layer_forward_rejects_short_tables_and_rows():
    """layer_forward (alodlm/model.py:49-76) checks the hidden width and the
    cos/sin tables against the layer before any launch."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer
    from alodlm_amd.model import layer_forward, training_layer
    cfg = Qwen3Config(hidden_size=32, intermediate_size=64, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=8, num_hidden_layers=1, vocab_size=64)
    layer = Qwen3DecoderLayer(cfg, 0)
    L = 6
    x = torch.zeros(L, 32)
    causal = torch.ones(L, L, dtype=torch.bool).tril()
    with pytest.raises(ValueError, match=r"cos/sin must be \[6, 8\]"):
        layer_forward(layer, x, torch.zeros(L - 1, 8), torch.zeros(L, 8), causal)
    with pytest.raises(ValueError, match=r"cos/sin must be \[6, 8\]"):
        training_layer(layer, x, torch.zeros(L, 8), torch.zeros(L, 4), causal)
    with pytest.raises(ValueError, match=r"hidden must be \[rows, 32\]"):
        layer_forward(layer, torch.zeros(L, 16), torch.zeros(L, 8), torch.zeros(L, 8), causal)
    with pytest.raises(ValueError, match="CUDA"):
        layer_forward(layer, x, torch.zeros(1, L, 8), torch.zeros(L, 8), causal)


def test_layer_functions_live_in_model_and_inference_binds_layer_forward():
    """The reference defines rotary, layer_forward and training_layer in
    alodlm/model.py:41-80 and its decoder imports layer_forward from there
    (alodlm/inference.py:11): the same names resolve here, and the decoder's
    module-level name is the one its layer calls look up."""
    import alodlm_amd as alodlm
    import alodlm_amd.inference as inference
    import alodlm_amd.model as model
    for name in ("rotary", "layer_forward", "training_layer", "GateHead", "ALoDLM"):
        assert hasattr(alodlm.model, name)
    assert inference.layer_forward is model.layer_forward
