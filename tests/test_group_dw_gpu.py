"""The looped layers' weight gradients as one product over the passes.

alodlm_gemm_segk sums A_i^T B_i over separate operand buffers in one float32
sum; the engine uses it to take a looped layer's projection gradients over
all of its recurrent applications (alodlm/model.py:152, whose autograd sums
the passes' nn.Linear gradients) at the layer's last backward application.
"""
import ctypes

import pytest
import torch

from alodlm_amd._lib import EPI_ACCUM, EPI_STORE_F32, call, ptr, query
from tests.helpers import log

pytestmark = pytest.mark.gpu

BF16 = 1


def _segk(As, Bs, C, epi, M, N, rows):
    a = (ctypes.c_void_p * len(As))(*[ptr(x) for x in As])
    b = (ctypes.c_void_p * len(Bs))(*[ptr(x) for x in Bs])
    need = query("alodlm_gemm_workspace", M, N, rows * len(As), epi, BF16)
    ws = torch.empty(max(need, 1), dtype=torch.float32, device="cuda")
    call("alodlm_gemm_segk", ctypes.addressof(a), ctypes.addressof(b), len(As), rows, M, N,
         ptr(C), N, M, N, 1.0, epi, ptr(ws) if need else None,
         torch.cuda.current_stream().cuda_stream)


def _gemm(A, B, C, epi, M, N, K):
    need = query("alodlm_gemm_workspace", M, N, K, epi, BF16)
    ws = torch.empty(max(need, 1), dtype=torch.float32, device="cuda")
    call("alodlm_gemm", ptr(A), M, 0, ptr(B), N, 0, ptr(C), N, None, 0, M, N, K, 1.0, epi, BF16,
         ptr(ws) if need else None, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("M,N,rows,nseg,epi", [
    (256, 256, 64, 2, EPI_STORE_F32),
    (512, 256, 1056, 3, EPI_ACCUM),      # two K splits, the second starting mid-segment
    (256, 256, 2048, 4, EPI_STORE_F32),  # eight splits of half a segment
    (768, 512, 96, 1, EPI_ACCUM),
    (4096, 1024, 512, 4, EPI_ACCUM),
])
def test_gemm_segk_equals_the_product_over_concatenated_rows(M, N, rows, nseg, epi):
    """The segmented product is bit-identical to alodlm_gemm over the
    segments' rows concatenated (same k order, same splits), and matches the
    float64 sum of A_i^T B_i."""
    log(f"gemm_segk M={M} N={N} rows={rows} segments={nseg} epi={epi}")
    g = torch.Generator(device="cuda").manual_seed(M + N + rows + nseg)
    As = [torch.randn(rows, M, generator=g, device="cuda").to(torch.bfloat16) for _ in range(nseg)]
    Bs = [torch.randn(rows, N, generator=g, device="cuda").to(torch.bfloat16) for _ in range(nseg)]
    C0 = torch.randn(M, N, generator=g, device="cuda")
    C = C0.clone()
    _segk(As, Bs, C, epi, M, N, rows)
    Ccat = C0.clone()
    _gemm(torch.cat(As), torch.cat(Bs), Ccat, epi, M, N, rows * nseg)
    torch.cuda.synchronize()
    assert torch.equal(C, Ccat)
    ref = sum(a.double().T @ b.double() for a, b in zip(As, Bs))
    if epi == EPI_ACCUM:
        ref = ref + C0.double()
    err = (C.double() - ref).abs().max().item()
    assert err <= 1e-5 * ref.abs().max().item() + 1e-4, err


def test_gemm_segk_rejects_unsupported_arguments():
    log("gemm_segk argument checks")
    A = torch.zeros(64, 256, dtype=torch.bfloat16, device="cuda")
    C = torch.zeros(256, 256, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        _segk([A] * 9, [A] * 9, C, EPI_ACCUM, 256, 256, 64)      # more than 8 segments
    with pytest.raises(ValueError):
        _segk([A[:48]], [A[:48]], C, EPI_ACCUM, 256, 256, 48)   # not a multiple of 32 rows
    with pytest.raises(ValueError):
        _segk([A], [A], C, 0, 256, 256, 64)                      # bf16 output epilogue


def _model(seed):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.model import ALoDLM
    cfg = Qwen3Config(hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                      tie_word_embeddings=False)
    with torch.device("meta"):
        backbone = Qwen3ForCausalLM(cfg)
    backbone = backbone.to_empty(device="cuda").to(torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(seed)
    with torch.no_grad():
        for name, p in backbone.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=g)
    model = ALoDLM(backbone, ModelConfig(loop_start=1, loop_end=3, max_depth=4,
                                         mask_token_id=151665, block_size=32))
    return model.cuda()


@pytest.mark.parametrize("accumulate", [False, True])
def test_grouped_weight_gradients_match_per_pass_products(accumulate):
    """A step whose looped layers (core 1-2, coda 3, four passes) take their
    projection gradients as one product per matrix gives the per-pass
    products' gradients up to float32 summation order; every other gradient
    is bit-identical."""
    log(f"grouped weight gradients, accumulate={accumulate}")
    model = _model(7)
    engine = model.engine()
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 151000, (512,), generator=g).cuda()
    bounds = torch.tensor([0, 256, 512])
    proj = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
    results = []
    for group in (False, True):
        engine.group_dw = group
        gen = torch.Generator(device="cuda").manual_seed(11)
        grads = None
        for _ in range(2 if accumulate else 1):
            out, state = engine.forward(ids, ids, bounds, True, generator=gen)
            grads = engine.backward(state, 1.0, accumulate=accumulate and grads is not None)
        torch.cuda.synchronize()
        results.append({n: engine.arena.view(grads, n).float().cpu().clone()
                        for n in engine.arena.names})
    engine.group_dw = None
    looped = [f"layers.{i}." for i in (1, 2, 3)]
    for name, a in results[0].items():
        b = results[1][name]
        if any(t in name for t in looped) and any(p in name for p in proj):
            scale = a.abs().max().item()
            assert scale > 0, name
            assert (a - b).abs().max().item() <= 1e-5 * scale, name
        else:
            assert torch.equal(a, b), name
