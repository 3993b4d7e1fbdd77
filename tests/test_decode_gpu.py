"""Cached adaptive decoding on the HIP kernels (alodlm/inference.py;
tests/test_inference.py): the reference's generations on the workflow
fixture's model (fresh and trained gate), the decode attention layout on both
attention paths, cache consistency and the reference's behavioural tests."""

import json
import math
import sys

import pytest
import torch

from tests.golden import HERE as GOLDEN

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
FIXTURE = GOLDEN / "workflow" / "fixture"
DECODE = json.loads((GOLDEN / "decode" / "decode.json").read_text())
RUN = json.loads((GOLDEN / "workflow" / "train.json").read_text())


def log(msg):
    print(f"[decode] {msg}", file=sys.stderr, flush=True)


def tokenizer():
    from alodlm_amd.data import load_tokenizer
    return load_tokenizer(FIXTURE / "base")


def base_model(dtype=torch.float32, **changes):
    from transformers import AutoModelForCausalLM
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.model import ALoDLM
    backbone = AutoModelForCausalLM.from_pretrained(str(FIXTURE / "base"), dtype=dtype)
    fields = dict(RUN["config"]["model"])
    fields["gate_init_pi"] = tuple(fields["gate_init_pi"])
    fields.update(changes)
    return ALoDLM(backbone, ModelConfig(**fields)).to(DEV)


def trained_model():
    from alodlm_amd.model import ALoDLM
    return ALoDLM.from_pretrained(GOLDEN / "decode" / "trained").to(DEV)


@pytest.mark.parametrize("which", ["base", "trained"])
def test_generation_matches_reference(which):
    """Token ids, exit depths, step/pass counts and stop reason equal the
    reference decoder's; first-pass halt probabilities to 1e-6."""
    from alodlm_amd.inference import DecodeConfig, Decoder
    model = base_model() if which == "base" else trained_model()
    decoder = Decoder(model, tokenizer())
    for case, want in zip(DECODE["cases"], DECODE[which]["runs"]):
        log(f"{which} {case['config']}")
        got = decoder.generate(case["prompt"], DecodeConfig(**case["config"]))
        for key in ("token_ids", "exit_depths", "outer_steps", "recurrent_passes",
                    "loop_token_passes", "stop_reason", "generated_tokens", "prompt_tokens"):
            assert got[key] == want[key], (which, case, key)
        assert got["first_pass_halt_probabilities"] == pytest.approx(
            want["first_pass_halt_probabilities"], abs=1e-6)
        assert got["wall_seconds"] >= got["prefill_seconds"] > 0


@pytest.mark.parametrize("which", ["base", "trained"])
def test_prefill_cache_matches_reference(which):
    from alodlm_amd.inference import DecodeConfig, Decoder, PrefixCache
    model = base_model() if which == "base" else trained_model()
    decoder = Decoder(model, tokenizer())
    cache = PrefixCache(model.config)
    empty = torch.empty(0, dtype=torch.long, device=DEV)
    with torch.inference_mode():
        window = decoder._window(torch.tensor([4, 7, 9, 12, 5], device=DEV),
                                 torch.arange(5, device=DEV), cache, empty, DecodeConfig(), empty)[0]
        cache.append(window, torch.arange(5, device=DEV))
    want = DECODE[which]["prefill_kv"]
    assert sorted(f"{a},{b}" for a, b in cache.values) == sorted(want)
    for key, (k, v) in cache.values.items():
        ref = want[f"{key[0]},{key[1]}"]
        torch.testing.assert_close(k.flatten().cpu(), torch.tensor(ref[0]), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(v.flatten().cpu(), torch.tensor(ref[1]), atol=1e-5, rtol=1e-5)


LAYOUT_CASES = [
    # (dtype, head_dim, tiled layout, prefix rows, window rows)
    (torch.bfloat16, 128, True, 0, 16),
    (torch.bfloat16, 128, True, 5, 16),
    (torch.bfloat16, 128, True, 127, 1),
    (torch.bfloat16, 128, True, 128, 16),
    (torch.bfloat16, 128, True, 300, 200),
    (torch.bfloat16, 64, True, 300, 16),
    (torch.bfloat16, 64, True, 0, 150),
    (torch.float32, 8, False, 0, 7),
    (torch.float32, 8, False, 37, 5),
    (torch.bfloat16, 8, False, 130, 16),
    (torch.float32, 64, False, 129, 3),
]


@pytest.mark.parametrize("dtype,dh,tiled,prefix,window", LAYOUT_CASES)
def test_window_attention_layout(dtype, dh, tiled, prefix, window):
    """The attention kernels on the decode layout equal softmax attention of
    each window row over every prefix key and the window keys up to itself
    (alodlm/inference.py:77-79), against torch float32."""
    from alodlm_amd import _lib
    from alodlm_amd.layers import WindowMask
    _lib.load()
    log(f"layout {dtype} dh={dh} tiled={tiled} P={prefix} W={window}")
    nq, nkv = 4, 2
    g = torch.Generator().manual_seed(prefix * 7 + window)
    q = torch.randn(window, nq * dh, generator=g).to(dtype)
    kc = torch.randn(prefix + window, nkv * dh, generator=g).to(dtype)
    vc = torch.randn(prefix + window, nkv * dh, generator=g).to(dtype)
    lay = WindowMask(prefix, window, tiled, DEV, block_size=4)
    q_all = torch.zeros(lay.q_rows, nq * dh, dtype=dtype, device=DEV)
    q_all[lay.q_off:] = q.to(DEV)
    kd, vd = kc.to(DEV), vc.to(DEV)
    o_all = torch.empty_like(q_all)
    lse = torch.empty(nq, lay.q_rows, dtype=torch.float32, device=DEV)
    shift = lay.base * nkv * dh * kd.element_size()
    _lib.call("alodlm_attention_fwd", _lib.ptr(q_all), _lib.ptr(kd) + shift, _lib.ptr(vd) + shift,
              nkv * dh, _lib.ptr(lay.boundaries), _lib.ptr(lay.row_segment), _lib.ptr(lay.tiles),
              0 if lay.tiles is None else lay.tiles.shape[0], _lib.ptr(o_all), _lib.ptr(lse),
              lay.q_rows, nq, nkv, dh, 4, _lib.dtype_code(dtype), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    qf = q.float().view(window, nq, dh)
    kf = kc.float().view(-1, nkv, dh).repeat_interleave(nq // nkv, 1)
    vf = vc.float().view(-1, nkv, dh).repeat_interleave(nq // nkv, 1)
    s = torch.einsum("qhd,khd->hqk", qf, kf) / math.sqrt(dh)
    allowed = torch.arange(prefix + window)[None, :] <= prefix + torch.arange(window)[:, None]
    s = s.masked_fill(~allowed, float("-inf"))
    ref = torch.einsum("hqk,khd->qhd", s.softmax(-1), vf).reshape(window, nq * dh)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(o_all[lay.q_off:].float().cpu(), ref, atol=tol, rtol=tol)


def test_generation_is_request_independent_and_respects_budget():
    """tests/test_inference.py:31-42."""
    from alodlm_amd.inference import DecodeConfig, Decoder
    decoder = Decoder(base_model(), tokenizer())
    cfg = DecodeConfig(q=.5, tau=.1, max_new_tokens=8, window_size=4)
    first = decoder.generate([4, 7, 9], cfg)
    decoder.generate([4, 7, 10, 11], DecodeConfig(q=.9, max_new_tokens=7, mode="left1"))
    second = decoder.generate([4, 7, 9], cfg)
    assert first["token_ids"] == second["token_ids"]
    assert first["exit_depths"] == second["exit_depths"]
    assert first["generated_tokens"] <= 8
    assert len(first["exit_depths"]) == len(first["token_ids"])


def test_q_controls_executed_recurrence():
    """tests/test_inference.py:44-49."""
    from alodlm_amd.inference import DecodeConfig, Decoder
    decoder = Decoder(base_model(), tokenizer())
    shallow = decoder.generate([4, 7, 9], DecodeConfig(q=0, tau=0, max_new_tokens=6, window_size=4))
    deep = decoder.generate([4, 7, 9], DecodeConfig(q=1, tau=0, max_new_tokens=6, window_size=4))
    assert shallow["recurrent_passes"] == shallow["outer_steps"]
    assert deep["recurrent_passes"] == 4 * deep["outer_steps"]


def _cache_matches_fresh_prefill(model, prompt, cfg, atol, rtol):
    """With one recurrent pass the cache after decoding holds the K/V a fresh
    prefill of the same tokens computes (tests/test_inference.py:51-84)."""
    from alodlm_amd.inference import Decoder, PrefixCache
    decoder = Decoder(model, tokenizer())
    out = decoder.generate(prompt, cfg)
    cache = decoder.cache
    tokens = torch.tensor(list(prompt) + out["token_ids"], device=DEV)[:cache.length]
    fresh = PrefixCache(model.config)
    empty = torch.empty(0, dtype=torch.long, device=DEV)
    with torch.inference_mode():
        window = decoder._window(tokens, torch.arange(len(tokens), device=DEV), fresh, empty, cfg,
                                 empty)[0]
        fresh.append(window, torch.arange(len(tokens), device=DEV))
    assert sorted(fresh.values) == sorted(cache.values)
    for key in cache.values:
        for actual, expected in zip(cache.values[key], fresh.values[key]):
            torch.testing.assert_close(actual.float(), expected.float(), atol=atol, rtol=rtol)
    return out


def test_prefix_cache_matches_observed_token_forward():
    from alodlm_amd.inference import DecodeConfig
    model = base_model()
    model.config.max_depth = 1  # after construction, as tests/test_inference.py:55 does
    out = _cache_matches_fresh_prefill(
        model, [4, 7, 9], DecodeConfig(q=0, mode="left1", max_new_tokens=8, window_size=4),
        1e-6, 1e-5)
    assert out["generated_tokens"] == 8


def test_bf16_head_dim_128_cache_matches_fresh_prefill():
    """The MFMA attention layout inside a real decode: a bf16 model with
    head_dim 128, a 150-token prompt (prefix rows past one 128-row tile)."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.inference import DecodeConfig
    from alodlm_amd.model import ALoDLM
    torch.manual_seed(0)
    backbone = Qwen3ForCausalLM(Qwen3Config(
        hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=2,
        num_key_value_heads=1, head_dim=128, vocab_size=64, max_position_embeddings=512,
        bos_token_id=1, eos_token_id=2, pad_token_id=0, tie_word_embeddings=False)).to(torch.bfloat16)
    model = ALoDLM(backbone, ModelConfig(loop_start=1, loop_end=2, mask_token_id=3,
                                         block_size=4)).to(DEV)
    model.config.max_depth = 1
    prompt = [5 + (i * 7) % 50 for i in range(150)]
    out = _cache_matches_fresh_prefill(
        model, prompt, DecodeConfig(q=0, mode="left1", max_new_tokens=20, window_size=8),
        3e-2, 3e-2)
    assert out["generated_tokens"] == 20


def test_committed_token_continues_as_latent_after_injection():
    """tests/test_inference.py:86-113 restated: the decoder's layer calls go
    through the module-level ``alodlm_amd.inference.layer_forward``
    (alodlm/inference.py:11,84), so a patched layer sees every core input.
    Row 0 commits on pass one (left-to-right, q = 1), restarts pass two from
    its token's embedding, and pass three carries the normalised output of
    pass two's core forward."""
    from unittest.mock import patch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.inference import DecodeConfig, Decoder, PrefixCache
    from alodlm_amd.model import ALoDLM
    log("latent carry through the patched layer_forward")
    torch.manual_seed(42)
    backbone = Qwen3ForCausalLM(Qwen3Config(
        hidden_size=32, intermediate_size=64, num_hidden_layers=3, num_attention_heads=4,
        num_key_value_heads=2, head_dim=8, vocab_size=64, max_position_embeddings=128,
        bos_token_id=1, eos_token_id=2, pad_token_id=0))
    model = ALoDLM(backbone, ModelConfig(loop_start=1, loop_end=2, mask_token_id=3,
                                         block_size=4)).to(DEV)
    cfg = DecodeConfig(q=1, tau=0, mode="left1", max_new_tokens=4)
    core_inputs = []

    def record_layer(layer, hidden, cos, sin, mask, prefix=None):
        if layer is model.backbone.model.layers[1]:
            core_inputs.append(hidden.clone())
        result = hidden + torch.arange(hidden.shape[-1], dtype=hidden.dtype,
                                       device=hidden.device) / 32
        return result, (hidden.unsqueeze(1), hidden.unsqueeze(1))

    ids = torch.full((4,), model.config.mask_token_id, device=DEV)
    rows = torch.arange(4, device=DEV)
    with torch.inference_mode(), patch("alodlm_amd.inference.layer_forward", record_layer):
        Decoder(model, tokenizer())._window(ids, rows, PrefixCache(model.config), rows, cfg, rows)
    assert len(core_inputs) == 4
    assert not torch.equal(core_inputs[1][0], core_inputs[2][0])
    with torch.inference_mode():
        expected = model.backbone.model.norm(
            core_inputs[1] + torch.arange(32, dtype=core_inputs[1].dtype, device=DEV) / 32)
    torch.testing.assert_close(core_inputs[2][0], expected[0])


def test_invalid_decode_config_and_context_fail():
    """tests/test_inference.py:115-122."""
    from alodlm_amd.inference import DecodeConfig, Decoder
    decoder = Decoder(base_model(), tokenizer())
    for cfg in (DecodeConfig(q=1.1), DecodeConfig(tau=float("nan")), DecodeConfig(window_size=0)):
        with pytest.raises(ValueError):
            decoder.generate([4, 7], cfg)
    with pytest.raises(ValueError):
        decoder.generate([4] * 100, DecodeConfig(max_new_tokens=40))
    with pytest.raises(ValueError):
        decoder.generate([], DecodeConfig())
    with pytest.raises(ValueError):
        decoder.generate([4, 64], DecodeConfig(max_new_tokens=4))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,vocab", [(7, 1000), (3, 64), (2, 151936)])
def test_decode_readout(dtype, rows, vocab):
    """argmax (first of equal maxima, as torch.argmax) and the entropy of
    log_softmax(logits.float()) (alodlm/inference.py:115-118); the logits are
    left unchanged."""
    from alodlm_amd import _lib
    _lib.load()
    g = torch.Generator().manual_seed(rows * vocab)
    logits = (3 * torch.randn(rows, vocab, generator=g)).to(dtype)
    logits[0, vocab // 3] = logits[0, 2 * vocab // 3] = logits[0].max() + 1  # tie: first wins
    if rows > 2:
        logits[2] = 0.5  # all equal: index 0, entropy log(V)
    dev = logits.to(DEV)
    before = dev.clone()
    idx = torch.empty(rows, dtype=torch.int64, device=DEV)
    ent = torch.empty(rows, dtype=torch.float32, device=DEV)
    _lib.call("alodlm_decode_readout", _lib.ptr(dev), rows, vocab, _lib.ptr(idx), _lib.ptr(ent),
              _lib.dtype_code(dtype), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    assert torch.equal(dev, before)
    assert idx.cpu().tolist() == logits.float().argmax(-1).tolist()
    logp = logits.double().log_softmax(-1)
    ref = -(logp.exp() * logp).sum(-1)
    torch.testing.assert_close(ent.cpu().double(), ref, atol=1e-4, rtol=1e-5)
    if rows > 2:
        assert abs(float(ent[2]) - math.log(vocab)) < 1e-4


def _ledger_state(n, ws, gen, cache_rows, seed, max_new=100000, stop=(2,), mode="entropy",
                  tau=0.4, q=0.5):
    """A decode state whose ledger holds n slots with a random committed/open
    pattern (committed slots carry tokens >= 5, open slots the mask id 3)."""
    from alodlm_amd.inference import (CACHE, GENERATED, HEADER, LEDGER, DecodeConfig,
                                      _DeviceState)
    cfg = DecodeConfig(window_size=ws, max_new_tokens=max_new, mode=mode, tau=tau, q=q)
    st = _DeviceState(DEV, 2 * ws, cfg, 4, 3, list(stop))
    g = torch.Generator().manual_seed(seed)
    lead = int(torch.randint(0, max(n, 1), (1,), generator=g)) if n else 0
    is_open = (torch.rand(n, generator=g) < 0.4).to(torch.int32)
    is_open[:lead] = 0
    tokens = torch.randint(5, 50, (n,), generator=g)
    tokens[is_open.bool()] = 3
    depth = torch.randint(1, 5, (n,), generator=g, dtype=torch.int32) * (1 - is_open)
    halt = torch.rand(n, generator=g) * (1 - is_open)
    for name, t in (("slot_token", tokens), ("slot_open", is_open), ("slot_depth", depth),
                    ("slot_halt", halt)):
        st[name][:n].copy_(t)
    h = torch.zeros(HEADER, dtype=torch.int64)
    h[LEDGER], h[GENERATED], h[CACHE] = n, gen, cache_rows
    st["header"].copy_(h)
    return st, cfg, tokens, is_open, depth, halt


def _expected_plan(tokens, is_open, ws, gen, cache_rows, max_new, penalty):
    import numpy as np
    n = len(tokens)
    opened = np.nonzero(is_open.numpy())[0]
    p = int(opened[0]) if len(opened) else n
    n2 = max(n, p + min(ws, max_new - gen - p))
    tok = np.concatenate([tokens.numpy(), np.full(n2 - n, 3)])
    op = np.concatenate([is_open.numpy(), np.ones(n2 - n, dtype=np.int32)])
    closed, masks = np.nonzero(op == 0)[0], np.nonzero(op == 1)[0]
    order = np.concatenate([closed, masks])
    offset = (masks - p).astype(np.float32) * np.float32(penalty)
    return dict(p=p, n2=n2, n_obs=len(closed), row_token=tok[order], row_position=cache_rows + order,
                mask_slot=masks, mask_offset=offset)


@pytest.mark.parametrize("n,ws,gen,seed", [(0, 4, 0, 0), (5, 8, 3, 1), (600, 700, 10, 2),
                                           (300, 256, 0, 3), (1000, 513, 7, 4)])
def test_decode_plan_lays_out_the_window(n, ws, gen, seed):
    """alodlm_decode_plan (inference.py:185-210) against numpy: the committed
    run, ledger growth, committed-first row order, positions, mask slots and
    position penalties, across several 256-slot chunks."""
    from alodlm_amd import _lib
    from alodlm_amd.inference import DONE, LEDGER, OBSERVED, PREFIX, WINDOW
    log(f"plan n={n} ws={ws} gen={gen}")
    n = min(n, ws)  # a ledger never holds more than window_size slots
    st, cfg, tokens, is_open, _, _ = _ledger_state(n, ws, gen, 77, seed)
    _lib.call("alodlm_decode_plan", st.ref, _lib.stream_handle(DEV))
    h = st.read_header()
    want = _expected_plan(tokens, is_open, ws, gen, 77, cfg.max_new_tokens, cfg.penalty)
    n2, n_obs = want["n2"], want["n_obs"]
    assert (h[DONE], h[LEDGER], h[WINDOW], h[OBSERVED], h[PREFIX]) == (0, n2, n2, n_obs, want["p"])
    assert st["row_token"][:n2].cpu().tolist() == want["row_token"].tolist()
    assert st["row_position"][:n2].cpu().tolist() == want["row_position"].tolist()
    assert st["mask_row"][:n2 - n_obs].cpu().tolist() == list(range(n_obs, n2))
    assert st["mask_slot"][:n2 - n_obs].cpu().tolist() == want["mask_slot"].tolist()
    assert torch.equal(st["mask_offset"][:n2 - n_obs].cpu(), torch.from_numpy(want["mask_offset"]))
    assert st["replace_depth"][:n2].cpu().tolist() == [4] * n2
    assert st["mask_survival"][:n2 - n_obs].cpu().tolist() == [1.0] * (n2 - n_obs)


@pytest.mark.parametrize("budget_left", [False, True])
def test_decode_plan_ends_on_stop_token_or_budget(budget_left):
    """A stop token inside the committed run ends decoding with the run up to
    it emitted (reason eos); a run that reaches the budget is emitted whole
    (reason length)."""
    from alodlm_amd import _lib
    from alodlm_amd.inference import DONE, GENERATED, REASON, REASON_EOS
    ws, n, gen = 300, 300, 5
    max_new = gen + 40 if budget_left else 100000
    st, _, tokens, is_open, depth, halt = _ledger_state(n, ws, gen, 0, 11, max_new=max_new)
    st["slot_open"][:60].zero_()
    run = 60 if budget_left else 59
    if budget_left:
        st["slot_open"][40] = 1  # the committed run is 40 slots = the budget left
        run = 40
    else:
        st["slot_token"][59] = 2  # a stop token at slot 59 of a 60-slot run
    tok = st["slot_token"][:run].cpu().clone()
    dep, hal = st["slot_depth"][:run].cpu().clone(), st["slot_halt"][:run].cpu().clone()
    _lib.call("alodlm_decode_plan", st.ref, _lib.stream_handle(DEV))
    h = st.read_header()
    emitted = 40 if budget_left else 59
    assert h[DONE] == 1 and h[GENERATED] == gen + emitted
    assert (h[REASON] == REASON_EOS) == (not budget_left)
    assert st["out_token"][gen:gen + emitted].cpu().tolist() == tok[:emitted].tolist()
    assert st["out_depth"][gen:gen + emitted].cpu().tolist() == dep[:emitted].tolist()
    assert torch.equal(st["out_halt"][gen:gen + emitted].cpu(), hal[:emitted])


def test_decode_commit_fallback_retires_and_replans():
    """At the last depth with nothing agreed (tau = 0) the mask row of least
    adjusted entropy commits (first of equal minima); with `finish` the
    window is retired - its committed run emitted, the commitment written to
    its slot, the ledger shifted across chunks - and the next window planned."""
    from alodlm_amd import _lib
    from alodlm_amd.inference import (CACHE, DONE, GENERATED, LEDGER, OBSERVED, PREFIX, STOP,
                                      WINDOW)
    ws, n, gen, cache_rows = 400, 400, 3, 50
    st, cfg, tokens, is_open, depth, halt = _ledger_state(n, ws, gen, cache_rows, 5, tau=0.0)
    sh = _lib.stream_handle(DEV)
    _lib.call("alodlm_decode_plan", st.ref, sh)
    h = st.read_header()
    rows, n_obs, p = h[WINDOW], h[OBSERVED], h[PREFIX]
    count = rows - n_obs
    assert count > 256 and p > 0
    ledger = st["slot_token"][:rows].cpu().clone()
    opened = st["slot_open"][:rows].cpu().clone()
    g = torch.Generator().manual_seed(9)
    entropy = torch.rand(count, generator=g) + 1.0
    pick = count - 3
    entropy[pick] = 0.0
    entropy[pick + 1] = 0.0  # equal minimum after the pick: the first wins
    st["mask_offset"][:count].zero_()
    predicted = torch.randint(100, 200, (count,), generator=g)
    st["entropy"][:count].copy_(entropy)
    st["predicted"][:count].copy_(predicted)
    gate = torch.randn(rows, generator=g).to(DEV)
    # without `finish` the window's state stays for inspection
    _lib.call("alodlm_decode_commit", st.ref, _lib.ptr(gate), count, 3, 0, sh)
    h1 = st.read_header()
    assert h1[STOP] == 1 and h1[GENERATED] == gen and h1[WINDOW] == rows
    committed = st["mask_committed"][:count].cpu()
    assert committed.nonzero().flatten().tolist() == [pick]
    assert int(st["mask_token"][pick]) == int(predicted[pick])
    assert int(st["mask_exit"][pick]) == 4
    hazard = torch.sigmoid(gate.cpu()[st["mask_row"][:count].cpu().long()])
    torch.testing.assert_close(st["mask_first_hazard"][:count].cpu(), torch.zeros(count))
    torch.testing.assert_close(st["mask_survival"][:count].cpu(), 1 - hazard, rtol=1e-6, atol=1e-7)
    slot = int(st["mask_slot"][pick])  # (the next plan rewrites the mask rows)
    # again with `finish`: the row committed above is kept (no second fallback)
    _lib.call("alodlm_decode_commit", st.ref, _lib.ptr(gate), count, 3, 1, sh)
    h2 = st.read_header()
    assert h2[STOP] == 1 and h2[DONE] == 0
    assert h2[GENERATED] == gen + p and h2[CACHE] == cache_rows + p
    assert st["out_token"][gen:gen + p].cpu().tolist() == ledger[:p].tolist()
    # the ledger after retirement, then the next plan from it
    after_tok, after_open = ledger.clone(), opened.clone()
    after_tok[slot], after_open[slot] = int(predicted[pick]), 0
    after_tok, after_open = after_tok[p:], after_open[p:]
    want = _expected_plan(after_tok, after_open, ws, gen + p, cache_rows + p, cfg.max_new_tokens,
                          cfg.penalty)
    assert (h2[LEDGER], h2[WINDOW], h2[OBSERVED], h2[PREFIX]) == (
        want["n2"], want["n2"], want["n_obs"], want["p"])
    assert st["row_token"][:want["n2"]].cpu().tolist() == want["row_token"].tolist()
    assert st["row_position"][:want["n2"]].cpu().tolist() == want["row_position"].tolist()
