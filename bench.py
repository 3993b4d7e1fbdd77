"""Benchmark: ALoDLM full training step on one MI355X.

One step = ALoDLM.forward on one pack of synthetic tokens + backward +
global-norm clip + AdamW with float32 masters, all on the HIP kernels.

  --model 1.7b (default)  Qwen3-1.7B shapes, recurrent core = layers 0-28 run
                          K = 4 times, one pack of 8 x 2048 tokens (dual-stream
                          N = 32768 rows)
  --model 8b              Qwen3-8B shapes, prelude 0-10 / core 10-26 / coda
                          26-36, K = 4, one sequence of 2048 tokens (N = 4096)

After the headline step, the other benchmark workloads run as sub-records of
the same line (``sub_records``; --no-sub-records skips them):

  8b_step       the ALoDLM-8B step above (when the headline is 1.7B)
  core_block    one Qwen3-8B layer (hidden 4096, 32/8 heads, intermediate
                12288) run 4 times with shared weights from N(0, 1) hidden
                states, 4 x 2048 tokens (16384 dual-stream rows) under the
                training mask, gates after each pass, committed rows
                re-embedded from a 151936 x 4096 table; forward + backward
  readout       final hidden states [8192 x 2048] for each of 4 passes,
                LM head 2048 x 151936, masked cross-entropy and the objective
                (masks Bernoulli(t), t ~ U(0, 1) per 2048-row sequence);
                forward + backward

Prints one JSON line (metric: train tokens/s of the headline step) with:
  roofline      the dominant kernel class (by time, from HIP events around its
                launches on the launch stream, over a few steps after the
                timed ones so that those carry no per-launch events):
                algorithmic FLOPs per launch / average launch time vs 2.5 PFLOP/s
  step_ms       min / median / max of the timed steps (HIP events between
                steps), and the caching allocator's free-and-retry count and
                device allocations over them (``allocator``)
  mfu           whole-step algorithmic FLOPs / step time / bf16 dense peak
  cpu_baseline  the CPU oracle timed on this host on a bounded sample (three
                decoder-layer fwd+bwd passes over one 4096-row dual-stream
                segment and one LM-head readout fwd+bwd over 2048 rows, about
                10-30 s), extrapolated to the full step by layer-application
                and readout-row counts.
"""

import argparse
import json
import math
import os
import sys
import time

import torch

PEAK_BF16 = 2516.6e12   # dense bf16 MFMA FLOP/s of MI355X (256 CU x 4096 FLOP/clk x 2.4 GHz)
PEAK_HBM = 8.0e12
ROOT = os.path.dirname(os.path.abspath(__file__))


MODELS = {
    # Qwen3-1.7B; the repository's 1.7B topology runs every layer as the core
    "1.7b": dict(hidden_size=2048, intermediate_size=6144, num_hidden_layers=28,
                 num_attention_heads=16, num_key_value_heads=8, loop=(0, 28),
                 segments=[2048] * 8, name="ALoDLM-1.7B", qwen="Qwen3-1.7B",
                 traffic="gemm_bf16_1p7b_step_traffic.md"),
    # Qwen3-8B; prelude [0, 10), core [10, 26), coda [26, 36)
    "8b": dict(hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
               num_attention_heads=32, num_key_value_heads=8, loop=(10, 26),
               segments=[2048], name="ALoDLM-8B", qwen="Qwen3-8B",
               traffic="gemm_bf16_8b_step_traffic.md"),
}


def qwen3_config(spec):
    from transformers import Qwen3Config
    return Qwen3Config(hidden_size=spec["hidden_size"], intermediate_size=spec["intermediate_size"],
                       num_hidden_layers=spec["num_hidden_layers"],
                       num_attention_heads=spec["num_attention_heads"],
                       num_key_value_heads=spec["num_key_value_heads"], head_dim=128,
                       vocab_size=151936, max_position_embeddings=40960, rms_norm_eps=1e-6,
                       rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                       tie_word_embeddings=False, bos_token_id=151643, eos_token_id=151645)


def build_model(spec, device, dtype, seed=0):
    """Random-init Qwen3 backbone (N(0, 0.02), unit norms) + a fresh gate with
    the configuration's loop topology."""
    from transformers import Qwen3ForCausalLM
    from alodlm_amd.config import ModelConfig
    from alodlm_amd.model import ALoDLM
    with torch.device("meta"):
        backbone = Qwen3ForCausalLM(qwen3_config(spec))
    backbone = backbone.to_empty(device=device).to(dtype)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in backbone.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=g)
    start, end = spec["loop"]
    cfg = ModelConfig(loop_start=start, loop_end=end, max_depth=4, mask_token_id=151665,
                      block_size=32)
    return ALoDLM(backbone, cfg)


def step_flops(dims, cfg, seg_lengths, rows_per_depth):
    """Algorithmic FLOPs of one step (recompute not credited)."""
    from alodlm_amd.batch import allowed_pairs
    H, I, V = dims.hidden, dims.intermediate, dims.vocab
    qd, kd = dims.heads * dims.head_dim, dims.kv_heads * dims.head_dim
    p_layer = H * (qd + 2 * kd) + qd * H + 3 * H * I
    n_rows = 2 * sum(seg_lengths)
    apps = cfg.loop_start + cfg.max_depth * (dims.layers - cfg.loop_start)
    pairs = sum(allowed_pairs(L, cfg.block_size) for L in seg_lengths)
    gemm = apps * 6 * p_layer * n_rows
    attn = apps * 12 * dims.head_dim * dims.heads * pairs
    head = 6 * H * V * sum(rows_per_depth) + 6 * H * n_rows * cfg.max_depth
    return gemm, attn, head


class KernelTimer:
    """HIP events around every GEMM / attention launch of the engine."""

    def __init__(self):
        self.records = {}
        self.gemm_bytes = 0

    def wrap(self, engine):
        timer = self
        gemm, fwd, bwd = engine._gemm, engine._attention_fwd, engine._attention_bwd

        def timed(kind, fn, flops_fn, bytes_fn=None):
            def run(*args, **kwargs):
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                out = fn(*args, **kwargs)
                end.record()
                timer.records.setdefault(kind, []).append((start, end, flops_fn(*args, **kwargs)))
                if bytes_fn is not None:
                    timer.gemm_bytes += bytes_fn(*args, **kwargs)
                return out
            return run

        def segk_flops(segs, rows, epi):  # a looped layer's grouped weight gradient
            return 2.0 * segs[0][6] * segs[0][7] * rows * len(segs)

        def segk_bytes(segs, rows, epi):
            A, lda, B, ldb, C, ldc, M, N = segs[0]
            return gemm_bytes(A, lda, 0, B, ldb, 0, C, ldc, M, N, rows * len(segs), epi=epi)

        engine._gemm = timed("gemm_bf16", gemm, lambda *a, **k: 2.0 * a[8] * a[9] * a[10],
                             gemm_bytes)
        engine._gemm_segk = timed("gemm_bf16", engine._gemm_segk, segk_flops, segk_bytes)
        engine._attention_fwd = timed("attention_fwd", fwd, engine._attention_fwd_flops)
        engine._attention_bwd = timed("attention_bwd", bwd, engine._attention_bwd_flops)

    def summary(self):
        out = {}
        for kind, recs in self.records.items():
            ms = sum(s.elapsed_time(e) for s, e, _ in recs)
            flops = sum(f for _, _, f in recs)
            out[kind] = {"launches": len(recs), "ms": ms, "flops": flops}
        return out


def device_info():
    """Compute units and peak engine clock of cuda:0 as the HIP runtime reports
    them, and the dense bf16 MFMA peak they imply (4096 FLOP per CU and clock);
    the published 2516.6 TFLOP/s is what the roofline fractions use."""
    import ctypes
    from alodlm_amd import _lib
    cus, khz = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.call("alodlm_device_info", 0, ctypes.addressof(cus), ctypes.addressof(khz))
    return {"compute_units": cus.value, "max_clock_mhz": round(khz.value / 1000.0, 1),
            "peak_bf16_tflops_from_clock": round(cus.value * 4096 * khz.value * 1e3 / 1e12, 1)}


def gemm_bytes(A, lda, a_k, B, ldb, b_k, C, ldc, M, N, K, alpha=1.0, epi=0, R=None, ldr=0):
    """Algorithmic HBM bytes of one GEMM launch: A and B read once (bf16), C
    written once (bf16 store, or float32 for the first contribution to a
    gradient), plus R read (residual) or the float32 C read and written back
    (accumulate)."""
    from alodlm_amd._lib import EPI_ACCUM, EPI_RESIDUAL, EPI_STORE, EPI_STORE_F32
    c_bytes = {EPI_STORE: 2 * M * N, EPI_RESIDUAL: 4 * M * N, EPI_ACCUM: 8 * M * N,
               EPI_STORE_F32: 4 * M * N}[epi]
    return 2 * (M * K + N * K) + c_bytes


def profiled_traffic(path):
    """HBM bytes per GEMM launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes over this benchmark, read from the committed profile summary."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def _roofline(timer, steps, spec=None):
    """Roofline of the dominant kernel class (by time) from the HIP events."""
    summary = timer.summary()
    dom = max(summary, key=lambda k: summary[k]["ms"])
    s = summary[dom]
    achieved = s["flops"] / s["launches"] / (s["ms"] / s["launches"] / 1000.0)
    roof = {"bound": "mfma", "kernel": dom, "launches_per_step": s["launches"] // steps,
            "avg_launch_us": round(1000.0 * s["ms"] / s["launches"], 1),
            "achieved": round(achieved / 1e12, 1), "peak": round(PEAK_BF16 / 1e12, 1),
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4), "traffic": None}
    if dom == "gemm_bf16":
        roof["algorithmic_bytes_per_launch"] = timer.gemm_bytes // s["launches"]
        if spec is not None:
            traffic_profile = os.path.join(ROOT, "profiles", spec["traffic"])
            roof["traffic"] = profiled_traffic(traffic_profile)
            roof["traffic_source"] = os.path.relpath(traffic_profile, ROOT)
    classes = {k: {"ms_per_step": round(v["ms"] / steps, 1),
                   "tflops": round(v["flops"] / (v["ms"] / 1000) / 1e12, 1)}
               for k, v in summary.items()}
    return roof, classes


def _allocator_counters(device):
    """Cumulative caching-allocator counters: free-and-retry events (each one
    synchronizes the device and returns cached blocks), device allocations
    and frees, and the peak of reserved bytes."""
    s = torch.cuda.memory_stats(device)
    return {"num_alloc_retries": s.get("num_alloc_retries", 0),
            "num_device_alloc": s.get("num_device_alloc", 0),
            "num_device_free": s.get("num_device_free", 0),
            "reserved_peak": s.get("reserved_bytes.all.peak", 0)}


def _release():
    import gc
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def run_step(spec, device, steps, warmup, kernel_timing):
    """The full training step of ``spec``: returns (record, model facts)."""
    from alodlm_amd.optim import FusedAdamW, param_groups
    torch.cuda.reset_peak_memory_stats(device)
    dtype = torch.bfloat16
    model = build_model(spec, device, dtype)
    engine = model.engine()
    timer = None
    gen = torch.Generator().manual_seed(0)
    seg_lengths = spec["segments"]
    ids = torch.randint(0, 151936, (sum(seg_lengths),), generator=gen).to(device)
    labels = ids.clone()
    bounds = torch.tensor([0] + [sum(seg_lengths[:i + 1]) for i in range(len(seg_lengths))])
    torch.cuda.manual_seed(0)
    opt = FusedAdamW(param_groups(model, 0.01), lr=1e-5, max_grad_norm=1.0)

    def one_step():
        loss, metrics = model(ids, labels, bounds)
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss.detach()

    for i in range(warmup):
        loss = one_step()
        print(f"[bench] {spec['name']} warmup step {i} loss {float(loss):.4f}", file=sys.stderr,
              flush=True)
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    alloc = [_allocator_counters(device)]
    t0 = time.perf_counter()
    marks[0].record()
    rows = []
    for i in range(steps):
        loss = one_step()
        marks[i + 1].record()
        alloc.append(_allocator_counters(device))
        rows.append(list(engine.last_rows))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = [a.elapsed_time(b) for a, b in zip(marks, marks[1:])]
    for i, t in enumerate(step_ms):
        d = {k: alloc[i + 1][k] - alloc[i][k] for k in alloc[0]}
        print(f"[bench] {spec['name']} step {i}: {t:.1f} ms, allocator retries "
              f"{d['num_alloc_retries']}, device mallocs {d['num_device_alloc']}, frees "
              f"{d['num_device_free']}", file=sys.stderr, flush=True)
    print(f"[bench] {spec['name']}: timed {steps} steps in {elapsed:.3f}s loss {float(loss):.4f}",
          file=sys.stderr, flush=True)
    if kernel_timing:
        # the kernel classes come from a separate pass of a few more steps
        # with HIP events around every GEMM / attention launch, so that the
        # timed steps above carry no per-launch instrumentation
        timer = KernelTimer()
        timer.wrap(engine)
        kernel_steps = min(steps, 3)
        for _ in range(kernel_steps):
            one_step()
        torch.cuda.synchronize()
    ms = 1000.0 * elapsed / steps
    tokens = sum(seg_lengths)
    gemm_f, attn_f, head_f = step_flops(engine.dims, model.config, seg_lengths,
                                        [sum(r) / len(r) for r in zip(*rows)])
    step_f = gemm_f + attn_f + head_f
    record = {
        "workload": (f"{spec['name']} full training step (fwd+bwd+clip+AdamW fp32 master): "
                     f"{spec['qwen']} shapes, random init, untied, loop "
                     f"{spec['loop'][0]}-{spec['loop'][1]}, max_depth 4"),
        "value": round(tokens * steps / elapsed, 2), "unit": "tokens/s", "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 2), "global_batch": len(seg_lengths),
        "seq_len": 2048, "dual_stream_rows": 2 * tokens,
        "memory": {"peak_allocated_gib": round(torch.cuda.max_memory_allocated(device) / 2**30, 1),
                   "kept_forward_outputs": {"rotary_qk": bool(engine._keep and engine._keep[0]),
                                            "norm_outputs": bool(engine._keep and engine._keep[1])}},
        "mfu": round(step_f / (ms / 1000.0) / PEAK_BF16, 4),
        "step_tflop": round(step_f / 1e12, 1),
        "step_ms": {"min": round(min(step_ms), 2),
                    "median": round(sorted(step_ms)[len(step_ms) // 2], 2),
                    "max": round(max(step_ms), 2)},
        "allocator": {"alloc_retries": alloc[-1]["num_alloc_retries"] - alloc[0]["num_alloc_retries"],
                      "device_mallocs": alloc[-1]["num_device_alloc"] - alloc[0]["num_device_alloc"],
                      "device_frees": alloc[-1]["num_device_free"] - alloc[0]["num_device_free"],
                      "reserved_peak_gib": round(alloc[-1]["reserved_peak"] / 2**30, 1)},
    }
    if timer is not None:
        record["roofline"], record["kernel_classes"] = _roofline(timer, kernel_steps, spec)
        record["roofline"]["timed_steps"] = kernel_steps
    cfg = model.config
    facts = {"apps": cfg.loop_start + cfg.max_depth * (engine.dims.layers - cfg.loop_start),
             "segments": len(seg_lengths), "tokens": tokens,
             "readout_rows": sum(sum(r) for r in rows) / len(rows)}
    del opt, model, engine, timer
    _release()
    return record, facts


def run_core_block(device, steps, warmup, kernel_timing):
    """One Qwen3-8B layer x 4 passes over 4 x 2048 tokens, forward + backward."""
    from alodlm_amd.batch import allowed_pairs, build_batch
    spec = dict(MODELS["8b"], num_hidden_layers=1, loop=(0, 1))
    model = build_model(spec, device, torch.bfloat16, seed=1)
    with torch.no_grad():
        model.backbone.model.embed_tokens.weight.normal_(
            0.0, 1.0, generator=torch.Generator(device=device).manual_seed(2))
    engine = model.engine()
    g = torch.Generator(device=device).manual_seed(3)
    tokens = [2048] * 4
    ids = torch.randint(0, 151936, (sum(tokens),), generator=g, device=device)
    batch = build_batch(ids, ids.clone(), torch.tensor([0, 2048, 4096, 6144, 8192]), 32, 151665,
                        generator=g)
    N, H = 2 * sum(tokens), 4096
    x0 = torch.randn(N, H, generator=g, device=device).to(torch.bfloat16)
    douts = [torch.randn(N, H, generator=g, device=device).to(torch.bfloat16) for _ in range(4)]

    def one_step():
        outs, gates, exits, state = engine.core_forward(x0, batch, True, generator=g)
        return engine.core_backward(state, douts)

    for _ in range(warmup):
        one_step()
    timer = None
    if kernel_timing:
        timer = KernelTimer()
        timer.wrap(engine)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = 1000.0 * elapsed / steps
    d = engine.dims
    qd, kd = d.heads * d.head_dim, d.kv_heads * d.head_dim
    p_layer = H * (qd + 2 * kd) + qd * H + 3 * H * d.intermediate
    pairs = sum(allowed_pairs(L, 32) for L in tokens)
    flops = 4 * (6 * p_layer * N + 12 * d.head_dim * d.heads * pairs)
    record = {"workload": ("core block: one Qwen3-8B layer (hidden 4096, 32/8 heads, head_dim "
                           "128, intermediate 12288) x 4 passes with shared weights, 4 x 2048 "
                           "tokens (16384 dual-stream rows) under the training mask, gates after "
                           "each pass, committed rows re-embedded from a 151936 x 4096 table; "
                           "fwd+bwd from N(0, 1) hidden states"),
              "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 2),
              "tflop_per_step": round(flops / 1e12, 2),
              "value": round(flops / (ms / 1000.0) / 1e12, 1), "unit": "TFLOP/s",
              "mfu": round(flops / (ms / 1000.0) / PEAK_BF16, 4)}
    if timer is not None:
        record["roofline"], record["kernel_classes"] = _roofline(timer, steps)
    print(f"[bench] core block: {ms:.2f} ms/step", file=sys.stderr, flush=True)
    del model, engine, timer, batch, x0, douts
    _release()
    return record


def run_readout(device, steps, warmup, kernel_timing):
    """Readout + objective from 4 passes of [8192 x 2048] final hidden states."""
    from alodlm_amd.core import readout_batch
    spec = dict(MODELS["1.7b"], num_hidden_layers=1, loop=(0, 1))
    model = build_model(spec, device, torch.bfloat16, seed=4)
    engine = model.engine()
    g = torch.Generator(device=device).manual_seed(5)
    N, H, S, L = 8192, 2048, 4, 2048
    finals = [torch.randn(N, H, generator=g, device=device).to(torch.bfloat16) for _ in range(4)]
    targets = torch.randint(0, 151936, (N,), generator=g, device=device)
    t = torch.rand(S, generator=g, device=device).clamp_min(1e-8).repeat_interleave(L)
    masked = torch.rand(N, generator=g, device=device) < t
    prob = torch.where(masked, t, torch.zeros_like(t))
    batch = readout_batch(targets, torch.arange(S + 1, device=device) * L, masked, prob)

    def one_step():
        out, state = engine.readout_forward(finals, batch, True, generator=g)
        engine.readout_backward(state, 1.0)
        return list(engine.last_rows)

    for _ in range(warmup):
        one_step()
    timer = None
    if kernel_timing:
        timer = KernelTimer()
        timer.wrap(engine)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rows = [one_step() for _ in range(steps)]
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = 1000.0 * elapsed / steps
    mean_rows = sum(sum(r) for r in rows) / len(rows)
    flops = 6 * H * 151936 * mean_rows + 6 * H * N * 4
    record = {"workload": ("fused readout/objective: final hidden states [8192 x 2048] per pass "
                           "x 4 passes, LM head 2048 x 151936, final norm + gate, exit sampling, "
                           "masked cross-entropy and the NELBO / sequence-credit objective "
                           "(masks Bernoulli(t), t ~ U(0, 1) per 2048-row sequence); fwd+bwd"),
              "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 2),
              "loss_bearing_rows_per_step": round(mean_rows, 1),
              "tflop_per_step": round(flops / 1e12, 2),
              "value": round(flops / (ms / 1000.0) / 1e12, 1), "unit": "TFLOP/s",
              "mfu": round(flops / (ms / 1000.0) / PEAK_BF16, 4)}
    if timer is not None:
        record["roofline"], record["kernel_classes"] = _roofline(timer, steps)
    print(f"[bench] readout: {ms:.2f} ms/step", file=sys.stderr, flush=True)
    del model, engine, timer, finals, batch
    _release()
    return record


def run_attention(spec, device, steps, warmup):
    """The attention kernels alone at a step configuration's layer shape: one
    pack of the configuration's segments under the training mask, random
    bf16 q/k/v/dO; forward, then backward (dQ pass, dK/dV pass), each timed
    with HIP events on the launch stream.  For kernel profiling; not a line
    of the benchmark's metric."""
    from alodlm_amd import _lib
    from alodlm_amd.layers import DualStreamMask
    nq, nkv, dh = spec["num_attention_heads"], spec["num_key_value_heads"], 128
    offsets = [0]
    for L in spec["segments"]:
        offsets.append(offsets[-1] + L)
    mask = DualStreamMask(offsets, 32, device)
    N = mask.rows
    g = torch.Generator(device=device).manual_seed(5)
    q, do = (torch.randn(N, nq * dh, generator=g, device=device).to(torch.bfloat16)
             for _ in range(2))
    k, v = (torch.randn(N, nkv * dh, generator=g, device=device).to(torch.bfloat16)
            for _ in range(2))
    o = torch.empty_like(q)
    lse = torch.empty(nq, N, dtype=torch.float32, device=device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    n_tiles = mask.tiles.shape[0]
    ws = torch.empty(_lib.query("alodlm_attention_bwd_workspace", N, nq, nkv, dh, n_tiles,
                                mask.ds_blocks),
                     dtype=torch.float32, device=device)
    st = _lib.stream_handle(device)
    P = _lib.ptr
    code = _lib.BF16_CODE

    def fwd():
        _lib.call("alodlm_attention_fwd", P(q), P(k), P(v), nkv * dh, P(mask.boundaries),
                  P(mask.row_segment), P(mask.tiles), n_tiles, P(o), P(lse), N, nq, nkv, dh, 32,
                  code, st)

    def bwd(stored=True):
        _lib.call("alodlm_attention_bwd", P(q), P(k), P(v), nkv * dh, P(o), P(lse), P(do),
                  P(mask.boundaries), P(mask.row_segment), P(mask.tiles), n_tiles, P(dq), P(dk),
                  P(dv), nkv * dh, P(ws), P(mask.ds_base) if stored else None, mask.ds_blocks,
                  N, nq, nkv, dh, 32, code, st)

    out = {}
    # attention_bwd: the step's path (dK/dV stores dS, dQ = dS K);
    # attention_bwd_recompute: the dQ pass that recomputes S, P and dP
    for name, fn, per_pair in (("attention_fwd", fwd, 4), ("attention_bwd", bwd, 8),
                               ("attention_bwd_recompute", lambda: bwd(False), 8)):
        for _ in range(warmup):
            fn()
        stream = torch.cuda.current_stream(device)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            fn()
        t1.record(stream)
        t1.synchronize()
        us = 1000.0 * t0.elapsed_time(t1) / steps
        flops = per_pair * dh * nq * mask.pairs
        out[name] = {"us_per_call": round(us, 1), "tflops": round(flops / us / 1e6, 1),
                     "frac": round(flops / (us / 1e6) / PEAK_BF16, 4)}
    print(json.dumps({"kernel": "attention", "workload": f"{spec['name']} layer shape: "
                      f"{len(spec['segments'])} x {spec['segments'][0]} tokens ({N} dual-stream "
                      f"rows), {nq}/{nkv} heads, head_dim 128", "pairs_per_head": mask.pairs,
                      "steps": steps, **out}), flush=True)


def run_gemm(spec, device, steps, warmup):
    """The bf16 GEMM alone on the products of one layer application of a step
    configuration (forward on the out-contiguous weight copies, dX on the
    weights, dW into the float32 gradient arena), each timed with HIP events
    over ``steps`` calls.  For kernel profiling; not a line of the benchmark's
    metric."""
    from alodlm_amd import _lib
    H, I = spec["hidden_size"], spec["intermediate_size"]
    nq, nkv, dh = spec["num_attention_heads"], spec["num_key_value_heads"], 128
    N = 2 * sum(spec["segments"])
    QW, QD = (nq + 2 * nkv) * dh, nq * dh
    E = (_lib.EPI_STORE, _lib.EPI_RESIDUAL, _lib.EPI_ACCUM)
    # name, M, N, K, A k-major, B k-major, epilogue
    shapes = [("qkv_fwd", N, QW, H, 1, 0, E[0]), ("o_fwd", N, H, QD, 1, 0, E[1]),
              ("gate_up_fwd", N, 2 * I, H, 1, 0, E[0]), ("down_fwd", N, H, I, 1, 0, E[1]),
              ("dx_gate_up", N, H, 2 * I, 1, 0, E[0]), ("dx_down", N, I, H, 1, 0, E[0]),
              ("dw_qkv", QW, H, N, 0, 0, E[2]), ("dw_o", H, QD, N, 0, 0, E[2]),
              ("dw_gate_up", 2 * I, H, N, 0, 0, E[2]), ("dw_down", H, I, N, 0, 0, E[2])]
    g = torch.Generator(device=device).manual_seed(7)
    st = _lib.stream_handle(device)
    stream = torch.cuda.current_stream(device)
    out = {}
    for name, M, Nn, K, ak, bk, epi in shapes:
        A = torch.randn(M * K, generator=g, device=device).to(torch.bfloat16)
        B = torch.randn(Nn * K, generator=g, device=device).to(torch.bfloat16)
        cdt = torch.float32 if epi == _lib.EPI_ACCUM else torch.bfloat16
        C = torch.zeros(M * Nn, dtype=cdt, device=device)
        R = torch.randn(M * Nn, generator=g, device=device).to(torch.bfloat16) \
            if epi == _lib.EPI_RESIDUAL else None
        need = _lib.query("alodlm_gemm_workspace", M, Nn, K, epi, _lib.BF16_CODE)
        ws = torch.empty(max(need, 1), dtype=torch.float32, device=device) if need else None
        lda, ldb = (K if ak else M), (K if bk else Nn)

        def call():
            _lib.call("alodlm_gemm", _lib.ptr(A), lda, ak, _lib.ptr(B), ldb, bk, _lib.ptr(C), Nn,
                      _lib.ptr(R), Nn, M, Nn, K, 1.0, epi, _lib.BF16_CODE, _lib.ptr(ws), st)

        for _ in range(warmup):
            call()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            call()
        t1.record(stream)
        t1.synchronize()
        us = 1000.0 * t0.elapsed_time(t1) / steps
        out[name] = {"mnk": [M, Nn, K], "us": round(us, 1),
                     "tflops": round(2.0 * M * Nn * K / us / 1e6, 1)}
        del A, B, C, R, ws
    print(json.dumps({"kernel": "gemm", "workload": f"{spec['name']} layer products "
                      f"({N} dual-stream rows)", "steps": steps, "products": out}), flush=True)


def cpu_baseline(spec, cfg_seg=2048, readout_rows=2048, layer_reps=3, threads=None):
    """Time the CPU oracle (float32, torch eager on this host) on a bounded
    sample: `layer_reps` decoder-layer fwd+bwd passes of the model's layer
    shape over one dual-stream segment and one LM-head readout fwd+bwd over
    `readout_rows` rows.  Returns (seconds per layer pass, seconds per readout
    row, threads)."""
    from oracle import step as O
    threads = threads or torch.get_num_threads()  # honours OMP_NUM_THREADS
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    H, I = spec["hidden_size"], spec["intermediate_size"]
    nq, nkv = spec["num_attention_heads"], spec["num_key_value_heads"]
    d = O.Dims(hidden=H, heads=nq, kv_heads=nkv, head_dim=128, intermediate=I,
               vocab=151936, layers=1, eps=1e-6, theta=1e6)
    pre = "model.layers.0."
    shapes = {"self_attn.q_proj.weight": (nq * 128, H), "self_attn.k_proj.weight": (nkv * 128, H),
              "self_attn.v_proj.weight": (nkv * 128, H), "self_attn.o_proj.weight": (H, nq * 128),
              "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    p = {pre + k: (torch.randn(*s, generator=g) * 0.02).requires_grad_(True) for k, s in shapes.items()}
    for k, n in (("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                 ("self_attn.q_norm.weight", 128), ("self_attn.k_norm.weight", 128)):
        p[pre + k] = torch.ones(n).requires_grad_(True)
    L = cfg_seg
    rows = 2 * L
    pos = torch.cat((torch.arange(L), torch.arange(L)))
    cos, sin = O.rope_tables(pos, 128, 1e6)
    allowed = torch.as_tensor(O.attention_mask(L, 32))
    x = torch.randn(rows, H, generator=g).requires_grad_(True)
    dy = torch.randn(rows, H, generator=g)
    t0 = time.perf_counter()
    for _ in range(layer_reps):
        y = O.layer_forward(p, pre, x, cos, sin, allowed, d)
        y.backward(dy)
    t_layer = (time.perf_counter() - t0) / layer_reps
    W = (torch.randn(151936, H, generator=g) * 0.02).requires_grad_(True)
    X = torch.randn(readout_rows, H, generator=g).requires_grad_(True)
    tgt = torch.randint(0, 151936, (readout_rows,), generator=g)
    t0 = time.perf_counter()
    loss = torch.nn.functional.cross_entropy(X @ W.T, tgt)
    loss.backward()
    t_readout = (time.perf_counter() - t0) / readout_rows
    return t_layer, t_readout, threads


def summarize_trace(directory, last_steps, out=sys.stdout):
    """Summarise a ``rocprofv3 --kernel-trace --output-format csv`` run of
    this benchmark: the last ``last_steps`` steps (a step ends with the
    optimizer's second AdamW launch, one per parameter group), each step's
    span, the time some kernel was running, the idle time between kernels and
    its largest gaps; then per-kernel time per step over those steps."""
    import csv
    import glob
    paths = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {directory}")
    with open(paths[0]) as f:
        rows = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                 r["Kernel_Name"].split("(")[0].strip().removeprefix("void "))
                for r in csv.DictReader(f)]
    rows.sort()
    adamw = sorted(e for s, e, n in rows if n.startswith("adamw_kernel"))
    ends = adamw[1::2]
    if len(ends) < last_steps + 1:
        raise SystemExit(f"the trace holds {len(ends)} steps, fewer than {last_steps + 1}")
    bounds = ends[-(last_steps + 1):]
    per_kernel, spans, busy_all, idle_all = {}, [], 0, 0
    print(f"steps summarised: {last_steps} (of {len(ends)} in the trace)", file=out)
    print("| step | span ms | kernels busy ms | idle ms | kernels | largest gaps (us, after -> before) |",
          file=out)
    print("|---|---|---|---|---|---|", file=out)
    for i, (a, b) in enumerate(zip(bounds, bounds[1:])):
        sel = [x for x in rows if x[0] >= a and x[1] <= b]
        busy, cur_s, cur_e, gaps, prev = 0, None, a, [], "step start"
        for s0, e0, n in sel:
            per_kernel.setdefault(n, [0, 0])
            per_kernel[n][0] += e0 - s0
            per_kernel[n][1] += 1
            if s0 > cur_e:
                gaps.append((s0 - cur_e, prev, n))
            if cur_s is None or s0 > cur_e:
                if cur_s is not None:
                    busy += cur_e - cur_s
                cur_s, cur_e = s0, e0
            else:
                cur_e = max(cur_e, e0)
            prev = n
        busy += (cur_e - cur_s) if cur_s is not None else 0
        span = b - a
        spans.append(span)
        busy_all += busy
        idle_all += span - busy
        top = "; ".join(f"{g / 1e3:.0f} ({p[:28]} -> {n[:28]})"
                        for g, p, n in sorted(gaps, reverse=True)[:3])
        print(f"| {i} | {span / 1e6:.1f} | {busy / 1e6:.1f} | {(span - busy) / 1e6:.1f} | "
              f"{len(sel)} | {top} |", file=out)
    n = last_steps
    print(f"\nmean per step: span {sum(spans) / n / 1e6:.1f} ms, kernels busy "
          f"{busy_all / n / 1e6:.1f} ms, idle {idle_all / n / 1e6:.1f} ms", file=out)
    print("\n| kernel | calls/step | ms/step | avg us |\n|---|---|---|---|", file=out)
    for name, (t, c) in sorted(per_kernel.items(), key=lambda kv: -kv[1][0])[:40]:
        print(f"| `{name[:70]}` | {c / n:g} | {t / n / 1e6:.1f} | {t / c / 1e3:.1f} |", file=out)


def summarize_counters(directories, out=sys.stdout, top=24):
    """Summarise ``rocprofv3 --pmc`` runs of this benchmark (one directory per
    counter pass): per kernel, its dispatches and each counter's mean per
    dispatch, then the derived columns the counters present allow:

    * MFMA util = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024): busy
      cycles are summed over the 1024 SIMDs, GRBM_GUI_ACTIVE over the 8 XCDs;
    * VALU / SALU / LDS instructions per MFMA instruction;
    * HBM MiB per dispatch = FETCH_SIZE and WRITE_SIZE (KiB), each scaled by
      what it reads for the 1 GiB device copy of ``--traffic-calibration``
      (the first dispatch of a kernel named like a copy: the fill that
      creates the copy's source comes before it and reads nothing), and the
      GEMMs' bytes per launch (`traffic_bytes_per_launch`)."""
    import csv
    import glob
    per, names = {}, {}
    for d in directories:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            disp = {}
            with open(path) as f:
                for r in csv.DictReader(f):
                    key = (path, int(r["Dispatch_Id"]))
                    name = r["Kernel_Name"].split("(")[0].strip().removeprefix("void ")
                    disp.setdefault(key, [name, {}])
                    c = disp[key][1]
                    c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            scale = {}
            copies = [c for _, (n, c) in sorted(disp.items()) if "copy" in n.lower()]
            for counter in ("FETCH_SIZE", "WRITE_SIZE"):
                if copies and copies[0].get(counter, 0) > 0:
                    scale[counter] = 1048576.0 / copies[0][counter]
            for key, (name, c) in disp.items():
                for counter, v in c.items():
                    acc = per.setdefault(name, {}).setdefault(counter, [0.0, 0])
                    acc[0] += v * scale.get(counter, 1.0)
                    acc[1] += 1
                names[name] = max(names.get(name, 0), sum(1 for k in disp if disp[k][0] == name))
    mean = {n: {k: v[0] / v[1] for k, v in cs.items()} for n, cs in per.items()}
    order = sorted(mean, key=lambda n: -(mean[n].get("SQ_BUSY_CYCLES", 0) * names[n] or
                                         (mean[n].get("FETCH_SIZE", 0) + mean[n].get("WRITE_SIZE", 0))
                                         * names[n]))
    cols = []
    have = lambda *ks: all(any(k in mean[n] for n in mean) for k in ks)
    if have("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"):
        cols.append(("MFMA util", lambda m: f"{100 * m['SQ_VALU_MFMA_BUSY_CYCLES'] / (m['GRBM_GUI_ACTIVE'] / 8 * 1024):.1f} %"))
    for k, label in (("SQ_INSTS_VALU", "VALU/MFMA"), ("SQ_INSTS_SALU", "SALU/MFMA"),
                     ("SQ_INSTS_LDS", "LDS/MFMA")):
        if have(k, "SQ_INSTS_MFMA"):
            cols.append((label, lambda m, k=k: f"{m[k] / m['SQ_INSTS_MFMA']:.2f}" if m["SQ_INSTS_MFMA"] else "-"))
    if have("SQ_LDS_BANK_CONFLICT"):
        cols.append(("LDS bank conflicts (M cycles/dispatch)", lambda m: f"{m['SQ_LDS_BANK_CONFLICT'] / 1e6:.2f}"))
    if have("FETCH_SIZE"):
        cols.append(("fetch MiB", lambda m: f"{m['FETCH_SIZE'] / 1024:.1f}"))
    if have("WRITE_SIZE"):
        cols.append(("write MiB", lambda m: f"{m['WRITE_SIZE'] / 1024:.1f}"))
    if have("FETCH_SIZE", "WRITE_SIZE"):
        # HBM bytes per GEMM launch, the reductions of split-K partials included
        # (the figure the bench line's roofline reports as `traffic`)
        gemm = [n for n in mean if n.startswith("gemm_")]
        red = [n for n in mean if n.startswith("splitk_")]
        calls = sum(names[n] for n in gemm)
        total = sum((mean[n].get("FETCH_SIZE", 0) + mean[n].get("WRITE_SIZE", 0)) * names[n]
                    for n in gemm + red) * 1024
        if calls:
            print(f"traffic_bytes_per_launch: {int(total / calls)}\n", file=out)
            print(f"GEMM calls: {calls}; HBM bytes per call (fetch + write, split-K "
                  f"reduction included): {total / calls / 1048576:.1f} MiB.\n", file=out)
    print("| kernel | dispatches | " + " | ".join(c for c, _ in cols) + " |", file=out)
    print("|---|---|" + "---|" * len(cols), file=out)
    for n in order[:top]:
        m = mean[n]
        cells = []
        for _, f in cols:
            try:
                cells.append(f(m))
            except (KeyError, ZeroDivisionError):
                cells.append("-")
        print(f"| `{n[:70]}` | {names[n]} | " + " | ".join(cells) + " |", file=out)


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--model", choices=sorted(MODELS), default="1.7b")
    parser.add_argument("--steps", type=int, default=5)
    # two warmup steps: the first optimizer step allocates the float32 masters
    # and moments, and the step after it is the first to run under the final
    # memory footprint (the caching allocator settles there once)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-kernel-timing", action="store_true")
    parser.add_argument("--no-sub-records", action="store_true",
                        help="time the headline step only")
    parser.add_argument("--traffic-calibration", action="store_true",
                        help="first run one plain 1 GiB device copy (read 1 GiB, write "
                             "1 GiB) so that HBM byte counters can be scaled against it")
    parser.add_argument("--kernel", choices=["attention", "gemm"],
                        help="time one kernel class alone at the --model layer shape "
                             "(for profiling) instead of the step")
    parser.add_argument("--summarize-trace", metavar="DIR",
                        help="print a summary of the rocprofv3 kernel trace under DIR (the "
                             "last --steps steps) and exit; needs no GPU")
    parser.add_argument("--summarize-counters", metavar="DIR", nargs="+",
                        help="print a per-kernel summary of rocprofv3 --pmc runs under the "
                             "DIRs (one per counter pass) and exit; needs no GPU")
    args = parser.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.steps)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.traffic_calibration:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    spec = MODELS[args.model]
    if args.kernel == "attention":
        run_attention(spec, device, args.steps, args.warmup)
        return
    if args.kernel == "gemm":
        run_gemm(spec, device, args.steps, args.warmup)
        return
    timing = not args.no_kernel_timing
    head, facts = run_step(spec, device, args.steps, args.warmup, timing)
    line = {
        "metric": "train tokens/s, ALoDLM-1.7B & 8B seq2048 on 1 MI355X; % bf16 MFMA peak",
        "value": head["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": head["workload"], "global_batch": head["global_batch"],
                   "seq_len": head["seq_len"], "dual_stream_rows": head["dual_stream_rows"],
                   "parallelism": "none (1 GPU)"},
        "device": device_info(),
        "memory": head["memory"], "mfu": head["mfu"], "step_tflop": head["step_tflop"],
        "step_ms": head["step_ms"], "allocator": head["allocator"],
    }
    if "roofline" in head:
        line["roofline"], line["kernel_classes"] = head["roofline"], head["kernel_classes"]
    if not args.no_cpu_baseline:
        t_layer, t_row, threads = cpu_baseline(spec)
        t_step = facts["apps"] * facts["segments"] * t_layer + facts["readout_rows"] * t_row
        line["cpu_baseline"] = {
            "value": round(facts["tokens"] / t_step, 4), "unit": "tokens/s", "cores": threads,
            "host_cpus": os.cpu_count(), "kind": "port", "extrapolated": True,
            "sample": (f"oracle fp32 eager on {threads} threads: {3} decoder-layer fwd+bwd "
                       f"passes on one 4096x{spec['hidden_size']} dual-stream segment "
                       f"({t_layer:.2f}s each) + LM head/CE fwd+bwd on 2048 rows x 151936 "
                       f"({1000 * t_row:.2f} ms/row); the step time is extrapolated from "
                       f"these to {facts['apps']} layer applications x {facts['segments']} "
                       f"segments + {facts['readout_rows']:.0f} readout rows"),
        }
    if not args.no_sub_records:
        subs = {}
        # the other step configuration at a handful of steps, then the stages
        other = "8b" if args.model == "1.7b" else "1.7b"
        rec, _ = run_step(MODELS[other], device, min(args.steps, 5), 2, timing)
        subs[f"{other.replace('.', 'p')}_step"] = rec
        subs["core_block"] = run_core_block(device, 10, 2, timing)
        subs["readout"] = run_readout(device, 10, 2, timing)
        line["sub_records"] = subs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
