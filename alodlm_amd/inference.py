"""Cached adaptive decoding on the training step's HIP kernels (drop-in for
alodlm/inference.py).

``Decoder(model, tokenizer).generate(prompt_ids, DecodeConfig(...))`` follows
alodlm/inference.py:66-246: windows of committed tokens and mask tokens run
through the prelude, the recurrent core (up to ``max_depth`` passes) and the
coda; after each pass the mask rows commit by entropy (or left to right), the
halting gate's survival decides whether to stop, and newly committed rows are
re-embedded for the next pass.  Committed prefix K/V are cached per (layer,
depth) for the recurrent layers and per layer elsewhere.

What runs where:

* every layer application uses the step's kernels (RMSNorm, the GEMMs on
  out-contiguous weight copies, q/k-norm + RoPE, attention, SwiGLU);
* the window's mask - every cached prefix key plus causal attention inside
  the window (alodlm/inference.py:77-79) - is the clean stream of one
  dual-stream segment of length P + W (P cached rows, W window rows): a
  clean row sees every earlier row.  The attention kernels therefore run
  unchanged on a synthetic layout: the segment starts ``base`` rows before
  the first query buffer row, and the key/value pointers are offset by
  ``base`` rows so that segment row r is cache row r;
* the carry norm between passes and the re-embedding of newly committed rows
  are one ``carry_select`` launch, the final norm and gate one
  ``final_norm_gate`` launch, and the readout's argmax and entropy one
  ``decode_readout`` launch over the LM-head logits of the mask rows;
* the commit rules are the reference's tensor operations on the mask rows.

K/V caches are preallocated device buffers that grow by doubling, so
appending the committed rows copies only those rows.
"""

from dataclasses import dataclass
import time

import torch

from . import _lib
from ._lib import call, ptr, query
from .layers import Rope, WindowMask


@dataclass
class DecodeConfig:
    """Decoding settings (alodlm/inference.py:14-31)."""
    q: float = 0.5
    tau: float = 0.4
    window_size: int = 16
    max_new_tokens: int = 4096
    position_penalty: float | None = None
    mode: str = "entropy"

    def validate(self):
        if not 0 <= self.q <= 1 or not 0 <= self.tau < float("inf"):
            raise ValueError("q must be in [0,1] and tau must be finite and nonnegative")
        if min(self.window_size, self.max_new_tokens) < 1:
            raise ValueError("Window size and generation budget must be positive")
        if self.mode not in ("entropy", "left1"):
            raise ValueError("mode must be entropy or left1")
        if self.position_penalty is not None and not 0 <= self.position_penalty < float("inf"):
            raise ValueError("position_penalty must be finite and nonnegative")


class PrefixCache:
    """Committed-prefix K/V per cache key (alodlm/inference.py:34-63).

    Recurrent layers have one key per depth, the others share depth 0.  Each
    key owns two device buffers [capacity, kv_heads, head_dim]; rows
    [0, length) hold the prefix and a window writes its rows right after it.
    """

    def __init__(self, config):
        self.config = config
        self.length = 0
        self._buffers = {}
        self._spec = None  # (kv_heads, head_dim, dtype, device)
        self._capacity = 0

    def key(self, layer, depth):
        c = self.config
        return layer, depth if c.loop_start <= layer < c.loop_end else 0

    @property
    def values(self):
        """key -> (k, v) views of the cached prefix, shape [length, kv_heads, head_dim]."""
        return {key: (k[:self.length], v[:self.length]) for key, (k, v) in self._buffers.items()}

    def _bind(self, kv_heads, head_dim, dtype, device):
        spec = (kv_heads, head_dim, dtype, device)
        if self._spec is None:
            self._spec = spec
        elif self._spec != spec:
            raise ValueError("PrefixCache used with a different model")

    def reserve(self, rows):
        """Make room for ``rows`` rows in every buffer (doubling, prefix kept)."""
        if rows <= self._capacity:
            return
        capacity = max(rows, 2 * self._capacity, 64)
        for key, (k, v) in self._buffers.items():
            self._buffers[key] = (self._grow(k, capacity), self._grow(v, capacity))
        self._capacity = capacity

    def _grow(self, t, capacity):
        kv_heads, head_dim, dtype, device = self._spec
        out = torch.empty(capacity, kv_heads, head_dim, dtype=dtype, device=device)
        out[:self.length].copy_(t[:self.length])
        return out

    def buffers(self, key):
        """The (k, v) buffers of a key, allocated on first use."""
        bufs = self._buffers.get(key)
        if bufs is None:
            kv_heads, head_dim, dtype, device = self._spec
            shape = (max(self._capacity, 1), kv_heads, head_dim)
            bufs = self._buffers[key] = (torch.empty(shape, dtype=dtype, device=device),
                                         torch.empty(shape, dtype=dtype, device=device))
        return bufs

    def rows(self, key, start, count):
        k, v = self.buffers(key)
        return k[start:start + count], v[start:start + count]

    def complete(self, window, completed):
        """Recurrent depths the window did not execute take the K/V of the last
        executed depth (alodlm/inference.py:45-51)."""
        c = self.config
        for layer in range(c.loop_start, c.loop_end):
            last_k, last_v = window[layer, completed - 1]
            for depth in range(completed, c.max_depth):
                key = (layer, depth)
                k, v = self.rows(key, self.length, last_k.shape[0])
                k.copy_(last_k)
                v.copy_(last_v)
                window[key] = (k, v)

    def append(self, window, rows):
        """Append the window rows ``rows`` (in that order) to every key's prefix
        (alodlm/inference.py:53-63)."""
        if rows.numel() == 0:
            return
        n = rows.numel()
        for key, (wk, wv) in window.items():
            k, v = self.buffers(key)
            sel_k, sel_v = wk[rows].clone(), wv[rows].clone()
            k[self.length:self.length + n].copy_(sel_k)
            v[self.length:self.length + n].copy_(sel_v)
        self.length += n


class Decoder:
    """Adaptive recurrent decoding (alodlm/inference.py:66-246) on the HIP kernels."""

    def __init__(self, model, tokenizer):
        self.model = model.eval()
        self.tokenizer = tokenizer
        self._weights_ready = None

    # ------------------------------------------------------------------ kernels
    def _engine(self):
        e = self.model.engine()
        if self._weights_ready is not e:
            # out-contiguous weight copies for the products (refreshed from the
            # parameters once per decoder and engine)
            e.transposed.refresh(e.code, e._stream())
            self._weights_ready = e
        return e

    def refresh_weights(self):
        """Call after changing the model's parameters between generations."""
        self._weights_ready = None

    def _layer(self, e, li, x, positions, cache, key, lay):
        """One decoder layer over the window rows (alodlm/model.py:49-76), with
        the prefix K/V of ``key``; the window's K/V land in the cache rows
        [P, P + W) of that key."""
        kbuf, vbuf = cache.buffers(key)
        return e.layer_window(e.layers[li], x, Rope(positions=positions, inv_freq=e.inv_freq),
                              lay, kbuf, vbuf)

    def _window(self, ids, positions, cache, mask_rows, config, logical_mask_positions):
        """Run one window (alodlm/inference.py:71-146).

        Returns ``(window, committed, tokens, exit_depths, executed_depths,
        first_hazard)`` like the reference; ``window`` maps cache keys to the
        window's (k, v) rows.
        """
        e = self._engine()
        d, c = e.dims, self.model.config
        st, code, dev = e._stream(), e.code, e.device
        K = c.max_depth
        ids = ids.to(device=dev, dtype=torch.int64)
        positions = positions.to(device=dev, dtype=torch.int64)
        mask_rows = mask_rows.to(device=dev, dtype=torch.int64)
        logical_mask_positions = logical_mask_positions.to(dev)
        length = ids.numel()
        P = cache.length
        cache._bind(d.kv_heads, d.head_dim, e.dtype, dev)
        cache.reserve(P + length)
        tiled = e.dtype == torch.bfloat16 and d.head_dim in (64, 128)
        lay = WindowMask(P, length, tiled, dev, block_size=c.block_size)
        H, V = d.hidden, d.vocab
        window = {}

        def run(layer, h, depth):
            key = cache.key(layer, depth)
            h = self._layer(e, layer, h, positions, cache, key, lay)
            window[key] = cache.rows(key, P, length)
            return h

        hidden = e._empty(length, H)
        call("alodlm_embed_gather", ptr(e.embed), ptr(ids), ptr(hidden), length, H, V, code, st)
        for layer in range(c.loop_start):
            hidden = run(layer, hidden, 0)
        count = mask_rows.numel()
        committed = torch.zeros(count, dtype=torch.bool, device=dev)
        newly_committed = committed.clone()
        tokens = torch.zeros(count, dtype=torch.long, device=dev)
        exit_depths = torch.zeros(count, dtype=torch.long, device=dev)
        survival = torch.ones(count, device=dev)
        first_hazard = torch.empty(count, device=dev)
        penalty = config.position_penalty if config.position_penalty is not None else config.tau * 0.05
        relative = (logical_mask_positions - logical_mask_positions[:1] if count
                    else logical_mask_positions)
        sel_rows = mask_rows.to(torch.int32)
        replace_ids = torch.zeros(length, dtype=torch.int64, device=dev)
        replace_at = torch.empty(length, dtype=torch.int32, device=dev)
        gate = torch.empty(length, dtype=torch.float32, device=dev)
        rstd = torch.empty(length, dtype=torch.float32, device=dev)
        core_out = None
        for depth in range(K):
            if depth:
                # the carry norm of the previous pass; newly committed mask rows
                # start this pass from their token's embedding instead
                # (alodlm/inference.py:101-105,145)
                replace_at.fill_(K)
                if count:
                    replace_ids[mask_rows] = tokens
                    replace_at[mask_rows[newly_committed]] = depth
                hidden = e._empty(length, H)
                call("alodlm_carry_select", ptr(core_out), ptr(e.final_norm), ptr(e.embed),
                     ptr(replace_ids), ptr(replace_at), depth, ptr(hidden), ptr(rstd), length, H,
                     V, d.eps, code, st)
            for layer in range(c.loop_start, c.loop_end):
                hidden = run(layer, hidden, depth)
            core_out = hidden
            readout = hidden
            for layer in range(c.loop_end, d.layers):
                readout = run(layer, readout, depth)
            features = e._empty(length, H)
            call("alodlm_final_norm_gate", ptr(readout), ptr(e.final_norm), ptr(e.gate_w),
                 ptr(e.gate_b), ptr(e.depth_bias), depth, ptr(features), ptr(rstd), ptr(gate),
                 length, H, d.eps, code, st)
            stop = depth == K - 1
            if count:
                selected = e._empty(count, H)
                call("alodlm_gather_rows", ptr(features), ptr(sel_rows), count, ptr(selected), H,
                     code, st)
                logits = e._empty(count, V)
                e._gemm(selected, H, 1, e.lm_head_t, V, 0, logits, V, count, V, H)
                predicted = torch.empty(count, dtype=torch.int64, device=dev)
                entropy = torch.empty(count, dtype=torch.float32, device=dev)
                call("alodlm_decode_readout", ptr(logits), count, V, ptr(predicted), ptr(entropy),
                     code, st)
                hazard = gate[mask_rows].sigmoid()
                if depth == 0:
                    first_hazard = hazard.clone()
                survival *= 1 - hazard
                adjusted = entropy + relative * penalty
                if config.mode == "left1":
                    agree = torch.zeros_like(committed)
                    remaining = (~committed).nonzero().flatten()
                    if len(remaining):
                        agree[remaining[0]] = True
                else:
                    agree = (adjusted < config.tau) & ~committed
                tokens = torch.where(agree, predicted, tokens)
                exit_depths = torch.where(agree, depth + 1, exit_depths)
                committed |= agree
                newly_committed = agree
                residual = ~committed
                stop |= not bool(residual.any()) or bool((1 - survival)[residual].mean() >= config.q)
                if stop and not bool(committed.any()):
                    index = adjusted.argmin()
                    tokens[index] = predicted[index]
                    exit_depths[index] = depth + 1
                    committed[index] = True
            if stop:
                cache.complete(window, depth + 1)
                return window, committed, tokens, exit_depths, depth + 1, first_hazard
        raise RuntimeError("Recurrent decoding did not terminate")

    @torch.inference_mode()
    def generate(self, prompt_ids, config=None):
        """Generate after ``prompt_ids`` (alodlm/inference.py:148-246); returns
        the reference's result dictionary."""
        config = config or DecodeConfig()
        config.validate()
        model = self.model
        device = next(model.parameters()).device
        if device.type != "cuda":
            raise ValueError("the HIP decoder needs the model on a CUDA (ROCm) device")
        prompt = torch.tensor(prompt_ids, dtype=torch.long, device=device)
        if not len(prompt):
            raise ValueError("Prompt must contain at least one token")
        context = model.backbone.config.max_position_embeddings
        if len(prompt) + config.max_new_tokens > context:
            raise ValueError("Prompt and generation budget exceed the model context")
        if bool(((prompt < 0) | (prompt >= model.backbone.config.vocab_size)).any()):
            raise ValueError("Prompt token is outside the model vocabulary")
        eos = self.tokenizer.eos_token_id
        stop_ids = set(eos if isinstance(eos, list) else [eos]) - {None}
        vocab = self.tokenizer.get_vocab()
        for token in ("<|im_end|>", "<|endoftext|>", "<|eot_id|>", "</s>"):
            if token in vocab:
                stop_ids.add(self.tokenizer.convert_tokens_to_ids(token))
        mask_id = model.config.mask_token_id
        torch.cuda.synchronize(device)
        started = time.perf_counter()
        cache = PrefixCache(model.config)
        empty = torch.empty(0, dtype=torch.long, device=device)
        prefill = self._window(prompt, torch.arange(len(prompt), device=device), cache, empty,
                               config, empty)[0]
        cache.append(prefill, torch.arange(len(prompt), device=device))
        torch.cuda.synchronize(device)
        prefill_seconds = time.perf_counter() - started
        generated, depths, hazards = [], [], []
        tokens, flags, window_depths, window_hazards = [], [], [], []
        steps = passes = loop_token_passes = 0
        stop_reason = "length"
        while len(generated) < config.max_new_tokens:
            # the committed run at the window's start becomes prefix (observed
            # tokens); newly predicted mask rows are not prefix keys
            prefix = next((i for i, masked in enumerate(flags) if masked), len(flags))
            finished = (len(generated) + prefix >= config.max_new_tokens
                        or any(t in stop_ids for t in tokens[:prefix]))
            if finished:
                for i in range(prefix):
                    if tokens[i] in stop_ids:
                        stop_reason = "eos"
                        break
                    generated.append(tokens[i])
                    depths.append(window_depths[i])
                    hazards.append(window_hazards[i])
                break
            desired = min(config.window_size, config.max_new_tokens - len(generated) - prefix)
            grow = max(0, prefix + desired - len(tokens))
            tokens.extend([mask_id] * grow)
            flags.extend([True] * grow)
            window_depths.extend([0] * grow)
            window_hazards.extend([0.0] * grow)
            observed = [i for i, masked in enumerate(flags) if not masked]
            masked = [i for i, is_mask in enumerate(flags) if is_mask]
            order = observed + masked
            order_tensor = torch.tensor(order, device=device)
            ids = torch.tensor([tokens[i] for i in order], dtype=torch.long, device=device)
            positions = cache.length + order_tensor
            mask_rows = torch.arange(len(observed), len(order), device=device)
            window, agreed, predicted, committed_depth, executed, halt = self._window(
                ids, positions, cache, mask_rows, config, torch.tensor(masked, device=device))
            steps += 1
            passes += executed
            loop_token_passes += len(order) * executed
            inverse = torch.argsort(order_tensor)
            cache.append(window, inverse[:prefix])
            generated.extend(tokens[:prefix])
            depths.extend(window_depths[:prefix])
            hazards.extend(window_hazards[:prefix])
            agreed, predicted = agreed.tolist(), predicted.tolist()
            committed_depth, halt = committed_depth.tolist(), halt.tolist()
            for j, original in enumerate(masked):
                if agreed[j]:
                    tokens[original] = int(predicted[j])
                    flags[original] = False
                    window_depths[original] = int(committed_depth[j])
                    window_hazards[original] = float(halt[j])
            tokens, flags = tokens[prefix:], flags[prefix:]
            window_depths, window_hazards = window_depths[prefix:], window_hazards[prefix:]
        torch.cuda.synchronize(device)
        elapsed = time.perf_counter() - started
        count = len(generated)
        return {
            "text": self.tokenizer.decode(generated, skip_special_tokens=True),
            "token_ids": generated, "prompt_tokens": len(prompt), "generated_tokens": count,
            "wall_seconds": elapsed, "prefill_seconds": prefill_seconds,
            "tokens_per_second": count / elapsed,
            "mean_exit_depth": sum(depths) / count if count else None,
            "loop_token_passes": loop_token_passes,
            "loop_token_passes_per_output_token": loop_token_passes / count if count else None,
            "outer_steps": steps, "recurrent_passes": passes, "exit_depths": depths,
            "first_pass_halt_probabilities": hazards, "stop_reason": stop_reason,
        }
