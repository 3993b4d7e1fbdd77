"""Adaptive recurrent decoding on the training step's HIP kernels, with the
decoding state kept on the GPU (drop-in for alodlm/inference.py).

The decoding rules are the reference's (alodlm/inference.py:71-246): a window
of committed tokens followed by mask tokens runs through the prelude, the
recurrent core (up to ``max_depth`` passes) and the coda; after each pass the
mask rows commit by entropy (or left to right), the halting gate's survival
decides whether the window stops, and rows committed at a pass restart the
next pass from their token's embedding.  The committed run at the start of
the pending text is emitted and becomes cached prefix once a window has run
it as observed tokens.

How this implementation is organised:

* **State on the device.**  The pending text (a ledger of slots: token, open
  or committed, exit depth, first-pass halt probability), the output stream
  and each window's per-mask-row state are device arrays
  (``alodlm_decode_state``, csrc/decode.hip).  One kernel applies a depth's
  commitments and stop rule; at the depth where the window stops the same
  launch retires the window and plans the next one (ledger growth, the
  committed-first row order, positions and position penalties).  The host
  reads a 16-entry header once per executed depth and never touches token
  lists; the output stream is read once, at the end.
* **Cache written in place.**  Every cache key owns device buffers that grow
  by doubling.  A window's layers write its keys and values straight into the
  rows after the cached prefix.  Committed rows come first in a window and the
  run being retired is the first of them, so keeping it is a length increment,
  not a copy.
* **Layers on the step's kernels.**  Every layer application is a call of
  the module-level ``layer_forward`` (``alodlm_amd.model``, bound here as the
  reference binds it), which runs ``Kernels.layer_window``: RMSNorm, the
  GEMMs, q/k-norm + RoPE, attention, SwiGLU, with the window's keys and
  values written in place (``layers.WindowSlot``).  The window's mask (every cached key, causal inside the window;
  alodlm/inference.py:77-79) is the clean stream of one dual-stream segment
  (``WindowMask``).  The carry norm plus re-embedding is one ``carry_select``
  launch, the final norm and gate one ``final_norm_gate`` launch, and the
  readout's argmax and entropy one ``decode_readout`` launch.
"""

from dataclasses import dataclass
import ctypes
import time

import torch

from ._lib import call, ptr
from .layers import WindowMask, WindowSlot
from .model import layer_forward

# header fields (include/alodlm_hip.h, ALODLM_DECODE_*)
HEADER = 16
LEDGER, GENERATED, CACHE, DONE, REASON, WINDOW, OBSERVED, PREFIX, STOP = range(9)
REASON_EOS = 1
MODES = {"entropy": 0, "left1": 1}
# special tokens that end generation besides the tokenizer's EOS
# (alodlm/inference.py:161-163)
STOP_TOKENS = ("<|im_end|>", "<|endoftext|>", "<|eot_id|>", "</s>")


@dataclass
class DecodeConfig:
    """Decoding settings; fields, defaults and validation as
    alodlm/inference.py:14-31."""
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

    @property
    def penalty(self):
        """Entropy penalty per position after the first mask slot (the
        default is tau / 20, alodlm/inference.py:100)."""
        return self.tau * 0.05 if self.position_penalty is None else self.position_penalty


def stop_token_ids(tokenizer):
    """Token ids that end generation: the tokenizer's EOS id(s) plus the chat
    end markers it knows (alodlm/inference.py:158-163)."""
    eos = tokenizer.eos_token_id
    ids = {t for t in (eos if isinstance(eos, (list, tuple)) else [eos]) if t is not None}
    vocab = tokenizer.get_vocab()
    ids.update(tokenizer.convert_tokens_to_ids(t) for t in STOP_TOKENS if t in vocab)
    return sorted(ids)


class PrefixCache:
    """Cached keys/values of the committed prefix, one entry per cache key:
    recurrent layers have one key per depth, the other layers share depth 0
    (the interface of alodlm/inference.py:34-63).

    Each key owns two device buffers [capacity, kv_heads, head_dim].  Rows
    [0, length) hold the prefix; a window writes its rows right after it, so
    keeping the first rows of a window is ``retire``.
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
        """key -> (k, v) of the cached prefix, [length, kv_heads, head_dim]."""
        return {key: (k[:self.length], v[:self.length]) for key, (k, v) in self._buffers.items()}

    def _bind(self, kv_heads, head_dim, dtype, device):
        spec = (kv_heads, head_dim, dtype, device)
        if self._spec is None:
            self._spec = spec
        elif self._spec != spec:
            raise ValueError("PrefixCache used with a different model")

    def reserve(self, rows):
        """Room for ``rows`` rows in every buffer (capacity doubles; the prefix
        moves with it)."""
        if rows <= self._capacity:
            return
        capacity = max(rows, 2 * self._capacity, 64)
        for key, pair in self._buffers.items():
            self._buffers[key] = tuple(self._moved(t, capacity) for t in pair)
        self._capacity = capacity

    def _moved(self, t, capacity):
        kv_heads, head_dim, dtype, device = self._spec
        out = torch.empty(capacity, kv_heads, head_dim, dtype=dtype, device=device)
        out[:self.length].copy_(t[:self.length])
        return out

    def buffers(self, key):
        """The (k, v) buffers of a key, allocated on first use."""
        pair = self._buffers.get(key)
        if pair is None:
            kv_heads, head_dim, dtype, device = self._spec
            shape = (max(self._capacity, 1), kv_heads, head_dim)
            pair = self._buffers[key] = (torch.empty(shape, dtype=dtype, device=device),
                                         torch.empty(shape, dtype=dtype, device=device))
        return pair

    def rows(self, key, start, count):
        k, v = self.buffers(key)
        return k[start:start + count], v[start:start + count]

    def fill_depths(self, executed, start, count):
        """Rows [start, start + count) of the recurrent depths a window did not
        run take the keys/values of its last executed depth
        (alodlm/inference.py:45-51)."""
        c = self.config
        if count == 0:
            return
        for layer in range(c.loop_start, c.loop_end):
            src_k, src_v = self.rows((layer, executed - 1), start, count)
            for depth in range(executed, c.max_depth):
                k, v = self.rows((layer, depth), start, count)
                k.copy_(src_k)
                v.copy_(src_v)

    def retire(self, count):
        """Keep the ``count`` rows written after the prefix."""
        self.length += count

    def complete(self, window, completed):
        """``window`` (key -> its rows) gains the unexecuted recurrent depths,
        filled from the last executed one."""
        c = self.config
        for layer in range(c.loop_start, c.loop_end):
            last_k, last_v = window[layer, completed - 1]
            for depth in range(completed, c.max_depth):
                k, v = self.rows((layer, depth), self.length, last_k.shape[0])
                k.copy_(last_k)
                v.copy_(last_v)
                window[layer, depth] = (k, v)

    def append(self, window, rows):
        """Add the window rows ``rows`` (indices into the window, in that order)
        to every key's prefix."""
        n = rows.numel()
        if n == 0:
            return
        self.reserve(self.length + n)
        in_place = bool(torch.equal(rows.cpu(), torch.arange(n)))
        for key, (wk, wv) in window.items():
            k, v = self.buffers(key)
            if in_place and wk.data_ptr() == k[self.length].data_ptr() \
                    and wv.data_ptr() == v[self.length].data_ptr():
                continue
            picked_k, picked_v = wk[rows].clone(), wv[rows].clone()
            k[self.length:self.length + n].copy_(picked_k)
            v[self.length:self.length + n].copy_(picked_v)
        self.length += n


class DecodeState(ctypes.Structure):
    """ctypes mirror of alodlm_decode_state (include/alodlm_hip.h)."""
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "slot_token", "slot_open", "slot_depth", "slot_halt",
        "out_token", "out_depth", "out_halt",
        "row_token", "row_position", "mask_row", "mask_slot", "mask_offset",
        "mask_token", "mask_exit", "mask_committed", "mask_fresh",
        "mask_survival", "mask_first_hazard", "predicted", "entropy",
        "replace_token", "replace_depth", "header", "stop_ids")] + [
        ("n_stop", ctypes.c_int64), ("capacity", ctypes.c_int64),
        ("max_new_tokens", ctypes.c_int64), ("window_size", ctypes.c_int64),
        ("mask_token_id", ctypes.c_int64), ("max_depth", ctypes.c_int64),
        ("tau", ctypes.c_float), ("q", ctypes.c_float), ("penalty", ctypes.c_float),
        ("mode", ctypes.c_int32)]


class _DeviceState:
    """The device arrays behind one DecodeState: windows of up to ``capacity``
    rows, a ledger of ``capacity`` slots, an output stream of
    ``max_new_tokens``."""

    _LAYOUT = {  # name -> dtype; every array has `capacity` entries
        "slot_token": torch.int64, "slot_open": torch.int32, "slot_depth": torch.int32,
        "slot_halt": torch.float32, "row_token": torch.int64, "row_position": torch.int64,
        "mask_row": torch.int32, "mask_slot": torch.int32, "mask_offset": torch.float32,
        "mask_token": torch.int64, "mask_exit": torch.int32, "mask_committed": torch.int32,
        "mask_fresh": torch.int32, "mask_survival": torch.float32,
        "mask_first_hazard": torch.float32, "predicted": torch.int64, "entropy": torch.float32,
        "replace_token": torch.int64, "replace_depth": torch.int32,
    }

    def __init__(self, device, capacity, config, max_depth, mask_token_id, stop_ids):
        self.device = device
        self.t = {name: torch.zeros(capacity, dtype=dtype, device=device)
                  for name, dtype in self._LAYOUT.items()}
        n_out = max(config.max_new_tokens, 1)
        self.t["out_token"] = torch.zeros(n_out, dtype=torch.int64, device=device)
        self.t["out_depth"] = torch.zeros(n_out, dtype=torch.int32, device=device)
        self.t["out_halt"] = torch.zeros(n_out, dtype=torch.float32, device=device)
        self.t["header"] = torch.zeros(HEADER, dtype=torch.int64, device=device)
        self.t["stop_ids"] = torch.tensor(list(stop_ids) or [0], dtype=torch.int64, device=device)
        self._host = torch.zeros(HEADER, dtype=torch.int64).pin_memory()
        s = self.struct = DecodeState()
        for name, _ in DecodeState._fields_[:24]:
            setattr(s, name, self.t[name].data_ptr())
        s.n_stop = len(stop_ids)
        s.capacity = capacity
        s.max_new_tokens = config.max_new_tokens
        s.window_size = config.window_size
        s.mask_token_id = mask_token_id
        s.max_depth = max_depth
        s.tau, s.q, s.penalty = config.tau, config.q, config.penalty
        s.mode = MODES[config.mode]

    def __getitem__(self, name):
        return self.t[name]

    @property
    def ref(self):
        return ctypes.byref(self.struct)

    def read_header(self):
        """The header as a list of ints (waits for the queued work)."""
        self._host.copy_(self.t["header"], non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return self._host.tolist()

    def start(self, cache_rows, stream):
        """Empty ledger and output after a prefill of ``cache_rows`` rows; the
        first window is planned."""
        h = torch.zeros(HEADER, dtype=torch.int64)
        h[CACHE] = cache_rows
        self.t["header"].copy_(h)
        call("alodlm_decode_plan", self.ref, stream)


def rope_tables(positions, inv_freq, dtype):
    """cos/sin [rows, head_dim] of the rotary embedding at ``positions``, the
    computation of [tf] modeling_qwen3.py:126-137 (float32 angles
    position x inverse frequency, duplicated halves, rounded to ``dtype``)."""
    freqs = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class Decoder:
    """Adaptive recurrent decoding (alodlm/inference.py:66-246) with the step's
    HIP kernels and device-side window state."""

    def __init__(self, model, tokenizer):
        self.model = model.eval()
        self.tokenizer = tokenizer
        self._weights_ready = None
        self.cache = None  # the prefix cache of the last generation

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

    def _state(self, capacity, config):
        return _DeviceState(self._engine().device, capacity, config, self.model.config.max_depth,
                            self.model.config.mask_token_id, stop_token_ids(self.tokenizer))

    def _run(self, cache, ids, positions, rows, count, state, finish, window=None):
        """The passes of one window of ``rows`` rows (token ids ``ids``, rotary
        positions ``positions``, device int64) whose ``count`` mask rows are
        state's mask_row entries.  Keys/values land in the cache rows after
        its prefix (and in ``window``, key -> rows, when given).  Returns the
        number of executed depths and the last header read (None without mask
        rows)."""
        e = self._engine()
        d, c = e.dims, self.model.config
        st, code = e._stream(), e.code
        K = c.max_depth
        P = cache.length
        cache._bind(d.kv_heads, d.head_dim, e.dtype, e.device)
        cache.reserve(P + rows)
        tiled = e.dtype == torch.bfloat16 and d.head_dim in (64, 128)
        lay = WindowMask(P, rows, tiled, e.device, block_size=c.block_size)
        cos, sin = rope_tables(positions, e.inv_freq, e.dtype)
        H, V = d.hidden, d.vocab
        modules = self.model.backbone.model.layers

        def layer(index, h, depth):
            # every layer application goes through the module-level
            # layer_forward, as alodlm/inference.py:83-88 does; the slot lets
            # it write the window's keys/values after the cached rows
            key = cache.key(index, depth)
            kbuf, vbuf = cache.buffers(key)
            slot = WindowSlot(e, e.layers[index], kbuf, vbuf, lay)
            h, kv = layer_forward(modules[index], h, cos, sin, lay, slot)
            if window is not None:
                window[key] = kv
            return h

        hidden = e._empty(rows, H)
        call("alodlm_embed_gather", ptr(e.embed), ptr(ids), ptr(hidden), rows, H, V, code, st)
        for index in range(c.loop_start):
            hidden = layer(index, hidden, 0)
        gate = e._empty(rows, dtype=torch.float32)
        rstd = e._empty(rows, dtype=torch.float32)
        header = None
        for depth in range(K):
            if depth:
                # carry norm of the previous pass; rows committed there start
                # from their token's embedding (alodlm/inference.py:101-105,145)
                carried = e._empty(rows, H)
                call("alodlm_carry_select", ptr(core_out), ptr(e.final_norm), ptr(e.embed),
                     ptr(state["replace_token"]), ptr(state["replace_depth"]), depth,
                     ptr(carried), ptr(rstd), rows, H, V, d.eps, code, st)
                hidden = carried
            for index in range(c.loop_start, c.loop_end):
                hidden = layer(index, hidden, depth)
            core_out = readout = hidden
            for index in range(c.loop_end, d.layers):
                readout = layer(index, readout, depth)
            features = e._empty(rows, H)
            call("alodlm_final_norm_gate", ptr(readout), ptr(e.final_norm), ptr(e.gate_w),
                 ptr(e.gate_b), ptr(e.depth_bias), depth, ptr(features), ptr(rstd), ptr(gate),
                 rows, H, d.eps, code, st)
            if count:
                picked = e._empty(count, H)
                call("alodlm_gather_rows", ptr(features), ptr(state["mask_row"]), count,
                     ptr(picked), H, code, st)
                logits = e._empty(count, V)
                e._gemm(picked, H, 1, e.lm_head, H, 1, logits, V, count, V, H)
                call("alodlm_decode_readout", ptr(logits), count, V, ptr(state["predicted"]),
                     ptr(state["entropy"]), code, st)
                call("alodlm_decode_commit", state.ref, ptr(gate), count, depth, int(finish), st)
                header = state.read_header()
                stop = bool(header[STOP])
            else:
                stop = depth == K - 1
            if stop:
                return depth + 1, header
        raise RuntimeError("Recurrent decoding did not terminate")

    @torch.inference_mode()
    def _window(self, ids, positions, cache, mask_rows, config, logical_mask_positions):
        """One window with caller-given rows (the signature of
        alodlm/inference.py:71): returns ``(window, committed, tokens,
        exit_depths, executed_depths, first_hazard)``, ``window`` mapping each
        cache key to the window's (k, v) rows."""
        e = self._engine()
        dev = e.device
        ids = ids.to(device=dev, dtype=torch.int64)
        positions = positions.to(device=dev, dtype=torch.int64)
        rows, count = ids.numel(), mask_rows.numel()
        state = self._state(max(rows, 1), config)
        if count:
            state["mask_row"][:count].copy_(mask_rows.to(dev, torch.int32))
        logical = logical_mask_positions.to(device=dev, dtype=torch.int64)
        call("alodlm_decode_begin", state.ref, ptr(logical) if count else None, rows, count,
             e._stream())
        window = {}
        executed, _ = self._run(cache, ids, positions, rows, count, state, False, window)
        cache.complete(window, executed)
        return (window, state["mask_committed"][:count].bool(), state["mask_token"][:count].clone(),
                state["mask_exit"][:count].long(), executed,
                state["mask_first_hazard"][:count].clone())

    @torch.inference_mode()
    def generate(self, prompt_ids, config=None):
        """Generate after ``prompt_ids``; the result dictionary of
        alodlm/inference.py:148-246."""
        config = config or DecodeConfig()
        config.validate()
        model = self.model
        device = next(model.parameters()).device
        if device.type != "cuda":
            raise ValueError("the HIP decoder needs the model on a CUDA (ROCm) device")
        prompt = torch.tensor(prompt_ids, dtype=torch.long, device=device)
        if not len(prompt):
            raise ValueError("Prompt must contain at least one token")
        if len(prompt) + config.max_new_tokens > model.backbone.config.max_position_embeddings:
            raise ValueError("Prompt and generation budget exceed the model context")
        if bool(((prompt < 0) | (prompt >= model.backbone.config.vocab_size)).any()):
            raise ValueError("Prompt token is outside the model vocabulary")
        e = self._engine()
        torch.cuda.synchronize(device)
        started = time.perf_counter()
        n = len(prompt)
        state = self._state(max(2 * config.window_size, n), config)
        self.cache = cache = PrefixCache(model.config)
        # the prompt: one window of observed rows, every depth, all rows kept
        call("alodlm_decode_begin", state.ref, None, n, 0, e._stream())
        executed, _ = self._run(cache, prompt, torch.arange(n, device=device), n, 0, state, False)
        cache.fill_depths(executed, 0, n)
        cache.retire(n)
        state.start(cache.length, e._stream())
        header = state.read_header()
        prefill_seconds = time.perf_counter() - started
        steps = passes = loop_token_passes = 0
        while not header[DONE]:
            rows, observed = header[WINDOW], header[OBSERVED]
            P = cache.length
            executed, header = self._run(cache, state["row_token"][:rows],
                                         state["row_position"][:rows], rows, rows - observed,
                                         state, True)
            steps += 1
            passes += executed
            loop_token_passes += rows * executed
            kept = header[CACHE] - P
            cache.fill_depths(executed, P, kept)
            cache.retire(kept)
        count = header[GENERATED]
        token_ids = state["out_token"][:count].tolist()
        depths = state["out_depth"][:count].tolist()
        hazards = state["out_halt"][:count].tolist()
        elapsed = time.perf_counter() - started
        return {
            "text": self.tokenizer.decode(token_ids, skip_special_tokens=True),
            "token_ids": token_ids, "prompt_tokens": n, "generated_tokens": count,
            "wall_seconds": elapsed, "prefill_seconds": prefill_seconds,
            "tokens_per_second": count / elapsed,
            "mean_exit_depth": sum(depths) / count if count else None,
            "loop_token_passes": loop_token_passes,
            "loop_token_passes_per_output_token": loop_token_passes / count if count else None,
            "outer_steps": steps, "recurrent_passes": passes, "exit_depths": depths,
            "first_pass_halt_probabilities": hazards,
            "stop_reason": "eos" if header[REASON] == REASON_EOS else "length",
        }
