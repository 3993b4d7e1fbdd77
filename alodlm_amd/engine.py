"""The fused ALoDLM training step on the HIP kernels.

``StepEngine`` owns the parameter arena of one ``ALoDLM`` module and runs the
whole step of alodlm/model.py:130-187 as an explicit schedule of kernel
launches on the current stream:

forward   weight transposes -> embed -> prelude -> for each depth: (re-embed/carry) -> core -> coda
          -> final norm + gate -> exit sampling -> loss-bearing row selection
          -> LM head GEMM -> vocabulary CE (writes dL/dlogits in place)
          -> LM head dX/dW (dL/dlogits is final at its depth)
          -> objective kernel (loss, metrics, dL/dgate)
backward  upstream gradient -> LM head gradient into the arena; per depth in
          reverse: gate head -> final norm -> coda -> carry/re-embed -> core;
          then prelude and the embedding.

Activation policy: every layer application keeps its input, the q|k|v
projections, the attention output and log-sum-exp, the post-attention
residual and the gate|up projections; norm outputs, rotary q/k and the SwiGLU
product are recomputed in the backward (cheap bandwidth-bound kernels), so no
GEMM or attention forward is ever recomputed.  The gradient checkpointing
settings of ModelConfig change memory in the reference, not results, and are
ignored here.

Parameters live in one contiguous arena per step engine (q|k|v and gate|up of
every layer adjacent, so each pair is one GEMM); gradients accumulate in a
float32 arena with the same offsets and are returned to autograd in the
parameter dtype.

Memory that varies from step to step (the loss-bearing row count of each
depth) never sizes an allocation: one depth's logits live in a persistent
buffer for the pack's row count, and the LM head's backward consumes them at
that depth, so every allocation of a step has the same size at every step of
the same pack shape and the caching allocator reuses its blocks.
"""

from dataclasses import dataclass
import ctypes
import math

import torch

from . import _lib
from ._lib import EPI_ACCUM, EPI_STORE_F32, call, ptr, query
from .batch import build_batch
from .layers import Kernels, LayerGrads, LayerWeights, Rope

METRIC_NAMES = ("denoising", "actor", "sampled_mean_depth", "prediction_cost",
                "regularization_cost", "profile_mean_depth", "first_pass_halt_probability")


@dataclass
class Dims:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    layers: int
    eps: float
    theta: float

    @classmethod
    def from_hf(cls, config):
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        rope = getattr(config, "rope_parameters", None) or {}
        theta = rope.get("rope_theta", getattr(config, "rope_theta", 10000.0))
        return cls(config.hidden_size, config.num_attention_heads, config.num_key_value_heads,
                   head_dim, config.intermediate_size, config.vocab_size,
                   config.num_hidden_layers, float(config.rms_norm_eps), float(theta))

    @property
    def qkv_width(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim


_LAYER_MATRICES = ("self_attn.q_proj.weight", "self_attn.k_proj.weight",
                   "self_attn.v_proj.weight", "self_attn.o_proj.weight", "mlp.gate_proj.weight",
                   "mlp.up_proj.weight", "mlp.down_proj.weight")
_LAYER_NORMS = ("input_layernorm.weight", "post_attention_layernorm.weight",
                "self_attn.q_norm.weight", "self_attn.k_norm.weight")
_ALIGN = 64  # elements


class Arena:
    """Parameters re-homed into one flat buffer, in a fixed order: the word
    embedding, every layer's projection matrices, the LM head, then one block
    of all the small tensors (norm weights, gate).  The float32 gradient arena
    has the same layout: its matrices receive their first contribution by
    overwriting, so only the embedding (sparse rows) and the small block are
    zeroed before a backward (``zero_spans``)."""

    def __init__(self, named_params, dims, device, dtype):
        self.dims, self.device, self.dtype = dims, device, dtype
        order = ["backbone.model.embed_tokens.weight"]
        for i in range(dims.layers):
            order += [f"backbone.model.layers.{i}.{s}" for s in _LAYER_MATRICES]
        order += ["backbone.lm_head.weight"]
        small = [f"backbone.model.layers.{i}.{s}" for i in range(dims.layers) for s in _LAYER_NORMS]
        small += ["backbone.model.norm.weight", "exit_gate.net.weight", "exit_gate.net.bias",
                  "exit_gate.depth_bias"]
        order += small
        params = dict(named_params)
        missing = set(order) ^ set(params)
        if missing:
            raise ValueError(f"unexpected parameter set for the Qwen3 ALoDLM arena: {sorted(missing)[:5]}")
        self.names = order
        self.offsets, total = {}, 0
        for name in order:
            numel = params[name].numel()
            keep_adjacent = name.endswith(("k_proj.weight", "v_proj.weight", "up_proj.weight"))
            if not keep_adjacent:
                total = (total + _ALIGN - 1) // _ALIGN * _ALIGN
            self.offsets[name] = total
            total += numel
        self.total = (total + _ALIGN - 1) // _ALIGN * _ALIGN
        embed_end = params["backbone.model.embed_tokens.weight"].numel()
        self.zero_spans = [(0, embed_end), (self.offsets[small[0]], self.total)]
        self.lm_span = (self.offsets["backbone.lm_head.weight"],
                        self.offsets["backbone.lm_head.weight"]
                        + params["backbone.lm_head.weight"].numel())
        self.flat = torch.empty(self.total, dtype=dtype, device=device)
        self.params = []
        for name in order:
            p = params[name]
            view = self.flat[self.offsets[name]:self.offsets[name] + p.numel()].view(p.shape)
            view.copy_(p.detach().to(device=device, dtype=dtype))
            p.data = view
            self.params.append(p)
        self.data_ptr = self.flat.data_ptr()

    def view(self, buf, name):
        p = self.params[self.names.index(name)]
        off = self.offsets[name]
        return buf[off:off + p.numel()].view(p.shape)

    def valid(self):
        return all(p.data.data_ptr() == self.flat.data_ptr() + self.offsets[n] * self.flat.element_size()
                   for n, p in zip(self.names, self.params))


def _layer_views(arena, buf, index, grads=False):
    """Views of one decoder layer's weights (or their gradients) in an arena
    buffer: q|k|v and gate|up are adjacent there, so each pair is one matrix."""
    d = arena.dims
    pre = f"backbone.model.layers.{index}."
    off = arena.offsets
    q = off[pre + "self_attn.q_proj.weight"]
    g = off[pre + "mlp.gate_proj.weight"]
    views = (buf[q:q + d.qkv_width * d.hidden].view(d.qkv_width, d.hidden),
             arena.view(buf, pre + "self_attn.o_proj.weight"),
             buf[g:g + 2 * d.intermediate * d.hidden].view(2 * d.intermediate, d.hidden),
             arena.view(buf, pre + "mlp.down_proj.weight"),
             arena.view(buf, pre + "input_layernorm.weight"),
             arena.view(buf, pre + "post_attention_layernorm.weight"),
             arena.view(buf, pre + "self_attn.q_norm.weight"),
             arena.view(buf, pre + "self_attn.k_norm.weight"))
    return LayerGrads(*views) if grads else LayerWeights(*views)


# Forward row count above which the QKV and gate/up products read
# out-contiguous weight copies: at 32768 rows (the 1.7B pack) the copies' products
# measured 2-4 % faster in the step than the [out, in] weights through the
# two-stage 64-deep kernel; at 4096 rows (the 8B pack) the products ran alike
# and refreshing those copies (read and write the weights each step) cost
# 3.6 ms of the 600 ms step.
ROWS_FOR_COPIES = 8192


class _TransposedWeights:
    """Out-contiguous copies ([in, out]) of projection weights, and the
    LM-head weight's finiteness flag.

    A forward product C = X . W^T through a copy reads W^T with out-contiguous
    rows (whole 512-byte rows per direct load).  The output and down
    projections always use their copies (2-7 % faster in the step); the QKV
    and gate/up projections use theirs in forwards of more than
    ROWS_FOR_COPIES rows (allocated at the first such forward) and read the
    arena weights otherwise; the LM head always reads its arena weight (3-6 %
    faster).  The copies in use are refreshed from the arena at the start of
    every forward, so they always match the parameters, and a copy not
    refreshed is unhooked from its layer; the backward uses the arena itself."""

    def __init__(self, engine):
        self.device, self.dtype = engine.device, engine.dtype
        self.jobs = self._allocate([(layer.wo, layer, "wo_t") for layer in engine.layers] +
                                   [(layer.wd, layer, "wd_t") for layer in engine.layers])
        self.optional = ([(layer.wqkv, layer, "wqkv_t") for layer in engine.layers] +
                         [(layer.wgu, layer, "wgu_t") for layer in engine.layers])
        self.optional_jobs = None
        self.lm_head = engine.lm_head
        # set by the refresh when an LM-head weight is inf or NaN: every row's
        # logits then hold a non-finite column, which makes the reference's
        # loss NaN through its 0 * sum(logits) term (alodlm/model.py:186)
        self.nonfinite = torch.zeros(1, dtype=torch.int32, device=engine.device)

    def _allocate(self, pairs):
        """One buffer for the copies of `pairs` (source [rows, cols], owner,
        attribute); each copy is hooked to its owner."""
        total, spans = 0, []
        for src, _, _ in pairs:
            spans.append(total)
            total += (src.numel() + _ALIGN - 1) // _ALIGN * _ALIGN
        buf = torch.empty(total, dtype=self.dtype, device=self.device)
        jobs = []
        for (src, owner, name), off in zip(pairs, spans):
            rows, cols = src.shape
            dst = buf[off:off + src.numel()].view(cols, rows)
            setattr(owner, name, dst)
            jobs.append((src, dst, rows, cols, owner, name))
        return jobs

    def refresh(self, code, stream, rows=0):
        """Refresh the copies a forward of `rows` rows reads (rows = 0: the
        decoder's windows, which read the QKV and gate/up arena weights)."""
        self.nonfinite.zero_()
        call("alodlm_check_finite", ptr(self.lm_head), self.lm_head.numel(), code,
             ptr(self.nonfinite), stream)
        use = rows > ROWS_FOR_COPIES
        if use and self.optional_jobs is None:
            self.optional_jobs = self._allocate(self.optional)
        jobs = self.jobs + (self.optional_jobs if use else [])
        for src, dst, r, c, _, _ in jobs:
            call("alodlm_transpose", ptr(src), ptr(dst), r, c, code, stream)
        for src, dst, r, c, owner, name in self.optional_jobs or []:
            setattr(owner, name, dst if use else None)


class StepEngine(Kernels):
    """Runs the ALoDLM step of one model on its GPU (see the module docstring)."""

    def __init__(self, model):
        backbone = model.backbone
        self.model = model
        self.cfg = model.config
        params = list(model.named_parameters())
        device, dtype = params[0][1].device, params[0][1].dtype
        if device.type != "cuda":
            raise ValueError("the HIP training step needs the model on a CUDA (ROCm) device")
        super().__init__(Dims.from_hf(backbone.config), dtype, device)
        self.arena = Arena(params, self.dims, self.device, self.dtype)
        d = self.dims
        if d.head_dim % 2:
            raise ValueError("head_dim must be even for the rotary embedding")
        self.layers = [_layer_views(self.arena, self.arena.flat, i) for i in range(d.layers)]
        a = self.arena
        self.embed = a.view(a.flat, "backbone.model.embed_tokens.weight")
        self.final_norm = a.view(a.flat, "backbone.model.norm.weight")
        self.lm_head = a.view(a.flat, "backbone.lm_head.weight")
        self.gate_w = a.view(a.flat, "exit_gate.net.weight")
        self.gate_b = a.view(a.flat, "exit_gate.net.bias")
        self.depth_bias = a.view(a.flat, "exit_gate.depth_bias")
        self.transposed = _TransposedWeights(self)
        # rotary inverse frequencies exactly as [tf] modeling_qwen3.py:115-117 (float32)
        inv = 1.0 / (d.theta ** (torch.arange(0, d.head_dim, 2, dtype=torch.float32) / d.head_dim))
        self.inv_freq = inv.to(self.device)
        # Which forward outputs the backward reuses instead of recomputing
        # (rotary q/k, then the two norm outputs of every layer application):
        # decided once, at the second step, from the first step's measured
        # memory peak; the values are the same either way.
        self._keep = None
        self._keep_rows = 0
        self._step_alloc = None
        self._step_peak = None
        # float32 gradients of the step in the arena layout (kept across steps)
        self.grads = None
        # a FusedAdamW that reads self.grads directly (see model._Step), and
        # whether self.grads holds gradients not yet consumed by its step
        self.fused_optimizer = None
        self.grads_pending = False
        self._written = None
        # weight-gradient products of the looped layers held until each
        # layer's last backward application (_flush_dw); group_dw forces the
        # choice (None: decided per backward by memory, _decide_group_dw)
        self.group_dw = None
        self._dw_pending = None
        # the readout's persistent buffers (_readout_buffers)
        self._readout = None

    # ------------------------------------------------------------------ memory policy
    KEEP_MARGIN = 0.06  # of the device memory left unplanned (allocator fragmentation)

    def _decide_keep(self, N):
        """(keep rotary q/k, keep norm outputs) for this step.  The first step
        keeps neither and measures how far its forward and backward raise the
        allocated memory (the device's peak statistics are reset at its start);
        the second step decides once, keeping each set only if that growth,
        plus optimizer state still to be allocated (the decision can precede
        the first optimizer step under gradient accumulation), plus the set's
        bytes fit in what this process can still allocate - the device's free
        memory (memory other processes hold is not free) plus the blocks the
        caching allocator holds unused - less KEEP_MARGIN of the device."""
        dev = self.device
        if self._keep is not None:
            # a pack with more rows than the one the decision was made for
            # keeps nothing: its activations alone outgrow that estimate
            return self._keep if N <= self._keep_rows else (False, False)
        if self._step_alloc is None:
            torch.cuda.reset_peak_memory_stats(dev)
            self._step_alloc = torch.cuda.memory_allocated(dev)
            self._grads_existed = self.grads is not None
            return (False, False)
        if self._step_peak is None:  # the first step ran no backward
            return (False, False)
        growth = self._step_peak - self._step_alloc
        allocated = torch.cuda.memory_allocated(dev)
        cached = torch.cuda.memory_reserved(dev) - allocated
        free, total = torch.cuda.mem_get_info(dev)
        headroom = free + cached - self.KEEP_MARGIN * total
        d, cfg = self.dims, self.cfg
        apps = cfg.loop_start + cfg.max_depth * (d.layers - cfg.loop_start)
        elem = 2 if self.dtype == torch.bfloat16 else 4
        rotary = apps * N * (d.heads + d.kv_heads) * d.head_dim * elem
        norms = apps * N * 2 * d.hidden * elem
        need = growth + self._optimizer_state_to_come()
        if not self._grads_existed and self.grads is not None:
            # the float32 gradient arena was allocated during the first step:
            # it is in the growth and already allocated now
            need -= self.grads.numel() * 4
        keep_rot = need + rotary <= headroom
        keep_norm = keep_rot and need + rotary + norms <= headroom
        self._keep = (keep_rot, keep_norm)
        self._keep_rows = N
        return self._keep

    def _optimizer_state_to_come(self):
        """Bytes of optimizer state that may still be allocated after the
        keep decision (with gradient accumulation the decision can come
        before the first optimizer step): the bound FusedAdamW's state not yet
        allocated, or - with no FusedAdamW bound - AdamW's float32 master and
        moments for every parameter (12 bytes each), counted conservatively
        because another optimizer's allocations are not visible here."""
        if self.fused_optimizer is not None:
            return self.fused_optimizer.state_bytes_to_come()
        return 12 * sum(p.numel() for p in self.arena.params)

    # ------------------------------------------------------------------ layer fwd/bwd
    def _layer_fwd(self, li, x, b, save):
        return self.layer_fwd(self.layers[li], x, b.kernel_mask, self._rope, save,
                              keep=self._keep_now if save is not None else (False, False), tag=li)

    def _layer_bwd(self, dy, saved, b, g, last=True):
        li = saved[0]
        # a layer's first backward application writes its matrices' gradients
        # (the arena is not zeroed there); later ones accumulate
        first = self._written is not None and li not in self._written
        if first:
            self._written.add(li)
        if self._dw_pending is None:
            return self.layer_bwd(dy, saved, self.layers[li], self.grad_layers[li],
                                  b.kernel_mask, self._rope, first=first)
        entries = []
        dx = self.layer_bwd(dy, saved, self.layers[li], self.grad_layers[li], b.kernel_mask,
                            self._rope, first=first, defer=entries)
        self._dw_pending.setdefault(li, []).append(entries)
        if last:
            self._flush_dw(li)
        return dx

    def _flush_dw(self, li):
        """The projection weight gradients of layer ``li`` over all its
        backward applications so far (alodlm/model.py:152: autograd sums the
        passes' gradients): per matrix one product whose k runs through the
        applications' rows in the order they were taken
        (alodlm_gemm_segk), written when the arena holds no earlier
        contribution of this backward, else added."""
        passes = self._dw_pending.pop(li)
        epi = EPI_ACCUM if self._written is None else EPI_STORE_F32
        for j in range(len(passes[0])):
            segs = [p[j] for p in passes]
            A, lda, B, ldb, C, ldc, M, Nc = segs[0]
            rows = A.shape[0]
            if len(segs) == 1 or not self._segk_eligible(segs, rows):
                for n, (A, lda, B, ldb, C, ldc, M, Nc) in enumerate(segs):
                    self._gemm(A, lda, 0, B, ldb, 0, C, ldc, M, Nc, A.shape[0],
                               epi=epi if n == 0 else EPI_ACCUM)
                continue
            self._gemm_segk(segs, rows, epi)

    def _gemm_segk(self, segs, rows, epi):
        """C (+)= sum_i A_i^T B_i over the segments' ``rows`` rows each
        (alodlm_gemm_segk); ``segs`` holds _layer_bwd's deferred operands."""
        A, lda, B, ldb, C, ldc, M, Nc = segs[0]
        a_ptrs = (ctypes.c_void_p * len(segs))(*[ptr(e[0]) for e in segs])
        b_ptrs = (ctypes.c_void_p * len(segs))(*[ptr(e[2]) for e in segs])
        need = query("alodlm_gemm_workspace", M, Nc, rows * len(segs), epi, self.code)
        ws = self._workspace(need) if need else None
        call("alodlm_gemm_segk", ctypes.addressof(a_ptrs), ctypes.addressof(b_ptrs), len(segs),
             rows, lda, ldb, ptr(C), ldc, M, Nc, 1.0, epi, ptr(ws), self._stream())

    def _segk_eligible(self, segs, rows):
        A, lda, B, ldb, C, ldc, M, Nc = segs[0]
        return (len(segs) <= 8 and self.dtype == torch.bfloat16 and rows % 32 == 0
                and M >= 256 and Nc >= 256 and M % 8 == 0 and Nc % 8 == 0
                and lda % 8 == 0 and ldb % 8 == 0
                and all(e[0].shape[0] == rows and e[2].shape[0] == rows
                        and ptr(e[0]) % 16 == 0 and ptr(e[2]) % 16 == 0 for e in segs))

    def _decide_group_dw(self, N, looped):
        """Whether this backward holds the looped layers' weight-gradient
        operands until their last application (one product per matrix over
        all passes instead of one per pass): only if those operands of
        max_depth - 1 passes fit in half of what this process can still
        allocate."""
        if self.group_dw is not None:
            return bool(self.group_dw)
        K, d = self.cfg.max_depth, self.dims
        if K < 2 or K > 8 or self.dtype != torch.bfloat16 or N % 32 or not looped:
            return False
        QD = d.heads * d.head_dim
        per_pass = N * (4 * d.hidden + 3 * d.intermediate + QD + d.qkv_width) * 2
        need = (K - 1) * looped * per_pass
        dev = self.device
        free, _ = torch.cuda.mem_get_info(dev)
        cached = torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev)
        return need < 0.5 * (free + cached)

    # ------------------------------------------------------------------ shared pieces
    def _carry(self, core_out, b, exits, depth):
        """Input of core pass ``depth``: exits <= depth ? E[original] :
        norm(core_out) (alodlm/model.py:150-151,168), one launch."""
        d = self.dims
        N, H = core_out.shape
        xin = self._empty(N, H)
        rstd = self._empty(N, dtype=torch.float32)
        call("alodlm_carry_select", ptr(core_out), ptr(self.final_norm), ptr(self.embed),
             ptr(b.original), ptr(exits), depth, ptr(xin), ptr(rstd), N, H, d.vocab, d.eps,
             self.code, self._stream())
        return xin, rstd

    def _carry_bwd(self, dnext, core_out, rstd, plan, exits, depth, dres, g_norm, g_embed):
        """Backward of ``_carry`` at ``depth``: carried rows go back through the
        carry norm into the previous core output (plus ``dres``), re-embedded
        rows into the embedding table (``plan``: the embed plan of the
        original tokens)."""
        N, H = core_out.shape
        dcore = self._empty(N, H)
        ws = self._workspace(query("alodlm_carry_select_bwd_workspace", N, H))
        call("alodlm_carry_select_bwd", ptr(dnext), ptr(core_out), ptr(rstd),
             ptr(self.final_norm), ptr(exits), depth, ptr(plan), ptr(dres), ptr(dcore),
             ptr(g_norm), ptr(g_embed), ptr(ws), N, H, self.dims.vocab, self.code, self._stream())
        return dcore

    def _gate_pass(self, r, depth, gates, exits, b, exit_uniforms, generator, rec):
        """Final norm and gate of pass ``depth`` (alodlm/model.py:160-162) and,
        before the last pass, the exit sampling (model.py:163-167)."""
        d, K = self.dims, self.cfg.max_depth
        N, H = r.shape
        st, c = self._stream(), self.code
        readout = self._empty(N, H)
        rstd_f = self._empty(N, dtype=torch.float32)
        call("alodlm_final_norm_gate", ptr(r), ptr(self.final_norm), ptr(self.gate_w),
             ptr(self.gate_b), ptr(self.depth_bias), depth, ptr(readout), ptr(rstd_f),
             ptr(gates[depth]), N, H, d.eps, c, st)
        rec["final_in"], rec["readout"], rec["rstd_f"] = r, readout, rstd_f
        if depth < K - 1:
            if exit_uniforms is not None:
                u = exit_uniforms[depth].to(device=self.device, dtype=torch.float32).contiguous()
            else:
                u = torch.rand(N, device=self.device, generator=generator)
            call("alodlm_exit_update", ptr(gates[depth]), ptr(u), ptr(b.masked), ptr(exits),
                 depth, K, N, st)
        return readout

    def _readout_buffers(self, N):
        """Persistent buffers of the readout for packs of N rows: the logits
        of one depth's loss-bearing rows ([R, V], R <= N, rounded up to 32),
        the gathered rows and their input gradient.  Allocated once per pack
        size, so the step's largest allocation has the same size at every
        step whatever the loss-bearing row counts."""
        cap = -(-N // 32) * 32
        if self._readout is None or self._readout[0] != cap:
            self._readout = None
            H, V = self.dims.hidden, self.dims.vocab
            self._readout = (cap, self._empty(cap, V), self._empty(cap, H), self._empty(cap, H))
        return self._readout[1:]

    def _lm_readout(self, readout, depth, gates, exits, b, wsum, ar_coef, ce_all, ent_all,
                    need_grad, rec, g_lm=None, lm_first=True):
        """Loss-bearing rows of pass ``depth`` through the LM head and the
        vocabulary cross-entropy (alodlm/model.py:161,180-181; loss.py:12-32):
        rows are selected and weighted by alodlm_select_rows, their logits
        become dL/dlogits in place (with a unit upstream gradient), and each
        row's cross-entropy and token entropy -sum p log p (the decoder's
        commit score, alodlm/inference.py:114-117) land in row order in
        ``ce_all[depth]`` / ``ent_all[depth]``.  That
        gradient is final here, so with ``need_grad`` the LM head's backward
        runs right away: the readout gradient [N, H] is kept in ``rec`` and
        the LM head's weight gradient goes into the float32 ``g_lm`` (written
        when ``lm_first``, else accumulated).  Returns whether it wrote
        ``g_lm``."""
        d, K = self.dims, self.cfg.max_depth
        N, H = readout.shape
        V = d.vocab
        st, c = self._stream(), self.code
        sel_rows = torch.empty(N, dtype=torch.int32, device=self.device)
        sel_target = torch.empty(N, dtype=torch.int32, device=self.device)
        sel_coef = torch.empty(N, dtype=torch.float32, device=self.device)
        sel_count = torch.empty(1, dtype=torch.int32, device=self.device)
        call("alodlm_select_rows", ptr(b.masked), ptr(exits), ptr(b.original), ptr(b.ar_target),
             ptr(gates), ptr(b.mask_probability), ptr(wsum), ar_coef, depth, K, N, ptr(sel_rows),
             ptr(sel_target), ptr(sel_coef), ptr(sel_count), st)
        R = int(sel_count.item())
        rec["R"], rec["sel_rows"] = R, sel_rows
        if need_grad:
            rec["dread"] = self._empty(N, H)
        if not R:
            if need_grad:
                rec["dread"].zero_()
            return False
        # Rows padded to a multiple of 32 with zeros: their logits and
        # dL/dlogits are exactly zero, and the LM-head dW product (whose
        # depth is the row count) runs on whole 32-deep k stages.
        Rp = -(-R // 32) * 32
        logits_buf, xsel_buf, dsel_buf = self._readout_buffers(N)
        xsel = xsel_buf[:Rp]
        if Rp > R:
            xsel[R:].zero_()
        call("alodlm_gather_rows", ptr(readout), ptr(sel_rows), R, ptr(xsel), H, c, st)
        logits = logits_buf[:Rp]
        self._gemm(xsel, H, 1, self.lm_head, H, 1, logits, V, Rp, V, H)
        ce = torch.empty(2, R, dtype=torch.float32, device=self.device)
        call("alodlm_cross_entropy", ptr(logits), ptr(sel_target), ptr(sel_coef),
             ptr(sel_count), R, V, ptr(ce[0]), ptr(ce[1]), c, st)
        call("alodlm_scatter_ce", ptr(ce[0]), ptr(sel_rows), ptr(sel_count), R,
             ptr(ce_all[depth]), N, st)
        call("alodlm_scatter_ce", ptr(ce[1]), ptr(sel_rows), ptr(sel_count), R,
             ptr(ent_all[depth]), N, st)
        if not need_grad:
            return False
        # d readout = dlogits . W_lm ; dW_lm (+)= dlogits^T . readout
        dsel = dsel_buf[:R]
        self._gemm(logits, V, 1, self.lm_head, H, 0, dsel, H, R, H, V)
        self._gemm(logits, V, 0, xsel, H, 0, g_lm, H, V, H, Rp,
                   epi=EPI_STORE_F32 if lm_first else EPI_ACCUM)
        call("alodlm_scatter_rows", ptr(dsel), ptr(sel_rows), R, ptr(rec["dread"]), N, H, c, st)
        return True

    def _objective(self, gates, exits, b, ce_all, N, S, K):
        out = torch.empty(10, dtype=torch.float32, device=self.device)
        dgate = torch.empty(K, N, dtype=torch.float32, device=self.device)
        cfg = self.cfg
        ws = self._workspace(query("alodlm_objective_workspace", N, S, K))
        call("alodlm_objective", ptr(gates), ptr(exits), ptr(b.masked), ptr(b.mask_probability),
             ptr(ce_all), ptr(ce_all), ptr(b.ar_target), ptr(b.boundaries), S, N, K,
             cfg.depth_prior_c, cfg.kl_beta_mi, cfg.kl_beta_marg, ptr(self.transposed.nonfinite),
             ptr(out), ptr(dgate), ptr(ws), self._stream())
        return out, dgate

    def _readout_bwd(self, rec, depth, dgate, scale, g_norm, g_gw, g_gb, g_db):
        """Backward of pass ``depth``'s readout after the LM head (whose
        backward ran in the forward): the upstream gradient ``scale`` (a
        float32 device scalar, or None for 1) applied to the readout
        gradient, the gate head, the final norm; returns d final_in."""
        N, H = rec["readout"].shape
        st, c = self._stream(), self.code
        dread = rec.pop("dread")
        if scale is not None:
            call("alodlm_scale", ptr(dread), ptr(scale), dread.numel(), c, st)
        ws = self._workspace(query("alodlm_gate_bwd_workspace", N, H))
        call("alodlm_gate_bwd", ptr(dgate), ptr(rec["readout"]), 1.0, ptr(g_gw), ptr(g_gb),
             ptr(g_db), depth, N, H, ptr(ws), c, st)
        dr = self._empty(N, H)
        ws = self._workspace(query("alodlm_rmsnorm_bwd_workspace", N, H))
        call("alodlm_rmsnorm_bwd", ptr(dread), ptr(rec["final_in"]), ptr(rec["rstd_f"]),
             ptr(self.final_norm), None, ptr(dr), ptr(g_norm), ptr(ws), N, H, c, st)
        return dr

    def _lm_grad_store(self, state, scale, grads, accumulate):
        """The LM head's weight gradient of the forward (unit upstream
        gradient, float32) into the arena: scaled by ``scale`` and written,
        or added under ``accumulate``; zero when no depth had loss-bearing
        rows."""
        lo, hi = self.arena.lm_span
        dst = grads[lo:hi]
        if state["lm_written"]:
            call("alodlm_scale_add_f32", ptr(state["g_lm"]), ptr(dst), hi - lo, ptr(scale),
                 int(accumulate), self._stream())
        elif not accumulate:
            dst.zero_()
        state["g_lm"] = None

    def _upstream(self, grad_scale, dgate):
        """The upstream gradient of the loss as a float32 device scalar (None
        for a host 1.0), applied to the gate-logit gradients ``dgate``."""
        if isinstance(grad_scale, (int, float)):
            if grad_scale == 1.0:
                return None
            scale = torch.tensor([float(grad_scale)], dtype=torch.float32, device=self.device)
        else:
            scale = grad_scale.detach().to(device=self.device, dtype=torch.float32).reshape(1)
        call("alodlm_scale_f32", ptr(dgate), ptr(scale), dgate.numel(), self._stream())
        return scale

    def _grad_views(self, grads):
        a = self.arena
        names = ("backbone.model.embed_tokens.weight", "backbone.model.norm.weight",
                 "backbone.lm_head.weight", "exit_gate.net.weight", "exit_gate.net.bias",
                 "exit_gate.depth_bias")
        return [a.view(grads, n) for n in names]

    # ------------------------------------------------------------------ step
    def forward(self, ids, labels, boundaries, need_grad, exit_uniforms=None, draws=None,
                generator=None):
        """Run the forward of the step; returns (out[10] float tensor, state)."""
        if not self.arena.valid():
            raise RuntimeError("model parameters were moved after the step engine was built")
        cfg, d = self.cfg, self.dims
        K = cfg.max_depth
        st, c = self._stream(), self.code
        # host inputs (a pack from the data loader): the labels are read on the
        # host and the copies to the device do not block
        labels_host = labels.numpy() if labels.device.type == "cpu" else None
        pin = lambda t: t.pin_memory() if t.device.type == "cpu" and not t.is_pinned() else t
        ids = pin(ids).to(self.device, non_blocking=True)
        labels = pin(labels).to(self.device, non_blocking=True)
        b = build_batch(ids, labels, boundaries, cfg.block_size, cfg.mask_token_id,
                        generator=generator, draws=draws, labels_host=labels_host)
        self._rope = Rope(positions=b.positions, inv_freq=self.inv_freq)
        N, H, V = b.ids.numel(), d.hidden, d.vocab
        self.transposed.refresh(c, st, N)
        S = b.boundaries.numel() - 1
        saves = [] if need_grad else None
        # the readout's persistent buffers and this step's LM-head gradient
        # exist before the keep decision measures the memory
        self._readout_buffers(N)
        g_lm = self._empty(V, H, dtype=torch.float32) if need_grad else None
        self._keep_now = self._decide_keep(N) if need_grad else (False, False)
        x = self._empty(N, H)
        call("alodlm_embed_gather", ptr(self.embed), ptr(b.ids), ptr(x), N, H, V, c, st)
        for li in range(cfg.loop_start):
            x = self._layer_fwd(li, x, b, saves)
        gates = torch.empty(K, N, dtype=torch.float32, device=self.device)
        exits = torch.full((N,), K, dtype=torch.int32, device=self.device)
        ce_all = torch.zeros(K, N, dtype=torch.float32, device=self.device)
        ent_all = torch.zeros(K, N, dtype=torch.float32, device=self.device)
        wsum = torch.empty(1, dtype=torch.float32, device=self.device)
        call("alodlm_inverse_weight_sum", ptr(b.masked), ptr(b.mask_probability), N, ptr(wsum), st)
        ar_coef = 0.5 / (K * b.ar_count) if b.ar_count else 0.0
        depths = []
        core_in = x
        lm_written = False
        for depth in range(K):
            rec = {}
            if depth:
                core_in, depths[-1]["carry_rstd"] = self._carry(core_out, b, exits, depth)
            h = core_in
            rec["core_saves"] = [] if need_grad else None
            for li in range(cfg.loop_start, cfg.loop_end):
                h = self._layer_fwd(li, h, b, rec["core_saves"])
            core_out = h
            rec["core_out"] = core_out
            r = core_out
            rec["coda_saves"] = [] if need_grad else None
            for li in range(cfg.loop_end, d.layers):
                r = self._layer_fwd(li, r, b, rec["coda_saves"])
            readout = self._gate_pass(r, depth, gates, exits, b, exit_uniforms, generator, rec)
            lm_written |= self._lm_readout(readout, depth, gates, exits, b, wsum, ar_coef, ce_all,
                                           ent_all, need_grad, rec, g_lm, not lm_written)
            depths.append(rec)
        out, dgate = self._objective(gates, exits, b, ce_all, N, S, K)
        self.last_rows = [rec["R"] for rec in depths]
        state = {"batch": b, "gates": gates, "exits": exits, "ce": ce_all, "entropy": ent_all,
                 "dgate": dgate, "prelude": saves, "depths": depths, "g_lm": g_lm,
                 "lm_written": lm_written}
        return out, state

    def backward(self, state, grad_scale, accumulate=False):
        """Backward of the step into the float32 gradient arena ``self.grads``
        (returned), for the loss's upstream gradient ``grad_scale`` (a float,
        or a device scalar that is never read on the host).  Without
        ``accumulate`` the arena's previous contents are replaced: each
        matrix's first contribution is written, the embedding and the small
        tensors are zeroed first; with it every contribution is added
        (gradient accumulation)."""
        cfg, d = self.cfg, self.dims
        K, st, c = cfg.max_depth, self._stream(), self.code
        b = state["batch"]
        N, H, V = b.ids.numel(), d.hidden, d.vocab
        if self.grads is None:
            self.grads = torch.zeros(self.arena.total, dtype=torch.float32, device=self.device)
        grads = self.grads
        self._written = None if accumulate else set()
        if not accumulate:
            for lo, hi in self.arena.zero_spans:
                grads[lo:hi].zero_()
        self.grad_layers = [_layer_views(self.arena, grads, i, grads=True) for i in range(d.layers)]
        g_embed, g_norm, g_lm, g_gw, g_gb, g_db = self._grad_views(grads)
        exits = state["exits"]
        scale = self._upstream(grad_scale, state["dgate"])
        self._lm_grad_store(state, scale, grads, accumulate)
        plan_original = self.embed_plan(b.original) if K > 1 else None
        # the looped layers' weight gradients: one product per matrix over the
        # passes, at each layer's last application (depth 0), when it fits
        looped = len(state["depths"][0]["coda_saves"]) + len(state["depths"][0]["core_saves"])
        self._dw_pending = {} if self._decide_group_dw(N, looped) else None
        dnext = None  # gradient at the core input of depth+1
        for depth in reversed(range(K)):
            rec = state["depths"][depth]
            dr = self._readout_bwd(rec, depth, state["dgate"][depth], scale, g_norm, g_gw, g_gb,
                                   g_db)
            for saved in reversed(rec["coda_saves"]):
                dr = self._layer_bwd(dr, saved, b, grads, last=depth == 0)
            if dnext is not None:
                # x_in(depth+1) = exits <= depth+1 ? E[original] : norm(core_out(depth))
                dr = self._carry_bwd(dnext, rec["core_out"], rec["carry_rstd"], plan_original,
                                     exits, depth + 1, dr, g_norm, g_embed)
            for saved in reversed(rec["core_saves"]):
                dr = self._layer_bwd(dr, saved, b, grads, last=depth == 0)
            dnext = dr
        dx = dnext
        for saved in reversed(state["prelude"]):
            dx = self._layer_bwd(dx, saved, b, grads)
        if self._dw_pending is not None:
            for li in list(self._dw_pending):
                self._flush_dw(li)
            self._dw_pending = None
        self.embed_scatter(dx, self.embed_plan(b.ids), g_embed)
        self._written = None
        return grads

    def note_step_peak(self):
        """Record the first step's memory peak (forward, backward and the
        gradients handed to autograd) for the keep decision."""
        if self._step_alloc is not None and self._step_peak is None:
            self._step_peak = torch.cuda.max_memory_allocated(self.device)

    # ------------------------------------------------------------------ stages
    def core_forward(self, x0, batch, need_grad=True, exit_uniforms=None, generator=None):
        """The shared recurrent core alone (alodlm/model.py:147-168 without the
        prelude, coda and LM head): K passes of the core layers
        [loop_start, loop_end) from the hidden states x0 [N, H], the gate on
        the final norm of each pass's output, exit sampling, and between
        passes the carry norm or, for committed rows, the re-embedding of
        ``batch.original``.  ``batch`` is a build_batch result.

        Returns (outputs: K tensors [N, H], gates [K, N] float32, exits [N]
        int32, state for core_backward)."""
        if not self.arena.valid():
            raise RuntimeError("model parameters were moved after the step engine was built")
        cfg, d = self.cfg, self.dims
        K, N = cfg.max_depth, x0.shape[0]
        if x0.shape != (batch.ids.numel(), d.hidden) or x0.dtype != self.dtype:
            raise ValueError("x0 must be [rows, hidden] in the parameter dtype")
        self.transposed.refresh(self.code, self._stream(), N)
        b = batch
        self._rope = Rope(positions=b.positions, inv_freq=self.inv_freq)
        self._keep_now = (False, False)
        gates = torch.empty(K, N, dtype=torch.float32, device=self.device)
        exits = torch.full((N,), K, dtype=torch.int32, device=self.device)
        depths, h = [], x0.contiguous()
        for depth in range(K):
            rec = {}
            if depth:
                h, depths[-1]["carry_rstd"] = self._carry(core_out, b, exits, depth)
            rec["core_saves"] = [] if need_grad else None
            for li in range(cfg.loop_start, cfg.loop_end):
                h = self._layer_fwd(li, h, b, rec["core_saves"])
            core_out = h
            rec["core_out"] = core_out
            self._gate_pass(core_out, depth, gates, exits, b, exit_uniforms, generator, rec)
            depths.append(rec)
        state = {"batch": b, "gates": gates, "exits": exits, "depths": depths}
        return [rec["core_out"] for rec in depths], gates, exits, state

    def core_backward(self, state, douts, dgates=None):
        """Backward of core_forward for output gradients ``douts`` (K tensors
        [N, H]) and optional gate-logit gradients ``dgates`` [K, N] float32
        (they reach only the gate parameters: the gate reads the detached
        readout).  Returns (dx0, float32 gradients in the arena layout)."""
        cfg, d = self.cfg, self.dims
        K = cfg.max_depth
        b = state["batch"]
        grads = torch.zeros(self.arena.total, dtype=torch.float32, device=self.device)
        self.grad_layers = [_layer_views(self.arena, grads, i, grads=True) for i in range(d.layers)]
        self._written = None
        g_embed, g_norm, _, g_gw, g_gb, g_db = self._grad_views(grads)
        exits = state["exits"]
        plan_original = self.embed_plan(b.original) if K > 1 else None
        first = state["depths"][0]
        self._dw_pending = ({} if self._decide_group_dw(first["core_out"].shape[0],
                                                        len(first["core_saves"])) else None)
        dnext = None
        for depth in reversed(range(K)):
            rec = state["depths"][depth]
            N, H = rec["core_out"].shape
            dr = douts[depth].to(self.dtype).contiguous()
            if dgates is not None:
                g = dgates[depth].to(torch.float32).contiguous()
                ws = self._workspace(query("alodlm_gate_bwd_workspace", N, H))
                call("alodlm_gate_bwd", ptr(g), ptr(rec["readout"]), 1.0, ptr(g_gw), ptr(g_gb),
                     ptr(g_db), depth, N, H, ptr(ws), self.code, self._stream())
            if dnext is not None:
                dr = self._carry_bwd(dnext, rec["core_out"], rec["carry_rstd"], plan_original,
                                     exits, depth + 1, dr, g_norm, g_embed)
            for saved in reversed(rec["core_saves"]):
                dr = self._layer_bwd(dr, saved, b, grads, last=depth == 0)
            dnext = dr
        if self._dw_pending is not None:
            for li in list(self._dw_pending):
                self._flush_dw(li)
            self._dw_pending = None
        return dnext, grads

    def readout_forward(self, finals, batch, need_grad=True, exit_uniforms=None, generator=None):
        """The fused readout and objective alone (alodlm/model.py:157-187 from
        the final hidden states): for each of the K passes, the final norm of
        ``finals[d]`` [N, H] with the gate, exit sampling, the LM head over the
        loss-bearing rows (masked rows not yet exited, and rows with an
        autoregressive target), the vocabulary cross-entropy; then the
        objective.  ``batch`` holds masked, original (targets),
        mask_probability, boundaries (segment offsets over the N rows),
        ar_target and ar_count.  The state holds the per-pass cross-entropy
        and token entropy of the loss-bearing rows (``ce``, ``entropy``
        [K, N] float32, zero elsewhere).

        Returns (out[10] as the step's, state for readout_backward)."""
        cfg, d = self.cfg, self.dims
        K = cfg.max_depth
        N = finals[0].shape[0]
        if len(finals) != K or any(f.shape != (N, d.hidden) or f.dtype != self.dtype
                                   for f in finals):
            raise ValueError("finals must be max_depth tensors [rows, hidden] in the parameter dtype")
        st = self._stream()
        self.transposed.refresh(self.code, st, N)
        b = batch
        g_lm = self._empty(d.vocab, d.hidden, dtype=torch.float32) if need_grad else None
        S = b.boundaries.numel() - 1
        gates = torch.empty(K, N, dtype=torch.float32, device=self.device)
        exits = torch.full((N,), K, dtype=torch.int32, device=self.device)
        ce_all = torch.zeros(K, N, dtype=torch.float32, device=self.device)
        ent_all = torch.zeros(K, N, dtype=torch.float32, device=self.device)
        wsum = torch.empty(1, dtype=torch.float32, device=self.device)
        call("alodlm_inverse_weight_sum", ptr(b.masked), ptr(b.mask_probability), N, ptr(wsum), st)
        ar_coef = 0.5 / (K * b.ar_count) if b.ar_count else 0.0
        depths = []
        lm_written = False
        for depth in range(K):
            rec = {}
            readout = self._gate_pass(finals[depth].contiguous(), depth, gates, exits, b,
                                      exit_uniforms, generator, rec)
            lm_written |= self._lm_readout(readout, depth, gates, exits, b, wsum, ar_coef, ce_all,
                                           ent_all, need_grad, rec, g_lm, not lm_written)
            depths.append(rec)
        out, dgate = self._objective(gates, exits, b, ce_all, N, S, K)
        self.last_rows = [rec["R"] for rec in depths]
        state = {"batch": b, "gates": gates, "exits": exits, "ce": ce_all, "entropy": ent_all,
                 "dgate": dgate, "depths": depths, "g_lm": g_lm, "lm_written": lm_written}
        return out, state

    def readout_backward(self, state, grad_scale=1.0):
        """Backward of readout_forward: returns (K gradients [N, H] of the final
        hidden states, float32 gradients in the arena layout: LM head, final
        norm, gate)."""
        K = self.cfg.max_depth
        grads = torch.zeros(self.arena.total, dtype=torch.float32, device=self.device)
        _, g_norm, _, g_gw, g_gb, g_db = self._grad_views(grads)
        scale = self._upstream(grad_scale, state["dgate"])
        self._lm_grad_store(state, scale, grads, False)
        dfinals = [None] * K
        for depth in reversed(range(K)):
            dfinals[depth] = self._readout_bwd(state["depths"][depth], depth,
                                               state["dgate"][depth], scale, g_norm, g_gw, g_gb,
                                               g_db)
        return dfinals, grads
