"""Clipped AdamW with float32 master weights on the HIP kernels.

Drop-in for the optimizer sub-step of alodlm/train.py:42-56,138-148:
``torch.optim.AdamW(groups, lr)`` with betas (0.9, 0.999), eps 1e-8 and the
reference's two weight-decay groups, preceded by ``clip_grad_norm_(params,
max_norm)``.  Differences by design: bf16 parameters keep a float32 master copy
and float32 moments (the reference's plain bf16 run keeps bf16 parameters and
moments; its ZeRO-2 run keeps float32 masters), and the clip coefficient is
applied inside the AdamW kernel from a device-side norm, so no host sync is
needed.  Over exactly the parameters of an ALoDLM model the optimizer reads
the step's float32 gradient arena itself (no rounding of the gradients to
bf16, no bf16 gradient copy); ``.grad`` then stays unset unless
``ALoDLM.materialize_grads()`` is called.
"""

import weakref

import torch

from . import _lib

CHUNK = 1 << 16


class _Table:
    """Device tensor list (pointers, sizes) and its fixed-size chunk table."""

    def __init__(self, tensors, device):
        numels = [t.numel() for t in tensors]
        chunk_tensor, chunk_start = [], []
        for i, n in enumerate(numels):
            for start in range(0, n, CHUNK):
                chunk_tensor.append(i)
                chunk_start.append(start)
        self.n_chunks = len(chunk_tensor)
        self.numels = torch.tensor(numels, dtype=torch.int64, device=device)
        self.chunk_tensor = torch.tensor(chunk_tensor, dtype=torch.int32, device=device)
        self.chunk_start = torch.tensor(chunk_start, dtype=torch.int64, device=device)

    @staticmethod
    def pointers(tensors, device):
        # staged through pinned memory and copied without blocking, so a step
        # never waits for the backward still queued on the stream
        host = torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64).pin_memory()
        return host.to(device, non_blocking=True)


class FusedAdamW(torch.optim.Optimizer):
    """AdamW over float32 masters with an optional fused global-norm clip.

    ``max_grad_norm``: when set, ``step()`` clips the gradients to this global
    L2 norm (torch.nn.utils.clip_grad_norm_ semantics) inside the kernel; the
    norm of the last step is ``self.last_grad_norm`` (a device scalar).
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01,
                 max_grad_norm=None):
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        super().__init__(params, defaults)
        self.max_grad_norm = max_grad_norm
        self.last_grad_norm = None
        self._tables = None
        self._norm_ready = False
        # Over exactly the parameters of an ALoDLM, read the step's float32
        # gradient arena directly instead of .grad (see model._Step).
        from .model import model_of
        model = model_of(self._params())
        self._model = None
        if model is not None:
            self._model = weakref.ref(model)
            self._names = {id(p): name for name, p in model.named_parameters()}
            model.bind_optimizer(self)

    def _bound_engine(self):
        model = self._model() if self._model is not None else None
        engine = model._engine if model is not None else None
        return engine if engine is not None and engine.fused_optimizer is self else None

    def state_bytes_to_come(self):
        """Bytes of float32 master / moment state not allocated yet (allocated
        at the first step): 8 per element, 12 when the parameter is not float32."""
        total = 0
        for p in self._params():
            if not self.state.get(p):
                total += p.numel() * (8 if p.dtype == torch.float32 else 12)
        return total

    def _arena_engine(self):
        """The bound model's engine when its float32 arena holds the gradients
        of a backward since the last zero_grad (else None)."""
        engine = self._bound_engine()
        return engine if engine is not None and engine.grads_pending else None

    def _has_grads(self):
        """Whether a step has gradients to apply: the bound arena's, or any
        ``.grad`` (a backward that ran before this optimizer was bound fills
        ``.grad``, as an unbound model always does)."""
        return (self._arena_engine() is not None
                or any(p.grad is not None for p in self._params()))

    def _grads(self, params):
        """(gradient tensors, dtype code) for ``params``: the bound model's
        float32 arena views, or ``.grad`` (zeros where unset).  None when there
        are no gradients since the last zero_grad."""
        engine = self._arena_engine()
        if engine is not None:
            return ([engine.arena.view(engine.grads, self._names[id(p)]) for p in params],
                    _lib.F32_CODE)
        if self._bound_engine() is not None and not self._has_grads():
            return None, None
        grads = [p.grad if p.grad is not None else torch.zeros_like(p) for p in params]
        for g in grads:
            if g.dtype != self._dtype or not g.is_contiguous():
                raise ValueError("gradients must be contiguous and of the parameter dtype")
        return grads, self._code

    def _check_tables(self):
        """(Re)build the pointer tables when parameters were moved or re-homed
        since they were built."""
        if self._tables is None or [p.data_ptr() for p in self._params()] != self._ptrs:
            self._prepare()

    def _params(self):
        return [p for g in self.param_groups for p in g["params"]]

    def _prepare(self):
        params = self._params()
        dtypes = {p.dtype for p in params}
        devices = {p.device for p in params}
        if len(dtypes) != 1 or len(devices) != 1:
            raise ValueError("FusedAdamW needs parameters of one dtype on one device")
        device = devices.pop()
        if device.type != "cuda":
            raise ValueError("FusedAdamW runs on the GPU")
        self._device, self._dtype = device, dtypes.pop()
        self._code = _lib.dtype_code(self._dtype)
        for p in params:
            state = self.state[p]
            if not state:
                state["step"] = 0
                state["master"] = (p.detach() if p.dtype == torch.float32
                                   else p.detach().float().clone())
                state["exp_avg"] = torch.zeros(p.shape, dtype=torch.float32, device=device)
                state["exp_avg_sq"] = torch.zeros(p.shape, dtype=torch.float32, device=device)
            elif p.dtype == torch.float32 and state["master"].data_ptr() != p.data_ptr():
                # a float32 parameter is its own master: follow it to its new
                # storage (the step engine re-homes parameters into its arena)
                p.data.copy_(state["master"])
                state["master"] = p.detach()
        self._tables = []
        for group in self.param_groups:
            ps = group["params"]
            if not ps:
                self._tables.append(None)
                continue
            table = _Table(ps, device)
            table.params = _Table.pointers(ps, device)
            table.master = _Table.pointers([self.state[p]["master"] for p in ps], device)
            table.m = _Table.pointers([self.state[p]["exp_avg"] for p in ps], device)
            table.v = _Table.pointers([self.state[p]["exp_avg_sq"] for p in ps], device)
            table.wd = torch.full((len(ps),), float(group["weight_decay"]), dtype=torch.float32,
                                  device=device)
            self._tables.append(table)
        self._all = _Table(params, device)
        self._partial = torch.empty(self._all.n_chunks, dtype=torch.float32, device=device)
        self._norm = torch.zeros(1, dtype=torch.float32, device=device)
        self._ptrs = [p.data_ptr() for p in params]

    def zero_grad(self, set_to_none=True):
        self._norm_ready = False
        engine = self._bound_engine()
        if engine is not None:
            engine.grads_pending = False
        super().zero_grad(set_to_none)

    def load_state_dict(self, state_dict):
        """Restore a ``state_dict()`` of this optimizer or of a
        ``torch.optim.AdamW`` over the same parameter groups.

        The float32 masters and moments are restored as float32 whatever the
        parameter dtype (``torch.optim.Optimizer.load_state_dict`` would cast
        them to it).  Float32 parameters take their master's values and share
        its storage again.  A state without masters (torch's AdamW keeps
        none) takes them from the parameters' current values.
        """
        saved_groups = state_dict["param_groups"]
        if len(saved_groups) != len(self.param_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        for group, saved in zip(self.param_groups, saved_groups):
            if len(group["params"]) != len(saved["params"]):
                raise ValueError("loaded state dict contains a parameter group that doesn't "
                                 "match the size of optimizer's group")
        self.state.clear()
        for group, saved in zip(self.param_groups, saved_groups):
            for key, value in saved.items():
                if key != "params":
                    group[key] = value
            for p, index in zip(group["params"], saved["params"]):
                entry = state_dict["state"].get(index)
                if not entry:
                    continue
                f32 = lambda t: t.to(device=p.device, dtype=torch.float32).clone()
                master = f32(entry["master"] if "master" in entry else p.detach())
                if p.dtype == torch.float32:
                    p.data.copy_(master)
                    master = p.detach()
                self.state[p] = {"step": int(entry["step"]), "master": master,
                                 "exp_avg": f32(entry["exp_avg"]),
                                 "exp_avg_sq": f32(entry["exp_avg_sq"])}
        self._tables = None
        self._norm_ready = False

    def grad_norm(self):
        """Global L2 norm of all gradients into a device scalar (no host sync).

        The next ``step()`` clips with this norm instead of computing it again,
        so the gradients must not change in between."""
        self._check_tables()
        params = self._params()
        grads, code = self._grads(params)
        if grads is None:
            self._norm.zero_()
            grads = []
        else:
            gptr = _Table.pointers(grads, self._device)
            _lib.call("alodlm_grad_norm", _lib.ptr(gptr), _lib.ptr(self._all.chunk_tensor),
                      _lib.ptr(self._all.chunk_start), _lib.ptr(self._all.numels),
                      self._all.n_chunks, CHUNK, code, _lib.ptr(self._partial),
                      _lib.ptr(self._norm), _lib.stream_handle(self._device))
        self.last_grad_norm = self._norm[0]
        self._norm_ready = True
        return self._norm[0], grads

    @torch.no_grad()
    def step(self, closure=None):
        loss = closure() if closure is not None else None
        self._check_tables()
        if self._bound_engine() is not None and not self._has_grads():
            # no gradients since zero_grad: nothing to update (torch's AdamW
            # skips parameters whose .grad is None)
            return loss
        norm_ptr = None
        if self.max_grad_norm is not None:
            if not self._norm_ready:
                self.grad_norm()
            norm_ptr = _lib.ptr(self._norm)
        self._norm_ready = False
        for group, table in zip(self.param_groups, self._tables):
            if table is None:
                continue
            ps = group["params"]
            grads, gcode = self._grads(ps)
            steps = {self.state[p]["step"] for p in ps}
            if len(steps) != 1:
                raise RuntimeError("parameters of one group must share their step count")
            step = steps.pop() + 1
            for p in ps:
                self.state[p]["step"] = step
            gptr = _Table.pointers(grads, self._device)
            beta1, beta2 = group["betas"]
            _lib.call("alodlm_adamw", _lib.ptr(table.params), _lib.ptr(table.master),
                      _lib.ptr(table.m), _lib.ptr(table.v), _lib.ptr(gptr),
                      _lib.ptr(table.chunk_tensor), _lib.ptr(table.chunk_start),
                      _lib.ptr(table.numels), _lib.ptr(table.wd), table.n_chunks, CHUNK,
                      norm_ptr, float(self.max_grad_norm or 0.0), float(group["lr"]),
                      float(beta1), float(beta2), float(group["eps"]), step, self._code, gcode,
                      _lib.stream_handle(self._device))
        return loss


def param_groups(model, weight_decay):
    """The reference's two groups (alodlm/train.py:42-48): names containing
    'bias', 'LayerNorm.weight' or 'layer_norm.weight' are not decayed."""
    no_decay = ("bias", "LayerNorm.weight", "layer_norm.weight")
    return [
        {"params": [p for n, p in model.named_parameters() if not any(s in n for s in no_decay)],
         "weight_decay": weight_decay},
        {"params": [p for n, p in model.named_parameters() if any(s in n for s in no_decay)],
         "weight_decay": 0.0},
    ]
