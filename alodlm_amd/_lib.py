"""ctypes binding of ``libalodlm_hip.so`` (the C ABI in include/alodlm_hip.h).

The library is mandatory: importing a compute entry point without it raises
immediately.  There is no CPU fallback.  Return codes map to exceptions:
ALODLM_EINVAL -> ValueError, anything else -> RuntimeError.
"""

import ctypes
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "libalodlm_hip.so"
ABI_VERSION = 7

P = ctypes.c_void_p
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
I32 = ctypes.c_int
F32 = ctypes.c_float

F32_CODE, BF16_CODE = 0, 1
EPI_STORE, EPI_RESIDUAL, EPI_ACCUM, EPI_STORE_F32 = 0, 1, 2, 3

# name -> argument types (every entry point returns int unless listed in _RESTYPE)
SIGNATURES = {
    "alodlm_abi_version": [],
    "alodlm_device_info": [I32, P, P],
    "alodlm_last_error": [],
    "alodlm_mask_draws": [U64, U64, P, I64, P, I64, I64, P, P, P, P, P, P, P, P],
    "alodlm_batch_build": [P, P, P, P, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, P, P, P],
    "alodlm_embed_gather": [P, P, P, I64, I64, I64, I32, P],
    "alodlm_embed_plan": [P, I64, I64, P, P],
    "alodlm_embed_scatter_add": [P, P, P, I64, P, P, I64, I64, I64, I32, P],
    "alodlm_rmsnorm_fwd": [P, P, P, P, I64, I64, F32, I32, P],
    "alodlm_rmsnorm_bwd_workspace": [I64, I64],
    "alodlm_embed_plan_size": [I64],
    "alodlm_embed_scatter_workspace": [I64, I64],
    "alodlm_carry_select_bwd_workspace": [I64, I64],
    "alodlm_rmsnorm_bwd": [P, P, P, P, P, P, P, P, I64, I64, I32, P],
    "alodlm_rmsnorm_bwd_noalloc": [P, P, P, P, P, P, P, I64, I64, I32, P],
    "alodlm_qknorm_rope_fwd": [P, P, P, P, P, P, P, I64, I64, I64, I64, F32, I32, P],
    "alodlm_qknorm_rope_bwd_workspace": [I64, I64, I64, I64],
    "alodlm_qknorm_rope_bwd": [P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, F32, I32, P],
    "alodlm_qknorm_rotary_fwd": [P, P, P, P, P, P, P, I64, I64, I64, I64, F32, I32, P],
    "alodlm_qknorm_rotary_bwd": [P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, F32, I32,
                                 P],
    "alodlm_rotary_fwd": [P, P, P, P, I64, I64, I64, I32, P],
    "alodlm_rotary_bwd": [P, P, P, P, I64, I64, I64, I32, P],
    "alodlm_gemm_workspace": [I64, I64, I64, I32, I32],
    "alodlm_gemm": [P, I64, I32, P, I64, I32, P, I64, P, I64, I64, I64, I64, F32, I32, I32, P, P],
    "alodlm_gemm_segk": [P, P, I32, I64, I64, I64, P, I64, I64, I64, F32, I32, P, P],
    "alodlm_attention_fwd": [P, P, P, I64, P, P, P, I64, P, P, I64, I64, I64, I64, I64, I32, P],
    "alodlm_attention_ds_blocks": [P, I64, I64, P],
    "alodlm_attention_bwd_workspace": [I64, I64, I64, I64, I64, I64],
    "alodlm_attention_bwd": [P, P, P, I64, P, P, P, P, P, P, I64, P, P, P, I64, P, P, I64, I64,
                             I64, I64, I64, I64, I32, P],
    "alodlm_swiglu_fwd": [P, P, I64, I64, I32, P],
    "alodlm_swiglu_bwd": [P, P, P, P, I64, I64, I32, P],
    "alodlm_final_norm_gate": [P, P, P, P, P, I64, P, P, P, I64, I64, F32, I32, P],
    "alodlm_carry_select": [P, P, P, P, P, I64, P, P, I64, I64, I64, F32, I32, P],
    "alodlm_carry_select_bwd": [P, P, P, P, P, I64, P, P, P, P, P, P, I64, I64, I64, I32, P],
    "alodlm_exit_update": [P, P, P, P, I64, I64, I64, P],
    "alodlm_select_rows": [P, P, P, P, P, P, P, F32, I64, I64, I64, P, P, P, P, P],
    "alodlm_inverse_weight_sum": [P, P, I64, P, P],
    "alodlm_gather_rows": [P, P, I64, P, I64, I32, P],
    "alodlm_scatter_rows": [P, P, I64, P, I64, I64, I32, P],
    "alodlm_cross_entropy": [P, P, P, P, I64, I64, P, P, I32, P],
    "alodlm_scatter_ce": [P, P, P, I64, P, I64, P],
    "alodlm_decode_readout": [P, I64, I64, P, P, I32, P],
    "alodlm_decode_plan": [P, P],
    "alodlm_decode_begin": [P, P, I64, I64, P],
    "alodlm_decode_commit": [P, P, I64, I64, I32, P],
    "alodlm_objective_workspace": [I64, I64, I64],
    "alodlm_objective": [P, P, P, P, P, P, P, P, I64, I64, I64, F32, F32, F32, P, P, P, P, P],
    "alodlm_outcome_loss": [P, P, P, P, P, P, I64, I64, I64, F32, F32, F32, P, P, P, P, P],
    "alodlm_masked_sequence_ids": [P, P, I64, I64, P, P, P],
    "alodlm_sequence_score": [P, P, P, I64, I64, P, P, P, P],
    "alodlm_ar_targets": [P, P, I64, I64, P, P],
    "alodlm_gate_bwd_workspace": [I64, I64],
    "alodlm_gate_bwd": [P, P, F32, P, P, P, I64, I64, I64, P, I32, P],
    "alodlm_grad_norm": [P, P, P, P, I64, I64, I32, P, P, P],
    "alodlm_adamw": [P, P, P, P, P, P, P, P, P, I64, I64, P, F32, F32, F32, F32, F32, I64, I32, I32,
                     P],
    "alodlm_cast_f32": [P, P, P, I64, I32, P],
    "alodlm_scale_f32": [P, P, I64, P],
    "alodlm_scale": [P, P, I64, I32, P],
    "alodlm_scale_add_f32": [P, P, I64, P, I32, P],
    "alodlm_transpose": [P, P, I64, I64, I32, P],
    "alodlm_check_finite": [P, I64, I32, P, P],
}
_RESTYPE = {
    "alodlm_last_error": ctypes.c_char_p,
    "alodlm_rmsnorm_bwd_workspace": I64,
    "alodlm_embed_plan_size": I64,
    "alodlm_embed_scatter_workspace": I64,
    "alodlm_carry_select_bwd_workspace": I64,
    "alodlm_qknorm_rope_bwd_workspace": I64,
    "alodlm_gemm_workspace": I64,
    "alodlm_attention_bwd_workspace": I64,
    "alodlm_attention_ds_blocks": I64,
    "alodlm_objective_workspace": I64,
    "alodlm_gate_bwd_workspace": I64,
}

_lib = None


class LibraryMissing(RuntimeError):
    """Raised when the HIP library has not been built."""


def load():
    """Load the library once (raises LibraryMissing if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise LibraryMissing(
            f"{LIBRARY} is missing: build it with `python -m alodlm_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(str(LIBRARY))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, I32)
    if lib.alodlm_abi_version() != ABI_VERSION:
        raise LibraryMissing(f"{LIBRARY} has ABI {lib.alodlm_abi_version()}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(device=None):
    return torch.cuda.current_stream(device).cuda_stream


def call(name, *args):
    """Invoke an int-returning entry point and raise on a nonzero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.alodlm_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def query(name, *args):
    """Invoke a size-query entry point."""
    return getattr(load(), name)(*args)


def dtype_code(dtype):
    if dtype == torch.float32:
        return F32_CODE
    if dtype == torch.bfloat16:
        return BF16_CODE
    raise ValueError(f"unsupported dtype {dtype}: the HIP kernels take float32 or bfloat16")
