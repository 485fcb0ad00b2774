"""ctypes binding of ``liboxr_verify.so``, the gfx950 C-ABI library (include/oxr_verify.h).

torch is imported before the library is loaded so that the library binds to the
HIP runtime torch already mapped (same SONAME), and stream handles and device
pointers from torch are valid in both.  There is no CPU fallback: a missing
library or a non-GPU tensor raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("liboxr_verify.so")

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); kept in step with include/oxr_verify.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "oxr_abi_version": (ctypes.c_int, []),
    "oxr_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "oxr_selftest_mfma_layout": (ctypes.c_int, [_P, _P, _P, _P]),
    "oxr_ngram_propose": (ctypes.c_int, [_P, _I64, _P, _P, _I32, _I32, _I32, _P, _P, _P, _P]),
    "oxr_propose_verify_inputs": (
        ctypes.c_int,
        [_P, _I64, _P, _I32, _I32, _I32, _P, _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P, _P, _P],
    ),
    "oxr_step_record_words": (ctypes.c_size_t, [_I32, _I32, _I32]),
    "oxr_unpack_step_inputs": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P]),
    "oxr_accept": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P]),
    "oxr_paged_extend_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _I32]),
    "oxr_paged_extend": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I64, _I32, _F32, _P, _P, _SZ, _P],
    ),
    "oxr_qk_norm_rope_paged_extend": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _F32, _P, _P, _P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32,
         _I64, _I32, _F32, _P, _I32, _P, _SZ, _P],
    ),
    "oxr_paged_extend_plan_ints": (ctypes.c_size_t, [_I32, _I32, _I32, _I32, _I32]),
    "oxr_paged_extend_plan": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _SZ, _P]),
    "oxr_paged_extend_planned": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I64, _I32, _F32, _P, _P, _SZ, _P, _SZ, _P],
    ),
    "oxr_qk_norm_rope_paged_extend_planned": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _F32, _P, _P, _P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32,
         _I64, _I32, _F32, _P, _I32, _P, _SZ, _P, _SZ, _P],
    ),
    "oxr_static_scratch_bytes": (ctypes.c_size_t, []),
    "oxr_qk_norm_rope_paged_extend_static": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _F32, _P, _P, _P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32,
         _I64, _I32, _F32, _P, _I32, _P],
    ),
    "oxr_qk_norm_rope_store_at": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _P, _F32, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P, _P],
    ),
    "oxr_rms_norm": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _F32, _P, _I64, _I32, _P]),
    "oxr_embed_rms_norm": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _P, _F32, _P, _P, _I32, _P]),
    "oxr_embed_gather": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "oxr_add_partials_rms_norm": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _P, _F32, _P, _I32, _P]),
    "oxr_add_partials_rms_norm_from": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _P, _P, _F32, _P, _I32, _P]),
    "oxr_mlp_block_workspace_bytes": (ctypes.c_size_t, []),
    "oxr_mlp_block_supported": (ctypes.c_int, [_I64, _I64, _I64, _I32]),
    "oxr_mlp_block": (ctypes.c_int, [_P, _I32, _P, _I64, _I64, _I64, _P, _F32, _P, _P, _P, _P, _P, _SZ, _P]),
    "oxr_gemm_bf16": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _I32, _P, _I64, _P]),
    "oxr_gemm_bf16_partial_splits": (ctypes.c_int32, [_I64, _I64]),
    "oxr_gemm_bf16_partial": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _P, _I32, _P]),
    "oxr_lm_head_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "oxr_lm_head_argmax": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "oxr_lm_head_accept_packed": (
        ctypes.c_int,
        [_P, _I64, _P, _I64, _I64, _P, _SZ, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _I64, _P, _P,
         _P],
    ),
    "oxr_argmax_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "oxr_argmax": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _P, _P, _SZ, _P]),
    "oxr_varlen_attention": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _P]),
    "oxr_packed_weight_elems": (ctypes.c_size_t, [_I64, _I64]),
    "oxr_pack_weight_bf16": (ctypes.c_int, [_P, _I64, _I64, _P, _P]),
    "oxr_gemm_bf16_packed": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _I32, _P, _I64, _I32, _P]),
    "oxr_gemm_bf16_partial_packed": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _P, _I32, _I32, _P]),
    "oxr_lm_head_argmax_packed": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "oxr_qk_norm_rope_store": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _F32, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P, _P],
    ),
}

_lib: ctypes.CDLL | None = None


class HipLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types declared."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipLibraryMissing(
                f"{LIB_PATH} is not built; run `python oxr-inference_amd/build.py` (hipcc, gfx950). "
                "There is no CPU fallback."
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, name: str) -> None:
    if status != 0:
        message = lib().oxr_status_string(status).decode()
        raise RuntimeError(f"{name} failed: {message} (status {status})")


def call(name: str, *args) -> None:
    """Call an entry point and raise on a non-zero status."""
    check(getattr(lib(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor, name: str) -> torch.device:
    """All tensors on one GPU; raises for CPU tensors (there is no CPU path)."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must be on a GPU (got {t.device}); this build has no CPU path")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"{name}: tensors on different devices ({device} and {t.device})")
    if device is None:
        raise RuntimeError(f"{name}: no tensor arguments")
    return device


def require(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)
