"""ctypes binding of libsinkattn.so (C ABI declared in include/sinkattn.h).

The library is built in-tree by ``python -m sinkattn_amd.build``.  Loading it needs the
HIP runtime that torch already loaded (same soname), so torch is imported first.  There
is no fallback: if the library is missing or no GPU is present, every kernel entry point
raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence

import torch

LIB_PATH = Path(os.environ.get("SINKATTN_LIB", Path(__file__).resolve().parent / "libsinkattn.so"))

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_i64_4 = ctypes.c_int64 * 4
_c_i64_3 = ctypes.c_int64 * 3

# name -> (restype, argtypes); must match include/sinkattn.h
SIGNATURES = {
    "sinkattn_last_error": (ctypes.c_char_p, []),
    "sinkattn_abi_version": (ctypes.c_int, []),
    "sinkattn_block_sparse_order_slots": (ctypes.c_int64, [_c_i64, _c_i64, _c_i64]),
    "sinkattn_block_sparse_plan": (
        ctypes.c_int,
        [_c_p, _c_i64_4, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p],
    ),
    "sinkattn_block_sparse_order_cache_ints": (ctypes.c_int64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "sinkattn_block_sparse_plan_cached": (
        ctypes.c_int,
        [_c_p, _c_i64_4, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sinkattn_block_sparse_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64_4, _c_i64_4, _c_i64_4, _c_p, _c_i64_4, _c_p, _c_p, _c_p, _c_p,
         _c_i64, _c_i64, ctypes.c_float, _c_p],
    ),
    "sinkattn_block_sparse_fwd_comp": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64_4, _c_i64_4, _c_i64_4, _c_p, _c_p, _c_i64_4, _c_i64_4, _c_i64, _c_i64, ctypes.c_float,
         _c_p, _c_i64_4, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, ctypes.c_float, _c_p],
    ),
    "sinkattn_mean_pool_tokens_rows": (ctypes.c_int64, [_c_i64, _c_i64, _c_i64]),
    "sinkattn_mean_pool_tokens": (
        ctypes.c_int,
        [_c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64_4, _c_i64, _c_i64, _c_p, _c_i64_4, _c_p],
    ),
    "sinkattn_qk_norm_rotary": (
        ctypes.c_int,
        [_c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, ctypes.c_float, ctypes.c_float,
         _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sinkattn_lse_mix": (
        ctypes.c_int,
        [_c_p, _c_i64_4, _c_p, _c_i64_3, _c_p, _c_i64_4, _c_p, _c_i64_3, ctypes.c_int, _c_i64, _c_i64,
         _c_i64, _c_i64, ctypes.c_float, _c_p, _c_i64_4, _c_p],
    ),
    "sinkattn_block_mass_pool_workspace_bytes": (
        ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int],
    ),
    "sinkattn_block_mass_pool": (
        ctypes.c_int,
        [_c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64_4, _c_i64_4,
         _c_i64, ctypes.c_float, _c_p, _c_p, _c_p],
    ),
    "sinkattn_max_pool_workspace_bytes": (
        ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int],
    ),
    "sinkattn_max_pool": (
        ctypes.c_int,
        [_c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64_4, _c_i64_4,
         _c_i64, ctypes.c_float, ctypes.c_int, _c_p, _c_p, _c_p],
    ),
    "sinkattn_mean_pool_workspace_bytes": (
        ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64],
    ),
    "sinkattn_mean_pool_scores": (
        ctypes.c_int,
        [_c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64_4, _c_i64_4,
         _c_i64, ctypes.c_float, _c_p, _c_p, _c_p],
    ),
    "sinkattn_block_sparse_attn_noalloc": (
        ctypes.c_int,
        [_c_p, _c_i64_4, _c_p, _c_p, _c_p, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64_4, _c_i64_4, _c_i64_4, _c_p, _c_i64_4, _c_p, ctypes.c_float, _c_p],
    ),
    "sinkattn_coverage_mask_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "sinkattn_coverage_mask": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int, _c_i64, _c_i64,
         ctypes.c_int, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p],
    ),
}

_LIB: Optional[ctypes.CDLL] = None


class SinkAttnError(RuntimeError):
    """A libsinkattn entry point returned a non-zero status."""


# Version of the entry-point signatures declared in include/sinkattn.h (raised whenever an
# existing signature changes).
ABI_VERSION = 4


def load_library() -> ctypes.CDLL:
    """Load libsinkattn.so and declare its signatures (no GPU needed)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            f"libsinkattn.so is not built ({LIB_PATH}); run `python -m sinkattn_amd.build`."
        )
    lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as exc:
            raise ImportError(f"{LIB_PATH} lacks {name}: it predates this source tree; rebuild it with "
                              "`python -m sinkattn_amd.build`") from exc
        fn.restype = res
        fn.argtypes = args
    if lib.sinkattn_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI version {lib.sinkattn_abi_version()}, this source tree "
                          f"expects {ABI_VERSION}; rebuild it with `python -m sinkattn_amd.build`")
    _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    """The library, checked to be usable for compute on the current process."""
    l = load_library()
    if not torch.cuda.is_available():
        raise RuntimeError("libsinkattn kernels need a ROCm GPU (torch.cuda.is_available() is False)")
    return l


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load_library().sinkattn_last_error().decode(errors="replace")
        if status < 0:
            raise ValueError(f"{what}: {msg}")
        raise SinkAttnError(f"{what}: HIP error {status}: {msg}")


def stream_ptr(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def strides4(t: torch.Tensor) -> "ctypes.Array":
    s: Sequence[int] = t.stride()
    return _c_i64_4(*[int(x) for x in s])


def strides3(t: torch.Tensor) -> "ctypes.Array":
    s: Sequence[int] = t.stride()
    return _c_i64_3(*[int(x) for x in s])


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in DTYPE_CODES:
        raise TypeError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32")
    return DTYPE_CODES[dtype]
