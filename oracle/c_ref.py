"""TEST INFRASTRUCTURE ONLY: ctypes loader of oracle/_build/liboracle.so."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB = ORACLE_DIR / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C")
        i64p = np.ctypeslib.ndpointer(np.int64, flags="C")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C")
        L.oracle_aten_row_sum.restype = ctypes.c_float
        L.oracle_aten_row_sum.argtypes = [f32p, ctypes.c_int64]
        L.oracle_cumsum_f32.restype = None
        L.oracle_cumsum_f32.argtypes = [f32p, ctypes.c_int64, f32p]
        for name in ("oracle_std_sort_desc", "oracle_libstdcxx_sort_desc"):
            fn = getattr(L, name)
            fn.restype = None
            fn.argtypes = [f32p, i64p, ctypes.c_int64]
        L.oracle_coverage_mask.restype = None
        L.oracle_coverage_mask.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_float, ctypes.c_int, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_int, ctypes.c_int64, u8p]
        _lib = L
    return _lib


def aten_row_sum(x: np.ndarray) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(lib().oracle_aten_row_sum(x, x.size))


def cumsum_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_cumsum_f32(x, x.size, out)
    return out


def std_sort_desc(v: np.ndarray, emulated: bool = True):
    """(sorted values, permutation) of one row; emulated=False runs the real std::sort."""
    v = np.ascontiguousarray(v, dtype=np.float32).copy()
    idx = np.arange(v.size, dtype=np.int64)
    fn = lib().oracle_std_sort_desc if emulated else lib().oracle_libstdcxx_sort_desc
    fn(v, idx, v.size)
    return v, idx


def coverage_mask(scores: np.ndarray, coverage: float = 0.85, keep_diagonal: bool = True,
                  req_q: int = 0, req_k: int = 0, video_text_blocks=None) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    H, nq, nk = s.shape
    out = np.zeros((H, nq, nk), dtype=np.uint8)
    mode = 0 if video_text_blocks is None else 1
    tb = 0 if video_text_blocks is None else int(video_text_blocks)
    cov = np.float32(min(max(float(coverage), 0.0), 1.0))
    lib().oracle_coverage_mask(s, H, nq, nk, float(cov), int(bool(keep_diagonal)), int(req_q),
                               int(req_k), mode, tb, out)
    return out.astype(bool)
