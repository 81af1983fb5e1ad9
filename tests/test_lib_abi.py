"""C-ABI checks that need no GPU: the library loads, exports every entry point declared
in include/sinkattn.h with the ctypes signature the binding uses, and rejects invalid
arguments with a negative status and a message (validation runs before any launch)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sinkattn.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sinkattn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from sinkattn_amd import _lib
    return _lib.load_library()


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("sinkattn_block_sparse_plan", "sinkattn_block_sparse_fwd", "sinkattn_block_mass_pool",
              "sinkattn_max_pool", "sinkattn_max_pool_workspace_bytes", "sinkattn_mean_pool_scores", "sinkattn_coverage_mask",
              "sinkattn_last_error", "sinkattn_abi_version"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    from sinkattn_amd import _lib
    so = _lib.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (sinkattn_[a-z0-9_]+)", out))
    for name in _declared():
        assert name in exported, name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        getattr(lib, name)


def test_header_compiles_as_c_and_cpp(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "sinkattn.h"\nint main(void) { return sinkattn_abi_version() < 0; }\n')
    for cc in ("gcc", "g++"):
        subprocess.run([cc, "-fsyntax-only", f"-I{ROOT / 'include'}", "-x", "c" if cc == "gcc" else "c++", str(src)],
                       check=True)


def _err(lib):
    return lib.sinkattn_last_error().decode()


def _i64x4(*v):
    return (ctypes.c_int64 * 4)(*v)


def test_fwd_rejects_bad_arguments(lib):
    s = _i64x4(0, 0, 128, 1)
    args = [None, None, None, 0, 1, 1, 128, 128, 96, s, s, s, None, s, None, None, None, None, 1, 1, 1.0, None]
    assert lib.sinkattn_block_sparse_fwd(*args) < 0
    assert "head dim" in _err(lib)
    args[8] = 128
    args[3] = 7
    assert lib.sinkattn_block_sparse_fwd(*args) < 0 and "dtype" in _err(lib)
    args[3] = 0
    args[18] = 3  # wrong nqb for Nq=128
    assert lib.sinkattn_block_sparse_fwd(*args) < 0 and "plan" in _err(lib)


def test_fwd_rejects_unaligned_or_strided_operands(lib):
    bad = _i64x4(0, 0, 128, 2)
    args = [16, 16, 16, 0, 1, 1, 128, 128, 128, bad, bad, bad, 16, bad, None, 16, 16, None, 1, 1, 1.0, None]
    assert lib.sinkattn_block_sparse_fwd(*args) < 0 and "innermost stride" in _err(lib)
    ok = _i64x4(0, 0, 128, 1)
    args[9:12] = [ok, ok, ok]
    args[13] = ok
    args[0] = 18  # not 16-byte aligned
    assert lib.sinkattn_block_sparse_fwd(*args) < 0 and "aligned" in _err(lib)


def test_pool_and_mask_validation(lib):
    s = _i64x4(0, 0, 128, 1)
    assert lib.sinkattn_block_mass_pool(16, 16, 0, 1, 1, 128, 128, 128, s, s, 0, 1.0, 16, 16, None) < 0
    assert "block_size" in _err(lib)
    # head dims above 256 only on the block-128 / head-dim-128 kernels' shapes
    s512 = _i64x4(0, 0, 512, 1)
    assert lib.sinkattn_block_mass_pool(16, 16, 0, 1, 1, 128, 128, 512, s512, s512, 64, 1.0, 16, 16, None) < 0
    assert "256" in _err(lib)
    # the generic kernels' LDS bounds the key-block count at a given head dim
    assert lib.sinkattn_block_mass_pool(16, 16, 0, 1, 1, 16, 16 * 25000, 256, _i64x4(0, 0, 256, 1),
                                        _i64x4(0, 0, 256, 1), 16, 1.0, 16, 16, None) < 0
    assert "LDS" in _err(lib)
    # max-pool keeps the reference's asserts on block size and head dim
    assert lib.sinkattn_max_pool(16, 16, 2, 1, 1, 1, 128, 128, s, s, 48, 1.0, 0, 16, 16, None) < 0
    assert "block_size" in _err(lib)
    s96 = _i64x4(0, 0, 96, 1)
    assert lib.sinkattn_max_pool(16, 16, 0, 1, 1, 1, 128, 96, s96, s96, 64, 1.0, 0, 16, 16, None) < 0
    assert "head dim" in _err(lib)
    assert lib.sinkattn_max_pool(16, 16, 0, 1, 4, 3, 128, 128, s, s, 128, 1.0, 0, 16, 16, None) < 0
    assert "multiple" in _err(lib)
    assert lib.sinkattn_coverage_mask(16, 1, 1, 5000, 0.85, 1, 0, 0, 0, 0, 16, None, None, 16, None) < 0
    assert "4096" in _err(lib)
    assert lib.sinkattn_coverage_mask(16, 1, 1, 8, 0.85, 1, 0, 0, 5, 0, 16, None, None, 16, None) < 0
    assert "mode" in _err(lib)
    # empty problems are no-ops
    assert lib.sinkattn_coverage_mask(None, 0, 4, 4, 0.85, 1, 0, 0, 0, 0, None, None, None, None, None) == 0
    assert lib.sinkattn_block_sparse_plan(None, s, 0, 1, 1, 1, None, None, None, None) == 0


def test_workspace_queries(lib):
    assert lib.sinkattn_mean_pool_workspace_bytes(2, 12, 32760, 32760, 128, 128) == 2 * 12 * 512 * 128 * 4
    assert lib.sinkattn_coverage_mask_workspace_bytes(12, 256) == 12 * 256
    assert lib.sinkattn_coverage_mask_workspace_bytes(1, 3) == 256
    assert lib.sinkattn_block_mass_pool_workspace_bytes(1, 12, 4096, 4096, 128, 2) == 0
    assert lib.sinkattn_block_mass_pool_workspace_bytes(2, 12, 32760, 32760, 128, 0) % (256 * 512) == 0
    assert lib.sinkattn_abi_version() >= 1


def test_fwd_rejects_heads_past_the_32bit_copy_range(lib):
    # K/V tiles are copied through buffer descriptors with a 32-bit byte range: one head of
    # k/v (and of the compensation kd/vd) must stay under 2 GiB.
    nk = 1 << 20
    sq, sk = _i64x4(0, 0, 128, 1), _i64x4(0, 0, 1536, 1)
    args = [16, 16, 16, 0, 1, 1, 128, nk, 128, sq, sk, sk, 16, sq, None, 16, 16, None, 1, nk // 128, 1.0, None]
    assert lib.sinkattn_block_sparse_fwd(*args) < 0 and "2 GiB" in _err(lib)
    comp = [16, 16, 16, 0, 1, 1, 128, 128, 128, sq, sk, sk, 16, 16, sk, sk, nk, 1, 1.0,
            16, sq, None, 16, 16, None, 1, 1, 1.0, None]
    assert lib.sinkattn_block_sparse_fwd_comp(*comp) < 0 and "kd or vd" in _err(lib)
