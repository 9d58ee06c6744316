"""The C ABI library (libflash_mlm_hip.so) loads on the host and exports exactly what
include/flash_mlm_hip.h declares, with matching struct layouts (CPU only: no kernel
launches; only argument-rejection paths that return before any HIP call)."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import REPO
from flash_mlm import _lib

HEADER = REPO / "include" / "flash_mlm_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"FMLM_API\s+[\w\s\*]+?\b(fmlm_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert {"fmlm_pack_metadata", "fmlm_pack", "fmlm_unpack", "fmlm_attn_fwd", "fmlm_tile_map",
            "fmlm_copy_segments"} <= set(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes binding"
    assert set(_lib.SIGNATURES) == set(_declared())


def test_struct_layouts_match():
    lib = _lib.load()
    assert lib.fmlm_abi_version() == _lib.ABI_VERSION
    assert lib.fmlm_attn_params_size() == ctypes.sizeof(_lib.AttnParams)
    assert lib.fmlm_pack_tensor_size() == ctypes.sizeof(_lib.PackTensor)
    assert lib.fmlm_attn_grads_size() == ctypes.sizeof(_lib.AttnGrads)


def test_argument_rejection_without_launch():
    lib = _lib.load()
    # invalid arguments return negative codes before any HIP call
    assert lib.fmlm_pack(None, 0, 2, 1, 1, 16, None, 1, 1, None) == -1
    assert lib.fmlm_pack(None, 1, 3, 1, 1, 16, None, 1, 1, None) == -2  # bad element size
    assert lib.fmlm_unpack(2, None, 0, None, 1, 1, 1, 16, None, None) == -1
    assert lib.fmlm_copy_segments(2, None, 16, 4, None, None, 16, 4, None, 1, 1, 16, None) == -1
    assert lib.fmlm_copy_segments(3, None, 16, 4, None, None, 16, 4, None, 1, 1, 16, None) == -2
    assert lib.fmlm_copy_segments(2, None, 16, 0, None, None, 16, 4, None, 1, 1, 16, None) == 0  # nothing to copy
    assert lib.fmlm_kv_append(None, 1, 2, 1, 16, 1, 4, 4, None, None, None, None) == -1
    assert lib.fmlm_kv_append(None, 1, 3, 1, 16, 1, 4, 4, None, None, None, None) == -2  # bad element size
    # a launch reads cu_old / cu_new up to index C, so null offsets are rejected even when
    # C == 0 (the tail slice reads index 0); nothing to move and no cu_out is accepted
    t = (_lib.AppendTensor * 1)()
    t[0].old = t[0].add = t[0].out = 256
    assert lib.fmlm_kv_append(t, 1, 2, 1, 16, 0, 4, 4, None, None, None, None) == -1
    assert lib.fmlm_kv_append(t, 1, 2, 1, 16, 0, 4, 4, None, 256, None, None) == -1
    assert lib.fmlm_kv_append(t, 1, 2, 1, 16, 0, 4, 4, 256, None, None, None) == -1
    assert lib.fmlm_kv_append(t, 1, 2, 0, 16, 0, 4, 4, None, None, None, None) == 0  # no heads, no offsets out
    assert lib.fmlm_pack_metadata(None, 0, 1, 4, 0, None, None, None, None, None, None) == -1
    assert lib.fmlm_tile_map(None, 1, 4, 0, None, None, None, None) == -1
    assert lib.fmlm_attn_fwd(None, None) == -1
    assert lib.fmlm_attn_fwd_noalloc(None, None) == -1
    p = _lib.AttnParams()
    p.dtype, p.B, p.H, p.D, p.N = _lib.DTYPE_BF16, 1, 1, 48, 4
    assert lib.fmlm_attn_workspace_bytes(p) == -3  # unsupported head dim
    p.D = 64
    assert lib.fmlm_attn_workspace_bytes(p) == 0  # dense: no schedule workspace
    p.dtype = 7
    assert lib.fmlm_attn_workspace_bytes(p) == -2
    # backward: argument checks return before any HIP call
    assert lib.fmlm_attn_bwd(None, None, None) == -1
    g = _lib.AttnGrads()
    p.dtype, p.D, p.total_q = _lib.DTYPE_BF16, 48, 4
    p.q = p.o = p.k = p.v = 256
    g.dout = g.dq = g.dk = g.dv = 256
    assert lib.fmlm_attn_bwd(p, g, None) == -3  # head dim without a backward kernel
    p.D = 64
    p.dtype = 7
    assert lib.fmlm_attn_bwd(p, g, None) == -2
    p.dtype = _lib.DTYPE_F32  # SIMT kernels: accepted, then the missing workspace is reported
    assert lib.fmlm_attn_bwd(p, g, None) == -5
    p.dtype = _lib.DTYPE_BF16
    assert lib.fmlm_attn_bwd(p, g, None) == -5  # no workspace
    # 2 floats per (head, row), the tile tables (ints), then a 64-byte record per unit of
    # either grid, counted at the smallest unit of 16 rows: total_q / 16 + B query units
    # and as many main-key units (no context here)
    def bwd_bytes(H, T, B=1):
        tables = 2 * H * T * 4 + 4 * (B + 2 * (B + 1) + 1 + 1)
        units = 2 * (T // 16 + B)
        return ((tables + 63) // 64 * 64 + units * 64 + 255) // 256 * 256
    assert lib.fmlm_attn_bwd_workspace_bytes(p) == bwd_bytes(1, 4) == 256
    p.H, p.total_q = 8, 4096
    assert lib.fmlm_attn_bwd_workspace_bytes(p) == bwd_bytes(8, 4096)
    p.q = 264  # not 16-byte aligned
    assert lib.fmlm_attn_bwd(p, g, None) == -4
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(-1, "x")
