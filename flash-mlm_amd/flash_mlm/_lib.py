"""ctypes binding of libflash_mlm_hip.so, the C ABI declared in include/flash_mlm_hip.h.

The library is the only compute path of this package: if it is missing or fails
to load, every compute entry point raises.  There is no CPU or torch fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libflash_mlm_hip.so"
_LIB_PATH = Path(os.environ.get("FMLM_LIB_PATH", Path(__file__).resolve().parent / "_native" / LIB_NAME))

ABI_VERSION = 5

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

FLAG_MLA = 1
FLAG_PREFILL = 2
FLAG_CAUSAL_SEQ = 4

LAYOUT_PADDED = 0
LAYOUT_PACKED = 1

_ERRORS = {
    -1: "invalid argument",
    -2: "unsupported dtype",
    -3: "unsupported head dimension",
    -4: "pointer or stride not aligned to the element size",
    -5: "workspace missing or too small",
}

_TORCH_DTYPES = {
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.float32: DTYPE_F32,
}

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p


class AttnParams(ctypes.Structure):
    """Mirror of fmlm_attn_params (include/flash_mlm_hip.h)."""

    _fields_ = [
        ("dtype", _c_i32),
        ("flags", _c_i32),
        ("B", _c_i32),
        ("H", _c_i32),
        ("D", _c_i32),
        ("N", _c_i32),
        ("total_q", _c_i32),
        ("ctx_len", _c_i32),
        ("ctx_batch", _c_i32),
        ("ctx_rows", _c_i32),
        ("q_layout", _c_i32),
        ("o_layout", _c_i32),
        ("kv_layout", _c_i32),
        ("scale", ctypes.c_float),
        ("cu_seqlens_q", _c_ptr),
        ("cu_seqlens_kv", _c_ptr),
        ("q", _c_ptr),
        ("q_sb", _c_i64),
        ("q_sh", _c_i64),
        ("q_sn", _c_i64),
        ("o", _c_ptr),
        ("o_sb", _c_i64),
        ("o_sh", _c_i64),
        ("o_sn", _c_i64),
        ("k", _c_ptr),
        ("k_sb", _c_i64),
        ("k_sh", _c_i64),
        ("k_sn", _c_i64),
        ("v", _c_ptr),
        ("v_sb", _c_i64),
        ("v_sh", _c_i64),
        ("v_sn", _c_i64),
        ("k_ctx", _c_ptr),
        ("v_ctx", _c_ptr),
        ("c_sb", _c_i64),
        ("c_sh", _c_i64),
        ("c_sn", _c_i64),
        ("workspace", _c_ptr),
        ("workspace_bytes", _c_i64),
        ("schedule", _c_ptr),
        ("ctx_index", _c_ptr),
        ("ctx_block_table", _c_ptr),
        ("ctx_page_stride", _c_i64),
        ("ctx_pages_per_batch", _c_i32),
        ("tile_config", _c_i32),
        ("lse", _c_ptr),
    ]


class AppendTensor(ctypes.Structure):
    """Mirror of fmlm_append_tensor (include/flash_mlm_hip.h)."""

    _fields_ = [("old", _c_ptr), ("add", _c_ptr), ("out", _c_ptr)]


class PackTensor(ctypes.Structure):
    """Mirror of fmlm_pack_tensor (include/flash_mlm_hip.h)."""

    _fields_ = [
        ("src", _c_ptr),
        ("s_sb", _c_i64),
        ("s_sh", _c_i64),
        ("s_sn", _c_i64),
        ("dst", _c_ptr),
        ("heads", _c_i32),
        ("reserved", _c_i32),
    ]


class AttnGrads(ctypes.Structure):
    """Mirror of fmlm_attn_grads (include/flash_mlm_hip.h)."""

    _fields_ = [
        (name if s == "" else f"{pre}{s}", _c_ptr if s == "" else _c_i64)
        for name, pre in (("dout", "do"), ("dq", "dq"), ("dk", "dk"), ("dv", "dv"))
        for s in ("", "_sb", "_sh", "_sn")
    ] + [
        ("dk_ctx", _c_ptr),
        ("dv_ctx", _c_ptr),
        ("workspace", _c_ptr),
        ("workspace_bytes", _c_i64),
    ]


# (name, restype, argtypes) of every exported entry point
SIGNATURES = {
    "fmlm_abi_version": (ctypes.c_int, []),
    "fmlm_attn_params_size": (ctypes.c_int, []),
    "fmlm_pack_tensor_size": (ctypes.c_int, []),
    "fmlm_pack_metadata": (
        ctypes.c_int,
        [_c_ptr, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fmlm_tile_map": (ctypes.c_int, [_c_ptr, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr]),
    "fmlm_pack": (
        ctypes.c_int,
        [ctypes.POINTER(PackTensor), _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr, _c_i32, _c_i32, _c_ptr],
    ),
    "fmlm_unpack": (
        ctypes.c_int,
        [_c_i32, _c_ptr, _c_i64, _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr],
    ),
    "fmlm_copy_segments": (
        ctypes.c_int,
        [_c_i32, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i32, _c_i32, _c_i32, _c_ptr],
    ),
    "fmlm_kv_append": (
        ctypes.c_int,
        [ctypes.POINTER(AppendTensor), _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr,
         _c_ptr, _c_ptr],
    ),
    "fmlm_attn_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(AttnParams)]),
    "fmlm_attn_schedule": (ctypes.c_int, [ctypes.POINTER(AttnParams), _c_ptr, _c_i64, _c_ptr]),
    "fmlm_attn_fwd": (ctypes.c_int, [ctypes.POINTER(AttnParams), _c_ptr]),
    "fmlm_attn_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(AttnParams), _c_ptr]),
    "fmlm_attn_grads_size": (ctypes.c_int, []),
    "fmlm_attn_bwd_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(AttnParams)]),
    "fmlm_attn_bwd": (ctypes.c_int, [ctypes.POINTER(AttnParams), ctypes.POINTER(AttnGrads), _c_ptr]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise RuntimeError if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"flash_mlm HIP library not found at {_LIB_PATH}; build it with "
                "`python flash-mlm_amd/build_lib.py` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(str(_LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.fmlm_abi_version() != ABI_VERSION:
            raise RuntimeError("flash_mlm HIP library ABI version mismatch; rebuild it")
        if lib.fmlm_attn_params_size() != ctypes.sizeof(AttnParams):
            raise RuntimeError("fmlm_attn_params layout mismatch between library and binding")
        if lib.fmlm_pack_tensor_size() != ctypes.sizeof(PackTensor):
            raise RuntimeError("fmlm_pack_tensor layout mismatch between library and binding")
        if lib.fmlm_attn_grads_size() != ctypes.sizeof(AttnGrads):
            raise RuntimeError("fmlm_attn_grads layout mismatch between library and binding")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    if rc < 0:
        raise RuntimeError(f"{what}: {_ERRORS.get(rc, 'error')} (code {rc})")
    raise RuntimeError(f"{what}: HIP error {rc}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32") from None


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
