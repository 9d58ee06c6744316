"""Numpy restatement of the reference's pack metadata / pack / pad / unpack.

Test infrastructure only (see oracle/__init__.py).  Every function cites the
reference function it restates (paths relative to the flash-mlm repository).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class MetaRef:
    B: int
    N: int
    lengths: np.ndarray  # int32 [B]
    cu_seqlens: np.ndarray  # int32 [B+1]
    token_indices: np.ndarray  # int64 [T]
    total_tokens: int
    block_n: int
    batch_ids: np.ndarray  # int32 [tiles]
    tile_starts: np.ndarray  # int32 [tiles]


def tile_map(cu_seqlens, block_n: int) -> tuple[np.ndarray, np.ndarray]:
    """(tile_starts, batch_ids) -- _build_query_tile_map_from_cu_seqlens,
    src/flash_mlm/host/host_utils.py:74-107."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    if cu.ndim != 1:
        raise ValueError("cu_seqlens_q must be rank-1")
    if cu.size < 2:
        raise ValueError("cu_seqlens_q must have at least 2 elements")
    if block_n < 1:
        raise ValueError("block_n must be >= 1")
    lengths = cu[1:] - cu[:-1]
    tiles = (lengths + block_n - 1) // block_n
    batch_ids = np.repeat(np.arange(lengths.size, dtype=np.int64), tiles)
    first_tile = np.cumsum(tiles) - tiles
    local = np.arange(batch_ids.size, dtype=np.int64) - np.repeat(first_tile, tiles)
    starts = cu[:-1][batch_ids] + local * block_n
    return starts.astype(np.int32), batch_ids.astype(np.int32)


def pack_metadata(lengths, N: int, block_n: int) -> MetaRef:
    """build_pack_metadata, src/flash_mlm/host/host_utils.py:27-71."""
    L = np.asarray(lengths)
    if L.ndim != 1:
        raise ValueError("lengths must be rank-1 [B]")
    if N < 0:
        raise ValueError("N must be >= 0")
    if block_n < 1:
        raise ValueError("block_n must be >= 1")
    if np.any(L < 0) or np.any(L > N):
        raise ValueError("lengths values must be in [0, N]")
    L = L.astype(np.int32)
    B = int(L.size)
    cu = np.zeros(B + 1, dtype=np.int32)
    cu[1:] = np.cumsum(L, dtype=np.int64).astype(np.int32)
    pos = np.arange(N, dtype=np.int64)[None, :]
    valid = pos < L[:, None]
    flat = np.arange(B, dtype=np.int64)[:, None] * N + pos
    token_indices = flat[valid].astype(np.int64)
    starts, bids = tile_map(cu, block_n)
    return MetaRef(B, N, L, cu, token_indices, int(cu[-1]), block_n, bids, starts)


def total_q_len_padded(total_q_len_unpadded: int, cu_seqlens, block_m: int, block_n: int) -> int:
    """_compute_total_q_len_padded, src/flash_mlm/host/host_utils.py:292-312."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    a = max(block_m, block_n)
    lengths = cu[1:] - cu[:-1]
    ends = cu[:-1] + ((lengths + a - 1) // a) * a
    required = int(ends.max()) if ends.size else 0
    return max(int(total_q_len_unpadded), required)


def pack(x: np.ndarray, meta: MetaRef, total_padded: int | None = None) -> np.ndarray:
    """[B, H, N, D] -> head-major [H*T_pad, D], rows T..T_pad of each head zero --
    pack_for_kernel / _pack_flatten_for_kernel_into, host_utils.py:266-289, 397-420."""
    B, H, N, D = x.shape
    if B != meta.B or N != meta.N:
        raise ValueError("x shape mismatch with PackMetadata")
    T = meta.total_tokens
    T_pad = T if total_padded is None else int(total_padded)
    x_hbn = np.transpose(x, (1, 0, 2, 3)).reshape(H, B * N, D)
    out = np.zeros((H, T_pad, D), dtype=x.dtype)
    out[:, :T] = x_hbn[:, meta.token_indices]
    return out.reshape(H * T_pad, D)


def pad_packed(x: np.ndarray, heads: int, T: int, T_pad: int) -> np.ndarray:
    """[heads*T, D] -> [heads*T_pad, D] with zero tails -- pad_packed_main_tensors_for_mlm_compressed,
    host_utils.py:494-584 (one tensor)."""
    D = x.shape[1]
    out = np.zeros((heads, T_pad, D), dtype=x.dtype)
    out[:, :T] = x.reshape(heads, T, D)
    return out.reshape(heads * T_pad, D)


def unpack(packed: np.ndarray, meta: MetaRef, H: int) -> np.ndarray:
    """[H*T, D] or [H, T, D] -> [B, H, N, D] with zeros at padding --
    unpack_from_kernel, host_utils.py:587-615."""
    T = meta.total_tokens
    D = packed.shape[-1]
    p = packed.reshape(H, T, D)
    x = np.zeros((H, meta.B * meta.N, D), dtype=packed.dtype)
    x[:, meta.token_indices] = p
    return np.transpose(x.reshape(H, meta.B, meta.N, D), (1, 0, 2, 3)).copy()


def append_segments(old: np.ndarray, cu_old, new: np.ndarray, cu_new, heads: int):
    """KV append (an extension with no reference counterpart; the reference's roadmap
    lists appends with paged KV, README.md:34-41): head-major caches old [heads*T_old, D]
    and new [heads*T_new, D] with per-batch offsets cu_old / cu_new -> (merged
    [heads*(T_old+T_new), D], cu_out) where batch c of every head holds its old rows then
    its new rows, cu_out = cu_old + cu_new.  Rows past cu_out[-1] of every head are zero,
    like the zero padding rows of a prefilled packed entry."""
    cu_old = np.asarray(cu_old, dtype=np.int64)
    cu_new = np.asarray(cu_new, dtype=np.int64)
    D = old.shape[1]
    t_old, t_new = old.shape[0] // heads, new.shape[0] // heads
    rows = t_old + t_new
    out = np.zeros((heads * rows, D), dtype=old.dtype)
    for h in range(heads):
        r = h * rows
        for c in range(len(cu_old) - 1):
            seg_old = old[h * t_old + cu_old[c] : h * t_old + cu_old[c + 1]]
            seg_new = new[h * t_new + cu_new[c] : h * t_new + cu_new[c + 1]]
            out[r : r + len(seg_old)] = seg_old
            r += len(seg_old)
            out[r : r + len(seg_new)] = seg_new
            r += len(seg_new)
    return out, cu_old + cu_new


def gather_pages(pool: np.ndarray, block_table, lengths):
    """Paged context (an extension; the reference's roadmap lists paged KV, README.md:41)
    -> contiguous head-major cache: pool [P, H_kv, page_rows, D]; batch c's key j is row
    j % page_rows of page block_table[c][j // page_rows].  Returns (cache [H_kv*T, D],
    cu [C+1]) with batch c at rows cu[c]..cu[c+1] of every head."""
    P, H, R, D = pool.shape
    lengths = [int(x) for x in lengths]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    T = int(cu[-1])
    out = np.zeros((H * T, D), dtype=pool.dtype)
    for c, n in enumerate(lengths):
        for j in range(n):
            page = int(block_table[c][j // R])
            out[np.arange(H) * T + cu[c] + j] = pool[page, :, j % R]
    return out, cu
