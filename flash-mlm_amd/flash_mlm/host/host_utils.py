"""Host utilities of the MLM attention path: pack metadata, pack / pad / unpack,
cache-context resolution and argument validation.

Public behaviour (names, arguments, return values, ValueError messages) follows
src/flash_mlm/host/host_utils.py of the reference.  Every data-moving function runs
a HIP kernel from libflash_mlm_hip.so through the C ABI (include/flash_mlm_hip.h);
there is no CPU compute path, so these functions require device tensors.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING

import torch

from flash_mlm import _lib
from flash_mlm.host.cache import InferenceCache, PackMetadata

if TYPE_CHECKING:
    from flash_mlm.host.cache import LayerKVEntry, PackingCache

# head dims of the reference (host_utils.py:337-339); MLA additionally allows a
# 512-wide latent (one shared K=V head).
_HEAD_DIMS = (16, 32, 64, 128, 256)
_MLA_HEAD_DIMS = _HEAD_DIMS + (512,)


def _require_device(*tensors: torch.Tensor | None, what: str) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                f"{what} runs on the GPU (HIP); got a tensor on {t.device}. "
                "flash_mlm has no CPU compute path."
            )


def _device_scope(device: torch.device):
    if device.index is None or device.index == torch.cuda.current_device():
        return _NullScope()
    return torch.cuda.device(device)


class _NullScope:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


@dataclass
class CacheContext:
    """Resolved cached context for one launch (host_utils.py:17-24)."""

    k_cache: torch.Tensor
    v_cache: torch.Tensor | None
    context_batch_size: int
    context_len: int
    total_context_len: int
    cu_seqlens_kv: torch.Tensor | None
    block_table: torch.Tensor | None = None  # paged entries (extension)


# ---------------------------------------------------------------------------
# pack metadata (host_utils.py:27-130)
# ---------------------------------------------------------------------------
def build_pack_metadata(lengths: torch.Tensor, N: int, block_n: int) -> PackMetadata:
    """Indexing for a padded [B, N] batch with ``lengths[b]`` real tokens per row.

    cu_seqlens = [0, cumsum(lengths)] (int32); token_indices = b*N + t for t < L_b
    (int64, (b, t) order); query tiles of ``block_n`` rows per sequence with
    batch_ids_q[i] = b and q_tile_starts_q[i] = cu_seqlens[b] + j*block_n (int32).
    Computed by one HIP scan kernel and one fill kernel; one device->host copy
    returns the totals (the reference synchronises the same way).
    """
    if lengths.ndim != 1:
        raise ValueError("lengths must be rank-1 [B]")
    if N < 0:
        raise ValueError("N must be >= 0")
    if block_n < 1:
        raise ValueError("block_n must be >= 1")
    _require_device(lengths, what="build_pack_metadata")

    if lengths.numel() == 0:
        # the reference's tile map rejects a one-element cu_seqlens (host_utils.py:78-79)
        raise ValueError("cu_seqlens_q must have at least 2 elements")

    lib = _lib.load()
    device = lengths.device
    if lengths.dtype not in (torch.int32, torch.int64):
        lengths = lengths.to(torch.int64)
    lengths = lengths.contiguous()
    B = int(lengths.numel())
    n_tile_cap = B * ((N + block_n - 1) // block_n)
    lengths_i32 = torch.empty(B, dtype=torch.int32, device=device)
    aux = torch.empty(2 * B + 6, dtype=torch.int32, device=device)
    token_indices = torch.empty(B * N, dtype=torch.int64, device=device)
    tiles = torch.empty(2 * n_tile_cap, dtype=torch.int32, device=device)
    batch_ids_buf = tiles[:n_tile_cap]
    tile_starts_buf = tiles[n_tile_cap:]
    with _device_scope(device):
        rc = lib.fmlm_pack_metadata(
            _lib.ptr(lengths),
            int(lengths.dtype == torch.int64),
            B,
            int(N),
            int(block_n),
            _lib.ptr(lengths_i32),
            _lib.ptr(aux),
            _lib.ptr(token_indices),
            _lib.ptr(batch_ids_buf),
            _lib.ptr(tile_starts_buf),
            _lib.stream_of(device),
        )
    _lib.check(rc, "fmlm_pack_metadata")
    host = aux[: B + 5].to("cpu").tolist()
    total_tokens, n_tiles, n_bad = host[B + 1], host[B + 2], host[B + 3]
    if n_bad:
        raise ValueError("lengths values must be in [0, N]")
    return PackMetadata(
        B=B,
        N=int(N),
        lengths=lengths_i32,
        cu_seqlens=aux[: B + 1],
        token_indices=token_indices[:total_tokens],
        total_tokens=int(total_tokens),
        batch_ids_block_n=int(block_n),
        batch_ids_q=batch_ids_buf[:n_tiles],
        q_tile_starts_q=tile_starts_buf[:n_tiles],
        cu_seqlens_host=tuple(host[: B + 1]),
    )


def _build_query_tile_map_from_cu_seqlens(cu_seqlens_q: torch.Tensor, block_n: int):
    """(q_tile_starts_q, batch_ids) for tiles of ``block_n`` rows (host_utils.py:74-107)."""
    if cu_seqlens_q.ndim != 1:
        raise ValueError("cu_seqlens_q must be rank-1")
    if cu_seqlens_q.numel() < 2:
        raise ValueError("cu_seqlens_q must have at least 2 elements")
    if block_n < 1:
        raise ValueError("block_n must be >= 1")
    _require_device(cu_seqlens_q, what="the query tile map")
    lib = _lib.load()
    device = cu_seqlens_q.device
    cu = cu_seqlens_q.to(torch.int32).contiguous()
    B = int(cu.numel()) - 1
    cu_host = cu.to("cpu").tolist()
    # sum_b ceil(L_b / block_n) <= B + total / block_n
    capacity = B + max(cu_host[-1] - cu_host[0], 0) // block_n + 1
    buf = torch.empty(2 * capacity + 1, dtype=torch.int32, device=device)
    with _device_scope(device):
        rc = lib.fmlm_tile_map(
            _lib.ptr(cu),
            B,
            int(block_n),
            capacity,
            _lib.ptr(buf),
            _lib.ptr(buf) + 4 * capacity,
            _lib.ptr(buf) + 8 * capacity,
            _lib.stream_of(device),
        )
    _lib.check(rc, "fmlm_tile_map")
    n_tiles = int(buf[2 * capacity].item())
    if n_tiles == 0:
        empty = torch.empty((0,), device=device, dtype=torch.int32)
        return empty, empty
    batch_ids = buf[:n_tiles]
    q_tile_starts = buf[capacity : capacity + n_tiles]
    return q_tile_starts, batch_ids


def build_batch_ids_from_cu_seqlens(cu_seqlens_q: torch.Tensor, block_n: int):
    """Tile -> sequence map of packed query tiles (host_utils.py:110-113)."""
    return _build_query_tile_map_from_cu_seqlens(cu_seqlens_q, block_n)[1]


def build_q_tile_starts_from_cu_seqlens(cu_seqlens_q: torch.Tensor, block_n: int):
    """Packed start offset of every query tile (host_utils.py:116-119)."""
    return _build_query_tile_map_from_cu_seqlens(cu_seqlens_q, block_n)[0]


def num_query_tiles_from_cu_seqlens(cu_seqlens_q: torch.Tensor, block_n: int) -> int:
    """Number of query tiles (host_utils.py:122-125)."""
    return int(build_q_tile_starts_from_cu_seqlens(cu_seqlens_q, block_n).numel())


def num_query_tiles_from_meta(meta: PackMetadata) -> int:
    """Number of query tiles stored in ``meta`` (host_utils.py:128-130)."""
    return int(meta.q_tile_starts_q.numel())


# ---------------------------------------------------------------------------
# validation (host_utils.py:142-153, 315-394)
# ---------------------------------------------------------------------------
def validate_cache_request(
    *,
    prefill: bool,
    inference_cache: InferenceCache | None,
    layer_id: int | str | None,
) -> None:
    if prefill and inference_cache is None:
        raise ValueError("prefill=True requires inference_cache")
    if (inference_cache is None) != (layer_id is None):
        raise ValueError("inference_cache and layer_id must be provided together or both omitted")


def require_cuda_tensors(*tensors: torch.Tensor | None, message: str = "All tensors must be CUDA tensors"):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(message)


def validate_qkv_same_shape_rank4(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    error_prefix: str,
) -> tuple[int, int, int, int]:
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError(f"{error_prefix} must be rank-4 tensors [B, H, N, D]")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must have the same shape")
    b, h, n, d = (int(x) for x in q.shape)
    return b, h, n, d


def validate_head_dim_supported(head_dim: int, *, is_mla: bool = False):
    """Reference set {16, 32, 64, 128, 256}; MLA latents may also be 512 wide."""
    if head_dim in _HEAD_DIMS:
        return
    if is_mla and head_dim in _MLA_HEAD_DIMS:
        return
    raise ValueError("HEAD_DIM must be one of {16, 32, 64, 128, 256}")


def validate_cu_seqlens_rank1_min2(*cu_seqlens: torch.Tensor):
    for cu in cu_seqlens:
        if cu.ndim != 1:
            raise ValueError("cu_seqlens tensors must be rank-1")
        if cu.numel() < 2:
            raise ValueError("cu_seqlens tensors must have at least 2 elements")


def validate_packed_cache_shapes(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor | None,
    *,
    num_heads: int,
    total_context_len: int,
    head_dim: int,
    is_mla: bool,
):
    if k_cache.ndim != 2:
        raise ValueError("k_cache must be a rank-2 packed tensor")
    if k_cache.shape[1] != head_dim:
        raise ValueError("k_cache second dim must match q/k/v head_dim")
    if is_mla:
        if v_cache is not None:
            if v_cache.ndim != 2:
                raise ValueError("MLA v_cache must be a rank-2 packed tensor")
            if v_cache.shape != k_cache.shape:
                raise ValueError("MLA v_cache shape must match k_cache shape")
    else:
        if v_cache is None:
            raise ValueError("non-MLA cache requires v_cache")
        if v_cache.ndim != 2:
            raise ValueError("v_cache must be a rank-2 packed tensor")
        if v_cache.shape != k_cache.shape:
            raise ValueError("v_cache shape must match k_cache shape")
        if v_cache.shape[1] != head_dim:
            raise ValueError("v_cache second dim must match q/k/v head_dim")
    rows = total_context_len * (1 if is_mla else num_heads)
    if k_cache.shape[0] != rows:
        raise ValueError(f"k_cache first dim mismatch: expected {rows} rows for is_mla={is_mla}")
    if not is_mla and v_cache.shape[0] != rows:
        raise ValueError(f"v_cache first dim mismatch: expected {rows} rows for is_mla={is_mla}")


def make_contiguous(*tensors: torch.Tensor | None) -> tuple[torch.Tensor | None, ...]:
    return tuple(None if t is None else t.contiguous() for t in tensors)


# ---------------------------------------------------------------------------
# cached context (host_utils.py:156-263)
# ---------------------------------------------------------------------------
def _maybe_get_cache_context(
    *,
    inference_cache: InferenceCache | None,
    layer_id: int | str | None,
    batch_size: int,
    num_heads: int,
    head_dim: int,
    is_mla: bool,
    context_batch_size: int | None,
    device: torch.device,
    dtype: torch.dtype,
    compressed: bool,
) -> CacheContext:
    """Resolve the context a launch attends to.

    A missing entry, or one whose mode / heads / head_dim / dtype / device differ from
    the request, gives an empty context (the lookup error is swallowed).  A hit keeps the
    stored context batch count unless ``context_batch_size`` asks for 1 (shared context:
    packed cu_seqlens_kv becomes [0, total]; dense context_len becomes total) and
    rejects any other differing count.
    """
    entry: LayerKVEntry | None = None
    if inference_cache is not None:
        try:
            entry = inference_cache.get_kv_cache(
                layer_id,
                is_mla=is_mla,
                num_heads=num_heads,
                head_dim=head_dim,
                dtype=dtype,
                device=device,
            )
        except ValueError:
            entry = None

    if entry is None:
        cbs = batch_size if context_batch_size is None else context_batch_size
        k_cache = torch.empty((0, head_dim), device=device, dtype=dtype)
        v_cache = torch.empty_like(k_cache)
        cu_kv = torch.zeros(cbs + 1, device=device, dtype=torch.int32) if compressed else None
        return CacheContext(
            k_cache=k_cache,
            v_cache=v_cache,
            context_batch_size=cbs,
            context_len=0,
            total_context_len=0,
            cu_seqlens_kv=cu_kv,
        )

    stored_cbs = entry.context_batch_size
    cbs = stored_cbs
    if context_batch_size is not None:
        if context_batch_size == 1:
            cbs = 1
        elif context_batch_size != stored_cbs:
            raise ValueError(
                f"context_batch_size ({context_batch_size}) must match cached entry "
                f"context_batch_size ({stored_cbs})"
            )
    if cbs < 1:
        raise ValueError("context_batch_size must be >= 1")

    total = int(entry.total_context_len)
    context_len = 0
    if entry.block_table is not None:  # paged entry (extension)
        if not compressed:
            raise ValueError("paged KV contexts serve the packed paths (flash_attn_mlm_compressed / _precompressed)")
        if cbs != stored_cbs:
            raise ValueError("a paged context cannot be shared with context_batch_size=1")
        return CacheContext(
            k_cache=entry.k_cache,
            v_cache=entry.v_cache,
            context_batch_size=cbs,
            context_len=0,
            total_context_len=total,
            cu_seqlens_kv=entry.cu_seqlens_kv,
            block_table=entry.block_table,
        )
    if compressed:
        cu_kv = entry.cu_seqlens_kv
        if cu_kv is None:
            if total % stored_cbs:
                raise ValueError(
                    "compressed path requires cu_seqlens_kv or uniform per-batch context lengths"
                )
            context_len = total // stored_cbs
            cu_kv = torch.arange(stored_cbs + 1, device=device, dtype=torch.int32) * context_len
        if cbs == 1 and stored_cbs != 1:
            cu_kv = torch.tensor([0, total], device=device, dtype=torch.int32)
    else:
        cu_kv = None
        if total % cbs:
            raise ValueError("dense flash_attn_mlm requires uniform per-batch context lengths")
        context_len = total // cbs
        rows = total * (1 if is_mla else num_heads)
        if entry.k_cache.shape[0] != rows or (not is_mla and entry.v_cache.shape[0] != rows):
            raise ValueError("cached dense k/v rows mismatch expected layout for is_mla/num_heads")

    return CacheContext(
        k_cache=entry.k_cache,
        v_cache=entry.v_cache,
        context_batch_size=cbs,
        context_len=context_len,
        total_context_len=total,
        cu_seqlens_kv=cu_kv,
    )


# ---------------------------------------------------------------------------
# pack / pad / unpack (host_utils.py:266-312, 397-615)
# ---------------------------------------------------------------------------
def _compute_total_q_len_padded(
    total_q_len_unpadded: int,
    cu_seqlens_q: torch.Tensor | tuple[int, ...] | list[int],
    block_m: int,
    block_n: int,
) -> int:
    """max(T, max_b(cu[b] + ceil(L_b / a) * a)) with a = max(block_m, block_n)
    (host_utils.py:292-312).  Accepts a device tensor (one synchronising copy) or a
    host sequence of the cumulative lengths."""
    if isinstance(cu_seqlens_q, torch.Tensor):
        cu = [int(x) for x in cu_seqlens_q.to("cpu").tolist()]
    else:
        cu = [int(x) for x in cu_seqlens_q]
    align = max(block_m, block_n)
    required = 0
    for b in range(len(cu) - 1):
        length = cu[b + 1] - cu[b]
        end = cu[b] + ((length + align - 1) // align) * align
        required = end if b == 0 else max(required, end)
    return max(int(total_q_len_unpadded), required)


def _pack_rows(
    sources: list[tuple[torch.Tensor, int]],
    outs: list[torch.Tensor],
    *,
    cu_seqlens: torch.Tensor | None,
    B: int,
    N: int,
    D: int,
    total: int,
    total_padded: int,
) -> None:
    """One fmlm_pack launch: rows (b, h < heads, p < L_b) of each 4-D source
    [B, H, N, D] -> out[h*total_padded + cu[b] + p], zero tail rows."""
    lib = _lib.load()
    descs = (_lib.PackTensor * len(sources))()
    keep = []
    esz = None
    for i, ((src, heads), out) in enumerate(zip(sources, outs)):
        if src.stride(-1) != 1:
            src = src.contiguous()
        keep.append(src)
        if not out.is_contiguous():
            raise ValueError("packed output buffer must be contiguous")
        esz = src.element_size()
        descs[i].src = src.data_ptr()
        descs[i].s_sb = src.stride(0)
        descs[i].s_sh = src.stride(1)
        descs[i].s_sn = src.stride(2)
        descs[i].dst = out.data_ptr()
        descs[i].heads = heads
    device = outs[0].device
    with _device_scope(device):
        rc = lib.fmlm_pack(
            descs,
            len(sources),
            esz,
            B,
            N,
            D,
            _lib.ptr(cu_seqlens),
            int(total),
            int(total_padded),
            _lib.stream_of(device),
        )
    _lib.check(rc, "fmlm_pack")


def pack_for_kernel(x: torch.Tensor, meta: PackMetadata, flatten_for_kernel: bool = False):
    """Pack padded [B, H, N, D] into [H, T, D] (or [H*T, D] when flattened)
    (host_utils.py:266-289)."""
    if x.ndim != 4:
        raise ValueError("x must be rank-4 [B, H, N, D]")
    B, H, N, D = (int(s) for s in x.shape)
    if B != meta.B or N != meta.N:
        raise ValueError("x shape mismatch with PackMetadata")
    _require_device(x, meta.cu_seqlens, what="pack_for_kernel")
    T = int(meta.total_tokens)
    out = torch.empty((H * T, D), dtype=x.dtype, device=x.device)
    if H * T > 0:
        _pack_rows(
            [(x, H)],
            [out],
            cu_seqlens=meta.cu_seqlens.to(torch.int32).contiguous(),
            B=B,
            N=N,
            D=D,
            total=T,
            total_padded=T,
        )
    return out if flatten_for_kernel else out.view(H, T, D)


def _pack_flatten_for_kernel_into(
    x: torch.Tensor,
    meta: PackMetadata,
    expected_heads: int,
    total_q_len_padded: int,
    out: torch.Tensor,
) -> torch.Tensor:
    """Pack [B, heads, N, D] into ``out`` [heads*T_pad, D], zeroing rows T..T_pad of
    every head (host_utils.py:397-420)."""
    if x.ndim != 4:
        raise ValueError("x must be rank-4 [B, H, N, D]")
    b, h, n, d = (int(s) for s in x.shape)
    if b != meta.B or n != meta.N:
        raise ValueError("x shape mismatch with PackMetadata")
    if h != expected_heads:
        raise ValueError("x head dimension mismatch for requested packed output")
    if tuple(out.shape) != (expected_heads * total_q_len_padded, d):
        raise ValueError("out has unexpected shape for packed output")
    _require_device(x, out, what="_pack_flatten_for_kernel_into")
    if out.numel():
        _pack_rows(
            [(x, h)],
            [out],
            cu_seqlens=meta.cu_seqlens.to(torch.int32).contiguous(),
            B=b,
            N=n,
            D=d,
            total=meta.total_tokens,
            total_padded=total_q_len_padded,
        )
    return out


def pack_and_pad_main_tensors_for_mlm_compressed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    q_meta: PackMetadata,
    num_heads: int,
    is_mla: bool,
    block_m: int,
    block_n: int,
    packing_cache: "PackingCache | None" = None,
    q_buffer_name: str = "q",
    k_buffer_name: str = "k",
    v_buffer_name: str = "v",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    """Pack q, k, v (MLA: q and head 0 of k, with v_out = k_out) into zero-padded
    head-major buffers [heads*T_pad, D] in one HIP launch (host_utils.py:423-491)."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q/k/v must be rank-4 padded tensors [B, H, N, D]")
    b, h, n, d = (int(s) for s in q.shape)
    if q_meta.B != b or q_meta.N != n:
        raise ValueError("q_meta shape metadata does not match q/k/v padded shape")
    if h != num_heads:
        raise ValueError("q/k/v head dimension must match num_heads")
    _require_device(q, k, v, what="pack_and_pad_main_tensors_for_mlm_compressed")

    T = int(q_meta.total_tokens)
    T_pad = _compute_total_q_len_padded(T, q_meta.host_cu_seqlens(), block_m, block_n)

    def alloc(name: str, rows: int, template: torch.Tensor) -> torch.Tensor:
        if packing_cache is None:
            return torch.empty((rows, d), dtype=template.dtype, device=template.device)
        return packing_cache.get_2d(name, rows, d, dtype=template.dtype, device=template.device)

    q_out = alloc(q_buffer_name, num_heads * T_pad, q)
    if is_mla:
        k_src = k[:, :1]
        k_out = alloc(k_buffer_name, T_pad, k)
        v_out = k_out
        sources = [(q, num_heads), (k_src, 1)]
        outs = [q_out, k_out]
    else:
        k_out = alloc(k_buffer_name, num_heads * T_pad, k)
        v_out = alloc(v_buffer_name, num_heads * T_pad, v)
        sources = [(q, num_heads), (k, num_heads), (v, num_heads)]
        outs = [q_out, k_out, v_out]
    if T_pad > 0 and d > 0:
        _pack_rows(
            sources,
            outs,
            cu_seqlens=q_meta.cu_seqlens.to(torch.int32).contiguous(),
            B=b,
            N=n,
            D=d,
            total=T,
            total_padded=T_pad,
        )
    return q_out, k_out, v_out, T_pad


def pad_packed_main_tensors_for_mlm_compressed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    num_heads: int,
    is_mla: bool,
    total_q_len_unpadded: int,
    cu_seqlens_q: torch.Tensor,
    block_m: int,
    block_n: int,
    packing_cache: "PackingCache | None" = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    """Zero-pad already packed [heads*T, D] tensors to [heads*T_pad, D]
    (host_utils.py:494-584).  Returns the inputs unchanged when T_pad == T."""
    T = int(total_q_len_unpadded)
    T_pad = _compute_total_q_len_padded(T, cu_seqlens_q, block_m, block_n)
    if T_pad == T:
        return q, k, v, T
    kv_heads = 1 if is_mla else num_heads

    def pad(x: torch.Tensor, heads: int, name: str) -> torch.Tensor:
        d = int(x.shape[1])
        if packing_cache is None:
            out = torch.empty((heads * T_pad, d), dtype=x.dtype, device=x.device)
        else:
            out = packing_cache.get_2d(name, heads * T_pad, d, dtype=x.dtype, device=x.device)
        _require_device(x, out, what="pad_packed_main_tensors_for_mlm_compressed")
        # a packed [heads*T, D] tensor is one sequence of T rows per head
        src = x.contiguous().view(1, heads, T, d)
        _pack_rows([(src, heads)], [out], cu_seqlens=None, B=1, N=T, D=d, total=T, total_padded=T_pad)
        return out

    return pad(q, num_heads, "q"), pad(k, kv_heads, "k"), pad(v, kv_heads, "v"), T_pad


def unpack_from_kernel(packed: torch.Tensor, meta: PackMetadata, H: int):
    """Packed [H*T, D] or [H, T, D] -> padded [B, H, N, D] with zeros at padding
    (host_utils.py:587-615), written in one HIP pass."""
    if packed.ndim == 3:
        total_tokens, D = int(packed.shape[1]), int(packed.shape[2])
        if int(packed.shape[0]) != H:
            raise ValueError("packed first dim must be H")
        packed_h = packed
    elif packed.ndim == 2:
        total_tokens = int(meta.total_tokens)
        D = int(packed.shape[1])
        if total_tokens == 0:
            packed_h = packed.new_empty((H, 0, D))
        else:
            if packed.shape[0] != H * total_tokens:
                raise ValueError("packed first dim must be H * total_tokens")
            packed_h = packed.view(H, total_tokens, D)
    else:
        raise ValueError("packed must be rank-2 or rank-3")
    if total_tokens != meta.total_tokens:
        raise ValueError("packed token count mismatch with PackMetadata")
    _require_device(packed, meta.cu_seqlens, what="unpack_from_kernel")

    out = torch.empty((meta.B, H, meta.N, D), dtype=packed.dtype, device=packed.device)
    if out.numel() == 0:
        return out
    packed_h = packed_h.contiguous()
    lib = _lib.load()
    cu = meta.cu_seqlens.to(torch.int32).contiguous()
    with _device_scope(packed.device):
        rc = lib.fmlm_unpack(
            packed.element_size(),
            packed_h.data_ptr(),
            total_tokens * D,
            out.data_ptr(),
            meta.B,
            H,
            meta.N,
            D,
            cu.data_ptr(),
            _lib.stream_of(packed.device),
        )
    _lib.check(rc, "fmlm_unpack")
    return out


def copy_segments(src: torch.Tensor | None, src_rows: int, src_cu: torch.Tensor, dst: torch.Tensor, dst_rows: int,
                  dst_start: torch.Tensor, C: int, H: int, D: int) -> None:
    """Head-major segment copy on the GPU (one HIP launch): for head h and segment c,
    rows src_cu[c]..src_cu[c+1] of head h of ``src`` ([H * src_rows, D]) go to rows
    dst_start[c].. of head h of ``dst`` ([H * dst_rows, D]); ``src=None`` writes zero rows
    there instead.  The kernel of :meth:`InferenceCache.append_kv_cache`; no counterpart in
    the reference."""
    _require_device(src, dst, src_cu, dst_start, what="copy_segments")
    lib = _lib.load()
    with _device_scope(dst.device):
        rc = lib.fmlm_copy_segments(
            dst.element_size(), None if src is None else src.data_ptr(), src_rows * D, src_rows, src_cu.data_ptr(),
            dst.data_ptr(), dst_rows * D, dst_rows, dst_start.data_ptr(), C, H, D, _lib.stream_of(dst.device),
        )
    _lib.check(rc, "fmlm_copy_segments")


def kv_append(pairs, cu_old: torch.Tensor, cu_new: torch.Tensor, *, heads: int, rows_old: int, rows_new: int):
    """The merge of :meth:`InferenceCache.append_kv_cache` in one HIP launch
    (fmlm_kv_append): for each (old [heads*rows_old, D], new [heads*rows_new, D]) pair a
    new head-major buffer whose batch c holds its old rows then its new rows, zero rows
    past the last batch; returns (buffers, int32 offsets cu_old + cu_new).  No
    counterpart in the reference."""
    old0 = pairs[0][0]
    dev, dt = old0.device, old0.dtype
    d = int(old0.shape[1])
    _require_device(cu_old, cu_new, *(t for pr in pairs for t in pr), what="kv_append")
    rows = rows_old + rows_new
    C = int(cu_old.numel()) - 1
    outs, keep = [], []
    arr = (_lib.AppendTensor * len(pairs))()
    for i, (old, new) in enumerate(pairs):
        old, new = old.contiguous(), new.contiguous()
        out = torch.empty((heads * rows, d), dtype=dt, device=dev)
        arr[i].old, arr[i].add, arr[i].out = old.data_ptr(), new.data_ptr(), out.data_ptr()
        outs.append(out)
        keep += [old, new]
    cu_out = torch.empty_like(cu_old)
    lib = _lib.load()
    with _device_scope(dev):
        rc = lib.fmlm_kv_append(arr, len(pairs), old0.element_size(), heads, d, C, rows_old, rows_new,
                                cu_old.data_ptr(), cu_new.data_ptr(), cu_out.data_ptr(), _lib.stream_of(dev))
    _lib.check(rc, "fmlm_kv_append")
    return outs, cu_out
