"""Host-side state of the MLM attention path: pack metadata, packing workspaces and
the per-layer KV context cache.

Mirrors src/flash_mlm/host/cache.py of the reference (PackMetadata :5-17,
PackingCache :20-73, LayerKVEntry :76-87, InferenceCache :90-280): the same
fields, the same lookup keys, the same ValueError messages, and the same
"store views, never copy" contract for cached KV.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class PackMetadata:
    """Indexing of a padded [B, N] batch as packed variable-length tokens.

    Fields follow the reference (cache.py:5-17).  ``cu_seqlens_host`` is an extra,
    optional host copy of ``cu_seqlens`` filled by :func:`build_pack_metadata`; it lets
    the launchers size padded workspaces without a device-to-host synchronisation.
    ``kernel_schedules`` caches the attention kernel's device work lists built from
    ``cu_seqlens`` (one per kernel tile size), so repeated layers skip rebuilding them;
    ``launch_memo`` the parameter blocks of earlier compressed calls on this metadata.
    """

    B: int
    N: int
    lengths: torch.Tensor
    cu_seqlens: torch.Tensor
    token_indices: torch.Tensor
    total_tokens: int
    batch_ids_block_n: int
    batch_ids_q: torch.Tensor
    q_tile_starts_q: torch.Tensor
    cu_seqlens_host: tuple[int, ...] | None = field(default=None, repr=False, compare=False)
    kernel_schedules: dict = field(default_factory=dict, repr=False, compare=False)
    launch_memo: dict = field(default_factory=dict, repr=False, compare=False)

    def host_cu_seqlens(self) -> tuple[int, ...]:
        if self.cu_seqlens_host is None:
            self.cu_seqlens_host = tuple(int(x) for x in self.cu_seqlens.to("cpu").tolist())
        return self.cu_seqlens_host


class PackingCache:
    """Grow-only named 2-D workspaces plus a memo of pack metadata (cache.py:20-73)."""

    def __init__(self) -> None:
        self._buffers: dict[tuple, torch.Tensor] = {}
        self._pack_meta: dict[tuple, PackMetadata] = {}

    def get_2d(
        self,
        name: str,
        rows: int,
        cols: int,
        *,
        dtype: torch.dtype,
        device: torch.device,
    ) -> torch.Tensor:
        """Return a [rows, cols] view of the workspace ``name``, reallocating only to grow."""
        if rows < 0:
            raise ValueError("rows must be >= 0")
        if cols < 1:
            raise ValueError("cols must be >= 1")
        device = torch.device(device)
        key = (name, device.type, device.index, dtype, cols)
        buf = self._buffers.get(key)
        if buf is None or buf.shape[0] < rows:
            buf = torch.empty((rows, cols), dtype=dtype, device=device)
            self._buffers[key] = buf
        return buf[:rows]

    def get_pack_metadata(self, lengths: torch.Tensor, *, N: int, block_n: int) -> PackMetadata:
        """Memoised :func:`build_pack_metadata`, keyed by (device, N, block_n, lengths)."""
        signature = tuple(int(x) for x in lengths.to(device="cpu", dtype=torch.int32).tolist())
        key = (lengths.device.type, lengths.device.index, N, block_n, signature)
        meta = self._pack_meta.get(key)
        if meta is None:
            from flash_mlm.host.host_utils import build_pack_metadata

            meta = build_pack_metadata(lengths, N, block_n)
            self._pack_meta[key] = meta
        return meta

    def clear(self) -> None:
        self._buffers.clear()
        self._pack_meta.clear()


@dataclass
class LayerKVEntry:
    """One layer's cached context (cache.py:76-87).

    Layout of ``k_cache`` / ``v_cache`` rows:
      * MLA: one shared latent head, row = token            ([total_context_len, D])
      * non-MLA, packed entries: head-major, row = h*total_context_len + token
      * non-MLA, dense entries: [context_batch, H, context_len] flattened
    """

    k_cache: torch.Tensor
    v_cache: torch.Tensor | None
    total_context_len: int
    cu_seqlens_kv: torch.Tensor | None
    context_batch_size: int
    is_mla: bool
    num_heads: int
    head_dim: int
    dtype: torch.dtype
    device: torch.device
    # paged entries (an extension, see InferenceCache.prefill_paged_kv_cache): k_cache /
    # v_cache are the page pool [H_kv, P, PAGE_ROWS, D] flattened to rank 2 (head-major,
    # like the packed entries), total_context_len = P * PAGE_ROWS, cu_seqlens_kv the prefix
    # sums of the batch lengths
    block_table: torch.Tensor | None = None


PAGE_ROWS = 64  # rows per page of a paged context (FMLM_PAGE_ROWS, the kernels' key tile)


def _check_rank2(t: torch.Tensor, what: str) -> None:
    if t.ndim != 2:
        raise ValueError(f"{what} must be a rank-2 packed tensor")


class InferenceCache:
    """Layer-scoped KV context store plus a :class:`PackingCache` (cache.py:90-280).

    Entries hold the given tensors themselves (views, no copies); storing a layer
    again replaces its entry.
    """

    def __init__(self) -> None:
        self.packing = PackingCache()
        self._layer_kv: dict[str, LayerKVEntry] = {}

    @staticmethod
    def _layer_key(layer_id: int | str) -> str:
        return str(layer_id)

    @staticmethod
    def _validate_kv_common_inputs(
        *,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor | None,
        total_context_len: int,
        is_mla: bool,
        num_heads: int,
        head_dim: int,
    ) -> None:
        _check_rank2(k_cache, "k_cache")
        if k_cache.shape[1] != head_dim:
            raise ValueError("k_cache second dim must match head_dim")
        if not k_cache.is_contiguous():
            raise ValueError("k_cache must be contiguous")
        if is_mla:
            if v_cache is not None:
                _check_rank2(v_cache, "MLA v_cache")
                if v_cache.shape != k_cache.shape:
                    raise ValueError("MLA v_cache shape must match k_cache shape")
                if not v_cache.is_contiguous():
                    raise ValueError("MLA v_cache must be contiguous")
        else:
            if v_cache is None:
                raise ValueError("non-MLA cache requires v_cache")
            _check_rank2(v_cache, "v_cache")
            if v_cache.shape != k_cache.shape:
                raise ValueError("v_cache shape must match k_cache shape")
            if v_cache.shape[1] != head_dim:
                raise ValueError("v_cache second dim must match head_dim")
            if not v_cache.is_contiguous():
                raise ValueError("v_cache must be contiguous")
        rows = total_context_len * (1 if is_mla else num_heads)
        if k_cache.shape[0] != rows:
            raise ValueError(f"k_cache first dim mismatch: expected {rows} rows for is_mla={is_mla}")
        if not is_mla and v_cache.shape[0] != rows:
            raise ValueError(f"v_cache first dim mismatch: expected {rows} rows for is_mla={is_mla}")

    @staticmethod
    def _validate_kv_entry_inputs(
        *,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor | None,
        total_context_len: int,
        cu_seqlens_kv: torch.Tensor,
        context_batch_size: int,
        is_mla: bool,
        num_heads: int,
        head_dim: int,
    ) -> None:
        InferenceCache._validate_kv_common_inputs(
            k_cache=k_cache,
            v_cache=v_cache,
            total_context_len=total_context_len,
            is_mla=is_mla,
            num_heads=num_heads,
            head_dim=head_dim,
        )
        if cu_seqlens_kv.ndim != 1 or cu_seqlens_kv.numel() < 2:
            raise ValueError("cu_seqlens_kv must be rank-1 with at least 2 elements")
        if context_batch_size < 1:
            raise ValueError("context_batch_size must be >= 1")
        if cu_seqlens_kv.numel() < context_batch_size + 1:
            raise ValueError("context_batch_size is incompatible with cu_seqlens_kv length")

    def prefill_kv_cache(
        self,
        layer_id: int | str,
        *,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor | None = None,
        total_context_len: int | None = None,
        cu_seqlens_kv: torch.Tensor | None = None,
        context_batch_size: int,
        is_mla: bool,
        num_heads: int,
        head_dim: int,
    ) -> None:
        """Store pre-packed KV buffers as the context of ``layer_id`` (no copy)."""
        if context_batch_size < 1:
            raise ValueError("context_batch_size must be >= 1")
        if num_heads < 1:
            raise ValueError("num_heads must be >= 1")

        if total_context_len is not None:
            total_context_len = int(total_context_len)
        elif is_mla:
            total_context_len = int(k_cache.shape[0])
        else:
            if k_cache.shape[0] % num_heads:
                raise ValueError("non-MLA k_cache rows must be divisible by num_heads")
            total_context_len = int(k_cache.shape[0] // num_heads)

        if cu_seqlens_kv is None:
            self._validate_kv_common_inputs(
                k_cache=k_cache,
                v_cache=v_cache,
                total_context_len=total_context_len,
                is_mla=is_mla,
                num_heads=num_heads,
                head_dim=head_dim,
            )
            if total_context_len % context_batch_size:
                raise ValueError(
                    "when cu_seqlens_kv is omitted, total_context_len must be divisible by "
                    "context_batch_size"
                )
        else:
            self._validate_kv_entry_inputs(
                k_cache=k_cache,
                v_cache=v_cache,
                total_context_len=total_context_len,
                cu_seqlens_kv=cu_seqlens_kv,
                context_batch_size=context_batch_size,
                is_mla=is_mla,
                num_heads=num_heads,
                head_dim=head_dim,
            )

        self._layer_kv[self._layer_key(layer_id)] = LayerKVEntry(
            k_cache=k_cache,
            v_cache=None if is_mla else v_cache,
            total_context_len=total_context_len,
            cu_seqlens_kv=None if cu_seqlens_kv is None else cu_seqlens_kv.contiguous(),
            context_batch_size=int(context_batch_size),
            is_mla=bool(is_mla),
            num_heads=int(num_heads),
            head_dim=int(head_dim),
            dtype=k_cache.dtype,
            device=k_cache.device,
        )

    def prefill_paged_kv_cache(
        self,
        layer_id: int | str,
        *,
        k_pages: torch.Tensor,
        v_pages: torch.Tensor | None = None,
        block_table: torch.Tensor,
        context_lens: torch.Tensor,
        is_mla: bool,
        num_heads: int,
        head_dim: int,
    ) -> None:
        """Store a paged context as ``layer_id``'s entry (no copy).

        This is an extension: the reference's roadmap lists paged KV (README.md:41).

        ``k_pages`` / ``v_pages`` are page pools [H_kv, P, 64, D] (contiguous, head-major
        like the packed entries: a head's pages are adjacent; H_kv = 1 and ``v_pages`` None
        for MLA).  ``block_table`` [C, max_pages] (int, on the
        device) lists the pages of each of the C context batches in key order.
        ``context_lens`` [C] gives their lengths: batch c's key j is row j % 64 of page
        ``block_table[c, j // 64]``.  The attention kernels read the pages in place,
        one page per key tile.  Served by the packed paths (flash_attn_mlm_compressed /
        _precompressed) for bf16/fp16.
        """
        if num_heads < 1:
            raise ValueError("num_heads must be >= 1")
        h_kv = 1 if is_mla else num_heads
        if k_pages.ndim != 4 or k_pages.shape[0] != h_kv or tuple(k_pages.shape[2:]) != (PAGE_ROWS, head_dim):
            raise ValueError(f"k_pages must be [{h_kv}, pages, {PAGE_ROWS}, head_dim]")
        if not k_pages.is_contiguous():
            raise ValueError("k_pages must be contiguous")
        if is_mla:
            if v_pages is not None:
                raise ValueError("MLA paged cache takes k_pages only (V = K)")
        elif v_pages is None or v_pages.shape != k_pages.shape or not v_pages.is_contiguous() \
                or v_pages.dtype != k_pages.dtype or v_pages.device != k_pages.device:
            raise ValueError("non-MLA paged cache requires contiguous v_pages shaped like k_pages")
        if k_pages.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("paged KV contexts need bf16 or fp16 pages")
        if block_table.ndim != 2 or block_table.dtype not in (torch.int32, torch.int64):
            raise ValueError("block_table must be a rank-2 integer tensor [context_batch, max_pages]")
        n_batch, max_pages = int(block_table.shape[0]), int(block_table.shape[1])
        if n_batch < 1:
            raise ValueError("block_table needs at least one context batch")
        if context_lens.ndim != 1 or int(context_lens.numel()) != n_batch:
            raise ValueError("context_lens must have one entry per block_table row")
        if not context_lens.is_cuda and n_batch:
            lo, hi = int(context_lens.min()), int(context_lens.max())
            if lo < 0 or hi > max_pages * PAGE_ROWS:
                raise ValueError(f"context_lens must lie in [0, {max_pages * PAGE_ROWS}]")
        dev = k_pages.device
        n_pages = int(k_pages.shape[1])
        cu = torch.zeros(n_batch + 1, dtype=torch.int32, device=dev)
        cu[1:] = torch.cumsum(context_lens.to(device=dev, dtype=torch.int32), 0)
        self._layer_kv[self._layer_key(layer_id)] = LayerKVEntry(
            k_cache=k_pages.view(n_pages * h_kv * PAGE_ROWS, head_dim),
            v_cache=None if is_mla else v_pages.view(n_pages * h_kv * PAGE_ROWS, head_dim),
            total_context_len=n_pages * PAGE_ROWS,
            cu_seqlens_kv=cu,
            context_batch_size=n_batch,
            is_mla=bool(is_mla),
            num_heads=int(num_heads),
            head_dim=int(head_dim),
            dtype=k_pages.dtype,
            device=dev,
            block_table=block_table.to(device=dev, dtype=torch.int32).contiguous(),
        )

    def append_kv_cache(
        self,
        layer_id: int | str,
        *,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor | None = None,
        cu_seqlens_kv: torch.Tensor,
    ) -> None:
        """Append rows to every context batch of ``layer_id``'s packed entry.

        This is an extension: the reference replaces a layer's context on prefill and
        lists appends with paged KV on its roadmap (README.md:34-41).

        ``k_cache`` / ``v_cache`` hold the new rows head-major like the entry: [T_new, D]
        for MLA (``v_cache`` must be None), else [H * T_new, D].  Batch c's new rows are
        ``cu_seqlens_kv[c] .. cu_seqlens_kv[c+1]``.  The entry becomes [old rows of c ||
        new rows of c] for every batch c: new buffers of T_old + T_new rows per head, and
        cu_seqlens_kv = old + new offsets.  Rows per head past the last batch are zero, as
        the zero padding rows of a prefilled packed entry are: a later call that asks for a
        shared context (``context_batch_size=1``) attends to every row of the entry.  The
        merge of K and V (and the new offsets) is one HIP launch, stream-ordered; nothing
        is read back to the host.
        """
        key = self._layer_key(layer_id)
        entry = self._layer_kv.get(key)
        if entry is None:
            raise ValueError(f"no cached KV entry for layer {layer_id!r}")
        if entry.cu_seqlens_kv is None or entry.block_table is not None:
            raise ValueError("append_kv_cache requires a packed entry (stored with cu_seqlens_kv)")
        h_kv = 1 if entry.is_mla else entry.num_heads
        d = entry.head_dim
        _check_rank2(k_cache, "k_cache")
        if k_cache.shape[1] != d:
            raise ValueError("k_cache second dim must match head_dim")
        if k_cache.dtype != entry.dtype or k_cache.device != entry.device:
            raise ValueError("k_cache dtype/device must match the cached entry")
        if k_cache.shape[0] % h_kv:
            raise ValueError("non-MLA k_cache rows must be divisible by num_heads")
        if entry.is_mla:
            if v_cache is not None:
                raise ValueError("MLA append takes k_cache only (V = K)")
        elif v_cache is None or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype \
                or v_cache.device != k_cache.device:
            raise ValueError("non-MLA append requires v_cache shaped like k_cache")
        n_batch = int(entry.cu_seqlens_kv.numel()) - 1
        if cu_seqlens_kv.ndim != 1 or int(cu_seqlens_kv.numel()) != n_batch + 1:
            raise ValueError("cu_seqlens_kv must have one entry per cached context batch, plus one")
        t_old, t_new = int(entry.total_context_len), int(k_cache.shape[0]) // h_kv
        if not cu_seqlens_kv.is_cuda:
            cu_host = cu_seqlens_kv.to(torch.int64)
            if int(cu_host[0]) != 0 or bool((cu_host[1:] < cu_host[:-1]).any()) or int(cu_host[-1]) > t_new:
                raise ValueError("cu_seqlens_kv must start at 0, be non-decreasing and end within the new rows")
        from flash_mlm.host.host_utils import kv_append

        dev = entry.device
        cu_old = entry.cu_seqlens_kv.to(device=dev, dtype=torch.int32).contiguous()
        cu_new = cu_seqlens_kv.to(device=dev, dtype=torch.int32).contiguous()
        rows = t_old + t_new
        pairs = [(entry.k_cache, k_cache)] + ([] if entry.is_mla else [(entry.v_cache, v_cache)])
        outs, cu_out = kv_append(pairs, cu_old, cu_new, heads=h_kv, rows_old=t_old, rows_new=t_new)
        k_out = outs[0]
        v_out = None if entry.is_mla else outs[1]
        self._layer_kv[key] = LayerKVEntry(
            k_cache=k_out,
            v_cache=v_out,
            total_context_len=rows,
            cu_seqlens_kv=cu_out,
            context_batch_size=entry.context_batch_size,
            is_mla=entry.is_mla,
            num_heads=entry.num_heads,
            head_dim=d,
            dtype=entry.dtype,
            device=dev,
        )

    def get_kv_cache(
        self,
        layer_id: int | str,
        *,
        is_mla: bool,
        num_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> LayerKVEntry:
        """Return the entry of ``layer_id``; ValueError if absent or of another shape/mode."""
        entry = self._layer_kv.get(self._layer_key(layer_id))
        if entry is None:
            raise ValueError(f"No cached KV context for layer_id={layer_id}")
        checks = (
            (entry.is_mla == is_mla, "Cached KV mode (is_mla) does not match request"),
            (entry.num_heads == num_heads, "Cached num_heads does not match request"),
            (entry.head_dim == head_dim, "Cached head_dim does not match request"),
            (entry.dtype == dtype, "Cached KV dtype does not match request"),
            (entry.device == device, "Cached KV device does not match request"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)
        return entry

    def layer_entry(self, layer_id: int | str) -> LayerKVEntry | None:
        """The entry of ``layer_id`` as stored, or None (no shape or mode checks)."""
        return self._layer_kv.get(self._layer_key(layer_id))

    def clear_layer(self, layer_id: int | str) -> None:
        self._layer_kv.pop(self._layer_key(layer_id), None)

    def clear(self) -> None:
        self.packing.clear()
        self._layer_kv.clear()
