"""Launchers of the fused MLM attention path on MI355X.

Public signatures, argument meaning, cache/prefill semantics and ValueError
messages follow src/flash_mlm/host/host.py of the reference:
  flash_attn_mlm                (host.py:47-225)
  flash_attn_mlm_compressed     (host.py:228-530)
  flash_attn_mlm_precompressed  (host.py:533-789)

What changes is below the API: one HIP kernel (fmlm_attn_fwd, C ABI in
include/flash_mlm_hip.h) reads the padded [B, H, N, D] q/k/v directly through
(sequence, head, position) addressing, so the compressed path does not pack
q/k/v at all unless prefill asks for a packed cache entry; the output is written
straight into the packed [H*T, D] result (no unpad copy).  ``block_m`` /
``block_n`` / ``auto_tune_tiles`` keep their role in the metadata contract and in
the padded prefill length; the HIP kernel picks its own tiles from the head dim.
"""

from __future__ import annotations

import threading
import warnings
import weakref

import torch

from flash_mlm import _lib
from flash_mlm.host.cache import PAGE_ROWS, InferenceCache, PackMetadata
from flash_mlm.host.host_utils import (
    _compute_total_q_len_padded,
    _device_scope,
    _maybe_get_cache_context,
    _pack_rows,
    make_contiguous,
    require_cuda_tensors,
    validate_cache_request,
    validate_cu_seqlens_rank1_min2,
    validate_head_dim_supported,
    validate_packed_cache_shapes,
    validate_qkv_same_shape_rank4,
)

# largest BLOCK_M the reference's autotuner may pick (mlm_kernel.py:114); it sets the
# padded prefill length when auto_tune_tiles=True (host.py:326)
_AUTOTUNE_MAX_BLOCK_M = 128

# fmlm_attn_params.tile_config of every launch: 0 lets the library choose the kernel's
# tile from the head dim and the work; k >= 1 forces compiled configuration k (tests and
# tuning sweeps; see tile_config())
_TILE_CONFIG = 0


class tile_config:
    """Force the attention kernel's tile configuration ``k`` (the library's k-th compiled
    configuration of the head dim, include/flash_mlm_hip.h) for the calls made inside the
    ``with`` block; ``k = 0`` restores the library's own choice.  A tuning and testing aid,
    like the reference's per-shape autotune configs (mlm_kernel.py:57-166)."""

    def __init__(self, k: int):
        self.k = int(k)

    def __enter__(self):
        global _TILE_CONFIG
        self.prev, _TILE_CONFIG = _TILE_CONFIG, self.k
        return self

    def __exit__(self, *exc):
        global _TILE_CONFIG
        _TILE_CONFIG = self.prev
        return False


def _aligned(t: torch.Tensor) -> bool:
    """Row-addressable by the kernel: unit stride in D, 16-byte aligned rows."""
    if t.numel() == 0:
        return True
    es = t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t if _aligned(t) else t.contiguous()


def _workspace(inference_cache: InferenceCache | None, nbytes: int, device: torch.device):
    if nbytes <= 0:
        return None
    if inference_cache is not None:
        return inference_cache.packing.get_2d("fmlm:attn_workspace", 1, nbytes, dtype=torch.uint8, device=device)
    return torch.empty((1, nbytes), dtype=torch.uint8, device=device)


# Set while a forward runs whose backward will follow (_Attention.forward): the launch
# then has the kernels store each row's log2-sum-exp, which the backward reads instead of
# recomputing it.
_ROW_STATS = threading.local()


class AttnLaunch:
    """A prepared fmlm_attn_fwd call: the parameter block plus the tensors it points to."""

    __slots__ = ("lib", "params", "stream", "device", "keep", "unpack_kv", "lse")

    def __init__(self, lib, params, stream, device, keep):
        self.lib, self.params, self.stream, self.device, self.keep = lib, params, stream, device, keep
        # (B, N, H, kv_heads, rows, cu_q) when the kernel read packed copies of padded
        # K/V (causal_query_seq_attn): the backward unpacks their gradient
        self.unpack_kv = None
        self.lse = None  # the row statistics of the last run, when it stored them

    def __call__(self) -> None:
        p = self.params
        # every run sets the field: a parameter block copied from a memo must not carry
        # an earlier call's buffer
        self.lse = None
        p.lse = None
        if getattr(_ROW_STATS, "on", False) and p.H > 0 and p.total_q > 0:
            self.lse = torch.empty(p.H * p.total_q, dtype=torch.float32, device=self.device)
            p.lse = self.lse.data_ptr()
        with _device_scope(self.device):
            rc = self.lib.fmlm_attn_fwd(p, self.stream)
        _lib.check(rc, "fmlm_attn_fwd")


def _launch(*, run: bool = True, **kw) -> AttnLaunch:
    plan = _prepare(**kw)
    if run:
        plan()
    return plan


# ---------------------------------------------------------------------------
# Launch memo.  A call that matches an earlier one in everything its checks and its
# parameter block depend on (the q/k/v pointers, shapes, strides, dtype and device, the
# arguments, the cached layer entry, the tile configuration) reuses that call's parameter
# block: it allocates the output, re-packs K/V where the call packs them, and launches,
# skipping the Python-side validation and the ~45 field writes of the block.  The cache
# replaces a layer's entry on prefill and append, never mutating it, so the entry object
# stands for its contents; the memo refers to it (and to the cache) weakly and holds no
# input tensor, only the small index tensors the call derived (int32 offsets, an empty
# context's zero offsets).  Compressed calls keep their memo on the PackMetadata, dense
# calls in a module-level table.
# ---------------------------------------------------------------------------
_MEMO_MAX = 16
_DENSE_MEMO: dict = {}


def _tkey(t: torch.Tensor):
    return (t.data_ptr(), t.shape, t.stride(), t.dtype, t.get_device())


class _Memo:
    __slots__ = ("params", "entry_ref", "extra", "out_shape", "repack", "unpack_kv")

    def __init__(self, plan: AttnLaunch, entry, extra, out_shape, repack=None):
        self.params = _lib.AttnParams.from_buffer_copy(plan.params)
        self.entry_ref = None if entry is None else weakref.ref(entry)
        self.extra, self.out_shape, self.repack, self.unpack_kv = extra, out_shape, repack, plan.unpack_kv


def _entry_of(inference_cache: InferenceCache | None, layer_id):
    if inference_cache is None or layer_id is None:
        return None
    return inference_cache.layer_entry(layer_id)


def _memo_lookup(memo: dict, key, entry) -> _Memo | None:
    m = memo.get(key)
    if m is None:
        return None
    if (m.entry_ref() if m.entry_ref is not None else None) is not entry:
        return None
    return m


def _memo_store(memo: dict, key, m: _Memo) -> None:
    if len(memo) >= _MEMO_MAX:
        memo.clear()
    memo[key] = m


def _memo_run(m: _Memo, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, entry):
    """Run a memoised call on this call's q/k/v (the same tensors, by the memo key)."""
    out = torch.empty(m.out_shape, dtype=q.dtype, device=q.device)
    p = _lib.AttnParams.from_buffer_copy(m.params)
    p.o = out.data_ptr()
    keep = [q, out, k, v, m.extra]
    if entry is not None:
        keep.append((entry.k_cache, entry.v_cache, entry.cu_seqlens_kv, entry.block_table))
    if m.repack is not None:
        packed = m.repack(k, v)
        if packed is None:
            return None
        k_pk, v_pk = packed
        p.k, p.v = k_pk.data_ptr(), v_pk.data_ptr()
        keep.append(packed)
    plan = AttnLaunch(_lib.load(), p, _lib.stream_of(q.device), q.device, tuple(keep))
    plan.unpack_kv = m.unpack_kv
    plan()
    return out, plan


# ---------------------------------------------------------------------------
# Backward (an extension: the reference's roadmap lists backpropagation,
# README.md:26-28).  Each entry point is differentiable in q, k, v and the cached
# context tensors: the forward runs as before inside an autograd Function, and its
# backward runs fmlm_attn_bwd on the forward's own parameter block.
# ---------------------------------------------------------------------------
_BWD_HEAD_DIMS = (16, 32, 64, 128, 256, 512)


def _cache_tensors(inference_cache, layer_id, prefill: bool):
    """The cached context tensors a call reads, (None, None) without a context."""
    if prefill or inference_cache is None or layer_id is None:
        return None, None, None
    entry = inference_cache.layer_entry(layer_id)
    if entry is None:
        return None, None, None
    return entry.k_cache, entry.v_cache, entry


def _wants_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


def _backward_unsupported(q: torch.Tensor, d: int, entry, is_mla: bool) -> str | None:
    """Why this call has no backward, or None (every head dim the forward runs has one)."""
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        return "the attention backward needs bf16, fp16 or fp32 inputs"
    if d not in _BWD_HEAD_DIMS:
        return "the attention backward supports head_dim 16, 32, 64, 128, 256 or 512"
    return None


def _run(impl, q, k, v, inference_cache, layer_id, prefill: bool, is_mla: bool):
    """Run one attention call, through autograd when an input requires grad.  A call
    without a backward (see _backward_unsupported) returns its output without a graph,
    as the reference's kernels do, and warns that no gradient will flow.  ``impl(owned)``
    runs the forward; ``owned`` asks it to keep every tensor the kernel reads in buffers
    of its own rather than the cache's reusable packing buffers, which a later call may
    overwrite before this call's backward runs."""
    kc, vc, entry = _cache_tensors(inference_cache, layer_id, prefill)
    if not _wants_grad(q, k, v, kc, vc):
        return impl(False)[0]
    why = _backward_unsupported(q, int(q.shape[-1]), entry, is_mla)
    if why is not None:
        warnings.warn(f"flash_mlm: {why}; the output carries no gradient", stacklevel=3)
        return impl(False)[0]
    return _Attention.apply(lambda: impl(True), q, k, v, kc, vc)


class _Attention(torch.autograd.Function):
    """One attention call made differentiable: ``impl()`` runs the forward and returns
    (out, prepared launch); the backward hands that launch's parameter block to
    fmlm_attn_bwd."""

    @staticmethod
    def forward(ctx, impl, q, k, v, k_cache, v_cache):
        _ROW_STATS.on = True
        try:
            out, plan = impl()
        finally:
            _ROW_STATS.on = False
        ctx.plan = plan
        # saved so that autograd rejects a backward after any of them changed in place
        ctx.save_for_backward(out, q, k, v, k_cache, v_cache)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout):
        out = ctx.saved_tensors[0]
        if ctx.plan is None:
            return (None,) * 6
        want_ctx = ctx.needs_input_grad[4] or ctx.needs_input_grad[5]
        dq, dk, dv, dkc, dvc = _attention_backward(ctx.plan, out, dout, want_ctx)
        return None, dq, dk, dv, dkc, dvc


def _attention_backward(plan: AttnLaunch, out: torch.Tensor, dout: torch.Tensor, want_ctx: bool):
    """Gradients (dq, dk, dv, dk_cache, dv_cache) of the prepared call ``plan`` whose
    output is ``out``, shaped like the caller's tensors (dv None for MLA: V is K and both
    gradients are in dk)."""
    g, (dq, dk, dv, dkc, dvc, _ws, _dout) = _backward_args(plan, out, dout, want_ctx)
    with _device_scope(out.device):
        rc = plan.lib.fmlm_attn_bwd(plan.params, g, plan.stream)
    _lib.check(rc, "fmlm_attn_bwd")
    if plan.unpack_kv is not None:
        mla = bool(plan.params.flags & _lib.FLAG_MLA)
        dk = _unpack_kv_grad(plan.lib, dk, plan, mla)
        dv = None if mla else _unpack_kv_grad(plan.lib, dv, plan, mla)
    if plan.params.ctx_block_table:  # float32 accumulation -> the pool's dtype
        dkc = None if dkc is None else dkc.to(out.dtype)
        dvc = None if dvc is None else dvc.to(out.dtype)
    return dq, dk, dv, dkc, dvc


def _backward_args(plan: AttnLaunch, out: torch.Tensor, dout: torch.Tensor, want_ctx: bool):
    """The fmlm_attn_grads block of one backward call and the tensors it points to:
    zeroed gradients shaped like the tensors the kernel read, the workspace and dout."""
    p, lib = plan.params, plan.lib
    q_, _, k_, v_, k_ctx, v_ctx = plan.keep[:6]
    mla = bool(p.flags & _lib.FLAG_MLA)
    prefill = bool(p.flags & _lib.FLAG_PREFILL)
    dout = dout.contiguous()
    if dout.shape != out.shape or not out.is_contiguous():
        raise ValueError("gradient of the attention output has the wrong shape")

    def grad_of(x: torch.Tensor, strides):
        gx = torch.zeros(x.shape, dtype=x.dtype, device=x.device)
        if x.ndim == 4:  # padded [B, H, N, D]; head stride 0 = rows shared by all heads
            return gx, (gx.stride(0), 0 if strides[1] == 0 else gx.stride(1), gx.stride(2))
        return gx, strides  # packed rows of a contiguous tensor

    g = _lib.AttnGrads()
    g.dout = dout.data_ptr()
    g.do_sb, g.do_sh, g.do_sn = p.o_sb, p.o_sh, p.o_sn
    dq, (g.dq_sb, g.dq_sh, g.dq_sn) = grad_of(q_, (p.q_sb, p.q_sh, p.q_sn))
    dk, (g.dk_sb, g.dk_sh, g.dk_sn) = grad_of(k_, (p.k_sb, p.k_sh, p.k_sn))
    g.dq, g.dk = dq.data_ptr(), dk.data_ptr()
    dv = None
    if not mla:
        dv, (g.dv_sb, g.dv_sh, g.dv_sn) = grad_of(v_, (p.v_sb, p.v_sh, p.v_sn))
        g.dv = dv.data_ptr()
    dkc = dvc = None
    if want_ctx and not prefill and k_ctx is not None and k_ctx.numel():
        # a paged context's gradient is accumulated in float32 (a page can serve several
        # context batches); _attention_backward rounds it to the cache dtype
        acc = torch.float32 if p.ctx_block_table else k_ctx.dtype
        dkc = torch.zeros(k_ctx.shape, dtype=acc, device=k_ctx.device)
        g.dk_ctx = dkc.data_ptr()
        if not mla:
            dvc = torch.zeros(v_ctx.shape, dtype=acc, device=v_ctx.device)
            g.dv_ctx = dvc.data_ptr()
    nbytes = int(lib.fmlm_attn_bwd_workspace_bytes(p))
    _lib.check(nbytes if nbytes < 0 else 0, "fmlm_attn_bwd_workspace_bytes")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=out.device)
    g.workspace, g.workspace_bytes = ws.data_ptr(), nbytes
    return g, (dq, dk, dv, dkc, dvc, ws, dout)


def _unpack_kv_grad(lib, packed: torch.Tensor, plan: AttnLaunch, mla: bool) -> torch.Tensor:
    """Gradient rows of packed K/V [kv_heads * rows, D] -> padded [B, H, N, D] (MLA: head 0)."""
    B, N, H, kv_heads, rows, cu_q = plan.unpack_kv
    D = int(packed.shape[1])
    dst = torch.empty((B, kv_heads, N, D), dtype=packed.dtype, device=packed.device)
    if dst.numel():
        with _device_scope(packed.device):
            rc = lib.fmlm_unpack(packed.element_size(), packed.data_ptr(), rows * D, dst.data_ptr(), B, kv_heads,
                                 N, D, cu_q.data_ptr(), plan.stream)
        _lib.check(rc, "fmlm_unpack")
    if mla and H > 1:
        full = torch.zeros((B, H, N, D), dtype=packed.dtype, device=packed.device)
        full[:, :1] = dst
        return full
    return dst


def _prepare(
    *,
    q: torch.Tensor,
    out: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor | None,
    B: int,
    H: int,
    D: int,
    N: int,
    total_q: int,
    cu_seqlens_q: torch.Tensor | None,
    q_strides: tuple[int, int, int],
    q_layout: int,
    o_strides: tuple[int, int, int],
    o_layout: int,
    k_strides: tuple[int, int, int],
    v_strides: tuple[int, int, int],
    kv_layout: int,
    k_ctx: torch.Tensor,
    v_ctx: torch.Tensor | None,
    c_strides: tuple[int, int, int],
    cu_seqlens_kv: torch.Tensor | None,
    ctx_len: int,
    ctx_batch: int,
    ctx_rows: int,
    scale: float,
    flags: int,
    inference_cache: InferenceCache | None,
    schedule_cache: dict | None = None,
    ctx_index: torch.Tensor | None = None,
    block_table: torch.Tensor | None = None,
    page_stride: int = 0,
) -> AttnLaunch:
    lib = _lib.load()
    p = _lib.AttnParams()
    p.dtype = _lib.dtype_code(q.dtype)
    p.flags = flags
    p.tile_config = _TILE_CONFIG
    p.B, p.H, p.D, p.N = B, H, D, N
    p.total_q = total_q
    p.ctx_len = ctx_len
    p.ctx_batch = ctx_batch
    p.ctx_rows = ctx_rows
    p.q_layout, p.o_layout, p.kv_layout = q_layout, o_layout, kv_layout
    p.scale = float(scale)
    p.cu_seqlens_q = _lib.ptr(cu_seqlens_q)
    p.cu_seqlens_kv = _lib.ptr(cu_seqlens_kv)
    p.ctx_index = _lib.ptr(ctx_index)
    p.ctx_block_table = _lib.ptr(block_table)
    if block_table is not None:
        p.ctx_page_stride = page_stride
        p.ctx_pages_per_batch = int(block_table.shape[1])
    p.q = q.data_ptr()
    p.q_sb, p.q_sh, p.q_sn = q_strides
    p.o = out.data_ptr()
    p.o_sb, p.o_sh, p.o_sn = o_strides
    p.k = k.data_ptr()
    p.k_sb, p.k_sh, p.k_sn = k_strides
    p.v = (v if v is not None else k).data_ptr()
    p.v_sb, p.v_sh, p.v_sn = v_strides
    p.k_ctx = k_ctx.data_ptr() if k_ctx.numel() else None
    p.v_ctx = v_ctx.data_ptr() if (v_ctx is not None and v_ctx.numel()) else p.k_ctx
    p.c_sb, p.c_sh, p.c_sn = c_strides
    ws_bytes = int(lib.fmlm_attn_workspace_bytes(p))
    _lib.check(ws_bytes if ws_bytes < 0 else 0, "fmlm_attn_workspace_bytes")
    stream = _lib.stream_of(q.device)
    with _device_scope(q.device):
        if ws_bytes > 0 and schedule_cache is not None:
            # what the unit list depends on: the kernel (dtype, head dim, flags, K/V
            # layout, paged context or not), whose tile size and occupancy fix the slots,
            # the split records and the grid, and the shape (B, H, N, total_q); context
            # lengths only steer where key ranges are split
            key = (p.dtype, D, B, H, N, total_q, p.flags, p.kv_layout, block_table is not None, p.tile_config)
            sched = schedule_cache.get(key)
            if sched is None:
                sched = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
                _lib.check(lib.fmlm_attn_schedule(p, sched.data_ptr(), ws_bytes, stream), "fmlm_attn_schedule")
                schedule_cache[key] = sched
            p.schedule = sched.data_ptr()
            ws = None
        else:
            sched = None
            ws = _workspace(inference_cache, ws_bytes, q.device)
            p.workspace = None if ws is None else ws.data_ptr()
            p.workspace_bytes = ws_bytes
    keep = (q, out, k, v, k_ctx, v_ctx, cu_seqlens_q, cu_seqlens_kv, ctx_index, block_table, ws, sched)
    return AttnLaunch(lib, p, stream, q.device, keep)


def _check_cache_dtype(k_cache: torch.Tensor, q: torch.Tensor) -> None:
    if k_cache.numel() and k_cache.dtype != q.dtype:
        raise ValueError("cached context dtype must match q dtype")


def _context_index(context_index, *, b: int, cbs: int, prefill: bool, context_batch_size, device):
    """Index-mapped context batching: sequence b attends to context batch
    ``context_index[b]`` of the layer's cached entry (any number of context batches).
    The reference supports only a shared or a full-batch context and lists this under
    "variable context batch sizes" on its roadmap (README.md:34-36).  Returns an int32
    copy on ``device``, or None.  A CPU index is range-checked here; a GPU index is not
    read back (no host sync) and the kernel clamps it to [0, cbs)."""
    if context_index is None:
        return None
    if prefill:
        raise ValueError("context_index cannot be combined with prefill=True")
    if context_batch_size is not None:
        raise ValueError("context_index and context_batch_size are mutually exclusive")
    if not isinstance(context_index, torch.Tensor) or context_index.ndim != 1 or context_index.numel() != b:
        raise ValueError("context_index must be a rank-1 tensor with one entry per sequence")
    if context_index.dtype not in (torch.int32, torch.int64):
        raise ValueError("context_index must be an int32 or int64 tensor")
    if not context_index.is_cuda and context_index.numel():
        lo, hi = int(context_index.min()), int(context_index.max())
        if lo < 0 or hi >= cbs:
            raise ValueError(f"context_index values must lie in [0, {cbs})")
    return context_index.to(device=device, dtype=torch.int32).contiguous()


def flash_attn_mlm(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    inference_cache: InferenceCache | None = None,
    layer_id: int | str | None = None,
    is_mla: bool = False,
    context_batch_size: int | None = None,
    block_m: int = 64,
    block_n: int = 32,
    auto_tune_tiles: bool = False,
    prefill: bool = False,
    context_index: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dense MLM attention: q, k, v [B, H, N, D] -> out [B, H, N, D].

    Every query attends (non-causally) to [cached context of its batch || all N keys
    of its (b, h)].  Cached context rows (``InferenceCache`` entry of ``layer_id``):
    MLA [context_batch * context_len, D] shared by all heads, otherwise
    [context_batch, H, context_len, D] flattened; ``context_batch_size`` 1 shares
    batch 0.  MLA keeps per-head main keys and uses V = K.  ``prefill=True`` skips
    the context and afterwards stores this call's K/V (MLA: head 0 of k) as the
    layer's new context with context_batch_size = B.  ``context_index`` (int [B], an
    extension) maps sequence b to cached context batch ``context_index[b]``.
    """
    def impl(owned: bool):
        return _dense_impl(
            q, k, v, scale, inference_cache, layer_id, is_mla, context_batch_size, prefill,
            context_index=context_index,
        )

    return _run(impl, q, k, v, inference_cache, layer_id, prefill, is_mla)


def _dense_impl(
    q, k, v, scale, inference_cache, layer_id, is_mla, context_batch_size, prefill, run=True, context_index=None
):
    """Body of :func:`flash_attn_mlm`; returns (out, prepared launch or None)."""
    memo_key = entry = None
    if run and not prefill and context_index is None and isinstance(q, torch.Tensor):
        entry = _entry_of(inference_cache, layer_id)
        memo_key = (_tkey(q), _tkey(k), _tkey(v), float(scale), is_mla, context_batch_size, _TILE_CONFIG,
                    None if entry is None else id(entry))
        m = _memo_lookup(_DENSE_MEMO, memo_key, entry)
        if m is not None:
            return _memo_run(m, q, k, v, entry)
    b, h, n, d = validate_qkv_same_shape_rank4(q, k, v, error_prefix="q/k/v")
    validate_cache_request(prefill=prefill, inference_cache=inference_cache, layer_id=layer_id)
    ctx = _maybe_get_cache_context(
        inference_cache=inference_cache,
        layer_id=layer_id,
        batch_size=b,
        is_mla=is_mla,
        num_heads=h,
        head_dim=d,
        context_batch_size=context_batch_size,
        dtype=q.dtype,
        device=q.device,
        compressed=False,
    )
    k_cache, v_cache = ctx.k_cache, ctx.v_cache
    cbs, context_len = ctx.context_batch_size, ctx.context_len

    require_cuda_tensors(q, k, v, k_cache, v_cache)
    if cbs is None or cbs < 1:
        raise ValueError("context_batch_size must be >= 1")
    validate_head_dim_supported(d, is_mla=is_mla)
    ctx_index = _context_index(
        context_index, b=b, cbs=cbs, prefill=prefill, context_batch_size=context_batch_size, device=q.device
    )
    if cbs > 1 and cbs < b and not prefill and context_len > 0 and ctx_index is None:
        raise ValueError("context_batch_size must be 1 or at least the batch size")
    _check_cache_dtype(k_cache, q)

    q_, k_, v_ = _rows(q), _rows(k), _rows(v)
    k_cache, v_cache = make_contiguous(k_cache, v_cache)
    out = torch.empty((b, h, n, d), dtype=q.dtype, device=q.device)

    # dense context layout (mlm_kernel_impl.py:132-141)
    if is_mla:
        c_strides = (context_len * d, 0, d)
    else:
        c_strides = (h * context_len * d, context_len * d, d)
    flags = (_lib.FLAG_MLA if is_mla else 0) | (_lib.FLAG_PREFILL if prefill else 0)
    plan = None
    if b * h * n > 0:
        plan = _launch(
            run=run,
            q=q_,
            out=out,
            k=k_,
            v=None if is_mla else v_,
            B=b,
            H=h,
            D=d,
            N=n,
            total_q=b * n,
            cu_seqlens_q=None,
            q_strides=(q_.stride(0), q_.stride(1), q_.stride(2)),
            q_layout=_lib.LAYOUT_PADDED,
            o_strides=(out.stride(0), out.stride(1), out.stride(2)),
            o_layout=_lib.LAYOUT_PADDED,
            k_strides=(k_.stride(0), k_.stride(1), k_.stride(2)),
            v_strides=(k_.stride(0), k_.stride(1), k_.stride(2))
            if is_mla
            else (v_.stride(0), v_.stride(1), v_.stride(2)),
            kv_layout=_lib.LAYOUT_PADDED,
            k_ctx=k_cache,
            v_ctx=None if is_mla else v_cache,
            c_strides=c_strides,
            cu_seqlens_kv=None,
            ctx_len=context_len,
            ctx_batch=cbs,
            ctx_rows=context_len,
            scale=scale,
            flags=flags,
            inference_cache=inference_cache,
            ctx_index=ctx_index,
        )
        # memoised when the launch reads the caller's tensors and the entry's own
        if (memo_key is not None and q_ is q and k_ is k and v_ is v and k_cache is ctx.k_cache
                and v_cache is ctx.v_cache and plan.keep[10] is None):
            extra = None if entry is not None else (k_cache, v_cache)  # an empty context's tensors
            _memo_store(_DENSE_MEMO, memo_key, _Memo(plan, entry, extra, tuple(out.shape)))

    if prefill and inference_cache is not None:
        # the dense entry stores this call's K/V with context_len = N per batch (host.py:206-223)
        if is_mla:
            k_prefill = torch.empty((b * n, d), dtype=k.dtype, device=k.device)
            if k_prefill.numel():
                _pack_rows(
                    [(k[:, :1], 1)], [k_prefill], cu_seqlens=None, B=b, N=n, D=d, total=b * n, total_padded=b * n
                )
            v_prefill = k_prefill
        else:
            k_prefill = k.contiguous().view(b * h * n, d)
            v_prefill = v.contiguous().view(b * h * n, d)
        inference_cache.prefill_kv_cache(
            layer_id,
            k_cache=k_prefill,
            v_cache=v_prefill,
            context_batch_size=int(b),
            is_mla=is_mla,
            num_heads=h,
            head_dim=d,
        )
    return out, plan


def _ctx_rows(ctx) -> int:
    """The kernel's ctx_rows: rows per head of a packed context, or pages of a paged pool."""
    total = int(ctx.total_context_len)
    return total // PAGE_ROWS if ctx.block_table is not None else total


def _page_stride(ctx, num_heads: int, d: int, is_mla: bool) -> int:
    """Elements between pages of a paged pool [H_kv, P, PAGE_ROWS, D] (0 when not paged)."""
    return 0 if ctx.block_table is None else PAGE_ROWS * d


def _packed_context(ctx, *, num_heads: int, d: int, is_mla: bool, b: int, prefill: bool, indexed: bool = False):
    """Strides / sizes of a packed (head-major) context entry, validated."""
    total_context_len = int(ctx.total_context_len)
    cu_kv = ctx.cu_seqlens_kv
    cbs = ctx.context_batch_size
    if cbs is None:
        cbs = int(cu_kv.numel() - 1)
    if cbs < 1:
        raise ValueError("context_batch_size must be >= 1")
    if cbs + 1 > cu_kv.numel():
        raise ValueError("context_batch_size is incompatible with cu_seqlens_kv length")
    if 1 < cbs < b and not prefill and total_context_len > 0 and not indexed:
        raise ValueError("context_batch_size must be 1 or at least the batch size")
    if ctx.block_table is not None:  # paged pool [H_kv, P, PAGE_ROWS, D]: heads total_context_len rows apart
        return cbs, (0, 0 if is_mla else total_context_len * d, d)
    c_strides = (0, 0 if is_mla else total_context_len * d, d)
    return cbs, c_strides


def flash_attn_mlm_compressed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    num_heads: int,
    q_meta: PackMetadata,
    scale: float,
    inference_cache: InferenceCache | None = None,
    layer_id: int | str | None = None,
    is_mla: bool = False,
    context_batch_size: int | None = None,
    block_m: int = 64,
    block_n: int = 32,
    auto_tune_tiles: bool = False,
    prefill: bool = False,
    causal_query_seq_attn: bool = False,
    context_index: torch.Tensor | None = None,
) -> torch.Tensor:
    """Packed variable-length MLM attention over padded q/k/v [B, H, N, D].

    Query token t < L_b of sequence b attends to [its cached context
    cu_seqlens_kv[cb]..cu_seqlens_kv[cb+1] || main keys], main keys being the tokens of
    sequence b, or with ``causal_query_seq_attn`` the packed tokens of sequences 0..b.
    Returns the packed output [H * T, D] (T = q_meta.total_tokens, head-major).
    MLA: main K = V = head 0 of k (``v`` is ignored), context is a shared latent.
    ``prefill=True`` skips the context and stores this call's packed, zero-padded
    K/V [H_kv * T_pad, D] as the layer's context (cu_seqlens_kv = q_meta.cu_seqlens,
    context_batch_size = B) before the attention runs.  ``context_index`` (int [B], an
    extension) maps sequence b to cached context batch ``context_index[b]`` instead.
    """
    def impl(owned: bool):
        return _compressed_impl(
            q, k, v, num_heads, q_meta, scale, inference_cache, layer_id, is_mla, context_batch_size,
            block_m, block_n, auto_tune_tiles, prefill, causal_query_seq_attn, context_index=context_index,
            owned_buffers=owned,
        )

    return _run(impl, q, k, v, inference_cache, layer_id, prefill, is_mla)


def _compressed_impl(
    q, k, v, num_heads, q_meta, scale, inference_cache, layer_id, is_mla, context_batch_size,
    block_m, block_n, auto_tune_tiles, prefill, causal_query_seq_attn, run=True, context_index=None,
    owned_buffers=False,
):
    """Body of :func:`flash_attn_mlm_compressed`; returns (out, prepared launch or None)."""
    memo = memo_key = entry = None
    if (run and not prefill and not owned_buffers and context_index is None and isinstance(q_meta, PackMetadata)
            and isinstance(q, torch.Tensor)):
        memo = q_meta.launch_memo
        entry = _entry_of(inference_cache, layer_id)
        memo_key = (_tkey(q), _tkey(k), _tkey(v), num_heads, float(scale), is_mla, context_batch_size, block_m,
                    block_n, auto_tune_tiles, causal_query_seq_attn, _TILE_CONFIG,
                    None if entry is None else id(entry), inference_cache is None)
        m = _memo_lookup(memo, memo_key, entry)
        if m is not None:
            res = _memo_run(m, q, k, v, entry)
            if res is not None:
                return res
    b, h, n, d = validate_qkv_same_shape_rank4(q, k, v, error_prefix="q/k/v")
    if h != num_heads:
        raise ValueError("q/k/v head dimension must match num_heads")
    validate_cache_request(prefill=prefill, inference_cache=inference_cache, layer_id=layer_id)
    if q_meta.B != b or q_meta.N != n:
        raise ValueError("q_meta shape metadata does not match q/k/v padded shape")
    if q_meta.batch_ids_block_n != block_n:
        raise ValueError("q_meta was built with different block_n")
    cu_seqlens_q = q_meta.cu_seqlens
    T = int(q_meta.total_tokens)

    ctx = _maybe_get_cache_context(
        inference_cache=inference_cache,
        layer_id=layer_id,
        batch_size=b,
        is_mla=is_mla,
        num_heads=num_heads,
        head_dim=d,
        context_batch_size=context_batch_size,
        dtype=q.dtype,
        device=q.device,
        compressed=True,
    )
    require_cuda_tensors(q, k, v, ctx.k_cache, ctx.v_cache, ctx.cu_seqlens_kv)
    if not (q_meta.batch_ids_q.is_cuda and cu_seqlens_q.is_cuda):
        raise ValueError("batch_ids_q and cu_seqlens_q must be CUDA tensors")
    if num_heads < 1:
        raise ValueError("num_heads must be >= 1")
    validate_packed_cache_shapes(
        ctx.k_cache,
        ctx.v_cache,
        num_heads=num_heads,
        total_context_len=int(ctx.total_context_len),
        head_dim=d,
        is_mla=is_mla,
    )
    validate_head_dim_supported(d, is_mla=is_mla)
    validate_cu_seqlens_rank1_min2(cu_seqlens_q, ctx.cu_seqlens_kv)
    cbs, c_strides = _packed_context(
        ctx, num_heads=num_heads, d=d, is_mla=is_mla, b=b, prefill=prefill, indexed=context_index is not None
    )
    ctx_index = _context_index(
        context_index, b=b, cbs=cbs, prefill=prefill, context_batch_size=context_batch_size, device=q.device
    )
    num_q_tiles = int(q_meta.q_tile_starts_q.numel())
    if q_meta.batch_ids_q.ndim != 1 or q_meta.batch_ids_q.numel() != num_q_tiles:
        raise ValueError("batch_ids_q must be rank-1 with exactly one entry per query tile")
    if q_meta.q_tile_starts_q.ndim != 1:
        raise ValueError("q_tile_starts_q must be rank-1")
    _check_cache_dtype(ctx.k_cache, q)

    packed_kv = None  # (k, v, rows per head) of a packed copy of this call's K/V
    if prefill and inference_cache is not None:
        # packed, zero-padded K/V written straight into the layer's named workspace and
        # stored (as views) before the launch (host.py:326-364)
        pad_block_m = _AUTOTUNE_MAX_BLOCK_M if auto_tune_tiles else block_m
        T_pad = _compute_total_q_len_padded(T, q_meta.host_cu_seqlens(), pad_block_m, block_n)
        key = str(layer_id)
        kv_heads = 1 if is_mla else num_heads
        packing = inference_cache.packing
        k_entry = packing.get_2d(f"layer:{key}:k_cache", kv_heads * T_pad, d, dtype=k.dtype, device=k.device)
        if is_mla:
            v_entry = k_entry
            sources, outs = [(k[:, :1], 1)], [k_entry]
        else:
            v_entry = packing.get_2d(f"layer:{key}:v_cache", kv_heads * T_pad, d, dtype=v.dtype, device=v.device)
            sources, outs = [(k, num_heads), (v, num_heads)], [k_entry, v_entry]
        if T_pad > 0:
            _pack_rows(
                sources,
                outs,
                cu_seqlens=cu_seqlens_q.to(torch.int32).contiguous(),
                B=b,
                N=n,
                D=d,
                total=T,
                total_padded=T_pad,
            )
        inference_cache.prefill_kv_cache(
            layer_id,
            k_cache=k_entry,
            v_cache=None if is_mla else v_entry,
            total_context_len=int(T_pad),
            cu_seqlens_kv=cu_seqlens_q,
            context_batch_size=int(b),
            is_mla=is_mla,
            num_heads=num_heads,
            head_dim=d,
        )
        packed_kv = (k_entry, v_entry, T_pad)

    out = torch.empty((num_heads * T, d), dtype=q.dtype, device=q.device)
    if T == 0 or num_heads == 0:
        return out, None
    q_, k_, v_ = _rows(q), _rows(k), _rows(v)
    k_cache, v_cache = make_contiguous(ctx.k_cache, ctx.v_cache)
    cu_q = cu_seqlens_q.to(torch.int32).contiguous()
    cu_kv = ctx.cu_seqlens_kv.to(torch.int32).contiguous()
    kv_layout = _lib.LAYOUT_PADDED
    unpack_kv = None
    if causal_query_seq_attn:
        # the causal key range [0, cu[b+1]) spans sequences: pack K/V once (or reuse the
        # prefill entry) so the kernel streams it linearly
        if packed_kv is None:
            kv_heads = 1 if is_mla else num_heads

            def alloc(name: str) -> torch.Tensor:
                if inference_cache is None or owned_buffers:
                    return torch.empty((kv_heads * T, d), dtype=k.dtype, device=k.device)
                return inference_cache.packing.get_2d(name, kv_heads * T, d, dtype=k.dtype, device=k.device)

            k_pk = alloc("k")
            v_pk = k_pk if is_mla else alloc("v")
            sources = [(k_[:, :1], 1)] if is_mla else [(k_, num_heads), (v_, num_heads)]
            outs = [k_pk] if is_mla else [k_pk, v_pk]
            _pack_rows(sources, outs, cu_seqlens=cu_q, B=b, N=n, D=d, total=T, total_padded=T)
            packed_kv = (k_pk, v_pk, T)
        k_, v_, rows = packed_kv
        k_strides = v_strides = (0, 0 if is_mla else rows * d, d)
        kv_layout = _lib.LAYOUT_PACKED
        unpack_kv = (b, n, num_heads, 1 if is_mla else num_heads, rows, cu_q)
    elif is_mla:
        k_strides = (k_.stride(0), 0, k_.stride(2))  # every head reads head 0
        v_strides = k_strides
    else:
        k_strides = (k_.stride(0), k_.stride(1), k_.stride(2))
        v_strides = (v_.stride(0), v_.stride(1), v_.stride(2))
    flags = (
        (_lib.FLAG_MLA if is_mla else 0)
        | (_lib.FLAG_PREFILL if prefill else 0)
        | (_lib.FLAG_CAUSAL_SEQ if causal_query_seq_attn else 0)
    )
    plan = _launch(
        run=run,
        q=q_,
        out=out,
        k=k_,
        v=None if is_mla else v_,
        B=b,
        H=num_heads,
        D=d,
        N=n,
        total_q=T,
        cu_seqlens_q=cu_q,
        q_strides=(q_.stride(0), q_.stride(1), q_.stride(2)),
        q_layout=_lib.LAYOUT_PADDED,
        o_strides=(0, T * d, d),
        o_layout=_lib.LAYOUT_PACKED,
        k_strides=k_strides,
        v_strides=v_strides,
        kv_layout=kv_layout,
        k_ctx=k_cache,
        v_ctx=None if is_mla else v_cache,
        c_strides=c_strides,
        cu_seqlens_kv=cu_kv,
        ctx_len=0,
        ctx_batch=cbs,
        ctx_rows=_ctx_rows(ctx),
        scale=scale,
        flags=flags,
        inference_cache=inference_cache,
        schedule_cache=q_meta.kernel_schedules if isinstance(q_meta, PackMetadata) else None,
        ctx_index=ctx_index,
        block_table=ctx.block_table,
        page_stride=_page_stride(ctx, num_heads, d, is_mla),
    )
    plan.unpack_kv = unpack_kv
    if (memo_key is not None and q_ is q and k_cache is ctx.k_cache and v_cache is ctx.v_cache
            and plan.keep[10] is None and (causal_query_seq_attn or (k_ is k and v_ is v))):
        repack = None
        if causal_query_seq_attn:
            repack = _causal_repack(inference_cache, is_mla=is_mla, num_heads=num_heads, b=b, n=n, d=d, T=T,
                                    cu_q=cu_q)
        # the offsets the launch reads when they are not the metadata's or the entry's own
        extra = (cu_q, cu_kv, k_cache if entry is None else None, v_cache if entry is None else None)
        _memo_store(memo, memo_key, _Memo(plan, entry, extra, tuple(out.shape), repack))
    return out, plan


def _causal_repack(inference_cache, *, is_mla: bool, num_heads: int, b: int, n: int, d: int, T: int, cu_q):
    """The K/V pack of a memoised causal_query_seq_attn call: this call's padded K/V into
    the cache's packing buffers (fresh buffers without a cache), as the first call did.
    Returns None when the cache is gone (the memo entry then misses)."""
    cache_ref = None if inference_cache is None else weakref.ref(inference_cache)
    kv_heads = 1 if is_mla else num_heads

    def repack(k, v):
        cache = None
        if cache_ref is not None:
            cache = cache_ref()
            if cache is None:
                return None

        def alloc(name: str) -> torch.Tensor:
            if cache is None:
                return torch.empty((kv_heads * T, d), dtype=k.dtype, device=k.device)
            return cache.packing.get_2d(name, kv_heads * T, d, dtype=k.dtype, device=k.device)

        k_pk = alloc("k")
        v_pk = k_pk if is_mla else alloc("v")
        k_, v_ = _rows(k), _rows(v)
        sources = [(k_[:, :1], 1)] if is_mla else [(k_, num_heads), (v_, num_heads)]
        outs = [k_pk] if is_mla else [k_pk, v_pk]
        _pack_rows(sources, outs, cu_seqlens=cu_q, B=b, N=n, D=d, total=T, total_padded=T)
        return k_pk, v_pk

    return repack


def flash_attn_mlm_precompressed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    num_heads: int,
    total_q_len: int,
    cu_seqlens_q: torch.Tensor,
    batch_ids_q: torch.Tensor,
    q_tile_starts_q: torch.Tensor,
    scale: float,
    inference_cache: InferenceCache | None = None,
    layer_id: int | str | None = None,
    is_mla: bool = False,
    context_batch_size: int | None = None,
    block_m: int = 64,
    block_n: int = 32,
    auto_tune_tiles: bool = False,
    prefill: bool = False,
    causal_query_seq_attn: bool = False,
    context_index: torch.Tensor | None = None,
) -> torch.Tensor:
    """Like :func:`flash_attn_mlm_compressed` for already packed inputs.

    q [H*total_q_len, D]; k, v [total_q_len, D] (MLA) or [H*total_q_len, D], head-major
    with sequence b at rows cu_seqlens_q[b]..cu_seqlens_q[b+1] of each head.  Returns
    [H*total_q_len, D]; rows of padding tokens are left unwritten.  The kernel schedules
    its own tiles from ``cu_seqlens_q``; ``batch_ids_q`` / ``q_tile_starts_q`` are
    validated as in the reference.  ``prefill=True`` stores k / v (views) as the
    layer's context after the launch.
    """

    def impl(owned: bool):
        return _precompressed_impl(
            q, k, v, num_heads, total_q_len, cu_seqlens_q, batch_ids_q, q_tile_starts_q, scale, inference_cache,
            layer_id, is_mla, context_batch_size, prefill, causal_query_seq_attn, context_index,
        )

    return _run(impl, q, k, v, inference_cache, layer_id, prefill, is_mla)


def _precompressed_impl(
    q, k, v, num_heads, total_q_len, cu_seqlens_q, batch_ids_q, q_tile_starts_q, scale, inference_cache, layer_id,
    is_mla, context_batch_size, prefill, causal_query_seq_attn, context_index,
):
    """Body of :func:`flash_attn_mlm_precompressed`; returns (out, prepared launch or None)."""
    validate_cache_request(prefill=prefill, inference_cache=inference_cache, layer_id=layer_id)
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("q/k/v must be pre-packed rank-2 tensors")
    d = int(q.shape[1])
    if k.shape[1] != d or v.shape[1] != d:
        raise ValueError("q/k/v head_dim (dim 1) must match")
    if q.shape[0] != num_heads * total_q_len:
        raise ValueError("q first dim must equal num_heads * total_q_len")
    kv_rows = total_q_len if is_mla else num_heads * total_q_len
    if k.shape[0] != kv_rows or v.shape[0] != kv_rows:
        raise ValueError(f"k/v first dim mismatch: expected {kv_rows} rows for is_mla={is_mla}")
    b = int(cu_seqlens_q.numel()) - 1
    ctx = _maybe_get_cache_context(
        inference_cache=inference_cache,
        layer_id=layer_id,
        batch_size=b,
        is_mla=is_mla,
        num_heads=num_heads,
        head_dim=d,
        context_batch_size=context_batch_size,
        dtype=q.dtype,
        device=q.device,
        compressed=True,
    )
    require_cuda_tensors(q, k, v, ctx.k_cache, ctx.v_cache, ctx.cu_seqlens_kv)
    validate_packed_cache_shapes(
        ctx.k_cache,
        ctx.v_cache,
        num_heads=num_heads,
        total_context_len=int(ctx.total_context_len),
        head_dim=d,
        is_mla=is_mla,
    )
    validate_head_dim_supported(d, is_mla=is_mla)
    validate_cu_seqlens_rank1_min2(cu_seqlens_q, ctx.cu_seqlens_kv)
    cbs, c_strides = _packed_context(
        ctx, num_heads=num_heads, d=d, is_mla=is_mla, b=b, prefill=prefill, indexed=context_index is not None
    )
    ctx_index = _context_index(
        context_index, b=b, cbs=cbs, prefill=prefill, context_batch_size=context_batch_size, device=q.device
    )
    num_q_tiles = int(q_tile_starts_q.numel())
    if batch_ids_q.ndim != 1 or batch_ids_q.numel() != num_q_tiles:
        raise ValueError("batch_ids_q must be rank-1 with exactly one entry per query tile")
    if q_tile_starts_q.ndim != 1:
        raise ValueError("q_tile_starts_q must be rank-1")
    require_cuda_tensors(cu_seqlens_q, message="cu_seqlens_q must be a CUDA tensor")
    _check_cache_dtype(ctx.k_cache, q)

    q_, k_, v_ = make_contiguous(q, k, v)
    k_cache, v_cache = make_contiguous(ctx.k_cache, ctx.v_cache)
    out = torch.empty_like(q_)
    plan = None
    if num_heads > 0 and total_q_len > 0 and b > 0:
        kv_sh = 0 if is_mla else total_q_len * d
        plan = _launch(
            q=q_,
            out=out,
            k=k_,
            v=None if is_mla else v_,
            B=b,
            H=num_heads,
            D=d,
            N=0,
            total_q=int(total_q_len),
            cu_seqlens_q=cu_seqlens_q.to(torch.int32).contiguous(),
            q_strides=(0, total_q_len * d, d),
            q_layout=_lib.LAYOUT_PACKED,
            o_strides=(0, total_q_len * d, d),
            o_layout=_lib.LAYOUT_PACKED,
            k_strides=(0, kv_sh, d),
            v_strides=(0, kv_sh, d),
            kv_layout=_lib.LAYOUT_PACKED,
            k_ctx=k_cache,
            v_ctx=None if is_mla else v_cache,
            c_strides=c_strides,
            cu_seqlens_kv=ctx.cu_seqlens_kv.to(torch.int32).contiguous(),
            ctx_len=0,
            ctx_batch=cbs,
            ctx_rows=_ctx_rows(ctx),
            scale=scale,
            flags=(_lib.FLAG_MLA if is_mla else 0)
            | (_lib.FLAG_PREFILL if prefill else 0)
            | (_lib.FLAG_CAUSAL_SEQ if causal_query_seq_attn else 0),
            inference_cache=inference_cache,
            ctx_index=ctx_index,
            block_table=ctx.block_table,
            page_stride=_page_stride(ctx, num_heads, d, is_mla),
        )

    if prefill and inference_cache is not None:
        # the contiguous tensors the kernel read, as the reference stores its
        # make_contiguous copies (host.py:663-683, 777-786)
        inference_cache.prefill_kv_cache(
            layer_id,
            k_cache=k_,
            v_cache=None if is_mla else v_,
            total_context_len=int(total_q_len),
            cu_seqlens_kv=cu_seqlens_q.contiguous(),
            context_batch_size=b,
            is_mla=is_mla,
            num_heads=num_heads,
            head_dim=d,
        )
    return out, plan
