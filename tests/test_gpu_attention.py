"""GPU parity of the HIP attention path against the numpy oracle (fp64 math on the
same bf16/fp16/fp32 inputs).  Tolerance: max-abs 1e-2 and rtol 1e-2 per element
(assert_allclose(out, ref, atol=1e-2, rtol=1e-2)).

The first group ports the reference's own integration tests
(src/flash_mlm/host/test_host.py, same seeds, shapes and API calls, checked here
against the oracle instead of torch fp16 math); the rest widens coverage (head dims,
dtypes, context sharing, prefill round trips, odd shapes) and runs the BASELINE
configs at full size with per-(sequence, head) oracle checks plus size-independent
properties."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flash_mlm import (
    InferenceCache,
    build_pack_metadata,
    flash_attn_mlm,
    flash_attn_mlm_compressed,
    flash_attn_mlm_precompressed,
    unpack_from_kernel,
)
from flash_mlm.host.host_utils import pack_for_kernel
from oracle import attention_ref as ar
from oracle import pack_ref

pytestmark = pytest.mark.gpu
ATOL = RTOL = 1e-2


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _close(out, ref, atol=ATOL, rtol=RTOL):
    np.testing.assert_allclose(_np(out) if isinstance(out, torch.Tensor) else out, ref, atol=atol, rtol=rtol)


def _randn(shape, device, dtype=torch.float16, std=1.0):
    return (torch.randn(shape, device=device) * std).to(dtype)


def _packed_oracle(q, k, v, lengths, scale, *, is_mla=False, causal=False, prefill=False, k_cache=None, v_cache=None, cu_kv=None, cbs=1, Tc=0, context_index=None):
    return ar.mlm_attention_packed(
        _np(q), _np(k), _np(v), [int(x) for x in lengths], scale, is_mla=is_mla,
        causal_query_seq_attn=causal, prefill=prefill,
        k_cache=None if k_cache is None else _np(k_cache),
        v_cache=None if v_cache is None else _np(v_cache),
        cu_seqlens_kv=None if cu_kv is None else [int(x) for x in cu_kv],
        total_context_len=Tc, context_batch_size=cbs, context_index=context_index,
    )


# ---------------------------------------------------------------------------
# reference integration tests (test_host.py), ported
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("is_mla", [False, True])
def test_dense_prefill_requires_cache(is_mla, device):
    torch.manual_seed(21)
    q = _randn((2, 2, 16, 64), device)
    with pytest.raises(ValueError, match="prefill=True requires inference_cache"):
        flash_attn_mlm(q, q, q, scale=0.5, inference_cache=None, layer_id=None, is_mla=is_mla, block_m=32, block_n=32, prefill=True)


@pytest.mark.parametrize("is_mla", [False, True])
def test_dense_no_cache_matches_reference(is_mla, device):
    torch.manual_seed(22)
    B, H, N, D, scale = 2, 3, 24, 64, 0.6
    q, k = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v = k if is_mla else _randn((B, H, N, D), device)
    out = flash_attn_mlm(q, k, v, scale=scale, is_mla=is_mla, block_m=32, block_n=32)
    _close(out, ar.mlm_attention_dense(_np(q), _np(k), _np(v), scale, is_mla=is_mla))


@pytest.mark.parametrize("is_mla", [False, True])
def test_dense_prefill_then_use_cached_context_matches_reference(is_mla, device):
    torch.manual_seed(23)
    B, H, N, D, scale = 2, 2, 20, 64, 0.55
    q1, k1 = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v1 = k1 if is_mla else _randn((B, H, N, D), device)
    q2, k2 = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v2 = k2 if is_mla else _randn((B, H, N, D), device)
    cache = InferenceCache()
    out1 = flash_attn_mlm(q1, k1, v1, scale=scale, inference_cache=cache, layer_id=3, is_mla=is_mla, block_m=32, block_n=32, prefill=True)
    _close(out1, ar.mlm_attention_dense(_np(q1), _np(k1), _np(v1), scale, is_mla=is_mla))
    out = flash_attn_mlm(q2, k2, v2, scale=scale, inference_cache=cache, layer_id=3, is_mla=is_mla, context_batch_size=B, block_m=32, block_n=32)
    entry = cache.get_kv_cache(3, is_mla=is_mla, num_heads=H, head_dim=D, dtype=q2.dtype, device=q2.device)
    # the stored entry is this call's K/V (MLA: head 0 of k), bit-exact
    if is_mla:
        assert torch.equal(entry.k_cache, k1[:, 0].reshape(B * N, D)) and entry.v_cache is None
    else:
        assert torch.equal(entry.k_cache, k1.reshape(B * H * N, D)) and torch.equal(entry.v_cache, v1.reshape(B * H * N, D))
    ctx_len = entry.total_context_len // entry.context_batch_size
    ref = ar.mlm_attention_dense(
        _np(q2), _np(k2), _np(v2), scale, is_mla=is_mla, k_cache=_np(entry.k_cache),
        v_cache=None if is_mla else _np(entry.v_cache), context_len=ctx_len, context_batch_size=entry.context_batch_size,
    )
    _close(out, ref)


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_prefill_requires_cache(is_mla, device):
    torch.manual_seed(11)
    q = _randn((2, 2, 16, 64), device)
    meta = build_pack_metadata(torch.tensor([16, 9], device=device, dtype=torch.int32), 16, block_n=32)
    with pytest.raises(ValueError, match="prefill=True requires inference_cache"):
        flash_attn_mlm_compressed(q, q, q, num_heads=2, scale=0.5, q_meta=meta, is_mla=is_mla, block_m=32, block_n=32, prefill=True)


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_no_prefill_empty_context_same_with_or_without_cache(is_mla, device):
    torch.manual_seed(12)
    B, H, N, D, scale = 2, 3, 24, 64, 0.6
    lengths = torch.tensor([24, 15], device=device, dtype=torch.int32)
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    meta = build_pack_metadata(lengths, N, block_n=32)
    out_no = flash_attn_mlm_compressed(q, k, v, num_heads=H, scale=scale, q_meta=meta, is_mla=is_mla, block_m=32, block_n=32)
    out_with = flash_attn_mlm_compressed(
        q, k, v, num_heads=H, scale=scale, q_meta=meta, inference_cache=InferenceCache(), layer_id=0, is_mla=is_mla, block_m=32, block_n=32
    )
    assert torch.equal(out_no, out_with)
    ref = _packed_oracle(q, k, v, lengths.tolist(), scale, is_mla=is_mla)
    _close(unpack_from_kernel(out_no, meta, H=H), ref)


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_prefill_with_cache_stores_entry(is_mla, device):
    torch.manual_seed(13)
    B, H, N, D = 2, 2, 20, 64
    lengths = torch.tensor([20, 7], device=device, dtype=torch.int32)
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    meta = build_pack_metadata(lengths, N, block_n=32)
    cache = InferenceCache()
    out = flash_attn_mlm_compressed(q, k, v, num_heads=H, scale=0.55, q_meta=meta, inference_cache=cache, layer_id=7, is_mla=is_mla, block_m=32, block_n=32, prefill=True)
    stored = cache.get_kv_cache(7, is_mla=is_mla, num_heads=H, head_dim=D, dtype=q.dtype, device=q.device)
    assert int(stored.cu_seqlens_kv[-1]) == 27
    assert stored.total_context_len >= 27
    assert stored.k_cache.shape[0] == (1 if is_mla else H) * stored.total_context_len
    assert stored.context_batch_size == B
    # exact layout: padded T_pad (host_utils.py:292-312) and zero tails, bit-exact
    ref_meta = pack_ref.pack_metadata(np.array([20, 7]), N, 32)
    T_pad = pack_ref.total_q_len_padded(27, ref_meta.cu_seqlens, 32, 32)
    assert stored.total_context_len == T_pad
    np.testing.assert_array_equal(_np(stored.k_cache), pack_ref.pack(_np(k[:, :1] if is_mla else k), ref_meta, T_pad))
    if not is_mla:
        np.testing.assert_array_equal(_np(stored.v_cache), pack_ref.pack(_np(v), ref_meta, T_pad))
    # prefill skips the (absent) context; output is plain per-sequence attention
    _close(unpack_from_kernel(out, meta, H), _packed_oracle(q, k, v, [20, 7], 0.55, is_mla=is_mla, prefill=True))


def _empty_context_cache(B, H, D, is_mla, device):
    k_cache = torch.empty((0, D), device=device, dtype=torch.float16)
    cache = InferenceCache()
    cache.prefill_kv_cache(
        layer_id=0, k_cache=k_cache, v_cache=torch.empty_like(k_cache), total_context_len=0,
        cu_seqlens_kv=torch.zeros(B + 1, device=device, dtype=torch.int32), context_batch_size=B,
        is_mla=is_mla, num_heads=H, head_dim=D,
    )
    return cache


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_matches_reference(is_mla, device):
    torch.manual_seed(0)
    B, H, N, D, scale = 2, 3, 48, 64, 0.7
    lengths = torch.tensor([48, 37], device=device, dtype=torch.int32)
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    meta = build_pack_metadata(lengths, N, block_n=32)
    out = flash_attn_mlm_compressed(q, k, v, num_heads=H, scale=scale, q_meta=meta, inference_cache=_empty_context_cache(B, H, D, is_mla, device), layer_id=0, is_mla=is_mla, block_m=32, block_n=32)
    _close(unpack_from_kernel(out, meta, H=H), _packed_oracle(q, k, v, [48, 37], scale, is_mla=is_mla))


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_prev_subseq_attention_matches_reference(is_mla, device):
    torch.manual_seed(2)
    B, H, N, D, scale = 3, 2, 32, 64, 0.65
    lengths = torch.tensor([9, 7, 5], device=device, dtype=torch.int32)
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    meta = build_pack_metadata(lengths, N, block_n=32)
    out = flash_attn_mlm_compressed(
        q, k, v, num_heads=H, scale=scale, q_meta=meta, inference_cache=_empty_context_cache(B, H, D, is_mla, device),
        layer_id=0, is_mla=is_mla, block_m=32, block_n=32, causal_query_seq_attn=True,
    )
    _close(unpack_from_kernel(out, meta, H=H), _packed_oracle(q, k, v, [9, 7, 5], scale, is_mla=is_mla, causal=True))


def _context_cache(B, H, D, is_mla, ctx_lengths, device, dtype=torch.float16, cbs=None, std=1.0):
    cu_kv = torch.zeros(len(ctx_lengths) + 1, dtype=torch.int32)
    cu_kv[1:] = torch.cumsum(torch.tensor(ctx_lengths), 0)
    Tc = int(cu_kv[-1])
    k_cache = _randn(((1 if is_mla else H) * Tc, D), device, dtype, std)
    v_cache = _randn(((1 if is_mla else H) * Tc, D), device, dtype, std)
    cache = InferenceCache()
    cache.prefill_kv_cache(
        layer_id=0, k_cache=k_cache, v_cache=v_cache, total_context_len=Tc, cu_seqlens_kv=cu_kv.to(device),
        context_batch_size=len(ctx_lengths) if cbs is None else cbs, is_mla=is_mla, num_heads=H, head_dim=D,
    )
    return cache, k_cache, v_cache, cu_kv, Tc


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("is_mla", [False, True])
def test_repeated_calls_follow_their_inputs(is_mla, causal, device):
    """A repeated call with the same tensors reuses the first call's launch parameters
    (the launch memo): it must still read the current contents of q/k/v (changed in
    place), a context replaced by a new prefill, and, with causal_query_seq_attn, re-pack
    this call's K/V; a call on new tensors of the same shape must not reuse them."""
    torch.manual_seed(7400 + 2 * is_mla + causal)
    lengths, ctx = [70, 1, 130, 0, 64], [40, 0, 7, 129, 64]
    B, H, N, D = len(lengths), 3, max(lengths), 64
    scale = 0.125
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, ctx, device, torch.bfloat16)

    def run():
        out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=is_mla, block_n=64,
                                        causal_query_seq_attn=causal)
        ref = _packed_oracle(q, k, v, lengths, scale, is_mla=is_mla, causal=causal, k_cache=kc,
                             v_cache=None if is_mla else vc, cu_kv=cu_kv, cbs=B, Tc=Tc)
        _close(unpack_from_kernel(out, meta, H), ref)

    run()
    run()
    assert len(meta.launch_memo) == 1
    for t in (q, k, v):
        t.copy_(_randn(t.shape, device, torch.bfloat16))
        run()
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, [x + 3 for x in ctx], device, torch.bfloat16)
    run()
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    run()
    # dense: the same, on the module-level memo
    cache, kc, vc, _, Tc = _context_cache(B, H, D, is_mla, [16] * B, device, torch.bfloat16)

    def run_dense():
        out = flash_attn_mlm(q, k, v, scale, inference_cache=cache, layer_id=0, is_mla=is_mla)
        ref = ar.mlm_attention_dense(_np(q), _np(k), _np(v), scale, k_cache=_np(kc),
                                     v_cache=None if is_mla else _np(vc), context_len=16, context_batch_size=B,
                                     is_mla=is_mla)
        _close(out, ref)

    run_dense()
    q.copy_(_randn(q.shape, device, torch.bfloat16))
    run_dense()


@pytest.mark.parametrize("is_mla", [False, True])
def test_compressed_matches_reference_with_cache(is_mla, device):
    torch.manual_seed(1)
    B, H, N, D, scale = 2, 3, 48, 64, 0.5
    lengths = torch.tensor([48, 37], device=device, dtype=torch.int32)
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, [13, 9], device)
    meta = build_pack_metadata(lengths, N, block_n=32)
    out = flash_attn_mlm_compressed(q, k, v, num_heads=H, scale=scale, q_meta=meta, inference_cache=cache, layer_id=0, is_mla=is_mla, block_m=32, block_n=32)
    ref = _packed_oracle(q, k, v, [48, 37], scale, is_mla=is_mla, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=B, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H=H), ref)


def _prepack(q, k, v, meta, is_mla):
    q_p = pack_for_kernel(q, meta, flatten_for_kernel=True)
    if is_mla:
        k_p = pack_for_kernel(k[:, :1], meta, flatten_for_kernel=False).squeeze(0)
        return q_p, k_p, k_p
    return q_p, pack_for_kernel(k, meta, flatten_for_kernel=True), pack_for_kernel(v, meta, flatten_for_kernel=True)


@pytest.mark.parametrize("is_mla", [False, True])
@pytest.mark.parametrize("with_cache", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_precompressed_matches_compressed(is_mla, with_cache, causal, device):
    torch.manual_seed(51 if with_cache else 50)
    B, H, N, D, scale = 2, 3, 48, 64, 0.5
    lengths = torch.tensor([48, 37], device=device, dtype=torch.int32)
    q, k = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v = k if is_mla else _randn((B, H, N, D), device)
    if with_cache:
        make = lambda: _context_cache(B, H, D, is_mla, [13, 9], device)[0]  # noqa: E731
        torch.manual_seed(5)
        c1 = make()
        torch.manual_seed(5)
        c2 = make()
    else:
        c1, c2 = (_empty_context_cache(B, H, D, is_mla, device) for _ in range(2))
    meta = build_pack_metadata(lengths, N, block_n=32)
    ref_out = flash_attn_mlm_compressed(q, k, v, num_heads=H, scale=scale, q_meta=meta, inference_cache=c1, layer_id=0, is_mla=is_mla, block_m=32, block_n=32, causal_query_seq_attn=causal)
    q_p, k_p, v_p = _prepack(q, k, v, meta, is_mla)
    pre = flash_attn_mlm_precompressed(
        q_p, k_p, v_p, num_heads=H, total_q_len=q_p.shape[0] // H, cu_seqlens_q=meta.cu_seqlens,
        batch_ids_q=meta.batch_ids_q, q_tile_starts_q=meta.q_tile_starts_q, scale=scale, inference_cache=c2,
        layer_id=0, is_mla=is_mla, block_m=32, block_n=32, causal_query_seq_attn=causal,
    )
    torch.testing.assert_close(pre, ref_out, atol=1e-5, rtol=0)


@pytest.mark.parametrize("is_mla", [False, True])
def test_precompressed_prefill_stores_cache_entry(is_mla, device):
    torch.manual_seed(52)
    B, H, N, D = 2, 2, 20, 64
    lengths = torch.tensor([20, 7], device=device, dtype=torch.int32)
    q, k = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v = k if is_mla else _randn((B, H, N, D), device)
    meta = build_pack_metadata(lengths, N, block_n=32)
    q_p, k_p, v_p = _prepack(q, k, v, meta, is_mla)
    cache = InferenceCache()
    out = flash_attn_mlm_precompressed(
        q_p, k_p, v_p, num_heads=H, total_q_len=q_p.shape[0] // H, cu_seqlens_q=meta.cu_seqlens,
        batch_ids_q=meta.batch_ids_q, q_tile_starts_q=meta.q_tile_starts_q, scale=0.55, inference_cache=cache,
        layer_id=7, is_mla=is_mla, block_m=32, block_n=32, prefill=True,
    )
    stored = cache.get_kv_cache(7, is_mla=is_mla, num_heads=H, head_dim=D, dtype=q.dtype, device=q.device)
    assert int(stored.cu_seqlens_kv[-1]) == 27 and stored.total_context_len >= 27
    assert stored.k_cache.shape[0] == (1 if is_mla else H) * stored.total_context_len
    assert stored.context_batch_size == B and stored.k_cache is k_p
    _close(unpack_from_kernel(out, meta, H), _packed_oracle(q, k, v, [20, 7], 0.55, is_mla=is_mla, prefill=True))


@pytest.mark.parametrize("is_mla", [False, True])
def test_precompressed_prefill_non_contiguous_kv(is_mla, device):
    # packed k / v given as strided views (row stride 2*D): the prefill stores the
    # contiguous copies the kernel read, as the reference stores its make_contiguous
    # outputs (host.py:663-683, 777-786), and a later call attends to them as context
    torch.manual_seed(53)
    B, H, N, D = 3, 2, 40, 64
    lens = [40, 9, 23]
    lengths = torch.tensor(lens, device=device, dtype=torch.int32)
    q, k = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v = k if is_mla else _randn((B, H, N, D), device)
    meta = build_pack_metadata(lengths, N, block_n=32)
    q_p, k_p, v_p = _prepack(q, k, v, meta, is_mla)

    def strided(x):
        wide = torch.zeros((x.shape[0], 2 * D), dtype=x.dtype, device=x.device)
        wide[:, :D] = x
        return wide[:, :D]

    k_s = strided(k_p)
    v_s = k_s if is_mla else strided(v_p)
    assert not k_s.is_contiguous()
    cache = InferenceCache()
    T = q_p.shape[0] // H
    kw = dict(num_heads=H, total_q_len=T, cu_seqlens_q=meta.cu_seqlens, batch_ids_q=meta.batch_ids_q,
              q_tile_starts_q=meta.q_tile_starts_q, scale=0.5, inference_cache=cache, layer_id=3, is_mla=is_mla,
              block_m=32, block_n=32)
    out = flash_attn_mlm_precompressed(q_p, k_s, v_s, prefill=True, **kw)
    _close(unpack_from_kernel(out, meta, H), _packed_oracle(q, k, v, lens, 0.5, is_mla=is_mla, prefill=True))
    stored = cache.get_kv_cache(3, is_mla=is_mla, num_heads=H, head_dim=D, dtype=q.dtype, device=q.device)
    assert stored.k_cache.is_contiguous() and torch.equal(stored.k_cache, k_p)
    if not is_mla:
        assert stored.v_cache.is_contiguous() and torch.equal(stored.v_cache, v_p)
    # second call: fresh queries attend to [stored context of b || main keys of b]
    q2, k2 = _randn((B, H, N, D), device), _randn((B, H, N, D), device)
    v2 = k2 if is_mla else _randn((B, H, N, D), device)
    q2_p, k2_p, v2_p = _prepack(q2, k2, v2, meta, is_mla)
    out2 = flash_attn_mlm_precompressed(q2_p, k2_p, v2_p, **kw)
    ref = _packed_oracle(q2, k2, v2, lens, 0.5, is_mla=is_mla, k_cache=k_p, v_cache=v_p,
                         cu_kv=meta.cu_seqlens.cpu(), cbs=B, Tc=T)
    _close(unpack_from_kernel(out2, meta, H), ref)


# ---------------------------------------------------------------------------
# wider coverage
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("mode", ["ctx", "causal_ctx", "mla_ctx", "mla_causal_prefill"])
def test_packed_head_dim_dtype_sweep(dtype, D, mode, device):
    torch.manual_seed(1000 + D)
    is_mla = mode.startswith("mla")
    causal = "causal" in mode
    prefill = "prefill" in mode
    lengths = [70, 1, 0, 133, 64, 17]
    B, H, N = len(lengths), 3, 140
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, [5, 0, 40, 129, 64, 3], device, dtype)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=is_mla, block_n=64, causal_query_seq_attn=causal, prefill=prefill)
    ref = _packed_oracle(q, k, v, lengths, scale, is_mla=is_mla, causal=causal, prefill=prefill, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=B, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)


# ---------------------------------------------------------------------------
# every compiled tile configuration (fmlm_attn_params.tile_config), forced
# ---------------------------------------------------------------------------
TILE_CONFIGS = {16: (1,), 32: (1,), 64: (1, 2, 3, 4), 128: (1, 2, 3, 4, 5), 256: (1, 2)}


def test_tile_config_table_matches_library(device):
    # configurations past the table are rejected (FMLM_E_ARG) before any launch
    from flash_mlm import _lib

    lib = _lib.load()
    for D, ks in TILE_CONFIGS.items():
        for dt in (_lib.DTYPE_BF16, _lib.DTYPE_F16):
            p = _lib.AttnParams()
            p.dtype, p.B, p.H, p.D, p.N, p.total_q = dt, 1, 1, D, 64, 64
            for k in ks:
                p.tile_config = k
                assert lib.fmlm_attn_workspace_bytes(p) == 0, (D, k)
            p.tile_config = max(ks) + 1
            assert lib.fmlm_attn_workspace_bytes(p) == -1, (D, p.tile_config)
    p.D, p.flags, p.tile_config = 512, _lib.FLAG_MLA, 2
    assert lib.fmlm_attn_workspace_bytes(p) == -1
    # the ping-pong configurations (D=64: 4, D=128: 5) read contiguous contexts only
    p.flags, p.ctx_block_table, p.ctx_pages_per_batch = 0, 4096, 1
    for D, k in ((64, 4), (128, 5)):
        p.D, p.tile_config = D, k
        assert lib.fmlm_attn_workspace_bytes(p) == -1, (D, k)
        p.tile_config = 1
        assert lib.fmlm_attn_workspace_bytes(p) >= 0, D


@pytest.mark.parametrize("D,k", [(D, k) for D, ks in TILE_CONFIGS.items() for k in ks])
@pytest.mark.parametrize("mode", ["ctx", "causal_ctx", "dense_shared", "split"])
def test_every_tile_config(D, k, mode, device):
    from flash_mlm.host.host import tile_config

    torch.manual_seed(8000 + D + 10 * k)
    dtype = torch.bfloat16 if (D + k) % 2 else torch.float16
    scale = 1.0 / math.sqrt(D)
    with tile_config(k):
        if mode == "dense_shared":
            B, H, N, C = 3, 4, 300, 150
            q, kk, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
            kc, vc = (_randn((1, H, C, D), device, dtype) for _ in range(2))
            cache = InferenceCache()
            cache.prefill_kv_cache(0, k_cache=kc.reshape(H * C, D), v_cache=vc.reshape(H * C, D),
                                   context_batch_size=1, is_mla=False, num_heads=H, head_dim=D)
            out = flash_attn_mlm(q, kk, v, scale, inference_cache=cache, layer_id=0)
            ref = ar.mlm_attention_dense(_np(q), _np(kk), _np(v), scale, k_cache=_np(kc.reshape(H * C, D)),
                                         v_cache=_np(vc.reshape(H * C, D)), context_len=C, context_batch_size=1)
            _close(out, ref)
            return
        causal = mode == "causal_ctx"
        lengths = [300, 1, 0, 257, 64, 130] if mode != "split" else [97, 300, 1]
        ctx = [5, 0, 40, 700, 64, 3] if mode != "split" else [3000, 4100, 65]
        B, H, N = len(lengths), 3, max(lengths)
        q, kk, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
        cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, ctx, device, dtype)
        meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
        out = flash_attn_mlm_compressed(q, kk, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    ref = _packed_oracle(q, kk, v, lengths, scale, causal=causal, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=B, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)


def test_library_tile_choice_by_query_rows(device):
    # tile_config 0 at D = 64 / 128: configuration 3 (64 query rows per workgroup) when the
    # sequences average at most 64 query rows (total_q <= 64 B), configuration 1 (128 rows)
    # otherwise.  The workspace holds the schedule's work units, whose count follows the
    # workgroup's row count, so its size shows which configuration was chosen.
    from flash_mlm import _lib

    lib = _lib.load()
    for D in (64, 128):
        for B, total_q, want in ((40, 64 * 40, 3), (40, 64 * 40 + 1, 1), (7, 7 * 30, 3), (7, 7 * 900, 1)):
            p = _lib.AttnParams()
            p.dtype, p.B, p.H, p.D, p.N, p.total_q = _lib.DTYPE_BF16, B, 8, D, 1024, total_q
            p.cu_seqlens_q = 4096  # packed rows (sizing reads no device memory)
            ws = {}
            for k in (0, 1, 3):
                p.tile_config = k
                ws[k] = lib.fmlm_attn_workspace_bytes(p)
            assert ws[1] > 0 and ws[3] > 0 and ws[1] != ws[3], (D, B, total_q, ws)
            assert ws[0] == ws[want], (D, B, total_q, ws)
    # other head dims keep configuration 1 for short sequences
    p.D, p.B, p.total_q = 256, 40, 64 * 40
    p.tile_config = 0
    w0 = lib.fmlm_attn_workspace_bytes(p)
    p.tile_config = 1
    assert w0 == lib.fmlm_attn_workspace_bytes(p)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mode", ["ctx", "causal_shared", "paged"])
def test_short_query_sequences_library_tile(D, mode, device):
    # sequences of at most 64 query rows: the library's choice is the 64-row configuration
    torch.manual_seed(8500 + D)
    dtype = torch.bfloat16 if mode != "ctx" else torch.float16
    scale = 1.0 / math.sqrt(D)
    lengths = [1, 64, 17, 0, 40, 63, 5, 33, 64, 2]
    B, H, N = len(lengths), 3, 64
    causal = mode == "causal_shared"
    q, kk, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
    if mode == "causal_shared":
        ctx, cbs = [300], 1
    else:
        ctx, cbs = [5, 0, 130, 700, 64, 3, 1, 90, 257, 40], B
    cache, kc, vc, cu_kv, Tc = _context_cache(cbs, H, D, False, ctx, device, dtype)
    if mode == "paged":  # the same context rows in 64-row pages, pool in reverse page order
        lens = (cu_kv[1:] - cu_kv[:-1]).tolist()
        need = [(n + 63) // 64 for n in lens]
        P = sum(need)
        bt = torch.zeros((len(lens), max(need)), dtype=torch.int32)
        kp, vp = (torch.zeros((H, P * 64, D), dtype=dtype, device=device) for _ in range(2))
        pg = 0
        for c, (n, npg) in enumerate(zip(lens, need)):
            for j in range(npg):
                slot, r0 = P - 1 - (pg + j), int(cu_kv[c]) + 64 * j
                m = min(64, n - 64 * j)
                bt[c, j] = slot
                kp[:, slot * 64 : slot * 64 + m] = kc.view(H, Tc, D)[:, r0 : r0 + m]
                vp[:, slot * 64 : slot * 64 + m] = vc.view(H, Tc, D)[:, r0 : r0 + m]
            pg += npg
        cache = InferenceCache()
        cache.prefill_paged_kv_cache(0, k_pages=kp.view(H, P, 64, D), v_pages=vp.view(H, P, 64, D),
                                     block_table=bt.to(device), context_lens=torch.tensor(lens, dtype=torch.int32),
                                     is_mla=False, num_heads=H, head_dim=D)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, kk, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    ref = _packed_oracle(q, kk, v, lengths, scale, causal=causal, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=cbs, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)


# ---------------------------------------------------------------------------
# split-KV: few work units over long key ranges are cut into parts whose partial
# results a second kernel merges (the schedule decides; these shapes have far fewer
# units than workgroup slots and tens of key tiles per unit)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("mode", ["ctx", "causal_ctx", "shared_ctx", "causal_prefill"])
def test_split_kv_long_key_ranges(dtype, D, mode, device):
    torch.manual_seed(7000 + D)
    causal = "causal" in mode
    prefill = "prefill" in mode
    lengths = [97, 1, 300, 0] if not prefill else [900, 1200, 64, 5]
    B, H, N = len(lengths), 2, max(lengths)
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
    if mode == "shared_ctx":
        cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, [4100], device, dtype, cbs=1)
        cbs = 1
    else:
        cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, [3000, 700, 5000, 1500], device, dtype)
        cbs = B
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    kw = dict(block_n=64, causal_query_seq_attn=causal, prefill=prefill, context_batch_size=cbs if mode == "shared_ctx" else None)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache if not prefill else InferenceCache(), 0, **kw)
    ref = _packed_oracle(q, k, v, lengths, scale, causal=causal, prefill=prefill,
                         k_cache=None if prefill else kc, v_cache=None if prefill else vc,
                         cu_kv=None if prefill else cu_kv, cbs=cbs, Tc=0 if prefill else Tc)
    _close(unpack_from_kernel(out, meta, H), ref)
    # the schedule split these units (header word 1 counts split groups)
    (sched,) = meta.kernel_schedules.values()
    assert int(sched[:8].view(torch.int32)[1]) > 0
    # the cached schedule (and its split records) is reused: same result again
    out2 = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache if not prefill else InferenceCache(), 0, **kw)
    assert torch.equal(out, out2)
    # The split parts keep O / l in fp32, so a split row is rounded to the output type once,
    # as an unsplit row is: its error stays within half an output ulp of the same heads
    # computed unsplit (the inputs repeated along the head axis until the schedule has
    # units enough not to split).  The two differ by more than summation order: each part
    # rounds its P against its own running maximum.
    got = unpack_from_kernel(out, meta, H).float().cpu().numpy().astype(np.float64)
    err_split = float(np.abs(got - ref).max())
    R = 32
    while True:
        qR, kR, vR = (x.repeat(1, R, 1, 1) for x in (q, k, v))
        cacheR = InferenceCache()
        if not prefill:
            hv = lambda t: t.view(H, Tc, D).repeat(R, 1, 1).reshape(H * R * Tc, D)  # noqa: E731
            cacheR.prefill_kv_cache(0, k_cache=hv(kc), v_cache=hv(vc), total_context_len=Tc, cu_seqlens_kv=cu_kv.to(device),
                                    context_batch_size=cbs if mode == "shared_ctx" else B, is_mla=False,
                                    num_heads=H * R, head_dim=D)
        metaR = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
        outR = flash_attn_mlm_compressed(qR, kR, vR, H * R, metaR, scale, cacheR, 0, **kw)
        (schedR,) = metaR.kernel_schedules.values()
        if int(schedR[:8].view(torch.int32)[1]) == 0:
            break
        R *= 2
    unsplit = unpack_from_kernel(outR, metaR, H * R)[:, :H].float().cpu().numpy().astype(np.float64)
    err_unsplit = float(np.abs(unsplit - ref).max())
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert err_split <= err_unsplit + ulp / 2 * float(np.abs(ref).max()), (err_split, err_unsplit)


def test_cached_schedule_per_head_count_and_mode(device):
    """One PackMetadata serves calls with different head counts, modes and contexts: each
    call gets a schedule built for its own heads and kernel, and every result matches the
    oracle (a schedule of another head count would skip or overrun heads)."""
    torch.manual_seed(7100)
    lengths = [97, 1, 300, 0]
    B, N, D = len(lengths), 300, 64
    scale = 1.0 / math.sqrt(D)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    for H, causal, ctx in ((4, False, [3000, 700, 5000, 1500]), (2, False, [3000, 700, 5000, 1500]),
                           (2, True, [10, 2000, 0, 64]), (4, False, [10, 2000, 0, 64])):
        q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
        cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, ctx, device, torch.bfloat16)
        out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
        ref = _packed_oracle(q, k, v, lengths, scale, causal=causal, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=B, Tc=Tc)
        _close(unpack_from_kernel(out, meta, H), ref)
    assert len(meta.kernel_schedules) == 3


def _schedule_units(sched):
    """Decoded work list of a cached schedule buffer: (xcd, b, h, tile, s, S) per unit.
    Header words: 5 = entries per queue (cap), 8 + x = length of queue x (the units meant
    for XCD x); units of 4 int32 from byte 256, queue x at entry x * cap: b,
    h | tile << 16, record, split word."""
    words = sched.view(torch.int32).cpu()
    cap = int(words[5])
    out = []
    for x in range(8):
        n = int(words[8 + x])
        assert 0 <= n <= cap
        base = 64 + 4 * x * cap
        for b, ht, _, w in words[base:base + 4 * n].view(n, 4).tolist():
            S = ((w >> 25) & 15) + 1 if w >= 0 else 1
            s = (w >> 20) & 31 if w >= 0 else 0
            out.append((x, b, ht & 0xFFFF, ht >> 16, s, S))
    return out


@pytest.mark.parametrize("H,lengths,causal", [
    (12, [300, 64, 1, 511, 200, 0, 77, 128, 129, 400, 5, 256, 90, 33, 480, 260], True),
    (12, [300, 64, 1, 511, 200, 0, 77, 128, 129, 400, 5, 256, 90, 33, 480, 260], False),
    (3, [700, 1, 130, 64, 0, 999], False),
    (5, [130] * 9 + [1], True),
    (16, [257, 1000, 3, 128], False),
    (1, [64 * i + 1 for i in range(20)], False),
])
def test_schedule_places_every_tile_once(H, lengths, causal, device):
    """The work list holds every (sequence, head, 128-row query tile) once, each split into
    its S parts exactly once, and keeps every head on ceil(8 / H) XCDs or one more (its
    queues; at most two from 8 heads up); the result matches the oracle."""
    torch.manual_seed(7200 + H)
    B, N, D = len(lengths), max(lengths), 64
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, [200], device, torch.bfloat16, cbs=1)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal,
                                    context_batch_size=1)
    ref = _packed_oracle(q, k, v, lengths, scale, causal=causal, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=1, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)
    (sched,) = meta.kernel_schedules.values()
    units = _schedule_units(sched)
    seen = {}
    for slot, b, h, tile, s, S in units:
        key = (b, h, tile)
        assert (key, s) not in seen, (key, s)
        seen[(key, s)] = S
    want = {(b, h, t) for b, L in enumerate(lengths) for h in range(H) for t in range((L + 127) // 128)}
    got = {key for key, _ in seen}
    assert got == want
    for key in want:  # every part of a split tile, once
        S = {seen[(k_, s)] for (k_, s) in seen if k_ == key}
        assert len(S) == 1
        (S,) = S
        assert {s for (k_, s) in seen if k_ == key} == set(range(S))
    for h in range(H):
        xcds = {x for x, _, hh, _, _, _ in units if hh == h}
        assert len(xcds) <= (8 + H - 1) // H + 1, (h, xcds)


def test_schedule_overflow_taken_by_spares(device):
    """One head, a sequence of 60 query tiles beside seven of one row: the long sequence's
    queue (its tiles' split parts) holds more entries than its XCD has workgroups in the
    launch (cap of them in all), so spare workgroups of the other XCDs take the overflow by
    rank; every row matches the oracle."""
    torch.manual_seed(7290)
    H, lengths = 1, [60 * 128, 1, 1, 1, 1, 1, 1, 1]
    B, N, D = len(lengths), max(lengths), 64
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, [200], device, torch.bfloat16, cbs=1)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=True,
                                    context_batch_size=1)
    (sched,) = meta.kernel_schedules.values()
    words = sched.view(torch.int32).cpu()
    G = int(words[5])  # workgroups of the launch: the queue capacity
    lens = [int(words[8 + x]) for x in range(8)]
    overflow = sum(max(n - (G - x + 7) // 8, 0) for x, n in enumerate(lens))
    assert overflow > 0, (G, lens)
    ref = _packed_oracle(q, k, v, lengths, scale, causal=True, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=1, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)


@pytest.mark.parametrize("lengths,ctx_lengths", [
    ([300, 64, 1, 511, 200, 0, 77, 400], [700, 0, 5, 1300, 64, 10, 300, 900]),
    ([130, 1, 64, 97, 200], [70, 0, 5, 129, 64]),
    ([900, 1000, 1100, 1200], [4000, 4000, 4000, 4000]),
])
def test_mla_schedule_keeps_sequences_together(lengths, ctx_lengths, device):
    """Head-packed tiles (the 512-wide latent, 128 of a sequence's H*L (head, row) rows per
    tile): every (sequence, tile) once, in all its split parts; a sequence's tiles sit on as
    few XCDs (queues) as its share of the work needs, plus one at each cut; and the XCDs'
    work (query tiles x key tiles) differs from an equal share by at most one tile's."""
    torch.manual_seed(7300 + len(lengths))
    B, H, N, D = len(lengths), 16, max(lengths), 512
    dtype = torch.bfloat16
    q = _randn((B, H, N, D), device, dtype, std=0.5)
    k = _randn((B, H, N, D), device, dtype, std=0.5)
    cache, kc, _, cu_kv, Tc = _context_cache(B, H, D, True, ctx_lengths, device, dtype, std=0.5)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, cache, 0, is_mla=True, block_n=64)
    ref = _packed_oracle(q, k, k, lengths, scale, is_mla=True, k_cache=kc, cu_kv=cu_kv, cbs=B, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)
    (sched,) = meta.kernel_schedules.values()
    units = _schedule_units(sched)
    seen = {}
    for slot, b, _, tile, s, S in units:
        assert ((b, tile), s) not in seen, (b, tile, s)
        seen[((b, tile), s)] = (S, slot % 8)
    tiles = [(H * L + 127) // 128 for L in lengths]
    want = {(b, t) for b in range(B) for t in range(tiles[b])}
    assert {key for key, _ in seen} == want
    for key in want:
        S = {seen[(k_, s)][0] for (k_, s) in seen if k_ == key}
        assert len(S) == 1
        (S,) = S
        assert {s for (k_, s) in seen if k_ == key} == set(range(S))
    kt = [max((c + 63) // 64 + (L + 63) // 64, 1) for c, L in zip(ctx_lengths, lengths)]
    work = [t * w for t, w in zip(tiles, kt)]
    W = sum(work)
    per_xcd = [0] * 8
    for ((b, _), s), (_, x) in seen.items():
        if s == 0:
            per_xcd[x] += kt[b]
    for b in range(B):
        xcds = {x for ((bb, _), _), (_, x) in seen.items() if bb == b}
        assert len(xcds) <= (8 * work[b]) // W + 2, (b, xcds)
    assert max(abs(w - W / 8) for w in per_xcd) <= max(kt), per_xcd


@pytest.mark.parametrize("seed", [7, 8])
def test_schedule_unbalanced_heads_every_tile(seed, device):
    """A shape whose by-head placement puts more units on one XCD than an even share (4
    heads, 64 sequences of 256-4096 query rows over 0-8192 context rows, no split): every
    (sequence, head, query tile) is in the work list once, and every row of the output
    matches a per-sequence fp32 attention on the GPU."""
    g = torch.Generator().manual_seed(seed)
    B, H, D = 64, 4, 64
    lengths = torch.randint(256, 4097, (B,), generator=g).tolist()
    ctx = torch.randint(0, 8193, (B,), generator=g).tolist()
    N = max(lengths)
    torch.manual_seed(seed)
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, ctx, device, torch.bfloat16)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    scale = 1.0 / math.sqrt(D)
    from flash_mlm.host.host import tile_config

    with tile_config(1):  # 128-row query tiles
        out = unpack_from_kernel(flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64), meta, H)
    (sched,) = meta.kernel_schedules.values()
    units = _schedule_units(sched)
    assert all(S == 1 for *_, S in units)
    got = sorted((b, h, t) for _, b, h, t, _, _ in units)
    want = sorted((b, h, t) for b, L in enumerate(lengths) for h in range(H) for t in range((L + 127) // 128))
    assert got == want
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        kcv, vcv = kc.view(H, Tc, D), vc.view(H, Tc, D)
        for b, L in enumerate(lengths):
            c0, c1 = int(cu_kv[b]), int(cu_kv[b + 1])
            K = torch.cat([kcv[:, c0:c1].float(), k[b, :, :L].float()], dim=1)
            V = torch.cat([vcv[:, c0:c1].float(), v[b, :, :L].float()], dim=1)
            s = torch.matmul(q[b, :, :L].float(), K.transpose(1, 2).contiguous()) * scale
            ref = torch.matmul(torch.softmax(s, dim=-1), V)
            err = (out[b, :, :L].float() - ref).abs() - (ATOL + RTOL * ref.abs())
            assert float(err.max()) <= 0, (b, float(err.max()))
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("is_mla", [False, True])
@pytest.mark.parametrize("cbs", [1, 3])
def test_dense_sweep_with_context(dtype, D, is_mla, cbs, device):
    torch.manual_seed(2000 + D + cbs)
    B, H, N, C = 3, 2, 77, 45
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
    rows = cbs * C * (1 if is_mla else H)
    kc, vc = _randn((rows, D), device, dtype), _randn((rows, D), device, dtype)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=None if is_mla else vc, context_batch_size=cbs, is_mla=is_mla, num_heads=H, head_dim=D,
                           total_context_len=cbs * C)
    out = flash_attn_mlm(q, k, v, scale, inference_cache=cache, layer_id=0, is_mla=is_mla)
    ref = ar.mlm_attention_dense(_np(q), _np(k), _np(v), scale, is_mla=is_mla, k_cache=_np(kc), v_cache=_np(vc), context_len=C, context_batch_size=cbs)
    _close(out, ref)


# ---------------------------------------------------------------------------
# index-mapped context batching (context_index, an extension): sequence b attends to
# context batch context_index[b] of a cache holding any number of context batches
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mode", ["plain", "causal", "mla", "gpu_index"])
def test_context_index_packed(dtype, D, mode, device):
    torch.manual_seed(4100 + D + len(mode))
    is_mla, causal = mode == "mla", mode == "causal"
    lengths = [70, 1, 0, 133, 64]
    B, H, N = len(lengths), 3, 140
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, dtype) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, [40, 0, 129], device, dtype)  # 3 contexts
    idx = [2, 0, 2, 1, 0]
    idx_t = torch.tensor(idx, dtype=torch.int32, device=device if mode == "gpu_index" else "cpu")
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=is_mla, block_n=64,
                                    causal_query_seq_attn=causal, context_index=idx_t)
    ref = _packed_oracle(q, k, v, lengths, scale, is_mla=is_mla, causal=causal, k_cache=kc, v_cache=vc,
                         cu_kv=cu_kv, cbs=3, Tc=Tc, context_index=idx)
    _close(unpack_from_kernel(out, meta, H), ref)


@pytest.mark.parametrize("is_mla", [False, True])
def test_context_index_mla512_and_precompressed(is_mla, device):
    torch.manual_seed(4200 + is_mla)
    D = 512 if is_mla else 128
    lengths = [150, 3, 96]
    B, H, N = len(lengths), 2, 150
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16, std=0.5) for _ in range(3))
    torch.manual_seed(9)
    c1, kc, vc, cu_kv, Tc = _context_cache(B, H, D, is_mla, [65, 200], device, torch.bfloat16, std=0.5)
    torch.manual_seed(9)
    c2 = _context_cache(B, H, D, is_mla, [65, 200], device, torch.bfloat16, std=0.5)[0]
    idx = torch.tensor([1, 1, 0], dtype=torch.int32)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, c1, 0, is_mla=is_mla, block_n=64, context_index=idx)
    ref = _packed_oracle(q, k, v, lengths, scale, is_mla=is_mla, k_cache=kc, v_cache=vc, cu_kv=cu_kv, cbs=2,
                         Tc=Tc, context_index=idx.tolist())
    _close(unpack_from_kernel(out, meta, H), ref)
    q_p, k_p, v_p = _prepack(q, k, v, meta, is_mla)
    pre = flash_attn_mlm_precompressed(
        q_p, k_p, v_p, num_heads=H, total_q_len=q_p.shape[0] // H, cu_seqlens_q=meta.cu_seqlens,
        batch_ids_q=meta.batch_ids_q, q_tile_starts_q=meta.q_tile_starts_q, scale=scale, inference_cache=c2,
        layer_id=0, is_mla=is_mla, block_n=64, context_index=idx,
    )
    torch.testing.assert_close(pre, out, atol=1e-5, rtol=0)


@pytest.mark.parametrize("is_mla", [False, True])
def test_context_index_dense(is_mla, device):
    torch.manual_seed(4300 + is_mla)
    B, H, N, D, C, cbs = 3, 2, 77, 64, 45, 2
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    rows = cbs * C * (1 if is_mla else H)
    kc, vc = _randn((rows, D), device, torch.bfloat16), _randn((rows, D), device, torch.bfloat16)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=None if is_mla else vc, context_batch_size=cbs, is_mla=is_mla,
                           num_heads=H, head_dim=D, total_context_len=cbs * C)
    idx = [1, 1, 0]
    out = flash_attn_mlm(q, k, v, scale, inference_cache=cache, layer_id=0, is_mla=is_mla,
                         context_index=torch.tensor(idx))
    ref = ar.mlm_attention_dense(_np(q), _np(k), _np(v), scale, is_mla=is_mla, k_cache=_np(kc), v_cache=_np(vc),
                                 context_len=C, context_batch_size=cbs, context_index=idx)
    _close(out, ref)


def test_context_index_errors(device):
    B, H, N, D = 3, 2, 32, 64
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    cache = _context_cache(B, H, D, False, [5, 6], device)[0]  # 2 contexts for 3 sequences
    meta = build_pack_metadata(torch.tensor([32, 10, 20], device=device), N, block_n=32)
    run = lambda **kw: flash_attn_mlm_compressed(q, k, v, H, meta, 0.3, cache, 0, **kw)  # noqa: E731
    with pytest.raises(ValueError, match="must be 1 or at least the batch size"):
        run()  # 2 contexts for 3 sequences need an index
    with pytest.raises(ValueError, match=r"context_index values must lie in \[0, 2\)"):
        run(context_index=torch.tensor([0, 2, 1]))
    with pytest.raises(ValueError, match="one entry per sequence"):
        run(context_index=torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="int32 or int64"):
        run(context_index=torch.tensor([0.0, 1.0, 1.0]))
    with pytest.raises(ValueError, match="mutually exclusive"):
        run(context_index=torch.tensor([0, 1, 1]), context_batch_size=1)
    with pytest.raises(ValueError, match="prefill"):
        run(context_index=torch.tensor([0, 1, 1]), prefill=True)


def test_shared_context_override_on_multi_batch_entry(device):
    # context_batch_size=1 on a multi-batch entry -> cu_seqlens_kv = [0, total] (host_utils.py:232-237)
    torch.manual_seed(31)
    B, H, N, D = 3, 2, 40, 64
    lengths = [40, 12, 33]
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, False, [7, 11, 5], device)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=32)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.3, cache, 0, context_batch_size=1)
    ref = _packed_oracle(q, k, v, lengths, 0.3, k_cache=kc, v_cache=vc, cu_kv=[0, Tc], cbs=1, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)
    with pytest.raises(ValueError, match=r"context_batch_size \(2\) must match cached entry context_batch_size \(3\)"):
        flash_attn_mlm_compressed(q, k, v, H, meta, 0.3, cache, 0, context_batch_size=2)


@pytest.mark.parametrize("is_mla", [False, True])
def test_prefill_then_attend_round_trip(is_mla, device):
    # layer 0: prefill stores padded packed K/V; a second call attends to it as context
    torch.manual_seed(41)
    B, H, N, D = 3, 4, 50, 128
    lengths1, lengths2 = [50, 20, 33], [17, 50, 8]
    q1, k1, v1 = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    q2, k2, v2 = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    cache = InferenceCache()
    m1 = cache.packing.get_pack_metadata(torch.tensor(lengths1, device=device), N=N, block_n=16)
    m2 = cache.packing.get_pack_metadata(torch.tensor(lengths2, device=device), N=N, block_n=16)
    flash_attn_mlm_compressed(q1, k1, v1, H, m1, 0.2, cache, "L", is_mla=is_mla, block_n=16, prefill=True, auto_tune_tiles=True)
    entry = cache.get_kv_cache("L", is_mla=is_mla, num_heads=H, head_dim=D, dtype=torch.bfloat16, device=q1.device)
    out = flash_attn_mlm_compressed(q2, k2, v2, H, m2, 0.2, cache, "L", is_mla=is_mla, block_n=16)
    ref = _packed_oracle(q2, k2, v2, lengths2, 0.2, is_mla=is_mla, k_cache=entry.k_cache, v_cache=entry.v_cache,
                         cu_kv=_np(entry.cu_seqlens_kv).astype(int), cbs=B, Tc=entry.total_context_len)
    _close(unpack_from_kernel(out, m2, H), ref)
    # the context a sequence sees is exactly its own prefilled tokens
    ref_alt = ar.mlm_attention_packed(
        _np(q2), _np(k2), _np(v2), lengths2, 0.2, is_mla=is_mla,
    )
    assert not np.allclose(ref, ref_alt, atol=1e-3)


def test_non_contiguous_inputs(device):
    torch.manual_seed(61)
    B, H, N, D = 2, 4, 33, 64
    base = _randn((B, N, H, D), device, torch.bfloat16)
    q = base.permute(0, 2, 1, 3)  # strided [B, H, N, D]
    k = _randn((B, H, N, D), device, torch.bfloat16)
    v = _randn((B, H, N, D * 2), device, torch.bfloat16)[..., ::2]  # non-unit D stride
    lengths = [33, 19]
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, block_n=32)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.125)
    _close(unpack_from_kernel(out, meta, H), _packed_oracle(q, k, v, lengths, 0.125))
    dense = flash_attn_mlm(q, k, v, 0.125)
    _close(dense, ar.mlm_attention_dense(_np(q), _np(k), _np(v), 0.125))


def test_deterministic(device):
    torch.manual_seed(71)
    B, H, N, D = 4, 8, 300, 128
    q, k, v = (_randn((B, H, N, D), device) for _ in range(3))
    meta = build_pack_metadata(torch.tensor([300, 1, 257, 128], device=device), N, block_n=64)
    a = flash_attn_mlm_compressed(q, k, v, H, meta, 0.1, causal_query_seq_attn=True, block_n=64)
    b = flash_attn_mlm_compressed(q, k, v, H, meta, 0.1, causal_query_seq_attn=True, block_n=64)
    assert torch.equal(a, b)


def test_normalisation_and_extreme_logits(device):
    # V constant -> output exactly that constant (weights sum to one) even with huge logits
    torch.manual_seed(81)
    B, H, N, D = 2, 2, 300, 64
    q = _randn((B, H, N, D), device, torch.bfloat16, std=8.0)
    k = _randn((B, H, N, D), device, torch.bfloat16, std=8.0)
    v = torch.full((B, H, N, D), 0.75, device=device, dtype=torch.bfloat16)
    meta = build_pack_metadata(torch.tensor([300, 299], device=device), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 1.0, block_n=64)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), torch.full_like(out, 0.75).float(), atol=4e-3, rtol=0)


# ---------------------------------------------------------------------------
# BASELINE configs at full size
# ---------------------------------------------------------------------------
def _check_sampled(case, out_unpacked, pairs, rows=None):
    t = case.tensors
    for b, h in pairs:
        Lq = case.lengths_q[b]
        sel = np.arange(Lq) if rows is None else np.unique(np.linspace(0, Lq - 1, rows).astype(int))
        if case.cfg in (1, 2):
            qn = _np(t["q"][b, h, sel])
            K = _np(t["k"][b, h])
            V = K if case.is_mla else _np(t["v"][b, h])
            if case.cfg == 2:
                C = case.config["context"]
                K = np.concatenate([_np(t["k0"][0, h]), K])
                V = np.concatenate([_np(t["v0"][0, h]), V])
        else:
            keys = ar.packed_key_rows(b, case.lengths_q, case.causal)
            sb = torch.tensor([r[0] for r in keys], device=t["q"].device)
            pb = torch.tensor([r[1] for r in keys], device=t["q"].device)
            kh = 0 if case.is_mla else h
            K = _np(t["k"][sb, kh, pb])
            V = K if case.is_mla else _np(t["v"][sb, h, pb])
            if not case.prefill:
                cb = b if t["cbs"] > 1 else 0
                c0, c1 = int(t["cu_kv"][cb]), int(t["cu_kv"][cb + 1])
                off = 0 if case.is_mla else h * t["Tc"]
                Kc = _np(t["k_cache"][off + c0 : off + c1])
                Vc = Kc if case.is_mla else _np(t["v_cache"][off + c0 : off + c1])
                K, V = np.concatenate([Kc, K]), np.concatenate([Vc, V])
            qn = _np(t["q"][b, h, torch.tensor(sel, device=t["q"].device)])
        ref = ar.attend(qn, K, V, t["scale"])
        _close(out_unpacked[b, h, torch.tensor(sel, device=out_unpacked.device)], ref)


def _torch_attention_rows(case, b):
    """fp32 torch attention of every head of sequence b of a BASELINE case on the GPU:
    (query rows [H, L_b, D], the expected output rows [H, L_b, D]).  The key set is the
    one _check_sampled builds row by row: [context of b || main keys of b], main keys the
    packed tokens [cu[b], cu[b+1]), or [0, cu[b+1]) under causal_query_seq_attn."""
    t = case.tensors
    q, k, v = t["q"], t["k"], t["v"]
    L = case.lengths_q[b]
    if case.cfg in (1, 2):
        K, V = k[b].float(), v[b].float()
        if case.cfg == 2:
            K = torch.cat([t["k0"][0].float(), K], dim=1)
            V = torch.cat([t["v0"][0].float(), V], dim=1)
    else:
        kh = 1 if case.is_mla else case.H
        seqs = range(b + 1) if case.causal else [b]
        K = torch.cat([k[s, :kh, : case.lengths_q[s]].float() for s in seqs], dim=1)
        V = K if case.is_mla else torch.cat([v[s, :, : case.lengths_q[s]].float() for s in seqs], dim=1)
        if not case.prefill:
            cb = b if t["cbs"] > 1 else 0
            c0, c1 = int(t["cu_kv"][cb]), int(t["cu_kv"][cb + 1])
            Kc = t["k_cache"].view(kh, t["Tc"], -1)[:, c0:c1].float()
            Vc = Kc if case.is_mla else t["v_cache"].view(kh, t["Tc"], -1)[:, c0:c1].float()
            K, V = torch.cat([Kc, K], dim=1), torch.cat([Vc, V], dim=1)
    Q = q[b, :, :L].float()
    out = torch.empty_like(Q)
    step = 16  # heads per product: bounds the score buffer (config 5: 16 x 2048 x 10240 fp32)
    for h0 in range(0, case.H, step):
        qh = Q[h0 : h0 + step]
        kh_ = K if K.shape[0] == 1 else K[h0 : h0 + step]
        vh_ = V if V.shape[0] == 1 else V[h0 : h0 + step]
        s = torch.matmul(qh, kh_.transpose(1, 2).contiguous()) * t["scale"]
        out[h0 : h0 + step] = torch.matmul(torch.softmax(s, dim=-1), vh_)
    return Q, out


@pytest.mark.parametrize("cfg,variant", [(1, ""), (2, ""), (3, ""), (4, ""), (5, ""), (5, "prefill")])
def test_baseline_config_full_size(cfg, variant, device):
    """A BASELINE config at full size: every real row of every (sequence, head) against a
    per-sequence fp32 torch attention on the GPU (atol = rtol = 1e-2), four (sequence,
    head) pairs against the fp64 oracle, and zeros at the padding positions."""
    import bench

    case = bench.make_case(cfg, device, variant=variant)
    out = case.step()
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    B = len(case.lengths_q)
    H = case.H
    if cfg in (3, 4, 5):
        # padding positions are zeros after unpack
        N = out.shape[2]
        L = torch.tensor(case.lengths_q, device=device)
        pad = torch.arange(N, device=device)[None, :] >= L[:, None]
        assert bool((out.permute(0, 2, 1, 3)[pad] == 0).all())
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        worst = 0.0
        for b in range(B):
            _, ref = _torch_attention_rows(case, b)
            got = out[b, :, : case.lengths_q[b]].float()
            excess = (got - ref).abs() - (ATOL + RTOL * ref.abs())
            worst = max(worst, float(excess.max()) if excess.numel() else -1.0)
            assert worst <= 0, f"sequence {b}: |out - ref| exceeds atol + rtol*|ref| by {worst:.3e}"
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    rng = np.random.default_rng(cfg)
    pairs = [(0, 0), (B - 1, H - 1)] + [(int(rng.integers(B)), int(rng.integers(H))) for _ in range(2)]
    _check_sampled(case, out, pairs, rows=None if cfg in (1, 2, 4) else 64)


def test_abi_causal_over_padded_kv(device):
    # the C ABI also accepts causal_query_seq_attn over padded K/V (per-row sequence
    # lookup); the Python launchers pack first, so exercise that kernel path directly
    from flash_mlm import _lib
    from flash_mlm.host import host as hh

    torch.manual_seed(91)
    B, H, N, D = 4, 3, 70, 64
    lengths = [70, 5, 33, 64]
    q, k, v = (_randn((B, H, N, D), device, torch.bfloat16) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    T = meta.total_tokens
    out = torch.empty((H * T, D), dtype=q.dtype, device=device)
    empty = torch.empty((0, D), dtype=q.dtype, device=device)
    hh._launch(
        q=q, out=out, k=k, v=v, B=B, H=H, D=D, N=N, total_q=T, cu_seqlens_q=meta.cu_seqlens,
        q_strides=(q.stride(0), q.stride(1), q.stride(2)), q_layout=_lib.LAYOUT_PADDED,
        o_strides=(0, T * D, D), o_layout=_lib.LAYOUT_PACKED,
        k_strides=(k.stride(0), k.stride(1), k.stride(2)), v_strides=(v.stride(0), v.stride(1), v.stride(2)),
        kv_layout=_lib.LAYOUT_PADDED, k_ctx=empty, v_ctx=empty, c_strides=(0, 0, D), cu_seqlens_kv=None,
        ctx_len=0, ctx_batch=1, ctx_rows=0, scale=0.3, flags=_lib.FLAG_CAUSAL_SEQ, inference_cache=None,
    )
    _close(unpack_from_kernel(out, meta, H), _packed_oracle(q, k, v, lengths, 0.3, causal=True))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["ctx", "causal_ctx", "prefill", "shared_ctx"])
def test_mla_latent512_packed(dtype, mode, device):
    # MLA with a 512-wide latent (BASELINE config 5 shape class), odd lengths and tails
    torch.manual_seed(3000 + len(mode))
    lengths = [130, 1, 64, 97, 200]
    B, H, N, D = len(lengths), 6, 200, 512
    causal, prefill = "causal" in mode, mode == "prefill"
    q = _randn((B, H, N, D), device, dtype, std=0.5)
    k = _randn((B, H, N, D), device, dtype, std=0.5)
    ctx_lengths = [70, 0, 5, 129, 64]
    # shared_ctx: a per-sequence entry requested with context_batch_size=1 attends to all
    # cached rows [0, total) (host_utils.py:232-237)
    cache, kc, vc, cu_kv, Tc = _context_cache(B, H, D, True, ctx_lengths, device, dtype, std=0.5)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    cbs = 1 if mode == "shared_ctx" else B
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, cache, 0, is_mla=True, block_n=64,
                                    causal_query_seq_attn=causal, prefill=prefill,
                                    context_batch_size=1 if mode == "shared_ctx" else None)
    cu_ref = [0, Tc] if mode == "shared_ctx" else cu_kv
    ref = _packed_oracle(q, k, k, lengths, scale, is_mla=True, causal=causal, prefill=prefill,
                         k_cache=kc, cu_kv=cu_ref, cbs=cbs, Tc=Tc)
    _close(unpack_from_kernel(out, meta, H), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mla_latent512_rising_scores(dtype, device):
    """Scores that rise along the keys by more than the rescale slack every 32 keys: each
    half of every 64-key latent tile raises the running maximum, so the kernel rescales
    O, l and the already computed P of the tile's first half at every step."""
    torch.manual_seed(3100)
    lengths = [300, 77]
    B, H, N, D = len(lengths), 2, 300, 512
    q = _randn((B, H, N, D), device, dtype, std=0.5)
    k = _randn((B, H, N, D), device, dtype, std=0.5)
    q[..., 0] = 4.0
    # +12 (log2 units) per 32 keys: 4 * 1.5 * 32 * scale * log2(e)
    ramp = torch.arange(N, device=device, dtype=torch.float32) * 1.5
    k[:, 0, :, 0] = ramp.to(dtype)  # MLA: head 0 of k is the latent
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, is_mla=True, block_n=64)
    assert torch.isfinite(out).all()
    ref = _packed_oracle(q, k, k, lengths, scale, is_mla=True)
    _close(unpack_from_kernel(out, meta, H), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mla_latent512_rescale_inside_tile(dtype, device):
    """A tile's second half raises the maximum of some rows of a wave by ~10 (log2 units),
    past the rescale slack, and leaves the others' (so the whole wave rescales, with
    factor 1 on those rows): the first half's P, computed against the old maximum, must
    keep each of its elements.  Its keys carry scores of +2 (keys 4g, 4g+1 of the first
    16-key block) and -2 (the rest), so P elements that trade places show, in the
    output's dim 1 (the latent is V: dim 1 holds the +-8 that set those scores)."""
    torch.manual_seed(3200)
    lengths = [64, 100]
    B, H, N, D = len(lengths), 2, 100, 512
    q = _randn((B, H, N, D), device, dtype, std=0.5)
    k = _randn((B, H, N, D), device, dtype, std=0.5)
    # dim d adds q_d * k_d * scale * log2(e) = 0.255 * k_d (log2 units) for q_d = 4
    q[:, :, 0::2, 0] = 4.0  # even positions see key 40's boost, odd ones do not
    q[:, :, 1::2, 0] = 0.0
    q[..., 1] = 4.0
    key = torch.arange(N, device=device)
    k0 = torch.zeros(N, device=device)
    k0[32:64] = -40.0
    k0[40] = 48.0  # +12.2 on even positions: their maximum rises by ~10 in the second half
    k1 = torch.where((key < 16) & (key % 4 < 2), 8.0, -8.0)
    k1[32:] = 0.0
    k[:, 0, :, 0] = k0.to(dtype)  # MLA: head 0 of k is the latent
    k[:, 0, :, 1] = k1.to(dtype)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, is_mla=True, block_n=64)
    ref = _packed_oracle(q, k, k, lengths, scale, is_mla=True)
    _close(unpack_from_kernel(out, meta, H), ref)


@pytest.mark.parametrize("cbs", [1, 2])
def test_mla_latent512_dense(cbs, device):
    torch.manual_seed(3100 + cbs)
    B, H, N, D, C = 2, 4, 150, 512, 77
    q = _randn((B, H, N, D), device, torch.bfloat16, std=0.5)
    k = _randn((B, H, N, D), device, torch.bfloat16, std=0.5)
    kc = _randn((cbs * C, D), device, torch.bfloat16, std=0.5)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, context_batch_size=cbs, is_mla=True, num_heads=H, head_dim=D)
    out = flash_attn_mlm(q, k, k, 1.0 / math.sqrt(D), inference_cache=cache, layer_id=0, is_mla=True)
    ref = ar.mlm_attention_dense(_np(q), _np(k), _np(k), 1.0 / math.sqrt(D), is_mla=True, k_cache=_np(kc),
                                 context_len=C, context_batch_size=cbs)
    _close(out, ref)
