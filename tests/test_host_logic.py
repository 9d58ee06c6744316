"""Host-side logic of the flash_mlm package on CPU: caches, cache-context resolution,
validators and error contract (reference: src/flash_mlm/host/cache.py,
host_utils.py:142-263,292-394; KATs test_host_utils.py:154-232, 314-420)."""

from __future__ import annotations

import json

import pytest
import torch

from conftest import GOLDEN
from flash_mlm import InferenceCache, PackingCache, PackMetadata
from flash_mlm.host import host_utils as hu
from flash_mlm.host.host import flash_attn_mlm, flash_attn_mlm_compressed, flash_attn_mlm_precompressed

KATS = json.loads((GOLDEN / "reference_kats.json").read_text())
CPU = torch.device("cpu")


def test_packing_cache_reuses_allocation_for_smaller_rows():
    cache = PackingCache()
    first = cache.get_2d("q", rows=8, cols=4, dtype=torch.float32, device=CPU)
    second = cache.get_2d("q", rows=6, cols=4, dtype=torch.float32, device=CPU)
    assert first.untyped_storage().data_ptr() == second.untyped_storage().data_ptr()
    assert second.shape == (6, 4)
    grown = cache.get_2d("q", rows=9, cols=4, dtype=torch.float32, device=CPU)
    assert grown.shape == (9, 4)
    other = cache.get_2d("q", rows=2, cols=5, dtype=torch.float32, device=CPU)
    assert other.untyped_storage().data_ptr() != grown.untyped_storage().data_ptr()


def test_packing_cache_rejects_bad_shapes():
    cache = PackingCache()
    with pytest.raises(ValueError, match="rows must be >= 0"):
        cache.get_2d("q", rows=-1, cols=1, dtype=torch.float32, device=CPU)
    with pytest.raises(ValueError, match="cols must be >= 1"):
        cache.get_2d("q", rows=1, cols=0, dtype=torch.float32, device=CPU)


def test_packing_cache_memoizes_metadata(monkeypatch):
    calls = []

    def fake_build(lengths, N, block_n):
        calls.append((tuple(lengths.tolist()), N, block_n))
        return object()

    monkeypatch.setattr(hu, "build_pack_metadata", fake_build)
    cache = PackingCache()
    lengths = torch.tensor([4, 2], dtype=torch.int32)
    m1 = cache.get_pack_metadata(lengths, N=4, block_n=3)
    m2 = cache.get_pack_metadata(lengths.clone(), N=4, block_n=3)
    m3 = cache.get_pack_metadata(lengths.to(torch.int64), N=4, block_n=3)
    assert m1 is m2 is m3 and len(calls) == 1
    assert cache.get_pack_metadata(lengths, N=4, block_n=2) is not m1
    assert cache.get_pack_metadata(torch.tensor([4, 1]), N=4, block_n=3) is not m1
    cache.clear()
    assert cache.get_pack_metadata(lengths, N=4, block_n=3) is not m1


@pytest.mark.parametrize("case", KATS["cache_context"], ids=lambda c: c["kind"])
def test_maybe_get_cache_context_reference_kats(case):
    cache = InferenceCache()
    d = case["d"]
    k_cache = torch.arange(case["k_rows"] * d, dtype=torch.float32).view(case["k_rows"], d)
    v_cache = None if case["is_mla"] else k_cache + 1000
    cu = None if case.get("cu_seqlens_kv") is None else torch.tensor(case["cu_seqlens_kv"], dtype=torch.int32)
    cache.prefill_kv_cache(
        0,
        k_cache=k_cache,
        v_cache=v_cache,
        total_context_len=case["total_context_len"],
        cu_seqlens_kv=cu,
        context_batch_size=case["stored_cbs"],
        is_mla=case["is_mla"],
        num_heads=case["num_heads"],
        head_dim=d,
    )
    ctx = hu._maybe_get_cache_context(
        inference_cache=cache,
        layer_id=0,
        batch_size=case["batch_size"],
        num_heads=case["num_heads"],
        head_dim=d,
        is_mla=case["is_mla"],
        context_batch_size=case["request_cbs"],
        device=CPU,
        dtype=torch.float32,
        compressed=case["expect_cu"] is not None,
    )
    assert ctx.context_batch_size == case["expect_cbs"]
    assert ctx.total_context_len == case["expect_total"]
    assert ctx.k_cache is k_cache
    if v_cache is not None:
        assert ctx.v_cache is v_cache
    if case["expect_cu"] is None:
        assert ctx.cu_seqlens_kv is None
        assert ctx.context_len == case["expect_context_len"]
    else:
        assert ctx.cu_seqlens_kv.tolist() == case["expect_cu"]


def test_cache_context_miss_is_empty_and_mismatch_is_silent():
    cache = InferenceCache()
    k = torch.zeros(6, 4)
    cache.prefill_kv_cache(1, k_cache=k, v_cache=k.clone(), context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    for kwargs in (
        dict(layer_id=2, is_mla=False, num_heads=2, head_dim=4, dtype=torch.float32),  # missing layer
        dict(layer_id=1, is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32),  # mode mismatch
        dict(layer_id=1, is_mla=False, num_heads=3, head_dim=4, dtype=torch.float32),  # heads mismatch
        dict(layer_id=1, is_mla=False, num_heads=2, head_dim=4, dtype=torch.float16),  # dtype mismatch
    ):
        ctx = hu._maybe_get_cache_context(
            inference_cache=cache,
            batch_size=3,
            context_batch_size=None,
            device=CPU,
            compressed=True,
            **kwargs,
        )
        assert ctx.total_context_len == 0 and ctx.k_cache.shape == (0, kwargs["head_dim"])
        assert ctx.context_batch_size == 3 and ctx.cu_seqlens_kv.tolist() == [0, 0, 0, 0]


def test_cache_context_errors():
    cache = InferenceCache()
    k = torch.zeros(6, 4)
    cache.prefill_kv_cache(0, k_cache=k, v_cache=k.clone(), context_batch_size=3, is_mla=False, num_heads=2, head_dim=4)
    common = dict(inference_cache=cache, layer_id=0, batch_size=3, num_heads=2, head_dim=4, is_mla=False, device=CPU, dtype=torch.float32)
    with pytest.raises(ValueError, match=r"context_batch_size \(2\) must match cached entry context_batch_size \(3\)"):
        hu._maybe_get_cache_context(context_batch_size=2, compressed=True, **common)
    # dense: uniform 1 token per batch -> context_len 1; packed without cu: arange * 1
    ctx = hu._maybe_get_cache_context(context_batch_size=None, compressed=False, **common)
    assert ctx.context_len == 1 and ctx.context_batch_size == 3
    ctx = hu._maybe_get_cache_context(context_batch_size=None, compressed=True, **common)
    assert ctx.cu_seqlens_kv.tolist() == [0, 1, 2, 3]


def test_inference_cache_validation_messages():
    cache = InferenceCache()
    k = torch.zeros(6, 4)
    with pytest.raises(ValueError, match="context_batch_size must be >= 1"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, context_batch_size=0, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="num_heads must be >= 1"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, context_batch_size=1, is_mla=False, num_heads=0, head_dim=4)
    with pytest.raises(ValueError, match="non-MLA k_cache rows must be divisible by num_heads"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, context_batch_size=1, is_mla=False, num_heads=4, head_dim=4)
    with pytest.raises(ValueError, match="non-MLA cache requires v_cache"):
        cache.prefill_kv_cache(0, k_cache=k, context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="k_cache second dim must match head_dim"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, context_batch_size=1, is_mla=False, num_heads=2, head_dim=8)
    with pytest.raises(ValueError, match="k_cache must be a rank-2 packed tensor"):
        cache.prefill_kv_cache(0, k_cache=k.view(2, 3, 4), v_cache=k, context_batch_size=1, is_mla=True, num_heads=2, head_dim=4, total_context_len=2)
    with pytest.raises(ValueError, match="k_cache must be contiguous"):
        cache.prefill_kv_cache(0, k_cache=torch.zeros(4, 6).t(), v_cache=k, context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="v_cache shape must match k_cache shape"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=torch.zeros(4, 4), context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="MLA v_cache shape must match k_cache shape"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=torch.zeros(4, 4), context_batch_size=1, is_mla=True, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="k_cache first dim mismatch: expected 10 rows for is_mla=False"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, total_context_len=5, context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="total_context_len must be divisible by context_batch_size"):
        cache.prefill_kv_cache(0, k_cache=torch.zeros(5, 4), context_batch_size=2, is_mla=True, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="cu_seqlens_kv must be rank-1 with at least 2 elements"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=torch.tensor([0]), context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    with pytest.raises(ValueError, match="context_batch_size is incompatible with cu_seqlens_kv length"):
        cache.prefill_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=torch.tensor([0, 3]), context_batch_size=2, is_mla=False, num_heads=2, head_dim=4)


def test_inference_cache_stores_views_and_replaces():
    cache = InferenceCache()
    k1, v1 = torch.zeros(6, 4), torch.ones(6, 4)
    cache.prefill_kv_cache("L0", k_cache=k1, v_cache=v1, context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    e = cache.get_kv_cache("L0", is_mla=False, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU)
    assert e.k_cache is k1 and e.v_cache is v1 and e.total_context_len == 3 and e.cu_seqlens_kv is None
    k2 = torch.zeros(4, 4)
    cache.prefill_kv_cache("L0", k_cache=k2, v_cache=k2, context_batch_size=1, is_mla=True, num_heads=2, head_dim=4)
    e = cache.get_kv_cache("L0", is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU)
    assert e.k_cache is k2 and e.v_cache is None and e.total_context_len == 4  # MLA drops v
    with pytest.raises(ValueError, match="Cached KV mode \\(is_mla\\) does not match request"):
        cache.get_kv_cache("L0", is_mla=False, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU)
    with pytest.raises(ValueError, match="Cached num_heads does not match request"):
        cache.get_kv_cache("L0", is_mla=True, num_heads=3, head_dim=4, dtype=torch.float32, device=CPU)
    with pytest.raises(ValueError, match="Cached head_dim does not match request"):
        cache.get_kv_cache("L0", is_mla=True, num_heads=2, head_dim=8, dtype=torch.float32, device=CPU)
    with pytest.raises(ValueError, match="Cached KV dtype does not match request"):
        cache.get_kv_cache("L0", is_mla=True, num_heads=2, head_dim=4, dtype=torch.float16, device=CPU)
    # int and str layer ids share a key space, as in the reference
    assert cache.get_kv_cache("L0", is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU) is e
    cache.prefill_kv_cache(3, k_cache=k2, context_batch_size=1, is_mla=True, num_heads=2, head_dim=4)
    assert cache.get_kv_cache("3", is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU).k_cache is k2
    cache.clear_layer(3)
    with pytest.raises(ValueError, match="No cached KV context for layer_id=3"):
        cache.get_kv_cache(3, is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU)
    cache.clear()
    with pytest.raises(ValueError, match="No cached KV context"):
        cache.get_kv_cache("L0", is_mla=True, num_heads=2, head_dim=4, dtype=torch.float32, device=CPU)


def test_validators():
    with pytest.raises(ValueError, match="prefill=True requires inference_cache"):
        hu.validate_cache_request(prefill=True, inference_cache=None, layer_id=None)
    with pytest.raises(ValueError, match="inference_cache and layer_id must be provided together or both omitted"):
        hu.validate_cache_request(prefill=False, inference_cache=InferenceCache(), layer_id=None)
    hu.validate_cache_request(prefill=False, inference_cache=None, layer_id=None)
    x = torch.zeros(1, 2, 3, 4)
    with pytest.raises(ValueError, match=r"q/k/v must be rank-4 tensors \[B, H, N, D\]"):
        hu.validate_qkv_same_shape_rank4(x[0], x, x, error_prefix="q/k/v")
    with pytest.raises(ValueError, match="q, k, v must have the same shape"):
        hu.validate_qkv_same_shape_rank4(x, x, torch.zeros(1, 2, 3, 5), error_prefix="q/k/v")
    assert hu.validate_qkv_same_shape_rank4(x, x, x, error_prefix="q/k/v") == (1, 2, 3, 4)
    for d in (16, 32, 64, 128, 256):
        hu.validate_head_dim_supported(d)
    for d in (8, 48, 512):
        with pytest.raises(ValueError, match=r"HEAD_DIM must be one of \{16, 32, 64, 128, 256\}"):
            hu.validate_head_dim_supported(d)
    hu.validate_head_dim_supported(512, is_mla=True)
    with pytest.raises(ValueError, match="cu_seqlens tensors must be rank-1"):
        hu.validate_cu_seqlens_rank1_min2(torch.zeros(2, 2))
    with pytest.raises(ValueError, match="cu_seqlens tensors must have at least 2 elements"):
        hu.validate_cu_seqlens_rank1_min2(torch.zeros(1))
    with pytest.raises(ValueError, match="All tensors must be CUDA tensors"):
        hu.require_cuda_tensors(x, None)
    with pytest.raises(ValueError, match="k_cache first dim mismatch: expected 6 rows for is_mla=False"):
        hu.validate_packed_cache_shapes(torch.zeros(5, 4), torch.zeros(5, 4), num_heads=2, total_context_len=3, head_dim=4, is_mla=False)
    with pytest.raises(ValueError, match="k_cache second dim must match q/k/v head_dim"):
        hu.validate_packed_cache_shapes(torch.zeros(6, 4), torch.zeros(6, 4), num_heads=2, total_context_len=3, head_dim=8, is_mla=False)
    hu.validate_packed_cache_shapes(torch.zeros(3, 4), None, num_heads=2, total_context_len=3, head_dim=4, is_mla=True)


def test_padded_length_accepts_host_and_tensor_cumsums():
    assert hu._compute_total_q_len_padded(6, torch.tensor([0, 4, 6], dtype=torch.int32), 4, 4) == 8
    assert hu._compute_total_q_len_padded(6, (0, 4, 6), 4, 4) == 8
    assert hu._compute_total_q_len_padded(6, (0, 4, 6), 1, 1) == 6
    assert hu._compute_total_q_len_padded(0, (0,), 64, 32) == 0


def test_compute_paths_refuse_cpu_tensors():
    # there is no CPU compute path: CPU inputs raise with the reference's messages
    q = torch.zeros(1, 2, 4, 16)
    with pytest.raises(ValueError, match="All tensors must be CUDA tensors"):
        flash_attn_mlm(q, q, q, scale=1.0)
    meta = PackMetadata(
        B=1, N=4, lengths=torch.tensor([4], dtype=torch.int32), cu_seqlens=torch.tensor([0, 4], dtype=torch.int32),
        token_indices=torch.arange(4), total_tokens=4, batch_ids_block_n=32,
        batch_ids_q=torch.zeros(1, dtype=torch.int32), q_tile_starts_q=torch.zeros(1, dtype=torch.int32),
    )
    with pytest.raises(ValueError, match="All tensors must be CUDA tensors"):
        flash_attn_mlm_compressed(q, q, q, num_heads=2, q_meta=meta, scale=1.0)
    with pytest.raises(ValueError, match="prefill=True requires inference_cache"):
        flash_attn_mlm_compressed(q, q, q, num_heads=2, q_meta=meta, scale=1.0, prefill=True)
    with pytest.raises(ValueError, match="q_meta was built with different block_n"):
        flash_attn_mlm_compressed(q, q, q, num_heads=2, q_meta=meta, scale=1.0, block_n=16)
    with pytest.raises(ValueError, match="q/k/v head dimension must match num_heads"):
        flash_attn_mlm_compressed(q, q, q, num_heads=3, q_meta=meta, scale=1.0)
    p = torch.zeros(8, 16)
    with pytest.raises(ValueError, match="q/k/v must be pre-packed rank-2 tensors"):
        flash_attn_mlm_precompressed(q, p, p, 2, 4, meta.cu_seqlens, meta.batch_ids_q, meta.q_tile_starts_q, 1.0)
    with pytest.raises(ValueError, match="All tensors must be CUDA tensors"):
        flash_attn_mlm_precompressed(p, p, p, 2, 4, meta.cu_seqlens, meta.batch_ids_q, meta.q_tile_starts_q, 1.0)
    with pytest.raises(ValueError, match="block_n must be >= 1"):
        hu.build_pack_metadata(torch.tensor([1, 1]), 2, 0)
    with pytest.raises(ValueError, match="no CPU compute path"):
        hu.build_pack_metadata(torch.tensor([1, 1]), 2, 1)
    with pytest.raises(ValueError, match="no CPU compute path"):
        hu.pack_for_kernel(q, meta)
    with pytest.raises(ValueError, match="no CPU compute path"):
        hu.unpack_from_kernel(torch.zeros(8, 16), meta, 2)


def test_layer_entry_returns_the_stored_tensors():
    cache = InferenceCache()
    k = torch.zeros(6, 4, requires_grad=True)
    v = torch.zeros(6, 4)
    cache.prefill_kv_cache("x", k_cache=k, v_cache=v, context_batch_size=1, is_mla=False, num_heads=2, head_dim=4)
    entry = cache.layer_entry("x")
    assert entry.k_cache is k and entry.v_cache is v  # gradients reach the caller's tensors
    assert cache.layer_entry("y") is None


def test_backward_available_for_every_forward_head_dim_and_dtype():
    from flash_mlm.host import host as hh

    for dt in (torch.bfloat16, torch.float16, torch.float32):
        q = torch.zeros(1, dtype=dt)
        for d in (16, 32, 64, 128, 256, 512):
            assert hh._backward_unsupported(q, d, None, is_mla=False) is None
    assert "bf16, fp16 or fp32" in hh._backward_unsupported(torch.zeros(1, dtype=torch.float64), 64, None, False)
    assert "head_dim" in hh._backward_unsupported(torch.zeros(1, dtype=torch.float32), 48, None, False)
