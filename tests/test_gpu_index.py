"""GPU parity of the HIP indexing kernels (pack metadata, tile map, pack, pad, unpack)
against the reference's known-answer tests and the numpy oracle: bit-exact."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from flash_mlm import InferenceCache, PackingCache, build_pack_metadata, unpack_from_kernel
from flash_mlm.host import host_utils as hu
from oracle import pack_ref

pytestmark = pytest.mark.gpu
KATS = json.loads((GOLDEN / "reference_kats.json").read_text())


def _np(t):
    return t.detach().cpu().numpy()


def _check_meta(meta, ref):
    assert meta.B == ref.B and meta.N == ref.N and meta.total_tokens == ref.total_tokens
    assert meta.cu_seqlens.dtype == torch.int32 and meta.token_indices.dtype == torch.int64
    assert meta.batch_ids_q.dtype == torch.int32 and meta.q_tile_starts_q.dtype == torch.int32
    assert meta.lengths.dtype == torch.int32
    np.testing.assert_array_equal(_np(meta.lengths), ref.lengths)
    np.testing.assert_array_equal(_np(meta.cu_seqlens), ref.cu_seqlens)
    np.testing.assert_array_equal(_np(meta.token_indices), ref.token_indices)
    np.testing.assert_array_equal(_np(meta.batch_ids_q), ref.batch_ids)
    np.testing.assert_array_equal(_np(meta.q_tile_starts_q), ref.tile_starts)
    assert meta.batch_ids_block_n == ref.block_n
    assert hu.num_query_tiles_from_meta(meta) == ref.batch_ids.size


@pytest.mark.parametrize("case", KATS["pack_metadata"], ids=lambda c: c["line"])
def test_metadata_reference_kat(case, device):
    meta = build_pack_metadata(torch.tensor(case["lengths"], dtype=torch.int32, device=device), case["N"], case["block_n"])
    if "cu_seqlens" in case:
        assert meta.total_tokens == case["total_tokens"]
        assert _np(meta.cu_seqlens).tolist() == case["cu_seqlens"]
        assert _np(meta.token_indices).tolist() == case["token_indices"]
        assert _np(meta.batch_ids_q).tolist() == case["batch_ids_q"]
        assert _np(meta.q_tile_starts_q).tolist() == case["q_tile_starts_q"]
    if "num_tiles" in case:
        assert hu.num_query_tiles_from_meta(meta) == case["num_tiles"]


def test_metadata_errors(device):
    with pytest.raises(ValueError, match="block_n must be >= 1"):
        build_pack_metadata(torch.tensor([1, 1], device=device), 2, 0)
    with pytest.raises(ValueError, match=r"lengths values must be in \[0, N\]"):
        build_pack_metadata(torch.tensor([1, 3], device=device), 2, 1)
    with pytest.raises(ValueError, match=r"lengths values must be in \[0, N\]"):
        build_pack_metadata(torch.tensor([-1, 1], device=device, dtype=torch.int64), 2, 1)
    with pytest.raises(ValueError, match=r"lengths values must be in \[0, N\]"):
        build_pack_metadata(torch.tensor([1, 2**40], device=device, dtype=torch.int64), 2, 1)
    with pytest.raises(ValueError, match=r"lengths must be rank-1 \[B\]"):
        build_pack_metadata(torch.zeros(2, 2, dtype=torch.int32, device=device), 2, 1)


@pytest.mark.parametrize("seed", range(8))
def test_metadata_random_vs_oracle(seed, device):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(0, 3000)) if seed == 7 else int(rng.integers(1, 70))
    N = int(rng.integers(1, 2100))
    block_n = int(rng.choice([1, 3, 16, 32, 64, 128, 1000]))
    L = rng.integers(0, N + 1, size=B)
    if seed % 3 == 0 and B:
        L[rng.integers(0, B)] = 0
        L[rng.integers(0, B)] = N
    dtype = torch.int64 if seed % 2 else torch.int32
    meta = build_pack_metadata(torch.tensor(L, dtype=dtype, device=device), N, block_n)
    _check_meta(meta, pack_ref.pack_metadata(L, N, block_n))


def test_metadata_empty_batch(device):
    # B = 0: the reference's tile map rejects cu_seqlens = [0] (host_utils.py:78-79)
    with pytest.raises(ValueError, match="cu_seqlens_q must have at least 2 elements"):
        build_pack_metadata(torch.zeros(0, dtype=torch.int32, device=device), 16, 4)
    with pytest.raises(ValueError, match="cu_seqlens_q must have at least 2 elements"):
        pack_ref.pack_metadata(np.zeros(0, dtype=np.int32), 16, 4)
    meta = build_pack_metadata(torch.zeros(3, dtype=torch.int32, device=device), 0, 4)
    _check_meta(meta, pack_ref.pack_metadata(np.zeros(3, dtype=np.int32), 0, 4))


@pytest.mark.parametrize("case", KATS["tile_map"], ids=lambda c: c["line"])
def test_tile_map_reference_kat(case, device):
    cu = torch.tensor(case["cu_seqlens"], dtype=torch.int32, device=device)
    assert _np(hu.build_batch_ids_from_cu_seqlens(cu, case["block_n"])).tolist() == case["batch_ids"]
    assert _np(hu.build_q_tile_starts_from_cu_seqlens(cu, case["block_n"])).tolist() == case["q_tile_starts"]
    assert hu.num_query_tiles_from_cu_seqlens(cu, case["block_n"]) == case["num_tiles"]


@pytest.mark.parametrize("seed", range(4))
def test_tile_map_random_vs_oracle(seed, device):
    rng = np.random.default_rng(50 + seed)
    L = rng.integers(0, 300, size=int(rng.integers(1, 2500)))
    cu = np.concatenate([[0], np.cumsum(L)]).astype(np.int32)
    bn = int(rng.integers(1, 100))
    starts, bids = hu._build_query_tile_map_from_cu_seqlens(torch.tensor(cu, device=device), bn)
    rs, rb = pack_ref.tile_map(cu, bn)
    np.testing.assert_array_equal(_np(starts), rs)
    np.testing.assert_array_equal(_np(bids), rb)


@pytest.mark.parametrize("case", KATS["pack_for_kernel"], ids=lambda c: c["line"])
def test_pack_reference_kat(case, device):
    meta = build_pack_metadata(torch.tensor(case["lengths"], dtype=torch.int32, device=device), case["N"], case["block_n"])
    x = torch.arange(int(np.prod(case["x_shape"])), dtype=torch.float32, device=device).view(case["x_shape"])
    assert _np(hu.pack_for_kernel(x, meta, flatten_for_kernel=False)).tolist() == case["nonflat"]
    assert _np(hu.pack_for_kernel(x, meta, flatten_for_kernel=True)).tolist() == case["flat"]


@pytest.mark.parametrize("case", KATS["unpack"], ids=lambda c: c["line"])
def test_unpack_reference_kat(case, device):
    meta = build_pack_metadata(torch.tensor(case["lengths"], dtype=torch.int32, device=device), case["N"], case["block_n"])
    x = torch.arange(int(np.prod(case["x_shape"])), dtype=torch.float32, device=device).view(case["x_shape"])
    restored = unpack_from_kernel(hu.pack_for_kernel(x, meta, flatten_for_kernel=True), meta, H=2)
    expected = x.clone()
    expected[1, :, 2:, :] = 0
    assert torch.equal(restored, expected)
    # rank-3 input [H, T, D]
    assert torch.equal(unpack_from_kernel(hu.pack_for_kernel(x, meta), meta, H=2), expected)


@pytest.mark.parametrize("case", KATS["pad_packed"], ids=lambda c: c["line"])
def test_pad_packed_reference_kat(case, device):
    H, T, d = case["num_heads"], case["total_q_len_unpadded"], case["d"]
    q = torch.arange(H * T, dtype=torch.float32, device=device).view(-1, d)
    k = q.clone()
    cu = torch.tensor(case["cu_seqlens"], dtype=torch.int32, device=device)
    for cache in (None, PackingCache()):
        q_p, k_p, v_p, T_pad = hu.pad_packed_main_tensors_for_mlm_compressed(
            q, k, k.clone(), num_heads=H, is_mla=False, total_q_len_unpadded=T, cu_seqlens_q=cu,
            block_m=case["block_m"], block_n=case["block_n"], packing_cache=cache,
        )
        assert T_pad == case["total_q_len_padded"]
        assert q_p.shape == (H * T_pad, d) and k_p.shape == v_p.shape == (H * T_pad, d)
        assert _np(q_p)[:, 0].tolist() == case["q_col0"]
        if cache is not None:
            for name, t in (("q", q_p), ("k", k_p), ("v", v_p)):
                buf = cache.get_2d(name, rows=16, cols=1, dtype=torch.float32, device=device)
                assert t.untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()


@pytest.mark.parametrize("case", KATS["pack_and_pad_mla"], ids=lambda c: c["line"])
def test_pack_and_pad_mla_reference_kat(case, device):
    cache = PackingCache()
    meta = cache.get_pack_metadata(torch.tensor(case["lengths"], dtype=torch.int32, device=device), N=case["N"], block_n=case["block_n"])
    q = torch.arange(2 * 2 * 4, dtype=torch.float32, device=device).view(2, 2, 4, 1)
    q_out, k_out, v_out, T_pad = hu.pack_and_pad_main_tensors_for_mlm_compressed(
        q, q + 10, q + 20, q_meta=meta, num_heads=case["num_heads"], is_mla=True,
        block_m=case["block_m"], block_n=case["block_n"], packing_cache=cache,
    )
    assert T_pad == case["total_q_len"]
    assert tuple(q_out.shape) == tuple(case["q_out_shape"]) and tuple(k_out.shape) == tuple(case["k_out_shape"])
    assert v_out is k_out
    assert q_out.untyped_storage().data_ptr() == cache.get_2d("q", 16, 1, dtype=torch.float32, device=device).untyped_storage().data_ptr()
    assert k_out.untyped_storage().data_ptr() == cache.get_2d("k", 8, 1, dtype=torch.float32, device=device).untyped_storage().data_ptr()
    m = pack_ref.pack_metadata(np.array(case["lengths"]), case["N"], case["block_n"])
    qn = _np(q)
    np.testing.assert_array_equal(_np(q_out), pack_ref.pack(qn, m, T_pad))
    np.testing.assert_array_equal(_np(k_out), pack_ref.pack(qn[:, :1] + 10, m, T_pad))


def test_pack_and_pad_matches_two_step(device):
    # test_host_utils.py:235-272: fused pack+pad == pack_for_kernel then pad
    meta = build_pack_metadata(torch.tensor([4, 2], dtype=torch.int32, device=device), N=4, block_n=4)
    q = torch.arange(2 * 2 * 4, dtype=torch.float32, device=device).view(2, 2, 4, 1)
    k, v = q + 100, q + 200
    refs = [hu.pack_for_kernel(t, meta, flatten_for_kernel=True) for t in (q, k, v)]
    q_r, k_r, v_r, t_r = hu.pad_packed_main_tensors_for_mlm_compressed(
        *refs, num_heads=2, is_mla=False, total_q_len_unpadded=meta.total_tokens, cu_seqlens_q=meta.cu_seqlens, block_m=4, block_n=4
    )
    q_n, k_n, v_n, t_n = hu.pack_and_pad_main_tensors_for_mlm_compressed(
        q, k, v, q_meta=meta, num_heads=2, is_mla=False, block_m=4, block_n=4
    )
    assert t_n == t_r
    for a, b in ((q_n, q_r), (k_n, k_r), (v_n, v_r)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.int64, torch.uint8])
@pytest.mark.parametrize("seed", range(3))
def test_pack_unpack_random_vs_oracle(dtype, seed, device):
    rng = np.random.default_rng(200 + seed)
    B, H, N = int(rng.integers(1, 12)), int(rng.integers(1, 6)), int(rng.integers(1, 300))
    D = int(rng.choice([1, 3, 8, 16, 64, 128]))
    L = rng.integers(0, N + 1, size=B)
    block_n, block_m = int(rng.integers(1, 70)), int(rng.integers(1, 130))
    meta = build_pack_metadata(torch.tensor(L, dtype=torch.int32, device=device), N, block_n)
    ref_meta = pack_ref.pack_metadata(L, N, block_n)
    if dtype.is_floating_point:
        x = torch.randn(B, H, N, D, device=device).to(dtype)
    else:
        x = torch.randint(0, 100, (B, H, N, D), device=device).to(dtype)
    xn = _np(x.float() if dtype == torch.bfloat16 else x)
    flat = hu.pack_for_kernel(x, meta, flatten_for_kernel=True)
    np.testing.assert_array_equal(_np(flat.float() if dtype == torch.bfloat16 else flat), pack_ref.pack(xn, ref_meta))
    T_pad = pack_ref.total_q_len_padded(ref_meta.total_tokens, ref_meta.cu_seqlens, block_m, block_n)
    out = torch.full((H * T_pad, D), 7, dtype=dtype, device=device)
    hu._pack_flatten_for_kernel_into(x, meta, H, T_pad, out)
    np.testing.assert_array_equal(_np(out.float() if dtype == torch.bfloat16 else out), pack_ref.pack(xn, ref_meta, T_pad))
    restored = unpack_from_kernel(flat, meta, H)
    np.testing.assert_array_equal(_np(restored.float() if dtype == torch.bfloat16 else restored), pack_ref.unpack(pack_ref.pack(xn, ref_meta), ref_meta, H))


def test_pack_non_contiguous_source(device):
    L = np.array([5, 0, 9, 3])
    meta = build_pack_metadata(torch.tensor(L, device=device), 9, 4)
    base = torch.randn(4, 9, 3, 32, device=device, dtype=torch.float16)
    x = base.permute(0, 2, 1, 3)  # [B, H, N, D] view with non-standard strides
    ref = pack_ref.pack(_np(x.float()), pack_ref.pack_metadata(L, 9, 4))
    np.testing.assert_array_equal(_np(hu.pack_for_kernel(x, meta, flatten_for_kernel=True).float()), ref)


@pytest.mark.parametrize("c0", [0, 5, 37])
def test_pack_offsets_not_starting_at_zero(c0, device):
    """fmlm_pack with cu_seqlens[0] > 0: sequence b's rows land at packed rows
    cu[b] + p and every other row of [0, T_pad) is zero, also when the leading span
    [0, cu[0]) is not a whole number of the kernel's zero-fill windows."""
    from flash_mlm import _lib

    B, H, N, D = 3, 2, 40, 64
    L = [9, 0, 23]
    cu = [c0]
    for n in L:
        cu.append(cu[-1] + n)
    T = cu[-1] + 3
    T_pad = T + 200
    x = torch.randn(B, H, N, D, device=device).to(torch.bfloat16)
    dst = torch.full((H * T_pad, D), 3.0, device=device, dtype=torch.bfloat16)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=device)
    t = (_lib.PackTensor * 1)()
    t[0].src, t[0].s_sb, t[0].s_sh, t[0].s_sn = x.data_ptr(), H * N * D, N * D, D
    t[0].dst, t[0].heads = dst.data_ptr(), H
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.fmlm_pack(t, 1, 2, B, N, D, cu_t.data_ptr(), T, T_pad, stream), "fmlm_pack")
    want = np.zeros((H, T_pad, D), np.float32)
    xn = _np(x.float())
    for b in range(B):
        want[:, cu[b] : cu[b] + L[b]] = xn[b, :, : L[b]]
    np.testing.assert_array_equal(_np(dst.float()).reshape(H, T_pad, D), want)


def test_pack_unpack_full_size_round_trip(device):
    # BASELINE config 3 shape: size-independent properties (round trip, zero padding, checksums)
    g = torch.Generator().manual_seed(1003)
    L = torch.randint(256, 1025, (32,), generator=g)
    meta = build_pack_metadata(L.to(device=device, dtype=torch.int32), 1024, 64)
    x = torch.randn(32, 16, 1024, 128, device=device, dtype=torch.float16)
    flat = hu.pack_for_kernel(x, meta, flatten_for_kernel=True)
    assert flat.shape == (16 * int(L.sum()), 128)
    back = unpack_from_kernel(flat, meta, 16)
    mask = (torch.arange(1024, device=device)[None, :] < L.to(device)[:, None])[:, None, :, None]
    assert torch.equal(back, x * mask)
    # checksum of checksums: per-column sums agree up to summation order
    torch.testing.assert_close(flat.double().sum(0), (x * mask).double().sum((0, 1, 2)), atol=1e-6, rtol=1e-9)
    # prefill-style padded pack writes zero tails of T_pad - T rows per head
    T_pad = hu._compute_total_q_len_padded(meta.total_tokens, meta.host_cu_seqlens(), 128, 64)
    q_o, k_o, v_o, tp = hu.pack_and_pad_main_tensors_for_mlm_compressed(
        x, x, x, q_meta=meta, num_heads=16, is_mla=False, block_m=128, block_n=64, packing_cache=InferenceCache().packing
    )
    assert tp == T_pad
    view = q_o.view(16, T_pad, 128)
    assert torch.equal(view[:, : meta.total_tokens].reshape(-1, 128), flat)
    assert bool((view[:, meta.total_tokens :] == 0).all())
