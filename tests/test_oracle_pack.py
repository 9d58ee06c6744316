"""Pin the numpy pack/metadata oracle against the reference's known-answer tests and
closed-form invariants (CPU only)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import pack_ref

KATS = json.loads((GOLDEN / "reference_kats.json").read_text())


@pytest.mark.parametrize("case", KATS["pack_metadata"], ids=lambda c: c["line"])
def test_metadata_matches_reference_kat(case):
    m = pack_ref.pack_metadata(np.array(case["lengths"], dtype=np.int32), case["N"], case["block_n"])
    if "num_tiles" in case:
        assert m.batch_ids.size == case["num_tiles"]
    if "cu_seqlens" in case:
        assert m.B == case["B"]
        assert m.total_tokens == case["total_tokens"]
        np.testing.assert_array_equal(m.cu_seqlens, case["cu_seqlens"])
        np.testing.assert_array_equal(m.token_indices, case["token_indices"])
        np.testing.assert_array_equal(m.batch_ids, case["batch_ids_q"])
        np.testing.assert_array_equal(m.tile_starts, case["q_tile_starts_q"])
        assert m.cu_seqlens.dtype == np.int32 and m.token_indices.dtype == np.int64
        assert m.batch_ids.dtype == np.int32 and m.tile_starts.dtype == np.int32


@pytest.mark.parametrize("case", KATS["pack_metadata_errors"], ids=lambda c: c["line"])
def test_metadata_errors_match_reference(case):
    with pytest.raises(ValueError, match=case["match"]):
        pack_ref.pack_metadata(np.array(case["lengths"]), case["N"], case["block_n"])


def test_metadata_rejects_empty_batch():
    with pytest.raises(ValueError, match="cu_seqlens_q must have at least 2 elements"):
        pack_ref.pack_metadata(np.zeros(0, dtype=np.int32), 16, 4)


def test_metadata_rejects_out_of_range_lengths():
    with pytest.raises(ValueError, match=r"lengths values must be in \[0, N\]"):
        pack_ref.pack_metadata(np.array([3, 5]), 4, 2)
    with pytest.raises(ValueError, match=r"lengths values must be in \[0, N\]"):
        pack_ref.pack_metadata(np.array([-1, 2]), 4, 2)


@pytest.mark.parametrize("case", KATS["pack_for_kernel"], ids=lambda c: c["line"])
def test_pack_matches_reference_kat(case):
    m = pack_ref.pack_metadata(np.array(case["lengths"]), case["N"], case["block_n"])
    x = np.arange(np.prod(case["x_shape"]), dtype=np.float32).reshape(case["x_shape"])
    flat = pack_ref.pack(x, m)
    np.testing.assert_array_equal(flat, np.array(case["flat"], dtype=np.float32))
    H = case["x_shape"][1]
    np.testing.assert_array_equal(flat.reshape(H, m.total_tokens, -1), np.array(case["nonflat"], dtype=np.float32))


@pytest.mark.parametrize("case", KATS["unpack"], ids=lambda c: c["line"])
def test_unpack_matches_reference_kat(case):
    m = pack_ref.pack_metadata(np.array(case["lengths"]), case["N"], case["block_n"])
    x = np.arange(np.prod(case["x_shape"]), dtype=np.float32).reshape(case["x_shape"])
    restored = pack_ref.unpack(pack_ref.pack(x, m), m, H=case["x_shape"][1])
    expected = x.copy()
    expected[1, :, 2:, :] = 0  # test_host_utils.py:95-96
    np.testing.assert_array_equal(restored, expected)


@pytest.mark.parametrize("case", KATS["tile_map"], ids=lambda c: c["line"])
def test_tile_map_matches_reference_kat(case):
    starts, bids = pack_ref.tile_map(np.array(case["cu_seqlens"]), case["block_n"])
    np.testing.assert_array_equal(bids, case["batch_ids"])
    np.testing.assert_array_equal(starts, case["q_tile_starts"])
    assert starts.size == case["num_tiles"]


@pytest.mark.parametrize("case", KATS["pad_packed"], ids=lambda c: c["line"])
def test_padded_length_and_pad_match_reference_kat(case):
    T_pad = pack_ref.total_q_len_padded(case["total_q_len_unpadded"], case["cu_seqlens"], case["block_m"], case["block_n"])
    assert T_pad == case["total_q_len_padded"]
    H, T, d = case["num_heads"], case["total_q_len_unpadded"], case["d"]
    q = np.arange(H * T, dtype=np.float32).reshape(-1, d)
    np.testing.assert_array_equal(pack_ref.pad_packed(q, H, T, T_pad)[:, 0], case["q_col0"])


@pytest.mark.parametrize("case", KATS["pack_and_pad_mla"], ids=lambda c: c["line"])
def test_mla_pack_shapes_match_reference_kat(case):
    m = pack_ref.pack_metadata(np.array(case["lengths"]), case["N"], case["block_n"])
    T_pad = pack_ref.total_q_len_padded(m.total_tokens, m.cu_seqlens, case["block_m"], case["block_n"])
    assert T_pad == case["total_q_len"]
    x = np.arange(2 * 2 * 4, dtype=np.float32).reshape(2, 2, 4, 1)
    assert pack_ref.pack(x, m, T_pad).shape == tuple(case["q_out_shape"])
    assert pack_ref.pack(x[:, :1] + 10, m, T_pad).shape == tuple(case["k_out_shape"])


# ---------------------------------------------------------------------------
# closed-form invariants on random inputs
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(6))
def test_metadata_invariants_random(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 40))
    N = int(rng.integers(1, 300))
    block_n = int(rng.integers(1, 70))
    L = rng.integers(0, N + 1, size=B)
    m = pack_ref.pack_metadata(L, N, block_n)
    assert m.total_tokens == L.sum()
    assert np.all(np.diff(m.cu_seqlens) == L)
    # token b*N + t appears exactly for t < L_b, in (b, t) order (strictly increasing)
    assert np.all(np.diff(m.token_indices) > 0)
    assert np.all(m.token_indices % N < L[m.token_indices // N])
    # tiles cover each sequence exactly once in block_n steps
    assert m.batch_ids.size == int(np.sum((L + block_n - 1) // block_n))
    ends = np.minimum(m.tile_starts + block_n, m.cu_seqlens[m.batch_ids + 1])
    covered = np.concatenate([np.arange(s, e) for s, e in zip(m.tile_starts, ends)]) if ends.size else np.array([])
    np.testing.assert_array_equal(np.sort(covered), np.arange(m.total_tokens))


@pytest.mark.parametrize("seed", range(4))
def test_pack_unpack_round_trip_random(seed):
    rng = np.random.default_rng(100 + seed)
    B, H, N, D = int(rng.integers(1, 9)), int(rng.integers(1, 5)), int(rng.integers(1, 40)), int(rng.integers(1, 9))
    L = rng.integers(0, N + 1, size=B)
    m = pack_ref.pack_metadata(L, N, int(rng.integers(1, 9)))
    x = rng.standard_normal((B, H, N, D)).astype(np.float32)
    T_pad = m.total_tokens + int(rng.integers(0, 5))
    packed = pack_ref.pack(x, m, T_pad)
    assert np.all(packed.reshape(H, T_pad, D)[:, m.total_tokens :] == 0)
    body = packed.reshape(H, T_pad, D)[:, : m.total_tokens].reshape(H * m.total_tokens, D)
    restored = pack_ref.unpack(body, m, H)
    mask = np.arange(N)[None, :] < L[:, None]
    np.testing.assert_array_equal(restored, x * mask[:, None, :, None])
    # packed row (h, cu[b] + p) is x[b, h, p] (closed form, no index array)
    for b in range(B):
        for p in range(int(L[b])):
            np.testing.assert_array_equal(packed.reshape(H, T_pad, D)[:, m.cu_seqlens[b] + p], x[b, :, p])


def test_padded_length_closed_form():
    # a = max(block_m, block_n); every sequence's tile end cu[b] + ceil(L_b/a)*a
    cu = np.array([0, 5, 5, 12])
    assert pack_ref.total_q_len_padded(12, cu, 4, 2) == max(12, 0 + 8, 5 + 0, 5 + 8)
    assert pack_ref.total_q_len_padded(12, cu, 1, 1) == 12
    assert pack_ref.total_q_len_padded(0, np.array([0]), 64, 64) == 0


# ---------------------------------------------------------------------------
# KV append oracle (extension): batch c of every head = old rows of c, then new rows of c
# ---------------------------------------------------------------------------
def test_append_segments_known_answer():
    # one head, two batches: old [a0 a1 | b0], new [A0 | B0 B1] -> [a0 a1 A0 | b0 B0 B1]
    old = np.array([[1.0], [2.0], [3.0]])
    new = np.array([[10.0], [20.0], [30.0]])
    out, cu = pack_ref.append_segments(old, [0, 2, 3], new, [0, 1, 3], heads=1)
    np.testing.assert_array_equal(out[:, 0], [1, 2, 10, 3, 20, 30])
    np.testing.assert_array_equal(cu, [0, 3, 6])
    # two heads keep their own rows; trailing rows nobody owns are zero
    old2 = np.arange(8, dtype=np.float64).reshape(8, 1)           # 2 heads x 4 rows, cu [0,1,3]
    new2 = 100 + np.arange(4, dtype=np.float64).reshape(4, 1)     # 2 heads x 2 rows, cu [0,2,2]
    out2, cu2 = pack_ref.append_segments(old2, [0, 1, 3], new2, [0, 2, 2], heads=2)
    np.testing.assert_array_equal(out2[:, 0], [0, 100, 101, 1, 2, 0, 4, 102, 103, 5, 6, 0])
    np.testing.assert_array_equal(cu2, [0, 3, 5])


@pytest.mark.parametrize("seed", range(4))
def test_append_segments_identities_and_associativity(seed):
    rng = np.random.default_rng(seed)
    H, D, C = 2, 3, 4

    def cache():
        lens = rng.integers(0, 5, size=C)
        cu = np.concatenate([[0], np.cumsum(lens)])
        t = int(cu[-1]) + int(rng.integers(0, 3))  # trailing rows nobody owns
        return rng.standard_normal((H * t, D)), cu

    A, ca = cache()
    B, cb = cache()
    Cc, cc = cache()
    # appending nothing / appending to nothing keeps exactly the owned rows
    empty, cz = np.zeros((0, D)), np.zeros(C + 1, dtype=np.int64)
    out, cu = pack_ref.append_segments(A, ca, empty, cz, H)
    np.testing.assert_array_equal(cu, ca)
    t = A.shape[0] // H
    for h in range(H):
        np.testing.assert_array_equal(out[h * t : h * t + ca[-1]], A[h * t : h * t + ca[-1]])
    out, cu = pack_ref.append_segments(empty, cz, B, cb, H)
    np.testing.assert_array_equal(cu, cb)
    # (A + B) + C == A + (B + C) on the owned rows
    ab, cab = pack_ref.append_segments(A, ca, B, cb, H)
    left, cl = pack_ref.append_segments(ab, cab, Cc, cc, H)
    bc, cbc = pack_ref.append_segments(B, cb, Cc, cc, H)
    right, cr = pack_ref.append_segments(A, ca, bc, cbc, H)
    np.testing.assert_array_equal(cl, cr)
    tl, tr = left.shape[0] // H, right.shape[0] // H
    for h in range(H):
        np.testing.assert_array_equal(left[h * tl : h * tl + cl[-1]], right[h * tr : h * tr + cr[-1]])


def test_gather_pages_known_answer():
    # pool of 3 pages x 1 head x 2 rows; batch 0 = pages [2, 0] (3 keys), batch 1 = page [1] (1 key)
    pool = np.arange(6, dtype=np.float64).reshape(3, 1, 2, 1)  # page p rows (2p, 2p+1)
    cache, cu = pack_ref.gather_pages(pool, [[2, 0], [1, 9]], [3, 1])
    np.testing.assert_array_equal(cu, [0, 3, 4])
    np.testing.assert_array_equal(cache[:, 0], [4, 5, 0, 2])
    # two heads: each head keeps its own rows of the page
    pool2 = np.arange(8, dtype=np.float64).reshape(2, 2, 2, 1)  # page p, head h rows (4p+2h, 4p+2h+1)
    cache2, _ = pack_ref.gather_pages(pool2, [[1, 0]], [3])
    np.testing.assert_array_equal(cache2[:, 0], [4, 5, 0, 6, 7, 2])
