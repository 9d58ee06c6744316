"""GPU tests of the KV append (InferenceCache.append_kv_cache, an extension with no
reference counterpart): the merged cache is bit-exact against the numpy oracle
(oracle/pack_ref.append_segments), attention over an appended context matches the
attention oracle over the merged rows, and the error paths raise ValueError."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flash_mlm import InferenceCache, build_pack_metadata, flash_attn_mlm_compressed, unpack_from_kernel
from oracle import attention_ref as ar
from oracle import pack_ref

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _cu(lengths):
    cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths), 0)
    return cu


def _entry(cache, *, H, D, mla, dtype, device, lengths, extra_rows=0, layer=0):
    cu = _cu(lengths)
    t = int(cu[-1]) + extra_rows
    h_kv = 1 if mla else H
    k = torch.randn((h_kv * t, D), device=device).to(dtype)
    v = None if mla else torch.randn((h_kv * t, D), device=device).to(dtype)
    cache.prefill_kv_cache(layer, k_cache=k, v_cache=v, total_context_len=t, cu_seqlens_kv=cu.to(device),
                           context_batch_size=len(lengths), is_mla=mla, num_heads=H, head_dim=D)
    return k, v, cu


def _owned(x, cu, rows, heads):
    """Rows a merged cache defines: [0, cu[-1]) of every head."""
    n = int(cu[-1])
    return np.concatenate([x[h * rows : h * rows + n] for h in range(heads)])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mla", [False, True])
def test_append_matches_oracle_bit_exact(dtype, mla, device):
    torch.manual_seed(5100 + mla)
    H, D = 3, 128 if not mla else 512
    cache = InferenceCache()
    k0, v0, cu0 = _entry(cache, H=H, D=D, mla=mla, dtype=dtype, device=device, lengths=[7, 0, 33, 5], extra_rows=3)
    h_kv = 1 if mla else H
    new_len = [2, 9, 0, 64]
    cu1 = _cu(new_len)
    t1 = int(cu1[-1])
    k1 = torch.randn((h_kv * t1, D), device=device).to(dtype)
    v1 = None if mla else torch.randn((h_kv * t1, D), device=device).to(dtype)
    cache.append_kv_cache(0, k_cache=k1, v_cache=v1, cu_seqlens_kv=cu1.to(device))
    e = cache._layer_kv["0"]
    ref_k, ref_cu = pack_ref.append_segments(_np(k0.float()), _np(cu0), _np(k1.float()), _np(cu1), h_kv)
    assert e.total_context_len == k0.shape[0] // h_kv + t1
    np.testing.assert_array_equal(_np(e.cu_seqlens_kv), ref_cu)
    rows = e.total_context_len
    np.testing.assert_array_equal(_owned(_np(e.k_cache.float()), ref_cu, rows, h_kv), _owned(ref_k, ref_cu, rows, h_kv))
    # the whole buffer, rows past the last batch (zero) included
    np.testing.assert_array_equal(_np(e.k_cache.float()), ref_k)
    if not mla:
        ref_v, _ = pack_ref.append_segments(_np(v0.float()), _np(cu0), _np(v1.float()), _np(cu1), h_kv)
        np.testing.assert_array_equal(_owned(_np(e.v_cache.float()), ref_cu, rows, h_kv), _owned(ref_v, ref_cu, rows, h_kv))
        np.testing.assert_array_equal(_np(e.v_cache.float()), ref_v)


@pytest.mark.parametrize("mla", [False, True])
def test_append_then_shared_context(mla, device):
    """An appended multi-batch entry read as a shared context (context_batch_size=1): every
    sequence attends to all rows of every head, cu_seqlens_kv = [0, total]
    (host_utils.py:232-237), so the rows past the last batch must be the zeros a prefilled
    packed entry holds there.  Checked against the oracle over the oracle's merge."""
    torch.manual_seed(5300 + mla)
    dtype, H, N = torch.bfloat16, 2, 80
    D = 512 if mla else 64
    lengths = [80, 33, 5]
    B = len(lengths)
    h_kv = 1 if mla else H
    cache = InferenceCache()
    # 4 padding rows per head past the last batch, filled with non-zero values: the append
    # must not carry them over as they are
    k0, v0, cu0 = _entry(cache, H=H, D=D, mla=mla, dtype=dtype, device=device, lengths=[20, 0, 45], extra_rows=4)
    new_len = [3, 17, 0]
    cu1 = _cu(new_len)
    t1 = int(cu1[-1])
    k1 = torch.randn((h_kv * t1, D), device=device).to(dtype)
    v1 = None if mla else torch.randn((h_kv * t1, D), device=device).to(dtype)
    # make the old padding rows zero in the oracle's input: the merged entry's tail is zero
    rows0 = k0.shape[0] // h_kv
    mk, mcu = pack_ref.append_segments(_np(k0.float()), _np(cu0), _np(k1.float()), _np(cu1), h_kv)
    mv = None if mla else pack_ref.append_segments(_np(v0.float()), _np(cu0), _np(v1.float()), _np(cu1), h_kv)[0]
    cache.append_kv_cache(0, k_cache=k1, v_cache=v1, cu_seqlens_kv=cu1.to(device))
    Tc = rows0 + t1
    assert cache._layer_kv["0"].total_context_len == Tc
    q, kq, vq = (torch.randn((B, H, N, D), device=device).to(dtype) * (0.5 if mla else 1.0) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, kq, vq, H, meta, scale, cache, 0, is_mla=mla, block_n=64,
                                    context_batch_size=1)
    ref = ar.mlm_attention_packed(_np(q.float()), _np(kq.float()), _np(vq.float()), lengths, scale, is_mla=mla,
                                  k_cache=mk, v_cache=mv, cu_seqlens_kv=[0, Tc], total_context_len=Tc,
                                  context_batch_size=1)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H).float()), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("mla", [False, True])
def test_attention_over_appended_context(mla, device):
    """Two appends (the second with a CPU offset tensor), then attention: the same as the
    oracle over the merged rows, and the same as a cache prefilled with those rows."""
    torch.manual_seed(5200 + mla)
    dtype, H, N = torch.bfloat16, 2, 96
    D = 512 if mla else 64
    lengths = [96, 40, 7]
    B = len(lengths)
    h_kv = 1 if mla else H
    cache = InferenceCache()
    k0, v0, cu0 = _entry(cache, H=H, D=D, mla=mla, dtype=dtype, device=device, lengths=[30, 0, 70])
    ks, vs, cus = [k0], [v0], [cu0]
    for new_len, on_gpu in (([5, 64, 0], True), ([1, 2, 100], False)):
        cu = _cu(new_len)
        t = int(cu[-1])
        k = torch.randn((h_kv * t, D), device=device).to(dtype)
        v = None if mla else torch.randn((h_kv * t, D), device=device).to(dtype)
        cache.append_kv_cache(0, k_cache=k, v_cache=v, cu_seqlens_kv=cu.to(device) if on_gpu else cu)
        ks.append(k)
        vs.append(v)
        cus.append(cu)
    # oracle merge of the three pieces
    mk, mcu = _np(ks[0].float()), _np(cus[0])
    mv = None if mla else _np(vs[0].float())
    for k, v, cu in zip(ks[1:], vs[1:], cus[1:]):
        nk, ncu = pack_ref.append_segments(mk, mcu, _np(k.float()), _np(cu), h_kv)
        if not mla:
            mv, _ = pack_ref.append_segments(mv, mcu, _np(v.float()), _np(cu), h_kv)
        mk, mcu = nk, ncu
    Tc = mk.shape[0] // h_kv
    q, kq, vq = (torch.randn((B, H, N, D), device=device).to(dtype) * (0.5 if mla else 1.0) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, kq, vq, H, meta, scale, cache, 0, is_mla=mla, block_n=64)
    ref = ar.mlm_attention_packed(_np(q.float()), _np(kq.float()), _np(vq.float()), lengths, scale, is_mla=mla,
                                  k_cache=mk, v_cache=mv, cu_seqlens_kv=mcu, total_context_len=Tc,
                                  context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H).float()), ref, atol=1e-2, rtol=1e-2)
    # a cache prefilled with the merged rows gives the same kernel result
    pre = InferenceCache()
    e = cache._layer_kv["0"]
    pre.prefill_kv_cache(0, k_cache=e.k_cache.clone(), v_cache=None if mla else e.v_cache.clone(),
                         total_context_len=e.total_context_len, cu_seqlens_kv=e.cu_seqlens_kv.clone(),
                         context_batch_size=B, is_mla=mla, num_heads=H, head_dim=D)
    out2 = flash_attn_mlm_compressed(q, kq, vq, H, meta, scale, pre, 0, is_mla=mla, block_n=64)
    assert torch.equal(out, out2)


def test_append_errors(device):
    cache = InferenceCache()
    H, D = 2, 64
    k = torch.zeros((H * 4, D), device=device, dtype=torch.bfloat16)
    cu = torch.tensor([0, 2, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="no cached KV entry"):
        cache.append_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=cu)
    # a dense entry (no cu_seqlens_kv) has no per-batch row ranges to append to
    cache.prefill_kv_cache(0, k_cache=k, v_cache=k, total_context_len=4, context_batch_size=2, is_mla=False,
                           num_heads=H, head_dim=D)
    with pytest.raises(ValueError, match="requires a packed entry"):
        cache.append_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=cu)
    cache.prefill_kv_cache(0, k_cache=k, v_cache=k, total_context_len=4, cu_seqlens_kv=cu.to(device),
                           context_batch_size=2, is_mla=False, num_heads=H, head_dim=D)
    with pytest.raises(ValueError, match="second dim must match head_dim"):
        cache.append_kv_cache(0, k_cache=k[:, :32], v_cache=k[:, :32], cu_seqlens_kv=cu)
    with pytest.raises(ValueError, match="dtype/device must match"):
        cache.append_kv_cache(0, k_cache=k.half(), v_cache=k.half(), cu_seqlens_kv=cu)
    with pytest.raises(ValueError, match="v_cache shaped like k_cache"):
        cache.append_kv_cache(0, k_cache=k, cu_seqlens_kv=cu)
    with pytest.raises(ValueError, match="one entry per cached context batch"):
        cache.append_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=torch.tensor([0, 4], dtype=torch.int32))
    with pytest.raises(ValueError, match="end within the new rows"):
        cache.append_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=torch.tensor([0, 2, 5], dtype=torch.int32))
    with pytest.raises(ValueError, match="non-decreasing"):
        cache.append_kv_cache(0, k_cache=k, v_cache=k, cu_seqlens_kv=torch.tensor([0, 3, 2], dtype=torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_copy_segments_and_zero_segments(dtype, device):
    """fmlm_copy_segments (the ABI's general segment copy) bit-exact against numpy, with a
    null source writing zero rows; offsets past the buffers are clamped."""
    from flash_mlm.host.host_utils import copy_segments

    torch.manual_seed(5400)
    H, D, src_rows, dst_rows = 3, 64, 50, 70
    src = torch.randn((H * src_rows, D), device=device).to(dtype)
    dst = torch.randn((H * dst_rows, D), device=device).to(dtype)
    ref = _np(dst.float()).copy()
    src_cu = [0, 10, 10, 45]
    dst_start = [5, 60, 30]
    copy_segments(src, src_rows, torch.tensor(src_cu, dtype=torch.int32, device=device), dst, dst_rows,
                  torch.tensor(dst_start, dtype=torch.int32, device=device), 3, H, D)
    s, r = _np(src.float()), ref
    for h in range(H):
        for c in range(3):
            n = src_cu[c + 1] - src_cu[c]
            n = min(n, dst_rows - dst_start[c])
            r[h * dst_rows + dst_start[c] : h * dst_rows + dst_start[c] + n] = \
                s[h * src_rows + src_cu[c] : h * src_rows + src_cu[c] + n]
    np.testing.assert_array_equal(_np(dst.float()), r)
    # zero rows [20, 33) of every head
    copy_segments(None, dst_rows, torch.tensor([0, 13], dtype=torch.int32, device=device), dst, dst_rows,
                  torch.tensor([20], dtype=torch.int32, device=device), 1, H, D)
    for h in range(H):
        r[h * dst_rows + 20 : h * dst_rows + 33] = 0
    np.testing.assert_array_equal(_np(dst.float()), r)


@pytest.mark.parametrize("case", ["no_new_rows", "no_old_rows", "empty_batches"])
def test_append_edge_cases(case, device):
    """The one-launch merge at its edges: nothing new, an entry of no rows, empty batches;
    bit-exact against the oracle's merge, zero tail included."""
    torch.manual_seed(5500)
    H, D, dtype = 2, 128, torch.float16
    lengths = {"no_new_rows": [4, 9], "no_old_rows": [0, 0], "empty_batches": [0, 7]}[case]
    new_len = {"no_new_rows": [0, 0], "no_old_rows": [3, 5], "empty_batches": [0, 2]}[case]
    cache = InferenceCache()
    k0, v0, cu0 = _entry(cache, H=H, D=D, mla=False, dtype=dtype, device=device, lengths=lengths, extra_rows=2)
    cu1 = _cu(new_len)
    t1 = int(cu1[-1])
    k1 = torch.randn((H * t1, D), device=device).to(dtype)
    v1 = torch.randn((H * t1, D), device=device).to(dtype)
    cache.append_kv_cache(0, k_cache=k1, v_cache=v1, cu_seqlens_kv=cu1.to(device))
    e = cache._layer_kv["0"]
    ref_k, ref_cu = pack_ref.append_segments(_np(k0.float()), _np(cu0), _np(k1.float()), _np(cu1), H)
    ref_v, _ = pack_ref.append_segments(_np(v0.float()), _np(cu0), _np(v1.float()), _np(cu1), H)
    np.testing.assert_array_equal(_np(e.cu_seqlens_kv), ref_cu)
    np.testing.assert_array_equal(_np(e.k_cache.float()), ref_k)
    np.testing.assert_array_equal(_np(e.v_cache.float()), ref_v)
