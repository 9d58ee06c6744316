"""GPU tests of paged KV contexts (InferenceCache.prefill_paged_kv_cache, an extension;
the reference's roadmap lists paged KV): attention over pages matches the attention
oracle over the gathered context (oracle/pack_ref.gather_pages), equals the same context
stored contiguously bit for bit, and the unsupported uses raise ValueError."""

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
from oracle import attention_ref as ar
from oracle import pack_ref

pytestmark = pytest.mark.gpu
PAGE = 64


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _paged(lens, *, H, D, mla, dtype, device, extra_pages=3, seed=0):
    """A shuffled page pool holding contexts of the given lengths; returns the paged cache,
    the pool / block table / lengths and a contiguous cache with the same rows."""
    g = torch.Generator().manual_seed(seed)
    h_kv = 1 if mla else H
    need = [(n + PAGE - 1) // PAGE for n in lens]
    max_pages = max(max(need), 1)
    P = sum(need) + extra_pages
    perm = torch.randperm(P, generator=g)
    bt = torch.full((len(lens), max_pages), -1, dtype=torch.int32)  # unused slots hold garbage ids
    k = 0
    for c, n in enumerate(need):
        bt[c, :n] = perm[k : k + n]
        k += n
    kp = torch.randn((h_kv, P, PAGE, D), generator=g).to(dtype).to(device)
    vp = None if mla else torch.randn((h_kv, P, PAGE, D), generator=g).to(dtype).to(device)
    cache = InferenceCache()
    cache.prefill_paged_kv_cache(0, k_pages=kp, v_pages=vp, block_table=bt.to(device),
                                 context_lens=torch.tensor(lens, dtype=torch.int32), is_mla=mla,
                                 num_heads=H, head_dim=D)
    kc, cu = pack_ref.gather_pages(_np(kp).transpose(1, 0, 2, 3), bt.numpy(), lens)
    vc = None if mla else pack_ref.gather_pages(_np(vp).transpose(1, 0, 2, 3), bt.numpy(), lens)[0]
    flat = InferenceCache()
    flat.prefill_kv_cache(0, k_cache=torch.from_numpy(kc).to(dtype).to(device),
                          v_cache=None if mla else torch.from_numpy(vc).to(dtype).to(device),
                          total_context_len=int(cu[-1]), cu_seqlens_kv=torch.from_numpy(cu).to(torch.int32).to(device),
                          context_batch_size=len(lens), is_mla=mla, num_heads=H, head_dim=D)
    return cache, flat, kc, vc, cu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_paged_context_packed(dtype, D, causal, device):
    torch.manual_seed(6100 + D + causal)
    lengths = [70, 1, 0, 133, 64]
    B, H, N = len(lengths), 3, 140
    scale = 1.0 / math.sqrt(D)
    q, k, v = (torch.randn((B, H, N, D), device=device).to(dtype) for _ in range(3))
    ctx = [129, 0, 64, 7, 300]
    cache, flat, kc, vc, cu = _paged(ctx, H=H, D=D, mla=False, dtype=dtype, device=device, seed=D)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(v), lengths, scale, causal_query_seq_attn=causal,
                                  k_cache=kc, v_cache=vc, cu_seqlens_kv=cu, total_context_len=int(cu[-1]),
                                  context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=1e-2, rtol=1e-2)
    # same rows stored contiguously: the kernels differ only in where they load a tile from
    out2 = flash_attn_mlm_compressed(q, k, v, H, meta, scale, flat, 0, block_n=64, causal_query_seq_attn=causal)
    assert torch.equal(out, out2)


def test_paged_context_mla512_index_and_precompressed(device):
    torch.manual_seed(6200)
    lengths = [150, 3, 96]
    B, H, N, D = len(lengths), 4, 150, 512
    scale = 1.0 / math.sqrt(D)
    q = (torch.randn((B, H, N, D), device=device) * 0.5).to(torch.bfloat16)
    k = (torch.randn((B, H, N, D), device=device) * 0.5).to(torch.bfloat16)
    cache, flat, kc, _, cu = _paged([65, 200], H=H, D=D, mla=True, dtype=torch.bfloat16, device=device, seed=5)
    idx = torch.tensor([1, 1, 0], dtype=torch.int32)  # 2 paged contexts for 3 sequences
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, cache, 0, is_mla=True, block_n=64, context_index=idx)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(k), lengths, scale, is_mla=True, k_cache=kc,
                                  cu_seqlens_kv=cu, total_context_len=int(cu[-1]), context_batch_size=2,
                                  context_index=idx.tolist())
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=1e-2, rtol=1e-2)
    out_flat = flash_attn_mlm_compressed(q, k, k, H, meta, scale, flat, 0, is_mla=True, block_n=64, context_index=idx)
    assert torch.equal(out, out_flat)
    qp = torch.cat([q[b, :, : lengths[b]] for b in range(B)], dim=1).reshape(-1, D).contiguous()
    kp = torch.cat([k[b, 0, : lengths[b]] for b in range(B)], dim=0).contiguous()
    pre = flash_attn_mlm_precompressed(
        qp, kp, kp, num_heads=H, total_q_len=sum(lengths), cu_seqlens_q=meta.cu_seqlens, batch_ids_q=meta.batch_ids_q,
        q_tile_starts_q=meta.q_tile_starts_q, scale=scale, inference_cache=cache, layer_id=0, is_mla=True,
        block_n=64, context_index=idx,
    )
    torch.testing.assert_close(pre, out, atol=1e-5, rtol=0)


@pytest.mark.parametrize("mla", [False, True])
def test_paged_context_longer_than_64_pages(mla, device):
    """Contexts of more than 64 pages: the kernels hold the page ids of 64 tiles at a time
    and reload them as a cursor moves on (or seeks, when few query tiles split the key
    range) past the window."""
    torch.manual_seed(6300 + mla)
    lengths = [40, 5, 1]
    B, H, N = len(lengths), 2, 40
    D = 512 if mla else 128
    dtype = torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    q = (torch.randn((B, H, N, D), device=device) * 0.5).to(dtype)
    k = (torch.randn((B, H, N, D), device=device) * 0.5).to(dtype)
    v = k if mla else (torch.randn((B, H, N, D), device=device) * 0.5).to(dtype)
    ctx = [64 * 150 + 17, 4200, 64 * 65]
    cache, flat, kc, vc, cu = _paged(ctx, H=H, D=D, mla=mla, dtype=dtype, device=device, seed=11 + mla)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=mla, block_n=64)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(v), lengths, scale, is_mla=mla, k_cache=kc,
                                  v_cache=vc, cu_seqlens_kv=cu, total_context_len=int(cu[-1]),
                                  context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=1e-2, rtol=1e-2)
    out_flat = flash_attn_mlm_compressed(q, k, v, H, meta, scale, flat, 0, is_mla=mla, block_n=64)
    assert torch.equal(out, out_flat)


def _scatter_to_pages(grad_ctx, block_table, lens, H_kv, P, D):
    """Inverse of gather_pages for gradients: contiguous context rows [H_kv*T, D] added
    into a pool [H_kv, P, PAGE, D] (rows of a page used by several batches sum)."""
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    pool = np.zeros((H_kv, P, PAGE, D))
    for c, n in enumerate(lens):
        for j in range(n):
            pool[:, int(block_table[c][j // PAGE]), j % PAGE] += grad_ctx[np.arange(H_kv) * T + cu[c] + j]
    return pool


@pytest.mark.parametrize("mla,D", [(False, 128), (True, 64), (False, 16), (False, 256)])
@pytest.mark.parametrize("shared_page", [False, True])
def test_paged_context_backward(mla, D, shared_page, device):
    """Backward over a paged context (float32 accumulation of the pool gradient): q/k/v
    gradients equal those of the same rows stored contiguously, and the pool gradient is
    the oracle's context gradient added back into the pages, pages used by two context
    batches (a shared prefix) receiving both batches' gradients."""
    g = torch.Generator().manual_seed(6400 + 2 * mla + shared_page + D)
    H, dtype = 2, torch.bfloat16  # D = 16 takes the SIMT backward kernels
    h_kv = 1 if mla else H
    lens = [130, 70, 64]
    P = 9
    bt = torch.tensor([[3, 5, 0], [3, 7, -1], [8, -1, -1]] if shared_page else [[3, 5, 0], [1, 7, -1], [8, -1, -1]],
                      dtype=torch.int32)
    kp = (torch.randn((h_kv, P, PAGE, D), generator=g) * 0.5).to(dtype).to(device).requires_grad_()
    vp = None if mla else (torch.randn((h_kv, P, PAGE, D), generator=g) * 0.5).to(dtype).to(device).requires_grad_()
    cache = InferenceCache()
    cache.prefill_paged_kv_cache(0, k_pages=kp, v_pages=vp, block_table=bt.to(device),
                                 context_lens=torch.tensor(lens, dtype=torch.int32), is_mla=mla, num_heads=H,
                                 head_dim=D)
    lengths = [50, 33, 64]
    B, N = len(lengths), 64
    q, k, v = ((torch.randn((B, H, N, D), generator=g) * 0.5).to(dtype).to(device).requires_grad_() for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, k if mla else v, H, meta, 0.125, cache, 0, is_mla=mla, block_n=64)
    dout = torch.randn(out.shape, generator=g).to(dtype).to(device)
    out.backward(dout)

    kc, cu = pack_ref.gather_pages(_np(kp).transpose(1, 0, 2, 3), bt.numpy(), lens)
    vc = None if mla else pack_ref.gather_pages(_np(vp).transpose(1, 0, 2, 3), bt.numpy(), lens)[0]
    ref = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(k if mla else v), _np(unpack_from_kernel(dout, meta, H)), lengths, 0.125, is_mla=mla,
        k_cache=kc, v_cache=vc, cu_seqlens_kv=cu, total_context_len=int(cu[-1]), context_batch_size=B)

    def close(got, want, what):
        scale = float(np.abs(want).max())
        assert scale > 0, what
        err = float(np.abs(_np(got) - want).max())
        assert err <= 2e-2 * scale, f"{what}: max err {err:.3e} (ref max {scale:.3e})"

    close(q.grad, ref[0], "dq")
    close(k.grad, ref[1], "dk")
    if not mla:
        close(v.grad, ref[2], "dv")
    close(kp.grad, _scatter_to_pages(ref[3], bt.numpy(), lens, h_kv, P, D), "d k_pages")
    if not mla:
        close(vp.grad, _scatter_to_pages(ref[4], bt.numpy(), lens, h_kv, P, D), "d v_pages")
    unused = sorted(set(range(P)) - {int(x) for row in bt.tolist() for x in row if x >= 0})
    assert torch.count_nonzero(kp.grad[:, unused]) == 0  # pages no batch uses get nothing


def test_paged_context_errors(device):
    B, H, N, D = 2, 2, 32, 64
    q, k, v = (torch.randn((B, H, N, D), device=device).to(torch.bfloat16) for _ in range(3))
    cache = _paged([10, 70], H=H, D=D, mla=False, dtype=torch.bfloat16, device=device)[0]
    with pytest.raises(ValueError, match="packed paths"):
        flash_attn_mlm(q, k, v, 0.3, inference_cache=cache, layer_id=0)
    meta = build_pack_metadata(torch.tensor([32, 10], device=device), N, block_n=32)
    with pytest.raises(ValueError, match="cannot be shared"):
        flash_attn_mlm_compressed(q, k, v, H, meta, 0.3, cache, 0, context_batch_size=1)
    with pytest.raises(ValueError, match="requires a packed entry"):
        cache.append_kv_cache(0, k_cache=torch.zeros((H * 4, D), device=device, dtype=torch.bfloat16),
                              v_cache=torch.zeros((H * 4, D), device=device, dtype=torch.bfloat16),
                              cu_seqlens_kv=torch.tensor([0, 2, 4], dtype=torch.int32))
    c = InferenceCache()
    pool = torch.zeros((H, 4, PAGE, D), device=device, dtype=torch.bfloat16)
    bt = torch.zeros((2, 2), dtype=torch.int32, device=device)
    lens = torch.tensor([3, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="bf16 or fp16"):
        c.prefill_paged_kv_cache(0, k_pages=pool.float(), v_pages=pool.float(), block_table=bt, context_lens=lens,
                                 is_mla=False, num_heads=H, head_dim=D)
    with pytest.raises(ValueError, match=r"k_pages must be \[2, pages, 64, head_dim\]"):
        c.prefill_paged_kv_cache(0, k_pages=pool[:, :, :32], v_pages=pool[:, :, :32], block_table=bt,
                                 context_lens=lens, is_mla=False, num_heads=H, head_dim=D)
    with pytest.raises(ValueError, match="context_lens must lie in"):
        c.prefill_paged_kv_cache(0, k_pages=pool, v_pages=pool, block_table=bt, context_lens=torch.tensor([3, 129]),
                                 is_mla=False, num_heads=H, head_dim=D)
    with pytest.raises(ValueError, match="takes k_pages only"):
        latent = pool[:1].contiguous()
        c.prefill_paged_kv_cache(0, k_pages=latent, v_pages=latent, block_table=bt, context_lens=lens,
                                 is_mla=True, num_heads=H, head_dim=D)
