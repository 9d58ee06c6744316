"""Seeded random parity sweep of the forward against the fp64 oracle: random batch shapes,
lengths (empty sequences included), cached contexts (per batch and shared), head dims, the
512-wide latent, causal_query_seq_attn, dtypes and score ranges.  Half of the cases add a
per-key score offset through one dimension (q[..., 0] = 4, k[..., 0] drawn per key), so that
the row maximum rises and falls inside and across key tiles: the lazy rescale, the latent
kernel's per-half check and its rescale of the first half's P, and (in the long cases) the
split-KV partial records and their merge."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flash_mlm import InferenceCache, build_pack_metadata, flash_attn_mlm, flash_attn_mlm_compressed, unpack_from_kernel
from oracle import attention_ref as ar

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _spike(q, k, rng, n_keys, device):
    """q[..., 0] = 4 and a per-key k[..., 0] in [-40, 40]: score offsets of up to
    160 * scale * log2(e) (log2 units) that change from key to key."""
    q[..., 0] = 4.0
    k0 = torch.from_numpy(rng.uniform(-40.0, 40.0, size=n_keys)).float().to(device)
    return k0


def _case(seed):
    """Shape and value ranges of one case: inputs of std up to 2 (scores of std 4), where
    bf16 needs the kernels' fp32 score scaling (a Q pre-scaled in bf16 would tilt P past
    the budget; fp16 kernels pre-scale Q, and its 11-bit mantissa keeps that inside)."""
    rng = np.random.default_rng(9000 + seed)
    D = int(rng.choice([32, 64, 128, 256, 512]))
    is_mla = D == 512 or bool(rng.random() < 0.25)
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    std = float(rng.choice([0.5, 1.0, 2.0]))
    spike = bool(rng.random() < 0.5)
    return rng, D, is_mla, dtype, std, spike


@pytest.mark.parametrize("seed", list(range(20)))
def test_random_packed(seed, device):
    rng, D, is_mla, dtype, std, spike = _case(seed)
    torch.manual_seed(9000 + seed)
    B = int(rng.integers(1, 6))
    H = int(rng.integers(1, 5))
    lengths = [int(x) for x in rng.integers(0, 200, size=B)]
    if max(lengths) == 0:
        lengths[0] = 1
    N = max(lengths)
    causal = bool(rng.random() < 0.3)
    ctx_mode = rng.choice(["none", "batch", "shared"])
    h_kv = 1 if is_mla else H
    q = (torch.randn((B, H, N, D), device=device) * (std if not spike else 0.5)).to(dtype)
    k = (torch.randn((B, H, N, D), device=device) * std).to(dtype)
    v = (torch.randn((B, H, N, D), device=device) * std).to(dtype)
    cache, kc, vc, cu_kv, Tc, cbs = None, None, None, None, 0, B
    if ctx_mode != "none":
        ctx = [int(x) for x in rng.integers(0, 200, size=B)]
        ctx[0] = max(ctx[0], 1)
        cu_kv = np.zeros(B + 1, dtype=np.int64)
        cu_kv[1:] = np.cumsum(ctx)
        Tc = int(cu_kv[-1])
        kc = (torch.randn((h_kv * Tc, D), device=device) * std).to(dtype)
        vc = (torch.randn((h_kv * Tc, D), device=device) * std).to(dtype)
        cache = InferenceCache()
        cache.prefill_kv_cache(layer_id=0, k_cache=kc, v_cache=vc, total_context_len=Tc,
                               cu_seqlens_kv=torch.tensor(cu_kv, dtype=torch.int32, device=device),
                               context_batch_size=B, is_mla=is_mla, num_heads=H, head_dim=D)
        if ctx_mode == "shared":
            cbs = 1
    if spike:
        # the latent (MLA) is head 0 of k; every head's keys carry the offsets otherwise
        k0 = _spike(q, k, rng, B * N, device).reshape(B, N).to(dtype)
        if is_mla:
            k[:, 0, :, 0] = k0
        else:
            k[..., 0] = k0[:, None, :]
        if kc is not None:
            kc[:, 0] = _spike(q, k, rng, h_kv * Tc, device).to(dtype)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = (-1.0 if rng.random() < 0.25 else 1.0) / math.sqrt(D)  # a negative scale flips Q's sign
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0 if cache is not None else None, is_mla=is_mla,
                                    block_n=64, causal_query_seq_attn=causal,
                                    context_batch_size=1 if ctx_mode == "shared" else None)
    assert torch.isfinite(out).all()
    ref = ar.mlm_attention_packed(
        _np(q), _np(k), _np(v), lengths, scale, is_mla=is_mla, causal_query_seq_attn=causal,
        k_cache=None if kc is None else _np(kc), v_cache=None if vc is None or is_mla else _np(vc),
        cu_seqlens_kv=None if cu_kv is None else ([0, Tc] if ctx_mode == "shared" else [int(x) for x in cu_kv]),
        total_context_len=Tc, context_batch_size=cbs)
    got = _np(unpack_from_kernel(out, meta, H))
    # V's scale sets the output's; with offsets, the latent's dim 0 reaches 40
    np.testing.assert_allclose(got, ref, atol=1e-2 * max(1.0, std), rtol=1e-2)


@pytest.mark.parametrize("seed", list(range(8)))
def test_random_dense(seed, device):
    rng, D, is_mla, dtype, std, spike = _case(100 + seed)
    if D == 512:
        D = 128
    torch.manual_seed(9100 + seed)
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    N = int(rng.integers(1, 160))
    q = (torch.randn((B, H, N, D), device=device) * (std if not spike else 0.5)).to(dtype)
    k = (torch.randn((B, H, N, D), device=device) * std).to(dtype)
    v = (torch.randn((B, H, N, D), device=device) * std).to(dtype)
    if spike:
        k0 = _spike(q, k, rng, B * N, device).reshape(B, 1, N).to(dtype)
        k[..., 0] = k0
    cache, kc, vc, C, cbs = None, None, None, 0, 1
    if rng.random() < 0.6:
        cbs = int(rng.choice([1, B]))
        C = int(rng.integers(1, 150))
        rows = cbs * C * (1 if is_mla else H)
        kc = (torch.randn((rows, D), device=device) * std).to(dtype)
        vc = (torch.randn((rows, D), device=device) * std).to(dtype)
        cache = InferenceCache()
        cache.prefill_kv_cache(0, k_cache=kc, v_cache=None if is_mla else vc, context_batch_size=cbs, is_mla=is_mla,
                               num_heads=H, head_dim=D, total_context_len=cbs * C)
    scale = (-1.0 if rng.random() < 0.25 else 1.0) / math.sqrt(D)
    out = flash_attn_mlm(q, k, v, scale, inference_cache=cache, layer_id=0 if cache is not None else None, is_mla=is_mla)
    assert torch.isfinite(out).all()
    ref = ar.mlm_attention_dense(_np(q), _np(k), _np(v), scale, is_mla=is_mla,
                                 k_cache=None if kc is None else _np(kc), v_cache=None if vc is None else _np(vc),
                                 context_len=C, context_batch_size=cbs)
    np.testing.assert_allclose(_np(out), ref, atol=1e-2 * max(1.0, std), rtol=1e-2)


@pytest.mark.parametrize("seed", list(range(4)))
def test_random_long_context_split(seed, device):
    """Few short query sequences over contexts of 2-6k keys: the schedule splits the key
    ranges, and the merge combines partial records whose maxima differ (offsets on)."""
    rng = np.random.default_rng(9200 + seed)
    torch.manual_seed(9200 + seed)
    D = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if seed % 2 else torch.float16
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    lengths = [int(x) for x in rng.integers(1, 48, size=B)]
    N = max(lengths)
    ctx = [int(x) for x in rng.integers(2000, 6000, size=B)]
    cu_kv = np.zeros(B + 1, dtype=np.int64)
    cu_kv[1:] = np.cumsum(ctx)
    Tc = int(cu_kv[-1])
    q = (torch.randn((B, H, N, D), device=device) * 0.5).to(dtype)
    k, v = ((torch.randn((B, H, N, D), device=device)).to(dtype) for _ in range(2))
    kc, vc = ((torch.randn((H * Tc, D), device=device)).to(dtype) for _ in range(2))
    kc[:, 0] = _spike(q, k, rng, H * Tc, device).to(dtype)
    k[..., 0] = 0.0
    cache = InferenceCache()
    cache.prefill_kv_cache(layer_id=0, k_cache=kc, v_cache=vc, total_context_len=Tc,
                           cu_seqlens_kv=torch.tensor(cu_kv, dtype=torch.int32, device=device), context_batch_size=B,
                           is_mla=False, num_heads=H, head_dim=D)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(v), lengths, scale, k_cache=_np(kc), v_cache=_np(vc),
                                  cu_seqlens_kv=[int(x) for x in cu_kv], total_context_len=Tc, context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("seed", list(range(4)))
def test_random_latent512_bf16_large_scores(seed, device):
    """The 512-wide latent kernel scales scores in fp32 (Q as stored, the scale in the
    FMA that subtracts the running max), so bf16 inputs of std 2 (scores of std 4), where
    a Q pre-scaled in bf16 would exceed the budget, stay inside 1e-2."""
    rng = np.random.default_rng(9300 + seed)
    torch.manual_seed(9300 + seed)
    B, H, D = int(rng.integers(1, 4)), int(rng.integers(1, 5)), 512
    lengths = [int(x) for x in rng.integers(1, 160, size=B)]
    N = max(lengths)
    ctx = [int(x) for x in rng.integers(0, 200, size=B)]
    cu_kv = np.zeros(B + 1, dtype=np.int64)
    cu_kv[1:] = np.cumsum(ctx)
    Tc = int(cu_kv[-1])
    q, k = ((torch.randn((B, H, N, D), device=device) * 2.0).to(torch.bfloat16) for _ in range(2))
    kc = (torch.randn((max(Tc, 1), D), device=device) * 2.0).to(torch.bfloat16)[:Tc]
    cache = None
    if Tc:
        cache = InferenceCache()
        cache.prefill_kv_cache(layer_id=0, k_cache=kc, v_cache=kc, total_context_len=Tc,
                               cu_seqlens_kv=torch.tensor(cu_kv, dtype=torch.int32, device=device),
                               context_batch_size=B, is_mla=True, num_heads=H, head_dim=D)
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = (-1.0 if seed == 3 else 1.0) / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, cache, 0 if cache is not None else None, is_mla=True,
                                    block_n=64)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(k), lengths, scale, is_mla=True,
                                  k_cache=_np(kc) if Tc else None, cu_seqlens_kv=[int(x) for x in cu_kv] if Tc else None,
                                  total_context_len=Tc, context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("seed", list(range(6)))
def test_random_paged_context(seed, device):
    """Contexts in a shuffled page pool (InferenceCache.prefill_paged_kv_cache): random
    lengths, head dims (the 512 latent included), dtypes, inputs up to std 2 and per-key
    score offsets in the pages, against the oracle over the gathered rows."""
    from oracle import pack_ref

    page = 64
    rng = np.random.default_rng(9400 + seed)
    gen = torch.Generator().manual_seed(9400 + seed)
    D = int(rng.choice([64, 128, 512]))
    mla = D == 512 or bool(rng.random() < 0.3)
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float16
    std = float(rng.choice([0.5, 1.0, 2.0]))
    spike = bool(rng.random() < 0.5)
    causal = bool(rng.random() < 0.3)
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    lengths = [int(x) for x in rng.integers(1, 150, size=B)]
    N = max(lengths)
    ctx = [int(x) for x in rng.integers(0, 300, size=B)]
    ctx[0] = max(ctx[0], 1)
    h_kv = 1 if mla else H
    need = [(n + page - 1) // page for n in ctx]
    P = sum(need) + 2
    perm = torch.randperm(P, generator=gen)
    bt = torch.full((B, max(max(need), 1)), -1, dtype=torch.int32)
    k_ = 0
    for b_, n in enumerate(need):
        bt[b_, :n] = perm[k_ : k_ + n]
        k_ += n
    kp = torch.randn((h_kv, P, page, D), generator=gen) * std
    vp = None if mla else (torch.randn((h_kv, P, page, D), generator=gen) * std).to(dtype).to(device)
    q = torch.randn((B, H, N, D), generator=gen) * (0.5 if spike else std)
    k = torch.randn((B, H, N, D), generator=gen) * std
    v = (torch.randn((B, H, N, D), generator=gen) * std).to(dtype).to(device)
    if spike:
        q[..., 0] = 4.0
        kp[..., 0] = torch.from_numpy(rng.uniform(-30.0, 30.0, size=(h_kv, P, page))).float()
        k[..., 0] = torch.from_numpy(rng.uniform(-30.0, 30.0, size=(B, 1, N))).float()
    kp = kp.to(dtype).to(device)
    q, k = q.to(dtype).to(device), k.to(dtype).to(device)
    cache = InferenceCache()
    cache.prefill_paged_kv_cache(0, k_pages=kp, v_pages=vp, block_table=bt.to(device),
                                 context_lens=torch.tensor(ctx, dtype=torch.int32), is_mla=mla, num_heads=H, head_dim=D)
    kc, cu = pack_ref.gather_pages(_np(kp).transpose(1, 0, 2, 3), bt.numpy(), ctx)
    vc = None if mla else pack_ref.gather_pages(_np(vp).transpose(1, 0, 2, 3), bt.numpy(), ctx)[0]
    meta = build_pack_metadata(torch.tensor(lengths, device=device), N, 64)
    scale = 1.0 / math.sqrt(D)
    out = flash_attn_mlm_compressed(q, k, k if mla else v, H, meta, scale, cache, 0, is_mla=mla, block_n=64,
                                    causal_query_seq_attn=causal)
    ref = ar.mlm_attention_packed(_np(q), _np(k), _np(k if mla else v), lengths, scale, is_mla=mla,
                                  causal_query_seq_attn=causal, k_cache=kc, v_cache=vc,
                                  cu_seqlens_kv=[int(x) for x in cu], total_context_len=int(cu[-1]),
                                  context_batch_size=B)
    np.testing.assert_allclose(_np(unpack_from_kernel(out, meta, H)), ref, atol=1e-2 * max(1.0, std), rtol=1e-2)
