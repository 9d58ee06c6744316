"""GPU tests of the forward's row statistics (fmlm_attn_params::lse, an extension: each
real query row's log2-sum-exp, which the forward stores when a backward will follow and
which fmlm_attn_bwd then reads instead of recomputing).  Every forward kernel is covered:
the pipelined MFMA kernel (dense and packed, unsplit and split key ranges, where
merge_kernel writes the statistic), the 512-wide MLA kernel (head-packed tiles and dense
rows), the fp32 SIMT kernel, and the paged-context instantiations (bit-equal to the same
context stored contiguously).  Reference: the float64 oracle's row_lse2
(oracle/attention_ref.py), pinned by closed forms in test_oracle_attention.py.

Tolerance, in log2 units: |gpu - ref| <= 2e-2 + 2e-3 |ref|.  The kernels round
q * scale * log2(e) to the input type before the products (a relative error of 2^-9 per
term for bf16) and sum P rounded to the input type (the pipelined kernel's row sums).

The backward with the statistics and without them (the dq kernel recomputing them) give
the same gradients: checked on one call through the C ABI with the field set and cleared.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from flash_mlm import InferenceCache, _lib, build_pack_metadata, flash_attn_mlm, flash_attn_mlm_compressed
from flash_mlm.host import host as hh
from oracle import attention_ref as ar

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _leaf(shape, dtype, device, gen, mult=0.5):
    return (torch.randn(shape, generator=gen) * mult).to(dtype).to(device).requires_grad_()


def _check(got, ref, what):
    err = np.abs(got - ref)
    bound = 2e-2 + 2e-3 * np.abs(ref)
    print(f"{what}: max |lse err| = {float(err.max()):.3e} over {ref.size} rows")
    assert np.all(np.isfinite(got)), f"{what}: non-finite statistic"
    assert float((err - bound).max()) <= 0, f"{what}: max err {float(err.max()):.3e}"


def _gpu_rows(plan, lengths, q0s):
    """The stored statistics of the real rows as [B][H, L_b] arrays."""
    p = plan.params
    lse = plan.lse.cpu().numpy().astype(np.float64).reshape(p.H, p.total_q)
    return [lse[:, q0s[b]:q0s[b] + int(L)] for b, L in enumerate(lengths)]


def _packed_cache(ctx_lens, *, H, D, mla, dtype, device, gen):
    cu = np.concatenate([[0], np.cumsum(ctx_lens)]).astype(np.int32)
    total = int(cu[-1]) + 3
    heads = 1 if mla else H
    kc = _leaf((heads * total, D), dtype, device, gen)
    vc = None if mla else _leaf((heads * total, D), dtype, device, gen)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=vc, total_context_len=total,
                           cu_seqlens_kv=torch.from_numpy(cu).to(device), context_batch_size=len(ctx_lens),
                           is_mla=mla, num_heads=H, head_dim=D)
    return cache, kc, cu, total


@pytest.mark.parametrize("dtype,D,mla,causal,ctx", [
    (torch.float16, 128, False, False, [129, 0, 64, 7, 90]),       # pipelined kernel
    (torch.bfloat16, 64, False, True, [129, 0, 64, 7, 90]),        # causal main keys
    (torch.bfloat16, 512, True, False, [129, 0, 64, 7, 90]),       # MLA, head-packed tiles
    (torch.bfloat16, 128, False, False, [3000, 700, 5000, 1500, 20]),  # split key ranges
])
def test_row_stats_packed(dtype, D, mla, causal, ctx, device):
    gen = torch.Generator().manual_seed(7700 + D + causal + 2 * mla + len(str(ctx)))
    lengths = [70, 1, 0, 133, 40] if ctx[0] < 1000 else [97, 1, 300, 0, 2]
    B, H, N = len(lengths), 2, max(lengths)
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, cu_kv, total = _packed_cache(ctx, H=H, D=D, mla=mla, dtype=dtype, device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=mla, block_n=64,
                                    causal_query_seq_attn=causal)
    plan = out.grad_fn.plan
    assert plan.lse is not None and plan.params.lse == plan.lse.data_ptr()
    if ctx[0] >= 1000:  # the schedule split these units (header word 1 counts split groups)
        (sched,) = meta.kernel_schedules.values()
        assert int(sched[:8].view(torch.int32)[1]) > 0
    ref = ar.mlm_row_lse2_packed(_np(q), _np(k), lengths, scale, is_mla=mla, causal_query_seq_attn=causal,
                                 k_cache=_np(kc), cu_seqlens_kv=cu_kv, total_context_len=total, context_batch_size=B)
    q0s = np.concatenate([[0], np.cumsum(lengths)])
    got = _gpu_rows(plan, lengths, q0s)
    for b, L in enumerate(lengths):
        if L:
            _check(got[b], ref[b, :, :L], f"b={b}")


@pytest.mark.parametrize("dtype,D,mla", [
    (torch.bfloat16, 64, False),   # pipelined kernel, dense rows
    (torch.bfloat16, 512, True),   # MLA kernel, dense rows
    (torch.float32, 64, False),    # SIMT kernel
])
def test_row_stats_dense(dtype, D, mla, device):
    gen = torch.Generator().manual_seed(7800 + D + mla)
    B, H, N, C = 3, 2, 96, 70
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    kc = _leaf((B * (1 if mla else H) * C, D), dtype, device, gen)
    vc = None if mla else _leaf(kc.shape, dtype, device, gen)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=vc, context_batch_size=B, is_mla=mla, num_heads=H, head_dim=D)
    out = flash_attn_mlm(q, k, v, scale, cache, 0, is_mla=mla)
    plan = out.grad_fn.plan
    ref = ar.mlm_row_lse2_dense(_np(q), _np(k), scale, is_mla=mla, k_cache=_np(kc), context_len=C,
                                context_batch_size=B)
    got = _gpu_rows(plan, [N] * B, [b * N for b in range(B)])
    for b in range(B):
        _check(got[b], ref[b], f"b={b}")


def test_forward_without_backward_stores_no_statistics(device):
    """Inference calls leave the field NULL (no buffer, no stores)."""
    gen = torch.Generator().manual_seed(7900)
    B, H, N, D = 2, 2, 64, 64
    q, k, v = (torch.randn((B, H, N, D), generator=gen).to(torch.bfloat16).to(device) for _ in range(3))
    with torch.no_grad():
        out, plan = hh._dense_impl(q, k, v, 0.125, None, None, False, 1, False)
    assert plan.lse is None and not plan.params.lse


@pytest.mark.parametrize("D", [64, 128])
def test_backward_with_and_without_statistics_agree(D, device):
    """fmlm_attn_bwd on one forward twice: reading the stored statistics (the dq kernel
    without a running max) and with the field cleared (the dq kernel recomputing them)."""
    gen = torch.Generator().manual_seed(7950 + D)
    lengths = [70, 1, 133, 40]
    B, H, N, dtype = len(lengths), 2, 140, torch.float16
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, cu_kv, total = _packed_cache([129, 0, 64, 7], H=H, D=D, mla=False, dtype=dtype, device=device,
                                            gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 1.0 / math.sqrt(D), cache, 0, block_n=64)
    plan = out.grad_fn.plan
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    grads = []
    for with_lse in (True, False):
        p = _lib.AttnParams.from_buffer_copy(plan.params)
        if not with_lse:
            p.lse = None
        g, keep = hh._backward_args(plan, out.detach(), dout, want_ctx=True)
        rc = plan.lib.fmlm_attn_bwd(ctypes.byref(p), ctypes.byref(g), plan.stream)
        _lib.check(rc, "fmlm_attn_bwd")
        torch.cuda.synchronize()
        grads.append([_np(t) for t in keep[:4]])
    for a, b, name in zip(grads[0], grads[1], ("dq", "dk", "dv", "dk_cache")):
        scale = float(np.abs(b).max())
        assert scale > 0
        err = float(np.abs(a - b).max())
        print(f"{name}: max |with - without| / max = {err / scale:.2e}")
        assert err <= 1e-2 * scale, name


@pytest.mark.parametrize("mla,D", [(True, 512), (False, 128)])
def test_row_stats_paged_context_equal_contiguous(mla, D, device):
    """The paged instantiations (MLA: its own LSE instantiation) store the same statistics,
    bit for bit, as the same context stored contiguously, and match the oracle."""
    from oracle import pack_ref
    PAGE = 64
    lens = [65, 200, 3]
    g = torch.Generator().manual_seed(8100 + D)
    H, dtype = 2, torch.bfloat16
    h_kv = 1 if mla else H
    need = [(n + PAGE - 1) // PAGE for n in lens]
    P = sum(need) + 2
    perm = torch.randperm(P, generator=g)
    bt = torch.full((len(lens), max(need)), -1, dtype=torch.int32)
    i = 0
    for c, n in enumerate(need):
        bt[c, :n] = perm[i:i + n]
        i += n
    kp = (torch.randn((h_kv, P, PAGE, D), generator=g) * 0.5).to(dtype).to(device)
    vp = None if mla else (torch.randn((h_kv, P, PAGE, D), generator=g) * 0.5).to(dtype).to(device)
    paged = InferenceCache()
    paged.prefill_paged_kv_cache(0, k_pages=kp, v_pages=vp, block_table=bt.to(device),
                                 context_lens=torch.tensor(lens, dtype=torch.int32), is_mla=mla, num_heads=H, head_dim=D)
    kc, cu = pack_ref.gather_pages(_np(kp).transpose(1, 0, 2, 3), bt.numpy(), lens)
    vc = None if mla else pack_ref.gather_pages(_np(vp).transpose(1, 0, 2, 3), bt.numpy(), lens)[0]
    flat = InferenceCache()
    flat.prefill_kv_cache(0, k_cache=torch.from_numpy(kc).to(dtype).to(device),
                          v_cache=None if mla else torch.from_numpy(vc).to(dtype).to(device),
                          total_context_len=int(cu[-1]), cu_seqlens_kv=torch.from_numpy(cu).to(torch.int32).to(device),
                          context_batch_size=len(lens), is_mla=mla, num_heads=H, head_dim=D)
    lengths = [40, 130, 7]
    B, N = len(lengths), 130
    q, k, v = (_leaf((B, H, N, D), dtype, device, g) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    stats = []
    for cache in (paged, flat):
        out = flash_attn_mlm_compressed(q, k, k if mla else v, H, meta, 1.0 / math.sqrt(D), cache, 0, is_mla=mla,
                                        block_n=64)
        stats.append(out.grad_fn.plan.lse.clone())
    assert torch.equal(stats[0], stats[1])
    ref = ar.mlm_row_lse2_packed(_np(q), _np(k), lengths, 1.0 / math.sqrt(D), is_mla=mla, k_cache=kc,
                                 cu_seqlens_kv=cu, total_context_len=int(cu[-1]), context_batch_size=B)
    plan = out.grad_fn.plan
    got = _gpu_rows(plan, lengths, np.concatenate([[0], np.cumsum(lengths)]))
    for b, L in enumerate(lengths):
        _check(got[b], ref[b, :, :L], f"b={b}")
