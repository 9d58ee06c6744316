"""GPU test of fmlm_attn_fwd_noalloc, the allocation-free variant of fmlm_attn_fwd (no
reference counterpart): called through the C ABI on the parameter block of a prepared
fmlm_attn_fwd call, it gives that call's output -- bit for bit when neither splits key
ranges, within the attention tolerance (atol = rtol = 1e-2) when the smaller scratch
array leaves fewer split records -- on consecutive calls, each smaller than the last, so
that every call runs over what the previous one left in the library's scratch array."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from flash_mlm import InferenceCache, build_pack_metadata
from flash_mlm import _lib
from flash_mlm.host import host as hh

pytestmark = pytest.mark.gpu


def _case(device, *, B, H, N, D, dtype, lq, lc, mla=False, causal=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lq[0], lq[1] + 1, (B,), generator=g)
    ctx = torch.randint(lc[0], lc[1] + 1, (B,), generator=g)
    q = (torch.randn((B, H, N, D), generator=g) * 0.5).to(dtype).to(device)
    k = (torch.randn((B, H, N, D), generator=g) * 0.5).to(dtype).to(device)
    v = k if mla else (torch.randn((B, H, N, D), generator=g) * 0.5).to(dtype).to(device)
    h_kv = 1 if mla else H
    cu_kv = torch.zeros(B + 1, dtype=torch.int32)
    cu_kv[1:] = torch.cumsum(ctx, 0)
    tc = int(cu_kv[-1])
    kc = (torch.randn((h_kv * tc, D), generator=g) * 0.5).to(dtype).to(device)
    vc = None if mla else (torch.randn((h_kv * tc, D), generator=g) * 0.5).to(dtype).to(device)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=vc, total_context_len=tc, cu_seqlens_kv=cu_kv.to(device),
                           context_batch_size=B, is_mla=mla, num_heads=H, head_dim=D)
    meta = build_pack_metadata(lengths.to(device=device, dtype=torch.int32), N, 64)
    out, plan = hh._compressed_impl(q, k, v, H, meta, 1.0 / math.sqrt(D), cache, 0, mla, None, 64, 64, False,
                                    False, causal, run=False)
    return out, plan


def _noalloc(plan, out_like):
    p = _lib.AttnParams.from_buffer_copy(plan.params)
    out = torch.full_like(out_like, float("nan"))
    p.o = out.data_ptr()
    p.workspace, p.workspace_bytes, p.schedule = None, 0, None
    rc = plan.lib.fmlm_attn_fwd_noalloc(ctypes.byref(p), plan.stream)
    _lib.check(rc, "fmlm_attn_fwd_noalloc")
    return out


def test_noalloc_matches_fwd_on_consecutive_calls(device):
    cases = [
        # BASELINE config 3 shape class: enough query tiles that no key range is split
        dict(B=32, H=16, N=1024, D=128, dtype=torch.float16, lq=(256, 1024), lc=(512, 2048), seed=1, exact=True),
        # few query tiles and long contexts: split-KV, records cut to fit the scratch array
        dict(B=6, H=4, N=300, D=64, dtype=torch.bfloat16, lq=(40, 300), lc=(1500, 4000), causal=True, seed=2,
             exact=False),
        # MLA 512-wide latent, head-packed tiles
        dict(B=2, H=8, N=200, D=512, dtype=torch.bfloat16, lq=(100, 200), lc=(300, 700), mla=True, seed=3,
             exact=True),
    ]
    for c in cases:
        exact = c.pop("exact")
        print(f"[no_alloc] {c}", flush=True)
        out, plan = _case(device, **c)
        plan()
        got = _noalloc(plan, out)
        again = _noalloc(plan, out)  # the same call twice: the array's leftovers do not matter
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, again)
        if exact:
            assert torch.equal(got, out)
        else:
            torch.testing.assert_close(got.float(), out.float(), atol=1e-2, rtol=1e-2)


def test_noalloc_dense_and_errors(device):
    # dense calls need no schedule: the same result as fmlm_attn_fwd
    B, H, N, D = 2, 4, 96, 64
    q, k, v = (torch.randn((B, H, N, D), device=device).to(torch.bfloat16) for _ in range(3))
    out, plan = hh._dense_impl(q, k, v, 0.125, None, None, False, None, False, run=False)
    plan()
    got = _noalloc(plan, out)
    torch.cuda.synchronize()
    assert torch.equal(got, out)
    # an unsupported head dim is rejected before any launch
    p = _lib.AttnParams.from_buffer_copy(plan.params)
    p.D = 48
    assert plan.lib.fmlm_attn_fwd_noalloc(ctypes.byref(p), plan.stream) == -3  # unsupported head dim
