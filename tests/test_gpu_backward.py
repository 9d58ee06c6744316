"""GPU tests of the attention backward (fmlm_attn_bwd through torch.autograd on the three
entry points; an extension: the reference's roadmap lists backpropagation,
README.md:26-28).  Gradients of q, k, v and of the cached context are compared with the
float64 oracle (oracle/attention_ref.py *_backward, itself pinned by finite differences
in test_oracle_backward.py), and at a larger size with torch autograd of a float32
per-sequence softmax attention.

Tolerance: bf16/fp16 inputs with fp32 accumulation, and P and dS rounded to the input
type before their products (as the forward rounds P), so each gradient is held to
|gpu - ref| <= TOL * max|ref| + TOL * |ref| with TOL = 2e-2 per element (max|ref| over
the whole gradient tensor, which must be nonzero).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flash_mlm import InferenceCache, build_pack_metadata, flash_attn_mlm, flash_attn_mlm_compressed, \
    flash_attn_mlm_precompressed
from oracle import attention_ref as ar

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _close(got, ref, what):
    got = _np(got)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    assert scale > 0, f"{what}: reference gradient is zero"
    err = np.abs(got - ref)
    bound = TOL * scale + TOL * np.abs(ref)
    worst = float((err - bound).max())
    print(f"{what}: max err / max |ref| = {float(err.max()) / scale:.2e}")
    assert worst <= 0, f"{what}: max err {float(err.max()):.3e} (ref max {scale:.3e})"


def _leaf(shape, dtype, device, gen, mult=0.5):
    return (torch.randn(shape, generator=gen) * mult).to(dtype).to(device).requires_grad_()


def _packed_cache(ctx_lens, *, H, D, mla, dtype, device, gen):
    cu = np.concatenate([[0], np.cumsum(ctx_lens)]).astype(np.int32)
    total = int(cu[-1]) + 3  # spare rows per head
    heads = 1 if mla else H
    kc = _leaf((heads * total, D), dtype, device, gen)
    vc = None if mla else _leaf((heads * total, D), dtype, device, gen)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=vc, total_context_len=total,
                           cu_seqlens_kv=torch.from_numpy(cu).to(device), context_batch_size=len(ctx_lens),
                           is_mla=mla, num_heads=H, head_dim=D)
    return cache, kc, vc, cu, total


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_compressed_with_context(dtype, D, mla, causal, device):
    gen = torch.Generator().manual_seed(7000 + D + 2 * mla + causal)
    lengths = [70, 1, 0, 133, 40]
    B, H, N = len(lengths), 3, 140
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache([129, 0, 64, 7, 90], H=H, D=D, mla=mla, dtype=dtype,
                                                device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, is_mla=mla, block_n=64,
                                    causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    # dout in padded form for the oracle
    from flash_mlm import unpack_from_kernel
    dout_pad = _np(unpack_from_kernel(dout, meta, H))
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(v), dout_pad, lengths, scale, is_mla=mla, causal_query_seq_attn=causal,
        k_cache=_np(kc), v_cache=None if mla else _np(vc), cu_seqlens_kv=cu_kv, total_context_len=total,
        context_batch_size=B)
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk")
    if mla:
        assert v.grad is None
    else:
        _close(v.grad, g[2], "dv")
    _close(kc.grad, g[3], "dk_cache")
    if not mla:
        _close(vc.grad, g[4], "dv_cache")


@pytest.mark.parametrize("D", [32, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_compressed_head_dims(D, causal, device):
    gen = torch.Generator().manual_seed(7100 + D + causal)
    lengths = [33, 64, 5]
    B, H, N, dtype = len(lengths), 2, 64, torch.bfloat16
    scale = 0.3
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache([20, 65, 1], H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)), lengths, scale, k_cache=_np(kc),
        v_cache=_np(vc), cu_seqlens_kv=cu_kv, total_context_len=total, context_batch_size=B,
        causal_query_seq_attn=causal)
    for got, ref, name in ((q.grad, g[0], "dq"), (k.grad, g[1], "dk"), (v.grad, g[2], "dv"),
                           (kc.grad, g[3], "dkc"), (vc.grad, g[4], "dvc")):
        _close(got, ref, name)


def test_backward_context_index_and_frozen_cache(device):
    """Two context batches shared by three sequences through context_index; the cache
    does not require grad, so only q, k, v get gradients."""
    gen = torch.Generator().manual_seed(7200)
    lengths = [50, 17, 80]
    B, H, N, D, dtype = len(lengths), 2, 80, 64, torch.float16
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache([100, 33], H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
    kc.requires_grad_(False)
    vc.requires_grad_(False)
    idx = torch.tensor([1, 0, 1], dtype=torch.int32)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.125, cache, 0, block_n=64, context_index=idx)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)), lengths, 0.125, k_cache=_np(kc),
        v_cache=_np(vc), cu_seqlens_kv=cu_kv, total_context_len=total, context_batch_size=2,
        context_index=idx.tolist())
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk")
    _close(v.grad, g[2], "dv")
    assert kc.grad is None and vc.grad is None


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("cbs", [1, 3, 2])
def test_backward_dense_with_context(mla, cbs, device):
    """cbs 1: shared context; 3: one per sequence; 2: two contexts for three sequences
    through context_index."""
    gen = torch.Generator().manual_seed(7300 + 2 * mla + cbs)
    B, H, N, D, C, dtype = 3, 2, 96, 64, 70, torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    kc = _leaf((cbs * (1 if mla else H) * C, D), dtype, device, gen)
    vc = None if mla else _leaf(kc.shape, dtype, device, gen)
    cache = InferenceCache()
    cache.prefill_kv_cache(0, k_cache=kc, v_cache=vc, context_batch_size=cbs, is_mla=mla, num_heads=H, head_dim=D)
    idx = torch.tensor([1, 0, 1], dtype=torch.int32) if cbs == 2 else None
    out = flash_attn_mlm(q, k, v, scale, cache, 0, is_mla=mla, context_index=idx)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    g = ar.mlm_attention_dense_backward(_np(q), _np(k), _np(v), _np(dout), scale, is_mla=mla, k_cache=_np(kc),
                                        v_cache=None if mla else _np(vc), context_len=C, context_batch_size=cbs,
                                        context_index=None if idx is None else idx.tolist())
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk")
    _close(kc.grad, g[3], "dk_cache")
    if not mla:
        _close(v.grad, g[2], "dv")
        _close(vc.grad, g[4], "dv_cache")


@pytest.mark.parametrize("causal", [False, True])
def test_backward_precompressed_matches_compressed(causal, device):
    """Same call through the precompressed and the compressed entry points, each with its
    own copy of a cached context: equal gradients for q, k, v and the context."""
    gen = torch.Generator().manual_seed(7400 + causal)
    lengths = [40, 3, 77]
    B, H, N, D, dtype = len(lengths), 2, 80, 128, torch.bfloat16
    q0, k0, v0 = ((torch.randn((B, H, N, D), generator=gen) * 0.5).to(dtype).to(device) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    T = sum(lengths)
    # packed copies as leaves
    qp = torch.cat([q0[b, :, : lengths[b]] for b in range(B)], dim=1).reshape(H * T, D).contiguous().requires_grad_()
    kp = torch.cat([k0[b, :, : lengths[b]] for b in range(B)], dim=1).reshape(H * T, D).contiguous().requires_grad_()
    vp = torch.cat([v0[b, :, : lengths[b]] for b in range(B)], dim=1).reshape(H * T, D).contiguous().requires_grad_()
    cache1, kc1, vc1, _, _ = _packed_cache([30, 0, 100], H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
    cache2, kc2, vc2, _, _ = _packed_cache([30, 0, 100], H=H, D=D, mla=False, dtype=dtype, device=device,
                                           gen=torch.Generator().manual_seed(0))
    with torch.no_grad():
        kc2.copy_(kc1)
        vc2.copy_(vc1)
    out = flash_attn_mlm_precompressed(qp, kp, vp, H, T, meta.cu_seqlens, meta.batch_ids_q, meta.q_tile_starts_q,
                                       0.2, cache1, 0, block_n=64, causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    qd, kd, vd = (t.clone().requires_grad_() for t in (q0, k0, v0))
    out2 = flash_attn_mlm_compressed(qd, kd, vd, H, meta, 0.2, cache2, 0, block_n=64, causal_query_seq_attn=causal)
    out2.backward(dout)
    torch.testing.assert_close(kc1.grad, kc2.grad, atol=1e-5, rtol=0)
    torch.testing.assert_close(vc1.grad, vc2.grad, atol=1e-5, rtol=0)
    assert torch.count_nonzero(kc1.grad) > 0

    def packed(x):
        return torch.cat([x[b, :, : lengths[b]] for b in range(B)], dim=1).reshape(H * T, D)

    torch.testing.assert_close(qp.grad, packed(qd.grad), atol=1e-5, rtol=0)
    torch.testing.assert_close(kp.grad, packed(kd.grad), atol=1e-5, rtol=0)
    torch.testing.assert_close(vp.grad, packed(vd.grad), atol=1e-5, rtol=0)


def test_backward_prefill_and_no_context(device):
    gen = torch.Generator().manual_seed(7500)
    lengths = [64, 9]
    B, H, N, D, dtype = 2, 2, 64, 64, torch.bfloat16
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    cache = InferenceCache()
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.25, cache, 0, block_n=64, prefill=True)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(_np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)), lengths,
                                         0.25)
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk")
    _close(v.grad, g[2], "dv")


def test_backward_against_torch_fp32_autograd(device):
    """Larger case (contexts and sequences of hundreds of keys) against torch autograd of a
    float32 per-sequence softmax attention on the GPU."""
    gen = torch.Generator().manual_seed(7600)
    lengths = [256, 100, 193, 7]
    ctx = [512, 300, 0, 64]
    B, H, N, D, dtype = len(lengths), 4, 256, 128, torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache(ctx, H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)

    qf, kf, vf = (x.detach().float().requires_grad_() for x in (q, k, v))
    kcf, vcf = (x.detach().float().requires_grad_() for x in (kc, vc))
    T = sum(lengths)
    cu_q = np.concatenate([[0], np.cumsum(lengths)])
    loss = 0.0
    doutf = dout.float()
    for b in range(B):
        L = lengths[b]
        if L == 0:
            continue
        for h in range(H):
            Kc = kcf[h * total + cu_kv[b]: h * total + cu_kv[b + 1]]
            Vc = vcf[h * total + cu_kv[b]: h * total + cu_kv[b + 1]]
            K = torch.cat([Kc, kf[b, h, :L]])
            V = torch.cat([Vc, vf[b, h, :L]])
            p = torch.softmax((qf[b, h, :L] @ K.t()) * scale, dim=-1)
            o = p @ V
            loss = loss + (o * doutf[h * T + cu_q[b]: h * T + cu_q[b] + L]).sum()
    loss.backward()
    for got, ref, name in ((q.grad, qf.grad, "dq"), (k.grad, kf.grad, "dk"), (v.grad, vf.grad, "dv"),
                           (kc.grad, kcf.grad, "dkc"), (vc.grad, vcf.grad, "dvc")):
        _close(got, ref.detach().cpu().numpy().astype(np.float64), name)


@pytest.mark.parametrize("dtype,D,mode", [
    (dt, d, m) for dt, d in [(torch.float32, 64), (torch.float32, 128), (torch.float32, 16),
                             (torch.bfloat16, 16), (torch.float16, 16)] for m in ("ctx", "causal_mla_ctx")
] + [(torch.float32, 512, "causal_mla_ctx")])
def test_backward_simt_kernels(dtype, D, mode, device):
    """fp32 inputs and head dim 16 take the SIMT backward kernels; fp32 gradients are held
    to 1e-4 of the largest reference entry, bf16/fp16 to the tolerance above."""
    gen = torch.Generator().manual_seed(8300 + D + (mode == "ctx"))
    mla, causal = "mla" in mode, "causal" in mode
    lengths = [70, 1, 0, 45]
    B, H, N = len(lengths), 3, 72
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache([65, 0, 130, 7], H=H, D=D, mla=mla, dtype=dtype, device=device,
                                                gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, k if mla else v, H, meta, scale, cache, 0, is_mla=mla, block_n=64,
                                    causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(k if mla else v), _np(unpack_from_kernel(dout, meta, H)), lengths, scale, is_mla=mla,
        causal_query_seq_attn=causal, k_cache=_np(kc), v_cache=None if mla else _np(vc), cu_seqlens_kv=cu_kv,
        total_context_len=total, context_batch_size=B)
    pairs = [(q.grad, g[0], "dq"), (k.grad, g[1], "dk"), (kc.grad, g[3], "dkc")]
    if not mla:
        pairs += [(v.grad, g[2], "dv"), (vc.grad, g[4], "dvc")]
    for got, ref, name in pairs:
        if dtype == torch.float32:
            err = float(np.abs(_np(got) - ref).max()) / float(np.abs(ref).max())
            assert err <= 1e-4, f"{name}: {err:.2e}"
        else:
            _close(got, ref, name)


def test_backward_dense_fp32_config1_shape(device):
    """The dense fp32 workload of the reference's CPU-runnable configuration, through the
    SIMT backward."""
    gen = torch.Generator().manual_seed(8400)
    B, H, N, D = 2, 8, 128, 64
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), torch.float32, device, gen, mult=1.0) for _ in range(3))
    out = flash_attn_mlm(q, k, v, scale)
    dout = torch.randn(out.shape, generator=gen).to(device)
    out.backward(dout)
    g = ar.mlm_attention_dense_backward(_np(q), _np(k), _np(v), _np(dout), scale)
    for got, ref, name in ((q.grad, g[0], "dq"), (k.grad, g[1], "dk"), (v.grad, g[2], "dv")):
        err = float(np.abs(_np(got) - ref).max()) / float(np.abs(ref).max())
        assert err <= 1e-4, f"{name}: {err:.2e}"


def test_backward_mla_shared_tensor_and_strided_views(device):
    """MLA called as (q, k, k) with one tensor (its gradient is the latent's), and q/k/v
    given as non-contiguous views of [B, N, H, D] buffers."""
    gen = torch.Generator().manual_seed(7700)
    lengths = [48, 20]
    B, H, N, D, dtype = 2, 4, 48, 64, torch.bfloat16
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    from flash_mlm import unpack_from_kernel

    q = _leaf((B, H, N, D), dtype, device, gen)
    k = _leaf((B, H, N, D), dtype, device, gen)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, 0.2, is_mla=True, block_n=64)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    g = ar.mlm_attention_packed_backward(_np(q), _np(k), _np(k), _np(unpack_from_kernel(dout, meta, H)), lengths,
                                         0.2, is_mla=True)
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk (latent = head 0)")
    assert torch.count_nonzero(k.grad[:, 1:]) == 0  # only head 0 is read

    base = [(torch.randn((B, N, H, D), generator=gen) * 0.5).to(dtype).to(device).requires_grad_() for _ in range(3)]
    qv, kv, vv = (t.transpose(1, 2) for t in base)  # [B, H, N, D] views, not contiguous
    out = flash_attn_mlm_compressed(qv, kv, vv, H, meta, 0.2, block_n=64)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    g = ar.mlm_attention_packed_backward(_np(qv), _np(kv), _np(vv), _np(unpack_from_kernel(dout, meta, H)),
                                         lengths, 0.2)
    for t, ref, name in zip(base, g[:3], ("dq", "dk", "dv")):
        _close(t.grad.transpose(1, 2), ref, name + " (strided)")


@pytest.mark.parametrize("causal", [False, True])
def test_backward_mla_latent_512(causal, device):
    """The 512-wide MLA latent (the BASELINE MLA shape) with a cached latent context."""
    gen = torch.Generator().manual_seed(7800 + causal)
    lengths = [70, 1, 0, 33]
    B, H, N, D, dtype = len(lengths), 4, 72, 512, torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    q = _leaf((B, H, N, D), dtype, device, gen)
    k = _leaf((B, H, N, D), dtype, device, gen)
    cache, kc, _, cu_kv, total = _packed_cache([65, 0, 130, 7], H=H, D=D, mla=True, dtype=dtype, device=device,
                                               gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, k, H, meta, scale, cache, 0, is_mla=True, block_n=64,
                                    causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(k), _np(unpack_from_kernel(dout, meta, H)), lengths, scale, is_mla=True,
        causal_query_seq_attn=causal, k_cache=_np(kc), cu_seqlens_kv=cu_kv, total_context_len=total,
        context_batch_size=B)
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk (latent)")
    _close(kc.grad, g[3], "dk_cache (latent)")


def test_backward_through_projections_matches_torch(device):
    """Training use: q, k, v are projections of activations (non-leaf tensors, permuted
    views); the gradients of the projection weights and the activations through the HIP
    attention match torch autograd of float32 per-sequence attention."""
    gen = torch.Generator().manual_seed(7900)
    lengths = [40, 64, 9]
    B, H, N, D, dm, dtype = len(lengths), 2, 64, 64, 96, torch.bfloat16
    x0 = (torch.randn((B, N, dm), generator=gen) * 0.5).to(dtype).to(device)
    w0 = [(torch.randn((dm, H * D), generator=gen) / math.sqrt(dm)).to(dtype).to(device) for _ in range(3)]
    y = torch.randn((H * sum(lengths), D), generator=gen).to(dtype).to(device)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)

    x = x0.clone().requires_grad_()
    w = [t.clone().requires_grad_() for t in w0]
    q, k, v = ((x @ wi).view(B, N, H, D).permute(0, 2, 1, 3) for wi in w)  # [B, H, N, D] views
    out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.125, block_n=64)
    (out.float() * y.float()).sum().backward()

    xf = x0.float().requires_grad_()
    wf = [t.float().requires_grad_() for t in w0]
    qf, kf, vf = ((xf @ wi).view(B, N, H, D).permute(0, 2, 1, 3) for wi in wf)
    T = sum(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    loss = 0.0
    for b, L in enumerate(lengths):
        for h in range(H):
            # keys rounded like the kernel's bf16 inputs, math in fp32
            qb, kb, vb = (t[b, h, :L].to(dtype).float() for t in (qf, kf, vf))
            o = torch.softmax(qb @ kb.t() * 0.125, dim=-1) @ vb
            loss = loss + (o * y[h * T + cu[b]: h * T + cu[b] + L].float()).sum()
    loss.backward()
    _close(x.grad, xf.grad.detach().cpu().numpy().astype(np.float64), "dx")
    for i, name in enumerate(("dWq", "dWk", "dWv")):
        _close(w[i].grad, wf[i].grad.detach().cpu().numpy().astype(np.float64), name)


@pytest.mark.parametrize("causal", [False, True])
def test_backward_long_sequences_against_torch(causal, device):
    """Thousands of keys per row (long sequences and contexts, many tiles accumulated per
    gradient row) against torch autograd of float32 attention on the GPU."""
    gen = torch.Generator().manual_seed(8000 + causal)
    lengths = [2048, 1500]
    ctx = [4096, 0] if not causal else [3000, 100]
    B, H, N, D, dtype = len(lengths), 2, 2048, 128, torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache(ctx, H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)

    qf, kf, vf, kcf, vcf = (x.detach().float().requires_grad_() for x in (q, k, v, kc, vc))
    T = sum(lengths)
    cu_q = np.concatenate([[0], np.cumsum(lengths)])
    loss = 0.0
    for b, L in enumerate(lengths):
        for h in range(H):
            Kc = kcf[h * total + cu_kv[b]: h * total + cu_kv[b + 1]]
            Vc = vcf[h * total + cu_kv[b]: h * total + cu_kv[b + 1]]
            seqs = range(b + 1) if causal else (b,)
            Km = torch.cat([kf[s, h, : lengths[s]] for s in seqs])
            Vm = torch.cat([vf[s, h, : lengths[s]] for s in seqs])
            p = torch.softmax((qf[b, h, :L] @ torch.cat([Kc, Km]).t()) * scale, dim=-1)
            loss = loss + ((p @ torch.cat([Vc, Vm])) * dout[h * T + cu_q[b]: h * T + cu_q[b] + L].float()).sum()
    loss.backward()
    for got, ref, name in ((q.grad, qf.grad, "dq"), (k.grad, kf.grad, "dk"), (v.grad, vf.grad, "dv"),
                           (kc.grad, kcf.grad, "dkc"), (vc.grad, vcf.grad, "dvc")):
        _close(got, ref.detach().cpu().numpy().astype(np.float64), name)


def test_backward_two_causal_calls_sharing_a_cache(device):
    """Two layers' causal calls through one InferenceCache, then one backward: the second
    forward must not overwrite the packed K/V the first call's backward reads (the
    cache's reusable packing buffers are not used for calls under autograd)."""
    gen = torch.Generator().manual_seed(8100)
    lengths = [40, 25, 64]
    B, H, N, D, dtype = len(lengths), 2, 64, 64, torch.bfloat16
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    cache = InferenceCache()
    calls = []
    for layer in range(2):
        q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
        out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.2, cache, layer, block_n=64, causal_query_seq_attn=True)
        dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
        calls.append((q, k, v, out, dout))
    sum((out.float() * dout.float()).sum() for _, _, _, out, dout in calls).backward()
    from flash_mlm import unpack_from_kernel
    for layer, (q, k, v, _, dout) in enumerate(calls):
        g = ar.mlm_attention_packed_backward(_np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)),
                                             lengths, 0.2, causal_query_seq_attn=True)
        _close(q.grad, g[0], f"layer {layer} dq")
        _close(k.grad, g[1], f"layer {layer} dk")
        _close(v.grad, g[2], f"layer {layer} dv")


def test_backward_rejects_inputs_changed_in_place(device):
    """The backward reads the tensors of the forward call: changing q or the cached
    context in place between forward and backward is an autograd error."""
    gen = torch.Generator().manual_seed(8200)
    lengths = [20, 9]
    B, H, N, D, dtype = 2, 2, 20, 64, torch.bfloat16
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    for target in ("q", "cache"):
        q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
        cache, kc, vc, _, _ = _packed_cache([10, 5], H=H, D=D, mla=False, dtype=dtype, device=device, gen=gen)
        out = flash_attn_mlm_compressed(q, k, v, H, meta, 0.2, cache, 0, block_n=64)
        with torch.no_grad():
            (q if target == "q" else kc).mul_(2.0)
        with pytest.raises(RuntimeError, match="modified by an inplace operation"):
            out.sum().backward()


@pytest.mark.parametrize("causal", [False, True])
def test_backward_more_sequences_than_the_rank_limit(causal, device):
    # the dq kernel visits sequences by key count for up to 1024 of them and in index
    # order beyond: 1030 short sequences (some empty) take the second path
    gen = torch.Generator().manual_seed(7300 + causal)
    lengths = torch.randint(0, 4, (1030,), generator=gen).tolist()
    B, H, N, D = len(lengths), 1, 4, 32
    scale = 1.0 / math.sqrt(D)
    q, k, v = (_leaf((B, H, N, D), torch.bfloat16, device, gen) for _ in range(3))
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, None, None, block_n=64, causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(torch.bfloat16).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(_np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)), lengths,
                                         scale, causal_query_seq_attn=causal)
    _close(q.grad, g[0], "dq")
    _close(k.grad, g[1], "dk")
    _close(v.grad, g[2], "dv")


@pytest.mark.parametrize("scale", [-0.2, 0.0])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_non_positive_scale(scale, causal, device):
    """A negative or zero softmax scale (the entry points pass any float through): keys a
    query does not see must still get P = 0 in every kernel, whatever sign the scale gives
    their masked scores."""
    gen = torch.Generator().manual_seed(7400 + int(scale * 10) + causal)
    lengths = [70, 1, 0, 133, 40]
    B, H, N, D, dtype = len(lengths), 2, 140, 64, torch.bfloat16
    q, k, v = (_leaf((B, H, N, D), dtype, device, gen) for _ in range(3))
    cache, kc, vc, cu_kv, total = _packed_cache([129, 0, 64, 7, 90], H=H, D=D, mla=False, dtype=dtype,
                                                device=device, gen=gen)
    meta = build_pack_metadata(torch.tensor(lengths, device=device, dtype=torch.int32), N, block_n=64)
    out = flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, block_n=64, causal_query_seq_attn=causal)
    dout = torch.randn(out.shape, generator=gen).to(dtype).to(device)
    out.backward(dout)
    from flash_mlm import unpack_from_kernel
    g = ar.mlm_attention_packed_backward(
        _np(q), _np(k), _np(v), _np(unpack_from_kernel(dout, meta, H)), lengths, scale, k_cache=_np(kc),
        v_cache=_np(vc), cu_seqlens_kv=cu_kv, total_context_len=total, context_batch_size=B,
        causal_query_seq_attn=causal)
    names = ("dq", "dk", "dv", "dk_cache", "dv_cache")
    for got, ref, name in zip((q.grad, k.grad, v.grad, kc.grad, vc.grad), g, names):
        if scale == 0.0 and name in ("dq", "dk", "dk_cache"):  # dS = scale * ... = 0
            assert float(got.abs().max()) == 0.0, name
            continue
        _close(got, ref, name)
