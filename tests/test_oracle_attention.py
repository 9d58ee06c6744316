"""Pin the numpy attention oracle (CPU only) with checks that do not restate its code:
closed forms, a library routine (torch SDPA) on explicitly concatenated key sets,
and invariances that a wrong index / sign / dropped segment / swapped operand breaks."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_ref as ar


def _rand(rng, *shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def _sdpa(q, K, V, scale):
    """torch's scaled_dot_product_attention (math path, fp64) on one head."""
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))[None, None]
    return F.scaled_dot_product_attention(t(q), t(K), t(V), scale=scale)[0, 0].numpy()


def _packed_case(rng, *, B=3, H=2, N=12, D=8, ctx=True, mla=False, cbs=None):
    L = np.array([int(rng.integers(1, N + 1)) for _ in range(B)])
    q, k, v = _rand(rng, B, H, N, D), _rand(rng, B, H, N, D), _rand(rng, B, H, N, D)
    cbs = B if cbs is None else cbs
    if ctx:
        Lc = rng.integers(0, 7, size=cbs)
    else:
        Lc = np.zeros(cbs, dtype=np.int64)
    cu_kv = np.concatenate([[0], np.cumsum(Lc)])
    Tc = int(cu_kv[-1]) + 2  # trailing rows nobody attends to
    kc = _rand(rng, (1 if mla else H) * Tc, D)
    vc = _rand(rng, (1 if mla else H) * Tc, D)
    return dict(q=q, k=k, v=v, L=L, kc=kc, vc=vc, cu_kv=cu_kv, Tc=Tc, cbs=cbs)


def _run_packed(c, scale, **kw):
    return ar.mlm_attention_packed(
        c["q"], c["k"], c["v"], c["L"], scale,
        k_cache=c["kc"], v_cache=c["vc"], cu_seqlens_kv=c["cu_kv"],
        total_context_len=c["Tc"], context_batch_size=c["cbs"], **kw,
    )


def _keys_for(c, b, h, *, mla, causal, prefill, cb=None):
    """Explicit key/value lists, written from test_host.py:48-105 (not from the oracle)."""
    L = c["L"]
    seqs = list(range(b + 1)) if causal else [b]
    K_main = np.concatenate([c["k"][s, 0 if mla else h, : L[s]] for s in seqs])
    V_main = K_main if mla else np.concatenate([c["v"][s, h, : L[s]] for s in seqs])
    if prefill:
        return K_main, V_main
    cb = (b if c["cbs"] > 1 else 0) if cb is None else cb
    c0, c1 = int(c["cu_kv"][cb]), int(c["cu_kv"][cb + 1])
    off = 0 if mla else h * c["Tc"]
    K_ctx = c["kc"][off + c0 : off + c1]
    V_ctx = K_ctx if mla else c["vc"][off + c0 : off + c1]
    return np.concatenate([K_ctx, K_main]), np.concatenate([V_ctx, V_main])


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("prefill", [False, True])
@pytest.mark.parametrize("shared_ctx", [False, True])
def test_packed_matches_sdpa_on_explicit_key_sets(mla, causal, prefill, shared_ctx):
    rng = np.random.default_rng(7 + 2 * mla + 4 * causal + 8 * prefill + 16 * shared_ctx)
    c = _packed_case(rng, mla=mla, cbs=1 if shared_ctx else None)
    scale = 0.37
    out = _run_packed(c, scale, is_mla=mla, causal_query_seq_attn=causal, prefill=prefill)
    B, H, N, _ = c["q"].shape
    for b in range(B):
        for h in range(H):
            K, V = _keys_for(c, b, h, mla=mla, causal=causal, prefill=prefill)
            np.testing.assert_allclose(out[b, h, : c["L"][b]], _sdpa(c["q"][b, h, : c["L"][b]], K, V, scale), atol=1e-12)
        assert np.all(out[b, :, c["L"][b] :] == 0)


@pytest.mark.parametrize("mla", [False, True])
def test_zero_queries_give_mean_of_attended_values(mla):
    rng = np.random.default_rng(3)
    c = _packed_case(rng, mla=mla)
    c["q"][:] = 0
    out = _run_packed(c, 1.0, is_mla=mla)
    for b in range(c["q"].shape[0]):
        for h in range(c["q"].shape[1]):
            _, V = _keys_for(c, b, h, mla=mla, causal=False, prefill=False)
            np.testing.assert_allclose(out[b, h, : c["L"][b]], np.broadcast_to(V.astype(np.float64).mean(0), out[b, h, : c["L"][b]].shape), atol=1e-12)


def test_single_key_returns_its_value_row():
    rng = np.random.default_rng(4)
    q, k, v = _rand(rng, 2, 3, 5, 8), _rand(rng, 2, 3, 5, 8), _rand(rng, 2, 3, 5, 8)
    out = ar.mlm_attention_packed(q, k, v, [1, 0], 0.9)
    np.testing.assert_allclose(out[0, :, 0], v[0, :, 0], atol=1e-12)
    assert np.all(out[1] == 0)


def test_large_scale_selects_argmax_key():
    rng = np.random.default_rng(5)
    q, k, v = _rand(rng, 1, 2, 6, 16), _rand(rng, 1, 2, 6, 16), _rand(rng, 1, 2, 6, 16)
    out = ar.mlm_attention_packed(q, k, v, [6], 1e4)
    for h in range(2):
        best = np.argmax(q[0, h] @ k[0, h].T, axis=1)
        np.testing.assert_allclose(out[0, h], v[0, h, best], atol=1e-6)
    # a negative scale selects the arg-min key instead
    out = ar.mlm_attention_packed(q, k, v, [6], -1e4)
    for h in range(2):
        worst = np.argmin(q[0, h] @ k[0, h].T, axis=1)
        np.testing.assert_allclose(out[0, h], v[0, h, worst], atol=1e-6)


def test_context_key_order_permutation_invariance_and_v_linearity():
    rng = np.random.default_rng(6)
    c = _packed_case(rng, B=2, H=2)
    out = _run_packed(c, 0.5)
    # permute cached rows inside each sequence's range (same permutation for K and V)
    kc, vc = c["kc"].copy(), c["vc"].copy()
    for h in range(2):
        for b in range(2):
            lo, hi = h * c["Tc"] + c["cu_kv"][b], h * c["Tc"] + c["cu_kv"][b + 1]
            perm = rng.permutation(hi - lo) + lo
            kc[lo:hi], vc[lo:hi] = c["kc"][perm], c["vc"][perm]
    c2 = dict(c, kc=kc, vc=vc)
    np.testing.assert_allclose(_run_packed(c2, 0.5), out, atol=1e-12)
    # linear in V (main and context values together)
    c3 = dict(c, v=2 * c["v"].astype(np.float64) + 1, vc=2 * c["vc"].astype(np.float64) + 1)
    np.testing.assert_allclose(_run_packed(c3, 0.5), np.where(out != 0, 2 * out + 1, 0), atol=1e-9)


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("cbs", [1, 2])
@pytest.mark.parametrize("prefill", [False, True])
def test_dense_matches_sdpa_on_explicit_key_sets(mla, cbs, prefill):
    rng = np.random.default_rng(20 + mla + 2 * cbs + 8 * prefill)
    B, H, N, D, ctx = 2, 3, 7, 8, 5
    q, k, v = _rand(rng, B, H, N, D), _rand(rng, B, H, N, D), _rand(rng, B, H, N, D)
    rows = cbs * ctx * (1 if mla else H)
    kc, vc = _rand(rng, rows, D), _rand(rng, rows, D)
    out = ar.mlm_attention_dense(q, k, v, 0.6, is_mla=mla, prefill=prefill, k_cache=kc, v_cache=vc,
                                 context_len=ctx, context_batch_size=cbs)
    # written from test_host.py:108-145
    for b in range(B):
        cb = 0 if cbs == 1 else b
        for h in range(H):
            K_main = k[b, h]
            V_main = K_main if mla else v[b, h]
            if prefill:
                K, V = K_main, V_main
            else:
                s = cb * ctx if mla else (cb * H + h) * ctx
                K_ctx = kc[s : s + ctx]
                V_ctx = K_ctx if mla else vc[s : s + ctx]
                K, V = np.concatenate([K_ctx, K_main]), np.concatenate([V_ctx, V_main])
            np.testing.assert_allclose(out[b, h], _sdpa(q[b, h], K, V, 0.6), atol=1e-12)


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_packed_context_index_matches_sdpa_on_explicit_key_sets(mla, causal):
    """Index-mapped context batching (an extension): sequence b attends to context batch
    context_index[b] of a 3-batch cache; checked against SDPA on the explicit key set of
    that batch, and context_index = arange(B) must reproduce the full-batch result."""
    rng = np.random.default_rng(90 + mla + 2 * causal)
    c = _packed_case(rng, B=4, mla=mla, cbs=3)
    idx = np.array([2, 0, 2, 1])
    scale = 0.41
    out = _run_packed(c, scale, is_mla=mla, causal_query_seq_attn=causal, context_index=idx)
    for b in range(4):
        for h in range(c["q"].shape[1]):
            K, V = _keys_for(c, b, h, mla=mla, causal=causal, prefill=False, cb=int(idx[b]))
            np.testing.assert_allclose(out[b, h, : c["L"][b]], _sdpa(c["q"][b, h, : c["L"][b]], K, V, scale), atol=1e-12)
    full = _packed_case(np.random.default_rng(95 + mla), B=3, mla=mla)
    np.testing.assert_array_equal(_run_packed(full, 0.3, is_mla=mla, context_index=np.arange(3)),
                                  _run_packed(full, 0.3, is_mla=mla))


@pytest.mark.parametrize("mla", [False, True])
def test_dense_context_index_matches_sdpa_on_explicit_key_sets(mla):
    rng = np.random.default_rng(97 + mla)
    B, H, N, D, ctx, C = 3, 2, 6, 8, 4, 2
    q, k, v = _rand(rng, B, H, N, D), _rand(rng, B, H, N, D), _rand(rng, B, H, N, D)
    rows = C * ctx * (1 if mla else H)
    kc, vc = _rand(rng, rows, D), _rand(rng, rows, D)
    idx = [1, 1, 0]
    out = ar.mlm_attention_dense(q, k, v, 0.6, is_mla=mla, k_cache=kc, v_cache=vc, context_len=ctx,
                                 context_batch_size=C, context_index=idx)
    for b in range(B):
        for h in range(H):
            s = idx[b] * ctx if mla else (idx[b] * H + h) * ctx
            K_main = k[b, h]
            V_main = K_main if mla else v[b, h]
            K = np.concatenate([kc[s : s + ctx], K_main])
            V = np.concatenate([K[:ctx] if mla else vc[s : s + ctx], V_main])
            np.testing.assert_allclose(out[b, h], _sdpa(q[b, h], K, V, 0.6), atol=1e-12)


def test_effective_flops_formula():
    # 4*H*D*sum Lq*(Lctx+Lmain); causal main = cu_q[b+1]; prefill drops context
    assert ar.effective_flops([2, 3], [5, 1], 2, 4) == 4 * 2 * 4 * (2 * 7 + 3 * 4)
    assert ar.effective_flops([2, 3], [5, 1], 2, 4, causal_query_seq_attn=True) == 4 * 2 * 4 * (2 * 7 + 3 * 6)
    assert ar.effective_flops([2, 3], [5, 1], 2, 4, prefill=True) == 4 * 2 * 4 * (2 * 2 + 3 * 3)
    assert ar.effective_flops([2, 3], 4, 1, 1) == 4 * (2 * 6 + 3 * 7)


def test_row_lse2_closed_forms():
    """row_lse2 (the forward's row statistic for the backward) against what the
    mathematics fixes: one key gives its own score in log2 units, M equal keys add
    log2(M), and 2^(z - lse) are the softmax weights, so they reproduce attend()."""
    rng = np.random.default_rng(11)
    q, K, V = _rand(rng, 5, 8), _rand(rng, 7, 8), _rand(rng, 7, 8)
    scale = 0.41
    z = (q.astype(np.float64) @ K.astype(np.float64).T) * scale / np.log(2.0)  # log2 units
    np.testing.assert_allclose(ar.row_lse2(q, K[:1], scale), z[:, 0], rtol=0, atol=1e-12)
    K3 = np.repeat(K[2:3], 3, axis=0)
    np.testing.assert_allclose(ar.row_lse2(q, K3, scale), z[:, 2] + np.log2(3.0), rtol=0, atol=1e-12)
    lse = ar.row_lse2(q, K, scale)
    w = np.exp2(z - lse[:, None])
    np.testing.assert_allclose(w.sum(axis=1), 1.0, atol=1e-12)
    np.testing.assert_allclose(w @ V.astype(np.float64), ar.attend(q, K, V, scale), atol=1e-12)
    # brute force on the explicit sum, for scores far from 0 (no overflow in float64)
    q40 = q.astype(np.float64) * 40
    big = ar.row_lse2(q40, K, scale)
    zb = (q40 @ K.astype(np.float64).T) * scale / np.log(2.0)
    np.testing.assert_allclose(big, np.log2(np.exp2(zb).sum(axis=1)), rtol=1e-12)


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_row_lse2_packed_and_dense_on_explicit_key_sets(mla, causal):
    rng = np.random.default_rng(21 + mla + 2 * causal)
    c = _packed_case(rng, mla=mla)
    scale = 0.37
    got = ar.mlm_row_lse2_packed(c["q"], c["k"], c["L"], scale, is_mla=mla, causal_query_seq_attn=causal,
                                 k_cache=c["kc"], cu_seqlens_kv=c["cu_kv"], total_context_len=c["Tc"],
                                 context_batch_size=c["cbs"])
    B, H, N, _ = c["q"].shape
    for b in range(B):
        for h in range(H):
            K, _ = _keys_for(c, b, h, mla=mla, causal=causal, prefill=False)
            np.testing.assert_allclose(got[b, h, : c["L"][b]], ar.row_lse2(c["q"][b, h, : c["L"][b]], K, scale),
                                       atol=1e-12)
        assert np.all(got[b, :, c["L"][b]:] == 0)
    # dense: every query sees [context || its own N keys]
    q, k = c["q"], c["k"]
    Lc = 3
    kc = _rand(rng, B * Lc, 8) if mla else _rand(rng, B * H * Lc, 8)
    got = ar.mlm_row_lse2_dense(q, k, scale, is_mla=mla, k_cache=kc, context_len=Lc, context_batch_size=B)
    for b in range(B):
        for h in range(H):
            start = b * Lc if mla else (b * H + h) * Lc
            K = np.concatenate([kc[start:start + Lc], k[b, h]])  # MLA keeps per-head main keys
            np.testing.assert_allclose(got[b, h], ar.row_lse2(q[b, h], K, scale), atol=1e-12)
