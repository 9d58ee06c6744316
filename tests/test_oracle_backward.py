"""Pins the attention-backward oracle (oracle/attention_ref.py *_backward) against the
mathematics, independently of its own formulas:

* central finite differences of the forward oracle (itself pinned by the forward tests):
  for f = sum(out * dout) over real rows and a random direction U per input tensor,
  (f(x + eps U) - f(x - eps U)) / 2 eps must equal <grad, U>;
* closed forms: one key (softmax = 1) gives dq = dK = 0 and dV = sum of dO; equal keys
  give dq = 0.

The reference has no backward pass (its roadmap lists one, README.md:26-28), so there
are no reference vectors for this path; the forward it differentiates follows
mlm_kernel_impl.py as restated by the forward oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention_ref as ar


def _dirderiv(f, args: dict, name: str, U: np.ndarray, eps: float = 1e-6) -> float:
    plus = dict(args)
    minus = dict(args)
    plus[name] = args[name] + eps * U
    minus[name] = args[name] - eps * U
    return (f(**plus) - f(**minus)) / (2 * eps)


def test_attend_backward_finite_differences_elementwise():
    rng = np.random.default_rng(0)
    q, K, V, dO = rng.standard_normal((3, 4)), rng.standard_normal((5, 4)), rng.standard_normal((5, 4)), rng.standard_normal((3, 4))
    scale = 0.7
    dq, dK, dV = ar.attend_backward(q, K, V, scale, dO)

    def f(q, K, V):
        return float((ar.attend(q, K, V, scale) * dO).sum())

    for name, g in (("q", dq), ("K", dK), ("V", dV)):
        base = {"q": q, "K": K, "V": V}
        num = np.zeros_like(g)
        for idx in np.ndindex(g.shape):
            U = np.zeros_like(g)
            U[idx] = 1.0
            num[idx] = _dirderiv(f, base, name, U)
        np.testing.assert_allclose(g, num, atol=1e-7, rtol=1e-6, err_msg=name)


def test_attend_backward_closed_forms():
    rng = np.random.default_rng(1)
    q, dO = rng.standard_normal((4, 8)), rng.standard_normal((4, 8))
    K, V = rng.standard_normal((1, 8)), rng.standard_normal((1, 8))
    dq, dK, dV = ar.attend_backward(q, K, V, 0.3, dO)  # one key: P = 1 everywhere
    np.testing.assert_allclose(dq, 0, atol=1e-12)
    np.testing.assert_allclose(dK, 0, atol=1e-12)
    np.testing.assert_allclose(dV, dO.sum(axis=0, keepdims=True), atol=1e-12)
    K2 = np.repeat(rng.standard_normal((1, 8)), 6, axis=0)  # equal keys: scores constant in q
    dq, _, dV = ar.attend_backward(q, K2, rng.standard_normal((6, 8)), 0.3, dO)
    np.testing.assert_allclose(dq, 0, atol=1e-12)
    np.testing.assert_allclose(dV, np.repeat(dO.sum(axis=0, keepdims=True) / 6, 6, axis=0), atol=1e-12)


def _packed_case(rng, *, mla, causal, prefill, index):
    B, H, N, D = 3, 2, 5, 4
    lengths = [5, 2, 3]
    q = rng.standard_normal((B, H, N, D))
    k = rng.standard_normal((B, H, N, D))
    v = rng.standard_normal((B, H, N, D))
    dout = rng.standard_normal((B, H, N, D))
    cbs = 2 if index else 3
    ctx_lens = [3, 0, 2][:cbs]
    cu_kv = np.concatenate([[0], np.cumsum(ctx_lens)]).astype(np.int64)
    total = int(cu_kv[-1]) + 1  # one spare row per head
    heads = 1 if mla else H
    k_cache = rng.standard_normal((heads * total, D))
    v_cache = None if mla else rng.standard_normal((heads * total, D))
    kw = dict(is_mla=mla, causal_query_seq_attn=causal, prefill=prefill, cu_seqlens_kv=cu_kv,
              total_context_len=total, context_batch_size=cbs, context_index=[1, 0, 1] if index else None)
    return q, k, v, dout, lengths, k_cache, v_cache, kw


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("index", [False, True])
def test_packed_backward_directional_derivatives(mla, causal, index):
    rng = np.random.default_rng(10 + 4 * mla + 2 * causal + index)
    q, k, v, dout, lengths, k_cache, v_cache, kw = _packed_case(rng, mla=mla, causal=causal, prefill=False, index=index)
    scale = 0.6
    mask = np.zeros(q.shape)
    for b, L in enumerate(lengths):
        mask[b, :, :L] = 1.0

    def f(q, k, v, k_cache, v_cache):
        out = ar.mlm_attention_packed(q, k, v, lengths, scale, k_cache=k_cache, v_cache=v_cache, **kw)
        return float((out * dout * mask).sum())

    grads = ar.mlm_attention_packed_backward(q, k, v, dout, lengths, scale, k_cache=k_cache, v_cache=v_cache, **kw)
    base = {"q": q, "k": k, "v": v, "k_cache": k_cache, "v_cache": v_cache}
    for name, g in zip(("q", "k", "v", "k_cache", "v_cache"), grads):
        if base[name] is None:
            assert g is None
            continue
        if g is None:  # MLA: v is ignored by the forward
            assert mla and name == "v"
            continue
        for _ in range(3):
            U = rng.standard_normal(g.shape)
            num = _dirderiv(f, base, name, U)
            assert abs(float((g * U).sum()) - num) <= 1e-6 * max(1.0, abs(num)), (name, float((g * U).sum()), num)
    # padding rows get no gradient; the gradient ignores dout's padding rows
    dq = grads[0]
    assert np.all(dq[mask == 0] == 0)
    dout2 = dout + 5.0 * (1 - mask)
    g2 = ar.mlm_attention_packed_backward(q, k, v, dout2, lengths, scale, k_cache=k_cache, v_cache=v_cache, **kw)
    for a, c in zip(grads, g2):
        if a is not None:
            np.testing.assert_allclose(a, c, atol=1e-12)


@pytest.mark.parametrize("mla", [False, True])
def test_packed_backward_prefill_has_no_context_gradient(mla):
    rng = np.random.default_rng(30 + mla)
    q, k, v, dout, lengths, k_cache, v_cache, kw = _packed_case(rng, mla=mla, causal=False, prefill=True, index=False)
    grads = ar.mlm_attention_packed_backward(q, k, v, dout, lengths, 0.5, k_cache=k_cache, v_cache=v_cache, **kw)
    assert np.all(grads[3] == 0)
    if not mla:
        assert np.all(grads[4] == 0)


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("cbs", [1, 2])
def test_dense_backward_directional_derivatives(mla, cbs):
    rng = np.random.default_rng(40 + 2 * mla + cbs)
    B, H, N, D, C = 2, 2, 3, 4, 2
    q, k, v, dout = (rng.standard_normal((B, H, N, D)) for _ in range(4))
    k_cache = rng.standard_normal((cbs * (1 if mla else H) * C, D))
    v_cache = None if mla else rng.standard_normal(k_cache.shape)
    scale = 0.8
    kw = dict(is_mla=mla, context_len=C, context_batch_size=cbs)

    def f(q, k, v, k_cache, v_cache):
        return float((ar.mlm_attention_dense(q, k, v, scale, k_cache=k_cache, v_cache=v_cache, **kw) * dout).sum())

    grads = ar.mlm_attention_dense_backward(q, k, v, dout, scale, k_cache=k_cache, v_cache=v_cache, **kw)
    base = {"q": q, "k": k, "v": v, "k_cache": k_cache, "v_cache": v_cache}
    for name, g in zip(("q", "k", "v", "k_cache", "v_cache"), grads):
        if g is None:
            continue
        for _ in range(3):
            U = rng.standard_normal(g.shape)
            num = _dirderiv(f, base, name, U)
            assert abs(float((g * U).sum()) - num) <= 1e-6 * max(1.0, abs(num)), (name, float((g * U).sum()), num)
