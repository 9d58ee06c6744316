"""Numpy restatement of the reference's MLM attention -- test infrastructure only.

The reference computes, per query tile, an online softmax over [cached context ||
main keys] (src/flash_mlm/mlm_kernel_impl.py:10-62); mathematically that is plain
softmax attention over the concatenated key set, which is what these functions
compute, in float64, one (sequence, head) at a time.  Which keys a query sees and
where they live follows the device bodies:
  packed  _mlm_compressed_kernel_impl  mlm_kernel_impl.py:219-390
  dense   _mlm_main_kernel_impl        mlm_kernel_impl.py:65-216
and the reference's own test oracles (src/flash_mlm/host/test_host.py:30-145).
"""

from __future__ import annotations

import numpy as np


def attend(q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float) -> np.ndarray:
    """softmax(scale * q K^T) V for q [L, D], K/V [M, D] (M >= 1), in float64."""
    q = q.astype(np.float64)
    K = K.astype(np.float64)
    V = V.astype(np.float64)
    s = (q @ K.T) * float(scale)
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ V


def row_lse2(q: np.ndarray, K: np.ndarray, scale: float) -> np.ndarray:
    """log2 of sum_j 2^(z_j) with z = scale * log2(e) * q K^T, per row of q [L, D] against
    K [M, D] (M >= 1), in float64: logsumexp(scale q K^T) / ln 2, the row statistic the
    forward stores for the backward (an extension: the reference's kernels return o
    only).  Then attend(q, K, V) = sum_j 2^(z_j - lse) V_j."""
    s = (q.astype(np.float64) @ K.astype(np.float64).T) * float(scale)
    m = s.max(axis=1)
    return (m + np.log(np.exp(s - m[:, None]).sum(axis=1))) / np.log(2.0)


def attend_backward(q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float, dO: np.ndarray):
    """Gradients of ``attend`` for an upstream gradient dO [L, D]: returns (dq, dK, dV) in
    float64.  With P = softmax(scale q K^T) and O = P V:
    dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)), dq = scale dS K,
    dK = scale dS^T q (the softmax Jacobian diag(P) - P P^T applied row by row)."""
    q = q.astype(np.float64)
    K = K.astype(np.float64)
    V = V.astype(np.float64)
    dO = dO.astype(np.float64)
    s = (q @ K.T) * float(scale)
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    o = p @ V
    dV = p.T @ dO
    dP = dO @ V.T
    delta = (dO * o).sum(axis=1, keepdims=True)
    dS = p * (dP - delta) * float(scale)
    return dS @ K, dS.T @ q, dV


def packed_key_rows(b: int, lengths, causal_query_seq_attn: bool) -> list[tuple[int, int]]:
    """(sequence, position) of the main keys of sequence b in packed order:
    sequence b's own tokens, or with causal_query_seq_attn all tokens of sequences
    0..b (mlm_kernel_impl.py:288-293)."""
    seqs = range(b + 1) if causal_query_seq_attn else (b,)
    return [(s, p) for s in seqs for p in range(int(lengths[s]))]


def mlm_attention_packed(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    lengths,
    scale: float,
    *,
    is_mla: bool = False,
    causal_query_seq_attn: bool = False,
    prefill: bool = False,
    k_cache: np.ndarray | None = None,
    v_cache: np.ndarray | None = None,
    cu_seqlens_kv=None,
    total_context_len: int = 0,
    context_batch_size: int = 1,
    context_index=None,
) -> np.ndarray:
    """Packed-path attention on padded q/k/v [B, H, N, D] -> [B, H, N, D] (float64),
    zeros at padding positions.

    Context of sequence b (skipped when ``prefill``): rows
    ``h_off + cu_seqlens_kv[cb] .. h_off + cu_seqlens_kv[cb+1]`` of the head-major cache,
    ``cb = b`` if context_batch_size > 1 else 0, ``h_off = h * total_context_len``
    (0 for MLA).  MLA: main K = V = head 0 of k, context V = context K.
    ``context_index`` (index-mapped context batching, an extension the reference lists on
    its roadmap, README.md:34-36) sets ``cb = context_index[b]`` instead.
    """
    return _mlm_packed(q, k, v, lengths, scale, is_mla, causal_query_seq_attn, prefill, k_cache, v_cache,
                       cu_seqlens_kv, total_context_len, context_batch_size, context_index, attend)


def mlm_row_lse2_packed(q, k, lengths, scale, *, is_mla=False, causal_query_seq_attn=False, prefill=False,
                        k_cache=None, cu_seqlens_kv=None, total_context_len=0, context_batch_size=1,
                        context_index=None) -> np.ndarray:
    """row_lse2 of every real query row over the key set of mlm_attention_packed (same
    arguments, values unused): [B, H, N], zeros at padding positions."""
    def lse(qq, K, V, sc):
        return row_lse2(qq, K, sc)[:, None]

    return _mlm_packed(q, k, k, lengths, scale, is_mla, causal_query_seq_attn, prefill, k_cache, k_cache,
                       cu_seqlens_kv, total_context_len, context_batch_size, context_index, lse)[..., 0]


def _mlm_packed(q, k, v, lengths, scale, is_mla, causal_query_seq_attn, prefill, k_cache, v_cache, cu_seqlens_kv,
                total_context_len, context_batch_size, context_index, fn):
    """fn(q rows, K_all, V_all, scale) -> [L, W] over each (sequence, head)'s key set."""
    B, H, N, D = q.shape
    out = None
    cu_kv = None if cu_seqlens_kv is None else np.asarray(cu_seqlens_kv, dtype=np.int64)
    for b in range(B):
        Lq = int(lengths[b])
        if Lq == 0:
            continue
        rows = packed_key_rows(b, lengths, causal_query_seq_attn)
        sb = np.array([r[0] for r in rows])
        pb = np.array([r[1] for r in rows])
        c0 = c1 = 0
        if not prefill and cu_kv is not None:
            cb = int(context_index[b]) if context_index is not None else (b if context_batch_size > 1 else 0)
            c0, c1 = int(cu_kv[cb]), int(cu_kv[cb + 1])
        for h in range(H):
            kh = 0 if is_mla else h
            K_main = k[sb, kh, pb]
            V_main = K_main if is_mla else v[sb, h, pb]
            if c1 > c0:
                off = 0 if is_mla else h * total_context_len
                K_ctx = k_cache[off + c0 : off + c1]
                V_ctx = K_ctx if is_mla else v_cache[off + c0 : off + c1]
                K_all = np.concatenate([K_ctx, K_main])
                V_all = np.concatenate([V_ctx, V_main])
            else:
                K_all, V_all = K_main, V_main
            r = fn(q[b, h, :Lq], K_all, V_all, scale)
            if out is None:
                out = np.zeros((B, H, N, r.shape[1]), dtype=np.float64)
            out[b, h, :Lq] = r
    return np.zeros((B, H, N, D), dtype=np.float64) if out is None else out


def mlm_attention_packed_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    dout: np.ndarray,
    lengths,
    scale: float,
    *,
    is_mla: bool = False,
    causal_query_seq_attn: bool = False,
    prefill: bool = False,
    k_cache: np.ndarray | None = None,
    v_cache: np.ndarray | None = None,
    cu_seqlens_kv=None,
    total_context_len: int = 0,
    context_batch_size: int = 1,
    context_index=None,
):
    """Gradients of :func:`mlm_attention_packed` (same arguments, plus the upstream
    gradient ``dout`` [B, H, N, D]; its padding rows are ignored).  Returns float64
    (dq, dk, dv, dk_cache, dv_cache) shaped like q, k, v, k_cache, v_cache; dv is None for
    MLA (V is K: both gradients land in dk, head 0) and the cache gradients are None
    without a cache.  The reference has no backward (its roadmap lists one,
    README.md:26-28): this differentiates the forward restated above, key set by key set.
    """
    B, H, N, D = q.shape
    dq = np.zeros(q.shape, dtype=np.float64)
    dk = np.zeros(k.shape, dtype=np.float64)
    dv = None if is_mla else np.zeros(v.shape, dtype=np.float64)
    dkc = None if k_cache is None else np.zeros(k_cache.shape, dtype=np.float64)
    dvc = None if (v_cache is None or is_mla) else np.zeros(v_cache.shape, dtype=np.float64)
    cu_kv = None if cu_seqlens_kv is None else np.asarray(cu_seqlens_kv, dtype=np.int64)
    for b in range(B):
        Lq = int(lengths[b])
        if Lq == 0:
            continue
        rows = packed_key_rows(b, lengths, causal_query_seq_attn)
        sb = np.array([r[0] for r in rows], dtype=np.int64)
        pb = np.array([r[1] for r in rows], dtype=np.int64)
        c0 = c1 = 0
        if not prefill and cu_kv is not None:
            cb = int(context_index[b]) if context_index is not None else (b if context_batch_size > 1 else 0)
            c0, c1 = int(cu_kv[cb]), int(cu_kv[cb + 1])
        nc = c1 - c0
        for h in range(H):
            kh = 0 if is_mla else h
            K_main = k[sb, kh, pb]
            V_main = K_main if is_mla else v[sb, h, pb]
            off = 0 if is_mla else h * total_context_len
            if nc > 0:
                K_ctx = k_cache[off + c0 : off + c1]
                V_ctx = K_ctx if is_mla else v_cache[off + c0 : off + c1]
                K_all = np.concatenate([K_ctx, K_main])
                V_all = np.concatenate([V_ctx, V_main])
            else:
                K_all, V_all = K_main, V_main
            g_q, g_K, g_V = attend_backward(q[b, h, :Lq], K_all, V_all, scale, dout[b, h, :Lq])
            dq[b, h, :Lq] += g_q
            if is_mla:  # V is K
                g_K = g_K + g_V
            if nc > 0:
                dkc[off + c0 : off + c1] += g_K[:nc]
                if not is_mla:
                    dvc[off + c0 : off + c1] += g_V[:nc]
            np.add.at(dk, (sb, kh, pb), g_K[nc:])
            if not is_mla:
                np.add.at(dv, (sb, h, pb), g_V[nc:])
    return dq, dk, dv, dkc, dvc


def mlm_attention_dense_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    dout: np.ndarray,
    scale: float,
    *,
    is_mla: bool = False,
    prefill: bool = False,
    k_cache: np.ndarray | None = None,
    v_cache: np.ndarray | None = None,
    context_len: int = 0,
    context_batch_size: int = 1,
    context_index=None,
):
    """Gradients of :func:`mlm_attention_dense`: (dq, dk, dv, dk_cache, dv_cache) in
    float64, dv None for MLA (V = K per head: both land in dk), cache gradients None
    without a cache.  No reference counterpart (roadmap, README.md:26-28)."""
    B, H, N, D = q.shape
    dq = np.zeros(q.shape, dtype=np.float64)
    dk = np.zeros(k.shape, dtype=np.float64)
    dv = None if is_mla else np.zeros(v.shape, dtype=np.float64)
    dkc = None if k_cache is None else np.zeros(k_cache.shape, dtype=np.float64)
    dvc = None if (v_cache is None or is_mla) else np.zeros(v_cache.shape, dtype=np.float64)
    for b in range(B):
        cb = int(context_index[b]) if context_index is not None else (b if context_batch_size > 1 else 0)
        for h in range(H):
            K_main = k[b, h]
            V_main = K_main if is_mla else v[b, h]
            nc = context_len if (not prefill and context_len > 0) else 0
            if nc:
                start = cb * context_len if is_mla else (cb * H + h) * context_len
                K_ctx = k_cache[start : start + nc]
                V_ctx = K_ctx if is_mla else v_cache[start : start + nc]
                K_all = np.concatenate([K_ctx, K_main])
                V_all = np.concatenate([V_ctx, V_main])
            else:
                K_all, V_all = K_main, V_main
            g_q, g_K, g_V = attend_backward(q[b, h], K_all, V_all, scale, dout[b, h])
            dq[b, h] += g_q
            if is_mla:
                g_K = g_K + g_V
            if nc:
                dkc[start : start + nc] += g_K[:nc]
                if not is_mla:
                    dvc[start : start + nc] += g_V[:nc]
            dk[b, h] += g_K[nc:]
            if not is_mla:
                dv[b, h] += g_V[nc:]
    return dq, dk, dv, dkc, dvc


def mlm_attention_dense(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    scale: float,
    *,
    is_mla: bool = False,
    prefill: bool = False,
    k_cache: np.ndarray | None = None,
    v_cache: np.ndarray | None = None,
    context_len: int = 0,
    context_batch_size: int = 1,
    context_index=None,
) -> np.ndarray:
    """Dense-path attention q/k/v [B, H, N, D] -> [B, H, N, D] (float64).

    Every query of (b, h) attends to [context || k[b, h, :N]].  Context rows (skipped
    when ``prefill``): MLA ``cb*context_len + [0, context_len)``; otherwise
    ``(cb*H + h)*context_len + [0, context_len)``, cb = b if context_batch_size > 1
    else 0 (mlm_kernel_impl.py:132-141), or ``context_index[b]`` when given (the
    extension above).  MLA keeps per-head main keys and V = K.
    """
    return _mlm_dense(q, k, v, scale, is_mla, prefill, k_cache, v_cache, context_len, context_batch_size,
                      context_index, attend)


def mlm_row_lse2_dense(q, k, scale, *, is_mla=False, prefill=False, k_cache=None, context_len=0,
                       context_batch_size=1, context_index=None) -> np.ndarray:
    """row_lse2 of every query row over the key set of mlm_attention_dense: [B, H, N]."""
    def lse(qq, K, V, sc):
        return row_lse2(qq, K, sc)[:, None]

    return _mlm_dense(q, k, k, scale, is_mla, prefill, k_cache, k_cache, context_len, context_batch_size,
                      context_index, lse)[..., 0]


def _mlm_dense(q, k, v, scale, is_mla, prefill, k_cache, v_cache, context_len, context_batch_size, context_index,
               fn):
    """fn(q rows, K_all, V_all, scale) -> [N, W] over each (sequence, head)'s key set."""
    B, H, N, D = q.shape
    out = None
    for b in range(B):
        cb = int(context_index[b]) if context_index is not None else (b if context_batch_size > 1 else 0)
        for h in range(H):
            K_main = k[b, h]
            V_main = K_main if is_mla else v[b, h]
            if not prefill and context_len > 0:
                start = cb * context_len if is_mla else (cb * H + h) * context_len
                K_ctx = k_cache[start : start + context_len]
                V_ctx = K_ctx if is_mla else v_cache[start : start + context_len]
                K_all = np.concatenate([K_ctx, K_main])
                V_all = np.concatenate([V_ctx, V_main])
            else:
                K_all, V_all = K_main, V_main
            r = fn(q[b, h], K_all, V_all, scale)
            if out is None:
                out = np.zeros((B, H, N, r.shape[1]), dtype=np.float64)
            out[b, h] = r
    return np.zeros((B, H, N, D), dtype=np.float64) if out is None else out


def effective_flops(lengths_q, lengths_ctx, num_heads: int, head_dim: int, *, causal_query_seq_attn=False, prefill=False) -> float:
    """4 * H * D * sum_b Lq_b * (Lctx_b + Lmain_b), padding excluded; Lmain_b = Lq_b, or
    cu_q[b+1] with causal_query_seq_attn; Lctx_b = 0 with prefill
    (src/benchmark/common.py:39-57 counts Lmain_b = Lq_b)."""
    lq = np.asarray(lengths_q, dtype=np.float64)
    lc = np.zeros_like(lq) if prefill else np.broadcast_to(np.asarray(lengths_ctx, dtype=np.float64), lq.shape)
    lm = np.cumsum(lq) if causal_query_seq_attn else lq
    return float(4.0 * num_heads * head_dim * np.sum(lq * (lc + lm)))
