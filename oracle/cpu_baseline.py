"""CPU baseline: the reference benchmark's two CPU-runnable attention paths, restated and
timed on the host's CPU cores in fp32 -- a reported baseline, not a checker, and test /
bench infrastructure only.

* "sdpa": per sequence b, K = [context rows of b || main keys of b] and one
  torch.nn.functional.scaled_dot_product_attention call over all heads
  (src/benchmark/standard_kernel/utils.py:410-461 packed, :464-517 dense).
* "eager": per (sequence b, head h), logits = q_bh K^T * scale, softmax, then P V with
  plain torch matmuls (utils.py:365-407 packed, :520-567 dense).

Main keys follow the kernel semantics (MLA: head 0 of k shared by all heads, V = K;
causal_query_seq_attn: sequences 0..b).  A bounded prefix of the workload's sequences
is timed so the run stays within `budget_s` seconds.
"""

from __future__ import annotations

import time

import torch
import torch.nn.functional as F


def _sequence_inputs(case, b: int):
    """fp32 CPU tensors (q [H, Lq, D], K [H|1, M, D], V) for sequence b of a bench Case."""
    t = case.tensors
    H = case.H
    Lq = case.lengths_q[b]
    q = t["q"][b, :, :Lq].float().cpu()
    seqs = range(b + 1) if case.causal else (b,)
    if case.cfg in (1, 2):  # dense
        K_main = t["k"][b].float().cpu()
        V_main = t["v"][b].float().cpu()
    elif case.is_mla:
        K_main = torch.cat([t["k"][s, :1, : case.lengths_q[s]] for s in seqs], dim=1).float().cpu()
        V_main = K_main
    else:
        K_main = torch.cat([t["k"][s, :, : case.lengths_q[s]] for s in seqs], dim=1).float().cpu()
        V_main = torch.cat([t["v"][s, :, : case.lengths_q[s]] for s in seqs], dim=1).float().cpu()
    if case.prefill:
        return q, K_main, V_main
    if case.cfg == 2:
        C = case.config["context"]
        kc = t["k0"][0].float().cpu()
        vc = t["v0"][0].float().cpu()
    elif case.cfg == 1:
        return q, K_main, V_main
    else:
        cb = b if t["cbs"] > 1 else 0
        cu = t["cu_kv"]
        c0, c1 = int(cu[cb]), int(cu[cb + 1])
        Tc = t["Tc"]
        if case.is_mla:
            kc = t["k_cache"][c0:c1].float().cpu()[None]
            vc = kc
        else:
            kc = t["k_cache"].view(H, Tc, -1)[:, c0:c1].float().cpu()
            vc = t["v_cache"].view(H, Tc, -1)[:, c0:c1].float().cpu()
    K = torch.cat([kc, K_main], dim=1)
    V = K if case.is_mla else torch.cat([vc, V_main], dim=1)
    return q, K, V


def _flops(case, b: int) -> float:
    lq = case.lengths_q[b]
    main = sum(case.lengths_q[: b + 1]) if case.causal else lq
    ctx = 0 if case.prefill else case.lengths_ctx[b]
    return 4.0 * case.H * case.D * lq * (ctx + main)


def _sdpa(q, K, V, scale):
    """One sequence, all heads: utils.py:410-461."""
    H = q.shape[0]
    return F.scaled_dot_product_attention(q[None], K.expand(H, -1, -1)[None], V.expand(H, -1, -1)[None],
                                          scale=scale)[0]


def _eager(q, K, V, scale):
    """One sequence, head by head: logits, softmax, P V (utils.py:365-407)."""
    out = torch.empty_like(q)
    for h in range(q.shape[0]):
        kh = K[0 if K.shape[0] == 1 else h]
        vh = V[0 if V.shape[0] == 1 else h]
        logits = torch.matmul(q[h], kh.transpose(0, 1)) * scale
        out[h] = torch.matmul(torch.softmax(logits, dim=-1), vh)
    return out


PATHS = {"sdpa": (_sdpa, "fp32 per-sequence torch SDPA (reference benchmark path, utils.py:410-517)"),
         "eager": (_eager, "fp32 per-(sequence, head) torch matmul + softmax (reference eager path, "
                   "utils.py:365-407, 520-567)")}


def time_case(case, budget_s: float = 20.0, min_s: float = 5.0, path: str = "sdpa") -> dict:
    """Time one CPU path over the workload's sequences in order until `budget_s` seconds
    of attention time (a bounded prefix when the workload is larger).  When one whole pass
    takes less than `min_s`, whole passes repeat until `min_s` and the median pass is
    reported."""
    fn, what = PATHS[path]
    scale = case.tensors["scale"]
    n_seq = len(case.lengths_q)
    # warm-up on the first sequence
    q, K, V = _sequence_inputs(case, 0)
    fn(q, K, V, scale)
    inputs = []
    elapsed, flops = 0.0, 0.0
    for b in range(n_seq):
        q, K, V = _sequence_inputs(case, b)
        inputs.append((q, K, V))
        t0 = time.perf_counter()
        fn(q, K, V, scale)
        elapsed += time.perf_counter() - t0
        flops += _flops(case, b)
        if elapsed > budget_s:
            break
    done = len(inputs)
    passes = [elapsed]
    while done == n_seq and sum(passes) < min_s and len(passes) < 50:
        t0 = time.perf_counter()
        for q, K, V in inputs:
            fn(q, K, V, scale)
        passes.append(time.perf_counter() - t0)
    t_pass = sorted(passes)[len(passes) // 2]
    total = sum(_flops(case, b) for b in range(n_seq))
    return {
        "value": round(flops / t_pass / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "path": path,
        "sample": f"first {done} of {n_seq} sequences, all {case.H} heads, {what}; {flops / 1e9:.2f} of "
        f"{total / 1e9:.2f} GFLOP per pass, median of {len(passes)} passes ({sum(passes):.2f} s)",
        "ms_per_step_extrapolated": round(t_pass / flops * total * 1e3, 3),
    }
