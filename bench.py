#!/usr/bin/env python
"""Benchmark of the fused MLM attention path (flash-mlm API on MI355X / gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]

A step is one pass of the hot path over one synthetic batch with inputs resident in
HBM: for the default workload (packed varlen fp16 with a
full-batch cached context) that is flash_attn_mlm_compressed + unpack_from_kernel
(pack metadata is built once and memoised, as in the reference's own benchmark).
Prints one JSON line: effective attention TFLOP/s (padding excluded, formula
4*H*D*sum_b Lq_b*(Lctx_b + Lmain_b)), ms per step (the K timed steps run after the
kernel-timing loops, at settled clocks; the same steps are then run once more with HIP
events around each, "step_device_ms"), the host time of one API call, the
attention kernel's roofline fraction against the MI355X dense fp16/bf16 MFMA peak
(kernel time: mean of HIP-event timings on its launch stream over back-to-back launches;
also with L2/MALL flushed before each launch), the kernel's HBM bytes per launch from two
rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE) run as child processes before this
process touches the GPU, each scaled by the counter's reading for a 256 MiB copy, the
HBM rate and counter-measured bytes of the pack, unpack and KV-append kernels on the same
tensors ("hbm_kernels"), and the reference's per-sequence PyTorch SDPA path and eager
per-(sequence, head) path timed on this host's CPU cores as a reported baseline.

The configs (BASELINE.json "configs") are built by `make_case`, which the GPU tests
reuse for parity checks.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "flash-mlm_amd"))

import torch  # noqa: E402

METRIC = "effective attention TFLOP/s + ms/call, packed varlen w/ context, 1 MI355X"
MFMA_PEAK_TFLOPS = {torch.bfloat16: 2516.6, torch.float16: 2516.6, torch.float32: 157.3}
HBM_PEAK_GBS = 8000.0
DEFAULT_CONFIG = 3

DTYPE_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@dataclass
class Case:
    cfg: int
    workload: str
    dtype: torch.dtype
    H: int
    D: int
    lengths_q: list[int]
    lengths_ctx: list[int]  # per query sequence (shared contexts repeated)
    causal: bool
    prefill: bool
    is_mla: bool
    call: Callable[[], torch.Tensor]  # the attention entry point of one step
    attention: Callable[[], None]  # the attention kernel alone (prepared ABI call)
    tensors: dict = field(default_factory=dict)  # inputs, kept for checks
    config: dict = field(default_factory=dict)
    post: Callable[[torch.Tensor], torch.Tensor] | None = None  # the rest of the step

    def step(self) -> torch.Tensor:
        """One pass of the hot path: the attention call, then (packed paths) the unpack."""
        out = self.call()
        return self.post(out) if self.post is not None else out

    @property
    def flops(self) -> float:
        lq = self.lengths_q
        main = list(_cumsum(lq)[1:]) if self.causal else lq
        ctx = [0] * len(lq) if self.prefill else self.lengths_ctx
        return 4.0 * self.H * self.D * sum(a * (c + m) for a, c, m in zip(lq, ctx, main))

    @property
    def flops_reference_formula(self) -> float:
        """src/benchmark/common.py:39-57 (Lmain = Lq even under causal_query_seq_attn)."""
        ctx = [0] * len(self.lengths_q) if self.prefill else self.lengths_ctx
        return 4.0 * self.H * self.D * sum(a * (c + a) for a, c in zip(self.lengths_q, ctx))

    @property
    def attention_bytes(self) -> float:
        """Algorithmic HBM bytes of the attention kernel: q and o once, main K/V once
        per head (MLA: one latent), each context row once per head it serves."""
        esz = torch.finfo(self.dtype).bits // 8
        T = sum(self.lengths_q)
        hk = 1 if self.is_mla else self.H
        m = 1 if self.is_mla else 2
        ctx_rows = 0 if self.prefill else self.config.get("unique_ctx_tokens", 0)
        return esz * self.D * (2 * self.H * T + m * hk * T + m * hk * ctx_rows)


def _cumsum(xs):
    out = [0]
    for x in xs:
        out.append(out[-1] + x)
    return out


def _randn(shape, gen, device, dtype, std=1.0):
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(dtype)


def _prefill_paged(cache, k_cache, v_cache, cu_kv, *, hk: int, H: int, D: int, mla: bool, seed: int,
                   shuffle: bool = True) -> None:
    """Store a contiguous head-major context [hk*Tc, D] as a paged one: every context batch's
    rows in 64-row pages [hk, P, 64, D], pages placed in a seeded random order (or in key
    order with shuffle=False)."""
    page = 64
    lens = (cu_kv[1:] - cu_kv[:-1]).tolist()
    need = [(n + page - 1) // page for n in lens]
    P = sum(need)
    order = torch.randperm(P, generator=torch.Generator().manual_seed(seed)) if shuffle else torch.arange(P)
    bt = torch.zeros((len(lens), max(need + [1])), dtype=torch.int32)
    src, dst, k0 = [], [], 0
    for c, (n, npg) in enumerate(zip(lens, need)):
        bt[c, :npg] = order[k0 : k0 + npg]
        j = torch.arange(n)
        src.append(int(cu_kv[c]) + j)
        dst.append(bt[c, j // page].long() * page + j % page)
        k0 += npg
    src_i = torch.cat(src).to(k_cache.device)
    dst_i = torch.cat(dst).to(k_cache.device)
    Tc = int(cu_kv[-1])

    def pool_of(x):
        pool = torch.zeros((hk, P * page, D), dtype=x.dtype, device=x.device)
        pool[:, dst_i] = x.view(hk, Tc, D)[:, src_i]
        return pool.view(hk, P, page, D)

    cache.prefill_paged_kv_cache(0, k_pages=pool_of(k_cache), v_pages=None if mla else pool_of(v_cache),
                                 block_table=bt.to(k_cache.device), context_lens=torch.tensor(lens, dtype=torch.int32),
                                 is_mla=mla, num_heads=H, head_dim=D)


def make_case(cfg: int, device: torch.device, *, variant: str = "", batch: int = 0,
              query_lens: tuple[int, int] | None = None, head_dim: int = 0) -> Case:
    """Build BASELINE config `cfg` (1..5; config 5 variant "prefill" is 5b, variant
    "paged" / "paged_seq" store configs 3-5's context as a paged KV pool, pages shuffled /
    in key order; for configs 3 and 4, `batch`, `query_lens` = (lo, hi) and `head_dim`
    replace the sequence count, the per-sequence query length range (N: the range's top
    rounded up to 64) and the head dim: shapes for the tile-configuration sweep, not
    BASELINE configs) with
    seeded synthetic inputs: lengths from a CPU generator seeded 1000+cfg (query
    lengths first, then context lengths), tensors from a device generator with the
    same seed, fp32 normal * std cast to the config dtype."""
    import flash_mlm as fm

    seed = 1000 + cfg
    gcpu = torch.Generator().manual_seed(seed)
    gdev = torch.Generator(device=device).manual_seed(seed)

    if cfg == 1:
        B, H, N, D = 2, 8, 128, 64
        dt = torch.float32
        q, k, v = (_randn((B, H, N, D), gdev, device, dt) for _ in range(3))
        scale = 1.0 / math.sqrt(D)
        out_plan = fm.host.host._dense_impl(q, k, v, scale, None, None, False, None, False, run=False)
        return Case(
            cfg, "cfg1 dense flash_attn_mlm fp32 [2,8,128,64], no cache", dt, H, D, [N] * B, [0] * B,
            False, False, False,
            call=lambda: fm.flash_attn_mlm(q, k, v, scale),
            attention=out_plan[1],
            tensors=dict(q=q, k=k, v=v, scale=scale),
            config=dict(B=B, H=H, N=N, D=D, seed=seed),
        )

    if cfg == 2:
        B, H, N, D, C = 8, 16, 512, 64, 2048
        dt = torch.bfloat16
        scale = 1.0 / math.sqrt(D)
        q0, k0, v0 = (_randn((1, H, C, D), gdev, device, dt) for _ in range(3))
        q, k, v = (_randn((B, H, N, D), gdev, device, dt) for _ in range(3))
        cache = fm.InferenceCache()
        fm.flash_attn_mlm(q0, k0, v0, scale, inference_cache=cache, layer_id=0, prefill=True)
        plan = fm.host.host._dense_impl(q, k, v, scale, cache, 0, False, None, False, run=False)[1]
        return Case(
            cfg, "cfg2 dense flash_attn_mlm bf16 [8,16,512,64] + shared prefilled ctx 2048", dt, H, D,
            [N] * B, [C] * B, False, False, False,
            call=lambda: fm.flash_attn_mlm(q, k, v, scale, inference_cache=cache, layer_id=0),
            attention=plan,
            tensors=dict(q=q, k=k, v=v, k0=k0, v0=v0, scale=scale, cache=cache),
            config=dict(B=B, H=H, N=N, D=D, context=C, seed=seed, unique_ctx_tokens=C),
        )

    if cfg in (3, 4, 5):
        if cfg == 3:
            B, H, N, D, bn = 32, 16, 1024, 128, 64
            dt, std = torch.float16, 1.0
            lq = torch.randint(256, 1024 + 1, (B,), generator=gcpu)
            lc = torch.randint(512, 2048 + 1, (B,), generator=gcpu)
            cbs, mla, causal = B, False, False
        elif cfg == 4:
            B, H, N, D, bn = 16, 12, 512, 64, 64
            dt, std = torch.bfloat16, 1.0
            lq = torch.randint(64, 512 + 1, (B,), generator=gcpu)
            lc = torch.tensor([4096])
            cbs, mla, causal = 1, False, True
        else:
            B, H, N, D, bn = 8, 64, 2048, 512, 64
            dt, std = torch.bfloat16, 0.5
            lq = torch.randint(512, 2048 + 1, (B,), generator=gcpu)
            lc = torch.full((B,), 8192)
            cbs, mla, causal = B, True, False
        if (batch or query_lens or head_dim) and cfg in (3, 4):
            B, D = batch or B, head_dim or D
            lo, hi = query_lens or (int(lq.min()), int(lq.max()))
            N = (hi + 63) // 64 * 64
            lq = torch.randint(lo, hi + 1, (B,), generator=gcpu)
            if cfg == 3:
                lc = torch.randint(512, 2048 + 1, (B,), generator=gcpu)
                cbs = B
        elif batch or query_lens or head_dim:
            raise ValueError("--batch / --query-lens / --head-dim apply to configs 3 and 4 only")
        prefill = variant == "prefill"
        scale = 1.0 / math.sqrt(D)
        q = _randn((B, H, N, D), gdev, device, dt, std)
        k = _randn((B, H, N, D), gdev, device, dt, std)
        v = k if mla else _randn((B, H, N, D), gdev, device, dt, std)
        cu_kv = torch.zeros(lc.numel() + 1, dtype=torch.int32)
        cu_kv[1:] = torch.cumsum(lc, 0)
        Tc = int(cu_kv[-1])
        hk = 1 if mla else H
        k_cache = _randn((hk * Tc, D), gdev, device, dt, std)
        v_cache = None if mla else _randn((hk * Tc, D), gdev, device, dt, std)
        cache = fm.InferenceCache()
        if variant in ("paged", "paged_seq"):  # the same context rows in a 64-row page pool
            _prefill_paged(cache, k_cache, v_cache, cu_kv, hk=hk, H=H, D=D, mla=mla, seed=seed,
                           shuffle=variant == "paged")
        else:
            cache.prefill_kv_cache(
                0, k_cache=k_cache, v_cache=v_cache, total_context_len=Tc, cu_seqlens_kv=cu_kv.to(device),
                context_batch_size=cbs, is_mla=mla, num_heads=H, head_dim=D,
            )
        meta = cache.packing.get_pack_metadata(lq.to(device=device, dtype=torch.int32), N=N, block_n=bn)
        kw = dict(is_mla=mla, block_n=bn, causal_query_seq_attn=causal)

        def call():
            return fm.flash_attn_mlm_compressed(q, k, v, H, meta, scale, cache, 0, prefill=prefill, **kw)

        # the attention launch alone; prefill replaces the layer entry, so plan it on a copy
        plan_cache = cache
        if prefill:
            plan_cache = fm.InferenceCache()
            plan_cache._layer_kv = dict(cache._layer_kv)
        plan = fm.host.host._compressed_impl(
            q, k, v, H, meta, scale, plan_cache, 0, mla, None, 64, bn, False, prefill, causal, run=False
        )[1]
        lengths_ctx = [int(lc[0])] * B if cbs == 1 else [int(x) for x in lc]
        names = {
            3: "cfg3 packed varlen fp16 B=32 H=16 N=1024 D=128, per-seq cached ctx U[512,2048]",
            4: "cfg4 packed causal_query_seq_attn bf16 B=16 H=12 D=64, shared ctx 4096",
            5: "cfg5 MLA bf16 B=8 64 heads : 1 latent D=512, cached latent ctx 8192/seq",
        }
        shape = ""
        if batch or query_lens or head_dim:
            shape = f" [sweep shape: B={B}, D={D}, query lengths U[{int(lq.min())}..{int(lq.max())}], N={N}]"
        return Case(
            cfg, names[cfg] + shape + (" (prefill=True)" if prefill else "") + (f" ({variant} KV context)" if variant.startswith("paged") else ""),
            dt, H, D,
            [int(x) for x in lq], lengths_ctx, causal, prefill, mla,
            call=call,
            post=lambda out: fm.unpack_from_kernel(out, meta, H),
            attention=plan,
            tensors=dict(q=q, k=k, v=v, k_cache=k_cache, v_cache=v_cache, cu_kv=cu_kv, meta=meta,
                         scale=scale, cache=cache, cbs=cbs, Tc=Tc),
            config=dict(B=B, H=H, N=N, D=D, block_n=bn, seed=seed, total_q_tokens=int(lq.sum()),
                        total_ctx_tokens=Tc, unique_ctx_tokens=Tc, context_batch_size=cbs),
        )
    raise ValueError(f"unknown config {cfg}")


def _median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


def _time_steps(case: "Case", steps: int, warmup: int) -> tuple[float, float, float]:
    """(ms per step, median host us of the attention API call, median host us of a whole
    step): K steps back to back between two device synchronisations.  The host times are
    what the Python API costs the caller per call (the launch memo's lookup, the output
    allocation, the launch); the launches are asynchronous, so they overlap the GPU's
    work."""
    for _ in range(warmup):
        case.step()
    torch.cuda.synchronize()
    call_us, step_us = [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        a = time.perf_counter()
        out = case.call()
        b = time.perf_counter()
        if case.post is not None:
            case.post(out)
        call_us.append((b - a) * 1e6)
        step_us.append((time.perf_counter() - a) * 1e6)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return ms, _median(call_us), _median(step_us)


def _step_events(case: "Case", steps: int) -> dict:
    """Device time of each of `steps` steps run as the timed ones are (after them, the
    clocks already settled), from HIP events on the current stream (the one the steps
    launch on) around each step: mean, median, first and maximum in ms."""
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for e0, e1 in events:
        e0.record()
        case.step()
        e1.record()
    torch.cuda.synchronize()
    t = [e0.elapsed_time(e1) for e0, e1 in events]
    return {"mean": round(sum(t) / len(t), 5), "median": round(_median(t), 5), "first": round(t[0], 5),
            "max": round(max(t), 5)}


def _launch_stream(attention):
    return torch.cuda.ExternalStream(attention.stream) if attention.stream else torch.cuda.current_stream()


def _kernel_device_ms(attention, reps: int) -> tuple[float, float]:
    """Device time of the prepared attention launch (the kernel, plus the split merge where
    there is one): `reps` launches back to back on the kernel's launch stream with HIP
    events recorded on that stream around each.  The host enqueues a launch in well under
    a kernel's duration, so the queue stays full and no host time falls inside an event
    pair.  Returns (mean, median) in ms."""
    stream = _launch_stream(attention)
    for _ in range(5):
        attention()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for e0, e1 in events:
            e0.record(stream)
            attention()
            e1.record(stream)
    torch.cuda.synchronize()
    times = [e0.elapsed_time(e1) for e0, e1 in events]
    return sum(times) / len(times), _median(times)


FLUSH_BYTES = 512 << 20  # > the 256 MB MALL (and the 4 MB L2s)
_flush_buf = None


def _flush_caches() -> None:
    """Evict L2 and MALL before a cold-cache launch by reading FLUSH_BYTES: the caches then
    hold clean lines.  (Writing the buffer instead leaves up to 256 MB of dirty lines whose
    write-back lands inside the next timed launch: the copy kernels measured 20-30% slower
    after a write flush than after a read flush.)"""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    _flush_buf.sum()


def _kernel_ms(attention, reps: int) -> tuple[float, float]:
    """Attention-kernel duration from HIP events recorded on the kernel's launch stream
    around each of `reps` prepared launches, with L2/MALL flushed before every launch by
    reading a 512 MiB buffer.  Returns (median, mean) in ms."""
    stream = _launch_stream(attention)
    for _ in range(3):
        attention()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    with torch.cuda.stream(stream):
        for e0, e1 in events:
            _flush_caches()
            e0.record(stream)
            attention()
            e1.record(stream)
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) for e0, e1 in events)
    return times[len(times) // 2], sum(times) / len(times)


COPY_KIB = (256 << 20) / 1024  # the --profile driver's calibration copy


def _kernel_class(name: str) -> str | None:
    """Which measured kernel a rocprofv3 dispatch belongs to (by demangled name)."""
    if "copyBuffer" in name:
        return "copy"
    if "fmlm::unpack_kernel" in name:
        return "unpack"
    if "fmlm::pack_kernel" in name:
        return "pack"
    if "fmlm::kv_append_kernel" in name:
        return "kv_append"
    if "bwd" in name:
        return "bwd"
    if "attn_" in name and "schedule" not in name:
        return "attn"
    return None


# shape overrides (--batch / --query-lens) handed to the counter passes' child processes
_SHAPE_ARGS: list[str] = []


def _counter_pass(counter: str, cfg: int, variant: str, launches: int, timeout_s: float, tile: int = 0) -> dict:
    """One `rocprofv3 --pmc <counter>` run of this script's --profile driver in a child
    process.  Returns {"attn": mean KiB per attention dispatch, "copy": KiB of the
    256 MiB calibration copy, and for each copy kernel of the path ("pack", "unpack",
    "kv_append") the KiB of its one profiled call, summed over its dispatches}."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        raise RuntimeError("rocprofv3 not on PATH")
    out = Path(tempfile.mkdtemp(prefix="fmlm_pmc_", dir="/tmp"))
    cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", str(out), "-o", "pmc", "--",
           sys.executable, str(REPO / "bench.py"), "--config", str(cfg), "--profile",
           "--steps", str(launches)]
    if variant:
        cmd += ["--variant", variant]
    if tile:
        cmd += ["--tile-config", str(tile)]
    cmd += _SHAPE_ARGS
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        # rocprofv3 may exit non-zero after writing complete results; the CSV decides
        subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, stdout=subprocess.DEVNULL,
                       stderr=subprocess.DEVNULL, check=False)
        files = list(out.rglob("*counter_collection.csv"))
        if not files:
            raise RuntimeError(f"rocprofv3 --pmc {counter} wrote no counter file")
        rows: list[tuple[int, str, float]] = []  # (dispatch id, kernel class, KiB)
        for f in files:
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    if row["Counter_Name"] != counter:
                        continue
                    kind = _kernel_class(row["Kernel_Name"])
                    if kind is not None:
                        rows.append((int(row["Dispatch_Id"]), kind, float(row["Counter_Value"])))
        rows.sort()
        attn = [v for _, kind, v in rows if kind == "attn"]
        copies = [v for _, kind, v in rows if kind == "copy"]
        if len(attn) < launches or not copies:
            raise RuntimeError(f"rocprofv3 --pmc {counter}: {len(attn)} attention dispatches, "
                               f"{len(copies)} copies")
        res = {"attn": sum(attn[-launches:]) / launches, "copy": max(copies)}
        # the copy kernels' profiled calls come after the last attention launch; earlier
        # dispatches (the pack the case's setup runs for causal_query_seq_attn) are not them
        last_attn = max(i for i, kind, _ in rows if kind == "attn")
        for kind in ("pack", "unpack", "kv_append"):
            vals = [v for i, k, v in rows if k == kind and i > last_attn]
            if vals:
                res[kind] = sum(vals)
        return res
    finally:
        shutil.rmtree(out, ignore_errors=True)


def hbm_traffic(cfg: int, variant: str, launches: int = 3, timeout_s: float = 120.0, tile: int = 0) -> dict:
    """HBM bytes per attention launch from two counter passes (FETCH_SIZE, WRITE_SIZE),
    each scaled by what the same counter reads for a copy of known size (256 MiB read +
    256 MiB written) in the same run."""
    f = _counter_pass("FETCH_SIZE", cfg, variant, launches, timeout_s, tile)
    w = _counter_pass("WRITE_SIZE", cfg, variant, launches, timeout_s, tile)
    ff, fw = COPY_KIB / f["copy"], COPY_KIB / w["copy"]
    res = {
        "bytes": 1024.0 * (f["attn"] * ff + w["attn"] * fw),
        "fetch_kib": f["attn"], "write_kib": w["attn"],
        "fetch_scale": round(ff, 4), "write_scale": round(fw, 4),
    }
    for kind in ("pack", "unpack", "kv_append"):
        if kind in f and kind in w:
            res[kind] = {"bytes": 1024.0 * (f[kind] * ff + w[kind] * fw), "fetch_kib": f[kind],
                         "write_kib": w[kind]}
    return res


def _event_ms(fn, reps: int) -> float:
    """Median duration of fn() from HIP events on the current stream, L2/MALL flushed
    (512 MiB read) before each call."""
    stream = torch.cuda.current_stream()
    for _ in range(2):
        fn()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in events:
        _flush_caches()
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) for e0, e1 in events)
    return times[len(times) // 2]


def copy_kernel_calls(case: Case) -> dict:
    """The path's copy kernels on this workload's tensors, as {name: (call, algorithmic
    bytes, note)}: unpack_from_kernel (read H*T*D, write B*H*N*D),
    pack_and_pad_main_tensors_for_mlm_compressed (per tensor: read heads*T*D, write
    heads*T_pad*D; MLA packs q and one latent head) and the KV append of this step's rows
    to the cached context (InferenceCache.append_kv_cache: reads and writes every row of
    the merged entry once; one fmlm_kv_append launch).  Each call is independent of the
    others' results."""
    import flash_mlm as fm
    from flash_mlm.host import host_utils as hu

    t = case.tensors
    if "meta" not in t:
        return {}
    meta = t["meta"]
    esz = torch.finfo(case.dtype).bits // 8
    B, H, N, D = (int(x) for x in t["q"].shape)
    T = int(meta.total_tokens)
    calls = {}

    packed = torch.randn((H * T, D), device="cuda").to(case.dtype)
    calls["unpack"] = (lambda: fm.unpack_from_kernel(packed, meta, H), esz * D * (H * T + B * H * N), "")

    pc = fm.PackingCache()
    bn = int(case.config.get("block_n", 64))
    pack = lambda: hu.pack_and_pad_main_tensors_for_mlm_compressed(  # noqa: E731
        t["q"], t["k"], t["v"], q_meta=meta, num_heads=H, is_mla=case.is_mla, block_m=64, block_n=bn,
        packing_cache=pc)
    T_pad = hu._compute_total_q_len_padded(T, meta.host_cu_seqlens(), 64, bn)
    heads = H + (1 if case.is_mla else 2 * H)
    calls["pack"] = (pack, esz * D * heads * (T + T_pad), "q + latent head" if case.is_mla else "q, k, v")

    ent = t["cache"].get_kv_cache(0, is_mla=case.is_mla, num_heads=H, head_dim=D, dtype=case.dtype,
                                  device=t["q"].device) if "cache" in t else None
    if ent is not None and ent.cu_seqlens_kv is not None and ent.block_table is None:
        h_kv = 1 if case.is_mla else H
        n_batch = int(ent.cu_seqlens_kv.numel()) - 1
        cu_new = meta.cu_seqlens if n_batch == B else torch.tensor([0, T], dtype=torch.int32, device="cuda")
        new_k = torch.randn((h_kv * T, D), device="cuda").to(case.dtype)
        new_v = None if case.is_mla else torch.randn((h_kv * T, D), device="cuda").to(case.dtype)

        def append():  # a cache holding (views of) the layer's entry; append replaces it
            c = fm.InferenceCache()
            c.prefill_kv_cache(0, k_cache=ent.k_cache, v_cache=ent.v_cache, total_context_len=ent.total_context_len,
                               cu_seqlens_kv=ent.cu_seqlens_kv, context_batch_size=ent.context_batch_size,
                               is_mla=case.is_mla, num_heads=H, head_dim=D)
            c.append_kv_cache(0, k_cache=new_k, v_cache=new_v, cu_seqlens_kv=cu_new)

        rows = int(ent.total_context_len) + T
        nbytes = esz * D * h_kv * (1 if case.is_mla else 2) * 2 * rows
        calls["kv_append"] = (append, nbytes, "latent" if case.is_mla else "k, v")
    return calls


def hbm_kernels(case: Case, reps: int = 30, traffic: dict | None = None) -> dict:
    """HBM rate of the path's copy kernels (copy_kernel_calls): algorithmic bytes / median
    HIP-event time with L2/MALL flushed (by a read) before each call, against the 8 TB/s
    HBM peak; with
    `traffic` (hbm_traffic's counter readings) also the measured HBM bytes per call."""
    out = {}
    for name, (fn, nbytes, note) in copy_kernel_calls(case).items():
        ms = _event_ms(fn, reps)
        out[name] = {"ms": round(ms, 5), "bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
                     "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
        if note:
            out[name]["tensors"] = note
        if traffic and name in traffic:
            tb = traffic[name]["bytes"]
            out[name]["traffic"] = round(tb)
            out[name]["traffic_over_algorithmic"] = round(tb / nbytes, 3)
    return out


def _backward_call(case: Case):
    """(fmlm_attn_bwd on this workload's prepared call: a callable, the gradient block and
    the tensors it points to), or None without a prepared call.  Runs the forward once
    first: the backward reads its output."""
    from flash_mlm import _lib
    from flash_mlm.host import host as hh

    plan = case.attention
    if plan is None:
        return None
    # as under autograd: the forward stores the row statistics the backward reads; the
    # backward keeps its own copy of the parameter block (later forward runs reset the field)
    hh._ROW_STATS.on = True
    try:
        plan()
    finally:
        hh._ROW_STATS.on = False
    params, lse = _lib.AttnParams.from_buffer_copy(plan.params), plan.lse
    out = plan.keep[1]
    dout = torch.randn(out.shape, device=out.device).to(out.dtype)
    g, keep = hh._backward_args(plan, out, dout, want_ctx=True)

    def call():
        _lib.check(plan.lib.fmlm_attn_bwd(params, g, plan.stream), "fmlm_attn_bwd")

    return call, g, (keep, out, dout, lse, params)


def backward_kernels(case: Case, reps: int = 20) -> dict | None:
    """fmlm_attn_bwd (the dq kernel, then the dK/dV kernels of the main keys and of the
    context) on this workload's prepared call, gradients of q, k, v and of the cached
    context: median of HIP-event times with L2/MALL flushed before each launch.
    Effective work = 2.5x the forward's FLOPs (the products dP = dO V^T, dV = P^T dO,
    dq = dS K, dK = dS^T q besides S = q K^T), padding excluded; the dK/dV kernel
    computes S and dP again, which is not counted.  The forward stores the row statistics first,
    as under autograd."""
    bc = _backward_call(case)
    if bc is None:
        return None
    call, g, _keep = bc
    ms = _event_ms(call, reps)
    F = 2.5 * case.flops
    peak = MFMA_PEAK_TFLOPS[case.dtype]
    return {"ms": round(ms, 5), "effective_gflop": round(F / 1e9, 4), "tflops": round(F / (ms * 1e-3) / 1e12, 3),
            "frac": round(F / (ms * 1e-3) / 1e12 / peak, 5),
            "grads": ("q, latent k" if case.is_mla else "q, k, v") + (", context" if g.dk_ctx else "")}


def cpu_baseline(case: Case, budget_s: float = 20.0, path: str = "sdpa") -> dict:
    """The reference's per-sequence PyTorch SDPA path, or its eager per-(sequence, head)
    path (oracle/cpu_baseline.py), on this host's CPU cores, fp32, over a bounded prefix
    of the workload's sequences."""
    sys.path.insert(0, str(REPO))
    from oracle import cpu_baseline as cb

    return cb.time_case(case, budget_s=budget_s, path=path)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # 200 steps (~0.1 s at config 3): with 20 the start of the timed region weighs ~15%
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=DEFAULT_CONFIG)
    ap.add_argument("--variant", default="")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--tile-config", type=int, default=0,
                    help="force the attention kernel's tile configuration k (0: the library's choice)")
    ap.add_argument("--batch", type=int, default=0,
                    help="configs 3 and 4: sequence count (tile-configuration sweep shapes)")
    ap.add_argument("--query-lens", default="",
                    help="configs 3 and 4: per-sequence query lengths LO:HI (tile-configuration sweep shapes)")
    ap.add_argument("--head-dim", type=int, default=0,
                    help="configs 3 and 4: head dim (tile-configuration sweep shapes)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure HBM traffic")
    ap.add_argument(
        "--profile",
        action="store_true",
        help="profiling driver for rocprofv3: one 256 MiB device copy (calibrates the HBM byte "
        "counters), --warmup attention launches, then --steps bare attention launches back to back, "
        "one call of each copy kernel and --steps backward launches; prints no JSON line",
    )
    args = ap.parse_args()
    query_lens = tuple(int(x) for x in args.query_lens.split(":")) if args.query_lens else None
    if args.batch:
        _SHAPE_ARGS.extend(["--batch", str(args.batch)])
    if args.query_lens:
        _SHAPE_ARGS.extend(["--query-lens", args.query_lens])
    if args.head_dim:
        _SHAPE_ARGS.extend(["--head-dim", str(args.head_dim)])

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU only: this path has no multi-GPU implementation in this "
            "build (it would shard by head with no exchange); run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)
    # counter passes run as child processes before this process touches the GPU
    traffic, traffic_note = None, None
    if not args.profile and not args.no_traffic:
        try:
            traffic = hbm_traffic(args.config, args.variant, tile=args.tile_config)
            print(f"[bench] HBM traffic per launch: {traffic}", file=sys.stderr, flush=True)
        except Exception as e:  # counters unavailable: report null, say why
            traffic_note = f"counter passes failed: {e}"
            print(f"[bench] {traffic_note}", file=sys.stderr, flush=True)

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.tile_config:
        from flash_mlm.host import host as hh

        hh._TILE_CONFIG = args.tile_config
    case = make_case(args.config, device, variant=args.variant, batch=args.batch, query_lens=query_lens,
                     head_dim=args.head_dim)
    print(f"[bench] {case.workload}: built inputs", file=sys.stderr, flush=True)

    if args.profile:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # 256 MiB read + 256 MiB write
        torch.cuda.synchronize()
        # the backward's arguments (this runs the forward once, before the launches below, so
        # that the copy kernels still follow the last attention launch)
        bc = _backward_call(case)
        for _ in range(args.warmup):  # as the timed bench: the clocks settle first
            case.attention()
        torch.cuda.synchronize()
        for _ in range(args.steps):
            case.attention()
        torch.cuda.synchronize()
        # then one call of each copy kernel of the path
        for name, (fn, _, _) in copy_kernel_calls(case).items():
            fn()
            torch.cuda.synchronize()
        # then --steps backward launches (the counter passes of the backward kernels)
        if bc is not None:
            for _ in range(args.steps):
                bc[0]()
            torch.cuda.synchronize()
        print(f"[bench] profiled {args.steps} attention launches, the copy kernels and {args.steps} backward "
              "launches", file=sys.stderr, flush=True)
        return

    # the kernel-timing loops first: the timed steps then run at settled clocks, whatever
    # the GPU did while this process built its inputs
    kms, kmed = _kernel_device_ms(case.attention, args.kernel_reps)
    print(f"[bench] attention launch on the device: mean {kms:.4f} ms, median {kmed:.4f} ms over "
          f"{args.kernel_reps} back-to-back launches", file=sys.stderr, flush=True)
    fms, fmean = _kernel_ms(case.attention, args.kernel_reps)
    print(f"[bench] attention kernel with cold caches: median {fms:.4f} ms, mean {fmean:.4f} ms over "
          f"{args.kernel_reps} flushed launches", file=sys.stderr, flush=True)
    ms, call_us, step_us = _time_steps(case, args.steps, args.warmup)
    print(f"[bench] timed {args.steps} steps: {ms:.4f} ms/step; host {call_us:.1f} us per attention API call, "
          f"{step_us:.1f} us per step (medians)", file=sys.stderr, flush=True)
    step_ev = _step_events(case, args.steps)
    print(f"[bench] the same steps with HIP events around each: {step_ev}", file=sys.stderr, flush=True)

    F = case.flops
    value = F / (ms * 1e-3) / 1e12
    k_tflops = F / (kms * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS[case.dtype]
    roofline = {
        "bound": "mfma",
        "achieved": round(k_tflops, 3),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(k_tflops / peak, 5),
        "traffic": None if traffic is None else round(traffic["bytes"]),
        "kernel_ms": round(kms, 5),
        "kernel_ms_median": round(kmed, 5),
        "kernel_timing": f"HIP events on the launch stream around each of {args.kernel_reps} back-to-back "
                         "launches of the prepared attention call (the kernel, plus the split merge when key "
                         "ranges are split), queue kept full; mean",
        "kernel_ms_cold": round(fms, 5),
        "kernel_ms_cold_mean": round(fmean, 5),
        "kernel_cold_timing": f"the same kernel launched alone {args.kernel_reps} times, L2/MALL flushed "
                              "(512 MiB read) before each (median)",
        "frac_cold": round(F / (fms * 1e-3) / 1e12 / peak, 5),
        "algorithmic_bytes": case.attention_bytes,
    }
    if traffic is not None:
        roofline["traffic_detail"] = {k: v for k, v in traffic.items() if k != "bytes"}
        roofline["traffic_over_algorithmic"] = round(traffic["bytes"] / case.attention_bytes, 3)
        roofline["hbm_gbs"] = round(traffic["bytes"] / (kms * 1e-3) / 1e9, 1)
    elif traffic_note:
        roofline["traffic_note"] = traffic_note
    hbm = hbm_kernels(case, traffic=traffic)
    if hbm:
        print(f"[bench] copy kernels: {hbm}", file=sys.stderr, flush=True)
    bwd = backward_kernels(case)
    if bwd:
        print(f"[bench] backward: {bwd}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(case)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
        cpu["eager"] = cpu_baseline(case, path="eager", budget_s=10.0)
        print(f"[bench] cpu eager path: {cpu['eager']}", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "host_us_per_call": round(call_us, 2),
        "host_us_per_step": round(step_us, 2),
        "step_device_ms": step_ev,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAMES[case.dtype],
        "data": "synthetic (seeded normal inputs, seeded uniform lengths)",
        "config": {"workload": case.workload, **case.config,
                   "effective_gflop": round(F / 1e9, 4),
                   "reference_formula_gflop": round(case.flops_reference_formula / 1e9, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "hbm_kernels": hbm or None,
        "backward": bwd,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
