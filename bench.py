"""Benchmark of one mixed draft/verify attention layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1] [--no-cpu-baseline]

A step is one pass of the hot path over one batch resident in HBM: the paged
KV append of the batch's new tokens followed by mixed draft/verify attention
(including the split-KV merge). Default workload: BASELINE config 1, the
Qwen3-8B-shape layer (32 q / 8 kv heads, head_dim 128, bf16, 16-token pages),
batch 32 x 32768-token contexts, 16 drafting rows (q_len 1 over 128 selected
pages) and 16 verifying rows (q_len 4, causal, full cache). ``--config 2`` runs
the Qwen3-8B refresh layer (batch 64, contexts U[8192, 32768], full attention
for every single-query row with the per-KV-head key-mean page scores and the
top-128 page selection).

value = algorithmic HBM bytes of the step / step time (GB/s). The roofline
object reports the dominant kernel (mixed attention) alone: its algorithmic
bytes per launch (KV pages read + q + o + page ids) over its average launch
time, measured with HIP events on the stream it runs on. Before the warm-up
steps an untimed clock-settle phase runs the step back to back for
--prewarm-ms (reported). The CPU baseline times the repository's CPU oracle
(torch fp32) on the host cores: configs 0 and 1 whole, config 2 on 16 of its
64 rows, each the median of 5 runs after 2 warm-ups.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X published HBM3E bandwidth
PROFILES = os.path.join(ROOT, "profiles")


def measured_traffic(config: int):
    """HBM bytes per attention launch from the committed rocprofv3 counter summary, if present.

    profiles/attention_config<N>_traffic.txt holds the calibrated FETCH_SIZE +
    WRITE_SIZE of the attention kernel (see the file for the commands).
    """
    path = os.path.join(PROFILES, f"attention_config{config}_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=1, choices=[1, 2, 3, 4],
                    help="1: mixed layer (default, also runs the components, config 4 and the config-3 decode "
                         "step); 2: refresh layer; 3: the full 36-layer decode step alone; 4: the long-context "
                         "layer at --draft-frac")
    ap.add_argument("--draft-frac", type=float, default=0.5, help="config 4: fraction of drafting rows")
    ap.add_argument("--selector", choices=["keymean", "first_last"], default="keymean",
                    help="config 3: the refresh layer's page selection (key-mean per KV head, or the reference's "
                         "first/last dump selector per row)")
    ap.add_argument("--class-mask", type=int, default=0,
                    help="config 4: plan only the rows of these row-tile classes (bit c-1 for class c: <=16, <=32, "
                         "<=48 query rows) and time their attention launch, no merge; value counts their KV bytes "
                         "(for per-class counters)")
    ap.add_argument("--waves-per-cu", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=5, help="timed CPU-baseline runs per config (after 2 warm-ups)")
    ap.add_argument("--no-components", action="store_true",
                    help="skip the per-component measurements (append, page list, merge, selectors, refresh layer)")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-3 full decode step")
    ap.add_argument("--decode-steps", type=int, default=30, help="timed graph replays of the config-3 step")
    ap.add_argument("--no-calibration", action="store_true",
                    help="skip the on-box HBM calibration (roofline.measured_peak_gbs is then null); for "
                         "counter passes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (read + write) for rocprofv3 counter calibration")
    ap.add_argument("--prewarm-ms", type=float, default=1000.0,
                    help="untimed clock-settle phase before the warm-up steps: the step runs back to back for "
                         "this long (wall clock), reported as config.timing.prewarm_ms")
    return ap.parse_args()


def timed(fn, steps, stream):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def timed_steps(fn, steps, stream):
    """Time ``steps`` back-to-back calls with one HIP event between consecutive calls (on
    ``stream``, where every kernel of the step launches). Returns (mean ms, per-call ms list):
    the mean is first-event-to-last-event over the calls."""
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for i in range(steps):
        fn()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return ev[0].elapsed_time(ev[steps]) / steps, per


def prewarm(fn, ms):
    """Run ``fn`` back to back for ``ms`` of wall clock (GPU clocks ramp up over the first tens
    of milliseconds of sustained work after an idle period). Returns (wall ms, calls)."""
    if ms <= 0:
        return 0.0, 0
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3, n


def summary(per):
    a = np.asarray(per, dtype=np.float64)
    return {"median_ms": round(float(np.median(a)), 5), "mean_ms": round(float(a.mean()), 5),
            "p10_ms": round(float(np.percentile(a, 10)), 5), "p90_ms": round(float(np.percentile(a, 90)), 5),
            "min_ms": round(float(a.min()), 5), "max_ms": round(float(a.max()), 5)}


def graph_timed(fn, steps, stream, reps=20, warm=2):
    """Average device ms per call of fn: `reps` calls captured in one HIP graph,
    replayed `steps` times (amortises the graph launch over the captured calls)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    ms = timed(g.replay, steps, stream) / reps
    del g
    return ms


def graph_settle(fn, ms, stream, reps=20):
    """Replay `reps` calls of fn captured in one HIP graph back to back for `ms` of wall clock.
    Right after a fresh multi-GB setup a memory-bound layer runs 4-5% slower until about 0.5 s
    of back-to-back replays have passed (idle time does not help, and eager calls with a host
    sync every few calls did not get there in 1 s); this times the settled state, as the
    headline's clock-settle phase does."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
    del g


def plan_rows_subset(w, st, keep):
    """Re-plan ``w`` over the rows of ``st`` where ``keep`` holds (the other rows get no queries):
    the plan spreads every class over all waves in one cost-ordered sequence, so a class is
    timed alone by planning its rows alone, not by masking classes out of a joint plan."""
    from aspire_amd.workloads import PAGE

    qo_full = st.qo_indptr_host.numpy()
    qo = qo_full.copy()  # same length (padding entries keep the bucket's end)
    qo[1 : st.batch + 1] = np.cumsum(np.where(keep, st.q_len, 0))
    qo = torch.from_numpy(qo.astype(np.int32)).to(st.q.device)
    w.plan(qo, st.kv_indptr, st.kv_indices, st.last_page_len, st.hq, st.hkv, 128, PAGE, causal=True)


def attention_only(w, q, cache, out, class_mask=None):
    """Launch only the attention kernels of w's current plan (no merge), as run() would;
    ``class_mask`` limits the launch to some row-tile classes."""
    import ctypes

    from aspire_amd import _lib

    k_cache, v_cache = cache[:, 0], cache[:, 1]
    a = _lib.AttentionArgs()
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.kv_cache = k_cache.data_ptr()
    a.cache_stride_p = k_cache.stride(0)
    a.cache_stride_kv = (v_cache.data_ptr() - k_cache.data_ptr()) // 2
    a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
    a.kv_indices = w._kv_indices.data_ptr()
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.plan_dev = w._int_workspace.data_ptr()
    a.float_ws = w._float_workspace.data_ptr()
    a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = w._num_qo_heads, w._num_kv_heads, 128, 16
    a.sm_scale, a.causal = 1.0 / 128 ** 0.5, 1
    info = w.plan_info
    a.class_mask = sum(1 << c for c in range(3) if info.num_items[c] > 0)
    if class_mask is not None:
        a.class_mask &= class_mask
    a.launch_merge = 0
    layout = w._layout

    def launch():
        rc = _lib.lib().aspire_attention_run(ctypes.byref(layout), ctypes.byref(a), _lib.stream_of(q))
        _lib.check(rc, "attention_only")

    return launch


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import aspire_amd.attention.kv_ops  # noqa: F401
    from aspire_amd import _lib
    from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
    from aspire_amd.backends.page_selector import KeyMeanPageSelector
    from aspire_amd.workloads import PAGE, config1, config2, config4

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(_lib.build_info())
    if args.config == 3:
        dec = measure_config3(args.decode_steps, min(args.warmup, 20), args.waves_per_cu, selector=args.selector)
        line = {
            "metric": "decode tokens/s (Qwen3-8B shape, 36 layers, B=64, ctx U[8k,32k], 50/50 draft/verify)",
            "value": dec["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.decode_steps,
            "warmup": min(args.warmup, 20), "ms_per_step": dec["step_ms"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (random-init bf16 weights, N(0,1) KV pages, random-permutation page pool)",
            "config": {"workload": dec["workload"], **{k: v for k, v in dec.items() if k != "workload"}},
        }
        print(json.dumps(line), flush=True)
        return
    t0 = time.time()
    if args.config == 1:
        step = config1(device=dev)
    elif args.config == 2:
        step = config2(device=dev)
    else:
        step = config4(device=dev, draft_frac=args.draft_frac)
    torch.cuda.synchronize()
    log(f"workload built in {time.time() - t0:.1f}s: batch {step.batch}, tokens {step.total_tokens}, "
        f"pool {step.cache.shape[0]} pages ({step.cache.numel() * 2 / 2**30:.2f} GiB)")
    cache = step.cache
    w = HolisticAttentionWrapper(torch.empty(1, device=dev), "NHD", waves_per_cu=args.waves_per_cu)
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, step.hq, step.hkv, 128, PAGE,
           causal=True)
    # host planning cost (plan_host: C++ planner + async upload), measured on its own
    reps = 20
    tp = time.perf_counter()
    for _ in range(reps):
        w.plan_host(step.qo_indptr_host, step.kv_indptr_host, step.kv_len_host, step.kv_indices, step.hq,
                    step.hkv, 128, PAGE, causal=True)
    plan_us = (time.perf_counter() - tp) / reps * 1e6
    torch.cuda.synchronize()
    info = w.plan_info
    log(f"plan: items {list(info.num_items)}, merges {info.num_merge}, partial rows {info.partial_rows}, "
        f"host {plan_us:.1f} us/plan")

    out = torch.empty_like(step.q)
    stream = torch.cuda.current_stream(dev)
    nbytes = step.algorithmic_bytes(include_append=args.config == 1)
    selector = None
    if args.config == 2:
        max_pages = int(step.block_table.shape[1])
        selector = KeyMeanPageSelector(step.batch, step.hkv, max_pages, k=128, L=0, device=dev)
        npg = torch.from_numpy((step.ctx_len + PAGE - 1) // PAGE).to(torch.int32).to(dev)
        nbytes["selection"] = step.batch * step.hkv * 128 * 4
        nbytes["total"] += nbytes["selection"]

        def run_step():
            w.run(step.q, cache, out=out, page_scores=selector.page_scores)
            selector.select(npg, step.block_table)
    elif args.config == 4 and args.class_mask:
        rows = step.q_len * (step.hq // step.hkv)
        cls = np.where(rows <= 16, 0, np.where(rows <= 32, 1, 2))
        keep = np.array([(args.class_mask >> c) & 1 for c in range(3)], dtype=bool)[cls]
        plan_rows_subset(w, step, keep)
        run_step = attention_only(w, step.q, cache, out)
        kvl = step.kv_len_host.numpy()[: step.batch].astype(np.int64)
        nbytes = {"kv": int(kvl[keep].sum()) * step.hkv * 128 * 4, "qo": 0, "indices": 0}
        nbytes["total"] = nbytes["kv"]
    elif args.config == 4:
        def run_step():
            w.run(step.q, cache, out=out)
    else:
        def run_step():
            torch.ops.mylib.update_kv_padded(step.k_new, step.v_new, step.qo_indptr, cache, step.kv_indices,
                                             step.kv_indptr, step.last_page_len, PAGE)
            w.run(step.q, cache, out=out)

    pw_ms, pw_steps = prewarm(run_step, args.prewarm_ms)
    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    log(f"clock settle {pw_ms:.0f} ms ({pw_steps} steps), {args.warmup} warm-up steps; timing {args.steps} steps")
    ms, per_step = timed_steps(run_step, args.steps, stream)
    value = nbytes["total"] / (ms * 1e-3) / 1e9

    # dominant kernel alone: mixed attention (no merge), same plan, same stream
    attn = attention_only(w, step.q, cache, out)
    for _ in range(3):
        attn()
    attn_ms, attn_per = timed_steps(attn, args.steps, stream)
    attn_bytes = nbytes["kv"] + nbytes["qo"] + nbytes["indices"]
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    log(f"step {ms * 1e3:.1f} us (median {np.median(per_step) * 1e3:.1f}) -> {value:.0f} GB/s; attention kernel "
        f"{attn_ms * 1e3:.1f} us (median {np.median(attn_per) * 1e3:.1f}) -> {achieved:.0f} GB/s "
        f"({achieved / PEAK_HBM_GBS:.1%} of 8 TB/s)")

    calib = None
    if not args.no_calibration:
        calib = measure_hbm_calibration(dev, stream)
        log(f"HBM calibration: streaming read {calib['measured_peak_gbs']:.0f} GB/s (best grid), copy "
            f"{calib['copy_gbs']:.0f} GB/s; attention kernel at {achieved / calib['measured_peak_gbs']:.1%} of the "
            "read")

    if args.calibrate_copy:
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev).random_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    components = None
    if args.config == 1 and not args.no_components:
        components = measure_components(step, w, out, min(args.steps, 50), plan_us)
        components["long_context_config4"] = measure_config4(min(args.steps, 100), args.waves_per_cu)
    decode = None
    if args.config == 1 and not args.no_decode:
        decode = measure_config3(args.decode_steps, min(args.warmup, 20), args.waves_per_cu)
        decode["first_last"] = measure_config3(args.decode_steps, min(args.warmup, 20), args.waves_per_cu,
                                               selector="first_last")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = run_cpu_baseline(step, args.config, args.cpu_runs)

    tokens = step.total_tokens
    if args.config == 1:
        workload = ("config1: Qwen3-8B-shape mixed layer (32 q / 8 kv heads, head_dim 128, bf16, 16-token pages), "
                    "batch 32 x 32768-token contexts, 16 draft rows (q_len 1 over 128 selected pages) + 16 verify "
                    "rows (q_len 4, causal, full cache); KV append of the 80 new tokens + attention")
        metric = "mixed-attn layer HBM GB/s (Qwen3-8B shape, B=32 x 32k, 16 draft + 16 verify)"
    elif args.config == 2:
        workload = ("config2: Qwen3-8B-shape refresh layer, batch 64, contexts U[8192, 32768], full attention for "
                    "64 single-query rows + per-KV-head key-mean page scores + top-128 selection")
        metric = "refresh-layer HBM GB/s (Qwen3-8B shape, B=64, ctx U[8k,32k])"
    else:
        workload = (f"config4: DS-Llama-8B-shape long-context layer (32 q / 8 kv heads), batch 16, contexts "
                    f"U[65536, 131072], draft fraction {args.draft_frac} (256-page drafts, verify q_len U{{2..9}}); "
                    "attention + split-KV merge")
        metric = f"long-context layer HBM GB/s (DS-Llama-8B shape, B=16, ctx U[64k,128k], f={args.draft_frac})"
        if args.class_mask:
            workload += (f"; only the rows of row-tile class mask {args.class_mask}, planned alone: attention "
                         "launch, KV bytes of those rows")
            metric += f", class mask {args.class_mask}"
    line = {
        "metric": metric,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q with per-page key bias; random-permutation page pool)",
        "config": {
            "workload": workload,
            "batch": step.batch,
            "context_tokens": int(step.ctx_len.max()),
            "tokens_per_step": tokens,
            "algorithmic_bytes": nbytes,
            "hbm_fraction_of_peak": round(value / PEAK_HBM_GBS, 4),
            "decode_tokens_per_s_layer": round(tokens / (ms * 1e-3), 1),
            "plan_host_us": round(plan_us, 1),
            "plan": {"items": list(info.num_items), "merges": info.num_merge, "waves": w._layout.num_waves},
            "timing": {"prewarm_ms": round(pw_ms, 1), "prewarm_steps": pw_steps,
                       "note": "untimed clock-settle phase (the step back to back) before the warm-up steps; "
                               "ms_per_step is the mean over the timed steps (first to last HIP event), "
                               "per_step the distribution of the per-step events",
                       "per_step": summary(per_step), "attention_kernel": summary(attn_per)},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "attention_kernel (mixed draft/verify persistent kernel, every row-tile class of the plan)",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(args.config),
            "measured_peak_gbs": calib["measured_peak_gbs"] if calib else None,
            "frac_of_measured": round(achieved / calib["measured_peak_gbs"], 4) if calib else None,
            "calibration": calib,
            "kernel_us": round(attn_ms * 1e3, 2),
            "bytes_per_launch": attn_bytes,
        },
        "cpu_baseline": cpu,
        "decode": decode,
        "components": components,
    }
    print(json.dumps(line), flush=True)


def measure_hbm_calibration(dev, stream, read_gib: int = 4, copy_gib: int = 2, launches: int = 10):
    """The bandwidth achieved on this box with the library's streaming kernels
    (``aspire_bandwidth_probe``): a single read of a ``read_gib`` GiB buffer as 1 KiB contiguous
    non-temporal buffer loads (the attention kernel's staged K/V access), swept over rows in
    flight per wave and grid sizes, and a plain read + write copy of ``copy_gib`` GiB. Each
    figure is the mean of ``launches`` launches after 3 warm-ups, timed with HIP events on
    ``stream``; the best read is the measured peak the roofline fraction is also read against."""
    import ctypes

    from aspire_amd import _lib

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    L = _lib.lib()
    st = ctypes.c_void_p(stream.cuda_stream)
    src = torch.empty(read_gib << 30, dtype=torch.uint8, device=dev)
    src[:: 1 << 20].fill_(1)
    sink = torch.zeros(cus * 64 * 1024, dtype=torch.uint8, device=dev)

    def probe(mode, a, nbytes, b, b_bytes, wgs, depth):
        def fn():
            _lib.check(L.aspire_bandwidth_probe(mode, _lib.ptr(a), nbytes, _lib.ptr(b), b_bytes, wgs, depth, st),
                       "bandwidth probe")
        return fn

    def rate(fn, nbytes):
        for _ in range(3):
            fn()
        ms = timed(fn, launches, stream)
        return round(nbytes / (ms * 1e-3) / 1e9, 1)

    grids = (0.75, 1, 1.5, 2, 3, 4)
    reads = {f"rows{d}_wg{g}": rate(probe(0, src, src.numel(), sink, sink.numel(), int(cus * g), d), src.numel())
             for d in (2, 4, 8) for g in grids}
    del src
    a = torch.empty(copy_gib << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a[:: 1 << 20].fill_(1)
    copies = {f"chunks{d}_wg{g}": rate(probe(1, a, a.numel(), b, b.numel(), int(cus * g), d), 2 * a.numel())
              for d in (1, 2, 4) for g in (1, 2, 4, 8)}
    del a, b, sink
    torch.cuda.synchronize()
    best = max(reads.values())
    return {"measured_peak_gbs": best, "copy_gbs": max(copies.values()), "read_gbs_by_grid": reads,
            "copy_gbs_by_grid": copies, "read_bytes": read_gib << 30, "copy_bytes": copy_gib << 30,
            "kernel": "aspire_bandwidth_probe: mode 0 reads 1 KiB rows with 128-bit non-temporal buffer loads "
                      "(rowsR: R rows in flight per wave; wgG: G 256-thread workgroups per CU); mode 1 copies "
                      "with 128-bit loads and stores (chunksR per thread; GB/s counts read + write)"}


def _gbs(nbytes, us):
    return round(nbytes / (us * 1e-6) / 1e9, 1)


def measure_components(step, w, out, steps, plan_us):
    """Per-row measurements beside the layer: every piece of the path, timed on its own.

    Each entry: average microseconds per call (HIP events, current stream),
    algorithmic bytes and the resulting GB/s with its fraction of 8 TB/s.
    """
    import ctypes

    from aspire_amd import _lib
    from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
    from aspire_amd.attention.page_list import build_unified_indices
    from aspire_amd.backends.page_selector import KeyMeanPageSelector, PageSelectorFirstLastAvg
    from aspire_amd.workloads import PAGE, config2

    dev = step.q.device
    stream = torch.cuda.current_stream(dev)
    res = {}

    def entry(us, nbytes, **extra):
        d = {"us": round(us, 2), "bytes": int(nbytes), "gbs": _gbs(nbytes, us),
             "frac_of_peak": round(_gbs(nbytes, us) / PEAK_HBM_GBS, 4)}
        d.update(extra)
        return d

    # (a1) KV append alone
    app = lambda: torch.ops.mylib.update_kv_padded(step.k_new, step.v_new, step.qo_indptr, step.cache,
                                                   step.kv_indices, step.kv_indptr, step.last_page_len, PAGE)
    us = graph_timed(app, steps, stream) * 1e3
    res["append"] = entry(us, step.total_tokens * step.hkv * 128 * 2 * 2 * 2, tokens=step.total_tokens,
                          note="20 calls per graph replay; latency-bound: one workgroup per token")

    # (f2) q/k RMSNorm + rotary permute + RoPE + append in one launch, against the same
    # sequence run as the reference runs it (torch norm and permute, then rope, then append)
    from aspire_amd.attention.rope import RopeConfig, apply_rope_inplace, qk_norm_rope_update_kv
    gq = torch.Generator(device=dev).manual_seed(5)
    T = step.total_tokens
    q0 = torch.randn(T, step.hq, 128, generator=gq, device=dev).to(torch.bfloat16)
    k0 = torch.randn(T, step.hkv, 128, generator=gq, device=dev).to(torch.bfloat16)
    wq = torch.rand(128, generator=gq, device=dev).to(torch.bfloat16) + 0.5
    wk = torch.rand(128, generator=gq, device=dev).to(torch.bfloat16) + 0.5
    offs = torch.from_numpy(np.append(step.ctx_len - step.q_len, 0).astype(np.int32)).to(dev)
    qb, kb = q0.clone(), k0.clone()
    rc = RopeConfig(1e6)

    def fused():
        qk_norm_rope_update_kv(qb, k0, step.v_new, wq, wk, 1e-6, step.qo_indptr, offs, step.cache, step.kv_indices,
                               step.kv_indptr, step.last_page_len, PAGE, config=rc)

    def norm(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * w

    def perm(x):
        return x.view(*x.shape[:-1], 2, 64).transpose(-2, -1).reshape(x.shape)

    def unfused():
        qn, kn = perm(norm(q0, wq)), perm(norm(k0, wk))
        apply_rope_inplace(qn, kn, step.qo_indptr, offs, rc)
        torch.ops.mylib.update_kv_padded(kn, step.v_new, step.qo_indptr, step.cache, step.kv_indices,
                                         step.kv_indptr, step.last_page_len, PAGE)

    us_f = graph_timed(fused, steps, stream) * 1e3
    us_u = graph_timed(unfused, steps, stream) * 1e3
    nb = T * (step.hq * 2 + step.hkv * 2 + step.hkv * 2) * 256
    res["qk_norm_rope_append"] = entry(us_f, nb, unfused_us=round(us_u, 2), tokens=T,
                                       note="20 calls per graph replay; q/k RMSNorm + permute + RoPE (theta 1e6) + "
                                            "K/V append in one launch; unfused_us: torch norm/permute + rope + append")

    # (a2) mixed page list from the draft selections and the block table
    B = step.batch
    width = int(step.block_table.shape[1])
    dtab = torch.zeros(B, 128, dtype=torch.int32, device=dev)
    dn = torch.zeros(B, dtype=torch.int32, device=dev)
    for b in range(B):
        if step.draft_pages[b] is not None:
            ph = step.block_table[b, torch.from_numpy(step.draft_pages[b]).to(dev)]
            dtab[b, : ph.numel()] = ph
            dn[b] = ph.numel()
    vn = torch.full((B,), width, dtype=torch.int32, device=dev)
    idx = torch.empty(B * width, dtype=torch.int32, device=dev)
    ptr = torch.empty(B + 2, dtype=torch.int32, device=dev)
    pl = lambda: build_unified_indices(step.mode_flags, dtab, step.block_table, dn, vn, idx, ptr, indptr_fill_to=B + 2)
    us = graph_timed(pl, steps, stream) * 1e3
    entries = int(step.kv_indptr_host[B])
    assert torch.equal(ptr, step.kv_indptr) and torch.equal(idx[:entries], step.kv_indices)
    res["page_list"] = entry(us, entries * 8 + B * 16, entries=entries, note="20 calls per graph replay")

    # (a7) host planner, and the native host mirror that renders its input arrays each step
    res["plan_host"] = {"us": round(plan_us, 1), "note": "C++ planner + async upload of the live plan segments"}
    from aspire_amd.backends.host_plan import HostPlanConfig, HostPlanState
    hp = HostPlanState(HostPlanConfig(page_size=PAGE, max_batch=step.batch, draft_kind="replan",
                                      full_kind="effective_full", subset_cache_size=128, table_width=2048,
                                      min_draft_pages=None, draft_percent=None, valid_floor_l=8,
                                      pages_per_slot=2048))
    seq = np.asarray(step.ctx_len, dtype=np.int64) - step.q_len
    hp.reset_all(seq)
    ver = ~np.asarray(step.is_draft, dtype=bool)
    fin = np.zeros(step.batch, dtype=bool)
    dcnt = np.where(ver, step.q_len - 1, 0).astype(np.int64)
    tot = int(np.where(ver, dcnt + 1, 1).sum())
    reps = 2000
    t0 = time.perf_counter()
    for _ in range(reps):
        hp.build_step(verify=ver, finished=fin, draft_counts=dcnt, seq_lens=seq, total_tokens=tot,
                      bucket_tokens=tot)
    res["host_plan_step"] = {"us": round((time.perf_counter() - t0) / reps * 1e6, 2), "rows": step.batch,
                             "note": "HostPlanState.build_step (native mirror) per decode step, host only"}

    # (a6) split-KV merge alone (partials from the last attention run)
    info = w.plan_info
    a = _lib.AttentionArgs()
    k_cache, v_cache = step.cache[:, 0], step.cache[:, 1]
    a.q, a.q_stride_t, a.q_stride_h = step.q.data_ptr(), step.q.stride(0), step.q.stride(1)
    a.kv_cache, a.cache_stride_p = k_cache.data_ptr(), k_cache.stride(0)
    a.cache_stride_kv = (v_cache.data_ptr() - k_cache.data_ptr()) // 2
    a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
    a.kv_indices = w._kv_indices.data_ptr()
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.plan_dev, a.float_ws = w._int_workspace.data_ptr(), w._float_workspace.data_ptr()
    a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = step.hq, step.hkv, 128, PAGE
    a.sm_scale, a.causal, a.class_mask, a.launch_merge = 1.0 / 128 ** 0.5, 1, 0, 1

    def merge():
        _lib.check(_lib.lib().aspire_attention_run(ctypes.byref(w._layout), ctypes.byref(a), _lib.stream_of(out)),
                   "merge")

    us = graph_timed(merge, steps, stream) * 1e3
    merge_bytes = info.partial_rows * 129 * 4 + info.num_merge * 16 * 256
    res["merge"] = entry(us, merge_bytes, merges=info.num_merge, partial_rows=info.partial_rows,
                         note="20 calls per graph replay; bytes = fp32 partials read + 16 bf16 rows out per merge")

    # (f4) sampling at the config-3 decode step's size: 208 tokens' top-50 candidates over the
    # 151,936-entry vocabulary, the temperature/softmax/top-p pipe, one draw per token, and the
    # speculative verification of 32 requests x 8 drafts over their top-50 candidates
    from aspire_amd.engine.sampling import local_topk_candidates, verify_topk_speculation
    from aspire_amd.logits_processor import build_logits_pipe
    from aspire_amd.sampling import sampling_from_probs
    gs = torch.Generator(device=dev).manual_seed(11)
    logits = torch.randn(208, 151936, generator=gs, device=dev).to(torch.bfloat16)
    pipe, pkw = build_logits_pipe(0.8, 0.9)
    u = torch.rand(208, generator=gs, device=dev)

    def sample_step():
        vals, ids = local_topk_candidates(logits, 50)
        sampling_from_probs(pipe(vals, **pkw), uniforms=u)

    us_s = graph_timed(sample_step, steps, stream) * 1e3
    R, D, K = 32, 8, 50
    tprobs = torch.softmax(torch.randn(R, D + 1, K, generator=gs, device=dev), -1)
    dprobs = torch.softmax(torch.randn(R, D, K, generator=gs, device=dev), -1)
    tids = torch.randint(0, 151936, (R, D + 1, K), generator=gs, device=dev)
    dids = tids[:, :D].clone()
    dtok = dids[:, :, 0].to(torch.int32)
    dcnt = torch.full((R,), D, dtype=torch.int32, device=dev)
    uv = torch.rand(R, D + 1, generator=gs, device=dev)
    us_v = graph_timed(lambda: verify_topk_speculation(dprobs, dids, dtok, dcnt, tprobs, tids, uniforms=uv),
                       steps, stream) * 1e3
    # the same verification at the largest top_k (candidate ids unique within a position)
    KL = 1024
    tprobs_l = torch.softmax(torch.randn(R, D + 1, KL, generator=gs, device=dev), -1)
    dprobs_l = torch.softmax(torch.randn(R, D, KL, generator=gs, device=dev), -1)
    off = torch.randint(0, 151936, (R, D + 1, 1), generator=gs, device=dev)
    tids_l = (off + 97 * torch.arange(KL, device=dev)) % 151936
    dids_l = tids_l[:, :D].clone()
    dtok_l = dids_l[:, :, 0].to(torch.int32)
    us_vl = graph_timed(lambda: verify_topk_speculation(dprobs_l, dids_l, dtok_l, dcnt, tprobs_l, tids_l,
                                                        uniforms=uv), steps, stream) * 1e3
    res["sampling"] = {"topk_pipe_draw_us": round(us_s, 2), "rows": 208, "vocab": 151936, "top_k": 50,
                       "logits_bytes": 208 * 151936 * 2,
                       "logits_gbs": _gbs(208 * 151936 * 2, us_s),
                       "verify_us": round(us_v, 2), "verify_requests": R, "verify_drafts": D,
                       "verify_us_top_k_1024": round(us_vl, 2),
                       "note": "20 calls per graph replay; top-k candidates + LogitsPipe(temperature 0.8, "
                               "top-p 0.9) + sampling_from_probs; verify_topk_speculation in one launch"}
    del logits

    # (f3) chunked prefill: one 8192-token prompt chunk (the reference's max_prefill_tokens) over an empty
    # prefix, and 4 x 2048-token chunks over 6144 cached tokens each, Qwen3-8B heads; causal
    from aspire_amd.attention.prefill import BatchPrefillWithPagedKVCacheWrapper
    from aspire_amd.workloads import build_step as _build
    pre = {}
    for name, ctx, ql in (("chunk_8192_prefix_0", [8192], [8192]),
                          ("4x2048_over_6144", [8192] * 4, [2048] * 4)):
        st = _build(hq=32, hkv=8, ctx_len=ctx, q_len=ql, is_draft=[0] * len(ctx), draft_budget=0, seed=4,
                    device=dev)
        po = torch.empty_like(st.q)
        times = {}
        for kernel in ("prefill", "decode"):
            pw = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=dev), "NHD", kernel=kernel)
            pw.plan(st.qo_indptr, st.kv_indptr, st.kv_indices, st.last_page_len, 32, 8, 128, PAGE, causal=True)
            run = lambda: pw.run(st.q, st.cache, out=po)
            # sustained work first: the chunk takes ~0.5 ms, so 20 calls from idle clocks
            # would time the clock ramp, not the kernel
            prewarm(run, 100)
            times[kernel] = timed(run, 20, stream) * 1e3
            del pw
        us = times["prefill"]
        # causal FLOPs: QK and PV, 2 flops per MAC, each token against its visible keys
        keys = sum(sum(c - q + t + 1 for t in range(q)) for c, q in zip(ctx, ql))
        flops = 4 * 128 * 32 * keys
        pre[name] = {"us": round(us, 1), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                     "frac_of_bf16_mfma_peak": round(flops / (us * 1e-6) / 2.5e15, 4),
                     "kernel": "prefill_kernel (aspire_prefill_run)",
                     "decode_kernel_us": round(times["decode"], 1)}
        del st, po
    res["prefill"] = pre

    # refresh layer (config 2): full attention + key-mean page scores + top-128 per (row, kv head)
    step2 = config2(device=dev)
    w2 = HolisticAttentionWrapper(torch.empty(1, device=dev), "NHD")
    w2.plan(step2.qo_indptr, step2.kv_indptr, step2.kv_indices, step2.last_page_len, 32, 8, 128, PAGE, causal=True)
    out2 = torch.empty_like(step2.q)
    max_pages = int(step2.block_table.shape[1])
    ks = KeyMeanPageSelector(step2.batch, 8, max_pages, k=128, L=0, device=dev)
    npg2 = torch.from_numpy((step2.ctx_len + PAGE - 1) // PAGE).to(torch.int32).to(dev)

    def refresh_attention():
        w2.run(step2.q, step2.cache, out=out2, page_scores=ks.page_scores)

    def refresh_topk():
        ks.select(npg2, step2.block_table)

    def refresh():
        refresh_attention()
        refresh_topk()

    graph_settle(refresh, 1000, stream)
    us = graph_timed(refresh, steps, stream) * 1e3
    us_att = graph_timed(refresh_attention, steps, stream) * 1e3
    us_topk = graph_timed(refresh_topk, steps, stream) * 1e3
    nb2 = step2.algorithmic_bytes(include_append=False)
    sel_bytes = step2.batch * 8 * 128 * 4 * 2 + int(npg2.sum()) * 8 * 4 * 2  # scores written + read, lists out
    res["refresh_layer_config2"] = entry(us, nb2["total"] + sel_bytes, batch=step2.batch,
                                         kv_tokens=int(step2.kv_len_host.sum()),
                                         attention_us=round(us_att, 2), topk_us=round(us_topk, 2),
                                         note="20 calls per graph replay: attention with the key-mean page-score epilogue"
                                              " + top-128 per (row, kv head)")

    # (a3) reference first/last selector at refresh-layer scale (B=64, 32 heads, 32k max context)
    Bs, H, max_seq = step2.batch, 32, 32768
    gen = torch.Generator(device=dev).manual_seed(7)
    dump = (torch.randn(Bs, H, 2, max_seq, generator=gen, device=dev) * 6).to(torch.float16)
    pos = torch.arange(max_seq, device=dev)
    ctx = torch.from_numpy(step2.ctx_len).to(dev)
    dump.masked_fill_(pos[None, None, None, :] >= ctx[:, None, None, None], float("-inf"))
    lse = torch.randn(Bs * 10, H, generator=gen, device=dev) + 8
    qo = torch.arange(Bs + 2, dtype=torch.int32, device=dev) * 4
    table = torch.arange(Bs * 2048, dtype=torch.int32, device=dev).view(Bs, 2048)
    sel = PageSelectorFirstLastAvg(Bs, 2048, 144, 8, H, PAGE, max_seq, dev, Bs, 9, draft_percent=7.0,
                                   min_draft_pages=32)
    selr = lambda: sel.select(dump.view(-1), lse, npg2, table, qo)
    us = graph_timed(selr, steps, stream) * 1e3
    dump_bytes = int(npg2.sum()) * 16 * H * 2 * 2
    res["select_first_last"] = entry(us, dump_bytes + Bs * 2048 * 4 * 2 + Bs * 144 * 4, rows=Bs, heads=H,
                                     note="20 calls per graph replay; reference (R) selector: dump read over each row's pages + top-k")
    del dump, step2, w2
    torch.cuda.synchronize()
    return res


def measure_config4(steps, waves_per_cu, fracs=(0.0, 0.25, 0.5, 0.75, 1.0)):
    """Config 4 (batch 16, contexts U[64k, 128k], verify q_len U{2..9}, 256-page drafts):
    attention + split-KV merge per draft fraction f, timed as 20 calls per graph replay: at
    f = 1.0 the layer takes less device time than the host needs to launch one call."""
    from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
    from aspire_amd.workloads import PAGE, config4

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    res = {}
    for f in fracs:
        st = config4(device=dev, draft_frac=f)
        w = HolisticAttentionWrapper(torch.empty(1, device=dev), "NHD", waves_per_cu=waves_per_cu)
        w.plan(st.qo_indptr, st.kv_indptr, st.kv_indices, st.last_page_len, st.hq, st.hkv, 128, PAGE, causal=True)
        out = torch.empty_like(st.q)
        fn = lambda: w.run(st.q, st.cache, out=out)
        graph_settle(fn, 1000, stream)
        ms = graph_timed(fn, steps, stream)
        nb = st.algorithmic_bytes(include_append=False)["total"]
        info = w.plan_info
        gbs = nb / (ms * 1e-3) / 1e9
        # each row-tile class alone (rows = q_len * group: <=16, <=32, <=48), planned alone
        rows = st.q_len * (st.hq // st.hkv)
        cls = np.where(rows <= 16, 0, np.where(rows <= 32, 1, 2))
        kvl = st.kv_len_host.numpy()[: st.batch].astype(np.int64)
        per_class = {}
        for c in range(3):
            if not (cls == c).any():
                continue
            plan_rows_subset(w, st, cls == c)
            fn_c = attention_only(w, st.q, st.cache, out)
            fn_c()
            us_c = graph_timed(fn_c, steps, stream) * 1e3
            nb_c = int(kvl[cls == c].sum()) * st.hkv * 128 * 4
            per_class[f"class{c + 1}"] = {"us": round(us_c, 1), "kv_bytes": nb_c,
                                          "gbs": round(nb_c / (us_c * 1e-6) / 1e9, 1)}
        res[f"f={f}"] = {"us": round(ms * 1e3, 1), "bytes": nb, "gbs": round(gbs, 1),
                         "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "draft_rows": int(st.is_draft.sum()),
                         "q_len": st.q_len.tolist(), "items_per_class": list(info.num_items),
                         "merges": info.num_merge, "partial_rows": info.partial_rows, "per_class": per_class}
        log(f"config4 f={f}: {ms * 1e3:.1f} us -> {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%}), "
            f"items {list(info.num_items)}, merges {info.num_merge}; per class {per_class}")
        del st, w, out
        torch.cuda.empty_cache()
    return res


def measure_config3(steps, warmup, waves_per_cu, selector="keymean"):
    """Config 3: one full 36-layer Qwen3-8B decode step (batch 64, contexts U[8k, 32k], 32 draft rows
    over top-128 page lists refreshed at layer 2, 32 verify rows with q_len U{2..9}), recorded in
    one HIP graph and replayed. ``selector``: "keymean" (per-KV-head key-mean lists) or
    "first_last" (the reference's first/last dump, per-row selection and row lists). Returns
    tokens/s, step time and the attention share."""
    from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
    from aspire_amd.decode_step import QWEN3_8B, DecodeWeights, MixedDecodeStep, alloc_kv_caches
    from aspire_amd.workloads import PAGE, config3_rows, random_block_table

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    shape = QWEN3_8B
    ctx, ql, dr = config3_rows(seed=0)
    n_pages = (ctx + PAGE - 1) // PAGE
    table, pool = random_block_table(n_pages, seed=0)
    t0 = time.time()
    weights = DecodeWeights(shape, dev, seed=0)
    caches = alloc_kv_caches(shape, pool, dev, seed=0)
    step = MixedDecodeStep(weights, caches, ctx, ql, dr, torch.from_numpy(table), budget=128, refresh_layer=2,
                           selector=selector, waves_per_cu=waves_per_cu)
    torch.cuda.synchronize()
    log(f"config3 ({selector}): built in {time.time() - t0:.1f}s: {int(dr.sum())} draft + {int((~dr).sum())} verify rows, "
        f"{step.T} tokens, pool {pool} pages x {shape.n_layer} layers "
        f"({caches.numel() * 2 / 1e9:.1f} GB KV), weights {(shape.n_layer * weights.layer_bytes() + 2 * weights.output.numel() * 2) / 1e9:.1f} GB")
    reps = 10
    tp = time.perf_counter()
    for _ in range(reps):
        step.plan()
    plan_us = (time.perf_counter() - tp) / reps * 1e6
    torch.cuda.synchronize()
    for _ in range(3):
        step.forward()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    eager_n = 5
    eager_ms = timed(step.forward, eager_n, stream)
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step.forward()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.forward()
    pw_ms, _ = prewarm(graph.replay, 500)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ms, per_step = timed_steps(graph.replay, steps, stream)
    attn_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(attn_graph):
        step.attention_only()
    for _ in range(3):
        attn_graph.replay()
    attn_ms = timed(attn_graph.replay, steps, stream)
    extra = {}
    if selector == "first_last":
        # the refresh layer with its dump against the same attention without it, and the
        # selection + row lists of the step's preparation, each graph-timed on its own
        q = step.qkv[:, : shape.q_size].view(step.T, shape.n_head, shape.head_dim)
        cache = step.caches[step.refresh_layer]
        plain = HolisticAttentionWrapper(torch.empty(1, device=dev), "NHD", waves_per_cu=waves_per_cu)
        plain.plan(step.qo_indptr, step.full_indptr, step.full_indices, step.last_page_len, shape.n_head,
                   shape.n_local_heads, 128, PAGE, causal=True)
        with_dump = lambda: step.attention(step.refresh_layer, q)
        no_dump = lambda: plain.run(q, cache, out=step.y)
        extra = {"refresh_layer_us": round(graph_timed(with_dump, steps, stream) * 1e3, 1),
                 "refresh_layer_us_without_dump": round(graph_timed(no_dump, steps, stream) * 1e3, 1),
                 "selection_and_lists_us": round(graph_timed(step.select_first_last, steps, stream) * 1e3, 1)}
        extra["dump_cost_share_of_refresh_layer"] = round(
            1 - extra["refresh_layer_us_without_dump"] / extra["refresh_layer_us"], 4)
        del plain
    nb = step.algorithmic_bytes()
    tps = step.T / (ms * 1e-3)
    gbs = nb["total"] / (ms * 1e-3) / 1e9
    attn_gbs = nb["kv"] / (attn_ms * 1e-3) / 1e9
    log(f"config3 ({selector}): step {ms:.2f} ms (eager {eager_ms:.2f} ms) -> {tps:.0f} tokens/s, {gbs:.0f} GB/s; "
        f"attention {attn_ms:.2f} ms ({attn_ms / ms:.1%}) at {attn_gbs:.0f} GB/s; {extra} "
        f"measured in {time.perf_counter() - t1:.1f}s")
    sel_text = ("top-128 pages per KV head by key-mean score, refreshed at layer 2" if selector == "keymean" else
                "top-128 pages per row by the reference's first/last selector (PageSelectorFirstLastAvg, last 8 "
                "pages forced) over the fp16 first/last logits dump of layer 2, selected in the next step's "
                "preparation; one page list per row (build_unified_indices)")
    res = {
        "workload": ("config3: full 36-layer Qwen3-8B decode step (hidden 4096, 32/8 heads, SwiGLU 12288, "
                     f"qk-norm, RoPE 1e6), batch 64, contexts U[8192, 32768], 32 draft rows (q_len 1, {sel_text}) "
                     "+ 32 verify rows (q_len U{2..9}); one HIP graph per step, greedy token pick"),
        "selector": selector,
        "tokens_per_s": round(tps, 1),
        "step_ms": round(ms, 3),
        "eager_step_ms": round(eager_ms, 3),
        "tokens_per_step": step.T,
        "algorithmic_bytes": nb,
        "step_gbs": round(gbs, 1),
        "step_frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
        "attention_ms": round(attn_ms, 3),
        "attention_share": round(attn_ms / ms, 4),
        "attention_kv_gbs": round(attn_gbs, 1),
        "plan_host_us": round(plan_us, 1),
        "verify_q_len": ql[~dr].tolist(),
        "timing": {"prewarm_ms": round(pw_ms, 1), "per_step": summary(per_step)},
        **extra,
    }
    del graph, attn_graph, step, caches, weights
    torch.cuda.empty_cache()
    return res


def _cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def _cpu_layer(step, rows, *, append: bool, select_k: int = 0):
    """CPU inputs of one layer restricted to ``rows``: only their pages cross to the host (gathered
    on the device, renumbered). Returns (fn, algorithmic bytes): fn runs the CPU oracle, the
    paged append in place (``append``) then attention over every listed row, plus the key-mean
    page scores and the top-``select_k`` pages per (row, kv head) when ``select_k``."""
    from aspire_amd.workloads import PAGE
    from oracle.append import paged_kv_append
    from oracle.attention import paged_attention
    from oracle.select import topk_pages_per_head

    qo = step.qo_indptr_host.numpy()
    kvp = step.kv_indptr_host.numpy()
    kvl = step.kv_len_host.numpy()
    lpl = step.last_page_len.cpu().numpy()
    idx = step.kv_indices.cpu()
    lists = [idx[int(kvp[b]) : int(kvp[b + 1])].long() for b in rows]
    uniq, inv = torch.unique(torch.cat(lists), return_inverse=True)
    cache = step.cache[uniq.to(step.cache.device)].cpu()
    cache_bits = cache.view(torch.int16).numpy()          # shares memory with ``cache``
    sub_kvp = np.concatenate([[0], np.cumsum([len(x) for x in lists])]).astype(np.int64)
    sub_idx = inv.to(torch.int32)
    sub_idx_np = sub_idx.numpy()
    toks = np.concatenate([np.arange(qo[b], qo[b + 1]) for b in rows]).astype(np.int64)
    sub_qo = np.concatenate([[0], np.cumsum([qo[b + 1] - qo[b] for b in rows])]).astype(np.int64)
    sub_kvl = [int(kvl[b]) for b in rows]
    sub_lpl = np.array([int(lpl[b]) for b in rows], dtype=np.int64)
    tok_d = torch.from_numpy(toks).to(step.q.device)
    q = step.q[tok_d].cpu()
    kn = step.k_new[tok_d].cpu().view(torch.int16).numpy()
    vn = step.v_new[tok_d].cpu().view(torch.int16).numpy()
    hkv = step.hkv
    n_pages = np.repeat([(n + PAGE - 1) // PAGE for n in sub_kvl], hkv)

    def fn():
        if append:
            paged_kv_append(kn, vn, sub_qo, cache_bits, sub_idx_np, sub_kvp, sub_lpl, PAGE, inplace=True)
        scores = torch.full((len(rows) * hkv, int(n_pages.max())), float("nan")) if select_k else None
        paged_attention(q, cache, sub_qo, sub_kvp, sub_idx, sub_kvl, num_kv_heads=hkv, page_scores=scores)
        if select_k:
            topk_pages_per_head(scores, n_pages, select_k, 0)

    t = int(sub_qo[-1])
    nbytes = (sum(sub_kvl) * hkv * 128 * 2 * 2 + t * step.hq * 128 * 2 * 2 + int(sub_kvp[-1]) * 4
              + (t * hkv * 128 * 2 * 2 * 2 if append else 0) + (len(rows) * hkv * select_k * 4 if select_k else 0))
    return fn, nbytes


def _cpu_time(fn, warmup: int, runs: int):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), times


def run_cpu_baseline(step, config: int, runs: int):
    """The CPU oracle (torch fp32 attention, numpy append, key-mean scores and top-k) on the host
    cores: 2 warm-up runs, then the median of ``runs`` (>= 5) runs on
    identical seeded inputs. Config 0 whole; config 1 whole (the bench workload: append +
    attention); config 2 on a bounded sample of 16 of its 64 rows (attention + key-mean scores +
    top-128), scaled to GB/s. Threads: the process's CPU share (OMP_NUM_THREADS, 16 on the GPU
    boxes) capped by os.cpu_count(); both are reported."""
    from aspire_amd.workloads import config0, config2

    host_cpus = os.cpu_count() or 1
    threads = min(host_cpus, int(os.environ.get("OMP_NUM_THREADS", host_cpus) or host_cpus))
    torch.set_num_threads(threads)
    dev = step.q.device
    per = {}
    t_all = time.perf_counter()

    def measure(name, st, rows, **kw):
        fn, nbytes = _cpu_layer(st, rows, **kw)
        med, times = _cpu_time(fn, 2, max(runs, 5))
        per[name] = {"median_s": round(med, 4), "runs_s": [round(x, 4) for x in times],
                     "bytes": nbytes, "gbs": round(nbytes / med / 1e9, 3), "rows": len(rows)}
        log(f"cpu baseline {name}: median {med * 1e3:.1f} ms over {len(times)} runs -> {nbytes / med / 1e9:.2f} GB/s")

    c0 = config0(device=dev)
    measure("config0", c0, list(range(c0.batch)), append=True)
    del c0
    main_name = f"config{config}"
    measure(main_name, step, list(range(step.batch)), append=config == 1, select_k=128 if config == 2 else 0)
    if config == 1:
        c2 = config2(device=dev)
        rng = np.random.default_rng(0)
        measure("config2", c2, sorted(rng.choice(c2.batch, 16, replace=False).tolist()), append=False, select_k=128)
        del c2
        torch.cuda.empty_cache()
    head = per[main_name]
    return {
        "value": head["gbs"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "host_cpu_count": host_cpus,
        "cpu_model": _cpu_model(),
        "protocol": f"torch.set_num_threads({threads}); 2 warm-up runs, then the median of {max(runs, 5)} runs on "
                    "identical seeded inputs; value = the bench workload's algorithmic bytes / median time",
        "sample": f"{main_name}: the whole layer ({head['rows']} rows) through the CPU oracle"
                  + (" (KV append + attention)" if config == 1 else " (attention + key-mean scores + top-128)")
                  + "; config0: whole; config2: 16 of its 64 rows (attention + key-mean scores + top-128)",
        "per_config": per,
        "wall_s": round(time.perf_counter() - t_all, 1),
    }


if __name__ == "__main__":
    main()
