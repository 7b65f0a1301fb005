"""Benchmark of the MI355X paged-attention hot path on one GPU.

    python bench.py [--steps K] [--warmup W] [--workload N] [--headline-only] [--no-cpu-baseline]

One step = one call of the hot path over one batch of synthetic input already
resident in HBM. The metric has two halves (decode GB/s against the HBM roofline,
extend TFLOP/s against the bf16 MFMA roofline), so one JSON line carries:

* the headline, workload 1 (``value``, ``roofline``, ``cpu_baseline``): batched ragged
  paged decode, B=64, ctx U[1024, 8192], 64 q / 8 kv heads, D=128, bf16, page size 1
  with shuffled slots. ``value`` = algorithmic GB/s (K+V once per token and kv head,
  4 B of slot index per token, q in and out) over the timed region;
* ``extend``: workload 2, prefix-aware extend, B=8, P U[0, 4096], E U[256, 2048],
  40 q / 8 kv heads, bf16: TFLOP/s of the visible query-key pairs (4 D Hq flop each),
  its MFMA roofline and a CPU baseline;
* ``fp8_decode``: workload 3 (B=128, ctx U[4096, 32768], 32 / 8 heads) over e4m3 and
  e5m2 pools; ``verify``: workload 4 (B=32, 4 draft tokens, P U[2048, 16384], 64 / 8
  heads); ``decode_b1``: workload 0's latency; ``kv_write``: the pool write of the
  extend batch into an e4m3 pool; ``head_dim_256`` and ``head_dim_512``: decode and
  extend at head dims 256 (workloads 5, 6) and 512 (7, 8); ``padded_head_dims``: the
  extend batch at head dims 96 and 192 (workloads 9, 10) on the padded tiled kernel;
  ``verify_fp8`` and ``extend_fp8``: the verify and extend batches over an e4m3 pool
  (workloads 11 and 12). ``--headline-only`` skips all of these.

``value`` is whole-job throughput: algorithmic bytes of the K timed steps over
the wall time between the two synchronisations. Warm-up is W untimed steps and
then more untimed steps until half a second has passed, so that the timed steps
run at settled clocks. ``roofline`` compares the
algorithmic bytes of one call with its HIP-event duration on the launch stream
against the 8 TB/s HBM peak; ``roofline.traffic`` is the measured HBM bytes per
launch of the dominant kernel, read from the committed counter summary
(profiles/<kernel>__<workload>.traffic.md) when one exists for this workload.
``cpu_baseline`` times the torch-native SDPA restatement of the same workload
(per-sequence gather + fp32 SDPA) on this host's cores, over a bounded sample of its
sequences (budgets: --cpu-seconds for the headline, --cpu-seconds-secondary for extend,
fp8 decode, verify and B=1 decode, --cpu-seconds-tertiary for the rest); the KV write's
is the numpy restatement of the pool write on one core. Prints exactly one JSON line.

    python bench.py --calibrate-copy 1024

copies a 1024 MiB float32 buffer five times with a plain elementwise kernel
(torch.neg into a second buffer: 1 GiB read, 1 GiB written per launch): the
FETCH_SIZE / WRITE_SIZE counters of those launches scale the counters of the
attention kernels to bytes.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "decode attn GB/s & % HBM roofline; extend attn TFLOP/s & % MFMA peak (1 GPU)"


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", type=int, default=1)
    p.add_argument("--kv-format", choices=("e4m3", "e5m2"), default="e4m3",
                   help="fp8 format of workload 3's KV")
    p.add_argument("--headline-only", action="store_true",
                   help="measure the headline workload only (default: every workload family)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=16.0,
                   help="CPU budget of the headline's torch-native baseline")
    p.add_argument("--cpu-seconds-secondary", type=float, default=10.0,
                   help="CPU budget of each other workload's baseline")
    p.add_argument("--cpu-seconds-tertiary", type=float, default=5.0,
                   help="CPU budget of the baselines of the head-dim, fp8 verify and KV write figures")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    return p.parse_args()


def _calibrate_copy(mib):
    import torch

    n = mib << 20
    src = torch.empty(n // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / 5
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5,
                      "GBps_read_plus_write": 2 * n / dt / 1e9}))


def _gather_ceiling(num_tokens, heads, row_bytes, steps=20):
    """Read bandwidth of a plain gather of ``num_tokens * heads`` rows of ``row_bytes``
    (libma_calibrate.so, csrc/calibrate/gather_ceiling.hip): the attainable rate of the
    KV access pattern without any attention arithmetic. Returns GB/s."""
    import ctypes

    import torch

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sglang_restomod_amd", "libma_calibrate.so")
    lib = ctypes.CDLL(path)
    lib.ma_gather_ceiling_sink_words.restype = ctypes.c_int64
    lib.ma_gather_ceiling_sink_words.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    lib.ma_gather_ceiling.restype = ctypes.c_int
    lib.ma_gather_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    pool = torch.randint(0, 256, (num_tokens * heads * row_bytes,), dtype=torch.uint8, device=dev, generator=g)
    perm = torch.randperm(num_tokens, device=dev, generator=g).to(torch.int32)
    chunks_per_wave = 4
    sink = torch.empty(lib.ma_gather_ceiling_sink_words(num_tokens, heads, chunks_per_wave), dtype=torch.int32,
                       device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run():
        rc = lib.ma_gather_ceiling(pool.data_ptr(), perm.data_ptr(), num_tokens, heads, row_bytes,
                                   chunks_per_wave, sink.data_ptr(), sink.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"ma_gather_ceiling failed ({rc})")

    _, per = _time_gpu(run, steps, 5)
    ms = statistics.median(per)
    del pool, perm, sink
    torch.cuda.empty_cache()
    return pool_bytes(num_tokens, heads, row_bytes) / (ms * 1e-3) / 1e9


def pool_bytes(num_tokens, heads, row_bytes):
    return num_tokens * heads * row_bytes


def _traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from its committed counter summary."""
    import re

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"{kernel}__{workload}.traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def _runner(w):
    """A zero-argument callable running the hot path once on workload ``w``."""
    from sglang_restomod_amd.attention.mi355x import ops

    hint = max(w.seq_lens_cpu)
    if w.mode == "decode":
        out = w.q.new_empty(w.q.shape)
        return lambda: ops.grouped_decode_forward(
            w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, softmax_scale=w.softmax_scale,
            k_scale=w.k_scale, v_scale=w.v_scale, out=out, row_index=w.req_pool_indices,
            max_seq_len_hint=hint)
    qsl = w.query_start_loc
    T = int(w.extend_lens.max())
    out = w.q.new_empty(w.q.shape)
    if w.mode == "verify":
        return lambda: ops.paged_verify_forward(
            w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, qsl, w.prefix_lens,
            max_q_per_seq=T, softmax_scale=w.softmax_scale, out=out, row_index=w.req_pool_indices,
            max_seq_len_hint=hint)
    return lambda: ops.paged_forward(
        w.q, w.k_pool, w.v_pool, w.req_to_token, w.seq_lens, qsl, w.prefix_lens, out=out, block_size=1,
        softmax_scale=w.softmax_scale, causal=True, row_index=w.req_pool_indices,
        max_seq_len_hint=hint, max_q_len_hint=T)[0]


WARMUP_MIN_S = 0.5


def _time_gpu(fn, steps, warmup):
    """Run ``warmup`` untimed steps, and more until WARMUP_MIN_S of wall time has passed
    (the GPU's clocks settle under sustained load; a few sub-millisecond calls do not get
    there), then time ``steps`` steps."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + WARMUP_MIN_S
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    # the timed steps: back to back, with nothing else on the stream
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the same number of steps again, each bracketed by HIP events on the launch stream
    # (the kernels of one call; the event markers themselves add gaps between calls, so
    # they stay out of the wall-clock loop above)
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]  # ms, kernels of one call
    return wall / steps * 1e3, per


def _cpu_baseline(w, budget_s):
    """torch-native restatement on this host's cores over a bounded sample of sequences:
    the sample grows until one pass takes about a quarter of ``budget_s``, then the median
    of up to three passes is kept. Returns (seconds, sequences, cores)."""
    import torch

    from oracle import torch_native as TN

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B = w.batch
    # the sequences in ascending order of size, so small samples stay small
    order = sorted(range(B), key=lambda b: w.seq_lens_cpu[b])
    kc, vc = w.k_pool.cpu(), w.v_pool.cpu()
    qc = w.q.cpu()
    r2t, rpi = w.req_to_token.cpu(), w.req_pool_indices.cpu()
    seq = w.seq_lens.cpu()
    pre = w.prefix_lens.cpu().tolist()
    ext = w.extend_lens.cpu().tolist()
    qsl = [0]
    for e in ext:
        qsl.append(qsl[-1] + e)

    def run(rows):
        if w.mode == "decode":
            TN.decode(qc, kc, vc, r2t, rpi, seq, softmax_scale=w.softmax_scale, k_scale=w.k_scale,
                      v_scale=w.v_scale, batch_subset=rows)
        else:
            sub_q = torch.cat([qc[qsl[b]:qsl[b + 1]] for b in rows])
            TN.extend(sub_q, kc, vc, r2t, rpi[rows], [pre[b] for b in rows], [ext[b] for b in rows],
                      softmax_scale=w.softmax_scale, k_scale=w.k_scale, v_scale=w.v_scale)

    n = 1
    while True:
        rows = sorted(order[:n])
        t0 = time.perf_counter()
        run(rows)
        t = time.perf_counter() - t0
        if n >= B or t >= budget_s / 4:
            break
        n = min(B, max(n + 1, int(n * min(8.0, max(2.0, (budget_s / 4) / max(t, 1e-3))))))
    # a whole batch that takes well under the budget (the single-sequence decode) is run
    # `inner` times per timed pass, so a pass is long enough for the clock to resolve
    inner = max(1, int((budget_s / 8) / max(t, 1e-6))) if t < budget_s / 8 else 1
    reps = max(1, min(3, int(budget_s / max(t * inner, 1e-3)) - 1))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(inner):
            run(rows)
        times.append((time.perf_counter() - t0) / inner)
    del kc, vc, qc
    return statistics.median(times), rows, cores, inner


def _graph_us_per_call(index, calls=20, replays=20):
    """Microseconds per call of workload ``index`` replayed from a captured HIP graph of
    ``calls`` back-to-back calls (as an engine's decode graph runner replays them), HIP
    events around ``replays`` replays: the GPU-side latency without the host's launch cost."""
    import torch

    from sglang_restomod_amd import workloads

    w = workloads.make(index, device=torch.device("cuda:0"))
    fn = _runner(w)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (replays * calls)
    del graph, w, fn
    torch.cuda.empty_cache()
    return us


def _cpu_kv_write(k, v, loc, slots, k_scale, v_scale, budget_s, nbytes):
    """The numpy restatement of the pool write (oracle.kv_write.set_kv_buffer, one core)
    over the same K, V and slots: median of up to three timed calls."""
    import numpy as np
    import torch

    from oracle import kv_write as KW

    kb = k.cpu().view(torch.int16).numpy().view(np.uint16)  # bf16 bit patterns
    vb = v.cpu().view(torch.int16).numpy().view(np.uint16)
    lc = loc.cpu().numpy()
    cache = np.zeros((slots,) + kb.shape[1:], dtype=np.uint8)

    def call():
        KW.set_kv_buffer(cache, lc, kb, "bf16", KW.E4M3, k_scale)
        KW.set_kv_buffer(cache, lc, vb, "bf16", KW.E4M3, v_scale)

    t0 = time.perf_counter()
    call()
    t = time.perf_counter() - t0
    times = [t]
    for _ in range(max(0, min(2, int(budget_s / max(t, 1e-3)) - 1))):
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    return {"value": round(nbytes / sec / 1e9, 5), "unit": "GB/s", "cores": 1, "kind": "port",
            "seconds_per_call": round(sec, 6),
            "sample": f"numpy restatement of the pool write (division in fp32, round to bf16, cast to e4m3) "
                      f"over the whole batch, K and V, median of {len(times)} calls of {sec:.4g} s"}


def _measure_kv_write(steps, warmup, cpu_seconds=0.0):
    """The pool write of an extend batch: the extend workload's new tokens (11,179 x 8 kv
    heads x 128, bf16 K and V) quantized into an e4m3 pool at shuffled slots."""
    import torch

    from sglang_restomod_amd import workloads
    from sglang_restomod_amd.attention.mi355x import ops

    spec = workloads.WORKLOADS[2]
    gen = torch.Generator().manual_seed(2)
    T = int(workloads.make(2, device=torch.device("cpu")).extend_lens.sum())
    H, D = spec["heads_kv"], spec["dim"]
    dev = torch.device("cuda:0")
    k = torch.randn(T, H, D, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(T, H, D, generator=gen).to(torch.bfloat16).to(dev)
    slots = 4 * T
    loc = torch.randperm(slots, generator=gen)[:T].to(dev)
    kc = torch.zeros(slots, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    fn = lambda: ops.set_kv_buffer(kc, vc, loc, k, v, 0.9, 1.1)
    wall_ms, per = _time_gpu(fn, steps, warmup)
    nbytes = 2 * T * H * D * (2 + 1) + 8 * T
    ev = statistics.mean(per)
    res = {"workload": f"kv_write_t{T}_h{H}_d{D}_bf16_to_e4m3", "mode": "kv_write",
           "ms_per_step": round(wall_ms, 5), "event_ms_mean": round(ev, 5),
           "event_ms_min": round(min(per), 5), "event_ms_median": round(statistics.median(per), 5),
           "GBps": round(nbytes / (ev * 1e-3) / 1e9, 2),
           "hbm_frac": round(nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_bytes": nbytes}
    if cpu_seconds:
        res["cpu_baseline"] = _cpu_kv_write(k, v, loc, slots, 0.9, 1.1, cpu_seconds, nbytes)
    return res


def _measure(index, steps, warmup, cpu_seconds, kv_format="e4m3"):
    """Time workload ``index`` on the GPU (wall clock over ``steps`` calls, and HIP events
    around every call on the launch stream), and its CPU baseline when ``cpu_seconds``."""
    import torch

    from sglang_restomod_amd import workloads

    w = workloads.make(index, device=torch.device("cuda:0"), kv_format=kv_format)
    fn = _runner(w)
    wall_ms, per = _time_gpu(fn, steps, warmup)
    nbytes, flops = workloads.algorithmic_bytes(w), workloads.algorithmic_flops(w)
    ev_ms = statistics.mean(per)
    res = {
        "workload": w.name,
        # profiles/<kernel>__<this>.traffic.md: the name plus the fp8 format for fp8 pools
        "profile_name": w.name + (f"_{w.kv_format}" if w.kv_format else ""),
        "mode": w.mode,
        "kv": str(w.k_pool.dtype).replace("torch.", ""),
        "ms_per_step": wall_ms,
        "event_ms_mean": ev_ms,
        "event_ms_min": min(per),
        "event_ms_median": statistics.median(per),
        "algorithmic_bytes": nbytes,
        "algorithmic_flops": flops,
        "GBps": nbytes / (ev_ms * 1e-3) / 1e9,
        "TFLOPs": flops / (ev_ms * 1e-3) / 1e12,
        "wall_GBps": nbytes / (wall_ms * 1e-3) / 1e9,
        "wall_TFLOPs": flops / (wall_ms * 1e-3) / 1e12,
        "tokens_per_s": int(w.extend_lens.sum()) / (wall_ms * 1e-3),
    }
    res["hbm_frac"] = res["GBps"] / HBM_PEAK_GBS
    res["mfma_frac"] = res["TFLOPs"] / MFMA_BF16_PEAK_TFLOPS
    if w.mode == "decode":
        from sglang_restomod_amd.attention.mi355x import ops

        res["kernel"] = ops.decode_kernel(w.batch, w.heads, w.heads_kv, w.dim, max(w.seq_lens_cpu))
    if w.mode != "extend":
        # the same number of K and V rows, gathered from random slots with no arithmetic
        row_bytes = w.dim * w.k_pool.element_size()
        tokens = 2 * int(sum(w.seq_lens_cpu))
        res["gather_ceiling_GBps"] = _gather_ceiling(tokens, w.heads_kv, row_bytes)
        res["gather_row_bytes"] = row_bytes
    if cpu_seconds:
        sec, rows, cores, inner = _cpu_baseline(w, cpu_seconds)
        sb, sf = workloads.algorithmic_bytes(w, rows), workloads.algorithmic_flops(w, rows)
        res["cpu"] = {"seconds": sec, "cores": cores, "sequences": len(rows), "of": w.batch, "inner": inner,
                      "GBps": sb / sec / 1e9, "TFLOPs": sf / sec / 1e12,
                      "tokens_per_s": sum(w.extend_lens.tolist()[b] for b in rows) / sec}
    del w, fn
    torch.cuda.empty_cache()
    return res


def _cpu_obj(r, bound_hbm):
    c = r["cpu"]
    rep = f" (each pass the mean of {c['inner']} back-to-back calls)" if c["inner"] > 1 else ""
    return {
        "value": round(c["GBps"] if bound_hbm else c["TFLOPs"], 5),
        "unit": "GB/s" if bound_hbm else "TFLOP/s",
        "cores": c["cores"],
        "kind": "port",
        "seconds_per_call": round(c["seconds"], 6),
        "sample": (f"torch-native SDPA restatement (per-sequence gather + fp32 SDPA) over the {c['sequences']} "
                   f"shortest of {c['of']} sequences, median of up to 3 passes of {c['seconds']:.4g} s{rep}; value = "
                   f"algorithmic {'bytes' if bound_hbm else 'flops'} of those sequences per second"),
    }


def _decode_kernel(r):
    """The kernel that carries a decode or verify call: the split-KV partial, or the
    any-head-dim kernel for head dims the tuned kernels do not take and for decode batches
    small enough to run as one launch (ops.decode_path)."""
    return r.get("kernel") or "splitkv_partial"


def _roofline(r, kernel, bound_hbm):
    achieved = r["GBps"] if bound_hbm else r["TFLOPs"]
    peak = HBM_PEAK_GBS if bound_hbm else MFMA_BF16_PEAK_TFLOPS
    obj = {
        "bound": "hbm" if bound_hbm else "mfma",
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": "GB/s" if bound_hbm else "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "traffic": _traffic(kernel, r["profile_name"]),
        "kernel_ms": round(r["event_ms_mean"], 5),
        "kernel_ms_min": round(r["event_ms_min"], 5),
        "kernel_ms_median": round(r["event_ms_median"], 5),
        "timing": "HIP events on the launch stream around each call ("
                  + (("any-head-dim kernel; above 512 keys per row over key pieces + merge" if r["mode"] == "decode"
                      else "any-head-dim kernel")
                     if kernel == "any_kernel" and bound_hbm
                     else "any-head-dim kernel, after the work-list plan" if kernel == "any_kernel"
                     else "split-KV partial + merge" if bound_hbm else "plan + extend kernel") + ")",
    }
    if bound_hbm:
        ceil = r["gather_ceiling_GBps"]
        obj["gather_ceiling"] = {
            "GBps": round(ceil, 1), "frac": round(r["GBps"] / ceil, 4),
            "pattern": f"the same K and V rows ({r['gather_row_bytes']} B per token and kv head) gathered from "
                       "random pool slots by a plain load kernel, measured in this run"}
    return obj


def _family(r, kernel, bound_hbm):
    """Compact object for a non-headline workload of the same JSON line."""
    obj = {
        "workload": r["workload"],
        "kv_dtype": r["kv"],
        "value": round(r["wall_GBps"] if bound_hbm else r["wall_TFLOPs"], 3),
        "unit": "GB/s" if bound_hbm else "TFLOP/s",
        "ms_per_step": round(r["ms_per_step"], 5),
        "tokens_per_s": round(r["tokens_per_s"], 1),
        "roofline": _roofline(r, kernel, bound_hbm),
    }
    if r["mode"] == "verify":
        obj["mfma_frac"] = round(r["mfma_frac"], 4)
    if "cpu" in r:
        obj["cpu_baseline"] = _cpu_obj(r, bound_hbm)
    return obj


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the attention path is measured on one GPU only; --gpus must be 1 "
                                   "(how it shards across GPUs is documented, not launched)"}))
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.calibrate_copy:
        _calibrate_copy(args.calibrate_copy)
        return
    cpu = 0 if args.no_cpu_baseline else args.cpu_seconds
    head = _measure(args.workload, args.steps, args.warmup, cpu, kv_format=args.kv_format)
    bound_hbm = head["mode"] != "extend"
    kernel = (_decode_kernel(head) if head["mode"] == "decode"
              else "splitkv_partial" if bound_hbm else "extend_kernel")
    line = {
        "metric": METRIC,
        "value": round(head["wall_GBps"] if bound_hbm else head["wall_TFLOPs"], 3),
        "unit": "GB/s" if bound_hbm else "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_s": WARMUP_MIN_S,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if "bf16" in head["workload"] or head["kv"].startswith("float8") else "fp16",
        "data": "synthetic (seeded N(0,1) q/k/v, shuffled token-pool slots)",
        "config": {"workload": head["workload"], "mode": head["mode"], "kv_dtype": head["kv"],
                   "tokens_per_s": round(head["tokens_per_s"], 1)},
        "roofline": _roofline(head, kernel, bound_hbm),
    }
    if "cpu" in head:
        line["cpu_baseline"] = _cpu_obj(head, bound_hbm)
    if not args.headline_only:
        # the other halves of the metric and the other configurations, each a compact object
        steps = max(10, args.steps // 2)
        sec_cpu = 0 if args.no_cpu_baseline else args.cpu_seconds_secondary
        if args.workload != 2:
            line["extend"] = _family(_measure(2, steps, args.warmup, sec_cpu), "extend_kernel", False)
        fp8 = {}
        for fmt in ("e4m3", "e5m2"):
            fp8[fmt] = _family(_measure(3, steps, args.warmup, sec_cpu, kv_format=fmt), "splitkv_partial", True)
        line["fp8_decode"] = fp8
        if args.workload != 4:
            line["verify"] = _family(_measure(4, steps, args.warmup, sec_cpu), "splitkv_partial", True)
        if args.workload != 0:
            # the single-sequence decode: latency-bound, so its call time in microseconds too
            r = _measure(0, max(steps, 50), args.warmup, sec_cpu)
            obj = _family(r, _decode_kernel(r), True)
            obj["us_per_call"] = round(r["event_ms_mean"] * 1e3, 2)
            obj["wall_us_per_call"] = round(r["ms_per_step"] * 1e3, 2)
            # the same call replayed from a HIP graph: no host launch cost between its kernels
            obj["graph_us_per_call"] = round(_graph_us_per_call(0), 2)
            line["decode_b1"] = obj
        ter = 0 if args.no_cpu_baseline else args.cpu_seconds_tertiary
        line["kv_write"] = _measure_kv_write(steps, args.warmup, ter)
        # the other head dims of the reference's tuned configurations: 256 on the split-KV and
        # tiled extend kernels, 512 on the any-head-dim kernel
        line["head_dim_256"] = {"decode": _family(_measure(5, steps, args.warmup, ter), "splitkv_partial", True),
                                "extend": _family(_measure(6, steps, args.warmup, ter), "extend_kernel", False)}
        line["head_dim_512"] = {"decode": _family(_measure(7, steps, args.warmup, ter), "any_kernel", True),
                                "extend": _family(_measure(8, steps, args.warmup, ter), "any_kernel", False)}
        # head dims without a tiled kernel of their own, padded onto the next one
        line["padded_head_dims"] = {"d96_extend": _family(_measure(9, steps, args.warmup, ter), "extend_kernel", False),
                                    "d192_extend": _family(_measure(10, steps, args.warmup, ter), "extend_kernel", False)}
        line["verify_fp8"] = _family(_measure(11, steps, args.warmup, ter, kv_format="e4m3"), "splitkv_partial",
                                     True)
        line["extend_fp8"] = _family(_measure(12, steps, args.warmup, ter, kv_format="e4m3"), "extend_kernel", False)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
