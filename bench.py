"""Benchmark of the MLA attention hot path on one MI355X.

Default workload (the headline one): Kimi-K2-shape absorbed-MLA paged decode,
batch 64, 64 heads, 576-dim q / latent KV, page_size 64, random
non-contiguous page table, seq_lens ~ U[1024, 8192], bf16 N(0,1) inputs.
A "step" is one layer's decode attention over the batch: one call of the
library's decode entry point (split-KV kernel, then the LSE merge kernel),
inputs resident in HBM. The same steps replayed from a HIP graph are reported
as an extra field. Two input sets
(680 MB of KV together, more than the 256 MB Infinity Cache) alternate so
every step streams its KV from HBM.

Prints one JSON line. ``value`` is the whole-step algorithmic HBM bandwidth
(TB/s); µs/layer and tokens/s are extra fields. ``roofline`` times the
dominant kernel (the split kernel) alone, 16 back-to-back launches per HIP
graph, with HIP events on its launch stream.
``cpu_baseline`` times the CPU oracle on the CPU decode workload (B=4, 16
heads, page 1, lengths U[64, 512]); ``measured_peaks`` holds a read-only HBM
stream and a bf16 MFMA loop measured on the same GPU.
Extra fields: the prefill attention batch, a long-context batch, a mixed
ragged batch, and ``layer``: whole Kimi-K2 MLA layer steps (projections,
RoPE, absorption, attention kernels, o_proj) for the same decode and prefill
batches (``--workload layer`` alone).

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mini-sglang_amd")]

HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mla_decode_kimi_k2_b64_traffic.md")
PREFILL_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mla_prefill_b4_e2048_kernel_trace.md")


def _committed_traffic(path):
    """HBM bytes per launch (copy-calibrated FETCH_SIZE + WRITE_SIZE) from a committed counter summary."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":")[1])
    return None


def _decode_workload(device, seed):
    from minisgl_amd.benchmark.inputs import make_decode_case

    return make_decode_case(64, 64, 64, len_range=(1024, 8192), device=device, seed=seed)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """Threads for the CPU oracle: the host cores this process may use (its affinity mask, or the
    OMP_NUM_THREADS share a shared GPU host gives one GPU's job), not every core of the host."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(omp))) if omp and omp.isdigit() else max(1, n)


def _cpu_baseline(case_gpu, runs: int = 10):
    """The CPU oracle (oracle/ref_mla.py, fp32 torch) on the CPU workload of the decode path: B=4,
    16 heads, page size 1, lengths U[64, 512] (warm-up, then the median of ``runs`` runs), plus one
    sample of the headline batch's first requests for scale."""
    import statistics

    import torch

    from minisgl_amd.benchmark.inputs import make_decode_case
    from oracle import ref_mla as R

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    c1 = make_decode_case(4, 16, 1, len_range=(64, 512), seed=0)
    R.mla_decode(c1.q, c1.kv_pool, c1.page_table, c1.lens)  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        R.mla_decode(c1.q, c1.kv_pool, c1.page_table, c1.lens)
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    alg1 = c1.algorithmic_bytes()

    # the headline batch's first requests, one run (about a second of CPU work)
    q, kv, pt, lens = case_gpu.q.cpu(), case_gpu.kv_pool.cpu(), case_gpu.page_table.cpu(), case_gpu.lens
    n = 8
    t0 = time.perf_counter()
    R.mla_decode(q[:n], kv, pt[:n], lens[:n])
    sec2 = time.perf_counter() - t0
    H = q.shape[1]
    pages = sum(-(-L // 64) for L in lens[:n])
    bytes2 = sum(lens[:n]) * 1152 + n * H * (576 + 512) * 2 + n * H * 4 + pages * 4 + 4 * n
    return {
        "value": alg1 / sec / 1e12,
        "unit": "TB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"CPU oracle (oracle/ref_mla.py, fp32 torch, {threads} threads) on the CPU decode workload: "
        f"B=4, 16 heads, page 1, lengths {c1.lens} ({sum(c1.lens)} KV tokens); median of {runs} runs",
        "us_per_layer": round(sec * 1e6, 1),
        "tokens_per_s": round(4 / sec, 1),
        "cpu_model": _cpu_model(),
        "host_cpu_count": os.cpu_count(),
        "headline_sample": {
            "requests": n,
            "kv_tokens": sum(lens[:n]),
            "ms": round(sec2 * 1e3, 1),
            "tb_per_s": round(bytes2 / sec2 / 1e12, 6),
            "gpu_over_cpu_note": "same batch shape as the GPU line (64 heads, page 64), first 8 requests",
        },
    }


CLOCK_WARM_S = 0.3


def _clock_warm(fn, seconds=CLOCK_WARM_S):
    """Run ``fn(i)`` back to back for ``seconds`` of wall time before a timed region (untimed).

    The GPU leaves its idle clocks over the first tens of milliseconds of load: per-launch HIP
    events put the first 100 decode layer steps after idle at 126 us on average against ~91 us in
    steady state, and the first prefill launches at 1.35-2.2 ms against ~1.22 ms. A timed region
    that followed only a few warm-up steps would measure that ramp, not the kernels."""
    import torch

    end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < end:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def bench_decode(args):
    import torch

    from minisgl_amd.benchmark.inputs import make_decode_case
    from minisgl_amd.kernel import lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sets = [_decode_workload(dev, 0)]
    # second input set: same lengths (so the same plan and work), different pages and values
    sets.append(make_decode_case(64, 64, 64, lens=sets[0].lens, device=dev, seed=100))
    case = sets[0]
    B, H, _ = case.q.shape
    ctas = lib.device_cu_count(0)
    plan_np, slots = lib.decode_plan(case.lens, case.page_size, ctas)
    plan = torch.from_numpy(plan_np).to(dev)
    ws_o, ws_lse = lib.decode_workspace(slots, H, dev)
    out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev)
    req_info = plan[ctas * lib.PLAN_CTA_INTS :]
    scale = (128 + 64) ** -0.5
    stream = torch.cuda.Stream()  # default priority

    def split(s):
        lib.mla_decode(s.q, s.kv_pool, s.page_table, s.seq_lens, plan, ctas, ws_o, ws_lse, scale, out, lse,
                       stream=stream, split_only=True)

    def merge():
        lib.mla_decode_merge(ws_o, ws_lse, req_info, out, lse, stream=stream, single_piece_final=True)

    def step(i):
        split(sets[i % 2])
        merge()

    def layer(i):  # the one-call entry point: split kernel then merge kernel, launched from C++
        c = sets[i % 2]
        lib.mla_decode(c.q, c.kv_pool, c.page_table, c.seq_lens, plan, ctas, ws_o, ws_lse, scale, out, lse,
                       stream=stream)

    def capture(fn, n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(i)
        return g

    with torch.cuda.stream(stream):
        # ---- timed: exactly args.steps layer steps, eager launches on one stream, after the clock
        # warm-up and args.warmup untimed steps
        _clock_warm(layer)
        for i in range(args.warmup):
            layer(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(args.steps):
            layer(i)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        step_ms = wall * 1e3 / args.steps
        dev_step_ms = e0.elapsed_time(e1) / args.steps

        # ---- the same steps replayed from one HIP graph (as a captured decode step), for reference;
        # a replay must equal the eager result of the same launches
        layer(0)
        stream.synchronize()
        ref_out = out.clone()
        g_check = capture(layer, 1)
        out.zero_()
        g_check.replay()
        stream.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), "graph replay differs from eager"
        # steady state: a graph of 10 steps (inputs alternating) replayed back to back between HIP events
        per_replay = 10
        g_steps = capture(layer, per_replay)
        _clock_warm(lambda i: g_steps.replay())  # the capture left the GPU idle
        replays = max(3, args.steps // per_replay)
        ga, gb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ga.record(stream)
        for _ in range(replays):
            g_steps.replay()
        gb.record(stream)
        torch.cuda.synchronize()
        graph_ms = ga.elapsed_time(gb) / (replays * per_replay)

        # ---- each kernel alone: back-to-back launches in one graph, HIP events on its stream
        per_graph = 16
        gs = capture(lambda i: split(sets[i % 2]), per_graph)
        gm = capture(lambda i: merge(), per_graph)
        reps = 4

        def timed(g):
            _clock_warm(lambda i: g.replay())
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(reps):
                g.replay()
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / (reps * per_graph)

        split_ms = timed(gs)
        merge_ms = timed(gm)

    alg_bytes = case.algorithmic_bytes()
    value_tbps = alg_bytes / (step_ms * 1e-3) / 1e12
    achieved = alg_bytes / (split_ms * 1e-3) / 1e9
    traffic = _committed_traffic(TRAFFIC_FILE)
    result = {
        "metric": "MLA decode achieved HBM TB/s + us/layer, Kimi-K2 shape, 1 MI355X",
        "value": round(value_tbps, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q and latent KV, random page table)",
        "config": {
            "workload": "Kimi-K2-shape absorbed-MLA paged decode, one layer (split-KV + LSE merge)",
            "batch": B,
            "heads": H,
            "kv_dim": 576,
            "v_dim": 512,
            "page_size": case.page_size,
            "seq_len_range": [1024, 8192],
            "kv_tokens": sum(case.lens),
            "input_sets": len(sets),
            "num_ctas": ctas,
            "partial_slots": slots,
        },
        "us_per_layer": round(step_ms * 1e3, 2),
        "us_per_layer_device": round(dev_step_ms * 1e3, 2),
        "us_per_layer_graph": round(graph_ms * 1e3, 2),
        "graph_timing": "steady state: 10-step graphs replayed back to back between HIP events",
        "tokens_per_s": round(B / (step_ms * 1e-3), 1),
        "split_kernel_us": round(split_ms * 1e3, 2),
        "merge_kernel_us": round(merge_ms * 1e3, 2),
        "kernel_timing": "each kernel alone: 64 back-to-back launches from graphs between HIP events, after "
        "the clock warm-up",
        "algorithmic_bytes_per_step": alg_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel": "mla_decode_ws_kernel (split step)",
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = _cpu_baseline(case)
    return result


MFMA_BF16_PEAK_TFLOPS = 2500.0


def bench_prefill(args):
    """Chunked MLA prefill, B=4, H=64, extend 2048 each, prefixes U[0, 8192], page 64 (one layer)."""
    import torch

    from minisgl_amd.benchmark.inputs import make_prefill_case
    from minisgl_amd.kernel import lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(0)
    prefixes = torch.randint(0, 8193, (4,), generator=g).tolist()
    case = make_prefill_case(64, 64, extends=[2048] * 4, prefixes=prefixes, device=dev, seed=0)
    T, H, _ = case.q.shape
    out = torch.empty((T, H, 128), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()
    scale = (128 + 64) ** -0.5

    def layer():
        lib.mla_prefill(case.q, case.k_pool, case.v_pool, case.page_table, case.cu_seqlens_q, case.seq_lens_k,
                        scale, out, lse, stream=stream)

    steps = max(1, args.steps // 2)
    with torch.cuda.stream(stream):
        _clock_warm(lambda i: layer())
        for _ in range(max(1, args.warmup // 2)):
            layer()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            layer()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    step_ms = wall * 1e3 / steps
    kern_ms = e0.elapsed_time(e1) / steps
    flops = case.flops()
    achieved = flops / (kern_ms * 1e-3) / 1e12
    res = {
        "workload": "MLA chunked prefill, one layer: B=4, H=64, extend 2048, prefix U[0,8192], qk 192, v 128, page 64",
        "prefixes": prefixes,
        "us_per_layer": round(step_ms * 1e3, 1),
        "kernel_us": round(kern_ms * 1e3, 1),
        "tokens_per_s": round(T / (step_ms * 1e-3), 1),
        "tflops": round(achieved, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": _committed_traffic(PREFILL_TRAFFIC_FILE)},
        "algorithmic_flops": flops,
    }
    del case
    torch.cuda.empty_cache()
    if args.no_extra:
        return res
    # the same batch through the backend over a latent-only pool: store the chunk, gather every key,
    # decompress per head (one GEMM), the prefill kernel; at page 64 and at the reference's default 1
    from minisgl_amd.benchmark.layer import BackendPrefill

    lens = [P + 2048 for P in prefixes]
    keys = sum(lens)
    decomp_flops = keys * 2 * 512 * H * 256
    res["from_latent_pool"] = {"keys_decompressed": keys, "decompress_gflop": round(decomp_flops / 1e9, 1)}
    for ps in (64, 1):
        bp = BackendPrefill(lens, [2048] * 4, ps, dev)
        ms = _time_device(bp, stream, max(2, args.steps // 10), 2)
        res["from_latent_pool"][f"page_{ps}_us_per_layer"] = round(ms * 1e3, 1)
        bp.close()
        del bp
        torch.cuda.empty_cache()
    return res


class _DecodeCall:
    """Plan, workspace and outputs of one decode batch; ``__call__`` is one layer's one-call decode."""

    def __init__(self, case, dev):
        import torch

        from minisgl_amd.kernel import lib

        self.lib, self.case = lib, case
        B, H, _ = case.q.shape
        self.ctas = lib.device_cu_count(0)
        plan_np, self.slots = lib.decode_plan(case.lens, case.page_size, self.ctas)
        self.plan = torch.from_numpy(plan_np).to(dev)
        self.ws_o, self.ws_lse = lib.decode_workspace(self.slots, H, dev)
        self.out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty((B, H), dtype=torch.float32, device=dev)

    def __call__(self, stream):
        c = self.case
        self.lib.mla_decode(c.q, c.kv_pool, c.page_table, c.seq_lens, self.plan, self.ctas, self.ws_o, self.ws_lse,
                            (128 + 64) ** -0.5, self.out, self.lse, stream=stream)


class _PrefillCall:
    def __init__(self, case, dev):
        import torch

        from minisgl_amd.kernel import lib

        self.lib, self.case = lib, case
        T, H, _ = case.q.shape
        self.out = torch.empty((T, H, 128), dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty((T, H), dtype=torch.float32, device=dev)

    def __call__(self, stream):
        c = self.case
        self.lib.mla_prefill(c.q, c.k_pool, c.v_pool, c.page_table, c.cu_seqlens_q, c.seq_lens_k, (128 + 64) ** -0.5,
                             self.out, self.lse, stream=stream)


def _time_device(fn, stream, steps, warmup):
    """Mean device time (ms) of ``fn()`` over ``steps`` launches on ``stream`` (HIP events on that stream),
    after the clock warm-up and ``warmup`` untimed launches."""
    import torch

    with torch.cuda.stream(stream):
        _clock_warm(lambda i: fn())
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def bench_page_size_one(args):
    """The decode workload's batch (same lengths) in a pool of 1-token pages, the reference's default
    page size (python/minisgl/engine/config.py:25): one-call step and split kernel alone."""
    import torch

    from minisgl_amd.benchmark.inputs import make_decode_case
    from minisgl_amd.benchmark.layer import decode_lens

    dev = torch.device("cuda:0")
    lens = decode_lens(64, seed=0)  # the lengths _decode_workload(dev, 0) draws
    case = make_decode_case(64, 64, 1, lens=lens, device=dev, seed=0)
    call = _DecodeCall(case, dev)
    stream = torch.cuda.Stream()
    ms = _time_device(lambda: call(stream), stream, args.steps, args.warmup)
    c = case

    def split():
        call.lib.mla_decode(c.q, c.kv_pool, c.page_table, c.seq_lens, call.plan, call.ctas, call.ws_o, call.ws_lse,
                            (128 + 64) ** -0.5, call.out, call.lse, stream=stream, split_only=True)

    split_ms = _time_device(split, stream, args.steps, args.warmup)
    alg = case.algorithmic_bytes()
    return {
        "workload": "Kimi-K2-shape decode batch of the headline line (same lengths), page size 1",
        "us_per_layer": round(ms * 1e3, 2),
        "tb_per_s": round(alg / (ms * 1e-3) / 1e12, 4),
        "split_kernel_us": round(split_ms * 1e3, 2),
        "partial_slots": call.slots,
    }


def bench_long_context(args):
    """Long-context split-KV decode: B=8, H=64, lengths U[32768, 131072], page 64 (one layer)."""
    import torch

    from minisgl_amd.benchmark.inputs import make_decode_case

    dev = torch.device("cuda:0")
    case = make_decode_case(8, 64, 64, len_range=(32768, 131072), device=dev, seed=0)
    call = _DecodeCall(case, dev)
    stream = torch.cuda.Stream()
    ms = _time_device(lambda: call(stream), stream, max(2, args.steps // 5), max(1, args.warmup // 5))
    alg = case.algorithmic_bytes()
    res = {
        "workload": "long-context absorbed-MLA decode, one layer: B=8, H=64, seq U[32768,131072], page 64",
        "kv_tokens": sum(case.lens),
        "partial_slots": call.slots,
        "us_per_layer": round(ms * 1e3, 1),
        "tb_per_s": round(alg / (ms * 1e-3) / 1e12, 3),
        "hbm_frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
    }
    del case, call
    torch.cuda.empty_cache()
    return res


def bench_mixed(args):
    """Ragged batch sharing radix prefixes: 32 decode requests (ctx U[512,16384]) + 4 prefill chunks of
    1024 tokens on 2048-token shared prefixes (8 groups), 64 heads, page 64 (one layer).

    Reported three ways: each half alone, both on one stream, and the two halves on two streams
    (HBM-bound decode beside MFMA-bound prefill)."""
    import torch

    from minisgl_amd.benchmark.inputs import make_mixed_case

    dev = torch.device("cuda:0")
    m = make_mixed_case(32, 4, 64, 64, (512, 16384), 1024, 2048, 8, device=dev, seed=0)
    dec, pre = _DecodeCall(m.decode, dev), _PrefillCall(m.prefill, dev)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    steps, warm = max(2, args.steps // 5), max(1, args.warmup // 5)
    dec_ms = _time_device(lambda: dec(s1), s1, steps, warm)
    pre_ms = _time_device(lambda: pre(s1), s1, steps, warm)
    seq_ms = _time_device(lambda: (dec(s1), pre(s1)), s1, steps, warm)

    def both():  # fork s2 off s1, join back
        ev = torch.cuda.Event()
        ev.record(s1)
        s2.wait_event(ev)
        pre(s2)
        dec(s1)
        ev2 = torch.cuda.Event()
        ev2.record(s2)
        s1.wait_event(ev2)

    par_ms = _time_device(both, s1, steps, warm)
    # roofline of the step: decode bytes (every page a decode row reads, counted once per row =
    # logical, or once per distinct page = unique: the shared prefix pages are read by several rows)
    # at 8 TB/s plus the prefill's unmasked FLOPs at 2.5 PFLOP/s
    d = m.decode
    H = d.q.shape[1]
    small = d.q.shape[0] * H * (576 + 512) * 2 + d.q.shape[0] * H * 4 + 4 * d.q.shape[0]
    logical = sum(d.lens) * 1152 + sum(-(-L // 64) for L in d.lens) * 4 + small
    seen, unique_tokens = set(), 0
    for b, L in enumerate(d.lens):
        row = d.page_table[b].tolist()
        for j in range(-(-L // 64)):
            if row[j] not in seen:
                seen.add(row[j])
                unique_tokens += min(64, L - 64 * j)
    unique = unique_tokens * 1152 + sum(-(-L // 64) for L in d.lens) * 4 + small
    flops = m.prefill.flops()
    t_roof_us = (unique / (HBM_PEAK_GBPS * 1e9) + flops / (MFMA_BF16_PEAK_TFLOPS * 1e12)) * 1e6
    res = {
        "workload": "mixed ragged batch, one layer: 32 decode (ctx U[512,16384]) + 4 prefill chunks of 1024 on "
        "2048-token shared prefixes (8 groups), H=64, page 64",
        "decode_us": round(dec_ms * 1e3, 1),
        "prefill_us": round(pre_ms * 1e3, 1),
        "one_stream_us_per_layer": round(seq_ms * 1e3, 1),
        "two_streams_us_per_layer": round(par_ms * 1e3, 1),
        "tokens_per_layer": len(m.decode.lens) + sum(m.prefill.extends),
        "decode_bytes_logical": logical,
        "decode_bytes_unique": unique,
        "prefill_flops": flops,
        "t_roof_us": round(t_roof_us, 1),
        "roofline_frac_one_stream": round(t_roof_us / (seq_ms * 1e3), 4),
        "roofline_frac_two_streams": round(t_roof_us / (par_ms * 1e3), 4),
        "t_roof_formula": "unique decode bytes / 8 TB/s + prefill unmasked FLOPs / 2.5 PFLOP/s",
    }
    del m, dec, pre
    torch.cuda.empty_cache()
    return res


def bench_layer(args):
    """Whole Kimi-K2-shape MLA layer steps (projections + RoPE + absorption + HIP attention + o_proj):
    decode over the headline batch and prefill over the prefill batch, two layers alternating."""
    import torch

    from minisgl_amd.benchmark import layer as LB

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    res = {"workload": "Kimi-K2 MLA attention layer (H=64, hidden 7168, q_lora 1536, YaRN), projections through "
           "hipBLASLt, attention through the HIP kernels; two layers alternate"}

    lens = LB.decode_lens()
    b = LB.LayerBench("decode", lens, [1] * len(lens), dev)
    n = [0]

    def dec_step():
        b.step(n[0])
        n[0] += 1

    ms = _time_device(dec_step, stream, max(4, args.steps // 2), max(2, args.warmup // 2))
    graphs = b.capture(stream)

    def replay():
        graphs[n[0] % 2].replay()
        n[0] += 1

    g_ms = _time_device(replay, stream, max(4, args.steps // 2), max(2, args.warmup // 2))
    H = b.cfg.attn.num_heads
    kv_bytes = sum(lens) * 576 * 2
    attn_flops = sum(lens) * H * 2 * (576 + 512)
    res["decode"] = {"batch": len(lens), "kv_tokens": sum(lens), "eager": LB.summary(b, ms, attn_flops, kv_bytes),
                     "graph": LB.summary(b, g_ms, attn_flops, kv_bytes)}
    del graphs
    b.close()
    del b
    torch.cuda.empty_cache()

    g = torch.Generator().manual_seed(0)
    prefixes = torch.randint(0, 8193, (4,), generator=g).tolist()
    extends = [2048] * 4
    b = LB.LayerBench("prefill", [P + E for P, E in zip(prefixes, extends)], extends, dev)
    n[0] = 0

    def pre_step():
        b.step(n[0])
        n[0] += 1

    ms = _time_device(pre_step, stream, max(2, args.steps // 10), max(2, args.warmup // 5))
    attn_flops = sum(E * P + E * (E + 1) // 2 for E, P in zip(extends, prefixes)) * H * 2 * (192 + 128)
    kv_bytes = sum(P + E for P, E in zip(prefixes, extends)) * H * (192 + 128) * 2
    res["prefill"] = {"batch": 4, "prefixes": prefixes, "extend": 2048, **LB.summary(b, ms, attn_flops, kv_bytes)}
    b.close()
    del b
    torch.cuda.empty_cache()
    return res


def bench_peaks(args):
    """Measured peaks alone: the read-only HBM stream and the bf16 MFMA loop."""
    import torch

    from minisgl_amd.benchmark import peaks
    from minisgl_amd.kernel import lib

    torch.cuda.set_device(0)
    cus = lib.device_cu_count(0)
    return {"hbm_read": peaks.hbm_read(cus), "mfma_bf16": peaks.mfma_bf16(cus)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode", choices=["decode", "prefill", "long", "mixed", "layer", "peaks"])
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill summary of the decode line")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the long-context and mixed-batch summaries and the prefill-from-latent-pool timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured HBM-read and MFMA peaks")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); multi-GPU runs are not part "
              "of this build", file=sys.stderr)
        sys.exit(2)
    one = {"prefill": bench_prefill, "long": bench_long_context, "mixed": bench_mixed, "layer": bench_layer,
           "peaks": bench_peaks}
    if args.workload in one:
        print(json.dumps(one[args.workload](args)))
        return
    res = bench_decode(args)
    if not args.no_peaks:
        from minisgl_amd.benchmark import peaks
        from minisgl_amd.kernel import lib

        cus = lib.device_cu_count(0)
        res["measured_peaks"] = {"hbm_read": peaks.hbm_read(cus), "mfma_bf16": peaks.mfma_bf16(cus)}
        res["roofline"]["frac_of_measured_read_peak"] = round(
            res["roofline"]["achieved"] / 1e3 / res["measured_peaks"]["hbm_read"]["tb_per_s"], 4)
    if not args.no_prefill:
        res["prefill"] = bench_prefill(args)
    if not args.no_extra:
        res["page_size_1"] = bench_page_size_one(args)
        res["long_context"] = bench_long_context(args)
        res["mixed"] = bench_mixed(args)
        res["layer"] = bench_layer(args)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
