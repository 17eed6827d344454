"""Benchmark of the affine-quantized matmul path on one MI355X.

Headline (the JSON line's `value`): mx.quantized_matmul as a decode GEMV,
4-bit, group 64, x bf16 [1, 3584] against W [18944, 3584] -- the
K=3584, N=18944 point of the quantized GEMM sweep, in HBM GB/s of algorithmic
traffic (packed codes + scales + biases + x + y).  16 weight replicas (611 MB,
more than the 256 MB Infinity Cache) are used in rotation so every launch
streams its weights from HBM; one step is one pass over them (16 launches,
each on a different replica), so even a short run times hundreds of launches.
The timed steps are replayed from a HIP graph so the GPU runs them back to
back; HIP events on the launch stream bracket the timed region.

Also reported: the expert GEMMs of an MoE layer's prefill (gather_qmm over
32768 expert-sorted (token, expert) pairs at the Qwen3-30B-A3B shape), the
full sweep M in {1,16,128,2048,8192} x (K,N) in
{(3584,18944), (18944,3584), (3584,4608)} x bits {4,8} (GB/s, TFLOP/s and the
fraction of the bounding roofline; for 4-bit M >= 128 also a dense bf16 GEMM
of the same shape through torch.matmul, for scale), greedy decode of the
Qwen2.5-7B-shaped 4-bit model (random init) at batch 1 and 32 in tokens/s,
the read-only HBM floor (one launch reading the same bytes), and the CPU
baseline: a vectorised float32 restatement of MLX's CPU quantized_matmul loop
(not MLX, which is not installed) on every host thread the box allots, on a
bounded sample of the headline workload.

    python bench.py [--steps 256] [--warmup 32] [--no-sweep] [--no-cpu] [--no-decode]
    python bench.py --profile   # eager launches + a copy kernel, for rocprofv3
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
RIDGE = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # FLOP per byte
METRIC = "decode tok/s (7B-shape 4-bit, bs=1/32); qmv HBM GB/s and qmm TFLOPS vs peak"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmv_4bit_K3584_N18944_traffic.txt")


def alg_bytes(M: int, N: int, K: int, bits: int, group_size: int = 64) -> int:
    """Packed codes + bf16 scales/biases + bf16 x + bf16 y."""
    return N * K * bits // 8 + N * (K // group_size) * 4 + 2 * M * K + 2 * M * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64,
                    help="timed steps; a step is one pass over the weight replicas")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--replicas", type=int, default=16)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile", action="store_true",
                    help="eager launches of the headline kernel + a 128 MiB copy (rocprofv3 runs)")
    ap.add_argument("--profile-prefill-attention", default=None, metavar="B,T,START,HEADS,KV",
                    help="only launch the paged prefill attention (B rows of T new tokens over "
                         "START cached positions, page size 16) warmup + steps times, for "
                         "rocprofv3")
    ap.add_argument("--profile-shape", default=None, metavar="M,K,N,BITS",
                    help="eager launches of quantized_matmul at one shape (rocprofv3 runs)")
    ap.add_argument("--profile-gather", action="store_true",
                    help="eager launches of the MoE-prefill expert GEMMs (rocprofv3 runs)")
    ap.add_argument("--trace-qmv", action="store_true",
                    help="per-wave timeline of the headline GEMV (mq_qmv_trace): one traced "
                         "launch after 15 plain ones, in a graph")
    ap.add_argument("--decode-only", type=int, default=None, metavar="BATCH",
                    help="only one decode benchmark: 7B at batch 1 or 32, or the MoE model "
                         "at batch 8 (rocprofv3 runs)")
    return ap.parse_args()


def trace_qmv(mq, torch, count: int = 16, replays: int = 20):
    """Per-wave timeline of the headline GEMV (4-bit, K=3584, N=18944, M=1).

    A HIP graph holds count - 1 plain launches and one traced launch
    (mq_qmv_trace: the same kernel, with every wave's constant-clock time at
    entry, after its block's prologue barrier and after its store, and its
    CU), each on its own weight replica; after `replays` replays the last
    traced launch is summarised: phase-time percentiles from the first wave's
    entry, the last wave end on CUs by how many waves they ran, the blocks by
    dispatch order, waves in flight per 0.25 us, and the part of the per-launch
    time outside [first entry, last end] (dispatch and completion)."""
    import ctypes

    import numpy as np

    K, N, bits = 3584, 18944, 4
    reps = make_replicas(mq, torch, N, K, bits, count, seed=0)
    x = torch.randn(1, K, generator=torch.Generator(device="cuda:0").manual_seed(1),
                    device="cuda:0").to(torch.bfloat16)
    y = torch.empty(count, N, dtype=torch.bfloat16, device="cuda:0")
    waves = (N + 15) // 16 * 4
    trace = torch.zeros(waves * 4, dtype=torch.int64, device="cuda:0")
    L = mq._lib.lib()

    def launch(i):
        wq, s, b = reps[i % count]
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        if i % count == count - 1:
            mq._lib.check(L.mq_qmv_trace(x.data_ptr(), wq.data_ptr(), s.data_ptr(), b.data_ptr(),
                                         y[i % count].data_ptr(), N, K, trace.data_ptr(),
                                         ctypes.c_size_t(trace.numel()), st), "qmv_trace")
        else:
            mq._lib.check(L.mq_quantized_matmul(x.data_ptr(), wq.data_ptr(), s.data_ptr(),
                                                b.data_ptr(), None, y[i % count].data_ptr(), 1, N,
                                                K, 64, bits, 1, st), "quantized_matmul")

    ms, _ = time_graph(torch, launch, count, warmup=count, reps=replays)
    ref = mq.quantized_matmul(x, *reps[count - 1], transpose=True, group_size=64, bits=bits)
    assert torch.equal(y[count - 1], ref[0]), "traced GEMV differs from quantized_matmul"
    a = trace.cpu().numpy().reshape(waves, 4).astype(np.int64)
    t = (a[:, :3] - a[:, 0].min()) * 0.01  # us (10 ns ticks)
    hw = a[:, 3]
    cu = (((hw >> 32) & 0xF) * 1000 + ((hw >> 13) & 0x7) * 100 + ((hw >> 12) & 1) * 16
          + ((hw >> 8) & 0xF))
    keys, inv, cnt = np.unique(cu, return_inverse=True, return_counts=True)
    cu_end = np.zeros(len(keys))
    np.maximum.at(cu_end, inv, t[:, 2])
    pct = lambda v: [round(float(q), 2) for q in np.percentile(v, [0, 10, 50, 90, 100])]
    blk = np.arange(waves) // 4
    nb = waves // 4
    by_order = []
    for lo in range(0, nb, 256):
        m = (blk >= lo) & (blk < min(nb, lo + 256))
        by_order.append({"blocks": [lo, int(min(nb, lo + 256)) - 1],
                         "entry_median_us": round(float(np.median(t[m, 0])), 2),
                         "prologue_median_us": round(float(np.median(t[m, 1])), 2),
                         "end_median_us": round(float(np.median(t[m, 2])), 2),
                         "end_max_us": round(float(t[m, 2].max()), 2)})
    grid = np.arange(0.0, float(t[:, 2].max()) + 0.25, 0.25)
    span = float(t[:, 2].max())
    return {
        "shape": {"M": 1, "K": K, "N": N, "bits": bits, "blocks": nb, "waves": waves,
                  "cus": int(len(keys))},
        "us_per_launch": round(ms * 1e3, 3),
        "span_first_entry_to_last_end_us": round(span, 3),
        "outside_waves_us": round(ms * 1e3 - span, 3),
        "percentiles_us_0_10_50_90_100": {"entry": pct(t[:, 0]), "prologue_done": pct(t[:, 1]),
                                          "end": pct(t[:, 2]), "wave_duration": pct(t[:, 2] - t[:, 0])},
        "cu_last_end_by_waves_per_cu": {
            str(int(c)): {"cus": int((cnt == c).sum()),
                          "mean_us": round(float(cu_end[cnt == c].mean()), 2),
                          "min_us": round(float(cu_end[cnt == c].min()), 2),
                          "max_us": round(float(cu_end[cnt == c].max()), 2)}
            for c in np.unique(cnt)},
        "blocks_by_dispatch_order": by_order,
        "waves_in_flight_per_0.25us": [int(((t[:, 0] <= g) & (t[:, 2] > g)).sum()) for g in grid],
    }


def make_replicas(mq, torch, N, K, bits, count, seed, group_size=64):
    """`count` independent quantized copies of W ~ N(0, 0.02), cast to bf16, quantized on GPU."""
    gen = torch.Generator(device="cuda:0")
    out = []
    for r in range(count):
        gen.manual_seed(seed + r)
        w = (torch.randn(N, K, generator=gen, device="cuda:0") * 0.02).to(torch.bfloat16)
        out.append(mq.quantize(w, group_size, bits))
        del w
    return out


SETTLE_S = 0.2  # untimed graph replays before a timed region


def time_graph(torch, launch, n_launch: int, warmup: int, reps: int = 1):
    """Capture `n_launch` launches (launch(i)) in a HIP graph; return ms per launch.

    After `warmup` eager launches the graph is replayed untimed for SETTLE_S
    seconds: the first milliseconds of GPU work in a process run ~12 % slower
    (clocks still rising), which a handful of warm-up launches do not cover.
    """
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_launch):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    settle_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < settle_end:
        g.replay()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    ms = start.elapsed_time(end)
    del g
    return ms / (n_launch * reps), wall / (n_launch * reps)


def read_traffic():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _host_cpu():
    """Model name of the host CPU, from /proc/cpuinfo (what lscpu prints)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args, orc, wq, s, b, x, N, K, bits):
    """The float32 CPU loop on a bounded sample: as many calls of the headline
    GEMV as fit in --cpu-seconds, on every thread this process may use
    (its CPU affinity, capped by OMP_NUM_THREADS, which the GPU boxes set to
    their per-GPU CPU share)."""
    affinity = len(os.sched_getaffinity(0))
    threads = affinity
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = max(1, min(threads, int(os.environ["OMP_NUM_THREADS"])))
    orc.qmm_f32_lanes(x, wq, s, b, 64, bits, threads=threads)  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        orc.qmm_f32_lanes(x, wq, s, b, 64, bits, threads=threads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or calls >= 200000:
            break
    gbs = alg_bytes(1, N, K, bits) * calls / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "label": "restatement, not MLX",
            "host": {"cpu": _host_cpu(), "nproc": os.cpu_count(), "affinity": affinity,
                     "omp_num_threads": os.environ.get("OMP_NUM_THREADS")},
            "sample": f"{calls} calls ({el:.1f} s) of the 4-bit K={K} N={N} M=1 qmv: a float32 "
                      "restatement of MLX's CPU quantized_matmul loop (w = s*q + b, x*w summed "
                      "in 16 float32 lanes per output), gcc -O3 AVX2/FMA, OpenMP over rows"}


def hbm_floor(mq, torch, nbytes: int, count: int = 16):
    """What one launch of a plain streaming kernel of the GEMV's size achieves:
    `read`, a read-only kernel (mq_hbm_read) over `nbytes`, and `copy`, a device
    copy moving `nbytes` in total (half read, half written); `count` rotating
    buffers so every launch reads from HBM."""
    import ctypes

    L = mq._lib.lib()
    nbytes -= nbytes % 16
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").fill_(i) for i in range(count)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def read(i):
        mq._lib.check(L.mq_hbm_read(ctypes.c_void_p(bufs[i % count].data_ptr()),
                                    ctypes.c_size_t(nbytes), ctypes.c_void_p(sink.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                      "hbm_read")

    rms, _ = time_graph(torch, read, 256, warmup=8)
    del bufs
    half = nbytes // 4  # bf16 elements per direction
    srcs = [torch.empty(half, dtype=torch.bfloat16, device="cuda:0").fill_(i) for i in range(count)]
    dst = torch.empty(half, dtype=torch.bfloat16, device="cuda:0")
    cms, _ = time_graph(torch, lambda i: dst.copy_(srcs[i % count]), 256, warmup=8)
    del srcs, dst
    return {"read": {"kind": "read-only kernel (mq_hbm_read), one launch per buffer",
                     "bytes": nbytes, "us": round(rms * 1e3, 3),
                     "GBps": round(nbytes / (rms * 1e-3) / 1e9, 1)},
            "copy": {"kind": "device copy (torch copy_), one launch per step", "bytes": 4 * half,
                     "us": round(cms * 1e3, 3), "GBps": round(4 * half / (cms * 1e-3) / 1e9, 1)}}


def _weight_bytes(model, batch: int) -> int:
    """Bytes of the quantized weights a decode step streams: every linear (not
    the embedding, of which a step reads one row per sequence) and, for an
    expert MLP, the expected number of distinct experts that `batch` tokens
    route to, E * (1 - (1 - k/E)^batch) per layer (uniform routing)."""
    def nbytes(*ts):
        return sum(t.numel() * t.element_size() for t in ts if t is not None)

    total = 0
    for layer in model.layers:
        for ql in (layer.qkv, layer.o, layer.gate_up, layer.down):
            if ql is not None:
                total += nbytes(ql.wq, ql.scales, ql.biases, ql.bias)
        if layer.moe is not None:
            m = layer.moe
            E, k = m.num_experts, m.top_k
            per_expert = sum(nbytes(qe.wq, qe.scales, qe.biases) for qe in (m.gate_up, m.down)) / E
            total += nbytes(m.gate.wq, m.gate.scales, m.gate.biases)
            total += int(E * (1 - (1 - k / E) ** batch) * per_expert)
    head = model.lm_head if model.lm_head is not None else model.embed
    return total + nbytes(head.wq, head.scales, head.biases)


def decode_bench(torch, batch: int, prompt_len: int, n_new: int, prefix_len: int = 0,
                 model_name: str = "qwen25_7b"):
    """Greedy decode of a 4-bit random-init model (Qwen2.5-7B shape, or the
    Qwen3-30B-A3B MoE shape): prefill `prompt_len` tokens per row (the first
    `prefix_len` shared by every row and prefilled once into shared pages),
    then `n_new` graph-replayed decode steps over the paged KV cache (pages of
    16)."""
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = getattr(q2.Qwen2Config, model_name)(bits=4)
    model = q2.Qwen2Model.random(cfg, seed=0, device="cuda:0")
    gen = torch.Generator(device="cuda:0").manual_seed(2)
    prompt = torch.randint(0, cfg.vocab_size, (batch, prompt_len), generator=gen, device="cuda:0")
    if prefix_len:
        prompt[:, :prefix_len] = prompt[0, :prefix_len]
    model.generate(prompt[:, :32], 4, prefix_len=16 if prefix_len else 0)  # warm-up
    torch.cuda.synchronize()
    cache = model.new_cache(batch, prompt_len + n_new, prefix_len)
    t0 = time.perf_counter()
    if prefix_len:
        model.prefill(prompt[:1, :prefix_len], cache, rows=torch.zeros(1, dtype=torch.long))
    logits = model.prefill(prompt[:, prefix_len:], cache, start=prefix_len)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    cos, sin = q2.rope_tables(cfg, cache.capacity, "cuda:0")
    tok = q2.greedy_tokens(logits)
    pos = torch.full((batch,), prompt_len, dtype=torch.int64, device="cuda:0")
    def step():
        # one greedy step in the graph: the logits, the next tokens fed back,
        # the positions advanced
        lg = model.decode_step(tok, pos, cache, cos, sin)
        tok.copy_(q2.greedy_tokens(lg))
        pos.add_(1)
        return lg

    tok0, pos0 = tok.clone(), pos.clone()
    g, static_logits = model._capture(step)  # its warm-up runs one step: undo its feedback
    tok.copy_(tok0)
    pos.copy_(pos0)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(n_new):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    wbytes = _weight_bytes(model, batch)
    kv_per_pos = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2
    step_bytes = wbytes + batch * kv_per_pos * (prompt_len + (n_new + 1) / 2)
    step_s = ms * 1e-3 / n_new
    del model, cache, g
    torch.cuda.empty_cache()
    return {"model": model_name, "batch": batch, "prompt_len": prompt_len,
            "shared_prefix": prefix_len,
            "new_tokens": n_new, "page_size": 16,
            "decode_tok_s": round(batch * n_new / (ms * 1e-3), 1),
            "ms_per_decode_step": round(ms / n_new, 3),
            "hbm_bytes_per_step": int(step_bytes),
            "hbm_frac": round(step_bytes / step_s / 8e12, 3),
            "prefill_ms": round(t_prefill * 1e3, 1),
            "prefill_tok_s": round(batch * (prompt_len - prefix_len) / t_prefill, 1)}


def sweep(mq, torch):
    rows = []
    for (K, N) in ((3584, 18944), (18944, 3584), (3584, 4608)):
        for bits in (4, 8):
            wbytes = alg_bytes(0, N, K, bits)
            n_rep = max(1, min(16, math.ceil(640e6 / wbytes)))
            reps = make_replicas(mq, torch, N, K, bits, n_rep, seed=100)
            wdt = None
            if bits == 4:
                wq0, s0, b0 = reps[0]
                wdt = mq.dequantize(wq0, s0, b0, 64, bits).t().contiguous()  # [K, N] bf16
            for M in (1, 16, 128, 2048, 8192):
                gen = torch.Generator(device="cuda:0").manual_seed(1)
                x = torch.randn(M, K, generator=gen, device="cuda:0").to(torch.bfloat16)
                flops = 2.0 * M * N * K
                # a graph replay has a fixed start-up latency (~0.15 ms): replay
                # enough launches that it stays under 1 % of the timed region
                n_launch, replays = (64, 4) if flops < 2e11 else (8, 4)

                def launch(i, x=x, reps=reps):
                    wq, s, b = reps[i % len(reps)]
                    mq.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits=bits)

                ms, _ = time_graph(torch, launch, n_launch, warmup=2, reps=replays)
                by = alg_bytes(M, N, K, bits)
                gbs = by / (ms * 1e-3) / 1e9
                tfl = flops / (ms * 1e-3) / 1e12
                bound = "hbm" if flops / by < RIDGE else "mfma"
                frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tfl / BF16_PEAK_TFLOPS
                row = {"M": M, "K": K, "N": N, "bits": bits, "us": round(ms * 1e3, 2),
                       "GBps": round(gbs, 1), "TFLOPs": round(tfl, 2), "bound": bound,
                       "frac": round(frac, 4)}
                if bits == 4 and M >= 128:
                    # For scale: a dense bf16 GEMM of the same shape through
                    # torch.matmul (hipBLASLt) on the dequantized weights.
                    dms, _ = time_graph(torch, lambda i, x=x: torch.matmul(x, wdt), n_launch,
                                        warmup=2, reps=replays)
                    row["dense_bf16_us"] = round(dms * 1e3, 2)
                    row["dense_bf16_TFLOPs"] = round(flops / (dms * 1e-3) / 1e12, 2)
                rows.append(row)
                del x
            del reps, wdt
            torch.cuda.empty_cache()
    return rows


def group_sweep(mq, torch):
    """Group sizes 32 and 128 (group 64 is the sweep above) on the 7B gate|up
    shape at 4 bits: the one-row GEMV, the skinny GEMM and the large-M GEMM
    index their scales per group at every size."""
    rows = []
    K, N, bits = 3584, 18944, 4
    for gs in (32, 128):
        wbytes = alg_bytes(0, N, K, bits, gs)
        reps = make_replicas(mq, torch, N, K, bits, max(1, min(16, math.ceil(640e6 / wbytes))),
                             seed=300, group_size=gs)
        for M in (1, 16, 128, 2048):
            gen = torch.Generator(device="cuda:0").manual_seed(1)
            x = torch.randn(M, K, generator=gen, device="cuda:0").to(torch.bfloat16)
            flops = 2.0 * M * N * K
            n_launch = 64 if flops < 2e11 else 8

            def launch(i, x=x, reps=reps, gs=gs):
                wq, s, b = reps[i % len(reps)]
                mq.quantized_matmul(x, wq, s, b, transpose=True, group_size=gs, bits=bits)

            ms, _ = time_graph(torch, launch, n_launch, warmup=2, reps=4)
            by = alg_bytes(M, N, K, bits, gs)
            gbs, tfl = by / (ms * 1e-3) / 1e9, flops / (ms * 1e-3) / 1e12
            bound = "hbm" if flops / by < RIDGE else "mfma"
            rows.append({"group_size": gs, "M": M, "K": K, "N": N, "bits": bits,
                         "us": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                         "TFLOPs": round(tfl, 2), "bound": bound,
                         "frac": round(gbs / HBM_PEAK_GBS if bound == "hbm"
                                       else tfl / BF16_PEAK_TFLOPS, 4)})
            del x
        del reps
        torch.cuda.empty_cache()
    return rows


def bits_sweep(mq, torch):
    """Codes of 2, 3, 5 and 6 bits on the headline shape, one row: the
    one-row GEMV reads them at their width (32 codes = `bits` words); bytes
    counted at that width.  The 4- and 8-bit rows are the sweep's."""
    rows = []
    K, N, M = 3584, 18944, 1
    for bits in (2, 3, 5, 6):
        wbytes = alg_bytes(0, N, K, bits)
        reps = make_replicas(mq, torch, N, K, bits, max(1, min(16, math.ceil(640e6 / wbytes))),
                             seed=400)
        gen = torch.Generator(device="cuda:0").manual_seed(1)
        x = torch.randn(M, K, generator=gen, device="cuda:0").to(torch.bfloat16)

        def launch(i, x=x, reps=reps, bits=bits):
            wq, s, b = reps[i % len(reps)]
            mq.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits=bits)

        ms, _ = time_graph(torch, launch, 64, warmup=2, reps=4)
        by = alg_bytes(M, N, K, bits)
        gbs = by / (ms * 1e-3) / 1e9
        rows.append({"bits": bits, "M": M, "K": K, "N": N, "us": round(ms * 1e3, 2),
                     "GBps": round(gbs, 1), "bound": "hbm", "frac": round(gbs / HBM_PEAK_GBS, 4)})
        del reps, x
        torch.cuda.empty_cache()
    return rows


def gather_sweep(mq, torch, eager_launches: int = 0):
    """The expert GEMMs of one MoE layer's prefill at the Qwen3-30B-A3B shape:
    8 x 512 tokens routed to 8 of 128 experts (uniform random), the 32768
    (token, expert) pairs sorted by expert (models/lfm2.py:204,613-618), then
    gather_qmm over the sorted rows (models/lfm2.py:176-187) -- the experts'
    gate|up projection (2 x 768 rows, K = 2048, x rows gathered by token) and
    the down projection (2048 rows, K = 768, rows already in pair order).  `us`
    is given the sort's segment offsets (as the MoE block passes them);
    `us_segments_derived` is the drop-in call that derives them from the ids."""
    E, k, H, inter, T = 128, 8, 2048, 768, 4096
    gen = torch.Generator(device="cuda:0").manual_seed(3)
    ids = torch.rand(T, E, generator=gen, device="cuda:0").topk(k, -1).indices.reshape(-1)
    order = torch.sort(ids, stable=True).indices
    rhs = ids[order].to(torch.int32).contiguous()
    lhs = (order // k).to(torch.int32).contiguous()
    offs = torch.searchsorted(rhs, torch.arange(E + 1, device="cuda:0", dtype=torch.int32)
                              ).to(torch.int32)
    x = torch.randn(T, 1, H, generator=gen, device="cuda:0").to(torch.bfloat16)
    act = torch.randn(T * k, 1, inter, generator=gen, device="cuda:0").to(torch.bfloat16)
    rows = []
    for name, N, K, xin, lhs_i in (("gate|up", 2 * inter, H, x, lhs), ("down", H, inter, act, None)):
        w = (torch.randn(E * N, K, generator=gen, device="cuda:0") * 0.02).to(torch.bfloat16)
        wq, sc, bi = (t.reshape(E, N, -1) for t in mq.quantize(w, 64, 4))
        del w

        def launch(i, xin=xin, wq=wq, sc=sc, bi=bi, lhs_i=lhs_i, seg=offs):
            mq.gather_qmm(xin, wq, sc, bi, lhs_indices=lhs_i, rhs_indices=rhs, group_size=64,
                          bits=4, sorted_indices=True, expert_offsets=seg)

        if eager_launches:  # for rocprofv3: plain launches, no graph, no timing
            for i in range(eager_launches):
                launch(i)
                if name == "gate|up":
                    core = importlib.import_module("mlx-server-runtime_amd.core")
                    core.gather_qmm_swiglu(x, wq, sc, bi, lhs, rhs, 64, 4, expert_offsets=offs)
            torch.cuda.synchronize()
            rows.append({"gemm": name, "launches": eager_launches})
            continue
        ms, _ = time_graph(torch, launch, 8, warmup=2, reps=4)
        ms_derive, _ = time_graph(torch, lambda i: launch(i, seg=None), 8, warmup=2, reps=4)
        flops = 2.0 * T * k * N * K
        wbytes = E * (N * K // 2 + N * (K // 64) * 4)
        tfl = flops / (ms * 1e-3) / 1e12
        rows.append({"gemm": name, "pairs": T * k, "experts": E, "N": N, "K": K, "bits": 4,
                     "us": round(ms * 1e3, 2), "TFLOPs": round(tfl, 2),
                     "us_segments_derived": round(ms_derive * 1e3, 2),
                     "GBps": round((wbytes + 2 * T * k * (N + K)) / (ms * 1e-3) / 1e9, 1),
                     "bound": "mfma", "frac": round(tfl / BF16_PEAK_TFLOPS, 4)})
        if name == "gate|up":
            # the form the MoE block runs: SiLU * up in the GEMM's epilogue
            core = importlib.import_module("mlx-server-runtime_amd.core")
            fms, _ = time_graph(torch, lambda i: core.gather_qmm_swiglu(
                x, wq, sc, bi, lhs, rhs, 64, 4, expert_offsets=offs), 8, warmup=2, reps=4)
            rows[-1]["us_with_swiglu_epilogue"] = round(fms * 1e3, 2)
            rows[-1]["frac_with_swiglu_epilogue"] = round(
                flops / (fms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)
        del wq, sc, bi
    torch.cuda.empty_cache()
    return rows


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              "(the path has no multi-GPU component; it would shard by heads, K groups and "
              "experts across one process per GPU).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    mq = importlib.import_module("mlx-server-runtime_amd")
    from oracle import oracle as orc

    if args.profile_shape:
        pM, pK, pN, pbits = (int(v) for v in args.profile_shape.split(","))
        reps = make_replicas(mq, torch, pN, pK, pbits, 2, seed=0)
        px = torch.randn(pM, pK, generator=torch.Generator(device="cuda:0").manual_seed(1),
                         device="cuda:0").to(torch.bfloat16)
        for i in range(args.warmup + args.steps):
            wq, s, b = reps[i % 2]
            mq.quantized_matmul(px, wq, s, b, transpose=True, group_size=64, bits=pbits)
        torch.cuda.synchronize()
        print(json.dumps({"profile_shape": [pM, pK, pN, pbits], "launches": args.warmup + args.steps}))
        return

    if args.profile_prefill_attention:
        pB, pT, pS, pH, pKV = (int(v) for v in args.profile_prefill_attention.split(","))
        ops = importlib.import_module("mlx-server-runtime_amd.decode_ops")
        gen = torch.Generator(device="cuda:0").manual_seed(pB * pT)
        cache = ops.PagedKV.contiguous(1, pB, pS + pT, pKV, 128, "cuda:0")
        cache.k[0].normal_(generator=gen)
        cache.v[0].normal_(generator=gen)
        q = torch.randn(pB, pT, pH, 128, generator=gen, device="cuda:0").to(torch.bfloat16)
        starts = torch.full((pB,), pS, dtype=torch.int64, device="cuda:0")
        lens = torch.full((pB,), pT, dtype=torch.int64, device="cuda:0")
        for _ in range(args.warmup + args.steps):
            ops.paged_prefill_attention(q, cache, 0, cache.page_table, starts, lens, 128 ** -0.5)
        torch.cuda.synchronize()
        print(json.dumps({"profile_prefill_attention": [pB, pT, pS, pH, pKV],
                          "launches": args.warmup + args.steps}))
        return

    if args.profile_gather:
        rows = gather_sweep(mq, torch, eager_launches=args.warmup + args.steps)
        print(json.dumps({"profile_gather": rows}))
        return

    if args.trace_qmv:
        print(json.dumps({"qmv_trace": trace_qmv(mq, torch)}))
        return

    if args.decode_only is not None:
        if args.decode_only == 1:
            res = decode_bench(torch, 1, 512, 128)
        elif args.decode_only == 8:
            res = decode_bench(torch, 8, 512, 128, model_name="qwen3_30b_a3b")
        else:
            res = decode_bench(torch, args.decode_only, 1024, 256, prefix_len=256)
        print(json.dumps({"decode": res}))
        return

    K, N, bits, M = 3584, 18944, 4, 1
    replicas = make_replicas(mq, torch, N, K, bits, args.replicas, seed=0)
    gen = torch.Generator(device="cuda:0").manual_seed(1)
    x = torch.randn(M, K, generator=gen, device="cuda:0").to(torch.bfloat16)

    def launch(i):
        wq, s, b = replicas[i % len(replicas)]
        mq.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits=bits)

    if args.profile:
        # Counter calibration first: a plain 128 MiB -> 128 MiB copy whose source
        # was pushed out of the 256 MB Infinity Cache by a 1 GiB fill, so that
        # FETCH_SIZE / WRITE_SIZE of the copy correspond to known HBM bytes.
        src = torch.empty(64 * 1024 * 1024, dtype=torch.bfloat16, device="cuda:0").fill_(1)
        flush = torch.empty(512 * 1024 * 1024, dtype=torch.bfloat16, device="cuda:0").fill_(2)
        dst = torch.empty_like(src)
        dst.copy_(src)
        del flush
        for i in range(args.warmup + args.steps):
            launch(i)
        torch.cuda.synchronize()
        print(json.dumps({"profile": "done", "launches": args.warmup + args.steps,
                          "copy_bytes_each_way": src.numel() * 2}))
        return

    R = len(replicas)  # launches per step: one pass over the replicas
    ms, wall_ms = time_graph(torch, launch, args.steps * R, args.warmup * R)
    by = alg_bytes(M, N, K, bits)
    gbs = by / (ms * 1e-3) / 1e9
    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(ms * R, 6),
        "ms_per_step_wall": round(wall_ms * R, 6),
        "launches_per_step": R,
        "launches_timed": args.steps * R,
        "us_per_launch": round(ms * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W ~ N(0,0.02) (seeds 0..15) cast to bf16 and quantized on the GPU; "
                "x ~ N(0,1) bf16 (seed 1)",
        "config": {"workload": "quantized_matmul decode GEMV (qmv): 4-bit affine, group 64, "
                               f"x bf16 [1,3584] @ W[18944,3584]^T; a step is {R} launches, "
                               f"one per rotating weight replica",
                   "M": M, "K": K, "N": N, "bits": bits, "group_size": 64,
                   "bytes_per_launch": by, "bytes_per_step": by * R},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
    }
    line["hbm_floor"] = hbm_floor(mq, torch, by)
    if not args.no_decode:
        # Qwen2.5-7B shape, 4-bit: batch 1 (512-token prompt, 128 tokens) and
        # batch 32 (1024-token prompts, 256 tokens).
        line["decode"] = [decode_bench(torch, 1, 512, 128),
                          decode_bench(torch, 32, 1024, 256, prefix_len=256),
                          decode_bench(torch, 8, 512, 128, model_name="qwen3_30b_a3b")]
    if not args.no_sweep:
        line["sweep"] = sweep(mq, torch)
        line["group_sweep"] = group_sweep(mq, torch)
        line["bits_sweep"] = bits_sweep(mq, torch)
        line["gather_sweep"] = gather_sweep(mq, torch)
    if not args.no_cpu:
        wq, s, b = replicas[0]
        line["cpu_baseline"] = cpu_baseline(
            args, orc, wq.cpu().numpy().view("uint32"), s.cpu().view(torch.int16).numpy().view("uint16"),
            b.cpu().view(torch.int16).numpy().view("uint16"),
            x.cpu().view(torch.int16).numpy().view("uint16"), N, K, bits)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
