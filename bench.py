"""Benchmark of the quantized Linear hot path on one MI355X.

Headline (`value`): the Q4_0 decode GEMV of configs[1].  A step is one
batch-1 Linear forward of the Llama-7B FFN up/gate shape (W 11008x4096 GGUF
Q4_0, x f32 [4096]) through the C ABI (rdl_linear_forward_dev: one kernel,
activation prep fused), i.e. rustml_quant::matmul_f32_q4 (quantize.rs:265-320)
with the weight resident in HBM.  Consecutive steps use different weight
copies (more than the 256 MB Infinity Cache in total) so each step streams
its weight from HBM.

Timed region: the K steps are captured once in a HIP graph (so host launch
overhead is not measured) and replayed once between two events.  A step is
one launch of the GEMV kernel, so the roofline's kernel duration is that
region's average per launch.  Each kernel is also timed at its boundaries
(hipExtLaunchKernel events) over K separate eager launches, reported as
eager_launch_* (an idle GPU between launches, so a different condition).

The same JSON line carries, under "workloads", the other configurations of
the metric: configs[0] (Q8_0 GEMV) and configs[2] (Q4_K GEMV pair) timed the
same way, configs[3] (Q4_0 prefill GEMM, M in {16, 64, 512, 2048}) as
TFLOP/s, and configs[4] (random-init 7B Q4_0 Llama, 128-token prompt, 256
greedy tokens) as decode tokens/s with its HBM roofline per token.
`--workload` restricts the run to one of them (for profiling).
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "rust-deeplearning_amd"))

METRIC = "Q4_0/Q4_K GEMV achieved HBM GB/s (% peak); 7B Q4_0 decode tokens/s"
PEAK_HBM_GBPS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense f16/bf16 MFMA, MI355X
PEAK_I8_TOPS = 5000.0     # dense int8 MFMA, MI355X
N_OUT, K_IN = 11008, 4096
SEED = 0x5EED0002
# the kernel the library launches for this workload (8-wave workgroups, 3 rows per wave)
KERNEL_KEY = "gemv_fused_kernel<2, false, 3, 2, true, 8, 0, 0>|config2"
# the kernels of configs 1 and 3 (keys of profiles/traffic.json)
Q8_KEY = "gemv_fused_kernel<8, false, 4, 2, true, 4, 0, 0>|config1"
Q4K_UP_KEY = "gemv_q4k_fused_kernel<4, 8, 0, 0>|config3 up"
Q4K_DOWN_KEY = "gemv_q4k_splitk_kernel<4, 4, 16, 0, 0>|config3 down"
# configs[4]
LLAMA_SEED = 0x5EED0005
PROMPT_LEN, GEN_TOKENS = 128, 256
LONG_PROMPT_LEN = 2040  # prefill figure beside the decode line (max_seq 2048)
# not a BASELINE config: the lm_head of a llama.cpp Q4_0 7B file is Q6_K
Q6K_LM_HEAD = "Q6_K GEMV 32000x4096 (the output matrix of llama.cpp Q4_0 7B files)"

# GGML type id -> (elements per block, bytes per block)
BLOCK = {2: (32, 18), 3: (32, 20), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def algorithmic_bytes(n, k, dtype=2):
    """Weight blocks + x (f32) + y (f32), each read or written once."""
    qk, bb = BLOCK[dtype]
    return n * (k // qk) * bb + 4 * k + 4 * n


def measured_traffic(kernel_key):
    """HBM bytes per launch of the timed kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (scaled by a known-size copy); None when no
    measurement for this kernel and workload is on file."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel_key)
    except (OSError, ValueError):
        return None
    return None if rec is None else int(rec["traffic_bytes_per_launch"])


def cpu_baseline(budget_s=10.0):
    """The reference decomposition of an M=1 matmul_f32_q4 (one rayon task -> one core),
    restated in C (oracle/), timed on this host over a bounded sample."""
    from oracle import oracle as orc
    from rdlquant import synth

    copies = 8  # 8 x 25.4 MB rotated so the host LLC does not hold the weight
    ws = [synth.q4_0_weights(N_OUT, K_IN, SEED + i) for i in range(copies)]
    x = synth.activations(1, K_IN, SEED + 100)
    orc.matmul("q4", x, ws[0], 1, K_IN, N_OUT, threads=1)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        orc.matmul("q4", x, ws[i % copies], 1, K_IN, N_OUT, threads=1)
        times.append(time.perf_counter() - t0)
        i += 1
    med = statistics.median(times)
    gbps = algorithmic_bytes(N_OUT, K_IN) / med / 1e9
    # not the reference: the same restatement with the N outputs split over
    # the host cores this job may use (the reference runs M = 1 on one core)
    threads = min(16, os.cpu_count() or 1)
    par = []
    t_end = time.perf_counter() + budget_s / 3
    while time.perf_counter() < t_end or len(par) < 5:
        t0 = time.perf_counter()
        orc.matmul("q4_cols", x, ws[len(par) % copies], 1, K_IN, N_OUT, threads=threads)
        par.append(time.perf_counter() - t0)
    pmed = statistics.median(par)
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{len(times)} single-thread matmul_f32_q4 calls, 11008x4096 Q4_0, M=1, "
                  f"median {med * 1e3:.2f} ms, weights rotated over {copies} copies "
                  f"(host nproc={os.cpu_count()})",
        "all_cores_not_reference": {
            "value": round(algorithmic_bytes(N_OUT, K_IN) / pmed / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "sample": f"{len(par)} calls of the same restatement with the N outputs split over "
                      f"{threads} threads, median {pmed * 1e3:.2f} ms",
        },
    }


def cpu_baseline_q4k(n, k, seed, budget_s=3.0):
    """The reference's run-time Q4_K work: an F32 GEMV over the matrix that
    load_tensors dequantized (parser.rs:321-325, linear.rs:167-170), restated
    in C and split over the host cores this job may use (faer parallelises
    it); the dequantization itself is load time and not timed."""
    from oracle import oracle as orc
    from rdlquant import synth

    threads = min(16, os.cpu_count() or 1)
    wf = orc.to_f32("q4k", synth.q4_k_weights(n, k, seed), n * k)
    x = synth.activations(1, k, seed + 100)
    orc.matmul_f32_f32(x, wf, 1, k, n, threads=threads)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        orc.matmul_f32_f32(x, wf, 1, k, n, threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(algorithmic_bytes(n, k, 12) / med / 1e9, 3),
        "unit": "GB/s (Q4_K algorithmic bytes / time)",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} F32 GEMVs over the dequantized {n}x{k} matrix ({n * k * 4 >> 20} MiB), "
                  f"median {med * 1e3:.2f} ms",
    }


def _timed(fn, budget_s, min_runs=3):
    """Median seconds of fn() over a time budget (at least min_runs calls)."""
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn(len(times))
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline_q8(budget_s=3.0):
    """matmul_f32_q8 at M = 1 (quantize.rs:201-260), one rayon task
    per input row -> one core, restated in C and timed on this host."""
    from oracle import oracle as orc
    from rdlquant import synth

    n = k = 4096
    copies = 8  # 8 x 17.8 MB rotated past the host LLC
    ws = [synth.q8_0_weights(n, k, 0x5EED0001 + i) for i in range(copies)]
    x = synth.activations(1, k, 0x5EED0101)
    orc.matmul("q8", x, ws[0], 1, k, n, threads=1)
    med, runs = _timed(lambda i: orc.matmul("q8", x, ws[i % copies], 1, k, n, threads=1), budget_s)
    return {
        "value": round(algorithmic_bytes(n, k, 8) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{runs} single-thread matmul_f32_q8 calls, 4096x4096 Q8_0, M=1, median {med * 1e3:.2f} ms, "
                  f"weights rotated over {copies} copies",
    }


def cpu_baseline_gemm(m, budget_s=3.0):
    """matmul_f32_q4 (the Linear default) at M rows, the reference
    decomposition -- one rayon task per input row (quantize.rs:284-287) over
    min(M, host cores) threads -- restated in C and timed on this host."""
    from oracle import oracle as orc
    from rdlquant import synth

    n = k = 4096
    threads = min(m, 16, os.cpu_count() or 1)
    # bounded sample: each thread's rows run one after another, so a call over
    # ms = 2 * threads rows (two rows a thread) times the same per-row work;
    # the M-row call is ceil(M / threads) / 2 times as long
    ms = min(m, 2 * threads)
    w = synth.q4_0_weights(n, k, 0x5EED0004)
    x = synth.activations(ms, k, 0x5EED0104 + m)
    med, runs = _timed(lambda i: orc.matmul("q4", x, w, ms, k, n, threads=threads), budget_s, min_runs=2)
    call = med * (-(-m // threads)) / (-(-ms // threads))
    flops = 2.0 * m * n * k
    return {
        "value": round(flops / call / 1e12, 5),
        "unit": "TFLOP/s",
        "gbs": round((n * (k // 32) * 18 + 4 * m * (k + n)) / call / 1e9, 3),
        "ms_per_call": round(call * 1e3, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{runs} matmul_f32_q4 calls over {ms} of the {m} rows (4096x4096 Q4_0), input rows split "
                  f"over {threads} threads, median {med * 1e3:.1f} ms, scaled to {-(-m // threads)} rows a thread",
    }


def cpu_baseline_decode(budget_s=6.0):
    """one 7B decode token on the reference's path is 32 layers of
    seven Q4_0 Linears at M = 1 (each one rayon task -> one core,
    quantize.rs:284-287) plus the Q4_0 lm_head; restated in C and timed on this
    host over one layer's matrices and the lm_head, scaled to 32 layers.  The
    non-matmul ops (RMSNorm, RoPE, attention over <= 384 cached rows, SwiGLU)
    are below 0.1% of that time on the reference and are not timed."""
    from oracle import oracle as orc
    from rdlquant import synth

    d, f, kv, vocab = 4096, 14336, 1024, 32000
    shapes = [("q", d, d), ("k", kv, d), ("v", kv, d), ("o", d, d), ("gate", f, d), ("up", f, d), ("down", d, f)]
    mats = {name: synth.q4_0_weights(n, k, 0x5EED0500 + i) for i, (name, n, k) in enumerate(shapes)}
    out_w = synth.q4_0_weights(vocab, d, 0x5EED0599)
    xs = {k: synth.activations(1, k, 0x5EED0600 + k) for k in (d, f)}

    def layer(_):
        for name, n, k in shapes:
            orc.matmul("q4", xs[k], mats[name], 1, k, n, threads=1)

    layer(0)
    lmed, lruns = _timed(layer, budget_s * 0.8, min_runs=2)
    hmed, hruns = _timed(lambda i: orc.matmul("q4", xs[d], out_w, 1, d, vocab, threads=1), budget_s * 0.2,
                         min_runs=2)
    per_token = 32 * lmed + hmed
    return {
        "value": round(1.0 / per_token, 4),
        "unit": "tokens/s",
        "ms_per_token": round(per_token * 1e3, 1),
        "cores": 1,
        "kind": "port",
        "sample": f"one layer's seven Q4_0 matmul_f32_q4 calls at M=1 ({lruns} runs, median {lmed * 1e3:.1f} ms) "
                  f"x 32 layers + the 32000x4096 lm_head ({hruns} runs, median {hmed * 1e3:.1f} ms), one thread",
    }


class Rig:
    """Device, stream and rotating weight copies for the GEMV/GEMM timings."""

    def __init__(self):
        import torch

        import rdlquant as rq
        from rdlquant import synth

        self.torch, self.rq, self.synth = torch, rq, synth
        self.dev = torch.device("cuda:0")
        torch.cuda.set_device(self.dev)
        self.stream = torch.cuda.current_stream()

    def weight_copies(self, dtype, n, k, seed, min_total=600 << 20, min_copies=8):
        torch, rq = self.torch, self.rq
        w_host = self.synth.weights(dtype, n, k, seed)
        nbytes = w_host.size
        copies = max(min_copies, -(-min_total // nbytes))
        w0 = torch.from_numpy(w_host).to(self.dev)
        out = []
        for _ in range(copies):
            t = torch.empty(nbytes + 256, dtype=torch.uint8, device=self.dev)
            t[:nbytes].copy_(w0)
            out.append((t, rq.Weight.wrap_device(t.data_ptr(), nbytes, dtype, n, k, t)))
        return w_host, out

    def time_gemv(self, weights, x, y, steps, warmup):
        """(graph-replay ms per step, sorted per-launch kernel ms) for y = W_i x."""
        rq = self.rq

        def step(i, s_handle):
            weights[i % len(weights)][1].forward_dev(x.data_ptr(), 1, y.data_ptr(), rq.MODE_FLOAT, s_handle)

        return self.time_launches(step, steps, warmup)

    def time_launches(self, step, steps, warmup):
        """(graph-replay ms per step, sorted per-launch kernel ms) for
        step(i, stream_handle), one library launch per step."""
        torch, rq = self.torch, self.rq
        sh = self.stream.cuda_stream
        for i in range(warmup):
            step(i, sh)
        torch.cuda.synchronize()
        # capture the K steps in one graph; one untimed replay, then the timed one
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cap = torch.cuda.current_stream().cuda_stream
            for i in range(steps):
                step(i, cap)
        graph.replay()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(self.stream)
        graph.replay()
        t1.record(self.stream)
        torch.cuda.synchronize()
        ms_per_step = t0.elapsed_time(t1) / steps
        del graph

        # kernel-boundary timing over K separate launches
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        for a, b in evs:  # materialize the events
            a.record(self.stream)
            b.record(self.stream)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(evs):
            rq.time_next_launch(a.cuda_event, b.cuda_event)
            step(i, sh)
        torch.cuda.synchronize()
        kern_ms = sorted(a.elapsed_time(b) for a, b in evs)
        return ms_per_step, kern_ms


def native_check(rig, w_host, x, y, m, n, k):
    """Native mode: y within 1e-3 rel + 1e-4 abs of the exact (f64) product of
    the Q8_0-quantized x (the library's byte-exact quantize_row_q8_0, codes
    times scales) with the weight's f32 values -- the real value of
    matmul_f32_q4_native's sum of int32 block dots times both block scales."""
    torch, rq = rig.torch, rig.rq
    nb = k // 32
    q8 = torch.empty(m * nb * 34, dtype=torch.uint8, device=rig.dev)
    for r in range(m):
        rq.quantize_row_q8_0_dev(x.reshape(m, k)[r].data_ptr(), k, q8[r * nb * 34:].data_ptr(), 0,
                                 rig.stream.cuda_stream)
    blk = q8.reshape(m, nb, 34)
    sc = blk[:, :, 0:2].contiguous().view(torch.float16).double()             # [m, nb, 1]
    codes = blk[:, :, 2:].contiguous().view(torch.int8).double()             # [m, nb, 32]
    xq = (codes * sc).reshape(m, k)
    wt = rq.Weight.upload(w_host, rq.DTYPE_Q4_0, n, k)
    rows = torch.arange(n, dtype=torch.int32, device=rig.dev)
    wf = torch.empty(n, k, dtype=torch.float32, device=rig.dev)
    wt.dequantize_rows_dev(rows.data_ptr(), n, wf.data_ptr(), rig.stream.cuda_stream)
    want = xq @ wf.double().T
    got = y.reshape(m, n).double()
    ok = bool(((got - want).abs() <= 1e-4 + 1e-3 * want.abs()).all().item())
    wt.free()
    del wf, q8
    return ok


def exact_check(rig, weight, x, y, m, n, k, cond=False):
    """y within 1e-3 rel + 1e-4 abs of the exact (f64) product over the weight's
    f32 values (Tensor::to_f32 / dequantize_q4k, expanded by the library's
    bit-exact row dequantization); torch does the f64 product on the device.
    cond: plus 1e-6 sum |x| |w| of each output (outputs that cancel far below
    their terms, beyond any f32 evaluation's value bar)."""
    torch = rig.torch
    rows = torch.arange(n, dtype=torch.int32, device=rig.dev)
    wf = torch.empty(n, k, dtype=torch.float32, device=rig.dev)
    weight.dequantize_rows_dev(rows.data_ptr(), n, wf.data_ptr(), rig.stream.cuda_stream)
    want = x.reshape(m, k).double() @ wf.double().T
    got = y.reshape(m, n).double()
    tol = 1e-4 + 1e-3 * want.abs()
    if cond:
        tol = tol + 1e-6 * (x.reshape(m, k).double().abs() @ wf.double().abs().T)
    ok = bool(((got - want).abs() <= tol).all().item())
    del wf
    return ok


def gemv_line(rig, name, dtype, n, k, seed, steps, warmup, traffic_key=None):
    """One GEMV configuration: throughput, kernel roofline (with the committed
    counter traffic for traffic_key when on file) and a parity spot check."""
    torch = rig.torch
    w_host, weights = rig.weight_copies(dtype, n, k, seed)
    x_host = rig.synth.activations(1, k, seed + 100)
    x = torch.from_numpy(x_host.reshape(-1)).to(rig.dev)
    y = torch.empty(n, dtype=torch.float32, device=rig.dev)
    ms, kern_ms = rig.time_gemv(weights, x, y, steps, warmup)
    kavg = ms  # one launch a step: the timed region's average launch duration
    abytes = algorithmic_bytes(n, k, dtype)
    ok = exact_check(rig, weights[0][1], x, y, 1, n, k)
    copies = len(weights)
    del weights
    torch.cuda.empty_cache()
    return {
        "workload": name,
        "value": round(abytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 6),
        "algorithmic_bytes_per_step": abytes,
        "weight_copies_rotated": copies,
        "roofline": {
            "bound": "hbm",
            "achieved": round(abytes / (kavg * 1e-3) / 1e9, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(abytes / (kavg * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "kernel_avg_us": round(kavg * 1e3, 3),
            "eager_launch_avg_us": round(sum(kern_ms) / len(kern_ms) * 1e3, 3),
            "eager_launch_median_us": round(kern_ms[len(kern_ms) // 2] * 1e3, 3),
            "traffic": measured_traffic(traffic_key) if traffic_key else None,
        },
        "parity_vs_exact": ok,
    }


TYPE_NAME = {2: "Q4_0", 3: "Q4_1", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}


def gemm_lines(rig, ms_list, seed=0x5EED0004, native=False, dtype=2):
    """Y = X W^T, W 4096x4096 Q4_0, X f32 [M, 4096]; the whole call
    (activation split or Q8_0 quantization + MFMA GEMM) timed over a loop of
    launches.  native: matmul_f32_q4_native (int8 MFMA on the Q8_0 codes).
    dtype: the same product for another weight format (not a BASELINE
    config; the tile GEMM of Q8_0, Q4_1, Q4_K and Q6_K)."""
    torch, rq = rig.torch, rig.rq
    n = k = 4096
    mode = rq.MODE_NATIVE if native else rq.MODE_FLOAT
    w_host, weights = rig.weight_copies(dtype, n, k, seed, min_copies=16)
    s = rig.stream
    out = []
    for m in ms_list:
        x_host = rig.synth.activations(m, k, seed + 100 + m)
        x = torch.from_numpy(x_host).to(rig.dev)
        y = torch.empty(m, n, dtype=torch.float32, device=rig.dev)
        for i in range(10):
            weights[i % len(weights)][1].forward_dev(x.data_ptr(), m, y.data_ptr(), mode, s.cuda_stream)
        torch.cuda.synchronize()
        it = 200 if m <= 512 else 60
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        for i in range(it):
            weights[i % len(weights)][1].forward_dev(x.data_ptr(), m, y.data_ptr(), mode, s.cuda_stream)
        b.record(s)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / it
        flops = 2.0 * m * n * k
        qk, bb = BLOCK[dtype]
        abytes = n * (k // qk) * bb + 4 * m * k + 4 * m * n
        ok = (native_check(rig, w_host, x, y, m, n, k) if native
              else exact_check(rig, weights[0][1], x, y, m, n, k, cond=dtype != 2))
        tflops = flops / (ms * 1e-3) / 1e12
        gbps = abytes / (ms * 1e-3) / 1e9
        peak_mm = PEAK_I8_TOPS if native else PEAK_F16_TFLOPS
        bound = "mfma" if flops / abytes > peak_mm * 1e12 / (PEAK_HBM_GBPS * 1e9) else "hbm"
        out.append({
            "workload": (f"config4 M={m}" + (" native (matmul_f32_q4_native, int8 MFMA)" if native else "")
                         if dtype == 2 else f"{TYPE_NAME[dtype]} GEMM 4096x4096 M={m} (not a BASELINE config)"),
            "m": m,
            "value": round(tflops, 2),
            "unit": "TOP/s" if native else "TFLOP/s",
            "ms_per_call": round(ms, 5),
            "hbm_GBs": round(gbps, 1),
            "roofline": {
                "bound": bound,
                "achieved": round(tflops, 2) if bound == "mfma" else round(gbps, 1),
                "peak": peak_mm if bound == "mfma" else PEAK_HBM_GBPS,
                "unit": ("TOP/s" if native else "TFLOP/s") if bound == "mfma" else "GB/s",
                "frac": round(tflops / peak_mm if bound == "mfma" else gbps / PEAK_HBM_GBPS, 4),
            },
            "parity_vs_exact": ok,
        })
        del x, y
    del weights
    torch.cuda.empty_cache()
    return out


# weight bytes of the GEMV configs the plain read is compared with
READ_SIZES = [("config1 Q8_0 4096x4096", 4096 * 128 * 34), ("config2 Q4_0 11008x4096", 11008 * 128 * 18),
              ("config3 down Q4_K 4096x14336", 4096 * 56 * 144)]


def read_lines(rig, steps=200, warmup=20):
    """The HBM read ceiling of a plain kernel (rdl_stream_read_dev: one
    streaming read, no arithmetic) at the weight sizes of configs 1-3, over
    rotated copies (>= 400 MB, beyond the 256 MB Infinity Cache), timed as the
    GEMV lines are: graph replay per step and per-launch kernel events."""
    torch, rq = rig.torch, rig.rq
    out_len = 2 * 256 * 4
    out = torch.empty(out_len, dtype=torch.int32, device=rig.dev)
    lines = []
    for name, nbytes in READ_SIZES:
        nbytes -= nbytes % 16
        copies = max(16, -(-400 * 2**20 // nbytes))
        bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=rig.dev) for _ in range(copies)]

        def step(i, s_handle):
            rq.stream_read_dev(bufs[i % copies].data_ptr(), nbytes, out.data_ptr(), out_len, s_handle)

        ms_step, kern_ms = rig.time_launches(step, steps, warmup)
        avg = ms_step  # one launch a step, as in the GEMV lines
        eager_avg = sum(kern_ms) / len(kern_ms)
        med = kern_ms[len(kern_ms) // 2]
        lines.append({
            "workload": f"plain streaming read of {nbytes} bytes ({name} weight bytes)",
            "bytes": nbytes,
            "copies_rotated": copies,
            "ms_per_step": round(ms_step, 6),
            "kernel_avg_us": round(avg * 1e3, 3),
            "eager_launch_avg_us": round(eager_avg * 1e3, 3),
            "eager_launch_median_us": round(med * 1e3, 3),
            "GBs_kernel_avg": round(nbytes / (avg * 1e-3) / 1e9, 1),
            "frac_of_8TBs": round(nbytes / (avg * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        })
        del bufs
        torch.cuda.empty_cache()
    return lines


def decode_bytes_per_token(cfg, ctx_mean):
    """Q4_0 Linear + lm_head weight bytes, one embedding row, and f16 K/V reads
    over ctx_mean cached positions, per decode token."""
    d, f, hd = cfg.dim, cfg.ffn_dim, cfg.head_dim
    per_layer = (d * cfg.n_heads * hd + 2 * d * cfg.n_kv_heads * hd + cfg.n_heads * hd * d + 3 * d * f)
    params = cfg.n_layers * per_layer + cfg.vocab * d
    kv = cfg.n_layers * 2 * cfg.n_kv_heads * hd * (2 if cfg.kv_f16 else 4)
    return params // 32 * 18 + (d // 32) * 18 + int(kv * ctx_mean)


def decode_line(rig, reps=2):
    """random-init 7B Q4_0 Llama, greedy decode of 256 tokens after a
    128-token prompt, each step one replay of the captured decode graph.  Also
    the prefill time of a 2040-token prompt (not part of the value)."""
    import numpy as np

    from rdlquant.llama import LlamaConfig, LlamaModel

    cfg = LlamaConfig()
    model = LlamaModel(cfg)
    model.init_random(LLAMA_SEED)
    prompt = np.random.default_rng(LLAMA_SEED).integers(0, cfg.vocab, PROMPT_LEN)
    runs = []
    toks0 = None
    for _ in range(reps + 1):  # the first run captures the graph; not timed
        model.reset()
        toks = model.generate_greedy(prompt, GEN_TOKENS + 1)
        runs.append(model.last_timing())
        if toks0 is None:
            toks0 = toks
        elif not np.array_equal(toks, toks0):
            raise RuntimeError("greedy decode is not deterministic across runs")
    # a long prompt: 16 chunks of 128 rows, the later ones attending to up to
    # 2040 cached keys (prefill only, the first token sampled)
    long_prompt = np.random.default_rng(LLAMA_SEED + 1).integers(0, cfg.vocab, LONG_PROMPT_LEN)
    long_ms = []
    for _ in range(2):
        model.reset()
        model.generate_greedy(long_prompt, 1)
        long_ms.append(model.last_timing()[0])
    model.close()
    rig.torch.cuda.empty_cache()
    decode_ms = min(r[1] for r in runs[1:])
    prefill_ms = min(r[0] for r in runs[1:])
    ms_tok = decode_ms / GEN_TOKENS
    # positions attended by the 256 steps: PROMPT_LEN+1 .. PROMPT_LEN+GEN_TOKENS
    ctx_mean = PROMPT_LEN + (GEN_TOKENS + 1) / 2
    bpt = decode_bytes_per_token(cfg, ctx_mean)
    gbps = bpt / (ms_tok * 1e-3) / 1e9
    return {
        "workload": "config5: random-init Llama-7B-shape Q4_0 (32 layers, 4096, 32/8 heads x 128, "
                    "FFN 14336, vocab 32000), f16 KV, 128-token prompt, 256 greedy tokens",
        "value": round(GEN_TOKENS / (decode_ms * 1e-3), 1),
        "unit": "tokens/s",
        "ms_per_token": round(ms_tok, 4),
        "prefill_ms_128_tokens": round(prefill_ms, 3),
        "prefill_tokens_s": round(PROMPT_LEN / (prefill_ms * 1e-3), 1),
        "prefill_ms_%d_tokens" % LONG_PROMPT_LEN: round(min(long_ms), 3),
        "prefill_%d_tokens_s" % LONG_PROMPT_LEN: round(LONG_PROMPT_LEN / (min(long_ms) * 1e-3), 1),
        "bytes_per_token": bpt,
        "tokens_s_at_100pct_hbm": round(PEAK_HBM_GBPS * 1e9 / bpt, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / PEAK_HBM_GBPS, 4),
        },
        "first_tokens": [int(t) for t in toks0[:8]],
    }


def q4_k_m_types(n_layers):
    """{(slot, layer): GGML type} of llama.cpp's Q4_K_M recipe for a Llama
    model: Q4_K everywhere except Q6_K for the output matrix and for attn_v /
    ffn_down in the first and last eighth of the layers and every third one
    between them."""
    import rdlquant.llama as L
    t = {(L.TOKEN_EMBEDDING, 0): 12, (L.OUTPUT, 0): 14}
    for i in range(n_layers):
        more = i < n_layers // 8 or i >= 7 * n_layers // 8 or (i - n_layers // 8) % 3 == 2
        for slot in (L.WQ, L.WK, L.WO, L.W_GATE, L.W_UP):
            t[(slot, i)] = 12
        t[(L.WV, i)] = 14 if more else 12
        t[(L.W_DOWN, i)] = 14 if more else 12
    return t


def decode_q4_k_m_line(rig, reps=2):
    """Not a BASELINE config: the config-5 model shape with llama.cpp's Q4_K_M
    type mix (Q4_K layers, Q6_K attn_v / ffn_down in 16 of 32 layers, Q4_K
    embedding, Q6_K output), synthetic weights (one seeded matrix per shape
    and type, repeated over the layers), greedy decode as config 5."""
    import numpy as np

    import rdlquant.llama as L
    from rdlquant.llama import LlamaConfig, LlamaModel

    cfg = LlamaConfig()
    types = q4_k_m_types(cfg.n_layers)
    model = LlamaModel(cfg, types=types)
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    shape = {L.TOKEN_EMBEDDING: (cfg.vocab, cfg.dim), L.OUTPUT: (cfg.vocab, cfg.dim), L.WQ: (q, cfg.dim),
             L.WK: (kv, cfg.dim), L.WV: (kv, cfg.dim), L.WO: (cfg.dim, q), L.W_GATE: (cfg.ffn_dim, cfg.dim),
             L.W_UP: (cfg.ffn_dim, cfg.dim), L.W_DOWN: (cfg.dim, cfg.ffn_dim)}
    cache = {}
    nbytes = 0
    for (slot, layer), t in sorted(types.items(), key=lambda kv_: (kv_[0][1], kv_[0][0])):
        n, k = shape[slot]
        key = (n, k, t)
        if key not in cache:
            cache[key] = rig.synth.weights(t, n, k, LLAMA_SEED + 0x100 + len(cache))
        model.set_weight(slot, layer, cache[key])
        if slot != L.TOKEN_EMBEDDING:
            nbytes += cache[key].size
    ones = np.ones(cfg.dim, np.float32)
    for layer in range(cfg.n_layers):
        model.set_weight(L.ATTN_NORM, layer, ones)
        model.set_weight(L.FFN_NORM, layer, ones)
    model.set_weight(L.FINAL_NORM, 0, ones)
    cache.clear()
    prompt = np.random.default_rng(LLAMA_SEED).integers(0, cfg.vocab, PROMPT_LEN)
    runs = []
    for _ in range(reps + 1):
        model.reset()
        model.generate_greedy(prompt, GEN_TOKENS + 1)
        runs.append(model.last_timing())
    model.close()
    rig.torch.cuda.empty_cache()
    decode_ms = min(r[1] for r in runs[1:])
    prefill_ms = min(r[0] for r in runs[1:])
    ms_tok = decode_ms / GEN_TOKENS
    ctx_mean = PROMPT_LEN + (GEN_TOKENS + 1) / 2
    kvb = cfg.n_layers * 2 * cfg.n_kv_heads * cfg.head_dim * 2
    bpt = nbytes + cfg.dim * 144 // 256 + int(kvb * ctx_mean)
    gbps = bpt / (ms_tok * 1e-3) / 1e9
    return {
        "workload": "7B Llama shape, llama.cpp Q4_K_M type mix (synthetic weights), f16 KV, 128-token prompt, "
                    "256 greedy tokens",
        "value": round(GEN_TOKENS / (decode_ms * 1e-3), 1),
        "unit": "tokens/s",
        "ms_per_token": round(ms_tok, 4),
        "prefill_ms_128_tokens": round(prefill_ms, 3),
        "prefill_tokens_s": round(PROMPT_LEN / (prefill_ms * 1e-3), 1),
        "bytes_per_token": bpt,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_HBM_GBPS, 4)},
    }


def load_line(rig):
    """A synthetic config-5 (Llama-7B-shape Q4_0) GGUF file written to TMPDIR,
    then loaded into a device-resident decoder (rdl_llama_load_gguf): parse of
    the mapped file, type/shape checks and the pinned-staged upload of every
    tensor.  The file was just written, so its pages are in the page cache:
    this is the load rate from memory, not from a cold disk."""
    import os
    import shutil
    import tempfile

    import numpy as np

    from rdlquant import gguf_writer
    from rdlquant.gguf import GGUFFile
    from rdlquant.llama import LlamaConfig, LlamaModel

    cfg = LlamaConfig()
    shapes = gguf_writer.llama_tensor_shapes(cfg)
    cache = {}

    def data(name):  # one seeded tensor per distinct shape (load time does not depend on values)
        dims, t = shapes[name]
        key = (tuple(dims), t)
        if key not in cache:
            if t == gguf_writer.GGML_F32:
                cache[key] = np.ones(dims[0], np.float32)
            else:
                cache[key] = rig.synth.q4_0_weights(dims[1], dims[0], LLAMA_SEED + len(cache))
        return cache[key]

    tmp = tempfile.mkdtemp(prefix="rdl_load_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        path = os.path.join(tmp, "llama7b_q4_0.gguf")
        t0 = time.perf_counter()
        size = gguf_writer.llama_builder(cfg, data).write(path)
        write_s = time.perf_counter() - t0
        cache.clear()
        loads = []
        for _ in range(2):
            t0 = time.perf_counter()
            f = GGUFFile.parse_header(path)
            t1 = time.perf_counter()
            m = LlamaModel.from_gguf(f, max_seq=2048, max_batch=128)
            rig.torch.cuda.synchronize()
            t2 = time.perf_counter()
            toks = m.generate_greedy([1, 2, 3, 4], 4)
            m.close()
            f.close()
            rig.torch.cuda.empty_cache()
            loads.append((t1 - t0, t2 - t0, [int(t) for t in toks]))
        # the reference's I/O pattern (parser.rs:143-148, 292-296, 346): the
        # file read into memory twice and every tensor copied out of it
        t0 = time.perf_counter()
        with open(path, "rb") as fh:
            head = fh.read()
        with open(path, "rb") as fh:
            whole = fh.read()
        ref_f = GGUFFile.parse_bytes(head)
        del head
        copies = [bytes(whole[ref_f.data_offset + ti.offset:ref_f.data_offset + ti.offset + ti.n_bytes])
                  for ti in ref_f.tensor_infos]
        ref_s = time.perf_counter() - t0
        del copies, whole, ref_f
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    parse_s, load_s, toks = min(loads, key=lambda r: r[1])
    return {
        "workload": "GGUF load: config5 Llama-7B-shape Q4_0 file (291 tensors) -> device decoder "
                    "(parse + checks + upload of every tensor), file in the page cache",
        "file_bytes": size,
        "write_s": round(write_s, 2),
        "parse_ms": round(parse_s * 1e3, 3),
        "load_s": round(load_s, 3),
        "value": round(size / load_s / 1e9, 2),
        "unit": "GB/s (file bytes / load time)",
        "reference_io_pattern_s": round(ref_s, 3),
        "reference_io_pattern_note": "host only: read_to_end twice + one Vec per tensor, no device upload",
        "first_tokens": toks,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=24)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", default="all", choices=["all", "gemv", "q8_0", "q4_k", "q6_k", "gemm", "gemm_formats", "decode", "decode_q4_k_m", "load", "read"],
                    help="all: the headline line plus configs 1, 3, 4, 5 and the Q6_K lm_head; otherwise only one "
                         "(load: the GGUF file load, decode_q4_k_m: a Q4_K_M-mixed 7B decode; run only "
                         "when asked)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (a known-size "
                         "reference for HBM traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the GEMV runs on a single MI355X and multi-GPU "
              "runs are not part of this path (rows would shard across GPUs with an "
              "all-gather of y).", file=sys.stderr)
        sys.exit(2)

    import torch

    rig = Rig()
    rq, synth = rig.rq, rig.synth
    dev = rig.dev

    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    wl = args.workload
    if wl in ("q8_0", "q4_k", "q6_k", "gemm", "gemm_formats", "decode", "decode_q4_k_m", "load", "read"):
        if wl == "read":
            line = read_lines(rig)
        elif wl == "q8_0":
            line = gemv_line(rig, "config1: Q8_0 GEMV 4096x4096", 8, 4096, 4096, 0x5EED0001,
                             args.steps, args.warmup, Q8_KEY)
        elif wl == "q4_k":
            line = [gemv_line(rig, "config3 up: Q4_K GEMV 14336x4096", 12, 14336, 4096, 0x5EED0003,
                              args.steps, args.warmup, Q4K_UP_KEY),
                    gemv_line(rig, "config3 down: Q4_K GEMV 4096x14336", 12, 4096, 14336, 0x5EED0013,
                              args.steps, args.warmup, Q4K_DOWN_KEY)]
        elif wl == "q6_k":
            line = gemv_line(rig, Q6K_LM_HEAD, 14, 32000, 4096, 0x5EED0006, args.steps, args.warmup)
        elif wl == "gemm":
            line = gemm_lines(rig, [16, 64, 512, 2048]) + gemm_lines(rig, [512, 2048], native=True)
        elif wl == "gemm_formats":
            line = [l for t in (8, 3, 12, 14) for l in gemm_lines(rig, [16, 128, 512, 2048], seed=0x5EED0040 + t, dtype=t)]
        elif wl == "load":
            line = load_line(rig)
        elif wl == "decode_q4_k_m":
            line = decode_q4_k_m_line(rig)
        else:
            line = decode_line(rig)
        print(json.dumps(line), flush=True)
        return

    wbytes = N_OUT * (K_IN // 32) * 18
    w_host = synth.q4_0_weights(N_OUT, K_IN, SEED)
    w0 = torch.from_numpy(w_host).to(dev)
    weights = []
    for i in range(args.copies):
        t = torch.empty(wbytes + 256, dtype=torch.uint8, device=dev)
        t[:wbytes].copy_(w0)
        weights.append((t, rq.Weight.wrap_device(t.data_ptr(), wbytes, rq.DTYPE_Q4_0, N_OUT, K_IN, t)))
    del w0
    x = torch.from_numpy(synth.activations(1, K_IN, SEED + 100).reshape(-1)).to(dev)
    y = torch.empty(N_OUT, dtype=torch.float32, device=dev)
    ms_per_step, kern_ms = rig.time_gemv(weights, x, y, args.steps, args.warmup)
    # each step is one launch of the GEMV kernel, back to back in the replayed
    # graph: the timed region's average launch duration
    kern_avg_ms = ms_per_step

    abytes = algorithmic_bytes(N_OUT, K_IN)
    value = abytes / (ms_per_step * 1e-3) / 1e9
    achieved = abytes / (kern_avg_ms * 1e-3) / 1e9

    parity_ok = exact_check(rig, weights[0][1], x, y, 1, N_OUT, K_IN)
    del weights
    torch.cuda.empty_cache()

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights x int4-digit x (v_dot8_i32_i4 -> i32), f32 combine",
        "data": "synthetic (seeded BASELINE config 2 bytes)",
        "config": {
            "workload": "config2: Q4_0 GEMV y=Wx, W 11008x4096 GGUF Q4_0, x f32[4096], batch 1, "
                        "float path (matmul_f32_q4, the Linear default); step = one fused prep+GEMV kernel",
            "weight_copies": args.copies,
            "weight_bytes_total": wbytes * args.copies,
            "algorithmic_bytes_per_step": abytes,
            "pct_of_hbm_peak": round(100 * value / PEAK_HBM_GBPS, 2),
            "parity_vs_exact": parity_ok,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_KEY.split("|")[0],
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "kernel_avg_us": round(kern_avg_ms * 1e3, 3),
            "eager_launch_avg_us": round(sum(kern_ms) / len(kern_ms) * 1e3, 3),
            "eager_launch_median_us": round(kern_ms[len(kern_ms) // 2] * 1e3, 3),
            "traffic": measured_traffic(KERNEL_KEY),
            "traffic_source": "profiles/gemv_q4_0_config2_pmc.md (FETCH_SIZE x2.0 + WRITE_SIZE, "
                              "scaled by a 256 MiB copy)",
        },
    }
    if wl == "all":
        sub_steps = min(args.steps, 500)
        sub_warm = min(args.warmup, 50)
        out["workloads"] = {
            "config1_q8_0": gemv_line(rig, "config1: Q8_0 GEMV 4096x4096", 8, 4096, 4096, 0x5EED0001,
                                      sub_steps, sub_warm, Q8_KEY),
            "config3_q4_k_up": gemv_line(rig, "config3 up: Q4_K GEMV 14336x4096", 12, 14336, 4096,
                                         0x5EED0003, sub_steps, sub_warm, Q4K_UP_KEY),
            "config3_q4_k_down": gemv_line(rig, "config3 down: Q4_K GEMV 4096x14336", 12, 4096, 14336,
                                           0x5EED0013, sub_steps, sub_warm, Q4K_DOWN_KEY),
            "q6_k_lm_head": gemv_line(rig, Q6K_LM_HEAD, 14, 32000, 4096, 0x5EED0006, sub_steps, sub_warm),
            "config4_gemm": gemm_lines(rig, [16, 64, 512, 2048]),
            "config4_gemm_native": gemm_lines(rig, [512, 2048], native=True),
            "config5_decode": decode_line(rig),
            "decode_q4_k_m": decode_q4_k_m_line(rig),
            "read_ceiling": read_lines(rig, sub_steps, sub_warm),
        }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if wl == "all":
            for key, (n, k, seed) in (("config3_q4_k_up", (14336, 4096, 0x5EED0003)),
                                      ("config3_q4_k_down", (4096, 14336, 0x5EED0013))):
                out["workloads"][key]["cpu_baseline"] = cpu_baseline_q4k(n, k, seed)
            out["workloads"]["config1_q8_0"]["cpu_baseline"] = cpu_baseline_q8()
            for line in out["workloads"]["config4_gemm"]:
                line["cpu_baseline"] = cpu_baseline_gemm(line["m"])
            out["workloads"]["config5_decode"]["cpu_baseline"] = cpu_baseline_decode()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
