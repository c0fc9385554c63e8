"""Benchmark of the Q4_0 decode GEMV on one MI355X.

A step is one batch-1 Linear forward of the Llama-7B FFN up/gate shape
(W 11008x4096 GGUF Q4_0, x f32 [4096]) through the C ABI
(rdl_linear_forward_dev: one kernel, activation prep fused), i.e.
rustml_quant::matmul_f32_q4 (quantize.rs:265-320) with the weight resident in
HBM.  Consecutive steps use different weight copies (more than the 256 MB
Infinity Cache in total) so each step streams its weight from HBM.

Timed region: the K steps are captured once in a HIP graph (so host launch
overhead is not measured) and replayed once between two events.  The
roofline figure times each GEMV kernel at its boundaries (hipExtLaunchKernel
events) over K separate launches.

Prints one JSON line (see the keys below).
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
N_OUT, K_IN = 11008, 4096
SEED = 0x5EED0002
# the kernel the library launches for this workload (8-wave workgroups, 3 rows per wave)
KERNEL_KEY = "gemv_fused_kernel<2, false, 3, 2, true, 8>|config2"


def algorithmic_bytes(n, k):
    """Weight blocks + x (f32) + y (f32), each read or written once."""
    return n * (k // 32) * 18 + 4 * k + 4 * n


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
    import numpy as np

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
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{len(times)} single-thread matmul_f32_q4 calls, 11008x4096 Q4_0, M=1, "
                  f"median {med * 1e3:.2f} ms, weights rotated over {copies} copies "
                  f"(host nproc={os.cpu_count()})",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=24)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (a known-size "
                         "reference for HBM traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the GEMV runs on a single MI355X and multi-GPU "
              "runs are not part of this path (rows would shard across GPUs with an "
              "all-gather of y).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import rdlquant as rq
    from rdlquant import synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream

    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

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

    def step(i, s_handle):
        weights[i % len(weights)][1].forward_dev(x.data_ptr(), 1, y.data_ptr(), rq.MODE_FLOAT, s_handle)

    for i in range(args.warmup):
        step(i, sh)
    torch.cuda.synchronize()

    # capture the K steps in one graph; one untimed replay, then the timed one
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream().cuda_stream
        for i in range(args.steps):
            step(i, cap)
    graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps

    # kernel-boundary timing of the GEMV kernel over K separate launches
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for a, b in evs:  # materialize the events
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(evs):
        rq.time_next_launch(a.cuda_event, b.cuda_event)
        step(i, sh)
    torch.cuda.synchronize()
    kern_ms = sorted(a.elapsed_time(b) for a, b in evs)
    kern_avg_ms = sum(kern_ms) / len(kern_ms)

    abytes = algorithmic_bytes(N_OUT, K_IN)
    value = abytes / (ms_per_step * 1e-3) / 1e9
    achieved = abytes / (kern_avg_ms * 1e-3) / 1e9

    # correctness spot check of the last step against the oracle
    from oracle import oracle as orc

    want = orc.matmul("q4", synth.activations(1, K_IN, SEED + 100), w_host, 1, K_IN, N_OUT, threads=8)
    got = y.cpu().numpy()
    parity_ok = bool(np.all(np.abs(got - want) <= 1e-4 + 1e-3 * np.abs(want)))

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
            "parity_vs_oracle": parity_ok,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_KEY.split("|")[0],
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "kernel_avg_us": round(kern_avg_ms * 1e3, 3),
            "kernel_median_us": round(kern_ms[len(kern_ms) // 2] * 1e3, 3),
            "traffic": measured_traffic(KERNEL_KEY),
            "traffic_source": "profiles/gemv_q4_0_config2_pmc.md (FETCH_SIZE x2.0 + WRITE_SIZE, "
                              "scaled by a 256 MiB copy)",
        },
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
