"""Benchmark of the MI355X-native XTR-T5 Q4_K encoder (BASELINE.json metric).

One step = one full encoder forward (embedding -> 12 blocks -> final norm -> 768->128
projection + row norms) over one packed batch whose token ids are already resident in
HBM.  Default workload: cfg2, 32 sequences padded to 256 with true lengths U[32, 256]
(the reference runs them one at a time; here they are packed, so padding costs nothing).

Prints ONE JSON line.  Extra fields:
  roofline      -- the dominant kernel (batched FFN gate/up dequant-GEMM) vs f16 MFMA peak,
                   timed with HIP events on the model's stream inside this process;
  cpu_baseline  -- restatements of the reference's CPU encoder (oracle/: the default
                   t5-quantized f32 path on torch CPU GEMMs and in C, and the x86 default
                   hybrid-dequant + fbgemm numerics in C) on a bounded sample of the same
                   workload, batch-1 per sequence as the reference runs it;
  kernels       -- per-kernel-class averages from the same event timing;
  query         -- (cfg2) the cfg3 query regime: p50 / p95 latency over 1,000 queries cycling
                   8 model replicas, and its dominant GEMV against the HBM roofline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "XTR-base Q4_K encoder tokens/sec (32×256) + dequant-GEMM % roofline"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0    # MI355X dense int8 MFMA

WORKLOADS = {
    # name: (n_seqs, min_len, max_len, padded_len, description)
    "cfg2": (32, 32, 256, 256, "XTR-base Q4_K encoder, 32 seqs padded to 256, true lengths U[32,256]"),
    "cfg3": (1, 32, 32, 32, "XTR-base Q4_K encoder, query regime: batch 1, 32 tokens"),
    "cfg4": (256, 64, 512, 512, "XTR-base Q4_K encoder, bulk: 256 seqs padded to 512, lengths U[64,512]"),
    "cfg5": (64, 16, 512, 512, "XTR-base hybrid layout (F32 q/k/v/o/wo, Q4_K FFN), 64 seqs padded to 512, U[16,512]"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_info() -> dict:
    """The host the CPU baseline runs on: model name, logical CPUs, CPUs this process may run
    on, and the thread count it uses (the box's CPU share: OMP_NUM_THREADS when set)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or affinity
    return {"model": model, "nproc": os.cpu_count(), "affinity": affinity, "threads": min(share, affinity)}


def _time_per_sequence(fn, ids, cu, budget_s: float):
    """The reference harness's protocol (tools/t5-bench/src/main.rs:44-69), batch-1 per
    sequence: 1 warmup + median of 7, over as many sequences as fit the budget.
    Returns (tokens, seconds, sequences)."""
    tok, secs, used = 0, 0.0, 0
    t_start = time.perf_counter()
    for b in range(cu.size - 1):
        seq = ids[cu[b]:cu[b + 1]]
        fn(seq)
        times = []
        for _ in range(7):
            t = time.perf_counter()
            fn(seq)
            times.append(time.perf_counter() - t)
        tok += seq.size
        secs += sorted(times)[3]
        used += 1
        if time.perf_counter() - t_start > budget_s:
            break
    return tok, secs, used


def cpu_baseline(img: bytes, cfg: dict, ids: np.ndarray, cu: np.ndarray, budget_s: float,
                 variants_run=("f32_torch", "f32_c", "hybrid_bf16_c")) -> dict:
    """The reference's CPU encoder numerics timed on this host, per sequence as the reference
    runs them, split evenly over the restatements named in `variants_run` (test infrastructure
    under oracle/):
      f32_torch     -- the default t5-quantized path (Q4_K dequantized to f32 at load, f32 GEMMs,
                       src/quantized_t5.rs:39-49) on torch's multithreaded CPU GEMMs: the
                       strong-BLAS figure;
      f32_c         -- the same path in the C oracle's loops (OpenMP over output rows);
      hybrid_c      -- the hybrid-dequant feature: Q8_K x Q4_K integer dots for wi_0/wi_1/linear
                       with the Pade gelu, f32 q/k/v/o/wo (src/fused_matmul.rs:27-59,138-177);
      hybrid_bf16_c -- the x86 default build (hybrid-dequant + fbgemm, Makefile:26-30): the same
                       with bf16-truncated q/k/v/o/wo (fbgemm-rs/src/bf16.rs:21-25), in the C
                       oracle's scalar loops (no fbgemm assembly kernels).
    The value is the fastest variant, so the GPU/CPU ratio is the least flattering one."""
    from oracle import oracle as orc

    info = cpu_info()
    threads = info["threads"]
    used_omp = orc.set_threads(threads)
    variants = {}
    share = budget_s / len(variants_run)
    for name in variants_run:
        if name == "f32_torch":
            from oracle.torch_port import TorchCpuEncoder
            port = TorchCpuEncoder(img, cfg, threads=threads)
            tok, secs, n = _time_per_sequence(port.forward, ids, cu, share)
            del port
            variants[name] = {"tokens_per_s": tok / secs, "sequences": n, "tokens": tok, "threads": threads}
            continue
        var = {"f32_c": orc.VARIANT_DEFAULT, "hybrid_c": orc.VARIANT_HYBRID,
               "hybrid_bf16_c": orc.VARIANT_HYBRID_BF16}[name]
        m = orc.OracleModel(img, cfg, variant=var)
        tok, secs, n = _time_per_sequence(lambda s: m.forward(s, acc64=False), ids, cu, share)
        m.close()
        variants[name] = {"tokens_per_s": tok / secs, "sequences": n, "tokens": tok, "threads": used_omp}
    best = max(variants, key=lambda k: variants[k]["tokens_per_s"])
    v = variants[best]
    return {"value": v["tokens_per_s"], "unit": "tokens/s", "cores": v["threads"], "kind": "port",
            "sample": f"{best}: {v['sequences']} of {cu.size - 1} sequences ({v['tokens']} tokens), batch-1 each, "
                      f"median of 7 after 1 warmup; CPU {info['model']}, nproc {info['nproc']}, "
                      f"{info['affinity']} CPUs in this process's affinity, {threads} threads "
                      f"(this GPU box's CPU share)",
            "cpu": info, "variants": variants}


def kernel_table(model, step, n: int, reps: int = 20, unit: str = "step") -> dict:
    """Per kernel class: launches per step, and the average in-forward launch duration over `n`
    profiled forwards.  The library times each launch by HIP events bound to the kernel dispatch
    itself (hipExtLaunchKernelGGL start/stop events on the model's stream), so avg_us is the
    kernel's execution time inside the forward, the figure rocprofv3's kernel trace reports for
    the same dispatches.  relaunch_avg_us: `reps` back-to-back relaunches of the class's last
    launch (t5h_replay_kernel), which run a few percent faster than inside the forward (the
    kernel's operands stay warm in L2 and the MALL).  Profiled forwards run on one lane, so a
    batch that normally splits across two streams is timed kernel by kernel on one.  Algorithmic
    FLOP and bytes per launch come from the library."""
    model.set_profiling(True)
    for _ in range(n):
        step()
    model.synchronize()
    stats = model.kernel_stats()
    out = {}
    for name, s in stats.items():
        if not s["launches"]:
            continue
        us = s["total_ms"] / s["launches"] * 1e3
        per = s["launches"] / n
        k = {f"launches_per_{unit}": per, "avg_us": us, "ms_per_step": us * per * 1e-3,
             "relaunch_avg_us": model.replay_kernel(s["kind"], reps)}
        if s["flops"]:
            k["flops_per_launch"] = s["flops"] / s["launches"]
            k["tflops"] = k["flops_per_launch"] / (us * 1e-6) / 1e12
            k["mfma_frac"] = k["tflops"] / PEAK_F16_TFLOPS
        if s["bytes"]:
            k["bytes_per_launch"] = s["bytes"] / s["launches"]
            k["gbs"] = k["bytes_per_launch"] / (us * 1e-6) / 1e9
            k["hbm_frac"] = k["gbs"] / PEAK_HBM_GBS
        out[name] = k
    model.set_profiling(False)
    return out


QUERY_BYTES = 47_947_392  # cfg3 per query: Q4_K weights + embedding rows + bias table + output + ids


def query_kernel_table(models, query, n: int) -> dict:
    """kernel_table for the query regime: `n` profiled queries cycling over every replica (so the
    GEMVs stream their weights as the timed queries do), per-class stats summed over the replicas;
    relaunch_avg_us from replica 0 (its weights warm in the MALL after the first relaunch)."""
    for m in models:
        m.set_profiling(True)
    for i in range(n):
        query(i)
    for m in models:
        m.synchronize()
    acc = {}
    for m in models:
        for name, st in m.kernel_stats().items():
            a = acc.setdefault(name, {"kind": st["kind"], "launches": 0, "total_ms": 0.0, "flops": 0.0, "bytes": 0.0})
            for f in ("launches", "total_ms", "flops", "bytes"):
                a[f] += st[f]
    out = {}
    for name, st in acc.items():
        if not st["launches"]:
            continue
        us = st["total_ms"] / st["launches"] * 1e3
        per = st["launches"] / n
        k = {"launches_per_query": per, "avg_us": us, "ms_per_step": us * per * 1e-3,
             "relaunch_avg_us": models[0].replay_kernel(st["kind"], 20)}
        if st["flops"]:
            k["flops_per_launch"] = st["flops"] / st["launches"]
            k["tflops"] = k["flops_per_launch"] / (us * 1e-6) / 1e12
            k["mfma_frac"] = k["tflops"] / PEAK_F16_TFLOPS
        if st["bytes"]:
            k["bytes_per_launch"] = st["bytes"] / st["launches"]
            k["gbs"] = k["bytes_per_launch"] / (us * 1e-6) / 1e9
            k["hbm_frac"] = k["gbs"] / PEAK_HBM_GBS
        out[name] = k
    for m in models:
        m.set_profiling(False)
    return out


def profiled_traffic(tag: str, cls: str, applies: bool):
    """HBM bytes per dispatch of kernel class `cls` from profiles/<tag>_traffic.json (rocprofv3
    FETCH_SIZE and WRITE_SIZE passes of this workload through bench.py --counter-pass, each scaled
    by the same counter's reading for a plain copy of known size; bench.py --summarize writes the
    file), or None when there is no such pass for this exact workload."""
    f = ROOT / "profiles" / f"{tag}_traffic.json"
    if not applies or not f.exists():
        return None
    t = json.loads(f.read_text())["bytes_per_dispatch"].get(cls)
    return t["fetch"] + t["write"] if t else None


def run_query(args, img: bytes | None = None, cpu: bool = True) -> dict:
    """cfg3 (query regime): B = 1, L = 32 tokens, one forward per query from HBM-resident ids,
    latency p50/p95 over `--queries` queries (>= 1000).  The queries cycle over `--rotate`
    independent model replicas (default 8: 8 x 47.8 MB of Q4_K weights > the 256 MB MALL), so
    weights stream from HBM as in a cold query; --rotate 1 measures the warm case.  Also the
    dominant GEMV class from HIP events on the model's stream (one replica) against the HBM
    roofline, and the CPU port's latency for the same queries."""
    import torch

    from witchcraft_amd import synth
    from witchcraft_amd.encoder import T5EncoderModel

    cfg = dict(synth.XTR_BASE)
    if img is None:
        img = synth.make_model(cfg, seed=args.seed)
    models = [T5EncoderModel.from_gguf(img, cfg, hip_device=0) for _ in range(args.rotate)]
    L = 32
    rng = np.random.default_rng(2000 + args.seed)
    pool = rng.integers(1, cfg["vocab_size"], size=(64, L)).astype(np.int32)
    cu = np.array([0, L], np.int32)
    dev = torch.device("cuda:0")
    d_ids = [torch.from_numpy(q).to(dev) for q in pool]
    d_out = torch.empty((L, cfg["proj_dim"]), dtype=torch.float32, device=dev)
    d_norm = torch.empty(L, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def query(i):
        m = models[i % len(models)]
        m.encode_device(d_ids[i % len(d_ids)].data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())
        m.synchronize()

    for i in range(max(args.warmup, 2 * len(models))):
        query(i)
    lat = np.empty(args.queries)
    t_all = time.perf_counter()
    for i in range(args.queries):
        t = time.perf_counter()
        query(i)
        lat[i] = time.perf_counter() - t
    wall = time.perf_counter() - t_all
    p50, p95 = float(np.percentile(lat, 50) * 1e6), float(np.percentile(lat, 95) * 1e6)
    log(f"[bench] cfg3: {args.queries} queries over {len(models)} replicas: p50 {p50:.1f} us, p95 {p95:.1f} us")

    # per-kernel in-forward durations over rotated queries (weights streamed as in the timed
    # queries) -> dominant GEMV class vs the HBM roofline
    kernels = query_kernel_table(models, query, 10 * len(models))
    for mm in models:
        mm.close()
    gemv = {k: v for k, v in kernels.items() if k.startswith("gemm_")}
    dom_name = max(gemv, key=lambda k: gemv[k]["ms_per_step"])
    dom = gemv[dom_name]
    avg_s = dom["avg_us"] * 1e-6
    bytes_per_launch = dom["bytes_per_launch"]
    achieved = bytes_per_launch / avg_s / 1e9
    res = {"workload": "cfg3: XTR-base Q4_K encoder, query regime: batch 1, 32 tokens",
           "p50_us": p50, "p95_us": p95, "queries": args.queries, "replicas_rotated": len(models),
           "queries_per_s": args.queries / wall,
           "query_bytes": QUERY_BYTES, "query_floor_us": QUERY_BYTES / PEAK_HBM_GBS / 1e3,
           "whole_query_hbm_frac": QUERY_BYTES / (p50 * 1e-6) / 1e9 / PEAK_HBM_GBS,
           "roofline": {"kernel": f"{dom_name} (Q4_K GEMV, M = 32)", "bound": "hbm", "achieved": achieved,
                        "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                        "traffic": profiled_traffic("query_cfg3", dom_name, args.seed == 0 and len(models) == 8),
                        "bytes_per_launch": bytes_per_launch, "avg_launch_us": avg_s * 1e6},
           "kernels": kernels, "cpu_baseline": None}
    if cpu and not args.no_cpu_baseline:
        from oracle.torch_port import TorchCpuEncoder
        info = cpu_info()
        port = TorchCpuEncoder(img, cfg, threads=info["threads"])
        port.forward(pool[0])
        times = []
        t0 = time.perf_counter()
        for i in range(64):
            t = time.perf_counter()
            port.forward(pool[i])
            times.append(time.perf_counter() - t)
            if time.perf_counter() - t0 > min(args.cpu_budget, 5.0):
                break
        res["cpu_baseline"] = {"value": float(np.percentile(times, 50) * 1e6), "unit": "us/query (p50)",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"{len(times)} queries of 32 tokens, batch-1, f32 dequantize-at-load "
                                         f"path on torch CPU GEMMs; CPU {info['model']}"}
    return res


def query_bench(args) -> None:
    """cfg3 as its own line: value = p50 latency per query."""
    q = run_query(args)
    line = {
        "metric": "XTR-base Q4_K query encode latency p50 (B=1, L=32)", "value": q["p50_us"], "unit": "us",
        "n_gpus": 1, "steps": args.queries, "warmup": args.warmup, "ms_per_step": q["p50_us"] * 1e-3,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": q["workload"], "global_batch": 1, "seq_len": 32,
                   "replicas_rotated": q["replicas_rotated"], "p95_us": q["p95_us"],
                   "queries_per_s": q["queries_per_s"], "parallelism": "single GPU"},
        "roofline": q["roofline"], "cpu_baseline": q["cpu_baseline"], "kernels": q["kernels"],
        "query_bytes": q["query_bytes"], "query_floor_us": q["query_floor_us"],
    }
    print(json.dumps(line), flush=True)


PEAK_F32_MFMA_TFLOPS = 157.3  # MI355X dense f32 MFMA


def _event_time(torch, fn, reps: int) -> float:
    """Average seconds per call of `fn` over `reps` back-to-back launches, from HIP events on
    torch's current stream (the stream the scoring kernels are enqueued on)."""
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def score_bench(args) -> None:
    """Query-side scoring (src/lib.rs:734-735): 32 query-token embeddings x N indexed residual
    embeddings (128-d f32) -> [32, N] scores, one matmul_t per step, all buffers resident in
    HBM.  HBM-bound: N*512 B of residuals + 32*N*4 B of scores per launch.  Also reports the
    k-means assignment step (src/lib.rs:233-236): matmul_argmax of `--kmeans-m` sampled rows
    against `--kmeans-k` centers, f32 MFMA-bound, in the f32 (candle) and bf16-B (fbgemm)
    numerics."""
    import torch

    from witchcraft_amd import score

    M, D, N = 32, 128, args.score_n
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn((M, D), device=dev, generator=g)
    q /= q.norm(dim=1, keepdim=True)
    res = torch.randn((N, D), device=dev, generator=g) * 0.1
    out = torch.empty((M, N), device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()

    def step():
        score.matmul_t_device(q.data_ptr(), M, res.data_ptr(), N, D, out.data_ptr(), stream=stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t = time.perf_counter()
    avg_s = _event_time(torch, step, args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    value = M * N * args.steps / elapsed
    bytes_per_launch = N * D * 4 + M * D * 4 + M * N * 4
    achieved = bytes_per_launch / avg_s / 1e9
    log(f"[bench] score: {args.steps} x matmul_t [{M},{D}]x[{N},{D}]^T: {avg_s * 1e6:.1f} us/launch, "
        f"{achieved:.0f} GB/s")

    traffic = None
    tfile = ROOT / "profiles" / "score_traffic.json"
    if N == 1 << 20 and tfile.exists():
        t = json.loads(tfile.read_text())["bytes_per_dispatch"]["matmul_t_stream_kernel"]
        traffic = t["fetch"] + t["write"]

    # The same scores straight from 4-bit residual codes (src/lib.rs:676-680,734-735 without the
    # f32 residual matrix): N*64 B of codes + 32*N*4 B of scores per launch.
    from witchcraft_amd import codec
    codes = torch.randint(0, 256, (N, D // 2), dtype=torch.uint8, device=dev, generator=g)

    def qstep():
        codec.matmul_t_q4_device(q.data_ptr(), M, codes.data_ptr(), N, D, out.data_ptr(), stream=stream)

    qstep()
    qs = _event_time(torch, qstep, args.steps)
    q_bytes = N * D // 2 + M * D * 4 + M * N * 4
    q_tf = 2.0 * M * N * D / qs / 1e12
    # bf16 MFMAs with both operands split in three parts: 6 bf16 products per f32 product
    q4 = {"kernel": "matmul_t_q4_split_kernel (code bytes -> LDS table of bf16 hi/mid/lo pairs -> "
                    "6 x v_mfma_f32_16x16x32_bf16 per block)",
          "bound": "hbm", "avg_launch_us": qs * 1e6, "bytes_per_launch": q_bytes, "gbs": q_bytes / qs / 1e9,
          "hbm_frac": q_bytes / qs / 1e9 / PEAK_HBM_GBS, "tflops_f32_equivalent": q_tf,
          "bf16_mfma_frac": 6 * q_tf / PEAK_F16_TFLOPS,
          "scores_per_s": M * N / qs, "speedup_vs_f32_residuals": avg_s / qs}
    log(f"[bench] score from q4 codes: {qs * 1e6:.1f} us/launch ({avg_s / qs:.2f}x the f32 residuals), "
        f"{q_bytes / qs / 1e9:.0f} GB/s, {q_tf:.1f} TFLOP/s f32-equivalent")

    # Index build: residual codes of N embeddings against their assigned centres
    # (src/lib.rs:1375-1376): N*512 B in, N*64 B out (centres stay in L2).
    kc = 1 << 14
    cent_e = torch.randn((kc, D), device=dev, generator=g)
    asg_e = torch.randint(0, kc, (N,), dtype=torch.int32, device=dev, generator=g)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)

    def estep():
        codec.residual_encode_device(res.data_ptr(), N, cent_e.data_ptr(), kc, asg_e.data_ptr(), D,
                                     codes.data_ptr(), bad.data_ptr(), stream=stream)

    estep()
    es = _event_time(torch, estep, args.steps)
    e_bytes = N * D * 4 + N * 4 + N * D // 2
    enc = {"kernel": "residual_encode_kernel (threshold ladder)", "avg_launch_us": es * 1e6,
           "rows_per_s": N / es, "bytes_per_launch": e_bytes, "gbs": e_bytes / es / 1e9,
           "hbm_frac": e_bytes / es / 1e9 / PEAK_HBM_GBS}
    log(f"[bench] residual encode [{N}x{D}]: {es * 1e6:.1f} us, {e_bytes / es / 1e9:.0f} GB/s")

    # k-means assignment: compute-bound leg
    km, kk = args.kmeans_m, args.kmeans_k
    data = torch.randn((km, D), device=dev, generator=g)
    cent = torch.randn((kk, D), device=dev, generator=g)
    asg = torch.empty(km, dtype=torch.int32, device=dev)
    kmeans = {}
    for bf in (False, True):
        def kstep(bf=bf):
            score.matmul_argmax_device(data.data_ptr(), km, cent.data_ptr(), kk, D, asg.data_ptr(), bf16_b=bf,
                                       stream=stream)
        kstep()
        ks = _event_time(torch, kstep, max(3, args.steps // 4))
        tf = 2.0 * km * kk * D / ks / 1e12
        kmeans["bf16_b" if bf else "f32"] = {"avg_launch_us": ks * 1e6, "tflops": tf,
                                             "mfma_frac": tf / PEAK_F32_MFMA_TFLOPS}
        log(f"[bench] kmeans assign {'bf16_b' if bf else 'f32'} [{km}x{kk}]: {ks * 1e3:.2f} ms, {tf:.1f} TFLOP/s")

    base = None
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        threads = orc.set_threads(cpu_info()["threads"])
        r = np.random.default_rng(args.seed)
        ns = 1 << 17
        qa = r.standard_normal((M, D)).astype(np.float32)
        rb = r.standard_normal((ns, D)).astype(np.float32)
        orc.matmul_t(qa, rb, acc64=False)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_budget, 10.0) or reps == 0:
            orc.matmul_t(qa, rb, acc64=False)
            reps += 1
        cpu_s = (time.perf_counter() - t0) / reps
        base = {"value": M * ns / cpu_s, "unit": "scores/s", "cores": threads, "kind": "port",
                "sample": f"{reps} x matmul_t [{M},{D}]x[{ns},{D}]^T in the C oracle (scalar loop per "
                          f"dot product, OpenMP over query rows)"}
        ce = r.standard_normal((kc, D)).astype(np.float32)
        ca = r.integers(0, kc, ns).astype(np.uint32)
        orc.residual_encode(rb, ce, ca)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 3.0 or reps == 0:
            orc.residual_encode(rb, ce, ca)
            reps += 1
        enc["cpu_rows_per_s"] = ns * reps / (time.perf_counter() - t0)
        enc["cpu_sample"] = f"{reps} x residual_encode of {ns} rows in the C oracle, OpenMP over rows, {threads} threads"
    line = {
        "metric": "query x residual scores/sec (fast_ops::matmul_t, 32 x N x 128 f32)", "value": value,
        "unit": "scores/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"score: 32 query tokens x {N} residual embeddings (d=128), f32, resident in HBM",
                   "M": M, "N": N, "D": D, "parallelism": "single GPU"},
        "roofline": {"kernel": "matmul_t_stream_kernel (persistent, v_mfma_f32_16x16x4_f32)", "bound": "hbm",
                     "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                     "traffic": traffic, "bytes_per_launch": bytes_per_launch, "avg_launch_us": avg_s * 1e6},
        "q4_scoring": q4,
        "residual_encode": enc,
        "kmeans_assign": {"kernel": "matmul_argmax_kernel", "M": km, "N": kk, "D": D, "bound": "mfma",
                          "peak_tflops": PEAK_F32_MFMA_TFLOPS, **kmeans},
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)


def embed_bench(args) -> None:
    """Embedder::embed over a batch of documents (src/embedder.rs:22-103, called once per
    document by Gatherer::next, src/lib.rs:930-934): `--embed-docs` documents of U[10, 5000]
    token ids, windows of 2048 overlapping by 256.  The value is document tokens/s of one
    t5h_embed_batch call (every window of every document in one packed encode; window sums,
    MIN_NORM filter and compaction on the GPU), host buffers in and out, so the PCIe copies of
    the ids and the kept rows are inside the timed region.  Reported beside it: the same
    documents through t5h_embed_ids one after another, as the reference's loop runs them."""
    from witchcraft_amd import synth
    from witchcraft_amd.encoder import T5EncoderModel

    cfg = dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=args.seed)
    model = T5EncoderModel.from_gguf(img, cfg, hip_device=0)
    r = np.random.default_rng(3000 + args.seed)
    lens = r.integers(10, 5001, args.embed_docs)
    docs = [r.integers(1, cfg["vocab_size"], n).astype(np.uint32) for n in lens]
    ntok = int(lens.sum())
    model.embed_batch(docs)  # warm-up: workspace and staging sized once
    t_batch = []
    for _ in range(max(3, args.steps // 4)):
        t = time.perf_counter()
        res = model.embed_batch(docs)
        t_batch.append(time.perf_counter() - t)
    tb = float(np.median(t_batch))
    kept = sum(k.size for _, k in res)
    t = time.perf_counter()
    for d in docs:
        model.embed_ids(d)
    tl = time.perf_counter() - t
    log(f"[bench] embed: {len(docs)} documents, {ntok} tokens: batch {tb * 1e3:.1f} ms "
        f"({ntok / tb:,.0f} tokens/s), one at a time {tl * 1e3:.1f} ms ({ntok / tl:,.0f} tokens/s), kept {kept}")
    kernels = kernel_table(model, lambda: model.embed_batch(docs), 2)
    model.close()
    base = None
    if not args.no_cpu_baseline:
        from oracle.torch_port import TorchCpuEncoder
        info = cpu_info()
        port = TorchCpuEncoder(img, cfg, threads=info["threads"])
        t0, done = time.perf_counter(), 0
        for d in docs:
            n, k = d.size, 0
            while True:  # the reference's windows: start k * 1792 until a window reaches the end
                port.forward(d[k * 1792:min(k * 1792 + 2048, n)])
                if k * 1792 + 2048 >= n:
                    break
                k += 1
            done += n
            if time.perf_counter() - t0 > min(args.cpu_budget, 20.0):
                break
        cpu = time.perf_counter() - t0
        base = {"value": done / cpu, "unit": "tokens/s", "cores": info["threads"], "kind": "port",
                "sample": f"{done} document tokens, windows encoded one by one (batch-1) on torch CPU GEMMs "
                          f"(f32 dequantize-at-load path); CPU {info['model']}"}
    line = {
        "metric": "XTR-base Q4_K document embedding tokens/sec (t5h_embed_batch, windows 2048/256)",
        "value": ntok / tb, "unit": "tokens/s", "n_gpus": 1, "steps": len(t_batch), "warmup": 1,
        "ms_per_step": tb * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"embed: {len(docs)} documents of U[10, 5000] token ids, {ntok} tokens",
                   "kept_rows": kept, "one_at_a_time_tokens_per_s": ntok / tl,
                   "batch_over_one_at_a_time": tl / tb, "parallelism": "single GPU",
                   "note": "host buffers in and out: PCIe copies inside the timed region"},
        "cpu_baseline": base, "kernels": kernels,
    }
    print(json.dumps(line), flush=True)


def codec_bench(args) -> None:
    """Chunk-embedding codec after the encoder (src/lib.rs:1091 embeddings_to_packed per chunk,
    decoded at :712,1178,1296): a batch of `--codec-docs` matrices of L ~ U[64, 512] unit
    128-d rows (the cfg4 document lengths), packed and unpacked in one GPU call each.  The
    value is the encoder side's throughput in embedding rows/s over the GPU time of the call's
    kernels (inputs already in HBM; the call's own PCIe copies are reported separately)."""
    from witchcraft_amd import codec

    r = np.random.default_rng(args.seed)
    lens = r.integers(64, 513, args.codec_docs)
    mats = []
    for L in lens:
        base = r.normal(0, 1, 128)
        x = base + np.cumsum(r.normal(0, 0.15, (L, 128)), axis=0) + r.normal(0, 0.3, (L, 128))
        mats.append((x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32))
    rows = int(lens.sum())
    packed, _ = codec.embeddings_to_packed_batch(mats, timing=True)  # warm-up
    enc_ms, dec_ms, wall = [], [], []
    for _ in range(max(3, args.steps // 4)):
        t = time.perf_counter()
        packed, ms = codec.embeddings_to_packed_batch(mats, timing=True)
        wall.append(time.perf_counter() - t)
        enc_ms.append(ms)
        _, ms = codec.embeddings_from_packed_batch(packed, 128, timing=True)
        dec_ms.append(ms)
    enc = sorted(enc_ms)[len(enc_ms) // 2] * 1e-3
    dec = sorted(dec_ms)[len(dec_ms) // 2] * 1e-3
    nbytes = sum(len(b) for b in packed)
    log(f"[bench] codec: {len(mats)} chunks, {rows} rows: pack {enc * 1e3:.2f} ms GPU "
        f"({rows / enc:.3g} rows/s), unpack {dec * 1e3:.2f} ms GPU, {8 * nbytes / (rows * 128):.2f} bits/value")
    base = None
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        sample = mats[: max(1, len(mats) // 8)]
        srows = sum(m.shape[0] for m in sample)
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_budget, 10.0) or reps == 0:
            for m in sample:
                orc.embeddings_to_packed(m)
            reps += 1
        cpu = (time.perf_counter() - t0) / reps
        base = {"value": srows / cpu, "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"{reps} x embeddings_to_packed of {len(sample)} chunks ({srows} rows) in the C oracle, "
                          f"one chunk after another on one thread as src/lib.rs:1091 does"}
    line = {
        "metric": "packed chunk-embedding encode rows/sec (embeddings_to_packed, 128-d)", "value": rows / enc,
        "unit": "rows/s", "n_gpus": 1, "steps": len(enc_ms), "warmup": 1, "ms_per_step": enc * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"codec: {len(mats)} chunks of L ~ U[64,512] unit 128-d rows ({rows} rows)",
                   "parallelism": "single GPU"},
        "decode_rows_per_s": rows / dec, "decode_ms": dec * 1e3, "bits_per_value": 8 * nbytes / (rows * 128),
        "encode_call_wall_ms": sorted(wall)[len(wall) // 2] * 1e3,
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)


NUMERICS = {"default": 0, "hybrid": 1, "hybrid_bf16": 2}


def run_batched(args, workload: str, numerics: str, steps: int, warmup: int, cpu_variants=None,
                cpu_budget: float = 0.0, img: bytes | None = None, ffn_one_launch: bool = False) -> dict:
    """One batched workload (cfg2 / cfg4 / cfg5): `warmup` untimed forwards, then `steps` forwards
    timed from the host between device synchronisations (whole-job tokens/s, ids resident in
    HBM), then the per-class in-forward kernel table, the dominant GEMM class against its
    matrix-core roofline, and the CPU baseline on a bounded sample (cpu_variants, or none).
    ffn_one_launch: also time the same batch with the gated FFN as one launch that keeps the d_ff
    intermediate on chip (T5H_FFN_FUSED; bit-identical, not the default) next to the two launches."""
    import torch

    from witchcraft_amd import synth
    from witchcraft_amd.encoder import T5EncoderModel

    n_seqs, lo, hi, pad, desc = WORKLOADS[workload]
    cfg = dict(synth.XTR_BASE)
    if img is None:
        t0 = time.perf_counter()
        img = synth.make_model(cfg, seed=args.seed, layout="hybrid" if workload == "cfg5" else "q4k")
        log(f"[bench] {workload}: model built in {time.perf_counter() - t0:.1f}s ({len(img) / 1e6:.1f} MB GGUF)")
    model = T5EncoderModel.from_gguf(img, cfg, hip_device=0)
    model.set_numerics(NUMERICS[numerics])
    ids, cu = synth.ragged_batch(n_seqs, lo, hi, cfg["vocab_size"], seed=1000 + args.seed)
    T = int(cu[-1])
    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids.astype(np.int32)).to(dev)
    d_out = torch.empty((T, cfg["proj_dim"]), dtype=torch.float32, device=dev)
    d_norm = torch.empty(T, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step():
        model.encode_device(d_ids.data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())

    for _ in range(warmup):
        step()
    model.synchronize()

    # ---- timed region: whole-job throughput ----
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(steps):
        step()
    model.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    ms_per_step = elapsed / steps * 1e3
    value = T * steps / elapsed
    log(f"[bench] {workload} ({numerics}): {steps} steps, {ms_per_step:.3f} ms/step, {value:,.0f} tokens/s")
    res = {"workload": f"{workload}: {desc}", "value": value, "unit": "tokens/s", "ms_per_step": ms_per_step,
           "steps": steps, "warmup": warmup, "tokens_per_step": T, "global_batch": n_seqs, "seq_len": pad,
           "numerics": numerics}
    if args.counter_pass:
        model.close()
        return res

    # ---- per-kernel in-forward durations; dominant GEMM class vs the matrix-core roofline ----
    kernels = kernel_table(model, step, min(steps, 10))
    model.close()
    gemms = {k: v for k, v in kernels.items() if k.startswith("gemm_")}
    dom_name = max(gemms, key=lambda k: gemms[k]["ms_per_step"])
    dom = gemms[dom_name]
    avg_s = dom["avg_us"] * 1e-6
    flops_per_launch = dom["flops_per_launch"]
    achieved = flops_per_launch / avg_s / 1e12
    tag = f"encoder_{workload}" + ("" if numerics == "default" else f"_{numerics}")
    applies = args.seed == 0
    counters = None
    tfile = ROOT / "profiles" / f"{tag}_traffic.json"
    if applies and tfile.exists():
        c = json.loads(tfile.read_text()).get("counters", {}).get(dom_name)
        if c:
            # MFMA work the counters saw the class's launches execute, over the in-forward duration
            # measured here, and the share of SIMD cycles the matrix cores were busy
            counters = {"mfma_flop_executed": c["mfma_flop_executed"],
                        "tflops_executed": c["mfma_flop_executed"] / avg_s / 1e12,
                        "frac_executed": c["mfma_flop_executed"] / avg_s / 1e12 / PEAK_F16_TFLOPS,
                        "mfma_busy_frac": c["mfma_busy_frac"],
                        "source": f"profiles/{tag}_traffic.json (rocprofv3 --pmc through bench.py)"}
    roofline = {"kernel": f"{dom_name} (Q4_K dequant-GEMM, v_mfma_f32_16x16x32_f16)",
                "bound": "mfma", "achieved": achieved, "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / PEAK_F16_TFLOPS, "traffic": profiled_traffic(tag, dom_name, applies),
                "flops_per_launch": flops_per_launch, "avg_launch_us": avg_s * 1e6,
                "relaunch_avg_us": dom["relaunch_avg_us"],
                "share_of_step": dom["ms_per_step"] / sum(v["ms_per_step"] for v in kernels.values()),
                "counters": counters}
    if numerics != "default" and dom_name in ("gemm_ffn_gate_up", "gemm_proj"):
        # the hybrid FFN's products run as int8 MFMAs (two weight planes per product, so the
        # matrix cores execute twice the algorithmic ops counted here), after the Q8_K quantizer
        roofline.update({"kernel": f"{dom_name} (Q8_K quantize + Q4_K x Q8_K on v_mfma_i32_16x16x64_i8)",
                         "unit": "TOP/s", "peak": PEAK_INT8_TOPS, "frac": achieved / PEAK_INT8_TOPS})
    roofline["library_reference"] = library_gemm(torch, dom_name, cfg, T)
    res.update({"roofline": roofline, "kernels": kernels, "cpu_baseline": None})
    if ffn_one_launch and numerics == "default":
        res["ffn_one_launch"] = ffn_one_launch_leg(img, cfg, cu, d_ids, d_out, d_norm, kernels, T)
    if cpu_variants and not args.no_cpu_baseline:
        log(f"[bench] {workload}: CPU baseline ({', '.join(cpu_variants)}, bounded sample) ...")
        res["cpu_baseline"] = cpu_baseline(img, cfg, ids, cu, cpu_budget, cpu_variants)
    res["_img"] = img
    return res


def ffn_one_launch_leg(img: bytes, cfg: dict, cu, d_ids, d_out, d_norm, kernels: dict, T: int,
                       steps: int = 5) -> dict:
    """The gated FFN as one launch per layer (k_ffn.hip: 64-token tiles, h kept in LDS, never
    written to memory; the same bits as the two launches), on a second handle created with
    T5H_FFN_FUSED=1: whole-step time over `steps` forwards and its in-forward kernel time, next to
    the default two launches (gate|up + wo) of the same batch from `kernels`."""
    import torch

    from witchcraft_amd.encoder import T5EncoderModel

    os.environ["T5H_FFN_FUSED"] = "1"
    try:
        fm = T5EncoderModel.from_gguf(img, cfg, hip_device=0)
    finally:
        del os.environ["T5H_FFN_FUSED"]
    try:
        def step():
            fm.encode_device(d_ids.data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())

        for _ in range(2):
            step()
        fm.synchronize()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            step()
        fm.synchronize()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t) / steps * 1e3
        fk = kernel_table(fm, step, 3).get("ffn_fused")
    finally:
        fm.close()
    two = sum(kernels[k]["avg_us"] for k in ("gemm_ffn_gate_up", "gemm_ffn_wo") if k in kernels)
    out = {"kernel": "ffn_fused_kernel (one launch per layer, d_ff intermediate in LDS, bit-identical; "
                     "opt-in T5H_FFN_FUSED)",
           "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3), "two_launch_avg_us": two}
    if fk:
        out.update({"avg_us": fk["avg_us"], "tflops": fk.get("tflops"), "frac": fk.get("mfma_frac")})
    log(f"[bench] one-launch FFN: {ms:.3f} ms/step; ffn_fused {out.get('avg_us', float('nan')):.1f} us "
        f"vs gate|up + wo {two:.1f} us per layer (one lane)")
    return out


def library_gemm(torch, cls: str, cfg: dict, M: int, reps: int = 20):
    """The vendor library's plain f16 GEMM of the same shape as kernel class `cls` (M tokens):
    torch.mm on f16 operands, which runs hipBLASLt, with no dequantization and no fused epilogue.
    Average of `reps` back-to-back launches from HIP events on torch's current stream."""
    D, F, inner = cfg["d_model"], cfg["d_ff"], cfg["num_heads"] * cfg["d_kv"]
    shapes = {"gemm_ffn_gate_up": (2 * F, D), "gemm_qkv": (3 * inner, D), "gemm_o": (D, inner),
              "gemm_ffn_wo": (D, F), "gemm_proj": (cfg["proj_dim"], D)}
    if cls not in shapes:
        return None
    N, K = shapes[cls]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randn((M, K), device=dev, generator=g).half()
    w_t = (torch.randn((N, K), device=dev, generator=g) * 0.02).half().t().contiguous()  # [K, N]
    out = torch.empty((M, N), device=dev, dtype=torch.float16)
    for _ in range(3):
        torch.mm(a, w_t, out=out)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        torch.mm(a, w_t, out=out)
    e1.record(st)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
    return {"kernel": f"torch.mm f16 [{M},{K}] x [{K},{N}] (hipBLASLt; no dequantization, no epilogue)",
            "avg_us": us, "tflops": tf, "frac": tf / PEAK_F16_TFLOPS}


def summarize(args) -> None:
    """Reads rocprofv3 CSV output (kernel trace and/or counter collection, each pass in its own
    directory) and prints, per encoder kernel class, the average dispatch duration and the
    counters per dispatch; with --copy-fetch / --copy-write (passes of --copy-calibration) the
    FETCH_SIZE / WRITE_SIZE readings are scaled to bytes by the copy's known size.  --out writes
    the bytes per dispatch as the JSON file the bench line reads (profiles/<tag>_traffic.json)."""
    import csv
    import glob
    import re

    def rows(d, suffix):
        fs = glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)
        if not fs:
            raise SystemExit(f"summarize: no *{suffix} under {d}")
        out = []
        for f in fs:
            out += list(csv.DictReader(open(f)))
        return out

    def base_class(name):
        m = re.search(r"(gemm|gemv)_kernel(?:<|ILi)(-?\d+)", name)
        if m:
            return {"4": "gemm_qkv", "2": "gemm_ffn_gate_up", "5": "gemm_ffn_gate_up", "3": "gemm_proj",
                    "1": "resid"}.get(m.group(2))
        for key, cls in (("embed_kernel", "embed_gather"), ("rownorm_kernel", "rownorm"),
                         ("rmsnorm_kernel", "rmsnorm"), ("attn_relbias_kernel", "attention"),
                         ("q8k_quantize_kernel", "q8k_quantize"), ("ffn_fused_kernel", "ffn_fused"),
                         ("copyBuffer", "copy")):
            if key in name:
                return key if cls is None else cls
        return None

    def classify(rs, name_key, id_key):
        """Dispatch id -> class; the residual GEMM/GEMV is O after attention and FFN wo after the
        gated FFN (the forward's launch order; relaunches of one class follow each other)."""
        cls, prev = {}, None
        for r in sorted(rs, key=lambda r: int(r[id_key])):
            c = base_class(r[name_key])
            if c == "resid":
                c = "gemm_o" if prev in ("attention", "gemm_o") else "gemm_ffn_wo"
            if c:
                cls[int(r[id_key])] = c
                if c != "copy":
                    prev = c
        return cls

    summary = {"workload": args.summarize_workload, "classes": {}}
    if args.trace:
        tr = rows(args.trace, "kernel_trace.csv")
        cls = classify(tr, "Kernel_Name", "Dispatch_Id")
        acc = {}
        for r in tr:
            c = cls.get(int(r["Dispatch_Id"]))
            if c:
                a = acc.setdefault(c, [])
                a.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
        for c, v in acc.items():
            summary["classes"].setdefault(c, {}).update({"dispatches": len(v), "avg_us": sum(v) / len(v),
                                                         "total_ms": sum(v) * 1e-3})

    def per_dispatch(d):
        rs = rows(d, "counter_collection.csv")
        cls = classify({int(r["Dispatch_Id"]): r for r in rs}.values(), "Kernel_Name", "Dispatch_Id")
        acc = {}
        for r in rs:
            c = cls.get(int(r["Dispatch_Id"]))
            if c:
                acc.setdefault(c, {}).setdefault(r["Counter_Name"], {}).setdefault(int(r["Dispatch_Id"]), 0.0)
                acc[c][r["Counter_Name"]][int(r["Dispatch_Id"])] += float(r["Counter_Value"])
        return {c: {k: sum(v.values()) / len(v) for k, v in cc.items()} for c, cc in acc.items()}

    scale = {}
    for key, d in (("FETCH_SIZE", args.copy_fetch), ("WRITE_SIZE", args.copy_write)):
        if d:
            kib = per_dispatch(d)["copy"][key]
            scale[key] = args.copy_bytes / (kib * 1024.0)
    for d in args.counters or []:
        for c, vals in per_dispatch(d).items():
            summary["classes"].setdefault(c, {}).update(vals)
    traffic = {}
    for c, v in summary["classes"].items():
        if "FETCH_SIZE" in v and "WRITE_SIZE" in v and scale:
            traffic[c] = {"fetch": v["FETCH_SIZE"] * 1024 * scale.get("FETCH_SIZE", 1.0),
                          "write": v["WRITE_SIZE"] * 1024 * scale.get("WRITE_SIZE", 1.0)}
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in v:
            # f16 MFMA work in units of 512 FLOP, whatever the instruction shape
            v["mfma_flop_executed"] = v["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512
        elif "SQ_INSTS_VALU_MFMA_F16" in v and c != "attention":
            # an instruction count: the GEMMs run only 16x16x32 products (attention mixes shapes)
            v["mfma_flop_executed"] = v["SQ_INSTS_VALU_MFMA_F16"] * 16 * 16 * 32 * 2
        if "SQ_VALU_MFMA_BUSY_CYCLES" in v and "GRBM_GUI_ACTIVE" in v:
            v["mfma_busy_frac"] = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * v["GRBM_GUI_ACTIVE"] / 8)
    summary["scale"] = scale
    summary["bytes_per_dispatch"] = traffic
    print(json.dumps(summary, indent=1))
    if args.out:
        counters = {c: {k: v[k] for k in ("mfma_flop_executed", "mfma_busy_frac") if k in v}
                    for c, v in summary["classes"].items() if "mfma_flop_executed" in v and "mfma_busy_frac" in v}
        Path(args.out).write_text(json.dumps({
            "workload": args.summarize_workload,
            "source": "rocprofv3 --pmc passes of bench.py --counter-pass, summarised by bench.py --summarize",
            "fetch_scale": scale.get("FETCH_SIZE"), "write_scale": scale.get("WRITE_SIZE"),
            "bytes_per_dispatch": traffic, "counters": counters,
            "trace_avg_us": {c: v["avg_us"] for c, v in summary["classes"].items() if "avg_us" in v}}, indent=1) + "\n")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg2", choices=sorted(WORKLOADS) + ["score", "codec", "embed"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--queries", type=int, default=1000, help="cfg3: number of timed queries")
    ap.add_argument("--rotate", type=int, default=8, help="cfg3: model replicas cycled (MALL defeat)")
    ap.add_argument("--no-query", action="store_true", help="cfg2: leave out the cfg3 query object")
    ap.add_argument("--no-configs", action="store_true",
                    help="cfg2: leave out the cfg4 / cfg5 objects of the default line")
    ap.add_argument("--numerics", default="default", choices=sorted(NUMERICS),
                    help="batched workloads: t5h_set_numerics mode (hybrid: the hybrid-dequant "
                         "feature's Q8_K x Q4_K FFN and projection; hybrid_bf16: also bf16-truncated "
                         "q/k/v/o/wo, the x86 hybrid-dequant + fbgemm build)")
    ap.add_argument("--counter-pass", action="store_true",
                    help="only the warmup and timed forwards (cfg3: the rotated queries) of the workload, "
                         "for rocprofv3 --pmc passes whose dispatches should all be that workload's")
    ap.add_argument("--score-n", type=int, default=1 << 20, help="score: residual rows")
    ap.add_argument("--kmeans-m", type=int, default=1 << 17, help="score: k-means rows")
    ap.add_argument("--kmeans-k", type=int, default=1 << 14, help="score: k-means centers")
    ap.add_argument("--codec-docs", type=int, default=256, help="codec: chunks per batch")
    ap.add_argument("--embed-docs", type=int, default=64, help="embed: documents per batch")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB 10 times (the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--summarize", action="store_true",
                    help="summarise rocprofv3 CSV output (no GPU): --trace DIR, --counters DIR..., "
                         "--copy-fetch DIR / --copy-write DIR (passes of --copy-calibration), --out FILE")
    ap.add_argument("--trace", default=None)
    ap.add_argument("--counters", nargs="*", default=None)
    ap.add_argument("--copy-fetch", default=None)
    ap.add_argument("--copy-write", default=None)
    ap.add_argument("--copy-bytes", type=float, default=256 * (1 << 20))
    ap.add_argument("--summarize-workload", default="")
    ap.add_argument("--out", default=None)
    args = ap.parse_args()
    if args.summarize:
        summarize(args)
        return
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 10}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (got --gpus {args.gpus}); sequences are "
              "independent, so N GPUs would each run this workload on their own share.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "cfg3":
        if args.counter_pass:
            run_query_counter_pass(args)
        else:
            query_bench(args)
        return
    if args.workload == "score":
        score_bench(args)
        return
    if args.workload == "codec":
        codec_bench(args)
        return
    if args.workload == "embed":
        embed_bench(args)
        return

    w = args.workload
    main_cpu = ("f32_torch", "f32_c", "hybrid_bf16_c") if args.numerics == "default" else \
        (("hybrid_c",) if args.numerics == "hybrid" else ("hybrid_bf16_c",))
    r = run_batched(args, w, args.numerics, args.steps, args.warmup, main_cpu, args.cpu_budget)
    if args.counter_pass:
        print(json.dumps({"counter_pass": w, "numerics": args.numerics, "value": r["value"],
                          "tokens_per_step": r["tokens_per_step"]}), flush=True)
        return
    img = r.pop("_img")
    line = {
        "metric": METRIC, "value": r["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16" if args.numerics == "default" else "f16+int8", "data": "synthetic",
        "config": {"workload": r["workload"], "global_batch": r["global_batch"], "seq_len": r["seq_len"],
                   "tokens_per_step": r["tokens_per_step"],
                   "weights": "random-init N(0,0.02^2), Q4_K by the quantize tool's scale/min search "
                              "(t5h_quantize_q4k); f32 embeddings and norms",
                   "numerics": args.numerics, "parallelism": "single GPU"},
        "roofline": r["roofline"], "cpu_baseline": r["cpu_baseline"], "kernels": r["kernels"],
    }
    if w == "cfg2" and not args.no_configs:
        # The compute-bound configurations beside the headline, each timed the same way (fewer
        # steps), with its dominant GEMM's in-forward roofline and a small CPU sample.
        extra = {}
        budget = min(args.cpu_budget, 4.0)
        r4 = run_batched(args, "cfg4", "default", 10, 3, ("f32_torch",), budget, ffn_one_launch=True)
        r4.pop("_img")
        extra["cfg4"] = r4
        img5 = None
        for num, cv in (("default", ("f32_torch",)), ("hybrid", ("hybrid_c",)), ("hybrid_bf16", ("hybrid_bf16_c",))):
            r5 = run_batched(args, "cfg5", num, 10, 3, cv, budget, img=img5)
            img5 = r5.pop("_img")
            extra["cfg5" if num == "default" else f"cfg5_{num}"] = r5
        line["configs"] = extra
    if w == "cfg2" and not args.no_query:
        line["query"] = run_query(args, img if args.seed == 0 else None)
    print(json.dumps(line), flush=True)


def run_query_counter_pass(args) -> None:
    """cfg3 for rocprofv3 --pmc passes: the rotated queries only (no profiled queries, relaunches
    or CPU leg), so every dispatch of the run streams its weights as a timed query does."""
    import torch

    from witchcraft_amd import synth
    from witchcraft_amd.encoder import T5EncoderModel

    cfg = dict(synth.XTR_BASE)
    img = synth.make_model(cfg, seed=args.seed)
    models = [T5EncoderModel.from_gguf(img, cfg, hip_device=0) for _ in range(args.rotate)]
    L = 32
    pool = np.random.default_rng(2000 + args.seed).integers(1, cfg["vocab_size"], size=(64, L)).astype(np.int32)
    cu = np.array([0, L], np.int32)
    dev = torch.device("cuda:0")
    d_ids = [torch.from_numpy(q).to(dev) for q in pool]
    d_out = torch.empty((L, cfg["proj_dim"]), dtype=torch.float32, device=dev)
    d_norm = torch.empty(L, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for i in range(args.queries):
        m = models[i % len(models)]
        m.encode_device(d_ids[i % len(d_ids)].data_ptr(), cu, d_out.data_ptr(), d_norm.data_ptr())
        m.synchronize()
    for m in models:
        m.close()
    print(json.dumps({"counter_pass": "cfg3", "queries": args.queries, "replicas": len(models)}), flush=True)


if __name__ == "__main__":
    main()
