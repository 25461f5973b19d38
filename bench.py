"""Benchmark: N:M sparse GEMV HBM throughput at Llama-3.1-8B decode shapes.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--ratio 32:64]

One step = every sparse GEMV of one Llama-3.1-8B decode token: 32 layers x
(q, k, v, o, gate, up, down) = 224 launches over 32 layers' distinct packed
weights (7.0 GB resident in HBM, far beyond the 256 MB Infinity Cache), fp16,
batch 1, captured once in a hipGraph and replayed. `value` is the algorithmic
bytes of the step (2*w*h weights + w index bytes + 2*K activations + 2*h
outputs per GEMV) divided by the step time.

Also reported: per-shape average launch time and GB/s for the sparse kernel
and for dense fp16 F.linear (hipBLASLt preferred) on the same shapes, the
roofline of the dominant kernel (HIP events on the launch stream), and a CPU
baseline (the oracle's gather-form GEMV on one layer's weights, host cores).
Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
LLAMA = {"n_layers": 32, "dim": 4096, "n_heads": 32, "n_kv_heads": 8, "head_dim": 128, "inter": 14336}
# name -> (K, h)
SHAPES = {
    "q_proj": (4096, 4096),
    "k_proj": (4096, 1024),
    "v_proj": (4096, 1024),
    "o_proj": (4096, 4096),
    "gate_proj": (4096, 14336),
    "up_proj": (4096, 14336),
    "down_proj": (14336, 4096),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def sparse_bytes(K: int, h: int, nnz: int, m: int) -> int:
    """Algorithmic bytes of one GEMV: packed weights, index bytes, activations, outputs."""
    w = (K // m) * nnz
    return 2 * w * h + w + 2 * K + 2 * h


def dense_bytes(K: int, h: int) -> int:
    return 2 * K * h + 2 * K + 2 * h


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--ratio", default="32:64", help="N:M (N kept of every M)")
    p.add_argument("--layers", type=int, default=LLAMA["n_layers"])
    p.add_argument("--no-dense", action="store_true", help="skip the dense hipBLASLt comparison")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    p.add_argument("--only-step", action="store_true", help="time only the sparse step (for profiling)")
    return p.parse_args()


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the path would shard by output rows / input groups across GPUs, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    nnz, m = (int(v) for v in args.ratio.split(":"))

    import torch
    
    from spmv_decode_amd import _lib, hip_spmv

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} ({getattr(props, 'gcnArchName', '?')}), {props.multi_processor_count} CUs")
    gen = torch.Generator(device=dev).manual_seed(0)

    # ---- synthetic resident weights: L layers x 7 Linears -----------------
    L = args.layers
    layers = []
    for li in range(L):
        lay = {}
        for name, (K, h) in SHAPES.items():
            banks = K // m
            keys = torch.rand(banks, m, generator=gen, device=dev)
            mi = keys.argsort(dim=1)[:, :nnz].sort(dim=1).values.to(torch.uint8).contiguous()
            md = (torch.randn(banks * nnz, h, generator=gen, device=dev) * 0.02).to(torch.float16)
            lay[name] = (md, mi)
        layers.append(lay)
    xs = {K: torch.randn(1, K, generator=gen, device=dev).to(torch.float16) for K in {4096, 14336}}
    outs = {name: torch.empty(1, h, dtype=torch.float16, device=dev) for name, (K, h) in SHAPES.items()}
    step_bytes = L * sum(sparse_bytes(K, h, nnz, m) for K, h in SHAPES.values())
    log(f"{L} layers x {len(SHAPES)} GEMVs at {nnz}:{m}: {step_bytes / 1e9:.3f} GB algorithmic per step")

    def gemv(name, li):
        K, h = SHAPES[name]
        md, mi = layers[li][name]
        return hip_spmv.nmsparse_spmv_forward_hip(xs[K], md, mi, md.shape[0], h, nnz, 128, m, 1, K,
                                                  out=outs[name])

    stream = torch.cuda.Stream(device=dev)

    def capture(fn):
        # eager warm-up on the capture stream creates its workspace, then capture
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        torch.cuda.synchronize()
        return g

    def step():
        for li in range(L):
            for name in SHAPES:
                gemv(name, li)

    # ---- the timed step ------------------------------------------------------
    g_step = capture(step)
    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        g_step.replay()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"step {ms_per_step:.4f} ms -> {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of {HBM_PEAK_GBS:.0f})")
    for name, (K, h) in SHAPES.items():
        if not torch.isfinite(outs[name].float()).all():
            raise RuntimeError(f"non-finite output for {name}")

    result = {
        "metric": "sparse GEMV HBM GB/s (% peak) + decode ms/token, Llama-3.1-8B-shape 32:64",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded on-device N(0,0.02) weights, random in-group patterns, N(0,1) activations)",
        "config": {
            "workload": f"Llama-3.1-8B decode-token sparse GEMVs: {L} layers x (q,k,v,o,gate,up,down) at {nnz}:{m}, "
                        "batch 1, fp16, hipGraph replay, distinct resident weights per layer",
            "ratio": f"{nnz}:{m}",
            "layers": L,
            "gemvs_per_step": L * len(SHAPES),
            "algorithmic_bytes_per_step": step_bytes,
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        },
    }
    if args.only_step:
        print(json.dumps(result), flush=True)
        return

    # ---- per-shape launch times, weights rotated over >= 1 GiB --------------
    from spmv_decode_amd import microbench as MB

    per_shape = {}
    classes = {"q_o": ("q_proj", "o_proj"), "k_v": ("k_proj", "v_proj"), "gate_up": ("gate_proj", "up_proj"),
               "down": ("down_proj",)}
    reps = max(10, args.steps // 2)
    for cls, names in classes.items():
        K, h = SHAPES[names[0]]
        case = MB.RotatingCase(h, K, nnz, m, torch.float16, rotate_bytes=1 << 30, seed=7)
        us = MB.time_sparse(case, reps=reps)
        b = sparse_bytes(K, h, nnz, m)
        plan = _lib.plan(h, (K // m) * nnz, nnz, m)
        per_shape[cls] = {"K": K, "h": h, "launches_per_step": L * len(names), "us_per_launch": round(us, 3),
                          "bytes_per_launch": b, "GBps": round(b / (us * 1e-6) / 1e9, 1),
                          "pct_peak": round(100 * b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
                          "kernel_config": plan["config"], "splits": plan["splits"], "blocks": plan["blocks"],
                          "rotated_copies": case.copies}
        log(f"sparse {cls:8s} K={K:5d} h={h:5d}: {us:7.2f} us/launch {per_shape[cls]['GBps']:7.1f} GB/s "
            f"({per_shape[cls]['pct_peak']}%) {plan} x{case.copies} copies")
        del case
        torch.cuda.empty_cache()
    # dominant kernel: largest share of the step
    dom = max(per_shape, key=lambda c: per_shape[c]["us_per_launch"] * per_shape[c]["launches_per_step"])
    d = per_shape[dom]
    result["roofline"] = {
        "bound": "hbm",
        "achieved": d["GBps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(d["GBps"] / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": f"nm_gemv_kernel {d['kernel_config']} ({dom}: K={d['K']} h={d['h']}, {nnz}:{m})",
        "bytes_per_launch": d["bytes_per_launch"],
        "us_per_launch": d["us_per_launch"],
    }
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.exists():
        t = json.loads(traffic_file.read_text()).get(f"{dom}_{nnz}:{m}")
        if t:
            result["roofline"]["traffic"] = t.get("bytes_per_launch")
    result["per_shape_sparse"] = per_shape

    # ---- dense fp16 baseline on the same shapes ------------------------------
    if not args.no_dense:
        try:
            torch.backends.cuda.preferred_blas_library("cublaslt")  # hipBLASLt on ROCm
        except Exception as exc:  # pragma: no cover - informational
            log(f"could not select hipBLASLt: {exc}")
        blas = str(torch.backends.cuda.preferred_blas_library())
        per_dense = {}
        dense_step_us = 0.0
        for cls, names in classes.items():
            K, h = SHAPES[names[0]]
            us = MB.time_dense(h, K, torch.float16, rotate_bytes=1 << 30, reps=reps)
            b = dense_bytes(K, h)
            per_dense[cls] = {"us_per_launch": round(us, 3), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                              "pct_peak": round(100 * b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
                              "speedup_sparse_vs_dense": round(us / per_shape[cls]["us_per_launch"], 3)}
            dense_step_us += us * L * len(names)
            log(f"dense  {cls:8s}: {us:7.2f} us/launch {per_dense[cls]['GBps']:7.1f} GB/s "
                f"-> sparse speedup {per_dense[cls]['speedup_sparse_vs_dense']}x")
            torch.cuda.empty_cache()
        sparse_step_us = sum(per_shape[c]["us_per_launch"] * per_shape[c]["launches_per_step"] for c in per_shape)
        result["dense_fp16_baseline"] = {
            "blas": blas,
            "per_shape": per_dense,
            "step_us_sum_of_launches": round(dense_step_us, 1),
            "sparse_step_us_sum_of_launches": round(sparse_step_us, 1),
            "speedup_sparse_vs_dense": round(dense_step_us / sparse_step_us, 3),
        }

    # ---- CPU baseline (rank 0, N=1): oracle gather form on one layer ----------
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(layers[0], xs, nnz, m, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def cpu_baseline(layer, xs, nnz, m, budget_s):
    """Time the oracle's CPU GEMV on one decoder layer's 7 GEMVs (the same
    weights as GPU layer 0, copied to host), all host threads, for about
    `budget_s` seconds; report GB/s of algorithmic bytes."""
    import torch

    from oracle import nm_oracle as O

    host = {name: (md.cpu(), mi.cpu()) for name, (md, mi) in layer.items()}
    xh = {K: x.cpu() for K, x in xs.items()}
    layer_bytes = sum(sparse_bytes(K, h, nnz, m) for K, h in SHAPES.values())
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)

    def one_layer():
        for name, (K, h) in SHAPES.items():
            md, mi = host[name]
            O.gemv_gather_torch(xh[K], md, mi, nnz, m)

    one_layer()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    gbs = layer_bytes / med / 1e9
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    log(f"cpu baseline: {gbs:.2f} GB/s ({med * 1e3:.1f} ms per layer, {threads} threads, {cpu_model})")
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle gather-form GEMV (fp16 weights -> fp32 torch.mv on gathered activations) over one "
                  f"Llama-3.1-8B layer's 7 GEMVs at {nnz}:{m} ({layer_bytes / 1e6:.1f} MB), median of "
                  f"{len(times)} passes in ~{budget_s:.0f} s; CPU: {cpu_model}",
        "ms_per_layer": round(med * 1e3, 2),
    }


if __name__ == "__main__":
    main()
