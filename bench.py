"""Benchmark: N:M sparse GEMV HBM throughput at Llama-3.1-8B decode shapes.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--ratio 32:64]

One step = every sparse GEMV of one Llama-3.1-8B decode token at 32:64, as the
decoder launches them: per layer one q/k/v launch with the input RMSNorm,
RoPE and KV-cache write fused in, o, one gate/up pair launch with the
post-attention RMSNorm, and down (4 launches x 32 layers), with the
accumulated carry of the decoder's default fused path: o, the gate/up pair
and down add their split-K sums into fp32 rows with atomics (as the reference
kernel accumulates), and the next launch finishes the epilogue as it gathers
its input: gate/up the residual add and RMSNorm, down the SiLU*mul, the next
layer's q/k/v the residual add and RMSNorm; the last down adds its residual
itself. Over 32 layers' distinct packed weights (7.0 GB resident in HBM, far
beyond the 256 MB Infinity Cache), fp16, batch 1, captured once in a hipGraph
and replayed. `value` is the algorithmic bytes of the step (2*w*h weights +
w index bytes per matrix, 2*K activations once per launch, norm weights,
residual reads, 2*h outputs per output vector, the RoPE table row; the fp32
rows passed between launches are not counted) divided by the step time. The
same layer with the bit-reproducible split carry (config.split_carry_step),
without a carry (o and down with the residual add,
config.fused_step_without_carry), without any fusion (config.plain_fused_step)
and the GEMVs as 224 separate launches (config.unfused_224_launches) are
timed too.

Also reported: per-shape average launch time and GB/s for the sparse kernel
and for dense fp16 hipBLASLt GEMVs on the same shapes (the faster of its
x * W^T and W * x problem forms per shape), the
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


def carried_gemv_chain(layers, cfg, nnz, m, dev, gen, S=512, carry="split"):
    """One decode token's sparse GEMV launches as the decoder's fused path
    issues them, over `layers` (one dict per layer: Linear name -> (mat_data,
    mat_index)) at the shapes of `cfg` (a DecoderConfig): per layer q/k/v with
    the input RMSNorm (and Qwen3's q/k head norms), RoPE and the KV-cache write,
    o leaving its split partials, the gate/up pair finishing them with the
    residual (+ RMSNorm, SiLU*mul), down leaving its partials for the next
    layer's q/k/v (the last down adds its residual itself). Synthetic
    activations, norm weights, caches of S positions and RoPE table; the
    position is S // 2. carry="accumulate": the accumulated carry of
    Decoder.carry_mode "accumulate" (o, the gate/up pair and down add into
    fp32 rows with atomics; the pair's SiLU product is formed where down
    gathers it). Returns (step function, algorithmic bytes per step, tensors
    the step writes); the bytes are the same for both carries (the
    intermediate fp32 rows, like split partials, are not counted)."""
    import torch

    from spmv_decode_amd import hip_spmv
    from spmv_decode_amd.decode.model import KEY_PAD
    from spmv_decode_amd.hip_spmv import GemvProblem
    from spmv_decode_amd.microbench import CARRIED_CLASSES, decode_form_bytes

    L = len(layers)
    dim, inter, hd = cfg.dim, cfg.inter, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    eps = cfg.norm_eps
    f16 = dict(dtype=torch.float16, device=dev)
    x_res = torch.randn(1, dim, generator=gen, device=dev).to(torch.float16)
    attn = torch.randn(1, qd, generator=gen, device=dev).to(torch.float16)
    qo = torch.zeros(cfg.n_heads, hd + KEY_PAD, **f16)  # the decoder's query rows
    ln1, ln2 = ((torch.rand(dim, generator=gen, device=dev) + 0.5).to(torch.float16) for _ in range(2))
    qn, kn = ((torch.rand(hd, generator=gen, device=dev) + 0.5).to(torch.float16) if cfg.qk_norm else None
              for _ in range(2))
    kcs = [torch.zeros(cfg.n_kv_heads, hd + KEY_PAD, S, **f16) for _ in range(L)]
    vcs = [torch.zeros(cfg.n_kv_heads, hd, S, **f16) for _ in range(L)]
    ang = torch.outer(torch.arange(S, dtype=torch.float64),
                      1.0 / (cfg.rope_theta ** (torch.arange(hd // 2, dtype=torch.float64) * 2.0 / hd)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)
    pos = torch.tensor([S // 2], device=dev)
    act = torch.empty(1, inter, **f16)
    h2, xa, hb = (torch.empty(1, dim, **f16) for _ in range(3))
    co = torch.zeros(hip_spmv.carry_splits(*layers[0]["o_proj"], nnz, m), dim, device=dev)
    cd = torch.zeros(hip_spmv.carry_splits(*layers[0]["down_proj"], nnz, m), dim, device=dev)
    acc_op = torch.zeros(dim + 2 * inter + 16, device=dev)  # o's and the pair's rows, cleared together by q/k/v
    acc_o, acc_p = acc_op[:dim].view(1, dim), acc_op[dim:]
    acc_d = torch.zeros(1, dim, device=dev)
    ssq_n = hip_spmv.gate_up_ssq_slots(layers[0]["gate_proj"], layers[0]["up_proj"], nnz, m, carried=True)

    def layer_accumulated(li):
        lay = layers[li]
        qkv = dict(q_out=qo, k_cache_t=kcs[li], v_cache_t=vcs[li], pos=pos, rope_table=rope, head_dim=hd,
                   norm=(ln1, eps), q_norm=qn, k_norm=kn, head_eps=eps, zero=acc_op)
        if li == 0:
            hip_spmv.nmsparse_qkv_decode(x_res, lay["q_proj"], lay["k_proj"], lay["v_proj"], nnz, m, **qkv)
        else:
            hip_spmv.nmsparse_qkv_decode(hb, lay["q_proj"], lay["k_proj"], lay["v_proj"], nnz, m, carry_in=acc_d,
                                         vec_out=xa, **qkv)
        hip_spmv.nmsparse_gemv_accumulate(attn, *lay["o_proj"], nnz, m, acc_o)
        hip_spmv.nmsparse_gate_up_accumulate(x_res if li == 0 else xa, lay["gate_proj"], lay["up_proj"], nnz, m,
                                             acc_p, norm=(ln2, eps), carry_in=acc_o, vec_out=hb, zero=acc_d)
        if li + 1 < L:
            hip_spmv.nmsparse_gemv_accumulate(None, *lay["down_proj"], nnz, m, acc_d, silu_in=acc_p,
                                              silu_ssq_n=ssq_n, silu_k=dim, silu_eps=eps)
        else:
            hip_spmv.nmsparse_gemv_silu(acc_p, *lay["down_proj"], nnz, m, ssq_n=ssq_n, silu_k=dim, silu_eps=eps,
                                        out=h2, residual=hb)

    def layer(li):
        lay = layers[li]
        qkv = dict(q_out=qo, k_cache_t=kcs[li], v_cache_t=vcs[li], pos=pos, rope_table=rope, head_dim=hd,
                   norm=(ln1, eps), q_norm=qn, k_norm=kn, head_eps=eps)
        if li == 0:
            hip_spmv.nmsparse_qkv_decode(x_res, lay["q_proj"], lay["k_proj"], lay["v_proj"], nnz, m, **qkv)
        else:
            hip_spmv.nmsparse_qkv_decode(hb, lay["q_proj"], lay["k_proj"], lay["v_proj"], nnz, m, carry_in=cd,
                                         vec_out=xa, **qkv)
        hip_spmv.nmsparse_gemv_partials(attn, *lay["o_proj"], nnz, m, co)
        hip_spmv.nmsparse_gate_up_silu(x_res if li == 0 else xa, lay["gate_proj"], lay["up_proj"], nnz, m, out=act,
                                       norm=(ln2, eps), carry_in=co, vec_out=hb)
        if li + 1 < L:
            hip_spmv.nmsparse_gemv_partials(act, *lay["down_proj"], nnz, m, cd)
        else:
            hip_spmv.nmsparse_gemv_launch(act, [GemvProblem(*lay["down_proj"], h2, residual=hb)], nnz, m)

    if carry not in ("split", "accumulate"):
        raise ValueError(f"carry must be 'split' or 'accumulate', got {carry!r}")
    one = layer if carry == "split" else layer_accumulated

    def step():
        for li in range(L):
            one(li)

    dims = dict(dim=dim, inter=inter, qd=qd, kvd=kvd, hd=hd, qk_norm=cfg.qk_norm)
    nbytes = (L * sum(decode_form_bytes(c, nnz, m, **dims) for c in CARRIED_CLASSES)
              - decode_form_bytes("qkv_decode_carried", nnz, m, **dims) + decode_form_bytes("qkv_decode", nnz, m, **dims)
              - decode_form_bytes("down_partials", nnz, m, **dims) + decode_form_bytes("down_resid", nnz, m, **dims))
    written = [qo, xa, hb, h2, kcs[-1][:, :, S // 2], vcs[-1][:, :, S // 2]] + ([act] if carry == "split" else [])
    return step, nbytes, written


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
    p.add_argument("--cpu-detail", action="store_true",
                   help="also time CPU-A (dense scatter + fp32 mv) and CPU-B (gather form) per shape, config 1 "
                        "and every Llama-3.1-8B shape, all host threads and one (minutes)")
    p.add_argument("--cpu-decode", action="store_true",
                   help="also time a CPU Llama-3.1-8B decode step (the decoder code, every Linear via CPU-B)")
    p.add_argument("--only-step", action="store_true", help="time only the sparse step (for profiling)")
    p.add_argument("--no-decode", action="store_true", help="skip the end-to-end decodes")
    p.add_argument("--no-qwen3", action="store_true", help="skip the Qwen3-14B / Qwen3-32B decodes (configs 4-5)")
    return p.parse_args()


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the GEMV would shard by output rows for q/k/v/gate/up and by input groups for o/down, with one "
              "all-reduce of the fp32 partials per row-parallel Linear)", file=sys.stderr)
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

    act = torch.empty(1, SHAPES["gate_proj"][1], dtype=torch.float16, device=dev)

    def fused_layer(li):
        # the decoder's launch pattern: grouped q/k/v, o, gate/up pair with SiLU*mul, down
        lay = layers[li]
        hip_spmv.nmsparse_gemv_grouped(xs[4096], [lay["q_proj"], lay["k_proj"], lay["v_proj"]], nnz, m,
                                       outs=[outs["q_proj"], outs["k_proj"], outs["v_proj"]])
        gemv("o_proj", li)
        hip_spmv.nmsparse_gate_up_silu(xs[4096], lay["gate_proj"], lay["up_proj"], nnz, m, out=act)
        gemv("down_proj", li)

    from spmv_decode_amd.decode.model import KEY_PAD
    from spmv_decode_amd.hip_spmv import GemvProblem
    from spmv_decode_amd.microbench import ACCUMULATED_CLASSES, CARRIED_CLASSES, DECODE_CLASSES, decode_form_bytes

    # decode-form buffers: residual stream, attention output, norms, KV cache, RoPE table, position
    S = 512
    x_res = torch.randn(1, 4096, generator=gen, device=dev).to(torch.float16)
    attn = torch.randn(1, 4096, generator=gen, device=dev).to(torch.float16)
    h1, h2 = (torch.empty(1, 4096, dtype=torch.float16, device=dev) for _ in range(2))
    qo = torch.zeros(32, 128 + KEY_PAD, dtype=torch.float16, device=dev)  # the decoder's query rows
    ln1, ln2 = ((torch.rand(4096, generator=gen, device=dev) + 0.5).to(torch.float16) for _ in range(2))
    kcs = [torch.zeros(8, 128 + KEY_PAD, S, dtype=torch.float16, device=dev) for _ in range(L)]
    vcs = [torch.zeros(8, 128, S, dtype=torch.float16, device=dev) for _ in range(L)]
    ang = torch.outer(torch.arange(S, dtype=torch.float64),
                      1.0 / (500000.0 ** (torch.arange(64, dtype=torch.float64) * 2.0 / 128)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)
    pos = torch.tensor([S // 2], device=dev)

    def decode_layer(li):
        # the decoder's fused layer: q/k/v (+norm, RoPE, cache write), o (+residual),
        # gate/up (+norm, SiLU*mul), down (+residual)
        lay = layers[li]
        hip_spmv.nmsparse_qkv_decode(x_res, lay["q_proj"], lay["k_proj"], lay["v_proj"], nnz, m, q_out=qo,
                                     k_cache_t=kcs[li], v_cache_t=vcs[li], pos=pos, rope_table=rope, head_dim=128,
                                     norm=(ln1, 1e-5))
        hip_spmv.nmsparse_gemv_launch(attn, [GemvProblem(*lay["o_proj"], h1, residual=x_res)], nnz, m)
        hip_spmv.nmsparse_gate_up_silu(h1, lay["gate_proj"], lay["up_proj"], nnz, m, out=act, norm=(ln2, 1e-5))
        hip_spmv.nmsparse_gemv_launch(act, [GemvProblem(*lay["down_proj"], h2, residual=h1)], nnz, m)

    decode_bytes = L * sum(decode_form_bytes(c, nnz, m) for c in DECODE_CLASSES)

    # the decoder's fused path: the split-K carry between the launches
    from spmv_decode_amd.decode.model import LLAMA31_8B

    # the decoder's default fused path: the accumulated carry; the bit-reproducible split carry beside it
    step_fn, step_bytes_carried, step_written = carried_gemv_chain(layers, LLAMA31_8B, nnz, m, dev, gen, S=S,
                                                                   carry="accumulate")
    split_step, split_bytes, split_written = carried_gemv_chain(layers, LLAMA31_8B, nnz, m, dev, gen, S=S)

    w4, w14 = 4096 // m * nnz, 14336 // m * nnz
    fused_bytes_layer = (
        sum(2 * w4 * SHAPES[n][1] + w4 + 2 * SHAPES[n][1] for n in ("q_proj", "k_proj", "v_proj")) + 2 * 4096
        + sparse_bytes(*SHAPES["o_proj"], nnz, m)
        + 2 * (2 * w4 * 14336 + w4) + 2 * 4096 + 2 * 14336
        + sparse_bytes(*SHAPES["down_proj"], nnz, m))
    fused_bytes = L * fused_bytes_layer

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

    def time_step(fn):
        g = capture(fn)
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    # ---- the timed step: one decode token's sparse GEMVs as the decoder runs them
    ms_per_step = time_step(step_fn)
    value = step_bytes_carried / (ms_per_step * 1e-3) / 1e9
    log(f"decode step, accumulated carry ({4 * L} launches) {ms_per_step:.4f} ms -> {value:.1f} GB/s "
        f"({100 * value / HBM_PEAK_GBS:.1f}% of {HBM_PEAK_GBS:.0f})")
    if not all(bool(torch.isfinite(o.float()).all()) for o in step_written):
        raise RuntimeError("non-finite GEMV output")
    ms_split = time_step(split_step)
    split_value = split_bytes / (ms_split * 1e-3) / 1e9
    log(f"decode step, split carry ({4 * L} launches) {ms_split:.4f} ms -> {split_value:.1f} GB/s")
    if not all(bool(torch.isfinite(o.float()).all()) for o in split_written):
        raise RuntimeError("non-finite GEMV output (split carry)")
    ms_nocarry = time_step(lambda: [decode_layer(li) for li in range(L)])
    nocarry_value = decode_bytes / (ms_nocarry * 1e-3) / 1e9
    log(f"decode step without the carry ({4 * L} launches) {ms_nocarry:.4f} ms -> {nocarry_value:.1f} GB/s")
    ms_plain = time_step(lambda: [fused_layer(li) for li in range(L)])
    plain_value = fused_bytes / (ms_plain * 1e-3) / 1e9
    log(f"plain fused step ({4 * L} launches, no norm/RoPE/residual fusions) {ms_plain:.4f} ms -> "
        f"{plain_value:.1f} GB/s")
    ms_unfused = time_step(lambda: [gemv(name, li) for li in range(L) for name in SHAPES])
    unfused_value = step_bytes / (ms_unfused * 1e-3) / 1e9
    log(f"unfused step ({len(SHAPES) * L} launches) {ms_unfused:.4f} ms -> {unfused_value:.1f} GB/s")

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
            "workload": f"Llama-3.1-8B decode-token sparse GEMVs at {nnz}:{m}: {L} layers x (q/k/v + input "
                        "RMSNorm + RoPE + KV-cache write, o, gate/up pair + RMSNorm + SiLU*mul, down), the decoder's "
                        "default fused path: o, the gate/up pair and down accumulate their split-K sums into fp32 "
                        "rows with atomics (the reference kernel's accumulation) and the next launch finishes the "
                        "epilogue (residual add, RMSNorm, SiLU*mul), batch 1, fp16, hipGraph replay, distinct "
                        "resident weights per layer",
            "ratio": f"{nnz}:{m}",
            "layers": L,
            "launches_per_step": 4 * L,
            "algorithmic_bytes_per_step": step_bytes_carried,
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "split_carry_step": {"ms_per_step": round(ms_split, 5), "GBps": round(split_value, 2),
                                 "algorithmic_bytes_per_step": split_bytes,
                                 "timed_step_speedup_over_it": round(ms_split / ms_per_step, 4),
                                 "launches": "the same 4 launches per layer with Decoder.carry_mode 'split': o and "
                                             "down leave fp32 split partials that gate/up and the next q/k/v sum in "
                                             "split order (bit-reproducible run to run, unlike the accumulated "
                                             "carry of the timed step, whose atomic adds' order varies)"},
            "fused_step_without_carry": {"ms_per_step": round(ms_nocarry, 5), "GBps": round(nocarry_value, 2),
                                         "algorithmic_bytes_per_step": decode_bytes,
                                         "launches": "q/k/v + norm/RoPE/cache, o + residual, gate/up pair + norm + "
                                                     "SiLU*mul, down + residual: every launch reduces its own "
                                                     "split-K partials"},
            "plain_fused_step": {"ms_per_step": round(ms_plain, 5), "GBps": round(plain_value, 2),
                                 "algorithmic_bytes_per_step": fused_bytes,
                                 "launches": "grouped q/k/v, o, gate/up pair with SiLU*mul, down (no norm, RoPE, "
                                             "cache or residual fusions)"},
            "unfused_224_launches": {"ms_per_step": round(ms_unfused, 5), "GBps": round(unfused_value, 2),
                                     "algorithmic_bytes_per_step": step_bytes},
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
    # the step's launch classes (decode forms, carried as in the step, and without the carry), weights rotated
    # over >= 1 GiB each
    forms = MB.DecodeForms(nnz, m, rotate_bytes=1 << 30)
    per_class = {}
    for c in ACCUMULATED_CLASSES + CARRIED_CLASSES + DECODE_CLASSES:
        us = forms.time(c, reps=reps)
        b = forms.bytes(c)
        per_class[c] = {"launches_per_step": L, "us_per_launch": round(us, 3), "bytes_per_launch": b,
                        "GBps": round(b / (us * 1e-6) / 1e9, 1),
                        "pct_peak": round(100 * b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
                        "rotated_copies": forms.copies[c]}
        log(f"decode class {c:26s}: {us:7.2f} us/launch {per_class[c]['GBps']:7.1f} GB/s "
            f"({per_class[c]['pct_peak']}%)")
    del forms
    torch.cuda.empty_cache()
    fused = {c: per_class[c] for c in ACCUMULATED_CLASSES}
    # dominant kernel: largest share of the step
    dom = max(fused, key=lambda c: fused[c]["us_per_launch"] * fused[c]["launches_per_step"])
    d = fused[dom]
    kernel_name = {
        "gate_up_pair_acc": "nm_gemv_kernel<fp16, pair_th64_u4, NMAT=2, NORM, CARRY=1> (gate/up pair + RMSNorm, input "
                            "finished from o_proj's accumulated row + residual, raw gate/up sums added into an fp32 "
                            "row, K=4096 h=14336)",
        "qkv_decode_acc": "nm_gemv_kernel<fp16, th32_u8, NORM, CARRY=1> (q/k/v + RMSNorm + RoPE + cache write, input "
                          "finished from down_proj's accumulated row + residual, K=4096 h=4096+1024+1024)",
        "down_silu_acc": "nm_gemv_kernel<fp16, th16_u8, SILU> (down on the pair's SiLU product, adding into an fp32 "
                         "row, K=14336 h=4096)",
        "o_acc": "nm_gemv_kernel<fp16, th16_u8> (o, adding into an fp32 row, K=4096 h=4096)",
        "gate_up_pair_norm_carried": "nm_gemv_kernel<fp16, pair_th64_u4, NMAT=2, NORM, CARRY=8> (gate/up pair + "
                                     "RMSNorm + SiLU*mul, input finished from o_proj's split partials + residual, "
                                     "K=4096 h=14336)",
        "qkv_decode_carried": "nm_gemv_kernel<fp16, th32_u8, NORM, CARRY=8> (q/k/v + RMSNorm + RoPE + cache write, "
                              "input finished from down_proj's split partials + residual, K=4096 h=4096+1024+1024)",
        "down_partials": "nm_gemv_kernel<fp16, th16_u8> (down, split partials left, K=14336 h=4096)",
        "o_partials": "nm_gemv_kernel<fp16, th16_u8> (o, split partials left, K=4096 h=4096)"}[dom]
    result["roofline"] = {
        "bound": "hbm",
        "achieved": d["GBps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(d["GBps"] / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": f"{kernel_name}, {nnz}:{m}",
        "bytes_per_launch": d["bytes_per_launch"],
        "us_per_launch": d["us_per_launch"],
    }
    result["per_launch_class"] = fused
    result["per_launch_class_split_carry"] = {c: per_class[c] for c in CARRIED_CLASSES}
    result["per_launch_class_without_carry"] = {c: per_class[c] for c in DECODE_CLASSES}
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.exists():
        t = json.loads(traffic_file.read_text()).get(f"{dom}_{nnz}:{m}")
        if t:
            result["roofline"]["traffic"] = t.get("bytes_per_launch")
    result["per_shape_sparse"] = per_shape

    # ---- batch > 1: the small-batch SpMM (up to 8 rows) and the matrix-core
    #      SpMM (16-128 rows, one launch plus its activation gather), per row vs
    #      the batch-1 GEMV ------------------------------------------------------
    spmm = {}
    for cls in ("q_o", "gate_up", "down"):
        K, h = SHAPES[classes[cls][0]]
        b1 = per_shape[cls]["us_per_launch"]
        rows = {}
        for batch in (2, 4, 8, 16, 32, 64, 128):
            routed = batch > 8 and hip_spmv.library_route(batch, K, h)
            us = MB.time_spmm(h, K, nnz, m, batch, reps=reps)  # the library's automatic choice
            rows[str(batch)] = {"kernel": ("small-batch" if batch <= 8 else
                                           "gather + hipBLASLt" if routed else "matrix-core"),
                                "us_per_launch": round(us, 3), "us_per_row": round(us / batch, 3),
                                "speedup_per_row_vs_batch1": round(b1 * batch / us, 3),
                                "weight_GBps": round(sparse_bytes(K, h, nnz, m) / (us * 1e-6) / 1e9, 1)}
            if batch > 8:  # the matrix-core kernel and the library route (gather + one hipBLASLt GEMM) side by side
                mc_us = MB.time_spmm(h, K, nnz, m, batch, reps=reps, matrix_cores=True) if routed else us
                lib_us = MB.time_gather_gemm(h, K, nnz, m, batch, reps=reps)
                rows[str(batch)]["matrix_core_us"] = round(mc_us, 3)
                rows[str(batch)]["matrix_core_weight_GBps"] = round(sparse_bytes(K, h, nnz, m) / (mc_us * 1e-6) / 1e9,
                                                                    1)
                rows[str(batch)]["gather_plus_hipblaslt_us"] = round(lib_us, 3)
                rows[str(batch)]["speedup_matrix_core_vs_gather_plus_hipblaslt"] = round(lib_us / mc_us, 3)
            log(f"spmm {cls:8s} batch {batch}: {us:7.2f} us/launch, {us / batch:6.2f} us/row "
                f"({rows[str(batch)]['speedup_per_row_vs_batch1']}x per row vs batch 1)")
        spmm[cls] = rows
        torch.cuda.empty_cache()
    result["spmm_batch"] = spmm
    # sibling products of one input in one grouped launch (q/k/v, gate/up) against one call per product
    group = {}
    for name, (hs, K) in {"q_k_v": ((4096, 1024, 1024), 4096), "gate_up": ((14336, 14336), 4096)}.items():
        wbytes = sum(((K // m) * nnz) * h * 2 for h in hs)
        group[name] = {}
        for batch in (16, 32, 64, 128):
            g_us, sep_us = MB.time_spmm_group(hs, K, nnz, m, batch, reps=reps)
            group[name][str(batch)] = {"grouped_us": round(g_us, 3), "separate_us": round(sep_us, 3),
                                       "grouped_weight_GBps": round(wbytes / (g_us * 1e-6) / 1e9, 1),
                                       "speedup_grouped_vs_separate": round(sep_us / g_us, 3)}
            log(f"spmm group {name:6s} batch {batch}: grouped {g_us:7.2f} us ({wbytes / g_us / 1e3:6.0f} GB/s), "
                f"separate {sep_us:7.2f} us")
        torch.cuda.empty_cache()
    result["spmm_group"] = group

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
            us, form = MB.time_dense(h, K, torch.float16, rotate_bytes=1 << 30, reps=reps, return_form=True)
            b = dense_bytes(K, h)
            per_dense[cls] = {"us_per_launch": round(us, 3), "form": form,
                              "GBps": round(b / (us * 1e-6) / 1e9, 1),
                              "pct_peak": round(100 * b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
                              "speedup_sparse_vs_dense": round(us / per_shape[cls]["us_per_launch"], 3)}
            dense_step_us += us * L * len(names)
            log(f"dense  {cls:8s}: {us:7.2f} us/launch ({form}) {per_dense[cls]['GBps']:7.1f} GB/s "
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
        if args.cpu_detail:
            result["cpu_baseline"]["detail"] = cpu_detail(nnz, m)
        if args.cpu_decode:
            result["cpu_baseline"]["decode"] = cpu_decode(nnz, m)

    # ---- end-to-end decode ms/token: dense hipBLASLt vs N:M sparse ------------
    if not args.no_decode:
        layers.clear()  # the closures above share this list: clearing it frees the weights
        torch.cuda.empty_cache()
        result["decode"] = decode_ms_per_token(m, log)
        if not args.no_qwen3:
            result["decode_qwen3"] = decode_qwen3(log)
        # torch.compile's worker pool (started by the compiled fixed-context runs) must not outlive the bench
        from torch._inductor.async_compile import shutdown_compile_workers

        shutdown_compile_workers()
    print(json.dumps(result), flush=True)


def _finite(v, digits=4):
    """v rounded, or None (JSON null) when it is not a finite number."""
    return round(v, digits) if v == v and abs(v) != float("inf") else None


def decode_ms_per_token(m, log):
    """Random-init Llama-3.1-8B, prompt 128 + 256 greedy steps per variant,
    hipGraph replay (spmv_decode_amd.decode.bench_decode protocol), then the
    reference benchmark's fixed-context protocol (CTX 512, with its sampling),
    eager and compiled."""
    import torch

    from spmv_decode_amd.decode.bench_decode import linear_bytes, prefill_ms, run_variant
    from spmv_decode_amd.decode.model import LLAMA31_8B, Decoder, init_weights_
    from spmv_decode_amd.decode.runner import fixed_context_logits_fp32, fixed_context_ms, logits_envelope
    from spmv_decode_amd.nmsparse_linear import swap_to_nmsparse
    from spmv_decode_amd.profiling import REFERENCE_A100_CTX512

    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device("cuda:0"):
            model = Decoder(LLAMA31_8B)
    finally:
        torch.set_default_dtype(prev)
    init_weights_(model, seed=0)
    prompt = torch.randint(0, LLAMA31_8B.vocab, (128,), generator=torch.Generator().manual_seed(1))

    envelope_failures = []

    def compiled_fixed(model, eager_ref, ref32, label):
        """The reference protocol with its torch.compile: compile the step, then capture and replay.
        The compiled step's logits must stay within the fp16 envelope of the eager step's (eager_ref),
        judged against the fp32 reference ref32 of the same step (runner.logits_envelope); a step outside
        it is collected in envelope_failures and fails the bench. A compiler failure is reported in the
        JSON, not raised (the compiled figures are then null)."""
        eager = model.forward_step
        torch._dynamo.reset()
        model.forward_step = torch.compile(eager, dynamic=False)
        try:
            r = fixed_context_ms(model, 512)
            diff = (r["logits"] - eager_ref["logits"]).abs().max().item()
            r["matches_eager"] = {"max_abs_logit_diff": round(diff, 5),
                                  **logits_envelope(eager_ref["logits"], r["logits"], ref32)}
            log(f"{label} compiled vs eager: {r['matches_eager']}")
            if not r["matches_eager"]["within"]:
                envelope_failures.append((label, r["matches_eager"]))
            return r
        except Exception as exc:  # noqa: BLE001 - torch.compile's failures have no common type
            log(f"compiled fixed-context decode failed: {type(exc).__name__}: {exc}")
            return {"median": float("nan"), "error": f"{type(exc).__name__}: {str(exc)[:300]}"}
        finally:
            model.forward_step = eager
            torch._dynamo.reset()

    dense_by_fusion, forms, fixed_dense, fixed_dense_c = {}, {}, {}, {}
    ref32_dense = fixed_context_logits_fp32(model, 512)  # the dense step in fp32: the envelope's reference
    for mode in ("qkv", "none", "qkv_gate_up"):  # "qkv": the reference's dense model (model.py:198 wqkv)
        model.set_dense_fusion(mode)
        forms.update(model.tune_dense_gemv())  # the faster hipBLASLt problem form per dense shape
        dense_by_fusion[mode] = run_variant(model, LLAMA31_8B, prompt, 256, f"dense ({mode} fused)", log)
        fixed_dense[mode] = fixed_context_ms(model, 512)  # the reference benchmark's protocol
        fixed_dense_c[mode] = compiled_fixed(model, fixed_dense[mode], ref32_dense, f"dense ({mode} fused)")
    model.set_dense_fusion("none")
    dense = dense_by_fusion["qkv"]
    prefill_dense = prefill_ms(model, prompt)
    swap_to_nmsparse(model, m, "cuda", seed=0, init="device", keep_dense=False)
    torch.cuda.empty_cache()
    prefill_sparse = prefill_ms(model, prompt)
    log(f"prefill of the {prompt.numel()}-token prompt in one pass: dense {prefill_dense} ms, "
        f"sparse {prefill_sparse} ms ({prefill_dense / prefill_sparse:.3f}x)")
    sparse = run_variant(model, LLAMA31_8B, prompt, 256, "sparse", log)
    fixed_sparse = fixed_context_ms(model, 512)
    ref32_sparse = fixed_context_logits_fp32(model, 512)
    fixed_sparse_c = compiled_fixed(model, fixed_sparse, ref32_sparse, "sparse")
    # the bit-reproducible split carry (Decoder.carry_mode "split") beside the default accumulated carry
    model.carry_mode = "split"
    try:
        sparse_split = run_variant(model, LLAMA31_8B, prompt, 256, "sparse, split carry", log)
        fixed_split = fixed_context_ms(model, 512)
        split_env = logits_envelope(fixed_split["logits"], fixed_sparse["logits"], ref32_sparse)
        log(f"accumulated carry vs split carry, fixed context: {split_env}")
        if not split_env["within"]:
            envelope_failures.append(("sparse accumulated carry vs split carry (eager)", split_env))
        fixed_split_c = compiled_fixed(model, fixed_split, ref32_sparse, "sparse split carry")
    finally:
        model.carry_mode = "accumulate"
    variants = {}
    for mode in ("per_linear", "grouped", "modules"):
        model.set_launch_mode(mode)
        variants[mode] = run_variant(model, LLAMA31_8B, prompt, 256, f"sparse {mode}", log)
    # the unmodified model (every projection a module call) compiled: the compile pass groups its siblings
    model.set_launch_mode("modules")
    fixed_mod = fixed_context_ms(model, 512)
    fixed_mod_c = compiled_fixed(model, fixed_mod, ref32_sparse, "sparse unmodified model (HF names)")
    model.set_launch_mode("fused")
    ref_dense, ref_sparse = REFERENCE_A100_CTX512["llama-3.1-8b"]
    del model
    torch.cuda.empty_cache()
    # the same under gpt-fast's names (the reference benchmark's model: fused wqkv, w1/w3/w2)
    t0 = time.time()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device("cuda:0"):
            gf = Decoder(LLAMA31_8B, layout="gpt-fast")
    finally:
        torch.set_default_dtype(prev)
    init_weights_(gf, seed=0)
    fixed_gf_dense = fixed_context_ms(gf, 512)
    fixed_gf_dense_c = compiled_fixed(gf, fixed_gf_dense, fixed_context_logits_fp32(gf, 512), "dense (gpt-fast names)")
    swap_to_nmsparse(gf, m, "cuda", seed=0, init="device", keep_dense=False)
    torch.cuda.empty_cache()
    fixed_gf = fixed_context_ms(gf, 512)
    fixed_gf_c = compiled_fixed(gf, fixed_gf, fixed_context_logits_fp32(gf, 512), "sparse unmodified model (gpt-fast names)")
    log(f"gpt-fast-named model: dense {fixed_gf_dense['median']:.4f} ms (compiled {fixed_gf_dense_c['median']:.4f}), "
        f"sparse {fixed_gf['median']:.4f} ms (compiled {fixed_gf_c['median']:.4f}) in {time.time() - t0:.0f} s")
    del gf
    torch.cuda.empty_cache()
    ms = {k: v["ms_per_token"] for k, v in dense_by_fusion.items()}
    fastest_dense = min(ms.values())
    fc = {k: v["median"] for k, v in fixed_dense.items()}
    fcc = {k: v["median"] for k, v in fixed_dense_c.items()}
    fcc_ok = [v for v in fcc.values() if v == v]
    fastest_fcc = min(fcc_ok) if fcc_ok else float("nan")

    def ratio(a, b):
        return _finite(a / b)

    out = {"model": "llama-3.1-8b (random init)", "prompt": 128, "gen": 256,
           "prefill_one_pass": {"dense_ms": prefill_dense, "sparse_ms": prefill_sparse,
                                "speedup_sparse_vs_dense": ratio(prefill_dense, prefill_sparse),
                                "what": "the 128-token prompt through Decoder.prefill as one hipGraph: every "
                                        "Linear over 128 rows (dense: hipBLASLt on the dense weights; sparse: the "
                                        "matrix-core SpMM's 128-row tiles, q/k/v and gate/up grouped), causal "
                                        "attention through PyTorch's scaled_dot_product_attention"},
           "dense_ms_per_token": dense["ms_per_token"], "sparse_ms_per_token": sparse["ms_per_token"],
           "dense_launches": "q/k/v fused into one GEMM (the reference's dense model), gate/up/o/down one each; "
                             "each shape in the faster of hipBLASLt's x*W^T and W*x forms",
           "dense_gemv_forms": forms,
           "speedup_sparse_vs_dense": round(dense["ms_per_token"] / sparse["ms_per_token"], 4),
           "dense_ms_per_token_by_fusion": ms,
           "speedup_sparse_vs_fastest_dense": round(fastest_dense / sparse["ms_per_token"], 4),
           "split_carry": {
               "sparse_ms_per_token": sparse_split["ms_per_token"],
               "default_speedup_over_it": round(sparse_split["ms_per_token"] / sparse["ms_per_token"], 4),
               "fixed_context_512_ms_per_token": round(fixed_split["median"], 4),
               "fixed_context_512_compiled_ms_per_token": _finite(fixed_split_c["median"]),
               "accumulated_matches_split": split_env,
               "compiled_matches_eager": fixed_split_c.get("matches_eager"),
               "note": "Decoder.carry_mode 'split': o_proj and down_proj leave fp32 split partials that the next "
                       "launch sums in split order, so logits are bit-reproducible run to run and graph replay to "
                       "eager; the default 'accumulate' (every other sparse figure here) adds into fp32 rows with "
                       "atomics, as the reference kernel accumulates, and its logits vary in the last bits"},
           "sparse_ms_per_token_by_launch_mode": {"fused": sparse["ms_per_token"],
                                                  **{k: v["ms_per_token"] for k, v in variants.items()}},
           "sparse_per_linear_ms_per_token": variants["per_linear"]["ms_per_token"],
           "speedup_sparse_per_linear_vs_dense": round(dense["ms_per_token"] / variants["per_linear"]["ms_per_token"],
                                                       4),
           "speedup_sparse_modules_vs_dense": round(dense["ms_per_token"] / variants["modules"]["ms_per_token"], 4),
           "sparse_modules_note": "the unmodified model after swap_to_nmsparse: every projection called as a module "
                                  "(lin(x)); q/k/v and gate/up share one launch each through the ties swap_to_nmsparse "
                                  "makes; norms, RoPE, SiLU*mul, residuals in PyTorch",
           "speedup_structure_matched": {
               "fused_vs_dense_qkv_fused": round(ms["qkv"] / sparse["ms_per_token"], 4),
               "per_linear_vs_dense_per_linear": round(ms["none"] / variants["per_linear"]["ms_per_token"], 4),
               "modules_vs_dense_per_linear": round(ms["none"] / variants["modules"]["ms_per_token"], 4),
               "grouped_vs_dense_qkv_gate_up_fused": round(ms["qkv_gate_up"] / variants["grouped"]["ms_per_token"],
                                                           4),
               "note": "each sparse launch structure over the dense model with the same launches per layer: per-Linear "
                       "and modules (one q/k/v and one gate/up launch) over one GEMM per Linear, grouped over q/k/v "
                       "and gate/up fused GEMMs; the fused layer (norms, RoPE, cache write, residuals inside the "
                       "launches) over the reference's dense model"},
           "sparse_linear_bytes_per_token": linear_bytes(LLAMA31_8B, m),
           "dense_linear_bytes_per_token": linear_bytes(LLAMA31_8B, 0),
           "fixed_context_512": {
               "protocol": "the reference benchmark's (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:144-189): "
                           "random-filled caches, one step at position 512 with the next token sampled (softmax, one "
                           "categorical draw as generate.py:46-63 makes with multinomial; drawn by the exponential "
                           "race) replayed, median of 30 x 10 replays",
               "dense_ms_per_token": round(fc["qkv"], 4),
               "dense_ms_per_token_by_fusion": {k: round(v, 4) for k, v in fc.items()},
               "sparse_ms_per_token": round(fixed_sparse["median"], 4),
               "speedup_sparse_vs_dense": round(fc["qkv"] / fixed_sparse["median"], 4),
               "compiled": {"dense_ms_per_token": _finite(fcc["qkv"]),
                            "dense_ms_per_token_by_fusion": {k: _finite(v) for k, v in fcc.items()},
                            "sparse_ms_per_token": _finite(fixed_sparse_c["median"]),
                            "speedup_sparse_vs_dense": ratio(fcc["qkv"], fixed_sparse_c["median"]),
                            "speedup_sparse_vs_fastest_dense": ratio(fastest_fcc, fixed_sparse_c["median"]),
                            "matches_eager": {**{f"dense_{k}": v.get("matches_eager")
                                                 for k, v in fixed_dense_c.items()},
                                              "sparse": fixed_sparse_c.get("matches_eager"),
                                              "rule": "each compiled step's logits within 2*e16 + 1e-3 (rel-L2) of "
                                                      "the same step in fp32 and within 3*e16 + 1e-3 of the eager "
                                                      "fp16 step, e16 = the eager fp16 step's rel-L2 from fp32; "
                                                      "the bench fails otherwise"},
                            "errors": [r["error"] for r in (*fixed_dense_c.values(), fixed_sparse_c)
                                       if "error" in r] or None,
                            "note": "torch.compile of each model's step before capture, as the reference "
                                    "benchmark (its published figures below are compiled); the sparse step's "
                                    "launches are torch.ops.nmsparse ops, so it compiles without graph breaks"},
               "reference_a100_published": {"dense_ms_per_token": ref_dense, "sparse_ms_per_token": ref_sparse.get(m),
                                            "speedup": round(ref_dense / ref_sparse[m], 4) if m in ref_sparse else None,
                                            "source": "README.md:86-93"}},
           "compiled_unmodified_model": {
               "protocol": "the fixed-context protocol above, torch.compile (inductor, fullgraph) of the step of the "
                           "model as written for dense Linears, swapped by swap_to_nmsparse: every projection a module "
                           "call; the compile pass (spmv_decode_amd/compile_pass.py) turns each layer's sibling gemv "
                           "calls into one grouped q/k/v launch (HF names) and one gate/up pair launch with SiLU*mul, "
                           "folds the RMSNorm in front of q/k/v and gate/up into those launches and the residual "
                           "adds after o and down into theirs",
               "hf_names": {"sparse_ms_per_token": _finite(fixed_mod_c["median"]),
                            "eager_sparse_ms_per_token": round(fixed_mod["median"], 4),
                            "speedup_vs_fastest_compiled_dense": ratio(fastest_fcc, fixed_mod_c["median"]),
                            "matches_eager": fixed_mod_c.get("matches_eager")},
               "gpt_fast_names": {"dense_ms_per_token": _finite(fixed_gf_dense_c["median"]),
                                  "sparse_ms_per_token": _finite(fixed_gf_c["median"]),
                                  "speedup_vs_its_dense": ratio(fixed_gf_dense_c["median"], fixed_gf_c["median"]),
                                  "speedup_vs_fastest_compiled_dense": ratio(min(fastest_fcc,
                                                                                 fixed_gf_dense_c["median"]),
                                                                             fixed_gf_c["median"]),
                                  "eager_dense_ms_per_token": round(fixed_gf_dense["median"], 4),
                                  "eager_sparse_ms_per_token": round(fixed_gf["median"], 4),
                                  "matches_eager": {"dense": fixed_gf_dense_c.get("matches_eager"),
                                                    "sparse": fixed_gf_c.get("matches_eager")}},
               "errors": [r["error"] for r in (fixed_mod_c, fixed_gf_dense_c, fixed_gf_c) if "error" in r] or None},
           "headline": {"speedup": ratio(fastest_fcc, fixed_sparse_c["median"]),
                        "what": "sparse over the fastest of the three dense launch structures, both compiled, "
                                "under the reference benchmark's fixed-context protocol (CTX 512, sampling)"}}
    if envelope_failures:
        raise RuntimeError(f"compiled fixed-context step outside the fp16 envelope of the eager step: "
                           f"{envelope_failures}")
    log(f"decode: dense {out['dense_ms_per_token']} ms/token, sparse {out['sparse_ms_per_token']} ms/token "
        f"({out['speedup_sparse_vs_dense']}x), unmodified model after the swap "
        f"{variants['modules']['ms_per_token']} ms ({out['speedup_sparse_modules_vs_dense']}x), per-Linear "
        f"{variants['per_linear']['ms_per_token']} ms; fixed context 512: {round(fc['qkv'], 4)} / "
        f"{round(fixed_sparse['median'], 4)} ms (compiled {_finite(fcc['qkv'])} / "
        f"{_finite(fixed_sparse_c['median'])} ms; over the fastest compiled dense {out['headline']['speedup']}x)")
    return out


QWEN3_DECODE = (  # the Qwen3 decode workloads: (model, M, prompt tokens, generated tokens)
    ("qwen3-14b", 64, 128, 256),
    ("qwen3-32b", 32, 512, 512),
)


def decode_qwen3(log, steps=20, warmup=5):
    """Configs 4-5: random-init Qwen3-14B at 32:64 and Qwen3-32B at 16:32, fp16,
    batch 1. Per model: the dense model under each of its three launch
    structures (one GEMM per Linear, q/k/v fused, q/k/v and gate/up fused; every
    dense shape in hipBLASLt's faster problem form) and the fused sparse decoder,
    each the prompt in one Decoder.prefill pass (untimed) then the generated
    tokens by hipGraph replay (ms/token: the mean over them); the speedup over
    the fastest dense structure; and one token's sparse GEMV launches as the
    decoder issues them (4 per layer, the accumulated carry, over the model's
    own resident weights) timed alone by graph replay: ms and algorithmic GB/s."""
    import gc

    import torch

    from spmv_decode_amd.decode.bench_decode import linear_bytes, run_variant
    from spmv_decode_amd.decode.model import CONFIGS, Decoder, init_weights_
    from spmv_decode_amd.nmsparse_linear import swap_to_nmsparse
    from spmv_decode_amd.profiling import REFERENCE_A100_CTX512

    dev = torch.device("cuda:0")
    out = {}
    for name, M, P, G in QWEN3_DECODE:
        cfg = CONFIGS[name]
        nnz = M // 2
        t0 = time.time()
        prev = torch.get_default_dtype()
        torch.set_default_dtype(torch.float16)
        try:
            with torch.device(dev):
                model = Decoder(cfg)
        finally:
            torch.set_default_dtype(prev)
        init_weights_(model, seed=0)
        model.eval()
        prompt = torch.randint(0, cfg.vocab, (P,), generator=torch.Generator().manual_seed(1))
        log(f"{name}: dense model built in {time.time() - t0:.1f} s")
        dense = {}
        for mode in ("qkv", "none", "qkv_gate_up"):
            model.set_dense_fusion(mode)
            model.tune_dense_gemv()
            dense[mode] = run_variant(model, cfg, prompt, G, f"{name} dense ({mode} fused)", log,
                                      batched_prompt=True)
        model.set_dense_fusion("none")
        swap_to_nmsparse(model, M, "cuda", seed=0, init="device", keep_dense=False)
        gc.collect()
        torch.cuda.empty_cache()
        sparse = run_variant(model, cfg, prompt, G, f"{name} sparse {nnz}:{M}", log, batched_prompt=True)
        layers = [{n: (getattr(sub, n).mat_data, getattr(sub, n).mat_index)
                   for sub, names in ((blk.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                                      (blk.mlp, ("gate_proj", "up_proj", "down_proj"))) for n in names}
                  for blk in model.layers]
        step, nbytes, written = carried_gemv_chain(layers, cfg, nnz, M, dev, torch.Generator(device=dev).manual_seed(3),
                                                   carry="accumulate")
        stream = torch.cuda.Stream(device=dev)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            step()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step()
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            g.replay()
        b.record()
        b.synchronize()
        step_ms = a.elapsed_time(b) / steps
        if not all(bool(torch.isfinite(o.float()).all()) for o in written):
            raise RuntimeError(f"{name}: non-finite GEMV output in the step")
        del g, layers, step, written
        ms = {k: v["ms_per_token"] for k, v in dense.items()}
        fastest = min(ms, key=ms.get)
        ref_dense, ref_sparse = REFERENCE_A100_CTX512.get(name, (None, {}))
        out[name] = {
            "ratio": f"{nnz}:{M}", "prompt": P, "gen": G, "layers": cfg.n_layers,
            "dense_ms_per_token_by_fusion": ms, "fastest_dense": fastest,
            "sparse_ms_per_token": sparse["ms_per_token"],
            "speedup_sparse_vs_fastest_dense": round(ms[fastest] / sparse["ms_per_token"], 4),
            "speedup_sparse_vs_dense_qkv_fused": round(ms["qkv"] / sparse["ms_per_token"], 4),
            "finite_logits": sparse["finite_logits"] and all(v["finite_logits"] for v in dense.values()),
            "sparse_linear_bytes_per_token": linear_bytes(cfg, M), "dense_linear_bytes_per_token": linear_bytes(cfg, 0),
            "gemv_step": {"launches": 4 * cfg.n_layers, "ms": round(step_ms, 5), "algorithmic_bytes": nbytes,
                          "GBps": round(nbytes / step_ms / 1e6, 1),
                          "pct_hbm_peak": round(100 * nbytes / step_ms / 1e6 / HBM_PEAK_GBS, 2)},
            "reference_a100_published_fixed_ctx512": {
                "dense_ms_per_token": ref_dense, "sparse_ms_per_token": ref_sparse.get(M),
                "note": "the reference's A100 table (README.md:99-121), fixed-context protocol (CTX 512), not this "
                        "generation protocol"},
        }
        log(f"{name} {nnz}:{M}: dense {ms} ms/token, sparse {sparse['ms_per_token']} ms/token "
            f"({out[name]['speedup_sparse_vs_fastest_dense']}x over the fastest dense); GEMV step "
            f"{out[name]['gemv_step']}")
        del model
        gc.collect()
        torch.cuda.empty_cache()
    return out


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
    # the reference benchmarks' own CPU thread default is 1 (BENCH_CPU_THREADS)
    torch.set_num_threads(1)
    one = []
    for _ in range(3):
        t0 = time.perf_counter()
        one_layer()
        one.append(time.perf_counter() - t0)
    torch.set_num_threads(threads)
    med1 = statistics.median(one)
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
        "one_thread": {"value": round(layer_bytes / med1 / 1e9, 3), "unit": "GB/s", "ms_per_layer": round(med1 * 1e3, 2),
                       "sample": "median of 3 passes over the same layer"},
        "decode_token_gemv_ms": round(LLAMA["n_layers"] * med * 1e3, 1),
        "decode_token_gemv_note": "32 layers x the measured per-layer time: the sparse GEMVs of one Llama-3.1-8B "
                                  "decode token on the host cores (attention, norms and lm_head not included)",
    }


def _median_stdev(fn, reps, warmup=3):
    for _ in range(warmup):
        fn()
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return statistics.median(t), (statistics.stdev(t) if len(t) > 1 else 0.0)


def cpu_detail(nnz, m, reps=20):
    """CPU-A (the oracle: scatter to dense, fp32 torch.mv) and CPU-B (gather
    form) per shape: config 1 (Qwen3-0.6B up-proj, 2:4, the reference's own
    generator) and the Llama-3.1-8B shapes at nnz:m, all host threads and one
    thread; median and stdev of `reps` calls after 3 warm-ups."""
    import torch

    from oracle import nm_oracle as O

    threads = os.cpu_count() or 1
    cases = []
    md1, mi1 = O.make_sparse(1024, 3072, 4, 0)[:2]
    cases.append(("config1_up_proj 1024->3072 2:4", 1024, 3072, 2, 4, md1, mi1))
    g = torch.Generator().manual_seed(7)
    for name, (K, h) in SHAPES.items():
        w = K // m * nnz
        md = (torch.randn(w, h, generator=g) * 0.02).half()
        mi = torch.stack([torch.randperm(m, generator=g)[:nnz].sort().values for _ in range(K // m)]).to(torch.uint8)
        cases.append((f"{name} {K}->{h} {nnz}:{m}", K, h, nnz, m, md, mi))
    rows = []
    for label, K, h, n_, m_, md, mi in cases:
        x = torch.randn(1, K, generator=g).half()
        b = sparse_bytes(K, h, n_, m_)
        row = {"shape": label, "bytes": b}
        for th in (threads, 1):
            torch.set_num_threads(th)
            for form, fn in (("cpu_a", lambda: O.gemv_fp32_dense(x, md, mi, n_, m_)),
                             ("cpu_b", lambda: O.gemv_gather_torch(x, md, mi, n_, m_))):
                med, sd = _median_stdev(fn, reps if th > 1 or b < 60e6 else max(5, reps // 4))
                row[f"{form}_{th}t_ms"] = round(med * 1e3, 3)
                row[f"{form}_{th}t_sd_ms"] = round(sd * 1e3, 3)
                row[f"{form}_{th}t_GBps"] = round(b / med / 1e9, 3)
        torch.set_num_threads(threads)
        log(f"cpu detail {label}: CPU-A {row[f'cpu_a_{threads}t_ms']:.2f} ms / CPU-B {row[f'cpu_b_{threads}t_ms']:.2f} "
            f"ms ({threads} threads); CPU-A {row['cpu_a_1t_ms']:.2f} / CPU-B {row['cpu_b_1t_ms']:.2f} ms (1 thread)")
        rows.append(row)
    return {"threads": threads, "reps": reps, "rows": rows}


def cpu_decode(nnz, m, tokens=4):
    """ms/token of a CPU decode step of the Llama-3.1-8B architecture with the
    decoder's own code (fp32 activations, static cache, per-Linear path) and
    every q/k/v/o/gate/up/down Linear computed in the CPU-B gather form from
    packed fp16 weights (random values; the timing does not depend on them)."""
    import torch
    import torch.nn as nn

    from oracle import nm_oracle as O
    from spmv_decode_amd.decode.model import LLAMA31_8B, Decoder, RMSNorm

    class CpuGatherLinear(nn.Module):
        def __init__(self, md, mi):
            super().__init__()
            self.md, self.mi = md, mi

        def forward(self, x):
            y = O.gemv_gather_torch(x, self.md, self.mi, nnz, m)
            return y.view(*x.shape[:-1], -1).to(x.dtype)

    cfg = LLAMA31_8B
    t0 = time.perf_counter()
    with torch.device("meta"):
        model = Decoder(cfg)
    g = torch.Generator().manual_seed(11)
    for blk in model.layers:
        for sub, names in ((blk.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                           (blk.mlp, ("gate_proj", "up_proj", "down_proj"))):
            for name in names:
                h, K = getattr(sub, name).weight.shape
                w = K // m * nnz
                md = (torch.randn(w, h, generator=g) * 0.02).half()  # fp32 draws: CPU fp16 randn is 5x slower
                mi = torch.rand(K // m, m, generator=g).argsort(dim=1)[:, :nnz].sort(dim=1).values.to(torch.uint8)
                setattr(sub, name, CpuGatherLinear(md, mi))
    for mod in model.modules():
        for pname, par in list(mod._parameters.items()):
            if par is not None and par.is_meta:
                val = torch.ones(par.shape) if isinstance(mod, RMSNorm) else torch.randn(par.shape, generator=g) * 0.02
                mod._parameters[pname] = nn.Parameter(val, requires_grad=False)
    model.eval()
    model.setup_cache(tokens + 2, "cpu", dtype=torch.float32)
    build_s = time.perf_counter() - t0
    token = torch.zeros(1, 1, dtype=torch.long)
    times = []
    with torch.no_grad():
        for i in range(tokens + 1):  # the first step is a warm-up
            t1 = time.perf_counter()
            logits = model.forward_step(token, torch.tensor([i]))
            token = torch.argmax(logits, dim=-1).view(1, 1)
            times.append(time.perf_counter() - t1)
    times = times[1:]
    ms = statistics.median(times) * 1e3
    log(f"cpu decode: {ms:.1f} ms/token over {tokens} tokens ({os.cpu_count()} threads; model built in {build_s:.0f} s)")
    return {"ms_per_token": round(ms, 1), "tokens": tokens, "threads": os.cpu_count(),
            "per_token_ms": [round(t * 1e3, 1) for t in times],
            "sample": "Llama-3.1-8B architecture, fp32 activations, every projection in the CPU-B gather form from "
                      f"packed fp16 {nnz}:{m} weights, dense fp32 embedding / lm_head, {tokens} greedy steps after "
                      "one warm-up step"}


if __name__ == "__main__":
    main()
