"""End-to-end decode benchmark: random-init decoder, dense fp16 vs N:M sparse.

    python -m spmv_decode_amd.decode.bench_decode --model llama-3.1-8b --m 64 \\
        [--prompt 128] [--gen 256] [--no-dense] [--json out.json]

Protocol (the Llama-3.1-8B / Qwen3 decode workloads): random-init weights of the named architecture
in fp16 on one GPU; the prompt (seeded random token ids) is fed one token per
graph replay (untimed), then `--gen` greedy decode steps are replayed from one
captured hipGraph and timed with HIP events. Dense first (nn.Linear ->
hipBLASLt, q/k/v as one GEMM like the reference's model.py:198 `wqkv`;
`--dense-fusion` changes that, `--dense-variants` times all three; each
dense weight shape issued in whichever of hipBLASLt's two problem forms,
x * W^T or W * x, runs faster on this GPU, `--no-tune` to keep x * W^T),
then every q/k/v/o/gate/up/down Linear is swapped to NmSparseLinear at
N:M = (M/2):M with on-device synthetic patterns, and the same protocol runs
again. Embeddings, norms and lm_head stay dense in both.
The sparse model runs the fused layer (norms, RoPE, cache write and residuals
inside the GEMV launches); `--per-linear` also times it with one launch per
Linear and PyTorch norms/RoPE (the step structure of the unfused dense
model), `--grouped` with one q/k/v and one gate/up launch and PyTorch
norms/RoPE (the structure of the fused dense modes), `--modules` as unmodified
model code calls it (each projection a module call; swap_to_nmsparse's ties
give q/k/v and gate/up one launch each). `--fixed-ctx 512` times
the reference benchmark's protocol instead (caches of random values, one
step at a fixed position replayed, the next token sampled as the reference
does; runner.fixed_context_ms) with its `RESULT CTX=...` line; `--compile` runs every variant's step through
torch.compile first, as the reference benchmark does.
Prints a `RESULT` line per model variant (like the reference benchmarks,
benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:186-189) and one JSON line.
"""
from __future__ import annotations

import argparse
import gc
import json
import sys
import time

import torch

from ..nmsparse_linear import swap_to_nmsparse
from .model import CONFIGS, Decoder, init_weights_
from .runner import GraphDecoder, fixed_context_ms


def linear_bytes(cfg, m: int) -> int:
    """Algorithmic bytes of one token's Linear weights (dense when m == 0)."""
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    shapes = [(cfg.dim, qd), (cfg.dim, kvd), (cfg.dim, kvd), (qd, cfg.dim), (cfg.dim, cfg.inter),
              (cfg.dim, cfg.inter), (cfg.inter, cfg.dim)]
    total = 0
    for K, h in shapes:
        if m:
            w = K // 2
            total += 2 * w * h + w + 2 * K + 2 * h
        else:
            total += 2 * K * h + 2 * K + 2 * h
    return total * cfg.n_layers


def prefill_ms(model, prompt, reps=10):
    """The prompt's GPU time in one Decoder.prefill pass (every Linear over all
    its rows: hipBLASLt on the dense weights for the dense model; for the
    sparse one the matrix-core SpMM, q/k/v and gate/up grouped, down_proj's
    SiLU product formed in its gather), captured as a hipGraph after an eager
    warm-up; median of reps replays, in ms."""
    from .runner import cache_length

    model.setup_cache(cache_length(prompt.numel() + 1), torch.device("cuda"), dtype=torch.float16)
    ids = prompt.cuda()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        model.prefill(ids)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        model.prefill(ids)
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    del g
    return round(sorted(times)[len(times) // 2], 4)


def run_variant(model, cfg, prompt, gen, label, log, batched_prompt=False):
    """Capture the decode step, feed the prompt (untimed; one graph replay per
    token, or with batched_prompt one Decoder.prefill pass), then time `gen`
    greedy steps by graph replay."""
    dec = GraphDecoder(model, prompt.numel() + gen)
    t0 = time.time()
    dec.capture()
    log(f"{label}: captured decode step in {time.time() - t0:.1f} s")
    dec.run_prompt(prompt, batched=batched_prompt)
    ids, ms_mean, ms_median = dec.generate(gen)
    ok = bool(torch.isfinite(dec.logits).all().item())
    del dec
    return {"ms_per_token": round(ms_mean, 4), "ms_per_token_median_of_16": round(ms_median, 4),
            "tokens_per_s": round(1e3 / ms_mean, 2), "finite_logits": ok,
            "first_tokens": ids[:8].tolist()}


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--model", default="llama-3.1-8b", choices=sorted(CONFIGS))
    p.add_argument("--m", type=int, default=64, help="group size M (N = M/2 kept); 0 = dense only")
    p.add_argument("--prompt", type=int, default=128)
    p.add_argument("--gen", type=int, default=256)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-dense", action="store_true")
    p.add_argument("--dense-fusion", default="qkv", choices=Decoder.DENSE_FUSIONS,
                   help="dense baseline's launches: q/k/v fused (the reference's model), none, or q/k/v and gate/up")
    p.add_argument("--dense-variants", action="store_true",
                   help="also time the dense model under the other two fusion modes")
    p.add_argument("--no-tune", action="store_true",
                   help="issue dense products as nn.Linear does (x * W^T) instead of the faster of the two "
                        "hipBLASLt problem forms per shape (Decoder.tune_dense_gemv)")
    p.add_argument("--per-linear", action="store_true",
                   help="also time the sparse model with one launch per Linear and PyTorch norms/RoPE (the "
                        "step structure of the unfused dense model, so that ratio isolates the GEMVs)")
    p.add_argument("--grouped", action="store_true",
                   help="also time the sparse model with one q/k/v and one gate/up launch and PyTorch norms/RoPE "
                        "(the step structure of the fused dense modes)")
    p.add_argument("--modules", action="store_true",
                   help="also time the sparse model as unmodified model code runs it: every projection called as a "
                        "module, q/k/v and gate/up sharing a launch through swap_to_nmsparse's ties")
    p.add_argument("--fixed-ctx", type=int, default=0, metavar="CTX",
                   help="time the reference benchmark's protocol instead: one decode step at position CTX over "
                        "random-filled caches, replayed (runner.fixed_context_ms)")
    p.add_argument("--compile", action="store_true",
                   help="torch.compile the decode step of every variant before capturing it, as the reference "
                        "benchmark does (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:152); the sparse launches "
                        "stay library calls the compiled code calls out to")
    p.add_argument("--fc-warmup", type=int, default=30)
    p.add_argument("--fc-repeat", type=int, default=30)
    p.add_argument("--fc-inner", type=int, default=10)
    p.add_argument("--prefill-only", action="store_true",
                   help="time only the --prompt tokens through Decoder.prefill in one pass (one hipGraph), dense "
                        "and sparse, instead of decoding")
    p.add_argument("--json", default=None)
    a = p.parse_args(argv)

    def log(msg):
        print(f"[decode] {msg}", file=sys.stderr, flush=True)

    cfg = CONFIGS[a.model]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    try:
        torch.backends.cuda.preferred_blas_library("cublaslt")  # hipBLASLt on ROCm
    except Exception:
        pass
    torch.manual_seed(a.seed)
    t0 = time.time()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(dev):
            model = Decoder(cfg)
    finally:
        torch.set_default_dtype(prev)
    init_weights_(model, seed=a.seed)
    model.eval()
    log(f"{cfg.name}: {sum(p.numel() for p in model.parameters()) / 1e9:.2f} B params built in {time.time() - t0:.1f} s")
    prompt = torch.randint(0, cfg.vocab, (a.prompt,), generator=torch.Generator().manual_seed(a.seed + 1))
    res = {"model": cfg.name, "prompt": a.prompt, "gen": a.gen, "dtype": "fp16", "batch": 1,
           "gpu": torch.cuda.get_device_name(dev)}
    if a.fixed_ctx:
        res.update(protocol="fixed_context", ctx=a.fixed_ctx, warmup=a.fc_warmup, repeat=a.fc_repeat,
                   inner=a.fc_inner)
        del res["prompt"], res["gen"]

    if a.prefill_only:
        res.update(protocol="prefill_one_pass")
        del res["gen"]
        if not a.no_dense:
            res["dense_prefill_ms"] = prefill_ms(model, prompt)
            print(f"RESULT model={cfg.name} dense_float16 prompt={a.prompt} prefill_ms={res['dense_prefill_ms']}",
                  flush=True)
        if a.m:
            swap_to_nmsparse(model, a.m, "cuda", seed=a.seed, init="device", keep_dense=False)
            gc.collect()
            torch.cuda.empty_cache()
            res["sparse_prefill_ms"] = prefill_ms(model, prompt)
            res["ratio"] = f"{a.m // 2}:{a.m}"
            print(f"RESULT model={cfg.name} M={a.m}({a.m // 2}:{a.m}) prompt={a.prompt} "
                  f"prefill_ms={res['sparse_prefill_ms']}", flush=True)
        if "dense_prefill_ms" in res and "sparse_prefill_ms" in res:
            res["speedup_sparse_vs_dense"] = round(res["dense_prefill_ms"] / res["sparse_prefill_ms"], 4)
        if a.json:
            with open(a.json, "w") as f:
                json.dump(res, f, indent=1)
        return 0

    eager_step = model.forward_step
    if a.compile:
        res["compiled"] = True

    def measure(label, tag):
        """Time the model as it stands under the selected protocol; print the RESULT line."""
        if a.compile:  # a fresh compilation for each launch configuration
            torch._dynamo.reset()
            model.forward_step = torch.compile(eager_step, dynamic=False)
            tag += " compiled"
        if not a.fixed_ctx:
            v = run_variant(model, cfg, prompt, a.gen, label, log)
            print(f"RESULT model={cfg.name} {tag} prompt={a.prompt} gen={a.gen} "
                  f"decode_ms_per_token={v['ms_per_token']:.6f} median={v['ms_per_token_median_of_16']:.6f}",
                  flush=True)
            return v
        r = fixed_context_ms(model, a.fixed_ctx, a.fc_warmup, a.fc_repeat, a.fc_inner)
        log(f"{label}: fixed context {a.fixed_ctx}, median {r['median']:.4f} ms")
        print(f"RESULT CTX={a.fixed_ctx} {tag} dtype=float16 measurement=fixed_context_hip_graph "
              f"warmup={a.fc_warmup} repeat={a.fc_repeat} decode_ms_per_token={r['median']:.6f} "
              f"mean={r['mean']:.6f} stdev={r['stdev']:.6f}", flush=True)
        return {"ms_per_token": round(r["median"], 4), "ms_per_token_mean": round(r["mean"], 4),
                "stdev": round(r["stdev"], 4), "tokens_per_s": round(1e3 / r["median"], 2),
                "finite_logits": r["finite_logits"]}

    if not a.no_dense:
        modes = [a.dense_fusion] + ([m for m in Decoder.DENSE_FUSIONS if m != a.dense_fusion]
                                    if a.dense_variants else [])
        for mode in modes:
            model.set_dense_fusion(mode)
            if not a.no_tune:
                for shape, r in model.tune_dense_gemv().items():
                    log(f"dense GEMV {shape}: x*W^T {r['mm']} us, W*x {r['mv']} us -> {r['form']}")
                    res.setdefault("dense_gemv_forms", {})[shape] = r
            d = measure(f"dense ({mode} fused)", f"dense_float16 fusion={mode}")
            d["linear_bytes_per_token"] = linear_bytes(cfg, 0)
            d["fusion"] = mode
            if mode == a.dense_fusion:
                res["dense"] = d
            else:
                res.setdefault("dense_variants", {})[mode] = d
        model.set_dense_fusion("none")
    if a.m:
        t0 = time.time()
        n = swap_to_nmsparse(model, a.m, "cuda", seed=a.seed, init="device", keep_dense=False)
        gc.collect()
        torch.cuda.empty_cache()
        log(f"swapped {n} Linears to {a.m // 2}:{a.m} in {time.time() - t0:.1f} s")
        if not a.no_tune:  # lm_head stays dense in the sparse model (already tuned if dense ran)
            for shape, r in model.tune_dense_gemv().items():
                log(f"dense GEMV {shape}: x*W^T {r['mm']} us, W*x {r['mv']} us -> {r['form']}")
                res.setdefault("dense_gemv_forms", {})[shape] = r
        tag = f"M={a.m}({a.m // 2}:{a.m})"
        s = measure("sparse", tag)
        s["linear_bytes_per_token"] = linear_bytes(cfg, a.m)
        s["ratio"] = f"{a.m // 2}:{a.m}"
        res["sparse"] = s
        if "dense" in res:
            res["speedup_sparse_vs_dense"] = round(res["dense"]["ms_per_token"] / s["ms_per_token"], 4)
            for mode, d in res.get("dense_variants", {}).items():
                res[f"speedup_sparse_vs_dense_{mode}"] = round(d["ms_per_token"] / s["ms_per_token"], 4)
        if a.per_linear:
            model.set_launch_mode("per_linear")
            u = measure("sparse per-Linear", f"{tag} per_linear")
            model.set_launch_mode("fused")
            res["sparse_per_linear"] = u
            if "dense" in res:
                res["speedup_sparse_per_linear_vs_dense"] = round(res["dense"]["ms_per_token"] / u["ms_per_token"], 4)
        if a.grouped:
            model.set_launch_mode("grouped")
            u = measure("sparse grouped", f"{tag} grouped")
            model.set_launch_mode("fused")
            res["sparse_grouped"] = u
            if "dense" in res:
                res["speedup_sparse_grouped_vs_dense"] = round(res["dense"]["ms_per_token"] / u["ms_per_token"], 4)
        if a.modules:
            model.set_launch_mode("modules")
            u = measure("sparse modules", f"{tag} modules")
            model.set_launch_mode("fused")
            res["sparse_modules"] = u
            if "dense" in res:
                res["speedup_sparse_modules_vs_dense"] = round(res["dense"]["ms_per_token"] / u["ms_per_token"], 4)
    structure = {}  # each sparse launch structure over the dense model with the same launches per layer
    dv = {res["dense"]["fusion"]: res["dense"]} if res.get("dense") else {}
    dv.update({k: v for k, v in res.get("dense_variants", {}).items()})
    for key, dense_mode, label in (("sparse", "qkv", "fused_vs_dense_qkv_fused"),
                                   ("sparse_per_linear", "none", "per_linear_vs_dense_per_linear"),
                                   ("sparse_modules", "none", "modules_vs_dense_per_linear"),
                                   ("sparse_grouped", "qkv_gate_up", "grouped_vs_dense_qkv_gate_up_fused")):
        if res.get(key) and dense_mode in dv:
            structure[label] = round(dv[dense_mode]["ms_per_token"] / res[key]["ms_per_token"], 4)
    if structure:
        res["speedup_structure_matched"] = structure
    print(json.dumps(res), flush=True)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
