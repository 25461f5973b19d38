"""Summarise rocprofv3 CSV output into the markdown/JSON kept under profiles/.

    python -m spmv_decode_amd.profiling traffic --fetch <out>/pmc_fetch/pmc_counter_collection.csv \\
        --write <out>/pmc_write/pmc_counter_collection.csv --md <summary> --json profiles/traffic.json
    python -m spmv_decode_amd.profiling stats --csv <out>/prof_bench/bench_kernel_stats.csv \\
        --bench <out>/bench.json --md <summary>
    python -m spmv_decode_amd.profiling cpu --bench <out>/bench_cpu.json --md <summary>

(<out>: the rocprofv3 output directory of the profiled run.)

`traffic` calibrates FETCH_SIZE / WRITE_SIZE (KiB per dispatch) against the
256 MiB copy that `microbench --traffic-probe` runs first (a kernel of known
size), then reports HBM bytes per launch for every GEMV kernel of the probe.
"""
from __future__ import annotations

import argparse
import csv
import json
from pathlib import Path

CALIBRATION_BYTES = 256 << 20  # the probe's fp16 copy: 128 Mi elements
COPY_GRID = "131072"

# Launch classes of the traffic probe, in probe order: (key, K, [h...], matrices, description).
PROBE_CLASSES = [
    ("q_o_32:64", 4096, [4096], 1, "q/o (4096 -> 4096)"),
    ("k_v_32:64", 4096, [1024], 1, "k/v (4096 -> 1024)"),
    ("gate_up_32:64", 4096, [14336], 1, "gate or up alone (4096 -> 14336)"),
    ("down_32:64", 14336, [4096], 1, "down (14336 -> 4096)"),
    ("qkv_grouped_32:64", 4096, [4096, 1024, 1024], 1, "grouped q/k/v (4096 -> 4096+1024+1024)"),
    ("gate_up_pair_32:64", 4096, [14336], 2, "gate/up pair with SiLU*mul (4096 -> 2x14336)"),
    ("qkv_decode_32:64", None, None, None, "q/k/v + input RMSNorm + RoPE + KV-cache write (decode form)"),
    ("o_resid_32:64", None, None, None, "o + residual add (decode form)"),
    ("gate_up_pair_norm_32:64", None, None, None, "gate/up pair + input RMSNorm (decode form)"),
    ("down_resid_32:64", None, None, None, "down + residual add (decode form)"),
    ("qkv_decode_carried_32:64", None, None, None, "q/k/v decode form, input carried from down's partials"),
    ("o_partials_32:64", None, None, None, "o, split partials left for the next launch"),
    ("gate_up_pair_norm_carried_32:64", None, None, None, "gate/up pair + RMSNorm, input carried from o's partials"),
    ("down_partials_32:64", None, None, None, "down, split partials left for the next launch"),
    ("qkv_decode_acc_32:64", None, None, None, "q/k/v decode form, input carried from down's accumulated row; "
                                               "clears o's and the pair's rows"),
    ("o_acc_32:64", None, None, None, "o, adding into an fp32 row (accumulated carry)"),
    ("gate_up_pair_acc_32:64", None, None, None, "gate/up pair + RMSNorm, input carried from o's row, adding its raw "
                                                 "sums into an fp32 row; clears down's row"),
    ("down_silu_acc_32:64", None, None, None, "down, input the pair's SiLU product, adding into an fp32 row"),
]


# SpMM calls of the traffic probe, after the GEMV classes: (key, K, h, rows, kernel, description); "mc" calls
# launch the operand-order gather and then the matrix-core kernel, "small" calls the small-batch kernel.
SPMM_PROBE_CLASSES = [
    ("spmm8_gate_up_32:64", 4096, 14336, 8, "small", "gate or up, 8 rows (small-batch SpMM)"),
    ("spmm8_down_32:64", 14336, 4096, 8, "small", "down, 8 rows (small-batch SpMM)"),
    ("mc16_gate_up_32:64", 4096, 14336, 16, "mc", "gate or up, 16 rows (matrix-core SpMM)"),
    ("mc64_gate_up_32:64", 4096, 14336, 64, "mc", "gate or up, 64 rows (matrix-core SpMM)"),
    ("mc16_down_32:64", 14336, 4096, 16, "mc", "down, 16 rows (matrix-core SpMM)"),
    ("mc64_down_32:64", 14336, 4096, 64, "mc", "down, 64 rows (matrix-core SpMM)"),
]


def spmm_algorithmic(K, h, rows, nnz=32, m=64):
    """Algorithmic bytes of one SpMM call: packed weights and index bytes once,
    every row's activations and outputs."""
    w = K // m * nnz
    return 2 * w * h + w + rows * (2 * K + 2 * h)


def _spmm_dispatches(rows):
    out = []
    for r in rows:
        n = r["Kernel_Name"]
        for k in ("nm_spmm_mc_kernel", "nm_gather_mc_kernel", "nm_spmm_kernel"):
            if k + "<" in n:
                out.append((k + n[n.index("<", n.index(k)):n.index(">", n.index(k)) + 1], float(r["Counter_Value"])))
                break
    return out


def _algorithmic(K, hs, nmat, nnz=32, m=64, key=None):
    if K is None:  # a decode-form class
        from .microbench import decode_form_bytes

        return decode_form_bytes(key.rsplit("_", 1)[0], nnz, m)
    w = K // m * nnz
    return sum(nmat * (2 * w * h + w) + 2 * h for h in hs) + 2 * K


def _read(path):
    return list(csv.DictReader(open(path)))


def gemv_args(name: str):
    """The template arguments of an nm_gemv_kernel name, <dtype, TH, U, G, NT,
    NMAT, NORM, CARRY, SILU>, as a dict (None for any other kernel)."""
    if "nm_gemv_kernel<" not in name:
        return None
    a = name[name.index("nm_gemv_kernel<") + len("nm_gemv_kernel<"):]
    a = [v.strip() for v in a[:a.index(">")].split(",")]
    keys = ("dtype", "th", "u", "g", "nt", "nmat", "norm", "carry", "silu")
    d = dict(zip(keys, a))
    return {k: (v == "true" if k in ("nt", "norm", "silu") else int(v)) for k, v in d.items()}


def _gemv_dispatches(rows):
    out = []
    for r in rows:
        n = r["Kernel_Name"]
        if "nm_gemv_kernel" in n:
            out.append((n[n.index("<"):n.index(">") + 1], float(r["Counter_Value"])))
    return out


def _copy_scale(rows):
    vals = [float(r["Counter_Value"]) for r in rows if "copy" in r["Kernel_Name"].lower() and r["Grid_Size"] == COPY_GRID]
    if not vals:
        raise SystemExit("calibration copy not found in the counter CSV")
    return (CALIBRATION_BYTES / 1024) / (sum(vals) / len(vals)), vals


def traffic(fetch_csv, write_csv, md_path, json_path, fetch_cmd, write_cmd):
    frows, wrows = _read(fetch_csv), _read(write_csv)
    fscale, fcopy = _copy_scale(frows)
    wscale, wcopy = _copy_scale(wrows)
    fd, wd = _gemv_dispatches(frows), _gemv_dispatches(wrows)
    if len(fd) != 3 * len(PROBE_CLASSES) or len(wd) != len(fd):
        raise SystemExit(f"expected {3 * len(PROBE_CLASSES)} GEMV dispatches per pass, got {len(fd)}/{len(wd)}")
    table, js = [], {}
    for i, (key, K, hs, nmat, desc) in enumerate(PROBE_CLASSES):
        fv = [v for _, v in fd[3 * i:3 * i + 3]]
        wv = [v for _, v in wd[3 * i:3 * i + 3]]
        fetch = sum(fv) / 3 * fscale * 1024
        write = sum(wv) / 3 * wscale * 1024
        alg = _algorithmic(K, hs, nmat, key=key)
        kern = fd[3 * i][0]
        js[key] = {"kernel": f"nm_gemv_kernel{kern}", "fetch_bytes": round(fetch), "write_bytes": round(write),
                   "bytes_per_launch": round(fetch + write), "algorithmic_bytes": alg,
                   "fetch_scale": round(fscale, 5), "write_scale": round(wscale, 5)}
        table.append(f"| {desc} | `nm_gemv_kernel{kern}` | {alg:,} | {round(fetch):,} | {round(write):,} | "
                     f"{(fetch + write) / alg:.4f} |")
    sf, sw = _spmm_dispatches(frows), _spmm_dispatches(wrows)
    per_call = {"small": 1, "mc": 2}
    need = sum(3 * per_call[c[4]] for c in SPMM_PROBE_CLASSES)
    if len(sf) != need or len(sw) != need:
        raise SystemExit(f"expected {need} SpMM dispatches per pass, got {len(sf)}/{len(sw)}")
    spmm_table, i = [], 0
    for key, K, h, nrows, kind, desc in SPMM_PROBE_CLASSES:
        n = per_call[kind]
        fcalls = [sf[i + j * n:i + (j + 1) * n] for j in range(3)]
        wcalls = [sw[i + j * n:i + (j + 1) * n] for j in range(3)]
        i += 3 * n
        alg = spmm_algorithmic(K, h, nrows)
        parts = []
        for d in range(n):  # per kernel of the call: average over the three calls
            kern = fcalls[0][d][0]
            fb = sum(c[d][1] for c in fcalls) / 3 * fscale * 1024
            wb = sum(c[d][1] for c in wcalls) / 3 * wscale * 1024
            parts.append((kern, fb, wb))
        fetch, write = sum(p[1] for p in parts), sum(p[2] for p in parts)
        js[key] = {"kernels": {k: {"fetch_bytes": round(f), "write_bytes": round(wv)} for k, f, wv in parts},
                   "fetch_bytes": round(fetch), "write_bytes": round(write), "bytes_per_call": round(fetch + write),
                   "algorithmic_bytes": alg}
        for kern, fb, wb in parts:
            spmm_table.append(f"| {desc} | `{kern}` | | {round(fb):,} | {round(wb):,} | |")
        spmm_table.append(f"| {desc}: the call | | {alg:,} | {round(fetch):,} | {round(write):,} | "
                          f"{(fetch + write) / alg:.4f} |")
    lines = ["# HBM traffic per launch: rocprofv3 FETCH_SIZE / WRITE_SIZE (Llama-3.1-8B shapes, 32:64, fp16)", "",
             "Commands (repository root, one MI355X; each counter in its own run), then the summary:", "", "```",
             "export TMPDIR=/tmp", fetch_cmd, write_cmd,
             "python -m spmv_decode_amd.profiling traffic --fetch gpurun_out/pmc_fetch/pmc_counter_collection.csv "
             "--write gpurun_out/pmc_write/pmc_counter_collection.csv --md <this file> --json profiles/traffic.json",
             "```", "",
             "The probe copies a 256 MiB fp16 buffer three times (the known-size calibration kernel), then launches",
             "each class three times on distinct weights with the library's default plan. Kernel template arguments:",
             "<dtype (0 = fp16), TH (tile = 8*TH rows), U (rows per lane per chunk), G (gather width / 256), NT, NMAT",
             "(2 = gate/up pair), NORM (input RMSNorm folded into the gather), CARRY (most producer splits a carried",
             "input reads; 0 = none)>. The decode-form classes are the launches of the decoder's fused layer",
             "(microbench.DecodeForms): plain, with the split carry and with the accumulated carry (`_acc`; the",
             "decoder's default, which bench.py times as its step).",
             "",
             f"Calibration: the 256 MiB copy reads {sum(fcopy) / len(fcopy):.1f} KiB by FETCH_SIZE (true "
             f"{CALIBRATION_BYTES // 1024} KiB) -> fetch scale {fscale:.4f}; it writes {sum(wcopy) / len(wcopy):.1f} KiB "
             f"by WRITE_SIZE -> write scale {wscale:.4f}. Scaled values below.", "",
             "| Launch | Kernel | Algorithmic bytes | Fetched (scaled) | Written (scaled) | Traffic / algorithmic |",
             "|---|---|---|---|---|---|", *table, "",
             "Extra fetch over the algorithmic bytes is the index bytes and activations re-read by every output tile",
             "of a split plus the partial sums read back by the last workgroup of each tile; extra writes are the fp32",
             "split-K partials (8 splits x h x 4 B per matrix). A carried launch also fetches the producer's partials",
             "(splits x K x 4 B, once per XCD's L2), and a producer writes them. An accumulating producer's adds",
             "are performed at the memory side (agent scope) and counted as writes of the fp32 rows; the launch",
             "that clears a row writes it once more. No weight byte is fetched twice.",
             "`profiles/traffic.json` holds the same numbers; bench.py reports `bytes_per_launch` of the dominant",
             "launch class as `roofline.traffic`.", "",
             "## SpMM calls (batch > 1)", "",
             "Three calls each on distinct weights, the library's default plans. A matrix-core call is two kernels: the",
             "gather of the activations into operand order (`nm_gather_mc_kernel<true>`) and the main kernel. The",
             "algorithmic bytes of a call count the packed weights and index bytes once and every row's activations",
             "and outputs.", "",
             "| Call | Kernel | Algorithmic bytes | Fetched (scaled) | Written (scaled) | Traffic / algorithmic |",
             "|---|---|---|---|---|---|", *spmm_table, "",
             "Over the algorithmic bytes: the fp32 split-K partials ([splits, rows, h], written once and read back by",
             "each tile's last workgroup), and for the matrix-core calls the gathered activations (written by the",
             "gather, then read by the main kernel: from L2 mostly, FETCH_SIZE counts only what reaches HBM)."]
    Path(md_path).write_text("\n".join(lines) + "\n")
    Path(json_path).write_text(json.dumps(js, indent=1) + "\n")


def stats(stats_csv, bench_json, md_path, cmd):
    rows = _read(stats_csv)
    b = json.loads(Path(bench_json).read_text()) if bench_json else None
    lines = ["# rocprofv3 kernel statistics: bench.py (Llama-3.1-8B decode-token sparse GEMVs, 32:64, fp16)", "",
             "Commands (repository root, one MI355X, one call):", "", "```", "export TMPDIR=/tmp",
             "python -u bench.py > gpurun_out/bench.json", cmd,
             "python -m spmv_decode_amd.profiling stats --csv gpurun_out/prof_bench/bench_kernel_stats.csv "
             "--bench gpurun_out/bench.json --md <this file>", "```", "",
             "The run covers the decode step graph with the accumulated carry (the timed step; per layer: q/k/v +",
             "RMSNorm + RoPE + cache write finishing the previous down's fp32 row, o adding into its row, the gate/up",
             "pair + RMSNorm finishing o's row and adding its raw sums into its own, down on the pair's SiLU product",
             "adding into its row), the same step with the split carry (o and down leave split partials, gate/up",
             "and q/k/v finish them), without a carry (o and down + residual), the plain fused step, the 224-launch",
             "step graph, per-class rotation graphs (>= 1 GiB of distinct weights each: accumulated, split-carried",
             "and plain classes), the SpMM graphs (batch 2-8: small-batch kernel; 16-64: the activation gather + the",
             "matrix-core kernel) and the dense",
             "hipBLASLt baseline graphs. `nm_gemv_kernel` template arguments: <dtype (0 = fp16), TH (tile = 8*TH",
             "rows), U (rows per lane per chunk), G (gather width / 256), NT, NMAT (2 = gate/up pair), NORM (input",
             "RMSNorm), CARRY (most producer splits of a carried input, 1 = an accumulated row; 0 = none), SILU",
             "(input the gate/up pair's SiLU product)>; `nm_spmm_kernel`: <dtype, TH, U,",
             "G, NT, batch rows per launch>; `nm_spmm_mc_kernel`: <dtype, batch rows per tile, output columns",
             "per tile, weights DMA-staged into LDS>.", "",
             "| Kernel | Calls | Avg (us) | Min (us) | Max (us) | Share of GPU time |", "|---|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:12]:
        n = r["Name"].replace("void nm_hip::", "").replace("(nm_hip::Args)", "")
        n = n if len(n) <= 90 else n[:87] + "..."
        lines.append(f"| `{n}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                     f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f}% |")
    if b:
        rf = b.get("roofline", {})
        pair = [r for r in rows if (gemv_args(r["Name"]) or {}).get("nmat") == 2]
        lines += ["", f"Unprofiled `python bench.py` from the same call: value {b['value']} GB/s, ms_per_step "
                      f"{b['ms_per_step']}; dominant launch class: {rf.get('kernel')} at {rf.get('us_per_launch')} us "
                      f"per launch (HIP events over replays of a graph of >= 64 of its launches, {rf.get('achieved')} "
                      f"GB/s, frac {rf.get('frac')})."]
        for r in pair:
            g = gemv_args(r["Name"])
            if not g["norm"]:
                continue
            what = ("with its input finished from an accumulated row (the timed step's)" if g.get("carry") == 1 else
                    "with its input finished from split partials" if g.get("carry") else "with its own input")
            lines.append(f"rocprof average kernel duration of the gate/up pair + RMSNorm kernel {what}: "
                         f"{float(r['AverageNs']) / 1e3:.2f} us over {r['Calls']} calls (the kernel alone, in the traced "
                         "run; the replay-timed figure is the interval per launch in the untraced one, gap included).")
    Path(md_path).write_text("\n".join(lines) + "\n")


def decode_stats(stats_csv, decode_json, md_path, cmd):
    """Per-token kernel time of a hipGraph decode run from its rocprofv3 stats."""
    from .decode.model import CONFIGS

    rows = _read(stats_csv)
    d = json.loads(Path(decode_json).read_text())
    layers = CONFIGS[d["model"]].n_layers
    pair = [r for r in rows if (gemv_args(r["Name"]) or {}).get("nmat") == 2]
    steps = sum(int(r["Calls"]) for r in pair) // layers  # one gate/up launch per layer and step

    def kind(r):
        n, per_step = r["Name"], int(r["Calls"]) / steps
        if per_step < 0.9:
            return None  # model set-up (random init, packing), not part of a step
        g = gemv_args(n)
        if g is not None:
            if g["nmat"] == 2:
                return "sparse GEMV: gate/up pair + RMSNorm (+ SiLU*mul, or its sums accumulated)"
            # the input norm marks the q/k/v launch
            return ("sparse GEMV: q/k/v + RMSNorm + RoPE + cache write" if g["norm"]
                    else "sparse GEMV: o or down (+ residual, or partials left / accumulated)")
        if n.startswith("Cijk_"):
            return "attention product (hipBLASLt)" if per_step > 1.5 else "lm_head (hipBLASLt, dense)"
        if "softmax" in n:
            return "attention softmax"
        return "other (embedding, norm, mask, greedy token, position)"

    def step_us(r):  # average duration x launches per step (set-up calls of a step kernel left out)
        return float(r["AverageNs"]) * round(int(r["Calls"]) / steps) / 1e3

    per = {}
    rows = [r for r in rows if kind(r) is not None]
    for r in rows:
        c = kind(r)
        per[c] = per.get(c, 0.0) + step_us(r)
    total = sum(per.values())
    sp = d["sparse"]
    lines = [f"# rocprofv3 kernel statistics: hipGraph decode, {d['model']} {sp.get('ratio', '')}, fp16, batch 1", "",
             "Command (repository root, one MI355X):", "", "```", "export TMPDIR=/tmp", cmd,
             "python -m spmv_decode_amd.profiling decode-stats --csv <stats csv> --decode <json> --command '<the line "
             "above>' --md <this file>",
             "```", "",
             f"{steps} decode steps were profiled (capture warm-up, the {d['prompt']}-token prompt and {d['gen']}",
             "generated tokens, one graph replay each). Kernel time per step, summed by role: rocprof durations of",
             "the kernels only (the graph's inter-kernel gaps are not included), each kernel's average duration",
             "times its launches per step; the model's set-up kernels (random init, packing, the lm_head form",
             "timing) are left out:", "",
             "| Role | us per step | Share |", "|---|---|---|"]
    for c, v in sorted(per.items(), key=lambda kv: -kv[1]):
        lines.append(f"| {c} | {v:.1f} | {100 * v / total:.1f}% |")
    lines += [f"| total kernel time | {total:.1f} | |", "",
              f"The profiled run itself measured {sp['ms_per_token']} ms/token (HIP events around the replays,",
              "under the profiler).", "",
              "| Kernel | Calls | Avg (us) | Per step (us) |", "|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -step_us(r))[:12]:
        n = r["Name"].replace("void nm_hip::", "").replace("(nm_hip::Args)", "")
        n = n if len(n) <= 90 else n[:87] + "..."
        lines.append(f"| `{n}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {step_us(r):.2f} |")
    Path(md_path).write_text("\n".join(lines) + "\n")


def decode_table(json_paths):
    """The decode tables of profiles/decode_*.md: one row per variant of each
    `bench_decode --json` file, then the speedups over dense (the headline
    dense variant, then over the fastest dense fusion mode when several ran)."""
    names = {"llama-3.1-8b": "Llama-3.1-8B", "qwen3-14b": "Qwen3-14B", "qwen3-32b": "Qwen3-32B"}
    fusion_label = {"qkv": "dense, q/k/v fused", "none": "dense, one GEMM per Linear",
                    "qkv_gate_up": "dense, q/k/v and gate/up fused"}
    rows, speed = [], []
    docs = [json.loads(Path(path).read_text()) for path in json_paths]
    fixed = bool(docs) and all(d.get("protocol") == "fixed_context" for d in docs)
    if any(d.get("protocol") == "fixed_context" for d in docs) and not fixed:
        raise SystemExit("decode-table: do not mix fixed-context and generation runs in one table")
    for d in docs:
        model = names.get(d["model"], d["model"])
        pg = f"CTX {d['ctx']}" if fixed else f"{d['prompt']} / {d['gen']}"
        ratio = d.get("sparse", {}).get("ratio", "")
        sparse_bytes = d.get("sparse", {}).get("linear_bytes_per_token")
        dense = [("dense", d["dense"])] if d.get("dense") else []
        dense += [(k, v) for k, v in d.get("dense_variants", {}).items()]
        variants = [(fusion_label.get(v.get("fusion"), "dense"), v, None) for _, v in dense]
        variants += [(f"{ratio} fused layer", d.get("sparse"), sparse_bytes),
                     (f"{ratio} per-Linear", d.get("sparse_per_linear"), sparse_bytes),
                     (f"{ratio} grouped", d.get("sparse_grouped"), sparse_bytes),
                     (f"{ratio} unmodified model (module calls, " + ("each its own launch" if d.get("compiled")
                      else "tied q/k/v and gate/up") + ")", d.get("sparse_modules"), sparse_bytes)]
        if d.get("compiled"):
            variants = [(f"{label}, compiled", v, nb) for label, v, nb in variants]
        for label, v, nbytes in variants:
            if not v:
                continue
            nb = v.get("linear_bytes_per_token", nbytes)
            second = (f"{v['ms_per_token_mean']:.4f} | {v['stdev']:.4f}" if fixed
                      else f"{v['ms_per_token_median_of_16']:.4f}")
            rows.append(f"| {model} | {pg} | {label} | {v['ms_per_token']:.4f} | {second} | {v['tokens_per_s']} | "
                        f"{nb:,} |")
        if "speedup_sparse_vs_dense" in d:
            line = f"{model} {ratio}: fused layer {d['speedup_sparse_vs_dense']:.4f}x"
            if "speedup_sparse_per_linear_vs_dense" in d:
                line += f", per-Linear {d['speedup_sparse_per_linear_vs_dense']:.4f}x"
            if "speedup_sparse_grouped_vs_dense" in d:
                line += f", grouped {d['speedup_sparse_grouped_vs_dense']:.4f}x"
            if "speedup_sparse_modules_vs_dense" in d:
                line += f", unmodified model {d['speedup_sparse_modules_vs_dense']:.4f}x"
            hd = fusion_label.get(d["dense"].get("fusion"), "dense")
            line += f" (over {hd})"
            if len(dense) > 1 and d.get("sparse"):
                best_label, best = min(((fusion_label.get(v.get("fusion"), k), v) for k, v in dense),
                                       key=lambda t: t[1]["ms_per_token"])
                line += (f"; fused layer over the fastest dense ({best_label}) "
                         f"{best['ms_per_token'] / d['sparse']['ms_per_token']:.4f}x")
                for key, lab in (("sparse_per_linear", "per-Linear"), ("sparse_grouped", "grouped"),
                                 ("sparse_modules", "unmodified model")):
                    if d.get(key):
                        line += f", {lab} {best['ms_per_token'] / d[key]['ms_per_token']:.4f}x"
            if d.get("speedup_structure_matched"):
                line += "; structure-matched: " + ", ".join(
                    f"{k.replace('_', ' ')} {v:.4f}x" for k, v in d["speedup_structure_matched"].items())
            speed.append(line)
    if fixed:
        head = ["| Model | Context | Variant | ms/token (median of samples) | mean | stdev | tokens/s | "
                "Linear bytes/token |", "|---|---|---|---|---|---|---|---|"]
    else:
        head = ["| Model | Prompt / gen | Variant | ms/token (mean) | median of 16-step chunks | tokens/s | "
                "Linear bytes/token |", "|---|---|---|---|---|---|---|"]
    return "\n".join(head + rows + [""] + [f"Speedup over dense: {x}." for x in speed]) + "\n"


# The reference's published decode table (README.md:86-119): A100-SXM4-80GB, CTX 512, fp16, batch 1,
# median ms/token of its fixed-context benchmark; dense, then by M at N = M/2.
REFERENCE_A100_CTX512 = {
    "llama-3.1-8b": (10.3904, {4: 8.0753, 8: 8.1507, 16: 6.9512, 32: 6.9400, 64: 6.8521, 128: 7.0335, 256: 7.2585}),
    "qwen3-14b": (25.0951, {4: 20.3801, 8: 20.4739, 16: 18.0455, 32: 17.8283, 64: 17.6093, 128: 17.9491,
                            256: 19.1014}),
    "qwen3-32b": (52.3758, {4: 39.8042, 8: 38.5639, 16: 33.7534, 32: 33.7054, 64: 33.7408, 128: 34.4702,
                            256: 36.5712}),
}


def fixed_compare(json_paths):
    """Fixed-context (`bench_decode --fixed-ctx`) results next to the
    reference's published table: per model, this build's dense (its headline
    structure) and each ratio's sparse ms/token with the speedup over that
    dense, then the reference's figures and speedups."""
    names = {"llama-3.1-8b": "Llama-3.1-8B", "qwen3-14b": "Qwen3-14B", "qwen3-32b": "Qwen3-32B"}
    dense, sparse = {}, {}
    for path in json_paths:
        d = json.loads(Path(path).read_text())
        if d.get("protocol") != "fixed_context":
            raise SystemExit(f"fixed-compare: {path} is not a --fixed-ctx run")
        if d.get("dense"):
            dense[d["model"]] = d["dense"]["ms_per_token"]
        if d.get("sparse"):
            m = int(d["sparse"]["ratio"].split(":")[1])
            sparse.setdefault(d["model"], {})[m] = d["sparse"]["ms_per_token"]
    lines = ["| Model | Pattern | This build, MI355X: ms/token | speedup over its dense | Reference, A100: ms/token "
             "| speedup over its dense |", "|---|---|---|---|---|---|"]
    for model in sorted(set(dense) | set(sparse), key=list(names).index):
        rd, rs = REFERENCE_A100_CTX512[model]
        ours = dense.get(model)
        lines.append(f"| {names[model]} | dense | {ours:.4f} | 1.000x | {rd:.4f} | 1.000x |" if ours else
                     f"| {names[model]} | dense | - | - | {rd:.4f} | 1.000x |")
        for m, v in sorted(sparse.get(model, {}).items()):
            sp = f"{ours / v:.3f}x" if ours else "-"
            rv = rs.get(m)
            ref = f"{rv:.4f} | {rd / rv:.3f}x" if rv else "- | -"
            lines.append(f"| {names[model]} | {m // 2}:{m} | {v:.4f} | {sp} | {ref} |")
    return "\n".join(lines) + "\n"


def sweep_stats(trace_csv, sweep_csv, md_path, cmd):
    """Per (configuration, split count) of a `microbench --sweep` run: the
    HIP-event time per launch it measured and the average kernel duration
    rocprofv3 traced for the same kernel and grid, with the GB/s of each."""
    import re

    sweep = _read(sweep_csv)
    groups = {}
    with open(trace_csv, newline="") as f:
        rd = csv.DictReader(f)
        for r in rd:
            name = r.get("Kernel_Name", "")
            # plain single-matrix launches (NMAT 1, no norm) and the gate/up pair with its norm (NMAT 2)
            mt = re.search(r"nm_gemv_kernel<\d+, (\d+), (\d+), \d+, (true|false), (\d), (true|false)>", name)
            if not mt:
                continue
            lanes = int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 256)
            grid = int(r.get("Grid_Size_X") or r.get("Grid_Size"))
            key = (int(mt.group(1)), int(mt.group(2)), mt.group(3) == "true", grid // max(lanes, 1),
                   int(mt.group(4)), mt.group(5) == "true")
            dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            g = groups.setdefault(key, [0, 0.0])
            g[0] += 1
            g[1] += dur
    lines = ["# Configuration sweep by rocprofv3 kernel duration (configuration x split count)", "",
             "Command (repository root, one MI355X):", "", "```", "export TMPDIR=/tmp", cmd,
             "python -m spmv_decode_amd.profiling sweep-stats --trace <the kernel trace csv> --sweep <the --csv file> "
             "--command '<the line above>' --md <this file>", "```", "",
             "Each row: one configuration (TH lanes across a 8*TH-row tile, U rows per lane per chunk; `_cached` =",
             "ordinary instead of non-temporal loads) at one split count, weights rotated over >= 1 GiB; `rocprof us`",
             "is the average duration rocprofv3 traced for the dispatches of that kernel with that grid, GB/s count",
             "the algorithmic bytes. The 10 fastest rows and the library's own choice are shown. The tracer's",
             "per-dispatch bookkeeping slows the launches (the same run's HIP-event times are inflated and left",
             "out); the library's defaults come from untraced graph-replay sweeps (the decoder's condition), where",
             "they are the fastest or within 0.3 us of it.", ""]
    by_shape = {}
    for r in sweep:
        by_shape.setdefault((r["n_out"], r["n_in"], r["ratio"]), []).append(r)
    for (n_out, n_in, ratio), rows in by_shape.items():
        nbytes = float(rows[0]["GBps"]) * float(rows[0]["us"]) * 1e3
        timed = []
        for r in rows:
            cfgname = r["config"].split(":")[-1]
            mt = re.match(r"(?:pair_)?th(\d+)_u(\d+)(_cached)?", cfgname)
            key = (int(mt.group(1)), int(mt.group(2)), not mt.group(3), int(r["blocks"]), int(r.get("nmat") or 1),
                   bool(int(r.get("norm") or 0)))
            n, tot = groups.get(key, (0, 0.0))
            if n:
                timed.append((tot / n / 1e3, n, r))
        auto = next((t for t in timed if t[2]["config"].startswith("auto:")), None)
        ranked = sorted((t for t in timed if not t[2]["config"].startswith("auto:")), key=lambda t: t[0])
        pair = any(str(r.get("nmat")) == "2" for r in rows)
        normed = any(str(r.get("norm")) == "1" for r in rows)
        title = (f"gate/up pair + RMSNorm + SiLU*mul, {n_in} -> 2 x {n_out}" if pair else
                 f"q/k/v + RMSNorm + RoPE + cache write, {n_in} -> {n_out}" if normed else f"{n_in} -> {n_out}")
        lines += [f"## {title}, {ratio} ({nbytes / 1e6:.1f} MB per launch)", "",
                  "| config | splits | workgroups | rocprof us | GB/s | % of 8 TB/s | dispatches |",
                  "|---|---|---|---|---|---|---|"]
        for rp, n, r in ([auto] if auto else []) + ranked[:10]:
            label = f"{r['config'].split(':')[-1]} (library choice)" if auto and r is auto[2] else r["config"]
            gbs = nbytes / rp / 1e3
            lines.append(f"| {label} | {r['splits']} | {r['blocks']} | {rp:.2f} | {gbs:.0f} | {gbs / 80:.1f}% | {n} |")
        if auto and ranked:
            lines.append(f"\nLibrary choice {auto[0]:.2f} us against the fastest traced {ranked[0][0]:.2f} us "
                         f"({100 * (auto[0] / ranked[0][0] - 1):+.1f}%).")
        lines.append("")
    Path(md_path).write_text("\n".join(lines))


def cpu(bench_json, md_path, cmd):
    """CPU baseline summary from a `bench.py --cpu-detail --cpu-decode` JSON line."""
    b = json.loads(Path(bench_json).read_text())
    c = b["cpu_baseline"]
    d = c["detail"]
    t = d["threads"]
    lines = ["# CPU baseline on the GPU box's host cores (the reference's PyTorch formulation of the op)", "",
             "Command (repository root, one MI355X box):", "", "```", cmd, "```", "",
             "The reference has no CPU kernel for this op (every call rejects CPU tensors), so its CPU path is its",
             "own PyTorch formulation: CPU-A = the microbenchmark's oracle, scatter to a dense weight then fp32",
             "`torch.mv`; CPU-B = the gather form `mat_data.float().T @ x.float()[sel]` (same math, no dense",
             "weight). Both from `oracle/nm_oracle.py`, timed with `time.perf_counter`: 3 warm-ups, then the median",
             f"(and stdev) of {d['reps']} calls ({max(5, d['reps'] // 4)} at one thread for the 58 MB shapes). GB/s counts",
             "the same algorithmic bytes as the GPU figures.", "",
             f"| Shape | Bytes | CPU-A {t} thr (ms) | CPU-B {t} thr (ms) | CPU-B {t} thr GB/s | CPU-A 1 thr (ms) | "
             "CPU-B 1 thr (ms) | CPU-B 1 thr GB/s |", "|---|---|---|---|---|---|---|---|"]
    for r in d["rows"]:
        lines.append(f"| {r['shape']} | {r['bytes']:,} | {r[f'cpu_a_{t}t_ms']:.2f} +- {r[f'cpu_a_{t}t_sd_ms']:.2f} | "
                     f"{r[f'cpu_b_{t}t_ms']:.2f} +- {r[f'cpu_b_{t}t_sd_ms']:.2f} | {r[f'cpu_b_{t}t_GBps']:.2f} | "
                     f"{r['cpu_a_1t_ms']:.2f} | {r['cpu_b_1t_ms']:.2f} | {r['cpu_b_1t_GBps']:.2f} |")
    dec = c.get("decode")
    lines += ["", f"Headline `cpu_baseline` of the same run: {c['value']} GB/s ({c['ms_per_layer']} ms per Llama-3.1-8B "
                  f"layer of 7 CPU-B GEMVs, {c['cores']} threads; one thread {c['one_thread']['value']} GB/s)."]
    if dec:
        lines.append(f"CPU decode step: {dec['ms_per_token']} ms/token ({dec['sample']}; per token "
                     f"{', '.join(str(v) for v in dec['per_token_ms'])} ms; {dec['threads']} threads), against "
                     f"{b['decode']['sparse_ms_per_token']} ms/token for the hipGraph decode on the GPU in the same run.")
    Path(md_path).write_text("\n".join(lines) + "\n")


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--md", required=True)
    t.add_argument("--json", required=True)
    c = sub.add_parser("cpu")
    c.add_argument("--bench", required=True)
    c.add_argument("--md", required=True)
    s = sub.add_parser("stats")
    s.add_argument("--csv", required=True)
    s.add_argument("--bench", default=None)
    s.add_argument("--md", required=True)
    sw = sub.add_parser("sweep-stats")
    sw.add_argument("--trace", required=True, help="rocprofv3 kernel trace CSV of a microbench --sweep run")
    sw.add_argument("--sweep", required=True, help="the microbench --csv of the same run")
    sw.add_argument("--md", required=True)
    sw.add_argument("--command", dest="command_line", required=True)
    fcmp = sub.add_parser("fixed-compare")
    fcmp.add_argument("json", nargs="+", help="bench_decode --fixed-ctx --json files")
    dt = sub.add_parser("decode-table")
    dt.add_argument("json", nargs="+", help="bench_decode --json files")
    ds = sub.add_parser("decode-stats")
    ds.add_argument("--csv", required=True)
    ds.add_argument("--decode", required=True)
    ds.add_argument("--md", required=True)
    ds.add_argument("--command", dest="command_line", required=True,
                    help="the rocprofv3 command line the stats come from")
    a = p.parse_args(argv)
    if a.cmd == "traffic":
        traffic(a.fetch, a.write, a.md, a.json,
                "rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o pmc --output-format csv -- "
                "python -u -m spmv_decode_amd.microbench --traffic-probe",
                "rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_write -o pmc --output-format csv -- "
                "python -u -m spmv_decode_amd.microbench --traffic-probe")
    elif a.cmd == "sweep-stats":
        sweep_stats(a.trace, a.sweep, a.md, a.command_line)
    elif a.cmd == "decode-table":
        print(decode_table(a.json), end="")
    elif a.cmd == "fixed-compare":
        print(fixed_compare(a.json), end="")
    elif a.cmd == "decode-stats":
        decode_stats(a.csv, a.decode, a.md, a.command_line)
    elif a.cmd == "cpu":
        cpu(a.bench, a.md, "python -u bench.py --cpu-detail --cpu-decode > gpurun_out/bench_cpu.json")
    else:
        stats(a.csv, a.bench, a.md,
              "rocprofv3 --kernel-trace --stats -d /tmp/prof_bench -o bench --output-format csv -- "
              "python -u bench.py --no-decode --no-cpu && mkdir -p gpurun_out/prof_bench && "
              "cp $(find /tmp/prof_bench -name bench_kernel_stats.csv) gpurun_out/prof_bench/")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
