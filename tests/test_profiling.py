"""The profile summarisers (spmv_decode_amd.profiling) on synthetic inputs:
the decode tables and the per-role accounting of a rocprofv3 decode run."""
import csv
import json

import pytest

from spmv_decode_amd import profiling as P


def _variant(ms, fusion=None):
    v = {"ms_per_token": ms, "ms_per_token_median_of_16": ms, "tokens_per_s": round(1e3 / ms, 2),
         "linear_bytes_per_token": 1000}
    if fusion:
        v["fusion"] = fusion
    return v


def test_decode_table_rows_and_speedups(tmp_path):
    d = {"model": "llama-3.1-8b", "prompt": 128, "gen": 256,
         "dense": _variant(5.0, "qkv"), "dense_variants": {"none": _variant(6.0, "none"),
                                                           "qkv_gate_up": _variant(4.0, "qkv_gate_up")},
         "sparse": {**_variant(2.0), "ratio": "32:64", "linear_bytes_per_token": 500},
         "sparse_per_linear": _variant(4.0), "sparse_grouped": _variant(3.2),
         "speedup_sparse_vs_dense": 2.5, "speedup_sparse_per_linear_vs_dense": 1.25,
         "speedup_sparse_grouped_vs_dense": 1.5625}
    path = tmp_path / "d.json"
    path.write_text(json.dumps(d))
    out = P.decode_table([str(path)])
    lines = out.splitlines()
    rows = [ln for ln in lines if ln.startswith("| Llama-3.1-8B")]
    assert [r.split(" | ")[2] for r in rows] == [
        "dense, q/k/v fused", "dense, one GEMM per Linear", "dense, q/k/v and gate/up fused",
        "32:64 fused layer", "32:64 per-Linear", "32:64 grouped"]
    assert "| 2.0000 |" in rows[3] and "| 500 |" in rows[3]
    speed = lines[-1]
    assert "fused layer 2.5000x" in speed and "grouped 1.5625x" in speed and "(over dense, q/k/v fused)" in speed
    # the fastest dense variant is the q/k/v + gate/up one (4.0 ms): 4.0 / 2.0, 4.0 / 4.0, 4.0 / 3.2
    assert "fastest dense (dense, q/k/v and gate/up fused) 2.0000x, per-Linear 1.0000x, grouped 1.2500x" in speed


def test_decode_table_unmodified_model_row_and_structure_matched_ratios(tmp_path):
    d = {"model": "llama-3.1-8b", "prompt": 128, "gen": 256,
         "dense": _variant(5.0, "qkv"), "dense_variants": {"none": _variant(6.0, "none")},
         "sparse": {**_variant(2.0), "ratio": "32:64"}, "sparse_modules": _variant(3.75),
         "speedup_sparse_vs_dense": 2.5, "speedup_sparse_modules_vs_dense": 1.3333,
         "speedup_structure_matched": {"fused_vs_dense_qkv_fused": 2.5, "modules_vs_dense_per_linear": 1.6}}
    path = tmp_path / "m.json"
    path.write_text(json.dumps(d))
    out = P.decode_table([str(path)])
    rows = [ln for ln in out.splitlines() if ln.startswith("| Llama-3.1-8B")]
    assert rows[-1].split(" | ")[2] == "32:64 unmodified model (module calls, tied q/k/v and gate/up)"
    speed = out.splitlines()[-1]
    assert "unmodified model 1.3333x" in speed and "fastest dense (dense, q/k/v fused) 2.5000x" in speed
    assert "structure-matched: fused vs dense qkv fused 2.5000x, modules vs dense per linear 1.6000x" in speed


def test_decode_table_compiled_unmodified_model_row_names_no_ties(tmp_path):
    """Under torch.compile the sibling ties stand aside: the row must not claim them."""
    fixed = lambda ms: {**_variant(ms), "ms_per_token_mean": ms, "stdev": 0.01}  # noqa: E731
    d = {"model": "qwen3-14b", "protocol": "fixed_context", "ctx": 512, "compiled": True,
         "sparse": {**fixed(4.0), "ratio": "32:64"}, "sparse_modules": fixed(6.5)}
    path = tmp_path / "c.json"
    path.write_text(json.dumps(d))
    rows = [ln for ln in P.decode_table([str(path)]).splitlines() if ln.startswith("| Qwen3-14B")]
    assert [r.split(" | ")[2] for r in rows] == [
        "32:64 fused layer, compiled", "32:64 unmodified model (module calls, each its own launch), compiled"]


def test_decode_table_sparse_only(tmp_path):
    d = {"model": "qwen3-14b", "prompt": 128, "gen": 256, "sparse": {**_variant(4.0), "ratio": "8:16"}}
    path = tmp_path / "s.json"
    path.write_text(json.dumps(d))
    out = P.decode_table([str(path)])
    assert "| Qwen3-14B | 128 / 256 | 8:16 fused layer | 4.0000 |" in out and "Speedup" not in out


def test_decode_table_fixed_context(tmp_path):
    fc = lambda ms, **kw: {"ms_per_token": ms, "ms_per_token_mean": ms + 0.01, "stdev": 0.002,  # noqa: E731
                           "tokens_per_s": round(1e3 / ms, 2), "linear_bytes_per_token": 1000, **kw}
    d = {"model": "llama-3.1-8b", "protocol": "fixed_context", "ctx": 512, "dense": fc(5.0, fusion="qkv"),
         "sparse": fc(2.5, ratio="32:64"), "speedup_sparse_vs_dense": 2.0}
    path = tmp_path / "f.json"
    path.write_text(json.dumps(d))
    out = P.decode_table([str(path)])
    assert "| Model | Context | Variant | ms/token (median of samples) | mean | stdev |" in out
    assert "| Llama-3.1-8B | CTX 512 | 32:64 fused layer | 2.5000 | 2.5100 | 0.0020 | 400.0 | 1,000 |" in out
    gen = tmp_path / "g.json"
    gen.write_text(json.dumps({"model": "qwen3-14b", "prompt": 1, "gen": 2, "sparse": {**_variant(4.0), "ratio": "x"}}))
    with pytest.raises(SystemExit, match="mix"):
        P.decode_table([str(path), str(gen)])


def test_fixed_compare_against_the_reference_table(tmp_path):
    fc = lambda ms, **kw: {"ms_per_token": ms, "ms_per_token_mean": ms, "stdev": 0.0,  # noqa: E731
                           "tokens_per_s": 1.0, **kw}
    paths = []
    for name, d in (("d", {"dense": fc(5.0, fusion="qkv")}), ("s4", {"sparse": fc(2.5, ratio="2:4")}),
                    ("s64", {"sparse": fc(2.0, ratio="32:64")})):
        path = tmp_path / f"{name}.json"
        path.write_text(json.dumps({"model": "llama-3.1-8b", "protocol": "fixed_context", "ctx": 512, **d}))
        paths.append(str(path))
    out = P.fixed_compare(paths)
    assert "| Llama-3.1-8B | dense | 5.0000 | 1.000x | 10.3904 | 1.000x |" in out
    assert "| Llama-3.1-8B | 2:4 | 2.5000 | 2.000x | 8.0753 | 1.287x |" in out
    assert "| Llama-3.1-8B | 32:64 | 2.0000 | 2.500x | 6.8521 | 1.516x |" in out
    gen = tmp_path / "g.json"
    gen.write_text(json.dumps({"model": "llama-3.1-8b", "prompt": 1, "gen": 2}))
    with pytest.raises(SystemExit, match="not a --fixed-ctx run"):
        P.fixed_compare([str(gen)])


def test_fixed_context_rejects_non_positive_arguments():
    from spmv_decode_amd.decode.model import Decoder, tiny_config
    from spmv_decode_amd.decode.runner import fixed_context_ms

    with pytest.raises(ValueError, match="positive"):
        fixed_context_ms(Decoder(tiny_config()), 0)


def _stats_csv(path, kernels):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writeheader()
        for name, calls, avg_us in kernels:
            w.writerow({"Name": name, "Calls": calls, "TotalDurationNs": calls * avg_us * 1e3,
                        "AverageNs": avg_us * 1e3, "Percentage": 1.0})


@pytest.mark.parametrize("setup_calls", [0, 11])
def test_decode_stats_roles_per_step(tmp_path, setup_calls):
    """Roles summed per step from average x launches per step; set-up kernels
    and the lm_head form timing calls (a few extra launches of a per-step
    kernel) do not change the per-step figures."""
    layers, steps = 32, 386  # llama-3.1-8b
    ls = layers * steps
    kernels = [
        # the carried layer: every gate/up and all but the first q/k/v read a carried input
        ("void nm_hip::nm_gemv_kernel<0, 32, 4, 1, true, 2, true, 8>(nm_hip::Args)", ls, 23.0),
        ("void nm_hip::nm_gemv_kernel<0, 16, 8, 4, true, 1, false, 0>(nm_hip::Args)", ls, 10.0),  # down
        ("void nm_hip::nm_gemv_kernel<0, 16, 8, 1, true, 1, false, 0>(nm_hip::Args)", ls, 10.0),  # o (G=1, NT)
        ("void nm_hip::nm_gemv_kernel<0, 32, 8, 1, true, 1, true, 8>(nm_hip::Args)", ls - steps, 9.5),
        ("void nm_hip::nm_gemv_kernel<0, 32, 8, 1, true, 1, true, 0>(nm_hip::Args)", steps, 9.5),
        ("Cijk_Alik_Bljk_HHS_MT256x16x32", ls, 8.0),
        ("Cijk_Ailk_Bljk_HHS_MT16x16x32", ls, 6.0),
        ("Cijk_Ailk_Bljk_HHS_MT1x4x256", steps + setup_calls, 180.0),
        ("void softmax_warp_forward<c10::Half>", ls, 5.0),
        ("void at::native::reduce_kernel<ArgMax>", steps, 5.0),
        ("void distribution_elementwise_grid_stride_kernel<normal>", 232, 48.0),  # random init: set-up
    ]
    _stats_csv(tmp_path / "k.csv", kernels)
    (tmp_path / "d.json").write_text(json.dumps({"model": "llama-3.1-8b", "prompt": 128, "gen": 256,
                                                 "sparse": {"ms_per_token": 2.6, "ratio": "32:64"}}))
    md = tmp_path / "out.md"
    P.decode_stats(str(tmp_path / "k.csv"), str(tmp_path / "d.json"), str(md), "cmd")
    text = md.read_text()
    assert f"{steps} decode steps were profiled" in text

    def role(name):
        line = next(ln for ln in text.splitlines() if ln.startswith(f"| {name} |"))
        return float(line.split(" | ")[1])

    assert role("sparse GEMV: gate/up pair + RMSNorm (+ SiLU*mul, or its sums accumulated)") == pytest.approx(32 * 23.0)
    assert role("sparse GEMV: o or down (+ residual, or partials left / accumulated)") == pytest.approx(64 * 10.0)
    assert role("sparse GEMV: q/k/v + RMSNorm + RoPE + cache write") == pytest.approx(32 * 9.5)
    assert role("attention product (hipBLASLt)") == pytest.approx(32 * 14.0)
    assert role("lm_head (hipBLASLt, dense)") == pytest.approx(180.0)
    assert role("attention softmax") == pytest.approx(32 * 5.0)
    assert role("other (embedding, norm, mask, greedy token, position)") == pytest.approx(5.0)
    total = 32 * 23.0 + 640 + 32 * 9.5 + 32 * 14.0 + 180 + 160 + 5
    assert role("total kernel time") == pytest.approx(total, abs=0.1)
    assert "distribution_elementwise" not in text


def test_sweep_stats_joins_pair_rows_to_the_pair_kernel(tmp_path):
    """A pair sweep row (pair_th32_u4, 448 workgroups) takes the duration of
    the traced NMAT=2 kernel with that grid, not a single-matrix kernel's."""
    trace = tmp_path / "trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Workgroup_Size_X", "Grid_Size_X", "Start_Timestamp",
                                          "End_Timestamp"])
        w.writeheader()
        for name, grid, dur in (("nm_gemv_kernel<0, 32, 4, 1, true, 2, true>(nm_hip::Args)", 448 * 256, 22_000),
                                ("nm_gemv_kernel<0, 32, 4, 1, true, 1, false>(nm_hip::Args)", 448 * 256, 11_000),
                                ("nm_gemv_kernel<0, 64, 8, 1, true, 2, true>(nm_hip::Args)", 448 * 256, 24_000)):
            for i in range(3):
                w.writerow({"Kernel_Name": name, "Workgroup_Size_X": 256, "Grid_Size_X": grid,
                            "Start_Timestamp": 1000 * i, "End_Timestamp": 1000 * i + dur})
    sweep = tmp_path / "sweep.csv"
    rows = [{"config": "auto:pair_th32_u4", "config_id": 1, "n_out": 14336, "n_in": 4096, "ratio": "32:64",
             "splits": 8, "blocks": 448, "us": 24.0, "GBps": 4895.4, "nmat": 2, "norm": 1},
            {"config": "pair_th64_u8", "config_id": 5, "n_out": 14336, "n_in": 4096, "ratio": "32:64",
             "splits": 16, "blocks": 448, "us": 25.0, "GBps": 4699.6, "nmat": 2, "norm": 1}]
    with open(sweep, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    md = tmp_path / "s.md"
    P.sweep_stats(str(trace), str(sweep), str(md), "cmd")
    text = md.read_text()
    assert "gate/up pair + RMSNorm + SiLU*mul, 4096 -> 2 x 14336" in text
    assert "| pair_th32_u4 (library choice) | 8 | 448 | 22.00 |" in text
    assert "| pair_th64_u8 | 16 | 448 | 24.00 |" in text
