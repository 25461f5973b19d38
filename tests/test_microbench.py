"""Measurement definitions of spmv_decode_amd.microbench: the algorithmic
byte counts every GB/s figure divides by (checked against the closed form
B = 2wh + w + 2K + 2h and the Llama-3.1-8B values), the summary writers, and
(GPU) the decoder-launch timing mode at a Qwen3 shape."""
import json

import pytest

from spmv_decode_amd import microbench as MB

LLAMA = dict(dim=4096, inter=14336, qd=4096, kvd=1024, hd=128)


def test_gemv_bytes_closed_form_and_llama_values():
    # w = K/2 at every 50% ratio: index bytes are w whatever M is
    for nnz, m in MB.DEFAULT_RATIOS:
        assert MB.sparse_bytes(4096, 4096, nnz, m) == 16_795_648
        assert MB.sparse_bytes(4096, 1024, nnz, m) == 4_206_592
        assert MB.sparse_bytes(4096, 14336, nnz, m) == 58_759_168
        assert MB.sparse_bytes(14336, 4096, nnz, m) == 58_764_288
    # one decode token's 224 GEMVs at 32:64
    per_layer = sum(MB.sparse_bytes(K, h, 32, 64) for K, h in
                    [(4096, 4096), (4096, 1024), (4096, 1024), (4096, 4096), (4096, 14336), (4096, 14336),
                     (14336, 4096)])
    assert 32 * per_layer == 6_985_187_328
    assert MB.dense_bytes(4096, 4096) == 2 * 4096 * 4096 + 2 * 4096 + 2 * 4096
    # 3:4 keeps 3 of 4: w = 3K/4
    assert MB.sparse_bytes(1024, 384, 3, 4) == 2 * 768 * 384 + 768 + 2 * 1024 + 2 * 384


def test_decode_form_bytes_are_the_gemvs_plus_their_extra_operands():
    g = lambda K, h: MB.sparse_bytes(K, h, 32, 64)  # noqa: E731
    f = lambda cls, **kw: MB.decode_form_bytes(cls, 32, 64, **{**LLAMA, **kw})  # noqa: E731
    # q/k/v: three GEMVs sharing x (x once), the RMSNorm weight, the RoPE row (64 complex64)
    assert f("qkv_decode") == g(4096, 4096) + g(4096, 1024) + g(4096, 1024) - 2 * 2 * 4096 + 2 * 4096 + 8 * 64
    assert f("qkv_decode", qk_norm=True) - f("qkv_decode") == 2 * 2 * 128  # Qwen3's q and k head-norm weights
    assert f("o_resid") == g(4096, 4096) + 2 * 4096  # + the residual read
    # the pair: two weight/index streams, x once, the norm weight, one SiLU*mul output
    assert f("gate_up_pair_norm") == 2 * g(4096, 14336) - 2 * 4096 - 2 * 14336 + 2 * 4096
    assert f("down_resid") == g(14336, 4096) + 2 * 4096
    # split-K carry: the producers read weights, index and input only; the
    # consumers add the residual read and the finished vector's write, so a
    # carried layer moves the plain layer's bytes less o's output write and
    # the pair's read of it (2 x 2 x dim)
    assert f("o_partials") == g(4096, 4096) - 2 * 4096
    assert f("down_partials") == g(14336, 4096) - 2 * 4096
    assert f("gate_up_pair_norm_carried") == f("gate_up_pair_norm") + 2 * 4096
    assert f("qkv_decode_carried") == f("qkv_decode") + 2 * 4096
    plain = sum(f(c) for c in MB.DECODE_CLASSES)
    assert sum(f(c) for c in MB.CARRIED_CLASSES) == plain - 2 * 2 * 4096
    with pytest.raises(ValueError):
        MB.decode_form_bytes("lm_head")


def test_parse_pairs_and_summary_writers(tmp_path):
    assert MB._parse_pairs("4096x4096,1024x4096", "x") == [(4096, 4096), (1024, 4096)]
    assert MB._parse_pairs("2:4,32:64,", ":") == [(2, 4), (32, 64)]
    tok = {"us": 256.0, "bytes": 128_000_000, "GBps": 500.0, "pct_peak": 6.2}
    res = {"32:64": {"classes": {c: {"us": 2.0, "us_sd": 0.1, "bytes": 1_000_000, "GBps": 500.0, "pct_peak": 6.2,
                                     "copies": 3} for c in MB.DECODE_CLASSES + MB.CARRIED_CLASSES},
                     "token": tok, "token_carried": tok}}
    md = tmp_path / "dc.md"
    MB.write_decode_classes_md("qwen3-14b", res, md, "python -u -m spmv_decode_amd.microbench --decode-classes x")
    text = md.read_text()
    assert "--decode-classes x" in text and "+ q/k head norms" in text and "160 launches" in text
    assert text.count("| 32:64 |") == 10 and "token, carried (160 launches)" in text
    rows = [{"config": "auto:th16_u8", "n_in": 4096, "n_out": 4096, "ratio": "32:64", "splits": 8, "us": 7.2,
             "us_sd": 0.05, "GBps": 2333.0, "pct_peak": 29.2, "dense_us": 11.9, "dense_us_sd": 0.1, "dense_form": "mv",
             "dense_GBps": 2800.0, "speedup_vs_dense": 1.65, "max_abs": 1e-3, "rel_l2": 2e-4},
            {**{"config": "th32_u8", "splits": 4}, **{k: 0 for k in ("n_in", "n_out", "us")}}]
    MB.write_sweep_md(rows, tmp_path / "s.md", "cmd")
    text = (tmp_path / "s.md").read_text()
    assert "| 4096 -> 4096 | 32:64 | th16_u8 s8 |" in text and "(mv)" in text
    assert text.count("\n| ") == 2  # the header and the auto: row; other configurations are left out


@pytest.mark.gpu
def test_decode_classes_times_every_launch_at_a_qwen3_shape(gpu, tmp_path):
    """The decoder-launch mode at Qwen3-14B's shapes (q/k head norms in the
    q/k/v launch), one copy of the weights per class: every class runs and
    reports its bytes; the token line sums the classes over the layers."""
    from spmv_decode_amd.decode.model import CONFIGS

    cfg = CONFIGS["qwen3-14b"]
    res = MB.decode_classes("qwen3-14b", [(32, 64)], reps=3, warmup=1, rotate_bytes=0, log=lambda s: None,
                            classes=MB.DECODE_CLASSES + MB.CARRIED_CLASSES)
    r = res["32:64"]
    assert set(r["classes"]) == set(MB.DECODE_CLASSES + MB.CARRIED_CLASSES)
    for c, v in r["classes"].items():
        assert v["us"] > 0 and v["copies"] == 1
        assert v["bytes"] == MB.decode_form_bytes(c, 32, 64, cfg.dim, cfg.inter, cfg.n_heads * cfg.head_dim,
                                                  cfg.n_kv_heads * cfg.head_dim, cfg.head_dim, True)
    for tag, group in (("token", MB.DECODE_CLASSES), ("token_carried", MB.CARRIED_CLASSES)):
        assert r[tag]["bytes"] == cfg.n_layers * sum(r["classes"][c]["bytes"] for c in group)
        assert r[tag]["us"] == pytest.approx(cfg.n_layers * sum(r["classes"][c]["us"] for c in group), rel=1e-3)
    (tmp_path / "r.json").write_text(json.dumps(res))


def test_launch_sweep_takes_the_fused_launches_only():
    with pytest.raises(ValueError, match="fused decoder launch"):
        MB.launch_sweep("o_resid")


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N > 1 exits with a message (one-GPU build) before any GPU work."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=root)
    assert r.returncode == 2 and "one GPU only" in r.stderr and r.stdout == ""
