"""GPU parity of the small-batch SpMM (batch > 1, f4) against the oracle and
against the batch-1 GEMV, which it reproduces bit for bit under the same
split plan."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import say
from oracle import nm_oracle as O
from spmv_decode_amd import _lib, hip_spmv, nmsparse_linear
from test_gemv_gpu import MIN_NORMAL_EXP, ULP_BITS, make_case, run

pytestmark = pytest.mark.gpu


def spmm(X, md, mi, nnz, m, **kw):
    w, h = md.shape
    return hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, nnz, m, **kw)


def check_rows(out, X, md, mi, nnz, m, tag):
    ref = O.spmm_f64(X.cpu(), md.cpu(), mi.cpu(), nnz, m)
    got = out.float().cpu().numpy().reshape(ref.shape)
    assert np.isfinite(got).all(), tag
    xg = np.abs(O.to_f64(X.cpu()).reshape(ref.shape[0], -1)[:, O.gather_positions(mi.cpu(), nnz, m)
                                                              .clip(max=X.shape[-1] - 1)])
    acc = 4.0 * np.sqrt(md.shape[0]) * 2.0 ** -24 * (xg @ np.abs(O.to_f64(md.cpu())))
    if out.dtype == torch.float32:
        bad = np.abs(got - ref) > acc + 1e-30
    else:
        exp = np.maximum(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))), MIN_NORMAL_EXP[out.dtype])
        bad = np.abs(got - ref) > np.exp2(exp - ULP_BITS[out.dtype]) + acc
        if out.dtype == torch.float16:
            e = O.error_metrics(ref, got)
            assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, (tag, e)
    assert not bad.any(), (tag, int(bad.sum()), float(np.abs(got - ref)[bad].max()))


@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 14336), (4096, 1024)], ids=str)
def test_rows_are_bitwise_the_gemv_of_each_row(gpu, shape):
    K, h = shape
    _, md, mi = make_case(K, h, 32, 64, seed=K + h)
    g = torch.Generator(device="cuda").manual_seed(h)
    X = torch.randn(11, K, generator=g, device="cuda").half()
    for cfg in (-1, 0, 1, 2, 3):
        for splits in (0, 1, 3):
            gcfg = cfg if cfg >= 0 else _lib.spmm_plan(8, h, md.shape[0], 32, 64, -1, splits)["config_id"]
            if _lib.plan(h, md.shape[0], 32, 64, gcfg, splits)["rows_per_split"] != \
                    _lib.spmm_plan(8, h, md.shape[0], 32, 64, gcfg, splits)["rows_per_split"]:
                continue
            say(f"spmm vs gemv {shape} cfg {cfg} splits {splits}")
            out = spmm(X, md, mi, 32, 64, config_id=gcfg, splits=splits)
            for b in range(X.shape[0]):
                ref = run(X[b:b + 1], md, mi, 32, 64, config_id=gcfg, splits=splits)
                assert torch.equal(out[b:b + 1], ref), (cfg, splits, b)
    check_rows(out, X, md, mi, 32, 64, f"{shape}")


@pytest.mark.parametrize("batch", [2, 4, 8])
@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120), (5120, 8192), (25600, 5120)], ids=str)
def test_default_plans_at_qwen3_shapes(gpu, shape, batch):
    """The SpMM's default plans (its tile rule for wide and short-column
    launches, the GEMV's split rule) at Qwen3-14B / Qwen3-32B shapes, every row
    against the oracle."""
    K, h = shape
    _, md, mi = make_case(K, h, 16, 32, seed=K * 7 + h)
    X = torch.randn(batch, K, generator=torch.Generator(device="cuda").manual_seed(batch), device="cuda").half()
    say(f"spmm qwen3 {shape} batch {batch} plan {_lib.spmm_plan(batch, h, md.shape[0], 16, 32, -1, 0)}")
    check_rows(spmm(X, md, mi, 16, 32), X, md, mi, 16, 32, f"{shape} b{batch}")


RAGGED = [(16, 128, 2, 4), (12, 384, 3, 4), (2000, 1152, 8, 16), (4096, 1280, 1, 4), (1024, 640, 128, 256),
          (7168, 2176, 5, 7)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
def test_ragged_shapes_batches_and_dtypes(gpu, dtype):
    for K, h, nnz, m in RAGGED:
        _, md, mi = make_case(K, h, nnz, m, seed=K + 3 * h, dtype=dtype)
        for batch in (2, 3, 5, 8, 13):
            X = torch.randn(batch, K, device="cuda").to(dtype)
            for cfg, splits in ((-1, 0), (0, 1), (3, 3)):
                say(f"spmm {dtype} K{K} h{h} {nnz}:{m} batch {batch} cfg {cfg} splits {splits}")
                check_rows(spmm(X, md, mi, nnz, m, config_id=cfg, splits=splits), X, md, mi, nnz, m,
                           f"{dtype} {K}x{h} {nnz}:{m} b{batch} cfg{cfg} s{splits}")


def test_c_abi_row_strides(gpu):
    """x and out with padded rows through the C ABI directly."""
    K, h, nnz, m, B = 4096, 4096, 32, 64, 6
    _, md, mi = make_case(K, h, nnz, m, seed=5)
    xs, os_ = K + 64, h + 128
    Xp = torch.randn(B, xs, device="cuda").half()
    outp = torch.full((B, os_), 7.0, device="cuda").half()
    lib = _lib.load()
    need = lib.nm_spmm_workspace_bytes(B, h, md.shape[0], nnz, m, -1, 0)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    say("spmm strided rows")
    rc = lib.nm_spmm(0, Xp.data_ptr(), xs, B, md.data_ptr(), mi.data_ptr(), outp.data_ptr(), os_, ws.data_ptr(),
                     need, h, md.shape[0], nnz, m, -1, 0, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "nm_spmm")
    torch.cuda.synchronize()
    check_rows(outp[:, :h].contiguous(), Xp[:, :K].contiguous(), md, mi, nnz, m, "strided")
    assert bool((outp[:, h:] == 7.0).all())  # padding untouched


def test_module_and_op_batch_rows(gpu):
    lin = nmsparse_linear.NmSparseLinear(1024, 2048, 16, 3, "cuda", init="device")
    for shape in ((5, 2048), (3, 1, 2048), (2, 4, 2048), (1, 20, 2048)):
        say(f"module batch {shape}")
        x = torch.randn(*shape, device="cuda").half()
        y = lin(x)
        assert y.shape == (*shape[:-1], 1024) and y.dtype == x.dtype
        check_rows(y.reshape(-1, 1024), x.reshape(-1, 2048), lin.mat_data, lin.mat_index, 8, 16, str(shape))
    x = torch.randn(3, 2048, device="cuda")  # fp32 input: cast to fp16 and back, as gemv
    y = torch.ops.nmsparse.spmm(x, lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width, lin.vec_width)
    assert y.dtype == torch.float32 and y.shape == (3, 1024)
    ref = torch.ops.nmsparse.spmm(x.half(), lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width,
                                  lin.vec_width)
    assert torch.equal(y, ref.float())


def test_graph_capture_replays(gpu):
    K, h, nnz, m = 4096, 14336, 32, 64
    _, md, mi = make_case(K, h, nnz, m, seed=8)
    X = torch.randn(8, K, device="cuda").half()
    eager = spmm(X, md, mi, nnz, m)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        spmm(X, md, mi, nnz, m, out=out)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            spmm(X, md, mi, nnz, m, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = spmm(X, md, mi, nnz, m)  # eager work between replays


def test_split_k_handoff_soak_1000_replays(gpu):
    """The SpMM publishes its partials with agent-scope atomic stores (the GEMV
    with atomic swaps) and orders them by hardware completion (vmcnt wait, a
    returning agent-scope ticket add, agent-scope loads after it). A rare
    visibility miss would show as a wrong sum, not a fault, so: batch 8 gate
    (448 workgroups), batch 8 down (256) and batch 4 q/o at the Llama-3.1-8B
    shapes (8 splits each) in one hipGraph, replayed 1000 times; every replay
    bitwise equal to the per-row GEMV (swap handoff) of the same plan, checked
    after each replay, stopping at the first mismatch."""
    cases = []
    for i, (K, h, batch) in enumerate(((4096, 14336, 8), (14336, 4096, 8), (4096, 4096, 4))):
        _, md, mi = make_case(K, h, 32, 64, seed=40 + i)
        X = torch.randn(batch, K, device="cuda").half()
        p = _lib.spmm_plan(batch, h, md.shape[0], 32, 64)
        assert p["splits"] == 8, p
        ref = torch.cat([run(X[b:b + 1], md, mi, 32, 64, config_id=p["config_id"], splits=p["splits"])
                         for b in range(batch)])
        cases.append((X, md, mi, torch.empty(batch, h, dtype=torch.float16, device="cuda"), ref))

    def launches():
        for X, md, mi, out, _ in cases:
            spmm(X, md, mi, 32, 64, out=out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launches()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            launches()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(1000):
        g.replay()
        torch.cuda.synchronize()
        for k, (_, _, _, out, ref) in enumerate(cases):
            if not torch.equal(out, ref.view(out.shape)):
                pytest.fail(f"replay {rep}: case {k} differs from the per-row GEMV")
