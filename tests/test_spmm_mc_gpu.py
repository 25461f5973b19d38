"""GPU parity of the matrix-core SpMM (nm_spmm_mc: 9-128 rows per launch,
fp16 / bf16) against the oracle, at the Llama-3.1-8B and Qwen3 shapes, on
ragged shapes (a last chunk shorter than 32 columns, a last tile past h,
positions outside x), every configuration and split count, groups of sibling
products in one launch, strided rows through the C ABI, graph replay and the
automatic routing."""
import numpy as np
import pytest
import torch

from conftest import say
from spmv_decode_amd import _lib, hip_spmv, nmsparse_linear
from test_gemv_gpu import make_case
from test_spmm_gpu import check_rows

pytestmark = pytest.mark.gpu


def mc(X, md, mi, nnz, m, **kw):
    w, h = md.shape
    return hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, nnz, m, matrix_cores=True, **kw)


@pytest.mark.parametrize("batch", [9, 16, 24, 33, 64, 96, 128])
@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096), (4096, 4096), (4096, 1024)], ids=str)
def test_llama_shapes_default_plan(gpu, shape, batch):
    K, h = shape
    _, md, mi = make_case(K, h, 32, 64, seed=K + h + batch)
    X = torch.randn(batch, K, generator=torch.Generator(device="cuda").manual_seed(batch), device="cuda").half()
    say(f"spmm_mc {shape} batch {batch} plan {_lib.spmm_mc_plan(batch, h, md.shape[0], 32, 64)}")
    check_rows(mc(X, md, mi, 32, 64), X, md, mi, 32, 64, f"{shape} b{batch}")


@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120), (5120, 25600), (25600, 5120)], ids=str)
def test_qwen3_shapes(gpu, shape):
    K, h = shape
    _, md, mi = make_case(K, h, 16, 32, seed=K * 3 + h)
    X = torch.randn(40, K, generator=torch.Generator(device="cuda").manual_seed(h), device="cuda").half()
    say(f"spmm_mc qwen3 {shape} plan {_lib.spmm_mc_plan(40, h, md.shape[0], 16, 32)}")
    check_rows(mc(X, md, mi, 16, 32), X, md, mi, 16, 32, f"{shape}")


# (K, h, nnz, m): w = (K/m)*nnz of 8, 9, 500, 1024, 2800 and 6144 columns, h an odd multiple of 128.
RAGGED = [(16, 128, 2, 4), (12, 384, 3, 4), (1000, 384, 4, 8), (4096, 1280, 1, 4), (7168, 2176, 5, 7),
          (24576, 640, 2, 8)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_ragged_shapes_configs_and_splits(gpu, dtype):
    for K, h, nnz, m in RAGGED:
        _, md, mi = make_case(K, h, nnz, m, seed=K + 5 * h, dtype=dtype)
        w = md.shape[0]
        for batch in (3, 9, 17, 40, 64, 100):
            X = torch.randn(batch, K, device="cuda").to(dtype)
            for cfg, splits in ((-1, 0), (0, 1), (1, 3), (2, 2), (2, 0), (0, 64), (3, 0), (3, 1), (4, 3), (4, 64),
                                (5, 2), (5, 0)):
                if batch > 64 and cfg in (2, 5):  # no 128-row tile of 256 columns
                    continue
                p = _lib.spmm_mc_plan(batch, h, w, nnz, m, cfg, splits)
                say(f"spmm_mc {dtype} K{K} h{h} {nnz}:{m} batch {batch} cfg {cfg} splits {splits} -> {p}")
                check_rows(mc(X, md, mi, nnz, m, config_id=cfg, splits=splits), X, md, mi, nnz, m,
                           f"{dtype} {K}x{h} {nnz}:{m} b{batch} cfg{cfg} s{splits}")


# (K, [h...], nnz, m): sibling products of one input (q/k/v, gate/up; ragged widths and groups of 4)
MC_GROUPS = [(4096, [4096, 1024, 1024], 32, 64), (4096, [14336, 14336], 32, 64), (5120, [5120, 1024, 1024], 16, 32),
             (1000, [384, 128, 256, 640], 4, 8), (2048, [1280, 128], 3, 4)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_grouped_products_match_single_launches(gpu, dtype):
    """nm_spmm_mc_group: each product of a group is bit for bit the
    single-product launch with the group's configuration and split count, and
    within the oracle bar, for the default plan and forced ones."""
    for K, hs, nnz, m in MC_GROUPS:
        cases = [make_case(K, h, nnz, m, seed=K + 7 * h + i, dtype=dtype) for i, h in enumerate(hs)]
        w = cases[0][1].shape[0]
        mats = [(md, mi) for _, md, mi in cases]
        for batch in (9, 16, 33, 64, 100):
            X = torch.randn(batch, K, generator=torch.Generator(device="cuda").manual_seed(batch), device="cuda")
            X = X.to(dtype)
            for cfg, splits in ((-1, 0), (0, 2), (4, 0), (5, 3), (3, 1)):
                if batch > 64 and cfg == 5:  # no 128-row tile of 256 columns
                    continue
                p = _lib.spmm_mc_group_plan(batch, hs, w, nnz, m, cfg, splits)
                say(f"spmm_mc group {dtype} K{K} h{hs} {nnz}:{m} batch {batch} cfg {cfg} splits {splits} -> {p}")
                outs = hip_spmv.nmsparse_spmm_group_hip(X, mats, nnz, m, config_id=cfg, splits=splits)
                alone = cfg < 0 and hip_spmv.library_route(batch, K, max(hs))  # each product on the library
                for (md, mi), o in zip(mats, outs):
                    check_rows(o, X, md, mi, nnz, m, f"group {dtype} {K}x{md.shape[1]} b{batch} cfg{cfg}")
                    ref = (hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, md.shape[1], nnz, m) if alone
                           else mc(X, md, mi, nnz, m, config_id=p["config_id"], splits=p["splits"]))
                    assert torch.equal(o, ref)


def test_grouped_products_replay_and_route(gpu):
    """A captured group (split-K arrival counters of every product in one
    workspace) replayed with eager launches between, each replay equal to
    eager; outside 9-128 rows the group helper runs each product through the
    single-product route (the same bits)."""
    K, hs, nnz, m = 4096, [4096, 1024, 1024], 32, 64
    cases = [make_case(K, h, nnz, m, seed=300 + i) for i, h in enumerate(hs)]
    mats = [(md, mi) for _, md, mi in cases]
    X = torch.randn(40, K, device="cuda").half()
    eager = [o.clone() for o in hip_spmv.nmsparse_spmm_group_hip(X, mats, nnz, m, config_id=4, splits=2)]
    outs = [torch.empty_like(o) for o in eager]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        hip_spmv.nmsparse_spmm_group_hip(X, mats, nnz, m, outs=outs, config_id=4, splits=2)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            hip_spmv.nmsparse_spmm_group_hip(X, mats, nnz, m, outs=outs, config_id=4, splits=2)
    torch.cuda.current_stream().wait_stream(s)
    say("spmm_mc group graph replays")
    for rep in range(6):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep
        hip_spmv.nmsparse_spmm_group_hip(X, mats, nnz, m, config_id=4, splits=2)  # eager work between replays
    for rows in (3, 8, 129, 150):
        Xr = torch.randn(rows, K, device="cuda").half()
        say(f"spmm group route {rows} rows")
        for (md, mi), o in zip(mats, hip_spmv.nmsparse_spmm_group_hip(Xr, mats, nnz, m)):
            assert torch.equal(o, hip_spmv.nmsparse_spmm_forward_hip(Xr, md, mi, md.shape[0], md.shape[1], nnz, m))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_silu_product_formed_in_the_gather(gpu, dtype):
    """nm_spmm_mc_silu_mul (the down projection of round(silu(gate) * up),
    the product formed at the gathered positions in fp32): within the oracle
    bar of the product formed in float64 and rounded to the element type (the
    kernel's SiLU, on the hardware's exp2 and reciprocal, is within about an
    ulp of fp32 before that rounding), at the Llama-3.1-8B down shape and a
    ragged one, 9-128 rows, default and forced plans; outside its rows (and
    where the automatic route takes the library) the helper forms the product
    in fp32 with one rounding and takes the single-product route (the same
    bits)."""
    for K, h, nnz, m in ((14336, 4096, 32, 64), (1000, 384, 4, 8)):
        _, md, mi = make_case(K, h, nnz, m, seed=K + 11 * h, dtype=dtype)
        w = md.shape[0]
        for rows in (9, 40, 100, 128):
            g = torch.Generator(device="cuda").manual_seed(rows)
            gate = torch.randn(rows, K, generator=g, device="cuda").to(dtype)
            up = torch.randn(rows, K, generator=g, device="cuda").to(dtype)
            act = (torch.nn.functional.silu(gate.double()) * up.double()).to(dtype)
            act32 = (torch.nn.functional.silu(gate.float()) * up.float()).to(dtype)
            for cfg, splits in ((-1, 0), (3, 2), (0, 1)):
                say(f"spmm silu product {dtype} K{K} h{h} {nnz}:{m} rows {rows} cfg {cfg} splits {splits}")
                out = hip_spmv.nmsparse_spmm_silu_mul_hip(gate, up, md, mi, w, h, nnz, m, config_id=cfg,
                                                          splits=splits)
                if cfg < 0 and hip_spmv.library_route(rows, K, h):  # the product in fp32, then the library
                    assert torch.equal(out, hip_spmv.nmsparse_spmm_forward_hip(act32, md, mi, w, h, nnz, m))
                    continue
                check_rows(out, act, md, mi, nnz, m, f"silu product {dtype} {K}x{h} rows {rows} cfg {cfg}")
        for rows in (4, 200):
            gate = torch.randn(rows, K, device="cuda").to(dtype)
            up = torch.randn(rows, K, device="cuda").to(dtype)
            act = (torch.nn.functional.silu(gate.float()) * up.float()).to(dtype)
            assert torch.equal(hip_spmv.nmsparse_spmm_silu_mul_hip(gate, up, md, mi, w, h, nnz, m),
                               hip_spmv.nmsparse_spmm_forward_hip(act, md, mi, w, h, nnz, m))


def test_more_than_128_rows_and_determinism(gpu):
    K, h = 4096, 4096
    _, md, mi = make_case(K, h, 32, 64, seed=77)
    X = torch.randn(150, K, device="cuda").half()
    say("spmm_mc 150 rows")
    y = mc(X, md, mi, 32, 64)
    check_rows(y, X, md, mi, 32, 64, "150 rows")
    for _ in range(3):
        assert torch.equal(mc(X, md, mi, 32, 64), y)
    # the first 128 rows are one launch of their own: the same bits alone
    assert torch.equal(mc(X[:128].contiguous(), md, mi, 32, 64), y[:128])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_past_the_matrix_core_rows_gather_and_library_gemm(gpu, dtype):
    """Past NM_MC_MAX_BATCH rows (past 64 for products of at most 1024
    outputs) the automatic route gathers the activations (nm_gather_columns)
    and multiplies them with mat_data in one hipBLASLt GEMM: the oracle bar at
    Llama-3.1-8B shapes and a ragged one, and the gather alone bit-exact
    against a PyTorch index_select."""
    for K, h, nnz, m, rows in ((4096, 14336, 32, 64, 160), (14336, 4096, 32, 64, 200), (4096, 1024, 32, 64, 96),
                               (1000, 384, 4, 8, 200)):
        _, md, mi = make_case(K, h, nnz, m, seed=K + rows, dtype=dtype)
        w = md.shape[0]
        X = torch.randn(rows, K, device="cuda").to(dtype)
        say(f"spmm gather + library gemm {dtype} K{K} h{h} {nnz}:{m} rows {rows}")
        check_rows(hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, nnz, m), X, md, mi, nnz, m,
                   f"{dtype} {K}x{h} rows {rows}")
        wp = (w + 7) // 8 * 8
        xg = torch.full((rows, wp + 8), 3.0, device="cuda").to(dtype)
        rc = _lib.load().nm_gather_columns(0 if dtype == torch.float16 else 1, X.data_ptr(), K, rows, mi.data_ptr(),
                                           w, nnz, m, xg.data_ptr(), wp + 8, torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "nm_gather_columns")
        pos = (torch.arange(w, device="cuda") // nnz) * m + mi.reshape(-1).long()
        assert torch.equal(xg[:, :w], X.index_select(1, pos))
        assert bool((xg[:, w:] == 0).all())


def test_automatic_route_keeps_the_matrix_cores_up_to_128_rows(gpu):
    """hip_spmv.library_route: up to 64 rows every shape, and up to 128 rows
    every shape of more than 1024 outputs, runs on the matrix-core kernel (the
    same bits as forcing it); past that the activations are gathered and
    multiplied on hipBLASLt (the same bits as the explicit gather + GEMM).
    Both within the oracle bar."""
    for K, h, rows, routed in ((4096, 14336, 32, False), (4096, 14336, 64, False), (5120, 17408, 40, False),
                               (4096, 4096, 32, False), (14336, 4096, 64, False), (4096, 14336, 65, False),
                               (14336, 4096, 128, False), (4096, 1024, 64, False), (4096, 1024, 65, True),
                               (4096, 14336, 129, True)):
        assert hip_spmv.library_route(rows, K, h) == routed, (K, h, rows)
        _, md, mi = make_case(K, h, 32, 64, seed=K + h + rows)
        w = md.shape[0]
        X = torch.randn(rows, K, generator=torch.Generator(device="cuda").manual_seed(rows), device="cuda").half()
        say(f"spmm auto route K{K} h{h} rows {rows} library {routed}")
        auto = hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, 32, 64)
        if routed:
            wp = (w + 7) // 8 * 8
            xg = torch.empty(rows, wp, dtype=X.dtype, device="cuda")
            _lib.check(_lib.load().nm_gather_columns(0, X.data_ptr(), K, rows, mi.data_ptr(), w, 32, 64, xg.data_ptr(),
                                                     wp, torch.cuda.current_stream().cuda_stream), "nm_gather_columns")
            assert torch.equal(auto, torch.matmul(xg[:, :w], md))
        else:
            assert torch.equal(auto, mc(X, md, mi, 32, 64))
        check_rows(auto, X, md, mi, 32, 64, f"auto K{K} h{h} rows {rows}")


def test_c_abi_row_strides(gpu):
    """x and out with padded rows through the C ABI directly."""
    K, h, nnz, m, B = 4096, 4096, 32, 64, 20
    _, md, mi = make_case(K, h, nnz, m, seed=6)
    xs, os_ = K + 64, h + 128
    Xp = torch.randn(B, xs, device="cuda").half()
    outp = torch.full((B, os_), 7.0, device="cuda").half()
    lib = _lib.load()
    need = lib.nm_spmm_mc_workspace_bytes(B, h, md.shape[0], nnz, m, -1, 0)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    say("spmm_mc strided rows")
    rc = lib.nm_spmm_mc(0, Xp.data_ptr(), xs, B, md.data_ptr(), mi.data_ptr(), outp.data_ptr(), os_, ws.data_ptr(),
                        need, h, md.shape[0], nnz, m, -1, 0, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "nm_spmm_mc")
    torch.cuda.synchronize()
    check_rows(outp[:, :h].contiguous(), Xp[:, :K].contiguous(), md, mi, nnz, m, "strided")
    assert bool((outp[:, h:] == 7.0).all())  # padding untouched
    with pytest.raises(_lib.NmSparseLibraryError):  # fp32 has no matrix-core path
        _lib.check(lib.nm_spmm_mc(2, Xp.data_ptr(), xs, B, md.data_ptr(), mi.data_ptr(), outp.data_ptr(), os_,
                                  ws.data_ptr(), need, h, md.shape[0], nnz, m, -1, 0, 0), "nm_spmm_mc")


def test_auto_routing_and_module(gpu):
    K, h = 2048, 1024
    _, md, mi = make_case(K, h, 16, 32, seed=9)
    w = md.shape[0]
    X = torch.randn(12, K, device="cuda").half()
    auto = hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, 16, 32)
    assert torch.equal(auto, mc(X, md, mi, 16, 32))  # > 8 rows of fp16: the matrix cores
    valu = hip_spmv.nmsparse_spmm_forward_hip(X, md, mi, w, h, 16, 32, matrix_cores=False)
    check_rows(valu, X, md, mi, 16, 32, "valu 12 rows")
    lin = nmsparse_linear.NmSparseLinear(1024, 2048, 16, 3, "cuda", init="device")
    x = torch.randn(2, 30, 2048, device="cuda").half()
    say("module 60 rows")
    y = lin(x)
    check_rows(y.reshape(-1, 1024), x.reshape(-1, 2048), lin.mat_data, lin.mat_index, 8, 16, "module 60 rows")
    with pytest.raises(TypeError):
        mc(X.float(), md.float(), mi, 16, 32)


def test_graph_capture_replays(gpu):
    K, h, nnz, m = 4096, 14336, 32, 64
    _, md, mi = make_case(K, h, nnz, m, seed=10)
    X = torch.randn(48, K, device="cuda").half()
    eager = mc(X, md, mi, nnz, m)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        mc(X, md, mi, nnz, m, out=out)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            mc(X, md, mi, nnz, m, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = mc(X, md, mi, nnz, m)  # eager work between replays


def test_split_k_handoff_soak_500_replays(gpu):
    """The matrix-core SpMM's split-K handoff (agent-scope atomic-store
    publish, ticket, ordered partial reads) under repetition: gate/up, down
    and q/o at the Llama-3.1-8B shapes with 48 rows (2-4 splits, 224-256
    workgroups), a grouped q/k/v launch (3 products' counters in one
    workspace, 2 splits) and down at 128 rows (4 splits) in one hipGraph,
    replayed 500 times, every replay bitwise equal to the first, stopping at
    the first mismatch."""
    cases = []
    # (K, h, config, splits, rows): gate/up on the 128-column DMA tiles with 2 splits (its default plan at 48
    # rows has none), down and q/o on their default plans (4 splits each)
    for i, (K, h, cfg, splits, rows) in enumerate(((4096, 14336, 4, 2, 48), (14336, 4096, -1, 0, 48),
                                                   (4096, 4096, -1, 0, 48), (14336, 4096, -1, 0, 128))):
        _, md, mi = make_case(K, h, 32, 64, seed=90 + i)
        X = torch.randn(rows, K, device="cuda").half()
        p = _lib.spmm_mc_plan(rows, h, md.shape[0], 32, 64, cfg, splits)
        assert p["splits"] > 1, p
        cases.append((X, md, mi, torch.empty(rows, h, dtype=torch.float16, device="cuda"), cfg, splits))
    qkv = [make_case(4096, h, 32, 64, seed=95 + i)[1:] for i, h in enumerate((4096, 1024, 1024))]
    Xq = torch.randn(48, 4096, device="cuda").half()
    assert _lib.spmm_mc_group_plan(48, [4096, 1024, 1024], 2048, 32, 64, 3, 2)["splits"] == 2
    qkv_outs = [torch.empty(48, md.shape[1], dtype=torch.float16, device="cuda") for md, _ in qkv]

    def launches():
        for X, md, mi, out, cfg, splits in cases:
            mc(X, md, mi, 32, 64, out=out, config_id=cfg, splits=splits)
        hip_spmv.nmsparse_spmm_group_hip(Xq, qkv, 32, 64, outs=qkv_outs, config_id=3, splits=2)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launches()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            launches()
    torch.cuda.current_stream().wait_stream(s)
    g.replay()
    torch.cuda.synchronize()
    first = [c[3].clone() for c in cases]
    first_qkv = [o.clone() for o in qkv_outs]
    check_rows(first[0], cases[0][0], cases[0][1], cases[0][2], 32, 64, "soak gate/up")
    check_rows(first[3], cases[3][0], cases[3][1], cases[3][2], 32, 64, "soak down 128 rows")
    for (md, mi), o in zip(qkv, first_qkv):
        check_rows(o, Xq, md, mi, 32, 64, "soak grouped q/k/v")
    for rep in range(1, 500):
        g.replay()
        torch.cuda.synchronize()
        for k, c in enumerate(cases):
            if not torch.equal(c[3], first[k]):
                pytest.fail(f"replay {rep}: case {k} differs from the first replay")
        for k, o in enumerate(qkv_outs):
            if not torch.equal(o, first_qkv[k]):
                pytest.fail(f"replay {rep}: grouped product {k} differs from the first replay")
