"""GPU parity of the HIP N:M GEMV against the CPU oracle.

Bar (north star): fp16 outputs within max-abs 1e-2 and rel-L2 1e-3 of the
fp32-accumulated reference value on the benchmark distributions (weights
N(0, 0.02), activations N(0, 1)); additionally every output must be within
one unit in the last place of its dtype from the float64 value (the kernel
rounds an fp32 sum once), fp32 outputs within 1e-5 relative of the row scale.
Integer/index properties (one-hot rows, zero vectors, power-of-two scaling,
determinism, graph replay) are checked bit-exactly.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import say
from oracle import nm_oracle as O
from spmv_decode_amd import _lib, hip_spmv, nmsparse_linear

pytestmark = pytest.mark.gpu

RATIOS = [(2, 4), (4, 8), (8, 16), (16, 32), (32, 64), (64, 128), (128, 256)]
LLAMA_SHAPES = {"q_o": (4096, 4096), "k_v": (4096, 1024), "gate_up": (4096, 14336), "down": (14336, 4096)}
ULP_BITS = {torch.float16: 10, torch.bfloat16: 7}
MIN_NORMAL_EXP = {torch.float16: -14, torch.bfloat16: -126}


def make_case(K, h, nnz, m, seed, dtype=torch.float16, wstd=0.02, device="cuda"):
    """Seeded packed case generated on the GPU; returns device tensors."""
    g = torch.Generator(device=device).manual_seed(seed)
    banks = K // m
    keys = torch.rand(banks, m, generator=g, device=device)
    mi = keys.argsort(dim=1)[:, :nnz].sort(dim=1).values.to(torch.uint8).contiguous()
    md = (torch.randn(banks * nnz, h, generator=g, device=device) * wstd).to(dtype)
    x = torch.randn(1, K, generator=g, device=device).to(dtype)
    return x, md, mi


def run(x, md, mi, nnz, m, **kw):
    w, h = md.shape
    return hip_spmv.nmsparse_spmv_forward_hip(x, md, mi, w, h, nnz, 128, m, 1, x.shape[1], **kw)


def check_parity(out, x, md, mi, nnz, m, tag=""):
    ref = O.gemv_f64(x.cpu(), md.cpu(), mi.cpu(), nnz, m)
    got = out.detach().float().cpu().numpy().reshape(-1)
    assert np.isfinite(got).all(), tag
    # fp32 accumulation error bound of a sum of w products (each within one
    # fp32 rounding): 4*sqrt(w)*eps32*sum|terms|, a probabilistic bound that
    # a wrong term or index exceeds by orders of magnitude.
    w = md.shape[0]
    abs_terms = O.to_f64(md.cpu()).__abs__().T @ np.abs(O.gather_activations(x.cpu(), mi.cpu(), nnz, m))
    acc_tol = 4.0 * np.sqrt(w) * 2.0 ** -24 * abs_terms
    dtype = out.dtype
    if dtype == torch.float32:
        bad = np.abs(got - ref) > acc_tol + 1e-30
        assert not bad.any(), (tag, int(bad.sum()))
        return
    e = O.error_metrics(ref, got)
    if dtype == torch.float16:
        assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, (tag, e)
    # one ulp of the output type around the float64 value, plus accumulation
    exp = np.floor(np.log2(np.maximum(np.abs(ref), 1e-30)))
    exp = np.maximum(exp, MIN_NORMAL_EXP[dtype])
    ulp = np.exp2(exp - ULP_BITS[dtype])
    bad = np.abs(got - ref) > ulp + acc_tol
    assert not bad.any(), (tag, int(bad.sum()), float(np.abs(got - ref)[bad].max()))


def test_config1_qwen06b_up_proj(gpu):
    """The Qwen3-0.6B up-projection case: dense W [3072, 1024] ~ N(0, 0.02), 2:4 pattern from the
    reference's index sequence, packed; x ~ N(0, 1); checked against the fp32
    dense matvec on the masked weight (the reference's own oracle)."""
    say("config1 3072<-1024 2:4")
    gen = torch.Generator().manual_seed(0)
    W = (torch.randn(3072, 1024, generator=gen) * 0.02).to(torch.float16)
    _, mi, _, nnz = nmsparse_linear._make_sparse(1024, 3072, 4, 0, "cpu")
    md = nmsparse_linear.pack_dense(W, mi, 4)
    x = torch.randn(1, 1024, generator=torch.Generator().manual_seed(1)).to(torch.float16)
    out = run(x.to(gpu), md.to(gpu), mi.to(gpu), nnz, 4)
    assert out.shape == (1, 3072) and out.dtype == torch.float16
    mask = torch.from_numpy(O.mask_from_index(mi, nnz, 4, 1024))
    dense_ref = torch.mv((W * mask).float(), x.float().reshape(-1))
    e = O.error_metrics(dense_ref, out.cpu())
    assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, e
    check_parity(out, x, md, mi, nnz, 4, "config1")


@pytest.mark.parametrize("nnz,m", RATIOS, ids=lambda v: str(v))
@pytest.mark.parametrize("shape", sorted(LLAMA_SHAPES))
def test_llama_shapes_all_ratios(gpu, shape, nnz, m):
    K, h = LLAMA_SHAPES[shape]
    say(f"llama {shape} {nnz}:{m}")
    x, md, mi = make_case(K, h, nnz, m, seed=K + h + m)
    check_parity(run(x, md, mi, nnz, m), x, md, mi, nnz, m, f"{shape} {nnz}:{m}")


QWEN3_SHAPES = {  # (K, h) of the Qwen3-14B and Qwen3-32B Linears, at their benchmark ratios
    "14b_q_o": (5120, 5120, 32, 64), "14b_k_v": (5120, 1024, 8, 16), "14b_gate_up": (5120, 17408, 32, 64),
    "14b_down": (17408, 5120, 128, 256), "32b_q": (5120, 8192, 16, 32), "32b_o": (8192, 5120, 16, 32),
    "32b_gate_up": (5120, 25600, 16, 32), "32b_down": (25600, 5120, 16, 32)}


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
def test_qwen3_shapes_default_plans(gpu, shape):
    """The library's default plans at the Qwen3 shapes (the split rule's
    long-column and round-filling cases, up to 12 splits): GEMV parity, and
    for the gate/up widths the pair launch with SiLU*mul (pair tiles of 512
    past 14336 outputs) against the oracle."""
    from spmv_decode_amd.hip_spmv import nmsparse_gate_up_silu

    K, h, nnz, m = QWEN3_SHAPES[shape]
    say(f"qwen3 {shape} {K}->{h} {nnz}:{m} plan {_lib.plan(h, K // m * nnz, nnz, m)}")
    x, md, mi = make_case(K, h, nnz, m, seed=K * 3 + h)
    check_parity(run(x, md, mi, nnz, m), x, md, mi, nnz, m, shape)
    if shape.endswith("gate_up"):
        _, ud, ui = make_case(K, h, nnz, m, seed=K * 3 + h + 1)
        ref = _silu_ref(x, md, mi, ud, ui, nnz, m)
        got = nmsparse_gate_up_silu(x, (md, mi), (ud, ui), nnz, m).float().cpu().numpy().reshape(-1)
        e = O.error_metrics(ref, got)
        assert np.isfinite(got).all() and e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, e


RAGGED = [  # (K, h, nnz, m): tails in both directions, odd N, tiny and wide
    (16, 128, 2, 4), (12, 384, 3, 4), (2000, 1152, 8, 16), (4096, 1280, 1, 4), (1024, 640, 128, 256),
    (8, 128, 1, 8), (7168, 2176, 5, 7)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
def test_every_config_dtype_and_ragged_shape(gpu, dtype):
    n = _lib.num_configs()
    for K, h, nnz, m in RAGGED:
        x, md, mi = make_case(K, h, nnz, m, seed=K * 7 + h, dtype=dtype)
        for cfg in range(n):
            for splits in (0, 1, 3):
                say(f"cfg {cfg} splits {splits} {dtype} K{K} h{h} {nnz}:{m}")
                check_parity(run(x, md, mi, nnz, m, config_id=cfg, splits=splits), x, md, mi, nnz, m,
                             f"cfg{cfg} s{splits} {dtype} {K}x{h} {nnz}:{m}")


@pytest.mark.parametrize("nnz,m", [(2, 4), (32, 64), (128, 256)])
def test_one_hot_rows_and_zero_vector_exact(gpu, nnz, m):
    K, h = 4096, 4096
    say(f"one-hot {nnz}:{m}")
    _, md, mi = make_case(K, h, nnz, m, seed=3)
    pos = O.gather_positions(mi.cpu(), nnz, m)
    w = md.shape[0]
    for c in (0, 1, w // 2 + 1, w - 1):
        x = torch.zeros(1, K, dtype=torch.float16, device=gpu)
        x[0, int(pos[c])] = 1.0
        out = run(x, md, mi, nnz, m)
        assert torch.equal(out[0], md[c]), c
    kept = set(pos.tolist())
    pruned = next(k for k in range(K) if k not in kept)
    x = torch.zeros(1, K, dtype=torch.float16, device=gpu)
    x[0, pruned] = 7.0
    assert not run(x, md, mi, nnz, m).any()
    assert not run(torch.zeros(1, K, dtype=torch.float16, device=gpu), md, mi, nnz, m).any()


def test_power_of_two_scaling_and_determinism_full_size(gpu):
    for K, h in LLAMA_SHAPES.values():
        say(f"scaling/determinism {K}x{h}")
        x, md, mi = make_case(K, h, 32, 64, seed=h)
        y = run(x, md, mi, 32, 64)
        for _ in range(4):
            assert torch.equal(run(x, md, mi, 32, 64), y)
        # Doubling x doubles every fp32 term and sum exactly; rounding to fp16
        # commutes with doubling except in the subnormal range (|y| < 2^-14),
        # where the two can differ by one subnormal step (2^-24).
        y2 = run(x * 2, md, mi, 32, 64).float()
        ref2 = y.float() * 2
        normal = y.float().abs() >= 2.0 ** -14
        assert torch.equal(y2[normal], ref2[normal])
        assert (y2[~normal] - ref2[~normal]).abs().max().item() <= 2.0 ** -24 if (~normal).any() else True


def test_tickets_rearm_and_workspace_reuse(gpu):
    for K, h in LLAMA_SHAPES.values():
        x, md, mi = make_case(K, h, 32, 64, seed=1)
        run(x, md, mi, 32, 64)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    ws = hip_spmv._workspaces[(gpu.index or 0, stream)]
    assert not ws[: _lib.NM_TICKET_BYTES].any()


def test_graph_capture_replays_match_eager(gpu):
    cases = [make_case(K, h, nnz, m, seed=i) + (nnz, m)
             for i, ((K, h), (nnz, m)) in enumerate(zip(list(LLAMA_SHAPES.values()) * 2, RATIOS))]
    eager = [run(x, md, mi, nnz, m).clone() for x, md, mi, nnz, m in cases]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm the capture stream's workspace
        for x, md, mi, nnz, m in cases:
            run(x, md, mi, nnz, m)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        outs = [run(x, md, mi, nnz, m) for x, md, mi, nnz, m in cases]
    for rep in range(4):
        say(f"graph replay {rep}")
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep
        # eager work between replays, on the default stream's own workspace
        x, md, mi, nnz, m = cases[rep]
        assert torch.equal(run(x, md, mi, nnz, m), eager[rep])
        torch.cuda.synchronize()


def test_capture_without_warmup_owns_its_workspace(gpu):
    """A capture on a stream that never ran a GEMV gets a workspace of its own
    (allocated in the capture, counters cleared by a fill node): two such graphs
    on one stream, replayed in turn with eager GEMVs between, each match eager,
    and neither borrows the default stream's workspace."""
    cases = [make_case(K, h, 32, 64, seed=20 + i) for i, (K, h) in enumerate(LLAMA_SHAPES.values())]
    eager = [run(x, md, mi, 32, 64).clone() for x, md, mi in cases]
    torch.cuda.synchronize()
    default_ws = hip_spmv._workspaces[(gpu.index or 0, torch.cuda.current_stream().cuda_stream)]
    # torch hands out streams from a small per-device pool, so an earlier test
    # may already have run GEMVs on the next one: take one that never has.
    for _ in range(64):
        s = torch.cuda.Stream()
        if (gpu.index or 0, s.cuda_stream) not in hip_spmv._workspaces:
            break
    else:
        pytest.skip("every pooled stream has already run a GEMV in this process")
    s.wait_stream(torch.cuda.current_stream())
    graphs, outs = [], []
    for half in (cases[:2], cases[2:]):
        g = torch.cuda.CUDAGraph()
        with pytest.warns(RuntimeWarning, match="warmed-up workspace"):
            with torch.cuda.graph(g, stream=s):
                outs.append([run(x, md, mi, 32, 64) for x, md, mi in half])
        graphs.append(g)
    assert (gpu.index or 0, s.cuda_stream) not in hip_spmv._workspaces
    ref = [eager[:2], eager[2:]]
    for rep in range(3):
        for gi, (g, o, e) in enumerate(zip(graphs, outs, ref)):
            say(f"no-warm-up graph {gi} replay {rep}")
            for t in o:
                t.zero_()
            g.replay()
            torch.cuda.synchronize()
            for t, u in zip(o, e):
                assert torch.equal(t, u), (rep, gi)
            x, md, mi = cases[rep]
            assert torch.equal(run(x, md, mi, 32, 64), eager[rep])
            torch.cuda.synchronize()
    assert not hip_spmv._capture_workspaces  # released to the graphs' pools after the captures
    assert not default_ws[: _lib.NM_TICKET_BYTES].any()


def test_capture_id_through_the_library(gpu):
    """hip_spmv.capture_id asks the library's own HIP runtime (nm_stream_capture_id):
    0 outside a capture, the same non-zero id throughout one capture, a new id for
    the next capture on the same stream."""
    s = torch.cuda.Stream()
    assert hip_spmv.capture_id(s.cuda_stream) == 0
    ids = []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        x = torch.zeros(16, device=gpu)
        with torch.cuda.graph(g, stream=s):
            first = hip_spmv.capture_id(s.cuda_stream)
            x.add_(1.0)
            assert hip_spmv.capture_id(s.cuda_stream) == first
        ids.append(first)
        g.replay()
        torch.cuda.synchronize()
        assert bool((x == 1.0).all())
        del g
    assert ids[0] != 0 and ids[1] != 0 and ids[0] != ids[1], ids
    assert hip_spmv.capture_id(s.cuda_stream) == 0


@pytest.mark.parametrize("m", [4, 64, 256])
def test_fused_wqkv_width_default_plan(gpu, m):
    """gpt-fast fuses q/k/v into one 4096 -> 6144 Linear (model.py:196-198, 219), which
    the reference's swap turns into one NmSparseLinear; its default plan (256-row tiles
    past 4096 outputs) against the oracle, through the module and the op."""
    lin = nmsparse_linear.NmSparseLinear(6144, 4096, m, 11, "cuda")
    say(f"wqkv 4096->6144 {m // 2}:{m} plan {_lib.plan(6144, lin.w, m // 2, m)}")
    x = torch.randn(1, 1, 4096, generator=torch.Generator(device="cuda").manual_seed(m), device=gpu).half()
    y = lin(x)
    assert y.shape == (1, 1, 6144)
    check_parity(y.reshape(1, -1), x.reshape(1, -1), lin.mat_data, lin.mat_index, m // 2, m, f"wqkv {m}")


def test_make_sparse_digests_on_this_box(gpu):
    """The synthetic weights NmSparseLinear draws on this machine are the reference's
    own (fixtures written by importing src/spmv/nmsparse_linear.py): every digest case,
    computed with this box's torch, whose version is printed."""
    import hashlib
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).parent / "golden" / "make_sparse.json").read_text())
    say(f"torch {torch.__version__} on this box; fixtures written with torch {fx['meta']['torch']}")
    for case in fx["digests"]:
        md, mi, w, nnz = nmsparse_linear._make_sparse(case["K"], case["N"], case["M"], case["seed"], "cpu")
        tag = (case["K"], case["N"], case["M"], case["seed"])
        assert (w, nnz) == (case["w"], case["nnz"]), tag
        assert hashlib.sha256(md.view(torch.int16).numpy().tobytes()).hexdigest() == case["mat_data_sha256"], tag
        assert hashlib.sha256(mi.numpy().tobytes()).hexdigest() == case["mat_index_sha256"], tag
    # and the module on the GPU holds exactly those buffers
    c0 = fx["digests"][0]
    lin = nmsparse_linear.NmSparseLinear(c0["N"], c0["K"], c0["M"], c0["seed"], "cuda")
    assert hashlib.sha256(lin.mat_data.cpu().view(torch.int16).numpy().tobytes()).hexdigest() == c0["mat_data_sha256"]


def test_op_and_module_on_gpu(gpu):
    lin = nmsparse_linear.NmSparseLinear(1024, 4096, 64, 3, "cuda")
    x = torch.randn(1, 1, 4096, device=gpu, dtype=torch.float16)
    y = lin(x)
    assert y.shape == (1, 1, 1024)
    check_parity(y.reshape(1, -1), x.reshape(1, -1), lin.mat_data, lin.mat_index, 32, 64, "module")
    xb = x.to(torch.bfloat16)
    yb = torch.ops.nmsparse.gemv(xb, lin.mat_data, lin.mat_index, lin.w, lin.h, 32, 64)
    assert yb.dtype == torch.bfloat16
    y16 = torch.ops.nmsparse.gemv(xb.half(), lin.mat_data, lin.mat_index, lin.w, lin.h, 32, 64)
    assert torch.equal(yb, y16.to(torch.bfloat16))
    with pytest.raises(RuntimeError, match="rows==1"):
        torch.ops.nmsparse.gemv(torch.zeros(1, 2, 4096, device=gpu, dtype=torch.float16),
                                lin.mat_data, lin.mat_index, lin.w, lin.h, 32, 64)


def test_large_h_and_misaligned_view(gpu):
    K, h, nnz, m = 4096, 128256, 32, 64  # lm_head-sized output
    say("large h 128256")
    x, md, mi = make_case(K, h, nnz, m, seed=8)
    out = run(x, md, mi, nnz, m)
    rows = torch.randperm(h, generator=torch.Generator().manual_seed(0))[:2048]
    ref = O.gemv_f64(x.cpu(), md[:, rows.to(gpu)].cpu(), mi.cpu(), nnz, m)
    e = O.error_metrics(ref, out[0, rows.to(gpu)].cpu())
    assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, e
    # a mat_data view whose base is not 16-byte aligned
    K2, h2 = 256, 384
    x2, md2, mi2 = make_case(K2, h2, 2, 4, seed=9)
    big = torch.empty(md2.numel() + 1, dtype=torch.float16, device=gpu)
    view = big[1:].view(md2.shape)
    view.copy_(md2)
    assert view.data_ptr() % 16
    assert torch.equal(run(x2, view, mi2, 2, 4), run(x2, md2, mi2, 2, 4))


def test_c_abi_strided_vec_and_in_range_foreign_positions(gpu):
    K, h, nnz, m = 1024, 512, 2, 4
    x, md, mi = make_case(K, h, nnz, m, seed=10)
    xs = torch.zeros(1, 3 * K, dtype=torch.float16, device=gpu)
    xs[0, ::3] = x[0]
    out = torch.empty(1, h, dtype=torch.float16, device=gpu)
    lib = _lib.load()
    need = lib.nm_gemv_workspace_bytes(h, md.shape[0], nnz, m)
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    rc = lib.nm_gemv_f16(xs.data_ptr(), 3, md.data_ptr(), mi.data_ptr(), out.data_ptr(), ws.data_ptr(),
                         ws.numel(), h, md.shape[0], nnz, m, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "nm_gemv_f16")
    assert torch.equal(out, run(x, md, mi, nnz, m))
    # positions >= M inside the vector read the next group's entry (reference
    # semantics); past the end of vec they contribute nothing.
    mi2 = mi.clone()
    mi2[0, 1] = 5      # group 0 -> position 5 (group 1's slot)
    mi2[-1, 1] = 7     # last group -> position K + 3, outside vec
    out2 = run(x, md, mi2, nnz, m)
    check_parity(out2, x, md, mi2, nnz, m, "foreign positions")


# ---------------------------------------------------------------------------
# Grouped launches (q/k/v in one grid) and the gate/up pair with SiLU·mul
# ---------------------------------------------------------------------------
GROUPS = [  # (K, [h...], nnz, m)
    (4096, [4096, 1024, 1024], 32, 64), (4096, [4096, 1024, 1024], 2, 4), (1024, [384, 128], 3, 4),
    (2048, [1152, 128, 256, 640], 8, 16)]


@pytest.mark.parametrize("K,hs,nnz,m", GROUPS, ids=lambda v: str(v))
def test_grouped_matches_single_launches_and_oracle(gpu, K, hs, nnz, m):
    from spmv_decode_amd.hip_spmv import nmsparse_gemv_grouped

    g = torch.Generator(device="cuda").manual_seed(K + len(hs))
    x = torch.randn(1, K, generator=g, device="cuda").half()
    probs = []
    for i, h in enumerate(hs):
        _, md, mi = make_case(K, h, nnz, m, seed=100 + i)
        probs.append((md, mi))
    say(f"grouped {K} {hs} {nnz}:{m}")
    outs = nmsparse_gemv_grouped(x, probs, nnz, m)
    for (md, mi), o in zip(probs, outs):
        check_parity(o, x, md, mi, nnz, m, f"grouped {hs}")
    for cfg in (1, 3, 6):
        for splits in (1, 3, 8):
            outs = nmsparse_gemv_grouped(x, probs, nnz, m, config_id=cfg, splits=splits)
            for (md, mi), o in zip(probs, outs):
                assert torch.equal(o, run(x, md, mi, nnz, m, config_id=cfg, splits=splits)), (cfg, splits)


def _silu_ref(x, gd, gi, ud, ui, nnz, m):
    gv = O.gemv_f64(x.cpu(), gd.cpu(), gi.cpu(), nnz, m)
    uv = O.gemv_f64(x.cpu(), ud.cpu(), ui.cpu(), nnz, m)
    return gv / (1.0 + np.exp(-gv)) * uv


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
def test_gate_up_silu_pair(gpu, dtype):
    from spmv_decode_amd.hip_spmv import nmsparse_gate_up_silu

    n = _lib.load().nm_num_gate_up_configs()
    for K, h, nnz, m in ((4096, 14336, 32, 64), (4096, 14336, 2, 4), (1024, 384, 3, 4), (5120, 17408, 8, 16)):
        x, gd, gi = make_case(K, h, nnz, m, seed=h, dtype=dtype)
        _, ud, ui = make_case(K, h, nnz, m, seed=h + 1, dtype=dtype)
        ref = _silu_ref(x, gd, gi, ud, ui, nnz, m)
        for cfg in [-1, *range(n)]:
            for splits in (0, 1, 3):
                say(f"gate/up {dtype} {K}x{h} {nnz}:{m} cfg {cfg} splits {splits}")
                out = nmsparse_gate_up_silu(x, (gd, gi), (ud, ui), nnz, m, config_id=cfg, splits=splits)
                got = out.float().cpu().numpy().reshape(-1)
                assert np.isfinite(got).all()
                if dtype == torch.float32:
                    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
                else:
                    e = O.error_metrics(ref, got)
                    bound = (1e-2, 1e-3) if dtype == torch.float16 else (4e-2, 8e-3)
                    assert e["max_abs"] <= bound[0] and e["rel_l2"] <= bound[1], (cfg, splits, e)


# ---------------------------------------------------------------------------
# Fusions at the GEMV's edges: input RMSNorm, residual, per-head norm, RoPE,
# KV-cache layout
# ---------------------------------------------------------------------------
def _fp_bound(ref, got, dtype, abs_terms, w):
    """|got - ref| <= one ulp of the output type + the fp32 accumulation bound
    + 1e-6 relative (the fp32 normalisation scale)."""
    if dtype == torch.float32:
        return np.abs(got - ref) <= 4.0 * np.sqrt(w) * 2.0 ** -24 * abs_terms + 1e-6 * np.abs(ref) + 1e-30
    exp = np.maximum(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))), MIN_NORMAL_EXP[dtype])
    ulp = np.exp2(exp - ULP_BITS[dtype])
    return np.abs(got - ref) <= ulp + 4.0 * np.sqrt(w) * 2.0 ** -24 * abs_terms + 1e-6 * np.abs(ref)


def _normed_ref(x, lnw, eps, md, mi, nnz, m):
    xn = O.rms_norm_f64(x.cpu().reshape(-1), lnw.cpu(), eps)
    ref = O.gemv_f64(xn, md.cpu(), mi.cpu(), nnz, m)
    terms = np.abs(O.to_f64(md.cpu())).T @ np.abs(O.gather_activations(xn, mi.cpu(), nnz, m))
    return ref, terms


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("K,hs,nnz,m", [(4096, [4096, 1024, 1024], 32, 64), (1024, [384, 128], 3, 4),
                                        (5120, [1280], 8, 16)], ids=str)
def test_input_rmsnorm_and_residual_grouped(gpu, K, hs, nnz, m, dtype):
    from spmv_decode_amd.hip_spmv import GemvProblem, nmsparse_gemv_launch

    g = torch.Generator(device="cuda").manual_seed(K + sum(hs))
    x = (torch.randn(1, K, generator=g, device="cuda") * 3).to(dtype)
    lnw = (torch.rand(K, generator=g, device="cuda") + 0.5).to(dtype)
    probs = [make_case(K, h, nnz, m, seed=200 + i, dtype=dtype)[1:] for i, h in enumerate(hs)]
    res = [torch.randn(1, h, generator=g, device="cuda").to(dtype) for h in hs]
    for cfg, splits in ((-1, 0), (1, 1), (3, 3), (6, 8)):
        say(f"norm+residual {dtype} K{K} {hs} {nnz}:{m} cfg {cfg} splits {splits}")
        keep = [r.clone() for r in res]
        inplace = [r.clone() for r in res]
        pr = [GemvProblem(md, mi, o, residual=o) for (md, mi), o in zip(probs, inplace)]
        outs = nmsparse_gemv_launch(x, pr, nnz, m, norm=(lnw, 1e-5), config_id=cfg, splits=splits)
        assert all(o.data_ptr() == r.data_ptr() for o, r in zip(outs, inplace))
        for (md, mi), o, r in zip(probs, outs, keep):
            ref, terms = _normed_ref(x, lnw, 1e-5, md, mi, nnz, m)
            ref = ref + O.to_f64(r.cpu()).reshape(-1)
            got = o.float().cpu().numpy().reshape(-1)
            ok = _fp_bound(ref, got, dtype, terms, md.shape[0])
            assert ok.all(), (cfg, splits, int((~ok).sum()), float(np.abs(got - ref).max()))
        # without the residual: the normalised GEMV alone
        outs = nmsparse_gemv_launch(x, [GemvProblem(md, mi) for md, mi in probs], nnz, m, norm=(lnw, 1e-5),
                                    config_id=cfg, splits=splits)
        for (md, mi), o in zip(probs, outs):
            ref, terms = _normed_ref(x, lnw, 1e-5, md, mi, nnz, m)
            got = o.float().cpu().numpy().reshape(-1)
            assert _fp_bound(ref, got, dtype, terms, md.shape[0]).all(), (cfg, splits)


def test_input_rmsnorm_rejections(gpu):
    from spmv_decode_amd.hip_spmv import GemvProblem, nmsparse_gemv_launch

    x, md, mi = make_case(1024, 256, 2, 4, seed=1)
    lnw = torch.ones(1024, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="norm weight"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, norm=(lnw[:512], 1e-5))
    with pytest.raises(ValueError, match="norm weight"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, norm=(lnw.float(), 1e-5))
    with pytest.raises(ValueError, match="residual"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi, residual=torch.zeros(128, device="cuda").half())], 2, 4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_gate_up_pair_with_input_rmsnorm_and_residual(gpu, dtype):
    from spmv_decode_amd.hip_spmv import nmsparse_gate_up_silu

    for K, h, nnz, m in ((4096, 14336, 32, 64), (1024, 384, 3, 4)):
        x, gd, gi = make_case(K, h, nnz, m, seed=h + 5, dtype=dtype)
        _, ud, ui = make_case(K, h, nnz, m, seed=h + 6, dtype=dtype)
        lnw = (torch.rand(K, device="cuda") + 0.5).to(dtype)
        res = torch.randn(1, h, device="cuda").to(dtype)
        xn = O.rms_norm_f64(x.cpu().reshape(-1), lnw.cpu(), 1e-6)
        gv = O.gemv_f64(xn, gd.cpu(), gi.cpu(), nnz, m)
        uv = O.gemv_f64(xn, ud.cpu(), ui.cpu(), nnz, m)
        for cfg in (-1, 0, 3):
            for splits in (0, 1, 3):
                say(f"gate/up norm {dtype} {K}x{h} {nnz}:{m} cfg {cfg} splits {splits}")
                out = nmsparse_gate_up_silu(x, (gd, gi), (ud, ui), nnz, m, norm=(lnw, 1e-6), residual=res,
                                            config_id=cfg, splits=splits)
                ref = O.silu_f64(gv) * uv + O.to_f64(res.cpu()).reshape(-1)
                got = out.float().cpu().numpy().reshape(-1)
                e = O.error_metrics(ref, got)
                bound = (1e-2, 1e-3) if dtype == torch.float16 else (4e-2, 8e-3)
                assert e["max_abs"] <= bound[0] and e["rel_l2"] <= bound[1], (cfg, splits, e)


def _qkv_case(K, nh, kvh, hd, S, nnz, m, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = (torch.randn(1, K, generator=g, device="cuda") * 2).to(dtype)
    q = make_case(K, nh * hd, nnz, m, seed=seed + 1, dtype=dtype)[1:]
    k = make_case(K, kvh * hd, nnz, m, seed=seed + 2, dtype=dtype)[1:]
    v = make_case(K, kvh * hd, nnz, m, seed=seed + 3, dtype=dtype)[1:]
    lnw = (torch.rand(K, generator=g, device="cuda") + 0.5).to(dtype)
    qn = (torch.rand(hd, generator=g, device="cuda") + 0.5).to(dtype)
    kn = (torch.rand(hd, generator=g, device="cuda") + 0.5).to(dtype)
    ang = torch.outer(torch.arange(S, dtype=torch.float64), 1.0 / (10000.0 ** (torch.arange(hd // 2) * 2.0 / hd)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).cuda()
    kc = torch.randn(kvh, hd, S, generator=g, device="cuda").to(dtype)
    vc = torch.randn(kvh, S, hd, generator=g, device="cuda").to(dtype)
    return x, q, k, v, lnw, qn, kn, ang, rope, kc, vc


def _check_heads(got, ref, dtype, what):
    got = got.float().cpu().numpy().reshape(ref.shape)
    scale = np.abs(ref).max()
    exp = np.maximum(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))), MIN_NORMAL_EXP[dtype])
    tol = np.exp2(exp - ULP_BITS[dtype]) + 1e-5 * scale
    bad = np.abs(got - ref) > tol
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))


@pytest.mark.parametrize("layout", ["plain", "decoder"])
@pytest.mark.parametrize("qk_norm", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("K,nh,kvh,hd,nnz,m", [(4096, 32, 8, 128, 32, 64), (512, 4, 2, 64, 2, 4),
                                               (5120, 40, 8, 128, 8, 16), (5120, 64, 8, 128, 16, 32)], ids=str)
def test_qkv_decode_rope_and_cache_write(gpu, K, nh, kvh, hd, nnz, m, dtype, qk_norm, layout):
    """plain: q_out [1, nh*hd], keys [kvh, hd, S], values [kvh, S, hd] (row pos).
    decoder: the decoder's buffers, q_out rows [nh, hd + 8] and keys
    [kvh, hd + 8, S] whose extra columns / rows must stay untouched, values
    [kvh, hd, S] (column pos). Values are read through a [kvh, S, hd] view."""
    from spmv_decode_amd.hip_spmv import nmsparse_qkv_decode

    S, pad = 48, 8
    x, q, k, v, lnw, qn, kn, ang, rope, kc, vc = _qkv_case(K, nh, kvh, hd, S, nnz, m, dtype, seed=K + nh)
    if layout == "decoder":
        g = torch.Generator(device="cuda").manual_seed(K)
        kc = torch.cat([kc, torch.randn(kvh, pad, S, generator=g, device="cuda").to(dtype)], dim=1)
    for pos_v, cfg, splits in ((0, -1, 0), (37, -1, 0), (S - 1, 3, 3), (5, 1, 1)):
        say(f"qkv decode {dtype} K{K} {nh}/{kvh}x{hd} {nnz}:{m} qk_norm {qk_norm} {layout} pos {pos_v} cfg {cfg}")
        kc1 = kc.clone()
        if layout == "decoder":
            vct = vc.transpose(1, 2).contiguous()
            vkw, vc1 = dict(v_cache_t=vct), vct.transpose(1, 2)
            qbuf = torch.full((nh, hd + pad), 3.0, device="cuda", dtype=dtype)
            qo = qbuf[:, :hd]
        else:
            vc1 = vc.clone()
            vkw = dict(v_cache=vc1)
            qbuf = qo = torch.empty(1, nh * hd, device="cuda", dtype=dtype)
        pos = torch.tensor([pos_v], device="cuda")
        nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=qbuf, k_cache_t=kc1, **vkw, pos=pos, rope_table=rope,
                            head_dim=hd, norm=(lnw, 1e-5), q_norm=qn if qk_norm else None,
                            k_norm=kn if qk_norm else None, head_eps=1e-6, config_id=cfg, splits=splits)
        rq, rk, rv = O.qkv_decode_f64(x.cpu().reshape(-1), (q[0].cpu(), q[1].cpu()), (k[0].cpu(), k[1].cpu()),
                                      (v[0].cpu(), v[1].cpu()), nnz, m, angle_row=ang[pos_v].numpy(), head_dim=hd,
                                      norm=(lnw.cpu(), 1e-5), q_norm=qn.cpu() if qk_norm else None,
                                      k_norm=kn.cpu() if qk_norm else None, eps=1e-6)
        _check_heads(qo, rq, dtype, "q")
        _check_heads(kc1[:, :hd, pos_v], rk, dtype, "k")
        _check_heads(vc1[:, pos_v, :], rv, dtype, "v")
        # every other cache slot, and the padding, is untouched, bit for bit
        km = torch.ones(S, dtype=torch.bool)
        km[pos_v] = False
        assert torch.equal(kc1[:, :, km.cuda()], kc[:, :, km.cuda()])
        assert torch.equal(kc1[:, hd:], kc[:, hd:])
        assert torch.equal(vc1[:, km.cuda(), :], vc[:, km.cuda(), :])
        if layout == "decoder":
            assert bool((qbuf[:, hd:] == 3.0).all())
    # a position outside the cache stores nothing at all
    kc1, vc1 = kc.clone(), vc.clone()
    qo = torch.full((1, nh * hd), 7.0, device="cuda", dtype=dtype)
    nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=qo, k_cache_t=kc1, v_cache=vc1, pos=torch.tensor([S], device="cuda"),
                        rope_table=rope, head_dim=hd, norm=(lnw, 1e-5))
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc) and torch.equal(vc1, vc) and bool((qo == 7.0).all())


def test_qkv_decode_graph_replays_follow_the_device_position(gpu):
    """Captured once, replayed at successive positions (the position is a
    device tensor): every replay writes its own cache slot, as eager calls do."""
    from spmv_decode_amd.hip_spmv import nmsparse_qkv_decode

    K, nh, kvh, hd, S, nnz, m = 1024, 8, 2, 128, 16, 8, 16
    x, q, k, v, lnw, qn, kn, ang, rope, kc, vc = _qkv_case(K, nh, kvh, hd, S, nnz, m, torch.float16, seed=9)
    pos = torch.tensor([0], device="cuda")
    qo = torch.empty(1, nh * hd, device="cuda", dtype=torch.float16)
    ke, ve = kc.clone(), vc.clone()
    kw = dict(rope_table=rope, head_dim=hd, norm=(lnw, 1e-5), q_norm=qn, k_norm=kn)
    eager_q = []
    for t in range(6):
        nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=qo, k_cache_t=ke, v_cache=ve,
                            pos=torch.tensor([t], device="cuda"), **kw)
        eager_q.append(qo.clone())
    kg, vg = kc.clone(), vc.clone()
    nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=qo, k_cache_t=kg, v_cache=vg, pos=pos, **kw)  # warm
    torch.cuda.synchronize()
    kg.copy_(kc)
    vg.copy_(vc)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=qo, k_cache_t=kg, v_cache=vg, pos=pos, **kw)
    torch.cuda.current_stream().wait_stream(s)
    for t in range(6):
        pos.fill_(t)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(qo, eager_q[t]), t
    assert torch.equal(kg, ke) and torch.equal(vg, ve)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_decoder_fused_layer_matches_grouped_and_per_linear_paths(gpu, qk_norm):
    """Three ways through the same sparse model give the same logits over
    several steps: the fused layer (norms, RoPE, cache write and residuals
    inside the GEMV launches), the grouped q/k/v + gate/up launches with
    PyTorch norms/RoPE, and one launch per Linear (within fp16 tolerance:
    the fused forms round less often)."""
    from spmv_decode_amd import swap_to_nmsparse
    from spmv_decode_amd.decode import model as dm

    cfg = dm.tiny_config(qk_norm=qk_norm)
    torch.manual_seed(0)
    mdl = dm.Decoder(cfg).to("cuda", torch.float16)
    dm.init_weights_(mdl, seed=0, std=0.05)
    with torch.no_grad():
        for name, prm in mdl.named_parameters():
            if name.endswith("norm.weight"):
                prm.uniform_(0.5, 1.5)  # non-trivial norm weights
    swap_to_nmsparse(mdl, 8, "cuda", seed=1, init="device", keep_dense=False)
    assert all(dm.fusable(b) for b in mdl.layers)
    toks = [3, 5, 7, 9, 11]

    mdl.carry_mode = "split"  # the split carry rounds what the plain fused layers round, the same way

    def run(mode, carry=True):
        mdl.set_launch_mode(mode)
        mdl.carry_splitk = carry
        try:
            mdl.setup_cache(16, "cuda", dtype=torch.float16)
            with torch.no_grad():
                return [mdl.forward_step(torch.tensor([[t]], device="cuda"), torch.tensor([i], device="cuda")).float()
                        for i, t in enumerate(toks)]
        finally:
            mdl.set_launch_mode("fused")
            mdl.carry_splitk = True

    fused = run("fused")
    assert mdl._carry is not None and mdl._carry[1] is not None  # the fused layers carried the split-K sums
    plain = run("fused", carry=False)
    grouped, per_linear, modules = run("grouped"), run("per_linear"), run("modules")
    for a, p, b, c, d in zip(fused, plain, grouped, per_linear, modules):
        # the carried and the plain fused layers round the same values the same
        # way; only the input norm's mean of squares is summed in another order
        torch.testing.assert_close(a, p, rtol=2e-3, atol=2e-3)
        torch.testing.assert_close(a, b, rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(b, c, rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(d, c, rtol=2e-2, atol=2e-2)


def test_tied_siblings_against_the_oracle(gpu, monkeypatch):
    """Linears tied by swap_to_nmsparse (q/k/v here) called one after another on
    the same input run as ONE grouped launch, in any call order, each output
    within the oracle bar and equal to the grouped launch's; a new input object
    or an in-place change of the input launches afresh (never a stale output);
    inputs the group does not take fall back to the member's own op; under
    hipGraph capture the graph holds the grouped launch and its replays follow
    the captured input buffer's new contents."""
    from spmv_decode_amd.nmsparse_linear import NmSparseLinear, tie_siblings

    K, M = 4096, 64
    mods = [NmSparseLinear(h, K, M, 30 + i, "cuda", init="device") for i, h in enumerate((4096, 1024, 1024))]
    tie_siblings(*mods)
    launches = []
    real = hip_spmv.nmsparse_gemv_grouped
    monkeypatch.setattr(hip_spmv, "nmsparse_gemv_grouped", lambda *a, **k: launches.append(1) or real(*a, **k))
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(1, 1, K, generator=g, device="cuda").half()
    outs = {i: mods[i](x) for i in (1, 0, 2)}  # k first: it launches for all three
    assert len(launches) == 1
    ref = real(x.view(1, -1), [(m.mat_data, m.mat_index) for m in mods], 32, 64)
    for i, mod in enumerate(mods):
        assert outs[i].shape == (1, 1, mod.h) and torch.equal(outs[i].view(1, -1), ref[i])
        check_parity(outs[i].view(1, -1), x.view(1, -1), mod.mat_data, mod.mat_index, 32, 64, f"tied {i}")
    x2 = x.clone()  # same values, another object: launched afresh
    assert torch.equal(mods[2](x2), outs[2]) and len(launches) == 2
    with pytest.warns(RuntimeWarning, match="streamed for nothing"):  # q and k of that launch never claimed
        assert torch.equal(mods[2](x2), outs[2]) and len(launches) == 3  # v again: no second hand-out
    y_q = mods[0](x)  # launches for x (k, v pending) ...
    x.mul_(2)  # ... then the input changes in place: k must see the new values
    y_k = mods[1](x)
    assert len(launches) == 5 and torch.equal(y_q, outs[0])
    check_parity(y_k.view(1, -1), x.view(1, -1), mods[1].mat_data, mods[1].mat_index, 32, 64, "k after x*2")
    xb = x.view(1, K).bfloat16()  # a dtype the group does not take: each member's own op
    assert mods[0](xb).dtype == torch.bfloat16 and len(launches) == 5
    # graph capture of the three calls on a static input
    xs = torch.zeros(1, 1, K, dtype=torch.float16, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):  # warm-up on the capture stream
        [m(xs) for m in mods]
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    n0 = len(launches)
    with torch.cuda.graph(graph, stream=st):
        gouts = [m(xs) for m in mods]
    assert len(launches) == n0 + 1
    for rep in range(3):
        say(f"tied siblings graph replay {rep}")
        xs.copy_(torch.randn(1, 1, K, generator=g, device="cuda").half())
        graph.replay()
        torch.cuda.synchronize()
        for i, mod in enumerate(mods):
            check_parity(gouts[i].view(1, -1), xs.view(1, -1), mod.mat_data, mod.mat_index, 32, 64, f"graph {rep} {i}")
        assert torch.equal(mods[1](x.clone()), y_k)  # eager work between the replays
        torch.cuda.synchronize()


def test_tied_siblings_group_multi_row_inputs(gpu, monkeypatch):
    """Tied siblings called with 9-128 rows of fp16 (a batch of short prompts)
    run as ONE grouped matrix-core SpMM: each member's output equal to the
    grouped launch's and within the oracle bar; 2-8 rows and more than 128
    rows go through each member's own op."""
    from spmv_decode_amd.nmsparse_linear import NmSparseLinear, tie_siblings
    from test_spmm_gpu import check_rows

    K, M = 4096, 64
    mods = [NmSparseLinear(h, K, M, 50 + i, "cuda", init="device") for i, h in enumerate((4096, 1024, 1024))]
    tie_siblings(*mods)
    launches = []
    real = hip_spmv.nmsparse_spmm_group_hip
    monkeypatch.setattr(hip_spmv, "nmsparse_spmm_group_hip", lambda *a, **k: launches.append(1) or real(*a, **k))
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(2, 12, K, generator=g, device="cuda").half()
    say("tied siblings 24 rows")
    outs = [mods[i](x) for i in (2, 0, 1)]
    outs = [outs[1], outs[2], outs[0]]
    assert len(launches) == 1
    ref = real(x, [(m.mat_data, m.mat_index) for m in mods], 32, 64)
    for mod, o, r in zip(mods, outs, ref):
        assert o.shape == (2, 12, mod.h) and torch.equal(o, r)
        check_rows(o.view(24, -1), x.view(24, -1), mod.mat_data, mod.mat_index, 32, 64, f"tied rows h{mod.h}")
    for rows in (4, 130):
        xr = torch.randn(rows, K, generator=g, device="cuda").half()
        say(f"tied siblings {rows} rows")
        for mod in mods:
            assert torch.equal(mod(xr), torch.ops.nmsparse.spmm(xr, mod.mat_data, mod.mat_index, mod.w, mod.h, 32, 64))
    assert len(launches) == 1


def test_swapped_model_decodes_under_inference_mode(gpu):
    """The reference's benchmarks swap the model and run it under
    torch.inference_mode() (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:87,
    132-140): the swapped decoder with its q/k/v and gate/up tied, every
    projection called as a module, decodes one-row steps there with one grouped
    launch per tied group, and its logits equal the same steps under no_grad."""
    from spmv_decode_amd.decode.model import Decoder, init_weights_, tiny_config
    from spmv_decode_amd.nmsparse_linear import swap_to_nmsparse

    cfg = tiny_config(qk_norm=True)
    model = Decoder(cfg).to(device="cuda", dtype=torch.float16)
    init_weights_(model, seed=3)
    swap_to_nmsparse(model, 16, "cuda", seed=5, init="device", keep_dense=False)
    model.set_launch_mode("modules")
    tokens = torch.randint(0, cfg.vocab, (6,), generator=torch.Generator().manual_seed(2)).cuda()

    def run():
        model.setup_cache(8, "cuda", dtype=torch.float16)
        return torch.cat([model.forward_step(t.view(1, 1), torch.tensor([i], device="cuda"))
                          for i, t in enumerate(tokens)])

    with torch.no_grad():
        ref = run()
    real = hip_spmv.nmsparse_gemv_grouped
    launches = []
    hip_spmv.nmsparse_gemv_grouped = lambda *a, **k: launches.append(1) or real(*a, **k)
    try:
        with torch.inference_mode():
            got = run()
    finally:
        hip_spmv.nmsparse_gemv_grouped = real
    torch.cuda.synchronize()
    assert len(launches) == 2 * cfg.n_layers * tokens.numel()  # q/k/v and gate/up: one launch each
    assert torch.equal(got, ref)


@pytest.mark.parametrize("layout", ["hf", "gpt-fast"])
def test_compiled_unmodified_model_groups_siblings(gpu, layout, monkeypatch):
    """The unmodified model (every projection called as a module) after the swap,
    compiled with inductor (fullgraph, as the reference benchmark compiles its
    step: benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:155): the compile pass
    gives each layer 4 launches (HF names: q/k/v grouped, o, the gate/up pair
    with SiLU*mul, down; gpt-fast names: wqkv, wo, the w1/w3 pair, w2), the
    RMSNorms in front of q/k/v and gate/up folded into those launches and the
    residual adds after o and down into theirs, counted at the library calls
    of one compiled step, and its logits agree with the eager steps' (which
    launch through the sibling ties) within fp16 rounding."""
    from spmv_decode_amd import nmsparse_op
    from spmv_decode_amd.decode.model import Decoder, init_weights_, tiny_config
    from spmv_decode_amd.nmsparse_linear import swap_to_nmsparse

    cfg = tiny_config(qk_norm=True, n_layers=3)
    model = Decoder(cfg, layout=layout).to(device="cuda", dtype=torch.float16)
    init_weights_(model, seed=7)
    swap_to_nmsparse(model, 16, "cuda", seed=9, init="device", keep_dense=False)
    model.set_launch_mode("modules")
    tokens = torch.randint(0, cfg.vocab, (5,), generator=torch.Generator().manual_seed(4)).cuda()

    def run(step):
        model.setup_cache(8, "cuda", dtype=torch.float16)
        return torch.cat([step(t.view(1, 1), torch.tensor([i], device="cuda")) for i, t in enumerate(tokens)])

    with torch.no_grad():
        eager = run(model.forward_step)
        torch._dynamo.reset()
        compiled = torch.compile(model.forward_step, fullgraph=True, dynamic=False)
        try:
            say(f"compiling the {layout} step")
            run(compiled)  # compile once
            counts = {}
            for name in ("nmsparse_spmv_forward_hip", "nmsparse_gemv_grouped", "nmsparse_gate_up_silu",
                         "nmsparse_gemv_launch"):
                real = getattr(nmsparse_op, name)

                def counted(*a, _real=real, _name=name, **k):
                    counts[_name] = counts.get(_name, 0) + 1
                    return _real(*a, **k)

                monkeypatch.setattr(nmsparse_op, name, counted)
            got = run(compiled)
        finally:
            torch._dynamo.reset()
    torch.cuda.synchronize()
    L, T = cfg.n_layers, tokens.numel()
    # q/k/v (HF: three siblings grouped; gpt-fast: wqkv) with the input RMSNorm folded in, the gate/up pair with
    # the post-attention RMSNorm, o and down with their residual adds (gemv_residual: one launch each)
    want = {"nmsparse_gemv_grouped": L * T, "nmsparse_gate_up_silu": L * T, "nmsparse_gemv_launch": 2 * L * T}
    assert counts == want, counts
    assert torch.isfinite(got).all()
    rel = float((got.float() - eager.float()).norm() / eager.float().norm())
    say(f"{layout}: compiled vs eager logits rel-L2 {rel:.2e}")
    assert rel <= 5e-3, rel
    torch.testing.assert_close(got.float(), eager.float(), rtol=2e-2, atol=2e-2)


def test_module_under_torch_compile_matches_eager(gpu):
    """The reference benchmarks compile the model around the op
    (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:155): a full-graph
    torch.compile (aot_eager: no code generation) of a block that uses
    NmSparseLinear traces through the op's fake implementation and calls the
    HIP kernel, bit for bit as eager."""
    import torch.nn as nn

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nmsparse_linear.NmSparseLinear(1024, 2048, 16, 1, "cuda", init="device")
            self.b = nmsparse_linear.NmSparseLinear(2048, 1024, 16, 2, "cuda", init="device")

        def forward(self, x):
            return self.b(torch.nn.functional.silu(self.a(x))) + x

    torch._dynamo.reset()
    blk = Block()
    x = torch.randn(1, 1, 2048, device="cuda").half()
    eager = blk(x)
    compiled = torch.compile(blk, backend="aot_eager", fullgraph=True)
    say("torch.compile aot_eager over NmSparseLinear")
    for _ in range(2):
        got = compiled(x)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)


def test_split_k_handoff_soak_2000_replays(gpu):
    """The split-K handoff orders its partials by hardware completion (no-return
    agent-scope atomic swaps waited for with vmcnt, a returning agent-scope ticket
    add, agent-scope loads after it), not by a language-level happens-before. A
    rare visibility miss would show as a wrong sum, not a fault, so: the four
    decode launch classes at the Llama-3.1-8B shapes (32:64; 8 splits each,
    192-448 workgroups over every XCD) in one hipGraph, made idempotent (fixed
    position, residuals read from other buffers than they write), replayed 2000
    times; every replay's outputs bitwise equal to the first replay's, checked
    after each replay, stopping at the first mismatch; the first replay's down
    output within the oracle bar."""
    from spmv_decode_amd.decode.model import KEY_PAD
    from spmv_decode_amd.hip_spmv import (GemvProblem, nmsparse_gate_up_silu, nmsparse_gemv_launch,
                                          nmsparse_qkv_decode)

    g = torch.Generator(device="cuda").manual_seed(11)
    mats = {}
    for i, (name, K, h) in enumerate((("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
                                      ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096))):
        _, md, mi = make_case(K, h, 32, 64, seed=100 + i)
        mats[name] = (md, mi)
    S = 256
    x = torch.randn(1, 4096, generator=g, device="cuda").half()
    attn = torch.randn(1, 4096, generator=g, device="cuda").half()
    ln1, ln2 = ((torch.rand(4096, generator=g, device="cuda") + 0.5).half() for _ in range(2))
    q_out = torch.zeros(32, 128 + KEY_PAD, dtype=torch.float16, device="cuda")
    kc = torch.zeros(8, 128 + KEY_PAD, S, dtype=torch.float16, device="cuda")
    vc = torch.zeros(8, 128, S, dtype=torch.float16, device="cuda")
    ang = torch.outer(torch.arange(S, dtype=torch.float64), torch.rand(64, dtype=torch.float64))
    rope = torch.view_as_real(torch.polar(torch.ones_like(ang), ang).to(torch.complex64)).cuda()
    pos = torch.tensor([S // 3], device="cuda")
    h1, h2 = torch.empty_like(x), torch.empty_like(x)
    act = torch.empty(1, 14336, dtype=torch.float16, device="cuda")

    def layer():
        nmsparse_qkv_decode(x, mats["q"], mats["k"], mats["v"], 32, 64, q_out=q_out, k_cache_t=kc, v_cache_t=vc,
                            pos=pos, rope_table=rope, head_dim=128, norm=(ln1, 1e-5))
        nmsparse_gemv_launch(attn, [GemvProblem(*mats["o"], h1, residual=x)], 32, 64)
        nmsparse_gate_up_silu(h1, mats["gate"], mats["up"], 32, 64, out=act, norm=(ln2, 1e-5))
        nmsparse_gemv_launch(act, [GemvProblem(*mats["down"], h2, residual=h1)], 32, 64)

    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        layer()
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        layer()
    outs = (q_out, kc, vc, h1, act, h2)
    graph.replay()
    torch.cuda.synchronize()
    first = [t.clone() for t in outs]
    ref = O.gemv_f64(act.cpu(), mats["down"][0].cpu(), mats["down"][1].cpu(), 32, 64) + h1.float().cpu().numpy()[0]
    e = O.error_metrics(ref, h2.float().cpu().numpy().reshape(-1))
    assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, e
    for rep in range(1, 2000):
        graph.replay()
        torch.cuda.synchronize()
        for t, f, name in zip(outs, first, ("q", "k cache", "v cache", "o+resid", "gate/up", "down+resid")):
            if not torch.equal(t, f):
                pytest.fail(f"replay {rep}: {name} differs from the first replay")
        if rep % 500 == 0:
            say(f"handoff soak: {rep} replays bit-identical")
