"""GPU parity of the HIP N:M GEMV against the CPU oracle.

Bar (north star): fp16 outputs within max-abs 1e-2 and rel-L2 1e-3 of the
fp32-accumulated reference value on the BASELINE distributions (weights
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
    """dense W [3072, 1024] ~ N(0, 0.02), 2:4 pattern from the
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


def test_decoder_uses_fused_launches_and_matches_unfused(gpu):
    """The decoder's grouped q/k/v and gate/up pair give the same logits as the
    per-Linear path (one rounding less in the MLP, so within fp16 tolerance)."""
    from spmv_decode_amd.decode import model as dm

    cfg = dm.tiny_config(qk_norm=True)
    torch.manual_seed(0)
    mdl = dm.Decoder(cfg).to("cuda", torch.float16)
    dm.init_weights_(mdl, seed=0, std=0.05)
    from spmv_decode_amd import swap_to_nmsparse

    swap_to_nmsparse(mdl, 8, "cuda", seed=1, init="device", keep_dense=False)
    mdl.setup_cache(16, "cuda", dtype=torch.float16)
    tok = torch.tensor([[3]], device="cuda")
    pos = torch.tensor([0], device="cuda")
    with torch.no_grad():
        fused = mdl.forward_step(tok, pos).float()
        orig = dm.grouped_sparse
        dm.grouped_sparse = lambda mods: False
        try:
            mdl.setup_cache(16, "cuda", dtype=torch.float16)
            unfused = mdl.forward_step(tok, pos).float()
        finally:
            dm.grouped_sparse = orig
    torch.testing.assert_close(fused, unfused, rtol=2e-2, atol=2e-2)
