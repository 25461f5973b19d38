"""GPU parity of the split-K carry between a decoder layer's launches.

A producer (o_proj / down_proj as `nmsparse_gemv_partials`) leaves its fp32
split partials; the next launch (gate/up or q/k/v with a carried input)
finishes its input x = round(sum of the partials + residual). Checked here:

* the finished vector each consumer writes (vec_out) is bit-identical to the
  producer's own epilogue, i.e. to the plain launch with the residual, under
  the same producer plan (the fp32 partials are summed in the same split
  order and rounded once) -- for fp16 / bf16 / fp32, 2:4 .. 128:256, producer
  split counts 1, 8 and 12 (the <= 8 and <= 16 kernels) and forced consumer
  plans;
* the consumer's outputs against the float64 oracle of the same layer
  (RMSNorm of the finished vector, then the GEMVs, SiLU * mul, the per-head
  norms and RoPE), to the bounds of the plain fused launches;
* the chain in a captured graph replayed many times, bit-identical to eager.
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import nm_oracle as O
from spmv_decode_amd.hip_spmv import (GemvProblem, carry_splits, launch_plan, nmsparse_gate_up_silu,
                                      nmsparse_gemv_launch, nmsparse_gemv_partials, nmsparse_qkv_decode)
from test_gemv_gpu import _check_heads, make_case

pytestmark = pytest.mark.gpu


def _producer(K_in, dim, nnz, m, dtype, seed):
    """o_proj-like [K_in -> dim] weights, its input and the residual stream."""
    y, md, mi = make_case(K_in, dim, nnz, m, seed=seed, dtype=dtype)
    g = torch.Generator(device="cuda").manual_seed(seed + 99)
    x = (torch.randn(1, dim, generator=g, device="cuda") * 2).to(dtype)
    return y, md, mi, x


def _finish_reference(y, md, mi, x, nnz, m, cfg=-1, splits=0):
    """The plain launch: out = round(W y + x) with the producer's plan."""
    ref = torch.empty_like(x)
    nmsparse_gemv_launch(y, [GemvProblem(md, mi, ref, residual=x)], nnz, m, config_id=cfg, splits=splits)
    return ref


def _carry(y, md, mi, nnz, m, cfg=-1, splits=0):
    """The producer's partials and the (config, splits) request under which
    the plain launch partitions the columns exactly as the producer did: the
    request itself when explicit, else the producer's own plan (a producer may
    plan differently from the plain launch), checked to re-plan identically."""
    plan = launch_plan([(md, mi)], nnz, m, config_id=cfg, splits=splits, producer=True)
    carry = torch.empty(plan["splits"], md.shape[1], dtype=torch.float32, device="cuda")
    nmsparse_gemv_launch(y, [GemvProblem(md, mi)], nnz, m, config_id=cfg, splits=splits, carry_out=carry)
    req = (cfg, splits) if (cfg, splits) != (-1, 0) else (plan["config_id"], plan["splits"])
    again = launch_plan([(md, mi)], nnz, m, config_id=req[0], splits=req[1])
    assert (again["config_id"], again["rows_per_split"]) == (plan["config_id"], plan["rows_per_split"]), (plan, again)
    return carry, plan, req


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("dim,inter,nnz,m", [(4096, 14336, 32, 64), (1024, 384, 2, 4), (2048, 1024, 128, 256),
                                             (5120, 17408, 32, 64)], ids=str)
def test_gate_up_consumer_finishes_the_producer_bitwise(gpu, dim, inter, nnz, m, dtype):
    y, od, oi, x = _producer(dim, dim, nnz, m, dtype, seed=dim + nnz)
    _, gd, gi = make_case(dim, inter, nnz, m, seed=dim + 1, dtype=dtype)
    _, ud, ui = make_case(dim, inter, nnz, m, seed=dim + 2, dtype=dtype)
    lnw = (torch.rand(dim, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3)) + 0.5).to(dtype)
    # producer plans: the library's (8 splits), one split, and 11-12 splits of
    # 512-row tiles (the consumer kernel that reads up to 16)
    for pcfg, psplits in ((-1, 0), (-1, 1), (5, 12)):
        carry, plan, req = _carry(y, od, oi, nnz, m, pcfg, psplits)
        ref_h = _finish_reference(y, od, oi, x, nnz, m, *req)
        if dim == 5120 and pcfg < 0 and psplits == 0:  # the Qwen3-14B o_proj: a producer plan of its own
            assert (plan["config_id"], plan["splits"], plan["blocks"]) == (1, 5, 200), plan
        if pcfg == 5:
            assert carry.shape[0] > 8
        xn = O.rms_norm_f64(ref_h.cpu().reshape(-1), lnw.cpu(), 1e-5)
        gv = O.gemv_f64(xn, gd.cpu(), gi.cpu(), nnz, m)
        uv = O.gemv_f64(xn, ud.cpu(), ui.cpu(), nnz, m)
        ref = O.silu_f64(gv) * uv
        for cfg, csplits in ((-1, 0), (0, 0), (1, 3)):
            say(f"carry gate/up {dtype} dim {dim} inter {inter} {nnz}:{m} producer splits {carry.shape[0]} "
                f"consumer cfg {cfg} splits {csplits}")
            h = torch.full_like(x, float("nan"))
            act = nmsparse_gate_up_silu(x, (gd, gi), (ud, ui), nnz, m, norm=(lnw, 1e-5), config_id=cfg,
                                        splits=csplits, carry_in=carry, vec_out=h)
            torch.cuda.synchronize()
            assert torch.equal(h, ref_h), (psplits, cfg, csplits)
            got = act.float().cpu().numpy().reshape(-1)
            e = O.error_metrics(ref, got)
            bound = {torch.float16: (1e-2, 1e-3), torch.bfloat16: (4e-2, 8e-3), torch.float32: (1e-4, 1e-5)}[dtype]
            assert e["max_abs"] <= bound[0] and e["rel_l2"] <= bound[1], (psplits, cfg, csplits, e)


@pytest.mark.parametrize("qk_norm", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("dim,inter,nh,kvh,nnz,m", [(4096, 14336, 32, 8, 32, 64), (5120, 17408, 40, 8, 32, 64),
                                                    (512, 1024, 4, 2, 2, 4)], ids=str)
def test_qkv_consumer_finishes_down_proj_bitwise(gpu, dim, inter, nh, kvh, nnz, m, dtype, qk_norm):
    """down_proj as the producer (its default plan: 8 or 12 splits at these
    shapes), the q/k/v launch with head norms, RoPE and the transposed-cache
    writes as the consumer; outputs against the float64 oracle."""
    hd = 128 if dim >= 4096 else 64
    act, dd, di, x = _producer(inter, dim, nnz, m, dtype, seed=inter + nnz)
    carry, _, req = _carry(act, dd, di, nnz, m)
    ref_x = _finish_reference(act, dd, di, x, nnz, m, *req)
    g = torch.Generator(device="cuda").manual_seed(dim)
    q = make_case(dim, nh * hd, nnz, m, seed=7, dtype=dtype)[1:]
    k = make_case(dim, kvh * hd, nnz, m, seed=8, dtype=dtype)[1:]
    v = make_case(dim, kvh * hd, nnz, m, seed=9, dtype=dtype)[1:]
    lnw = (torch.rand(dim, generator=g, device="cuda") + 0.5).to(dtype)
    qn = (torch.rand(hd, generator=g, device="cuda") + 0.5).to(dtype) if qk_norm else None
    kn = (torch.rand(hd, generator=g, device="cuda") + 0.5).to(dtype) if qk_norm else None
    S, pos = 64, 37
    ang = torch.outer(torch.arange(S, dtype=torch.float64), 1.0 / (10000.0 ** (torch.arange(hd // 2) * 2.0 / hd)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).cuda()
    q_out = torch.zeros(1, nh * hd, dtype=dtype, device="cuda")
    kc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    vc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    xo = torch.full_like(x, float("nan"))
    say(f"carry q/k/v {dtype} dim {dim} {nnz}:{m} qk_norm {qk_norm} producer splits {carry.shape[0]}")
    nmsparse_qkv_decode(x, q, k, v, nnz, m, q_out=q_out, k_cache_t=kc, v_cache_t=vc,
                        pos=torch.tensor([pos], device="cuda"), rope_table=rope, head_dim=hd, norm=(lnw, 1e-5),
                        q_norm=qn, k_norm=kn, head_eps=1e-5, carry_in=carry, vec_out=xo)
    torch.cuda.synchronize()
    assert torch.equal(xo, ref_x)
    xn = O.rms_norm_f64(ref_x.cpu().reshape(-1), lnw.cpu(), 1e-5)
    rot = np.exp(1j * ang[pos].numpy())

    def heads(md, mi, norm_w, rotate):
        r = O.gemv_f64(xn, md.cpu(), mi.cpu(), nnz, m).reshape(-1, hd)
        if norm_w is not None:
            r = r / np.sqrt((r * r).mean(axis=1, keepdims=True) + 1e-5) * O.to_f64(norm_w.cpu())
        if rotate:
            c = (r[:, 0::2] + 1j * r[:, 1::2]) * rot
            r = np.stack([c.real, c.imag], axis=-1).reshape(r.shape)
        return r

    for what, got, ref in (("q", q_out.view(nh, hd), heads(*q, qn, True)),
                           ("k", kc[:, :, pos], heads(*k, kn, True)), ("v", vc[:, :, pos], heads(*v, None, False))):
        _check_heads(got, ref, dtype, what)


def test_carry_chain_graph_replays_match_eager(gpu):
    """o producer -> gate/up consumer -> down producer -> q/k/v consumer, two
    layers' worth, captured once and replayed 1000 times with eager work in
    between: every replay's outputs and finished vectors equal the eager
    chain's bit for bit."""
    dim, inter, nh, kvh, hd, nnz, m = 4096, 14336, 32, 8, 128, 32, 64
    dtype = torch.float16
    y, od, oi, x0 = _producer(dim, dim, nnz, m, dtype, seed=11)
    _, gd, gi = make_case(dim, inter, nnz, m, seed=12)
    _, ud, ui = make_case(dim, inter, nnz, m, seed=13)
    _, dd, di = make_case(inter, dim, nnz, m, seed=14)
    q = make_case(dim, nh * hd, nnz, m, seed=15)[1:]
    k = make_case(dim, kvh * hd, nnz, m, seed=16)[1:]
    v = make_case(dim, kvh * hd, nnz, m, seed=17)[1:]
    lnw = (torch.rand(dim, device="cuda") + 0.5).half()
    S = 64
    ang = torch.outer(torch.arange(S, dtype=torch.float64), 1.0 / (10000.0 ** (torch.arange(hd // 2) * 2.0 / hd)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).cuda()
    pos = torch.tensor([5], device="cuda")
    co = torch.empty(carry_splits(od, oi, nnz, m), dim, dtype=torch.float32, device="cuda")
    cd = torch.empty(carry_splits(dd, di, nnz, m), dim, dtype=torch.float32, device="cuda")
    xa, hb = x0.clone(), torch.empty_like(x0)
    q_out = torch.zeros(1, nh * hd, dtype=dtype, device="cuda")
    kc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    vc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    acts = []

    def chain():
        xa.copy_(x0)
        acts.clear()
        for _ in range(2):
            nmsparse_gemv_partials(y, od, oi, nnz, m, co)
            act = nmsparse_gate_up_silu(xa, (gd, gi), (ud, ui), nnz, m, norm=(lnw, 1e-5), carry_in=co, vec_out=hb)
            acts.append(act)
            nmsparse_gemv_partials(act, dd, di, nnz, m, cd)
            nmsparse_qkv_decode(hb, q, k, v, nnz, m, q_out=q_out, k_cache_t=kc, v_cache_t=vc, pos=pos,
                                rope_table=rope, head_dim=hd, norm=(lnw, 1e-5), carry_in=cd, vec_out=xa)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        chain()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = [t.clone() for t in (xa, hb, q_out, kc, vc, *acts)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        chain()
    big = torch.randn(1 << 22, device="cuda")
    say("carry chain: 1000 graph replays")
    for rep in range(1000):
        for t in (xa, hb, q_out, kc, vc):
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        got = (xa, hb, q_out, kc, vc, *acts)
        assert all(torch.equal(a, b) for a, b in zip(got, want)), rep
        if rep % 100 == 0:
            assert torch.isfinite(big.sum())  # eager multi-block work between replays


def test_carry_argument_errors(gpu):
    x, md, mi = make_case(1024, 512, 2, 4, seed=1)
    lnw = torch.ones(1024, device="cuda", dtype=torch.float16)
    carry = torch.zeros(8, 1024, device="cuda")
    with pytest.raises(ValueError, match="carry_out holds"):
        nmsparse_gemv_partials(x, md, mi, 2, 4, torch.zeros(3, 512, device="cuda"))
    with pytest.raises(ValueError, match="carry_in must be"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, norm=(lnw, 1e-5), carry_in=carry.half(),
                             vec_out=torch.empty_like(x))
    with pytest.raises(ValueError, match="needs vec_out"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, norm=(lnw, 1e-5), carry_in=carry)
    with pytest.raises(ValueError, match="vec_out is the output"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, vec_out=torch.empty_like(x))
    from spmv_decode_amd import _lib

    with pytest.raises(_lib.NmSparseLibraryError):  # a consumer needs the input norm
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, carry_in=carry, vec_out=torch.empty_like(x))
