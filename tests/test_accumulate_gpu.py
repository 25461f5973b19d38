"""GPU checks of the accumulated carry between a decoder layer's launches.

The producers (o_proj, the gate/up pair, down_proj) add their partial sums
into one fp32 row with atomics; the next launch finishes the epilogue as it
gathers its input. The order of the atomic adds varies from run to run, so
these checks bound values instead of comparing bits:

* an accumulating GEMV's row against the float64 oracle within the fp32
  accumulation bound, against the split producer's partials summed on the
  host, and adding (not storing) into what the row held;
* the accumulating pair's raw sums W (x * g) and its input's sums of squares
  against float64, with and without a carried input (whose finished vector
  vec_out is bit-exact given the accumulated row it read);
* the SiLU-product consumer (down_proj) against the float64 layer and against
  the split-carry launches of the same layer;
* the zero_buf clears, and a two-layer chain captured in a graph and replayed
  many times staying within the bound of its eager run (a missed clear would
  double an accumulator on the next replay).
"""
import numpy as np
import pytest
import torch

from conftest import say
from oracle import nm_oracle as O
from spmv_decode_amd.hip_spmv import (GemvProblem, carry_splits, gate_up_ssq_slots, launch_plan,
                                      nmsparse_gate_up_accumulate, nmsparse_gate_up_silu, nmsparse_gemv_accumulate,
                                      nmsparse_gemv_launch, nmsparse_gemv_partials, nmsparse_gemv_silu,
                                      nmsparse_qkv_decode)
from test_gemv_gpu import make_case

pytestmark = pytest.mark.gpu

# fp16 / bf16 / fp32 outputs of a fused layer against float64: (max_abs, rel_l2), as for the split carry
BOUND = {torch.float16: (1e-2, 1e-3), torch.bfloat16: (4e-2, 8e-3), torch.float32: (1e-4, 1e-5)}


def _acc_bound(act, md, mi, nnz, m):
    """fp32 accumulation bound of each row's sum of w products: 4 sqrt(w)
    eps32 sum|terms| (a wrong term or index exceeds it by orders of
    magnitude). act: float64 activations [K]."""
    terms = np.abs(O.to_f64(md.cpu())).T @ np.abs(O.gather_activations(act, mi.cpu(), nnz, m))
    return 4.0 * np.sqrt(md.shape[0]) * 2.0 ** -24 * terms + 1e-30


def _check_f32(got, ref, tol, tag):
    d = np.abs(got.detach().float().cpu().numpy().reshape(-1) - ref)
    assert np.isfinite(d).all() and (d <= tol).all(), (tag, int((d > tol).sum()), float(d.max()))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("K,h,nnz,m", [(4096, 4096, 32, 64), (14336, 4096, 32, 64), (1024, 512, 2, 4),
                                       (5120, 5120, 16, 32), (2048, 1024, 128, 256)], ids=str)
def test_accumulating_gemv_adds_its_sum(gpu, K, h, nnz, m, dtype):
    y, md, mi = make_case(K, h, nnz, m, seed=K + h + nnz, dtype=dtype)
    say(f"accumulate gemv {dtype} {K}->{h} {nnz}:{m}")
    ref = O.gemv_f64(y.cpu(), md.cpu(), mi.cpu(), nnz, m)
    tol = _acc_bound(O.to_f64(y.cpu()).reshape(-1), md, mi, nnz, m)
    acc = torch.zeros(1, h, device="cuda")
    zero = torch.full((1024,), float("nan"), device="cuda")
    nmsparse_gemv_accumulate(y, md, mi, nnz, m, acc, zero=zero)
    torch.cuda.synchronize()
    _check_f32(acc, ref, tol, "first")
    assert torch.equal(zero, torch.zeros_like(zero))
    # the producer's split partials summed on the host: the same tiles, another order of at most 16 adds
    parts = torch.empty(carry_splits(md, mi, nnz, m), h, device="cuda")
    nmsparse_gemv_partials(y, md, mi, nnz, m, parts)
    s = parts.sum(0, dtype=torch.float64).cpu().numpy()
    spread = parts.abs().sum(0, dtype=torch.float64).cpu().numpy() * parts.shape[0] * 2.0 ** -24
    _check_f32(acc, s, spread + 1e-30, "partials")
    # a second launch adds into the row
    nmsparse_gemv_accumulate(y, md, mi, nnz, m, acc)
    torch.cuda.synchronize()
    _check_f32(acc, 2 * ref, 2 * tol, "second")


def _pair_case(dim, inter, nnz, m, dtype, seed):
    x, gd, gi = make_case(dim, inter, nnz, m, seed=seed, dtype=dtype)
    _, ud, ui = make_case(dim, inter, nnz, m, seed=seed + 1, dtype=dtype)
    _, dd, di = make_case(inter, dim, nnz, m, seed=seed + 2, dtype=dtype)
    g = torch.Generator(device="cuda").manual_seed(seed + 3)
    lnw = (torch.rand(dim, generator=g, device="cuda") + 0.5).to(dtype)
    r = (torch.randn(1, dim, generator=g, device="cuda")).to(dtype)
    return x, (gd, gi), (ud, ui), (dd, di), lnw, r


def _check_pair_buffer(acc, xin, gate, up, lnw, slots, nnz, m, tag):
    """acc [2h + 16]: W_g (x g), W_u (x g) and `slots` sums of squares of x."""
    h = gate[0].shape[1]
    xg = O.to_f64(xin.cpu()).reshape(-1) * O.to_f64(lnw.cpu())  # x * g is exact in fp32 for 16-bit inputs
    for q, (md, mi) in enumerate((gate, up)):
        ref = O.gemv_f64(xg, md.cpu(), mi.cpu(), nnz, m)
        _check_f32(acc[q * h:(q + 1) * h], ref, _acc_bound(xg, md, mi, nnz, m), (tag, q))
    xv = O.to_f64(xin.cpu()).reshape(-1)
    ssq = float(acc[2 * h:2 * h + slots].double().sum().item())
    assert abs(ssq - float((xv * xv).sum())) <= 4.0 * np.sqrt(xv.size) * 2.0 ** -24 * float((xv * xv).sum()), tag


def _silu_reference(acc, h, slots, K, eps, dtype):
    """The consumer's input from the pair's buffer (as read back), float64,
    then rounded to the weights' dtype as the kernel rounds it."""
    a = acc.double().cpu().numpy()
    s = 1.0 / np.sqrt(a[2 * h:2 * h + slots].sum() / K + eps) if slots else 1.0
    act = O.silu_f64(s * a[:h]) * (s * a[h:2 * h])
    return act, torch.from_numpy(act).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("dim,inter,nnz,m", [(4096, 14336, 32, 64), (5120, 17408, 32, 64), (1024, 384, 2, 4),
                                             (5120, 25600, 16, 32)], ids=str)
def test_pair_producer_and_silu_consumer(gpu, dim, inter, nnz, m, dtype):
    """Uncarried pair -> buffer (raw sums, one sum of squares) -> down_proj
    with the SiLU-product input and a residual, against float64 and against
    the split-carry launches of the same layer (gate_up_silu, then the
    GEMV with the residual)."""
    x, gate, up, down, lnw, r = _pair_case(dim, inter, nnz, m, dtype, seed=dim + inter)
    say(f"accumulate pair + silu consumer {dtype} dim {dim} inter {inter} {nnz}:{m}")
    acc = torch.full((2 * inter + 16,), float("nan"), device="cuda")
    acc[:2 * inter].zero_()
    slots = nmsparse_gate_up_accumulate(x, gate, up, nnz, m, acc, norm=(lnw, 1e-5))
    assert slots == 1
    torch.cuda.synchronize()
    _check_pair_buffer(acc, x, gate, up, lnw, slots, nnz, m, "uncarried")
    out = nmsparse_gemv_silu(acc, *down, nnz, m, ssq_n=slots, silu_k=dim, silu_eps=1e-5, residual=r)
    torch.cuda.synchronize()
    # against the float64 layer: RMSNorm, both GEMVs, SiLU * mul, down_proj, residual
    xn = O.rms_norm_f64(x.cpu().reshape(-1), lnw.cpu(), 1e-5)
    act64 = O.silu_f64(O.gemv_f64(xn, gate[0].cpu(), gate[1].cpu(), nnz, m)) * O.gemv_f64(xn, up[0].cpu(),
                                                                                          up[1].cpu(), nnz, m)
    ref = O.gemv_f64(act64, down[0].cpu(), down[1].cpu(), nnz, m) + O.to_f64(r.cpu()).reshape(-1)
    e = O.error_metrics(ref, out.float().cpu().numpy().reshape(-1))
    assert e["max_abs"] <= BOUND[dtype][0] * 4 and e["rel_l2"] <= BOUND[dtype][1], e
    # against the same layer through the split launches
    act = nmsparse_gate_up_silu(x, gate, up, nnz, m, norm=(lnw, 1e-5))
    split = torch.empty_like(r)
    nmsparse_gemv_launch(act, [GemvProblem(*down, split, residual=r)], nnz, m)
    _, act_acc = _silu_reference(acc, inter, slots, dim, 1e-5, dtype)
    ea = O.error_metrics(act.float().cpu().numpy().reshape(-1), act_acc.float().numpy())
    assert ea["rel_l2"] <= BOUND[dtype][1], ea
    es = O.error_metrics(split.float().cpu().numpy().reshape(-1), out.float().cpu().numpy().reshape(-1))
    assert es["rel_l2"] <= BOUND[dtype][1], es
    # the consumer as an accumulating producer (down_proj of a middle layer): its row finished with the
    # residual matches the plain consumer's output up to the order of the adds (one rounding apart)
    acc_d = torch.zeros(1, dim, device="cuda")
    nmsparse_gemv_accumulate(None, *down, nnz, m, acc_d, silu_in=acc, silu_ssq_n=slots, silu_k=dim, silu_eps=1e-5)
    fin = (acc_d + r.float()).to(dtype)
    torch.cuda.synchronize()
    torch.testing.assert_close(fin, out, rtol=2 ** -7 if dtype == torch.bfloat16 else 2 ** -10, atol=1e-3)


def test_pair_without_norm_and_consumer_without_scale(gpu):
    """No input norm: the pair stores no sum of squares and the consumer takes
    s = 1, i.e. silu(W_g x) * (W_u x)."""
    dim, inter, nnz, m, dtype = 1024, 1536, 8, 16, torch.float16
    x, gate, up, down, _, _ = _pair_case(dim, inter, nnz, m, dtype, seed=5)
    acc = torch.zeros(2 * inter + 16, device="cuda")
    assert nmsparse_gate_up_accumulate(x, gate, up, nnz, m, acc) == 0
    out = nmsparse_gemv_silu(acc, *down, nnz, m, ssq_n=0, silu_k=0, silu_eps=0.0)
    torch.cuda.synchronize()
    xv = O.to_f64(x.cpu()).reshape(-1)
    act = O.silu_f64(O.gemv_f64(xv, gate[0].cpu(), gate[1].cpu(), nnz, m)) * O.gemv_f64(xv, up[0].cpu(),
                                                                                        up[1].cpu(), nnz, m)
    ref = O.gemv_f64(act, down[0].cpu(), down[1].cpu(), nnz, m)
    e = O.error_metrics(ref, out.float().cpu().numpy().reshape(-1))
    assert e["rel_l2"] <= 1e-3, e
    assert torch.equal(acc[2 * inter:], torch.zeros(16, device="cuda"))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("dim,inter,nnz,m", [(4096, 14336, 32, 64), (5120, 17408, 32, 64), (1024, 384, 2, 4)],
                         ids=str)
def test_carried_pair_producer(gpu, dim, inter, nnz, m, dtype):
    """o_proj accumulating into one row -> the pair reading it as a one-row
    carry: vec_out = round(row + x) bit for bit, one sum of squares per split
    of the pair's plan, raw sums against float64 on that finished vector."""
    x, gate, up, _, lnw, _ = _pair_case(dim, inter, nnz, m, dtype, seed=dim + 7)
    y, od, oi = make_case(dim, dim, nnz, m, seed=dim + 8, dtype=dtype)
    acc_o = torch.zeros(1, dim, device="cuda")
    nmsparse_gemv_accumulate(y, od, oi, nnz, m, acc_o)
    h = torch.full_like(x, float("nan"))
    acc = torch.zeros(2 * inter + 16, device="cuda")
    acc[2 * inter:] = float("nan")
    say(f"accumulate carried pair {dtype} dim {dim} inter {inter} {nnz}:{m}")
    slots = nmsparse_gate_up_accumulate(x, gate, up, nnz, m, acc, norm=(lnw, 1e-5), carry_in=acc_o, vec_out=h)
    plan = launch_plan([gate, up], nnz, m, gate_up=True, carried=True)
    assert slots == plan["splits"] == gate_up_ssq_slots(gate, up, nnz, m, carried=True) <= 16
    torch.cuda.synchronize()
    assert torch.equal(h, (acc_o + x.float()).to(dtype))
    assert torch.isfinite(acc[2 * inter:2 * inter + slots]).all()
    _check_pair_buffer(acc, h, gate, up, lnw, slots, nnz, m, "carried")


def test_accumulated_chain_graph_replays(gpu):
    """Two layers of the accumulated chain (q/k/v, o, gate/up, down) with the
    decoder's clearing schedule, captured once and replayed 300 times with
    eager work in between: every replay within the fp16 bound of the eager
    run, and the eager run within it of the split-carry chain."""
    dim, inter, nh, kvh, hd, nnz, m = 4096, 14336, 32, 8, 128, 32, 64
    dtype = torch.float16
    x0, gate, up, down, lnw, _ = _pair_case(dim, inter, nnz, m, dtype, seed=21)
    y, od, oi = make_case(dim, dim, nnz, m, seed=22)
    q = make_case(dim, nh * hd, nnz, m, seed=23)[1:]
    k = make_case(dim, kvh * hd, nnz, m, seed=24)[1:]
    v = make_case(dim, kvh * hd, nnz, m, seed=25)[1:]
    S = 64
    ang = torch.outer(torch.arange(S, dtype=torch.float64), 1.0 / (10000.0 ** (torch.arange(hd // 2) * 2.0 / hd)))
    rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).cuda()
    pos = torch.tensor([5], device="cuda")
    acc_op = torch.full((dim + 2 * inter + 16,), float("nan"), device="cuda")  # o_proj's and the pair's rows
    acc_o, acc_p = acc_op[:dim].view(1, dim), acc_op[dim:]
    acc_d = torch.full((1, dim), float("nan"), device="cuda")
    ssq_n = gate_up_ssq_slots(gate, up, nnz, m, carried=True)
    xa, hb = x0.clone(), torch.empty_like(x0)
    q_out = torch.zeros(1, nh * hd, dtype=dtype, device="cuda")
    kc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    vc = torch.zeros(kvh, hd, S, dtype=dtype, device="cuda")
    qkv = dict(q_out=q_out, k_cache_t=kc, v_cache_t=vc, pos=pos, rope_table=rope, head_dim=hd, norm=(lnw, 1e-5))

    def chain():
        xa.copy_(x0)
        for i in range(2):
            if i == 0:
                nmsparse_qkv_decode(xa, q, k, v, nnz, m, **qkv, zero=acc_op)
            else:
                nmsparse_qkv_decode(hb, q, k, v, nnz, m, **qkv, carry_in=acc_d, vec_out=xa, zero=acc_op)
            nmsparse_gemv_accumulate(y, od, oi, nnz, m, acc_o)
            nmsparse_gate_up_accumulate(xa, gate, up, nnz, m, acc_p, norm=(lnw, 1e-5), carry_in=acc_o, vec_out=hb,
                                        zero=acc_d)
            if i == 0:
                nmsparse_gemv_accumulate(None, *down, nnz, m, acc_d, silu_in=acc_p, silu_ssq_n=ssq_n, silu_k=dim,
                                         silu_eps=1e-5)
            else:
                nmsparse_gemv_silu(acc_p, *down, nnz, m, ssq_n=ssq_n, silu_k=dim, silu_eps=1e-5, out=hb,
                                   residual=hb)

    def split_chain():
        co = torch.empty(carry_splits(od, oi, nnz, m), dim, device="cuda")
        cd = torch.empty(carry_splits(*down, nnz, m), dim, device="cuda")
        xs, hs = x0.clone(), torch.empty_like(x0)
        for i in range(2):
            if i == 0:
                nmsparse_qkv_decode(xs, q, k, v, nnz, m, **qkv)
            else:
                nmsparse_qkv_decode(hs, q, k, v, nnz, m, **qkv, carry_in=cd, vec_out=xs)
            nmsparse_gemv_partials(y, od, oi, nnz, m, co)
            act = nmsparse_gate_up_silu(xs, gate, up, nnz, m, norm=(lnw, 1e-5), carry_in=co, vec_out=hs)
            if i == 0:
                nmsparse_gemv_partials(act, *down, nnz, m, cd)
            else:
                nmsparse_gemv_launch(act, [GemvProblem(*down, hs, residual=hs)], nnz, m)
        return xs, hs, q_out.clone(), kc.clone(), vc.clone()

    say("accumulated chain: split reference, eager, capture")
    split = split_chain()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        chain()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = [t.clone() for t in (xa, hb, q_out, kc, vc)]
    for a, b in zip(want, split):
        torch.testing.assert_close(a, b, rtol=1e-2, atol=1e-2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        chain()
    big = torch.randn(1 << 22, device="cuda")
    say("accumulated chain: 300 graph replays")
    for rep in range(300):
        for t in (xa, hb, q_out, kc, vc):
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip((xa, hb, q_out, kc, vc), want):
            torch.testing.assert_close(a, b, rtol=1e-2, atol=1e-2, msg=lambda t, rep=rep: f"replay {rep}: {t}")
        if rep % 50 == 0:
            assert torch.isfinite(big.sum())  # eager multi-block work between replays


def test_accumulate_argument_errors(gpu):
    x, md, mi = make_case(1024, 512, 2, 4, seed=1)
    with pytest.raises(ValueError, match="adds into 512 floats"):
        nmsparse_gemv_accumulate(x, md, mi, 2, 4, torch.zeros(2, 512, device="cuda"))
    with pytest.raises(ValueError, match="carry_accumulate needs carry_out"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, carry_accumulate=True)
    with pytest.raises(ValueError, match="only with carry_accumulate"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi), GemvProblem(md, mi)], 2, 4, gate_up=True,
                             carry_out=torch.zeros(2 * 512 + 16, device="cuda"))
    with pytest.raises(ValueError, match="pass vec=None"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, silu_in=torch.zeros(2 * 1024 + 16, device="cuda"))
    with pytest.raises(ValueError, match="silu_in must be"):
        nmsparse_gemv_silu(torch.zeros(2 * 1024, device="cuda").half(), md, mi, 2, 4, ssq_n=0, silu_k=0,
                           silu_eps=0.0)
    with pytest.raises(ValueError, match="zero must be"):
        nmsparse_gemv_launch(x, [GemvProblem(md, mi)], 2, 4, zero=torch.zeros(6, device="cuda"))


@pytest.mark.parametrize("qk_norm,dtype", [(False, torch.float16), (True, torch.float16), (True, torch.bfloat16)],
                         ids=str)
def test_decoder_accumulated_carry_matches_split_carry(gpu, qk_norm, dtype):
    """The tiny decoder with carry_mode "accumulate" (fused_layers_accumulated,
    the default) against the split carry over several eager steps, then its
    graph replays against its eager steps (within 16-bit tolerance: the atomic
    adds' order varies)."""
    from spmv_decode_amd import swap_to_nmsparse
    from spmv_decode_amd.decode import model as dm
    from spmv_decode_amd.decode.runner import GraphDecoder

    cfg = dm.tiny_config(qk_norm=qk_norm)
    torch.manual_seed(0)
    mdl = dm.Decoder(cfg).to("cuda", dtype)
    tol = 5e-3 if dtype == torch.float16 else 4e-2
    dm.init_weights_(mdl, seed=0, std=0.05)
    with torch.no_grad():
        for name, prm in mdl.named_parameters():
            if name.endswith("norm.weight"):
                prm.uniform_(0.5, 1.5)
    swap_to_nmsparse(mdl, 8, "cuda", seed=1, init="device", keep_dense=False)
    if dtype != torch.float16:  # the swap packs fp16 (the reference's layout); the fused launches take bf16 weights
        assert not dm.fusable(mdl.layers[0], dtype)
        mdl.setup_cache(16, "cuda", dtype=dtype)
        # fp16 packed weights under bf16 activations: the op's own dtype check
        # refuses them, as the reference wrapper does (triton_spmv.py:245-283).
        with torch.no_grad(), pytest.raises(TypeError, match="same dtype"):
            mdl.forward_step(torch.tensor([[3]], device="cuda"), torch.tensor([0], device="cuda"))
        for mod in mdl.modules():
            if hasattr(mod, "mat_data"):
                mod.mat_data = mod.mat_data.to(dtype)
    assert dm.accumulate_supported(mdl.layers) and all(dm.fusable(b, dtype) for b in mdl.layers)
    toks = [3, 5, 7, 9, 11, 13]

    def run(mode):
        mdl.carry_mode = mode
        mdl.setup_cache(16, "cuda", dtype=dtype)
        with torch.no_grad():
            return [mdl.forward_step(torch.tensor([[t]], device="cuda"), torch.tensor([i], device="cuda")).float()
                    for i, t in enumerate(toks)]

    say(f"decoder accumulated carry qk_norm {qk_norm} {dtype}: eager")
    split = run("split")
    assert len(mdl._carry[1]) == 3
    acc = run("accumulate")
    assert len(mdl._carry[1]) == 4
    for a, b in zip(acc, split):
        torch.testing.assert_close(a, b, rtol=tol, atol=tol)
    say(f"decoder accumulated carry qk_norm {qk_norm} {dtype}: graph replays")
    gd = GraphDecoder(mdl, 12)
    prompt = torch.tensor([3, 5, 7])
    gd.run_prompt(prompt)
    eager = [gd.eager_step().clone() for _ in range(4)]
    eager_tokens = gd.tokens[3:8].clone()
    gd.capture()
    for rep in range(3):
        gd.run_prompt(prompt)
        for i in range(4):
            if not torch.equal(gd.tokens[3:4 + i], eager_tokens[:1 + i]):
                break  # a near-tie of a greedy choice went the other way: this step would see another token
            gd.replay()
            torch.cuda.synchronize()
            torch.testing.assert_close(gd.logits.float(), eager[i].float(), rtol=tol, atol=tol)
    mdl.carry_mode = "split"
