"""The torch.compile pass that turns sibling `nmsparse::gemv` calls into one
launch (spmv_decode_amd/compile_pass.py), on the CPU: which nodes it rewrites,
in graphs traced from the decoder in both layouts and in an inductor compile.
The GPU tests (test_gemv_gpu.py::test_compiled_unmodified_model_*) run the
rewritten graphs against eager."""
import operator

import pytest
import torch
import torch.nn.functional as F
from torch.fx.experimental.proxy_tensor import make_fx

from spmv_decode_amd import compile_pass
from spmv_decode_amd.decode.model import Decoder, init_weights_, tiny_config
from spmv_decode_amd.nmsparse_linear import NmSparseLinear, swap_to_nmsparse

OPS = torch.ops.nmsparse


def _counts(graph):
    c = {}
    for n in graph.nodes:
        if n.op == "call_function" and n.target in (OPS.gemv.default, OPS.gemv_grouped.default,
                                                    OPS.gemv_silu_mul.default):
            c[n.target._opname] = c.get(n.target._opname, 0) + 1
    return c


def _trace_step(model):
    """forward_step traced with fake tensors and inductor's decompositions (the
    form of graph the post-grad pass sees)."""
    from torch._inductor.decomposition import select_decomp_table

    model.setup_cache(8, "cpu", dtype=torch.float16)

    def step(token, pos):
        return model.forward_step(token, pos)

    with torch.no_grad():
        gm = make_fx(step, tracing_mode="fake", decomposition_table=select_decomp_table(),
                     _allow_non_fake_inputs=True)(
            torch.zeros(1, 1, dtype=torch.long), torch.tensor([3]))
    return gm


def _sparse_tiny(layout, qk_norm=False):
    cfg = tiny_config(qk_norm=qk_norm, n_layers=2)
    model = Decoder(cfg, layout=layout).half()
    init_weights_(model, seed=1)
    swap_to_nmsparse(model, 16, "cpu", seed=3, keep_dense=False)
    model.set_launch_mode("modules")
    return model.eval()


@pytest.mark.parametrize("layout,qk_norm", [("hf", False), ("hf", True), ("gpt-fast", False)])
def test_pass_rewrites_the_decoder_step(layout, qk_norm):
    """HF layout, each projection a module call: q/k/v become one grouped launch,
    gate/up one SiLU-gated pair launch; o and down stay single. gpt-fast layout:
    wqkv, wo and w2 stay single, w1/w3 become the pair. 4 launches per layer."""
    model = _sparse_tiny(layout, qk_norm)
    gm = _trace_step(model)
    L = model.cfg.n_layers
    per_layer = 7 if layout == "hf" else 5
    assert _counts(gm.graph) == {"gemv": per_layer * L}
    replaced = compile_pass.group_sibling_gemvs(gm.graph)
    gm.recompile()
    want = ({"gemv_grouped": L, "gemv_silu_mul": L, "gemv": 2 * L} if layout == "hf"
            else {"gemv_silu_mul": L, "gemv": 3 * L})
    assert _counts(gm.graph) == want
    assert replaced == (5 if layout == "hf" else 2) * L
    for n in gm.graph.nodes:  # every new node carries its fake value, as inductor's lowering needs
        if n.op == "call_function" and n.target in (OPS.gemv_grouped.default, OPS.gemv_silu_mul.default):
            assert "val" in n.meta
            if n.target is OPS.gemv_grouped.default:
                assert [len(n.args[1]), len(n.args[2])] == [3, 3] and list(n.args[4]) == [256, 128, 128]
                assert all(u.target is operator.getitem for u in n.users)


@pytest.mark.parametrize("layout,qk_norm", [("hf", False), ("hf", True), ("gpt-fast", False)])
def test_pass_folds_input_norms_and_residual_adds(layout, qk_norm):
    """After the grouping, the RMSNorm in front of q/k/v and of the gate/up pair
    folds into those launches (they read the residual stream with the norm's
    weight and eps; the norm's own nodes are gone), and each residual add
    after o and down folds into that gemv (gemv_residual). Left: the final
    norm before the dense lm_head and Qwen3's q/k norms."""
    model = _sparse_tiny(layout, qk_norm)
    gm = _trace_step(model)
    L = model.cfg.n_layers
    compile_pass.group_sibling_gemvs(gm.graph)
    assert compile_pass.fold_input_norms(gm.graph) == 2 * L
    assert compile_pass.fold_residuals(gm.graph) == 2 * L
    gm.recompile()
    assert _counts(gm.graph) == {"gemv_grouped": L, "gemv_silu_mul": L}
    res = [n for n in gm.graph.nodes if n.op == "call_function" and n.target is OPS.gemv_residual.default]
    assert len(res) == 2 * L and all("val" in n.meta for n in res)
    for n in gm.graph.nodes:
        if n.op == "call_function" and n.target in (OPS.gemv_grouped.default, OPS.gemv_silu_mul.default):
            assert n.args[-2] is not None and abs(n.args[-1] - model.cfg.norm_eps) < 1e-9
            assert n.args[0].meta["val"].dtype == torch.float16
    rsqrt = sum(1 for n in gm.graph.nodes if n.op == "call_function" and n.target is torch.ops.aten.rsqrt.default)
    assert rsqrt == 1 + (2 * L if qk_norm else 0)


def test_norm_and_residual_folds_need_their_exact_forms():
    """Norm forms as Hugging Face and gpt-fast write them fold too (weight after
    the rounding, x*x for the square); a norm whose weight is fp32, an add
    that broadcasts and a gemv with a second use stay as they are."""
    lin = NmSparseLinear(128, 64, 8, 1, "cpu")
    w16 = torch.rand(64).half()
    w32 = torch.rand(64)
    from torch._inductor.decomposition import select_decomp_table

    def hf_norm(x, w):
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)
        return w * h.to(x.dtype)

    def gpt_fast_norm(x, w):
        h = x.float()
        h = h * torch.rsqrt(torch.mean(h * h, dim=-1, keepdim=True) + 1e-5)
        return h.type_as(x) * w

    def trace(f, x):
        return make_fx(f, tracing_mode="fake", decomposition_table=select_decomp_table(),
                       _allow_non_fake_inputs=True)(x)

    x = torch.randn(1, 1, 64).half()
    for norm, w, folds in ((hf_norm, w16, 1), (gpt_fast_norm, w16, 1), (hf_norm, w32, 0)):
        gm = trace(lambda t: lin(norm(t, w)), x)
        assert compile_pass.fold_input_norms(gm.graph) == folds, (norm.__name__, w.dtype)
    r = torch.randn(1, 1, 128).half()
    gm = trace(lambda t: lin(t) + r, x)
    assert compile_pass.fold_residuals(gm.graph) == 1
    gm = trace(lambda t: lin(t) + r[..., :1], x)  # broadcasts
    assert compile_pass.fold_residuals(gm.graph) == 0
    gm = trace(lambda t: (lin(t) + r) * lin(t).sum(), x)
    before = sum(1 for n in gm.graph.nodes if n.op == "call_function")
    compile_pass.fold_residuals(gm.graph)  # two separate gemv calls: each used once, so the add folds
    assert sum(1 for n in gm.graph.nodes if n.op == "call_function") == before - 1

    def used_twice(t):
        y = lin(t)
        return (y + r) * y.sum()

    gm = trace(used_twice, x)
    assert compile_pass.fold_residuals(gm.graph) == 0


def test_pass_leaves_other_graphs_alone():
    """No gemv nodes, a single gemv, or siblings of different N:M or input:
    nothing to group."""
    a = NmSparseLinear(128, 64, 8, 1, "cpu")
    b = NmSparseLinear(128, 64, 16, 2, "cpu")

    def f(x, y):
        return a(x) + b(x) + a(y) + torch.sin(x).sum()

    gm = make_fx(f, tracing_mode="fake", _allow_non_fake_inputs=True)(torch.randn(1, 1, 64).half(), torch.randn(1, 1, 64).half())
    before = str(gm.graph)
    assert compile_pass.group_sibling_gemvs(gm.graph) == 0
    assert str(gm.graph) == before


def test_silu_pair_needs_exclusive_use_and_fp16():
    """The SiLU-gated pair is fused only when the two outputs are used for
    nothing else (else: one grouped launch), and only for fp16 inputs."""
    g = NmSparseLinear(128, 64, 8, 1, "cpu")
    u = NmSparseLinear(128, 64, 8, 2, "cpu")

    def used_twice(x):
        gx = g(x)
        return F.silu(gx) * u(x) + gx

    def pair(x):
        return F.silu(g(x)) * u(x)

    from torch._inductor.decomposition import select_decomp_table

    dt = select_decomp_table()
    gm = make_fx(used_twice, tracing_mode="fake", decomposition_table=dt, _allow_non_fake_inputs=True)(torch.randn(1, 1, 64).half())
    compile_pass.group_sibling_gemvs(gm.graph)
    assert _counts(gm.graph) == {"gemv_grouped": 1}
    gm = make_fx(pair, tracing_mode="fake", decomposition_table=dt, _allow_non_fake_inputs=True)(torch.randn(1, 1, 64).half())
    compile_pass.group_sibling_gemvs(gm.graph)
    assert _counts(gm.graph) == {"gemv_silu_mul": 1}
    gm = make_fx(pair, tracing_mode="fake", decomposition_table=dt, _allow_non_fake_inputs=True)(torch.randn(1, 1, 64).bfloat16())
    compile_pass.group_sibling_gemvs(gm.graph)
    assert _counts(gm.graph) == {"gemv_grouped": 1}


def test_installed_pass_runs_inside_inductor(monkeypatch):
    """Importing the package installs the pass as inductor's post-grad pre-pass;
    a full-graph inductor compile of sibling module calls gets the grouped and
    pair nodes, and the compiled code then calls the HIP ops, which refuse CPU
    tensors (no CPU fallback)."""
    import torch._inductor.config as ic

    assert isinstance(ic.post_grad_custom_pre_pass, compile_pass.SiblingGemvPass)
    seen = []
    real = compile_pass.group_sibling_gemvs

    def spy(graph):
        n = real(graph)
        seen.append(_counts(graph))
        return n

    monkeypatch.setattr(compile_pass, "group_sibling_gemvs", spy)
    monkeypatch.setattr(ic, "force_disable_caches", True)  # a cached compile would not run the pass again
    q, k, v = (NmSparseLinear(h, 128, 8, i, "cpu") for i, h in enumerate((256, 128, 128)))
    w1, w3, w2 = NmSparseLinear(256, 128, 8, 5, "cpu"), NmSparseLinear(256, 128, 8, 6, "cpu"), \
        NmSparseLinear(128, 256, 8, 7, "cpu")

    def block(x):
        a = torch.cat([q(x), k(x), v(x)], dim=-1)
        return w2(F.silu(w1(x)) * w3(x)) + a[..., :128]

    torch._dynamo.reset()
    try:
        with torch.inference_mode(), pytest.raises(ValueError, match="GPU"):
            torch.compile(block, fullgraph=True)(torch.randn(1, 1, 128).half())
    finally:
        torch._dynamo.reset()
    assert seen == [{"gemv_grouped": 1, "gemv_silu_mul": 1, "gemv": 1}]  # after the grouping, before the folds


def test_install_keeps_an_existing_pass_and_uninstall_restores_it(monkeypatch):
    import torch._inductor.config as ic

    calls = []
    monkeypatch.setattr(ic, "post_grad_custom_pre_pass", None)
    user = lambda graph: calls.append(graph)  # noqa: E731
    ic.post_grad_custom_pre_pass = user
    assert compile_pass.install()
    p = ic.post_grad_custom_pre_pass
    assert isinstance(p, compile_pass.SiblingGemvPass) and p.before is user
    assert compile_pass.install() and ic.post_grad_custom_pre_pass is p  # once
    p(torch.fx.Graph())
    assert len(calls) == 1
    assert p.uuid() is not None
    compile_pass.uninstall()
    assert ic.post_grad_custom_pre_pass is user
    monkeypatch.setattr(ic, "post_grad_custom_pre_pass", compile_pass.SiblingGemvPass())


def test_gpt_fast_layout_matches_hf_layout():
    """The gpt-fast-named decoder computes what the HF-named one does with the
    same weights (wqkv = [q; k; v], w1 = gate, w3 = up, w2 = down): decode
    steps and the one-pass prompt; swap_to_nmsparse walks it in gpt-fast's
    order (wqkv, wo, w1, w3, w2) and ties w1 / w3."""
    cfg = tiny_config(qk_norm=True)
    hf = Decoder(cfg)
    init_weights_(hf, seed=5)
    gf = Decoder(cfg, layout="gpt-fast")
    with torch.no_grad():
        gf.embed_tokens.weight.copy_(hf.embed_tokens.weight)
        gf.norm.weight.copy_(hf.norm.weight)
        gf.lm_head.weight.copy_(hf.lm_head.weight)
        for a, b in zip(hf.layers, gf.layers):
            at, ga = a.self_attn, b.attention
            ga.wqkv.weight.copy_(torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]))
            ga.wo.weight.copy_(at.o_proj.weight)
            ga.q_norm.weight.copy_(at.q_norm.weight)
            ga.k_norm.weight.copy_(at.k_norm.weight)
            b.feed_forward.w1.weight.copy_(a.mlp.gate_proj.weight)
            b.feed_forward.w3.weight.copy_(a.mlp.up_proj.weight)
            b.feed_forward.w2.weight.copy_(a.mlp.down_proj.weight)
            b.attention_norm.weight.copy_(a.input_layernorm.weight)
            b.ffn_norm.weight.copy_(a.post_attention_layernorm.weight)
    tokens = torch.randint(0, cfg.vocab, (7,), generator=torch.Generator().manual_seed(3))
    outs = []
    for model in (hf, gf):
        model.set_launch_mode("per_linear")
        model.setup_cache(16, "cpu", dtype=torch.float32)
        with torch.no_grad():
            steps = torch.cat([model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)])
            model.setup_cache(16, "cpu", dtype=torch.float32)
            pre = model.prefill(tokens)
        outs.append((steps, pre))
    torch.testing.assert_close(outs[1][0], outs[0][0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(outs[1][1], outs[0][1], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(outs[0][1], outs[0][0][-1:], rtol=1e-4, atol=1e-4)
    n = swap_to_nmsparse(gf, 8, "cpu", seed=0, keep_dense=False)
    assert n == 5 * cfg.n_layers
    ff = gf.layers[0].feed_forward
    assert ff.w1.__dict__["_siblings"].members == [ff.w1, ff.w3]
    ref = NmSparseLinear(ff.w3.h, cfg.dim, 8, 3, "cpu")  # seed + j: wqkv 0, wo 1, w1 2, w3 3
    assert torch.equal(ff.w3.mat_data, ref.mat_data) and torch.equal(ff.w3.mat_index, ref.mat_index)
