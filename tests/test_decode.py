"""The decode-step caller (f1): KV-cached single-token decode vs an independent
full-sequence reference, RoPE scaling, sparse swap, and hipGraph replay."""
import math

import pytest
import torch
import torch.nn.functional as F

from spmv_decode_amd import NmSparseLinear, swap_to_nmsparse
from spmv_decode_amd.decode.model import LLAMA31_8B, Decoder, init_weights_, rope_inv_freq, tiny_config


def _llama31_freqs_loop(cfg):
    """Per-frequency rule as published for Llama 3.1 rope scaling, in plain floats."""
    sc = cfg.rope_scaling
    out = []
    for i in range(cfg.head_dim // 2):
        f = 1.0 / (cfg.rope_theta ** (2 * i / cfg.head_dim))
        wl = 2 * math.pi / f
        lo_wl = sc["original_max_position_embeddings"] / sc["low_freq_factor"]
        hi_wl = sc["original_max_position_embeddings"] / sc["high_freq_factor"]
        if wl < hi_wl:
            out.append(f)
        elif wl > lo_wl:
            out.append(f / sc["factor"])
        else:
            s = (sc["original_max_position_embeddings"] / wl - sc["low_freq_factor"]) / (
                sc["high_freq_factor"] - sc["low_freq_factor"])
            out.append((1 - s) * f / sc["factor"] + s * f)
    return torch.tensor(out, dtype=torch.float64)


def test_rope_scaling_matches_published_rule():
    torch.testing.assert_close(rope_inv_freq(LLAMA31_8B), _llama31_freqs_loop(LLAMA31_8B), rtol=1e-12, atol=0)


def _reference_logits(model, tokens):
    """Full-sequence forward without a cache: causal attention recomputed over
    all tokens, GQA by repeating KV heads. Independent of forward_step."""
    c = model.cfg
    T = tokens.numel()
    x = model.embed_tokens(tokens.view(1, T))[0]  # [T, dim]
    inv = rope_inv_freq(c)
    ang = torch.outer(torch.arange(T, dtype=torch.float64), inv)
    cos, sin = ang.cos().float(), ang.sin().float()

    def rope(t):  # t [T, heads, hd]; rotate each (even, odd) pair by the position's angle
        a, b = t[..., 0::2], t[..., 1::2]
        ra = a * cos[:, None] - b * sin[:, None]
        rb = b * cos[:, None] + a * sin[:, None]
        return torch.stack((ra, rb), -1).flatten(-2)

    def rms(t, mod):
        return (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + mod.eps)) * mod.weight

    for blk in model.layers:
        at = blk.self_attn
        hn = rms(x, blk.input_layernorm)
        q = F.linear(hn, at.q_proj.weight).view(T, c.n_heads, c.head_dim)
        k = F.linear(hn, at.k_proj.weight).view(T, c.n_kv_heads, c.head_dim)
        v = F.linear(hn, at.v_proj.weight).view(T, c.n_kv_heads, c.head_dim)
        if c.qk_norm:
            q, k = rms(q, at.q_norm), rms(k, at.k_norm)
        q, k = rope(q), rope(k)
        rep = c.n_heads // c.n_kv_heads
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        s = torch.einsum("thd,shd->hts", q, k) / math.sqrt(c.head_dim)
        s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
        y = torch.einsum("hts,shd->thd", torch.softmax(s, -1), v).reshape(T, -1)
        x = x + F.linear(y, at.o_proj.weight)
        hn = rms(x, blk.post_attention_layernorm)
        mlp = blk.mlp
        x = x + F.linear(F.silu(F.linear(hn, mlp.gate_proj.weight)) * F.linear(hn, mlp.up_proj.weight),
                         mlp.down_proj.weight)
    return F.linear(rms(x, model.norm), model.lm_head.weight)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_cached_decode_matches_full_sequence_reference(qk_norm):
    torch.manual_seed(0)
    model = Decoder(tiny_config(qk_norm=qk_norm)).float()
    init_weights_(model, seed=1, std=0.05)
    T = 9
    tokens = torch.randint(0, model.cfg.vocab, (T,), generator=torch.Generator().manual_seed(2))
    model.setup_cache(16, "cpu", dtype=torch.float32)
    got = []
    with torch.no_grad():
        for t in range(T):
            got.append(model.forward_step(tokens[t].view(1, 1), torch.tensor([t]))[0])
        ref = _reference_logits(model, tokens)
    torch.testing.assert_close(torch.stack(got), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_prefill_matches_full_sequence_reference_and_steps(qk_norm):
    """Decoder.prefill (the prompt in one pass) against the independent
    full-sequence reference at the last position; its caches equal the ones
    the per-token steps write; the step after it gives the same logits."""
    torch.manual_seed(0)
    model = Decoder(tiny_config(qk_norm=qk_norm)).float()
    init_weights_(model, seed=4, std=0.05)
    T = 9
    tokens = torch.randint(0, model.cfg.vocab, (T,), generator=torch.Generator().manual_seed(6))
    hd = model.cfg.head_dim
    with torch.no_grad():
        ref = _reference_logits(model, tokens)
        model.setup_cache(16, "cpu", dtype=torch.float32)
        got = model.prefill(tokens)
        torch.testing.assert_close(got[0], ref[-1], rtol=1e-4, atol=1e-4)
        kv = ([k[:, :hd, :T].clone() for k in model.k_cache_t], [v[:, :, :T].clone() for v in model.v_cache_t])
        after = model.forward_step(tokens[:1].view(1, 1), torch.tensor([T]))
        model.setup_cache(16, "cpu", dtype=torch.float32)
        for t in range(T):
            model.forward_step(tokens[t].view(1, 1), torch.tensor([t]))
        for a, b in zip(kv[0], model.k_cache_t):
            torch.testing.assert_close(a, b[:, :hd, :T], rtol=1e-5, atol=1e-5)
        for a, b in zip(kv[1], model.v_cache_t):
            torch.testing.assert_close(a, b[:, :, :T], rtol=1e-5, atol=1e-5)
        step = model.forward_step(tokens[:1].view(1, 1), torch.tensor([T]))
        torch.testing.assert_close(after, step, rtol=1e-4, atol=1e-4)
        with pytest.raises(ValueError):
            model.prefill(torch.zeros(17, dtype=torch.long))


def test_linear_like_projection_modules_run_the_decoder():
    """Projections that are neither nn.Linear nor NmSparseLinear (e.g. a
    CPU gather-form module) go through their own forward: same logits as the
    dense model."""
    import torch.nn as nn

    class Wrapped(nn.Module):
        def __init__(self, lin):
            super().__init__()
            self.lin = lin

        def forward(self, x):
            return F.linear(x, self.lin.weight)

    torch.manual_seed(0)
    model = Decoder(tiny_config()).float()
    init_weights_(model, seed=3, std=0.05)
    model.setup_cache(8, "cpu", dtype=torch.float32)
    tokens = torch.tensor([5, 17, 300, 2])
    with torch.no_grad():
        ref = [model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)]
        for blk in model.layers:
            for sub, names in ((blk.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                               (blk.mlp, ("gate_proj", "up_proj", "down_proj"))):
                for n in names:
                    setattr(sub, n, Wrapped(getattr(sub, n)))
        model.setup_cache(8, "cpu", dtype=torch.float32)
        got = [model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)]
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_dense_fusion_modes_match_per_linear(qk_norm):
    """Dense q/k/v (and gate/up) as one GEMM give the per-Linear logits; the
    fused copies are dropped by "none" and ignored once a projection is swapped."""
    torch.manual_seed(0)
    model = Decoder(tiny_config(qk_norm=qk_norm)).float()
    init_weights_(model, seed=6, std=0.05)
    tokens = torch.tensor([7, 99, 3, 250, 41])

    def run():
        model.setup_cache(8, "cpu", dtype=torch.float32)
        with torch.no_grad():
            return torch.cat([model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)])

    ref = run()
    with pytest.raises(ValueError, match="dense fusion"):
        model.set_dense_fusion("all")
    model.set_dense_fusion("qkv")
    at, mlp = model.layers[0].self_attn, model.layers[0].mlp
    assert at.wqkv.shape == (at.q_proj.out_features + 2 * at.k_proj.out_features, model.cfg.dim)
    assert mlp.w13 is None and "wqkv" not in dict(model.named_parameters())
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)
    model.set_dense_fusion("qkv_gate_up")
    assert mlp.w13.shape == (2 * model.cfg.inter, model.cfg.dim)
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)
    # once a projection is replaced (as swap_to_nmsparse does), its block runs
    # the replacement, not the fused copy
    qd = at.q_proj.out_features

    class Zeroed(torch.nn.Module):
        def forward(self, x):
            return torch.zeros(*x.shape[:-1], qd, dtype=x.dtype)

    q_dense = at.q_proj
    at.q_proj = Zeroed()
    assert not torch.allclose(run(), ref, rtol=1e-3, atol=1e-3)
    at.q_proj = q_dense
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)
    model.set_dense_fusion("none")
    assert all(b.self_attn.wqkv is None and b.mlp.w13 is None for b in model.layers)


def test_dense_gemv_forms_agree_and_are_applied_per_shape():
    """Both dense_gemv forms compute x·Wᵀ (with and without out=); forms set per
    shape reach every site of that shape, the fused copies included, and the
    decoder's logits do not change."""
    from spmv_decode_amd.decode.model import GEMV_FORMS, dense_gemv

    g = torch.Generator().manual_seed(3)
    W, x = torch.randn(48, 80, generator=g), torch.randn(1, 80, generator=g)
    ref = x @ W.t()
    for form in GEMV_FORMS:
        torch.testing.assert_close(dense_gemv(x, W, form), ref, rtol=1e-5, atol=1e-5)
        out = torch.empty(1, 48)
        assert dense_gemv(x, W, form, out=out) is out
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
    model = Decoder(tiny_config(qk_norm=True)).float()
    init_weights_(model, seed=8, std=0.05)
    tokens = torch.tensor([3, 14, 159, 26])

    def run():
        model.setup_cache(8, "cpu", dtype=torch.float32)
        with torch.no_grad():
            return torch.cat([model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)])

    ref = run()
    c = model.cfg
    qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    model.gemv_forms = {(kvd, c.dim): "mv", (c.dim, c.inter): "mv", (c.vocab, c.dim): "mv",
                        (2 * c.inter, c.dim): "mv"}
    model.set_dense_fusion("qkv_gate_up")
    at, mlp = model.layers[1].self_attn, model.layers[1].mlp
    assert at.k_proj.gemv_form == at.v_proj.gemv_form == "mv" and mlp.down_proj.gemv_form == "mv"
    assert mlp.gate_proj.gemv_form == "mm" and model.lm_head.gemv_form == "mv"
    # the fused q/k/v copy takes the form of its own shape, which may coincide with another entry's
    assert mlp.w13_form == "mv" and at.wqkv_form == model.gemv_forms.get((qd + 2 * kvd, c.dim), "mm")
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)
    model.set_dense_fusion("none")
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(RuntimeError, match="on the GPU"):
        model.tune_dense_gemv()


def test_swap_applies_to_decoder_layout():
    model = Decoder(tiny_config())
    n = swap_to_nmsparse(model, 8, "cpu", seed=3, keep_dense=False)
    assert n == 7 * model.cfg.n_layers
    blk = model.layers[0]
    for mod in (blk.self_attn.q_proj, blk.self_attn.k_proj, blk.mlp.down_proj):
        assert isinstance(mod, NmSparseLinear) and mod.weight is None
    assert blk.self_attn.k_proj.h == model.cfg.n_kv_heads * model.cfg.head_dim


# ---------------------------------------------------------------------------
# GPU: graph replay and sparse vs masked-dense
# ---------------------------------------------------------------------------
def _masked_pair(cfg, M, seed=0):
    """A dense fp16 model whose Linear weights are N:M-masked, and the sparse
    model packed from exactly those weights (NmSparseLinear.from_dense)."""
    torch.manual_seed(seed)
    dense = Decoder(cfg).to("cuda", torch.float16)
    init_weights_(dense, seed=seed, std=0.05)
    sparse = Decoder(cfg).to("cuda", torch.float16)
    sparse.load_state_dict(dense.state_dict())
    g = torch.Generator(device="cuda").manual_seed(seed + 7)
    for bd, bs in zip(dense.layers, sparse.layers):
        for sub_d, sub_s, names in ((bd.self_attn, bs.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                                    (bd.mlp, bs.mlp, ("gate_proj", "up_proj", "down_proj"))):
            for name in names:
                lin = getattr(sub_d, name)
                N, K = lin.weight.shape
                keys = torch.rand(K // M, M, generator=g, device="cuda")
                mi = keys.argsort(1)[:, : M // 2].sort(1).values.to(torch.uint8)
                mask = torch.zeros(K // M, M, dtype=torch.bool, device="cuda")
                mask.scatter_(1, mi.long(), True)
                with torch.no_grad():
                    lin.weight.mul_(mask.view(1, K))
                setattr(sub_s, name, NmSparseLinear.from_dense(lin.weight.detach(), mi, M))
    return dense, sparse


@pytest.mark.gpu
def test_graph_replay_matches_eager_and_masked_dense(gpu):
    from spmv_decode_amd.decode.runner import GraphDecoder

    cfg = tiny_config(qk_norm=True)
    dense, sparse = _masked_pair(cfg, 8)
    sparse.carry_mode = "split"  # the bit-reproducible carry (the accumulated one varies in the last bits)
    prompt = torch.randint(0, cfg.vocab, (5,), generator=torch.Generator().manual_seed(3))
    # eager reference tokens and logits
    eager = GraphDecoder(sparse, 32)
    eager.run_prompt(prompt)
    eager_logits = [eager.eager_step().clone() for _ in range(6)]
    eager_tokens = eager.tokens[: eager.host_pos + 1].clone()
    # the dense masked model, eager, same tokens
    dref = GraphDecoder(dense, 32)
    dref.run_prompt(prompt)
    dense_logits = [dref.eager_step().clone() for _ in range(6)]
    for a, b in zip(eager_logits, dense_logits):
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=2e-2)
    # graph replays of the sparse model, three times over, bit-identical to eager
    gd = GraphDecoder(sparse, 32)
    gd.capture()
    for rep in range(3):
        gd.run_prompt(prompt)
        logits = []
        for _ in range(6):
            gd.replay()
            logits.append(gd.logits.clone())
        torch.cuda.synchronize()
        assert torch.equal(gd.tokens[: gd.host_pos + 1], eager_tokens), rep
        for a, b in zip(logits, eager_logits):
            assert torch.equal(a, b), rep
    with pytest.raises(RuntimeError, match="static cache"):
        gd.generate(64)


@pytest.mark.gpu
@pytest.mark.parametrize("prompt_len", [5, 24, 70])
def test_sparse_prefill_matches_per_token_prompt(gpu, prompt_len):
    """The sparse model's one-pass prompt (every projection through the SpMM:
    5 rows on the small-batch kernel, 24 on the matrix cores, 70 on gather +
    hipBLASLt: products of at most 1024 outputs past 64 rows) against
    feeding the prompt one step at a time: last-position logits and the KV
    caches within fp16 tolerance, and the masked dense twin's prefill within
    the same tolerance; decoding after either continues with the same logits
    (graph replay)."""
    from spmv_decode_amd.decode.runner import GraphDecoder

    cfg = tiny_config(qk_norm=True)
    dense, sparse = _masked_pair(cfg, 8)
    prompt = torch.randint(0, cfg.vocab, (prompt_len,), generator=torch.Generator().manual_seed(prompt_len))
    hd = cfg.head_dim
    step = GraphDecoder(sparse, 96)
    step.run_prompt(prompt)
    step_logits = step.logits.clone()
    caches = ([k[:, :hd, :prompt_len].clone() for k in sparse.k_cache_t],
              [v[:, :, :prompt_len].clone() for v in sparse.v_cache_t])
    nxt_step = [step.eager_step().clone() for _ in range(3)]
    one = GraphDecoder(sparse, 96)
    one.capture()
    one.run_prompt(prompt, batched=True)
    torch.testing.assert_close(one.logits.float(), step_logits.float(), rtol=2e-2, atol=2e-2)
    assert int(one.pos) == prompt_len and one.host_pos == prompt_len
    for a, b in zip(caches[0], sparse.k_cache_t):
        torch.testing.assert_close(a.float(), b[:, :hd, :prompt_len].float(), rtol=2e-2, atol=2e-2)
    for a, b in zip(caches[1], sparse.v_cache_t):
        torch.testing.assert_close(a.float(), b[:, :, :prompt_len].float(), rtol=2e-2, atol=2e-2)
    if int(one.token) == int(step.tokens[prompt_len]):  # same first token: the continuations compare
        nxt_one = []
        for _ in range(3):
            one.replay()
            nxt_one.append(one.logits.clone())
        torch.cuda.synchronize()
        for a, b in zip(nxt_one, nxt_step):
            torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=2e-2)
    dref = GraphDecoder(dense, 96)
    dref.run_prompt(prompt, batched=True)
    torch.testing.assert_close(dref.logits.float(), step_logits.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("fusion", ["none", "qkv", "qkv_gate_up"])
def test_tuned_dense_decode_replays_match_eager(gpu, fusion):
    """The dense baseline as the decode benchmark runs it (fused copies, GEMV
    forms tuned on the GPU): logits within fp16 tolerance of the untuned
    per-Linear model, graph replays bit-identical to eager, three times over."""
    from spmv_decode_amd.decode.model import GEMV_FORMS
    from spmv_decode_amd.decode.runner import GraphDecoder

    cfg = tiny_config(qk_norm=True)
    torch.manual_seed(0)
    model = Decoder(cfg).to("cuda", torch.float16)
    init_weights_(model, seed=9, std=0.05)
    prompt = torch.randint(0, cfg.vocab, (4,), generator=torch.Generator().manual_seed(5))
    base = GraphDecoder(model, 32)
    base.run_prompt(prompt)
    ref = [base.eager_step().clone() for _ in range(5)]
    del base
    model.set_dense_fusion(fusion)
    report = model.tune_dense_gemv(reps=3, warmup=1)
    assert report and all(r["form"] in GEMV_FORMS and r["mm"] > 0 and r["mv"] > 0 for r in report.values())
    assert model.tune_dense_gemv() == {}  # every shape already tuned
    eager = GraphDecoder(model, 32)
    eager.run_prompt(prompt)
    eager_logits = [eager.eager_step().clone() for _ in range(5)]
    for a, b in zip(eager_logits, ref):
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=2e-2)
    gd = GraphDecoder(model, 32)
    gd.capture()
    for rep in range(3):
        gd.run_prompt(prompt)
        for i in range(5):
            gd.replay()
            torch.cuda.synchronize()
            assert torch.equal(gd.logits, eager_logits[i]), (rep, i)


@pytest.mark.gpu
def test_fixed_context_protocol_dense_and_sparse(gpu):
    """The reference benchmark's protocol (one step at a fixed position over
    random-filled caches, replayed): finite logits, and an eager step at the
    same position afterwards picks the token the replays picked."""
    from spmv_decode_amd.decode.runner import fixed_context_ms

    cfg = tiny_config(qk_norm=True)
    torch.manual_seed(0)
    model = Decoder(cfg).to("cuda", torch.float16)
    init_weights_(model, seed=2, std=0.05)
    for sparse in (False, True):
        if sparse:
            swap_to_nmsparse(model, 16, "cuda", seed=3, init="device", keep_dense=False)
        r = fixed_context_ms(model, 20, warmup=2, repeat=3, inner=2)
        assert r["finite_logits"] and r["median"] > 0 and len(r["samples"]) == 3
        with torch.no_grad():
            logits = model.forward_step(torch.tensor([[123]], device="cuda"), torch.tensor([20], device="cuda"))
        assert int(torch.argmax(logits, dim=-1)) == r["token"], sparse


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [20, 300])
def test_compiled_step_is_one_graph_and_matches_eager(gpu, ctx):
    """The reference benchmark compiles the decode step before capturing it
    (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:152-155). The fused sparse
    step, whose launches are torch.ops.nmsparse ops, compiles with
    fullgraph=True (no graph break), and so does the dense step; under the
    fixed-context protocol (with the reference's sampling) the compiled step's
    logits match the eager step's within fp16 tolerance and pick the same
    greedy token wherever the top two logits are apart by more than that; at
    20 and at 300 positions (a cache of 384: the compiled attention's
    reduction over the positions)."""
    from spmv_decode_amd.decode.runner import fixed_context_ms

    cfg = tiny_config(qk_norm=True)
    torch.manual_seed(0)
    model = Decoder(cfg).to("cuda", torch.float16)
    init_weights_(model, seed=2, std=0.05)
    eager_step = model.forward_step
    for sparse in (False, True):
        if sparse:
            swap_to_nmsparse(model, 16, "cuda", seed=3, init="device", keep_dense=False)
        ref = fixed_context_ms(model, ctx, warmup=2, repeat=2, inner=2)
        torch._dynamo.reset()
        model.forward_step = torch.compile(eager_step, dynamic=False, fullgraph=True)
        try:
            got = fixed_context_ms(model, ctx, warmup=2, repeat=2, inner=2)
        finally:
            model.forward_step = eager_step
            torch._dynamo.reset()
        assert got["finite_logits"] and got["sampling"] == "categorical" and 0 <= got["sampled_token"] < cfg.vocab
        torch.testing.assert_close(got["logits"], ref["logits"], rtol=2e-2, atol=2e-2)
        top2 = torch.topk(ref["logits"].view(-1), 2).values
        if float(top2[0] - top2[1]) > 4e-2:
            assert got["token"] == ref["token"], sparse


def test_compiled_module_step_writes_the_caches_like_eager():
    """torch.compile of the module-by-module step (fp32 on the CPU): the key
    goes into the cache through the mutating op nmsparse_decode::cache_write,
    which the compiler runs in place (indexing into a view of the one
    key-cache tensor made it copy the view out and back around the write).
    Four steps compiled give the eager steps' logits, and the key caches
    (mask rows included) and value caches end up the same."""
    cfg = tiny_config(n_layers=2)
    model = Decoder(cfg).float()
    init_weights_(model, seed=0)
    tokens = [3, 7, 11, 5]

    def run(step):
        model.setup_cache(64, "cpu", dtype=torch.float32)
        with torch.no_grad():
            logits = [step(torch.tensor([[t]]), torch.tensor([i])) for i, t in enumerate(tokens)]
        return logits, model.k_store.clone(), [v.clone() for v in model.v_cache_t]

    eager, k_eager, v_eager = run(model.forward_step)
    torch._dynamo.reset()
    try:
        from torch._inductor.utils import run_and_get_code

        step = torch.compile(model.forward_step, dynamic=False, fullgraph=True)
        model.setup_cache(64, "cpu", dtype=torch.float32)
        with torch.no_grad():
            _, code = run_and_get_code(step, torch.tensor([[1]]), torch.tensor([0]))
        assert sum(c.count("nmsparse_decode.cache_write") for c in code) >= cfg.n_layers
        compiled, k_comp, v_comp = run(step)
    finally:
        torch._dynamo.reset()
    for a, b in zip(eager, compiled):
        torch.testing.assert_close(b, a, rtol=1e-5, atol=1e-5)
    assert torch.equal(torch.isinf(k_comp), torch.isinf(k_eager))
    torch.testing.assert_close(k_comp.nan_to_num(0.0, 0.0, 0.0), k_eager.nan_to_num(0.0, 0.0, 0.0), rtol=1e-5, atol=1e-5)
    for a, b in zip(v_eager, v_comp):
        torch.testing.assert_close(b, a, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_restored_compressed_checkpoint_decodes_identically(gpu):
    """A swapped model saved with torch.save and restored into a fresh
    skeleton (weights_only load) produces bit-identical logits."""
    import io

    cfg = tiny_config(qk_norm=True)
    torch.manual_seed(0)
    a = Decoder(cfg).to("cuda", torch.float16)
    init_weights_(a, seed=4, std=0.05)
    swap_to_nmsparse(a, 16, "cuda", seed=5, init="device", keep_dense=False)
    buf = io.BytesIO()
    torch.save(a.state_dict(), buf)
    buf.seek(0)
    b = Decoder(cfg).to("cuda", torch.float16)
    swap_to_nmsparse(b, 16, "cuda", seed=77, init="device", keep_dense=False)
    b.load_state_dict(torch.load(buf, weights_only=True))
    outs = []
    for mdl in (a, b):
        mdl.carry_mode = "split"  # bit-reproducible run to run
        mdl.setup_cache(8, "cuda", dtype=torch.float16)
        with torch.no_grad():
            outs.append([mdl.forward_step(torch.tensor([[t]], device="cuda"), torch.tensor([i], device="cuda"))
                         for i, t in enumerate((1, 2, 3))])
    for x, y in zip(*outs):
        assert torch.equal(x, y)


def test_launch_modes_are_validated_and_applied():
    model = Decoder(tiny_config())
    with pytest.raises(ValueError, match="launch mode"):
        model.set_launch_mode("fast")
    model.set_launch_mode("per_linear")
    assert not model.fuse_epilogues and not model.layers[0].self_attn.group_launches
    assert not model.layers[0].self_attn.call_modules
    model.set_launch_mode("grouped")
    assert not model.fuse_epilogues and model.layers[1].mlp.group_launches
    model.set_launch_mode("modules")
    at, mlp = model.layers[1].self_attn, model.layers[1].mlp
    assert not model.fuse_epilogues and not at.group_launches and at.call_modules and mlp.call_modules
    model.set_launch_mode("fused")
    assert model.fuse_epilogues and not at.call_modules


def test_modules_mode_runs_the_same_dense_model():
    """"modules" calls every projection as a module; on a dense model it computes
    the per-Linear logits."""
    torch.manual_seed(0)
    model = Decoder(tiny_config(qk_norm=True)).float()
    init_weights_(model, seed=12, std=0.05)
    tokens = torch.tensor([9, 8, 400, 33])

    def run():
        model.setup_cache(8, "cpu", dtype=torch.float32)
        with torch.no_grad():
            return torch.cat([model.forward_step(t.view(1, 1), torch.tensor([i])) for i, t in enumerate(tokens)])

    model.set_launch_mode("per_linear")
    ref = run()
    model.set_launch_mode("modules")
    torch.testing.assert_close(run(), ref, rtol=1e-5, atol=1e-5)


def test_swap_ties_the_siblings_of_each_layout():
    """q/k/v and gate/up (gpt-fast: w1/w3) of each block become one sibling group;
    the group is neither a submodule nor in the state_dict; untie_siblings drops it;
    tie=False leaves every Linear on its own."""
    import torch.nn as nn

    from spmv_decode_amd.nmsparse_linear import SiblingLaunch, untie_siblings

    model = Decoder(tiny_config())
    swap_to_nmsparse(model, 8, "cpu", seed=1, keep_dense=False)
    for blk in model.layers:
        at, mlp = blk.self_attn, blk.mlp
        g = at.q_proj.__dict__["_siblings"]
        assert isinstance(g, SiblingLaunch) and g.members == [at.q_proj, at.k_proj, at.v_proj]
        assert at.k_proj.__dict__["_siblings"] is g and "_siblings" not in at.o_proj.__dict__
        g2 = mlp.up_proj.__dict__["_siblings"]
        assert g2.members == [mlp.gate_proj, mlp.up_proj] and "_siblings" not in mlp.down_proj.__dict__
    assert all(not isinstance(m, SiblingLaunch) for m in model.modules())
    model2 = Decoder(tiny_config())
    swap_to_nmsparse(model2, 8, "cpu", seed=1, keep_dense=False, tie=False)
    assert all("_siblings" not in m.__dict__ for m in model2.modules())
    sd, sd2 = model.state_dict(), model2.state_dict()
    assert list(sd) == list(sd2)  # ties add no state; the swapped buffers are the same seeded draws
    assert all(torch.equal(sd[k], sd2[k]) for k in sd if ".mat_" in k)
    assert untie_siblings(model) == 5 * model.cfg.n_layers
    assert all("_siblings" not in m.__dict__ for m in model.modules())

    class GptFastBlock(nn.Module):  # gpt-fast's layout: fused wqkv, MLP w1/w3/w2
        def __init__(self):
            super().__init__()
            self.attention = nn.Module()
            self.attention.wqkv, self.attention.wo = nn.Linear(128, 384, bias=False), nn.Linear(128, 128, bias=False)
            self.feed_forward = nn.Module()
            ff = self.feed_forward
            ff.w1, ff.w3 = nn.Linear(128, 256, bias=False), nn.Linear(128, 256, bias=False)
            ff.w2 = nn.Linear(256, 128, bias=False)

    stack = nn.Module()
    stack.layers = nn.ModuleList([GptFastBlock(), GptFastBlock()])
    assert swap_to_nmsparse(stack, 8, "cpu", seed=0, keep_dense=False) == 10
    ff = stack.layers[1].feed_forward
    assert ff.w1.__dict__["_siblings"].members == [ff.w1, ff.w3]
    assert "_siblings" not in stack.layers[1].attention.wqkv.__dict__
    with pytest.raises(ValueError, match="same K"):
        from spmv_decode_amd.nmsparse_linear import tie_siblings
        tie_siblings(ff.w1, ff.w2)


def test_sibling_bookkeeping_under_inference_mode_and_the_waste_warning(monkeypatch):
    """The sibling group's host bookkeeping with the grouped launch replaced by a
    CPU stand-in (the launch itself needs a GPU): inference tensors, which have
    no version counter, are matched by identity (the reference's benchmarks run
    under torch.inference_mode(): benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:87),
    so q/k/v of one input are one launch there too; a launch that leaves outputs
    unclaimed before the next one warns once (siblings fed different inputs)."""
    import warnings

    from spmv_decode_amd import hip_spmv
    from spmv_decode_amd.nmsparse_linear import NmSparseLinear, SiblingLaunch, tie_siblings

    mods = [NmSparseLinear(h, 64, 8, 40 + i, "cpu") for i, h in enumerate((128, 256, 128))]
    dense = [m.to_dense(torch.float32) for m in mods]
    launches = []

    def grouped(vec, problems, nnz, m, outs):
        launches.append(vec)
        for (md, mi), o in zip(problems, outs):
            j = next(k for k, mod in enumerate(mods) if mod.mat_data is md)
            o.copy_((vec.float() @ dense[j].t()).to(o.dtype))
        return outs

    monkeypatch.setattr(hip_spmv, "nmsparse_gemv_grouped", grouped)
    monkeypatch.setattr(SiblingLaunch, "_usable", lambda self, x: True)
    tie_siblings(*mods)
    g = torch.Generator().manual_seed(0)
    with torch.inference_mode():
        x = torch.randn(1, 1, 64, generator=g).half()
        assert x.is_inference()
        outs = [m(x) for m in mods]  # no "Inference tensors do not track version counter"
        assert len(launches) == 1
        for o, d in zip(outs, dense):
            assert torch.equal(o.view(-1), (x.view(1, -1).float() @ d.t()).half().view(-1))
        x2 = torch.randn(1, 1, 64, generator=g).half()
        with warnings.catch_warnings():
            warnings.simplefilter("error")  # every output was claimed: no warning
            mods[1](x2), mods[0](x2), mods[2](x2)
        assert len(launches) == 2
    # outside inference mode the version counter still guards against in-place changes
    x3 = torch.randn(1, 1, 64, generator=g).half()
    mods[0](x3)
    x3.mul_(2)
    with pytest.warns(RuntimeWarning, match="streamed for nothing"):
        y = mods[1](x3)  # relaunch: k and v of the first launch were never claimed
    assert len(launches) == 4
    assert torch.equal(y.view(-1), (x3.view(1, -1).float() @ dense[1].t()).half().view(-1))
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # warned once per group
        mods[0](x3.clone()), mods[0](x3.clone())
    assert len(launches) == 6


@pytest.mark.parametrize("V", [128256, 151936, 512, 1000, 97])
def test_greedy_token_matches_argmax_with_ties(V):
    """The two-stage greedy argmax returns torch.argmax's index (the first
    occurrence of the maximum), also when the maximum repeats across chunks."""
    from spmv_decode_amd.decode.runner import greedy_token

    g = torch.Generator().manual_seed(V)
    for trial in range(6):
        logits = torch.randn(1, V, generator=g).half()
        if trial >= 2:  # plant the maximum at several positions (first one wins)
            k = 2 + trial
            pos = torch.randperm(V, generator=g)[:k]
            logits[0, pos] = 30.0
        if trial == 5:
            logits.fill_(1.0)  # all equal: index 0
        assert int(greedy_token(logits)) == int(torch.argmax(logits, dim=-1)), (V, trial)
        out = torch.full((1,), -1, dtype=torch.long)
        assert greedy_token(logits, out=out) is out and int(out) == int(torch.argmax(logits, dim=-1)), (V, trial)


def test_cache_length_rounds_up_to_the_alignment():
    from spmv_decode_amd.decode.runner import CACHE_ALIGN, cache_length

    assert CACHE_ALIGN == 128
    assert [cache_length(n) for n in (1, 127, 128, 129, 384, 392, 1024, 1032)] == \
        [128, 128, 128, 256, 384, 512, 1024, 1152]


@pytest.mark.gpu
def test_greedy_token_in_a_captured_graph(gpu):
    """The two-stage greedy argmax at Llama-3.1's vocabulary, captured in a
    hipGraph and replayed over new logits, equals torch.argmax each time."""
    from spmv_decode_amd.decode.runner import greedy_token

    V = 128256
    logits = torch.randn(1, V, device="cuda").half()
    out = torch.zeros(1, dtype=torch.long, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out.copy_(greedy_token(logits))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out.copy_(greedy_token(logits))
    gen = torch.Generator(device="cuda").manual_seed(0)
    for rep in range(4):
        logits.copy_(torch.randn(1, V, generator=gen, device="cuda").half())
        if rep == 3:
            logits[0, 5000] = logits[0, 90000] = 40.0  # a repeated maximum: the first one wins
        g.replay()
        torch.cuda.synchronize()
        assert int(out) == int(torch.argmax(logits, dim=-1)), rep


def test_sample_token_draws_from_the_softmax_distribution():
    """The exponential race (argmax p / E, E ~ Exp(1)) samples Categorical(softmax(logits)):
    on the CPU, 40000 draws over 5 classes land within 5 standard errors of the
    softmax probabilities (a wrong race, e.g. argmax p * E or argmax E, does not)."""
    from spmv_decode_amd.decode.runner import sample_token

    logits = torch.tensor([[2.0, 1.0, 0.0, -1.0, 0.5]]).half()
    p = torch.softmax(logits.float(), dim=-1).half().float().view(-1)
    p = p / p.sum()
    g = torch.Generator().manual_seed(7)
    n = 40000
    counts = torch.zeros(5)
    out = torch.zeros(1, dtype=torch.long)
    for _ in range(n):
        counts[int(sample_token(logits, out, generator=g))] += 1
    freq = counts / n
    se = (p * (1 - p) / n).sqrt()
    assert ((freq - p).abs() <= 5 * se).all(), (freq, p)


@pytest.mark.parametrize("V", [151936, 128256, 1009])
def test_softmax_row_matches_torch_softmax(V):
    """The sampling step's two-stage softmax equals torch.softmax in fp32 up to
    the order of its sums (a prime vocabulary takes torch.softmax itself), and
    sums to one; an omitted max shift or a sum over one chunk only would not."""
    from spmv_decode_amd.decode.runner import softmax_row

    logits = (torch.randn(1, V, generator=torch.Generator().manual_seed(V)) * 4).half()
    logits[0, V // 3] = 30.0
    got = softmax_row(logits)
    want = torch.softmax(logits.float(), dim=-1)
    assert got.dtype == torch.float32 and got.shape == (1, V)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-9)
    assert abs(float(got.sum()) - 1.0) < 1e-5


@pytest.mark.gpu
def test_sample_token_in_a_captured_graph_over_many_replays(gpu):
    """sample_token captured in a hipGraph at Qwen3's vocabulary (151936) and replayed
    400 times, eager multi-block reductions and synchronisations between replays:
    a dominant logit is drawn every time, and two equal logits split about evenly
    (within 5 standard errors); no replay asserts or faults."""
    from spmv_decode_amd.decode.runner import sample_token

    V = 151936
    logits = torch.randn(1, V, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1)).half()
    out = torch.zeros(1, dtype=torch.long, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sample_token(logits, out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sample_token(logits, out)
    big = torch.randn(1 << 22, device="cuda")
    for case, (hot, n) in enumerate((([777], 200), ([5, 150000], 400))):
        logits.copy_(torch.randn(1, V, device="cuda").half())
        logits[0, hot] = 40.0  # the rest is negligible: exp(-40) per token
        counts = {}
        for rep in range(n):
            g.replay()
            torch.cuda.synchronize()
            t = int(out)
            counts[t] = counts.get(t, 0) + 1
            if rep % 50 == 0:
                assert torch.isfinite(big.sum())  # eager multi-block work between replays
        assert set(counts) <= set(hot), (case, counts)
        if len(hot) == 2:
            se = (0.25 / n) ** 0.5
            assert abs(counts.get(hot[0], 0) / n - 0.5) <= 5 * se, counts


def test_carry_is_chosen_only_where_the_plans_take_it():
    """carry_supported (host-only planning, no kernel runs): the swapped tiny
    decoder can carry o_proj's and down_proj's split-K sums into the next
    launch; a dense decoder, a decoder whose layers differ in shape, and an
    M that is not a multiple of 4 cannot. The buffers are only set up on a GPU
    device (prepare_decode)."""
    from spmv_decode_amd.decode.model import carry_supported

    cfg = tiny_config()
    dense = Decoder(cfg)
    assert not carry_supported(dense.layers)
    sparse = Decoder(cfg)
    swap_to_nmsparse(sparse, 8, "cpu", seed=1, keep_dense=False)
    assert carry_supported(sparse.layers)
    odd = Decoder(cfg)
    swap_to_nmsparse(odd, 8, "cpu", seed=1, keep_dense=False)
    odd.layers[1].mlp.down_proj = NmSparseLinear.empty(cfg.dim, 2 * cfg.inter, 8, "cpu")
    assert not carry_supported(odd.layers)
    m2 = Decoder(cfg)
    swap_to_nmsparse(m2, 2, "cpu", seed=1, keep_dense=False)  # 1:2, M = 2
    assert not carry_supported(m2.layers)
    sparse.setup_cache(16, "cpu", dtype=torch.float32)
    assert sparse._carry is not None and sparse._carry[1] is None  # no carry buffers off the GPU
    # the buffers' key follows what the plans depend on: repacked as 2:4 instead of 4:8 (the packed
    # weights keep their shapes at half density), the decision is taken again
    key = sparse._carry[0]
    for blk in sparse.layers:
        for lin in (blk.self_attn.q_proj, blk.self_attn.k_proj, blk.self_attn.v_proj, blk.self_attn.o_proj,
                    blk.mlp.gate_proj, blk.mlp.up_proj, blk.mlp.down_proj):
            assert (lin.block_width, lin.vec_width) == (4, 8)
            lin.block_width, lin.vec_width = 2, 4
            lin.mat_index = lin.mat_index.reshape(-1, 2)
    sparse.prepare_decode()
    assert sparse._carry[0] != key


def test_fixed_context_fp32_reference_and_envelope():
    """The fp32 reference of the fixed-context step (runner.fixed_context_logits_fp32)
    of a sparse model is its masked dense twin's step in fp32 on the same cache
    values, and the model comes back unchanged (fp16, its NmSparseLinear
    modules and ties); logits_envelope accepts what rounds like the eager step
    and rejects a planted error."""
    from spmv_decode_amd.decode.runner import _fill_fixed_context, fixed_context_logits_fp32, logits_envelope
    from spmv_decode_amd.nmsparse_linear import NmSparseLinear

    cfg = tiny_config(qk_norm=True)
    model = Decoder(cfg).half()
    init_weights_(model, seed=2)
    swap_to_nmsparse(model, 8, "cpu", seed=4, keep_dense=False)
    before = {k: v.clone() for k, v in model.state_dict().items()}
    ref = fixed_context_logits_fp32(model, 20, device="cpu")
    after = model.state_dict()
    assert list(after) == list(before) and all(torch.equal(after[k], before[k]) for k in before)
    assert after["layers.0.self_attn.q_proj.mat_data"].dtype == torch.float16
    assert isinstance(model.layers[0].mlp.up_proj, NmSparseLinear)
    assert model.layers[0].mlp.up_proj.__dict__["_siblings"].members[0] is model.layers[0].mlp.gate_proj
    # the same step by hand: an fp32 dense twin on the same (fp16-drawn) caches
    twin = Decoder(cfg)
    sd = {k: v.float() for k, v in before.items() if ".mat_" not in k}
    for i, blk in enumerate(model.layers):
        for sub, names in (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
                           ("mlp", ("gate_proj", "up_proj", "down_proj"))):
            for n in names:
                sd[f"layers.{i}.{sub}.{n}.weight"] = getattr(getattr(blk, sub), n).to_dense(torch.float32)
    twin.load_state_dict(sd)
    _fill_fixed_context(model, 20, 1234, torch.device("cpu"))
    keys, vals = model.k_store[:, :, :cfg.head_dim].float(), [v.float() for v in model.v_cache_t]
    twin.setup_cache(model.max_seq, "cpu", dtype=torch.float32)
    twin.k_store[:, :, :cfg.head_dim].copy_(keys)
    for v, s in zip(twin.v_cache_t, vals):
        v.copy_(s)
    with torch.no_grad():
        want = twin.forward_step(torch.full((1, 1), 123), torch.tensor([20]))
    torch.testing.assert_close(ref, want, rtol=1e-6, atol=1e-6)
    # the envelope: an fp16 rounding of the reference passes, a planted error does not
    e16 = ref.half().float() + 1e-3 * torch.randn(ref.shape, generator=torch.Generator().manual_seed(0))
    ok = logits_envelope(e16, ref.half().float(), ref)
    assert ok["within"] and ok["same_greedy_token"] in (True, False)
    bad = ref.clone()
    bad[0, :50] += 10 * ref.abs().max()
    assert not logits_envelope(e16, bad, ref)["within"]
