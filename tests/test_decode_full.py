"""Decode parity at the benchmark configurations themselves (the decode workloads):
Llama-3.1-8B at 32:64 (32 layers), Qwen3-14B at 32:64 (40 layers) and at 8:16 /
128:256 (4 layers), Qwen3-32B at 16:32 (64 layers), random-init, fp16, batch 1.

For each: a short prompt and 8 greedy steps of the fused sparse model, eager and
then by hipGraph replay (tokens and logits bit-identical, the reference harness's
finiteness guards at benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:141-142,
164-165,181-182 included); then that token sequence teacher-forced through every
launch structure of the sparse model (fused, per-Linear, grouped) and through
its masked dense twins (every projection replaced by NmSparseLinear.to_dense:
the same weights scattered to dense, run by hipBLASLt) in fp16 and in fp32.

Tolerance (fp16): the fp32 dense twin is the reference. The fp16 dense twin's
distance from it (relative L2 of the logits, worst step) is what fp16 storage
and rounding alone cost at this depth; every fp16 sparse structure must stay
within twice that plus 1e-3, and two fp16 structures within three times that
plus 1e-3 of each other. A wrong index, term or fusion moves the logits by
orders of magnitude more.

The configurations' own context lengths (test_decode_parity_at_the_configs_context):
Llama-3.1-8B 32:64 with config 3's 128-token prompt in a 384-position cache and
Qwen3-32B 16:32 with config 5's 512-token prompt in a 1024-position cache; the
prompt through Decoder.prefill (every sparse Linear through the SpMM), then
graph-replayed steps at positions 128+ / 512+, bitwise equal to the eager steps
from the same caches, and every launch structure and both dense twins, each
prefilled the same way, held to the same envelope at those positions.
"""
import dataclasses
import gc

import pytest
import torch
import torch.nn as nn

from conftest import say
from spmv_decode_amd import NmSparseLinear, swap_to_nmsparse
from spmv_decode_amd.decode.model import CONFIGS, Decoder, RMSNorm
from spmv_decode_amd.decode.runner import GraphDecoder, cache_length

pytestmark = pytest.mark.gpu

PROJECTIONS = (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
               ("mlp", ("gate_proj", "up_proj", "down_proj")))
PROMPT, STEPS = 8, 8


def _free():
    gc.collect()
    torch.cuda.empty_cache()


def _set_param(model, name, tensor):
    mod_name, _, leaf = name.rpartition(".")
    model.get_submodule(mod_name)._parameters[leaf] = nn.Parameter(tensor, requires_grad=False)


def sparse_model(cfg, M, seed):
    """The decoder with every projection swapped to NmSparseLinear (synthetic
    on-device patterns, as the decode benchmark builds it), built without ever
    allocating the dense projections; embeddings, lm_head N(0, 0.02), norm
    weights 1 + N(0, 0.1) (so the fused norms see non-trivial weights)."""
    with torch.device("meta"):
        model = Decoder(cfg)
    n = swap_to_nmsparse(model, M, "cuda", seed=seed, init="device", keep_dense=False)
    assert n == 7 * cfg.n_layers
    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    for name, p in list(model.named_parameters()):
        assert p.is_meta, name
        t = torch.empty(p.shape, dtype=torch.float16, device="cuda")
        owner = model.get_submodule(name.rpartition(".")[0])
        if isinstance(owner, RMSNorm):
            t.normal_(1.0, 0.1, generator=gen)
        else:
            t.normal_(0.0, 0.02, generator=gen)
        _set_param(model, name, t)
    return model.eval()


def dense_twin(sparse, dtype):
    """The same model with every projection a dense nn.Linear holding the sparse
    module's weights scattered to dense (zeros at pruned positions), in dtype."""
    with torch.device("meta"):
        twin = Decoder(sparse.cfg)
    for name, p in sparse.named_parameters():
        _set_param(twin, name, p.detach().to(dtype))
    for i, blk in enumerate(sparse.layers):
        for sub, names in PROJECTIONS:
            for n in names:
                lin = getattr(getattr(blk, sub), n)
                assert isinstance(lin, NmSparseLinear)
                _set_param(twin, f"layers.{i}.{sub}.{n}.weight", lin.to_dense(dtype))
    assert not any(p.is_meta for p in twin.parameters())
    return twin.eval()


@torch.no_grad()
def teacher_forced(model, seq, first):
    """Eager decode steps over the token sequence `seq` (every position fed its
    token of seq); returns the fp32 logits of positions first .. len(seq)-1."""
    model.setup_cache(cache_length(seq.numel()), "cuda", dtype=model.embed_tokens.weight.dtype)
    out = []
    for i in range(seq.numel()):
        logits = model.forward_step(seq[i].view(1, 1), torch.tensor([i], device="cuda"))
        if i >= first:
            out.append(logits.float().view(-1))
    return torch.stack(out)


def rel_l2(a, b):
    """Worst step's relative L2 distance of logits a from b ([steps, vocab])."""
    return float(((a - b).norm(dim=1) / b.norm(dim=1)).max())


@torch.no_grad()
def graph_matches_eager(model, prompt, steps):
    """Fused sparse decode: eager steps, then graph replays of the same prompt;
    tokens and logits bit-identical, every logit finite. Returns the fed token
    sequence (prompt, then the generated tokens) and the eager logits."""
    gd = GraphDecoder(model, prompt.numel() + steps)
    gd.run_prompt(prompt)
    eager = [gd.eager_step().clone() for _ in range(steps)]
    gen_tokens = gd.tokens[prompt.numel(): prompt.numel() + steps].clone()
    assert all(bool(torch.isfinite(e).all()) for e in eager)
    gd.capture()
    gd.run_prompt(prompt)
    for i in range(steps):
        gd.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(gd.logits).all(), i
        assert torch.equal(gd.logits, eager[i]), f"graph replay {i} differs from eager"
    assert torch.equal(gd.tokens[prompt.numel(): prompt.numel() + steps], gen_tokens)
    del gd
    seq = torch.cat((prompt.to("cuda"), gen_tokens))
    return seq, torch.stack([e.float().view(-1) for e in eager])


CASES = [  # (model, M, layers or None for the full depth)
    ("llama-3.1-8b", 64, None),
    ("qwen3-14b", 64, None),
    ("qwen3-14b", 16, 4),
    ("qwen3-14b", 256, 4),
    ("qwen3-32b", 32, None),
]


@pytest.mark.parametrize("name,M,layers", CASES, ids=lambda v: str(v))
def test_full_depth_decode_parity(gpu, name, M, layers):
    cfg = CONFIGS[name]
    if layers is not None:
        cfg = dataclasses.replace(cfg, n_layers=layers)
    tag = f"{name} {M // 2}:{M} x{cfg.n_layers} layers"
    _free()
    say(f"{tag}: building the sparse model")
    model = sparse_model(cfg, M, seed=M + cfg.n_layers)
    model.carry_mode = "split"  # graph replay bit-identical to eager; the accumulated carry is checked below
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=torch.Generator().manual_seed(M))
    say(f"{tag}: eager vs graph replay, {STEPS} steps")
    seq, eager = graph_matches_eager(model, prompt, STEPS)
    logits = {}
    for mode in Decoder.LAUNCH_MODES:
        say(f"{tag}: teacher-forced {mode}")
        model.set_launch_mode(mode)
        logits[mode] = teacher_forced(model, seq, PROMPT)
    model.set_launch_mode("fused")
    assert torch.equal(logits["fused"], eager)  # the same computation, fed the same tokens
    say(f"{tag}: teacher-forced fused, accumulated carry")
    model.carry_mode = "accumulate"
    logits["fused_accumulate"] = teacher_forced(model, seq, PROMPT)
    assert len(model._carry[1]) == 4  # the accumulated layers ran
    model.carry_mode = "split"
    for dtype in (torch.float32, torch.float16):
        say(f"{tag}: masked dense twin {dtype}")
        twin = dense_twin(model, dtype)
        if dtype == torch.float16:  # the twin's weights pack back to the sparse buffers exactly
            lin = model.layers[-1].mlp.down_proj
            back = NmSparseLinear.from_dense(twin.layers[-1].mlp.down_proj.weight, lin.mat_index, M)
            assert torch.equal(back.mat_data.view(torch.int16), lin.mat_data.view(torch.int16))
        logits[f"dense_{str(dtype)[6:]}"] = teacher_forced(twin, seq, PROMPT)
        del twin
        _free()
    ref = logits.pop("dense_float32")
    e16 = rel_l2(logits["dense_float16"], ref)
    err = {k: rel_l2(v, ref) for k, v in logits.items()}
    cross = rel_l2(logits["fused"], logits["per_linear"])
    to_dense16 = rel_l2(logits["fused"], logits["dense_float16"])
    say(f"{tag}: rel-L2 of logits vs the fp32 dense twin (worst of {STEPS} steps): "
        + ", ".join(f"{k} {v:.2e}" for k, v in err.items())
        + f"; fused vs per-Linear {cross:.2e}; fused vs fp16 dense twin {to_dense16:.2e}")
    assert all(torch.isfinite(v).all() for v in logits.values())
    assert e16 < 0.05, e16  # the fp16 model tracks fp32 at this depth at all
    bound = 2 * e16 + 1e-3
    for k in ("fused", "fused_accumulate", "per_linear", "grouped"):
        assert err[k] <= bound, (k, err[k], bound)
    assert cross <= 3 * e16 + 1e-3, cross
    assert to_dense16 <= 3 * e16 + 1e-3, to_dense16
    del model
    _free()


LONG_CASES = [  # (model, M, prompt tokens, positions): the Llama-3.1-8B and Qwen3-32B workloads
    ("llama-3.1-8b", 64, 128, 128 + 256),
    ("qwen3-32b", 32, 512, 512 + 512),
]
LONG_STEPS = 6


@torch.no_grad()
def prefilled_then_steps(model, prompt, fed, positions):
    """Decoder.prefill of `prompt` into a cache for `positions`, then eager steps
    feeding fed[i] at position P + i; fp32 logits [1 + len(fed), vocab], the
    prompt's last position first."""
    model.setup_cache(cache_length(positions), "cuda", dtype=model.embed_tokens.weight.dtype)
    P = prompt.numel()
    out = [model.prefill(prompt.to("cuda")).float().view(-1)]
    for i in range(fed.numel()):
        out.append(model.forward_step(fed[i].view(1, 1), torch.tensor([P + i], device="cuda")).float().view(-1))
    return torch.stack(out)


@pytest.mark.parametrize("name,M,P,positions", LONG_CASES, ids=lambda v: str(v))
def test_decode_parity_at_the_configs_context(gpu, name, M, P, positions):
    """Decode at the positions the benchmark configurations run at: the mask
    rows of caches rounded up to whole 128 positions, the causal mask rewritten
    every step, prefill-written keys and values (reference protocol:
    benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:141-142,164-165,181-182)."""
    cfg = CONFIGS[name]
    tag = f"{name} {M // 2}:{M} prompt {P} positions {positions}"
    _free()
    say(f"{tag}: building the sparse model")
    model = sparse_model(cfg, M, seed=M + P)
    model.carry_mode = "split"  # graph replay bit-identical to eager; the accumulated carry is checked below
    prompt = torch.randint(0, cfg.vocab, (P,), generator=torch.Generator().manual_seed(P))
    gd = GraphDecoder(model, positions)
    assert model.max_seq == cache_length(positions)
    say(f"{tag}: prefill, then {LONG_STEPS} eager steps")
    gd.run_prompt(prompt, batched=True)
    prefill_logits = gd.logits.float().view(-1).clone()
    snap_k, snap_v = model.k_store.clone(), [v.clone() for v in model.v_cache_t]
    snap_tok, snap_tokens = gd.token.clone(), gd.tokens.clone()
    eager = [gd.eager_step().clone() for _ in range(LONG_STEPS)]
    assert all(bool(torch.isfinite(e).all()) for e in eager)
    fed = gd.tokens[P:P + LONG_STEPS].clone()
    eager_tokens = gd.tokens[P:P + LONG_STEPS + 1].clone()
    say(f"{tag}: graph replays from the same caches")
    gd.capture()
    model.k_store.copy_(snap_k)
    for v, sv in zip(model.v_cache_t, snap_v):
        v.copy_(sv)
    gd.token.copy_(snap_tok)
    gd.tokens.copy_(snap_tokens)
    gd.pos.fill_(P)
    gd.host_pos = P
    for i in range(LONG_STEPS):
        gd.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(gd.logits).all(), i
        assert torch.equal(gd.logits, eager[i]), f"graph replay at position {P + i} differs from eager"
    assert torch.equal(gd.tokens[P:P + LONG_STEPS + 1], eager_tokens)
    del gd, snap_k, snap_v
    _free()
    logits = {"eager": torch.cat((prefill_logits.view(1, -1), torch.stack([e.float().view(-1) for e in eager])))}
    for mode in Decoder.LAUNCH_MODES:
        say(f"{tag}: prefill + teacher-forced {mode}")
        model.set_launch_mode(mode)
        logits[mode] = prefilled_then_steps(model, prompt, fed, positions)
    model.set_launch_mode("fused")
    say(f"{tag}: prefill + teacher-forced fused, accumulated carry")
    model.carry_mode = "accumulate"
    logits["fused_accumulate"] = prefilled_then_steps(model, prompt, fed, positions)
    assert len(model._carry[1]) == 4  # the accumulated layers ran
    model.carry_mode = "split"
    for dtype in (torch.float32, torch.float16):
        say(f"{tag}: masked dense twin {dtype}")
        twin = dense_twin(model, dtype)
        logits[f"dense_{str(dtype)[6:]}"] = prefilled_then_steps(twin, prompt, fed, positions)
        del twin
        _free()
    ref = logits.pop("dense_float32")
    e16 = rel_l2(logits["dense_float16"], ref)
    err = {k: rel_l2(v, ref) for k, v in logits.items()}
    cross = rel_l2(logits["fused"], logits["per_linear"])
    to_dense16 = rel_l2(logits["eager"], logits["dense_float16"])
    say(f"{tag}: rel-L2 of logits vs the fp32 dense twin (worst of the prefill and {LONG_STEPS} steps): "
        + ", ".join(f"{k} {v:.2e}" for k, v in err.items())
        + f"; fused vs per-Linear {cross:.2e}; eager vs fp16 dense twin {to_dense16:.2e}")
    assert all(torch.isfinite(v).all() for v in logits.values())
    assert e16 < 0.05, e16
    bound = 2 * e16 + 1e-3
    for k in ("eager", "fused", "fused_accumulate", "per_linear", "grouped", "modules"):
        assert err[k] <= bound, (k, err[k], bound)
    assert cross <= 3 * e16 + 1e-3, cross
    assert to_dense16 <= 3 * e16 + 1e-3, to_dense16
    del model
    _free()
