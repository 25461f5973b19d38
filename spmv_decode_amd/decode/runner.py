"""hipGraph-captured greedy decode for `Decoder` (dense or N:M-sparse Linears).

One replay of the captured graph runs one decode step entirely on the device:
embed the current token, run every layer (KV cache written at the device-side
position), final norm and lm_head, greedy argmax, store the token, advance the
position. The host only replays the graph, so per-token time is GPU time
(the reference captures a fixed-position step in a CUDA graph,
benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:155-180; here the position moves).
"""
from __future__ import annotations

import statistics

import torch

from .model import Decoder


def _chunk_width(n: int) -> int:
    """Largest divisor of n in [64, 1024] (0 if none)."""
    for c in range(min(1024, n), 63, -1):
        if n % c == 0:
            return c
    return 0


def greedy_token(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """argmax over the last dim of [1, V] logits -> [1] int64 (written to
    `out` when given), the first index of the maximum like torch.argmax, in
    two parallel stages: the maximum (and its first index) of each C-wide
    chunk, then the first chunk holding the largest of those. A single-row
    torch.argmax over a 128K vocabulary is one workgroup's reduction (~46 us
    on MI355X). Four kernels, no host synchronisation (graph capture)."""
    V = logits.shape[-1]
    C = _chunk_width(V)
    if C == 0 or V // C < 2:
        r = torch.argmax(logits, dim=-1)
        return r if out is None else out.copy_(r.view_as(out))
    vals, idx = logits.reshape(V // C, C).max(dim=1)
    j = torch.argmax(vals).view(1)
    return torch.add(idx.index_select(0, j), j, alpha=C, out=out)  # j * C + idx[j]


CACHE_ALIGN = 128


def cache_length(max_seq: int) -> int:
    """Static KV-cache length for `max_seq` positions: rounded up to a
    multiple of CACHE_ALIGN. The attention products over the cache pick much
    slower BLAS kernels at other lengths (MI355X, 8 KV heads x 128: the three
    attention kernels take 17.2 us per layer at 384 positions but 19.8 us at
    392; 19.4 us at 1024 but 28.2 us at 1032)."""
    return -(-max_seq // CACHE_ALIGN) * CACHE_ALIGN


def softmax_row(logits: torch.Tensor) -> torch.Tensor:
    """torch.softmax(logits.float(), dim=-1) of [1, V] logits in two parallel
    stages over the C-wide chunks greedy_token uses (the maximum and the sum
    of exponentials per chunk, then over the chunks): a single-row softmax over
    a 128K vocabulary is one workgroup's pass (~40 us on MI355X). Exact up to
    the order of the fp32 sum."""
    x = logits.float()
    V = x.shape[-1]
    C = _chunk_width(V)
    if C == 0 or V // C < 2:
        return torch.softmax(x, dim=-1)
    xv = x.reshape(V // C, C)
    e = torch.exp(xv - xv.amax(dim=1).amax())
    return (e / e.sum(dim=1).sum()).reshape(x.shape)


def sample_token(logits: torch.Tensor, out: torch.Tensor, generator: torch.Generator | None = None) -> torch.Tensor:
    """The reference's sampling step (generate.py:46-63;
    benchmarks/bench_qwen_31_14b_fp16_fixed_ptx.py:356-357): the softmax of the
    logits in fp32, cast back to the logits' dtype, and one draw from that
    categorical distribution, written into `out` [1].

    The draw is the exponential race that torch.multinomial itself uses for
    one sample: with E_i ~ Exp(1) independent, argmax_i p_i / E_i is
    distributed as Categorical(p) (the Gumbel-max trick, exponentiated). It is
    written here with graph-safe pieces, torch's device generator
    (`exponential_`) and the two-stage greedy_token argmax, because
    torch.multinomial first checks its input with vocabulary-wide max/min
    reductions whose multi-block form clears its semaphores with memset nodes
    when captured; replayed, those gave wrong results on MI355X and the check's
    device-side assert then aborted the run."""
    probs = softmax_row(logits).to(logits.dtype)
    race = torch.empty(probs.shape, dtype=torch.float32, device=probs.device).exponential_(generator=generator)
    return greedy_token(probs.float() / race, out=out)


def _fill_fixed_context(model: Decoder, ctx: int, seed: int, dev: torch.device) -> None:
    """The fixed-context protocol's caches: ctx + 1 positions (rounded up by
    cache_length) of the model's dtype, keys and values N(0, 0.02) from a
    seeded device generator, layer by layer (the mask and padding rows stay as
    set up)."""
    hd = model.cfg.head_dim
    model.setup_cache(cache_length(ctx + 1), dev, dtype=model.embed_tokens.weight.dtype)
    gen = torch.Generator(device=dev).manual_seed(seed)
    for k, v in zip(model.k_cache_t, model.v_cache_t):
        k[:, :hd].normal_(0.0, 0.02, generator=gen)
        v.normal_(0.0, 0.02, generator=gen)


@torch.no_grad()
def fixed_context_logits_fp32(model: Decoder, ctx: int, seed: int = 1234, token_id: int = 123,
                              device="cuda") -> torch.Tensor:
    """The logits of fixed_context_ms's step computed in fp32 throughout: the
    same weights and cache values (drawn in the model's dtype exactly as
    fixed_context_ms draws them, then widened, which is exact), every sparse
    projection replaced for the step by an fp32 nn.Linear holding its masked
    dense weight (NmSparseLinear.to_dense: the packed weights scattered back),
    every activation fp32, one eager step. The fp32 reference against which
    the fp16 steps (eager and compiled) are held (fp16 rounding envelope). The
    model is widened in place for the step and narrowed back afterwards (an
    exact round trip: every weight is an fp16 value), its sparse projections
    put back and its dense fusion copies rebuilt. Returns fp32 logits
    [1, vocab] on the host."""
    import torch.nn as nn

    from ..nmsparse_linear import NmSparseLinear

    dev = torch.device(device)
    dt = model.embed_tokens.weight.dtype
    hd = model.cfg.head_dim
    _fill_fixed_context(model, ctx, seed, dev)
    keys = model.k_store[:, :, :hd].clone()
    vals = [v.clone() for v in model.v_cache_t]
    fusion = model.dense_fusion
    swapped = []
    try:
        for mod in list(model.modules()):
            for name, child in list(mod.named_children()):
                if isinstance(child, NmSparseLinear):
                    dense = nn.Linear(1, 1, bias=False, device="meta")
                    dense.weight = nn.Parameter(child.to_dense(torch.float32), requires_grad=False)
                    setattr(mod, name, dense)
                    swapped.append((mod, name, child))
        model.float()
        model.set_dense_fusion(fusion)
        model.setup_cache(cache_length(ctx + 1), dev, dtype=torch.float32)
        model.k_store[:, :, :hd].copy_(keys)
        for v, src in zip(model.v_cache_t, vals):
            v.copy_(src)
        del keys, vals
        token = torch.full((1, 1), token_id, dtype=torch.long, device=dev)
        pos = torch.full((1,), ctx, dtype=torch.long, device=dev)
        logits = model.forward_step(token, pos).float().cpu()
    finally:
        for mod, name, child in swapped:
            setattr(mod, name, child)
        model.to(dt)
        model.set_dense_fusion(fusion)
        model.setup_cache(cache_length(ctx + 1), dev, dtype=dt)
    return logits


def logits_envelope(eager16: torch.Tensor, other16: torch.Tensor, ref32: torch.Tensor) -> dict:
    """Whether `other16` (e.g. the compiled step's logits) stays within the
    fp16 envelope of `eager16` (the eager step's), both judged against the
    fp32 reference `ref32` of the same step: e16 = rel-L2(eager16, ref32) is
    what fp16 rounding costs at this depth; `other16` must be within
    2 * e16 + 1e-3 of ref32 and within 3 * e16 + 1e-3 of eager16 (the rule of
    the full-depth decode parity tests). Relative L2 over the vocabulary."""
    def rel(a, b):
        return float((a.float() - b.float()).norm() / b.float().norm())

    e16 = rel(eager16, ref32)
    to_ref, to_eager = rel(other16, ref32), rel(other16, eager16)
    ok = to_ref <= 2 * e16 + 1e-3 and to_eager <= 3 * e16 + 1e-3
    return {"within": ok, "e16_eager_vs_fp32": float(f"{e16:.3e}"), "rel_l2_vs_fp32": float(f"{to_ref:.3e}"),
            "rel_l2_vs_eager": float(f"{to_eager:.3e}"),
            "same_greedy_token": int(torch.argmax(other16)) == int(torch.argmax(eager16))}


@torch.no_grad()
def fixed_context_ms(model: Decoder, ctx: int, warmup: int = 30, repeat: int = 30, inner: int = 10,
                     seed: int = 1234, token_id: int = 123, device="cuda", sample: bool = True) -> dict:
    """The reference benchmark's fixed-context protocol
    (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:144-189): KV caches for
    ctx + 1 positions filled with N(0, 0.02), one decode step of `token_id` at
    position `ctx`, with the next token sampled as the reference's step does
    (softmax, one categorical draw: sample_token; `sample=False`: greedy), captured as
    one hipGraph, `warmup` replays, then `repeat` samples of `inner` replays
    each; every replay decodes the same position. Returns the median, mean and
    stdev of the samples in ms per replay, the samples, the last replay's
    logits (fp32, host), their greedy token and the last sampled token."""
    if min(ctx, warmup, repeat, inner) < 1:
        raise ValueError("ctx, warmup, repeat and inner must be positive")
    dev = torch.device(device)
    _fill_fixed_context(model, ctx, seed, dev)
    token = torch.full((1, 1), token_id, dtype=torch.long, device=dev)
    pos = torch.full((1,), ctx, dtype=torch.long, device=dev)
    nxt = torch.zeros(1, dtype=torch.long, device=dev)

    def step():
        logits = model.forward_step(token, pos)
        if sample:
            sample_token(logits, out=nxt)
        else:
            greedy_token(logits, out=nxt)
        return logits

    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for _ in range(3):  # workspaces and library handles are created outside the capture
            step()
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        logits = step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize(dev)
    samples = []
    for _ in range(repeat):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(inner):
            graph.replay()
        b.record()
        b.synchronize()
        samples.append(a.elapsed_time(b) / inner)
    finite = bool(torch.isfinite(logits).all().item())
    host_logits = logits.float().cpu()
    del graph
    return {"median": statistics.median(samples), "mean": statistics.mean(samples),
            "stdev": statistics.stdev(samples) if repeat > 1 else 0.0, "samples": samples,
            "finite_logits": finite, "token": int(torch.argmax(host_logits, dim=-1)), "logits": host_logits,
            "sampled_token": int(nxt.item()) if sample else None, "sampling": "categorical" if sample else "greedy"}


class GraphDecoder:
    def __init__(self, model: Decoder, max_seq: int, device="cuda"):
        """max_seq: positions the decode may use (prompt + generated tokens);
        the cache itself is cache_length(max_seq) long, the extra slots masked."""
        self.model = model
        self.device = torch.device(device)
        model.setup_cache(cache_length(max_seq), self.device, dtype=model.embed_tokens.weight.dtype)
        self.max_seq = max_seq
        self.host_pos = 0  # host mirror of `pos`: no step may index past the static cache
        self.token = torch.zeros(1, 1, dtype=torch.long, device=self.device)
        self.pos = torch.zeros(1, dtype=torch.long, device=self.device)
        self.tokens = torch.zeros(max_seq + 1, dtype=torch.long, device=self.device)
        self.logits = None
        self.graph = None
        self.stream = torch.cuda.Stream(device=self.device)

    @torch.no_grad()
    def _step(self):
        logits = self.model.forward_step(self.token, self.pos)
        nxt = greedy_token(logits, out=self.token.view(1))  # the next step's input token
        self.tokens[1:].index_copy_(0, self.pos, nxt)  # tokens[pos + 1]
        self.pos.add_(1)
        return logits

    def _advance(self, n: int = 1):
        if self.host_pos + n > self.max_seq:
            raise RuntimeError(f"decode past the static cache: position {self.host_pos} + {n} > {self.max_seq}")
        self.host_pos += n

    @torch.no_grad()
    def eager_step(self):
        self._advance()
        self.logits = self._step()
        return self.logits

    @torch.no_grad()
    def capture(self, warmup: int = 2):
        """Warm up on the capture stream (creates every workspace the sparse
        kernels need), then capture one step. Cache contents and counters are
        reset afterwards."""
        self.reset()
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            for _ in range(min(warmup, self.max_seq)):
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.logits = self._step()
        torch.cuda.synchronize(self.device)
        self.reset()

    @torch.no_grad()
    def reset(self, first_token: int = 0):
        self.model.reset_cache()
        self.pos.zero_()
        self.host_pos = 0
        self.token.fill_(first_token)
        self.tokens.zero_()

    def replay(self):
        self._advance()
        self.graph.replay()

    @torch.no_grad()
    def run_prompt(self, prompt_ids: torch.Tensor, batched: bool = False):
        """Feed the prompt (untimed): one step per token, or with batched=True
        all tokens in one Decoder.prefill pass. After it `token` holds the
        first generated token and `pos` the prompt length."""
        ids = prompt_ids.to(self.device).view(-1)
        self.reset(int(0))
        self.tokens[0] = ids[0]
        if batched:
            self._advance(ids.numel())
            logits = self.model.prefill(ids)
            if self.graph is not None:  # self.logits is the captured step's output buffer: keep it
                self.logits.copy_(logits)
            else:
                self.logits = logits
            nxt = greedy_token(logits, out=self.token.view(1))
            self.tokens[ids.numel():ids.numel() + 1].copy_(nxt)
            self.pos.fill_(ids.numel())
            return
        for i in range(ids.numel()):
            self.token.copy_(ids[i].view(1, 1))
            self.replay() if self.graph is not None else self.eager_step()

    @torch.no_grad()
    def generate(self, n: int, chunk: int = 16):
        """n greedy steps by graph replay; returns (generated ids [n], ms/token,
        median ms/token over chunks of `chunk` steps)."""
        if self.host_pos + n > self.max_seq:
            raise RuntimeError(f"decode past the static cache: position {self.host_pos} + {n} > {self.max_seq}")
        first = self.host_pos + 1
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(n // chunk + 2)]
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        k = 0
        ev[0].record()
        for i in range(n):
            self.replay()
            if (i + 1) % chunk == 0:
                k += 1
                ev[k].record()
        end.record()
        end.synchronize()
        total = begin.elapsed_time(end)
        chunks = [ev[j].elapsed_time(ev[j + 1]) / chunk for j in range(k)]
        gen = self.tokens[first:first + n].clone()
        return gen, total / n, (statistics.median(chunks) if chunks else total / n)
