"""A compact Llama-3.1 / Qwen3 decoder for batch-1 decode on MI355X.

This is the caller of the sparse GEMV on the decode path (the role of the
reference's gpt-fast `model.py` / Hugging Face Qwen3 decoders): every
attention and MLP projection is a `nn.Linear` under the Hugging Face names
(`self_attn.{q,k,v,o}_proj`, `mlp.{gate,up,down}_proj`) on `model.layers`, so
`swap_to_nmsparse(model, M, device)` turns each into an `NmSparseLinear`
unchanged. Only decode (one token per step) is implemented: the KV cache is
static, the position is a device tensor, and a step contains no host
synchronisation, so it can be captured once in a hipGraph and replayed.

Keys and values are cached transposed, [kv_heads, head_dim, S]: the score
product then reads contiguous rows of keys, and the probability-times-values
product takes the values as a transposed operand, which the BLAS library runs
faster at these shapes (MI355X, S = 384: 6.6 µs against 8.2 µs for a
[kv_heads, S, head_dim] cache; S = 1024: 4.3 µs against 12-16 µs). The causal
mask lives in the key cache: each head has KEY_PAD extra rows, the first of
them holding the additive mask (0 at positions <= pos, -inf after), and the
query buffer holds a 1 in that column, so one plain batched product yields the
masked scores (an additive mask operand makes PyTorch copy it into the output
before the product: one more kernel per layer and a slower GEMM).

Numerics follow the published architectures: RMSNorm in fp32 (one fused
`F.rms_norm` kernel), rotary embeddings on interleaved (even, odd) pairs as a
complex multiply (the convention of the reference's gpt-fast model,
model.py:310-322; Hugging Face checkpoints need the usual q/k row permutation),
Llama-3.1's frequency scaling, grouped-query attention with the softmax
computed in fp32, SiLU-gated MLP, Qwen3's per-head RMSNorm on queries and keys
before the rotary embedding.

A step is written for few kernel launches, since at batch 1 every small
kernel costs a few microseconds: the q/k/v projections write into slices of
one buffer, so the rotary embedding runs once over queries and keys; the
attention scale and causal mask are folded into one batched product.

`Decoder(cfg, layout="gpt-fast")` names the layers as gpt-fast does (the
reference benchmark's model.py: `attention.wqkv` / `wo`, `feed_forward.w1` /
`w3` / `w2`, `attention_norm`, `ffn_norm`); those layers call every projection
as a module, as unmodified model code does.

When every projection of every layer is an `NmSparseLinear` (after
`swap_to_nmsparse`), `forward_step` runs the fused layer instead
(`fuse_epilogues`, on by default): the input RMSNorm, Qwen3's q/k norms, the
rotary embedding and the KV-cache write happen inside the grouped q/k/v
launch, the residual adds inside the o and down launches (in place on the
residual stream), and the post-attention RMSNorm inside the gate/up launch.
A layer is then 7 kernels: q/k/v, three attention kernels, o, gate/up, down.
The per-Linear path above stays for dense models and for comparison.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class DecoderConfig:
    name: str
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    rope_theta: float
    norm_eps: float
    qk_norm: bool = False
    rope_scaling: dict | None = field(default=None, hash=False, compare=False)


LLAMA31_8B = DecoderConfig("llama-3.1-8b", 32, 4096, 32, 8, 128, 14336, 128256, 500000.0, 1e-5, False,
                           dict(factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                original_max_position_embeddings=8192))
QWEN3_14B = DecoderConfig("qwen3-14b", 40, 5120, 40, 8, 128, 17408, 151936, 1000000.0, 1e-6, True)
QWEN3_32B = DecoderConfig("qwen3-32b", 64, 5120, 64, 8, 128, 25600, 151936, 1000000.0, 1e-6, True)
QWEN3_06B = DecoderConfig("qwen3-0.6b", 28, 1024, 16, 8, 128, 3072, 151936, 1000000.0, 1e-6, True)
CONFIGS = {c.name: c for c in (LLAMA31_8B, QWEN3_14B, QWEN3_32B, QWEN3_06B)}


def tiny_config(qk_norm: bool = False, n_layers: int = 2) -> DecoderConfig:
    """A small config with the same structure, for tests."""
    return DecoderConfig("tiny", n_layers, 256, 4, 2, 64, 384, 512, 10000.0, 1e-5, qk_norm)


def rope_inv_freq(cfg: DecoderConfig) -> torch.Tensor:
    """Inverse rotary frequencies (float64), with Llama-3.1 scaling when configured:
    wavelengths shorter than original/high_freq_factor keep their frequency,
    longer than original/low_freq_factor are divided by `factor`, and the band
    between is interpolated linearly in original_len/wavelength."""
    half = cfg.head_dim // 2
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(half, dtype=torch.float64) * 2.0 / cfg.head_dim))
    sc = cfg.rope_scaling
    if sc:
        orig = sc["original_max_position_embeddings"]
        lo, hi, factor = sc["low_freq_factor"], sc["high_freq_factor"], sc["factor"]
        wavelen = 2 * math.pi / inv
        smooth = ((orig / wavelen) - lo) / (hi - lo)
        scaled = torch.where(wavelen > orig / lo, inv / factor, inv)
        mid = (wavelen <= orig / lo) & (wavelen >= orig / hi)
        scaled = torch.where(mid, (1 - smooth) * inv / factor + smooth * inv, scaled)
        inv = scaled
    return inv


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)


def rotate(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """Rotary embedding on interleaved (even, odd) pairs, in fp32.
    x: [..., head_dim]; freqs: complex64 [head_dim/2] (cos + i sin), or the
    same as fp32 (cos, sin) pairs [head_dim/2, 2], which torch.compile fuses
    with its neighbours (it runs complex products as library kernels of their
    own)."""
    xp = x.float().reshape(*x.shape[:-1], -1, 2)
    if freqs.is_complex():
        return torch.view_as_real(torch.view_as_complex(xp) * freqs).flatten(-2).to(x.dtype)
    x0, x1, c, s = xp[..., 0], xp[..., 1], freqs[..., 0], freqs[..., 1]
    return torch.stack((x0 * c - x1 * s, x0 * s + x1 * c), dim=-1).flatten(-2).to(x.dtype)


# Rows per head after head_dim in the key cache (and columns in the query
# buffer). 32 rather than the 1 the mask needs: the BLAS library's score
# product over head_dim + 32 = 160 runs 0.3-0.5 us per layer faster than
# over 136 or 144 (MI355X, 384 and 1024 positions, caches cold).
KEY_PAD = 32


def attend(q_pad: torch.Tensor, k_cache_t: torch.Tensor, v_cache_t: torch.Tensor, cfg: "DecoderConfig",
           zero: torch.Tensor) -> torch.Tensor:
    """softmax(q k / sqrt(head_dim) + mask) v for one decode token, grouped
    query heads. q_pad [n_heads, head_dim + KEY_PAD]: the query, then 1, then
    zeros; k_cache_t [kv_heads, head_dim + KEY_PAD, S]: the keys, then the
    additive mask row, then zero rows; v_cache_t [kv_heads, head_dim, S]; zero:
    a 0-dim tensor (the product's ignored addend). Returns [kv_heads, g,
    head_dim] with g = n_heads / kv_heads, contiguous."""
    kvh = cfg.n_kv_heads
    q3 = q_pad.view(kvh, cfg.n_heads // kvh, q_pad.shape[1])
    if torch.compiler.is_compiling():
        # Traced: baddbmm's addend would be written out by a kernel of its own
        # before the product, so the scale joins the softmax kernel instead;
        # and probabilities x values as a reduction over the positions (fp32),
        # which the compiler generates in place of the library's batched
        # product of 4-row matrices (Llama-3.1-8B, 512 positions: 0.26 ms per
        # token less).
        scores = torch.bmm(q3, k_cache_t) * (1.0 / math.sqrt(cfg.head_dim))
        probs = torch.softmax(scores, dim=-1)
        return (probs.float().unsqueeze(2) * v_cache_t.float().unsqueeze(1)).sum(-1).to(q_pad.dtype)
    scores = torch.baddbmm(zero, q3, k_cache_t, beta=0.0, alpha=1.0 / math.sqrt(cfg.head_dim))
    probs = torch.softmax(scores, dim=-1)  # fp16 in/out, fp32 inside
    return torch.bmm(probs, v_cache_t.transpose(1, 2))


def linear_into(lin: nn.Module, x2d: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """y = lin(x) written into `out` ([1, h] contiguous slice): the sparse GEMV's
    `out=` for NmSparseLinear, torch.mm (hipBLASLt) for a dense nn.Linear, the
    module's own forward for any other Linear-like module."""
    from ..nmsparse_linear import NmSparseLinear

    if isinstance(lin, NmSparseLinear):
        from ..hip_spmv import nmsparse_spmv_forward_hip

        return nmsparse_spmv_forward_hip(x2d, lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width, 128,
                                         lin.vec_width, 1, x2d.shape[1], out=out)
    if type(lin) is nn.Linear and lin.bias is None:
        return dense_gemv(x2d, lin.weight, getattr(lin, "gemv_form", "mm"), out=out)
    if isinstance(lin, nn.Linear):
        return torch.mm(x2d, lin.weight.t(), out=out)
    return out.copy_(lin(x2d).view_as(out))


GEMV_FORMS = ("mm", "mv")


def dense_gemv(x2d: torch.Tensor, weight: torch.Tensor, form: str = "mm", out=None) -> torch.Tensor:
    """y [1, n_out] = x2d [1, K] · weightᵀ through the BLAS library in one of
    two problem statements, which it serves with different kernels: "mm" (a
    one-row product x · Wᵀ, what nn.Linear issues) or "mv" (the matrix-vector
    product W · x, stated as a one-column product so that torch.compile also
    leaves it to the library instead of generating its own kernel). Which is
    faster depends on the shape (Decoder.tune_dense_gemv)."""
    if form == "mv":
        if out is None:
            return torch.mm(weight, x2d.view(-1, 1)).view(1, -1)
        torch.mm(weight, x2d.view(-1, 1), out=out.view(-1, 1))
        return out
    return torch.mm(x2d, weight.t(), out=out) if out is not None else torch.mm(x2d, weight.t())


def project(lin: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """lin(x) for one row x [..., K] as one launch of its own: a bias-free
    nn.Linear through dense_gemv in its tuned form, an NmSparseLinear through
    its op (never through a sibling group's shared launch), any other module
    through its own forward."""
    from ..nmsparse_linear import NmSparseLinear

    if x.numel() == x.shape[-1]:
        if type(lin) is nn.Linear and lin.bias is None:
            return dense_gemv(x.reshape(1, -1), lin.weight, getattr(lin, "gemv_form", "mm")).view(*x.shape[:-1], -1)
        if isinstance(lin, NmSparseLinear):
            return torch.ops.nmsparse.gemv(x, lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width,
                                           lin.vec_width)
    return lin(x)


def project_rows(lin: nn.Module, x2d: torch.Tensor) -> torch.Tensor:
    """lin(x) for every row of x2d [rows, K] -> [rows, h]: an NmSparseLinear
    through the SpMM on its packed weights (the small-batch kernel up to 8
    rows, the matrix-core kernel above for fp16 / bf16), even when it also
    holds a dense weight; any other module through its own forward."""
    from ..nmsparse_linear import NmSparseLinear

    if isinstance(lin, NmSparseLinear):
        from ..hip_spmv import nmsparse_spmm_forward_hip

        return nmsparse_spmm_forward_hip(x2d, lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width,
                                         lin.vec_width)
    return lin(x2d)


def project_rows_group(lins, x2d: torch.Tensor) -> list:
    """[project_rows(lin, x2d) for lin in lins] for sibling Linears of one
    input (q/k/v, gate/up): NmSparseLinears of one packed width and N:M run as
    one grouped SpMM (hip_spmv.nmsparse_spmm_group_hip: one gather and one
    matrix-core launch for all of them from 9 to 128 rows), anything else one
    at a time."""
    from ..nmsparse_linear import NmSparseLinear

    lins = list(lins)
    if len(lins) > 1 and all(isinstance(l, NmSparseLinear) for l in lins):
        l0 = lins[0]
        if all(l.w == l0.w and l.block_width == l0.block_width and l.vec_width == l0.vec_width
               and l.mat_data.dtype == x2d.dtype for l in lins):
            from ..hip_spmv import nmsparse_spmm_group_hip

            return nmsparse_spmm_group_hip(x2d, [(l.mat_data, l.mat_index) for l in lins], l0.block_width,
                                           l0.vec_width)
    return [project_rows(l, x2d) for l in lins]


def project_rows_silu_mul(lin: nn.Module, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """project_rows(lin, silu(gate) * up): an NmSparseLinear forms the SiLU
    product inside its SpMM's activation gather (hip_spmv.
    nmsparse_spmm_silu_mul_hip: in fp32 with one rounding, as the decode
    steps' gate/up pair does), any other module gets F.silu(gate) * up."""
    from ..nmsparse_linear import NmSparseLinear

    if isinstance(lin, NmSparseLinear) and lin.mat_data.dtype == gate.dtype:
        from ..hip_spmv import nmsparse_spmm_silu_mul_hip

        return nmsparse_spmm_silu_mul_hip(gate, up, lin.mat_data, lin.mat_index, lin.w, lin.h, lin.block_width,
                                          lin.vec_width)
    return project_rows(lin, F.silu(gate) * up)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_kv_heads: int) -> torch.Tensor:
    """softmax(q kᵀ / sqrt(d) + causal mask) v over P positions, grouped query
    heads: q [P, n_heads, d], k and v [P, kv_heads, d] -> [P, n_heads * d].
    PyTorch's scaled_dot_product_attention (is_causal, grouped heads): one
    fused kernel on the GPU (fp32 accumulation), where scores in fp32 through
    two batched products, a mask and a softmax took about 12 kernels per layer
    and 1.3-1.8 ms more per 64-128-token Llama-3.1-8B prompt on MI355X."""
    P, nh, d = q.shape
    o = F.scaled_dot_product_attention(q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0),
                                       v.transpose(0, 1).unsqueeze(0), is_causal=True,
                                       enable_gqa=nh != n_kv_heads)  # [1, nh, P, d]
    return o.squeeze(0).transpose(0, 1).reshape(P, nh * d)


def grouped_sparse(mods) -> bool:
    """True when every module is an NmSparseLinear with the same w and N:M, so
    they can share one launch (grouped GEMV, or the gate/up pair)."""
    from ..nmsparse_linear import NmSparseLinear

    if not all(isinstance(m, NmSparseLinear) for m in mods):
        return False
    m0 = mods[0]
    return all((m.w, m.block_width, m.vec_width) == (m0.w, m0.block_width, m0.vec_width) for m in mods)


class Attention(nn.Module):
    group_launches = True  # one q/k/v launch when all three are sparse (Decoder.set_launch_mode)
    call_modules = False   # every projection through its module's forward (Decoder.set_launch_mode)

    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.cfg = cfg
        qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        self.q_proj = nn.Linear(cfg.dim, qd, bias=False)
        self.k_proj = nn.Linear(cfg.dim, kvd, bias=False)
        self.v_proj = nn.Linear(cfg.dim, kvd, bias=False)
        self.o_proj = nn.Linear(qd, cfg.dim, bias=False)
        self.wqkv = None  # fused dense q/k/v weight (Decoder.set_dense_fusion), not a parameter
        self.wqkv_form = "mm"
        if cfg.qk_norm:
            self.q_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)
            self.k_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)

    def forward(self, x, freqs, k_cache_t, v_cache_t, pos, q_pad, zero):
        """x [1, 1, dim]; freqs complex64 [1, head_dim/2]; k_cache_t [kvh,
        head_dim + KEY_PAD, S] and v_cache_t [kvh, head_dim, S] (see attend);
        pos [1] int64; q_pad [n_heads, head_dim + KEY_PAD] query buffer; zero a
        0-dim tensor."""
        c = self.cfg
        g = c.n_heads // c.n_kv_heads
        qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        x2d = x.view(1, -1)
        qkv = torch.empty(1, qd + 2 * kvd, dtype=x.dtype, device=x.device)
        slices = (qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:])
        projs = (self.q_proj, self.k_proj, self.v_proj)
        if self.group_launches and grouped_sparse(projs):
            from ..hip_spmv import nmsparse_gemv_grouped

            nmsparse_gemv_grouped(x2d, [(p.mat_data, p.mat_index) for p in projs], projs[0].block_width,
                                  projs[0].vec_width, outs=slices)
        elif self.wqkv is not None and all(type(p) is nn.Linear for p in projs):
            dense_gemv(x2d, self.wqkv, self.wqkv_form, out=qkv)
        elif self.call_modules:  # as model code that knows nothing of the swap calls them
            torch.cat([p(x) for p in projs], dim=-1, out=qkv.view(1, 1, -1))
        else:
            for proj, sl in zip(projs, slices):
                linear_into(proj, x2d, sl)
        y = attention_core(self, qkv, freqs, k_cache_t, v_cache_t, pos, q_pad, zero)  # [kvh, g, head_dim]
        if self.call_modules:
            return self.o_proj(y.view(1, 1, qd))
        return project(self.o_proj, y.view(1, 1, qd))


@torch.library.custom_op("nmsparse_decode::cache_write", mutates_args=("cache",))
def cache_write(cache: torch.Tensor, pos: torch.Tensor, values: torch.Tensor) -> None:
    """cache[:, :rows, pos] = values ([heads, rows]) in place. An op of its
    own so that torch.compile writes the cache in place: traced as indexing
    into a view of a tensor that other graph inputs alias (the key caches
    are views of one tensor), the compiler copied the view out and back
    around the write, every layer, every step."""
    cache[:, :values.shape[1]].index_copy_(2, pos, values.unsqueeze(-1))


@cache_write.register_fake
def _(cache, pos, values):
    return None


def attention_core(at, qkv, freqs, k_cache_t, v_cache_t, pos, q_pad, zero):
    """The attention of one decode token from its projections qkv [1, q + k + v]
    (at: the attention module, for its config and Qwen3's q/k norms): head
    norms, rotary embedding, the cache write at `pos`, attend. Returns
    [kv_heads, g, head_dim]."""
    c = at.cfg
    qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    qk = qkv[0, :qd + kvd].view(c.n_heads + c.n_kv_heads, c.head_dim)
    if c.qk_norm:
        qk = torch.cat((at.q_norm(qk[:c.n_heads]), at.k_norm(qk[c.n_heads:])))
    qk = rotate(qk, freqs)
    q, k = qk[:c.n_heads], qk[c.n_heads:]
    v = qkv[0, qd + kvd:].view(c.n_kv_heads, c.head_dim, 1)
    q_pad[:, :c.head_dim].copy_(q)
    if torch.compiler.is_compiling():
        cache_write(k_cache_t, pos, k)
    else:
        k_cache_t[:, :c.head_dim].index_copy_(2, pos, k.unsqueeze(-1))
    v_cache_t.index_copy_(2, pos, v)
    return attend(q_pad, k_cache_t, v_cache_t, c, zero)


class MLP(nn.Module):
    group_launches = True  # one gate/up launch when both are sparse (Decoder.set_launch_mode)
    call_modules = False   # every projection through its module's forward (Decoder.set_launch_mode)

    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.dim, cfg.inter, bias=False)
        self.up_proj = nn.Linear(cfg.dim, cfg.inter, bias=False)
        self.down_proj = nn.Linear(cfg.inter, cfg.dim, bias=False)
        self.w13 = None  # fused dense gate/up weight (Decoder.set_dense_fusion), not a parameter
        self.w13_form = "mm"

    def forward(self, x):
        if self.call_modules:
            return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))
        if self.group_launches and grouped_sparse((self.gate_proj, self.up_proj)):
            from ..hip_spmv import nmsparse_gate_up_silu

            g, u = self.gate_proj, self.up_proj
            act = nmsparse_gate_up_silu(x.view(1, -1), (g.mat_data, g.mat_index), (u.mat_data, u.mat_index),
                                        g.block_width, g.vec_width)
            return project(self.down_proj, act.view(1, 1, -1))
        if self.w13 is not None and type(self.gate_proj) is nn.Linear and type(self.up_proj) is nn.Linear:
            gu = dense_gemv(x.reshape(1, -1), self.w13, self.w13_form)
            g, u = gu.chunk(2, dim=1)
            return project(self.down_proj, (F.silu(g) * u).view(1, 1, -1))
        return project(self.down_proj, F.silu(project(self.gate_proj, x)) * project(self.up_proj, x))


class Block(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.dim, cfg.norm_eps)
        self.self_attn = Attention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.dim, cfg.norm_eps)
        self.mlp = MLP(cfg)

    def forward(self, x, freqs, k_cache_t, v_cache_t, pos, q_pad, zero):
        h = x + self.self_attn(self.input_layernorm(x), freqs, k_cache_t, v_cache_t, pos, q_pad, zero)
        return h + self.mlp(self.post_attention_layernorm(h))


class GptFastAttention(nn.Module):
    """Attention under gpt-fast's names (the reference's model.py:191-246): one
    fused `wqkv` Linear [q + k + v rows] and `wo`; Qwen3's q/k norms when the
    config has them. Same math as Attention; every projection is a module call,
    as unmodified gpt-fast code makes it."""

    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.cfg = cfg
        qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        self.wqkv = nn.Linear(cfg.dim, qd + 2 * kvd, bias=False)
        self.wo = nn.Linear(qd, cfg.dim, bias=False)
        if cfg.qk_norm:
            self.q_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)
            self.k_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)

    def forward(self, x, freqs, k_cache_t, v_cache_t, pos, q_pad, zero):
        y = attention_core(self, self.wqkv(x).view(1, -1), freqs, k_cache_t, v_cache_t, pos, q_pad, zero)
        return self.wo(y.view(1, 1, -1))


class GptFastFeedForward(nn.Module):
    """The SiLU-gated MLP under gpt-fast's names (the reference's model.py:248-256):
    w2(silu(w1(x)) * w3(x)), each a module call."""

    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.w1 = nn.Linear(cfg.dim, cfg.inter, bias=False)
        self.w3 = nn.Linear(cfg.dim, cfg.inter, bias=False)
        self.w2 = nn.Linear(cfg.inter, cfg.dim, bias=False)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class GptFastBlock(nn.Module):
    """A decoder layer under gpt-fast's names (the reference's model.py:177-189):
    attention_norm, attention, ffn_norm, feed_forward."""

    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.attention_norm = RMSNorm(cfg.dim, cfg.norm_eps)
        self.attention = GptFastAttention(cfg)
        self.ffn_norm = RMSNorm(cfg.dim, cfg.norm_eps)
        self.feed_forward = GptFastFeedForward(cfg)

    def forward(self, x, freqs, k_cache_t, v_cache_t, pos, q_pad, zero):
        h = x + self.attention(self.attention_norm(x), freqs, k_cache_t, v_cache_t, pos, q_pad, zero)
        return h + self.feed_forward(self.ffn_norm(h))


def fusable(block: Block, dtype=None) -> bool:
    """True when the block's projections can run as the fused sparse layer:
    q/k/v and gate/up each share one launch, o and down are sparse too, and
    (with `dtype`, the activations' type) every packed weight has that type.
    Activations of another type than the packed weights are not fused: the
    projections then run one op at a time, whose own dtype check refuses them
    as the reference wrapper does (triton_spmv.py:245-283)."""
    from ..nmsparse_linear import NmSparseLinear

    if not isinstance(block, Block):
        return False
    at, mlp = block.self_attn, block.mlp
    mods = (at.q_proj, at.k_proj, at.v_proj, at.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj)
    if dtype is not None and not all(getattr(getattr(m, "mat_data", None), "dtype", None) == dtype for m in mods):
        return False
    return (grouped_sparse((at.q_proj, at.k_proj, at.v_proj)) and grouped_sparse((mlp.gate_proj, mlp.up_proj))
            and isinstance(at.o_proj, NmSparseLinear) and isinstance(mlp.down_proj, NmSparseLinear))


def fused_block_step(blk: Block, x2d, k_cache_t, v_cache_t, pos, q_pad, zero, rope):
    """One fused sparse layer on the residual stream x2d [1, dim], updated in
    place. rope: fp32 [S, head_dim/2, 2] (cos, sin) table of the cache's
    positions; caches, q_pad and zero as in attend. Four launches, each a
    `torch.ops.nmsparse` op (so torch.compile traces the step whole)."""
    at, mlp = blk.self_attn, blk.mlp
    c = at.cfg
    qd = c.n_heads * c.head_dim
    ln1, ln2 = blk.input_layernorm, blk.post_attention_layernorm
    qp, kp, vp = at.q_proj, at.k_proj, at.v_proj
    ops = torch.ops.nmsparse
    ops.qkv_decode(x2d, qp.mat_data, qp.mat_index, kp.mat_data, kp.mat_index, vp.mat_data, vp.mat_index,
                   qp.block_width, qp.vec_width, q_pad, k_cache_t, v_cache_t, pos, rope, c.head_dim, ln1.weight,
                   ln1.eps, at.q_norm.weight if c.qk_norm else None, at.k_norm.weight if c.qk_norm else None,
                   c.norm_eps, None)
    y = attend(q_pad, k_cache_t, v_cache_t, c, zero).view(1, qd)
    o = at.o_proj
    ops.gemv_add_(y, o.mat_data, o.mat_index, o.block_width, o.vec_width, x2d)
    gp, up = mlp.gate_proj, mlp.up_proj
    act = ops.gate_up_silu(x2d, gp.mat_data, gp.mat_index, up.mat_data, up.mat_index, gp.block_width, gp.vec_width,
                           ln2.weight, ln2.eps)
    d = mlp.down_proj
    ops.gemv_add_(act, d.mat_data, d.mat_index, d.block_width, d.vec_width, x2d)
    return x2d


def carry_supported(layers) -> bool:
    """True when the fused layers can hand o_proj's and down_proj's split-K
    reduction to the next launch (fused_layers_carried): every layer has the
    first one's shapes, both producers leave at most 16 splits, and both
    consumers' plans (whole groups of columns per split, at most 512 columns
    and 1024 positions of K per split, M a multiple of 4) take a carried
    input. Mirrors the library's checks, so that the choice is made once,
    before any launch, rather than by a launch failing."""
    from ..hip_spmv import carry_splits, launch_plan

    if not layers or not all(fusable(b) for b in layers):
        return False

    def shapes(b):
        at, mlp = b.self_attn, b.mlp
        return tuple(tuple(m.mat_data.shape) + (m.block_width, m.vec_width) for m in
                     (at.q_proj, at.k_proj, at.v_proj, at.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj))

    first = shapes(layers[0])
    if any(shapes(b) != first for b in layers[1:]):
        return False
    at, mlp = layers[0].self_attn, layers[0].mlp
    nnz, m = at.q_proj.block_width, at.q_proj.vec_width
    if m % 4 or any(x.block_width != nnz or x.vec_width != m for x in (at.o_proj, mlp.gate_proj, mlp.down_proj)):
        return False
    for prod in (at.o_proj, mlp.down_proj):
        if carry_splits(prod.mat_data, prod.mat_index, nnz, m) > 16:
            return False
    for mats, pair in (((at.q_proj, at.k_proj, at.v_proj), False), ((mlp.gate_proj, mlp.up_proj), True)):
        plan = launch_plan([(x.mat_data, x.mat_index) for x in mats], nnz, m, gate_up=pair, carried=True)
        rows = plan["rows_per_split"]
        if rows % nnz or rows > 512 or (rows // nnz) * m > 1024:
            return False
    return True


def fused_layers_carried(layers, x2d, h2d, carry_o, carry_d, k_caches, v_caches, pos, q_pad, zero, rope):
    """The fused sparse layers with the split-K reduction of o_proj and
    down_proj carried into the next launch: o_proj and down_proj leave their
    fp32 split partials (carry_o / carry_d) and end without a handoff; the
    gate/up launch finishes h = x + o_proj(y) (the same rounding as o +
    residual) from them, writes h to h2d and runs on it; the next layer's
    q/k/v launch finishes x = h + down_proj(act) into x2d likewise. The first
    layer's q/k/v reads x2d (the embeddings) and the last layer's down_proj
    adds its residual itself. x2d and h2d are [1, dim]; the final residual
    stream is returned (h2d). Four launches per layer, as fused_block_step."""
    ops = torch.ops.nmsparse
    n = len(layers)
    for i, blk in enumerate(layers):
        at, mlp = blk.self_attn, blk.mlp
        c = at.cfg
        ln1, ln2 = blk.input_layernorm, blk.post_attention_layernorm
        qp, kp, vp = at.q_proj, at.k_proj, at.v_proj
        qn = at.q_norm.weight if c.qk_norm else None
        kn = at.k_norm.weight if c.qk_norm else None
        qkv = (qp.mat_data, qp.mat_index, kp.mat_data, kp.mat_index, vp.mat_data, vp.mat_index, qp.block_width,
               qp.vec_width, q_pad, k_caches[i], v_caches[i], pos, rope, c.head_dim, ln1.weight, ln1.eps, qn, kn,
               c.norm_eps)
        if i == 0:
            ops.qkv_decode(x2d, *qkv, None)
        else:
            ops.qkv_decode_carried(h2d, carry_d, x2d, *qkv, None)
        y = attend(q_pad, k_caches[i], v_caches[i], c, zero).view(1, c.n_heads * c.head_dim)
        o = at.o_proj
        ops.gemv_partials_(y, o.mat_data, o.mat_index, o.block_width, o.vec_width, carry_o)
        gp, up = mlp.gate_proj, mlp.up_proj
        act = ops.gate_up_silu_carried(x2d, carry_o, h2d, gp.mat_data, gp.mat_index, up.mat_data, up.mat_index,
                                       gp.block_width, gp.vec_width, ln2.weight, ln2.eps)
        d = mlp.down_proj
        if i + 1 < n:
            ops.gemv_partials_(act, d.mat_data, d.mat_index, d.block_width, d.vec_width, carry_d)
        else:
            ops.gemv_add_(act, d.mat_data, d.mat_index, d.block_width, d.vec_width, h2d)
    return h2d


def fused_layers_accumulated(layers, x2d, h2d, acc_op, acc_d, ssq_n, k_caches, v_caches, pos, q_pad, zero, rope):
    """The fused sparse layers with an accumulated carry: o_proj, the gate/up
    pair and down_proj are producers whose workgroups add their partial sums
    into one fp32 row with atomics (the reference's accumulation medium,
    triton_spmv.py:209-214), and the next launch finishes the epilogue as it
    gathers its input: gate/up finishes h = x + o_proj(y) from acc_o, down_proj
    takes silu(s G) * (s U) from acc_p (the pair's raw sums and sums of
    squares, ssq_n of them), the next q/k/v finishes x = h + down_proj(act)
    from acc_d. acc_o [dim] and acc_p [2 * inter + 16] are one fp32 buffer
    acc_op, which each layer's q/k/v launch clears (after their last readers,
    the previous gate/up and down); the gate/up launch clears acc_d [1, dim]
    (after q/k/v read it). Clearing acc_p in o_proj instead measured 35-40 us
    slower per Llama-3.1-8B step: o_proj is short and its clearing stores
    delay its adds. The order of the atomic adds varies, so the sums' last
    bits (and, through the roundings, the outputs') vary from run to run.
    x2d, h2d, caches, pos, q_pad, zero and rope as for fused_layers_carried;
    the final residual stream is returned (h2d)."""
    ops = torch.ops.nmsparse
    n = len(layers)
    dim = x2d.shape[-1]
    acc_o, acc_p = acc_op[:dim].view(1, dim), acc_op[dim:]
    for i, blk in enumerate(layers):
        at, mlp = blk.self_attn, blk.mlp
        c = at.cfg
        ln1, ln2 = blk.input_layernorm, blk.post_attention_layernorm
        qp, kp, vp = at.q_proj, at.k_proj, at.v_proj
        qn = at.q_norm.weight if c.qk_norm else None
        kn = at.k_norm.weight if c.qk_norm else None
        qkv = (qp.mat_data, qp.mat_index, kp.mat_data, kp.mat_index, vp.mat_data, vp.mat_index, qp.block_width,
               qp.vec_width, q_pad, k_caches[i], v_caches[i], pos, rope, c.head_dim, ln1.weight, ln1.eps, qn, kn,
               c.norm_eps)
        if i == 0:
            ops.qkv_decode(x2d, *qkv, acc_op)
        else:
            ops.qkv_decode_carried(h2d, acc_d, x2d, *qkv, acc_op)
        y = attend(q_pad, k_caches[i], v_caches[i], c, zero).view(1, c.n_heads * c.head_dim)
        o = at.o_proj
        ops.gemv_accumulate_(y, o.mat_data, o.mat_index, o.block_width, o.vec_width, acc_o, None)
        gp, up = mlp.gate_proj, mlp.up_proj
        ops.gate_up_accumulate_(x2d, acc_o, h2d, gp.mat_data, gp.mat_index, up.mat_data, up.mat_index,
                                gp.block_width, gp.vec_width, ln2.weight, ln2.eps, acc_p, acc_d)
        d = mlp.down_proj
        if i + 1 < n:
            ops.gemv_silu_accumulate_(acc_p, d.mat_data, d.mat_index, d.block_width, d.vec_width, ssq_n, dim, ln2.eps,
                                      acc_d, None)
        else:
            ops.gemv_silu_add_(acc_p, d.mat_data, d.mat_index, d.block_width, d.vec_width, ssq_n, dim, ln2.eps, h2d)
    return h2d


def accumulate_supported(layers) -> bool:
    """True when the fused layers can run fused_layers_accumulated: the split
    carry's conditions (carry_supported) and an accumulating gate/up pair of
    at most 16 splits with its carried input (one sum of squares per split)."""
    from ..hip_spmv import gate_up_ssq_slots

    if not carry_supported(layers):
        return False
    mlp = layers[0].mlp
    gp, up = mlp.gate_proj, mlp.up_proj
    return gate_up_ssq_slots((gp.mat_data, gp.mat_index), (up.mat_data, up.mat_index), gp.block_width,
                             gp.vec_width, carried=True) <= 16


class Decoder(nn.Module):
    """Decoder stack with a static KV cache; `model.layers` is what
    `swap_to_nmsparse` walks. layout="hf" (default) builds Hugging Face-named
    blocks (Block: self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj), which
    every launch mode and the fused sparse layer serve; layout="gpt-fast"
    builds gpt-fast-named blocks (GptFastBlock: attention.wqkv / wo,
    feed_forward.w1 / w3 / w2, the reference benchmark's model), which always
    call their projections as modules (the unmodified-model path)."""

    LAYOUTS = ("hf", "gpt-fast")

    def __init__(self, cfg: DecoderConfig, layout: str = "hf"):
        super().__init__()
        if layout not in self.LAYOUTS:
            raise ValueError(f"layout must be one of {self.LAYOUTS}, got {layout!r}")
        self.cfg = cfg
        self.layout = layout
        self.fuse_epilogues = True
        # Fused sparse layers: carry o_proj's / down_proj's split-K reduction
        # into the next launch where the shapes allow. carry_mode
        # "accumulate" (default; fused_layers_accumulated: fp32 atomic adds
        # into one row as the reference kernel accumulates, the gate/up pair
        # a producer too; the sums' last bits vary from run to run) or
        # "split" (fused_layers_carried: fp32 split partials summed in split
        # order, bit-reproducible run to run and graph replay to eager).
        self.carry_splitk = True
        self.carry_mode = "accumulate"
        self._carry = None  # (key, x2d-independent buffers) set up by _carry_buffers
        self.embed_tokens = nn.Embedding(cfg.vocab, cfg.dim)
        block = Block if layout == "hf" else GptFastBlock
        self.layers = nn.ModuleList(block(cfg) for _ in range(cfg.n_layers))
        self.norm = RMSNorm(cfg.dim, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.dim, cfg.vocab, bias=False)
        self.max_seq = 0
        self.gemv_forms = {}  # (n_out, n_in) -> dense_gemv form, filled by tune_dense_gemv
        self.dense_fusion = "none"  # set_dense_fusion's mode

    LAUNCH_MODES = ("fused", "grouped", "per_linear", "modules")
    CARRY_MODES = ("split", "accumulate")

    def set_launch_mode(self, mode: str) -> None:
        """How sparse projections are launched: "fused" (the fused layer, the
        default), "grouped" (one q/k/v and one gate/up launch, norms and RoPE
        in PyTorch), "per_linear" (one launch per Linear, like the reference's
        decode step and the dense model) or "modules" (each projection called
        as a module, lin(x), as model code written for dense Linears does: an
        NmSparseLinear then runs its own forward, so q/k/v and gate/up share a
        launch when swap_to_nmsparse tied them, else one launch each)."""
        if mode not in self.LAUNCH_MODES:
            raise ValueError(f"launch mode must be one of {self.LAUNCH_MODES}, got {mode!r}")
        self.fuse_epilogues = mode == "fused"
        for blk in self.layers:
            if not isinstance(blk, Block):
                continue  # gpt-fast blocks always call their projections as modules
            blk.self_attn.group_launches = blk.mlp.group_launches = mode in ("fused", "grouped")
            blk.self_attn.call_modules = blk.mlp.call_modules = mode == "modules"

    DENSE_FUSIONS = ("none", "qkv", "qkv_gate_up")

    def set_dense_fusion(self, mode: str) -> None:
        """How dense (nn.Linear) projections are launched: "none" (one GEMM per
        Linear), "qkv" (q/k/v as one [q+k+v rows] GEMM, the reference's dense
        model: model.py:198 `wqkv`, model.py:219) or "qkv_gate_up" (also gate/up
        as one GEMM). The fused weights are copies taken now, held outside the
        parameters (so swap_to_nmsparse and state_dict do not see them): change
        the Linears' weights afterwards and set the mode again. Blocks whose
        projections are not all nn.Linear ignore them; "none" frees them."""
        if mode not in self.DENSE_FUSIONS:
            raise ValueError(f"dense fusion must be one of {self.DENSE_FUSIONS}, got {mode!r}")
        self.dense_fusion = mode
        with torch.no_grad():
            for blk in self.layers:
                if not isinstance(blk, Block):
                    continue  # gpt-fast blocks: wqkv is one Linear already
                at, mlp = blk.self_attn, blk.mlp
                projs = (at.q_proj, at.k_proj, at.v_proj)
                at.wqkv = (torch.cat([p.weight for p in projs])
                           if mode != "none" and all(type(p) is nn.Linear for p in projs) else None)
                pair = (mlp.gate_proj, mlp.up_proj)
                mlp.w13 = (torch.cat([p.weight for p in pair])
                           if mode == "qkv_gate_up" and all(type(p) is nn.Linear for p in pair) else None)
        self._apply_gemv_forms()

    def _dense_gemv_sites(self):
        """(weight, owner, attribute) for every dense weight the decode step
        multiplies with dense_gemv: bias-free nn.Linears and the fused copies."""
        sites = []
        for blk in self.layers:
            if not isinstance(blk, Block):
                continue  # gpt-fast blocks call nn.Linear's own forward
            at, mlp = blk.self_attn, blk.mlp
            for mod in (at.q_proj, at.k_proj, at.v_proj, at.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj):
                if type(mod) is nn.Linear and mod.bias is None:
                    sites.append((mod.weight, mod, "gemv_form"))
            if at.wqkv is not None:
                sites.append((at.wqkv, at, "wqkv_form"))
            if mlp.w13 is not None:
                sites.append((mlp.w13, mlp, "w13_form"))
        if type(self.lm_head) is nn.Linear and self.lm_head.bias is None:
            sites.append((self.lm_head.weight, self.lm_head, "gemv_form"))
        return sites

    def _apply_gemv_forms(self):
        for w, owner, attr in self._dense_gemv_sites():
            setattr(owner, attr, self.gemv_forms.get(tuple(w.shape), "mm"))

    def tune_dense_gemv(self, reps: int = 8, warmup: int = 2) -> dict:
        """Choose, per dense weight shape, the faster dense_gemv form on this
        GPU: each form is timed over every weight of that shape in the model
        (all layers in order, so the weights stream from HBM as in a decode
        step), captured in one hipGraph and replayed `reps` times; the median
        replay decides. Shapes already tuned are kept. Returns {"n_out x n_in":
        {"mm": us, "mv": us, "form": ...}} (us per product) for the shapes
        timed now. Changes only how dense products are issued, not their math
        (both forms accumulate in fp32; the roundings can differ in the last bit)."""
        groups = {}
        for w, _, _ in self._dense_gemv_sites():
            if not w.is_cuda:
                raise RuntimeError(f"tune_dense_gemv times the products on the GPU; a dense weight is on {w.device}")
            groups.setdefault(tuple(w.shape), {})[w.data_ptr()] = w
        report = {}
        for shape, ws in groups.items():
            if shape in self.gemv_forms:
                continue
            ws = list(ws.values())
            x = torch.randn(1, shape[1], device=ws[0].device, dtype=ws[0].dtype,
                            generator=torch.Generator(device=ws[0].device).manual_seed(0))
            out = torch.empty(1, shape[0], device=ws[0].device, dtype=ws[0].dtype)
            with torch.no_grad():
                us = {form: _graph_median_us([lambda w=w, f=form: dense_gemv(x, w, f, out=out) for w in ws], reps,
                                             warmup) / len(ws) for form in GEMV_FORMS}
            best = min(GEMV_FORMS, key=us.get)
            self.gemv_forms[shape] = best
            report[f"{shape[0]}x{shape[1]}"] = {**{k: round(v, 2) for k, v in us.items()}, "form": best}
        self._apply_gemv_forms()
        return report

    def setup_cache(self, max_seq: int, device, dtype=torch.float16):
        """Static caches for max_seq positions (see attend for the layouts); the
        key caches of all layers are views of one tensor so that one kernel per
        step rewrites every layer's mask row."""
        c = self.cfg
        self.max_seq = max_seq
        hd, D = c.head_dim, c.head_dim + KEY_PAD
        self.k_store = torch.zeros(c.n_layers, c.n_kv_heads, D, max_seq, device=device, dtype=dtype)
        self.k_cache_t = list(self.k_store.unbind(0))
        self.k_mask = self.k_store[:, :, hd, :]  # [layers, kv_heads, S] view: the mask rows
        self.v_cache_t = [torch.zeros(c.n_kv_heads, hd, max_seq, device=device, dtype=dtype)
                          for _ in range(c.n_layers)]
        self.q_pad = torch.zeros(c.n_heads, D, device=device, dtype=dtype)
        self.q_pad[:, hd] = 1.0
        self.zero = torch.zeros((), device=device, dtype=dtype)
        self.neg_inf = torch.full((), float("-inf"), device=device, dtype=dtype)
        t = torch.arange(max_seq, dtype=torch.float64)
        ang = torch.outer(t, rope_inv_freq(c))
        self.rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(device)
        self.rope_real = torch.view_as_real(self.rope)  # the same table as fp32 (cos, sin) pairs
        self.positions = torch.arange(max_seq, device=device)
        self._carry = None
        self.prepare_decode()

    def prepare_decode(self) -> None:
        """Set up what the fused sparse step needs beyond the caches: the
        buffers of fused_layers_carried (the h stream and the fp32 partials of
        o_proj and down_proj) or, with carry_mode "accumulate", of
        fused_layers_accumulated (the h stream, the fp32 accumulators of
        o_proj and the gate/up pair in one buffer, down_proj's, and the pair's
        count of sums of squares), when the layers
        support the carry. Run by every
        eager step (cheap once done; redone when the layers' shapes change) and
        by the runners before capturing or compiling a step: a step traced by
        torch.compile uses what was prepared before it, and the plain fused
        layers when nothing was."""
        if not self.layers or not hasattr(self, "q_pad"):
            return
        if not all(isinstance(b, Block) for b in self.layers):
            self._carry = ("gpt-fast", None)  # the fused path needs q/k/v as separate matrices
            return
        at, mlp = self.layers[0].self_attn, self.layers[0].mlp
        o, d = at.o_proj, mlp.down_proj
        dev, dt = self.q_pad.device, self.q_pad.dtype
        def shape(mod):  # what the plans depend on: packed shapes and the N:M ratio
            md, mi = getattr(mod, "mat_data", None), getattr(mod, "mat_index", None)
            return (type(mod).__name__, tuple(md.shape) if isinstance(md, torch.Tensor) else None,
                    tuple(mi.shape) if isinstance(mi, torch.Tensor) else None, getattr(mod, "block_width", None),
                    getattr(mod, "vec_width", None))

        key = (dev, dt, len(self.layers), self.carry_mode,
               tuple(shape(mod) for b in self.layers for mod in (b.self_attn.q_proj, b.self_attn.k_proj,
                                                                  b.self_attn.v_proj, b.self_attn.o_proj,
                                                                  b.mlp.gate_proj, b.mlp.up_proj, b.mlp.down_proj)))
        if self._carry is not None and self._carry[0] == key:
            return
        if self.carry_mode not in self.CARRY_MODES:
            raise ValueError(f"carry_mode must be one of {self.CARRY_MODES}, got {self.carry_mode!r}")
        accumulate = self.carry_mode == "accumulate"
        if dev.type != "cuda" or not (accumulate_supported if accumulate else carry_supported)(self.layers):
            self._carry = (key, None)
            return
        from ..hip_spmv import carry_splits, gate_up_ssq_slots

        dim = self.cfg.dim
        if accumulate:
            gp, up = mlp.gate_proj, mlp.up_proj
            inter = gp.mat_data.shape[1]
            ssq_n = gate_up_ssq_slots((gp.mat_data, gp.mat_index), (up.mat_data, up.mat_index), gp.block_width,
                                      gp.vec_width, carried=True)
            f32 = dict(device=dev, dtype=torch.float32)
            self._carry = (key, (torch.empty(1, dim, device=dev, dtype=dt), torch.empty(dim + 2 * inter + 16, **f32),
                                 torch.empty(1, dim, **f32), ssq_n))
            return
        so = carry_splits(o.mat_data, o.mat_index, o.block_width, o.vec_width)
        sd = carry_splits(d.mat_data, d.mat_index, d.block_width, d.vec_width)
        self._carry = (key, (torch.empty(1, dim, device=dev, dtype=dt),
                             torch.empty(so, dim, device=dev, dtype=torch.float32),
                             torch.empty(sd, dim, device=dev, dtype=torch.float32)))

    def reset_cache(self):
        """Zero every cached key and value (the mask rows are rewritten by each step)."""
        self.k_store[:, :, :self.cfg.head_dim].zero_()
        for v in self.v_cache_t:
            v.zero_()

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor) -> torch.Tensor:
        """The prompt in one pass: tokens [P] int64 at positions 0 .. P-1 on
        the device. Every Linear sees all P rows (sparse ones through the SpMM:
        project_rows; q/k/v and gate/up as one grouped SpMM each,
        project_rows_group), causal attention over the prompt in PyTorch
        (causal_attention), keys and values written to the static caches at
        positions 0 .. P-1 as the decode steps write them. Returns the logits
        of position P-1 [1, vocab]; decoding continues at position P (each
        step rewrites the mask rows itself)."""
        c = self.cfg
        ids = tokens.view(-1)
        P = ids.numel()
        if P < 1 or P > self.max_seq:
            raise ValueError(f"prompt of {P} tokens for a cache of {self.max_seq} positions")
        hd = c.head_dim
        x = self.embed_tokens(ids)  # [P, dim]
        freqs = self.rope[:P].view(P, 1, -1)
        qd, kvd = c.n_heads * hd, c.n_kv_heads * hd
        for i, blk in enumerate(self.layers):
            if isinstance(blk, Block):
                at, mlp = blk.self_attn, blk.mlp
                ln1, ln2, o_proj = blk.input_layernorm, blk.post_attention_layernorm, at.o_proj
                gate, up, down = mlp.gate_proj, mlp.up_proj, mlp.down_proj
                h = ln1(x)
                q, k, v = project_rows_group((at.q_proj, at.k_proj, at.v_proj), h)
            else:  # gpt-fast names
                at, ff = blk.attention, blk.feed_forward
                ln1, ln2, o_proj = blk.attention_norm, blk.ffn_norm, at.wo
                gate, up, down = ff.w1, ff.w3, ff.w2
                h = ln1(x)
                q, k, v = project_rows(at.wqkv, h).split([qd, kvd, kvd], dim=-1)
            q, k, v = q.reshape(P, c.n_heads, hd), k.reshape(P, c.n_kv_heads, hd), v.reshape(P, c.n_kv_heads, hd)
            if c.qk_norm:
                q, k = at.q_norm(q), at.k_norm(k)
            q, k = rotate(q, freqs), rotate(k, freqs)
            self.k_cache_t[i][:, :hd, :P].copy_(k.permute(1, 2, 0))
            self.v_cache_t[i][:, :, :P].copy_(v.permute(1, 2, 0))
            x = x + project_rows(o_proj, causal_attention(q, k, v, c.n_kv_heads))
            h = ln2(x)
            g_out, u_out = project_rows_group((gate, up), h)
            x = x + project_rows_silu_mul(down, g_out, u_out)
        return project(self.lm_head, self.norm(x[-1:].view(1, 1, -1))).view(1, -1)

    def forward_step(self, token: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One decode step: token [1, 1] int64 and pos [1] int64 on the device
        -> logits [1, vocab]. No host synchronisation."""
        x = self.embed_tokens(token)  # [1, 1, dim]
        # causal mask of this step in every layer's key cache: 0 up to pos, -inf after
        keep = (self.positions <= pos).expand_as(self.k_mask)
        if torch.compiler.is_compiling():  # the tracer takes no strided out=; the compiler fuses the copy
            self.k_mask.copy_(torch.where(keep, self.zero, self.neg_inf))
        else:
            torch.where(keep, self.zero, self.neg_inf, out=self.k_mask)
        if self.fuse_epilogues and all(fusable(b, x.dtype) and b.self_attn.group_launches for b in self.layers):
            x2d = x.view(1, -1)
            if not torch.compiler.is_compiling():
                self.prepare_decode()
            bufs = self._carry[1] if (self.carry_splitk and self._carry is not None) else None
            if bufs is not None:
                run = fused_layers_accumulated if len(bufs) == 4 else fused_layers_carried
                h2d = run(self.layers, x2d, *bufs, self.k_cache_t, self.v_cache_t, pos, self.q_pad, self.zero,
                          self.rope_real)
                return project(self.lm_head, self.norm(h2d.view(1, 1, -1))).view(1, -1)
            for i, blk in enumerate(self.layers):
                fused_block_step(blk, x2d, self.k_cache_t[i], self.v_cache_t[i], pos, self.q_pad, self.zero,
                                 self.rope_real)
            return project(self.lm_head, self.norm(x)).view(1, -1)
        freqs = (self.rope_real if torch.compiler.is_compiling() else self.rope).index_select(0, pos)
        for i, layer in enumerate(self.layers):
            x = layer(x, freqs, self.k_cache_t[i], self.v_cache_t[i], pos, self.q_pad, self.zero)
        return project(self.lm_head, self.norm(x)).view(1, -1)


def _graph_median_us(launches, reps: int, warmup: int) -> float:
    """Median time of one replay of `launches` captured as one hipGraph, in us."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in launches:  # library handles and workspaces are set up outside the capture
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for fn in launches:
            fn()
    for _ in range(warmup):
        graph.replay()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e3)
    del graph
    return sorted(times)[len(times) // 2]


def init_weights_(model: Decoder, seed: int = 0, std: float = 0.02) -> Decoder:
    """Random-init every weight in place on its device (N(0, std) for
    matrices and embeddings, ones for norms)."""
    gen = torch.Generator(device=next(model.parameters()).device).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=gen)
    return model
