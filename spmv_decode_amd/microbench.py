"""Kernel timing harness for the N:M sparse GEMV (role of the reference's
microbench_triton_torchmv.py, re-designed for MI355X).

    python -m spmv_decode_amd.microbench [--dims 4096x4096,...] [--ratios 2:4,...]
        [--dtype fp16|bf16] [--sweep] [--rotate-mib 1024] [--csv out.csv]

Differences from the reference harness (microbench_triton_torchmv.py:218-364):
* Weights are rotated over enough distinct copies (default >= 1 GiB) that
  every timed launch streams from HBM, not from the 256 MB Infinity Cache.
* Launches are captured in a hipGraph (the rotation repeated to >= 64
  launches, as many as a decode step's graph holds) and replayed; time per
  launch is the replay time divided by the number of launches (HIP events on
  the stream).
* `--sweep` times every kernel configuration and split count of the static
  table (the replacement for Triton autotuning, triton_spmv.py:40-55,
  122-148) and reports the fastest; the library's own choice is `cfg=-1`.
* Correctness uses the harness's own fp32 dense reference on the scattered
  masked weight, like the reference (microbench_triton_torchmv.py:371-430),
  and reports max_abs / mean_abs / rmse / rel_l2.
"""
from __future__ import annotations

import argparse
import csv
import json
import math
import statistics
import sys
from pathlib import Path

import torch

from . import _lib
from .decode.model import KEY_PAD
from .hip_spmv import nmsparse_spmv_forward_hip

HBM_PEAK_GBS = 8000.0
DEFAULT_DIMS = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]  # (n_out, n_in) Llama-3.1-8B
DEFAULT_RATIOS = [(2, 4), (4, 8), (8, 16), (16, 32), (32, 64), (64, 128), (128, 256)]
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def sparse_bytes(n_in: int, n_out: int, nnz: int, m: int, elem: int = 2) -> int:
    """Algorithmic bytes of one GEMV: packed weights + index bytes + activations + outputs."""
    w = (n_in // m) * nnz
    return elem * w * n_out + w + elem * n_in + elem * n_out


def dense_bytes(n_in: int, n_out: int, elem: int = 2) -> int:
    return elem * n_in * n_out + elem * n_in + elem * n_out


def make_patterns(banks: int, m: int, nnz: int, gen: torch.Generator, device) -> torch.Tensor:
    """Seeded random sorted in-group positions [banks, nnz] uint8 on `device`."""
    keys = torch.rand(banks, m, generator=gen, device=device)
    return keys.argsort(dim=1)[:, :nnz].sort(dim=1).values.to(torch.uint8).contiguous()


class RotatingCase:
    """`copies` independent packed weights of one shape, plus one activation vector."""

    def __init__(self, n_out, n_in, nnz, m, dtype=torch.float16, rotate_bytes=1 << 30, min_copies=1,
                 seed=0, device="cuda", wstd=0.02):
        self.n_out, self.n_in, self.nnz, self.m, self.dtype = n_out, n_in, nnz, m, dtype
        self.w = (n_in // m) * nnz
        self.bytes = sparse_bytes(n_in, n_out, nnz, m, torch.finfo(dtype).bits // 8)
        self.copies = max(min_copies, math.ceil(rotate_bytes / self.bytes))
        g = torch.Generator(device=device).manual_seed(seed)
        banks = n_in // m
        self.mats = []
        for _ in range(self.copies):
            mi = make_patterns(banks, m, nnz, g, device)
            md = (torch.randn(self.w, n_out, generator=g, device=device) * wstd).to(dtype)
            self.mats.append((md, mi))
        self.x = torch.randn(1, n_in, generator=g, device=device).to(dtype)
        self.out = torch.empty(1, n_out, dtype=dtype, device=device)

    def launch(self, i, config_id=-1, splits=0):
        md, mi = self.mats[i % self.copies]
        return nmsparse_spmv_forward_hip(self.x, md, mi, self.w, self.n_out, self.nnz, 128, self.m, 1, self.n_in,
                                         out=self.out, config_id=config_id, splits=splits)


def graph_us_per_launch(launches, reps=20, warmup=3, stream=None, stats=False, min_launches=64):
    """Capture `launches` (callables) in one hipGraph, the list repeated until
    the graph holds at least `min_launches` launches; median replay time per
    launch in us (with stats=True: (median, sample stdev) over the `reps`
    replays). A replay's own fixed cost (the graph launch and its first
    dispatch, a few us) is thereby spread over as many launches as in a decode
    step's graph (128 GEMV launches for Llama-3.1-8B) instead of over a short
    rotation (9 copies of the gate/up pair per GiB); repeating the rotation
    keeps every copy's reuse distance >= the rotated bytes."""
    launches = list(launches)
    seq = launches * max(1, math.ceil(min_launches / len(launches)))
    stream = stream or torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in launches:
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in seq:
            fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    samples = []
    for _ in range(reps):
        s.record()
        g.replay()
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e) * 1e3 / len(seq))
    del g
    med = statistics.median(samples)
    if stats:
        return med, (statistics.stdev(samples) if len(samples) > 1 else 0.0)
    return med


def dense_reference_check(case: RotatingCase, out: torch.Tensor) -> dict:
    """fp32 dense matvec on the scattered masked weight vs `out` (copy 0)."""
    md, mi = case.mats[0]
    pos = (torch.arange(case.w, device=md.device) // case.nnz) * case.m + mi.reshape(-1).long()
    dense = torch.zeros(case.n_out, case.n_in, dtype=torch.float32, device=md.device)
    dense[:, pos] = md.float().t()
    ref = torch.mv(dense, case.x.float().reshape(-1))
    d = (ref - out.float().reshape(-1)).abs()
    return {"max_abs": d.max().item(), "mean_abs": d.mean().item(), "rmse": d.pow(2).mean().sqrt().item(),
            "rel_l2": (d.norm() / ref.norm().clamp_min(1e-12)).item()}


def time_sparse(case: RotatingCase, config_id=-1, splits=0, reps=20, warmup=3, stats=False):
    return graph_us_per_launch([lambda i=i: case.launch(i, config_id, splits) for i in range(case.copies)], reps,
                               warmup, stats=stats)


def time_grouped(cases, reps=20) -> float:
    """One grouped launch over `cases` (RotatingCase list with equal copies,
    sharing cases[0].x) per rotation step; us per launch."""
    from .hip_spmv import nmsparse_gemv_grouped

    c0 = cases[0]
    copies = min(c.copies for c in cases)

    def launch(i):
        nmsparse_gemv_grouped(c0.x, [c.mats[i] for c in cases], c0.nnz, c0.m, outs=[c.out for c in cases])

    return graph_us_per_launch([lambda i=i: launch(i) for i in range(copies)], reps)


def time_pair(gate: RotatingCase, up: RotatingCase, reps=20, config_id=-1, splits=0) -> float:
    """One gate/up SiLU pair launch per rotation step; us per launch."""
    from .hip_spmv import nmsparse_gate_up_silu

    copies = min(gate.copies, up.copies)

    def launch(i):
        nmsparse_gate_up_silu(gate.x, gate.mats[i], up.mats[i], gate.nnz, gate.m, out=gate.out,
                              config_id=config_id, splits=splits)

    return graph_us_per_launch([lambda i=i: launch(i) for i in range(copies)], reps)


def grouped_bytes(cases) -> int:
    """Algorithmic bytes of one grouped launch: every problem's weights, index
    bytes and outputs, the shared activations once."""
    c0 = cases[0]
    elem = torch.finfo(c0.dtype).bits // 8
    return sum(elem * c.w * c.n_out + c.w + elem * c.n_out for c in cases) + elem * c0.n_in


def pair_bytes(gate: RotatingCase, up: RotatingCase) -> int:
    """Algorithmic bytes of one gate/up pair launch: both weights and index
    tables, the activations once, one output."""
    elem = torch.finfo(gate.dtype).bits // 8
    return 2 * (elem * gate.w * gate.n_out + gate.w) + elem * gate.n_in + elem * gate.n_out


def decode_form_bytes(cls, nnz=32, m=64, dim=4096, inter=14336, qd=4096, kvd=1024, hd=128, qk_norm=False) -> int:
    """Algorithmic bytes of one decode-form launch (fp16): packed weights and
    index bytes, activations once, norm weights (Qwen3's per-head q/k norms
    with qk_norm), residual reads, outputs (the k/v outputs are the cache slots
    written) and the RoPE table row."""
    wd, wi, wq = dim // m * nnz, inter // m * nnz, qd // m * nnz
    if cls == "qkv_decode":
        return (sum(2 * wd * h + wd for h in (qd, kvd, kvd)) + 2 * dim + 2 * dim + 2 * (qd + 2 * kvd) + 8 * (hd // 2)
                + (4 * hd if qk_norm else 0))
    if cls == "o_resid":
        return 2 * wq * dim + wq + 2 * qd + 2 * dim + 2 * dim
    if cls == "gate_up_pair_norm":
        return 2 * (2 * wd * inter + wd) + 2 * dim + 2 * dim + 2 * inter
    if cls == "down_resid":
        return 2 * wi * dim + wi + 2 * inter + 2 * dim + 2 * dim
    # split-K carry: the producers read weights, index and input only; each
    # consumer also reads the residual stream and writes the finished vector
    # (the split partials passed between them are not counted, as the
    # partials of every split-K launch are not)
    if cls == "o_partials":
        return 2 * wq * dim + wq + 2 * qd
    if cls == "down_partials":
        return 2 * wi * dim + wi + 2 * inter
    if cls in ("qkv_decode_carried", "gate_up_pair_norm_carried"):
        return decode_form_bytes(cls[:-len("_carried")], nnz, m, dim, inter, qd, kvd, hd, qk_norm) + 2 * dim
    # accumulated carry: the same work as the split carry's launch in the same place (the fp32 rows passed
    # between them are not counted, as split partials are not)
    same = {"qkv_decode_acc": "qkv_decode_carried", "o_acc": "o_partials",
            "gate_up_pair_acc": "gate_up_pair_norm_carried", "down_silu_acc": "down_partials"}
    if cls in same:
        return decode_form_bytes(same[cls], nnz, m, dim, inter, qd, kvd, hd, qk_norm)
    raise ValueError(cls)


class DecodeForms:
    """The four launches of one fused decoder layer as the decoder issues them
    (Llama-3.1-8B shapes): q/k/v with the input RMSNorm, RoPE and the KV-cache
    write; o with the residual add; gate/up with the post-attention RMSNorm
    and SiLU*mul; down with the residual add. Each class rotates over its own
    packed weights (>= rotate_bytes); activations, norms, cache and position
    are shared and fixed (no residual accumulates across replays)."""

    KV_SLOTS = 512

    def __init__(self, nnz=32, m=64, rotate_bytes=1 << 30, dim=4096, inter=14336, n_heads=32, n_kv_heads=8,
                 head_dim=128, device="cuda", seed=50, min_copies=1, qk_norm=False):
        self.nnz, self.m, self.hd, self.qk_norm = nnz, m, head_dim, qk_norm
        self.dim, self.inter = dim, inter
        qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
        self.hs = {"q": qd, "kv": kvd}
        w_dim = dim // m * nnz
        qkv_b = sum(2 * w_dim * h + w_dim for h in (qd, kvd, kvd))
        cq = max(min_copies, math.ceil(rotate_bytes / qkv_b))
        self.q = RotatingCase(qd, dim, nnz, m, rotate_bytes=0, min_copies=cq, seed=seed, device=device)
        self.k = RotatingCase(kvd, dim, nnz, m, rotate_bytes=0, min_copies=cq, seed=seed + 1, device=device)
        self.v = RotatingCase(kvd, dim, nnz, m, rotate_bytes=0, min_copies=cq, seed=seed + 2, device=device)
        self.o = RotatingCase(dim, qd, nnz, m, rotate_bytes=rotate_bytes, min_copies=min_copies, seed=seed + 3,
                              device=device)
        pair_b = 2 * (2 * w_dim * inter + w_dim)
        cp = max(min_copies, math.ceil(rotate_bytes / pair_b))
        self.gate = RotatingCase(inter, dim, nnz, m, rotate_bytes=0, min_copies=cp, seed=seed + 4, device=device)
        self.up = RotatingCase(inter, dim, nnz, m, rotate_bytes=0, min_copies=cp, seed=seed + 5, device=device)
        self.down = RotatingCase(dim, inter, nnz, m, rotate_bytes=rotate_bytes, min_copies=min_copies,
                                 seed=seed + 6, device=device)
        g = torch.Generator(device=device).manual_seed(seed + 7)
        f16 = torch.float16
        self.x = torch.randn(1, dim, generator=g, device=device).to(f16)
        self.attn = torch.randn(1, qd, generator=g, device=device).to(f16)
        self.act = torch.randn(1, inter, generator=g, device=device).to(f16) * 0.1
        self.h1 = torch.empty(1, dim, dtype=f16, device=device)
        self.h2 = torch.empty(1, dim, dtype=f16, device=device)
        self.ln1 = (torch.rand(dim, generator=g, device=device) + 0.5).to(f16)
        self.ln2 = (torch.rand(dim, generator=g, device=device) + 0.5).to(f16)
        self.q_norm = self.k_norm = None
        if qk_norm:  # Qwen3's per-head norms, folded into the q/k/v launch as the decoder does
            self.q_norm = (torch.rand(head_dim, generator=g, device=device) + 0.5).to(f16)
            self.k_norm = (torch.rand(head_dim, generator=g, device=device) + 0.5).to(f16)
        self.qo = torch.zeros(n_heads, head_dim + KEY_PAD, dtype=f16, device=device)  # the decoder's query rows
        self.pair_out = torch.empty(1, inter, dtype=f16, device=device)
        S = self.KV_SLOTS
        self.k_cache = torch.zeros(n_kv_heads, head_dim + KEY_PAD, S, dtype=f16, device=device)
        self.v_cache = torch.zeros(n_kv_heads, head_dim, S, dtype=f16, device=device)  # transposed, as the decoder
        ang = torch.outer(torch.arange(S, dtype=torch.float64),
                          1.0 / (500000.0 ** (torch.arange(head_dim // 2, dtype=torch.float64) * 2.0 / head_dim)))
        self.rope = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(device)
        self.pos = torch.tensor([S // 2], device=device)
        self.copies = {"qkv_decode": cq, "o_resid": self.o.copies, "gate_up_pair_norm": cp,
                       "down_resid": self.down.copies}
        self.copies.update({"qkv_decode_carried": cq, "o_partials": self.o.copies, "gate_up_pair_norm_carried": cp,
                            "down_partials": self.down.copies})
        # split-K carry: the producers' fp32 partials and the consumers' finished vectors
        from .hip_spmv import carry_splits

        self.carry_o = torch.zeros(carry_splits(*self.o.mats[0], nnz, m), dim, device=device)
        self.carry_d = torch.zeros(carry_splits(*self.down.mats[0], nnz, m), dim, device=device)
        self.x_fin, self.h_fin = (torch.empty(1, dim, dtype=f16, device=device) for _ in range(2))
        # accumulated carry: o's and the pair's rows in one buffer (cleared by q/k/v), down's row (cleared by
        # the pair), as the decoder keeps them
        from .hip_spmv import gate_up_ssq_slots

        self.copies.update({"qkv_decode_acc": cq, "o_acc": self.o.copies, "gate_up_pair_acc": cp,
                            "down_silu_acc": self.down.copies})
        self.acc_op = torch.zeros(dim + 2 * inter + 16, device=device)
        self.acc_o, self.acc_p = self.acc_op[:dim].view(1, dim), self.acc_op[dim:]
        self.acc_d = torch.zeros(1, dim, device=device)
        self.ssq_n = gate_up_ssq_slots(self.gate.mats[0], self.up.mats[0], nnz, m, carried=True)

    def launch(self, cls, i, config_id=-1, splits=0):
        from .hip_spmv import GemvProblem, nmsparse_gate_up_silu, nmsparse_gemv_launch, nmsparse_qkv_decode

        nnz, m = self.nnz, self.m
        kw = dict(config_id=config_id, splits=splits)
        if cls == "qkv_decode":
            nmsparse_qkv_decode(self.x, self.q.mats[i], self.k.mats[i], self.v.mats[i], nnz, m, q_out=self.qo,
                                k_cache_t=self.k_cache, v_cache_t=self.v_cache, pos=self.pos, rope_table=self.rope,
                                head_dim=self.hd, norm=(self.ln1, 1e-5), q_norm=self.q_norm, k_norm=self.k_norm, **kw)
        elif cls == "o_resid":
            nmsparse_gemv_launch(self.attn, [GemvProblem(*self.o.mats[i], self.h1, residual=self.x)], nnz, m, **kw)
        elif cls == "gate_up_pair_norm":
            nmsparse_gate_up_silu(self.h1, self.gate.mats[i], self.up.mats[i], nnz, m, out=self.pair_out,
                                  norm=(self.ln2, 1e-5), **kw)
        elif cls == "down_resid":
            nmsparse_gemv_launch(self.act, [GemvProblem(*self.down.mats[i], self.h2, residual=self.h1)], nnz, m,
                                 **kw)
        elif cls == "o_partials":
            nmsparse_gemv_launch(self.attn, [GemvProblem(*self.o.mats[i])], nnz, m, carry_out=self.carry_o, **kw)
        elif cls == "gate_up_pair_norm_carried":
            nmsparse_gate_up_silu(self.x, self.gate.mats[i], self.up.mats[i], nnz, m, out=self.pair_out,
                                  norm=(self.ln2, 1e-5), carry_in=self.carry_o, vec_out=self.h_fin, **kw)
        elif cls == "down_partials":
            nmsparse_gemv_launch(self.act, [GemvProblem(*self.down.mats[i])], nnz, m, carry_out=self.carry_d, **kw)
        elif cls == "qkv_decode_carried":
            nmsparse_qkv_decode(self.x, self.q.mats[i], self.k.mats[i], self.v.mats[i], nnz, m, q_out=self.qo,
                                k_cache_t=self.k_cache, v_cache_t=self.v_cache, pos=self.pos, rope_table=self.rope,
                                head_dim=self.hd, norm=(self.ln1, 1e-5), q_norm=self.q_norm, k_norm=self.k_norm,
                                carry_in=self.carry_d, vec_out=self.x_fin, **kw)
        elif cls == "qkv_decode_acc":
            nmsparse_qkv_decode(self.x, self.q.mats[i], self.k.mats[i], self.v.mats[i], nnz, m, q_out=self.qo,
                                k_cache_t=self.k_cache, v_cache_t=self.v_cache, pos=self.pos, rope_table=self.rope,
                                head_dim=self.hd, norm=(self.ln1, 1e-5), q_norm=self.q_norm, k_norm=self.k_norm,
                                carry_in=self.acc_d, vec_out=self.x_fin, zero=self.acc_op, **kw)
        elif cls == "o_acc":
            nmsparse_gemv_launch(self.attn, [GemvProblem(*self.o.mats[i])], nnz, m, carry_out=self.acc_o,
                                 carry_accumulate=True, **kw)
        elif cls == "gate_up_pair_acc":
            nmsparse_gemv_launch(self.x, [GemvProblem(*self.gate.mats[i]), GemvProblem(*self.up.mats[i])], nnz, m,
                                 gate_up=True, norm=(self.ln2, 1e-5), carry_in=self.acc_o, vec_out=self.h_fin,
                                 carry_out=self.acc_p, carry_accumulate=True, zero=self.acc_d, **kw)
        elif cls == "down_silu_acc":
            nmsparse_gemv_launch(None, [GemvProblem(*self.down.mats[i])], nnz, m, carry_out=self.acc_d,
                                 carry_accumulate=True, silu_in=self.acc_p, silu_ssq_n=self.ssq_n, silu_k=self.dim,
                                 silu_eps=1e-5, **kw)
        else:
            raise ValueError(cls)

    def bytes(self, cls) -> int:
        return decode_form_bytes(cls, self.nnz, self.m, self.dim, self.inter, self.hs["q"], self.hs["kv"], self.hd,
                                 self.qk_norm)

    def time(self, cls, reps=20) -> float:
        return graph_us_per_launch([lambda i=i: self.launch(cls, i) for i in range(self.copies[cls])], reps)


DECODE_CLASSES = ("qkv_decode", "o_resid", "gate_up_pair_norm", "down_resid")
# The same layer with the split-K carry (Decoder.carry_mode "split", bit-reproducible):
# o and down leave their partials, gate/up and the next q/k/v finish them.
CARRIED_CLASSES = ("qkv_decode_carried", "o_partials", "gate_up_pair_norm_carried", "down_partials")
# The same layer with the accumulated carry (the decoder's default, Decoder.carry_mode "accumulate"): o,
# the gate/up pair and down add into fp32 rows; gate/up, down and the next q/k/v finish them.
ACCUMULATED_CLASSES = ("qkv_decode_acc", "o_acc", "gate_up_pair_acc", "down_silu_acc")


def time_spmm(n_out, n_in, nnz, m, batch, rotate_bytes=1 << 30, reps=20, seed=60, matrix_cores=None) -> float:
    """us per SpMM call of `batch` rows (matrix_cores=None: the library's
    choice, the small-batch SpMM up to 8 rows, then the matrix-core SpMM or the
    gather + hipBLASLt route, hip_spmv.library_route; True: the matrix-core
    kernel), weights rotated."""
    from .hip_spmv import nmsparse_spmm_forward_hip

    case = RotatingCase(n_out, n_in, nnz, m, rotate_bytes=rotate_bytes, seed=seed)
    X = torch.randn(batch, n_in, device="cuda").to(case.dtype)
    out = torch.empty(batch, n_out, dtype=case.dtype, device="cuda")

    def launch(i):
        md, mi = case.mats[i]
        nmsparse_spmm_forward_hip(X, md, mi, case.w, n_out, nnz, m, out=out, matrix_cores=matrix_cores)

    us = graph_us_per_launch([lambda i=i: launch(i) for i in range(case.copies)], reps)
    del case
    return us


def time_gather_gemm(n_out, n_in, nnz, m, batch, rotate_bytes=1 << 30, reps=20, seed=60) -> float:
    """us per call of the library route for the same product: the gathered
    activations (nm_gather_columns, [batch, w]) times the packed weights as one
    hipBLASLt GEMM (torch.matmul), weights rotated as in time_spmm."""
    from . import _lib

    case = RotatingCase(n_out, n_in, nnz, m, rotate_bytes=rotate_bytes, seed=seed)
    X = torch.randn(batch, n_in, device="cuda").to(case.dtype)
    out = torch.empty(batch, n_out, dtype=case.dtype, device="cuda")
    wp = (case.w + 7) // 8 * 8
    xg = torch.empty(batch, wp, dtype=case.dtype, device="cuda")
    lib = _lib.load()

    def launch(i):
        md, mi = case.mats[i]
        rc = lib.nm_gather_columns(_lib.NM_DTYPE_F16, X.data_ptr(), n_in, batch, mi.data_ptr(), case.w, nnz, m,
                                   xg.data_ptr(), wp, torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "nm_gather_columns")
        torch.matmul(xg[:, :case.w], md, out=out)

    us = graph_us_per_launch([lambda i=i: launch(i) for i in range(case.copies)], reps)
    del case
    return us


# name: (outputs, inputs, N, M) of the products a batched decode or a prompt runs through the SpMM
SPMM_COMPARE_SHAPES = {
    "Llama-3.1-8B q/o": (4096, 4096, 32, 64), "Llama-3.1-8B k/v": (1024, 4096, 32, 64),
    "Llama-3.1-8B gate/up": (14336, 4096, 32, 64), "Llama-3.1-8B down": (4096, 14336, 32, 64),
    "Qwen3-14B q/o": (5120, 5120, 32, 64), "Qwen3-14B k/v": (1024, 5120, 32, 64),
    "Qwen3-14B gate/up": (17408, 5120, 32, 64), "Qwen3-14B down": (5120, 17408, 32, 64),
    "Qwen3-32B q": (8192, 5120, 16, 32), "Qwen3-32B o": (5120, 8192, 16, 32), "Qwen3-32B k/v": (1024, 5120, 16, 32),
    "Qwen3-32B gate/up": (25600, 5120, 16, 32), "Qwen3-32B down": (5120, 25600, 16, 32),
}


def spmm_compare(shapes=SPMM_COMPARE_SHAPES, rows=(9, 16, 32, 64, 96, 128), reps=20, log=print):
    """The matrix-core SpMM (its default plan, the activation gather included)
    beside the library route (the same gather, then one hipBLASLt GEMM) per
    shape and row count: us per call, weight bytes per second, graph replay
    over >= 1 GiB of rotated weights."""
    out = {}
    for name, (h, K, nnz, m) in shapes.items():
        wbytes = (K // m * nnz) * h * 2
        for b in rows:
            mc = time_spmm(h, K, nnz, m, b, reps=reps, matrix_cores=True)
            lib = time_gather_gemm(h, K, nnz, m, b, reps=reps)
            out[f"{name}|{b}"] = {"shape": name, "rows": b, "weight_bytes": wbytes, "matrix_core_us": round(mc, 3),
                                  "library_us": round(lib, 3), "matrix_core_weight_GBps": round(wbytes / mc / 1e3, 1),
                                  "speedup": round(lib / mc, 3)}
            log(f"spmm {name:22s} {b:3d} rows: matrix-core {mc:7.2f} us ({wbytes / mc / 1e3:6.0f} GB/s), "
                f"gather + hipBLASLt {lib:7.2f} us ({lib / mc:.2f}x)")
        torch.cuda.empty_cache()
    return out


def write_spmm_compare_md(res, path, cmd):
    lines = ["# Matrix-core SpMM against gather + hipBLASLt (MI355X, fp16)", "",
             "Command (repository root, one MI355X):", "", "```", cmd, "```", "",
             "Per shape and activation-row count: `nm_spmm_mc` with its default plan (`nmsparse_spmm_forward_hip(...,",
             "matrix_cores=True)`: the activation gather into operand order, then the matrix-core kernel) and the",
             "library route for the same product (`nm_gather_columns`, then one `torch.matmul` of the gathered",
             "activations and `mat_data`, hipBLASLt). us per call, median of graph replays over >= 1 GiB of rotated",
             "weights (`microbench.time_spmm`, `time_gather_gemm`); GB/s counts the packed weight bytes.", "",
             "| Shape | Rows | Weight bytes | matrix-core us | GB/s | gather + hipBLASLt us | speedup |",
             "|---|---|---|---|---|---|---|"]
    for r in res.values():
        lines.append(f"| {r['shape']} | {r['rows']} | {r['weight_bytes']:,} | {r['matrix_core_us']:.2f} | "
                     f"{r['matrix_core_weight_GBps']:.0f} | {r['library_us']:.2f} | {r['speedup']:.2f}x |")
    Path(path).write_text("\n".join(lines) + "\n")


def time_spmm_group(hs, n_in, nnz, m, batch, rotate_bytes=1 << 30, reps=20, seed=80) -> tuple:
    """us per call of sibling products of one input (output widths hs):
    (grouped, separate) = nmsparse_spmm_group_hip (one gather and one
    matrix-core launch for all of them) and one nmsparse_spmm_forward_hip per
    product, weights rotated over >= rotate_bytes as in time_spmm."""
    from .hip_spmv import nmsparse_spmm_forward_hip, nmsparse_spmm_group_hip

    group_bytes = sum(sparse_bytes(n_in, h, nnz, m, 2) for h in hs)
    copies = max(1, math.ceil(rotate_bytes / group_bytes))
    cases = [RotatingCase(h, n_in, nnz, m, rotate_bytes=0, min_copies=copies, seed=seed + i) for i, h in enumerate(hs)]
    X = torch.randn(batch, n_in, device="cuda").to(cases[0].dtype)
    sets = [[c.mats[i] for c in cases] for i in range(copies)]
    grouped = graph_us_per_launch([lambda st=st: nmsparse_spmm_group_hip(X, st, nnz, m) for st in sets], reps)
    separate = graph_us_per_launch(
        [lambda st=st: [nmsparse_spmm_forward_hip(X, md, mi, md.shape[0], md.shape[1], nnz, m) for md, mi in st]
         for st in sets], reps)
    del cases, sets
    return grouped, separate


# name: (output widths, inputs, N, M) of sibling products of one input
SPMM_GROUP_SHAPES = {
    "Llama-3.1-8B q/k/v": ((4096, 1024, 1024), 4096, 32, 64), "Llama-3.1-8B gate/up": ((14336, 14336), 4096, 32, 64),
    "Qwen3-14B q/k/v": ((5120, 1024, 1024), 5120, 32, 64), "Qwen3-14B gate/up": ((17408, 17408), 5120, 32, 64),
    "Qwen3-32B q/k/v": ((8192, 1024, 1024), 5120, 16, 32), "Qwen3-32B gate/up": ((25600, 25600), 5120, 16, 32),
}


def spmm_group(shapes=SPMM_GROUP_SHAPES, rows=(9, 16, 32, 64, 96, 128), reps=20, log=print):
    """Grouped against separate matrix-core SpMMs of sibling products per
    shape and row count: us per call and the group's weight bytes per second."""
    out = {}
    for name, (hs, K, nnz, m) in shapes.items():
        wbytes = sum((K // m * nnz) * h * 2 for h in hs)
        for b in rows:
            g, sep = time_spmm_group(hs, K, nnz, m, b, reps=reps)
            out[f"{name}|{b}"] = {"shape": name, "rows": b, "weight_bytes": wbytes, "grouped_us": round(g, 3),
                                  "separate_us": round(sep, 3), "grouped_weight_GBps": round(wbytes / g / 1e3, 1),
                                  "speedup": round(sep / g, 3)}
            log(f"spmm group {name:22s} {b:3d} rows: grouped {g:7.2f} us ({wbytes / g / 1e3:6.0f} GB/s), "
                f"separate {sep:7.2f} us ({sep / g:.2f}x)")
        torch.cuda.empty_cache()
    return out


def write_spmm_group_md(res, path, cmd):
    lines = ["# Grouped matrix-core SpMM of sibling products (MI355X, fp16)", "",
             "Command (repository root, one MI355X):", "", "```", cmd, "```", "",
             "Per group of sibling products of one input and activation-row count: `nm_spmm_mc_group` through",
             "`nmsparse_spmm_group_hip` (one gather launch for every product's activations, one matrix-core launch",
             "over all their tiles; the default plan) against one `nmsparse_spmm_forward_hip` call per product (a",
             "gather and a matrix-core launch each). us per call of the whole group, median of graph replays over",
             ">= 1 GiB of rotated weights (`microbench.time_spmm_group`); GB/s counts the group's packed weight",
             "bytes.", "",
             "| Group | Rows | Weight bytes | grouped us | GB/s | separate us | speedup |",
             "|---|---|---|---|---|---|---|"]
    for r in res.values():
        lines.append(f"| {r['shape']} | {r['rows']} | {r['weight_bytes']:,} | {r['grouped_us']:.2f} | "
                     f"{r['grouped_weight_GBps']:.0f} | {r['separate_us']:.2f} | {r['speedup']:.2f}x |")
    Path(path).write_text("\n".join(lines) + "\n")


def time_dense(n_out, n_in, dtype=torch.float16, rotate_bytes=1 << 30, reps=20, seed=1, device="cuda", warmup=3,
               stats=False, form="best", return_form=False):
    """Dense GEMV y = x * W^T through the BLAS library, weights rotated over
    `rotate_bytes`, graph-replayed. form: "mm" (a one-row product x * W^T, what
    nn.Linear issues), "mv" (W * x) or "best" (both timed, the faster kept:
    the library serves the two with different kernels and neither wins at
    every shape). Returns us per launch ((median, sd) with stats=True), and
    with return_form=True also the form that took it: (time, form)."""
    from .decode.model import dense_gemv

    b = dense_bytes(n_in, n_out, torch.finfo(dtype).bits // 8)
    copies = max(1, math.ceil(rotate_bytes / b))
    g = torch.Generator(device=device).manual_seed(seed)
    Ws = [(torch.randn(n_out, n_in, generator=g, device=device) * 0.02).to(dtype) for _ in range(copies)]
    x = torch.randn(1, n_in, generator=g, device=device).to(dtype)
    o = torch.empty(1, n_out, dtype=dtype, device=device)
    res = {}
    for f in (("mm", "mv") if form == "best" else (form,)):
        res[f] = graph_us_per_launch([lambda W=W, f=f: dense_gemv(x, W, f, out=o) for W in Ws], reps, warmup,
                                     stats=stats)
    del Ws
    best = min(res, key=lambda f: res[f][0] if stats else res[f])
    return (res[best], best) if return_form else res[best]


def candidate_splits(case: RotatingCase):
    return [0, 1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128, 192, 256]


def run(dims, ratios, dtype_name="fp16", sweep=False, rotate_mib=1024, reps=20, csv_path=None, dense=True,
        log=print, warmup=3):
    dtype = DTYPES[dtype_name]
    rows = []
    try:
        torch.backends.cuda.preferred_blas_library("cublaslt")
    except Exception:
        pass
    for n_out, n_in in dims:
        (dense_us, dense_sd), dense_form = (
            time_dense(n_out, n_in, dtype, rotate_mib << 20, reps, warmup=warmup, stats=True, return_form=True)
            if dense else ((float("nan"), float("nan")), ""))
        db = dense_bytes(n_in, n_out, torch.finfo(dtype).bits // 8)
        log(f"--- ({n_out},{n_in}) dense {dense_us:.2f} us ({dense_form}) {db / dense_us / 1e3:.1f} GB/s")
        for nnz, m in ratios:
            case = RotatingCase(n_out, n_in, nnz, m, dtype, rotate_mib << 20)
            plan = _lib.plan(n_out, case.w, nnz, m)
            out = case.launch(0).clone()
            err = dense_reference_check(case, out)
            configs = [(-1, 0)]
            if sweep:
                configs += [(c, s) for c in range(_lib.num_configs()) for s in candidate_splits(case)]
            best = None
            seen = set()
            for cfg, sp in configs:
                p = _lib.plan(n_out, case.w, nnz, m, cfg, sp)
                key = (p["config_id"], p["splits"])
                if key in seen and cfg != -1:
                    continue
                seen.add(key)
                us, sd = time_sparse(case, cfg, sp, reps, warmup, stats=True)
                gbs = case.bytes / us / 1e3
                row = {"n_out": n_out, "n_in": n_in, "ratio": f"{nnz}:{m}", "dtype": dtype_name,
                       "config": p["config"] if cfg >= 0 else f"auto:{plan['config']}", "splits": p["splits"],
                       "blocks": p["blocks"], "rows_per_split": p["rows_per_split"], "us": round(us, 3),
                       "us_sd": round(sd, 3), "GBps": round(gbs, 1), "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                       "dense_us": round(dense_us, 3), "dense_us_sd": round(dense_sd, 3), "dense_form": dense_form,
                       "dense_GBps": round(dense_bytes(n_in, n_out, torch.finfo(dtype).bits // 8) / dense_us / 1e3, 1),
                       "speedup_vs_dense": round(dense_us / us, 3),
                       "copies": case.copies, **{k: float(f"{v:.3e}") for k, v in err.items()}}
                rows.append(row)
                if best is None or us < best["us"]:
                    best = row
            log(f"  {nnz}:{m} auto {rows[-len(seen)]['us']:.2f} us {rows[-len(seen)]['GBps']:.0f} GB/s | best "
                f"{best['config']} s={best['splits']} {best['us']:.2f} us {best['GBps']:.0f} GB/s "
                f"({best['pct_peak']}%) x{best['speedup_vs_dense']} vs dense | max_abs {err['max_abs']:.2e} "
                f"rel_l2 {err['rel_l2']:.2e}")
            del case
            torch.cuda.empty_cache()
    if csv_path:
        Path(csv_path).parent.mkdir(parents=True, exist_ok=True)
        with open(csv_path, "w", newline="") as f:
            wr = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
            wr.writeheader()
            wr.writerows(rows)
    return rows


def read_ceiling(sizes=(4_206_592, 16_795_648, 58_759_168, 268_435_456, 1 << 30), pool_bytes=2 << 30,
                 blocks_list=(64, 128, 256, 512, 1024, 2048, 4096), us_list=(4, 8, 16), reps=10, log=print):
    """Best time of one plain streaming-read launch per byte count: the
    practical HBM ceiling for a bandwidth-bound kernel of that size. Reads
    rotate through a `pool_bytes` buffer so no launch hits the Infinity Cache."""
    import ctypes

    from .build import PROBE_LIB_PATH

    lib = ctypes.CDLL(str(PROBE_LIB_PATH))
    lib.nm_probe_stream_read.restype = ctypes.c_int
    lib.nm_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_void_p]
    buf = torch.randint(0, 255, (pool_bytes,), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(max(blocks_list), dtype=torch.int32, device="cuda")
    out = {}
    for nb in sizes:
        copies = min(256, max(1, pool_bytes // nb))
        best = None
        for blocks in blocks_list:
            for u in us_list:
                def launch(i, blocks=blocks, u=u, nb=nb):
                    rc = lib.nm_probe_stream_read(buf.data_ptr() + i * nb, nb, blocks, u, sink.data_ptr(),
                                                  torch.cuda.current_stream().cuda_stream)
                    if rc != 0:
                        raise RuntimeError(f"nm_probe_stream_read failed: {rc}")
                us = graph_us_per_launch([lambda i=i: launch(i) for i in range(copies)], reps)
                if best is None or us < best[0]:
                    best = (us, blocks, u)
        out[nb] = {"us": round(best[0], 3), "GBps": round(nb / best[0] / 1e3, 1), "blocks": best[1], "u": best[2]}
        log(f"read ceiling {nb / 1e6:9.1f} MB: {best[0]:8.2f} us {nb / best[0] / 1e3:7.0f} GB/s "
            f"(blocks {best[1]}, {best[2]} loads/lane)")
    return out


STRIPE_SHAPES = {  # name: (rows R = w, outputs h) of the fp16 weights one launch streams, 32:64
    "q_o": (2048, 4096), "k_v": (2048, 1024), "gate_up": (2048, 14336), "down": (7168, 4096),
    "gate_up_pair": (2048, 28672),  # gate and up side by side: the pair's bytes
}


def stripe_ceiling(shapes=STRIPE_SHAPES, pool_bytes=2 << 30, reps=10, log=print):
    """Best time of one launch that only reads the weights of a GEMV launch
    in the GEMV's pattern (column stripes of 128 B - 2 KB per row, split over
    rows; roofline_probe.hip: nm_probe_stripe_read), over stripe widths and
    split counts: the ceiling for this access pattern, graph replay, weights
    rotated through `pool_bytes`; also the best with a single split (no
    split-K reduction would be needed)."""
    import ctypes

    from .build import PROBE_LIB_PATH

    lib = ctypes.CDLL(str(PROBE_LIB_PATH))
    lib.nm_probe_stripe_read.restype = ctypes.c_int
    lib.nm_probe_stripe_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_void_p]
    buf = torch.randint(0, 255, (pool_bytes,), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    out = {}
    for name, (R, h) in shapes.items():
        nb = R * h * 2
        C16 = h // 8
        copies = min(256, max(1, pool_bytes // nb))
        best = best1 = None
        for sw in (8, 16, 32, 64, 128):
            for splits in (1, 2, 4, 8, 16, 32):
                if C16 % sw or R % splits or (C16 // sw) * splits > sink.numel():
                    continue

                def launch(i, sw=sw, splits=splits):
                    rc = lib.nm_probe_stripe_read(buf.data_ptr() + i * nb, R, C16, sw, splits, sink.data_ptr(),
                                                  torch.cuda.current_stream().cuda_stream)
                    if rc != 0:
                        raise RuntimeError(f"nm_probe_stripe_read failed: {rc}")
                us = graph_us_per_launch([lambda i=i: launch(i) for i in range(copies)], reps)
                if best is None or us < best[0]:
                    best = (us, sw * 16, splits, (C16 // sw) * splits)
                if splits == 1 and (best1 is None or us < best1[0]):
                    best1 = (us, sw * 16)
        out[name] = {"bytes": nb, "us": round(best[0], 3), "GBps": round(nb / best[0] / 1e3, 1),
                     "stripe_bytes": best[1], "splits": best[2], "workgroups": best[3],
                     "one_split_us": round(best1[0], 3), "one_split_stripe_bytes": best1[1]}
        log(f"stripe ceiling {name:13s} {nb / 1e6:7.1f} MB: {best[0]:7.2f} us {nb / best[0] / 1e3:6.0f} GB/s "
            f"(stripe {best[1]} B, {best[2]} splits, {best[3]} workgroups)")
    return out


def write_stripe_md(res, path, cmd):
    lines = ["# Read ceiling in the GEMV's access pattern (MI355X, fp16 weights of the Llama-3.1-8B shapes, 32:64)", "",
             "Command (repository root, one MI355X):", "", "```", cmd, "```", "",
             "Each row: the fastest launch, over stripe widths (128 B - 2 KB of a row per workgroup; the GEMV's",
             "128- to 1024-row output tiles read 256 B - 2 KB) and split counts (1-32), of a kernel that only reads",
             "the launch's weights in column stripes as the GEMV does (`roofline_probe.hip: nm_probe_stripe_read`,",
             "8 rows per lane in flight), and the fastest with a single split (a GEMV launch of that shape would",
             "need no split-K reduction). Graph replay over >= 1 GiB of rotated copies, inter-kernel gap included,",
             "as for the GEMV classes in bench.py. `gate_up_pair` reads gate and up side by side (the pair",
             "launch's weight bytes).", "",
             "| Launch | Weight bytes | us | GB/s | % of 8 TB/s | stripe | splits | workgroups | one split: us | stripe |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for name, r in res.items():
        lines.append(f"| {name} | {r['bytes']:,} | {r['us']:.2f} | {r['GBps']:.0f} | {r['GBps'] / 80:.1f}% | "
                     f"{r['stripe_bytes']} B | {r['splits']} | {r['workgroups']} | {r['one_split_us']:.2f} | "
                     f"{r['one_split_stripe_bytes']} B |")
    Path(path).write_text("\n".join(lines) + "\n")


def decode_classes(model, ratios, reps=20, warmup=5, rotate_bytes=1 << 30, log=print, classes=None):
    """The decoder's four fused launches (DecodeForms) at one model's shapes,
    per ratio: us per launch (median of graph replays over >= 1 GiB of rotated
    weights per class), algorithmic GB/s and % of the 8 TB/s HBM peak, and the
    sum over one token's launches (layers x 4). With the carried classes in
    `classes`, the token sum of the layer with the split-K carry too."""
    from .decode.model import CONFIGS

    cfg = CONFIGS[model]
    classes = tuple(classes or DECODE_CLASSES)
    res = {}
    for nnz, m in ratios:
        forms = DecodeForms(nnz, m, rotate_bytes=rotate_bytes, dim=cfg.dim, inter=cfg.inter, n_heads=cfg.n_heads,
                            n_kv_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, qk_norm=cfg.qk_norm)
        per = {}
        for c in classes:
            fns = [lambda i=i, c=c: forms.launch(c, i) for i in range(forms.copies[c])]
            us, sd = graph_us_per_launch(fns, reps, warmup, stats=True)
            b = forms.bytes(c)
            per[c] = {"us": round(us, 3), "us_sd": round(sd, 3), "bytes": b, "GBps": round(b / us / 1e3, 1),
                      "pct_peak": round(b / us / 1e3 / 80.0, 1), "copies": forms.copies[c]}
            log(f"{model} {nnz}:{m} {c:26s}: {us:7.2f} +- {sd:.2f} us {per[c]['GBps']:7.1f} GB/s "
                f"({per[c]['pct_peak']}%)")
        r = {"classes": per}
        for tag, group in (("token", DECODE_CLASSES), ("token_carried", CARRIED_CLASSES),
                           ("token_accumulated", ACCUMULATED_CLASSES)):
            if all(c in per for c in group):
                t_us = sum(per[c]["us"] for c in group) * cfg.n_layers
                t_b = sum(per[c]["bytes"] for c in group) * cfg.n_layers
                r[tag] = {"us": round(t_us, 1), "bytes": t_b, "GBps": round(t_b / t_us / 1e3, 1),
                          "pct_peak": round(t_b / t_us / 1e3 / 80.0, 1)}
                log(f"{model} {nnz}:{m}: one token's {4 * cfg.n_layers} sparse launches ({tag}) {t_us:.1f} us, "
                    f"{r[tag]['GBps']} GB/s")
        res[f"{nnz}:{m}"] = r
        del forms
        torch.cuda.empty_cache()
    return res


def write_decode_classes_md(model, res, path, cmd):
    from .decode.model import CONFIGS

    cfg = CONFIGS[model]
    qkv = "q/k/v + input RMSNorm + RoPE + KV-cache write" + (" + q/k head norms" if cfg.qk_norm else "")
    names = {"qkv_decode": qkv, "o_resid": "o + residual", "gate_up_pair_norm": "gate/up pair + RMSNorm + SiLU*mul",
             "down_resid": "down + residual", "qkv_decode_carried": qkv + ", carried input",
             "o_partials": "o, partials left", "gate_up_pair_norm_carried": "gate/up pair + RMSNorm + SiLU*mul, carried input",
             "down_partials": "down, partials left", "qkv_decode_acc": qkv + ", input from an accumulated row",
             "o_acc": "o, adding into an fp32 row", "gate_up_pair_acc": "gate/up pair + RMSNorm, input from o's row, "
                                                                   "adding its sums into an fp32 row",
             "down_silu_acc": "down on the pair's SiLU product, adding into an fp32 row"}
    lines = [f"# Sparse GEMV launches of the fused decoder layer: {cfg.name} shapes (MI355X, fp16, batch 1)", "",
             "Command (repository root, one MI355X):", "", "```", cmd, "```", "",
             f"The decoder's four launches per layer at {cfg.name}'s shapes (dim {cfg.dim}, intermediate "
             f"{cfg.inter}, {cfg.n_heads} query / {cfg.n_kv_heads} KV heads, head_dim {cfg.head_dim}), each",
             "rotating over >= 1 GiB of distinct packed weights in one hipGraph of >= 64 launches (so neither L2 nor",
             "the 256 MB Infinity Cache serves them), the library's default plan; median +- sd over the replays, per",
             "launch, inter-kernel gap included. GB/s counts the algorithmic bytes of the launch (packed weights and index,",
             "activations once, norm weights, residual, outputs, RoPE row); % of the 8 TB/s HBM peak. 'Token' sums",
             f"one decode token's {4 * cfg.n_layers} launches ({cfg.n_layers} layers); 'carried' rows are the layer",
             "with the split-K carry (o and down leave their fp32 partials; gate/up and the next q/k/v finish",
             "them, reading the residual and writing the finished vector; the partials are not counted);",
             "'accumulated' rows are the layer with the accumulated carry (the decoder's default: o, the gate/up",
             "pair and down add into fp32 rows, the next launch finishes them; the rows are not counted).", "",
             "| N:M | Launch | us (median +- sd) | Algorithmic bytes | GB/s | % peak |", "|---|---|---|---|---|---|"]
    for ratio, r in res.items():
        for c, v in r["classes"].items():
            lines.append(f"| {ratio} | {names[c]} | {v['us']:.2f} +- {v['us_sd']:.2f} | {v['bytes']:,} | "
                         f"{v['GBps']:.0f} | {v['pct_peak']:.1f}% |")
        for tag, label in (("token", "token"), ("token_carried", "token, carried"),
                           ("token_accumulated", "token, accumulated carry")):
            if tag in r:
                t = r[tag]
                lines.append(f"| {ratio} | {label} ({4 * cfg.n_layers} launches) | {t['us']:.1f} | {t['bytes']:,} | "
                             f"{t['GBps']:.0f} | {t['pct_peak']:.1f}% |")
    Path(path).write_text("\n".join(lines) + "\n")


def launch_sweep(cls="gate_up_pair_norm", nnz=32, m=64, splits_list=(4, 6, 7, 8, 9, 10, 12, 14, 16), reps=20,
                 warmup=5, log=print, model=None):
    """One of the decoder's fused launches at the Llama-3.1-8B shapes under
    every configuration x split count (weights rotated over >= 1 GiB, graph
    replay): "gate_up_pair_norm" (the pair configurations) or "qkv_decode"
    (the plain configurations, grouped q/k/v with the input RMSNorm, RoPE and
    cache write), or either with "_carried" (its input finished from the
    producer's split partials; plans that cannot carry are skipped). Rows in
    the --sweep CSV layout, the configuration named from the plan (TH from the
    tile count, U from the chunk; `pair_` for the pair), with the kernel's NMAT
    and NORM so that profiling sweep-stats can match them to the traced
    kernels."""
    from .hip_spmv import launch_plan

    carried = cls.endswith("_carried") or cls in ("gate_up_pair_acc", "qkv_decode_acc")
    pair = cls.startswith("gate_up_pair")
    single = {"o_acc": "o", "down_silu_acc": "down"}.get(cls)  # accumulating producers: one matrix
    if cls not in ("gate_up_pair_norm", "qkv_decode", "gate_up_pair_norm_carried", "qkv_decode_carried",
                   "gate_up_pair_acc", "qkv_decode_acc", "o_acc", "down_silu_acc"):
        raise ValueError(f"launch_sweep: {cls!r} is not a fused decoder launch with its own plan")
    if model:  # another model's shapes (default: Llama-3.1-8B)
        from .decode.model import CONFIGS

        c = CONFIGS[model]
        forms = DecodeForms(nnz, m, dim=c.dim, inter=c.inter, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                            head_dim=c.head_dim, qk_norm=c.qk_norm)
    else:
        forms = DecodeForms(nnz, m)
    if single:
        mats = [getattr(forms, single).mats[0]]
    else:
        mats = ([forms.gate.mats[0], forms.up.mats[0]] if pair
                else [forms.q.mats[0], forms.k.mats[0], forms.v.mats[0]])
    hs = [forms.inter] if pair else [int(md.shape[1]) for md, _ in mats]
    nbytes = forms.bytes(cls)
    n = forms.copies[cls]
    n_cfg = _lib.load().nm_num_gate_up_configs() if pair else _lib.num_configs()
    rows, seen = [], set()
    for cfg in [-1, *range(n_cfg)]:
        for sp in ((0,) if cfg < 0 else splits_list):
            plan = launch_plan(mats, nnz, m, gate_up=pair, config_id=cfg, splits=sp, carried=carried,
                               producer=bool(single))
            key = (plan["config_id"], plan["splits"])
            if cfg >= 0 and key in seen:
                continue
            seen.add(key)
            tiles = plan["blocks"] // plan["splits"]
            th = next(t for t in (16, 32, 64, 128, 256) if sum(-(-h // (8 * t)) for h in hs) == tiles)
            u = plan["chunk_rows"] * th // 256
            cached = not pair and "cached" in _lib.describe(plan["config_id"])
            name = ("auto:" if cfg < 0 else "") + ("pair_" if pair else "") + f"th{th}_u{u}" + ("_cached" if cached
                                                                                           else "")

            def launch(i, cfg=cfg, sp=sp):
                forms.launch(cls, i, config_id=cfg, splits=sp)

            if carried or single:
                try:
                    launch(0)
                except _lib.NmSparseLibraryError:
                    log(f"{cls} {name} s={plan['splits']}: the library rejects this plan for the launch, skipped")
                    continue
            us = graph_us_per_launch([lambda i=i: launch(i) for i in range(n)], reps, warmup)
            rows.append({"config": name, "config_id": plan["config_id"], "n_out": sum(hs),
                         "n_in": forms.inter if single == "down" else forms.dim,
                         "ratio": f"{nnz}:{m}", "splits": plan["splits"], "blocks": plan["blocks"],
                         "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1), "nmat": 2 if pair else 1,
                         "norm": 0 if single else 1})
            log(f"{cls} {name} s={plan['splits']} blocks {plan['blocks']}: {us:.2f} us {nbytes / us / 1e3:.0f} GB/s")
    del forms
    torch.cuda.empty_cache()
    return rows


def traffic_probe(shapes=DEFAULT_DIMS, nnz=32, m=64, log=print):
    """Workload for `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` passes:
    three copies of a 256 MiB buffer (the known-size calibration kernel), then
    three GEMV launches per shape, each on distinct weights, then three grouped
    q/k/v launches and three gate/up pair launches at the Llama-3.1-8B shapes,
    then three of each decoder-layer launch, plain and carried."""
    x = torch.empty(128 << 20, dtype=torch.float16, device="cuda").normal_()
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    for n_out, n_in in shapes:
        case = RotatingCase(n_out, n_in, nnz, m, rotate_bytes=0, min_copies=3, seed=3)
        for i in range(3):
            case.launch(i)
        torch.cuda.synchronize()
        log(f"traffic probe: {n_out}x{n_in} {nnz}:{m} plan {_lib.plan(n_out, case.w, nnz, m)}")
    from .hip_spmv import nmsparse_gate_up_silu, nmsparse_gemv_grouped

    qkv = [RotatingCase(h, 4096, nnz, m, rotate_bytes=0, min_copies=3, seed=10 + i)
           for i, h in enumerate((4096, 1024, 1024))]
    for i in range(3):
        nmsparse_gemv_grouped(qkv[0].x, [c.mats[i] for c in qkv], nnz, m, outs=[c.out for c in qkv])
    torch.cuda.synchronize()
    del qkv
    g, u = (RotatingCase(14336, 4096, nnz, m, rotate_bytes=0, min_copies=3, seed=20 + i) for i in range(2))
    for i in range(3):
        nmsparse_gate_up_silu(g.x, g.mats[i], u.mats[i], nnz, m, out=g.out)
    torch.cuda.synchronize()
    del g, u
    log("traffic probe: grouped q/k/v and gate/up pair done")
    forms = DecodeForms(nnz, m, rotate_bytes=0, min_copies=3)
    for cls in DECODE_CLASSES + CARRIED_CLASSES + ACCUMULATED_CLASSES:
        for i in range(3):
            forms.launch(cls, i)
        torch.cuda.synchronize()
    del forms
    log("traffic probe: decode-form launches (plain, split carry, accumulated carry) done")
    from .hip_spmv import nmsparse_spmm_forward_hip
    from .profiling import SPMM_PROBE_CLASSES

    for key, K, h, rows, kind, _ in SPMM_PROBE_CLASSES:
        case = RotatingCase(h, K, nnz, m, rotate_bytes=0, min_copies=3, seed=30)
        X = torch.randn(rows, K, device="cuda").half()
        out = torch.empty(rows, h, dtype=torch.float16, device="cuda")
        for i in range(3):
            md, mi = case.mats[i]
            nmsparse_spmm_forward_hip(X, md, mi, case.w, h, nnz, m, out=out, matrix_cores=kind == "mc")
        torch.cuda.synchronize()
        del case
        log(f"traffic probe: {key} done")


def write_sweep_md(rows, path, cmd):
    """Markdown table of the library's own plan (`auto:` rows) per (shape, ratio)."""
    lines = ["# N:M sparse GEMV vs dense hipBLASLt per shape and ratio (MI355X, fp16, batch 1)", "",
             "Command (repository root, one MI355X):", "", "```", cmd, "```", "",
             "Each (shape, ratio) rotates over >= 1 GiB of distinct packed weights in one hipGraph of >= 64 launches",
             "(so neither L2 nor the 256 MB Infinity Cache serves them); median and stdev over the timed replays, per launch, including",
             "the graph's inter-kernel gap. GB/s counts the algorithmic bytes 2*w*h + w + 2*K + 2*h (dense:",
             "2*K*h + 2*K + 2*h); % of the 8 TB/s HBM peak. Errors are against the fp32 dense matvec on the",
             "scattered masked weight (the reference microbenchmark's oracle). Dense = hipBLASLt in the faster of",
             "its two problem statements for the shape, x * W^T (`mm`, what nn.Linear issues) or W * x (`mv`).", "",
             "| Shape (K -> h) | N:M | Plan | us (median +- sd) | GB/s | % peak | Dense us | Dense GB/s | Speedup | "
             "max_abs | rel_l2 |", "|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        if not str(r["config"]).startswith("auto:"):
            continue
        lines.append(f"| {r['n_in']} -> {r['n_out']} | {r['ratio']} | {r['config'][5:]} s{r['splits']} | "
                     f"{r['us']:.2f} +- {r['us_sd']:.2f} | {r['GBps']:.0f} | {r['pct_peak']:.1f}% | "
                     f"{r['dense_us']:.2f} +- {r['dense_us_sd']:.2f} ({r.get('dense_form', '')}) | {r['dense_GBps']:.0f} | "
                     f"{r['speedup_vs_dense']:.2f}x | {r['max_abs']:.1e} | {r['rel_l2']:.1e} |")
    Path(path).write_text("\n".join(lines) + "\n")


def _parse_pairs(text, sep):
    return [tuple(int(v) for v in item.split(sep)) for item in text.split(",") if item]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--dims", default=",".join(f"{a}x{b}" for a, b in DEFAULT_DIMS), help="n_out x n_in list")
    p.add_argument("--ratios", default=",".join(f"{a}:{b}" for a, b in DEFAULT_RATIOS))
    p.add_argument("--dtype", default="fp16", choices=sorted(DTYPES))
    p.add_argument("--sweep", action="store_true", help="time every config / split count")
    p.add_argument("--rotate-mib", type=int, default=1024)
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3, help="untimed graph replays before the timed ones")
    p.add_argument("--md", default=None, help="write a markdown summary of the library's choice per (shape, ratio)")
    p.add_argument("--no-dense", action="store_true")
    p.add_argument("--csv", default=None)
    p.add_argument("--json", default=None, help="write the best row per (shape, ratio) as JSON")
    p.add_argument("--read-ceiling", action="store_true", help="measure plain streaming-read launches only")
    p.add_argument("--stripe-ceiling", action="store_true",
                   help="measure launches that only read each Llama shape's weights in the GEMV's pattern")
    p.add_argument("--traffic-probe", action="store_true", help="run the rocprof --pmc calibration workload only")
    p.add_argument("--spmm-compare", action="store_true",
                   help="the matrix-core SpMM beside gather + hipBLASLt at the Llama / Qwen3 shapes, 9-128 rows")
    p.add_argument("--spmm-group", action="store_true",
                   help="grouped against separate matrix-core SpMMs of q/k/v and gate/up, Llama / Qwen3, 9-128 rows")
    p.add_argument("--pair-sweep", action="store_true",
                   help="time the decoder's gate/up pair launch under every pair configuration x split count "
                        "(Llama-3.1-8B shapes, the first --ratios entry); --csv for profiling sweep-stats")
    p.add_argument("--qkv-sweep", action="store_true",
                   help="the same for the decoder's q/k/v launch (norm, RoPE, cache write) and the plain "
                        "configurations")
    p.add_argument("--launch-sweep", default=None, metavar="CLASS",
                   help="the same for one accumulated-carry launch class: gate_up_pair_acc, qkv_decode_acc, o_acc "
                        "or down_silu_acc")
    p.add_argument("--decode-classes", default=None, metavar="MODEL",
                   help="time the fused decoder layer's four launches at MODEL's shapes (llama-3.1-8b, qwen3-14b, "
                        "qwen3-32b) for each --ratios entry")
    p.add_argument("--model", default=None,
                   help="with --pair-sweep / --qkv-sweep: that model's shapes (qwen3-14b, qwen3-32b; default "
                        "llama-3.1-8b)")
    p.add_argument("--carried", action="store_true",
                   help="with --decode-classes: also the four launches of the layer with the split-K carry "
                        "(o and down leave their partials, gate/up and q/k/v finish them); with --pair-sweep / "
                        "--qkv-sweep: sweep the launch with a carried input")
    a = p.parse_args(argv)
    if a.pair_sweep or a.qkv_sweep or a.launch_sweep:
        nnz, m = _parse_pairs(a.ratios, ":")[0]
        cls = a.launch_sweep or (("gate_up_pair_norm" if a.pair_sweep else "qkv_decode")
                                 + ("_carried" if a.carried else ""))
        rows = launch_sweep(cls, nnz, m, reps=a.reps, warmup=a.warmup, log=lambda s: print(s, flush=True),
                            model=a.model)
        if a.csv:
            with open(a.csv, "w", newline="") as f:
                wr = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
                wr.writeheader()
                wr.writerows(rows)
        return 0
    if a.decode_classes:
        res = decode_classes(a.decode_classes, _parse_pairs(a.ratios, ":"), a.reps, a.warmup, a.rotate_mib << 20,
                             log=lambda s: print(s, flush=True),
                             classes=(DECODE_CLASSES + CARRIED_CLASSES + ACCUMULATED_CLASSES if a.carried
                                      else DECODE_CLASSES))
        if a.json:
            Path(a.json).write_text(json.dumps(res, indent=1))
        if a.md:
            write_decode_classes_md(a.decode_classes, res, a.md,
                                    " ".join(["python -u -m spmv_decode_amd.microbench", *(argv or sys.argv[1:])]))
        return 0
    if a.read_ceiling:
        res = read_ceiling(log=lambda s: print(s, flush=True))
        if a.json:
            Path(a.json).write_text(json.dumps({str(k): v for k, v in res.items()}, indent=1))
        return 0
    if a.stripe_ceiling:
        res = stripe_ceiling(log=lambda s: print(s, flush=True))
        if a.json:
            Path(a.json).write_text(json.dumps(res, indent=1))
        if a.md:
            write_stripe_md(res, a.md, "python -u -m spmv_decode_amd.microbench --stripe-ceiling --json <json> --md <md>")
        return 0
    if a.traffic_probe:
        traffic_probe(_parse_pairs(a.dims, "x"), log=lambda s: print(s, flush=True))
        return 0
    if a.spmm_compare:
        res = spmm_compare(reps=a.reps, log=lambda s: print(s, flush=True))
        if a.json:
            Path(a.json).write_text(json.dumps(res, indent=1))
        if a.md:
            write_spmm_compare_md(res, a.md, "python -u -m spmv_decode_amd.microbench --spmm-compare --json <json> --md <md>")
        return 0
    if a.spmm_group:
        res = spmm_group(reps=a.reps, log=lambda s: print(s, flush=True))
        if a.json:
            Path(a.json).write_text(json.dumps(res, indent=1))
        if a.md:
            write_spmm_group_md(res, a.md, "python -u -m spmv_decode_amd.microbench --spmm-group --json <json> --md <md>")
        return 0
    rows = run(_parse_pairs(a.dims, "x"), _parse_pairs(a.ratios, ":"), a.dtype, a.sweep, a.rotate_mib, a.reps,
               a.csv, not a.no_dense, log=lambda s: print(s, flush=True), warmup=a.warmup)
    if a.md:
        write_sweep_md(rows, a.md, " ".join(["python -u -m spmv_decode_amd.microbench", *(argv or sys.argv[1:])]))
    if a.json:
        best = {}
        for r in rows:
            k = f"{r['n_out']}x{r['n_in']}_{r['ratio']}"
            if k not in best or r["us"] < best[k]["us"]:
                best[k] = r
        Path(a.json).write_text(json.dumps(best, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
