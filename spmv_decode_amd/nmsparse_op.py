"""The `nmsparse::gemv` PyTorch custom op, backed by the gfx950 HIP kernel.

Same schema, argument handling and errors as the reference op
(src/spmv/nmsparse_op.py:77-123) in its shared-mask mode: x is reshaped to
[-1, K] and must have exactly one row (decode), x and mat_data are cast to
fp16 if needed, the result is cast back to x.dtype and reshaped to
[*x.shape[:-1], h]. A fake (meta) implementation lets torch.compile trace it.

`nmsparse::spmm` (no reference counterpart) is the batch > 1 form: any number
of rows, NM_MAX_BATCH per launch of the small-batch SpMM kernel, same casts
and output shape rule as `gemv`.

The fused decode-layer launches are ops too, so that torch.compile traces a
decode step that uses them without graph breaks (no reference counterpart;
they replace the PyTorch operations around the reference's sparse Linears):
`nmsparse::qkv_decode` (q/k/v with the input RMSNorm, Qwen3's head norms,
RoPE and the KV-cache write; mutates the query buffer and both caches),
`nmsparse::gemv_add_` (out += W x, the residual add inside the GEMV; mutates
out) and `nmsparse::gate_up_silu` (silu(W_gate x) * (W_up x) with the input
RMSNorm folded in). They take fp16/bf16/fp32 inputs as they are (no casts).
The split-K carry between a layer's launches adds `nmsparse::gemv_partials_`
(a GEMV left as fp32 split partials; mutates its carry buffer) and the
`_carried` forms of the q/k/v and gate/up launches, which finish their input
from those partials and the residual stream (mutating vec_out). The
accumulated carry (fp32 atomic adds into one row; sums' last bits vary from
run to run) adds `nmsparse::gemv_accumulate_`, `nmsparse::gate_up_accumulate_`
(the pair as a producer of raw sums), `nmsparse::gemv_silu_accumulate_` and
`nmsparse::gemv_silu_add_` (down_proj taking the pair's SiLU product as it
gathers its input), and the `zero` argument of the q/k/v ops (an accumulator
cleared by the launch).

`nmsparse::gemv_grouped` (one launch for 1-4 gemv calls on the same input),
`nmsparse::gemv_silu_mul` (silu(gemv gate) * gemv up in one launch), both
with an optional input RMSNorm folded in, and `nmsparse::gemv_residual`
(residual + gemv in one launch) are what the torch.compile pass of
compile_pass.py rewrites `gemv` calls into, so that unmodified model code
compiled with torch.compile gets one q/k/v and one gate/up launch per layer,
with the RMSNorm in front of them and the residual adds after o and down
inside the launches (no reference counterpart).

Backend selection keeps the reference's `NM_KERNEL` contract of refusing
unknown values (src/spmv/nmsparse_op.py:20-22). Unset, "hip" and
"triton_ptx" all select the one shared-mask HIP kernel. `_mode` reads
"triton_ptx" under NM_KERNEL=triton_ptx, as the reference module sets it
(src/spmv/nmsparse_op.py:29-32): the reference's benchmarks refuse any other
value (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:95), and in that mode the
shared-mask layout they check for is the one this kernel serves. Otherwise
`_mode` is "hip". "guarded", "fp16" and "fp16_split" name per-row-index CUDA
backends whose sources are absent from the reference; they raise instead of
silently changing layout.
"""
from __future__ import annotations

import os

import torch

from typing import Optional

from .hip_spmv import (GemvProblem, nmsparse_gate_up_accumulate, nmsparse_gate_up_silu, nmsparse_gemv_accumulate,
                       nmsparse_gemv_grouped, nmsparse_gemv_launch, nmsparse_gemv_partials, nmsparse_gemv_silu,
                       nmsparse_qkv_decode, nmsparse_spmm_forward_hip, nmsparse_spmv_forward_hip)

_kernel = os.environ.get("NM_KERNEL", "")
if _kernel not in ("", "hip", "triton_ptx", "guarded", "fp16", "fp16_split"):
    raise ValueError(f"Unknown NM_KERNEL={_kernel!r}; refusing silent fallback")
if _kernel in ("guarded", "fp16", "fp16_split"):
    raise NotImplementedError(
        f"NM_KERNEL={_kernel!r} selects a per-row-index CUDA backend that this MI355X build does not "
        "provide; leave NM_KERNEL unset (or set it to 'hip' / 'triton_ptx') for the shared-mask HIP kernel"
    )
_mode = "triton_ptx" if _kernel == "triton_ptx" else "hip"


@torch.library.custom_op("nmsparse::gemv", mutates_args=())
def gemv(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor,
         w: int, h: int, block_width: int, vec_width: int) -> torch.Tensor:
    """y = W_sparse @ x for one decode row; see module docstring."""
    K = x.shape[-1]
    x2d = x.reshape(-1, K).contiguous()
    if x2d.shape[0] != 1:
        raise RuntimeError(f"nmsparse gemv only supports decode (rows==1), got {tuple(x2d.shape)}")
    xh = x2d if x2d.dtype == torch.float16 else x2d.to(torch.float16)
    md = mat_data if mat_data.dtype == torch.float16 else mat_data.to(torch.float16)
    out = nmsparse_spmv_forward_hip(xh, md, mat_index, int(w), int(h), int(block_width), 128,
                                    int(vec_width), 1, int(K))
    out = out.to(dtype=x.dtype)
    return out.reshape(*x.shape[:-1], int(h))


@gemv.register_fake
def _(x, mat_data, mat_index, w, h, block_width, vec_width):
    return x.new_empty((*x.shape[:-1], int(h)))


@torch.library.custom_op("nmsparse::spmm", mutates_args=())
def spmm(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor,
         w: int, h: int, block_width: int, vec_width: int) -> torch.Tensor:
    """y[..., r, :] = W_sparse @ x[..., r, :] for every row (batch >= 1)."""
    xh = x if x.dtype == torch.float16 else x.to(torch.float16)
    md = mat_data if mat_data.dtype == torch.float16 else mat_data.to(torch.float16)
    out = nmsparse_spmm_forward_hip(xh, md, mat_index, int(w), int(h), int(block_width), int(vec_width))
    return out.to(dtype=x.dtype)


@spmm.register_fake
def _(x, mat_data, mat_index, w, h, block_width, vec_width):
    return x.new_empty((*x.shape[:-1], int(h)))


def _decode_rows(x: torch.Tensor, name: str) -> torch.Tensor:
    """x as one fp16 row [1, K], with gemv's rows check and cast."""
    K = x.shape[-1]
    x2d = x.reshape(-1, K).contiguous()
    if x2d.shape[0] != 1:
        raise RuntimeError(f"nmsparse {name} only supports decode (rows==1), got {tuple(x2d.shape)}")
    return x2d if x2d.dtype == torch.float16 else x2d.to(torch.float16)


def _fp16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float16 else t.to(torch.float16)


def _norm(x16: torch.Tensor, weight: Optional[torch.Tensor], eps: float):
    """The launch's input RMSNorm argument: (weight as x16's dtype, eps), or None."""
    return None if weight is None else (weight.to(x16.dtype).contiguous(), float(eps))


def _normed_input(x: torch.Tensor, weight: Optional[torch.Tensor], name: str) -> torch.Tensor:
    """_decode_rows(x), copied to fresh memory when a folded RMSNorm needs a
    16-byte aligned input and x is a view that starts elsewhere."""
    xh = _decode_rows(x, name)
    return xh.clone() if weight is not None and xh.data_ptr() % 16 else xh


@torch.library.custom_op("nmsparse::gemv_grouped", mutates_args=())
def gemv_grouped(x: torch.Tensor, mat_data: list[torch.Tensor], mat_index: list[torch.Tensor], w: int,
                 h: list[int], block_width: int, vec_width: int, norm_weight: Optional[torch.Tensor],
                 norm_eps: float) -> list[torch.Tensor]:
    """[gemv(x', mat_data[i], mat_index[i], w, h[i], ...) for i] as one launch
    (1-4 problems sharing x, w and N:M; hip_spmv.nmsparse_gemv_grouped), with
    gemv's rows check, casts and output shapes; x' = RMSNorm(x) * norm_weight
    folded into the launch when norm_weight is given, else x. What the
    compile pass (compile_pass.py) puts in place of sibling gemv calls, and of
    gemv calls on an RMSNorm's output."""
    xh = _normed_input(x, norm_weight, "gemv_grouped")
    outs = nmsparse_gemv_grouped(xh, [(_fp16(md), mi) for md, mi in zip(mat_data, mat_index)], int(block_width),
                                 int(vec_width), norm=_norm(xh, norm_weight, norm_eps))
    return [o.to(dtype=x.dtype).reshape(*x.shape[:-1], int(hi)) for o, hi in zip(outs, h)]


@gemv_grouped.register_fake
def _(x, mat_data, mat_index, w, h, block_width, vec_width, norm_weight, norm_eps):
    return [x.new_empty((*x.shape[:-1], int(hi))) for hi in h]


@torch.library.custom_op("nmsparse::gemv_silu_mul", mutates_args=())
def gemv_silu_mul(x: torch.Tensor, gate_data: torch.Tensor, gate_index: torch.Tensor, up_data: torch.Tensor,
                  up_index: torch.Tensor, w: int, h: int, block_width: int, vec_width: int,
                  norm_weight: Optional[torch.Tensor], norm_eps: float) -> torch.Tensor:
    """silu(gemv(x', gate)) * gemv(x', up) as one launch of the gate/up pair
    kernel (fp32 sums, SiLU and product, one rounding to fp16), with gemv's
    rows check, casts and output shape; x' = RMSNorm(x) * norm_weight folded
    into the launch when norm_weight is given. What the compile pass puts in
    place of a SiLU-gated pair of sibling gemv calls."""
    xh = _normed_input(x, norm_weight, "gemv_silu_mul")
    y = nmsparse_gate_up_silu(xh, (_fp16(gate_data), gate_index), (_fp16(up_data), up_index), int(block_width),
                              int(vec_width), norm=_norm(xh, norm_weight, norm_eps))
    return y.to(dtype=x.dtype).reshape(*x.shape[:-1], int(h))


@gemv_silu_mul.register_fake
def _(x, gate_data, gate_index, up_data, up_index, w, h, block_width, vec_width, norm_weight, norm_eps):
    return x.new_empty((*x.shape[:-1], int(h)))


@torch.library.custom_op("nmsparse::gemv_residual", mutates_args=())
def gemv_residual(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, w: int, h: int,
                  block_width: int, vec_width: int, residual: torch.Tensor) -> torch.Tensor:
    """residual + gemv(x, ...) with the add inside the launch (fp32, one
    rounding to fp16), shaped like residual ([..., h], fp16). What the compile
    pass puts in place of a gemv call whose only use is a residual add."""
    xh = _decode_rows(x, "gemv_residual")
    res = residual.reshape(-1).contiguous()
    if res.numel() != int(h) or res.dtype != torch.float16:
        raise RuntimeError(f"gemv_residual: residual must hold {int(h)} fp16 values, got {tuple(residual.shape)} "
                           f"{residual.dtype}")
    out = torch.empty(1, int(h), dtype=torch.float16, device=xh.device)
    nmsparse_gemv_launch(xh, [GemvProblem(_fp16(mat_data), mat_index, out, residual=res)], int(block_width),
                         int(vec_width))
    return out.reshape(residual.shape)


@gemv_residual.register_fake
def _(x, mat_data, mat_index, w, h, block_width, vec_width, residual):
    return residual.new_empty(residual.shape)


@torch.library.custom_op("nmsparse::qkv_decode", mutates_args=("q_out", "k_cache_t", "v_cache_t", "zero"))
def qkv_decode(x: torch.Tensor, q_data: torch.Tensor, q_index: torch.Tensor, k_data: torch.Tensor,
               k_index: torch.Tensor, v_data: torch.Tensor, v_index: torch.Tensor, block_width: int, vec_width: int,
               q_out: torch.Tensor, k_cache_t: torch.Tensor, v_cache_t: torch.Tensor, pos: torch.Tensor,
               rope_table: torch.Tensor, head_dim: int, norm_weight: Optional[torch.Tensor], norm_eps: float,
               q_norm: Optional[torch.Tensor], k_norm: Optional[torch.Tensor], head_eps: float,
               zero: Optional[torch.Tensor]) -> None:
    """hip_spmv.nmsparse_qkv_decode with transposed key and value caches
    ([kv_heads, >= head_dim, S] and [kv_heads, head_dim, S]) and rope_table
    fp32 [S', head_dim / 2, 2] (S' >= S); `zero` (fp32) is cleared by the
    launch (an accumulator of the accumulated carry)."""
    nmsparse_qkv_decode(x.view(1, -1), (q_data, q_index), (k_data, k_index), (v_data, v_index), int(block_width),
                        int(vec_width), q_out=q_out, k_cache_t=k_cache_t, v_cache_t=v_cache_t, pos=pos,
                        rope_table=rope_table, head_dim=int(head_dim),
                        norm=None if norm_weight is None else (norm_weight, float(norm_eps)), q_norm=q_norm,
                        k_norm=k_norm, head_eps=float(head_eps), zero=zero)


@qkv_decode.register_fake
def _(x, q_data, q_index, k_data, k_index, v_data, v_index, block_width, vec_width, q_out, k_cache_t, v_cache_t,
      pos, rope_table, head_dim, norm_weight, norm_eps, q_norm, k_norm, head_eps, zero):
    return None


@torch.library.custom_op("nmsparse::gemv_add_", mutates_args=("out",))
def gemv_add_(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, block_width: int, vec_width: int,
              out: torch.Tensor) -> None:
    """out [1, h] += W_sparse x, added in fp32 inside the launch before the one
    rounding (the residual add of a decoder layer, in place)."""
    nmsparse_gemv_launch(x.view(1, -1), [GemvProblem(mat_data, mat_index, out, residual=out)], int(block_width),
                         int(vec_width))


@gemv_add_.register_fake
def _(x, mat_data, mat_index, block_width, vec_width, out):
    return None


@torch.library.custom_op("nmsparse::gate_up_silu", mutates_args=())
def gate_up_silu(x: torch.Tensor, gate_data: torch.Tensor, gate_index: torch.Tensor, up_data: torch.Tensor,
                 up_index: torch.Tensor, block_width: int, vec_width: int, norm_weight: Optional[torch.Tensor],
                 norm_eps: float) -> torch.Tensor:
    """silu(W_gate x') * (W_up x') -> [1, h], x' = RMSNorm(x) when norm_weight is given."""
    return nmsparse_gate_up_silu(x.view(1, -1), (gate_data, gate_index), (up_data, up_index), int(block_width),
                                 int(vec_width), norm=None if norm_weight is None else (norm_weight, float(norm_eps)))


@gate_up_silu.register_fake
def _(x, gate_data, gate_index, up_data, up_index, block_width, vec_width, norm_weight, norm_eps):
    return x.new_empty((1, gate_data.shape[1]))


@torch.library.custom_op("nmsparse::gemv_partials_", mutates_args=("carry",))
def gemv_partials_(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, block_width: int,
                   vec_width: int, carry: torch.Tensor) -> None:
    """W_sparse x left as fp32 split partials in carry [splits, h], for the
    next launch to finish (hip_spmv.nmsparse_gemv_partials)."""
    nmsparse_gemv_partials(x.view(1, -1), mat_data, mat_index, int(block_width), int(vec_width), carry)


@gemv_partials_.register_fake
def _(x, mat_data, mat_index, block_width, vec_width, carry):
    return None


@torch.library.custom_op("nmsparse::qkv_decode_carried",
                         mutates_args=("q_out", "k_cache_t", "v_cache_t", "vec_out", "zero"))
def qkv_decode_carried(x: torch.Tensor, carry: torch.Tensor, vec_out: torch.Tensor, q_data: torch.Tensor,
                       q_index: torch.Tensor, k_data: torch.Tensor, k_index: torch.Tensor, v_data: torch.Tensor,
                       v_index: torch.Tensor, block_width: int, vec_width: int, q_out: torch.Tensor,
                       k_cache_t: torch.Tensor, v_cache_t: torch.Tensor, pos: torch.Tensor, rope_table: torch.Tensor,
                       head_dim: int, norm_weight: torch.Tensor, norm_eps: float, q_norm: Optional[torch.Tensor],
                       k_norm: Optional[torch.Tensor], head_eps: float, zero: Optional[torch.Tensor]) -> None:
    """qkv_decode on the input round(sum of carry's partials + x), which is
    also written to vec_out (x: the residual stream before the producer);
    carry [S, K] fp32 (S = 1: an accumulated carry)."""
    nmsparse_qkv_decode(x.view(1, -1), (q_data, q_index), (k_data, k_index), (v_data, v_index), int(block_width),
                        int(vec_width), q_out=q_out, k_cache_t=k_cache_t, v_cache_t=v_cache_t, pos=pos,
                        rope_table=rope_table, head_dim=int(head_dim), norm=(norm_weight, float(norm_eps)),
                        q_norm=q_norm, k_norm=k_norm, head_eps=float(head_eps), carry_in=carry,
                        vec_out=vec_out.view(1, -1), zero=zero)


@qkv_decode_carried.register_fake
def _(x, carry, vec_out, q_data, q_index, k_data, k_index, v_data, v_index, block_width, vec_width, q_out, k_cache_t,
      v_cache_t, pos, rope_table, head_dim, norm_weight, norm_eps, q_norm, k_norm, head_eps, zero):
    return None


@torch.library.custom_op("nmsparse::gate_up_silu_carried", mutates_args=("vec_out",))
def gate_up_silu_carried(x: torch.Tensor, carry: torch.Tensor, vec_out: torch.Tensor, gate_data: torch.Tensor,
                         gate_index: torch.Tensor, up_data: torch.Tensor, up_index: torch.Tensor, block_width: int,
                         vec_width: int, norm_weight: torch.Tensor, norm_eps: float) -> torch.Tensor:
    """gate_up_silu on the input round(sum of carry's partials + x), which is
    also written to vec_out."""
    return nmsparse_gate_up_silu(x.view(1, -1), (gate_data, gate_index), (up_data, up_index), int(block_width),
                                 int(vec_width), norm=(norm_weight, float(norm_eps)), carry_in=carry,
                                 vec_out=vec_out.view(1, -1))


@gate_up_silu_carried.register_fake
def _(x, carry, vec_out, gate_data, gate_index, up_data, up_index, block_width, vec_width, norm_weight, norm_eps):
    return x.new_empty((1, gate_data.shape[1]))


@torch.library.custom_op("nmsparse::gemv_accumulate_", mutates_args=("acc", "zero"))
def gemv_accumulate_(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, block_width: int,
                     vec_width: int, acc: torch.Tensor, zero: Optional[torch.Tensor]) -> None:
    """acc [1, h] fp32 += W_sparse x with fp32 atomics (accumulated carry;
    hip_spmv.nmsparse_gemv_accumulate); `zero` is cleared by the launch."""
    nmsparse_gemv_accumulate(x.view(1, -1), mat_data, mat_index, int(block_width), int(vec_width), acc, zero=zero)


@gemv_accumulate_.register_fake
def _(x, mat_data, mat_index, block_width, vec_width, acc, zero):
    return None


@torch.library.custom_op("nmsparse::gate_up_accumulate_", mutates_args=("vec_out", "acc", "zero"))
def gate_up_accumulate_(x: torch.Tensor, carry: Optional[torch.Tensor], vec_out: Optional[torch.Tensor],
                        gate_data: torch.Tensor, gate_index: torch.Tensor, up_data: torch.Tensor,
                        up_index: torch.Tensor, block_width: int, vec_width: int, norm_weight: torch.Tensor,
                        norm_eps: float, acc: torch.Tensor, zero: Optional[torch.Tensor]) -> None:
    """The gate/up pair adding its raw sums and leaving its input's sums of
    squares in acc [2h + 16] fp32 (hip_spmv.nmsparse_gate_up_accumulate), on
    the input round(sum of carry's partials + x) written to vec_out when carry
    is given, else on x."""
    nmsparse_gate_up_accumulate(x.view(1, -1), (gate_data, gate_index), (up_data, up_index), int(block_width),
                                int(vec_width), acc, norm=(norm_weight, float(norm_eps)), carry_in=carry,
                                vec_out=None if vec_out is None else vec_out.view(1, -1), zero=zero)


@gate_up_accumulate_.register_fake
def _(x, carry, vec_out, gate_data, gate_index, up_data, up_index, block_width, vec_width, norm_weight, norm_eps, acc,
      zero):
    return None


@torch.library.custom_op("nmsparse::gemv_silu_accumulate_", mutates_args=("acc", "zero"))
def gemv_silu_accumulate_(silu_in: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, block_width: int,
                          vec_width: int, ssq_n: int, silu_k: int, silu_eps: float, acc: torch.Tensor,
                          zero: Optional[torch.Tensor]) -> None:
    """acc [1, h] fp32 += W_sparse x with fp32 atomics, x the SiLU product of
    an accumulating gate/up pair's buffer silu_in (hip_spmv.nmsparse_gemv_silu)."""
    nmsparse_gemv_accumulate(None, mat_data, mat_index, int(block_width), int(vec_width), acc, zero=zero,
                             silu_in=silu_in, silu_ssq_n=int(ssq_n), silu_k=int(silu_k), silu_eps=float(silu_eps))


@gemv_silu_accumulate_.register_fake
def _(silu_in, mat_data, mat_index, block_width, vec_width, ssq_n, silu_k, silu_eps, acc, zero):
    return None


@torch.library.custom_op("nmsparse::gemv_silu_add_", mutates_args=("out",))
def gemv_silu_add_(silu_in: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, block_width: int,
                   vec_width: int, ssq_n: int, silu_k: int, silu_eps: float, out: torch.Tensor) -> None:
    """out [1, h] += W_sparse x (one rounding), x the SiLU product of an
    accumulating gate/up pair's buffer silu_in (hip_spmv.nmsparse_gemv_silu)."""
    nmsparse_gemv_silu(silu_in, mat_data, mat_index, int(block_width), int(vec_width), ssq_n=int(ssq_n),
                       silu_k=int(silu_k), silu_eps=float(silu_eps), out=out, residual=out)


@gemv_silu_add_.register_fake
def _(silu_in, mat_data, mat_index, block_width, vec_width, ssq_n, silu_k, silu_eps, out):
    return None


__all__ = ["gemv", "spmm", "gemv_grouped", "gemv_silu_mul", "gemv_residual", "qkv_decode", "gemv_add_", "gate_up_silu", "gemv_partials_",
           "qkv_decode_carried", "gate_up_silu_carried", "gemv_accumulate_", "gate_up_accumulate_",
           "gemv_silu_accumulate_", "gemv_silu_add_"]
