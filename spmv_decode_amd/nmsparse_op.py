"""The `nmsparse::gemv` PyTorch custom op, backed by the gfx950 HIP kernel.

Same schema, argument handling and errors as the reference op
(src/spmv/nmsparse_op.py:77-123) in its shared-mask mode: x is reshaped to
[-1, K] and must have exactly one row (decode), x and mat_data are cast to
fp16 if needed, the result is cast back to x.dtype and reshaped to
[*x.shape[:-1], h]. A fake (meta) implementation lets torch.compile trace it.

`nmsparse::spmm` (no reference counterpart) is the batch > 1 form: any number
of rows, NM_MAX_BATCH per launch of the small-batch SpMM kernel, same casts
and output shape rule as `gemv`.

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

from .hip_spmv import nmsparse_spmm_forward_hip, nmsparse_spmv_forward_hip

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


__all__ = ["gemv", "spmm"]
