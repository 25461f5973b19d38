"""Reference restatement of the N:M shared-mask GEMV path (CPU, test-only).

TEST INFRASTRUCTURE ONLY — see oracle/__init__.py for who may import this and
which check pins each function. Every function cites the reference lines it
restates (paths relative to the reference checkout).
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np
import torch

_HERE = Path(__file__).resolve().parent


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def to_f64(a) -> np.ndarray:
    """Exact widening of fp16/bf16/fp32 data (torch tensor or numpy) to float64."""
    if isinstance(a, torch.Tensor):
        return a.detach().cpu().to(torch.float64).numpy()
    return np.asarray(a).astype(np.float64)


def _flat_index(mat_index) -> np.ndarray:
    if isinstance(mat_index, torch.Tensor):
        mat_index = mat_index.detach().cpu().numpy()
    return np.asarray(mat_index).reshape(-1).astype(np.int64)


# ---------------------------------------------------------------------------
# GEMV value
# ---------------------------------------------------------------------------
def gather_positions(mat_index, nnz: int, m: int) -> np.ndarray:
    """Global input position of every compressed column c: (c // nnz) * m + mat_index[c].

    mat_index is [w/nnz, nnz] row-major, so its flat element c belongs to
    group c // nnz (triton_spmv.py:82-98 / 176-195: base = group * NNZ,
    vec_base = group * M, x index = vec_base + idx).
    """
    idx = _flat_index(mat_index)
    return (np.arange(idx.size, dtype=np.int64) // nnz) * m + idx


def gather_activations(x, mat_index, nnz: int, m: int) -> np.ndarray:
    """Activations seen by each compressed column, float64 (exact widening).

    Positions at or past len(x) contribute 0 (the library's documented
    behaviour; the reference kernel reads outside vec there).
    """
    xv = to_f64(x).reshape(-1)
    pos = gather_positions(mat_index, nnz, m)
    out = np.zeros(pos.size, dtype=np.float64)
    ok = pos < xv.size
    out[ok] = xv[pos[ok]]
    return out


def gemv_f64(x, mat_data, mat_index, nnz: int, m: int) -> np.ndarray:
    """y[r] = sum_c mat_data[c, r] * x[pos(c)], accumulated in float64.

    The value the reference kernel approximates in fp32 (triton_spmv.py:175-214).
    Products of two fp16/bf16/fp32 values are exact in float64, so this is
    the reference sum up to float64 summation error (~1e-16 relative).
    """
    md = to_f64(mat_data)
    return md.T @ gather_activations(x, mat_index, nnz, m)


def spmm_f64(x, mat_data, mat_index, nnz: int, m: int) -> np.ndarray:
    """Rows of x [B, K] each through gemv_f64: [B, h] in float64 (the batch > 1
    extension; the reference op itself rejects rows != 1,
    src/spmv/nmsparse_op.py:83-86)."""
    xv = to_f64(x).reshape(-1, to_f64(x).shape[-1])
    md = to_f64(mat_data)
    pos = gather_positions(mat_index, nnz, m)
    g = np.zeros((xv.shape[0], pos.size), dtype=np.float64)
    ok = pos < xv.shape[1]
    g[:, ok] = xv[:, pos[ok]]
    return g @ md


def gemv_fp32_dense(x, mat_data, mat_index, nnz: int, m: int) -> torch.Tensor:
    """The reference microbenchmark's own oracle: fp32 dense matvec on the
    scattered masked weight, `torch.mv(weight_sparse.float(), vec.float())`
    (microbench_triton_torchmv.py:383-386), on the CPU."""
    xt = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x))
    xt = xt.detach().cpu().reshape(-1).float()
    md = mat_data if isinstance(mat_data, torch.Tensor) else torch.from_numpy(np.asarray(mat_data))
    dense = scatter(md, mat_index, nnz, m, xt.numel())
    return torch.mv(dense.float(), xt)


def gemv_gather_torch(x, mat_data, mat_index, nnz: int, m: int) -> torch.Tensor:
    """Gather form of the same math on the CPU, `mat_data.float().T @ x.float()[sel]`
    (the CPU-B formulation: no dense materialisation). Used for the timed CPU
    baseline; fp32 accumulation in BLAS order."""
    xt = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x))
    xt = xt.detach().cpu().reshape(-1).float()
    pos = torch.from_numpy(gather_positions(mat_index, nnz, m))
    md = mat_data if isinstance(mat_data, torch.Tensor) else torch.from_numpy(np.asarray(mat_data))
    return torch.mv(md.detach().cpu().float().t(), xt[pos])


# ---------------------------------------------------------------------------
# Decode-layer operations around the GEMV (the fused prologue / epilogues)
# ---------------------------------------------------------------------------
def rms_norm_f64(x, weight, eps: float) -> np.ndarray:
    """RMSNorm in float64 over the last axis: x / sqrt(mean(x^2) + eps) * weight
    (model.py:258-270, RMSNorm._norm and forward; the reference rounds the
    normalised value to the input dtype before the weight, this value does not)."""
    xv = to_f64(x)
    s = 1.0 / np.sqrt(np.mean(xv * xv, axis=-1, keepdims=True) + eps)
    return xv * s * to_f64(weight)


def rope_f64(v, angle_row) -> np.ndarray:
    """Rotary embedding of interleaved (even, odd) pairs of the last axis by
    the angles angle_row [head_dim/2] (radians), float64: (a, b) ->
    (a cos - b sin, b cos + a sin) (model.py:310-322, apply_rotary_emb)."""
    vv = to_f64(v)
    a, b = vv[..., 0::2], vv[..., 1::2]
    c, s = np.cos(angle_row), np.sin(angle_row)
    out = np.empty_like(vv)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = b * c + a * s
    return out


def silu_f64(g) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)) (model.py:255-256, F.silu)."""
    gv = np.asarray(g, dtype=np.float64)
    return gv / (1.0 + np.exp(-gv))


def qkv_decode_f64(x, q, k, v, nnz: int, m: int, *, angle_row, head_dim: int, norm=None, q_norm=None,
                   k_norm=None, eps: float = 1e-6):
    """Queries, keys and values of one decode step in float64 (model.py:186,
    attention_norm(x); model.py:219-231, the projections, apply_rotary_emb and
    the cache update; Qwen3 adds a per-head RMSNorm of q and k before the
    rotation). q/k/v are (mat_data, mat_index); norm = (weight, eps).
    Returns (q [n_heads, hd], k [kv_heads, hd], v [kv_heads, hd])."""
    xin = x
    if norm is not None:
        xin = rms_norm_f64(x, norm[0], norm[1]).reshape(-1)
    outs = []
    for (md, mi), hn in ((q, q_norm), (k, k_norm), (v, None)):
        y = gemv_f64(xin, md, mi, nnz, m).reshape(-1, head_dim)
        if hn is not None:
            y = rms_norm_f64(y, hn, eps)
        outs.append(y)
    return rope_f64(outs[0], angle_row), rope_f64(outs[1], angle_row), outs[2]


# ---------------------------------------------------------------------------
# Packing
# ---------------------------------------------------------------------------
def scatter(mat_data, mat_index, nnz: int, m: int, K: int):
    """Compressed [w, h] -> dense masked [h, K] (microbench_triton_torchmv.py:145-164:
    weight_sparse[:, group*m + local] = mat_data[group*nnz : group*nnz+nnz, :].T).
    A pure copy in the input's dtype; returns the same kind (torch / numpy) it got."""
    pos = gather_positions(mat_index, nnz, m)
    if isinstance(mat_data, torch.Tensor):
        md = mat_data.detach().cpu()
        if pos.size != md.shape[0]:
            raise ValueError("mat_index has the wrong number of entries for mat_data")
        dense = torch.zeros((md.shape[1], K), dtype=md.dtype)
        dense[:, torch.from_numpy(pos)] = md.t()
        return dense
    md = np.asarray(mat_data)
    if pos.size != md.shape[0]:
        raise ValueError("mat_index has the wrong number of entries for mat_data")
    dense = np.zeros((md.shape[1], K), dtype=md.dtype)
    dense[:, pos] = md.T
    return dense


def pack(dense, mat_index, nnz: int, m: int):
    """Dense [h, K] -> compressed [w, h]: the gather inverse of `scatter`
    (mat_data[c, :] = dense[:, pos(c)]). Pure copy; same kind as the input."""
    pos = gather_positions(mat_index, nnz, m)
    if isinstance(dense, torch.Tensor):
        return dense.detach().cpu()[:, torch.from_numpy(pos)].t().contiguous()
    return np.ascontiguousarray(np.asarray(dense)[:, pos].T)


def mask_from_index(mat_index, nnz: int, m: int, K: int) -> np.ndarray:
    """Boolean [K] mask of kept input positions (shared by every output row)."""
    mask = np.zeros(K, dtype=bool)
    mask[gather_positions(mat_index, nnz, m)] = True
    return mask


# ---------------------------------------------------------------------------
# Synthetic packing (bit-exact target)
# ---------------------------------------------------------------------------
def make_sparse(K: int, N: int, M: int, seed: int):
    """Restatement of `_make_sparse(K, N, M, seed, device)` for the shared-mask
    layout (src/spmv/nmsparse_linear.py:14-33, the `_SHARED_MASK` branch).

    Same generator, same calls in the same order, because the result is the
    CPU RNG stream itself: a seeded CPU generator, `randn(w, N)` in fp32
    divided by sqrt(K) then cast to fp16, then per bank one
    `randperm(M)[:nnz]` sorted ascending, as uint8. Returns CPU tensors
    (mat_data [w, N] fp16, mat_index [K/M, M/2] uint8, w, nnz).
    """
    nnz = M // 2
    banks = K // M
    w = banks * nnz
    gen = torch.Generator().manual_seed(seed)
    mat_data = (torch.randn(w, N, generator=gen, dtype=torch.float32) / (K ** 0.5)).to(torch.float16)
    mat_index = torch.empty(banks, nnz, dtype=torch.uint8)
    for b in range(banks):
        mat_index[b] = torch.randperm(M, generator=gen)[:nnz].sort().values.to(torch.uint8)
    return mat_data, mat_index, w, nnz


# ---------------------------------------------------------------------------
# Error metrics
# ---------------------------------------------------------------------------
def error_metrics(ref, out) -> dict:
    """max_abs, mean_abs, rmse and rel_l2 = ||ref - out|| / max(||ref||, 1e-12)
    (microbench_triton_torchmv.py:408-423), computed in float64."""
    r = to_f64(ref).reshape(-1)
    o = to_f64(out).reshape(-1)
    d = np.abs(r - o)
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "mean_abs": float(d.mean()) if d.size else 0.0,
        "rmse": float(math.sqrt(float(np.mean(d * d)))) if d.size else 0.0,
        "rel_l2": float(np.linalg.norm(d) / max(float(np.linalg.norm(r)), 1e-12)),
    }


# ---------------------------------------------------------------------------
# Argument checks of the reference wrapper (pinned by tests/golden/wrapper_validation.json)
# ---------------------------------------------------------------------------
def expected_exception(spec: dict):
    """Exception type the reference raises for a call described by `spec`, or None.

    Restates, in order, triton_spmv.py:245-283 (wrapper) — the op's rows check
    (src/spmv/nmsparse_op.py:83-86) is handled by the caller. `spec` keys:
    is_cuda (3 bools), vec_dtype, mat_dtype, index_dtype, vec_shape,
    mat_shape, index_shape, w, h, bw, threads, vw, minibatch, vecnum,
    contiguous (3 bools), arch.
    """
    if not all(spec["is_cuda"]):
        return ValueError
    if spec["vec_dtype"] not in (torch.float16, torch.bfloat16, torch.float32):
        return TypeError
    if spec["mat_dtype"] != spec["vec_dtype"]:
        return TypeError
    if spec["index_dtype"] != torch.uint8:
        return TypeError
    vs = spec["vec_shape"]
    if len(vs) != 2 or vs[0] != spec["minibatch"]:
        return ValueError
    if spec["minibatch"] != 1:
        return NotImplementedError
    if vs[1] != spec["vecnum"]:
        return ValueError
    if spec["threads"] != 128:
        return NotImplementedError
    if spec["h"] % 128 != 0:
        return ValueError
    if spec["w"] % spec["bw"] != 0:
        return ValueError
    groups = spec["w"] // spec["bw"]
    if tuple(spec["mat_shape"]) != (spec["w"], spec["h"]):
        return ValueError
    if tuple(spec["index_shape"]) != (groups, spec["bw"]):
        return ValueError
    if not all(spec["contiguous"]):
        return ValueError
    arch = spec.get("arch", "auto")
    if arch != "auto" and arch.lower() not in ("a100", "sm80", "generic", "default"):
        return ValueError
    return None


# ---------------------------------------------------------------------------
# The C oracle (oracle/nm_gemv_ref.c)
# ---------------------------------------------------------------------------
_C = None
DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def c_oracle(build: bool = True):
    """ctypes handle of oracle/liboracle_nm.so (built with `make -C oracle`)."""
    global _C
    if _C is not None:
        return _C
    path = _HERE / "liboracle_nm.so"
    if not path.exists() and build:
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    lib = ctypes.CDLL(str(path))
    f = lib.nm_oracle_gemv
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    g = lib.nm_oracle_gemv_f16_fast
    g.restype = ctypes.c_int
    g.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4
    for name, res, arg in (("nm_oracle_f16_to_f32", ctypes.c_float, ctypes.c_uint16),
                           ("nm_oracle_bf16_to_f32", ctypes.c_float, ctypes.c_uint16),
                           ("nm_oracle_f32_to_f16", ctypes.c_uint16, ctypes.c_float),
                           ("nm_oracle_f32_to_bf16", ctypes.c_uint16, ctypes.c_float)):
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = [arg]
    lib.nm_oracle_init_tables.restype = None
    _C = lib
    return lib


def gemv_c(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, nnz: int, m: int,
           vec_stride: int = 1):
    """Run the C oracle on CPU tensors. Returns (out_f32 [h] float32, out [h] input dtype)."""
    lib = c_oracle()
    x = x.detach().cpu().contiguous()
    md = mat_data.detach().cpu().contiguous()
    mi = mat_index.detach().cpu().contiguous()
    w, h = md.shape
    acc = torch.empty(h, dtype=torch.float32)
    out = torch.empty(h, dtype=md.dtype)
    rc = lib.nm_oracle_gemv(DTYPE_CODE[md.dtype], x.data_ptr(), vec_stride, md.data_ptr(), mi.data_ptr(),
                            acc.data_ptr(), out.data_ptr(), h, w, nnz, m)
    if rc != 0:
        raise ValueError("nm_oracle_gemv rejected its arguments")
    return acc, out


def gemv_c_fast_f16(x: torch.Tensor, mat_data: torch.Tensor, mat_index: torch.Tensor, nnz: int, m: int,
                    acc: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """Table-driven fp16 variant of the C oracle (same arithmetic and order); for timing."""
    lib = c_oracle()
    w, h = mat_data.shape
    acc = torch.empty(h, dtype=torch.float32) if acc is None else acc
    out = torch.empty(h, dtype=torch.float16) if out is None else out
    rc = lib.nm_oracle_gemv_f16_fast(x.data_ptr(), mat_data.data_ptr(), mat_index.data_ptr(),
                                     acc.data_ptr(), out.data_ptr(), h, w, nnz, m)
    if rc != 0:
        raise ValueError("nm_oracle_gemv_f16_fast rejected its arguments")
    return acc, out
