"""Launch wrapper of the shared-mask N:M sparse GEMV on MI355X.

`nmsparse_spmv_forward_hip` keeps the signature, argument meaning and
exception types of the reference wrapper `nmsparse_spmv_forward_triton_ptx`
(triton_spmv.py:229-318), so it is also exported under that name. Instead of
a Triton launch it calls the C ABI of libnmsparse_hip.so
(include/nmsparse_hip.h): one HIP kernel per call that streams the packed
weights, reduces split-K partials deterministically and writes the result in
the input dtype. The reference's per-call fp32 zero buffer
(triton_spmv.py:285) and cast kernel (triton_spmv.py:318) do not exist here.

Workspace: the kernel needs a small device workspace (arrival counters that
must start at zero, plus fp32 split-K partials). One zero-initialised
workspace is kept per (device, stream) and reused by every call on that
stream; it is grown outside of graph capture only, and retired workspaces are
kept alive so that captured graphs never see their memory reused. Calls on
different streams use different workspaces. During hipGraph capture a call
uses the capture stream's workspace, or any initialised workspace of the
device that is large enough (the graph must then not be replayed concurrently
with eager calls on the stream that owns it); call the op once eagerly on the
device before capturing, as the reference's benchmarks do per shape
(benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:134-144).
"""
from __future__ import annotations

import ctypes
import warnings

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.NM_DTYPE_F16, torch.bfloat16: _lib.NM_DTYPE_BF16, torch.float32: _lib.NM_DTYPE_F32}
_TYPED_ENTRY = {torch.float16: "nm_gemv_f16", torch.bfloat16: "nm_gemv_bf16", torch.float32: "nm_gemv_f32"}
_KNOWN_ARCH = ("auto", "a100", "sm80", "generic", "default", "gfx950")

# Initial workspace: counters plus 16 MiB of partials, enough for every
# Llama-3.1-8B / Qwen3 decode shape; grown on demand outside capture.
_MIN_WORKSPACE = _lib.NM_TICKET_BYTES + (16 << 20)
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []


def validate_args(vec, mat_data, mat_index, w, h, BLOCK_WIDTH, NUM_THREADS, VEC_WIDTH, minibatch, vecNum,
                  arch="auto", require_device=True):
    """The reference wrapper's argument checks, in its order (triton_spmv.py:245-283),
    then its `arch` check (triton_spmv.py:287-294). `require_device=False`
    skips only the first check, so the rest can be exercised on CPU tensors."""
    if require_device and (not vec.is_cuda or not mat_data.is_cuda or not mat_index.is_cuda):
        raise ValueError("vec, mat_data, and mat_index must be GPU (HIP) tensors")
    if vec.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported vec dtype: {vec.dtype}")
    if mat_data.dtype != vec.dtype:
        raise TypeError("vec and mat_data must have same dtype")
    if mat_index.dtype != torch.uint8:
        raise TypeError("mat_index must be uint8")
    if vec.ndim != 2 or vec.shape[0] != minibatch:
        raise ValueError(f"vec must have shape [{minibatch}, {vecNum}]")
    if minibatch != 1:
        raise NotImplementedError("this specialization requires minibatch=1")
    if vec.shape[1] != vecNum:
        raise ValueError(f"vec.shape[1]={vec.shape[1]} != vecNum={vecNum}")
    if NUM_THREADS != 128:
        raise NotImplementedError("this kernel family assumes 128-thread base execution")
    if h % 128 != 0:
        raise ValueError("h must be divisible by 128")
    if w % BLOCK_WIDTH != 0:
        raise ValueError(f"w={w} must be divisible by N={BLOCK_WIDTH}")
    num_groups = w // BLOCK_WIDTH
    if tuple(mat_data.shape) != (w, h):
        raise ValueError(f"mat_data must have shape {(w, h)}, got {tuple(mat_data.shape)}")
    if tuple(mat_index.shape) != (num_groups, BLOCK_WIDTH):
        raise ValueError(f"mat_index must have shape {(num_groups, BLOCK_WIDTH)}, got {tuple(mat_index.shape)}")
    if not mat_data.is_contiguous():
        raise ValueError("mat_data must be contiguous")
    if not mat_index.is_contiguous():
        raise ValueError("mat_index must be contiguous")
    if not vec.is_contiguous():
        raise ValueError("vec must be contiguous")
    if arch != "auto" and str(arch).lower() not in _KNOWN_ARCH:
        raise ValueError(f"unknown arch={arch!r}; use auto, a100/sm80, generic or gfx950")
    # Limits of this implementation (the reference has none of these):
    if VEC_WIDTH < BLOCK_WIDTH or VEC_WIDTH > 256:
        raise ValueError(f"need N <= M <= 256 (uint8 positions), got N={BLOCK_WIDTH}, M={VEC_WIDTH}")
    if num_groups * VEC_WIDTH != vecNum:
        raise ValueError(f"vecNum={vecNum} must equal (w/N)*M={num_groups * VEC_WIDTH}")


def workspace_for(device: torch.device, nbytes: int, stream_ptr: int) -> torch.Tensor:
    """A zero-initialised uint8 workspace of at least `nbytes` for (device, stream)."""
    key = (device.index, int(stream_ptr))
    ws = _workspaces.get(key)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        for (dev, _), cand in _workspaces.items():
            if dev == device.index and cand.numel() >= nbytes:
                return cand
        warnings.warn(
            "nmsparse: no initialised workspace for this device during graph capture; allocating one "
            "inside the graph (an extra fill node). Call the op once eagerly before capturing.",
            RuntimeWarning,
            stacklevel=3,
        )
        return torch.zeros(nbytes, dtype=torch.uint8, device=device)
    if ws is not None:
        _retired.append(ws)
    ws = torch.zeros(max(int(nbytes), _MIN_WORKSPACE), dtype=torch.uint8, device=device)
    _workspaces[key] = ws
    return ws


def nmsparse_spmv_forward_hip(
    vec: torch.Tensor,
    mat_data: torch.Tensor,
    mat_index: torch.Tensor,
    w: int,
    h: int,
    BLOCK_WIDTH: int,
    NUM_THREADS: int,
    VEC_WIDTH: int,
    minibatch: int,
    vecNum: int,
    groups_per_program: int = 1,
    arch: str = "auto",
    *,
    out: torch.Tensor | None = None,
    config_id: int = -1,
    splits: int = 0,
) -> torch.Tensor:
    """Shared-mask N:M sparse GEMV: returns [1, h] in vec.dtype.

    Arguments as in triton_spmv.py:229-242: BLOCK_WIDTH is N (kept per
    group), VEC_WIDTH is M (group size), vecNum is K. `groups_per_program`
    is accepted and ignored (the reference clamps it and never uses it,
    triton_spmv.py:269); every `arch` value selects the gfx950 kernel.
    Keyword-only extras: `out` (a contiguous [1, h] tensor of vec.dtype to
    write into), `config_id` / `splits` (explicit kernel configuration, see
    nm_gemv_ex; -1 / 0 = the library's choice).
    """
    validate_args(vec, mat_data, mat_index, w, h, BLOCK_WIDTH, NUM_THREADS, VEC_WIDTH, minibatch, vecNum, arch)
    lib = _lib.load()
    device = vec.device
    if mat_data.data_ptr() % 16:
        mat_data = mat_data.clone()  # the kernel streams 16-byte words
    if out is None:
        out = torch.empty((1, h), dtype=vec.dtype, device=device)
    elif (out.dtype != vec.dtype or out.numel() != h or not out.is_contiguous() or out.device != device
          or out.data_ptr() % 16):
        raise ValueError("out must be a contiguous, 16-byte aligned tensor of h elements of vec.dtype on vec.device")
    w, h, nnz, m = int(w), int(h), int(BLOCK_WIDTH), int(VEC_WIDTH)
    explicit = config_id >= 0 or splits > 0
    if explicit:
        need = lib.nm_gemv_workspace_bytes_ex(h, w, nnz, m, int(config_id), int(splits))
    else:
        need = lib.nm_gemv_workspace_bytes(h, w, nnz, m)
    if need == 0:
        raise ValueError(f"shape h={h}, w={w}, N={nnz}, M={m} (config {config_id}, splits {splits}) "
                         "is outside what libnmsparse_hip supports")
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        ws = workspace_for(device, need, stream)
        args = (vec.data_ptr(), vec.stride(1), mat_data.data_ptr(), mat_index.data_ptr(), out.data_ptr(),
                ws.data_ptr(), ws.numel(), h, w, nnz, m)
        if explicit:
            rc = lib.nm_gemv_ex(_DTYPE_CODE[vec.dtype], *args, int(config_id), int(splits), stream)
        else:
            rc = getattr(lib, _TYPED_ENTRY[vec.dtype])(*args, stream)
    _lib.check(rc, _TYPED_ENTRY[vec.dtype])
    return out


# Drop-in name of the reference wrapper (triton_spmv.py:229).
nmsparse_spmv_forward_triton_ptx = nmsparse_spmv_forward_hip


def _prepare_out(out, h, like):
    if out is None:
        return torch.empty((1, h), dtype=like.dtype, device=like.device)
    if (out.dtype != like.dtype or out.numel() != h or not out.is_contiguous() or out.device != like.device
            or out.data_ptr() % 16):
        raise ValueError("out must be a contiguous, 16-byte aligned tensor of h elements of vec.dtype on vec.device")
    return out


def _aligned(md):
    return md if md.data_ptr() % 16 == 0 else md.clone()


def nmsparse_gemv_grouped(vec, problems, BLOCK_WIDTH, VEC_WIDTH, *, outs=None, config_id=-1, splits=0):
    """Several N:M GEMVs that read the same `vec` [1, K], in one launch.

    `problems` is a sequence of 1-4 (mat_data [w, h_i], mat_index [w/N, N])
    pairs with the same w; returns a list of [1, h_i] outputs (or writes into
    `outs`). Each output equals what nmsparse_spmv_forward_hip computes for that
    problem with the same configuration. Used for the q/k/v projections of a
    decoder layer (one launch instead of three).
    """
    if not 1 <= len(problems) <= 4:
        raise ValueError("nmsparse_gemv_grouped takes 1 to 4 problems")
    w = problems[0][0].shape[0]
    K = vec.shape[-1]
    for md, mi in problems:
        validate_args(vec, md, mi, w, md.shape[1], BLOCK_WIDTH, 128, VEC_WIDTH, 1, K)
    hs = [int(md.shape[1]) for md, _ in problems]
    outs = [None] * len(problems) if outs is None else list(outs)
    outs = [_prepare_out(o, h, vec) for o, h in zip(outs, hs)]
    mats = [_aligned(md) for md, _ in problems]
    lib = _lib.load()
    n = len(problems)
    hs_c = (ctypes.c_int * n)(*hs)
    need = lib.nm_gemv_grouped_workspace_bytes(n, hs_c, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits))
    if need == 0:
        raise ValueError("grouped shape outside what libnmsparse_hip supports")
    device = vec.device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        ws = workspace_for(device, need, stream)
        md_c = (ctypes.c_void_p * n)(*[m.data_ptr() for m in mats])
        mi_c = (ctypes.c_void_p * n)(*[mi.data_ptr() for _, mi in problems])
        out_c = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        rc = lib.nm_gemv_grouped(_DTYPE_CODE[vec.dtype], vec.data_ptr(), vec.stride(1), n, md_c, mi_c, out_c, hs_c,
                                 ws.data_ptr(), ws.numel(), w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits),
                                 stream)
    _lib.check(rc, "nm_gemv_grouped")
    return outs


def nmsparse_gate_up_silu(vec, gate, up, BLOCK_WIDTH, VEC_WIDTH, *, out=None, config_id=-1, splits=0):
    """silu(W_gate @ vec) * (W_up @ vec) for two N:M-sparse [w, h] weights in one
    launch; `gate` and `up` are (mat_data, mat_index) pairs. fp32 throughout,
    one rounding to vec.dtype. Returns [1, h]."""
    (gd, gi), (ud, ui) = gate, up
    if gd.shape != ud.shape:
        raise ValueError(f"gate {tuple(gd.shape)} and up {tuple(ud.shape)} must have the same shape")
    w, h = gd.shape
    K = vec.shape[-1]
    validate_args(vec, gd, gi, w, h, BLOCK_WIDTH, 128, VEC_WIDTH, 1, K)
    validate_args(vec, ud, ui, w, h, BLOCK_WIDTH, 128, VEC_WIDTH, 1, K)
    out = _prepare_out(out, h, vec)
    gd, ud = _aligned(gd), _aligned(ud)
    lib = _lib.load()
    need = lib.nm_gemv_gate_up_workspace_bytes(h, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits))
    if need == 0:
        raise ValueError("gate/up shape outside what libnmsparse_hip supports")
    device = vec.device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        ws = workspace_for(device, need, stream)
        rc = lib.nm_gemv_gate_up_silu(_DTYPE_CODE[vec.dtype], vec.data_ptr(), vec.stride(1), gd.data_ptr(),
                                      gi.data_ptr(), ud.data_ptr(), ui.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                      ws.numel(), h, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits), stream)
    _lib.check(rc, "nm_gemv_gate_up_silu")
    return out


__all__ = ["nmsparse_spmv_forward_hip", "nmsparse_spmv_forward_triton_ptx", "nmsparse_gemv_grouped",
           "nmsparse_gate_up_silu", "validate_args", "workspace_for"]
