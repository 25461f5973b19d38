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
different streams use different workspaces, and no call ever uses another
stream's. During hipGraph capture a call uses the capture stream's own
workspace when a warm-up call on that stream created one large enough (the
reference's benchmarks warm every shape up before capturing,
benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:134-144); replays then share it
with eager calls on the capture stream, so they must be ordered with them.
Otherwise the capture gets a workspace of its own, allocated inside the
capture from the graph's memory pool with its counters cleared by a fill
kernel recorded in the graph (one fill node per replay, as the reference's
per-call `torch.zeros` scratch, triton_spmv.py:285); it is keyed by the HIP
capture id, so two graphs never share one.
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
# Workspaces owned by a capture in progress: (device, capture id) -> tensors from
# the capture's pool (the last one is grown into). Dropped once no capture is
# active: the graph's pool then keeps the memory for its replays, as it does
# for every intermediate tensor of the capture.
_capture_workspaces: dict[tuple[int, int], list[torch.Tensor]] = {}


def capture_id(stream_ptr: int) -> int:
    """Id of the hipGraph capture in progress on `stream_ptr`, 0 when the stream
    is not capturing (nm_stream_capture_id: hipStreamGetCaptureInfo of the HIP
    runtime the library links, so no runtime soname is assumed here)."""
    cid = ctypes.c_ulonglong(0)
    rc = _lib.load().nm_stream_capture_id(ctypes.c_void_p(int(stream_ptr)), ctypes.byref(cid))
    if rc != 0:
        raise _lib.NmSparseLibraryError(f"hipStreamGetCaptureInfo failed with status {rc}")
    return int(cid.value)


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
    """A uint8 workspace of at least `nbytes` for a launch on (device, stream)
    whose arrival counters (its first NM_TICKET_BYTES) are zero.

    Outside capture: the stream's own zero-initialised workspace (grown when
    too small). During capture: the capture stream's own workspace if one
    large enough exists, else one owned by this capture (see the module
    docstring); never another stream's."""
    key = (device.index, int(stream_ptr))
    ws = _workspaces.get(key)
    capturing = torch.cuda.is_current_stream_capturing() if (_capture_workspaces or ws is None
                                                             or ws.numel() < nbytes) else False
    if not capturing and _capture_workspaces:
        _capture_workspaces.clear()  # no capture in progress: the graphs' pools own those now
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if capturing:
        ckey = (device.index, capture_id(stream_ptr))
        owned = _capture_workspaces.setdefault(ckey, [])
        if owned and owned[-1].numel() >= nbytes:
            return owned[-1]
        if not owned:
            warnings.warn(
                "nmsparse: graph capture on a stream without a warmed-up workspace; the capture gets its own, "
                "cleared by a fill node in the graph on every replay. Call the op once eagerly on the capture "
                "stream before capturing to avoid it.",
                RuntimeWarning,
                stacklevel=3,
            )
        cws = torch.empty(max(int(nbytes), _MIN_WORKSPACE), dtype=torch.uint8, device=device)
        cws[:_lib.NM_TICKET_BYTES].zero_()  # a fill kernel, recorded in the graph
        owned.append(cws)  # earlier ones stay referenced: launches recorded before still use them
        return cws
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


def library_route(rows: int, K: int, h: int) -> bool:
    """Whether nmsparse_spmm_forward_hip's automatic choice, for a 16-bit
    product of `rows` (> NM_MAX_BATCH) rows, is the gathered activations times
    mat_data on hipBLASLt rather than the matrix-core SpMM: past
    NM_MC_MAX_BATCH rows, where one GEMM replaces several launches of the
    kernel, and past 64 rows for products of at most 1024 outputs. Measured on
    MI355X at every Llama-3.1-8B and Qwen3 shape: from 9 to 64 rows the
    matrix-core kernel is faster everywhere (1.05-2.5x); from 65 to 128 rows
    (its 128-row tiles) it is 1.3-2.15x faster at the down and o projections,
    level at gate/up (0.89-1.20x), and 8-23% slower at the 1024-output k/v
    products, which stay on the library. K is kept for callers that route by
    shape."""
    del K
    return rows > _lib.NM_MC_MAX_BATCH or (rows > 64 and h <= 1024)


def nmsparse_spmm_forward_hip(x, mat_data, mat_index, w, h, BLOCK_WIDTH, VEC_WIDTH, *, out=None, config_id=-1,
                              splits=0, matrix_cores=None):
    """out[..., r, :] = W_sparse @ x[..., r, :] for every row of x ([..., rows, K]),
    each launch streaming the packed weights once.

    Same layout and limits as nmsparse_spmv_forward_hip; rows may be any
    number >= 1. Returns [..., rows, h] in x.dtype (or writes `out`, a
    contiguous tensor of that shape).

    Two kernels: the small-batch SpMM (NM_MAX_BATCH rows per launch; with
    the same config_id and splits each row equals the batch-1 GEMV of that
    row bit for bit when at most 1024 compressed columns fall in a split, see
    _lib.spmm_plan) and, for fp16 / bf16, the matrix-core SpMM
    (NM_MC_MAX_BATCH rows per launch; fp32 accumulation in the matrix cores'
    own order, see _lib.spmm_mc_plan). matrix_cores=None takes the matrix
    cores for NM_MAX_BATCH < rows <= NM_MC_MAX_BATCH of a 16-bit type when
    config_id and splits are left to the library, and the library route
    instead (library_route) past NM_MC_MAX_BATCH rows: the gathered activations (nm_gather_columns, [rows, w]) times
    mat_data as one hipBLASLt GEMM (torch.matmul: a plain GEMM over half the
    input width); else the small-batch kernel. True / False forces one of the
    two HIP kernels (True needs fp16 or bf16). config_id and splits are those
    of the kernel that runs.
    """
    if not (x.is_cuda and mat_data.is_cuda and mat_index.is_cuda):
        raise ValueError("x, mat_data, and mat_index must be GPU (HIP) tensors")
    if x.dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported x dtype: {x.dtype}")
    if mat_data.dtype != x.dtype:
        raise TypeError("x and mat_data must have same dtype")
    if mat_index.dtype != torch.uint8:
        raise TypeError("mat_index must be uint8")
    if h % 128 != 0:
        raise ValueError("h must be divisible by 128")
    if w % BLOCK_WIDTH != 0:
        raise ValueError(f"w={w} must be divisible by N={BLOCK_WIDTH}")
    if VEC_WIDTH < BLOCK_WIDTH or VEC_WIDTH > 256:
        raise ValueError(f"need N <= M <= 256 (uint8 positions), got N={BLOCK_WIDTH}, M={VEC_WIDTH}")
    K = (w // BLOCK_WIDTH) * VEC_WIDTH
    if x.ndim < 2 or x.shape[-1] != K:
        raise ValueError(f"x must be [..., rows, {K}], got {tuple(x.shape)}")
    if tuple(mat_data.shape) != (w, h) or not mat_data.is_contiguous():
        raise ValueError(f"mat_data must be a contiguous {(w, h)} tensor, got {tuple(mat_data.shape)}")
    if tuple(mat_index.shape) != (w // BLOCK_WIDTH, BLOCK_WIDTH) or not mat_index.is_contiguous():
        raise ValueError(f"mat_index must be a contiguous {(w // BLOCK_WIDTH, BLOCK_WIDTH)} tensor")
    lead = x.shape[:-1]
    x2d = x.reshape(-1, K).contiguous()
    rows = x2d.shape[0]
    if out is None:
        out = torch.empty(*lead, h, dtype=x.dtype, device=x.device)
    elif (out.dtype != x.dtype or tuple(out.shape) != (*lead, h) or not out.is_contiguous()
          or out.device != x.device or out.data_ptr() % 16):
        raise ValueError(f"out must be a contiguous, 16-byte aligned {(*lead, h)} tensor of x.dtype")
    if rows == 0:
        return out
    sixteen = x.dtype in (torch.float16, torch.bfloat16)
    library_gemm = False
    if matrix_cores is None:
        matrix_cores = sixteen and rows > _lib.NM_MAX_BATCH and config_id < 0 and splits <= 0
        library_gemm = matrix_cores and library_route(rows, K, h)
    elif matrix_cores and not sixteen:
        raise TypeError("the matrix-core SpMM takes fp16 or bf16")
    md = _aligned(mat_data)
    lib = _lib.load()
    if library_gemm:
        wp = (w + 7) // 8 * 8
        with torch.cuda.device(x.device):
            xg = torch.empty(rows, wp, dtype=x.dtype, device=x.device)
            rc = lib.nm_gather_columns(_DTYPE_CODE[x.dtype], x2d.data_ptr(), K, rows, mat_index.data_ptr(), w,
                                       BLOCK_WIDTH, VEC_WIDTH, xg.data_ptr(), wp,
                                       torch.cuda.current_stream(x.device).cuda_stream)
            _lib.check(rc, "nm_gather_columns")
            torch.matmul(xg[:, :w], md, out=out.view(rows, h))
        return out
    if matrix_cores:
        per, fn, ws_fn, name = _lib.NM_MC_MAX_BATCH, lib.nm_spmm_mc, lib.nm_spmm_mc_workspace_bytes, "nm_spmm_mc"
    else:
        per, fn, ws_fn, name = _lib.NM_MAX_BATCH, lib.nm_spmm, lib.nm_spmm_workspace_bytes, "nm_spmm"
    need = ws_fn(min(rows, per), h, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits))
    if need == 0:
        raise ValueError("spmm shape outside what libnmsparse_hip supports")
    o2d = out.view(rows, h)
    esize = x.element_size()
    device = x.device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        ws = workspace_for(device, need, stream)
        for r0 in range(0, rows, per):
            b = min(per, rows - r0)
            rc = fn(_DTYPE_CODE[x.dtype], x2d.data_ptr() + r0 * K * esize, K, b, md.data_ptr(), mat_index.data_ptr(),
                    o2d.data_ptr() + r0 * h * esize, h, ws.data_ptr(), ws.numel(), h, w, BLOCK_WIDTH, VEC_WIDTH,
                    int(config_id), int(splits), stream)
            _lib.check(rc, name)
    return out


def nmsparse_spmm_silu_mul_hip(gate, up, mat_data, mat_index, w, h, BLOCK_WIDTH, VEC_WIDTH, *, out=None,
                               config_id=-1, splits=0):
    """W applied to every row of round(silu(gate) * up) (the down projection
    of a SwiGLU MLP; gate and up [..., rows, K] of one 16-bit dtype): from 9 to
    NM_MC_MAX_BATCH rows on the matrix cores with the SiLU product formed at
    the gathered positions inside the activation gather (nm_spmm_mc_silu_mul:
    no separate SiLU and multiply launches, one rounding, like the GEMV
    gate/up pair's epilogue), otherwise the product formed in fp32 with one
    rounding and then nmsparse_spmm_forward_hip. Returns [..., rows, h]."""
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.device != up.device:
        raise ValueError("gate and up must have one shape, dtype and device")
    K = gate.shape[-1]
    rows = gate.numel() // K if K else 0
    explicit = config_id >= 0 or splits > 0
    fused = (gate.dtype in (torch.float16, torch.bfloat16) and gate.is_cuda and _lib.NM_MAX_BATCH < rows
             <= _lib.NM_MC_MAX_BATCH and (explicit or not library_route(rows, K, h)))
    if not fused:
        act = (torch.nn.functional.silu(gate.float()) * up.float()).to(gate.dtype)
        return nmsparse_spmm_forward_hip(act, mat_data, mat_index, w, h, BLOCK_WIDTH, VEC_WIDTH, out=out,
                                         config_id=config_id, splits=splits)
    if not (mat_data.is_cuda and mat_index.is_cuda) or mat_data.device != gate.device:
        raise ValueError("gate, up, mat_data, and mat_index must be GPU (HIP) tensors on one device")
    if mat_data.dtype != gate.dtype:
        raise TypeError("x and mat_data must have same dtype")
    if mat_index.dtype != torch.uint8:
        raise TypeError("mat_index must be uint8")
    if w % BLOCK_WIDTH != 0 or K != (w // BLOCK_WIDTH) * VEC_WIDTH:
        raise ValueError(f"x has {K} columns; w={w}, N={BLOCK_WIDTH}, M={VEC_WIDTH} need {w // BLOCK_WIDTH * VEC_WIDTH}")
    if tuple(mat_data.shape) != (w, h) or not mat_data.is_contiguous():
        raise ValueError(f"mat_data must be a contiguous {(w, h)} tensor, got {tuple(mat_data.shape)}")
    if tuple(mat_index.shape) != (w // BLOCK_WIDTH, BLOCK_WIDTH) or not mat_index.is_contiguous():
        raise ValueError(f"mat_index must be a contiguous {(w // BLOCK_WIDTH, BLOCK_WIDTH)} tensor")
    lead = gate.shape[:-1]
    g2d, u2d = gate.reshape(-1, K).contiguous(), up.reshape(-1, K).contiguous()
    if out is None:
        out = torch.empty(*lead, h, dtype=gate.dtype, device=gate.device)
    elif (out.dtype != gate.dtype or tuple(out.shape) != (*lead, h) or not out.is_contiguous()
          or out.device != gate.device or out.data_ptr() % 16):
        raise ValueError(f"out must be a contiguous, 16-byte aligned {(*lead, h)} tensor of x.dtype")
    md = _aligned(mat_data)
    lib = _lib.load()
    need = lib.nm_spmm_mc_workspace_bytes(rows, h, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits))
    if need == 0:
        raise ValueError("spmm shape outside what libnmsparse_hip supports")
    with torch.cuda.device(gate.device):
        stream = torch.cuda.current_stream(gate.device).cuda_stream
        ws = workspace_for(gate.device, need, stream)
        rc = lib.nm_spmm_mc_silu_mul(_DTYPE_CODE[gate.dtype], g2d.data_ptr(), u2d.data_ptr(), K, rows, md.data_ptr(),
                                     mat_index.data_ptr(), out.data_ptr(), h, ws.data_ptr(), ws.numel(), h, w,
                                     BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits), stream)
        _lib.check(rc, "nm_spmm_mc_silu_mul")
    return out


def nmsparse_spmm_group_hip(x, mats, BLOCK_WIDTH, VEC_WIDTH, *, outs=None, config_id=-1, splits=0):
    """[W_i x[..., r, :] for every row r] for the products mats = [(mat_data,
    mat_index), ...] of one input (sibling Linears: q/k/v, gate/up), each as
    nmsparse_spmm_forward_hip would compute it; returns the list of outputs
    [..., rows, h_i] in x.dtype (or writes `outs`).

    fp16 / bf16 with NM_MAX_BATCH < rows <= NM_MC_MAX_BATCH and up to
    NM_MC_MAX_GROUP products of the same w: one gather launch for every
    product's activations and one matrix-core launch over all their tiles
    (nm_spmm_mc_group; each product's rows equal nm_spmm_mc's with the same
    config_id and splits). Otherwise (fewer or more rows, fp32, more
    products, or with the plan left to the library past 64 rows of products
    of at most 1024 outputs: library_route) each product runs through
    nmsparse_spmm_forward_hip on its own.
    """
    mats = list(mats)
    if not mats:
        return []
    K = x.shape[-1]
    lead = x.shape[:-1]
    rows = x.reshape(-1, K).shape[0]
    w = mats[0][0].shape[0]
    hs = [int(md.shape[1]) for md, _ in mats]
    if outs is None:
        outs = [None] * len(mats)
    elif len(outs) != len(mats):
        raise ValueError(f"{len(outs)} outputs for {len(mats)} products")
    explicit = config_id >= 0 or splits > 0  # a matrix-core plan named by the caller
    grouped = (x.dtype in (torch.float16, torch.bfloat16) and _lib.NM_MAX_BATCH < rows <= _lib.NM_MC_MAX_BATCH
               and (explicit or not library_route(rows, K, max(hs))) and 1 < len(mats) <= _lib.NM_MC_MAX_GROUP
               and all(md.shape[0] == w for md, _ in mats))
    if not grouped:
        return [nmsparse_spmm_forward_hip(x, md, mi, w, h, BLOCK_WIDTH, VEC_WIDTH, out=o, config_id=config_id,
                                          splits=splits)
                for (md, mi), h, o in zip(mats, hs, outs)]
    if not x.is_cuda or any(not (md.is_cuda and mi.is_cuda) for md, mi in mats):
        raise ValueError("x, mat_data, and mat_index must be GPU (HIP) tensors")
    if w % BLOCK_WIDTH != 0 or K != (w // BLOCK_WIDTH) * VEC_WIDTH:
        raise ValueError(f"x has {K} columns; w={w}, N={BLOCK_WIDTH}, M={VEC_WIDTH} need {w // BLOCK_WIDTH * VEC_WIDTH}")
    for (md, mi), h in zip(mats, hs):
        if md.dtype != x.dtype:
            raise TypeError("x and mat_data must have same dtype")
        if mi.dtype != torch.uint8:
            raise TypeError("mat_index must be uint8")
        if md.device != x.device or mi.device != x.device:
            raise ValueError("x, mat_data and mat_index must be on one device")
        if not md.is_contiguous() or tuple(mi.shape) != (w // BLOCK_WIDTH, BLOCK_WIDTH) or not mi.is_contiguous():
            raise ValueError(f"mat_data must be a contiguous [{w}, h] tensor, mat_index a contiguous "
                             f"{(w // BLOCK_WIDTH, BLOCK_WIDTH)} tensor")
    x2d = x.reshape(-1, K).contiguous()
    res = []
    for o, h in zip(outs, hs):
        if o is None:
            o = torch.empty(*lead, h, dtype=x.dtype, device=x.device)
        elif (o.dtype != x.dtype or tuple(o.shape) != (*lead, h) or not o.is_contiguous() or o.device != x.device
              or o.data_ptr() % 16):
            raise ValueError(f"out must be a contiguous, 16-byte aligned {(*lead, h)} tensor of x.dtype")
        res.append(o)
    mds = [_aligned(md) for md, _ in mats]
    n = len(mats)
    per = _lib.NM_MC_MAX_BATCH
    lib = _lib.load()
    harr = (ctypes.c_int * n)(*hs)
    need = lib.nm_spmm_mc_group_workspace_bytes(min(rows, per), n, harr, w, BLOCK_WIDTH, VEC_WIDTH, int(config_id),
                                                int(splits))
    if need == 0:
        raise ValueError("spmm group shape outside what libnmsparse_hip supports")
    esize = x.element_size()
    mds_arr = (ctypes.c_void_p * n)(*[md.data_ptr() for md in mds])
    mis_arr = (ctypes.c_void_p * n)(*[mi.data_ptr() for _, mi in mats])
    ostr = (ctypes.c_longlong * n)(*hs)
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        ws = workspace_for(x.device, need, stream)
        for r0 in range(0, rows, per):
            b = min(per, rows - r0)
            outs_arr = (ctypes.c_void_p * n)(*[o.data_ptr() + r0 * h * esize for o, h in zip(res, hs)])
            rc = lib.nm_spmm_mc_group(_DTYPE_CODE[x.dtype], x2d.data_ptr() + r0 * K * esize, K, b, n, mds_arr,
                                      mis_arr, outs_arr, ostr, harr, ws.data_ptr(), ws.numel(), w, BLOCK_WIDTH,
                                      VEC_WIDTH, int(config_id), int(splits), stream)
            _lib.check(rc, "nm_spmm_mc_group")
    return res


def _check_vector(t, n, like, what):
    """t must be a contiguous [n] or [1, n] tensor of like.dtype on like.device."""
    if t.device != like.device or t.dtype != like.dtype or t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous tensor of {n} elements of {like.dtype} on {like.device}")


class GemvProblem:
    """One GEMV of a fused launch (struct nm_gemv_problem).

    mat_data [w, h] / mat_index [w/N, N] as for nmsparse_spmv_forward_hip;
    `out` receives the result ([1, h], or a heads-layout base with `layout`);
    `residual` ([h]) is added before the rounding and may be `out` itself;
    `head_norm` ([head_dim]) applies a per-head RMSNorm; `rope` rotates each
    (even, odd) row pair of a head by the angle at the launch's position;
    `layout` = (head_stride, elem_stride, pos_stride) in elements writes row r
    to out[(r // head_dim) * head_stride + (r % head_dim) * elem_stride +
    pos * pos_stride].
    """

    __slots__ = ("mat_data", "mat_index", "out", "residual", "head_norm", "rope", "layout")

    def __init__(self, mat_data, mat_index, out=None, *, residual=None, head_norm=None, rope=False, layout=None):
        self.mat_data, self.mat_index, self.out = mat_data, mat_index, out
        self.residual, self.head_norm, self.rope, self.layout = residual, head_norm, bool(rope), layout


def launch_plan(problems, BLOCK_WIDTH, VEC_WIDTH, *, gate_up=False, config_id=-1, splits=0, carried=False,
                producer=False) -> dict:
    """The library's plan for a launch over `problems` ((mat_data, mat_index)
    pairs): configuration, splits, grid, compressed rows per split and rows
    per chunk (the rows a workgroup streams first). `carried`: the plan of a
    launch with a carried input (nmsparse_gemv_launch's carry_in);
    `producer`: of one that leaves its partials (carry_out)."""
    desc = _lib.NmGemvLaunchDesc()
    if carried:
        desc.carry_in = 16  # only its presence is read by the planner
    if producer:
        desc.carry_out = 16
    desc.dtype, desc.kind = _lib.NM_DTYPE_F16, _lib.NM_KIND_GATE_UP if gate_up else _lib.NM_KIND_GROUPED
    desc.nprob = len(problems)
    w = problems[0][0].shape[0]
    desc.w, desc.nnz, desc.m, desc.config_id, desc.splits = w, BLOCK_WIDTH, VEC_WIDTH, int(config_id), int(splits)
    for i, (md, _) in enumerate(problems):
        desc.prob[i].h = int(md.shape[1])
    out = [ctypes.c_int() for _ in range(5)]
    rc = _lib.load().nm_gemv_launch_plan(ctypes.byref(desc), *[ctypes.byref(v) for v in out])
    _lib.check(rc, "nm_gemv_launch_plan")
    keys = ("config_id", "splits", "blocks", "rows_per_split", "chunk_rows")
    return {k: v.value for k, v in zip(keys, out)}


def nmsparse_gemv_launch(vec, problems, BLOCK_WIDTH, VEC_WIDTH, *, gate_up=False, norm=None, head_dim=0,
                         head_eps=1e-6, pos=None, pos_limit=None, rope_table=None, config_id=-1, splits=0,
                         carry_out=None, carry_in=None, vec_out=None, carry_accumulate=False, zero=None,
                         silu_in=None, silu_ssq_n=0, silu_k=0, silu_eps=0.0):
    """One launch of 1-4 GEMVs that share `vec` [1, K] (or the gate/up pair),
    with the fusions of include/nmsparse_hip.h's nm_gemv_launch.

    `norm` = (weight [K], eps) folds an RMSNorm of vec into the gather.
    `gate_up=True` takes exactly two problems (gate, up) and writes
    silu(gate) * up into problems[0].out. Heads fusions need `head_dim`, and
    `pos` (device int64 [1]) plus `rope_table` (fp32 [S, head_dim/2, 2] or
    complex64 [S, head_dim/2]) when used; positions outside [0, pos_limit)
    store nothing (pos_limit defaults to the rope table's length). Returns the
    list of outputs (the pair: one). Outputs left as None are allocated ([1, h]).

    Split-K carry (a decoder chain's residual add moved into the next
    launch): `carry_out` (fp32 [splits, h], splits from `launch_plan`) makes
    this one plain GEMV leave its unreduced split partials there (nothing is
    returned); `carry_in` (fp32 [S, K]: a producer's partials) with `vec_out`
    ([K] of vec.dtype, not vec) makes the launch's input round(sum of the
    partials + vec), written to vec_out; it needs `norm`.

    Accumulated carry (nm_gemv_launch_desc.carry_accumulate; the sums' last
    bits then vary from run to run): with `carry_accumulate=True` a plain
    producer adds its partials into `carry_out` (fp32 [1, h], zero before
    the launch) and the gate/up pair (carried input or not) becomes a
    producer adding its raw gate and up sums into `carry_out` (fp32 [2h + 16]:
    sums, then the input's sums of squares). `silu_in` (fp32 [2K + 16], a
    pair's accumulator; vec may then be None) makes the input of one plain
    GEMV round(silu(s G) * (s U)) with s from the first `silu_ssq_n` sums of
    squares, `silu_k` and `silu_eps`. `zero` (fp32, a multiple of 4
    elements) is cleared by the launch.
    """
    n = len(problems)
    if gate_up and n != 2:
        raise ValueError("the gate/up pair takes exactly two problems")
    if not 1 <= n <= 4:
        raise ValueError("a fused launch takes 1 to 4 problems")
    w = problems[0].mat_data.shape[0]
    if silu_in is not None:
        if vec is not None:
            raise ValueError("a SiLU-product input replaces vec: pass vec=None")
        md0 = problems[0].mat_data
        K = (w // BLOCK_WIDTH) * VEC_WIDTH
        if (silu_in.dtype != torch.float32 or not silu_in.is_contiguous() or silu_in.device != md0.device
                or silu_in.numel() < 2 * K + max(int(silu_ssq_n), 0) or silu_in.data_ptr() % 16):
            raise ValueError(f"silu_in must be a contiguous, 16-byte aligned fp32 tensor of >= 2K + ssq_n "
                             f"({2 * K} + {silu_ssq_n}) elements on the weights' device")
        vec = silu_in.view(md0.dtype)[:K].view(1, K)  # carries K, dtype and device only: desc.vec stays null
    K = vec.shape[-1]
    for pr in problems:
        validate_args(vec, pr.mat_data, pr.mat_index, w, pr.mat_data.shape[1], BLOCK_WIDTH, 128, VEC_WIDTH, 1, K)
    if gate_up and problems[0].mat_data.shape != problems[1].mat_data.shape:
        raise ValueError(f"gate {tuple(problems[0].mat_data.shape)} and up {tuple(problems[1].mat_data.shape)} "
                         "must have the same shape")
    n_out = 0 if carry_out is not None else (1 if gate_up else n)
    desc = _lib.NmGemvLaunchDesc()
    desc.dtype = _DTYPE_CODE[vec.dtype]
    desc.kind = _lib.NM_KIND_GATE_UP if gate_up else _lib.NM_KIND_GROUPED
    desc.nprob = n
    desc.vec_stride = vec.stride(1)
    desc.vec = vec.data_ptr()
    desc.w, desc.nnz, desc.m = w, BLOCK_WIDTH, VEC_WIDTH
    desc.config_id, desc.splits = int(config_id), int(splits)
    keep = []  # tensors whose pointers the descriptor holds
    if norm is not None:
        weight, eps = norm
        _check_vector(weight, K, vec, "norm weight")
        if vec.data_ptr() % 16 or (K * vec.element_size()) % 16:
            raise ValueError("an input RMSNorm needs a 16-byte aligned vec with K * element size a multiple of 16")
        desc.norm_weight, desc.norm_eps = weight.data_ptr(), float(eps)
    heads = any(pr.head_norm is not None or pr.rope or pr.layout is not None for pr in problems[:n_out])
    needs_pos = any(pr.rope or (pr.layout is not None and pr.layout[2] != 0) for pr in problems[:n_out])
    if heads:
        if gate_up:
            raise ValueError("the gate/up pair writes a plain [h] output (no heads fusions)")
        if head_dim <= 0 or head_dim % 64:
            raise ValueError(f"head_dim must be a positive multiple of 64, got {head_dim}")
        desc.head_dim, desc.head_norm_eps = int(head_dim), float(head_eps)
    pos_limit = 0 if pos_limit is None else int(pos_limit)
    if needs_pos:
        if pos is None or pos.dtype != torch.int64 or pos.numel() != 1 or pos.device != vec.device:
            raise ValueError("pos must be a device int64 tensor of one element")
        desc.pos = pos.data_ptr()
    if any(pr.rope for pr in problems[:n_out]):
        if rope_table is None:
            raise ValueError("rope needs rope_table")
        rt = torch.view_as_real(rope_table) if rope_table.is_complex() else rope_table
        if (rt.dtype != torch.float32 or rt.ndim != 3 or rt.shape[1:] != (head_dim // 2, 2) or not rt.is_contiguous()
                or rt.device != vec.device):
            raise ValueError(f"rope_table must be contiguous fp32 [S, {head_dim // 2}, 2] (or complex64) on the device")
        desc.rope_table = rt.data_ptr()
        if not pos_limit:
            pos_limit = rt.shape[0]
        elif pos_limit > rt.shape[0]:
            raise ValueError(f"pos_limit {pos_limit} exceeds the rope table's {rt.shape[0]} positions")
        keep.append(rt)
    if needs_pos and pos_limit <= 0:
        raise ValueError("a position-dependent launch needs pos_limit (or a rope_table)")
    outs = []
    for i, pr in enumerate(problems):
        h = int(pr.mat_data.shape[1])
        P = desc.prob[i]
        md = _aligned(pr.mat_data)
        keep.append(md)
        P.mat_data, P.mat_index, P.h = md.data_ptr(), pr.mat_index.data_ptr(), h
        if i >= n_out:
            continue
        if pr.layout is None:
            out = _prepare_out(pr.out, h, vec)
        else:
            out = pr.out
            hs_, es_, ps_ = (int(v) for v in pr.layout)
            if out is None or out.dtype != vec.dtype or out.device != vec.device or out.data_ptr() % 16:
                raise ValueError("a heads-layout output must be a 16-byte aligned tensor of vec.dtype on vec.device")
            if min(hs_, es_, ps_) < 0:
                raise ValueError("layout strides must be non-negative")
            top = (h // head_dim - 1) * hs_ + (head_dim - 1) * es_ + max(pos_limit - 1, 0) * ps_
            if not out.is_contiguous() or top >= out.numel():
                raise ValueError(f"heads layout {pr.layout} reaches element {top} of a {out.numel()}-element output")
            P.head_stride, P.elem_stride, P.pos_stride = hs_, es_, ps_
        outs.append(out)
        P.out = out.data_ptr()
        if pr.residual is not None:
            _check_vector(pr.residual, h, vec, "residual")
            P.residual = pr.residual.data_ptr()
        if pr.head_norm is not None:
            _check_vector(pr.head_norm, head_dim, vec, "head_norm")
            P.head_norm = pr.head_norm.data_ptr()
        P.rope = int(pr.rope)
    desc.pos_limit = pos_limit
    if carry_out is not None:
        if (carry_out.dtype != torch.float32 or not carry_out.is_contiguous() or carry_out.device != vec.device
                or carry_out.data_ptr() % 16):
            raise ValueError("carry_out must be a contiguous, 16-byte aligned fp32 tensor on vec.device")
        h0 = int(problems[0].mat_data.shape[1])
        if carry_accumulate:
            want = 2 * h0 + 16 if gate_up else h0
            if carry_out.numel() != want:
                raise ValueError(f"an accumulating producer adds into {want} floats, carry_out holds "
                                 f"{carry_out.numel()}")
        else:
            if gate_up:
                raise ValueError("the gate/up pair is a producer only with carry_accumulate")
            plan = launch_plan([(pr.mat_data, pr.mat_index) for pr in problems], BLOCK_WIDTH, VEC_WIDTH,
                               gate_up=gate_up, config_id=config_id, splits=splits, producer=True)
            if carry_out.numel() != plan["splits"] * h0:
                raise ValueError(f"carry_out holds {carry_out.numel()} floats, the producer leaves "
                                 f"{plan['splits']} x {h0}")
        desc.carry_out = carry_out.data_ptr()
        desc.carry_accumulate = int(bool(carry_accumulate))
    elif carry_accumulate:
        raise ValueError("carry_accumulate needs carry_out")
    if carry_in is not None:
        if carry_in.dtype != torch.float32 or carry_in.dim() != 2 or carry_in.shape[1] != K \
                or not carry_in.is_contiguous() or carry_in.device != vec.device or carry_in.data_ptr() % 16:
            raise ValueError(f"carry_in must be a contiguous, 16-byte aligned fp32 [splits, {K}] tensor on vec.device")
        if vec_out is None:
            raise ValueError("a carried input needs vec_out")
        _check_vector(vec_out, K, vec, "vec_out")
        if vec_out.data_ptr() % 16:
            raise ValueError("vec_out must be 16-byte aligned")
        desc.carry_in, desc.carry_splits, desc.vec_out = carry_in.data_ptr(), carry_in.shape[0], vec_out.data_ptr()
    elif vec_out is not None:
        raise ValueError("vec_out is the output of a carried input (carry_in)")
    if silu_in is not None:
        desc.vec = None
        desc.silu_in, desc.silu_ssq_n, desc.silu_k = silu_in.data_ptr(), int(silu_ssq_n), int(silu_k)
        desc.silu_eps = float(silu_eps)
    if zero is not None:
        if (zero.dtype != torch.float32 or not zero.is_contiguous() or zero.device != vec.device or zero.numel() % 4
                or zero.data_ptr() % 16 or zero.numel() == 0):
            raise ValueError("zero must be a contiguous, 16-byte aligned fp32 tensor of a multiple of 4 elements")
        desc.zero_buf, desc.zero_len = zero.data_ptr(), zero.numel()
    lib = _lib.load()
    need = lib.nm_gemv_launch_workspace_bytes(ctypes.byref(desc))
    if need == 0:
        raise ValueError("launch shape outside what libnmsparse_hip supports")
    device = vec.device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        ws = workspace_for(device, need, stream)
        rc = lib.nm_gemv_launch(ctypes.byref(desc), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "nm_gemv_launch")
    return outs


def nmsparse_gemv_grouped(vec, problems, BLOCK_WIDTH, VEC_WIDTH, *, outs=None, norm=None, residuals=None,
                          config_id=-1, splits=0):
    """Several N:M GEMVs that read the same `vec` [1, K], in one launch.

    `problems` is a sequence of 1-4 (mat_data [w, h_i], mat_index [w/N, N])
    pairs with the same w; returns a list of [1, h_i] outputs (or writes into
    `outs`). Each output equals what nmsparse_spmv_forward_hip computes for that
    problem with the same configuration. Used for the q/k/v projections of a
    decoder layer (one launch instead of three). `norm` = (weight [K], eps)
    applies an RMSNorm to vec first; `residuals[i]` is added to output i.
    """
    if not 1 <= len(problems) <= 4:
        raise ValueError("nmsparse_gemv_grouped takes 1 to 4 problems")
    outs = [None] * len(problems) if outs is None else list(outs)
    residuals = [None] * len(problems) if residuals is None else list(residuals)
    probs = [GemvProblem(md, mi, o, residual=r) for (md, mi), o, r in zip(problems, outs, residuals)]
    return nmsparse_gemv_launch(vec, probs, BLOCK_WIDTH, VEC_WIDTH, norm=norm, config_id=config_id, splits=splits)


def nmsparse_gate_up_silu(vec, gate, up, BLOCK_WIDTH, VEC_WIDTH, *, out=None, norm=None, residual=None,
                          config_id=-1, splits=0, carry_in=None, vec_out=None):
    """silu(W_gate @ vec) * (W_up @ vec) for two N:M-sparse [w, h] weights in one
    launch; `gate` and `up` are (mat_data, mat_index) pairs. fp32 throughout,
    one rounding to vec.dtype. Returns [1, h]. `norm` = (weight [K], eps)
    applies an RMSNorm to vec first; `residual` ([h]) is added last.
    `carry_in` / `vec_out`: the input is round(sum of a producer's partials +
    vec), written to vec_out (nmsparse_gemv_launch)."""
    (gd, gi), (ud, ui) = gate, up
    probs = [GemvProblem(gd, gi, out, residual=residual), GemvProblem(ud, ui)]
    return nmsparse_gemv_launch(vec, probs, BLOCK_WIDTH, VEC_WIDTH, gate_up=True, norm=norm, config_id=config_id,
                                splits=splits, carry_in=carry_in, vec_out=vec_out)[0]


def carry_splits(mat_data, mat_index, BLOCK_WIDTH, VEC_WIDTH) -> int:
    """Split count of the plain GEMV `mat_data` as a producer: the rows of
    the fp32 [splits, h] partials buffer nmsparse_gemv_partials fills."""
    return launch_plan([(mat_data, mat_index)], BLOCK_WIDTH, VEC_WIDTH, producer=True)["splits"]


def nmsparse_gemv_partials(vec, mat_data, mat_index, BLOCK_WIDTH, VEC_WIDTH, carry):
    """The GEMV W @ vec left unreduced: its fp32 split partials go to `carry`
    [splits, h] (splits = carry_splits(...)), for a following launch that takes
    round(sum of them + residual) as its input (carry_in=carry). The split-K
    reduction and the residual add of a decoder layer's o_proj / down_proj
    move into that launch, so this one ends without a split-K handoff."""
    nmsparse_gemv_launch(vec, [GemvProblem(mat_data, mat_index)], BLOCK_WIDTH, VEC_WIDTH, carry_out=carry)
    return carry


def gate_up_ssq_slots(gate, up, BLOCK_WIDTH, VEC_WIDTH, *, carried: bool, norm: bool = True) -> int:
    """Sums of squares the accumulating gate/up pair leaves after its sums
    (nmsparse_gate_up_accumulate): one per split of its plan with a carried
    input, one without, none without an input norm."""
    if not norm:
        return 0
    if not carried:
        return 1
    return launch_plan([gate, up], BLOCK_WIDTH, VEC_WIDTH, gate_up=True, carried=True)["splits"]


def nmsparse_gemv_accumulate(vec, mat_data, mat_index, BLOCK_WIDTH, VEC_WIDTH, acc, *, zero=None, silu_in=None,
                             silu_ssq_n=0, silu_k=0, silu_eps=0.0):
    """acc [1, h] (fp32, zero beforehand) += W @ vec, each split adding its
    partial tile with fp32 atomics (accumulated carry: the order of the adds,
    hence the sum's last bits, varies from run to run). A following launch
    reads acc as a one-row carry (carry_in=acc). `silu_in` (an accumulating
    gate/up pair's buffer; vec None) makes the input that pair's SiLU
    product; `zero` is cleared by the launch."""
    nmsparse_gemv_launch(vec, [GemvProblem(mat_data, mat_index)], BLOCK_WIDTH, VEC_WIDTH, carry_out=acc,
                         carry_accumulate=True, zero=zero, silu_in=silu_in, silu_ssq_n=silu_ssq_n, silu_k=silu_k,
                         silu_eps=silu_eps)
    return acc


def nmsparse_gate_up_accumulate(vec, gate, up, BLOCK_WIDTH, VEC_WIDTH, acc, *, norm=None, carry_in=None,
                                vec_out=None, zero=None) -> int:
    """The gate/up pair as an accumulating producer: gate's and up's raw sums
    (W_gate x * g, W_up x * g with x the input and g the norm weight) are
    added into acc[0, h) and acc[h, 2h) (fp32 [2h + 16], the sums zero
    beforehand) and the input's sums of squares stored after them; a
    following GEMV applies the norm's scale and silu(gate) * up as it gathers
    its input (nmsparse_gemv_silu). Returns the number of sums of squares
    stored (that GEMV's silu_ssq_n). carry_in / vec_out as for
    nmsparse_gate_up_silu; `zero` is cleared by the launch."""
    (gd, gi), (ud, ui) = gate, up
    nmsparse_gemv_launch(vec, [GemvProblem(gd, gi), GemvProblem(ud, ui)], BLOCK_WIDTH, VEC_WIDTH, gate_up=True,
                         norm=norm, carry_in=carry_in, vec_out=vec_out, carry_out=acc, carry_accumulate=True,
                         zero=zero)
    return gate_up_ssq_slots(gate, up, BLOCK_WIDTH, VEC_WIDTH, carried=carry_in is not None, norm=norm is not None)


def nmsparse_gemv_silu(silu_in, mat_data, mat_index, BLOCK_WIDTH, VEC_WIDTH, *, ssq_n, silu_k, silu_eps, out=None,
                       residual=None, zero=None):
    """W @ x (+ residual) with x = round(silu(s G) * (s U)) gathered from an
    accumulating gate/up pair's buffer silu_in ([2K + 16] fp32: G, U, then
    ssq_n sums of squares; s = rsqrt(sum of them / silu_k + silu_eps), 1 when
    ssq_n is 0): the pair's epilogue done where its output is read. Returns
    [1, h] of the weights' dtype."""
    return nmsparse_gemv_launch(None, [GemvProblem(mat_data, mat_index, out, residual=residual)], BLOCK_WIDTH,
                                VEC_WIDTH, silu_in=silu_in, silu_ssq_n=ssq_n, silu_k=silu_k, silu_eps=silu_eps,
                                zero=zero)[0]


def nmsparse_qkv_decode(vec, q, k, v, BLOCK_WIDTH, VEC_WIDTH, *, q_out, k_cache_t, v_cache=None, v_cache_t=None,
                        pos, rope_table, head_dim, norm=None, q_norm=None, k_norm=None, head_eps=1e-6, config_id=-1,
                        splits=0, carry_in=None, vec_out=None, zero=None):
    """The q/k/v projections of one decode step in one launch.

    q, k, v are (mat_data, mat_index) pairs sharing `vec` [1, K]. Writes the
    rotated queries to `q_out`, either [1, n_heads * head_dim] or a buffer of
    rows [n_heads, D] with D >= head_dim (head h in row h, columns past
    head_dim untouched); the rotated keys into `k_cache_t` [kv_heads, D, S]
    (D >= head_dim; rows past head_dim untouched) at column pos; the values
    either into `v_cache` [kv_heads, S, head_dim] at row pos or into
    `v_cache_t` [kv_heads, head_dim, S] at column pos (exactly one of the two;
    the decoder keeps both caches transposed). `norm` = (weight [K], eps) is
    the layer's input RMSNorm; `q_norm` / `k_norm` ([head_dim]) are Qwen3's
    per-head norms. `carry_in` / `vec_out`: the input is round(sum of a
    producer's partials + vec), written to vec_out (nmsparse_gemv_launch);
    `zero` (fp32) is cleared by the launch.
    """
    kvh, kd, S = k_cache_t.shape
    hd = head_dim
    nh = q[0].shape[1] // hd if q[0].dim() == 2 else 0
    if (v_cache is None) == (v_cache_t is None):
        raise ValueError("pass exactly one of v_cache [kv_heads, S, head_dim] and v_cache_t [kv_heads, head_dim, S]")
    if v_cache is not None:
        vc, want, v_layout = v_cache, (kvh, S, hd), (S * hd, 1, hd)
    else:
        vc, want, v_layout = v_cache_t, (kvh, hd, S), (hd * S, S, 1)
    if kd < hd or tuple(vc.shape) != want:
        raise ValueError(f"k_cache_t {tuple(k_cache_t.shape)} / value cache {tuple(vc.shape)} do not match "
                         f"head_dim {head_dim}")
    if tuple(q_out.shape) == (1, nh * hd):
        q_layout = None
    elif q_out.dim() == 2 and q_out.shape[0] == nh and q_out.shape[1] >= hd and q_out.stride(1) == 1:
        q_layout = (q_out.stride(0), 1, 0)
    else:
        raise ValueError(f"q_out {tuple(q_out.shape)} is neither [1, {nh * hd}] nor [{nh}, >= {hd}]")
    for name, (md, _), rows in (("k", k, kvh * hd), ("v", v, kvh * hd)):
        if md.shape[1] != rows:
            raise ValueError(f"{name} projection has {md.shape[1]} outputs, the cache holds {rows}")
    rt = torch.view_as_real(rope_table) if rope_table.is_complex() else rope_table
    if rt.shape[0] < S:
        raise ValueError(f"rope_table has {rt.shape[0]} positions, the cache {S}")
    probs = [GemvProblem(q[0], q[1], q_out, head_norm=q_norm, rope=True, layout=q_layout),
             GemvProblem(k[0], k[1], k_cache_t, head_norm=k_norm, rope=True, layout=(kd * S, S, 1)),
             GemvProblem(v[0], v[1], vc, layout=v_layout)]
    return nmsparse_gemv_launch(vec, probs, BLOCK_WIDTH, VEC_WIDTH, norm=norm, head_dim=head_dim,
                                head_eps=head_eps, pos=pos, rope_table=rt[:S], config_id=config_id,
                                splits=splits, carry_in=carry_in, vec_out=vec_out, zero=zero)


__all__ = ["nmsparse_spmv_forward_hip", "nmsparse_spmv_forward_triton_ptx", "nmsparse_gemv_grouped",
           "nmsparse_gate_up_silu", "nmsparse_gemv_launch", "nmsparse_qkv_decode", "nmsparse_spmm_forward_hip",
           "nmsparse_gemv_partials", "carry_splits", "GemvProblem", "launch_plan", "validate_args", "workspace_for",
           "nmsparse_gemv_accumulate", "nmsparse_gate_up_accumulate", "nmsparse_gemv_silu", "gate_up_ssq_slots",
           "library_route"]
