"""ctypes binding of libnmsparse_hip.so (the C ABI in include/nmsparse_hip.h).

The library is loaded lazily on first use. If it has not been built, every
entry point raises: there is no CPU or PyTorch fallback for the GEMV.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnmsparse_hip.so"

# Status / dtype constants mirrored from include/nmsparse_hip.h.
NM_TICKET_BYTES = 65536
NM_OK = 0
NM_DTYPE_F16, NM_DTYPE_BF16, NM_DTYPE_F32 = 0, 1, 2
NM_ERR = {
    -1: "NM_ERR_NULL_POINTER",
    -2: "NM_ERR_BAD_SHAPE",
    -3: "NM_ERR_H_NOT_MULTIPLE_128",
    -4: "NM_ERR_W_NOT_MULTIPLE_NNZ",
    -5: "NM_ERR_MISALIGNED",
    -6: "NM_ERR_WORKSPACE",
    -7: "NM_ERR_BAD_CONFIG",
    -8: "NM_ERR_BAD_EPILOGUE",
    -9: "NM_ERR_STATIC_SCRATCH",
}
NM_KIND_GROUPED, NM_KIND_GATE_UP = 0, 1
NM_MAX_BATCH = 8
NM_MC_MAX_BATCH = 128
NM_MC_MAX_GROUP = 4
NM_STATIC_SCRATCH_BYTES = NM_TICKET_BYTES + (16 << 20)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_ip = ctypes.POINTER(ctypes.c_int)
_GEMV_ARGS = [_vp, _i, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]
_ll = ctypes.c_longlong


class NmGemvProblem(ctypes.Structure):
    """struct nm_gemv_problem (include/nmsparse_hip.h)."""

    _fields_ = [("mat_data", _vp), ("mat_index", _vp), ("out", _vp), ("residual", _vp), ("head_norm", _vp),
                ("head_stride", _ll), ("elem_stride", _ll), ("pos_stride", _ll), ("h", _i), ("rope", _i)]


class NmGemvLaunchDesc(ctypes.Structure):
    """struct nm_gemv_launch_desc (include/nmsparse_hip.h)."""

    _fields_ = [("dtype", _i), ("kind", _i), ("nprob", _i), ("vec_stride", _i), ("vec", _vp),
                ("norm_weight", _vp), ("norm_eps", ctypes.c_float), ("head_norm_eps", ctypes.c_float),
                ("head_dim", _i), ("pos_limit", _i), ("pos", _vp), ("rope_table", _vp), ("w", _i), ("nnz", _i),
                ("m", _i), ("config_id", _i), ("splits", _i), ("prob", NmGemvProblem * 4), ("carry_out", _vp),
                ("carry_in", _vp), ("vec_out", _vp), ("carry_splits", _i), ("carry_accumulate", _i),
                ("zero_buf", _vp), ("zero_len", _i), ("silu_in", _vp), ("silu_ssq_n", _i), ("silu_k", _i),
                ("silu_eps", ctypes.c_float)]


_descp = ctypes.POINTER(NmGemvLaunchDesc)

# Every function declared in include/nmsparse_hip.h: name -> (restype, argtypes).
ABI = {
    "nm_gemv_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "nm_gemv_f16": (_i, _GEMV_ARGS),
    "nm_gemv_bf16": (_i, _GEMV_ARGS),
    "nm_gemv_f32": (_i, _GEMV_ARGS),
    "nm_gemv_ex": (_i, [_i, _vp, _i, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "nm_gemv_workspace_bytes_ex": (_sz, [_i, _i, _i, _i, _i, _i]),
    "nm_num_configs": (_i, []),
    "nm_gemv_grouped_workspace_bytes": (_sz, [_i, _ip, _i, _i, _i, _i, _i]),
    "nm_gemv_grouped": (_i, [_i, _vp, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), _ip,
                             _vp, _sz, _i, _i, _i, _i, _i, _vp]),
    "nm_gemv_gate_up_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "nm_gemv_gate_up_silu": (_i, [_i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "nm_num_gate_up_configs": (_i, []),
    "nm_gemv_launch_workspace_bytes": (_sz, [_descp]),
    "nm_gemv_launch": (_i, [_descp, _vp, _sz, _vp]),
    "nm_gemv_launch_static": (_i, [_descp, _vp]),
    "nm_gemv_launch_plan": (_i, [_descp, _ip, _ip, _ip, _ip, _ip]),
    "nm_spmm_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "nm_spmm": (_i, [_i, _vp, _ll, _i, _vp, _vp, _vp, _ll, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "nm_spmm_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _ip, _ip, _ip, _ip]),
    "nm_spmm_mc_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "nm_spmm_mc": (_i, [_i, _vp, _ll, _i, _vp, _vp, _vp, _ll, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "nm_spmm_mc_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _ip, _ip, _ip, _ip]),
    "nm_spmm_mc_silu_mul": (_i, [_i, _vp, _vp, _ll, _i, _vp, _vp, _vp, _ll, _vp, _sz, _i, _i, _i, _i, _i, _i, _vp]),
    "nm_spmm_mc_group_workspace_bytes": (_sz, [_i, _i, _ip, _i, _i, _i, _i, _i]),
    "nm_spmm_mc_group": (_i, [_i, _vp, _ll, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                              ctypes.POINTER(_ll), _ip, _vp, _sz, _i, _i, _i, _i, _i, _vp]),
    "nm_spmm_mc_group_plan": (_i, [_i, _i, _ip, _i, _i, _i, _i, _i, _ip, _ip, _ip, _ip]),
    "nm_gather_columns": (_i, [_i, _vp, _ll, _i, _vp, _i, _i, _i, _vp, _ll, _vp]),
    "nm_config_describe": (_i, [_i, ctypes.c_char_p, _i]),
    "nm_gemv_plan": (_i, [_i, _i, _i, _i, _i, _i, _ip, _ip, _ip, _ip]),
    "nm_strerror": (ctypes.c_char_p, [_i]),
    "nm_abi_version": (_i, []),
    "nm_stream_capture_id": (_i, [_vp, ctypes.POINTER(ctypes.c_ulonglong)]),
}
ABI_VERSION = 12

_lib = None
_lock = threading.Lock()


class NmSparseLibraryError(RuntimeError):
    """The HIP library is missing, stale, or returned an error status."""


def load() -> ctypes.CDLL:
    """Load and type the library (once). Raises NmSparseLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NmSparseLibraryError(
                f"{LIB_PATH} is not built; run `python -m spmv_decode_amd.build` "
                "(or __graft_entry__.build()). There is no fallback path."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in ABI.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.nm_abi_version() != ABI_VERSION:
            raise NmSparseLibraryError(
                f"{LIB_PATH} has ABI version {lib.nm_abi_version()}, expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


def strerror(code: int) -> str:
    s = load().nm_strerror(int(code))
    return s.decode() if s else f"status {code}"


def check(code: int, what: str) -> None:
    if code != NM_OK:
        name = NM_ERR.get(code, "hipError")
        raise NmSparseLibraryError(f"{what} failed: {name} ({code}): {strerror(code)}")


def plan(h: int, w: int, nnz: int, m: int, config_id: int = -1, splits: int = 0) -> dict:
    """Configuration, split count, grid size and rows per split the library uses."""
    cfg, sp, blocks, rows = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = load().nm_gemv_plan(h, w, nnz, m, config_id, splits, ctypes.byref(cfg), ctypes.byref(sp),
                             ctypes.byref(blocks), ctypes.byref(rows))
    check(rc, "nm_gemv_plan")
    return {"config_id": cfg.value, "splits": sp.value, "blocks": blocks.value, "rows_per_split": rows.value,
            "config": describe(cfg.value)}


def spmm_plan(batch: int, h: int, w: int, nnz: int, m: int, config_id: int = -1, splits: int = 0) -> dict:
    """Configuration, split count, grid size and rows per split of an SpMM launch."""
    cfg, sp, blocks, rows = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = load().nm_spmm_plan(batch, h, w, nnz, m, config_id, splits, ctypes.byref(cfg), ctypes.byref(sp),
                             ctypes.byref(blocks), ctypes.byref(rows))
    check(rc, "nm_spmm_plan")
    return {"config_id": cfg.value, "splits": sp.value, "blocks": blocks.value, "rows_per_split": rows.value,
            "config": describe(cfg.value)}


MC_CONFIGS = ("mc_h64", "mc_h128", "mc_h256",  # matrix-core SpMM: output tile columns; weights staged
              "mc_h64_dma", "mc_h128_dma", "mc_h256_dma")  # through registers (0-2) or DMA into LDS (3-5)


def spmm_mc_plan(batch: int, h: int, w: int, nnz: int, m: int, config_id: int = -1, splits: int = 0) -> dict:
    """Configuration, split count, grid size and rows per split of a matrix-core SpMM launch."""
    cfg, sp, blocks, rows = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = load().nm_spmm_mc_plan(batch, h, w, nnz, m, config_id, splits, ctypes.byref(cfg), ctypes.byref(sp),
                                ctypes.byref(blocks), ctypes.byref(rows))
    check(rc, "nm_spmm_mc_plan")
    return {"config_id": cfg.value, "splits": sp.value, "blocks": blocks.value, "rows_per_split": rows.value,
            "config": MC_CONFIGS[cfg.value]}


def spmm_mc_group_plan(batch: int, hs, w: int, nnz: int, m: int, config_id: int = -1, splits: int = 0) -> dict:
    """Configuration, split count, grid size and rows per split of a grouped
    matrix-core SpMM launch (products of output widths hs)."""
    n = len(hs)
    harr = (ctypes.c_int * max(n, 1))(*hs)
    cfg, sp, blocks, rows = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = load().nm_spmm_mc_group_plan(batch, n, harr, w, nnz, m, config_id, splits, ctypes.byref(cfg),
                                      ctypes.byref(sp), ctypes.byref(blocks), ctypes.byref(rows))
    check(rc, "nm_spmm_mc_group_plan")
    return {"config_id": cfg.value, "splits": sp.value, "blocks": blocks.value, "rows_per_split": rows.value,
            "config": MC_CONFIGS[cfg.value]}


def describe(config_id: int) -> str:
    buf = ctypes.create_string_buffer(64)
    check(load().nm_config_describe(config_id, buf, 64), "nm_config_describe")
    return buf.value.decode()


def num_configs() -> int:
    return int(load().nm_num_configs())
