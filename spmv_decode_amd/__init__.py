"""MI355X-native shared-mask N:M sparse GEMV for LLM decode.

Public API (same names as the reference's src/spmv package):
    NmSparseLinear, swap_to_nmsparse        -- module + model surgery
    torch.ops.nmsparse.gemv                 -- the custom op (registered on import)
    nmsparse_spmv_forward_hip               -- launch wrapper (alias nmsparse_spmv_forward_triton_ptx)
"""
from .hip_spmv import nmsparse_spmv_forward_hip, nmsparse_spmv_forward_triton_ptx
from .nmsparse_linear import NmSparseLinear, pack_dense, swap_to_nmsparse

__all__ = [
    "NmSparseLinear",
    "swap_to_nmsparse",
    "pack_dense",
    "nmsparse_spmv_forward_hip",
    "nmsparse_spmv_forward_triton_ptx",
]
