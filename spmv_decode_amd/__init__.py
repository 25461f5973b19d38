"""MI355X-native shared-mask N:M sparse GEMV for LLM decode.

Public API (same names as the reference's src/spmv package):
    NmSparseLinear, swap_to_nmsparse        -- module + model surgery
    torch.ops.nmsparse.gemv                 -- the custom op (registered on import)
    nmsparse_spmv_forward_hip               -- launch wrapper (alias nmsparse_spmv_forward_triton_ptx)

Importing the package also installs compile_pass's torch.compile pass, which
turns sibling `nmsparse::gemv` calls of a compiled graph into one launch.
"""
from . import compile_pass
from .hip_spmv import nmsparse_spmv_forward_hip, nmsparse_spmv_forward_triton_ptx
from .nmsparse_linear import NmSparseLinear, pack_dense, swap_to_nmsparse

# torch.compile: sibling gemv calls of a compiled model become one launch (compile_pass; NM_COMPILE_GROUPING=0
# leaves compiled graphs as they are)
compile_pass.install()

__all__ = [
    "NmSparseLinear",
    "swap_to_nmsparse",
    "pack_dense",
    "nmsparse_spmv_forward_hip",
    "nmsparse_spmv_forward_triton_ptx",
]
