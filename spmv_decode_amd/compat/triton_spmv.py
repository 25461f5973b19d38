"""Flat-import shim for callers of the reference's kernel wrapper module
(`from triton_spmv import nmsparse_spmv_forward_triton_ptx`, triton_spmv.py:229).
The function runs the gfx950 HIP kernel; there is no Triton here."""
from spmv_decode_amd.hip_spmv import nmsparse_spmv_forward_hip, nmsparse_spmv_forward_triton_ptx  # noqa: F401
