"""Flat-import shim: `import nmsparse_op` with this directory on sys.path, as the
reference's benchmarks import src/spmv/nmsparse_op.py (nmsparse_op.py:3)."""
from spmv_decode_amd.nmsparse_op import *  # noqa: F401,F403
from spmv_decode_amd.nmsparse_op import _mode, gemv  # noqa: F401
