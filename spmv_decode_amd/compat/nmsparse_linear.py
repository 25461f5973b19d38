"""Flat-import shim: `import nmsparse_linear` with this directory on sys.path, as the
reference's benchmarks import src/spmv/nmsparse_linear.py (nmsparse_linear.py:3)."""
from spmv_decode_amd.nmsparse_linear import *  # noqa: F401,F403
from spmv_decode_amd.nmsparse_linear import DECODE_ONLY, WEIGHT_CPU, _make_sparse  # noqa: F401
