"""Build the HIP library `libnmsparse_hip.so` for gfx950, in-tree.

    python -m spmv_decode_amd.build          # or __graft_entry__.build()

The library is a plain C-ABI shared object (include/nmsparse_hip.h) compiled
by hipcc from spmv_decode_amd/csrc/: nm_gemv.hip (host side and C ABI) and
nm_gemv_inst.hip once per element type (the kernels) and nm_spmm_mc.hip (the
matrix-core SpMM), compiled in parallel and linked; nothing links against torch.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
# (source, extra defines): the host side, then the kernels of each element type.
UNITS = [(CSRC / "nm_gemv.hip", []), *[(CSRC / "nm_gemv_inst.hip", [f"-DNM_INST_DTYPE={dt}"]) for dt in (0, 1, 2)],
         (CSRC / "nm_spmm_mc.hip", [])]
LIB_PATH = PKG / "libnmsparse_hip.so"
# Measurement-only streaming-read kernel used by the microbenchmark.
PROBE_SOURCES = [PKG / "csrc" / "roofline_probe.hip"]
PROBE_LIB_PATH = PKG / "libnm_roofline_probe.so"
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for every HIP build of this project; the
# compiler's host pass warns that it does not know the feature (harmless).
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(sources, out: Path, verbose: bool) -> Path:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{ROOT / 'include'}", "-o", str(tmp), *map(str, sources)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    os.replace(tmp, out)
    return out


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")


def _compile_units(out: Path, verbose: bool) -> Path:
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="nmsparse_build_") as tmpdir:
        objs = [Path(tmpdir) / f"unit{i}.o" for i in range(len(UNITS))]
        cmds = [[hipcc(), *flags, *defs, f"-I{ROOT / 'include'}", "-c", "-o", str(o), str(src)]
                for (src, defs), o in zip(UNITS, objs)]
        with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
            for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        tmp = out.with_suffix(".so.tmp")
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False) -> Path:
    """Compile the GEMV library and the measurement probe (always recompiles)."""
    _compile(PROBE_SOURCES, PROBE_LIB_PATH, verbose)
    return _compile_units(LIB_PATH, verbose)


if __name__ == "__main__":
    print(build_library(verbose=True))
