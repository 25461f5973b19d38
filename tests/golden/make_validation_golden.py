"""Write the golden fixture for the launch wrapper's argument checks.

Run in the development container only (it needs the reference checkout at
/root/reference, which does not exist on the GPU box):

    python tests/golden/make_validation_golden.py

It imports the reference's own `triton_spmv.py` and calls
`nmsparse_spmv_forward_triton_ptx` (triton_spmv.py:229-318) once per case
below, on CPU tensors that report `is_cuda` as the case says (the wrapper's
first check, triton_spmv.py:245-246, reads only that attribute). The
wrapper's device work is replaced for the duration of the calls: the A100
probe (`_is_a100_sm80`) answers False and both Triton kernels are stubs that
raise a marker, so a call either raises from one of the argument checks
(triton_spmv.py:245-294) or reaches the launch. For each case the fixture
records, as data only, the exception type and message the reference raised
(or that the launch was reached). Nothing from the reference is copied into
the fixture except these outputs.
"""
from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import torch

REF = Path(os.environ.get("NM_REFERENCE_ROOT", "/root/reference"))
OUT = Path(__file__).resolve().parent / "wrapper_validation.json"

# Each case changes one thing of a valid call (fp16, w=128, h=256, N=2, M=4,
# vec [1, 256]); the last ones combine two faults, so the fixture also fixes
# which check comes first.
BASE = dict(is_cuda=[True, True, True], vec_dtype="float16", mat_dtype="float16", index_dtype="uint8",
            vec_shape=[1, 256], mat_shape=[128, 256], index_shape=[64, 2], w=128, h=256, bw=2, threads=128,
            vw=4, minibatch=1, vecnum=256, contiguous=[True, True, True], arch="auto")
CASES = {
    "ok": {},
    "ok_bf16": dict(vec_dtype="bfloat16", mat_dtype="bfloat16"),
    "ok_f32": dict(vec_dtype="float32", mat_dtype="float32"),
    "ok_arch_a100": dict(arch="A100"),
    "ok_arch_sm80": dict(arch="sm80"),
    "ok_arch_generic": dict(arch="generic"),
    "ok_arch_default": dict(arch="default"),
    "vec_not_cuda": dict(is_cuda=[False, True, True]),
    "mat_not_cuda": dict(is_cuda=[True, False, True]),
    "index_not_cuda": dict(is_cuda=[True, True, False]),
    "vec_int32": dict(vec_dtype="int32", mat_dtype="int32"),
    "vec_float64": dict(vec_dtype="float64", mat_dtype="float64"),
    "mat_dtype_differs": dict(mat_dtype="bfloat16"),
    "index_int8": dict(index_dtype="int8"),
    "index_int32": dict(index_dtype="int32"),
    "vec_1d": dict(vec_shape=[256]),
    "vec_two_rows": dict(vec_shape=[2, 256]),
    "minibatch2": dict(vec_shape=[2, 256], minibatch=2),
    "vecnum_differs": dict(vecnum=512),
    "threads_256": dict(threads=256),
    "h_not_128": dict(h=200, mat_shape=[128, 200]),
    "w_not_n": dict(w=127, mat_shape=[127, 256]),
    "mat_shape": dict(mat_shape=[128, 384]),
    "mat_shape_rows": dict(mat_shape=[64, 256]),
    "index_shape": dict(index_shape=[32, 4]),
    "mat_noncontig": dict(contiguous=[True, False, True]),
    "index_noncontig": dict(contiguous=[True, True, False]),
    "vec_noncontig": dict(contiguous=[False, True, True]),
    "arch_h100": dict(arch="h100"),
    "arch_gfx950": dict(arch="gfx950"),
    # two faults: the earlier check decides
    "not_cuda_and_int32": dict(is_cuda=[False, True, True], vec_dtype="int32", mat_dtype="int32"),
    "int32_and_threads": dict(vec_dtype="int32", mat_dtype="int32", threads=256),
    "h_and_w": dict(h=200, mat_shape=[127, 200], w=127),
    "shape_and_noncontig": dict(mat_shape=[128, 384], contiguous=[True, False, True]),
    "noncontig_and_arch": dict(contiguous=[False, True, True], arch="h100"),
}


class _Reached(Exception):
    """The call got past every argument check to the kernel launch."""


class _FakeCuda(torch.Tensor):
    @property
    def is_cuda(self):  # the wrapper's device check reads only this
        return True


class _KernelStub:
    def __getitem__(self, grid):
        def launch(*args, **kwargs):
            raise _Reached()

        return launch


def spec_of(name):
    spec = json.loads(json.dumps(BASE))
    spec.update(CASES[name])
    return spec


def tensors(spec):
    """The three tensors of a spec: CPU tensors of the given dtype and shape,
    made non-contiguous (a strided view) where the spec says so."""
    def dt(n):
        return getattr(torch, n)

    vec = torch.zeros(spec["vec_shape"], dtype=dt(spec["vec_dtype"]))
    md = torch.zeros(spec["mat_shape"], dtype=dt(spec["mat_dtype"]))
    mi = torch.zeros(spec["index_shape"], dtype=dt(spec["index_dtype"]))
    if not spec["contiguous"][0]:
        r, k = spec["vec_shape"]
        vec = torch.zeros(r, 2 * k, dtype=dt(spec["vec_dtype"]))[:, ::2]
    if not spec["contiguous"][1]:
        md = torch.zeros(spec["mat_shape"][::-1], dtype=dt(spec["mat_dtype"])).t()
    if not spec["contiguous"][2]:
        mi = torch.zeros(spec["index_shape"][::-1], dtype=dt(spec["index_dtype"])).t()
    return vec, md, mi


def main():
    sys.path.insert(0, str(REF))
    import triton_spmv as ref  # noqa: E402  (the reference module)

    ref._is_a100_sm80 = lambda device: False
    ref.nmsparse_generic_kernel = _KernelStub()
    ref.nmsparse_a100_sm80_kernel = _KernelStub()
    out = {"torch": torch.__version__, "source": "triton_spmv.py:229-318 (nmsparse_spmv_forward_triton_ptx)",
           "cases": {}}
    for name in CASES:
        spec = spec_of(name)
        ts = [t.as_subclass(_FakeCuda) if cuda else t for t, cuda in zip(tensors(spec), spec["is_cuda"])]
        try:
            ref.nmsparse_spmv_forward_triton_ptx(*ts, spec["w"], spec["h"], spec["bw"], spec["threads"], spec["vw"],
                                                 spec["minibatch"], spec["vecnum"], arch=spec["arch"])
            raise RuntimeError(f"{name}: the stubbed launch returned")
        except _Reached:
            got = {"raises": None, "message": None}
        except (ValueError, TypeError, NotImplementedError) as e:
            got = {"raises": type(e).__name__, "message": str(e)}
        out["cases"][name] = {"spec": spec, **got}
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT} ({len(CASES)} cases)")


if __name__ == "__main__":
    main()
