"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/nmsparse_hip.h declares, and rejects bad arguments before launching.

Every call below that passes placeholder device pointers carries an argument
the library rejects before any HIP call, so no kernel is ever launched.
"""
import ctypes
import re
import subprocess

import pytest

from conftest import ROOT
from spmv_decode_amd import _lib

HEADER = ROOT / "include" / "nmsparse_hip.h"
FAKE = 0x10000  # 256-byte aligned placeholder address, never dereferenced


def _gpu_visible() -> bool:
    import torch

    return torch.cuda.device_count() > 0  # counts devices without initialising HIP


# A descriptor these checks accept goes on to hipLaunchKernelGGL with the
# placeholder pointers: with no GPU that call fails, on a GPU the kernel would
# run on them. The module is for machines without one.
pytestmark = pytest.mark.skipif(_gpu_visible(), reason="placeholder-pointer launches need a machine without a GPU")


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(nm_[a-z0-9_]+)\s*\(", text))


def test_header_declarations_match_binding_table():
    assert _declared_functions() == set(_lib.ABI)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in _declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None
    assert lib.nm_abi_version() == _lib.ABI_VERSION


def test_constants_match_header():
    text = HEADER.read_text()
    assert f"#define NM_TICKET_BYTES {_lib.NM_TICKET_BYTES}" in text
    for code, name in _lib.NM_ERR.items():
        assert re.search(rf"#define {name} \({code}\)", text), name
    assert "#define NM_DTYPE_F16 0" in text and "#define NM_DTYPE_BF16 1" in text and "#define NM_DTYPE_F32 2" in text


def _gemv(fn="nm_gemv_f16", vec=FAKE, stride=1, md=FAKE, mi=FAKE, out=FAKE, ws=FAKE, ws_bytes=1 << 30,
          h=4096, w=2048, nnz=32, m=64):
    return getattr(_lib.load(), fn)(vec, stride, md, mi, out, ws, ws_bytes, h, w, nnz, m, None)


@pytest.mark.parametrize("fn", ["nm_gemv_f16", "nm_gemv_bf16", "nm_gemv_f32"])
def test_rejections_before_launch(fn):
    assert _gemv(fn, vec=None) == -1
    assert _gemv(fn, md=None) == -1
    assert _gemv(fn, mi=None) == -1
    assert _gemv(fn, out=None) == -1
    assert _gemv(fn, ws=None) == -1
    assert _gemv(fn, h=100) == -3
    assert _gemv(fn, h=0) == -2
    assert _gemv(fn, w=2047) == -4
    assert _gemv(fn, nnz=0) == -2
    assert _gemv(fn, nnz=65, m=64) == -2
    assert _gemv(fn, m=257, nnz=2) == -2
    assert _gemv(fn, stride=0) == -2
    assert _gemv(fn, md=FAKE + 2) == -5
    assert _gemv(fn, out=FAKE + 8) == -5
    assert _gemv(fn, ws=FAKE + 16) == -5
    assert _gemv(fn, ws_bytes=1024) == -6


def test_ex_rejects_bad_dtype_and_config():
    lib = _lib.load()
    args = (FAKE, 1, FAKE, FAKE, FAKE, FAKE, 1 << 30, 4096, 2048, 32, 64)
    assert lib.nm_gemv_ex(3, *args, -1, 0, None) == -7
    assert lib.nm_gemv_ex(0, *args, lib.nm_num_configs(), 0, None) == -7
    assert lib.nm_gemv_workspace_bytes_ex(4096, 2048, 32, 64, 999, 0) == 0


def test_workspace_and_plan_invariants():
    lib = _lib.load()
    n = _lib.num_configs()
    assert n >= 1
    shapes = [(3072, 512, 2, 4), (4096, 2048, 32, 64), (1024, 2048, 32, 64), (14336, 2048, 32, 64),
              (4096, 7168, 32, 64), (128, 2, 2, 4), (384, 96, 3, 4), (128256, 2048, 32, 64), (5120, 12800, 8, 16)]
    for h, w, nnz, m in shapes:
        for cfg in [-1, *range(n)]:
            for splits in (0, 1, 3, 1000):
                p = _lib.plan(h, w, nnz, m, cfg, splits)
                th = int(re.match(r"th(\d+)_u(\d+)", p["config"]).group(1))
                u = int(re.match(r"th(\d+)_u(\d+)", p["config"]).group(2))
                chunk = (256 // th) * u
                tiles = -(-h // (8 * th))
                assert p["blocks"] == tiles * p["splits"]
                assert p["rows_per_split"] % chunk == 0 and 0 < p["rows_per_split"] <= 2048
                assert (p["splits"] - 1) * p["rows_per_split"] < w <= p["splits"] * p["rows_per_split"]
                need = lib.nm_gemv_workspace_bytes_ex(h, w, nnz, m, cfg, splits)
                expect = _lib.NM_TICKET_BYTES + (p["splits"] * h * 4 if p["splits"] > 1 else 0)
                assert need == expect
        assert lib.nm_gemv_workspace_bytes(h, w, nnz, m) == lib.nm_gemv_workspace_bytes_ex(h, w, nnz, m, -1, 0)
    assert lib.nm_gemv_workspace_bytes(100, 2048, 32, 64) == 0


def test_strerror_names_every_code():
    for code in [0, *_lib.NM_ERR]:
        assert _lib.strerror(code)
    assert "unknown" in _lib.strerror(-99)


def test_describe_configs():
    names = [_lib.describe(i) for i in range(_lib.num_configs())]
    assert len(set(names)) == len(names)
    buf = ctypes.create_string_buffer(8)
    assert _lib.load().nm_config_describe(-1, buf, 8) == -7


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.NmSparseLibraryError, match="not built"):
        _lib.load()


def test_grouped_and_pair_rejections_before_launch():
    lib = _lib.load()
    n = 3
    hs = (ctypes.c_int * n)(4096, 1024, 1024)
    ptrs = (ctypes.c_void_p * n)(FAKE, FAKE, FAKE)
    common = (1 << 30, 2048, 32, 64, -1, 0, None)
    assert lib.nm_gemv_grouped(0, FAKE, 1, 0, ptrs, ptrs, ptrs, hs, FAKE, *common) == -2
    assert lib.nm_gemv_grouped(0, FAKE, 1, 5, ptrs, ptrs, ptrs, hs, FAKE, *common) == -2
    assert lib.nm_gemv_grouped(0, FAKE, 1, n, None, ptrs, ptrs, hs, FAKE, *common) == -1
    bad_h = (ctypes.c_int * n)(4096, 1000, 1024)
    assert lib.nm_gemv_grouped(0, FAKE, 1, n, ptrs, ptrs, ptrs, bad_h, FAKE, *common) == -3
    mis = (ctypes.c_void_p * n)(FAKE, FAKE + 2, FAKE)
    assert lib.nm_gemv_grouped(0, FAKE, 1, n, mis, ptrs, ptrs, hs, FAKE, *common) == -5
    assert lib.nm_gemv_grouped(0, FAKE, 1, n, ptrs, ptrs, ptrs, hs, FAKE, 1024, 2048, 32, 64, -1, 0, None) == -6
    need = lib.nm_gemv_grouped_workspace_bytes(n, hs, 2048, 32, 64, -1, 0)
    one = sum(lib.nm_gemv_workspace_bytes_ex(h, 2048, 32, 64, 1, 0) - _lib.NM_TICKET_BYTES for h in (4096, 1024, 1024))
    assert need == _lib.NM_TICKET_BYTES + one  # 8 splits each, as alone
    # the gate/up pair
    args = (0, FAKE, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30, 14336, 2048, 32, 64)
    assert lib.nm_gemv_gate_up_silu(*args[:3], None, *args[4:], -1, 0, None) == -1
    assert lib.nm_gemv_gate_up_silu(*args[:5], FAKE + 4, *args[6:], -1, 0, None) == -5
    assert lib.nm_gemv_gate_up_silu(*args, lib.nm_num_gate_up_configs(), 0, None) == -7
    a2 = list(args)
    a2[9] = 4096
    assert lib.nm_gemv_gate_up_silu(*a2, -1, 0, None) == -6
    ws = lib.nm_gemv_gate_up_workspace_bytes(14336, 2048, 32, 64, -1, 0)
    assert ws == _lib.NM_TICKET_BYTES + 2 * 8 * 14336 * 4
    for j in range(lib.nm_num_gate_up_configs()):
        assert _lib.describe(_lib.num_configs() + j).startswith("pair_th")


def test_launch_descriptor_layout_matches_header(tmp_path):
    """ctypes' nm_gemv_problem / nm_gemv_launch_desc agree with the C compiler's
    layout of the header's structs (offset of every field, and sizes)."""
    gcc = subprocess.run(["which", "gcc"], capture_output=True, text=True).stdout.strip()
    if not gcc:
        pytest.skip("gcc not available")
    fields = []
    for sname, cls in (("nm_gemv_problem", _lib.NmGemvProblem), ("nm_gemv_launch_desc", _lib.NmGemvLaunchDesc)):
        fields += [(sname, f[0], getattr(cls, f[0]).offset) for f in cls._fields_]
    src = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "nmsparse_hip.h"', "int main(void) {"]
    for sname, fname, _ in fields:
        lines.append(f'  printf("%zu\\n", offsetof({sname}, {fname}));')
    lines += ['  printf("%zu\\n%zu\\n", sizeof(nm_gemv_problem), sizeof(nm_gemv_launch_desc));', "  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[:-2] == [off for _, _, off in fields]
    assert got[-2:] == [ctypes.sizeof(_lib.NmGemvProblem), ctypes.sizeof(_lib.NmGemvLaunchDesc)]


def _desc(kind=0, nprob=3, hs=(4096, 1024, 1024), **kw):
    d = _lib.NmGemvLaunchDesc()
    d.dtype, d.kind, d.nprob, d.vec_stride, d.vec = 0, kind, nprob, 1, FAKE
    d.w, d.nnz, d.m, d.config_id, d.splits = 2048, 32, 64, -1, 0
    for i in range(nprob):
        d.prob[i].mat_data, d.prob[i].mat_index, d.prob[i].out, d.prob[i].h = FAKE, FAKE, FAKE, hs[i]
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def _launch(d, ws_bytes=1 << 30):
    return _lib.load().nm_gemv_launch(ctypes.byref(d), FAKE, ws_bytes, None)


def test_launch_descriptor_rejections_before_launch():
    lib = _lib.load()
    assert lib.nm_gemv_launch(None, FAKE, 1 << 30, None) == -1
    assert lib.nm_gemv_launch_workspace_bytes(None) == 0
    assert _launch(_desc(dtype=3)) == -7
    assert _launch(_desc(kind=2)) == -7
    assert _launch(_desc(nprob=0)) == -2
    assert _launch(_desc(kind=1, nprob=3)) == -2          # the pair takes exactly two matrices
    assert _launch(_desc(kind=1, nprob=2, hs=(4096, 1024))) == -2
    assert _launch(_desc(vec=None)) == -1
    assert _launch(_desc(), ws_bytes=1024) == -6
    # input RMSNorm: contiguous, aligned vec; non-negative eps
    assert _launch(_desc(norm_weight=FAKE, vec_stride=2)) == -8
    assert _launch(_desc(norm_weight=FAKE, vec=FAKE + 2)) == -8
    assert _launch(_desc(norm_weight=FAKE, norm_eps=-1.0)) == -8
    # heads fusions: head_dim a multiple of 64 dividing h and the tile; pos and table when used
    d = _desc()
    d.prob[0].rope = 1
    assert _launch(d) == -8                               # no head_dim
    d.head_dim = 96
    assert _launch(d) == -8
    d.head_dim = 128
    assert _launch(d) == -8                               # no pos / pos_limit
    d.pos, d.pos_limit = FAKE, 16
    assert _launch(d) == -8                               # no rope table
    d.config_id = 9                                       # tile 2048 rows, fine for head_dim 128
    e = _desc(config_id=1, head_dim=256)
    e.prob[1].head_norm = FAKE                            # th16: a tile of 128 rows < head_dim
    assert _launch(e) == -8
    p = _desc(kind=1, nprob=2, hs=(14336, 14336))
    p.prob[0].pos_stride, p.head_dim = 1, 128
    assert _launch(p) == -8                               # the pair has no heads layout
    assert lib.nm_gemv_launch_workspace_bytes(ctypes.byref(_desc())) == lib.nm_gemv_grouped_workspace_bytes(
        3, (ctypes.c_int * 3)(4096, 1024, 1024), 2048, 32, 64, -1, 0)
    assert lib.nm_gemv_launch_workspace_bytes(ctypes.byref(p)) == lib.nm_gemv_gate_up_workspace_bytes(
        14336, 2048, 32, 64, -1, 0)


def test_spmm_rejections_and_plans():
    lib = _lib.load()

    def call(dtype=0, x=FAKE, xs=4096, batch=4, md=FAKE, mi=FAKE, out=FAKE, os_=4096, ws=FAKE, wsb=1 << 30,
             h=4096, w=2048, nnz=32, m=64, cfg=-1, splits=0):
        return lib.nm_spmm(dtype, x, xs, batch, md, mi, out, os_, ws, wsb, h, w, nnz, m, cfg, splits, None)

    assert call(batch=0) == -2 and call(batch=_lib.NM_MAX_BATCH + 1) == -2
    assert call(cfg=4) == -7 and call(dtype=3) == -7
    assert call(x=None) == -1 and call(out=None) == -1
    assert call(xs=4095) == -2 and call(os_=4000) == -2
    assert call(md=FAKE + 2) == -5 and call(out=FAKE + 4) == -5
    assert call(wsb=1024) == -6
    assert call(h=100) == -3 and call(w=2047) == -4
    for batch in range(1, _lib.NM_MAX_BATCH + 1):
        for h, w in ((4096, 2048), (4096, 7168), (14336, 2048), (384, 768)):
            for cfg in (-1, 0, 1, 2, 3):
                for splits in (0, 1, 3):
                    sp = _lib.spmm_plan(batch, h, w, 32 if w % 32 == 0 else 3, 64 if w % 32 == 0 else 4, cfg, splits)
                    assert 0 < sp["rows_per_split"] <= 1024
                    need = lib.nm_spmm_workspace_bytes(batch, h, w, 32 if w % 32 == 0 else 3,
                                                       64 if w % 32 == 0 else 4, cfg, splits)
                    assert need == _lib.NM_TICKET_BYTES + (sp["splits"] * batch * h * 4 if sp["splits"] > 1 else 0)
    # same configuration and splits -> the GEMV's plan where it has <= 1024 rows per split
    for cfg in range(4):
        g, s = _lib.plan(4096, 7168, 32, 64, cfg, 0), _lib.spmm_plan(8, 4096, 7168, 32, 64, cfg, 0)
        assert (g["rows_per_split"], g["splits"]) == (s["rows_per_split"], s["splits"])


def test_spmm_mc_group_rejections_and_plans():
    """The grouped matrix-core SpMM: rejections before any launch, and its plan
    and workspace against the single-product ones."""
    lib = _lib.load()
    n_max = _lib.NM_MC_MAX_GROUP

    def arr(t, vals):
        return (t * max(len(vals), 1))(*vals)

    def call(n=3, hs=(4096, 1024, 1024), x=FAKE, xs=4096, batch=20, md=FAKE, mi=FAKE, out=FAKE, ostr=None,
             ws=FAKE, wsb=1 << 30, w=2048, nnz=32, m=64, cfg=-1, splits=0, dtype=0):
        k = len(hs)
        ostr = hs if ostr is None else ostr
        return lib.nm_spmm_mc_group(dtype, x, xs, batch, n, arr(ctypes.c_void_p, [md] * k),
                                    arr(ctypes.c_void_p, [mi] * k), arr(ctypes.c_void_p, [out] * k),
                                    arr(ctypes.c_longlong, list(ostr)), arr(ctypes.c_int, list(hs)), ws, wsb, w, nnz,
                                    m, cfg, splits, None)

    assert call(n=0, hs=()) == -2 and call(n=n_max + 1, hs=(128,) * (n_max + 1)) == -2
    assert call(batch=0) == -2 and call(batch=_lib.NM_MC_MAX_BATCH + 1) == -2
    assert call(dtype=2) == -7 and call(cfg=6) == -7
    assert call(x=None) == -1 and call(md=None) == -1 and call(out=None) == -1 and call(ws=None) == -1
    assert call(hs=(4096, 1000, 1024)) == -3 and call(w=2047) == -4
    assert call(xs=4095) == -2 and call(ostr=(4096, 1000, 1024)) == -2
    assert call(md=FAKE + 2) == -5 and call(ws=FAKE + 16) == -5 and call(wsb=1024) == -6
    for batch in (9, 16, 33, 64):
        for hs, w in (((4096, 1024, 1024), 2048), ((14336, 14336), 2048), ((384, 128, 256, 640), 500)):
            for cfg, splits in ((-1, 0), (0, 2), (3, 0), (5, 3)):
                nnz, m = (32, 64) if w == 2048 else (4, 8)
                g = _lib.spmm_mc_group_plan(batch, list(hs), w, nnz, m, cfg, splits)
                tiles = sum(-(-h // (64, 128, 256)[g["config_id"] % 3]) for h in hs)
                assert g["blocks"] == tiles * g["splits"]
                wp = -(-w // 64) * 64
                part = g["splits"] * batch * sum(hs) * 4 if g["splits"] > 1 else 0
                xg_off = -(-(_lib.NM_TICKET_BYTES + part) // 256) * 256
                need = lib.nm_spmm_mc_group_workspace_bytes(batch, len(hs), arr(ctypes.c_int, list(hs)), w, nnz, m,
                                                            cfg, splits)
                assert need == xg_off + len(hs) * (-(-batch // 16) * 16 * wp * 2)
                # a group of one is the single-product plan
                for h in hs:
                    one = _lib.spmm_mc_group_plan(batch, [h], w, nnz, m, cfg, splits)
                    assert one == _lib.spmm_mc_plan(batch, h, w, nnz, m, cfg, splits)
                    assert (lib.nm_spmm_mc_group_workspace_bytes(batch, 1, arr(ctypes.c_int, [h]), w, nnz, m, cfg,
                                                                 splits)
                            == lib.nm_spmm_mc_workspace_bytes(batch, h, w, nnz, m, cfg, splits))


def test_launch_plan_query():
    """Host-only plan query of a fused launch (shapes only: no kernel runs)."""
    import torch

    from spmv_decode_amd.hip_spmv import launch_plan

    def mats(K, h):
        return torch.empty(K // 64 * 32, h, dtype=torch.float16), torch.empty(K // 64, 32, dtype=torch.uint8)

    def summary(p):
        return p["config_id"], p["splits"], p["blocks"]

    # Llama-3.1-8B: 256-row tiles past 4096 outputs, 8 splits
    qkv = [mats(4096, 4096), mats(4096, 1024), mats(4096, 1024)]
    p = launch_plan(qkv, 32, 64)
    assert p == {"config_id": 3, "splits": 8, "blocks": (16 + 4 + 4) * 8, "rows_per_split": 256, "chunk_rows": 64}
    pair = launch_plan([mats(4096, 14336), mats(4096, 14336)], 32, 64, gate_up=True)
    assert pair["config_id"] == 1 and pair["chunk_rows"] == 32 and pair["blocks"] == 56 * 8
    down = launch_plan([mats(14336, 4096)], 32, 64)
    assert down["rows_per_split"] == 896 and down["chunk_rows"] == 128 and down["blocks"] == 256
    # Qwen3 shapes: long columns take up to 12 splits while the grid fits one
    # workgroup per CU; grids whose last round of workgroups would be mostly
    # empty take the split count (nearest 8) that fills their rounds best
    assert summary(launch_plan([mats(17408, 5120)], 32, 64)) == (3, 12, 20 * 12)
    assert summary(launch_plan([mats(5120, 8192), mats(5120, 1024), mats(5120, 1024)], 32, 64)) == (3, 6, 40 * 6)
    # the widest launches take 512-row tiles; a pair of them one round of workgroups (<= 7/8 of the CUs)
    assert summary(launch_plan([mats(5120, 25600), mats(5120, 25600)], 32, 64, gate_up=True)) == (5, 4, 50 * 4)
    assert summary(launch_plan([mats(5120, 17408), mats(5120, 17408)], 32, 64, gate_up=True)) == (5, 6, 34 * 6)
    # with a carried input the pair takes 512-row tiles at every width (half the carried reads of 256-row tiles)
    assert summary(launch_plan([mats(4096, 14336)] * 2, 32, 64, gate_up=True, carried=True)) == (4, 8, 28 * 8)
    assert summary(launch_plan([mats(5120, 17408)], 32, 64)) == (6, 7, 34 * 7)
    with pytest.raises(_lib.NmSparseLibraryError):
        launch_plan([mats(4096, 1000)], 32, 64)


def test_static_scratch_entry_rejections_before_any_hip_call():
    """nm_gemv_launch_static checks everything before it looks up its scratch:
    a missing descriptor, a rejected shape, a launch whose workspace exceeds
    NM_STATIC_SCRATCH_BYTES and bad pointers all return without a HIP call."""
    lib = _lib.load()
    assert lib.nm_gemv_launch_static(None, None) == -1
    d = _lib.NmGemvLaunchDesc()
    d.dtype, d.kind, d.nprob, d.vec_stride, d.vec = 0, 0, 1, 1, FAKE
    d.w, d.nnz, d.m, d.config_id, d.splits = 8192, 32, 64, -1, 0
    d.prob[0].mat_data, d.prob[0].mat_index, d.prob[0].out, d.prob[0].h = FAKE, FAKE, FAKE, 100
    assert lib.nm_gemv_launch_static(ctypes.byref(d), None) == -3
    d.prob[0].h = 128256
    d.splits = 40  # 37 splits x 128256 fp32 partials: more than the static scratch
    assert lib.nm_gemv_launch_workspace_bytes(ctypes.byref(d)) > _lib.NM_STATIC_SCRATCH_BYTES
    assert lib.nm_gemv_launch_static(ctypes.byref(d), None) == -9
    d.splits = 0
    assert 0 < lib.nm_gemv_launch_workspace_bytes(ctypes.byref(d)) <= _lib.NM_STATIC_SCRATCH_BYTES
    d.prob[0].out = FAKE + 8
    assert lib.nm_gemv_launch_static(ctypes.byref(d), None) == -5
    d.prob[0].out = None
    assert lib.nm_gemv_launch_static(ctypes.byref(d), None) == -1
    assert f"#define NM_STATIC_SCRATCH_BYTES (NM_TICKET_BYTES + (16 << 20))" in HEADER.read_text()
    assert _lib.NM_STATIC_SCRATCH_BYTES == _lib.NM_TICKET_BYTES + (16 << 20)


def test_carried_vec_out_must_not_overlap_any_launch_buffer():
    """A carried consumer's tile-0 workgroups write vec_out while the other
    workgroups still read the launch's inputs and write its outputs, so the
    host rejects (NM_ERR_BAD_EPILOGUE) a vec_out that overlaps any of them:
    norm weight, every matrix and index, every output (plain or heads
    layout), residual, head norm, RoPE table, position, workspace, carry_in."""
    VO = FAKE + (1 << 36)
    K = 4096  # w = 2048 at 32:64
    ok = dict(carry_in=FAKE, carry_splits=8, vec_out=VO)
    pair = dict(kind=1, nprob=2, hs=(14336, 14336), norm_weight=FAKE)
    inside = VO + 2 * K - 16   # the last 16 bytes of vec_out

    def pair_with(**fields):
        d = _desc(**pair, **ok)
        for k, v in fields.items():
            if k.startswith("p0_") or k.startswith("p1_"):
                setattr(d.prob[int(k[1])], k[3:], v)
            else:
                setattr(d, k, v)
        return d

    def rejected(d):
        return _lib.load().nm_gemv_launch_workspace_bytes(ctypes.byref(d)) > 0 and _launch(d) == -8

    assert rejected(pair_with(norm_weight=inside))
    assert rejected(pair_with(p0_mat_data=VO - 2 * 2048 * 14336 + 16))  # the gate matrix's last bytes
    assert rejected(pair_with(p1_mat_data=inside))                       # the up matrix
    assert rejected(pair_with(p1_mat_index=VO - 2048 + 16))
    assert rejected(pair_with(p0_out=VO - 2 * 14336 + 16))               # the pair's output
    assert rejected(pair_with(p0_residual=inside))
    assert _launch(_desc(**pair, **ok), ws_bytes=(1 << 36) + 16) == -8   # the workspace at FAKE reaches vec_out
    assert not rejected(pair_with(norm_weight=VO - 2 * K))             # ends where vec_out begins
    assert not rejected(pair_with(p0_out=VO - 2 * 14336))
    assert not rejected(pair_with(p0_residual=VO + 2 * K))             # begins where vec_out ends
    # q/k/v consumer with heads layouts, head norms, the RoPE table and the position
    qkv = dict(kind=0, nprob=3, hs=(4096, 1024, 1024), norm_weight=FAKE, head_dim=128, pos=FAKE, pos_limit=512,
               rope_table=FAKE)

    def qkv_with(**fields):
        d = _desc(**qkv, **ok)
        for i in range(3):
            d.prob[i].rope = int(i < 2)
        d.prob[1].head_stride, d.prob[1].elem_stride, d.prob[1].pos_stride = 160 * 512, 512, 1  # key cache
        for k, v in fields.items():
            if k[0] == "p" and k[2] == "_":
                setattr(d.prob[int(k[1])], k[3:], v)
            else:
                setattr(d, k, v)
        return d

    assert _launch(qkv_with(), ws_bytes=1 << 20) != -8
    # the key cache [8, 160, 512] ends at (7 * 160 * 512 + 127 * 512 + 511 + 1) elements past its base
    extent = 2 * (7 * 160 * 512 + 127 * 512 + 512)
    assert _launch(qkv_with(p1_out=VO - extent + 16), ws_bytes=1 << 20) == -8
    assert _launch(qkv_with(p1_out=VO - extent), ws_bytes=1 << 20) != -8
    assert _launch(qkv_with(p0_head_norm=VO - 2 * 128 + 16), ws_bytes=1 << 20) == -8
    assert _launch(qkv_with(rope_table=VO - 512 * 64 * 8 + 16), ws_bytes=1 << 20) == -8
    assert _launch(qkv_with(pos=VO), ws_bytes=1 << 20) == -8
    assert _launch(qkv_with(p2_out=inside), ws_bytes=1 << 20) == -8


def test_split_k_carry_rejections_and_plans_before_launch():
    """The carry descriptor fields: producer and consumer roles, their limits
    and the consumer's plan (whole groups, <= 512 columns and <= 1024
    positions of K per split), all decided on the host."""
    import torch

    from spmv_decode_amd.hip_spmv import launch_plan

    lib = _lib.load()
    pair = dict(kind=1, nprob=2, hs=(14336, 14336), norm_weight=FAKE)
    VO = FAKE + (1 << 36)  # far from every other placeholder range
    ok = dict(carry_in=FAKE, carry_splits=8, vec_out=VO)
    # a consumer needs the input norm, 1..16 producer splits, M a multiple of 4, vec_out apart from vec
    assert _launch(_desc(**{**pair, "norm_weight": None}, **ok)) == -8
    assert _launch(_desc(**pair, **{**ok, "carry_splits": 0})) == -8
    assert _launch(_desc(**pair, **{**ok, "carry_splits": 17})) == -8
    assert _launch(_desc(**pair, **{**ok, "vec_out": None})) == -8
    assert _launch(_desc(**pair, **{**ok, "vec_out": FAKE})) == -8                  # overlaps vec
    assert _launch(_desc(**pair, **{**ok, "carry_in": VO - 16})) == -8              # vec_out inside carry_in
    assert _launch(_desc(**pair, **{**ok, "vec_out": VO + 8})) == -5                # misaligned
    assert _launch(_desc(**pair, **{**ok, "carry_in": FAKE + 4})) == -5
    assert _launch(_desc(**{**pair, "norm_weight": FAKE + 2}, **ok)) == -5
    assert _launch(_desc(**pair, **ok, m=6, nnz=3, w=2040)) == -8                    # M not a multiple of 4
    # a split of more than 1024 positions of K (1:4 density, 512 columns) cannot carry
    assert _launch(_desc(**pair, **ok, nnz=16, m=64, w=1024, splits=2)) == -8
    # producer and consumer at once; a producer is one plain GEMV without epilogue
    assert _launch(_desc(**pair, **ok, carry_out=FAKE)) == -8
    prod = dict(nprob=1, hs=(4096,), carry_out=FAKE)
    assert _launch(_desc(**prod, norm_weight=FAKE)) == -8
    d = _desc(**prod)
    d.prob[0].residual = FAKE
    assert _launch(d) == -8
    d = _desc(**prod)
    d.prob[0].rope, d.head_dim = 1, 128
    assert _launch(d) == -8
    d = _desc(**prod)
    d.carry_out = FAKE + 4
    assert _launch(d) == -5
    # the consumer's workspace adds one float per workgroup for the slices' sums of squares
    plain = lib.nm_gemv_launch_workspace_bytes(ctypes.byref(_desc(**pair)))
    carried = lib.nm_gemv_launch_workspace_bytes(ctypes.byref(_desc(**pair, **ok)))
    assert carried == plain + 28 * 8 * 4  # the carried plan: 28 tiles of 512 rows x 8 splits

    def mats(K, h, nnz=32, m=64):
        return (torch.empty(K // m * nnz, h, dtype=torch.float16), torch.empty(K // m, nnz, dtype=torch.uint8))

    # consumer plans of the decoder shapes: whole groups, <= 512 columns, <= 1024 positions per split
    for K, hs, nnz, m, gate_up in ((4096, (14336, 14336), 32, 64, True), (4096, (4096, 1024, 1024), 32, 64, False),
                                   (5120, (17408, 17408), 32, 64, True), (5120, (5120, 1024, 1024), 32, 64, False),
                                   (5120, (25600, 25600), 16, 32, True), (5120, (8192, 1024, 1024), 16, 32, False),
                                   (4096, (14336, 14336), 128, 256, True), (4096, (4096, 1024, 1024), 2, 4, False)):
        p = launch_plan([mats(K, h, nnz, m) for h in hs], nnz, m, gate_up=gate_up, carried=True)
        rows = p["rows_per_split"]
        assert rows % nnz == 0 and rows % p["chunk_rows"] == 0 and rows <= 512 and rows // nnz * m <= 1024, (K, hs, p)
    # the Llama-3.1-8B q/k/v consumer keeps the plain plan
    qkv = [mats(4096, h) for h in (4096, 1024, 1024)]
    assert launch_plan(qkv, 32, 64, carried=True) == launch_plan(qkv, 32, 64)
    # a producer whose plan would leave a quarter of the CUs idle takes 128-row tiles and more splits
    # (Qwen3-14B / Qwen3-32B o_proj); the Llama-3.1-8B o_proj and every down_proj keep their plans
    for K, h, nnz, m, want in ((5120, 5120, 32, 64, (1, 5, 200)), (8192, 5120, 16, 32, (1, 6, 240)),
                               (4096, 4096, 32, 64, None), (14336, 4096, 32, 64, None), (17408, 5120, 32, 64, None)):
        plain = launch_plan([mats(K, h, nnz, m)], nnz, m)
        prod = launch_plan([mats(K, h, nnz, m)], nnz, m, producer=True)
        got = (prod["config_id"], prod["splits"], prod["blocks"])
        assert got == (want or (plain["config_id"], plain["splits"], plain["blocks"])), (K, h, plain, prod)
        if want:
            assert plain["blocks"] <= 192 < prod["blocks"] <= 256 and prod["splits"] <= 16
    # explicit configurations and split counts are kept as asked
    p = launch_plan([mats(5120, 5120)], 32, 64, producer=True, config_id=3, splits=8)
    assert (p["config_id"], p["splits"], p["blocks"]) == (3, 8, 160)


def test_accumulated_carry_rejections_before_launch():
    """The accumulated carry's descriptor fields: carry_accumulate needs
    carry_out; the gate/up pair is a producer only in that form, without a
    residual, and with a carried input at most 16 splits (one sum of squares
    per split); the SiLU-product input feeds one plain GEMV without norm,
    carried input or heads fusions, 16-byte aligned, with 0..16 sums of
    squares, silu_k > 0 when it has some and eps >= 0 (vec may then be null);
    zero_buf is 16-byte aligned, a positive multiple of 4 floats, apart from
    every buffer of the launch."""
    VO = FAKE + (1 << 36)
    ACC = FAKE + (1 << 38)
    h = 14336
    pair = dict(kind=1, nprob=2, hs=(h, h), norm_weight=FAKE)
    carried = dict(carry_in=FAKE, carry_splits=1, vec_out=VO)

    def accepted(d):  # every check passed: the launch itself fails (no GPU here)
        return _launch(d) not in (-1, -2, -5, -6, -7, -8)

    # carry_accumulate without carry_out; the pair as a producer without it, or with a residual
    assert _launch(_desc(nprob=1, hs=(4096,), carry_accumulate=1)) == -8
    assert _launch(_desc(**pair, carry_out=ACC)) == -8
    d = _desc(**pair, carry_out=ACC, carry_accumulate=1)
    d.prob[0].residual = FAKE
    assert _launch(d) == -8
    assert accepted(_desc(**pair, carry_out=ACC, carry_accumulate=1))
    assert accepted(_desc(**pair, **carried, carry_out=ACC, carry_accumulate=1))
    assert accepted(_desc(nprob=1, hs=(4096,), carry_out=ACC, carry_accumulate=1))
    # a carried pair of more than 16 splits has no room for its sums of squares; as a plain consumer it runs
    big = dict(w=16384, **{**carried, "carry_splits": 1})
    assert accepted(_desc(**pair, **big))
    assert _launch(_desc(**pair, **big, carry_out=ACC, carry_accumulate=1)) == -8
    # the pair's buffer [2h + 16] must not overlap its other buffers
    assert _launch(_desc(**pair, **carried, carry_out=VO - 16, carry_accumulate=1)) == -8
    assert _launch(_desc(**pair, **carried, carry_out=ACC, carry_accumulate=1,
                         zero_buf=ACC + 4 * (2 * h + 12), zero_len=4)) == -8
    assert accepted(_desc(**pair, **carried, carry_out=ACC, carry_accumulate=1,
                          zero_buf=ACC + 4 * (2 * h + 16), zero_len=4))
    # the SiLU-product input: one plain GEMV, K = 4096 (w 2048 at 32:64), vec unused
    silu = dict(nprob=1, hs=(4096,), vec=None, silu_in=ACC, silu_ssq_n=4, silu_k=4096, silu_eps=1e-5)
    assert accepted(_desc(**silu))
    assert accepted(_desc(**silu, carry_out=VO, carry_accumulate=1))
    assert _launch(_desc(**silu, norm_weight=FAKE)) == -8
    assert _launch(_desc(**silu, **carried)) == -8
    assert _launch(_desc(**{**silu, "nprob": 2, "hs": (4096, 4096)})) == -8
    assert _launch(_desc(**{**pair, "vec": None}, silu_in=ACC, silu_ssq_n=1, silu_k=4096)) == -8
    assert _launch(_desc(**{**silu, "silu_ssq_n": 17})) == -8
    assert _launch(_desc(**{**silu, "silu_ssq_n": -1})) == -8
    assert _launch(_desc(**{**silu, "silu_k": 0})) == -8
    assert accepted(_desc(**{**silu, "silu_k": 0, "silu_ssq_n": 0}))
    assert _launch(_desc(**{**silu, "silu_eps": -1.0})) == -8
    assert _launch(_desc(**{**silu, "silu_in": ACC + 8})) == -5
    d = _desc(**silu)
    d.prob[0].rope, d.head_dim = 1, 128
    assert _launch(d) == -8
    d = _desc(**silu)
    d.prob[0].out = ACC + 4 * 100  # the output inside silu_in [2K + 4]
    assert _launch(d) == -8
    # zero_buf: shape, alignment, and apart from vec, outputs and every other buffer
    plain = dict(nprob=1, hs=(4096,))
    Z = FAKE + (1 << 40)
    assert accepted(_desc(**plain, zero_buf=Z, zero_len=4096))
    assert _launch(_desc(**plain, zero_buf=Z, zero_len=0)) == -8
    assert _launch(_desc(**plain, zero_buf=Z, zero_len=6)) == -8
    assert _launch(_desc(**plain, zero_buf=Z + 4, zero_len=4)) == -5
    assert _launch(_desc(**plain, zero_buf=FAKE, zero_len=4)) == -8          # vec (and the matrix, output)
    d = _desc(**plain, zero_buf=Z, zero_len=4096)
    d.prob[0].out = Z + 4096 * 4 - 16                                         # the buffer's last 16 bytes
    assert _launch(d) == -8
    d.prob[0].out = Z + 4096 * 4
    assert accepted(d)
    assert _launch(_desc(**plain, zero_buf=Z, zero_len=4096, carry_out=Z + 4 * 4092, carry_accumulate=1)) == -8
    assert _launch(_desc(**silu, zero_buf=ACC + 4 * 8192, zero_len=4)) == -8  # the sums of squares of silu_in
    assert accepted(_desc(**silu, zero_buf=ACC + 4 * 8196, zero_len=4))
