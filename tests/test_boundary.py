"""Host-side behaviour of the drop-in boundary, on CPU tensors (no GPU).

Covers the launch wrapper's argument checks (compared with the oracle's
restatement of triton_spmv.py:245-294), the `nmsparse::gemv` op schema, fake
implementation and rows check (src/spmv/nmsparse_op.py:77-123), and the
module API: `_make_sparse` bit-exactness, `NmSparseLinear`, and
`swap_to_nmsparse` against fixtures written from the reference itself.
"""
import hashlib
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch
import torch.nn as nn

from conftest import GOLDEN, ROOT
from oracle import nm_oracle as O
from spmv_decode_amd import hip_spmv, nmsparse_linear, nmsparse_op  # noqa: F401


# ---------------------------------------------------------------------------
# wrapper argument checks
# ---------------------------------------------------------------------------
def _spec_tensors(spec):
    vec = torch.zeros(spec["vec_shape"], dtype=spec["vec_dtype"])
    md = torch.zeros(spec["mat_shape"], dtype=spec["mat_dtype"])
    mi = torch.zeros(spec["index_shape"], dtype=spec["index_dtype"])
    if not spec["contiguous"][0]:
        r, k = spec["vec_shape"]
        vec = torch.zeros(r, 2 * k, dtype=spec["vec_dtype"])[:, ::2]
    if not spec["contiguous"][1]:
        md = torch.zeros(spec["mat_shape"][::-1], dtype=spec["mat_dtype"]).t()
    if not spec["contiguous"][2]:
        mi = torch.zeros(spec["index_shape"][::-1], dtype=spec["index_dtype"]).t()
    return vec, md, mi


def _base(**kw):
    spec = dict(is_cuda=(True, True, True), vec_dtype=torch.float16, mat_dtype=torch.float16,
                index_dtype=torch.uint8, vec_shape=(1, 256), mat_shape=(128, 256), index_shape=(64, 2),
                w=128, h=256, bw=2, threads=128, vw=4, minibatch=1, vecnum=256,
                contiguous=(True, True, True), arch="auto")
    spec.update(kw)
    return spec


CASES = {
    "ok": _base(),
    "vec_dtype": _base(vec_dtype=torch.int32),
    "mat_dtype": _base(mat_dtype=torch.bfloat16),
    "index_dtype": _base(index_dtype=torch.int8),
    "vec_1d": _base(vec_shape=(256,)),
    "vec_rows": _base(vec_shape=(2, 256)),
    "minibatch2": _base(vec_shape=(2, 256), minibatch=2),
    "vecnum": _base(vecnum=512),
    "threads": _base(threads=256),
    "h_not_128": _base(h=200, mat_shape=(128, 200)),
    "w_not_bw": _base(w=127, mat_shape=(127, 256)),
    "mat_shape": _base(mat_shape=(128, 384)),
    "index_shape": _base(index_shape=(32, 4)),
    "mat_noncontig": _base(contiguous=(True, False, True)),
    "index_noncontig": _base(contiguous=(True, True, False)),
    "vec_noncontig": _base(vec_shape=(1, 256), contiguous=(False, True, True)),
    "arch_bad": _base(arch="h100"),
    "arch_a100": _base(arch="A100"),
    "bf16": _base(vec_dtype=torch.bfloat16, mat_dtype=torch.bfloat16),
    "f32": _base(vec_dtype=torch.float32, mat_dtype=torch.float32),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_validation_matches_reference_order(name):
    spec = CASES[name]
    vec, md, mi = _spec_tensors(spec)
    expected = O.expected_exception(spec)
    args = (vec, md, mi, spec["w"], spec["h"], spec["bw"], spec["threads"], spec["vw"], spec["minibatch"],
            spec["vecnum"], spec["arch"])
    if expected is None:
        hip_spmv.validate_args(*args, require_device=False)
    else:
        with pytest.raises(expected):
            hip_spmv.validate_args(*args, require_device=False)


def _fixture_spec(spec):
    spec = dict(spec)
    for k in ("vec_dtype", "mat_dtype", "index_dtype"):
        spec[k] = getattr(torch, spec[k])
    return spec


WRAPPER_CASES = json.loads((GOLDEN / "wrapper_validation.json").read_text())["cases"]


@pytest.mark.parametrize("name", sorted(WRAPPER_CASES))
def test_validation_matches_reference_fixture(name):
    """The oracle's restatement and the product's checks against what the
    reference wrapper raised for the same call (tests/golden/
    make_validation_golden.py): same exception type, and the same message
    except where this build differs on purpose (a device check that names
    HIP, and `arch` also accepting "gfx950")."""
    case = WRAPPER_CASES[name]
    spec = _fixture_spec(case["spec"])
    want = case["raises"]
    got = O.expected_exception(spec)
    assert (got.__name__ if got else None) == want
    vec, md, mi = _spec_tensors(spec)
    args = (vec, md, mi, spec["w"], spec["h"], spec["bw"], spec["threads"], spec["vw"], spec["minibatch"],
            spec["vecnum"], spec["arch"])
    if not all(spec["is_cuda"]):
        with pytest.raises(ValueError, match="GPU"):  # CPU tensors here: the device check fires first
            hip_spmv.nmsparse_spmv_forward_hip(*args)
        return
    if spec["arch"] == "gfx950":
        hip_spmv.validate_args(*args, require_device=False)  # accepted by this build (its own target)
        return
    if want is None:
        hip_spmv.validate_args(*args, require_device=False)
        return
    exc = {"ValueError": ValueError, "TypeError": TypeError, "NotImplementedError": NotImplementedError}[want]
    with pytest.raises(exc) as e:
        hip_spmv.validate_args(*args, require_device=False)
    if spec["arch"] == "auto" or want != "ValueError" or "arch" not in str(e.value):
        assert str(e.value) == case["message"]


def test_cpu_tensors_rejected_first():
    vec, md, mi = _spec_tensors(_base(vec_dtype=torch.int32))  # dtype also wrong: device check comes first
    with pytest.raises(ValueError, match="GPU"):
        hip_spmv.nmsparse_spmv_forward_hip(vec, md, mi, 128, 256, 2, 128, 4, 1, 256)
    assert hip_spmv.nmsparse_spmv_forward_triton_ptx is hip_spmv.nmsparse_spmv_forward_hip


def test_implementation_limits_raise_value_error():
    # M > 256 cannot be addressed by uint8 positions; vecNum must be (w/N)*M.
    spec = _base(vw=512, vec_shape=(1, 512 * 64), vecnum=512 * 64)
    vec, md, mi = _spec_tensors(spec)
    with pytest.raises(ValueError):
        hip_spmv.validate_args(vec, md, mi, 128, 256, 2, 128, 512, 1, 512 * 64, require_device=False)
    spec = _base(vec_shape=(1, 300), vecnum=300)
    vec, md, mi = _spec_tensors(spec)
    with pytest.raises(ValueError):
        hip_spmv.validate_args(vec, md, mi, 128, 256, 2, 128, 4, 1, 300, require_device=False)


def test_qkv_decode_buffer_arguments():
    """Exactly one value cache, of the layout its name states; queries as one
    row or as padded head rows; keys with at least head_dim rows. Checked
    before any launch (these CPU tensors never reach one)."""
    kvh, hd, S, K = 2, 64, 16, 256
    x = torch.zeros(1, K, dtype=torch.float16)
    mat = (torch.zeros(128, kvh * hd, dtype=torch.float16), torch.zeros(64, 2, dtype=torch.uint8))
    rows, cols = torch.zeros(kvh, S, hd, dtype=torch.float16), torch.zeros(kvh, hd, S, dtype=torch.float16)
    good = dict(q_out=torch.zeros(1, kvh * hd, dtype=torch.float16), k_cache_t=torch.zeros(kvh, hd + 8, S,
                dtype=torch.float16), v_cache_t=cols, pos=torch.zeros(1, dtype=torch.long),
                rope_table=torch.zeros(S, hd // 2, dtype=torch.complex64), head_dim=hd)
    bad = [dict(v_cache_t=None), dict(v_cache=rows), dict(v_cache_t=None, v_cache=cols), dict(v_cache_t=rows),
           dict(q_out=torch.zeros(1, kvh * hd + 8, dtype=torch.float16)),
           dict(q_out=torch.zeros(kvh, hd - 8, dtype=torch.float16)),
           dict(k_cache_t=torch.zeros(kvh, hd - 8, S, dtype=torch.float16))]
    for change in bad:
        with pytest.raises(ValueError):
            hip_spmv.nmsparse_qkv_decode(x, mat, mat, mat, 2, 4, **{**good, **change})
    # the same arguments get past these checks to the device check of the launch
    for q_out in (good["q_out"], torch.zeros(kvh, hd + 8, dtype=torch.float16)):
        with pytest.raises(ValueError, match="GPU"):
            hip_spmv.nmsparse_qkv_decode(x, mat, mat, mat, 2, 4, **{**good, "q_out": q_out})


# ---------------------------------------------------------------------------
# the custom op
# ---------------------------------------------------------------------------
def test_op_schema_matches_reference():
    schema = str(torch.ops.nmsparse.gemv.default._schema)
    assert schema == ("nmsparse::gemv(Tensor x, Tensor mat_data, Tensor mat_index, SymInt w, SymInt h, "
                      "SymInt block_width, SymInt vec_width) -> Tensor")
    assert nmsparse_op._mode == "hip"


def test_op_fake_impl_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(1, 1, 4096, dtype=torch.float16)
        md = torch.empty(2048, 1024, dtype=torch.float16)
        mi = torch.empty(64, 32, dtype=torch.uint8)
        y = torch.ops.nmsparse.gemv(x, md, mi, 2048, 1024, 32, 64)
        assert tuple(y.shape) == (1, 1, 1024) and y.dtype == torch.float16
        y = torch.ops.nmsparse.gemv(x.bfloat16(), md, mi, 2048, 1024, 32, 64)
        assert y.dtype == torch.bfloat16


def test_fused_decode_ops_schemas_and_fakes():
    """The fused decode launches are ops (so a compiled step traces them): their
    mutated arguments are declared, gate_up_silu's fake output is [1, h]."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    assert "Tensor(a9!) q_out" in str(torch.ops.nmsparse.qkv_decode.default._schema)
    assert "Tensor(a5!) out" in str(torch.ops.nmsparse.gemv_add_.default._schema)
    with FakeTensorMode():
        x = torch.empty(1, 4096, dtype=torch.float16)
        md = torch.empty(2048, 14336, dtype=torch.float16)
        mi = torch.empty(64, 32, dtype=torch.uint8)
        y = torch.ops.nmsparse.gate_up_silu(x, md, mi, md, mi, 32, 64, torch.empty(4096, dtype=torch.float16), 1e-5)
        assert tuple(y.shape) == (1, 14336) and y.dtype == torch.float16


def test_op_rejects_more_than_one_row():
    x = torch.zeros(1, 2, 256, dtype=torch.float16)
    md = torch.zeros(128, 256, dtype=torch.float16)
    mi = torch.zeros(64, 2, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="rows==1"):
        torch.ops.nmsparse.gemv(x, md, mi, 128, 256, 2, 4)


def _run_py(code, **env):
    e = dict(os.environ)
    e.update(env)
    return subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=e, capture_output=True, text=True)


def test_nm_kernel_env_contract():
    imp = "import spmv_decode_amd.nmsparse_op as m; print(m._mode)"
    assert _run_py(imp, NM_KERNEL="triton_ptx").stdout.strip() == "triton_ptx"
    assert _run_py(imp).stdout.strip() == "hip"
    assert _run_py(imp, NM_KERNEL="hip").stdout.strip() == "hip"
    r = _run_py(imp, NM_KERNEL="bogus")
    assert r.returncode != 0 and "refusing silent fallback" in r.stderr
    r = _run_py(imp, NM_KERNEL="fp16_split")
    assert r.returncode != 0 and "NotImplementedError" in r.stderr


def test_flat_import_shims():
    code = ("import sys; sys.path.insert(0, 'spmv_decode_amd/compat'); import nmsparse_linear as s, nmsparse_op, "
            "triton_spmv; print(s.NmSparseLinear.__module__, nmsparse_op._mode, "
            "triton_spmv.nmsparse_spmv_forward_triton_ptx.__name__)")
    r = _run_py(code)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == ["spmv_decode_amd.nmsparse_linear", "hip", "nmsparse_spmv_forward_hip"]


def test_reference_harness_mode_check_passes_through_the_flat_imports():
    """The reference benchmarks import `nmsparse_op` flat under NM_KERNEL=triton_ptx and
    refuse to run unless `nmsparse_op._mode == "triton_ptx"`
    (benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:95); the shared-mask layout branch of
    `_make_sparse` is the one that mode selects (src/spmv/nmsparse_linear.py:11,22)."""
    code = ("import sys; sys.path.insert(0, 'spmv_decode_amd/compat'); import nmsparse_op, nmsparse_linear as s\n"
            "if nmsparse_op._mode != 'triton_ptx':\n"
            "    raise RuntimeError('This benchmark requires NM_KERNEL=triton_ptx')\n"
            "md, mi, w, nnz = s._make_sparse(256, 128, 16, 0, 'cpu')\n"
            "print(nmsparse_op._mode, tuple(mi.shape), mi.dtype)")
    r = _run_py(code, NM_KERNEL="triton_ptx")
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == ["triton_ptx", "(16,", "8)", "torch.uint8"]


# ---------------------------------------------------------------------------
# module API
# ---------------------------------------------------------------------------
MS = json.loads((GOLDEN / "make_sparse.json").read_text())
MS_ARR = np.load(GOLDEN / "make_sparse_small.npz")


@pytest.mark.parametrize("case", MS["small"], ids=lambda c: c["tag"])
def test_product_make_sparse_bit_exact(case):
    md, mi, w, nnz = nmsparse_linear._make_sparse(case["K"], case["N"], case["M"], case["seed"], "cpu")
    assert (w, nnz) == (case["w"], case["nnz"])
    np.testing.assert_array_equal(md.view(torch.int16).numpy().view(np.uint16), MS_ARR[f"{case['tag']}_mat_data_bits"])
    np.testing.assert_array_equal(mi.numpy(), MS_ARR[f"{case['tag']}_mat_index"])


def test_product_make_sparse_digest_config1():
    case = MS["digests"][0]
    md, mi, _, _ = nmsparse_linear._make_sparse(case["K"], case["N"], case["M"], case["seed"], "cpu")
    assert hashlib.sha256(md.view(torch.int16).numpy().tobytes()).hexdigest() == case["mat_data_sha256"]
    assert hashlib.sha256(mi.numpy().tobytes()).hexdigest() == case["mat_index_sha256"]


def test_linear_attributes_and_buffers():
    lin = nmsparse_linear.NmSparseLinear(256, 64, 8, 0, "cpu")
    ref_md, ref_mi, w, nnz = O.make_sparse(64, 256, 8, 0)
    assert (lin.h, lin.w, lin.block_width, lin.vec_width) == (256, 32, 4, 8)
    assert torch.equal(lin.mat_data.view(torch.int16), ref_md.view(torch.int16)) and torch.equal(lin.mat_index, ref_mi)
    assert set(dict(lin.named_buffers())) == {"mat_data", "mat_index"}
    assert lin.weight is None
    with pytest.raises(AssertionError):
        nmsparse_linear.NmSparseLinear(200, 64, 8, 0, "cpu")
    with pytest.raises(AssertionError):
        nmsparse_linear.NmSparseLinear(256, 60, 8, 0, "cpu")


def test_linear_prefill_uses_dense_weight():
    dense = nn.Parameter(torch.randn(256, 64))
    lin = nmsparse_linear.NmSparseLinear(256, 64, 8, 0, "cpu", dense_weight=dense)
    x = torch.randn(1, 3, 64)
    torch.testing.assert_close(lin(x), torch.nn.functional.linear(x, dense))
    bare = nmsparse_linear.NmSparseLinear(256, 64, 8, 0, "cpu")
    # without a dense weight this build computes batch > 1 with the sparse
    # SpMM (a device kernel: CPU tensors are rejected like the GEMV's) ...
    with pytest.raises(ValueError, match="must be GPU"):
        bare(x)
    # ... and NM_SPARSE_BATCH=0 restores the reference's error
    code = ("import torch; from spmv_decode_amd import nmsparse_linear as s; "
            "m = s.NmSparseLinear(256, 64, 8, 0, 'cpu'); m(torch.randn(1, 3, 64))")
    r = _run_py(code, NM_SPARSE_BATCH="0")
    assert r.returncode != 0 and "prefill requires dense weight" in r.stderr
    r = _run_py("import spmv_decode_amd", NM_SPARSE_BATCH="2")
    assert r.returncode != 0 and "Unknown NM_SPARSE_BATCH" in r.stderr


def test_decode_only_env_drops_dense_weight():
    code = ("import torch, torch.nn as nn; from spmv_decode_amd import nmsparse_linear as s; "
            "m = nn.Module(); m.layers = nn.ModuleList([nn.Module()]); b = m.layers[0]; "
            "b.attention = nn.Module(); b.attention.wqkv = nn.Linear(128, 384, bias=False); "
            "b.attention.wo = nn.Linear(128, 128, bias=False); b.feed_forward = nn.Module(); "
            "b.feed_forward.w1 = nn.Linear(128, 256, bias=False); b.feed_forward.w3 = nn.Linear(128, 256, bias=False); "
            "b.feed_forward.w2 = nn.Linear(256, 128, bias=False); "
            "print(s.swap_to_nmsparse(m, 4, 'cpu'), s.DECODE_ONLY, s.WEIGHT_CPU, b.attention.wqkv.weight is None)")
    r = _run_py(code, NM_DECODE_ONLY="1")
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == ["5", "True", "True", "True"]


def test_pack_dense_matches_oracle_pack():
    K, N, M = 256, 384, 8
    _, mi, _, nnz = O.make_sparse(K, N, M, 1)
    W = torch.randn(N, K, dtype=torch.float16)
    packed = nmsparse_linear.pack_dense(W, mi, M)
    assert torch.equal(packed, O.pack(W, mi, nnz, M))
    lin = nmsparse_linear.NmSparseLinear.from_dense(W, mi, M)
    assert torch.equal(lin.mat_data, packed) and (lin.h, lin.w, lin.block_width, lin.vec_width) == (N, K // 2, 4, 8)
    with pytest.raises(ValueError):
        nmsparse_linear.NmSparseLinear.from_dense(W, mi[:-1], M)


# ---------------------------------------------------------------------------
# swap_to_nmsparse vs the reference's own output
# ---------------------------------------------------------------------------
SWAP = json.loads((GOLDEN / "swap_to_nmsparse.json").read_text())


class _GptFastBlock(nn.Module):
    def __init__(self, dim, n_kv, inter):
        super().__init__()
        self.attention = nn.Module()
        self.attention.wqkv = nn.Linear(dim, dim + 2 * n_kv, bias=False)
        self.attention.wo = nn.Linear(dim, dim, bias=False)
        self.feed_forward = nn.Module()
        self.feed_forward.w1 = nn.Linear(dim, inter, bias=False)
        self.feed_forward.w3 = nn.Linear(dim, inter, bias=False)
        self.feed_forward.w2 = nn.Linear(inter, dim, bias=False)


class _HfBlock(nn.Module):
    def __init__(self, dim, n_kv, inter):
        super().__init__()
        self.self_attn = nn.Module()
        for name, (o, i) in dict(q_proj=(dim, dim), k_proj=(n_kv, dim), v_proj=(n_kv, dim), o_proj=(dim, dim)).items():
            setattr(self.self_attn, name, nn.Linear(i, o, bias=False))
        self.mlp = nn.Module()
        for name, (o, i) in dict(gate_proj=(inter, dim), up_proj=(inter, dim), down_proj=(dim, inter)).items():
            setattr(self.mlp, name, nn.Linear(i, o, bias=False))


class _Stack(nn.Module):
    def __init__(self, block_cls, n_layers, dim, n_kv, inter):
        super().__init__()
        self.layers = nn.ModuleList(block_cls(dim, n_kv, inter) for _ in range(n_layers))


@pytest.mark.parametrize("name,block,M,seed", [("gptfast_L2_d256_kv128_i384_M8_seed5", _GptFastBlock, 8, 5),
                                               ("hf_L2_d256_kv128_i384_M4_seed0", _HfBlock, 4, 0)])
def test_swap_to_nmsparse_matches_reference(name, block, M, seed):
    model = _Stack(block, 2, 256, 128, 384)
    count = nmsparse_linear.swap_to_nmsparse(model, M, "cpu", seed=seed)
    ref = SWAP["models"][name]
    assert count == ref["count"]
    got = [(n, m) for n, m in model.named_modules() if isinstance(m, nmsparse_linear.NmSparseLinear)]
    assert [n for n, _ in got] == [e["path"] for e in ref["linears"]]
    for (n, mod), e in zip(got, ref["linears"]):
        assert (mod.h, mod.w, mod.block_width, mod.vec_width) == (e["h"], e["w"], e["block_width"], e["vec_width"])
        assert hashlib.sha256(mod.mat_data.view(torch.int16).numpy().tobytes()).hexdigest() == e["mat_data_sha256"], n
        assert hashlib.sha256(mod.mat_index.numpy().tobytes()).hexdigest() == e["mat_index_sha256"], n
        assert (mod.weight is not None) == e["has_dense_weight"]


def test_swap_rejects_unknown_layout_and_places_blocks():
    model = nn.Module()
    model.layers = nn.ModuleList([nn.Module()])
    with pytest.raises(AttributeError, match="attention"):
        nmsparse_linear.swap_to_nmsparse(model, 4, "cpu")
    stack = _Stack(_HfBlock, 2, 128, 128, 256)
    assert nmsparse_linear.swap_to_nmsparse(stack, 4, "cuda", block_devices=["cpu", "cpu"]) == 14


# ---------------------------------------------------------------------------
# workspaces: per stream, never lent to another stream's capture
# ---------------------------------------------------------------------------
def test_workspace_for_never_lends_another_streams_workspace(monkeypatch):
    """Eager calls get their stream's own zeroed workspace; a capture uses the capture
    stream's own warmed workspace or one owned by that capture (keyed by capture id,
    counters cleared, earlier ones kept while the capture lasts), never another
    stream's. The reference's per-call scratch is always capture-private
    (triton_spmv.py:285). Run on CPU tensors with the capture state simulated."""
    from spmv_decode_amd import _lib
    from spmv_decode_amd import hip_spmv as H

    dev = torch.device("cpu")
    monkeypatch.setattr(H, "_workspaces", {})
    monkeypatch.setattr(H, "_capture_workspaces", {})
    monkeypatch.setattr(H, "_retired", [])
    state = {"on": False, "id": 0}
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: state["on"])
    monkeypatch.setattr(H, "capture_id", lambda stream: state["id"])
    T = _lib.NM_TICKET_BYTES

    a = H.workspace_for(dev, 1000, 11)  # eager, stream 11
    assert a.numel() >= H._MIN_WORKSPACE and not a.any()
    assert H.workspace_for(dev, 1000, 11) is a
    state.update(on=True, id=5)  # capture 5 on stream 22, which has no workspace of its own
    with pytest.warns(RuntimeWarning, match="warmed-up workspace"):
        c = H.workspace_for(dev, 1000, 22)
    assert c is not a and not c[:T].any()
    assert H.workspace_for(dev, 1000, 22) is c  # reused within the capture
    big = H.workspace_for(dev, H._MIN_WORKSPACE + 64, 22)  # grows; the first stays referenced
    assert big is not c and big.numel() >= H._MIN_WORKSPACE + 64 and not big[:T].any()
    assert [t is u for t, u in zip(H._capture_workspaces[(None, 5)], (c, big))] == [True, True]
    assert H.workspace_for(dev, 1000, 11) is a  # a capture on stream 11 uses its warmed workspace
    state.update(id=6)  # a second capture on stream 22: a workspace of its own
    with pytest.warns(RuntimeWarning, match="warmed-up workspace"):
        d = H.workspace_for(dev, 1000, 22)
    assert d is not c and d is not big
    state.update(on=False, id=0)  # captures over: their pools own their workspaces
    e = H.workspace_for(dev, 1000, 22)
    assert not H._capture_workspaces and all(e is not t for t in (a, c, big, d))
    assert H._workspaces[(None, 22)] is e and not e.any()
    grown = H.workspace_for(dev, 2 * H._MIN_WORKSPACE, 11)  # eager growth retires the old one
    assert grown is not a and H._retired[-1] is a and not grown.any()
