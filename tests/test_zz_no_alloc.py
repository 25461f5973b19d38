"""nm_gemv_launch_static, the entry point that allocates nothing: its counters and
split-K partials live in the library's static device scratch. Its outputs must
equal nm_gemv_launch's (same kernels, same plans) bit for bit, call after call
on the shared scratch, the second call smaller than the first; the plain GEMV
is also checked against the float64 oracle (max-abs 1e-2, rel-L2 1e-3), and a
split-K carry producer / consumer pair runs through it as through the
workspace entry point."""
import ctypes

import pytest
import torch

from conftest import say
from oracle import nm_oracle as O
from spmv_decode_amd import _lib

pytestmark = pytest.mark.gpu


def _case(K, h, nnz, m, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    mi = torch.rand(K // m, m, generator=g, device="cuda").argsort(1)[:, :nnz].sort(1).values.to(torch.uint8)
    md = (torch.randn(K // m * nnz, h, generator=g, device="cuda") * 0.02).half()
    return md, mi.contiguous()


def _desc(vec, mats, outs, nnz, m, *, gate_up=False, norm=None):
    d = _lib.NmGemvLaunchDesc()
    d.dtype, d.kind = _lib.NM_DTYPE_F16, (_lib.NM_KIND_GATE_UP if gate_up else _lib.NM_KIND_GROUPED)
    d.nprob, d.vec_stride, d.vec = len(mats), 1, vec.data_ptr()
    d.w, d.nnz, d.m, d.config_id, d.splits = mats[0][0].shape[0], nnz, m, -1, 0
    if norm is not None:
        d.norm_weight, d.norm_eps = norm.data_ptr(), 1e-5
    for i, (md, mi) in enumerate(mats):
        d.prob[i].mat_data, d.prob[i].mat_index, d.prob[i].h = md.data_ptr(), mi.data_ptr(), md.shape[1]
    for i, o in enumerate(outs):
        d.prob[i].out = o.data_ptr()
    return d


def test_static_entry_outputs(gpu):
    """Bitwise equality with nm_gemv_launch on consecutive calls of decreasing size,
    oracle parity for the plain GEMV, and the pair once more at the end."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(1, 4096, generator=g, device="cuda").half()
    ln = (torch.rand(4096, generator=g, device="cuda") + 0.5).half()
    gate, up = _case(4096, 14336, 32, 64, 1), _case(4096, 14336, 32, 64, 2)
    xs = torch.randn(1, 1024, generator=g, device="cuda").half()
    small = _case(1024, 3072, 2, 4, 3)
    qkv = [_case(4096, h, 32, 64, 10 + i) for i, h in enumerate((4096, 1024, 1024))]

    def launch_pair():
        o_ref, o_st = (torch.full((1, 14336), float("nan"), dtype=torch.float16, device="cuda") for _ in range(2))
        return (_desc(x, [gate, up], [o_ref], 32, 64, gate_up=True, norm=ln), [o_ref]), \
               (_desc(x, [gate, up], [o_st], 32, 64, gate_up=True, norm=ln), [o_st])

    def launch_plain():
        o_ref, o_st = (torch.full((1, 3072), float("nan"), dtype=torch.float16, device="cuda") for _ in range(2))
        return (_desc(xs, [small], [o_ref], 2, 4), [o_ref]), (_desc(xs, [small], [o_st], 2, 4), [o_st])

    def launch_grouped():
        outs = [[torch.full((1, md.shape[1]), float("nan"), dtype=torch.float16, device="cuda") for md, _ in qkv]
                for _ in range(2)]
        return (_desc(x, qkv, outs[0], 32, 64), outs[0]), (_desc(x, qkv, outs[1], 32, 64), outs[1])

    for tag, make in (("gate/up pair + norm", launch_pair), ("plain 1024->3072 2:4", launch_plain),
                      ("grouped q/k/v", launch_grouped), ("gate/up pair + norm again", launch_pair)):
        say(f"static scratch: {tag}")
        (d_ref, o_ref), (d_st, o_st) = make()
        need = lib.nm_gemv_launch_workspace_bytes(ctypes.byref(d_ref))
        assert 0 < need <= _lib.NM_STATIC_SCRATCH_BYTES, (tag, need)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        _lib.check(lib.nm_gemv_launch(ctypes.byref(d_ref), ws.data_ptr(), need, stream), "nm_gemv_launch")
        _lib.check(lib.nm_gemv_launch_static(ctypes.byref(d_st), stream), "nm_gemv_launch_static")
        torch.cuda.synchronize()
        for a, b in zip(o_ref, o_st):
            assert torch.isfinite(a.float()).all(), tag
            assert torch.equal(a, b), tag
        if tag.startswith("plain"):
            ref = O.gemv_f64(xs.cpu(), small[0].cpu(), small[1].cpu(), 2, 4)
            e = O.error_metrics(ref, o_st[0].float().cpu().numpy().reshape(-1))
            assert e["max_abs"] <= 1e-2 and e["rel_l2"] <= 1e-3, e
        assert not ws[: _lib.NM_TICKET_BYTES].any()


def test_static_entry_rejects_what_does_not_fit(gpu):
    """A launch whose plan needs more than the static scratch is refused before
    anything runs (here a 128256-row GEMV forced to 40 splits)."""
    lib = _lib.load()
    md, mi = _case(16384, 128256, 32, 64, 4)
    x = torch.randn(1, 16384, device="cuda").half()
    o = torch.zeros(1, 128256, dtype=torch.float16, device="cuda")
    d = _desc(x, [(md, mi)], [o], 32, 64)
    d.splits = 40
    assert lib.nm_gemv_launch_workspace_bytes(ctypes.byref(d)) > _lib.NM_STATIC_SCRATCH_BYTES
    rc = lib.nm_gemv_launch_static(ctypes.byref(d), torch.cuda.current_stream().cuda_stream)
    assert rc == -9 and "static scratch" in _lib.strerror(rc)
    torch.cuda.synchronize()
    assert not o.any()


def test_static_entry_carried_chain(gpu):
    """o_proj as a split-K carry producer, then the gate/up pair finishing its
    input from the partials, both through the static scratch: the finished
    vector and the pair's output equal the workspace entry point's bit for bit
    (the consumer's per-workgroup norm slots live in the scratch too)."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(9)
    y = torch.randn(1, 4096, generator=g, device="cuda").half()
    x = torch.randn(1, 4096, generator=g, device="cuda").half()
    ln = (torch.rand(4096, generator=g, device="cuda") + 0.5).half()
    o = _case(4096, 4096, 32, 64, 21)
    gate, up = _case(4096, 14336, 32, 64, 22), _case(4096, 14336, 32, 64, 23)
    results = []
    for static in (False, True):
        say(f"carried chain through the {'static scratch' if static else 'workspace entry point'}")
        prod = _desc(y, [o], [], 32, 64)
        prod.carry_out = 16  # a producer's plan is asked for with carry_out set (only its presence is read)
        splits = ctypes.c_int()
        _lib.check(lib.nm_gemv_launch_plan(ctypes.byref(prod), None, ctypes.byref(splits), None, None, None), "plan")
        carry = torch.full((splits.value, 4096), float("nan"), device="cuda")
        prod.carry_out = carry.data_ptr()
        h = torch.full((1, 4096), float("nan"), dtype=torch.float16, device="cuda")
        act = torch.full((1, 14336), float("nan"), dtype=torch.float16, device="cuda")
        cons = _desc(x, [gate, up], [act], 32, 64, gate_up=True, norm=ln)
        cons.carry_in, cons.carry_splits, cons.vec_out = carry.data_ptr(), splits.value, h.data_ptr()
        for d in (prod, cons):
            if static:
                _lib.check(lib.nm_gemv_launch_static(ctypes.byref(d), stream), "nm_gemv_launch_static")
            else:
                need = lib.nm_gemv_launch_workspace_bytes(ctypes.byref(d))
                assert 0 < need <= _lib.NM_STATIC_SCRATCH_BYTES
                ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
                _lib.check(lib.nm_gemv_launch(ctypes.byref(d), ws.data_ptr(), need, stream), "nm_gemv_launch")
                torch.cuda.synchronize()
                assert not ws[: _lib.NM_TICKET_BYTES].any()
        torch.cuda.synchronize()
        assert torch.isfinite(h.float()).all() and torch.isfinite(act.float()).all()
        results.append((h, act))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
