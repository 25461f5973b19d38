"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (dropped term,
wrong index or sign, transposed operand, wrong rounding) fails at least one:
golden vectors written from the reference itself, exhaustive conversion
checks against IEEE library routines, closed-form KATs and brute force.
"""
import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import nm_oracle as O

# ---------------------------------------------------------------------------
# _make_sparse restatement vs the reference's own output (golden fixtures)
# ---------------------------------------------------------------------------
MS = json.loads((GOLDEN / "make_sparse.json").read_text())
MS_ARR = np.load(GOLDEN / "make_sparse_small.npz")


@pytest.mark.parametrize("case", MS["small"], ids=lambda c: c["tag"])
def test_make_sparse_small_bit_exact(case):
    md, mi, w, nnz = O.make_sparse(case["K"], case["N"], case["M"], case["seed"])
    assert (w, nnz) == (case["w"], case["nnz"])
    got_bits = md.view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got_bits, MS_ARR[f"{case['tag']}_mat_data_bits"])
    np.testing.assert_array_equal(mi.numpy(), MS_ARR[f"{case['tag']}_mat_index"])


@pytest.mark.parametrize("case", MS["digests"], ids=lambda c: f"K{c['K']}_N{c['N']}_M{c['M']}_s{c['seed']}")
def test_make_sparse_large_digest(case):
    import hashlib

    md, mi, w, nnz = O.make_sparse(case["K"], case["N"], case["M"], case["seed"])
    assert (w, nnz) == (case["w"], case["nnz"])
    assert mi[:4].tolist() == case["mat_index_first_rows"]
    assert md.view(torch.int16)[0, :8].numpy().view(np.uint16).tolist() == case["mat_data_first"]
    assert hashlib.sha256(mi.numpy().tobytes()).hexdigest() == case["mat_index_sha256"]
    assert hashlib.sha256(md.view(torch.int16).numpy().tobytes()).hexdigest() == case["mat_data_sha256"]


def test_fixture_torch_version_matches():
    # The RNG stream is only pinned for the torch version that wrote the fixtures.
    assert MS["meta"]["torch"].split("+")[0] == torch.__version__.split("+")[0]


def test_make_sparse_index_invariants():
    for K, M in ((4096, 4), (4096, 64), (14336, 256), (1024, 8)):
        _, mi, w, nnz = O.make_sparse(K, 128, M, 3)
        a = mi.numpy().astype(int)
        assert a.shape == (K // M, M // 2) and mi.dtype == torch.uint8
        assert (a >= 0).all() and (a < M).all()
        assert (np.diff(a, axis=1) > 0).all()  # strictly increasing => distinct


# ---------------------------------------------------------------------------
# C oracle conversions vs IEEE library conversions
# ---------------------------------------------------------------------------
def test_c_f16_to_f32_exhaustive():
    lib = O.c_oracle()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.nm_oracle_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f32_probe_values():
    rng = np.random.default_rng(0)
    vals = [rng.standard_normal(20000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1.0, 1e3, 6e4)]
    # exact ties and neighbours around every fp16 spacing, subnormal edges, overflow edges
    halfs = np.arange(0, 0x7c00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(0, 0x7c00, 7, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    mids = ((halfs + nxt) / 2).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e38, np.inf, -np.inf,
                      2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 2.0 ** -14,
                      2.0 ** -14 * (1 - 2.0 ** -11)], dtype=np.float32)
    allv = np.concatenate(vals + [mids, np.nextafter(mids, np.float32(np.inf)),
                                  np.nextafter(mids, np.float32(-np.inf)), edges])
    return np.concatenate([allv, -allv])


def test_c_f32_to_f16_matches_numpy():
    lib = O.c_oracle()
    x = _f32_probe_values()
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([lib.nm_oracle_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(ref[i])) for i in bad[:5]]
    assert lib.nm_oracle_f32_to_f16(float("nan")) & 0x7c00 == 0x7c00


def test_c_bf16_conversions_match_torch():
    lib = O.c_oracle()
    x = torch.from_numpy(_f32_probe_values())
    ref = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([lib.nm_oracle_f32_to_bf16(float(v)) for v in x.numpy()], dtype=np.uint16)
    np.testing.assert_array_equal(got, ref)
    bits = np.arange(0, 65536, 13, dtype=np.uint16)
    back = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    got_back = np.array([lib.nm_oracle_bf16_to_f32(int(b)) for b in bits], dtype=np.float32)
    ok = ~np.isnan(back)
    np.testing.assert_array_equal(got_back[ok].view(np.uint32), back[ok].view(np.uint32))


# ---------------------------------------------------------------------------
# GEMV closed forms
# ---------------------------------------------------------------------------
def _case(K, h, nnz, m, seed=0, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    banks = K // m
    mi = torch.stack([torch.randperm(m, generator=g)[:nnz].sort().values for _ in range(banks)]).to(torch.uint8)
    md = (torch.randn(banks * nnz, h, generator=g) * 0.02).to(dtype)
    x = torch.randn(K, generator=g).to(dtype)
    return x, md, mi


@pytest.mark.parametrize("nnz,m", [(2, 4), (1, 4), (3, 4), (4, 8), (32, 64), (128, 256)])
def test_one_hot_kat_reproduces_packed_rows(nnz, m):
    K, h = 4 * m, 256
    _, md, mi = _case(K, h, nnz, m, seed=nnz * m)
    pos = O.gather_positions(mi, nnz, m)
    for c in (0, 1, len(pos) // 2, len(pos) - 1):
        x = torch.zeros(K, dtype=torch.float16)
        x[pos[c]] = 1.0
        np.testing.assert_array_equal(O.gemv_f64(x, md, mi, nnz, m), md[c].double().numpy())
        acc, out = O.gemv_c(x, md, mi, nnz, m)
        np.testing.assert_array_equal(acc.numpy(), md[c].float().numpy())
        assert torch.equal(out, md[c])
    kept = set(pos.tolist())
    pruned = next(k for k in range(K) if k not in kept)
    x = torch.zeros(K, dtype=torch.float16)
    x[pruned] = 3.0
    assert not O.gemv_f64(x, md, mi, nnz, m).any()
    assert not O.gemv_c(x, md, mi, nnz, m)[0].any()


def test_zero_and_linearity_powers_of_two():
    x, md, mi = _case(256, 384, 2, 4, seed=1)
    assert not O.gemv_c(torch.zeros_like(x), md, mi, 2, 4)[0].any()
    acc1, _ = O.gemv_c(x, md, mi, 2, 4)
    for s in (2.0, 0.25, -4.0):
        acc_s, _ = O.gemv_c((x.float() * s).half(), md, mi, 2, 4)
        np.testing.assert_array_equal(acc_s.numpy(), (acc1 * s).numpy())


def test_group_permutation_invariance():
    K, h, nnz, m = 512, 128, 4, 8
    x, md, mi = _case(K, h, nnz, m, seed=2)
    perm = torch.randperm(K // m, generator=torch.Generator().manual_seed(9))
    x_p = x.view(K // m, m)[perm].reshape(-1)
    md_p = md.view(K // m, nnz, h)[perm].reshape(-1, h)
    mi_p = mi[perm]
    np.testing.assert_allclose(O.gemv_f64(x_p, md_p, mi_p, nnz, m), O.gemv_f64(x, md, mi, nnz, m), rtol=0, atol=1e-12)


def test_brute_force_all_2of4_patterns():
    """Every pair of 2:4 patterns on K=8 vs an independently built masked dense matvec."""
    import itertools

    h = 128
    rng = np.random.default_rng(5)
    dense = rng.standard_normal((h, 8)).astype(np.float32).astype(np.float16)
    x = rng.standard_normal(8).astype(np.float16)
    pats = list(itertools.combinations(range(4), 2))
    for p0, p1 in itertools.product(pats, pats):
        mi = torch.tensor([p0, p1], dtype=torch.uint8)
        keep = [p0[0], p0[1], 4 + p1[0], 4 + p1[1]]
        md = np.stack([dense[:, k] for k in keep])  # [w=4, h]
        masked = np.zeros_like(dense)
        masked[:, keep] = dense[:, keep]
        ref = masked.astype(np.float64) @ x.astype(np.float64)
        np.testing.assert_allclose(O.gemv_f64(x, md, mi, 2, 4), ref, rtol=0, atol=1e-12)
        np.testing.assert_allclose(O.gemv_c(torch.from_numpy(x), torch.from_numpy(md), mi, 2, 4)[0].numpy(),
                                   ref, rtol=1e-6, atol=1e-6)


def test_planted_index_mistake_is_caught(monkeypatch):
    """A wrong position formula in the oracle fails the one-hot KAT."""
    K, h, nnz, m = 64, 128, 2, 4
    _, md, mi = _case(K, h, nnz, m, seed=3)
    good = O.gather_positions(mi, nnz, m)
    monkeypatch.setattr(O, "gather_positions", lambda mi_, n_, m_: (np.arange(good.size) // n_) * n_ + O._flat_index(mi_))
    x = torch.zeros(K, dtype=torch.float16)
    x[good[-1]] = 1.0
    assert not np.array_equal(O.gemv_f64(x, md, mi, nnz, m), md[-1].double().numpy())


def test_c_oracle_agrees_with_f64_and_dense_reference():
    for K, h, nnz, m, dt in ((1024, 3072, 2, 4, torch.float16), (4096, 1024, 32, 64, torch.float16),
                             (1024, 512, 8, 16, torch.bfloat16), (512, 256, 4, 8, torch.float32)):
        x, md, mi = _case(K, h, nnz, m, seed=K + h, dtype=dt)
        ref = O.gemv_f64(x, md, mi, nnz, m)
        acc, out = O.gemv_c(x, md, mi, nnz, m)
        np.testing.assert_allclose(acc.numpy(), ref, rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(out.float().numpy(), acc.to(dt).float().numpy())
        dense = O.gemv_fp32_dense(x, md, mi, nnz, m)
        np.testing.assert_allclose(dense.numpy(), ref, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(O.gemv_gather_torch(x, md, mi, nnz, m).numpy(), ref, rtol=1e-5, atol=1e-5)
    x, md, mi = _case(1024, 3072, 2, 4, seed=11)
    acc, out = O.gemv_c(x, md, mi, 2, 4)
    acc2, out2 = O.gemv_c_fast_f16(x, md, mi, 2, 4)
    assert torch.equal(acc, acc2) and torch.equal(out, out2)


def test_out_of_range_position_contributes_zero():
    # idx = M-1 in the last group with a vec shortened by one element
    K, h, nnz, m = 16, 128, 2, 4
    x, md, mi = _case(K, h, nnz, m, seed=4)
    mi[-1] = torch.tensor([0, 3], dtype=torch.uint8)
    xs = x[:-1]
    y = O.gemv_f64(xs, md, mi, nnz, m)
    md2 = md.clone()
    md2[-1] = 0
    np.testing.assert_allclose(y, O.gemv_f64(x, md2, mi, nnz, m), rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# Packing and metrics
# ---------------------------------------------------------------------------
def test_scatter_pack_round_trips():
    K, h, nnz, m = 512, 256, 8, 16
    x, md, mi = _case(K, h, nnz, m, seed=6)
    dense = O.scatter(md, mi, nnz, m, K)
    assert dense.shape == (h, K)
    np.testing.assert_array_equal(O.pack(dense, mi, nnz, m), md.numpy())
    mask = O.mask_from_index(mi, nnz, m, K)
    assert mask.sum() == K // 2
    W = np.random.default_rng(1).standard_normal((h, K)).astype(np.float16)
    Wm = W * mask[None, :]
    np.testing.assert_array_equal(O.scatter(O.pack(Wm, mi, nnz, m), mi, nnz, m, K), Wm)
    # dense masked matvec == packed gemv
    np.testing.assert_allclose(Wm.astype(np.float64) @ x.double().numpy(),
                               O.gemv_f64(x, O.pack(Wm, mi, nnz, m), mi, nnz, m), rtol=0, atol=1e-12)


def test_error_metrics_hand_values():
    ref = np.array([3.0, -4.0, 0.0, 0.0])
    out = np.array([3.0, -4.0, 1.0, -1.0])
    e = O.error_metrics(ref, out)
    assert e["max_abs"] == 1.0 and e["mean_abs"] == 0.5
    assert abs(e["rmse"] - np.sqrt(0.5)) < 1e-15
    assert abs(e["rel_l2"] - np.sqrt(2.0) / 5.0) < 1e-15
    assert O.error_metrics(np.zeros(3), np.ones(3))["rel_l2"] == pytest.approx(np.sqrt(3) / 1e-12)


# ---------------------------------------------------------------------------
# Decode-layer operations around the GEMV (fused prologue / epilogues)
# ---------------------------------------------------------------------------
def test_rms_norm_matches_library_and_closed_form():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 320, generator=g, dtype=torch.float64)
    wt = torch.randn(320, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.rms_norm(x, (320,), wt, 1e-5).numpy()
    np.testing.assert_allclose(O.rms_norm_f64(x, wt, 1e-5), ref, rtol=1e-13, atol=0)
    # constant input c: every element becomes c / sqrt(c^2 + eps) * weight
    c, eps = 3.0, 0.25
    out = O.rms_norm_f64(np.full(64, c), np.arange(64.0), eps)
    np.testing.assert_allclose(out, c / np.sqrt(c * c + eps) * np.arange(64.0), rtol=1e-15)


def test_rope_matches_complex_multiply_and_invariants():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((5, 128))
    ang = rng.uniform(-7, 7, 64)
    got = O.rope_f64(v, ang)
    z = (v[:, 0::2] + 1j * v[:, 1::2]) * np.exp(1j * ang)
    np.testing.assert_allclose(got[:, 0::2], z.real, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(got[:, 1::2], z.imag, rtol=1e-13, atol=1e-13)
    np.testing.assert_array_equal(O.rope_f64(v, np.zeros(64)), v)            # position 0: identity
    pair_norm = np.hypot(v[:, 0::2], v[:, 1::2])
    np.testing.assert_allclose(np.hypot(got[:, 0::2], got[:, 1::2]), pair_norm, rtol=1e-13)
    # a quarter turn maps (a, b) to (-b, a); pairs, not halves, are rotated
    q = O.rope_f64(np.array([1.0, 2.0, 3.0, 4.0]), np.full(2, np.pi / 2))
    np.testing.assert_allclose(q, [-2.0, 1.0, -4.0, 3.0], atol=1e-15)


def test_silu_matches_library():
    g = torch.linspace(-30, 30, 1001, dtype=torch.float64)
    np.testing.assert_allclose(O.silu_f64(g.numpy()), torch.nn.functional.silu(g).numpy(), rtol=1e-14, atol=1e-300)


def test_qkv_decode_composes_norms_gemv_and_rope():
    """qkv_decode_f64 against the same steps written out with torch float64
    library calls (dense masked weights, F.rms_norm, complex rotation)."""
    K, hd, nnz, m = 256, 64, 2, 4
    x, qd, qi = _case(K, 2 * hd, nnz, m, seed=11)
    _, kd, ki = _case(K, hd, nnz, m, seed=12)
    _, vd, vi = _case(K, hd, nnz, m, seed=13)
    g = torch.Generator().manual_seed(14)
    lnw = torch.rand(K, generator=g, dtype=torch.float64) + 0.5
    qn = torch.rand(hd, generator=g, dtype=torch.float64) + 0.5
    kn = torch.rand(hd, generator=g, dtype=torch.float64) + 0.5
    ang = np.linspace(0.1, 3.0, hd // 2)
    q, k, v = O.qkv_decode_f64(x, (qd, qi), (kd, ki), (vd, vi), nnz, m, angle_row=ang, head_dim=hd,
                               norm=(lnw, 1e-5), q_norm=qn, k_norm=kn, eps=1e-6)
    xn = torch.nn.functional.rms_norm(torch.from_numpy(O.to_f64(x)).reshape(1, K), (K,), lnw, 1e-5).reshape(-1)

    def lin(md, mi):
        dense = O.scatter(torch.from_numpy(O.to_f64(md)), mi, nnz, m, K)
        return dense @ xn

    def rot(t):
        z = torch.view_as_complex(t.reshape(*t.shape[:-1], -1, 2).contiguous()) * torch.polar(
            torch.ones(hd // 2, dtype=torch.float64), torch.from_numpy(ang))
        return torch.view_as_real(z).flatten(-2)

    rq = rot(torch.nn.functional.rms_norm(lin(qd, qi).reshape(2, hd), (hd,), qn, 1e-6))
    rk = rot(torch.nn.functional.rms_norm(lin(kd, ki).reshape(1, hd), (hd,), kn, 1e-6))
    np.testing.assert_allclose(q, rq.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(k, rk.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(v, lin(vd, vi).reshape(1, hd).numpy(), rtol=1e-11, atol=1e-12)


def test_spmm_rows_match_gemv_and_dense_matmul():
    x0, md, mi = _case(256, 384, 3, 4, seed=21)
    g = torch.Generator().manual_seed(22)
    X = torch.randn(5, 256, generator=g).to(torch.float16)
    got = O.spmm_f64(X, md, mi, 3, 4)
    dense = O.scatter(torch.from_numpy(O.to_f64(md)), mi, 3, 4, 256)  # [h, K] float64
    np.testing.assert_allclose(got, (torch.from_numpy(O.to_f64(X)) @ dense.T).numpy(), rtol=1e-12, atol=1e-12)
    for b in range(5):
        np.testing.assert_array_equal(got[b], O.gemv_f64(X[b], md, mi, 3, 4))
