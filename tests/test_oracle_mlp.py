"""Pins of the oracle's MLP pieces (oracle/xtern_oracle.c or_silu_inplace,
or_act_mul_inplace, or_rms_norm) by means independent of the oracle code:

* the C library's expf called directly through ctypes, with the rest of the
  scalar SiLU formulas evaluated in numpy float32 (IEEE ops, one rounding
  each, in the reference's order);
* numpy float32 closed forms for ReLU^2;
* numpy's sequential float32 accumulate (np.cumsum) for rms_norm's sum of
  squares, which the reference's own naive check also uses
  (tests/tensor_ops_tests.rs:318-340: `iter().map(|v| v * v).sum()`);
* for the AVX-512 polynomial SiLU (quantization.rs:243-272): agreement with
  float64 silu within the polynomial's error (a dropped or wrong Taylor term
  exceeds it), exact special values, and the scalar tail for n % 16 lanes;
* the reference's own known inputs (tests/tensor_ops_tests.rs:47-99,
  tests/tensor_arithmetic_tests.rs).
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.argtypes = [ctypes.c_float]
_libm.expf.restype = ctypes.c_float


def libm_expf(a):
    return np.array([_libm.expf(float(v)) for v in np.asarray(a, np.float32).ravel()],
                    np.float32).reshape(np.shape(a))


f32 = np.float32


def special_values(rng, n):
    base = rng.standard_normal(n).astype(f32) * f32(4)
    sp = np.array([0.0, -0.0, 1.0, -1.0, 88.0, -88.0, 88.5, -88.5, 100.0, -100.0, 1e-30,
                   -1e-30, 1e-45, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38], f32)
    base[:sp.size] = sp
    return base


def test_relu2_closed_form():
    rng = np.random.default_rng(1)
    g, u = special_values(rng, 1000), rng.standard_normal(1000).astype(f32)
    r = np.where(g > 0, g, f32(0)).astype(f32)
    with np.errstate(all="ignore"):
        want = (r * r).astype(f32) * u
    for avx in (0, 1):
        got = oracle.silu_inplace(g, u, False, avx512=bool(avx))
        assert np.array_equal(got.view(np.int32), want.astype(f32).view(np.int32)) or \
            np.array_equal(np.isnan(got), np.isnan(want)) and \
            np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    got = oracle.act_mul(g, u, False)
    assert np.array_equal(np.nan_to_num(got, nan=7.0), np.nan_to_num(want, nan=7.0))


def test_scalar_silu_formulas_use_libm_expf():
    rng = np.random.default_rng(2)
    g, u = special_values(rng, 3000), rng.standard_normal(3000).astype(f32)
    e = libm_expf(-g)
    with np.errstate(all="ignore"):
        sig = (f32(1) / (f32(1) + e)).astype(f32)
        want_inplace = ((g * sig).astype(f32) * u).astype(f32)
        want_div = ((g / (f32(1) + e)).astype(f32) * u).astype(f32)
    got = oracle.silu_inplace(g, u, True, avx512=False)
    np.testing.assert_array_equal(got, want_inplace)
    np.testing.assert_array_equal(oracle.act_mul(g, u, True), want_div)


def test_avx512_silu_polynomial():
    rng = np.random.default_rng(3)
    n = 4096 + 7  # 7 tail lanes
    g = (rng.standard_normal(n) * 6).astype(f32)
    u = np.ones(n, f32)
    got = oracle.silu_inplace(g, u, True, avx512=True)
    gd = g.astype(np.float64)
    exact = gd / (1.0 + np.exp(-gd))
    rel = np.abs(got - exact) / np.maximum(np.abs(exact), 1e-30)
    # 4th-order Taylor of exp on |t| <= ln2/2: remainder t^5/120 <= 4.2e-5
    # relative (a dropped t^4 term would give ~6e-4), plus f32 rounding.
    assert rel[:4096].max() < 1e-4, rel.max()
    assert rel[:4096].max() > 1e-5  # it is the polynomial, not libm
    # tail lanes take the scalar (libm) formula
    tail = oracle.silu_inplace(g[4096:], u[4096:], True, avx512=False)
    np.testing.assert_array_equal(got[4096:], tail)
    # special values: silu(0) = 0, large positive -> g, large negative -> ~0
    sp = np.array([0.0, 50.0, -50.0, 100.0, -100.0, np.nan] + [0.0] * 10, f32)
    r = oracle.silu_inplace(sp, np.ones(16, f32), True, avx512=True)
    assert r[0] == 0 and r[1] == f32(50) and r[3] == f32(100)
    assert abs(r[2]) < 1e-19 and abs(r[4]) < 1e-35 and np.isnan(r[5])


def test_reference_silu_mul_kat():
    # tests/tensor_ops_tests.rs:48-67 and tests/tensor_arithmetic_tests.rs:15,47-62
    a = np.array([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 3.0], f32)
    b = np.array([1.5, 2.5, -0.5, 0.1, 10.0, 4.0, 0.0, -3.0], f32)
    want = a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64))) * b
    assert np.allclose(oracle.act_mul(a, b, True), want, atol=1e-6)
    assert np.all(oracle.act_mul(np.zeros(3, f32), np.ones(3, f32), True) == 0)


def seq_rms_norm(x, w, eps):
    sq = (x * x).astype(f32)
    s = np.cumsum(sq, dtype=f32)[-1]
    rms = np.sqrt(f32(s / f32(x.size) + f32(eps)), dtype=f32)
    inv = f32(1) / rms
    return ((x * inv).astype(f32) * w).astype(f32), s


@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 15, 16, 17, 31, 32, 33, 64, 100, 128, 256, 3200,
                               6912])
def test_rms_norm_is_sequential(n):
    # inputs of tests/tensor_ops_tests.rs:318-322, then random ones
    x = (np.arange(n, dtype=f32) * f32(0.1) - f32(n / 2)).astype(f32)
    w = (f32(1) + np.arange(n, dtype=f32) * f32(0.01)).astype(f32)
    for xs in (x, np.random.default_rng(n).standard_normal(n).astype(f32)):
        want, s = seq_rms_norm(xs, w, 1e-6)
        got, sums = oracle.rms_norm(xs, w, 1e-6)
        np.testing.assert_array_equal(got, want)
        assert sums[0] == s


def test_rms_norm_order_matters():
    # A row whose pairwise and sequential f32 sums differ: the oracle must give
    # the sequential one.
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = (rng.standard_normal(777) * np.exp(rng.standard_normal(777) * 3)).astype(f32)
        sq = (x * x).astype(f32)
        seq = np.cumsum(sq, dtype=f32)[-1]
        if seq != np.sum(sq, dtype=f32):
            break
    else:
        pytest.skip("no differing row found")
    _, sums = oracle.rms_norm(x, np.ones(777, f32), 1e-5)
    assert sums[0] == seq


def test_reference_rmsnorm_kat():
    # tests/tensor_ops_tests.rs:70-99 (hidden 4, eps 1e-6)
    data = np.array([1.0, 2.0, 3.0, 4.0, -1.0, 0.5, 1.5, -2.0, 0.0, 0.0, 0.0, 1.0,
                     2.0, -2.0, 2.0, -2.0, 1.1, 2.2, 3.3, 4.4, -0.5, -0.5, -0.5, -0.5],
                    f32).reshape(6, 4)
    w = np.array([0.5, 1.0, 1.5, 2.0], f32)
    got, _ = oracle.rms_norm(data, w, 1e-6)
    d = data.astype(np.float64)
    want = d / np.sqrt((d * d).mean(-1, keepdims=True) + 1e-6) * w
    assert np.allclose(got, want, atol=1e-5)


def test_mlp_forward_dispatch():
    """Mlp::forward: one token = fused_mlp_all, several = unfused; with ReLU^2
    the two paths are the same computation, with SiLU they differ only by the
    activation formula (bounded by the polynomial's error after
    requantisation)."""
    rng = np.random.default_rng(7)
    K, I, N = 256, 320, 128

    def lin(k, n):
        t = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
        wb = np.concatenate([oracle.pack4(r.astype(f32), 1.0) for r in t])
        return (0, k, n, np.full(n, 0.5, f32), dict(wbytes=wb))

    g, u, d = lin(K, I), lin(K, I), lin(I, N)
    x = rng.standard_normal((3, K)).astype(f32)
    nw = (1 + rng.standard_normal(I) * 0.1).astype(f32)
    for silu in (False, True):
        rows = [oracle.mlp_forward(x[i:i + 1], g, u, d, nw, 1e-5, silu)[0] for i in range(3)]
        batch = oracle.mlp_forward(x, g, u, d, nw, 1e-5, silu)[0]
        fused = oracle.mlp_forward(x, g, u, d, nw, 1e-5, silu, fused=True)[0]
        np.testing.assert_array_equal(np.concatenate(rows), fused)
        if not silu:
            np.testing.assert_array_equal(batch, fused)
        else:
            assert np.allclose(batch, fused, rtol=0.05, atol=0.05)
