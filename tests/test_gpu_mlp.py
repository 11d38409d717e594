"""GPU parity of the MLP pieces against the oracle, bit-exact:

* xt_activation_mul for every activation variant (ReLU^2, silu_inplace's
  AVX-512 polynomial and scalar paths, silu_mul_inplace), on special values
  and on a sweep of 2^24 float bit patterns (exp of the C library reproduced);
* xt_rms_norm on rows built to stress the exact sequential f32 sum of squares
  (ties on the summation grid, tiny leading elements, many binades, overflow
  to inf, subnormals, NaN / inf inputs) and at model sizes;
* xt_ternary_mlp_q (fused_mlp_all per row) and xt_ternary_mlp_f32
  (Mlp::forward: fused for one token, unfused for several) against
  oracle.mlp_forward, i8 mid activations, inverse scales and f32 outputs
  all bit-identical (tolerance rel 1e-5 / abs 1e-4 asserted as well).
"""
import zlib

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
f32 = np.float32


def log(msg):
    print(f"[case] {msg}", flush=True)


def same_bits(a, b):
    """Bit equality, any NaN equal to any NaN."""
    a, b = np.asarray(a, f32), np.asarray(b, f32)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), f"NaN positions differ ({np.sum(na != nb)})"
    diff = a[~na].view(np.int32) != b[~nb].view(np.int32)
    assert not diff.any(), f"{diff.sum()} of {a.size} values differ"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def specials(rng, shape):
    x = (rng.standard_normal(shape) * 4).astype(f32)
    sp = np.array([0.0, -0.0, 1.0, -1.0, 88.0, -88.0, 88.37, -88.37, 88.5, -88.5, 100.0, -100.0,
                   1e-30, -1e-30, 1e-45, -1e-45, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38,
                   87.3, -103.9, -104.0, 0.5, -0.5], f32)
    flat = x.reshape(-1)
    k = min(sp.size, flat.size)
    flat[:k] = sp[:k]
    return x


ACTS = [(xtern.XT_ACT_RELU2_MUL, "relu2"), (xtern.XT_ACT_SILU_INPLACE_AVX512, "silu_avx512"),
        (xtern.XT_ACT_SILU_INPLACE_SCALAR, "silu_scalar"), (xtern.XT_ACT_SILU_MUL, "silu_mul")]


def oracle_act(act, g, u):
    if act == xtern.XT_ACT_RELU2_MUL:
        return oracle.silu_inplace(g, u, False)
    if act == xtern.XT_ACT_SILU_INPLACE_AVX512:
        return oracle.silu_inplace(g, u, True, avx512=True)
    if act == xtern.XT_ACT_SILU_INPLACE_SCALAR:
        return oracle.silu_inplace(g, u, True, avx512=False)
    return oracle.act_mul(g, u, True)


@pytest.mark.parametrize("act,name", ACTS)
@pytest.mark.parametrize("M,n", [(1, 1), (3, 17), (2, 6912), (4, 8640), (1, 16384), (5, 333)])
def test_activation_matches_oracle(act, name, M, n):
    log(f"activation {name} M={M} n={n}")
    rng = np.random.default_rng(zlib.crc32(f"{name}{M}{n}".encode()))
    g, u = specials(rng, (M, n)), rng.standard_normal((M, n)).astype(f32)
    got = xtern.activation_mul(act, dev(g), dev(u)).cpu().numpy()
    same_bits(got, oracle_act(act, g, u))


@pytest.mark.parametrize("act,name", ACTS[1:])
def test_activation_bit_pattern_sweep(act, name):
    """2^24 inputs spread over all 2^32 float bit patterns (stride 256, with a
    per-variant offset), up = 1: covers every exponent and the exp special
    ranges."""
    log(f"activation sweep {name}")
    off = {1: 17, 2: 101, 3: 211}[act]
    bits = (np.arange(1 << 24, dtype=np.uint64) * 256 + off).astype(np.uint32)
    g = bits.view(f32).reshape(1024, 16384)
    u = np.ones_like(g)
    got = xtern.activation_mul(act, dev(g), dev(u)).cpu().numpy()
    same_bits(got, oracle_act(act, g, u))


def norm_rows(rng, n):
    """Rows that exercise the exact sequential sum."""
    rows = {}
    rows["normal"] = rng.standard_normal(n).astype(f32)
    rows["wide"] = (rng.standard_normal(n) * np.exp(rng.standard_normal(n) * 6)).astype(f32)
    t = rng.standard_normal(n).astype(f32)
    t[0] = 1e-30
    rows["tiny_first"] = t
    rows["ties"] = (rng.integers(-8, 9, n) * 0.5).astype(f32)        # few mantissa bits
    rows["ones"] = np.ones(n, f32)
    rows["thirds"] = np.full(n, 1 / 3, f32)
    rows["growing"] = np.sqrt(np.arange(1, n + 1, dtype=np.float64)).astype(f32)
    rows["decay"] = (np.exp(-np.arange(n) / max(n / 40, 1)) * 1e3).astype(f32)
    rows["zeros"] = np.zeros(n, f32)
    rows["subnormal"] = (rng.standard_normal(n) * 1e-22).astype(f32)
    big = rng.standard_normal(n).astype(f32) * f32(1e18)
    rows["overflow"] = big                                          # squares sum past f32 max
    rows["huge_one"] = np.where(np.arange(n) == n // 2, f32(1e19), f32(1.0)).astype(f32)
    rows["inf"] = np.where(np.arange(n) == n // 3, f32(np.inf), f32(1.0)).astype(f32)
    rows["nan"] = np.where(np.arange(n) == n - 1, f32(np.nan), f32(1.0)).astype(f32)
    rows["alternating"] = np.where(np.arange(n) % 2 == 0, f32(1e4), f32(1e-3)).astype(f32)
    return rows


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 64, 65, 100, 1000, 2560, 3200, 6912, 8640,
                               14336, 16384])
def test_rms_norm_matches_oracle(n):
    log(f"rms_norm n={n}")
    rng = np.random.default_rng(n)
    rows = norm_rows(rng, n)
    names = list(rows)
    x = np.stack([rows[k] for k in names])
    w = (1 + rng.standard_normal(n) * 0.1).astype(f32)
    got = xtern.rms_norm(dev(x), dev(w), 1e-6).cpu().numpy()
    want, _ = oracle.rms_norm(x, w, 1e-6)
    for r, name in enumerate(names):
        try:
            same_bits(got[r], want[r])
        except AssertionError as e:
            raise AssertionError(f"row '{name}': {e}") from None


def test_rms_norm_random_stress():
    """Many random rows of random lengths and scales."""
    log("rms_norm stress")
    rng = np.random.default_rng(99)
    for n in (4096, 6912, 5504):
        x = (rng.standard_normal((64, n)) * np.exp(rng.standard_normal((64, 1)) * 8) *
             np.exp(rng.standard_normal((64, n)))).astype(f32)
        x[::7, :5] *= f32(1e-12)
        w = np.ones(n, f32)
        got = xtern.rms_norm(dev(x), dev(w), 1e-5).cpu().numpy()
        same_bits(got, oracle.rms_norm(x, w, 1e-5)[0])


def test_reference_rmsnorm_kat_on_gpu():
    # tests/tensor_ops_tests.rs:318-340 inputs
    for n in [1, 3, 7, 8, 9, 15, 16, 17, 31, 32, 33, 64, 100, 128, 256, 3200]:
        x = (np.arange(n, dtype=f32) * f32(0.1) - f32(n / 2)).astype(f32)
        w = (f32(1) + np.arange(n, dtype=f32) * f32(0.01)).astype(f32)
        got = xtern.rms_norm(dev(x[None]), dev(w), 1e-6).cpu().numpy()[0]
        same_bits(got, oracle.rms_norm(x, w, 1e-6)[0])


# ------------------------------------------------------------------ MLP ---

def make_lin(rng, fmt, K, N, scale):
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[0.33, 0.34, 0.33])
    ws = np.full(N, scale, f32)
    if fmt == xtern.XT_XORSPARSE:
        blob = xtern.encode_sparse_tensor(t, K, N)[0]
        masks, signs, _ = oracle.sparse_from_blob(blob, N, K)
        lin = xtern.DeviceWeights(fmt, K, N, np.frombuffer(blob, np.uint8), ws)
        return lin, (2, K, N, ws, dict(masks=masks, signs=signs))
    pack = xtern.pack_ternary4 if fmt == xtern.XT_PACK4 else xtern.pack_ternary5
    wb = np.concatenate([pack(r) for r in t])
    return xtern.DeviceWeights(fmt, K, N, wb, ws), (fmt, K, N, ws, dict(wbytes=wb))


MLP_CASES = [
    # fmt, hidden, inter, use_silu, norm, M
    (xtern.XT_PACK4, 2560, 6912, False, True, 1),     # BitNet-2B block (config 4)
    (xtern.XT_PACK4, 2560, 6912, False, True, 8),
    (xtern.XT_PACK4, 2560, 6912, False, True, 32),
    (xtern.XT_PACK5, 3200, 8640, True, False, 1),     # 3B-class SiLU block (config 2)
    (xtern.XT_PACK5, 3200, 8640, True, False, 8),
    (xtern.XT_PACK4, 256, 333, True, True, 3),        # ragged intermediate size
    (xtern.XT_XORSPARSE, 640, 1000, False, True, 2),
    (xtern.XT_PACK4, 2560, 6912, True, True, 64),     # prefill GEMM path
]


@pytest.mark.parametrize("fmt,H,I,silu,norm,M", MLP_CASES)
@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
def test_mlp_matches_oracle(fmt, H, I, silu, norm, M, mode):
    log(f"mlp fmt={fmt} H={H} I={I} silu={silu} norm={norm} M={M} mode={mode}")
    rng = np.random.default_rng(zlib.crc32(f"{fmt}{H}{I}{silu}{norm}{M}{mode}".encode()))
    gl, go = make_lin(rng, fmt, H, I, 0.8)
    ul, uo = make_lin(rng, fmt, H, I, 0.6)
    dl, do = make_lin(rng, fmt, I, H, 0.9)
    nw = (1 + rng.standard_normal(I) * 0.2).astype(f32) if norm else None
    x = rng.standard_normal((M, H)).astype(f32)
    x[:, :3] *= 20
    nwd = dev(nw) if norm else None
    # Mlp::forward semantics
    y = xtern.mlp_f32(gl, ul, dl, dev(x), norm_w=nwd, eps=1e-5, use_silu=silu,
                      mode=mode).cpu().numpy()
    y_ref, _, _ = oracle.mlp_forward(x, go, uo, do, nw, 1e-5, silu, quant_mode=mode)
    assert np.allclose(y, y_ref, rtol=1e-5, atol=1e-4)
    same_bits(y, y_ref)
    # fused_mlp_all on every row, from the quantised input
    q, inv = xtern.quantize_i8(dev(x), mode=mode)
    yq = xtern.mlp_q(gl, ul, dl, q, inv, norm_w=nwd, eps=1e-5, use_silu=silu,
                     mode=mode).cpu().numpy()
    yq_ref, _, _ = oracle.mlp_forward(x, go, uo, do, nw, 1e-5, silu, quant_mode=mode, fused=True)
    same_bits(yq, yq_ref)


def test_mlp_layer_mirror_and_errors():
    log("Mlp mirror")
    rng = np.random.default_rng(11)
    H, I = 512, 1024
    w = lambda k, n: rng.integers(-1, 2, size=(n, k)).astype(f32).ravel()
    P4 = xtern.TernaryPackType.Pack4
    g = xtern.TernaryLinear.new(H, I, w(H, I), P4)
    u = xtern.TernaryLinear.new(H, I, w(H, I), P4)
    d = xtern.TernaryLinear.new(I, H, w(I, H), P4)
    norm = xtern.FastRmsNorm(dev((1 + rng.standard_normal(I) * 0.1).astype(f32)), 1e-5)
    mlp = xtern.Mlp(g, u, d, norm, "relu2")
    x = dev(rng.standard_normal((1, 1, H)).astype(f32))
    y = mlp.forward(x)
    assert tuple(y.shape) == (1, 1, H)
    q, inv = xtern.quantize_i8(x.reshape(1, H))
    y2 = xtern.TernaryLinear.fused_mlp_all(x, q, inv, g, u, d, norm, False)
    same_bits(y.cpu().numpy(), y2.cpu().numpy())
    # unfused pieces give the same result: forward, relu2, norm, forward
    gg, uu = g.forward(x), u.forward(x)
    mid = xtern.activation_mul(xtern.XT_ACT_RELU2_MUL, gg, uu)
    same_bits(d.forward(norm.forward(mid)).cpu().numpy(), y.cpu().numpy())
    assert mlp.weight_bytes() == 3 * I * H // 4
    with pytest.raises(xtern.XternError, match="Input dimension mismatch"):
        mlp.forward(dev(np.zeros((1, H + 1), f32)))
    with pytest.raises(xtern.XternError, match="down in_dim"):
        xtern.mlp_f32(g.weights, u.weights, g.weights, x.reshape(1, H))
    # empty batch
    assert xtern.mlp_f32(g.weights, u.weights, d.weights,
                         dev(np.zeros((0, H), f32))).shape == (0, H)
