"""Pins the CPU oracle (oracle/xtern_oracle.c) before it is trusted as the
checker: the reference's own known-answer tests (tests/golden/reference_kats.json),
hand-derived values, brute force on unpacked weights, and invariants chosen so
that a dropped term, a wrong sign/index or a wrong rounding mode fails."""
import itertools
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")
KATS = json.load(open(GOLDEN))


# ---------------------------------------------------------------- codecs ---

def test_pack4_hand_values():
    # code table 00=-1 01=0 10=+1, weight j in bits 2j (quantization.rs:7-27)
    assert oracle.pack4([-1, 0, 1, -1]).tolist() == [0b00_10_01_00]
    assert oracle.pack4([1, 1, 1, 1]).tolist() == [0b10_10_10_10]
    assert oracle.pack4([0]).tolist() == [0b01]          # short group: high bits stay 0
    assert oracle.pack4([0, 0, 0, 0, -1]).tolist() == [0x55, 0x00]


def test_pack5_hand_values():
    # first weight = least-significant trit, digits 0=-1 1=0 2=+1
    assert oracle.pack5([-1, 0, 1, -1, 1]).tolist() == [0 + 1 * 3 + 2 * 9 + 0 * 27 + 2 * 81]
    assert oracle.pack5([1, 1, 1, 1, 1]).tolist() == [242]
    assert oracle.pack5([0, 1]).tolist() == [1 + 2 * 3]


def test_unpack4_all_bytes():
    # every byte value, including the never-packed code 11 (reads as 0)
    b = np.arange(256, dtype=np.uint8)
    u = oracle.unpack4(b, 1024).reshape(256, 4)
    for v in range(256):
        for j in range(4):
            code = (v >> (2 * j)) & 3
            assert u[v, j] == {0: -1.0, 1: 0.0, 2: 1.0, 3: 0.0}[code]


def test_codecs_bijective_on_ternary():
    for t in itertools.product([-1.0, 0.0, 1.0], repeat=4):
        assert oracle.unpack4(oracle.pack4(t), 4).tolist() == list(t)
    vals = set()
    for t in itertools.product([-1.0, 0.0, 1.0], repeat=5):
        p = oracle.pack5(t)
        vals.add(int(p[0]))
        assert oracle.unpack5(p, 5).tolist() == list(t)
    assert vals == set(range(243))


@pytest.mark.parametrize("kat", KATS["roundtrip"], ids=lambda k: k["src"])
def test_roundtrip_kats(kat):
    w = np.array(kat["w"], np.float32)
    assert oracle.unpack4(oracle.pack4(w), w.size).tolist() == w.tolist()
    assert oracle.unpack5(oracle.pack5(w), w.size).tolist() == w.tolist()


@pytest.mark.parametrize("n", [1, 2, 3, 5, 6, 7, 9, 11, 13, 15, 17, 21])
def test_roundtrip_unaligned(n):
    # quantization_158bit_tests.rs:30-38 and :70-77
    w = np.array([[-1.0, 0.0, 1.0][i % 3] for i in range(n)], np.float32)
    assert oracle.unpack4(oracle.pack4(w), n).tolist() == w.tolist()
    assert oracle.unpack5(oracle.pack5(w), n).tolist() == w.tolist()


def test_pack_scale_semantics():
    # w / scale rounded half away from zero then clamped: 0.5 -> 1, -0.5 -> -1,
    # 0.49 -> 0; a scale above 2 zeroes ternary input (layers.rs:100-108 quirk)
    assert oracle.unpack4(oracle.pack4([0.5, -0.5, 0.49, 7.0], 1.0), 4).tolist() == [1, -1, 0, 1]
    assert oracle.unpack4(oracle.pack4([1.0, -1.0], 2.5), 2).tolist() == [0, 0]
    assert oracle.unpack4(oracle.pack4([1.0, -1.0], 0.0), 2).tolist() == [0, 0]


# ------------------------------------------------------------- quantiser ---

@pytest.mark.parametrize("kat", KATS["quantize"], ids=lambda k: k["src"])
@pytest.mark.parametrize("mode", [0, 1])
def test_quantize_kats(kat, mode):
    q, inv = oracle.quantize(kat["x"], mode)
    if "q" in kat:
        assert q.tolist() == kat["q"]
    for i, v in kat.get("q_at", {}).items():
        assert q[int(i)] == v
    assert abs(float(inv) - kat["inv"]) <= kat["inv_tol"]


def test_quantize_reconstruction_bound():
    # quantization_158bit_tests.rs:104-121
    x = np.array([(i - 128.0) * 0.01 for i in range(256)], np.float32)
    for mode in (0, 1):
        q, inv = oracle.quantize(x, mode)
        assert np.all(np.abs(x - q.astype(np.float32) * inv) <= inv + 1e-6)


def test_quantize_rounding_modes_on_ties():
    # max |x| = 127 -> scale = 1.0, so x*scale hits exact .5 ties.
    # AVX-512 path: lanes < floor(n/16)*16 round half-to-even, the tail half
    # away from zero; scalar path: half away everywhere.
    x = np.zeros(20, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3] = 2.5, -2.5, 3.5
    x[17], x[18], x[19] = 2.5, -2.5, 0.5
    qa, inva = oracle.quantize(x, 0)
    qs, invs = oracle.quantize(x, 1)
    assert inva == invs == np.float32(1.0)
    assert qa[[1, 2, 3]].tolist() == [2, -2, 4]
    assert qa[[17, 18, 19]].tolist() == [3, -3, 1]
    assert qs[[1, 2, 3, 17, 18, 19]].tolist() == [3, -3, 4, 3, -3, 1]


def test_quantize_invariants_random():
    rng = np.random.default_rng(0)
    for n in (1, 15, 16, 17, 2560, 6913):
        x = rng.standard_normal(n).astype(np.float32) * 3
        for mode in (0, 1):
            q, inv = oracle.quantize(x, mode)
            am = int(np.argmax(np.abs(x)))
            assert abs(int(q[am])) == 127 and np.sign(q[am]) == np.sign(x[am])
            assert np.all(np.abs(q.astype(int)) <= 127)
            assert inv == np.float32(np.abs(x).max()) / np.float32(127.0)
            # within half a step of x/inv, except ties
            err = np.abs(x * (np.float32(127.0) / np.abs(x).max()) - q)
            assert np.all(err <= 0.5 + 1e-5)


def test_quantize_modes_agree_off_ties():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4096).astype(np.float32)
    qa, ia = oracle.quantize(x, 0)
    qs, is_ = oracle.quantize(x, 1)
    assert ia == is_
    scaled = x * (np.float32(127.0) / np.abs(x).max())
    ties = np.abs(scaled - np.trunc(scaled)) == 0.5
    assert np.array_equal(qa[~ties], qs[~ties])


# ----------------------------------------------------------------- dots ----

def _brute(a, t):
    return int(np.dot(np.asarray(a, np.int64), np.asarray(t, np.int64)))


@pytest.mark.parametrize("kat", KATS["dot"], ids=lambda k: k["src"])
def test_dot_kats(kat):
    a, w, n = kat["a"], np.array(kat["w"], np.float32), len(kat["a"])
    if kat["fmt"] == "pack4":
        assert oracle.dot_pack4(a, oracle.pack4(w), n) == kat["dot"]
    else:
        assert oracle.dot_pack5(a, oracle.pack5(w), n) == kat["dot"]


@pytest.mark.parametrize("n", [4, 8, 12, 16, 20, 32, 36, 64, 68, 128, 132, 200, 1000, 2560])
def test_dot_cross_path_and_brute(n):
    # bit1_58_tests.rs:37-66 (scalar = SIMD = Pack5) plus brute force
    a = np.array([(i % 255) - 127 for i in range(n)], np.int8)
    t = np.array([[-1, 0, 1][i % 3] for i in range(n)], np.int8)
    ref = _brute(a, t)
    p4, p5 = oracle.pack4(t.astype(np.float32)), oracle.pack5(t.astype(np.float32))
    assert oracle.dot_pack4(a, p4, n) == ref
    assert oracle.dot_pack5(a, p5, n) == ref
    if oracle.has_vnni():
        assert oracle.dot_pack4_vnni(a, p4, n) == ref


@pytest.mark.parametrize("n", [20, 40, 60, 100, 200])
def test_pack4_vs_pack5_wrapping_acts(n):
    # simd_dot_product_tests.rs:67-82: acts ((i*7+13) % 255) as i8 (wraps)
    a = np.array([((i * 7 + 13) % 255) for i in range(n)], np.int64).astype(np.uint8).view(np.int8)
    t = np.array([[-1, 0, 1][i % 3] for i in range(n)], np.float32)
    assert oracle.dot_pack4(a, oracle.pack4(t), n) == oracle.dot_pack5(a, oracle.pack5(t), n) \
        == _brute(a, t)


def test_dot_code11_reads_zero():
    a = np.arange(1, 5, dtype=np.int8)
    assert oracle.dot_pack4(a, np.array([0xFF], np.uint8), 4) == 0
    if oracle.has_vnni():
        a64 = np.ones(64, np.int8)
        assert oracle.dot_pack4_vnni(a64, np.full(16, 0xFF, np.uint8), 64) == 0


@pytest.mark.skipif(not oracle.has_vnni(), reason="host has no AVX-512 VNNI")
def test_vnni_matches_scalar_random():
    rng = np.random.default_rng(2)
    for n in (64, 1024, 1088, 2560, 6912, 6913):
        a = rng.integers(-127, 128, n).astype(np.int8)
        t = rng.integers(-1, 2, n).astype(np.float32)
        p = oracle.pack4(t)
        assert oracle.dot_pack4_vnni(a, p, n) == oracle.dot_pack4(a, p, n) == _brute(a, t)


@pytest.mark.skipif(not oracle.has_vnni(), reason="host has no AVX-512 VNNI")
def test_vnni_minus128_quirk():
    # simd.rs:297: sa = 0 - a in i8, so a = -128 against w = -1 contributes
    # -128 on the VNNI path (+128 on the scalar path).  Off-contract input:
    # the quantiser never emits -128.
    a = np.zeros(64, np.int8)
    a[5] = -128
    t = np.zeros(64, np.float32)
    t[5] = -1
    p = oracle.pack4(t)
    assert oracle.dot_pack4(a, p, 64) == 128
    assert oracle.dot_pack4_vnni(a, p, 64) == -128


# --------------------------------------------------------------- sparse ----

def test_sparse_encode_hand_value():
    row = np.zeros(64, np.int8)
    row[0], row[2] = 1, -1
    blob = oracle.sparse_encode_row(row, 64)
    assert blob == bytes([1, 0, 0, 0]) + bytes([5, 0, 0, 0, 0, 0, 0, 0]) + bytes([2])
    row70 = np.zeros(70, np.int8)
    row70[69] = -1
    blob = oracle.sparse_encode_row(row70, 70)
    assert blob == (bytes([2, 0, 0, 0]) + bytes(8) + bytes([32, 0, 0, 0, 0, 0, 0, 0]) + bytes([1]))


def _lcg_dense(rng, in_dim, out_dim):
    # simd.rs:567-575
    return np.array([[-1, 0, 1][rng.below(3)] for _ in range(in_dim * out_dim)], np.int8)


def test_lcg_matches_formula():
    seed = KATS["lcg"]["seed"]
    r = oracle.Lcg(seed)
    x = seed
    for _ in range(5):
        x = (x * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        assert r.next() == x >> 33


@pytest.mark.parametrize("shape", [(256, 48), (2560, 16), (100, 20), (64, 3)])
def test_sparse_roundtrip_and_dot(shape):
    # simd.rs:581-625 / :667-682, at sizes that run quickly in the oracle
    in_dim, out_dim = shape
    rng = oracle.Lcg(0x1234_5678_9abc_def0)
    w = _lcg_dense(rng, in_dim, out_dim).reshape(out_dim, in_dim)
    act = np.array([rng.below(7) - 3 for _ in range(in_dim)], np.int8)
    blob, offs = oracle.sparse_encode_tensor(w, in_dim, out_dim)
    masks, signs, nb = oracle.sparse_from_blob(blob, out_dim, in_dim)
    assert nb == (in_dim + 63) // 64
    p4 = np.concatenate([oracle.pack4(w[r].astype(np.float32)) for r in range(out_dim)])
    bpr = (in_dim + 3) // 4
    for r in range(out_dim):
        assert oracle.sparse_decode_row(blob, offs[r], in_dim).tolist() == w[r].tolist()
        d = oracle.dot_sparse(act, masks[r], signs[r], nb, in_dim)
        assert d == oracle.dot_pack4(act, p4[r * bpr:(r + 1) * bpr], in_dim) == _brute(act, w[r])
        # lane-order signs only where the mask is set, and only for -1 lanes
        for b in range(nb):
            for lane in range(64):
                k = b * 64 + lane
                m, s = (int(masks[r, b]) >> lane) & 1, (int(signs[r, b]) >> lane) & 1
                val = w[r, k] if k < in_dim else 0
                assert m == (val != 0) and s == (val < 0)


def test_sparse_avx_block_case():
    # simd.rs:627-665: a = (i % 5) - 2, mask 0xAAAA..., set-order sign bit for
    # the non-zeros at lanes k % 3 == 0
    a = np.array([(i % 5) - 2 for i in range(64)], np.int8)
    t = np.zeros(64, np.int8)
    for k in range(64):
        if k % 2 == 1:
            t[k] = -1 if k % 3 == 0 else 1
    blob = oracle.sparse_encode_row(t, 64)
    masks, signs, nb = oracle.sparse_from_blob(blob, 1, 64)
    assert int(masks[0, 0]) == 0xAAAA_AAAA_AAAA_AAAA
    assert oracle.dot_sparse(a, masks[0], signs[0], 1, 64) == _brute(a, t)


def test_sparse_truncated_blob():
    blob = oracle.sparse_encode_row(np.ones(64, np.int8), 64)
    with pytest.raises(ValueError):
        oracle.sparse_from_blob(blob[:-1], 1, 64)


# --------------------------------------------------------------- linear ----

@pytest.mark.parametrize("kat", KATS["linear"], ids=lambda k: k["src"])
def test_linear_kats(kat):
    K, N = kat["in_dim"], kat["out_dim"]
    w = np.array(kat["weights"], np.float32).reshape(N, K)
    for fmt, pack in ((0, oracle.pack4), (1, oracle.pack5)):
        wb = np.concatenate([pack(w[o]) for o in range(N)])
        y, q, inv, acc = oracle.linear_forward(fmt, K, N, kat["x"], np.ones(N, np.float32), wb)
        assert np.allclose(y[0], kat["y"], atol=kat["tol"], rtol=0)


def test_linear_formula_order_and_threads():
    rng = np.random.default_rng(3)
    K, N = 320, 300
    t = rng.integers(-1, 2, (N, K)).astype(np.float32)
    wb = np.concatenate([oracle.pack4(t[o]) for o in range(N)])
    ws = rng.uniform(0.5, 2.0, N).astype(np.float32)
    x = rng.standard_normal((3, K)).astype(np.float32)
    y1, q1, inv1, acc1 = oracle.linear_forward(0, K, N, x, ws, wb, threads=1)
    y8, q8, inv8, acc8 = oracle.linear_forward(0, K, N, x, ws, wb, threads=8,
                                               kernel=1 if oracle.has_vnni() else 0)
    assert np.array_equal(y1, y8) and np.array_equal(acc1, acc8)
    for m in range(3):
        qm, im = oracle.quantize(x[m], 0)
        assert np.array_equal(q1[m], qm) and inv1[m] == im
        dots = (t.astype(np.int64) @ qm.astype(np.int64))
        assert np.array_equal(acc1[m], dots)
        # (f32(dot) * inv) * w_scale, each product rounded to f32
        expect = (dots.astype(np.float32) * np.float32(im)).astype(np.float32) * ws
        assert np.array_equal(y1[m], expect.astype(np.float32))
    # M == 1 path equals row 0 of the batched path
    y0, _, _, _ = oracle.linear_forward(0, K, N, x[:1], ws, wb)
    assert np.array_equal(y0[0], y1[0])


def test_linear_q_matches_forward():
    rng = np.random.default_rng(4)
    K, N = 200, 40
    t = rng.integers(-1, 2, (N, K)).astype(np.float32)
    wb = np.concatenate([oracle.pack5(t[o]) for o in range(N)])
    ws = np.full(N, 0.8, np.float32)
    x = rng.standard_normal((2, K)).astype(np.float32)
    y, q, inv, acc = oracle.linear_forward(1, K, N, x, ws, wb)
    y2, acc2 = oracle.linear_forward_q(1, K, N, q, inv, ws, wb)
    assert np.array_equal(y, y2) and np.array_equal(acc, acc2)


def test_golden_fixture_consistent():
    """The committed fixture's dots equal brute force over the decoded weights,
    and its outputs follow the reference epilogue."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "seeded_small.npz"),
                allow_pickle=False)
    for name in sorted({k.split("__")[0] for k in g.files}):
        fmt, K, N = (int(v) for v in g[name + "__meta"])
        wb = g[name + "__wbytes"]
        if fmt == 2:
            blob = wb.tobytes()
            offs = [0]
            for r in range(N - 1):
                offs.append(offs[-1] + len(oracle.sparse_encode_row(
                    oracle.sparse_decode_row(blob, offs[-1], K), K)))
            t = np.stack([oracle.sparse_decode_row(blob, offs[r], K) for r in range(N)])
        else:
            bpr = (K + 3) // 4 if fmt == 0 else (K + 4) // 5
            un = oracle.unpack4 if fmt == 0 else oracle.unpack5
            t = np.stack([un(wb[r * bpr:(r + 1) * bpr], K) for r in range(N)]).astype(np.int8)
        q, inv, acc, y = g[name + "__q"], g[name + "__inv"], g[name + "__acc"], g[name + "__y"]
        for m in range(q.shape[0]):
            qo, io = oracle.quantize(g[name + "__x"][m])
            assert np.array_equal(q[m], qo) and inv[m] == io
        assert np.array_equal(acc, q.astype(np.int64) @ t.astype(np.int64).T)
        ws = g[name + "__ws"]
        assert np.array_equal(y, (acc.astype(np.float32) * inv[:, None]).astype(np.float32)
                              * ws[None, :])
