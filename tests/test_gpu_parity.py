"""GPU parity of libxtern (HIP, gfx950) against the CPU oracle.

Bar: i8 activations and inv_scale bit-exact, i32 accumulators bit-exact,
f32 outputs bit-exact (the epilogue (f32)dot * inv * w_scale is the same two
IEEE multiplies on both sides); the stated tolerance rel 1e-5 / abs 1e-4 is
asserted as well so a failure reports both.  Full BASELINE sizes are checked
against an exact float64 matmul of the unpacked ternary weights (integers
below 2^53, so the float64 product is exact)."""
import zlib

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_REL, TOL_ABS = 1e-5, 1e-4


def log(msg):
    print(f"[case] {msg}", flush=True)


def tern(rng, N, K, p0=0.35):
    p = (1 - p0) / 2
    return rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[p, p0, p])


def make_bytes(t, fmt):
    N, K = t.shape
    if fmt == xtern.XT_PACK4:
        return np.concatenate([xtern.pack_ternary4(r) for r in t])
    if fmt == xtern.XT_PACK5:
        return np.concatenate([xtern.pack_ternary5(r) for r in t])
    return np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)


def oracle_q(fmt, t, q, inv, ws):
    """Oracle forward_with_quantized over the reference layout of `fmt`."""
    N, K = t.shape
    if fmt == xtern.XT_XORSPARSE:
        blob = xtern.encode_sparse_tensor(t, K, N)[0]
        masks, signs, _ = oracle.sparse_from_blob(blob, N, K)
        return oracle.linear_forward_q(2, K, N, q, inv, ws, masks=masks, signs=signs)
    return oracle.linear_forward_q(fmt, K, N, q, inv, ws, wbytes=make_bytes(t, fmt))


def exact_acc(t, q):
    return (q.astype(np.float64) @ t.astype(np.float64).T).astype(np.int64)


def check_y(y, y_ref):
    assert np.allclose(y, y_ref, rtol=TOL_REL, atol=TOL_ABS)
    assert np.array_equal(y.view(np.int32), y_ref.view(np.int32)), \
        f"{np.sum(y != y_ref)} f32 outputs differ in bits"


FMTS = [xtern.XT_PACK4, xtern.XT_PACK5, xtern.XT_XORSPARSE]
FMT_ID = {xtern.XT_PACK4: "pack4", xtern.XT_PACK5: "pack5", xtern.XT_XORSPARSE: "sparse"}


# ---------------------------------------------------------------- quantiser ---

@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
@pytest.mark.parametrize("M,K", [(1, 1), (2, 4), (1, 8), (1, 15), (2, 16), (3, 17), (1, 2560), (5, 6912),
                                 (128, 2560), (4, 14336), (2, 3203)])
def test_quantize_exact(M, K, mode):
    log(f"quantize M={M} K={K} mode={mode}")
    rng = np.random.default_rng(M * 1000 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    out = rng.random((M, K)) < 0.01
    x[out] *= 20
    if M > 1:
        x[1] = 0.0                                   # all-zero row -> inv 1.0
    if K >= 20:                                      # exact .5 ties in body and tail
        x[0, :] = np.round(x[0, :] * 4) / 4
        x[0, 0] = 127.0 / 4
    q, inv = xtern.quantize_i8(torch.from_numpy(x).to(DEV), mode=mode)
    q, inv = q.cpu().numpy(), inv.cpu().numpy()
    for m in range(M):
        qo, io = oracle.quantize(x[m], mode)
        assert np.array_equal(q[m], qo), f"row {m}: {np.sum(q[m] != qo)} i8 mismatches"
        assert inv[m].view(np.int32) == np.float32(io).view(np.int32)


# ------------------------------------------------------- product vs oracle ---

@pytest.mark.parametrize("fmt", FMTS, ids=FMT_ID.get)
@pytest.mark.parametrize("K,N,M", [(256, 16, 1), (300, 37, 3), (64, 1, 1), (5, 3, 2),
                                   (2560, 96, 16), (1000, 50, 17), (640, 64, 40),
                                   (1281, 33, 128), (320, 16, 5), (4000, 48, 20),
                                   (7168, 80, 33)])
def test_linear_q_matches_oracle(fmt, K, N, M):
    log(f"linear_q fmt={FMT_ID[fmt]} K={K} N={N} M={M}")
    rng = np.random.default_rng(K + 7 * N + 13 * M + fmt)
    t = tern(rng, N, K)
    ws = rng.uniform(0.2, 2.0, N).astype(np.float32)
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    inv = rng.uniform(1e-3, 0.1, M).astype(np.float32)
    w = xtern.DeviceWeights(fmt, K, N, make_bytes(t, fmt), ws)
    y, acc = xtern.linear_q(w, torch.from_numpy(q).to(DEV), torch.from_numpy(inv).to(DEV),
                            acc=True)
    y, acc = y.cpu().numpy(), acc.cpu().numpy()
    y_ref, acc_ref = oracle_q(fmt, t, q, inv, ws)
    assert np.array_equal(acc, acc_ref), f"{np.sum(acc != acc_ref)} i32 mismatches"
    check_y(y, y_ref)


@pytest.mark.parametrize("fmt", FMTS, ids=FMT_ID.get)
@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
@pytest.mark.parametrize("K,N,M", [(2560, 128, 1), (333, 40, 4), (6912, 32, 20), (64, 17, 33)])
def test_linear_f32_matches_oracle(fmt, mode, K, N, M):
    log(f"linear_f32 fmt={FMT_ID[fmt]} mode={mode} K={K} N={N} M={M}")
    rng = np.random.default_rng(K + N + M + 31 * fmt + mode)
    t = tern(rng, N, K)
    ws = np.full(N, 0.8, np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = xtern.DeviceWeights(fmt, K, N, make_bytes(t, fmt), ws)
    y = xtern.linear_f32(w, torch.from_numpy(x).to(DEV), mode=mode).cpu().numpy()
    if fmt == xtern.XT_XORSPARSE:
        masks, signs, _ = oracle.sparse_from_blob(make_bytes(t, fmt), N, K)
        y_ref, _, _, _ = oracle.linear_forward(2, K, N, x, ws, masks=masks, signs=signs,
                                               quant_mode=mode)
    else:
        y_ref, _, _, _ = oracle.linear_forward(fmt, K, N, x, ws, wbytes=make_bytes(t, fmt),
                                               quant_mode=mode)
    check_y(y, y_ref)


def test_golden_fixtures():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "seeded_small.npz")
    g = np.load(path, allow_pickle=False)
    for name in sorted({k.split("__")[0] for k in g.files}):
        log(f"golden {name}")
        fmt, K, N = (int(v) for v in g[name + "__meta"])
        w = xtern.DeviceWeights(fmt, K, N, g[name + "__wbytes"], g[name + "__ws"])
        x = torch.from_numpy(g[name + "__x"]).to(DEV)
        q, inv = xtern.quantize_i8(x)
        assert np.array_equal(q.cpu().numpy(), g[name + "__q"])
        assert np.array_equal(inv.cpu().numpy(), g[name + "__inv"])
        y, acc = xtern.linear_q(w, q, inv, acc=True)
        assert np.array_equal(acc.cpu().numpy(), g[name + "__acc"])
        check_y(y.cpu().numpy(), g[name + "__y"])
        check_y(xtern.linear_f32(w, x).cpu().numpy(), g[name + "__y"])


# ---------------------------------------------------------- full-size configs ---

CONFIGS = [
    ("c0_pack4_gemv", xtern.XT_PACK4, 2560, 6912, [1], 0.35),
    ("c1_pack4_up", xtern.XT_PACK4, 2560, 6912, [128], 0.35),
    ("c1_pack4_down", xtern.XT_PACK4, 6912, 2560, [128], 0.35),
    ("c2_pack5_up", xtern.XT_PACK5, 3200, 8640, [1, 8], 0.4),
    ("c2_pack5_down", xtern.XT_PACK5, 8640, 3200, [1, 8], 0.4),
    ("c3_sparse_up", xtern.XT_XORSPARSE, 4096, 14336, [1, 4, 16], None),
    ("c3_sparse_down", xtern.XT_XORSPARSE, 14336, 4096, [1, 4, 16], None),
]


def sparse_tern(rng, N, K):
    nb = K // 64
    zf = rng.uniform(0.3, 0.7, (N, nb, 1))
    u = rng.random((N, nb, 64))
    sign = np.where(rng.random((N, nb, 64)) < 0.5, -1, 1)
    return np.where(u < zf, 0, sign).astype(np.int8).reshape(N, K)


@pytest.mark.parametrize("name,fmt,K,N,Ms,p0", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_config_full_size(name, fmt, K, N, Ms, p0):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    t = sparse_tern(rng, N, K) if p0 is None else tern(rng, N, K, p0)
    wb = make_bytes(t, fmt)
    if fmt == xtern.XT_XORSPARSE:
        # the encoded weights are lossless w.r.t. the Pack4 encoding
        p4 = make_bytes(t, xtern.XT_PACK4)
        assert np.array_equal(xtern.repack_host(xtern.XT_XORSPARSE, K, N, wb),
                              xtern.repack_host(xtern.XT_PACK4, K, N, p4))
    ws = np.full(N, 0.8, np.float32)
    w = xtern.DeviceWeights(fmt, K, N, wb, ws)
    for M in Ms:
        log(f"{name} M={M}")
        x = rng.standard_normal((M, K)).astype(np.float32)
        x[rng.random((M, K)) < 0.01] *= 20
        xd = torch.from_numpy(x).to(DEV)
        q, inv = xtern.quantize_i8(xd)
        y, acc = xtern.linear_q(w, q, inv, acc=True)
        q, inv, y, acc = (v.cpu().numpy() for v in (q, inv, y, acc))
        for m in range(M):
            qo, io = oracle.quantize(x[m])
            assert np.array_equal(q[m], qo) and inv[m] == io
        a64 = exact_acc(t, q)
        assert np.array_equal(acc, a64)
        y_ref = ((a64.astype(np.float32) * inv[:, None]).astype(np.float32) * ws[None, :])
        check_y(y, y_ref.astype(np.float32))
        yf = xtern.linear_f32(w, xd).cpu().numpy()
        check_y(yf, y)
        # spot rows through the oracle's own dot kernels
        if fmt != xtern.XT_XORSPARSE:
            bpr = (K + 3) // 4 if fmt == xtern.XT_PACK4 else (K + 4) // 5
            dot = oracle.dot_pack4 if fmt == xtern.XT_PACK4 else oracle.dot_pack5
            for o in (0, N // 2, N - 1):
                assert dot(q[0], wb[o * bpr:(o + 1) * bpr], K) == acc[0, o]


def test_c4_stack_layer_shapes():
    """One BitNet-2B layer (q, k, v, o, gate, up, down) at M in {1, 8, 32},
    with the fused q/k/v and gate/up launches equal to separate ones."""
    rng = np.random.default_rng(44)
    shapes = {"q": (2560, 2560), "k": (2560, 640), "v": (2560, 640), "o": (2560, 2560),
              "gate": (2560, 6912), "up": (2560, 6912), "down": (6912, 2560)}
    T, W = {}, {}
    for n, (K, N) in shapes.items():
        T[n] = tern(rng, N, K)
        W[n] = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(T[n], xtern.XT_PACK4),
                                   np.full(N, 0.9, np.float32))
    for M in (1, 8, 32):
        log(f"c4 layer M={M}")
        x = torch.from_numpy(rng.standard_normal((M, 2560)).astype(np.float32)).to(DEV)
        q, inv = xtern.quantize_i8(x)
        qn = q.cpu().numpy()
        fused = xtern.linear_multi_q([W["q"], W["k"], W["v"]], q, inv)
        for n, yf in zip(("q", "k", "v"), fused):
            ys, acc = xtern.linear_q(W[n], q, inv, acc=True)
            assert np.array_equal(acc.cpu().numpy(), exact_acc(T[n], qn))
            assert torch.equal(ys, yf)
        g, u = xtern.linear_multi_f32([W["gate"], W["up"]], x)
        assert torch.equal(g, xtern.linear_f32(W["gate"], x))
        assert torch.equal(u, xtern.linear_f32(W["up"], x))
        # the f32 entry points (quantiser fused into the GEMV at M = 1) equal
        # the separate quantiser plus the product
        assert torch.equal(g, xtern.linear_q(W["gate"], q, inv))
        assert torch.equal(u, xtern.linear_q(W["up"], q, inv))
        xd = torch.from_numpy(rng.standard_normal((M, 6912)).astype(np.float32)).to(DEV)
        qd, invd = xtern.quantize_i8(xd)
        _, acc = xtern.linear_q(W["down"], qd, invd, acc=True)
        assert np.array_equal(acc.cpu().numpy(), exact_acc(T["down"], qd.cpu().numpy()))


# ------------------------------------------------------------- edge cases ---

def test_empty_batch_is_noop():
    w = xtern.DeviceWeights(xtern.XT_PACK4, 64, 16, np.zeros(16 * 16, np.uint8),
                            np.ones(16, np.float32))
    y = xtern.linear_f32(w, torch.zeros((0, 64), device=DEV))
    assert y.shape == (0, 16)


def test_unaligned_and_ragged_q_pointer():
    log("unaligned q")
    rng = np.random.default_rng(9)
    K, N, M = 300, 20, 3
    t = tern(rng, N, K)
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                            np.ones(N, np.float32))
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    buf = torch.zeros(M * K + 1, dtype=torch.int8, device=DEV)
    buf[1:] = torch.from_numpy(q.ravel()).to(DEV)
    qv = buf[1:].view(M, K)                      # 1-byte offset: not 16-byte aligned
    inv = torch.full((M,), 0.01, device=DEV)
    _, acc = xtern.linear_q(w, qv, inv, acc=True)
    assert np.array_equal(acc.cpu().numpy(), exact_acc(t, q))


def test_minus128_is_exact_integer():
    # Off-contract: the quantiser never emits -128.  The GPU gives the exact
    # integer (as the reference's scalar path), not the VNNI path's wrap.
    K, N = 64, 16
    t = np.zeros((N, K), np.int8)
    t[0, 5] = -1
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                            np.ones(N, np.float32))
    q = torch.zeros((1, K), dtype=torch.int8, device=DEV)
    q[0, 5] = -128
    _, acc = xtern.linear_q(w, q, torch.ones(1, device=DEV), acc=True)
    assert acc[0, 0].item() == 128


def test_repeat_is_deterministic():
    rng = np.random.default_rng(10)
    K, N = 2560, 6912
    t = tern(rng, N, K)
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                            np.ones(N, np.float32))
    x = torch.from_numpy(rng.standard_normal((4, K)).astype(np.float32)).to(DEV)
    y0 = xtern.linear_f32(w, x)
    for _ in range(5):
        assert torch.equal(xtern.linear_f32(w, x), y0)


# ------------------------------------------------- reference-API mirror ---

def test_ternary_linear_reference_kat():
    # tests/bit1_58_tests.rs:68-92 with the current scale semantics
    weights = [1.0, 0.0, -1.0, 1.0, 0.0, -1.0, 1.0, 0.0]
    x = torch.tensor([[0.5, 1.0, -0.5, 2.0]], device=DEV)
    l4 = xtern.TernaryLinear.new(4, 2, weights, xtern.TernaryPackType.Pack4)
    l5 = xtern.TernaryLinear.new(4, 2, weights, xtern.TernaryPackType.Pack5)
    o4, o5 = l4.forward(x).cpu().numpy(), l5.forward(x).cpu().numpy()
    assert np.array_equal(o4, o5)
    assert abs(o4[0, 0] - 3.007874) < 1e-4 and abs(o4[0, 1] + 1.511811) < 1e-4


def test_ternary_linear_shapes_and_errors():
    rng = np.random.default_rng(11)
    w = rng.standard_normal(20 * 4).astype(np.float32)
    l = xtern.TernaryLinear.new(20, 4, w, xtern.TernaryPackType.Pack4)
    x = torch.from_numpy(rng.standard_normal((2, 3, 20)).astype(np.float32)).to(DEV)
    assert l.forward(x).shape == (2, 3, 4)
    with pytest.raises(xtern.XternError, match="Input dimension mismatch"):
        l.forward(torch.zeros((1, 19), device=DEV))
    with pytest.raises(xtern.XternError, match="at least 1 dimension"):
        l.forward(torch.tensor(1.0, device=DEV))
    with pytest.raises(xtern.XternError, match="in_dim \\* out_dim"):
        xtern.TernaryLinear.new(20, 5, w, xtern.TernaryPackType.Pack4)
    # per-row mean-|w| scale (layers.rs:120-134) and the f32 path vs oracle
    y = l.forward(x[0]).cpu().numpy()
    tern4 = np.frombuffer(l.host_bytes, np.uint8) if isinstance(l.host_bytes, bytes) else l.host_bytes
    y_ref, _, _, _ = oracle.linear_forward(0, 20, 4, x[0].cpu().numpy(), l.w_scales, wbytes=tern4)
    check_y(y, y_ref)


def test_dense_vs_sparse_layers_bit_identical():
    # simd.rs:581-625 at layer level: dense Pack4 and XorSparse give the same output
    rng = oracle.Lcg(0x1234_5678_9abc_def0)
    for K, N in ((2560, 640), (640, 256)):
        w = np.array([[-1.0, 0.0, 1.0][rng.below(3)] for _ in range(K * N)], np.float32)
        dense = xtern.TernaryLinear.new(K, N, w, xtern.TernaryPackType.Pack4)
        sparse = xtern.TernaryLinear.new_sparse(K, N, w, xtern.TernaryPackType.Pack4)
        packed = xtern.TernaryLinear.new_sparse_from_packed(
            dense.host_bytes, K, N, xtern.TernaryPackType.Pack4, dense.w_scales)
        x = torch.from_numpy(np.random.default_rng(K).standard_normal((3, K))
                             .astype(np.float32)).to(DEV)
        y = dense.forward(x)
        assert torch.equal(y, sparse.forward(x)) and torch.equal(y, packed.forward(x))
        assert sparse.packed_bytes() < dense.packed_bytes() * 1.2


def test_forward_with_quantized_and_fused():
    rng = np.random.default_rng(12)
    K = 256
    lins = [xtern.TernaryLinear.new(K, n, rng.integers(-1, 2, n * K).astype(np.float32),
                                    xtern.TernaryPackType.Pack4, 0.5) for n in (64, 32, 32)]
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).to(DEV)
    q, inv = xtern.quantize_i8(x)
    qkv = xtern.TernaryLinear.fused_forward_qkv(x, q, inv, *lins)
    for l, y in zip(lins, qkv):
        assert torch.equal(y, l.forward(x))
        assert torch.equal(y, l.forward_with_quantized(x, q, float(inv[0])))
    a, b = xtern.TernaryLinear.fused_forward_mlp(x, q, inv, lins[0], lins[1])
    assert torch.equal(a, qkv[0]) and torch.equal(b, qkv[1])
    dl = xtern.DynamicLinear(lins[0])
    assert torch.equal(dl.forward(x), qkv[0])


# ------------------------------------------------------------ HIP graphs ---

@pytest.mark.parametrize("M", [1, 8, 128])
def test_graph_replay_matches_eager(M):
    """Captured linear_f32 launches (including split-K shapes, whose workspace
    the kernels clear themselves) replay to the eager result every time, with
    eager work on another stream between replays."""
    log(f"graph replay M={M}")
    rng = np.random.default_rng(20 + M)
    mats = [(2560, 640), (6912, 2560), (2560, 6912)]
    ws = [xtern.DeviceWeights(xtern.XT_PACK4, K, N,
                              make_bytes(tern(rng, N, K), xtern.XT_PACK4),
                              np.full(N, 0.7, np.float32)) for K, N in mats]
    xs = [torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(DEV)
          for K, _ in mats]
    ys = [torch.empty((M, N), device=DEV) for _, N in mats]
    eager = [xtern.linear_f32(w, x) for w, x in zip(ws, xs)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for w, x, y in zip(ws, xs, ys):
            xtern.linear_f32(w, x, out=y)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for w, x, y in zip(ws, xs, ys):
            xtern.linear_f32(w, x, out=y)
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert torch.equal(y, e), f"replay {rep} differs"
        # eager work in between, on the default stream
        assert torch.equal(xtern.linear_f32(ws[1], xs[1]), eager[1])


def test_splitk_workspace_alternating_shapes():
    """Split-K shapes of different sizes on one stream, interleaved, stay exact
    (each launch must leave the shared zeroed workspace clean)."""
    rng = np.random.default_rng(30)
    cases = [(2560, 640, 1), (6912, 2560, 128), (2560, 640, 16), (6912, 2560, 33), (4096, 160, 3)]
    prepared = []
    for K, N, M in cases:
        t = tern(rng, N, K)
        w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                                np.ones(N, np.float32))
        q = rng.integers(-127, 128, (M, K)).astype(np.int8)
        prepared.append((w, torch.from_numpy(q).to(DEV), exact_acc(t, q)))
    for rnd in range(3):
        for (K, N, M), (w, q, ref) in zip(cases, prepared):
            log(f"alternating round={rnd} K={K} N={N} M={M}")
            _, acc = xtern.linear_q(w, q, torch.ones(M, device=DEV), acc=True)
            assert np.array_equal(acc.cpu().numpy(), ref)


@pytest.mark.parametrize("cfg", ["1,1,4,4,3", "1,4,4,2,2", "2,8,4,2,4", "g32,2", "g32,3", "g32,5"])
def test_forced_splitk_configs(cfg, monkeypatch):
    """Split-K across workgroups (only taken when forced) stays exact, across
    shape changes that move the partial-sum planes."""
    monkeypatch.setenv("XTERN_CONFIG", cfg)
    rng = np.random.default_rng(40)
    for K, N, M in ((2560, 640, 1), (6912, 2560, 128), (2560, 6912, 40), (1024, 96, 16)):
        log(f"forced {cfg} K={K} N={N} M={M}")
        t = tern(rng, N, K)
        w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                                np.ones(N, np.float32))
        q = rng.integers(-127, 128, (M, K)).astype(np.int8)
        _, acc = xtern.linear_q(w, torch.from_numpy(q).to(DEV), torch.ones(M, device=DEV),
                                acc=True)
        assert np.array_equal(acc.cpu().numpy(), exact_acc(t, q))


@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", [(1, 4), (1, 16), (1, 20), (2, 100), (3, 2560), (1, 8192),
                                 (4, 2048), (1, 2561), (16, 512)])
def test_small_forward_quantiser_ties(fmt, mode, M, K):
    """Small M*K forwards quantise inside the GEMV.  Rows whose absmax is 127
    make the scale exactly 1, so x.5 values are exact ties: half-to-even in
    the AVX-512 body, half-away in its tail and in scalar mode."""
    log(f"fused quant fmt={fmt} mode={mode} M={M} K={K}")
    rng = np.random.default_rng(zlib.crc32(f"fq{fmt}{mode}{M}{K}".encode()))
    N = 40
    t = tern(rng, N, K)
    wb = make_bytes(t, fmt)
    ws = np.full(N, 0.7, np.float32)
    w = xtern.DeviceWeights(fmt, K, N, wb, ws)
    x = (rng.integers(-60, 61, size=(M, K)) + 0.5).astype(np.float32)
    x[:, 0] = 127.0
    if M > 1:
        x[1] *= np.float32(0.37)  # a row without ties
    y = xtern.linear_f32(w, torch.from_numpy(x).to(DEV), mode=mode).cpu().numpy()
    q = np.stack([oracle.quantize(x[m], mode)[0] for m in range(M)])
    inv = np.array([oracle.quantize(x[m], mode)[1] for m in range(M)], np.float32)
    check_y(y, oracle_q(fmt, t, q, inv, ws)[0])
    # multi-projection forward on the same input
    w2 = xtern.DeviceWeights(fmt, K, N, wb, ws * np.float32(2))
    ys = xtern.linear_multi_f32([w, w2], torch.from_numpy(x).to(DEV), mode=mode)
    check_y(ys[0].cpu().numpy(), y)
    check_y(ys[1].cpu().numpy(), oracle_q(fmt, t, q, inv, ws * np.float32(2))[0])


@pytest.mark.parametrize("K,N,M", [(2560, 3840, 32), (2560, 2560, 32), (2560, 6912, 24),
                                   (2560, 13824, 32), (6912, 2560, 32)])
def test_small_prefill_default_config(K, N, M):
    """Short prefills of the BitNet-2B shapes (the decode-stack config at
    M = 24 / 32), whichever kernel the default choice takes, are exact."""
    log(f"small prefill K={K} N={N} M={M}")
    rng = np.random.default_rng(K + N + M)
    t = tern(rng, N, K)
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, make_bytes(t, xtern.XT_PACK4),
                            np.ones(N, np.float32))
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    _, acc = xtern.linear_q(w, torch.from_numpy(q).to(DEV), torch.ones(M, device=DEV),
                            acc=True)
    assert np.array_equal(acc.cpu().numpy(), exact_acc(t, q))


@pytest.mark.parametrize("fmt,K,N", [(xtern.XT_PACK5, 3200, 16016), (xtern.XT_PACK4, 2560, 32784),
                                     (xtern.XT_PACK4, 4096, 14352)])
@pytest.mark.parametrize("M", [1, 3, 16])
def test_tall_decode_row_groups(fmt, K, N, M):
    """Tall matrices, where the decode GEMV runs several 16-row groups per
    workgroup (including a last workgroup with fewer groups), are exact."""
    log(f"tall decode fmt={FMT_ID[fmt]} K={K} N={N} M={M}")
    rng = np.random.default_rng(K + N + M)
    t = tern(rng, N, K)
    w = xtern.DeviceWeights(fmt, K, N, make_bytes(t, fmt), np.ones(N, np.float32))
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    _, acc = xtern.linear_q(w, torch.from_numpy(q).to(DEV), torch.ones(M, device=DEV), acc=True)
    assert np.array_equal(acc.cpu().numpy(), exact_acc(t, q))


@pytest.mark.parametrize("fmt", [xtern.XT_PACK4, xtern.XT_PACK5], ids=FMT_ID.get)
@pytest.mark.parametrize("K,N", [(6912, 2560), (8192, 300), (2600, 700), (2560, 6912), (100, 40),
                                 (8640, 3200)])
@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
def test_one_row_forward_equals_quantiser_plus_product(fmt, K, N, mode):
    """f32 forward of one row (the quantiser fused into the decode GEMV,
    several chunks per wave, K not a multiple of the chunk) gives exactly the
    separate quantiser followed by the product."""
    log(f"one-row forward fmt={FMT_ID[fmt]} K={K} N={N} mode={mode}")
    rng = np.random.default_rng(K + N + mode)
    t = tern(rng, N, K)
    w = xtern.DeviceWeights(fmt, K, N, make_bytes(t, fmt),
                            rng.uniform(0.2, 2.0, N).astype(np.float32))
    x = rng.standard_normal((1, K)).astype(np.float32)
    x[0, rng.integers(0, K, 3)] *= 40
    xd = torch.from_numpy(x).to(DEV)
    y = xtern.linear_f32(w, xd, mode=mode)
    q, inv = xtern.quantize_i8(xd, mode=mode)
    y2, acc = xtern.linear_q(w, q, inv, acc=True)
    assert torch.equal(y, y2)
    assert np.array_equal(acc.cpu().numpy(), exact_acc(t, q.cpu().numpy()))
