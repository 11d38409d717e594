"""The decode stack (xt_stack_*: every projection of several layers in one
persistent launch) against the oracle, bit for bit.  Layers follow the
BitNet-2B decode step (q/k/v fused, o, gate/up fused, down; reference
src/models/llama/mod.rs:420-470) with the real dependency of the residual
stream: layer L's q/k/v and gate/up read layer L-1's down output, written
inside the same launch.  Each op's expected output is the oracle's
TernaryLinear::forward (layers.rs:262-313) of the oracle's own input chain."""
import zlib

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu

BITNET = {"q": (2560, 2560), "k": (2560, 640), "v": (2560, 640), "o": (2560, 2560),
          "gate": (2560, 6912), "up": (2560, 6912), "down": (6912, 2560)}
SMALL = {"q": (256, 96), "k": (256, 32), "v": (256, 48), "o": (256, 256),
         "gate": (256, 300), "up": (256, 300), "down": (300 + 4, 256)}
# K = 4096 (16 chunks: 4 row groups per M = 1 item) and K = 8192 (the
# largest in_dim: 2 row groups per item, 4 waves per row group)
MID = {"q": (4096, 256), "k": (4096, 64), "v": (4096, 80), "o": (4096, 512),
       "gate": (4096, 1000), "up": (4096, 1000), "down": (8192, 4096)}


def log(msg):
    print(f"[case] {msg}", flush=True)


def pack4(t):
    c = (t + 1).astype(np.uint8)
    pad = (-t.shape[1]) % 4
    if pad:
        c = np.concatenate([c, np.ones((t.shape[0], pad), np.uint8)], axis=1)
    g = c.reshape(t.shape[0], -1, 4)
    return (g[..., 0] | (g[..., 1] << 2) | (g[..., 2] << 4) | (g[..., 3] << 6)).astype(np.uint8).ravel()


class Mat:
    def __init__(self, rng, K, N, sparse=False, pack5=False, ws_scale=1.0):
        p0 = rng.uniform(0.3, 0.7)
        u = rng.random((N, K))
        t = np.where(u < p0, 0, np.where(rng.random((N, K)) < 0.5, -1, 1)).astype(np.int8)
        self.K, self.N, self.t = K, N, t
        self.fmt = 1 if pack5 else 0
        self.wb = np.concatenate([xtern.pack_ternary5(r) for r in t]) if pack5 else pack4(t)
        self.ws = (rng.uniform(0.02, 0.1, N) * ws_scale).astype(np.float32)
        if sparse:
            blob = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
            self.w = xtern.DeviceWeights(xtern.XT_XORSPARSE, K, N, blob, self.ws)
        else:
            self.w = xtern.DeviceWeights(xtern.XT_PACK5 if pack5 else xtern.XT_PACK4, K, N, self.wb, self.ws)

    def ref(self, x, mode):
        return oracle.linear_forward(self.fmt, self.K, self.N, x, self.ws, wbytes=self.wb, quant_mode=mode)[0]


def build(rng, shapes, layers, M, order, sparse_down=False):
    """Returns (ops for xtern.Stack, list of (op index, [outputs], [expected]))."""
    dev = "cuda"
    f32 = torch.float32
    mats = [{n: Mat(rng, K, N, sparse=(sparse_down and n == "down")) for n, (K, N) in shapes.items()}
            for _ in range(layers)]
    Kd = shapes["down"][0]
    Ka = shapes["q"][0]
    ops, checks = [], []
    x0 = torch.from_numpy(rng.standard_normal((M, Ka)).astype(np.float32)).to(dev)
    h_prev, dep_prev = x0, None
    for L, m in enumerate(mats):
        xa = torch.from_numpy(rng.standard_normal((M, Ka)).astype(np.float32) * 2).to(dev)
        xd = torch.from_numpy(rng.standard_normal((M, Kd)).astype(np.float32)).to(dev)
        outs = {n: torch.full((M, m[n].N), float("nan"), dtype=f32, device=dev) for n in m}
        down_op = ([m["down"].w], xd, [outs["down"]], None, ["down"], xd)
        qkv_op = ([m["q"].w, m["k"].w, m["v"].w], h_prev, [outs["q"], outs["k"], outs["v"]], "prev",
                  ["q", "k", "v"], h_prev)
        o_op = ([m["o"].w], xa, [outs["o"]], None, ["o"], xa)
        gu_op = ([m["gate"].w, m["up"].w], h_prev, [outs["gate"], outs["up"]], "prev", ["gate", "up"],
                 h_prev)
        seq = [down_op, qkv_op, o_op, gu_op] if order == "down_first" else [qkv_op, o_op, gu_op, down_op]
        for ws, x, ys, dep, names, xin in seq:
            d = dep_prev if dep == "prev" else None
            ops.append((ws, x, ys, d))
            checks.append((len(ops) - 1, names, ys, xin, m))
            if names == ["down"]:
                down_idx = len(ops) - 1
        h_prev, dep_prev = outs["down"], down_idx
    return ops, checks


def expected(checks, mode):
    """Oracle outputs in op order (inputs of dependent ops are the oracle's
    own outputs of the op they depend on)."""
    got = {}
    exp = []
    for idx, names, ys, xin, m in checks:
        key = xin.data_ptr()
        x = got.get(key)
        if x is None:
            x = xin.cpu().numpy()
        e = [m[n].ref(x, mode) for n in names]
        for y, v in zip(ys, e):
            got[y.data_ptr()] = v
        exp.append(e)
    return exp


def compare(checks, exp, tag):
    for (idx, names, ys, _, _), e in zip(checks, exp):
        for n, y, v in zip(names, ys, e):
            g = y.cpu().numpy()
            assert np.array_equal(g.view(np.int32), v.view(np.int32)), \
                f"{tag}: op {idx} {n}: {int((g != v).sum())} of {g.size} outputs differ"


CASES = [("bitnet_m1_down_first", BITNET, 2, 1, "down_first", xtern.XT_QUANT_AVX512),
         ("bitnet_m1_chain", BITNET, 2, 1, "chain", xtern.XT_QUANT_AVX512),
         ("bitnet_m8_chain", BITNET, 2, 8, "chain", xtern.XT_QUANT_SCALAR),
         ("bitnet_m32_down_first", BITNET, 1, 32, "down_first", xtern.XT_QUANT_AVX512),
         ("small_m1", SMALL, 4, 1, "chain", xtern.XT_QUANT_SCALAR),
         ("small_m3", SMALL, 4, 3, "chain", xtern.XT_QUANT_AVX512),
         ("small_m17", SMALL, 3, 17, "down_first", xtern.XT_QUANT_SCALAR),
         ("mid_m1_chain", MID, 2, 1, "chain", xtern.XT_QUANT_AVX512),
         ("mid_m3_down_first", MID, 1, 3, "down_first", xtern.XT_QUANT_SCALAR),
         ("bitnet_m16_down_first", BITNET, 1, 16, "down_first", xtern.XT_QUANT_SCALAR),
         ("small_m16_chain", SMALL, 3, 16, "chain", xtern.XT_QUANT_AVX512),
         ("mid_m12_chain", MID, 2, 12, "chain", xtern.XT_QUANT_AVX512)]


@pytest.mark.parametrize("plan", ["one_launch", "per_op"])
@pytest.mark.parametrize("name,shapes,layers,M,order,mode", CASES, ids=[c[0] for c in CASES])
def test_stack_matches_oracle(name, shapes, layers, M, order, mode, plan):
    log(f"stack {name}: layers={layers} M={M} order={order} mode={mode} plan={plan}")
    rng = np.random.default_rng(zlib.crc32(name.encode()) & 0xffff)
    ops, checks = build(rng, shapes, layers, M, order, sparse_down=(M == 3))
    exp = expected(checks, mode)
    st = xtern.Stack(ops, M, mode, plan=plan)
    assert st.plan_name == plan
    for rep in range(3):  # repeated launches: the counters reset themselves
        for _, _, ys, _, _ in checks:
            for y in ys:
                y.fill_(float("nan"))
        st.run()
        torch.cuda.synchronize()
        assert not st.gave_up()
        compare(checks, exp, f"run {rep}")


@pytest.mark.parametrize("plan", ["one_launch", "per_op"])
def test_stack_in_graph_replays(plan):
    log(f"stack graph replay plan={plan}")
    rng = np.random.default_rng(5)
    ops, checks = build(rng, SMALL, 3, 2, "chain")
    exp = expected(checks, xtern.XT_QUANT_AVX512)
    st = xtern.Stack(ops, 2, plan=plan)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        st.run(stream=s)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        st.run(stream=s)
    for rep in range(3):
        for _, _, ys, _, _ in checks:
            for y in ys:
                y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        compare(checks, exp, f"replay {rep}")
    assert not st.gave_up()


def test_stack_rejects_bad_ops():
    log("stack argument errors")
    rng = np.random.default_rng(1)
    m = Mat(rng, 256, 32)
    x = torch.zeros((1, 256), device="cuda")
    y = torch.zeros((1, 32), device="cuda")
    with pytest.raises(xtern.XternError):
        xtern.Stack([([m.w], x, [y], 0)], 1)          # dep on itself
    with pytest.raises(xtern.XternError):
        xtern.Stack([([m.w], x, [y], None)], 33)      # M above 32
    p5 = xtern.DeviceWeights(xtern.XT_PACK5, 256, 32,
                             np.concatenate([xtern.pack_ternary5(r) for r in m.t]), m.ws)
    xs = xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, 256, 32,
                             np.frombuffer(xtern.encode_sparse_tensor(m.t, 256, 32)[0], np.uint8), m.ws)
    with pytest.raises(xtern.XternError):
        xtern.Stack([([xs], x, [y], None)], 1, plan="one_launch")  # compact stream: per op only
    with pytest.raises(xtern.XternError):
        xtern.Stack([([m.w], x, [y], None)], 1, plan="fastest")      # unknown plan
    with pytest.raises(xtern.XternError):
        xtern.Stack([([m.w], x, [y], None), ([m.w], x, [y], 0)], 1)  # x not an output of dep
    with pytest.raises(xtern.XternError):
        xtern.Stack([([m.w, p5], x, [y, y], None)], 1)  # Pack4 and Pack5 in one op


def build_chain(rng, mats, M, x0):
    """The strict projection chain: q/k/v read the previous down output, o
    reads q, gate/up read o, down reads up (every op waits for the one
    before it).  mats: per layer {name: Mat}."""
    dev = "cuda"
    ops, checks = [], []
    h_prev, dep_prev = x0, None
    for m in mats:
        outs = {n: torch.full((M, m[n].N), float("nan"), dtype=torch.float32, device=dev) for n in m}
        seq = [(["q", "k", "v"], h_prev, dep_prev), (["o"], outs["q"], "last"),
               (["gate", "up"], outs["o"], "last"), (["down"], outs["up"], "last")]
        for names, x, dep in seq:
            d = len(ops) - 1 if dep == "last" else dep
            ys = [outs[n] for n in names]
            ops.append(([m[n].w for n in names], x, ys, d))
            checks.append((len(ops) - 1, names, ys, x, m))
        h_prev, dep_prev = outs["down"], len(ops) - 1
    return ops, checks


def run_and_compare(ops, checks, M, mode, reps=2, plan="one_launch"):
    exp = expected(checks, mode)
    st = xtern.Stack(ops, M, mode, plan=plan)
    if plan is not None:
        assert st.plan_name == plan
    for rep in range(reps):
        for _, _, ys, _, _ in checks:
            for y in ys:
                y.fill_(float("nan"))
        st.run()
        torch.cuda.synchronize()
        assert not st.gave_up()
        compare(checks, exp, f"run {rep}")


def test_stack_m1_strict_chain_bitnet():
    """Two BitNet-2B layers as the strict chain q/k/v -> o -> gate/up -> down."""
    log("stack strict chain, bitnet, M=1")
    rng = np.random.default_rng(zlib.crc32(b"strict_chain") & 0xffff)
    mats = [{n: Mat(rng, K, N, ws_scale=0.3) for n, (K, N) in BITNET.items()} for _ in range(2)]
    x0 = torch.from_numpy(rng.standard_normal((1, 2560)).astype(np.float32)).cuda()
    ops, checks = build_chain(rng, mats, 1, x0)
    run_and_compare(ops, checks, 1, xtern.XT_QUANT_AVX512, reps=3)


def test_stack_m1_bitnet_30_layers():
    """The full 30-layer BitNet-2B projection chain at M = 1 (120 ops, 210
    projections) against the oracle.  Layers share one set of 7 matrices (the
    device weights are the same handles; the host builds 7 matrices, not
    210); every layer still reads the previous layer's output from inside the
    launch."""
    log("stack 30-layer bitnet chain, M=1")
    rng = np.random.default_rng(zlib.crc32(b"bitnet30") & 0xffff)
    shared = {n: Mat(rng, K, N, ws_scale=0.3) for n, (K, N) in BITNET.items()}
    x0 = torch.from_numpy(rng.standard_normal((1, 2560)).astype(np.float32)).cuda()
    ops, checks = build_chain(rng, [shared] * 30, 1, x0)
    assert len(ops) == 120
    run_and_compare(ops, checks, 1, xtern.XT_QUANT_SCALAR)


def test_stack_m8_bitnet_30_layers():
    """The 30-layer BitNet-2B projection chain at M = 8 (120 ops) in one
    launch against the oracle (shared matrices, as at M = 1)."""
    log("stack 30-layer bitnet chain, M=8")
    rng = np.random.default_rng(zlib.crc32(b"bitnet30_m8") & 0xffff)
    shared = {n: Mat(rng, K, N, ws_scale=0.3) for n, (K, N) in BITNET.items()}
    x0 = torch.from_numpy(rng.standard_normal((8, 2560)).astype(np.float32)).cuda()
    ops, checks = build_chain(rng, [shared] * 30, 8, x0)
    run_and_compare(ops, checks, 8, xtern.XT_QUANT_AVX512, reps=1)


PACK5_3B = {"q": (3200, 3200), "k": (3200, 320), "v": (3200, 320), "o": (3200, 3200),
            "gate": (3200, 8640), "up": (3200, 8640), "down": (8640, 3200)}


@pytest.mark.parametrize("M,mode", [(1, xtern.XT_QUANT_AVX512), (1, xtern.XT_QUANT_SCALAR),
                                    (8, xtern.XT_QUANT_AVX512), (16, xtern.XT_QUANT_SCALAR),
                                    (24, xtern.XT_QUANT_AVX512)])
def test_stack_pack5_chain(M, mode):
    """Pack5 weights (BitNet-3B shapes) in one launch,
    strict chain, two layers."""
    log(f"stack pack5 chain M={M} mode={mode}")
    rng = np.random.default_rng(zlib.crc32(b"pack5_chain") & 0xffff + mode + M)
    mats = [{n: Mat(rng, K, N, pack5=True, ws_scale=0.3) for n, (K, N) in PACK5_3B.items()} for _ in range(2)]
    x0 = torch.from_numpy(rng.standard_normal((M, 3200)).astype(np.float32)).cuda()
    ops, checks = build_chain(rng, mats, M, x0)
    run_and_compare(ops, checks, M, mode)


@pytest.mark.parametrize("M", [1, 2, 5, 8, 13, 16])
def test_stack_ragged_mixed_formats(M):
    """Ragged shapes (N not a multiple of 16, K not of 256, Pack5 rows of an
    odd number of 320-column chunks), XorSparse and Pack4 projections, and
    a Pack5 op in one launch."""
    log(f"stack ragged mixed formats M={M}")
    rng = np.random.default_rng(zlib.crc32(b"ragged_mixed") & 0xffff + M)
    a = Mat(rng, 300, 76)
    b = Mat(rng, 300, 45, sparse=True)
    c = Mat(rng, 76, 132, pack5=True)
    d = Mat(rng, 132, 300, sparse=True)
    e = Mat(rng, 300, 37, pack5=True)
    x0 = torch.from_numpy(rng.standard_normal((M, 300)).astype(np.float32)).cuda()
    ya = torch.full((M, 76), float("nan"), device="cuda")
    yb = torch.full((M, 45), float("nan"), device="cuda")
    yc = torch.full((M, 132), float("nan"), device="cuda")
    yd = torch.full((M, 300), float("nan"), device="cuda")
    ye = torch.full((M, 37), float("nan"), device="cuda")
    ops = [([a.w, b.w], x0, [ya, yb], None), ([c.w], ya, [yc], 0), ([d.w], yc, [yd], 1),
           ([a.w], yd, [torch.full((M, 76), float("nan"), device="cuda")], 2), ([e.w], yd, [ye], 2)]
    checks = [(0, ["a", "b"], [ya, yb], x0, {"a": a, "b": b}), (1, ["c"], [yc], ya, {"c": c}),
              (2, ["d"], [yd], yc, {"d": d}), (3, ["a"], ops[3][2], yd, {"a": a}),
              (4, ["e"], [ye], yd, {"e": e})]
    run_and_compare(ops, checks, M, xtern.XT_QUANT_AVX512, reps=3)


@pytest.mark.parametrize("M", [1, 3, 8, 13, 20, 32])
def test_stack_pack5_heavy_mixed_formats(M):
    """A list whose bytes are mostly Pack5 (the one-launch plan then runs its
    base-3 token forms) with a Pack4 and an XorSparse projection
    running in those forms too, ragged shapes, dependencies inside the
    launch."""
    log(f"stack pack5-heavy mixed formats M={M}")
    rng = np.random.default_rng(zlib.crc32(b"pack5_heavy") & 0xffff + M)
    a = Mat(rng, 1000, 720, pack5=True)
    b = Mat(rng, 1000, 61)
    c = Mat(rng, 720, 1000, pack5=True)
    d = Mat(rng, 1000, 83, sparse=True)
    tiles = lambda K, N, cols: -(-N // 16) * -(-K // cols)
    p5 = tiles(1000, 720, 320) + tiles(720, 1000, 320)
    assert 2 * p5 > p5 + tiles(1000, 61, 256) + tiles(1000, 83, 256)
    x0 = torch.from_numpy(rng.standard_normal((M, 1000)).astype(np.float32)).cuda()
    ya = torch.full((M, 720), float("nan"), device="cuda")
    yb = torch.full((M, 61), float("nan"), device="cuda")
    yc = torch.full((M, 1000), float("nan"), device="cuda")
    yd = torch.full((M, 83), float("nan"), device="cuda")
    # (the projections of one op share a tile format)
    ops = [([a.w], x0, [ya], None), ([b.w], x0, [yb], None), ([c.w], ya, [yc], 0), ([d.w], yc, [yd], 2)]
    checks = [(0, ["a"], [ya], x0, {"a": a}), (1, ["b"], [yb], x0, {"b": b}), (2, ["c"], [yc], ya, {"c": c}),
              (3, ["d"], [yd], yc, {"d": d})]
    run_and_compare(ops, checks, M, xtern.XT_QUANT_SCALAR, reps=3)


def test_stack_auto_plan_choice():
    """XT_STACK_AUTO: the strict 8-layer chain (32 dependency levels) runs
    per op; the residual-only list (two levels, 32 ops) in one launch; a
    compact-stream XorSparse op (not taken by the one-launch kernels) per op.  Each is
    checked against the oracle in the plan it got."""
    log("stack auto plan choice")
    rng = np.random.default_rng(zlib.crc32(b"auto_plan") & 0xffff)
    shared = {n: Mat(rng, K, N, ws_scale=0.3) for n, (K, N) in BITNET.items()}
    x0 = torch.from_numpy(rng.standard_normal((1, 2560)).astype(np.float32)).cuda()
    ops, checks = build_chain(rng, [shared] * 8, 1, x0)
    st = xtern.Stack(ops, 1)
    assert st.plan_name == "per_op"
    run_and_compare(ops, checks, 1, xtern.XT_QUANT_AVX512, reps=1, plan=None)

    # residual only: layer L's q/k/v and gate/up read layer L-1's down output;
    # o and down read inputs ready before the run
    ops, checks = [], []
    h, dep = x0, None
    for L in range(8):
        outs = {n: torch.full((1, shared[n].N), float("nan"), device="cuda") for n in shared}
        xo = torch.from_numpy(rng.standard_normal((1, 2560)).astype(np.float32)).cuda()
        xd = torch.from_numpy(rng.standard_normal((1, 6912)).astype(np.float32)).cuda()
        for names, x, d in ((["down"], xd, None), (["q", "k", "v"], h, dep), (["o"], xo, None),
                            (["gate", "up"], h, dep)):
            ys = [outs[n] for n in names]
            ops.append(([shared[n].w for n in names], x, ys, d))
            checks.append((len(ops) - 1, names, ys, x, shared))
            if names == ["down"]:
                dn = len(ops) - 1
        h, dep = outs["down"], dn
    st = xtern.Stack(ops, 1)
    assert st.plan_name == "one_launch"
    run_and_compare(ops, checks, 1, xtern.XT_QUANT_SCALAR, reps=1, plan=None)

    m = Mat(rng, 320, 48)
    xs = xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, 320, 48,
                             np.frombuffer(xtern.encode_sparse_tensor(m.t, 320, 48)[0], np.uint8), m.ws)
    m.w = xs  # (the oracle reference stays the Pack4 bytes of the same matrix)
    x2 = torch.from_numpy(rng.standard_normal((5, 320)).astype(np.float32)).cuda()
    y2 = torch.full((5, 48), float("nan"), device="cuda")
    st = xtern.Stack([([m.w], x2, [y2], None)], 5)
    assert st.plan_name == "per_op"
    run_and_compare([([m.w], x2, [y2], None)], [(0, ["p"], [y2], x2, {"p": m})], 5,
                    xtern.XT_QUANT_AVX512, reps=1, plan=None)


@pytest.mark.parametrize("M", [1, 6])
def test_stack_long_rows(M):
    """in_dim well above the BitNet shapes (Pack4 16000, Pack5 12800 -> 40
    chunks of 320): the quantiser tasks take the row in several rounds and
    the group tasks walk 63 / 40 chunks; chained in one launch."""
    log(f"stack long rows M={M}")
    rng = np.random.default_rng(zlib.crc32(b"long_rows") & 0xffff + M)
    a = Mat(rng, 16000, 40)
    b = Mat(rng, 40, 12800, pack5=False)
    c = Mat(rng, 12800, 23, pack5=True)
    x0 = torch.from_numpy(rng.standard_normal((M, 16000)).astype(np.float32)).cuda()
    ya = torch.full((M, 40), float("nan"), device="cuda")
    yb = torch.full((M, 12800), float("nan"), device="cuda")
    yc = torch.full((M, 23), float("nan"), device="cuda")
    ops = [([a.w], x0, [ya], None), ([b.w], ya, [yb], 0), ([c.w], yb, [yc], 1)]
    checks = [(0, ["a"], [ya], x0, {"a": a}), (1, ["b"], [yb], ya, {"b": b}), (2, ["c"], [yc], yb, {"c": c})]
    run_and_compare(ops, checks, M, xtern.XT_QUANT_SCALAR, reps=2)
