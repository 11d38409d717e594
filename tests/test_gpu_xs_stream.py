"""XorSparse weights kept compact on the GPU (XT_XORSPARSE_STREAM): the
product kernel reads the block masks and set-order sign bits of the
reference's blob (src/bit1_58/sparse.rs:61-86, decoded as simd.rs:416-548)
and must give bit-exact i32 dots and f32 outputs: against an exact float64
matmul of the ternary weights, against the 2-bit tile path of the same blob
(XT_XORSPARSE), and, on small shapes, against the oracle's own sparse dot.
C3's shapes (LLaMA-3-8B-1.58: 4096 -> 14336, 14336 -> 4096) at M in
{1, 4, 16}, plus ragged and limit shapes."""
import zlib

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def log(msg):
    print(f"[case] {msg}", flush=True)


def sparse_tern(rng, N, K):
    """Zero fraction uniform in [0.3, 0.7] per 64-block."""
    nb = (K + 63) // 64
    zf = rng.uniform(0.3, 0.7, (N, nb, 1))
    u = rng.random((N, nb, 64))
    sign = np.where(rng.random((N, nb, 64)) < 0.5, -1, 1)
    return np.where(u < zf, 0, sign).astype(np.int8).reshape(N, nb * 64)[:, :K].copy()


def check_bits(y, ref, what):
    assert np.array_equal(y.view(np.int32), ref.view(np.int32)), \
        f"{what}: {int(np.sum(y != ref))} of {y.size} f32 outputs differ in bits"


CASES = [("c3_up", 4096, 14336, [1, 4, 16]),
         ("c3_down", 14336, 4096, [1, 4, 16, 20]),
         ("ragged", 300, 50, [1, 3, 17]),
         ("k16384", 16384, 64, [1, 5]),
         ("one_row", 64, 1, [1, 2])]


@pytest.mark.parametrize("name,K,N,Ms", CASES, ids=[c[0] for c in CASES])
def test_stream_matches_exact_and_tiles(name, K, N, Ms):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    t = sparse_tern(rng, N, K)
    blob = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
    ws = rng.uniform(0.02, 0.1, N).astype(np.float32)
    w = xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, K, N, blob, ws)
    wt = xtern.DeviceWeights(xtern.XT_XORSPARSE, K, N, blob, ws)
    # the device holds the host-built layout, which is smaller than the tiles
    host, _ = xtern.xorsparse_stream_host(K, N, blob)
    assert np.array_equal(w.read_tiles(), host)
    for M in Ms:
        log(f"stream {name} K={K} N={N} M={M}")
        x = rng.standard_normal((M, K)).astype(np.float32)
        xd = torch.from_numpy(x).to(DEV)
        q, inv = xtern.quantize_i8(xd)
        y, acc = xtern.linear_q(w, q, inv, acc=True)
        yt = xtern.linear_q(wt, q, inv)
        qn, invn = q.cpu().numpy(), inv.cpu().numpy()
        y, acc, yt = y.cpu().numpy(), acc.cpu().numpy(), yt.cpu().numpy()
        a64 = (qn.astype(np.float64) @ t.astype(np.float64).T).astype(np.int64)
        assert np.array_equal(acc, a64), f"{int(np.sum(acc != a64))} i32 dots differ"
        y_ref = ((a64.astype(np.float32) * invn[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
        check_bits(y, y_ref, "vs exact")
        check_bits(y, yt, "vs the tile path")
        yf = xtern.linear_f32(w, xd).cpu().numpy()
        check_bits(yf, y, "f32 forward vs q forward")
        if K * N <= 1 << 16:  # the oracle's own sparse dot (simd.rs:416-548)
            masks, signs, _ = oracle.sparse_from_blob(blob, N, K)
            yo = oracle.linear_forward_q(2, K, N, qn, invn, ws, masks=masks, signs=signs)[0]
            check_bits(y, yo, "vs oracle")


def test_stream_fused_projections():
    """Two projections on one quantised input (fused_forward_qkv's shape of
    call) equal two separate calls."""
    rng = np.random.default_rng(5)
    K = 2560
    ts = [sparse_tern(rng, n, K) for n in (640, 1000)]
    ws = [rng.uniform(0.02, 0.1, t.shape[0]).astype(np.float32) for t in ts]
    W = [xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, K, t.shape[0],
                             np.frombuffer(xtern.encode_sparse_tensor(t, K, t.shape[0])[0], np.uint8), s)
         for t, s in zip(ts, ws)]
    xd = torch.randn(3, K, device=DEV)
    outs = [torch.empty(3, t.shape[0], device=DEV) for t in ts]
    xtern.linear_multi_f32(W, xd, outs=outs)
    for w, o in zip(W, outs):
        check_bits(o.cpu().numpy(), xtern.linear_f32(w, xd).cpu().numpy(), "fused vs separate")


def test_stream_refused_where_unsupported():
    rng = np.random.default_rng(6)
    K, N = 256, 64
    t = sparse_tern(rng, N, K)
    blob = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
    w = xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, K, N, blob, np.ones(N, np.float32))
    x = torch.randn(1, K, device=DEV)
    y = torch.zeros(1, N, device=DEV)
    # the one-launch stack kernels take tile formats only; the automatic plan
    # runs a compact-stream op as its own call
    with pytest.raises(xtern.XternError, match="stack weights"):
        xtern.Stack([([w], x, [y], None)], 1, plan="one_launch")
    st = xtern.Stack([([w], x, [y], None)], 1)
    assert st.plan_name == "per_op"
    st.run()
    check_bits(y.cpu().numpy(), xtern.linear_f32(w, x).cpu().numpy(), "per-op stack vs call")
    big = sparse_tern(rng, 1, 16384 + 64)
    with pytest.raises(xtern.XternError, match="in_dim up to 16384"):
        xtern.DeviceWeights(xtern.XT_XORSPARSE_STREAM, 16384 + 64, 1,
                            np.frombuffer(xtern.encode_sparse_tensor(big, 16384 + 64, 1)[0], np.uint8),
                            np.ones(1, np.float32))
