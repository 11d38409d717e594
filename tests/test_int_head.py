"""Int8 / Int4 LM head (Int8Linear / Int4Linear, src/nn/dynamic_linear.rs:229-535).

The reference has no tests for these types, so the oracle is pinned by closed
forms computed independently in numpy: per-row absmax scales, round half away
from zero done exactly (floor + fraction compare, no float re-rounding),
clamping; nibble sign extension; brute-force integer dots; Int4's
chunks_exact(2) pairing, which skips the last column of an odd in_dim.  The
library's host quantiser equals the oracle, and an independent numpy decoder
of the Int8 / Int4 tile layout recovers the weights.  GPU: forward and
forward_with_quantized bit-exact against the oracle, up to a full
128256 x 2560 LM head.
"""
import numpy as np
import pytest

import oracle
import xtern

f32 = np.float32


def round_half_away(v):
    a = np.abs(v)
    fl = np.floor(a)
    r = fl + (a - fl >= f32(0.5))
    return np.sign(v) * r


def np_int_new(bits, w):
    qmax = f32(127) if bits == 8 else f32(7)
    lo, hi = (-127, 127) if bits == 8 else (-8, 7)
    mx = np.max(np.abs(w), axis=1).astype(f32)
    scale = np.where(mx > 0, (mx / qmax).astype(f32), f32(1)).astype(f32)
    q = np.clip(round_half_away((w / scale[:, None]).astype(f32)), lo, hi).astype(np.int8)
    return q, scale


def pack_nibbles(q):
    N, K = q.shape
    if K % 2:
        q = np.concatenate([q, np.zeros((N, 1), np.int8)], axis=1)
    u = q.astype(np.uint8) & 15
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8).ravel()


def decode_nibbles(b, N, K):
    b = b.reshape(N, (K + 1) // 2)
    lo = ((b & 15).astype(np.int8) ^ 8) - 8
    hi = ((b >> 4).astype(np.int8) ^ 8) - 8
    out = np.empty((N, 2 * b.shape[1]), np.int8)
    out[:, 0::2], out[:, 1::2] = lo, hi
    return out[:, :K]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("N,K", [(3, 1), (5, 7), (16, 64), (33, 333), (10, 2560)])
def test_weight_quantisation(bits, N, K):
    rng = np.random.default_rng(N * K + bits)
    w = (rng.standard_normal((N, K)) * np.exp(rng.standard_normal((N, 1)))).astype(f32)
    w[0, :] = 0.0  # zero row -> scale 1
    if K > 3:
        w[1, :3] = [0.5, -0.5, 1.5]  # ties for round-half-away
    q, sc = np_int_new(bits, w)
    ob, osc = oracle.int_new(bits, w, N, K)
    lb, lsc = xtern.int_quantize_host(bits, w, N, K)
    np.testing.assert_array_equal(osc, sc)
    np.testing.assert_array_equal(lsc, sc)
    want = q.view(np.uint8).ravel() if bits == 8 else pack_nibbles(q)
    np.testing.assert_array_equal(ob, want)
    np.testing.assert_array_equal(lb, want)
    assert sc[0] == 1.0


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("K", [64, 333, 2560])
def test_oracle_forward(bits, K):
    rng = np.random.default_rng(K + bits)
    N, M = 37, 3
    w = rng.standard_normal((N, K)).astype(f32)
    wb, sc = oracle.int_new(bits, w, N, K)
    wq = wb.view(np.int8).reshape(N, K) if bits == 8 else decode_nibbles(wb, N, K)
    if bits == 4 and K % 2:
        wq = wq.copy()
        wq[:, -1] = 0  # chunks_exact(2) never reaches the last column
    x = rng.standard_normal((M, K)).astype(f32)
    y, acc = oracle.int_forward(bits, wb, sc, K, N, x)
    q = np.stack([oracle.quantize(x[m])[0] for m in range(M)])
    inv = np.array([oracle.quantize(x[m])[1] for m in range(M)], f32)
    want_acc = q.astype(np.int64) @ wq.astype(np.int64).T
    np.testing.assert_array_equal(acc, want_acc)
    want_y = ((acc.astype(f32) * inv[:, None]).astype(f32) * sc[None, :]).astype(f32)
    np.testing.assert_array_equal(y, want_y)


def decode_int_tiles(tiles, bits, K, N):
    nch, ng = -(-K // 256), -(-N // 16)
    tpc = 4 if bits == 8 else 2
    t = tiles.reshape(ng, nch, tpc, 4, 16, 16)  # G, c, tile, g, j, byte
    out = np.zeros((ng * 16, nch * 256), np.int16)
    for s in range(4):
        for g in range(4):
            cols = np.arange(nch)[:, None] * 256 + s * 64 + g * 16 + np.arange(16)[None, :]
            if bits == 8:
                vals = t[:, :, s, g].view(np.int8)                     # G, c, j, b
            else:
                byte = t[:, :, s >> 1, g].astype(np.int16)
                vals = ((byte >> (4 * (s & 1))) & 15) - 8               # codes are q + 8
            for j in range(16):
                rows = np.arange(ng) * 16 + j
                out[np.ix_(rows, cols.ravel())] = vals[:, :, j, :].reshape(ng, -1)
    return out[:N, :K]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("N,K", [(16, 256), (20, 333), (40, 700)])
def test_tile_layout(bits, N, K):
    rng = np.random.default_rng(N + K)
    w = rng.standard_normal((N, K)).astype(f32)
    wb, _ = oracle.int_new(bits, w, N, K)
    tiles = xtern.repack_host(xtern.XT_INT8 if bits == 8 else xtern.XT_INT4, K, N, wb)
    got = decode_int_tiles(tiles, bits, K, N)
    want = wb.view(np.int8).reshape(N, K) if bits == 8 else decode_nibbles(wb, N, K)
    want = want.astype(np.int16)
    if bits == 4 and K % 2:
        want[:, -1] = 0
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------------- GPU ---

@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("K,N,M", [(2560, 1000, 1), (2560, 1000, 3), (333, 77, 5), (3200, 4096, 16),
                                   (2560, 4096, 40), (7000, 300, 20), (9000, 200, 2),
                                   (2560, 6416, 2)])
@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
def test_int_linear_matches_oracle(bits, K, N, M, mode):
    import torch
    print(f"[case] int{bits} K={K} N={N} M={M} mode={mode}", flush=True)
    rng = np.random.default_rng(K * 7 + N + M + bits)
    w = rng.standard_normal((N, K)).astype(f32)
    cls = xtern.Int8Linear if bits == 8 else xtern.Int4Linear
    lin = cls.new(w, N, K)
    x = rng.standard_normal((M, K)).astype(f32)
    x[:, :2] *= 30
    y = lin.forward(torch.from_numpy(x).to("cuda:0"), mode=mode).cpu().numpy()
    y_ref, acc_ref = oracle.int_forward(bits, lin.weight_bytes, lin.scales, K, N, x, quant_mode=mode)
    assert np.allclose(y, y_ref, rtol=1e-5, atol=1e-4)
    assert np.array_equal(y.view(np.int32), y_ref.view(np.int32))
    q, inv = xtern.quantize_i8(torch.from_numpy(x).to("cuda:0"), mode=mode)
    y2, acc = xtern.linear_q(lin.weights, q, inv, acc=True)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    assert np.array_equal(y2.cpu().numpy().view(np.int32), y_ref.view(np.int32))
    yq = lin.forward_with_quantized(torch.from_numpy(x).to("cuda:0"), q, inv).cpu().numpy()
    assert np.array_equal(yq.view(np.int32), y_ref.view(np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_full_lm_head(bits):
    """BitNet-2B LM head: 128256 x 2560, one token (the decode-step head)."""
    import torch
    print(f"[case] lm head int{bits}", flush=True)
    N, K = 128256, 2560
    rng = np.random.default_rng(bits)
    w = rng.standard_normal((N, K), dtype=np.float32)
    lin = xtern.DynamicLinear.new_int8(w, N, K) if bits == 8 else xtern.DynamicLinear.new_int4(w, N, K)
    del w
    x = rng.standard_normal((1, K)).astype(f32)
    y = lin.forward(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    y_ref, _ = oracle.int_forward(bits, lin.inner.weight_bytes, lin.inner.scales, K, N, x)
    assert np.array_equal(y.view(np.int32), y_ref.view(np.int32))
    assert int(np.argmax(y)) == int(np.argmax(y_ref))


@pytest.mark.gpu
def test_mlp_with_int8_down():
    """mlp.rs:76-95: ternary gate/up with an Int8 down take the fused path
    (fused_mlp_gate_up_down); an Int4 down takes the unfused path."""
    import torch
    print("[case] mlp int8 down", flush=True)
    rng = np.random.default_rng(5)
    H, I = 512, 1024
    P4 = xtern.TernaryPackType.Pack4
    g = xtern.TernaryLinear.new(H, I, rng.integers(-1, 2, (I, H)).astype(f32).ravel(), P4)
    u = xtern.TernaryLinear.new(H, I, rng.integers(-1, 2, (I, H)).astype(f32).ravel(), P4)
    wd = rng.standard_normal((H, I)).astype(f32)
    x = rng.standard_normal((1, H)).astype(f32)
    xd = torch.from_numpy(x).to("cuda:0")
    for bits, fused in ((8, True), (4, False)):
        d = (xtern.Int8Linear if bits == 8 else xtern.Int4Linear).new(wd, H, I)
        y = xtern.mlp_f32(g.weights, u.weights, d.weights, xd, use_silu=True).cpu().numpy()
        gg = g.forward(xd).cpu().numpy()
        uu = u.forward(xd).cpu().numpy()
        mid = oracle.silu_inplace(gg, uu, True, avx512=True) if fused else oracle.act_mul(gg, uu, True)
        y_ref, _ = oracle.int_forward(bits, d.weight_bytes, d.scales, I, H, mid)
        assert np.array_equal(y.view(np.int32), y_ref.view(np.int32)), bits
