"""HF prepacked (output-dim striped) checkpoint bytes, loader/mod.rs:301-394.

CPU: the oracle's destripe is pinned by a hand-worked byte, by the striping
rule applied forwards to random ternary matrices (stripe -> destripe must
give the rows' own Pack4/Pack5 encoding), and by the digit rules of the
reference unpackers on every byte value (Pack4 code 11 -> 0, Pack5 bytes
243..255 -> repeated %3 and /3).  The library's host xt_hf_destripe must equal
the oracle on arbitrary bytes.  GPU: tiles built on the device by
xt_weights_create_hf equal the host repack of the destriped bytes, byte for
byte, and a layer built from striped bytes computes what the oracle computes
from the destriped rows (bit-exact i32 and f32)."""
import numpy as np
import pytest

import oracle
import xtern

P4, P5 = xtern.XT_PACK4, xtern.XT_PACK5


def stripe(t, fmt):
    """Forward striping rule: digit j of byte [p][i] = code of row j*R + p."""
    f = 4 if fmt == P4 else 5
    N, K = t.shape
    R = N // f
    codes = (t.astype(np.int64) + 1).reshape(f, R, K)  # [j][p][i]
    if fmt == P4:
        return sum(codes[j] << (2 * j) for j in range(f)).astype(np.uint8)
    return sum(codes[j] * 3 ** j for j in range(f)).astype(np.uint8)


def pack_rows(t, fmt):
    pack = oracle.pack4 if fmt == P4 else oracle.pack5
    return np.concatenate([pack(r.astype(np.float32), 1.0) for r in t])


def test_hand_worked_byte():
    # K = 1, N = 4: byte 0b10_01_00_10 holds rows 0..3 = +1, -1, 0, +1 (j = 0..3).
    stored = np.array([[0b10010010]], np.uint8)
    got = oracle.hf_destripe(P4, 1, 4, stored)
    assert got.tolist() == [0b10, 0b00, 0b01, 0b10]
    # Pack5, K = 1, N = 5: 2 + 0*3 + 1*9 + 2*27 + 0*81 = 65 -> +1, -1, 0, +1, -1.
    got = oracle.hf_destripe(P5, 1, 5, np.array([[65]], np.uint8))
    assert got.tolist() == [2, 0, 1, 2, 0]


@pytest.mark.parametrize("fmt", [P4, P5])
@pytest.mark.parametrize("K,N", [(1, 20), (7, 40), (64, 60), (333, 20), (1000, 120)])
def test_oracle_inverts_striping(fmt, K, N):
    rng = np.random.default_rng(K * 1000 + N + fmt)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    got = oracle.hf_destripe(fmt, K, N, stripe(t, fmt))
    assert np.array_equal(got, pack_rows(t, fmt))


@pytest.mark.parametrize("fmt", [P4, P5])
def test_oracle_digit_rules_every_byte(fmt):
    f = 4 if fmt == P4 else 5
    stored = np.arange(256, dtype=np.uint8).reshape(1, 256)  # K = 256, N = f
    got = oracle.hf_destripe(fmt, 256, f, stored)
    bpr = -(-256 // f)
    for j in range(f):
        row = (oracle.unpack4 if fmt == P4 else oracle.unpack5)(got[j * bpr:(j + 1) * bpr], 256)
        for x in range(256):
            if fmt == P4:
                fld = (x >> (2 * j)) & 3
                want = -1.0 if fld == 0 else (1.0 if fld == 2 else 0.0)
            else:
                want = float((x // 3 ** j) % 3 - 1)
            assert row[x] == want, (j, x)


@pytest.mark.parametrize("fmt", [P4, P5])
@pytest.mark.parametrize("K,N", [(1, 20), (13, 40), (333, 20), (2560, 640), (3200, 160)])
def test_library_destripe_matches_oracle(fmt, K, N):
    f = 4 if fmt == P4 else 5
    rng = np.random.default_rng(K + 7 * N + fmt)
    stored = rng.integers(0, 256, size=(N // f, K), dtype=np.uint8)
    assert np.array_equal(xtern.hf_destripe(fmt, K, N, stored),
                          oracle.hf_destripe(fmt, K, N, stored))


def test_destripe_errors():
    with pytest.raises(xtern.XternError, match="pre-packed U8"):
        xtern.hf_destripe(P4, 8, 6, np.zeros(12, np.uint8))  # 6 % 4 != 0
    with pytest.raises(xtern.XternError, match="pre-packed U8"):
        xtern.hf_destripe(P5, 8, 10, np.zeros(17, np.uint8))  # needs 16 bytes
    with pytest.raises(xtern.XternError, match="Pack4 or Pack5"):
        xtern.hf_destripe(xtern.XT_XORSPARSE, 8, 8, np.zeros(16, np.uint8))


def test_get_prepacked_ternary_mirror():
    t = np.array([[1, 0, -1], [0, 1, 1], [-1, -1, 0], [1, 1, 1]], np.int8)
    stored = stripe(t, P4)
    packed, ws, k, n = xtern.get_prepacked_ternary(
        stored, "U8", (4, 3), xtern.TernaryPackType.Pack4, 0.3, True)
    assert (k, n) == (3, 4)
    assert np.array_equal(packed, pack_rows(t, P4))
    assert ws.dtype == np.float32 and np.all(ws == np.float32(1.0) / np.float32(0.3))
    _, ws2, _, _ = xtern.get_prepacked_ternary(
        stored, "U8", (4, 3), xtern.TernaryPackType.Pack4, 0.3, False)
    assert np.all(ws2 == np.float32(0.3))
    for bad in [(stored, "BF16", (4, 3)), (stored, "U8", (8, 3)), (stored, "U8", (4, 4))]:
        with pytest.raises(xtern.XternError, match="pre-packed U8"):
            xtern.get_prepacked_ternary(bad[0], bad[1], bad[2], xtern.TernaryPackType.Pack4,
                                        1.0, False)


# ---------------------------------------------------------------------- GPU ---

GPU_CASES = [(P4, 333, 20), (P5, 1000, 35), (P4, 2560, 6912), (P5, 3200, 8640),
             (P5, 8640, 3200), (P4, 6912, 2560), (P4, 64, 4), (P5, 321, 5)]


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,K,N", GPU_CASES)
def test_device_tiles_equal_host_repack(fmt, K, N):
    print(f"[case] hf tiles fmt={fmt} K={K} N={N}", flush=True)
    f = 4 if fmt == P4 else 5
    rng = np.random.default_rng(3 * K + N + fmt)
    stored = rng.integers(0, 256, size=(N // f, K), dtype=np.uint8)
    dev = xtern.DeviceWeights.from_hf(fmt, K, N, stored, 0.5)
    want = xtern.repack_host(fmt, K, N, oracle.hf_destripe(fmt, K, N, stored))
    assert np.array_equal(dev.read_tiles(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,K,N,M", [(P4, 2560, 640, 1), (P5, 3200, 160, 8),
                                       (P4, 2560, 6912, 32), (P5, 1000, 35, 3)])
@pytest.mark.parametrize("inverted", [False, True])
def test_hf_layer_matches_oracle(fmt, K, N, M, inverted):
    import torch
    print(f"[case] hf layer fmt={fmt} K={K} N={N} M={M} inv={inverted}", flush=True)
    f = 4 if fmt == P4 else 5
    rng = np.random.default_rng(K + N + M)
    stored = rng.integers(0, 256, size=(N // f, K), dtype=np.uint8)
    pt = xtern.TernaryPackType.Pack4 if fmt == P4 else xtern.TernaryPackType.Pack5
    lin = xtern.TernaryLinear.from_hf_prepacked(stored, K, N, pt, 0.37, inverted)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = lin.forward(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    packed, ws, _, _ = xtern.get_prepacked_ternary(stored, "U8", (N, K), pt, 0.37, inverted)
    y_ref, q_ref, inv_ref, acc_ref = oracle.linear_forward(fmt, K, N, x, ws, wbytes=packed)
    assert np.allclose(y, y_ref, rtol=1e-5, atol=1e-4)
    assert np.array_equal(y.view(np.int32), y_ref.view(np.int32))
    _, acc = xtern.linear_q(lin.weights, torch.from_numpy(q_ref).to("cuda:0"),
                            torch.from_numpy(inv_ref).to("cuda:0"), acc=True)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    assert lin.packed_bytes() == N * (-(-K // f))
    # sparse=True goes through the host destripe and new_sparse_from_packed
    lin_s = xtern.TernaryLinear.from_hf_prepacked(stored, K, N, pt, 0.37, inverted, sparse=True)
    y_s = lin_s.forward(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    assert np.array_equal(y_s.view(np.int32), y_ref.view(np.int32))
