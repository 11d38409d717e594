"""XorSparse compact stream (XT_XORSPARSE_STREAM) device layout, on the CPU.

The layout keeps the reference blob's block masks and set-order sign bits
(src/bit1_58/sparse.rs:9-17, :61-86) regrouped by 16-row group and 64-column
block.  Decoding it back here -- independently of the library, from the
documented sections -- must give the original ternary matrix for ragged
shapes, and its size must be the masks plus the sign bits (no per-block byte
padding), i.e. below the 2-bit tiles at realistic sparsity."""
import numpy as np
import pytest

import xtern


def decode_stream(buf, sec, K, N):
    seg_off, mask_off, sign_off = sec
    nb, ng = (K + 63) // 64, (N + 15) // 16
    seg = np.frombuffer(buf[seg_off:seg_off + ng * nb * 4].tobytes(), np.uint32).reshape(ng, nb)
    msk = np.frombuffer(buf[mask_off:mask_off + ng * nb * 128].tobytes(), np.uint64).reshape(ng, nb, 16)
    words = np.frombuffer(buf[sign_off:].tobytes(), np.uint32)
    bits = np.unpackbits(words.view(np.uint8), bitorder="little")
    w = np.zeros((ng * 16, nb * 64), np.int8)
    for G in range(ng):
        for b in range(nb):
            pos = int(seg[G, b])
            for j in range(16):
                m = int(msk[G, b, j])
                for lane in range(64):
                    if (m >> lane) & 1:
                        w[G * 16 + j, b * 64 + lane] = -1 if bits[pos] else 1
                        pos += 1
            if b + 1 < nb:
                assert pos == int(seg[G, b + 1]), "segments follow each other"
    return w[:N, :K], msk, seg


def ternary(rng, N, K, p0):
    return np.where(rng.random((N, K)) < p0, 0, np.where(rng.random((N, K)) < 0.5, -1, 1)).astype(np.int8)


@pytest.mark.parametrize("K,N,p0", [(64, 1, 0.5), (100, 15, 0.3), (256, 16, 0.7), (300, 17, 0.5),
                                    (130, 50, 0.0), (64, 33, 1.0), (1000, 40, 0.5)])
def test_stream_layout_round_trip(K, N, p0):
    rng = np.random.default_rng(K * 131 + N)
    t = ternary(rng, N, K, p0)
    blob = xtern.encode_sparse_tensor(t, K, N)[0]
    buf, sec = xtern.xorsparse_stream_host(K, N, blob)
    w, msk, seg = decode_stream(buf, sec, K, N)
    assert np.array_equal(w, t)
    # rows past N carry empty masks; sections are 256-byte aligned, in order
    ng = (N + 15) // 16
    assert not msk.transpose(0, 2, 1).reshape(ng * 16, -1)[N:].any()
    assert sec[0] == 0 and sec[1] % 256 == 0 and sec[2] % 256 == 0 and sec[0] < sec[1] < sec[2]
    # the sign stream is exactly the set bits (+ the 3-word read-ahead)
    nnz = int((t != 0).sum())
    assert buf.size - sec[2] == 4 * ((nnz + 31) // 32 + 3)


def test_stream_is_smaller_than_tiles():
    """C3-like sparsity (zero fraction 0.3-0.7 per block): masks + signs come
    to about 0.77x the 2-bit tiles, the same as the blob itself."""
    K, N = 4096, 256
    rng = np.random.default_rng(7)
    p0 = rng.uniform(0.3, 0.7, size=(N, K // 64)).repeat(64, axis=1)
    t = np.where(rng.random((N, K)) < p0, 0, np.where(rng.random((N, K)) < 0.5, -1, 1)).astype(np.int8)
    blob = xtern.encode_sparse_tensor(t, K, N)[0]
    buf, _ = xtern.xorsparse_stream_host(K, N, blob)
    tiles = xtern.tile_bytes(xtern.XT_XORSPARSE, K, N)
    assert buf.size < 0.8 * tiles
    assert abs(buf.size - len(blob)) < 0.06 * len(blob)


def test_stream_rejects_bad_blobs():
    t = np.ones((2, 64), np.int8)
    blob = bytearray(xtern.encode_sparse_tensor(t, 64, 2)[0])
    with pytest.raises(xtern.XternError, match="truncated"):
        xtern.xorsparse_stream_host(64, 2, bytes(blob[:-1]))
    bad = bytearray(blob)
    bad[0] = 2  # num_blocks of row 0
    with pytest.raises(xtern.XternError, match="num_blocks"):
        xtern.xorsparse_stream_host(64, 2, bytes(bad))
    with pytest.raises(xtern.XternError, match="beyond in_dim"):
        xtern.xorsparse_stream_host(60, 2, bytes(blob))
