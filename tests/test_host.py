"""CPU tests of libxtern's host side: the library loads and exports every
symbol include/xtern.h declares, the load-time repack into the device tile
layout is lossless for Pack4 / Pack5 / XorSparse (checked by an independent
numpy decoder of the documented tile geometry), argument errors come back as
statuses with messages, and the Python mirror's codecs equal the oracle's."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
import xtern

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exports_every_declared_symbol():
    hdr = open(os.path.join(ROOT, "include", "xtern.h")).read()
    names = set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(xt_[a-z_0-9]+)\s*\(", hdr, re.M))
    assert len(names) >= 12, names
    lib = xtern.lib()
    for n in sorted(names):
        assert hasattr(lib, n), f"libxtern.so does not export {n}"
    assert "gfx950" in xtern.version()


def decode_tiles(tiles, fmt, K, N):
    """Independent decoder of the device tile layout -> ternary [N, K]."""
    if fmt == xtern.XT_PACK5:
        ch, steps = 320, 5
    else:
        ch, steps = 256, 4
    nch, ng = -(-K // ch), -(-N // 16)
    t = tiles.reshape(ng, nch, 4, 16, 16)  # G, c, g, j, byte
    out = np.zeros((ng * 16, nch * ch), np.int8)
    G, c, g, j = np.meshgrid(np.arange(ng), np.arange(nch), np.arange(4), np.arange(16),
                             indexing="ij")
    rows = G * 16 + j
    if fmt == xtern.XT_PACK5:
        x = t.astype(np.uint32)
        for s in range(5):
            y = x * 3
            trit = (y >> 8).astype(np.int8)
            x = y & 255
            for b in range(16):
                cols = c * ch + s * 64 + g * 16 + b
                out[rows, cols] = trit[..., b] - 1
    else:
        dw = t.reshape(ng, nch, 4, 16, 4, 4).astype(np.uint32)
        dw = dw[..., 0] | (dw[..., 1] << 8) | (dw[..., 2] << 16) | (dw[..., 3] << 24)
        for s in range(4):
            for jj in range(4):
                for d in range(4):
                    code = ((dw[..., s] >> (8 * d + 2 * jj)) & 3).astype(np.int8)
                    assert not np.any(code == 3), "code 11 must be canonicalised"
                    cols = c * ch + s * 64 + g * 16 + 4 * jj + d
                    out[rows, cols] = code - 1
    return out


SHAPES = [(256, 16), (2560, 48), (300, 37), (5, 3), (640, 20), (1000, 17)]


@pytest.mark.parametrize("K,N", SHAPES)
def test_repack_pack4_lossless(K, N):
    rng = np.random.default_rng(K * 7 + N)
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    packed = np.concatenate([xtern.pack_ternary4(r) for r in t])
    tiles = xtern.repack_host(xtern.XT_PACK4, K, N, packed)
    dec = decode_tiles(tiles, xtern.XT_PACK4, K, N)
    assert np.array_equal(dec[:N, :K], t)
    assert not dec[N:, :].any() and not dec[:, K:].any()  # padding is weight 0


def test_repack_pack4_code11_is_zero():
    K, N = 64, 1
    packed = np.full(16, 0xFF, np.uint8)
    dec = decode_tiles(xtern.repack_host(xtern.XT_PACK4, K, N, packed), xtern.XT_PACK4, K, N)
    assert not dec.any()


@pytest.mark.parametrize("K,N", SHAPES + [(3200, 16), (321, 2)])
def test_repack_pack5_lossless(K, N):
    rng = np.random.default_rng(K * 11 + N)
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    packed = np.concatenate([xtern.pack_ternary5(r) for r in t])
    tiles = xtern.repack_host(xtern.XT_PACK5, K, N, packed)
    dec = decode_tiles(tiles, xtern.XT_PACK5, K, N)
    assert np.array_equal(dec[:N, :K], t)
    assert not dec[N:, :].any() and not dec[:, K:].any()


def test_repack_pack5_invalid_bytes_follow_reference():
    # bytes 243..255 are never packed; the reference decodes them with %3 /3
    # (quantization.rs:72-91), which the repack reproduces
    K, N = 5 * 13, 1
    packed = np.arange(243, 256, dtype=np.uint8)
    dec = decode_tiles(xtern.repack_host(xtern.XT_PACK5, K, N, packed), xtern.XT_PACK5, K, N)
    assert np.array_equal(dec[0, :K], oracle.unpack5(packed, K).astype(np.int8))


@pytest.mark.parametrize("K,N", SHAPES)
def test_repack_sparse_lossless(K, N):
    rng = np.random.default_rng(K * 13 + N)
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    blob, _ = oracle.sparse_encode_tensor(t, K, N)
    dec = decode_tiles(xtern.repack_host(xtern.XT_XORSPARSE, K, N, blob), xtern.XT_PACK4, K, N)
    assert np.array_equal(dec[:N, :K], t)


def test_sparse_encoder_matches_oracle():
    rng = np.random.default_rng(5)
    for K, N in ((64, 3), (70, 4), (300, 9), (1, 2)):
        t = rng.integers(-1, 2, (N, K)).astype(np.int8)
        t[0] = 0
        blob, offs = xtern.encode_sparse_tensor(t, K, N)
        blob_o, offs_o = oracle.sparse_encode_tensor(t, K, N)
        assert blob == blob_o and offs == offs_o


def test_packers_match_oracle():
    rng = np.random.default_rng(6)
    for n in (1, 4, 5, 17, 640, 1001):
        w = (rng.standard_normal(n) * 1.2).astype(np.float32)
        w[:3] = [0.5, -0.5, 1.5][: min(3, n)]
        for scale in (1.0, 0.7, 2.5, 0.0):
            assert np.array_equal(xtern.pack_1_58bit_4pack(w, scale), oracle.pack4(w, scale))
            assert np.array_equal(xtern.pack_1_58bit_5pack(w, scale), oracle.pack5(w, scale))
        p4, p5 = oracle.pack4(w), oracle.pack5(w)
        assert np.array_equal(xtern.unpack_1_58bit_4pack(p4, n), oracle.unpack4(p4, n))
        assert np.array_equal(xtern.unpack_1_58bit_5pack(p5, n), oracle.unpack5(p5, n))


# ------------------------------------------------------------ error paths ---

def _raw_repack(fmt, K, N, buf):
    lib = xtern.lib()
    src = np.frombuffer(bytes(buf), np.uint8) if len(buf) else np.zeros(1, np.uint8)
    out = np.zeros(max(1, xtern.tile_bytes(fmt, max(K, 1), max(N, 1))), np.uint8)
    rc = lib.xt_repack_host(fmt, K, N, src.ctypes.data_as(ctypes.c_void_p), len(buf),
                            out.ctypes.data_as(ctypes.c_void_p))
    return rc, lib.xt_last_error().decode()


def test_error_short_pack4():
    rc, msg = _raw_repack(xtern.XT_PACK4, 64, 2, bytes(31))
    assert rc == xtern.XT_ERR_INVALID and "Pack4" in msg and "32" in msg


def test_error_short_pack5():
    rc, msg = _raw_repack(xtern.XT_PACK5, 10, 2, bytes(3))
    assert rc == xtern.XT_ERR_INVALID and "Pack5" in msg


def test_error_bad_format_and_dims():
    rc, msg = _raw_repack(7, 64, 2, bytes(64))
    assert rc == xtern.XT_ERR_INVALID and "format" in msg
    rc, msg = _raw_repack(0, 0, 2, bytes(64))
    assert rc == xtern.XT_ERR_INVALID and "positive" in msg


def test_error_sparse_malformed():
    blob = oracle.sparse_encode_row(np.ones(64, np.int8), 64)
    rc, msg = _raw_repack(xtern.XT_XORSPARSE, 64, 1, blob[:-1])
    assert rc == xtern.XT_ERR_INVALID and "truncated" in msg
    rc, msg = _raw_repack(xtern.XT_XORSPARSE, 128, 1, blob)
    assert rc == xtern.XT_ERR_INVALID and "num_blocks" in msg
    bad = bytearray(oracle.sparse_encode_row(np.zeros(60, np.int8), 60))
    bad[4 + 7] = 0x80  # lane 63 set although in_dim = 60
    bad += b"\x00"    # its sign byte
    rc, msg = _raw_repack(xtern.XT_XORSPARSE, 60, 1, bytes(bad))
    assert rc == xtern.XT_ERR_INVALID and "beyond" in msg


def test_error_null_handle_and_args():
    lib = xtern.lib()
    assert lib.xt_ternary_linear_q(None, None, None, 1, None, None, None) == xtern.XT_ERR_INVALID
    assert "NULL" in lib.xt_last_error().decode()
    h = ctypes.c_void_p()
    assert lib.xt_weights_create(0, 64, 1, None, 0, None, ctypes.byref(h)) == xtern.XT_ERR_INVALID
    assert lib.xt_quantize_i8(None, 1, 0, None, None, 0, None) == xtern.XT_ERR_INVALID
    assert lib.xt_quantize_i8(None, 1, 16, None, None, 9, None) == xtern.XT_ERR_INVALID
    assert lib.xt_weights_destroy(None) == xtern.XT_OK


def test_tile_bytes():
    assert xtern.tile_bytes(xtern.XT_PACK4, 2560, 6912) == 432 * 10 * 1024
    assert xtern.tile_bytes(xtern.XT_PACK5, 3200, 8640) == 540 * 10 * 1024
    assert xtern.tile_bytes(xtern.XT_XORSPARSE, 4096, 14336) == 896 * 16 * 1024
    assert xtern.tile_bytes(0, 0, 5) == 0


def test_stack_create_rejects_null_weights_on_cpu():
    """xt_stack_create validates every op before any device call: a NULL
    weight handle (first or later projection) or output is an argument error,
    not a crash."""
    for bad in range(3):
        arr = (xtern._StackOp * 1)()
        arr[0].n = 2
        arr[0].x = 0x1000
        arr[0].dep = -1
        arr[0].y[0] = 0x2000
        arr[0].y[1] = 0x3000
        if bad == 0:
            arr[0].w[1] = 0x4000            # w[0] NULL
        elif bad == 1:
            arr[0].w[0] = 0x4000            # w[1] NULL
        else:
            arr[0].w[0] = arr[0].w[1] = 0x4000
            arr[0].y[1] = None              # y[1] NULL
        h = ctypes.c_void_p()
        rc = xtern._lib.xt_stack_create(arr, 1, 1, 0, ctypes.byref(h))
        assert rc == xtern.XT_ERR_INVALID
        assert b"NULL weights or output" in xtern._lib.xt_last_error()


def test_stack_plan_flags_on_cpu():
    """Unknown plan flags in xt_stack_create's mode are an argument error
    found before any device call; xt_stack_plan of NULL is one too."""
    arr = (xtern._StackOp * 1)()
    arr[0].n = 1
    arr[0].x = 0x1000
    arr[0].dep = -1
    arr[0].w[0] = 0x4000
    arr[0].y[0] = 0x2000
    h = ctypes.c_void_p()
    for bad in (xtern.XT_STACK_ONE_LAUNCH | xtern.XT_STACK_PER_OP, 0x400, 0x100 | 7):
        rc = xtern._lib.xt_stack_create(arr, 1, 1, bad, ctypes.byref(h))
        assert rc == xtern.XT_ERR_INVALID
    assert xtern._lib.xt_stack_plan(None) == xtern.XT_ERR_INVALID
