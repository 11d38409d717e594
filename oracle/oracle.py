"""ctypes wrapper of liboracle.so — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker / the timed CPU baseline.  It is a CPU
restatement of xor-net's ternary path (oracle/xtern_oracle.c cites the
reference lines each function follows).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} missing; run `make -C oracle`")
_o = ctypes.CDLL(LIB_PATH)

_vp, _i64 = ctypes.c_void_p, ctypes.c_int64
_o.or_pack4.argtypes = [_vp, _i64, ctypes.c_float, _vp]
_o.or_unpack4.argtypes = [_vp, _i64, _vp]
_o.or_pack5.argtypes = [_vp, _i64, ctypes.c_float, _vp]
_o.or_unpack5.argtypes = [_vp, _i64, _vp]
for f in ("or_quantize_avx512", "or_quantize_scalar"):
    getattr(_o, f).argtypes = [_vp, _i64, _vp]
    getattr(_o, f).restype = ctypes.c_float
for f in ("or_dot_pack4", "or_dot_pack5", "or_dot_pack4_vnni"):
    getattr(_o, f).argtypes = [_vp, _vp, _i64]
    getattr(_o, f).restype = ctypes.c_int32
_o.or_dot_sparse.argtypes = [_vp, _vp, _vp, _i64, _i64]
_o.or_dot_sparse.restype = ctypes.c_int32
_o.or_sparse_row_bytes.argtypes = [_vp, _i64]
_o.or_sparse_row_bytes.restype = _i64
_o.or_sparse_encode_row.argtypes = [_vp, _i64, _vp]
_o.or_sparse_encode_row.restype = _i64
_o.or_sparse_from_blob.argtypes = [_vp, _i64, _i64, _vp, _vp, _i64]
_o.or_sparse_from_blob.restype = _i64
_o.or_sparse_decode_row.argtypes = [_vp, _i64, _i64, _vp]
_o.or_linear_forward.argtypes = [ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp,
                                 _vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
_o.or_linear_forward_q.argtypes = [ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64,
                                   _vp, _vp]
_o.or_hf_destripe.argtypes = [ctypes.c_int, _i64, _i64, _vp, _vp]
_o.or_hf_destripe.restype = ctypes.c_int
_o.or_silu_inplace.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int]
_o.or_act_mul_inplace.argtypes = [_vp, _vp, _i64, ctypes.c_int]
_o.or_rms_norm.argtypes = [_vp, _vp, _i64, ctypes.c_float]
_o.or_rms_norm.restype = ctypes.c_float
_o.or_int_new.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _vp]
_o.or_int_forward.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, ctypes.c_int]
_o.or_lcg_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
_o.or_lcg_next.restype = ctypes.c_uint64
_o.or_cpu_has_vnni.restype = ctypes.c_int
_o.or_cpu_has_avx512f.restype = ctypes.c_int


def _p(a):
    return a.ctypes.data_as(_vp) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(np.asarray(a, dtype=dt))


def pack4(w, scale=1.0):
    w = _c(w, np.float32)
    out = np.zeros((w.size + 3) // 4, np.uint8)
    _o.or_pack4(_p(w), w.size, scale, _p(out))
    return out


def unpack4(b, n):
    b = _c(b, np.uint8)
    out = np.zeros(n, np.float32)
    _o.or_unpack4(_p(b), n, _p(out))
    return out


def pack5(w, scale=1.0):
    w = _c(w, np.float32)
    out = np.zeros((w.size + 4) // 5, np.uint8)
    _o.or_pack5(_p(w), w.size, scale, _p(out))
    return out


def unpack5(b, n):
    b = _c(b, np.uint8)
    out = np.zeros(n, np.float32)
    _o.or_unpack5(_p(b), n, _p(out))
    return out


def quantize(x, mode=0):
    """mode 0: AVX-512 path semantics, 1: scalar path.  Returns (q, inv)."""
    x = _c(x, np.float32)
    q = np.zeros(x.size, np.int8)
    f = _o.or_quantize_avx512 if mode == 0 else _o.or_quantize_scalar
    inv = f(_p(x), x.size, _p(q))
    return q, np.float32(inv)


def dot_pack4(a, w, n):
    return int(_o.or_dot_pack4(_p(_c(a, np.int8)), _p(_c(w, np.uint8)), n))


def dot_pack4_vnni(a, w, n):
    return int(_o.or_dot_pack4_vnni(_p(_c(a, np.int8)), _p(_c(w, np.uint8)), n))


def dot_pack5(a, w, n):
    return int(_o.or_dot_pack5(_p(_c(a, np.int8)), _p(_c(w, np.uint8)), n))


def has_vnni():
    return bool(_o.or_cpu_has_vnni())


def has_avx512f():
    return bool(_o.or_cpu_has_avx512f())


def sparse_encode_row(vals, in_dim):
    v = _c(vals, np.int8)
    out = np.zeros(int(_o.or_sparse_row_bytes(_p(v), in_dim)), np.uint8)
    n = _o.or_sparse_encode_row(_p(v), in_dim, _p(out))
    return out[:n].tobytes()


def sparse_encode_tensor(vals, in_dim, out_dim):
    v = _c(vals, np.int8).reshape(out_dim, in_dim)
    rows = [sparse_encode_row(v[r], in_dim) for r in range(out_dim)]
    offs = np.concatenate([[0], np.cumsum([len(r) for r in rows])[:-1]]).astype(int)
    return b"".join(rows), list(offs)


def sparse_from_blob(blob, out_dim, in_dim):
    """-> (masks [out_dim, nb] u64, signs [out_dim, nb] u64, nb)."""
    b = np.frombuffer(bytes(blob), np.uint8)
    nb = (in_dim + 63) // 64
    masks = np.zeros(out_dim * nb, np.uint64)
    signs = np.zeros(out_dim * nb, np.uint64)
    r = _o.or_sparse_from_blob(_p(b), b.size, out_dim, _p(masks), _p(signs), masks.size)
    if r < 0:
        raise ValueError("XorSparse blob shorter than its headers")
    return masks.reshape(out_dim, nb), signs.reshape(out_dim, nb), int(r)


def sparse_decode_row(blob, off, in_dim):
    b = np.frombuffer(bytes(blob), np.uint8)
    out = np.zeros(in_dim, np.int8)
    _o.or_sparse_decode_row(_p(b), off, in_dim, _p(out))
    return out


def dot_sparse(a, masks, signs, nb, in_dim):
    return int(_o.or_dot_sparse(_p(_c(a, np.int8)), _p(_c(masks, np.uint64)),
                                _p(_c(signs, np.uint64)), nb, in_dim))


def linear_forward(fmt, K, N, x, w_scales, wbytes=None, masks=None, signs=None, quant_mode=0,
                   threads=0, kernel=0):
    """TernaryLinear::forward for x [M, K]; returns (y, q, inv, acc)."""
    x = _c(x, np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.zeros((M, N), np.float32)
    q = np.zeros((M, K), np.int8)
    inv = np.zeros(M, np.float32)
    acc = np.zeros((M, N), np.int32)
    wb = _c(wbytes, np.uint8) if wbytes is not None else None
    mk = _c(masks, np.uint64) if masks is not None else None
    sg = _c(signs, np.uint64) if signs is not None else None
    ws = _c(w_scales, np.float32)
    _o.or_linear_forward(fmt, _p(wb), _p(mk), _p(sg), _p(ws), K, N, _p(x), M, _p(y), _p(q),
                         _p(inv), _p(acc), quant_mode, threads, kernel)
    return y, q, inv, acc


def linear_forward_q(fmt, K, N, q, inv, w_scales, wbytes=None, masks=None, signs=None):
    q = _c(q, np.int8).reshape(-1, K)
    M = q.shape[0]
    inv = _c(inv, np.float32)
    y = np.zeros((M, N), np.float32)
    acc = np.zeros((M, N), np.int32)
    wb = _c(wbytes, np.uint8) if wbytes is not None else None
    mk = _c(masks, np.uint64) if masks is not None else None
    sg = _c(signs, np.uint64) if signs is not None else None
    _o.or_linear_forward_q(fmt, _p(wb), _p(mk), _p(sg), _p(_c(w_scales, np.float32)), K, N,
                           _p(q), _p(inv), M, _p(y), _p(acc))
    return y, acc


def hf_destripe(fmt, in_dim, out_dim, stored):
    """loader/mod.rs:301-394 destripe -> input-dim packed rows."""
    f = 5 if fmt == 1 else 4
    st = _c(stored, np.uint8)
    out = np.zeros(out_dim * ((in_dim + f - 1) // f), np.uint8)
    if _o.or_hf_destripe(fmt, in_dim, out_dim, _p(st), _p(out)) != 0:
        raise ValueError("out_dim must be a multiple of the pack factor")
    return out


def silu_inplace(gate, up, use_silu, avx512=True):
    """quantization::silu_inplace on each row of gate/up [..., n]; returns a copy."""
    g = _c(gate, np.float32).copy()
    u = _c(up, np.float32)
    n = g.shape[-1]
    g2, u2 = g.reshape(-1, n), u.reshape(-1, n)
    for r in range(g2.shape[0]):
        _o.or_silu_inplace(_p(g2[r]), _p(u2[r]), n, int(use_silu), int(avx512))
    return g


def act_mul(x, up, use_silu):
    """FastTensor::silu_mul_inplace / relu2_mul_inplace; returns a copy."""
    g = _c(x, np.float32).copy()
    u = _c(up, np.float32)
    _o.or_act_mul_inplace(_p(g), _p(u), g.size, int(use_silu))
    return g


def rms_norm(x, w, eps):
    """rms_norm on each row of x [..., n]; returns (normed copy, row sums of squares)."""
    y = _c(x, np.float32).copy()
    n = y.shape[-1]
    y2 = y.reshape(-1, n)
    wv = _c(w, np.float32)
    sums = np.array([_o.or_rms_norm(_p(y2[r]), _p(wv), n, eps) for r in range(y2.shape[0])],
                    np.float32)
    return y, sums


def mlp_forward(x, gate, up, down, norm_w, eps, use_silu, quant_mode=0, fused=None):
    """Mlp::forward (models/llama/mlp.rs:43-128) for all-ternary projections.

    gate/up/down: (fmt, K, N, w_scales, dict(wbytes=... | masks=..., signs=...)).
    fused=None follows the reference's dispatch: one token -> fused_mlp_all
    (layers.rs:497-645: silu_inplace, optional norm, quantise, down); several
    tokens -> the fallback (silu_mul_inplace / relu2_mul_inplace, norm,
    c_proj.forward).  Returns (y, mid_q, mid_inv)."""
    x = _c(x, np.float32)
    K = gate[1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if fused is None:
        fused = (M == 1)
    g = linear_forward(gate[0], gate[1], gate[2], x2, gate[3], quant_mode=quant_mode, **gate[4])[0]
    u = linear_forward(up[0], up[1], up[2], x2, up[3], quant_mode=quant_mode, **up[4])[0]
    if fused:
        mid = silu_inplace(g, u, use_silu, avx512=(quant_mode == 0))
    else:
        mid = act_mul(g, u, use_silu)
    if norm_w is not None:
        mid, _ = rms_norm(mid, norm_w, eps)
    y, q, inv, _ = linear_forward(down[0], down[1], down[2], mid, down[3], quant_mode=quant_mode,
                                  **down[4])
    return y.reshape(x.shape[:-1] + (down[2],)), q, inv


def sparse_container_serialize(entries):
    """SparseFile::serialize (src/loader/sparse_loader.rs:124-139):
    entries = [(name, out_dim, in_dim, w_scale, blob)]."""
    import struct
    out = bytearray(b"XORSPARE1")
    out += struct.pack("<I", 1)
    out += struct.pack("<I", len(entries))
    for name, od, idim, ws, blob in entries:
        nb = name.encode()
        out += struct.pack("<I", len(nb)) + nb
        out += struct.pack("<IIfI", od, idim, ws, len(blob))
        out += bytes(blob)
    return bytes(out)


def sparse_container_parse(data):
    """The layout serialize writes (SPARSE_FORMAT.md:30-50): a dict
    name -> (out_dim, in_dim, w_scale, blob); later duplicates win."""
    import struct
    if data[:9] != b"XORSPARE1":
        raise ValueError("bad magic")
    ver, n = struct.unpack_from("<II", data, 9)
    if ver != 1:
        raise ValueError("version")
    p, out = 17, {}
    for _ in range(n):
        (nl,) = struct.unpack_from("<I", data, p)
        name = data[p + 4:p + 4 + nl].decode()
        p += 4 + nl
        od, idim, ws, bl = struct.unpack_from("<IIfI", data, p)
        p += 16
        out[name] = (od, idim, ws, bytes(data[p:p + bl]))
        p += bl
    return out


def convert_sparse_tensor(stored, in_dim, out_dim, destripe=True):
    """convert_sparse.rs:101-105 for one Pack4 tensor: the linear unpack of
    the stored bytes (destripe=False, as the reference does) or the
    get_prepacked_ternary destripe (loader/mod.rs:351-390), then
    encode_sparse_tensor (sparse.rs:90-103).  Returns the blob."""
    if destripe:
        packed = hf_destripe(0, in_dim, out_dim, stored)
        vals = np.concatenate([unpack4(packed[o * ((in_dim + 3) // 4):(o + 1) * ((in_dim + 3) // 4)],
                                       in_dim) for o in range(out_dim)])
    else:
        vals = unpack4(np.asarray(stored, np.uint8).ravel(), in_dim * out_dim)
    return sparse_encode_tensor(vals.astype(np.int8), in_dim, out_dim)[0]


def int_new(bits, w, N, K):
    """Int8Linear::new / Int4Linear::new: (weight bytes, scales)."""
    wv = _c(w, np.float32).reshape(N, K)
    out = np.zeros(N * (K if bits == 8 else (K + 1) // 2), np.uint8)
    sc = np.zeros(N, np.float32)
    _o.or_int_new(bits, _p(wv), N, K, _p(out), _p(sc))
    return out, sc


def int_forward(bits, wbytes, scales, K, N, x, quant_mode=0):
    """Int8Linear::forward / Int4Linear::forward: (y, acc)."""
    xv = _c(x, np.float32).reshape(-1, K)
    M = xv.shape[0]
    y = np.zeros((M, N), np.float32)
    acc = np.zeros((M, N), np.int32)
    _o.or_int_forward(bits, _p(_c(wbytes, np.uint8)), _p(_c(scales, np.float32)), K, N, _p(xv), M,
                      _p(y), _p(acc), quant_mode)
    return y, acc


class Lcg:
    """The reference's test RNG (simd.rs:556-565)."""

    def __init__(self, seed):
        self.s = ctypes.c_uint64(seed)

    def next(self):
        return int(_o.or_lcg_next(ctypes.byref(self.s)))

    def below(self, n):
        return self.next() % n
