"""xtern — Python mirror of xor-net's bit1_58 ternary linear API on MI355X.

The compute path is libxtern.so (hand-written HIP for gfx950) reached through
its C ABI (include/xtern.h) with ctypes.  PyTorch is only used for device
memory and streams.  There is no CPU fallback: importing this package raises
if libxtern.so is missing, and every compute call raises XternError on a
failed status.

Mirrored reference API (paths relative to xor-net):
  TernaryPackType                 src/bit1_58/quantization.rs:1-5
  pack_1_58bit_4pack / 5pack      src/bit1_58/quantization.rs:7-91
  quantize_f32_to_i8              src/bit1_58/quantization.rs:170-195
  encode_sparse_row_into /
  encode_sparse_tensor            src/bit1_58/sparse.rs:61-103
  TernaryLinear                   src/bit1_58/layers.rs:34-750
  DynamicLinear (Ternary arm)     src/nn/dynamic_linear.rs:610-680
"""
import ctypes
import enum
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libxtern.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libxtern.so not found at {LIB_PATH}; build it with "
        "`python xor-net_amd/build_lib.py` (or __graft_entry__.build())")

# torch bundles its own HIP runtime.  Loading libxtern.so first would bring
# ROCm's copy into the process ahead of torch's and the two then disagree
# about the device ("No HIP GPUs are available" / "no ROCm-capable device").
# Importing torch first makes libxtern bind to the runtime torch already
# loaded, so both share one device context.
try:
    import torch as _torch_mod  # noqa: F401
except ImportError:  # the C ABI itself does not need torch
    _torch_mod = None

_lib = ctypes.CDLL(LIB_PATH)

XT_INT8 = 3
XT_INT4 = 4

XT_ACT_RELU2_MUL = 0
XT_ACT_SILU_INPLACE_AVX512 = 1
XT_ACT_SILU_INPLACE_SCALAR = 2
XT_ACT_SILU_MUL = 3

XT_OK = 0
XT_ERR_INVALID = -1
XT_ERR_HIP = -2
XT_ERR_NOMEM = -3
XT_ERR_UNSUPPORTED = -4

XT_PACK4, XT_PACK5, XT_XORSPARSE = 0, 1, 2
XT_XORSPARSE_STREAM = 5   # the XorSparse blob kept compact on the device
XT_QUANT_AVX512, XT_QUANT_SCALAR = 0, 1
XT_STACK_AUTO, XT_STACK_ONE_LAUNCH, XT_STACK_PER_OP = 0, 256, 512

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

_lib.xt_version.restype = ctypes.c_char_p
_lib.xt_last_error.restype = ctypes.c_char_p
_lib.xt_weights_create.argtypes = [ctypes.c_int, _i64, _i64, _vp, _sz, _vp, ctypes.POINTER(_vp)]
_lib.xt_weights_destroy.argtypes = [_vp]
_lib.xt_weights_info.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_i64),
                                 ctypes.POINTER(_i64), ctypes.POINTER(_sz)]
_lib.xt_tile_bytes.argtypes = [ctypes.c_int, _i64, _i64]
_lib.xt_tile_bytes.restype = _sz
_lib.xt_repack_host.argtypes = [ctypes.c_int, _i64, _i64, _vp, _sz, _vp]
_lib.xt_xorsparse_stream_host.argtypes = [_i64, _i64, _vp, _sz, _vp, _sz, ctypes.POINTER(_sz),
                                          ctypes.POINTER(ctypes.c_uint64)]
_lib.xt_hf_destripe.argtypes = [ctypes.c_int, _i64, _i64, _vp, _sz, _vp]
_lib.xt_weights_create_hf.argtypes = [ctypes.c_int, _i64, _i64, _vp, _sz, ctypes.c_float,
                                      ctypes.c_int, ctypes.POINTER(_vp)]
_lib.xt_weights_read_tiles.argtypes = [_vp, _vp, _sz]
_lib.xt_activation_mul.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _vp, _vp]
_lib.xt_rms_norm.argtypes = [_vp, _vp, _i64, _i64, ctypes.c_float, _vp, _vp]
_lib.xt_ternary_mlp_q.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_float, ctypes.c_int, _vp, _vp,
                                  _i64, _vp, ctypes.c_int, _vp]
_lib.xt_ternary_mlp_f32.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_float, ctypes.c_int, _vp, _i64,
                                    _vp, ctypes.c_int, _vp]
_lib.xt_sparse_file_open.argtypes = [_vp, _sz, ctypes.POINTER(_vp)]
_lib.xt_sparse_file_close.argtypes = [_vp]
_lib.xt_sparse_file_count.argtypes = [_vp, ctypes.POINTER(_i64)]
_lib.xt_sparse_file_entry.argtypes = [_vp, _i64, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                      ctypes.POINTER(ctypes.c_float), ctypes.POINTER(_vp),
                                      ctypes.POINTER(_sz)]
_lib.xt_sparse_file_find.argtypes = [_vp, ctypes.c_char_p, ctypes.POINTER(_i64)]
_lib.xt_weights_create_from_sparse_file.argtypes = [_vp, ctypes.c_char_p, _i64, _i64,
                                                    ctypes.POINTER(_vp)]
_lib.xt_sparse_file_serialized_size.argtypes = [_i64, _vp, _vp]
_lib.xt_sparse_file_serialized_size.restype = _sz
_lib.xt_sparse_file_serialize.argtypes = [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz]
_lib.xt_hf_to_sparse_blob.argtypes = [ctypes.c_int, _i64, _i64, _vp, _sz, ctypes.c_int, _vp, _sz,
                                      ctypes.POINTER(_sz)]
_lib.xt_int_quantize_host.argtypes = [ctypes.c_int, _vp, _i64, _i64, _vp, _vp]
_lib.xt_quantize_i8.argtypes = [_vp, _i64, _i64, _vp, _vp, ctypes.c_int, _vp]
_lib.xt_quantize_i8_rowsum.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, ctypes.c_int, _vp]
_lib.xt_ternary_linear_q.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp, _vp]
_lib.xt_ternary_linear_q_rowsum.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp]
_lib.xt_ternary_linear_f32.argtypes = [_vp, _vp, _i64, _vp, ctypes.c_int, _vp]
_lib.xt_ternary_linear_multi_q.argtypes = [_vp, ctypes.c_int, _vp, _vp, _i64, _vp, _vp]
_lib.xt_workspace_release.argtypes = []
_lib.xt_ternary_linear_f32_noalloc.argtypes = [_vp, _vp, _i64, _vp, ctypes.c_int, _vp]
_lib.xt_ternary_linear_multi_f32.argtypes = [_vp, ctypes.c_int, _vp, _i64, _vp, ctypes.c_int, _vp]


class _StackOp(ctypes.Structure):
    """struct xt_stack_op (include/xtern.h)."""
    _fields_ = [("w", _vp * 4), ("n", ctypes.c_int), ("x", _vp), ("y", _vp * 4),
                ("dep", ctypes.c_int)]


_lib.xt_stack_create.argtypes = [ctypes.POINTER(_StackOp), ctypes.c_int, _i64, ctypes.c_int,
                                 ctypes.POINTER(_vp)]
_lib.xt_stack_run.argtypes = [_vp, _vp]
_lib.xt_stack_plan.argtypes = [_vp]
_lib.xt_stack_check.argtypes = [_vp, ctypes.POINTER(ctypes.c_int)]
_lib.xt_stack_destroy.argtypes = [_vp]


class XternError(RuntimeError):
    """A libxtern call returned a negative status (message from xt_last_error)."""

    def __init__(self, code, msg):
        super().__init__(f"xtern error {code}: {msg}")
        self.code = code


def _check(rc):
    if rc != XT_OK:
        raise XternError(rc, _lib.xt_last_error().decode())


def version():
    return _lib.xt_version().decode()


def lib():
    """The loaded ctypes library (for tests of the raw ABI)."""
    return _lib


# ---------------------------------------------------------------------------
# Formats and host-side codecs (load-time work, as in the reference)
# ---------------------------------------------------------------------------

class TernaryPackType(enum.Enum):
    """quantization.rs:1-5."""
    Pack4 = XT_PACK4
    Pack5 = XT_PACK5


def _ternarise(w, w_scale):
    """Per-weight rule of quantization.rs:12-21: clamp(round_half_away(w/s), -1, 1),
    then < -0.5 -> -1, > 0.5 -> +1, else 0; s <= 0 gives 0; NaN gives -1."""
    w = np.asarray(w, dtype=np.float32)
    if w_scale > 0:
        scaled = (w / np.float32(w_scale)).astype(np.float32)
    else:
        scaled = np.zeros_like(w)
    # Rust f32::round: half away from zero (trunc, then step on |frac| >= 0.5;
    # both operations are exact in f32).
    whole = np.trunc(scaled)
    r = whole + np.where(np.abs(scaled - whole) >= 0.5, np.sign(scaled), 0).astype(np.float32)
    q = np.where(np.isnan(scaled), np.float32(-1.0), np.clip(r, -1, 1))
    return np.where(q < -0.5, -1, np.where(q > 0.5, 1, 0)).astype(np.int8)


def pack_ternary4(t):
    """Ternary values (int8 in {-1,0,1}, one row) -> Pack4 bytes (quantization.rs:7-27)."""
    t = np.asarray(t, dtype=np.int8).ravel()
    n = t.size
    codes = np.where(t < 0, 0, np.where(t > 0, 2, 1)).astype(np.uint8)
    padded = np.zeros(((n + 3) // 4) * 4, dtype=np.uint8)
    padded[:n] = codes
    g = padded.reshape(-1, 4)
    return (g[:, 0] | (g[:, 1] << 2) | (g[:, 2] << 4) | (g[:, 3] << 6)).astype(np.uint8)


def pack_ternary5(t):
    """Ternary values -> Pack5 bytes (quantization.rs:48-70); a short last group
    only sums the trits it has."""
    t = np.asarray(t, dtype=np.int8).ravel()
    n = t.size
    digits = np.zeros(((n + 4) // 5) * 5, dtype=np.uint32)
    digits[:n] = np.where(t < 0, 0, np.where(t > 0, 2, 1))
    g = digits.reshape(-1, 5)
    return (g[:, 0] + 3 * g[:, 1] + 9 * g[:, 2] + 27 * g[:, 3] + 81 * g[:, 4]).astype(np.uint8)


def pack_1_58bit_4pack(weights, w_scale):
    """quantization.rs:7-27."""
    return pack_ternary4(_ternarise(weights, w_scale))


def pack_1_58bit_5pack(weights, w_scale):
    """quantization.rs:48-70."""
    return pack_ternary5(_ternarise(weights, w_scale))


def unpack_1_58bit_4pack(packed, n):
    """quantization.rs:29-46 (code 11 reads as 0)."""
    packed = np.asarray(packed, dtype=np.uint8)
    codes = np.stack([(packed >> (2 * j)) & 3 for j in range(4)], axis=1).ravel()[:n]
    return np.where(codes == 0, -1.0, np.where(codes == 2, 1.0, 0.0)).astype(np.float32)


def unpack_1_58bit_5pack(packed, n):
    """quantization.rs:72-91."""
    b = np.asarray(packed, dtype=np.uint32)
    digits = np.stack([(b // 3 ** j) % 3 for j in range(5)], axis=1).ravel()[:n]
    return np.where(digits == 0, -1.0, np.where(digits == 2, 1.0, 0.0)).astype(np.float32)


def encode_sparse_tensor(vals, in_dim, out_dim):
    """[out_dim*in_dim] ternary -> (blob, row_offsets) (sparse.rs:61-103).

    Per row: u32 num_blocks; per 64-block: u64 mask (bit i: lane i non-zero)
    then ceil(nnz/8) bytes of set-order sign bits (bit j: j-th non-zero is -1),
    all little-endian."""
    v = np.asarray(vals, dtype=np.int8).reshape(out_dim, in_dim)
    nb = (in_dim + 63) // 64
    blk = np.zeros((out_dim, nb * 64), dtype=np.int8)
    blk[:, :in_dim] = v
    blk = blk.reshape(out_dim, nb, 64)
    nz = blk != 0
    lanes = np.arange(64, dtype=np.uint64)
    mask = np.bitwise_or.reduce(np.where(nz, np.uint64(1) << lanes, np.uint64(0)), axis=2)
    rank = (np.cumsum(nz, axis=2) - 1).astype(np.uint64)
    sgn = np.bitwise_or.reduce(
        np.where(nz & (blk < 0), np.uint64(1) << np.minimum(rank, np.uint64(63)), np.uint64(0)),
        axis=2)
    nsb = (nz.sum(axis=2) + 7) // 8                       # [out_dim, nb]
    rec = 8 + nsb                                         # bytes per block record
    row_len = 4 + rec.sum(axis=1)
    row_off = np.concatenate([[0], np.cumsum(row_len)[:-1]]).astype(np.int64)
    out = np.zeros(int(row_len.sum()), dtype=np.uint8)
    hdr = np.frombuffer(np.uint32(nb).tobytes(), dtype=np.uint8)
    out[row_off[:, None] + np.arange(4)] = hdr
    blk_off = (row_off[:, None] + 4 +
               np.concatenate([np.zeros((out_dim, 1), np.int64), np.cumsum(rec, axis=1)[:, :-1]],
                              axis=1))                    # [out_dim, nb]
    mbytes = mask.astype("<u8").view(np.uint8).reshape(out_dim, nb, 8)
    out[blk_off[..., None] + np.arange(8)] = mbytes
    sbytes = sgn.astype("<u8").view(np.uint8).reshape(out_dim, nb, 8)
    keep = np.arange(8)[None, None, :] < nsb[..., None]
    idx = blk_off[..., None] + 8 + np.arange(8)
    out[idx[keep]] = sbytes[keep]
    return out.tobytes(), [int(o) for o in row_off]


def encode_sparse_row(vals, in_dim):
    """One ternary row -> XorSparse row bytes (sparse.rs:61-86)."""
    return encode_sparse_tensor(np.asarray(vals, dtype=np.int8)[:in_dim], in_dim, 1)[0]


# ---------------------------------------------------------------------------
# Device weights and raw entry points
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _stream_ptr(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dev_ptr(t, dtype, what):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise XternError(XT_ERR_INVALID, f"{what} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise XternError(XT_ERR_INVALID, f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise XternError(XT_ERR_INVALID, f"{what} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


class DeviceWeights:
    """Owns an xt_weights handle (device tiles + w_scales)."""

    def __init__(self, fmt, in_dim, out_dim, host_bytes, w_scales):
        buf = np.ascontiguousarray(np.frombuffer(bytes(host_bytes), dtype=np.uint8)
                                   if isinstance(host_bytes, (bytes, bytearray))
                                   else np.asarray(host_bytes, dtype=np.uint8))
        ws = np.ascontiguousarray(np.asarray(w_scales, dtype=np.float32))
        if ws.size != out_dim:
            raise XternError(XT_ERR_INVALID, f"w_scales needs {out_dim} values, got {ws.size}")
        h = ctypes.c_void_p()
        _check(_lib.xt_weights_create(fmt, in_dim, out_dim, buf.ctypes.data_as(_vp), buf.size,
                                      ws.ctypes.data_as(_vp), ctypes.byref(h)))
        self.handle = h
        self.fmt, self.in_dim, self.out_dim = fmt, in_dim, out_dim

    @classmethod
    def from_hf(cls, fmt, in_dim, out_dim, stored, weight_scale, is_inverted_scale=False):
        """xt_weights_create_hf: tiles built on the device from the HF
        checkpoint's output-dim striped bytes [out_dim/f][in_dim]."""
        buf = np.ascontiguousarray(np.asarray(stored, dtype=np.uint8).ravel())
        h = ctypes.c_void_p()
        _check(_lib.xt_weights_create_hf(fmt, in_dim, out_dim, buf.ctypes.data_as(_vp), buf.size,
                                         float(weight_scale), int(bool(is_inverted_scale)),
                                         ctypes.byref(h)))
        self = cls.__new__(cls)
        self.handle = h
        self.fmt, self.in_dim, self.out_dim = fmt, in_dim, out_dim
        return self

    def read_tiles(self):
        """The device tiles (XT_XORSPARSE_STREAM: the stream layout), copied
        to a host uint8 array."""
        n = (self.device_bytes() - 4 * self.out_dim if self.fmt == XT_XORSPARSE_STREAM
             else tile_bytes(self.fmt, self.in_dim, self.out_dim))
        out = np.zeros(n, dtype=np.uint8)
        _check(_lib.xt_weights_read_tiles(self.handle, out.ctypes.data_as(_vp), out.size))
        return out

    def device_bytes(self):
        nb = _sz()
        _check(_lib.xt_weights_info(self.handle, None, None, None, ctypes.byref(nb)))
        return nb.value

    def close(self):
        if self.handle:
            _check(_lib.xt_weights_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def tile_bytes(fmt, in_dim, out_dim):
    return _lib.xt_tile_bytes(fmt, in_dim, out_dim)



def xorsparse_stream_host(in_dim, out_dim, blob):
    """xt_xorsparse_stream_host: the device layout of XT_XORSPARSE_STREAM
    weights built on the host.  Returns (uint8 array, (seg_off, mask_off,
    sign_off))."""
    buf = np.ascontiguousarray(np.frombuffer(bytes(blob), dtype=np.uint8))
    n = _sz()
    sec = (ctypes.c_uint64 * 3)()
    _check(_lib.xt_xorsparse_stream_host(in_dim, out_dim, buf.ctypes.data_as(_vp), buf.size, None, 0,
                                         ctypes.byref(n), sec))
    out = np.zeros(n.value, dtype=np.uint8)
    _check(_lib.xt_xorsparse_stream_host(in_dim, out_dim, buf.ctypes.data_as(_vp), buf.size,
                                         out.ctypes.data_as(_vp), out.size, ctypes.byref(n), sec))
    return out, (int(sec[0]), int(sec[1]), int(sec[2]))

def repack_host(fmt, in_dim, out_dim, host_bytes):
    """Host repack into the device tile layout (no GPU needed)."""
    src = np.ascontiguousarray(np.frombuffer(bytes(host_bytes), dtype=np.uint8))
    out = np.zeros(tile_bytes(fmt, in_dim, out_dim), dtype=np.uint8)
    _check(_lib.xt_repack_host(fmt, in_dim, out_dim, src.ctypes.data_as(_vp), src.size,
                               out.ctypes.data_as(_vp)))
    return out


def int_quantize_host(bits, weights_f32, out_dim, in_dim):
    """xt_int_quantize_host: Int8Linear::new / Int4Linear::new -> (bytes, scales)."""
    w = np.ascontiguousarray(np.asarray(weights_f32, dtype=np.float32).ravel())
    if w.size != out_dim * in_dim:
        raise XternError(XT_ERR_INVALID, "Weight length must match in_dim * out_dim")
    out = np.zeros(out_dim * (in_dim if bits == 8 else (in_dim + 1) // 2), np.uint8)
    sc = np.zeros(out_dim, np.float32)
    _check(_lib.xt_int_quantize_host(bits, w.ctypes.data_as(_vp), out_dim, in_dim,
                                     out.ctypes.data_as(_vp), sc.ctypes.data_as(_vp)))
    return out, sc


def hf_destripe(fmt, in_dim, out_dim, stored):
    """xt_hf_destripe: HF output-dim striped bytes [out_dim/f][in_dim] ->
    input-dim packed rows [out_dim][ceil(in_dim/f)] (loader/mod.rs:351-390)."""
    src = np.ascontiguousarray(np.asarray(stored, dtype=np.uint8).ravel())
    f = 5 if fmt == XT_PACK5 else 4
    out = np.zeros(out_dim * ((in_dim + f - 1) // f), dtype=np.uint8)
    _check(_lib.xt_hf_destripe(fmt, in_dim, out_dim, src.ctypes.data_as(_vp), src.size,
                               out.ctypes.data_as(_vp)))
    return out


def get_prepacked_ternary(stored, stored_dtype, expected_shape, pack_type, weight_scale,
                          is_inverted_scale):
    """VarBuilder::get_prepacked_ternary (loader/mod.rs:301-394) on an
    already-read tensor: `stored` is the checkpoint array (its shape is the
    stored shape), `stored_dtype` its safetensors dtype name, `weight_scale`
    the first element of the companion weight_scale tensor as f32.  Returns
    (packed input-dim bytes, w_scales, in_dim, out_dim) like the reference."""
    out_dim, in_dim = int(expected_shape[0]), int(expected_shape[1])
    f = 4 if pack_type == TernaryPackType.Pack4 else 5
    shape = tuple(np.shape(stored))
    if not (stored_dtype == "U8" and len(shape) == 2 and shape[1] == in_dim
            and shape[0] * f == out_dim):
        raise XternError(XT_ERR_INVALID, "Tensor is not in pre-packed U8 ternary format")
    s = np.float32(weight_scale)
    ws = np.float32(1.0) / s if is_inverted_scale else s
    packed = hf_destripe(pack_type.value, in_dim, out_dim, stored)
    return packed, np.full(out_dim, ws, dtype=np.float32), in_dim, out_dim


class SparseFile:
    """sparse_loader.rs:34-140 — a parsed XorSparse container (xt_sparse_file)."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def from_bytes(cls, data):
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        h = ctypes.c_void_p()
        _check(_lib.xt_sparse_file_open(buf.ctypes.data_as(_vp), buf.size, ctypes.byref(h)))
        return cls(h)

    @classmethod
    def open(cls, path):
        with open(path, "rb") as f:
            return cls.from_bytes(f.read())

    def __len__(self):
        n = _i64()
        _check(_lib.xt_sparse_file_count(self.handle, ctypes.byref(n)))
        return n.value

    def entry(self, idx):
        """(name, out_dim, in_dim, w_scale, blob bytes) of entry idx."""
        name, od, idim = ctypes.c_char_p(), _i64(), _i64()
        ws, blob, bl = ctypes.c_float(), _vp(), _sz()
        _check(_lib.xt_sparse_file_entry(self.handle, idx, ctypes.byref(name), ctypes.byref(od),
                                         ctypes.byref(idim), ctypes.byref(ws), ctypes.byref(blob),
                                         ctypes.byref(bl)))
        data = ctypes.string_at(blob.value, bl.value) if bl.value else b""
        return name.value.decode("utf-8", "surrogateescape"), od.value, idim.value, ws.value, data

    def names(self):
        return [self.entry(i)[0] for i in range(len(self))]

    def get_sparse(self, name, in_dim, out_dim):
        """sparse_loader.rs:106-122: (blob, w_scale) after the shape check."""
        idx = _i64()
        _check(_lib.xt_sparse_file_find(self.handle, name.encode(), ctypes.byref(idx)))
        _, od, idim, ws, blob = self.entry(idx.value)
        if od != out_dim or idim != in_dim:
            raise XternError(XT_ERR_INVALID,
                             f"XorSparse '{name}' shape mismatch: expected [{out_dim}, {in_dim}], "
                             f"got [{od}, {idim}]")
        return blob, ws

    def device_weights(self, name, in_dim, out_dim):
        """xt_weights_create_from_sparse_file: the entry uploaded as XorSparse."""
        h = ctypes.c_void_p()
        _check(_lib.xt_weights_create_from_sparse_file(self.handle, name.encode(), in_dim, out_dim,
                                                       ctypes.byref(h)))
        dw = DeviceWeights.__new__(DeviceWeights)
        dw.handle = h
        dw.fmt, dw.in_dim, dw.out_dim = XT_XORSPARSE, in_dim, out_dim
        return dw

    @staticmethod
    def serialize(entries):
        """sparse_loader.rs:124-139: entries = [(name, out_dim, in_dim, w_scale, blob)]."""
        n = len(entries)
        names = (ctypes.c_char_p * max(n, 1))(*[e[0].encode() for e in entries])
        od = (ctypes.c_int64 * max(n, 1))(*[e[1] for e in entries])
        idim = (ctypes.c_int64 * max(n, 1))(*[e[2] for e in entries])
        ws = (ctypes.c_float * max(n, 1))(*[e[3] for e in entries])
        blobs_b = [bytes(e[4]) for e in entries]
        blobs = (ctypes.c_void_p * max(n, 1))(*[ctypes.cast(ctypes.c_char_p(b), ctypes.c_void_p)
                                                 for b in blobs_b])
        lens = (ctypes.c_size_t * max(n, 1))(*[len(b) for b in blobs_b])
        size = _lib.xt_sparse_file_serialized_size(n, names, lens)
        out = np.zeros(size, np.uint8)
        _check(_lib.xt_sparse_file_serialize(n, names, od, idim, ws, blobs, lens,
                                             out.ctypes.data_as(_vp), out.size))
        return out.tobytes()

    def close(self):
        if self.handle:
            _lib.xt_sparse_file_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def hf_to_sparse_blob(fmt, in_dim, out_dim, stored, destripe=True):
    """xt_hf_to_sparse_blob: HF striped U8 bytes -> XorSparse row blob."""
    src = np.ascontiguousarray(np.asarray(stored, dtype=np.uint8).ravel())
    n = _sz()
    _check(_lib.xt_hf_to_sparse_blob(fmt, in_dim, out_dim, src.ctypes.data_as(_vp), src.size,
                                     int(bool(destripe)), None, 0, ctypes.byref(n)))
    out = np.zeros(n.value, np.uint8)
    _check(_lib.xt_hf_to_sparse_blob(fmt, in_dim, out_dim, src.ctypes.data_as(_vp), src.size,
                                     int(bool(destripe)), out.ctypes.data_as(_vp), out.size,
                                     ctypes.byref(n)))
    return out.tobytes()


def convert_sparse(tensors, invert=True, destripe=True):
    """convert_sparse (src/bin/convert_sparse.rs:86-139) over already-read
    checkpoint tensors: `tensors` maps names to arrays; every 2-D uint8
    `*.weight` with a `<name>_scale` companion is converted (Pack4, out_dim =
    4 * stored rows) with scale 1/s (invert) or s.  Returns the container
    bytes.  destripe=False reproduces the reference converter's row order."""
    entries = []
    for name in sorted(tensors):
        arr = np.asarray(tensors[name])
        if not name.endswith(".weight") or arr.dtype != np.uint8 or arr.ndim != 2:
            continue
        sk = name + "_scale"
        if sk not in tensors:
            continue
        stored_out, in_dim = arr.shape
        out_dim = stored_out * 4
        if out_dim == 0 or in_dim == 0:
            continue
        s = np.float32(np.asarray(tensors[sk], dtype=np.float32).ravel()[0])
        ws = np.float32(1.0) / s if invert else s
        blob = hf_to_sparse_blob(XT_PACK4, in_dim, out_dim, arr, destripe=destripe)
        entries.append((name, out_dim, in_dim, float(ws), blob))
    if not entries:
        raise XternError(XT_ERR_INVALID, "no packed-ternary weight tensors found to convert")
    return SparseFile.serialize(entries)


def quantize_i8(x, mode=XT_QUANT_AVX512, stream=None):
    """Device quantize_f32_to_i8 over the rows of x [M, K] (or [K]).
    Returns (q int8 [M, K], inv_scale f32 [M])."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    inv = torch.empty((M,), dtype=torch.float32, device=x.device)
    _check(_lib.xt_quantize_i8(_dev_ptr(x2, torch.float32, "x"), M, K,
                               _dev_ptr(q, torch.int8, "q"), _dev_ptr(inv, torch.float32, "inv"),
                               mode, _stream_ptr(stream)))
    return q, inv


def quantize_i8_rowsum(x, mode=XT_QUANT_AVX512, stream=None):
    """quantize_i8 plus the exact i32 row sums of q (an xtern extension)."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    inv = torch.empty((M,), dtype=torch.float32, device=x.device)
    rs = torch.empty((M,), dtype=torch.int32, device=x.device)
    _check(_lib.xt_quantize_i8_rowsum(_dev_ptr(x2, torch.float32, "x"), M, K,
                                      _dev_ptr(q, torch.int8, "q"),
                                      _dev_ptr(inv, torch.float32, "inv"),
                                      _dev_ptr(rs, torch.int32, "rowsum"), mode,
                                      _stream_ptr(stream)))
    return q, inv, rs


def linear_q_rowsum(w, q, inv, rowsum, out=None, stream=None):
    """linear_q with caller-provided row sums of q (an xtern extension)."""
    torch = _torch()
    q2 = q.reshape(-1, q.shape[-1])
    M = q2.shape[0]
    y = out if out is not None else torch.empty((M, w.out_dim), dtype=torch.float32, device=q.device)
    _check(_lib.xt_ternary_linear_q_rowsum(w.handle, _dev_ptr(q2, torch.int8, "q"),
                                           _dev_ptr(inv, torch.float32, "inv_scale"),
                                           _dev_ptr(rowsum, torch.int32, "rowsum"), M,
                                           _dev_ptr(y, torch.float32, "y"), None,
                                           _stream_ptr(stream)))
    return y


def linear_q(w, q, inv, acc=False, out=None, stream=None):
    """y = dot(q, W) * inv * w_scales for q [M, K] int8, inv [M] f32."""
    torch = _torch()
    q2 = q.reshape(-1, q.shape[-1])
    M = q2.shape[0]
    if q2.shape[1] != w.in_dim:
        raise XternError(XT_ERR_INVALID,
                         f"Input dimension mismatch: expected {w.in_dim}, got {q2.shape[1]}")
    y = out if out is not None else torch.empty((M, w.out_dim), dtype=torch.float32, device=q.device)
    a = torch.empty((M, w.out_dim), dtype=torch.int32, device=q.device) if acc else None
    _check(_lib.xt_ternary_linear_q(w.handle, _dev_ptr(q2, torch.int8, "q"),
                                    _dev_ptr(inv, torch.float32, "inv_scale"), M,
                                    _dev_ptr(y, torch.float32, "y"),
                                    _dev_ptr(a, torch.int32, "acc") if acc else None,
                                    _stream_ptr(stream)))
    return (y, a) if acc else y


def linear_f32_noalloc(w, x, mode=XT_QUANT_AVX512, out=None, stream=None):
    """linear_f32 through xt_ternary_linear_f32_noalloc (static device scratch,
    no allocation in the library; calls overlapping on one GPU race)."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    y = out if out is not None else torch.empty((M, w.out_dim), dtype=torch.float32, device=x.device)
    _check(_lib.xt_ternary_linear_f32_noalloc(w.handle, _dev_ptr(x2, torch.float32, "x"), M,
                                              _dev_ptr(y, torch.float32, "y"), mode,
                                              _stream_ptr(stream)))
    return y


def workspace_release():
    """Free the library's device workspaces (waits for the device)."""
    _check(_lib.xt_workspace_release())


def linear_f32(w, x, mode=XT_QUANT_AVX512, out=None, stream=None):
    """Quantise rows of x [M, K] f32 and apply the ternary product."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    if x2.shape[1] != w.in_dim:
        raise XternError(XT_ERR_INVALID,
                         f"Input dimension mismatch: expected {w.in_dim}, got {x2.shape[1]}")
    y = out if out is not None else torch.empty((M, w.out_dim), dtype=torch.float32, device=x.device)
    _check(_lib.xt_ternary_linear_f32(w.handle, _dev_ptr(x2, torch.float32, "x"), M,
                                      _dev_ptr(y, torch.float32, "y"), mode, _stream_ptr(stream)))
    return y


def activation_mul(act, gate, up, out=None, stream=None):
    """xt_activation_mul: act(gate) * up row-wise for [..., n] f32 tensors."""
    torch = _torch()
    if gate.shape != up.shape:
        raise XternError(XT_ERR_INVALID, f"shape mismatch: {tuple(gate.shape)} != {tuple(up.shape)}")
    n = gate.shape[-1]
    g2, u2 = gate.reshape(-1, n).contiguous(), up.reshape(-1, n).contiguous()
    y = out if out is not None else torch.empty_like(g2)
    _check(_lib.xt_activation_mul(act, _dev_ptr(g2, torch.float32, "gate"),
                                  _dev_ptr(u2, torch.float32, "up"), g2.shape[0], n,
                                  _dev_ptr(y, torch.float32, "out"), _stream_ptr(stream)))
    return y.reshape(gate.shape)


def rms_norm(x, weight, eps, out=None, stream=None):
    """xt_rms_norm: rms_norm of each row of x [..., n]."""
    torch = _torch()
    n = x.shape[-1]
    if weight.numel() != n:
        raise XternError(XT_ERR_INVALID,
                         f"FastTensor::rmsnorm weight size mismatch: expected {n}, got {weight.numel()}")
    x2 = x.reshape(-1, n).contiguous()
    y = out if out is not None else torch.empty_like(x2)
    _check(_lib.xt_rms_norm(_dev_ptr(x2, torch.float32, "x"),
                            _dev_ptr(weight.contiguous(), torch.float32, "weight"), x2.shape[0], n,
                            float(eps), _dev_ptr(y, torch.float32, "y"), _stream_ptr(stream)))
    return y.reshape(x.shape)


def _mlp_check(gate, up, down, x_last):
    if x_last != gate.in_dim:
        raise XternError(XT_ERR_INVALID,
                         f"Input dimension mismatch: expected {gate.in_dim}, got {x_last}")


def mlp_q(gate, up, down, q, inv, norm_w=None, eps=1e-5, use_silu=False,
          mode=XT_QUANT_AVX512, out=None, stream=None):
    """xt_ternary_mlp_q: fused_mlp_all on every row of q [M, in_dim] i8."""
    torch = _torch()
    _mlp_check(gate, up, down, q.shape[-1])
    q2 = q.reshape(-1, q.shape[-1]).contiguous()
    M = q2.shape[0]
    y = out if out is not None else torch.empty((M, down.out_dim), dtype=torch.float32,
                                                device=q.device)
    _check(_lib.xt_ternary_mlp_q(gate.handle, up.handle, down.handle,
                                 _dev_ptr(norm_w, torch.float32, "norm_w") if norm_w is not None
                                 else None, float(eps), int(bool(use_silu)),
                                 _dev_ptr(q2, torch.int8, "q"),
                                 _dev_ptr(inv.contiguous(), torch.float32, "inv_scale"), M,
                                 _dev_ptr(y, torch.float32, "y"), mode, _stream_ptr(stream)))
    return y


def mlp_f32(gate, up, down, x, norm_w=None, eps=1e-5, use_silu=False, mode=XT_QUANT_AVX512,
            out=None, stream=None):
    """xt_ternary_mlp_f32: Mlp::forward for x [M, in_dim] f32."""
    torch = _torch()
    _mlp_check(gate, up, down, x.shape[-1])
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    M = x2.shape[0]
    y = out if out is not None else torch.empty((M, down.out_dim), dtype=torch.float32,
                                                device=x.device)
    _check(_lib.xt_ternary_mlp_f32(gate.handle, up.handle, down.handle,
                                   _dev_ptr(norm_w, torch.float32, "norm_w") if norm_w is not None
                                   else None, float(eps), int(bool(use_silu)),
                                   _dev_ptr(x2, torch.float32, "x"), M,
                                   _dev_ptr(y, torch.float32, "y"), mode, _stream_ptr(stream)))
    return y


def _multi(ws, ys):
    n = len(ws)
    harr = (_vp * n)(*[w.handle for w in ws])
    yarr = (_vp * n)(*[ctypes.c_void_p(y.data_ptr()) for y in ys])
    return harr, yarr


def linear_multi_f32(ws, x, mode=XT_QUANT_AVX512, stream=None, outs=None):
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    ys = outs if outs is not None else [torch.empty((M, w.out_dim), dtype=torch.float32,
                                                    device=x.device) for w in ws]
    harr, yarr = _multi(ws, ys)
    _check(_lib.xt_ternary_linear_multi_f32(harr, len(ws), _dev_ptr(x2, torch.float32, "x"), M,
                                            yarr, mode, _stream_ptr(stream)))
    return ys


def linear_multi_q(ws, q, inv, stream=None):
    torch = _torch()
    q2 = q.reshape(-1, q.shape[-1])
    M = q2.shape[0]
    ys = [torch.empty((M, w.out_dim), dtype=torch.float32, device=q.device) for w in ws]
    harr, yarr = _multi(ws, ys)
    _check(_lib.xt_ternary_linear_multi_q(harr, len(ws), _dev_ptr(q2, torch.int8, "q"),
                                          _dev_ptr(inv, torch.float32, "inv_scale"), M, yarr,
                                          _stream_ptr(stream)))
    return ys


from .layers import (TernaryLinear, DynamicLinear, TernaryRep, FastRmsNorm, Mlp,  # noqa: E402,F401
                     Int8Linear, Int4Linear)


class Stack:
    """A decode stack (xt_stack_*): ops = [(weights list, x, ys list, dep)],
    x [M, in_dim] f32 and ys [M, out_dim] f32 device tensors that the stack
    keeps referencing.  plan: None (the library picks), "one_launch" (every
    op in one persistent launch) or "per_op" (one library call per op);
    run() runs the whole list, `plan_name` says which plan it has."""

    _PLANS = {None: XT_STACK_AUTO, "auto": XT_STACK_AUTO, "one_launch": XT_STACK_ONE_LAUNCH,
              "per_op": XT_STACK_PER_OP}

    def __init__(self, ops, M, mode=XT_QUANT_AVX512, plan=None):
        if plan not in self._PLANS:
            raise XternError(XT_ERR_INVALID, f"unknown stack plan {plan!r}")
        torch = _torch()
        arr = (_StackOp * len(ops))()
        self._keep = []
        for i, (ws, x, ys, dep) in enumerate(ops):
            if len(ws) != len(ys) or not 1 <= len(ws) <= 4:
                raise XternError(XT_ERR_INVALID, f"op {i}: need 1..4 weights and as many outputs")
            o = arr[i]
            o.n = len(ws)
            o.x = _dev_ptr(x, torch.float32, "x").value
            o.dep = -1 if dep is None else int(dep)
            for p, (w, y) in enumerate(zip(ws, ys)):
                o.w[p] = w.handle.value
                o.y[p] = _dev_ptr(y, torch.float32, "y").value
            self._keep += [x] + list(ys) + list(ws)
        h = ctypes.c_void_p()
        _check(_lib.xt_stack_create(arr, len(ops), M, mode | self._PLANS[plan], ctypes.byref(h)))
        self.handle = h

    @property
    def plan_name(self):
        p = _lib.xt_stack_plan(self.handle)
        if p < 0:
            _check(p)
        return "per_op" if p == XT_STACK_PER_OP else "one_launch"

    def run(self, stream=None):
        _check(_lib.xt_stack_run(self.handle, _stream_ptr(stream)))

    def gave_up(self):
        """Wait for the device; True if a dependency wait gave up since the
        last check (then those runs' outputs are not valid)."""
        f = ctypes.c_int()
        _check(_lib.xt_stack_check(self.handle, ctypes.byref(f)))
        return bool(f.value)

    def __del__(self):
        if getattr(self, "handle", None):
            _lib.xt_stack_destroy(self.handle)
            self.handle = None
