"""TernaryLinear / DynamicLinear with the reference's constructors and forward
signatures, computing on the GPU through libxtern.

Reference (paths relative to xor-net): src/bit1_58/layers.rs,
src/nn/dynamic_linear.rs.  Tensors are torch tensors on the HIP device
(the reference's FastTensor holds data + shape; a torch tensor holds both).
"""
import enum

import numpy as np

from . import (XT_ERR_INVALID, XT_PACK4, XT_PACK5, XT_QUANT_AVX512, XT_XORSPARSE,
               DeviceWeights, TernaryPackType, XternError, _ternarise, encode_sparse_tensor,
               hf_destripe, mlp_f32, mlp_q, rms_norm, XT_INT8, XT_INT4, int_quantize_host,
               linear_f32, linear_multi_q, linear_q, pack_ternary4, pack_ternary5,
               unpack_1_58bit_4pack, unpack_1_58bit_5pack)


class TernaryRep(enum.Enum):
    """layers.rs:23-27 — which byte layout the weights were uploaded from."""
    Dense = 0
    Sparse = 1


def _row_mean_abs(row):
    """Sequential f32 sum of |w| / len, as `row.iter().map(abs).sum() / len`."""
    if row.size == 0:
        return np.float32(1.0)
    return np.float32(np.cumsum(np.abs(row.astype(np.float32)), dtype=np.float32)[-1]
                      / np.float32(row.size))


def _pack_rows(tern, pack_type):
    pack = pack_ternary4 if pack_type == TernaryPackType.Pack4 else pack_ternary5
    return np.concatenate([pack(r) for r in tern]) if tern.shape[0] else np.zeros(0, np.uint8)


class TernaryLinear:
    """layers.rs:34-41: weights (rep), in_dim, out_dim, pack_type, w_scales."""

    def __init__(self, rep, in_dim, out_dim, pack_type, w_scales, host_bytes, weights=None):
        self.rep = rep
        self.in_dim = int(in_dim)
        self.out_dim = int(out_dim)
        self.pack_type = pack_type
        self.w_scales = np.asarray(w_scales, dtype=np.float32)
        self.host_bytes = host_bytes
        fmt = XT_XORSPARSE if rep == TernaryRep.Sparse else pack_type.value
        self.weights = weights if weights is not None else DeviceWeights(
            fmt, self.in_dim, self.out_dim, host_bytes, self.w_scales)

    # --- constructors -----------------------------------------------------

    @classmethod
    def new(cls, in_dim, out_dim, weights_f32, pack_type, provided_scale=None):
        """layers.rs:91-146.  Already-ternary weights are packed as
        round(w / scale) with scale = provided or 1.0 (so a provided scale
        above 2 zeroes every weight, as in the reference); other weights use
        the provided global scale or a per-row mean |w|."""
        w = np.asarray(weights_f32, dtype=np.float32).ravel()
        if w.size != in_dim * out_dim:
            raise XternError(XT_ERR_INVALID, "Weight length must match in_dim * out_dim")
        rows = w.reshape(out_dim, in_dim)
        already = bool(np.all((w == -1.0) | (w == 0.0) | (w == 1.0)))
        if already or provided_scale is not None:
            s = np.float32(1.0 if provided_scale is None else provided_scale)
            scales = np.full(out_dim, s, dtype=np.float32)
        else:
            scales = np.array([_row_mean_abs(r) for r in rows], dtype=np.float32)
        tern = np.stack([_ternarise(rows[o], scales[o]) for o in range(out_dim)])
        return cls(TernaryRep.Dense, in_dim, out_dim, pack_type, scales,
                   _pack_rows(tern, pack_type))

    @classmethod
    def new_sparse(cls, in_dim, out_dim, weights_f32, pack_type, provided_scale=None):
        """layers.rs:151-179 with ternarize_row (:45-88): already-ternary rows
        are taken as-is (`w as i8`) with scale = provided or 1.0."""
        w = np.asarray(weights_f32, dtype=np.float32).ravel()
        if w.size != in_dim * out_dim:
            raise XternError(XT_ERR_INVALID, "Weight length must match in_dim * out_dim")
        rows = w.reshape(out_dim, in_dim)
        already = bool(np.all((w == -1.0) | (w == 0.0) | (w == 1.0)))
        if already:
            s = np.float32(1.0 if provided_scale is None else provided_scale)
            scales = np.full(out_dim, s, dtype=np.float32)
            tern = rows.astype(np.int8)
        else:
            if provided_scale is not None:
                scales = np.full(out_dim, provided_scale, dtype=np.float32)
            else:
                scales = np.array([_row_mean_abs(r) for r in rows], dtype=np.float32)
            tern = np.stack([_ternarise(rows[o], scales[o]) for o in range(out_dim)])
        blob, _ = encode_sparse_tensor(tern, in_dim, out_dim)
        return cls(TernaryRep.Sparse, in_dim, out_dim, pack_type, scales, blob)

    @classmethod
    def new_sparse_from_packed(cls, packed, in_dim, out_dim, pack_type, w_scales):
        """layers.rs:183-210: unpack Pack4/Pack5 bytes, re-encode as XorSparse."""
        n = in_dim * out_dim
        if pack_type == TernaryPackType.Pack4:
            flat = unpack_1_58bit_4pack(packed, n)
        else:
            flat = unpack_1_58bit_5pack(packed, n)
        blob, _ = encode_sparse_tensor(flat.astype(np.int8), in_dim, out_dim)
        return cls(TernaryRep.Sparse, in_dim, out_dim, pack_type, w_scales, blob)

    @classmethod
    def new_direct(cls, packed, in_dim, out_dim, pack_type, w_scales):
        """DynamicLinear::new_ternary_direct (dynamic_linear.rs:670-680):
        already-packed row-major Pack4/Pack5 bytes plus per-row scales."""
        return cls(TernaryRep.Dense, in_dim, out_dim, pack_type, w_scales,
                   np.asarray(packed, dtype=np.uint8))

    @classmethod
    def from_sparse_blob(cls, blob, in_dim, out_dim, w_scales, pack_type=TernaryPackType.Pack4):
        """A TernaryLinear over an XorSparse row blob, as DynamicLinear::load
        builds from SparseFile::get_sparse (dynamic_linear.rs:697-715)."""
        return cls(TernaryRep.Sparse, in_dim, out_dim, pack_type, w_scales, blob)

    @classmethod
    def from_hf_prepacked(cls, stored, in_dim, out_dim, pack_type, weight_scale,
                          is_inverted_scale, sparse=False):
        """DynamicLinear::load's prepacked arm (dynamic_linear.rs:729-741) for
        one tensor: `stored` is the checkpoint's U8 [out_dim/f][in_dim] array.
        Dense: the tiles are built on the device from the striped bytes
        (xt_weights_create_hf) and the host keeps no copy.  sparse=True
        (XORNET_WEIGHT_FMT=sparse): destripe on the host, then
        new_sparse_from_packed, as the reference does."""
        f = 4 if pack_type == TernaryPackType.Pack4 else 5
        if np.shape(stored) != (out_dim // f, in_dim) or out_dim % f:
            raise XternError(XT_ERR_INVALID, "Tensor is not in pre-packed U8 ternary format")
        s = np.float32(weight_scale)
        ws = np.full(out_dim, np.float32(1.0) / s if is_inverted_scale else s, np.float32)
        if sparse:
            packed = hf_destripe(pack_type.value, in_dim, out_dim, stored)
            return cls.new_sparse_from_packed(packed, in_dim, out_dim, pack_type, ws)
        dev = DeviceWeights.from_hf(pack_type.value, in_dim, out_dim, stored, weight_scale,
                                    is_inverted_scale)
        return cls(TernaryRep.Dense, in_dim, out_dim, pack_type, ws, None, weights=dev)

    @classmethod
    def from_sparse_file(cls, sparse_file, name, in_dim, out_dim,
                         pack_type=TernaryPackType.Pack4):
        """DynamicLinear::load's XorSparse-container arm (dynamic_linear.rs:
        697-716): the named entry, w_scales = out_dim copies of its scale."""
        blob, ws = sparse_file.get_sparse(name, in_dim, out_dim)
        return cls(TernaryRep.Sparse, in_dim, out_dim, pack_type,
                   np.full(out_dim, ws, np.float32), np.frombuffer(blob, np.uint8))

    # --- queries ----------------------------------------------------------

    def packed_bytes(self):
        """layers.rs:234-239 — bytes of the packed weights (Pack4/Pack5:
        out_dim * ceil(in_dim/f); XorSparse: the row blob)."""
        if self.host_bytes is None:
            f = 4 if self.pack_type == TernaryPackType.Pack4 else 5
            return self.out_dim * ((self.in_dim + f - 1) // f)
        return len(self.host_bytes)

    def device_bytes(self):
        return self.weights.device_bytes()

    # --- forward ----------------------------------------------------------

    def _out_shape(self, xs):
        if xs.dim() == 0:
            raise XternError(XT_ERR_INVALID, "Input must have at least 1 dimension")
        if xs.shape[-1] != self.in_dim:
            raise XternError(XT_ERR_INVALID,
                             f"Input dimension mismatch: expected {self.in_dim}, got {xs.shape[-1]}")
        return tuple(xs.shape[:-1]) + (self.out_dim,)

    def forward(self, xs, mode=XT_QUANT_AVX512):
        """layers.rs:262-313: per-row absmax i8 quantisation, ternary product,
        y = (f32)dot * inv_scale[row] * w_scales[o]."""
        shape = self._out_shape(xs)
        return linear_f32(self.weights, xs.contiguous(), mode=mode).reshape(shape)

    def forward_with_quantized(self, xs, quantized_in, inv_scale):
        """layers.rs:315-345 (for any number of rows): `xs` only supplies the
        shape; quantized_in [.., in_dim] int8 and inv_scale (float or [rows]
        f32 tensor) are the input."""
        import torch
        shape = self._out_shape(xs)
        q = quantized_in.reshape(-1, self.in_dim).contiguous()
        if not torch.is_tensor(inv_scale):
            inv_scale = torch.full((q.shape[0],), float(inv_scale), dtype=torch.float32,
                                   device=q.device)
        return linear_q(self.weights, q, inv_scale.contiguous()).reshape(shape)

    @staticmethod
    def fused_forward_qkv(xs, quantized_in, inv_scale, q_lin, k_lin, v_lin):
        """layers.rs:347-424: q/k/v share one quantised input, one launch."""
        return TernaryLinear._fused(xs, quantized_in, inv_scale, [q_lin, k_lin, v_lin])

    @staticmethod
    def fused_forward_mlp(xs, quantized_in, inv_scale, fc1_lin, fc2_lin):
        """layers.rs:426-486: two projections sharing one quantised input."""
        return TernaryLinear._fused(xs, quantized_in, inv_scale, [fc1_lin, fc2_lin])

    @staticmethod
    def _fused(xs, quantized_in, inv_scale, lins):
        import torch
        in_dim = lins[0].in_dim
        for l in lins:
            if l.in_dim != in_dim:
                raise XternError(XT_ERR_INVALID, "fused projections must share in_dim")
        q = quantized_in.reshape(-1, in_dim).contiguous()
        if not torch.is_tensor(inv_scale):
            inv_scale = torch.full((q.shape[0],), float(inv_scale), dtype=torch.float32,
                                   device=q.device)
        ys = linear_multi_q([l.weights for l in lins], q, inv_scale.contiguous())
        lead = tuple(xs.shape[:-1])
        return tuple(y.reshape(lead + (l.out_dim,)) for y, l in zip(ys, lins))


    @staticmethod
    def fused_mlp_all(xs, quantized_in, inv_scale, gate_lin, up_lin, down_lin, ffn_norm,
                      use_silu, mode=XT_QUANT_AVX512):
        """layers.rs:497-645: gate+up on the shared quantised input, SiLU /
        ReLU^2 (silu_inplace), optional ffn norm, requantisation, down — for
        every row of quantized_in.  `mode` is the host ISA the reference would
        run on (it selects silu_inplace's path and the requantisation
        rounding)."""
        import torch
        q = quantized_in.reshape(-1, gate_lin.in_dim).contiguous()
        if not torch.is_tensor(inv_scale):
            inv_scale = torch.full((q.shape[0],), float(inv_scale), dtype=torch.float32,
                                   device=q.device)
        y = mlp_q(gate_lin.weights, up_lin.weights, down_lin.weights, q, inv_scale,
                  norm_w=ffn_norm.weight if ffn_norm is not None else None,
                  eps=ffn_norm.eps if ffn_norm is not None else 0.0, use_silu=use_silu,
                  mode=mode)
        return y.reshape(tuple(xs.shape[:-1]) + (down_lin.out_dim,))


class _IntLinear:
    """Int8Linear / Int4Linear (dynamic_linear.rs:229-535): per-row scaled
    integer weights; forward quantises each activation row (absmax i8) and
    computes (f32)dot * inv_scale * scales[o] on the GPU."""

    BITS = 8
    NAME = "Int8Linear"

    def __init__(self, weight_bytes, scales, in_dim, out_dim):
        self.in_dim, self.out_dim = int(in_dim), int(out_dim)
        self.weight_bytes = np.asarray(weight_bytes, np.uint8)
        self.scales = np.asarray(scales, np.float32)
        fmt = XT_INT8 if self.BITS == 8 else XT_INT4
        self.weights = DeviceWeights(fmt, self.in_dim, self.out_dim, self.weight_bytes, self.scales)

    @classmethod
    def new(cls, weights_f32, out_dim, in_dim):
        b, sc = int_quantize_host(cls.BITS, weights_f32, out_dim, in_dim)
        return cls(b, sc, in_dim, out_dim)

    def _check(self, xs):
        if xs.dim() == 0:
            raise XternError(XT_ERR_INVALID, "Input must have at least 1 dimension")
        if xs.shape[-1] != self.in_dim:
            raise XternError(XT_ERR_INVALID, f"{self.NAME} shape mismatch")
        return tuple(xs.shape[:-1]) + (self.out_dim,)

    def forward(self, xs, mode=XT_QUANT_AVX512):
        shape = self._check(xs)
        return linear_f32(self.weights, xs.contiguous(), mode=mode).reshape(shape)

    def forward_with_quantized(self, xs, quantized_in, inv_scale):
        import torch
        shape = self._check(xs)
        q = quantized_in.reshape(-1, self.in_dim).contiguous()
        if not torch.is_tensor(inv_scale):
            inv_scale = torch.full((q.shape[0],), float(inv_scale), dtype=torch.float32,
                                   device=q.device)
        return linear_q(self.weights, q, inv_scale.contiguous()).reshape(shape)


class Int8Linear(_IntLinear):
    BITS = 8
    NAME = "Int8Linear"


class Int4Linear(_IntLinear):
    BITS = 4
    NAME = "Int4Linear"


class FastRmsNorm:
    """nn::FastRmsNorm: weight [n] (device f32 tensor) and eps; forward is
    rms_norm on each row (tensor.rs:242-265)."""

    def __init__(self, weight, eps):
        self.weight = weight.contiguous()
        self.eps = float(eps)

    def forward(self, xs):
        return rms_norm(xs, self.weight, self.eps)


class Mlp:
    """models/llama/mlp.rs:33-128 with ternary gate (c_fc1), up (c_fc2) and
    down (c_proj) projections, optional ffn_layernorm / ffn_sub_norm, and
    hidden_act "relu2" or "silu"."""

    def __init__(self, c_fc1, c_fc2, c_proj, ffn_layernorm=None, hidden_act="relu2"):
        if hidden_act not in ("relu2", "silu"):
            raise XternError(XT_ERR_INVALID, f"unknown activation {hidden_act}")
        self.c_fc1, self.c_fc2, self.c_proj = c_fc1, c_fc2, c_proj
        self.ffn_layernorm = ffn_layernorm
        self.hidden_act = hidden_act

    def forward(self, x, mode=XT_QUANT_AVX512):
        """One fused launch sequence; one token follows fused_mlp_all, several
        follow the reference's unfused path (mlp.rs:51-127)."""
        if x.dim() == 0:
            raise XternError(XT_ERR_INVALID, "Input must have at least 1 dimension")
        n = self.ffn_layernorm
        y = mlp_f32(self.c_fc1.weights, self.c_fc2.weights, self.c_proj.weights, x.contiguous(),
                    norm_w=n.weight if n is not None else None, eps=n.eps if n is not None else 0.0,
                    use_silu=self.hidden_act == "silu", mode=mode)
        return y.reshape(tuple(x.shape[:-1]) + (self.c_proj.out_dim,))

    def weight_bytes(self):
        """mlp.rs:140-143: packed weight bytes of the three projections."""
        return sum(l.packed_bytes() for l in (self.c_fc1, self.c_fc2, self.c_proj))


class DynamicLinear:
    """dynamic_linear.rs:619-643 — the Ternary arm of LinearKind."""

    def __init__(self, inner):
        self.inner = inner

    @classmethod
    def new_ternary(cls, in_dim, out_dim, weights_f32, pack_type, provided_scale=None):
        return cls(TernaryLinear.new(in_dim, out_dim, weights_f32, pack_type, provided_scale))

    @classmethod
    def new_ternary_direct(cls, packed, in_dim, out_dim, pack_type, w_scales):
        return cls(TernaryLinear.new_direct(packed, in_dim, out_dim, pack_type, w_scales))

    @classmethod
    def new_int8(cls, weights_f32, out_dim, in_dim):
        """dynamic_linear.rs:655-659"""
        return cls(Int8Linear.new(weights_f32, out_dim, in_dim))

    @classmethod
    def new_int4(cls, weights_f32, out_dim, in_dim):
        """dynamic_linear.rs:661-665"""
        return cls(Int4Linear.new(weights_f32, out_dim, in_dim))

    def forward(self, xs):
        return self.inner.forward(xs)

    def forward_with_quantized(self, xs, quantized_in, inv_scale):
        return self.inner.forward_with_quantized(xs, quantized_in, inv_scale)


__all__ = ["TernaryLinear", "DynamicLinear", "TernaryRep", "FastRmsNorm", "Mlp", "Int8Linear",
           "Int4Linear", "TernaryPackType", "XT_PACK4",
           "XT_PACK5"]
