// xtern C++ host API: xor-net's bit1_58 TernaryLinear / DynamicLinear on
// MI355X through the xtern C ABI (include/xtern.h).  Header-only, C++17.
//
// Mirrors (paths relative to the xor-net tree):
//   TernaryPackType, pack/unpack codecs   src/bit1_58/quantization.rs:1-91
//   quantize_f32_to_i8                     src/bit1_58/quantization.rs:170-195
//   encode_sparse_row_into / _tensor       src/bit1_58/sparse.rs:61-103
//   TernaryLinear                          src/bit1_58/layers.rs:34-486
//   DynamicLinear (Ternary arm)            src/nn/dynamic_linear.rs:610-680
//   FastTensor {data, shape}               src/tensor.rs:6-40 (device-resident here)
//
// The reference returns anyhow::Result; here the same conditions throw
// xtern::Error carrying the same message (and the C ABI status).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/xtern.h"

namespace xtern {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

inline void check(int rc) {
    if (rc != XT_OK) throw Error(rc, std::string("xtern error ") + std::to_string(rc) + ": " + xt_last_error());
}
inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(XT_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}
[[noreturn]] inline void bail(const std::string& msg) { throw Error(XT_ERR_INVALID, msg); }

enum class TernaryPackType { Pack4 = XT_PACK4, Pack5 = XT_PACK5 };

// ------------------------------------------------------------------ codecs

namespace detail {
// quantization.rs:12-21: clamp(round_half_away(w / s), -1, 1); s <= 0 -> 0;
// then < -0.5 -> -1, > 0.5 -> +1, else 0 (a NaN weight becomes -1).
inline int ternarise(float w, float s) {
    const float scaled = s > 0.0f ? w / s : 0.0f;
    float q = std::round(scaled);
    if (std::isnan(q)) q = -1.0f;
    q = q < -1.0f ? -1.0f : (q > 1.0f ? 1.0f : q);
    return q < -0.5f ? -1 : (q > 0.5f ? 1 : 0);
}
}  // namespace detail

// quantization.rs:7-27
inline std::vector<uint8_t> pack_1_58bit_4pack(const float* w, size_t n, float w_scale) {
    std::vector<uint8_t> out((n + 3) / 4, 0);
    for (size_t i = 0; i < n; ++i) {
        const int t = detail::ternarise(w[i], w_scale);
        const unsigned code = t < 0 ? 0u : (t > 0 ? 2u : 1u);
        out[i / 4] = (uint8_t)(out[i / 4] | (code << (2 * (i % 4))));
    }
    return out;
}

// quantization.rs:48-70
inline std::vector<uint8_t> pack_1_58bit_5pack(const float* w, size_t n, float w_scale) {
    std::vector<uint8_t> out((n + 4) / 5, 0);
    for (size_t c = 0; c < out.size(); ++c) {
        unsigned b = 0, mul = 1;
        for (size_t j = 0; j < 5 && c * 5 + j < n; ++j) {
            const int t = detail::ternarise(w[c * 5 + j], w_scale);
            b += (t < 0 ? 0u : (t > 0 ? 2u : 1u)) * mul;
            mul *= 3;
        }
        out[c] = (uint8_t)b;
    }
    return out;
}

// quantization.rs:29-46 (code 11 reads as 0)
inline std::vector<float> unpack_1_58bit_4pack(const uint8_t* p, size_t n) {
    std::vector<float> w(n);
    for (size_t i = 0; i < n; ++i) {
        const unsigned c = (p[i / 4] >> (2 * (i % 4))) & 3u;
        w[i] = c == 0 ? -1.0f : (c == 2 ? 1.0f : 0.0f);
    }
    return w;
}

// quantization.rs:72-91
inline std::vector<float> unpack_1_58bit_5pack(const uint8_t* p, size_t n) {
    std::vector<float> w(n);
    for (size_t c = 0; c * 5 < n; ++c) {
        unsigned b = p[c];
        for (size_t j = 0; j < 5 && c * 5 + j < n; ++j) {
            const unsigned v = b % 3;
            b /= 3;
            w[c * 5 + j] = v == 0 ? -1.0f : (v == 2 ? 1.0f : 0.0f);
        }
    }
    return w;
}

// sparse.rs:61-86: u32 num_blocks; per 64-block u64 mask + ceil(nnz/8)
// set-order sign bytes (bit j: the j-th non-zero is -1), little-endian.
inline void encode_sparse_row_into(std::vector<uint8_t>& buf, const int8_t* vals, size_t in_dim) {
    const uint32_t nb = (uint32_t)((in_dim + 63) / 64);
    for (int k = 0; k < 4; ++k) buf.push_back((uint8_t)(nb >> (8 * k)));
    for (size_t b = 0; b < nb; ++b) {
        uint64_t mask = 0, sgn = 0;
        unsigned si = 0;
        for (size_t i = b * 64; i < in_dim && i < b * 64 + 64; ++i)
            if (vals[i] != 0) {
                mask |= 1ull << (i - b * 64);
                if (vals[i] < 0) sgn |= 1ull << si;
                ++si;
            }
        for (int k = 0; k < 8; ++k) buf.push_back((uint8_t)(mask >> (8 * k)));
        for (unsigned k = 0; k < (si + 7) / 8; ++k) buf.push_back((uint8_t)(sgn >> (8 * k)));
    }
}

// sparse.rs:90-103
inline std::pair<std::vector<uint8_t>, std::vector<size_t>> encode_sparse_tensor(
    const int8_t* vals, size_t in_dim, size_t out_dim) {
    std::vector<uint8_t> blob;
    std::vector<size_t> offs;
    for (size_t r = 0; r < out_dim; ++r) {
        offs.push_back(blob.size());
        encode_sparse_row_into(blob, vals + r * in_dim, in_dim);
    }
    return {blob, offs};
}

// ------------------------------------------------------------ device data

template <typename T>
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) : n_(n) {
        if (n) check_hip(hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)), "hipMalloc");
    }
    DeviceBuffer(const T* host, size_t n) : DeviceBuffer(n) { upload(host, n); }
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr, o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        std::swap(p_, o.p_);
        std::swap(n_, o.n_);
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    ~DeviceBuffer() {
        if (p_) (void)hipFree(p_);
    }
    void upload(const T* host, size_t n) {
        check_hip(hipMemcpy(p_, host, n * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    std::vector<T> download() const {
        std::vector<T> h(n_);
        if (n_) check_hip(hipMemcpy(h.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
        return h;
    }
    T* data() { return p_; }
    const T* data() const { return p_; }
    size_t size() const { return n_; }

   private:
    T* p_ = nullptr;
    size_t n_ = 0;
};

// tensor.rs:6-40, with the data on the device.
struct FastTensor {
    DeviceBuffer<float> data;
    std::vector<size_t> shape;
    FastTensor() = default;
    FastTensor(const std::vector<float>& host, std::vector<size_t> shp)
        : data(host.data(), host.size()), shape(std::move(shp)) {}
    FastTensor(DeviceBuffer<float>&& d, std::vector<size_t> shp)
        : data(std::move(d)), shape(std::move(shp)) {}
    size_t rows() const {
        return shape.empty() ? 0
                             : std::accumulate(shape.begin(), shape.end() - 1, (size_t)1,
                                               std::multiplies<size_t>());
    }
};

// quantization.rs:170-195 on the device for every row of x (the AVX-512 host
// path's rounding unless `scalar_rounding`).  Returns (q, inv_scale).
inline std::pair<DeviceBuffer<int8_t>, DeviceBuffer<float>> quantize_f32_to_i8(
    const FastTensor& xs, bool scalar_rounding = false, hipStream_t stream = nullptr) {
    if (xs.shape.empty()) bail("Input must have at least 1 dimension");
    const size_t K = xs.shape.back(), M = xs.rows();
    DeviceBuffer<int8_t> q(M * K);
    DeviceBuffer<float> inv(M);
    check(xt_quantize_i8(xs.data.data(), (int64_t)M, (int64_t)K, q.data(), inv.data(),
                         scalar_rounding ? XT_QUANT_SCALAR : XT_QUANT_AVX512, stream));
    return {std::move(q), std::move(inv)};
}

// ------------------------------------------------------------ HF loader

// VarBuilder::get_prepacked_ternary (loader/mod.rs:301-394) on tensor bytes
// already read from the checkpoint: `stored` is the U8 [out_dim/f][in_dim]
// tensor, `weight_scale` the first element of its weight_scale companion.
struct PrepackedTernary {
    std::vector<uint8_t> packed;  // input-dim packed rows [out_dim][ceil(in_dim/f)]
    std::vector<float> w_scales;  // out_dim copies of the (inverted) scale
    size_t in_dim, out_dim;
};

inline PrepackedTernary get_prepacked_ternary(const uint8_t* stored, size_t nbytes,
                                              size_t out_dim, size_t in_dim, TernaryPackType pt,
                                              float weight_scale, bool is_inverted_scale) {
    const size_t f = pt == TernaryPackType::Pack4 ? 4 : 5;
    PrepackedTernary r;
    r.packed.resize(out_dim * ((in_dim + f - 1) / f));
    check(xt_hf_destripe((int)pt, (int64_t)in_dim, (int64_t)out_dim, stored, nbytes,
                         r.packed.data()));
    r.w_scales.assign(out_dim, is_inverted_scale ? 1.0f / weight_scale : weight_scale);
    r.in_dim = in_dim;
    r.out_dim = out_dim;
    return r;
}

// ------------------------------------------------------------ layers

enum class TernaryRep { Dense, Sparse };  // layers.rs:23-27

class TernaryLinear {
   public:
    TernaryRep rep;
    size_t in_dim, out_dim;
    TernaryPackType pack_type;
    std::vector<float> w_scales;
    std::vector<uint8_t> host_bytes;  // the packed bytes as uploaded

    // layers.rs:91-146
    static TernaryLinear new_(size_t in_dim, size_t out_dim, const std::vector<float>& w,
                              TernaryPackType pt, const float* provided_scale = nullptr) {
        if (w.size() != in_dim * out_dim) bail("Weight length must match in_dim * out_dim");
        bool already = true;
        for (float v : w) already = already && (v == -1.0f || v == 0.0f || v == 1.0f);
        std::vector<float> scales(out_dim);
        std::vector<uint8_t> packed;
        for (size_t o = 0; o < out_dim; ++o) {
            const float* row = w.data() + o * in_dim;
            float s;
            if (already || provided_scale) {
                s = provided_scale ? *provided_scale : 1.0f;
            } else {  // per-row mean |w| (sequential f32 sum, as the reference)
                float sum = 0.0f;
                for (size_t k = 0; k < in_dim; ++k) sum += std::fabs(row[k]);
                s = in_dim ? sum / (float)in_dim : 1.0f;
            }
            scales[o] = s;
            auto b = pt == TernaryPackType::Pack4 ? pack_1_58bit_4pack(row, in_dim, s)
                                                   : pack_1_58bit_5pack(row, in_dim, s);
            packed.insert(packed.end(), b.begin(), b.end());
        }
        return TernaryLinear(TernaryRep::Dense, in_dim, out_dim, pt, std::move(scales),
                             std::move(packed));
    }

    // layers.rs:151-179 (ternarize_row, :45-88: already-ternary rows as-is)
    static TernaryLinear new_sparse(size_t in_dim, size_t out_dim, const std::vector<float>& w,
                                    TernaryPackType pt, const float* provided_scale = nullptr) {
        if (w.size() != in_dim * out_dim) bail("Weight length must match in_dim * out_dim");
        bool already = true;
        for (float v : w) already = already && (v == -1.0f || v == 0.0f || v == 1.0f);
        std::vector<float> scales(out_dim);
        std::vector<int8_t> tern(in_dim * out_dim);
        for (size_t o = 0; o < out_dim; ++o) {
            const float* row = w.data() + o * in_dim;
            float s;
            if (already) {
                s = provided_scale ? *provided_scale : 1.0f;
                for (size_t k = 0; k < in_dim; ++k) tern[o * in_dim + k] = (int8_t)row[k];
            } else {
                if (provided_scale) {
                    s = *provided_scale;
                } else {
                    float sum = 0.0f;
                    for (size_t k = 0; k < in_dim; ++k) sum += std::fabs(row[k]);
                    s = in_dim ? sum / (float)in_dim : 1.0f;
                }
                for (size_t k = 0; k < in_dim; ++k)
                    tern[o * in_dim + k] = (int8_t)detail::ternarise(row[k], s);
            }
            scales[o] = s;
        }
        auto enc = encode_sparse_tensor(tern.data(), in_dim, out_dim);
        return TernaryLinear(TernaryRep::Sparse, in_dim, out_dim, pt, std::move(scales),
                             std::move(enc.first));
    }

    // layers.rs:183-210
    static TernaryLinear new_sparse_from_packed(const std::vector<uint8_t>& packed, size_t in_dim,
                                                size_t out_dim, TernaryPackType pt,
                                                std::vector<float> w_scales) {
        const size_t n = in_dim * out_dim;
        const auto flat = pt == TernaryPackType::Pack4 ? unpack_1_58bit_4pack(packed.data(), n)
                                                       : unpack_1_58bit_5pack(packed.data(), n);
        std::vector<int8_t> tern(n);
        for (size_t i = 0; i < n; ++i) tern[i] = (int8_t)flat[i];
        auto enc = encode_sparse_tensor(tern.data(), in_dim, out_dim);
        return TernaryLinear(TernaryRep::Sparse, in_dim, out_dim, pt, std::move(w_scales),
                             std::move(enc.first));
    }

    // dynamic_linear.rs:670-680 (new_ternary_direct)
    static TernaryLinear new_direct(std::vector<uint8_t> packed, size_t in_dim, size_t out_dim,
                                    TernaryPackType pt, std::vector<float> w_scales) {
        return TernaryLinear(TernaryRep::Dense, in_dim, out_dim, pt, std::move(w_scales),
                             std::move(packed));
    }

    // DynamicLinear::load's prepacked arm (dynamic_linear.rs:729-741): the
    // tiles are built on the device from the striped bytes
    // (xt_weights_create_hf); host_bytes stays empty.
    static TernaryLinear from_hf_prepacked(const uint8_t* stored, size_t nbytes, size_t in_dim,
                                           size_t out_dim, TernaryPackType pt,
                                           float weight_scale, bool is_inverted_scale) {
        xt_weights* h = nullptr;
        check(xt_weights_create_hf((int)pt, (int64_t)in_dim, (int64_t)out_dim, stored, nbytes,
                                   weight_scale, is_inverted_scale ? 1 : 0, &h));
        std::vector<float> ws(out_dim, is_inverted_scale ? 1.0f / weight_scale : weight_scale);
        return TernaryLinear(pt, in_dim, out_dim, std::move(ws), h);
    }

    // layers.rs:234-239 (Dense: out_dim * ceil(in_dim/f); Sparse: blob bytes)
    size_t packed_bytes() const {
        if (rep == TernaryRep::Dense && host_bytes.empty()) {
            const size_t f = pack_type == TernaryPackType::Pack4 ? 4 : 5;
            return out_dim * ((in_dim + f - 1) / f);
        }
        return host_bytes.size();
    }

    // layers.rs:262-313
    FastTensor forward(const FastTensor& xs, bool scalar_rounding = false,
                       hipStream_t stream = nullptr) const {
        auto shape = out_shape(xs);
        const size_t M = xs.rows();
        DeviceBuffer<float> y(M * out_dim);
        check(xt_ternary_linear_f32(w_.get(), xs.data.data(), (int64_t)M, y.data(),
                                    scalar_rounding ? XT_QUANT_SCALAR : XT_QUANT_AVX512, stream));
        return FastTensor(std::move(y), shape);
    }

    // layers.rs:315-345, for every row: q [rows][in_dim] i8 and inv [rows]
    // on the device.
    FastTensor forward_with_quantized(const FastTensor& xs, const int8_t* q_dev,
                                      const float* inv_dev, hipStream_t stream = nullptr) const {
        auto shape = out_shape(xs);
        const size_t M = xs.rows();
        DeviceBuffer<float> y(M * out_dim);
        check(xt_ternary_linear_q(w_.get(), q_dev, inv_dev, (int64_t)M, y.data(), nullptr, stream));
        return FastTensor(std::move(y), shape);
    }

    // layers.rs:347-424
    static std::vector<FastTensor> fused_forward_qkv(const FastTensor& xs, const int8_t* q_dev,
                                                     const float* inv_dev, const TernaryLinear& ql,
                                                     const TernaryLinear& kl,
                                                     const TernaryLinear& vl,
                                                     hipStream_t stream = nullptr) {
        return fused(xs, q_dev, inv_dev, {&ql, &kl, &vl}, stream);
    }
    // layers.rs:426-486
    static std::vector<FastTensor> fused_forward_mlp(const FastTensor& xs, const int8_t* q_dev,
                                                     const float* inv_dev,
                                                     const TernaryLinear& fc1,
                                                     const TernaryLinear& fc2,
                                                     hipStream_t stream = nullptr) {
        return fused(xs, q_dev, inv_dev, {&fc1, &fc2}, stream);
    }

    const xt_weights* handle() const { return w_.get(); }

   private:
    struct Deleter {
        void operator()(xt_weights* w) const { (void)xt_weights_destroy(w); }
    };
    std::shared_ptr<xt_weights> w_;

    TernaryLinear(TernaryRep r, size_t in, size_t out, TernaryPackType pt, std::vector<float> ws,
                  std::vector<uint8_t> bytes)
        : rep(r), in_dim(in), out_dim(out), pack_type(pt), w_scales(std::move(ws)),
          host_bytes(std::move(bytes)) {
        if (w_scales.size() != out_dim) bail("w_scales must hold out_dim values");
        xt_weights* h = nullptr;
        const int fmt = r == TernaryRep::Sparse ? XT_XORSPARSE : (int)pt;
        check(xt_weights_create(fmt, (int64_t)in_dim, (int64_t)out_dim, host_bytes.data(),
                                host_bytes.size(), w_scales.data(), &h));
        w_.reset(h, Deleter());
    }

    TernaryLinear(TernaryPackType pt, size_t in, size_t out, std::vector<float> ws, xt_weights* h)
        : rep(TernaryRep::Dense), in_dim(in), out_dim(out), pack_type(pt),
          w_scales(std::move(ws)) {
        w_.reset(h, Deleter());
    }

    std::vector<size_t> out_shape(const FastTensor& xs) const {
        if (xs.shape.empty()) bail("Input must have at least 1 dimension");
        if (xs.shape.back() != in_dim)
            bail("Input dimension mismatch: expected " + std::to_string(in_dim) + ", got " +
                 std::to_string(xs.shape.back()));
        auto s = xs.shape;
        s.back() = out_dim;
        return s;
    }

    static std::vector<FastTensor> fused(const FastTensor& xs, const int8_t* q_dev,
                                         const float* inv_dev,
                                         std::vector<const TernaryLinear*> lins,
                                         hipStream_t stream) {
        const size_t M = xs.rows();
        std::vector<const xt_weights*> hs;
        std::vector<DeviceBuffer<float>> ys;
        std::vector<float*> yp;
        for (auto* l : lins) {
            l->out_shape(xs);
            hs.push_back(l->w_.get());
            ys.emplace_back(M * l->out_dim);
            yp.push_back(ys.back().data());
        }
        check(xt_ternary_linear_multi_q(hs.data(), (int)hs.size(), q_dev, inv_dev, (int64_t)M,
                                        yp.data(), stream));
        std::vector<FastTensor> out;
        for (size_t p = 0; p < lins.size(); ++p) {
            auto s = xs.shape;
            s.back() = lins[p]->out_dim;
            out.emplace_back(std::move(ys[p]), s);
        }
        return out;
    }
};

// dynamic_linear.rs:610-643 — the Ternary arm of LinearKind.
class DynamicLinear {
   public:
    explicit DynamicLinear(TernaryLinear inner) : inner_(std::move(inner)) {}
    static DynamicLinear new_ternary(size_t in_dim, size_t out_dim, const std::vector<float>& w,
                                     TernaryPackType pt, const float* provided_scale = nullptr) {
        return DynamicLinear(TernaryLinear::new_(in_dim, out_dim, w, pt, provided_scale));
    }
    static DynamicLinear new_ternary_direct(std::vector<uint8_t> packed, size_t in_dim,
                                            size_t out_dim, TernaryPackType pt,
                                            std::vector<float> w_scales) {
        return DynamicLinear(
            TernaryLinear::new_direct(std::move(packed), in_dim, out_dim, pt, std::move(w_scales)));
    }
    FastTensor forward(const FastTensor& xs) const { return inner_.forward(xs); }
    FastTensor forward_with_quantized(const FastTensor& xs, const int8_t* q, const float* inv) const {
        return inner_.forward_with_quantized(xs, q, inv);
    }
    const TernaryLinear& inner() const { return inner_; }

   private:
    TernaryLinear inner_;
};

}  // namespace xtern
