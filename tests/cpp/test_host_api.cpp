// C++ host-API tests, in the shape of xor-net's own Rust tests (file:line of
// the reference tree in each comment).  `--cpu` runs the codec tests only
// (no HIP calls); without arguments every test runs and needs the GPU.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../xor-net_amd/host/xtern.hpp"

using namespace xtern;

static int g_fail = 0;
#define CHECK(cond, ...)                                               \
    do {                                                               \
        if (!(cond)) {                                                 \
            std::fprintf(stderr, "FAIL %s:%d: %s: ", __FILE__, __LINE__, #cond); \
            std::fprintf(stderr, __VA_ARGS__);                         \
            std::fprintf(stderr, "\n");                                \
            ++g_fail;                                                  \
        }                                                              \
    } while (0)

// tests/bit1_58_tests.rs:10-21
static void test_ternary_pack_unpack_roundtrip() {
    std::vector<float> w = {1, 0, -1, 1, 0, -1, -1, 0, 1, 1};
    auto p4 = pack_1_58bit_4pack(w.data(), w.size(), 1.0f);
    auto p5 = pack_1_58bit_5pack(w.data(), w.size(), 1.0f);
    CHECK(unpack_1_58bit_4pack(p4.data(), w.size()) == w, "pack4 roundtrip");
    CHECK(unpack_1_58bit_5pack(p5.data(), w.size()) == w, "pack5 roundtrip");
}

// tests/quantization_158bit_tests.rs:30-38, :70-77
static void test_roundtrip_non_aligned_length() {
    for (size_t n : {1, 2, 3, 5, 6, 7, 9, 11, 13, 15, 17, 21}) {
        std::vector<float> w(n);
        for (size_t i = 0; i < n; ++i) w[i] = (float)((int)(i % 3) - 1);
        auto p4 = pack_1_58bit_4pack(w.data(), n, 1.0f);
        auto p5 = pack_1_58bit_5pack(w.data(), n, 1.0f);
        CHECK(unpack_1_58bit_4pack(p4.data(), n) == w, "pack4 len %zu", n);
        CHECK(unpack_1_58bit_5pack(p5.data(), n) == w, "pack5 len %zu", n);
    }
}

// sparse.rs:61-86 layout, hand-computed
static void test_sparse_row_bytes() {
    std::vector<int8_t> row(64, 0);
    row[0] = 1;
    row[2] = -1;
    std::vector<uint8_t> buf;
    encode_sparse_row_into(buf, row.data(), 64);
    const std::vector<uint8_t> want = {1, 0, 0, 0, 5, 0, 0, 0, 0, 0, 0, 0, 2};
    CHECK(buf == want, "sparse row bytes");
}

// tests/bit1_58_tests.rs:25-34
static void test_absmax_quantization() {
    FastTensor x(std::vector<float>{0.0f, -2.5f, 5.0f, 1.25f}, {4});
    auto qi = quantize_f32_to_i8(x);
    auto q = qi.first.download();
    auto inv = qi.second.download();
    CHECK((q == std::vector<int8_t>{0, -64, 127, 32}), "q");
    CHECK(std::fabs(inv[0] - 5.0f / 127.0f) < 1e-5f, "inv %f", inv[0]);
    FastTensor z(std::vector<float>{0, 0, 0}, {3});
    auto zi = quantize_f32_to_i8(z);
    CHECK(zi.second.download()[0] == 1.0f, "zero inv");
}

// tests/bit1_58_tests.rs:68-92, with the current scale semantics (w_scale
// 1.0 for already-ternary weights): dots 191 and -96 times 2/127.
static void test_ternary_linear_layer() {
    std::vector<float> w = {1, 0, -1, 1, 0, -1, 1, 0};
    auto l4 = TernaryLinear::new_(4, 2, w, TernaryPackType::Pack4);
    auto l5 = TernaryLinear::new_(4, 2, w, TernaryPackType::Pack5);
    FastTensor x(std::vector<float>{0.5f, 1.0f, -0.5f, 2.0f}, {1, 4});
    auto o4 = l4.forward(x).data.download();
    auto o5 = l5.forward(x).data.download();
    CHECK(o4 == o5, "pack4 == pack5");
    CHECK(std::fabs(o4[0] - 3.007874f) < 1e-4f && std::fabs(o4[1] + 1.511811f) < 1e-4f,
          "got %f %f", o4[0], o4[1]);
}

// tests/linear_layer_tests.rs:66-80 and :82-91
static void test_linear_parity_and_zero_input() {
    const size_t K = 20, N = 4;
    std::vector<float> w(K * N);
    for (size_t i = 0; i < w.size(); ++i) w[i] = (float)((int)(i % 3) - 1);
    std::vector<float> xin(K);
    for (size_t i = 0; i < K; ++i) xin[i] = ((float)i - 10.0f) * 0.1f;
    FastTensor x(xin, {1, K});
    auto a = TernaryLinear::new_(K, N, w, TernaryPackType::Pack4).forward(x).data.download();
    auto b = TernaryLinear::new_(K, N, w, TernaryPackType::Pack5).forward(x).data.download();
    for (size_t i = 0; i < N; ++i) CHECK(std::fabs(a[i] - b[i]) < 1e-5f, "idx %zu", i);
    auto z = TernaryLinear::new_(2, 2, {1, -1, 0, 1}, TernaryPackType::Pack4)
                 .forward(FastTensor(std::vector<float>{0, 0}, {1, 2}))
                 .data.download();
    CHECK(z[0] == 0.0f && z[1] == 0.0f, "zero input");
}

// src/bit1_58/simd.rs:581-625 at layer level: dense Pack4 and XorSparse
// (built from floats and from the packed bytes) give identical outputs.
static void test_dense_and_sparse_match() {
    uint64_t s = 0x123456789abcdef0ull;
    auto below = [&](uint64_t n) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return (s >> 33) % n;
    };
    const size_t pairs[][2] = {{2560, 2560}, {6912, 2560}, {2560, 640}, {2560, 6912}};
    for (auto& kn : pairs) {
        const size_t K = kn[0], N = kn[1];
        std::vector<float> w(K * N);
        for (auto& v : w) v = (float)((int)below(3) - 1);
        auto dense = TernaryLinear::new_(K, N, w, TernaryPackType::Pack4);
        auto sparse = TernaryLinear::new_sparse(K, N, w, TernaryPackType::Pack4);
        auto from_packed = TernaryLinear::new_sparse_from_packed(dense.host_bytes, K, N,
                                                                 TernaryPackType::Pack4,
                                                                 dense.w_scales);
        std::vector<float> xin(2 * K);
        for (size_t i = 0; i < xin.size(); ++i) xin[i] = (float)((int)below(7) - 3);
        FastTensor x(xin, {2, K});
        auto yd = dense.forward(x).data.download();
        CHECK(sparse.forward(x).data.download() == yd, "sparse K=%zu N=%zu", K, N);
        CHECK(from_packed.forward(x).data.download() == yd, "from_packed K=%zu N=%zu", K, N);
    }
}

// layers.rs:266-272 error texts; layers.rs:347-424 fused QKV
static void test_errors_and_fused() {
    std::vector<float> w(256 * 64);
    for (size_t i = 0; i < w.size(); ++i) w[i] = (float)((int)((i * 7) % 3) - 1);
    auto l = TernaryLinear::new_(256, 64, w, TernaryPackType::Pack4);
    bool threw = false;
    try {
        l.forward(FastTensor(std::vector<float>(255, 1.0f), {1, 255}));
    } catch (const Error& e) {
        threw = std::string(e.what()).find("Input dimension mismatch: expected 256, got 255") != std::string::npos;
    }
    CHECK(threw, "dimension mismatch error");
    threw = false;
    try {
        TernaryLinear::new_(256, 65, w, TernaryPackType::Pack4);
    } catch (const Error& e) {
        threw = std::string(e.what()) == "Weight length must match in_dim * out_dim";
    }
    CHECK(threw, "weight length error");

    std::vector<float> xin(3 * 256);
    for (size_t i = 0; i < xin.size(); ++i) xin[i] = std::sin(0.37f * (float)i);
    FastTensor x(xin, {3, 256});
    auto lk = TernaryLinear::new_(256, 32, std::vector<float>(w.begin(), w.begin() + 256 * 32),
                                  TernaryPackType::Pack4);
    auto qi = quantize_f32_to_i8(x);
    auto fused = TernaryLinear::fused_forward_qkv(x, qi.first.data(), qi.second.data(), l, lk, lk);
    CHECK(fused.size() == 3 && fused[1].shape == (std::vector<size_t>{3, 32}), "fused shapes");
    CHECK(fused[0].data.download() == l.forward(x).data.download(), "fused q");
    CHECK(fused[1].data.download() == lk.forward(x).data.download(), "fused k");
    CHECK(l.forward_with_quantized(x, qi.first.data(), qi.second.data()).data.download() ==
              fused[0].data.download(),
          "forward_with_quantized");
    DynamicLinear dl(l);
    CHECK(dl.forward(x).data.download() == fused[0].data.download(), "DynamicLinear");
}

// loader/mod.rs:301-394: striped bytes -> the same layer as its destriped rows.
// Rows 0..7 of a K=3 matrix striped over R = 2 stored rows (Pack4).
static void test_hf_prepacked() {
    const int8_t t[8][3] = {{1, 0, -1}, {0, 1, 1}, {-1, -1, 0}, {1, 1, 1},
                            {0, 0, 0},  {-1, 1, 0}, {1, -1, 1}, {0, -1, -1}};
    std::vector<uint8_t> stored(2 * 3, 0);
    for (int o = 0; o < 8; ++o)
        for (int i = 0; i < 3; ++i)
            stored[(o % 2) * 3 + i] |= (uint8_t)((t[o][i] + 1) << (2 * (o / 2)));
    auto pp = get_prepacked_ternary(stored.data(), stored.size(), 8, 3, TernaryPackType::Pack4,
                                    0.25f, true);
    for (int o = 0; o < 8; ++o) {
        auto row = unpack_1_58bit_4pack(pp.packed.data() + o, 3);
        for (int i = 0; i < 3; ++i) CHECK(row[i] == (float)t[o][i], "row %d col %d", o, i);
    }
    CHECK(pp.w_scales.size() == 8 && pp.w_scales[0] == 4.0f, "inverted scale");
    bool threw = false;
    try {
        get_prepacked_ternary(stored.data(), 5, 8, 3, TernaryPackType::Pack4, 1.0f, false);
    } catch (const Error& e) {
        threw = std::string(e.what()).find("pre-packed U8") != std::string::npos;
    }
    CHECK(threw, "bad byte count");
}

static void test_hf_prepacked_layer() {
    std::vector<uint8_t> stored(160 * 2560);
    uint64_t s = 0x9e3779b97f4a7c15ull;
    for (auto& b : stored) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        b = (uint8_t)(s >> 33);
    }
    auto hf = TernaryLinear::from_hf_prepacked(stored.data(), stored.size(), 2560, 640,
                                               TernaryPackType::Pack4, 0.5f, false);
    auto pp = get_prepacked_ternary(stored.data(), stored.size(), 640, 2560,
                                    TernaryPackType::Pack4, 0.5f, false);
    auto direct = TernaryLinear::new_direct(pp.packed, 2560, 640, TernaryPackType::Pack4,
                                            pp.w_scales);
    CHECK(hf.packed_bytes() == direct.packed_bytes(), "packed_bytes");
    std::vector<float> xin(3 * 2560);
    for (size_t i = 0; i < xin.size(); ++i) xin[i] = std::cos(0.11f * (float)i);
    FastTensor x(xin, {3, 2560});
    CHECK(hf.forward(x).data.download() == direct.forward(x).data.download(), "hf layer");
}

// No allocation inside graph capture: a call whose workspace would have to
// grow while its stream is captured fails with XT_ERR_UNSUPPORTED; after one
// eager call of that shape on the stream and thread the same call captures,
// and replays of the graph equal the eager output.
static void test_capture_never_allocates() {
    std::vector<float> w(640 * 2560);
    for (size_t i = 0; i < w.size(); ++i) w[i] = (float)((int)((i * 2654435761u) >> 7) % 3 - 1);
    auto l = TernaryLinear::new_(2560, 640, w, TernaryPackType::Pack4);
    std::vector<float> xin(8 * 2560);
    for (size_t i = 0; i < xin.size(); ++i) xin[i] = std::sin(0.37f * (float)i);
    FastTensor x(xin, {8, 2560});
    DeviceBuffer<float> y1(8 * 640), y2(8 * 640);
    hipStream_t s = nullptr;
    CHECK(hipStreamCreate(&s) == hipSuccess, "stream");
    hipGraph_t g = nullptr;
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed) == hipSuccess, "begin capture");
    const int rc = xt_ternary_linear_f32(l.handle(), x.data.data(), 8, y1.data(), XT_QUANT_AVX512, s);
    CHECK(hipStreamEndCapture(s, &g) == hipSuccess, "end capture");
    CHECK(rc == XT_ERR_UNSUPPORTED, "first call under capture: rc %d", rc);
    CHECK(std::string(xt_last_error()).find("capture") != std::string::npos, "message: %s",
          xt_last_error());
    if (g) (void)hipGraphDestroy(g);
    g = nullptr;
    // eager call on the stream, then capture and replay
    CHECK(xt_ternary_linear_f32(l.handle(), x.data.data(), 8, y1.data(), XT_QUANT_AVX512, s) == XT_OK,
          "eager: %s", xt_last_error());
    CHECK(hipStreamSynchronize(s) == hipSuccess, "sync");
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed) == hipSuccess, "begin capture 2");
    const int rc2 = xt_ternary_linear_f32(l.handle(), x.data.data(), 8, y2.data(), XT_QUANT_AVX512, s);
    CHECK(hipStreamEndCapture(s, &g) == hipSuccess, "end capture 2");
    CHECK(rc2 == XT_OK, "captured call: %s", xt_last_error());
    hipGraphExec_t ge = nullptr;
    if (g && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess) {
        const auto want = y1.download();
        for (int r = 0; r < 3; ++r) {
            CHECK(hipMemset(y2.data(), 0, y2.size() * sizeof(float)) == hipSuccess, "clear");
            CHECK(hipGraphLaunch(ge, s) == hipSuccess, "launch");
            CHECK(hipStreamSynchronize(s) == hipSuccess, "sync");
            CHECK(y2.download() == want, "replay %d", r);
        }
        (void)hipGraphExecDestroy(ge);
    } else {
        CHECK(false, "instantiate");
    }
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(s);
}

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    test_ternary_pack_unpack_roundtrip();
    test_roundtrip_non_aligned_length();
    test_sparse_row_bytes();
    test_hf_prepacked();
    if (!cpu_only) {
        test_hf_prepacked_layer();
        test_absmax_quantization();
        test_ternary_linear_layer();
        test_linear_parity_and_zero_input();
        test_dense_and_sparse_match();
        test_errors_and_fused();
        test_capture_never_allocates();
    }
    std::printf("%s: %d failure(s)\n", cpu_only ? "cpu tests" : "all tests", g_fail);
    return g_fail ? 1 : 0;
}
