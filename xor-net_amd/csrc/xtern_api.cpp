// xtern C ABI (include/xtern.h): weight handles, per-stream workspaces,
// argument checking and kernel dispatch.
//
// Error behaviour follows the reference layer (src/bit1_58/layers.rs:266-272,
// :318-325): a shape mismatch is reported, never computed through; here it
// is a negative status plus xt_last_error() instead of anyhow::bail!.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <utility>
#include <vector>

#include "../../include/xtern.h"
#include "xtern_internal.h"
#include "xtern_layout.h"
#include "xtern_workspace.h"

struct xt_weights {
    int fmt;
    int64_t K, N;
    int64_t nch;        // tile chunks along K
    uint8_t* tiles;     // device, tile_bytes()
    float* ws;          // device, N floats
    size_t tile_bytes;
    int device;
    // XT_XORSPARSE_STREAM: the sections of `tiles` (build_xs_stream)
    int64_t xs_nb;
    size_t xs_mask_off, xs_sign_off, xs_seg_bytes, xs_mask_bytes, xs_sign_bytes;
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(XT_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define XT_HIP(call)                                    \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// Device workspaces (xtern_workspace.h): one buffer per (device, stream,
// host thread, kind), never freed while queued work or a captured graph may
// use it, never allocated during graph capture.
//   kind 0: quantised activations, inv scales and row sums of the f32 entry
//           points, padded copies of caller activations;
//   kind 1: split-K partial-sum planes and arrival counters.  Zeroed when
//           allocated; every product launch leaves the counters zero again
//           (the last workgroup of a tile resets its counter);
//   kind 2: the MLP's gate / up rows and requantised intermediate.
int hipb_device(int* d) { return (int)hipGetDevice(d); }
int hipb_alloc(void** p, size_t n) { return (int)hipMalloc(p, n); }
int hipb_free(void* p) { return (int)hipFree(p); }
int hipb_capturing(void* s, bool* c) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(static_cast<hipStream_t>(s), &st);
    *c = st != hipStreamCaptureStatusNone;
    return (int)e;
}
int hipb_zero(void* p, size_t n, void* s) {
    return (int)hipMemsetAsync(p, 0, n, static_cast<hipStream_t>(s));
}
int hipb_sync() { return (int)hipDeviceSynchronize(); }
const char* hipb_str(int e) { return hipGetErrorString((hipError_t)e); }

xt::WorkspaceTable& ws_table() {
    static xt::WorkspaceTable* t = new xt::WorkspaceTable(xt::WsBackend{
        hipb_device, hipb_alloc, hipb_free, hipb_capturing, hipb_zero, hipb_sync, hipb_str});
    return *t;  // (left to process teardown: HIP may be gone by static destruction)
}

// Hands the calling thread's buffers to the table's pool when the thread
// ends (constructed on a thread's first workspace request).
struct WsThreadGuard {
    ~WsThreadGuard() { ws_table().thread_exit(std::this_thread::get_id()); }
};
thread_local WsThreadGuard g_ws_thread_guard;

int ws_status(int st, const std::string& err) {
    switch (st) {
        case xt::WorkspaceTable::kOk: return XT_OK;
        case xt::WorkspaceTable::kNoMem: return fail(XT_ERR_NOMEM, err);
        case xt::WorkspaceTable::kCapture: return fail(XT_ERR_UNSUPPORTED, err);
        default: return fail(XT_ERR_HIP, err);
    }
}

// Caller-provided scratch (the allocation-free entry point): requests of
// kind 0 are carved from it in order; other kinds are refused.
struct Scratch {
    char* base;
    size_t cap;
    size_t used;
};

int workspace(hipStream_t s, size_t bytes, void** out, int kind = 0, Scratch* sc = nullptr) {
    if (sc) {
        if (kind != 0)
            return fail(XT_ERR_UNSUPPORTED,
                        "this product configuration needs a split-K workspace, which the "
                        "allocation-free entry point does not provide");
        const size_t need = (bytes + 255) / 256 * 256;
        if (sc->used + need > sc->cap)
            return fail(XT_ERR_INVALID, "needs " + std::to_string(sc->used + need) +
                                            " bytes of scratch, the static scratch holds " +
                                            std::to_string(sc->cap));
        *out = sc->base + sc->used;
        sc->used += need;
        return XT_OK;
    }
    (void)&g_ws_thread_guard;  // (constructs this thread's guard)
    std::string err;
    const int st = ws_table().get(s, bytes, kind, kind == 1, out, &err);
    return ws_status(st, err);
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Split-K workspace of a stream: [counters: g_cnt_region bytes][planes].  The
// counter region only grows by replacing every split-K buffer (zeroed).
std::mutex g_cnt_mu;
size_t g_cnt_region = 1 << 16;

int splitk_workspace(hipStream_t s, size_t cbytes, size_t pbytes, void** out, size_t* region,
                     Scratch* sc) {
    {
        std::lock_guard<std::mutex> lk(g_cnt_mu);
        if (cbytes > g_cnt_region) {
            g_cnt_region = cbytes;
            ws_table().mark_stale(1);
        }
        *region = g_cnt_region;
    }
    return workspace(s, *region + pbytes, out, 1, sc);
}

int check_weights(const xt_weights* w) {
    if (!w) return fail(XT_ERR_INVALID, "weights handle is NULL");
    return XT_OK;
}

// Shared tail of every product entry point: quantised activations (ldq with
// zero padding up to nch*CH, 16-byte aligned) are ready; launch the product.
// Int8 / Int4 weights: the GEMV (which sums the activation rows itself) over
// blocks of at most 16 rows that fit its LDS activation stage.
int run_product_int(const xt_weights* const* ws, int n, const int8_t* q, int ldq, const float* inv,
                    int64_t M, float* const* ys, int32_t* acc, hipStream_t s) {
    const int fmt = ws[0]->fmt;
    const int nch = (int)ws[0]->nch;
    // The staging-free GEMV takes 16 rows per launch at any K it accepts;
    // the staged one as many as its LDS stage holds.
    const bool direct = xt::gemv2_takes(fmt, nch);
    int mb = 16;
    while (!direct && mb > 1 && !xt::gemv_fits(fmt, mb, nch, 16, xt::gemv_ncw(16))) mb >>= 1;
    if (!direct && !xt::gemv_fits(fmt, mb, nch, 16, xt::gemv_ncw(16)))
        return fail(XT_ERR_UNSUPPORTED, "in_dim too large for the Int8/Int4 product");
    const int waves = direct ? 16 : xt::int_gemv_waves(fmt, mb, nch);
    int ng_total = 0;
    for (int p = 0; p < n; ++p) ng_total += (int)((ws[p]->N + 15) / 16);
    const int rg = xt::gemv_row_groups(fmt, nch, ng_total);
    for (int64_t m0 = 0; m0 < M; m0 += mb) {
        const int mr = (int)std::min<int64_t>(mb, M - m0);
        xt::MMArgs a;
        memset(&a, 0, sizeof a);
        int tiles = 0;
        for (int p = 0; p < n; ++p) {
            const int ng = (int)((ws[p]->N + 15) / 16);
            a.proj[p].tiles = ws[p]->tiles;
            a.proj[p].ws = ws[p]->ws;
            a.proj[p].y = ys[p] + m0 * ws[p]->N;
            a.proj[p].acc = (n == 1 && acc) ? acc + m0 * ws[p]->N : nullptr;
            a.proj[p].N = (int)ws[p]->N;
            a.proj[p].tile0 = tiles;
            tiles += (ng + rg - 1) / rg;
        }
        a.rg = rg;
        a.nproj = n;
        a.q = q + m0 * ldq;
        a.inv = inv + m0;
        a.M = mr;
        a.ldq = ldq;
        a.nch = nch;
        a.cps = nch;
        hipError_t e = xt::launch_gemv(fmt, a, tiles, waves, s);
        if (e != hipSuccess) return hip_fail(e, "Int8/Int4 GEMV launch");
    }
    return XT_OK;
}

// XorSparse compact stream: one launch per projection and 16 token rows
// (ldq >= ceil(K/64) * 64: the callers pad to whole 256-column chunks).
int run_product_xs(const xt_weights* const* ws, int n, const int8_t* q, int ldq, const float* inv,
                   int64_t M, float* const* ys, int32_t* acc, hipStream_t s) {
    const int mb = xt::xs_max_rows();
    for (int p = 0; p < n; ++p) {
        const xt_weights* w = ws[p];
        for (int64_t m0 = 0; m0 < M; m0 += mb) {
            const int mr = (int)std::min<int64_t>(mb, M - m0);
            xt::XsArgs a;
            memset(&a, 0, sizeof a);
            a.seg = reinterpret_cast<const uint32_t*>(w->tiles);
            a.mask = reinterpret_cast<const uint32_t*>(w->tiles + w->xs_mask_off);
            a.sign = reinterpret_cast<const uint32_t*>(w->tiles + w->xs_sign_off);
            a.seg_bytes = (unsigned)w->xs_seg_bytes;
            a.mask_bytes = (unsigned)w->xs_mask_bytes;
            a.sign_bytes = (unsigned)w->xs_sign_bytes;
            a.q = q + m0 * ldq;
            a.q_bytes = (unsigned)((size_t)mr * ldq);
            a.ldq = ldq;
            a.inv = inv + m0;
            a.ws = w->ws;
            a.y = ys[p] + m0 * w->N;
            a.acc = (n == 1 && acc) ? acc + m0 * w->N : nullptr;
            a.M = mr;
            a.N = (int)w->N;
            a.nb = (int)w->xs_nb;
            hipError_t e = xt::launch_xs_gemv(a, s);
            if (e != hipSuccess) return hip_fail(e, "XorSparse stream GEMV launch");
        }
    }
    return XT_OK;
}

// Row groups from which a single decode product takes the streaming GEMV.
constexpr int kGStreamMinGroups = 16384;

// Compute units of the current device (cached per device).
int device_cus(int* cus) {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    XT_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(mu);
    if ((int)cache.size() <= dev) cache.resize((size_t)dev + 1, 0);
    if (cache[(size_t)dev] == 0)
        XT_HIP(hipDeviceGetAttribute(&cache[(size_t)dev], hipDeviceAttributeMultiprocessorCount, dev));
    *cus = cache[(size_t)dev];
    return XT_OK;
}

int run_product(const xt_weights* const* ws, int n, const int8_t* q, int ldq, const float* inv,
                const int32_t* rowsum, int64_t M, float* const* ys, int32_t* acc,
                hipStream_t s, Scratch* sc = nullptr) {
    const int fmt = ws[0]->fmt;
    if (xt::is_int_format(fmt)) return run_product_int(ws, n, q, ldq, inv, M, ys, acc, s);
    if (fmt == XT_XORSPARSE_STREAM) return run_product_xs(ws, n, q, ldq, inv, M, ys, acc, s);
    int ng_total = 0;
    for (int p = 0; p < n; ++p) ng_total += (int)((ws[p]->N + 15) / 16);
    // Tall matrices at decode sizes: the streaming GEMV (every wave walks its
    // own row groups; xtern_gstream.hip).  Measured on MI355X: 121 stacked C0
    // matrices (52272 row groups) at M = 1 6.5 TB/s against 4.7 TB/s on the
    // one-shot GEMV; 17280 row groups at M = 2 / 4 / 8 5.9 / 5.4 / 5.2 TB/s.
    if (n == 1 && M >= 1 && M <= 16 && (fmt == XT_PACK4 || fmt == XT_XORSPARSE) &&
        ng_total >= kGStreamMinGroups && xt::gstream_fits(fmt, (int)M, (int)ws[0]->nch) &&
        (reinterpret_cast<uintptr_t>(q) & 15) == 0 && ldq % 16 == 0) {
        int cus = 0;
        if (int rc = device_cus(&cus)) return rc;
        xt::GStreamArgs g;
        memset(&g, 0, sizeof g);
        g.tiles = ws[0]->tiles;
        g.ws = ws[0]->ws;
        g.y = ys[0];
        g.acc = acc;
        g.q = q;
        g.inv = inv;
        g.M = (int)M;
        g.ldq = ldq;
        g.nch = (int)ws[0]->nch;
        g.NG = ng_total;
        g.N = (int)ws[0]->N;
        hipError_t e = xt::launch_gstream(fmt, g, 4 * cus, M == 1 ? 2 : 4, s);
        if (e != hipSuccess) return hip_fail(e, "streaming GEMV launch");
        return XT_OK;
    }
    const xt::MMConfig cfg =
        xt::choose_config(fmt, (int)M, ng_total, (int)ws[0]->nch, rowsum != nullptr);
    xt::MMArgs a;
    memset(&a, 0, sizeof a);
    int tiles = 0, cols = 0;
    for (int p = 0; p < n; ++p) {
        const int ng = (int)((ws[p]->N + 15) / 16);
        a.proj[p].tiles = ws[p]->tiles;
        a.proj[p].ws = ws[p]->ws;
        a.proj[p].y = ys[p];
        a.proj[p].acc = (n == 1) ? acc : nullptr;
        a.proj[p].N = (int)ws[p]->N;
        a.proj[p].tile0 = tiles;
        a.proj[p].col0 = cols;
        tiles += (ng + cfg.nb - 1) / cfg.nb;
        cols += ng * 16;
    }
    a.nproj = n;
    a.q = q;
    a.inv = inv;
    a.rowsum = rowsum;
    a.M = (int)M;
    a.ldq = ldq;
    a.nch = (int)ws[0]->nch;
    a.cps = (a.nch + cfg.splitk - 1) / cfg.splitk;
    const int64_t gy = (M + 16 * cfg.mb - 1) / (16 * cfg.mb);
    if (gy > 65535) return fail(XT_ERR_UNSUPPORTED, "M too large for one launch");
    if (cfg.kind == 2) {
        a.rg = cfg.nb;
        hipError_t e = xt::launch_gemv(fmt, a, tiles, cfg.waves, s);
        if (e != hipSuccess) return hip_fail(e, "ternary GEMV launch");
        return XT_OK;
    }
    if (cfg.kind == 1 || cfg.kind == 3) {
        if (cfg.splitk > 1) {
            void* wsp = nullptr;
            size_t region = 0;
            const size_t pbytes = align_up((size_t)cfg.splitk * M * cols * sizeof(int32_t), 256);
            if (int rc = splitk_workspace(s, 0, pbytes, &wsp, &region, sc)) return rc;
            a.part = reinterpret_cast<int32_t*>(static_cast<char*>(wsp) + region);
        }
        a.ldp = cols;
        hipError_t e = cfg.kind == 3 ? xt::launch_gemm32(a, tiles, cfg.splitk, s)
                                     : xt::launch_gemm(fmt, a, tiles, cfg.splitk, s);
        if (e != hipSuccess) return hip_fail(e, "ternary GEMM launch");
        return XT_OK;
    }
    if (cfg.splitk > 1) {
        // Counters first, at a fixed offset, so every call finds them zero
        // (launches reset the counters they use; the planes after them are
        // fully overwritten before they are read).
        const size_t cbytes = align_up((size_t)tiles * gy * sizeof(unsigned), 4096);
        const size_t pbytes = align_up((size_t)cfg.splitk * M * cols * sizeof(int32_t), 256);
        void* wsp = nullptr;
        size_t region = 0;
        if (int rc = splitk_workspace(s, cbytes, pbytes, &wsp, &region, sc)) return rc;
        a.cnt = static_cast<unsigned*>(wsp);
        a.part = reinterpret_cast<int32_t*>(static_cast<char*>(wsp) + region);
        a.ldp = cols;
    }
    hipError_t e = xt::launch_mm(fmt, cfg, a, tiles, s);
    if (e != hipSuccess) return hip_fail(e, "ternary product launch");
    return XT_OK;
}

// Whether the product for M rows needs the quantiser's activation row sums:
// only the Pack5 prefill GEMM multiplies codes with a caller row sum; the
// other kernels decode signed weights or sum the rows themselves (measured:
// computing them for the long-K kernel costs more in the quantiser than the
// kernel's own extra MFMA per k-step saves).
bool wants_rowsum(const xt_weights* w, int64_t M) {
    if (xt::is_int_format(w->fmt) || w->fmt == XT_XORSPARSE_STREAM) return false;
    return xt::choose_config(w->fmt, (int)M, 0, (int)w->nch, true).kind == 1;
}

int check_group(const xt_weights* const* ws, int n, const void* in, int64_t M, float* const* ys) {
    if (!ws || n < 1 || n > 4) return fail(XT_ERR_INVALID, "need 1..4 weight handles");
    for (int p = 0; p < n; ++p) {
        if (check_weights(ws[p])) return XT_ERR_INVALID;
        if (ws[p]->K != ws[0]->K || ws[p]->fmt != ws[0]->fmt)
            return fail(XT_ERR_INVALID, "fused projections must share in_dim and format");
        if (M > 0 && (!ys || !ys[p])) return fail(XT_ERR_INVALID, "output pointer is NULL");
    }
    if (M < 0) return fail(XT_ERR_INVALID, "M must be >= 0");
    if (M > 0 && !in) return fail(XT_ERR_INVALID, "input pointer is NULL");
    if (M > (int64_t)1 << 24) return fail(XT_ERR_UNSUPPORTED, "M above 2^24 is not supported");
    return XT_OK;
}

int linear_q(const xt_weights* const* ws, int n, const int8_t* q, const float* inv,
             const int32_t* user_rowsum, int64_t M, float* const* ys, int32_t* acc,
             hipStream_t s) {
    if (int rc = check_group(ws, n, q, M, ys)) return rc;
    if (M > 0 && !inv) return fail(XT_ERR_INVALID, "inv_scale pointer is NULL");
    if (M == 0) return XT_OK;
    const int64_t K = ws[0]->K;
    const int64_t kpad = ws[0]->nch * xt::chunk_cols(ws[0]->fmt);
    const bool need_rowsum = wants_rowsum(ws[0], M);
    const bool direct = (kpad == K) && ((((uintptr_t)q) & 15) == 0);
    if (direct && user_rowsum)
        return run_product(ws, n, q, (int)K, inv, user_rowsum, M, ys, acc, s);
    if (direct && !need_rowsum)
        return run_product(ws, n, q, (int)K, inv, nullptr, M, ys, acc, s);
    // Padded copy and/or row sums in the workspace.
    const size_t qbytes = direct ? 0 : align_up((size_t)M * kpad, 256);
    void* wsp = nullptr;
    if (int rc = workspace(s, qbytes + align_up((size_t)M * 4, 256), &wsp)) return rc;
    int8_t* qpad = direct ? nullptr : static_cast<int8_t*>(wsp);
    int32_t* rowsum = reinterpret_cast<int32_t*>(static_cast<char*>(wsp) + qbytes);
    hipError_t e = xt::launch_rowsum(q, K, (int)M, (int)K, qpad, (int)kpad, rowsum, s);
    if (e != hipSuccess) return hip_fail(e, "row-sum launch");
    return run_product(ws, n, direct ? q : qpad, (int)(direct ? K : kpad), inv, rowsum, M, ys, acc,
                       s);
}

// Small inputs on the GEMV: the kernel quantises the f32 rows itself (no
// separate quantiser launch).  Returns 1 when the case does not apply.
// Largest workgroups x K for which the decode GEMV quantises its f32 row in
// every workgroup rather than after a separate quantiser launch.
constexpr int64_t kFusedRowReads = 1200 * 1024;

int gemv_fused_quant(const xt_weights* const* ws, int n, const float* x, int64_t M,
                     float* const* ys, int mode, hipStream_t s) {
    const int fmt = ws[0]->fmt;
    if (fmt == XT_XORSPARSE_STREAM) return 1;  // (its kernel takes i8 rows)
    const int64_t K = ws[0]->K;
    const int nch = (int)ws[0]->nch;
    const bool direct = !xt::is_int_format(fmt);
    // staging-free GEMV: one row only (measured: K = 6912, 8.1 -> 6.6 us at
    // M = 1; already slower at M = 2 for N = 6912, where every workgroup
    // re-reads and re-quantises the rows)
    if (direct && M > 1) return 1;
    // Int8 / Int4 on the staging-free GEMV: the separate quantiser costs a
    // few us against the ~50 us of a 128256-row head (measured: Int8 head
    // forward 158 us fused on the staged GEMV, 50 us product on this one)
    if (xt::is_int_format(fmt) && xt::gemv2_takes(fmt, nch)) return 1;
    if (M > 16 || M * K > (direct ? xt::kGemv2FusedQuantMax : xt::kGemvFusedQuantMax) ||
        (((uintptr_t)x) & 15) || (K & 3))
        return 1;
    int ng_total = 0;
    for (int p = 0; p < n; ++p) ng_total += (int)((ws[p]->N + 15) / 16);
    // The fused GEMV saves the quantiser launch, but every workgroup reads
    // and quantises the whole f32 row: worth it while workgroups x K stays
    // small (measured, Pack4 at M = 1: gate+up 2 x 6912 rows at K = 2560,
    // 432 workgroups, 6.6 us fused vs 7.2 quantiser + GEMV; K = 4096 ->
    // 14336, 448 workgroups, 10.1 vs 8.6).
    int waves = 16;
    if (xt::is_int_format(fmt)) {
        waves = xt::int_gemv_waves(fmt, (int)M, nch);
    } else if (!(fmt == XT_PACK5 && nch > 16)) {
        // (Pack5 above 16 chunks always fuses: 8640 -> 3200, 200 workgroups,
        // 7.8 vs 8.7 us; at or below, as the other formats: 3200 -> 3200 4.7
        // vs 6.1, 3200 -> 8640 with 540 workgroups 8.9 vs 7.5)
        const int g = xt::gemv_row_groups(fmt, nch, ng_total);
        if ((int64_t)((ng_total + g - 1) / g) * K > kFusedRowReads) return 1;
    }
    // Ternary tiles take the staging-free GEMV (one chunk per wave, so
    // K <= 16 chunks); Int8 / Int4 the staged one (one piece per thread).
    const int segs = xt::chunk_cols(fmt) / 16;
    const int rg = direct ? xt::gemv_row_groups(fmt, nch, ng_total) : 1;
    if (direct ? (M * K > xt::gemv2_fused_max(fmt, nch, rg))
               : (!xt::gemv_fits(fmt, (int)M, nch, waves, xt::gemv_ncw(waves)) ||
                  M * nch * segs > (int64_t)waves * 64))
        return 1;
    xt::MMArgs a;
    memset(&a, 0, sizeof a);
    int tiles = 0;
    // (Int8 / Int4 rows quantised in the kernel run on the staged GEMV)
    for (int p = 0; p < n; ++p) {
        a.proj[p].tiles = ws[p]->tiles;
        a.proj[p].ws = ws[p]->ws;
        a.proj[p].y = ys[p];
        a.proj[p].N = (int)ws[p]->N;
        a.proj[p].tile0 = tiles;
        tiles += (int)((ws[p]->N + 15) / 16 + rg - 1) / rg;
    }
    a.nproj = n;
    a.M = (int)M;
    a.nch = nch;
    a.cps = nch;
    a.x = x;
    a.rg = rg;
    a.ldx = K;
    a.K = (int)K;
    a.mode = mode;
    hipError_t e = xt::launch_gemv(fmt, a, tiles, waves, s);
    if (e != hipSuccess) return hip_fail(e, "fused GEMV launch");
    return XT_OK;
}

int linear_f32(const xt_weights* const* ws, int n, const float* x, int64_t M, float* const* ys,
               int mode, hipStream_t s, Scratch* sc = nullptr) {
    if (int rc = check_group(ws, n, x, M, ys)) return rc;
    if (mode != XT_QUANT_AVX512 && mode != XT_QUANT_SCALAR)
        return fail(XT_ERR_INVALID, "unknown quantisation mode");
    if (M == 0) return XT_OK;
    const int fr = gemv_fused_quant(ws, n, x, M, ys, mode, s);
    if (fr <= 0) return fr;
    const int64_t K = ws[0]->K;
    const int64_t kpad = ws[0]->nch * xt::chunk_cols(ws[0]->fmt);
    const size_t qbytes = align_up((size_t)M * kpad, 256);
    const size_t fbytes = align_up((size_t)M * 4, 256);
    void* wsp = nullptr;
    if (int rc = workspace(s, qbytes + 2 * fbytes, &wsp, 0, sc)) return rc;
    int8_t* q = static_cast<int8_t*>(wsp);
    float* inv = reinterpret_cast<float*>(static_cast<char*>(wsp) + qbytes);
    int32_t* rowsum = wants_rowsum(ws[0], M)
                          ? reinterpret_cast<int32_t*>(static_cast<char*>(wsp) + qbytes + fbytes)
                          : nullptr;
    hipError_t e = xt::launch_quantize(x, K, (int)M, (int)K, q, (int)kpad, inv, rowsum, mode, s);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    return run_product(ws, n, q, (int)kpad, inv, rowsum, M, ys, nullptr, s, sc);
}

int launch_mid(const xt::MidArgs& a, int64_t M, hipStream_t s) {
    hipError_t e = xt::launch_mlp_mid(a, (int)M, s);
    if (e != hipSuccess) return hip_fail(e, "MLP activation / norm launch");
    return XT_OK;
}

int check_row_len(int64_t n) {
    if (n <= 0) return fail(XT_ERR_INVALID, "row length must be positive");
    if (n > xt::mid_max_cols())
        return fail(XT_ERR_UNSUPPORTED, "row length " + std::to_string(n) + " above " +
                                            std::to_string(xt::mid_max_cols()) + " is not supported");
    return XT_OK;
}

// gate+up on one quantised input (done by the caller: `first` runs the
// product into g/u), then activation [+ norm] + requantisation, then down.
// Shared by xt_ternary_mlp_q and xt_ternary_mlp_f32.
int mlp_run(const xt_weights* gate, const xt_weights* up, const xt_weights* down,
            const float* norm_w, float eps, int act, int mode, int64_t M, float* y, hipStream_t s,
            const void* in, bool in_is_f32, const float* inv_in) {
    if (check_weights(gate) || check_weights(up) || check_weights(down)) return XT_ERR_INVALID;
    if (gate->K != up->K || gate->N != up->N || gate->fmt != up->fmt)
        return fail(XT_ERR_INVALID, "gate and up projections must have the same shape and format");
    if (xt::is_int_format(gate->fmt))
        return fail(XT_ERR_UNSUPPORTED, "gate/up projections must be ternary");
    if (gate->fmt == XT_XORSPARSE_STREAM || down->fmt == XT_XORSPARSE_STREAM)
        return fail(XT_ERR_UNSUPPORTED,
                    "the fused MLP takes tile formats; run XorSparse stream weights as separate products");
    if (down->K != gate->N)
        return fail(XT_ERR_INVALID, "down in_dim " + std::to_string(down->K) +
                                        " != intermediate size " + std::to_string(gate->N));
    if (mode != XT_QUANT_AVX512 && mode != XT_QUANT_SCALAR)
        return fail(XT_ERR_INVALID, "unknown quantisation mode");
    if (M < 0) return fail(XT_ERR_INVALID, "M must be >= 0");
    if (M == 0) return XT_OK;
    if (!in || !y || (!in_is_f32 && !inv_in)) return fail(XT_ERR_INVALID, "NULL pointer");
    if (int rc = check_row_len(gate->N)) return rc;
    const int64_t I = gate->N;
    const int64_t kpad = down->nch * xt::chunk_cols(down->fmt);
    const size_t fb = align_up((size_t)M * I * sizeof(float), 256);
    const size_t qb = align_up((size_t)M * kpad, 256);
    const size_t sb = align_up((size_t)M * 4, 256);
    void* wsp = nullptr;
    if (int rc = workspace(s, 2 * fb + qb + 2 * sb, &wsp, 2)) return rc;
    char* base = static_cast<char*>(wsp);
    float* g = reinterpret_cast<float*>(base);
    float* u = reinterpret_cast<float*>(base + fb);
    int8_t* qm = reinterpret_cast<int8_t*>(base + 2 * fb);
    float* invm = reinterpret_cast<float*>(base + 2 * fb + qb);
    int32_t* rsm = reinterpret_cast<int32_t*>(base + 2 * fb + qb + sb);
    const xt_weights* gu[2] = {gate, up};
    float* gy[2] = {g, u};
    int rc = in_is_f32 ? linear_f32(gu, 2, static_cast<const float*>(in), M, gy, mode, s)
                       : linear_q(gu, 2, static_cast<const int8_t*>(in), inv_in, nullptr, M, gy,
                                  nullptr, s);
    if (rc) return rc;
    xt::MidArgs a;
    memset(&a, 0, sizeof a);
    a.gate = g;
    a.up = u;
    a.ldg = I;
    a.n = (int)I;
    a.act = act;
    a.norm_w = norm_w;
    a.eps = eps;
    a.mode = mode;
    a.q = qm;
    a.ldq = (int)kpad;
    a.inv = invm;
    // row sums of the requantised rows only for a down product that uses them
    a.rowsum = wants_rowsum(down, M) ? rsm : nullptr;
    if ((rc = launch_mid(a, M, s))) return rc;
    float* ys[1] = {y};
    const xt_weights* dw[1] = {down};
    return run_product(dw, 1, qm, (int)kpad, invm, a.rowsum, M, ys, nullptr, s);
}

}  // namespace

// Error reporting for the other host source files (xtern_container.cpp).
int xt_internal_fail(int code, const std::string& msg) { return fail(code, msg); }

extern "C" {

const char* xt_version(void) { return "xtern 0.1 gfx950"; }

const char* xt_last_error(void) { return g_err.c_str(); }

size_t xt_tile_bytes(int fmt, int64_t in_dim, int64_t out_dim) {
    if (in_dim <= 0 || out_dim <= 0 || fmt < 0 || fmt > 4) return 0;
    return xt::tile_bytes(fmt, in_dim, out_dim);
}

int xt_repack_host(int fmt, int64_t in_dim, int64_t out_dim, const void* host_bytes,
                   size_t nbytes, void* tiles_out) {
    if (!host_bytes || !tiles_out) return fail(XT_ERR_INVALID, "NULL buffer");
    if (fmt < 0 || fmt > 4)
        return fail(XT_ERR_INVALID, "unknown tile format (XorSparse stream: xt_xorsparse_stream_host)");
    std::string err;
    if (xt::repack(fmt, in_dim, out_dim, host_bytes, nbytes, tiles_out, &err))
        return fail(XT_ERR_INVALID, err);
    return XT_OK;
}

namespace {

// A handle with device memory for `fmt`'s tiles and N scales (scales
// uploaded, tiles left for the caller to fill).
int weights_alloc(int fmt, int64_t K, int64_t N, const float* w_scales, xt_weights** out,
                  size_t bytes = 0) {
    xt_weights* w = new (std::nothrow) xt_weights();
    if (!w) return fail(XT_ERR_NOMEM, "handle");
    w->fmt = fmt;
    w->K = K;
    w->N = N;
    w->nch = (K + xt::chunk_cols(fmt) - 1) / xt::chunk_cols(fmt);
    w->tile_bytes = bytes ? bytes : xt::tile_bytes(fmt, K, N);
    hipError_t e = hipGetDevice(&w->device);
    if (e == hipSuccess) e = hipMalloc(&w->tiles, w->tile_bytes);
    if (e == hipSuccess) e = hipMalloc(&w->ws, (size_t)N * sizeof(float));
    if (e == hipSuccess)
        e = hipMemcpy(w->ws, w_scales, (size_t)N * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (w->tiles) (void)hipFree(w->tiles);
        if (w->ws) (void)hipFree(w->ws);
        delete w;
        return hip_fail(e, "weight allocation");
    }
    *out = w;
    return XT_OK;
}

// XT_XORSPARSE_STREAM: the blob re-laid as masks + set-order sign stream
// (build_xs_stream), uploaded as one buffer.
int weights_create_xs(int64_t K, int64_t N, const void* blob, size_t nbytes, const float* w_scales,
                      xt_weights** out) {
    if (K > (int64_t)xt::xs_max_blocks() * 64)
        return fail(XT_ERR_UNSUPPORTED, "XorSparse stream weights take in_dim up to " +
                                            std::to_string(xt::xs_max_blocks() * 64));
    if (N > (int64_t)1 << 30) return fail(XT_ERR_UNSUPPORTED, "out_dim above 2^30 is not supported");
    std::vector<uint8_t> host;
    xt::XsLayout L;
    std::string err;
    if (xt::build_xs_stream(K, N, static_cast<const uint8_t*>(blob), nbytes, &host, &L, &err))
        return fail(XT_ERR_INVALID, err);
    xt_weights* w = nullptr;
    if (int rc = weights_alloc(XT_XORSPARSE_STREAM, K, N, w_scales, &w, L.total)) return rc;
    w->xs_nb = L.nb;
    w->xs_mask_off = L.mask_off;
    w->xs_sign_off = L.sign_off;
    w->xs_seg_bytes = (size_t)(L.ng * L.nb) * 4;
    w->xs_mask_bytes = (size_t)(L.ng * L.nb) * 128;
    w->xs_sign_bytes = L.sign_bytes;
    hipError_t e = hipMemcpy(w->tiles, host.data(), L.total, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)xt_weights_destroy(w);
        return hip_fail(e, "weight upload");
    }
    *out = w;
    return XT_OK;
}

}  // namespace

int xt_xorsparse_stream_host(int64_t in_dim, int64_t out_dim, const void* blob, size_t nbytes,
                             void* out, size_t cap, size_t* len, uint64_t* sections) {
    if (!blob || !len) return fail(XT_ERR_INVALID, "NULL blob or length pointer");
    if (in_dim <= 0 || out_dim <= 0) return fail(XT_ERR_INVALID, "in_dim and out_dim must be positive");
    std::vector<uint8_t> host;
    xt::XsLayout L;
    std::string err;
    if (xt::build_xs_stream(in_dim, out_dim, static_cast<const uint8_t*>(blob), nbytes, &host, &L, &err))
        return fail(XT_ERR_INVALID, err);
    *len = L.total;
    if (sections) {
        sections[0] = L.seg_off;
        sections[1] = L.mask_off;
        sections[2] = L.sign_off;
    }
    if (out) {
        if (cap < L.total) return fail(XT_ERR_INVALID, "buffer too small for the XorSparse stream");
        memcpy(out, host.data(), L.total);
    }
    return XT_OK;
}

int xt_weights_create(int fmt, int64_t in_dim, int64_t out_dim, const void* host_bytes,
                      size_t nbytes, const float* w_scales, xt_weights** out) {
    if (!out) return fail(XT_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (!host_bytes || !w_scales) return fail(XT_ERR_INVALID, "NULL weight bytes or w_scales");
    if (fmt < 0 || fmt > XT_XORSPARSE_STREAM) return fail(XT_ERR_INVALID, "unknown weight format");
    if (in_dim <= 0 || out_dim <= 0) return fail(XT_ERR_INVALID, "in_dim and out_dim must be positive");
    if (fmt == XT_XORSPARSE_STREAM) return weights_create_xs(in_dim, out_dim, host_bytes, nbytes, w_scales, out);
    const size_t tb = xt::tile_bytes(fmt, in_dim, out_dim);
    std::vector<uint8_t> host;
    try {
        host.resize(tb);
    } catch (...) {
        return fail(XT_ERR_NOMEM, "host repack buffer");
    }
    std::string err;
    if (xt::repack(fmt, in_dim, out_dim, host_bytes, nbytes, host.data(), &err))
        return fail(XT_ERR_INVALID, err);
    xt_weights* w = nullptr;
    if (int rc = weights_alloc(fmt, in_dim, out_dim, w_scales, &w)) return rc;
    hipError_t e = hipMemcpy(w->tiles, host.data(), tb, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)xt_weights_destroy(w);
        return hip_fail(e, "weight upload");
    }
    *out = w;
    return XT_OK;
}

int xt_hf_destripe(int fmt, int64_t in_dim, int64_t out_dim, const void* stored, size_t nbytes,
                   void* packed_out) {
    if (!stored || !packed_out) return fail(XT_ERR_INVALID, "NULL buffer");
    std::string err;
    if (xt::hf_destripe(fmt, in_dim, out_dim, static_cast<const uint8_t*>(stored), nbytes,
                        static_cast<uint8_t*>(packed_out), &err))
        return fail(XT_ERR_INVALID, err);
    return XT_OK;
}

int xt_weights_create_hf(int fmt, int64_t in_dim, int64_t out_dim, const void* stored,
                         size_t nbytes, float weight_scale, int is_inverted_scale,
                         xt_weights** out) {
    if (!out) return fail(XT_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (!stored) return fail(XT_ERR_INVALID, "NULL weight bytes");
    if (fmt != XT_PACK4 && fmt != XT_PACK5)
        return fail(XT_ERR_INVALID, "HF prepacked weights are Pack4 or Pack5 only");
    if (in_dim <= 0 || out_dim <= 0) return fail(XT_ERR_INVALID, "in_dim and out_dim must be positive");
    if (in_dim > (int64_t)1 << 30 || out_dim > (int64_t)1 << 30)
        return fail(XT_ERR_UNSUPPORTED, "in_dim/out_dim above 2^30 are not supported");
    const int64_t f = fmt == XT_PACK5 ? 5 : 4;
    if (out_dim % f != 0 || (uint64_t)nbytes != (uint64_t)(in_dim * (out_dim / f)))
        return fail(XT_ERR_INVALID,
                    "Tensor is not in pre-packed U8 ternary format: expected [" +
                        std::to_string(out_dim / f) + "][" + std::to_string(in_dim) +
                        "] bytes for out_dim " + std::to_string(out_dim) + ", got " +
                        std::to_string(nbytes));
    // loader/mod.rs:343-347 (f32 division) and :392 (one scale per row).
    const float ws = is_inverted_scale ? 1.0f / weight_scale : weight_scale;
    std::vector<float> scales;
    try {
        scales.assign((size_t)out_dim, ws);
    } catch (...) {
        return fail(XT_ERR_NOMEM, "host scale buffer");
    }
    xt_weights* w = nullptr;
    if (int rc = weights_alloc(fmt, in_dim, out_dim, scales.data(), &w)) return rc;
    void* dstored = nullptr;
    hipError_t e = hipMalloc(&dstored, nbytes);
    if (e == hipSuccess) e = hipMemcpy(dstored, stored, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = xt::launch_hf_tiles(fmt, static_cast<const uint8_t*>(dstored), in_dim, out_dim, w->tiles,
                                nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (dstored) {
        hipError_t ef = hipFree(dstored);
        if (e == hipSuccess) e = ef;
    }
    if (e != hipSuccess) {
        (void)xt_weights_destroy(w);
        return hip_fail(e, "HF weight upload");
    }
    *out = w;
    return XT_OK;
}

int xt_weights_read_tiles(const xt_weights* w, void* host_out, size_t nbytes) {
    if (check_weights(w)) return XT_ERR_INVALID;
    if (!host_out) return fail(XT_ERR_INVALID, "NULL buffer");
    if (nbytes < w->tile_bytes)
        return fail(XT_ERR_INVALID, "buffer holds " + std::to_string(nbytes) + " bytes, tiles need " +
                                        std::to_string(w->tile_bytes));
    int prev = 0;
    XT_HIP(hipGetDevice(&prev));
    if (prev != w->device) XT_HIP(hipSetDevice(w->device));
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(host_out, w->tiles, w->tile_bytes, hipMemcpyDeviceToHost);
    if (prev != w->device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "read tiles");
    return XT_OK;
}

int xt_weights_destroy(xt_weights* w) {
    if (!w) return XT_OK;
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != w->device) e = hipSetDevice(w->device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    hipError_t e1 = hipFree(w->tiles), e2 = hipFree(w->ws);
    if (prev != w->device) (void)hipSetDevice(prev);
    delete w;
    if (e != hipSuccess) return hip_fail(e, "weights destroy");
    if (e1 != hipSuccess) return hip_fail(e1, "weights destroy");
    if (e2 != hipSuccess) return hip_fail(e2, "weights destroy");
    return XT_OK;
}

int xt_weights_info(const xt_weights* w, int* fmt, int64_t* in_dim, int64_t* out_dim,
                    size_t* device_bytes) {
    if (check_weights(w)) return XT_ERR_INVALID;
    if (fmt) *fmt = w->fmt;
    if (in_dim) *in_dim = w->K;
    if (out_dim) *out_dim = w->N;
    if (device_bytes) *device_bytes = w->tile_bytes + (size_t)w->N * sizeof(float);
    return XT_OK;
}

int xt_quantize_i8(const float* x, int64_t M, int64_t K, int8_t* q, float* inv_scale, int mode,
                   void* stream) {
    return xt_quantize_i8_rowsum(x, M, K, q, inv_scale, nullptr, mode, stream);
}

int xt_quantize_i8_rowsum(const float* x, int64_t M, int64_t K, int8_t* q, float* inv_scale,
                          int32_t* rowsum, int mode, void* stream) {
    if (M < 0 || K <= 0) return fail(XT_ERR_INVALID, "need M >= 0 and K > 0");
    if (K > (int64_t)1 << 30 || M > (int64_t)1 << 31) return fail(XT_ERR_UNSUPPORTED, "size too large");
    if (mode != XT_QUANT_AVX512 && mode != XT_QUANT_SCALAR)
        return fail(XT_ERR_INVALID, "unknown quantisation mode");
    if (M == 0) return XT_OK;
    if (!x || !q || !inv_scale) return fail(XT_ERR_INVALID, "NULL pointer");
    hipError_t e = xt::launch_quantize(x, K, (int)M, (int)K, q, (int)K, inv_scale, rowsum, mode,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    return XT_OK;
}

int xt_ternary_linear_q(const xt_weights* w, const int8_t* q, const float* inv_scale, int64_t M,
                        float* y, int32_t* acc, void* stream) {
    const xt_weights* ws[1] = {w};
    float* ys[1] = {y};
    return linear_q(ws, 1, q, inv_scale, nullptr, M, ys, acc, static_cast<hipStream_t>(stream));
}

int xt_ternary_linear_q_rowsum(const xt_weights* w, const int8_t* q, const float* inv_scale,
                               const int32_t* rowsum, int64_t M, float* y, int32_t* acc,
                               void* stream) {
    if (M > 0 && !rowsum) return fail(XT_ERR_INVALID, "rowsum pointer is NULL");
    const xt_weights* ws[1] = {w};
    float* ys[1] = {y};
    return linear_q(ws, 1, q, inv_scale, rowsum, M, ys, acc, static_cast<hipStream_t>(stream));
}

int xt_ternary_linear_f32(const xt_weights* w, const float* x, int64_t M, float* y, int mode,
                          void* stream) {
    const xt_weights* ws[1] = {w};
    float* ys[1] = {y};
    return linear_f32(ws, 1, x, M, ys, mode, static_cast<hipStream_t>(stream));
}

int xt_ternary_linear_f32_noalloc(const xt_weights* w, const float* x, int64_t M, float* y,
                                  int mode, void* stream) {
    if (check_weights(w)) return XT_ERR_INVALID;
    void* base = nullptr;
    size_t cap = 0;
    hipError_t e = xt::scratch_region(&base, &cap);
    if (e != hipSuccess) return hip_fail(e, "static scratch address");
    Scratch sc{static_cast<char*>(base), cap, 0};
    const xt_weights* ws[1] = {w};
    float* ys[1] = {y};
    return linear_f32(ws, 1, x, M, ys, mode, static_cast<hipStream_t>(stream), &sc);
}

int xt_ternary_linear_multi_q(const xt_weights* const* ws, int n, const int8_t* q,
                              const float* inv_scale, int64_t M, float* const* ys, void* stream) {
    return linear_q(ws, n, q, inv_scale, nullptr, M, ys, nullptr, static_cast<hipStream_t>(stream));
}

int xt_ternary_linear_multi_f32(const xt_weights* const* ws, int n, const float* x, int64_t M,
                                float* const* ys, int mode, void* stream) {
    return linear_f32(ws, n, x, M, ys, mode, static_cast<hipStream_t>(stream));
}

int xt_activation_mul(int act, const float* gate, const float* up, int64_t M, int64_t n,
                      float* out, void* stream) {
    if (act < XT_ACT_RELU2_MUL || act > XT_ACT_SILU_MUL)
        return fail(XT_ERR_INVALID, "unknown activation " + std::to_string(act));
    if (M < 0) return fail(XT_ERR_INVALID, "M must be >= 0");
    if (int rc = check_row_len(n)) return rc;
    if (M == 0) return XT_OK;
    if (!gate || !up || !out) return fail(XT_ERR_INVALID, "NULL pointer");
    xt::MidArgs a;
    memset(&a, 0, sizeof a);
    a.gate = gate;
    a.up = up;
    a.ldg = n;
    a.n = (int)n;
    a.act = act;
    a.out = out;
    a.ldo = n;
    return launch_mid(a, M, static_cast<hipStream_t>(stream));
}

int xt_rms_norm(const float* x, const float* weight, int64_t M, int64_t n, float eps, float* y,
                void* stream) {
    if (M < 0) return fail(XT_ERR_INVALID, "M must be >= 0");
    if (int rc = check_row_len(n)) return rc;
    if (M == 0) return XT_OK;
    if (!x || !weight || !y) return fail(XT_ERR_INVALID, "NULL pointer");
    xt::MidArgs a;
    memset(&a, 0, sizeof a);
    a.gate = x;
    a.ldg = n;
    a.n = (int)n;
    a.act = xt::kActIdentity;
    a.norm_w = weight;
    a.eps = eps;
    a.out = y;
    a.ldo = n;
    return launch_mid(a, M, static_cast<hipStream_t>(stream));
}

int xt_ternary_mlp_q(const xt_weights* gate, const xt_weights* up, const xt_weights* down,
                     const float* norm_weight, float eps, int use_silu, const int8_t* q,
                     const float* inv_scale, int64_t M, float* y, int mode, void* stream) {
    const int act = !use_silu ? XT_ACT_RELU2_MUL
                              : (mode == XT_QUANT_SCALAR ? XT_ACT_SILU_INPLACE_SCALAR
                                                         : XT_ACT_SILU_INPLACE_AVX512);
    return mlp_run(gate, up, down, norm_weight, eps, act, mode, M, y,
                   static_cast<hipStream_t>(stream), q, false, inv_scale);
}

int xt_ternary_mlp_f32(const xt_weights* gate, const xt_weights* up, const xt_weights* down,
                       const float* norm_weight, float eps, int use_silu, const float* x,
                       int64_t M, float* y, int mode, void* stream) {
    // mlp.rs:51-100: one token with ternary gate/up and a ternary or Int8
    // down takes the fused path (silu_inplace); everything else the unfused
    // one (silu_mul_inplace).
    int act = XT_ACT_RELU2_MUL;
    const bool fused = M == 1 && down && (down->fmt != XT_INT4);
    if (use_silu)
        act = fused ? (mode == XT_QUANT_SCALAR ? XT_ACT_SILU_INPLACE_SCALAR
                                               : XT_ACT_SILU_INPLACE_AVX512)
                    : XT_ACT_SILU_MUL;
    return mlp_run(gate, up, down, norm_weight, eps, act, mode, M, y,
                   static_cast<hipStream_t>(stream), x, true, nullptr);
}

int xt_workspace_release(void) {
    std::string err;
    return ws_status(ws_table().release_all(&err), err);
}

struct xt_stack {
    xt::SStackArgs sargs;  // the one-launch plan: the streaming kernel (xtern_sstack.hip)
    int blocks;
    int device;
    void* dev_mem;  // ops, items, counters, scratch (one allocation)
    // the per-op plan: the ops in dependency order, run as library calls
    bool per_op = false;
    int64_t M = 0;
    int qmode = 0;
    std::vector<xt_stack_op> seq;
};

}  // extern "C"

namespace {

// Op order shared by both stack forms: ops that others wait for go as early
// as their own inputs allow, the rest keep the caller's order.  (Ops with no
// dependency path between them may run in any order: they share no buffers,
// per the contract in xtern.h.)  Every op still follows the op it depends on.
std::vector<int> stack_order(const xt_stack_op* ops, int nops, const std::vector<char>& pub) {
    std::vector<int> order;
    std::vector<char> placed((size_t)nops, 0);
    while ((int)order.size() < nops) {
        int pick = -1;
        for (int i = 0; i < nops && pick < 0; ++i)
            if (!placed[(size_t)i] && (ops[i].dep < 0 || placed[(size_t)ops[i].dep]) && pub[(size_t)i]) pick = i;
        for (int i = 0; i < nops && pick < 0; ++i)
            if (!placed[(size_t)i] && (ops[i].dep < 0 || placed[(size_t)ops[i].dep])) pick = i;
        placed[(size_t)pick] = 1;
        order.push_back(pick);
    }
    return order;
}

// Which plan runs a list faster, from measured figures (BitNet-2B
// projection shapes, weights streamed from HBM, MI355X):
//  * one call per op: about 4.7 us per op at M = 1, 6.5 at M <= 8 and 9.4 up
//    to M = 32 (launch to launch in a HIP graph), or the op's weight bytes at
//    2.7 TB/s where that is longer;
//  * one launch: the weights at 4.8 TB/s (M = 1), 3.4 (M <= 8) or 1.7 TB/s,
//    plus about 18 / 24 / 30 us per dependency level after the first: a
//    level's ops start only once the level before has published its outputs
//    (device-scope stores and a count; at M > 1 also the quantiser tasks and
//    their count), and each of its waves then walks its share of the op's
//    tiles one chunk at a time, where a one-op launch loads all of a
//    workgroup's tiles at once.
// The 30-layer projection stack with the residual dependency (2 levels) runs
// in one launch in 108.5 us against 562 us per op at M = 1; the strict chain
// (120 levels) took 2307 us in one launch against 602 us per op.
bool stack_prefers_per_op(const xt_stack_op* ops, int nops, int64_t M) {
    const double call_us = M == 1 ? 4.7 : (M <= 8 ? 6.5 : 9.4);
    const double call_bpus = 2.7e6, launch_bpus = M == 1 ? 4.8e6 : (M <= 8 ? 3.4e6 : 1.7e6);
    const double level_us = M == 1 ? 18.0 : (M <= 8 ? 24.0 : 30.0);
    std::vector<int> lvl((size_t)nops, 0);
    int depth = 0;
    double bytes = 0, per_op_us = 0;
    for (int i = 0; i < nops; ++i) {
        lvl[(size_t)i] = ops[i].dep < 0 ? 0 : lvl[(size_t)ops[i].dep] + 1;
        depth = std::max(depth, lvl[(size_t)i] + 1);
        double b = 0;
        for (int p = 0; p < ops[i].n; ++p) b += (double)ops[i].w[p]->tile_bytes;
        bytes += b;
        per_op_us += std::max(call_us, b / call_bpus);
    }
    const double launch_us = bytes / launch_bpus + level_us * (depth - 1);
    return per_op_us < launch_us;
}

// The per-op plan: the ops' shapes checked as the calls will check them, the
// list kept in its given order (every dep points to an earlier op).
int create_per_op(const xt_stack_op* ops, int nops, int64_t M, int qmode, xt_stack** out) {
    for (int i = 0; i < nops; ++i) {
        if (int rc = check_group(ops[i].w, ops[i].n, ops[i].x, M, ops[i].y))
            return fail(rc, "op " + std::to_string(i) + ": " + g_err);
    }
    int dev = 0;
    XT_HIP(hipGetDevice(&dev));
    xt_stack* st = new (std::nothrow) xt_stack();
    if (!st) return fail(XT_ERR_NOMEM, "stack handle");
    st->per_op = true;
    st->M = M;
    st->qmode = qmode;
    st->seq.assign(ops, ops + nops);
    st->device = dev;
    st->dev_mem = nullptr;
    *out = st;
    return XT_OK;
}

// The one-launch plan (xtern_sstack.hip, M = 1 .. 32).  Tasks in list order:
// the quantiser tasks (one per token) of ops without a dependency, then per
// op (in stack_order) its blocks of 16-row groups followed by the quantiser
// tasks of the ops that read its outputs.
int create_sstack(const xt_stack_op* ops, int nops, int64_t M, int mode, xt_stack** out) {
    if (nops > xt::kSStackMaxOps)
        return fail(XT_ERR_UNSUPPORTED, "at most " + std::to_string(xt::kSStackMaxOps) + " ops per stack");
    struct OpInfo {
        int fmt, nch, ldq, K, ngroups;
        size_t qoff;
    };
    std::vector<OpInfo> info((size_t)nops);
    std::vector<char> pub((size_t)nops, 0);
    size_t scratch = 0, ntasks = 0;
    for (int i = 0; i < nops; ++i) {
        const xt_stack_op& op = ops[i];
        const std::string at = "op " + std::to_string(i) + ": ";
        const int fmt = op.w[0]->fmt;
        const int ch = fmt == XT_PACK5 ? 320 : 256;
        OpInfo& f = info[(size_t)i];
        f.ngroups = 0;
        for (int p = 0; p < op.n; ++p) {
            const xt_weights* w = op.w[p];
            if (w->fmt != XT_PACK4 && w->fmt != XT_XORSPARSE && w->fmt != XT_PACK5)
                return fail(XT_ERR_UNSUPPORTED, at + "stack weights must be Pack4, Pack5 or XorSparse");
            if ((w->fmt == XT_PACK5) != (fmt == XT_PACK5))
                return fail(XT_ERR_UNSUPPORTED, at + "projections of one op must share the tile format");
            if (w->K != op.w[0]->K) return fail(XT_ERR_INVALID, at + "projections must share in_dim");
            if (w->K % 4 != 0 || w->nch * ch > xt::kSStackMaxRowBytes)
                return fail(XT_ERR_UNSUPPORTED, at + "in_dim must be a multiple of 4 and at most " +
                                                    std::to_string(xt::kSStackMaxRowBytes / ch * ch));
            f.ngroups += (int)((w->N + 15) / 16);
        }
        f.fmt = fmt == XT_PACK5 ? XT_PACK5 : XT_PACK4;
        f.K = (int)op.w[0]->K;
        f.nch = (int)op.w[0]->nch;
        // (each token's row fills whole 128-byte lines of its own: rows
        // written on one XCD are read with ordinary loads on others)
        f.ldq = (int)align_up((size_t)f.nch * ch, 128);
        f.qoff = scratch;
        scratch += align_up((size_t)M * f.ldq + 8 * (size_t)M, 256);  // rows, then sums and scales
        ntasks += (size_t)M + (size_t)f.ngroups;
        if (op.dep >= 0) pub[(size_t)op.dep] = 1;
    }
    int dev0 = 0, cus0 = 0;
    XT_HIP(hipGetDevice(&dev0));
    XT_HIP(hipDeviceGetAttribute(&cus0, hipDeviceAttributeMultiprocessorCount, dev0));
    // the token form: Pack5 forms when Pack5 tiles are most of the bytes
    double p5_bytes = 0.0, all_bytes = 0.0;
    for (int i = 0; i < nops; ++i)
        for (int p = 0; p < ops[i].n; ++p) {
            const double b = (double)((ops[i].w[p]->N + 15) / 16) * (double)ops[i].w[p]->nch;
            all_bytes += b;
            if (info[(size_t)i].fmt == XT_PACK5) p5_bytes += b;
        }
    const bool p5 = 2.0 * p5_bytes > all_bytes;
    // 16-row groups per task (the kernel loads and multiplies all of a
    // task's groups' tiles per step and shares the chunk's activation pieces
    // among them)
    const int rg = xt::sstack_groups_per_task((int)M, p5);
    // (M = 1: no quantiser tasks; each group task quantises the op's row)
    const bool qtasks = xt::sstack_quant_tasks((int)M);
    if (!qtasks) scratch = 0;
    ntasks = qtasks ? (size_t)nops * (size_t)M : 0;
    for (int i = 0; i < nops; ++i)
        for (int p = 0; p < ops[i].n; ++p) ntasks += (size_t)(((ops[i].w[p]->N + 15) / 16 + rg - 1) / rg);
    if (ntasks > (size_t)1 << 30) return fail(XT_ERR_UNSUPPORTED, "stack too large");
    const size_t tasks_b = align_up(ntasks * sizeof(xt::SStackTask), 256);
    const size_t ctr_b = (size_t)(4 + 2 * nops) * 128;
    char* mem = nullptr;
    const size_t woff_b = align_up(((size_t)cus0 * 64 + 1) * 4, 256);  // (at most 64 waves per CU)
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&mem), tasks_b + ctr_b + scratch + woff_b);
    if (e != hipSuccess) return fail(XT_ERR_NOMEM, std::string("stack allocation: ") + hipGetErrorString(e));
    char* sc = mem + tasks_b + ctr_b;

    std::vector<xt::SStackTask> tasks;
    tasks.reserve(ntasks);
    auto base = [&](int i) {
        const OpInfo& f = info[(size_t)i];
        xt::SStackTask t;
        memset(&t, 0, sizeof t);
        t.q = reinterpret_cast<int8_t*>(sc + f.qoff);
        t.opi = i;
        t.nch = f.nch;
        t.K = f.K;
        t.ldq = f.ldq;
        t.dep = ops[i].dep;
        t.dep_groups = ops[i].dep >= 0 ? info[(size_t)ops[i].dep].ngroups : 0;
        return t;
    };
    auto quant_task = [&](int i) {  // one per token
        const OpInfo& f = info[(size_t)i];
        for (int64_t m = 0; m < M && qtasks; ++m) {
            xt::SStackTask t = base(i);
            t.tiles = ops[i].x + m * f.K;
            t.q = reinterpret_cast<int8_t*>(sc + f.qoff + (size_t)m * f.ldq);
            t.ws = reinterpret_cast<const float*>(sc + f.qoff + (size_t)M * f.ldq + 4 * (size_t)m);
            t.flags = 1;
            tasks.push_back(t);
        }
    };
    for (int i = 0; i < nops; ++i)
        if (ops[i].dep < 0) quant_task(i);
    for (int i : stack_order(ops, nops, pub)) {
        const xt_stack_op& op = ops[i];
        for (int p = 0; p < op.n; ++p) {
            const xt_weights* w = op.w[p];
            const int64_t ng = (w->N + 15) / 16;
            for (int64_t G = 0; G < ng; G += rg) {
                const int n_g = (int)std::min<int64_t>(rg, ng - G);
                xt::SStackTask t = base(i);
                t.tiles = w->tiles + (size_t)G * w->nch * xt::kTileBytes;
                t.ws = w->ws + G * 16;
                t.y = op.y[p] + G * 16;
                if (qtasks) {
                    t.K = (int)w->N;  // (a group task's output row stride)
                } else {
                    t.q = reinterpret_cast<int8_t*>(const_cast<float*>(op.x));  // the f32 row it quantises
                    t.K = info[(size_t)i].K;                                   // (its length)
                }
                t.flags = (pub[(size_t)i] ? 2 : 0) | (info[(size_t)i].fmt == XT_PACK5 ? 4 : 0) | (n_g << 16);
                t.nrows = (int)std::min<int64_t>(16, w->N - (G + n_g - 1) * 16);
                tasks.push_back(t);
            }
        }
        for (int k = i + 1; k < nops; ++k)
            if (ops[k].dep == i) quant_task(k);
    }
    // Every wave resident at once (see xtern_sstack.hip): at most the
    // occupancy, and four workgroups per CU (16 waves) stream best.
    const int wpb = xt::sstack_waves_per_block();
    int per_cu = 0;
    int row_bytes = 1024;
    for (const OpInfo& f : info)
        row_bytes = std::max(row_bytes, xt::sstack_lds_rows((int)M) * (xt::chunk_cols(f.fmt) + 16));
    e = xt::sstack_blocks_per_cu((int)M, p5, row_bytes, &per_cu);
    if (e == hipSuccess && per_cu < 1) e = hipErrorInvalidConfiguration;
    const int grid = std::max(1, std::min(cus0 * std::min(per_cu, 4), ((int)tasks.size() + wpb - 1) / wpb));
    const int nw = grid * wpb;
    // deal the list out: each task, in list order, to the wave with the least
    // weight bytes so far (a task's start costs about 4 KiB of streaming)
    std::vector<std::vector<int>> per((size_t)nw);
    {
        typedef std::pair<double, int> Slot;
        std::vector<Slot> heap;
        for (int w = 0; w < nw; ++w) heap.push_back(Slot(0.0, w));
        auto later = [](const Slot& x, const Slot& y) { return x > y; };
        std::make_heap(heap.begin(), heap.end(), later);
        for (size_t t = 0; t < tasks.size(); ++t) {
            const xt::SStackTask& k = tasks[t];
            // (M > 1 group tasks also read each chunk's M activation rows)
            const double cost = 4096.0 + ((k.flags & 1) ? 8.0 * k.K
                                                         : k.nch * (1024.0 * (k.flags >> 16) + 320.0 * M));
            std::pop_heap(heap.begin(), heap.end(), later);
            per[(size_t)heap.back().second].push_back((int)t);
            heap.back().first += cost;
            std::push_heap(heap.begin(), heap.end(), later);
        }
    }
    std::vector<xt::SStackTask> dealt;
    dealt.reserve(tasks.size());
    std::vector<int> woff((size_t)nw + 1, 0);
    for (int w = 0; w < nw; ++w) {
        for (int t : per[(size_t)w]) dealt.push_back(tasks[(size_t)t]);
        woff[(size_t)w + 1] = (int)dealt.size();
    }
    if (e == hipSuccess) e = hipMemcpy(mem, dealt.data(), dealt.size() * sizeof(xt::SStackTask), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(mem + tasks_b + ctr_b + scratch, woff.data(), woff.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(mem + tasks_b, 0, ctr_b + scratch);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(mem);
        return hip_fail(e, "stack setup");
    }
    xt_stack* st = new (std::nothrow) xt_stack();
    if (!st) {
        (void)hipFree(mem);
        return fail(XT_ERR_NOMEM, "stack handle");
    }
    st->sargs.tasks = reinterpret_cast<const xt::SStackTask*>(mem);
    st->sargs.ctr = reinterpret_cast<unsigned*>(mem + tasks_b);
    st->sargs.ntasks = (int)tasks.size();
    st->sargs.nops = nops;
    st->sargs.mode = mode;
    st->sargs.spin_limit = 1 << 20;  // polls (about a microsecond each) before a wait gives up
    st->sargs.woff = reinterpret_cast<const int*>(mem + tasks_b + ctr_b + scratch);
    st->sargs.row_bytes = row_bytes;
    st->sargs.M = (int)M;
    st->sargs.pack5 = p5 ? 1 : 0;
    st->blocks = grid;
    st->device = dev0;
    st->dev_mem = mem;
    *out = st;
    return XT_OK;
}

}  // namespace

extern "C" {

int xt_stack_create(const xt_stack_op* ops, int nops, int64_t M, int mode, xt_stack** out) {
    if (!out) return fail(XT_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (!ops || nops < 1) return fail(XT_ERR_INVALID, "need at least one op");
    const int max_ops = xt::kSStackMaxOps;
    if (nops > max_ops)
        return fail(XT_ERR_UNSUPPORTED, "at most " + std::to_string(max_ops) +
                                            " ops per stack (split longer lists into several stacks)");
    if (M < 1 || M > 32) return fail(XT_ERR_UNSUPPORTED, "stack M must be 1..32");
    const int plan = mode & ~0xff;
    mode &= 0xff;
    if (plan != XT_STACK_AUTO && plan != XT_STACK_ONE_LAUNCH && plan != XT_STACK_PER_OP)
        return fail(XT_ERR_INVALID, "unknown stack plan flags");
    if (mode != XT_QUANT_AVX512 && mode != XT_QUANT_SCALAR)
        return fail(XT_ERR_INVALID, "unknown quantisation mode");
    for (int i = 0; i < nops; ++i) {
        const xt_stack_op& op = ops[i];
        const std::string at = "op " + std::to_string(i) + ": ";
        if (op.n < 1 || op.n > 4) return fail(XT_ERR_INVALID, at + "n must be 1..4");
        if (!op.x) return fail(XT_ERR_INVALID, at + "x is NULL");
        if (op.dep < -1 || op.dep >= i) return fail(XT_ERR_INVALID, at + "dep must be -1 or an earlier op");
        for (int p = 0; p < op.n; ++p)
            if (!op.w[p] || !op.y[p]) return fail(XT_ERR_INVALID, at + "NULL weights or output");
        if (op.dep >= 0) {
            int src = -1;
            for (int p = 0; p < ops[op.dep].n; ++p)
                if (ops[op.dep].y[p] == op.x) src = p;
            if (src < 0) return fail(XT_ERR_INVALID, at + "x must be one of the dep op's outputs");
            if (ops[op.dep].w[src]->N != op.w[0]->K)
                return fail(XT_ERR_INVALID, at + "x (an output of the dep op) differs in length from in_dim");
        }
    }
    if (plan == XT_STACK_PER_OP || (plan == XT_STACK_AUTO && stack_prefers_per_op(ops, nops, M)))
        return create_per_op(ops, nops, M, mode, out);
    const int rc = create_sstack(ops, nops, M, mode, out);
    // (a list the one-launch kernels do not take runs per op unless the
    // caller asked for one launch)
    if (rc == XT_ERR_UNSUPPORTED && plan == XT_STACK_AUTO) return create_per_op(ops, nops, M, mode, out);
    return rc;
}

int xt_stack_plan(const xt_stack* st) {
    if (!st) return fail(XT_ERR_INVALID, "stack is NULL");
    return st->per_op ? XT_STACK_PER_OP : XT_STACK_ONE_LAUNCH;
}

}  // extern "C"

extern "C" {

int xt_stack_run(const xt_stack* st, void* stream) {
    if (!st) return fail(XT_ERR_INVALID, "stack is NULL");
    if (st->per_op) {
        for (size_t i = 0; i < st->seq.size(); ++i) {
            const xt_stack_op& op = st->seq[i];
            if (int rc = linear_f32(op.w, op.n, op.x, st->M, op.y, st->qmode, static_cast<hipStream_t>(stream)))
                return fail(rc, "stack op " + std::to_string(i) + ": " + g_err);
        }
        return XT_OK;
    }
    hipError_t e = xt::launch_sstack(st->sargs, st->blocks, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "stack launch");
    return XT_OK;
}

int xt_stack_check(xt_stack* st, int* gave_up) {
    if (!st || !gave_up) return fail(XT_ERR_INVALID, "NULL argument");
    XT_HIP(hipDeviceSynchronize());
    if (st->per_op) {
        *gave_up = 0;
        return XT_OK;
    }
    unsigned flag = 0;
    unsigned* slot = st->sargs.ctr + 2 * 32;  // the error slot (xtern_sstack.hip kSsError)
    XT_HIP(hipMemcpy(&flag, slot, sizeof flag, hipMemcpyDeviceToHost));
    if (flag) XT_HIP(hipMemset(slot, 0, sizeof flag));
    *gave_up = flag ? 1 : 0;
    return XT_OK;
}

int xt_stack_destroy(xt_stack* st) {
    if (!st) return XT_OK;
    hipError_t e = hipDeviceSynchronize();
    hipError_t e2 = st->dev_mem ? hipFree(st->dev_mem) : hipSuccess;
    delete st;
    if (e != hipSuccess) return hip_fail(e, "stack destroy");
    if (e2 != hipSuccess) return hip_fail(e2, "stack destroy");
    return XT_OK;
}

int xt_int_quantize_host(int bits, const float* w, int64_t out_dim, int64_t in_dim, void* out,
                         float* scales) {
    if (bits != 8 && bits != 4) return fail(XT_ERR_INVALID, "bits must be 8 or 4");
    if (out_dim <= 0 || in_dim <= 0) return fail(XT_ERR_INVALID, "in_dim and out_dim must be positive");
    if (!w || !out || !scales) return fail(XT_ERR_INVALID, "NULL buffer");
    xt::int_quantize(bits, w, out_dim, in_dim, static_cast<uint8_t*>(out), scales);
    return XT_OK;
}

}  // extern "C"
