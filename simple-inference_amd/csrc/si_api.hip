// si_api.hip -- extern "C" entry points of include/si_abi.h.
//
// Argument checking, the layer object (device weights, RoPE tables,
// workspaces) and the three layer schedules: single-token decode
// (run_layer, qwen_one_layer.c:237-281), batched decode, and causal prefill
// (pf_run_batch, prefill_weight_stationary.h:183-311).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <cxxabi.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/si_abi.h"
#include "si_device.hpp"
#include "si_gemv.hpp"
#include "si_kernels.hpp"

using namespace si;

static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

static int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return SI_OK;
}

#define SI_REQUIRE(cond, ...) \
    do {                      \
        if (!(cond)) return fail(SI_ERR_ARG, __VA_ARGS__); \
    } while (0)

#define HIP_TRY(call)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) return fail(SI_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

static inline hipStream_t S(void *stream) { return (hipStream_t)stream; }

// Q4_0 nibble bytes of an n x k matrix: the mat-vec kernels address a
// weight array with 32-bit buffer offsets
static bool q4_fits(long long n, long long k) { return n * (k / 32) * 16 < (1ll << 32); }

static int check_shape(const si_shape_t *s) {
    SI_REQUIRE(s, "shape is NULL");
    SI_REQUIRE(s->hidden > 0 && s->hidden % 32 == 0, "hidden %d must be a positive multiple of 32",
               s->hidden);
    SI_REQUIRE(attn_supported(s->qheads, s->kvheads, s->hdim),
               "unsupported heads %d/%d x hdim %d (need qheads %% kvheads == 0, ratio <= 16, "
               "hdim 32, 64, 96 or 128)",
               s->qheads, s->kvheads, s->hdim);
    SI_REQUIRE(s->ffn >= 0 && s->ffn % 32 == 0, "ffn %d must be a multiple of 32", s->ffn);
    SI_REQUIRE(s->hidden <= 8192, "hidden %d exceeds 8192", s->hidden);
    {
        const long long h = s->hidden, qd = (long long)s->qheads * s->hdim,
                        kvd = (long long)s->kvheads * s->hdim, f = s->ffn;
        SI_REQUIRE(q4_fits(qd + 2 * kvd, h) && q4_fits(h, qd) && q4_fits(2 * f, h) &&
                       q4_fits(h, f),
                   "a weight matrix reaches 4 GiB of Q4_0 nibbles");
    }
    return SI_OK;
}

// Per-dispatch kernel timing: filter alternatives and a pool of event
// pairs, handed out in launch order while timing is on (launches under
// stream capture and past the pool's capacity are not timed), with the name
// of each timed launch's kernel (demangled, without the "si::" namespace or
// the parameter list, e.g. "k_dec_attn<64, 8, false, false, 1>").
namespace si {
std::atomic<bool> g_kernel_timing_on{false};
}
static std::mutex g_kt_mu;
static std::vector<std::string> g_kt_filter;
static std::vector<hipEvent_t> g_kt_events;  // 2 per launch
static std::vector<const char *> g_kt_names;
static std::map<const void *, std::string> g_kt_name_of;  // kernel -> name
static int g_kt_used = 0;

static const char *kernel_name(const void *kernel, hipStream_t st) {
    auto it = g_kt_name_of.find(kernel);
    if (it != g_kt_name_of.end()) return it->second.c_str();
    const char *raw = hipKernelNameRefByPtr(kernel, st);
    std::string name = raw ? raw : "?";
    if (name.compare(0, 2, "_Z") == 0) {
        int status = 0;
        char *dm = abi::__cxa_demangle(name.c_str(), nullptr, nullptr, &status);
        if (dm && status == 0) name = dm;
        free(dm);
    }
    // "void si::k_x<...>(args)" -> "k_x<...>"
    size_t b = name.find("si::");
    if (b != std::string::npos) name = name.substr(b + 4);
    int depth = 0;
    for (size_t i = 0; i < name.size(); ++i) {
        if (name[i] == '<') ++depth;
        if (name[i] == '>') --depth;
        if (name[i] == '(' && depth == 0) {
            name.resize(i);
            break;
        }
    }
    return g_kt_name_of.emplace(kernel, name).first->second.c_str();
}

bool si::kernel_timing_events(const void *kernel, hipStream_t st, hipEvent_t *start,
                              hipEvent_t *stop) {
    std::lock_guard<std::mutex> lock(g_kt_mu);
    if (!g_kernel_timing_on || 2 * (g_kt_used + 1) > (int)g_kt_events.size()) return false;
    const char *kernel_text = kernel_name(kernel, st);
    bool match = false;
    for (const std::string &f : g_kt_filter) match = match || strstr(kernel_text, f.c_str());
    if (!match) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return false;
    *start = g_kt_events[2 * g_kt_used];
    *stop = g_kt_events[2 * g_kt_used + 1];
    g_kt_names[g_kt_used] = kernel_text;
    ++g_kt_used;
    return true;
}

extern "C" {

const char *si_last_error(void) { return g_err.c_str(); }

int si_kernel_timing_start(const char *filter, int capacity) {
    SI_REQUIRE(filter && capacity > 0 && capacity <= (1 << 16),
               "kernel_timing_start: filter and 1..65536 launches required");
    std::lock_guard<std::mutex> lock(g_kt_mu);
    SI_REQUIRE(!g_kernel_timing_on, "kernel timing is already on");
    for (hipEvent_t e : g_kt_events) (void)hipEventDestroy(e);
    g_kt_events.clear();
    for (int i = 0; i < 2 * capacity; ++i) {
        hipEvent_t e;
        HIP_TRY(hipEventCreate(&e));
        g_kt_events.push_back(e);
    }
    g_kt_names.assign(capacity, nullptr);
    g_kt_filter.clear();
    for (const char *p = filter;; ++p) {  // '|'-separated alternatives
        const char *e = strchr(p, '|');
        g_kt_filter.emplace_back(p, e ? (size_t)(e - p) : strlen(p));
        if (!e) break;
        p = e;
    }
    g_kt_used = 0;
    g_kernel_timing_on.store(true);
    return SI_OK;
}

int si_kernel_timing_stop(float *ms, int capacity, int *count) {
    std::lock_guard<std::mutex> lock(g_kt_mu);
    SI_REQUIRE(g_kernel_timing_on, "kernel timing is not on");
    g_kernel_timing_on.store(false);
    const int n = g_kt_used < capacity ? g_kt_used : capacity;
    if (count) *count = n;
    for (int i = 0; i < n; ++i) {
        HIP_TRY(hipEventSynchronize(g_kt_events[2 * i + 1]));
        HIP_TRY(hipEventElapsedTime(&ms[i], g_kt_events[2 * i], g_kt_events[2 * i + 1]));
    }
    return SI_OK;
}

const char *si_kernel_timing_name(int i) {
    std::lock_guard<std::mutex> lock(g_kt_mu);
    if (g_kernel_timing_on || i < 0 || i >= g_kt_used) return nullptr;
    return g_kt_names[i];
}

static bool tile_ok(int tile) { return tile == 8 || tile == 16 || tile == 32 || tile == 64; }

int si_q4_tile(int n, int k) {
    (void)k;
    return n > 0 ? gemv_tile_for(n) : 8;
}

size_t si_q4_scale_count(int n, int k, int tile) {
    if (n <= 0 || k <= 0 || k % 32 || !tile_ok(tile)) return 0;
    return q4_scale_count(n, k / 32, tile);
}

int si_q4_repack(const uint8_t *src, int n, int k, int tile, uint8_t *qs, uint16_t *d,
                 void *stream) {
    SI_REQUIRE(n > 0 && k > 0 && k % 32 == 0, "repack: bad size n=%d k=%d", n, k);
    SI_REQUIRE(tile_ok(tile), "repack: tile %d not 8, 16, 32 or 64", tile);
    SI_REQUIRE(src && qs && d, "repack: NULL pointer");
    launch_q4_repack(src, n, k, tile, qs, d, S(stream));
    return check_launch("si_q4_repack");
}

int si_q4_unpack(const uint8_t *qs, const uint16_t *d, int n, int k, int tile, uint8_t *dst,
                 void *stream) {
    SI_REQUIRE(n > 0 && k > 0 && k % 32 == 0, "unpack: bad size n=%d k=%d", n, k);
    SI_REQUIRE(tile_ok(tile), "unpack: tile %d not 8, 16, 32 or 64", tile);
    SI_REQUIRE(dst && qs && d, "unpack: NULL pointer");
    launch_q4_unpack(qs, d, n, k, tile, dst, S(stream));
    return check_launch("si_q4_unpack");
}

int si_quantize_q8(const float *src, void *dst, int count, void *stream) {
    // qwen_one_layer.c:99: the reference dies unless count % 32 == 0
    SI_REQUIRE(count >= 0 && count % 32 == 0, "Q8 quantization length must be multiple of 32");
    SI_REQUIRE(count == 0 || (src && dst), "quantize_q8: NULL pointer");
    launch_quantize_q8_aos(src, dst, count, S(stream));
    return check_launch("si_quantize_q8");
}

int si_quantize_q8_rows(const float *src, int rows, int k, int8_t *qs, uint16_t *d, int16_t *s,
                        void *stream) {
    SI_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "Q8 quantization length must be multiple of 32");
    SI_REQUIRE(rows == 0 || (src && qs && d), "quantize_q8_rows: NULL pointer");
    launch_quantize_q8_rows(src, rows, k, qs, d, s, S(stream));
    return check_launch("si_quantize_q8_rows");
}

int si_rmsnorm_q8(const float *x, const float *gain, int rows, int n, float eps, float *normed,
                  int8_t *qs, uint16_t *d, int16_t *s, void *stream) {
    SI_REQUIRE(rows >= 0 && n > 0 && n % 32 == 0 && n <= 8192, "rmsnorm: bad size n=%d", n);
    SI_REQUIRE(rows == 0 || (x && qs && d), "rmsnorm: NULL pointer");
    launch_rmsnorm_q8(x, nullptr, gain, rows, n, eps, nullptr, normed, qs, d, s, S(stream));
    return check_launch("si_rmsnorm_q8");
}

int si_residual_rmsnorm_q8(const float *x, const float *y, const float *gain, int rows, int n,
                           float eps, float *h, float *normed, int8_t *qs, uint16_t *d,
                           int16_t *s, void *stream) {
    SI_REQUIRE(rows >= 0 && n > 0 && n % 32 == 0 && n <= 8192, "rmsnorm: bad size n=%d", n);
    SI_REQUIRE(rows == 0 || (x && y && h && qs && d), "residual_rmsnorm: NULL pointer");
    launch_rmsnorm_q8(x, y, gain, rows, n, eps, h, normed, qs, d, s, S(stream));
    return check_launch("si_residual_rmsnorm_q8");
}

int si_q4q8_block_dots(const uint8_t *wqs, const uint16_t *wd, int n, int k, const int8_t *xqs,
                       const int16_t *xs, int32_t *dots, void *stream) {
    (void)wd;
    SI_REQUIRE(n > 0 && k > 0 && k % 32 == 0, "block_dots: bad size");
    SI_REQUIRE(wqs && xqs && xs && dots, "block_dots: NULL pointer");
    launch_block_dots(wqs, n, k, xqs, xs, dots, S(stream));
    return check_launch("si_q4q8_block_dots");
}

int si_matvec_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                   const int8_t *xqs, const uint16_t *xd, const int16_t *xs, const float *bias,
                   const float *residual, float *out, int flags, void *stream) {
    SI_REQUIRE(n > 0 && k > 0 && k % 32 == 0, "matvec: bad size n=%d k=%d", n, k);
    SI_REQUIRE(tile_ok(tile), "matvec: tile %d not 8, 16, 32 or 64", tile);
    SI_REQUIRE(q4_fits(n, k), "matvec: %d x %d reaches 4 GiB of Q4_0 nibbles", n, k);
    SI_REQUIRE(wqs && wd && xqs && xd && xs && out, "matvec: NULL pointer");
    SI_REQUIRE(((uintptr_t)wqs & 15) == 0 && ((uintptr_t)xqs & 15) == 0,
               "matvec: wqs and xqs must be 16-byte aligned");
    SI_REQUIRE((flags & ~SI_GEMM_EXACT) == 0, "matvec: unknown flags %d", flags);
    launch_matvec(xqs, xd, xs, k, wqs, wd, tile, n, bias, residual, out,
                  (flags & SI_GEMM_EXACT) != 0, S(stream));
    return check_launch("si_matvec_q4q8");
}

int si_ffn_gateup_q8(const float *h, const float *gain, int hidden, float eps,
                     const uint8_t *wqs, const uint16_t *wd, int tile, int f, float *act,
                     int8_t *qs, uint16_t *d, int16_t *bsum, int flags, void *stream) {
    SI_REQUIRE(hidden > 0 && hidden % 32 == 0 && hidden <= 8192, "ffn_gateup: bad hidden %d",
               hidden);
    SI_REQUIRE(f > 0 && f % 32 == 0, "ffn_gateup: ffn %d must be a multiple of 32", f);
    SI_REQUIRE(q4_fits(2ll * f, hidden), "ffn_gateup: gate|up reaches 4 GiB of Q4_0 nibbles");
    SI_REQUIRE(tile == 32, "ffn_gateup: the gate|up weights need scale tile 32 (got %d)", tile);
    SI_REQUIRE(h && wqs && wd && qs && d && bsum, "ffn_gateup: NULL pointer");
    SI_REQUIRE(((uintptr_t)wqs & 15) == 0 && ((uintptr_t)h & 15) == 0 &&
                   (!gain || ((uintptr_t)gain & 15) == 0),
               "ffn_gateup: wqs, h and gain must be 16-byte aligned");
    SI_REQUIRE((flags & ~SI_GEMM_EXACT) == 0, "ffn_gateup: unknown flags %d", flags);
    launch_dec_gateup(h, gain, hidden, eps, wqs, wd, tile, f, nullptr, nullptr, nullptr, nullptr,
                      nullptr, act, qs, d, bsum, (flags & SI_GEMM_EXACT) != 0, S(stream));
    return check_launch("si_ffn_gateup_q8");
}

// SI_GEMM_F6 workspace: the fp6 weights w6 and scales d6, the activations
// x6, then the K-split partials (none for the fused gate|up pass), each part
// 256-byte aligned.
struct F6Ws {
    size_t w6 = 0, d6 = 0, x6 = 0, part = 0, total = 0;
};
static F6Ws f6_ws(int m, int n, int k, bool partials) {
    const size_t nb = (size_t)k / 32;
    const auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    F6Ws o;
    o.d6 = up((size_t)n * nb * 24);
    o.x6 = o.d6 + up((size_t)n * nb * 2);
    o.part = o.x6 + up((size_t)m * nb * 48);
    o.total = o.part + (partials ? up(gemm_f6_partial_bytes(m, n, k)) : 0);
    return o;
}

int si_gemm_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                 const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                 const float *residual, float *out, int ldo, int flags, void *workspace,
                 size_t ws_bytes, void *stream) {
    SI_REQUIRE(n > 0 && k > 0 && k % 32 == 0 && m >= 0, "gemm: bad size m=%d n=%d k=%d", m, n,
               k);
    SI_REQUIRE(tile_ok(tile), "gemm: tile %d not 8, 16, 32 or 64", tile);
    SI_REQUIRE(ldo >= n, "gemm: ldo %d < n %d", ldo, n);
    // the kernels address each operand with 32-bit byte offsets
    SI_REQUIRE((size_t)m * k < ((size_t)1 << 31) && (size_t)n * k / 2 < ((size_t)1 << 31) &&
                   q4_scale_count(n, k / 32, tile) * 2 < ((size_t)1 << 31),
               "gemm: operands beyond 2 GiB (m=%d n=%d k=%d)", m, n, k);
    SI_REQUIRE(m == 0 || (wqs && wd && xqs && xd && out), "gemm: NULL pointer");
    SI_REQUIRE(((uintptr_t)wqs & 15) == 0 && ((uintptr_t)xqs & 15) == 0,
               "gemm: wqs and xqs must be 16-byte aligned");
    SI_REQUIRE((flags & ~(SI_GEMM_EXACT | SI_GEMM_TILED_A | SI_GEMM_F6)) == 0,
               "gemm: unknown flags %d", flags);
    if (flags & SI_GEMM_F6) {
        SI_REQUIRE(flags == SI_GEMM_F6, "gemm: SI_GEMM_F6 takes no other flag");
        SI_REQUIRE((size_t)m * k / 32 * 48 < ((size_t)1 << 31) &&
                       (size_t)n * k / 32 * 24 < ((size_t)1 << 31),
                   "gemm: SI_GEMM_F6 operands beyond 2 GiB (m=%d n=%d k=%d)", m, n, k);
        if (m == 0) return SI_OK;
        const F6Ws L = f6_ws(m, n, k, true);
        SI_REQUIRE(workspace && ws_bytes >= L.total && ((uintptr_t)workspace & 255) == 0,
                   "gemm: SI_GEMM_F6 needs si_gemm_f6_workspace(m, n, k) = %zu bytes of "
                   "256-byte aligned workspace", L.total);
        uint8_t *ws = (uint8_t *)workspace;
        const hipStream_t st = S(stream);
        launch_q4_to_w6(wqs, wd, n, k / 32, tile, 0, ws + L.w6, (uint16_t *)(ws + L.d6), st);
        launch_q8_to_x6(xqs, m, k / 32, ws + L.x6, st);
        launch_gemm_f6(ws + L.w6, (const uint16_t *)(ws + L.d6), n, k, ws + L.x6, xd, m, bias,
                       residual, out, ldo, ws + L.part, L.total - L.part, false, 0, nullptr,
                       nullptr, nullptr, nullptr, st);
        return check_launch("si_gemm_q4q8");
    }
    if (flags & SI_GEMM_TILED_A) {
        SI_REQUIRE(!(flags & SI_GEMM_EXACT), "gemm: SI_GEMM_TILED_A has no exact mode");
        SI_REQUIRE(m <= 512, "gemm: SI_GEMM_TILED_A takes at most 512 rows (m=%d)", m);
        launch_gemm_q4q8_tiled(wqs, wd, tile, n, k, xqs, xd, m, bias, residual, out, ldo,
                               S(stream));
        return check_launch("si_gemm_q4q8");
    }
    launch_gemm_q4q8(wqs, wd, tile, n, k, xqs, xd, m, bias, residual, out, ldo,
                     (flags & SI_GEMM_EXACT) != 0, workspace, workspace ? ws_bytes : 0,
                     S(stream));
    return check_launch("si_gemm_q4q8");
}

int si_q8_tile(const int8_t *qs, const uint16_t *d, int m, int k, int8_t *tq, uint16_t *td,
               void *stream) {
    SI_REQUIRE(m >= 0 && k > 0 && k % 32 == 0, "q8_tile: bad size m=%d k=%d", m, k);
    SI_REQUIRE((size_t)(m + 31) / 32 * 32 * k < ((size_t)1 << 31),
               "q8_tile: operands beyond 2 GiB (m=%d k=%d)", m, k);
    SI_REQUIRE(m == 0 || (qs && d && tq && td), "q8_tile: NULL pointer");
    SI_REQUIRE(((uintptr_t)qs & 15) == 0 && ((uintptr_t)tq & 15) == 0,
               "q8_tile: qs and tq must be 16-byte aligned");
    launch_q8_tile(qs, d, m, k, tq, td, S(stream));
    return check_launch("si_q8_tile");
}

int si_gemm_gateup_q8(const uint8_t *wqs, const uint16_t *wd, int tile, int f, int k,
                      const int8_t *xqs, const uint16_t *xd, int m, float *gu, float *act,
                      int8_t *qs, uint16_t *d, int16_t *bsum, int flags, void *workspace,
                      size_t ws_bytes, void *stream) {
    SI_REQUIRE(f > 0 && f % 32 == 0 && k > 0 && k % 32 == 0 && m >= 0,
               "gemm_gateup: bad size m=%d f=%d k=%d", m, f, k);
    SI_REQUIRE(tile_ok(tile), "gemm_gateup: tile %d not 8, 16, 32 or 64", tile);
    SI_REQUIRE((size_t)m * k < ((size_t)1 << 31) && (size_t)f * k < ((size_t)1 << 31) &&
                   q4_scale_count(2 * f, k / 32, tile) * 2 < ((size_t)1 << 31),
               "gemm_gateup: operands beyond 2 GiB (m=%d f=%d k=%d)", m, f, k);
    SI_REQUIRE(m == 0 || (wqs && wd && xqs && xd && qs && d), "gemm_gateup: NULL pointer");
    {
        const size_t need = gemm_gateup_workspace_bytes(m, f, k);
        const bool gu_needed = (flags & SI_GEMM_EXACT) || (need > 0 && (!workspace || ws_bytes < need));
        SI_REQUIRE(m == 0 || gu || !gu_needed,
                   "gemm_gateup: gu is the intermediate here (exact mode, or a K split "
                   "without its workspace)");
    }
    SI_REQUIRE(((uintptr_t)wqs & 15) == 0 && ((uintptr_t)xqs & 15) == 0 &&
                   ((uintptr_t)qs & 15) == 0 && ((uintptr_t)act & 15) == 0,
               "gemm_gateup: wqs, xqs, qs and act must be 16-byte aligned");
    SI_REQUIRE((flags & ~(SI_GEMM_EXACT | SI_GEMM_F16 | SI_GEMM_TILED_A | SI_GEMM_F6)) == 0,
               "gemm_gateup: unknown flags %d", flags);
    if (flags & SI_GEMM_F6) {
        SI_REQUIRE(flags == SI_GEMM_F6, "gemm_gateup: SI_GEMM_F6 takes no other flag");
        SI_REQUIRE((size_t)m * k / 32 * 48 < ((size_t)1 << 31) &&
                       (size_t)2 * f * k / 32 * 24 < ((size_t)1 << 31),
                   "gemm_gateup: SI_GEMM_F6 operands beyond 2 GiB (m=%d f=%d k=%d)", m, f, k);
        if (m == 0) return SI_OK;
        SI_REQUIRE(gemm_f6_partial_bytes(m, 2 * f, k) == 0,
                   "gemm_gateup: SI_GEMM_F6 runs the fused one-pass plan only; this shape "
                   "splits K (m=%d f=%d k=%d)", m, f, k);
        const F6Ws L = f6_ws(m, 2 * f, k, false);
        SI_REQUIRE(workspace && ws_bytes >= L.total && ((uintptr_t)workspace & 255) == 0,
                   "gemm_gateup: SI_GEMM_F6 needs si_gemm_f6_workspace(m, 2f, k) = %zu bytes "
                   "of 256-byte aligned workspace", L.total);
        uint8_t *ws = (uint8_t *)workspace;
        const hipStream_t st = S(stream);
        launch_q4_to_w6(wqs, wd, 2 * f, k / 32, tile, f, ws + L.w6, (uint16_t *)(ws + L.d6), st);
        launch_q8_to_x6(xqs, m, k / 32, ws + L.x6, st);
        launch_gemm_f6(ws + L.w6, (const uint16_t *)(ws + L.d6), 2 * f, k, ws + L.x6, xd, m,
                       nullptr, nullptr, gu, 2 * f, nullptr, 0, false, f, act, qs, d, bsum, st);
        return check_launch("si_gemm_gateup_q8");
    }
    SI_REQUIRE(!(flags & SI_GEMM_F16) || !(flags & SI_GEMM_EXACT),
               "gemm_gateup: SI_GEMM_F16 is a fast-path formulation (not with SI_GEMM_EXACT)");
    if (flags & SI_GEMM_TILED_A) {
        SI_REQUIRE(flags == SI_GEMM_TILED_A, "gemm_gateup: SI_GEMM_TILED_A takes no other flag");
        SI_REQUIRE(m == 0 || gemm_gateup_streams(m, f, k),
                   "gemm_gateup: SI_GEMM_TILED_A needs m <= 64 and k <= 3840 (m=%d f=%d k=%d)",
                   m, f, k);
        launch_gemm_gateup_q8(wqs, wd, tile, f, k, xqs, xd, m, gu, act, qs, d, bsum, false,
                              nullptr, 0, S(stream), false, nullptr, nullptr, xqs, xd);
        return check_launch("si_gemm_gateup_q8");
    }
    launch_gemm_gateup_q8(wqs, wd, tile, f, k, xqs, xd, m, gu, act, qs, d, bsum,
                          (flags & SI_GEMM_EXACT) != 0, workspace, workspace ? ws_bytes : 0,
                          S(stream), (flags & SI_GEMM_F16) != 0);
    return check_launch("si_gemm_gateup_q8");
}

size_t si_gemm_workspace(int m, int n, int k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 32) return 0;
    return gemm_workspace_bytes(m, n, k);
}

size_t si_gemm_f6_workspace(int m, int n, int k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 32) return 0;
    return f6_ws(m, n, k, true).total;
}

int si_rope_table(int npos, int hdim, float base, float *c, float *s) {
    SI_REQUIRE(npos > 0 && hdim > 0 && hdim % 2 == 0 && c && s, "rope_table: bad args");
    const int half = hdim / 2;
    for (int p = 0; p < npos; ++p)
        for (int i = 0; i < half; ++i) {
            // qwen_one_layer.c:176-177: float theta, libm powf/cosf/sinf
            const float theta = (float)p / powf(base, (float)(2 * i) / (float)hdim);
            c[(size_t)p * half + i] = cosf(theta);
            s[(size_t)p * half + i] = sinf(theta);
        }
    return SI_OK;
}

int si_rope_kv_append(const si_shape_t *s, const float *qkv, int ldqkv, int ntok, int pos0,
                      int pos_step, int max_pos, const int *ctx_dev, const float *rc,
                      const float *rs, float *q_out, uint16_t *kc, uint16_t *vc,
                      size_t kv_seq_stride, void *stream) {
    int rc_ = check_shape(s);
    if (rc_) return rc_;
    SI_REQUIRE(ntok >= 0 && pos0 >= 0 && pos_step >= 0, "rope: bad ntok/pos0/pos_step");
    SI_REQUIRE(max_pos >= 1, "rope: max_pos must be >= 1");
    SI_REQUIRE(ctx_dev || ntok == 0 || (long)pos0 + (long)(ntok - 1) * pos_step < max_pos,
               "rope: positions exceed max_pos");
    SI_REQUIRE(ldqkv >= (s->qheads + 2 * s->kvheads) * s->hdim, "rope: ldqkv too small");
    SI_REQUIRE(kv_seq_stride % 8 == 0, "rope: kv_seq_stride must be a multiple of 8");
    SI_REQUIRE(ntok == 0 || (qkv && rc && rs && q_out && kc && vc), "rope: NULL pointer");
    launch_rope_kv(qkv, ldqkv, ntok, s->qheads, s->kvheads, s->hdim, pos0, pos_step, max_pos,
                   ctx_dev, rc, rs, q_out, kc, vc, kv_seq_stride, S(stream));
    return check_launch("si_rope_kv_append");
}

size_t si_attention_workspace(const si_shape_t *s, int nq, int max_ctx) {
    if (!s || nq <= 0 || max_ctx <= 0) return 0;
    // either schedule: context splits, or the causal prefill's split tiles
    const size_t a = attn_workspace_bytes(s->qheads, s->hdim, s->kvheads, nq, max_ctx);
    const size_t p = attn_prefill_workspace_bytes(s->qheads, s->hdim, nq);
    return a > p ? a : p;
}

}  // extern "C"

// Shared body of si_attention and si_attention_static: argument checks, then
// the causal-prefill flash kernel or the split-context decode kernels with
// their partial states in ws (ws_bytes of it).
static int attention_impl(const char *what, const si_shape_t *s, const float *q, int nq,
                          const uint16_t *kc, const uint16_t *vc, size_t kv_seq_stride,
                          const int *ctx_dev, int ctx0, int ctx_step, int max_ctx, float *attn,
                          int8_t *qs, uint16_t *d, int16_t *bsum, void *ws, size_t ws_bytes,
                          void *stream) {
    int r = check_shape(s);
    if (r) return r;
    SI_REQUIRE(nq >= 0 && max_ctx >= 1, "%s: bad nq/max_ctx", what);
    SI_REQUIRE(kv_seq_stride % 8 == 0, "%s: kv_seq_stride must be a multiple of 8", what);
    if (!ctx_dev) {
        // attention_kernels.h:95 handles context <= 0 by zeroing; a layer call
        // always has context >= 1 (qwen_one_layer.c:608), required here.
        SI_REQUIRE(ctx0 >= 1 && ctx_step >= 0, "%s: contexts must be >= 1", what);
        SI_REQUIRE((long)ctx0 + (long)(nq - 1) * ctx_step <= max_ctx,
                   "%s: context exceeds max_ctx", what);
    }
    SI_REQUIRE(nq == 0 || (q && kc && vc && attn && ws), "%s: NULL pointer", what);
    SI_REQUIRE(!qs || d, "%s: qs without d", what);
    SI_REQUIRE(ws_bytes >= si_attention_workspace(s, nq, max_ctx), "%s: workspace too small",
               what);
    if (!ctx_dev && ctx_step == 1 && kv_seq_stride == 0 && nq > 1 &&
        attn_prefill_supported(s->qheads, s->kvheads, s->hdim))
        // causal prefill of one sequence: the flash kernel (query i at
        // cache row ctx0 - 1 + i)
        launch_attn_prefill(q, nq, s->qheads, s->kvheads, s->hdim, ctx0 - 1, kc, vc, attn, qs, d,
                            bsum, ws, ws_bytes, S(stream));
    else
        launch_attention(q, nq, s->qheads, s->kvheads, s->hdim, kc, vc, kv_seq_stride, ctx_dev,
                         ctx0, ctx_step, max_ctx, attn, qs, d, bsum, ws, S(stream));
    return check_launch(what);
}

// The attention partial states of si_attention_static: one fixed buffer per
// GPU, in the code object's device memory, so the call allocates nothing.
// Its host-side name is only a stand-in: kernels and copies use the device
// address hipGetSymbolAddress returns, taken once per device (each GPU
// holds its own copy of the array at its own address).
static __device__ __align__(256) uint8_t scratch[SI_ATTENTION_STATIC_MAX];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_dev[kMaxDevices];

static int static_scratch(void **out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    SI_REQUIRE(dev >= 0 && dev < kMaxDevices, "attention_static: device %d beyond %d", dev,
               kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(SI_ERR_HIP, "attention_static: hipGetSymbolAddress: %s",
                        hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return SI_OK;
}

extern "C" {

int si_attention(const si_shape_t *s, const float *q, int nq, const uint16_t *kc,
                 const uint16_t *vc, size_t kv_seq_stride, const int *ctx_dev, int ctx0,
                 int ctx_step, int max_ctx, float *attn, int8_t *qs, uint16_t *d,
                 int16_t *bsum, void *ws, size_t ws_bytes, void *stream) {
    return attention_impl("si_attention", s, q, nq, kc, vc, kv_seq_stride, ctx_dev, ctx0,
                          ctx_step, max_ctx, attn, qs, d, bsum, ws, ws_bytes, stream);
}

int si_attention_static(const si_shape_t *s, const float *q, int nq, const uint16_t *kc,
                        const uint16_t *vc, size_t kv_seq_stride, const int *ctx_dev, int ctx0,
                        int ctx_step, int max_ctx, float *attn, int8_t *qs, uint16_t *d,
                        int16_t *bsum, void *stream) {
    int r = check_shape(s);
    if (r) return r;
    SI_REQUIRE(nq >= 0 && max_ctx >= 1, "si_attention_static: bad nq/max_ctx");
    const size_t need = si_attention_workspace(s, nq, max_ctx);
    SI_REQUIRE(need <= (size_t)SI_ATTENTION_STATIC_MAX,
               "si_attention_static: %d queries over max_ctx %d need %zu bytes of partial "
               "states, beyond the static buffer's %zu (use si_attention with a workspace)",
               nq, max_ctx, need, (size_t)SI_ATTENTION_STATIC_MAX);
    void *ws = nullptr;
    if (nq > 0) {
        r = static_scratch(&ws);
        if (r) return r;
    }
    return attention_impl("si_attention_static", s, q, nq, kc, vc, kv_seq_stride, ctx_dev,
                          ctx0, ctx_step, max_ctx, attn, qs, d, bsum, ws,
                          (size_t)SI_ATTENTION_STATIC_MAX, stream);
}

int si_stream_read(const void *buf, size_t bytes, uint32_t *sink, int workgroups, int depth,
                   void *stream) {
    SI_REQUIRE(buf && sink, "stream_read: NULL pointer");
    SI_REQUIRE(bytes > 0 && bytes % 16 == 0 && (uintptr_t)buf % 16 == 0,
               "stream_read: %zu bytes: a positive multiple of 16 at a 16-byte aligned address",
               bytes);
    SI_REQUIRE(workgroups >= 1 && workgroups <= 65536, "stream_read: %d workgroups",
               workgroups);
    SI_REQUIRE(depth == 4 || depth == 8 || depth == 16, "stream_read: depth %d", depth);
    launch_stream_read(buf, bytes, sink, workgroups, depth, S(stream));
    return check_launch("si_stream_read");
}

int si_f32_to_f16(const float *src, uint16_t *dst, size_t n, void *stream) {
    SI_REQUIRE(n == 0 || (src && dst), "f32_to_f16: NULL pointer");
    SI_REQUIRE(n < ((size_t)1 << 40), "f32_to_f16: %zu values", n);
    launch_f16_convert(src, dst, n, true, S(stream));
    return check_launch("si_f32_to_f16");
}

int si_f16_to_f32(const uint16_t *src, float *dst, size_t n, void *stream) {
    SI_REQUIRE(n == 0 || (src && dst), "f16_to_f32: NULL pointer");
    SI_REQUIRE(n < ((size_t)1 << 40), "f16_to_f32: %zu values", n);
    launch_f16_convert(src, dst, n, false, S(stream));
    return check_launch("si_f16_to_f32");
}

int si_matvec_q4q8_rowmajor(const uint8_t *w, const void *x, int inputs, int outputs,
                            const float *bias, float *out, void *stream) {
    // qwen_one_layer.c:150 takes inputs / QK blocks
    SI_REQUIRE(inputs > 0 && inputs % 32 == 0 && outputs >= 0,
               "matvec_q4q8: inputs %d must be a positive multiple of 32", inputs);
    SI_REQUIRE((long long)outputs * (inputs / 32) * 18 < (1ll << 40),
               "matvec_q4q8: %d x %d too large", outputs, inputs);
    SI_REQUIRE(outputs == 0 || (w && x && out), "matvec_q4q8: NULL pointer");
    SI_REQUIRE(((uintptr_t)w & 1) == 0 && ((uintptr_t)x & 1) == 0,
               "matvec_q4q8: weights and blocks must be 2-byte aligned");
    launch_matvec_rowmajor(w, x, inputs, outputs, bias, out, S(stream));
    return check_launch("si_matvec_q4q8_rowmajor");
}

int si_colsoa_matvec(const uint8_t *tiles, int ntiles, const void *x, int nblocks,
                     const float *bias_lo, const float *bias_hi, float *out, int add,
                     void *stream) {
    SI_REQUIRE(ntiles >= 0 && nblocks > 0, "colsoa_matvec: bad ntiles %d / nblocks %d", ntiles,
               nblocks);
    SI_REQUIRE(ntiles == 0 || (tiles && x && out), "colsoa_matvec: NULL pointer");
    SI_REQUIRE(((uintptr_t)tiles & 3) == 0 && ((uintptr_t)x & 1) == 0,
               "colsoa_matvec: tiles must be 4-byte and blocks 2-byte aligned");
    launch_colsoa_matvec(tiles, ntiles, x, nblocks, add ? nullptr : bias_lo,
                         add ? nullptr : bias_hi, out, add != 0, S(stream));
    return check_launch("si_colsoa_matvec");
}

int si_rmsnorm(const float *x, const float *gain, int rows, int n, float eps, float *out,
               void *stream) {
    SI_REQUIRE(rows >= 0 && n > 0, "rmsnorm: bad size rows=%d n=%d", rows, n);
    SI_REQUIRE(rows == 0 || (x && out), "rmsnorm: NULL pointer");
    launch_rmsnorm(x, gain, rows, n, eps, out, S(stream));
    return check_launch("si_rmsnorm");
}

int si_rope(const si_shape_t *s, float *heads, int nheads, int position, const float *rc,
            const float *rs, int max_pos, void *stream) {
    SI_REQUIRE(s && s->hdim > 0 && s->hdim % 2 == 0, "rope: bad shape");
    SI_REQUIRE(nheads >= 0 && position >= 0 && position < max_pos,
               "rope: position %d outside the table's 0..%d", position, max_pos - 1);
    SI_REQUIRE(nheads == 0 || (heads && rc && rs), "rope: NULL pointer");
    launch_rope_inplace(heads, nheads, s->hdim, position, rc, rs, S(stream));
    return check_launch("si_rope");
}

size_t si_attention_group_workspace(const si_shape_t *s, int nheads, int context) {
    if (!s || nheads <= 0 || context <= 0) return 0;
    return attn_workspace_bytes(nheads, s->hdim, 1, 1, context);
}

int si_attention_group(const si_shape_t *s, const float *q, int nheads, int group,
                       const uint16_t *kc, const uint16_t *vc, int context, float *out,
                       void *ws, size_t ws_bytes, void *stream) {
    int r = check_shape(s);
    if (r) return r;
    SI_REQUIRE(nheads >= 1 && nheads <= s->qheads / s->kvheads,
               "attention_group: %d heads, a KV group serves %d", nheads,
               s->qheads / s->kvheads);
    SI_REQUIRE(group >= 0 && group < s->kvheads, "attention_group: group %d outside 0..%d",
               group, s->kvheads - 1);
    SI_REQUIRE(context >= 1, "attention_group: context must be >= 1");
    SI_REQUIRE(q && kc && vc && out && ws, "attention_group: NULL pointer");
    SI_REQUIRE(((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0,
               "attention_group: kc and vc must be 16-byte aligned");
    SI_REQUIRE(ws_bytes >= si_attention_group_workspace(s, nheads, context),
               "attention_group: workspace too small");
    // the group's heads as a one-group shape over the wider cache rows
    const int kvd = s->kvheads * s->hdim;
    launch_attention(q, 1, nheads, 1, s->hdim, kc + (size_t)group * s->hdim,
                     vc + (size_t)group * s->hdim, 0, nullptr, context, 0, context, out, nullptr,
                     nullptr, nullptr, ws, S(stream), KvPages(), kvd);
    return check_launch("si_attention_group");
}

int si_attention_standard(const si_shape_t *s, const float *q, const uint16_t *kc,
                          const uint16_t *vc, int context, float *out, float *scores,
                          void *stream) {
    int r = check_shape(s);
    if (r) return r;
    SI_REQUIRE(context >= 0, "attention_standard: negative context");
    SI_REQUIRE(attn_standard_supported(s->qheads, s->kvheads, s->hdim),
               "attention_standard: unsupported head dimension %d", s->hdim);
    SI_REQUIRE(out && (context == 0 || (q && kc && vc && scores)),
               "attention_standard: NULL pointer");
    SI_REQUIRE(context == 0 || ((uintptr_t)kc % 16 == 0 && (uintptr_t)vc % 16 == 0),
               "attention_standard: kc and vc must be 16-byte aligned");
    launch_attn_standard(q, s->qheads, s->kvheads, s->hdim, kc, vc, context, out, scores,
                         S(stream));
    return check_launch("si_attention_standard");
}

int si_swiglu_q8(const float *gu, int rows, int f, float *act, int8_t *qs, uint16_t *d,
                 int16_t *s, void *stream) {
    SI_REQUIRE(rows >= 0 && f > 0 && f % 32 == 0, "swiglu: bad size");
    SI_REQUIRE(rows == 0 || (gu && qs && d), "swiglu: NULL pointer");
    launch_swiglu_q8(gu, rows, f, act, qs, d, s, S(stream));
    return check_launch("si_swiglu_q8");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Layer object
// ---------------------------------------------------------------------------
struct Q4Dev {
    uint8_t *qs = nullptr;
    uint16_t *d = nullptr;
    int n = 0, k = 0, tile = 8;
};

// A Q4 matrix for the fp6 GEMM formulation (prefill of more than 512 rows):
// w [nb][n][24] fp6 codes of (nibble - 8) / 2, d [nb][n] fp16 scales, logical
// row order (gate|up interleaved as the fused pass reads it)
struct Q6Dev {
    uint8_t *w = nullptr;
    uint16_t *d = nullptr;
};

struct Q8Buf {
    int8_t *qs = nullptr;
    uint16_t *d = nullptr;
    int16_t *s = nullptr;
    int8_t *tq = nullptr;    // optional operand-tiled copy (q8_tiled_byte), up to 64 rows
    uint16_t *td = nullptr;
};

// Device allocations owned by one object, released with it.
struct DevArena {
    std::vector<void *> allocs;
    DevArena() = default;
    DevArena(const DevArena &) = delete;
    DevArena &operator=(const DevArena &) = delete;
    ~DevArena() {
        for (void *p : allocs) (void)hipFree(p);
    }
    template <typename T>
    int alloc(T **p, size_t count) {
        *p = nullptr;
        if (count == 0) return SI_OK;
        void *q = nullptr;
        if (hipMalloc(&q, count * sizeof(T)) != hipSuccess)
            return fail(SI_ERR_NOMEM, "hipMalloc(%zu bytes) failed", count * sizeof(T));
        allocs.push_back(q);
        *p = (T *)q;
        return SI_OK;
    }
};

#define TRY(x)               \
    do {                     \
        int r_ = (x);        \
        if (r_) return r_;   \
    } while (0)

// Activation buffers, attention partials and RoPE tables: everything a
// layer call uses besides its weights and the KV cache.  Layers of one
// model can share one workspace (they run one after another on a stream).
struct Workspace {
    si_shape_t s;
    int max_tokens = 0, max_pos = 0;
    bool ffn = false;
    DevArena mem;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *normed = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr;
    float *attn_out = nullptr, *h = nullptr, *normed2 = nullptr, *gu = nullptr, *act = nullptr;
    Q8Buf xq, attq, xq2, actq;
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void *gemm_ws = nullptr;  // split-K partial sums of the matrix-core GEMMs
    size_t gemm_ws_bytes = 0;
    float *scores = nullptr;  // [qheads][max_pos]: the standard attention mode
    uint8_t *x6 = nullptr;    // past 512 rows: a GEMM input as fp6 hi/lo codes
};

struct si_workspace {
    std::shared_ptr<Workspace> p;
};

static int upload_f32(DevArena &mem, float **dst, const float *src, size_t n) {
    *dst = nullptr;
    if (!src) return SI_OK;
    TRY(mem.alloc(dst, n));
    HIP_TRY(hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice));
    return SI_OK;
}

static int make_workspace(const si_shape_t *s, int max_tokens, int max_pos,
                          std::shared_ptr<Workspace> *out) {
    TRY(check_shape(s));
    SI_REQUIRE(max_tokens >= 1 && max_pos >= 1, "workspace: bad max_tokens/max_pos");
    auto W = std::make_shared<Workspace>();
    W->s = *s;
    W->max_tokens = max_tokens;
    W->max_pos = max_pos;
    W->ffn = s->ffn > 0;
    const int H = s->hidden, QD = s->qheads * s->hdim, KVD = s->kvheads * s->hdim, F = s->ffn;
    const int NQKV = QD + 2 * KVD;
    const size_t M = max_tokens, MH = M * H;
    DevArena &m = W->mem;
    {
        const size_t te = (size_t)max_pos * (s->hdim / 2);
        std::vector<float> c(te), sn(te);
        si_rope_table(max_pos, s->hdim, s->rope_base, c.data(), sn.data());
        TRY(upload_f32(m, &W->rope_cos, c.data(), te));
        TRY(upload_f32(m, &W->rope_sin, sn.data(), te));
    }
    TRY(m.alloc(&W->normed, MH));
    TRY(m.alloc(&W->qkv, M * NQKV));
    TRY(m.alloc(&W->q, M * QD));
    TRY(m.alloc(&W->attn, M * QD));
    TRY(m.alloc(&W->attn_out, MH));
    TRY(m.alloc(&W->xq.qs, MH));
    TRY(m.alloc(&W->xq.d, MH / 32));
    TRY(m.alloc(&W->xq.s, MH / 32));
    TRY(m.alloc(&W->attq.qs, M * QD));
    TRY(m.alloc(&W->attq.d, M * QD / 32));
    TRY(m.alloc(&W->attq.s, M * QD / 32));
    if (W->ffn) {
        TRY(m.alloc(&W->h, MH));
        TRY(m.alloc(&W->normed2, MH));
        TRY(m.alloc(&W->gu, M * 2 * F));
        TRY(m.alloc(&W->act, M * F));
        TRY(m.alloc(&W->xq2.qs, MH));
        TRY(m.alloc(&W->xq2.d, MH / 32));
        TRY(m.alloc(&W->xq2.s, MH / 32));
        TRY(m.alloc(&W->actq.qs, M * F));
        TRY(m.alloc(&W->actq.d, M * F / 32));
        TRY(m.alloc(&W->actq.s, M * F / 32));
    }
    if (max_tokens >= 2) {
        // operand-tiled copies of the four GEMM inputs for calls of 2..512
        // rows (the projections then stream them); padding rows stay zero
        const size_t tr = (size_t)(std::min(max_tokens, 512) + 31) / 32 * 32;
        auto tiled = [&](Q8Buf &b, size_t k) -> int {
            TRY(m.alloc(&b.tq, tr * k));
            TRY(m.alloc(&b.td, tr * k / 32));
            HIP_TRY(hipMemset(b.tq, 0, tr * k));
            HIP_TRY(hipMemset(b.td, 0, tr * k / 32 * sizeof(uint16_t)));
            return SI_OK;
        };
        TRY(tiled(W->xq, H));
        TRY(tiled(W->attq, QD));
        if (W->ffn) {
            TRY(tiled(W->xq2, H));
            TRY(tiled(W->actq, F));
        }
    }
    // attention partials: the split count depends on the row count, so the
    // size is the worst case over 1..max_tokens rows of either schedule
    for (int nq = 1; nq <= max_tokens; ++nq) {
        size_t b = si_attention_workspace(s, nq, max_pos);
        const size_t bd = dec_attn_workspace_bytes(s->qheads, s->hdim, s->kvheads, nq, max_pos);
        if (bd > b) b = bd;
        if (b > W->attn_ws_bytes) W->attn_ws_bytes = b;
    }
    uint8_t *ws = nullptr;
    TRY(m.alloc(&ws, W->attn_ws_bytes));
    W->attn_ws = ws;
    TRY(m.alloc(&W->scores, (size_t)s->qheads * max_pos));
    // past 64 rows the gate|up GEMM (past 512 all four) runs in the fp6 formulation
    if (max_tokens > 64)
        TRY(m.alloc(&W->x6, M * (size_t)(std::max(std::max(H, QD), F) / 32) * 48));
    // GEMM split-K partials: the largest need over the layer's projections
    // and every row count up to max_tokens (the split depends on both)
    {
        const int dims[4][2] = {{NQKV, H}, {H, QD}, {2 * F, H}, {H, F}};
        for (int r = 2; r <= max_tokens; ++r)
            for (const auto &d : dims)
                if (d[0] > 0 && d[1] > 0) {
                    const size_t b = gemm_workspace_bytes(r, d[0], d[1]);
                    if (b > W->gemm_ws_bytes) W->gemm_ws_bytes = b;
                }
        uint8_t *gw = nullptr;
        TRY(m.alloc(&gw, W->gemm_ws_bytes));
        W->gemm_ws = gw;
    }
    *out = std::move(W);
    return SI_OK;
}

struct si_layer {
    si_shape_t s;
    int max_tokens = 0, max_pos = 0;
    bool ffn = false;
    DevArena mem;  // weights
    Q4Dev wqkv, wo, wgu, wdown;
    // prefill of more than 64 rows: Q|K|V with its output rows in
    // rope_perm_row order (and its bias), for the projection that applies
    // RoPE and appends K/V in its epilogue
    Q4Dev wqkv_rope;
    float *bqkv_rope = nullptr;
    bool has_rope = false;
    // the matrices for the fp6 GEMMs: gate|up past 64 rows, all four past 512
    Q6Dev wqkv6, wo6, wgu6, wdown6;
    bool has_f6 = false, has_f6_gu = false;
    uint8_t *x6 = nullptr;
    float *norm = nullptr, *bqkv = nullptr, *post_norm = nullptr;
    std::shared_ptr<Workspace> ws;
    // views of the workspace buffers
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *normed = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr;
    float *attn_out = nullptr, *h = nullptr, *normed2 = nullptr, *gu = nullptr, *act = nullptr;
    Q8Buf xq, attq, xq2, actq;
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void *gemm_ws = nullptr;
    size_t gemm_ws_bytes = 0;
    float *scores = nullptr;
    // phase timing: events[i] marks the start of phase i, events[COUNT] the end
    bool timing = false;
    hipEvent_t events[SI_PHASE_COUNT + 1] = {};
    bool phase_hit[SI_PHASE_COUNT] = {};
    int last_phase = -1;
    ~si_layer() {
        for (hipEvent_t &e : events)
            if (e) (void)hipEventDestroy(e);
    }
};

static void mark(si_layer *L, int phase, hipStream_t st) {
    if (!L->timing) return;
    (void)hipEventRecord(L->events[phase], st);
    if (phase < SI_PHASE_COUNT) L->phase_hit[phase] = true;
    L->last_phase = phase;
}

// Uploads row-major Q4_0 matrices stacked along N and repacks them.
static int upload_q4(DevArena &mem, Q4Dev *w, const std::vector<const uint8_t *> &parts,
                     const std::vector<int> &rows, int k, int tile) {
    int n = 0;
    for (int r : rows) n += r;
    const size_t row_bytes = (size_t)(k / 32) * 18;
    w->n = n;
    w->k = k;
    w->tile = tile;
    TRY(mem.alloc(&w->qs, (size_t)n * k / 2));
    TRY(mem.alloc(&w->d, q4_scale_count(n, k / 32, tile)));
    uint8_t *tmp = nullptr;
    HIP_TRY(hipMalloc(&tmp, (size_t)n * row_bytes));
    size_t off = 0;
    for (size_t i = 0; i < parts.size(); ++i) {
        hipError_t e = hipMemcpy(tmp + off, parts[i], rows[i] * row_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(tmp);
            return fail(SI_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
        }
        off += rows[i] * row_bytes;
    }
    launch_q4_repack(tmp, n, k, tile, w->qs, w->d, 0);
    hipError_t e = hipDeviceSynchronize();
    (void)hipFree(tmp);
    if (e != hipSuccess) return fail(SI_ERR_HIP, "repack: %s", hipGetErrorString(e));
    return SI_OK;
}

// The fp6 copy of a repacked Q4 matrix (gu_f > 0: the gate|up pair of gu_f
// features, stored in the fused pass's row order).
static int make_q6(DevArena &mem, const Q4Dev &q, int gu_f, Q6Dev *o) {
    const size_t cnt = (size_t)q.n * (q.k / 32);
    TRY(mem.alloc(&o->w, cnt * 24));
    TRY(mem.alloc(&o->d, cnt));
    launch_q4_to_w6(q.qs, q.d, q.n, q.k / 32, q.tile, gu_f, o->w, o->d, 0);
    HIP_TRY(hipDeviceSynchronize());
    return SI_OK;
}

// Argument checks of a layer's host weights, before anything is allocated.
static int check_host(const si_shape_t *s, const si_layer_host_t *w, si_layer_t **out) {
    TRY(check_shape(s));
    SI_REQUIRE(w && out, "layer_create: NULL pointer");
    SI_REQUIRE(w->wq && w->wk && w->wv && w->wo, "layer_create: wq/wk/wv/wo are required");
    const bool ffn = w->wgate || w->wup || w->wdown;
    SI_REQUIRE(!ffn || (w->wgate && w->wup && w->wdown && s->ffn > 0),
               "layer_create: FFN needs wgate, wup, wdown and shape.ffn > 0");
    return SI_OK;
}

static int build_layer(const si_layer_host_t *w, std::shared_ptr<Workspace> W,
                       si_layer_t **out) {
    const si_shape_t *s = &W->s;
    TRY(check_host(s, w, out));
    const bool ffn = w->wgate || w->wup || w->wdown;
    std::unique_ptr<si_layer> L(new si_layer());
    L->s = *s;
    L->max_tokens = W->max_tokens;
    L->max_pos = W->max_pos;
    L->ffn = ffn;
    const int H = s->hidden, QD = s->qheads * s->hdim, KVD = s->kvheads * s->hdim, F = s->ffn;
    const int NQKV = QD + 2 * KVD;
    // scale tiles: the decode mat-vec's rows per workgroup; gate|up pairs 32
    // gate with 32 up rows per workgroup (tile 32)
    TRY(upload_q4(L->mem, &L->wqkv, {w->wq, w->wk, w->wv}, {QD, KVD, KVD}, H,
                  gemv_tile_for(NQKV)));
    TRY(upload_q4(L->mem, &L->wo, {w->wo}, {H}, QD, gemv_tile_for(H)));
    if (ffn) {
        TRY(upload_q4(L->mem, &L->wgu, {w->wgate, w->wup}, {F, F}, H, 32));
        TRY(upload_q4(L->mem, &L->wdown, {w->wdown}, {H}, F, gemv_tile_for(H)));
    }
    TRY(upload_f32(L->mem, &L->norm, w->norm, H));
    TRY(upload_f32(L->mem, &L->post_norm, w->post_norm, H));
    if (w->bq || w->bk || w->bv) {
        std::vector<float> b(NQKV, 0.0f);  // absent bias = zero (qwen_one_layer.c:154)
        if (w->bq) memcpy(b.data(), w->bq, QD * sizeof(float));
        if (w->bk) memcpy(b.data() + QD, w->bk, KVD * sizeof(float));
        if (w->bv) memcpy(b.data() + QD + KVD, w->bv, KVD * sizeof(float));
        TRY(upload_f32(L->mem, &L->bqkv, b.data(), NQKV));
        if (L->max_tokens > 64 && s->hdim % 2 == 0) {
            std::vector<float> bp(NQKV);
            for (int pr = 0; pr < NQKV; ++pr) bp[pr] = b[rope_perm_row(pr, s->hdim)];
            TRY(upload_f32(L->mem, &L->bqkv_rope, bp.data(), NQKV));
        }
    }
    if (L->max_tokens > 64 && s->hdim % 2 == 0) {
        // the Q|K|V rows regathered in rope_perm_row order (row-major Q4_0)
        const size_t rb = (size_t)(H / SI_QK) * 18;
        std::vector<uint8_t> perm((size_t)NQKV * rb);
        for (int pr = 0; pr < NQKV; ++pr) {
            const int o = rope_perm_row(pr, s->hdim);
            const uint8_t *src = o < QD         ? w->wq + (size_t)o * rb
                                 : o < QD + KVD ? w->wk + (size_t)(o - QD) * rb
                                                : w->wv + (size_t)(o - QD - KVD) * rb;
            memcpy(perm.data() + (size_t)pr * rb, src, rb);
        }
        TRY(upload_q4(L->mem, &L->wqkv_rope, {perm.data()}, {NQKV}, H, gemv_tile_for(NQKV)));
        L->has_rope = true;
    }
    if (L->max_tokens > 64 && W->x6 && ffn) {
        TRY(make_q6(L->mem, L->wgu, F, &L->wgu6));
        L->x6 = W->x6;
        L->has_f6_gu = true;
    }
    if (L->max_tokens > 512 && W->x6) {
        TRY(make_q6(L->mem, L->wqkv, 0, &L->wqkv6));
        TRY(make_q6(L->mem, L->wo, 0, &L->wo6));
        if (ffn) TRY(make_q6(L->mem, L->wdown, 0, &L->wdown6));
        L->x6 = W->x6;
        L->has_f6 = true;
    }
    L->rope_cos = W->rope_cos;
    L->rope_sin = W->rope_sin;
    L->normed = W->normed;
    L->qkv = W->qkv;
    L->q = W->q;
    L->attn = W->attn;
    L->attn_out = W->attn_out;
    L->h = W->h;
    L->normed2 = W->normed2;
    L->gu = W->gu;
    L->act = W->act;
    L->xq = W->xq;
    L->attq = W->attq;
    L->xq2 = W->xq2;
    L->actq = W->actq;
    L->attn_ws = W->attn_ws;
    L->attn_ws_bytes = W->attn_ws_bytes;
    L->gemm_ws = W->gemm_ws;
    L->gemm_ws_bytes = W->gemm_ws_bytes;
    L->scores = W->scores;
    L->ws = std::move(W);
    *out = L.release();
    return SI_OK;
}

extern "C" {

int si_workspace_create(const si_shape_t *s, int max_tokens, int max_pos,
                        si_workspace_t **out) {
    SI_REQUIRE(out, "workspace_create: NULL pointer");
    std::shared_ptr<Workspace> W;
    TRY(make_workspace(s, max_tokens, max_pos, &W));
    *out = new si_workspace{std::move(W)};
    return SI_OK;
}

int si_workspace_destroy(si_workspace_t *ws) {
    if (!ws) return SI_OK;
    (void)hipDeviceSynchronize();
    delete ws;  // the memory goes when the last layer using it is destroyed
    return SI_OK;
}

int si_layer_create(const si_shape_t *s, const si_layer_host_t *w, int max_tokens, int max_pos,
                    si_layer_t **out) {
    TRY(check_host(s, w, out));
    std::shared_ptr<Workspace> W;
    TRY(make_workspace(s, max_tokens, max_pos, &W));
    return build_layer(w, std::move(W), out);
}

int si_layer_create_in(si_workspace_t *ws, const si_layer_host_t *w, si_layer_t **out) {
    SI_REQUIRE(ws && ws->p, "layer_create_in: NULL workspace");
    return build_layer(w, ws->p, out);
}

int si_layer_destroy(si_layer_t *L) {
    if (!L) return SI_OK;
    (void)hipDeviceSynchronize();
    delete L;
    return SI_OK;
}

void *si_layer_buffer(si_layer_t *L, int which) {
    if (!L) return nullptr;
    switch (which) {
        case SI_BUF_NORMED: return L->normed;
        case SI_BUF_XQ_QS: return L->xq.qs;
        case SI_BUF_XQ_D: return L->xq.d;
        case SI_BUF_XQ_S: return L->xq.s;
        case SI_BUF_QKV: return L->qkv;
        case SI_BUF_Q: return L->q;
        case SI_BUF_ATTN: return L->attn;
        case SI_BUF_ATTQ_QS: return L->attq.qs;
        case SI_BUF_ATTQ_D: return L->attq.d;
        case SI_BUF_ATTQ_S: return L->attq.s;
        case SI_BUF_ATTN_OUT: return L->attn_out;
        case SI_BUF_H: return L->h;
        case SI_BUF_NORMED2: return L->normed2;
        case SI_BUF_XQ2_QS: return L->xq2.qs;
        case SI_BUF_XQ2_D: return L->xq2.d;
        case SI_BUF_XQ2_S: return L->xq2.s;
        case SI_BUF_GU: return L->gu;
        case SI_BUF_ACT: return L->act;
        case SI_BUF_ACTQ_QS: return L->actq.qs;
        case SI_BUF_ACTQ_D: return L->actq.d;
        case SI_BUF_ACTQ_S: return L->actq.s;
        case SI_BUF_ACTQ_TQ: return L->actq.tq;
        case SI_BUF_ACTQ_TD: return L->actq.td;
        default: return nullptr;
    }
}

int si_layer_set_timing(si_layer_t *L, int enable) {
    SI_REQUIRE(L, "layer_set_timing: NULL layer");
    if (enable && !L->events[0])
        for (hipEvent_t &e : L->events) HIP_TRY(hipEventCreate(&e));
    L->timing = enable != 0;
    return SI_OK;
}

int si_layer_phase_ms(si_layer_t *L, float *ms) {
    SI_REQUIRE(L && ms, "layer_phase_ms: NULL pointer");
    SI_REQUIRE(L->timing && L->last_phase == SI_PHASE_COUNT, "no timed layer call recorded");
    HIP_TRY(hipEventSynchronize(L->events[SI_PHASE_COUNT]));
    for (int p = 0; p < SI_PHASE_COUNT; ++p) {
        ms[p] = 0.0f;
        if (!L->phase_hit[p]) continue;
        int q = p + 1;
        while (q < SI_PHASE_COUNT && !L->phase_hit[q]) ++q;
        HIP_TRY(hipEventElapsedTime(&ms[p], L->events[p], L->events[q]));
    }
    return SI_OK;
}

int si_layer_weights(si_layer_t *L, int which, const uint8_t **qs, const uint16_t **d,
                     int *tile, int *n, int *k) {
    SI_REQUIRE(L && qs && d && tile && n && k, "layer_weights: NULL pointer");
    const Q4Dev *w = which == 0 ? &L->wqkv : which == 1 ? &L->wo : which == 2 ? &L->wgu
                   : which == 3 ? &L->wdown : nullptr;
    SI_REQUIRE(w && w->n, "layer_weights: no matrix %d", which);
    *qs = w->qs;
    *d = w->d;
    *tile = w->tile;
    *n = w->n;
    *k = w->k;
    return SI_OK;
}

}  // extern "C"

// Projection of rows activation rows: mat-vec for one row, matrix-core
// GEMM otherwise.
static void project(si_layer *L, const Q4Dev &w, int rows, const Q8Buf &x, const float *bias,
                    const float *residual, float *out, int flags, hipStream_t st) {
    if (rows == 1)
        launch_matvec(x.qs, x.d, x.s, w.k, w.qs, w.d, w.tile, w.n, bias, residual, out,
                      (flags & SI_LAYER_EXACT) != 0, st);
    else
        launch_gemm_q4q8(w.qs, w.d, w.tile, w.n, w.k, x.qs, x.d, rows, bias, residual, out, w.n,
                         (flags & SI_LAYER_EXACT) != 0, L->gemm_ws, L->gemm_ws_bytes, st);
}

static int run_decode_ffn(si_layer *L, float *out, bool exact, bool cap, hipStream_t st);

// A capture buffer when SI_LAYER_CAPTURE is set, else NULL (not written).
template <typename T>
static inline T *capt(bool cap, T *p) {
    return cap ? p : nullptr;
}

// Single-token decode: five fused kernels (si_decode.hip).
static int run_decode(si_layer *L, const float *x, uint16_t *kc, uint16_t *vc, int ctx,
                      float *out, int flags, hipStream_t st) {
    const si_shape_t &s = L->s;
    const int H = s.hidden, QD = s.qheads * s.hdim, NQKV = QD + 2 * s.kvheads * s.hdim;
    const bool full = !(flags & SI_LAYER_ATTN_ONLY);
    const bool exact = (flags & SI_LAYER_EXACT) != 0;
    const bool cap = (flags & SI_LAYER_CAPTURE) != 0;
    SI_REQUIRE(!full || L->ffn, "layer has no FFN weights: use SI_LAYER_ATTN_ONLY");
    for (bool &h : L->phase_hit) h = false;
    const bool standard = (flags & SI_LAYER_ATTN_STANDARD) != 0;
    // a small layer projects Q|K|V inside the attention kernel (no q|k|v
    // round trip); the exact projections and standard attention take the
    // staged kernels
    const bool fused_qkv =
        !exact && !standard && dec_qkv_attn_ok(H, s.qheads, s.kvheads, s.hdim, ctx);
    if (!fused_qkv) {
        // qwen_one_layer.c:247-258: RMSNorm -> Q8 -> Q, K, V (+bias)
        mark(L, SI_PHASE_QKV, st);
        launch_dec_qkv(x, L->norm, H, s.rms_eps, L->wqkv.qs, L->wqkv.d, L->wqkv.tile, NQKV,
                       L->bqkv, capt(cap, L->normed), capt(cap, L->xq.qs), capt(cap, L->xq.d),
                       capt(cap, L->xq.s), L->qkv, exact, st);
    }
    if (standard) {
        // the reference's staged order with attention_standard
        // (qwen_one_layer.c:260-275, attention_kernels.h:33-78)
        mark(L, SI_PHASE_ROPE_KV, st);
        launch_rope_kv(L->qkv, NQKV, 1, s.qheads, s.kvheads, s.hdim, ctx - 1, 1, ctx, nullptr,
                       L->rope_cos, L->rope_sin, L->q, kc, vc, 0, st);
        mark(L, SI_PHASE_ATTENTION_Q8, st);
        launch_attn_standard(L->q, s.qheads, s.kvheads, s.hdim, kc, vc, ctx, L->attn, L->scores,
                             st);
        launch_quantize_q8_rows(L->attn, 1, QD, L->attq.qs, L->attq.d, L->attq.s, st);
        mark(L, SI_PHASE_OUT_PROJ, st);
        launch_matvec(L->attq.qs, L->attq.d, L->attq.s, QD, L->wo.qs, L->wo.d, L->wo.tile, H,
                      nullptr, full ? x : nullptr, full ? L->h : out, exact, st,
                      full ? capt(cap, L->attn_out) : nullptr);
        if (!full) {
            mark(L, SI_PHASE_COUNT, st);
            return check_launch("layer decode (standard attention sublayer)");
        }
        return run_decode_ffn(L, out, exact, cap, st);
    }
    // :260-270: RoPE, fp16 K/V append at context-1, attention over the cache
    mark(L, SI_PHASE_ATTENTION_Q8, st);
    const int ns = dec_attn_chunks(s.qheads, s.kvheads, s.hdim, 1, ctx);
    if (fused_qkv) {
        DecQkvIn fq;
        fq.x = x;
        fq.gain = L->norm;
        fq.hidden = H;
        fq.eps = s.rms_eps;
        fq.wqs = L->wqkv.qs;
        fq.wd = L->wqkv.d;
        fq.tile = L->wqkv.tile;
        fq.n = NQKV;
        fq.bias = L->bqkv;
        fq.cap_normed = capt(cap, L->normed);
        fq.cap_qs = capt(cap, L->xq.qs);
        fq.cap_d = capt(cap, L->xq.d);
        fq.cap_s = capt(cap, L->xq.s);
        fq.cap_qkv = capt(cap, L->qkv);
        launch_dec_qkv_attn(fq, s.qheads, s.kvheads, s.hdim, L->rope_cos, L->rope_sin, kc, vc,
                            ctx, ns, capt(cap, L->q), L->attn_ws, st);
    } else {
        launch_dec_attn(L->qkv, NQKV, 1, s.qheads, s.kvheads, s.hdim, L->rope_cos, L->rope_sin,
                        kc, vc, 0, nullptr, ctx, ctx, capt(cap, L->q), ns, L->attn_ws, nullptr,
                        nullptr, nullptr, nullptr, st);
    }
    // :272-275: Q8 of the attention output, W_O (no bias); + x in the full layer
    mark(L, SI_PHASE_OUT_PROJ, st);
    const float *pm = (const float *)L->attn_ws;
    const float *pl = pm + (size_t)s.qheads * ns;
    const float *po = pl + (size_t)s.qheads * ns;
    if ((size_t)s.qheads * ns * (s.hdim + 2) * sizeof(float) > 32 * 1024) {
        // many chunk partials (7B at long contexts): merge them once instead
        // of in every W_O workgroup (each would re-read all of them)
        launch_attn_combine(1, s.qheads, s.hdim, ns, L->attn_ws, L->attn, L->attq.qs, L->attq.d,
                            L->attq.s, st);
        launch_matvec(L->attq.qs, L->attq.d, L->attq.s, QD, L->wo.qs, L->wo.d, L->wo.tile, H,
                      nullptr, full ? x : nullptr, full ? L->h : out, exact, st,
                      full ? capt(cap, L->attn_out) : nullptr);
    } else {
        launch_dec_wo(pm, pl, po, ns, s.qheads, s.hdim, L->wo.qs, L->wo.d, L->wo.tile, H,
                      full ? x : nullptr, capt(cap, L->attn), capt(cap, L->attq.qs),
                      capt(cap, L->attq.d), capt(cap, L->attq.s),
                      full ? capt(cap, L->attn_out) : nullptr, full ? L->h : out, exact, st);
    }
    if (!full) {
        mark(L, SI_PHASE_COUNT, st);
        return check_launch("layer decode (attention sublayer)");
    }
    return run_decode_ffn(L, out, exact, cap, st);
}

// FFN half of the decode layer: RMSNorm(h) -> Q8 -> gate|up -> SwiGLU -> Q8
// -> down + h
static int run_decode_ffn(si_layer *L, float *out, bool exact, bool cap, hipStream_t st) {
    const si_shape_t &s = L->s;
    const int H = s.hidden;
    mark(L, SI_PHASE_GATE_UP, st);
    launch_dec_gateup(L->h, L->post_norm, H, s.rms_eps, L->wgu.qs, L->wgu.d, L->wgu.tile, s.ffn,
                      capt(cap, L->normed2), capt(cap, L->xq2.qs), capt(cap, L->xq2.d),
                      capt(cap, L->xq2.s), capt(cap, L->gu), capt(cap, L->act), L->actq.qs,
                      L->actq.d, L->actq.s, exact, st);
    mark(L, SI_PHASE_DOWN, st);
    launch_matvec(L->actq.qs, L->actq.d, L->actq.s, s.ffn, L->wdown.qs, L->wdown.d,
                  L->wdown.tile, H, nullptr,
                  L->h, out, exact, st);
    mark(L, SI_PHASE_COUNT, st);
    return check_launch("layer decode");
}

// Shared schedule of the matrix-core paths.  rows activation rows;
// positions and attention contexts come either from (pos0, ctx0, ctx_step)
// or from ctx_dev.  ctx_step 0 is batched decode (one new token per
// sequence), ctx_step 1 causal prefill.
static int run_rows(si_layer *L, const float *x, int rows, uint16_t *kc, uint16_t *vc,
                    size_t kv_seq_stride, int pos0, const int *ctx_dev, int ctx0, int ctx_step,
                    int max_ctx, float *out, int flags, hipStream_t st,
                    KvPages pg = KvPages()) {
    const int pos_step = ctx_step;  // positions advance with the contexts
    const si_shape_t &s = L->s;
    const int H = s.hidden, QD = s.qheads * s.hdim, NQKV = QD + 2 * s.kvheads * s.hdim;
    const bool full = !(flags & SI_LAYER_ATTN_ONLY);
    const bool cap = (flags & SI_LAYER_CAPTURE) != 0;
    SI_REQUIRE(!full || L->ffn, "layer has no FFN weights: use SI_LAYER_ATTN_ONLY");
    for (bool &h : L->phase_hit) h = false;
    // 2..512 rows, not exact: the Q8 activations are also written operand-
    // tiled, and the projections whose plan is the one-tile kernel stream
    // them (k_gemm_bd's streamed mode, gemm_streams)
    const bool ex = (flags & SI_LAYER_EXACT) != 0;
    const bool tl = rows >= 2 && rows <= 512 && !ex && L->xq.tq;
    // qwen_one_layer.c:247-250: RMSNorm -> Q8
    mark(L, SI_PHASE_RMS_Q8, st);
    // up to 64 rows every projection streams; past that only down (below)
    const bool tl_x = tl && rows <= 64;
    launch_rmsnorm_q8(x, nullptr, L->norm, rows, H, s.rms_eps, nullptr, capt(cap, L->normed),
                      L->xq.qs, L->xq.d, L->xq.s, st, tl_x ? L->xq.tq : nullptr,
                      tl_x ? L->xq.td : nullptr);
    // :253-258: Q, K, V projections (+bias), fused into one N = qd + 2 kvd matrix
    mark(L, SI_PHASE_QKV, st);
    // past 64 rows only the down projection streams: there the K-split
    // partials and their reduce disappear (0.5B, 512 rows: 21.0 -> 16.6 us),
    // while Q|K|V gains little (10.1 -> 10.0 us) and its changed sum order
    // would move the fp16 K/V rows the later rows attend to
    // a prefill of 65-512 rows: RoPE and the K/V append in the projection's
    // epilogue (the rope_kv phase is then empty)
    bool roped = false;
    if (ctx_step == 1 && !ctx_dev && !pg.pages && !ex && L->has_rope) {
        const RopeOut ro{L->rope_cos, L->rope_sin, L->q, kc, vc, kv_seq_stride,
                         pos0, max_ctx, s.hdim, QD, s.kvheads * s.hdim};
        roped = launch_gemm_qkv_rope(L->wqkv_rope.qs, L->wqkv_rope.d, L->wqkv_rope.tile, NQKV,
                                     H, L->xq.qs, L->xq.d, rows, L->bqkv_rope, capt(cap, L->qkv),
                                     ro, st);
    }
    // past 512 rows the four GEMMs run in the fp6 formulation, each input
    // first converted to fp6 hi/lo codes
    const bool f6 = L->has_f6 && rows > 512 && !ex;
    if (roped)
        ;
    else if (f6) {
        launch_q8_to_x6(L->xq.qs, rows, H / SI_QK, L->x6, st);
        launch_gemm_f6(L->wqkv6.w, L->wqkv6.d, NQKV, H, L->x6, L->xq.d, rows, L->bqkv, nullptr,
                       L->qkv, NQKV, L->gemm_ws, L->gemm_ws_bytes, false, 0, nullptr, nullptr,
                       nullptr, nullptr, st);
    } else if (tl_x && gemm_streams(rows, NQKV, H))
        launch_gemm_q4q8_tiled(L->wqkv.qs, L->wqkv.d, L->wqkv.tile, NQKV, H, L->xq.tq, L->xq.td,
                               rows, L->bqkv, nullptr, L->qkv, NQKV, st);
    else
        project(L, L->wqkv, rows, L->xq, L->bqkv, nullptr, L->qkv, flags, st);
    bool tl_att = false;  // the attention's Q8 written operand-tiled too
    if (ctx_step == 0) {
        // batched decode: RoPE + K/V append inside the attention kernel,
        // contiguous caches or a paged pool (pg)
        mark(L, SI_PHASE_ATTENTION_Q8, st);
        const int ns = dec_attn_chunks(s.qheads, s.kvheads, s.hdim, rows, max_ctx);
        if (ns == 1) {
            launch_dec_attn(L->qkv, NQKV, rows, s.qheads, s.kvheads, s.hdim, L->rope_cos,
                            L->rope_sin, kc, vc, kv_seq_stride, ctx_dev, ctx0, max_ctx,
                            capt(cap, L->q), 1, L->attn_ws, L->attn, L->attq.qs, L->attq.d,
                            L->attq.s, st, pg);
        } else {
            launch_dec_attn(L->qkv, NQKV, rows, s.qheads, s.kvheads, s.hdim, L->rope_cos,
                            L->rope_sin, kc, vc, kv_seq_stride, ctx_dev, ctx0, max_ctx,
                            capt(cap, L->q), ns, L->attn_ws, nullptr, nullptr, nullptr, nullptr,
                            st, pg);
            tl_att = tl_x;
            launch_attn_combine(rows, s.qheads, s.hdim, ns, L->attn_ws, L->attn, L->attq.qs,
                                L->attq.d, L->attq.s, st, tl_x ? L->attq.tq : nullptr,
                                tl_x ? L->attq.td : nullptr);
        }
    } else {
        mark(L, SI_PHASE_ROPE_KV, st);
        // :260-266: RoPE at the token's position, fp16 K/V append
        if (!roped)
            launch_rope_kv(L->qkv, NQKV, rows, s.qheads, s.kvheads, s.hdim, pos0, pos_step,
                           max_ctx, ctx_dev, L->rope_cos, L->rope_sin, L->q, kc, vc,
                           kv_seq_stride, st);
        // :268-272: attention over the fp16 cache -> Q8
        mark(L, SI_PHASE_ATTENTION_Q8, st);
        if (ctx_dev == nullptr && attn_prefill_supported(s.qheads, s.kvheads, s.hdim))
            launch_attn_prefill(L->q, rows, s.qheads, s.kvheads, s.hdim, pos0, kc, vc, L->attn,
                                L->attq.qs, L->attq.d, L->attq.s, L->attn_ws, L->attn_ws_bytes,
                                st);
        else
            launch_attention(L->q, rows, s.qheads, s.kvheads, s.hdim, kc, vc, kv_seq_stride,
                             ctx_dev, ctx0, ctx_step, max_ctx, L->attn, L->attq.qs, L->attq.d,
                             L->attq.s, L->attn_ws, st);
    }
    mark(L, SI_PHASE_OUT_PROJ, st);
    if (!full) {
        // :275: W_O, no bias, no residual
        project(L, L->wo, rows, L->attq, nullptr, nullptr, out, flags, st);
        mark(L, SI_PHASE_COUNT, st);
        return check_launch("layer (attention sublayer)");
    }
    // W_O; a K-split leaves its partials to the post-norm kernel, which sums
    // them (o, kept in attn_out) on the way
    int osplits = 0;
    if (tl_att && gemm_streams(rows, L->wo.n, L->wo.k))
        launch_gemm_q4q8_tiled(L->wo.qs, L->wo.d, L->wo.tile, L->wo.n, L->wo.k, L->attq.tq,
                               L->attq.td, rows, nullptr, nullptr, L->attn_out, L->wo.n, st);
    else if (f6) {
        launch_q8_to_x6(L->attq.qs, rows, QD / SI_QK, L->x6, st);
        osplits = launch_gemm_f6(L->wo6.w, L->wo6.d, L->wo.n, L->wo.k, L->x6, L->attq.d, rows,
                                 nullptr, nullptr, L->attn_out, L->wo.n, L->gemm_ws,
                                 L->gemm_ws_bytes, true, 0, nullptr, nullptr, nullptr, nullptr,
                                 st);
    } else
        osplits = launch_gemm_q4q8_parts(L->wo.qs, L->wo.d, L->wo.tile, L->wo.n, L->wo.k,
                                         L->attq.qs, L->attq.d, rows, L->attn_out, ex,
                                         L->gemm_ws, L->gemm_ws_bytes, st);
    mark(L, SI_PHASE_POST_NORM_Q8, st);
    // past 64 rows the gate|up GEMM runs in the fp6 formulation; up to 512
    // rows the norm writes its input codes itself (past that its scattered
    // 4-byte code stores cost the norm more than a separate conversion)
    const bool f6gu = L->has_f6_gu && rows > 64 && !ex;
    uint8_t *norm_x6 = f6gu && rows <= 512 ? L->x6 : nullptr;
    // build-defined FFN half: h = x + o; RMSNorm -> Q8; gate|up; SwiGLU -> Q8; down + h
    if (osplits > 1)
        launch_rmsnorm_q8_parts(x, (const float *)L->gemm_ws, osplits, L->post_norm, rows, H,
                                s.rms_eps, L->attn_out, L->h, capt(cap, L->normed2), L->xq2.qs,
                                L->xq2.d, L->xq2.s, st, tl_x ? L->xq2.tq : nullptr,
                                tl_x ? L->xq2.td : nullptr, norm_x6);
    else
        launch_rmsnorm_q8(x, L->attn_out, L->post_norm, rows, H, s.rms_eps, L->h,
                          capt(cap, L->normed2), L->xq2.qs, L->xq2.d, L->xq2.s, st,
                          tl_x ? L->xq2.tq : nullptr, tl_x ? L->xq2.td : nullptr, norm_x6);
    mark(L, SI_PHASE_GATE_UP, st);
    // the SwiGLU Q8 also operand-tiled; a streamed down projection runs in
    // one pass (no K split, no reduce)
    const bool tiled = tl && gemm_streams(rows, H, s.ffn);
    if (rows == 1) {
        project(L, L->wgu, rows, L->xq2, nullptr, nullptr, L->gu, flags, st);
        mark(L, SI_PHASE_SWIGLU_Q8, st);
        launch_swiglu_q8(L->gu, rows, s.ffn, capt(cap, L->act), L->actq.qs, L->actq.d, L->actq.s,
                         st);
    } else {
        // SwiGLU -> Q8 in the gate|up GEMM's epilogue (the swiglu_q8 phase
        // is then empty); gu is written only as a capture or where it is the
        // intermediate (exact mode)
        // past 64 rows in the fp6 formulation (the fused pass also writes the
        // operand-tiled Q8 a streamed down projection reads)
        bool fused6 = false;
        if (f6gu) {
            if (!norm_x6) launch_q8_to_x6(L->xq2.qs, rows, H / SI_QK, L->x6, st);
            fused6 = launch_gemm_f6(L->wgu6.w, L->wgu6.d, 2 * s.ffn, H, L->x6, L->xq2.d, rows,
                                    nullptr, nullptr, capt(cap, L->gu), 2 * s.ffn, nullptr, 0,
                                    false, s.ffn, capt(cap, L->act), L->actq.qs, L->actq.d,
                                    L->actq.s, st, tiled ? L->actq.tq : nullptr,
                                    tiled ? L->actq.td : nullptr) >= 0;
        }
        if (!fused6)
            launch_gemm_gateup_q8(L->wgu.qs, L->wgu.d, L->wgu.tile, s.ffn, H, L->xq2.qs,
                                  L->xq2.d, rows, capt(cap || ex, L->gu), capt(cap, L->act),
                                  L->actq.qs, L->actq.d, L->actq.s, ex, L->gemm_ws,
                                  L->gemm_ws_bytes, st, false, tiled ? L->actq.tq : nullptr,
                                  tiled ? L->actq.td : nullptr, tl_x ? L->xq2.tq : nullptr,
                                  tl_x ? L->xq2.td : nullptr);
        mark(L, SI_PHASE_SWIGLU_Q8, st);
    }
    mark(L, SI_PHASE_DOWN, st);
    if (tiled)
        launch_gemm_q4q8_tiled(L->wdown.qs, L->wdown.d, L->wdown.tile, H, s.ffn, L->actq.tq,
                               L->actq.td, rows, nullptr, L->h, out, H, st);
    else if (f6) {
        launch_q8_to_x6(L->actq.qs, rows, s.ffn / SI_QK, L->x6, st);
        launch_gemm_f6(L->wdown6.w, L->wdown6.d, H, s.ffn, L->x6, L->actq.d, rows, nullptr, L->h,
                       out, H, L->gemm_ws, L->gemm_ws_bytes, false, 0, nullptr, nullptr, nullptr,
                       nullptr, st);
    } else
        project(L, L->wdown, rows, L->actq, nullptr, L->h, out, flags, st);
    mark(L, SI_PHASE_COUNT, st);
    return check_launch("layer");
}

extern "C" {

int si_layer_decode(si_layer_t *L, const float *x, uint16_t *kc, uint16_t *vc, int context,
                    float *out, int flags, void *stream) {
    SI_REQUIRE(L && x && kc && vc && out, "layer_decode: NULL pointer");
    SI_REQUIRE((flags & ~(SI_LAYER_ATTN_ONLY | SI_LAYER_EXACT | SI_LAYER_ATTN_STANDARD |
                          SI_LAYER_CAPTURE)) == 0,
               "layer_decode: unknown flags %d", flags);
    SI_REQUIRE(!(flags & SI_LAYER_ATTN_STANDARD) ||
                   ((uintptr_t)kc % 16 == 0 && (uintptr_t)vc % 16 == 0),
               "layer_decode: standard attention needs 16-byte aligned kc and vc");
    // qwen_one_layer.c:608: context 1..32768 (here bounded by the RoPE table)
    SI_REQUIRE(context >= 1 && context <= L->max_pos, "context %d outside 1..%d", context,
               L->max_pos);
    return run_decode(L, x, kc, vc, context, out, flags, S(stream));
}

int si_layer_decode_batch(si_layer_t *L, const float *x, int nseq, uint16_t *kc, uint16_t *vc,
                          size_t kv_seq_stride, const int *ctx_dev, int context, int max_ctx,
                          float *out, int flags, void *stream) {
    SI_REQUIRE(L && x && kc && vc && out, "layer_decode_batch: NULL pointer");
    SI_REQUIRE((flags & ~(SI_LAYER_ATTN_ONLY | SI_LAYER_EXACT | SI_LAYER_CAPTURE)) == 0,
               "layer_decode_batch: unsupported flags %d (standard attention is "
               "single-token decode only)", flags);
    SI_REQUIRE(nseq >= 1 && nseq <= L->max_tokens, "nseq %d outside 1..%d", nseq, L->max_tokens);
    SI_REQUIRE(max_ctx >= 1 && max_ctx <= L->max_pos, "max_ctx %d outside 1..%d", max_ctx,
               L->max_pos);
    SI_REQUIRE(ctx_dev || (context >= 1 && context <= max_ctx), "context %d outside 1..%d",
               context, max_ctx);
    SI_REQUIRE(kv_seq_stride % 8 == 0 &&
                   kv_seq_stride >= (size_t)max_ctx * L->s.kvheads * L->s.hdim,
               "kv_seq_stride must hold max_ctx rows and be a multiple of 8");
    return run_rows(L, x, nseq, kc, vc, kv_seq_stride, context - 1, ctx_dev, context, 0, max_ctx,
                    out, flags, S(stream));
}

int si_layer_decode_paged(si_layer_t *L, const float *x, int nseq, uint16_t *k_pool,
                          uint16_t *v_pool, int npages, int page_size, const int *pages,
                          int max_pages, const int *ctx_dev, int context, int max_ctx, float *out,
                          int flags, void *stream) {
    SI_REQUIRE(L && x && k_pool && v_pool && pages && out, "layer_decode_paged: NULL pointer");
    SI_REQUIRE((flags & ~(SI_LAYER_ATTN_ONLY | SI_LAYER_EXACT | SI_LAYER_CAPTURE)) == 0,
               "layer_decode_paged: unsupported flags %d (standard attention is "
               "single-token decode only)", flags);
    SI_REQUIRE(nseq >= 1 && nseq <= L->max_tokens, "nseq %d outside 1..%d", nseq, L->max_tokens);
    SI_REQUIRE(page_size >= 1 && page_size <= (1 << 20) && (page_size & (page_size - 1)) == 0,
               "page_size %d must be a power of two in 1..2^20", page_size);
    SI_REQUIRE(npages >= 1 && max_pages >= 1, "npages and max_pages must be >= 1");
    SI_REQUIRE(max_ctx >= 1 && max_ctx <= L->max_pos, "max_ctx %d outside 1..%d", max_ctx,
               L->max_pos);
    SI_REQUIRE((long long)max_pages * page_size >= max_ctx,
               "max_pages * page_size must cover max_ctx");
    SI_REQUIRE((long long)npages * page_size * L->s.kvheads * L->s.hdim < (1LL << 40),
               "KV pool too large");
    SI_REQUIRE(ctx_dev || (context >= 1 && context <= max_ctx), "context %d outside 1..%d",
               context, max_ctx);
    KvPages pg;
    pg.pages = pages;
    pg.max_pages = max_pages;
    pg.npages = npages;
    while ((1 << pg.shift) < page_size) ++pg.shift;
    return run_rows(L, x, nseq, k_pool, v_pool, 0, context - 1, ctx_dev, context, 0, max_ctx,
                    out, flags, S(stream), pg);
}

int si_attention_paged(const si_shape_t *s, const float *q, int nq, const uint16_t *k_pool,
                       const uint16_t *v_pool, int npages, int page_size, const int *pages,
                       int max_pages, const int *ctx_dev, int max_ctx, float *attn, int8_t *qs,
                       uint16_t *d, int16_t *bsum, void *ws, size_t ws_bytes, void *stream) {
    int r = check_shape(s);
    if (r) return r;
    SI_REQUIRE(nq >= 1 && max_ctx >= 1, "attention_paged: bad nq/max_ctx");
    SI_REQUIRE(q && k_pool && v_pool && pages && ctx_dev && attn && ws,
               "attention_paged: NULL pointer");
    SI_REQUIRE(page_size >= 1 && page_size <= (1 << 20) && (page_size & (page_size - 1)) == 0,
               "page_size %d must be a power of two in 1..2^20", page_size);
    SI_REQUIRE(npages >= 1 && max_pages >= 1 && (long long)max_pages * page_size >= max_ctx,
               "attention_paged: pages do not cover max_ctx");
    SI_REQUIRE(!qs || d, "attention_paged: qs without d");
    SI_REQUIRE(ws_bytes >= si_attention_workspace(s, nq, max_ctx),
               "attention_paged: workspace too small");
    KvPages pg;
    pg.pages = pages;
    pg.max_pages = max_pages;
    pg.npages = npages;
    while ((1 << pg.shift) < page_size) ++pg.shift;
    launch_attention(q, nq, s->qheads, s->kvheads, s->hdim, k_pool, v_pool, 0, ctx_dev, max_ctx,
                     0, max_ctx, attn, qs, d, bsum, ws, S(stream), pg);
    return check_launch("si_attention_paged");
}

int si_layer_prefill(si_layer_t *L, const float *x, int ntok, int prefix, uint16_t *kc,
                     uint16_t *vc, float *out, int flags, void *stream) {
    SI_REQUIRE(L && x && kc && vc && out, "layer_prefill: NULL pointer");
    SI_REQUIRE((flags & ~(SI_LAYER_ATTN_ONLY | SI_LAYER_EXACT | SI_LAYER_CAPTURE)) == 0,
               "layer_prefill: unsupported flags %d (standard attention is "
               "single-token decode only)", flags);
    // prefill_weight_stationary.h:187: 1 <= ntok, 0 <= prefix, prefix+ntok within range
    SI_REQUIRE(ntok >= 1 && ntok <= L->max_tokens, "ntok %d outside 1..%d", ntok, L->max_tokens);
    SI_REQUIRE(prefix >= 0 && prefix + ntok <= L->max_pos, "prefix+ntok exceeds %d", L->max_pos);
    return run_rows(L, x, ntok, kc, vc, 0, prefix, nullptr, prefix + 1, 1, prefix + ntok, out,
                    flags, S(stream));
}

}  // extern "C"
