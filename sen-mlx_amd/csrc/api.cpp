// api.cpp -- the C ABI (include/miqmm.h): argument validation on the host,
// route choice and launch.  Validation mirrors the checks MLX performs before
// recording a quantized_matmul node, returning a status the way mlx-c does
// (src/engine/mlx_lm/utils/moe.rs:66-76: nonzero status, message on the side).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/miqmm.h"
#include "miqmm_internal.h"

namespace miqmm {

int num_cus() {
    // per device id: 0 = not queried yet; two threads racing both store the same value
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace miqmm

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return MIQMM_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

constexpr int64_t kMaxDim = (int64_t)1 << 31;
// The kernels address a tile's rows of x, codes and scales through 32-bit
// buffer offsets (256 rows of x take 512 K bytes): K up to 2^22 keeps every
// such range below 2^31 bytes.
constexpr int64_t kMaxK = (int64_t)1 << 22;
// selections per expert (on average) from which gather_qmm groups them by
// expert into the tiled matmul, when given a workspace
#ifndef MIQMM_GROUPED_MIN
#define MIQMM_GROUPED_MIN 8
#endif
constexpr int64_t kGroupedMinPerExpert = MIQMM_GROUPED_MIN;
// ... and into the grouped MFMA GEMV (fewer selections per expert; below
// about 4 the per-selection GEMV, which streams some experts several times
// but at a higher rate, is faster: DeepSeek-V2-Lite gate/down at 16 tokens
// 39/38 us per-selection vs 67/51 grouped, at 64 tokens 136/134 vs 83/64)
#ifndef MIQMM_GROUPED_GEMV_MIN
#define MIQMM_GROUPED_GEMV_MIN 4
#endif
constexpr int64_t kGroupedGemvMinPerExpert = MIQMM_GROUPED_GEMV_MIN;

int check_quant(int64_t N, int64_t K, int group_size, int bits, int sb_dtype) {
    if (bits != 4 && bits != 8) {
        if (bits == 2 || bits == 3 || bits == 5 || bits == 6)
            return fail(MIQMM_ENOTSUP, "bits=%d is a valid MLX width but only 4 and 8 are provided", bits);
        return fail(MIQMM_EINVAL, "bits must be 4 or 8, got %d", bits);
    }
    if (group_size != 32 && group_size != 64 && group_size != 128)
        return fail(MIQMM_EINVAL, "group_size must be 32, 64 or 128, got %d", group_size);
    if (N <= 0 || K <= 0 || N >= kMaxDim || K >= kMaxDim)
        return fail(MIQMM_EINVAL, "N and K must be in [1, 2^31), got N=%lld K=%lld", (long long)N, (long long)K);
    if (K > kMaxK)
        return fail(MIQMM_EINVAL, "K=%lld exceeds %lld (the kernels' 32-bit tile offsets)", (long long)K,
                    (long long)kMaxK);
    if (K % group_size != 0)
        return fail(MIQMM_EINVAL, "K=%lld is not a multiple of group_size=%d", (long long)K, group_size);
    if (sb_dtype != MIQMM_DT_BF16 && sb_dtype != MIQMM_DT_F16)
        return fail(MIQMM_ENOTSUP, "scales/biases dtype %d not supported (bf16=0, f16=1)", sb_dtype);
    return MIQMM_OK;
}

int check_launch(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(MIQMM_EHIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

// Measured on MI355X (4-bit g64 unless noted, cold weights):
//   M <= 4: the K-sliced GEMV wherever it takes the shape (rows of at most 15
//          KiB of codes, 8 KiB with more than two rows of x; an even number of
//          groups; 4-byte aligned scales and biases): each row of codes is
//          unpacked once for every row of x and dotted on v_dot2.  M = 1:
//          4096 -> 14336 8.4 us against 8.6 for v_dot2, rows of 33-63 chunks
//          (1536 -> 4096) 2.98 against 3.75, the 896 -> 151936 head 14.3
//          against 17.9 for the LDS-staged MFMA GEMV; M = 2: 4096 -> 14336 9.8
//          against 12.3 (LDS-staged MFMA), 896 -> 4864 2.99 against 3.6; M = 3
//          / 4: 4096 -> 6144 7.3 / 7.7 against 9.1 / 9.0 (LDS-staged MFMA),
//          4096 -> 14336 12.1 / 12.5 against 13.0 / 13.1 (group-diagonal
//          MFMA); 8-bit, M = 4, 4096 -> 14336: 15.0 against 25.7;
//   M = 1, other shapes: the v_dot2 GEMV, except for many-row heads with K <=
//          2048, where the LDS-staged MFMA GEMV wins;
//   2 <= M <= 4, other shapes: the LDS-staged MFMA GEMV when it supports the
//          shape (min(M, 4) K <= 32768), except at M = 3 and 4 with N >= 8192,
//          where the group-diagonal MFMA GEMV is faster; rows the LDS-staged
//          GEMV does not take go to the group-diagonal one too;
//   5 <= M <= 16: the group-diagonal MFMA GEMV, whose cost barely grows with M;
//   17 <= M <= 32 (64 for rows of K >= 8192): the GEMVs in passes of 16 rows
//          of x (the last pass routed by its own rows), against 256-row tiles
//          of the tiled matmul that are mostly empty: M = 17 / 32, 4096 ->
//          14336 33.3 / 34.9 -> 23.7 / 30.5 us, 14336 -> 4096 63.3 / 64.0 ->
//          22.1 / 28.3, 4096 -> 4096 24.0 / 24.3 -> 13.5 / 18.2; at M = 48
//          three passes lose to the tiled matmul at K = 4096 (about 45
//          against 36.4 and 27.6 against 24.5 us) and win on 14336 -> 4096
//          (about 43 against 64.0);
//   larger M: the tiled MFMA matmul.
constexpr int64_t kGemvRows = 16;  // rows of x per pass of the GEMVs

// the largest M the auto route gives the GEMVs (in passes of 16 rows)
int64_t gemv_max_m(int64_t K) { return K >= 8192 ? 64 : 32; }

int auto_route(int64_t M, int64_t N, int64_t K, int group_size, int bits, bool sb_aligned4 = true) {
    if (M <= 4 && sb_aligned4 && miqmm::qmvs_supported(M, N, K, bits, group_size)) return MIQMM_ROUTE_QMVS;
    if (M == 1) {
        const bool wide_head = N >= 65536 && K <= 2048 && miqmm::qmvx_supported(M, K, group_size);
        return wide_head ? MIQMM_ROUTE_QMVX : MIQMM_ROUTE_QMV_DOT;
    }
    if (M <= 4 && miqmm::qmvx_supported(M, K, group_size) && !(M >= 3 && N >= 8192)) return MIQMM_ROUTE_QMVX;
    if (M <= 4 && (K / group_size) % 2 != 0) return MIQMM_ROUTE_QMV_DOT;
    return M <= gemv_max_m(K) ? MIQMM_ROUTE_QMV : MIQMM_ROUTE_QMM;
}

// argument checks shared by the single and grouped entry points; MIQMM_OK
// with *noop set when M == 0
int check_args(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases, int64_t M,
               int64_t N, int64_t K, int transpose, int group_size, int bits, int x_dtype, int sb_dtype,
               int y_dtype, int route, bool* noop) {
    *noop = false;
    if (!transpose)
        return fail(MIQMM_ENOTSUP, "transpose=false is not provided (every live call site uses transpose=true)");
    int st = check_quant(N, K, group_size, bits, sb_dtype);
    if (st != MIQMM_OK) return st;
    if (M < 0 || M >= kMaxDim) return fail(MIQMM_EINVAL, "M must be in [0, 2^31), got %lld", (long long)M);
    if (x_dtype != MIQMM_DT_BF16) return fail(MIQMM_ENOTSUP, "x dtype %d not supported (bf16=0)", x_dtype);
    if (y_dtype != MIQMM_DT_BF16 && y_dtype != MIQMM_DT_F16 && y_dtype != MIQMM_DT_F32)
        return fail(MIQMM_EINVAL, "y dtype %d invalid", y_dtype);
    if (route != MIQMM_ROUTE_AUTO && route != MIQMM_ROUTE_QMV && route != MIQMM_ROUTE_QMM &&
        route != MIQMM_ROUTE_QMV_DOT && route != MIQMM_ROUTE_QMVX && route != MIQMM_ROUTE_QMVS)
        return fail(MIQMM_EINVAL, "route %d invalid", route);
    if (route == MIQMM_ROUTE_QMVS && M > 4)
        return fail(MIQMM_ENOTSUP, "route qmvs takes one to four rows of x (M <= 4)");
    if (route == MIQMM_ROUTE_QMVS && !miqmm::qmvs_supported(M > 1 ? M : 1, N, K, bits, group_size))
        return fail(MIQMM_ENOTSUP,
                    "route qmvs needs K*bits/8 <= 15 KiB (8 KiB with more than two rows of x) and an even "
                    "K/group_size");
    if (route == MIQMM_ROUTE_QMVS && M > 0 && (!aligned4(scales) || !aligned4(biases)))
        return fail(MIQMM_ENOTSUP, "route qmvs needs 4-byte aligned scales and biases");
    if (route == MIQMM_ROUTE_QMVX && !miqmm::qmvx_supported(M < 4 ? M : 4, K, group_size))
        return fail(MIQMM_ENOTSUP, "route qmvx needs K/group_size even and min(M,4)*K <= 32768");
    if (M == 0) {
        *noop = true;
        return ok();
    }
    if (!y || !x || !w || !scales || !biases) return fail(MIQMM_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(w))
        return fail(MIQMM_EINVAL, "x and w must be 16-byte aligned");
    if (M * K >= ((int64_t)1 << 40) || M * N >= ((int64_t)1 << 40))
        return fail(MIQMM_EINVAL, "M*K or M*N too large");
    return ok();
}

// workspace: fp32 partials for the tiled matmul's k split (nullptr / 0 bytes:
// the plan never splits)
int qmm_common(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
               const void* bias, int64_t M, int64_t N, int64_t K, int transpose, int group_size,
               int bits, int x_dtype, int sb_dtype, int y_dtype, int route, void* stream,
               void* workspace = nullptr, int64_t workspace_bytes = 0) {
    bool noop;
    int st = check_args(y, x, w, scales, biases, M, N, K, transpose, group_size, bits, x_dtype, sb_dtype, y_dtype,
                        route, &noop);
    if (st != MIQMM_OK || noop) return st;

    miqmm::QmmArgs a{y, x, w, scales, biases, bias, M, N, K, group_size, bits, x_dtype, sb_dtype, y_dtype,
                     reinterpret_cast<hipStream_t>(stream)};
    const bool sb4 = aligned4(scales) && aligned4(biases);
    const bool automatic = route == MIQMM_ROUTE_AUTO;
    if (automatic) route = auto_route(M, N, K, group_size, bits, sb4);
    if (route == MIQMM_ROUTE_QMVS) return check_launch(miqmm::launch_qmvs(a), "qmvs launch");
    if (route == MIQMM_ROUTE_QMV || route == MIQMM_ROUTE_QMV_DOT || route == MIQMM_ROUTE_QMVX) {
        // the GEMV kernels handle at most 16 (qmvx: 4) rows of x per pass over
        // W; passes run in order on the stream, so the split GEMV's partials
        // reuse one workspace; with the route chosen here each pass takes the
        // route of its own rows (the last pass at M > 16 may be a few rows)
        const int64_t step = route == MIQMM_ROUTE_QMVX ? 4 : kGemvRows;
        for (int64_t m0 = 0; m0 < M; m0 += step) {
            miqmm::QmmArgs part = a;
            const int64_t mm = M - m0 < step ? M - m0 : step;
            part.M = mm;
            part.x = static_cast<const uint16_t*>(x) + m0 * K;
            const int ysz = y_dtype == MIQMM_DT_F32 ? 4 : 2;
            part.y = static_cast<char*>(y) + m0 * N * ysz;
            const int r = automatic && mm < M ? auto_route(mm, N, K, group_size, bits, sb4) : route;
            st = r == MIQMM_ROUTE_QMV    ? check_launch(miqmm::launch_qmv_mfma_split(part, workspace,
                                                                                     workspace_bytes),
                                                        "qmv launch")
                 : r == MIQMM_ROUTE_QMVS ? check_launch(miqmm::launch_qmvs(part), "qmvs launch")
                 : r == MIQMM_ROUTE_QMVX ? check_launch(miqmm::launch_qmvx(part), "qmvx launch")
                                         : check_launch(miqmm::launch_qmv(part), "qmv_dot launch");
            if (st != MIQMM_OK) return st;
        }
        return ok();
    }
    return check_launch(miqmm::launch_qmm(a, workspace, workspace_bytes), "qmm launch");
}

// bytes of k-split partials the auto route takes for a shape (0: none)
int64_t split_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
    const int route = auto_route(M, N, K, group_size, bits);
    if (route != MIQMM_ROUTE_QMM && route != MIQMM_ROUTE_QMV) return 0;
    miqmm::QmmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.group_size = group_size;
    a.bits = bits;
    if (route == MIQMM_ROUTE_QMM) return miqmm::qmm_workspace_bytes(a);
    // passes of 16 rows (one workspace, reused in order): the largest need
    int64_t need = 0;
    for (int64_t m0 = 0; m0 < M; m0 += kGemvRows) {
        a.M = M - m0 < kGemvRows ? M - m0 : kGemvRows;
        if (a.M < M && auto_route(a.M, N, K, group_size, bits) != MIQMM_ROUTE_QMV) continue;
        const int64_t n = miqmm::qmv_split_bytes(a);
        need = n > need ? n : need;
    }
    return need;
}



// gather_qmm: validation, then the expert-grouped tiled matmul when a
// workspace is given and there are enough selections per expert to fill its
// M tiles, else the per-selection v_dot2 GEMV
int gather_common(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                  const int32_t* rhs_indices, int64_t batch, int64_t top_k, int x_per_index, int64_t M, int64_t N,
                  int64_t K, int64_t experts, int transpose, int group_size, int bits, int x_dtype, int sb_dtype,
                  int y_dtype, int sorted_indices, void* workspace, int64_t workspace_bytes, void* stream) {
    (void)sorted_indices;  // a scheduling hint only: every order gives the same result here
    if (batch < 0 || top_k < 0 || batch >= kMaxDim || top_k >= kMaxDim)
        return fail(MIQMM_EINVAL, "batch and top_k must be in [0, 2^31), got %lld and %lld", (long long)batch,
                    (long long)top_k);
    if (experts <= 0 || experts >= kMaxDim)
        return fail(MIQMM_EINVAL, "experts must be in [1, 2^31), got %lld", (long long)experts);
    if (x_per_index != 0 && x_per_index != 1) return fail(MIQMM_EINVAL, "x_per_index must be 0 or 1");
    if (workspace_bytes < 0) return fail(MIQMM_EINVAL, "workspace_bytes must be >= 0");
    const int64_t problems = batch * top_k;
    bool noop;  // no selections or no rows: nothing to read, pointers may be null
    int st = check_args(y, x, w, scales, biases, problems == 0 ? 0 : M, N, K, transpose, group_size, bits, x_dtype,
                        sb_dtype, y_dtype, MIQMM_ROUTE_AUTO, &noop);
    if (st != MIQMM_OK || noop) return st;
    if (!rhs_indices) return fail(MIQMM_EINVAL, "null pointer argument");
    if (problems * M * (K > N ? K : N) >= ((int64_t)1 << 40)) return fail(MIQMM_EINVAL, "batch*top_k*M*K too large");
    const int64_t x_bytes = (x_per_index ? problems : batch) * M * K * 2;
    // with a workspace and one row of x per selection, the selections are
    // grouped by expert so each selected expert's weights stream once: on the
    // tiled MFMA matmul when there are many selections per expert, on the
    // MFMA GEMV (16 selections per tile) from 4 selections per expert
    if (workspace && M == 1 && problems >= kGroupedGemvMinPerExpert * experts && experts <= 1024 &&
        x_bytes < ((int64_t)1 << 31) && workspace_bytes >= miqmm::gather_grouped_workspace(problems, experts)) {
        if (!aligned16(workspace)) return fail(MIQMM_EINVAL, "workspace must be 16-byte aligned");
        miqmm::QmmArgs a{y, x, w, scales, biases, nullptr, problems, N, K, group_size, bits, x_dtype, sb_dtype,
                         y_dtype, reinterpret_cast<hipStream_t>(stream)};
        if (problems >= kGroupedMinPerExpert * experts)
            return check_launch(miqmm::launch_gather_grouped(a, rhs_indices, batch, (int)top_k, x_per_index,
                                                              experts, x_bytes, workspace),
                                "grouped gather launch");
        return check_launch(miqmm::launch_gather_gemv(a, rhs_indices, batch, (int)top_k, x_per_index, experts,
                                                       x_bytes, workspace),
                            "grouped gather GEMV launch");
    }
    // the GEMV handles 16 rows of x per pass over a weight tile; more rows
    // (rare in decode) take several passes, one per 16-row slice of every matrix
    const int ysz = y_dtype == MIQMM_DT_F32 ? 4 : 2;
    for (int64_t m0 = 0; m0 < M; m0 += 16) {
        miqmm::QmmArgs a{static_cast<char*>(y) + m0 * N * ysz, static_cast<const uint16_t*>(x) + m0 * K, w, scales,
                         biases, nullptr, M - m0 < 16 ? M - m0 : 16, N, K, group_size, bits, x_dtype, sb_dtype,
                         y_dtype, reinterpret_cast<hipStream_t>(stream)};
        st = check_launch(
            miqmm::launch_qmv_gather(a, rhs_indices, batch, (int)top_k, x_per_index, experts, M * K, M * N),
            "gather qmv launch");
        if (st != MIQMM_OK) return st;
    }
    return ok();
}

// Scratch of miqmm_quantized_matmul_noalloc: the tiled matmul's k-split
// partials, in device memory the code object holds (each GPU the library
// runs on has its own copy, kept until the process ends).  Its address on a
// device comes from hipGetSymbolAddress, once per device, with the device
// current; host code uses only that address.
constexpr int64_t kNoallocScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) char scratch[kNoallocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];  // per device id, set once under g_scratch_mu

int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MIQMM_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return fail(MIQMM_EINVAL, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail(MIQMM_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MIQMM_OK;
}

}  // namespace

extern "C" {

int miqmm_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                           int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                           void* stream) {
    return qmm_common(y, x, w, scales, biases, nullptr, M, N, K, transpose, group_size, bits, x_dtype,
                      sb_dtype, y_dtype, MIQMM_ROUTE_AUTO, stream);
}

int miqmm_quantized_matmul_ex(void* y, const void* x, const uint32_t* w, const void* scales,
                              const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                              int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                              int route, void* stream) {
    return qmm_common(y, x, w, scales, biases, nullptr, M, N, K, transpose, group_size, bits, x_dtype,
                      sb_dtype, y_dtype, route, stream);
}

int miqmm_quantized_linear(void* y, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                           int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                           void* stream) {
    return qmm_common(y, x, w, scales, biases, bias, M, N, K, 1, group_size, bits, x_dtype, sb_dtype,
                      y_dtype, MIQMM_ROUTE_AUTO, stream);
}

int miqmm_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                          int64_t* bytes) {
    if (!bytes) return fail(MIQMM_EINVAL, "null pointer argument");
    int st = check_quant(N, K, group_size, bits, MIQMM_DT_BF16);
    if (st != MIQMM_OK) return st;
    if (M < 0 || M >= kMaxDim) return fail(MIQMM_EINVAL, "M must be in [0, 2^31), got %lld", (long long)M);
    *bytes = M == 0 ? 0 : split_workspace_bytes(M, N, K, group_size, bits);
    return ok();
}

int miqmm_quantized_matmul_ws(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                              const void* bias, int64_t M, int64_t N, int64_t K, int transpose, int group_size,
                              int bits, int x_dtype, int sb_dtype, int y_dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
    if (workspace_bytes < 0) return fail(MIQMM_EINVAL, "workspace_bytes must be >= 0");
    if (workspace && !aligned16(workspace)) return fail(MIQMM_EINVAL, "workspace must be 16-byte aligned");
    return qmm_common(y, x, w, scales, biases, bias, M, N, K, transpose, group_size, bits, x_dtype, sb_dtype,
                      y_dtype, MIQMM_ROUTE_AUTO, stream, workspace, workspace ? workspace_bytes : 0);
}

int miqmm_quantized_matmul_grouped(const miqmm_problem* problems, int count, int64_t M, int64_t K,
                                   int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                                   void* stream) {
    if (count < 0 || (count > 0 && !problems)) return fail(MIQMM_EINVAL, "problems must hold count >= 0 entries");
    // decode-sized projections (M <= 2, none of them a wide head) run as one
    // grouped GEMV launch per four (the K-sliced GEMV when they are stored
    // contiguously, else the v_dot2 GEMV): at these sizes the launches are
    // latency-bound, so fewer of them beat a faster per-shape route
    bool grouped = M >= 1 && M <= 2;
    for (int i = 0; i < count; ++i) {
        const miqmm_problem& p = problems[i];
        bool noop;
        const int st = check_args(p.y, p.x, p.w, p.scales, p.biases, M, p.N, K, 1, group_size, bits, x_dtype,
                                  sb_dtype, y_dtype, MIQMM_ROUTE_AUTO, &noop);
        if (st != MIQMM_OK) return st;
        if (p.N >= 65536) grouped = false;
    }
    if (M == 0 || count == 0) return ok();
    if (!grouped) {  // one call per problem on its own route
        for (int i = 0; i < count; ++i) {
            const miqmm_problem& p = problems[i];
            const int st = qmm_common(p.y, p.x, p.w, p.scales, p.biases, p.bias, M, p.N, K, 1, group_size, bits,
                                      x_dtype, sb_dtype, y_dtype, MIQMM_ROUTE_AUTO, stream);
            if (st != MIQMM_OK) return st;
        }
        return ok();
    }
    miqmm::QmmArgs a[miqmm::kMaxGroup];
    // one row of x and problems stored one after another (fused at load),
    // with rows the K-sliced GEMV takes: one launch over all their rows
    if (M == 1 && count <= miqmm::kMaxGroup &&
        aligned4(problems[0].scales) && aligned4(problems[0].biases)) {
        for (int i = 0; i < count; ++i) {
            const miqmm_problem& p = problems[i];
            a[i] = miqmm::QmmArgs{p.y, p.x, p.w, p.scales, p.biases, p.bias, M, p.N, K, group_size, bits,
                                  x_dtype, sb_dtype, y_dtype, reinterpret_cast<hipStream_t>(stream)};
        }
        if (miqmm::qmvs_group_ok(a, count))
            return check_launch(miqmm::launch_qmvs_grouped(a, count), "grouped qmvs launch");
    }
    // a problem that the GEMV alone would run with K split over a block's
    // waves is launched alone, so that every result equals the v_dot2 route
    // on that problem bit for bit (the split changes the order of the sums)
    int n = 0;
    for (int i = 0; i <= count; ++i) {
        if (i < count) {
            const miqmm_problem& p = problems[i];
            const miqmm::QmmArgs q{p.y, p.x, p.w, p.scales, p.biases, p.bias, M, p.N, K, group_size, bits,
                                   x_dtype, sb_dtype, y_dtype, reinterpret_cast<hipStream_t>(stream)};
            if (miqmm::qmv_ksplit(M, p.N, K, bits)) {
                const int st = check_launch(miqmm::launch_qmv(q), "qmv_dot launch");
                if (st != MIQMM_OK) return st;
                continue;
            }
            a[n++] = q;
        }
        if (n == miqmm::kMaxGroup || (i == count && n > 0)) {
            const int st = check_launch(miqmm::launch_qmv_grouped(a, n), "grouped qmv_dot launch");
            if (st != MIQMM_OK) return st;
            n = 0;
        }
    }
    return ok();
}

int miqmm_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                     const int32_t* rhs_indices, int64_t batch, int64_t top_k, int x_per_index, int64_t M,
                     int64_t N, int64_t K, int64_t experts, int transpose, int group_size, int bits, int x_dtype,
                     int sb_dtype, int y_dtype, int sorted_indices, void* stream) {
    return gather_common(y, x, w, scales, biases, rhs_indices, batch, top_k, x_per_index, M, N, K, experts, transpose,
                         group_size, bits, x_dtype, sb_dtype, y_dtype, sorted_indices, nullptr, 0, stream);
}

int miqmm_gather_qmm_workspace_size(int64_t batch, int64_t top_k, int64_t experts, int64_t* bytes) {
    if (!bytes) return fail(MIQMM_EINVAL, "null pointer argument");
    if (batch < 0 || top_k < 0 || experts <= 0 || batch >= kMaxDim || top_k >= kMaxDim || experts >= kMaxDim)
        return fail(MIQMM_EINVAL, "batch, top_k and experts out of range");
    *bytes = miqmm::gather_grouped_workspace(batch * top_k, experts);
    return ok();
}

int miqmm_gather_qmm_ws(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                        const int32_t* rhs_indices, int64_t batch, int64_t top_k, int x_per_index, int64_t M,
                        int64_t N, int64_t K, int64_t experts, int transpose, int group_size, int bits, int x_dtype,
                        int sb_dtype, int y_dtype, int sorted_indices, void* workspace, int64_t workspace_bytes,
                        void* stream) {
    return gather_common(y, x, w, scales, biases, rhs_indices, batch, top_k, x_per_index, M, N, K, experts, transpose,
                         group_size, bits, x_dtype, sb_dtype, y_dtype, sorted_indices, workspace, workspace_bytes,
                         stream);
}

int miqmm_quantized_matmul_noalloc(void* y, const void* x, const uint32_t* w, const void* scales,
                                   const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                                   int transpose, int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                                   void* stream) {
    bool noop;
    int st = check_args(y, x, w, scales, biases, M, N, K, transpose, group_size, bits, x_dtype, sb_dtype, y_dtype,
                        MIQMM_ROUTE_AUTO, &noop);
    if (st != MIQMM_OK || noop) return st;
    const int64_t need = split_workspace_bytes(M, N, K, group_size, bits);
    if (need > kNoallocScratchBytes)
        return fail(MIQMM_EINVAL,
                    "M=%lld N=%lld K=%lld needs %lld bytes of k-split scratch, more than the %lld this entry "
                    "point holds; use miqmm_quantized_matmul_ws",
                    (long long)M, (long long)N, (long long)K, (long long)need, (long long)kNoallocScratchBytes);
    void* ptr = nullptr;
    if (need > 0) {
        st = scratch_address(&ptr);
        if (st != MIQMM_OK) return st;
    }
    return qmm_common(y, x, w, scales, biases, bias, M, N, K, transpose, group_size, bits, x_dtype, sb_dtype,
                      y_dtype, MIQMM_ROUTE_AUTO, stream, ptr, need > 0 ? kNoallocScratchBytes : 0);
}

int miqmm_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                     int64_t N, int64_t K, int group_size, int bits, int sb_dtype, int out_dtype,
                     void* stream) {
    int st = check_quant(N, K, group_size, bits, sb_dtype);
    if (st != MIQMM_OK) return st;
    if (out_dtype != MIQMM_DT_BF16 && out_dtype != MIQMM_DT_F16 && out_dtype != MIQMM_DT_F32)
        return fail(MIQMM_EINVAL, "out dtype %d invalid", out_dtype);
    if (!out || !w || !scales || !biases) return fail(MIQMM_EINVAL, "null pointer argument");
    return check_launch(miqmm::launch_dequantize(out, w, scales, biases, N, K, group_size, bits, sb_dtype,
                                                 out_dtype, reinterpret_cast<hipStream_t>(stream)),
                        "dequantize launch");
}

int miqmm_quantized_embedding(void* out, const int32_t* ids, int64_t T, const uint32_t* w, const void* scales,
                              const void* biases, int64_t V, int64_t K, int group_size, int bits, int sb_dtype,
                              int out_dtype, void* stream) {
    int st = check_quant(V, K, group_size, bits, sb_dtype);
    if (st != MIQMM_OK) return st;
    if (out_dtype != MIQMM_DT_BF16 && out_dtype != MIQMM_DT_F16 && out_dtype != MIQMM_DT_F32)
        return fail(MIQMM_EINVAL, "out dtype %d invalid", out_dtype);
    if (T < 0 || T >= kMaxDim) return fail(MIQMM_EINVAL, "T must be in [0, 2^31), got %lld", (long long)T);
    if (T == 0) return ok();
    if (!out || !ids || !w || !scales || !biases) return fail(MIQMM_EINVAL, "null pointer argument");
    if (!aligned16(w) || !aligned16(out)) return fail(MIQMM_EINVAL, "w and out must be 16-byte aligned");
    if (T * K >= ((int64_t)1 << 40)) return fail(MIQMM_EINVAL, "T*K too large");
    return check_launch(miqmm::launch_embedding(out, ids, T, w, scales, biases, V, K, group_size, bits, sb_dtype,
                                                out_dtype, reinterpret_cast<hipStream_t>(stream)),
                        "embedding launch");
}

int miqmm_unpack(uint8_t* codes, const uint32_t* w, int64_t N, int64_t K, int bits, void* stream) {
    if (bits != 4 && bits != 8) return fail(MIQMM_EINVAL, "bits must be 4 or 8, got %d", bits);
    if (N <= 0 || K <= 0 || K % 32 != 0) return fail(MIQMM_EINVAL, "need N > 0 and K > 0 with K %% 32 == 0");
    if (!codes || !w) return fail(MIQMM_EINVAL, "null pointer argument");
    return check_launch(miqmm::launch_unpack(codes, w, N, K, bits, reinterpret_cast<hipStream_t>(stream)),
                        "unpack launch");
}

int miqmm_query_route(int64_t M, int64_t N, int64_t K, int group_size, int bits, int* route_out,
                      int* tile_out) {
    int st = check_quant(N, K, group_size, bits, MIQMM_DT_BF16);
    if (st != MIQMM_OK) return st;
    if (M < 0) return fail(MIQMM_EINVAL, "M must be >= 0");
    miqmm::QmmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.group_size = group_size;
    a.bits = bits;
    const int route = M == 0 ? MIQMM_ROUTE_QMV_DOT : auto_route(M, N, K, group_size, bits);
    if (route_out) *route_out = route;
    if (tile_out) {
        tile_out[0] = tile_out[1] = tile_out[2] = tile_out[3] = 0;
        if (route == MIQMM_ROUTE_QMV) {  // the first pass's launch (16 rows of x at M > 16)
            a.M = M < kGemvRows ? M : kGemvRows;
            miqmm::qmv_mfma_config(a, &tile_out[0], &tile_out[1], &tile_out[2]);
        }
        else if (route == MIQMM_ROUTE_QMVX) miqmm::qmvx_config(a, &tile_out[0], &tile_out[1], &tile_out[2]);
        else if (route == MIQMM_ROUTE_QMV_DOT) miqmm::qmv_config(a, &tile_out[0], &tile_out[1], &tile_out[2]);
        else if (route == MIQMM_ROUTE_QMVS) miqmm::qmvs_config(a, &tile_out[0], &tile_out[1], &tile_out[2]);
        else miqmm::qmm_config(a, &tile_out[0], &tile_out[1], &tile_out[2], &tile_out[3]);
    }
    return ok();
}

int miqmm_synth_problem(void* x, uint32_t* w, void* scales, void* biases, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int x_dtype, int sb_dtype,
                        uint64_t seed, uint64_t stream_id, void* stream) {
    int st = check_quant(N, K, group_size, bits, sb_dtype);
    if (st != MIQMM_OK) return st;
    if (x_dtype != MIQMM_DT_BF16 && x_dtype != MIQMM_DT_F16)
        return fail(MIQMM_EINVAL, "x dtype %d invalid", x_dtype);
    if (M < 0) return fail(MIQMM_EINVAL, "M must be >= 0");
    if ((scales == nullptr) != (biases == nullptr))
        return fail(MIQMM_EINVAL, "scales and biases are generated together");
    return check_launch(miqmm::launch_synth(x, w, scales, biases, M, N, K, group_size, bits, x_dtype, sb_dtype,
                                            seed, stream_id, reinterpret_cast<hipStream_t>(stream)),
                        "synth launch");
}

int miqmm_stream_read(const void* p, int64_t bytes, void* sink, void* stream) {
    if (!p || !sink) return fail(MIQMM_EINVAL, "null pointer argument");
    if (!aligned16(p) || bytes <= 0 || bytes % 16384 != 0 || bytes >= ((int64_t)1 << 31))
        return fail(MIQMM_EINVAL, "p must be 16-byte aligned and bytes a multiple of 16384 below 2^31");
    return check_launch(miqmm::launch_stream_read(p, bytes, sink, reinterpret_cast<hipStream_t>(stream)),
                        "stream read launch");
}

const char* miqmm_last_error(void) { return g_last_error.c_str(); }

const char* miqmm_version(void) { return "miqmm 0.1.0 gfx950"; }

}  // extern "C"
