// qmm.hip -- large-M (prefill) route of affine group-quantized matmul on bf16 MFMA.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])      (transpose=true)
//
// Reached by the reference's quantized projections during chunked prefill
// (src/engine/mlx_lm/models/llama.rs:195-197,249,293-294 with x [1, L, K],
// L up to prefill_chunk; src/engine/mlx_native.rs:1918-1922,2094-2102).
//
// Block tile BM x BN x 64 (BM = 2*WM, BN = 2*WN), four waves in a 2x2 grid,
// each owning a WM x WN sub-tile computed with v_mfma_f32_32x32x16_bf16.  Per
// 64-wide k-step the block
//   - copies the x tile [BM, 64] bf16 into LDS unchanged,
//   - dequantizes the W tile [BN, 64] in fp32 (fma(s, q, b), the reference's
//     formula) and stores it to LDS as bf16, k-contiguous per output column,
// while the next k-step's x rows, packed codes, scales and biases are already
// in flight into registers.  LDS rows are padded to 72 bf16 (144 B) so the
// 16-byte fragment reads of eight consecutive rows hit disjoint banks.
#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

constexpr int kBK = 64;
constexpr int kLDK = kBK + 8;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// 16 bytes of 4-bit codes (32 codes) -> 32 bf16 of fma(s, q, b), natural k order
__device__ __forceinline__ void dequant_chunk4(const u32x4_t& q, float s, float b, u32x4_t out[4]) {
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const uint32_t lo = q[wi] & 0x0F0F0F0Fu;         // codes 0,2,4,6 of the word
        const uint32_t hi = (q[wi] >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
        out[wi][0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(lo), b),
                                 fmaf(s, ubyte_f32<0>(hi), b));
        out[wi][1] = pack_bf16x2(fmaf(s, ubyte_f32<1>(lo), b),
                                 fmaf(s, ubyte_f32<1>(hi), b));
        out[wi][2] = pack_bf16x2(fmaf(s, ubyte_f32<2>(lo), b),
                                 fmaf(s, ubyte_f32<2>(hi), b));
        out[wi][3] = pack_bf16x2(fmaf(s, ubyte_f32<3>(lo), b),
                                 fmaf(s, ubyte_f32<3>(hi), b));
    }
}

// 16 bytes of 8-bit codes (16 codes) -> 16 bf16 of fma(s, q, b)
__device__ __forceinline__ void dequant_chunk8(const u32x4_t& q, float s, float b, u32x4_t out[2]) {
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const uint32_t v = q[wi];
        out[wi >> 1][(wi & 1) * 2 + 0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(v), b),
                                                     fmaf(s, ubyte_f32<1>(v), b));
        out[wi >> 1][(wi & 1) * 2 + 1] = pack_bf16x2(fmaf(s, ubyte_f32<2>(v), b),
                                                     fmaf(s, ubyte_f32<3>(v), b));
    }
}

template <int BITS, int SBT, int WM, int WN>
__global__ __launch_bounds__(256) void qmm_kernel(const uint16_t* __restrict__ x,
                                                  const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ sc,
                                                  const uint16_t* __restrict__ bi,
                                                  void* __restrict__ y, const void* __restrict__ bias,
                                                  int M, int N, int K, int gs_shift, int y_dtype) {
    constexpr int BM = 2 * WM, BN = 2 * WN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int CPC_SHIFT = BITS == 4 ? 5 : 4;       // codes per 16-byte chunk
    constexpr int CPR = kBK >> CPC_SHIFT;              // code chunks per row per k-step
    constexpr int A_PER = BM * (kBK / 8) / 256;        // 16-byte x chunks per thread
    constexpr int W_PER = BN * CPR / 256;              // 16-byte code chunks per thread
    static_assert(A_PER >= 1 && W_PER >= 1, "tile too small for 256 threads");

    __shared__ __attribute__((aligned(16))) uint16_t sA[BM * kLDK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN * kLDK];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int KT = (K + kBK - 1) / kBK;
    const int64_t KW = (int64_t)K * BITS / 32;
    const int G = K >> gs_shift;

    u32x4_t ra[A_PER], rw[W_PER];
    float rs[W_PER], rb[W_PER];

    auto load_tile = [&](int kt) {
        const int kb = kt * kBK;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
            const int gm = m0 + row, k = kb + ch * 8;
            ra[i] = (gm < M && k < K) ? ldg16(x + (int64_t)gm * K + k) : u32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < W_PER; ++i) {
            const int idx = tid + 256 * i, row = idx / CPR, ch = idx % CPR;
            const int gn = n0 + row, kc = kb + (ch << CPC_SHIFT);
            const bool ok = gn < N && kc < K;
            const int gnc = min(gn, N - 1);
            rw[i] = ok ? ldg16(w + (int64_t)gn * KW + (kc * BITS) / 32) : u32x4_t{0, 0, 0, 0};
            const int64_t sidx = (int64_t)gnc * G + (min(kc, K - 1) >> gs_shift);
            rs[i] = ok ? half_to_f32<SBT>(sc[sidx]) : 0.f;
            rb[i] = ok ? half_to_f32<SBT>(bi[sidx]) : 0.f;
        }
    };

    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
            *reinterpret_cast<u32x4_t*>(&sA[row * kLDK + ch * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < W_PER; ++i) {
            const int idx = tid + 256 * i, row = idx / CPR, ch = idx % CPR;
            uint16_t* dst = &sB[row * kLDK + (ch << CPC_SHIFT)];
            if constexpr (BITS == 4) {
                u32x4_t o[4];
                dequant_chunk4(rw[i], rs[i], rb[i], o);
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(dst + j * 8) = o[j];
            } else {
                u32x4_t o[2];
                dequant_chunk8(rw[i], rs[i], rb[i], o);
#pragma unroll
                for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4_t*>(dst + j * 8) = o[j];
            }
        }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
    load_tile(0);
    for (int kt = 0; kt < KT; ++kt) {
        store_tile();
        __syncthreads();
        if (kt + 1 < KT) load_tile(kt + 1);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            bf16x8_t af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const bf16x8_t*>(
                    &sA[(wm * WM + i * 32 + frag_row) * kLDK + kk * 16 + frag_k]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const bf16x8_t*>(
                    &sB[(wn * WN + j * 32 + frag_row) * kLDK + kk * 16 + frag_k]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // D of a 32x32 MFMA: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int col = n0 + wn * WN + j * 32 + (lane & 31);
                if (row < M && col < N) store_out(y, (int64_t)row * N + col, y_dtype, acc[i][j][r], bias, col);
            }
}

constexpr int kWM = 64, kWN = 64;

template <int BITS, int SBT>
hipError_t launch_t(const QmmArgs& a) {
    const dim3 grid((unsigned)((a.N + 2 * kWN - 1) / (2 * kWN)), (unsigned)((a.M + 2 * kWM - 1) / (2 * kWM)));
    const int gs_shift = __builtin_ctz((unsigned)a.group_size);
    hipLaunchKernelGGL((qmm_kernel<BITS, SBT, kWM, kWN>), grid, dim3(256), 0, a.stream,
                       (const uint16_t*)a.x, a.w, (const uint16_t*)a.scales,
                       (const uint16_t*)a.biases, a.y, a.bias, (int)a.M, (int)a.N, (int)a.K,
                       gs_shift, a.y_dtype);
    return hipGetLastError();
}

}  // namespace

void qmm_config(const QmmArgs&, int* bm, int* bn, int* bk) {
    if (bm) *bm = 2 * kWM;
    if (bn) *bn = 2 * kWN;
    if (bk) *bk = kBK;
}

hipError_t launch_qmm(const QmmArgs& a) {
    if (a.bits == 4) return a.sb_dtype == DT_F16 ? launch_t<4, DT_F16>(a) : launch_t<4, DT_BF16>(a);
    return a.sb_dtype == DT_F16 ? launch_t<8, DT_F16>(a) : launch_t<8, DT_BF16>(a);
}

}  // namespace miqmm
