// qmv.hip -- small-M route (M = 1..16) of affine group-quantized matmul.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])      (transpose=true)
//
// The operator is MLX's quantized_matmul as called from the reference's
// quantized projections (src/engine/mlx_lm/utils/mod.rs:70-78,
// src/engine/mlx_lm/models/llama.rs:195-197,249,293-294) during decode, where
// x is one token (M=1) or a handful of speculative/batched rows.
//
// HBM-bound design (no MFMA): a wave owns RPS output rows n; lane l streams the
// 16-byte chunks l, l+64, ... of each of those rows, so every load instruction
// of the wave reads 1 KiB of one row contiguously.  A chunk holds 32 (4-bit)
// or 16 (8-bit) codes and always lies inside one quantization group, so its
// scale and bias are two scalars per row.  Codes become exact bf16 operands
// (4-bit: 0x4300|q = 128+q; 8-bit: top half of the fp32 value) and are dotted
// with x by v_dot2_f32_bf16 in fp32.  Per chunk the dequant is applied in
// factorised form, exactly:
//     sum_k x_k (s q_k + b) = s * sum_k x_k (q_k + c) + (b - c s) * sum_k x_k
// with c = 128 for 4-bit, 0 for 8-bit.  The 64 lane partials of each output
// are summed with a butterfly across the wave.
#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int BITS, int SBT, int MT, int RPS>
__global__ __launch_bounds__(256) void qmv_kernel(const uint16_t* __restrict__ x,
                                                  const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ sc,
                                                  const uint16_t* __restrict__ bi,
                                                  void* __restrict__ y, const void* __restrict__ bias,
                                                  int M, int N, int K, int gs_shift, int y_dtype) {
    constexpr int CPC_SHIFT = BITS == 4 ? 5 : 4;  // codes per 16-byte chunk: 32 or 16
    constexpr int CPC = 1 << CPC_SHIFT;
    constexpr int NP = CPC / 2;                   // bf16 pairs per chunk
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPS;
    if (row0 >= N) return;  // wave-uniform
    const int C = K >> CPC_SHIFT;
    const int64_t KW = (int64_t)K * BITS / 32;
    const int G = K >> gs_shift;

    const uint32_t* wrow[RPS];
    int64_t srow[RPS];
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
        const int n = min(row0 + r, N - 1);
        wrow[r] = w + (int64_t)n * KW;
        srow[r] = (int64_t)n * G;
    }

    float acc[RPS][MT];
#pragma unroll
    for (int r = 0; r < RPS; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    // one chunk of prefetch: the next chunk's codes are in flight while the
    // current one is computed
    u32x4_t qn[RPS];
    int c = lane;
    if (c < C) {
#pragma unroll
        for (int r = 0; r < RPS; ++r) qn[r] = ldg16(wrow[r] + c * 4);
    }
    for (; c < C; c += 64) {
        u32x4_t q[RPS];
#pragma unroll
        for (int r = 0; r < RPS; ++r) q[r] = qn[r];
        if (c + 64 < C) {
#pragma unroll
            for (int r = 0; r < RPS; ++r) qn[r] = ldg16(wrow[r] + (c + 64) * 4);
        }
        const int g = (c << CPC_SHIFT) >> gs_shift;
        float s[RPS], bb[RPS];
#pragma unroll
        for (int r = 0; r < RPS; ++r) {
            s[r] = half_to_f32<SBT>(sc[srow[r] + g]);
            bb[r] = half_to_f32<SBT>(bi[srow[r] + g]);
            if constexpr (BITS == 4) bb[r] = fmaf(-128.f, s[r], bb[r]);
        }
        uint32_t p[RPS][NP];
#pragma unroll
        for (int r = 0; r < RPS; ++r)
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                if constexpr (BITS == 4) unpack4_magic(q[r][wi], &p[r][wi * 4]);
                else unpack8_pairs(q[r][wi], &p[r][wi * 2]);
            }
        const uint16_t* xc = x + (int64_t)c * CPC;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                uint32_t xw[NP];
#pragma unroll
                for (int i = 0; i < NP / 4; ++i) {
                    u32x4_t v = ldg16(xc + (int64_t)m * K + i * 8);
                    xw[4 * i + 0] = v[0];
                    xw[4 * i + 1] = v[1];
                    xw[4 * i + 2] = v[2];
                    xw[4 * i + 3] = v[3];
                }
                float xs = 0.f;
#pragma unroll
                for (int i = 0; i < NP; ++i) xs = dot2(xw[i], kOnesBf16x2, xs);
                uint32_t X[NP];
                if constexpr (BITS == 4) {
#pragma unroll
                    for (int wi = 0; wi < 4; ++wi) perm_x_for4(&xw[4 * wi], &X[4 * wi]);
                } else {
#pragma unroll
                    for (int i = 0; i < NP; ++i) X[i] = xw[i];
                }
#pragma unroll
                for (int r = 0; r < RPS; ++r) {
                    float a = 0.f;
#pragma unroll
                    for (int i = 0; i < NP; ++i) a = dot2(X[i], p[r][i], a);
                    acc[r][m] = fmaf(s[r], a, acc[r][m]);
                    acc[r][m] = fmaf(bb[r], xs, acc[r][m]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < RPS; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float v = wave_sum(acc[r][m]);
            const int n = row0 + r;
            if (lane == ((r * MT + m) & 63) && m < M && n < N)
                store_out(y, (int64_t)m * N + n, y_dtype, v, bias, n);
        }
}

template <int BITS, int SBT, int MT, int RPS>
hipError_t launch_t(const QmmArgs& a) {
    const int rows_per_block = 4 * RPS;
    const int blocks = (int)((a.N + rows_per_block - 1) / rows_per_block);
    const int gs_shift = __builtin_ctz((unsigned)a.group_size);
    hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, RPS>), dim3(blocks), dim3(256), 0, a.stream,
                       (const uint16_t*)a.x, a.w, (const uint16_t*)a.scales,
                       (const uint16_t*)a.biases, a.y, a.bias, (int)a.M, (int)a.N, (int)a.K,
                       gs_shift, a.y_dtype);
    return hipGetLastError();
}

int pick_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// 4 rows per wave unless that leaves fewer than 2 blocks per CU on 256 CUs
int pick_rps(int64_t N) { return (N + 15) / 16 >= 512 ? 4 : 2; }

template <int BITS, int SBT, int MT>
hipError_t launch_rps(const QmmArgs& a) {
    return pick_rps(a.N) == 4 ? launch_t<BITS, SBT, MT, 4>(a) : launch_t<BITS, SBT, MT, 2>(a);
}

template <int BITS, int SBT>
hipError_t launch_mt(const QmmArgs& a) {
    switch (pick_mt(a.M)) {
        case 1: return launch_rps<BITS, SBT, 1>(a);
        case 2: return launch_rps<BITS, SBT, 2>(a);
        case 4: return launch_rps<BITS, SBT, 4>(a);
        case 8: return launch_rps<BITS, SBT, 8>(a);
        default: return launch_rps<BITS, SBT, 16>(a);
    }
}

}  // namespace

void qmv_config(const QmmArgs& a, int* rows_per_wave, int* m_tile) {
    if (rows_per_wave) *rows_per_wave = pick_rps(a.N);
    if (m_tile) *m_tile = pick_mt(a.M);
}

hipError_t launch_qmv(const QmmArgs& a) {
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_mt<4, DT_F16>(a) : launch_mt<4, DT_BF16>(a);
    return a.sb_dtype == DT_F16 ? launch_mt<8, DT_F16>(a) : launch_mt<8, DT_BF16>(a);
}

}  // namespace miqmm
