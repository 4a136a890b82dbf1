// ceilings.hip -- measured ceilings for the tiled matmul's (qmm.hip) M = 2048
// configuration on one MI355X, each part of its k-step alone:
//   mfma_regs  v_mfma_f32_32x32x16_bf16 with operands in registers: eight
//              waves per block, eight 32x32 accumulators per wave (the
//              matmul's 128 x 64 wave tile), one block per CU-slot;
//   mfma_lds   the same MFMAs fed from LDS as the matmul feeds them: per
//              16-wide k step a wave reads four A and two B fragments of
//              1 KiB (ds_read_b128) from tiles in the matmul's swizzled
//              layout, with one block barrier per 64-wide k-step;
//   x_stage    the x tile ring alone: per k-step 256 rows x 64 bf16 of x
//              copied HBM -> LDS with direct-to-LDS loads (32 per block),
//              three stages, one wait and barrier per k-step, over the
//              448 blocks and 64 k-steps of x[2048, 4096] -> N = 14336.
// and the compute of the two ways to apply the affine dequant, operands in
// registers (no x or W traffic):
//   dequant    the matmul's: per 64-wide k-step a wave's 32 MFMAs plus its
//              share of the W tile (32 codes per lane) dequantized in fp32,
//              fma(s, q, b), packed to bf16 and stored to LDS; eight waves;
//   exact      exact integer codes in the MFMA and the dequant applied to the
//              accumulators: per k-step (one group at g = 64) the 32 MFMAs
//              start from zero and the group's sums are folded into fp32
//              totals, tot += s_n D + b'_n X_m (256 fused multiply-adds per
//              lane, X_m the group sums of x read from LDS), the codes only
//              unpacked; the second accumulator set leaves room for one wave
//              per SIMD, four per block.
// Usage: ceilings [iterations]; prints one line per part.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#define CK(e)                                                                                   \
    do {                                                                                        \
        hipError_t _e = (e);                                                                    \
        if (_e != hipSuccess) {                                                                 \
            printf("HIP error %s at line %d\n", hipGetErrorString(_e), __LINE__);               \
            return 1;                                                                           \
        }                                                                                       \
    } while (0)

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kTM = 4, kTN = 2;        // 32x32 tiles per wave: 128 x 64
constexpr int kBM = 256, kBN = 256;    // block tile
constexpr int kSlice = 32;             // bytes per row of one 16-wide k-slice

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(kThreads) void mfma_regs(float* out, int iters) {
    const u32x4 av = {threadIdx.x * 0x10001u, 0x3f803f80u, 0x3f003f00u, threadIdx.x};
    const bf16x8 a = as_bf16x8(av), b = as_bf16x8(av ^ 0x00400040u);
    f32x16 acc[kTM * kTN];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t) acc[t] = f32x16{};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int t = 0; t < kTM * kTN; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[t], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[t][e];
    out[blockIdx.x * kThreads + threadIdx.x] = s;
}

// byte offset of the 16-byte half fk of row r in k-slice kk of an R-row tile:
// the halves swap when bit 3 of r is set, so 16 consecutive rows' reads cover
// the 64 banks once
__device__ __forceinline__ int lds_off(int R, int r, int kk, int fk) {
    return kk * R * kSlice + r * kSlice + ((fk ^ ((r >> 3) & 1)) << 4);
}

__global__ __launch_bounds__(kThreads) void mfma_lds(float* out, int iters) {
    __shared__ __attribute__((aligned(16))) char A[kBM * 64 * 2];
    __shared__ __attribute__((aligned(16))) char B[kBN * 64 * 2];
    for (int i = threadIdx.x; i < kBM * 64 * 2 / 16; i += kThreads) {
        reinterpret_cast<u32x4*>(A)[i] = u32x4{0x3f803f80u, (unsigned)i, 0x3f003f00u, 0x3e803e80u};
        reinterpret_cast<u32x4*>(B)[i] = u32x4{0x3f003f00u, 0x3f803f80u, (unsigned)i, 0x3e003e00u};
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int wm = wid / 4, wn = wid % 4;  // 2 x 4 waves
    const int r = lane & 31, fk = lane >> 5;
    f32x16 acc[kTM * kTN];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t) acc[t] = f32x16{};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8 af[kTM], bfr[kTN];
#pragma unroll
            for (int tm = 0; tm < kTM; ++tm)
                af[tm] = as_bf16x8(*reinterpret_cast<const u32x4*>(A + lds_off(kBM, wm * 128 + tm * 32 + r, kk, fk)));
#pragma unroll
            for (int tn = 0; tn < kTN; ++tn)
                bfr[tn] = as_bf16x8(*reinterpret_cast<const u32x4*>(B + lds_off(kBN, wn * 64 + tn * 32 + r, kk, fk)));
#pragma unroll
            for (int tm = 0; tm < kTM; ++tm)
#pragma unroll
                for (int tn = 0; tn < kTN; ++tn)
                    acc[tm * kTN + tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bfr[tn], acc[tm * kTN + tn],
                                                                                0, 0, 0);
        }
        __syncthreads();  // the matmul's one barrier per k-step
    }
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[t][e];
    out[blockIdx.x * kThreads + threadIdx.x] = s;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// x[M, K] bf16; block (bx, by) stages rows 256 by .. of every k-step
__global__ __launch_bounds__(kThreads) void x_stage(const unsigned short* x, int M, int K, float* out) {
    constexpr int XST = 3, STAGE = kBM * 64 * 2;
    extern __shared__ __attribute__((aligned(16))) char ring[];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int m0 = blockIdx.y * kBM;
    const auto xr = make_rsrc(x + (size_t)m0 * K, (unsigned)(kBM * K * 2));
    const int slice = wid & 3, row0 = (wid >> 2) * 128;  // wave: one k-slice, 128 rows (4 x 32)
    const int KT = K / 64;
    auto issue = [&](int kt) {
        char* dst = ring + (kt % XST) * STAGE + slice * kBM * kSlice + row0 * kSlice;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = row0 + j * 32 + (lane >> 1);
            const int half = (lane & 1) ^ ((row >> 3) & 1);
            const unsigned off = (unsigned)row * K * 2 + (unsigned)(kt * 64 + slice * 16 + half * 8) * 2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(dst + j * 1024), 16, off, 0, 0, 0);
        }
    };
    issue(0);
    issue(1);
    float s = 0.f;
    for (int kt = 0; kt < KT; ++kt) {
        if (kt + 2 < KT) {
            issue(kt + 2);
            __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));  // vmcnt(8): two stages in flight
        } else {
            __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));  // vmcnt(0)
        }
        __syncthreads();
        s += reinterpret_cast<const float*>(ring + (kt % XST) * STAGE)[threadIdx.x];
        __syncthreads();
    }
    out[(blockIdx.y * gridDim.x + blockIdx.x) * kThreads + threadIdx.x] = s;
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)lo, (__bf16)hi});
}

__global__ __launch_bounds__(kThreads) void dequant(float* out, int iters) {
    __shared__ u32x4 wst[kThreads * 4];
    const u32x4 av = {threadIdx.x * 0x10001u, 0x3f803f80u, 0x3f003f00u, threadIdx.x};
    bf16x8 a[kTM], b[kTN];
#pragma unroll
    for (int tm = 0; tm < kTM; ++tm) a[tm] = as_bf16x8(av ^ (0x00010001u * (tm + 1)));
#pragma unroll
    for (int tn = 0; tn < kTN; ++tn) b[tn] = as_bf16x8(av ^ (0x00400040u + 0x00020002u * tn));
    f32x16 acc[kTM * kTN];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t) acc[t] = f32x16{};
    uint32_t code = threadIdx.x * 0x9E3779B9u + 1u;
    float sc = 0.25f + threadIdx.x * 1e-3f, bi = -1.f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int t = 0; t < kTM * kTN; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t / kTN], b[t % kTN], acc[t], 0, 0, 0);
        const u32x4 q = {code, code ^ (uint32_t)i, code + (uint32_t)i, code * 3u};
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint32_t lo = q[wi] & 0x0F0F0F0Fu, hi = (q[wi] >> 4) & 0x0F0F0F0Fu;
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = pack2(fmaf(sc, (float)((lo >> (8 * j)) & 0xFFu), bi), fmaf(sc, (float)((hi >> (8 * j)) & 0xFFu), bi));
            wst[threadIdx.x * 4 + wi] = o;
        }
        code = code * 1664525u + 1013904223u;
        sc += 1e-7f;
    }
    float s = reinterpret_cast<const float*>(wst)[threadIdx.x];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[t][e];
    out[blockIdx.x * kThreads + threadIdx.x] = s;
}

constexpr int kExactThreads = 256;  // one wave per SIMD
__global__ __launch_bounds__(kExactThreads) void exact(float* out, int iters) {
    __shared__ float xs[64 * 64];  // group sums X_m, 64 groups x 64 rows
    __shared__ u32x4 wst[kExactThreads * 4];
    for (int i = threadIdx.x; i < 64 * 64; i += kExactThreads) xs[i] = 1.f + i * 1e-4f;
    __syncthreads();
    const u32x4 av = {threadIdx.x * 0x10001u, 0x3f803f80u, 0x3f003f00u, threadIdx.x};
    bf16x8 a[kTM], b[kTN];  // distinct fragments per tile row and column, as in the matmul
#pragma unroll
    for (int tm = 0; tm < kTM; ++tm) a[tm] = as_bf16x8(av ^ (0x00010001u * (tm + 1)));
#pragma unroll
    for (int tn = 0; tn < kTN; ++tn) b[tn] = as_bf16x8(av ^ (0x00400040u + 0x00020002u * tn));
    const int lane = threadIdx.x & 63;
    float tot[kTM * kTN][16];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) tot[t][e] = 0.f;
    uint32_t code = threadIdx.x * 0x9E3779B9u + 1u;
    for (int i = 0; i < iters; ++i) {
        f32x16 D[kTM * kTN];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int t = 0; t < kTM * kTN; ++t)
                D[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t / kTN], b[t % kTN], kk == 0 ? f32x16{} : D[t], 0,
                                                               0, 0);
        // exact codes: 128 + q as bf16 by one and-or per pair
        const u32x4 q = {code, code ^ (uint32_t)i, code + (uint32_t)i, code * 3u};
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = ((q[wi] >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
            wst[threadIdx.x * 4 + wi] = o;
        }
        code = code * 1664525u + 1013904223u;
        // this lane's two output columns' scale and bias, this group's X of its 64 rows
        const float s0 = 0.25f + (i & 7) * 1e-3f, s1 = s0 + 1e-3f, b0 = -1.f - s0 * 128.f, b1 = -1.f - s1 * 128.f;
        const float* xg = xs + (i & 63) * 64;
#pragma unroll
        for (int tm = 0; tm < kTM; ++tm)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float X = xg[(tm * 16 + e + lane) & 63];
#pragma unroll
                for (int tn = 0; tn < kTN; ++tn) {
                    const int t = tm * kTN + tn;
                    tot[t][e] = fmaf(tn ? s1 : s0, D[t][e], tot[t][e]);
                    tot[t][e] = fmaf(tn ? b1 : b0, X, tot[t][e]);
                }
            }
    }
    float s = reinterpret_cast<const float*>(wst)[threadIdx.x];
#pragma unroll
    for (int t = 0; t < kTM * kTN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += tot[t][e];
    out[blockIdx.x * kExactThreads + threadIdx.x] = s;
}

template <typename F>
float time_us(hipStream_t st, int reps, F launch) {
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    launch();
    (void)hipStreamSynchronize(st);
    std::vector<float> t;
    for (int r = 0; r < reps; ++r) {
        (void)hipEventRecord(e0, st);
        launch();
        (void)hipEventRecord(e1, st);
        (void)hipEventSynchronize(e1);
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        t.push_back(ms * 1e3f);
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

int main(int argc, char** argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 2048;
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    const int blocks = cus;  // one block per CU, as the matmul
    float* out;
    CK(hipMalloc(&out, (size_t)448 * kThreads * sizeof(float)));

    const double flop_wave_iter = 2.0 * 32 * 32 * 16 * kTM * kTN;  // per wave and k-substep
    float us = time_us(st, 9, [&] { hipLaunchKernelGGL(mfma_regs, dim3(blocks), dim3(kThreads), 0, st, out, iters); });
    CK(hipGetLastError());
    printf("mfma_regs: %d blocks x 8 waves, %d x 8 MFMA 32x32x16 bf16 per wave: %.1f us, %.1f TFLOP/s\n", blocks,
           iters, us, flop_wave_iter * kWaves * blocks * iters / us / 1e6);
    fflush(stdout);

    const int kiters = iters / 4;  // k-steps of four substeps
    us = time_us(st, 9, [&] { hipLaunchKernelGGL(mfma_lds, dim3(blocks), dim3(kThreads), 0, st, out, kiters); });
    CK(hipGetLastError());
    printf("mfma_lds: %d blocks x 8 waves, %d k-steps (4 A + 2 B fragments, 8 MFMAs per substep): %.1f us, "
           "%.1f TFLOP/s\n", blocks, kiters, us, flop_wave_iter * kWaves * blocks * kiters * 4 / us / 1e6);
    fflush(stdout);

    const int ksteps = iters / 4;
    us = time_us(st, 9, [&] { hipLaunchKernelGGL(dequant, dim3(blocks), dim3(kThreads), 0, st, out, ksteps); });
    CK(hipGetLastError());
    printf("dequant: %d blocks x 8 waves, %d k-steps (32 MFMAs + 32 codes dequantized per lane): %.1f us, "
           "%.1f TFLOP/s\n", blocks, ksteps, us, flop_wave_iter * kWaves * blocks * ksteps * 4 / us / 1e6);
    fflush(stdout);
    us = time_us(st, 9, [&] { hipLaunchKernelGGL(exact, dim3(blocks), dim3(kExactThreads), 0, st, out, ksteps); });
    CK(hipGetLastError());
    printf("exact: %d blocks x 4 waves, %d k-steps (32 MFMAs from zero + 256 fused multiply-adds per lane): %.1f us, "
           "%.1f TFLOP/s\n", blocks, ksteps, us, flop_wave_iter * 4 * blocks * ksteps * 4 / us / 1e6);
    fflush(stdout);

    const int M = 2048, K = 4096, NT = 56;  // N = 14336 in 256-wide tiles
    unsigned short* x;
    CK(hipMalloc(&x, (size_t)M * K * 2));
    CK(hipMemset(x, 0x3c, (size_t)M * K * 2));
    const size_t ring = 3 * kBM * 64 * 2;
    CK(hipFuncSetAttribute((const void*)x_stage, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ring));
    us = time_us(st, 9, [&] { hipLaunchKernelGGL(x_stage, dim3(NT, M / kBM), dim3(kThreads), ring, st, x, M, K, out); });
    CK(hipGetLastError());
    const double bytes = (double)NT * M * K * 2;
    printf("x_stage: %d x %d blocks, %d k-steps of 32 KiB: %.1f us, %.1f GB/s into LDS (x re-read per N tile)\n", NT,
           M / kBM, K / 64, us, bytes / us / 1e3);
    CK(hipStreamSynchronize(st));
    printf("PASSED\n");
    return 0;
}
