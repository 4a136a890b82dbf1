// qmv_mfma.hip -- small-M route (M = 1..16) of affine group-quantized matmul on
// bf16 MFMA with exact integer codes.
//
//   y[m, n] = sum_k x[m, k] * (s[n, g(k)] * q[n, k] + b[n, g(k)])   (transpose=true)
//
// The reference reaches this through its quantized projections during decode
// (src/engine/mlx_lm/utils/mod.rs:70-78; src/engine/mlx_lm/models/llama.rs:
// 195-197,249,293-294,511-517) with x of one token, or a few rows when
// verifying speculative tokens.
//
// Why MFMA for a bandwidth-bound GEMV: the VALU cost of unpacking codes and
// dotting them with x is what keeps a VALU GEMV from streaming at HBM speed;
// here the dot products run on the matrix cores and the VALU only unpacks.
//
// v_mfma_f32_16x16x32_bf16 computes D[16 x 16] += A[16 x 32] * B[32 x 16].
//   B: 32 codes (one "k-block") of 16 rows n of W, as exact bf16 values 128+q
//      (4-bit: bits 0x4300|q) or q (8-bit: top half of the fp32 value).
//   A: the matching 32 values of x, one copy per MFMA row that is live for
//      this k-block.  MFMA rows are "group slots": row r = (m, slot) with
//      m = r / GS, slot = r % GS, GS = 16 / MT.  The A row of (m, slot) holds
//      x[m] only for k-blocks whose quantization group g has g % GS == slot,
//      zero otherwise.  So after GS consecutive groups, D[(m, slot)][n] holds
//      sum_{k in group} x[m,k] * code[n,k] for GS different groups at once,
//      and the per-group dequant is applied once per GS groups:
//        y[m,n] += s[n,g] * D[(m,slot)][n] + (b[n,g] - c*s[n,g]) * X[(m,slot)]
//      with c = 128 (4-bit) or 0 (8-bit) and X the per-group sums of x, taken
//      by one more MFMA of A against an all-ones B.
//   This keeps the dequant exact (fp32, as the reference's fp32 fma) and
//   needs ~1 VALU op per code.
//
// Work split: a block owns T tiles of 16 output rows n and all of K; its WPB
// waves split K into contiguous k-quad ranges (a k-quad is 4 k-blocks = 128
// codes) and combine their partial sums through LDS at the end.
//
// Scales and biases: each wave copies those of its k range for the block's
// rows into its own LDS area when it starts (direct-to-LDS dword loads, ahead
// of the first stages' loads), so a group cycle's dequant reads LDS.  Read
// from memory at the cycle's end instead, the wait for them drains every
// stage in flight with them (measured on MI355X, 4-bit g64: M = 16, 4096 ->
// 14336 31.3 -> 26.7 us, 14336 -> 4096 36.2 -> 26.3 us; M = 8, 14336 ->
// 4096 28.8 -> 19.5 us).  Odd G or scales not 4-byte aligned keep the
// memory reads.
//
// Loads: 4-bit -- lane (n, q) loads 16 bytes = chunk 4u+q (k-block 4u+q) of
// row n, so the 4 lanes of a row read 64 contiguous bytes; a 4x4 transpose of
// words across the lane quarters (v_permlane32_swap, v_permlane16_swap) then
// gives lane (n, q) quad q of each of the four k-blocks, which is what the B
// operand layout wants.  8-bit -- lane (n, q) loads quad q (8 bytes) of one
// k-block directly.  All loads are raw buffer loads with 32-bit offsets from
// per-block bases; offsets past the end read as zero, which masks ragged K,
// ragged N and the A rows of inactive group slots.
#include <atomic>
#include <type_traits>

#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) { return __builtin_bit_cast(bf16x8_t, v); }

// 4x4 transpose of words across the four 16-lane rows of a wave: afterwards
// register i of row q holds what register q of row i held
// (permlane32_swap(a, b) exchanges a's lanes 32-63 with b's lanes 0-31;
// permlane16_swap(a, b) exchanges a's rows 1 and 3 with b's rows 0 and 2)
__device__ __forceinline__ void transpose4x4(u32x4_t& v) {
    auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v[0] = c[0];
    v[1] = c[1];
    v[2] = d[0];
    v[3] = d[1];
}

// group pairs per row that a wave stages: the whole group cycles (GS groups)
// its k range (QS k-quads of 128 codes) touches, from an even group on; and
// the pairs of one array (scales or biases) of a wave's LDS area: rows x
// pairs, rounded up to whole 64-lane direct-to-LDS loads
__host__ __device__ constexpr int sb_pairs(int K, int gs_shift, int wpb, int gs) {
    return (((((K >> 5) + 3) >> 2) + wpb - 1) / wpb * (128 >> gs_shift) + 2 * gs + 1) / 2 + 1;
}
__host__ __device__ constexpr int sb_area_pairs(int T, int npr) { return (16 * T * npr + 63) / 64 * 64; }

template <int BITS, int T>
struct QStage {
    // 4-bit: one 16-byte chunk per tile (transposed to 4 k-blocks' quads);
    // 8-bit: 8 bytes per tile per k-block
    u32x4_t code[BITS == 4 ? T : 2 * T];
    u32x4_t xa[4];  // x for the 4 k-blocks (zero unless this lane's slot is live)
};

// GATHER: blockIdx.y picks one tile of the expert grouping (up to MT = 16
// selections of one expert, listed by the gather plan); the block streams
// that expert's weights once for all of them, with each MFMA row's x row
// gathered through the selection list and each output row scattered back.
struct MfmaGather {
    const int32_t* perm;    // selection ids grouped by expert
    const int32_t* seg;     // seg[e] .. seg[e+1]: expert e's range of perm (e == E: invalid ids)
    const int32_t* tiles;   // (expert, first position in perm) of each tile
    const int32_t* ntiles;  // number of tiles
    int top_k, x_per_index, experts;
    uint32_t x_bytes;       // bytes of x (all its matrices)
};

__device__ __forceinline__ int sload(const int32_t* p) {  // wave-uniform scalar load
    return __builtin_amdgcn_readfirstlane(*(const __attribute__((address_space(4))) int32_t*)p);
}

template <int BITS, int SBT, int MT, int T, int WPB, bool GATHER, bool SBL>
__global__ __launch_bounds__(WPB * 64) void qmv_mfma_kernel(const uint16_t* __restrict__ x,
                                                            const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ sc,
                                                            const uint16_t* __restrict__ bi,
                                                            void* __restrict__ y,
                                                            const void* __restrict__ bias, int M, int N,
                                                            int K, int gs_shift, int y_dtype,
                                                            const MfmaGather g = MfmaGather{}) {
    constexpr int GS = 16 / MT;                 // group slots per m
    constexpr int NMT = MT >= 4 ? MT / 4 : 1;   // distinct m per lane
    constexpr float kCentre = BITS == 4 ? 128.f : 0.f;
    using St = QStage<BITS, T>;
    // vector-memory loads of one stage: the codes (4-bit: one per tile;
    // 8-bit: two 8-byte loads per tile and register) and four x loads
    constexpr int kStageLoads = (BITS == 4 ? T : 4 * T) + 4;
    // stages in flight (measured on MI355X, M = 16 on 4096 -> 14336: 26.3,
    // 27.0 and 28.1 us with 2, 3 and 4)
    constexpr int DEPTH = 2;
    static_assert(DEPTH * kStageLoads < 64, "vmcnt range");

    extern __shared__ float red[];  // [WPB][T][64 lanes][NMT], then the waves' scale / bias areas

    const int lane = threadIdx.x & 63;
    const int nl = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16 * T;
    const int KB = K >> 5;            // k-blocks of 32 codes
    const int KQ = (KB + 3) >> 2;     // k-quads
    const int QS = (KQ + WPB - 1) / WPB;
    const int u0 = wv * QS;
    const int u1 = min(u0 + QS, KQ);
    const int G = K >> gs_shift;
    const int cl_shift = gs_shift - 5 + __builtin_ctz(GS);  // log2(k-blocks per GS-group cycle)
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    int rows_here = min(16 * T, N - n0);
    size_t erow0 = 0;  // GATHER: first W row of the expert
    int p0 = 0;        // GATHER: first position of the tile in the selection list
    if constexpr (GATHER) {
        if ((int)blockIdx.y >= sload(g.ntiles)) return;  // block-uniform: past the listed tiles
        const int e = sload(g.tiles + 2 * blockIdx.y);
        p0 = sload(g.tiles + 2 * blockIdx.y + 1);
        M = min(MT, sload(g.seg + e + 1) - p0);
        if (e >= g.experts) rows_here = 0;  // out-of-range ids: zero rows
        erow0 = (size_t)min(e, g.experts - 1) * N;
    }
    const auto wr = make_rsrc((const char*)w + (erow0 + n0) * row_bytes, (uint32_t)rows_here * row_bytes);
    const auto sr = make_rsrc(sc + (erow0 + n0) * G, (uint32_t)rows_here * G * 2);
    const auto br = make_rsrc(bi + (erow0 + n0) * G, (uint32_t)rows_here * G * 2);
    const auto xr = make_rsrc(x, GATHER ? g.x_bytes : (uint32_t)M * K * 2);
    const uint32_t kMask = vgpr_const(0x000F000Fu), kMagic = kMagic128x2;

    // this lane's A row: (m_a, slot_a), and the byte offset of its row of x
    const int m_a = nl / GS, slot_a = nl % GS;
    uint32_t xrow = m_a < M ? (uint32_t)m_a * K * 2 : kOOB;
    if constexpr (GATHER) {
        const int sel = m_a < M ? g.perm[p0 + m_a] : -1;
        const int xi = g.x_per_index ? sel : sel / g.top_k;
        xrow = sel >= 0 ? (uint32_t)xi * K * 2 : kOOB;
    }

    f32x4_t D[T], DX;
    float tot[T][NMT];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        D[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NMT; ++i) tot[t][i] = 0.f;
    }
    DX = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // k-quad u of this wave's range into a stage; u >= u1 (the pipeline runs
    // up to two k-quads past the range) reads zeros.  Codes are streamed once,
    // so they are loaded non-temporal.
    auto issue = [&](int u, St& st) {
        const int kbe = u < u1 ? KB : 0;  // k-blocks below kbe are live
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t row = (uint32_t)(16 * t + nl);
            if constexpr (BITS == 4) {
                const int chunk = 4 * u + q;
                st.code[t] = bload16_nt(wr, chunk < kbe ? row * row_bytes + (uint32_t)chunk * 16 : kOOB);
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // two k-blocks per 16-byte register: quads of k-blocks 4u+2h, 4u+2h+1
                    const int kb0 = 4 * u + 2 * h;
                    const uint32_t o0 = kb0 < kbe ? row * row_bytes + (uint32_t)kb0 * 32 + q * 8 : kOOB;
                    const uint32_t o1 = kb0 + 1 < kbe ? row * row_bytes + (uint32_t)(kb0 + 1) * 32 + q * 8 : kOOB;
                    const auto lo = __builtin_amdgcn_raw_buffer_load_b64(wr, o0, 0, kNonTemporal);
                    const auto hi = __builtin_amdgcn_raw_buffer_load_b64(wr, o1, 0, kNonTemporal);
                    st.code[2 * t + h] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kb = 4 * u + i;
            const int gidx = kb >> (gs_shift - 5);
            const bool live = kb < kbe && xrow != kOOB && (gidx % GS) == slot_a;
            st.xa[i] = bload16(xr, live ? xrow + (uint32_t)(kb * 32 + 8 * q) * 2 : kOOB);
        }
    };

    // apply the dequant of one group cycle c (groups c*GS .. c*GS+GS-1) and clear D
    // This lane's four D rows r = 4q + j hold groups c*GS + r % GS: with
    // GS < 4 only GS of them differ (r % GS = j % GS), so each distinct
    // scale / bias is loaded once (M = 16: one pair per row instead of four)
    constexpr int NG = GS < 4 ? GS : 4;
    // this wave's LDS area (SBL): scales then biases, [16T rows][2 npr]
    // halves of groups g0 .. g0 + 2 npr - 1, from the first group of its
    // first cycle rounded down to even, zero past G
    const int npr = sb_pairs(K, gs_shift, WPB, GS), area = sb_area_pairs(T, npr);
    const int g0 = ((u0 << (7 - gs_shift)) / GS * GS) & ~1;
    uint16_t* const sl = reinterpret_cast<uint16_t*>(red + WPB * T * 64 * NMT) + wv * 4 * area;
    uint16_t* const bl = sl + 2 * area;
    auto rescale = [&](int c) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t row = (uint32_t)(16 * t + nl);
            float sv[NG], bv[NG];
#pragma unroll
            for (int jj = 0; jj < NG; ++jj) {
                const int g = c * GS + ((4 * q + jj) % GS);
                uint16_t sh, bh;
                if constexpr (SBL) {
                    const int li = (int)row * 2 * npr + (g - g0);
                    sh = sl[li];
                    bh = bl[li];
                } else {
                    const uint32_t off = g < G ? (row * G + g) * 2 : kOOB;
                    sh = bload2(sr, off);
                    bh = bload2(br, off);
                }
                sv[jj] = half_to_f32<SBT>(sh);
                bv[jj] = half_to_f32<SBT>(bh) - kCentre * sv[jj];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float s = sv[GS >= 4 ? j : j % GS], b = bv[GS >= 4 ? j : j % GS];
                const int mi = GS >= 4 ? 0 : j / GS;  // which of this lane's m (compile time)
                tot[t][mi] = fmaf(s, D[t][j], tot[t][mi]);
                tot[t][mi] = fmaf(b, DX[j], tot[t][mi]);
            }
            D[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        DX = f32x4_t{0.f, 0.f, 0.f, 0.f};
    };

    const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
    auto compute = [&](int u, St& st) {
        if constexpr (BITS == 4) {
#pragma unroll
            for (int t = 0; t < T; ++t) transpose4x4(st.code[t]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kb = 4 * u + i;
            u32x4_t a;
            if constexpr (BITS == 4) {
                uint32_t xw[4] = {st.xa[i][0], st.xa[i][1], st.xa[i][2], st.xa[i][3]};
                uint32_t X[4];
                perm_x_for4(xw, X);
                a = u32x4_t{X[0], X[1], X[2], X[3]};
            } else {
                a = st.xa[i];
            }
            const bf16x8_t A = as_bf16x8(a);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                uint32_t p[4];
                if constexpr (BITS == 4) {
                    unpack4_magic(st.code[t][i], p, kMask, kMagic);
                } else {
                    // quad q of k-block 4u+i: words 2*(i&1), 2*(i&1)+1 of register 2t + i/2
                    const u32x4_t& c = st.code[2 * t + (i >> 1)];
                    unpack8_pairs(c[2 * (i & 1)], &p[0]);
                    unpack8_pairs(c[2 * (i & 1) + 1], &p[2]);
                }
                D[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, as_bf16x8(u32x4_t{p[0], p[1], p[2], p[3]}), D[t], 0, 0, 0);
            }
            DX = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, as_bf16x8(ones), DX, 0, 0, 0);
            // end of a group cycle (or of K): fold the cycle into the totals
            if (kb < KB && (((kb + 1) >> cl_shift) != (kb >> cl_shift) || kb + 1 == KB)) rescale(kb >> cl_shift);
        }
    };

    // pipeline over k-quads, DEPTH stages in flight.  Each stage is
    // refilled right after it is computed, unconditionally: a conditional
    // issue makes the compiler's wait before each compute count from the path
    // without the loads, i.e. wait for the stage just issued.
    if (u0 < u1) {
        if constexpr (SBL) {  // stage the scales and biases, ahead of the stages' loads
            const int npairs = 16 * T * npr;
            for (int d = 0; d * 64 < npairs; ++d) {
                const int e = d * 64 + lane;
                const int row = e / npr, gp = g0 + 2 * (e - row * npr);
                const uint32_t off = e < npairs && gp < G ? ((uint32_t)row * G + gp) * 2 : kOOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(sl + 128 * d), 4, off, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_void*)(bl + 128 * d), 4, off, 0, 0, 0);
            }
        }
        St S[DEPTH];
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) issue(u0 + i, S[i]);
        // the staged scales land before any cycle reads them (the compiler
        // does not see that dependency): issued after them and still allowed
        // in flight are the stages' loads
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(DEPTH * kStageLoads));
        asm volatile("" ::: "memory");
        int u = u0;
        for (; u + DEPTH <= u1; u += DEPTH) {
#pragma unroll
            for (int i = 0; i < DEPTH; ++i) {
                compute(u + i, S[i]);
                issue(u + i + DEPTH, S[i]);
            }
        }
#pragma unroll
        for (int i = 0; i + 1 < DEPTH; ++i)
            if (u + i < u1) compute(u + i, S[i]);
        // a slice that ends mid-cycle has partial sums left in D
        const int last = min(4 * u1, KB) - 1;
        if (((last + 1) >> cl_shift) == (last >> cl_shift) && last + 1 != KB) rescale(last >> cl_shift);
    }

    // combine the waves' partial sums and store
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < NMT; ++i) red[((wv * T + t) * 64 + lane) * NMT + i] = tot[t][i];
    __syncthreads();
    // output (t, m, nl): sum over waves and over the lanes (quarters q, rows j) that hold m
    for (int o = threadIdx.x; o < T * MT * 16; o += WPB * 64) {
        const int t = o / (MT * 16), m = (o / 16) % MT, n = o % 16;
        const int nn = n0 + 16 * t + n;
        if (m >= M || nn >= N) continue;
        float v = 0.f;
        for (int ww = 0; ww < WPB; ++ww) {
            // rows r with r / GS == m live in quarters q = r / 4
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
                for (int i = 0; i < NMT; ++i) {
                    const int r = 4 * qq + (NMT == 1 ? 0 : i * GS);
                    if (r / GS != m) continue;
                    v += red[((ww * T + t) * 64 + qq * 16 + n) * NMT + i];
                }
            }
        }
        const int64_t yrow = GATHER ? g.perm[p0 + m] : m;  // GATHER: the selection's own output row
        store_out(y, yrow * N + nn, y_dtype, v, bias, nn);
    }
}

// LDS of a launch: the cross-wave reduction, and the waves' scale / bias
// areas when they stage them (an even number of groups per row, 4-byte
// aligned arrays: the copies move group pairs; and room in the 160 KiB)
size_t mfma_lds(const QmmArgs& a, int T, int wpb, int mt, int nmt, int* sbl) {
    const size_t red = sizeof(float) * wpb * T * 64 * nmt;
    const int npr = sb_pairs((int)a.K, __builtin_ctz((unsigned)a.group_size), wpb, 16 / mt);
    const size_t stage = (size_t)wpb * 2 * sb_area_pairs(T, npr) * 4;
    const bool al = ((reinterpret_cast<uintptr_t>(a.scales) | reinterpret_cast<uintptr_t>(a.biases)) & 3) == 0;
    *sbl = (a.K / a.group_size) % 2 == 0 && al && red + stage <= 160 * 1024 ? 1 : 0;
    return red + (*sbl ? stage : 0);
}
// dynamic LDS above the default 64 KiB needs the kernel's attribute raised,
// once per kernel and device (two threads racing both set it: harmless)
template <auto kernel>
hipError_t allow_lds(size_t lds) {
    static std::atomic<uint64_t> set{0};
    if (lds <= 65536) return hipSuccess;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev >= 64) return hipErrorInvalidDevice;
    if (set.load(std::memory_order_relaxed) >> dev & 1) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             160 * 1024);
    if (e == hipSuccess) set.fetch_or(uint64_t{1} << dev, std::memory_order_relaxed);
    return e;
}

template <int BITS, int SBT, int MT, int T, int WPB, bool GATHER, bool SBL>
hipError_t launch_k(const QmmArgs& a, dim3 grid, size_t lds, const MfmaGather& g) {
    const hipError_t e = allow_lds<qmv_mfma_kernel<BITS, SBT, MT, T, WPB, GATHER, SBL>>(lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((qmv_mfma_kernel<BITS, SBT, MT, T, WPB, GATHER, SBL>), grid, dim3(WPB * 64), lds, a.stream,
                       (const uint16_t*)a.x, a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.y,
                       GATHER ? nullptr : a.bias, GATHER ? MT : (int)a.M, (int)a.N, (int)a.K,
                       __builtin_ctz((unsigned)a.group_size), a.y_dtype, g);
    return hipGetLastError();
}

template <int BITS, int SBT, int MT, int T, int WPB>
hipError_t launch_t(const QmmArgs& a) {
    constexpr int NMT = MT >= 4 ? MT / 4 : 1;
    const dim3 grid((unsigned)((a.N + 16 * T - 1) / (16 * T)));
    int sbl = 0;
    const size_t lds = mfma_lds(a, T, WPB, MT, NMT, &sbl);
    return sbl ? launch_k<BITS, SBT, MT, T, WPB, false, true>(a, grid, lds, MfmaGather{})
               : launch_k<BITS, SBT, MT, T, WPB, false, false>(a, grid, lds, MfmaGather{});
}

int pick_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// tiles per block and waves per block: 16 K-splitting waves once K has at
// least 64 k-quads (K >= 8192) and M <= 8, else 4; then the most 16-row
// tiles per block (4, 2 or 1: more tiles amortise the x operand, which every
// block reads whole from L2) that still give 192 blocks, three quarters of
// the CUs.  Measured on MI355X with the scales staged in LDS (4-bit g64, us,
// M = 8 / 16; the choice first): 4096 -> 14336 (T 4) 15.7 / 19.1, T 2 14.9 /
// 18.9, T 1 18.0 / 23.6; 14336 -> 4096 (T 1, 16 waves) 18.2 / 24.5, four
// waves 22.4 / 20.6 (hence four at M = 16), T 2 with 16 waves 23.8 / 30.0;
// 4096 -> 4096 (T 1) 9.1 / 8.9, T 2 10.9 / 11.8.
void pick_tw(int64_t M, int64_t N, int64_t K, int bits, int* T, int* WPB) {
    const int64_t KQ = (K / 32 + 3) / 4;
    const int nmt = M > 4 ? (M > 8 ? 4 : 2) : 1;
    const int wpb = KQ >= 64 && M <= 8 ? 16 : 4;
    int t = 4;
    while (t > 1 && (N + 16 * t - 1) / (16 * t) < 192) t /= 2;
    while (t > 1 && wpb * t * 64 * nmt * 4 > 32768) t /= 2;  // cross-wave reduction LDS
    // 16 waves of a block get at most 128 registers each: four tiles' stages
    // and accumulators do not fit in them (they spilled)
    if (wpb == 16 && t > 2) t = 2;
    (void)bits;
    *T = t;
    *WPB = wpb;
}

template <int BITS, int SBT, int MT, int T>
hipError_t launch_w(const QmmArgs& a, int wpb) {
    if constexpr (T == 4) {  // four waves only (pick_tw)
        return launch_t<BITS, SBT, MT, T, 4>(a);
    } else {
        return wpb == 16 ? launch_t<BITS, SBT, MT, T, 16>(a) : launch_t<BITS, SBT, MT, T, 4>(a);
    }
}

template <int BITS, int SBT, int MT>
hipError_t launch_tt(const QmmArgs& a) {
    int T, WPB;
    pick_tw(a.M, a.N, a.K, a.bits, &T, &WPB);
    if (T == 1) return launch_w<BITS, SBT, MT, 1>(a, WPB);
    return T == 4 ? launch_w<BITS, SBT, MT, 4>(a, WPB) : launch_w<BITS, SBT, MT, 2>(a, WPB);
}

// expert-grouped GEMV: one block row per tile of the plan (surplus blocks of
// the max-tiles grid exit at once), 16 selections per tile
template <int BITS, int SBT, int T, int WPB>
hipError_t launch_gather_t(const QmmArgs& a, const MfmaGather& g, int64_t max_tiles) {
    constexpr int MT = kGatherGemvRows, NMT = MT / 4;
    const dim3 grid((unsigned)((a.N + 16 * T - 1) / (16 * T)), (unsigned)max_tiles);
    int sbl = 0;
    const size_t lds = mfma_lds(a, T, WPB, MT, NMT, &sbl);
    return sbl ? launch_k<BITS, SBT, MT, T, WPB, true, true>(a, grid, lds, g)
               : launch_k<BITS, SBT, MT, T, WPB, true, false>(a, grid, lds, g);
}

template <int BITS, int SBT>
hipError_t launch_gather_tw(const QmmArgs& a, const MfmaGather& g, int64_t max_tiles, int64_t experts) {
    // the grid already holds a block per (tile, 64 rows): four waves per
    // block, each a quarter of K (measured on MI355X, DeepSeek-V2-Lite gate at
    // 64 tokens: 83 us against 132 with 16 K-splitting waves of two tiles)
    (void)experts;
    return launch_gather_t<BITS, SBT, 4, 4>(a, g, max_tiles);
}

template <int BITS, int SBT>
hipError_t launch_mt(const QmmArgs& a) {
    switch (pick_mt(a.M)) {
        case 1: return launch_tt<BITS, SBT, 1>(a);
        case 2: return launch_tt<BITS, SBT, 2>(a);
        case 4: return launch_tt<BITS, SBT, 4>(a);
        case 8: return launch_tt<BITS, SBT, 8>(a);
        default: return launch_tt<BITS, SBT, 16>(a);
    }
}

}  // namespace

void qmv_mfma_config(const QmmArgs& a, int* tiles_per_block, int* m_tile, int* waves_per_block) {
    int T, WPB;
    pick_tw(a.M, a.N, a.K, a.bits, &T, &WPB);
    if (tiles_per_block) *tiles_per_block = T;
    if (m_tile) *m_tile = pick_mt(a.M);
    if (waves_per_block) *waves_per_block = WPB;
}

hipError_t launch_gather_gemv(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_index,
                              int64_t experts, int64_t x_bytes, void* workspace) {
    const int64_t S = T * top_k;
    const GatherPlan pl = gather_plan_layout(workspace, S, experts, kGatherGemvRows);
    hipError_t e = launch_gather_plan(idx, S, experts, kGatherGemvRows, pl, a.stream);
    if (e != hipSuccess) return e;
    const MfmaGather g{pl.perm, pl.seg, pl.tiles, pl.ntiles, top_k, x_per_index, (int)experts, (uint32_t)x_bytes};
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_gather_tw<4, DT_F16>(a, g, pl.max_tiles, experts)
                                    : launch_gather_tw<4, DT_BF16>(a, g, pl.max_tiles, experts);
    return a.sb_dtype == DT_F16 ? launch_gather_tw<8, DT_F16>(a, g, pl.max_tiles, experts)
                                : launch_gather_tw<8, DT_BF16>(a, g, pl.max_tiles, experts);
}

hipError_t launch_qmv_mfma(const QmmArgs& a) {
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_mt<4, DT_F16>(a) : launch_mt<4, DT_BF16>(a);
    return a.sb_dtype == DT_F16 ? launch_mt<8, DT_F16>(a) : launch_mt<8, DT_BF16>(a);
}

}  // namespace miqmm
