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
// Group cycles: the per-group dequant is applied once per cycle of GS
// groups.  A cycle of up to 8 k-blocks starts and ends at fixed k-blocks of
// a pipeline iteration (two k-quads; a wave's range starts an iteration and a
// cycle), so its first MFMAs take a zero accumulator and its last k-block
// folds D into the totals with no clearing; longer cycles span whole
// iterations.  The accumulators live in VGPRs (built with
// -amdgpu-mfma-vgpr-form), where the fused multiply-adds read them directly.
// Together: 26.5 -> 16.4 VALU instructions per MFMA (M = 16, 4-bit g64).
//
// Work split: a block owns T tiles of 16 output rows n and all of K; its WPB
// waves split K into contiguous k-quad ranges (a k-quad is 4 k-blocks = 128
// codes) and combine their partial sums through LDS at the end.
//
// K split (SPLIT, with a caller workspace): blocks of 8 waves own a tile each
// over one of S k ranges; the block stages its x range in LDS once, as the
// A rows already masked to their group slot and permuted for the code unpack,
// each wave streams its tile's codes four k-quads ahead, and writes fp32
// partials that the split-reduce kernel adds in range order.  What bounds the
// kernel is the bytes a CU loads: each CU's vector-memory path delivers
// about 30 GB/s whether a load hits L1, L2 or HBM (measured on MI355X: 16
// rows of x re-read by every block, 4.6-9 TB/s in total; the same bytes read
// by the four waves of a block from L1, the same time), so x re-read per
// block of 16-64 rows costs as much as the codes at M = 16.
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

// log2 of the k-blocks (32 codes) of one group cycle (GS groups of 2^gs_shift
// codes), and the cycle class a kernel is built for: 0-3 a cycle of 1-8
// k-blocks, which starts and ends at fixed places of the two k-quads of a
// pipeline iteration; 4 a longer cycle, a whole number of iterations
__host__ __device__ constexpr int cycle_shift(int gs_shift, int gs) { return gs_shift - 5 + __builtin_ctz(gs); }
__host__ __device__ constexpr int cycle_class(int cl_shift) { return cl_shift <= 3 ? cl_shift : 4; }
// k-quads per wave: the K split over the block's waves, in whole iterations
// (two k-quads) and whole group cycles, so every wave starts a cycle
__host__ __device__ constexpr int wave_kquads(int K, int wpb, int cl_shift) {
    const int span = cl_shift <= 3 ? 2 : 1 << (cl_shift - 2);
    return ((((K >> 5) + 3) >> 2) + wpb - 1) / wpb + span - 1 & ~(span - 1);
}
// SPLIT: bytes per A row of the block's x in LDS (qs k-quads of 128 codes;
// 16 bytes of padding put the 16 rows of an operand read in different banks)
__host__ __device__ constexpr int split_x_stride(int qs) { return qs * 256 + 16; }
// group pairs per row that a wave stages (those of its k range: a whole
// number of pairs, its k range spans an even number of k-quads), and the
// pairs of one array (scales or biases) of a wave's LDS area: rows x pairs,
// rounded up to whole 64-lane direct-to-LDS loads
__host__ __device__ constexpr int sb_pairs(int K, int gs_shift, int wpb, int gs) {
    return (wave_kquads(K, wpb, cycle_shift(gs_shift, gs)) << (7 - gs_shift)) >> 1;
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

// CLS: the cycle class (cycle_class) of the launch's group size and MT.
// SPLIT: K is cut into ksplit ranges (blockIdx.y), the waves of a block own
// different tiles over one range, and each wave writes its fp32 partial sums
// to y = partials [ksplit][M][N] (added in range order by the split-reduce
// kernel); otherwise a block's waves split K over its tiles.
template <int BITS, int SBT, int MT, int T, int WPB, bool GATHER, bool SBL, int CLS, bool SPLIT>
__global__ __launch_bounds__(WPB * 64) void qmv_mfma_kernel(const uint16_t* __restrict__ x,
                                                            const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ sc,
                                                            const uint16_t* __restrict__ bi,
                                                            void* __restrict__ y,
                                                            const void* __restrict__ bias, int M, int N,
                                                            int K, int gs_shift, int y_dtype, int ksplit,
                                                            const MfmaGather g = MfmaGather{}) {
    constexpr int GS = 16 / MT;                 // group slots per m
    constexpr int NMT = MT >= 4 ? MT / 4 : 1;   // distinct m per lane
    constexpr float kCentre = BITS == 4 ? 128.f : 0.f;
    using St = QStage<BITS, T>;
    // vector-memory loads of one stage: the codes (4-bit: one per tile;
    // 8-bit: two 8-byte loads per tile and register) and four x loads
    // (SPLIT: x comes from LDS, no x loads)
    constexpr int kStageLoads = (BITS == 4 ? T : 4 * T) + (SPLIT ? 0 : 4);
    // stages in flight (measured on MI355X, M = 16 on 4096 -> 14336: 26.3,
    // 27.0 and 28.1 us with 2, 3 and 4)
#ifndef QMV_MFMA_DEPTH
#define QMV_MFMA_DEPTH 2
#endif
    constexpr int kMaxDepth = (63 / kStageLoads) & ~1;  // the loads a vmcnt wait can count
    // SPLIT stages hold only codes: four k-quads in flight (measured on
    // MI355X, M = 16: 14336 -> 4096 15.5 / 16.2 / 18.2 us with 4 / 8 / 16);
    // unsplit one-tile blocks also take four (M = 8, 4096 -> 4096: 8.9 -> 7.1
    // us), more tiles two (M = 8, 4096 -> 14336, two tiles: 13.3 -> 15.2)
    constexpr int kDepth = SPLIT || T == 1 ? 4 : QMV_MFMA_DEPTH;
    constexpr int DEPTH = kDepth < kMaxDepth ? kDepth : kMaxDepth;
    static_assert(DEPTH >= 2 && DEPTH * kStageLoads < 64, "vmcnt range");

    // [WPB][T][64 lanes][NMT] (not with SPLIT), then the waves' scale / bias areas
    extern __shared__ float red[];

    const int lane = threadIdx.x & 63;
    const int nl = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = (SPLIT ? blockIdx.x * WPB + wv : blockIdx.x) * 16 * T;
    const int KB = K >> 5;            // k-blocks of 32 codes
    const int KQ = (KB + 3) >> 2;     // k-quads
    const int cl_shift = CLS < 4 ? CLS : cycle_shift(gs_shift, GS);  // log2(k-blocks per GS-group cycle)
    const int QS = wave_kquads(K, SPLIT ? ksplit : WPB, cl_shift);
    const int u0 = (SPLIT ? (int)blockIdx.y : wv) * QS;
    const int u1 = min(u0 + QS, KQ);
    const int G = K >> gs_shift;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    int rows_here = max(0, min(16 * T, N - n0));
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
        if constexpr (!SPLIT) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kb = 4 * u + i;
                const int gidx = kb >> (gs_shift - 5);
                const bool live = kb < kbe && xrow != kOOB && (gidx % GS) == slot_a;
                st.xa[i] = bload16(xr, live ? xrow + (uint32_t)(kb * 32 + 8 * q) * 2 : kOOB);
            }
        }
    };

    // apply the dequant of one group cycle c (groups c*GS .. c*GS+GS-1): the
    // next cycle's first MFMAs start from zero (CLS < 4) or D is cleared at
    // the next cycle's start (CLS 4).
    // This lane's four D rows r = 4q + j hold groups c*GS + r % GS: with
    // GS < 4 only GS of them differ (r % GS = j % GS), so each distinct
    // scale / bias is loaded once (M = 16: one pair per row instead of four)
    constexpr int NG = GS < 4 ? GS : 4;
    // this wave's LDS area (SBL): scales then biases, [16T rows][2 npr]
    // halves of groups g0 .. g0 + 2 npr - 1, the groups of its k range (its
    // first group starts a cycle and is even), zero past G
    const int npr = sb_pairs(K, gs_shift, SPLIT ? ksplit : WPB, GS), area = sb_area_pairs(T, npr);
    const int g0 = u0 << (7 - gs_shift);
    // SPLIT: the block's A rows (m, slot) of x over its k range, then the scale areas
    char* const xs = reinterpret_cast<char*>(red);
    const int xstride = split_x_stride(QS);
    const int xa_lane = nl * xstride + q * 16;  // this lane's A operand in a k-block's 64-byte run
    uint16_t* const sl =
        reinterpret_cast<uint16_t*>(red + (SPLIT ? 4 * xstride : WPB * T * 64 * NMT)) + wv * 4 * area;
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
        }
    };
    auto clear = [&] {
#pragma unroll
        for (int t = 0; t < T; ++t) D[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        DX = f32x4_t{0.f, 0.f, 0.f, 0.f};
    };

    const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
    // k-quad u, the POS-th (0 or 1) of its pipeline iteration.  With CLS < 4
    // a cycle of 2^CLS k-blocks starts and ends at fixed k-blocks of the
    // iteration: its first MFMAs take a zero accumulator and its last folds
    // it into the totals, with no clearing of D.
    auto compute = [&](int u, St& st, auto pos) {
        constexpr int POS = decltype(pos)::value;
        if constexpr (BITS == 4) {
#pragma unroll
            for (int t = 0; t < T; ++t) transpose4x4(st.code[t]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kb = 4 * u + i;
            constexpr int CB = 1 << (CLS < 4 ? CLS : 0);
            const int p = 4 * POS + i;  // k-block of the iteration
            const bool restart = CLS < 4 && (p & (CB - 1)) == 0;
            const bool end = CLS < 4 && (p & (CB - 1)) == CB - 1;
            u32x4_t a;
            if constexpr (SPLIT) {
                // A row nl of this k-block, staged (masked, permuted) in LDS
                a = *reinterpret_cast<const u32x4_t*>(xs + xa_lane + (kb - 4 * u0) * 64);
            } else if constexpr (BITS == 4) {
                uint32_t xw[4] = {st.xa[i][0], st.xa[i][1], st.xa[i][2], st.xa[i][3]};
                uint32_t X[4];
                perm_x_for4(xw, X);
                a = u32x4_t{X[0], X[1], X[2], X[3]};
            } else {
                a = st.xa[i];
            }
            const bf16x8_t A = as_bf16x8(a);
            const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < T; ++t) {
                uint32_t pw[4];
                if constexpr (BITS == 4) {
                    unpack4_magic(st.code[t][i], pw, kMask, kMagic);
                } else {
                    // quad q of k-block 4u+i: words 2*(i&1), 2*(i&1)+1 of register 2t + i/2
                    const u32x4_t& c = st.code[2 * t + (i >> 1)];
                    unpack8_pairs(c[2 * (i & 1)], &pw[0]);
                    unpack8_pairs(c[2 * (i & 1) + 1], &pw[2]);
                }
                D[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, as_bf16x8(u32x4_t{pw[0], pw[1], pw[2], pw[3]}),
                                                               restart ? zero : D[t], 0, 0, 0);
            }
            DX = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, as_bf16x8(ones), restart ? zero : DX, 0, 0, 0);
            if (end) rescale(kb >> cl_shift);
        }
    };

    // pipeline over iterations of two k-quads, one stage each in flight.
    // Each stage is refilled right after it is computed, unconditionally: a
    // conditional issue makes the compiler's wait before each compute count
    // from the path without the loads, i.e. wait for the stage just issued.
    if (u0 < u1) {  // (SPLIT: true for every block)
        // SPLIT: the block's x over its k range as the MFMA's A rows: row r =
        // (m, slot) holds x[m] where the group is slot mod GS (zero elsewhere
        // and past M or K), 4-bit: in the code unpack's pair order; each 16
        // bytes loaded once per block, up to XU per thread ahead of the codes
        constexpr int XU = 8;
        const int units = SPLIT ? 16 * QS * 16 : 0;  // rows x 16-byte units of the range
        u32x4_t xv[XU];
        auto x_unit = [&](int e, bool load) {
            const int r = e / (QS * 16), c8 = e - r * (QS * 16);
            const int m = r / GS, slot = r % GS;
            const int k = u0 * 128 + c8 * 8;
            const bool live = e < units && m < M && k < K && ((k >> gs_shift) & (GS - 1)) == slot;
            return load ? bload16(xr, live ? (uint32_t)(m * K + k) * 2 : kOOB)
                        : u32x4_t{(uint32_t)(r * xstride + c8 * 16), (uint32_t)(e < units), 0u, 0u};
        };
        auto x_store = [&](int e, u32x4_t v) {
            const u32x4_t at = x_unit(e, false);
            if (!at[1]) return;
            if constexpr (BITS == 4) {
                uint32_t xw[4] = {v[0], v[1], v[2], v[3]}, X[4];
                perm_x_for4(xw, X);
                v = u32x4_t{X[0], X[1], X[2], X[3]};
            }
            *reinterpret_cast<u32x4_t*>(xs + at[0]) = v;
        };
        if constexpr (SPLIT) {
#pragma unroll
            for (int j = 0; j < XU; ++j) xv[j] = x_unit(threadIdx.x + j * WPB * 64, true);
        }
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
        if constexpr (SPLIT) {
#pragma unroll
            for (int j = 0; j < XU; ++j) x_store(threadIdx.x + j * WPB * 64, xv[j]);
            for (int e = threadIdx.x + XU * WPB * 64; e < units; e += WPB * 64) x_store(e, x_unit(e, true));
            __syncthreads();
            if (rows_here == 0) return;  // a wave past N (after the block's barrier)
        }
        // the staged scales land before any cycle reads them (the compiler
        // does not see that dependency): issued after them and still allowed
        // in flight are the stages' loads
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(DEPTH * kStageLoads));
        asm volatile("" ::: "memory");
        // CLS 4: a cycle of 2^cl_shift k-blocks spans whole iterations
        const int cb_mask = (1 << cl_shift) - 1;
        // the k-quads uu (and uu + 1 when two) of one iteration
        auto iteration = [&](int uu, St& s0, St& s1, bool two) {
            if constexpr (CLS == 4)
                if (((4 * uu) & cb_mask) == 0) clear();
            compute(uu, s0, std::integral_constant<int, 0>{});
            if (two) compute(uu + 1, s1, std::integral_constant<int, 1>{});
            // CLS 4: the cycle ends with the iteration, or the range does;
            // CLS 3: a single k-quad ends its cycle part-filled
            if constexpr (CLS == 4) {
                if (((4 * (uu + 2)) & cb_mask) == 0 || uu + 2 >= u1) rescale((4 * uu) >> cl_shift);
            } else if constexpr (CLS == 3) {
                if (!two) rescale((4 * uu) >> cl_shift);
            }
        };
        int u = u0;
        for (; u + DEPTH <= u1; u += DEPTH) {
#pragma unroll
            for (int i = 0; i < DEPTH; i += 2) {
                if constexpr (CLS == 4)
                    if (((4 * (u + i)) & cb_mask) == 0) clear();
                compute(u + i, S[i], std::integral_constant<int, 0>{});
                issue(u + i + DEPTH, S[i]);
                compute(u + i + 1, S[i + 1], std::integral_constant<int, 1>{});
                issue(u + i + 1 + DEPTH, S[i + 1]);
                if constexpr (CLS == 4)
                    if (((4 * (u + i + 2)) & cb_mask) == 0 || u + i + 2 == u1) rescale((4 * (u + i)) >> cl_shift);
            }
        }
#pragma unroll
        for (int i = 0; i < DEPTH; i += 2)  // the k-quads left, fewer than DEPTH
            if (u + i < u1) iteration(u + i, S[i], S[i + 1], u + i + 1 < u1);
    }

    if constexpr (SPLIT) {
        // lane (nl, q) holds m = q NMT + i of row n0 + 16 t + nl: this wave's
        // partial sums of its range, or with one range the outputs
        float* const part = static_cast<float*>(y) + (size_t)blockIdx.y * M * N;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int n = n0 + 16 * t + nl;
#pragma unroll
            for (int i = 0; i < NMT; ++i) {
                const int m = q * NMT + i;
                if (m >= M || n >= N) continue;
                if (ksplit == 1) store_out(y, (int64_t)m * N + n, y_dtype, tot[t][i], bias, n);
                else part[(size_t)m * N + n] = tot[t][i];
            }
        }
        return;
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
    *sbl = *sbl && (a.K / a.group_size) % 2 == 0 && al && red + stage <= 160 * 1024 ? 1 : 0;
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

template <int BITS, int SBT, int MT, int T, int WPB, bool GATHER, bool SBL, int CLS, bool SPLIT>
hipError_t launch_kc(const QmmArgs& a, dim3 grid, size_t lds, const MfmaGather& g, float* part) {
    constexpr auto kernel = qmv_mfma_kernel<BITS, SBT, MT, T, WPB, GATHER, SBL, CLS, SPLIT>;
    const hipError_t e = allow_lds<kernel>(lds);
    if (e != hipSuccess) return e;
    // SPLIT with one k range (part == nullptr) writes y itself
    hipLaunchKernelGGL(kernel, grid, dim3(WPB * 64), lds, a.stream, (const uint16_t*)a.x, a.w,
                       (const uint16_t*)a.scales, (const uint16_t*)a.biases, part ? (void*)part : a.y,
                       GATHER || part ? nullptr : a.bias, GATHER ? MT : (int)a.M, (int)a.N, (int)a.K,
                       __builtin_ctz((unsigned)a.group_size), a.y_dtype, (int)grid.y, g);
    return hipGetLastError();
}

// the kernel of the launch's cycle class: group sizes 32, 64 and 128 give
// three consecutive classes from log2(16 / MT) on
template <int BITS, int SBT, int MT, int T, int WPB, bool GATHER, bool SBL, bool SPLIT = false>
hipError_t launch_k(const QmmArgs& a, dim3 grid, size_t lds, const MfmaGather& g, float* part = nullptr) {
    constexpr int L = __builtin_ctz(16 / MT);
    constexpr int C0 = cycle_class(L), C1 = cycle_class(L + 1), C2 = cycle_class(L + 2);
    const int cls = cycle_class(cycle_shift(__builtin_ctz((unsigned)a.group_size), 16 / MT));
    if (cls == C0) return launch_kc<BITS, SBT, MT, T, WPB, GATHER, SBL, C0, SPLIT>(a, grid, lds, g, part);
    if (cls == C1) return launch_kc<BITS, SBT, MT, T, WPB, GATHER, SBL, C1, SPLIT>(a, grid, lds, g, part);
    return launch_kc<BITS, SBT, MT, T, WPB, GATHER, SBL, C2, SPLIT>(a, grid, lds, g, part);
}

template <int BITS, int SBT, int MT, int T, int WPB>
hipError_t launch_t(const QmmArgs& a) {
    constexpr int NMT = MT >= 4 ? MT / 4 : 1;
    const dim3 grid((unsigned)((a.N + 16 * T - 1) / (16 * T)));
    int sbl = 1;
    const size_t lds = mfma_lds(a, T, WPB, MT, NMT, &sbl);
    if (sbl) return launch_k<BITS, SBT, MT, T, WPB, false, true>(a, grid, lds, MfmaGather{});
    // scales and biases read from memory (an odd number of groups per row,
    // arrays not 4-byte aligned): one tile and four waves per block
    const dim3 grid1((unsigned)((a.N + 15) / 16));
    return launch_k<BITS, SBT, MT, 1, 4, false, false>(a, grid1, mfma_lds(a, 1, 4, MT, NMT, &sbl), MfmaGather{});
}

constexpr int kSplitBlocks = 256;  // blocks a K split aims at (one per CU)
constexpr int kMaxGemvSplit = 16;

// rows of x per MFMA tile: 4, 8 or 16 (M <= 4 reaches this kernel only as a
// forced route, with the rows past M masked)
int pick_mt(int64_t M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// tiles per block and waves per block (unsplit): 8 K-splitting waves once K
// has at least 64 k-quads (K >= 8192) and M <= 8, else 4; then four 16-row
// tiles per block where that still gives a block per CU, else two or one
// where that gives 192 blocks (more tiles amortise the x operand, which every
// block reads whole).  Measured on MI355X (4-bit g64, us, M = 8 / 16, four
// waves; the choice first): 4096 -> 14336 (T 2) 13.7 / 18.3, T 4 13.6 /
// 19.5, T 1 16.6 / 23.6; 4096 -> 6144 (T 2) 8.5 / 12.1, T 1 9.7 / 13.7;
// 4096 -> 4096 (T 1) 7.3 / 9.4, T 2 8.2 / 11.9; 14336 -> 4096 (T 1) with 8
// waves 16.0 / 22.8, four 17.2 / 21.4 (with a workspace these split).
void pick_tw(int64_t M, int64_t N, int64_t K, int bits, int* T, int* WPB) {
    const int64_t KQ = (K / 32 + 3) / 4;
    const int nmt = M > 4 ? (M > 8 ? 4 : 2) : 1;
    const int wpb = KQ >= 64 && M <= 8 ? 8 : 4;
    int t = (N + 63) / 64 >= 256 ? 4 : 2;
    while (t > 1 && (N + 16 * t - 1) / (16 * t) < 192) t /= 2;
    while (t > 1 && wpb * t * 64 * nmt * 4 > 32768) t /= 2;  // cross-wave reduction LDS
    // four tiles only with four waves (the instantiated kernels)
    if (wpb == 8 && t > 2) t = 2;
    (void)bits;
    *T = t;
    *WPB = wpb;
}

template <int BITS, int SBT, int MT, int T>
hipError_t launch_w(const QmmArgs& a, int wpb) {
    if constexpr (T == 4) {  // four waves only (pick_tw)
        return launch_t<BITS, SBT, MT, T, 4>(a);
    } else {
        return wpb == 8 ? launch_t<BITS, SBT, MT, T, 8>(a) : launch_t<BITS, SBT, MT, T, 4>(a);
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
    int sbl = 1;
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
        case 4: return launch_tt<BITS, SBT, 4>(a);
        case 8: return launch_tt<BITS, SBT, 8>(a);
        default: return launch_tt<BITS, SBT, 16>(a);
    }
}

// The K split (a caller workspace holds the partials): blocks of WPB waves
// own 16 T WPB rows over one of S k ranges each.  Every block reads its
// range of x once for all its rows; without the split a block reads all of x
// for at most 64 rows, and at M = 16 that re-read of x from L2 moves more
// bytes than the codes do (x 2 M bytes per k, the codes K / 2 per row).
// S brings the blocks to about one per CU.
// LDS of a split launch: the block's A rows of x over its k range, then the
// waves' scale / bias areas
size_t split_lds(const QmmArgs& a, int T, int WPB, int MT, int S) {
    const int gsh = __builtin_ctz((unsigned)a.group_size);
    const int npr = sb_pairs((int)a.K, gsh, S, 16 / MT);
    const int qs = wave_kquads((int)a.K, S, cycle_shift(gsh, 16 / MT));
    return (size_t)16 * split_x_stride(qs) + (size_t)WPB * 2 * sb_area_pairs(T, npr) * 4;
}

struct SplitPlan {
    int T, WPB, S;
};
SplitPlan split_plan(const QmmArgs& a) {
    SplitPlan p{1, 8, 1};
    const int mt = pick_mt(a.M);
    const int cl = cycle_shift(__builtin_ctz((unsigned)a.group_size), 16 / mt);
    const int64_t KQ = (a.K / 32 + 3) / 4;
    const int64_t rows = 16 * p.T * p.WPB;
    const int64_t groups = (a.N + rows - 1) / rows;
    int64_t S = (kSplitBlocks + groups / 2) / groups;
    S = S < 1 ? 1 : S > kMaxGemvSplit ? kMaxGemvSplit : S;
    // more ranges where a range's x and scales would not fit the LDS
    for (int64_t s = S; S > 1; ++s) {
        if (s > kMaxGemvSplit) {
            S = 1;
            break;
        }
        const int64_t qs = wave_kquads((int)a.K, (int)s, cl);
        const int64_t se = (KQ + qs - 1) / qs;
        if (split_lds(a, p.T, p.WPB, mt, (int)se) <= 160 * 1024) {
            S = se;
            break;
        }
    }
    p.S = (int)S;
    return p;
}

template <int BITS, int SBT, int MT, int T, int WPB>
hipError_t launch_split_t(const QmmArgs& a, int S, float* part) {
    const dim3 grid((unsigned)((a.N + 16 * T * WPB - 1) / (16 * T * WPB)), (unsigned)S);
    return launch_k<BITS, SBT, MT, T, WPB, false, true, true>(a, grid, split_lds(a, T, WPB, MT, S), MfmaGather{},
                                                              part);
}

template <int BITS, int SBT, int MT>
hipError_t launch_split_mt(const QmmArgs& a, const SplitPlan& p, float* part) {
    (void)p;
    return launch_split_t<BITS, SBT, MT, 1, 8>(a, p.S, part);
}

template <int BITS, int SBT>
hipError_t launch_split(const QmmArgs& a, const SplitPlan& p, float* part) {
    switch (pick_mt(a.M)) {
        case 4: return launch_split_mt<BITS, SBT, 4>(a, p, part);
        case 8: return launch_split_mt<BITS, SBT, 8>(a, p, part);
        default: return launch_split_mt<BITS, SBT, 16>(a, p, part);
    }
}

}  // namespace

// Split where it measured faster (MI355X, 4-bit g64, one tile per wave and
// eight waves per block against the unsplit kernel's best launch shape, us):
// K >= 8192 (M = 16: 14336 -> 4096 20.4 -> 15.5; M = 8: 15.0 -> 14.2) and
// long outputs at M > 8 (M = 16: 4096 -> 14336 18.3 -> 16.1); not at M <= 8
// with K = 4096 (M = 8: 4096 -> 14336 13.3 unsplit, 14.5 split) nor on
// 4096 x 4096 (M = 16: 9.2 unsplit, 10.0 split).
int64_t qmv_split_bytes(const QmmArgs& a) {
    if (a.M < 1 || a.M > 16 || (a.K / a.group_size) % 2 != 0) return 0;
    if (a.K < 8192 && !(a.M > 8 && a.N >= 8192)) return 0;
    const SplitPlan p = split_plan(a);
    return p.S > 1 ? (int64_t)p.S * a.M * a.N * 4 : 0;
}

hipError_t launch_qmv_mfma_split(const QmmArgs& a, void* workspace, int64_t workspace_bytes) {
    const int64_t need = qmv_split_bytes(a);
    const bool al = ((reinterpret_cast<uintptr_t>(a.scales) | reinterpret_cast<uintptr_t>(a.biases)) & 3) == 0;
    if (need == 0 || workspace == nullptr || workspace_bytes < need || !al) return launch_qmv_mfma(a);
    const SplitPlan p = split_plan(a);
    float* part = static_cast<float*>(workspace);
    hipError_t e;
    if (a.bits == 4)
        e = a.sb_dtype == DT_F16 ? launch_split<4, DT_F16>(a, p, part) : launch_split<4, DT_BF16>(a, p, part);
    else
        e = a.sb_dtype == DT_F16 ? launch_split<8, DT_F16>(a, p, part) : launch_split<8, DT_BF16>(a, p, part);
    if (e != hipSuccess) return e;
    return launch_split_reduce(part, p.S, a);
}

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
    // long outputs (a block per CU or more at 128 rows per block): the
    // row-split blocks with one k range, x staged once per 128 rows
    const bool al = ((reinterpret_cast<uintptr_t>(a.scales) | reinterpret_cast<uintptr_t>(a.biases)) & 3) == 0;
    if (a.M >= 5 && a.N >= 128 * kSplitBlocks && (a.K / a.group_size) % 2 == 0 && al &&
        split_lds(a, 1, 8, pick_mt(a.M), 1) <= 160 * 1024) {
        const SplitPlan p{1, 8, 1};
        if (a.bits == 4)
            return a.sb_dtype == DT_F16 ? launch_split<4, DT_F16>(a, p, nullptr) : launch_split<4, DT_BF16>(a, p, nullptr);
        return a.sb_dtype == DT_F16 ? launch_split<8, DT_F16>(a, p, nullptr) : launch_split<8, DT_BF16>(a, p, nullptr);
    }
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_mt<4, DT_F16>(a) : launch_mt<4, DT_BF16>(a);
    return a.sb_dtype == DT_F16 ? launch_mt<8, DT_F16>(a) : launch_mt<8, DT_BF16>(a);
}

}  // namespace miqmm
