// qmvx.hip -- small-M route (M = 1..4) of affine group-quantized matmul:
// bandwidth-first GEMV with the dot products on bf16 MFMA.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])      (transpose=true)
//
// The reference reaches this through its quantized projections during decode
// (src/engine/mlx_lm/utils/mod.rs:70-78; src/engine/mlx_lm/models/llama.rs:
// 195-197,249,293-294,511-517): x is one token, or a few rows when several
// sequences or speculative tokens are verified together.
//
// A GEMV streams W once, so the kernel is built around the loads: every lane
// reads 16 contiguous bytes of one W row per segment (a wave covers 16 rows x
// 64 bytes), non-temporal, two pipeline stages ahead, and the VALU only turns
// codes into exact bf16 MFMA operands (4-bit: 0x4300|q = 128+q with one and-or
// per pair; 8-bit: the top half of the fp32 value of q).
//
// v_mfma_f32_16x16x32_bf16, D[16 x 16] += A[16 x 32] * B[32 x 16]:
//   B: lane (n, h) = (l % 16, l / 16) holds 8 codes of row n.  Within a
//      segment, lane h's 16 bytes are codes [CPL*h, CPL*h + CPL) and MFMA t
//      takes their word t (4-bit) or words 2t, 2t+1 (8-bit).  This permutes k
//      inside the MFMA (lane group h of MFMA t is codes CPL*h + 8t ..), so no
//      lane transposes are needed; A is permuted the same way.
//   A: MFMA rows are (m, slot) pairs, r = m * GS + slot, GS = 16 / MT.  Row
//      (m, slot) carries x[m] only for codes whose quantization group gg has
//      gg % GS == slot, zero elsewhere.  A stage spans at most GS groups, so
//      at its end D[(m, slot)][n] = sum_{k in gg} x[m,k] * code[n,k] for each
//      of the stage's groups, and the dequant is applied once per stage:
//        y[m,n] += s[n,gg] * D[(m,slot)][n] + (b[n,gg] - c*s[n,gg]) * X[m,gg]
//      with c = 128 (4-bit) or 0 (8-bit) and X the group sums of x.  Exact
//      fp32 dequant, as the reference's fp32 fma; ~1 VALU op per code.
//   x lives in LDS (copied in with buffer_load ... lds, then each 8-run is
//   re-paired (x_j, x_{j+4}) to match the 4-bit unpack); X is computed there
//   once per block.  Lanes whose A row is inactive read a 64-byte zero block.
//
// Work: a block is 4 waves = (4 / KS) row tiles of 16 x KS contiguous
// k-ranges; the KS partial sums of a tile are combined through LDS.
#include <atomic>

#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

constexpr int kMaxXElems = 32768;  // MT * K bf16 of x held in LDS (64 KiB)

// s_waitcnt immediate for vmcnt(n) lgkmcnt(0) (vmcnt bits 3:0 and 15:14, expcnt 6:4 left at 7)
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// block barrier for LDS written by this block's ds_write: lgkmcnt(0), then
// s_barrier, fenced against compiler reordering.  (__syncthreads() would also
// wait for every buffer load still in flight that the compiler cannot tell
// apart from an LDS write.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int BITS, int GSH, int MT>
struct Shape {
    static constexpr int GS = 16 / MT;                     // group slots per m
    static constexpr int CPL = 128 / BITS;                 // codes per lane per segment (16 bytes)
    static constexpr int SEG = 4 * CPL;                    // codes per row per segment (64 bytes)
    static constexpr int RUNS = CPL / 8;                   // MFMAs per segment
    static constexpr int CYC_FULL = GS * (1 << GSH) / SEG;  // segments that fill the slots
    static constexpr int CYC = CYC_FULL < 8 ? CYC_FULL : 8;  // segments per stage
    static constexpr int NG = CYC * SEG >> GSH;            // groups per stage
    static constexpr int SB = CYC * 64;                    // bytes per row per stage
    static constexpr int CPR = SB / 16;                    // 16-byte chunks per row per stage
    static constexpr int NI = SB / 64;                     // copy instructions per stage (16 rows)
    static constexpr int RPI = 64 / CPR;                   // rows per copy instruction
    static constexpr int R256 = SB >= 256 ? 1 : 256 / SB;  // rows per 256-byte bank cycle
    static constexpr int LOADS = NI + 4;                   // buffer loads per stage per lane
    static constexpr int STAGE_BYTES = 16 * SB;            // one wave's stage in LDS
    static_assert(CYC >= 1 && NG >= 4 && NG % 4 == 0 && GS % NG == 0, "stage shape");
    static_assert(NI >= 1 && RPI * CPR == 64, "copy shape");
    // LDS slot of chunk c of row n in a stage: chunks are XOR-swizzled per row
    // so that the 16 rows of one operand read fall in 16 distinct bank groups
    static __device__ __forceinline__ int swz(int n) { return (n / R256) & (CPR - 1) & 15; }
};

// LDS layout (bytes): x [MT][K] bf16 (rounded up to 1 KiB), a 64-byte zero
// block, group sums X [MT][GP] fp32, partial sums [4 waves][64] fp32, then
// two W stages per wave
struct Lds {
    uint32_t xbytes, zero, xs, red, stages, total;
    int GP;
};
__host__ __device__ inline Lds lds_layout(int MT, int K, int G, int stage_bytes) {
    Lds l;
    l.xbytes = ((uint32_t)MT * K * 2 + 1023) & ~1023u;
    l.zero = l.xbytes;
    l.xs = l.zero + 64;
    l.GP = (G + 15) & ~15;
    l.red = l.xs + (uint32_t)MT * l.GP * 4;
    l.stages = (l.red + 4 * 64 * 4 + 1023) & ~1023u;
    l.total = l.stages + 4 * 2 * (uint32_t)stage_bytes;
    return l;
}

template <int BITS, int SBT, int MT, int GSH>
__global__ __launch_bounds__(256) void qmvx_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
                                                   const uint16_t* __restrict__ sc,
                                                   const uint16_t* __restrict__ bi, void* __restrict__ y,
                                                   const void* __restrict__ bias, int M, int N, int K, int KS,
                                                   int y_dtype) {
    using S = Shape<BITS, GSH, MT>;
    constexpr int GS = S::GS, CPL = S::CPL, SEG = S::SEG, RUNS = S::RUNS, CYC = S::CYC, NG = S::NG;
    constexpr int SB = S::SB, CPR = S::CPR, NI = S::NI, RPI = S::RPI, LOADS = S::LOADS;
    constexpr float kCentre = BITS == 4 ? 128.f : 0.f;

    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K >> GSH;
    const Lds L = lds_layout(MT, K, G, S::STAGE_BYTES);
    const int NT = (N + 15) / 16;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const auto xr = make_rsrc(x, (uint32_t)M * K * 2);
    const int STG = (K + CYC * SEG - 1) / (CYC * SEG);

    // work: KS > 1 -- one tile per wave and stages [s_lo, s_hi) of it;
    // KS == 1 -- tiles tile0, tile0 + NW, ... (persistent), every stage of each
    int tile0, s_lo, s_hi, n_items, tstride;
    if (KS > 1) {
        tile0 = blockIdx.x * (4 / KS) + wv / KS;
        const int per = (STG + KS - 1) / KS;
        s_lo = min((wv % KS) * per, STG);
        s_hi = min(s_lo + per, STG);
        n_items = tile0 < NT ? s_hi - s_lo : 0;
        tstride = 0;
    } else {
        const int NW = gridDim.x * 4;
        tile0 = blockIdx.x * 4 + wv;
        s_lo = 0;
        s_hi = STG;
        n_items = tile0 < NT ? ((NT - 1 - tile0) / NW + 1) * STG : 0;
        tstride = NW;
    }
    n_items = __builtin_amdgcn_readfirstlane(n_items);
    const int span = max(s_hi - s_lo, 1);  // stages per tile visit (the max keeps dead items well defined)

    const int nl = lane & 15, h = lane >> 4;
    const int m_a = nl / GS, slot_a = nl % GS;               // A row of this lane
    const int m_d = (4 * h) / GS, slot_d0 = (4 * h) % GS;    // D rows 4h + j of this lane

    // ---- x -> LDS (direct copy, 1 KiB per wave instruction), before the W
    // stages so that waiting for it leaves those in flight
    {
        const int chunks = (int)(L.xbytes >> 10);
        for (int c = wv; c < chunks; c += 4) {
            const uint32_t off = (uint32_t)c * 1024 + lane * 16;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(smem + c * 1024), 16, off, 0, 0, 0);
        }
    }

    // a pipeline item: tile and stage; st_* keep the scales / biases of the
    // lane's four D rows (groups gb..gb+3, bf16 or fp16 pairs)
    struct Sb {
        uint32_t s[2], b[2];
    };
    auto item_tile = [&](int i) { return tile0 + (i / span) * tstride; };
    auto item_stage = [&](int i) { return s_lo + i % span; };
    auto d_group = [&](int s, int& gb) {
        const int G0 = s * NG;
        gb = G0 + ((slot_d0 - G0) & (GS - 1));
        return gb - G0 < NG;
    };
    char* const stage_base = smem + L.stages + wv * 2 * S::STAGE_BYTES;
    // copy item i's W stage (16 rows x SB bytes) into LDS region `reg` and
    // load its scales / biases; items past n_items read zeros.  Offsets are
    // pushed out of range by OR-ing in kOOB rather than selected (a select on
    // the offset lets the compiler split a load into branches).
    auto issue = [&](int i, int reg, Sb& sb) {
        const uint32_t dead = i < n_items ? 0u : kOOB;
        const int tile = __builtin_amdgcn_readfirstlane(item_tile(i));
        const int s = __builtin_amdgcn_readfirstlane(item_stage(i));
        const int n0 = tile * 16;
        const uint32_t rows_here =
            (uint32_t)__builtin_amdgcn_readfirstlane(min(max(N - n0, 0), 16));
        const auto wr = make_rsrc((const char*)w + (size_t)n0 * row_bytes, rows_here * row_bytes);
        const auto sr = make_rsrc(sc + (size_t)n0 * G, rows_here * G * 2);
        const auto br = make_rsrc(bi + (size_t)n0 * G, rows_here * G * 2);
        const uint32_t b0 = (uint32_t)s * SB;  // first byte of the stage within a row
        char* dst = stage_base + reg * S::STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int n = j * RPI + lane / CPR;
            const int chunk = (lane % CPR) ^ S::swz(n);
            const uint32_t bo = b0 + (uint32_t)chunk * 16;
            const uint32_t off = ((uint32_t)n * row_bytes + bo) | dead | (bo < row_bytes ? 0u : kOOB);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(dst + j * 1024), 16, off, 0, 0, kNonTemporal);
        }
        int gb;
        const bool act = d_group(s, gb) && gb < G;
        const uint32_t so = (((uint32_t)nl * G + gb) * 2) | dead | (act ? 0u : kOOB);
        const uint32_t so2 = (so + 4) | (gb + 2 < G ? 0u : kOOB);
        sb.s[0] = bload4(sr, so);
        sb.s[1] = bload4(sr, so2);
        sb.b[0] = bload4(br, so);
        sb.b[1] = bload4(br, so2);
    };

    // x landed: re-pair 8-runs for the 4-bit unpack, zero block, group sums
    auto prep_x = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if constexpr (BITS == 4) {
            for (int p = tid; p < MT * K / 8; p += 256) {
                u32x4_t* q = reinterpret_cast<u32x4_t*>(smem + p * 16);
                const u32x4_t v = *q;
                const uint32_t xw[4] = {v[0], v[1], v[2], v[3]};
                uint32_t X[4];
                perm_x_for4(xw, X);
                *q = u32x4_t{X[0], X[1], X[2], X[3]};
            }
        }
        if (tid < 16) reinterpret_cast<uint32_t*>(smem + L.zero)[tid] = 0;
        lds_barrier();
        const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
        float* xs = reinterpret_cast<float*>(smem + L.xs);
        for (int e = tid; e < MT * L.GP; e += 256) {
            const int m = e / L.GP, gg = e % L.GP;
            float v = 0.f;
            if (gg < G) {
                const u32x4_t* p = reinterpret_cast<const u32x4_t*>(smem + ((size_t)m * K + (gg << GSH)) * 2);
                for (int i = 0; i < (1 << GSH) / 8; ++i) {
                    const u32x4_t q = p[i];
#pragma unroll
                    for (int j = 0; j < 4; ++j) v = dot2(q[j], ones[j], v);
                }
            }
            xs[e] = v;
        }
        lds_barrier();
    };

    const uint32_t kMask = vgpr_const(0x000F000Fu), kMagic = kMagic128x2;
    const float* xs = reinterpret_cast<const float*>(smem + L.xs);
    float tot = 0.f;
    const bool owner = MT == 1 ? h == 0 : MT == 2 ? (h & 1) == 0 : true;

    // lanes (n, h) holding the same m: MT=1 all four h, MT=2 h pairs, MT=4 one
    auto lane_sum = [&](float v) {
        if constexpr (MT == 1) {
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
        } else if constexpr (MT == 2) {
            v += __shfl_xor(v, 16);
        }
        return v;
    };

    // item i from LDS region `reg`; stores the tile when it is its last stage
    // (single-tile k-split waves store after the cross-wave sum instead)
    // x operands (A) of segment c of a stage starting at code kst
    auto read_a = [&](int kst, int c, u32x4_t* a) {
        const int k = kst + c * SEG + h * CPL;
        const int gg = k >> GSH;
        const bool act = m_a < M && (gg & (GS - 1)) == slot_a && k < K;
        const char* ap = smem + (act ? ((uint32_t)m_a * K + k) * 2 : L.zero);
#pragma unroll
        for (int t = 0; t < RUNS; ++t) a[t] = *reinterpret_cast<const u32x4_t*>(ap + 16 * t);
    };
    auto compute = [&](int i, int reg, const Sb& sb) {
        const int tile = item_tile(i), s = item_stage(i);
        const char* src = stage_base + reg * S::STAGE_BYTES + nl * SB;
        const int kst = s * CYC * SEG;
        f32x4_t D = {0.f, 0.f, 0.f, 0.f};
        // software pipeline: all of the stage's code chunks up front, the x
        // operands one segment ahead, so LDS latency overlaps the unpack
        u32x4_t code[CYC];
#pragma unroll
        for (int c = 0; c < CYC; ++c)
            code[c] = *reinterpret_cast<const u32x4_t*>(src + 16 * ((4 * c + h) ^ S::swz(nl)));
        u32x4_t a[2][RUNS];
        read_a(kst, 0, a[0]);
#pragma unroll
        for (int c = 0; c < CYC; ++c) {
            if (c + 1 < CYC) read_a(kst, c + 1, a[(c + 1) & 1]);
#pragma unroll
            for (int t = 0; t < RUNS; ++t) {
                uint32_t p[4];
                if constexpr (BITS == 4) {
                    unpack4_magic(code[c][t], p, kMask, kMagic);
                } else {
                    unpack8_pairs(code[c][2 * t], &p[0]);
                    unpack8_pairs(code[c][2 * t + 1], &p[2]);
                }
                D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[c & 1][t]),
                                                          __builtin_bit_cast(bf16x8_t, u32x4_t{p[0], p[1], p[2], p[3]}),
                                                          D, 0, 0, 0);
            }
        }
        // the stage's dequant: rows 4h + j of D hold groups gb + j (or nothing)
        int gb;
        const bool act = d_group(s, gb);
        const f32x4_t X = *reinterpret_cast<const f32x4_t*>(xs + m_d * L.GP + (act ? gb : 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t sw = sb.s[j >> 1], bw = sb.b[j >> 1];
            const float sv = half_to_f32<SBT>((uint16_t)(j & 1 ? sw >> 16 : sw));
            const float bv = half_to_f32<SBT>((uint16_t)(j & 1 ? bw >> 16 : bw));
            // groups past G read as zero scales; X past G is zero
            tot = fmaf(sv, D[j], tot);
            tot = fmaf(fmaf(-kCentre, sv, bv), act ? X[j] : 0.f, tot);
        }
        if (KS == 1 && s == s_hi - 1) {
            const float v = lane_sum(tot);
            tot = 0.f;
            const int n = tile * 16 + nl;
            if (owner && m_d < M && n < N) store_out(y, (int64_t)m_d * N + n, y_dtype, v, bias, n);
        }
    };

    // explicit wait: everything but the youngest `n` buffer loads has landed
    // (loads retire in order), and LDS reads/writes of this wave are done
#define MIQMM_WAIT_VM(n)                                   \
    do {                                                  \
        asm volatile("" ::: "memory");                    \
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(n));  \
        asm volatile("" ::: "memory");                    \
    } while (0)

    Sb A, B;
    issue(0, 0, A);
    if (n_items >= 2) {
        // one-deep pipeline over items, refilled unconditionally (past
        // n_items the loads read zero) so every wait counts the same
        issue(1, 1, B);
        MIQMM_WAIT_VM(2 * LOADS);
        prep_x();
        int i = 0;
        for (; i + 2 <= n_items; i += 2) {
            MIQMM_WAIT_VM(LOADS);
            compute(i, 0, A);
            issue(i + 2, 0, A);
            MIQMM_WAIT_VM(LOADS);
            compute(i + 1, 1, B);
            issue(i + 3, 1, B);
        }
        if (i < n_items) {
            MIQMM_WAIT_VM(LOADS);
            compute(i, 0, A);
        }
    } else {
        MIQMM_WAIT_VM(LOADS);
        prep_x();
        if (n_items == 1) {
            MIQMM_WAIT_VM(0);
            compute(0, 0, A);
        }
    }
#undef MIQMM_WAIT_VM

    if (KS > 1) {
        // k-split partial sums of one tile through LDS
        float* red = reinterpret_cast<float*>(smem + L.red);
        tot = lane_sum(tot);
        red[wv * 64 + lane] = tot;
        lds_barrier();
        if (wv % KS == 0) {
            for (int k = 1; k < KS; ++k) tot += red[(wv + k) * 64 + lane];
            const int n = tile0 * 16 + nl;
            if (owner && m_d < M && n < N) store_out(y, (int64_t)m_d * N + n, y_dtype, tot, bias, n);
        }
    }
}

template <int BITS, int SBT, int MT, int GSH>
hipError_t launch_t(const QmmArgs& a, int KS) {
    using S = Shape<BITS, GSH, MT>;
    const int G = (int)(a.K >> GSH);
    const Lds L = lds_layout(MT, (int)a.K, G, S::STAGE_BYTES);
    // the LDS attribute, once per device (a bit per device id; two threads
    // racing both set it, which is harmless)
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev >= 64) return hipErrorInvalidDevice;
    if (!(attr_set.load(std::memory_order_relaxed) >> dev & 1)) {
        hipError_t e = hipFuncSetAttribute((const void*)qmvx_kernel<BITS, SBT, MT, GSH>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(uint64_t{1} << dev, std::memory_order_relaxed);
    }
    const int64_t tiles = (a.N + 15) / 16;
    int blocks;
    if (KS > 1) {
        blocks = (int)((tiles + 4 / KS - 1) / (4 / KS));
    } else {
        // persistent waves: as many blocks as fit on the chip at once
        const int per_cu = (int)((160 * 1024) / L.total);
        const int64_t cap = (int64_t)num_cus() * (per_cu < 1 ? 1 : per_cu > 4 ? 4 : per_cu);
        const int64_t want = (tiles + 3) / 4;
        blocks = (int)(want < cap ? want : cap);
    }
    hipLaunchKernelGGL((qmvx_kernel<BITS, SBT, MT, GSH>), dim3(blocks), dim3(256), L.total, a.stream,
                       (const uint16_t*)a.x, a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.y,
                       a.bias, (int)a.M, (int)a.N, (int)a.K, KS, a.y_dtype);
    return hipGetLastError();
}

int pick_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }

template <int BITS, int MT, int GSH>
int stage_codes() {
    using S = Shape<BITS, GSH, MT>;
    return S::CYC * S::SEG;
}

int stage_codes_rt(int bits, int mt, int gsh) {
#define MIQMM_SC(B, T, GH) \
    if (bits == B && mt == T && gsh == GH) return stage_codes<B, T, GH>();
    MIQMM_SC(4, 1, 5) MIQMM_SC(4, 1, 6) MIQMM_SC(4, 1, 7) MIQMM_SC(4, 2, 5) MIQMM_SC(4, 2, 6) MIQMM_SC(4, 2, 7)
    MIQMM_SC(4, 4, 5) MIQMM_SC(4, 4, 6) MIQMM_SC(4, 4, 7) MIQMM_SC(8, 1, 5) MIQMM_SC(8, 1, 6) MIQMM_SC(8, 1, 7)
    MIQMM_SC(8, 2, 5) MIQMM_SC(8, 2, 6) MIQMM_SC(8, 2, 7) MIQMM_SC(8, 4, 5) MIQMM_SC(8, 4, 6) MIQMM_SC(8, 4, 7)
#undef MIQMM_SC
    return 0;
}

// k-splits per tile: enough (tile, split) waves to keep ~4096 loads streams
// busy, at most one split per stage, 1, 2 or 4
int pick_ks(int64_t M, int64_t N, int64_t K, int bits, int gsh) {
    const int64_t tiles = (N + 15) / 16;
    const int64_t stg = (K + stage_codes_rt(bits, pick_mt(M), gsh) - 1) / stage_codes_rt(bits, pick_mt(M), gsh);
    int ks = 1;
    while (ks < 4 && tiles * ks < 2048 && stg >= 2 * ks) ks *= 2;
    return ks;
}

template <int BITS, int SBT, int MT>
hipError_t launch_g(const QmmArgs& a, int KS) {
    switch (__builtin_ctz((unsigned)a.group_size)) {
        case 5: return launch_t<BITS, SBT, MT, 5>(a, KS);
        case 6: return launch_t<BITS, SBT, MT, 6>(a, KS);
        default: return launch_t<BITS, SBT, MT, 7>(a, KS);
    }
}

template <int BITS, int SBT>
hipError_t launch_m(const QmmArgs& a) {
    const int ks = pick_ks(a.M, a.N, a.K, a.bits, __builtin_ctz((unsigned)a.group_size));
    switch (pick_mt(a.M)) {
        case 1: return launch_g<BITS, SBT, 1>(a, ks);
        case 2: return launch_g<BITS, SBT, 2>(a, ks);
        default: return launch_g<BITS, SBT, 4>(a, ks);
    }
}

}  // namespace

bool qmvx_supported(int64_t M, int64_t K, int group_size) {
    const int64_t G = K / group_size;
    return M >= 1 && M <= 4 && pick_mt(M) * K <= kMaxXElems && G % 2 == 0;
}

void qmvx_config(const QmmArgs& a, int* m_tile, int* k_splits, int* stage_codes) {
    const int gsh = __builtin_ctz((unsigned)a.group_size);
    if (m_tile) *m_tile = pick_mt(a.M);
    if (k_splits) *k_splits = pick_ks(a.M, a.N, a.K, a.bits, gsh);
    if (stage_codes) *stage_codes = stage_codes_rt(a.bits, pick_mt(a.M), gsh);
}

hipError_t launch_qmvx(const QmmArgs& a) {
    if (a.bits == 4) return a.sb_dtype == DT_F16 ? launch_m<4, DT_F16>(a) : launch_m<4, DT_BF16>(a);
    return a.sb_dtype == DT_F16 ? launch_m<8, DT_F16>(a) : launch_m<8, DT_BF16>(a);
}

}  // namespace miqmm
