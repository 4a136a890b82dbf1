// qmm.hip -- large-M (prefill) route of affine group-quantized matmul on bf16 MFMA.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])      (transpose=true)
//
// Reached by the reference's quantized projections during chunked prefill
// (src/engine/mlx_lm/models/llama.rs:195-197,249,293-294 with x [1, L, K],
// L up to prefill_chunk; src/engine/mlx_native.rs:1918-1922,2094-2102).
//
// Block tile 256 x BN x 64: for BN = 256 (and 8-bit codes) eight waves in a
// 2 x 4 grid, each a 128 x 64 sub-tile (two waves per SIMD, so one wave's
// dequant VALU and LDS traffic overlap the other's MFMAs); for 4-bit BN = 128
// four waves in a 2 x 2 grid, 128 x 64 each (waves_per_block).  Sub-tiles are
// computed with v_mfma_f32_32x32x16_bf16, the 128 fp32 accumulators per lane
// in AGPRs; each 16-wide k step a wave reads 4 A and 2 B fragments of 1 KiB
// for 8 MFMAs.
//
// One block per CU, so the pipeline, not other blocks, hides memory latency.
// At k-step t the block
//   - loads the packed codes, scales and biases of step t+2 into registers,
//   - copies the x tile of step t+2 straight from HBM into a 3-stage LDS ring
//     (buffer_load ... lds; no registers, no VALU),
//   - runs the MFMAs of step t from LDS,
//   - dequantizes the codes of step t+1 in fp32 (fma(s, q, b), the reference's
//     formula) and stores them into the other half of a 2-stage LDS buffer
//     as bf16, k-contiguous per output column,
// with one barrier per k-step.  LDS: 3 x 32 KiB of x + 2 x BN*128 B of W.
//
// LDS layout of a tile [R rows, 64 k] (bf16): four k-slices of 16, each
// [R rows x 32 B]; within a slice row r holds its two 16-byte halves (k 0-7,
// 8-15) swapped when bit 3 of r is set, and in the W tile swapped once more in
// slices 2 and 3.  gfx950's LDS serves sixteen 16-byte lanes per pass (64
// banks): a fragment read of 16 consecutive rows covers all 64 banks once, and
// every fragment address is one of two per-lane bases plus compile-time
// offsets (slice * R * 32 + tile row * 32), which keeps address registers out
// of the way of the 256 accumulators.  The extra swap is for the W stores: the
// two lanes of a row write slices s and s + 2 (R * 64 bytes apart, the same
// banks); with it they write different halves, so a store's sixteen lanes per
// pass cover the 64 banks once.
//
// Rounding the dequantized weight to bf16 before the MFMA follows MLX's qmm,
// which dequantizes W tiles into threadgroup memory in the activation type.
#include <algorithm>
#include <atomic>

#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

constexpr int kBM = 256;
#ifndef QMM_XST128
#define QMM_XST128 3
#endif
// x ring depth (LDS stages of the x tile) per tile width: the x tile of step
// t is copied XST-1 steps ahead, and the codes XST steps ahead
template <int BN>
constexpr int x_stages() { return BN == 128 ? QMM_XST128 : 3; }
constexpr int kBK = 64;
constexpr int kRowBytes = kBK * 2;  // one LDS row: 64 bf16

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
        out[wi][0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
        out[wi][1] = pack_bf16x2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
        out[wi][2] = pack_bf16x2(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
        out[wi][3] = pack_bf16x2(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
    }
}

// 16 bytes of 8-bit codes (16 codes) -> 16 bf16 of fma(s, q, b)
__device__ __forceinline__ void dequant_chunk8(const u32x4_t& q, float s, float b, u32x4_t out[2]) {
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const uint32_t v = q[wi];
        out[wi >> 1][(wi & 1) * 2 + 0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(v), b), fmaf(s, ubyte_f32<1>(v), b));
        out[wi >> 1][(wi & 1) * 2 + 1] = pack_bf16x2(fmaf(s, ubyte_f32<2>(v), b), fmaf(s, ubyte_f32<3>(v), b));
    }
}

// s_waitcnt immediate for vmcnt(n) lgkmcnt(0) (vmcnt bits 3:0 and 15:14, expcnt 6:4 left at 7)
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// s_waitcnt with the given immediate, then s_barrier, fenced against compiler
// reordering of memory operations (the barrier builtin alone is not a memory
// barrier for the compiler; __syncthreads() would add a release fence that
// waits for the x copies still in flight)
#define MIQMM_WAIT_BARRIER(imm)                   \
    do {                                          \
        asm volatile("" ::: "memory");            \
        __builtin_amdgcn_s_waitcnt(imm);          \
        __builtin_amdgcn_s_barrier();             \
        asm volatile("" ::: "memory");            \
    } while (0)

// byte offset of the 16-byte piece (k-slice kk, half fk) of row r in a W tile of R rows
__device__ __forceinline__ uint32_t lds_off(int R, int r, int kk, int fk) {
    return kk * R * 32 + r * 32 + ((fk ^ ((r >> 3) & 1) ^ ((kk >> 1) & 1)) << 4);
}

template <int BITS, int W_PER>
struct WRegs {
    u32x4_t q[W_PER];
    uint16_t s[W_PER], b[W_PER];
};

// The expert-grouped matmul (GATHER): each M tile holds up to 256 selections
// of one expert, listed by gather_plan_kernel; its x rows are gathered through
// the selection list and its output rows scattered back, and W, scales and
// biases are the expert's slices of the stacked tensors.
struct QmmGather {
    const int32_t* perm;    // selection ids grouped by expert
    const int32_t* seg;     // seg[e] .. seg[e+1]: expert e's range of perm (e == E: invalid ids)
    const int32_t* tiles;   // (expert, first position in perm) of each M tile
    const int32_t* ntiles;  // number of M tiles
    int top_k, x_per_index, experts;
    uint32_t x_bytes;       // bytes of x (all its matrices)
};

// Split of the k-steps over gridDim.z blocks per output tile (ks > 1): each
// block writes its fp32 partial tile to part[z]; a second kernel
// (qmm_split_reduce_kernel) adds the ks partials of every output in split
// order and writes y.  The partials live in a workspace the caller owns.
struct QmmSplit {
    float* part;  // [ks][M][N] fp32 partial sums
    int ks;       // number of k ranges (1: no split)
};

// fp32 partials are written and read at device scope (cache policy SC1:
// written through to, and read from, the level coherent across the XCDs'
// L2s), so no L2 write-back or invalidate is needed between the splits
constexpr int kDeviceScope = 16;

__device__ __forceinline__ void part_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4_t& v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, kDeviceScope);
}
__device__ __forceinline__ f32x4_t part_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDeviceScope));
}
__device__ __forceinline__ void part_store1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kDeviceScope);
}
__device__ __forceinline__ float part_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kDeviceScope));
}

__device__ __forceinline__ int sload(const int32_t* p) {
    return __builtin_amdgcn_readfirstlane(*(const __attribute__((address_space(4))) int32_t*)p);
}

// Waves per block.  Eight (two per SIMD: one wave's dequant VALU and LDS
// traffic overlap the other's MFMAs) for 256-wide tiles, whose waves keep
// 128 x 64 tiles, and for 8-bit codes; four for 4-bit 128-wide tiles, where
// eight waves would shrink the wave tile to 64 x 64 and raise the LDS reads
// per MFMA (measured on MI355X, M = 2048: 830 vs 720 TFLOP/s at N = 14336,
// 750 vs 870 at 14336 -> 4096).
template <int BITS, int BN>
constexpr int waves_per_block() { return BN == 256 || BITS == 8 ? 8 : 4; }

// dynamic LDS: the x ring, two W stages, and one 16-byte slot per idle W thread
template <int BITS, int BN>
constexpr size_t qmm_lds_bytes() {
    constexpr int NT = 64 * waves_per_block<BITS, BN>();
    constexpr int W_CH = BN * (kBK >> (BITS == 4 ? 5 : 4));
    constexpr int W_PER = W_CH >= NT ? W_CH / NT : 1;
    constexpr int idle = NT - W_CH / W_PER;
    return (size_t)x_stages<BN>() * kBM * kRowBytes + 2 * (size_t)BN * kRowBytes + (idle > 0 ? idle : 0) * 16;
}

template <int BITS, int SBT, int BN, bool GATHER>
__global__ __launch_bounds__((64 * waves_per_block<BITS, BN>()), 1) void qmm_kernel(const uint16_t* __restrict__ x,
                                                     const uint32_t* __restrict__ w,
                                                     const uint16_t* __restrict__ sc,
                                                     const uint16_t* __restrict__ bi,
                                                     void* __restrict__ y, const void* __restrict__ bias,
                                                     int M, int N, int K, int gs_shift, int y_dtype,
                                                     const QmmGather gq, const QmmSplit sp) {
    constexpr int NW = waves_per_block<BITS, BN>(), NT = 64 * NW;
    // wave grid GM x GN: 2 x 2 for four waves; 2 x 4 (BN = 256) or 4 x 2 (BN = 128) for eight
    constexpr int GN = NW == 4 ? 2 : (BN == 256 ? 4 : 2), GM = NW / GN;
    constexpr int WM = kBM / GM, WN = BN / GN;    // wave tile WM x WN
    constexpr int TM = WM / 32, TN = WN / 32;     // 32x32 MFMA tiles per wave
    constexpr int XI = 32 / NW;                   // 1 KiB x copies per wave per k-step
    constexpr int CPC_SHIFT = BITS == 4 ? 5 : 4;  // codes per 16-byte chunk
    constexpr int CPR = kBK >> CPC_SHIFT;         // code chunks per W row per k-step (2 or 4)
    constexpr int W_CH = BN * CPR;                // code chunks per k-step
    constexpr int W_PER = W_CH >= NT ? W_CH / NT : 1;  // code chunks per thread (1, 2 or 4)
    // threads from W_CH / W_PER on (4-bit, BN = 128, eight waves) load out of
    // range (zeros) and store into a dummy LDS slot, with no branch
    constexpr int XST = x_stages<BN>();           // x ring stages
    constexpr int XD = XST - 1;                   // k-steps the x tile is copied ahead
    constexpr int WD = XST;                       // k-steps the codes are loaded ahead
    constexpr int A_STAGE = kBM * kRowBytes;      // 32 KiB
    constexpr int B_STAGE = BN * kRowBytes;
    constexpr int B_BASE = XST * A_STAGE;
    constexpr int DUMMY = B_BASE + 2 * B_STAGE;   // LDS slots of the idle threads' W stores
    static_assert(NW * 32 * (WN + 32) * 4 <= (int)qmm_lds_bytes<BITS, BN>(), "epilogue staging fits");
    static_assert(W_PER >= 1 && CPR % W_PER == 0, "code chunks per thread");
    // vector-memory loads one thread issues per k-step: XI x copies + codes,
    // scales and biases of W_PER chunks
    constexpr int LOADS = XI + 3 * W_PER;
    static_assert((XD - 1) * LOADS < 64, "vmcnt range");
    static_assert(WD >= XD + 1, "codes of t+2 issued before the x tile of t+1");

    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid / GN, wn = wid % GN;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * BN;
    // this block's k-steps: kt0 .. kt0 + KT (all of them unless split)
    int KT = (K + kBK - 1) / kBK, kt0 = 0;
    if (sp.ks > 1) {
        const int chunk = (KT + sp.ks - 1) / sp.ks;
        kt0 = blockIdx.z * chunk;
        KT = min(KT, kt0 + chunk) - kt0;
    }
    const uint32_t xrow = (uint32_t)K * 2;
    const uint32_t wrow = (uint32_t)K * BITS / 8;
    const int G = K >> gs_shift;
    int mrows = min(kBM, M - m0), nrows = min(BN, N - n0);
    int p0 = 0;           // GATHER: first position of this tile in the selection list
    size_t erow0 = 0;     // GATHER: first W row of the expert
    if constexpr (GATHER) {
        if ((int)blockIdx.y >= sload(gq.ntiles)) return;  // block-uniform: past the listed tiles
        const int e = sload(gq.tiles + 2 * blockIdx.y);
        p0 = sload(gq.tiles + 2 * blockIdx.y + 1);
        mrows = min(kBM, sload(gq.seg + e + 1) - p0);
        if (e >= gq.experts) nrows = 0;  // out-of-range ids: zero rows
        erow0 = (size_t)min(e, gq.experts - 1) * N;
    }
    const auto xr = GATHER ? make_rsrc(x, gq.x_bytes) : make_rsrc(x + (size_t)m0 * K, (uint32_t)mrows * xrow);
    const auto wr = make_rsrc((const char*)w + (erow0 + n0) * wrow, (uint32_t)nrows * wrow);
    const auto sr = make_rsrc(sc + (erow0 + n0) * G, (uint32_t)nrows * G * 2);
    const auto br = make_rsrc(bi + (erow0 + n0) * G, (uint32_t)nrows * G * 2);
    // x copies: wave `wid` fills rows xrow0 .. xrow0 + 32*XI of k-slice wid % 4
    const int xslice = wid & 3, xrow0 = (wid >> 2) * XI * 32;
    // GATHER: byte offset of the x row of each of this lane's copy rows
    uint32_t xbase[XI];
    if constexpr (GATHER) {
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const int row = xrow0 + j * 32 + (lane >> 1);
            const int sel = row < mrows ? gq.perm[p0 + row] : -1;
            const int xi = gq.x_per_index ? sel : sel / gq.top_k;
            xbase[j] = sel >= 0 ? (uint32_t)xi * xrow : kOOB;
        }
    }

    // x tile -> LDS: the k-slice [256 rows x 32 B] is filled by 32-row 1 KiB
    // instructions; lane i of an instruction lands at byte 16*i, i.e. row i/2
    // of its 32-row group, stored half i%2, so it loads logical half
    // (i%2) ^ (bit 3 of the row)
    auto issue_a = [&](int kt) {
        const int kb = (kt0 + kt) * kBK + xslice * 16;
        char* slice = smem + (kt % XST) * A_STAGE + xslice * kBM * 32 + xrow0 * 32;
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const int row = xrow0 + j * 32 + (lane >> 1);
            const int fk = (lane & 1) ^ ((row >> 3) & 1);
            const int k = kb + fk * 8;
            uint32_t off;
            if constexpr (GATHER) off = k < K ? xbase[j] + (uint32_t)k * 2 : kOOB;
            else off = k < K ? (uint32_t)row * xrow + (uint32_t)k * 2 : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(slice + j * 1024), 16, off, 0, 0, 0);
        }
    };

    // this thread's W row and first code chunk (adjacent lanes share a row:
    // the code loads of a wave cover 32-byte runs of 32 rows; mapping
    // consecutive lanes to consecutive rows instead, which makes the LDS
    // stores below conflict-free, measured 15 % slower on MI355X)
    const int wrow_t = tid / (CPR / W_PER);
    const int wch0 = (tid % (CPR / W_PER)) * W_PER;
    const bool widle = tid >= W_CH / W_PER;
    const uint32_t wid_oob = widle ? kOOB : 0u;
    using WR = WRegs<BITS, W_PER>;
    auto load_w = [&](int kt, WR& r) {
        const int kb = (kt0 + kt) * kBK;
#pragma unroll
        for (int i = 0; i < W_PER; ++i) {
            const int kc = kb + ((wch0 + i) << CPC_SHIFT);
            // past the end of K (last step when K % 64 == 32): offsets pushed out of range
            const uint32_t oob = (kc < K ? 0u : kOOB) | wid_oob;
            r.q[i] = bload16(wr, ((uint32_t)wrow_t * wrow + (uint32_t)kc * BITS / 8) | oob);
            const uint32_t so = (((uint32_t)wrow_t * G + (uint32_t)(kc >> gs_shift)) * 2) | oob;
            r.s[i] = bload2(sr, so);
            r.b[i] = bload2(br, so);
        }
    };
    // dequantize one 16-byte LDS chunk (8 codes, one W word for 4-bit, two
    // half-words for 8-bit) of the codes in `r` into B stage kt&1.  Chunk
    // index e runs over the thread's W_PER*CPC/8 chunks.
    constexpr int W_CHUNKS = W_PER * (1 << CPC_SHIFT) / 8;  // LDS chunks per thread per k-step
    auto store_w_chunk = [&](int kt, const WR& r, int e) {
        char* sB = smem + B_BASE + (kt & 1) * B_STAGE;
        const int i = e / ((1 << CPC_SHIFT) / 8), j = e % ((1 << CPC_SHIFT) / 8);
        const float s = half_to_f32<SBT>(r.s[i]), b = half_to_f32<SBT>(r.b[i]);
        const int c = (((wch0 + i) << CPC_SHIFT) >> 3) + j;
        u32x4_t o;
        if constexpr (BITS == 4) {
            const uint32_t word = r.q[i][j];
            uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
            // opaque to known-bits analysis, so each code converts with one
            // v_cvt_f32_ubyteN instead of a 4-bit extract plus a convert
            asm("" : "+v"(lo), "+v"(hi));
            o[0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
            o[1] = pack_bf16x2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
            o[2] = pack_bf16x2(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
            o[3] = pack_bf16x2(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
        } else {
            const uint32_t w0 = r.q[i][2 * j], w1 = r.q[i][2 * j + 1];
            o[0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w0), b), fmaf(s, ubyte_f32<1>(w0), b));
            o[1] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w0), b), fmaf(s, ubyte_f32<3>(w0), b));
            o[2] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w1), b), fmaf(s, ubyte_f32<1>(w1), b));
            o[3] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w1), b), fmaf(s, ubyte_f32<3>(w1), b));
        }
        char* dst = widle ? smem + DUMMY + (tid - W_CH / W_PER) * 16 : sB + lds_off(BN, wrow_t, c >> 1, c & 1);
        *reinterpret_cast<u32x4_t*>(dst) = o;
    };
    auto store_w = [&](int kt, const WR& r) {
#pragma unroll
        for (int e = 0; e < W_CHUNKS; ++e) store_w_chunk(kt, r, e);
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // fragment of a 32x32x16 MFMA: lane l holds row l%32, k = 8*(l/32) .. +8 of the 16-wide step
    const int frow = lane & 31, fk = lane >> 5;
    // per-lane part of a fragment address: row frow of a 32-row tile, half fk
    const uint32_t fbase = (uint32_t)frow * 32 + ((fk ^ ((frow >> 3) & 1)) << 4);
    const uint32_t fbase_w2 = fbase ^ 16u;  // W tile, k-slices 2 and 3
    auto read_frags = [&](int kt, int kk, bf16x8_t* af, bf16x8_t* bf) {
        const char* sA = smem + (kt % XST) * A_STAGE + fbase;
        const char* sB = smem + B_BASE + (kt & 1) * B_STAGE + ((kk & 2) ? fbase_w2 : fbase);
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const bf16x8_t*>(sA + kk * kBM * 32 + (wm * WM + i * 32) * 32);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *reinterpret_cast<const bf16x8_t*>(sB + kk * BN * 32 + (wn * WN + j * 32) * 32);
    };

    // step t: codes of t+WD into `nxt`, x of t+XD into the ring, MFMAs of t,
    // dequant of t+1 (held in `cur`) spread over the four 16-wide sub-steps so
    // its VALU work issues between MFMAs.  The loads are issued on every step,
    // also past the last one (out-of-range offsets read zeros into a stage
    // nobody reads again): the compiler's wait counts for `cur` are then the
    // same on every path.  The end-of-step barrier is a bare s_barrier with
    // explicit waits, because __syncthreads() would also wait for the x copies
    // still in flight, which are LDS writes.
    constexpr int E_PER_KK = (W_CHUNKS + 3) / 4;
#ifdef QMM_VPM
    constexpr int kValuPerMfma = QMM_VPM;
#else
    // about 24 VALU per dequantized 16-byte chunk, spread over the sub-step's MFMAs
    constexpr int kValuPerMfma = (E_PER_KK * 24 + TM * TN - 1) / (TM * TN);
#endif
    auto step = [&](int t, const WR& cur, WR& nxt) {
        load_w(t + WD, nxt);
        issue_a(t + XD);
        bf16x8_t af[2][TM], bf[2][TN];
        read_frags(t, 0, af[0], bf[0]);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            if (kk + 1 < kBK / 16) read_frags(t, kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk & 1][i], bf[kk & 1][j], acc[i][j], 0,
                                                                      0, 0);
            // unconditional: on the last step this dequantizes the zeros
            // loaded past K into the W stage nobody reads again
#pragma unroll
            for (int e = kk * E_PER_KK; e < (kk + 1) * E_PER_KK && e < W_CHUNKS; ++e) store_w_chunk(t + 1, cur, e);
            // issue order: each MFMA followed by a few VALU (the dequant runs
            // on the vector ALU while the matrix core works) and one LDS read
#pragma unroll
            for (int g = 0; g < TM * TN; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU
                if (g < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // the x tile of step t+1 (direct-to-LDS, issued XD-1 steps ago) must
        // have landed while the loads of the last XD-1 steps stay in flight
        // (loads retire in order; that also covers the codes of t+2, issued
        // WD-1 >= XD steps ago); the LDS writes of the dequantized W of t+1
        // must be done before other waves read them
        MIQMM_WAIT_BARRIER(waitcnt_vm_lgkm0((XD - 1) * LOADS));
    };

    // The codes of step s live in wq[s % WD].  The prologue issues the loads
    // of the steps before 0 in the loop's own order (skipping negative
    // targets), so the loop starts with the wait counts it keeps.
    WR wq[WD];
#pragma unroll
    for (int s = -WD; s < 0; ++s) {
        load_w(s + WD, wq[s + WD]);
        if (s + XD >= 0) issue_a(s + XD);
    }
    store_w(0, wq[0]);
    MIQMM_WAIT_BARRIER(waitcnt_vm_lgkm0((XD - 1) * LOADS));  // x of step 0 and codes of step 1 landed
    int t = 0;
    for (; t + WD - 1 < KT; t += WD) {
#pragma unroll
        for (int u = 0; u < WD; ++u) step(t + u, wq[(u + 1) % WD], wq[u]);
    }
#pragma unroll
    for (int u = 0; u + 1 < WD; ++u)
        if (t + u < KT) step(t + u, wq[(u + 1) % WD], wq[u]);
    // the prefetches past the last step (out of range, zero-filled) still
    // write the x ring; they must land before the ring is reused below
    MIQMM_WAIT_BARRIER(0x0070);  // vmcnt(0) lgkmcnt(0)

    // Epilogue, one 32-row band at a time: each wave stages its fp32 results
    // in its own LDS region (the pipeline buffers are free after the last
    // barrier), then writes runs of 8 columns per lane.  D of a 32x32 MFMA:
    // lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.  Rows
    // are padded to WN+32 floats so the two row groups of one store fall in
    // different banks.
    constexpr int ES = WN + 32;
    float* stage = reinterpret_cast<float*>(smem) + wid * 32 * ES;
    const int wrow0 = m0 + wm * WM, wcol0 = n0 + wn * WN;
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    static_assert(NW * 32 * ES * 4 <= (int)qmm_lds_bytes<BITS, BN>(), "epilogue staging fits");
    // unsplit: the output; split: this block's fp32 partial tile -> part[z]
    const bool partial = sp.ks > 1;
    {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    stage[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * ES + j * 32 + (lane & 31)] = acc[i][j][r];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
            __builtin_amdgcn_wave_barrier();
            constexpr int RUNS = WN / 8;
#pragma unroll 1
            for (int p = lane; p < 32 * RUNS; p += 64) {
                const int row = p / RUNS, c8 = p % RUNS;
                int gr = wrow0 + i * 32 + row;
                const int gc = wcol0 + c8 * 8;
                if constexpr (GATHER) {  // the tile's row -> its selection, one output row each
                    const int lr = gr - m0;
                    if (lr >= mrows || gc >= N) continue;
                    gr = gq.perm[p0 + lr];
                } else {
                    if (gr >= M || gc >= N) continue;
                }
                f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(stage + row * ES + c8 * 8);
                f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(stage + row * ES + c8 * 8 + 4);
                const int64_t o = (int64_t)gr * N + gc;
                const uint32_t po = (uint32_t)o * 4;  // byte offset in one split's partials
                if (partial) {
                    const auto pr = make_rsrc(sp.part + (int64_t)blockIdx.z * M * N, (uint32_t)M * N * 4);
                    if (vec) {
                        part_store4(pr, po, v0);
                        part_store4(pr, po + 16, v1);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (gc + e < N) part_store1(pr, po + 4 * e, e < 4 ? v0[e] : v1[e - 4]);
                    }
                    continue;
                }
                const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                if (vec && y_dtype != DT_F32) {  // gc + 8 <= N since N % 8 == 0
                    u32x4_t h;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        h[e] = (uint32_t)out_half_bits(y_dtype, v[2 * e], bias, gc + 2 * e) |
                               ((uint32_t)out_half_bits(y_dtype, v[2 * e + 1], bias, gc + 2 * e + 1) << 16);
                    *reinterpret_cast<u32x4_t*>((uint16_t*)y + o) = h;
                } else if (vec) {
                    f32x4_t a = v0, b = v1;
                    if (bias) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            a[e] += ((const float*)bias)[gc + e];
                            b[e] += ((const float*)bias)[gc + 4 + e];
                        }
                    }
                    *reinterpret_cast<f32x4_t*>((float*)y + o) = a;
                    *reinterpret_cast<f32x4_t*>((float*)y + o + 4) = b;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gc + e < N) store_out(y, o + e, y_dtype, v[e], bias, gc + e);
                }
            }
            __builtin_amdgcn_wave_barrier();  // reads of this band before the next band's writes
        }
    }
}

// y = sum over z of part[z] (z = 0 .. ks-1 in order, the same bits for any
// grid), rounded to y's dtype (+ bias as a separate rounding): one thread per
// run of 4 outputs of a row, all planes' loads in flight at once (a few rows
// of x give few threads, each with ks planes to add)
__global__ __launch_bounds__(256) void qmm_split_reduce_kernel(const float* __restrict__ part, int ks, int M, int N,
                                                               void* __restrict__ y, const void* __restrict__ bias,
                                                               int y_dtype) {
    const int runs = (N + 3) / 4;
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (int64_t)M * runs) return;
    const int gr = (int)(q / runs), gc = (int)(q % runs) * 4;
    const int64_t o = (int64_t)gr * N + gc;
    const int64_t plane = (int64_t)M * N;
    const bool vec = (N & 3) == 0;
    auto ld = [&](int z) {
        const float* p = part + z * plane + o;
        if (vec) return *reinterpret_cast<const f32x4_t*>(p);
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (gc + e < N) a[e] = p[e];
        return a;
    };
    // every plane's load in flight before the first add (ks <= 16 here)
    constexpr int kPlanes = 16;
    f32x4_t a[kPlanes];
#pragma unroll
    for (int z = 0; z < kPlanes; ++z)
        if (z < ks) a[z] = ld(z);
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int z = 0; z < kPlanes; ++z)
        if (z < ks)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += a[z][e];
    for (int z = kPlanes; z < ks; ++z) {
        const f32x4_t b = ld(z);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (gc + e < N) store_out(y, o + e, y_dtype, v[e], bias, gc + e);
}


template <int BITS, int SBT, int BN, bool GATHER>
hipError_t launch_t(const QmmArgs& a, const QmmGather& gq, int64_t m_tiles, const QmmSplit& sp) {
    constexpr size_t lds = qmm_lds_bytes<BITS, BN>();
    static_assert(lds <= 160 * 1024, "LDS per workgroup");
    // the LDS attribute, once per device (a bit per device id; two threads
    // racing both set it, which is harmless)
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev >= 64) return hipErrorInvalidDevice;
    if (!(attr_set.load(std::memory_order_relaxed) >> dev & 1)) {
        hipError_t e = hipFuncSetAttribute((const void*)qmm_kernel<BITS, SBT, BN, GATHER>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(uint64_t{1} << dev, std::memory_order_relaxed);
    }
    const dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)m_tiles, (unsigned)sp.ks);
    const int gs_shift = __builtin_ctz((unsigned)a.group_size);
    constexpr int threads = 64 * waves_per_block<BITS, BN>();
    hipLaunchKernelGGL((qmm_kernel<BITS, SBT, BN, GATHER>), grid, dim3(threads), lds, a.stream, (const uint16_t*)a.x,
                       a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.y, a.bias, (int)a.M, (int)a.N,
                       (int)a.K, gs_shift, a.y_dtype, gq, sp);
    return hipGetLastError();
}

// One block groups the selections by expert for the expert-grouped kernels:
// a histogram of the indices in LDS, its prefix sum (the experts' ranges of
// the selection list; ids outside [0, E) form range E), the selections
// placed into their ranges, and the list of tiles of up to `tr` rows.  The
// order of selections inside a range is arbitrary; every output row is
// computed on its own, so the results do not depend on it.
__global__ __launch_bounds__(1024) void gather_plan_kernel(const int32_t* idx, int S, int E, int tr, int32_t* seg,
                                                           int32_t* ntiles, int32_t* perm, int32_t* tiles) {
    extern __shared__ int32_t cnt[];  // [E + 1] counts, then [E + 1] fill positions
    int32_t* pos = cnt + E + 1;
    for (int e = threadIdx.x; e <= E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < S; i += blockDim.x) {
        const int e = idx[i];
        atomicAdd(&cnt[e >= 0 && e < E ? e : E], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0, t = 0;
        for (int e = 0; e <= E; ++e) {
            seg[e] = run;
            pos[e] = run;
            for (int r = 0; r < cnt[e]; r += tr) {
                tiles[2 * t] = e;
                tiles[2 * t + 1] = run + r;
                ++t;
            }
            run += cnt[e];
        }
        seg[E + 1] = run;
        *ntiles = t;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < S; i += blockDim.x) {
        const int e = idx[i];
        perm[atomicAdd(&pos[e >= 0 && e < E ? e : E], 1)] = i;
    }
}

// Tile width and k split by a rounds model of MI355X: tiles run in rounds
// of one block per CU; a 128-wide tile (four waves) over K takes about
// 0.0202 us per unit of K, a 256-wide one (eight waves) 1.3x that; a split
// into ks k ranges divides the tile time by ks and adds the partial traffic
// (ks fp32 values per output written, then read back by the reduce kernel,
// at 2.4 TB/s effective: fitted to forced plans on MI355X, 2.2-3.1 TB/s at
// M = 256-1024) and the reduce kernel's launch.  E.g. M = 2048: N = 14336
// and 6144 -> 256 wide, N = 4096 -> 128 wide at K = 4096 and 256 wide in two
// k ranges at K = 14336; M = 1024, N = K = 4096 -> 128 wide in two k ranges
// (60.8 us against 67.2 unsplit); M = 256, N = 4096, K = 4096 -> 128 wide in
// four k ranges.
struct QmmPlan {
    int bn, ks;
};

QmmPlan plan_qmm(int64_t M, int64_t N, int64_t K, int max_ks) {
    const int64_t mt = (M + kBM - 1) / kBM, KT = (K + kBK - 1) / kBK;
    const int64_t cus = num_cus();
    QmmPlan best{128, 1};
    double best_us = 1e300;
    for (int bn : {128, 256}) {
        const int64_t tiles = mt * ((N + bn - 1) / bn);
        for (int ks = 1; ks <= max_ks; ++ks) {
            if (ks > 1 && (KT < 8 * ks || (double)ks * M * N * 4 >= 2147483648.0)) break;  // >= 8 k-steps per range
            const double rounds = (double)((tiles * ks + cus - 1) / cus);
            double us = rounds * (bn == 256 ? 1.3 : 1.0) * 0.0202 * (double)K / ks;
            if (ks > 1) us += (double)M * N * 4 * (2 * ks) / 2.4e6 + 2.0;
            if (us < best_us) {
                best_us = us;
                best = {bn, ks};
            }
        }
    }
    return best;
}

}  // namespace

// y = the sum of ks fp32 partial planes [ks][M][N] (in order), rounded to y's
// dtype, plus the bias
hipError_t launch_split_reduce(const float* part, int ks, const QmmArgs& a) {
    const int64_t threads = a.M * ((a.N + 3) / 4);
    hipLaunchKernelGGL(qmm_split_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, a.stream,
                       part, ks, (int)a.M, (int)a.N, a.y, a.bias, a.y_dtype);
    return hipGetLastError();
}

namespace {

constexpr int kMaxSplit = 4;

// the plan with k ranges only where `workspace_bytes` holds their partials
QmmPlan plan_with_workspace(const QmmArgs& a, int64_t workspace_bytes) {
    QmmPlan pl = plan_qmm(a.M, a.N, a.K, kMaxSplit);
    if (pl.ks > 1 && (double)pl.ks * a.M * a.N * 4 > (double)workspace_bytes) pl = plan_qmm(a.M, a.N, a.K, 1);
    return pl;
}

template <int BITS, int SBT>
hipError_t launch_bn(const QmmArgs& a, void* workspace, int64_t workspace_bytes) {
    const QmmGather none{};
    const int64_t mt = (a.M + kBM - 1) / kBM;
    const QmmPlan pl = plan_with_workspace(a, workspace ? workspace_bytes : 0);
    const QmmSplit sp{static_cast<float*>(workspace), pl.ks};
    hipError_t e = pl.bn == 256 ? launch_t<BITS, SBT, 256, false>(a, none, mt, sp)
                                : launch_t<BITS, SBT, 128, false>(a, none, mt, sp);
    if (e != hipSuccess || pl.ks == 1) return e;
    return launch_split_reduce(static_cast<const float*>(workspace), pl.ks, a);
}

template <int BITS, int SBT>
hipError_t launch_gather_bn(const QmmArgs& a, const QmmGather& gq, int64_t m_tiles) {
    // the expert-grouped grid has as many M tiles as experts or more: 128-wide
    // tiles fill the chip whenever 256-wide ones would not
    const QmmSplit unsplit{nullptr, 1};
    return plan_qmm(kBM * m_tiles, a.N, a.K, 1).bn == 256 ? launch_t<BITS, SBT, 256, true>(a, gq, m_tiles, unsplit)
                                                         : launch_t<BITS, SBT, 128, true>(a, gq, m_tiles, unsplit);
}

}  // namespace

int64_t qmm_workspace_bytes(const QmmArgs& a) {
    const QmmPlan pl = plan_qmm(a.M, a.N, a.K, kMaxSplit);
    return pl.ks > 1 ? (int64_t)pl.ks * a.M * a.N * 4 : 0;
}

void qmm_config(const QmmArgs& a, int* bm, int* bn, int* bk, int* ks) {
    const QmmPlan pl = plan_qmm(a.M, a.N, a.K, kMaxSplit);
    if (bm) *bm = kBM;
    if (bn) *bn = pl.bn;
    if (bk) *bk = kBK;
    if (ks) *ks = pl.ks;
}

hipError_t launch_qmm(const QmmArgs& a, void* workspace, int64_t workspace_bytes) {
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_bn<4, DT_F16>(a, workspace, workspace_bytes)
                                    : launch_bn<4, DT_BF16>(a, workspace, workspace_bytes);
    return a.sb_dtype == DT_F16 ? launch_bn<8, DT_F16>(a, workspace, workspace_bytes)
                                : launch_bn<8, DT_BF16>(a, workspace, workspace_bytes);
}

int64_t gather_grouped_max_tiles(int64_t S, int64_t E, int tr) { return S / tr + E + 1; }

int64_t gather_grouped_workspace(int64_t S, int64_t E) {
    return 4 * ((E + 2) + 1 + S + 2 * gather_grouped_max_tiles(S, E, kGatherGemvRows));
}

GatherPlan gather_plan_layout(void* workspace, int64_t S, int64_t E, int tr) {
    GatherPlan p;
    p.seg = static_cast<int32_t*>(workspace);
    p.ntiles = p.seg + E + 2;
    p.perm = p.ntiles + 1;
    p.tiles = p.perm + S;
    p.max_tiles = gather_grouped_max_tiles(S, E, tr);
    return p;
}

hipError_t launch_gather_plan(const int32_t* idx, int64_t S, int64_t E, int tr, const GatherPlan& p,
                              hipStream_t stream) {
    const size_t plan_lds = 2 * (size_t)(E + 1) * sizeof(int32_t);
    hipLaunchKernelGGL(gather_plan_kernel, dim3(1), dim3(1024), plan_lds, stream, idx, (int)S, (int)E, tr, p.seg,
                       p.ntiles, p.perm, p.tiles);
    return hipGetLastError();
}

hipError_t launch_gather_grouped(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_index,
                                 int64_t experts, int64_t x_bytes, void* workspace) {
    const int64_t S = T * top_k;
    const GatherPlan pl = gather_plan_layout(workspace, S, experts, kBM);
    hipError_t e = launch_gather_plan(idx, S, experts, kBM, pl, a.stream);
    if (e != hipSuccess) return e;
    const int64_t mt = pl.max_tiles;
    int32_t *perm = pl.perm, *seg = pl.seg, *tiles = pl.tiles, *ntiles = pl.ntiles;
    const QmmGather gq{perm, seg, tiles, ntiles, top_k, x_per_index, (int)experts, (uint32_t)x_bytes};
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_gather_bn<4, DT_F16>(a, gq, mt) : launch_gather_bn<4, DT_BF16>(a, gq, mt);
    return a.sb_dtype == DT_F16 ? launch_gather_bn<8, DT_F16>(a, gq, mt) : launch_gather_bn<8, DT_BF16>(a, gq, mt);
}

}  // namespace miqmm
