// qmvs.hip -- K-sliced GEMV for one to four rows of x (M <= 4).
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])       (transpose=true)
//
// The decode-time call of every quantized projection of the reference
// (src/engine/mlx_lm/models/llama.rs:195-197,249,293-294 with x [1, 1, K]),
// and the few-row calls of several sequences or speculative tokens; also the
// decode step's grouped q/k/v and gate/up (QmvsGroup).
//
// HBM-bound design (no MFMA).  A row of W is cut into K-slices of 1 KiB of
// codes (2048 4-bit or 1024 8-bit codes).  A block covers RB consecutive rows
// with one wave per K-slice; lane l of wave w owns the 16-byte chunk l of
// slice w in each of the block's rows.  A wave runs straight through, with
// no loop:
//   - it loads its x chunk of every row of x (the same for every row of W it
//     computes; with several rows of x each row of codes is unpacked once and
//     dotted with all of them), then issues
//     the scales and biases of its RB rows (one 1 KiB run per row stride,
//     copied straight to the wave's LDS by direct-to-LDS loads) and the
//     codes of its RB rows (each load instruction 1 KiB contiguous bytes of
//     one row), so everything the wave reads is in flight at once;
//   - it prepares x once (the bf16 pairs the code unpack needs, and its
//     sum) while the codes are in flight, then computes the rows in order as
//     they land (the compiler waits for each row's codes on its own);
//   - it reduces its lanes' partial sums of all its rows at once (a
//     transposed reduction: lane-half swaps, then DPP); wave 0 adds the
//     K-slices' partials through LDS in slice order and writes the outputs.
// The grid has one block per RB rows: a chip-full of waves runs at once and
// later blocks take the CUs as earlier ones finish.  Load instructions that
// read nothing are not issued: out-of-range loads still take a slot in the
// CU's memory pipeline, which is what the kernel's time is made of.
// The arithmetic per chunk is the exact factorised dequant of the other
// GEMVs: sum_k x_k (s q_k + b) = s * sum_k x_k q_k + b * sum_k x_k, with the
// codes made exact 16-bit float operands by one and-or with a magic
// exponent: 4-bit codes as bf16 128 + q against x re-paired to match, or
// (one row of x, 16 full rows per lane: f16_operands) as fp16 1024 + q
// (bits 0-3) or 1024 + 16 q (bits 4-7), one shift per word of eight codes,
// against x scaled per lane by an exact power of two (and by 1/16 for the
// second kind) into fp16; 8-bit codes as the bf16 top half of their fp32
// value against bf16 x.  The offsets and scales are undone per row in fp32:
//   sum_k x_k q_k = dot - 128 * sum x, or 2^E (dot - 1024 * sum of the x operands).
// Measured on MI355X (cold weights, back-to-back graph launches, 4-bit g64):
// M = 1, 4096 -> 14336 and 14336 -> 4096 in 7.9-8.4 us (about 4 TB/s) against
// 9.2 and 9.9 us for the v_dot2 GEMV, beside 5.9-6.2 us for a bare streaming
// read of the same 33 MB; the 5376 -> 262144 head (g32, fp16 scales) in
// 113-131 us (6.7-7.8 TB/s); M = 2 and 4 on 4096 -> 14336 in 8.9 and 11.8 us.
#include <climits>
#include <type_traits>

#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

constexpr int kSliceBytes = 1024;  // codes per K-slice: 64 lanes x 16 bytes


// Operands of the 4-bit dot products: fp16 (codes at bits 0-3 and 4-7 of each
// half are exact fp16 mantissas: per word of eight codes one shift and four
// and-ors, against three shifts and four for bf16) costs x a preparation of
// ~150 VALU instructions per lane (its largest exponent, a power-of-two scale
// and the conversions) against ~30 for bf16 (a re-pairing), so it pays only
// where a lane has many rows to amortise it: one row of x and 16 full rows per
// lane (measured on MI355X, 4-bit g64: 14336 -> 4096 8.39 -> 8.13 us with fp16;
// with bf16 the decode step's launches 2.47 -> 2.36 us (q/k/v), 3.33 -> 3.13
// (gate/up), 896 -> 4864 2.95 -> 2.71 us, and two rows of x, 4096 -> 14336,
// 10.8 -> 9.8 us)
template <int BITS, int RB, bool HALF, int MX>
constexpr bool f16_operands() { return BITS == 4 && MX == 1 && RB == 16 && !HALF; }
typedef __attribute__((ext_vector_type(2))) _Float16 half2_t;
typedef __attribute__((ext_vector_type(2))) unsigned short u16x2_t;


struct QmvsArgs {
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    void* y;
    const void* bias;
    int N, K, gs_shift, y_dtype;
};

// Problems 1..3 of a group (one row of x shared by all); problem 0 is the
// kernel's own arguments.  Contiguous (codes, scales and biases following
// problem 0's): the kernel reads one matrix of all their rows, and row0 is
// each one's first row in it (unused: INT_MAX), y / bias its output and
// bias.  Separate (the NC kernels): w / s / b are its own codes, scales and
// biases, n its rows and blk0 its first block; every block computes rows of
// one problem and every problem starts a block.  With the rows per block of
// the problems' concatenation either way gives each row bit for bit as a
// launch over that one matrix: a row's sum does not depend on where in a
// block it sits.  (The separate layout's per-block lookup reads arguments
// past the preloaded ones before the first loads, a scalar memory round trip
// the other launches do not take.)
struct QmvsGroup {
    void* y[3];
    const void* bias[3];
    int row0[3];
    const uint32_t* w[3];
    const uint16_t* s[3];
    const uint16_t* b[3];
    int n[3];
    int blk0[3];
    int n_first;  // NC: rows of problem 0 (0: not a separate-allocation group)
};

// LDS per wave: scales then biases of its rows, ND KiB each (a direct-to-LDS
// load moves 1 KiB); after all waves' areas, the slice partials [waves][RB]
template <int ND>
constexpr int wave_lds() { return 2 * ND * kSliceBytes; }

// DPP moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_ror:8)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sums RB per-lane values v[0..RB) over the wave's 64 lanes, one row per
// value, as a transposed reduction: lane halves trade values
// (permlane32_swap), then 16-lane rows (permlane16_swap), then 8- and
// 4-lane groups (DPP), each exchange halving the values a lane keeps, and
// the last lanes of a group add what they hold.  Afterwards lane l holds the
// sum of value l >> (6 - log2 RB): lanes 64/RB * j .. of row j.  About
// 3 RB instructions for the RB values, against 12 per value for one
// butterfly per value.
// From the state after the first exchange: H = RB / 2 values per lane,
// lanes 0-31 holding values j and lanes 32-63 values j + H (also the state
// of a wave whose two halves compute different rows).
template <int RB>
__device__ __forceinline__ float transposed_sum32(const float (&b)[RB / 2], int lane) {
    static_assert(RB == 4 || RB == 8 || RB == 16 || RB == 32, "rows per reduction");
    constexpr int H = RB / 2;
    constexpr int Q = H / 2;
    float c[Q];
#pragma unroll
    for (int j = 0; j < Q; ++j) {  // 16-lane row G: value j + (G & 1) Q + (G >> 1) H
        const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[j]), __float_as_uint(b[j + Q]), false,
                                                        false);
        c[j] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
    float r;
    if constexpr (RB == 4) {
        r = c[0];  // value l >> 4: sum its 16 lanes
        r += dpp<0xB1>(r);
        r += dpp<0x4E>(r);
        r += dpp<0x141>(r);
        r += dpp<0x128>(r);
    } else {
        // halves of 8 lanes within each 16-lane row (row_ror:8 pairs lane l with l ^ 8)
        const bool hi8 = (lane & 8) != 0;
        constexpr int E = Q / 2 > 0 ? Q / 2 : 1;
        float d[E];
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float keep = hi8 ? c[j + E] : c[j], give = hi8 ? c[j] : c[j + E];
            d[j] = keep + dpp<0x128>(give);
        }
        if constexpr (RB == 8) {
            r = d[0];  // value l >> 3: sum its 8 lanes
            r += dpp<0xB1>(r);
            r += dpp<0x4E>(r);
            r += dpp<0x141>(r);
        } else {
            // lanes l and 7 - l of each 8 (row_half_mirror) hold the same values
            const bool hi4 = (lane & 4) != 0;
            constexpr int F = E / 2;
            float f[F];
#pragma unroll
            for (int j = 0; j < F; ++j) {
                const float keep = hi4 ? d[j + F] : d[j], give = hi4 ? d[j] : d[j + F];
                f[j] = keep + dpp<0x141>(give);
            }
            if constexpr (RB == 16) {
                r = f[0];  // value l >> 2: sum its 4 lanes
                r += dpp<0xB1>(r);
                r += dpp<0x4E>(r);
            } else {
                // lanes l and l ^ 2 (quad_perm [2,3,0,1]) hold the same two values
                const bool hi2 = (lane & 2) != 0;
                const float keep = hi2 ? f[1] : f[0], give = hi2 ? f[0] : f[1];
                r = keep + dpp<0x4E>(give);  // value l >> 1: sum its 2 lanes
                r += dpp<0xB1>(r);
            }
        }
    }
    return r;
}

template <int RB>
__device__ __forceinline__ float transposed_sum(const float (&v)[RB], int lane) {
    constexpr int H = RB / 2;
    float b[H];
#pragma unroll
    for (int j = 0; j < H; ++j) {  // lanes 0-31: value j, lanes 32-63: value j + H
        const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + H]), false,
                                                        false);
        b[j] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
    return transposed_sum32<RB>(b, lane);
}

// RB rows per block; ND direct-to-LDS loads per scale (and bias) array:
// RB * (bytes of scales per row and slice) / 1 KiB, rounded up
// waves (K-slices) per block: up to 15, or 8 where a lane needs more than 128
// registers (32 rows of codes; four rows of x)
template <int RB, int MX>
constexpr int max_threads() { return RB >= 32 || MX == 4 ? 512 : 1024; }
constexpr int max_slices(int64_t M) { return M > 2 ? 8 : 15; }

// The arguments are scalars, the ones the first loads need leading: the build
// preloads leading kernel arguments into SGPRs at wave launch, which spares
// the scalar memory round trip before the first load (bias, read last, is
// past the preloaded registers).  meta = log2 group size | y dtype << 8 |
// waves per block << 16 | rows of x << 24 (blockDim would be a load of the
// implicit arguments).
//
// HALF (rows of at most 32 chunks, one slice): the wave's halves compute
// different rows, lanes 32h .. 32h + 31 the rows h RB/2 .. h RB/2 + RB/2 - 1
// of the block, so no lane idles past a short row's end (K = 896 at 4 bits
// is 28 chunks); the reduction starts from its 32-lane state.
//
// MX rows of x (1, 2 or 4; three rows run as four, the fourth reading zeros and
// storing nothing): each row of codes is unpacked once and dotted with
// every row of x; the wave reduces RB * MX sums (value m * RB + j, or with
// HALF m * RB/2 + j in each half).
template <int BITS, int SBT, int RB, int ND, bool YF32, bool BIAS, bool HALF, int MX, bool NC>
__global__ __launch_bounds__((max_threads<RB, MX>())) void qmvs_kernel(const uint16_t* xp, const uint32_t* wp,
                                                                 const uint16_t* sp, const uint16_t* bp, int n, int k,
                                                                 uint32_t meta, void* yp, const void* biasp,
                                                                 const QmvsGroup grp) {
    const QmvsArgs P{xp, wp, sp, bp, yp, biasp, n, k, (int)(meta & 0xff), (int)((meta >> 8) & 0xff)};
    constexpr int CPC_SHIFT = BITS == 4 ? 5 : 4;  // codes per 16-byte chunk: 32 or 16
    constexpr int CPC = 1 << CPC_SHIFT;
    constexpr int NP = CPC / 2;                   // bf16 pairs of x per chunk
    constexpr int XQ = NP / 4;                    // 16-byte x loads per chunk

    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63;
    const int ws = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's K-slice
    const int KS = (int)((meta >> 16) & 0xff);
    const int K = P.K, gs_shift = P.gs_shift;
    const int C = K >> CPC_SHIFT;       // chunks per row
    constexpr int RL = HALF ? RB / 2 : RB;          // rows per lane
    const int lc = HALF ? lane & 31 : lane;          // this lane's chunk within the slice
    const int rh = HALF ? (lane >> 5) * RL : 0;      // first of this lane's rows in the block
    const int c = ws * 64 + lc;         // this lane's chunk of every row
    const bool cv = c < C;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int G = K >> gs_shift;
    // NC: this block's problem (uniform) and its first row in it
    const int bx = blockIdx.x;
    const int gp = NC ? (bx >= grp.blk0[0]) + (bx >= grp.blk0[1]) + (bx >= grp.blk0[2]) : 0;
    const int r0 = NC ? (bx - (gp == 0 ? 0 : gp == 1 ? grp.blk0[0] : gp == 2 ? grp.blk0[1] : grp.blk0[2])) * RB
                      : bx * RB;
    const int Np = !NC || gp == 0 ? P.N : gp == 1 ? grp.n[0] : gp == 2 ? grp.n[1] : grp.n[2];
    const uint32_t* const pw = !NC || gp == 0 ? P.w : gp == 1 ? grp.w[0] : gp == 2 ? grp.w[1] : grp.w[2];
    const uint16_t* const ps = !NC || gp == 0 ? P.s : gp == 1 ? grp.s[0] : gp == 2 ? grp.s[1] : grp.s[2];
    const uint16_t* const pb = !NC || gp == 0 ? P.b : gp == 1 ? grp.b[0] : gp == 2 ? grp.b[1] : grp.b[2];
    const int nrows = min(RB, Np - r0);
    constexpr int ysz = YF32 ? 4 : 2;

    constexpr int RV = RB * MX;  // sums the wave reduces
    const int MR = (int)(meta >> 24);  // rows of x (MX, or 3 with MX = 4)
    // x chunk of this lane in each row of x (zero past the row end and past
    // the last row); prepared below, once the codes are in flight
    uint32_t xw[MX][NP];
    {
        const auto xr = make_rsrc(P.x, (uint32_t)(MR * K) * 2);
#pragma unroll
        for (int m = 0; m < MX; ++m)
#pragma unroll
            for (int i = 0; i < XQ; ++i) {
                const u32x4_t v = bload16(xr, cv ? (uint32_t)(m * K + c * CPC) * 2 + i * 16 : kOOB);
                xw[m][4 * i + 0] = v[0];
                xw[m][4 * i + 1] = v[1];
                xw[m][4 * i + 2] = v[2];
                xw[m][4 * i + 3] = v[3];
            }
    }

    // The loads are issued in this order, fenced against the scheduler: the
    // x chunk, the direct-to-LDS scales and biases, then the codes (and bias),
    // so that (1) the explicit wait below, which counts the loads issued after
    // the scales and biases, is exact, and (2) every code load is in flight
    // before any arithmetic (left alone, the scheduler sinks the later rows'
    // loads below the first rows' arithmetic).
    __builtin_amdgcn_sched_barrier(0);
    // scales and biases of this wave's slice of the block's rows, to LDS:
    // row j's gps scales at j * sb (sb = 2 * gps bytes, a multiple of 16);
    // DMA lane l of load d carries 16 bytes of row (d * 64 + l) / lpr
    const auto sr = make_rsrc(ps + (size_t)r0 * G, (uint32_t)nrows * G * 2);
    const auto br = make_rsrc(pb + (size_t)r0 * G, (uint32_t)nrows * G * 2);
    const int gps = (kSliceBytes * 8 / BITS) >> gs_shift;
    const int sb = 2 * gps;
    const int lpr_shift = __builtin_ctz((unsigned)sb >> 4);  // DMA lanes per row: a power of two
    char* const wl = smem + ws * wave_lds<ND>();
#pragma unroll
    for (int d = 0; d < ND; ++d) {
        const int dl = d * 64 + lane;
        const int row = dl >> lpr_shift, g0 = ws * gps + (dl & ((1 << lpr_shift) - 1)) * 8;
        const uint32_t off = row < RB && g0 < G ? ((uint32_t)row * G + g0) * 2 : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(wl + d * kSliceBytes), 16, off, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_void*)(wl + (ND + d) * kSliceBytes), 16, off, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // codes of the block's rows (rows past the block's last read zero)
    const auto wr = make_rsrc((const char*)pw + (size_t)r0 * row_bytes, (uint32_t)nrows * row_bytes);
    u32x4_t q[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j)
        q[j] = bload16_nt(wr, cv ? (uint32_t)(rh + j) * row_bytes + (uint32_t)c * 16 : kOOB);
    // the row this lane stores: row t of the block by lane t of wave 0, into
    // its problem's output (and with its bias)
    // (one slice per row: the lanes that end the wave's reduction holding a
    // row's sum store it, lane (64 / RB) t for row t, with no trip through LDS)
    // (the value a lane stores: t_v, of row of x t_m and row of the block t_row)
    const bool one = KS == 1;
    const int t_v = one ? lane / (64 / RV) : lane;
    const int t_m = HALF ? (t_v % (RV / 2)) / (RB / 2) : t_v / RB;
    const int t_row = HALF ? (t_v / (RV / 2)) * (RB / 2) + t_v % (RB / 2) : t_v % RB;
    const bool t_mine = (one ? (lane & (64 / RV - 1)) == 0 : ws == 0 && t_v < RV) && t_row < nrows && t_m < MR;
    const int t_glob = r0 + t_row;
    constexpr bool F16 = f16_operands<BITS, RB, HALF, MX>();
    // the problem of the stored row, and its output column there
    const int t_p = NC ? gp : (t_glob >= grp.row0[0]) + (t_glob >= grp.row0[1]) + (t_glob >= grp.row0[2]);
    const size_t t_n = (size_t)(t_glob - (NC || t_p == 0 ? 0 : grp.row0[t_p - 1]));
    const size_t t_off = ((size_t)t_m * Np + t_n) * ysz;
    uint32_t bias_bits = 0;
    if constexpr (BIAS) {  // every lane loads (a lane past the rows reads row 0's): one load, counted below
        // the bias is per output column, the same for every row of x
        const char* const bp0 = t_p == 0 ? (const char*)P.bias : (const char*)grp.bias[t_p - 1];
        const char* const ba = t_mine ? bp0 + t_n * ysz : (const char*)P.bias;
        if constexpr (YF32) bias_bits = *reinterpret_cast<const uint32_t*>(ba);
        else bias_bits = *reinterpret_cast<const uint16_t*>(ba);
    }

    __builtin_amdgcn_sched_barrier(0);
    // x prepared: pairs (x_j, x_{j+4}) matching the 4-bit unpack, and the sum
    uint32_t X[MX][NP];
    float xs[MX];
    float xsc[MX], xoff[MX];  // fp16 operands only
#pragma unroll
    for (int m = 0; m < MX; ++m) {
        xs[m] = 0.f;
#pragma unroll
        for (int i = 0; i < NP; ++i) xs[m] = dot2(xw[m][i], kOnesBf16x2, xs[m]);
        // fp16 operands: x scaled by 2^-E (E: exponent of the chunk's largest
        // |x|, so every operand is below 2 and exact unless below fp16's normal
        // range), the operands facing the codes taken at bits 4-7 further by
        // 1/16; xsc = 2^E and xoff = -2^E * 1024 * (sum of the operands) undo
        // the scale and the codes' 1024 offset
        if constexpr (F16) {
            // the largest exponent field: a packed 16-bit max of the pairs'
            // exponent bits
            uint32_t em = 0;
#pragma unroll
            for (int i = 0; i < NP; ++i)
                em = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, xw[m][i] & 0x7F807F80u),
                                                                            __builtin_bit_cast(u16x2_t, em)));
            const int e = (int)(max(em & 0xFFFFu, em >> 16) >> 7) - 127;
            xsc[m] = __builtin_amdgcn_ldexpf(1.f, e);
            // x_k of the chunk times 2^-e (or 2^-e-4) as fp16 bits: the product
            // is exact in fp32, so the multiply and the conversion fuse into one
            // v_fma_mixlo_f16 with the bits of ldexp then convert
            const float sc0 = __builtin_amdgcn_ldexpf(1.f, -e), sc4 = __builtin_amdgcn_ldexpf(1.f, -e - 4);
            auto h = [&](int k, float sc) {
                const uint32_t w = xw[m][k >> 1];
                const float f = __uint_as_float((k & 1) ? (w & 0xFFFF0000u) : (w << 16));
                return (uint32_t)f32_to_f16_bits(f * sc);
            };
            float ssum = 0.f;
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                const int k0 = 8 * wi;
                X[m][4 * wi + 0] = h(k0 + 0, sc0) | (h(k0 + 4, sc0) << 16);
                X[m][4 * wi + 1] = h(k0 + 1, sc4) | (h(k0 + 5, sc4) << 16);
                X[m][4 * wi + 2] = h(k0 + 2, sc0) | (h(k0 + 6, sc0) << 16);
                X[m][4 * wi + 3] = h(k0 + 3, sc4) | (h(k0 + 7, sc4) << 16);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    ssum = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, X[m][4 * wi + t]),
                                                  __builtin_bit_cast(half2_t, 0x3C003C00u), ssum, false);
            }
            xoff[m] = -xsc[m] * 1024.f * ssum;
        } else if constexpr (BITS == 4) {
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) perm_x_for4(&xw[m][4 * wi], &X[m][4 * wi]);
        } else {
#pragma unroll
            for (int i = 0; i < NP; ++i) X[m][i] = xw[m][i];
        }
    }

    // the DMA must land before the stage is read from LDS (the compiler does
    // not track that dependency): issued after it and still allowed in
    // flight are the codes (and the bias)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(RL + (BIAS ? 1 : 0)));
    asm volatile("" ::: "memory");

    const uint32_t kMask = vgpr_const(0x000F000Fu), kMagic = kMagic128x2;
    const uint32_t kMaskHi = vgpr_const(0x00F000F0u);  // fp16 operands only
    // this lane's scale / bias of row j at j * sb + 2 * (group in slice)
    const uint32_t sl_off = (uint32_t)((lc << CPC_SHIFT) >> gs_shift) * 2;
    // per-lane partial of every row; in the wave of the slice that runs past
    // the row end (if any), lanes past it add nothing whatever their LDS
    // holds: with one row of x their partials are zeroed (one select per
    // row), with more their scales and biases (two per row, not one per row
    // of x); their x reads zero
    const bool partial = __builtin_amdgcn_readfirstlane((int)(ws == KS - 1 && (C & 63) != 0)) != 0;
    float part[RL * MX];  // value m * RL + j
    auto rows = [&](auto masked) {
#pragma unroll
        for (int j = 0; j < RL; ++j) {
            uint32_t p[NP];
            const int jr = rh + j;  // row of the block
            float s = half_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(wl + jr * sb + sl_off));
            float b = half_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(wl + ND * kSliceBytes + jr * sb + sl_off));
            if constexpr (decltype(masked)::value && MX > 1) {
                s = cv ? s : 0.f;
                b = cv ? b : 0.f;
            }
            if constexpr (F16) {
                constexpr uint32_t kMagic1024 = 0x64006400u;  // fp16 1024 | q: exact 1024 + q (and 1024 + 16 q)
#pragma unroll
                for (int wi = 0; wi < 4; ++wi) {
                    const uint32_t w = q[j][wi], w8 = w >> 8;
                    p[4 * wi + 0] = and_or(w, kMask, kMagic1024);
                    p[4 * wi + 1] = and_or(w, kMaskHi, kMagic1024);
                    p[4 * wi + 2] = and_or(w8, kMask, kMagic1024);
                    p[4 * wi + 3] = and_or(w8, kMaskHi, kMagic1024);
                }
#pragma unroll
                for (int m = 0; m < MX; ++m) {
                    float a = 0.f;
#pragma unroll
                    for (int i = 0; i < NP; ++i)
                        a = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, X[m][i]),
                                                   __builtin_bit_cast(half2_t, p[i]), a, false);
                    part[m * RL + j] = fmaf(s, fmaf(a, xsc[m], xoff[m]), b * xs[m]);
                    if constexpr (decltype(masked)::value && MX == 1) part[m * RL + j] = cv ? part[m * RL + j] : 0.f;
                }
                continue;
            }
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                if constexpr (BITS == 4) unpack4_magic(q[j][wi], &p[wi * 4], kMask, kMagic);
                else unpack8_pairs(q[j][wi], &p[wi * 2]);
            }
            if constexpr (BITS == 4) b = fmaf(-128.f, s, b);
#pragma unroll
            for (int m = 0; m < MX; ++m) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < NP; ++i) a = dot2(X[m][i], p[i], a);
                part[m * RL + j] = fmaf(b, xs[m], s * a);
                if constexpr (decltype(masked)::value && MX == 1) part[m * RL + j] = cv ? part[m * RL + j] : 0.f;
            }
        }
    };
    // always masked: a uniform branch to an unmasked copy for full slices
    // was slower (measured on MI355X: 4096 -> 14336 7.95 -> 11.8 us)
    (void)partial;
    rows(std::true_type{});
    // the wave's sum of row j lands in lanes (64 / RB) j .. (64 / RB) (j + 1) - 1
    float tot;
    if constexpr (HALF) tot = transposed_sum32<RV>(part, lane);
    else tot = transposed_sum<RV>(part, lane);
    float v = 0.f;
    if (one) {
        if (!t_mine) return;
        v += tot;
    } else {
        // the slice partials meet in LDS; row t is summed (slices in order)
        // and stored by lane t of wave 0
        float* const kp = reinterpret_cast<float*>(smem + KS * wave_lds<ND>());
        if ((lane & (64 / RV - 1)) == 0) kp[ws * RV + lane / (64 / RV)] = tot;
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (!t_mine) return;
        for (int w = 0; w < KS; ++w) v += kp[w * RV + t_v];
    }
    // plain stores (measured on MI355X: a non-temporal store per block added
    // 3.5 us to a 6 us streaming read)
    char* const ya = (t_p == 0 ? (char*)P.y : (char*)grp.y[t_p - 1]) + t_off;
    if constexpr (YF32) {
        if constexpr (BIAS) v += __uint_as_float(bias_bits);
        *reinterpret_cast<float*>(ya) = v;
    } else {
        // rounded to y's dtype, then the bias added and rounded again (two MLX ops)
        uint16_t h;
        if (P.y_dtype == DT_F16) {
            h = f32_to_f16_bits(f32_pinned(v));
            if constexpr (BIAS) h = f32_to_f16_bits(f32_pinned(f16_bits_to_f32(h) + f16_bits_to_f32(bias_bits)));
        } else {
            h = f32_to_bf16_bits(v);
            if constexpr (BIAS) h = f32_to_bf16_bits(bf16_bits_to_f32(h) + bf16_bits_to_f32(bias_bits));
        }
        *reinterpret_cast<uint16_t*>(ya) = h;
    }
}

// waves (K-slices) per block
int slices(int64_t K, int bits) {
    const int64_t slice_codes = (int64_t)kSliceBytes * 8 / bits;
    return (int)((K + slice_codes - 1) / slice_codes);
}

// rows per block: 16 when that still gives the chip about 6 waves per CU
// (fewer, longer waves: x is loaded once per 16 rows), else 8, else 4
#ifndef QMVS_RB_FORCE
#define QMVS_RB_FORCE 0
#endif
int rows_per_block(int64_t N, int ks) {
    if (QMVS_RB_FORCE) return QMVS_RB_FORCE == 32 && ks > 7 ? 16 : QMVS_RB_FORCE;
    const int64_t waves_wanted = (int64_t)num_cus() * 6;
    if ((N + 15) / 16 * ks >= waves_wanted) return 16;
    if ((N + 7) / 8 * ks >= waves_wanted / 2) return 8;
    return 4;
}

// rows per block for M rows of x
int rows_for(int64_t M, int64_t N, int ks) {
    int rb = rows_per_block(N, ks);
    if (M > 2 && rb > 8) rb = 8;  // four rows of x: RB * 4 <= 32 sums per wave
    // two rows of x on rows of one or two slices: 8 rows per block unless 16
    // still gives 12 waves per CU (measured on MI355X, 4-bit g64: 4096 ->
    // 14336 9.9-10.4 -> 9.1-9.5 us; with more slices, or more waves, 16 rows
    // stay faster: 14336 -> 4096 10.0 against 10.2, the 896 -> 151936 head
    // 18.3-18.8 against 20.9)
    if (M == 2 && rb == 16 && ks <= 2 && (N + 15) / 16 * ks < 12 * (int64_t)num_cus()) rb = 8;
    return rb;
}

// NC: a group in separate allocations; a.N is then all the problems' rows
// (for the rows per block of their concatenation) and n_first problem 0's
template <int BITS, int SBT, int RB, int ND, bool YF32, bool BIAS, bool HALF, int MX, bool NC>
hipError_t launch_t(const QmmArgs& a, const QmvsGroup& g0, int ks, int n_first) {
    const int n0 = NC ? n_first : (int)a.N;
    const QmvsArgs P{(const uint16_t*)a.x, a.w, (const uint16_t*)a.scales, (const uint16_t*)a.biases, a.y, a.bias,
                     n0, (int)a.K, __builtin_ctz((unsigned)a.group_size), a.y_dtype};
    const size_t lds = (size_t)ks * wave_lds<ND>() + (size_t)ks * RB * MX * 4;
    QmvsGroup g = g0;
    int blocks = (n0 + RB - 1) / RB;
    if (NC) {  // each problem starts a block
        for (int i = 0; i < 3; ++i) {
            g.blk0[i] = g.n[i] > 0 ? blocks : INT_MAX;
            blocks += (g.n[i] + RB - 1) / RB;
        }
    }
    hipLaunchKernelGGL((qmvs_kernel<BITS, SBT, RB, ND, YF32, BIAS, HALF, MX, NC>), dim3(blocks), dim3(64 * ks), lds, a.stream, P.x,
                       P.w, P.s, P.b, P.N, P.K,
                       (uint32_t)P.gs_shift | (uint32_t)P.y_dtype << 8 | (uint32_t)ks << 16 | (uint32_t)a.M << 24, P.y,
                       P.bias, g);
    return hipGetLastError();
}

// rows of at most 32 chunks in one slice: the half-wave rows
bool half_rows(int64_t K, int bits) { return slices(K, bits) == 1 && K * bits / 128 <= 32; }

template <int BITS, int SBT, int RB, int ND, bool YF32, bool BIAS, int MX>
hipError_t launch_h(const QmmArgs& a, const QmvsGroup& g, int ks) {
    const bool half = half_rows(a.K, BITS);
    if constexpr (MX == 1) {
        if (g.n_first > 0)
            return half ? launch_t<BITS, SBT, RB, ND, YF32, BIAS, true, MX, true>(a, g, ks, g.n_first)
                        : launch_t<BITS, SBT, RB, ND, YF32, BIAS, false, MX, true>(a, g, ks, g.n_first);
    }
    return half ? launch_t<BITS, SBT, RB, ND, YF32, BIAS, true, MX, false>(a, g, ks, 0)
                : launch_t<BITS, SBT, RB, ND, YF32, BIAS, false, MX, false>(a, g, ks, 0);
}

template <int BITS, int SBT, int RB, bool YF32, bool BIAS, int MX>
hipError_t launch_nd(const QmmArgs& a, const QmvsGroup& g, int ks) {
    // bytes of scales per row and slice: (1 KiB of codes / group) * 2
    const int sb = 2 * ((kSliceBytes * 8 / BITS) / a.group_size);
    if (RB * sb > 2 * kSliceBytes) return launch_h<BITS, SBT, RB, 4, YF32, BIAS, MX>(a, g, ks);
    if (RB * sb > kSliceBytes) return launch_h<BITS, SBT, RB, 2, YF32, BIAS, MX>(a, g, ks);
    return launch_h<BITS, SBT, RB, 1, YF32, BIAS, MX>(a, g, ks);
}

template <int BITS, int SBT, bool YF32, bool BIAS, int MX>
hipError_t launch_rb(const QmmArgs& a, const QmvsGroup& g) {
    const int ks = slices(a.K, BITS);
    switch (rows_for(a.M, a.N, ks)) {
#if QMVS_RB_FORCE == 32
        case 32: return launch_nd<BITS, SBT, 32, YF32, BIAS, 1>(a, g, ks);
#endif
        case 16:
            if constexpr (MX < 4) return launch_nd<BITS, SBT, 16, YF32, BIAS, MX>(a, g, ks);
            [[fallthrough]];
        case 8: return launch_nd<BITS, SBT, 8, YF32, BIAS, MX>(a, g, ks);
        default: return launch_nd<BITS, SBT, 4, YF32, BIAS, MX>(a, g, ks);
    }
}

template <bool YF32, bool BIAS, int MX>
hipError_t launch_y(const QmmArgs& a, const QmvsGroup& g) {
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? launch_rb<4, DT_F16, YF32, BIAS, MX>(a, g)
                                    : launch_rb<4, DT_BF16, YF32, BIAS, MX>(a, g);
    return a.sb_dtype == DT_F16 ? launch_rb<8, DT_F16, YF32, BIAS, MX>(a, g)
                                : launch_rb<8, DT_BF16, YF32, BIAS, MX>(a, g);
}

template <int MX>
hipError_t launch_m(const QmmArgs& a, const QmvsGroup& g) {
    if (a.y_dtype == DT_F32) return a.bias ? launch_y<true, true, MX>(a, g) : launch_y<true, false, MX>(a, g);
    return a.bias ? launch_y<false, true, MX>(a, g) : launch_y<false, false, MX>(a, g);
}

// one to four rows of x (more than one: no grouped problems)
hipError_t launch_g(const QmmArgs& a, const QmvsGroup& g) {
    if (a.M == 1) return launch_m<1>(a, g);
    if (g.row0[0] != INT_MAX || g.n_first > 0) return hipErrorInvalidValue;
    if (a.M == 2) return launch_m<2>(a, g);
    if (a.M == 3 || a.M == 4) return launch_m<4>(a, g);
    return hipErrorInvalidValue;
}

}  // namespace

bool qmvs_supported(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
    (void)N;
    // up to 15 waves per block, 8 with more than two rows of x (LDS within
    // the default 64 KiB; the registers of four rows of x); an even
    // number of groups per row keeps the scale rows 4-byte aligned for the
    // 16-byte direct-to-LDS loads
    const int ks = slices(K, bits);
    return M >= 1 && M <= 4 && ks >= 1 && ks <= max_slices(M) && (K / group_size) % 2 == 0;
}

void qmvs_config(const QmmArgs& a, int* rows_per_blk, int* slices_out, int* blocks) {
    const int ks = slices(a.K, a.bits), rb = rows_for(a.M, a.N, ks);
    if (rows_per_blk) *rows_per_blk = rb;
    if (slices_out) *slices_out = ks;
    if (blocks) *blocks = (int)((a.N + rb - 1) / rb);
}

namespace {

QmvsGroup no_group() {
    QmvsGroup g{};
    for (int i = 0; i < 3; ++i) g.row0[i] = g.blk0[i] = INT_MAX;
    return g;
}

// a group the K-sliced GEMV takes in one launch: 1 stored one after another,
// 2 in separate allocations, 0 neither
int qmvs_group_kind(const QmmArgs* a, int count) {
    if (count < 2 || count > 4 || a[0].M != 1) return 0;
    const int64_t row_bytes = a[0].K * a[0].bits / 8, sb_row = a[0].K / a[0].group_size * 2;
    int64_t rows = 0;
    bool contiguous = true;
    for (int i = 0; i < count; ++i) {
        if (a[i].x != a[0].x || (a[i].bias == nullptr) != (a[0].bias == nullptr) || a[i].N < 1) return 0;
        if (((reinterpret_cast<uintptr_t>(a[i].scales) | reinterpret_cast<uintptr_t>(a[i].biases)) & 3) != 0)
            return 0;
        contiguous = contiguous && (const char*)a[i].w == (const char*)a[0].w + rows * row_bytes &&
                     (const char*)a[i].scales == (const char*)a[0].scales + rows * sb_row &&
                     (const char*)a[i].biases == (const char*)a[0].biases + rows * sb_row;
        rows += a[i].N;
    }
    if (rows >= ((int64_t)1 << 31) || !qmvs_supported(1, rows, a[0].K, a[0].bits, a[0].group_size)) return 0;
    return contiguous ? 1 : 2;
}

}  // namespace

hipError_t launch_qmvs(const QmmArgs& a) { return launch_g(a, no_group()); }

bool qmvs_group_ok(const QmmArgs* a, int count) { return qmvs_group_kind(a, count) != 0; }

hipError_t launch_qmvs_grouped(const QmmArgs* a, int count) {
    const int kind = qmvs_group_kind(a, count);
    if (kind == 0) return hipErrorInvalidValue;
    QmvsGroup g = no_group();
    QmmArgs all = a[0];  // N: all the rows (the rows per block of their concatenation)
    all.N = 0;
    for (int i = 0; i < count; ++i) {
        if (i > 0) {
            g.y[i - 1] = a[i].y;
            g.bias[i - 1] = a[i].bias;
            if (kind == 1) {
                g.row0[i - 1] = (int)all.N;
            } else {
                g.w[i - 1] = a[i].w;
                g.s[i - 1] = static_cast<const uint16_t*>(a[i].scales);
                g.b[i - 1] = static_cast<const uint16_t*>(a[i].biases);
                g.n[i - 1] = (int)a[i].N;
            }
        }
        all.N += a[i].N;
    }
    if (kind == 2) g.n_first = (int)a[0].N;
    return launch_g(all, g);
}

}  // namespace miqmm
