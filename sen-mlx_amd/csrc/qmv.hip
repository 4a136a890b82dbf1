// qmv.hip -- small-M route (M = 1..16) of affine group-quantized matmul.
//
//   y[m, n] = sum_k x[m, k] * (s[n, k/g] * q[n, k] + b[n, k/g])      (transpose=true)
//
// The operator is MLX's quantized_matmul as called from the reference's
// quantized projections (src/engine/mlx_lm/utils/mod.rs:70-78,
// src/engine/mlx_lm/models/llama.rs:195-197,249,293-294) during decode, where
// x is one token (M=1) or a handful of speculative/batched rows.
//
// HBM-bound design (no MFMA).  A row of W is a sequence of C 16-byte chunks
// (32 4-bit or 16 8-bit codes each; a chunk never straddles a quantization
// group).  A wave is split into 64/L sub-groups of L lanes; a sub-group owns R
// rows at a time and its lane li streams chunks li, li+L, ... of those rows,
// so each load instruction reads L*16 contiguous bytes of each row.  L is
// chosen per K so that few lanes idle (K=896: 28 chunks -> L=32).
//
// Waves are persistent: a wave walks row tiles tile, tile+nwaves, ... and the
// (tile, chunk) iterations are software-pipelined one deep: the next
// iteration's codes, scales, biases (and x, unless the block holds x in its
// LDS table) are in flight while the current one is computed, so a wave keeps
// ~R*16 bytes per lane outstanding at all times.
//
// Arithmetic: codes become exact bf16 operands (4-bit: 0x4300|q = 128+q;
// 8-bit: the top half of the fp32 value of q) and are dotted with x by
// v_dot2_f32_bf16 in fp32.  Per chunk the dequant is applied in factorised
// form, exactly:
//     sum_k x_k (s q_k + b) = s * sum_k x_k (q_k + c) + (b - c s) * sum_k x_k
// with c = 128 (4-bit) or 0 (8-bit).  Lane partials of one row are summed with
// a butterfly over its L lanes.
#include "miqmm_device.h"
#include "miqmm_internal.h"

namespace miqmm {
namespace {

// blocks per CU at most, beyond which the waves walk several tiles each:
// 4 for the matrix GEMVs (measured on MI355X: N = 14336, K = 4096, M = 1 at
// R = 2, 10.2 us with a cap of 8, 9.8 with 4), 8 for the expert gather (its
// per-selection tiles: 16 tokens of DeepSeek-V2-Lite 39.5 us at 8, 42.5 at 4)
constexpr int kMaxBlocksPerCU = 4;
constexpr int kMaxGatherBlocksPerCU = 8;
constexpr int64_t kFillTiles = 1536;  // row tiles that keep the chip busy (see pick_r)

// one pipeline stage: the codes, scales and biases of R rows at one chunk
// position, and (when XPF) the matching x chunk of every row of x
template <int BITS, int R, int MT, bool XPF>
struct Stage {
    static constexpr int NP = (128 / BITS) / 2;  // bf16 pairs of x per chunk
    u32x4_t q[R];
    uint16_t s[R], b[R];
    uint32_t xw[XPF ? MT : 1][NP];
    uint32_t xoff;  // byte offset of this chunk in row 0 of x, or kOOB past the row end
};

// A grouped launch reads its problem table (P.p, in the kernel arguments)
// with one vector load at entry, dword i of the table into lane i, and takes
// a field of the tile's problem with v_readlane.  Left to itself
// the compiler reads the table's tile0 fields, waits, forms a pointer to the
// chosen entry and reads that: three dependent scalar round trips before the
// first code load (measured on MI355X: gate/up 896 -> 2 x 4864 at M = 1,
// 4.50 us grouped against 3.96 us for the same rows as one matrix).
constexpr int kProblemDwords = (int)(sizeof(GemvProblem) / 4);
static_assert(sizeof(GemvProblem) % 8 == 0 && kMaxGroup * kProblemDwords <= 64, "one table dword per lane");
__device__ __forceinline__ uint32_t table_dword(uint32_t tabv, int d) {
    return (uint32_t)__builtin_amdgcn_readlane((int)tabv, d);
}
__device__ __forceinline__ uint64_t table_qword(uint32_t tabv, int d) {
    return (uint64_t)table_dword(tabv, d) | (uint64_t)table_dword(tabv, d + 1) << 32;
}

// block barrier over LDS written with ds_write: lgkmcnt(0), then s_barrier,
// fenced against compiler reordering (__syncthreads() would also wait for
// every buffer load in flight)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// where one row tile of the grid reads and writes
struct TileRef {
    const void* x;
    const char* w;       // first code byte of the tile's first row
    const uint16_t* s;   // scales / biases of the tile's first row
    const uint16_t* b;
    char* y;             // the problem's output matrix
    const void* bias;
    int N, row0, rows;   // problem rows, first row of the tile, rows present (0: read nothing)
};

// bytes of dynamic LDS the x table of one row of x takes: the prepared x
// words of every chunk (plus a zero chunk for lanes past the row end), then
// each chunk's sum of x
int64_t x_table_bytes(int64_t K, int bits) {
    const int64_t C = K * bits / 128, NP = (128 / bits) / 2;
    return (C + 1) * NP * 4 + (C + 1) * 4;
}
constexpr int64_t kMaxXTable = 64 * 1024;
// Rows shorter than this, and split tiles, keep the per-stage x: their
// blocks are short-lived and the table's build (an x load, then a barrier,
// before the first code load) is exposed (measured on MI355X: the 0.5B
// decode step 367 -> 389 us with the table on every shape, 378 with it on
// the split 4864 -> 896 projections only).
constexpr int64_t kMinXTableK = 2048;

// MODE 0: P holds one problem (every lookup folds to problem 0 at compile
// time); 1: P.count problems, grouped; 2: expert gather.
// XL (one row of x shared by every problem): the block prepares x once into
// an LDS table at start (the pairing the code unpack needs and each chunk's
// sum of x), and the stages read their chunk from it; otherwise every stage
// loads its x chunk and prepares it again.  The same arithmetic on the same
// values either way: the results are identical bit for bit.
//
// Arguments: what the first loads of problem 0 need, as scalars, first (the
// build preloads the leading kernel arguments into SGPRs at wave launch, so a
// single-problem wave issues its first loads without a scalar memory round
// trip; measured on MI355X, a chain of 1 MiB streaming kernels in a HIP
// graph: 2.41 -> 2.06 us per launch), then y and bias, then the table of
// every problem (grouped, gather).  meta packs M (bits 0-7), log2 group size
// (8-15), y dtype (16-23), ksplit (bit 24) and contiguous (bit 25); nblocks
// is the grid size (gridDim would be a load of the implicit arguments); tq
// and tr are the quotient and remainder of the tile count by the tile stride
// (nblocks with ksplit, else 4 nblocks), so a wave counts its tiles without
// a division.
// Contiguous (grouped only): the problems' codes, scales and biases follow
// one another in memory, every problem but the last fills whole row tiles and
// all read the same x, so the loads treat them as one matrix of n0 rows from
// the scalar bases, and only the stores look up their problem in the table.
template <int BITS, int SBT, int MT, int L, int R, int MODE, bool XL = false>
__global__ __launch_bounds__(256) void qmv_kernel(const void* x0, const uint32_t* w0, const void* s0, const void* b0,
                                                  int n0, int tq, int tr, int K, uint32_t meta, int nblocks, void* y0,
                                                  const void* bias0, const GemvProblems P) {
    const int M = (int)(meta & 0xff), gs_shift = (int)((meta >> 8) & 0xff), y_dtype = (int)((meta >> 16) & 0xff);
    constexpr int CPC_SHIFT = BITS == 4 ? 5 : 4;  // codes per 16-byte chunk: 32 or 16
    constexpr int CPC = 1 << CPC_SHIFT;
    constexpr int NP = CPC / 2;
    constexpr int NQ = NP / 4;                    // 16-byte quads of prepared x per chunk
    constexpr int SG = 64 / L;                    // sub-groups (row slots) per wave
    constexpr int TILE = SG * R;                  // rows per wave tile
    constexpr bool XPF = MT <= 2 && !XL;          // prefetch x with the codes (registers allow it)
    static_assert(!XL || (MT == 1 && MODE != 2), "x table: one shared row of x");
    using St = Stage<BITS, R, MT, XPF>;

    const int lane = threadIdx.x & 63;
    const int sg = lane / L, li = lane % L;
    // wave index, made provably wave-uniform so tile bases live in SGPRs
    const int gwave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int nwaves = nblocks * 4;
    const int C = K >> CPC_SHIFT;
    const int J = (C + L - 1) / L;  // chunk iterations per row
    uint32_t tabv = 0;
    if constexpr (MODE == 1) {
        const uint32_t* const tab = reinterpret_cast<const uint32_t*>(&P.p[0]);
        tabv = tab[lane < kMaxGroup * kProblemDwords ? lane : 0];
    }
    constexpr int kW = offsetof(GemvProblem, w) / 4, kS = offsetof(GemvProblem, s) / 4;
    constexpr int kB = offsetof(GemvProblem, b) / 4, kX = offsetof(GemvProblem, x) / 4;
    constexpr int kY = offsetof(GemvProblem, y) / 4, kBias = offsetof(GemvProblem, bias) / 4;
    constexpr int kN = offsetof(GemvProblem, n) / 4, kT0 = offsetof(GemvProblem, tile0) / 4;
    // problem owning a tile (tiles of problem p: [tile0[p], tile0[p+1]))
    auto prob_of = [&](int tile) {
        int p = 0;
        if constexpr (MODE == 1) {
#pragma unroll
            for (int i = 1; i < kMaxGroup; ++i)  // an unused slot's tile0 is the tile count: never passed
                p += tile >= (int)table_dword(tabv, i * kProblemDwords + kT0) ? 1 : 0;
            p = __builtin_amdgcn_readfirstlane(p);
        }
        return p;
    };
    // tiles and chunk iterations of this wave: its own tiles over all J chunk
    // passes, or with ksplit the block's tiles over this wave's quarter of them
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool ks = (meta >> 24) & 1;
    const int tile_first = ks ? (int)blockIdx.x : gwave;
    const int tile_stride = ks ? nblocks : nwaves;
    const int j_begin = ks ? wv * J / 4 : 0;
    const int j_count = ks ? (wv + 1) * J / 4 - j_begin : J;
    const int my_tiles = tq + (tile_first < tr ? 1 : 0);
    const int iters = my_tiles * j_count;
    // x table: quad q of chunk c at quad c*NQ + (q + (c >> ROT)) % NQ, so the
    // quads that 16 lanes read from 16 consecutive chunks cover all 64 banks;
    // the chunk sums follow
    extern __shared__ u32x4_t xtab[];
    constexpr int ROT = NQ == 4 ? 2 : 3;  // chunks per 256 bytes: 4 or 8
    __shared__ float kpart[2][4][64];  // ksplit partial sums, double-buffered by tile parity
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int G = K >> gs_shift;
    const int ysz = y_dtype == DT_F32 ? 4 : 2;
    const bool contig = MODE == 1 && ((meta >> 25) & 1);
    // the tile's bases; `store`: where its results go (contiguous groups read
    // from the scalar bases and store through the table)
    auto locate = [&](int tile, bool store) {
        TileRef t;
        if (MODE == 0 || (contig && !store)) {
            t.x = x0;
            t.row0 = tile * TILE;
            t.w = (const char*)w0 + (size_t)t.row0 * row_bytes;
            t.s = (const uint16_t*)s0 + (size_t)t.row0 * G;
            t.b = (const uint16_t*)b0 + (size_t)t.row0 * G;
            t.y = (char*)y0;
            t.bias = bias0;
            t.N = n0;
            t.rows = min(n0 - t.row0, TILE);
        } else if constexpr (MODE == 2) {
            const int b = __builtin_amdgcn_readfirstlane(tile / P.tiles_per_problem);
            const int lt = tile - b * P.tiles_per_problem;
            // a scalar load: waiting for it leaves the vector loads in flight
            const int e = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int32_t*)P.idx)[b]);
            const bool ok = e >= 0 && e < P.experts;  // an index out of range gives zero rows
            const int eb = ok ? e : 0;
            const int xm = P.x_per_expert ? b : b / P.top_k;  // x matrix of this problem
            t.x = (const uint16_t*)x0 + xm * P.x_stride;
            t.row0 = lt * TILE;
            t.w = (const char*)w0 + ((size_t)eb * n0 + t.row0) * row_bytes;
            t.s = (const uint16_t*)s0 + ((size_t)eb * n0 + t.row0) * G;
            t.b = (const uint16_t*)b0 + ((size_t)eb * n0 + t.row0) * G;
            t.y = (char*)y0 + b * P.y_stride * ysz;
            t.bias = nullptr;
            t.N = n0;
            t.rows = ok ? min(n0 - t.row0, TILE) : 0;
        } else if constexpr (MODE == 1) {
            const int p0 = prob_of(tile) * kProblemDwords;
            const int n = (int)table_dword(tabv, p0 + kN);
            t.x = (const void*)table_qword(tabv, p0 + kX);
            t.row0 = (tile - (int)table_dword(tabv, p0 + kT0)) * TILE;
            t.w = (const char*)table_qword(tabv, p0 + kW) + (size_t)t.row0 * row_bytes;
            t.s = (const uint16_t*)table_qword(tabv, p0 + kS) + (size_t)t.row0 * G;
            t.b = (const uint16_t*)table_qword(tabv, p0 + kB) + (size_t)t.row0 * G;
            t.y = (char*)table_qword(tabv, p0 + kY);
            t.bias = (const void*)table_qword(tabv, p0 + kBias);
            t.N = n;
            t.rows = min(n - t.row0, TILE);
        }
        return t;
    };
    const uint32_t xrow_bytes = (uint32_t)K * 2;
    const uint32_t kMask = vgpr_const(0x000F000Fu), kMagic = kMagic128x2;

    // x of one chunk position for every row of x (zero past the row end or m >= M)
    auto load_x = [&](__amdgpu_buffer_rsrc_t xr, uint32_t xoff, uint32_t (*xw)[NP]) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t off = m < M ? xoff + (uint32_t)m * xrow_bytes : kOOB;
#pragma unroll
            for (int i = 0; i < NP / 4; ++i) {
                const u32x4_t v = bload16(xr, off + i * 16);
                xw[m][4 * i + 0] = v[0];
                xw[m][4 * i + 1] = v[1];
                xw[m][4 * i + 2] = v[2];
                xw[m][4 * i + 3] = v[3];
            }
        }
    };
    // x sums and (4-bit) the pairing (x_j, x_{j+4}) matching unpack4_magic
    auto prep_x = [&](const uint32_t (*xw)[NP], uint32_t (*X)[NP], float* xs) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            xs[m] = 0.f;
#pragma unroll
            for (int i = 0; i < NP; ++i) xs[m] = dot2(xw[m][i], kOnesBf16x2, xs[m]);
            if constexpr (BITS == 4) {
#pragma unroll
                for (int wi = 0; wi < 4; ++wi) perm_x_for4(&xw[m][4 * wi], &X[m][4 * wi]);
            } else {
#pragma unroll
                for (int i = 0; i < NP; ++i) X[m][i] = xw[m][i];
            }
        }
    };

    // (tile, chunk iteration) of the next stage to issue and of the stage being computed
    int tile_i = tile_first, j_i = 0, tile_c = tile_first, j_c = 0, k_c = 0;
    auto issue = [&](St& st) {
        const int tile = tile_i;
        const int c = li + (j_begin + j_i) * L;
        if (++j_i == j_count) {
            j_i = 0;
            tile_i += tile_stride;
        }
        const TileRef t = locate(tile, false);
        const uint32_t valid_rows = (uint32_t)t.rows;
        // resources rebased on the tile: 32-bit offsets, and rows past N read as zero
        const auto wr = make_rsrc(t.w, valid_rows * row_bytes);
        const auto sr = make_rsrc(t.s, valid_rows * G * 2);
        const auto br = make_rsrc(t.b, valid_rows * G * 2);
        const bool cv = c < C;
        const uint32_t g = (uint32_t)((c << CPC_SHIFT) >> gs_shift);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = (uint32_t)(sg * R + r);
            st.q[r] = bload16_nt(wr, cv ? row * row_bytes + (uint32_t)c * 16 : kOOB);  // streamed once
            st.s[r] = bload2(sr, (row * G + g) * 2);
            st.b[r] = bload2(br, (row * G + g) * 2);
        }
        if constexpr (XL) st.xoff = cv ? (uint32_t)c : (uint32_t)C;  // the zero chunk past the row end
        else st.xoff = cv ? (uint32_t)c * CPC * 2 : kOOB;
        if constexpr (XPF) load_x(make_rsrc(t.x, (uint32_t)M * xrow_bytes), st.xoff, st.xw);
    };

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    auto compute = [&](const St& st) {
        uint32_t X[MT][NP];
        float xs[MT];
        if constexpr (XL) {
            const int c = (int)st.xoff;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const u32x4_t v = xtab[c * NQ + ((q + (c >> ROT)) & (NQ - 1))];
                X[0][4 * q + 0] = v[0];
                X[0][4 * q + 1] = v[1];
                X[0][4 * q + 2] = v[2];
                X[0][4 * q + 3] = v[3];
            }
            xs[0] = reinterpret_cast<const float*>(xtab + (C + 1) * NQ)[c];
        } else if constexpr (XPF) {
            prep_x(st.xw, X, xs);
        } else {
            uint32_t xw[MT][NP];
            load_x(make_rsrc(locate(tile_c, false).x, (uint32_t)M * xrow_bytes), st.xoff, xw);
            prep_x(xw, X, xs);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t p[NP];
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                if constexpr (BITS == 4) unpack4_magic(st.q[r][wi], &p[wi * 4], kMask, kMagic);
                else unpack8_pairs(st.q[r][wi], &p[wi * 2]);
            }
            const float s = half_to_f32<SBT>(st.s[r]);
            float b = half_to_f32<SBT>(st.b[r]);
            if constexpr (BITS == 4) b = fmaf(-128.f, s, b);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < NP; ++i) a = dot2(X[m][i], p[i], a);
                acc[r][m] = fmaf(s, a, acc[r][m]);
                acc[r][m] = fmaf(b, xs[m], acc[r][m]);
            }
        }
        if (++j_c == j_count) {  // tile complete: reduce over the sub-group and store
            const TileRef tc = locate(tile_c, true);
            const int N = tc.N;
            void* const y = tc.y;
            const void* const bias = tc.bias;
            const int row0 = tc.row0 + sg * R;
            j_c = 0;
            tile_c += tile_stride;
            float v[MT][R];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    v[m][r] = lane_group_sum<L>(acc[r][m]);
                    acc[r][m] = 0.f;
                }
            bool owner = true;
            if (ks) {  // the block's four partials of this tile meet in LDS; wave 0 stores
                float* const kp = kpart[k_c & 1][0];
                if (li == L - 1) {
#pragma unroll
                    for (int m = 0; m < MT; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) kp[wv * 64 + (sg * MT + m) * R + r] = v[m][r];
                }
                lds_barrier();
                owner = wv == 0;
                if (owner && li == L - 1) {
#pragma unroll
                    for (int m = 0; m < MT; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const int o = (sg * MT + m) * R + r;
                            v[m][r] = (kp[o] + kp[64 + o]) + (kp[128 + o] + kp[192 + o]);
                        }
                }
                ++k_c;
            }
            if (owner && li == L - 1) {  // holds every sum of its sub-group: one store per row of x
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m < M) store_run<R>(y, (int64_t)m * N, row0, N, y_dtype, v[m], bias);
            }
        }
    };

    // one-deep software pipeline over (tile, chunk) iterations, ping-ponging
    // between two stages so no stage is ever copied.  Without the x table the
    // first two stages are issued first thing (measured 3 % faster on the
    // 0.5B decode step than after the early exit); with it the table is
    // built first (issuing the code loads before it was 5 % slower: the
    // table's x loads then return behind the codes).
    St A, B;
    if constexpr (!XL) {
        if (iters > 0) issue(A);
        if (iters > 1) issue(B);
    }
    if constexpr (XL) {  // build the x table
        float* const xsum = reinterpret_cast<float*>(xtab + (C + 1) * NQ);
        const auto xr = make_rsrc(x0, (uint32_t)K * 2);
        for (int c = threadIdx.x; c <= C; c += 256) {
            uint32_t xw[NP], X[NP];
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                const u32x4_t v = bload16(xr, c < C ? (uint32_t)c * CPC * 2 + i * 16 : kOOB);
                xw[4 * i + 0] = v[0];
                xw[4 * i + 1] = v[1];
                xw[4 * i + 2] = v[2];
                xw[4 * i + 3] = v[3];
            }
            float xs = 0.f;
#pragma unroll
            for (int i = 0; i < NP; ++i) xs = dot2(xw[i], kOnesBf16x2, xs);
            if constexpr (BITS == 4) {
#pragma unroll
                for (int wi = 0; wi < 4; ++wi) perm_x_for4(&xw[4 * wi], &X[4 * wi]);
            } else {
#pragma unroll
                for (int i = 0; i < NP; ++i) X[i] = xw[i];
            }
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                xtab[c * NQ + ((q + (c >> ROT)) & (NQ - 1))] = u32x4_t{X[4 * q], X[4 * q + 1], X[4 * q + 2], X[4 * q + 3]};
            xsum[c] = xs;
        }
        __syncthreads();  // every wave of the block, before any of them may return
    }
    if (iters == 0) return;  // uniform over the block when ksplit (J >= 4 gives every wave chunks)
    if constexpr (XL) {
        issue(A);
        if (iters > 1) issue(B);
    }
    for (int it = 0; it < iters; it += 2) {
        if (it > 0 && it + 1 < iters) issue(B);
        compute(A);
        if (it + 1 >= iters) break;
        if (it + 2 < iters) issue(A);
        compute(B);
    }
}

// Too few row tiles to fill the chip even at one row per sub-group, and rows
// long enough (J >= 4 chunk passes) to split: the four waves of a block
// share each tile, each streaming a quarter of its chunks.
int use_ksplit(int64_t tiles, int64_t K, int bits, int L) {
    const int64_t J = (K * bits / 128 + L - 1) / L;
    return J >= 4 && tiles < kFillTiles ? 1 : 0;
}

// blocks of 4 waves: one tile per wave (or per block when split), at most
// per_cu blocks per CU, the waves then walking further tiles
int gemv_blocks(int64_t tiles, int ksplit, int per_cu = kMaxBlocksPerCU) {
    const int64_t want = ksplit ? tiles : (tiles + 3) / 4;
    return (int)(want < (int64_t)num_cus() * per_cu ? want : (int64_t)num_cus() * per_cu);
}

// the kernel's meta argument: M, log2 group size, y dtype, ksplit
uint32_t pack_meta(const QmmArgs& a, int ksplit) {
    return (uint32_t)a.M | (uint32_t)__builtin_ctz((unsigned)a.group_size) << 8 | (uint32_t)a.y_dtype << 16 |
           (uint32_t)(ksplit ? 1 : 0) << 24;
}

int64_t total_rows(const QmmArgs* a, int count) {
    int64_t n = 0;
    for (int i = 0; i < count; ++i) n += a[i].N;
    return n;
}

// whether the problems' codes, scales and biases each continue the previous
// problem's, every problem but the last fills whole tiles of `tile` rows and
// all share x: the kernel then loads them as one matrix
bool contiguous_group(const QmmArgs* a, int count, int tile) {
    const int64_t row_bytes = a[0].K * a[0].bits / 8, sb_row = a[0].K / a[0].group_size * 2;
    int64_t rows = 0;
    for (int i = 0; i < count; ++i) {
        if (a[i].x != a[0].x) return false;
        if ((const char*)a[i].w != (const char*)a[0].w + rows * row_bytes) return false;
        if ((const char*)a[i].scales != (const char*)a[0].scales + rows * sb_row) return false;
        if ((const char*)a[i].biases != (const char*)a[0].biases + rows * sb_row) return false;
        if (i + 1 < count && a[i].N % tile != 0) return false;
        rows += a[i].N;
    }
    return rows < ((int64_t)1 << 31);
}

// a[0..count) share M, K, group size, bits and dtypes; one grid covers all
// (grouped grids are built for one or two rows of x only)
template <int BITS, int SBT, int MT, int L, int R>
hipError_t launch_t(const QmmArgs* a, int count) {
    if (count > 1 && MT > 2) return hipErrorInvalidValue;
    constexpr int TILE = (64 / L) * R;
    GemvProblems P{};
    P.count = count;
    int64_t tiles = 0;
    for (int i = 0; i < kMaxGroup; ++i) {
        const QmmArgs& q = a[i < count ? i : count - 1];  // unused slots: the last problem, tile0 = the tile count
        P.p[i] = GemvProblem{q.x, q.w, q.scales, q.biases, q.y, q.bias, (int)q.N, (int)tiles};
        if (i < count) tiles += (q.N + TILE - 1) / TILE;
    }
    if (tiles >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if (tiles == 0) return hipSuccess;
    P.tiles = (int)tiles;
    P.ksplit = use_ksplit(tiles, a[0].K, a[0].bits, L);
    const int blocks = gemv_blocks(tiles, P.ksplit);
    GemvProblem p0 = P.p[0];
    const bool contig = count > 1 && contiguous_group(a, count, TILE);
    if (contig) p0.n = (int)total_rows(a, count);  // the loads' one matrix
    const uint32_t meta = pack_meta(a[0], P.ksplit) | (contig ? 1u << 25 : 0u);
    const int stride = P.ksplit ? blocks : 4 * blocks, tq = (int)(tiles / stride), tr = (int)(tiles % stride);
    if constexpr (MT == 1) {  // one row of x shared by every problem: the LDS x table
        bool shared = true;
        for (int i = 1; i < count; ++i) shared = shared && a[i].x == a[0].x;
        const int64_t xt = x_table_bytes(a[0].K, BITS);
        if (shared && !P.ksplit && a[0].K >= kMinXTableK && xt <= kMaxXTable) {
            if (count > 1)
                hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, L, R, 1, true>), dim3(blocks), dim3(256), (size_t)xt,
                                   a[0].stream, p0.x, p0.w, p0.s, p0.b, p0.n, tq, tr, (int)a[0].K, meta, blocks, p0.y, p0.bias, P);
            else
                hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, L, R, 0, true>), dim3(blocks), dim3(256), (size_t)xt,
                                   a[0].stream, p0.x, p0.w, p0.s, p0.b, p0.n, tq, tr, (int)a[0].K, meta, blocks, p0.y, p0.bias, P);
            return hipGetLastError();
        }
    }
    if constexpr (MT <= 2) {
        if (count > 1) {
            hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, L, R, 1>), dim3(blocks), dim3(256), 0, a[0].stream, p0.x,
                               p0.w, p0.s, p0.b, p0.n, tq, tr, (int)a[0].K, meta, blocks, p0.y, p0.bias, P);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, L, R, 0>), dim3(blocks), dim3(256), 0, a[0].stream, p0.x, p0.w,
                       p0.s, p0.b, p0.n, tq, tr, (int)a[0].K, meta, blocks, p0.y, p0.bias, P);
    return hipGetLastError();
}

// a: expert 0's problem (N rows each); T * top_k problems, one per (token, slot)
template <int BITS, int SBT, int MT, int L, int R>
hipError_t launch_gather_t(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_expert,
                           int64_t experts, int64_t x_stride, int64_t y_stride) {
    constexpr int TILE = (64 / L) * R;
    GemvProblems P{};
    P.count = 1;
    P.p[0] = GemvProblem{a.x, a.w, a.scales, a.biases, a.y, nullptr, (int)a.N, 0};
    P.idx = idx;
    P.top_k = top_k;
    P.x_per_expert = x_per_expert;
    P.experts = (int)experts;
    P.tiles_per_problem = (int)((a.N + TILE - 1) / TILE);
    P.x_stride = x_stride;
    P.y_stride = y_stride;
    const int64_t tiles = (int64_t)P.tiles_per_problem * T * top_k;
    if (tiles >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if (tiles == 0) return hipSuccess;
    P.tiles = (int)tiles;
    P.ksplit = use_ksplit(tiles, a.K, a.bits, L);
    const int blocks = gemv_blocks(tiles, P.ksplit, kMaxGatherBlocksPerCU);
    const int64_t stride = P.ksplit ? blocks : 4 * blocks;
    const GemvProblem& p0 = P.p[0];
    hipLaunchKernelGGL((qmv_kernel<BITS, SBT, MT, L, R, 2>), dim3(blocks), dim3(256), 0, a.stream, p0.x, p0.w, p0.s,
                       p0.b, p0.n, (int)(tiles / stride), (int)(tiles % stride), (int)a.K, pack_meta(a, P.ksplit),
                       blocks, p0.y, p0.bias, P);
    return hipGetLastError();
}

int pick_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// lanes per row: the largest of 64/32/16 whose ragged last pass idles at
// most an eighth of the lanes, else the one idling the fewest
int pick_l(int64_t K, int bits) {
    const int64_t C = K * bits / 128;
    int best = 64;
    int64_t best_waste = -1;
    for (int L : {64, 32, 16}) {
        const int64_t waste = ((C + L - 1) / L) * L - C;
        if (waste * 8 <= ((C + L - 1) / L) * L) return L;
        if (best_waste < 0 || waste < best_waste) {
            best = L;
            best_waste = waste;
        }
    }
    return best;
}

// rows per sub-group.  More rows amortise the lane reduction and the x chunk
// (M <= 2 affords 4, M <= 4 two, more rows of x one, for registers), but a
// small N then leaves most of the chip idle and the launch latency-bound: take
// the largest R that still gives kFillTiles row tiles, else 1 (measured on
// MI355X, 4-bit g64, M = 1: N = 896 runs 2.60 -> 2.16 us with R = 1, N = 9728
// 4.12 -> 3.80 us with R = 2).  One row of x with rows of at least
// kMinXTableK codes (read from the LDS x table, so more rows no longer save
// x loads): at most 2 (N = 14336 at K = 4096: 10.4 -> 9.9 us against R = 4),
// except for rows of 8192 codes or more, where four rows keep more of W in
// flight per wave (N = 8192 at K = 28672: 37.4 -> 31.3 us, N = 28672 at
// K = 8192: 31.7 -> 30.0 us; R = 1 there: 45.7 and 37.3 us).
int pick_r(int64_t M, int64_t rows, int L, int64_t K) {
    const int rmax = M <= 1 && K >= kMinXTableK ? (K >= 8192 ? 4 : 2) : M <= 2 ? 4 : M <= 4 ? 2 : 1;
    const int64_t sg = 64 / L;
    for (int r = rmax; r > 1; r /= 2)
        if ((rows + sg * r - 1) / (sg * r) >= kFillTiles) return r;
    return 1;
}

template <int BITS, int SBT, int MT, int R>
hipError_t launch_l(const QmmArgs* a, int count) {
    switch (pick_l(a[0].K, a[0].bits)) {
        case 16: return launch_t<BITS, SBT, MT, 16, R>(a, count);
        case 32: return launch_t<BITS, SBT, MT, 32, R>(a, count);
        default: return launch_t<BITS, SBT, MT, 64, R>(a, count);
    }
}

template <int BITS, int SBT, int MT>
hipError_t launch_r(const QmmArgs* a, int count, int r) {
    if constexpr (MT <= 2) {
        if (r == 4) return launch_l<BITS, SBT, MT, 4>(a, count);
        if (r == 2) return launch_l<BITS, SBT, MT, 2>(a, count);
        return launch_l<BITS, SBT, MT, 1>(a, count);
    } else if constexpr (MT == 4) {
        return launch_l<BITS, SBT, MT, 2>(a, count);
    } else {
        return launch_l<BITS, SBT, MT, 1>(a, count);
    }
}

template <int BITS, int SBT>
hipError_t launch_mt(const QmmArgs* a, int count) {
    int64_t rows = 0;
    for (int i = 0; i < count; ++i) rows += a[i].N;
    const int r = pick_r(a[0].M, rows, pick_l(a[0].K, a[0].bits), a[0].K);
    switch (pick_mt(a[0].M)) {
        case 1: return launch_r<BITS, SBT, 1>(a, count, r);
        case 2: return launch_r<BITS, SBT, 2>(a, count, r);
        case 4: return launch_r<BITS, SBT, 4>(a, count, r);
        case 8: return launch_r<BITS, SBT, 8>(a, count, r);
        default: return launch_r<BITS, SBT, 16>(a, count, r);
    }
}

}  // namespace

bool qmv_ksplit(int64_t M, int64_t N, int64_t K, int bits) {
    const int L = pick_l(K, bits);
    const int64_t tile = (64 / L) * pick_r(M, N, L, K);
    return use_ksplit((N + tile - 1) / tile, K, bits, L) != 0;
}

void qmv_config(const QmmArgs& a, int* rows_per_subgroup, int* m_tile, int* lanes_per_row) {
    if (rows_per_subgroup) *rows_per_subgroup = pick_r(a.M, a.N, pick_l(a.K, a.bits), a.K);
    if (m_tile) *m_tile = pick_mt(a.M);
    if (lanes_per_row) *lanes_per_row = pick_l(a.K, a.bits);
}

hipError_t launch_qmv_grouped(const QmmArgs* a, int count) {
    if (count < 1 || count > kMaxGroup) return hipErrorInvalidValue;
    if (a[0].bits == 4)
        return a[0].sb_dtype == DT_F16 ? launch_mt<4, DT_F16>(a, count) : launch_mt<4, DT_BF16>(a, count);
    return a[0].sb_dtype == DT_F16 ? launch_mt<8, DT_F16>(a, count) : launch_mt<8, DT_BF16>(a, count);
}

hipError_t launch_qmv(const QmmArgs& a) { return launch_qmv_grouped(&a, 1); }

namespace {
template <int BITS, int SBT, int MT, int R>
hipError_t gather_l(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int xpe, int64_t E, int64_t xs,
                    int64_t ys) {
    switch (pick_l(a.K, a.bits)) {
        case 16: return launch_gather_t<BITS, SBT, MT, 16, R>(a, idx, T, top_k, xpe, E, xs, ys);
        case 32: return launch_gather_t<BITS, SBT, MT, 32, R>(a, idx, T, top_k, xpe, E, xs, ys);
        default: return launch_gather_t<BITS, SBT, MT, 64, R>(a, idx, T, top_k, xpe, E, xs, ys);
    }
}
template <int BITS, int SBT>
hipError_t gather_mt(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int xpe, int64_t E, int64_t xs,
                     int64_t ys) {
    const int r = pick_r(a.M, a.N * T * top_k, pick_l(a.K, a.bits), 0);  // gather: no x table
    switch (pick_mt(a.M)) {
        case 1:
            return r == 4   ? gather_l<BITS, SBT, 1, 4>(a, idx, T, top_k, xpe, E, xs, ys)
                   : r == 2 ? gather_l<BITS, SBT, 1, 2>(a, idx, T, top_k, xpe, E, xs, ys)
                            : gather_l<BITS, SBT, 1, 1>(a, idx, T, top_k, xpe, E, xs, ys);
        case 2:
            return r == 4   ? gather_l<BITS, SBT, 2, 4>(a, idx, T, top_k, xpe, E, xs, ys)
                   : r == 2 ? gather_l<BITS, SBT, 2, 2>(a, idx, T, top_k, xpe, E, xs, ys)
                            : gather_l<BITS, SBT, 2, 1>(a, idx, T, top_k, xpe, E, xs, ys);
        case 4: return gather_l<BITS, SBT, 4, 2>(a, idx, T, top_k, xpe, E, xs, ys);
        case 8: return gather_l<BITS, SBT, 8, 1>(a, idx, T, top_k, xpe, E, xs, ys);
        default: return gather_l<BITS, SBT, 16, 1>(a, idx, T, top_k, xpe, E, xs, ys);
    }
}
}  // namespace

hipError_t launch_qmv_gather(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_expert,
                             int64_t experts, int64_t x_stride, int64_t y_stride) {
    if (a.M < 1 || a.M > 16) return hipErrorInvalidValue;
    const int64_t xs = x_stride, ys = y_stride;
    if (a.bits == 4)
        return a.sb_dtype == DT_F16 ? gather_mt<4, DT_F16>(a, idx, T, top_k, x_per_expert, experts, xs, ys)
                                    : gather_mt<4, DT_BF16>(a, idx, T, top_k, x_per_expert, experts, xs, ys);
    return a.sb_dtype == DT_F16 ? gather_mt<8, DT_F16>(a, idx, T, top_k, x_per_expert, experts, xs, ys)
                                : gather_mt<8, DT_BF16>(a, idx, T, top_k, x_per_expert, experts, xs, ys);
}

}  // namespace miqmm
