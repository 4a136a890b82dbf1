/*
 * miqmm.h -- C ABI of the MI355X (gfx950) affine group-quantized matmul.
 *
 * Drop-in for the quantized-projection hot path of SenClaw/sen-mlx, which
 * calls MLX's
 *     quantized_matmul(x, w, scales, biases, transpose=true, group_size, bits)
 * through mlx-rs (call shape: src/engine/mlx_lm/utils/mod.rs:70-78,
 * src/engine/mlx_lm/models/bonsai_q1.rs:469-477) on every QuantizedLinear
 * projection (src/engine/mlx_lm/models/llama.rs:195-197,249,293-294) and tied
 * lm_head (llama.rs:511-517).  mlx-rs binds it to mlx-c's C function of the
 * same name, whose conventions (int status, 0 = ok; caller-owned result;
 * borrowed inputs; explicit stream) are those shown for the sibling op at
 * src/engine/mlx_lm/utils/moe.rs:50-76.  This header keeps those conventions
 * with plain device pointers instead of mlx_array handles.
 *
 * Layout (MLX affine quantization, transpose=true):
 *   x       [M, K]            activation, row-major, dtype x_dtype (bf16)
 *   w       [N, K*bits/32]    uint32 words; code k of row n is bits
 *                             bits*(k mod 32/bits) .. of word k/(32/bits), LSB first
 *   scales  [N, K/group_size] dtype sb_dtype (bf16 or fp16)
 *   biases  [N, K/group_size] dtype sb_dtype
 *   y       [M, N]            dtype y_dtype (bf16, fp16 or fp32)
 *   y[m,n] = sum_k x[m,k] * (scales[n,k/g] * q[n,k] + biases[n,k/g])
 *
 * All pointers are device pointers owned by the caller; no entry point
 * allocates device memory, synchronizes or waits on the host.  Calls are
 * asynchronous on `stream` (a hipStream_t; NULL = the default stream) and may
 * be captured into a HIP graph.  Every function returns a miqmm_status; on
 * failure miqmm_last_error() returns a message for the calling thread.
 * Calls are safe from several threads on distinct streams, except
 * miqmm_quantized_matmul_noalloc (see there).
 */
#ifndef MIQMM_H
#define MIQMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MIQMM_OK = 0,
    MIQMM_EINVAL = 1,  /* bad shape, pointer, alignment or argument value */
    MIQMM_ENOTSUP = 2, /* valid for MLX but not provided here (e.g. transpose=false, bits=2) */
    MIQMM_EHIP = 3     /* a HIP runtime error; miqmm_last_error() names it */
} miqmm_status;

typedef enum { MIQMM_DT_BF16 = 0, MIQMM_DT_F16 = 1, MIQMM_DT_F32 = 2 } miqmm_dtype;

/* QMV: small-M GEMV on MFMA with exact integer codes; QMM: large-M tiled MFMA
 * with bf16-dequantized W tiles; QMV_DOT: small-M GEMV on v_dot2 (no MFMA);
 * QMVX: small-M GEMV on MFMA with x staged in LDS (M <= 4 per pass, needs
 * K/group_size even and min(M,4)*K <= 32768); QMVS: GEMV on v_dot2 for one to
 * four rows of x with K cut into 1 KiB slices of codes, one wave per slice, or
 * two rows of W per wave on rows of at most 32 chunks (M <= 4, needs
 * K*bits/8 <= 15 KiB -- 8 KiB with M > 2 --, K/group_size even, scales and
 * biases 4-byte aligned; each wave dots its unpacked codes with every row of
 * x). */
typedef enum {
    MIQMM_ROUTE_AUTO = 0,
    MIQMM_ROUTE_QMV = 1,
    MIQMM_ROUTE_QMM = 2,
    MIQMM_ROUTE_QMV_DOT = 3,
    MIQMM_ROUTE_QMVX = 4,
    MIQMM_ROUTE_QMVS = 5
} miqmm_route;

/*
 * y = quantized_matmul(x, w, scales, biases, transpose, group_size, bits).
 * Replaces mlx_rs::ops::quantized_matmul / mlx-c mlx_quantized_matmul
 * (reached at src/engine/mlx_lm/utils/mod.rs:70-78 and from every
 * QuantizedLinear::forward).  transpose must be 1; bits in {4, 8};
 * group_size in {32, 64, 128}; K % group_size == 0; x and w 16-byte aligned.
 * M == 0 is a no-op.  Route (HBM-bound GEMVs for M <= 32): M <= 4 -> qmvs
 * wherever it takes the shape (K*bits/8 <= 15 KiB, 8 KiB with M > 2;
 * K/group_size even; 4-byte aligned scales and biases); else M == 1 ->
 * qmv_dot, or qmvx for N >= 65536 with K <= 2048; 2 <= M <= 4 -> qmvx where
 * supported, else qmv (or qmv_dot with an odd K/group_size); M <= 16 -> qmv;
 * M <= 32 (64 with K >= 8192) -> the GEMVs in passes of 16 rows of x, the
 * last pass routed by its own rows;
 * else qmm (MFMA-bound tiled matmul).
 */
int miqmm_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                           int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                           void* stream);

/*
 * One projection of a grouped call: y = quantized_matmul(x, w, scales, biases)
 * (+ bias when non-null), N output rows.
 */
typedef struct miqmm_problem {
    void* y;
    const void* x;
    const uint32_t* w;
    const void* scales;
    const void* biases;
    const void* bias;
    int64_t N;
} miqmm_problem;

/*
 * Several independent projections that share M, K, group_size, bits and
 * dtypes.  When M <= 2 and every N < 65536 (decode projections) they run as
 * one launch per four problems:
 *  - M == 1, up to four problems sharing x (the same pointer), on rows the
 *    K-sliced GEMV takes (K*bits/8 <= 15 KiB, K/group_size even) with 4-byte
 *    aligned scales and biases: one K-sliced GEMV over all their rows, each
 *    row stored to its problem's output; every result equals, bit for bit,
 *    the matching rows of miqmm_quantized_matmul_ex with MIQMM_ROUTE_QMVS on
 *    the problems' matrices stacked into one (plus the bias as
 *    miqmm_quantized_linear adds it).  Codes, scales and biases stored one
 *    after another (a loader that fuses q/k/v or gate/up) are read as that
 *    one matrix; in separate allocations each block reads one problem's
 *    rows, which costs one scalar memory round trip per launch more;
 *  - otherwise one v_dot2 GEMV launch per four problems, each result equal,
 *    bit for bit, to miqmm_quantized_matmul_ex with MIQMM_ROUTE_QMV_DOT on it
 *    alone (plus the bias).
 * Else one call per problem on its own route, each equal to
 * miqmm_quantized_matmul (or miqmm_quantized_linear) on it alone.  This has
 * no single counterpart in the reference: it replaces the reference's
 * separate quantized projections that read the same activation -- q/k/v
 * (src/engine/mlx_lm/models/llama.rs:195-197) and gate/up (:293-294) --
 * whose decode-step launches are otherwise latency-bound.
 */
int miqmm_quantized_matmul_grouped(const miqmm_problem* problems, int count, int64_t M, int64_t K,
                                   int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                                   void* stream);

/*
 * As miqmm_quantized_matmul, with the route forced (MIQMM_ROUTE_QMV and
 * MIQMM_ROUTE_QMV_DOT accept any M, one pass over W per 16 rows of x;
 * MIQMM_ROUTE_QMM any M >= 1).
 * Used by tests to hold both routes to the same oracle on one shape.
 */
int miqmm_quantized_matmul_ex(void* y, const void* x, const uint32_t* w, const void* scales,
                              const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                              int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                              int route, void* stream);

/*
 * Bytes of scratch that miqmm_quantized_matmul_ws would use for this shape
 * (fp32 partials of a k split: k ranges * M * N * 4, else 0).  The tiled
 * matmul (larger M) splits its k-steps over several blocks per output tile
 * when the output tiles are fewer than the CUs; the small-M MFMA GEMV
 * (5 <= M <= 16 rows per pass) splits K over blocks of 128 rows, each reading its range
 * of x once, for rows of K >= 8192 codes and, at M > 8, outputs of
 * N >= 8192.
 * No reference counterpart: the workspace query of the caller that can
 * pass scratch memory.
 */
int miqmm_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                          int64_t* bytes);

/*
 * miqmm_quantized_matmul (+ bias when non-null, as miqmm_quantized_linear)
 * with a caller-owned device workspace (16-byte aligned, any contents;
 * NULL / 0 bytes: no split).  With at least
 * miqmm_quantized_matmul_workspace_size bytes the tiled matmul or the small-M
 * GEMV may split K over several blocks, write fp32 partials there and add
 * them in a second kernel in split order (the same bits for any grid);
 * with less it runs unsplit, exactly as miqmm_quantized_matmul.  The call
 * only reads and writes the workspace on `stream`: the caller keeps it alive
 * until the work completes (a workspace captured into a graph stays in use
 * by every replay) and must not share it between calls that may overlap.
 * No reference counterpart beyond quantized_matmul itself: the caller that
 * can pass scratch memory for prefill-sized products and few-row batches.
 */
int miqmm_quantized_matmul_ws(void* y, const void* x, const uint32_t* w, const void* scales,
                              const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                              int transpose, int group_size, int bits, int x_dtype, int sb_dtype,
                              int y_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * miqmm_quantized_matmul_ws with the library's own scratch in place of a
 * workspace argument: allocates nothing (no hipMalloc, no allocating library
 * call), for callers that cannot allocate -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid it.  The scratch is a 32 MiB
 * device array the code object holds on every GPU the library runs on (kept
 * until the process ends); a shape whose k split needs more
 * (miqmm_quantized_matmul_workspace_size > 32 MiB) returns MIQMM_EINVAL
 * instead.  Every call on a GPU shares that GPU's array: calls that may
 * overlap on one GPU (several streams, threads or graph replays in flight at
 * once) race on it and must be serialized by the caller.  No counterpart in
 * the reference.
 */
int miqmm_quantized_matmul_noalloc(void* y, const void* x, const uint32_t* w, const void* scales,
                                   const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                                   int transpose, int group_size, int bits, int x_dtype, int sb_dtype,
                                   int y_dtype, void* stream);

/*
 * QuantizedLinear forward: y = quantized_matmul(...) rounded to y_dtype, then
 * + bias[n] rounded again (bias may be NULL; dtype y_dtype), i.e. the two ops
 * of MaybeQuantized<Linear>::forward for a quantized slot with a bias
 * (src/engine/mlx_lm/models/llama.rs:94-98,139-147 q/k/v bias of Qwen2).
 */
int miqmm_quantized_linear(void* y, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                           int group_size, int bits, int x_dtype, int sb_dtype, int y_dtype,
                           void* stream);

/*
 * Expert-gathered quantized matmul:
 *   y[b, j] = x[b or (b, j)] @ dequant(w[rhs_indices[b, j]]).T
 * for b < batch, j < top_k, each product an M x N matrix (b-major, then j).
 * w: the stacked experts, [experts, N, K*bits/32] uint32; scales / biases
 * [experts, N, K/group_size].  rhs_indices: [batch, top_k] int32 on the
 * device.  x_per_index = 0: x holds batch matrices [M, K], each shared by
 * its top_k selections (the SwitchGLU gate / up projections,
 * x [..., 1, 1, K]); 1: x holds batch*top_k matrices, one per selection
 * (the down projection, h [..., top_k, 1, K]).  An index outside
 * [0, experts) yields zero rows instead of an out-of-bounds read.
 * sorted_indices is accepted as a hint and changes nothing.
 * Replaces mlx_sys::mlx_gather_qmm as wrapped by
 * src/engine/mlx_lm/utils/moe.rs:33-77 (lhs_indices absent, transpose=true),
 * called from src/engine/mlx_lm/models/deepseek_v2.rs:430-442 and
 * src/engine/mlx_lm/models/gemma4.rs:770-782.
 */
int miqmm_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                     const int32_t* rhs_indices, int64_t batch, int64_t top_k, int x_per_index, int64_t M,
                     int64_t N, int64_t K, int64_t experts, int transpose, int group_size, int bits, int x_dtype,
                     int sb_dtype, int y_dtype, int sorted_indices, void* stream);

/*
 * out[n, k] = scales[n,k/g] * q[n,k] + biases[n,k/g] (fp32 fma, stored as
 * out_dtype).  Replaces mlx_rs::ops::dequantize as used beside the
 * reference's quantized-matmul test (src/engine/mlx_lm/utils/moe.rs:118-126).
 */
int miqmm_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                     int64_t N, int64_t K, int group_size, int bits, int sb_dtype, int out_dtype,
                     void* stream);

/*
 * miqmm_gather_qmm with a caller-provided device workspace (16-byte aligned,
 * at least miqmm_gather_qmm_workspace_size bytes).  With M == 1 and enough
 * selections per expert, the selections are grouped by expert on the device
 * and each selected expert's weights are streamed once instead of once per
 * selection: from 8 selections per expert on average (prefill-sized batches)
 * through the tiled MFMA matmul (the qmm route's arithmetic: W rounded to
 * bf16 after the fp32 dequant), from 4 through the MFMA GEMV, 16 selections
 * per tile (exact fp32 dequant, as the GEMV routes); otherwise, or without a
 * workspace, this is miqmm_gather_qmm.  No counterpart in the reference (its
 * wrapper, src/engine/mlx_lm/utils/moe.rs:33-77, always passes
 * sorted_indices=false): the caller that can pass scratch memory for it.
 */
int miqmm_gather_qmm_workspace_size(int64_t batch, int64_t top_k, int64_t experts, int64_t* bytes);
int miqmm_gather_qmm_ws(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                        const int32_t* rhs_indices, int64_t batch, int64_t top_k, int x_per_index, int64_t M,
                        int64_t N, int64_t K, int64_t experts, int transpose, int group_size, int bits, int x_dtype,
                        int sb_dtype, int y_dtype, int sorted_indices, void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * Quantized embedding lookup: out[t, k] = scales[id,k/g] * q[id,k] +
 * biases[id,k/g] (fp32 fma, stored as out_dtype) with id = ids[t], for
 * t < T, from a table of V rows of K codes (w [V, K*bits/32], scales and
 * biases [V, K/g]).  An id outside [0, V) gives a zero row.  ids: int32 on
 * the device.  Replaces QuantizedEmbedding::forward as the reference
 * restates it (src/engine/mlx_lm/models/bonsai_q1.rs:603-613: take the rows,
 * then mlx dequantize), the step before the first projection of every token;
 * the table is the one loaded at src/engine/mlx_native.rs:3532-3560,3712-3731.
 */
int miqmm_quantized_embedding(void* out, const int32_t* ids, int64_t T, const uint32_t* w, const void* scales,
                              const void* biases, int64_t V, int64_t K, int group_size, int bits, int sb_dtype,
                              int out_dtype, void* stream);

/*
 * codes[n*K + k] = q[n, k] (uint8): the kernels' unpacking convention,
 * exposed so it can be checked bit-exactly against the packed layout of
 * src/engine/mlx_lm/models/bonsai_q1.rs:137-143 (bits=1), generalised.
 */
int miqmm_unpack(uint8_t* codes, const uint32_t* w, int64_t N, int64_t K, int bits, void* stream);

/*
 * Which route and tiling miqmm_quantized_matmul picks for a shape (host
 * only, no GPU access).  route_out: a miqmm_route.  tile_out[4]:
 * qmv -> {16-row tiles per block, M tile, waves per block, 0};
 * qmv_dot -> {rows per lane group, M tile, lanes per row, 0};
 * qmvs -> {rows per block, K-slices (waves) per block, blocks, 0};
 * qmm -> {BM, BN, BK, k ranges} (k ranges > 1: with a large enough
 * workspace, miqmm_quantized_matmul_ws splits the k-steps over that many
 * blocks per output tile; miqmm_quantized_matmul never splits).
 * No reference counterpart: reporting for benches and tests.
 */
int miqmm_query_route(int64_t M, int64_t N, int64_t K, int group_size, int bits, int* route_out,
                      int* tile_out);

/*
 * Seeded synthetic problem on the device, bit-identical to the oracle's
 * generator: x ~ N(0,1) (Irwin-Hall(4)), codes uniform in [0, 2^bits),
 * scales = |N(0,1)|*0.02, biases = -2^(bits-1)*scale + N(0,1)*0.002.  Any
 * of x, w, scales/biases may be NULL to skip it.  No reference counterpart:
 * input generation for benches and tests.
 */
int miqmm_synth_problem(void* x, uint32_t* w, void* scales, void* biases, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int x_dtype, int sb_dtype,
                        uint64_t seed, uint64_t stream_id, void* stream);

/*
 * A plain streaming read of bytes (a multiple of 16384, below 2^31) from p
 * (16-byte aligned): 16-byte non-temporal loads, 16 KiB per block, nothing
 * written (sink: 4 KiB the kernel could write, never does in practice).
 * No reference counterpart: the bandwidth ceiling the GEMVs are measured
 * against in the benchmark.
 */
int miqmm_stream_read(const void* p, int64_t bytes, void* sink, void* stream);

/* Message for the last failing call on this thread ("" if none). */
const char* miqmm_last_error(void);

/* Library version string. */
const char* miqmm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MIQMM_H */
