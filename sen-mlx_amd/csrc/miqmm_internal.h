// miqmm_internal.h -- launcher declarations shared between the kernels and
// the C ABI (api.cpp).  Host-side only types; no torch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace miqmm {

struct QmmArgs {
    void* y;
    const void* x;
    const uint32_t* w;
    const void* scales;
    const void* biases;
    const void* bias;  // optional [N] (QuantizedLinear), dtype of y
    int64_t M, N, K;
    int group_size, bits;
    int x_dtype, sb_dtype, y_dtype;
    hipStream_t stream;
};

// Up to kMaxGroup independent GEMV problems sharing M, K, group size, bits and
// dtypes, run as one grid (kernel argument, passed by value): problem p owns
// the row tiles [tile0[p], tile0[p+1]).
constexpr int kMaxGroup = 4;
struct GemvProblem {  // one problem's fields together: a single-problem kernel reads one contiguous run
    const void* x;
    const uint32_t* w;
    const void* s;
    const void* b;
    void* y;
    const void* bias;
    int n;
    int tile0;  // first row tile of this problem in the grid
};
struct GemvProblems {
    GemvProblem p[kMaxGroup];
    int tiles;  // row tiles of all problems
    int count;
    // gather mode (MoE experts): problem b = (token b / top_k, slot b % top_k)
    // multiplies its x by expert idx[b] of the stacked weights in p[0]
    const int32_t* idx;
    int top_k, x_per_expert, experts, tiles_per_problem;
    int64_t x_stride, y_stride;  // elements between consecutive x / y matrices
    // 1: the 4 waves of a block share each row tile, wave w taking the w-th
    // quarter of its chunks, and add their partial sums through LDS
    int ksplit;
};

// route launchers; return hipSuccess or the launch error
hipError_t launch_qmv(const QmmArgs& a);       // VALU dot2 GEMV
hipError_t launch_qmv_grouped(const QmmArgs* a, int count);  // same, count <= kMaxGroup problems
// whether launch_qmv on this shape alone splits K over a block's waves (a
// grouped launch never does, so such problems are launched on their own)
bool qmv_ksplit(int64_t M, int64_t N, int64_t K, int bits);
// expert-gathered GEMVs: a describes one expert (w/scales/biases = expert 0 of
// the stack), x holds T*(x_per_expert ? top_k : 1) matrices, y holds T*top_k
// matrices of N columns, x_stride / y_stride elements apart; a.M <= 16 rows of
// each are computed; idx is [T, top_k] on the device
hipError_t launch_qmv_gather(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_expert,
                             int64_t experts, int64_t x_stride, int64_t y_stride);
hipError_t launch_qmv_mfma(const QmmArgs& a);  // group-diagonal MFMA GEMV
// the same with its K split over blocks when `workspace_bytes` holds the
// partials (qmv_split_bytes; less, nullptr or unaligned scales: unsplit)
hipError_t launch_qmv_mfma_split(const QmmArgs& a, void* workspace, int64_t workspace_bytes);
// workspace bytes of the MFMA GEMV's K split for this shape (0: unsplit)
int64_t qmv_split_bytes(const QmmArgs& a);
// y = sum of ks fp32 partial planes [ks][M][N] in order, in y's dtype, + bias
hipError_t launch_split_reduce(const float* part, int ks, const QmmArgs& a);
// workspace: fp32 partials of a k split (the plan splits only where
// workspace_bytes holds them; nullptr / 0: never split)
hipError_t launch_qmm(const QmmArgs& a, void* workspace = nullptr, int64_t workspace_bytes = 0);
// workspace bytes the qmm plan's k split takes for this shape (0: unsplit)
int64_t qmm_workspace_bytes(const QmmArgs& a);
// expert grouping of gather_qmm's selections (M = 1 per selection): the
// workspace (gather_grouped_workspace bytes) holds, per expert, its range of
// the selection list, and the list of tiles of up to `tr` selections of one
// expert.  a describes expert 0 (w / scales / biases bases, N, K); T * top_k
// selections.  Two consumers: the tiled MFMA matmul (tiles of 256 rows, for
// prefill-sized batches) and the MFMA GEMV (tiles of 16 rows, for batches
// with a few selections per expert).
constexpr int kGatherGemvRows = 16;  // selections per tile of the grouped MFMA GEMV
struct GatherPlan {
    int32_t* seg;     // [E + 2]: expert e's range of perm is seg[e] .. seg[e+1] (e == E: invalid ids)
    int32_t* ntiles;  // number of tiles
    int32_t* perm;    // [S] selection ids grouped by expert
    int32_t* tiles;   // [max tiles][2]: (expert, first position in perm)
    int64_t max_tiles;
};
int64_t gather_grouped_max_tiles(int64_t S, int64_t E, int tr);
int64_t gather_grouped_workspace(int64_t S, int64_t E);  // enough for either consumer
GatherPlan gather_plan_layout(void* workspace, int64_t S, int64_t E, int tr);
hipError_t launch_gather_plan(const int32_t* idx, int64_t S, int64_t E, int tr, const GatherPlan& plan,
                              hipStream_t stream);
hipError_t launch_gather_grouped(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_index,
                                 int64_t experts, int64_t x_bytes, void* workspace);
hipError_t launch_gather_gemv(const QmmArgs& a, const int32_t* idx, int64_t T, int top_k, int x_per_index,
                              int64_t experts, int64_t x_bytes, void* workspace);
hipError_t launch_qmvx(const QmmArgs& a);      // MFMA GEMV, M <= 4, x in LDS
hipError_t launch_qmvs(const QmmArgs& a);      // K-sliced v_dot2 GEMV, M == 1
// M == 1, at most 15 K-slices, an even number of groups per row (the scale
// and bias pointers must also be 4-byte aligned, checked by the caller)
bool qmvs_supported(int64_t M, int64_t N, int64_t K, int bits, int group_size);
// a[0..count) (2..4 problems, M == 1) share x and store their codes, scales
// and biases one after another (a loader that fuses q/k/v or gate/up): the
// K-sliced GEMV reads them as one matrix and writes each problem's rows to
// its own output
bool qmvs_group_ok(const QmmArgs* a, int count);
hipError_t launch_qmvs_grouped(const QmmArgs* a, int count);
// compute units of the current device (queried once per device): the GEMV
// grids are sized by it
int num_cus();
bool qmvx_supported(int64_t M, int64_t K, int group_size);

// tiling used for a given problem; for reporting
void qmv_config(const QmmArgs& a, int* rows_per_subgroup, int* m_tile, int* lanes_per_row);
void qmv_mfma_config(const QmmArgs& a, int* tiles_per_block, int* m_tile, int* waves_per_block);
// ks: k ranges of the plan given a large enough workspace (split when > 1)
void qmm_config(const QmmArgs& a, int* bm, int* bn, int* bk, int* ks);
void qmvx_config(const QmmArgs& a, int* m_tile, int* k_splits, int* stage_codes);
void qmvs_config(const QmmArgs& a, int* rows_per_block, int* slices, int* blocks);

hipError_t launch_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                             int64_t N, int64_t K, int group_size, int bits, int sb_dtype,
                             int out_dtype, hipStream_t stream);
hipError_t launch_embedding(void* out, const int32_t* ids, int64_t T, const uint32_t* w, const void* scales,
                            const void* biases, int64_t V, int64_t K, int group_size, int bits, int sb_dtype,
                            int out_dtype, hipStream_t stream);
hipError_t launch_unpack(uint8_t* codes, const uint32_t* w, int64_t N, int64_t K, int bits,
                         hipStream_t stream);
hipError_t launch_stream_read(const void* p, int64_t bytes, void* sink, hipStream_t stream);
hipError_t launch_synth(void* x, uint32_t* w, void* scales, void* biases, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int x_dtype, int sb_dtype,
                        uint64_t seed, uint64_t stream_id, hipStream_t stream);

}  // namespace miqmm
