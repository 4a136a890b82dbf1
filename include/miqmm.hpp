// miqmm.hpp -- C++ host layer over the C ABI (miqmm.h), mirroring the
// operator surface the reference engine programs against (mlx-rs, Rust):
//
//   ops::quantized_matmul(x, w, scales, biases, transpose, group_size, bits)
//       -> Result<Array, Exception>          src/engine/mlx_lm/utils/mod.rs:70-78
//   nn::QuantizedLinear / MaybeQuantized<Linear>::forward(&Array)
//       -> Result<Array, Exception>          src/engine/mlx_lm/models/llama.rs:115-126,195-197
//   ops::dequantize(w, scales, biases, group_size, bits)
//                                            src/engine/mlx_lm/utils/moe.rs:118-126
//   gather_qmm(x, w, scales, biases, None, Some(indices), true, g, bits, false)
//       -> Result<Array, Exception>          src/engine/mlx_lm/utils/moe.rs:33-77
//   SwitchLinear::forward(x, indices)         src/engine/mlx_lm/models/deepseek_v2.rs:397-445
//   QuantizedEmbedding::forward / as_linear   src/engine/mlx_lm/models/bonsai_q1.rs:603-613,
//                                            src/engine/mlx_lm/models/llama.rs:511-517
//   the quantized half of load_llama_any      src/engine/mlx_native.rs:3585-3760
//
// Arrays here are non-owning views of device memory (pointer, shape, dtype);
// the caller allocates outputs, as the engine's allocator would.  Failures throw
// miqmm::Exception carrying the C status, the counterpart of mlx-rs's
// Exception built from a nonzero mlx-c status (moe.rs:66-76).
#pragma once

#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <vector>

#include "miqmm.h"
#include "miqmm_checkpoint.h"

namespace miqmm {

enum class Dtype : int { bfloat16 = MIQMM_DT_BF16, float16 = MIQMM_DT_F16, float32 = MIQMM_DT_F32, uint32 = 16,
                        int32 = 17 };

class Exception : public std::runtime_error {
   public:
    Exception(int status, const std::string& what) : std::runtime_error(what), status_(status) {}
    int status() const { return status_; }

   private:
    int status_;
};

inline void check(int status) {
    if (status != MIQMM_OK) throw Exception(status, std::string("miqmm: ") + miqmm_last_error());
}

inline void check_bits(int bits) {  // same statuses as the C ABI, before any shape math
    if (bits != 4 && bits != 8)
        throw Exception(bits == 2 || bits == 3 || bits == 5 || bits == 6 ? MIQMM_ENOTSUP : MIQMM_EINVAL,
                        "miqmm: bits must be 4 or 8");
}

// non-owning device array view (row-major, contiguous)
struct Array {
    void* data = nullptr;
    std::vector<int64_t> shape;
    Dtype dtype = Dtype::bfloat16;

    Array() = default;
    Array(void* d, std::initializer_list<int64_t> s, Dtype t) : data(d), shape(s), dtype(t) {}
    Array(void* d, std::vector<int64_t> s, Dtype t) : data(d), shape(std::move(s)), dtype(t) {}
    int64_t dim(int i) const { return shape.at(i < 0 ? shape.size() + i : i); }
    int64_t size() const {
        int64_t n = 1;
        for (int64_t v : shape) n *= v;
        return n;
    }
};

// MLX type promotion of (x, scales, biases): equal dtypes are kept; bfloat16
// with float16 (or anything with float32) gives float32.
inline Dtype result_type(Dtype x, Dtype scales) { return x == scales ? x : Dtype::float32; }

// out [..., N] = x [..., K] @ dequant(w, scales, biases).T (transpose=true)
inline void quantized_matmul(Array& out, const Array& x, const Array& w, const Array& scales,
                             const Array& biases, bool transpose, int group_size, int bits,
                             void* stream = nullptr, const Array* bias = nullptr) {
    check_bits(bits);
    if (w.shape.size() != 2 || w.dtype != Dtype::uint32)
        throw Exception(MIQMM_EINVAL, "miqmm: w must be a 2-D uint32 array");
    if (x.shape.empty()) throw Exception(MIQMM_EINVAL, "miqmm: x must have at least one dimension");
    const int64_t N = w.dim(0), K = w.dim(1) * 32 / bits;
    if (x.dim(-1) != K) throw Exception(MIQMM_EINVAL, "miqmm: x inner dimension does not match w");
    const int64_t M = x.size() / K;
    if (out.size() != M * N || out.dim(-1) != N)
        throw Exception(MIQMM_EINVAL, "miqmm: out must have shape [..., N] with x's leading dims");
    if (bias) {
        check(miqmm_quantized_linear(out.data, x.data, static_cast<const uint32_t*>(w.data), scales.data,
                                     biases.data, bias->data, M, N, K, group_size, bits, (int)x.dtype,
                                     (int)scales.dtype, (int)out.dtype, stream));
        return;
    }
    check(miqmm_quantized_matmul(out.data, x.data, static_cast<const uint32_t*>(w.data), scales.data,
                                 biases.data, M, N, K, transpose ? 1 : 0, group_size, bits, (int)x.dtype,
                                 (int)scales.dtype, (int)out.dtype, stream));
}

// out [N, K] = scales * q + biases per group
inline void dequantize(Array& out, const Array& w, const Array& scales, const Array& biases,
                       int group_size, int bits, void* stream = nullptr) {
    check_bits(bits);
    const int64_t N = w.dim(0), K = w.dim(1) * 32 / bits;
    if (out.size() != N * K) throw Exception(MIQMM_EINVAL, "miqmm: out must be [N, K]");
    check(miqmm_dequantize(out.data, static_cast<const uint32_t*>(w.data), scales.data, biases.data, N, K,
                           group_size, bits, (int)scales.dtype, (int)out.dtype, stream));
}

// nn::QuantizedLinear: packed weight [out, in*bits/32], scales/biases
// [out, in/group_size], optional bias [out]
class QuantizedLinear {
   public:
    QuantizedLinear(Array weight, Array scales, Array biases, int group_size = 64, int bits = 4,
                    const Array* bias = nullptr)
        : weight_(std::move(weight)), scales_(std::move(scales)), biases_(std::move(biases)),
          group_size_(group_size), bits_(bits), has_bias_(bias != nullptr) {
        if (bias) bias_ = *bias;
        if (scales_.shape != biases_.shape || scales_.shape.size() != 2 ||
            scales_.dim(0) != weight_.dim(0) || scales_.dim(1) * group_size_ != in_features())
            throw Exception(MIQMM_EINVAL, "miqmm: QuantizedLinear weight/scales/biases shapes disagree");
    }
    int64_t out_features() const { return weight_.dim(0); }
    int64_t in_features() const { return weight_.dim(1) * 32 / bits_; }

    void forward(Array& out, const Array& x, void* stream = nullptr) const {
        quantized_matmul(out, x, weight_, scales_, biases_, true, group_size_, bits_, stream,
                         has_bias_ ? &bias_ : nullptr);
    }

   private:
    Array weight_, scales_, biases_, bias_;
    int group_size_, bits_;
    bool has_bias_;
};

// Device scratch for gather_qmm's expert-grouped path (see
// gather_qmm_workspace_size); a default Workspace withholds it.
struct Workspace {
    void* data = nullptr;
    int64_t bytes = 0;
};

inline int64_t gather_qmm_workspace_size(int64_t batch, int64_t top_k, int64_t experts) {
    int64_t bytes = 0;
    check(miqmm_gather_qmm_workspace_size(batch, top_k, experts, &bytes));
    return bytes;
}

// out [*B, M, N] = x [..., M, K] @ dequant(w[rhs_indices]).T over the batch
// B = rhs_indices.shape.  w: stacked experts [E, N, K*bits/32] uint32,
// scales / biases [E, N, K/group_size], rhs_indices int32.  x's batch dims
// either equal B (one x matrix per selection: the down projection) or equal
// a prefix of B followed by ones (x shared by the trailing selections: the
// gate / up projections, x [..., 1, 1, K] against indices [..., top_k]);
// other broadcasts throw EINVAL (materialise x first).  An index outside
// [0, E) gives zero rows.
inline void gather_qmm(Array& out, const Array& x, const Array& w, const Array& scales, const Array& biases,
                       const Array& rhs_indices, bool transpose, int group_size, int bits,
                       bool sorted_indices = false, void* stream = nullptr, Workspace workspace = {}) {
    check_bits(bits);
    if (w.shape.size() != 3 || w.dtype != Dtype::uint32 || scales.shape.size() != 3 ||
        scales.shape != biases.shape || scales.dim(0) != w.dim(0) || scales.dim(1) != w.dim(1))
        throw Exception(MIQMM_EINVAL, "miqmm: w must be [E, N, K*bits/32] uint32 with scales/biases [E, N, K/g]");
    if (rhs_indices.dtype != Dtype::int32) throw Exception(MIQMM_EINVAL, "miqmm: rhs_indices must be int32");
    const int64_t E = w.dim(0), N = w.dim(1), K = w.dim(2) * 32 / bits;
    if (x.shape.size() < 2 || x.dim(-1) != K) throw Exception(MIQMM_EINVAL, "miqmm: x must be [..., M, K]");
    const int64_t M = x.dim(-2);
    const std::vector<int64_t>& B = rhs_indices.shape;
    const size_t xr = x.shape.size() - 2;
    if (xr > B.size()) throw Exception(MIQMM_EINVAL, "miqmm: x has more batch dims than rhs_indices");
    std::vector<int64_t> xb(B.size() - xr, 1);
    xb.insert(xb.end(), x.shape.begin(), x.shape.end() - 2);
    size_t j = B.size();
    while (j > 0 && xb[j - 1] == 1) --j;
    int64_t batch = 1, top_k = 1;
    for (size_t i = 0; i < B.size(); ++i) (i < j ? batch : top_k) *= B[i];
    if (!std::equal(xb.begin(), xb.begin() + j, B.begin()))
        throw Exception(MIQMM_EINVAL, "miqmm: x batch dims must be rhs_indices' dims or a prefix of them then ones");
    const int per_index = top_k == 1 ? 1 : 0;
    std::vector<int64_t> oshape(B);
    oshape.push_back(M);
    oshape.push_back(N);
    if (out.shape != oshape) throw Exception(MIQMM_EINVAL, "miqmm: out must have shape [*rhs_indices.shape, M, N]");
    check(miqmm_gather_qmm_ws(out.data, x.data, static_cast<const uint32_t*>(w.data), scales.data, biases.data,
                              static_cast<const int32_t*>(rhs_indices.data), batch, top_k, per_index, M, N, K, E,
                              transpose ? 1 : 0, group_size, bits, (int)x.dtype, (int)scales.dtype,
                              (int)out.dtype, sorted_indices ? 1 : 0, workspace.data, workspace.bytes, stream));
}

// out [*ids.shape, K] = dequantize(w[ids], scales[ids], biases[ids]); an id
// outside [0, V) gives a zero row.
inline void quantized_embedding(Array& out, const Array& ids, const Array& w, const Array& scales,
                                const Array& biases, int group_size, int bits, void* stream = nullptr) {
    check_bits(bits);
    if (w.shape.size() != 2 || w.dtype != Dtype::uint32)
        throw Exception(MIQMM_EINVAL, "miqmm: w must be a 2-D uint32 array");
    if (ids.dtype != Dtype::int32) throw Exception(MIQMM_EINVAL, "miqmm: ids must be int32");
    const int64_t V = w.dim(0), K = w.dim(1) * 32 / bits, T = ids.size();
    std::vector<int64_t> oshape(ids.shape);
    oshape.push_back(K);
    if (out.shape != oshape) throw Exception(MIQMM_EINVAL, "miqmm: out must have shape [*ids.shape, K]");
    check(miqmm_quantized_embedding(out.data, static_cast<const int32_t*>(ids.data), T,
                                    static_cast<const uint32_t*>(w.data), scales.data, biases.data, V, K,
                                    group_size, bits, (int)scales.dtype, (int)out.dtype, stream));
}

// Stacked quantized experts (the switch_mlp projections): forward is gather_qmm.
class SwitchLinear {
   public:
    SwitchLinear(Array weight, Array scales, Array biases, int group_size = 64, int bits = 4)
        : weight_(std::move(weight)), scales_(std::move(scales)), biases_(std::move(biases)),
          group_size_(group_size), bits_(bits) {
        check_bits(bits_);
        if (weight_.shape.size() != 3 || scales_.shape != biases_.shape || scales_.shape.size() != 3 ||
            scales_.dim(0) != weight_.dim(0) || scales_.dim(1) != weight_.dim(1) ||
            scales_.dim(2) * group_size_ != in_features())
            throw Exception(MIQMM_EINVAL, "miqmm: SwitchLinear weight/scales/biases shapes disagree");
    }
    int64_t experts() const { return weight_.dim(0); }
    int64_t out_features() const { return weight_.dim(1); }
    int64_t in_features() const { return weight_.dim(2) * 32 / bits_; }

    void forward(Array& out, const Array& x, const Array& indices, void* stream = nullptr,
                 Workspace workspace = {}) const {
        gather_qmm(out, x, weight_, scales_, biases_, indices, true, group_size_, bits_, false, stream, workspace);
    }

   private:
    Array weight_, scales_, biases_;
    int group_size_, bits_;
};

// Quantized token table: forward looks rows up, as_linear is the tied lm_head.
class QuantizedEmbedding {
   public:
    QuantizedEmbedding(Array weight, Array scales, Array biases, int group_size = 64, int bits = 4)
        : weight_(std::move(weight)), scales_(std::move(scales)), biases_(std::move(biases)),
          group_size_(group_size), bits_(bits) {
        check_bits(bits_);
        if (weight_.shape.size() != 2 || scales_.shape != biases_.shape || scales_.shape.size() != 2 ||
            scales_.dim(0) != weight_.dim(0) || scales_.dim(1) * group_size_ != dims())
            throw Exception(MIQMM_EINVAL, "miqmm: QuantizedEmbedding weight/scales/biases shapes disagree");
    }
    int64_t vocab() const { return weight_.dim(0); }
    int64_t dims() const { return weight_.dim(1) * 32 / bits_; }

    void forward(Array& out, const Array& ids, void* stream = nullptr) const {
        quantized_embedding(out, ids, weight_, scales_, biases_, group_size_, bits_, stream);
    }
    void as_linear(Array& out, const Array& x, void* stream = nullptr) const {
        quantized_matmul(out, x, weight_, scales_, biases_, true, group_size_, bits_, stream);
    }

   private:
    Array weight_, scales_, biases_;
    int group_size_, bits_;
};

// An opened MLX model directory (config.json + safetensors shards): the
// quantized modules with their bits / group size, and the tensors' bytes.
class Checkpoint {
   public:
    explicit Checkpoint(const std::string& model_dir) {
        const int st = miqmm_checkpoint_open(model_dir.c_str(), &h_);
        if (st != MIQMM_OK) throw Exception(st, std::string("miqmm: ") + miqmm_checkpoint_last_error());
    }
    ~Checkpoint() { miqmm_checkpoint_close(h_); }
    Checkpoint(const Checkpoint&) = delete;
    Checkpoint& operator=(const Checkpoint&) = delete;

    std::vector<miqmm_qmodule> modules() const {
        std::vector<miqmm_qmodule> out(static_cast<size_t>(miqmm_checkpoint_num_modules(h_)));
        for (size_t i = 0; i < out.size(); ++i) ck(miqmm_checkpoint_module(h_, (int64_t)i, &out[i]));
        return out;
    }
    miqmm_tensor_info tensor(const std::string& name) const {
        miqmm_tensor_info t;
        ck(miqmm_checkpoint_tensor(h_, name.c_str(), 0, &t));
        return t;
    }
    std::vector<unsigned char> read(const std::string& name) const {
        std::vector<unsigned char> bytes(static_cast<size_t>(tensor(name).nbytes));
        ck(miqmm_checkpoint_read(h_, name.c_str(), bytes.data(), (int64_t)bytes.size()));
        return bytes;
    }

   private:
    static void ck(int st) {
        if (st != MIQMM_OK) throw Exception(st, std::string("miqmm: ") + miqmm_checkpoint_last_error());
    }
    miqmm_checkpoint* h_ = nullptr;
};

}  // namespace miqmm
