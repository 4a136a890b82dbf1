// miqmm.hpp -- C++ host layer over the C ABI (miqmm.h), mirroring the
// operator surface the reference engine programs against (mlx-rs, Rust):
//
//   ops::quantized_matmul(x, w, scales, biases, transpose, group_size, bits)
//       -> Result<Array, Exception>          src/engine/mlx_lm/utils/mod.rs:70-78
//   nn::QuantizedLinear / MaybeQuantized<Linear>::forward(&Array)
//       -> Result<Array, Exception>          src/engine/mlx_lm/models/llama.rs:115-126,195-197
//   ops::dequantize(w, scales, biases, group_size, bits)
//                                            src/engine/mlx_lm/utils/moe.rs:118-126
//
// Arrays here are non-owning views of device memory (pointer, shape, dtype);
// the caller allocates outputs, as the engine's allocator would.  Failures throw
// miqmm::Exception carrying the C status, the counterpart of mlx-rs's
// Exception built from a nonzero mlx-c status (moe.rs:66-76).
#pragma once

#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <vector>

#include "miqmm.h"

namespace miqmm {

enum class Dtype : int { bfloat16 = MIQMM_DT_BF16, float16 = MIQMM_DT_F16, float32 = MIQMM_DT_F32, uint32 = 16 };

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
    if (bits != 4 && bits != 8)  // same statuses as the C ABI, before any shape math
        throw Exception(bits == 2 || bits == 3 || bits == 5 || bits == 6 ? MIQMM_ENOTSUP : MIQMM_EINVAL,
                        "miqmm: bits must be 4 or 8");
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
    if (bits != 4 && bits != 8)
        throw Exception(bits == 2 || bits == 3 || bits == 5 || bits == 6 ? MIQMM_ENOTSUP : MIQMM_EINVAL,
                        "miqmm: bits must be 4 or 8");
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

}  // namespace miqmm
