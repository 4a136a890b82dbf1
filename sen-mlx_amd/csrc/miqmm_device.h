// miqmm_device.h -- gfx950 device helpers shared by the miqmm kernels.
//
// Packed affine layout (MLX, LSB-first; reference src/engine/mlx_lm/models/
// bonsai_q1.rs:137-143 for bits=1, generalised): row n of W holds K*bits/32
// uint32 words and code k sits in word k/(32/bits) at bit bits*(k mod 32/bits).
// Dequant is w = scale*q + bias per group of `group_size` consecutive k
// (bonsai_q1.rs:172).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace miqmm {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

enum : int { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };

// Materialises an fp32 value in a register.  Without it the backend may fuse
// the multiply or add that produced it with a following fp16 conversion into
// one v_fma_mixlo_f16, which rounds once where fp32-then-fp16 rounds twice.
__device__ __forceinline__ float f32_pinned(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
__device__ __forceinline__ float half_to_f32(uint16_t h) {
    if constexpr (DT == DT_F16) return f16_bits_to_f32(h);
    else return bf16_bits_to_f32(h);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);  // v_cvt_pk_bf16_f32, RNE
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}

// one output element rounded to y's 16-bit dtype (fp16 or bf16); `bias`
// (nullable, dtype of y) is added after the matmul result is rounded, as
// QuantizedLinear does (quantized_matmul, then + bias as a separate op).
__device__ __forceinline__ uint16_t out_half_bits(int y_dtype, float v, const void* bias, int64_t bidx) {
    if (y_dtype == DT_F16) {
        uint16_t h = f32_to_f16_bits(f32_pinned(v));
        if (bias)
            h = f32_to_f16_bits(f32_pinned(f16_bits_to_f32(h) + f16_bits_to_f32(((const uint16_t*)bias)[bidx])));
        return h;
    }
    uint16_t h = f32_to_bf16_bits(v);
    if (bias) h = f32_to_bf16_bits(bf16_bits_to_f32(h) + bf16_bits_to_f32(((const uint16_t*)bias)[bidx]));
    return h;
}

// store one output element in the requested dtype (bias as above)
__device__ __forceinline__ void store_out(void* y, int64_t idx, int y_dtype, float v,
                                          const void* bias, int64_t bidx) {
    if (y_dtype == DT_F32) {
        if (bias) v += ((const float*)bias)[bidx];
        ((float*)y)[idx] = v;
    } else {
        ((uint16_t*)y)[idx] = out_half_bits(y_dtype, v, bias, bidx);
    }
}

// R consecutive outputs y[base + n0 .. base + n0 + R) of one output row (each
// as store_out would write it), stored by the calling lane as one vector store
// when all R lie below N and the address allows it, else one by one.  A GEMV
// tile's rows are adjacent in y, so this replaces R partial-line stores from R
// lanes with one.
template <int R>
__device__ __forceinline__ void store_run(void* y, int64_t base, int n0, int N, int y_dtype, const float (&v)[R],
                                          const void* bias) {
    using u32x2_t = uint32_t __attribute__((ext_vector_type(2)));
    if (y_dtype == DT_F32) {
        float* p = (float*)y + base + n0;
        if (R >= 2 && n0 + R <= N && (reinterpret_cast<uintptr_t>(p) & (4 * R - 1)) == 0) {
            uint32_t o[R];
#pragma unroll
            for (int r = 0; r < R; ++r) o[r] = __float_as_uint(bias ? v[r] + ((const float*)bias)[n0 + r] : v[r]);
            if constexpr (R == 4) *reinterpret_cast<u32x4_t*>(p) = u32x4_t{o[0], o[1], o[2], o[3]};
            else if constexpr (R == 2) *reinterpret_cast<u32x2_t*>(p) = u32x2_t{o[0], o[1]};
            return;
        }
    } else {
        uint16_t* p = (uint16_t*)y + base + n0;
        if (R >= 2 && n0 + R <= N && (reinterpret_cast<uintptr_t>(p) & (2 * R - 1)) == 0) {
            uint32_t h[R];
#pragma unroll
            for (int r = 0; r < R; ++r) h[r] = out_half_bits(y_dtype, v[r], bias, n0 + r);
            if constexpr (R == 4) *reinterpret_cast<u32x2_t*>(p) = u32x2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            else if constexpr (R == 2) *reinterpret_cast<uint32_t*>(p) = h[0] | (h[1] << 16);
            return;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (n0 + r < N) store_out(y, base + n0 + r, y_dtype, v[r], bias, n0 + r);
}

// ---------------------------------------------------------------- bit tricks
// bf16 with bits 0x4300|q is exactly 128+q for q < 128: a 4-bit code becomes
// an exact bf16 operand with one and-or.  Pairs are (q_j, q_{j+4}) of a word.
constexpr uint32_t kMagic128x2 = 0x43004300u;
constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;  // (1.0, 1.0)

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t u) { return __builtin_bit_cast(bf16x2_t, u); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a), as_bf16x2(b), c, false);
}

// (a & mask) | magic.  With `mask` held in a VGPR (see vgpr_const) and `magic`
// a constant this selects one v_and_or_b32; with both as constants gfx950's
// single constant-bus operand forces an and plus an or.  Written in C, not
// inline asm, so the hazard recognizer sees the result register when an MFMA
// consumes it (an MFMA reading a VALU result needs wait states the compiler
// only inserts for instructions it can see).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
    return (a & mask) | magic;
}

// a constant materialised in a VGPR once, opaque to constant folding
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    uint32_t v;
    asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "i"(c));
    return v;
}

// word of eight 4-bit codes -> four bf16 pairs (q_j+128, q_{j+4}+128), j=0..3;
// mask and magic are passed in registers (0x000F000F, 0x43004300)
__device__ __forceinline__ void unpack4_magic(uint32_t w, uint32_t p[4], uint32_t mask, uint32_t magic) {
    p[0] = and_or(w, mask, magic);
    p[1] = and_or(w >> 4, mask, magic);
    p[2] = and_or(w >> 8, mask, magic);
    p[3] = and_or(w >> 12, mask, magic);
}

// ---------------------------------------------------------------- buffer loads
// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes
// return zero, which the kernels use to mask ragged rows and chunks.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset past any resource this library builds

// s_waitcnt immediate: vmcnt(n), expcnt and lgkmcnt left unconstrained
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// LDS destination of a direct-to-LDS buffer load
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ u32x4_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// cache policy of loads that stream data read once (gfx950 "nt")
constexpr int kNonTemporal = 2;
__device__ __forceinline__ u32x4_t bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNonTemporal));
}
__device__ __forceinline__ uint16_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// ---------------------------------------------------------------- reductions
// Sum over groups of L consecutive lanes (L = 16, 32 or 64) with DPP moves.
// Afterwards lanes li >= L-16 of each group (li = lane % L) hold the group sum.
template <int L>
__device__ __forceinline__ float lane_group_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    if constexpr (L >= 32)  // row_bcast15 into rows 1 and 3
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    if constexpr (L >= 64)  // row_bcast31 into rows 2 and 3
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    return v;
}

// x words (x0|x1, x2|x3, x4|x5, x6|x7) -> pairs (x_j, x_{j+4}) matching unpack4_magic
__device__ __forceinline__ void perm_x_for4(const uint32_t xw[4], uint32_t X[4]) {
    X[0] = __builtin_amdgcn_perm(xw[2], xw[0], 0x05040100u);
    X[1] = __builtin_amdgcn_perm(xw[2], xw[0], 0x07060302u);
    X[2] = __builtin_amdgcn_perm(xw[3], xw[1], 0x05040100u);
    X[3] = __builtin_amdgcn_perm(xw[3], xw[1], 0x07060302u);
}

// float value of byte I of w (selected as one v_cvt_f32_ubyteI)
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t w) { return (float)((w >> (8 * I)) & 0xffu); }

// word of four 8-bit codes -> two exact bf16 pairs (q0,q1), (q2,q3): the fp32
// value of an integer <= 255 has zero low 16 bits, so its top half is exact.
__device__ __forceinline__ void unpack8_pairs(uint32_t w, uint32_t p[2]) {
    uint32_t f0 = __float_as_uint(ubyte_f32<0>(w));
    uint32_t f1 = __float_as_uint(ubyte_f32<1>(w));
    uint32_t f2 = __float_as_uint(ubyte_f32<2>(w));
    uint32_t f3 = __float_as_uint(ubyte_f32<3>(w));
    p[0] = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    p[1] = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
}

__device__ __forceinline__ u32x4_t ldg16(const void* p) {
    return *reinterpret_cast<const u32x4_t*>(p);
}

}  // namespace miqmm
