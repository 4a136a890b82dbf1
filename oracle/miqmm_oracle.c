/*
 * miqmm_oracle.c -- CPU restatement of MLX affine group-quantized matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (sen-mlx_amd/) never links, loads or calls it.
 *
 * What it restates (citations are into the reference tree, SenClaw/sen-mlx):
 *   - operator surface  y = quantized_matmul(x, w, scales, biases,
 *     transpose=true, group_size, bits): src/engine/mlx_lm/utils/mod.rs:70-78
 *     (argument order), src/engine/mlx_lm/models/bonsai_q1.rs:469-477;
 *     the op itself lives in the un-vendored mlx-rs/mlx-sys v0.25.3
 *     (Cargo.lock:1297-1328) and is restated from its published algorithm.
 *   - packed layout: row n of w holds K*bits/32 uint32 words, code k sits in
 *     word k/(32/bits) at bit offset bits*(k mod 32/bits), LSB first; this is
 *     the bits=1 layout of src/engine/mlx_lm/models/bonsai_q1.rs:137-143,168-170
 *     generalised to bits 4 and 8.
 *   - shapes: w [N, K*bits/32], scales/biases [N, K/group_size]
 *     (src/engine/mlx_lm/utils/moe.rs:20-31).
 *   - dequant: w = fma(scale, q, bias) in fp32
 *     (src/engine/mlx_lm/models/bonsai_q1.rs:172, f32::mul_add).
 *
 * Two accumulators are provided:
 *   orc_qmm_f32  fp32 dequant (fmaf) and fp32 accumulation, 8 interleaved
 *                partial sums combined in a fixed order (deterministic).
 *   orc_qmm_f64  exact dequant in double and double accumulation: the ground
 *                truth the fp32 path and the GPU kernels are both held against.
 *
 * The synthetic-input generator (splitmix64 counter hash + Irwin-Hall(4)
 * approximate normal) uses only integer arithmetic plus single IEEE fp32
 * multiplies/adds, so this file, oracle.py (numpy) and the HIP generator in
 * the product produce bit-identical tensors.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype codes shared with include/miqmm.h */
enum { ORC_BF16 = 0, ORC_F16 = 1, ORC_F32 = 2 };

/* ------------------------------------------------------------------ */
/* scalar conversions (round to nearest even)                          */
/* ------------------------------------------------------------------ */
float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* |f| < 2^-14 */
        if (ax <= 0x33000000u) return (uint16_t)sign;          /* <= 2^-25 -> 0 */
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value in units of 2^-24 is m >> shift */
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

static inline float ld_half(const uint16_t* p, int64_t i, int dtype) {
    return dtype == ORC_F16 ? orc_f16_to_f32(p[i]) : orc_bf16_to_f32(p[i]);
}

static inline uint16_t st_half(float f, int dtype) {
    return dtype == ORC_F16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f);
}

/* ------------------------------------------------------------------ */
/* portable generator                                                  */
/* ------------------------------------------------------------------ */
#define ORC_GAMMA 0x9E3779B97F4A7C15ull

uint64_t orc_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* stream key for (seed, tag); draw i of the stream is mix64(key + i*GAMMA) */
uint64_t orc_key(uint64_t seed, uint64_t tag) { return orc_mix64(seed * ORC_GAMMA + tag); }

uint64_t orc_draw(uint64_t key, uint64_t i) { return orc_mix64(key + i * ORC_GAMMA); }

/* Irwin-Hall(4) over the four 16-bit fields of r, centred and scaled to unit
 * variance: (S - 131070) * (1/37837.2272...) with one fp32 rounding. */
#define ORC_IH_SCALE 2.6428997e-05f
float orc_normal(uint64_t r) {
    int32_t s = (int32_t)(r & 0xffffu) + (int32_t)((r >> 16) & 0xffffu) +
                (int32_t)((r >> 32) & 0xffffu) + (int32_t)((r >> 48) & 0xffffu);
    return (float)(s - 131070) * ORC_IH_SCALE;
}

/* tags of one synthetic problem (x, codes, scales, bias noise) */
uint64_t orc_tag(uint64_t stream, uint64_t kind) { return stream * 8u + kind; }

/* x[i] = round_dtype(normal * sigma) for i < count */
void orc_gen_normal(uint16_t* out, int64_t count, float sigma, int dtype, uint64_t seed, uint64_t tag) {
    uint64_t key = orc_key(seed, tag);
    for (int64_t i = 0; i < count; ++i) {
        float v = orc_normal(orc_draw(key, (uint64_t)i)) * sigma;
        out[i] = st_half(v, dtype);
    }
}

/* codes uniform in [0, 2^bits): the top `bits` bits of draw (n*K + k), packed
 * LSB-first into words (layout of bonsai_q1.rs:137-143 generalised). */
void orc_gen_codes(uint32_t* w, int64_t N, int64_t K, int bits, uint64_t seed, uint64_t tag) {
    uint64_t key = orc_key(seed, tag);
    int per = 32 / bits;
    int64_t words = K / per;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t j = 0; j < words; ++j) {
            uint32_t word = 0;
            for (int t = 0; t < per; ++t) {
                uint64_t idx = (uint64_t)(n * K + j * per + t);
                uint32_t q = (uint32_t)(orc_draw(key, idx) >> (64 - bits));
                word |= q << (bits * t);
            }
            w[n * words + j] = word;
        }
    }
}

/* scales = round(|normal| * 0.02); biases = round(-2^(bits-1) * scale + normal' * 0.002)
 * where `scale` is the stored (rounded) scale. */
void orc_gen_scales_biases(uint16_t* s, uint16_t* b, int64_t count, int bits, int dtype,
                           uint64_t seed, uint64_t tag_s, uint64_t tag_b) {
    uint64_t ks = orc_key(seed, tag_s), kb = orc_key(seed, tag_b);
    float centre = -(float)(1u << (bits - 1));
    for (int64_t i = 0; i < count; ++i) {
        float sv = fabsf(orc_normal(orc_draw(ks, (uint64_t)i))) * 0.02f;
        uint16_t sh = st_half(sv, dtype);
        float sr = ld_half(&sh, 0, dtype);
        float noise = orc_normal(orc_draw(kb, (uint64_t)i)) * 0.002f;
        float bv = centre * sr;
        bv = bv + noise;
        s[i] = sh;
        b[i] = st_half(bv, dtype);
    }
}

/* one problem: x [M,K], w [N,K*bits/32], scales/biases [N,K/g] */
void orc_synth_problem(uint16_t* x, uint32_t* w, uint16_t* s, uint16_t* b, int64_t M, int64_t N,
                       int64_t K, int group_size, int bits, int x_dtype, int sb_dtype,
                       uint64_t seed, uint64_t stream) {
    if (x) orc_gen_normal(x, M * K, 1.0f, x_dtype, seed, orc_tag(stream, 1));
    if (w) orc_gen_codes(w, N, K, bits, seed, orc_tag(stream, 2));
    if (s && b)
        orc_gen_scales_biases(s, b, N * (K / group_size), bits, sb_dtype, seed, orc_tag(stream, 3),
                              orc_tag(stream, 4));
}

/* ------------------------------------------------------------------ */
/* layout + dequant                                                    */
/* ------------------------------------------------------------------ */

/* q[n*K + k] = code k of row n */
void orc_unpack(const uint32_t* w, uint8_t* q, int64_t N, int64_t K, int bits) {
    int per = 32 / bits;
    uint32_t mask = (bits == 32) ? 0xffffffffu : ((1u << bits) - 1u);
    int64_t words = K / per;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = w[n * words + k / per];
            q[n * K + k] = (uint8_t)((word >> (bits * (k % per))) & mask);
        }
}

/* inverse of orc_unpack */
void orc_pack(const uint8_t* q, uint32_t* w, int64_t N, int64_t K, int bits) {
    int per = 32 / bits;
    int64_t words = K / per;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t j = 0; j < words; ++j) {
            uint32_t word = 0;
            for (int t = 0; t < per; ++t) word |= (uint32_t)q[n * K + j * per + t] << (bits * t);
            w[n * words + j] = word;
        }
}

/* row n of dequant(W) in fp32: fma(scale, q, bias) (bonsai_q1.rs:172) */
static void dequant_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out,
                        int64_t n, int64_t K, int g, int bits, int sb_dtype) {
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    int64_t words = K / per, G = K / g;
    const uint32_t* wr = w + n * words;
    for (int64_t k = 0; k < K; ++k) {
        uint32_t q = (wr[k / per] >> (bits * (k % per))) & mask;
        float sc = ld_half(s, n * G + k / g, sb_dtype);
        float bi = ld_half(b, n * G + k / g, sb_dtype);
        out[k] = fmaf(sc, (float)q, bi);
    }
}

void orc_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out, int64_t N,
                    int64_t K, int group_size, int bits, int sb_dtype) {
    for (int64_t n = 0; n < N; ++n) dequant_row(w, s, b, out + n * K, n, K, group_size, bits, sb_dtype);
}

static int clamp_threads(int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    return nthreads < 1 ? 1 : nthreads;
}

/* y[m*N+n] (fp32, unrounded) = sum_k x[m,k] * fma(s,q,b), fp32 accumulation in
 * 8 interleaved partial sums (k mod 8) combined as ((p0+p4)+(p2+p6))+((p1+p5)+(p3+p7)). */
void orc_qmm_f32(const uint16_t* x, int x_dtype, const uint32_t* w, const uint16_t* s,
                 const uint16_t* b, float* y, int64_t M, int64_t N, int64_t K, int group_size,
                 int bits, int sb_dtype, int nthreads) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) xf[i] = ld_half(x, i, x_dtype);
    nthreads = clamp_threads(nthreads);
#pragma omp parallel num_threads(nthreads)
    {
        float* wrow = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            dequant_row(w, s, b, wrow, n, K, group_size, bits, sb_dtype);
            for (int64_t m = 0; m < M; ++m) {
                const float* xr = xf + m * K;
                float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int64_t k = 0; k < K; k += 8)
                    for (int j = 0; j < 8; ++j) p[j] += xr[k + j] * wrow[k + j];
                y[m * N + n] = ((p[0] + p[4]) + (p[2] + p[6])) + ((p[1] + p[5]) + (p[3] + p[7]));
            }
        }
        free(wrow);
    }
    free(xf);
}

/* exact dequant s*q+b in double (exact: 8+8 significant bits) and a double
 * accumulation in k order */
void orc_qmm_f64(const uint16_t* x, int x_dtype, const uint32_t* w, const uint16_t* s,
                 const uint16_t* b, double* y, int64_t M, int64_t N, int64_t K, int group_size,
                 int bits, int sb_dtype, int nthreads) {
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    int64_t words = K / per, G = K / group_size;
    nthreads = clamp_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                uint32_t q = (w[n * words + k / per] >> (bits * (k % per))) & mask;
                double sc = ld_half(s, n * G + k / group_size, sb_dtype);
                double bi = ld_half(b, n * G + k / group_size, sb_dtype);
                acc += (double)ld_half(x, m * K + k, x_dtype) * (sc * (double)q + bi);
            }
            y[m * N + n] = acc;
        }
    }
}

/* out[i] = round_dtype(y[i]); dtype ORC_F32 copies the bits */
void orc_round(const float* y, void* out, int64_t count, int dtype) {
    if (dtype == ORC_F32) {
        memcpy(out, y, sizeof(float) * (size_t)count);
        return;
    }
    uint16_t* o = (uint16_t*)out;
    for (int64_t i = 0; i < count; ++i) o[i] = st_half(y[i], dtype);
}

/* bulk conversions for tests */
void orc_half_to_f32(const uint16_t* h, float* f, int64_t count, int dtype) {
    for (int64_t i = 0; i < count; ++i) f[i] = ld_half(h, i, dtype);
}
