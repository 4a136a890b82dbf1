// test_host_api.cpp -- exercises the C++ host layer (include/miqmm.hpp) on
// the GPU: QuantizedLinear forward (with and without bias), quantized_matmul
// on both routes, dequantize, and the exception path, checked against the C
// oracle (oracle/miqmm_oracle.c) on the same seeded inputs.
//
// Built by __graft_entry__.build() into tests/cpp/bin/test_host_api; run by
// tests/test_gpu_host_api.py.  Prints one line per case and exits nonzero on
// the first failure.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/miqmm.hpp"

extern "C" {
void orc_qmm_f64(const uint16_t* x, int x_dtype, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                 double* y, int64_t M, int64_t N, int64_t K, int group_size, int bits, int sb_dtype,
                 int nthreads);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
}

#define HIP_OK(e)                                                                      \
    do {                                                                               \
        hipError_t err_ = (e);                                                         \
        if (err_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(err_), __FILE__, \
                         __LINE__);                                                    \
            std::exit(3);                                                              \
        }                                                                              \
    } while (0)

template <typename T>
struct Dev {
    T* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { HIP_OK(hipMalloc(&p, count * sizeof(T))); }
    ~Dev() { (void)hipFree(p); }
    std::vector<T> host() const {
        std::vector<T> h(n);
        HIP_OK(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
};

static int failures = 0;

static void expect(bool ok, const char* what) {
    std::printf("%s: %s\n", ok ? "ok" : "FAIL", what);
    if (!ok) ++failures;
}

// max|err| <= 1e-3 + 1e-2 * max|ref| and <= 2 bf16 ulps of max|ref|
static bool within(const std::vector<uint16_t>& y, const std::vector<double>& ref) {
    double mag = 0, err = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
        mag = std::fmax(mag, std::fabs(ref[i]));
        err = std::fmax(err, std::fabs((double)orc_bf16_to_f32(y[i]) - ref[i]));
    }
    const double ulp2 = 2.0 * std::ldexp(1.0, (int)std::floor(std::log2(mag)) - 7);
    std::printf("  max_err %.3g max_ref %.3g\n", err, mag);
    return err <= 1e-3 + 1e-2 * mag && err <= ulp2;
}

int main() {
    const int64_t N = 640, K = 1024;
    const int g = 64, bits = 4;
    for (int64_t M : {1, 5, 40}) {
        Dev<uint16_t> x(M * K), s(N * K / g), b(N * K / g), y(M * N), bias(N), yb(M * N);
        Dev<uint32_t> w(N * K * bits / 32);
        miqmm::check(miqmm_synth_problem(x.p, w.p, s.p, b.p, M, N, K, g, bits, MIQMM_DT_BF16, MIQMM_DT_BF16,
                                         3, (uint64_t)M, nullptr));
        miqmm::check(miqmm_synth_problem(bias.p, nullptr, nullptr, nullptr, 1, N, N, 32, 4, MIQMM_DT_BF16,
                                         MIQMM_DT_BF16, 4, 0, nullptr));
        using miqmm::Array;
        using miqmm::Dtype;
        Array W(w.p, {N, K * bits / 32}, Dtype::uint32), S(s.p, {N, K / g}, Dtype::bfloat16),
            B(b.p, {N, K / g}, Dtype::bfloat16), X(x.p, {M, K}, Dtype::bfloat16), Y(y.p, {M, N}, Dtype::bfloat16),
            BIAS(bias.p, {N}, Dtype::bfloat16), YB(yb.p, {M, N}, Dtype::bfloat16);
        miqmm::QuantizedLinear plain(W, S, B, g, bits);
        miqmm::QuantizedLinear with_bias(W, S, B, g, bits, &BIAS);
        plain.forward(Y, X);
        with_bias.forward(YB, X);
        HIP_OK(hipDeviceSynchronize());

        auto xh = x.host(), sh = s.host(), bh = b.host(), yh = y.host(), ybh = yb.host(), biash = bias.host();
        auto wh = w.host();
        std::vector<double> ref(M * N);
        orc_qmm_f64(xh.data(), 0, wh.data(), sh.data(), bh.data(), ref.data(), M, N, K, g, bits, 0, 0);
        char what[128];
        std::snprintf(what, sizeof what, "QuantizedLinear M=%lld", (long long)M);
        expect(within(yh, ref), what);
        // bias is added after rounding the matmul to bf16, then rounded again
        bool bias_ok = true;
        for (int64_t i = 0; i < M * N; ++i) {
            const uint16_t want = orc_f32_to_bf16(orc_bf16_to_f32(yh[i]) + orc_bf16_to_f32(biash[i % N]));
            bias_ok &= want == ybh[i];
        }
        std::snprintf(what, sizeof what, "QuantizedLinear+bias M=%lld (bf16 round, add, round)", (long long)M);
        expect(bias_ok, what);
    }
    // exception path: unsupported width and mismatched shapes throw with the C status
    try {
        miqmm::Array W(nullptr, {8, 32}, miqmm::Dtype::uint32), S(nullptr, {8, 2}, miqmm::Dtype::bfloat16);
        miqmm::Array X(nullptr, {1, 64}, miqmm::Dtype::bfloat16), Y(nullptr, {1, 8}, miqmm::Dtype::bfloat16);
        miqmm::quantized_matmul(Y, X, W, S, S, true, 32, 3);
        expect(false, "bits=3 throws");
    } catch (const miqmm::Exception& e) {
        expect(e.status() == MIQMM_ENOTSUP, "bits=3 throws ENOTSUP");
    }
    try {
        miqmm::Array W(nullptr, {8, 8}, miqmm::Dtype::uint32), S(nullptr, {8, 1}, miqmm::Dtype::bfloat16);
        miqmm::QuantizedLinear bad(W, S, S, 32, 4);
        expect(false, "shape mismatch throws");
    } catch (const miqmm::Exception& e) {
        expect(e.status() == MIQMM_EINVAL, "QuantizedLinear shape mismatch throws EINVAL");
    }
    std::printf("%s\n", failures ? "FAILED" : "PASSED");
    return failures ? 1 : 0;
}
