// test_host_api.cpp -- exercises the C++ host layer (include/miqmm.hpp) on
// the GPU: QuantizedLinear forward (with and without bias), gather_qmm /
// SwitchLinear (shared and per-selection x, with and without the grouped
// workspace), QuantizedEmbedding (lookup and tied lm_head), the Checkpoint
// reader feeding those modules, and the exception path, checked against the
// C oracle (oracle/miqmm_oracle.c) on the same seeded inputs.
//
// Built by __graft_entry__.build() into tests/cpp/bin/test_host_api; run by
// tests/test_gpu_host_api.py, which passes a small MLX model directory as
// argv[1] for the checkpoint cases.  Prints one line per case and exits
// nonzero if any failed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/miqmm.hpp"

extern "C" {
void orc_qmm_f64(const uint16_t* x, int x_dtype, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                 double* y, int64_t M, int64_t N, int64_t K, int group_size, int bits, int sb_dtype,
                 int nthreads);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
void orc_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out, int64_t N, int64_t K,
                    int group_size, int bits, int sb_dtype);
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
    explicit Dev(size_t count) : n(count) { HIP_OK(hipMalloc(&p, (count ? count : 1) * sizeof(T))); }
    explicit Dev(const std::vector<T>& h) : Dev(h.size()) {
        HIP_OK(hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice));
    }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
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

using miqmm::Array;
using miqmm::Dtype;

// reference rows of a gather: for selection i (b-major, then j) with expert
// e = idx[i], ref[i] = x[xrow(i)] @ dequant(w[e]).T, zero for e outside [0, E)
static std::vector<double> gather_ref(const std::vector<uint16_t>& xh, const std::vector<uint32_t>& wh,
                                      const std::vector<uint16_t>& sh, const std::vector<uint16_t>& bh,
                                      const std::vector<int32_t>& idx, int64_t top_k, bool per_index, int64_t E,
                                      int64_t N, int64_t K, int g, int bits, int sb_dtype) {
    const int64_t S = (int64_t)idx.size(), wrow = K * bits / 32, srow = K / g;
    std::vector<double> ref(S * N, 0.0), tmp(N);
    for (int64_t i = 0; i < S; ++i) {
        const int32_t e = idx[i];
        if (e < 0 || e >= E) continue;
        const uint16_t* xr = xh.data() + (per_index ? i : i / top_k) * K;
        orc_qmm_f64(xr, 0, wh.data() + e * N * wrow, sh.data() + e * N * srow, bh.data() + e * N * srow,
                    tmp.data(), 1, N, K, g, bits, sb_dtype, 0);
        std::copy(tmp.begin(), tmp.end(), ref.begin() + i * N);
    }
    return ref;
}

static void test_gather() {
    const int64_t E = 4, N = 256, K = 512;
    const int g = 64, bits = 4;
    Dev<uint32_t> w(E * N * K * bits / 32);
    Dev<uint16_t> s(E * N * K / g), b(E * N * K / g);
    miqmm::check(miqmm_synth_problem(nullptr, w.p, s.p, b.p, 1, E * N, K, g, bits, MIQMM_DT_BF16, MIQMM_DT_BF16,
                                     11, 0, nullptr));
    const auto wh = w.host();
    const auto sh = s.host(), bh = b.host();
    miqmm::SwitchLinear sw(Array(w.p, {E, N, K * bits / 32}, Dtype::uint32), Array(s.p, {E, N, K / g}, Dtype::bfloat16),
                           Array(b.p, {E, N, K / g}, Dtype::bfloat16), g, bits);
    expect(sw.experts() == E && sw.out_features() == N && sw.in_features() == K, "SwitchLinear shape accessors");
    struct Case {
        const char* what;
        int64_t batch, top_k;
        bool per_index, workspace;
    };
    const Case cases[] = {{"gather_qmm shared x [3,1,1,K] x idx [3,2] (+ out-of-range id)", 3, 2, false, false},
                          {"gather_qmm per-selection x [3,2,1,K]", 3, 2, true, false},
                          {"SwitchLinear grouped x [96,1,1,K] x idx [96,2] with workspace", 96, 2, false, true},
                          {"SwitchLinear grouped GEMV x [10,2,1,K] x idx [10,2] with workspace", 10, 2, true, true}};
    for (const Case& c : cases) {
        const int64_t S = c.batch * c.top_k, xm = c.per_index ? S : c.batch;
        Dev<uint16_t> x(xm * K), y(S * N);
        miqmm::check(miqmm_synth_problem(x.p, nullptr, nullptr, nullptr, xm, 1, K, g, bits, MIQMM_DT_BF16,
                                         MIQMM_DT_BF16, 12, (uint64_t)S, nullptr));
        std::vector<int32_t> idx(S);
        for (int64_t i = 0; i < S; ++i) idx[i] = (int32_t)((i * 7 + i / 3) % E);
        if (!c.workspace) idx[1] = (int32_t)E + 3;  // out of range: zero rows
        Dev<int32_t> id(idx);
        Array X = c.per_index ? Array(x.p, {c.batch, c.top_k, 1, K}, Dtype::bfloat16)
                              : Array(x.p, {c.batch, 1, 1, K}, Dtype::bfloat16);
        Array I(id.p, {c.batch, c.top_k}, Dtype::int32), Y(y.p, {c.batch, c.top_k, 1, N}, Dtype::bfloat16);
        miqmm::Workspace ws;
        Dev<unsigned char> wsbuf(c.workspace ? miqmm::gather_qmm_workspace_size(c.batch, c.top_k, E) : 0);
        if (c.workspace) ws = {wsbuf.p, (int64_t)wsbuf.n};
        sw.forward(Y, X, I, nullptr, ws);
        HIP_OK(hipDeviceSynchronize());
        const auto ref = gather_ref(x.host(), wh, sh, bh, idx, c.top_k, c.per_index, E, N, K, g, bits, 0);
        const auto yh = y.host();
        bool zero_ok = true;
        if (!c.workspace)
            for (int64_t n = 0; n < N; ++n) zero_ok &= yh[N + n] == 0;
        expect(within(yh, ref) && zero_ok, c.what);
    }
    // a broadcast the host layer does not materialise
    try {
        Array X(nullptr, {1, 2, 1, K}, Dtype::bfloat16), I(nullptr, {3, 2}, Dtype::int32),
            Y(nullptr, {3, 2, 1, N}, Dtype::bfloat16);
        miqmm::gather_qmm(Y, X, Array(w.p, {E, N, K * bits / 32}, Dtype::uint32),
                          Array(s.p, {E, N, K / g}, Dtype::bfloat16), Array(b.p, {E, N, K / g}, Dtype::bfloat16), I,
                          true, g, bits);
        expect(false, "gather_qmm x [1,2,1,K] x idx [3,2] throws");
    } catch (const miqmm::Exception& e) {
        expect(e.status() == MIQMM_EINVAL, "gather_qmm x [1,2,1,K] x idx [3,2] throws EINVAL");
    }
}

static void test_embedding() {
    const int64_t V = 300, K = 512;
    const int g = 32, bits = 8;
    Dev<uint32_t> w(V * K * bits / 32);
    Dev<uint16_t> s(V * K / g), b(V * K / g);
    miqmm::check(miqmm_synth_problem(nullptr, w.p, s.p, b.p, 1, V, K, g, bits, MIQMM_DT_BF16, MIQMM_DT_BF16, 21, 0,
                                     nullptr));
    miqmm::QuantizedEmbedding emb(Array(w.p, {V, K * bits / 32}, Dtype::uint32), Array(s.p, {V, K / g}, Dtype::bfloat16),
                                  Array(b.p, {V, K / g}, Dtype::bfloat16), g, bits);
    const std::vector<int32_t> ids = {5, 299, 0, -1, 17, 300, 42, 5, 123, 7};
    Dev<int32_t> id(ids);
    Dev<uint16_t> out(ids.size() * K);
    Array I(id.p, {2, 5}, Dtype::int32), O(out.p, {2, 5, K}, Dtype::bfloat16);
    emb.forward(O, I);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> table(V * K);
    orc_dequantize(w.host().data(), s.host().data(), b.host().data(), table.data(), V, K, g, bits, 0);
    const auto oh = out.host();
    bool ok = true;
    for (size_t t = 0; t < ids.size(); ++t)
        for (int64_t k = 0; k < K; ++k) {
            const bool in = ids[t] >= 0 && ids[t] < V;
            ok &= oh[t * K + k] == (in ? orc_f32_to_bf16(table[ids[t] * K + k]) : 0);
        }
    expect(ok, "QuantizedEmbedding forward ids [2,5] (+ out-of-range ids) bit-exact vs dequantize");
    // tied lm_head: as_linear is quantized_matmul on the table
    const int64_t M = 3;
    Dev<uint16_t> x(M * K), y1(M * V), y2(M * V);
    miqmm::check(miqmm_synth_problem(x.p, nullptr, nullptr, nullptr, M, 1, K, g, bits, MIQMM_DT_BF16, MIQMM_DT_BF16,
                                     22, 0, nullptr));
    Array X(x.p, {M, K}, Dtype::bfloat16), Y1(y1.p, {M, V}, Dtype::bfloat16), Y2(y2.p, {M, V}, Dtype::bfloat16);
    emb.as_linear(Y1, X);
    miqmm::QuantizedLinear(Array(w.p, {V, K * bits / 32}, Dtype::uint32), Array(s.p, {V, K / g}, Dtype::bfloat16),
                           Array(b.p, {V, K / g}, Dtype::bfloat16), g, bits)
        .forward(Y2, X);
    HIP_OK(hipDeviceSynchronize());
    expect(y1.host() == y2.host(), "QuantizedEmbedding as_linear == QuantizedLinear forward");
}

// Loads every quantized module of an MLX model directory through
// miqmm::Checkpoint and runs it: QuantizedLinear (M = 3), QuantizedEmbedding,
// SwitchLinear (idx [2, 2]), each against the oracle on the file's bytes.
static void test_checkpoint(const char* dir) {
    miqmm::Checkpoint ck(dir);
    const auto mods = ck.modules();
    char what[256];
    std::snprintf(what, sizeof what, "Checkpoint %s: %zu quantized modules", dir, mods.size());
    expect(!mods.empty(), what);
    for (const miqmm_qmodule& m : mods) {
        const auto wb = ck.read(m.weight), sb = ck.read(m.scales), bb = ck.read(m.biases);
        std::vector<uint32_t> wh(wb.size() / 4);
        std::vector<uint16_t> sh(sb.size() / 2), bh(bb.size() / 2);
        std::memcpy(wh.data(), wb.data(), wb.size());
        std::memcpy(sh.data(), sb.data(), sb.size());
        std::memcpy(bh.data(), bb.data(), bb.size());
        Dev<uint32_t> w(wh);
        Dev<uint16_t> s(sh), b(bh);
        const int g = m.group_size, bits = m.bits;
        const int64_t N = m.rows, K = m.cols;
        const Dtype sdt = static_cast<Dtype>(m.sb_dtype);
        const std::string path = m.path;
        if (m.experts) {
            const int64_t E = m.experts;
            miqmm::SwitchLinear sw(Array(w.p, {E, N, K * bits / 32}, Dtype::uint32), Array(s.p, {E, N, K / g}, sdt),
                                   Array(b.p, {E, N, K / g}, sdt), g, bits);
            const std::vector<int32_t> idx = {0, (int32_t)(E - 1), 1 % (int32_t)E, 2 % (int32_t)E};
            Dev<int32_t> id(idx);
            Dev<uint16_t> x(2 * K), y(4 * N);
            miqmm::check(miqmm_synth_problem(x.p, nullptr, nullptr, nullptr, 2, 1, K, g, bits, MIQMM_DT_BF16,
                                             MIQMM_DT_BF16, 31, 0, nullptr));
            Array X(x.p, {2, 1, 1, K}, Dtype::bfloat16), I(id.p, {2, 2}, Dtype::int32),
                Y(y.p, {2, 2, 1, N}, result_type(Dtype::bfloat16, sdt));
            sw.forward(Y, X, I);
            HIP_OK(hipDeviceSynchronize());
            const auto ref = gather_ref(x.host(), wh, sh, bh, idx, 2, false, E, N, K, g, bits, m.sb_dtype);
            std::snprintf(what, sizeof what, "  %s: SwitchLinear E=%lld %lldx%lld %d-bit g%d", path.c_str(),
                          (long long)E, (long long)N, (long long)K, bits, g);
            expect(within(y.host(), ref), what);
        } else if (path.size() >= 12 && path.compare(path.size() - 12, 12, "embed_tokens") == 0) {
            miqmm::QuantizedEmbedding emb(Array(w.p, {N, K * bits / 32}, Dtype::uint32), Array(s.p, {N, K / g}, sdt),
                                          Array(b.p, {N, K / g}, sdt), g, bits);
            const std::vector<int32_t> ids = {0, (int32_t)(N - 1), (int32_t)(N / 2)};
            Dev<int32_t> id(ids);
            Dev<uint16_t> out(3 * K);
            Array I(id.p, {3}, Dtype::int32), O(out.p, {3, K}, Dtype::bfloat16);
            emb.forward(O, I);
            HIP_OK(hipDeviceSynchronize());
            std::vector<float> table(N * K);
            orc_dequantize(wh.data(), sh.data(), bh.data(), table.data(), N, K, g, bits, m.sb_dtype);
            const auto oh = out.host();
            bool ok = true;
            for (int t = 0; t < 3; ++t)
                for (int64_t k = 0; k < K; ++k) ok &= oh[t * K + k] == orc_f32_to_bf16(table[ids[t] * K + k]);
            std::snprintf(what, sizeof what, "  %s: QuantizedEmbedding %lldx%lld %d-bit g%d", path.c_str(),
                          (long long)N, (long long)K, bits, g);
            expect(ok, what);
        } else {
            miqmm::QuantizedLinear lin(Array(w.p, {N, K * bits / 32}, Dtype::uint32), Array(s.p, {N, K / g}, sdt),
                                       Array(b.p, {N, K / g}, sdt), g, bits);
            const int64_t M = 3;
            Dev<uint16_t> x(M * K), y(M * N);
            miqmm::check(miqmm_synth_problem(x.p, nullptr, nullptr, nullptr, M, 1, K, g, bits, MIQMM_DT_BF16,
                                             MIQMM_DT_BF16, 32, 0, nullptr));
            Array X(x.p, {M, K}, Dtype::bfloat16), Y(y.p, {M, N}, result_type(Dtype::bfloat16, sdt));
            lin.forward(Y, X);
            HIP_OK(hipDeviceSynchronize());
            std::vector<double> ref(M * N);
            orc_qmm_f64(x.host().data(), 0, wh.data(), sh.data(), bh.data(), ref.data(), M, N, K, g, bits,
                        m.sb_dtype, 0);
            std::snprintf(what, sizeof what, "  %s: QuantizedLinear %lldx%lld %d-bit g%d", path.c_str(),
                          (long long)N, (long long)K, bits, g);
            expect(within(y.host(), ref), what);
        }
    }
    try {
        miqmm::Checkpoint missing(std::string(dir) + "/no-such-model");
        expect(false, "Checkpoint on a missing directory throws");
    } catch (const miqmm::Exception& e) {
        expect(e.status() == MIQMM_EINVAL, "Checkpoint on a missing directory throws EINVAL");
    }
}

int main(int argc, char** argv) {
    const int64_t N = 640, K = 1024;
    const int g = 64, bits = 4;
    for (int64_t M : {1, 5, 40}) {
        Dev<uint16_t> x(M * K), s(N * K / g), b(N * K / g), y(M * N), bias(N), yb(M * N);
        Dev<uint32_t> w(N * K * bits / 32);
        miqmm::check(miqmm_synth_problem(x.p, w.p, s.p, b.p, M, N, K, g, bits, MIQMM_DT_BF16, MIQMM_DT_BF16,
                                         3, (uint64_t)M, nullptr));
        miqmm::check(miqmm_synth_problem(bias.p, nullptr, nullptr, nullptr, 1, N, N, 32, 4, MIQMM_DT_BF16,
                                         MIQMM_DT_BF16, 4, 0, nullptr));
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
    test_gather();
    test_embedding();
    if (argc > 1) test_checkpoint(argv[1]);
    std::printf("%s\n", failures ? "FAILED" : "PASSED");
    return failures ? 1 : 0;
}
