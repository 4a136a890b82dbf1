"""CPU tests of the oracle (oracle/miqmm_oracle.c + oracle/oracle.py).

The reference holds no golden vectors for quantized matmul (its one test of
the op family, src/engine/mlx_lm/utils/moe.rs:84-146, checks the Metal kernel
against dequantize+matmul on the device), so the oracle is pinned by:
  - published test vectors (SplitMix64) and hand-computed known answers for
    the packed layout (src/engine/mlx_lm/models/bonsai_q1.rs:137-143,168-172)
    and the dequant formula (bonsai_q1.rs:172);
  - closed forms and invariants (one-hot x, zero codes, zero scales,
    linearity, group permutation, row independence);
  - two independent restatements (C and numpy) and two accumulations (fp32
    and exact float64) agreeing;
  - mutated oracles (a wrong nibble order, a dropped bias, a transposed
    operand, a wrong group index) that these checks must reject.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


# ------------------------------------------------------------------ generator
def test_splitmix64_published_vector(c_oracle):
    # SplitMix64 seeded with 1234567 (Vigna's splitmix64.c): state += gamma, then mix
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    L = c_oracle.c_oracle()
    assert [L.orc_draw(1234567, i) for i in range(1, 6)] == want
    got = O.draws(np.uint64(1234567), 5, start=1)
    assert [int(v) for v in got] == want


def test_generator_c_numpy_bit_exact(c_oracle):
    for (M, N, K, g, bits, xd, sbd, seed, stream) in [
        (2, 48, 128, 64, 4, O.BF16, O.BF16, 0, 3), (3, 40, 256, 32, 8, O.BF16, O.F16, 1, 7),
        (1, 17, 384, 128, 4, O.F16, O.BF16, 9, 0), (5, 33, 64, 32, 4, O.BF16, O.F16, 2**40, 11)]:
        a = O.synth_problem(M, N, K, g, bits, xd, sbd, seed, stream)
        c = c_oracle.c_synth_problem(M, N, K, g, bits, xd, sbd, seed, stream)
        for u, v in zip(a, c):
            assert u.dtype == v.dtype and u.shape == v.shape
            assert np.array_equal(u, v)


def test_generator_distribution(c_oracle):
    v = O.half_to_f32(O.gen_normal(1 << 20, 1.0, O.BF16, 0, 1), O.BF16).astype(np.float64)
    assert abs(v.mean()) < 5e-3 and abs(v.std() - 1.0) < 5e-3
    assert np.abs(v).max() <= 3.47  # Irwin-Hall(4) support is +-sqrt(12)
    q = O.gen_codes(256, 4096, 4, 0, 2)
    counts = np.bincount(q.ravel(), minlength=16)
    assert counts.min() > 0.97 * q.size / 16 and counts.max() < 1.03 * q.size / 16
    s, b = O.gen_scales_biases(1 << 16, 4, O.BF16, 0, 3, 4)
    sf, bf = O.bf16_to_f32(s), O.bf16_to_f32(b)
    assert (sf >= 0).all() and abs(sf.mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4
    assert np.abs(bf + 8 * sf).max() < 0.002 * 3.47 + 1e-3


def test_golden_generator_and_config0(c_oracle):
    g = np.load(GOLDEN)
    k = c_oracle.c_oracle().orc_key(0, 9)
    assert np.array_equal(O.draws(np.uint64(k), 16), g["draws_seed0_tag9"])
    assert np.array_equal(O.normal(g["draws_seed0_tag9"]), g["normal_seed0_tag9"])
    x, w, s, b = O.synth_problem(1, 4864, 896, 64, 4, seed=0, stream=0)
    assert np.array_equal(w[:2, :4], g["cfg0_words_head"])
    assert np.array_equal(s[:2, :4], g["cfg0_scales_head"])
    assert np.array_equal(b[:2, :4], g["cfg0_biases_head"])
    assert np.array_equal(x[0, :16], g["cfg0_x_head"])
    y = O.qmm_f64(x, w, s, b, 896, 64, 4)
    np.testing.assert_allclose(y, g["cfg0_y64"], rtol=0, atol=1e-9)


def test_golden_small_cases(c_oracle):
    import golden.make_golden as mg  # tests/golden/make_golden.py

    g = np.load(GOLDEN)
    for i, (bits, gs, sbd) in enumerate(mg.SMALL):
        x, w, s, b = O.synth_problem(3, 40, 256, gs, bits, sb_dtype=sbd, seed=5, stream=i)
        y = O.qmm_f64(x, w, s, b, 256, gs, bits, sb_dtype=sbd)
        np.testing.assert_allclose(y, g[f"small{i}_y64"], rtol=0, atol=1e-9)


# ------------------------------------------------------------------ conversions
def test_half_conversions_match_ieee(c_oracle):
    L = c_oracle.c_oracle()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 2000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24, 3.0 * 2 ** -26,
                  np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)])
    for v in vals:
        assert L.orc_f32_to_f16(float(v)) == int(np.float32(v).astype(np.float16).view(np.uint16)), v
    # bf16 RNE: halfway cases round to even
    assert L.orc_f32_to_bf16(1.0 + 2 ** -8) == 0x3F80      # tie -> even (down)
    assert L.orc_f32_to_bf16(1.0 + 3 * 2 ** -8) == 0x3F82  # tie -> even (up)
    assert L.orc_f32_to_bf16(1.0 + 2 ** -8 + 2 ** -20) == 0x3F81
    assert np.array_equal(O.f32_to_bf16(np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)),
                          np.array([0x3F80, 0x3F82], np.uint16))


# ------------------------------------------------------------------ known answers
def test_unpack_known_words(c_oracle):
    # LSB-first: code k of a word sits at bits [bits*k, bits*(k+1))
    w4 = np.array([[0x76543210, 0x89ABCDEF]], np.uint32)
    want4 = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 15, 14, 13, 12, 11, 10, 9, 8]], np.uint8)
    w8 = np.array([[0x04030201, 0xFF80007F]], np.uint32)
    want8 = np.array([[1, 2, 3, 4, 0x7F, 0, 0x80, 0xFF]], np.uint8)
    assert np.array_equal(O.unpack(w4, 16, 4), want4)
    assert np.array_equal(O.unpack(w8, 8, 8), want8)
    assert np.array_equal(c_oracle.c_unpack(w4, 1, 16, 4), want4)
    assert np.array_equal(c_oracle.c_unpack(w8, 1, 8, 8), want8)
    for want, bits in ((want4, 4), (want8, 8)):
        assert np.array_equal(O.pack(want, bits), w4 if bits == 4 else w8)


def test_pack_unpack_roundtrip_extremes(c_oracle):
    for bits in (4, 8):
        top = (1 << bits) - 1
        rng = np.random.default_rng(bits)
        for q in (np.zeros((3, 64), np.uint8), np.full((3, 64), top, np.uint8),
                  np.tile(np.array([0, top], np.uint8), (3, 32)),
                  rng.integers(0, top + 1, (5, 128)).astype(np.uint8)):
            w = O.pack(q, bits)
            assert np.array_equal(O.unpack(w, q.shape[1], bits), q)
            assert np.array_equal(c_oracle.c_unpack(w, q.shape[0], q.shape[1], bits), q)
    # alternating nibbles 0x0F0F... / 0xF0F0...
    assert np.array_equal(O.unpack(np.array([[0x0F0F0F0F]], np.uint32), 8, 4), [[15, 0] * 4])
    assert np.array_equal(O.unpack(np.array([[0xF0F0F0F0]], np.uint32), 8, 4), [[0, 15] * 4])


def _bf(v):
    return O.f32_to_bf16(np.asarray(v, np.float32))


def test_dequant_known_answer(c_oracle):
    # one row, K=32 (one group of 32): codes 0..7,0..7,..., scale 0.5, bias -1
    w = np.array([[0x76543210] * 4], np.uint32)
    s, b = _bf([[0.5]]), _bf([[-1.0]])
    want = np.tile(np.array([-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5], np.float32), 4)[None]
    assert np.array_equal(O.dequantize(w, s, b, 32, 32, 4), want)
    assert np.array_equal(c_oracle.c_dequantize(w, s, b, 1, 32, 32, 4), want)
    # 8-bit, two groups of 32 with different affine maps: q=200 -> 0.25*200-25 = 25
    q = np.full((1, 64), 200, np.uint8)
    w8 = O.pack(q, 8)
    s8, b8 = _bf([[0.25, 2.0]]), _bf([[-25.0, 3.0]])
    want8 = np.concatenate([np.full(32, 25.0), np.full(32, 403.0)]).astype(np.float32)[None]
    assert np.array_equal(c_oracle.c_dequantize(w8, s8, b8, 1, 64, 32, 8), want8)
    # fp16 scales: s=0 gives w=b
    s16 = O.f32_to_f16(np.zeros((1, 1), np.float32))
    b16 = O.f32_to_f16(np.full((1, 1), 0.125, np.float32))
    assert np.array_equal(c_oracle.c_dequantize(w, s16, b16, 1, 32, 32, 4, O.F16), np.full((1, 32), 0.125, np.float32))


def test_qmm_known_answer(c_oracle):
    # x = 1..32, codes alternating 0,15 (word 0xF0F0F0F0), s = 0.25, b = 0.5:
    # w = 0.5, 4.25, 0.5, 4.25, ...; y = 0.5*sum(odd-position x) + 4.25*sum(even-position x)
    # positions k=0,2,.. hold x=1,3,..,31 (sum 256); k=1,3,.. hold x=2,4,..,32 (sum 272)
    x = _bf(np.arange(1, 33, dtype=np.float32)[None])
    w = np.array([[0xF0F0F0F0] * 4], np.uint32)
    s, b = _bf([[0.25]]), _bf([[0.5]])
    want = 0.5 * 256 + 4.25 * 272
    assert O.qmm_f64(x, w, s, b, 32, 32, 4)[0, 0] == want
    assert c_oracle.c_qmm_f64(x, w, s, b, 1, 1, 32, 32, 4)[0, 0] == want
    assert c_oracle.c_qmm_f32(x, w, s, b, 1, 1, 32, 32, 4)[0, 0] == np.float32(want)


# ------------------------------------------------------------------ invariants
@pytest.mark.parametrize("bits,g", [(4, 32), (4, 64), (4, 128), (8, 64)])
def test_invariants(c_oracle, bits, g):
    M, N, K = 4, 24, 256
    x, w, s, b = O.synth_problem(M, N, K, g, bits, seed=3, stream=bits * 1000 + g)
    wd = O.dequantize(w, s, b, K, g, bits, exact=True)
    # one-hot x picks column k of dequant(W) (and rows n are the output columns)
    for k in (0, 1, 7, g - 1, g, K - 1):
        xo = np.zeros((1, K), np.float32)
        xo[0, k] = 1.0
        y = c_oracle.c_qmm_f64(_bf(xo), w, s, b, 1, N, K, g, bits)
        assert np.array_equal(y[0], wd[:, k])
    # zero codes: y = sum_g b_g * sum_{k in g} x_k
    wz = np.zeros_like(w)
    yz = c_oracle.c_qmm_f64(x, wz, s, b, M, N, K, g, bits)
    xs = O.bf16_to_f32(x).astype(np.float64).reshape(M, K // g, g).sum(-1)
    np.testing.assert_allclose(yz, xs @ O.bf16_to_f32(b).astype(np.float64).T, rtol=1e-12, atol=1e-12)
    # zero scales: w = b regardless of codes
    s0 = np.zeros_like(s)
    np.testing.assert_allclose(c_oracle.c_qmm_f64(x, w, s0, b, M, N, K, g, bits), yz, rtol=1e-12, atol=1e-12)
    # linearity in x (exact in float64 for the bf16 sums used here)
    y = c_oracle.c_qmm_f64(x, w, s, b, M, N, K, g, bits)
    x2 = _bf(O.bf16_to_f32(x) * 2.0)
    np.testing.assert_allclose(c_oracle.c_qmm_f64(x2, w, s, b, M, N, K, g, bits), 2 * y, rtol=1e-12, atol=1e-9)
    # row independence: each output row depends only on its own x row
    for m in range(M):
        ym = c_oracle.c_qmm_f64(np.ascontiguousarray(x[m:m + 1]), w, s, b, 1, N, K, g, bits)
        np.testing.assert_allclose(ym[0], y[m], rtol=1e-12, atol=1e-12)
    # permuting whole groups consistently in x, codes and scales leaves y unchanged
    G = K // g
    perm = np.random.default_rng(g).permutation(G)
    q = O.unpack(w, K, bits).reshape(N, G, g)[:, perm].reshape(N, K)
    xp = np.ascontiguousarray(x.reshape(M, G, g)[:, perm].reshape(M, K))
    yp = c_oracle.c_qmm_f64(xp, O.pack(q, bits), np.ascontiguousarray(s[:, perm]),
                            np.ascontiguousarray(b[:, perm]), M, N, K, g, bits)
    np.testing.assert_allclose(yp, y, rtol=1e-10, atol=1e-9)


def test_c_numpy_and_fp32_fp64_agree(c_oracle):
    for (M, N, K, g, bits, sbd) in [(3, 40, 256, 64, 4, O.BF16), (2, 33, 512, 32, 8, O.F16),
                                    (16, 64, 4096, 128, 4, O.BF16)]:
        x, w, s, b = O.synth_problem(M, N, K, g, bits, sb_dtype=sbd, seed=11, stream=K)
        y64 = O.qmm_f64(x, w, s, b, K, g, bits, sb_dtype=sbd)
        yc64 = c_oracle.c_qmm_f64(x, w, s, b, M, N, K, g, bits, sb_dtype=sbd)
        np.testing.assert_allclose(yc64, y64, rtol=1e-12, atol=1e-9)
        y32 = c_oracle.c_qmm_f32(x, w, s, b, M, N, K, g, bits, sb_dtype=sbd)
        rep = O.parity_report(y32, y64)
        assert rep["max_err"] <= 1e-5 * max(1.0, rep["max_ref"]) * np.sqrt(K), rep
        # the fp32 dequant equals the exact value rounded once (fma semantics)
        np.testing.assert_array_equal(c_oracle.c_dequantize(w, s, b, N, K, g, bits, sbd),
                                      O.dequantize(w, s, b, K, g, bits, sbd).astype(np.float32))


def test_round_matches_numpy(c_oracle):
    y = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100
    assert np.array_equal(c_oracle.c_round(y, O.BF16), O.f32_to_bf16(y))
    assert np.array_equal(c_oracle.c_round(y, O.F16), O.f32_to_f16(y))


# ------------------------------------------------------------------ mutated oracles must fail the pins
def _unpack_msb_first(w, K, bits):
    per = 32 // bits
    shifts = (np.arange(per)[::-1] * bits).astype(np.uint32)
    q = (w.astype(np.uint32)[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(w.shape[0], K).astype(np.uint8)


def test_pins_reject_planted_mistakes(c_oracle):
    # wrong nibble order fails the known-word check
    w4 = np.array([[0x76543210, 0x89ABCDEF]], np.uint32)
    assert not np.array_equal(_unpack_msb_first(w4, 16, 4), O.unpack(w4, 16, 4))
    K, g, bits, M, N = 128, 32, 4, 2, 8
    x, w, s, b = O.synth_problem(M, N, K, g, bits, seed=4, stream=1)
    xf = O.bf16_to_f32(x).astype(np.float64)
    sf = np.repeat(O.bf16_to_f32(s), g, 1).astype(np.float64)
    bf = np.repeat(O.bf16_to_f32(b), g, 1).astype(np.float64)
    q = O.unpack(w, K, bits).astype(np.float64)
    good = xf @ (sf * q + bf).T
    np.testing.assert_allclose(c_oracle.c_qmm_f64(x, w, s, b, M, N, K, g, bits), good, rtol=1e-12, atol=1e-12)
    # dropped bias: fails the zero-code closed form
    wz = np.zeros_like(w)
    no_bias = xf @ (sf * 0.0).T
    assert not np.allclose(no_bias, c_oracle.c_qmm_f64(x, wz, s, b, M, N, K, g, bits), atol=1e-3)
    # transposed operand (x @ W instead of x @ W.T) has the wrong shape/values
    assert (xf @ (sf * q + bf).T).shape == (M, N)
    # wrong group index (k // (g/2)) changes the result of the one-hot probe
    sf_bad = O.bf16_to_f32(s)[:, np.minimum(np.arange(K) // (g // 2), K // g - 1)].astype(np.float64)
    assert not np.allclose(xf @ (sf_bad * q + bf).T, good, atol=1e-3)
    # a wrong sign on the bias fails too
    assert not np.allclose(xf @ (sf * q - bf).T, good, atol=1e-3)


# ------------------------------------------------------------------ gather_qmm
def _experts(E, N, K, g, bits, seed):
    ws, ss, bs = [], [], []
    for e in range(E):
        _, w, s, b = O.synth_problem(1, N, K, g, bits, seed=seed, stream=100 + e)
        ws.append(w), ss.append(s), bs.append(b)
    return np.stack(ws), np.stack(ss), np.stack(bs)


def _brute_gather(x, w, s, b, idx, K, g, bits):
    # independent restatement: scalar loops, codes read bit by bit from the words
    E, N = w.shape[0], w.shape[1]
    xf = O.bf16_to_f32(x).astype(np.float64)
    sf = O.bf16_to_f32(s).astype(np.float64)
    bf = O.bf16_to_f32(b).astype(np.float64)
    per = 32 // bits
    out = np.zeros(idx.shape + (x.shape[-2], N))
    for pos in np.ndindex(*idx.shape):
        e = int(idx[pos])
        xm = xf[pos[0]] if xf.ndim == 3 else xf[pos]
        if not 0 <= e < E:
            continue
        for m in range(xm.shape[0]):
            for n in range(N):
                acc = 0.0
                for k in range(K):
                    word = int(w[e, n, k // per])
                    q = (word >> (bits * (k % per))) & ((1 << bits) - 1)
                    acc += xm[m, k] * (sf[e, n, k // g] * q + bf[e, n, k // g])
                out[pos + (m, n)] = acc
    return out


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_brute_force(bits):
    E, N, K, g, M = 3, 5, 64, 32, 2
    w, s, b = _experts(E, N, K, g, bits, seed=11)
    x, _, _, _ = O.synth_problem(2 * M, N, K, g, bits, seed=12)
    x = x.reshape(2, M, K)
    idx = np.array([[2, 0, 1], [1, 1, -1]], np.int64)  # [batch 2, top_k 3]; -1 is out of range
    got = O.gather_qmm_f64(x[:, None], w, s, b, idx, K, g, bits)
    assert got.shape == (2, 3, M, N)
    want = _brute_gather(x, w, s, b, idx, K, g, bits)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert not got[1, 2].any()


def test_gather_reference_test_shape():
    # the reference's test geometry (moe.rs:84-146): E=4, out=32, in=64, g=64,
    # bits=4, x [3, 1, 1, 64] against inds [3, 2] = [0,1,2,3,1,0] -> [3, 2, 1, 32],
    # each slice equal to dequantize(w[e]) @ x[m]
    E, N, K, g, bits = 4, 32, 64, 64, 4
    w, s, b = _experts(E, N, K, g, bits, seed=5)
    x, _, _, _ = O.synth_problem(3, N, K, g, bits, seed=6)
    inds = np.array([0, 1, 2, 3, 1, 0]).reshape(3, 2)
    got = O.gather_qmm_f64(x.reshape(3, 1, 1, K), w, s, b, inds, K, g, bits)
    assert got.shape == (3, 2, 1, N)
    xf = O.bf16_to_f32(x).astype(np.float64)
    for mi in range(3):
        for ki in range(2):
            e = inds[mi, ki]
            wd = O.dequantize(w[e], s[e], b[e], K, g, bits, exact=True)
            np.testing.assert_allclose(got[mi, ki, 0], wd @ xf[mi], rtol=1e-12, atol=1e-12)


def test_gather_constant_index_is_quantized_matmul():
    E, N, K, g, bits, M = 4, 16, 128, 64, 4, 3
    w, s, b = _experts(E, N, K, g, bits, seed=7)
    x, _, _, _ = O.synth_problem(M, N, K, g, bits, seed=8)
    for e in range(E):
        got = O.gather_qmm_f64(x, w, s, b, np.full((5,), e), K, g, bits)
        want = O.qmm_f64(x, w[e], s[e], b[e], K, g, bits)
        for i in range(5):
            np.testing.assert_array_equal(got[i], want)


def test_gather_pins_reject_planted_mistakes():
    # an index read transposed ([top_k, batch] order) or an x taken per
    # selection instead of per token changes the brute-force result
    E, N, K, g, bits, M = 3, 4, 32, 32, 4, 1
    w, s, b = _experts(E, N, K, g, bits, seed=9)
    x, _, _, _ = O.synth_problem(2 * M, N, K, g, bits, seed=10)
    x = x.reshape(2, M, K)
    idx = np.array([[0, 1, 2], [2, 2, 0]])
    want = _brute_gather(x, w, s, b, idx, K, g, bits)
    bad_t = O.gather_qmm_f64(x[:, None], w, s, b, idx.T.reshape(2, 3), K, g, bits)
    assert not np.allclose(bad_t, want, atol=1e-3)
    bad_x = O.gather_qmm_f64(x[::-1].copy()[:, None], w, s, b, idx, K, g, bits)
    assert not np.allclose(bad_x, want, atol=1e-3)
    np.testing.assert_allclose(O.gather_qmm_f64(x[:, None], w, s, b, idx, K, g, bits), want, rtol=1e-12)


# ------------------------------------------------------------------ embedding lookup
def test_embedding_known_answer():
    # one row of 64 4-bit codes 0..15 repeated, group 32: scales (0.5, 2), biases (-1, 3)
    K, g, bits = 64, 32, 4
    q = (np.arange(K) % 16).astype(np.uint8).reshape(1, K)
    w = O.pack(q, bits)
    s = O.f32_to_bf16(np.array([[0.5, 2.0]], np.float32))
    b = O.f32_to_bf16(np.array([[-1.0, 3.0]], np.float32))
    got = O.embedding(np.array([0]), w, s, b, K, g, bits, out_dtype=O.F32)
    want = np.concatenate([0.5 * (np.arange(32) % 16) - 1.0, 2.0 * (np.arange(32, 64) % 16) + 3.0])
    np.testing.assert_array_equal(got[0], want.astype(np.float32))


def test_embedding_rows_dot_x_equal_quantized_matmul():
    # the looked-up rows are the rows of dequant(W): dotting them with x gives
    # quantized_matmul(x, W[ids]) (fp32 dequant vs exact: within 2^-20 relative)
    V, K, g, bits = 50, 256, 64, 4
    x, w, s, b = O.synth_problem(1, V, K, g, bits, seed=21)
    ids = np.array([3, 49, 0, 3, 17])
    rows = O.embedding(ids, w, s, b, K, g, bits, out_dtype=O.F32).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)[0]
    want = O.qmm_f64(x, w[ids], s[ids], b[ids], K, g, bits)[0]
    np.testing.assert_allclose(rows @ xf, want, rtol=1e-5, atol=1e-6)
    # a planted off-by-one row fails it
    bad = O.embedding(ids + 1, w, s, b, K, g, bits, out_dtype=O.F32).astype(np.float64)
    assert not np.allclose(bad @ xf, want, rtol=1e-3, atol=1e-4)


def test_embedding_out_of_range_and_rounding():
    V, K, g, bits = 7, 128, 32, 8
    _, w, s, b = O.synth_problem(1, V, K, g, bits, seed=22)
    ids = np.array([[6, -1], [7, 2]])
    f32 = O.embedding(ids, w, s, b, K, g, bits, out_dtype=O.F32)
    assert f32.shape == (2, 2, K) and not f32[0, 1].any() and not f32[1, 0].any()
    h = O.embedding(ids, w, s, b, K, g, bits, out_dtype=O.BF16)
    np.testing.assert_array_equal(h, O.f32_to_bf16(f32))


# ------------------------------------------------------------------ large-M route (bf16 weight tiles)
def test_qmm_bf16w_equals_exact_when_weights_fit_bf16():
    """With power-of-two scales and biases that keep s*q + b within 8
    significant bits, the bf16 rounding of W changes nothing: the bf16-tile
    product equals the exact one"""
    rng = np.random.default_rng(5)
    M, N, K, g, bits = 3, 16, 128, 32, 4
    q = rng.integers(0, 16, size=(N, K)).astype(np.uint32)
    w = O.pack(q, bits)
    G = K // g
    s = O.f32_to_bf16((2.0 ** rng.integers(-6, 3, size=(N, G))).astype(np.float32))
    b = O.f32_to_bf16((rng.integers(-100, 100, size=(N, G)) * O.bf16_to_f32(s)).astype(np.float32))
    x, _, _, _ = O.synth_problem(M, N, K, g, bits, seed=5, stream=2)
    np.testing.assert_array_equal(O.qmm_bf16w_f64(x, w, s, b, K, g, bits), O.qmm_f64(x, w, s, b, K, g, bits))


def test_qmm_bf16w_rounding_matches_torch():
    """the weight tile rounding is round-to-nearest-even, checked against
    torch's independent float32 -> bfloat16 conversion; a truncating
    conversion (a plausible mistake) is rejected by the same comparison"""
    import torch

    M, N, K, g, bits = 2, 64, 256, 64, 4
    x, w, s, b = O.synth_problem(M, N, K, g, bits, seed=6, stream=3)
    wd = O.dequantize(w, s, b, K, g, bits)
    wt = torch.from_numpy(wd).to(torch.bfloat16).to(torch.float64).numpy()
    want = O.bf16_to_f32(x).astype(np.float64) @ wt.T
    np.testing.assert_array_equal(O.qmm_bf16w_f64(x, w, s, b, K, g, bits), want)
    trunc = (wd.view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    assert not np.array_equal(O.bf16_to_f32(x).astype(np.float64) @ trunc.T, want)
