"""numpy restatement of MLX affine group-quantized matmul, plus a ctypes loader
for the C oracle (oracle/miqmm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

Reference citations (SenClaw/sen-mlx tree):
  - quantized_matmul(x, w, scales, biases, transpose=true, group_size, bits):
    src/engine/mlx_lm/utils/mod.rs:70-78; src/engine/mlx_lm/models/bonsai_q1.rs:469-477.
  - packed layout, LSB-first codes: src/engine/mlx_lm/models/bonsai_q1.rs:137-143,168-170
    (bits=1), generalised to bits 4 and 8.
  - shapes w [N, K*bits/32], scales/biases [N, K/g]: src/engine/mlx_lm/utils/moe.rs:20-31.
  - dequant fma(scale, q, bias) in fp32: src/engine/mlx_lm/models/bonsai_q1.rs:172.
  - quantized embedding lookup: src/engine/mlx_lm/models/bonsai_q1.rs:603-613.
  - gather_qmm (stacked experts [E, N, ...] selected per batch entry):
    src/engine/mlx_lm/utils/moe.rs:20-31, test at moe.rs:84-146.

The generator is the same splitmix64 counter hash + Irwin-Hall(4) normal as the
C oracle; every float step is a single IEEE fp32 operation, so numpy, C and HIP
agree bit for bit.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

BF16, F16, F32 = 0, 1, 2
GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
IH_SCALE = np.float32(2.6428997e-05)

HERE = os.path.dirname(os.path.abspath(__file__))
C_LIB = os.path.join(HERE, "libmiqmm_oracle.so")


# ---------------------------------------------------------------- conversions
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)"""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return r.astype(np.uint16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    return np.asarray(f, dtype=np.float32).astype(np.float16).view(np.uint16)


def half_to_f32(h: np.ndarray, dtype: int) -> np.ndarray:
    return f16_to_f32(h) if dtype == F16 else bf16_to_f32(h)


def f32_to_half(f: np.ndarray, dtype: int) -> np.ndarray:
    return f32_to_f16(f) if dtype == F16 else f32_to_bf16(f)


# ---------------------------------------------------------------- generator
def mix64(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def key(seed: int, tag: int) -> np.uint64:
    with np.errstate(over="ignore"):
        k = np.array([seed], dtype=np.uint64) * GAMMA + np.array([tag], dtype=np.uint64)
    return mix64(k)[0]


def draws(k: np.uint64, count: int, start: int = 0) -> np.ndarray:
    i = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(k) + i * GAMMA)


def normal(r: np.ndarray) -> np.ndarray:
    m = np.uint64(0xFFFF)
    s = (r & m) + ((r >> np.uint64(16)) & m) + ((r >> np.uint64(32)) & m) + ((r >> np.uint64(48)) & m)
    return (s.astype(np.int64) - 131070).astype(np.float32) * IH_SCALE


def tag(stream: int, kind: int) -> int:
    return stream * 8 + kind


def gen_normal(count: int, sigma: float, dtype: int, seed: int, tg: int) -> np.ndarray:
    v = normal(draws(key(seed, tg), count)) * np.float32(sigma)
    return f32_to_half(v, dtype)


def gen_codes(N: int, K: int, bits: int, seed: int, tg: int) -> np.ndarray:
    """unpacked codes q[N, K] (uint8), uniform in [0, 2^bits)"""
    r = draws(key(seed, tg), N * K)
    return (r >> np.uint64(64 - bits)).astype(np.uint8).reshape(N, K)


def gen_scales_biases(count: int, bits: int, dtype: int, seed: int, tag_s: int, tag_b: int):
    sv = np.abs(normal(draws(key(seed, tag_s), count))) * np.float32(0.02)
    sh = f32_to_half(sv, dtype)
    sr = half_to_f32(sh, dtype)
    noise = normal(draws(key(seed, tag_b), count)) * np.float32(0.002)
    bv = np.float32(-(1 << (bits - 1))) * sr
    bv = bv + noise
    return sh, f32_to_half(bv, dtype)


def synth_problem(M, N, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16, seed=0, stream=0):
    """(x[M,K] u16, w[N,K*bits/32] u32, scales[N,K/g] u16, biases[N,K/g] u16)"""
    x = gen_normal(M * K, 1.0, x_dtype, seed, tag(stream, 1)).reshape(M, K)
    q = gen_codes(N, K, bits, seed, tag(stream, 2))
    w = pack(q, bits)
    s, b = gen_scales_biases(N * (K // group_size), bits, sb_dtype, seed, tag(stream, 3), tag(stream, 4))
    return x, w, s.reshape(N, K // group_size), b.reshape(N, K // group_size)


# ---------------------------------------------------------------- layout
def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """codes [N, K] -> words [N, K*bits/32], code k at bit bits*(k mod per) of word k/per"""
    N, K = q.shape
    per = 32 // bits
    qq = q.astype(np.uint32).reshape(N, K // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * np.uint32(bits))
    return np.bitwise_or.reduce(qq << shifts, axis=2).astype(np.uint32)


def unpack(w: np.ndarray, K: int, bits: int) -> np.ndarray:
    N = w.shape[0]
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * np.uint32(bits))
    q = (w.astype(np.uint32)[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(N, K).astype(np.uint8)


def dequantize(w, s, b, K, group_size, bits, sb_dtype=BF16, exact=False) -> np.ndarray:
    """fp32 dequant fma(s, q, b) (exact=False) or exact float64 s*q+b"""
    q = unpack(w, K, bits)
    sf = np.repeat(half_to_f32(s, sb_dtype), group_size, axis=1)
    bf = np.repeat(half_to_f32(b, sb_dtype), group_size, axis=1)
    if exact:
        return sf.astype(np.float64) * q.astype(np.float64) + bf.astype(np.float64)
    # fp32 fma: the exact double value rounded once to fp32 (8+8 bit products are exact in double)
    return (sf.astype(np.float64) * q + bf.astype(np.float64)).astype(np.float32)


def qmm_f64(x, w, s, b, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16) -> np.ndarray:
    wd = dequantize(w, s, b, K, group_size, bits, sb_dtype, exact=True)
    return half_to_f32(x, x_dtype).astype(np.float64) @ wd.T


def qmm_bf16w_f64(x, w, s, b, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16) -> np.ndarray:
    """The large-M route's arithmetic (MLX's qmm, reached from the reference's
    prefill, src/engine/mlx_native.rs:1918-1922,2094-2102): W dequantized with
    the fp32 fma, rounded to bf16 (the activation type of the dequantized
    tiles), then multiplied exactly (float64) by x."""
    wb = bf16_to_f32(f32_to_bf16(dequantize(w, s, b, K, group_size, bits, sb_dtype)))
    return half_to_f32(x, x_dtype).astype(np.float64) @ wb.astype(np.float64).T


def embedding(ids, w, s, b, K, group_size, bits, sb_dtype=BF16, out_dtype=BF16) -> np.ndarray:
    """out[..., k] = fma(s, q, b) of row ids[...] in fp32, rounded to out_dtype
    (bit patterns for bf16/fp16, float32 values for F32); an id outside
    [0, V) gives a zero row.  Restates the lookup at
    src/engine/mlx_lm/models/bonsai_q1.rs:603-613 (take rows, then dequantize)."""
    ids = np.asarray(ids)
    V = w.shape[0]
    flat = ids.reshape(-1).astype(np.int64)
    ok = (flat >= 0) & (flat < V)
    rows = np.where(ok, flat, 0)
    d = dequantize(w[rows], s[rows], b[rows], K, group_size, bits, sb_dtype)  # fp32
    d[~ok] = 0.0
    d = d.reshape(ids.shape + (K,))
    if out_dtype == F32:
        return d.astype(np.float32)
    return f32_to_half(d, out_dtype)


def gather_qmm_f64(x, w, s, b, idx, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16) -> np.ndarray:
    """out[i] = x[i] @ dequant(w[idx[i]]).T over the broadcast batch i (float64).

    Restates the gather_qmm wrapper's contract (src/engine/mlx_lm/utils/moe.rs:20-31,
    lhs_indices absent, transpose=true): w [E, N, K*bits/32], s/b [E, N, K/g],
    x [..., M, K] whose batch dims broadcast against idx [...]; the result is
    [*broadcast, M, N].  An index outside [0, E) gives zero rows (MLX leaves it
    undefined; the library defines it this way)."""
    x = np.asarray(x)
    idx = np.asarray(idx)
    E, N = w.shape[0], w.shape[1]
    M = x.shape[-2]
    bshape = np.broadcast_shapes(x.shape[:-2], idx.shape)
    xb = np.broadcast_to(x, bshape + (M, K)).reshape(-1, M, K)
    ib = np.broadcast_to(idx, bshape).reshape(-1)
    out = np.zeros((ib.size, M, N), np.float64)
    for i, e in enumerate(ib.tolist()):
        if 0 <= e < E:
            out[i] = qmm_f64(xb[i], w[e], s[e], b[e], K, group_size, bits, x_dtype, sb_dtype)
    return out.reshape(bshape + (M, N))


# ---------------------------------------------------------------- tolerance
def bf16_ulp(v: float) -> float:
    """spacing of bfloat16 numbers at |v| (8 significant bits)"""
    v = abs(float(v))
    if v == 0.0:
        return 2.0 ** -133
    e = np.floor(np.log2(v))
    return float(2.0 ** (e - 7))


def parity_report(y, y_ref, rtol=1e-2, atol=1e-3):
    """max |err|, the 2-bf16-ulp bar at max|y_ref|, and the rtol/atol bar at max|y_ref|"""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    err = np.abs(y - y_ref)
    mag = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    return {
        "max_err": float(err.max()) if err.size else 0.0,
        "max_ref": mag,
        "ulp2_bar": 2.0 * bf16_ulp(mag),
        "mag_bar": atol + rtol * mag,
        "elem_ok_frac": float(np.mean(err <= atol + rtol * np.abs(y_ref))) if err.size else 1.0,
    }


# ---------------------------------------------------------------- C oracle
def build_c_oracle(force: bool = False) -> str:
    if force or not os.path.exists(C_LIB):
        subprocess.run(["make", "-C", HERE, "-s"], check=True)
    return C_LIB


_c = None


def c_oracle():
    """ctypes handle to oracle/libmiqmm_oracle.so (built by oracle/Makefile)"""
    global _c
    if _c is not None:
        return _c
    if not os.path.exists(C_LIB):
        raise RuntimeError(f"C oracle not built: {C_LIB} (run make -C oracle)")
    lib = ctypes.CDLL(C_LIB)
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    U64 = ctypes.c_uint64
    I = ctypes.c_int
    lib.orc_mix64.argtypes, lib.orc_mix64.restype = [U64], U64
    lib.orc_key.argtypes, lib.orc_key.restype = [U64, U64], U64
    lib.orc_draw.argtypes, lib.orc_draw.restype = [U64, U64], U64
    lib.orc_normal.argtypes, lib.orc_normal.restype = [U64], ctypes.c_float
    lib.orc_f32_to_bf16.argtypes, lib.orc_f32_to_bf16.restype = [ctypes.c_float], ctypes.c_uint16
    lib.orc_f32_to_f16.argtypes, lib.orc_f32_to_f16.restype = [ctypes.c_float], ctypes.c_uint16
    lib.orc_synth_problem.argtypes = [P, P, P, P, I64, I64, I64, I, I, I, I, U64, U64]
    lib.orc_synth_problem.restype = None
    lib.orc_unpack.argtypes = [P, P, I64, I64, I]
    lib.orc_pack.argtypes = [P, P, I64, I64, I]
    lib.orc_dequantize.argtypes = [P, P, P, P, I64, I64, I, I, I]
    lib.orc_qmm_f32.argtypes = [P, I, P, P, P, P, I64, I64, I64, I, I, I, I]
    lib.orc_qmm_f64.argtypes = [P, I, P, P, P, P, I64, I64, I64, I, I, I, I]
    lib.orc_round.argtypes = [P, P, I64, I]
    lib.orc_half_to_f32.argtypes = [P, P, I64, I]
    _c = lib
    return lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def c_synth_problem(M, N, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16, seed=0, stream=0):
    lib = c_oracle()
    x = np.empty((M, K), np.uint16)
    w = np.empty((N, K * bits // 32), np.uint32)
    s = np.empty((N, K // group_size), np.uint16)
    b = np.empty_like(s)
    lib.orc_synth_problem(_p(x), _p(w), _p(s), _p(b), M, N, K, group_size, bits, x_dtype, sb_dtype, seed, stream)
    return x, w, s, b


def c_qmm_f32(x, w, s, b, M, N, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16, nthreads=0):
    y = np.empty((M, N), np.float32)
    c_oracle().orc_qmm_f32(_p(np.ascontiguousarray(x)), x_dtype, _p(np.ascontiguousarray(w)),
                           _p(np.ascontiguousarray(s)), _p(np.ascontiguousarray(b)), _p(y),
                           M, N, K, group_size, bits, sb_dtype, nthreads)
    return y


def c_qmm_f64(x, w, s, b, M, N, K, group_size, bits, x_dtype=BF16, sb_dtype=BF16, nthreads=0):
    y = np.empty((M, N), np.float64)
    c_oracle().orc_qmm_f64(_p(np.ascontiguousarray(x)), x_dtype, _p(np.ascontiguousarray(w)),
                           _p(np.ascontiguousarray(s)), _p(np.ascontiguousarray(b)), _p(y),
                           M, N, K, group_size, bits, sb_dtype, nthreads)
    return y


def c_unpack(w, N, K, bits):
    q = np.empty((N, K), np.uint8)
    c_oracle().orc_unpack(_p(np.ascontiguousarray(w)), _p(q), N, K, bits)
    return q


def c_dequantize(w, s, b, N, K, group_size, bits, sb_dtype=BF16):
    out = np.empty((N, K), np.float32)
    c_oracle().orc_dequantize(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(s)),
                              _p(np.ascontiguousarray(b)), _p(out), N, K, group_size, bits, sb_dtype)
    return out


def c_round(y32: np.ndarray, dtype: int) -> np.ndarray:
    y32 = np.ascontiguousarray(y32, dtype=np.float32)
    out = np.empty(y32.shape, np.float32 if dtype == F32 else np.uint16)
    c_oracle().orc_round(_p(y32), _p(out), y32.size, dtype)
    return out
