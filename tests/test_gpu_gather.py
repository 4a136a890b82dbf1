"""GPU parity tests of gather_qmm (stacked experts selected per token).

The contract follows the reference's wrapper and its test
(src/engine/mlx_lm/utils/moe.rs:20-31, :84-146): out[b] = x[b] @
dequant(w[idx[b]]).T with x's batch dims broadcast against the indices.
Every case is held to the oracle's float64 gather (oracle.gather_qmm_f64) at
the same bar as quantized_matmul (max|err| <= atol + rtol*max|y_ref| and
<= 2 bf16 ulps of max|y_ref|; the v_dot2 GEMV dequantizes exactly, so also
elementwise).  Full-size MoE shapes add a size-independent property: each
selection equals quantized_matmul on the selected expert, bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_parity import check, dev16, dev32, u16

pytestmark = pytest.mark.gpu


def _miqmm():
    import miqmm

    return miqmm


def _experts(E, N, K, g, bits, sbd=O.BF16, seed=0):
    """E seeded experts from the C oracle's generator, stacked [E, N, ...]"""
    ws, ss, bs = [], [], []
    for e in range(E):
        _, w, s, b = O.c_synth_problem(1, N, K, g, bits, sb_dtype=sbd, seed=seed, stream=100 + e)
        ws.append(w), ss.append(s), bs.append(b)
    w, s, b = np.stack(ws), np.stack(ss), np.stack(bs)
    sdt = torch.float16 if sbd == O.F16 else torch.bfloat16
    return (w, s, b), (dev32(w), dev16(s, sdt), dev16(b, sdt))


def _x(shape, K, seed):
    rows = int(np.prod(shape))
    x, _, _, _ = O.c_synth_problem(rows, 8, K, 32, 4, seed=seed, stream=7)
    x = x.reshape(tuple(shape) + (K,))
    return x, dev16(x)


# (bits, g, scale dtype, E, N, K, token batch, top_k, M, x shared by the top_k selections)
CASES = [
    (4, 64, O.BF16, 8, 96, 256, 1, 2, 1, True),
    (4, 64, O.BF16, 8, 96, 256, 3, 4, 1, False),
    (4, 32, O.F16, 5, 130, 192, 2, 3, 2, True),
    (4, 128, O.BF16, 4, 64, 512, 2, 2, 3, False),
    (8, 64, O.BF16, 6, 100, 128, 2, 3, 1, True),
    (8, 32, O.F16, 3, 33, 96, 1, 3, 5, False),
    (4, 64, O.BF16, 4, 48, 1408, 2, 2, 16, True),
    (8, 128, O.BF16, 4, 40, 256, 1, 2, 17, False),
    (4, 64, O.BF16, 3, 200, 64, 4, 1, 1, True),
]


@pytest.mark.parametrize("bits,g,sbd,E,N,K,T,top_k,M,shared", CASES)
def test_gather_matches_oracle(gpu, c_oracle, bits, g, sbd, E, N, K, T, top_k, M, shared):
    m = _miqmm()
    (w, s, b), (wd, sd, bd) = _experts(E, N, K, g, bits, sbd, seed=E * 31 + N)
    rng = np.random.default_rng(K + N)
    idx = rng.integers(0, E, size=(T, top_k)).astype(np.int32)
    xshape = (T, 1, M) if shared else (T, top_k, M)
    x, xd = _x(xshape, K, seed=M + T)
    y = m.gather_qmm(xd, wd, sd, bd, torch.from_numpy(idx).cuda(), True, g, bits)
    assert y.shape == (T, top_k, M, N)
    ref = O.gather_qmm_f64(x, w, s, b, idx, K, g, bits, sb_dtype=sbd)
    check(y, ref, True, f"gather bits={bits} g={g} E={E} N={N} K={K} T={T} k={top_k} M={M} shared={shared}")


def test_gather_reference_test(gpu, c_oracle):
    """The reference's own test (moe.rs:84-146): deterministic fills
    ((i%7)-3)*0.05 for w [4, 32, 64] and ((i%5)-2)*0.1 for x [3, 64], g=64,
    bits=4, inds [0,1,2,3,1,0] as [3, 2], x reshaped [3, 1, 1, 64]; the result
    is [3, 2, 1, 32] and each slice matches dequantize(w[e]) @ x[m] within 1e-2."""
    from test_gpu_parity import _mlx_style_quantize

    m = _miqmm()
    E, out, k_in, g, bits, M, K = 4, 32, 64, 64, 4, 3, 2
    wf = ((np.arange(E * out * k_in) % 7) - 3.0).astype(np.float32).reshape(E, out, k_in) * np.float32(0.05)
    xf = ((np.arange(M * k_in) % 5) - 2.0).astype(np.float32).reshape(M, k_in) * np.float32(0.1)
    quant = [_mlx_style_quantize(wf[e], g, bits) for e in range(E)]
    wq = np.stack([q[0] for q in quant])
    sc = np.stack([q[1] for q in quant])
    bi = np.stack([q[2] for q in quant])
    wd, sd, bd = dev32(wq), dev16(sc), dev16(bi)
    x = dev16(O.f32_to_bf16(xf))
    inds_v = [0, 1, 2, 3, 1, 0]
    inds = torch.tensor(inds_v, dtype=torch.int32).reshape(M, K).cuda()
    got = m.gather_qmm(x.reshape(M, 1, 1, k_in), wd, sd, bd, inds, True, g, bits, False)
    assert tuple(got.shape) == (M, K, 1, out)
    for mi in range(M):
        for ki in range(K):
            e = inds_v[mi * K + ki]
            w_de = m.dequantize(wd[e], sd[e], bd[e], g, bits, dtype=torch.float32)
            ref = (w_de @ x[mi].float().reshape(k_in, 1)).reshape(out)
            diff = (got[mi, ki, 0].float() - ref).abs().max().item()
            assert diff < 1e-2, (mi, ki, e, diff)
    ref = O.gather_qmm_f64(u16(x).reshape(M, 1, 1, k_in), wq, sc, bi, np.array(inds_v).reshape(M, K), k_in, g, bits)
    check(got, ref, True, "reference test")


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_deepseek_decode_shapes_equal_quantized_matmul(gpu, c_oracle, bits):
    """DeepSeek-V2-Lite routed experts (64 experts, top-6, hidden 2048, expert
    inter 1408), one decode token and a 64-token batch: gate/up take the token's
    x for every selection, down takes one h per selection.  Every selection
    equals quantized_matmul on its expert bit for bit (same GEMV, same order),
    and the one-token case is held to the oracle."""
    m = _miqmm()
    E, H, I, top_k, g = 64, 2048, 1408, 6, 64
    gate = m.synth_problem(1, E * I, H, g, bits, seed=1, stream_id=1)[1:]
    down = m.synth_problem(1, E * H, I, g, bits, seed=2, stream_id=2)[1:]
    gw, gs, gb = (t.reshape(E, I, -1) for t in gate)
    dw, ds, db = (t.reshape(E, H, -1) for t in down)
    for T in (1, 64):
        gen = torch.Generator().manual_seed(T)
        idx = torch.stack([torch.randperm(E, generator=gen)[:top_k] for _ in range(T)]).to(torch.int32).cuda()
        x = m.synth_problem(T, 8, H, g, bits, seed=3, stream_id=T)[0].reshape(T, 1, 1, H)
        h = m.synth_problem(T * top_k, 8, I, g, bits, seed=4, stream_id=T)[0].reshape(T, top_k, 1, I)
        # the per-selection path (the 64-token batch would otherwise be grouped
        # by expert, whose MFMA GEMV sums in another order)
        yg = m.gather_qmm(x, gw, gs, gb, idx, True, g, bits, grouped=False)
        yd = m.gather_qmm(h, dw, ds, db, idx, True, g, bits, grouped=False)
        assert yg.shape == (T, top_k, 1, I) and yd.shape == (T, top_k, 1, H)
        torch.cuda.synchronize()
        idx_h = idx.cpu().numpy()
        for t in range(T) if T == 1 else (0, T // 2, T - 1):
            for j in range(top_k):
                e = int(idx_h[t, j])
                wg = m.quantized_matmul(x[t, 0], gw[e], gs[e], gb[e], True, g, bits, route=m.ROUTE_QMV_DOT)
                wdn = m.quantized_matmul(h[t, j], dw[e], ds[e], db[e], True, g, bits, route=m.ROUTE_QMV_DOT)
                assert torch.equal(yg[t, j], wg), (T, t, j, e)
                assert torch.equal(yd[t, j], wdn), (T, t, j, e)
        if T == 1:
            sel = sorted(set(idx_h.reshape(-1).tolist()))
            remap = {e: i for i, e in enumerate(sel)}
            ridx = np.vectorize(remap.get)(idx_h)
            sub = lambda t: t[sel].cpu().contiguous()  # noqa: E731
            w_n = sub(gw).view(torch.int32).numpy().view(np.uint32)
            s_n = sub(gs).view(torch.int16).numpy().view(np.uint16)
            b_n = sub(gb).view(torch.int16).numpy().view(np.uint16)
            ref = O.gather_qmm_f64(u16(x), w_n, s_n, b_n, ridx, H, g, bits)
            check(yg, ref, True, f"deepseek gate bits={bits}")


def test_gather_out_of_range_indices_give_zero_rows(gpu, c_oracle):
    m = _miqmm()
    E, N, K, g, bits = 4, 64, 256, 64, 4
    (w, s, b), (wd, sd, bd) = _experts(E, N, K, g, bits, seed=3)
    idx = np.array([[0, -1, 3], [4, 2, 2 ** 31 - 1]], np.int64)
    x, xd = _x((2, 1, 1), K, seed=9)
    y = m.gather_qmm(xd, wd, sd, bd, torch.from_numpy(idx).cuda(), True, g, bits)
    yf = y.float().cpu()
    for pos in [(0, 1), (1, 0), (1, 2)]:
        assert not yf[pos].any(), pos
    ref = O.gather_qmm_f64(x, w, s, b, idx, K, g, bits)
    check(y, ref, True, "out-of-range indices")


def test_gather_broadcast_forms(gpu, c_oracle):
    """x batch broadcast in the leading dims (materialised), a bare [M, K] x
    shared by every selection, index dtypes int64 / uint8, fp32 output from
    mixed dtypes, and an empty index set."""
    m = _miqmm()
    E, N, K, g, bits = 5, 40, 128, 32, 8
    (w, s, b), (wd, sd, bd) = _experts(E, N, K, g, bits, seed=4)
    idx = np.array([[1, 4], [0, 0], [3, 2]])
    x, xd = _x((1, 2, 2), K, seed=5)  # batch (1, 2) against (3, 2)
    y = m.gather_qmm(xd, wd, sd, bd, torch.from_numpy(idx).cuda(), True, g, bits)
    assert y.shape == (3, 2, 2, N)
    check(y, O.gather_qmm_f64(x, w, s, b, idx, K, g, bits), True, "leading broadcast")
    x2, xd2 = _x((3,), K, seed=6)  # [M=3, K], no batch dims
    idx2 = np.array([4, 1, 1, 0], np.uint8)
    y2 = m.gather_qmm(xd2, wd, sd, bd, torch.from_numpy(idx2).cuda(), True, g, bits)
    assert y2.shape == (4, 3, N)
    check(y2, O.gather_qmm_f64(x2, w, s, b, idx2, K, g, bits), True, "shared bare x")
    sh, bh = sd.to(torch.float16), bd.to(torch.float16)
    y3 = m.gather_qmm(xd, wd, sh, bh, torch.from_numpy(idx).cuda(), True, g, bits)
    assert y3.dtype == torch.float32
    check(y3, O.gather_qmm_f64(x, w, u16(sh), u16(bh), idx, K, g, bits, sb_dtype=O.F16), True, "fp16 scales")
    y4 = m.gather_qmm(xd, wd, sd, bd, torch.zeros((0, 2), dtype=torch.int32, device="cuda"), True, g, bits)
    assert y4.shape == (0, 2, 2, N)


# (bits, g, scale dtype, E, N, K, tokens, top_k, x shared) -- enough selections per expert for the
# expert-grouped tiled matmul (>= 8 on average)
GROUPED = [
    (4, 64, O.BF16, 8, 256, 512, 128, 2, True),
    (4, 32, O.F16, 4, 200, 256, 64, 2, False),
    (8, 64, O.BF16, 6, 136, 384, 100, 3, True),
    (4, 128, O.BF16, 2, 320, 1024, 300, 1, False),
]


@pytest.mark.parametrize("bits,g,sbd,E,N,K,T,top_k,shared", GROUPED)
def test_gather_grouped_matches_oracle(gpu, c_oracle, bits, g, sbd, E, N, K, T, top_k, shared):
    """the expert-grouped path (selections grouped by expert on the device,
    each expert streamed once through the tiled MFMA matmul) against the
    oracle, with out-of-range ids among them; held to the qmm route's bar"""
    m = _miqmm()
    (w, s, b), (wd, sd, bd) = _experts(E, N, K, g, bits, sbd, seed=E * 7 + K)
    rng = np.random.default_rng(N + T)
    idx = rng.integers(0, E, size=(T, top_k)).astype(np.int32)
    idx[rng.integers(0, T, size=3), 0] = E + 5  # out of range: zero rows
    xshape = (T, 1, 1) if shared else (T, top_k, 1)
    x, xd = _x(xshape, K, seed=T)
    y = m.gather_qmm(xd, wd, sd, bd, torch.from_numpy(idx).cuda(), True, g, bits, grouped=True)
    assert y.shape == (T, top_k, 1, N)
    ref = O.gather_qmm_f64(x, w, s, b, idx, K, g, bits, sb_dtype=sbd)
    check(y, ref, False, f"grouped bits={bits} g={g} E={E} N={N} K={K} T={T} k={top_k} shared={shared}")
    bad = np.argwhere(idx >= E)
    yf = y.float().cpu().numpy()
    for t, j in bad:
        assert not yf[t, j].any()


# (bits, g, scale dtype, E, N, K, tokens, top_k, x shared, skew) -- 4 to 8
# selections per expert: the expert-grouped MFMA GEMV (16 selections per
# tile); skew sends most selections to expert 0, which then spans tiles
GROUPED_GEMV = [
    (4, 64, O.BF16, 16, 200, 512, 40, 2, True, False),
    (8, 32, O.F16, 8, 136, 384, 12, 3, False, False),
    (4, 128, O.BF16, 4, 320, 1024, 12, 2, True, False),
    (4, 64, O.F16, 8, 96, 256, 40, 1, True, True),
    (8, 64, O.BF16, 8, 64, 512, 20, 2, False, True),
]


@pytest.mark.parametrize("bits,g,sbd,E,N,K,T,top_k,shared,skew", GROUPED_GEMV)
def test_gather_grouped_gemv_matches_oracle(gpu, c_oracle, bits, g, sbd, E, N, K, T, top_k, shared, skew):
    """the expert-grouped MFMA GEMV (selections grouped by expert on the
    device, each selected expert's weights streamed once for up to 16 of its
    selections, exact fp32 dequant) against the oracle, with out-of-range ids;
    and against the per-selection path"""
    m = _miqmm()
    (w, s, b), (wd, sd, bd) = _experts(E, N, K, g, bits, sbd, seed=E * 11 + K)
    rng = np.random.default_rng(N + T + 1)
    idx = rng.integers(0, E, size=(T, top_k)).astype(np.int32)
    if skew:
        idx[: (3 * T) // 4, 0] = 0
    idx[rng.integers(0, T, size=2), -1] = -3  # out of range: zero rows
    xshape = (T, 1, 1) if shared else (T, top_k, 1)
    x, xd = _x(xshape, K, seed=T + 7)
    ti = torch.from_numpy(idx).cuda()
    y = m.gather_qmm(xd, wd, sd, bd, ti, True, g, bits, grouped=True)
    assert y.shape == (T, top_k, 1, N)
    ref = O.gather_qmm_f64(x, w, s, b, idx, K, g, bits, sb_dtype=sbd)
    check(y, ref, True, f"grouped GEMV bits={bits} g={g} E={E} N={N} K={K} T={T} k={top_k} shared={shared}")
    yf = y.float().cpu().numpy()
    for t, j in np.argwhere((idx < 0) | (idx >= E)):
        assert not yf[t, j].any()
    ys = m.gather_qmm(xd, wd, sd, bd, ti, True, g, bits, grouped=False)
    rep = O.parity_report(yf.astype(np.float64), ys.float().cpu().numpy().astype(np.float64))
    assert rep["max_err"] <= rep["mag_bar"] and rep["max_err"] <= rep["ulp2_bar"], rep


def test_gather_grouped_deepseek_prefill(gpu, c_oracle):
    """DeepSeek-V2-Lite experts at a 1024-token prefill (6144 selections over
    64 experts): grouped and per-selection paths agree within the bar, and
    sampled selections meet the oracle"""
    m = _miqmm()
    E, H, I, top_k, g, T = 64, 2048, 1408, 6, 64, 1024
    gate = m.synth_problem(1, E * I, H, g, 4, seed=1, stream_id=1)[1:]
    gw, gs, gb = (t.reshape(E, I, -1) for t in gate)
    gen = torch.Generator().manual_seed(5)
    idx = torch.stack([torch.randperm(E, generator=gen)[:top_k] for _ in range(T)]).to(torch.int32).cuda()
    x = m.synth_problem(T, 8, H, g, 4, seed=3, stream_id=9)[0].reshape(T, 1, 1, H)
    yg = m.gather_qmm(x, gw, gs, gb, idx, True, g, 4, grouped=True)
    ys = m.gather_qmm(x, gw, gs, gb, idx, True, g, 4, grouped=False)
    torch.cuda.synchronize()
    rep = O.parity_report(yg.float().cpu().numpy(), ys.float().cpu().numpy().astype(np.float64))
    assert rep["max_err"] <= rep["mag_bar"] and rep["max_err"] <= rep["ulp2_bar"], rep
    idx_h = idx.cpu().numpy()
    xs = u16(x)
    for t in (0, 511, 1023):
        for j in range(top_k):
            e = int(idx_h[t, j])
            w_n = gw[e].cpu().contiguous().view(torch.int32).numpy().view(np.uint32)
            s_n = gs[e].cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
            b_n = gb[e].cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
            ref = O.qmm_f64(xs[t, 0], w_n, s_n, b_n, H, g, 4)
            check(yg[t, j], ref, False, f"prefill t={t} j={j}")
