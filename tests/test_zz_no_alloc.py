"""GPU test of miqmm_quantized_matmul_noalloc, the entry point that allocates
nothing (its k-split scratch is a device array the code object holds): called
through the C ABI, it matches miqmm_quantized_matmul_ws (caller workspace) bit
for bit on two calls in a row, the second with a smaller input, both of which
split their k-steps into the scratch, and each meets the oracle bar on sampled
rows; a GEMV-route call needs no scratch; a shape whose split needs more
scratch than the array holds is refused with MIQMM_EINVAL."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _call(m, fn, dv, y, g, bits, *extra):
    x, w, s, b = dv
    M, K = x.shape
    N = w.shape[0]
    return fn(m._ptr(y), m._ptr(x), m._ptr(w), m._ptr(s), m._ptr(b), None, M, N, K, 1, g, bits, m._dt(x), m._dt(s),
              m._dt(y), *extra, m._stream(None))


def _problem(m, M, N, K, g, seed):
    x, w, s, b = m.synth_problem(M, N, K, g, 4, seed=seed, stream_id=M + N)
    return (x, w, s, b)


def test_noalloc_matches_workspace_entry_point(gpu, c_oracle):
    import miqmm as m

    L = m.lib()
    g = 64
    for i, (M, N, K) in enumerate([(256, 4096, 4096), (128, 2048, 4096)]):  # the second call is smaller
        need = m.workspace_size(M, N, K, g, 4)
        assert 0 < need <= SCRATCH_BYTES, (M, N, K, need)
        dv = _problem(m, M, N, K, g, seed=30 + i)
        y_ws = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        assert _call(m, L.miqmm_quantized_matmul_ws, dv, y_ws, g, 4, m._ptr(ws), need) == 0
        st = _call(m, L.miqmm_quantized_matmul_noalloc, dv, y_na, g, 4)
        assert st == 0, L.miqmm_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ws), (M, N, K)
        x, w, s, b = dv
        xh, wh = x.view(torch.int16).cpu().numpy().view(np.uint16), w.cpu().numpy().view(np.uint32)
        sh, bh = (t.view(torch.int16).cpu().numpy().view(np.uint16) for t in (s, b))
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(i).choice(M, 9, replace=False)]))
        ref = c_oracle.c_qmm_f64(np.ascontiguousarray(xh[rows]), wh, sh, bh, len(rows), N, K, g, 4)
        got = y_na[torch.from_numpy(rows).cuda()].float().cpu().numpy().astype(np.float64)
        rep = O.parity_report(got, ref, 1e-2, 1e-3)
        print("noalloc", (M, N, K), rep, flush=True)
        assert rep["max_err"] <= rep["mag_bar"] and rep["max_err"] <= rep["ulp2_bar"], rep


def test_noalloc_gemv_route_and_refusal(gpu, c_oracle):
    import miqmm as m

    L = m.lib()
    M, N, K, g = 1, 2048, 4096, 64
    assert m.workspace_size(M, N, K, g, 4) == 0
    dv = _problem(m, M, N, K, g, seed=40)
    y_na = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    assert _call(m, L.miqmm_quantized_matmul_noalloc, dv, y_na, g, 4) == 0
    y_ref = m.quantized_matmul(*dv, True, g, 4)
    torch.cuda.synchronize()
    assert torch.equal(y_na, y_ref)
    # a split that needs more scratch than the array holds is refused before any launch
    big = (512, 14336, 14336)
    need = m.workspace_size(*big, g, 4)
    assert need > SCRATCH_BYTES, need
    P = ctypes.c_void_p
    st = L.miqmm_quantized_matmul_noalloc(P(256), P(256), P(256), P(256), P(256), None, *big, 1, g, 4, 0, 0, 0, None)
    assert st == m.EINVAL and "miqmm_quantized_matmul_ws" in L.miqmm_last_error().decode()
