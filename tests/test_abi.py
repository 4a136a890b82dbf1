"""CPU tests of the C ABI (include/miqmm.h): the library loads, exports every
declared function, and rejects invalid arguments on the host before touching
a GPU, with mlx-c's status convention (0 ok, nonzero + message;
src/engine/mlx_lm/utils/moe.rs:66-76).  No compute call runs here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"\b(miqmm_[a-z_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import miqmm

    return miqmm.lib()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert {"miqmm_quantized_matmul", "miqmm_quantized_linear", "miqmm_dequantize",
            "miqmm_unpack", "miqmm_last_error", "miqmm_checkpoint_open"} <= set(names)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in miqmm.h but not exported"


def test_version(lib):
    import miqmm

    assert "gfx950" in miqmm.version()


def _qmm(lib, **kw):
    a = dict(y=ctypes.c_void_p(16), x=ctypes.c_void_p(16), w=ctypes.c_void_p(16), s=ctypes.c_void_p(16),
             b=ctypes.c_void_p(16), M=1, N=64, K=128, transpose=1, g=64, bits=4, xd=0, sd=0, yd=0, route=0)
    a.update(kw)
    return lib.miqmm_quantized_matmul_ex(a["y"], a["x"], a["w"], a["s"], a["b"], a["M"], a["N"], a["K"],
                                         a["transpose"], a["g"], a["bits"], a["xd"], a["sd"], a["yd"],
                                         a["route"], None)


@pytest.mark.parametrize("kw,status,msg", [
    (dict(transpose=0), 2, "transpose=false"),
    (dict(bits=3), 2, "bits=3"),
    (dict(bits=7), 1, "bits must be 4 or 8"),
    (dict(g=16), 1, "group_size"),
    (dict(K=96, g=64), 1, "not a multiple of group_size"),
    (dict(N=0), 1, "N and K"),
    (dict(K=-64), 1, "N and K"),
    (dict(K=(1 << 22) + 64), 1, "32-bit tile offsets"),
    (dict(M=-1), 1, "M must be"),
    (dict(xd=1), 2, "x dtype"),
    (dict(sd=2), 2, "scales/biases dtype"),
    (dict(yd=7), 1, "y dtype"),
    (dict(route=9), 1, "route"),
    (dict(route=5, M=5), 2, "qmvs takes one to four rows"),
    (dict(route=5, K=32768, g=64), 2, "15 KiB"),
    (dict(route=5, K=192, g=64), 2, "even K/group_size"),
    (dict(route=5, s=ctypes.c_void_p(18)), 2, "4-byte aligned"),
    (dict(x=ctypes.c_void_p(8)), 1, "16-byte aligned"),
    (dict(w=ctypes.c_void_p(20)), 1, "16-byte aligned"),
    (dict(y=None), 1, "null pointer"),
])
def test_validation_errors(lib, kw, status, msg):
    assert _qmm(lib, **kw) == status
    assert msg in lib.miqmm_last_error().decode()


def test_m_zero_is_noop_and_clears_error(lib):
    assert _qmm(lib, bits=7) == 1
    assert _qmm(lib, M=0, y=None, x=None) == 0
    assert lib.miqmm_last_error().decode() == ""


def test_other_entry_points_validate(lib):
    P = ctypes.c_void_p(16)
    assert lib.miqmm_dequantize(P, P, P, P, 8, 96, 64, 4, 0, 0, None) == 1
    assert lib.miqmm_dequantize(P, P, P, P, 8, 128, 64, 4, 0, 5, None) == 1
    assert lib.miqmm_unpack(P, P, 8, 100, 4, None) == 1
    assert lib.miqmm_unpack(P, P, 8, 128, 2, None) == 1
    assert lib.miqmm_synth_problem(P, P, P, None, 1, 8, 128, 64, 4, 0, 0, 0, 0, None) == 1
    assert lib.miqmm_quantized_linear(None, P, P, P, P, None, 1, 8, 128, 64, 4, 0, 0, 0, None) == 1


def test_grouped_entry_point_validates(lib):
    import miqmm

    G = lib.miqmm_quantized_matmul_grouped
    assert G(None, -1, 1, 128, 64, 4, 0, 0, 0, None) == miqmm.EINVAL
    assert G(None, 2, 1, 128, 64, 4, 0, 0, 0, None) == miqmm.EINVAL  # no table for two problems
    assert G(None, 0, 1, 128, 64, 4, 0, 0, 0, None) == miqmm.OK      # nothing to do
    probs = (miqmm.Problem * 2)()
    probs[0] = miqmm.Problem(16, 16, 16, 16, 16, None, 8)
    probs[1] = miqmm.Problem(16, 16, 16, 16, 16, None, 8)
    assert G(probs, 2, 1, 96, 64, 4, 0, 0, 0, None) == miqmm.EINVAL  # K % group_size != 0
    assert G(probs, 2, 1, 128, 64, 3, 0, 0, 0, None) == miqmm.ENOTSUP
    probs[1] = miqmm.Problem(None, 16, 16, 16, 16, None, 8)
    assert G(probs, 2, 1, 128, 64, 4, 0, 0, 0, None) == miqmm.EINVAL  # null y in the second problem
    assert b"null" in lib.miqmm_last_error()
    assert G(probs, 2, 0, 128, 64, 4, 0, 0, 0, None) == miqmm.OK      # M == 0 is a no-op


def test_gather_entry_point_validates(lib):
    import miqmm

    P = ctypes.c_void_p(16)

    def G(idx=P, batch=1, top_k=6, xpi=0, M=1, N=64, K=128, E=8, transpose=1, g=64, bits=4, y=P):
        return lib.miqmm_gather_qmm(y, P, P, P, P, idx, batch, top_k, xpi, M, N, K, E, transpose, g, bits,
                                    0, 0, 0, 0, None)

    assert G(batch=-1) == miqmm.EINVAL and "batch and top_k" in lib.miqmm_last_error().decode()
    assert G(E=0) == miqmm.EINVAL and "experts" in lib.miqmm_last_error().decode()
    assert G(xpi=2) == miqmm.EINVAL
    assert G(transpose=0) == miqmm.ENOTSUP
    assert G(bits=3) == miqmm.ENOTSUP
    assert G(K=96) == miqmm.EINVAL
    assert G(idx=None) == miqmm.EINVAL and "null" in lib.miqmm_last_error().decode()
    assert G(y=None) == miqmm.EINVAL
    # no selections or no rows: nothing is read, so null pointers are accepted
    assert G(batch=0, idx=None, y=None) == miqmm.OK
    assert G(M=0, idx=None, y=None) == miqmm.OK


def test_gather_workspace_entry_points_validate(lib):
    import miqmm

    nb = ctypes.c_int64()
    assert lib.miqmm_gather_qmm_workspace_size(1024, 6, 64, ctypes.byref(nb)) == miqmm.OK
    assert nb.value >= 4 * (1024 * 6 + 64)
    assert lib.miqmm_gather_qmm_workspace_size(1, 6, 0, ctypes.byref(nb)) == miqmm.EINVAL
    P = ctypes.c_void_p(16)
    W = lib.miqmm_gather_qmm_ws
    args = [P, P, P, P, P, P, 1024, 6, 0, 1, 64, 128, 8, 1, 64, 4, 0, 0, 0, 0]
    assert W(*args, P, -1, None) == miqmm.EINVAL  # negative workspace size
    assert W(*args[:8], 2, *args[9:], P, 0, None) == miqmm.EINVAL  # x_per_index
    assert W(*args[:13], 0, *args[14:], P, 0, None) == miqmm.ENOTSUP  # transpose


def test_embedding_entry_point_validates(lib):
    import miqmm

    P = ctypes.c_void_p(16)
    E = lib.miqmm_quantized_embedding
    assert E(P, P, 4, P, P, P, 100, 96, 64, 4, 0, 0, None) == miqmm.EINVAL  # K % g
    assert E(P, P, 4, P, P, P, 100, 128, 64, 3, 0, 0, None) == miqmm.ENOTSUP
    assert E(P, P, 4, P, P, P, 100, 128, 64, 4, 0, 7, None) == miqmm.EINVAL  # out dtype
    assert E(P, P, -1, P, P, P, 100, 128, 64, 4, 0, 0, None) == miqmm.EINVAL
    assert E(P, None, 4, P, P, P, 100, 128, 64, 4, 0, 0, None) == miqmm.EINVAL
    assert E(ctypes.c_void_p(8), P, 4, P, P, P, 100, 128, 64, 4, 0, 0, None) == miqmm.EINVAL  # alignment
    assert E(None, None, 0, P, P, P, 100, 128, 64, 4, 0, 0, None) == miqmm.OK  # no ids: nothing to do


def test_gather_python_shape_checks(lib):
    import torch

    import miqmm

    w = torch.zeros((4, 8, 16), dtype=torch.int32)
    s = torch.zeros((4, 8, 2), dtype=torch.bfloat16)
    x = torch.zeros((2, 1, 1, 128), dtype=torch.bfloat16)
    idx = torch.zeros((2, 3), dtype=torch.int32)
    with pytest.raises(miqmm.MiqmmError, match="stacked"):
        miqmm.gather_qmm(x, w[0], s[0], s[0], idx)
    with pytest.raises(miqmm.MiqmmError, match="must be"):
        miqmm.gather_qmm(x[..., :64], w, s, s, idx)
    with pytest.raises(miqmm.MiqmmError, match="broadcast"):
        miqmm.gather_qmm(x, w, s, s, torch.zeros((3, 3), dtype=torch.int32))
    with pytest.raises(miqmm.MiqmmError, match="integers"):
        miqmm.gather_qmm(x, w, s, s, idx.float())


def test_workspace_entry_points_validate(lib):
    import miqmm

    n = ctypes.c_int64(-1)
    # GEMV routes and unsplit plans take no workspace; a split plan k ranges * M * N * 4
    assert lib.miqmm_quantized_matmul_workspace_size(1, 4096, 4096, 64, 4, ctypes.byref(n)) == 0 and n.value == 0
    assert lib.miqmm_quantized_matmul_workspace_size(2048, 14336, 4096, 64, 4, ctypes.byref(n)) == 0
    assert n.value == 0
    assert lib.miqmm_quantized_matmul_workspace_size(256, 4096, 4096, 64, 4, ctypes.byref(n)) == 0
    ks = miqmm.query_route(256, 4096, 4096, 64, 4)[1][3]
    assert ks > 1 and n.value == ks * 256 * 4096 * 4
    assert miqmm.workspace_size(256, 4096, 4096) == n.value
    assert lib.miqmm_quantized_matmul_workspace_size(0, 4096, 4096, 64, 4, ctypes.byref(n)) == 0 and n.value == 0
    assert lib.miqmm_quantized_matmul_workspace_size(1, 4096, 4096, 64, 4, None) == 1
    assert lib.miqmm_quantized_matmul_workspace_size(-1, 4096, 4096, 64, 4, ctypes.byref(n)) == 1
    assert lib.miqmm_quantized_matmul_workspace_size(1, 4096, 4096, 48, 4, ctypes.byref(n)) == 1
    P = ctypes.c_void_p
    ws = lambda **kw: lib.miqmm_quantized_matmul_ws(
        P(16), P(16), P(16), P(16), P(16), None, kw.get("M", 256), 4096, 4096, kw.get("transpose", 1), 64, 4, 0,
        0, 0, kw.get("work", P(256)), kw.get("nbytes", 1 << 20), None)
    assert ws(nbytes=-1) == 1 and "workspace_bytes" in lib.miqmm_last_error().decode()
    assert ws(work=P(8)) == 1 and "16-byte aligned" in lib.miqmm_last_error().decode()
    assert ws(transpose=0) == 2 and "transpose" in lib.miqmm_last_error().decode()
    assert ws(M=0) == 0  # M == 0: nothing to do, nothing touched


def test_query_route(lib):
    import miqmm

    # M = 1 with rows of 2048 codes or more: the K-sliced GEMV, one wave per
    # 1 KiB slice of a row, 16 rows per block while that gives ~6 waves per CU
    # (the CU count is 256 without a device)
    assert miqmm.query_route(1, 14336, 4096, 64, 4) == (miqmm.ROUTE_QMVS, (16, 2, 896, 0))
    assert miqmm.query_route(1, 4096, 14336, 64, 4) == (miqmm.ROUTE_QMVS, (16, 7, 256, 0))
    assert miqmm.query_route(1, 6144, 4096, 64, 4) == (miqmm.ROUTE_QMVS, (8, 2, 768, 0))
    assert miqmm.query_route(1, 262144, 5376, 32, 4) == (miqmm.ROUTE_QMVS, (16, 3, 16384, 0))
    assert miqmm.query_route(1, 262144, 5376, 64, 8) == (miqmm.ROUTE_QMVS, (16, 6, 16384, 0))
    # an odd number of groups per row keeps the v_dot2 GEMV (scale rows not 4-byte aligned)
    assert miqmm.query_route(1, 4096, 2080, 32, 4)[0] == miqmm.ROUTE_QMV_DOT
    # rows of at most 32 chunks (K <= 1024 at 4 bits): the K-sliced GEMV, two
    # rows per wave slice; 4 rows per block below ~3 waves per CU
    assert miqmm.query_route(1, 4864, 896, 64, 4) == (miqmm.ROUTE_QMVS, (4, 1, 1216, 0))
    assert miqmm.query_route(1, 151936, 896, 64, 4) == (miqmm.ROUTE_QMVS, (16, 1, 9496, 0))
    # and rows in between (48 chunks: one slice, a quarter of the lanes idle)
    assert miqmm.query_route(1, 4864, 1536, 64, 4) == (miqmm.ROUTE_QMVS, (4, 1, 1216, 0))
    # 2 <= M <= 4: the K-sliced GEMV too, each row of codes unpacked once for
    # every row of x (three rows as four), on rows of up to 15 KiB of codes
    # (8 KiB with more than two rows of x)
    for M in (2, 3, 4):
        for N, K in ((14336, 4096), (4096, 14336), (4096, 4096), (6144, 4096), (4864, 896), (151936, 896)):
            assert miqmm.query_route(M, N, K, 64, 4)[0] == miqmm.ROUTE_QMVS, (M, N, K)
    # longer rows: the LDS-staged MFMA GEMV where it takes them (x of the
    # padded M rows within 64 KiB) ...
    route, tiles = miqmm.query_route(2, 4096, 16384, 64, 8)  # 16 KiB of codes per row
    assert route == miqmm.ROUTE_QMVX and tiles[0] == 2
    # ... else the group-diagonal MFMA GEMV
    for M, N, K in ((3, 4096, 20480), (4, 4096, 20480)):
        assert miqmm.query_route(M, N, K, 64, 4)[0] == miqmm.ROUTE_QMV, (M, N, K)
    # qmvx needs an even number of groups per row: K = 96, g = 32 falls back to v_dot2
    assert miqmm.query_route(2, 128, 96, 32, 4)[0] == miqmm.ROUTE_QMV_DOT
    for M in (5, 8, 16):
        route, tiles = miqmm.query_route(M, 14336, 4096, 64, 4)
        assert route == miqmm.ROUTE_QMV and tiles[0] in (1, 2, 4) and tiles[1] >= M and tiles[2] in (4, 16)
    # M = 17..32: the GEMVs in two passes (the launch of the first, 16 rows, reported)
    for M in (17, 24, 32):
        route, tiles = miqmm.query_route(M, 14336, 4096, 64, 4)
        assert route == miqmm.ROUTE_QMV and tiles[1] == 16, (M, tiles)
    assert miqmm.query_route(33, 14336, 4096, 64, 4)[0] == miqmm.ROUTE_QMM
    # rows of K >= 8192: passes up to M = 64
    assert miqmm.query_route(64, 4096, 14336, 64, 4)[0] == miqmm.ROUTE_QMV
    assert miqmm.query_route(65, 4096, 14336, 64, 4)[0] == miqmm.ROUTE_QMM
    # the workspace of two passes: the larger pass's partials, reused in order
    assert miqmm.workspace_size(32, 4096, 14336) == miqmm.workspace_size(16, 4096, 14336) > 0
    assert miqmm.workspace_size(17, 4096, 14336) == miqmm.workspace_size(16, 4096, 14336)
    route, tiles = miqmm.query_route(2048, 14336, 4096, 64, 4)
    assert route == miqmm.ROUTE_QMM and tiles[2] == 64
    # the qmm plan (rounds of one tile per CU): width and k ranges
    for (M, N, K), (bn, ks) in {(2048, 14336, 4096): (256, 1), (2048, 6144, 4096): (256, 1),
                                (2048, 4096, 4096): (128, 1), (2048, 4096, 14336): (256, 2),
                                (256, 4096, 4096): (128, 4), (33, 64, 256): (128, 1)}.items():
        route, tiles = miqmm.query_route(M, N, K, 64, 4)
        assert route == miqmm.ROUTE_QMM and tiles == (256, bn, 64, ks), ((M, N, K), tiles)
    # the MFMA GEMV's launch shape (unsplit): four tiles per block where that
    # gives a block per CU, else two or one where that gives 192 blocks
    assert miqmm.query_route(8, 14336, 4096, 64, 4)[1] == (2, 8, 4, 0)  # 448 blocks of two tiles
    assert miqmm.query_route(8, 32768, 4096, 64, 4)[1] == (4, 8, 4, 0)  # 512 blocks of four tiles
    assert miqmm.query_route(8, 6144, 4096, 64, 4)[1] == (2, 8, 4, 0)
    # K >= 8192: eight K-splitting waves at M <= 8, four at M = 16
    assert miqmm.query_route(8, 4096, 14336, 64, 4)[1] == (1, 8, 8, 0)
    assert miqmm.query_route(16, 4096, 14336, 64, 4)[1] == (1, 16, 4, 0)
    # with a workspace the MFMA GEMV splits K where long rows or a long
    # output at M > 8 make that faster: S k ranges of fp32 partials
    for M, N, K in ((16, 4096, 14336), (8, 4096, 14336), (16, 14336, 4096), (5, 512, 8192), (4, 4096, 20480)):
        n = miqmm.workspace_size(M, N, K)
        assert n > 0 and n % (M * N * 4) == 0 and n // (M * N * 4) <= 16, (M, N, K, n)
    for M, N, K in ((8, 14336, 4096), (16, 4096, 4096), (1, 4096, 14336), (2, 4096, 14336), (4, 14336, 4096),
                    (4, 4096, 14336)):
        assert miqmm.workspace_size(M, N, K) == 0, (M, N, K)
    with pytest.raises(miqmm.MiqmmError) as e:
        miqmm.query_route(1, 64, 96, 64, 4)
    assert e.value.status == miqmm.EINVAL


def test_python_mirror_validation():
    import torch

    import miqmm

    w = torch.zeros((64, 16), dtype=torch.int32)
    s = torch.zeros((64, 2), dtype=torch.bfloat16)
    x = torch.zeros((1, 128), dtype=torch.bfloat16)
    with pytest.raises(miqmm.MiqmmError, match="inner dim"):
        miqmm.quantized_matmul(torch.zeros((1, 64), dtype=torch.bfloat16), w, s, s, True, 64, 4)
    with pytest.raises(miqmm.MiqmmError, match="scales shape"):
        miqmm.quantized_matmul(x, w, s, s, True, 32, 4)
    with pytest.raises(miqmm.MiqmmError, match="uint32 words"):
        miqmm.quantized_matmul(x, w.float(), s, s, True, 64, 4)
    with pytest.raises(miqmm.MiqmmError) as e:
        miqmm.quantized_matmul(x, w, s, s, True, 64, 2)
    assert e.value.status == miqmm.ENOTSUP
    assert miqmm.result_type(torch.bfloat16, torch.float16) == torch.float32
    assert miqmm.result_type(torch.bfloat16, torch.bfloat16) == torch.bfloat16
    lin = miqmm.QuantizedLinear(w, s, s, group_size=64, bits=4)
    assert (lin.out_features, lin.in_features) == (64, 128)
