"""miqmm -- MI355X (gfx950) affine group-quantized matmul behind a C ABI.

Host-side mirror of the operator surface the reference (SenClaw/sen-mlx) uses
on its quantized decode/prefill path:

  quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
      mlx_rs::ops::quantized_matmul, called at src/engine/mlx_lm/utils/mod.rs:70-78
      and from every QuantizedLinear projection (src/engine/mlx_lm/models/llama.rs:195-197,
      249, 293-294) and tied lm_head (llama.rs:511-517).
  QuantizedLinear(weight, scales, biases, bias, group_size, bits)
      nn::QuantizedLinear behind MaybeQuantized<Linear> (llama.rs:115-126, 262-271);
      forward = quantized_matmul, then + bias when the Linear had one (llama.rs:139-147).
  dequantize(w, scales, biases, group_size, bits)
      mlx_rs::ops::dequantize as used at src/engine/mlx_lm/utils/moe.rs:118-126.
  gather_qmm(x, w, scales, biases, rhs_indices, transpose, group_size, bits, sorted_indices)
      the MoE expert matmul wrapped at src/engine/mlx_lm/utils/moe.rs:33-77.
  QuantizedEmbedding(weight, scales, biases, group_size, bits)
      lookup (src/engine/mlx_lm/models/bonsai_q1.rs:603-613) and as_linear, the tied
      lm_head (src/engine/mlx_lm/models/llama.rs:511-517).

Errors are raised as MiqmmError, the counterpart of mlx-rs's Exception built from
a nonzero mlx-c status (moe.rs:66-76).  Every call goes through libmiqmm.so;
there is no CPU fallback: if the library is missing the import-time loader
raises.  torch provides device memory and the current HIP stream only.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch

__all__ = [
    "MiqmmError", "quantized_matmul", "quantized_linear", "QuantizedLinear", "dequantize",
    "unpack", "synth_problem", "query_route", "result_type", "lib", "LIB_PATH", "quantized_matmul_grouped",
    "workspace_size",
    "Problem", "gather_qmm", "quantized_embedding", "QuantizedEmbedding",
    "OK", "EINVAL", "ENOTSUP", "EHIP", "ROUTE_AUTO", "ROUTE_QMV", "ROUTE_QMM", "ROUTE_QMV_DOT", "ROUTE_QMVX",
    "ROUTE_QMVS",
]

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmiqmm.so")

OK, EINVAL, ENOTSUP, EHIP = 0, 1, 2, 3
ROUTE_AUTO, ROUTE_QMV, ROUTE_QMM, ROUTE_QMV_DOT, ROUTE_QMVX, ROUTE_QMVS = 0, 1, 2, 3, 4, 5
DT_BF16, DT_F16, DT_F32 = 0, 1, 2

_DT = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}


class MiqmmError(RuntimeError):
    """a nonzero miqmm_status, with the library's message"""

    def __init__(self, status: int, message: str):
        super().__init__(f"miqmm status {status}: {message}")
        self.status = status


_lib = None


class Problem(ctypes.Structure):
    """miqmm_problem: one projection of a grouped call"""
    _fields_ = [("y", ctypes.c_void_p), ("x", ctypes.c_void_p), ("w", ctypes.c_void_p),
                ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("N", ctypes.c_int64)]


def lib() -> ctypes.CDLL:
    """the loaded libmiqmm.so (raises if it has not been built)"""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing; build it with `python sen-mlx_amd/build.py`")
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I, U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint64
    L.miqmm_quantized_matmul.argtypes = [P, P, P, P, P, I64, I64, I64, I, I, I, I, I, I, P]
    L.miqmm_quantized_matmul_ex.argtypes = [P, P, P, P, P, I64, I64, I64, I, I, I, I, I, I, I, P]
    L.miqmm_quantized_linear.argtypes = [P, P, P, P, P, P, I64, I64, I64, I, I, I, I, I, P]
    L.miqmm_dequantize.argtypes = [P, P, P, P, I64, I64, I, I, I, I, P]
    L.miqmm_unpack.argtypes = [P, P, I64, I64, I, P]
    L.miqmm_query_route.argtypes = [I64, I64, I64, I, I, ctypes.POINTER(I), ctypes.POINTER(I)]
    L.miqmm_synth_problem.argtypes = [P, P, P, P, I64, I64, I64, I, I, I, I, U64, U64, P]
    L.miqmm_quantized_matmul_grouped.argtypes = [ctypes.POINTER(Problem), I, I64, I64, I, I, I, I, I, P]
    L.miqmm_gather_qmm.argtypes = [P, P, P, P, P, P, I64, I64, I, I64, I64, I64, I64, I, I, I, I, I, I, I, P]
    L.miqmm_quantized_embedding.argtypes = [P, P, I64, P, P, P, I64, I64, I, I, I, I, P]
    L.miqmm_gather_qmm_workspace_size.argtypes = [I64, I64, I64, ctypes.POINTER(I64)]
    L.miqmm_quantized_matmul_workspace_size.argtypes = [I64, I64, I64, I, I, ctypes.POINTER(I64)]
    L.miqmm_quantized_matmul_ws.argtypes = [P, P, P, P, P, P, I64, I64, I64, I, I, I, I, I, I, P, I64, P]
    L.miqmm_quantized_matmul_noalloc.argtypes = [P, P, P, P, P, P, I64, I64, I64, I, I, I, I, I, I, P]
    L.miqmm_stream_read.argtypes = [P, I64, P, P]
    L.miqmm_gather_qmm_ws.argtypes = [P, P, P, P, P, P, I64, I64, I, I64, I64, I64, I64, I, I, I, I, I, I, I, P,
                                      I64, P]
    for name in ("miqmm_quantized_matmul", "miqmm_quantized_matmul_ex", "miqmm_quantized_linear",
                 "miqmm_dequantize", "miqmm_unpack", "miqmm_query_route", "miqmm_synth_problem",
                 "miqmm_quantized_matmul_grouped", "miqmm_quantized_matmul_workspace_size",
                 "miqmm_quantized_matmul_ws", "miqmm_quantized_matmul_noalloc", "miqmm_stream_read"):
        getattr(L, name).restype = I
    L.miqmm_last_error.argtypes, L.miqmm_last_error.restype = [], ctypes.c_char_p
    L.miqmm_version.argtypes, L.miqmm_version.restype = [], ctypes.c_char_p
    _lib = L
    return L


def _check(status: int) -> None:
    if status != OK:
        raise MiqmmError(status, lib().miqmm_last_error().decode())


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _dt(t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise MiqmmError(ENOTSUP, f"dtype {t.dtype} not supported")
    return _DT[t.dtype]


def result_type(x_dtype: torch.dtype, scale_dtype: torch.dtype) -> torch.dtype:
    """MLX type promotion of (x, scales, biases): equal dtypes are kept, and
    bfloat16 with float16 (or anything with float32) promotes to float32."""
    if x_dtype == scale_dtype:
        return x_dtype
    return torch.float32


def _check_weights(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int,
                   bits: int):
    if w.dim() != 2 or scales.dim() != 2 or biases.shape != scales.shape:
        raise MiqmmError(EINVAL, f"w {tuple(w.shape)} and scales/biases {tuple(scales.shape)}/"
                                 f"{tuple(biases.shape)} must be 2-D with equal scales/biases shapes")
    if w.dtype not in (torch.int32, torch.uint32):
        raise MiqmmError(EINVAL, f"w must hold uint32 words (int32/uint32 tensor), got {w.dtype}")
    if bits not in (4, 8):
        raise MiqmmError(ENOTSUP if bits in (2, 3, 5, 6) else EINVAL, f"bits={bits} not provided")
    N = w.shape[0]
    K = w.shape[1] * 32 // bits
    if scales.shape != (N, K // max(group_size, 1)):
        raise MiqmmError(EINVAL, f"scales shape {tuple(scales.shape)} != ({N}, {K}/{group_size})")
    for t in (w, scales, biases):
        if not t.is_contiguous():
            raise MiqmmError(EINVAL, "w, scales and biases must be contiguous")
    return N, K


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     transpose: bool = True, group_size: int = 64, bits: int = 4, *,
                     out: Optional[torch.Tensor] = None, route: int = ROUTE_AUTO,
                     stream=None, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[..., N] = x[..., K] @ dequant(w, scales, biases).T  (transpose=True)

    Argument order and meaning follow mlx_rs::ops::quantized_matmul
    (src/engine/mlx_lm/utils/mod.rs:70-78).  x's leading dims are flattened into M.
    The output dtype is MLX's result type of (x, scales, biases)."""
    N, K = _check_weights(w, scales, biases, group_size, bits)
    if x.shape[-1] != K:
        raise MiqmmError(EINVAL, f"x inner dim {x.shape[-1]} != K={K} implied by w {tuple(w.shape)}")
    xc = x.contiguous()
    M = xc.numel() // K
    ydt = result_type(x.dtype, scales.dtype)
    shape = tuple(x.shape[:-1]) + (N,)
    if out is None:
        out = torch.empty(shape, dtype=ydt, device=x.device)
    elif out.shape != shape or not out.is_contiguous():
        raise MiqmmError(EINVAL, f"out must be contiguous with shape {shape}")
    if bias is not None:
        if bias.shape != (N,) or bias.dtype != out.dtype:
            raise MiqmmError(EINVAL, f"bias must be [{N}] of dtype {out.dtype}")
        bias = bias.contiguous()
        if route != ROUTE_AUTO and route != query_route(M, N, K, group_size, bits)[0]:
            raise MiqmmError(EINVAL, "a bias takes the automatic route (a forced route only where it is that one)")
        route = ROUTE_AUTO
    if route == ROUTE_AUTO:
        # the tiled matmul's k split needs scratch for its fp32 partials: taken
        # from torch's caching allocator per call (stream-ordered, and from the
        # graph's own pool under capture), so calls never share it
        ws = workspace_size(M, N, K, group_size, bits)
        wt = torch.empty(ws, dtype=torch.uint8, device=x.device) if ws > 0 else None
        _check(lib().miqmm_quantized_matmul_ws(_ptr(out), _ptr(xc), _ptr(w), _ptr(scales), _ptr(biases),
                                               _ptr(bias), M, N, K, int(bool(transpose)), group_size, bits,
                                               _dt(xc), _dt(scales), _dt(out), _ptr(wt), ws, _stream(stream)))
        return out
    _check(lib().miqmm_quantized_matmul_ex(_ptr(out), _ptr(xc), _ptr(w), _ptr(scales), _ptr(biases), M, N,
                                           K, int(bool(transpose)), group_size, bits, _dt(xc), _dt(scales),
                                           _dt(out), route, _stream(stream)))
    return out


def stream_read(buf: torch.Tensor, sink: torch.Tensor, stream=None) -> None:
    """a plain streaming read of buf (bandwidth ceiling probe; nothing written)"""
    _check(lib().miqmm_stream_read(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink), _stream(stream)))


def workspace_size(M: int, N: int, K: int, group_size: int = 64, bits: int = 4) -> int:
    """bytes of scratch the automatic route's k split takes for this shape (0: none)"""
    n = ctypes.c_int64(0)
    _check(lib().miqmm_quantized_matmul_workspace_size(M, N, K, group_size, bits, ctypes.byref(n)))
    return n.value


def quantized_matmul_grouped(xs, ws, scales, biases, group_size: int = 64, bits: int = 4, *,
                             outs=None, bias=None, stream=None):
    """[quantized_matmul(xs[i], ws[i], scales[i], biases[i]) (+ bias[i])] as one
    launch per four projections where the route allows (decode, M <= 2).  The
    projections share M, K, group size, bits and dtypes -- the reference's
    q/k/v (src/engine/mlx_lm/models/llama.rs:195-197) and gate/up (:293-294)."""
    n = len(ws)
    if not (len(xs) == len(scales) == len(biases) == n):
        raise MiqmmError(EINVAL, "xs, ws, scales and biases must have the same length")
    if n == 0:
        return []
    bias = list(bias) if bias is not None else [None] * n
    outs = list(outs) if outs is not None else [None] * n
    probs = (Problem * n)()
    keep = []
    M = K = None
    for i in range(n):
        N, Ki = _check_weights(ws[i], scales[i], biases[i], group_size, bits)
        x = xs[i]
        if x.shape[-1] != Ki:
            raise MiqmmError(EINVAL, f"x[{i}] inner dim {x.shape[-1]} != K={Ki}")
        xc = x.contiguous()
        Mi = xc.numel() // Ki
        if M is None:
            M, K = Mi, Ki
        elif (Mi, Ki) != (M, K) or scales[i].dtype != scales[0].dtype or xs[i].dtype != xs[0].dtype:
            raise MiqmmError(EINVAL, "grouped projections must share M, K and dtypes")
        shape = tuple(x.shape[:-1]) + (N,)
        ydt = result_type(x.dtype, scales[i].dtype)
        if outs[i] is None:
            outs[i] = torch.empty(shape, dtype=ydt, device=x.device)
        elif outs[i].shape != shape or not outs[i].is_contiguous() or outs[i].dtype != ydt:
            raise MiqmmError(EINVAL, f"outs[{i}] must be contiguous {shape} of {ydt}")
        b = bias[i]
        if b is not None:
            if b.shape != (N,) or b.dtype != ydt:
                raise MiqmmError(EINVAL, f"bias[{i}] must be [{N}] of dtype {ydt}")
            b = b.contiguous()
        keep += [xc, b]
        probs[i] = Problem(outs[i].data_ptr(), xc.data_ptr(), ws[i].data_ptr(), scales[i].data_ptr(),
                           biases[i].data_ptr(), None if b is None else b.data_ptr(), N)
    _check(lib().miqmm_quantized_matmul_grouped(probs, n, M, K, group_size, bits, _dt(xs[0].contiguous()),
                                                _dt(scales[0]), _dt(outs[0]), _stream(stream)))
    return outs


# selections per expert (on average) from which gather_qmm groups them by
# expert (api.cpp): on the tiled MFMA matmul from 8, on the MFMA GEMV from 4
GROUPED_MIN_PER_EXPERT = 8
GROUPED_GEMV_MIN_PER_EXPERT = 4


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               rhs_indices: torch.Tensor, transpose: bool = True, group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False, *, out: Optional[torch.Tensor] = None,
               stream=None, grouped: Optional[bool] = None) -> torch.Tensor:
    """out[b] = x[b] @ dequant(w[rhs_indices[b]]).T over the broadcast batch b.

    Argument order and meaning follow the reference's gather_qmm wrapper
    (src/engine/mlx_lm/utils/moe.rs:33-43; lhs_indices absent): w is the
    stacked experts [E, N, K*bits/32], scales/biases [E, N, K/group_size],
    x [..., M, K] whose batch dims broadcast against rhs_indices [...];
    the result is [*broadcast, M, N].  An index outside [0, E) gives zero rows.
    sorted_indices is a hint that changes nothing here.  With M == 1 and many
    selections per expert (grouped=None: the library decides; True/False:
    pass or withhold the workspace) the selections are grouped by expert and
    each expert's weights are read once (miqmm_gather_qmm_ws)."""
    if w.dim() != 3 or scales.dim() != 3 or biases.shape != scales.shape or scales.shape[0] != w.shape[0]:
        raise MiqmmError(EINVAL, f"w {tuple(w.shape)} and scales/biases {tuple(scales.shape)}/"
                                 f"{tuple(biases.shape)} must be stacked [E, N, ...] with equal shapes")
    E = w.shape[0]
    if E == 0:
        raise MiqmmError(EINVAL, "w holds no experts")
    N, K = _check_weights(w[0], scales[0], biases[0], group_size, bits)
    if x.dim() < 2 or x.shape[-1] != K:
        raise MiqmmError(EINVAL, f"x {tuple(x.shape)} must be [..., M, {K}]")
    if rhs_indices.dtype.is_floating_point or rhs_indices.dtype == torch.bool:
        raise MiqmmError(EINVAL, f"rhs_indices must hold integers, got {rhs_indices.dtype}")
    M = x.shape[-2]
    try:
        bshape = tuple(torch.broadcast_shapes(tuple(x.shape[:-2]), tuple(rhs_indices.shape)))
    except RuntimeError as e:
        raise MiqmmError(EINVAL, f"x batch {tuple(x.shape[:-2])} does not broadcast against "
                                 f"rhs_indices {tuple(rhs_indices.shape)}") from e
    idx = rhs_indices.expand(bshape).to(torch.int32).contiguous()
    # x shared by a trailing block of the batch (x [..., 1, 1, M, K] against
    # indices [..., top_k]) is passed once per leading batch entry; any other
    # broadcast is materialised, one x matrix per selection
    xb = (1,) * (len(bshape) - (x.dim() - 2)) + tuple(x.shape[:-2])
    j = len(bshape)
    while j > 0 and xb[j - 1] == 1:
        j -= 1
    if xb[:j] == bshape[:j]:
        batch = math.prod(bshape[:j])
        top_k = math.prod(bshape[j:])
        xc = x.contiguous()
        per_index = 0
    else:
        batch, top_k = math.prod(bshape), 1
        xc = x.expand(bshape + (M, K)).contiguous()
        per_index = 1
    if top_k == 1:
        per_index = 1
    ydt = result_type(x.dtype, scales.dtype)
    shape = bshape + (M, N)
    if out is None:
        out = torch.empty(shape, dtype=ydt, device=x.device)
    elif out.shape != shape or not out.is_contiguous() or out.dtype != ydt:
        raise MiqmmError(EINVAL, f"out must be contiguous {shape} of {ydt}")
    ws, ws_bytes = None, 0
    if grouped is not False and M == 1 and batch * top_k >= GROUPED_GEMV_MIN_PER_EXPERT * E:
        nb = ctypes.c_int64()
        _check(lib().miqmm_gather_qmm_workspace_size(batch, top_k, E, ctypes.byref(nb)))
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=x.device)
        ws_bytes = nb.value
    _check(lib().miqmm_gather_qmm_ws(_ptr(out), _ptr(xc), _ptr(w), _ptr(scales), _ptr(biases), _ptr(idx), batch,
                                     top_k, per_index, M, N, K, E, int(bool(transpose)), group_size, bits, _dt(xc),
                                     _dt(scales), _dt(out), int(bool(sorted_indices)), _ptr(ws), ws_bytes,
                                     _stream(stream)))
    return out


def quantized_embedding(ids: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                        group_size: int = 64, bits: int = 4, *, dtype: Optional[torch.dtype] = None,
                        out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """out[..., k] = dequantize(w[ids], scales[ids], biases[ids]): the lookup of a
    quantized embedding table as the reference restates it
    (src/engine/mlx_lm/models/bonsai_q1.rs:603-613: take rows, then dequantize).
    The result is ids.shape + (K,) in `dtype` (default: the scales' dtype, as
    MLX's dequantize returns); an id outside [0, V) gives a zero row."""
    V, K = _check_weights(w, scales, biases, group_size, bits)
    if ids.dtype.is_floating_point or ids.dtype == torch.bool:
        raise MiqmmError(EINVAL, f"ids must hold integers, got {ids.dtype}")
    idc = ids.to(torch.int32).contiguous()
    dt = dtype or scales.dtype
    shape = tuple(ids.shape) + (K,)
    if out is None:
        out = torch.empty(shape, dtype=dt, device=w.device)
    elif out.shape != shape or not out.is_contiguous() or out.dtype != dt:
        raise MiqmmError(EINVAL, f"out must be contiguous {shape} of {dt}")
    _check(lib().miqmm_quantized_embedding(_ptr(out), _ptr(idc), idc.numel(), _ptr(w), _ptr(scales), _ptr(biases),
                                           V, K, group_size, bits, _dt(scales), _dt(out), _stream(stream)))
    return out


class QuantizedEmbedding:
    """mlx-rs QuantizedEmbedding: `forward(ids)` looks rows up (the step before
    the first projection of each token), `as_linear(x)` is the tied lm_head,
    quantized_matmul(x, weight, scales, biases) (src/engine/mlx_lm/models/llama.rs:511-517)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = 64, bits: int = 4):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits
        _check_weights(weight, scales, biases, group_size, bits)

    def __call__(self, ids: torch.Tensor, **kw) -> torch.Tensor:
        return self.forward(ids, **kw)

    def forward(self, ids: torch.Tensor, **kw) -> torch.Tensor:
        return quantized_embedding(ids, self.weight, self.scales, self.biases, self.group_size, self.bits, **kw)

    def as_linear(self, x: torch.Tensor, **kw) -> torch.Tensor:
        return quantized_matmul(x, self.weight, self.scales, self.biases, True, self.group_size, self.bits, **kw)


def quantized_linear(x, w, scales, biases, bias=None, group_size: int = 64, bits: int = 4, **kw):
    """QuantizedLinear forward: quantized_matmul, then + bias (two roundings, as two MLX ops)"""
    return quantized_matmul(x, w, scales, biases, True, group_size, bits, bias=bias, **kw)


class QuantizedLinear:
    """nn::QuantizedLinear: the swap-in slot of MaybeQuantized<Linear>
    (src/engine/mlx_lm/models/llama.rs:115-126).  Holds the packed weight
    [out, in*bits/32], scales/biases [out, in/group_size] and an optional
    bias [out]; calling it runs quantized_matmul (+ bias)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, group_size: int = 64, bits: int = 4):
        self.out_features, self.in_features = _check_weights(weight, scales, biases, group_size, bits)
        self.weight, self.scales, self.biases, self.bias = weight, scales, biases, bias
        self.group_size, self.bits = group_size, bits

    def __call__(self, x: torch.Tensor, **kw) -> torch.Tensor:
        return self.forward(x, **kw)

    def forward(self, x: torch.Tensor, **kw) -> torch.Tensor:
        return quantized_matmul(x, self.weight, self.scales, self.biases, True, self.group_size,
                                self.bits, bias=self.bias, **kw)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = 64,
               bits: int = 4, dtype: Optional[torch.dtype] = None, stream=None) -> torch.Tensor:
    """out[N, K] = scales * q + biases per group (mlx_rs::ops::dequantize)"""
    N, K = _check_weights(w, scales, biases, group_size, bits)
    out = torch.empty((N, K), dtype=dtype or scales.dtype, device=w.device)
    _check(lib().miqmm_dequantize(_ptr(out), _ptr(w), _ptr(scales), _ptr(biases), N, K, group_size, bits,
                                  _dt(scales), _dt(out), _stream(stream)))
    return out


def unpack(w: torch.Tensor, bits: int, stream=None) -> torch.Tensor:
    """codes[N, K] uint8 of packed words w[N, K*bits/32]"""
    N = w.shape[0]
    K = w.shape[1] * 32 // bits
    out = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    _check(lib().miqmm_unpack(_ptr(out), _ptr(w.contiguous()), N, K, bits, _stream(stream)))
    return out


def synth_problem(M: int, N: int, K: int, group_size: int = 64, bits: int = 4,
                  x_dtype: torch.dtype = torch.bfloat16, sb_dtype: torch.dtype = torch.bfloat16,
                  seed: int = 0, stream_id: int = 0, device="cuda", with_x: bool = True,
                  stream=None):
    """seeded synthetic (x, w, scales, biases) generated on the device"""
    x = torch.empty((M, K), dtype=x_dtype, device=device) if with_x else None
    w = torch.empty((N, K * bits // 32), dtype=torch.int32, device=device)
    s = torch.empty((N, K // group_size), dtype=sb_dtype, device=device)
    b = torch.empty_like(s)
    _check(lib().miqmm_synth_problem(_ptr(x), _ptr(w), _ptr(s), _ptr(b), M, N, K, group_size, bits,
                                     _DT[x_dtype], _DT[sb_dtype], seed, stream_id, _stream(stream)))
    return x, w, s, b


def query_route(M: int, N: int, K: int, group_size: int = 64, bits: int = 4):
    """(route, tile info) the dispatcher picks; host only"""
    route = ctypes.c_int(0)
    tiles = (ctypes.c_int * 4)()
    _check(lib().miqmm_query_route(M, N, K, group_size, bits, ctypes.byref(route), tiles))
    return route.value, tuple(tiles)


def version() -> str:
    return lib().miqmm_version().decode()
