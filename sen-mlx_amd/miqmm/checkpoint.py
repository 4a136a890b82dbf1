"""Loading MLX quantized checkpoints into miqmm modules.

Host-side mirror of include/miqmm_checkpoint.h (the plan and the shard reads
are done by libmiqmm.so's C++ code).  `load_quantized(model_dir)` replaces the
quantized half of the reference's per-model loaders (e.g. load_llama_any,
src/engine/mlx_native.rs:3585-3760): every module stored with a ".scales"
tensor becomes a QuantizedLinear (2-D weight), QuantizedEmbedding (a module
named "...embed_tokens") or SwitchLinear (3-D stacked experts, the
switch_mlp / switch_glu tensors of src/engine/mlx_lm/models/deepseek_v2.rs:
397-445), with bits and group size from config.json's quantization section
and its per-module overrides (src/engine/mlx_lm/models/gemma4.rs:1755-1834).
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional

import numpy as np
import torch

from . import (EINVAL, MiqmmError, QuantizedEmbedding, QuantizedLinear, gather_qmm, lib)

_NP = {"U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16, "F16": np.float16, "BF16": np.uint16,
       "U32": np.uint32, "I32": np.int32, "F32": np.float32, "U64": np.uint64, "I64": np.int64, "F64": np.float64}
_TORCH_VIEW = {"BF16": torch.bfloat16, "U32": torch.int32}


class QModule(ctypes.Structure):
    """miqmm_qmodule"""
    _fields_ = [("path", ctypes.c_char_p), ("weight", ctypes.c_char_p), ("scales", ctypes.c_char_p),
                ("biases", ctypes.c_char_p), ("bias", ctypes.c_char_p), ("bits", ctypes.c_int),
                ("group_size", ctypes.c_int), ("sb_dtype", ctypes.c_int), ("experts", ctypes.c_int64),
                ("rows", ctypes.c_int64), ("cols", ctypes.c_int64)]


class TensorInfo(ctypes.Structure):
    """miqmm_tensor_info"""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("file", ctypes.c_char_p),
                ("ndim", ctypes.c_int), ("shape", ctypes.c_int64 * 8), ("offset", ctypes.c_int64),
                ("nbytes", ctypes.c_int64)]


def _api():
    L = lib()
    if not getattr(L, "_ckpt_bound", False):
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.miqmm_checkpoint_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(P)]
        L.miqmm_checkpoint_close.argtypes, L.miqmm_checkpoint_close.restype = [P], None
        L.miqmm_checkpoint_num_modules.argtypes, L.miqmm_checkpoint_num_modules.restype = [P], I64
        L.miqmm_checkpoint_num_tensors.argtypes, L.miqmm_checkpoint_num_tensors.restype = [P], I64
        L.miqmm_checkpoint_module.argtypes = [P, I64, ctypes.POINTER(QModule)]
        L.miqmm_checkpoint_tensor.argtypes = [P, ctypes.c_char_p, I64, ctypes.POINTER(TensorInfo)]
        L.miqmm_checkpoint_read.argtypes = [P, ctypes.c_char_p, P, I64]
        L.miqmm_checkpoint_last_error.argtypes, L.miqmm_checkpoint_last_error.restype = [], ctypes.c_char_p
        L._ckpt_bound = True
    return L


def _check(status: int) -> None:
    if status != 0:
        raise MiqmmError(status, _api().miqmm_checkpoint_last_error().decode())


class Checkpoint:
    """An opened model directory: its quantized modules and tensor index."""

    def __init__(self, model_dir: str):
        self._h = ctypes.c_void_p()
        _check(_api().miqmm_checkpoint_open(str(model_dir).encode(), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            _api().miqmm_checkpoint_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def modules(self) -> Dict[str, dict]:
        """path -> {weight, scales, biases, bias, bits, group_size, sb_dtype, experts, rows, cols}"""
        L = _api()
        out = {}
        for i in range(L.miqmm_checkpoint_num_modules(self._h)):
            m = QModule()
            _check(L.miqmm_checkpoint_module(self._h, i, ctypes.byref(m)))
            out[m.path.decode()] = {
                "weight": m.weight.decode(), "scales": m.scales.decode(), "biases": m.biases.decode(),
                "bias": m.bias.decode() if m.bias else None, "bits": m.bits, "group_size": m.group_size,
                "sb_dtype": m.sb_dtype, "experts": m.experts, "rows": m.rows, "cols": m.cols}
        return out

    def tensor(self, name: str) -> dict:
        t = TensorInfo()
        _check(_api().miqmm_checkpoint_tensor(self._h, name.encode(), 0, ctypes.byref(t)))
        return {"name": t.name.decode(), "dtype": t.dtype.decode(), "file": t.file.decode(),
                "shape": tuple(t.shape[i] for i in range(t.ndim)), "offset": t.offset, "nbytes": t.nbytes}

    def tensor_names(self):
        L = _api()
        names = []
        for i in range(L.miqmm_checkpoint_num_tensors(self._h)):
            t = TensorInfo()
            _check(L.miqmm_checkpoint_tensor(self._h, None, i, ctypes.byref(t)))
            names.append(t.name.decode())
        return names

    def read(self, name: str) -> np.ndarray:
        """the tensor's bytes as a numpy array (BF16 as uint16 bit patterns)"""
        info = self.tensor(name)
        if info["dtype"] not in _NP:
            raise MiqmmError(EINVAL, f"tensor {name}: dtype {info['dtype']} not readable here")
        arr = np.empty(info["shape"], dtype=_NP[info["dtype"]])
        _check(_api().miqmm_checkpoint_read(self._h, name.encode(), arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))
        return arr

    def to_device(self, name: str, device="cuda") -> torch.Tensor:
        """the tensor on `device` in its torch dtype (U32 codes as int32 words)"""
        info = self.tensor(name)
        arr = self.read(name)
        t = torch.from_numpy(arr.view(np.int32) if info["dtype"] == "U32" else arr)
        if info["dtype"] == "BF16":
            t = t.view(torch.bfloat16)
        return t.pin_memory().to(device, non_blocking=False) if device != "cpu" else t


class SwitchLinear:
    """Stacked quantized experts [E, N, K*bits/32] (the switch_mlp tensors of
    src/engine/mlx_lm/models/deepseek_v2.rs:397-445): forward(x, indices) is
    gather_qmm(x, weight, scales, biases, indices)."""

    def __init__(self, weight, scales, biases, group_size: int = 64, bits: int = 4):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits

    def __call__(self, x, indices, **kw):
        return self.forward(x, indices, **kw)

    def forward(self, x, indices, **kw):
        return gather_qmm(x, self.weight, self.scales, self.biases, indices, True, self.group_size, self.bits,
                          False, **kw)


def load_quantized(model_dir: str, device="cuda", ckpt: Optional[Checkpoint] = None):
    """{module path: QuantizedLinear | QuantizedEmbedding | SwitchLinear} for
    every quantized module of the checkpoint, its tensors on `device`."""
    own = ckpt is None
    ckpt = ckpt or Checkpoint(model_dir)
    try:
        out = {}
        for path, m in ckpt.modules().items():
            w = ckpt.to_device(m["weight"], device)
            s = ckpt.to_device(m["scales"], device)
            b = ckpt.to_device(m["biases"], device)
            g, bits = m["group_size"], m["bits"]
            if m["experts"]:
                out[path] = SwitchLinear(w, s, b, g, bits)
            elif path.endswith("embed_tokens"):
                out[path] = QuantizedEmbedding(w, s, b, g, bits)
            else:
                bias = ckpt.to_device(m["bias"], device) if m["bias"] else None
                out[path] = QuantizedLinear(w, s, b, bias, g, bits)
        return out
    finally:
        if own:
            ckpt.close()
