"""CPU tests of the checkpoint reader (include/miqmm_checkpoint.h).

Synthetic model directories are written with the safetensors library itself
(the format MLX saves: U32 packed codes, BF16/F16 scales and biases), from the
oracle's seeded generator, so the reader is held to that library's layout.
The quantization rules restated here follow src/engine/mlx_lm/models/gemma4.rs:
1755-1834 (default + per-module overrides, ".scales" marks a quantized
module) and src/engine/mlx_native.rs:3603-3623,3684-3703 (shards, index,
".inner.weight" spelling).
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O

st = pytest.importorskip("safetensors.torch")


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _u32(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).view(torch.uint32)


def _module(tensors, path, N, K, g, bits, seed, experts=0, bias=False, inner=False):
    E = max(experts, 1)
    ws, ss, bs = [], [], []
    for e in range(E):
        _, w, s, b = O.synth_problem(1, N, K, g, bits, seed=seed, stream=e)
        ws.append(w), ss.append(s), bs.append(b)
    w, s, b = (np.stack(a) if experts else a[0] for a in (ws, ss, bs))
    tensors[path + (".inner.weight" if inner else ".weight")] = _u32(w)
    tensors[path + ".scales"] = _bf16(s)
    tensors[path + ".biases"] = _bf16(b)
    if bias:
        tensors[path + ".bias"] = _bf16(O.f32_to_bf16(np.linspace(-1, 1, N).astype(np.float32)))
    return w, s, b


def make_model(d, quant, shards=2):
    os.makedirs(d, exist_ok=True)
    t = {}
    ref = {
        "model.embed_tokens": _module(t, "model.embed_tokens", 64, 128, 64, 4, 1),
        "model.layers.0.self_attn.q_proj": _module(t, "model.layers.0.self_attn.q_proj", 32, 128, 64, 4, 2,
                                                   bias=True),
        "model.layers.0.mlp.down_proj": _module(t, "model.layers.0.mlp.down_proj", 16, 256, 64, 8, 3, inner=True),
        "model.layers.0.mlp.switch_mlp.gate_proj": _module(t, "model.layers.0.mlp.switch_mlp.gate_proj", 16, 128,
                                                           64, 4, 4, experts=4),
    }
    t["model.norm.weight"] = torch.ones(128, dtype=torch.bfloat16)
    names = sorted(t)
    if shards == 1:
        st.save_file(t, os.path.join(d, "model.safetensors"), metadata={"format": "mlx"})
    else:
        wm = {}
        for i in range(shards):
            part = {n: t[n] for n in names[i::shards]}
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            st.save_file(part, os.path.join(d, fn), metadata={"format": "mlx"})
            wm.update({n: fn for n in part})
        json.dump({"metadata": {}, "weight_map": wm}, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    json.dump({"model_type": "llama", **quant}, open(os.path.join(d, "config.json"), "w"))
    return t, ref


QUANT = {"quantization": {"group_size": 64, "bits": 4,
                          "model.layers.0.mlp.down_proj": {"bits": 8}}}


@pytest.mark.parametrize("shards", [1, 2, 3])
def test_plan_and_bytes(tmp_path, shards):
    from miqmm.checkpoint import Checkpoint

    t, ref = make_model(str(tmp_path), QUANT, shards)
    with Checkpoint(str(tmp_path)) as c:
        mods = c.modules()
        assert set(mods) == set(ref)
        q = mods["model.layers.0.self_attn.q_proj"]
        assert (q["bits"], q["group_size"], q["rows"], q["cols"], q["experts"]) == (4, 64, 32, 128, 0)
        assert q["bias"] == "model.layers.0.self_attn.q_proj.bias"
        d = mods["model.layers.0.mlp.down_proj"]
        assert (d["bits"], d["group_size"], d["rows"], d["cols"]) == (8, 64, 16, 256)
        assert d["weight"] == "model.layers.0.mlp.down_proj.inner.weight" and d["bias"] is None
        e = mods["model.layers.0.mlp.switch_mlp.gate_proj"]
        assert (e["experts"], e["rows"], e["cols"]) == (4, 16, 128)
        assert "model.norm.weight" in c.tensor_names() and "model.norm" not in mods
        for path, (w, s, b) in ref.items():
            m = mods[path]
            np.testing.assert_array_equal(c.read(m["weight"]), w)
            np.testing.assert_array_equal(c.read(m["scales"]), s)
            np.testing.assert_array_equal(c.read(m["biases"]), b)


def test_quantization_config_alias_and_defaults(tmp_path):
    from miqmm.checkpoint import Checkpoint

    q = {"quantization_config": dict(QUANT["quantization"])}
    make_model(str(tmp_path), q)
    with Checkpoint(str(tmp_path)) as c:
        assert c.modules()["model.layers.0.mlp.down_proj"]["bits"] == 8


def test_wrong_bits_is_a_load_error(tmp_path):
    """without the per-module override the 8-bit down_proj would be read as
    4-bit words: the shapes disagree and the open fails, naming the module.
    (A misdescription with the same bits * group_size product, e.g. 8-bit g32
    read as 4-bit g64, implies consistent shapes and cannot be caught here.)"""
    import miqmm
    from miqmm.checkpoint import Checkpoint

    make_model(str(tmp_path), {"quantization": {"group_size": 64, "bits": 4}})
    with pytest.raises(miqmm.MiqmmError, match="down_proj") as ei:
        Checkpoint(str(tmp_path))
    assert ei.value.status == miqmm.EINVAL


def test_mode_and_missing_tensors(tmp_path):
    import miqmm
    from miqmm.checkpoint import Checkpoint

    d1 = str(tmp_path / "mx")
    make_model(d1, {"quantization": {"group_size": 64, "bits": 4, "mode": "mxfp4"}})
    with pytest.raises(miqmm.MiqmmError, match="mode"):
        Checkpoint(d1)
    d2 = str(tmp_path / "nob")
    t, _ = make_model(d2, QUANT, shards=1)
    del t["model.embed_tokens.biases"]
    st.save_file(t, os.path.join(d2, "model.safetensors"), metadata={"format": "mlx"})
    with pytest.raises(miqmm.MiqmmError, match="biases"):
        Checkpoint(d2)


def test_malformed_shards(tmp_path):
    import miqmm
    from miqmm.checkpoint import Checkpoint

    d = str(tmp_path)
    make_model(d, QUANT, shards=1)
    p = os.path.join(d, "model.safetensors")
    raw = open(p, "rb").read()
    open(p, "wb").write(raw[:100])  # header cut short
    with pytest.raises(miqmm.MiqmmError):
        Checkpoint(d)
    os.remove(p)
    with pytest.raises(miqmm.MiqmmError, match="model.safetensors"):
        Checkpoint(d)
    open(os.path.join(d, "config.json"), "w").write("{not json")
    with pytest.raises(miqmm.MiqmmError, match="config.json"):
        Checkpoint(d)


def test_overflowing_shape_is_refused(tmp_path):
    """a shard whose shape product overflows int64 (2^32 x 2^32 wraps to 0)
    must not pass the byte-range check with an empty range"""
    import json
    import struct

    import miqmm
    from miqmm.checkpoint import Checkpoint

    d = str(tmp_path)
    make_model(d, QUANT, shards=1)
    p = os.path.join(d, "model.safetensors")
    hdr = {"model.norm.weight": {"dtype": "BF16", "shape": [1 << 32, 1 << 32], "data_offsets": [0, 0]}}
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    open(p, "wb").write(struct.pack("<Q", len(h)) + h)
    with pytest.raises(miqmm.MiqmmError, match="too large"):
        Checkpoint(d)
