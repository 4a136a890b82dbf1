"""GPU test of loading a synthetic MLX quantized checkpoint into miqmm modules
and running them: the loaded codes are the written ones (unpack, bit for bit)
and each module's output meets the oracle (tests/test_checkpoint.py builds the
directory with the safetensors library, as MLX writes it)."""
import numpy as np
import pytest
import torch

import oracle as O
from test_checkpoint import QUANT, make_model
from test_gpu_parity import check, dev16, u16

pytestmark = pytest.mark.gpu


def test_load_and_run(gpu, c_oracle, tmp_path):
    import miqmm
    from miqmm.checkpoint import SwitchLinear, load_quantized

    _, ref = make_model(str(tmp_path), QUANT, shards=2)
    mods = load_quantized(str(tmp_path))
    # codes as written
    for path, (w, s, b) in ref.items():
        m = mods[path]
        bits = 8 if path.endswith("down_proj") else 4
        W = m.weight.reshape(-1, m.weight.shape[-1])
        K = W.shape[1] * 32 // bits
        codes = miqmm.unpack(W, bits).cpu().numpy()
        np.testing.assert_array_equal(codes, O.unpack(w.reshape(-1, w.shape[-1]), K, bits))
    # QuantizedLinear with bias (q_proj), 8-bit override (down_proj)
    for path, K, N, g, bits in [("model.layers.0.self_attn.q_proj", 128, 32, 64, 4),
                                ("model.layers.0.mlp.down_proj", 256, 16, 64, 8)]:
        w, s, b = ref[path]
        x, _, _, _ = O.synth_problem(3, 8, K, g, bits, seed=9)
        y = mods[path](dev16(x))
        want = O.qmm_f64(x, w, s, b, K, g, bits)
        if mods[path].bias is not None:
            bias = O.bf16_to_f32(u16(mods[path].bias)).astype(np.float64)
            want = O.bf16_to_f32(O.f32_to_bf16(want.astype(np.float32))).astype(np.float64) + bias
        check(y, want, True, path)
    # embedding, bit for bit
    w, s, b = ref["model.embed_tokens"]
    ids = np.array([[0, 63, 5], [5, 1, 2]])
    y = mods["model.embed_tokens"](torch.from_numpy(ids).cuda())
    np.testing.assert_array_equal(u16(y), O.embedding(ids, w, s, b, 128, 64, 4))
    # stacked experts through gather_qmm
    sw = mods["model.layers.0.mlp.switch_mlp.gate_proj"]
    assert isinstance(sw, SwitchLinear)
    w, s, b = ref["model.layers.0.mlp.switch_mlp.gate_proj"]
    x, _, _, _ = O.synth_problem(2, 8, 128, 64, 4, seed=10)
    idx = np.array([[3, 0], [1, 1]])
    y = sw(dev16(x).reshape(2, 1, 1, 128), torch.from_numpy(idx).cuda())
    check(y, O.gather_qmm_f64(x.reshape(2, 1, 1, 128), w, s, b, idx, 128, 64, 4), True, "switch")
