"""GPU tests of the quantized embedding lookup (miqmm_quantized_embedding).

The reference restates QuantizedEmbedding's lookup as take-rows-then-dequantize
(src/engine/mlx_lm/models/bonsai_q1.rs:603-613).  The kernel computes each
element as one fp32 fma rounded once to the output dtype, so it is held to the
oracle bit for bit; at the full Qwen2.5-0.5B table (151936 x 896) the selected
rows are compared bit for bit with miqmm_dequantize of the whole table.
"""
import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_parity import dev16, dev32, u16

pytestmark = pytest.mark.gpu


def _miqmm():
    import miqmm

    return miqmm


@pytest.mark.parametrize("V,K,g,bits,sbd", [(100, 256, 64, 4, O.BF16), (33, 96, 32, 4, O.F16),
                                            (50, 512, 128, 8, O.BF16), (9, 64, 32, 8, O.F16)])
@pytest.mark.parametrize("odt", [O.BF16, O.F16, O.F32])
def test_embedding_matches_oracle(gpu, c_oracle, V, K, g, bits, sbd, odt):
    m = _miqmm()
    _, w, s, b = c_oracle.c_synth_problem(1, V, K, g, bits, sb_dtype=sbd, seed=V, stream=5)
    sdt = torch.float16 if sbd == O.F16 else torch.bfloat16
    wd, sd, bd = dev32(w), dev16(s, sdt), dev16(b, sdt)
    rng = np.random.default_rng(V + K)
    ids = rng.integers(-2, V + 2, size=(3, 7))  # repeats and out-of-range ids
    tdt = {O.BF16: torch.bfloat16, O.F16: torch.float16, O.F32: torch.float32}[odt]
    y = m.quantized_embedding(torch.from_numpy(ids).cuda(), wd, sd, bd, g, bits, dtype=tdt)
    assert y.shape == (3, 7, K) and y.dtype == tdt
    want = O.embedding(ids, w, s, b, K, g, bits, sb_dtype=sbd, out_dtype=odt)
    got = y.cpu().numpy() if odt == O.F32 else u16(y)
    np.testing.assert_array_equal(got, want)


def test_embedding_qwen_table_equals_dequantize(gpu):
    m = _miqmm()
    V, K, g, bits = 151936, 896, 64, 4
    _, w, s, b = m.synth_problem(1, V, K, g, bits, seed=0, stream_id=11)
    full = m.dequantize(w, s, b, g, bits)
    ids = torch.tensor([0, 151935, 42, 42, 100000, 7], dtype=torch.int64, device="cuda")
    emb = m.QuantizedEmbedding(w, s, b, g, bits)
    y = emb(ids)
    assert torch.equal(y, full[ids])
    # the tied head of the same table
    x = m.synth_problem(2, 8, K, g, bits, seed=3, stream_id=12)[0]
    assert torch.equal(emb.as_linear(x), m.quantized_matmul(x, w, s, b, True, g, bits))


def test_embedding_empty_and_errors(gpu):
    m = _miqmm()
    _, w, s, b = m.synth_problem(1, 16, 128, 64, 4, seed=1, stream_id=1)
    y = m.quantized_embedding(torch.zeros((0, 3), dtype=torch.int32, device="cuda"), w, s, b)
    assert y.shape == (0, 3, 128)
    with pytest.raises(m.MiqmmError):
        m.quantized_embedding(torch.zeros(2, device="cuda"), w, s, b)
