"""Write tests/golden/golden.npz: regression vectors for the oracle.

    python tests/golden/make_golden.py

The reference (SenClaw/sen-mlx) holds no golden outputs for quantized matmul
(its only test of the op family, src/engine/mlx_lm/utils/moe.rs:84-146, is a
self-consistency check on the Metal device), and MLX is not importable here,
so these vectors come from this repo's oracle: the C generator and the exact
float64 accumulation.  They pin the oracle against silent drift; the
mathematical checks in tests/test_oracle.py pin it against the algorithm.
Inputs are not stored: they are regenerated from (seed, stream) and the
generator itself is pinned by the stored draws.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

# (bits, group_size, sb_dtype) small cases: M=3, N=40, K=256, seed 5, stream = index
SMALL = [(4, 32, O.BF16), (4, 64, O.BF16), (4, 128, O.BF16), (8, 64, O.BF16),
         (8, 32, O.F16), (4, 32, O.F16), (8, 128, O.F16)]


def main():
    O.build_c_oracle()
    out = {}
    k = O.c_oracle().orc_key(0, 9)
    out["draws_seed0_tag9"] = np.array([O.c_oracle().orc_draw(k, i) for i in range(16)], np.uint64)
    out["normal_seed0_tag9"] = np.array([O.c_oracle().orc_normal(int(d)) for d in out["draws_seed0_tag9"]],
                                        np.float32)
    # configuration 0: M=1, N=4864, K=896, 4-bit g64, bf16, seed 0
    x, w, s, b = O.c_synth_problem(1, 4864, 896, 64, 4, seed=0, stream=0)
    y64 = O.c_qmm_f64(x, w, s, b, 1, 4864, 896, 64, 4)
    out["cfg0_y64"] = y64
    out["cfg0_words_head"] = w[:2, :4].copy()
    out["cfg0_scales_head"] = s[:2, :4].copy()
    out["cfg0_biases_head"] = b[:2, :4].copy()
    out["cfg0_x_head"] = x[0, :16].copy()
    for i, (bits, g, sbd) in enumerate(SMALL):
        x, w, s, b = O.c_synth_problem(3, 40, 256, g, bits, sb_dtype=sbd, seed=5, stream=i)
        out[f"small{i}_y64"] = O.c_qmm_f64(x, w, s, b, 3, 40, 256, g, bits, sb_dtype=sbd)
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
