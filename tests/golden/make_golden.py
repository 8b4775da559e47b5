"""Write tests/golden/attn_golden.npz: small seeded attention cases.

Each case stores fp16 q/k/v, the scale and the float64 output of
oracle.attention.attention_fp64. The reference ships no golden vectors for
this path (its tests draw random inputs at run time, test.py:5-9), so these
fixtures pin the oracle and the kernel to fixed inputs across rounds. Shapes
cover every accepted head-dim class, odd Sq != Skv as in the reference's CPU
model check (model_check.py:143-145: 37 x 83) and variant harness
(test_variants.py:78-80: 100 x 300, 77 x 411), a single key, and negative and
zero scales.

Run: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.attention import attention_fp64, make_inputs  # noqa: E402

CASES = [
    # name, B, H, Sq, Skv, D, qk_mult, v_mult, scale, seed
    ("d64_37x83", 1, 2, 37, 83, 64, 1.0, 1.0, 0.125, 1),
    ("d128_37x83", 1, 1, 37, 83, 128, 1.0, 1.0, 0.125, 2),
    ("d128_77x411", 1, 1, 77, 411, 128, 1.0, 1.0, 128 ** -0.5, 3),
    ("d64_100x300", 1, 1, 100, 300, 64, 1.0, 1.0, 0.125, 4),
    ("d512_17x40", 1, 1, 17, 40, 512, 0.5, 0.5, 512 ** -0.5, 5),
    ("d32_64x64", 2, 1, 64, 64, 32, 1.0, 1.0, 0.125, 6),
    ("d16_50x130", 1, 1, 50, 130, 16, 1.0, 1.0, 0.125, 7),
    ("d8_20x20", 1, 1, 20, 20, 8, 1.0, 1.0, 8 ** -0.5, 8),
    ("d64_sharp_64x96", 1, 1, 64, 96, 64, 2.0, 1.0, 0.125, 9),
    ("d128_skv1", 1, 1, 10, 1, 128, 1.0, 1.0, 0.1, 10),
    ("d64_negscale", 1, 1, 40, 90, 64, 1.0, 1.0, -0.125, 11),
    ("d64_zeroscale", 1, 1, 16, 33, 64, 1.0, 1.0, 0.0, 12),
]


def main():
    arrays = {}
    for name, B, H, Sq, Skv, D, qm, vm, scale, seed in CASES:
        q, k, v = make_inputs(B, H, Sq, Skv, D, qm, vm, seed)
        arrays[f"{name}/q"] = q.numpy()
        arrays[f"{name}/k"] = k.numpy()
        arrays[f"{name}/v"] = v.numpy()
        arrays[f"{name}/scale"] = np.float64(scale)
        arrays[f"{name}/o"] = attention_fp64(q, k, v, scale)
    path = os.path.join(HERE, "attn_golden.npz")
    np.savez_compressed(path, **arrays)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
