"""Writes tests/golden/kat.json: the known-answer cases of the reference's own
tests, as data (inputs and expected outputs).

Sources (sahan974/DeepSeek-V2-Lite-CUDA):
  tests/test_moe_scan_kernel.py:64-76    random counts: np.random.seed(42); randint(0, 20, 64)
  tests/test_moe_scan_kernel.py:79-95    32 tokens * 6 / 64 = 3 per expert -> sentinel 192
  tests/test_moe_scan_kernel.py:98-112   all zeros
  tests/test_moe_scan_kernel.py:115-126  single expert [7]
  tests/test_moe_scan_kernel.py:129-145  uniform 5 per expert -> sentinel 320
  tests/test_moe_scan_kernel.py:148-164  skewed [192, 0, ..., 0]
  tests/test_moe_routing_kernel.py:155-173  all-zero logits (16 tokens) -> 6 distinct
      experts per token; with ties broken by the lower expert index the set is {0..5}
      and every weight is exactly 1/64.
Expected scan outputs are written out by hand from the closed form
(offsets[e] = sum of counts before e), not by the code under test.
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    np.random.seed(42)
    rnd = np.random.randint(0, 20, size=64).astype(np.int32).tolist()
    rnd_exp = [0]
    for c in rnd:
        rnd_exp.append(rnd_exp[-1] + c)
    kat = {
        "scan": [
            {"name": "random_seed42", "counts": rnd, "offsets": rnd_exp},
            {"name": "uniform3", "counts": [3] * 64, "offsets": [3 * i for i in range(65)]},
            {"name": "zeros", "counts": [0] * 64, "offsets": [0] * 65},
            {"name": "single", "counts": [7], "offsets": [0, 7]},
            {"name": "uniform5", "counts": [5] * 64, "offsets": [5 * i for i in range(65)]},
            {"name": "skewed", "counts": [192] + [0] * 63, "offsets": [0] + [192] * 64},
        ],
        "routing_all_zero": {
            "num_tokens": 16, "num_experts": 64, "top_k": 6,
            "topk_indices_row": [0, 1, 2, 3, 4, 5],
            "topk_weight": 1.0 / 64.0,
            "expert_counts": [16] * 6 + [0] * 58,
        },
    }
    with open(os.path.join(HERE, "kat.json"), "w") as f:
        json.dump(kat, f, indent=1)


if __name__ == "__main__":
    main()
