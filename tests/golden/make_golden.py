"""Writes kat.json: known-answer vectors for the entropy-patching path.

Every expected value here comes from the reference's own tests or from
closed forms worked by hand, not from any implementation in this repository:
  - entropy of equal logits = ln V (tests/test_fused_entropy.rs:155-177,
    179-203), entropy of a one-hot-like row ~ 0;
  - byte tokens = byte + 4 (tests/test_blt_core.rs:38-51, tokenizer.rs:4-10);
  - patch-start masks, start indices and lengths for hand-worked entropy rows
    following patcher.rs:80-164, with f32 arithmetic: (H[t] - H[t-1]) > f32(thr).
    Case "f32_threshold" sits exactly on the threshold, where an f64 comparison
    would flip the answer; sum(lengths) = T (tests/test_blt_core.rs:124-126).
Run: python tests/golden/make_golden.py
"""
import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(xs):
    return [float(np.float32(x)) for x in xs]


KAT = {
    "entropy": [
        {"name": "zeros_v256", "shape": [2, 8, 256], "fill": 0.0, "expected": math.log(256),
         "tol": 1e-3, "source": "tests/test_fused_entropy.rs:155-177"},
        {"name": "const_neg100_v256", "shape": [1, 1, 256], "fill": -100.0,
         "expected": math.log(256), "tol": 1e-3,
         "source": "tests/test_fused_entropy.rs:179-203 (equal logits => uniform)"},
        {"name": "zeros_v260", "shape": [4, 3, 260], "fill": 0.0, "expected": math.log(260),
         "tol": 1e-3, "source": "closed form ln V"},
        {"name": "one_hot_v260", "shape": [1, 1, 260], "fill": -100.0, "hot": 100.0,
         "expected": 0.0, "tol": 1e-6, "source": "closed form: p0 = 1/(1 + 259 e^-200)"},
    ],
    "tokens": [
        {"text": "ABC", "tokens": [69, 70, 71], "source": "tests/test_blt_core.rs:38-51"},
        {"text": "Hello", "tokens": [76, 105, 112, 112, 115],
         "source": "tests/test_blt_core.rs:53-60"},
    ],
    "patch": [
        {"name": "monotonic_basic", "mode": "monotonic", "thr": 0.2,
         "H": [f32([5.0, 1.0, 1.3, 1.2, 1.5, 1.5, 2.0, 0.1, 0.35, 0.5])],
         "mask": [[1, 1, 1, 0, 1, 0, 1, 0, 1, 0]],
         "starts": [[0, 1, 2, 4, 6, 8]], "lengths": [[1, 1, 2, 2, 2, 2]]},
        {"name": "f32_threshold", "mode": "monotonic", "thr": 0.2,
         "H": [f32([0.0, 0.0, 0.2, 0.2, 0.4])],
         "mask": [[1, 1, 0, 0, 0]], "starts": [[0, 1]], "lengths": [[1, 4]]},
        {"name": "two_rows", "mode": "monotonic", "thr": 1.335,
         "H": [f32([3.0, 0.0, 1.4, 1.4, 3.0, 0.0]), f32([0.0, 0.0, 0.0, 0.0, 0.0, 2.0])],
         "mask": [[1, 1, 1, 0, 1, 0], [1, 1, 0, 0, 0, 1]],
         "starts": [[0, 1, 2, 4], [0, 1, 5]], "lengths": [[1, 1, 2, 2], [1, 4, 1]]},
        {"name": "seq_len_1", "mode": "monotonic", "thr": 0.2, "H": [[7.0], [0.0]],
         "mask": [[1], [1]], "starts": [[0], [0]], "lengths": [[1], [1]],
         "source": "patcher.rs:90-93"},
        {"name": "seq_len_2", "mode": "monotonic", "thr": 0.2, "H": [[0.0, 9.0]],
         "mask": [[1, 1]], "starts": [[0, 1]], "lengths": [[1, 1]], "source": "patcher.rs:95-98"},
        {"name": "seq_len_3_no_cut", "mode": "monotonic", "thr": 0.2, "H": [[1.0, 1.0, 1.0]],
         "mask": [[1, 1, 0]], "starts": [[0, 1]], "lengths": [[1, 2]]},
        {"name": "global_basic", "mode": "global", "thr": 1.33,
         "H": [f32([0.1, 0.2, 1.33, 1.34, 0.5, 2.0])],
         "mask": [[1, 1, 0, 1, 0, 1]], "starts": [[0, 1, 3, 5]], "lengths": [[1, 2, 2, 1]]},
    ],
}

if __name__ == "__main__":
    with open(os.path.join(HERE, "kat.json"), "w") as f:
        json.dump(KAT, f, indent=1)
    print("wrote", os.path.join(HERE, "kat.json"))
