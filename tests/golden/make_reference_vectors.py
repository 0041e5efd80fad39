"""Write ``reference_vectors.json``: known-answer vectors held by the reference's tests.

Every case is data copied from an assertion of the reference test suite (file:line
below). Expected outputs that the reference states as a formula over literal inputs
(e.g. ``F.softmax(tensor([28., 32., 60., 64.]))``) are evaluated here with the same
library routine and stored as numbers. No reference code is imported or run.

Run: ``python tests/golden/make_reference_vectors.py``.
"""
from __future__ import annotations

import json
import math
from pathlib import Path


def _softmax(xs: list[float]) -> list[float]:
    m = max(xs)
    e = [math.exp(x - m) for x in xs]
    s = sum(e)
    return [v / s for v in e]


def build() -> dict:
    cases = {}
    # tests/unit/test_numerical_correctness.py:40-66 — [1,1,8,4] arange(1..32), block 4.
    cases["pool_block4"] = {
        "source": "tests/unit/test_numerical_correctness.py:40-66",
        "block_size": 4,
        "x": [[[[float(r * 4 + c + 1) for c in range(4)] for r in range(8)]]],
        "expected": [[[[7.0, 8.0, 9.0, 10.0], [23.0, 24.0, 25.0, 26.0]]]],
    }
    # tests/unit/test_numerical_correctness.py:68-81 — ones [1,1,6,2], block 4, pad zeros.
    cases["pool_padding"] = {
        "source": "tests/unit/test_numerical_correctness.py:68-81",
        "block_size": 4,
        "x": [[[[1.0, 1.0] for _ in range(6)]]],
        "expected": [[[[1.0, 1.0], [0.5, 0.5]]]],
    }
    # tests/unit/test_numerical_correctness.py:83-98 — single block mean.
    cases["pool_single_block"] = {
        "source": "tests/unit/test_numerical_correctness.py:83-98",
        "block_size": 4,
        "x": [[[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0], [7.0, 8.0, 9.0], [10.0, 11.0, 12.0]]] * 2],
        "expected": [[[[5.5, 6.5, 7.5]], [[5.5, 6.5, 7.5]]]],
    }
    # tests/unit/test_objectives.py:169-191 — 4x4 arange(1..16), block 2 -> softmax([6,8,14,16]).
    cases["gate_target_4x4"] = {
        "source": "tests/unit/test_objectives.py:169-191",
        "block_size": 2,
        "scores": [[[[float(r * 4 + c + 1) for c in range(4)] for r in range(4)]]],
        "pooled": [6.0, 8.0, 14.0, 16.0],
        "expected": [[[[v for v in _softmax([6.0, 8.0, 14.0, 16.0])[0:2]],
                       [v for v in _softmax([6.0, 8.0, 14.0, 16.0])[2:4]]]]],
    }
    # tests/unit/test_numerical_correctness.py:119-157 — 8x8 arange(1..64), block 4.
    sm = _softmax([28.0, 32.0, 60.0, 64.0])
    cases["gate_target_8x8"] = {
        "source": "tests/unit/test_numerical_correctness.py:119-157",
        "block_size": 4,
        "scores": [[[[float(r * 8 + c + 1) for c in range(8)] for r in range(8)]]],
        "pooled": [28.0, 32.0, 60.0, 64.0],
        "expected": [[[sm[0:2], sm[2:4]]]],
    }
    # tests/unit/test_objectives.py:714-721 — all scores 5.0, block 4 -> uniform 0.25.
    cases["gate_target_uniform"] = {
        "source": "tests/unit/test_objectives.py:714-721",
        "block_size": 4,
        "scores": [[[[5.0] * 8 for _ in range(8)]]],
        "expected": [[[[0.25, 0.25], [0.25, 0.25]]]],
    }
    # tests/unit/test_kernel.py:66-78, :144-173 — speedup model and full-grid stats.
    cases["speedup"] = {
        "source": "tests/unit/test_kernel.py:66-78",
        "points": [[0.0, 1.0], [0.5, 1.0 / (1.0 - 0.5 * 0.98)], [0.9, 1.0 / (1.0 - 0.9 * 0.98)]],
        "bounds": {"at_0": [0.95, 1.05], "at_0.9_min": 3.0},
    }
    cases["sparsity_stats"] = {
        "source": "tests/unit/test_kernel.py:144-161",
        "mask_shape": [1, 4, 8, 8],
        "active_rows": 4,
        "total": 256,
        "active": 128,
        "sparsity": 0.5,
    }
    return cases


if __name__ == "__main__":
    out = Path(__file__).with_name("reference_vectors.json")
    out.write_text(json.dumps(build(), indent=1) + "\n")
    print(f"wrote {out}")
