"""Writes the golden fixtures for the gated-delta scan.

The reference stores no fixture files: its scan test regenerates seeded
inputs (tests/test_gated_delta_metal.py:10-23, numpy default_rng(42)) and
checks against a float64 recurrence computed at test time (:26-39). This
script regenerates the same inputs for the same shapes (:42-46, plus the
2048-token carry test, :74-98) and stores the float64 oracle's outputs, with
a SHA-256 of the inputs so a test can tell if numpy's generator ever drifts.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.gated_delta_ref import metal_test_inputs, metal_test_reference  # noqa: E402

# (L, Dk, Dv, Hk, Hv) of tests/test_gated_delta_metal.py:42-46
METAL_SHAPES = [(1, 32, 5, 3, 6), (7, 64, 32, 2, 2), (17, 128, 128, 16, 32), (129, 256, 7, 2, 6)]
LONG_LENGTH = 2048


def inputs_digest(inputs) -> str:
    h = hashlib.sha256()
    for a in inputs:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    return h.hexdigest()


def fixture_name(shape) -> str:
    return "metal_" + "_".join(map(str, shape)) + ".npz"


def main() -> None:
    cases = [(s, metal_test_inputs(*s)) for s in METAL_SHAPES]
    cases.append(((LONG_LENGTH,), metal_test_inputs(LONG_LENGTH)))
    for shape, inputs in cases:
        y, state = metal_test_reference(inputs)
        big = state.size > 100_000 or y.size > 100_000
        store = np.float32 if big else np.float64
        path = os.path.join(HERE, fixture_name(shape))
        np.savez_compressed(path, y=y.astype(store), state=state.astype(store),
                            digest=np.array(inputs_digest(inputs)), shape=np.array(shape))
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
