"""Loads the golden fixtures written by tests/golden/make_golden.py."""
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_cases(name: str) -> dict:
    """{case: {field: array}} with shared blobs resolved."""
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    blobs = {k[5:]: z[k] for k in z.files if k.startswith("blob/")}
    cases = {}
    for k in z.files:
        if k.startswith("blob/"):
            continue
        case, field = k.rsplit("/", 1)
        v = z[k]
        if v.dtype.kind == "U" and v.ndim == 0 and str(v).startswith("@"):
            v = blobs[str(v)[1:]]
        cases.setdefault(case, {})[field] = v
    return cases


def f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint32).view(np.float32)
