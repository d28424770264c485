"""Loader for the golden vectors written by make_golden.py (data only: npz without pickles, JSON index)."""
from __future__ import annotations

import json
import os
from typing import Dict, Iterator, Tuple

import numpy as np

import inputs as gi

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = os.path.join(HERE, "vectors")


def index() -> Dict[str, dict]:
    with open(os.path.join(VEC, "index.json")) as f:
        return json.load(f)["cases"]


def load(name: str) -> Tuple[dict, Dict[str, np.ndarray]]:
    meta = index()[name]
    with np.load(os.path.join(VEC, f"{name}.npz"), allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return meta, arrays


def cases(kind: str) -> Iterator[str]:
    return sorted(n for n, m in index().items() if m["kind"] == kind)


def x_values(meta: dict, arrays: Dict[str, np.ndarray]) -> np.ndarray:
    """Activation values of a small case as float32."""
    x = arrays["x"]
    if meta["x_dtype"] == "f32":
        return x.astype(np.float32)
    if meta["x_dtype"] == "f16":
        return x.view(np.float16).astype(np.float32)
    return (x.astype(np.uint32) << 16).view(np.float32)


def out_values(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return bits.astype(np.float32)
    if dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def regenerate(meta: dict):
    """Inputs of a c1/c3 case from the seeded recipes: (x bf16 bits, q, s_rel, s_ch, cb).  Asserts their hash."""
    m, k, n = meta["m"], meta["k"], meta["n"]
    xb = gi.activations(m, k, seed=0)
    if meta["s_kind"] == "f16":
        w = gi.weight_int4_g128(n, k, seed=0, group=meta["group"], convrot=meta["convrot"])
    else:
        w = gi.weight_fp8_g16(n, k, seed=0, group=meta["group"])
    got = gi.sha(xb, *w)
    if got != meta["sha_inputs"]:
        raise AssertionError(f"regenerated inputs differ from the golden run ({got} != {meta['sha_inputs']}): "
                             "the torch RNG changed; re-run tests/golden/make_golden.py")
    return (xb, *w)
