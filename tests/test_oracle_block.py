"""Pinning of the CPU block oracle (oracle/block_ref.py) against the block's float64 definition."""
import numpy as np
import pytest
import torch

import inputs as gi
from oracle import block_ref as br

SMALL = dict(hidden=256, heads=2, head_dim=128, ffn=512, s=40)


def rows_of(segments, s):
    rows = torch.zeros(s, dtype=torch.long)
    for a, b, r in segments:
        rows[a:b] = r
    return rows


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_reference_order_in_fp32_with_dense_weights_equals_the_definition(act):
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act=act, seed=3, **SMALL)
    dense = {n: br.dense_of(w).float() for n, w in lin.items()}
    w = {**dense, **norms}
    got = br.block_ref(x.float(), w, mods, segs, cos.float(), sin.float(), SMALL["heads"], SMALL["head_dim"], act,
                       1e-5, 1e-5)
    want = br.block_naive(x.float(), w, mods, rows_of(segs, SMALL["s"]), cos.double(), sin.double(), SMALL["heads"],
                          SMALL["head_dim"], act, 1e-5, 1e-5)
    assert rel(got - x.float(), want - x.double()) < 1e-5


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_naive_block_catches_plausible_mistakes(act):
    """The definition tells apart the mistakes a restatement could make (so the test above pins something)."""
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act=act, seed=4, **SMALL)
    w = {**{n: br.dense_of(v) for n, v in lin.items()}, **norms}
    rows = rows_of(segs, SMALL["s"])
    args = (SMALL["heads"], SMALL["head_dim"], act, 1e-5, 1e-5)
    base = br.block_naive(x, w, mods, rows, cos.double(), sin.double(), *args) - x.double()
    swapped = br.block_naive(x, w, [mods[1], mods[0]] + list(mods[2:]), rows, cos.double(), sin.double(), *args) - x.double()
    norope = br.block_naive(x, w, mods, rows, torch.ones_like(cos).double(), torch.zeros_like(sin).double(), *args) - x.double()
    gates = br.block_naive(x, w, list(mods[:5]) + [mods[2]], rows, cos.double(), sin.double(), *args) - x.double()
    for other in (swapped, norope, gates):
        assert rel(other, base) > 1e-2


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_w4a8_block_is_the_dense_block_within_activation_quantisation_noise(act):
    """fp32 compute isolates the int8 activation quantisation (about 1 % per linear, the reference's measured
    per-layer error, README.md:132); in bf16 the residual's own rounding dominates the block's small update."""
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act=act, seed=5, **SMALL)
    dense = {**{n: br.dense_of(v) for n, v in lin.items()}, **norms}
    want = br.block_naive(x, dense, mods, rows_of(segs, SMALL["s"]), cos.double(), sin.double(), SMALL["heads"],
                          SMALL["head_dim"], act, 1e-5, 1e-5)
    got32 = br.block_ref(x.float(), {**lin, **norms}, mods, segs, cos.float(), sin.float(), SMALL["heads"],
                         SMALL["head_dim"], act, 1e-5, 1e-5)
    r_delta = rel(got32.double() - x.double(), want - x.double())
    assert 1e-3 < r_delta < 4e-2, r_delta
    got16 = br.block_ref(x, {**lin, **norms}, mods, segs, cos, sin, SMALL["heads"], SMALL["head_dim"], act, 1e-5, 1e-5)
    assert rel(got16, want) < 1e-2


# ------------------------------------------------------------------------------------------------ q/k norm + rope
def _golden_normrope():
    import fixtures as fx

    return [n for n, m in fx.index().items() if m["kind"] == "normrope"]


def _t16(a):
    import numpy as np

    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("name", _golden_normrope())
def test_norm_rope_oracle_matches_the_reference_bit_for_bit(name):
    import fixtures as fx

    meta, a = fx.load(name)
    q, k = _t16(a["q"]).clone(), _t16(a["k"]).clone()
    br.norm_rope_ref(q, k, _t16(a["wq"]), _t16(a["wk"]), meta["eps"], _t16(a["cos"]), _t16(a["sin"]), meta["impl"])
    assert torch.equal(q, _t16(a["q_out"])) and torch.equal(k, _t16(a["k_out"]))
    if "q_norm_only" in a:
        assert torch.equal(br._rms_lanes(_t16(a["q"]), _t16(a["wq"]), meta["eps"]), _t16(a["q_norm_only"]))
