"""The rotate+quant kernel divides by the activation scale through a multiply by its fp32 reciprocal:
q = clamp(rint(round_dtype(fl(y * fl(1 / s)))), -128, 127) where the reference computes round_dtype(y / s)
(h3turbo/h3/qlinear.py:286-292).  Exhaustive over every scale s of the dtype the kernel can meet (positive,
finite, at least round_dtype(1e-30)) and every non-negative finite y of the dtype with y / s <= 130 (y never
exceeds the row's absmax, so |y / s| stays near 127; the sign is symmetric):

- bf16: round_bf16(fl(y * fl(1 / s))) == round_bf16(fl(y / s)) itself;
- f16: the two f16 values can differ (ties between f16 subnormals, |y / s| < 2^-14), never the int8 level.
"""
import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16, as fp32 (finite inputs)."""
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def level(t: np.ndarray) -> np.ndarray:
    return np.clip(np.rint(t), -128, 127)


def sweep(values: np.ndarray, rnd, compare_levels: bool, s_min: float = 0.0) -> int:
    """Number of (s, y) pairs where the reciprocal form differs (values: sorted non-negative finite, fp32; scales
    from s_min)."""
    pos = values[values > max(s_min, 0.0)]
    bad = 0
    chunk = 32
    for i in range(0, pos.size, chunk):
        s = pos[i: i + chunk][:, None]
        hi = np.searchsorted(values, np.float32(130.0) * s.max(), side="right")
        y = values[:hi][None, :]
        with np.errstate(over="ignore", invalid="ignore"):
            q = (y / s).astype(np.float32)
            rs = (np.float32(1.0) / s).astype(np.float32)
            m = (y * rs).astype(np.float32)
        keep = q <= 130.0
        a, b = rnd(q[keep]), rnd(m[keep])
        if compare_levels:
            bad += int(np.count_nonzero(level(a) != level(b)))
        else:
            bad += int(np.count_nonzero(a != b))
    return bad


def test_bf16_reciprocal_gives_the_same_rounded_quotient():
    bits = np.arange(0, 0x7F80, dtype=np.uint32) << 16  # non-negative finite bf16, ascending
    values = bits.view(np.float32)
    # the kernel's scale is round_bf16(max(amax / 127, 1e-30)): never a bf16 subnormal, whose reciprocal overflows
    s_min = float(bf16_round(np.array([1e-30], dtype=np.float32))[0])
    assert sweep(values, bf16_round, compare_levels=False, s_min=s_min * 0.999) == 0


def test_f16_reciprocal_gives_the_same_int8_level():
    values = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)  # ascending
    f16 = lambda x: x.astype(np.float16).astype(np.float32)  # noqa: E731  (numpy rounds to nearest even)
    assert sweep(values, f16, compare_levels=True) == 0
    # the f16 values themselves do differ (here at s = 14, y = 0x1.6cp-18: a tie between f16 subnormals), so the
    # level comparison above is what carries the identity
    s14, y = np.float32(14.0), np.float32(float.fromhex("0x1.6cp-18"))
    assert f16(np.array([y / s14], np.float32))[0] != f16(np.array([y * (np.float32(1.0) / s14)], np.float32))[0]
