"""Pin the CPU oracle (oracle/qlinear_ref.py) against things other than its own formulas:
closed forms, brute force, the reference's own known-answer tables and the golden vectors written by running
the reference's qlinear (tests/golden/make_golden.py).  CPU only."""
from fractions import Fraction

import numpy as np
import pytest
import torch

import fixtures as fx
import inputs as gi
from oracle import qlinear_ref as ref


# ------------------------------------------------------------------------------------------ Hadamard
@pytest.mark.parametrize("size", [4, 16, 64, 256, 1024])
def test_hadamard_is_the_digitwise_product_of_h4(size):
    """Closed form independent of kron: H[i, j] = prod_d H4[i_d, j_d] / sqrt(size) over base-4 digits."""
    h = ref.hadamard_regular(size)
    h4 = [[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]]
    nd = int(round(np.log(size) / np.log(4)))
    rng = np.random.default_rng(size)
    for i, j in rng.integers(0, size, size=(300, 2)):
        sign = 1
        a, b = int(i), int(j)
        for _ in range(nd):
            sign *= h4[a % 4][b % 4]
            a //= 4
            b //= 4
        assert h[i, j] == sign / np.sqrt(size)
    assert np.array_equal(h, h.T)
    assert np.array_equal(h @ h, np.eye(size))  # dyadic entries: exact
    assert set(np.abs(h).ravel().tolist()) == {1.0 / np.sqrt(size)}


@pytest.mark.parametrize("bad", [0, 1, 2, 3, 8, 12, 32, 100, 128, 512, -4])
def test_hadamard_rejects_non_powers_of_four(bad):
    with pytest.raises(ValueError, match="power of 4"):
        ref.hadamard_regular(bad)


# ------------------------------------------------------------------------------------------ rotation
@pytest.mark.parametrize("size", [16, 64, 256])
def test_rotation_equals_exact_rational_sum_rounded_once(size):
    """Brute force in exact rationals: y[j] = sum_i x[i] H[i, j], then one rounding to fp32."""
    rng = np.random.default_rng(size)
    x = ref.bf16_round((rng.standard_normal((2, size)) * np.exp(rng.standard_normal((2, size)) * 2)).astype(np.float32))
    y = ref.rotate_f32(x, size)
    h4 = [[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]]
    nd = int(round(np.log(size) / np.log(4)))
    inv = Fraction(1, int(np.sqrt(size)))
    for r in range(2):
        for j in range(0, size, 7):
            s = Fraction(0)
            for i in range(size):
                sign, a, b = 1, i, j
                for _ in range(nd):
                    sign *= h4[a % 4][b % 4]
                    a //= 4
                    b //= 4
                s += sign * Fraction(float(x[r, i])) * inv
            f64 = float(s)
            assert Fraction(f64) == s  # the exact sum fits fp64 here, so fp64 -> fp32 is the single rounding
            assert y[r, j] == np.float32(f64)


def test_rotation_is_blockwise_and_involutory():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    y = ref.rotate_f32(x, 256)
    assert np.allclose(ref.rotate_f32(y, 256), x, atol=1e-5)
    x2 = x.copy()
    x2[:, :256] = 0
    assert np.array_equal(ref.rotate_f32(x2, 256)[:, 256:], y[:, 256:])
    with pytest.raises(ValueError, match="multiple"):
        ref.rotate_f32(np.zeros((2, 250), np.float32), 256)


# ------------------------------------------------------------------------------------------ number formats
def test_bf16_round_matches_torch_on_random_and_edge_values():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(100000).astype(np.float32) * np.float32(1e3),
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf, 1.0 + 2 ** -8,
                                  1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9 + 2 ** -20], np.float32)])
    want = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ref.bf16_round(v), want)
    assert np.isnan(ref.bf16_round(np.array([np.nan], np.float32)))[0]


def test_fp8_e4m3fn_closed_form_matches_torch_for_every_byte():
    raw = np.arange(256, dtype=np.uint8)
    ours = ref.fp8_e4m3fn_to_f32(raw)
    theirs = torch.from_numpy(raw).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ours)
    assert nan.sum() == 2 and np.array_equal(nan, np.isnan(theirs))
    assert np.array_equal(ours[~nan], theirs[~nan])


def test_reciprocal_division_lemma_for_bf16_quotients():
    """The GPU quantiser computes bf16(y * fl(1/s)) instead of bf16(fl(y / s)) for bf16 y, s.  Exhaustive over all
    bf16 mantissa pairs at several exponents (the only thing that matters away from under/overflow): the two agree."""
    mant = np.arange(128, 256, dtype=np.float32) / np.float32(128.0)  # 1.m with 7 fraction bits = every bf16 mantissa
    for ey in (-3, 0, 5, 7):
        for es in (-20, -4, 0, 3):
            y = (mant * np.float32(2.0 ** ey))[:, None]
            s = (mant * np.float32(2.0 ** es))[None, :]
            exact = ref.bf16_round((y / s).astype(np.float32))
            recip = (np.float32(1.0) / s).astype(np.float32)
            fast = ref.bf16_round((y * recip).astype(np.float32))
            assert np.array_equal(exact, fast), (ey, es)
            assert np.array_equal(ref.bf16_round((-y / s).astype(np.float32)), ref.bf16_round((-y * recip).astype(np.float32)))


# ------------------------------------------------------------------------------------------ quantiser
def test_quantiser_degenerate_rows():
    """KATs of the reference's tests (tests/test_h3_qlinear.py:291-300): a zero row gives xs = 1e-30 and q = 0;
    no NaN/inf; the absmax element lands on the grid end."""
    for dt in ("f32", "bf16", "f16"):
        x = np.zeros((4, 256), np.float32)
        x[1, 3], x[2], x[3, 0] = 1e-3, 3.0, (6e4 if dt == "f16" else 1e30)
        x = ref.round_to(x, dt)
        for mode in ("ck", "eager"):
            q, s = ref.quantize_rows(x, dt, 256, mode)
            assert np.isfinite(s).all() and (s > 0).all()
            assert np.abs(q[0]).sum() == 0 and s[0, 0] == np.float32(1e-30)
            assert np.abs(q.astype(np.int32)).max() <= 128
            assert np.abs(q[3].astype(np.int32)).max() >= 120 and np.abs(q[2].astype(np.int32)).max() >= 120


def test_quantiser_fp32_closed_form():
    """fp32 input, either mode: q = clamp(rint(xr / (amax/127)), -128, 127) with xr the fp32 rotation."""
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((11, 512)) * np.exp(rng.standard_normal((11, 512)))).astype(np.float32)
    xr = ref.rotate_f32(x, 256)
    scale = np.maximum(np.abs(xr).max(-1, keepdims=True) / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    want = np.clip(np.rint(xr / scale), -128, 127).astype(np.int8)
    for mode in ("ck", "eager"):
        q, s = ref.quantize_rows(x, "f32", 256, mode)
        assert np.array_equal(q, want) and np.array_equal(s, scale)
        assert (np.abs(q.astype(np.int32)).max(-1) >= 126).all()


@pytest.mark.parametrize("name", list(fx.cases("small")))
def test_oracle_matches_reference_small_cases(name):
    meta, a = fx.load(name)
    x = fx.x_values(meta, a)
    q, xs = ref.quantize_rows(x, meta["x_dtype"], meta["convrot"], meta["mode"])
    assert np.array_equal(xs, a["xs"])
    assert np.array_equal(q, a["xq"])
    w8 = ref.decode_int8_grid(a["q"], a["s_rel"], meta["s_kind"], a["cb"], meta["group"])
    if "w8" in a:
        assert np.array_equal(w8, a["w8"])
    acc = ref.int8_mm(q, w8)
    assert np.array_equal(acc, a["acc"])
    out = ref.epilogue(acc, xs, a["s_ch"], meta["x_dtype"], meta["mode"], a.get("bias"))
    assert np.array_equal(out, fx.out_values(a["out"], meta["x_dtype"]))


def test_oracle_matches_reference_swiglu_case():
    meta, a = fx.load("swiglu_m9_k512_n40")
    h = fx.out_values(a["h"], "bf16")
    act = ref.swiglu_bf16(h)
    assert np.array_equal(act, fx.out_values(a["act"], "bf16"))
    out, *_ = ref.linear_a8(act, "bf16", a["q"], a["s_rel"], "fp8", a["s_ch"], a["cb"], 16, 256)
    assert np.array_equal(out, fx.out_values(a["out"], "bf16"))


@pytest.mark.parametrize("name", ["c1_f16", "c1_fp8"])
def test_oracle_matches_reference_config1_bit_for_bit(name):
    meta, a = fx.load(name)
    xb, q, s_rel, s_ch, cb = fx.regenerate(meta)
    x = ref.bf16_from_bits(xb)
    out, xq, xs, acc = ref.linear_a8(x, "bf16", q, s_rel, meta["s_kind"], s_ch, cb, meta["group"], 256)
    assert gi.sha(xq) == meta["sha_xq"] and gi.sha(xs) == meta["sha_xs"]
    assert gi.sha(acc) == meta["sha_acc"]
    assert gi.sha(ref.bf16_bits(out)) == meta["sha_out"]
    out_e, *_ = ref.linear_a8(x, "bf16", q, s_rel, meta["s_kind"], s_ch, cb, meta["group"], 256, mode="eager")
    assert gi.sha(ref.bf16_bits(out_e)) == meta["sha_out_eager"]
    # the emulated (reference-algorithm) GEMM equals the exact one
    assert np.array_equal(ref.int8_mm_emulated(xq, ref.decode_int8_grid(q, s_rel, meta["s_kind"], cb, meta["group"])), acc)


def test_oracle_matches_reference_config2_quantiser():
    meta, a = fx.load("c2")
    xb = gi.activations(meta["m"], meta["k"], seed=0)
    assert gi.sha(xb) == meta["sha_inputs"]
    q, xs = ref.quantize_rows(ref.bf16_from_bits(xb), "bf16", 256, "ck")
    assert gi.sha(q) == meta["sha_xq"] and gi.sha(xs) == meta["sha_xs"]


# ------------------------------------------------------------------------------------------ decode
def _spec_decode(q, s_bytes, cb, group):
    """Element loops straight from the format description (types.py:14-17, qlinear.py:157-166)."""
    n, kh = q.shape
    out = np.zeros((n, kh * 2), dtype=np.int8)
    for i in range(n):
        for j in range(kh * 2):
            byte = int(q[i, j // 2]) & 0xFF
            nib = (byte >> 4) if j % 2 else (byte & 0xF)
            s = np.float32(ref.fp8_e4m3fn_to_f32(np.array([s_bytes[i, j // group]], np.uint8))[0])
            out[i, j] = int(np.clip(np.rint(np.float32(cb[nib]) * s), -127, 127))
    return out


@pytest.mark.parametrize("group", [16, 4, 32])
def test_decode_matches_element_loops(group):
    q, s, s_ch, cb = gi.weight_fp8_g16(7, 128, seed=3, group=group)
    want = _spec_decode(q, s, cb, group)
    got = ref.decode_int8_grid(q, s, "fp8", cb, group)
    assert np.array_equal(got, want)
    assert want.min() < -100 and want.max() > 100


def test_decode_ties_round_half_even_and_clamp_symmetric():
    """Known-answer table of the reference's tests (tests/test_h3_qlinear.py:171-184)."""
    cb = np.array([0.5, -0.5, 1.0, -1.0, 0.25, -0.25, 0.75, -0.75, 0.0, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5], np.float32)
    cases = [(0, 3.0, 2), (0, 5.0, 2), (1, 5.0, -2), (2, 448.0, 127), (3, 448.0, -127), (4, 6.0, 2), (5, 6.0, -2),
             (6, 7.0, 5), (8, 448.0, 0), (0, 7.0, 4)]
    codes = np.array([c[0] for c in cases])
    byte = (codes | (codes << 4)).astype(np.uint8)
    q = np.repeat(byte[:, None], 8, axis=1).view(np.int8)
    s = torch.tensor([[c[1]] for c in cases]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = ref.decode_int8_grid(q, s, "fp8", cb, 16)
    assert got.tolist() == [[c[2]] * 16 for c in cases]


def test_decode_scale_kinds_agree_and_nan_scales_give_zero():
    q, s, _, cb = gi.weight_fp8_g16(5, 64, seed=9)
    a = ref.decode_int8_grid(q, s, "fp8", cb, 16)
    s32 = ref.fp8_e4m3fn_to_f32(s)
    assert np.array_equal(ref.decode_int8_grid(q, s32, "f32", cb, 16), a)
    s16 = s32.astype(np.float16).view(np.uint16)  # 20..200 fp8 values are exact in fp16
    assert np.array_equal(ref.decode_int8_grid(q, s16, "f16", cb, 16), a)
    sb = ref.bf16_bits(s32)  # and in bf16 (3 mantissa bits)
    assert np.array_equal(ref.decode_int8_grid(q, sb, "bf16", cb, 16), a)
    s_nan = s.copy()
    s_nan[0, 0] = 0x7F
    d = ref.decode_int8_grid(q, s_nan, "fp8", cb, 16)
    assert (d[0, :16] == 0).all() and np.array_equal(d[:, 16:], a[:, 16:])


# ------------------------------------------------------------------------------------------ int8 GEMM
@pytest.mark.parametrize("k", [8, 256, 1000, 1024, 1032, 3000, 4096])
def test_int8_mm_exact_including_worst_case_magnitudes(k):
    rng = np.random.default_rng(k)
    a = rng.integers(-128, 128, (5, k)).astype(np.int8)
    w = rng.integers(-127, 128, (9, k)).astype(np.int8)
    want = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    assert np.array_equal(ref.int8_mm(a, w), want)
    assert np.array_equal(ref.int8_mm_emulated(a, w), want)
    a = np.full((3, k), 127, np.int8)
    w = np.full((2, k), 127, np.int8)
    assert ref.int8_mm(a, w)[2, 1] == 16129 * k and ref.int8_mm_emulated(a, w)[2, 1] == 16129 * k
    a = np.full((3, k), -128, np.int8)
    a[:, 1::2] = -127
    for v in (-127, 127):
        w = np.full((2, k), v, np.int8)
        want = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
        assert np.array_equal(ref.int8_mm(a, w), want) and np.array_equal(ref.int8_mm_emulated(a, w), want)


def test_epilogue_orders_differ_in_fp32():
    """ck = (acc * xs) * s_ch, eager = acc * (xs * s_ch): the two orders differ in fp32, so the golden checks pin one."""
    rng = np.random.default_rng(5)
    acc = rng.integers(-2 ** 20, 2 ** 20, (64, 64)).astype(np.int32)
    xs = rng.random((64, 1)).astype(np.float32)
    sc = rng.random(64).astype(np.float32)
    assert not np.array_equal(ref.epilogue(acc, xs, sc, "f32", "ck"), ref.epilogue(acc, xs, sc, "f32", "eager"))


# ------------------------------------------------------------------------------------------------ rotation extension
# Sizes that are not powers of 4 (8, 32, 128, 512) are an extension: the reference rejects them.  These checks pin
# the oracle's definition by means other than its own formula.
EXT_SIZES = [8, 32, 128, 512]


@pytest.mark.parametrize("size", EXT_SIZES)
def test_pow2_hadamard_is_the_elementwise_sign_formula(size):
    """H[i, j] = (-1)^(top bit of i and j) * prod over 2-bit digits d of H4[i_d, j_d], with H4[a, b] = -1 iff
    a + b = 3: built by loops, independently of np.kron."""
    bits = size.bit_length() - 1
    want = np.ones((size, size))
    for i in range(size):
        for j in range(size):
            sign = -1.0 if (i >> (bits - 1)) & (j >> (bits - 1)) & 1 else 1.0
            for d in range((bits - 1) // 2):
                if ((i >> (2 * d)) & 3) + ((j >> (2 * d)) & 3) == 3:
                    sign = -sign
            want[i, j] = sign
    h = ref.hadamard_pow2(size)
    assert np.array_equal(h, want)
    assert np.array_equal(h @ h.T, size * np.eye(size)) and np.array_equal(h, h.T)


@pytest.mark.parametrize("size", EXT_SIZES)
def test_extension_scale_is_the_rounded_inverse_square_root(size):
    c = ref.rotation_scale(size)
    assert ref.rotation_scale(128) == float.fromhex("0x1.6a09e667f3bcdp-4")  # RN(sqrt 2) / 16
    # c is fp64's nearest to 1/sqrt(size): c^2 * size lies within a few ulps of 1
    assert abs(c * c * size - 1.0) < 4e-16


@pytest.mark.parametrize("size", EXT_SIZES)
def test_extension_rotation_of_ones_has_the_closed_form(size):
    """All-ones rows: column sums of H are 2 per H4 digit and (2, 0) for the H2 top bit, so y_j = 2^((bits+1)/2) * c
    where the top bit of j is 0 and 0 where it is 1: H2 sits on the top index bit, not the bottom one."""
    bits = size.bit_length() - 1
    y = ref.rotate_f32(np.ones((1, size), np.float32), size)
    top = (np.arange(size) >> (bits - 1)) & 1
    want = np.where(top == 0, np.float32(2.0 ** ((bits + 1) // 2) * ref.rotation_scale(size)), np.float32(0.0))
    assert np.array_equal(y[0], want.astype(np.float32))


@pytest.mark.parametrize("size", EXT_SIZES)
def test_extension_rotation_equals_the_digit_by_digit_transform(size):
    """The dense fp64 matmul against applying H2 on the top bit and H4 on each 2-bit digit separately (an FWHT):
    exact integer sums, so the two orders agree bit for bit after the same scaling and rounding."""
    bits = size.bit_length() - 1
    rng = np.random.default_rng(size)
    x = rng.integers(-1000, 1000, (3, 2 * size)).astype(np.float32) * np.float32(0.125)
    v = x.astype(np.float64).reshape(3, 2, size)
    axes = [2] + [4] * ((bits - 1) // 2)  # most significant first
    v = v.reshape(3, 2, *axes)
    v = np.moveaxis(np.tensordot(v, ref._H2, axes=([2], [0])), -1, 2)
    for a in range(len(axes) - 1):
        v = np.moveaxis(np.tensordot(v, ref._H4, axes=([3 + a], [0])), -1, 3 + a)
    y = (v.reshape(3, 2 * size) * ref.rotation_scale(size)).astype(np.float32)
    assert np.array_equal(ref.rotate_f32(x, size), y)
