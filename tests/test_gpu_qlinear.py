"""GPU parity of the HIP W4A8 path against the reference's golden vectors and the CPU oracle.

Bar: bit-exact for the int8 activations, their fp32 scales, the int8 weight grid, the int32 accumulators and the
bf16/f16/f32 outputs (the reference's torch backend rounds the same way).  Full BASELINE sizes are checked
through SHA-256 of the reference's outputs (configs 1-3) or through sampled rows recomputed by the oracle.
"""
import numpy as np
import pytest
import torch

import fixtures as fx
import inputs as gi
from h3turbo_amd import _lib
from h3turbo_amd import qlinear as ql
from h3turbo_amd.types import W4A8Weight
from oracle import qlinear_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def t_bits16(bits: np.ndarray, dt: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(dt).to(DEV)


def np_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def make_w(q, s_rel, s_kind, s_ch, cb, group, convrot) -> W4A8Weight:
    if s_kind == "fp8":
        s = torch.from_numpy(np.ascontiguousarray(s_rel)).view(torch.float8_e4m3fn)
    elif s_kind == "f16":
        s = torch.from_numpy(np.ascontiguousarray(s_rel).view(np.int16)).view(torch.float16)
    elif s_kind == "bf16":
        s = torch.from_numpy(np.ascontiguousarray(s_rel).view(np.int16)).view(torch.bfloat16)
    else:
        s = torch.from_numpy(np.ascontiguousarray(s_rel, dtype=np.float32))
    return W4A8Weight(torch.from_numpy(np.ascontiguousarray(q)).to(DEV), s.to(DEV), torch.from_numpy(s_ch).to(DEV),
                      torch.from_numpy(cb).to(DEV), group_size=group, convrot=convrot)


def gpu_acc(xq: torch.Tensor, xs: torch.Tensor, w8: torch.Tensor, s_ch: torch.Tensor) -> torch.Tensor:
    """int32 accumulators of the HIP GEMM (its acc_out side channel)."""
    m, k = xq.shape
    n = w8.shape[0]
    acc = torch.empty(m, n, dtype=torch.int32, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, s_ch.data_ptr(), None, m, n, k, 0,
                                 out.data_ptr(), _lib.BF16, n, acc.data_ptr(), _lib.stream_of(DEV)), "gemm")
    return acc


# ---------------------------------------------------------------------------------------------- golden: small
@pytest.mark.parametrize("name", list(fx.cases("small")))
def test_small_golden_cases_bit_exact(name):
    meta, a = fx.load(name)
    print(f"case {name}", flush=True)
    dt = DT[meta["x_dtype"]]
    x = (torch.from_numpy(a["x"]).to(DEV) if meta["x_dtype"] == "f32" else t_bits16(a["x"], dt))
    w = make_w(a["q"], a["s_rel"], meta["s_kind"], a["s_ch"], a["cb"], meta["group"], meta["convrot"])
    xq, xs = ql.quantize_activation(x, size=meta["convrot"], quant_mode=meta["mode"])
    assert np.array_equal(xs.cpu().numpy(), a["xs"]), "scales"
    assert np.array_equal(xq.cpu().numpy(), a["xq"]), "int8 activations"
    w8 = ql.decode_int8_grid(w)
    want_w8 = a["w8"] if "w8" in a else ref.decode_int8_grid(a["q"], a["s_rel"], meta["s_kind"], a["cb"], meta["group"])
    assert np.array_equal(w8.cpu().numpy(), want_w8), "int8 weight grid"
    assert np.array_equal(gpu_acc(xq, xs, w8, w.s_ch).cpu().numpy(), a["acc"]), "int32 accumulators"
    b = torch.from_numpy(a["bias"]).to(DEV) if "bias" in a else None
    out = ql.linear(x, w, b, quant_mode=meta["mode"])
    assert out.dtype == dt
    assert np.array_equal(np_bits(out), a["out"]), "outputs"


def test_swiglu_golden_case():
    meta, a = fx.load("swiglu_m9_k512_n40")
    h = t_bits16(a["h"], torch.bfloat16)
    w = make_w(a["q"], a["s_rel"], "fp8", a["s_ch"], a["cb"], 16, 256)
    act = ql._swiglu(h)
    out = ql.linear(h, w, input_act="swiglu")
    if np.array_equal(np_bits(act), a["act"]):  # torch's GPU silu agrees with the CPU one here: the chain is exact
        assert np.array_equal(np_bits(out), a["out"])
    ref_out = fx.out_values(a["out"], "bf16")
    err = np.abs(out.float().cpu().numpy() - ref_out).max() / np.sqrt((ref_out ** 2).mean())
    assert err < 1e-2
    assert torch.equal(out, ql.linear(act, w))


# ---------------------------------------------------------------------------------------------- golden: configs 1-3
@pytest.mark.parametrize("name", ["c1_f16", "c1_fp8"])
def test_config1_full_chain_bit_exact(name):
    meta, a = fx.load(name)
    xb, q, s_rel, s_ch, cb = fx.regenerate(meta)
    x = t_bits16(xb, torch.bfloat16)
    w = make_w(q, s_rel, meta["s_kind"], s_ch, cb, meta["group"], 256)
    xq, xs = ql.quantize_activation(x)
    assert gi.sha(xq.cpu().numpy()) == meta["sha_xq"]
    assert gi.sha(xs.cpu().numpy()) == meta["sha_xs"]
    w8 = ql.decode_int8_grid(w)
    assert gi.sha(w8.cpu().numpy()) == meta["sha_w8"]
    assert gi.sha(gpu_acc(xq, xs, w8, w.s_ch).cpu().numpy()) == meta["sha_acc"]
    assert gi.sha(np_bits(ql.linear(x, w))) == meta["sha_out"]
    assert gi.sha(np_bits(ql.linear(x, w, quant_mode="eager"))) == meta["sha_out_eager"]


def test_config2_rotate_quant_bit_exact():
    meta, a = fx.load("c2")
    xb = gi.activations(meta["m"], meta["k"], seed=0)
    assert gi.sha(xb) == meta["sha_inputs"]
    xq, xs = ql.quantize_activation(t_bits16(xb, torch.bfloat16))
    assert np.array_equal(xs.cpu().numpy(), a["xs"])
    assert np.array_equal(xq[:4].cpu().numpy(), a["xq"])
    assert gi.sha(xq.cpu().numpy()) == meta["sha_xq"]


@pytest.mark.parametrize("name", list(fx.cases("c3")))
def test_config3_m512_bit_exact(name):
    meta, a = fx.load(name)
    xb, q, s_rel, s_ch, cb = fx.regenerate(meta)
    x = t_bits16(xb, torch.bfloat16)
    w = make_w(q, s_rel, "f16", s_ch, cb, 128, 256)
    xq, xs = ql.quantize_activation(x)
    assert gi.sha(xq.cpu().numpy()) == meta["sha_xq"] and gi.sha(xs.cpu().numpy()) == meta["sha_xs"]
    acc = gpu_acc(xq, xs, ql.decode_int8_grid(w), w.s_ch)
    assert np.array_equal(acc[:1].cpu().numpy(), a["acc"])
    assert gi.sha(acc.cpu().numpy()) == meta["sha_acc"]
    out = ql.linear(x, w)
    assert np.array_equal(np_bits(out[:2]), a["out"])
    assert gi.sha(np_bits(out)) == meta["sha_out"]


# ---------------------------------------------------------------------------------------------- full sizes, sampled rows
def random_weight_gpu(n, k, seed, group=128, s_kind="f16"):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8, device=DEV)
    if s_kind == "f16":
        s = (torch.rand(n, k // group, generator=g, device=DEV) * 15.0 + 0.875).to(torch.float16)
    else:
        s = (torch.rand(n, k // group, generator=g, device=DEV) * 180 + 20).to(torch.float8_e4m3fn)
    s_ch = torch.rand(n, generator=g, device=DEV) * 1e-3 + 1e-4
    cb = torch.arange(-8, 8, dtype=torch.float32, device=DEV)
    return W4A8Weight(q, s, s_ch, cb, group_size=group, convrot=256)


def random_acts_gpu(m, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, generator=g, device=DEV)
    idx = torch.randperm(k, generator=g, device=DEV)[: round(0.01 * k)]
    x[:, idx] *= 20
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("m,k,n", [(4096, 5120, 13824), (12090, 5120, 5120), (12090, 5120, 15360), (12090, 13824, 5120),
                                   (32768, 5120, 13824)])
def test_full_size_sampled_rows_match_the_oracle(m, k, n):
    print(f"shape m={m} k={k} n={n}", flush=True)
    x = random_acts_gpu(m, k, seed=m + k)
    w = random_weight_gpu(n, k, seed=n + k)
    out = ql.linear(x, w)
    xq, xs = ql.quantize_activation(x)
    torch.cuda.synchronize()
    rng = np.random.default_rng(m)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, 257, m - 1, m - 2], rng.integers(0, m, 9)]))
    rows_t = torch.from_numpy(rows).to(DEV)
    xr = x.index_select(0, rows_t).contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    q_ref, xs_ref = ref.quantize_rows(ref.bf16_from_bits(xr), "bf16", 256, "ck")
    assert np.array_equal(xs.index_select(0, rows_t).cpu().numpy(), xs_ref)
    assert np.array_equal(xq.index_select(0, rows_t).cpu().numpy(), q_ref)
    s_bits = w.s_rel.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    w8 = ref.decode_int8_grid(w.q.cpu().numpy(), s_bits, "f16", w.codebook.cpu().numpy(), 128)
    acc = ref.int8_mm(q_ref, w8)
    want = ref.epilogue(acc, xs_ref, w.s_ch.cpu().numpy(), "bf16", "ck")
    assert np.array_equal(np_bits(out.index_select(0, rows_t)), ref.bf16_bits(want))
    # every row and column: the reference's CUDA formulation of the GEMM and the "ck" epilogue as torch ops
    # (h3turbo/h3/qlinear.py:242-247, :401) on the kernel's own int8 operands
    w8g = ql.decode_int8_grid(w)
    assert np.array_equal(w8g[:64].cpu().numpy(), w8[:64])
    full = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    torch.mul(torch.mul(torch._int_mm(xq, w8g.t()), xs), w.s_ch.float().reshape(1, -1), out=full)
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))


# ---------------------------------------------------------------------------------------------- API behaviour
N, K = 40, 512


@pytest.fixture(scope="module")
def wq():
    q, s, s_ch, cb = gi.weight_fp8_g16(N, K, seed=11)
    return make_w(q, s, "fp8", s_ch, cb, 16, 256)


def oracle_linear(x: torch.Tensor, w: W4A8Weight, mode="ck", bias=None, out_dtype=None):
    dts = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
    xd = dts[x.dtype]
    xv = x.float().cpu().numpy()
    s_kind = "fp8"
    sb = w.s_rel.view(torch.uint8).cpu().numpy()
    out, *_ = ref.linear_a8(xv.reshape(-1, xv.shape[-1]), xd, w.q.cpu().numpy(), sb, s_kind, w.s_ch.cpu().numpy(),
                            w.codebook.cpu().numpy(), w.group_size, w.convrot, out_dtype=dts[out_dtype or x.dtype],
                            mode=mode, bias=None if bias is None else bias.cpu().numpy())
    return out


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 7, 17, 257])
def test_token_counts_and_dtypes_match_the_oracle(wq, m, dt):
    x = torch.randn(m, K, generator=torch.Generator().manual_seed(m)).to(dt).to(DEV)
    for mode in ("ck", "eager"):
        got = ql.linear(x, wq, quant_mode=mode)
        assert got.dtype == dt
        assert np.array_equal(got.float().cpu().numpy(), oracle_linear(x, wq, mode)), mode


@pytest.mark.parametrize("shape", [(1, K), (2, 5, K), (3, 1, 4, K)])
def test_leading_dims_and_token_independence(wq, shape):
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape))).to(DEV)
    y = ql.linear(x, wq)
    assert y.shape == (*shape[:-1], N) and y.dtype == torch.float32
    assert torch.equal(y.reshape(-1, N), ql.linear(x.reshape(-1, K), wq))
    assert torch.equal(y.reshape(-1, N)[:1], ql.linear(x.reshape(-1, K)[:1], wq))


def test_noncontiguous_unaligned_and_empty_inputs(wq):
    x = torch.randn(K, 13, generator=torch.Generator().manual_seed(20)).to(DEV).T
    assert not x.is_contiguous() and torch.equal(ql.linear(x, wq), ql.linear(x.contiguous(), wq))
    xb = torch.randn(9, K + 8, generator=torch.Generator().manual_seed(21)).to(torch.bfloat16).to(DEV)
    view = xb[:, 8:]  # rows 16-byte aligned but base offset by 16 bytes: still the fast path
    odd = torch.randn(9, K + 1, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16).to(DEV)[:, 1:]  # unaligned: generic path
    for v in (view, odd):
        assert torch.equal(ql.linear(v, wq), ql.linear(v.contiguous(), wq))
        q1, s1 = ql.quantize_activation(v)
        q2, s2 = ql.quantize_activation(v.contiguous())
        assert torch.equal(q1, q2) and torch.equal(s1, s2)
    assert ql.linear(torch.zeros(0, K, device=DEV), wq).shape == (0, N)
    assert ql.linear(torch.zeros(2, 0, K, device=DEV), wq).shape == (2, 0, N)


def test_chunking_is_exact(wq):
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn(37, K, generator=torch.Generator().manual_seed(14)).to(dt).to(DEV)
        full = ql.linear(x, wq)
        for c in (1, 2, 5, 36, 37, 1000):
            assert torch.equal(ql.linear(x, wq, chunk_tokens=c), full), (dt, c)


def test_bias_is_added_after_output_rounding(wq):
    b = torch.randn(N, generator=torch.Generator().manual_seed(21)).to(DEV)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = torch.randn(9, K, generator=torch.Generator().manual_seed(22)).to(dt).to(DEV)
        for mode in ("ck", "eager"):
            plain = ql.linear(x, wq, quant_mode=mode)
            with_b = ql.linear(x, wq, b, quant_mode=mode)
            assert torch.equal(with_b, plain + b.to(dt)), (dt, mode)
            assert np.array_equal(with_b.float().cpu().numpy(), oracle_linear(x, wq, mode, bias=b))


def test_out_dtype(wq):
    x = torch.randn(5, K, generator=torch.Generator().manual_seed(24)).to(torch.bfloat16).to(DEV)
    y = ql.linear(x, wq, out_dtype=torch.float32)
    assert y.dtype == torch.float32 and torch.equal(y.to(torch.bfloat16), ql.linear(x, wq))


@pytest.mark.parametrize("rot", [4, 16, 64, 256, 1024])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_rotation_sizes_and_dtypes_match_the_oracle(rot, dt):
    k = 2048
    x = (torch.randn(6, k, generator=torch.Generator().manual_seed(rot)) * 3).to(dt)
    xv = x.float().numpy()
    dts = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dt]
    for mode in ("ck", "eager"):
        q, s = ql.quantize_activation(x.to(DEV), size=rot, quant_mode=mode)
        qr, sr = ref.quantize_rows(xv, dts, rot, mode)
        assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(q.cpu().numpy(), qr), mode
    y = ql.rotate(x.to(DEV), size=rot)
    yr = ref.round_to(ref.rotate_f32(xv, rot), dts)
    assert y.dtype == dt and np.array_equal(y.float().cpu().numpy(), yr)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rows_over_many_scales_match_the_oracle(dt):
    """Row magnitudes from 1e-7 to 5e4 (f16: subnormal, tiny-clamped and large scales, the largest rows overflowing
    to inf): the kernel's multiply by the reciprocal scale against the oracle's true division, bit for bit (NaN
    scales of rows holding inf compare equal)."""
    g = torch.Generator().manual_seed(77)
    rows, k = 384, 1024
    mag = torch.logspace(-7, 4.7, rows).unsqueeze(1)
    x = (torch.randn(rows, k, generator=g) * mag).to(dt)
    dts = {torch.bfloat16: "bf16", torch.float16: "f16"}[dt]
    for mode in ("ck", "eager"):
        q, s = ql.quantize_activation(x.to(DEV), quant_mode=mode)
        qr, sr = ref.quantize_rows(x.float().numpy(), dts, 256, mode)
        assert_scales(s.cpu().numpy(), sr, mode)
        assert np.array_equal(q.cpu().numpy(), qr), mode


def assert_scales(got, want, what):
    """Finite scales bit for bit; where the reference scale is inf or NaN this one is the same or NaN (the s - 2x
    butterfly turns a lone inf input into inf - inf) -- the row's levels are 0 and its linear output NaN either way."""
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin]), what
    assert (np.isnan(got[~fin]) | (got[~fin] == want[~fin])).all(), what


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_non_finite_rows_match_the_oracle(dt):
    """A row holding one inf (every rotated value +-inf: reference scale inf, levels 0), +inf and -inf (inf - inf:
    NaN), a NaN, a zero row and a finite one: scales NaN-propagating like torch's amax, NaN quotients at level 0."""
    k = 512
    x = torch.randn(6, k, generator=torch.Generator().manual_seed(5))
    x[1, 7] = float("inf")
    x[2, 3], x[2, 300] = float("inf"), float("-inf")
    x[3, 100] = float("nan")
    x[4] = 0.0
    x[5, 9] = float("-inf")
    x = x.to(dt)
    dts = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dt]
    for mode in ("ck", "eager"):
        q, s = ql.quantize_activation(x.to(DEV), quant_mode=mode)
        qr, sr = ref.quantize_rows(x.float().numpy(), dts, 256, mode)
        assert_scales(s.cpu().numpy(), sr, (mode, s.cpu().numpy().ravel(), sr.ravel()))
        assert np.isfinite(sr[[0, 4, 5 - 5]]).all() and np.isnan(sr[3]).all()
        assert np.array_equal(q.cpu().numpy(), qr), mode
        assert not q[1:4].any()  # rows holding inf or NaN: every level 0


def test_degenerate_rows():
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = torch.zeros(4, 256, dtype=dt)
        x[1, 3], x[2], x[3, 0] = 1e-3, 3.0, (6e4 if dt == torch.float16 else 1e30)
        for mode in ("ck", "eager"):
            q, s = ql.quantize_activation(x.to(DEV), quant_mode=mode)
            qr, sr = ref.quantize_rows(x.float().numpy(), {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dt], 256, mode)
            assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)
            assert q[0].abs().sum() == 0 and s[0].item() == np.float32(1e-30)


# ---------------------------------------------------------------------------------------------- decode
@pytest.mark.parametrize("group", [4, 8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("s_kind", ["fp8", "f16", "bf16", "f32"])
def test_decode_all_scale_kinds_and_groups(group, s_kind):
    n, k = 37, 512
    q, s8, _, cb = gi.weight_fp8_g16(n, k, seed=group, group=group)
    sv = ref.fp8_e4m3fn_to_f32(s8)
    s_raw = {"fp8": s8, "f16": sv.astype(np.float16).view(np.uint16), "bf16": ref.bf16_bits(sv), "f32": sv}[s_kind]
    w = make_w(q, s_raw, s_kind, np.ones(n, np.float32), cb, group, 256)
    want = ref.decode_int8_grid(q, s_raw, s_kind, cb, group)
    assert np.array_equal(ql.decode_int8_grid(w).cpu().numpy(), want)


def test_decode_ties_clamp_and_views_into_larger_buffers():
    cb = np.array([0.5, -0.5, 1.0, -1.0, 0.25, -0.25, 0.75, -0.75, 0.0, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5], np.float32)
    cases = [(0, 3.0, 2), (0, 5.0, 2), (1, 5.0, -2), (2, 448.0, 127), (3, 448.0, -127), (4, 6.0, 2), (5, 6.0, -2),
             (6, 7.0, 5), (8, 448.0, 0), (0, 7.0, 4)]
    codes = np.array([c[0] for c in cases])
    q = np.repeat((codes | (codes << 4)).astype(np.uint8)[:, None], 8, axis=1).view(np.int8)
    s = torch.tensor([[c[1]] for c in cases]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    w = make_w(q, s, "fp8", np.ones(len(cases), np.float32), cb, 16, 16)
    assert ql.decode_int8_grid(w).cpu().tolist() == [[c[2]] * 16 for c in cases]
    qq, ss, s_ch, cbb = gi.weight_fp8_g16(37, 128, seed=5)
    full = ql.decode_int8_grid(make_w(qq, ss, "fp8", s_ch, cbb, 16, 128))
    big = torch.cat([torch.zeros(3, 64, dtype=torch.int8), torch.from_numpy(qq), torch.zeros(2, 64, dtype=torch.int8)]).to(DEV)
    sub = W4A8Weight(big[3:-2], torch.from_numpy(ss).view(torch.float8_e4m3fn).to(DEV), torch.from_numpy(s_ch).to(DEV),
                     torch.from_numpy(cbb).to(DEV), 16, 128)
    assert torch.equal(ql.decode_int8_grid(sub), full)


@pytest.mark.parametrize("group", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("pad", [0, 8, 16])
def test_decode_table_path_every_byte_nan_and_clamp_scales(group, pad):
    """fp8 scales decode through byte tables (groups of 32 or more: one per scale, built in registers; groups of 16
    and rows with an 8-byte stride: the workgroup's table of all 256 scale bytes): every packed byte value, NaN /
    +-448 / zero / negative scales, rows that are views with a 16-byte or an 8-byte stride."""
    n, k = 24, 1024
    rng = np.random.default_rng(group + pad)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    q[0] = np.arange(256, dtype=np.uint8).repeat(k // 512)
    s = rng.integers(0, 256, (n, k // group), dtype=np.uint8)  # every e4m3fn byte: NaN 0x7F/0xFF, negatives
    s[1], s[2], s[3], s[4] = 0x7F, 0x7E, 0xFE, 0x00  # NaN, 448, -448, 0
    _, _, _, cb = gi.weight_fp8_g16(4, 64, seed=1)
    want = ref.decode_int8_grid(q.view(np.int8), s, "fp8", cb, group)
    big = torch.zeros(n, k // 2 + pad + 16, dtype=torch.int8)
    big[:, pad:pad + k // 2] = torch.from_numpy(q.view(np.int8))
    qd = big.to(DEV)[:, pad:pad + k // 2]
    w = W4A8Weight(qd, torch.from_numpy(s).view(torch.float8_e4m3fn).to(DEV), torch.ones(n, device=DEV),
                   torch.from_numpy(cb).to(DEV), group, 256)
    assert np.array_equal(ql.decode_int8_grid(w).cpu().numpy(), want)


# ---------------------------------------------------------------------------------------------- accuracy (a8 / a16)
def test_a8_error_is_the_predicted_quantisation_noise_and_a16_removes_it(wq):
    x = torch.randn(64, K, generator=torch.Generator().manual_seed(12)).to(DEV)
    y = ql.linear(x, wq)
    dense = ql.dequantize(wq, torch.float64, rotated=False)
    want = x.double() @ dense.T
    rel = ((y.double() - want).norm() / want.norm()).item()
    q, s = ql.quantize_activation(x)
    xr = ql.rotate(x)
    predicted = ((s.double() ** 2 / 12).mean().sqrt() / xr.double().pow(2).mean().sqrt()).item()
    assert 0.8 * predicted < rel < 1.25 * predicted and rel < 0.015
    y16 = ql.linear(x, wq, precision="a16")
    assert ((y16.double() - want).norm() / want.norm()).item() < 2e-6
    xb = x.to(torch.bfloat16)
    want_b = xb.double() @ dense.T
    y16b = ql.linear(xb, wq, precision="a16")
    y8b = ql.linear(xb, wq)
    r16 = ((y16b.double() - want_b).norm() / want_b.norm()).item()
    r8 = ((y8b.double() - want_b).norm() / want_b.norm()).item()
    assert y16b.dtype == torch.bfloat16 and r16 < 0.004 and r16 < 0.5 * r8


# ---------------------------------------------------------------------------------------------- epilogue rounding
def _gemm(xq, xs, w8, s_ch, mode, odt, bias=None):
    m, k = xq.shape
    n = w8.shape[0]
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.F32: torch.float32}[odt]
    out = torch.empty(m, n, dtype=dt, device=DEV)
    acc = torch.empty(m, n, dtype=torch.int32, device=DEV)
    lib = _lib.load()
    _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, s_ch.data_ptr(), _lib.ptr(bias), m, n, k,
                                 _lib.MODE[mode], out.data_ptr(), odt, n, acc.data_ptr(), _lib.stream_of(DEV)), "gemm")
    return out, acc


def test_epilogue_keeps_the_fp32_rounding_before_narrowing():
    """acc * (xs * s_ch) rounds to fp32 exactly on an f16 tie (23.5078125); the reference then rounds to even
    (23.5).  A fused multiply-and-narrow would round the exact product once (23.515625)."""
    a = torch.zeros(1, 16, dtype=torch.int8)
    w = torch.zeros(1, 16, dtype=torch.int8)
    a[0, :6] = torch.tensor([127, 127, 127, 127, 127, 5], dtype=torch.int8)
    w[0, :6] = torch.tensor([127, 127, 127, 127, 60, 10], dtype=torch.int8)
    xs = torch.tensor([[0.02083846]], dtype=torch.float32)
    sc = torch.tensor([0.015627649], dtype=torch.float32)
    out, acc = _gemm(a.to(DEV), xs.to(DEV), w.to(DEV), sc.to(DEV), "eager", _lib.F16)
    assert acc.item() == 72186
    assert out.float().item() == 23.5
    assert out.float().item() == ref.epilogue(np.array([[72186]], np.int32), xs.numpy(), sc.numpy(), "f16", "eager")[0, 0]


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
def test_epilogue_matches_the_oracle_on_random_accumulators(mode, odt):
    g = torch.Generator().manual_seed(odt * 7 + (mode == "eager"))
    m, n, k = 512, 520, 1024
    xq = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    xs = (torch.rand(m, 1, generator=g) * 0.05 + 1e-4)
    sc = (torch.rand(n, generator=g) * 0.03 + 1e-4)
    name = {_lib.BF16: "bf16", _lib.F16: "f16", _lib.F32: "f32"}[odt]
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.F32: torch.float32}[odt]
    bias = torch.randn(n, generator=g).to(dt)
    out, acc = _gemm(xq.to(DEV), xs.to(DEV), w8.to(DEV), sc.to(DEV), mode, odt, bias.to(DEV))
    want_acc = ref.int8_mm(xq.numpy(), w8.numpy())
    assert np.array_equal(acc.cpu().numpy(), want_acc)
    want = ref.epilogue(want_acc, xs.numpy(), sc.numpy(), name, mode, bias.float().numpy())
    assert np.array_equal(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("heads,hd,m,n", [(40, 128, 300, 256), (4, 64, 33, 72), (2, 256, 7, 40), (16, 16, 1, 24),
                                          (40, 128, 2049, 512)])
def test_linear_heads_equals_linear_on_the_transposed_input(heads, hd, m, n):
    """The out projection reading the head-major attention output equals the transpose + reshape + linear of the
    reference (h3turbo/h3/model.py:226-228): bit-exact outputs, including the row-split quantiser for few rows."""
    print(f"linear_heads heads={heads} hd={hd} m={m} n={n}", flush=True)
    k = heads * hd
    w = random_weight_gpu(n, k, seed=heads + hd)
    g = torch.Generator(device=DEV).manual_seed(m)
    big = (torch.randn(heads, m + 5, hd, generator=g, device=DEV) * 3).to(torch.bfloat16)
    xh = big[:, 2:2 + m]  # a strided view: head stride (m + 5) * hd, token stride hd
    want = ql.linear(xh.transpose(0, 1).reshape(m, k), w)
    got = ql.linear_heads(xh, w)
    assert torch.equal(got, want)
    for mode in ("ck", "eager"):
        assert torch.equal(ql.linear_heads(xh.contiguous(), w, quant_mode=mode),
                           ql.linear(xh.transpose(0, 1).reshape(m, k), w, quant_mode=mode))
