"""The "a16" W4A8 linear (unquantised activations, reference h3turbo/h3/qlinear.py:407-424) on the hand-written 16-bit
MFMA GEMM (h3k_gemm_a16), and dequantize (qlinear.py:207-226), against the oracle.

* h3k_gemm_a16 through the C ABI on integer-valued activations: every fp32 partial sum is an exact integer below
  2^24, so any accumulation order gives the exact sum and the output must equal the oracle's epilogue bit for bit
  (ragged M, N and K, bias, every output dtype, bf16 and f16 activations).
* qlinear.linear(precision="a16") on Gaussian + outlier activations: within the fp32 accumulation bound
  K * 2^-24 * sum|xr * level| * |s_ch| (plus half an output ulp) of the oracle's exact-sum result.
* dequantize: rotated=True is the fp32 product grid * s_ch bit for bit; rotated=False is within fp32 matmul error
  of the oracle's fp64 dense weight (oracle.block_ref.dense_of).
"""
import numpy as np
import pytest
import torch

import inputs as gi
from h3turbo_amd import _lib
from h3turbo_amd import qlinear as ql
from oracle import block_ref as br
from oracle import qlinear_ref as ref
from test_gpu_qlinear import make_w

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TD = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
CODE = {"bf16": _lib.BF16, "f16": _lib.F16, "f32": _lib.F32}


@pytest.mark.parametrize("m,n,k", [(1, 64, 16), (130, 200, 1024), (300, 1000, 5120), (257, 129, 48)])
@pytest.mark.parametrize("adt", ["bf16", "f16"])
def test_a16_gemm_is_exact_on_integer_activations(m, n, k, adt):
    print(f"a16 gemm m={m} n={n} k={k} {adt}", flush=True)
    rng = np.random.default_rng(m * 31 + n + k)
    xa = rng.integers(-16, 17, (m, k)).astype(np.float32)  # exact in bf16 / f16; |partial sums| < 2^24
    w8 = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s_ch = (rng.random(n) * 0.02 + 1e-3).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    acc = xa.astype(np.int64) @ w8.astype(np.int64).T
    a = torch.from_numpy(xa).to(TD[adt]).to(DEV)
    w = torch.from_numpy(w8).to(DEV)
    sch = torch.from_numpy(s_ch).to(DEV)
    lib = _lib.load()
    for odt in ("bf16", "f16", "f32"):
        for b in (None, bias):
            out = torch.full((m, n), float("nan"), dtype=TD[odt], device=DEV)
            bt = None if b is None else torch.from_numpy(b).to(DEV)
            _lib.check(lib.h3k_gemm_a16(a.data_ptr(), CODE[adt], k, w.data_ptr(), k, sch.data_ptr(),
                                        _lib.ptr(bt), m, n, k, out.data_ptr(), CODE[odt], n, _lib.stream_of(DEV)), "a16")
            y = (acc.astype(np.float32) * s_ch[None, :]).astype(np.float32)
            if b is not None:
                y = (y + b[None, :]).astype(np.float32)
            want = ref.round_to(y, odt)
            assert np.array_equal(out.float().cpu().numpy(), want), (odt, b is None)


def test_a16_gemm_rejects_what_it_does_not_serve():
    lib = _lib.load()
    assert lib.h3k_gemm_a16(None, _lib.F32, 64, None, 64, None, None, 4, 4, 64, None, _lib.BF16, 4, None) == _lib.EINVAL
    assert lib.h3k_gemm_a16(None, _lib.BF16, 40, None, 40, None, None, 4, 4, 40, None, _lib.BF16, 4, None) == _lib.EINVAL


@pytest.mark.parametrize("adt", ["bf16", "f16"])
@pytest.mark.parametrize("m", [3, 300])
def test_linear_a16_within_the_fp32_accumulation_bound(adt, m):
    n, k = 768, 5120
    q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=21)
    w = make_w(q, s_rel, "f16", s_ch, cb, 128, 256)
    xb = gi.activations(m, k, seed=22)  # bf16 bits, Gaussian with outlier channels
    x = torch.from_numpy(xb.view(np.int16).copy()).view(torch.bfloat16).to(TD[adt])
    bias = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(TD[adt])
    got = ql.linear(x.to(DEV), w, bias.to(DEV), precision="a16", out_dtype=torch.float32)
    want, exact, abs_sum = ref.linear_a16(x.float().numpy(), adt, q, s_rel, "f16", s_ch, cb, 128, 256,
                                          out_dtype="f32", bias=bias.float().numpy())
    bound = (k * 2.0 ** -24 * abs_sum + 2.0 ** -24 * np.abs(exact)) * s_ch[None, :] * 1.01 + 1e-6 * np.abs(want)
    err = np.abs(got.cpu().numpy().astype(np.float64) - want)
    assert (err <= bound + 1e-30).all(), float((err / (bound + 1e-30)).max())
    assert float(np.abs(got.cpu().numpy() - want).max()) < 1e-2 * float(np.sqrt((want ** 2).mean()))


def test_dequantize_against_the_oracle():
    n, k = 300, 1024
    q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=5)
    w = make_w(q, s_rel, "f16", s_ch, cb, 128, 256)
    grid = ref.decode_int8_grid(q, s_rel, "f16", cb, 128)
    rot = ql.dequantize(w, torch.float32, rotated=True).cpu().numpy()
    assert np.array_equal(rot, (grid.astype(np.float32) * s_ch[:, None]).astype(np.float32))
    dense = ql.dequantize(w, torch.float32, rotated=False).cpu().double()
    want = br.dense_of({"q": q, "s_rel": s_rel, "s_kind": "f16", "cb": cb, "group": 128, "s_ch": s_ch,
                        "convrot": 256})
    # fp32 grid * s_ch (one rounding) and a 256-term fp32 matmul against the fp64 definition
    bound = (256 * 2.0 ** -24 + 2.0 ** -24) * (np.abs(grid) * s_ch[:, None]).max() * 16 + 1e-12
    assert float((dense - want).abs().max()) <= bound
    rows = ql.dequantize(w, torch.float32, rotated=False, rows=slice(7, 19)).cpu().double()
    assert float((rows - want[7:19]).abs().max()) <= bound
