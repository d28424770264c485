"""Rotate + quantise with the MLP activation fused into its loads (h3k_rotate_quant_act) through the C ABI.

The unfused chain is the reference's: the activation as torch ops in x.dtype (silu(gate) * up, qlinear.py:376-379;
tanh-approximate GELU for the config-4 block), then rotate + quantise (qlinear.py:295-303).  The fused kernel
evaluates the same fp32 formula and rounds where torch rounds, so its int8 rows and fp32 scales equal the chain's
bit for bit; the swiglu golden vector (the reference's CPU activation) pins the chain itself.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fixtures as fx
from h3turbo_amd import _lib
from h3turbo_amd import qlinear as ql
from oracle import qlinear_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def unfused(x: torch.Tensor, act: str, mode: str):
    return ql.quantize_activation(ql.apply_input_act(x, act), quant_mode=mode)


def fused(x: torch.Tensor, act: str, mode: str):
    k = x.shape[-1] // (2 if act == "swiglu" else 1)
    return ql._quantize_rows_act(x, ql.ACT_CODE[act], k, mode)


def assert_same(got, want, what):
    (q, s), (qw, sw) = got, want
    bad_s = (s.view(-1).view(torch.int32) != sw.view(-1).view(torch.int32)).sum().item()  # NaN scales compare too
    bad_q = (q != qw).sum().item()
    assert bad_s == 0 and bad_q == 0, f"{what}: {bad_s} scales and {bad_q} of {q.numel()} levels differ"


@pytest.mark.parametrize("act", ["swiglu", "gelu_tanh"])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("m,k", [(1, 256), (7, 1280), (300, 5120), (64, 13824)])
def test_fused_activation_equals_the_torch_ops(act, dt, mode, m, k):
    print(f"act-quant {act} {dt} {mode} m={m} k={k}", flush=True)
    width = 2 * k if act == "swiglu" else k
    g = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn(m, width, generator=g) * 2.5).to(dt).to(DEV)
    assert_same(fused(x, act, mode), unfused(x, act, mode), f"{act} {dt} {mode} {m}x{k}")


@pytest.mark.parametrize("act", ["swiglu", "gelu_tanh"])
def test_extreme_values_and_strided_rows(act):
    """Saturating and tiny inputs (exp overflow, tanh saturation, subnormal products) in rows that are views into a
    wider buffer: the fused kernel reads only the row's own width."""
    k = 512
    width = 2 * k if act == "swiglu" else k
    g = torch.Generator().manual_seed(5)
    base = torch.randn(9, width + 64, generator=g) * 3
    base[0, :width] = torch.linspace(-90, 90, width)
    base[1, :width] = torch.linspace(-1e-3, 1e-3, width)
    base[2, :width] = 0.0
    base[3, :width:2] = 1e4
    for dt in (torch.bfloat16, torch.float16):
        xb = base.to(dt).to(DEV)
        x = xb[:, :width]
        for mode in ("ck", "eager"):
            assert_same(fused(x, act, mode), unfused(x.contiguous(), act, mode), f"{act} {dt} {mode}")


def test_gelu_on_every_bf16_value():
    """Every finite bf16 value through the bf16 GELU path (a table of the in-kernel formula, filled on the GPU on
    first use) against the torch ops: 64 rows of 1024, each row one slice of the 65 280 finite codes (padded with
    zeros), so every code is quantised once, and the row maxima span the whole exponent range."""
    codes = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    finite = codes[torch.isfinite(codes.float())]
    x = torch.zeros(64 * 1024, dtype=torch.bfloat16)
    x[: finite.numel()] = finite
    x = x.view(64, 1024).to(DEV)
    for mode in ("ck", "eager"):
        assert_same(fused(x, "gelu_tanh", mode), unfused(x, "gelu_tanh", mode), f"every bf16 value, {mode}")


def test_swiglu_golden_vector_pins_the_chain():
    """The reference's own CPU activation for the swiglu golden case, rotated and quantised by the oracle, against
    the fused kernel on the same bf16 input."""
    meta, a = fx.load("swiglu_m9_k512_n40")
    h = torch.from_numpy(np.ascontiguousarray(a["h"]).view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    act = ql._swiglu(h)
    act_bits = act.cpu().view(torch.int16).numpy().view(np.uint16)
    if not np.array_equal(act_bits, a["act"]):
        pytest.skip("torch's GPU silu differs from the reference's CPU one on this vector")
    k = h.shape[-1] // 2
    for mode in ("ck", "eager"):
        q, s = fused(h, "swiglu", mode)
        qr, sr = ref.quantize_rows(fx.out_values(a["act"], "bf16"), "bf16", 256, mode)
        assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy().reshape(-1), sr.reshape(-1))
        assert q.shape == (h.shape[0], k)


@pytest.mark.parametrize("act", ["swiglu", "gelu_tanh"])
def test_linear_routes_the_activation_through_the_fused_kernel(act, monkeypatch):
    """qlinear.linear(x, w, input_act=act) on the W4A8 a8 path equals linear(act(x), w) bit for bit, in both GEMM
    routes (few rows and many), and does not evaluate the activation as torch ops."""
    import inputs as gi
    from test_gpu_qlinear import make_w

    k, n = 1024, 96
    q, s8, s_ch, cb = gi.weight_fp8_g16(n, k, seed=3)
    w = make_w(q, s8, "fp8", s_ch, cb, 16, 256)
    width = 2 * k if act == "swiglu" else k
    for m in (16, 700):
        x = (torch.randn(m, width, generator=torch.Generator().manual_seed(m)) * 2).to(torch.bfloat16).to(DEV)
        want = ql.linear(ql.apply_input_act(x, act), w)
        calls = []
        orig = ql.apply_input_act
        monkeypatch.setattr(ql, "apply_input_act", lambda t, a: (calls.append(a), orig(t, a))[1])
        got = ql.linear(x, w, input_act=act)
        monkeypatch.setattr(ql, "apply_input_act", orig)
        assert torch.equal(got, want), f"m={m}"
        assert all(c is None for c in calls), f"activation ran as torch ops: {calls}"
    # f32 input: not covered by the fused kernel, the torch ops run first and the result is the same chain
    x = torch.randn(5, width, generator=torch.Generator().manual_seed(1)).to(DEV)
    assert torch.equal(ql.linear(x, w, input_act=act), ql.linear(ql.apply_input_act(x, act), w))


def test_gelu_matches_torch_gelu_elementwise():
    """Rows of powers of two from 2^-20 to 2^7, both signs (GELU's linear, curved and saturated ranges): the fused
    and unfused chains quantise them identically."""
    vals = torch.tensor([2.0 ** e for e in range(-20, 8)] + [-(2.0 ** e) for e in range(-20, 8)])
    x = vals.repeat_interleave(256 // 8).reshape(-1, 256)[:, :256].to(torch.bfloat16).to(DEV)
    for mode in ("ck", "eager"):
        assert_same(fused(x, "gelu_tanh", mode), unfused(x, "gelu_tanh", mode), mode)
    y = F.gelu(x.float(), approximate="tanh")
    assert torch.isfinite(y).all()

