"""Rotation sizes beyond the reference's powers of 4 (BASELINE configs 1-2 name block-Hadamard 128): the HIP
rotation and rotate+quantise kernels against the oracle's definition (oracle.qlinear_ref.hadamard_pow2 /
rotation_scale, pinned in tests/test_oracle.py), bit for bit: the fast path (rotation 128, bf16/f16, aligned
rows, K a multiple of 256) and the generic path (f32, unaligned rows, sizes 8/32/512); config 2's shape at rotation
128 on sampled rows; and the W4A8 linear with a rotation-128 weight against the oracle's linear."""
import numpy as np
import pytest
import torch

import inputs as gi
from h3turbo_amd import qlinear as ql
from oracle import qlinear_ref as ref
from test_gpu_qlinear import make_w

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
DTS = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _check(x: torch.Tensor, rot: int):
    xv = x.float().numpy()
    name = DTS[x.dtype]
    for mode in ("ck", "eager"):
        q, s = ql.quantize_activation(x.to(DEV), size=rot, quant_mode=mode)
        qr, sr = ref.quantize_rows(xv, name, rot, mode)
        assert np.array_equal(s.cpu().numpy(), sr), (rot, mode)
        assert np.array_equal(q.cpu().numpy(), qr), (rot, mode)
    y = ql.rotate(x.to(DEV), size=rot)
    assert y.dtype == x.dtype and np.array_equal(y.float().cpu().numpy(), ref.round_to(ref.rotate_f32(xv, rot), name))


@pytest.mark.parametrize("rot", [8, 32, 128, 512])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_extension_sizes_match_the_oracle(rot, dt):
    print(f"rotation {rot} {dt}", flush=True)
    x = (torch.randn(10, 2048, generator=torch.Generator().manual_seed(rot)) * 3).to(dt)
    _check(x, rot)


def test_rotation128_fast_and_generic_paths_agree_with_the_oracle():
    g = torch.Generator().manual_seed(5)
    # aligned bf16 rows, K a multiple of 256: the fast kernel; many rows so several workgroups run
    x = (torch.randn(300, 5120, generator=g) * torch.logspace(-3, 2, 300).unsqueeze(1)).to(torch.bfloat16)
    _check(x, 128)
    # K = 384 (not a multiple of 256): the generic kernel
    _check(torch.randn(7, 384, generator=g).to(torch.bfloat16), 128)
    # rows at an odd element offset (not 16-byte aligned): the generic kernel on a view
    big = torch.randn(9, 1024 + 1, generator=g).to(torch.float16)
    x = big[:, 1:]
    for mode in ("ck", "eager"):
        q, s = ql.quantize_activation(x.to(DEV), size=128, quant_mode=mode)
        qr, sr = ref.quantize_rows(x.float().numpy(), "f16", 128, mode)
        assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(q.cpu().numpy(), qr), mode


def test_config2_shape_at_rotation_128_on_sampled_rows():
    """bf16 [12090, 5120], ~N(0,1) with 1 % outlier channels x20, rotation 128, per-token int8;
    the whole tensor on the GPU, 600 rows (the first 300 and 300 scattered ones) against the oracle."""
    m, k = 12090, 5120
    xb = gi.activations(m, k, seed=0)  # bf16 bits
    x = torch.from_numpy(xb.view(np.int16).copy()).view(torch.bfloat16)
    q, s = ql.quantize_activation(x.to(DEV), size=128)
    rows = np.concatenate([np.arange(300), np.random.default_rng(1).choice(np.arange(300, m), 300, replace=False)])
    qr, sr = ref.quantize_rows(ref.bf16_from_bits(xb[rows]), "bf16", 128, "ck")
    assert np.array_equal(s.cpu().numpy()[rows], sr) and np.array_equal(q.cpu().numpy()[rows], qr)


@pytest.mark.parametrize("m", [5, 300])
def test_w4a8_linear_with_a_rotation_128_weight(m):
    n, k = 512, 1024
    q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=9)
    w = make_w(q, s_rel, "f16", s_ch, cb, 128, 128)
    xb = gi.activations(m, k, seed=10)
    x = torch.from_numpy(xb.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    for mode in ("ck", "eager"):
        got = ql.linear(x, w, quant_mode=mode)
        want, *_ = ref.linear_a8(ref.bf16_from_bits(xb), "bf16", q, s_rel, "f16", s_ch, cb, 128, 128, mode=mode)
        assert np.array_equal(got.float().cpu().numpy(), want), mode
