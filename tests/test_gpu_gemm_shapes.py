"""The GEMM kernels (persistent and pipelined on 256 x 256 tiles where at least 160 such tiles exist on 256 CUs;
the same pipeline on 64 x 64, 64 x 128, 128 x 128 (two K groups of wavefronts when the tiles fit in one round) or
128 x 256 tiles below that; the register-staged kernel for K
not a multiple of 64) against the CPU oracle
on whole outputs: ragged M and N tails, K-step counts that do not divide the pipeline depth, every epilogue
variant (ck / eager, bf16 / f16 / f32 out, bias, the int32 accumulator dump, unaligned output strides), and grids
where every persistent workgroup walks several tiles (full tiles only, and full tiles mixed with cut ones).
Bit-exact."""
import numpy as np
import pytest
import torch

from h3turbo_amd import _lib
from oracle import qlinear_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
ODT = {_lib.BF16: (torch.bfloat16, "bf16"), _lib.F16: (torch.float16, "f16"), _lib.F32: (torch.float32, "f32")}


def run(m, n, k, mode, odt, with_bias, ldo_pad=0, acc=False, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=DEV)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=DEV)
    xs = torch.rand(m, generator=g, device=DEV) * 1e-2 + 1e-4
    sch = torch.rand(n, generator=g, device=DEV) * 1e-2 + 1e-4
    tdt, name = ODT[odt]
    bias = (torch.randn(n, generator=g, device=DEV)).to(tdt) if with_bias else None
    ldo = n + ldo_pad
    out = torch.full((m, ldo), -7.0, dtype=tdt, device=DEV)
    accb = torch.empty(m, n, dtype=torch.int32, device=DEV) if acc else None
    lib = _lib.load()
    _lib.check(lib.h3k_gemm_a8w8(a.data_ptr(), k, xs.data_ptr(), w.data_ptr(), k, sch.data_ptr(), _lib.ptr(bias), m, n, k,
                                 _lib.MODE[mode], out.data_ptr(), odt, ldo, _lib.ptr(accb), _lib.stream_of(DEV)), "gemm")
    torch.cuda.synchronize()
    want_acc = ref.int8_mm(a.cpu().numpy(), w.cpu().numpy())
    b = None if bias is None else bias.float().cpu().numpy()
    want = ref.epilogue(want_acc, xs.cpu().numpy(), sch.cpu().numpy(), name, mode, b)
    got = out[:, :n].float().cpu().numpy()
    assert np.array_equal(got, want), f"outputs differ in {(got != want).sum()} places"
    if ldo_pad:
        assert (out[:, n:].float() == -7.0).all(), "wrote past the row"
    if acc:
        assert np.array_equal(accb.cpu().numpy(), want_acc)


@pytest.mark.parametrize("m,n,k", [(4100, 2600, 640), (4100, 2602, 192), (2304, 4500, 576), (4200, 2560, 64)])
def test_large_kernels_ragged_shapes_bf16(m, n, k):
    # 160-187 tiles of 256 x 256: persistent kernel (K >= 512, N % 4 == 0), per-tile pipeline otherwise
    print(f"gemm m={m} n={n} k={k}", flush=True)
    run(m, n, k, "ck", _lib.BF16, False)


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
@pytest.mark.parametrize("with_bias", [False, True])
def test_large_kernels_every_epilogue(mode, odt, with_bias):
    run(4100, 2600, 640, mode, odt, with_bias, seed=3)  # persistent kernel
    run(4100, 2602, 192, mode, odt, with_bias, seed=8)  # per-tile pipeline


@pytest.mark.parametrize("m,n,k", [(200, 700, 320), (512, 5120, 576), (77, 130, 1040), (512, 8320, 256), (300, 16400, 128),
                                   (1100, 520, 640), (700, 256, 64), (513, 1028, 1344), (2304, 768, 192),
                                   (1030, 5000, 512), (600, 3000, 320), (4000, 5100, 192), (1, 300, 256), (5, 4100, 192),
                                   (16, 2048, 1024), (256, 5120, 768), (512, 5120, 1024), (520, 4100, 640),
                                   (640, 4500, 128)])
def test_small_m_kernel_tile_shapes(m, n, k):
    # tile shapes picked by tile count on 256 CUs: (200, 700), (1100, 520), (700, 256), (513, 1028) 64 x 64;
    # (2304, 768), (600, 3000), (256, 5120) 64 x 128 -- the last with 12 K-steps, two per barrier in steady state, so
    # stage pairs straddle the wrap of the 5-stage ring; (512, 5120), (512, 8320) 128 x 128 (160 tiles but 9 K-steps,
    # and 260 tiles: one K group); (512, 5120, 1024), (520, 4100), (640, 4500) 128 x 128 with two K groups -- 16, 10
    # and 2 K-steps, the last shorter than the 6-stage ring; (300, 16400), (1030, 5000) 128 x 256;
    # (4000, 5100): 320 tiles of 256 x 256 would leave the second round mostly idle, so 128 x 256;
    # 1, 5 and 16 rows: 64 x 64 tiles whose rows past M repeat the last row;
    # K=1040 is not a multiple of 64 (register-staged kernel)
    run(m, n, k, "ck", _lib.BF16, False, seed=m + n)


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
def test_small_m_kernel_every_epilogue(mode, odt):
    run(130, 600, 448, mode, odt, True, ldo_pad=8, acc=True, seed=3)  # 64 x 64 tiles
    run(260, 4000, 256, mode, odt, True, ldo_pad=8, acc=True, seed=5)  # 64 x 128 tiles
    run(260, 4000, 768, mode, odt, True, ldo_pad=8, acc=True, seed=9)  # 64 x 128 tiles, 12 K-steps (steady pairs)
    run(520, 4100, 384, mode, odt, True, ldo_pad=8, acc=True, seed=11)  # 128 x 128 tiles, two K groups
    run(384, 11000, 192, mode, odt, True, ldo_pad=8, acc=True, seed=4)  # 128 x 128 tiles
    run(500, 13000, 320, mode, odt, True, ldo_pad=8, acc=True, seed=6)  # 128 x 256 tiles
    run(130, 600, 464, mode, odt, True, ldo_pad=8, acc=True, seed=7)  # K % 64 != 0: register-staged kernel


@pytest.mark.parametrize("m,n,k", [(6144, 8448, 512), (5000, 8000, 576)])
def test_persistent_kernel_walks_several_tiles_per_workgroup(m, n, k):
    print(f"gemm m={m} n={n} k={k}", flush=True)
    run(m, n, k, "ck", _lib.BF16, False, seed=7)


def test_large_kernels_accumulator_dump_and_unaligned_output_rows():
    run(4100, 2600, 640, "ck", _lib.BF16, True, ldo_pad=1, acc=True, seed=4)
    run(4100, 2604, 256, "eager", _lib.F32, False, ldo_pad=3, acc=True, seed=5)
    run(1030, 772, 256, "eager", _lib.F32, False, ldo_pad=3, acc=True, seed=5)  # 64 x 64 tiles
