"""The fused few-row W4A8 GEMM (h3k_gemm_w4a8: int4 decoded in registers, no int8 grid) through the C ABI, against
the CPU oracle (decode_int8_grid, int8_mm, epilogue): every row count up to 128, ragged N, one K split and many, all
group kinds (16, 32, multiples of 64), every scale dtype, NaN / clamp scales, both epilogue orders, every output
dtype, bias, the accumulator dump, padded output rows; both kernels of up to 32 rows (32-row MFMA tiles for narrow N
or K not a multiple of 128, 16-row tiles for up to 16 rows otherwise).  Bit-exact."""
import numpy as np
import pytest
import torch

import inputs as gi
from h3turbo_amd import _lib
from oracle import qlinear_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
ODT = {_lib.BF16: (torch.bfloat16, "bf16"), _lib.F16: (torch.float16, "f16"), _lib.F32: (torch.float32, "f32")}
SKIND = {"fp8": _lib.scale_code(torch.float8_e4m3fn), "f16": _lib.scale_code(torch.float16),
         "bf16": _lib.scale_code(torch.bfloat16), "f32": _lib.scale_code(torch.float32)}


def scales(n, k, group, kind, g):
    """Raw scale storage [n, k/group] (numpy) with a NaN and a clamp-provoking entry."""
    v = 20 + 180 * torch.rand(n, k // group, generator=g)
    v[0, 0] = float("nan")
    v[-1, -1] = 448.0
    if kind == "fp8":
        return v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    if kind == "f16":
        return v.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    if kind == "bf16":
        return ref.bf16_bits(v.numpy())
    return v.numpy().astype(np.float32)


def scale_tensor(raw, kind):
    t = torch.from_numpy(np.ascontiguousarray(raw))
    return {"fp8": lambda: t.view(torch.float8_e4m3fn), "f16": lambda: t.view(torch.int16).view(torch.float16),
            "bf16": lambda: t.view(torch.int16).view(torch.bfloat16), "f32": lambda: t}[kind]().to(DEV)


def run(m, n, k, group=128, kind="f16", mode="ck", odt=_lib.BF16, with_bias=False, acc=False, ldo_pad=0, seed=0,
        special=False):
    print(f"w4 gemm m={m} n={n} k={k} g={group} {kind} {mode} odt={odt} bias={with_bias}", flush=True)
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8).numpy()
    s_raw = scales(n, k, group, kind, g)
    cb = (torch.linspace(-1, 1, 16) + 0.05 * torch.randn(16, generator=g)).float().numpy()
    if special:  # non-finite and zero codebook entries, infinite scales: NaN products must decode to 0
        cb[3], cb[5], cb[7], cb[8] = np.inf, -np.inf, np.nan, 0.0
        if kind == "fp8":  # e4m3fn has no infinity: NaN bytes (both signs) and zero instead
            s_raw[1, :] = 0x7F
            s_raw[2, 0] = 0xFF
            s_raw[3, :] = 0x00
        else:
            s_raw[1, :] = np.inf
            s_raw[2, 0] = -np.inf
    xs = torch.rand(m, generator=g) * 1e-2 + 1e-4
    sch = torch.rand(n, generator=g) * 1e-2 + 1e-4
    tdt, name = ODT[odt]
    bias = torch.randn(n, generator=g).to(tdt) if with_bias else None
    lib = _lib.load()
    ldo = n + ldo_pad
    out = torch.full((m, ldo), -7.0, dtype=tdt, device=DEV)
    accb = torch.empty(m, n, dtype=torch.int32, device=DEV) if acc else None
    nbytes = lib.h3k_gemm_w4a8_workspace(m, n, k)
    ws = torch.full((max(1, nbytes // 4),), 12345, dtype=torch.int32, device=DEV) if nbytes else None
    ad, qd = a.to(DEV), torch.from_numpy(q).to(DEV)
    sd, cbd = scale_tensor(s_raw, kind), torch.from_numpy(cb).to(DEV)
    xsd, schd = xs.to(DEV), sch.to(DEV)
    bd = None if bias is None else bias.to(DEV)
    _lib.check(lib.h3k_gemm_w4a8(ad.data_ptr(), k, xsd.data_ptr(), qd.data_ptr(), k // 2, sd.data_ptr(), SKIND[kind],
                                 k // group, cbd.data_ptr(), group, schd.data_ptr(), _lib.ptr(bd), m, n, k,
                                 _lib.MODE[mode], out.data_ptr(), odt, ldo, _lib.ptr(ws), _lib.ptr(accb),
                                 _lib.stream_of(DEV)), "h3k_gemm_w4a8")
    torch.cuda.synchronize()
    w8 = ref.decode_int8_grid(q, s_raw, kind, cb, group)
    want_acc = ref.int8_mm(a.numpy(), w8)
    want = ref.epilogue(want_acc, xs.numpy(), sch.numpy(), name, mode, None if bias is None else bias.float().numpy())
    got = out[:, :n].float().cpu().numpy()
    assert np.array_equal(got, want), f"outputs differ in {(got != want).sum()} of {got.size} places"
    if ldo_pad:
        assert (out[:, n:].float() == -7.0).all(), "wrote past the row"
    if acc:
        assert np.array_equal(accb.cpu().numpy(), want_acc)
    return nbytes


@pytest.mark.parametrize("m", [1, 5, 31, 32, 33, 64, 65, 100, 128])
def test_every_row_count(m):
    run(m, 200, 1024, group=128, seed=m)


@pytest.mark.parametrize("group,kind", [(16, "fp8"), (32, "bf16"), (64, "f32"), (128, "f16"), (256, "fp8"),
                                        (512, "f16"), (16, "f16"), (32, "fp8")])
def test_groups_and_scale_kinds(group, kind):
    run(37, 130, 2048, group=group, kind=kind, seed=group)


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
def test_epilogue_variants(mode, odt):
    run(24, 96, 512, group=16, kind="fp8", mode=mode, odt=odt, with_bias=True, acc=True, ldo_pad=8, seed=3)


@pytest.mark.parametrize("group", [16, 128])
def test_non_finite_codebook_and_scales(group):
    run(20, 64, 1024, group=group, kind="f32", seed=11, special=True)
    run(70, 64, 1024, group=group, kind="f32", seed=12, special=True)


def test_split_and_unsplit_k():
    # few columns and long K: many K splits accumulate through the workspace; short K: one split, fused epilogue
    assert run(64, 256, 5120, group=128, acc=True, seed=5) > 0
    assert run(64, 256, 256, group=128, acc=True, seed=6) == 0
    assert run(128, 640, 5120, group=128, seed=7) > 0  # BASELINE K, 5 column tiles x 10 splits


# 16-row MFMA tiles (gemm_w4_c16_kernel): up to 16 rows, K a multiple of 128, at least 128 tiles of 32 columns; the
# same shapes with 17-32 rows run on the 32-row column kernel.
C16_N = 4100  # 129 column tiles, the last one ragged


@pytest.mark.parametrize("m", [1, 7, 16, 17, 32])
def test_c16_every_row_group(m):
    run(m, C16_N, 1152, group=128, seed=100 + m)  # 9 super-steps over 8 wavefronts: uneven K split


@pytest.mark.parametrize("group,kind", [(16, "fp8"), (32, "bf16"), (32, "fp8"), (64, "f32"), (128, "f16"),
                                        (256, "fp8"), (512, "f16"), (384, "bf16")])
def test_c16_groups_and_scale_kinds(group, kind):
    k = 1536 if group == 384 else 1024
    run(13, C16_N, k, group=group, kind=kind, seed=group + 1)
    run(29, C16_N, k, group=group, kind=kind, seed=group + 2)


@pytest.mark.parametrize("k", [128, 640, 5120])
def test_c16_short_and_long_k(k):
    run(16, C16_N, k, group=128, seed=k)  # one super-step (wave 0 alone), fewer than 8, the BASELINE K


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
def test_c16_epilogue_variants(mode, odt):
    run(24, C16_N, 512, group=64, kind="fp8", mode=mode, odt=odt, with_bias=True, acc=True, ldo_pad=8, seed=33)


@pytest.mark.parametrize("group", [16, 64, 128])
def test_c16_non_finite_codebook_and_scales(group):
    run(9, C16_N, 1024, group=group, kind="f32", seed=41, special=True)
    run(30, C16_N, 1024, group=group, kind="f32", seed=42, special=True)


@pytest.mark.parametrize("group", [16, 32])
def test_fp8_scale_table_with_non_finite_codebook(group):
    """fp8 scales of groups 16 and 32 take their level tables from a per-workgroup table of all 256 scale bytes
    (16-row and column kernels): non-finite codebook entries, NaN scale bytes of both signs and zero scales."""
    run(9, C16_N, 1024, group=group, kind="fp8", seed=43, special=True)
    run(16, C16_N, 5120, group=group, kind="fp8", seed=44, special=True)
    run(30, C16_N, 5120, group=group, kind="fp8", seed=45, special=True)  # column kernel, one K split
    run(20, 64, 1024, group=group, kind="fp8", seed=46, special=True)  # column kernel, K split over workgroups


def test_rejects_what_it_does_not_cover():
    lib = _lib.load()
    dummy = torch.zeros(64, dtype=torch.int32, device=DEV)
    p = dummy.data_ptr()
    args = lambda m, n, k, group, ws: (p, k, p, p, k // 2, p, SKIND["f16"], max(1, k // group), p, group, p, None, m,  # noqa: E731
                                       n, k, 0, p, _lib.BF16, n, ws, None, _lib.stream_of(DEV))
    assert lib.h3k_gemm_w4a8(*args(129, 64, 512, 128, p)) != 0  # too many rows
    assert lib.h3k_gemm_w4a8(*args(8, 64, 544, 32, p)) != 0  # k not a multiple of 64
    assert lib.h3k_gemm_w4a8(*args(8, 64, 512, 8, p)) != 0  # group 8
    assert lib.h3k_gemm_w4a8(*args(8, 64, 4096, 128, None)) != 0  # splits K without a workspace
    assert "workspace" in lib.h3k_last_error().decode()
