"""The packed int8 weight grid and the large-shape GEMM that reads it (h3k_decode_w4_packed, h3k_pack_w8,
h3k_gemm_a8w8_packed).

Layout: K-step t (64 bytes), block b (32 weight rows; n padded to a multiple of 256, NBP = padded n / 32), half h,
lane l -> byte ((t * NBP + b) * 2 + h) * 1024 + l * 16 holds row 32b + (l & 31), bytes 64t + 32(l >> 5) + 16h .. + 16;
rows past n are zero.  Pinned here against a numpy
restatement of that definition on the oracle's row-major grid.  The GEMM is bit-exact against the reference's CUDA
formulation as torch ops (torch._int_mm for the accumulators, h3turbo/h3/qlinear.py:242-247; the ck / eager
epilogue, :399-405) and against h3k_gemm_a8w8 on the row-major grid, on full tiles, tiles cut by M and N, bias,
both quant modes and every output dtype.
"""
import numpy as np
import pytest
import torch

import inputs as gi
from h3turbo_amd import _lib
from oracle import qlinear_ref as ref
from test_gpu_qlinear import random_weight_gpu

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def packed_from_rowmajor(w8: np.ndarray) -> np.ndarray:
    """The packed layout's definition, restated in numpy on a row-major [n, k] grid."""
    n, k = w8.shape
    nb, kt = (n + 255) // 256 * 8, k // 64
    g = np.zeros((nb * 32, k), np.int8)
    g[:n] = w8
    # [nb, 32 rows, kt, 2 (lane >> 5), 2 (h), 16] -> [kt, nb, h, lane >> 5, 32 rows, 16]
    v = g.reshape(nb, 32, kt, 2, 2, 16).transpose(2, 0, 4, 3, 1, 5)
    return np.ascontiguousarray(v).reshape(-1)


def decode_packed(w) -> torch.Tensor:
    lib = _lib.load()
    n, k = w.q.shape[0], w.q.shape[1] * 2
    out = torch.full((lib.h3k_w8_packed_bytes(n, k),), 77, dtype=torch.int8, device=DEV)
    _lib.check(lib.h3k_decode_w4_packed(w.q.data_ptr(), w.q.stride(0), w.s_rel.data_ptr(), _lib.scale_code(w.s_rel.dtype),
                                        w.s_rel.stride(0), w.codebook.data_ptr(), n, k, w.group_size, out.data_ptr(),
                                        _lib.stream_of(DEV)), "decode packed")
    return out


def pack(w8: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    n, k = w8.shape
    out = torch.full((lib.h3k_w8_packed_bytes(n, k),), 77, dtype=torch.int8, device=DEV)
    _lib.check(lib.h3k_pack_w8(w8.data_ptr(), w8.stride(0), n, k, out.data_ptr(), _lib.stream_of(DEV)), "pack")
    return out


@pytest.mark.parametrize("n,k,group,kind", [(37, 256, 16, "fp8"), (64, 512, 128, "f16"), (100, 1024, 32, "fp8"),
                                            (40, 320, 64, "bf16"), (33, 192, 8, "fp8"), (96, 384, 48, "f32")])
def test_packed_decode_is_the_packed_layout_of_the_oracle_grid(n, k, group, kind):
    q, s8, _, cb = gi.weight_fp8_g16(n, k, seed=n + group, group=group)
    sv = ref.fp8_e4m3fn_to_f32(s8)
    s_raw = {"fp8": s8, "f16": sv.astype(np.float16).view(np.uint16), "bf16": ref.bf16_bits(sv), "f32": sv}[kind]
    from test_gpu_qlinear import make_w
    w = make_w(q, s_raw, kind, np.ones(n, np.float32), cb, group, 64)
    want = packed_from_rowmajor(ref.decode_int8_grid(q, s_raw, kind, cb, group))
    got = decode_packed(w)
    assert np.array_equal(got.cpu().numpy(), want)
    w8 = torch.from_numpy(ref.decode_int8_grid(q, s_raw, kind, cb, group)).to(DEV)
    assert np.array_equal(pack(w8).cpu().numpy(), want)


@pytest.mark.parametrize("special", [False, True])
def test_packed_decode_fp8_group16_every_scale_byte(special):
    """fp8 scales of group 16 take their tables from the workgroup's table of all 256 scale bytes: every byte value
    (NaN 0x7F / 0xFF, negatives, zero), with a finite codebook and with infinite / NaN codebook entries."""
    n, k = 300, 512
    rng = np.random.default_rng(7 + special)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8).view(np.int8)
    s = rng.integers(0, 256, (n, k // 16), dtype=np.uint8)
    s.reshape(-1)[:256] = np.arange(256, dtype=np.uint8)
    _, _, _, cb = gi.weight_fp8_g16(4, 64, seed=3)
    if special:
        cb[3], cb[5], cb[7], cb[8] = np.inf, -np.inf, np.nan, 0.0
    from test_gpu_qlinear import make_w
    w = make_w(q, s, "fp8", np.ones(n, np.float32), cb, 16, 64)
    want = packed_from_rowmajor(ref.decode_int8_grid(q, s, "fp8", cb, 16))
    assert np.array_equal(decode_packed(w).cpu().numpy(), want)


def test_packed_layout_restatement_is_a_permutation_within_blocks():
    """The numpy restatement itself, against its defining formula element by element on a small grid."""
    n, k = 45, 128
    w8 = np.random.default_rng(3).integers(-127, 128, (n, k)).astype(np.int8)
    p = packed_from_rowmajor(w8)
    kt, nbp = k // 64, 8
    assert p.size == kt * nbp * 2048
    for b in range(nbp):
        for t in range(kt):
            for h in range(2):
                for lane in range(64):
                    row, c0 = 32 * b + (lane & 31), 64 * t + 32 * (lane >> 5) + 16 * h
                    off = ((t * nbp + b) * 2 + h) * 1024 + lane * 16
                    want = w8[row, c0:c0 + 16] if row < n else np.zeros(16, np.int8)
                    assert np.array_equal(p[off:off + 16], want)


def run_packed(xq, xs, w8p, s_ch, n, mode, odt, bias=None, acc=False, ldo=None):
    m, k = xq.shape
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.F32: torch.float32}[odt]
    ldo = ldo or n
    out_buf = torch.zeros(m, ldo, dtype=dt, device=DEV)
    acc_t = torch.zeros(m, n, dtype=torch.int32, device=DEV) if acc else None
    lib = _lib.load()
    _lib.check(lib.h3k_gemm_a8w8_packed(xq.data_ptr(), k, xs.data_ptr(), w8p.data_ptr(), s_ch.data_ptr(), _lib.ptr(bias),
                                        m, n, k, _lib.MODE[mode], out_buf.data_ptr(), odt, ldo, _lib.ptr(acc_t),
                                        _lib.stream_of(DEV)), "gemm packed")
    return out_buf[:, :n], acc_t


def torch_epilogue(acc, xs, s_ch, mode, dt, bias=None):
    out = torch.empty(acc.shape, dtype=dt, device=DEV)
    if mode == "ck":
        torch.mul(torch.mul(acc, xs), s_ch.reshape(1, -1), out=out)
    else:
        torch.mul(acc, xs * s_ch.reshape(1, -1), out=out)
    if bias is not None:
        out.add_(bias.to(dt))
    return out


# served shapes: at least 160 tiles of 256 x 256 on 256 CUs; cut by M (2000, 4090) and by N (3000, 7000)
SHAPES = [(2048, 5120, 1024), (2000, 5120, 1024), (4096, 3000, 512), (4090, 7000, 768), (8192, 4096, 2048)]


@pytest.mark.parametrize("m,n,k", SHAPES, ids=[f"m{m}_n{n}_k{k}" for m, n, k in SHAPES])
def test_packed_gemm_matches_int_mm_and_the_rowmajor_gemm(m, n, k):
    print(f"packed gemm m={m} n={n} k={k}", flush=True)
    lib = _lib.load()
    assert lib.h3k_gemm_packed_serves(m, n, k) == 1
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    xq = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=DEV)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=DEV)
    xs = torch.rand(m, 1, generator=g, device=DEV) * 0.05 + 1e-4
    s_ch = torch.rand(n, generator=g, device=DEV) * 0.03 + 1e-4
    w8p = pack(w8)
    want_acc = torch._int_mm(xq, w8.t())
    out, acc = run_packed(xq, xs, w8p, s_ch, n, "ck", _lib.BF16, acc=True)
    assert torch.equal(acc, want_acc), "int32 accumulators"
    want = torch_epilogue(want_acc, xs, s_ch, "ck", torch.bfloat16)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), "bf16 (acc_out path)"
    fast, _ = run_packed(xq, xs, w8p, s_ch, n, "ck", _lib.BF16)
    assert torch.equal(fast.view(torch.int16), want.view(torch.int16)), "bf16 (streaming-store path)"
    # the row-major kernel on the same operands
    rm = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, s_ch.data_ptr(), None, m, n, k, 0,
                                 rm.data_ptr(), _lib.BF16, n, None, _lib.stream_of(DEV)), "gemm row-major")
    assert torch.equal(rm.view(torch.int16), fast.view(torch.int16))


@pytest.mark.parametrize("mode", ["ck", "eager"])
@pytest.mark.parametrize("odt", [_lib.BF16, _lib.F16, _lib.F32])
@pytest.mark.parametrize("m,n,k", [(2000, 5120, 512), (4090, 7000, 512)], ids=["cut_m", "cut_m_n_odd_rows"])
def test_packed_gemm_epilogues_bias_and_strided_outputs(mode, odt, m, n, k):
    # whole tiles and tiles cut by M (and N); M % 4 != 0 puts the last xs chunk across the end of xs; ldo = n + 4
    # leaves 16-bit output rows 8-byte aligned only (element stores)
    print(f"packed epilogue mode={mode} odt={odt} m={m} n={n} k={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(odt * 3 + (mode == "eager"))
    xq = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=DEV)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=DEV)
    xs = torch.rand(m, 1, generator=g, device=DEV) * 0.05 + 1e-4
    s_ch = torch.rand(n, generator=g, device=DEV) * 0.03 + 1e-4
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.F32: torch.float32}[odt]
    bias = torch.randn(n, generator=g, device=DEV).to(dt)
    w8p = pack(w8)
    acc = torch._int_mm(xq, w8.t())
    for b in (None, bias):
        for ldo in (n, n + 8, n + 4):
            got, _ = run_packed(xq, xs, w8p, s_ch, n, mode, odt, bias=b, ldo=ldo)
            want = torch_epilogue(acc, xs, s_ch, mode, dt, b)
            assert torch.equal(got.contiguous().view(torch.uint8), want.view(torch.uint8)), (b is not None, ldo)


def test_packed_gemm_on_the_baseline_weight_through_qlinear():
    """A served shape through qlinear.linear (decode into the packed grid + packed GEMM) against the oracle on
    sampled rows and against the row-major route on every element."""
    from h3turbo_amd import qlinear as ql
    from test_gpu_qlinear import np_bits, random_acts_gpu

    m, k, n = 2048, 5120, 5120
    x = random_acts_gpu(m, k, seed=5)
    w = random_weight_gpu(n, k, seed=6)
    lib = _lib.load()
    assert lib.h3k_gemm_packed_serves(m, n, k) == 1
    out = ql.linear(x, w)
    xq, xs = ql.quantize_activation(x)
    w8 = ql.decode_int8_grid(w)
    rm = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, w.s_ch.data_ptr(), None, m, n, k, 0,
                                 rm.data_ptr(), _lib.BF16, n, None, _lib.stream_of(DEV)), "gemm row-major")
    assert torch.equal(out.view(torch.int16), rm.view(torch.int16))
    rows = np.array([0, 1, 777, m - 1])
    xr = x[torch.from_numpy(rows).to(DEV)].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    s_bits = w.s_rel.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    want, *_ = ref.linear_a8(ref.bf16_from_bits(xr), "bf16", w.q.cpu().numpy(), s_bits, "f16", w.s_ch.cpu().numpy(),
                             w.codebook.cpu().numpy(), 128, 256)
    assert np.array_equal(np_bits(out[torch.from_numpy(rows).to(DEV)]), ref.bf16_bits(want))


def test_packed_entry_points_reject_what_they_do_not_serve():
    lib = _lib.load()
    assert lib.h3k_gemm_packed_serves(512, 5120, 5120) == 0  # too few tiles
    assert lib.h3k_gemm_packed_serves(4096, 5120, 5120 + 64) == 0  # K not a multiple of 256
    assert lib.h3k_w8_packed_bytes(33, 128) == 256 * 128 and lib.h3k_w8_packed_bytes(10, 100) == -1
    x = torch.zeros(512, 5120, dtype=torch.int8, device=DEV)
    rc = lib.h3k_gemm_a8w8_packed(x.data_ptr(), 5120, x.data_ptr(), x.data_ptr(), x.data_ptr(), None, 512, 5120, 5120, 0,
                                  x.data_ptr(), _lib.BF16, 5120, None, _lib.stream_of(DEV))
    assert rc == _lib.EINVAL and b"packed" in lib.h3k_last_error()


# Split tail: the last round's tiles cut along K, int32 partial sums added by the fix-up kernel.  Shapes where the
# launch's cost model takes it: one round plus 64 tiles cut by M and N (P = 3), no whole round at all (P = 6), and
# ten rounds plus 32 tiles cut by M (P = 5).
SPLIT = [(4000, 5000, 13824), (512, 5120, 13824), (12090, 13824, 5120)]


def run_packed_ws(xq, xs, w8p, s_ch, n, mode, odt, bias=None, ldo=None, split=True):
    m, k = xq.shape
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.F32: torch.float32}[odt]
    ldo = ldo or n
    out_buf = torch.zeros(m, ldo, dtype=dt, device=DEV)
    lib = _lib.load()
    nbytes = lib.h3k_gemm_packed_split_bytes(m, n, k) if split else 0
    ws = torch.full((max(nbytes, 4) // 4,), -7, dtype=torch.int32, device=DEV)  # stale contents: no zeroing is assumed
    _lib.check(lib.h3k_gemm_a8w8_packed_ws(xq.data_ptr(), k, xs.data_ptr(), w8p.data_ptr(), s_ch.data_ptr(),
                                           _lib.ptr(bias), m, n, k, _lib.MODE[mode], out_buf.data_ptr(), odt, ldo,
                                           ws.data_ptr(), nbytes, _lib.stream_of(DEV)), "gemm packed ws")
    return out_buf[:, :n]


@pytest.mark.parametrize("m,n,k", SPLIT, ids=[f"m{m}_n{n}_k{k}" for m, n, k in SPLIT])
def test_split_tail_matches_int_mm_and_whole_tiles(m, n, k):
    print(f"split tail m={m} n={n} k={k}", flush=True)
    lib = _lib.load()
    assert lib.h3k_gemm_packed_split_bytes(m, n, k) > 0, "the cost model no longer splits this shape"
    g = torch.Generator(device=DEV).manual_seed(m + n + k + 1)
    xq = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=DEV)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=DEV)
    xs = torch.rand(m, 1, generator=g, device=DEV) * 0.05 + 1e-4
    s_ch = torch.rand(n, generator=g, device=DEV) * 0.03 + 1e-4
    w8p = pack(w8)
    acc = torch._int_mm(xq, w8.t())
    want = torch_epilogue(acc, xs, s_ch, "ck", torch.bfloat16)
    got = run_packed_ws(xq, xs, w8p, s_ch, n, "ck", _lib.BF16)
    assert torch.equal(got.contiguous().view(torch.int16), want.view(torch.int16)), "split tail, ck bf16"
    whole = run_packed_ws(xq, xs, w8p, s_ch, n, "ck", _lib.BF16, split=False)
    assert torch.equal(whole.contiguous().view(torch.int16), want.view(torch.int16)), "whole tiles, ck bf16"


@pytest.mark.parametrize("mode,odt", [("eager", _lib.F16), ("ck", _lib.F16), ("eager", _lib.BF16)])
def test_split_tail_epilogues_bias_and_strided_outputs(mode, odt):
    m, n, k = SPLIT[0]
    print(f"split tail epilogue mode={mode} odt={odt}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(odt * 5 + (mode == "eager"))
    xq = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=DEV)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=DEV)
    xs = torch.rand(m, 1, generator=g, device=DEV) * 0.05 + 1e-4
    s_ch = torch.rand(n, generator=g, device=DEV) * 0.03 + 1e-4
    dt = {_lib.BF16: torch.bfloat16, _lib.F16: torch.float16}[odt]
    bias = torch.randn(n, generator=g, device=DEV).to(dt)
    w8p = pack(w8)
    acc = torch._int_mm(xq, w8.t())
    for b, ldo in ((bias, n), (None, n + 8), (bias, n + 4)):
        got = run_packed_ws(xq, xs, w8p, s_ch, n, mode, odt, bias=b, ldo=ldo)
        want = torch_epilogue(acc, xs, s_ch, mode, dt, b)
        assert torch.equal(got.contiguous().view(torch.int16), want.view(torch.int16)), (b is not None, ldo)


def test_split_tail_through_the_w4a8_linear_entry():
    """h3k_w4a8_linear with its full workspace (split tail) against the same call with only the required part of the
    workspace (whole tiles), on the BASELINE weight recipe: equal bit for bit."""
    from test_gpu_qlinear import random_acts_gpu

    m, n, k = 4096, 5120, 13824
    lib = _lib.load()
    full = lib.h3k_w4a8_linear_workspace(m, n, k)
    split = lib.h3k_gemm_packed_split_bytes(m, n, k)
    assert split > 0 and full == m * k + m * 4 + n * k + split
    x = random_acts_gpu(m, k, seed=11)
    w = random_weight_gpu(n, k, seed=12)
    outs = []
    for nbytes in (full, full - split):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        _lib.check(lib.h3k_w4a8_linear(x.data_ptr(), _lib.BF16, m, k, k, w.q.data_ptr(), w.q.stride(0), w.s_rel.data_ptr(),
                                       _lib.scale_code(w.s_rel.dtype), w.s_rel.stride(0), w.s_ch.data_ptr(),
                                       w.codebook.data_ptr(), n, w.group_size, w.convrot, None, 0, out.data_ptr(),
                                       _lib.BF16, n, ws.data_ptr(), nbytes, _lib.stream_of(DEV)), "w4a8 linear")
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
