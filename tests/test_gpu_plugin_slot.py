"""The C entry point that fills the reference's kitchen slot (h3turbo/h3/qlinear.py:427-429), called exactly as a
reference maintainer would call it (tests/hip_slot_stub.py, the binding the integration notes print).

Both of h3k_w4a8_linear's routes are covered: chunks of at most 32 rows take the fused few-row GEMM (int4 decoded
in registers), larger ones the weight decode + int8 GEMM.  Every result is bit-exact with the reference's golden
vectors or the CPU oracle, and has the shape, dtype and contiguity the reference checks of a backend result
(h3turbo/h3/qlinear.py:449-450).
"""
import numpy as np
import pytest
import torch

import fixtures as fx
import hip_slot_stub as stub
import inputs as gi
from oracle import qlinear_ref as ref
from test_gpu_qlinear import DT, make_w, np_bits, t_bits16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def check_result(out, m, n, dt):
    assert tuple(out.shape) == (m, n) and out.dtype == dt and out.is_contiguous()


@pytest.mark.parametrize("name", list(fx.cases("small")))
def test_slot_small_golden_cases(name):
    meta, a = fx.load(name)
    print(f"slot case {name}", flush=True)
    dt = DT[meta["x_dtype"]]
    x = torch.from_numpy(a["x"]).to(DEV) if meta["x_dtype"] == "f32" else t_bits16(a["x"], dt)
    w = make_w(a["q"], a["s_rel"], meta["s_kind"], a["s_ch"], a["cb"], meta["group"], meta["convrot"])
    b = torch.from_numpy(a["bias"]).to(DEV) if "bias" in a else None
    out = stub._run_hip(x, w, b, dt, meta["mode"])
    check_result(out, meta["m"], meta["n"], dt)
    assert np.array_equal(np_bits(out), a["out"])


@pytest.mark.parametrize("name", ["c1_f16", "c1_fp8"])
def test_slot_config1_bit_exact(name):
    meta, _ = fx.load(name)
    xb, q, s_rel, s_ch, cb = fx.regenerate(meta)
    x = t_bits16(xb, torch.bfloat16)
    w = make_w(q, s_rel, meta["s_kind"], s_ch, cb, meta["group"], 256)
    out = stub._run_hip(x, w, None, torch.bfloat16)
    check_result(out, meta["m"], meta["n"], torch.bfloat16)
    assert gi.sha(np_bits(out)) == meta["sha_out"]
    assert gi.sha(np_bits(stub._run_hip(x, w, None, torch.bfloat16, "eager"))) == meta["sha_out_eager"]


@pytest.fixture(scope="module")
def weights():
    k, n = 1024, 320
    qa, sa, cha, cba = gi.weight_int4_g128(n, k, seed=41)
    qb, sb, chb, cbb = gi.weight_fp8_g16(n, k, seed=42)
    return {"g128_f16": (make_w(qa, sa, "f16", cha, cba, 128, 256), (qa, sa, "f16", cha, cba, 128)),
            "g16_fp8": (make_w(qb, sb, "fp8", chb, cbb, 16, 256), (qb, sb, "fp8", chb, cbb, 16))}


@pytest.mark.parametrize("fmt", ["g128_f16", "g16_fp8"])
def test_slot_every_row_count_from_1_to_40_and_600(weights, fmt):
    """Rows 1..32 take the fused few-row GEMM, 33..40 and 600 the decode + int8 GEMM."""
    w, (q, s, kind, s_ch, cb, group) = weights[fmt]
    k, n = 1024, 320
    xb = gi.activations(600, k, seed=43)
    xall = t_bits16(xb, torch.bfloat16)
    xv = ref.bf16_from_bits(xb)
    for m in list(range(1, 41)) + [600]:
        for mode in ("ck", "eager"):
            out = stub._run_hip(xall[:m], w, None, torch.bfloat16, mode)
            check_result(out, m, n, torch.bfloat16)
            want, *_ = ref.linear_a8(xv[:m], "bf16", q, s, kind, s_ch, cb, group, 256, mode=mode)
            assert np.array_equal(np_bits(out), ref.bf16_bits(want)), (fmt, m, mode)
    print(f"slot rows 1-40, 600 ok ({fmt})", flush=True)


def test_slot_bias_out_dtypes_and_errors(weights):
    w, (q, s, kind, s_ch, cb, group) = weights["g128_f16"]
    k, n = 1024, 320
    xb = gi.activations(48, k, seed=44)
    xv = ref.bf16_from_bits(xb)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(45))
    for m in (5, 48):
        for odt, name in ((torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")):
            out = stub._run_hip(t_bits16(xb[:m], torch.bfloat16), w, bias.to(DEV), odt)
            check_result(out, m, n, odt)
            want, *_ = ref.linear_a8(xv[:m], "bf16", q, s, kind, s_ch, cb, group, 256, out_dtype=name,
                                     bias=bias.to(odt).float().numpy())
            assert np.array_equal(out.float().cpu().numpy(), want), (m, name)
    # the C entry point's own checks: workspace too small, unaligned workspace, bad rotation size
    lib = stub._h3k
    x = t_bits16(xb[:8], torch.bfloat16)
    out = torch.empty(8, n, dtype=torch.bfloat16, device=DEV)
    need = lib.h3k_w4a8_linear_workspace(8, n, k)
    ws = torch.empty(need + 512, dtype=torch.uint8, device=DEV)
    sp = torch.cuda.current_stream(DEV).cuda_stream
    args = lambda wsp, nbytes, rot: (x.data_ptr(), 0, 8, k, k, w.q.data_ptr(), k // 2, w.s_rel.data_ptr(), 1,  # noqa: E731
                                     w.s_rel.shape[1], w.s_ch.data_ptr(), w.codebook.data_ptr(), n, 128, rot, None, 0,
                                     out.data_ptr(), 0, n, wsp, nbytes, sp)
    assert lib.h3k_w4a8_linear(*args(ws.data_ptr(), need - 1, 256)) == -3
    assert lib.h3k_w4a8_linear(*args(ws.data_ptr() + 16, need, 256)) == -1
    assert lib.h3k_w4a8_linear(*args(ws.data_ptr(), need, 48)) == -1
    assert b"power of 4" in lib.h3k_last_error() or b"rotation" in lib.h3k_last_error()
    assert lib.h3k_w4a8_linear(*args(ws.data_ptr(), need, 256)) == 0
    torch.cuda.synchronize()
