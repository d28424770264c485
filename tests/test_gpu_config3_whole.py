"""BASELINE config 3 on the GPU, every shape, every output element.

The sixteen GEMM shapes (M in {512, 4096, 12090, 32768}; (K, N) in {(5120, 5120), (5120, 15360), (5120, 13824),
(13824, 5120)}) run the W4A8 QLinear with the BASELINE recipe's activations (N(0,1), 1 % outlier channels x20,
bf16) and random int4 group-128 weights with fp16 scales.  Whole tensors are compared against the reference's
own CUDA formulation of each step, run as torch ops on the same GPU:

  int8 activations, scales   _quantize_rows "ck" (h3turbo/h3/qlinear.py:267-292): fp64 block rotation rounded
                             once to fp32 (exact: every product x * (+-2^-4) and every partial sum of 256 of them
                             is exact in fp64), aminmax, max(amax / 127, 1e-30), bf16 scale, bf16 quotient,
                             round half to even, clamp
  int32 accumulators         _int8_mm (qlinear.py:236-247): torch._int_mm(xq, w8.t()), the vendor int8 GEMM
  bf16 outputs               the "ck" epilogue (qlinear.py:401): torch.mul(torch.mul(acc, xs), s_ch, out=bf16)

The accumulators come from h3k_gemm_a8w8's acc_out side channel; the outputs from qlinear.linear, whose full
tiles take the GEMM's streaming-store epilogue (acc_out off).  Sampled rows are also recomputed by the CPU
oracle, which pins the torch restatement above.
"""
import numpy as np
import pytest
import torch

from h3turbo_amd import _lib
from h3turbo_amd import qlinear as ql
from oracle import qlinear_ref as ref
from test_gpu_qlinear import np_bits, random_acts_gpu, random_weight_gpu

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

SHAPES = [(m, k, n) for m in (512, 4096, 12090, 32768) for k, n in ((5120, 5120), (5120, 15360), (5120, 13824),
                                                                    (13824, 5120))]


def torch_quantize_rows_ck(x: torch.Tensor, size: int = 256):
    """_quantize_rows(x, size, "ck") of the reference (qlinear.py:267-292) as torch ops on the GPU, bf16 input."""
    m, k = x.shape
    h = torch.from_numpy(ref.hadamard_regular(size)).to(DEV)
    y32 = torch.matmul(x.double().view(m, k // size, size), h).view(m, k).float()
    mn, mx = torch.aminmax(y32, dim=-1, keepdim=True)
    # the scale on the CPU, as the reference computes it: torch's GPU division by a Python scalar multiplies by
    # the rounded reciprocal instead, which differs from the true quotient in the last bit for some rows
    xs = (torch.maximum(mx, -mn).cpu() / 127.0).clamp_(min=1e-30).to(DEV)
    s = xs.to(x.dtype)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(x.dtype).tiny), s)
    y = y32.to(x.dtype)
    del y32
    y.div_(s).round_().clamp_(-128, 127)
    return y.to(torch.int8), xs


def hip_acc(xq, xs, w8, s_ch):
    m, k = xq.shape
    n = w8.shape[0]
    acc = torch.empty(m, n, dtype=torch.int32, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, s_ch.data_ptr(), None, m, n, k,
                                 0, out.data_ptr(), _lib.BF16, n, acc.data_ptr(), _lib.stream_of(DEV)), "gemm")
    return acc, out


@pytest.mark.parametrize("m,k,n", SHAPES, ids=[f"m{m}_k{k}_n{n}" for m, k, n in SHAPES])
def test_config3_shape_whole_outputs(m, k, n):
    print(f"config-3 whole-output m={m} k={k} n={n}", flush=True)
    x = random_acts_gpu(m, k, seed=3 * m + k)
    w = random_weight_gpu(n, k, seed=7 * n + k)

    # activations: every int8 level and every scale
    xq, xs = ql.quantize_activation(x)
    tq, txs = torch_quantize_rows_ck(x)
    assert torch.equal(xs, txs), "activation scales"
    assert torch.equal(xq, tq), "int8 activations"
    del tq, txs

    # weight grid, then the exact accumulators against the vendor int8 GEMM
    w8 = ql.decode_int8_grid(w)
    acc, out_general = hip_acc(xq, xs, w8, w.s_ch)
    want_acc = torch._int_mm(xq, w8.t())
    assert torch.equal(acc, want_acc), "int32 accumulators"

    # outputs of the public op (fast epilogue) against the reference's epilogue on those accumulators
    want = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    torch.mul(torch.mul(want_acc, xs), w.s_ch.float().reshape(1, -1), out=want)
    del want_acc, acc
    out = ql.linear(x, w)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), "bf16 outputs (linear)"
    assert torch.equal(out_general.view(torch.int16), want.view(torch.int16)), "bf16 outputs (acc_out path)"

    # sampled rows through the CPU oracle: pins the torch restatement above
    rng = np.random.default_rng(m + n)
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 4)]))
    rows_t = torch.from_numpy(rows).to(DEV)
    xr = x.index_select(0, rows_t).contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    q_ref, xs_ref = ref.quantize_rows(ref.bf16_from_bits(xr), "bf16", 256, "ck")
    assert np.array_equal(xq.index_select(0, rows_t).cpu().numpy(), q_ref)
    assert np.array_equal(xs.index_select(0, rows_t).cpu().numpy(), xs_ref)
    s_bits = w.s_rel.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    w8_ref = ref.decode_int8_grid(w.q.cpu().numpy(), s_bits, "f16", w.codebook.cpu().numpy(), 128)
    assert np.array_equal(w8.cpu().numpy(), w8_ref), "int8 weight grid"
    o_ref = ref.epilogue(ref.int8_mm(q_ref, w8_ref), xs_ref, w.s_ch.cpu().numpy(), "bf16", "ck")
    assert np.array_equal(np_bits(out.index_select(0, rows_t)), ref.bf16_bits(o_ref))
    print(f"  ok m={m} k={k} n={n}", flush=True)
