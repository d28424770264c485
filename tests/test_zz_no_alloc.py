"""h3k_w4a8_linear_noalloc (no workspace argument, scratch in a static device array) against h3k_w4a8_linear with a
caller workspace, through the C ABI: bit-identical outputs on two calls in a row -- the packed-grid route at 2048
rows, then the fused few-row route at 24 rows, which reuses the same scratch -- and a clear ESPACE for a call whose
scratch need exceeds the static array."""
import ctypes

import numpy as np
import pytest
import torch

import hip_slot_stub as stub
import inputs as gi
from test_gpu_qlinear import make_w, t_bits16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

_P, _I, _L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
NOALLOC = stub._h3k.h3k_w4a8_linear_noalloc
NOALLOC.argtypes = [_P, _I, _L, _L, _L, _P, _L, _P, _I, _L, _P, _P, _L, _I, _I, _P, _I, _P, _I, _L, _P]
NOALLOC.restype = _I


def noalloc(x, w, out):
    m, k = x.shape
    n = w.q.shape[0]
    return NOALLOC(x.data_ptr(), 0, m, k, k, w.q.data_ptr(), k // 2, w.s_rel.data_ptr(), 1, w.s_rel.shape[1],
                   w.s_ch.data_ptr(), w.codebook.data_ptr(), n, w.group_size, w.convrot, None, 0, out.data_ptr(), 0, n,
                   torch.cuda.current_stream(DEV).cuda_stream)


def test_noalloc_equals_the_workspace_entry_on_two_calls_in_a_row():
    k, n = 5120, 5120
    q, s, s_ch, cb = gi.weight_int4_g128(n, k, seed=71)
    w = make_w(q, s, "f16", s_ch, cb, 128, 256)
    xb = gi.activations(2048, k, seed=72)
    x = t_bits16(xb, torch.bfloat16)
    for m in (2048, 24):  # the second, smaller call reuses the scratch the first one filled
        print(f"noalloc m={m}", flush=True)
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        rc = noalloc(x[:m], w, got)
        assert rc == 0, stub._h3k.h3k_last_error()
        want = stub._run_hip(x[:m], w, None, torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), m


def test_noalloc_rejects_calls_beyond_its_scratch():
    k, n, m = 5120, 13824, 32768  # 168 MB of int8 activations + the 71 MB grid: above the 128 MiB array
    x = torch.zeros(16, k, dtype=torch.bfloat16, device=DEV)  # never read: the size check comes first
    w = make_w(np.zeros((n, k // 2), np.int8), np.zeros((n, k // 128), np.uint16), "f16", np.ones(n, np.float32),
               np.arange(-8, 8, dtype=np.float32), 128, 256)
    out = torch.empty(16, n, dtype=torch.bfloat16, device=DEV)
    rc = NOALLOC(x.data_ptr(), 0, m, k, k, w.q.data_ptr(), k // 2, w.s_rel.data_ptr(), 1, w.s_rel.shape[1],
                 w.s_ch.data_ptr(), w.codebook.data_ptr(), n, 128, 256, None, 0, out.data_ptr(), 0, n,
                 torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == -3
    assert b"static scratch" in stub._h3k.h3k_last_error()
