"""The reference-side binding of the HIP backend: the `_run_hip` a reference maintainer adds to
h3turbo/h3/qlinear.py next to `_run_ck` (h3turbo/h3/qlinear.py:427-429), calling the one C entry point
h3k_w4a8_linear through ctypes.  The integration notes print this function as the binding to add; the GPU tests
call it as written, with only the library path filled in.

Test infrastructure: it binds the built library directly (no h3turbo_amd import), as the reference would.
"""
import ctypes
import os

import torch

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "minimax-h3-turbo_amd", "h3turbo_amd",
                   "libh3k.so")

_h3k = ctypes.CDLL(LIB)
_P, _I, _L, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
_h3k.h3k_w4a8_linear.argtypes = [_P, _I, _L, _L, _L, _P, _L, _P, _I, _L, _P, _P, _L, _I, _I, _P, _I, _P, _I, _L, _P, _Z, _P]
_h3k.h3k_w4a8_linear_workspace.restype = _Z
_h3k.h3k_w4a8_linear_workspace.argtypes = [_L, _L, _L]
_h3k.h3k_last_error.restype = ctypes.c_char_p
_ACT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
_SC = {torch.float8_e4m3fn: 3, torch.uint8: 3, torch.float16: 1, torch.bfloat16: 0, torch.float32: 2}


def _run_hip(x2, w, bias, out_dtype, quant_mode="ck"):
    m, k = x2.shape; n = w.q.shape[0]
    x2 = x2.contiguous(); q = w.q.contiguous(); s = w.s_rel.contiguous()
    out = torch.empty(m, n, dtype=out_dtype, device=x2.device)
    ws = torch.empty(_h3k.h3k_w4a8_linear_workspace(m, n, k), dtype=torch.uint8, device=x2.device)
    b = None if bias is None else bias.to(out_dtype).contiguous()
    rc = _h3k.h3k_w4a8_linear(x2.data_ptr(), _ACT[x2.dtype], m, k, k, q.data_ptr(), k // 2, s.data_ptr(),
                              _SC[s.dtype], s.shape[1], w.s_ch.float().contiguous().data_ptr(),
                              w.codebook.float().to(x2.device).contiguous().data_ptr(), n, w.group_size, w.convrot,
                              None if b is None else b.data_ptr(), {"ck": 0, "eager": 1}[quant_mode],
                              out.data_ptr(), _ACT[out_dtype], n, ws.data_ptr(), ws.numel(),
                              torch.cuda.current_stream(x2.device).cuda_stream)
    if rc != 0:
        raise (ValueError if rc == -1 else RuntimeError)(_h3k.h3k_last_error().decode())
    return out
