"""ConvRot W4A8 linear ops on MI355X: the drop-in for h3turbo/h3/qlinear.py.

Same public surface and error behaviour as the reference module (h3turbo/h3/qlinear.py:44-523):
`linear`, `quantize_activation`, `rotate`, `decode_int8_grid`, `dequantize`, `hadamard_regular`,
`available_backends`, `resolve_backend`, with one more backend, "hip", that runs the hand-written gfx950 kernels
of libh3k.so (include/h3k.h).  "auto" resolves to "hip".  The reference's other backends are not part of this
build: "ck" (comfy_kitchen CUDA) and "torch" (portable) raise RuntimeError when requested, like the reference
does for an unusable backend.  Argument errors raise ValueError with the reference's messages before any device
check; W4A8 compute on CPU tensors raises RuntimeError (the product never falls back to a CPU path).

Numerics (bit-exact with the reference's torch backend, quant_mode "ck" or "eager"):
  quantize_activation : fp64 Walsh-Hadamard rotation rounded once to fp32, per-row absmax int8
  decode_int8_grid    : clamp(rint(codebook[nib] * s_rel), +-127)
  linear (a8)         : exact int32 GEMM on int8 MFMA, (acc * xs) * s_ch rounded once, bias after rounding
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib
from .types import W4A8Weight, Weight

CONVROT = 256
_H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))
_HAD_CACHE: Dict[Tuple[int, str, int, torch.dtype], torch.Tensor] = {}
_BACKENDS = ("auto", "hip", "ck", "torch")


# --------------------------------------------------------------------------------------------- Hadamard
def hadamard_regular(size: int, device="cpu", dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Normalised regular Hadamard H = kron(H4, ..., H4) / sqrt(size); symmetric, H @ H = I (qlinear.py:44-66).
    Entries are +-2^-j, exact in every float dtype.  Cached: do not mutate the result."""
    n = size
    while n > 1 and n % 4 == 0:
        n //= 4
    if size < 4 or n != 1:
        raise ValueError(f"regular Hadamard size must be a power of 4 (>= 4), got {size}")
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    key = (size, dev.type, -1 if dev.index is None else dev.index, dtype)
    h = _HAD_CACHE.get(key)
    if h is None:
        h4 = torch.tensor(_H4, dtype=torch.float32)
        full = h4
        for _ in range(round(math.log(size, 4)) - 1):
            full = torch.kron(full, h4)
        h = (full / math.sqrt(size)).to(device=dev, dtype=dtype).contiguous()
        _HAD_CACHE[key] = h
    return h


def _check_rotation(size: int) -> None:
    """Rotation sizes: the reference's powers of 4, plus the other powers of 2 in [8, 512] as an extension (H2 on
    the top index bit, scale 1/sqrt(size) rounded once in fp64; see hadamard)."""
    if size < 4 or size > 1024 or size & (size - 1):
        raise ValueError(f"rotation block must be a power of 2 in [4, 1024] (the reference: a power of 4), got {size}")


def hadamard(size: int, device="cpu", dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The rotation matrix of any supported size: hadamard_regular for powers of 4; for the other powers of 2
    (an extension the reference rejects) kron(H2, H4, ..., H4) / sqrt(size) with H2 = [[1, 1], [1, -1]] as the
    most significant factor, built in fp64 and rounded once to `dtype`."""
    _check_rotation(size)
    if size & 0x155555:
        return hadamard_regular(size, device, dtype)
    h4 = torch.tensor(_H4, dtype=torch.float64)
    full = torch.tensor(((1.0, 1.0), (1.0, -1.0)), dtype=torch.float64)
    inner = h4
    while inner.shape[0] * 2 < size:
        inner = torch.kron(inner, h4)
    full = torch.kron(full, inner) * (math.sqrt(2.0) * 2.0 ** -((size.bit_length()) // 2))
    return full.to(device=device, dtype=dtype).contiguous()


# --------------------------------------------------------------------------------------------- helpers
def _need_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: h3turbo_amd computes W4A8 ops on the GPU (HIP, gfx950) only; got a {t.device} "
                           "tensor (move it to the ROCm device)")


def _rows(x2: torch.Tensor) -> torch.Tensor:
    """[M, K] view whose last dim is contiguous (the kernels take a row stride)."""
    return x2 if x2.stride(-1) == 1 and (x2.shape[0] <= 1 or x2.stride(0) >= x2.shape[1]) else x2.contiguous()


def _ld(x2: torch.Tensor) -> int:
    """Row stride of a row-contiguous [M, K] view (any value >= K serves a single row)."""
    return x2.stride(0) if x2.shape[0] > 1 else x2.shape[1]


def _check_mode(mode: str) -> None:
    if mode not in ("ck", "eager"):
        raise ValueError(f"quant_mode must be 'ck' or 'eager', got {mode!r}")


def _check_weight(w: W4A8Weight) -> Tuple[int, int]:
    """The reference's weight validation (qlinear.py:140-154), same messages."""
    if w.q.dim() != 2 or w.q.dtype not in (torch.int8, torch.uint8):
        raise ValueError(f"W4A8 q must be a 2D int8 tensor, got {tuple(w.q.shape)} {w.q.dtype}")
    n, k = w.q.shape[0], w.q.shape[1] * 2
    gs, cr = w.group_size, w.convrot
    if gs < 4 or k % 16 or k % gs or k % cr or (16 % gs and gs % 16):
        raise ValueError(f"K={k} must be divisible by 16, group_size={gs} and convrot={cr}; group_size >= 4 dividing 16 or a multiple of 16")
    if tuple(w.s_rel.shape) != (n, k // gs):
        raise ValueError(f"s_rel must have shape {(n, k // gs)}, got {tuple(w.s_rel.shape)}")
    if tuple(w.s_ch.shape) != (n,):
        raise ValueError(f"s_ch must have shape {(n,)}, got {tuple(w.s_ch.shape)}")
    if tuple(w.codebook.shape) != (16,):
        raise ValueError(f"codebook must have shape (16,), got {tuple(w.codebook.shape)}")
    return n, k


class _DevWeight:
    """Kernel-ready views of a W4A8Weight: q with contiguous, 8-byte aligned rows, s_rel with contiguous rows,
    float32 s_ch / codebook.  Copies only what is not already in that form."""

    __slots__ = ("q", "ldq", "s", "lds", "scode", "s_ch", "cb", "n", "k")

    def __init__(self, w: W4A8Weight):
        self.n, self.k = _check_weight(w)
        q = w.q.view(torch.int8) if w.q.dtype == torch.uint8 else w.q
        if q.stride(-1) != 1 or (q.data_ptr() % 8) or (q.shape[0] > 1 and q.stride(0) % 8):
            q = q.contiguous()
        self.q, self.ldq = q, (q.stride(0) if q.shape[0] > 1 else q.shape[1])
        s = w.s_rel
        self.scode = _lib.scale_code(s.dtype)
        if s.stride(-1) != 1:
            s = s.contiguous()
        self.s, self.lds = s, (s.stride(0) if s.shape[0] > 1 else s.shape[1])
        self.s_ch = w.s_ch.to(torch.float32).contiguous()
        self.cb = w.codebook.to(device=q.device, dtype=torch.float32).contiguous()


# --------------------------------------------------------------------------------------------- rotation / quantiser
def rotate(x: torch.Tensor, size: int = CONVROT) -> torch.Tensor:
    """x[..., K] -> per-`size`-block x @ H in x.dtype, accumulated exactly and rounded once (qlinear.py:118-132)."""
    if not x.is_floating_point():
        raise ValueError(f"rotate expects a floating tensor, got {x.dtype}")
    k = x.shape[-1]
    if k % size:
        raise ValueError(f"last dim {k} is not a multiple of the rotation block {size}")
    _check_rotation(size)
    if x.numel() == 0:
        return x.clone()
    _need_gpu(x, "rotate")
    x2 = x.reshape(-1, k)
    if x.dtype == torch.float64:  # the reference's own fp64 path: one fp64 GEMM
        y = torch.matmul(x2.reshape(-1, k // size, size), hadamard(size, x.device, x.dtype)).reshape(-1, k)
        return y.reshape(x.shape)
    x2 = _rows(x2)
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    lib = _lib.load()
    _lib.check(lib.h3k_rotate(x2.data_ptr(), _lib.act_code(x.dtype), x2.shape[0], k, _ld(x2), size, y.data_ptr(),
                              k, _lib.stream_of(x.device)), "h3k_rotate")
    return y.reshape(x.shape)


@torch.no_grad()
def _quantize_rows(x2: torch.Tensor, size: int, mode: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotate + per-row int8 quantisation on the GPU: (int8 [M, K], fp32 [M, 1]) (qlinear.py:267-292)."""
    m, k = x2.shape
    q = torch.empty(m, k, dtype=torch.int8, device=x2.device)
    xs = torch.empty(m, 1, dtype=torch.float32, device=x2.device)
    if m == 0:
        return q, xs
    x2 = _rows(x2)
    lib = _lib.load()
    _lib.check(lib.h3k_rotate_quant(x2.data_ptr(), _lib.act_code(x2.dtype), m, k, _ld(x2), size, _lib.MODE[mode],
                                    q.data_ptr(), k, xs.data_ptr(), _lib.stream_of(x2.device)), "h3k_rotate_quant")
    return q, xs


def quantize_activation(x: torch.Tensor, *, size: int = CONVROT, quant_mode: str = "ck") -> Tuple[torch.Tensor, torch.Tensor]:
    """x[..., K] -> (int8 [..., K], fp32 scale [..., 1]) of the rotated activation (qlinear.py:295-303)."""
    _check_mode(quant_mode)
    k = x.shape[-1]
    if k % size:
        raise ValueError(f"last dim {k} is not a multiple of the rotation block {size}")
    _check_rotation(size)
    _need_gpu(x, "quantize_activation")
    q, s = _quantize_rows(x.reshape(math.prod(x.shape[:-1]), k), size, quant_mode)
    return q.reshape(x.shape), s.reshape(*x.shape[:-1], 1)


# --------------------------------------------------------------------------------------------- weights
def _decode(dw: _DevWeight, group: int) -> torch.Tensor:
    w8 = torch.empty(dw.n, dw.k, dtype=torch.int8, device=dw.q.device)
    if dw.n:
        lib = _lib.load()
        _lib.check(lib.h3k_decode_w4(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds, dw.cb.data_ptr(), dw.n,
                                     dw.k, group, w8.data_ptr(), dw.k, _lib.stream_of(dw.q.device)), "h3k_decode_w4")
    return w8


def _decode_packed(dw: _DevWeight, group: int) -> torch.Tensor:
    """The grid in the packed layout of the large-shape GEMM (h3k_decode_w4_packed): a flat int8 buffer."""
    lib = _lib.load()
    w8p = torch.empty(lib.h3k_w8_packed_bytes(dw.n, dw.k), dtype=torch.int8, device=dw.q.device)
    _lib.check(lib.h3k_decode_w4_packed(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds, dw.cb.data_ptr(),
                                        dw.n, dw.k, group, w8p.data_ptr(), _lib.stream_of(dw.q.device)),
               "h3k_decode_w4_packed")
    return w8p


@torch.no_grad()
def decode_int8_grid(w: W4A8Weight) -> torch.Tensor:
    """int8 [N, K]: the exact grid the int8 GEMM consumes (qlinear.py:194-204)."""
    _check_weight(w)
    _need_gpu(w.q, "decode_int8_grid")
    return _decode(_DevWeight(w), w.group_size)


@torch.no_grad()
def dequantize(w: W4A8Weight, dtype: torch.dtype = torch.float32, rotated: bool = False, *, rows: Optional[slice] = None) -> torch.Tensor:
    """Dense [N, K] weight (qlinear.py:207-226): rotated=True the ConvRot basis (grid * s_ch), False the original
    basis (W_rot @ H per block, fp32, rounded once to dtype).  `rows` restricts to a contiguous row slice."""
    n, k = _check_weight(w)
    if rows is not None and rows.step not in (None, 1):
        raise ValueError("rows must be a contiguous slice")
    r0, r1, _ = (rows or slice(0, n)).indices(n)
    _need_gpu(w.q, "dequantize")
    sub = W4A8Weight(w.q[r0:r1], w.s_rel[r0:r1], w.s_ch[r0:r1], w.codebook, w.group_size, w.convrot)
    wr = decode_int8_grid(sub).float().mul_(sub.s_ch.float().unsqueeze(1))
    if not rotated:
        h = hadamard(w.convrot, w.q.device, torch.float32)
        wr = torch.matmul(wr.view(max(r1 - r0, 0), k // w.convrot, w.convrot), h).view(max(r1 - r0, 0), k)
    return wr.to(dtype)


# --------------------------------------------------------------------------------------------- backends
def available_backends() -> Dict[str, Dict[str, Any]]:
    """{"hip": {...}, "ck": {...}, "torch": {...}} with availability and why a backend is missing."""
    ok, why = True, None
    try:
        _lib.load()
    except (RuntimeError, OSError) as e:
        ok, why = False, str(e)
    gpu = torch.cuda.is_available()
    return {
        "hip": {"available": ok and gpu, "library": _lib.LIB_PATH if ok else None,
                "reason": why if not ok else (None if gpu else "no ROCm device")},
        "ck": {"available": False, "reason": "comfy_kitchen's CUDA kernels are not part of this build (use 'hip')", "version": None},
        "torch": {"available": False, "reason": "the portable torch backend is not part of this build (use 'hip')"},
    }


def resolve_backend(x: torch.Tensor, w: Weight, backend: str = "auto", precision: str = "a8") -> str:
    """The backend `linear` will use: "hip" for a W4A8 weight, "dense" for a dense one (qlinear.py:345-361)."""
    if backend not in _BACKENDS:
        raise ValueError(f"backend must be 'auto', 'hip', 'ck' or 'torch', got {backend!r}")
    if precision not in ("a8", "a16"):
        raise ValueError(f"precision must be 'a8' or 'a16', got {precision!r}")
    if not isinstance(w, W4A8Weight):
        return "dense"
    if backend in ("ck", "torch"):
        raise RuntimeError(f"backend {backend!r} unavailable: {available_backends()[backend]['reason']}")
    return "hip"


INPUT_ACTS = (None, "none", "swiglu", "gelu_tanh")
ACT_CODE = {"swiglu": 1, "gelu_tanh": 2}


def apply_input_act(x: torch.Tensor, act: Optional[str]) -> torch.Tensor:
    """The input activation as torch ops in x.dtype: "swiglu" (qlinear.py:376-379) or "gelu_tanh"
    (F.gelu(x, approximate="tanh"), the config-4 block's MLP; an extension of the reference's input_act)."""
    if act == "swiglu":
        return _swiglu(x)
    if act == "gelu_tanh":
        return F.gelu(x, approximate="tanh")
    return x


def _swiglu(x: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up on [gate | up] halves, in x.dtype (qlinear.py:376-379)."""
    gate, up = x.chunk(2, dim=-1)
    return F.silu(gate).mul_(up)


# token chunks up to this many rows take the fused int4 GEMM (h3k_gemm_w4a8); above it the per-call decode + int8
# GEMM pair is faster (N=13824, K=5120, g128 fp16: 35 against 42 us at 64 rows, 44 against 73 at 128), at 16 the
# fused GEMM (15 against 34 us)
FEW_ROWS = 32


class _HipRunner:
    """W4A8 forward for one weight on the GPU.  Each token chunk runs rotate+quantise, then either the fused
    few-row GEMM that decodes the int4 weight in registers (chunks of at most FEW_ROWS rows), or the int8 MFMA GEMM
    over the weight's int8 grid, decoded once per call when first needed.  Both end in the fused epilogue written
    into the chunk's `out` slice."""

    def __init__(self, w: W4A8Weight, bias: Optional[torch.Tensor], out_dtype: torch.dtype, precision: str, mode: str):
        self.w, self.out_dtype, self.precision, self.mode = w, out_dtype, precision, mode
        self.dw = _DevWeight(w)
        self.n, self.k = self.dw.n, self.dw.k
        self.ocode = _lib.act_code(out_dtype)
        self.bias = None if bias is None else bias.to(device=w.q.device, dtype=out_dtype).contiguous()
        # a16 adds the bias in fp32 from its own dtype (qlinear.py:423), a8 after rounding it to out_dtype (:405)
        self.bias32 = None if bias is None else bias.to(device=w.q.device, dtype=torch.float32).contiguous()
        self._w8: Optional[torch.Tensor] = None
        self._w8p: Optional[torch.Tensor] = None
        self.lib = _lib.load()
        g = w.group_size
        q_lines = self.dw.q.data_ptr() % 16 == 0 and self.dw.ldq % 16 == 0
        self.few_rows_ok = self.k % 64 == 0 and (g in (16, 32) or g % 64 == 0) and self.k % g == 0 and q_lines
        self.packed_ok = (q_lines and self.k % 64 == 0 and self.dw.s_ch.data_ptr() % 16 == 0
                          and (self.bias is None or self.bias.data_ptr() % 16 == 0))

    @property
    def w8(self) -> torch.Tensor:
        """The row-major int8 grid, decoded once per call when first needed."""
        if self._w8 is None:
            self._w8 = _decode(self.dw, self.w.group_size)
        return self._w8

    @property
    def w8p(self) -> torch.Tensor:
        """The packed int8 grid of the large-shape GEMM, decoded once per call when first needed."""
        if self._w8p is None:
            self._w8p = _decode_packed(self.dw, self.w.group_size)
        return self._w8p

    def __call__(self, x2: torch.Tensor, out: torch.Tensor, act: Optional[str] = None) -> None:
        if self.precision == "a8":
            self._a8(x2, out, act)
        else:
            self._a16(apply_input_act(x2, act), out)

    def _a8(self, x2: torch.Tensor, out: torch.Tensor, act: Optional[str] = None) -> None:
        if act in ACT_CODE and self._act_fused_ok(x2, act):
            xq, xs = _quantize_rows_act(x2, ACT_CODE[act], self.k, self.mode)
        else:
            xq, xs = _quantize_rows(apply_input_act(x2, act), self.w.convrot, self.mode)
        self.gemm(xq, xs, out)

    def _act_fused_ok(self, x2: torch.Tensor, act: str) -> bool:
        """The activation runs inside rotate+quantise (h3k_rotate_quant_act): 16-bit rows, rotation 256."""
        k = self.k
        width = 2 * k if act == "swiglu" else k
        return (x2.dtype in (torch.bfloat16, torch.float16) and self.w.convrot == 256 and k % 256 == 0
                and k <= 256 * 128 and x2.shape[-1] == width and x2.stride(-1) == 1 and x2.data_ptr() % 16 == 0
                and (x2.shape[0] <= 1 or (x2.stride(0) * 2) % 16 == 0))

    def gemm(self, xq: torch.Tensor, xs: torch.Tensor, out: torch.Tensor) -> None:
        """The int8 GEMM with the fused epilogue on quantised activations xq [m, K], scales xs [m, 1]."""
        m = xq.shape[0]
        if m <= FEW_ROWS and self.few_rows_ok:
            dw = self.dw
            nbytes = self.lib.h3k_gemm_w4a8_workspace(m, self.n, self.k)
            ws = torch.empty(max(1, nbytes // 4), dtype=torch.int32, device=xq.device) if nbytes else None
            _lib.check(self.lib.h3k_gemm_w4a8(xq.data_ptr(), self.k, xs.data_ptr(), dw.q.data_ptr(), dw.ldq,
                                              dw.s.data_ptr(), dw.scode, dw.lds, dw.cb.data_ptr(), self.w.group_size,
                                              dw.s_ch.data_ptr(), _lib.ptr(self.bias), m, self.n, self.k,
                                              _lib.MODE[self.mode], out.data_ptr(), self.ocode, out.stride(0),
                                              _lib.ptr(ws), None, _lib.stream_of(xq.device)), "h3k_gemm_w4a8")
            return
        if (self.packed_ok and xs.data_ptr() % 16 == 0 and out.stride(0) >= self.n and m * self.k < (1 << 32)
                and self.lib.h3k_gemm_packed_serves(m, self.n, self.k)):
            # the split tail's int32 partial sums, where the launch takes it (0 bytes otherwise)
            nbytes = self.lib.h3k_gemm_packed_split_bytes(m, self.n, self.k)
            ws = torch.empty(nbytes // 4, dtype=torch.int32, device=xq.device) if nbytes else None
            _lib.check(self.lib.h3k_gemm_a8w8_packed_ws(xq.data_ptr(), self.k, xs.data_ptr(), self.w8p.data_ptr(),
                                                        self.dw.s_ch.data_ptr(), _lib.ptr(self.bias), m, self.n, self.k,
                                                        _lib.MODE[self.mode], out.data_ptr(), self.ocode, out.stride(0),
                                                        _lib.ptr(ws), nbytes, _lib.stream_of(xq.device)),
                       "h3k_gemm_a8w8_packed_ws")
            return
        _lib.check(self.lib.h3k_gemm_a8w8(xq.data_ptr(), self.k, xs.data_ptr(), self.w8.data_ptr(), self.k,
                                          self.dw.s_ch.data_ptr(), _lib.ptr(self.bias), m, self.n, self.k,
                                          _lib.MODE[self.mode], out.data_ptr(), self.ocode, out.stride(0), None,
                                          _lib.stream_of(xq.device)), "h3k_gemm_a8w8")

    def _a16(self, x2: torch.Tensor, out: torch.Tensor) -> None:
        """Unquantised activation (qlinear.py:407-424): rotated x (rounded to x.dtype) times the exact int8 levels
        with fp32 accumulation, s_ch applied to the fp32 result, rounded once.  bf16 / f16 activations run on the
        16-bit MFMA GEMM h3k_gemm_a16 (the levels widened exactly); fp32 ones (the reference's plain fp32 GEMM) on
        torch.mm in fp32."""
        xr = rotate(x2, self.w.convrot)
        if xr.dtype in (torch.bfloat16, torch.float16):
            xr = _rows(xr)
            w8 = self.w8
            _lib.check(self.lib.h3k_gemm_a16(xr.data_ptr(), _lib.act_code(xr.dtype), _ld(xr), w8.data_ptr(), self.k,
                                             self.dw.s_ch.data_ptr(), _lib.ptr(self.bias32), xr.shape[0], self.n, self.k,
                                             out.data_ptr(), self.ocode, out.stride(0) if out.shape[0] > 1 else self.n,
                                             _lib.stream_of(xr.device)), "h3k_gemm_a16")
            return
        y = torch.mm(xr.to(torch.float32), self.w8.to(torch.float32).t())
        y.mul_(self.dw.s_ch)
        if self.bias32 is not None:
            y.add_(self.bias32)
        out.copy_(y)


def _quantize_rows_act(x2: torch.Tensor, act_code: int, k: int, mode: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotate + quantise act(x2) in one pass (h3k_rotate_quant_act): (int8 [M, k], fp32 [M, 1])."""
    m = x2.shape[0]
    q = torch.empty(m, k, dtype=torch.int8, device=x2.device)
    xs = torch.empty(m, 1, dtype=torch.float32, device=x2.device)
    if m == 0:
        return q, xs
    lib = _lib.load()
    _lib.check(lib.h3k_rotate_quant_act(x2.data_ptr(), _lib.act_code(x2.dtype), m, k, _ld(x2), act_code, CONVROT,
                                        _lib.MODE[mode], q.data_ptr(), k, xs.data_ptr(), _lib.stream_of(x2.device)),
               "h3k_rotate_quant_act")
    return q, xs


@torch.no_grad()
def _linear_w4a8(x2, w, bias, out_dtype, backend, precision, act, chunk_tokens, quant_mode):
    swiglu = act == "swiglu"
    n, k = _check_weight(w)
    kx = x2.shape[-1] // (2 if swiglu else 1)
    if kx != k:
        raise ValueError(f"input features {kx}{' (after swiglu)' if swiglu else ''} do not match the weight's K={k}")
    if x2.device != w.q.device:
        raise ValueError(f"input on {x2.device} but weight on {w.q.device}")
    if bias is not None and tuple(bias.shape) != (n,):
        raise ValueError(f"bias must have shape {(n,)}, got {tuple(bias.shape)}")
    m = x2.shape[0]
    if m == 0:
        return torch.empty(0, n, dtype=out_dtype, device=x2.device)
    _need_gpu(x2, "linear")
    resolve_backend(x2, w, backend, precision)
    if x2.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"the HIP path takes bf16, f16 or f32 activations, got {x2.dtype}")
    out = torch.empty(m, n, dtype=out_dtype, device=x2.device)
    runner = _HipRunner(w, bias, out_dtype, precision, quant_mode)
    step = min(chunk_tokens or m, m)
    for a in range(0, m, step):
        runner(x2[a: a + step], out[a: a + step], act)
    return out


@torch.no_grad()
def linear_heads(xh: torch.Tensor, w: W4A8Weight, *, out_dtype: Optional[torch.dtype] = None,
                 quant_mode: str = "ck") -> torch.Tensor:
    """linear(x, w) for x given head-major: xh [heads, tokens, head_dim] is read as x [tokens, heads * head_dim]
    (row t = concatenation over heads of xh[h, t]) without materialising the transpose.  This is the attention
    output feeding the out projection (h3turbo/h3/model.py:226-228: transpose + reshape, then _matmul).  W4A8 a8
    on the HIP kernels only; bit-identical to linear(xh.transpose(0, 1).reshape(tokens, -1), w)."""
    _check_mode(quant_mode)
    if xh.dim() != 3:
        raise ValueError(f"xh must be [heads, tokens, head_dim], got {tuple(xh.shape)}")
    heads, m, hd = xh.shape
    n, k = _check_weight(w)
    if heads * hd != k:
        raise ValueError(f"input features {heads * hd} do not match the weight's K={k}")
    if xh.device != w.q.device:
        raise ValueError(f"input on {xh.device} but weight on {w.q.device}")
    out_dtype = out_dtype or xh.dtype
    if m == 0:
        return torch.empty(0, n, dtype=out_dtype, device=xh.device)
    _need_gpu(xh, "linear_heads")
    if (xh.dtype not in (torch.bfloat16, torch.float16) or w.convrot != 256 or hd < 16 or hd & (hd - 1)
            or k % 256 or k > 256 * 128):
        # no head-major kernel for this case: the transpose copy and the plain linear
        return linear(xh.transpose(0, 1).reshape(m, k), w, out_dtype=out_dtype, quant_mode=quant_mode)
    if (xh.stride(2) != 1 or xh.stride(1) < hd or (heads > 1 and xh.stride(0) < m * xh.stride(1))
            or xh.data_ptr() % 16 or (2 * xh.stride(1)) % 16 or (heads > 1 and (2 * xh.stride(0)) % 16)):
        xh = xh.contiguous()
    ldx, hstride = xh.stride(1), (xh.stride(0) if heads > 1 else m * xh.stride(1))
    runner = _HipRunner(w, None, out_dtype, "a8", quant_mode)
    q = torch.empty(m, k, dtype=torch.int8, device=xh.device)
    xs = torch.empty(m, 1, dtype=torch.float32, device=xh.device)
    lib = _lib.load()
    _lib.check(lib.h3k_rotate_quant_heads(xh.data_ptr(), _lib.act_code(xh.dtype), m, k, ldx, hd, hstride, w.convrot,
                                          _lib.MODE[quant_mode], q.data_ptr(), k, xs.data_ptr(),
                                          _lib.stream_of(xh.device)), "h3k_rotate_quant_heads")
    out = torch.empty(m, n, dtype=out_dtype, device=xh.device)
    runner.gemm(q, xs, out)
    return out


def linear(
    x: torch.Tensor,
    w: Weight,
    bias: Optional[torch.Tensor] = None,
    *,
    out_dtype: Optional[torch.dtype] = None,
    backend: str = "auto",
    precision: str = "a8",
    input_act: Optional[str] = None,
    chunk_tokens: Optional[int] = None,
    quant_mode: str = "ck",
) -> torch.Tensor:
    """out = act(x) @ W.T + bias over the last dim of x (qlinear.py:466-523).

    w: dense [N, K] tensor (plain F.linear in x.dtype) or W4A8Weight (HIP kernels).
    precision "a8" quantises activations to int8 per token (the native W4A8 path); "a16" keeps them (rotated x
    times the exact int8 levels, fp32 accumulation).  input_act="swiglu": x is [gate | up], silu(gate) * up in
    x.dtype first; "gelu_tanh" (an extension for the config-4 block): tanh-approximate GELU in x.dtype.  On the
    W4A8 a8 path the activation runs inside the rotate+quantise kernel.  chunk_tokens bounds peak memory; a8 is
    token-wise, so chunking is bit-exact.
    """
    if not x.is_floating_point():
        raise ValueError(f"x must be floating point, got {x.dtype}")
    if input_act not in INPUT_ACTS:
        raise ValueError(f"input_act must be None, 'swiglu' or 'gelu_tanh', got {input_act!r}")
    if chunk_tokens is not None and chunk_tokens < 1:
        raise ValueError("chunk_tokens must be >= 1")
    _check_mode(quant_mode)
    swiglu = input_act == "swiglu"
    if swiglu and x.shape[-1] % 2:
        raise ValueError(f"swiglu needs an even last dim, got {x.shape[-1]}")
    out_dtype = out_dtype or x.dtype
    kind = resolve_backend(x, w, backend, precision)
    lead = x.shape[:-1]
    x2 = x.reshape(math.prod(lead), x.shape[-1])
    if kind != "dense":
        y = _linear_w4a8(x2, w, bias, out_dtype, backend, precision, None if input_act == "none" else input_act,
                         chunk_tokens, quant_mode)
        return y.reshape(*lead, y.shape[-1])
    if x2.shape[-1] // (2 if swiglu else 1) != w.shape[-1]:
        raise ValueError(f"input features {x2.shape[-1]} do not match the dense weight {tuple(w.shape)}")
    step = chunk_tokens or max(x2.shape[0], 1)
    cpu_lowp = x.device.type == "cpu" and x.dtype in (torch.bfloat16, torch.float16)
    wd = w.to(dtype=torch.float32 if cpu_lowp else x.dtype)
    bd = None if bias is None else bias.to(dtype=wd.dtype)
    outs = []
    for a in range(0, max(x2.shape[0], 1), step):
        xc = apply_input_act(x2[a: a + step], input_act)
        outs.append(F.linear(xc.to(wd.dtype), wd, bd).to(out_dtype))
    y = outs[0] if len(outs) == 1 else torch.cat(outs, 0)
    return y.reshape(*lead, y.shape[-1])

