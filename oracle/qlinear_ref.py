"""CPU oracle for the W4A8 ConvRot QLinear path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the numerics of the reference's portable torch backend with
quant_mode="ck" (and "eager"), function by function.  It is the checker the HIP kernels are compared
against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it; the product
(the h3turbo_amd package and its HIP library) never does.

Pinning (what checks each function against something other than its own formula) lives in
tests/test_oracle_*.py:
  hadamard_regular      closed form (kron of H4) + symmetric/involutory/dyadic entries + golden vectors
  hadamard_pow2 / rotation_scale (sizes that are not powers of 4: an extension the reference rejects)
                        an element-wise sign formula built independently of np.kron, orthogonality, the
                        all-ones closed form that places H2 on the top bit, correctly rounded sqrt(2)
  rotate_f32            brute-force rational arithmetic on tiny inputs + golden vectors; for the extension
                        sizes, a digit-by-digit separable application of the factors
  quantize_rows         closed form KATs (degenerate rows), the division lemma, golden vectors of the
                        reference's own quantize_activation (tests/golden/)
  fp8_e4m3fn_to_f32     element-by-element OCP E4M3FN definition for all 256 bytes
  decode_int8_grid      element loops, the tie/clamp known-answer table of the reference's tests,
                        golden vectors
  int8_mm / int8_mm_emulated   brute-force int64 products including worst-case magnitudes
  epilogue / linear_a8  golden vectors of the reference's linear() on Gaussian+outlier inputs

Floating-point types without numpy support are modelled on float32 arrays: a "bf16 value" is a float32
whose low 16 bits are zero, produced by round-to-nearest-even (bf16_round).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

EPS_SCALE = np.float32(1e-30)  # reference h3turbo/h3/qlinear.py:35
EXACT_K = 1024  # reference h3turbo/h3/qlinear.py:36 (fp32-exact K chunk of the CPU GEMM emulation)
_H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)  # qlinear.py:31

BF16_TINY = np.float32(2.0 ** -126)  # torch.finfo(torch.bfloat16).tiny
F16_TINY = np.float32(2.0 ** -14)  # torch.finfo(torch.float16).tiny


# ----------------------------------------------------------------------------------------- number formats
def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32.  NaN stays NaN (quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, (x.view(np.uint32) | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), out)
    return out.view(np.float32).reshape(x.shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16-valued float32 array -> uint16 bit patterns."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values -> values of `dtype` ('bf16' | 'f16' | 'f32'), as float32 (RNE)."""
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unsupported dtype {dtype!r}")


def fp8_e4m3fn_to_f32(b: np.ndarray) -> np.ndarray:
    """OCP E4M3FN bytes -> float32: bias 7, subnormals below 2^-6, no infinities, S.1111.111 is NaN."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e, m = (b >> 3) & 0xF, b & 7
    val = np.where(e == 0, (m / 8.0) * 2.0 ** -6, (1 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 0xF) & (m == 7), np.nan, val)
    return (sign * val).astype(np.float32)


# ----------------------------------------------------------------------------------------- Hadamard / rotation
def hadamard_regular(size: int) -> np.ndarray:
    """H = kron(H4, ..., H4) / sqrt(size), float64.  Reference h3turbo/h3/qlinear.py:44-66 (power of 4 only)."""
    n = size
    while n > 1 and n % 4 == 0:
        n //= 4
    if size < 4 or n != 1:
        raise ValueError(f"regular Hadamard size must be a power of 4 (>= 4), got {size}")
    h = _H4
    while h.shape[0] < size:
        h = np.kron(h, _H4)
    return h / math.sqrt(size)


_H2 = np.array([[1, 1], [1, -1]], dtype=np.float64)


def hadamard_pow2(size: int) -> np.ndarray:
    """Unnormalised +-1 Hadamard of a power-of-2 size in [4, 1024]: kron(H4, ..., H4) for powers of 4, else
    kron(H2, H4, ..., H4) with H2 as the most significant factor.  Extension of the reference (which accepts powers
    of 4 only): for a power of 4 it is hadamard_regular(size) * sqrt(size)."""
    if size < 4 or size > 1024 or size & (size - 1):
        raise ValueError(f"rotation size must be a power of 2 in [4, 1024], got {size}")
    h = _H4
    while h.shape[0] * 4 <= size:
        h = np.kron(h, _H4)
    return np.kron(_H2, h) if h.shape[0] < size else h


def rotation_scale(size: int) -> float:
    """1/sqrt(size) in fp64: exact for powers of 4; RN(sqrt(2)) * 2^-(log2(size) + 1) / 2 otherwise."""
    bits = size.bit_length() - 1
    if bits % 2 == 0:
        return 2.0 ** -(bits // 2)
    return math.sqrt(2.0) * 2.0 ** -((bits + 1) // 2)


def rotate_f32(x: np.ndarray, size: int) -> np.ndarray:
    """[M, K] float values -> float32 [M, K]: block-wise x @ H accumulated in float64, rounded once.

    Reference h3turbo/h3/qlinear.py:105-115 (`_rot32`, CPU branch: fp64 matmul then .float()).  Sizes that are not
    powers of 4 (extension): the exact fp64 sum x @ hadamard_pow2(size), times rotation_scale(size) (one fp64
    rounding), rounded to float32.
    """
    x = np.asarray(x)
    m, k = x.shape
    if k % size:
        raise ValueError(f"last dim {k} is not a multiple of the rotation block {size}")
    blocks = x.astype(np.float64).reshape(m, k // size, size)
    if size & 0x155555:  # a power of 4: the reference's normalised matrix
        y = np.matmul(blocks, hadamard_regular(size))
    else:
        y = np.matmul(blocks, hadamard_pow2(size)) * rotation_scale(size)
    return y.reshape(m, k).astype(np.float32)


# ----------------------------------------------------------------------------------------- activation quantiser
def quantize_rows(x: np.ndarray, dtype: str, size: int = 256, mode: str = "ck") -> Tuple[np.ndarray, np.ndarray]:
    """Rotate + per-row int8 quantisation of x (float32 array holding `dtype` values).

    Reference h3turbo/h3/qlinear.py:267-292 (`_quantize_rows`):
      y32 = rotation (fp32); amax from y32 ("ck") or from y = round_dtype(y32) ("eager");
      xs = max(amax / 127, 1e-30) in fp32; s = round_dtype(xs), 0 -> finfo(dtype).tiny;
      q = clamp(rint_half_even(round_dtype(y / s)), -128, 127).
    Returns (q int8 [M, K], xs float32 [M, 1]).
    """
    if mode not in ("ck", "eager"):
        raise ValueError(f"quant_mode must be 'ck' or 'eager', got {mode!r}")
    x = np.asarray(x, dtype=np.float32)
    y32 = rotate_f32(x, size)
    y = round_to(y32, dtype)
    src = y32 if mode == "ck" else y
    if src.shape[1] == 0:
        amax = np.zeros((src.shape[0], 1), np.float32)
    else:
        amax = np.maximum(src.max(axis=1, keepdims=True), -src.min(axis=1, keepdims=True)).astype(np.float32)
    xs = np.maximum(amax / np.float32(127.0), EPS_SCALE).astype(np.float32)
    s = round_to(xs, dtype)
    tiny = {"bf16": BF16_TINY, "f16": F16_TINY, "f32": np.float32(np.finfo(np.float32).tiny)}[dtype]
    s = np.where(s == 0, tiny, s).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        quot = round_to((y / s).astype(np.float32), dtype)
    q = np.clip(np.rint(quot), -128, 127).astype(np.int8)
    return q, xs


# ----------------------------------------------------------------------------------------- int4 -> int8 grid
def unpack_nibbles(q: np.ndarray) -> np.ndarray:
    """int8/uint8 [N, K/2] -> codes [N, K]: code 2j is the LOW nibble of byte j (types.py:14-17)."""
    b = np.asarray(q).view(np.uint8).astype(np.int64)
    n, kh = b.shape
    codes = np.empty((n, 2 * kh), dtype=np.int64)
    codes[:, 0::2] = b & 0xF
    codes[:, 1::2] = b >> 4
    return codes


def decode_int8_grid(q: np.ndarray, s_rel: np.ndarray, s_kind: str, codebook: np.ndarray, group: int) -> np.ndarray:
    """int8 [N, K] = clamp(rint_half_even(f32(codebook[nibble]) * f32(s_rel[n, k // group])), -127, 127).

    Reference h3turbo/h3/qlinear.py:157-191: the fp8 scale path uses a pair LUT of exactly this formula with
    NaN scales mapped to 0 (nan_to_num, :162); the generic (fp16/bf16/fp32 scale) path uses it directly.
    s_kind: 'fp8' (uint8 bytes of E4M3FN), 'f16', 'bf16' (uint16 bits) or 'f32'.
    """
    codes = unpack_nibbles(q)
    n, k = codes.shape
    if s_kind == "fp8":
        s = fp8_e4m3fn_to_f32(s_rel)
    elif s_kind == "f16":
        s = np.asarray(s_rel).view(np.float16).astype(np.float32)
    elif s_kind == "bf16":
        s = bf16_from_bits(np.asarray(s_rel).view(np.uint16))
    elif s_kind == "f32":
        s = np.asarray(s_rel, dtype=np.float32)
    else:
        raise ValueError(f"unknown scale kind {s_kind!r}")
    if s.shape != (n, k // group):
        raise ValueError(f"s_rel must have shape {(n, k // group)}, got {s.shape}")
    cb = np.asarray(codebook, dtype=np.float32)
    prod = (cb[codes].reshape(n, k // group, group) * s[:, :, None]).astype(np.float32).reshape(n, k)
    with np.errstate(invalid="ignore"):
        lv = np.clip(np.rint(np.nan_to_num(prod, nan=0.0)), -127, 127)
    return lv.astype(np.int8)


# ----------------------------------------------------------------------------------------- int8 GEMM
def int8_mm(a: np.ndarray, w8: np.ndarray) -> np.ndarray:
    """Exact int32 a[M, K] @ w8[N, K].T.  float64 BLAS is exact here: |sum| <= K * 16384 < 2^53."""
    a = np.asarray(a, dtype=np.int8)
    w8 = np.asarray(w8, dtype=np.int8)
    if a.shape[1] * 16384 >= 2 ** 53:
        raise ValueError("K too large for the float64-exact product")
    return np.matmul(a.astype(np.float64), w8.astype(np.float64).T).astype(np.int64).astype(np.int32)


def int8_mm_emulated(a: np.ndarray, w8: np.ndarray, chunk: int = EXACT_K) -> np.ndarray:
    """The reference's CPU algorithm: fp32 GEMMs over K chunks of 1024 (each partial sum an exact integer
    below 2^24), summed in int32.  Reference h3turbo/h3/qlinear.py:250-254."""
    m, k = a.shape
    acc = np.zeros((m, w8.shape[0]), dtype=np.int32)
    for k0 in range(0, k, chunk):
        part = np.matmul(a[:, k0:k0 + chunk].astype(np.float32), w8[:, k0:k0 + chunk].astype(np.float32).T)
        acc += part.astype(np.int32)
    return acc


# ----------------------------------------------------------------------------------------- epilogue / full op
def epilogue(acc: np.ndarray, xs: np.ndarray, s_ch: np.ndarray, out_dtype: str, mode: str = "ck",
             bias: Optional[np.ndarray] = None) -> np.ndarray:
    """Reference h3turbo/h3/qlinear.py:399-405.
      ck    : out = round_out(f32(f32(acc) * xs) * s_ch)
      eager : out = round_out(f32(acc) * f32(xs * s_ch))
      bias  : out = round_out(f32(out) + f32(round_out(bias)))  (added after the output rounding)
    """
    accf = np.asarray(acc).astype(np.float32)
    xs = np.asarray(xs, dtype=np.float32).reshape(-1, 1)
    ws = np.asarray(s_ch, dtype=np.float32).reshape(1, -1)
    if mode == "ck":
        out = round_to((accf * xs).astype(np.float32) * ws, out_dtype)
    else:
        out = round_to(accf * (xs * ws).astype(np.float32), out_dtype)
    if bias is not None:
        b = round_to(np.asarray(bias, dtype=np.float32).reshape(1, -1), out_dtype)
        out = round_to((out + b).astype(np.float32), out_dtype)
    return out.astype(np.float32)


def linear_a8(x: np.ndarray, x_dtype: str, q: np.ndarray, s_rel: np.ndarray, s_kind: str, s_ch: np.ndarray,
              codebook: np.ndarray, group: int, convrot: int, *, out_dtype: Optional[str] = None, mode: str = "ck",
              bias: Optional[np.ndarray] = None, emulate: bool = False):
    """Full W4A8 a8 linear on [M, K] rows: returns (out float32 holding out_dtype values, xq, xs, acc).
    Reference h3turbo/h3/qlinear.py:396-405 (`_TorchRunner._a8`) with decode per call (:388)."""
    out_dtype = out_dtype or x_dtype
    xq, xs = quantize_rows(x, x_dtype, convrot, mode)
    w8 = decode_int8_grid(q, s_rel, s_kind, codebook, group)
    acc = (int8_mm_emulated if emulate else int8_mm)(xq, w8)
    return epilogue(acc, xs, s_ch, out_dtype, mode, bias), xq, xs, acc


def linear_a16(x: np.ndarray, x_dtype: str, q: np.ndarray, s_rel: np.ndarray, s_kind: str, s_ch: np.ndarray,
               codebook: np.ndarray, group: int, convrot: int, *, out_dtype: Optional[str] = None,
               bias: Optional[np.ndarray] = None):
    """W4A8 linear with unquantised activations.  Reference h3turbo/h3/qlinear.py:407-424 (`_TorchRunner._a16`):
    xr = rotate(x) rounded to x's dtype; y = xr @ levels^T accumulated in fp32 (tensor cores, any order); y *= s_ch;
    y += bias (fp32); rounded once to out_dtype.  The oracle takes the exact sum (fp64 of bf16/f16 values times int8
    levels), rounds it once to fp32, then applies s_ch and bias in fp32: the fp32-accumulated result of any summation
    order lies within K * 2^-24 * sum|xr * level| of that sum.  Returns (out float32 holding out_dtype values, y_exact
    fp64, abs_sum fp64) so a test can bound the accumulation error."""
    out_dtype = out_dtype or x_dtype
    xr = round_to(rotate_f32(x, convrot), x_dtype).astype(np.float64)
    w8 = decode_int8_grid(q, s_rel, s_kind, codebook, group).astype(np.float64)
    y_exact = xr @ w8.T
    abs_sum = np.abs(xr) @ np.abs(w8).T
    y = (y_exact.astype(np.float32) * np.asarray(s_ch, np.float32)[None, :]).astype(np.float32)
    if bias is not None:
        y = (y + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    return round_to(y, out_dtype), y_exact, abs_sum


# ----------------------------------------------------------------------------------------- swiglu / gelu
def swiglu_bf16(h: np.ndarray) -> np.ndarray:
    """silu(gate) * up on [gate | up] halves, each op rounded to bf16 (qlinear.py:376-379)."""
    k = h.shape[-1] // 2
    gate, up = h[..., :k].astype(np.float32), h[..., k:].astype(np.float32)
    silu = bf16_round((gate / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32))
    return bf16_round((silu * up).astype(np.float32))
