"""Seeded synthetic inputs shared by the golden-vector generator, the tests and bench.py.

Everything here is deterministic on a given torch build (CPU generator) and returns plain numpy arrays in the
storage formats of the reference's W4A8Weight (h3turbo/h3/types.py:10-25):
    q      int8  [N, K/2]   two 4-bit codebook indices per byte, LOW nibble = even k
    s_rel  fp8-e4m3 bytes (uint8) [N, K/g]  or fp16 bits (uint16) [N, K/g]
    s_ch   float32 [N]
    cb     float32 [16]
Activations are bf16 bit patterns (uint16).
"""
from __future__ import annotations

import hashlib
import math

import numpy as np
import torch

# the 16 Lloyd-Max levels of a real checkpoint layer, as printed in the reference's tests
# (tests/test_h3_qlinear.py:11-13); data, not code
REAL_CB = [-0.9807561635971069, -0.7949668765068054, -0.6386534571647644, -0.5035541653633118, -0.38370054960250854,
           -0.2726648449897766, -0.1664646714925766, -0.06367518752813339, 0.03837905079126358, 0.1426069736480713,
           0.2516845762729645, 0.3661285936832428, 0.4894854724407196, 0.6280644536018372, 0.787971019744873, 0.979333221912384]


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str((a.dtype.str, a.shape)).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def bf16_bits_of(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def activations(m: int, k: int, seed: int = 0, outlier_frac: float = 0.01, outlier_scale: float = 20.0) -> np.ndarray:
    """bf16 [m, k] ~N(0,1) with round(outlier_frac*k) channels scaled x20, as uint16 bits."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    n_out = round(outlier_frac * k)
    if n_out:
        idx = torch.randperm(k, generator=g)[:n_out]
        x[:, idx] *= outlier_scale
    return bf16_bits_of(x)


def hadamard(size: int) -> np.ndarray:
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < size:
        h = np.kron(h, h4)
    return h / math.sqrt(size)


def weight_int4_g128(n: int, k: int, seed: int = 0, group: int = 128, convrot: int = 256, std: float = 0.02):
    """BASELINE recipe: W ~N(0, std) fp32 [n, k] rotated into the ConvRot basis, symmetric int4 per group with
    fp16 relative scales.  s_g = amax|W_rot| / 7 per group, c = clamp(rint(W_rot / s_g), -8, 7), nibble = c + 8,
    codebook = arange(-8, 8), s_ch = max_g s_g / 15.875, s_rel = fp16(s_g / s_ch) (<= 15.875, so |level| <= 127).
    Returns (q int8 [n, k/2], s_rel fp16 bits uint16 [n, k/group], s_ch f32 [n], cb f32 [16])."""
    g = torch.Generator().manual_seed(seed + 1000)
    w = (torch.randn(n, k, generator=g) * std).numpy().astype(np.float64)
    w_rot = np.matmul(w.reshape(n, k // convrot, convrot), hadamard(convrot)).reshape(n, k).astype(np.float32)
    blocks = w_rot.reshape(n, k // group, group)
    s_g = np.abs(blocks).max(axis=-1) / np.float32(7.0)
    s_g = np.maximum(s_g, np.float32(1e-12)).astype(np.float32)
    c = np.clip(np.rint(blocks / s_g[:, :, None]), -8, 7).astype(np.int64).reshape(n, k)
    nib = (c + 8).astype(np.uint8)
    q = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8).view(np.int8)
    s_ch = (s_g.max(axis=1) / np.float32(15.875)).astype(np.float32)
    s_rel = (s_g / s_ch[:, None]).astype(np.float16).view(np.uint16)
    cb = np.arange(-8, 8, dtype=np.float32)
    return q, s_rel, s_ch, cb


def weight_fp8_g16(n: int, k: int, seed: int = 0, group: int = 16, codebook=None):
    """The reference tests' make_weight recipe (tests/test_h3_qlinear.py:46-53): random packed codes, fp8-e4m3
    group scales 20..200 (exercises the +-127 clamp), s_ch in [0.005, 0.025), the real codebook.
    Returns (q int8 [n, k/2], s_rel fp8 bytes uint8 [n, k/group], s_ch f32 [n], cb f32 [16])."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8)
    s = (torch.rand(n, k // group, generator=g) * 180 + 20).to(torch.float8_e4m3fn)
    s_ch = torch.rand(n, generator=g) * 0.02 + 0.005
    cb = np.asarray(REAL_CB if codebook is None else codebook, dtype=np.float32)
    return q.numpy().copy(), s.view(torch.uint8).numpy().copy(), s_ch.numpy().astype(np.float32), cb


def bias(n: int, seed: int = 0) -> np.ndarray:
    g = torch.Generator().manual_seed(seed + 77)
    return torch.randn(n, generator=g).numpy().astype(np.float32)


# --------------------------------------------------------------------------------------------- DiT block inputs
def block_case(hidden: int, heads: int, head_dim: int, ffn: int, act: str, s: int, seed: int = 0, rope_freqs: int = 16,
               fmt: str = "g128"):
    """Synthetic inputs of one DiT block, all CPU torch / numpy:
    x bf16 [s, hidden] ~N(0,1); six modulation tensors fp32 [3, hidden] ~N(0, 0.1); segments (token ranges on rows
    0, 1 and a per-token row tensor); rotary cos/sin bf16 [s, 3F] from random integer (t, h, w) positions;
    norm weights ~1 + N(0, 0.1); four W4A8 linears (qkv [3*inner, hidden], out [hidden, inner],
    fc1 [ffn or 2*ffn, hidden], fc2 [hidden, ffn]) in the BASELINE int4 group-128 recipe (fmt "g128") or the
    reference tests' fp8 group-16 recipe (fmt "fp8")."""
    g = torch.Generator().manual_seed(seed)
    inner = heads * head_dim
    x = torch.randn(s, hidden, generator=g).to(torch.bfloat16)
    mods = [torch.randn(3, hidden, generator=g) * 0.1 for _ in range(6)]
    cut1, cut2 = s // 3, (2 * s) // 3
    per_token = torch.randint(0, 3, (s - cut2,), generator=g)
    segments = [(0, cut1, 0), (cut1, cut2, 1), (cut2, s, per_token)]
    pos = torch.randint(0, 64, (s, 3), generator=g)
    inv_freq = 1.0 / (10000.0 ** (torch.arange(rope_freqs, dtype=torch.float32) / rope_freqs))
    ang = (pos.float()[:, :, None] * inv_freq[None, None, :]).reshape(s, -1)
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    norms = {n: (1.0 + 0.1 * torch.randn(d, generator=g)) for n, d in
             (("norm1", hidden), ("norm2", hidden), ("q_norm", head_dim), ("k_norm", head_dim))}
    fc1_out = 2 * ffn if act == "swiglu" else ffn
    lin = {}
    for i, (name, n, k) in enumerate((("qkv", 3 * inner, hidden), ("out", hidden, inner), ("fc1", fc1_out, hidden),
                                      ("fc2", hidden, ffn))):
        if fmt == "g128":
            q, s_rel, s_ch, cb = weight_int4_g128(n, k, seed=seed * 10 + i)
            lin[name] = {"q": q, "s_rel": s_rel, "s_kind": "f16", "s_ch": s_ch, "cb": cb, "group": 128, "convrot": 256}
        else:
            q, s_rel, s_ch, cb = weight_fp8_g16(n, k, seed=seed * 10 + i)
            lin[name] = {"q": q, "s_rel": s_rel, "s_kind": "fp8", "s_ch": (s_ch * 0.05).astype(np.float32), "cb": cb,
                         "group": 16, "convrot": 256}
    return x, mods, segments, (cos, sin), norms, lin
