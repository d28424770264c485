"""CPU oracle of the H3 DiT block -- TEST INFRASTRUCTURE ONLY (never imported by the product).

Two restatements of the reference's block (h3turbo/h3/model.py:64-242 with h3turbo/h3/layout.py:264-355):

block_ref      the reference's op order in the compute dtype on the CPU (torch CPU ops), with every W4A8 linear
               computed by oracle.qlinear_ref.linear_a8 (the exact numpy restatement of the torch backend).  The
               GPU block is compared against it within a stated tolerance: attention (PyTorch-ROCm SDPA against
               fp32 CPU attention here) and norm reduction orders differ by final-bit roundings, which the int8
               activation quantiser of the following linear can amplify to one quantisation step.

block_naive    the block written straight from its mathematical definition in float64, with dense weights:
               no in-place ops, no chunking, plain softmax attention.  It pins block_ref: with fp32 compute and
               dense weights the two agree to fp32 rounding (tests/test_oracle_block.py), so a dropped term, a
               wrong gate, a swapped shift/scale or a wrong rotary pairing in block_ref fails there.

Tensors are CPU torch tensors.  Weights are dicts: dense {"qkv","out","fc1","fc2": [N, K]} or W4A8 numpy parts
{"q","s_rel","s_kind","s_ch","cb","group","convrot"} per linear, plus "norm1","norm2","q_norm","k_norm".
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

from . import qlinear_ref as ql

_DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


# --------------------------------------------------------------------------------------------- naive fp64
def block_naive(x: torch.Tensor, w: Dict[str, torch.Tensor], mods: Sequence[torch.Tensor], rows: torch.Tensor,
                cos: torch.Tensor, sin: torch.Tensor, heads: int, head_dim: int, act: str, eps: float,
                qk_eps: float) -> torch.Tensor:
    """float64 block from the definition.  rows [S]: modulation row of each token; cos/sin [S, half] (float64)."""
    d = lambda t: t.double()  # noqa: E731
    x = d(x)
    s = x.shape[0]
    norm = lambda v, g, e: v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + e) * d(g)  # noqa: E731
    sh_a, sc_a, g_a, sh_m, sc_m, g_m = (d(m)[rows] for m in mods)
    half = cos.shape[1]
    c, sn = d(cos)[:, None, :], d(sin)[:, None, :]

    def rotate(t):
        a, b, rest = t[..., :half], t[..., half:2 * half], t[..., 2 * half:]
        return torch.cat([a * c - b * sn, a * sn + b * c, rest], dim=-1)

    h = norm(x, w["norm1"], eps) * (1 + sc_a) + sh_a
    qkv = h @ d(w["qkv"]).T
    q, k, v = (qkv[:, i * heads * head_dim:(i + 1) * heads * head_dim].reshape(s, heads, head_dim) for i in range(3))
    q = rotate(norm(q, w["q_norm"], qk_eps))
    k = rotate(norm(k, w["k_norm"], qk_eps))
    att = torch.softmax(torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(head_dim), dim=-1)
    o = torch.einsum("hqk,khd->qhd", att, v).reshape(s, heads * head_dim)
    x = x + g_a * (o @ d(w["out"]).T)
    h = norm(x, w["norm2"], eps) * (1 + sc_m) + sh_m
    z = h @ d(w["fc1"]).T
    if act == "swiglu":
        gate, up = z.chunk(2, dim=-1)
        z = gate * torch.sigmoid(gate) * up
    else:
        z = 0.5 * z * (1 + torch.tanh(math.sqrt(2 / math.pi) * (z + 0.044715 * z ** 3)))
    return x + g_m * (z @ d(w["fc2"]).T)


# --------------------------------------------------------------------------------------------- reference op order
def _linear(x: torch.Tensor, wl, input_act: Optional[str] = None, mode: str = "ck") -> torch.Tensor:
    """qlinear.linear on the CPU: W4A8 through the numpy oracle, dense through F.linear (model.py:179-184)."""
    if input_act == "swiglu":  # silu(gate) * up in x.dtype (qlinear.py:376-379)
        gate, up = x.chunk(2, dim=-1)
        x = F.silu(gate).mul_(up)
    if isinstance(wl, torch.Tensor):
        return F.linear(x, wl.to(x.dtype))
    xv = x.float().numpy()
    out, *_ = ql.linear_a8(xv, _DT[x.dtype], wl["q"], wl["s_rel"], wl["s_kind"], wl["s_ch"], wl["cb"], wl["group"],
                           wl["convrot"], mode=mode)
    return torch.from_numpy(np.ascontiguousarray(out)).to(x.dtype)


def _rms_lanes(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """The fused q/k-norm order (layout.py:309-326): 32 strided partial sums, halving tree, one rounding."""
    dd = x.shape[-1]
    if x.dtype == torch.float32 or dd % 32:
        return F.rms_norm(x, (dd,), w.to(x.dtype), eps)
    xf = x.float()
    parts = xf.square().reshape(*x.shape[:-1], dd // 32, 32)
    acc = parts[..., 0, :]
    for j in range(1, dd // 32):
        acc = acc + parts[..., j, :]
    for off in (16, 8, 4, 2, 1):
        acc = acc[..., :off] + acc[..., off:2 * off]
    return (xf * torch.rsqrt(acc / dd + eps) * w.float()).to(x.dtype)


def norm_rope_ref(q: torch.Tensor, k: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, eps: float, cos: torch.Tensor,
                  sin: torch.Tensor, impl: str = "torch") -> None:
    """In place on [S, heads, D]: per-head RMSNorm then split-half rotation of the leading 2*half dims
    (layout.py:329-355).  "torch": lane-order norm rounded to the dtype, rotation in fp32 (cos/sin widened), one
    rounding.  "eager" (and fp32 inputs): F.rms_norm, rotation in the compute dtype.  Pinned by the reference's own
    norm_rope_ outputs (tests/golden/make_golden_normrope.py)."""
    half = cos.shape[1]
    c, sn = cos.unsqueeze(1), sin.unsqueeze(1)
    for t, g in ((q, wq), (k, wk)):
        if impl == "eager" or t.dtype == torch.float32:
            n = F.rms_norm(t, (t.shape[-1],), g.to(t.dtype), eps)
            t1, t2 = n[..., :half], n[..., half:2 * half]
            o1, o2 = (t1 * c).addcmul_(t2, -sn), (t2 * c).addcmul_(t1, sn)
        else:
            n = _rms_lanes(t, g, eps)
            t1, t2 = n[..., :half].float(), n[..., half:2 * half].float()
            o1, o2 = t1 * c.float() - t2 * sn.float(), t1 * sn.float() + t2 * c.float()
        n[..., :half], n[..., half:2 * half] = o1, o2
        t.copy_(n)


def _modulate(h, shift, scale, segments):  # model.py:106-109
    for a, b, r in segments:
        h[a:b].mul_(1.0 + scale[r].to(h.dtype)).add_(shift[r].to(h.dtype))
    return h


def attention_ref(h: torch.Tensor, w: Dict[str, object], cos: torch.Tensor, sin: torch.Tensor, heads: int,
                  head_dim: int, qk_eps: float, rope_impl: str = "torch", mode: str = "ck") -> torch.Tensor:
    """out(SDPA(norm_rope(q), norm_rope(k), v)) on the CPU (model.py:196-228, layout.py:329-355)."""
    return _linear(attend_ref(h, w, cos, sin, heads, head_dim, qk_eps, rope_impl, mode), w["out"], mode=mode)


def attend_ref(h: torch.Tensor, w: Dict[str, object], cos: torch.Tensor, sin: torch.Tensor, heads: int,
               head_dim: int, qk_eps: float, rope_impl: str = "torch", mode: str = "ck") -> torch.Tensor:
    """The attention output before the out projection; fp32 softmax attention rounded once to the compute dtype."""
    dt, s, inner = h.dtype, h.shape[0], heads * head_dim
    qkv = _linear(h, w["qkv"], mode=mode)
    q, k, v = (t.reshape(s, heads, head_dim).clone() for t in qkv.split(inner, dim=-1))
    norm_rope_ref(q, k, w["q_norm"], w["k_norm"], qk_eps, cos, sin, rope_impl)
    qf, kf, vf = (t.transpose(0, 1).float() for t in (q, k, v))
    att = torch.softmax((qf @ kf.transpose(1, 2)) / math.sqrt(head_dim), dim=-1)
    return (att @ vf).transpose(0, 1).reshape(s, inner).to(dt)


def mlp_ref(h: torch.Tensor, w: Dict[str, object], act: str, mode: str = "ck") -> torch.Tensor:
    """fc2(act(fc1(h))) on the CPU (model.py:186-194); gelu is the tanh approximation."""
    z = _linear(h, w["fc1"], mode=mode)
    if act == "swiglu":
        return _linear(z, w["fc2"], "swiglu", mode=mode)
    return _linear(F.gelu(z, approximate="tanh"), w["fc2"], mode=mode)


def block_ref(x: torch.Tensor, w: Dict[str, object], mods: Sequence[torch.Tensor], segments, cos: torch.Tensor,
              sin: torch.Tensor, heads: int, head_dim: int, act: str, eps: float, qk_eps: float,
              rope_impl: str = "torch", mode: str = "ck", attend: Optional[torch.Tensor] = None,
              modulated: Optional[Sequence[torch.Tensor]] = None) -> torch.Tensor:
    """The reference block (model.py:234-242) on the CPU in x.dtype; returns the new residual (x is not mutated).

    attend: an attention output [S, heads * head_dim] (before the out projection) to use in place of the one
    attend_ref computes; modulated: the two RMSNorm + modulation outputs (before attention, before the MLP) to use
    in place of the ones computed here.  With a GPU block's own values of those two steps -- whose reduction orders
    are not the reference's -- a comparison covers every other step exactly."""
    x = x.clone()
    dt = x.dtype
    sh_a, sc_a, g_a, sh_m, sc_m, g_m = mods

    def gate_add(y, gate):  # model.py:112-115
        for a, b, r in segments:
            x[a:b].addcmul_(y[a:b], gate[r].to(dt))

    rmsn = lambda v, g: F.rms_norm(v, (v.shape[-1],), g.to(v.dtype), eps)  # noqa: E731
    h = _modulate(rmsn(x, w["norm1"]), sh_a, sc_a, segments) if modulated is None else modulated[0].to(dt)
    if attend is None:
        gate_add(attention_ref(h, w, cos, sin, heads, head_dim, qk_eps, rope_impl, mode), g_a)
    else:
        gate_add(_linear(attend.to(dt), w["out"], mode=mode), g_a)
    h = _modulate(rmsn(x, w["norm2"]), sh_m, sc_m, segments) if modulated is None else modulated[1].to(dt)
    gate_add(mlp_ref(h, w, act, mode), g_m)
    return x


def dense_of(wl) -> torch.Tensor:
    """Dense fp64 [N, K] weight in the original basis of a W4A8 oracle weight: (grid * s_ch) @ H per block
    (qlinear.py:207-226, rotated=False)."""
    if isinstance(wl, torch.Tensor):
        return wl.double()
    grid = ql.decode_int8_grid(wl["q"], wl["s_rel"], wl["s_kind"], wl["cb"], wl["group"]).astype(np.float64)
    wr = grid * np.asarray(wl["s_ch"], np.float64)[:, None]
    n, k = wr.shape
    h = ql.hadamard_regular(wl["convrot"])
    return torch.from_numpy((wr.reshape(n, k // wl["convrot"], wl["convrot"]) @ h).reshape(n, k))
