"""The H3 DiT block over W4A8 ConvRot linears, and the block loop that drives a BlockProvider.

Mirrors the reference's block (h3turbo/h3/model.py:64-242, h3turbo/h3/layout.py:264-355) op for op, so a block
computed here matches the reference's block up to the attention kernel (PyTorch-ROCm SDPA) and the reduction
order of the norms.  The four large linears (qkv, out, fc1, fc2) run through `qlinear.linear` on the HIP kernels;
norms, modulation, q/k norm + rotary embedding and the residual updates are torch ops on the same stream.

Sequence of one block (x is the bf16 residual stream [S, hidden], updated in place):
    h = modulate(rms(x) * norm1, shift_a, scale_a)            modulate: h * (1 + scale) + shift, per token row
    x += gate_a * out(SDPA(norm_rope(split(qkv(h)))))
    h = modulate(rms(x) * norm2, shift_m, scale_m)
    x += gate_m * fc2(act(fc1(h)))                             act: swiglu (the H3 block) or gelu (BASELINE shape)

`act="gelu"` (tanh approximation) is an extension for the BASELINE config-4 shape: the reference block only
has SwiGLU (h3turbo/h3/model.py:186-194), so that variant has no reference oracle.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F

from . import qlinear
from .types import BlockProvider, BlockWeights, W4A8Weight, Weight

# a modulation segment: tokens [start, stop) use row `row` (an int, or a LongTensor of per-token rows)
Segment = Tuple[int, int, Union[int, torch.Tensor]]
_GATHER_ROWS = 4096  # per-token row tensors are applied in pieces of this many tokens (bounds the gather)


@dataclass(frozen=True)
class BlockConfig:
    """Shape of one DiT block.  Defaults: the BASELINE config-4 block (hidden 5120, 40 x 128 heads, GELU FFN
    13824).  The real H3 block is hidden 5376, 56 heads, SwiGLU ffn 14336 (h3turbo/h3/config.py:12-19)."""

    hidden: int = 5120
    heads: int = 40
    head_dim: int = 128
    ffn: int = 13824
    act: str = "gelu"
    norm_eps: float = 1e-5
    qk_norm_eps: float = 1e-5
    rope_freqs: int = 16  # rotary frequencies per axis (3 axes: t, h, w); rotates 6 * rope_freqs head dims

    def __post_init__(self):
        if self.act not in ("swiglu", "gelu"):
            raise ValueError(f"act must be 'swiglu' or 'gelu', got {self.act!r}")
        if 6 * self.rope_freqs > self.head_dim:
            raise ValueError(f"rotary width {6 * self.rope_freqs} exceeds head_dim {self.head_dim}")

    @property
    def inner(self) -> int:
        return self.heads * self.head_dim

    @property
    def fc1_out(self) -> int:
        return 2 * self.ffn if self.act == "swiglu" else self.ffn


# ------------------------------------------------------------------------------------------------ token-wise ops
def rms(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim in x.dtype with the weight cast to x.dtype (h3turbo/h3/model.py:64-65)."""
    w = weight if weight.dtype == x.dtype else weight.to(x.dtype)
    return F.rms_norm(x, (x.shape[-1],), w, eps)


def _row_pieces(segments: Sequence[Segment]):
    for start, stop, row in segments:
        if isinstance(row, torch.Tensor):
            for c in range(0, stop - start, _GATHER_ROWS):
                yield start + c, min(stop, start + c + _GATHER_ROWS), row[c:c + _GATHER_ROWS]
        elif stop > start:
            yield start, stop, row


def modulate_(h: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, segments: Sequence[Segment]) -> torch.Tensor:
    """In place h[tokens] = (h * (1 + scale[row])) + shift[row], each step rounded to h.dtype
    (h3turbo/h3/model.py:106-109)."""
    for a, b, row in _row_pieces(segments):
        one_plus = scale[row].to(h.dtype) + 1.0
        h[a:b].mul_(one_plus).add_(shift[row].to(h.dtype))
    return h


def token_rows(segments: Sequence[Segment], s: int, device) -> Optional[torch.Tensor]:
    """The modulation row of every token as int32 [s] on `device`, or None when the segments do not cover
    [0, s) contiguously (tokens outside every segment stay unmodulated, which the fused kernel cannot express)."""
    pos = 0
    rows = torch.empty(s, dtype=torch.int32, device=device)
    for start, stop, row in segments:
        if start != pos or stop < start:
            return None
        rows[start:stop] = row.to(device=device, dtype=torch.int32) if isinstance(row, torch.Tensor) else int(row)
        pos = stop
    return rows if pos == s else None


def _kernel_vectors(k: int, *vecs: torch.Tensor):
    """The weight / modulation vectors of a fused block kernel as (tensors [R, k], their row strides, dtype code):
    fp32 vectors go to the kernel as they are when all are fp32 with unit element stride, 16-byte aligned rows and
    row strides a multiple of 8 (the kernel rounds them to bf16 as .to(torch.bfloat16) would; strided AdaLN chunks
    need no copy); otherwise each is rounded to a contiguous bf16 copy here."""
    from . import _lib

    rows = [v.reshape(-1, k) for v in vecs]
    if all(r.dtype == torch.float32 and r.stride(-1) == 1 and r.data_ptr() % 16 == 0
           and (r.shape[0] == 1 or r.stride(0) % 8 == 0) for r in rows):
        return rows, [r.stride(0) if r.shape[0] > 1 else k for r in rows], _lib.F32
    rows = [r.to(torch.bfloat16).contiguous() for r in rows]
    return rows, [k] * len(rows), _lib.BF16


def rms_modulate(x: torch.Tensor, weight: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float,
                 segments: Sequence[Segment], rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """modulate_(rms(x, weight, eps), shift, scale, segments) (h3turbo/h3/model.py:64-65, 106-109), in one HIP pass
    (h3k_rms_modulate) for bf16 on the GPU when the segments cover every token; `rows` is token_rows(segments)
    when already built.  The fused pass sums the squares in its own order, so it can differ from F.rms_norm in the
    last bit of the norm on some rows."""
    k = x.shape[-1]
    fused = (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and k % 8 == 0 and k <= 8192
             and x.stride(-1) == 1 and (x.shape[0] <= 1 or x.stride(0) % 8 == 0) and x.data_ptr() % 16 == 0)
    if fused and rows is None:
        rows = token_rows(segments, x.shape[0], x.device)
    if not fused or rows is None or shift.shape[-1] != k or scale.shape[-1] != k:
        return modulate_(rms(x, weight, eps), shift, scale, segments)
    from . import _lib

    (w, sh, sc), (_, ldsh, ldsc), vdt = _kernel_vectors(k, weight, shift, scale)
    if ldsh != ldsc:  # one row stride serves both modulation tensors
        (w, sh, sc), (_, ldsh, _), vdt = _kernel_vectors(k, weight.to(torch.bfloat16), shift, scale)
    h = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    lib = _lib.load()
    _lib.check(lib.h3k_rms_modulate(x.data_ptr(), x.stride(0) if x.shape[0] > 1 else k, x.shape[0], k, w.data_ptr(),
                                    sh.data_ptr(), sc.data_ptr(), ldsh, rows.data_ptr(), eps, h.data_ptr(), k, vdt,
                                    _lib.stream_of(x.device)), "h3k_rms_modulate")
    return h


def gated_add_(x: torch.Tensor, gate: torch.Tensor, y: torch.Tensor, segments: Sequence[Segment],
               rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """In place x[tokens] += y[tokens] * gate[row], one rounding (h3turbo/h3/model.py:112-115).  bf16 on the GPU with
    every token covered by a segment: one HIP pass over x and y (h3k_gated_add) with the gate rows rounded to bf16
    once, bit-identical to the per-segment addcmul_ (the bf16 product is exact in fp32); `rows` is
    token_rows(segments) when already built."""
    k = x.shape[-1]
    fused = (x.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16 and x.dim() == 2 and y.dim() == 2
             and k % 8 == 0 and gate.shape[-1] == k and x.stride(-1) == 1 and y.stride(-1) == 1
             and x.data_ptr() % 16 == 0 and y.data_ptr() % 16 == 0
             and (x.shape[0] <= 1 or (x.stride(0) % 8 == 0 and y.stride(0) % 8 == 0)))
    if fused and rows is None:
        rows = token_rows(segments, x.shape[0], x.device)
    if not fused or rows is None:
        for a, b, row in _row_pieces(segments):
            x[a:b].addcmul_(y[a:b], gate[row].to(x.dtype))
        return x
    from . import _lib

    (g,), (ldg,), gdt = _kernel_vectors(k, gate)
    lib = _lib.load()
    _lib.check(lib.h3k_gated_add(x.data_ptr(), x.stride(0) if x.shape[0] > 1 else k, y.data_ptr(),
                                 y.stride(0) if y.shape[0] > 1 else k, g.data_ptr(), ldg, rows.data_ptr(), x.shape[0],
                                 k, gdt, _lib.stream_of(x.device)), "h3k_gated_add")
    return x


def gated_add_rms_modulate(x: torch.Tensor, gate: torch.Tensor, y: torch.Tensor, weight: torch.Tensor,
                           shift: torch.Tensor, scale: torch.Tensor, eps: float, segments: Sequence[Segment],
                           rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gated_add_(x, gate, y) then rms_modulate(x, weight, shift, scale) (h3turbo/h3/model.py:112-115, then :64-65,
    106-109, as _block runs them between the attention and the MLP): in one HIP pass over x
    (h3k_gated_add_rms_modulate) where both would take their fused form, bit-identical to the two in sequence;
    otherwise the two in sequence.  Returns h; x is updated in place."""
    k = x.shape[-1]
    fused = (x.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16 and x.dim() == 2 and y.dim() == 2
             and k % 8 == 0 and k <= 8192 and gate.shape[-1] == k and shift.shape[-1] == k and scale.shape[-1] == k
             and x.stride(-1) == 1 and y.stride(-1) == 1 and x.data_ptr() % 16 == 0 and y.data_ptr() % 16 == 0
             and (x.shape[0] <= 1 or (x.stride(0) % 8 == 0 and y.stride(0) % 8 == 0)))
    if fused and rows is None:
        rows = token_rows(segments, x.shape[0], x.device)
    if not fused or rows is None:
        gated_add_(x, gate, y, segments, rows)
        return rms_modulate(x, weight, shift, scale, eps, segments, rows)
    from . import _lib

    (g, w, sh, sc), (ldg, _, ldsh, ldsc), vdt = _kernel_vectors(k, gate, weight, shift, scale)
    if ldsh != ldsc:  # one row stride serves both modulation tensors
        (g, w, sh, sc), (ldg, _, ldsh, _), vdt = _kernel_vectors(k, gate, weight.to(torch.bfloat16), shift, scale)
    h = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    lib = _lib.load()
    _lib.check(lib.h3k_gated_add_rms_modulate(x.data_ptr(), x.stride(0) if x.shape[0] > 1 else k, y.data_ptr(),
                                              y.stride(0) if y.shape[0] > 1 else k, g.data_ptr(), ldg, x.shape[0], k,
                                              w.data_ptr(), sh.data_ptr(), sc.data_ptr(), ldsh, rows.data_ptr(), eps,
                                              h.data_ptr(), k, vdt, _lib.stream_of(x.device)),
               "h3k_gated_add_rms_modulate")
    return h


def rope_angles(position_ids: torch.Tensor, inv_freq: torch.Tensor, device) -> torch.Tensor:
    """[S, 3] positions x [F] inverse frequencies -> fp32 angles [S, 3F], axis-major (h3turbo/h3/layout.py:264-271)."""
    pos = position_ids.to(device=device, dtype=torch.float32)
    return (pos[:, :, None] * inv_freq.to(device=device, dtype=torch.float32)[None, None, :]).reshape(pos.shape[0], -1)


def rope_tables(position_ids: torch.Tensor, inv_freq: torch.Tensor, device, dtype: torch.dtype):
    """(cos, sin) [S, 3F] rounded to the compute dtype (h3turbo/h3/model.py:283-289)."""
    ang = rope_angles(position_ids, inv_freq, device)
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def rms_lanewise(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm with the summation order of the fused q/k-norm kernel the reference reproduces
    (h3turbo/h3/layout.py:309-326): 32 partial sums, partial l collecting the squares of elements l, l+32, ... in
    order, then a halving tree (16, 8, 4, 2, 1); x * rsqrt(sum/d + eps) * w in fp32, rounded once."""
    d = x.shape[-1]
    if x.dtype == torch.float32 or d % 32:
        return F.rms_norm(x, (d,), weight.to(x.dtype), eps)
    xf = x.float()
    cols = xf.square().unflatten(-1, (d // 32, 32))
    part = cols[..., 0, :]
    for j in range(1, d // 32):
        part = part + cols[..., j, :]
    width = 32
    while width > 1:
        width //= 2
        part = part[..., :width] + part[..., width:2 * width]
    return (xf * torch.rsqrt(part / d + eps) * weight.float()).to(x.dtype)


def norm_rope_(q: torch.Tensor, k: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, eps: float, cos: torch.Tensor,
               sin: torch.Tensor, impl: str = "torch", chunk: int = 1024) -> None:
    """Per-head RMSNorm, then split-half rotation of the leading 2 * half dims, in place on [S, heads, D] views
    (h3turbo/h3/layout.py:329-355).
      "torch": lane-order norm rounded to the dtype, rotation in fp32, one rounding (the fused kernel's numerics)
      "eager": F.rms_norm and the rotation in the compute dtype (two roundings); fp32 inputs always take it."""
    if impl not in ("torch", "eager"):
        raise ValueError(f"rope impl must be 'torch' or 'eager', got {impl!r}")
    half = cos.shape[1]
    if impl == "torch" and _fused_norm_rope_ok(q, k):
        _fused_norm_rope(q, k, wq, wk, eps, cos, sin)
        return
    for t, w in ((q, wq), (k, wk)):
        for a in range(0, t.shape[0], chunk):
            rows = slice(a, a + chunk)
            c, s = cos[rows].unsqueeze(1), sin[rows].unsqueeze(1)
            if impl == "eager" or t.dtype == torch.float32:
                n = F.rms_norm(t[rows], (t.shape[-1],), w.to(t.dtype), eps)
                lo, hi = n[..., :half], n[..., half:2 * half]
                new_lo = (lo * c).addcmul_(hi, -s)
                new_hi = (hi * c).addcmul_(lo, s)
            else:
                n = rms_lanewise(t[rows], w, eps)
                cf, sf = c.float(), s.float()
                lo, hi = n[..., :half].float(), n[..., half:2 * half].float()
                new_lo, new_hi = lo * cf - hi * sf, lo * sf + hi * cf
            n[..., :half] = new_lo
            n[..., half:2 * half] = new_hi
            t[rows] = n


def _fused_norm_rope_ok(q: torch.Tensor, k: torch.Tensor) -> bool:
    d = q.shape[-1]
    return (q.is_cuda and q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and q.shape == k.shape
            and d % 32 == 0 and d <= 256 and all(t.stride(2) == 1 and t.stride(1) == d for t in (q, k)))


def _fused_norm_rope(q, k, wq, wk, eps, cos, sin) -> None:
    """The same numerics in one HIP kernel over both tensors (h3k_qk_norm_rope)."""
    from . import _lib

    tokens, heads, d = q.shape
    c, s = cos.float().contiguous(), sin.float().contiguous()
    w_q, w_k = wq.float().contiguous(), wk.float().contiguous()
    lib = _lib.load()
    _lib.check(lib.h3k_qk_norm_rope(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), tokens, heads, d,
                                    w_q.data_ptr(), w_k.data_ptr(), c.data_ptr(), s.data_ptr(), c.shape[1], c.shape[1],
                                    eps, _lib.stream_of(q.device)), "h3k_qk_norm_rope")


def _split_norm_rope_ok(qkv: torch.Tensor, heads: int, head_dim: int, rope) -> bool:
    """The fused split kernel's preconditions: bf16 rows with a contiguous last dim, each lane's head_dim/16-byte
    access aligned."""
    vb = head_dim // 16
    return (rope is not None and qkv.is_cuda and qkv.dtype == torch.bfloat16 and head_dim in (32, 64, 128, 256)
            and qkv.stride(-1) == 1 and qkv.shape[-1] == 3 * heads * head_dim and qkv.data_ptr() % vb == 0
            and (qkv.shape[0] <= 1 or (2 * qkv.stride(0)) % vb == 0))


_ROPE_F32: dict = {}


def _rope_f32(cos: torch.Tensor, sin: torch.Tensor):
    """The rope tables widened to contiguous fp32 (exact), once per pair of tables: every block of a forward passes
    the same two tensors.  One entry, kept with the source tensors (so their ids cannot be reused while cached) and
    their version counters (an in-place change invalidates it).  Inference-mode tensors keep no version counter,
    so they are widened on every call."""
    if cos.is_inference() or sin.is_inference():
        return cos.float().contiguous(), sin.float().contiguous()
    key = (id(cos), id(sin))
    hit = _ROPE_F32.get(key)
    if hit is not None and hit[0] is cos and hit[1] is sin and hit[2] == (cos._version, sin._version):
        return hit[3], hit[4]
    c, sn = cos.float().contiguous(), sin.float().contiguous()
    _ROPE_F32.clear()
    _ROPE_F32[key] = (cos, sin, (cos._version, sin._version), c, sn)
    return c, sn


def qkv_split_norm_rope(qkv: torch.Tensor, heads: int, head_dim: int, wq: torch.Tensor, wk: torch.Tensor, eps: float,
                        cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The qkv projection output [S, 3 * heads * head_dim] -> head-major [3, heads, S, head_dim] (q, k, v) with the
    "torch" norm + rope applied to q and k, in one HIP kernel (h3k_qkv_split_norm_rope).  Bit-identical to
    splitting, norm_rope_(q, k, ..., impl="torch") and transposing each part to [heads, S, head_dim]
    (h3turbo/h3/model.py:196-214, layout.py:329-355)."""
    from . import _lib

    s = qkv.shape[0]
    out = torch.empty(3, heads, s, head_dim, dtype=qkv.dtype, device=qkv.device)
    c, sn = _rope_f32(cos, sin)
    w_q, w_k = wq.float().contiguous(), wk.float().contiguous()
    lib = _lib.load()
    _lib.check(lib.h3k_qkv_split_norm_rope(qkv.data_ptr(), qkv.stride(0) if s > 1 else qkv.shape[1], s, heads, head_dim,
                                           w_q.data_ptr(), w_k.data_ptr(), c.data_ptr(), sn.data_ptr(), c.shape[1],
                                           c.shape[1], eps, out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
                                           s * head_dim, _lib.stream_of(qkv.device)), "h3k_qkv_split_norm_rope")
    return out


# ------------------------------------------------------------------------------------------------ the block
class DiTBlock:
    """Runs H3 DiT blocks on the GPU with W4A8 (or dense) linears.

    backend / precision / quant_mode: passed to qlinear.linear ("hip"; "a8" native W4A8 or "a16").
    mlp_chunk / attn_chunk: token / query chunks bounding peak memory (both exact: the ops are token-wise and
    query rows are independent), as the reference's mlp_chunk / attn_chunk (h3turbo/h3/model.py:186-228).
    rope_impl: "torch" or "eager" (see norm_rope_).
    """

    def __init__(self, cfg: BlockConfig, *, backend: str = "auto", precision: str = "a8", quant_mode: str = "ck",
                 mlp_chunk: Optional[int] = None, attn_chunk: Optional[int] = None, rope_impl: str = "torch",
                 rope_chunk: int = 1024):
        for name, v in (("mlp_chunk", mlp_chunk), ("attn_chunk", attn_chunk), ("rope_chunk", rope_chunk)):
            if v is not None and v < 1:
                raise ValueError(f"{name} must be >= 1")
        if rope_impl not in ("torch", "eager"):
            raise ValueError(f"rope_impl must be 'torch' or 'eager', got {rope_impl!r}")
        self.cfg, self.backend, self.precision, self.quant_mode = cfg, backend, precision, quant_mode
        self.mlp_chunk, self.attn_chunk, self.rope_impl, self.rope_chunk = mlp_chunk, attn_chunk, rope_impl, rope_chunk

    # -------------------------------------------------------------------------------------------- linears
    def linear(self, x: torch.Tensor, w: Weight, input_act: Optional[str] = None) -> torch.Tensor:
        """One of the block's four large linears (h3turbo/h3/model.py:179-184)."""
        if isinstance(w, torch.Tensor):  # dense weight: plain F.linear in x.dtype
            x = qlinear.apply_input_act(x, input_act)
            return F.linear(x, w if w.dtype == x.dtype else w.to(x.dtype))
        return qlinear.linear(x, w, backend=self.backend, precision=self.precision, input_act=input_act,
                              quant_mode=self.quant_mode)

    def mlp(self, h: torch.Tensor, w: BlockWeights) -> torch.Tensor:
        """fc2(act(fc1(h))), in token chunks when mlp_chunk is set (h3turbo/h3/model.py:186-194)."""
        def run(hc):
            z = self.linear(hc, w.fc1)
            if self.cfg.act == "swiglu":
                return self.linear(z, w.fc2, "swiglu")
            return self.linear(z, w.fc2, "gelu_tanh")  # W4A8 a8: the GELU runs inside rotate+quantise

        s = h.shape[0]
        step = self.mlp_chunk or s
        if step >= s:
            return run(h)
        out = torch.empty(s, self.cfg.hidden, dtype=h.dtype, device=h.device)
        for a in range(0, s, step):
            out[a:a + step] = run(h[a:a + step])
        return out

    def attention(self, h: torch.Tensor, w: BlockWeights, rope: Optional[Tuple[torch.Tensor, torch.Tensor]]) -> torch.Tensor:
        """out(SDPA(norm_rope(q), norm_rope(k), v)) (h3turbo/h3/model.py:196-228).  rope None: plain per-head norm."""
        o = self.attend(h, w, rope, head_major=self._fused_attention(w))
        if o.dim() == 3:  # head-major [heads, S, head_dim]: the out projection reads it without a transpose copy
            return qlinear.linear_heads(o, w.out, quant_mode=self.quant_mode)
        return self.linear(o, w.out)

    def _fused_attention(self, w: BlockWeights) -> bool:
        """Whether the attention runs on the fused HIP prologue / epilogue (split + norm + rope into head-major
        q, k, v; the out projection reading the head-major attention output): W4A8 a8 linears, "torch" rope."""
        return (isinstance(w.qkv, W4A8Weight) and isinstance(w.out, W4A8Weight) and self.precision == "a8"
                and self.rope_impl == "torch" and self.cfg.head_dim in (32, 64, 128, 256))

    def attend(self, h: torch.Tensor, w: BlockWeights, rope: Optional[Tuple[torch.Tensor, torch.Tensor]],
               head_major: bool = False) -> torch.Tensor:
        """The attention output before the out projection: [S, heads * head_dim] in h.dtype, or with head_major
        (and the fused prologue applicable) [heads, S, head_dim]."""
        cfg = self.cfg
        s = h.shape[0]
        qkv = self.linear(h, w.qkv)
        if head_major and _split_norm_rope_ok(qkv, cfg.heads, cfg.head_dim, rope):
            qkvh = qkv_split_norm_rope(qkv, cfg.heads, cfg.head_dim, w.q_norm, w.k_norm, cfg.qk_norm_eps, rope[0], rope[1])
            del qkv
            qh, kh, vh = (qkvh[i].unsqueeze(0) for i in range(3))
            step = self.attn_chunk or s
            if step >= s:
                return _sdpa(qh, kh, vh)[0]
            o = torch.empty(cfg.heads, s, cfg.head_dim, dtype=h.dtype, device=h.device)
            for a in range(0, s, step):
                o[:, a:a + step] = _sdpa(qh[:, :, a:a + step], kh, vh)[0]
            return o
        q, k, v = (t.view(s, cfg.heads, cfg.head_dim) for t in qkv.split(cfg.inner, dim=-1))
        if rope is None:
            q, k = rms(q, w.q_norm, cfg.qk_norm_eps), rms(k, w.k_norm, cfg.qk_norm_eps)
        else:
            norm_rope_(q, k, w.q_norm, w.k_norm, cfg.qk_norm_eps, rope[0], rope[1], self.rope_impl, self.rope_chunk)
        # [1, heads, S, D], each contiguous: the flash / memory-efficient kernels take them directly
        qh, kh, vh = (t.transpose(0, 1).unsqueeze(0).contiguous() for t in (q, k, v))
        del qkv, q, k, v
        step = self.attn_chunk or s
        if step >= s:
            o = _sdpa(qh, kh, vh)[0].transpose(0, 1).reshape(s, cfg.inner)
        else:
            o = torch.empty(s, cfg.inner, dtype=h.dtype, device=h.device)
            for a in range(0, s, step):
                o[a:a + step] = _sdpa(qh[:, :, a:a + step], kh, vh)[0].transpose(0, 1).reshape(-1, cfg.inner)
        return o

    # -------------------------------------------------------------------------------------------- modulation
    @staticmethod
    def adaln(t_emb: torch.Tensor, w: BlockWeights, parts: int = 6, mods: int = 3) -> List[torch.Tensor]:
        """Modulation rows from the timestep embedding: F.linear(t_emb, adaln_w, adaln_b) viewed as
        [T * mods, parts * hidden] and split into `parts` tensors (h3turbo/h3/model.py:230-232)."""
        if w.adaln_w is None or w.adaln_b is None:
            raise ValueError("DiT block weights need adaln_w/adaln_b")
        z = F.linear(t_emb, w.adaln_w.to(t_emb.dtype), w.adaln_b.to(t_emb.dtype))
        return list(z.view(t_emb.shape[0] * mods, -1).chunk(parts, dim=-1))

    def forward(self, x: torch.Tensor, w: BlockWeights, mods: Sequence[torch.Tensor], segments: Sequence[Segment],
                rope: Optional[Tuple[torch.Tensor, torch.Tensor]]) -> torch.Tensor:
        """One block, in place on the residual x [S, hidden] (h3turbo/h3/model.py:234-242).
        mods: (shift_a, scale_a, gate_a, shift_m, scale_m, gate_m), each [rows, hidden]; segments map tokens to rows."""
        if len(mods) != 6:
            raise ValueError(f"a DiT block takes 6 modulation tensors, got {len(mods)}")
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = mods
        eps = self.cfg.norm_eps
        rows = token_rows(segments, x.shape[0], x.device) if x.is_cuda else None
        h = rms_modulate(x, w.norm1, sh_a, sc_a, eps, segments, rows)
        h = gated_add_rms_modulate(x, g_a, self.attention(h, w, rope), w.norm2, sh_m, sc_m, eps, segments, rows)
        return gated_add_(x, g_m, self.mlp(h, w), segments, rows)

    __call__ = forward

    def forward_temb(self, x, w: BlockWeights, t_emb: torch.Tensor, segments, rope) -> torch.Tensor:
        """The reference's `_block(x, w, t_emb, segments, rope)`: modulation computed from t_emb first."""
        return self.forward(x, w, self.adaln(t_emb, w), segments, rope)


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Exact attention on the GPU's flash / memory-efficient kernels for 16-bit inputs.  The unfused math backend
    never sees 16-bit inputs on the GPU (it would materialise [heads, S, S] scores and run batched 16-bit products
    on transposed operands); fp32 inputs, which the flash kernels do not take, use it."""
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        fp32 = q.dtype == torch.float32
        with sdpa_kernel([SDPBackend.MATH] if fp32 else [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v)
    return F.scaled_dot_product_attention(q, k, v)


# ------------------------------------------------------------------------------------------------ providers / loop
class ResidentProvider:
    """Every block already on the compute device (h3turbo/h3/model.py:45-61)."""

    def __init__(self, blocks: Sequence[BlockWeights]):
        self.blocks = list(blocks)

    def begin_forward(self) -> None:
        pass

    def acquire(self, i: int) -> BlockWeights:
        return self.blocks[i]

    def release(self, i: int) -> None:
        pass

    def end_forward(self) -> None:
        pass


def run_blocks(block: DiTBlock, x: torch.Tensor, provider: BlockProvider, layers: int, mods_of, segments,
               rope) -> torch.Tensor:
    """The model's block loop over a provider (h3turbo/h3/model.py:434-444): begin_forward; for each block
    acquire -> block -> release (release also on error); end_forward always.  mods_of(i, w) returns the six
    modulation tensors of block i (for example DiTBlock.adaln of a timestep embedding, or fixed tensors)."""
    provider.begin_forward()
    try:
        for i in range(layers):
            w = provider.acquire(i)
            try:
                x = block.forward(x, w, mods_of(i, w), segments, rope)
            finally:
                provider.release(i)
    finally:
        provider.end_forward()
    return x
