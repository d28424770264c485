"""CPU oracle of the whole H3 model forward -- TEST INFRASTRUCTURE ONLY (never imported by the product).

Two restatements of the reference's forward (h3turbo/h3/model.py:251-448):

model_ref    the reference's op order in the compute dtype with torch CPU ops: condition_proj + token refiner
             (model.py:244-266), fp32 patch projections and assembly (model.py:302-343), AdaLN rows from the
             curve table (layout.py:380-386), every DiT block through oracle.block_ref.block_ref (W4A8 linears by
             the numpy QLinear oracle), the final RMSNorm + modulation + output heads (model.py:345-365) and
             unpatchify / unpack (model.py:446-448).  The checkpoint's fp32 "islands" are rounded through the
             compute dtype as the reference does by default (model.py:168-171).

model_naive  the forward written from its mathematical definition in float64 with dense weights: no in-place
             ops, no chunking, plain softmax attention.  It pins model_ref: with fp32 compute the two agree to fp32
             rounding (tests/test_oracle_model.py), so a dropped term, a swapped shift / scale, a wrong gate or a
             wrong token order fails there.

Both take the packed-sequence plan as data (`plan`: segments, position ids, modulation rows, t values, final
rows), built by the caller with the layout module, whose bookkeeping is pinned separately by the reference's
known-answer tests and golden vectors (tests/test_layout.py).  Conditioning rows are passed already packed.

Weights: `sd` is a ComfyUI-layout state dict of CPU tensors (dense linears); `linears` optionally maps a linear's
prefix (e.g. "blocks.0.attn.qkv_proj") to a W4A8 weight in the numpy form oracle.qlinear_ref uses.
"""
from __future__ import annotations

import math
from typing import Dict, Mapping, Optional, Sequence

import torch
import torch.nn.functional as F

from . import block_ref as br

_LIN = {"qkv": "attn.qkv_proj", "out": "attn.out_proj", "fc1": "mlp.fc1", "fc2": "mlp.fc2"}


# --------------------------------------------------------------------------------------------- shared helpers
def patchify(latent: torch.Tensor) -> torch.Tensor:
    """[1, C, T, H, W] -> [T*(H/2)*(W/2), C*4]: rows (t, h, w), features (c, ph, pw) (layout.py:60-67)."""
    _, c, t, h, w = latent.shape
    return latent.reshape(c, t, h // 2, 2, w // 2, 2).permute(1, 2, 4, 0, 3, 5).reshape(t * (h // 2) * (w // 2), c * 4)


def unpatchify(rows: torch.Tensor, t: int, h: int, w: int, c: int) -> torch.Tensor:
    """Inverse of patchify; h, w are pixel sizes (layout.py:70-74)."""
    return rows.reshape(t, h // 2, w // 2, c, 2, 2).permute(3, 0, 1, 4, 2, 5).reshape(1, c, t, h, w)


def pack(audio: torch.Tensor) -> torch.Tensor:
    """[1, C, 2, T] -> [2T, C], channel 0's frames first (layout.py:77-82)."""
    return audio[0].permute(1, 2, 0).reshape(-1, audio.shape[1])


def unpack(rows: torch.Tensor) -> torch.Tensor:
    return rows.reshape(2, rows.shape[0] // 2, rows.shape[1]).permute(2, 0, 1).unsqueeze(0)


def lerp_rows(table: torch.Tensor, t_values: Sequence[float]) -> torch.Tensor:
    """fp32 rows of `table` interpolated at t in [0, 1] (layout.py:380-386)."""
    t = torch.tensor(list(t_values), dtype=torch.float32)
    pos = t.clamp(0.0, 1.0) * (table.shape[0] - 1)
    i0 = pos.floor().long().clamp(max=table.shape[0] - 2)
    return torch.lerp(table[i0].float(), table[i0 + 1].float(), (pos - i0).unsqueeze(1))


def token_rows(mod_segments, s: int) -> torch.Tensor:
    rows = torch.zeros(s, dtype=torch.long)
    for a, b, r in mod_segments:
        rows[a:b] = r
    return rows


def _assemble(segments, text_rows, video_rows, audio_rows, cond_v, cond_a):
    """Token rows in layout order: text, conditioning / reference rows from cond_v / cond_a in segment order, the
    target audio and video rows (model.py:310-343)."""
    out, iv, ia = [], 0, 0
    for a, b, kind in segments:
        n = b - a
        if kind == "text":
            out.append(text_rows)
        elif kind == "video":
            out.append(video_rows)
        elif kind == "audio":
            out.append(audio_rows)
        elif kind in ("cond", "ref_img"):
            out.append(cond_v[iv:iv + n])
            iv += n
        else:
            out.append(cond_a[ia:ia + n])
            ia += n
    return out


# --------------------------------------------------------------------------------------------- naive fp64
def model_naive(sd: Mapping[str, torch.Tensor], cfg, video: torch.Tensor, audio: torch.Tensor, text: torch.Tensor,
                plan: Mapping[str, object], cond_video_rows: Optional[torch.Tensor] = None,
                cond_audio_rows: Optional[torch.Tensor] = None):
    """float64 forward from the definition; video [1, C, T, H, W] with even H, W; single output head."""
    d = {k: v.double() for k, v in sd.items() if v.is_floating_point()}
    hid, hd, heads = cfg.hidden, cfg.head_dim, cfg.heads

    def rms(v, w, e):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + e) * w

    def attention(h, p, ang):
        s = h.shape[0]
        q, k, v = (h @ d[p + ".attn.qkv_proj.weight"].T).reshape(s, 3, heads, hd).unbind(1)
        q = rms(q, d[p + ".attn.q_norm.weight"], cfg.qk_norm_eps)
        k = rms(k, d[p + ".attn.k_norm.weight"], cfg.qk_norm_eps)
        if ang is not None:
            half = ang.shape[1]
            c, sn = torch.cos(ang)[:, None], torch.sin(ang)[:, None]

            def rot(t):
                a, b = t[..., :half], t[..., half:2 * half]
                return torch.cat([a * c - b * sn, a * sn + b * c, t[..., 2 * half:]], -1)

            q, k = rot(q), rot(k)
        p_ = torch.softmax(torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(hd), -1)
        return torch.einsum("hqk,khd->qhd", p_, v).reshape(s, -1) @ d[p + ".attn.out_proj.weight"].T

    def mlp(h, p):
        gate, up = (h @ d[p + ".mlp.fc1.weight"].T).chunk(2, -1)
        return (gate * torch.sigmoid(gate) * up) @ d[p + ".mlp.fc2.weight"].T

    ctx = text[0].double() @ d["condition_proj.weight"].T + d["condition_proj.bias"]
    for j in range(cfg.refiner_layers):
        p = f"token_refiner.blocks.{j}"
        ctx = ctx + attention(rms(ctx, d[p + ".norm1.weight"], cfg.norm_eps), p, None)
        ctx = ctx + mlp(rms(ctx, d[p + ".norm2.weight"], cfg.norm_eps), p)
    ctx = rms(ctx, d["token_refiner.final_norm.weight"], cfg.final_norm_eps)

    def vproj(r):
        return r.double() @ d["video_patch_proj.weight"].T + d["video_patch_proj.bias"]

    def aproj(r):
        return r.double() @ d["audio_patch_proj.weight"].T + d["audio_patch_proj.bias"]

    h = torch.cat(_assemble(plan["segments"], ctx, vproj(patchify(video)), aproj(pack(audio)),
                            None if cond_video_rows is None else vproj(cond_video_rows),
                            None if cond_audio_rows is None else aproj(cond_audio_rows)))
    rows = token_rows(plan["mod_segments"], h.shape[0])
    pos = plan["position_ids"].double()
    ang = (pos[:, :, None] * d["rope.inv_freq"][None, None, :]).reshape(pos.shape[0], -1)
    t_emb = lerp_rows(sd["adaln_t_table"], plan["t_values"]).double()
    for i in range(cfg.layers):
        p = f"blocks.{i}"
        m = (t_emb @ d[p + ".adaln_proj.linear.weight"].T + d[p + ".adaln_proj.linear.bias"]).reshape(-1, 6, hid)[rows]
        sh1, sc1, g1, sh2, sc2, g2 = m.unbind(1)
        h = h + g1 * attention(rms(h, d[p + ".norm1.weight"], cfg.norm_eps) * (1 + sc1) + sh1, p, ang)
        h = h + g2 * mlp(rms(h, d[p + ".norm2.weight"], cfg.norm_eps) * (1 + sc2) + sh2, p)
    fsh, fsc = (t_emb @ d["final_layer.adaln_proj.linear.weight"].T + d["final_layer.adaln_proj.linear.bias"]).chunk(2, -1)

    def head(seg, name):
        a, b, r = seg
        y = rms(h[a:b], d["final_layer.norm.weight"], cfg.final_norm_eps) * (1 + fsc[r]) + fsh[r]
        return y @ d[f"final_layer.{name}.weight"].T + d[f"final_layer.{name}.bias"]

    _, c, t, hh, ww = video.shape
    return [-unpatchify(head(plan["video_seg"], "video_out"), t, hh, ww, c), -unpack(head(plan["audio_seg"], "audio_out"))]


# --------------------------------------------------------------------------------------------- reference op order
def model_ref(sd: Mapping[str, torch.Tensor], cfg, video: torch.Tensor, audio: torch.Tensor, text: torch.Tensor,
              plan: Mapping[str, object], *, dtype: torch.dtype = torch.bfloat16,
              linears: Optional[Dict[str, object]] = None, cond_video_rows: Optional[torch.Tensor] = None,
              cond_audio_rows: Optional[torch.Tensor] = None, rope_impl: str = "torch", mode: str = "ck"):
    """The reference forward on the CPU in `dtype` (fp32 islands rounded through it).  Returns [-video_v,
    -audio_v] in the input dtypes."""
    f32 = torch.float32
    linears = linears or {}
    hid, hd, heads = cfg.hidden, cfg.head_dim, cfg.heads

    def isl(t):
        return t.to(dtype).to(f32)

    def weights(p: str) -> Dict[str, object]:
        w = {k: linears.get(f"{p}.{name}", sd.get(f"{p}.{name}.weight")) for k, name in _LIN.items()}
        for k, name in (("norm1", "norm1"), ("norm2", "norm2"), ("q_norm", "attn.q_norm"), ("k_norm", "attn.k_norm")):
            w[k] = sd[f"{p}.{name}.weight"].to(dtype)
        for k in ("qkv", "out", "fc1", "fc2"):
            if isinstance(w[k], torch.Tensor):
                w[k] = w[k].to(dtype)
        return w

    def rms(v, g, e):
        return F.rms_norm(v, (v.shape[-1],), g.to(v.dtype), e)

    def refiner_block(x, w):  # model.py:244-247 with _attention's rope=None branch (:200-203)
        s = x.shape[0]
        h = rms(x, w["norm1"], cfg.norm_eps)
        qkv = br._linear(h, w["qkv"], mode=mode)
        q, k, v = (t.reshape(s, heads, hd) for t in qkv.split(heads * hd, dim=-1))
        q, k = rms(q, w["q_norm"], cfg.qk_norm_eps), rms(k, w["k_norm"], cfg.qk_norm_eps)
        qf, kf, vf = (t.transpose(0, 1).float() for t in (q, k, v))
        att = torch.softmax((qf @ kf.transpose(1, 2)) / math.sqrt(hd), dim=-1)
        o = (att @ vf).transpose(0, 1).reshape(s, heads * hd).to(dtype)
        x = br._linear(o, w["out"], mode=mode).add_(x)
        return br.mlp_ref(rms(x, w["norm2"], cfg.norm_eps), w, "swiglu", mode).add_(x)

    ctx = F.linear(text[0].to(dtype), sd["condition_proj.weight"].to(dtype), sd["condition_proj.bias"].to(dtype))
    for j in range(cfg.refiner_layers):
        ctx = refiner_block(ctx, weights(f"token_refiner.blocks.{j}"))
    ctx = rms(ctx, sd["token_refiner.final_norm.weight"].to(dtype), cfg.final_norm_eps)

    vpw, vpb = isl(sd["video_patch_proj.weight"]), isl(sd["video_patch_proj.bias"])
    apw, apb = isl(sd["audio_patch_proj.weight"]), isl(sd["audio_patch_proj.bias"])
    vrows = F.linear(patchify(video.float()), vpw, vpb).to(dtype)
    arows = F.linear(pack(audio.float()), apw, apb).to(dtype)
    cv = None if cond_video_rows is None else F.linear(cond_video_rows.float(), vpw, vpb).to(dtype)
    ca = None if cond_audio_rows is None else F.linear(cond_audio_rows.float(), apw, apb).to(dtype)
    x = torch.cat(_assemble(plan["segments"], ctx, vrows, arows, cv, ca))

    t_emb = lerp_rows(sd["adaln_t_table"], plan["t_values"])
    pos = plan["position_ids"].to(f32)
    ang = (pos[:, :, None] * sd["rope.inv_freq"].float()[None, None, :]).reshape(pos.shape[0], -1)
    cos, sin = torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)
    segments = list(plan["mod_segments"])
    for i in range(cfg.layers):
        p = f"blocks.{i}"
        z = F.linear(t_emb, isl(sd[p + ".adaln_proj.linear.weight"]), isl(sd[p + ".adaln_proj.linear.bias"]))
        mods = z.view(t_emb.shape[0] * 3, -1).chunk(6, dim=-1)
        x = br.block_ref(x, weights(p), mods, segments, cos, sin, heads, hd, "swiglu", cfg.norm_eps, cfg.qk_norm_eps,
                         rope_impl, mode)

    z = F.linear(t_emb, isl(sd["final_layer.adaln_proj.linear.weight"]), isl(sd["final_layer.adaln_proj.linear.bias"]))
    shift, scale = z.view(t_emb.shape[0], -1).chunk(2, dim=-1)
    fnorm = sd["final_layer.norm.weight"].to(dtype)

    def head(seg, name):
        a, b, r = seg
        y = rms(x[a:b], fnorm, cfg.final_norm_eps) * (1.0 + scale[r]) + shift[r]
        return F.linear(y, isl(sd[f"final_layer.{name}.weight"]), isl(sd[f"final_layer.{name}.bias"]))

    _, c, t, hh, ww = video.shape
    v = unpatchify(head(plan["video_seg"], "video_out"), t, hh, ww, c)
    a = unpack(head(plan["audio_seg"], "audio_out"))
    return [(-v).to(video.dtype), (-a).to(audio.dtype)]
