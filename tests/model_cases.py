"""Seeded tiny H3 networks and inputs for the whole-model tests (CPU tensors; ComfyUI-layout state dicts)."""
from __future__ import annotations

import json
from typing import Dict, Tuple

import numpy as np
import torch

from h3turbo_amd import layout as L
from h3turbo_amd.config import H3Config

# dense tiny network (the reference's test shape) and a W4A8-capable one (every linear's K a multiple of 256)
CFG = H3Config(hidden=64, layers=2, refiner_layers=1, heads=2, head_dim=32, ffn=48, text_dim=40, t_dim=8, curve_grid=17,
               rope_inv_freq_len=4)
W4CFG = H3Config(hidden=256, layers=2, refiner_layers=1, heads=4, head_dim=64, ffn=256, text_dim=40, t_dim=8,
                 curve_grid=17, rope_inv_freq_len=4)
LINEARS = ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")


def make_sd(cfg: H3Config, seed: int = 0, head_bank: int = 1) -> Dict[str, torch.Tensor]:
    """Dense fp32 state dict with weights scaled so activations stay O(1) through the blocks."""
    g = torch.Generator().manual_seed(seed)

    def r(*shape, std):
        return torch.randn(*shape, generator=g) * std

    hid, inner, ffn = cfg.hidden, cfg.inner, cfg.ffn
    sd: Dict[str, torch.Tensor] = {}

    def block(p, adaln):
        sd[p + ".attn.qkv_proj.weight"] = r(3 * inner, hid, std=hid ** -0.5)
        sd[p + ".attn.out_proj.weight"] = r(hid, inner, std=0.7 * inner ** -0.5)
        sd[p + ".mlp.fc1.weight"] = r(2 * ffn, hid, std=hid ** -0.5)
        sd[p + ".mlp.fc2.weight"] = r(hid, ffn, std=0.7 * ffn ** -0.5)
        for n, d in (("norm1", hid), ("norm2", hid), ("attn.q_norm", cfg.head_dim), ("attn.k_norm", cfg.head_dim)):
            sd[f"{p}.{n}.weight"] = 1.0 + r(d, std=0.2)
        if adaln:
            sd[p + ".adaln_proj.linear.weight"] = r(18 * hid, cfg.t_dim, std=0.35)
            sd[p + ".adaln_proj.linear.bias"] = r(18 * hid, std=0.4)

    for i in range(cfg.layers):
        block(f"blocks.{i}", True)
    for j in range(cfg.refiner_layers):
        block(f"token_refiner.blocks.{j}", False)
    sd["token_refiner.final_norm.weight"] = 1.0 + r(hid, std=0.2)
    sd["video_patch_proj.weight"], sd["video_patch_proj.bias"] = r(hid, cfg.video_patch_dim, std=0.15), r(hid, std=0.1)
    sd["audio_patch_proj.weight"], sd["audio_patch_proj.bias"] = r(hid, cfg.audio_channels, std=0.15), r(hid, std=0.1)
    sd["condition_proj.weight"] = r(hid, cfg.text_dim, std=cfg.text_dim ** -0.5)
    sd["condition_proj.bias"] = r(hid, std=0.1)
    grid = torch.linspace(0, 1, cfg.curve_grid)
    sd["adaln_t_table"] = torch.stack([0.5 * 0.4 ** j * torch.sin(6.28 * (1 + j) * grid + j) for j in range(cfg.t_dim)], 1)
    sd["rope.inv_freq"] = 10.0 ** (-torch.arange(cfg.rope_inv_freq_len, dtype=torch.float32) / 4.0)
    sd["final_layer.norm.weight"] = 1.0 + r(hid, std=0.2)
    sd["final_layer.adaln_proj.linear.weight"] = r(2 * hid, cfg.t_dim, std=0.35)
    sd["final_layer.adaln_proj.linear.bias"] = r(2 * hid, std=0.3)
    sd["final_layer.video_out.weight"] = r(head_bank * cfg.video_patch_dim, hid, std=hid ** -0.5)
    sd["final_layer.video_out.bias"] = r(head_bank * cfg.video_patch_dim, std=0.1)
    sd["final_layer.audio_out.weight"] = r(head_bank * cfg.audio_channels, hid, std=hid ** -0.5)
    sd["final_layer.audio_out.bias"] = r(head_bank * cfg.audio_channels, std=0.1)
    return sd


def inputs(cfg: H3Config, seed: int = 1, t: int = 2, h: int = 4, w: int = 6, ta: int = 4, text_len: int = 5):
    """(video [1, C, t, h, w], audio [1, Ca, 2, ta], text states [1, L, text_dim]), fp32."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, cfg.video_channels, t, h, w, generator=g), torch.randn(1, cfg.audio_channels, 2, ta, generator=g),
            torch.randn(1, text_len, cfg.text_dim, generator=g))


def plan_data(cfg: H3Config, text_len: int, video: torch.Tensor, audio: torch.Tensor, sigma: float, **kw) -> Dict:
    """The oracle's plan input for a forward at `sigma`, from the layout module (t2va unless keyframes / refs)."""
    lay = L.PackedLayout.build(text_len, *video.shape[2:], audio.shape[-1], keyframes=kw.pop("keyframes", None),
                               refs=kw.pop("refs", None))
    plan = L.plan_time(lay, torch.tensor(sigma, dtype=torch.float32), (cfg.sigma_shift_video, cfg.sigma_shift_audio), **kw)
    return {"segments": [(s.start, s.stop, s.kind) for s in lay.segments], "position_ids": lay.position_ids,
            "mod_segments": plan.mod_segments, "t_values": plan.t_values, "video_seg": plan.video_seg,
            "audio_seg": plan.audio_seg}


def w4a8_parts(n: int, k: int, seed: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """(q int8 [n, k/2], fp8 e4m3 scale bytes [n, k/16], s_ch f32 [n], codebook f32 [16]): levels up to ~120,
    dense-equivalent weights of std ~ k^-0.5."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int64).to(torch.int8)
    s_rel = (20 + 100 * torch.rand(n, k // 16, generator=g)).to(torch.float8_e4m3fn).view(torch.uint8)
    s_ch = (0.8 + 0.4 * torch.rand(n, generator=g)) * k ** -0.5 / 40.0
    cb = torch.linspace(-1, 1, 16) + 0.02 * torch.randn(16, generator=g)
    return q.numpy(), s_rel.numpy(), s_ch.float().numpy(), cb.float().numpy()


def with_w4a8(cfg: H3Config, sd: Dict[str, torch.Tensor], seed: int, prefixes) -> Tuple[Dict[str, torch.Tensor], Dict]:
    """Replace the four linears of each block prefix by W4A8 entries (group 16, rotation 256, fp8 scales).
    Returns (the state dict with ComfyUI W4A8 entries, {linear prefix: numpy W4A8 weight for the oracle})."""
    sd = dict(sd)
    oracle = {}
    shapes = {"attn.qkv_proj": (3 * cfg.inner, cfg.hidden), "attn.out_proj": (cfg.hidden, cfg.inner),
              "mlp.fc1": (2 * cfg.ffn, cfg.hidden), "mlp.fc2": (cfg.hidden, cfg.ffn)}
    conf = torch.tensor(list(json.dumps({"format": "asym_w4a8_int8", "group_size": 16,
                                         "convrot_groupsize": 256}).encode()), dtype=torch.uint8)
    for bi, p in enumerate(prefixes):
        for li, name in enumerate(LINEARS):
            n, k = shapes[name]
            q, s8, s_ch, cb = w4a8_parts(n, k, seed * 1000 + bi * 10 + li)
            base = f"{p}.{name}"
            sd[base + ".weight"] = torch.from_numpy(q)
            sd[base + ".weight_s_rel"] = torch.from_numpy(s8).view(torch.float8_e4m3fn)
            sd[base + ".weight_s_channel"] = torch.from_numpy(s_ch)
            sd[base + ".weight_codebook"] = torch.from_numpy(cb)
            sd[base + ".comfy_quant"] = conf
            oracle[base] = {"q": q, "s_rel": s8, "s_kind": "fp8", "s_ch": s_ch, "cb": cb, "group": 16, "convrot": 256}
    return sd, oracle


def dense_equivalent(sd: Dict[str, torch.Tensor], oracle: Dict) -> Dict[str, torch.Tensor]:
    """The state dict with every W4A8 linear replaced by its dense fp32 weight in the original basis."""
    from oracle import block_ref as br

    out = {k: v for k, v in sd.items() if not any(k.startswith(p + ".") for p in oracle)}
    for p, w in oracle.items():
        out[p + ".weight"] = br.dense_of(w).float()
    return out


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()
