"""Deterministic tiny H3 checkpoints (ComfyUI tensor layout) for the .h3t container tests.

Every tensor comes from a numpy generator seeded by (seed, CRC-32 of its name), so the same call gives the same
bytes on any machine; make_golden_h3t.py feeds the same tensors to the reference writer.  Names, dtypes and
shapes follow the checkpoint layout the reference converter produces (h3turbo/h3/convert.py:335-379).
"""
from __future__ import annotations

import json
import zlib
from typing import Dict

import numpy as np
import torch

TINY = dict(hidden=64, layers=2, refiner_layers=1, heads=2, head_dim=32, ffn=48, video_channels=4, audio_channels=8,
            text_dim=32, t_dim=8, curve_grid=17, rope_inv_freq_len=16, quant_group=16, quant_convrot=16)


def _rng(name: str, seed: int) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def state_dict(c: Dict[str, int] = TINY, *, quant: bool = True, seed: int = 0, refiner: bool = True) -> Dict[str, torch.Tensor]:
    h, inner, ffn = c["hidden"], c["heads"] * c["head_dim"], c["ffn"]
    qjson = json.dumps({"format": "asym_w4a8_int8", "group_size": c["quant_group"],
                        "convrot_groupsize": c["quant_convrot"]}, separators=(",", ":")).encode()
    sd: Dict[str, torch.Tensor] = {}

    def normal(name, shape, dtype, scale=0.05, off=0.0):
        v = _rng(name, seed).standard_normal(shape).astype(np.float32) * scale + off
        sd[name] = torch.from_numpy(v).to(dtype)

    dims = {"attn.qkv_proj": (3 * inner, h), "attn.out_proj": (h, inner), "mlp.fc1": (2 * ffn, h), "mlp.fc2": (h, ffn)}

    def block(pre: str, quantised: bool, adaln: bool):
        for p, (n, k) in dims.items():
            if quantised:
                g = c["quant_group"]
                sd[f"{pre}{p}.weight"] = torch.from_numpy(_rng(f"{pre}{p}.weight", seed).integers(-128, 128, (n, k // 2), dtype=np.int8))
                s = _rng(f"{pre}{p}.weight_s_rel", seed).random((n, k // g), dtype=np.float32) * 2 + 0.25
                sd[f"{pre}{p}.weight_s_rel"] = torch.from_numpy(s).to(torch.float8_e4m3fn)
                sd[f"{pre}{p}.weight_s_channel"] = torch.from_numpy(_rng(f"{pre}{p}.weight_s_channel", seed).random(n, dtype=np.float32) * 0.01 + 0.001)
                cb = np.linspace(-1.0, 1.0, 16, dtype=np.float32) + _rng(f"{pre}{p}.weight_codebook", seed).random(16, dtype=np.float32) * 0.01
                sd[f"{pre}{p}.weight_codebook"] = torch.from_numpy(cb)
                sd[f"{pre}{p}.comfy_quant"] = torch.tensor(list(qjson), dtype=torch.uint8)
            else:
                normal(f"{pre}{p}.weight", (n, k), torch.bfloat16, 0.02)
        for nm in ("norm1.weight", "norm2.weight"):
            normal(pre + nm, (h,), torch.bfloat16, 0.05, 1.0)
        for nm in ("attn.q_norm.weight", "attn.k_norm.weight"):
            normal(pre + nm, (c["head_dim"],), torch.bfloat16, 0.05, 1.0)
        if adaln:
            normal(pre + "adaln_proj.linear.weight", (18 * h, c["t_dim"]), torch.bfloat16)
            normal(pre + "adaln_proj.linear.bias", (18 * h,), torch.float32)

    for i in range(c["layers"]):
        block(f"blocks.{i}.", quant, True)
    if refiner:
        for j in range(c["refiner_layers"]):
            block(f"token_refiner.blocks.{j}.", False, False)
        normal("token_refiner.final_norm.weight", (h,), torch.bfloat16, 0.05, 1.0)
    vpd = c["video_channels"] * 4
    for nm, dt, shp in (("video_patch_proj.weight", torch.float32, (h, vpd)), ("video_patch_proj.bias", torch.float32, (h,)),
                        ("audio_patch_proj.weight", torch.float32, (h, c["audio_channels"])),
                        ("audio_patch_proj.bias", torch.float32, (h,)), ("condition_proj.weight", torch.bfloat16, (h, c["text_dim"])),
                        ("condition_proj.bias", torch.bfloat16, (h,)),
                        ("final_layer.adaln_proj.linear.weight", torch.bfloat16, (2 * h, c["t_dim"])),
                        ("final_layer.adaln_proj.linear.bias", torch.float32, (2 * h,)),
                        ("final_layer.video_out.weight", torch.float32, (vpd, h)), ("final_layer.video_out.bias", torch.float32, (vpd,)),
                        ("final_layer.audio_out.weight", torch.float32, (c["audio_channels"], h)),
                        ("final_layer.audio_out.bias", torch.float32, (c["audio_channels"],)),
                        ("final_layer.norm.weight", torch.bfloat16, (h,)), ("adaln_t_table", torch.float32, (c["curve_grid"], c["t_dim"])),
                        ("rope.inv_freq", torch.float32, (c["rope_inv_freq_len"],)), ("adaln_basis", torch.float32, (c["t_dim"], h // 2)),
                        ("adaln_mean", torch.float32, (h // 2,))):
        normal(nm, shp, dt)
    return sd
