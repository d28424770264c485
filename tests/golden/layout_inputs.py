"""Seeded inputs of the packed-layout / timestep-plan golden vectors (make_golden_layout.py writes the vectors
with the reference's layout module; tests/test_layout.py rebuilds these inputs and compares this build's layout
module with them).  Pure data recipes: shapes, seeds and scalar options."""
from __future__ import annotations

from typing import Any, Dict, List

import torch


def _z(*shape):
    return torch.zeros(*shape)


def keyframes(spec):
    """[(frame index, video latent frames or None, audio latent frames or None), ...] -> keyframe dicts."""
    out = []
    for idx, vt, at in spec:
        kf: Dict[str, Any] = {"resolved_frame_index": idx}
        if vt is not None:
            kf["latent"] = _z(1, 24, vt[0], vt[1], vt[2])
        if at is not None:
            kf["audio_latent"] = _z(1, 32, 2, at)
        out.append(kf)
    return out


def refs(spec):
    return [dict(r) for r in spec]


def video_mask(seed: int, t: int, h: int, w: int) -> torch.Tensor:
    """[1, 1, t, h, w]: frame 0 preserved, a few patches at partial values, the rest generating."""
    g = torch.Generator().manual_seed(seed)
    m = torch.ones(1, 1, t, h, w)
    m[:, :, 0] = 0.0
    if t > 1:
        vals = torch.tensor([0.25, 0.5, 0.75])
        for _ in range(3):
            y = int(torch.randint(0, h, (1,), generator=g))
            x = int(torch.randint(0, w, (1,), generator=g))
            m[:, :, t - 1, y, x] = vals[int(torch.randint(0, 3, (1,), generator=g))]
    return m


def audio_mask(seed: int, ta: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    m = torch.ones(1, 1, 2, ta)
    m[..., :max(1, ta // 3)] = 0.0
    m[..., ta - 1] = float(torch.rand(1, generator=g)) * 0.8 + 0.1
    return m


# name -> build arguments and the plans evaluated on the layout
SCENARIOS: List[Dict[str, Any]] = [
    {"name": "t2va", "text": 5, "shape": (6, 4, 8), "audio": 3, "keyframes": [], "refs": [],
     "plans": [{"sigma": 0.6}, {"sigma": 1.0}, {"sigma": 0.0005}, {"sigma": 0.37, "shifts": (5.0, 2.0)}]},
    {"name": "full", "text": 5, "shape": (2, 4, 6), "audio": 4,
     "keyframes": [(0, (1, 4, 6), 3), (9, (2, 4, 6), None)],
     "refs": [{"kind": "image", "latent_h": 4, "latent_w": 2},
              {"kind": "video_audio", "latent_t": 2, "latent_h": 2, "latent_w": 4, "ref_audio_t": 3},
              {"kind": "audio", "ref_audio_t": 4},
              {"kind": "video", "latent_t": 1, "latent_h": 2, "latent_w": 2, "ref_audio_t": 0}],
     "plans": [{"sigma": 0.6}, {"sigma": 0.0005, "visual_aug": 0.5}, {"sigma": 0.9, "audio_aug": 0.97},
               {"sigma": 0.8, "video_mask": 11, "audio_mask": 12}]},
    {"name": "tags", "text": 7, "shape": (2, 4, 6), "audio": 4, "keyframes": [], "refs": [],
     "plans": [{"sigma": 0.5, "tags": [1, 1, 0, 0, 0, 2, 1]}, {"sigma": 0.5, "tags": [0, 0, 0, 0, 0, 0, 0]}]},
    {"name": "masks", "text": 5, "shape": (3, 6, 8), "audio": 6, "keyframes": [], "refs": [],
     "plans": [{"sigma": 0.8, "video_mask": 3, "audio_mask": 4}, {"sigma": 0.8, "video_uniform": 0.4},
               {"sigma": 0.3, "video_mask": 5}, {"sigma": 0.55, "audio_mask": 6}]},
    {"name": "odd", "text": 0, "shape": (5, 6, 10), "audio": 7,
     "keyframes": [(4, None, 5), (2, (1, 6, 10), None)],
     "refs": [{"kind": "video", "latent_t": 3, "latent_h": 4, "latent_w": 4, "ref_audio_t": 0},
              {"kind": "image", "latent_h": 6, "latent_w": 4}],
     "plans": [{"sigma": 0.72}, {"sigma": 0.2, "video_mask": 8}]},
]


def plan_kwargs(scn: Dict[str, Any], p: Dict[str, Any]) -> Dict[str, Any]:
    """plan_time keyword arguments of plan p of scenario scn (the same for both implementations)."""
    t, h, w = scn["shape"]
    kw: Dict[str, Any] = {}
    if "visual_aug" in p:
        kw["visual_aug"] = p["visual_aug"]
    if "audio_aug" in p:
        kw["audio_aug"] = p["audio_aug"]
    if "tags" in p:
        kw["text_tags"] = torch.tensor([p["tags"]])
    if "video_mask" in p:
        kw["denoise_mask"] = video_mask(p["video_mask"], t, h, w)
    if "video_uniform" in p:
        kw["denoise_mask"] = torch.full((1, 1, t, h, w), p["video_uniform"])
    if "audio_mask" in p:
        kw["audio_denoise_mask"] = audio_mask(p["audio_mask"], scn["audio"])
    return kw


def misc_inputs() -> Dict[str, Any]:
    """Inputs of the scalar / table helpers."""
    g = torch.Generator().manual_seed(21)
    return {
        "sigmas": torch.tensor([0.0005, 0.05, 0.3, 0.5, 0.6, 0.8, 0.999, 1.0], dtype=torch.float32),
        "shift_pairs": [(12.0, 3.0), (3.0, 12.0), (5.0, 5.0), (12.0, 1.0)],
        "table": torch.randn(17, 8, generator=g),
        "t_list": [0.0, 1.0, 0.5, 0.125, 0.3337, 0.9995, 2.0, -1.0],
        "bank": [([1.0, 0.8, 0.6, 0.3, 0.0], s, 12.0, 3) for s in (1.0, 0.8, 0.6, 0.3, 0.0)]
                + [([1.0, 0.95, 0.7, 0.2, 0.05, 0.0], s, 5.0, 4) for s in (0.95, 0.7, 0.2, 0.05)],
        "pixel_mask": torch.rand(3, 5, 7, generator=g),
        "grid_video": torch.rand(1, 1, 2, 5, 7, generator=g),
        "grid_audio": torch.rand(1, 32, 2, 3, generator=g),
    }
