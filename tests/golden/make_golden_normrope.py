"""Write golden vectors of the reference's q/k norm + rope (h3turbo/h3/layout.py:309-355) by running the REFERENCE's
own `rms_norm_fused_order` and `norm_rope_` (torch CPU) on seeded inputs.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden_normrope.py [--reference /root/reference]

What it pins: the summation order of the fused q/k RMSNorm (32 strided partial sums, halving tree) and the
rotation's rounding, which no closed form fixes.  Cases: bf16 "torch" impl (the fused kernel's numerics) and
"eager" impl, head_dim 128 with a rotary half of 48 (3 axes x 16 frequencies) and head_dim 64 with half 12.
Outputs are added to vectors/index.json next to the qlinear cases.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "vectors")


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    from h3turbo.h3.layout import norm_rope_, rms_norm_fused_order  # the reference, in this container only

    with open(os.path.join(OUT, "index.json")) as f:
        meta = json.load(f)
    for (s, heads, hd, half, impl, seed) in [(37, 3, 128, 48, "torch", 1), (37, 3, 128, 48, "eager", 2),
                                             (29, 2, 64, 12, "torch", 3), (96, 4, 128, 48, "torch", 4)]:
        g = torch.Generator().manual_seed(seed)
        q = (3 * torch.randn(s, heads, hd, generator=g)).bfloat16()
        k = (torch.randn(s, heads, hd, generator=g) * torch.exp(torch.randn(s, heads, 1, generator=g))).bfloat16()
        wq = (1 + 0.3 * torch.randn(hd, generator=g)).bfloat16()
        wk = (1 + 0.3 * torch.randn(hd, generator=g)).bfloat16()
        ang = torch.rand(s, half, generator=g, dtype=torch.float64) * 40
        cos, sin = torch.cos(ang).bfloat16(), torch.sin(ang).bfloat16()
        qn = rms_norm_fused_order(q, wq, 1e-5) if impl == "torch" else None
        q_out, k_out = q.clone(), k.clone()
        norm_rope_(q_out, k_out, wq, wk, 1e-5, cos, sin, impl=impl, chunk=16)
        name = f"normrope_s{s}_h{heads}_d{hd}_half{half}_{impl}"
        arrays = dict(q=bits(q), k=bits(k), wq=bits(wq), wk=bits(wk), cos=bits(cos), sin=bits(sin), q_out=bits(q_out),
                      k_out=bits(k_out))
        if qn is not None:
            arrays["q_norm_only"] = bits(qn)
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **arrays)
        meta["cases"][name] = dict(kind="normrope", s=s, heads=heads, head_dim=hd, half=half, impl=impl, eps=1e-5, seed=seed)
        print(f"  wrote {name}", flush=True)
    meta["normrope_generator"] = "tests/golden/make_golden_normrope.py (h3turbo.h3.layout, torch CPU)"
    with open(os.path.join(OUT, "index.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
