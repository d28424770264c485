"""Write tests/golden/vectors/layout.npz (+ layout.json) with the REFERENCE's own layout module.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden_layout.py [--reference /root/reference]

What it pins: the packed layouts (float64 position ids, segment tiling, image / audio row sets) and the timestep
plans (the fp32-derived t values, every token's AdaLN row, the final layer's rows) of the scenarios in
layout_inputs.py, bit for bit, plus the scalar / table helpers (time_shift_sigma, curve_lerp, head_bank_range,
mask pooling).  The reference's own tests check these with tolerances and hand-derived values; the bit-level
results that decide which AdaLN row and interpolation weight a token gets are pinned only by running its code.
The files are data: inputs are rebuilt from layout_inputs.py.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import layout_inputs as li  # noqa: E402

OUT = os.path.join(HERE, "vectors", "layout.npz")


def expand(seg_rows, n_tokens_of):
    """(start, stop, row int | LongTensor) segments -> per-token int64 rows and a tensor-or-int flag per segment."""
    rows, flags = [], []
    for a, b, r in seg_rows:
        if isinstance(r, torch.Tensor):
            rows.append(r.to(torch.int64).numpy())
            flags.append(1)
        else:
            rows.append(np.full(b - a, int(r), np.int64))
            flags.append(0)
    return np.concatenate(rows) if rows else np.zeros(0, np.int64), np.asarray(flags, np.int64)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    a = ap.parse_args()
    sys.path.insert(0, a.reference)
    from h3turbo.h3 import layout as L

    arrays, meta = {}, {"generator": "tests/golden/make_golden_layout.py", "scenarios": {}}
    for scn in li.SCENARIOS:
        nm = scn["name"]
        t, h, w = scn["shape"]
        kfs, rfs = li.keyframes(scn["keyframes"]), li.refs(scn["refs"])
        lay = L.PackedLayout.build(scn["text"], t, h, w, scn["audio"], keyframes=kfs, refs=rfs)
        arrays[f"{nm}.pos"] = lay.position_ids.numpy()
        arrays[f"{nm}.segs"] = np.asarray([[s.start, s.stop] for s in lay.segments], np.int64)
        arrays[f"{nm}.img_pos"] = lay.img_pos.numpy()
        arrays[f"{nm}.img_update"] = lay.img_update.numpy().astype(np.uint8)
        arrays[f"{nm}.audio_pos"] = lay.audio_pos.numpy()
        arrays[f"{nm}.audio_update"] = lay.audio_update.numpy().astype(np.uint8)
        meta["scenarios"][nm] = {"kinds": [s.kind for s in lay.segments], "seq_len": lay.seq_len,
                                 "signature": list(lay.signature), "plans": len(scn["plans"])}
        for i, p in enumerate(scn["plans"]):
            sigma = torch.tensor(p["sigma"], dtype=torch.float32)
            plan = L.plan_time(lay, sigma, tuple(p.get("shifts", (12.0, 3.0))), **li.plan_kwargs(scn, p))
            pre = f"{nm}.p{i}"
            arrays[pre + ".t_values"] = np.asarray(plan.t_values, np.float64)
            rows, flags = expand(plan.mod_segments, None)
            arrays[pre + ".rows"] = rows
            arrays[pre + ".mod"] = np.asarray([[s, e, f] for (s, e, _), f in zip(plan.mod_segments, flags)], np.int64)
            for which, seg in (("video", plan.video_seg), ("audio", plan.audio_seg)):
                r, f = expand([seg], None)
                arrays[f"{pre}.{which}_rows"] = r
                arrays[f"{pre}.{which}_seg"] = np.asarray([seg[0], seg[1], int(f[0])], np.int64)
            arrays[pre + ".t_va"] = np.asarray([plan.t_video, plan.t_audio], np.float64)

    m = li.misc_inputs()
    arrays["misc.shift"] = np.stack([L.time_shift_sigma(m["sigmas"], a_, b_).numpy() for a_, b_ in m["shift_pairs"]])
    arrays["misc.lerp"] = L.curve_lerp(m["table"], m["t_list"]).numpy()
    arrays["misc.bank"] = np.asarray([L.head_bank_range(s, torch.tensor(sig), sh, n) for s, sig, sh, n in m["bank"]],
                                     np.int64)
    arrays["misc.mask_rows"] = L.mask_row_values(m["pixel_mask"], 3, 6, 8).numpy()
    gv, ga = L.token_grid_masks(m["grid_video"], m["grid_audio"])
    arrays["misc.grid_video"], arrays["misc.grid_audio"] = gv.numpy(), ga.numpy()

    np.savez(OUT, **arrays)
    meta["sha256"] = hashlib.sha256(open(OUT, "rb").read()).hexdigest()
    with open(os.path.join(HERE, "vectors", "layout.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print(json.dumps({"file": os.path.relpath(OUT, HERE), "arrays": len(arrays), "sha256": meta["sha256"]}))


if __name__ == "__main__":
    main()
