"""Packed layout, timestep plan and helpers (h3turbo_amd.layout) on the CPU: bit for bit against the reference's own
outputs (tests/golden/vectors/layout.npz, written by tests/golden/make_golden_layout.py) and the reference's
known-answer checks (hand-derived positions, tag runs, mask levels, head-bank ranges; after tests/test_h3_layout.py).
The CPU model oracle's patchify / pack helpers are pinned here too."""
import json
import math
import os

import numpy as np
import pytest
import torch

import layout_inputs as li
from h3turbo_amd import layout as L
from oracle import model_ref as mr

VEC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vectors")
T, H, W, TA, NT = 2, 4, 6, 4, 5


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(VEC, "layout.npz"), allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    with open(os.path.join(VEC, "layout.json")) as f:
        meta = json.load(f)
    return meta, arrays


def per_token(seg_rows):
    out, flags = [], []
    for a, b, r in seg_rows:
        if isinstance(r, torch.Tensor):
            out.append(r.to(torch.int64).numpy())
            flags.append(1)
        else:
            out.append(np.full(b - a, int(r), np.int64))
            flags.append(0)
    return np.concatenate(out), flags


# ------------------------------------------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("scn", li.SCENARIOS, ids=[s["name"] for s in li.SCENARIOS])
def test_layouts_and_plans_match_the_reference_bit_for_bit(golden, scn):
    meta, g = golden
    nm = scn["name"]
    t, h, w = scn["shape"]
    lay = L.PackedLayout.build(scn["text"], t, h, w, scn["audio"], keyframes=li.keyframes(scn["keyframes"]),
                               refs=li.refs(scn["refs"]))
    sm = meta["scenarios"][nm]
    assert [s.kind for s in lay.segments] == sm["kinds"] and lay.seq_len == sm["seq_len"]
    assert list(lay.signature) == sm["signature"]
    assert np.array_equal(np.asarray([[s.start, s.stop] for s in lay.segments]), g[f"{nm}.segs"])
    assert lay.position_ids.dtype == torch.float64
    assert np.array_equal(lay.position_ids.numpy(), g[f"{nm}.pos"])  # float64, exact
    assert np.array_equal(lay.img_pos.numpy(), g[f"{nm}.img_pos"])
    assert np.array_equal(lay.img_update.numpy().astype(np.uint8), g[f"{nm}.img_update"])
    assert np.array_equal(lay.audio_pos.numpy(), g[f"{nm}.audio_pos"])
    assert np.array_equal(lay.audio_update.numpy().astype(np.uint8), g[f"{nm}.audio_update"])
    assert sm["plans"] == len(scn["plans"])
    for i, p in enumerate(scn["plans"]):
        pre = f"{nm}.p{i}"
        plan = L.plan_time(lay, torch.tensor(p["sigma"], dtype=torch.float32), tuple(p.get("shifts", (12.0, 3.0))),
                           **li.plan_kwargs(scn, p))
        assert np.array_equal(np.asarray(plan.t_values, np.float64), g[pre + ".t_values"]), pre
        assert np.array_equal(np.asarray([plan.t_video, plan.t_audio]), g[pre + ".t_va"]), pre
        rows, flags = per_token(plan.mod_segments)
        assert np.array_equal(rows, g[pre + ".rows"]), pre
        assert np.array_equal(np.asarray([[s, e, f] for (s, e, _), f in zip(plan.mod_segments, flags)]), g[pre + ".mod"])
        for which, seg in (("video", plan.video_seg), ("audio", plan.audio_seg)):
            r, f = per_token([seg])
            assert np.array_equal(r, g[f"{pre}.{which}_rows"]), (pre, which)
            assert np.array_equal(np.asarray([seg[0], seg[1], f[0]]), g[f"{pre}.{which}_seg"]), (pre, which)


def test_scalar_and_table_helpers_match_the_reference_bit_for_bit(golden):
    _, g = golden
    m = li.misc_inputs()
    shift = np.stack([L.time_shift_sigma(m["sigmas"], a, b).numpy() for a, b in m["shift_pairs"]])
    assert shift.dtype == np.float32 and np.array_equal(shift, g["misc.shift"])
    assert np.array_equal(L.curve_lerp(m["table"], m["t_list"]).numpy(), g["misc.lerp"])
    bank = np.asarray([L.head_bank_range(s, torch.tensor(sig), sh, n) for s, sig, sh, n in m["bank"]])
    assert np.array_equal(bank, g["misc.bank"])
    assert np.array_equal(L.mask_row_values(m["pixel_mask"], 3, 6, 8).numpy(), g["misc.mask_rows"])
    gv, ga = L.token_grid_masks(m["grid_video"], m["grid_audio"])
    assert np.array_equal(gv.numpy(), g["misc.grid_video"]) and np.array_equal(ga.numpy(), g["misc.grid_audio"])


# ------------------------------------------------------------------------------------------------ known answers
def test_time_shift_inverts_keeps_fp32_and_fixes_one():
    s = torch.tensor([0.05, 0.3, 0.8, 1.0])
    assert torch.allclose(L.time_shift_sigma(L.time_shift_sigma(s, 12.0, 3.0), 3.0, 12.0), s, atol=1e-6)
    assert torch.allclose(L.time_shift_sigma(s, 5.0, 5.0), s, atol=1e-6)
    assert L.time_shift_sigma(s, 12.0, 3.0).dtype == torch.float32
    assert L.time_shift_sigma(1.0, 12.0, 3.0) == pytest.approx(1.0)


@pytest.mark.parametrize("impl", ["layout", "oracle"])
def test_patchify_row_order_and_round_trip(impl):
    x = torch.randn(1, 24, 3, 6, 8)
    if impl == "layout":
        rows = L.patchify_video(x)
        back = L.unpatchify_video(rows, 3, 3, 4, 24)
    else:
        rows = mr.patchify(x)
        back = mr.unpatchify(rows, 3, 6, 8, 24)
    assert rows.shape == (3 * 3 * 4, 96) and torch.equal(back, x)
    # token (t=1, h=2, w=3) is the 2x2 pixel block at h 4..5, w 6..7, features in (c, ph, pw) order
    assert torch.equal(rows[(1 * 3 + 2) * 4 + 3].reshape(24, 1, 2, 2), x[0, :, 1:2, 4:6, 6:8])
    if impl == "layout":
        with pytest.raises(ValueError):
            L.patchify_video(torch.randn(1, 24, 1, 5, 6))


def test_pad_to_patch_is_circular_and_a_no_op_when_aligned():
    x = torch.arange(2 * 3 * 5, dtype=torch.float32).reshape(1, 1, 2, 3, 5)
    y = L.pad_to_patch(x)
    assert y.shape == (1, 1, 2, 4, 6)
    assert torch.equal(y[..., :3, :5], x) and torch.equal(y[..., 3, :5], x[..., 0, :]) and torch.equal(y[..., 5], y[..., 0])
    assert torch.equal(L.pad_to_patch(y), y)


@pytest.mark.parametrize("impl", ["layout", "oracle"])
def test_audio_packing_is_channel_major(impl):
    a = torch.randn(1, 32, 2, 5)
    rows = L.pack_audio(a) if impl == "layout" else mr.pack(a)
    assert rows.shape == (10, 32)
    assert torch.equal(rows[:5], a[0, :, 0].T) and torch.equal(rows[5:], a[0, :, 1].T)
    assert torch.equal(L.unpack_audio(rows) if impl == "layout" else mr.unpack(rows), a)
    if impl == "layout":
        with pytest.raises(ValueError):
            L.pack_audio(torch.randn(2, 32, 2, 5))


def test_t2va_positions_from_first_principles():
    lay = L.PackedLayout.build(NT, 6, 4, 8, 3)
    per_frame = 2 * 4
    assert [tuple(s) for s in lay.segments] == [(0, NT, "text"), (NT, NT + 6, "audio"),
                                                (NT + 6, NT + 6 + 6 * per_frame, "video")]
    pos = lay.position_ids
    assert torch.equal(pos[:NT, 0], torch.arange(NT, dtype=torch.float64)) and not pos[:NT, 1:].any()
    root = math.sqrt(4 * 8)
    w_axis = [(i * (8 / root / 4) + (1 - 8 / root) / 2) * 32 for i in range(4)]
    h_axis = [(i * (4 / root / 2) + (1 - 4 / root) / 2) * 32 for i in range(2)]
    aud = pos[NT:NT + 6]
    assert aud[:, 0].tolist() == [NT + v for v in (0.0, 1.0, 2.0, 0.0, 1.0, 2.0)] and not aud[:, 1].any()
    assert aud[0, 2].item() == pytest.approx(w_axis[0]) and aud[3, 2].item() == pytest.approx(w_axis[-1])
    vid = pos[NT + 6:].reshape(6, per_frame, 3)
    spans = [L.FRAME_RESCALE * k for k in (1, 4, 4, 4, 4, 1)]
    for f in range(6):
        assert vid[f, :, 0].tolist() == pytest.approx([NT + sum(spans[:f])] * per_frame)
    assert vid[0, 0, 1].item() == pytest.approx(h_axis[0]) and vid[0, -1, 1].item() == pytest.approx(h_axis[1])
    assert vid[0, 0, 2].item() == pytest.approx(w_axis[0]) and vid[0, -1, 2].item() == pytest.approx(w_axis[-1])
    assert lay.img_update.all() and lay.audio_update.all()


def _full():
    scn = li.SCENARIOS[1]
    t, h, w = scn["shape"]
    return L.PackedLayout.build(scn["text"], t, h, w, scn["audio"], keyframes=li.keyframes(scn["keyframes"]),
                                refs=li.refs(scn["refs"]))


def test_conditioned_layout_tiles_the_sequence_and_anchors_the_streams():
    lay = _full()
    assert [s.kind for s in lay.segments] == ["text", "cond", "cond_audio", "cond", "ref_img", "ref_audio", "ref_img",
                                              "ref_audio", "ref_img", "audio", "video"]
    assert lay.segments[0].start == 0 and lay.segments[-1].stop == lay.seq_len
    assert all(a.stop == b.start for a, b in zip(lay.segments, lay.segments[1:]))
    every = torch.cat([torch.arange(NT), lay.img_pos, lay.audio_pos]).sort().values
    assert torch.equal(every, torch.arange(lay.seq_len))
    assert lay.img_update.sum() == T * (H // 2) * (W // 2) and lay.audio_update.sum() == 2 * TA
    assert not lay.img_update[:-T * (H // 2) * (W // 2)].any()
    # target origin: text + image 1 + video_audio max(3, 5/3 * (1 + 4)) + audio 4 + video max(0, 5/3)
    origin = NT + 1.0 + max(3.0, L.FRAME_RESCALE * 5) + 4.0 + L.FRAME_RESCALE
    assert lay.position_ids[lay.span("audio").start, 0].item() == pytest.approx(origin)
    assert lay.position_ids[lay.segments[1].start, 0].item() == pytest.approx(origin)
    assert lay.position_ids[lay.segments[3].start, 0].item() == pytest.approx(origin + L.FRAME_RESCALE * 9)
    assert lay.position_ids[lay.segments[4].start:lay.segments[4].stop, 0].eq(NT).all()


def test_layout_rejects_bad_input():
    for args, kw in (((NT, 2, 5, 6, 3), {}), ((NT, 0, 4, 6, 3), {}), ((NT, 2, 4, 6, 3), {"refs": [{"kind": "hologram"}]})):
        with pytest.raises(ValueError):
            L.PackedLayout.build(*args, **kw)
    with pytest.raises(KeyError):
        L.find_segment(L.PackedLayout.build(NT, 1, 2, 2, 1), "cond")


def test_plan_rows_tags_and_conditioning_pins():
    lay = _full()
    sig = torch.tensor(0.6, dtype=torch.float32)
    plan = L.plan_time(lay, sig, (12.0, 3.0))
    tv, ta = float(1 - sig), float(1 - L.time_shift_sigma(sig, 12.0, 3.0))
    assert plan.t_values == sorted(plan.t_values) and {tv, ta, 0.999, 1.0} <= set(plan.t_values)
    rows = {s.kind: r for s, (_, _, r) in zip(lay.segments, plan.mod_segments)}
    idx = {t: i for i, t in enumerate(plan.t_values)}
    assert rows["text"] == idx[tv] * 3 + 1 and rows["video"] == idx[tv] * 3 and rows["audio"] == idx[ta] * 3 + 2
    assert rows["cond"] == idx[0.999] * 3 and rows["ref_img"] == idx[0.999] * 3 and rows["cond_audio"] == idx[1.0] * 3 + 2
    assert plan.video_seg[2] == idx[tv] and plan.audio_seg[2] == idx[ta]
    assert [(a, b) for a, b, _ in plan.mod_segments] == [(s.start, s.stop) for s in lay.segments]
    late = L.plan_time(lay, torch.tensor(0.0005, dtype=torch.float32), (12.0, 3.0), visual_aug=0.5)
    assert late.t_video == pytest.approx(0.9995, abs=1e-6) and late.t_audio < 1.0
    assert 0.5 not in late.t_values and max(late.t_values) == 1.0


def test_plan_text_tag_runs_and_validation():
    lay = L.PackedLayout.build(7, T, H, W, TA)
    plan = L.plan_time(lay, torch.tensor(0.5), (12.0, 3.0), text_tags=torch.tensor([[1, 1, 0, 0, 0, 2, 1]]))
    text = [seg for seg in plan.mod_segments if seg[1] <= 7]
    assert [(a, b) for a, b, _ in text] == [(0, 2), (2, 5), (5, 6), (6, 7)]
    base = text[0][2] - 1
    assert [r - base for _, _, r in text] == [1, 0, 2, 1]
    for bad in (torch.tensor([[1, 1, 0]]), torch.tensor([[1, 1, 0, 0, 0, 2, 3]])):
        with pytest.raises(ValueError):
            L.plan_time(lay, torch.tensor(0.5), (12.0, 3.0), text_tags=bad)


def test_plan_denoise_mask_levels():
    lay = L.PackedLayout.build(NT, T, H, W, TA)
    sig = torch.tensor(0.8, dtype=torch.float32)
    m = torch.ones(1, 1, T, H, W)
    m[:, :, 0] = 0.0
    m[:, :, 1, :2, :2] = 0.5
    plan = L.plan_time(lay, sig, (12.0, 3.0), denoise_mask=m)
    va, vb, rows = plan.video_seg
    assert isinstance(rows, torch.Tensor) and rows.shape == (vb - va,)
    levels = sorted(plan.t_values[i] for i in rows.unique().tolist())
    assert levels[0] == pytest.approx(0.2, abs=1e-6) and levels[1] == pytest.approx(0.6, abs=1e-6)
    assert levels[-1] == pytest.approx(0.999, abs=1e-6)
    per = (H // 2) * (W // 2)
    assert plan.t_values[rows[0].item()] == pytest.approx(0.999, abs=1e-6)
    assert plan.t_values[rows[per].item()] == pytest.approx(0.6, abs=1e-6)
    assert plan.t_values[rows[per + 5].item()] == pytest.approx(0.2, abs=1e-6)
    mod_video = [r for a, b, r in plan.mod_segments if a == va][0]
    assert isinstance(mod_video, torch.Tensor) and (mod_video % 3 == 0).all()
    uni = L.plan_time(lay, sig, (12.0, 3.0), denoise_mask=torch.full((1, 1, T, H, W), 0.4))
    assert isinstance(uni.video_seg[2], int) and uni.t_values[uni.video_seg[2]] == pytest.approx(1 - 0.4 * 0.8, abs=1e-6)
    am = torch.ones(1, 1, 2, TA)
    am[..., :2] = 0.0
    pa = L.plan_time(lay, sig, (12.0, 3.0), audio_denoise_mask=am)
    assert pa.audio_seg[2].shape == (2 * TA,) and (pa.audio_seg[2][:2] != pa.audio_seg[2][2]).all()


def test_mask_pooling_helpers():
    m = torch.ones(3, 5, 7)
    assert L.mask_row_values(m, 3, 6, 8) is None
    m[1, 3, 2] = 0.25  # one preserved pixel beside generating ones: the patch max keeps it generating
    assert L.mask_row_values(m, 3, 6, 8) is None
    m[1, 2:4, 2:4] = 0.0
    v = L.mask_row_values(m, 3, 6, 8)
    assert v.shape == (36,) and v[(1 * 3 + 1) * 4 + 1] == 0 and v.sum() == v.numel() - 1
    assert L.mask_row_values(torch.zeros(3, 5, 7), 3, 6, 8).eq(0).all()
    assert L.mask_row_values(torch.full((3, 5, 7), 0.7), 3, 6, 8) is not None
    assert L.mask_row_values(torch.full((3, 5, 7), 0.9995), 3, 6, 8) is None
    vm, am = torch.rand(1, 1, 2, 5, 7), torch.rand(1, 32, 2, 3)
    gv, ga = L.token_grid_masks(vm, am)
    assert gv.shape == vm.shape and ga.shape == am.shape
    assert torch.equal(gv, torch.ceil(gv * 256) / 256) and (gv >= vm).all()
    assert torch.equal(ga[:, 0], ga[:, 5]) and (ga >= am).all()


def test_curve_lerp_endpoints_midpoints_and_clamp():
    table = torch.arange(15, dtype=torch.float32).reshape(5, 3)
    out = L.curve_lerp(table, [0.0, 1.0, 0.5, 0.125, 2.0, -1.0])
    assert torch.equal(out[0], table[0]) and torch.equal(out[1], table[4]) and torch.equal(out[2], table[2])
    assert torch.allclose(out[3], 0.5 * (table[0] + table[1])) and torch.equal(out[4], table[4])
    assert torch.equal(out[5], table[0])
    assert torch.equal(mr.lerp_rows(table, [0.0, 1.0, 0.5, 0.125, 2.0, -1.0]), out)


def test_head_bank_ranges_and_mixed_weights():
    sched = torch.tensor([1.0, 0.8, 0.6, 0.3, 0.0])
    for sigma, want in ((1.0, (0, 2)), (0.8, (2, 3)), (0.3, (2, 3)), (0.0, (2, 3))):
        assert L.head_bank_range(sched, torch.tensor(sigma), 12.0, 3) == want
    w, b = torch.randn(6, 5, dtype=torch.float64), torch.randn(6, dtype=torch.float64)
    we, be = L.bank_head_weights(w, b, 3, 0, 1, 12.0)
    assert torch.equal(we, w[:2]) and torch.equal(be, b[:2])
    we, be = L.bank_head_weights(w, b, 3, 1, 3, 12.0)
    grid = torch.linspace(1.0, 0.0, 4, dtype=torch.float64)
    dt = (1.0 - 12.0 * grid / (1.0 + 11.0 * grid)).diff()[1:3]
    wt = dt / dt.sum()
    assert torch.allclose(we, w[:2] + wt[0] * w[2:4] + wt[1] * w[4:6])
    assert torch.allclose(be, b[:2] + wt[0] * b[2:4] + wt[1] * b[4:6])


def test_rope_impl_resolution():
    assert L.resolve_rope_impl("auto") == "torch" and L.resolve_rope_impl("eager") == "eager"
    with pytest.raises(ValueError):
        L.resolve_rope_impl("magic")
    with pytest.raises(RuntimeError):
        L.resolve_rope_impl("ck")
