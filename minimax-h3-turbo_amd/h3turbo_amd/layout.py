"""Packed-sequence bookkeeping of the H3 DiT: which token sits where, at which 3-axis position, with which
timestep and AdaLN modulation row (reference h3turbo/h3/layout.py:1-502).

The network sees one token sequence per forward:

    [text | keyframe conditions | reference blocks | target audio | target video]

Everything here is host-side integer / position / scalar bookkeeping (no weights, no kernels): the layout and its
float64 position ids, video patchify / audio packing, the per-token timestep and modulation-row plan, the output
head bank of the final layer and the denoise-mask helpers.  Scalar timestep arithmetic is done on fp32 0-d
tensors in a fixed operation order, because the AdaLN table coordinates derive from it and a float64 shortcut
moves them by ~1e-8 (h3turbo/h3/layout.py:8-11).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Mapping, NamedTuple, Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F

from .block import rms_lanewise, rope_angles  # noqa: F401  (re-exported: the reference keeps them in layout)

# pixel frames covered by latent frame k (the causal video VAE: the first frame alone, then 4 per latent frame)
FRAME_PER_TOKEN = (1, 4, 4, 4, 4)
FRAME_RESCALE = 5.0 / 3.0  # position units per pixel frame
VISUAL_COND_TIMESTEP = 0.999  # timestep label of conditioning image rows
AUDIO_COND_TIMESTEP = 1.0
GRID_EXTENT = 32.0  # spatial position range of one frame, centred on 0
SPATIAL_PATCH = 2  # a token is a 2x2 patch of latent pixels

# the AdaLN input holds three modulation sets per timestep row: row index = t_row * 3 + tag
TAG_VIDEO, TAG_TEXT, TAG_AUDIO = 0, 1, 2
KIND_TAG = {"text": TAG_TEXT, "video": TAG_VIDEO, "cond": TAG_VIDEO, "ref_img": TAG_VIDEO,
            "audio": TAG_AUDIO, "cond_audio": TAG_AUDIO, "ref_audio": TAG_AUDIO}
VIDEO_KINDS = ("cond", "ref_img", "video")
AUDIO_KINDS = ("cond_audio", "ref_audio", "audio")

ModRow = Union[int, torch.Tensor]  # one modulation row, or a LongTensor with one row per token

rms_norm_fused_order = rms_lanewise  # h3turbo/h3/layout.py:309-326


def time_shift_sigma(sigma, from_shift: float, to_shift: float):
    """A flow-matching sigma of a `from_shift` schedule re-expressed on a `to_shift` schedule
    (h3turbo/h3/layout.py:39-45).  Floats or tensors; the operation order is part of the fp32 result."""
    base = sigma / (from_shift + sigma * (1.0 - from_shift))
    return to_shift * base / (1.0 + (to_shift - 1.0) * base)


# ------------------------------------------------------------------------------------------------ patchify / audio
def pad_to_patch(x: torch.Tensor, patch: Sequence[int] = (1, 2, 2)) -> torch.Tensor:
    """[B, C, T, H, W]: each of T, H, W right-padded to a multiple of its patch size with its own leading
    entries (circular), h3turbo/h3/layout.py:51-57."""
    for axis, p in zip((2, 3, 4), patch):
        short = -x.shape[axis] % p
        if short:
            x = torch.cat([x, x.narrow(axis, 0, short)], dim=axis)
    return x


def patchify_video(latent: torch.Tensor, patch: Sequence[int] = (1, 2, 2)) -> torch.Tensor:
    """[B, C, T, H, W] -> [B*t*h*w, C*pt*ph*pw]: token rows in (b, t, h, w) order, features in (c, pt, ph, pw)
    order (h3turbo/h3/layout.py:60-67)."""
    b, c, tt, hh, ww = latent.shape
    pt, ph, pw = patch
    if tt % pt or hh % ph or ww % pw:
        raise ValueError(f"latent {tuple(latent.shape)} is not a multiple of patch {tuple(patch)}; pad_to_patch first")
    g = latent.reshape(b, c, tt // pt, pt, hh // ph, ph, ww // pw, pw)
    return g.permute(0, 2, 4, 6, 1, 3, 5, 7).reshape(-1, c * pt * ph * pw)


def unpatchify_video(rows: torch.Tensor, t: int, h: int, w: int, c: int, patch: Sequence[int] = (1, 2, 2)) -> torch.Tensor:
    """Inverse of patchify_video; (t, h, w) are patch-grid sizes -> [B, C, t*pt, h*ph, w*pw]
    (h3turbo/h3/layout.py:70-74)."""
    pt, ph, pw = patch
    g = rows.reshape(-1, t, h, w, c, pt, ph, pw).permute(0, 4, 1, 5, 2, 6, 3, 7)
    return g.reshape(-1, c, t * pt, h * ph, w * pw)


def pack_audio(latent: torch.Tensor) -> torch.Tensor:
    """[1, C, ch, T] -> [ch*T, C], channel-major: every frame of channel 0, then channel 1
    (h3turbo/h3/layout.py:77-82)."""
    if latent.shape[0] != 1:
        raise ValueError("audio latent must have batch size 1")
    c, ch, t = latent.shape[1:]
    return latent[0].permute(1, 2, 0).reshape(ch * t, c)


def unpack_audio(rows: torch.Tensor, ch: int = 2) -> torch.Tensor:
    """[ch*T, C] -> [1, C, ch, T] (h3turbo/h3/layout.py:85-87)."""
    t = rows.shape[0] // ch
    return rows.reshape(ch, t, rows.shape[-1]).permute(2, 0, 1).unsqueeze(0)


# ------------------------------------------------------------------------------------------------ positions
def _patch_axis(pixels: int, sqrt_area: float) -> torch.Tensor:
    """Patch-centre coordinates along one spatial axis, area-normalised so that every resolution spans about
    [-16, 16] (h3turbo/h3/layout.py:93-97), float64."""
    ratio = pixels / sqrt_area
    n = pixels // SPATIAL_PATCH
    return (torch.arange(n, dtype=torch.float64) * (ratio / n) + (1.0 - ratio) / 2.0) * GRID_EXTENT


def frame_coords(h: int, w: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(h, w) coordinates [(h/2)*(w/2), 2] of one latent frame's patch rows (row-major), and its w axis
    (h3turbo/h3/layout.py:100-108)."""
    if h < SPATIAL_PATCH or w < SPATIAL_PATCH or h % SPATIAL_PATCH or w % SPATIAL_PATCH:
        raise ValueError(f"latent h/w must be positive multiples of {SPATIAL_PATCH}, got {h}x{w}")
    root = math.sqrt(h * w)
    ys, xs = _patch_axis(h, root), _patch_axis(w, root)
    grid = torch.stack([ys[:, None].expand(-1, xs.shape[0]), xs[None, :].expand(ys.shape[0], -1)], dim=-1)
    return grid.reshape(-1, 2), xs


def frame_spans(n: int) -> List[float]:
    """Time-axis extent of each of n latent frames (h3turbo/h3/layout.py:111-112)."""
    return [FRAME_RESCALE * FRAME_PER_TOKEN[k % len(FRAME_PER_TOKEN)] for k in range(n)]


def video_positions(frames: int, coords: torch.Tensor, origin: float) -> torch.Tensor:
    """[frames * rows, 3]: frame k's rows at t = origin + the spans of frames 0..k-1 (float64 running sum),
    (h, w) from coords (h3turbo/h3/layout.py:115-123)."""
    spans = torch.tensor(frame_spans(frames), dtype=torch.float64)
    before = torch.zeros(frames, dtype=torch.float64)
    if frames > 1:
        before[1:] = spans[:-1].cumsum(0)
    t = origin + before
    n = coords.shape[0]
    return torch.cat([t[:, None, None].expand(frames, n, 1), coords[None].expand(frames, n, 2)], dim=-1).reshape(-1, 3)


def audio_positions(origin: float, frames: int, w_low: float, w_high: float) -> torch.Tensor:
    """Stereo rows, channel-major: t = origin + frame, h = 0, w pinned to one end of the grid per channel
    (h3turbo/h3/layout.py:126-133)."""
    pos = torch.zeros(2, frames, 3, dtype=torch.float64)
    pos[:, :, 0] = origin + torch.arange(frames, dtype=torch.float64)
    pos[0, :, 2], pos[1, :, 2] = w_low, w_high
    return pos.reshape(-1, 3)


def ref_span(blk: Mapping[str, Any]) -> float:
    """Time-axis extent a reference block occupies ahead of the target streams (h3turbo/h3/layout.py:136-146)."""
    kind = blk["kind"]
    if kind == "image":
        return 1.0
    if kind == "audio":
        return float(blk["ref_audio_t"])
    if kind in ("video", "video_audio"):
        return max(float(blk["ref_audio_t"]), sum(frame_spans(blk["latent_t"])))
    raise ValueError(f"unknown reference kind {kind!r} (expected image/audio/video/video_audio)")


class Segment(NamedTuple):
    """Tokens [start, stop) of one kind: text / cond / cond_audio / ref_img / ref_audio / audio / video."""

    start: int
    stop: int
    kind: str


@dataclass(eq=False)
class PackedLayout:
    """Static structure of one (shapes, conditioning) signature; holds no per-step values
    (h3turbo/h3/layout.py:176-246)."""

    seq_len: int
    position_ids: torch.Tensor  # [S, 3] float64 (t, h, w)
    img_pos: torch.Tensor  # rows of every video-type token (cond, ref image, target video)
    img_update: torch.Tensor  # bool over img_pos: True for the generated (target video) rows
    audio_pos: torch.Tensor
    audio_update: torch.Tensor
    signature: Tuple[int, int, int, int, int]  # (text_len, latent_t, latent_h, latent_w, audio_t)
    segments: List[Segment]

    @classmethod
    def build(cls, text_len: int, latent_t: int, latent_h: int, latent_w: int, audio_t: int,
              keyframes: Optional[Sequence[Mapping[str, Any]]] = None,
              refs: Optional[Sequence[Mapping[str, Any]]] = None) -> "PackedLayout":
        if text_len < 0 or latent_t < 1 or audio_t < 1:
            raise ValueError(f"need text_len>=0, latent_t>=1, audio_t>=1; got {text_len}, {latent_t}, {audio_t}")
        frame, w_axis = frame_coords(latent_h, latent_w)
        w_ends = (float(w_axis[0]), float(w_axis[-1]))
        parts: List[Tuple[str, torch.Tensor, bool]] = []

        text = torch.zeros(text_len, 3, dtype=torch.float64)
        text[:, 0] = torch.arange(text_len, dtype=torch.float64)
        parts.append(("text", text, False))
        origin = float(text_len)  # the target streams start after every reference block
        for blk in refs or ():
            origin += ref_span(blk)
        for kf in keyframes or ():  # keyframes share the target grid, anchored at their pixel frame
            anchor = origin + FRAME_RESCALE * kf["resolved_frame_index"]
            if kf.get("latent") is not None:
                parts.append(("cond", video_positions(kf["latent"].shape[2], frame, anchor), False))
            if kf.get("audio_latent") is not None:
                parts.append(("cond_audio", audio_positions(anchor, kf["audio_latent"].shape[-1], *w_ends), False))
        cursor = float(text_len)
        for blk in refs or ():
            kind, span = blk["kind"], ref_span(blk)
            if kind == "image":
                coords, _ = frame_coords(blk["latent_h"], blk["latent_w"])
                pos = torch.cat([torch.full((coords.shape[0], 1), cursor, dtype=torch.float64), coords], dim=1)
                parts.append(("ref_img", pos, False))
            elif kind == "audio":
                if blk["ref_audio_t"] > 0:
                    parts.append(("ref_audio", audio_positions(cursor, blk["ref_audio_t"], *w_ends), False))
            else:  # video / video_audio: the block's audio rows come right before its video rows, same origin
                coords, r_axis = frame_coords(blk["latent_h"], blk["latent_w"])
                if blk["ref_audio_t"] > 0:
                    parts.append(("ref_audio", audio_positions(cursor, blk["ref_audio_t"], float(r_axis[0]),
                                                               float(r_axis[-1])), False))
                parts.append(("ref_img", video_positions(blk["latent_t"], coords, cursor), False))
            cursor += span
        parts.append(("audio", audio_positions(origin, audio_t, *w_ends), True))
        parts.append(("video", video_positions(latent_t, frame, origin), True))

        segments, row = [], 0
        img, img_upd, aud, aud_upd = [], [], [], []
        for kind, pos, update in parts:
            n = pos.shape[0]
            ids = torch.arange(row, row + n)
            if kind in VIDEO_KINDS:
                img.append(ids)
                img_upd.append(torch.full((n,), update, dtype=torch.bool))
            elif kind in AUDIO_KINDS:
                aud.append(ids)
                aud_upd.append(torch.full((n,), update, dtype=torch.bool))
            segments.append(Segment(row, row + n, kind))
            row += n
        return cls(seq_len=row, position_ids=torch.cat([p for _, p, _ in parts]), img_pos=torch.cat(img),
                   img_update=torch.cat(img_upd), audio_pos=torch.cat(aud), audio_update=torch.cat(aud_upd),
                   signature=(text_len, latent_t, latent_h, latent_w, audio_t), segments=segments)

    def span(self, kind: str) -> Segment:
        return find_segment(self, kind)


def find_segment(layout, kind: str) -> Segment:
    """The first segment of `kind` of any layout whose segments unpack as (start, stop, kind)."""
    for start, stop, k in layout.segments:
        if k == kind:
            return Segment(start, stop, k)
    raise KeyError(kind)


def layout_key(text_len: int, shape: Tuple[int, int, int, int], keyframes, refs) -> tuple:
    """Hashable identity of every input of PackedLayout.build (h3turbo/h3/layout.py:256-261)."""
    kf = tuple((k["resolved_frame_index"],
                None if k.get("latent") is None else int(k["latent"].shape[2]),
                None if k.get("audio_latent") is None else int(k["audio_latent"].shape[-1])) for k in keyframes or ())
    rf = tuple((r["kind"], r.get("latent_t"), r.get("latent_h"), r.get("latent_w"), r.get("ref_audio_t"))
               for r in refs or ())
    return (text_len, tuple(shape), kf, rf)


def resolve_rope_impl(impl: str, device=None, dtype=None, table_dtype=None) -> str:
    """"auto" -> "torch" (h3turbo/h3/layout.py:292-300).  The fused "torch" numerics run as one HIP kernel on the
    GPU; "ck" names comfy_kitchen's CUDA op, which this build does not have."""
    if impl not in ("auto", "ck", "torch", "eager"):
        raise ValueError(f"rope_impl must be auto/ck/torch/eager, got {impl!r}")
    if impl == "ck":
        raise RuntimeError("rope_impl='ck' needs comfy_kitchen (CUDA); use 'torch', which runs the same numerics "
                           "as a HIP kernel")
    return "torch" if impl == "auto" else impl


# ------------------------------------------------------------------------------------------------ output head bank
def head_bank_range(sample_sigmas, sigma: torch.Tensor, shift_video: float, n: int) -> Tuple[int, int]:
    """Heads [start, stop) of an n-head output bank that the step from `sigma` to the next sampler sigma spans
    (h3turbo/h3/layout.py:358-364)."""
    ss = torch.as_tensor(sample_sigmas, dtype=torch.float32).cpu()
    at = int((ss - sigma).abs().argmin())
    nxt = ss[min(at + 1, ss.shape[0] - 1)]
    start = round(float(1.0 - time_shift_sigma(sigma, shift_video, 1.0)) * n)
    stop = round(float(1.0 - time_shift_sigma(nxt, shift_video, 1.0)) * n)
    start = min(start, n - 1)
    return start, max(stop, start + 1)


def bank_head_weights(weight: torch.Tensor, bias: torch.Tensor, n: int, start: int, stop: int, flow_shift: float):
    """(weight, bias) of the heads [start, stop) of an n-head bank: head 0 is a full head and heads 1.. are
    offsets from it, mixed by the step sizes dt of the shifted n-step schedule (h3turbo/h3/layout.py:367-377)."""
    grid = torch.linspace(1.0, 0.0, n + 1, dtype=torch.float64)
    dt = (1.0 - flow_shift * grid / (1.0 + (flow_shift - 1.0) * grid)).diff()[start:stop]
    mix = (dt / dt.sum()).to(weight)
    rows, brows = weight.reshape(n, -1, weight.shape[1]), bias.reshape(n, -1)
    first = max(start, 1)
    m = mix[first - start:]
    o, i = rows.shape[1], rows.shape[2]
    w_off = torch.matmul(m[None], rows[first:stop].reshape(stop - first, o * i)).reshape(o, i)
    b_off = torch.matmul(m[None], brows[first:stop]).reshape(o)
    return rows[0] + w_off, brows[0] + b_off


def curve_lerp(table: torch.Tensor, t_values: Sequence[float]) -> torch.Tensor:
    """AdaLN input rows: `table` [grid, k] linearly interpolated at timesteps t in [0, 1] (clamped), fp32
    (h3turbo/h3/layout.py:380-386)."""
    t = torch.tensor(list(t_values), dtype=torch.float32, device=table.device)
    pos = t.clamp(0.0, 1.0) * (table.shape[0] - 1)
    lo = pos.floor().long().clamp(max=table.shape[0] - 2)
    return torch.lerp(table[lo], table[lo + 1], (pos - lo).unsqueeze(1))


# ------------------------------------------------------------------------------------------------ denoise masks
def mask_row_values(mask: torch.Tensor, latent_t: int, lat_h: int, lat_w: int) -> Optional[torch.Tensor]:
    """[T, H, W] denoise mask (1 = generate) -> one value per 2x2 patch row (max over the patch, edge-replicated
    to the padded latent), or None when every row fully generates (h3turbo/h3/layout.py:392-397)."""
    m = F.pad(mask, (0, lat_w - mask.shape[-1], 0, lat_h - mask.shape[-2]), mode="replicate")
    values = m.reshape(latent_t, lat_h // 2, 2, lat_w // 2, 2).amax(dim=(2, 4)).reshape(-1)
    return None if bool((values >= 1.0 - 1e-3).all()) else values


def token_grid_masks(video_mask: torch.Tensor, audio_mask: Optional[torch.Tensor] = None,
                     patch: Sequence[int] = (1, 2, 2)) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Per-pixel denoise masks pooled to the token grid: video max over each 2x2 patch, audio max over channels,
    both broadcast back and rounded up to a multiple of 1/256 (h3turbo/h3/layout.py:400-418)."""
    ph, pw = patch[1:]
    h, w = video_mask.shape[-2:]
    lead = video_mask.shape[:-2]
    v = F.pad(video_mask.reshape((-1,) + video_mask.shape[-3:]), (0, -w % pw, 0, -h % ph), mode="replicate")
    v = v.reshape(lead + v.shape[-2:])
    v = v.reshape(v.shape[:-2] + (v.shape[-2] // ph, ph, v.shape[-1] // pw, pw)).amax(dim=(-3, -1))
    v = v.repeat_interleave(ph, dim=-2).repeat_interleave(pw, dim=-1)[..., :h, :w]
    a = None if audio_mask is None else audio_mask.amax(dim=1, keepdim=True).expand_as(audio_mask).contiguous()

    def up(m):
        return torch.ceil(m * 256.0) / 256.0

    return up(v), (None if a is None else up(a))


# ------------------------------------------------------------------------------------------------ timestep plan
@dataclass
class TimePlan:
    """Per-step timestep labels and modulation rows (h3turbo/h3/layout.py:424-432)."""

    t_values: List[float]  # ascending distinct timesteps: the rows of the AdaLN input
    mod_segments: List[Tuple[int, int, ModRow]]  # (start, stop, modulation row), tiling the sequence
    video_seg: Tuple[int, int, ModRow]  # target video rows; the row indexes t_values (the final layer has no tags)
    audio_seg: Tuple[int, int, ModRow]
    t_video: float
    t_audio: float


def plan_time(layout: PackedLayout, sigma: torch.Tensor, shifts: Tuple[float, float], *,
              visual_aug: float = VISUAL_COND_TIMESTEP, audio_aug: float = AUDIO_COND_TIMESTEP,
              text_tags: Optional[torch.Tensor] = None, denoise_mask: Optional[torch.Tensor] = None,
              audio_denoise_mask: Optional[torch.Tensor] = None) -> TimePlan:
    """Every token's timestep label and AdaLN row (h3turbo/h3/layout.py:435-502).

    sigma: the video sigma as an fp32 0-d CPU tensor.  Text and video share the clock t = 1 - sigma; audio runs
    on its own shifted schedule; conditioning rows sit at max(clock, aug).  A denoise mask value m labels its
    row 1 - m * sigma, capped at the conditioning label.
    """
    text_len, lat_t, lat_h, lat_w, _ = layout.signature
    t_v = float(1.0 - sigma)
    t_a = float(1.0 - time_shift_sigma(sigma, shifts[0], shifts[1]))
    label: Dict[str, float] = {"text": t_v, "video": t_v, "audio": t_a,
                               "cond": max(t_v, visual_aug), "ref_img": max(t_v, visual_aug),
                               "cond_audio": max(t_a, audio_aug), "ref_audio": max(t_a, audio_aug)}
    cap_v, cap_a = max(t_v, VISUAL_COND_TIMESTEP), max(t_a, AUDIO_COND_TIMESTEP)

    def per_row(kind: str, rows_t: torch.Tensor) -> Optional[torch.Tensor]:
        """Per-row labels, or None after folding a uniform one into the segment's label."""
        if rows_t.unique().numel() == 1:
            label[kind] = float(rows_t[0])
            return None
        return rows_t

    video_rows = audio_rows = None
    if denoise_mask is not None:
        m = mask_row_values(denoise_mask[0, 0].to(torch.float32).cpu(), lat_t, lat_h, lat_w)
        if m is not None:
            video_rows = per_row("video", (1.0 - m * sigma).clamp(max=cap_v))
    if audio_denoise_mask is not None:
        m = audio_denoise_mask[0, 0].to(torch.float32).cpu().reshape(-1)
        if not bool((m >= 1.0 - 1e-3).all()):
            audio_rows = per_row("audio", (1.0 - m * (1.0 - t_a)).clamp(max=cap_a))

    values = {t_v, t_a} | {label[k] for _, _, k in layout.segments}
    for rows_t in (video_rows, audio_rows):
        if rows_t is not None:
            values |= set(rows_t.unique().tolist())
    t_values = sorted(values)
    index = {t: i for i, t in enumerate(t_values)}

    def rows_of(rows_t: torch.Tensor, tag: int) -> torch.Tensor:
        levels = rows_t.unique()  # sorted
        lut = torch.tensor([index[v] * 3 + tag for v in levels.tolist()], dtype=torch.long)
        return lut[torch.searchsorted(levels, rows_t)]

    tags = None
    if text_tags is not None:
        tags = [int(v) for v in text_tags.reshape(-1).tolist()]
        if len(tags) != text_len or any(v not in (TAG_VIDEO, TAG_TEXT, TAG_AUDIO) for v in tags):
            raise ValueError(f"text_token_tags must hold {text_len} values in {{0,1,2}}")

    mod: List[Tuple[int, int, ModRow]] = []
    for start, stop, kind in layout.segments:
        base = index[label[kind]] * 3
        if kind == "text" and tags is not None:  # runs of equal tag (vision-pad tokens carry the video tag)
            run = 0
            for i in range(1, len(tags) + 1):
                if i == len(tags) or tags[i] != tags[run]:
                    mod.append((start + run, start + i, base + tags[run]))
                    run = i
        elif kind == "video" and video_rows is not None:
            mod.append((start, stop, rows_of(video_rows, TAG_VIDEO)))
        elif kind == "audio" and audio_rows is not None:
            mod.append((start, stop, rows_of(audio_rows, TAG_AUDIO)))
        else:
            mod.append((start, stop, base + KIND_TAG[kind]))

    def final_rows(kind: str, rows_t: Optional[torch.Tensor]) -> Tuple[int, int, ModRow]:
        seg = find_segment(layout, kind)
        return (seg.start, seg.stop, rows_of(rows_t, 0) // 3 if rows_t is not None else index[label[kind]])

    return TimePlan(t_values, mod, final_rows("video", video_rows), final_rows("audio", audio_rows), t_v, t_a)
