"""Whole-model forward of the H3 audio-video DiT over pluggable block weights (reference h3turbo/h3/model.py:118-448).

One velocity prediction runs, on the compute device:

    text   condition_proj + token refiner (plain pre-norm blocks) + RMSNorm   (once per prompt: encode_text)
    embed  patchify video / pack audio, fp32 patch projections, conditioning rows, assembly in layout order
    blocks the DiT block loop through a BlockProvider (resident or streamed), every block on DiTBlock: the four
           W4A8 linears on the HIP kernels, the fused attention prologue / epilogue and RMSNorm + modulation kernels
    final  RMSNorm + AdaLN modulation + the output heads (an n-head bank mixed by the sampler step), unpatchify

The numerics follow the reference op by op: fp32 AdaLN and head math, the checkpoint's fp32 "islands" rounded
through the compute dtype unless fp32_islands=True (h3turbo/h3/model.py:1-12), in-place modulation and gating in
the compute dtype, rope tables rounded to rope_dtype.
"""
from __future__ import annotations

import json
import math
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from .block import BlockConfig, DiTBlock, ResidentProvider, rms, rope_tables  # noqa: F401  (ResidentProvider re-exported)
from .config import H3Config
from .layout import (AUDIO_COND_TIMESTEP, VIDEO_KINDS, VISUAL_COND_TIMESTEP, PackedLayout, TimePlan,
                     bank_head_weights, curve_lerp, head_bank_range, layout_key, pack_audio, pad_to_patch,
                     patchify_video, plan_time, resolve_rope_impl, time_shift_sigma, unpack_audio, unpatchify_video)
from .types import BlockProvider, BlockWeights, GlobalWeights, W4A8Weight, Weight

# fp32 patch projections and output heads run as one GEMM up to this many rows, as the reference does
# (h3turbo/h3/model.py:31-35): the GEMM's tiling follows the row count, so splitting changes last bits.
_PROJ_ROWS = 1 << 16
_LAYOUT_CACHE = 4


class _SequencePlan:
    """Where each source's rows go in the packed sequence of one layout (built once per layout object).

    The packed sequence interleaves text, video, audio and conditioning segments (layout.segments).  Visual rows
    (target video, keyframe / reference images) share the video patch projection and audio rows the audio one, so
    each modality's rows are gathered in segment order, projected as ONE matrix (the projection's row count fixes
    its tiling and thus its last bits, as in the reference) and scattered to their positions with one index copy.
    """

    def __init__(self, layout: PackedLayout, device: torch.device):
        self.text: List[Tuple[int, int]] = []
        self.pieces: Dict[bool, List[Tuple[str, int]]] = {True: [], False: []}  # visual? -> [(kind, rows)]
        where: Dict[bool, List[torch.Tensor]] = {True: [], False: []}
        for start, stop, kind in layout.segments:
            if kind == "text":
                self.text.append((start, stop))
                continue
            visual = kind in VIDEO_KINDS
            self.pieces[visual].append((kind, stop - start))
            where[visual].append(torch.arange(start, stop, dtype=torch.long))
        self.index = {v: torch.cat(w).to(device) if w else None for v, w in where.items()}

    def gather(self, visual: bool, target: torch.Tensor, cond: Optional[torch.Tensor]) -> torch.Tensor:
        """The modality's input rows in segment order: the target's rows for its own segment, the next rows of the
        conditioning rows for each conditioning segment (all of them must be used)."""
        own = "video" if visual else "audio"
        rows, used = [], 0
        for kind, n in self.pieces[visual]:
            if kind == own:
                rows.append(target)
                continue
            if cond is None or used + n > cond.shape[0]:
                raise ValueError(f"payload has too few conditioning {'video' if visual else 'audio'} rows "
                                 f"for segment {kind}")
            rows.append(cond[used:used + n])
            used += n
        if cond is not None and used != cond.shape[0]:
            raise ValueError("payload conditioning rows do not match the layout (keyframes/refs vs cond latents)")
        return torch.cat(rows)


class _AudioCarry:
    """The sampler carries audio on the video sigma schedule, scaled by `audio_scale`; the model undoes the carry on
    its audio input and redoes it on the audio velocity (h3turbo/h3/model.py:384-414)."""

    def __init__(self, audio: torch.Tensor, sigma: torch.Tensor, shifts: Tuple[float, float], scale: float):
        self.scale, self.source = scale, audio
        if scale != 1.0:
            self.sigma_a = time_shift_sigma(sigma, *shifts)
            self.factor = (self.sigma_a / sigma).to(audio.dtype)

    def model_input(self) -> torch.Tensor:
        return self.source if self.scale == 1.0 else self.source * self.factor

    def velocity(self, v: torch.Tensor) -> torch.Tensor:
        if self.scale == 1.0:
            return v
        carried = self.source.to(v.device) * self.factor.to(v.device)
        return (1.0 - self.scale) * carried + (1.0 + (self.scale - 1.0) * self.sigma_a).to(v.dtype) * v


def _sigma_scalar(sigma) -> torch.Tensor:
    """The video sigma as an fp32 CPU scalar, floored at 1e-6 (finite only)."""
    s = (sigma.detach().flatten()[0].to("cpu", torch.float32) if isinstance(sigma, torch.Tensor)
         else torch.tensor(float(sigma), dtype=torch.float32))
    if not math.isfinite(float(s)):
        raise ValueError("sigma must be finite")
    return s.clamp(min=1e-6)


def _check_latents(cfg: H3Config, video: torch.Tensor, audio: torch.Tensor, masks) -> None:
    if video.ndim != 5 or video.shape[0] != 1 or video.shape[1] != cfg.video_channels:
        raise ValueError(f"video latent must be [1, {cfg.video_channels}, T, H, W], got {tuple(video.shape)}")
    if audio.ndim != 4 or audio.shape[0] != 1 or audio.shape[1] != cfg.audio_channels or audio.shape[2] != 2:
        raise ValueError(f"audio latent must be [1, {cfg.audio_channels}, 2, Ta], got {tuple(audio.shape)}")
    for name, m, body in (("denoise_mask", masks[0], video.shape[2:]), ("audio_denoise_mask", masks[1], audio.shape[2:])):
        if m is None:
            continue
        if m.ndim != len(body) + 2 or m.shape[0] != 1 or tuple(m.shape[2:]) != tuple(body):
            raise ValueError(f"{name} must be [1, C, {', '.join(map(str, body))}], got {tuple(m.shape)}")


# device copies of the globals: attribute -> (GlobalWeights field, how it is held)
#   "island": an fp32 tensor as it lives in the checkpoint dtype (rounded through island_dtype unless fp32_islands)
#   "compute": the compute dtype;  "fp32": exact fp32
_GLOBALS = {"vpw": ("video_patch_w", "island"), "vpb": ("video_patch_b", "island"),
            "apw": ("audio_patch_w", "island"), "apb": ("audio_patch_b", "island"),
            "cond_w": ("condition_w", "compute"), "cond_b": ("condition_b", "compute"),
            "table": ("adaln_t_table", "fp32"), "inv_freq": ("rope_inv_freq", "fp32"),
            "final_norm": ("final_norm", "compute"),
            "final_adaln_w": ("final_adaln_w", "island"), "final_adaln_b": ("final_adaln_b", "island"),
            "vow": ("video_out_w", "island"), "vob": ("video_out_b", "island"),
            "aow": ("audio_out_w", "island"), "aob": ("audio_out_b", "island")}


class H3Model:
    """H3 DiT over a BlockProvider (h3turbo/h3/model.py:118-166).

    backend / precision / quant_mode: the W4A8 linears' qlinear options ("hip"; "a8" or "a16").
    mlp_chunk / attn_chunk / rope_chunk: token / query / row chunks bounding peak memory (exact).
    rope_impl: "auto" (= "torch", the fused kernel's numerics, one HIP kernel on the GPU) or "eager".
    attn_backend: "auto" or "default" (accepted for the reference's API; attention runs on PyTorch-ROCm's flash /
    memory-efficient SDPA kernels either way).  attn_impl: "sdpa" (the int8 attention of comfy_kitchen is not part
    of this build).  fp32_islands: keep the checkpoint's fp32 tensors at fp32 instead of rounding them through the
    compute dtype.
    """

    def __init__(self, cfg: H3Config, glob: GlobalWeights, provider: BlockProvider, *, device,
                 dtype: torch.dtype = torch.bfloat16, backend: str = "auto", precision: str = "a8",
                 mlp_chunk: Optional[int] = None, attn_chunk: Optional[int] = None,
                 rope_dtype: Optional[torch.dtype] = None, rope_chunk: int = 1024, rope_impl: str = "auto",
                 fp32_islands: bool = False, attn_backend: str = "auto", attn_impl: str = "sdpa",
                 quant_mode: str = "ck"):
        problems = []
        if dtype not in (torch.bfloat16, torch.float32):
            problems.append(f"compute dtype must be bfloat16 or float32, got {dtype}")
        if backend not in ("auto", "hip", "ck", "torch"):
            problems.append(f"backend {backend!r}")
        if precision not in ("a8", "a16"):
            problems.append(f"precision {precision!r}")
        if attn_backend not in ("auto", "default"):
            problems.append(f"attn_backend {attn_backend!r}")
        if attn_impl not in ("sdpa", "int8"):
            problems.append(f"attn_impl must be 'sdpa' (exact, the reference) or 'int8', got {attn_impl!r}")
        problems += [f"{n} must be >= 1" for n, v in (("mlp_chunk", mlp_chunk), ("attn_chunk", attn_chunk),
                                                     ("rope_chunk", rope_chunk)) if v is not None and v < 1]
        if 6 * cfg.rope_inv_freq_len > cfg.head_dim:
            problems.append(f"rotary width {6 * cfg.rope_inv_freq_len} exceeds head_dim {cfg.head_dim}")
        if problems:
            raise ValueError("; ".join(problems))
        if attn_impl == "int8":
            raise RuntimeError("attn_impl='int8' needs comfy_kitchen's CUDA extension, which this build does not have")
        if cfg.curve_grid < 2 or glob.adaln_t_table is None:
            raise NotImplementedError("only curve-form checkpoints (adaln_t_table, no time embedder) are supported")
        if tuple(cfg.patch[1:]) != (2, 2):
            raise NotImplementedError("the packed layout assumes 2x2 spatial patches")
        self.cfg, self.glob, self.provider = cfg, glob, provider
        self.device, self.dtype = torch.device(device), dtype
        self.backend, self.precision, self.attn_impl = backend, precision, attn_impl
        self.rope_chunk, self.rope_dtype = rope_chunk, rope_dtype or dtype
        self.rope_impl = resolve_rope_impl(rope_impl, device, dtype, self.rope_dtype)
        self.island_dtype = torch.float32 if fp32_islands else dtype
        self.block = DiTBlock(BlockConfig(hidden=cfg.hidden, heads=cfg.heads, head_dim=cfg.head_dim, ffn=cfg.ffn,
                                          act="swiglu", norm_eps=cfg.norm_eps, qk_norm_eps=cfg.qk_norm_eps,
                                          rope_freqs=cfg.rope_inv_freq_len),
                              backend=backend, precision=precision, quant_mode=quant_mode, mlp_chunk=mlp_chunk,
                              attn_chunk=attn_chunk, rope_impl=self.rope_impl, rope_chunk=rope_chunk)
        held = {"island": self._island, "compute": lambda t: t.to(self.dtype), "fp32": lambda t: t.to(torch.float32)}
        for attr, (field, how) in _GLOBALS.items():
            setattr(self, attr, held[how](getattr(glob, field).to(self.device)))
        self.refiner_norm = (None if glob.refiner_final_norm is None
                             else glob.refiner_final_norm.to(self.device, self.dtype))
        rows_v, rows_a = self.vow.shape[0], self.aow.shape[0]
        pd, ac = cfg.video_patch_dim, cfg.audio_channels
        if rows_v % pd or rows_a % ac or rows_v // pd != rows_a // ac:
            raise ValueError(f"output heads {tuple(self.vow.shape)}/{tuple(self.aow.shape)} do not tile {pd}/{ac} rows")
        self.head_bank = rows_v // pd
        self._plans: Dict[tuple, Tuple[PackedLayout, _SequencePlan]] = {}
        self._rope: Optional[tuple] = None

    # chunk knobs of the blocks, settable between forwards
    @property
    def mlp_chunk(self) -> Optional[int]:
        """Tokens per MLP pass of the blocks (None: all)."""
        return self.block.mlp_chunk

    @mlp_chunk.setter
    def mlp_chunk(self, v: Optional[int]) -> None:
        if v is not None and v < 1:
            raise ValueError("mlp_chunk must be >= 1")
        self.block.mlp_chunk = v

    @property
    def attn_chunk(self) -> Optional[int]:
        return self.block.attn_chunk

    @attn_chunk.setter
    def attn_chunk(self, v: Optional[int]) -> None:
        if v is not None and v < 1:
            raise ValueError("attn_chunk must be >= 1")
        self.block.attn_chunk = v

    def _island(self, t: torch.Tensor) -> torch.Tensor:
        """fp32 copy of a tensor as it lives natively in island_dtype (rounded through it)."""
        return t.to(self.island_dtype).to(torch.float32)

    def _modulation(self, t_emb: torch.Tensor, w: Optional[torch.Tensor], b: Optional[torch.Tensor], parts: int,
                    rows_per_t: int) -> Tuple[torch.Tensor, ...]:
        """fp32 AdaLN rows: F.linear(t_emb, w, b) viewed as [T * rows_per_t, parts * hidden], split into `parts`
        (h3turbo/h3/model.py:230-232)."""
        if w is None or b is None:
            raise ValueError("DiT block weights need adaln_w/adaln_b")
        z = F.linear(t_emb, self._island(w.to(self.device)), self._island(b.to(self.device)))
        return z.view(t_emb.shape[0] * rows_per_t, -1).chunk(parts, dim=-1)

    # -------------------------------------------------------------------------------------------- text
    @torch.no_grad()
    def encode_text(self, text_states: torch.Tensor) -> torch.Tensor:
        """[1, L, text_dim] encoder states -> [1, L, hidden] refined embeddings; already-refined input (width
        hidden) passes through (h3turbo/h3/model.py:251-266).  The token refiner is plain pre-norm blocks (no
        modulation, no positions); blocks held off the device come over one at a time."""
        cfg = self.cfg
        if text_states.ndim != 3 or text_states.shape[0] != 1:
            raise ValueError(f"text_states must be [1, L, C], got {tuple(text_states.shape)}")
        width = text_states.shape[-1]
        if width == cfg.hidden:
            return text_states.to(self.device, self.dtype)
        if width != cfg.text_dim or len(self.glob.refiner) != cfg.refiner_layers or self.refiner_norm is None:
            raise ValueError(f"text_states width {width} is neither hidden nor text_dim {cfg.text_dim}, "
                             "or the refiner is missing")
        x = F.linear(text_states[0].to(self.device, self.dtype), self.cond_w, self.cond_b)
        eps = cfg.norm_eps
        for held in self.glob.refiner:
            w = BlockWeights(**{k: None if v is None else v.to(self.device) for k, v in vars(held).items()})
            x = self.block.attention(rms(x, w.norm1, eps), w, None).add_(x)
            x = self.block.mlp(rms(x, w.norm2, eps), w).add_(x)
            del w
        return rms(x, self.refiner_norm, cfg.final_norm_eps).unsqueeze(0)

    # -------------------------------------------------------------------------------------------- sequence
    def _plan_for(self, payload: Mapping[str, Any], text_len: int, latent: Tuple[int, int, int],
                  audio_t: int) -> Tuple[PackedLayout, _SequencePlan]:
        """The layout (the payload's own when its signature matches, else a cached build, h3turbo/h3/model.py:
        270-281) and its sequence plan."""
        given = payload.get("layout")
        if given is not None and tuple(given.signature) == (text_len, *latent, audio_t):
            key = ("given", id(given))
            if key not in self._plans or self._plans[key][0] is not given:
                self._remember(key, (given, _SequencePlan(given, self.device)))
            return self._plans[key]
        key = layout_key(text_len, (*latent, audio_t), payload.get("keyframes"), payload.get("refs"))
        if key not in self._plans:
            layout = PackedLayout.build(text_len, *latent, audio_t, keyframes=payload.get("keyframes"),
                                        refs=payload.get("refs"))
            self._remember(key, (layout, _SequencePlan(layout, self.device)))
        return self._plans[key]

    def _remember(self, key, value) -> None:
        if len(self._plans) >= _LAYOUT_CACHE:
            self._plans.pop(next(iter(self._plans)))
        self._plans[key] = value

    def _rope_for(self, layout: PackedLayout) -> Tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) in rope_dtype on the device, kept while the same layout object is in use."""
        if self._rope is None or self._rope[0] is not layout:
            self._rope = (layout, *rope_tables(layout.position_ids, self.inv_freq, self.device, self.rope_dtype))
        return self._rope[1], self._rope[2]

    def _conditioning(self, latents, pack, aug: float, seed: int) -> Optional[torch.Tensor]:
        """Packed fp32 conditioning rows; below aug 1 each latent's rows are mixed with noise from a CPU stream
        restarted at the same seed (h3turbo/h3/model.py:291-300)."""
        out = []
        for z in latents or ():
            r = pack(z.to(torch.float32))
            if aug < 1.0:
                noise = torch.randn(r.shape, generator=torch.Generator("cpu").manual_seed(seed), dtype=torch.float32)
                r = aug * r + (1.0 - aug) * noise.to(r.device)
            out.append(r.to(self.device))
        return torch.cat(out) if out else None

    def _project(self, rows: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """fp32 rows through a patch projection into the compute dtype, one GEMM per _PROJ_ROWS rows."""
        out = torch.empty(rows.shape[0], w.shape[0], dtype=self.dtype, device=rows.device)
        for lo in range(0, rows.shape[0], _PROJ_ROWS):
            out[lo:lo + _PROJ_ROWS] = F.linear(rows[lo:lo + _PROJ_ROWS], w, b)
        return out

    def _sequence(self, layout: PackedLayout, plan: _SequencePlan, ctx: torch.Tensor, video: torch.Tensor,
                  audio: torch.Tensor, payload: Mapping[str, Any], v_aug: float, a_aug: float) -> torch.Tensor:
        """The hidden sequence [S, hidden] in layout order (h3turbo/h3/model.py:310-343)."""
        patch, seed = tuple(self.cfg.patch), int(payload.get("seed") or 0)
        cond_v = self._conditioning(payload.get("cond_video_latents"), lambda z: patchify_video(z, patch), v_aug, seed)
        cond_a = self._conditioning(payload.get("cond_audio_latents"), pack_audio, a_aug, seed + 1)
        h = torch.empty(layout.seq_len, self.cfg.hidden, dtype=self.dtype, device=self.device)
        for lo, hi in plan.text:
            h[lo:hi] = ctx[0]
        sources = ((True, patchify_video(video.to(self.device, torch.float32), patch), cond_v, self.vpw, self.vpb),
                   (False, pack_audio(audio.to(self.device, torch.float32)), cond_a, self.apw, self.apb))
        for visual, target, cond, w, b in sources:
            rows = plan.gather(visual, target, cond)
            h.index_copy_(0, plan.index[visual], self._project(rows, w, b))
        return h

    def _heads(self, h: torch.Tensor, t_emb: torch.Tensor, tp: TimePlan, sigma, sample_sigmas, shifts):
        """fp32 outputs of the target video and audio rows: RMSNorm, the final AdaLN and the (bank-mixed) output
        heads, one GEMM per _PROJ_ROWS rows (h3turbo/h3/model.py:345-365)."""
        shift, scale = self._modulation(t_emb, self.final_adaln_w, self.final_adaln_b, 2, 1)
        weights = {"video": (self.vow, self.vob), "audio": (self.aow, self.aob)}
        n = self.head_bank
        if n > 1:
            if sample_sigmas is None:
                raise ValueError("this checkpoint has a multi-head output bank; pass the sampler's sigma schedule "
                                 "as sample_sigmas")
            lo, hi = head_bank_range(sample_sigmas, sigma, shifts[0], n)
            weights = {"video": bank_head_weights(self.vow, self.vob, n, lo, hi, shifts[0]),
                       "audio": bank_head_weights(self.aow, self.aob, n, lo, hi, shifts[1])}
        eps = self.cfg.final_norm_eps

        def run(seg, w, b):
            start, stop, mod = seg
            if isinstance(mod, torch.Tensor):
                mod = mod.to(self.device)
            parts = []
            for lo in range(start, stop, _PROJ_ROWS):
                hi = min(stop, lo + _PROJ_ROWS)
                r = mod[lo - start:hi - start] if isinstance(mod, torch.Tensor) else mod
                parts.append(F.linear(rms(h[lo:hi], self.final_norm, eps) * (1.0 + scale[r]) + shift[r], w, b))
            return torch.cat(parts)

        return run(tp.video_seg, *weights["video"]), run(tp.audio_seg, *weights["audio"])

    # -------------------------------------------------------------------------------------------- forward
    @torch.no_grad()
    def forward(self, x: Sequence[torch.Tensor], sigma, text_states: Optional[torch.Tensor], *,
                payload: Optional[Mapping[str, Any]] = None, denoise_mask: Optional[torch.Tensor] = None,
                audio_denoise_mask: Optional[torch.Tensor] = None, sample_sigmas=None,
                refined_text: Optional[torch.Tensor] = None,
                shifts: Optional[Tuple[float, float]] = None) -> List[torch.Tensor]:
        """One velocity prediction (h3turbo/h3/model.py:367-415).  x = [video [1, C, T, H, W], audio
        [1, Ca, 2, Ta]], sigma = the video sigma.  Returns [-video_v, -audio_v] times the denoise masks.  Per-step
        callers pass refined_text = encode_text(...) computed once."""
        cfg, payload = self.cfg, payload or {}
        if len(x) != 2:
            raise ValueError("x must be [video, audio]")
        video, audio = x
        _check_latents(cfg, video, audio, (denoise_mask, audio_denoise_mask))
        sigma_v = _sigma_scalar(sigma)
        shifts = ((float(shifts[0]), float(shifts[1])) if shifts is not None
                  else (cfg.sigma_shift_video, cfg.sigma_shift_audio))
        carry = _AudioCarry(audio, sigma_v, shifts,
                            float(1.0 if payload.get("audio_scale") is None else payload["audio_scale"]))
        v, a = self._predict(video, carry.model_input(), sigma_v, shifts, text_states, refined_text, payload,
                             denoise_mask, audio_denoise_mask, sample_sigmas)
        # masked rows predict at mask * sigma: their velocity scales with the mask
        if denoise_mask is not None:
            v = v * denoise_mask.to(v.device, v.dtype)
        if audio_denoise_mask is not None:
            a = a * audio_denoise_mask.to(a.device, a.dtype)
        return [v, carry.velocity(a)]

    __call__ = forward

    def _predict(self, video, audio, sigma, shifts, text_states, refined_text, payload, denoise_mask,
                 audio_denoise_mask, sample_sigmas) -> List[torch.Tensor]:
        cfg, home = self.cfg, video.device
        t0, h0, w0 = video.shape[2:]
        padded = pad_to_patch(video.to(self.device), cfg.patch)
        lat = tuple(padded.shape[2:])
        text = refined_text if refined_text is not None else text_states
        if text is None:
            raise ValueError("pass text_states or refined_text")
        ctx = self.encode_text(text)
        layout, seq = self._plan_for(payload, ctx.shape[1], lat, audio.shape[-1])
        v_aug = VISUAL_COND_TIMESTEP if payload.get("visual_cond_noise_aug") is None else float(payload["visual_cond_noise_aug"])
        a_aug = AUDIO_COND_TIMESTEP if payload.get("audio_cond_noise_aug") is None else float(payload["audio_cond_noise_aug"])
        tp = plan_time(layout, sigma, shifts, visual_aug=v_aug, audio_aug=a_aug,
                       text_tags=payload.get("text_token_tags"), denoise_mask=denoise_mask,
                       audio_denoise_mask=audio_denoise_mask)
        h = self._sequence(layout, seq, ctx, padded, audio, payload, v_aug, a_aug)
        t_emb = curve_lerp(self.table, tp.t_values)
        segments = [(lo, hi, r.to(self.device) if isinstance(r, torch.Tensor) else r) for lo, hi, r in tp.mod_segments]
        h = self._blocks(h, t_emb, segments, self._rope_for(layout))
        v, a = self._heads(h, t_emb, tp, sigma, sample_sigmas, shifts)
        video_v = unpatchify_video(v, lat[0], lat[1] // 2, lat[2] // 2, cfg.video_channels, cfg.patch)[:, :, :t0, :h0, :w0]
        return [(-video_v).to(home, video.dtype), (-unpack_audio(a)).to(home, audio.dtype)]

    def _blocks(self, h: torch.Tensor, t_emb: torch.Tensor, segments, rope) -> torch.Tensor:
        """The DiT block loop through the provider: acquire block i, run it on its six AdaLN rows, release it."""
        prov = self.provider
        prov.begin_forward()
        try:
            for i in range(self.cfg.layers):
                w = prov.acquire(i)
                try:
                    h = self.block.forward(h, w, self._modulation(t_emb, w.adaln_w, w.adaln_b, 6, 3), segments, rope)
                finally:
                    prov.release(i)
        finally:
            prov.end_forward()
        return h


# ------------------------------------------------------------------------------------------------ weights
class _StateDict:
    """Typed, shape-checked reads of a ComfyUI-layout state dict; every missing name is collected, not raised."""

    def __init__(self, sd: Mapping[str, torch.Tensor], prefix: str, device, dtype: torch.dtype, group: int, rot: int):
        self.sd, self.prefix, self.device, self.dtype = sd, prefix, device, dtype
        self.group, self.rot = group, rot  # W4A8 defaults when a layer's comfy_quant JSON does not say
        self.missing: List[str] = []

    def raw(self, name: str, shape: Optional[Tuple[int, ...]] = None) -> Optional[torch.Tensor]:
        t = self.sd.get(self.prefix + name)
        if t is None:
            self.missing.append(self.prefix + name)
        elif shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{self.prefix + name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
        return t

    def get(self, name: str, shape, dt: Optional[torch.dtype]) -> Optional[torch.Tensor]:
        """On the device in `dt` (None: the stored dtype)."""
        t = self.raw(name, shape)
        return None if t is None else t.to(device=self.device, dtype=dt or t.dtype)

    def linear(self, name: str, n: int, k: int) -> Optional[Weight]:
        """A dense [n, k] matrix in the compute dtype, or a W4A8 layer (one with `weight_s_rel`) whose comfy_quant
        JSON, when present, names the format, group size and rotation size."""
        q = self.raw(name + ".weight")
        if q is None:
            return None
        if self.prefix + name + ".weight_s_rel" not in self.sd:
            if tuple(q.shape) != (n, k):
                raise ValueError(f"{self.prefix + name}.weight: expected {(n, k)}, got {tuple(q.shape)}")
            return q.to(device=self.device, dtype=self.dtype)
        blob = self.sd.get(self.prefix + name + ".comfy_quant")
        conf = json.loads(blob.cpu().numpy().tobytes()) if blob is not None else {}
        if conf.get("format", "asym_w4a8_int8") != "asym_w4a8_int8" or conf.get("full_precision_matrix_mult"):
            raise NotImplementedError(f"{self.prefix + name}: unsupported quantization config {conf}")
        params = conf.get("params") if isinstance(conf.get("params"), dict) else {}
        group = int(conf.get("group_size", params.get("group_size", self.group)))
        rot = int(conf.get("convrot_groupsize", params.get("convrot_groupsize", self.rot)))
        s_rel = self.raw(name + ".weight_s_rel")
        s_ch = self.raw(name + ".weight_s_channel", (n,))
        book = self.raw(name + ".weight_codebook", (16,))
        if s_rel is None or s_ch is None or book is None:
            return None
        if s_rel.dtype == torch.uint8:
            s_rel = s_rel.view(torch.float8_e4m3fn)
        if (q.ndim != 2 or (q.shape[0], 2 * q.shape[1]) != (n, k) or k % group or k % rot
                or tuple(s_rel.shape) != (n, k // group)):
            raise ValueError(f"{self.prefix + name}: W4A8 shapes q{tuple(q.shape)} s_rel{tuple(s_rel.shape)} do not "
                             f"match {(n, k)}/g{group}/r{rot}")
        f32 = torch.float32
        return W4A8Weight(q.to(device=self.device, dtype=torch.int8), s_rel.to(self.device),
                          s_ch.to(device=self.device, dtype=f32), book.to(device=self.device, dtype=f32), group, rot)


def weights_from_state_dict(sd: Mapping[str, torch.Tensor], cfg: H3Config, device, dtype: torch.dtype,
                            *, prefix: str = "") -> Tuple[GlobalWeights, List[BlockWeights]]:
    """Model weights from a ComfyUI-layout state dict of dense and/or W4A8 layers (h3turbo/h3/model.py:451-525).

    Dense linears and norms are cast to the compute dtype; the fp32 islands (patch projections, output heads,
    AdaLN table and biases) stay fp32.  Shapes are checked against cfg; every missing key is reported at once.
    A W4A8 layer is one whose `<name>.weight_s_rel` is present; its `comfy_quant` JSON (when given) names the
    format, group size and rotation size (defaults: cfg.quant_group, cfg.quant_convrot).
    """
    f32 = torch.float32
    r = _StateDict(sd, prefix, device, dtype, cfg.quant_group, cfg.quant_convrot)
    hid, inner, hd, ffn, td = cfg.hidden, cfg.inner, cfg.head_dim, cfg.ffn, cfg.t_dim

    def block(base: str, modulated: bool) -> BlockWeights:
        return BlockWeights(
            qkv=r.linear(f"{base}.attn.qkv_proj", 3 * inner, hid), out=r.linear(f"{base}.attn.out_proj", hid, inner),
            fc1=r.linear(f"{base}.mlp.fc1", 2 * ffn, hid), fc2=r.linear(f"{base}.mlp.fc2", hid, ffn),
            norm1=r.get(f"{base}.norm1.weight", (hid,), dtype), norm2=r.get(f"{base}.norm2.weight", (hid,), dtype),
            q_norm=r.get(f"{base}.attn.q_norm.weight", (hd,), dtype),
            k_norm=r.get(f"{base}.attn.k_norm.weight", (hd,), dtype),
            adaln_w=r.get(f"{base}.adaln_proj.linear.weight", (18 * hid, td), None) if modulated else None,
            adaln_b=r.get(f"{base}.adaln_proj.linear.bias", (18 * hid,), f32) if modulated else None)

    blocks = [block(f"blocks.{i}", True) for i in range(cfg.layers)]
    refiner = [block(f"token_refiner.blocks.{j}", False) for j in range(cfg.refiner_layers)]
    # GlobalWeights field -> (state-dict name, shape or None (any), dtype)
    spec = {"video_patch_w": ("video_patch_proj.weight", (hid, cfg.video_patch_dim), f32),
            "video_patch_b": ("video_patch_proj.bias", (hid,), f32),
            "audio_patch_w": ("audio_patch_proj.weight", (hid, cfg.audio_channels), f32),
            "audio_patch_b": ("audio_patch_proj.bias", (hid,), f32),
            "condition_w": ("condition_proj.weight", (hid, cfg.text_dim), dtype),
            "condition_b": ("condition_proj.bias", (hid,), dtype),
            "adaln_t_table": ("adaln_t_table", (cfg.curve_grid, td), f32),
            "rope_inv_freq": ("rope.inv_freq", (cfg.rope_inv_freq_len,), f32),
            "final_norm": ("final_layer.norm.weight", (hid,), dtype),
            "final_adaln_w": ("final_layer.adaln_proj.linear.weight", (2 * hid, td), f32),
            "final_adaln_b": ("final_layer.adaln_proj.linear.bias", (2 * hid,), f32),
            "video_out_w": ("final_layer.video_out.weight", None, f32),
            "video_out_b": ("final_layer.video_out.bias", None, f32),
            "audio_out_w": ("final_layer.audio_out.weight", None, f32),
            "audio_out_b": ("final_layer.audio_out.bias", None, f32),
            "refiner_final_norm": ("token_refiner.final_norm.weight", (hid,), dtype)}
    glob = GlobalWeights(refiner=refiner, **{f: r.get(name, shape, dt) for f, (name, shape, dt) in spec.items()})
    if r.missing:
        raise KeyError(f"state dict is missing {len(r.missing)} tensors, e.g. {r.missing[:6]}")
    return glob, blocks
