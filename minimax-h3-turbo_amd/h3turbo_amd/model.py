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
from .layout import (AUDIO_COND_TIMESTEP, AUDIO_KINDS, VIDEO_KINDS, VISUAL_COND_TIMESTEP, PackedLayout, TimePlan,
                     bank_head_weights, curve_lerp, head_bank_range, layout_key, pack_audio, pad_to_patch,
                     patchify_video, plan_time, resolve_rope_impl, time_shift_sigma, unpack_audio, unpatchify_video)
from .types import BlockProvider, BlockWeights, GlobalWeights, W4A8Weight, Weight

_COND_VIDEO, _COND_AUDIO = ("cond", "ref_img"), ("cond_audio", "ref_audio")
# fp32 patch projections and output heads run as one GEMM up to this many rows, as the reference does
# (h3turbo/h3/model.py:31-35): the GEMM's tiling follows the row count, so splitting changes last bits.
_PROJ_ROWS = 1 << 16
_LAYOUT_CACHE = 4


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
        if dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"compute dtype must be bfloat16 or float32, got {dtype}")
        if (backend not in ("auto", "hip", "ck", "torch") or precision not in ("a8", "a16")
                or attn_backend not in ("auto", "default")):
            raise ValueError(f"bad backend/precision/attn_backend: {backend!r}/{precision!r}/{attn_backend!r}")
        if attn_impl not in ("sdpa", "int8"):
            raise ValueError(f"attn_impl must be 'sdpa' (exact, the reference) or 'int8', got {attn_impl!r}")
        if attn_impl == "int8":
            raise RuntimeError("attn_impl='int8' needs comfy_kitchen's CUDA extension, which this build does not have")
        if cfg.curve_grid < 2 or glob.adaln_t_table is None:
            raise NotImplementedError("only curve-form checkpoints (adaln_t_table, no time embedder) are supported")
        if tuple(cfg.patch[1:]) != (2, 2):
            raise NotImplementedError("the packed layout assumes 2x2 spatial patches")
        if 6 * cfg.rope_inv_freq_len > cfg.head_dim:
            raise ValueError(f"rotary width {6 * cfg.rope_inv_freq_len} exceeds head_dim {cfg.head_dim}")
        for name, v in (("mlp_chunk", mlp_chunk), ("attn_chunk", attn_chunk), ("rope_chunk", rope_chunk)):
            if v is not None and v < 1:
                raise ValueError(f"{name} must be >= 1")
        self.cfg, self.provider, self.device, self.dtype = cfg, provider, torch.device(device), dtype
        self.backend, self.precision, self.attn_impl = backend, precision, attn_impl
        self.rope_chunk = rope_chunk
        self.rope_dtype = rope_dtype or dtype
        self.rope_impl = resolve_rope_impl(rope_impl, device, dtype, self.rope_dtype)
        self.glob = glob
        self.island_dtype = torch.float32 if fp32_islands else dtype
        self.block = DiTBlock(BlockConfig(hidden=cfg.hidden, heads=cfg.heads, head_dim=cfg.head_dim, ffn=cfg.ffn,
                                          act="swiglu", norm_eps=cfg.norm_eps, qk_norm_eps=cfg.qk_norm_eps,
                                          rope_freqs=cfg.rope_inv_freq_len),
                              backend=backend, precision=precision, quant_mode=quant_mode, mlp_chunk=mlp_chunk,
                              attn_chunk=attn_chunk, rope_impl=self.rope_impl, rope_chunk=rope_chunk)
        f32 = torch.float32

        def dev(t: torch.Tensor, dt: Optional[torch.dtype] = None) -> torch.Tensor:
            return t.to(device=self.device, dtype=dt or t.dtype)

        def isl(t: torch.Tensor) -> torch.Tensor:
            return self._island(dev(t))

        self.vpw, self.vpb = isl(glob.video_patch_w), isl(glob.video_patch_b)
        self.apw, self.apb = isl(glob.audio_patch_w), isl(glob.audio_patch_b)
        self.cond_w, self.cond_b = dev(glob.condition_w, dtype), dev(glob.condition_b, dtype)
        self.table, self.inv_freq = dev(glob.adaln_t_table, f32), dev(glob.rope_inv_freq, f32)
        self.final_norm = dev(glob.final_norm, dtype)
        self.final_adaln_w, self.final_adaln_b = isl(glob.final_adaln_w), isl(glob.final_adaln_b)
        self.vow, self.vob = isl(glob.video_out_w), isl(glob.video_out_b)
        self.aow, self.aob = isl(glob.audio_out_w), isl(glob.audio_out_b)
        self.refiner_norm = None if glob.refiner_final_norm is None else dev(glob.refiner_final_norm, dtype)
        pd, ac = cfg.video_patch_dim, cfg.audio_channels
        if self.vow.shape[0] % pd or self.aow.shape[0] % ac or self.vow.shape[0] // pd != self.aow.shape[0] // ac:
            raise ValueError(f"output heads {tuple(self.vow.shape)}/{tuple(self.aow.shape)} do not tile {pd}/{ac} rows")
        self.head_bank = self.vow.shape[0] // pd
        self._layouts: Dict[tuple, PackedLayout] = {}
        self._rope: Optional[tuple] = None

    @property
    def mlp_chunk(self) -> Optional[int]:
        """Tokens per MLP pass of the blocks (None: all); settable between forwards."""
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

    # -------------------------------------------------------------------------------------------- primitives
    def _island(self, t: torch.Tensor) -> torch.Tensor:
        """fp32 copy of a tensor as it lives natively in island_dtype (rounded through it)."""
        return t.to(self.island_dtype).to(torch.float32)

    def _adaln(self, t_emb: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], parts: int,
               mods: int) -> Tuple[torch.Tensor, ...]:
        """fp32 modulation rows: F.linear(t_emb, w, b) as [T * mods, parts * hidden], split into `parts`
        (h3turbo/h3/model.py:230-232)."""
        if weight is None or bias is None:
            raise ValueError("DiT block weights need adaln_w/adaln_b")
        z = F.linear(t_emb, self._island(weight.to(self.device)), self._island(bias.to(self.device)))
        return z.view(t_emb.shape[0] * mods, -1).chunk(parts, dim=-1)

    def _refiner_block(self, x: torch.Tensor, w: BlockWeights) -> torch.Tensor:
        """Pre-norm block without modulation or positions (h3turbo/h3/model.py:244-247)."""
        eps = self.cfg.norm_eps
        x = self.block.attention(rms(x, w.norm1, eps), w, None).add_(x)
        return self.block.mlp(rms(x, w.norm2, eps), w).add_(x)

    # -------------------------------------------------------------------------------------------- text
    @torch.no_grad()
    def encode_text(self, text_states: torch.Tensor) -> torch.Tensor:
        """[1, L, text_dim] encoder states -> [1, L, hidden] refined embeddings; already-refined input (width
        hidden) passes through (h3turbo/h3/model.py:251-266).  Refiner blocks held off the device come over one at
        a time."""
        cfg = self.cfg
        if text_states.ndim != 3 or text_states.shape[0] != 1:
            raise ValueError(f"text_states must be [1, L, C], got {tuple(text_states.shape)}")
        if text_states.shape[-1] == cfg.hidden:
            return text_states.to(self.device, self.dtype)
        if (text_states.shape[-1] != cfg.text_dim or len(self.glob.refiner) != cfg.refiner_layers
                or self.refiner_norm is None):
            raise ValueError(f"text_states width {text_states.shape[-1]} is neither hidden nor text_dim {cfg.text_dim}, "
                             "or the refiner is missing")
        x = F.linear(text_states[0].to(self.device, self.dtype), self.cond_w, self.cond_b)
        for blk in self.glob.refiner:
            on_dev = BlockWeights(**{k: None if v is None else v.to(self.device) for k, v in vars(blk).items()})
            x = self._refiner_block(x, on_dev)
            del on_dev
        return rms(x, self.refiner_norm, cfg.final_norm_eps).unsqueeze(0)

    # -------------------------------------------------------------------------------------------- forward parts
    def _layout(self, payload: Mapping[str, Any], text_len: int, shape: Tuple[int, int, int], audio_t: int) -> PackedLayout:
        """The payload's prebuilt layout when its signature matches, else a cached build (h3turbo/h3/model.py:270-281)."""
        given = payload.get("layout")
        if given is not None and tuple(given.signature) == (text_len, *shape, audio_t):
            return given
        key = layout_key(text_len, (*shape, audio_t), payload.get("keyframes"), payload.get("refs"))
        if key not in self._layouts:
            if len(self._layouts) >= _LAYOUT_CACHE:
                self._layouts.pop(next(iter(self._layouts)))
            self._layouts[key] = PackedLayout.build(text_len, *shape, audio_t, keyframes=payload.get("keyframes"),
                                                    refs=payload.get("refs"))
        return self._layouts[key]

    def _rope_tables(self, layout: PackedLayout) -> Tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) in rope_dtype on the device, cached while the same layout object is in use."""
        if self._rope is None or self._rope[0] is not layout:
            cos, sin = rope_tables(layout.position_ids, self.inv_freq, self.device, self.rope_dtype)
            self._rope = (layout, cos, sin)
        return self._rope[1], self._rope[2]

    def _cond_rows(self, latents, pack, aug: float, seed: int) -> Optional[torch.Tensor]:
        """Packed fp32 conditioning rows; below aug 1 each is mixed with noise that restarts the same seeded CPU
        stream (h3turbo/h3/model.py:291-300)."""
        rows = []
        for z in latents or ():
            r = pack(z.to(torch.float32))
            if aug < 1.0:
                g = torch.Generator("cpu").manual_seed(seed)
                noise = torch.randn(r.shape, generator=g, dtype=torch.float32)
                r = aug * r + (1.0 - aug) * noise.to(r.device)
            rows.append(r.to(self.device))
        return torch.cat(rows, dim=0) if rows else None

    def _project(self, rows: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """fp32 patch projection into the compute dtype, one GEMM per _PROJ_ROWS rows."""
        out = torch.empty(rows.shape[0], w.shape[0], dtype=self.dtype, device=rows.device)
        for a in range(0, rows.shape[0], _PROJ_ROWS):
            out[a:a + _PROJ_ROWS] = F.linear(rows[a:a + _PROJ_ROWS], w, b)
        return out

    def _embed(self, layout: PackedLayout, ctx: torch.Tensor, video_x: torch.Tensor, audio_x: torch.Tensor,
               payload: Mapping[str, Any], v_aug: float, a_aug: float) -> torch.Tensor:
        """The hidden sequence [S, hidden] in layout order (h3turbo/h3/model.py:310-343)."""
        cfg, patch, seed = self.cfg, tuple(self.cfg.patch), int(payload.get("seed") or 0)
        cond_v = self._cond_rows(payload.get("cond_video_latents"), lambda z: patchify_video(z, patch), v_aug, seed)
        cond_a = self._cond_rows(payload.get("cond_audio_latents"), pack_audio, a_aug, seed + 1)
        img: List[torch.Tensor] = []
        aud: List[torch.Tensor] = []
        used = {True: 0, False: 0}  # conditioning rows consumed: video, audio
        for start, stop, kind in layout.segments:
            n = stop - start
            if kind == "video":
                img.append(patchify_video(video_x.to(self.device, torch.float32), patch))
            elif kind == "audio":
                aud.append(pack_audio(audio_x.to(self.device, torch.float32)))
            elif kind in _COND_VIDEO or kind in _COND_AUDIO:
                is_v = kind in _COND_VIDEO
                src = cond_v if is_v else cond_a
                at = used[is_v]
                if src is None or at + n > src.shape[0]:
                    raise ValueError(f"payload has too few conditioning {'video' if is_v else 'audio'} rows "
                                     f"for segment {kind}")
                (img if is_v else aud).append(src[at:at + n])
                used[is_v] = at + n
        if (cond_v is not None and used[True] != cond_v.shape[0]) or (cond_a is not None and used[False] != cond_a.shape[0]):
            raise ValueError("payload conditioning rows do not match the layout (keyframes/refs vs cond latents)")
        img_e = self._project(torch.cat(img), self.vpw, self.vpb)
        aud_e = self._project(torch.cat(aud), self.apw, self.apb)
        h = torch.empty(layout.seq_len, cfg.hidden, dtype=self.dtype, device=self.device)
        at_i = at_a = 0
        for start, stop, kind in layout.segments:
            n = stop - start
            if kind == "text":
                h[start:stop] = ctx[0]
            elif kind in VIDEO_KINDS:
                h[start:stop] = img_e[at_i:at_i + n]
                at_i += n
            else:
                h[start:stop] = aud_e[at_a:at_a + n]
                at_a += n
        return h

    def _final(self, h: torch.Tensor, t_emb: torch.Tensor, plan: TimePlan, sigma, sample_sigmas, shifts):
        """Output heads of the target video and audio rows, fp32 (h3turbo/h3/model.py:345-365)."""
        cfg = self.cfg
        shift, scale = self._adaln(t_emb, self.final_adaln_w, self.final_adaln_b, 2, 1)

        def head(seg, w, b):
            start, stop, row = seg
            row = row.to(self.device) if isinstance(row, torch.Tensor) else row
            outs = []
            for a in range(start, stop, _PROJ_ROWS):
                e = min(stop, a + _PROJ_ROWS)
                r = row[a - start:e - start] if isinstance(row, torch.Tensor) else row
                normed = rms(h[a:e], self.final_norm, cfg.final_norm_eps)
                outs.append(F.linear(normed * (1.0 + scale[r]) + shift[r], w, b))
            return torch.cat(outs)

        n, vw, vb, aw, ab = self.head_bank, self.vow, self.vob, self.aow, self.aob
        if n > 1:
            if sample_sigmas is None:
                raise ValueError("this checkpoint has a multi-head output bank; pass the sampler's sigma schedule "
                                 "as sample_sigmas")
            start, stop = head_bank_range(sample_sigmas, sigma, shifts[0], n)
            vw, vb = bank_head_weights(vw, vb, n, start, stop, shifts[0])
            aw, ab = bank_head_weights(aw, ab, n, start, stop, shifts[1])
        return head(plan.video_seg, vw, vb), head(plan.audio_seg, aw, ab)

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
        video_x, audio_x = x
        if video_x.ndim != 5 or video_x.shape[0] != 1 or video_x.shape[1] != cfg.video_channels:
            raise ValueError(f"video latent must be [1, {cfg.video_channels}, T, H, W], got {tuple(video_x.shape)}")
        if (audio_x.ndim != 4 or audio_x.shape[0] != 1 or audio_x.shape[1] != cfg.audio_channels
                or audio_x.shape[2] != 2):
            raise ValueError(f"audio latent must be [1, {cfg.audio_channels}, 2, Ta], got {tuple(audio_x.shape)}")
        for name, m, ref_shape in (("denoise_mask", denoise_mask, video_x.shape[2:]),
                                   ("audio_denoise_mask", audio_denoise_mask, audio_x.shape[2:])):
            if m is not None and (m.shape[0] != 1 or tuple(m.shape[2:]) != tuple(ref_shape)
                                  or m.ndim != len(ref_shape) + 2):
                raise ValueError(f"{name} must be [1, C, {', '.join(map(str, ref_shape))}], got {tuple(m.shape)}")
        if isinstance(sigma, torch.Tensor):
            sigma_v = sigma.detach().flatten()[0].to("cpu", torch.float32)
        else:
            sigma_v = torch.tensor(float(sigma), dtype=torch.float32)
        if not math.isfinite(float(sigma_v)):
            raise ValueError("sigma must be finite")
        sigma_v = sigma_v.clamp(min=1e-6)
        shifts = ((float(shifts[0]), float(shifts[1])) if shifts is not None
                  else (cfg.sigma_shift_video, cfg.sigma_shift_audio))

        # audio carried on the video schedule by the sampler: undone here, redone on the velocity
        scale = float(1.0 if payload.get("audio_scale") is None else payload["audio_scale"])
        audio_src = audio_x
        if scale != 1.0:
            sigma_a = time_shift_sigma(sigma_v, *shifts)
            carry = (sigma_a / sigma_v).to(audio_src.dtype)
            audio_x = audio_src * carry

        out_v, out_a = self._forward(video_x, audio_x, sigma_v, shifts, text_states, refined_text, payload,
                                     denoise_mask, audio_denoise_mask, sample_sigmas)
        if denoise_mask is not None:  # masked rows predict at mask * sigma: their velocity scales with it
            out_v = out_v * denoise_mask.to(out_v.device, out_v.dtype)
        if audio_denoise_mask is not None:
            out_a = out_a * audio_denoise_mask.to(out_a.device, out_a.dtype)
        if scale != 1.0:
            out_a = ((1.0 - scale) * (audio_src.to(out_a.device) * carry.to(out_a.device))
                     + (1.0 + (scale - 1.0) * sigma_a).to(out_a.dtype) * out_a)
        return [out_v, out_a]

    __call__ = forward

    def _forward(self, video_x, audio_x, sigma, shifts, text_states, refined_text, payload, denoise_mask,
                 audio_denoise_mask, sample_sigmas) -> List[torch.Tensor]:
        cfg, in_device = self.cfg, video_x.device
        orig_t, orig_h, orig_w = video_x.shape[2:]
        padded = pad_to_patch(video_x.to(self.device), cfg.patch)
        lat_t, lat_h, lat_w = padded.shape[2:]
        src = refined_text if refined_text is not None else text_states
        if src is None:
            raise ValueError("pass text_states or refined_text")
        ctx = self.encode_text(src)
        layout = self._layout(payload, ctx.shape[1], (lat_t, lat_h, lat_w), audio_x.shape[-1])

        def aug(key: str, default: float) -> float:
            return default if payload.get(key) is None else float(payload[key])

        v_aug, a_aug = aug("visual_cond_noise_aug", VISUAL_COND_TIMESTEP), aug("audio_cond_noise_aug", AUDIO_COND_TIMESTEP)
        plan = plan_time(layout, sigma, shifts, visual_aug=v_aug, audio_aug=a_aug,
                         text_tags=payload.get("text_token_tags"), denoise_mask=denoise_mask,
                         audio_denoise_mask=audio_denoise_mask)
        h = self._embed(layout, ctx, padded, audio_x, payload, v_aug, a_aug)
        t_emb = curve_lerp(self.table, plan.t_values)
        segments = [(a, b, r.to(self.device) if isinstance(r, torch.Tensor) else r) for a, b, r in plan.mod_segments]
        rope = self._rope_tables(layout)
        prov = self.provider
        prov.begin_forward()
        try:
            for i in range(cfg.layers):
                w = prov.acquire(i)
                try:
                    h = self.block.forward(h, w, self._adaln(t_emb, w.adaln_w, w.adaln_b, 6, 3), segments, rope)
                finally:
                    prov.release(i)
        finally:
            prov.end_forward()
        v, a = self._final(h, t_emb, plan, sigma, sample_sigmas, shifts)
        video = unpatchify_video(v, lat_t, lat_h // 2, lat_w // 2, cfg.video_channels, cfg.patch)
        video = video[:, :, :orig_t, :orig_h, :orig_w]
        return [(-video).to(in_device, video_x.dtype), (-unpack_audio(a)).to(in_device, audio_x.dtype)]


# ------------------------------------------------------------------------------------------------ weights
def weights_from_state_dict(sd: Mapping[str, torch.Tensor], cfg: H3Config, device, dtype: torch.dtype,
                            *, prefix: str = "") -> Tuple[GlobalWeights, List[BlockWeights]]:
    """Model weights from a ComfyUI-layout state dict of dense and/or W4A8 layers (h3turbo/h3/model.py:451-525).

    Dense linears and norms are cast to the compute dtype; the fp32 islands (patch projections, output heads,
    AdaLN table and biases) stay fp32.  Shapes are checked against cfg; every missing key is reported at once.
    A W4A8 layer is one whose `<name>.weight_s_rel` is present; its `comfy_quant` JSON (when given) names the
    format, group size and rotation size.
    """
    f32 = torch.float32
    missing: List[str] = []
    hid, inner, hd = cfg.hidden, cfg.inner, cfg.head_dim

    def fetch(name: str, shape: Optional[Tuple[int, ...]] = None) -> Optional[torch.Tensor]:
        t = sd.get(prefix + name)
        if t is None:
            missing.append(prefix + name)
            return None
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{prefix + name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
        return t

    def cast(name: str, shape, dt) -> Optional[torch.Tensor]:
        t = fetch(name, shape)
        return None if t is None else t.to(device=device, dtype=dt or t.dtype)

    def linear(name: str, n: int, k: int) -> Optional[Weight]:
        q = fetch(name + ".weight")
        if q is None:
            return None
        if prefix + name + ".weight_s_rel" not in sd:
            if tuple(q.shape) != (n, k):
                raise ValueError(f"{prefix + name}.weight: expected {(n, k)}, got {tuple(q.shape)}")
            return q.to(device=device, dtype=dtype)
        raw = sd.get(prefix + name + ".comfy_quant")
        conf = json.loads(raw.cpu().numpy().tobytes()) if raw is not None else {}
        if conf.get("format", "asym_w4a8_int8") != "asym_w4a8_int8" or conf.get("full_precision_matrix_mult"):
            raise NotImplementedError(f"{prefix + name}: unsupported quantization config {conf}")
        params = conf.get("params") if isinstance(conf.get("params"), dict) else {}
        group = int(conf.get("group_size", params.get("group_size", cfg.quant_group)))
        rot = int(conf.get("convrot_groupsize", params.get("convrot_groupsize", cfg.quant_convrot)))
        s_rel = fetch(name + ".weight_s_rel")
        s_ch = fetch(name + ".weight_s_channel", (n,))
        book = fetch(name + ".weight_codebook", (16,))
        if s_rel is None or s_ch is None or book is None:
            return None
        if s_rel.dtype == torch.uint8:
            s_rel = s_rel.view(torch.float8_e4m3fn)
        if (q.ndim != 2 or (q.shape[0], q.shape[1] * 2) != (n, k) or k % group or k % rot
                or tuple(s_rel.shape) != (n, k // group)):
            raise ValueError(f"{prefix + name}: W4A8 shapes q{tuple(q.shape)} s_rel{tuple(s_rel.shape)} do not match "
                             f"{(n, k)}/g{group}/r{rot}")
        return W4A8Weight(q.to(device=device, dtype=torch.int8), s_rel.to(device), s_ch.to(device=device, dtype=f32),
                          book.to(device=device, dtype=f32), group, rot)

    def block(base: str, adaln: bool) -> BlockWeights:
        return BlockWeights(
            qkv=linear(base + ".attn.qkv_proj", 3 * inner, hid), out=linear(base + ".attn.out_proj", hid, inner),
            fc1=linear(base + ".mlp.fc1", 2 * cfg.ffn, hid), fc2=linear(base + ".mlp.fc2", hid, cfg.ffn),
            norm1=cast(base + ".norm1.weight", (hid,), dtype), norm2=cast(base + ".norm2.weight", (hid,), dtype),
            q_norm=cast(base + ".attn.q_norm.weight", (hd,), dtype),
            k_norm=cast(base + ".attn.k_norm.weight", (hd,), dtype),
            adaln_w=cast(base + ".adaln_proj.linear.weight", (18 * hid, cfg.t_dim), None) if adaln else None,
            adaln_b=cast(base + ".adaln_proj.linear.bias", (18 * hid,), f32) if adaln else None)

    blocks = [block(f"blocks.{i}", True) for i in range(cfg.layers)]
    refiner = [block(f"token_refiner.blocks.{j}", False) for j in range(cfg.refiner_layers)]
    pd, ac = cfg.video_patch_dim, cfg.audio_channels
    glob = GlobalWeights(
        video_patch_w=cast("video_patch_proj.weight", (hid, pd), f32),
        video_patch_b=cast("video_patch_proj.bias", (hid,), f32),
        audio_patch_w=cast("audio_patch_proj.weight", (hid, ac), f32),
        audio_patch_b=cast("audio_patch_proj.bias", (hid,), f32),
        condition_w=cast("condition_proj.weight", (hid, cfg.text_dim), dtype),
        condition_b=cast("condition_proj.bias", (hid,), dtype),
        adaln_t_table=cast("adaln_t_table", (cfg.curve_grid, cfg.t_dim), f32),
        rope_inv_freq=cast("rope.inv_freq", (cfg.rope_inv_freq_len,), f32),
        final_norm=cast("final_layer.norm.weight", (hid,), dtype),
        final_adaln_w=cast("final_layer.adaln_proj.linear.weight", (2 * hid, cfg.t_dim), f32),
        final_adaln_b=cast("final_layer.adaln_proj.linear.bias", (2 * hid,), f32),
        video_out_w=cast("final_layer.video_out.weight", None, f32),
        video_out_b=cast("final_layer.video_out.bias", None, f32),
        audio_out_w=cast("final_layer.audio_out.weight", None, f32),
        audio_out_b=cast("final_layer.audio_out.bias", None, f32),
        refiner=refiner, refiner_final_norm=cast("token_refiner.final_norm.weight", (hid,), dtype))
    if missing:
        raise KeyError(f"state dict is missing {len(missing)} tensors, e.g. {missing[:6]}")
    return glob, blocks
