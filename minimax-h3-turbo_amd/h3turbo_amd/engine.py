"""Engine façade over a block store: streaming provider + DiT block runner + whole-model forward and sampler
(the API of the reference's H3Engine, h3turbo/h3/engine.py:1-132).

An engine over an .h3t file that holds the model's global tensors (patch projections, AdaLN table, token refiner,
output heads) runs the whole H3 model: encode_text, velocity (one forward) and sample (the Euler sampler on each
stream's own sigma schedule).  Over a store of blocks only (for example a synthetic block stack) it runs the block
loop (blocks).  Text states and the VAEs are inputs / outputs of the engine, not part of it.
"""
from __future__ import annotations

import dataclasses
from typing import Any, Callable, Dict, List, Mapping, Optional, Sequence, Tuple

import torch

from . import qlinear
from .block import BlockConfig, DiTBlock, Segment, run_blocks
from .blockstore import HostBlockStore
from .layout import time_shift_sigma
from .model import H3Model
from .stream import StreamingProvider
from .types import GlobalWeights

_GIB = 1 << 30


def h3_sigmas(steps: int, shift: float) -> torch.Tensor:
    """Flow-matching sigmas with time shift `shift`: steps + 1 fp32 values from 1 down to 0
    (h3turbo/h3/engine.py:22-28)."""
    if steps < 1:
        raise ValueError("steps must be >= 1")
    t = torch.linspace(1.0, 0.0, steps + 1, dtype=torch.float64)
    return (shift * t / (1.0 + (shift - 1.0) * t)).to(torch.float32)


class H3Engine:
    def __init__(self, store, provider: StreamingProvider, block: DiTBlock, owns_store: bool = False,
                 model: Optional[H3Model] = None, model_error: Optional[str] = None):
        self.store, self.provider, self.block, self._owns_store = store, provider, block, owns_store
        self.model, self._model_error = model, model_error
        self.cfg = model.cfg if model is not None else getattr(store, "cfg", None) or block.cfg

    @classmethod
    def from_h3t(cls, path, device: Optional[str] = None, *, load_pinned: Optional[bool] = None,
                 whole_model="auto", refiner_on_gpu: bool = False, **kw) -> "H3Engine":
        """Open an .h3t file and build an engine over it (h3turbo/h3/engine.py:33-44).  The block config comes from
        the file's H3Config (the H3 block: SwiGLU MLP).  load_pinned (default: on a GPU) first copies every block
        into page-locked host memory, so the streamed blocks reach HBM as direct DMA transfers; with False the
        engine streams from the file mapping through its staging buffers.  whole_model: "auto" builds the
        whole-model forward when the file holds the global tensors and its config is runnable, True requires it,
        False runs the block loop only.  The token refiner stays in host memory unless refiner_on_gpu."""
        from .h3t import H3TFile

        f = H3TFile(path)
        try:
            c = f.cfg
            if kw.get("block_config") is None:
                kw["block_config"] = BlockConfig(hidden=c.hidden, heads=c.heads, head_dim=c.head_dim, ffn=c.ffn,
                                                 act="swiglu", norm_eps=c.norm_eps, qk_norm_eps=c.qk_norm_eps,
                                                 rope_freqs=c.rope_inv_freq_len)
            dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
            glob = None
            if whole_model and f.has_globals():
                glob = f.load_globals(dev, refiner_device=dev if refiner_on_gpu else "cpu")
            elif whole_model is True:
                raise ValueError(f"{path}: no global tensors, so no whole-model forward (whole_model=True)")
            if load_pinned is None:
                load_pinned = dev.type == "cuda"
            if load_pinned:
                store = HostBlockStore.from_h3t(f, pinned=True)
                if glob is not None and not refiner_on_gpu:  # the refiner's mapping views die with the file
                    glob.refiner = [type(b)(**{k: _host_copy(v) for k, v in vars(b).items()}) for b in glob.refiner]
                    glob.refiner_final_norm = _host_copy(glob.refiner_final_norm)
                f.close()
            else:
                store = f
            return cls.from_store(store, str(dev), owns_store=True, glob=glob, model_cfg=c, whole_model=whole_model, **kw)
        except BaseException:
            f.close()
            raise

    @classmethod
    def from_store(cls, store, device: Optional[str] = None, *, block_config: Optional[BlockConfig] = None,
                   owns_store: bool = False, resident="auto", precision: str = "a8", backend: str = "auto",
                   reserve_gb: float = 1.5, free_vram_bytes: Optional[int] = None, prefetch: int = 2, ring: int = 3,
                   pin="auto", pin_mode: str = "auto", mlp_chunk: Optional[int] = None, attn_chunk: Optional[int] = None,
                   quant_mode: str = "ck", glob: Optional[GlobalWeights] = None, model_cfg=None, whole_model="auto",
                   refiner_on_gpu: bool = False, **model_kw) -> "H3Engine":
        """Provider + block runner (+ the whole model when global weights are at hand) over an open store
        (h3turbo/h3/engine.py:46-65).  free_vram_bytes overrides the measured free HBM (a host application hands the
        engine a budget); reserve_gb is still kept for activations.  glob / model_cfg: the model's global weights and
        H3Config; by default taken from the store when it has them (an H3TFile).  model_kw go to H3Model."""
        dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
        c = getattr(store, "cfg", None)
        if block_config is None and c is not None:  # the store's H3 block (SwiGLU MLP)
            block_config = BlockConfig(hidden=c.hidden, heads=c.heads, head_dim=c.head_dim, ffn=c.ffn, act="swiglu",
                                       norm_eps=c.norm_eps, qk_norm_eps=c.qk_norm_eps, rope_freqs=c.rope_inv_freq_len)
        cfg = block_config or BlockConfig()
        if whole_model and glob is None and hasattr(store, "has_globals") and store.has_globals():
            glob = store.load_globals(dev, refiner_device=dev if refiner_on_gpu else "cpu")
            model_cfg = model_cfg or store.cfg
        blk = DiTBlock(cfg, backend=backend, precision=precision, quant_mode=quant_mode, mlp_chunk=mlp_chunk,
                       attn_chunk=attn_chunk)
        provider = StreamingProvider(store, dev, resident=resident, prefetch=prefetch, pin=pin, pin_mode=pin_mode,
                                     ring=ring, reserve_bytes=int(reserve_gb * _GIB), free_vram_bytes=free_vram_bytes)
        model, why = None, None
        if glob is None:
            why = "the store holds no global tensors (patch projections, AdaLN table, refiner, output heads)"
        else:
            try:
                model = H3Model(model_cfg, glob, provider, device=dev, backend=backend, precision=precision,
                                mlp_chunk=mlp_chunk, attn_chunk=attn_chunk, quant_mode=quant_mode, **model_kw)
            except (ValueError, NotImplementedError) as e:
                if whole_model is True:
                    provider.close()
                    raise
                why = f"the file's model is not runnable here: {e}"
        return cls(store, provider, blk, owns_store, model, why)

    # -------------------------------------------------------------------------------------------- whole model
    def _need_model(self) -> H3Model:
        if self.model is None:
            raise RuntimeError(f"no whole-model forward on this engine: {self._model_error}")
        return self.model

    def encode_text(self, text_states: torch.Tensor) -> torch.Tensor:
        """condition_proj + token refiner, once per prompt; pass the result as refined_text to every step."""
        return self._need_model().encode_text(text_states)

    @torch.inference_mode()
    def velocity(self, x: Sequence[torch.Tensor], sigma, text_states: Optional[torch.Tensor] = None,
                 **kw) -> List[torch.Tensor]:
        """One model forward (H3Model.forward)."""
        return self._need_model().forward(x, sigma, text_states, **kw)

    @torch.inference_mode()
    def sample(self, video_shape: Tuple[int, int, int], audio_len: int, text_states: torch.Tensor, *, steps: int = 8,
               seed: int = 0, payload: Optional[Mapping[str, Any]] = None, callback=None,
               video_noise: Optional[torch.Tensor] = None,
               audio_noise: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Euler sampler on each stream's own sigma schedule (video shift, audio shift) (h3turbo/h3/engine.py:76-98).
        video_shape = latent (T, H, W), audio_len = latent audio frames.  Returns fp32 (video [1, C, T, H, W],
        audio [1, Ca, 2, Ta]) latents at sigma 0."""
        m = self._need_model()
        cfg, dev = m.cfg, m.device
        g = torch.Generator("cpu").manual_seed(seed)
        t, h, w = video_shape
        xv = video_noise if video_noise is not None else torch.randn(1, cfg.video_channels, t, h, w, generator=g)
        xa = audio_noise if audio_noise is not None else torch.randn(1, cfg.audio_channels, 2, audio_len, generator=g)
        xv, xa = xv.to(dev, torch.float32), xa.to(dev, torch.float32)
        refined = m.encode_text(text_states.to(dev, m.dtype))
        sv = h3_sigmas(steps, cfg.sigma_shift_video)
        sa = time_shift_sigma(sv, cfg.sigma_shift_video, cfg.sigma_shift_audio)
        for i in range(steps):
            vv, va = m.forward([xv.to(m.dtype), xa.to(m.dtype)], sv[i], None, payload=payload, sample_sigmas=sv,
                               refined_text=refined)
            xv = xv + vv.float() * float(sv[i + 1] - sv[i])
            xa = xa + va.float() * float(sa[i + 1] - sa[i])
            if callback is not None:
                callback(i, xv, xa)
        return xv, xa

    @torch.inference_mode()
    def blocks(self, x: torch.Tensor, mods_of: Callable[[int, object], Sequence[torch.Tensor]],
               segments: Sequence[Segment], rope, layers: Optional[int] = None) -> torch.Tensor:
        """Every block over the residual x [S, hidden] (in place), weights through the provider."""
        return run_blocks(self.block, x, self.provider, layers or self.provider.n_blocks, mods_of, segments, rope)

    def linear_backend(self) -> str:
        """Which kernels run the 4-bit linears: "hip" (the gfx950 kernels of libh3k) when they can run on this
        engine's device, else "unavailable" (this build has no other W4A8 backend)."""
        ok = qlinear.available_backends()["hip"]["available"] and self.provider.device.type == "cuda"
        return "hip" if ok else "unavailable"

    def stats(self) -> Dict[str, object]:
        return self.provider.stats()

    def gpu_bytes(self) -> int:
        """Device memory held by weights: resident blocks, streaming slots and the model's resident globals."""
        total = int(self.provider.stats().get("gpu_bytes", 0))
        if self.model is not None:
            for f in dataclasses.fields(self.model.glob):
                v = getattr(self.model.glob, f.name)
                if isinstance(v, torch.Tensor) and v.device.type == "cuda":
                    total += v.numel() * v.element_size()
        return total

    def close(self) -> None:
        self.provider.close()
        if self._owns_store and hasattr(self.store, "close"):
            self.store.close()

    def __enter__(self) -> "H3Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def _host_copy(v):
    """An owned host copy of a tensor or W4A8Weight that may be a view of a file mapping."""
    if v is None:
        return None
    if isinstance(v, torch.Tensor):
        return v.clone()
    return dataclasses.replace(v, q=v.q.clone(), s_rel=v.s_rel.clone(), s_ch=v.s_ch.clone(), codebook=v.codebook.clone())
