"""The DiT stand-in a host application (ComfyUI) drives: an .h3t file behind the streaming engine, built inside the
VRAM budget the host grants, parked or shrunk when the host wants memory back (reference comfy_h3_nodes.py:79-286).

Nothing here imports ComfyUI.  The host's memory manager comes in through `MemoryHost` (device, free device memory,
host RAM to keep free when blocks leaving the GPU get page-locked copies); comfy_h3_nodes.py plugs ComfyUI's
model_management into it.  Lifecycle:

    ensure_loaded(budget)   build the engine with as many resident blocks as the budget allows (the rest stream
                            through a 3-slot ring), or bring a parked engine back from its page-locked host copies
    unload()                park: free every block buffer on the GPU, keep the host copies and the small globals
    shrink(bytes)           give back at least `bytes`: the ring first, then resident blocks from the top
    close_engine()          free everything (GPU and page-locked host memory); the file stays open

forward() has the call signature of ComfyUI's MiniMax H3 diffusion model: timestep = sigma * 1000, context = the
refined text from preprocess_text_embeds, the payload's conditioning, denoise masks and the sampler's sigmas.
"""
from __future__ import annotations

import gc
import logging
import threading
from typing import Optional, Protocol

import torch

from .engine import H3Engine
from .h3t import H3TFile
from .stream import HBM_MARGIN, plan_residency

LOG = logging.getLogger("h3turbo_amd")
ACT_MIB_PER_TOKEN = 0.18  # activation peak of an unchunked forward, MiB per token (bf16)
MIN_BUDGET = 1 << 30  # never plan the weights into less than this when the host offers an amount
RING = 3


class MemoryHost(Protocol):
    def device(self) -> torch.device: ...

    def free_memory(self, device: torch.device) -> int: ...

    def park_headroom(self) -> int: ...


class TorchMemoryHost:
    """Memory queries straight from torch, for use outside a host application."""

    def __init__(self, device=None, park_headroom_bytes: int = (3 << 30) + (512 << 20)):
        self._dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
        self._headroom = park_headroom_bytes

    def device(self) -> torch.device:
        return self._dev

    def free_memory(self, device: torch.device) -> int:
        if device.type == "cuda":
            return int(torch.cuda.mem_get_info(device)[0])
        return 1 << 62

    def park_headroom(self) -> int:
        return self._headroom


class _LoraKeyStub(torch.nn.Module):
    """Zero-element parameter named like a block linear, so a host's LoRA key mapping finds the keys and its patch
    call can refuse them."""

    def __init__(self):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.empty(0), requires_grad=False)


class _Attn(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.qkv_proj, self.out_proj = _LoraKeyStub(), _LoraKeyStub()


class _Mlp(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1, self.fc2 = _LoraKeyStub(), _LoraKeyStub()


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.attn, self.mlp = _Attn(), _Mlp()


class H3TurboDiT(torch.nn.Module):
    """Stands in for the host's H3 diffusion model: same forward signature, the engine inside, no weights of its own."""

    def __init__(self, path: str, precision: str = "a8", resident_blocks: int = 0, mlp_chunk: int = 0,
                 attention: str = "exact", dtype: torch.dtype = torch.bfloat16, host: Optional[MemoryHost] = None):
        super().__init__()
        if attention != "exact":
            raise ValueError(f"attention {attention!r}: this build runs the exact SDPA only ('exact')")
        self.path, self.precision, self.resident_blocks, self.mlp_chunk = path, precision, resident_blocks, mlp_chunk
        self.host = host or TorchMemoryHost()
        self.store = H3TFile(path)
        cfg = self.store.cfg
        self.cfg, self.dtype = cfg, dtype
        self.patch_size = tuple(cfg.patch)
        self.hidden_size, self.latents_dim, self.audio_latents_dim = cfg.hidden, cfg.video_channels, cfg.audio_channels
        self.sigma_shift_video, self.sigma_shift_audio = cfg.sigma_shift_video, cfg.sigma_shift_audio
        self.blocks = torch.nn.ModuleList([_Block() for _ in range(cfg.layers)])
        self.engine: Optional[H3Engine] = None
        self._lock = threading.RLock()

    # -------------------------------------------------------------------------------------------- engine lifecycle
    def model_bytes(self) -> int:
        return int(self.store.file_size)

    def gpu_bytes(self) -> int:
        e = self.engine
        return e.gpu_bytes() if e is not None else 0

    def _resident_for(self, budget: int) -> int:
        if self.resident_blocks:
            return int(self.resident_blocks)
        return plan_residency(self.store, budget, int(0.25 * 2 ** 30) + HBM_MARGIN, RING)

    def ensure_loaded(self, budget: Optional[int] = None) -> int:
        """Build the engine inside `budget` bytes of device memory (default: what is free now), or bring a parked
        engine back onto the GPU.  Returns the bytes newly placed on the device."""
        with self._lock:
            dev = self.host.device()
            free = int(self.host.free_memory(dev))
            budget = free if budget is None else int(min(max(budget, MIN_BUDGET), free))
            if self.engine is not None:
                p = self.engine.provider
                if not p.parked:
                    return 0
                before = p.device_bytes()
                p.resize(self._resident_for(budget + before), RING)
                st = p.stats()
                LOG.info("H3-Turbo engine back on the GPU: %d/%d blocks resident, %d streamed (budget %.2f GiB)",
                         st.get("resident", 0), self.cfg.layers, st.get("streamed", 0), budget / 2 ** 30)
                return p.device_bytes() - before
            e = H3Engine.from_store(self.store, str(dev), owns_store=False, precision=self.precision,
                                    resident=self.resident_blocks or "auto", reserve_gb=0.25, free_vram_bytes=budget,
                                    ring=RING, dtype=self.dtype, whole_model=True)
            self.engine = e
            st = e.stats()
            LOG.info("H3-Turbo engine loaded: %d/%d blocks resident, %d streamed, %.2f GiB on the GPU (budget %.2f GiB)",
                     st.get("resident", 0), self.cfg.layers, st.get("streamed", 0), e.gpu_bytes() / 2 ** 30,
                     budget / 2 ** 30)
            return e.gpu_bytes()

    def unload(self) -> int:
        """Park the engine: free its block buffers on the device, keep the host side and the globals, so the next
        run re-uploads from RAM.  Returns the device bytes freed."""
        with self._lock:
            e = self.engine
            if e is None:
                return 0
            before = e.provider.device_bytes()
            try:
                e.provider.resize(0, 0, ram_headroom_bytes=self.host.park_headroom())
            except Exception as err:  # never leave device memory held because parking failed
                LOG.warning("H3-Turbo engine: parking failed (%r); closing it", err)
                return self.close_engine()
            return before - e.provider.device_bytes()

    def shrink(self, memory_to_free: int) -> int:
        """Give back at least `memory_to_free` bytes of device memory: the streaming ring first, then resident
        blocks from the top; the rest stays for the next run.  Returns the device bytes freed."""
        with self._lock:
            e = self.engine
            if e is None:
                return 0
            p, blk = e.provider, self.store.block_nbytes
            before, ring_bytes, r = p.device_bytes(), len(p._slots) * blk, len(p._resident)
            keep = r if memory_to_free <= ring_bytes else max(0, r - -(-(memory_to_free - ring_bytes) // blk))
            try:
                p.resize(keep, 0, ram_headroom_bytes=self.host.park_headroom())
            except Exception as err:
                LOG.warning("H3-Turbo engine: shrink failed (%r); closing it", err)
                return self.close_engine()
            return before - p.device_bytes()

    def close_engine(self) -> int:
        """Free everything the engine holds (device and page-locked host memory); the file stays mapped."""
        with self._lock:
            e, self.engine = self.engine, None
            if e is None:
                return 0
            freed = e.gpu_bytes()
            e.close()
            del e
        gc.collect()
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        return freed

    def close(self) -> None:
        self.close_engine()
        self.store.close()

    # -------------------------------------------------------------------------------------------- sampler calls
    def preprocess_text_embeds(self, text_states: torch.Tensor) -> torch.Tensor:
        """[1, L, text_dim] encoder states -> [1, L, hidden] (condition_proj + token refiner), once per run."""
        self.ensure_loaded()
        if text_states.shape[-1] == self.hidden_size:
            return text_states
        return self.engine.encode_text(text_states)

    def pick_mlp_chunk(self, x, context) -> Optional[int]:
        """The configured MLP chunk, else 4096 tokens when an unchunked forward's activations would not fit in
        three quarters of the free device memory (chunking is exact)."""
        if self.mlp_chunk:
            return self.mlp_chunk
        t, h, w = x[0].shape[2:]
        tokens = context.shape[1] + t * ((h + 1) // 2) * ((w + 1) // 2) + 2 * x[1].shape[-1]
        free = self.host.free_memory(x[0].device)
        return 4096 if tokens * ACT_MIB_PER_TOKEN * 2 ** 20 > 0.75 * free else None

    def forward(self, x, timestep, context, control=None, transformer_options=None, minimax_payload=None,
                denoise_mask=None, audio_denoise_mask=None, **kwargs):
        to = transformer_options or {}
        self.ensure_loaded()
        if getattr(x, "is_nested", False):
            x = list(x.unbind())
        sigma = (timestep.flatten()[0] / 1000.0).float()  # on the timestep's device, as the host computes it
        shifts = (float(to.get("minimax_h3_sigma_shift_video", self.sigma_shift_video)),
                  float(to.get("minimax_h3_sigma_shift_audio", self.sigma_shift_audio)))
        # a host-built layout is dropped: the model builds (and caches) its own from the same keyframes / refs
        payload = {k: v for k, v in (minimax_payload or {}).items() if k != "layout"}
        model = self.engine.model
        model.mlp_chunk = self.pick_mlp_chunk(x, context)
        with torch.inference_mode():
            return model.forward(list(x), sigma, None, payload=payload, denoise_mask=denoise_mask,
                                 audio_denoise_mask=audio_denoise_mask, sample_sigmas=to.get("sample_sigmas"),
                                 refined_text=context, shifts=shifts)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
