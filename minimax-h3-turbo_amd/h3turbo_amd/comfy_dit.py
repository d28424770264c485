"""The diffusion-model object a host application (ComfyUI) drives: an .h3t file behind the streaming engine, whose
device footprint the host can grant, shrink and take back (reference comfy_h3_nodes.py:79-286).

Nothing here imports ComfyUI: the host's memory manager comes in through `MemoryHost` and comfy_h3_nodes.py plugs
ComfyUI's model_management into it.

The object moves between three states:

    EMPTY   no engine; forward() or ensure_loaded() builds one inside the granted budget
    ACTIVE  blocks in HBM: as many leading blocks resident as the budget allows, the rest through a 3-slot ring
    PARKED  no block buffers on the device; page-locked host copies and the small globals kept, so the way back
            is a host -> HBM copy of the resident blocks, not a re-read of the file

    ensure_loaded(budget)   EMPTY -> ACTIVE (build)  or  PARKED -> ACTIVE (re-upload);  ACTIVE: nothing to do
    shrink(bytes)           ACTIVE -> ACTIVE with the ring and then the top resident blocks given back
    unload()                ACTIVE -> PARKED
    close_engine()          any -> EMPTY (device and page-locked host memory freed; the file stays open)

On MI355X the whole 4-bit stack normally fits in HBM (288 GB), so the usual state is ACTIVE with every block
resident; the ring and parking matter when the host shares the card with other models.

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
MIN_BUDGET = 1 << 30  # a budget the host offers is never taken below this
RING = 3  # ring slots for the streamed blocks
ACTIVATION_RESERVE = 1 << 28  # device bytes kept for activations when the budget is planned (0.25 GiB)
CHUNK_TOKENS = 4096  # MLP chunk when an unchunked forward would not fit


class MemoryHost(Protocol):
    """What the DiT asks its host: the compute device, its free memory, and the host RAM to keep free when blocks
    leaving the GPU get page-locked copies."""

    def device(self) -> torch.device: ...

    def free_memory(self, device: torch.device) -> int: ...

    def park_headroom(self) -> int: ...


class TorchMemoryHost:
    """The host's answers taken from torch, for use outside a host application."""

    def __init__(self, device=None, park_headroom_bytes: int = (3 << 30) + (512 << 20)):
        self._device = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
        self._headroom = park_headroom_bytes

    def device(self) -> torch.device:
        return self._device

    def free_memory(self, device: torch.device) -> int:
        return int(torch.cuda.mem_get_info(device)[0]) if device.type == "cuda" else 1 << 62

    def park_headroom(self) -> int:
        return self._headroom


def _lora_stub() -> torch.nn.Module:
    """An empty module with a zero-element `weight`: named like a block linear, so a host's LoRA key mapping finds
    the keys and its patch call can refuse them."""
    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(torch.empty(0), requires_grad=False)
    return m


def _block_stub() -> torch.nn.Module:
    """blocks.<i>.attn.{qkv_proj,out_proj} and blocks.<i>.mlp.{fc1,fc2}, each a LoRA key stub."""
    blk, attn, mlp = torch.nn.Module(), torch.nn.Module(), torch.nn.Module()
    attn.qkv_proj, attn.out_proj = _lora_stub(), _lora_stub()
    mlp.fc1, mlp.fc2 = _lora_stub(), _lora_stub()
    blk.attn, blk.mlp = attn, mlp
    return blk


class H3TurboDiT(torch.nn.Module):
    """Stands in for the host's H3 diffusion model: the same forward signature, the engine inside, no weights of its
    own (the module tree holds only empty LoRA key stubs)."""

    def __init__(self, path: str, precision: str = "a8", resident_blocks: int = 0, mlp_chunk: int = 0,
                 attention: str = "exact", dtype: torch.dtype = torch.bfloat16, host: Optional[MemoryHost] = None):
        super().__init__()
        if attention != "exact":
            raise ValueError(f"attention {attention!r}: this build runs the exact SDPA only ('exact')")
        self.path, self.precision, self.dtype = path, precision, dtype
        self.resident_blocks, self.mlp_chunk = resident_blocks, mlp_chunk
        self.host: MemoryHost = host or TorchMemoryHost()
        self.store = H3TFile(path)
        self.cfg = cfg = self.store.cfg
        # the attributes a host reads off its diffusion model
        self.patch_size = tuple(cfg.patch)
        self.hidden_size, self.latents_dim, self.audio_latents_dim = cfg.hidden, cfg.video_channels, cfg.audio_channels
        self.sigma_shift_video, self.sigma_shift_audio = cfg.sigma_shift_video, cfg.sigma_shift_audio
        self.blocks = torch.nn.ModuleList(_block_stub() for _ in range(cfg.layers))
        self.engine: Optional[H3Engine] = None
        self._lock = threading.RLock()

    # -------------------------------------------------------------------------------------------- state
    @property
    def state(self) -> str:
        e = self.engine
        return "EMPTY" if e is None else ("PARKED" if e.provider.parked else "ACTIVE")

    def model_bytes(self) -> int:
        return int(self.store.file_size)

    def gpu_bytes(self) -> int:
        return self.engine.gpu_bytes() if self.engine is not None else 0

    def _grant(self, budget: Optional[int]) -> int:
        """Device bytes to plan into: what is free, or the host's offer (at least MIN_BUDGET, at most what is free)."""
        free = int(self.host.free_memory(self.host.device()))
        return free if budget is None else int(min(max(budget, MIN_BUDGET), free))

    def _resident_within(self, budget: int) -> int:
        if self.resident_blocks:
            return int(self.resident_blocks)
        return plan_residency(self.store, budget, ACTIVATION_RESERVE + HBM_MARGIN, RING)

    def _report(self, what: str, budget: int) -> None:
        p = self.engine.provider
        LOG.info("H3-Turbo engine %s: %d/%d blocks resident, %d ring slots, %.2f GiB on the GPU (budget %.2f GiB)",
                 what, p.resident_count, self.cfg.layers, p.ring_count, self.gpu_bytes() / 2 ** 30, budget / 2 ** 30)

    # -------------------------------------------------------------------------------------------- transitions
    def ensure_loaded(self, budget: Optional[int] = None) -> int:
        """EMPTY -> ACTIVE or PARKED -> ACTIVE inside `budget` device bytes (default: what is free now).  Returns
        the device bytes newly placed."""
        with self._lock:
            state, grant = self.state, self._grant(budget)
            if state == "ACTIVE":
                return 0
            if state == "PARKED":
                p = self.engine.provider
                held = p.device_bytes()
                p.resize(self._resident_within(grant + held), RING)
                self._report("back on the GPU", grant)
                return p.device_bytes() - held
            self.engine = H3Engine.from_store(self.store, str(self.host.device()), owns_store=False,
                                              precision=self.precision, resident=self.resident_blocks or "auto",
                                              reserve_gb=ACTIVATION_RESERVE / 2 ** 30, free_vram_bytes=grant,
                                              ring=RING, dtype=self.dtype, whole_model=True)
            self._report("loaded", grant)
            return self.gpu_bytes()

    def _resize_or_close(self, resident: int, what: str) -> int:
        """Resize to `resident` blocks and no ring; a failed resize closes the engine rather than leave device
        memory held.  Returns the device bytes freed."""
        p = self.engine.provider
        held = p.device_bytes()
        try:
            p.resize(resident, 0, ram_headroom_bytes=self.host.park_headroom())
        except Exception as err:
            LOG.warning("H3-Turbo engine: %s failed (%r); closing it", what, err)
            return self.close_engine()
        return held - p.device_bytes()

    def unload(self) -> int:
        """ACTIVE -> PARKED: free every block buffer on the device, keep the host side.  Returns the bytes freed."""
        with self._lock:
            return 0 if self.engine is None else self._resize_or_close(0, "parking")

    def shrink(self, memory_to_free: int) -> int:
        """Give back at least `memory_to_free` device bytes: the ring slots go first, then as few resident blocks
        from the top as cover the rest.  Returns the bytes freed."""
        with self._lock:
            if self.engine is None:
                return 0
            p, blk = self.engine.provider, self.store.block_nbytes
            beyond_ring = memory_to_free - p.ring_count * blk
            drop = -(-beyond_ring // blk) if beyond_ring > 0 else 0
            return self._resize_or_close(max(0, p.resident_count - drop), "shrink")

    def close_engine(self) -> int:
        """any -> EMPTY: free everything the engine holds, device and page-locked host memory."""
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
        return text_states if text_states.shape[-1] == self.hidden_size else self.engine.encode_text(text_states)

    def pick_mlp_chunk(self, x, context) -> Optional[int]:
        """The configured MLP chunk, else CHUNK_TOKENS when an unchunked forward's activations would not fit in
        three quarters of the free device memory (chunking is exact)."""
        if self.mlp_chunk:
            return self.mlp_chunk
        t, h, w = x[0].shape[2:]
        tokens = context.shape[1] + t * ((h + 1) // 2) * ((w + 1) // 2) + 2 * x[1].shape[-1]
        need = tokens * ACT_MIB_PER_TOKEN * 2 ** 20
        return CHUNK_TOKENS if need > 0.75 * self.host.free_memory(x[0].device) else None

    def forward(self, x, timestep, context, control=None, transformer_options=None, minimax_payload=None,
                denoise_mask=None, audio_denoise_mask=None, **kwargs):
        opts = transformer_options or {}
        self.ensure_loaded()
        if getattr(x, "is_nested", False):
            x = list(x.unbind())
        x = list(x)
        sigma = (timestep.flatten()[0] / 1000.0).float()  # on the timestep's device, as the host computes it
        shifts = (float(opts.get("minimax_h3_sigma_shift_video", self.sigma_shift_video)),
                  float(opts.get("minimax_h3_sigma_shift_audio", self.sigma_shift_audio)))
        # a layout the host built is not reused: the model builds (and caches) its own from the same keyframes/refs
        payload = {k: v for k, v in (minimax_payload or {}).items() if k != "layout"}
        model = self.engine.model
        model.mlp_chunk = self.pick_mlp_chunk(x, context)
        with torch.inference_mode():
            return model.forward(x, sigma, None, payload=payload, denoise_mask=denoise_mask,
                                 audio_denoise_mask=audio_denoise_mask, sample_sigmas=opts.get("sample_sigmas"),
                                 refined_text=context, shifts=shifts)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
