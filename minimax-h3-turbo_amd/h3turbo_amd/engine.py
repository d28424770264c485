"""Engine façade over a block store: streaming provider + DiT block runner (the API surface of the reference's
H3Engine, h3turbo/h3/engine.py:29-132, restricted to the block stack).

The reference engine also embeds the inputs, runs the token refiner, the output heads and an Euler sampler; those
whole-model parts are not part of this build.  What it keeps is the part on the hot path: building the provider
with the same options (from_store, from_h3t), running the block loop over it (blocks), and the introspection
calls (linear_backend, stats, gpu_bytes, close).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Sequence

import torch

from . import qlinear
from .block import BlockConfig, DiTBlock, Segment, run_blocks
from .blockstore import HostBlockStore
from .stream import StreamingProvider

_GIB = 1 << 30


class H3Engine:
    def __init__(self, store, provider: StreamingProvider, block: DiTBlock, owns_store: bool = False):
        self.store, self.provider, self.block, self._owns_store = store, provider, block, owns_store
        self.cfg = block.cfg

    @classmethod
    def from_h3t(cls, path, device: Optional[str] = None, *, load_pinned: Optional[bool] = None, **kw) -> "H3Engine":
        """Open an .h3t file and build an engine over its blocks (h3turbo/h3/engine.py:33-44).  The block config
        comes from the file's H3Config (the H3 block: SwiGLU MLP).  load_pinned (default: on a GPU) first copies
        every block into page-locked host memory, so the streamed blocks reach HBM as direct DMA transfers; with
        False the engine streams from the file mapping through its staging buffers."""
        from .h3t import H3TFile

        f = H3TFile(path)
        try:
            c = f.cfg
            if kw.get("block_config") is None:
                kw["block_config"] = BlockConfig(hidden=c.hidden, heads=c.heads, head_dim=c.head_dim, ffn=c.ffn,
                                                 act="swiglu", norm_eps=c.norm_eps, qk_norm_eps=c.qk_norm_eps,
                                                 rope_freqs=c.rope_inv_freq_len)
            dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
            if load_pinned is None:
                load_pinned = dev.type == "cuda"
            if load_pinned:
                store = HostBlockStore.from_h3t(f, pinned=True)
                f.close()
            else:
                store = f
            return cls.from_store(store, str(dev), owns_store=True, **kw)
        except BaseException:
            f.close()
            raise

    @classmethod
    def from_store(cls, store, device: Optional[str] = None, *, block_config: Optional[BlockConfig] = None,
                   owns_store: bool = False, resident="auto", precision: str = "a8", backend: str = "auto",
                   reserve_gb: float = 1.5, free_vram_bytes: Optional[int] = None, prefetch: int = 2, ring: int = 3,
                   pin="auto", pin_mode: str = "auto", mlp_chunk: Optional[int] = None, attn_chunk: Optional[int] = None,
                   quant_mode: str = "ck") -> "H3Engine":
        """Provider + block runner over an open store (h3turbo/h3/engine.py:46-65).  free_vram_bytes overrides the
        measured free HBM (a host application hands the engine a budget); reserve_gb is still kept for activations."""
        dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
        cfg = block_config or BlockConfig()
        blk = DiTBlock(cfg, backend=backend, precision=precision, quant_mode=quant_mode, mlp_chunk=mlp_chunk,
                       attn_chunk=attn_chunk)
        provider = StreamingProvider(store, dev, resident=resident, prefetch=prefetch, pin=pin, pin_mode=pin_mode,
                                     ring=ring, reserve_bytes=int(reserve_gb * _GIB), free_vram_bytes=free_vram_bytes)
        return cls(store, provider, blk, owns_store)

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
        """Device memory held by weights: resident blocks plus streaming slots."""
        return int(self.provider.stats().get("gpu_bytes", 0))

    def close(self) -> None:
        self.provider.close()
        if self._owns_store and hasattr(self.store, "close"):
            self.store.close()

    def __enter__(self) -> "H3Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
