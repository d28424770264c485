"""Block-contiguous host storage of DiT block weights, and zero-copy typed views of one block's bytes.

The streaming engine moves a block as ONE contiguous byte range (host -> HBM) and then reads its tensors as typed
views of the device buffer.  That needs a layout that is identical for every block: each tensor at a fixed byte
offset, 256-byte aligned (16-byte vector loads and the kernels' alignment rules hold with a wide margin), and each
block a multiple of 4 KiB (page granular).  These are the alignment rules of the reference's .h3t container
(h3turbo/h3/store.py:39-40) and its block views (store.py:155-178, 289-320).

Tensor names follow the reference's checkpoint layout inside a block:
    attn.qkv_proj.weight[_s_rel|_s_channel|_codebook], attn.out_proj.*, mlp.fc1.*, mlp.fc2.*,
    norm1.weight, norm2.weight, attn.q_norm.weight, attn.k_norm.weight, adaln_proj.linear.{weight,bias}
A linear with a `.weight_codebook` entry is W4A8; without one, `.weight` is a dense matrix.

HostBlockStore keeps all blocks in one host allocation, optionally page-locked (allocated pinned, so host -> HBM
copies are DMA transfers straight from it; on this platform memory is page-locked by allocating it pinned, never
by registering existing pages).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np
import torch

from .types import BlockWeights, W4A8Weight, Weight

TENSOR_ALIGN = 256
BLOCK_ALIGN = 4096
LINEARS = ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")
_FIELD = {"attn.qkv_proj": "qkv", "attn.out_proj": "out", "mlp.fc1": "fc1", "mlp.fc2": "fc2"}


def _round_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


@dataclass(frozen=True)
class LayoutEntry:
    name: str
    dtype: torch.dtype
    shape: Tuple[int, ...]
    offset: int
    nbytes: int


class BlockLayout:
    """Byte layout shared by every block: name -> (dtype, shape, offset), tensors 256-B aligned, size 4 KiB-rounded."""

    def __init__(self, entries: Sequence[LayoutEntry]):
        self.entries = list(entries)
        self._by_name = {e.name: e for e in self.entries}
        end = max((e.offset + e.nbytes for e in self.entries), default=0)
        self.nbytes = _round_up(max(end, 1), BLOCK_ALIGN)
        for e in self.entries:
            if e.offset % TENSOR_ALIGN:
                raise ValueError(f"{e.name}: offset {e.offset} is not {TENSOR_ALIGN}-byte aligned")

    @classmethod
    def of(cls, tensors: Mapping[str, torch.Tensor]) -> "BlockLayout":
        """Pack tensors in the given order, each at the next 256-byte boundary."""
        entries, off = [], 0
        for name, t in tensors.items():
            nb = t.numel() * t.element_size()
            entries.append(LayoutEntry(name, t.dtype, tuple(t.shape), off, nb))
            off = _round_up(off + nb, TENSOR_ALIGN)
        return cls(entries)

    def __contains__(self, name: str) -> bool:
        return name in self._by_name

    def names(self) -> List[str]:
        return [e.name for e in self.entries]

    def view(self, buf: torch.Tensor, name: str) -> torch.Tensor:
        """Zero-copy typed view of tensor `name` inside a block buffer (1-D uint8, any device)."""
        e = self._by_name[name]
        v = buf[e.offset:e.offset + e.nbytes]
        if e.dtype != torch.uint8:
            v = v.view(e.dtype)
        return v.view(e.shape)

    def pack_into(self, buf: torch.Tensor, tensors: Mapping[str, torch.Tensor]) -> None:
        """Write one block's tensors into `buf` (1-D uint8 of nbytes) at their offsets; gaps are zeroed."""
        if set(tensors) != set(self._by_name):
            raise ValueError(f"block tensors {sorted(tensors)} do not match the layout {sorted(self._by_name)}")
        buf.zero_()
        for e in self.entries:
            t = tensors[e.name]
            if t.dtype != e.dtype or tuple(t.shape) != e.shape:
                raise ValueError(f"{e.name}: got {t.dtype} {tuple(t.shape)}, layout has {e.dtype} {e.shape}")
            self.view(buf, e.name).copy_(t)

    def block_weights(self, buf: torch.Tensor, group: int, convrot: int) -> BlockWeights:
        """BlockWeights of zero-copy views into `buf` (the reference's build_block_weights, store.py:164-178)."""
        if buf.dtype != torch.uint8 or buf.dim() != 1 or buf.numel() != self.nbytes:
            raise ValueError(f"expected a 1-D uint8 buffer of {self.nbytes} bytes, got {tuple(buf.shape)} {buf.dtype}")

        def lin(prefix: str) -> Weight:
            if f"{prefix}.weight_codebook" in self:
                return W4A8Weight(self.view(buf, f"{prefix}.weight"), self.view(buf, f"{prefix}.weight_s_rel"),
                                  self.view(buf, f"{prefix}.weight_s_channel"),
                                  self.view(buf, f"{prefix}.weight_codebook"), group, convrot)
            return self.view(buf, f"{prefix}.weight")

        opt = lambda n: self.view(buf, n) if n in self else None  # noqa: E731
        return BlockWeights(qkv=lin("attn.qkv_proj"), out=lin("attn.out_proj"), fc1=lin("mlp.fc1"), fc2=lin("mlp.fc2"),
                            norm1=self.view(buf, "norm1.weight"), norm2=self.view(buf, "norm2.weight"),
                            q_norm=self.view(buf, "attn.q_norm.weight"), k_norm=self.view(buf, "attn.k_norm.weight"),
                            adaln_w=opt("adaln_proj.linear.weight"), adaln_b=opt("adaln_proj.linear.bias"))


def block_tensors(w: BlockWeights) -> Dict[str, torch.Tensor]:
    """The named tensors of one block (CPU), in layout order: the inverse of BlockLayout.block_weights."""
    out: Dict[str, torch.Tensor] = {}
    for prefix in LINEARS:
        lw = getattr(w, _FIELD[prefix])
        if isinstance(lw, W4A8Weight):
            out[f"{prefix}.weight"] = lw.q
            out[f"{prefix}.weight_s_rel"] = lw.s_rel
            out[f"{prefix}.weight_s_channel"] = lw.s_ch
            out[f"{prefix}.weight_codebook"] = lw.codebook
        else:
            out[f"{prefix}.weight"] = lw
    for name, t in (("norm1.weight", w.norm1), ("norm2.weight", w.norm2), ("attn.q_norm.weight", w.q_norm),
                    ("attn.k_norm.weight", w.k_norm), ("adaln_proj.linear.weight", w.adaln_w),
                    ("adaln_proj.linear.bias", w.adaln_b)):
        if t is not None:
            out[name] = t
    return {k: v.detach().cpu().contiguous() for k, v in out.items()}


class HostBlockStore:
    """n_blocks blocks of one layout in one host allocation: block i occupies bytes [i * block_nbytes, ...).

    The BlockProvider source the streaming engine reads: block_nbytes, n_blocks, block_tensor(i) (uint8 view, the
    copy source), block_bytes(i) (numpy view), block_weights_from(buf) and block_weights_cpu(i).
    pinned=True allocates the backing page-locked, so every block is a DMA-ready source without a second copy.
    """

    def __init__(self, layout: BlockLayout, n_blocks: int, group: int, convrot: int, *, pinned: bool = False):
        if n_blocks < 0:
            raise ValueError("n_blocks must be >= 0")
        self.layout, self.n_blocks, self.group, self.convrot = layout, n_blocks, group, convrot
        self.block_nbytes = layout.nbytes
        total = max(1, n_blocks * self.block_nbytes)
        self.pinned = bool(pinned)
        self._u8 = torch.empty(total, dtype=torch.uint8, pin_memory=self.pinned)
        self._np = self._u8.numpy()

    @classmethod
    def from_blocks(cls, blocks: Sequence[BlockWeights], *, pinned: bool = False) -> "HostBlockStore":
        """Pack BlockWeights (W4A8 linears share group/convrot) into a new store."""
        if not blocks:
            raise ValueError("no blocks")
        first = block_tensors(blocks[0])
        lw = next((getattr(blocks[0], f) for f in ("qkv", "out", "fc1", "fc2") if isinstance(getattr(blocks[0], f), W4A8Weight)), None)
        group, convrot = (lw.group_size, lw.convrot) if lw is not None else (16, 256)
        st = cls(BlockLayout.of(first), len(blocks), group, convrot, pinned=pinned)
        for i, b in enumerate(blocks):
            st.write_block(i, first if i == 0 else block_tensors(b))
        return st

    @classmethod
    def from_h3t(cls, f, *, pinned: bool = False) -> "HostBlockStore":
        """Copy every block of an open .h3t file (h3t.H3TFile) into a new store with the file's block layout, so the
        blocks become DMA-ready host memory (pinned=True) instead of pageable file pages."""
        from .h3t import torch_dtype

        layout = BlockLayout([LayoutEntry(e.name, torch_dtype(e.dtype), tuple(e.shape), e.offset, e.nbytes)
                              for e in f.block_layout])
        if layout.nbytes != f.block_nbytes:
            raise ValueError(f"{f.path}: block layout spans {layout.nbytes} bytes, the file's blocks are {f.block_nbytes}")
        st = cls(layout, f.n_blocks, f.quant_group, f.quant_convrot, pinned=pinned)
        for i in range(f.n_blocks):
            np.copyto(st.block_bytes(i), f.block_bytes(i))
        return st

    def _check(self, i: int) -> None:
        if not 0 <= i < self.n_blocks:
            raise IndexError(f"block {i} out of range [0, {self.n_blocks})")

    def write_block(self, i: int, tensors: Mapping[str, torch.Tensor]) -> None:
        self._check(i)
        self.layout.pack_into(self.block_tensor(i), tensors)

    def block_tensor(self, i: int) -> torch.Tensor:
        self._check(i)
        return self._u8[i * self.block_nbytes:(i + 1) * self.block_nbytes]

    def block_bytes(self, i: int) -> np.ndarray:
        self._check(i)
        return self._np[i * self.block_nbytes:(i + 1) * self.block_nbytes]

    def block_weights_from(self, buf: torch.Tensor) -> BlockWeights:
        return self.layout.block_weights(buf, self.group, self.convrot)

    def block_weights_cpu(self, i: int) -> BlockWeights:
        return self.block_weights_from(self.block_tensor(i))

    @property
    def nbytes(self) -> int:
        return self.n_blocks * self.block_nbytes
