""".h3t: the block-contiguous safetensors container the weight-streaming engine reads (h3turbo/h3/store.py,
h3turbo/h3/writer.py).

An .h3t file is a valid safetensors file whose tensors are ordered globals first, then block 0 .. N-1.  Every
block is one BLOCK_ALIGN-aligned byte range with the same tensor layout in every block, every tensor starts on a
TENSOR_ALIGN boundary, and the gaps are explicit `__pad.<i>` U8 tensors (safetensors has no holes).  The
metadata carries the format tag, the H3Config JSON, the block size / start / ranges and the block layout.  This
module writes byte-identical files to the reference writer for the same tensors and reads the reference's files.

On MI355X the reader is the host side of the streaming engine: `H3TFile` maps the file read-only and hands out
zero-copy views (`block_tensor(i)`, a block's raw bytes; `block_weights_from(buf)`, typed views of a block held in
any buffer, e.g. an HBM slot).  `blockstore.HostBlockStore.from_h3t` copies the blocks into pinned host memory,
so each block then reaches HBM as one DMA transfer.
"""
from __future__ import annotations

import json
import math
import mmap
import os
import re
import struct
import sys
import warnings
from typing import Callable, Dict, Iterable, Iterator, List, Mapping, NamedTuple, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .config import H3Config
from .types import BlockWeights, GlobalWeights, W4A8Weight, Weight

if sys.byteorder != "little":  # pragma: no cover - safetensors data is little-endian
    raise ImportError(".h3t files are little-endian; big-endian hosts are unsupported")

FORMAT = "h3turbo-h3"
VERSION = 1
TENSOR_ALIGN = 256
BLOCK_ALIGN = 4096
PAD_PREFIX = "__pad."
_HEADER_CAP = 100_000_000

# safetensors dtype name -> (torch dtype, bytes per element)
_DT: Dict[str, Tuple[torch.dtype, int]] = {
    "F64": (torch.float64, 8), "F32": (torch.float32, 4), "F16": (torch.float16, 2), "BF16": (torch.bfloat16, 2),
    "I64": (torch.int64, 8), "I32": (torch.int32, 4), "I16": (torch.int16, 2), "I8": (torch.int8, 1),
    "U8": (torch.uint8, 1), "BOOL": (torch.bool, 1), "F8_E4M3": (torch.float8_e4m3fn, 1),
    "F8_E5M2": (torch.float8_e5m2, 1),
}
_NAME_OF = {t: name for name, (t, _) in _DT.items()}

# The W4A8 linears of a block and the tensors each one carries (the checkpoint's naming).
LINEARS = ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")
QUANT_PARTS = ("weight", "weight_s_rel", "weight_s_channel", "weight_codebook", "comfy_quant")
# Canonical tensor order inside a block and among the globals; anything else follows sorted by name.  The order
# decides every offset, so it is part of the format (the reference writer uses the same order).
BLOCK_ORDER = ("adaln_proj.linear.weight", "adaln_proj.linear.bias", "norm1.weight", "attn.q_norm.weight",
               "attn.k_norm.weight", *(f"attn.qkv_proj.{p}" for p in QUANT_PARTS),
               *(f"attn.out_proj.{p}" for p in QUANT_PARTS), "norm2.weight", *(f"mlp.fc1.{p}" for p in QUANT_PARTS),
               *(f"mlp.fc2.{p}" for p in QUANT_PARTS))
GLOBAL_ORDER = ("video_patch_proj.weight", "video_patch_proj.bias", "audio_patch_proj.weight", "audio_patch_proj.bias",
                "condition_proj.weight", "condition_proj.bias", "adaln_t_table", "rope.inv_freq",
                "final_layer.norm.weight", "final_layer.adaln_proj.linear.weight", "final_layer.adaln_proj.linear.bias",
                "final_layer.video_out.weight", "final_layer.video_out.bias", "final_layer.audio_out.weight",
                "final_layer.audio_out.bias")
_BLOCK_NAME = re.compile(r"^blocks\.(\d+)\.(.+)$")
_REFINER_NAME = re.compile(r"^token_refiner\.blocks\.(\d+)\.(.+)$")


class H3TError(ValueError):
    """Not a valid .h3t container, or an inconsistent write request."""


def itemsize(dtype: str) -> int:
    if dtype not in _DT:
        raise H3TError(f"unsupported safetensors dtype {dtype!r}")
    return _DT[dtype][1]


def torch_dtype(dtype: str) -> torch.dtype:
    itemsize(dtype)
    return _DT[dtype][0]


def st_dtype(t: torch.dtype) -> str:
    if t not in _NAME_OF:
        raise H3TError(f"torch dtype {t} has no safetensors name")
    return _NAME_OF[t]


def nbytes_of(dtype: str, shape: Sequence[int]) -> int:
    return math.prod(shape) * itemsize(dtype)


def _up(v: int, a: int) -> int:
    return -(-v // a) * a


# ------------------------------------------------------------------------------------------------ safetensors header
class Header(NamedTuple):
    tensors: Dict[str, dict]  # name -> {"dtype", "shape", "data_offsets"} (offsets from the data section start)
    meta: Dict[str, str]
    data_start: int
    file_size: int
    raw: bytes


def read_header(path: Union[str, os.PathLike]) -> Header:
    """The safetensors header of `path`, checked against the file: every entry inside the data section, byte counts
    matching dtype x shape.  Tensor data is not read."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        lead = f.read(8)
        if len(lead) < 8:
            raise H3TError(f"{path}: {size} bytes is too small for a safetensors file")
        (n,) = struct.unpack("<Q", lead)
        if n > _HEADER_CAP or 8 + n > size:
            raise H3TError(f"{path}: header size {n} does not fit the {size}-byte file")
        raw = f.read(n)
    if not raw.lstrip(b" ").startswith(b"{"):
        raise H3TError(f"{path}: the safetensors header is not a JSON object")
    try:
        table = json.loads(raw)
    except ValueError as e:
        raise H3TError(f"{path}: the safetensors header is not valid JSON: {e}") from None
    if not isinstance(table, dict):
        raise H3TError(f"{path}: the safetensors header is not a JSON object")
    meta = table.pop("__metadata__", None) or {}
    data_len = size - 8 - n
    for name, e in table.items():
        try:
            a, b = e["data_offsets"]
            dtype, shape = e["dtype"], e["shape"]
        except (KeyError, TypeError, ValueError):
            raise H3TError(f"{path}: header entry {name!r} is malformed") from None
        if not 0 <= a <= b <= data_len:
            raise H3TError(f"{path}: {name!r} spans [{a}, {b}), outside the {data_len}-byte data section "
                           "(truncated file?)")
        if dtype in _DT and b - a != nbytes_of(dtype, shape):
            raise H3TError(f"{path}: {name!r} holds {b - a} bytes, {dtype}{list(shape)} needs {nbytes_of(dtype, shape)}")
    return Header(table, meta, 8 + n, size, raw)


class BlockEntry(NamedTuple):
    name: str  # relative to the block
    dtype: str
    shape: Tuple[int, ...]
    offset: int  # from the block start
    nbytes: int


class TensorInfo(NamedTuple):
    dtype: str
    shape: Tuple[int, ...]
    start: int  # absolute file offset
    nbytes: int


def quant_linear_names(names: Iterable[str]) -> List[str]:
    """The W4A8 linears (prefixes) present among a block's tensor names: those with a codebook."""
    have = set(names)
    return [p for p in LINEARS if f"{p}.weight_codebook" in have]


def typed_view(buf: torch.Tensor, offset: int, dtype: str, shape: Sequence[int]) -> torch.Tensor:
    """Zero-copy `dtype[shape]` view at byte `offset` of a 1-D uint8 tensor (any device)."""
    v = buf[offset:offset + nbytes_of(dtype, shape)]
    t = torch_dtype(dtype)
    return (v if t is torch.uint8 else v.view(t)).view(tuple(shape))


def build_block_weights(get: Callable[[str], torch.Tensor], has: Callable[[str], bool], group: int, convrot: int,
                        adaln: bool = True) -> BlockWeights:
    """BlockWeights from a block-relative name accessor: a linear with a codebook is W4A8, else dense."""

    def linear(p: str) -> Weight:
        if has(f"{p}.weight_codebook"):
            return W4A8Weight(get(f"{p}.weight"), get(f"{p}.weight_s_rel"), get(f"{p}.weight_s_channel"),
                              get(f"{p}.weight_codebook"), group, convrot)
        return get(f"{p}.weight")

    mod = adaln and has("adaln_proj.linear.weight")
    return BlockWeights(qkv=linear("attn.qkv_proj"), out=linear("attn.out_proj"), fc1=linear("mlp.fc1"),
                        fc2=linear("mlp.fc2"), norm1=get("norm1.weight"), norm2=get("norm2.weight"),
                        q_norm=get("attn.q_norm.weight"), k_norm=get("attn.k_norm.weight"),
                        adaln_w=get("adaln_proj.linear.weight") if mod else None,
                        adaln_b=get("adaln_proj.linear.bias") if mod else None)


_GLOBALS_NEEDED = ("video_patch_proj.weight", "video_patch_proj.bias", "audio_patch_proj.weight",
                   "audio_patch_proj.bias", "condition_proj.weight", "condition_proj.bias", "rope.inv_freq",
                   "final_layer.norm.weight", "final_layer.adaln_proj.linear.weight",
                   "final_layer.adaln_proj.linear.bias", "final_layer.video_out.weight", "final_layer.video_out.bias",
                   "final_layer.audio_out.weight", "final_layer.audio_out.bias")


# ------------------------------------------------------------------------------------------------ reader
class H3TFile:
    """A read-only memory-mapped .h3t file (h3turbo/h3/store.py:182-400).  Every accessor returns a zero-copy view of
    the mapping; never write into one.  The store interface of the streaming engine: n_blocks, block_nbytes,
    block_tensor(i), block_bytes(i), block_weights_from(buf)."""

    pinned = False  # the mapping is pageable: the streaming engine stages or pins copies of its blocks

    def __init__(self, path: Union[str, os.PathLike]):
        self.path = os.fspath(path)
        hdr = read_header(self.path)
        m = hdr.meta
        if m.get("format") != FORMAT:
            raise H3TError(f"{self.path}: not an h3t file (format tag {m.get('format')!r}, expected {FORMAT!r})")
        try:
            version = int(m.get("version", "0"))
        except (TypeError, ValueError):
            version = -1
        if version != VERSION:
            raise H3TError(f"{self.path}: unsupported h3t version {m.get('version')!r} (this reader reads {VERSION})")
        try:
            self.cfg = H3Config.from_json(m["config"])
            self.n_blocks = int(m["n_blocks"])
            self.block_nbytes = int(m["block_nbytes"])
            self.blocks_start = int(m["blocks_start"])
            self.block_layout = [BlockEntry(n, d, tuple(s), int(o), int(b)) for n, d, s, o, b in json.loads(m["block_layout"])]
            self.quant = json.loads(m.get("quant") or "{}")
            self.meta = dict(m)
            self.source_name = m.get("source_name", "")
            self.source_size = int(m.get("source_size") or 0)
            self.data_start, self.file_size = hdr.data_start, hdr.file_size
            self._check(hdr)
        except H3TError:
            raise
        except (KeyError, TypeError, ValueError, IndexError) as e:
            raise H3TError(f"{self.path}: corrupt h3t metadata: {e!r}") from None
        self.quant_group = int(self.quant.get("group_size", self.cfg.quant_group))
        self.quant_convrot = int(self.quant.get("convrot_groupsize", self.cfg.quant_convrot))
        self._layout = {e.name: e for e in self.block_layout}
        self._info = {name: TensorInfo(e["dtype"], tuple(e["shape"]), self.data_start + e["data_offsets"][0],
                                       e["data_offsets"][1] - e["data_offsets"][0])
                      for name, e in hdr.tensors.items() if not name.startswith(PAD_PREFIX)}
        with open(self.path, "rb") as fh:
            self._mm: Optional[mmap.mmap] = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        self._np: Optional[np.ndarray] = np.frombuffer(self._mm, dtype=np.uint8)
        with warnings.catch_warnings():  # torch notes the buffer is read-only; nothing here writes to it
            warnings.simplefilter("ignore")
            self._u8: Optional[torch.Tensor] = torch.frombuffer(self._mm, dtype=torch.uint8)

    def _check(self, hdr: Header) -> None:
        p = self.path
        if self.n_blocks < 1 or self.n_blocks != self.cfg.layers:
            raise H3TError(f"{p}: n_blocks={self.n_blocks} but config.layers={self.cfg.layers}")
        if self.data_start % BLOCK_ALIGN or self.blocks_start % BLOCK_ALIGN or self.block_nbytes % BLOCK_ALIGN:
            raise H3TError(f"{p}: data section or block offsets are not {BLOCK_ALIGN}-byte aligned")
        need = self.data_start + self.blocks_start + self.n_blocks * self.block_nbytes
        if hdr.file_size != need:
            raise H3TError(f"{p}: the layout needs exactly {need} bytes, the file has {hdr.file_size} "
                           "(truncated, or trailing data)")
        ranges = json.loads(hdr.meta["block_ranges"])
        if not isinstance(ranges, list) or len(ranges) != self.n_blocks:
            raise H3TError(f"{p}: block_ranges does not list {self.n_blocks} blocks")
        for i, (a, b) in enumerate(ranges):
            if a != self.blocks_start + i * self.block_nbytes or b - a != self.block_nbytes:
                raise H3TError(f"{p}: block_ranges[{i}] = [{a}, {b}) disagrees with blocks_start / block_nbytes")
        for i in range(self.n_blocks):  # header entries of every block against the shared layout
            base = self.blocks_start + i * self.block_nbytes
            for e in self.block_layout:
                got = hdr.tensors.get(f"blocks.{i}.{e.name}")
                if (got is None or got["dtype"] != e.dtype or tuple(got["shape"]) != e.shape
                        or list(got["data_offsets"]) != [base + e.offset, base + e.offset + e.nbytes]):
                    raise H3TError(f"{p}: blocks.{i}.{e.name} does not match the block layout")
        pos = 0
        for name, e in sorted(hdr.tensors.items(), key=lambda kv: kv[1]["data_offsets"][0]):
            a, b = e["data_offsets"]
            if a != pos:
                raise H3TError(f"{p}: hole or overlap before {name!r}")
            if a % TENSOR_ALIGN and not name.startswith(PAD_PREFIX):
                raise H3TError(f"{p}: {name!r} starts at {a}, not {TENSOR_ALIGN}-byte aligned")
            pos = b
        if pos != hdr.file_size - self.data_start:
            raise H3TError(f"{p}: the tensors cover {pos} of the {hdr.file_size - self.data_start} data bytes")
        have = {e.name for e in self.block_layout}
        for lin in quant_linear_names(have):
            missing = [part for part in QUANT_PARTS if f"{lin}.{part}" not in have]
            if missing:
                raise H3TError(f"{p}: W4A8 linear {lin} lacks {missing}")

    def _open(self) -> None:
        if self._mm is None:
            raise ValueError("H3TFile is closed")

    # ---- raw block bytes
    def block_range(self, i: int) -> Tuple[int, int]:
        """[start, end) file offsets of block i."""
        if not 0 <= i < self.n_blocks:
            raise IndexError(f"block {i} outside [0, {self.n_blocks})")
        a = self.data_start + self.blocks_start + i * self.block_nbytes
        return a, a + self.block_nbytes

    def block_bytes(self, i: int) -> np.ndarray:
        """Read-only uint8 numpy view of block i."""
        self._open()
        a, b = self.block_range(i)
        return self._np[a:b]

    def block_tensor(self, i: int) -> torch.Tensor:
        """uint8 torch view of block i: the source of a host -> device block copy."""
        self._open()
        a, b = self.block_range(i)
        return self._u8[a:b]

    @property
    def block_layout_size(self) -> int:
        return self.block_layout[-1].offset + self.block_layout[-1].nbytes

    # ---- typed tensors
    def keys(self) -> List[str]:
        return list(self._info)

    def info(self, name: str) -> TensorInfo:
        if name not in self._info:
            raise KeyError(f"{name!r} is not in {self.path}")
        return self._info[name]

    def tensor(self, name: str) -> torch.Tensor:
        """Zero-copy CPU view of one tensor."""
        self._open()
        t = self.info(name)
        return typed_view(self._u8, t.start, t.dtype, t.shape)

    def block_weights_from(self, buf: torch.Tensor) -> BlockWeights:
        """Typed zero-copy views of a block held in `buf` (1-D uint8, block_nbytes long, any device)."""
        if buf.dtype != torch.uint8 or buf.dim() != 1 or buf.numel() != self.block_nbytes:
            raise ValueError(f"need a 1-D uint8 buffer of {self.block_nbytes} bytes, got {tuple(buf.shape)} {buf.dtype}")
        lay = self._layout
        return build_block_weights(lambda r: typed_view(buf, lay[r].offset, lay[r].dtype, lay[r].shape),
                                   lay.__contains__, self.quant_group, self.quant_convrot)

    def block_weights_cpu(self, i: int) -> BlockWeights:
        return self.block_weights_from(self.block_tensor(i))

    def load_globals(self, device="cpu", *, refiner_device=None) -> GlobalWeights:
        """GlobalWeights on `device`, the token refiner on `refiner_device` (default: the same) (reference
        h3turbo/h3/store.py:329-365).  On the CPU the globals are copies and the refiner stays zero-copy views of
        the mapping; refiner_device="cpu" keeps the refiner out of HBM until the text is encoded."""
        dev = torch.device(device)
        rdev = torch.device(refiner_device) if refiner_device is not None else dev

        def get(name: str, d: torch.device = dev, view: bool = False) -> torch.Tensor:
            t = self.tensor(name)
            if d.type != "cpu":
                return t.to(d)
            return t if view else t.clone()

        missing = [n for n in _GLOBALS_NEEDED if n not in self._info]
        if missing:
            raise H3TError(f"{self.path}: missing global tensors {missing}")
        refiner = []
        for j in range(self.cfg.refiner_layers):
            pre = f"token_refiner.blocks.{j}."
            refiner.append(build_block_weights(lambda r, pre=pre: get(pre + r, rdev, True),
                                               lambda r, pre=pre: pre + r in self._info, self.quant_group,
                                               self.quant_convrot, adaln=False))
        fnorm = "token_refiner.final_norm.weight"
        return GlobalWeights(
            video_patch_w=get("video_patch_proj.weight"), video_patch_b=get("video_patch_proj.bias"),
            audio_patch_w=get("audio_patch_proj.weight"), audio_patch_b=get("audio_patch_proj.bias"),
            condition_w=get("condition_proj.weight"), condition_b=get("condition_proj.bias"),
            adaln_t_table=get("adaln_t_table") if "adaln_t_table" in self._info else None,
            rope_inv_freq=get("rope.inv_freq"), final_norm=get("final_layer.norm.weight"),
            final_adaln_w=get("final_layer.adaln_proj.linear.weight"),
            final_adaln_b=get("final_layer.adaln_proj.linear.bias"),
            video_out_w=get("final_layer.video_out.weight"), video_out_b=get("final_layer.video_out.bias"),
            audio_out_w=get("final_layer.audio_out.weight"), audio_out_b=get("final_layer.audio_out.bias"),
            refiner=refiner, refiner_final_norm=get(fnorm, rdev, True) if fnorm in self._info else None)

    def has_globals(self) -> bool:
        """Whether the file holds every global tensor the whole-model forward needs."""
        return all(n in self._info for n in _GLOBALS_NEEDED)

    def globals_nbytes(self, refiner: bool = True) -> int:
        """Bytes of the tensors outside the blocks (the token refiner optional)."""
        return sum(t.nbytes for n, t in self._info.items()
                   if not _BLOCK_NAME.match(n) and (refiner or not n.startswith("token_refiner.")))

    # ---- lifecycle
    def close(self) -> None:
        if self._mm is None:
            return
        mm, self._mm, self._np, self._u8 = self._mm, None, None, None
        try:
            mm.close()
        except BufferError:  # views handed out are alive: the mapping goes away with the last of them
            pass

    def __enter__(self) -> "H3TFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"H3TFile({self.path!r}, blocks={self.n_blocks}, block={self.block_nbytes / 2**20:.1f} MiB)"


# ------------------------------------------------------------------------------------------------ writer
class TensorSource:
    """The little-endian bytes of one tensor, produced in chunks (a writer holds one chunk at a time)."""

    dtype: str
    shape: Tuple[int, ...]
    nbytes: int

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        raise NotImplementedError

    def read(self) -> torch.Tensor:
        data = bytearray(self.nbytes)
        pos = 0
        for c in self.chunks(32 << 20):
            data[pos:pos + len(c)] = c
            pos += len(c)
        buf = torch.frombuffer(data, dtype=torch.uint8) if self.nbytes else torch.empty(0, dtype=torch.uint8)
        return typed_view(buf, 0, self.dtype, self.shape)


class TorchSource(TensorSource):
    def __init__(self, t: torch.Tensor):
        t = t.detach().cpu().contiguous()
        self._t, self.dtype, self.shape = t, st_dtype(t.dtype), tuple(t.shape)
        self.nbytes = t.numel() * t.element_size()

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        if self.nbytes:
            mv = memoryview(self._t.reshape(-1).view(torch.uint8).numpy())
            for a in range(0, self.nbytes, chunk_bytes):
                yield mv[a:a + chunk_bytes]


class LazySource(TensorSource):
    """A tensor made by `fn()` only when it is written."""

    def __init__(self, dtype: str, shape: Sequence[int], fn: Callable[[], torch.Tensor]):
        self.dtype, self.shape, self._fn = dtype, tuple(shape), fn
        self.nbytes = nbytes_of(dtype, shape)

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        src = TorchSource(self._fn())
        if (src.dtype, src.shape) != (self.dtype, self.shape):
            raise H3TError(f"lazy tensor made {src.dtype}{src.shape}, declared {self.dtype}{self.shape}")
        yield from src.chunks(chunk_bytes)


def as_source(x: Union[TensorSource, torch.Tensor]) -> TensorSource:
    if isinstance(x, TensorSource):
        return x
    if isinstance(x, torch.Tensor):
        return TorchSource(x)
    raise TypeError(f"expected a Tensor or TensorSource, got {type(x).__name__}")


def _ordered(names: Iterable[str], first: Sequence[str]) -> List[str]:
    have = set(names)
    lead = [n for n in first if n in have]
    return lead + sorted(have.difference(lead))


def classify(names: Iterable[str]):
    """(globals, {refiner block: names}, other token_refiner.* names, {block: names}); names in blocks relative."""
    glob: List[str] = []
    refiner: Dict[int, List[str]] = {}
    refiner_other: List[str] = []
    blocks: Dict[int, List[str]] = {}
    for n in names:
        if n.startswith(PAD_PREFIX):
            raise H3TError(f"tensor {n!r} uses the reserved padding prefix {PAD_PREFIX!r}")
        m = _BLOCK_NAME.match(n)
        if m:
            blocks.setdefault(int(m.group(1)), []).append(m.group(2))
            continue
        m = _REFINER_NAME.match(n)
        if m:
            refiner.setdefault(int(m.group(1)), []).append(m.group(2))
        elif n.startswith("token_refiner."):
            refiner_other.append(n)
        else:
            glob.append(n)
    return glob, refiner, refiner_other, blocks


def _pack(items: Sequence[Tuple[str, str, Tuple[int, ...]]]) -> Tuple[List[BlockEntry], int]:
    """Each tensor at the next TENSOR_ALIGN boundary from 0, in order; returns the entries and the end offset."""
    out, pos = [], 0
    for name, dt, shape in items:
        pos = _up(pos, TENSOR_ALIGN)
        nb = nbytes_of(dt, shape)
        out.append(BlockEntry(name, dt, tuple(shape), pos, nb))
        pos += nb
    return out, pos


def _compact(v) -> str:
    return json.dumps(v, separators=(",", ":"))


def write_h3t(dst: Union[str, os.PathLike], cfg: H3Config, tensors: Mapping[str, Union[TensorSource, torch.Tensor]], *,
              quant: Optional[Mapping[str, object]] = None, source_name: str = "", source_size: int = 0,
              source_sha256: str = "", extra_meta: Optional[Mapping[str, str]] = None, chunk_bytes: int = 32 << 20,
              progress: Optional[Callable[[str, int, int], None]] = None) -> Dict[str, int]:
    """Write ComfyUI-layout tensors as an .h3t file (h3turbo/h3/writer.py:137-262).  The bytes go to `<dst>.part`,
    which replaces `dst` only once complete and synced, so an interrupted write never leaves a plausible file."""
    if chunk_bytes < 4096 or chunk_bytes % 8:
        raise ValueError("chunk_bytes must be a multiple of 8, at least 4096")
    src = {k: as_source(v) for k, v in tensors.items()}
    glob, refiner, refiner_other, blocks = classify(src)
    n_blocks = cfg.layers
    if n_blocks < 1 or sorted(blocks) != list(range(n_blocks)):
        raise H3TError(f"config has {n_blocks} blocks, the tensors carry block indices {sorted(blocks)[:8]}")
    names0 = _ordered(blocks[0], BLOCK_ORDER)
    sig = {r: (src[f"blocks.0.{r}"].dtype, tuple(src[f"blocks.0.{r}"].shape)) for r in names0}
    for i in range(1, n_blocks):
        if set(blocks[i]) != set(names0):
            raise H3TError(f"block {i}'s tensor set differs from block 0: missing {sorted(set(names0) - set(blocks[i]))[:4]},"
                           f" extra {sorted(set(blocks[i]) - set(names0))[:4]}")
        for r in names0:
            s = src[f"blocks.{i}.{r}"]
            if (s.dtype, tuple(s.shape)) != sig[r]:
                raise H3TError(f"blocks.{i}.{r} is {s.dtype}{tuple(s.shape)}, block 0 has {sig[r][0]}{sig[r][1]}")
    block_layout, block_end = _pack([(r, *sig[r]) for r in names0])
    block_nbytes = _up(block_end, BLOCK_ALIGN)

    gnames = _ordered(glob, GLOBAL_ORDER)
    for j in sorted(refiner):
        gnames += [f"token_refiner.blocks.{j}.{r}" for r in _ordered(refiner[j], BLOCK_ORDER)]
    gnames += _ordered(refiner_other, ("token_refiner.final_norm.weight",))
    glob_layout, glob_end = _pack([(n, src[n].dtype, tuple(src[n].shape)) for n in gnames])
    blocks_start = _up(glob_end, BLOCK_ALIGN)
    data_end = blocks_start + n_blocks * block_nbytes
    if quant:
        qmeta = dict(quant)
    elif quant_linear_names(names0):
        qmeta = {"format": "asym_w4a8_int8", "group_size": cfg.quant_group, "convrot_groupsize": cfg.quant_convrot}
    else:
        qmeta = {}

    # every byte of the data section in order: (offset, name, nbytes, source or None for padding)
    placed = [(e.offset, e.name, e.nbytes, src[e.name]) for e in glob_layout]
    for i in range(n_blocks):
        base = blocks_start + i * block_nbytes
        placed += [(base + e.offset, f"blocks.{i}.{e.name}", e.nbytes, src[f"blocks.{i}.{e.name}"]) for e in block_layout]
    placed.sort(key=lambda it: it[0])
    runs: List[Tuple[int, str, int, Optional[TensorSource]]] = []
    pos, pads = 0, 0
    for off, name, nb, s in placed + [(data_end, "", 0, None)]:
        if off < pos:
            raise H3TError(f"internal layout overlap at {name!r}")
        if off > pos:
            runs.append((pos, f"{PAD_PREFIX}{pads}", off - pos, None))
            pads += 1
        if name:
            runs.append((off, name, nb, s))
        pos = off + nb

    meta = {"format": FORMAT, "version": str(VERSION), "config": cfg.to_json(), "n_blocks": str(n_blocks),
            "tensor_align": str(TENSOR_ALIGN), "block_align": str(BLOCK_ALIGN), "block_nbytes": str(block_nbytes),
            "blocks_start": str(blocks_start),
            "block_ranges": _compact([[blocks_start + i * block_nbytes, blocks_start + (i + 1) * block_nbytes]
                                      for i in range(n_blocks)]),
            "block_layout": _compact([[e.name, e.dtype, list(e.shape), e.offset, e.nbytes] for e in block_layout]),
            "globals_layout": _compact([[e.name, e.dtype, list(e.shape), e.offset, e.nbytes] for e in glob_layout]),
            "quant": json.dumps(qmeta, sort_keys=True), "source_name": source_name, "source_size": str(source_size),
            "source_header_sha256": source_sha256}
    meta.update({str(k): str(v) for k, v in (extra_meta or {}).items()})
    table: Dict[str, object] = {"__metadata__": meta}
    for off, name, nb, s in runs:
        table[name] = {"dtype": s.dtype if s else "U8", "shape": list(s.shape) if s else [nb], "data_offsets": [off, off + nb]}
    head = _compact(table).encode("ascii")
    data_start = _up(8 + len(head), BLOCK_ALIGN)
    head += b" " * (data_start - 8 - len(head))  # JSON whitespace: aligns the data section

    dst = os.fspath(dst)
    part = dst + ".part"
    payload = sum(nb for _, name, nb, _ in runs if not name.startswith(PAD_PREFIX))
    done = 0
    try:
        with open(part, "wb") as f:
            f.write(struct.pack("<Q", data_start - 8))
            f.write(head)
            for off, name, nb, s in runs:
                if s is None:
                    f.write(bytes(nb))
                    continue
                wrote = 0
                for c in s.chunks(chunk_bytes):
                    f.write(c)
                    wrote += len(c)
                if wrote != nb:
                    raise H3TError(f"{name}: the source gave {wrote} bytes, expected {nb}")
                done += nb
                if progress and nb >= (1 << 20):
                    progress(name, done, payload)
            f.flush()
            os.fsync(f.fileno())  # data on disk before the rename makes it visible
        os.replace(part, dst)
    except BaseException:
        try:
            os.remove(part)
        except OSError:
            pass
        raise
    return {"file_size": data_start + data_end, "data_start": data_start, "blocks_start": blocks_start,
            "block_nbytes": block_nbytes, "n_blocks": n_blocks, "n_pads": pads, "n_tensors": len(runs) - pads}
