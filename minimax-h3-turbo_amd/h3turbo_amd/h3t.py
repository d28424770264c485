""".h3t: the block-contiguous safetensors container of the H3 DiT weights (format of h3turbo/h3/store.py:1-40 and
h3turbo/h3/writer.py:137-262; files written here are byte-identical to the reference writer's for the same tensors).

The format, as this module implements it:
  * a safetensors file: an 8-byte little-endian header length, a compact JSON header ("__metadata__" first, then
    one entry per tensor in file order), then the data section;
  * the JSON is padded with spaces so the data section starts on a BLOCK_ALIGN (4 KiB) boundary;
  * the data section holds the globals (patch/condition projections, final layer, token refiner), then block
    0 .. N-1; every tensor starts on a TENSOR_ALIGN (256 B) boundary, every block is one BLOCK_ALIGN-aligned range
    of the same size with the same relative layout; gaps are explicit "__pad.<i>" U8 tensors, since safetensors
    has no holes;
  * tensors are placed in a canonical order (below), which fixes every offset;
  * the metadata carries the format tag and version, the H3Config JSON, the block size / start / ranges, the block
    and globals layouts and the quantisation parameters.

Why the layout matters on MI355X: a block is one contiguous range, so it reaches HBM as ONE DMA transfer (from a
pinned copy, `blockstore.HostBlockStore.from_h3t`), and the kernels read its tensors as typed views of the HBM
slot (`H3TFile.block_weights_from`), 256-byte aligned for the 16-byte vector loads.
"""
from __future__ import annotations

import dataclasses
import json
import math
import mmap
import os
import re
import struct
import sys
import warnings
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, Iterator, List, Mapping, NamedTuple, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .blockstore import BlockLayout, LayoutEntry
from .config import H3Config
from .types import BlockWeights, GlobalWeights, W4A8Weight, Weight

if sys.byteorder != "little":  # pragma: no cover - safetensors data is little-endian
    raise ImportError(".h3t files are little-endian; big-endian hosts are unsupported")

FORMAT = "h3turbo-h3"
VERSION = 1
TENSOR_ALIGN = 256
BLOCK_ALIGN = 4096
PAD_PREFIX = "__pad."
_MAX_HEADER = 100_000_000  # a larger header is taken as garbage, not parsed

_TORCH = {"F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
          "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8, "U8": torch.uint8,
          "BOOL": torch.bool, "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2}
_ST_NAME = {t: n for n, t in _TORCH.items()}

LINEARS = ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")
QUANT_PARTS = ("weight", "weight_s_rel", "weight_s_channel", "weight_codebook", "comfy_quant")


class H3TError(ValueError):
    """Not a valid .h3t container, or an inconsistent write request."""


def torch_dtype(dtype: str) -> torch.dtype:
    try:
        return _TORCH[dtype]
    except KeyError:
        raise H3TError(f"unsupported safetensors dtype {dtype!r}") from None


def itemsize(dtype: str) -> int:
    return torch.empty((), dtype=torch_dtype(dtype)).element_size()


def st_dtype(t: torch.dtype) -> str:
    try:
        return _ST_NAME[t]
    except KeyError:
        raise H3TError(f"torch dtype {t} has no safetensors name") from None


def nbytes_of(dtype: str, shape: Sequence[int]) -> int:
    return itemsize(dtype) * math.prod(shape)


def _ceil(v: int, a: int) -> int:
    return -(-v // a) * a


def _compact(v) -> str:
    return json.dumps(v, separators=(",", ":"))


# ------------------------------------------------------------------------------------------------ canonical order
def _lin(prefix: str) -> Tuple[str, ...]:
    return tuple(f"{prefix}.{p}" for p in QUANT_PARTS)


# Inside a block, then among the globals: these names first, in this order; every other name after them, sorted.
_BLOCK_FIRST = ("adaln_proj.linear.weight", "adaln_proj.linear.bias", "norm1.weight", "attn.q_norm.weight",
                "attn.k_norm.weight", *_lin("attn.qkv_proj"), *_lin("attn.out_proj"), "norm2.weight",
                *_lin("mlp.fc1"), *_lin("mlp.fc2"))
_GLOBAL_FIRST = ("video_patch_proj.weight", "video_patch_proj.bias", "audio_patch_proj.weight", "audio_patch_proj.bias",
                 "condition_proj.weight", "condition_proj.bias", "adaln_t_table", "rope.inv_freq",
                 "final_layer.norm.weight", "final_layer.adaln_proj.linear.weight",
                 "final_layer.adaln_proj.linear.bias", "final_layer.video_out.weight", "final_layer.video_out.bias",
                 "final_layer.audio_out.weight", "final_layer.audio_out.bias")
_REFINER_TAIL_FIRST = ("token_refiner.final_norm.weight",)
# what the whole-model forward needs from the globals (adaln_t_table is optional)
_GLOBALS_NEEDED = tuple(n for n in _GLOBAL_FIRST if n != "adaln_t_table")

_IN_BLOCK = re.compile(r"blocks\.(\d+)\.(.+)")
_IN_REFINER = re.compile(r"token_refiner\.blocks\.(\d+)\.(.+)")


def _canonical(names: Iterable[str], first: Sequence[str]) -> List[str]:
    rank = {n: i for i, n in enumerate(first)}
    return sorted(names, key=lambda n: (0, rank[n], "") if n in rank else (1, 0, n))


def quant_linear_names(names: Iterable[str]) -> List[str]:
    """The W4A8 linears among a block's tensor names: the prefixes that carry a codebook."""
    have = set(names)
    return [p for p in LINEARS if f"{p}.weight_codebook" in have]


# ------------------------------------------------------------------------------------------------ layout plan
@dataclass(frozen=True)
class Slot:
    """One tensor's place: offset from the data section (globals) or from the block start (block slots)."""
    name: str
    dtype: str
    shape: Tuple[int, ...]
    offset: int
    nbytes: int

    def row(self) -> list:
        return [self.name, self.dtype, list(self.shape), self.offset, self.nbytes]


BlockEntry = Slot  # the reader's name for a block slot


def _place(specs: Sequence[Tuple[str, str, Tuple[int, ...]]]) -> Tuple[List[Slot], int]:
    """Slots for the tensors in order, each at the next TENSOR_ALIGN boundary from 0; and the end offset."""
    slots, end = [], 0
    for name, dt, shape in specs:
        at = _ceil(end, TENSOR_ALIGN)
        slots.append(Slot(name, dt, tuple(shape), at, nbytes_of(dt, shape)))
        end = at + slots[-1].nbytes
    return slots, end


class Plan:
    """Where every tensor of a checkpoint goes in its .h3t file: the globals region, then N equal blocks."""

    def __init__(self, cfg: H3Config, specs: Mapping[str, Tuple[str, Tuple[int, ...]]]):
        glob, refiner, refiner_tail, blocks = [], {}, [], {}
        for name in specs:
            if name.startswith(PAD_PREFIX):
                raise H3TError(f"tensor {name!r} uses the reserved padding prefix {PAD_PREFIX!r}")
            m = _IN_BLOCK.fullmatch(name)
            if m:
                blocks.setdefault(int(m.group(1)), set()).add(m.group(2))
                continue
            m = _IN_REFINER.fullmatch(name)
            if m:
                refiner.setdefault(int(m.group(1)), []).append(m.group(2))
            elif name.startswith("token_refiner."):
                refiner_tail.append(name)
            else:
                glob.append(name)
        self.n_blocks = cfg.layers
        if self.n_blocks < 1 or sorted(blocks) != list(range(self.n_blocks)):
            raise H3TError(f"the config has {self.n_blocks} blocks, the tensors carry block indices "
                           f"{sorted(blocks)[:8]}")
        rel = _canonical(blocks[0], _BLOCK_FIRST)
        sig0 = {r: specs[f"blocks.0.{r}"] for r in rel}
        for i in range(1, self.n_blocks):
            if blocks[i] != blocks[0]:
                raise H3TError(f"block {i}'s tensor set differs from block 0: missing "
                               f"{sorted(blocks[0] - blocks[i])[:4]}, extra {sorted(blocks[i] - blocks[0])[:4]}")
            for r in rel:
                dt, shape = specs[f"blocks.{i}.{r}"]
                if (dt, tuple(shape)) != (sig0[r][0], tuple(sig0[r][1])):
                    raise H3TError(f"blocks.{i}.{r} is {dt}{tuple(shape)}, block 0 has {sig0[r][0]}{tuple(sig0[r][1])}")
        self.block, end = _place([(r, sig0[r][0], sig0[r][1]) for r in rel])
        self.block_nbytes = _ceil(end, BLOCK_ALIGN)
        order = _canonical(glob, _GLOBAL_FIRST)
        for j in sorted(refiner):
            order += [f"token_refiner.blocks.{j}.{r}" for r in _canonical(refiner[j], _BLOCK_FIRST)]
        order += _canonical(refiner_tail, _REFINER_TAIL_FIRST)
        self.globals, end = _place([(n, specs[n][0], specs[n][1]) for n in order])
        self.blocks_start = _ceil(end, BLOCK_ALIGN)
        self.data_end = self.blocks_start + self.n_blocks * self.block_nbytes

    def block_start(self, i: int) -> int:
        return self.blocks_start + i * self.block_nbytes

    def placements(self) -> List[Tuple[int, str, int]]:
        """(offset, name, nbytes) of every tensor and every padding run, in file order, covering [0, data_end)."""
        tensors = [(s.offset, s.name, s.nbytes) for s in self.globals]
        for i in range(self.n_blocks):
            tensors += [(self.block_start(i) + s.offset, f"blocks.{i}.{s.name}", s.nbytes) for s in self.block]
        out, at, pads = [], 0, 0
        for off, name, nb in sorted(tensors, key=lambda t: t[0]) + [(self.data_end, None, 0)]:
            if off > at:
                out.append((at, f"{PAD_PREFIX}{pads}", off - at))
                pads += 1
            if name is not None:
                out.append((off, name, nb))
            at = off + nb
        return out

    def metadata(self, cfg: H3Config, quant: Mapping[str, object], source_name: str, source_size: int,
                 source_sha256: str) -> Dict[str, str]:
        ranges = [[self.block_start(i), self.block_start(i) + self.block_nbytes] for i in range(self.n_blocks)]
        return {"format": FORMAT, "version": str(VERSION), "config": cfg.to_json(), "n_blocks": str(self.n_blocks),
                "tensor_align": str(TENSOR_ALIGN), "block_align": str(BLOCK_ALIGN),
                "block_nbytes": str(self.block_nbytes), "blocks_start": str(self.blocks_start),
                "block_ranges": _compact(ranges), "block_layout": _compact([s.row() for s in self.block]),
                "globals_layout": _compact([s.row() for s in self.globals]),
                "quant": json.dumps(dict(quant), sort_keys=True), "source_name": source_name,
                "source_size": str(source_size), "source_header_sha256": source_sha256}


# ------------------------------------------------------------------------------------------------ header
class Header(NamedTuple):
    tensors: Dict[str, dict]  # name -> {"dtype", "shape", "data_offsets"} (offsets from the data section)
    meta: Dict[str, str]
    data_start: int
    file_size: int
    raw: bytes


def read_header(path: Union[str, os.PathLike]) -> Header:
    """The safetensors header of `path`, each entry checked to lie in the data section with dtype x shape bytes.
    Reads no tensor data."""
    size = os.path.getsize(path)
    with open(path, "rb") as fh:
        prefix = fh.read(8)
        n = struct.unpack("<Q", prefix)[0] if len(prefix) == 8 else -1
        if n < 0 or n > _MAX_HEADER or 8 + n > size:
            raise H3TError(f"{path}: not a safetensors file ({size} bytes, header length field {n})")
        blob = fh.read(n)
    try:
        table = json.loads(blob)
    except ValueError as e:
        raise H3TError(f"{path}: the safetensors header is not valid JSON: {e}") from None
    if not isinstance(table, dict):
        raise H3TError(f"{path}: the safetensors header is not a JSON object")
    meta = table.pop("__metadata__", None) or {}
    room = size - 8 - n
    for name, e in table.items():
        try:
            lo, hi = e["data_offsets"]
            dt, shape = e["dtype"], e["shape"]
        except (KeyError, TypeError, ValueError):
            raise H3TError(f"{path}: header entry {name!r} is malformed") from None
        if not 0 <= lo <= hi <= room:
            raise H3TError(f"{path}: {name!r} spans [{lo}, {hi}), outside the {room}-byte data section "
                           "(truncated file?)")
        if dt in _TORCH and hi - lo != nbytes_of(dt, shape):
            raise H3TError(f"{path}: {name!r} holds {hi - lo} bytes, {dt}{list(shape)} needs {nbytes_of(dt, shape)}")
    return Header(table, meta, 8 + n, size, blob)


# ------------------------------------------------------------------------------------------------ weights from views
def _weights(view: Callable[[str], Optional[torch.Tensor]], group: int, convrot: int) -> BlockWeights:
    """BlockWeights from a name -> tensor accessor (None when absent): a linear with a codebook is W4A8."""

    def linear(p: str) -> Weight:
        book = view(f"{p}.weight_codebook")
        if book is None:
            return view(f"{p}.weight")
        return W4A8Weight(view(f"{p}.weight"), view(f"{p}.weight_s_rel"), view(f"{p}.weight_s_channel"), book,
                          group, convrot)

    return BlockWeights(qkv=linear("attn.qkv_proj"), out=linear("attn.out_proj"), fc1=linear("mlp.fc1"),
                        fc2=linear("mlp.fc2"), norm1=view("norm1.weight"), norm2=view("norm2.weight"),
                        q_norm=view("attn.q_norm.weight"), k_norm=view("attn.k_norm.weight"),
                        adaln_w=view("adaln_proj.linear.weight"), adaln_b=view("adaln_proj.linear.bias"))


class TensorInfo(NamedTuple):
    dtype: str
    shape: Tuple[int, ...]
    start: int  # absolute file offset
    nbytes: int


# ------------------------------------------------------------------------------------------------ reader
class H3TFile:
    """A read-only, memory-mapped .h3t file (the reader of h3turbo/h3/store.py:182-400).  Every accessor hands out a
    zero-copy view of the mapping; views stay valid after close().  As a block source of the streaming engine it has
    n_blocks, block_nbytes, block_tensor(i), block_bytes(i) and block_weights_from(buf)."""

    pinned = False  # file pages are pageable: the engine stages or pins copies of the blocks

    def __init__(self, path: Union[str, os.PathLike]):
        self.path = os.fspath(path)
        hdr = read_header(self.path)
        meta = hdr.meta
        if meta.get("format") != FORMAT:
            raise H3TError(f"{self.path}: not an h3t file (format tag {meta.get('format')!r}, expected {FORMAT!r})")
        if meta.get("version") != str(VERSION):
            raise H3TError(f"{self.path}: h3t version {meta.get('version')!r}, this reader reads version {VERSION}")
        try:
            self.cfg = H3Config.from_json(meta["config"])
            self.n_blocks = int(meta["n_blocks"])
            self.block_nbytes = int(meta["block_nbytes"])
            self.blocks_start = int(meta["blocks_start"])
            self.block_layout = [Slot(n, d, tuple(s), int(o), int(b)) for n, d, s, o, b in json.loads(meta["block_layout"])]
            ranges = json.loads(meta["block_ranges"])
            self.quant = json.loads(meta.get("quant") or "{}")
            self.source_name = meta.get("source_name", "")
            self.source_size = int(meta.get("source_size") or 0)
            self.meta = dict(meta)
            self.layout = BlockLayout([LayoutEntry(s.name, torch_dtype(s.dtype), s.shape, s.offset, s.nbytes)
                                       for s in self.block_layout])
        except H3TError:
            raise
        except (KeyError, TypeError, ValueError, IndexError, AttributeError) as e:
            raise H3TError(f"{self.path}: corrupt h3t metadata: {e!r}") from None
        self.data_start, self.file_size = hdr.data_start, hdr.file_size
        self._verify(hdr, ranges)
        self.quant_group = int(self.quant.get("group_size", self.cfg.quant_group))
        self.quant_convrot = int(self.quant.get("convrot_groupsize", self.cfg.quant_convrot))
        self._info = {n: TensorInfo(e["dtype"], tuple(e["shape"]), self.data_start + e["data_offsets"][0],
                                    e["data_offsets"][1] - e["data_offsets"][0])
                      for n, e in hdr.tensors.items() if not n.startswith(PAD_PREFIX)}
        with open(self.path, "rb") as fh:
            self._map: Optional[mmap.mmap] = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        with warnings.catch_warnings():  # the mapping is read-only; nothing here writes through these views
            warnings.simplefilter("ignore")
            self._bytes: Optional[torch.Tensor] = torch.frombuffer(self._map, dtype=torch.uint8)

    def _verify(self, hdr: Header, ranges) -> None:
        """The format's invariants, against the header: block count, alignment, exact size, contiguity, the shared
        block layout, complete W4A8 linears."""
        p = self.path
        if self.n_blocks < 1 or self.n_blocks != self.cfg.layers:
            raise H3TError(f"{p}: n_blocks={self.n_blocks} but config.layers={self.cfg.layers}")
        if any(v % BLOCK_ALIGN for v in (self.data_start, self.blocks_start, self.block_nbytes)):
            raise H3TError(f"{p}: data section or block offsets are not {BLOCK_ALIGN}-byte aligned")
        want = self.data_start + self.blocks_start + self.n_blocks * self.block_nbytes
        if hdr.file_size != want:
            raise H3TError(f"{p}: the layout needs exactly {want} bytes, the file has {hdr.file_size} "
                           "(truncated, or trailing data)")
        if not isinstance(ranges, list) or len(ranges) != self.n_blocks:
            raise H3TError(f"{p}: block_ranges does not list {self.n_blocks} blocks")
        for i, r in enumerate(ranges):
            lo = self.blocks_start + i * self.block_nbytes
            if not isinstance(r, list) or r != [lo, lo + self.block_nbytes]:
                raise H3TError(f"{p}: block_ranges[{i}] = {r} disagrees with blocks_start / block_nbytes")
        if self.layout.nbytes > self.block_nbytes:
            raise H3TError(f"{p}: the block layout spans {self.layout.nbytes} bytes, blocks are {self.block_nbytes}")
        for i in range(self.n_blocks):
            lo = self.blocks_start + i * self.block_nbytes
            for s in self.block_layout:
                e = hdr.tensors.get(f"blocks.{i}.{s.name}")
                if (e is None or e["dtype"] != s.dtype or tuple(e["shape"]) != s.shape
                        or list(e["data_offsets"]) != [lo + s.offset, lo + s.offset + s.nbytes]):
                    raise H3TError(f"{p}: blocks.{i}.{s.name} does not match the block layout")
        at = 0
        for name, e in sorted(hdr.tensors.items(), key=lambda kv: kv[1]["data_offsets"][0]):
            lo, hi = e["data_offsets"]
            if lo != at:
                raise H3TError(f"{p}: hole or overlap before {name!r}")
            if lo % TENSOR_ALIGN and not name.startswith(PAD_PREFIX):
                raise H3TError(f"{p}: {name!r} starts at {lo}, not {TENSOR_ALIGN}-byte aligned")
            at = hi
        if at != hdr.file_size - self.data_start:
            raise H3TError(f"{p}: the tensors cover {at} of the {hdr.file_size - self.data_start} data bytes")
        names = {s.name for s in self.block_layout}
        for lin in quant_linear_names(names):
            absent = [q for q in QUANT_PARTS if f"{lin}.{q}" not in names]
            if absent:
                raise H3TError(f"{p}: W4A8 linear {lin} lacks {absent}")

    def _mapped(self) -> torch.Tensor:
        if self._bytes is None:
            raise ValueError("H3TFile is closed")
        return self._bytes

    # ---- blocks
    def block_range(self, i: int) -> Tuple[int, int]:
        """[start, end) file offsets of block i."""
        if not 0 <= i < self.n_blocks:
            raise IndexError(f"block {i} outside [0, {self.n_blocks})")
        lo = self.data_start + self.blocks_start + i * self.block_nbytes
        return lo, lo + self.block_nbytes

    def block_tensor(self, i: int) -> torch.Tensor:
        """uint8 view of block i: the source of its host -> device copy."""
        lo, hi = self.block_range(i)
        return self._mapped()[lo:hi]

    def block_bytes(self, i: int) -> np.ndarray:
        """Read-only numpy view of block i."""
        a = self.block_tensor(i).numpy()
        a.flags.writeable = False
        return a

    @property
    def block_layout_size(self) -> int:
        return max((s.offset + s.nbytes for s in self.block_layout), default=0)

    def block_weights_from(self, buf: torch.Tensor) -> BlockWeights:
        """Typed zero-copy views of one block held in `buf` (1-D uint8 of block_nbytes, any device)."""
        if buf.dtype != torch.uint8 or buf.dim() != 1 or buf.numel() != self.block_nbytes:
            raise ValueError(f"need a 1-D uint8 buffer of {self.block_nbytes} bytes, got {tuple(buf.shape)} {buf.dtype}")
        lay = self.layout
        return _weights(lambda n: lay.view(buf, n) if n in lay else None, self.quant_group, self.quant_convrot)

    def block_weights_cpu(self, i: int) -> BlockWeights:
        return self.block_weights_from(self.block_tensor(i))

    # ---- named tensors
    def keys(self) -> List[str]:
        return list(self._info)

    def info(self, name: str) -> TensorInfo:
        try:
            return self._info[name]
        except KeyError:
            raise KeyError(f"{name!r} is not in {self.path}") from None

    def tensor(self, name: str) -> torch.Tensor:
        """Zero-copy CPU view of one tensor."""
        t = self.info(name)
        v = self._mapped()[t.start:t.start + t.nbytes]
        dt = torch_dtype(t.dtype)
        return (v if dt == torch.uint8 else v.view(dt)).view(t.shape)

    def has_globals(self) -> bool:
        """Whether the file holds every global tensor the whole-model forward needs."""
        return all(n in self._info for n in _GLOBALS_NEEDED)

    def globals_nbytes(self, refiner: bool = True) -> int:
        """Bytes of the tensors outside the blocks (with or without the token refiner)."""
        return sum(t.nbytes for n, t in self._info.items()
                   if not _IN_BLOCK.fullmatch(n) and (refiner or not n.startswith("token_refiner.")))

    def load_globals(self, device="cpu", *, refiner_device=None) -> GlobalWeights:
        """GlobalWeights on `device`, the token refiner on `refiner_device` (default: the same) (reference
        h3turbo/h3/store.py:329-365).  On the CPU the globals are copies and the refiner stays zero-copy views of
        the mapping; refiner_device="cpu" keeps the refiner out of HBM until the text is encoded."""
        dev = torch.device(device)
        rdev = torch.device(refiner_device) if refiner_device is not None else dev
        absent = [n for n in _GLOBALS_NEEDED if n not in self._info]
        if absent:
            raise H3TError(f"{self.path}: missing global tensors {absent}")

        def on(name: str, d: torch.device, keep_view: bool) -> torch.Tensor:
            t = self.tensor(name)
            return t.to(d) if d.type != "cpu" else (t if keep_view else t.clone())

        g = lambda name: on(name, dev, False)  # noqa: E731
        refiner = []
        for j in range(self.cfg.refiner_layers):
            pre = f"token_refiner.blocks.{j}."
            w = _weights(lambda r: on(pre + r, rdev, True) if pre + r in self._info else None, self.quant_group,
                         self.quant_convrot)
            refiner.append(dataclasses.replace(w, adaln_w=None, adaln_b=None))  # refiner blocks are unmodulated
        fnorm = "token_refiner.final_norm.weight"
        return GlobalWeights(
            video_patch_w=g("video_patch_proj.weight"), video_patch_b=g("video_patch_proj.bias"),
            audio_patch_w=g("audio_patch_proj.weight"), audio_patch_b=g("audio_patch_proj.bias"),
            condition_w=g("condition_proj.weight"), condition_b=g("condition_proj.bias"),
            adaln_t_table=g("adaln_t_table") if "adaln_t_table" in self._info else None,
            rope_inv_freq=g("rope.inv_freq"), final_norm=g("final_layer.norm.weight"),
            final_adaln_w=g("final_layer.adaln_proj.linear.weight"),
            final_adaln_b=g("final_layer.adaln_proj.linear.bias"),
            video_out_w=g("final_layer.video_out.weight"), video_out_b=g("final_layer.video_out.bias"),
            audio_out_w=g("final_layer.audio_out.weight"), audio_out_b=g("final_layer.audio_out.bias"),
            refiner=refiner, refiner_final_norm=on(fnorm, rdev, True) if fnorm in self._info else None)

    # ---- lifecycle
    def close(self) -> None:
        """Release the mapping (views already handed out keep it alive until they go)."""
        if self._map is None:
            return
        m, self._map, self._bytes = self._map, None, None
        try:
            m.close()
        except BufferError:  # live views: the mapping goes with the last of them
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
    """The little-endian bytes of one tensor, produced in chunks: the writer holds one chunk at a time."""

    dtype: str
    shape: Tuple[int, ...]
    nbytes: int

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        raise NotImplementedError

    def read(self) -> torch.Tensor:
        buf = torch.empty(self.nbytes, dtype=torch.uint8)
        at = 0
        for c in self.chunks(32 << 20):
            buf[at:at + len(c)] = torch.frombuffer(bytearray(c), dtype=torch.uint8)
            at += len(c)
        dt = torch_dtype(self.dtype)
        return (buf if dt == torch.uint8 else buf.view(dt)).view(self.shape)


class TorchSource(TensorSource):
    def __init__(self, t: torch.Tensor):
        self._t = t.detach().cpu().contiguous()
        self.dtype, self.shape = st_dtype(self._t.dtype), tuple(self._t.shape)
        self.nbytes = self._t.numel() * self._t.element_size()

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        if self.nbytes:
            whole = memoryview(self._t.reshape(-1).view(torch.uint8).numpy())
            for lo in range(0, self.nbytes, chunk_bytes):
                yield whole[lo:lo + chunk_bytes]


class LazySource(TensorSource):
    """A tensor produced by `fn()` only when the writer reaches it."""

    def __init__(self, dtype: str, shape: Sequence[int], fn: Callable[[], torch.Tensor]):
        self.dtype, self.shape, self._fn = dtype, tuple(shape), fn
        self.nbytes = nbytes_of(dtype, self.shape)

    def chunks(self, chunk_bytes: int) -> Iterator[memoryview]:
        made = TorchSource(self._fn())
        if (made.dtype, made.shape) != (self.dtype, self.shape):
            raise H3TError(f"lazy tensor made {made.dtype}{made.shape}, declared {self.dtype}{self.shape}")
        yield from made.chunks(chunk_bytes)


def as_source(x: Union[TensorSource, torch.Tensor]) -> TensorSource:
    if isinstance(x, TensorSource):
        return x
    if isinstance(x, torch.Tensor):
        return TorchSource(x)
    raise TypeError(f"expected a Tensor or TensorSource, got {type(x).__name__}")


def write_h3t(dst: Union[str, os.PathLike], cfg: H3Config, tensors: Mapping[str, Union[TensorSource, torch.Tensor]], *,
              quant: Optional[Mapping[str, object]] = None, source_name: str = "", source_size: int = 0,
              source_sha256: str = "", extra_meta: Optional[Mapping[str, str]] = None, chunk_bytes: int = 32 << 20,
              progress: Optional[Callable[[str, int, int], None]] = None) -> Dict[str, int]:
    """Write ComfyUI-layout tensors as an .h3t file (h3turbo/h3/writer.py:137-262).  The bytes go to `<dst>.part`,
    renamed to `dst` only once complete and synced: an interrupted write never leaves a plausible file."""
    if chunk_bytes < 4096 or chunk_bytes % 8:
        raise ValueError("chunk_bytes must be a multiple of 8, at least 4096")
    src = {name: as_source(v) for name, v in tensors.items()}
    plan = Plan(cfg, {name: (s.dtype, s.shape) for name, s in src.items()})
    if quant:
        qmeta = dict(quant)
    elif quant_linear_names(s.name for s in plan.block):
        qmeta = {"format": "asym_w4a8_int8", "group_size": cfg.quant_group, "convrot_groupsize": cfg.quant_convrot}
    else:
        qmeta = {}
    meta = plan.metadata(cfg, qmeta, source_name, source_size, source_sha256)
    meta.update({str(k): str(v) for k, v in (extra_meta or {}).items()})
    runs = plan.placements()
    table: Dict[str, object] = {"__metadata__": meta}
    for off, name, nb in runs:
        s = src.get(name)
        table[name] = {"dtype": s.dtype if s else "U8", "shape": list(s.shape) if s else [nb],
                       "data_offsets": [off, off + nb]}
    head = _compact(table).encode("ascii")
    data_start = _ceil(8 + len(head), BLOCK_ALIGN)
    head = head.ljust(data_start - 8, b" ")  # JSON whitespace aligns the data section

    dst = os.fspath(dst)
    part = dst + ".part"
    payload = sum(src[name].nbytes for _, name, _ in runs if name in src)
    written = 0
    try:
        with open(part, "wb") as fh:
            fh.write(struct.pack("<Q", len(head)))
            fh.write(head)
            for _, name, nb in runs:
                s = src.get(name)
                if s is None:
                    fh.write(bytes(nb))
                    continue
                got = 0
                for c in s.chunks(chunk_bytes):
                    fh.write(c)
                    got += len(c)
                if got != nb:
                    raise H3TError(f"{name}: the source gave {got} bytes, expected {nb}")
                written += nb
                if progress and nb >= (1 << 20):
                    progress(name, written, payload)
            fh.flush()
            os.fsync(fh.fileno())  # on disk before the rename makes it visible
        os.replace(part, dst)
    except BaseException:
        try:
            os.remove(part)
        except OSError:
            pass
        raise
    n_pads = sum(1 for _, name, _ in runs if name.startswith(PAD_PREFIX))
    return {"file_size": data_start + plan.data_end, "data_start": data_start, "blocks_start": plan.blocks_start,
            "block_nbytes": plan.block_nbytes, "n_blocks": plan.n_blocks, "n_pads": n_pads,
            "n_tensors": len(runs) - n_pads}
