"""Weight streaming for the H3 DiT on MI355X: resident blocks in HBM plus a ring of device slots fed by
asynchronous host -> HBM copies on a side stream.

Same BlockProvider contract, constructor and state machine as the reference's StreamingProvider
(h3turbo/h3/stream.py:115-623), so it plugs into the same model loop:

* Blocks 0..resident-1 live in HBM for good.  The others cycle through `ring` slots, each one device buffer of
  block_nbytes; a block's BlockWeights are zero-copy typed views of its slot (blockstore.BlockLayout).
* One worker thread issues the copies: one contiguous hipMemcpyAsync per block (libh3k's h3k_copy_h2d_async) on
  a dedicated copy stream.  Slot reuse is ordered on the device, never by blocking the host: the copy stream waits
  for the slot's `done` event (recorded by release() on the compute stream) and the compute stream waits for the
  slot's `ready` event in acquire().  acquire() only waits until the copy has been issued.
* Lookahead is cyclic over the streamed blocks, so the next forward's first streamed blocks are fetched while the
  last blocks of this one still compute.
* Host sources, per streamed block ("host kind"):
    registered  the store itself is page-locked (allocated pinned): DMA straight from it, no second copy
    pinned      a page-locked copy of the block made at construction
    staged      filled into one of two page-locked staging buffers by the worker, then DMA'd
    pageable    copied synchronously from pageable memory (pin=False, or no lockable memory)
  Page-locked memory is always allocated pinned (hipHostMalloc through torch); existing pages are never
  registered.

Nothing here computes: on MI355X with 288 GB of HBM a whole 4-bit stack is normally resident (resident="auto"
plans that), and the ring only matters for stacks larger than free HBM.  device="cpu" runs the identical state
machine with plain copies and no events, so the bookkeeping, ordering and error paths are tested without a GPU.
"""
from __future__ import annotations

import atexit
import os
import threading
import time
import weakref
from typing import Callable, Dict, List, Optional, Tuple, Union

import numpy as np
import torch

from .types import BlockWeights

_GIB = 1 << 30
_DEVICE_MARGIN = 512 << 20  # HBM that torch does not see (library workspaces, code objects), kept free by "auto"
FREE, PENDING, READY, ACQUIRED, IDLE = range(5)
_STATE_NAMES = ("free", "pending", "ready", "acquired", "idle")


def free_ram_bytes() -> int:
    """Host memory available without swapping (reclaimable page cache included)."""
    try:
        import psutil

        return int(psutil.virtual_memory().available)
    except ImportError:
        pass
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        pass
    raise RuntimeError("cannot determine free RAM (install psutil, or pass pin_blocks explicitly)")


def plan_residency(store, free_vram_bytes: int, reserve_bytes: int = 0, ring: int = 3) -> int:
    """Largest r such that r resident blocks plus min(ring, n - r) ring slots fit in free_vram_bytes - reserve_bytes
    (h3turbo/h3/stream.py:61-71).  0 when not even the ring fits (the slot allocation then reports the OOM)."""
    if ring < 1:
        raise ValueError("ring must be >= 1")
    room, blk, n = free_vram_bytes - reserve_bytes, store.block_nbytes, store.n_blocks
    best = 0
    for r in range(n + 1):
        if (r + min(ring, n - r)) * blk <= room:
            best = r
    return best


def plan_pinned_blocks(store, streamed: int, free_ram: int, pin_fraction: float = 0.5, headroom: int = 4 * _GIB) -> int:
    """How many streamed blocks get a page-locked host copy: within pin_fraction of free RAM, never leaving less
    than `headroom` free, after reserving two staging buffers (h3turbo/h3/stream.py:74-78)."""
    budget = min(free_ram * pin_fraction, free_ram - headroom) - 2 * store.block_nbytes
    return int(max(0, min(streamed, budget // store.block_nbytes)))


_OPEN: "weakref.WeakSet[StreamingProvider]" = weakref.WeakSet()


@atexit.register
def _close_open_providers() -> None:
    """A provider left open at interpreter exit must not leave its worker inside a device call."""
    for p in list(_OPEN):
        try:
            p.close()
        except Exception:
            pass


def hip_transfer(dst: torch.Tensor, src: torch.Tensor, non_blocking: bool) -> None:
    """Default slot copy: host -> HBM as one hipMemcpyAsync on the current (copy) stream, through libh3k
    (replaces slot.buf.copy_(src, non_blocking) of h3turbo/h3/stream.py:346-354).  A synchronous copy waits for
    the stream.  Anything that is not host -> device falls back to torch's copy."""
    if not dst.is_cuda or src.is_cuda:
        dst.copy_(src, non_blocking=non_blocking)
        return
    from . import _lib

    nbytes = dst.numel() * dst.element_size()
    if src.numel() * src.element_size() != nbytes or not dst.is_contiguous() or not src.is_contiguous():
        raise ValueError("slot copy needs two contiguous buffers of the same size")
    stream = torch.cuda.current_stream(dst.device)
    _lib.check(_lib.load().h3k_copy_h2d_async(dst.data_ptr(), src.data_ptr(), nbytes, stream.cuda_stream),
               "h3k_copy_h2d_async")
    if not non_blocking:
        stream.synchronize()


class _Slot:
    __slots__ = ("idx", "buf", "weights", "state", "block", "ready", "done", "stamp")

    def __init__(self, idx: int, buf: torch.Tensor, weights: BlockWeights):
        self.idx, self.buf, self.weights = idx, buf, weights
        self.state, self.block, self.ready, self.done, self.stamp = FREE, None, None, None, 0


class StreamingProvider:
    """BlockProvider over a block store (blockstore.HostBlockStore or any object with n_blocks, block_nbytes,
    block_tensor(i), block_bytes(i), block_weights_from(buf)): resident blocks plus a prefetching ring.
    Use as a context manager or call close(): the worker thread and page-locked host memory live until then."""

    def __init__(self, store, device: Union[str, torch.device] = "cuda", resident: Union[int, str] = "auto",
                 prefetch: int = 2, pin: Union[bool, str] = "auto", ring: int = 3, *, reserve_bytes: int = 1536 << 20,
                 free_vram_bytes: Optional[int] = None, pin_fraction: float = 0.5, ram_headroom_bytes: int = 4 * _GIB,
                 pin_blocks: Optional[int] = None, pin_mode: str = "auto",
                 transfer: Optional[Callable[[torch.Tensor, torch.Tensor, bool], None]] = None,
                 wait_timeout: float = 600.0):
        if ring < 1 or prefetch < 0 or pin not in (True, False, "auto") or pin_mode not in ("auto", "register", "copy", "stage"):
            raise ValueError("ring >= 1, prefetch >= 0, pin in (True, False, 'auto'), "
                             "pin_mode in ('auto', 'register', 'copy', 'stage')")
        if not (resident == "auto" or (isinstance(resident, int) and not isinstance(resident, bool) and resident >= 0)):
            raise ValueError("resident must be 'auto' or a non-negative int")
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.store, self.device, self._gpu = store, dev, dev.type == "cuda"
        self.n_blocks, self._prefetch, self._timeout = store.n_blocks, prefetch, wait_timeout
        self._transfer = transfer or (hip_transfer if self._gpu else (lambda d, s, nb: d.copy_(s)))
        self._cv = threading.Condition()
        self._slots: List[_Slot] = []
        self._slot_of: Dict[int, _Slot] = {}
        self._resident: Dict[int, Tuple[torch.Tensor, BlockWeights]] = {}
        self._kind: Dict[int, str] = {}
        self._src: Dict[int, torch.Tensor] = {}
        self._stage: List[torch.Tensor] = []
        self._stage_done: List[Optional[torch.cuda.Event]] = []
        self._stage_turn = 0
        self._locked_bytes = 0
        self._streamed: List[int] = []
        self._pos, self._demand, self._clock = -1, None, 0
        self._stop = self._closed = self._in_forward = False
        self._error: Optional[BaseException] = None
        self._thread: Optional[threading.Thread] = None
        self._plan_info: Dict[str, object] = {}
        self._st = self._zero_stats()
        self._copy_stream = torch.cuda.Stream(dev) if self._gpu else None
        _OPEN.add(self)
        try:
            self._build(resident, ring, pin, pin_mode, reserve_bytes, free_vram_bytes, pin_fraction, ram_headroom_bytes,
                        pin_blocks)
        except BaseException:
            self.close()
            raise

    @staticmethod
    def _zero_stats() -> Dict[str, float]:
        return dict(acquires=0, waits=0, wait_s=0.0, copies=0, bytes=0, busy_s=0.0)

    # ----------------------------------------------------------------------------------------- construction
    def _device_buffer(self) -> torch.Tensor:
        return torch.empty(self.store.block_nbytes, dtype=torch.uint8, device=self.device)

    def _locked_buffer(self) -> Optional[torch.Tensor]:
        """A page-locked host buffer of one block (plain memory on the CPU path); None when none can be had."""
        if not self._gpu:
            return torch.empty(self.store.block_nbytes, dtype=torch.uint8)
        try:
            t = torch.empty(self.store.block_nbytes, dtype=torch.uint8, pin_memory=True)
        except RuntimeError:
            return None
        self._locked_bytes += self.store.block_nbytes
        return t

    def _make_resident(self, b: int) -> bool:
        try:
            buf = self._device_buffer()
        except torch.cuda.OutOfMemoryError:
            return False
        src = self._src.get(b)
        buf.copy_(src if src is not None else self.store.block_tensor(b))  # synchronous; the store is the truth
        self._resident[b] = (buf, self.store.block_weights_from(buf))
        return True

    def _add_slots(self, count: int, strict: bool) -> None:
        for k in range(count):
            try:
                buf = self._device_buffer()
            except torch.cuda.OutOfMemoryError as e:
                if k and not strict:
                    break
                raise torch.cuda.OutOfMemoryError(
                    f"cannot allocate streaming slot {k + 1} of {count} ({self.store.block_nbytes / 2**20:.0f} MiB): "
                    "lower resident/ring or free HBM") from e
            self._slots.append(_Slot(k, buf, self.store.block_weights_from(buf)))

    def _build(self, resident, ring, pin, pin_mode, reserve, free_vram, pin_fraction, headroom, pin_blocks) -> None:
        n = self.n_blocks
        auto = resident == "auto"
        if auto:
            if free_vram is None:
                free_vram = torch.cuda.mem_get_info(self.device)[0] if self._gpu else free_ram_bytes() // 2
            resident = plan_residency(self.store, free_vram, reserve + (_DEVICE_MARGIN if self._gpu else 0), ring)
        for b in range(min(int(resident), n)):
            if not self._make_resident(b):
                if auto:
                    break  # the plan was optimistic: the rest streams
                raise torch.cuda.OutOfMemoryError(f"cannot keep block {b} resident")
        self._streamed = list(range(len(self._resident), n))
        self._add_slots(min(ring, len(self._streamed)), strict=True)
        if self._streamed:
            self._plan_host(pin, pin_mode, pin_fraction, headroom, pin_blocks)
            self._start_worker()

    def _plan_host(self, pin, pin_mode, pin_fraction, headroom, pin_blocks) -> None:
        """Choose each streamed block's host source (h3turbo/h3/stream.py:219-268)."""
        streamed = self._streamed
        if getattr(self.store, "pinned", False) and self._gpu and pin is not False:
            for b in streamed:  # the store's own pages are page-locked: zero copy
                self._kind[b] = "registered"
            return
        if pin is False or pin_mode == "stage" or pin_mode == "register":
            want = 0  # "register": locking existing pages in place is not done on this platform
        elif pin is True:
            want = len(streamed)
        elif pin_blocks is not None:
            want = max(0, min(len(streamed), pin_blocks))
        elif self._gpu:
            avail = free_ram_bytes()
            self._plan_info["ram_available_gib"] = round(avail / _GIB, 2)
            want = plan_pinned_blocks(self.store, len(streamed), avail, pin_fraction, headroom)
        else:
            want = 0
        self._plan_info["pinned_wanted"] = want
        for b in streamed[:want]:
            t = self._locked_buffer()
            if t is None:
                break  # out of lockable memory: the rest is staged
            np.copyto(t.numpy(), self.store.block_bytes(b))
            self._src[b], self._kind[b] = t, "pinned"
        rest = [b for b in streamed if b not in self._kind]
        staging = rest and pin is not False and (pin is True or want > 0 or pin_mode in ("stage", "register")
                                                 or (pin == "auto" and self._gpu))
        if staging:
            self._open_staging()
        for b in rest:
            self._kind[b] = "staged" if self._stage else "pageable"

    def _open_staging(self) -> None:
        while len(self._stage) < 2:
            t = self._locked_buffer()
            if t is None:
                break
            self._stage.append(t)
        self._stage_done = [None] * len(self._stage)

    # ----------------------------------------------------------------------------------------- worker
    def _start_worker(self) -> None:
        self._thread = threading.Thread(target=self._worker, name="h3k-stream", daemon=True)
        self._thread.start()

    def _wanted(self) -> List[int]:
        """The demanded block first, then the cyclic lookahead after the current position."""
        s = self._streamed
        out = [self._demand] if self._demand is not None else []
        out += [s[(self._pos + 1 + k) % len(s)] for k in range(min(self._prefetch, len(s)))]
        return out

    def _victim(self, keep) -> Optional[_Slot]:
        """A slot to (re)fill: a free one, else the least recently used released one, else the least recently
        used prefetched one that is not itself wanted."""
        for s in self._slots:
            if s.state == FREE:
                return s
        for state in (IDLE, READY):
            cands = [s for s in self._slots if s.state == state and s.block not in keep]
            if cands:
                return min(cands, key=lambda s: s.stamp)
        return None

    def _plan_copy(self, commit: bool = True) -> Optional[Tuple[_Slot, int]]:
        wanted = self._wanted()
        for k, b in enumerate(wanted):
            if b in self._slot_of:
                continue
            demanded = k == 0 and b == self._demand
            slot = self._victim(() if demanded else wanted)
            if slot is None:
                return None
            if commit:
                if slot.block is not None:
                    del self._slot_of[slot.block]
                self._clock += 1
                slot.state, slot.block, slot.stamp = PENDING, b, self._clock
                self._slot_of[b] = slot
            return slot, b
        return None

    def _worker(self) -> None:
        # inference mode is per thread: slots created under torch.inference_mode() are inference tensors, and
        # copies into them from this thread must run in the mode too
        with torch.inference_mode():
            if self._gpu:
                torch.cuda.set_device(self.device)
            try:
                while True:
                    with self._cv:
                        while not self._stop:
                            job = self._plan_copy()
                            if job:
                                break
                            self._cv.wait()
                        if self._stop:
                            return
                    self._copy(*job)
                    with self._cv:
                        job[0].state = READY
                        self._cv.notify_all()
            except BaseException as e:  # re-raised by the next acquire()
                with self._cv:
                    self._error = e
                    self._cv.notify_all()

    def _copy(self, slot: _Slot, b: int) -> None:
        t0, kind, stage = time.perf_counter(), self._kind[b], None
        if kind == "staged":
            stage = self._stage_turn
            self._stage_turn = (stage + 1) % len(self._stage)
            if self._stage_done[stage] is not None:
                self._stage_done[stage].synchronize()  # the previous DMA out of this buffer has finished
            np.copyto(self._stage[stage].numpy(), self.store.block_bytes(b))
            src = self._stage[stage]
        elif kind == "pageable":
            src = self.store.block_tensor(b)
        elif kind == "registered":
            src = self.store.block_tensor(b)
        else:
            src = self._src[b]
        if self._gpu:
            cs = self._copy_stream
            with torch.cuda.stream(cs):
                if slot.done is not None:
                    cs.wait_event(slot.done)  # on the device: the slot's last reader has finished
                self._transfer(slot.buf, src, kind != "pageable")
                ev = torch.cuda.Event()
                ev.record(cs)
            slot.ready = ev
            if stage is not None:
                self._stage_done[stage] = ev
        else:
            self._transfer(slot.buf, src, False)
        with self._cv:
            self._st["copies"] += 1
            self._st["bytes"] += self.store.block_nbytes
            self._st["busy_s"] += time.perf_counter() - t0

    # ----------------------------------------------------------------------------------------- BlockProvider
    def _raise_if_broken(self) -> None:
        if self._closed:
            raise RuntimeError("StreamingProvider is closed")
        if self._error is not None:
            raise RuntimeError(f"H3 streaming worker failed: {self._error!r}") from self._error

    def begin_forward(self) -> None:
        if self._in_forward:  # the last forward never reached end_forward
            self.end_forward()
        self._in_forward = True

    def acquire(self, i: int) -> BlockWeights:
        if not 0 <= i < self.n_blocks:
            raise IndexError(f"block {i} out of range [0, {self.n_blocks})")
        if self._closed:
            raise RuntimeError("StreamingProvider is closed")
        if i in self._resident:
            return self._resident[i][1]
        if not self._slots:
            raise RuntimeError("the streaming provider is parked (no device slots); resize() it before a forward")
        t0 = time.perf_counter()
        deadline, waited = t0 + self._timeout, False
        with self._cv:
            self._raise_if_broken()
            while True:
                slot = self._slot_of.get(i)
                if slot is None:
                    if all(s.state == ACQUIRED for s in self._slots):
                        raise RuntimeError(f"all {len(self._slots)} ring slots are held; release() a block before "
                                           f"acquiring block {i} (ring too small?)")
                    self._demand = i
                    self._cv.notify_all()
                elif slot.state == ACQUIRED:
                    raise RuntimeError(f"block {i} is already acquired")
                elif slot.state in (READY, IDLE):
                    break
                waited = True
                left = deadline - time.perf_counter()
                if left <= 0:
                    raise TimeoutError(f"timed out after {self._timeout:.0f}s waiting for block {i}: {self._describe()}")
                self._cv.wait(min(left, 1.0))
                self._raise_if_broken()
            slot.state = ACQUIRED
            self._clock += 1
            slot.stamp = self._clock
            if self._demand == i:
                self._demand = None
            self._pos = self._streamed.index(i)
            self._st["acquires"] += 1
            if waited:
                self._st["waits"] += 1
                self._st["wait_s"] += time.perf_counter() - t0
            self._cv.notify_all()  # the lookahead window moved
        if self._gpu and slot.ready is not None:
            torch.cuda.current_stream(self.device).wait_event(slot.ready)
        return slot.weights

    def release(self, i: int) -> None:
        if i in self._resident:
            return
        ev = None
        if self._gpu:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))  # after every kernel that reads the slot
        with self._cv:
            slot = self._slot_of.get(i)
            if slot is None or slot.state != ACQUIRED:
                raise RuntimeError(f"release({i}) but block {i} is not acquired")
            slot.done, slot.state = ev, IDLE
            self._clock += 1
            slot.stamp = self._clock
            self._cv.notify_all()

    def end_forward(self) -> None:
        """Reset for the next forward, also after an exception: held slots are released behind an event on the
        current stream and the lookahead restarts at the first streamed block."""
        ev = None
        if self._gpu and not self._closed:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
        with self._cv:
            for s in self._slots:
                if s.state == ACQUIRED:
                    s.state, s.done = IDLE, ev
            self._pos, self._demand, self._in_forward = -1, None, False
            self._cv.notify_all()

    # ----------------------------------------------------------------------------------------- residency changes
    def device_bytes(self) -> int:
        return (len(self._resident) + len(self._slots)) * self.store.block_nbytes

    def _stop_worker(self) -> None:
        if self._thread is None:
            return
        with self._cv:
            self._stop = True
            self._cv.notify_all()
        if self._thread is not threading.current_thread():
            self._thread.join(timeout=120)
        self._thread, self._stop = None, False

    def resize(self, resident: int, ring: int = 3, *, lock_host: bool = True, ram_headroom_bytes: int = 3 * _GIB) -> int:
        """Between forwards: change the resident prefix and the number of ring slots, keeping every host source
        (h3turbo/h3/stream.py:484-551).  resize(0, 0) parks the provider (no device memory; acquiring a streamed
        block raises until the next resize).  lock_host: blocks leaving HBM get a page-locked host copy while free
        RAM stays above ram_headroom_bytes.  Returns the device bytes now held."""
        if self._closed:
            raise RuntimeError("StreamingProvider is closed")
        if self._in_forward:
            raise RuntimeError("resize() during a forward")
        self._stop_worker()
        if self._gpu:
            torch.cuda.synchronize(self.device)  # copies into slots and out of staging buffers are done
        n = self.n_blocks
        resident = max(0, min(int(resident), n))
        with self._cv:
            self._slots, self._slot_of = [], {}
            self._pos, self._demand = -1, None
        for b in sorted(self._resident, reverse=True):
            if b >= resident:
                if lock_host:
                    self._lock_host(b, ram_headroom_bytes)
                del self._resident[b]
        if self._gpu:
            torch.cuda.empty_cache()
        for b in range(resident):
            if b not in self._resident and not self._make_resident(b):
                resident = b
                break
        for b in [b for b in self._resident if b >= resident]:
            del self._resident[b]
        self._streamed = list(range(resident, n))
        if self._streamed:
            if lock_host:
                for b in self._streamed:
                    if not self._lock_host(b, ram_headroom_bytes):
                        break
            if not self._stage and self._gpu and any(self._kind.get(b) not in ("registered", "pinned") for b in self._streamed):
                self._open_staging()
            for b in self._streamed:
                if self._kind.get(b) not in ("registered", "pinned"):
                    self._kind[b] = "staged" if self._stage else "pageable"
            self._add_slots(min(max(0, ring), len(self._streamed)), strict=False)
            if self._slots:
                self._start_worker()
        return self.device_bytes()

    def _lock_host(self, b: int, headroom: int) -> bool:
        """Give block b a page-locked host source if it has none and RAM allows; True when it has one."""
        if self._kind.get(b) in ("registered", "pinned"):
            return True
        if not self._gpu:
            return False
        if getattr(self.store, "pinned", False):
            self._kind[b] = "registered"
            return True
        try:
            if free_ram_bytes() - self.store.block_nbytes < headroom:
                return False
        except RuntimeError:
            return False
        t = self._locked_buffer()
        if t is None:
            return False
        np.copyto(t.numpy(), self.store.block_bytes(b))
        self._src[b], self._kind[b] = t, "pinned"
        return True

    @property
    def parked(self) -> bool:
        return bool(self._streamed) and not self._slots

    # ----------------------------------------------------------------------------------------- introspection
    def buffer_of(self, i: int) -> Optional[torch.Tensor]:
        """The device buffer holding block i now (resident, or a loaded ring slot), else None."""
        if i in self._resident:
            return self._resident[i][0]
        with self._cv:
            s = self._slot_of.get(i)
            return s.buf if s is not None and s.state in (READY, IDLE, ACQUIRED) else None

    def wait_prefetch(self, timeout: float = 60.0) -> None:
        """Block until the worker has nothing left to issue (the lookahead window is loaded)."""
        deadline = time.perf_counter() + timeout
        with self._cv:
            while self._thread is not None and not self._stop and self._error is None and (
                    any(s.state == PENDING for s in self._slots) or self._plan_copy(commit=False) is not None):
                left = deadline - time.perf_counter()
                if left <= 0:
                    raise TimeoutError(f"prefetch did not settle: {self._describe()}")
                self._cv.wait(min(left, 0.5))
            self._raise_if_broken()

    def _describe(self) -> str:
        return ("slots " + ", ".join(f"{s.idx}:{_STATE_NAMES[s.state]}:{s.block}" for s in self._slots)
                + f"; pos={self._pos} demand={self._demand}")

    def stats(self) -> Dict[str, object]:
        with self._cv:
            kinds: Dict[str, int] = {}
            for k in self._kind.values():
                kinds[k] = kinds.get(k, 0) + 1
            blk = self.store.block_nbytes
            return dict(self._st, resident=len(self._resident), streamed=len(self._streamed), slots=len(self._slots),
                        host_kinds=kinds, gpu_bytes=(len(self._resident) + len(self._slots)) * blk,
                        locked_host_bytes=self._locked_bytes, plan=dict(self._plan_info), state=self._describe())

    def reset_stats(self) -> None:
        with self._cv:
            self._st = self._zero_stats()

    def close(self) -> None:
        if self._closed:
            return
        with self._cv:
            self._closed = self._stop = True
            self._cv.notify_all()
        if self._thread is not None and self._thread is not threading.current_thread():
            self._thread.join(timeout=120)
        if self._gpu:
            try:
                torch.cuda.synchronize(self.device)
            except Exception:
                pass
        self._slots, self._slot_of, self._resident, self._src, self._stage = [], {}, {}, {}, []
        self._kind, self._locked_bytes = {}, 0
        if self._gpu:
            torch.cuda.empty_cache()

    def __enter__(self) -> "StreamingProvider":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
