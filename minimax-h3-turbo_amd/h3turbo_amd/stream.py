"""Weight streaming for the H3 DiT on MI355X: a resident prefix of blocks in HBM plus a ring of device slots that
are refilled by asynchronous host -> HBM copies.

Contract (kept from the reference's StreamingProvider, h3turbo/h3/stream.py:115-623, so the model loop and the
ComfyUI node drive it unchanged): the constructor and its keyword arguments, the BlockProvider protocol
(begin_forward / acquire / release / end_forward), resize / parked / buffer_of / wait_prefetch / stats / close,
the stats keys, and the error types and messages callers match on.

Design.  On MI355X the whole 4-bit stack normally fits in HBM (288 GB; resident="auto" plans that), and streaming
only matters for stacks larger than free HBM.  The engine is built around three facts of the HIP runtime:

* A copy from page-locked host memory is asynchronous for the host: hipMemcpyAsync on a side stream returns at
  once.  So the thread that runs the model schedules everything itself, inside acquire() / release(): which block
  goes into which slot, the lookahead window, the evictions.  Nothing else decides.
* Slot reuse needs no host waits.  Each slot carries two events: `landed` (recorded on the copy stream after its
  fill) and `retired` (recorded on the compute stream by release(), after every kernel that reads the slot has been
  enqueued).  A fill makes the copy stream wait for `retired`; acquire() makes the compute stream wait for `landed`.
* Only host-side work needs a thread: staging a pageable block into a page-locked buffer is a CPU memcpy, and a
  copy from pageable memory is synchronous.  A single fill thread executes the fills the model thread queues for
  such sources, in queue order, and completes a ticket per fill; acquire() waits on the ticket (the fill has been
  issued to the device -- or, on the CPU path, done).  Fills from page-locked memory (registered, pinned) are
  issued by the model thread itself, when they are scheduled: their tickets are complete at once.

Host sources per streamed block ("host kind"):
    registered  the store itself is page-locked (allocated pinned): zero-copy DMA straight from its pages
    pinned      a page-locked copy of the block made at construction (or at resize)
    staged      copied into one of two page-locked staging buffers by the fill thread, then DMA'd
    pageable    copied synchronously from pageable memory (pin=False, or no page-locked memory to be had)
Page-locked memory is always allocated pinned; existing pages are never registered.

device="cpu" runs the same scheduling with plain copies and no events, so the bookkeeping, ordering and error
paths are tested without a GPU.
"""
from __future__ import annotations

import atexit
import collections
import os
import threading
import time
import weakref
from typing import Callable, Deque, Dict, List, Optional, Sequence, Set, Tuple, Union

import numpy as np
import torch

from .types import BlockWeights

_GIB = 1 << 30
HBM_MARGIN = 512 << 20  # HBM torch does not account for (library workspaces, code objects), left free by "auto"

Transfer = Callable[[torch.Tensor, torch.Tensor, bool], None]


# ------------------------------------------------------------------------------------------------ planning
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
    """The longest prefix of resident blocks that, with min(ring, streamed) ring slots, fits in free_vram_bytes -
    reserve_bytes (h3turbo/h3/stream.py:61-71); 0 when not even the ring fits (allocating the slots then reports
    the shortage)."""
    if ring < 1:
        raise ValueError("ring must be >= 1")
    n, blk = store.n_blocks, store.block_nbytes
    room = free_vram_bytes - reserve_bytes
    if n * blk <= room:
        return n  # everything resident: no ring needed
    # with r resident and at least `ring` streamed blocks the footprint is (r + ring) blocks; fewer streamed blocks
    # than the ring means the ring shrinks to them, so the footprint is n blocks -- already excluded above
    r = min(n - ring, room // blk - ring) if n > ring else -1
    return max(0, int(r))


def plan_pinned_blocks(store, streamed: int, free_ram: int, pin_fraction: float = 0.5, headroom: int = 4 * _GIB) -> int:
    """Streamed blocks that get a page-locked host copy: within pin_fraction of free RAM, never leaving less than
    `headroom` free, two staging buffers reserved first (h3turbo/h3/stream.py:74-78)."""
    budget = min(free_ram * pin_fraction, free_ram - headroom) - 2 * store.block_nbytes
    return int(max(0, min(streamed, budget // store.block_nbytes)))


def hip_transfer(dst: torch.Tensor, src: torch.Tensor, non_blocking: bool) -> None:
    """The slot copy: host -> HBM as one hipMemcpyAsync on the current (copy) stream, through libh3k
    (replaces slot.buf.copy_(src, non_blocking) of h3turbo/h3/stream.py:346-354).  A synchronous copy waits for the
    stream.  Anything that is not host -> device falls back to torch's copy."""
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


# ------------------------------------------------------------------------------------------------ fill engine
class _Ticket:
    """The host-side completion of one queued slot fill."""

    __slots__ = ("_done", "error")

    def __init__(self):
        self._done = threading.Event()
        self.error: Optional[BaseException] = None

    def done(self) -> bool:
        return self._done.is_set()

    def wait(self, timeout: Optional[float]) -> bool:
        return self._done.wait(timeout)

    def finish(self, error: Optional[BaseException] = None) -> None:
        self.error = error
        self._done.set()


class _FillEngine:
    """One thread that runs queued fill functions in queue order and completes their tickets.  It runs in
    inference mode: slot buffers created under torch.inference_mode() (ComfyUI builds models that way) are inference
    tensors, and copies into them from another thread must run in the mode too."""

    def __init__(self, device: torch.device, on_error: Callable[[BaseException], None]):
        self._device, self._on_error = device, on_error
        self._queue: Deque[Tuple[Callable[[], None], _Ticket]] = collections.deque()
        self._cv = threading.Condition()
        self._running = False
        self._stopping = False
        self.thread = threading.Thread(target=self._main, name="h3k-fill", daemon=True)
        self.thread.start()

    def submit(self, fn: Callable[[], None]) -> _Ticket:
        ticket = _Ticket()
        with self._cv:
            if self._stopping:
                ticket.finish(RuntimeError("StreamingProvider is closed"))
                return ticket
            self._queue.append((fn, ticket))
            self._cv.notify_all()
        return ticket

    def idle(self) -> bool:
        with self._cv:
            return not self._queue and not self._running

    def drain(self, timeout: Optional[float] = None) -> bool:
        """Wait until every queued fill has run; False on timeout."""
        deadline = None if timeout is None else time.perf_counter() + timeout
        with self._cv:
            while self._queue or self._running:
                left = None if deadline is None else deadline - time.perf_counter()
                if left is not None and left <= 0:
                    return False
                self._cv.wait(left if left is not None else 1.0)
        return True

    def stop(self) -> None:
        with self._cv:
            self._stopping = True
            abandoned = list(self._queue)
            self._queue.clear()
            self._cv.notify_all()
        for _, ticket in abandoned:
            ticket.finish(RuntimeError("StreamingProvider is closed"))
        if self.thread is not threading.current_thread():
            self.thread.join(timeout=120)

    def _main(self) -> None:
        with torch.inference_mode():
            if self._device.type == "cuda":
                torch.cuda.set_device(self._device)
            while True:
                with self._cv:
                    while not self._queue and not self._stopping:
                        self._cv.wait()
                    if self._stopping:
                        return
                    fn, ticket = self._queue.popleft()
                    self._running = True
                error = None
                try:
                    fn()
                except BaseException as e:  # surfaces in the acquire() that waits for this fill, and every later one
                    error = e
                    self._on_error(e)
                ticket.finish(error)
                with self._cv:
                    self._running = False
                    self._cv.notify_all()


class _Slot:
    """One device buffer of the ring and what it holds."""

    __slots__ = ("index", "buf", "weights", "block", "ticket", "landed", "retired", "held", "used", "last_use")

    def __init__(self, index: int, buf: torch.Tensor, weights: BlockWeights):
        self.index, self.buf, self.weights = index, buf, weights
        self.block: Optional[int] = None          # the block it holds or is being filled with
        self.ticket: Optional[_Ticket] = None     # the fill of `block`
        self.landed = None                        # copy-stream event after the fill (GPU)
        self.retired = None                       # compute-stream event after the last reader (GPU)
        self.held = False                         # acquired and not yet released
        self.used = False                         # acquired since its fill: a cheap eviction candidate
        self.last_use = 0


_providers: "weakref.WeakSet[StreamingProvider]" = weakref.WeakSet()


@atexit.register
def _close_providers_at_exit() -> None:
    """A provider left open at interpreter exit must not leave its fill thread inside a device call."""
    for p in list(_providers):
        try:
            p.close()
        except Exception:
            pass


# ------------------------------------------------------------------------------------------------ provider
class StreamingProvider:
    """BlockProvider over a block store (blockstore.HostBlockStore, or any object with n_blocks, block_nbytes,
    block_tensor(i), block_bytes(i), block_weights_from(buf) and optionally `pinned`): a resident prefix of blocks
    plus a prefetching ring.  Use as a context manager or call close()."""

    def __init__(self, store, device: Union[str, torch.device] = "cuda", resident: Union[int, str] = "auto",
                 prefetch: int = 2, pin: Union[bool, str] = "auto", ring: int = 3, *, reserve_bytes: int = 1536 << 20,
                 free_vram_bytes: Optional[int] = None, pin_fraction: float = 0.5, ram_headroom_bytes: int = 4 * _GIB,
                 pin_blocks: Optional[int] = None, pin_mode: str = "auto", transfer: Optional[Transfer] = None,
                 wait_timeout: float = 600.0):
        if ring < 1 or prefetch < 0 or pin not in (True, False, "auto") or pin_mode not in ("auto", "register", "copy",
                                                                                             "stage"):
            raise ValueError("ring >= 1, prefetch >= 0, pin in (True, False, 'auto'), "
                             "pin_mode in ('auto', 'register', 'copy', 'stage')")
        if not (resident == "auto" or (isinstance(resident, int) and not isinstance(resident, bool) and resident >= 0)):
            raise ValueError("resident must be 'auto' or a non-negative int")
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.store, self.device, self._gpu = store, dev, dev.type == "cuda"
        self.n_blocks = store.n_blocks
        self._prefetch, self._timeout = prefetch, wait_timeout
        self._transfer: Transfer = transfer or (hip_transfer if self._gpu else (lambda d, s, nb: d.copy_(s)))
        self._lock = threading.Lock()
        self._resident: Dict[int, Tuple[torch.Tensor, BlockWeights]] = {}
        self._slots: List[_Slot] = []
        self._holder: Dict[int, _Slot] = {}       # block -> the slot that holds (or is being filled with) it
        self._streamed: List[int] = []
        self._source: Dict[int, Tuple[str, Optional[torch.Tensor]]] = {}  # block -> (host kind, locked copy)
        self._staging: List[torch.Tensor] = []
        self._staging_free: List[Optional[object]] = []  # per staging buffer: the event of its last copy out
        self._staging_next = 0
        self._locked_bytes = 0
        self._cursor = -1                          # position in _streamed of the last acquired block
        self._clock = 0
        self._in_forward = self._closed = False
        self._error: Optional[BaseException] = None
        self._plan: Dict[str, object] = {}
        self._counts = self._zero_counts()
        self._copy_stream = torch.cuda.Stream(dev) if self._gpu else None
        self._engine: Optional[_FillEngine] = None
        _providers.add(self)
        try:
            self._setup(resident, ring, pin, pin_mode, reserve_bytes, free_vram_bytes, pin_fraction,
                        ram_headroom_bytes, pin_blocks)
        except BaseException:
            self.close()
            raise

    @staticmethod
    def _zero_counts() -> Dict[str, float]:
        return dict(acquires=0, waits=0, wait_s=0.0, copies=0, bytes=0, busy_s=0.0)

    # ------------------------------------------------------------------------------ construction
    def _device_block(self) -> torch.Tensor:
        return torch.empty(self.store.block_nbytes, dtype=torch.uint8, device=self.device)

    def _locked_block(self) -> Optional[torch.Tensor]:
        """A page-locked host buffer of one block (plain memory on the CPU path); None when none can be had."""
        if not self._gpu:
            return torch.empty(self.store.block_nbytes, dtype=torch.uint8)
        try:
            buf = torch.empty(self.store.block_nbytes, dtype=torch.uint8, pin_memory=True)
        except RuntimeError:
            return None
        self._locked_bytes += self.store.block_nbytes
        return buf

    def _host_bytes(self, b: int) -> torch.Tensor:
        kind, copy = self._source.get(b, ("pageable", None))
        return copy if copy is not None else self.store.block_tensor(b)

    def _setup(self, resident, ring, pin, pin_mode, reserve, free_vram, pin_fraction, headroom, pin_blocks) -> None:
        n = self.n_blocks
        auto = resident == "auto"
        if auto:
            if free_vram is None:
                free_vram = torch.cuda.mem_get_info(self.device)[0] if self._gpu else free_ram_bytes() // 2
            resident = plan_residency(self.store, free_vram, reserve + (HBM_MARGIN if self._gpu else 0), ring)
        for b in range(min(int(resident), n)):
            try:
                buf = self._device_block()
            except torch.cuda.OutOfMemoryError:
                if auto:
                    break  # the plan was optimistic: the rest streams
                raise
            buf.copy_(self.store.block_tensor(b))  # synchronous; the store is the source of truth
            self._resident[b] = (buf, self.store.block_weights_from(buf))
        self._streamed = list(range(len(self._resident), n))
        self._make_slots(min(ring, len(self._streamed)), all_or_error=True)
        if self._streamed:
            self._choose_sources(pin, pin_mode, pin_fraction, headroom, pin_blocks)
            self._engine = _FillEngine(self.device, self._fail)

    def _make_slots(self, count: int, all_or_error: bool) -> None:
        for k in range(count):
            try:
                buf = self._device_block()
            except torch.cuda.OutOfMemoryError as e:
                if k and not all_or_error:
                    break
                raise torch.cuda.OutOfMemoryError(
                    f"cannot allocate streaming slot {k + 1} of {count} ({self.store.block_nbytes / 2**20:.0f} MiB): "
                    "lower resident/ring or free HBM") from e
            self._slots.append(_Slot(k, buf, self.store.block_weights_from(buf)))

    def _choose_sources(self, pin, pin_mode, pin_fraction, headroom, pin_blocks) -> None:
        """Each streamed block's host source (the policy of h3turbo/h3/stream.py:219-268; existing pages are never
        page-locked here, so "register" means the store's own pinned pages or nothing)."""
        streamed = self._streamed
        if self._gpu and pin is not False and getattr(self.store, "pinned", False):
            self._source.update({b: ("registered", None) for b in streamed})
            return
        if pin is False or pin_mode in ("stage", "register"):
            copies = 0
        elif pin is True:
            copies = len(streamed)
        elif pin_blocks is not None:
            copies = max(0, min(len(streamed), pin_blocks))
        elif self._gpu:
            avail = free_ram_bytes()
            self._plan["ram_available_gib"] = round(avail / _GIB, 2)
            copies = plan_pinned_blocks(self.store, len(streamed), avail, pin_fraction, headroom)
        else:
            copies = 0
        self._plan["pinned_wanted"] = copies
        for b in streamed[:copies]:
            if not self._pin_copy(b):
                break  # out of page-locked memory: the rest is staged
        rest = [b for b in streamed if b not in self._source]
        use_staging = bool(rest) and pin is not False and (
            pin is True or copies > 0 or pin_mode in ("stage", "register") or (pin == "auto" and self._gpu))
        if use_staging:
            self._open_staging()
        for b in rest:
            self._source[b] = ("staged" if self._staging else "pageable", None)

    def _pin_copy(self, b: int) -> bool:
        buf = self._locked_block()
        if buf is None:
            return False
        np.copyto(buf.numpy(), self.store.block_bytes(b))
        self._source[b] = ("pinned", buf)
        return True

    def _open_staging(self) -> None:
        while len(self._staging) < 2:
            buf = self._locked_block()
            if buf is None:
                break
            self._staging.append(buf)
            self._staging_free.append(None)

    # ------------------------------------------------------------------------------ fills
    def _fail(self, error: BaseException) -> None:
        with self._lock:
            if self._error is None:
                self._error = error

    def _run_fill(self, slot: _Slot, b: int, retired) -> None:
        """Executed by the fill thread: the host side of the copy, then the copy itself."""
        t0 = time.perf_counter()
        self._copy_into(slot, b, retired)
        with self._lock:
            self._count_fill(time.perf_counter() - t0)

    def _count_fill(self, busy: float) -> None:
        self._counts["copies"] += 1
        self._counts["bytes"] += self.store.block_nbytes
        self._counts["busy_s"] += busy

    def _copy_into(self, slot: _Slot, b: int, retired) -> None:
        """The host side of block b's copy into slot (staging, when its source needs it), then the copy, ordered
        after the slot's last reader on the device (`retired`)."""
        kind, copy = self._source[b]
        stage = None
        if kind == "staged":
            stage = self._staging_next
            self._staging_next = (stage + 1) % len(self._staging)
            if self._staging_free[stage] is not None:
                self._staging_free[stage].synchronize()  # its previous copy out must be over before it is refilled
            np.copyto(self._staging[stage].numpy(), self.store.block_bytes(b))  # numpy's memcpy releases the GIL
            src = self._staging[stage]
        elif kind == "pageable":
            src = self.store.block_tensor(b)
        else:
            src = copy if copy is not None else self.store.block_tensor(b)
        if self._gpu:
            cs = self._copy_stream
            with torch.cuda.stream(cs):
                if retired is not None:
                    cs.wait_event(retired)  # on the device: the slot's last reader has finished
                self._transfer(slot.buf, src, kind != "pageable")
                landed = torch.cuda.Event()
                landed.record(cs)
            slot.landed = landed
            if stage is not None:
                self._staging_free[stage] = landed
        else:
            self._transfer(slot.buf, src, False)

    def _fill(self, slot: _Slot, b: int) -> None:
        """Queue block b into slot (lock held).  The slot forgets its previous block at once; its copy is ordered
        after the slot's last reader on the device.  From page-locked memory the copy is only enqueued on the copy
        stream, with no host work, so this thread issues it at once: handed to the fill thread it waited until that
        thread was scheduled behind the caller's Python work, and acquire() then found the copy of a prefetched
        block not yet issued.  Sources that need host work (staging, pageable) go to the fill thread."""
        if slot.block is not None and self._holder.get(slot.block) is slot:
            del self._holder[slot.block]
        slot.block, slot.used = b, False
        self._holder[b] = slot
        if self._gpu and self._source[b][0] in ("registered", "pinned"):
            ticket = _Ticket()
            t0 = time.perf_counter()
            try:
                self._copy_into(slot, b, slot.retired)
            except BaseException as e:  # surfaces in this acquire() and every later one, as a fill-thread error does
                if self._error is None:
                    self._error = e
                ticket.finish(e)
            else:
                self._count_fill(time.perf_counter() - t0)
                ticket.finish()
            slot.ticket = ticket
            return
        slot.ticket = self._engine.submit(lambda s=slot, blk=b, ev=slot.retired: self._run_fill(s, blk, ev))

    def _window(self) -> List[int]:
        """The streamed blocks expected next: the cyclic lookahead after the last acquired one."""
        s = self._streamed
        return [s[(self._cursor + 1 + k) % len(s)] for k in range(min(self._prefetch, len(s)))]

    def _spare_slot(self, keep: Set[int]) -> Optional[_Slot]:
        """A slot that may be refilled (lock held): an empty one; else, least recently used first, one whose block
        was already used; else one prefetched for a block nobody is about to ask for.  Never a held slot and never
        one holding a block in `keep`."""
        empty = [s for s in self._slots if s.block is None]
        if empty:
            return empty[0]
        free = [s for s in self._slots if not s.held and s.block not in keep]
        if not free:
            return None
        return min(free, key=lambda s: (not s.used, s.last_use))

    def _top_up(self) -> None:
        """Queue the lookahead window's missing blocks into spare slots (lock held)."""
        window = self._window()
        keep = set(window) | {s.block for s in self._slots if s.held}
        for b in window:
            if b in self._holder:
                continue
            slot = self._spare_slot(keep)
            if slot is None:
                break
            self._fill(slot, b)

    # ------------------------------------------------------------------------------ BlockProvider
    def _check_usable(self) -> None:
        if self._closed:
            raise RuntimeError("StreamingProvider is closed")
        if self._error is not None:
            raise RuntimeError(f"H3 streaming worker failed: {self._error!r}") from self._error

    def begin_forward(self) -> None:
        if self._in_forward:  # the previous forward never reached end_forward (an exception without finally)
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
        with self._lock:
            self._check_usable()
            slot = self._holder.get(i)
            if slot is None:
                if all(s.held for s in self._slots):
                    raise RuntimeError(f"all {len(self._slots)} ring slots are held; release() a block before "
                                       f"acquiring block {i} (ring too small?)")
                slot = self._spare_slot(keep={s.block for s in self._slots if s.held})
                self._fill(slot, i)
            elif slot.held:
                raise RuntimeError(f"block {i} is already acquired")
            slot.held = True
            self._clock += 1
            slot.last_use = self._clock
            self._cursor = self._streamed.index(i)
            ticket = slot.ticket
            self._top_up()
        waited = not ticket.done()
        if waited and not ticket.wait(self._timeout):
            raise TimeoutError(f"timed out after {self._timeout:.0f}s waiting for block {i}: {self._describe()}")
        if ticket.error is not None:
            raise RuntimeError(f"H3 streaming worker failed: {ticket.error!r}") from ticket.error
        with self._lock:
            self._counts["acquires"] += 1
            if waited:
                self._counts["waits"] += 1
                self._counts["wait_s"] += time.perf_counter() - t0
        if self._gpu and slot.landed is not None:
            torch.cuda.current_stream(self.device).wait_event(slot.landed)
        return slot.weights

    def _retire_event(self):
        """An event after every kernel enqueued so far on the compute stream (GPU), else None."""
        if not self._gpu:
            return None
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        return ev

    def release(self, i: int) -> None:
        if i in self._resident:
            return
        ev = self._retire_event()
        with self._lock:
            slot = self._holder.get(i)
            if slot is None or not slot.held:
                raise RuntimeError(f"release({i}) but block {i} is not acquired")
            slot.held, slot.used, slot.retired = False, True, ev
            self._clock += 1
            slot.last_use = self._clock
            if self._error is None and not self._closed:
                self._top_up()

    def end_forward(self) -> None:
        """Reset for the next forward (safe after an exception): held slots are released behind an event on the
        current stream and the lookahead restarts at the first streamed block."""
        ev = self._retire_event() if not self._closed else None
        with self._lock:
            for s in self._slots:
                if s.held:
                    s.held, s.used, s.retired = False, True, ev
            self._cursor = -1
            self._in_forward = False
            if self._slots and self._error is None and not self._closed:
                self._top_up()

    # ------------------------------------------------------------------------------ residency changes
    def device_bytes(self) -> int:
        return (len(self._resident) + len(self._slots)) * self.store.block_nbytes

    @property
    def resident_count(self) -> int:
        """Blocks held in HBM for good (the leading ones)."""
        return len(self._resident)

    @property
    def ring_count(self) -> int:
        """Ring slots the streamed blocks rotate through (0 when parked or nothing streams)."""
        return len(self._slots)

    def resize(self, resident: int, ring: int = 3, *, lock_host: bool = True, ram_headroom_bytes: int = 3 * _GIB) -> int:
        """Change how many leading blocks live in HBM and how many ring slots exist, between forwards, keeping the
        host side (page-locked copies, staging buffers) so nothing is re-read from the store.  resize(r, 0) with
        blocks left to stream parks the provider: no ring slots, and acquiring a streamed block raises until the next
        resize.  lock_host: blocks leaving HBM, and streamed blocks without a page-locked source, get a page-locked
        host copy while free RAM stays above ram_headroom_bytes.  Returns the HBM bytes now held."""
        if self._closed:
            raise RuntimeError("StreamingProvider is closed")
        if self._in_forward:
            raise RuntimeError("resize() during a forward")
        if self._engine is not None:
            self._engine.drain()
        if self._gpu:
            torch.cuda.synchronize(self.device)  # fills into slots and copies out of staging buffers are over
        n, blk = self.n_blocks, self.store.block_nbytes
        want = max(0, min(int(resident), n))
        with self._lock:
            self._slots, self._holder, self._cursor = [], {}, -1
        for b in [b for b in self._resident if b >= want]:
            if lock_host:
                self._lock_host(b, ram_headroom_bytes)
            del self._resident[b]
        if self._gpu:
            torch.cuda.empty_cache()
        for b in range(want):
            if b in self._resident:
                continue
            try:
                buf = self._device_block()
            except torch.cuda.OutOfMemoryError:
                want = b
                break
            buf.copy_(self._host_bytes(b))
            self._resident[b] = (buf, self.store.block_weights_from(buf))
        for b in [b for b in self._resident if b >= want]:  # an allocation failure above cut the prefix short
            del self._resident[b]
        self._streamed = list(range(want, n))
        if self._streamed:
            if lock_host:
                for b in self._streamed:
                    if not self._lock_host(b, ram_headroom_bytes):
                        break
            unlocked = [b for b in self._streamed if self._source.get(b, ("pageable", None))[0] not in ("registered",
                                                                                                       "pinned")]
            if unlocked and self._gpu and not self._staging:
                self._open_staging()
            for b in unlocked:
                self._source[b] = ("staged" if self._staging else "pageable", None)
            self._make_slots(min(max(0, ring), len(self._streamed)), all_or_error=False)
            if self._slots and self._engine is None:
                self._engine = _FillEngine(self.device, self._fail)
        return self.device_bytes()

    def _lock_host(self, b: int, headroom: int) -> bool:
        """Give block b a page-locked host source if free RAM allows; True when it has one."""
        kind = self._source.get(b, ("pageable", None))[0]
        if kind in ("registered", "pinned"):
            return True
        if self._gpu and getattr(self.store, "pinned", False):
            self._source[b] = ("registered", None)
            return True
        if not self._gpu:
            return False
        try:
            if free_ram_bytes() - self.store.block_nbytes < headroom:
                return False
        except RuntimeError:
            return False
        return self._pin_copy(b)

    @property
    def parked(self) -> bool:
        return bool(self._streamed) and not self._slots

    # ------------------------------------------------------------------------------ introspection / lifecycle
    def buffer_of(self, i: int) -> Optional[torch.Tensor]:
        """The device buffer that holds block i (resident, or a ring slot whose fill has been issued), else None."""
        if i in self._resident:
            return self._resident[i][0]
        with self._lock:
            s = self._holder.get(i)
            if s is None or s.ticket is None or not s.ticket.done() or s.ticket.error is not None:
                return None
            return s.buf

    def wait_prefetch(self, timeout: float = 60.0) -> None:
        """Block until every queued fill has been issued (the lookahead window is loaded)."""
        if self._engine is not None and not self._engine.drain(timeout):
            raise TimeoutError(f"prefetch did not settle: {self._describe()}")
        with self._lock:
            self._check_usable()

    def _describe(self) -> str:
        def one(s: _Slot) -> str:
            state = "held" if s.held else ("empty" if s.block is None else
                                           ("filling" if s.ticket is not None and not s.ticket.done() else "ready"))
            return f"{s.index}:{state}:{s.block}"

        return "slots " + ", ".join(one(s) for s in self._slots) + f"; cursor={self._cursor}"

    def stats(self) -> Dict[str, object]:
        with self._lock:
            kinds: Dict[str, int] = {}
            for b in self._streamed:
                k = self._source.get(b, ("pageable", None))[0]
                kinds[k] = kinds.get(k, 0) + 1
            return dict(self._counts, resident=len(self._resident), streamed=len(self._streamed),
                        slots=len(self._slots), host_kinds=kinds, gpu_bytes=self.device_bytes(),
                        locked_host_bytes=self._locked_bytes, plan=dict(self._plan), state=self._describe())

    def reset_stats(self) -> None:
        with self._lock:
            self._counts = self._zero_counts()

    def close(self) -> None:
        if self._closed:
            return
        self._closed = True
        if self._engine is not None:
            self._engine.stop()
        if self._gpu:
            try:
                torch.cuda.synchronize(self.device)
            except Exception:
                pass
        self._slots, self._holder, self._resident = [], {}, {}
        self._source, self._staging, self._staging_free = {}, [], []
        if self._gpu:
            torch.cuda.empty_cache()

    def __enter__(self) -> "StreamingProvider":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
