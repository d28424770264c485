"""Streaming engine and block store on the CPU path: slot ring, prefetch, hazards, error paths, planning.

The device="cpu" provider runs the same state machine as on the GPU with plain copies; the `transfer` hook
injects latency and faults from the host (a slow copy, a copy that raises, a copy stuck behind a gate) so every
kernel-free path is exercised here.  The GPU variants are in test_gpu_stream.py.
"""
import dataclasses
import threading
import time
from types import SimpleNamespace

import pytest
import torch

from h3turbo_amd.blockstore import BlockLayout, HostBlockStore, block_tensors
from h3turbo_amd.stream import StreamingProvider, free_ram_bytes, plan_pinned_blocks, plan_residency
from h3turbo_amd.types import BlockWeights, W4A8Weight

LAYERS = 6


def tiny_block(seed: int, hidden=64, inner=64, ffn=48) -> BlockWeights:
    g = torch.Generator().manual_seed(seed)

    def lin(n, k):
        q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8)
        s = (torch.rand(n, k // 16, generator=g) * 180 + 20).to(torch.float8_e4m3fn)
        return W4A8Weight(q, s, torch.rand(n, generator=g) * 0.02, torch.randn(16, generator=g), 16, 16)

    return BlockWeights(qkv=lin(3 * inner, hidden), out=lin(hidden, inner), fc1=lin(2 * ffn, hidden), fc2=lin(hidden, ffn),
                        norm1=torch.randn(hidden, generator=g).bfloat16(), norm2=torch.randn(hidden, generator=g).bfloat16(),
                        q_norm=torch.randn(32, generator=g).bfloat16(), k_norm=torch.randn(32, generator=g).bfloat16(),
                        adaln_w=torch.randn(18 * hidden, 8, generator=g).bfloat16(), adaln_b=torch.randn(18 * hidden, generator=g))


def raw(t: torch.Tensor) -> bytes:
    return t.detach().cpu().contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()


def tensors_of(w: BlockWeights):
    out = []
    for f in dataclasses.fields(w):
        v = getattr(w, f.name)
        out += [v.q, v.s_rel, v.s_ch, v.codebook] if isinstance(v, W4A8Weight) else [v]
    return out


def same(a: BlockWeights, b: BlockWeights) -> bool:
    for x, y in zip(tensors_of(a), tensors_of(b)):
        if x is None or y is None:
            if x is not y:
                return False
        elif (x.dtype, tuple(x.shape)) != (y.dtype, tuple(y.shape)) or raw(x) != raw(y):
            return False
    return True


@pytest.fixture(scope="module")
def blocks():
    return [tiny_block(100 + i) for i in range(LAYERS)]


@pytest.fixture(scope="module")
def store(blocks):
    return HostBlockStore.from_blocks(blocks)


def forward(p, store, compute=None, check=True):
    p.begin_forward()
    try:
        for i in range(p.n_blocks):
            w = p.acquire(i)
            if check:
                assert same(w, store.block_weights_cpu(i)), f"block {i} differs from the store"
            if compute:
                compute(i, w)
            p.release(i)
    finally:
        p.end_forward()


def no_slot_held(p):
    return all(not s.held for s in p._slots)


# ------------------------------------------------------------------------------------------------ block store
def test_layout_alignment_and_round_trip(blocks, store):
    lay = store.layout
    assert store.block_nbytes % 4096 == 0
    assert all(e.offset % 256 == 0 for e in lay.entries)
    assert store.n_blocks == LAYERS
    for i, b in enumerate(blocks):
        assert same(store.block_weights_cpu(i), b)
        got = block_tensors(store.block_weights_cpu(i))
        assert list(got) == lay.names()
    # views are zero-copy: writing through one changes the block bytes
    buf = store.block_tensor(0).clone()
    w = store.block_weights_from(buf)
    w.norm1[0] = 123.0
    assert lay.view(buf, "norm1.weight")[0].item() == 123.0
    with pytest.raises(ValueError, match="1-D uint8"):
        store.block_weights_from(buf[:-1])
    with pytest.raises(IndexError):
        store.block_tensor(LAYERS)
    with pytest.raises(ValueError, match="do not match"):
        lay.pack_into(buf, {"norm1.weight": blocks[0].norm1})


def test_dense_linears_and_missing_adaln_round_trip():
    g = torch.Generator().manual_seed(3)
    b = BlockWeights(qkv=torch.randn(12, 8, generator=g), out=torch.randn(8, 4, generator=g), fc1=torch.randn(6, 8, generator=g),
                     fc2=torch.randn(8, 3, generator=g), norm1=torch.ones(8), norm2=torch.ones(8), q_norm=torch.ones(2),
                     k_norm=torch.ones(2))
    st = HostBlockStore.from_blocks([b, b])
    w = st.block_weights_cpu(1)
    assert same(w, b) and w.adaln_w is None and isinstance(w.qkv, torch.Tensor)


# ------------------------------------------------------------------------------------------------ planning
def test_plan_residency_known_answers():
    st = SimpleNamespace(block_nbytes=100, n_blocks=50)
    assert plan_residency(st, 5000, 0, 3) == 50
    assert plan_residency(st, 4999, 0, 3) == 46
    assert plan_residency(st, 5000, 1000, 3) == 37
    assert plan_residency(st, 5000, 0, 1) == 50 and plan_residency(st, 4999, 0, 1) == 48
    assert plan_residency(st, 250, 0, 3) == 0
    assert plan_residency(st, 100_000, 0, 3) == 50
    two = SimpleNamespace(block_nbytes=100, n_blocks=2)
    assert plan_residency(two, 150, 0, 3) == 0
    assert plan_residency(two, 200, 0, 3) == 2
    assert plan_residency(SimpleNamespace(block_nbytes=100, n_blocks=10), 700, 0, 3) == 4
    with pytest.raises(ValueError):
        plan_residency(st, 1, 0, 0)


def test_plan_residency_is_the_largest_prefix_that_fits_brute_force():
    for n in range(0, 9):
        for ring in (1, 2, 3, 5):
            for room in range(0, 1200, 37):
                st = SimpleNamespace(block_nbytes=100, n_blocks=n)
                fits = [r for r in range(n + 1) if (r + min(ring, n - r)) * 100 <= room]
                assert plan_residency(st, room, 0, ring) == (max(fits) if fits else 0)


def test_plan_pinned_blocks_respects_free_ram():
    st = SimpleNamespace(block_nbytes=100)
    assert plan_pinned_blocks(st, 10, 1000, 0.5, 0) == 3
    assert plan_pinned_blocks(st, 2, 1000, 0.5, 0) == 2
    assert plan_pinned_blocks(st, 10, 1000, 0.5, 900) == 0
    assert plan_pinned_blocks(st, 10, 100, 0.5, 0) == 0
    assert free_ram_bytes() > 0


# ------------------------------------------------------------------------------------------------ exactness
@pytest.mark.parametrize("resident", [0, 1, 3, 6])
@pytest.mark.parametrize("ring,prefetch", [(1, 0), (1, 2), (2, 1), (3, 2), (4, 5)])
def test_streaming_equals_the_store_over_many_forwards(store, resident, ring, prefetch):
    with StreamingProvider(store, "cpu", resident=resident, prefetch=prefetch, pin=False, ring=ring) as p:
        assert p.stats()["resident"] == resident and p.stats()["slots"] == min(ring, LAYERS - resident)
        for _ in range(3):
            forward(p, store)
            assert no_slot_held(p)


@pytest.mark.parametrize("kwargs,kinds", [
    (dict(pin=False), {"pageable": 4}),
    (dict(pin=True), {"pinned": 4}),
    (dict(pin="auto", pin_blocks=1), {"pinned": 1, "staged": 3}),
    (dict(pin="auto", pin_blocks=9), {"pinned": 4}),
    (dict(pin="auto", pin_mode="stage"), {"staged": 4}),
    (dict(pin="auto"), {"pageable": 4}),  # nothing to page-lock on the CPU path
])
def test_host_source_modes_are_all_exact(store, kwargs, kinds):
    with StreamingProvider(store, "cpu", resident=2, prefetch=2, ring=3, **kwargs) as p:
        assert p.stats()["host_kinds"] == kinds
        for _ in range(2):
            forward(p, store)


def test_device_bytes_equal_store_bytes(store):
    with StreamingProvider(store, "cpu", resident=2, prefetch=2, ring=3, pin=True) as p:
        forward(p, store)
        p.wait_prefetch()
        seen = 0
        for i in range(LAYERS):
            buf = p.buffer_of(i)
            if buf is not None:
                seen += 1
                assert buf.dtype == torch.uint8 and raw(buf) == bytes(store.block_bytes(i)), i
        assert seen >= 2 + 2


def test_cross_forward_prefetch_warms_the_next_forward(store):
    with StreamingProvider(store, "cpu", resident=2, prefetch=2, ring=3, pin=True) as p:
        forward(p, store)
        p.wait_prefetch()
        assert p.buffer_of(2) is not None and p.buffer_of(3) is not None
        c0 = p.stats()["copies"]
        forward(p, store)
        p.wait_prefetch()
        assert p.stats()["copies"] - c0 == LAYERS - 2


def test_ring_that_holds_every_streamed_block_copies_once(store):
    with StreamingProvider(store, "cpu", resident=3, prefetch=2, ring=3, pin=True) as p:
        for _ in range(4):
            forward(p, store)
        p.wait_prefetch()
        assert p.stats()["copies"] == 3


def test_resident_auto_uses_the_plan(store):
    blk = store.block_nbytes
    for free_blocks, ring in ((4.5, 3), (100, 3), (2.5, 2)):
        want = plan_residency(store, int(free_blocks * blk), 0, ring)
        with StreamingProvider(store, "cpu", resident="auto", free_vram_bytes=int(free_blocks * blk), reserve_bytes=0,
                               ring=ring, pin=False) as p:
            assert p.stats()["resident"] == want
            forward(p, store)


# ------------------------------------------------------------------------------------------------ hazards and ordering
def test_no_slot_is_written_while_the_model_holds_it(store):
    holder, log = {}, []
    ready = threading.Event()  # the worker starts prefetching inside the constructor, before `p` exists

    def hook(dst, src, nb):
        assert ready.wait(10)
        p = holder["p"]
        slot = next(s for s in p._slots if s.buf is dst)
        b = next(b for b in range(LAYERS) if p.store.block_tensor(b).data_ptr() == src.data_ptr())
        # a copy writes only the block its slot is assigned to, and a held slot only while its acquire() still waits
        # for this very fill (the model has not been handed the weights yet)
        assert slot.block == b, f"copy of block {b} into slot {slot.index} assigned to block {slot.block}"
        assert not slot.held or not slot.ticket.done(), f"copy into slot {slot.index} while the model reads it"
        log.append(slot.index)
        time.sleep(0.003)
        dst.copy_(src)

    with StreamingProvider(store, "cpu", resident=0, prefetch=3, ring=3, pin=False, transfer=hook) as p:
        holder["p"] = p
        ready.set()
        p.begin_forward()
        held = [p.acquire(0), p.acquire(1)]
        expect = [raw(t) for w in held for t in tensors_of(w)]
        time.sleep(0.15)
        assert [raw(t) for w in held for t in tensors_of(w)] == expect
        assert sum(s.held for s in p._slots) == 2
        with pytest.raises(RuntimeError, match="already acquired"):
            p.acquire(0)
        third = p.acquire(2)
        with pytest.raises(RuntimeError, match="ring slots are held"):
            p.acquire(3)
        for i in (0, 1, 2):
            p.release(i)
        assert same(third, store.block_weights_cpu(2))
        for i in range(3, LAYERS):
            assert same(p.acquire(i), store.block_weights_cpu(i))
            p.release(i)
        p.end_forward()
    assert len(log) >= LAYERS


def test_acquire_waits_for_a_slow_copy(store):
    def slow(dst, src, nb):
        time.sleep(0.05)
        dst.copy_(src)

    with StreamingProvider(store, "cpu", resident=0, prefetch=1, ring=2, pin=False, transfer=slow) as p:
        t0 = time.perf_counter()
        forward(p, store)
        assert time.perf_counter() - t0 >= 0.05 * LAYERS * 0.9
        assert p.stats()["waits"] >= 1 and p.stats()["wait_s"] > 0


def test_copies_overlap_compute(store):
    def slow(dst, src, nb):
        time.sleep(0.04)
        dst.copy_(src)

    def compute(i, w):
        time.sleep(0.04)

    def timed(**kw):
        with StreamingProvider(store, "cpu", resident=0, pin=False, transfer=slow, **kw) as p:
            forward(p, store, compute, check=False)
            p.wait_prefetch()
            t0 = time.perf_counter()
            forward(p, store, compute, check=False)
            return time.perf_counter() - t0

    serial = timed(prefetch=0, ring=1)
    overlapped = timed(prefetch=2, ring=3)
    assert serial > 0.04 * 2 * LAYERS * 0.9
    assert overlapped < 0.8 * serial, (overlapped, serial)


@pytest.mark.parametrize("call_end", [True, False])
def test_exception_mid_forward_resets_state(store, call_end):
    with StreamingProvider(store, "cpu", resident=1, prefetch=2, ring=3, pin=True) as p:
        forward(p, store)
        for stop_at in (0, 1, 4):
            with pytest.raises(ZeroDivisionError):
                p.begin_forward()
                for i in range(LAYERS):
                    p.acquire(i)
                    if i == stop_at:
                        1 / 0
                    p.release(i)
            if call_end:
                p.end_forward()
                assert no_slot_held(p)
            forward(p, store)
            assert no_slot_held(p)
        p.wait_prefetch()


def test_out_of_order_and_repeated_access(store):
    with StreamingProvider(store, "cpu", resident=1, prefetch=2, ring=2, pin=False) as p:
        p.begin_forward()
        for i in (5, 1, 1, 4, 2, 5, 3, 3):
            assert same(p.acquire(i), store.block_weights_cpu(i)), i
            p.release(i)
        with pytest.raises(RuntimeError, match="not acquired"):
            p.release(2)
        with pytest.raises(IndexError):
            p.acquire(LAYERS)
        p.end_forward()
        forward(p, store)


def test_worker_error_surfaces_and_provider_still_closes(store):
    n = {"calls": 0}

    def flaky(dst, src, nb):
        n["calls"] += 1
        if n["calls"] == 3:
            raise OSError("disk fell off")
        dst.copy_(src)

    p = StreamingProvider(store, "cpu", resident=0, prefetch=1, ring=2, pin=False, transfer=flaky)
    with pytest.raises(RuntimeError, match="disk fell off"):
        for _ in range(3):
            forward(p, store, check=False)
    p.close()
    assert not p._engine.thread.is_alive()


def test_wait_timeout_reports_state(store):
    gate = threading.Event()

    def stuck(dst, src, nb):
        gate.wait(10)
        dst.copy_(src)

    p = StreamingProvider(store, "cpu", resident=0, prefetch=1, ring=2, pin=False, transfer=stuck, wait_timeout=0.3)
    try:
        p.begin_forward()
        with pytest.raises(TimeoutError, match="block 0"):
            p.acquire(0)
    finally:
        gate.set()
        p.close()


def test_close_is_idempotent_joins_and_blocks_further_use(store):
    p = StreamingProvider(store, "cpu", resident=1, prefetch=2, ring=2, pin=True)
    forward(p, store)
    th = p._engine.thread
    p.close()
    p.close()
    assert not th.is_alive()
    for i in (3, 0):
        with pytest.raises(RuntimeError, match="closed"):
            p.acquire(i)


def test_all_resident_needs_no_worker(store):
    with StreamingProvider(store, "cpu", resident=LAYERS) as p:
        assert p._engine is None and p.stats()["slots"] == 0
        forward(p, store)
        forward(p, store)


def test_stats_counters(store):
    with StreamingProvider(store, "cpu", resident=2, prefetch=2, ring=3, pin=True) as p:
        p.reset_stats()
        forward(p, store)
        p.wait_prefetch()
        s = p.stats()
        assert s["acquires"] == LAYERS - 2 and s["bytes"] == s["copies"] * store.block_nbytes and s["copies"] >= LAYERS - 2
        assert s["gpu_bytes"] == (2 + 3) * store.block_nbytes


def test_constructor_validation(store):
    for kw in (dict(ring=0), dict(prefetch=-1), dict(pin="maybe"), dict(pin_mode="x"), dict(resident=-1),
               dict(resident="some")):
        with pytest.raises(ValueError):
            StreamingProvider(store, "cpu", **kw)


@pytest.mark.parametrize("inference", [True, False])
def test_provider_works_when_built_inside_inference_mode(store, inference):
    with torch.inference_mode(inference):
        p = StreamingProvider(store, "cpu", resident=1, ring=2, prefetch=1, pin=False, wait_timeout=20)
    try:
        for _ in range(3):
            forward(p, store)
        assert no_slot_held(p)
    finally:
        p.close()


@pytest.mark.parametrize("plan", [[(2, 3), (0, 0), (2, 3)], [(3, 2), (1, 0), (4, 3), (6, 3)], [(6, 0), (0, 0), (0, 1)],
                                  [(1, 3), (5, 2), (0, 0), (3, 3)]])
def test_resize_keeps_every_block_exact(store, plan):
    with StreamingProvider(store, "cpu", resident=plan[0][0], prefetch=2, ring=max(1, plan[0][1]), pin="auto") as p:
        forward(p, store)
        for resident, ring in plan[1:]:
            held = p.resize(resident, ring)
            assert held == p.device_bytes()
            st = p.stats()
            assert st["resident"] == resident
            if resident < LAYERS and ring == 0:
                assert p.parked
                p.begin_forward()
                if resident < LAYERS:
                    with pytest.raises(RuntimeError, match="parked"):
                        p.acquire(resident)
                p.end_forward()
            else:
                forward(p, store)
        with pytest.raises(RuntimeError, match="during a forward"):
            p.begin_forward()
            p.resize(1, 1)
        p.end_forward()
