"""Streaming engine on the GPU: slots hold exactly the store's bytes, kernels that read a slot run after its copy and
before its reuse, and a streamed stack of DiT blocks computes bit for bit what the all-resident stack computes."""
import pytest
import torch

from h3turbo_amd import block as bk
from h3turbo_amd.blockstore import HostBlockStore
from h3turbo_amd.stream import StreamingProvider
from test_stream import LAYERS, forward, raw, tiny_block

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.fixture(scope="module")
def blocks():
    return [tiny_block(200 + i) for i in range(LAYERS)]


@pytest.fixture(scope="module", params=[False, True], ids=["pageable-store", "pinned-store"])
def store(request, blocks):
    return HostBlockStore.from_blocks(blocks, pinned=request.param)


@pytest.mark.parametrize("resident,kw", [
    (0, dict(pin="auto", pin_blocks=99)),
    (2, dict(pin=True, pin_mode="copy")),
    (1, dict(pin="auto", pin_mode="stage")),
    (0, dict(pin=False)),
    (LAYERS, dict()),
])
def test_slots_match_the_store_and_kernels_are_ordered(store, resident, kw):
    print(f"stream resident={resident} {kw} pinned_store={store.pinned}", flush=True)
    want = {i: sum(int(t.to(torch.int64).sum()) for t in (store.block_weights_cpu(i).qkv.q, store.block_weights_cpu(i).fc2.q))
            for i in range(LAYERS)}
    big = torch.randn(1024, 1024, device=DEV)
    with StreamingProvider(store, DEV, resident=resident, prefetch=2, ring=3, **kw) as p:
        for _ in range(4):
            sums = []

            def compute(i, w):
                x = big
                for _ in range(20):  # keep the GPU busy so the host runs ahead of the device
                    x = torch.tanh(x @ big)
                # reads the slot AFTER the busy work: a copy into a slot still in use would change the sum
                sums.append((w.qkv.q.to(torch.int64).sum() + w.fc2.q.to(torch.int64).sum(), x))

            forward(p, store, compute, check=False)
            assert [int(s) for s, _ in sums] == [want[i] for i in range(LAYERS)]
        torch.cuda.synchronize()
        for i in range(LAYERS):
            buf = p.buffer_of(i)
            if buf is not None:
                assert raw(buf) == bytes(store.block_bytes(i))
        if resident < LAYERS:
            kinds = p.stats()["host_kinds"]
            assert sum(kinds.values()) == LAYERS - resident
            if store.pinned and kw.get("pin") is not False:
                assert kinds == {"registered": LAYERS - resident}


def test_staging_ring_is_used_when_nothing_can_be_pinned(blocks):
    st = HostBlockStore.from_blocks(blocks)
    p = StreamingProvider(st, DEV, resident=1, ring=2, prefetch=1, pin="auto", pin_blocks=0, wait_timeout=20)
    try:
        assert p.stats()["host_kinds"] == {"staged": LAYERS - 1}
        for _ in range(2):
            forward(p, st)
    finally:
        p.close()


@pytest.mark.parametrize("plan", [[(2, 3), (0, 0), (2, 3)], [(3, 2), (1, 1), (6, 3)]])
def test_resize_on_the_gpu_keeps_blocks_exact(blocks, plan):
    st = HostBlockStore.from_blocks(blocks)
    with StreamingProvider(st, DEV, resident=plan[0][0], prefetch=2, ring=plan[0][1], pin="auto") as p:
        forward(p, st)
        for resident, ring in plan[1:]:
            p.resize(resident, ring)
            if not p.parked:
                forward(p, st)


def test_streamed_dit_stack_equals_the_resident_stack():
    """8 W4A8 DiT blocks (hidden 512, 4 heads, SwiGLU 1024), 700 tokens: streaming through a 2-slot ring computes
    exactly the all-resident result (same kernels on the same bytes)."""
    torch.manual_seed(0)
    cfg = bk.BlockConfig(hidden=512, heads=4, head_dim=128, ffn=1024, act="swiglu")
    import inputs as gi
    from test_gpu_block import block_weights_gpu

    ws = []
    for i in range(8):
        _, _, _, _, norms, lin = gi.block_case(act="swiglu", seed=30 + i, hidden=512, heads=4, head_dim=128, ffn=1024, s=4)
        w = block_weights_gpu(lin, norms)
        ws.append(type(w)(**{f: (getattr(w, f).to("cpu") if getattr(w, f) is not None else None) for f in w.__dataclass_fields__}))
    st = HostBlockStore.from_blocks(ws, pinned=True)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(700, 512, generator=g, device=DEV).to(torch.bfloat16)
    mods = [torch.randn(1, 512, generator=g, device=DEV) * 0.1 for _ in range(6)]
    pos = torch.randint(0, 50, (700, 3))
    rope = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), DEV, torch.bfloat16)
    blk = bk.DiTBlock(cfg)
    outs = []
    for resident, ring in ((8, 3), (0, 2), (3, 2)):
        with StreamingProvider(st, DEV, resident=resident, ring=ring, prefetch=2) as p:
            for _ in range(2):  # the second forward starts from the cyclic prefetch of the first
                outs.append(bk.run_blocks(blk, x.clone(), p, 8, lambda i, w: mods, [(0, 700, 0)], rope))
    assert all(torch.equal(o, outs[0]) for o in outs[1:])


def test_engine_from_h3t_streams_the_file_blocks():
    """A W4A8 .h3t file (the reference writer's golden file) through H3Engine.from_h3t: streamed from pinned host
    memory, streamed from the file mapping, and run block by block from the file's own views all give the same
    residual, bit for bit."""
    import os

    from h3turbo_amd import h3t
    from h3turbo_amd.engine import H3Engine
    from h3turbo_amd.types import BlockWeights, W4A8Weight

    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vectors", "h3t_tiny_quant.h3t")
    cfg = bk.BlockConfig(hidden=64, heads=2, head_dim=32, ffn=48, act="swiglu", rope_freqs=4)
    g = torch.Generator(device=DEV).manual_seed(3)
    s = 40
    x0 = torch.randn(s, 64, generator=g, device=DEV).to(torch.bfloat16)
    mods = [torch.randn(2, 64, generator=g, device=DEV) * 0.1 for _ in range(6)]
    segs = [(0, 25, 0), (25, s, 1)]
    ang = torch.rand(s, 12, generator=g, device=DEV) * 6
    rope = (torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16))
    outs = []
    for kw in (dict(resident=0, ring=2), dict(load_pinned=False, resident=0, ring=2, pin=False), dict(resident="auto")):
        with H3Engine.from_h3t(golden, "cuda", block_config=cfg, **kw) as eng:
            assert eng.linear_backend() == "hip"
            outs.append(eng.blocks(x0.clone(), lambda i, w: mods, segs, rope))
    torch.cuda.synchronize()
    blk = bk.DiTBlock(cfg)
    x = x0.clone()
    with h3t.H3TFile(golden) as f:
        for i in range(f.n_blocks):
            w = f.block_weights_cpu(i)
            dev = lambda t: t.to(DEV) if isinstance(t, torch.Tensor) else (t.to(DEV) if isinstance(t, W4A8Weight) else t)  # noqa: E731
            wd = BlockWeights(**{k: dev(getattr(w, k)) for k in ("qkv", "out", "fc1", "fc2", "norm1", "norm2", "q_norm",
                                                                  "k_norm", "adaln_w", "adaln_b")})
            x = blk(x, wd, mods, segs, rope)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, x)
