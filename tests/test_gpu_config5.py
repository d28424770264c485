"""BASELINE config 5 on the GPU: a 60-block stack of config-4 DiT blocks (hidden 5120, 40 x 128 heads, GELU FFN
13824, W4A8 int4 group-128 fp16 scales) whose weights live in pinned host RAM, one step at 12090 + 512 tokens.

Streaming the stack through a 3-slot ring with 2-block lookahead must compute bit for bit what the all-resident
stack computes (the same kernels on the same bytes; the reference's stream check compares the same two runs,
scripts/h3_check_stream_gpu.py, and its tests pin the kernel ordering, tests/test_h3_stream.py:353-377).  The
copies and the host waits of the streamed forward are recorded; from page-locked memory there are none (the
reference reports 0 waits on its real forwards, README.md:130).
"""
import time

import pytest
import torch

from h3turbo_amd import block as bk
from h3turbo_amd.blockstore import BlockLayout, HostBlockStore, block_tensors
from h3turbo_amd.stream import StreamingProvider
from test_gpu_block import _config4_weights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
N_BLOCKS, S, HIDDEN = 60, 12602, 5120


def test_config5_streamed_stack_equals_the_resident_stack():
    t0 = time.perf_counter()
    cfg = bk.BlockConfig(hidden=HIDDEN, heads=40, head_dim=128, ffn=13824, act="gelu")
    g = torch.Generator(device=DEV).manual_seed(55)
    first = block_tensors(_config4_weights(HIDDEN, 5120, cfg.fc1_out, 13824, g))
    store = HostBlockStore(BlockLayout.of(first), N_BLOCKS, 128, 256, pinned=True)
    store.write_block(0, first)
    for i in range(1, N_BLOCKS):
        store.write_block(i, block_tensors(_config4_weights(HIDDEN, 5120, cfg.fc1_out, 13824, g)))
    del first
    print(f"config-5 store: {N_BLOCKS} blocks x {store.block_nbytes / 1e6:.1f} MB pinned, "
          f"{time.perf_counter() - t0:.1f} s", flush=True)

    x0 = torch.randn(S, HIDDEN, generator=g, device=DEV).to(torch.bfloat16)
    mods = [torch.randn(1, HIDDEN, generator=g, device=DEV) * 0.1 for _ in range(6)]
    pos = torch.stack(torch.meshgrid(torch.arange(31), torch.arange(15), torch.arange(26), indexing="ij"), -1).reshape(-1, 3)
    pos = torch.cat([pos + 1, torch.zeros(512, 3, dtype=pos.dtype)], 0)
    rope = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), DEV, torch.bfloat16)
    blk = bk.DiTBlock(cfg)

    def run(p):
        return bk.run_blocks(blk, x0.clone(), p, N_BLOCKS, lambda i, w: mods, [(0, S, 0)], rope)

    with StreamingProvider(store, DEV, resident=N_BLOCKS) as p:
        want = run(p)
        torch.cuda.synchronize()
    print(f"resident forward done ({time.perf_counter() - t0:.1f} s)", flush=True)
    with StreamingProvider(store, DEV, resident=0, ring=3, prefetch=2) as p:
        first_out = run(p)
        torch.cuda.synchronize()
        p.wait_prefetch()  # the wrap-around copies of blocks 0 and 1 belong to the first forward's count
        p.reset_stats()
        t1 = time.perf_counter()
        second_out = run(p)  # starts from the cyclic prefetch of the first forward
        torch.cuda.synchronize()
        dt = time.perf_counter() - t1
        st = p.stats()
    print(f"streamed forward {dt:.3f} s: copies {st['copies']}, waits {st['waits']} ({st['wait_s']:.4f} s), "
          f"host kinds {st['host_kinds']}", flush=True)
    assert st["host_kinds"] == {"registered": N_BLOCKS}
    assert st["acquires"] == N_BLOCKS and st["copies"] == N_BLOCKS
    # copies from page-locked memory are issued by the model thread when scheduled: no acquire waits for one
    assert st["waits"] == 0
    assert torch.isfinite(want.float()).all()
    assert torch.equal(first_out, want) and torch.equal(second_out, want)
