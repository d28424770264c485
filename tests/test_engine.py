"""Engine façade on the CPU path: a dense fp32 block stack through store -> provider -> block loop equals the
float64 block definition applied block after block."""
import torch

from h3turbo_amd import block as bk
from h3turbo_amd.blockstore import HostBlockStore
from h3turbo_amd.engine import H3Engine
from h3turbo_amd.types import BlockWeights
from oracle import block_ref as br


def dense_block(seed, hidden=64, heads=2, hd=32, ffn=48):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.1  # noqa: E731
    return BlockWeights(qkv=r(3 * heads * hd, hidden), out=r(hidden, heads * hd), fc1=r(2 * ffn, hidden), fc2=r(hidden, ffn),
                        norm1=1 + r(hidden), norm2=1 + r(hidden), q_norm=1 + r(hd), k_norm=1 + r(hd))


def test_engine_block_stack_equals_the_definition():
    blocks = [dense_block(i) for i in range(4)]
    store = HostBlockStore.from_blocks(blocks)
    cfg = bk.BlockConfig(hidden=64, heads=2, head_dim=32, ffn=48, act="swiglu", rope_freqs=4)
    g = torch.Generator().manual_seed(9)
    s = 20
    x = torch.randn(s, 64, generator=g)
    mods = [torch.randn(2, 64, generator=g) * 0.1 for _ in range(6)]
    segs = [(0, 12, 0), (12, s, 1)]
    ang = torch.rand(s, 12, generator=g) * 6
    cos, sin = torch.cos(ang), torch.sin(ang)
    with H3Engine.from_store(store, "cpu", block_config=cfg, resident=1, ring=2, pin=False) as eng:
        assert eng.linear_backend() == "unavailable"
        assert eng.gpu_bytes() == 3 * store.block_nbytes
        out = eng.blocks(x.clone(), lambda i, w: mods, segs, (cos, sin))
        assert eng.stats()["acquires"] == 3
    rows = torch.tensor([0] * 12 + [1] * (s - 12))
    want = x.double()
    for b in blocks:
        w = {"qkv": b.qkv, "out": b.out, "fc1": b.fc1, "fc2": b.fc2, "norm1": b.norm1, "norm2": b.norm2,
             "q_norm": b.q_norm, "k_norm": b.k_norm}
        want = br.block_naive(want, w, mods, rows, cos.double(), sin.double(), 2, 32, "swiglu", 1e-5, 1e-5)
    assert ((out.double() - want).norm() / want.norm()).item() < 1e-5
