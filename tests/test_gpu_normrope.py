"""The fused q/k norm + rope kernel (h3k_qk_norm_rope) against the reference's own norm_rope_ outputs (golden
vectors) and the CPU oracle on random inputs: bit-exact."""
import numpy as np
import pytest
import torch

import fixtures as fx
from h3turbo_amd import block as bk
from oracle import block_ref as br

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def t16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("name", [n for n, m in fx.index().items() if m["kind"] == "normrope" and m["impl"] == "torch"])
def test_fused_kernel_matches_the_reference_golden_vectors(name):
    meta, a = fx.load(name)
    q, k = t16(a["q"]).to(DEV), t16(a["k"]).to(DEV)
    bk.norm_rope_(q, k, t16(a["wq"]).to(DEV), t16(a["wk"]).to(DEV), meta["eps"], t16(a["cos"]).to(DEV),
                  t16(a["sin"]).to(DEV), impl="torch")
    assert torch.equal(q.cpu(), t16(a["q_out"])) and torch.equal(k.cpu(), t16(a["k_out"]))


@pytest.mark.parametrize("s,heads,hd,half", [(1, 1, 32, 0), (5, 3, 64, 12), (77, 40, 128, 48), (300, 7, 128, 64),
                                             (33, 2, 256, 96), (9, 4, 96, 20)])
def test_fused_kernel_matches_the_oracle_on_qkv_views(s, heads, hd, half):
    g = torch.Generator().manual_seed(s * 7 + hd)
    inner = heads * hd
    qkv = (torch.randn(s, 3 * inner, generator=g) * torch.exp(torch.randn(s, 1, generator=g))).bfloat16()
    wq, wk = (1 + 0.3 * torch.randn(hd, generator=g)).bfloat16(), (1 + 0.3 * torch.randn(hd, generator=g)).float()
    ang = torch.rand(s, max(half, 1), generator=g) * 30
    cos, sin = torch.cos(ang)[:, :half].bfloat16(), torch.sin(ang)[:, :half].bfloat16()
    qkv_g = qkv.to(DEV)
    qg, kg, _ = (t.view(s, heads, hd) for t in qkv_g.split(inner, dim=-1))
    bk.norm_rope_(qg, kg, wq.to(DEV), wk.to(DEV), 1e-5, cos.to(DEV), sin.to(DEV), impl="torch")
    q, k, v = (t.reshape(s, heads, hd).clone() for t in qkv.split(inner, dim=-1))
    br.norm_rope_ref(q, k, wq, wk, 1e-5, cos, sin, "torch")
    got = qkv_g.cpu()
    assert torch.equal(got[:, :inner].reshape(s, heads, hd), q)
    assert torch.equal(got[:, inner:2 * inner].reshape(s, heads, hd), k)
    assert torch.equal(got[:, 2 * inner:], qkv[:, 2 * inner:])  # v untouched


def split_reference(qkv, heads, hd, wq, wk, cos, sin, eps=1e-5):
    """norm_rope_ on q, k views of a copy of qkv (the in-place kernel), then each part transposed head-major."""
    s = qkv.shape[0]
    ref = qkv.clone()
    q, k, v = (t.view(s, heads, hd) for t in ref.split(heads * hd, dim=-1))
    bk.norm_rope_(q, k, wq, wk, eps, cos, sin, impl="torch")
    return torch.stack([t.transpose(0, 1) for t in (q, k, v)])


@pytest.mark.parametrize("s,heads,hd,half", [(1, 1, 32, 0), (5, 3, 64, 12), (77, 40, 128, 48), (300, 7, 128, 64),
                                             (33, 2, 256, 96), (13, 5, 128, 0)])
def test_split_kernel_equals_in_place_kernel_and_transpose(s, heads, hd, half):
    print(f"split s={s} heads={heads} hd={hd} half={half}", flush=True)
    g = torch.Generator().manual_seed(s * 13 + hd)
    inner = heads * hd
    qkv = (torch.randn(s, 3 * inner, generator=g) * torch.exp(torch.randn(s, 1, generator=g))).bfloat16().to(DEV)
    wq, wk = (1 + 0.3 * torch.randn(hd, generator=g)).bfloat16().to(DEV), (1 + 0.3 * torch.randn(hd, generator=g)).to(DEV)
    ang = torch.rand(s, max(half, 1), generator=g) * 30
    cos, sin = torch.cos(ang)[:, :half].bfloat16().to(DEV), torch.sin(ang)[:, :half].bfloat16().to(DEV)
    before = qkv.clone()
    got = bk.qkv_split_norm_rope(qkv, heads, hd, wq, wk, 1e-5, cos, sin)
    want = split_reference(qkv, heads, hd, wq, wk, cos, sin)
    assert torch.equal(qkv, before), "the split kernel must not modify its input"
    assert torch.equal(got, want)


@pytest.mark.parametrize("name", [n for n, m in fx.index().items() if m["kind"] == "normrope" and m["impl"] == "torch"
                                  and m.get("head_dim", 128) in (32, 64, 128, 256)])
def test_split_kernel_matches_the_reference_golden_vectors(name):
    meta, a = fx.load(name)
    q, k = t16(a["q"]), t16(a["k"])
    s, heads, hd = q.shape
    if hd not in (32, 64, 128, 256):
        pytest.skip(f"head_dim {hd} is not a split-kernel size")
    v = torch.arange(s * heads * hd, dtype=torch.int32).remainder(977).to(torch.bfloat16).view(s, heads, hd)
    qkv = torch.cat([q.reshape(s, -1), k.reshape(s, -1), v.reshape(s, -1)], 1).to(DEV)
    got = bk.qkv_split_norm_rope(qkv, heads, hd, t16(a["wq"]).to(DEV), t16(a["wk"]).to(DEV), meta["eps"],
                                 t16(a["cos"]).to(DEV), t16(a["sin"]).to(DEV)).cpu()
    assert torch.equal(got[0], t16(a["q_out"]).transpose(0, 1))
    assert torch.equal(got[1], t16(a["k_out"]).transpose(0, 1))
    assert torch.equal(got[2], v.transpose(0, 1))
