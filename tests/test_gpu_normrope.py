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
