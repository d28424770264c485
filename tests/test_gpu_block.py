"""GPU DiT block (h3turbo_amd.block) against the CPU block oracle (oracle/block_ref.py).

Bar: bf16 outputs within max-abs-err 1e-2 of the output RMS.  The sub-paths are held
tighter: the MLP is the W4A8 linears (bit-exact) around one torch activation, and the attention path differs from
the oracle only in SDPA's kernel and the norms' reduction order.  At the full config-4 shape the W4A8 block is
compared with the same block on the dequantised dense weights (hipBLASLt bf16 GEMMs): the difference is the int8
activation quantisation noise, about 1 % of each linear's output.
"""
import math
import time

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import inputs as gi
from h3turbo_amd import block as bk
from h3turbo_amd.types import BlockWeights, W4A8Weight
from oracle import block_ref as br

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def w4a8_gpu(p) -> W4A8Weight:
    if p["s_kind"] == "fp8":
        s = torch.from_numpy(np.ascontiguousarray(p["s_rel"])).view(torch.float8_e4m3fn)
    else:
        s = torch.from_numpy(np.ascontiguousarray(p["s_rel"]).view(np.int16)).view(torch.float16)
    return W4A8Weight(torch.from_numpy(np.ascontiguousarray(p["q"])).to(DEV), s.to(DEV),
                      torch.from_numpy(p["s_ch"]).to(DEV), torch.from_numpy(p["cb"]).to(DEV), group_size=p["group"],
                      convrot=p["convrot"])


def block_weights_gpu(lin, norms) -> BlockWeights:
    return BlockWeights(qkv=w4a8_gpu(lin["qkv"]), out=w4a8_gpu(lin["out"]), fc1=w4a8_gpu(lin["fc1"]),
                        fc2=w4a8_gpu(lin["fc2"]), norm1=norms["norm1"].to(DEV), norm2=norms["norm2"].to(DEV),
                        q_norm=norms["q_norm"].to(DEV), k_norm=norms["k_norm"].to(DEV))


def segs_gpu(segments):
    return [(a, b, r.to(DEV) if isinstance(r, torch.Tensor) else r) for a, b, r in segments]


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def within_north_star(got, want):
    """max |got - want| <= 1e-2 * RMS(want)"""
    err = (got.double() - want.double()).abs().max().item()
    rms = want.double().pow(2).mean().sqrt().item()
    return err <= 1e-2 * rms, err / rms


def bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    """spacing of bf16 values at |v| (8 significant bits)"""
    a = v.double().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)




SHAPE = dict(hidden=512, heads=4, head_dim=128, ffn=1024, s=300)


@pytest.mark.parametrize("act", ["swiglu", "gelu"])
def test_block_matches_the_cpu_oracle(act):
    print(f"block act={act} {SHAPE}", flush=True)
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act=act, seed=7, **SHAPE)
    cfg = bk.BlockConfig(hidden=SHAPE["hidden"], heads=SHAPE["heads"], head_dim=SHAPE["head_dim"], ffn=SHAPE["ffn"],
                         act=act)
    blk = bk.DiTBlock(cfg)
    w = block_weights_gpu(lin, norms)
    mods_g = [m.to(DEV) for m in mods]
    rope = (cos.to(DEV), sin.to(DEV))
    xg = x.to(DEV)
    out = blk(xg.clone(), w, mods_g, segs_gpu(segs), rope)
    want = br.block_ref(x, {**lin, **norms}, mods, segs, cos, sin, SHAPE["heads"], SHAPE["head_dim"], act, 1e-5, 1e-5)
    # Sub-paths at full magnitude.  The MLP (W4A8 linears around one torch activation) meets the north-star bar.
    # The attention output before its projection is PyTorch-ROCm's bf16 flash kernel (P rounded to bf16 before
    # P.V) against fp32 attention rounded once: rel-L2 1e-2, max-abs 5e-2 of its RMS.  After the out projection, a
    # final-bit difference of its input can move one int8 activation by one quantisation step, which moves that
    # output row by up to a few % of its RMS: held to rel-L2 there, and in the residual.
    h = x.to(DEV)
    ref_w = {**lin, **norms}
    mlp, mlp_ref = blk.mlp(h, w).cpu(), br.mlp_ref(x, ref_w, act)
    o, o_ref = blk.attend(h, w, rope).cpu(), br.attend_ref(x, ref_w, cos, sin, SHAPE["heads"], SHAPE["head_dim"], 1e-5)
    att = blk.attention(h, w, rope).cpu()
    att_ref = br.attention_ref(x, ref_w, cos, sin, SHAPE["heads"], SHAPE["head_dim"], 1e-5)
    report = dict(mlp_rel=rel(mlp, mlp_ref), mlp_ns=within_north_star(mlp, mlp_ref)[1], sdpa_rel=rel(o, o_ref),
                  sdpa_ns=within_north_star(o, o_ref)[1], att_rel=rel(att, att_ref), out_rel=rel(out.cpu(), want),
                  update_rel=rel(out.cpu().double() - x.double(), want.double() - x.double()))
    print(report, flush=True)
    assert within_north_star(mlp, mlp_ref)[0] and report["mlp_rel"] < 1e-3
    assert report["sdpa_rel"] < 1e-2 and report["sdpa_ns"] < 5e-2
    assert report["att_rel"] < 2e-2
    assert report["out_rel"] < 2e-3 and report["update_rel"] < 0.1


def _random_w4a8_parts(n, k, g):
    """Random W4A8 weight parts of the BASELINE format (int4 codes around arange(-8, 8), group-128 fp16 scales,
    per-channel scale for ~N(0, 0.02) weights), built on the CPU for the block oracle."""
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8).numpy()
    s_rel = (torch.rand(n, k // 128, generator=g) * 3.0 + 12.875).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    s_ch = np.full(n, 0.02 * math.sqrt(3.0) / (7.5 * 14.375), np.float32)
    return {"q": q, "s_rel": s_rel, "s_kind": "f16", "s_ch": s_ch, "cb": np.arange(-8, 8, dtype=np.float32),
            "group": 128, "convrot": 256}


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_config4_width_block_within_the_north_star_tolerance(act):
    """The config-4 block width (hidden 5120, 40 x 128 heads, FFN 13824) against the CPU block oracle at S = 384.

    north_star's bar, max|out - ref| <= 1e-2 * RMS(ref) on the bf16 output, is asserted with the oracle given the
    GPU's own results of the two steps whose arithmetic order is not the reference's: the attention kernel
    (PyTorch-ROCm SDPA, outside the hand-written path) and the fused RMSNorm + modulation (its sum of squares runs
    in its own order; test_fused_rms_modulate_matches_the_torch_ops holds it within one bf16 ulp).  Everything else
    -- the four W4A8 linears, the q/k norm + rope, the gated residual adds, the activation -- must then agree; the
    attention prologue (q/k/v after norm + rope) is also held bit-exact.

    The fully independent comparison (oracle norms and fp32 attention) is reported and held to rel-L2 1e-2: SDPA's
    bf16 numerics (P rounded to bf16 before P.V) and one-ulp norm differences move individual int8 activations by a
    quantisation step, and the two requantisations downstream amplify that -- measured max-abs 0.06 (GELU) and
    0.11 (SwiGLU) of RMS at rel-L2 0.4-0.6 %."""
    s, hidden, heads, hd, ffn = 384, 5120, 40, 128, 13824
    print(f"config-4-width block act={act} S={s}", flush=True)
    g = torch.Generator().manual_seed(404 + (act == "swiglu"))
    x = torch.randn(s, hidden, generator=g).to(torch.bfloat16)
    mods = [torch.randn(3, hidden, generator=g) * 0.1 for _ in range(6)]
    segs = [(0, 100, 0), (100, 250, 1), (250, s, torch.randint(0, 3, (s - 250,), generator=g))]
    pos = torch.randint(0, 64, (s, 3), generator=g)
    inv_freq = 1.0 / (10000.0 ** (torch.arange(16, dtype=torch.float32) / 16))
    ang = (pos.float()[:, :, None] * inv_freq[None, None, :]).reshape(s, -1)
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    norms = {n: (1.0 + 0.1 * torch.randn(d, generator=g)) for n, d in
             (("norm1", hidden), ("norm2", hidden), ("q_norm", hd), ("k_norm", hd))}
    cfg = bk.BlockConfig(hidden=hidden, heads=heads, head_dim=hd, ffn=ffn, act=act)
    lin = {"qkv": _random_w4a8_parts(3 * heads * hd, hidden, g), "out": _random_w4a8_parts(hidden, heads * hd, g),
           "fc1": _random_w4a8_parts(cfg.fc1_out, hidden, g), "fc2": _random_w4a8_parts(hidden, ffn, g)}
    w = block_weights_gpu(lin, norms)
    blk = bk.DiTBlock(cfg)
    seen = {"h": []}
    real_sdpa, real_rms_modulate, real_gated_rms = bk._sdpa, bk.rms_modulate, bk.gated_add_rms_modulate

    def capture_sdpa(q, k, v):  # the attention kernel's inputs and output, as the block ran them
        o = real_sdpa(q, k, v)
        seen.update(q=q[0].cpu(), k=k[0].cpu(), v=v[0].cpu(), o=o[0].cpu())
        return o

    def capture_rms_modulate(*a, **kw):  # the two RMSNorm + modulation outputs (the second from the fused call)
        h = real_rms_modulate(*a, **kw)
        seen["h"].append(h.cpu())
        return h

    def capture_gated_rms(*a, **kw):
        h = real_gated_rms(*a, **kw)
        seen["h"].append(h.cpu())
        return h

    bk._sdpa, bk.rms_modulate, bk.gated_add_rms_modulate = capture_sdpa, capture_rms_modulate, capture_gated_rms
    try:
        out = blk(x.to(DEV), w, [m.to(DEV) for m in mods], segs_gpu(segs), (cos.to(DEV), sin.to(DEV))).cpu()
    finally:
        bk._sdpa, bk.rms_modulate, bk.gated_add_rms_modulate = real_sdpa, real_rms_modulate, real_gated_rms
    assert len(seen["h"]) == 2
    mlp = blk.mlp(x.to(DEV), w).cpu()
    print("  GPU block done; CPU oracle running", flush=True)
    ref_w = {**lin, **norms}
    o_gpu = seen["o"].transpose(0, 1).reshape(s, heads * hd)  # [heads, S, D] -> [S, heads * D]
    want = br.block_ref(x, ref_w, mods, segs, cos, sin, heads, hd, act, 1e-5, 1e-5, attend=o_gpu, modulated=seen["h"])
    full = br.block_ref(x, ref_w, mods, segs, cos, sin, heads, hd, act, 1e-5, 1e-5)

    # the attention prologue on the GPU's own modulated input: q, k, v bit for bit
    qkv = br._linear(seen["h"][0], lin["qkv"])
    q, k, v = (t.reshape(s, heads, hd).clone() for t in qkv.split(heads * hd, dim=-1))
    br.norm_rope_ref(q, k, norms["q_norm"], norms["k_norm"], 1e-5, cos, sin, "torch")
    h_ref = br._modulate(F.rms_norm(x, (hidden,), norms["norm1"].to(x.dtype), 1e-5), mods[0], mods[1], segs)

    err = (out.double() - want.double()).abs()
    rms = want.double().pow(2).mean().sqrt().item()
    report = dict(max_abs_over_rms=err.max().item() / rms, out_rel=rel(out, want),
                  modulated_input_ulps=int((seen["h"][0] != h_ref).sum()),
                  full_chain_max_abs_over_rms=(out.double() - full.double()).abs().max().item() / rms,
                  full_chain_rel=rel(out, full), mlp_ns=within_north_star(mlp, mlp_ref := br.mlp_ref(x, ref_w, act))[1],
                  mlp_rel=rel(mlp, mlp_ref))
    print(report, flush=True)
    assert torch.equal(seen["q"].transpose(0, 1), q) and torch.equal(seen["k"].transpose(0, 1), k)
    assert torch.equal(seen["v"].transpose(0, 1), v)
    assert within_north_star(mlp, mlp_ref)[0], "MLP sub-path beyond 1e-2 * RMS"
    assert report["max_abs_over_rms"] <= 1e-2, "block beyond 1e-2 * RMS of the oracle on the same attention and norms"
    assert report["full_chain_rel"] < 1e-2


def test_chunked_block_is_exact_and_inputs_are_only_the_residual():
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act="swiglu", seed=8, **SHAPE)
    cfg = bk.BlockConfig(hidden=SHAPE["hidden"], heads=SHAPE["heads"], head_dim=SHAPE["head_dim"], ffn=SHAPE["ffn"],
                         act="swiglu")
    w = block_weights_gpu(lin, norms)
    mods_g = [m.to(DEV) for m in mods]
    rope = (cos.to(DEV), sin.to(DEV))
    mods_before = [m.clone() for m in mods_g]
    a = bk.DiTBlock(cfg)(x.to(DEV), w, mods_g, segs_gpu(segs), rope)
    b = bk.DiTBlock(cfg, mlp_chunk=64)(x.to(DEV), w, mods_g, segs_gpu(segs), rope)
    assert torch.equal(a, b)  # MLP token chunks: exact
    # query chunks: exact up to the attention kernel's tiling (it may split the key loop by query count)
    c = bk.DiTBlock(cfg, attn_chunk=128)(x.to(DEV), w, mods_g, segs_gpu(segs), rope)
    assert rel(c, a) < 2e-3
    xd = x.to(DEV).double()
    assert rel(c.double() - xd, a.double() - xd) < 0.1
    assert all(torch.equal(m, m0) for m, m0 in zip(mods_g, mods_before))


def test_block_loop_protocol_order_and_release_on_error():
    x, mods, segs, (cos, sin), norms, lin = gi.block_case(act="swiglu", seed=9, **SHAPE)
    cfg = bk.BlockConfig(hidden=SHAPE["hidden"], heads=SHAPE["heads"], head_dim=SHAPE["head_dim"], ffn=SHAPE["ffn"],
                         act="swiglu")
    w = block_weights_gpu(lin, norms)
    log = []

    class Recorder(bk.ResidentProvider):
        def begin_forward(self):
            log.append("begin")

        def acquire(self, i):
            log.append(("acquire", i))
            return super().acquire(i)

        def release(self, i):
            log.append(("release", i))

        def end_forward(self):
            log.append("end")

    mods_g = [m.to(DEV) for m in mods]
    blk = bk.DiTBlock(cfg)
    out = bk.run_blocks(blk, x.to(DEV), Recorder([w, w]), 2, lambda i, wi: mods_g, segs_gpu(segs), (cos.to(DEV), sin.to(DEV)))
    assert log == ["begin", ("acquire", 0), ("release", 0), ("acquire", 1), ("release", 1), "end"]
    once = blk(blk(x.to(DEV), w, mods_g, segs_gpu(segs), (cos.to(DEV), sin.to(DEV))), w, mods_g, segs_gpu(segs),
               (cos.to(DEV), sin.to(DEV)))
    assert torch.equal(out, once)
    log.clear()
    with pytest.raises(ValueError):
        bk.run_blocks(blk, x.to(DEV), Recorder([w]), 1, lambda i, wi: mods_g[:5], segs_gpu(segs), None)
    assert log == ["begin", ("acquire", 0), ("release", 0), "end"]


def _dense_block_weights(w: BlockWeights) -> BlockWeights:
    from h3turbo_amd import qlinear as ql

    d = lambda lw: ql.dequantize(lw, torch.bfloat16)  # noqa: E731
    return BlockWeights(qkv=d(w.qkv), out=d(w.out), fc1=d(w.fc1), fc2=d(w.fc2), norm1=w.norm1, norm2=w.norm2,
                        q_norm=w.q_norm, k_norm=w.k_norm)


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_config4_block_full_shape_is_the_dense_block_within_quantisation_noise(act):
    """hidden 5120, 40 x 128 heads, FFN 13824, S = 12090 video + 512 text tokens, bf16."""
    s, hidden, heads, hd, ffn = 12602, 5120, 40, 128, 13824
    print(f"config-4 block act={act} S={s}", flush=True)
    cfg = bk.BlockConfig(hidden=hidden, heads=heads, head_dim=hd, ffn=ffn, act=act)
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(s, hidden, generator=g, device=DEV).to(torch.bfloat16)
    mods = [torch.randn(1, hidden, generator=g, device=DEV) * 0.1 for _ in range(6)]
    segs = [(0, s, 0)]
    pos = torch.stack(torch.meshgrid(torch.arange(31), torch.arange(15), torch.arange(26), indexing="ij"), -1).reshape(-1, 3)
    pos = torch.cat([pos + 1, torch.zeros(512, 3, dtype=pos.dtype)], 0)
    cos, sin = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), DEV, torch.bfloat16)
    w = _config4_weights(hidden, heads * hd, cfg.fc1_out, ffn, g)
    blk = bk.DiTBlock(cfg)
    out = blk(x.clone(), w, mods, segs, (cos, sin))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    blk(x.clone(), w, mods, segs, (cos, sin))
    torch.cuda.synchronize()
    print(f"block ms {1e3 * (time.perf_counter() - t0):.2f}", flush=True)
    dense = bk.DiTBlock(cfg)(x.clone(), _dense_block_weights(w), mods, segs, (cos, sin))
    assert torch.isfinite(out.float()).all()
    # a8 against dense is the activation quantisation itself (about 1 % per linear), not a parity error: held to
    # rel-L2 of the block's update and of the residual
    d_rel = rel(out.double() - x.double(), dense.double() - x.double())
    o_rel = rel(out, dense)
    print(f"update rel-L2 {d_rel:.3e}, residual rel-L2 {o_rel:.3e}, max-abs/RMS {within_north_star(out, dense)[1]:.3e}",
          flush=True)
    assert d_rel < 3e-2 and o_rel < 1e-2


def _config4_weights(hidden, inner, fc1_out, ffn, g) -> BlockWeights:
    """Random-init W4A8 weights of the BASELINE recipe's distribution, built on the GPU (int4 codes uniform in
    [-8, 7] around the codebook arange(-8, 8), group-128 fp16 scales, per-channel scale for ~N(0, 0.02) weights)."""
    def lin(n, k):
        q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8, device=DEV)
        s_rel = (torch.rand(n, k // 128, generator=g, device=DEV) * 3.0 + 12.875).to(torch.float16)
        s_ch = torch.full((n,), 0.02 * math.sqrt(3.0) / (7.5 * 14.375), device=DEV)
        return W4A8Weight(q, s_rel, s_ch, torch.arange(-8, 8, dtype=torch.float32, device=DEV), group_size=128, convrot=256)

    ones = lambda d: 1.0 + 0.1 * torch.randn(d, generator=g, device=DEV)  # noqa: E731
    return BlockWeights(qkv=lin(3 * inner, hidden), out=lin(hidden, inner), fc1=lin(fc1_out, hidden), fc2=lin(hidden, ffn),
                        norm1=ones(hidden), norm2=ones(hidden), q_norm=ones(128), k_norm=ones(128))


@pytest.mark.parametrize("s,k,int_valued", [(37, 5120, True), (300, 1024, True), (5, 5376, True), (129, 5120, False),
                                             (2051, 1024, True), (2051, 1024, False)])
def test_fused_rms_modulate_matches_the_torch_ops(s, k, int_valued):
    """h3k_rms_modulate against F.rms_norm + the in-place modulation on the CPU (h3turbo/h3/model.py:64-65,
    106-109), on one row per workgroup and (from 2048 rows) four, the last workgroup partly empty.  With
    integer-valued rows the sum of squares is exact in any order and the outputs are bit-exact;
    on Gaussian rows the kernel's own summation order may move the norm by an ulp on a few rows: every output is
    then the modulation of the reference norm or of one of its two bf16 neighbours, bit for bit."""
    print(f"rms_modulate s={s} k={k} int={int_valued}", flush=True)
    g = torch.Generator().manual_seed(s + k)
    if int_valued:
        x = torch.randint(-8, 9, (s, k), generator=g).to(torch.bfloat16)
    else:
        x = (torch.randn(s, k, generator=g) * torch.exp(torch.randn(s, 1, generator=g))).to(torch.bfloat16)
    w = 1 + 0.2 * torch.randn(k, generator=g)
    shift, scale = 0.1 * torch.randn(3, k, generator=g), 0.1 * torch.randn(3, k, generator=g)
    a, b = s // 3, 2 * s // 3
    segments = [(0, a, 0), (a, b, torch.randint(0, 3, (b - a,), generator=g)), (b, s, 2)]
    want = bk.modulate_(bk.rms(x, w, 1e-5), shift, scale, segments)
    seg_gpu = [(p, q, r.to(DEV) if isinstance(r, torch.Tensor) else r) for p, q, r in segments]
    got = bk.rms_modulate(x.to(DEV), w.to(DEV), shift.to(DEV), scale.to(DEV), 1e-5, seg_gpu).cpu()
    if int_valued:
        assert torch.equal(got, want)
    else:
        n = bk.rms(x, w, 1e-5)
        bits = n.view(torch.int16)
        neighbours = []
        for d in (-1, 1):  # the adjacent bf16 values of each nonzero norm (zero norms come from zero inputs)
            nb = torch.where(n != 0, (bits + d).view(torch.bfloat16), n)
            neighbours.append(bk.modulate_(nb.clone(), shift, scale, segments))
        ok = (got == want) | (got == neighbours[0]) | (got == neighbours[1])
        assert ok.all(), f"{int((~ok).sum())} outputs are not the modulation of the norm or of a neighbour"
        assert (got != want).float().mean().item() < 0.01


@pytest.mark.parametrize("vec_bf16", [False, True])
@pytest.mark.parametrize("s,k", [(37, 5120), (300, 1024), (1, 5376), (4099, 768), (2050, 5120)])
def test_gated_add_rms_modulate_equals_the_two_passes(s, k, vec_bf16):
    """h3k_gated_add_rms_modulate against h3k_gated_add then h3k_rms_modulate on the same inputs, bit for bit: the
    updated residual and the modulated rows, with scalar and per-token modulation rows, below and above the
    2048-row switch to 4 rows per workgroup, and a row count that leaves the last workgroup partly empty.  The
    two passes take the fp32 vectors (rounded to bf16 in the kernels); with vec_bf16 the fused call takes them
    rounded to bf16 by torch, which must give the same bits."""
    print(f"gated_add_rms_modulate s={s} k={k}", flush=True)
    g = torch.Generator().manual_seed(3 * s + k)
    x = (torch.randn(s, k, generator=g) * torch.exp(torch.randn(s, 1, generator=g))).to(torch.bfloat16).to(DEV)
    y = torch.randn(s, k, generator=g).to(torch.bfloat16).to(DEV)
    gate, shift, scale = (0.3 * torch.randn(3, k, generator=g)).to(DEV), (0.1 * torch.randn(3, k, generator=g)).to(DEV), \
        (0.1 * torch.randn(3, k, generator=g)).to(DEV)
    w = (1 + 0.2 * torch.randn(k, generator=g)).to(DEV)
    a, b = s // 3, 2 * s // 3
    segments = [(0, a, 0), (a, b, torch.randint(0, 3, (b - a,), generator=g).to(DEV)), (b, s, 2)]
    x2 = x.clone()
    vecs = [t.to(torch.bfloat16) if vec_bf16 else t for t in (gate, w, shift, scale)]
    h_fused = bk.gated_add_rms_modulate(x, vecs[0], y, vecs[1], vecs[2], vecs[3], 1e-5, segments)
    bk.gated_add_(x2, gate, y, segments)
    h_two = bk.rms_modulate(x2, w, shift, scale, 1e-5, segments)
    assert torch.equal(x.view(torch.int16), x2.view(torch.int16)), "residual differs"
    assert torch.equal(h_fused.view(torch.int16), h_two.view(torch.int16)), "modulated rows differ"


@pytest.mark.parametrize("s,k", [(37, 5120), (300, 1024), (1, 5376), (4099, 768)])
def test_fused_gated_add_matches_the_torch_ops(s, k):
    """h3k_gated_add (one pass) against the reference's per-segment x[a:b].addcmul_(y[a:b], gate[row].to(bf16)) on
    the CPU (h3turbo/h3/model.py:112-115), bit for bit: scalar and per-token modulation rows, gates from fp32 AdaLN
    rows as strided views, outputs and residuals over several magnitudes."""
    print(f"gated_add s={s} k={k}", flush=True)
    g = torch.Generator().manual_seed(s * 7 + k)
    x = (torch.randn(s, k, generator=g) * torch.exp(2 * torch.randn(s, 1, generator=g))).to(torch.bfloat16)
    y = (torch.randn(s, k, generator=g) * 3).to(torch.bfloat16)
    z = torch.randn(3, 6 * k, generator=g) * 0.3  # fp32 modulation rows; the gate is a strided chunk of them
    gate = z.view(3, -1).chunk(6, dim=-1)[2]
    a, b = s // 3, 2 * s // 3
    segments = [(0, a, 0), (a, b, torch.randint(0, 3, (b - a,), generator=g)), (b, s, 2)]
    want = x.clone()
    for p, q, r in segments:
        want[p:q].addcmul_(y[p:q], gate[r].to(torch.bfloat16))
    seg_gpu = [(p, q, r.to(DEV) if isinstance(r, torch.Tensor) else r) for p, q, r in segments]
    xg = x.to(DEV)
    out = bk.gated_add_(xg, gate.to(DEV), y.to(DEV), seg_gpu)
    assert out is xg and torch.equal(xg.cpu(), want)
