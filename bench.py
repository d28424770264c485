"""Benchmark of the W4A8 ConvRot QLinear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 32768 --k 5120 --n 13824] [--no-cpu]

A step is one full W4A8 QLinear over a resident synthetic batch: per-token rotation + int8 quantisation of
x bf16 [M, K], int4 -> int8 decode of the weight [N, K] (group 128, fp16 scales), int8 MFMA GEMM with the
fused (acc * xs) * s_ch epilogue writing bf16 [M, N].  Prints ONE JSON line (rank 0):
  value        int8 TOPS of the whole op = 2*M*N*K / step time
  roofline     the GEMM kernel: algorithmic int8 ops per launch / its mean duration (HIP events on the stream
               the kernels run on, inside the timed region) against the dense int8 MFMA peak
  cpu_baseline the CPU oracle (numpy restatement of the reference's torch CPU path) on a row sample of the
               same workload, scaled to the whole op; the thread count it used is reported
Only one GPU is used; --gpus N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "minimax-h3-turbo_amd"), os.path.join(ROOT, "tests", "golden")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA (AMD public figure, no sparsity)
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=12,
                    help="untimed steps first: the GEMM's launch time settles only after about ten launches")
    ap.add_argument("--m", type=int, default=32768)
    ap.add_argument("--k", type=int, default=5120)
    ap.add_argument("--n", type=int, default=13824)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-block", action="store_true", help="skip the config-4 DiT block measurement")
    ap.add_argument("--block-steps", type=int, default=5)
    ap.add_argument("--no-stream", action="store_true", help="skip the config-5 streamed 60-block stack")
    ap.add_argument("--no-sweep", action="store_true", help="skip the config-3 GEMM sweep (16 shapes)")
    ap.add_argument("--stream-blocks", type=int, default=60)
    ap.add_argument("--no-h3t", action="store_true", help="skip the .h3t container measurement")
    ap.add_argument("--no-model", action="store_true", help="skip the whole-model forward at the H3 shape")
    ap.add_argument("--no-few-rows", action="store_true", help="skip the small-M (16-128 rows) W4A8 GEMM measurement")
    ap.add_argument("--model-layers", type=int, default=50)
    ap.add_argument("--h3t-blocks", type=int, default=8)
    ap.add_argument("--cpu-rows", type=int, default=512, help="rows of the CPU baseline sample")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="after the timed region, run 3 plain device-to-device copies of BYTES bytes: the reference "
                         "kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the HBM traffic figures")
    return ap.parse_args()


def traffic_from_profiles(key: str):
    """HBM bytes per launch of `key` ("<kernel> m=.. k=.. n=.."), from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    summarised under profiles/ (None when that workload was not profiled)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def synth_weight(n: int, k: int, dev, seed: int = 0, group: int = 128, convrot: int = 256):
    """BASELINE weight recipe on the device: W ~ N(0, 0.02) [n, k] rotated into the ConvRot basis, symmetric int4
    per group of 128 with fp16 relative scales: s_g = amax|W_rot| / 7, code = clamp(rint(W_rot / s_g), -8, 7) + 8
    (low nibble = even k), codebook arange(-8, 8), s_ch = max_g s_g / 15.875, s_rel = fp16(s_g / s_ch)."""
    import torch

    from h3turbo_amd import qlinear as ql

    g = torch.Generator(device=dev).manual_seed(seed + 1000)
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    h = ql.hadamard_regular(convrot, dev, torch.float32)
    w_rot = torch.mm(w.view(-1, convrot), h).view(n, k // group, group)
    del w
    s_g = (w_rot.abs().amax(-1) / 7.0).clamp_min(1e-12)
    code = torch.clamp(torch.round(w_rot / s_g[..., None]), -8, 7).to(torch.int16).view(n, k) + 8
    del w_rot
    q = (code[:, 0::2] | (code[:, 1::2] << 4)).to(torch.uint8).view(torch.int8).contiguous()
    s_ch = (s_g.amax(1) / 15.875).contiguous()
    s_rel = (s_g / s_ch[:, None]).to(torch.float16).contiguous()
    cb = torch.arange(-8, 8, dtype=torch.float32, device=dev)
    return q, s_rel, s_ch, cb


def decode_packed_g16_fp8(dev, n: int = 13824, k: int = 5120, calls: int = 40) -> dict:
    """The packed-grid decode of the checkpoint weight format (fp8 e4m3 relative scales per group of 16) at the
    headline weight shape: random codes and finite scale bytes, codebook arange(-8, 8).  A bounded spin kernel ahead
    of the loop lets the host enqueue every call first, so the event pair times the kernels alone."""
    import torch

    from h3turbo_amd import _lib

    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(16)
    q = torch.randint(0, 256, (n, k // 2), generator=g, device=dev, dtype=torch.uint8)
    s = torch.randint(0, 0x7E, (n, k // 16), generator=g, device=dev, dtype=torch.uint8)  # no NaN bytes
    cb = torch.arange(-8, 8, dtype=torch.float32, device=dev)
    out = torch.empty(lib.h3k_w8_packed_bytes(n, k), dtype=torch.int8, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    def call():
        _lib.check(lib.h3k_decode_w4_packed(q.data_ptr(), k // 2, s.data_ptr(), _lib.FP8E4M3, k // 16, cb.data_ptr(), n,
                                            k, 16, out.data_ptr(), sp), "decode packed g16")

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(4_000_000)  # a few ms of one spinning wavefront: the host gets ahead of the GPU
    e0.record(stream)
    for _ in range(calls):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / calls
    nbytes = n * k // 2 + n * (k // 16) + (n + 255) // 256 * 256 * k
    return {"n": n, "k": k, "group": 16, "scales": "fp8e4m3", "ms": round(ms, 4),
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def gemm_kernel_name(m: int, n: int, k: int, packed: bool, cus: int = 256) -> str:
    """The GEMM kernel the W4A8 linear runs for this shape with aligned operands: the packed-weight kernel where
    h3k_gemm_packed_serves accepts the shape, otherwise the rule of gemm_a8w8_launch (h3k_gemm.hip)."""
    if packed:
        return "gemm_w8p_kernel"
    t256 = -(-m // 256) * -(-n // 256)
    t128 = -(-m // 128) * -(-n // 256)

    def fill(t):
        return t / (-(-t // cus) * cus)

    big = k % 64 == 0 and m > 512 and n >= 256 and t256 >= cus * 5 // 8 and fill(t256) >= 0.83 * fill(t128)
    if big and n % 4 == 0 and k >= 512:
        return "gemm_persist_kernel"
    if k % 64 == 0:
        return "gemm_pipe_kernel"
    return "gemm_a8w8_kernel"


def block_measurement(dev, steps: int, warmup: int):
    """one H3-shape DiT block on the GPU (hidden 5120, 40 x 128 heads, GELU FFN 13824,
    S = 12090 video + 512 text tokens, bf16, AdaLN modulation precomputed ~N(0, 0.1), all four large linears
    W4A8 ConvRot QLinear with random-init weights of the BASELINE recipe, attention on PyTorch-ROCm SDPA).
    Returns the block's mean time over `steps` plus a split measured by running the same linears and SDPA alone."""
    import torch

    from h3turbo_amd import block as bk
    from h3turbo_amd import qlinear as ql
    from h3turbo_amd.types import BlockWeights, W4A8Weight

    s, hidden, heads, hd, ffn = 12602, 5120, 40, 128, 13824
    cfg = bk.BlockConfig(hidden=hidden, heads=heads, head_dim=hd, ffn=ffn, act="gelu")
    g = torch.Generator(device=dev).manual_seed(1)

    def lin(n, k, seed):
        q, s_rel, s_ch, cb = synth_weight(n, k, dev, seed=seed)
        return W4A8Weight(q, s_rel, s_ch, cb, group_size=128, convrot=256)

    ones = lambda d: 1.0 + 0.1 * torch.randn(d, generator=g, device=dev)  # noqa: E731
    w = BlockWeights(qkv=lin(3 * cfg.inner, hidden, 11), out=lin(hidden, cfg.inner, 12), fc1=lin(ffn, hidden, 13),
                     fc2=lin(hidden, ffn, 14), norm1=ones(hidden), norm2=ones(hidden), q_norm=ones(hd), k_norm=ones(hd))
    x0 = torch.randn(s, hidden, generator=g, device=dev).to(torch.bfloat16)
    mods = [torch.randn(1, hidden, generator=g, device=dev) * 0.1 for _ in range(6)]
    segs = [(0, s, 0)]
    pos = torch.stack(torch.meshgrid(torch.arange(31), torch.arange(15), torch.arange(26), indexing="ij"), -1).reshape(-1, 3)
    pos = torch.cat([pos + 1, torch.zeros(512, 3, dtype=pos.dtype)], 0)
    rope = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), dev, torch.bfloat16)
    blk = bk.DiTBlock(cfg)
    stream = torch.cuda.current_stream(dev)

    def timed(fn, n):
        evs = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            evs.append((e0, e1))
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in evs) / n

    xs = [x0.clone() for _ in range(warmup + steps)]
    it = iter(xs)
    timed(lambda: blk(next(it), w, mods, segs, rope), warmup)
    t_block = timed(lambda: blk(next(it), w, mods, segs, rope), steps)
    # split: the same calls alone, on inputs of the block's shapes
    h = torch.randn(s, hidden, generator=g, device=dev).to(torch.bfloat16)
    o = torch.randn(s, cfg.inner, generator=g, device=dev).to(torch.bfloat16)
    z = torch.randn(s, ffn, generator=g, device=dev).to(torch.bfloat16)
    t_lin = {name: timed(fn, steps) for name, fn in (("qkv", lambda: ql.linear(h, w.qkv)), ("out", lambda: ql.linear(o, w.out)),
                                                     ("fc1", lambda: ql.linear(h, w.fc1)), ("fc2", lambda: ql.linear(z, w.fc2)))}
    qh, kh, vh = (torch.randn(1, heads, s, hd, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    t_sdpa = timed(lambda: bk._sdpa(qh, kh, vh), steps)
    lin_ms = sum(t_lin.values())
    ops = 2.0 * s * hidden * (3 * cfg.inner + cfg.inner + 2 * ffn)
    sdpa_flop = 4.0 * s * s * hd * heads
    return {"config": "hidden 5120, 40x128 heads, GELU FFN 13824, S=12090+512, bf16, W4A8 linears, SDPA",
            "ms": round(t_block, 3), "steps": steps,
            "split_standalone_ms": {"linears": round(lin_ms, 3), **{k: round(v, 3) for k, v in t_lin.items()},
                                    "sdpa": round(t_sdpa, 3), "rest": round(t_block - lin_ms - t_sdpa, 3)},
            "linears_int8_TOPS": round(ops / (lin_ms * 1e-3) / 1e12, 1),
            "sdpa_bf16_TFLOPS": round(sdpa_flop / (t_sdpa * 1e-3) / 1e12, 1)}


def _config4_block_weights(dev, g):
    """Random-init W4A8 weights of one config-4 block (GELU), made on the GPU: int4 codes uniform over the codebook
    arange(-8, 8), group-128 fp16 scales in [12.875, 15.875], per-channel scale for ~N(0, 0.02) weights."""
    import torch

    from h3turbo_amd.types import BlockWeights, W4A8Weight

    def lin(n, k):
        q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8, device=dev)
        s_rel = (torch.rand(n, k // 128, generator=g, device=dev) * 3.0 + 12.875).to(torch.float16)
        s_ch = torch.full((n,), 0.02 * 3 ** 0.5 / (7.5 * 14.375), device=dev)
        return W4A8Weight(q, s_rel, s_ch, torch.arange(-8, 8, dtype=torch.float32, device=dev), group_size=128, convrot=256)

    ones = lambda d: (1.0 + 0.1 * torch.randn(d, generator=g, device=dev))  # noqa: E731
    return BlockWeights(qkv=lin(15360, 5120), out=lin(5120, 5120), fc1=lin(13824, 5120), fc2=lin(5120, 13824),
                        norm1=ones(5120), norm2=ones(5120), q_norm=ones(128), k_norm=ones(128))


def model_measurement(dev, layers: int, steps: int):
    """The whole H3 model forward (one sampler step) at the real H3 shape: hidden 5376, 56 x 128 heads, SwiGLU FFN
    14336, `layers` DiT blocks resident in HBM with W4A8 linears in the checkpoint's format (fp8 e4m3 group-16
    scales, rotation 256, random codes), a dense bf16 2-block token refiner, S = 112 text + 400 audio + 12090 video
    tokens (latent 31 x 30 x 52), bf16 compute.  Times encode_text once and the forward (embedding, every block,
    final layer) over `steps` calls after one warmup."""
    import torch

    from h3turbo_amd.block import ResidentProvider
    from h3turbo_amd.config import H3Config
    from h3turbo_amd.model import H3Model
    from h3turbo_amd.types import BlockWeights, GlobalWeights, W4A8Weight

    cfg = H3Config(layers=layers)
    hid, inner, ffn, td = cfg.hidden, cfg.inner, cfg.ffn, cfg.t_dim
    g = torch.Generator(device=dev).manual_seed(7)
    f32, bf = torch.float32, torch.bfloat16

    def rn(*shape, std=1.0, dtype=f32):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dtype)

    cb = torch.linspace(-1, 1, 16, device=dev)

    def w4(n, k):
        q = torch.randint(-128, 128, (n, k // 2), generator=g, device=dev, dtype=torch.int8)
        s_rel = (20 + 100 * torch.rand(n, k // 16, generator=g, device=dev)).to(torch.float8_e4m3fn)
        s_ch = torch.full((n,), k ** -0.5 / 40.0, device=dev)
        return W4A8Weight(q, s_rel, s_ch, cb, group_size=16, convrot=256)

    def ones(d):
        return (1.0 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf)

    blocks = [BlockWeights(qkv=w4(3 * inner, hid), out=w4(hid, inner), fc1=w4(2 * ffn, hid), fc2=w4(hid, ffn),
                           norm1=ones(hid), norm2=ones(hid), q_norm=ones(cfg.head_dim), k_norm=ones(cfg.head_dim),
                           adaln_w=rn(18 * hid, td, std=0.05), adaln_b=rn(18 * hid, std=0.05)) for _ in range(layers)]
    refiner = [BlockWeights(qkv=rn(3 * inner, hid, std=hid ** -0.5, dtype=bf), out=rn(hid, inner, std=inner ** -0.5, dtype=bf),
                            fc1=rn(2 * ffn, hid, std=hid ** -0.5, dtype=bf), fc2=rn(hid, ffn, std=ffn ** -0.5, dtype=bf),
                            norm1=ones(hid), norm2=ones(hid), q_norm=ones(cfg.head_dim), k_norm=ones(cfg.head_dim))
               for _ in range(cfg.refiner_layers)]
    grid = torch.linspace(0, 1, cfg.curve_grid, device=dev)
    pd, ac = cfg.video_patch_dim, cfg.audio_channels
    glob = GlobalWeights(
        video_patch_w=rn(hid, pd, std=0.1), video_patch_b=rn(hid, std=0.1), audio_patch_w=rn(hid, ac, std=0.1),
        audio_patch_b=rn(hid, std=0.1), condition_w=rn(hid, cfg.text_dim, std=cfg.text_dim ** -0.5, dtype=bf),
        condition_b=rn(hid, std=0.1, dtype=bf),
        adaln_t_table=torch.stack([torch.sin(6.28 * (1 + j) * grid + j) * 0.5 for j in range(td)], 1),
        rope_inv_freq=1.0 / (10000.0 ** (torch.arange(cfg.rope_inv_freq_len, device=dev) / cfg.rope_inv_freq_len)),
        final_norm=ones(hid), final_adaln_w=rn(2 * hid, td, std=0.05), final_adaln_b=rn(2 * hid, std=0.05),
        video_out_w=rn(pd, hid, std=hid ** -0.5), video_out_b=rn(pd, std=0.1), audio_out_w=rn(ac, hid, std=hid ** -0.5),
        audio_out_b=rn(ac, std=0.1), refiner=refiner, refiner_final_norm=ones(hid))
    m = H3Model(cfg, glob, ResidentProvider(blocks), device=dev, dtype=bf)
    video = rn(1, cfg.video_channels, 31, 30, 52, dtype=bf)
    audio = rn(1, ac, 2, 200, dtype=bf)
    text = rn(1, 112, cfg.text_dim, dtype=bf)
    weights_gb = sum(w.nbytes for b in blocks for w in (b.qkv, b.out, b.fc1, b.fc2)) / 1e9
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    refined = m.encode_text(text)
    torch.cuda.synchronize()
    t_text = time.perf_counter() - t0
    out = m.forward([video, audio], 0.7, None, refined_text=refined)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = m.forward([video, audio], 0.7, None, refined_text=refined)
    torch.cuda.synchronize()
    t_fwd = (time.perf_counter() - t0) / steps
    ok = bool(torch.isfinite(out[0]).all() and torch.isfinite(out[1]).all())
    del blocks, glob, m, out
    torch.cuda.empty_cache()
    return {"config": f"H3 shape: hidden 5376, {layers} blocks, 56x128 heads, SwiGLU FFN 14336, W4A8 fp8 g16 (resident), "
                      "dense bf16 refiner x2, S=12602 (text 112 + audio 2x200 + video 31x15x26), bf16",
            "blocks_GB": round(weights_gb, 2), "encode_text_ms": round(t_text * 1e3, 2),
            "forward_s": round(t_fwd, 4), "ms_per_block": round(t_fwd * 1e3 / layers, 3), "steps": steps,
            "outputs_finite": ok}


def stream_measurement(dev, n_blocks: int):
    """a stack of n_blocks config-4 blocks whose random-init W4A8 weights live in pinned host
    RAM, run for one denoising step (12090 + 512 tokens) three ways: all resident in HBM (t_comp), streamed through
    a 3-slot ring with 2-block lookahead on a side stream (t_both), and the copies alone (t_copy: every block
    host -> HBM back to back).  overlap = (t_comp + t_copy - t_both) / min(t_comp, t_copy), the definition of the
    reference's stream check (scripts/h3_check_stream_gpu.py:204-205).  The streamed output must equal the resident
    output bit for bit."""
    import torch

    from h3turbo_amd import block as bk
    from h3turbo_amd.blockstore import BlockLayout, HostBlockStore, block_tensors
    from h3turbo_amd.stream import StreamingProvider, hip_transfer

    g = torch.Generator(device=dev).manual_seed(5)
    t0 = time.perf_counter()
    first = block_tensors(_config4_block_weights(dev, g))
    store = HostBlockStore(BlockLayout.of(first), n_blocks, 128, 256, pinned=True)
    store.write_block(0, first)
    for i in range(1, n_blocks):
        store.write_block(i, block_tensors(_config4_block_weights(dev, g)))
    t_setup = time.perf_counter() - t0
    s, hidden = 12602, 5120
    cfg = bk.BlockConfig(hidden=hidden, heads=40, head_dim=128, ffn=13824, act="gelu")
    x0 = torch.randn(s, hidden, generator=g, device=dev).to(torch.bfloat16)
    mods = [torch.randn(1, hidden, generator=g, device=dev) * 0.1 for _ in range(6)]
    pos = torch.stack(torch.meshgrid(torch.arange(31), torch.arange(15), torch.arange(26), indexing="ij"), -1).reshape(-1, 3)
    pos = torch.cat([pos + 1, torch.zeros(512, 3, dtype=pos.dtype)], 0)
    rope = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), dev, torch.bfloat16)
    blk = bk.DiTBlock(cfg)

    def forward_time(p):
        bk.run_blocks(blk, x0.clone(), p, n_blocks, lambda i, w: mods, [(0, s, 0)], rope)  # warm (and prefetch)
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = bk.run_blocks(blk, x0.clone(), p, n_blocks, lambda i, w: mods, [(0, s, 0)], rope)
        torch.cuda.synchronize()
        return time.perf_counter() - t, out

    with StreamingProvider(store, dev, resident=n_blocks) as p:
        t_comp, out_res = forward_time(p)
    with StreamingProvider(store, dev, resident=0, ring=3, prefetch=2) as p:
        t_both, out_str = forward_time(p)
        st = p.stats()
    slot = torch.empty(store.block_nbytes, dtype=torch.uint8, device=dev)
    cs = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cs):
        e0.record(cs)
        for i in range(n_blocks):
            hip_transfer(slot, store.block_tensor(i), True)
        e1.record(cs)
    torch.cuda.synchronize()
    t_copy = e0.elapsed_time(e1) * 1e-3
    overlap = (t_comp + t_copy - t_both) / min(t_comp, t_copy)
    return {"config": f"{n_blocks} config-4 blocks (GELU, W4A8 g128 fp16 scales), S=12090+512, weights in pinned host RAM",
            "block_MB": round(store.block_nbytes / 1e6, 1), "stack_GB": round(store.nbytes / 1e9, 2),
            "resident_forward_s": round(t_comp, 4), "streamed_forward_s": round(t_both, 4), "copy_only_s": round(t_copy, 4),
            "h2d_GB_per_s": round(store.nbytes / t_copy / 1e9, 1), "overlap": round(overlap, 3),
            "streamed_equals_resident": bool(torch.equal(out_res, out_str)),
            "waits": st["waits"], "host_kinds": st["host_kinds"], "setup_s": round(t_setup, 1)}


def h3t_measurement(dev, n_blocks: int):
    """The .h3t container at the config-4 block shape: n_blocks random-init W4A8 blocks (GELU, g128 fp16 scales)
    written as an .h3t file (the format of h3turbo/h3/store.py), loaded into pinned host memory
    (HostBlockStore.from_h3t), then one streamed step (12090 + 512 tokens) with the blocks coming from the pinned
    copy and from the file mapping (pageable pages copied through two pinned staging buffers).  Both outputs must equal
    the all-resident output bit for bit."""
    import json as _json
    import tempfile

    import torch

    from h3turbo_amd import block as bk
    from h3turbo_amd import h3t
    from h3turbo_amd.blockstore import HostBlockStore, block_tensors
    from h3turbo_amd.config import H3Config
    from h3turbo_amd.stream import StreamingProvider

    g = torch.Generator(device=dev).manual_seed(7)
    qjson = torch.tensor(list(_json.dumps({"format": "asym_w4a8_int8", "group_size": 128, "convrot_groupsize": 256},
                                          separators=(",", ":")).encode()), dtype=torch.uint8)
    tensors = {}
    for i in range(n_blocks):
        for name, t in block_tensors(_config4_block_weights(dev, g)).items():
            tensors[f"blocks.{i}.{name}"] = t
        for p in ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2"):
            tensors[f"blocks.{i}.{p}.comfy_quant"] = qjson
    cfg = H3Config(hidden=5120, layers=n_blocks, heads=40, head_dim=128, ffn=13824, quant_group=128, quant_convrot=256)
    tmpdir = tempfile.mkdtemp(prefix="h3t_bench_")
    path = os.path.join(tmpdir, "stack.h3t")
    try:
        t0 = time.perf_counter()
        h3t.write_h3t(path, cfg, tensors)
        t_write = time.perf_counter() - t0
        del tensors
        nbytes = os.path.getsize(path)
        with h3t.H3TFile(path) as f:
            t0 = time.perf_counter()
            pinned = HostBlockStore.from_h3t(f, pinned=True)
            t_load = time.perf_counter() - t0
            s, hidden = 12602, 5120
            blk = bk.DiTBlock(bk.BlockConfig(hidden=hidden, heads=40, head_dim=128, ffn=13824, act="gelu"))
            x0 = torch.randn(s, hidden, generator=g, device=dev).to(torch.bfloat16)
            mods = [torch.randn(1, hidden, generator=g, device=dev) * 0.1 for _ in range(6)]
            pos = torch.stack(torch.meshgrid(torch.arange(31), torch.arange(15), torch.arange(26), indexing="ij"), -1).reshape(-1, 3)
            pos = torch.cat([pos + 1, torch.zeros(512, 3, dtype=pos.dtype)], 0)
            rope = bk.rope_tables(pos, 1.0 / (10000.0 ** (torch.arange(16) / 16.0)), dev, torch.bfloat16)

            def forward_time(p):
                bk.run_blocks(blk, x0.clone(), p, n_blocks, lambda i, w: mods, [(0, s, 0)], rope)
                torch.cuda.synchronize()
                t = time.perf_counter()
                out = bk.run_blocks(blk, x0.clone(), p, n_blocks, lambda i, w: mods, [(0, s, 0)], rope)
                torch.cuda.synchronize()
                return time.perf_counter() - t, out

            with StreamingProvider(pinned, dev, resident=n_blocks) as p:
                t_res, out_res = forward_time(p)
            with StreamingProvider(pinned, dev, resident=0, ring=3, prefetch=2) as p:
                t_pin, out_pin = forward_time(p)
                kinds_pin = p.stats()["host_kinds"]
            with StreamingProvider(f, dev, resident=0, ring=3, prefetch=2, pin_mode="stage") as p:
                t_map, out_map = forward_time(p)
                kinds_map = p.stats()["host_kinds"]
        return {"config": f"{n_blocks} config-4 blocks (GELU, W4A8 g128 fp16 scales) in one .h3t file, S=12090+512",
                "file_MB": round(nbytes / 1e6, 1), "block_MB": round(pinned.block_nbytes / 1e6, 1),
                "write_s": round(t_write, 2), "load_pinned_s": round(t_load, 3),
                "load_pinned_GB_per_s": round(pinned.nbytes / t_load / 1e9, 2),
                "resident_forward_s": round(t_res, 4), "streamed_from_pinned_s": round(t_pin, 4),
                "streamed_from_file_mapping_s": round(t_map, 4), "host_kinds_pinned": kinds_pin,
                "host_kinds_mapping": kinds_map,
                "outputs_equal_resident": bool(torch.equal(out_pin, out_res) and torch.equal(out_map, out_res))}
    finally:
        try:
            os.remove(path)
        except OSError:
            pass
        os.rmdir(tmpdir)


def sweep_measurement(dev, steps: int):
    """the QLinear at M in {512, 4096, 12090, 32768} x (K, N) in {(5120, 5120), (5120, 15360),
    (5120, 13824), (13824, 5120)}, weights of the BASELINE recipe.  Per shape: mean time of rotate+quant, decode,
    GEMM (HIP events on the launch stream) and int8 TOPS of the GEMM and of the whole op."""
    import torch

    from h3turbo_amd import _lib
    from h3turbo_amd import qlinear as ql
    from h3turbo_amd.types import W4A8Weight

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rows = []
    for k, n in ((5120, 5120), (5120, 15360), (5120, 13824), (13824, 5120)):
        q, s_rel, s_ch, cb = synth_weight(n, k, dev)
        dw = ql._DevWeight(W4A8Weight(q, s_rel, s_ch, cb, group_size=128, convrot=256))
        w8 = torch.empty(lib.h3k_w8_packed_bytes(n, k), dtype=torch.int8, device=dev)  # >= n * k
        for m in (512, 4096, 12090, 32768):
            g = torch.Generator(device=dev).manual_seed(m)
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            xq = torch.empty(m, k, dtype=torch.int8, device=dev)
            xs = torch.empty(m, 1, dtype=torch.float32, device=dev)
            out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            packed = bool(lib.h3k_gemm_packed_serves(m, n, k))  # the route qlinear.linear takes
            split = lib.h3k_gemm_packed_split_bytes(m, n, k) if packed else 0  # ... with the split tail where it pays
            ws = torch.empty(max(split, 4) // 4, dtype=torch.int32, device=dev)
            rq = lambda: lib.h3k_rotate_quant(x.data_ptr(), _lib.BF16, m, k, k, 256, 0, xq.data_ptr(), k, xs.data_ptr(), sp)
            if packed:
                calls = [rq,
                         lambda: lib.h3k_decode_w4_packed(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds,
                                                          dw.cb.data_ptr(), n, k, 128, w8.data_ptr(), sp),
                         lambda: lib.h3k_gemm_a8w8_packed_ws(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(),
                                                             dw.s_ch.data_ptr(), None, m, n, k, 0, out.data_ptr(), _lib.BF16,
                                                             n, ws.data_ptr(), split, sp)]
            else:
                calls = [rq,
                         lambda: lib.h3k_decode_w4(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds, dw.cb.data_ptr(),
                                                   n, k, 128, w8.data_ptr(), k, sp),
                         lambda: lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, dw.s_ch.data_ptr(), None,
                                                   m, n, k, 0, out.data_ptr(), _lib.BF16, n, None, sp)]
            for _ in range(2):
                for c in calls:
                    _lib.check(c(), "sweep")
            ev = [[] for _ in calls]
            for _ in range(steps):
                for i, c in enumerate(calls):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    _lib.check(c(), "sweep")
                    e1.record(stream)
                    ev[i].append((e0, e1))
            torch.cuda.synchronize()
            t = [sum(a.elapsed_time(b) for a, b in e) / len(e) for e in ev]
            ops = 2.0 * m * n * k
            rows.append({"m": m, "k": k, "n": n,
                         "kernel": gemm_kernel_name(m, n, k, packed, cus) + (" + w8p_fixup_kernel" if split else ""),
                         "rotquant_ms": round(t[0], 4), "decode_ms": round(t[1], 4),
                         "gemm_ms": round(t[2], 4), "gemm_TOPS": round(ops / (t[2] * 1e-3) / 1e12, 1),
                         "op_TOPS": round(ops / (sum(t) * 1e-3) / 1e12, 1),
                         "gemm_frac_peak": round(ops / (t[2] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)})
            del x, xq, xs, out
        del dw, w8
    return rows


def rotquant_config2(dev, steps: int = 20, rot: int = 128):
    """rotate + quantise bf16 activations [12090, 5120] (1 % outlier channels x20) with the
    config's 128-wide block-Hadamard (an extension of the reference, which takes powers of 4), per-token int8 output
    and fp32 scales; mean of `steps` launches (HIP events on the launch stream), HBM bytes = 2 MK read + MK + 4 M
    written."""
    import torch

    from h3turbo_amd import _lib

    lib = _lib.load()
    m, k = 12090, 5120
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(m, k, generator=g, device=dev)
    x[:, torch.randperm(k, generator=g, device=dev)[: round(0.01 * k)]] *= 20
    x = x.to(torch.bfloat16)
    xq = torch.empty(m, k, dtype=torch.int8, device=dev)
    xs = torch.empty(m, 1, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    def call():
        _lib.check(lib.h3k_rotate_quant(x.data_ptr(), _lib.BF16, m, k, k, rot, 0, xq.data_ptr(), k, xs.data_ptr(), sp), "rq2")

    for _ in range(3):
        call()
    ev = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        call()
        e1.record(stream)
        ev.append((e0, e1))
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
    nbytes = 2 * m * k + m * k + 4 * m
    return {"m": m, "k": k, "rot": rot, "ms": round(ms, 4), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def few_rows_measurement(dev, steps: int):
    """Small-M W4A8 GEMMs against HBM: the BASELINE weight shape (N=13824, K=5120) with the BASELINE recipe (group
    128, fp16 scales) and the checkpoint format (group 16, fp8 scales), M in {16, 32, 48, 64, 128}.  The fused few-row GEMM
    (h3k_gemm_w4a8: int4 decoded in registers; zero-fill, GEMM and epilogue launches when it splits K) against the
    decode + int8 GEMM pair it replaces.  HBM figure = algorithmic bytes (packed weight + scales + int8 activations
    + xs + s_ch + bf16 out) / time of the fused call: back-to-back calls between HIP events on the launch stream."""
    import torch

    from h3turbo_amd import _lib
    from h3turbo_amd import qlinear as ql
    from h3turbo_amd.types import W4A8Weight

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    n, k = 13824, 5120
    rows = []

    def timed(fn):
        # back-to-back calls between one pair of events: a single call of ~10-20 us bracketed by events would also
        # time the dispatch gap in front of it
        for _ in range(3):
            _lib.check(fn(), "few rows")
        reps = max(20, 4 * steps)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            _lib.check(fn(), "few rows")
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for fmt in ("g128_f16", "g16_fp8"):
        if fmt == "g128_f16":
            q, s_rel, s_ch, cb = synth_weight(n, k, dev)
            w = W4A8Weight(q, s_rel, s_ch, cb, group_size=128, convrot=256)
        else:
            g = torch.Generator(device=dev).manual_seed(5)
            q = torch.randint(-128, 128, (n, k // 2), generator=g, device=dev, dtype=torch.int8)
            s8 = (20 + 100 * torch.rand(n, k // 16, generator=g, device=dev)).to(torch.float8_e4m3fn)
            w = W4A8Weight(q, s8, torch.full((n,), 1e-3, device=dev), torch.linspace(-1, 1, 16, device=dev), 16, 256)
        dw = ql._DevWeight(w)
        grp = w.group_size
        sbytes = dw.s.numel() * dw.s.element_size()
        w8 = torch.empty(n, k, dtype=torch.int8, device=dev)
        for m in (16, 32, 48, 64, 128):  # the routing cut (32 rows) sits between the 32 and 48 measurements
            g = torch.Generator(device=dev).manual_seed(m)
            xq = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
            xs = torch.rand(m, 1, generator=g, device=dev) * 1e-3
            out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            out2 = torch.empty_like(out)
            nb = lib.h3k_gemm_w4a8_workspace(m, n, k)
            ws = torch.empty(max(1, nb // 4), dtype=torch.int32, device=dev)
            fused = lambda: lib.h3k_gemm_w4a8(xq.data_ptr(), k, xs.data_ptr(), dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(),  # noqa: E731
                                               dw.scode, dw.lds, dw.cb.data_ptr(), grp, dw.s_ch.data_ptr(), None, m, n, k,
                                               0, out.data_ptr(), _lib.BF16, n, ws.data_ptr(), None, sp)
            dec = lambda: lib.h3k_decode_w4(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds,  # noqa: E731
                                            dw.cb.data_ptr(), n, k, grp, w8.data_ptr(), k, sp)
            gemm = lambda: lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, dw.s_ch.data_ptr(),  # noqa: E731
                                             None, m, n, k, 0, out2.data_ptr(), _lib.BF16, n, None, sp)
            t_f, t_d, t_g = timed(fused), timed(dec), timed(gemm)
            same = bool(torch.equal(out, out2))
            alg = n * k // 2 + sbytes + m * k + 4 * m + 4 * n + 2 * m * n
            gbs = alg / (t_f * 1e-3) / 1e9
            rows.append({"weight": fmt, "m": m, "fused_ms": round(t_f, 4), "fused_GB/s": round(gbs, 1),
                         "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "decode_plus_gemm_ms": round(t_d + t_g, 4),
                         "speedup": round((t_d + t_g) / t_f, 2), "outputs_equal": same})
            del xq, xs, out, out2, ws
        del dw, w8, w
    return {"config": "N=13824 K=5120 (BASELINE weight), bf16 out, ck epilogue", "rows": rows}


def cpu_baseline(m: int, k: int, n: int, rows: int):
    """Time the CPU oracle (restatement of the reference's torch CPU backend) on `rows` rows of the workload plus
    one per-call weight decode, and scale to M rows: TOPS = 2MNK / (t_decode + t_rows * M / rows)."""
    import numpy as np

    import inputs as gi
    from oracle import qlinear_ref as ref

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads") or 1) for i in threadpool_info()) if threadpool_info() else 1
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    xb = gi.activations(rows, k, seed=0)
    q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=0)
    x = ref.bf16_from_bits(xb)
    t_dec, t_rows = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        w8 = ref.decode_int8_grid(q, s_rel, "f16", cb, 128)
        t1 = time.perf_counter()
        xq, xs = ref.quantize_rows(x, "bf16", 256, "ck")
        acc = ref.int8_mm_emulated(xq, w8)
        ref.epilogue(acc, xs, s_ch, "bf16", "ck")
        t2 = time.perf_counter()
        t_dec.append(t1 - t0)
        t_rows.append(t2 - t1)
    td, tr = sorted(t_dec)[1], sorted(t_rows)[1]
    total = td + tr * m / rows
    return {"value": round(2.0 * m * n * k / total / 1e12, 4), "unit": "TOPS", "cores": int(threads), "kind": "port",
            "sample": f"oracle/qlinear_ref.py on {rows} of {m} rows (K={k}, N={n}) + one per-call weight decode, "
                      f"median of 3; scaled to {m} rows: decode {td:.2f} s + rows {tr:.2f} s x {m / rows:.0f}",
            "seconds_for_full_op": round(total, 2), "config1": cpu_config1(threads)}


def cpu_config1(threads: int, runs: int = 7):
    """BASELINE config 1 measured whole on the host: one W4A8 ConvRot QLinear, bf16 activations [256, 1024] with 1 %
    outlier channels x20, int4 group-128 weight with fp16 scales [1024, 1024], seed 0, the config's rotation 128
    (the oracle's extension of the reference), through the CPU oracle (weight decode + rotate/quantise + exact int8
    GEMM + epilogue); one warm-up, then the median of `runs` runs."""
    import numpy as np

    import inputs as gi
    from oracle import qlinear_ref as ref

    m, k, n = 256, 1024, 1024
    x = ref.bf16_from_bits(gi.activations(m, k, seed=0))
    q, s_rel, s_ch, cb = gi.weight_int4_g128(n, k, seed=0)

    def once():
        w8 = ref.decode_int8_grid(q, s_rel, "f16", cb, 128)
        xq, xs = ref.quantize_rows(x, "bf16", 128, "ck")
        return ref.epilogue(ref.int8_mm_emulated(xq, w8), xs, s_ch, "bf16", "ck")

    once()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"ms": round(med * 1e3, 2), "TOPS": round(2.0 * m * n * k / med / 1e12, 6), "cores": int(threads),
            "runs": runs, "sample": f"config 1 whole: M={m} K={k} N={n}, rotation 128, median of {runs} after 1 warm-up"}


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    from h3turbo_amd import _lib
    from h3turbo_amd import qlinear as ql
    from h3turbo_amd.types import W4A8Weight

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    m, k, n = args.m, args.k, args.n
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(m, k, generator=g, device=dev)
    idx = torch.randperm(k, generator=g, device=dev)[: round(0.01 * k)]
    x[:, idx] *= 20
    x = x.to(torch.bfloat16)
    q, s_rel, s_ch, cb = synth_weight(n, k, dev)
    w = W4A8Weight(q, s_rel, s_ch, cb, group_size=128, convrot=256)

    lib = _lib.load()
    dw = ql._DevWeight(w)
    packed = bool(lib.h3k_gemm_packed_serves(m, n, k))
    xq = torch.empty(m, k, dtype=torch.int8, device=dev)
    xs = torch.empty(m, 1, dtype=torch.float32, device=dev)
    w8 = torch.empty(lib.h3k_w8_packed_bytes(n, k) if packed else n * k, dtype=torch.int8, device=dev)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    ev = {name: [] for name in ("rq", "dec", "gemm")}

    def step(record: bool):
        def mark():
            if record:
                e = torch.cuda.Event(enable_timing=True)
                e.record(stream)
                return e
            return None

        e0 = mark()
        _lib.check(lib.h3k_rotate_quant(x.data_ptr(), _lib.BF16, m, k, k, 256, 0, xq.data_ptr(), k, xs.data_ptr(), sp), "rq")
        e1 = mark()
        if packed:  # the route qlinear.linear takes for this shape: packed weight grid + packed-weight GEMM
            _lib.check(lib.h3k_decode_w4_packed(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds,
                                                dw.cb.data_ptr(), n, k, 128, w8.data_ptr(), sp), "decode")
        else:
            _lib.check(lib.h3k_decode_w4(dw.q.data_ptr(), dw.ldq, dw.s.data_ptr(), dw.scode, dw.lds, dw.cb.data_ptr(), n,
                                         k, 128, w8.data_ptr(), k, sp), "decode")
        e2 = mark()
        if packed:
            _lib.check(lib.h3k_gemm_a8w8_packed(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), dw.s_ch.data_ptr(), None,
                                                m, n, k, 0, out.data_ptr(), _lib.BF16, n, None, sp), "gemm")
        else:
            _lib.check(lib.h3k_gemm_a8w8(xq.data_ptr(), k, xs.data_ptr(), w8.data_ptr(), k, dw.s_ch.data_ptr(), None, m,
                                         n, k, 0, out.data_ptr(), _lib.BF16, n, None, sp), "gemm")
        e3 = mark()
        if record:
            ev["rq"].append((e0, e1))
            ev["dec"].append((e1, e2))
            ev["gemm"].append((e2, e3))

    # the step must equal the public API's result (checked first: the warmup then runs right before the timed
    # region, so the timed launches start at the sustained shader clock)
    step(False)
    torch.cuda.synchronize()
    assert torch.equal(out, ql.linear(x, w)), "bench step differs from qlinear.linear"
    for _ in range(args.warmup):
        step(False)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps

    def mean_ms(pairs):
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    t_rq, t_dec, t_gemm = mean_ms(ev["rq"]), mean_ms(ev["dec"]), mean_ms(ev["gemm"])
    ops = 2.0 * m * n * k
    kname = gemm_kernel_name(m, n, k, packed, torch.cuda.get_device_properties(dev).multi_processor_count)
    tops = ops / (ms_step * 1e-3) / 1e12
    gemm_tops = ops / (t_gemm * 1e-3) / 1e12
    rq_bytes = 2 * m * k + m * k + 4 * m
    dec_bytes = n * k // 2 + n * (k // 128) * 2 + n * k
    line = {
        "metric": "int8 TOPS (% MFMA peak) for W4A8 QLinear at M=32768; H3 DiT block ms",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"W4A8 ConvRot QLinear M={m} K={k} N={n}: bf16 x (1% outlier channels x20), int4 weight "
                               "group 128 fp16 scales, block-Hadamard 256, bf16 out",
                   "m": m, "k": k, "n": n, "group": 128, "convrot": 256},
        "pct_mfma_peak": round(100.0 * tops / PEAK_INT8_TOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(gemm_tops / PEAK_INT8_TOPS, 4), "traffic": traffic_from_profiles(f"{kname} m={m} k={k} n={n}"),
                     "kernel": kname, "kernel_ms": round(t_gemm, 4)},
        "kernels": {
            "rotate_quant": {"ms": round(t_rq, 4), "GB/s": round(rq_bytes / (t_rq * 1e-3) / 1e9, 1),
                             "frac_hbm": round(rq_bytes / (t_rq * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
            "decode_w4": {"ms": round(t_dec, 4), "GB/s": round(dec_bytes / (t_dec * 1e-3) / 1e9, 1),
                          "frac_hbm": round(dec_bytes / (t_dec * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
            "gemm_a8w8": {"ms": round(t_gemm, 4), "TOPS": round(gemm_tops, 1)},
        },
    }
    line["kernels"]["rotate_quant_config2"] = rotquant_config2(dev, rot=128)
    line["kernels"]["rotate_quant_config2_rot256"] = rotquant_config2(dev, rot=256)
    line["kernels"]["decode_w4_packed_g16_fp8"] = decode_packed_g16_fp8(dev)
    if not args.no_block:
        del xq, w8, out
        line["block"] = block_measurement(dev, args.block_steps, max(1, args.warmup))
    if not args.no_sweep:
        line["sweep"] = sweep_measurement(dev, 10)
    if not args.no_few_rows:
        line["few_rows"] = few_rows_measurement(dev, 20)
    if not args.no_model:
        line["model"] = model_measurement(dev, args.model_layers, 2)
    if not args.no_stream:
        line["stream"] = stream_measurement(dev, args.stream_blocks)
    if not args.no_h3t:
        line["h3t"] = h3t_measurement(dev, args.h3t_blocks)
    if args.copy_probe:
        src = torch.full((args.copy_probe,), 1, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            torch.bitwise_not(src, out=dst)  # one plain read + write pass over copy_probe bytes
        torch.cuda.synchronize()
        line["copy_probe_bytes"] = args.copy_probe
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(m, k, n, args.cpu_rows)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
