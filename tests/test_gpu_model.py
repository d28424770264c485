"""The whole-model forward on the GPU (h3turbo_amd.model: W4A8 linears on the HIP kernels, fused attention prologue /
epilogue, fused RMSNorm + modulation) against the CPU model oracle (oracle/model_ref.py), streamed against resident,
and the engine's sampler over an .h3t file."""
import pytest
import torch

import model_cases as mc
from h3turbo_amd import _lib
from h3turbo_amd.block import ResidentProvider
from h3turbo_amd.model import H3Model, weights_from_state_dict
from oracle import model_ref as mr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
CFG4 = mc.W4CFG
PREFIXES = [f"blocks.{i}" for i in range(CFG4.layers)] + ["token_refiner.blocks.0"]


def w4a8_case(seed):
    sd, lin = mc.with_w4a8(CFG4, mc.make_sd(CFG4, seed), seed + 1, PREFIXES)
    return sd, lin


def gpu_model(cfg, sd, dtype=torch.bfloat16, provider=None, **kw) -> H3Model:
    glob, blocks = weights_from_state_dict(sd, cfg, DEV, dtype)
    return H3Model(cfg, glob, provider(blocks) if provider else ResidentProvider(blocks), device=DEV, dtype=dtype, **kw)


def test_w4a8_forward_matches_the_cpu_oracle():
    """bf16 compute, every linear W4A8 (12 of them, fp8 group-16 scales).  Each W4A8 linear is bit-exact with the
    oracle's; what differs is attention (PyTorch-ROCm's bf16 flash kernel against fp32 softmax attention rounded
    once) and norm reduction orders, whose final-bit differences the next int8 quantiser can turn into one step:
    held to rel-L2 against the oracle, and to the activation-quantisation noise against the dense fp64 network."""
    assert _lib.load() is not None
    sd, lin = w4a8_case(41)
    video, audio, text = mc.inputs(CFG4, 42, t=3, h=6, w=8, ta=6, text_len=7)
    print(f"model W4A8 cfg={CFG4} video={tuple(video.shape)}", flush=True)
    m = gpu_model(CFG4, sd)
    xb = [video.bfloat16(), audio.bfloat16()]
    got = m.forward([t.to(DEV) for t in xb], 0.6, text.bfloat16().to(DEV))
    assert got[0].device.type == "cuda" and got[0].dtype == torch.bfloat16
    plan = mc.plan_data(CFG4, text.shape[1], video, audio, 0.6)
    want = mr.model_ref(sd, CFG4, xb[0], xb[1], text.bfloat16(), plan, dtype=torch.bfloat16, linears=lin)
    dense = mr.model_naive(mc.dense_equivalent(sd, lin), CFG4, video, audio, text, plan)
    r = [mc.rel(got[i].cpu(), want[i]) for i in range(2)]
    r_dense = [mc.rel(got[i].cpu(), dense[i]) for i in range(2)]
    r_oracle_dense = [mc.rel(want[i], dense[i]) for i in range(2)]
    print({"rel_vs_oracle": r, "rel_vs_dense": r_dense, "oracle_vs_dense": r_oracle_dense}, flush=True)
    assert max(r) < 3e-2
    assert max(r_dense) < 5e-2


def test_fp32_dense_forward_equals_the_definition():
    sd = mc.make_sd(mc.CFG, 43)
    video, audio, text = mc.inputs(mc.CFG, 44)
    m = gpu_model(mc.CFG, sd, dtype=torch.float32)
    got = m.forward([video.to(DEV), audio.to(DEV)], 0.7, text.to(DEV))
    want = mr.model_naive(sd, mc.CFG, video, audio, text, mc.plan_data(mc.CFG, text.shape[1], video, audio, 0.7))
    assert mc.rel(got[0].cpu(), want[0]) < 1e-5 and mc.rel(got[1].cpu(), want[1]) < 1e-5


def test_conditioned_forward_with_masks_matches_the_cpu_oracle():
    sd, lin = w4a8_case(45)
    video, audio, text = mc.inputs(CFG4, 46)
    g = torch.Generator().manual_seed(47)
    kv, ka = torch.randn(1, 24, 1, 4, 6, generator=g), torch.randn(1, 32, 2, 3, generator=g)
    kfs = [{"resolved_frame_index": 4, "latent": kv, "audio_latent": ka}]
    payload = {"keyframes": kfs, "cond_video_latents": [kv], "cond_audio_latents": [ka], "visual_cond_noise_aug": 1.0,
               "audio_cond_noise_aug": 1.0, "text_token_tags": torch.tensor([[1, 1, 0, 2, 1]])}
    dm = torch.ones(1, 1, 2, 4, 6)
    dm[:, :, 0] = 0.0
    dm[:, :, 1, :2, :2] = 0.5
    m = gpu_model(CFG4, sd)
    xb = [video.bfloat16(), audio.bfloat16()]
    got = m.forward([t.to(DEV) for t in xb], 0.45, text.bfloat16().to(DEV), payload=payload, denoise_mask=dm.to(DEV))
    plan = mc.plan_data(CFG4, text.shape[1], video, audio, 0.45, keyframes=kfs, visual_aug=1.0, audio_aug=1.0,
                        text_tags=payload["text_token_tags"], denoise_mask=dm)
    want = mr.model_ref(sd, CFG4, xb[0], xb[1], text.bfloat16(), plan, dtype=torch.bfloat16, linears=lin,
                        cond_video_rows=mr.patchify(kv), cond_audio_rows=mr.pack(ka))
    want[0] = (want[0] * dm).to(torch.bfloat16)  # masked rows: velocity scaled by the mask (model.py:404-407)
    r = [mc.rel(got[i].cpu(), want[i]) for i in range(2)]
    print({"rel_vs_oracle": r}, flush=True)
    assert max(r) < 3e-2
    assert not got[0][:, :, 0].any()


def test_streamed_engine_equals_resident_and_samples(tmp_path):
    """A W4A8 .h3t with the globals: the engine streaming every block through two slots gives the resident
    engine's velocity bit for bit, and its sampler is the Euler loop over those velocities."""
    from h3turbo_amd.engine import H3Engine, h3_sigmas
    from h3turbo_amd.h3t import write_h3t
    from h3turbo_amd.layout import time_shift_sigma

    sd, _ = w4a8_case(48)
    path = tmp_path / "w4.h3t"
    write_h3t(path, CFG4, sd)
    video, audio, text = mc.inputs(CFG4, 49)
    x = [video.bfloat16().to(DEV), audio.bfloat16().to(DEV)]
    outs = []
    for kw in (dict(resident="auto"), dict(resident=0, ring=2), dict(resident=0, ring=2, load_pinned=False, pin=False)):
        with H3Engine.from_h3t(path, "cuda", **kw) as eng:
            assert eng.model is not None and eng.linear_backend() == "hip"
            outs.append(eng.velocity(x, 0.6, text.to(DEV)))
            if kw.get("resident") == 0 and kw.get("load_pinned") is None:
                steps = 2
                xv, xa = eng.sample((2, 4, 6), 4, text, steps=steps, seed=3)
                assert torch.isfinite(xv).all() and torch.isfinite(xa).all()
                g = torch.Generator("cpu").manual_seed(3)
                v = torch.randn(1, 24, 2, 4, 6, generator=g).to(DEV)
                a = torch.randn(1, 32, 2, 4, generator=g).to(DEV)
                refined = eng.encode_text(text.to(DEV, torch.bfloat16))
                sv = h3_sigmas(steps, CFG4.sigma_shift_video)
                sa = time_shift_sigma(sv, CFG4.sigma_shift_video, CFG4.sigma_shift_audio)
                for i in range(steps):
                    dv, da = eng.velocity([v.bfloat16(), a.bfloat16()], sv[i], None, sample_sigmas=sv, refined_text=refined)
                    v, a = v + dv.float() * float(sv[i + 1] - sv[i]), a + da.float() * float(sa[i + 1] - sa[i])
                assert torch.equal(xv, v) and torch.equal(xa, a)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o[0], outs[0][0]) and torch.equal(o[1], outs[0][1])


def test_comfy_dit_streams_parks_and_shrinks_on_the_gpu(tmp_path):
    """The host-application stand-in over a W4A8 .h3t: one resident block and the rest streamed through the ring give
    the all-resident velocity bit for bit, before and after parking (no device memory) and shrinking."""
    from h3turbo_amd.comfy_dit import H3TurboDiT, TorchMemoryHost
    from h3turbo_amd.h3t import write_h3t

    sd, _ = w4a8_case(50)
    path = tmp_path / "w4.h3t"
    write_h3t(path, CFG4, sd)
    video, audio, text = mc.inputs(CFG4, 51)
    x = [video.bfloat16().to(DEV), audio.bfloat16().to(DEV)]
    ts = torch.tensor([620.0], device=DEV)
    full = H3TurboDiT(str(path), host=TorchMemoryHost(DEV))
    part = H3TurboDiT(str(path), resident_blocks=1, host=TorchMemoryHost(DEV))
    try:
        refined = full.preprocess_text_embeds(text.to(DEV))
        want = full.forward(x, ts, refined)
        assert full.engine.provider.stats()["resident"] == CFG4.layers
        got = part.forward(x, ts, part.preprocess_text_embeds(text.to(DEV)))
        st = part.engine.provider.stats()
        assert st["resident"] == 1 and st["streamed"] == CFG4.layers - 1
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        blk = part.store.block_nbytes
        assert part.unload() > 0 and part.engine.provider.device_bytes() == 0
        again = part.forward(x, ts, refined)
        assert torch.equal(again[0], want[0])
        assert part.shrink(blk) >= blk
        assert torch.equal(part.forward(x, ts, refined)[0], want[0])
        torch.cuda.synchronize()
    finally:
        part.close()
        full.close()
