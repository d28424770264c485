"""The whole-model forward's host logic (h3turbo_amd.model) on the CPU with dense fp32 weights: the float64
definition (oracle/model_ref.py), chunk exactness, the provider protocol, payloads and masks, the audio carry,
padding, text paths, the head bank, weight loading and option validation (after the reference's
tests/test_h3_model.py).  W4A8 layers run on the GPU only: their numerics are in tests/test_gpu_model.py."""
import dataclasses

import pytest
import torch

import model_cases as mc
from h3turbo_amd import block as bk
from h3turbo_amd import layout as L
from h3turbo_amd import model as model_mod
from h3turbo_amd.block import ResidentProvider
from h3turbo_amd.model import H3Model, weights_from_state_dict
from h3turbo_amd.types import W4A8Weight
from oracle import model_ref as mr

CFG = mc.CFG
T, H, W, TA, NT = 2, 4, 6, 4, 5


def make_model(cfg=CFG, sd=None, dtype=torch.float32, provider=None, **kw) -> H3Model:
    glob, blocks = weights_from_state_dict(sd or mc.make_sd(cfg), cfg, "cpu", dtype)
    return H3Model(cfg, glob, provider(blocks) if provider else ResidentProvider(blocks), device="cpu", dtype=dtype, **kw)


def inputs(seed=1, **kw):
    v, a, t = mc.inputs(CFG, seed, **kw)
    return [v, a], t


def test_forward_equals_the_definition_and_is_deterministic():
    sd = mc.make_sd(CFG, 3)
    m = make_model(CFG, sd)
    x, text = inputs(2)
    out = m.forward(x, 0.7, text)
    want = mr.model_naive(sd, CFG, x[0], x[1], text, mc.plan_data(CFG, NT, x[0], x[1], 0.7))
    assert out[0].shape == x[0].shape and out[1].shape == x[1].shape
    assert mc.rel(out[0], want[0]) < 5e-6 and mc.rel(out[1], want[1]) < 5e-6
    again = m.forward(x, 0.7, text)
    assert torch.equal(out[0], again[0]) and torch.equal(out[1], again[1])


def test_forward_depends_on_every_input():
    m = make_model()
    x, text = inputs(2)
    base = m.forward(x, 0.7, text)
    assert mc.rel(m.forward(x, 0.71, text)[0], base[0]) > 1e-4
    assert mc.rel(m.forward(x, 0.7, text + 0.1)[0], base[0]) > 1e-4
    assert mc.rel(m.forward([x[0], x[1] + 0.1], 0.7, text)[0], base[0]) > 1e-5  # joint attention: audio reaches video


def test_chunking_and_rope_impl_leave_results_unchanged():
    sd = mc.make_sd(CFG, 4)
    x, text = inputs(5)
    base = make_model(CFG, sd).forward(x, 0.6, text)
    for kw in ({"mlp_chunk": 3}, {"attn_chunk": 7}, {"rope_chunk": 4}, {"mlp_chunk": 5, "attn_chunk": 11, "rope_chunk": 2},
               {"rope_impl": "eager"}):
        out = make_model(CFG, sd, **kw).forward(x, 0.6, text)
        assert mc.rel(out[0], base[0]) < 1e-6 and mc.rel(out[1], base[1]) < 1e-6, kw


def test_bf16_compute_stays_close_to_fp32():
    sd = mc.make_sd(CFG, 6)
    x, text = inputs(7)
    ref32 = make_model(CFG, sd).forward(x, 0.5, text)
    out = make_model(CFG, sd, dtype=torch.bfloat16).forward([t.bfloat16() for t in x], 0.5, text.bfloat16())
    assert out[0].dtype == torch.bfloat16 and out[1].dtype == torch.bfloat16
    assert mc.rel(out[0].float(), ref32[0]) < 5e-2 and mc.rel(out[1].float(), ref32[1]) < 5e-2


class Recorder(ResidentProvider):
    def __init__(self, blocks, fail_at=None):
        super().__init__(blocks)
        self.log, self.fail_at = [], fail_at

    def begin_forward(self):
        self.log.append("begin")

    def acquire(self, i):
        self.log.append(f"acquire{i}")
        if i == self.fail_at:
            raise RuntimeError("copy failed")
        return super().acquire(i)

    def release(self, i):
        self.log.append(f"release{i}")

    def end_forward(self):
        self.log.append("end")


def test_provider_protocol_order_and_cleanup_after_an_abort():
    sd = mc.make_sd(CFG, 8)
    x, text = inputs(9)
    glob, blocks = weights_from_state_dict(sd, CFG, "cpu", torch.float32)
    rec = Recorder(blocks)
    m = H3Model(CFG, glob, rec, device="cpu", dtype=torch.float32)
    m.forward(x, 0.5, text)
    m.forward(x, 0.4, text)
    one = ["begin", "acquire0", "release0", "acquire1", "release1", "end"]
    assert rec.log == one + one
    bad = Recorder(blocks, fail_at=1)
    mb = H3Model(CFG, glob, bad, device="cpu", dtype=torch.float32)
    with pytest.raises(RuntimeError, match="copy failed"):
        mb.forward(x, 0.5, text)
    assert bad.log == ["begin", "acquire0", "release0", "acquire1", "end"]
    bad.fail_at = None
    assert mc.rel(mb.forward(x, 0.5, text)[0], make_model(CFG, sd).forward(x, 0.5, text)[0]) < 1e-6


def _payload(g):
    kfs = [{"resolved_frame_index": 0, "latent": torch.randn(1, 24, 1, H, W, generator=g),
            "audio_latent": torch.randn(1, 32, 2, 3, generator=g)},
           {"resolved_frame_index": 9, "latent": torch.randn(1, 24, 2, H, W, generator=g)}]
    refs = [{"kind": "image", "latent_h": 4, "latent_w": 2, "latent": torch.randn(1, 24, 1, 4, 2, generator=g)},
            {"kind": "video_audio", "latent_t": 2, "latent_h": 2, "latent_w": 4, "ref_audio_t": 3,
             "latent": torch.randn(1, 24, 2, 2, 4, generator=g), "audio_latent": torch.randn(1, 32, 2, 3, generator=g)},
            {"kind": "audio", "ref_audio_t": 4, "audio_latent": torch.randn(1, 32, 2, 4, generator=g)}]
    return {"keyframes": kfs, "refs": refs, "seed": 5,
            "cond_video_latents": [kfs[0]["latent"], kfs[1]["latent"], refs[0]["latent"], refs[1]["latent"]],
            "cond_audio_latents": [kfs[0]["audio_latent"], refs[1]["audio_latent"], refs[2]["audio_latent"]],
            "text_token_tags": torch.tensor([[1, 1, 0, 0, 2]])}


def test_conditioning_payloads_and_denoise_masks():
    m = make_model()
    x, text = inputs(3)
    payload = _payload(torch.Generator().manual_seed(4))
    out = m.forward(x, 0.6, text, payload=payload)
    assert torch.isfinite(out[0]).all() and torch.isfinite(out[1]).all()
    assert mc.rel(out[0], m.forward(x, 0.6, text)[0]) > 1e-4
    assert mc.rel(m.forward(x, 0.6, text, payload={**payload, "seed": 6})[0], out[0]) > 1e-6  # aug < 1 mixes noise
    p1 = {**payload, "visual_cond_noise_aug": 1.0, "audio_cond_noise_aug": 1.0}
    assert torch.equal(m.forward(x, 0.6, text, payload={**p1, "seed": 1})[0], m.forward(x, 0.6, text, payload={**p1, "seed": 2})[0])
    kfs, refs = payload["keyframes"], payload["refs"]
    good = L.PackedLayout.build(NT, T, H, W, TA, kfs, refs)
    assert torch.equal(m.forward(x, 0.6, text, payload={**payload, "layout": good})[0], out[0])
    stale = L.PackedLayout.build(NT + 1, T, H, W, TA)
    assert torch.equal(m.forward(x, 0.6, text, payload={**payload, "layout": stale})[0], out[0])
    dm = torch.ones(1, 1, T, H, W)
    dm[:, :, 0] = 0.0
    adm = torch.ones(1, 1, 2, TA)
    adm[..., :1] = 0.0
    mv, ma = m.forward(x, 0.6, text, denoise_mask=dm, audio_denoise_mask=adm)
    assert not mv[:, :, 0].any() and not ma[..., 0].any() and mv[:, :, 1:].abs().sum() > 0


def test_conditioning_rows_equal_the_definition_when_not_noised():
    sd = mc.make_sd(CFG, 21)
    m = make_model(CFG, sd)
    x, text = inputs(22)
    g = torch.Generator().manual_seed(23)
    kv, ka = torch.randn(1, 24, 1, H, W, generator=g), torch.randn(1, 32, 2, 3, generator=g)
    kfs = [{"resolved_frame_index": 4, "latent": kv, "audio_latent": ka}]
    payload = {"keyframes": kfs, "cond_video_latents": [kv], "cond_audio_latents": [ka],
               "visual_cond_noise_aug": 1.0, "audio_cond_noise_aug": 1.0}
    out = m.forward(x, 0.55, text, payload=payload)
    plan = mc.plan_data(CFG, NT, x[0], x[1], 0.55, keyframes=kfs, visual_aug=1.0, audio_aug=1.0)
    want = mr.model_naive(sd, CFG, x[0], x[1], text, plan, cond_video_rows=mr.patchify(kv), cond_audio_rows=mr.pack(ka))
    assert mc.rel(out[0], want[0]) < 5e-6 and mc.rel(out[1], want[1]) < 5e-6


def test_audio_scale_carry_is_undone_and_redone():
    m = make_model()
    x, text = inputs(3)
    sigma, scale = torch.tensor(0.5, dtype=torch.float32), 1.25
    sa = L.time_shift_sigma(sigma, 12.0, 3.0)
    carry = sa / sigma
    inner = m.forward([x[0], x[1] * carry], 0.5, text)
    out = m.forward(x, 0.5, text, payload={"audio_scale": scale})
    assert mc.rel(out[0], inner[0]) < 1e-6
    assert mc.rel(out[1], (1.0 - scale) * (x[1] * carry) + (1.0 + (scale - 1.0) * sa) * inner[1]) < 1e-6


def test_odd_latent_sizes_are_padded_circularly_then_cropped():
    m = make_model()
    x, text = inputs(3, t=2, h=3, w=5)
    out = m.forward(x, 0.5, text)
    assert out[0].shape == x[0].shape
    full = m.forward([L.pad_to_patch(x[0]), x[1]], 0.5, text)
    assert torch.equal(out[0], full[0][:, :, :, :3, :5]) and torch.equal(out[1], full[1])


def test_text_paths_and_input_validation():
    m = make_model()
    x, text = inputs(3)
    refined = m.encode_text(text)
    assert refined.shape == (1, NT, CFG.hidden) and torch.equal(m.encode_text(refined), refined)
    a, b, c = m.forward(x, 0.5, text), m.forward(x, 0.5, None, refined_text=refined), m.forward(x, 0.5, refined)
    assert torch.equal(a[0], b[0]) and torch.equal(a[0], c[0])
    bad = [
        lambda: m.forward(x, 0.5, None),
        lambda: m.forward(x, float("nan"), text),
        lambda: m.forward([x[0].repeat(2, 1, 1, 1, 1), x[1]], 0.5, text),
        lambda: m.forward([x[0], x[1][:, :, :1]], 0.5, text),
        lambda: m.forward(x[:1], 0.5, text),
        lambda: m.encode_text(torch.randn(1, NT, 11)),
        lambda: m.encode_text(torch.randn(2, NT, CFG.text_dim)),
        lambda: m.forward(x, 0.5, text, denoise_mask=torch.ones(1, 1, T, H, W + 2)),
        lambda: m.forward(x, 0.5, text, audio_denoise_mask=torch.ones(1, 1, 2, TA + 1)),
        lambda: m.forward(x, 0.5, text, payload={"text_token_tags": torch.tensor([[1, 0]])}),
        lambda: m.forward(x, 0.5, text, payload={"cond_video_latents": [torch.randn(1, 24, 1, H, W)]}),
        lambda: m.forward(x, 0.5, text, payload={"keyframes": [{"resolved_frame_index": 0, "latent": torch.randn(1, 24, 1, H, W)}]}),
    ]
    for i, f in enumerate(bad):
        with pytest.raises(ValueError):
            f()


def test_head_bank_needs_the_schedule_and_reduces_to_one_head():
    sd1 = mc.make_sd(CFG, 11)
    sd3 = dict(sd1)
    for name in ("video_out", "audio_out"):
        w, b = sd1[f"final_layer.{name}.weight"], sd1[f"final_layer.{name}.bias"]
        sd3[f"final_layer.{name}.weight"] = torch.cat([w, torch.zeros_like(w), torch.zeros_like(w)])
        sd3[f"final_layer.{name}.bias"] = torch.cat([b, torch.zeros_like(b), torch.zeros_like(b)])
    m1, m3 = make_model(CFG, sd1), make_model(CFG, sd3)
    assert m3.head_bank == 3 and m1.head_bank == 1
    x, text = inputs(3)
    with pytest.raises(ValueError):
        m3.forward(x, 0.6, text)
    sched = torch.tensor([1.0, 0.8, 0.6, 0.3, 0.0])
    for s in (0.8, 0.6, 0.3):
        a, b = m3.forward(x, s, text, sample_sigmas=sched), m1.forward(x, s, text)
        assert mc.rel(a[0], b[0]) < 1e-6 and mc.rel(a[1], b[1]) < 1e-6


def test_head_bank_mixes_the_offset_heads():
    sd = mc.make_sd(CFG, 12, head_bank=3)
    m = make_model(CFG, sd)
    x, text = inputs(13)
    sched = torch.tensor([1.0, 0.8, 0.6, 0.3, 0.0])
    outs = [m.forward(x, s, text, sample_sigmas=sched)[0] for s in (1.0, 0.3)]
    assert mc.rel(outs[0], outs[1]) > 1e-3  # different sampler steps use different head mixtures
    start, stop = L.head_bank_range(sched, torch.tensor(0.3), 12.0, 3)
    sd1 = dict(sd)
    for name, shift in (("video_out", 12.0), ("audio_out", 3.0)):
        w, b = L.bank_head_weights(sd[f"final_layer.{name}.weight"], sd[f"final_layer.{name}.bias"], 3, start, stop, shift)
        sd1[f"final_layer.{name}.weight"], sd1[f"final_layer.{name}.bias"] = w, b
    single = make_model(CFG, sd1).forward(x, 0.3, text)[0]
    assert mc.rel(outs[1], single) < 1e-6


def test_unsupported_configurations_fail_loudly():
    sd = mc.make_sd(CFG)
    glob, blocks = weights_from_state_dict(sd, CFG, "cpu", torch.float32)
    glob.adaln_t_table = None
    with pytest.raises(NotImplementedError):
        H3Model(CFG, glob, ResidentProvider(blocks), device="cpu", dtype=torch.float32)
    glob, blocks = weights_from_state_dict(sd, CFG, "cpu", torch.float32)
    with pytest.raises(ValueError):
        H3Model(CFG, glob, ResidentProvider(blocks), device="cpu", dtype=torch.float16)
    with pytest.raises(ValueError):
        H3Model(dataclasses.replace(CFG, rope_inv_freq_len=6), glob, ResidentProvider(blocks), device="cpu",
                dtype=torch.float32)
    with pytest.raises(RuntimeError):
        H3Model(CFG, glob, ResidentProvider(blocks), device="cpu", dtype=torch.float32, attn_impl="int8")


def test_w4a8_layers_load_and_refuse_to_run_off_the_gpu():
    cfg = mc.W4CFG
    sd, _ = mc.with_w4a8(cfg, mc.make_sd(cfg, 12), 13, ["blocks.0"])
    glob, blocks = weights_from_state_dict(sd, cfg, "cpu", torch.float32)
    assert all(isinstance(getattr(blocks[0], f), W4A8Weight) for f in ("qkv", "out", "fc1", "fc2"))
    assert blocks[0].qkv.convrot == 256 and blocks[0].qkv.group_size == 16
    assert blocks[0].qkv.s_rel.dtype == torch.float8_e4m3fn and isinstance(blocks[1].qkv, torch.Tensor)
    bad = dict(sd)
    bad["blocks.0.mlp.fc2.weight_s_rel"] = bad["blocks.0.mlp.fc2.weight_s_rel"][:, :-1]
    with pytest.raises(ValueError, match="W4A8"):
        weights_from_state_dict(bad, cfg, "cpu", torch.float32)
    m = H3Model(cfg, glob, ResidentProvider(blocks), device="cpu", dtype=torch.float32)
    v, a, t = mc.inputs(cfg, 14)
    with pytest.raises(RuntimeError, match="GPU"):  # no CPU fallback for the W4A8 path
        m.forward([v, a], 0.6, t)


def test_weights_from_state_dict_validation_and_prefix():
    sd = mc.make_sd(CFG)
    glob, blocks = weights_from_state_dict({"model.dm." + k: v for k, v in sd.items()}, CFG, "cpu", torch.bfloat16,
                                           prefix="model.dm.")
    assert len(blocks) == CFG.layers and len(glob.refiner) == CFG.refiner_layers
    assert blocks[0].qkv.dtype == torch.bfloat16 and glob.video_patch_w.dtype == torch.float32
    assert glob.final_norm.dtype == torch.bfloat16
    assert blocks[0].adaln_w.shape == (18 * CFG.hidden, CFG.t_dim) and glob.refiner[0].adaln_w is None
    broken = dict(sd)
    del broken["blocks.1.mlp.fc2.weight"], broken["rope.inv_freq"]
    with pytest.raises(KeyError, match="2 tensors"):
        weights_from_state_dict(broken, CFG, "cpu", torch.float32)
    wrong = dict(sd)
    wrong["blocks.0.attn.qkv_proj.weight"] = torch.zeros(5, 5)
    with pytest.raises(ValueError, match="expected"):
        weights_from_state_dict(wrong, CFG, "cpu", torch.float32)


def test_islands_round_through_the_compute_dtype_unless_asked_not_to():
    sd = mc.make_sd(CFG, 15)
    x, text = inputs(16)
    native = make_model(CFG, sd, dtype=torch.bfloat16)
    exact = make_model(CFG, sd, dtype=torch.bfloat16, fp32_islands=True)
    w = sd["video_patch_proj.weight"]
    assert torch.equal(native.vpw, w.bfloat16().float()) and torch.equal(exact.vpw, w)
    assert torch.equal(native.vob, sd["final_layer.video_out.bias"].bfloat16().float())
    xb = [t.bfloat16() for t in x]
    a, b = native.forward(xb, 0.6, text.bfloat16()), exact.forward(xb, 0.6, text.bfloat16())
    assert 1e-4 < mc.rel(a[0].float(), b[0].float()) < 5e-2
    f32 = make_model(CFG, sd)
    assert torch.equal(f32.vpw, w) and torch.equal(f32.final_adaln_b, sd["final_layer.adaln_proj.linear.bias"])


def test_row_chunking_of_projections_and_heads_is_exact(monkeypatch):
    sd = mc.make_sd(CFG, 17)
    x, text = inputs(18)
    dm = torch.ones(1, 1, T, H, W)
    dm[:, :, 0] = 0.0
    dm[:, :, 1, :2, :3] = 0.5  # per-token modulation rows
    adm = torch.ones(1, 1, 2, TA)
    adm[..., 1] = 0.3
    base = make_model(CFG, sd).forward(x, 0.6, text, denoise_mask=dm, audio_denoise_mask=adm)
    monkeypatch.setattr(model_mod, "_PROJ_ROWS", 3)
    monkeypatch.setattr(bk, "_GATHER_ROWS", 3)
    small = make_model(CFG, sd, mlp_chunk=2).forward(x, 0.6, text, denoise_mask=dm, audio_denoise_mask=adm)
    assert mc.rel(small[0], base[0]) < 1e-6 and mc.rel(small[1], base[1]) < 1e-6


def test_option_validation():
    for kw in ({"attn_backend": "flash"}, {"backend": "cuda"}, {"precision": "a4"}, {"attn_chunk": -1}, {"rope_chunk": 0},
               {"mlp_chunk": 0}, {"rope_impl": "magic"}):
        with pytest.raises(ValueError):
            make_model(**kw)


# ------------------------------------------------------------------------------------------------ engine
def _h3t(tmp_path, cfg, sd):
    from h3turbo_amd.h3t import write_h3t

    path = tmp_path / "tiny.h3t"
    write_h3t(path, cfg, sd)
    return str(path)


def test_engine_from_h3t_runs_the_whole_model_and_the_sampler(tmp_path):
    from h3turbo_amd.engine import H3Engine, h3_sigmas

    sd = mc.make_sd(CFG, 31)
    path = _h3t(tmp_path, CFG, sd)
    x, text = inputs(32)
    want = make_model(CFG, sd).forward(x, 0.7, text)
    with H3Engine.from_h3t(path, "cpu", resident=1, ring=2, pin=False, dtype=torch.float32) as eng:
        assert eng.model is not None and eng.cfg == CFG and eng.model.dtype == torch.float32
        got = eng.velocity(x, 0.7, text)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])  # streamed blocks, same numbers
        refined = eng.encode_text(text)
        steps, seen = 3, []
        xv, xa = eng.sample((T, H, W), TA, text, steps=steps, seed=4, callback=lambda i, v, a: seen.append(i))
        assert seen == list(range(steps)) and xv.shape == (1, 24, T, H, W) and xa.shape == (1, 32, 2, TA)
        # the same Euler loop by hand
        g = torch.Generator("cpu").manual_seed(4)
        v = torch.randn(1, 24, T, H, W, generator=g)
        a = torch.randn(1, 32, 2, TA, generator=g)
        sv = h3_sigmas(steps, CFG.sigma_shift_video)
        sa = L.time_shift_sigma(sv, CFG.sigma_shift_video, CFG.sigma_shift_audio)
        for i in range(steps):
            dv, da = eng.velocity([v, a], sv[i], None, sample_sigmas=sv, refined_text=refined)
            v, a = v + dv * float(sv[i + 1] - sv[i]), a + da * float(sa[i + 1] - sa[i])
        assert torch.equal(xv, v) and torch.equal(xa, a)


def test_sigma_schedule():
    from h3turbo_amd.engine import h3_sigmas

    s = h3_sigmas(4, 12.0)
    assert s.dtype == torch.float32 and s.shape == (5,) and s[0] == 1.0 and s[-1] == 0.0
    assert (s[1:] < s[:-1]).all()
    t = torch.linspace(1.0, 0.0, 5, dtype=torch.float64)
    assert torch.equal(s, (12.0 * t / (1.0 + 11.0 * t)).float())
    with pytest.raises(ValueError):
        h3_sigmas(0, 12.0)


def test_engine_without_globals_runs_blocks_only(tmp_path):
    from h3turbo_amd.engine import H3Engine

    sd = {k: v for k, v in mc.make_sd(CFG, 33).items() if k.startswith("blocks.")}
    path = _h3t(tmp_path, CFG, sd)
    with H3Engine.from_h3t(path, "cpu", resident=0, ring=2, pin=False) as eng:
        assert eng.model is None
        with pytest.raises(RuntimeError, match="no whole-model forward"):
            eng.velocity(*inputs(1))
    with pytest.raises(ValueError):
        H3Engine.from_h3t(path, "cpu", pin=False, whole_model=True)
