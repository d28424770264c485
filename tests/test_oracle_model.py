"""Pinning of the CPU model oracle (oracle/model_ref.py): the reference-order forward against the float64
definition, and the definition's sensitivity to the mistakes a restatement could make."""
import pytest
import torch

import model_cases as mc
from oracle import model_ref as mr

CFG = mc.CFG


def test_reference_order_in_fp32_equals_the_definition():
    sd = mc.make_sd(CFG, 3)
    video, audio, text = mc.inputs(CFG, 2)
    plan = mc.plan_data(CFG, text.shape[1], video, audio, 0.7)
    got = mr.model_ref(sd, CFG, video, audio, text, plan, dtype=torch.float32)
    want = mr.model_naive(sd, CFG, video, audio, text, plan)
    assert got[0].shape == video.shape and got[1].shape == audio.shape
    assert mc.rel(got[0], want[0]) < 5e-6 and mc.rel(got[1], want[1]) < 5e-6
    assert want[0].abs().max() > 0.05 and want[1].abs().max() > 0.05  # not vacuous


def test_reference_order_with_conditioning_rows_equals_the_definition():
    sd = mc.make_sd(CFG, 4)
    video, audio, text = mc.inputs(CFG, 5)
    g = torch.Generator().manual_seed(6)
    kv, ka = torch.randn(1, 24, 1, 4, 6, generator=g), torch.randn(1, 32, 2, 3, generator=g)
    kfs = [{"resolved_frame_index": 4, "latent": kv, "audio_latent": ka}]
    plan = mc.plan_data(CFG, text.shape[1], video, audio, 0.55, keyframes=kfs)
    cv, ca = mr.patchify(kv), mr.pack(ka)
    got = mr.model_ref(sd, CFG, video, audio, text, plan, dtype=torch.float32, cond_video_rows=cv, cond_audio_rows=ca)
    want = mr.model_naive(sd, CFG, video, audio, text, plan, cond_video_rows=cv, cond_audio_rows=ca)
    assert mc.rel(got[0], want[0]) < 5e-6 and mc.rel(got[1], want[1]) < 5e-6
    plain = mr.model_naive(sd, CFG, video, audio, text, mc.plan_data(CFG, text.shape[1], video, audio, 0.55))
    assert mc.rel(want[0], plain[0]) > 1e-3  # the conditioning rows reach the target tokens


def test_definition_catches_plausible_mistakes():
    """Each variant is a mistake a restatement could make in the plan or the input handling; the definition
    must tell it apart from the right forward, so the equality above pins those parts of model_ref."""
    sd = mc.make_sd(CFG, 7)
    video, audio, text = mc.inputs(CFG, 8)
    plan = mc.plan_data(CFG, text.shape[1], video, audio, 0.6)
    base = mr.model_naive(sd, CFG, video, audio, text, plan)

    def variant(**changes):
        return mr.model_naive(sd, CFG, video, audio, text, {**plan, **changes})

    shifted_tags = [(a, b, r + 1 if r % 3 == 0 else r - 1) for a, b, r in plan["mod_segments"]]  # video <-> text tag
    no_rope = torch.zeros_like(plan["position_ids"])
    wrong_t = [min(1.0, t + 0.05) for t in plan["t_values"]]
    wrong_head_row = (plan["video_seg"][0], plan["video_seg"][1], (plan["video_seg"][2] + 1) % len(plan["t_values"]))
    audio_swapped = mr.model_naive(sd, CFG, video, audio.flip(2), text, plan)
    mistakes = {"tags": variant(mod_segments=shifted_tags), "rope": variant(position_ids=no_rope),
                "t": variant(t_values=wrong_t), "head_row": variant(video_seg=wrong_head_row),
                "audio_channels": audio_swapped}
    for name, out in mistakes.items():
        assert max(mc.rel(out[0], base[0]), mc.rel(out[1], base[1])) > 1e-3, name


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_bf16_reference_order_stays_close_to_the_definition(dtype):
    sd = mc.make_sd(CFG, 9)
    video, audio, text = mc.inputs(CFG, 10)
    plan = mc.plan_data(CFG, text.shape[1], video, audio, 0.5)
    got = mr.model_ref(sd, CFG, video.to(dtype), audio.to(dtype), text.to(dtype), plan, dtype=dtype)
    want = mr.model_naive(sd, CFG, video, audio, text, plan)
    assert got[0].dtype == dtype
    assert mc.rel(got[0], want[0]) < 5e-2 and mc.rel(got[1], want[1]) < 5e-2


def test_w4a8_reference_order_is_the_dense_forward_within_quantisation_noise():
    """Every block linear W4A8 (fp8 group-16 scales, rotation 256): fp32 compute isolates the int8 activation
    quantisation of the 12 linears."""
    cfg = mc.W4CFG
    sd0 = mc.make_sd(cfg, 11)
    prefixes = [f"blocks.{i}" for i in range(cfg.layers)] + ["token_refiner.blocks.0"]
    sd, lin = mc.with_w4a8(cfg, sd0, 12, prefixes)
    video, audio, text = mc.inputs(cfg, 13)
    plan = mc.plan_data(cfg, text.shape[1], video, audio, 0.6)
    got = mr.model_ref(sd, cfg, video, audio, text, plan, dtype=torch.float32, linears=lin)
    want = mr.model_naive(mc.dense_equivalent(sd, lin), cfg, video, audio, text, plan)
    r = max(mc.rel(got[0], want[0]), mc.rel(got[1], want[1]))
    assert 1e-4 < r < 5e-2, r
