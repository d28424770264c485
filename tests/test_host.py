"""Host-side logic without a GPU: the C-ABI library loads and exports every declared entry point, argument
validation mirrors the reference's messages, and W4A8 compute on CPU tensors fails loudly (no CPU fallback)."""
import os
import re

import pytest
import torch

from h3turbo_amd import _lib
from h3turbo_amd import qlinear as ql
from h3turbo_amd.types import W4A8Weight

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "h3k.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(h3k_\w+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.h3k_version() == _lib.ABI_VERSION


def test_c_abi_rejects_bad_arguments_without_touching_a_device():
    lib = _lib.load()
    # rotation block not a power of 2 (128 and the other powers of 2 are accepted: an extension of the reference)
    assert lib.h3k_rotate_quant(None, _lib.BF16, 4, 384, 384, 48, 0, None, 384, None, None) == _lib.EINVAL
    assert "power of 2" in lib.h3k_last_error().decode()
    assert lib.h3k_rotate_quant(None, _lib.BF16, 0, 384, 384, 128, 0, None, 384, None, None) == 0  # no rows: no-op
    assert lib.h3k_rotate_quant(None, _lib.BF16, 4, 384, 384, 2048, 0, None, 384, None, None) == _lib.EINVAL
    # k not a multiple of the block
    assert lib.h3k_rotate_quant(None, _lib.BF16, 4, 250, 250, 256, 0, None, 250, None, None) == _lib.EINVAL
    assert "multiple" in lib.h3k_last_error().decode()
    # bad group size
    assert lib.h3k_decode_w4(None, 64, None, _lib.FP8E4M3, 4, None, 4, 128, 12, None, 128, None) == _lib.EINVAL
    assert "group_size" in lib.h3k_last_error().decode()
    # GEMM k not a multiple of 16
    assert lib.h3k_gemm_a8w8(None, 40, None, None, 40, None, None, 4, 4, 40, 0, None, _lib.BF16, 4, None, None) == _lib.EINVAL
    # workspace too small
    assert lib.h3k_w4a8_linear(None, 0, 4, 256, 256, None, 128, None, 3, 16, None, None, 8, 16, 256, None, 0, None, 0, 8,
                               None, 0, None) == _lib.ESPACE
    # int8 activations + scales + the weight region: the decoded grid with n rounded up to 256 rows (the packed
    # layout's padding), or, for calls of at most 32 rows, the few-row GEMM's accumulators if larger
    assert lib.h3k_w4a8_linear_workspace(4, 8, 256) == 1024 + 256 + 256 * 256
    assert lib.h3k_w4a8_linear_workspace(600, 13824, 5120) == 600 * 5120 + 2560 + 13824 * 5120
    # past the fused few-row GEMM's 32 rows no split-K accumulators are reserved: activations + scales + grid only
    assert lib.h3k_w4a8_linear_workspace(4096, 13824, 5120) == 4096 * 5120 + 4096 * 4 + 13824 * 5120
    # where the packed GEMM takes its split tail, the partial sums on top; the required part still fits the no-alloc
    # entry's scratch
    split = lib.h3k_gemm_packed_split_bytes(4096, 5120, 13824)
    assert split == 64 * 3 * 256 * 256 * 4  # one round + 64 tiles, cut in 3 along K
    base = 4096 * 13824 + 4096 * 4 + 5120 * 13824
    assert lib.h3k_w4a8_linear_workspace(4096, 5120, 13824) == base + split and base <= 128 << 20
    assert lib.h3k_gemm_packed_split_bytes(32768, 13824, 5120) == 0  # whole rounds only
    # the packed grid's size and the shapes its GEMM serves
    assert lib.h3k_w8_packed_bytes(33, 128) == 256 * 128 and lib.h3k_w8_packed_bytes(32, 100) == -1
    assert lib.h3k_gemm_packed_serves(32768, 13824, 5120) == 1 and lib.h3k_gemm_packed_serves(512, 13824, 5120) == 0
    assert lib.h3k_gemm_a8w8_packed(None, 5120, None, None, None, None, 512, 13824, 5120, 0, None, _lib.BF16, 13824, None,
                                    None) == _lib.EINVAL
    # empty work is a no-op
    assert lib.h3k_rotate_quant(None, _lib.BF16, 0, 256, 256, 256, 0, None, 256, None, None) == 0
    # split norm + rope: head_dim outside {32, 64, 128, 256}; overlapping head-major outputs
    assert lib.h3k_qkv_split_norm_rope(None, 288, 4, 2, 48, None, None, None, None, 24, 24, 1e-5, None, None, None, 192,
                                       None) == _lib.EINVAL
    assert "head_dim" in lib.h3k_last_error().decode()
    assert lib.h3k_qkv_split_norm_rope(None, 768, 4, 2, 128, None, None, None, None, 48, 48, 1e-5, None, None, None, 256,
                                       None) == _lib.EINVAL
    assert "head_stride" in lib.h3k_last_error().decode()
    # head-major rotate+quant: only rotation 256 on 16-bit activations; head_dim a power of two
    assert lib.h3k_rotate_quant_heads(None, _lib.BF16, 4, 512, 128, 128, 512, 64, 0, None, 512, None, None) == _lib.EINVAL
    assert "rotation 256" in lib.h3k_last_error().decode()
    assert lib.h3k_rotate_quant_heads(None, _lib.BF16, 4, 480, 96, 96, 384, 256, 0, None, 480, None, None) == _lib.EINVAL
    assert "power of two" in lib.h3k_last_error().decode()
    # fused RMSNorm + modulation: k a multiple of 8 up to 8192
    assert lib.h3k_rms_modulate(None, 100, 4, 100, None, None, None, 100, None, 1e-5, None, 100, 0, None) == _lib.EINVAL
    assert "multiple of 8" in lib.h3k_last_error().decode()
    # the weight / shift / scale vectors: bf16 or fp32 only
    assert lib.h3k_rms_modulate(None, 5120, 4, 5120, None, None, None, 5120, None, 1e-5, None, 5120, _lib.F16,
                                None) == _lib.EINVAL
    assert "bf16 or f32" in lib.h3k_last_error().decode()
    assert lib.h3k_rms_modulate(None, 5120, 0, 5120, None, None, None, 5120, None, 1e-5, None, 5120, 0, None) == 0
    # fused few-row W4A8 GEMM: at most 128 rows, k a multiple of 64, group 16 / 32 / multiple of 64
    w4 = lambda m, k, group: lib.h3k_gemm_w4a8(None, k, None, None, k // 2, None, _lib.FP8E4M3, max(1, k // group),  # noqa: E731
                                               None, group, None, None, m, 64, k, 0, None, _lib.BF16, 64, None, None,
                                               None)
    assert w4(129, 512, 16) == _lib.EINVAL and "rows" in lib.h3k_last_error().decode()
    assert w4(8, 544, 32) == _lib.EINVAL and "multiple of 64" in lib.h3k_last_error().decode()
    assert w4(8, 512, 8) == _lib.EINVAL and "group_size" in lib.h3k_last_error().decode()
    assert w4(0, 512, 16) == 0
    assert lib.h3k_gemm_w4a8_workspace(64, 256, 5120) == 64 * 256 * 4  # split K: int32 accumulators
    assert lib.h3k_gemm_w4a8_workspace(64, 256, 256) == 0
    # activation-fused rotate+quant: 16-bit input, act 1 or 2, rotation 256, the full input width per row
    act = lambda dt, k, ldx, a, rot=256: lib.h3k_rotate_quant_act(None, dt, 4, k, ldx, a, rot, 0, None, k, None,  # noqa: E731
                                                                  None)
    assert act(_lib.F32, 256, 256, 2) == _lib.EINVAL and "bf16 or f16" in lib.h3k_last_error().decode()
    assert act(_lib.BF16, 256, 256, 3) == _lib.EINVAL and "act" in lib.h3k_last_error().decode()
    assert act(_lib.BF16, 256, 256, 2, rot=64) == _lib.EINVAL and "rotation 256" in lib.h3k_last_error().decode()
    assert act(_lib.BF16, 256, 256, 1) == _lib.EINVAL and "ldx" in lib.h3k_last_error().decode()
    assert act(_lib.BF16, 256 * 129, 256 * 129, 2) == _lib.EINVAL and "too long" in lib.h3k_last_error().decode()
    assert lib.h3k_rotate_quant_act(None, _lib.F16, 0, 512, 1024, 1, 256, 1, None, 512, None, None) == 0


def make_weight(n=40, k=512, group=16):
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8)
    s = (torch.rand(n, k // group, generator=g) * 180 + 20).to(torch.float8_e4m3fn)
    return W4A8Weight(q, s, torch.rand(n, generator=g) * 0.02 + 0.005, torch.linspace(-1, 1, 16), group_size=group, convrot=256)


@pytest.mark.parametrize("bad", [0, 1, 2, 3, 8, 12, 32, 100, 128, 512, -4])
def test_hadamard_rejects_non_powers_of_four(bad):
    with pytest.raises(ValueError, match="power of 4"):
        ql.hadamard_regular(bad)


@pytest.mark.parametrize("size", [4, 16, 64, 256, 1024])
def test_hadamard_symmetric_involutory_cached(size):
    h = ql.hadamard_regular(size, "cpu", torch.float32)
    assert torch.equal(h, h.T) and torch.equal(h @ h, torch.eye(size))
    assert ql.hadamard_regular(size, "cpu", torch.float32) is h
    assert torch.equal(ql.hadamard_regular(size, "cpu", torch.bfloat16).float(), h)


def test_validation_messages_match_the_reference():
    w = make_weight()
    x = torch.randn(3, 512)
    for kw, msg in (({"backend": "cuda"}, "backend"), ({"precision": "a4"}, "precision"), ({"quant_mode": "x"}, "quant_mode"),
                    ({"input_act": "gelu"}, "input_act"), ({"chunk_tokens": 0}, "chunk_tokens")):
        with pytest.raises(ValueError, match=msg):
            ql.linear(x, w, **kw)
    with pytest.raises(ValueError, match="do not match"):
        ql.linear(torch.zeros(2, 256), w)
    with pytest.raises(ValueError, match="floating"):
        ql.linear(torch.zeros(2, 512, dtype=torch.int8), w)
    with pytest.raises(ValueError, match="even"):
        ql.linear(torch.zeros(2, 5), w, input_act="swiglu")
    with pytest.raises(ValueError, match="do not match"):
        ql.linear(torch.zeros(2, 512), w, input_act="swiglu")
    with pytest.raises(ValueError, match="bias"):
        ql.linear(x, w, torch.zeros(39))
    bad = [(W4A8Weight(w.q, w.s_rel[:, :-1], w.s_ch, w.codebook), "s_rel"), (W4A8Weight(w.q, w.s_rel, w.s_ch[:-1], w.codebook), "s_ch"),
           (W4A8Weight(w.q, w.s_rel, w.s_ch, w.codebook[:8]), "codebook"), (W4A8Weight(w.q.float(), w.s_rel, w.s_ch, w.codebook), "int8"),
           (W4A8Weight(torch.zeros(2, 100, dtype=torch.int8), torch.zeros(2, 12).to(torch.float8_e4m3fn), torch.ones(2), w.codebook), "divisible")]
    for weight, msg in bad:
        with pytest.raises(ValueError, match=msg):
            ql.decode_int8_grid(weight)
    with pytest.raises(ValueError, match="multiple"):
        ql.rotate(torch.zeros(3, 250))
    with pytest.raises(ValueError, match="multiple"):
        ql.quantize_activation(torch.zeros(2, 100))
    with pytest.raises(ValueError, match="floating"):
        ql.rotate(torch.zeros(3, 256, dtype=torch.int8))
    with pytest.raises(ValueError, match="contiguous"):
        ql.dequantize(w, rows=slice(0, 10, 2))


def test_backend_resolution():
    w = make_weight()
    x = torch.randn(3, 512)
    info = ql.available_backends()
    assert set(info) == {"hip", "ck", "torch"}
    assert not info["ck"]["available"] and info["ck"]["reason"]
    assert ql.resolve_backend(x, w) == "hip" and ql.resolve_backend(x, w, "hip", "a16") == "hip"
    assert ql.resolve_backend(x, torch.zeros(4, 512)) == "dense"
    for b in ("ck", "torch"):
        with pytest.raises(RuntimeError, match=b):
            ql.linear(x, w, backend=b)


def test_cpu_tensors_fail_loudly_instead_of_falling_back():
    w = make_weight()
    x = torch.randn(3, 512)
    for fn in (lambda: ql.linear(x, w), lambda: ql.quantize_activation(x), lambda: ql.rotate(x), lambda: ql.decode_int8_grid(w)):
        with pytest.raises(RuntimeError, match="GPU"):
            fn()
    # empty inputs need no device work
    assert ql.linear(torch.zeros(0, 512), w).shape == (0, 40)
    assert ql.linear(torch.zeros(2, 0, 512), w).shape == (2, 0, 40)
    assert ql.rotate(torch.zeros(0, 256)).shape == (0, 256)


def test_dense_weight_path_is_plain_f_linear():
    g = torch.Generator().manual_seed(26)
    x, w, b = torch.randn(6, 48, generator=g), torch.randn(10, 48, generator=g), torch.randn(10, generator=g)
    assert torch.equal(ql.linear(x, w), torch.nn.functional.linear(x, w))
    assert torch.equal(ql.linear(x, w, b), torch.nn.functional.linear(x, w, b))
    # chunked rows go through BLAS with another row count: equal up to the BLAS's blocking
    assert torch.allclose(ql.linear(x, w, chunk_tokens=4), torch.nn.functional.linear(x, w), rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError, match="do not match"):
        ql.linear(x, w[:, :40])


def test_rope_table_widening_is_cached_per_table_pair_and_invalidated():
    """qkv_split_norm_rope widens the rope tables to fp32 once per pair (every block of a forward passes the same
    two tensors); an in-place change or another pair recomputes them."""
    from h3turbo_amd import block as bk

    cos, sin = torch.randn(7, 4).bfloat16(), torch.randn(7, 4).bfloat16()
    a = bk._rope_f32(cos, sin)
    assert bk._rope_f32(cos, sin)[0] is a[0]
    assert torch.equal(a[0], cos.float()) and torch.equal(a[1], sin.float())
    cos.mul_(3)
    b = bk._rope_f32(cos, sin)
    assert b[0] is not a[0] and torch.equal(b[0], cos.float())
    other = bk._rope_f32(cos.clone(), sin)
    assert other[0] is not b[0] and torch.equal(other[0], cos.float())
    with torch.inference_mode():  # no version counter: widened every time, never cached
        ci, si = cos.clone(), sin.clone()
        first = bk._rope_f32(ci, si)
        ci.mul_(2)
        assert torch.equal(bk._rope_f32(ci, si)[0], ci.float()) and not torch.equal(first[0], ci.float())
