"""The .h3t container (h3turbo_amd.h3t) against the reference writer's own output and the reference's store tests
(tests/test_h3_store.py): byte-identical files, lossless tensors, alignment and contiguity, block views, the
reader's validation, the writer's checks and atomicity.  CPU only."""
import dataclasses
import json
import os
import struct

import numpy as np
import pytest
import torch

import h3t_inputs as hi
from h3turbo_amd import h3t
from h3turbo_amd.blockstore import HostBlockStore
from h3turbo_amd.config import H3Config
from h3turbo_amd.stream import StreamingProvider
from h3turbo_amd.types import W4A8Weight

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vectors", "h3t_tiny_quant.h3t")


def cfg(layers=2) -> H3Config:
    return dataclasses.replace(H3Config(**hi.TINY), layers=layers)


def raw(t: torch.Tensor) -> bytes:
    return t.detach().cpu().contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()


@pytest.fixture(scope="module")
def quant_sd():
    return hi.state_dict(quant=True, seed=0)


@pytest.fixture(scope="module")
def dense_sd():
    return hi.state_dict(quant=False, seed=2)


def write(tmp_path, sd, name="m.h3t", c=None, **kw):
    dst = str(tmp_path / name)
    rep = h3t.write_h3t(dst, c or cfg(), sd, **kw)
    return dst, rep


def test_writer_output_is_byte_identical_to_the_reference_writer(tmp_path, quant_sd):
    dst, rep = write(tmp_path, quant_sd, source_name="tiny", source_size=123)
    assert open(dst, "rb").read() == open(GOLDEN, "rb").read()
    assert rep["n_tensors"] == len(quant_sd) and rep["file_size"] == os.path.getsize(GOLDEN)


def test_reader_reads_the_reference_file_losslessly(quant_sd):
    with h3t.H3TFile(GOLDEN) as f:
        assert f.cfg == cfg() and f.n_blocks == 2 and f.source_name == "tiny" and f.source_size == 123
        assert f.quant == {"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": 16}
        assert set(f.keys()) == set(quant_sd)
        for name, want in quant_sd.items():
            t = f.tensor(name)
            assert (t.dtype, tuple(t.shape)) == (want.dtype, tuple(want.shape)), name
            assert raw(t) == raw(want), name


@pytest.mark.parametrize("quant", [True, False])
def test_safetensors_reads_our_files(tmp_path, quant, quant_sd, dense_sd):
    safe_open = pytest.importorskip("safetensors").safe_open
    sd = quant_sd if quant else dense_sd
    dst, _ = write(tmp_path, sd)
    with safe_open(dst, "pt") as f:
        assert {k for k in f.keys() if not k.startswith(h3t.PAD_PREFIX)} == set(sd)
        for name, want in sd.items():
            assert raw(f.get_tensor(name)) == raw(want), name


@pytest.mark.parametrize("quant", [True, False])
def test_alignment_contiguity_and_identical_block_layout(tmp_path, quant, quant_sd, dense_sd):
    dst, _ = write(tmp_path, quant_sd if quant else dense_sd)
    hdr = h3t.read_header(dst)
    assert hdr.data_start % h3t.BLOCK_ALIGN == 0
    pos = 0
    for name, e in sorted(hdr.tensors.items(), key=lambda kv: kv[1]["data_offsets"][0]):
        a, b = e["data_offsets"]
        assert a == pos, name
        if not name.startswith(h3t.PAD_PREFIX):
            assert (hdr.data_start + a) % h3t.TENSOR_ALIGN == 0, name
        pos = b
    assert hdr.data_start + pos == hdr.file_size
    with h3t.H3TFile(dst) as f:
        assert f.block_nbytes % h3t.BLOCK_ALIGN == 0
        for i in range(f.n_blocks):
            a, b = f.block_range(i)
            assert a % h3t.BLOCK_ALIGN == 0 and b - a == f.block_nbytes and f.block_bytes(i).shape == (f.block_nbytes,)
            for e in f.block_layout:
                info = f.info(f"blocks.{i}.{e.name}")
                assert info.start == a + e.offset and info.nbytes == e.nbytes and e.offset + e.nbytes <= f.block_nbytes
        assert f.block_range(1)[0] == f.block_range(0)[1]


def test_block_weights_are_views_of_any_buffer(tmp_path, quant_sd):
    with h3t.H3TFile(GOLDEN) as f:
        for i in range(f.n_blocks):
            w = f.block_weights_cpu(i)
            for lin, p in ((w.qkv, "attn.qkv_proj"), (w.out, "attn.out_proj"), (w.fc1, "mlp.fc1"), (w.fc2, "mlp.fc2")):
                pre = f"blocks.{i}.{p}."
                assert isinstance(lin, W4A8Weight) and (lin.group_size, lin.convrot) == (16, 16)
                assert lin.q.dtype == torch.int8 and lin.s_rel.dtype == torch.float8_e4m3fn and lin.s_ch.dtype == torch.float32
                assert raw(lin.q) == raw(quant_sd[pre + "weight"]) and raw(lin.s_rel) == raw(quant_sd[pre + "weight_s_rel"])
                assert raw(lin.s_ch) == raw(quant_sd[pre + "weight_s_channel"])
                assert raw(lin.codebook) == raw(quant_sd[pre + "weight_codebook"])
            assert raw(w.adaln_w) == raw(quant_sd[f"blocks.{i}.adaln_proj.linear.weight"])
            buf = torch.empty(f.block_nbytes, dtype=torch.uint8)
            buf.copy_(f.block_tensor(i))
            w2 = f.block_weights_from(buf)
            assert raw(w2.fc2.q) == raw(w.fc2.q) and w2.fc2.q.data_ptr() != w.fc2.q.data_ptr()
        with pytest.raises(ValueError):
            f.block_weights_from(torch.empty(10, dtype=torch.uint8))


def test_dense_blocks_are_plain_tensors(tmp_path, dense_sd):
    dst, _ = write(tmp_path, dense_sd)
    with h3t.H3TFile(dst) as f:
        w = f.block_weights_cpu(1)
        assert all(isinstance(t, torch.Tensor) and t.dtype == torch.bfloat16 for t in (w.qkv, w.out, w.fc1, w.fc2))
        assert w.qkv.shape == (192, 64) and w.fc2.shape == (64, 48) and f.quant == {}


def test_output_is_deterministic_and_chunk_size_independent(tmp_path, quant_sd):
    a, _ = write(tmp_path, quant_sd, "a.h3t", chunk_bytes=4096)
    b, _ = write(tmp_path, quant_sd, "b.h3t", chunk_bytes=1 << 20)
    assert open(a, "rb").read() == open(b, "rb").read()


def test_interrupted_write_leaves_no_file(tmp_path, quant_sd):
    def boom():
        raise RuntimeError("source failed")

    sd = dict(quant_sd)
    sd["blocks.1.norm2.weight"] = h3t.LazySource("BF16", (64,), boom)
    dst = str(tmp_path / "x.h3t")
    with pytest.raises(RuntimeError, match="source failed"):
        h3t.write_h3t(dst, cfg(), sd)
    assert not os.path.exists(dst) and not os.path.exists(dst + ".part")


def test_lazy_sources_write_the_same_file(tmp_path, quant_sd):
    lazy = {k: h3t.LazySource(h3t.st_dtype(v.dtype), tuple(v.shape), lambda v=v: v) for k, v in quant_sd.items()}
    a, _ = write(tmp_path, lazy, "lazy.h3t", source_name="tiny", source_size=123)
    assert open(a, "rb").read() == open(GOLDEN, "rb").read()


def test_reader_rejects_foreign_truncated_and_corrupt_files(tmp_path):
    plain = str(tmp_path / "plain.safetensors")
    head = json.dumps({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    open(plain, "wb").write(struct.pack("<Q", len(head)) + head + bytes(16))
    with pytest.raises(h3t.H3TError, match="not an h3t"):
        h3t.H3TFile(plain)
    data = open(GOLDEN, "rb").read()
    for cut in (len(data) - 1, len(data) // 2, 10):
        p = str(tmp_path / f"cut{cut}.h3t")
        open(p, "wb").write(data[:cut])
        with pytest.raises(h3t.H3TError):
            h3t.H3TFile(p)
    p = str(tmp_path / "junk.h3t")
    open(p, "wb").write(b"\x05\x00\x00\x00\x00\x00\x00\x00hello world")
    with pytest.raises(h3t.H3TError):
        h3t.H3TFile(p)
    p = str(tmp_path / "trailing.h3t")
    open(p, "wb").write(data + bytes(8))
    with pytest.raises(h3t.H3TError, match="exactly|trailing"):
        h3t.H3TFile(p)
    n = struct.unpack("<Q", data[:8])[0]
    table = json.loads(data[8:8 + n])
    table["__metadata__"]["version"] = "99"
    new = json.dumps(table).encode()
    p = str(tmp_path / "v99.h3t")
    open(p, "wb").write(struct.pack("<Q", n) + new.ljust(n, b" ") + data[8 + n:])
    with pytest.raises(h3t.H3TError, match="version"):
        h3t.H3TFile(p)


def _patch_meta(path, **changes):
    with open(path, "r+b") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        table = json.loads(f.read(n))
        for k, v in changes.items():
            if v is None:
                table["__metadata__"].pop(k)
            else:
                table["__metadata__"][k] = v
        blob = json.dumps(table, separators=(",", ":")).encode()
        f.seek(8)
        f.write(blob.ljust(n, b" "))


@pytest.mark.parametrize("change", [{"block_ranges": None}, {"version": "x"}, {"block_ranges": "5"},
                                    {"block_ranges": "[[1, 2]]"}, {"block_layout": "[]x"}, {"n_blocks": "3"}])
def test_corrupt_metadata_raises_h3terror(tmp_path, quant_sd, change):
    dst, _ = write(tmp_path, quant_sd)
    _patch_meta(dst, **change)
    with pytest.raises(h3t.H3TError):
        h3t.H3TFile(dst)


def test_closed_file_refuses_access_and_views_outlive_it():
    f = h3t.H3TFile(GOLDEN)
    view = f.tensor("rope.inv_freq")
    f.close()
    f.close()
    with pytest.raises(ValueError, match="closed"):
        f.block_bytes(0)
    assert view.shape == (16,)


def test_writer_rejects_inconsistent_inputs(tmp_path, quant_sd):
    with pytest.raises(h3t.H3TError, match="reserved padding"):
        h3t.write_h3t(str(tmp_path / "a"), cfg(), {**quant_sd, "__pad.1": torch.zeros(1)})
    bad = dict(quant_sd)
    bad["blocks.1.attn.k_norm.weight"] = torch.zeros(32, dtype=torch.float32)
    with pytest.raises(h3t.H3TError, match="block 0 has"):
        h3t.write_h3t(str(tmp_path / "b"), cfg(), bad)
    bad = {k: v for k, v in quant_sd.items() if k != "blocks.1.attn.k_norm.weight"}
    with pytest.raises(h3t.H3TError, match="differs from block 0"):
        h3t.write_h3t(str(tmp_path / "c"), cfg(), bad)
    with pytest.raises(h3t.H3TError, match="blocks"):
        h3t.write_h3t(str(tmp_path / "d"), cfg(layers=3), quant_sd)


def test_config_json_round_trip_and_from_shapes(quant_sd):
    c = cfg()
    assert H3Config.from_json(c.to_json()) == c
    shapes = {k: tuple(v.shape) for k, v in quant_sd.items()}
    shapes["blocks.0.attn.qkv_proj.weight"] = (192, 32)
    got = H3Config.from_shapes(shapes)
    assert (got.hidden, got.layers, got.refiner_layers, got.heads, got.head_dim, got.ffn) == (64, 2, 1, 2, 32, 48)
    assert (got.curve_grid, got.t_dim, got.text_dim) == (17, 8, 32)


def test_host_block_store_from_h3t_holds_the_file_blocks():
    with h3t.H3TFile(GOLDEN) as f:
        st = HostBlockStore.from_h3t(f)
        assert (st.n_blocks, st.block_nbytes) == (f.n_blocks, f.block_nbytes)
        for i in range(f.n_blocks):
            assert np.array_equal(st.block_bytes(i), f.block_bytes(i))
            a, b = st.block_weights_cpu(i), f.block_weights_cpu(i)
            assert raw(a.qkv.q) == raw(b.qkv.q) and raw(a.fc2.s_rel) == raw(b.fc2.s_rel) and raw(a.norm2) == raw(b.norm2)


def test_streaming_provider_reads_an_h3t_file_on_the_cpu():
    with h3t.H3TFile(GOLDEN) as f, StreamingProvider(f, "cpu", resident=0, ring=2, prefetch=1) as p:
        for _ in range(2):
            p.begin_forward()
            for i in range(f.n_blocks):
                w = p.acquire(i)
                assert raw(w.out.q) == raw(f.block_weights_cpu(i).out.q)
                p.release(i)
            p.end_forward()
