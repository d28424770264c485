"""The ComfyUI node and its DiT stand-in (comfy_h3_nodes.py, h3turbo_amd/comfy_dit.py) on the CPU with a tiny dense
.h3t file.  ComfyUI is not installed here: its modules are replaced by minimal stand-ins with the attributes the
node touches, so what is tested is the node's own wiring (node mapping, inputs, LoRA refusal, partially_load /
partially_unload / detach routing) and the engine lifecycle (build inside a budget, park, come back, shrink,
close) with forwards equal to the model's own."""
import contextlib
import importlib.util
import os
import sys
import types

import pytest
import torch

import model_cases as mc
from h3turbo_amd.comfy_dit import H3TurboDiT, TorchMemoryHost
from h3turbo_amd.h3t import write_h3t

CFG = mc.CFG
PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "minimax-h3-turbo_amd")


class FixedHost(TorchMemoryHost):
    """A memory host with a fixed free amount (the CPU has no device memory to query)."""

    def __init__(self, free):
        super().__init__("cpu", park_headroom_bytes=0)
        self.free = free

    def free_memory(self, device):
        return self.free


@pytest.fixture()
def tiny_h3t(tmp_path):
    sd = mc.make_sd(CFG, 51)
    path = tmp_path / "tiny.h3t"
    write_h3t(path, CFG, sd)
    return str(path), sd


def reference_velocity(sd, x, sigma, refined):
    from h3turbo_amd.block import ResidentProvider
    from h3turbo_amd.model import H3Model, weights_from_state_dict

    glob, blocks = weights_from_state_dict(sd, CFG, "cpu", torch.float32)
    m = H3Model(CFG, glob, ResidentProvider(blocks), device="cpu", dtype=torch.float32)
    return m.forward(x, sigma, None, refined_text=refined)


def test_dit_lifecycle_budget_park_shrink_close(tiny_h3t):
    path, sd = tiny_h3t
    dit = H3TurboDiT(path, dtype=torch.float32, host=FixedHost(1 << 40))
    try:
        blk = dit.store.block_nbytes
        assert len(dit.blocks) == CFG.layers and dit.gpu_bytes() == 0 and dit.model_bytes() == os.path.getsize(path)
        with pytest.raises(ValueError):
            H3TurboDiT(path, attention="int8_fast")
        placed = dit.ensure_loaded()
        p = dit.engine.provider
        assert placed == dit.gpu_bytes() and p.stats()["resident"] == CFG.layers  # everything fits
        assert dit.ensure_loaded() == 0  # already loaded: nothing new
        v, a, text = mc.inputs(CFG, 52)
        refined = dit.preprocess_text_embeds(text)
        assert refined.shape == (1, text.shape[1], CFG.hidden)
        assert torch.equal(dit.preprocess_text_embeds(refined), refined)
        ts = torch.tensor([700.0])
        out = dit.forward([v, a], ts, refined)
        want = reference_velocity(sd, [v, a], (ts[0] / 1000.0).float(), refined)
        assert torch.equal(out[0], want[0]) and torch.equal(out[1], want[1])
        # park: no device memory; the next forward brings the blocks back and gives the same numbers
        freed = dit.unload()
        assert freed == CFG.layers * blk and p.device_bytes() == 0 and p.parked
        assert dit.ensure_loaded(budget=0) > 0 and not p.parked
        assert torch.equal(dit.forward([v, a], ts, refined)[0], out[0])
        # shrink by one block: the ring is empty, so one resident block goes
        before = p.device_bytes()
        assert dit.shrink(blk) == blk and p.device_bytes() == before - blk
        assert torch.equal(dit.forward([v, a], ts, refined)[0], out[0])
        assert dit.close_engine() > 0 and dit.engine is None and dit.gpu_bytes() == 0
        assert torch.equal(dit.forward([v, a], ts, refined)[0], out[0])  # rebuilt on demand
    finally:
        dit.close()


def test_dit_forward_options(tiny_h3t):
    path, sd = tiny_h3t
    dit = H3TurboDiT(path, dtype=torch.float32, host=FixedHost(1 << 40), mlp_chunk=3)
    try:
        v, a, text = mc.inputs(CFG, 53)
        refined = dit.preprocess_text_embeds(text)
        ts = torch.tensor([450.0])
        base = dit.forward([v, a], ts, refined)
        assert dit.engine.model.mlp_chunk == 3
        want = reference_velocity(sd, [v, a], (ts[0] / 1000.0).float(), refined)
        assert mc.rel(base[0], want[0]) < 1e-6  # chunked MLP: exact up to GEMM tiling
        shifted = dit.forward([v, a], ts, refined, transformer_options={"minimax_h3_sigma_shift_audio": 5.0})
        assert not torch.equal(shifted[0], base[0])  # the audio schedule reaches both streams
        stale = {"layout": object()}  # a host-built layout is ignored
        assert torch.equal(dit.forward([v, a], ts, refined, minimax_payload=stale)[0], base[0])
        dit.mlp_chunk = 0
        small = FixedHost(1 << 20)  # 1 MiB free: the automatic chunk kicks in
        dit.host = small
        assert dit.pick_mlp_chunk([v, a], refined) == 4096
        dit.host = FixedHost(1 << 40)
        assert dit.pick_mlp_chunk([v, a], refined) is None
    finally:
        dit.close()


# ------------------------------------------------------------------------------------------------ the node
def _fake_comfy(models_dir, device, free):
    """Stand-ins for the ComfyUI modules the node imports (only the attributes it uses)."""
    comfy = types.ModuleType("comfy")
    mb = types.ModuleType("comfy.model_base")

    class BaseModel(torch.nn.Module):
        def __init__(self, model_config, model_type, device=None, unet_model=None):
            super().__init__()
            self.model_config, self.model_type, self.device = model_config, model_type, device
            self.diffusion_model = unet_model()

    class MiniMaxH3(BaseModel):
        def __init__(self, *a, **k):
            raise AssertionError("the node must not build the full-precision network")

    mb.BaseModel, mb.MiniMaxH3 = BaseModel, MiniMaxH3
    mb.ModelType = types.SimpleNamespace(FLOW_AV="flow_av")
    mm = types.ModuleType("comfy.model_management")
    mm.get_torch_device = lambda: device
    mm.get_free_memory = lambda dev=None: free
    mm.unet_offload_device = lambda: torch.device("cpu")
    mm.unet_dtype = lambda dev, supported_dtypes=None: torch.float32
    mm.unet_manual_cast = lambda dtype, dev, supported: None
    mp = types.ModuleType("comfy.model_patcher")

    class ModelPatcher:
        def __init__(self, model, load_device, offload_device):
            self.model, self.load_device, self.offload_device = model, load_device, offload_device
            self.patches_uuid, self.forced_hooks, self.detached = "uuid", [], False

        @contextlib.contextmanager
        def use_ejected(self, skip_and_inject_on_exit_only=False):
            yield

        def unpatch_hooks(self):
            pass

        def unpatch_model(self, device_to=None, unpatch_weights=True):
            pass

        def patch_model(self, load_weights=True):
            pass

        def get_all_callbacks(self, kind):
            return []

        def apply_hooks(self, hooks, force_apply=False):
            pass

        def detach(self, unpatch_all=True):
            self.detached = True
            return self

    mp.ModelPatcher = ModelPatcher
    pe = types.ModuleType("comfy.patcher_extension")
    pe.CallbacksMP = types.SimpleNamespace(ON_LOAD="on_load")
    sm = types.ModuleType("comfy.supported_models")

    class MiniMaxH3Config:
        supported_inference_dtypes = [torch.bfloat16, torch.float32]

        def __init__(self, unet_config):
            self.unet_config = unet_config

        def set_inference_dtype(self, dtype, manual_cast, device=None):
            self.dtype = dtype

    sm.MiniMaxH3 = MiniMaxH3Config
    fp = types.ModuleType("folder_paths")
    fp.models_dir = models_dir
    fp.folder_names_and_paths = {}

    def add_model_folder_path(name, path):
        fp.folder_names_and_paths.setdefault(name, ([], set()))[0].append(path)

    fp.add_model_folder_path = add_model_folder_path
    fp.get_filename_list = lambda name: sorted(f for d in fp.folder_names_and_paths[name][0] if os.path.isdir(d)
                                               for f in os.listdir(d) if f.endswith(".h3t"))
    fp.get_full_path_or_raise = lambda name, f: os.path.join(fp.folder_names_and_paths[name][0][0], f)
    comfy.model_base, comfy.model_management, comfy.model_patcher = mb, mm, mp
    comfy.patcher_extension, comfy.supported_models = pe, sm
    return {"comfy": comfy, "comfy.model_base": mb, "comfy.model_management": mm, "comfy.model_patcher": mp,
            "comfy.patcher_extension": pe, "comfy.supported_models": sm, "folder_paths": fp}


def test_node_wiring_with_stand_in_comfy_modules(tmp_path, monkeypatch):
    sd = mc.make_sd(CFG, 54)
    os.makedirs(tmp_path / "h3turbo")
    write_h3t(tmp_path / "h3turbo" / "tiny.h3t", CFG, sd)
    for name, mod in _fake_comfy(str(tmp_path), torch.device("cpu"), 1 << 40).items():
        monkeypatch.setitem(sys.modules, name, mod)
    spec = importlib.util.spec_from_file_location("comfy_h3_nodes_under_test", os.path.join(PKG, "comfy_h3_nodes.py"))
    nodes = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(nodes)
    assert list(nodes.NODE_CLASS_MAPPINGS) == ["H3TurboFastUNetLoader"]
    req = nodes.H3TurboFastUNetLoader.INPUT_TYPES()["required"]
    assert req["h3t_name"][0] == ["tiny.h3t"] and req["precision"][0] == ["a8", "a16"]
    assert nodes.unet_config(CFG)["num_layers"] == CFG.layers and nodes.unet_config(CFG)["hidden_size"] == CFG.hidden
    (patcher,) = nodes.H3TurboFastUNetLoader().load("tiny.h3t", "a8", 0, 0)
    dit = patcher.model.diffusion_model
    try:
        assert isinstance(dit, H3TurboDiT) and dit.dtype == torch.float32
        assert patcher.model_size() == dit.model_bytes() and patcher.loaded_size() == 0
        assert patcher.add_patches({}) == []
        with pytest.raises(RuntimeError, match="LoRA"):
            patcher.add_patches({"diffusion_model.blocks.0.attn.qkv_proj.weight": (1,)})
        placed = patcher.partially_load(torch.device("cpu"), extra_memory=1 << 40)
        assert placed == dit.gpu_bytes() > 0 and patcher.model.model_loaded_weight_memory == placed
        blk = dit.store.block_nbytes
        assert patcher.partially_unload(torch.device("cpu"), memory_to_free=blk) == blk  # shrink, not park
        assert dit.engine.provider.device_bytes() == (CFG.layers - 1) * blk
        assert patcher.partially_unload(torch.device("cpu"), memory_to_free=0) == (CFG.layers - 1) * blk  # park
        assert dit.engine.provider.parked
        patcher.partially_load(torch.device("cpu"), extra_memory=1 << 40)
        assert not dit.engine.provider.parked
        assert patcher.detach() is patcher and patcher.detached and dit.engine.provider.parked
    finally:
        dit.close()
