"""ComfyUI node "H3-Turbo Fast UNET Loader (h3t)": an H3 4-bit checkpoint (.h3t) as an ordinary MODEL whose DiT forward
runs on this build's MI355X engine (the reference's node: comfy_h3_nodes.py:1-355).

Only the diffusion model is replaced, by h3turbo_amd.comfy_dit.H3TurboDiT, an object without weights of its own;
ComfyUI's conditioning, samplers and VAE nodes are unchanged.  ComfyUI's memory manager sees the engine through a
ModelPatcher whose "weights" are the engine's device footprint:

    partially_load(extra_memory)    build the engine in that budget (or bring a parked one back)
    partially_unload(memory_to_free) give back that much (ring slots first, then resident blocks), or park it all
    detach()                        park

Limits: run-time LoRAs and weight patches are refused with a clear error (the 4-bit weights are streamed, never
patched); block-level model patches are not honoured; only the exact attention exists.
"""
import logging
import os
import sys

import torch

import comfy.model_base
import comfy.model_management as mm
import comfy.model_patcher
import comfy.patcher_extension
import comfy.supported_models
import folder_paths

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from h3turbo_amd.comfy_dit import H3TurboDiT  # noqa: E402

LOG = logging.getLogger("h3turbo_amd")
FOLDER = "h3turbo_h3t"  # <models>/h3turbo, *.h3t files only
folder_paths.add_model_folder_path(FOLDER, os.path.join(folder_paths.models_dir, "h3turbo"))
folder_paths.folder_names_and_paths[FOLDER] = (folder_paths.folder_names_and_paths[FOLDER][0], {".h3t"})

_NO_PATCHES = ("H3-Turbo Fast UNET Loader cannot apply LoRAs or weight patches at run time (the 4-bit weights are "
               "streamed, never patched). Merge the LoRA into the checkpoint, or use the core UNETLoader for this "
               "workflow.")


class ComfyMemoryHost:
    """ComfyUI's model_management answering the DiT's memory questions."""

    def device(self) -> torch.device:
        return mm.get_torch_device()

    def free_memory(self, device: torch.device) -> int:
        return int(mm.get_free_memory(device))

    def park_headroom(self) -> int:
        """Host RAM kept free when blocks leaving the GPU are page-locked (3.5 GiB): pinned copies must not push the
        host into the RAM pressure that makes ComfyUI evict models."""
        return (3 << 30) + (512 << 20)


class H3TurboBaseModel(comfy.model_base.MiniMaxH3):
    """ComfyUI's MiniMax H3 model object (conditioning, latent scaling, masks, layout payload) around the DiT
    stand-in.  MiniMaxH3.__init__ would build the full-precision network, so BaseModel's is called with the stand-in
    as the unet."""

    def __init__(self, model_config, dit, device=None):
        comfy.model_base.BaseModel.__init__(self, model_config, comfy.model_base.ModelType.FLOW_AV, device=device,
                                            unet_model=lambda **_: dit)


class H3TurboPatcher(comfy.model_patcher.ModelPatcher):
    """ModelPatcher over the engine's device footprint instead of module weights."""

    @property
    def dit(self) -> H3TurboDiT:
        return self.model.diffusion_model

    def model_size(self):
        return self.dit.model_bytes()

    def loaded_size(self):
        return self.dit.gpu_bytes()

    def add_patches(self, patches, strength_patch=1.0, strength_model=1.0):
        if patches:
            raise RuntimeError(_NO_PATCHES)
        return []

    def load(self, device_to=None, lowvram_model_memory=0, force_patch_weights=False, full_load=False):
        # ModelPatcher.load's bookkeeping without moving any module weights (the stand-in has none)
        with self.use_ejected():
            self.unpatch_hooks()
            self.model.device = device_to
            self.model.current_weight_patches_uuid = self.patches_uuid
            self.model.model_loaded_weight_memory = self.loaded_size()
            for cb in self.get_all_callbacks(comfy.patcher_extension.CallbacksMP.ON_LOAD):
                cb(self, device_to, lowvram_model_memory, force_patch_weights, full_load)
            self.apply_hooks(self.forced_hooks, force_apply=True)

    def partially_load(self, device_to, extra_memory=0, force_patch_weights=False):
        grant = extra_memory if extra_memory and extra_memory < 1e30 else None  # "no limit" -> what is free
        with self.use_ejected(skip_and_inject_on_exit_only=True):
            self.unpatch_model(self.offload_device, unpatch_weights=False)
            self.patch_model(load_weights=False)  # object patches only, e.g. a sigma-shift model_sampling
            placed = self.dit.ensure_loaded(grant)
            self.load(device_to, lowvram_model_memory=extra_memory, force_patch_weights=force_patch_weights)
        return placed

    def partially_unload(self, device_to, memory_to_free=0, force_patch_weights=False):
        part = 0 < memory_to_free < self.dit.gpu_bytes()
        freed = self.dit.shrink(int(memory_to_free)) if part else self.dit.unload()
        self.model.model_loaded_weight_memory = self.dit.gpu_bytes()
        return freed

    def detach(self, unpatch_all=True):
        if unpatch_all:  # detach(False) hands the engine to a clone of this patcher: keep it on the device
            self.dit.unload()
        return super().detach(unpatch_all)


# ComfyUI's detected unet_config key -> H3Config field, for a curve-form H3 checkpoint
_UNET_KEYS = (("num_layers", "layers"), ("token_refiner_num_layers", "refiner_layers"), ("hidden_size", "hidden"),
              ("latents_dim", "video_channels"), ("audio_latents_dim", "audio_channels"),
              ("attention_head_dim", "head_dim"), ("num_attention_heads", "heads"), ("ffn_hidden_size", "ffn"),
              ("text_dim", "text_dim"), ("adaln_curve_grid", "curve_grid"), ("time_embed_dim", "t_dim"),
              ("rope_inv_freq_len", "rope_inv_freq_len"))


def unet_config(cfg) -> dict:
    """The dict ComfyUI's model detection derives from a curve-form H3 checkpoint."""
    out = {"image_model": "minimax_h3"}
    out.update({key: getattr(cfg, field) for key, field in _UNET_KEYS})
    out["gate_compress"] = False
    return out


def _compute_dtype(load_device) -> torch.dtype:
    """ComfyUI's own choice for H3 (honours --fp32-unet); anything but bf16 / fp32 runs in fp32."""
    probe = comfy.supported_models.MiniMaxH3({"image_model": "minimax_h3"})
    dtype = mm.unet_dtype(load_device, supported_dtypes=list(probe.supported_inference_dtypes))
    return dtype if dtype in (torch.bfloat16, torch.float32) else torch.float32


def build_model_patcher(path: str, precision: str = "a8", resident_blocks: int = 0, mlp_chunk: int = 0,
                        attention: str = "exact") -> H3TurboPatcher:
    load_device, offload_device = mm.get_torch_device(), mm.unet_offload_device()
    dtype = _compute_dtype(load_device)
    dit = H3TurboDiT(path, precision, resident_blocks, mlp_chunk, attention, dtype, host=ComfyMemoryHost())
    conf = comfy.supported_models.MiniMaxH3(unet_config(dit.cfg))
    conf.set_inference_dtype(dtype, mm.unet_manual_cast(dtype, load_device, conf.supported_inference_dtypes),
                             device=load_device)
    LOG.info("H3-Turbo Fast UNET Loader: %s, compute dtype %s", os.path.basename(path), dtype)
    return H3TurboPatcher(H3TurboBaseModel(conf, dit, device=offload_device), load_device=load_device,
                          offload_device=offload_device)


class H3TurboFastUNetLoader:
    CATEGORY = "H3-Turbo"
    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load"
    DESCRIPTION = ("Loads a converted official-H3 4-bit checkpoint (.h3t) and runs it on the MI355X H3-Turbo engine: "
                   "the same MODEL output as UNETLoader, weight copies hidden behind compute, no run-time LoRAs.")

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {
            "h3t_name": (folder_paths.get_filename_list(FOLDER),),
            "precision": (["a8", "a16"], {"default": "a8", "tooltip": "a8: the checkpoint's native int8 activations "
                                                                       "(fast). a16: unquantised activations (slower)."}),
            "resident_blocks": ("INT", {"default": 0, "min": 0, "max": 200,
                                        "tooltip": "Blocks kept on the GPU; 0 = as many as ComfyUI's VRAM budget allows."}),
            "mlp_chunk": ("INT", {"default": 0, "min": 0, "max": 65536,
                                  "tooltip": "Rows per MLP pass; 0 = automatic (chunks only when a long clip would not fit)."}),
            "attention": (["exact"], {"default": "exact", "tooltip": "exact: PyTorch SDPA, the reference's attention."}),
        }}

    def load(self, h3t_name, precision, resident_blocks, mlp_chunk, attention="exact"):
        return (build_model_patcher(folder_paths.get_full_path_or_raise(FOLDER, h3t_name), precision,
                                    resident_blocks, mlp_chunk, attention),)


NODE_CLASS_MAPPINGS = {"H3TurboFastUNetLoader": H3TurboFastUNetLoader}
NODE_DISPLAY_NAME_MAPPINGS = {"H3TurboFastUNetLoader": "H3-Turbo Fast UNET Loader (h3t)"}
