"""ComfyUI node "H3-Turbo Fast UNET Loader (h3t)": the H3 4-bit checkpoint (.h3t) as an ordinary MODEL whose DiT forward
runs on this build's MI355X engine (reference comfy_h3_nodes.py:1-355).

ComfyUI's conditioning, samplers and VAE nodes are unchanged; only the diffusion model is replaced by
h3turbo_amd.comfy_dit.H3TurboDiT, a stub without weights.  The ModelPatcher subclass lets ComfyUI's memory manager
treat the engine like a partially loaded model: partially_load hands over the VRAM budget the engine builds itself
in (resident blocks + a 3-slot streaming ring), partially_unload shrinks it (ring first, then resident blocks) or
parks it (no device memory, page-locked host copies kept), detach parks it.

Limits: run-time LoRAs are refused with a clear error (the 4-bit weights stream and are never patched); block-level
model patches are not honoured.  Only the exact attention is available.
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
FOLDER = "h3turbo_h3t"  # models/h3turbo, *.h3t only
folder_paths.add_model_folder_path(FOLDER, os.path.join(folder_paths.models_dir, "h3turbo"))
_paths, _ = folder_paths.folder_names_and_paths[FOLDER]
folder_paths.folder_names_and_paths[FOLDER] = (_paths, {".h3t"})


class ComfyMemoryHost:
    """ComfyUI's model_management as the DiT's memory host."""

    def device(self) -> torch.device:
        return mm.get_torch_device()

    def free_memory(self, device: torch.device) -> int:
        return int(mm.get_free_memory(device))

    def park_headroom(self) -> int:
        """Free host RAM to keep when page-locking blocks that leave the GPU: 3.5 GiB, so the pinned copies never
        push the host into the RAM pressure that makes ComfyUI evict models."""
        return (3 << 30) + (512 << 20)


class H3TurboBaseModel(comfy.model_base.MiniMaxH3):
    """ComfyUI's MiniMax H3 model object (conditioning, latent scaling, masks, layout payload) around the stub DiT."""

    def __init__(self, model_config, dit, device=None):
        # MiniMaxH3.__init__ would build the full-precision network; BaseModel gets the stub instead
        comfy.model_base.BaseModel.__init__(self, model_config, comfy.model_base.ModelType.FLOW_AV, device=device,
                                            unet_model=lambda **_: dit)


class H3TurboPatcher(comfy.model_patcher.ModelPatcher):
    """ModelPatcher whose 'weights' are the engine's device state: built on partially_load, shrunk or parked on
    partially_unload, parked on detach."""

    def _dit(self) -> H3TurboDiT:
        return self.model.diffusion_model

    def model_size(self):
        return self._dit().model_bytes()

    def loaded_size(self):
        return self._dit().gpu_bytes()

    def add_patches(self, patches, strength_patch=1.0, strength_model=1.0):
        if patches:
            raise RuntimeError("H3-Turbo Fast UNET Loader cannot apply LoRAs or weight patches at run time (the 4-bit "
                               "weights are streamed, never patched). Merge the LoRA into the checkpoint, or use the core "
                               "UNETLoader for this workflow.")
        return []

    def load(self, device_to=None, lowvram_model_memory=0, force_patch_weights=False, full_load=False):
        with self.use_ejected():
            self.unpatch_hooks()
            self.model.device = device_to
            self.model.current_weight_patches_uuid = self.patches_uuid
            self.model.model_loaded_weight_memory = self.loaded_size()
            for callback in self.get_all_callbacks(comfy.patcher_extension.CallbacksMP.ON_LOAD):
                callback(self, device_to, lowvram_model_memory, force_patch_weights, full_load)
            self.apply_hooks(self.forced_hooks, force_apply=True)

    def partially_load(self, device_to, extra_memory=0, force_patch_weights=False):
        with self.use_ejected(skip_and_inject_on_exit_only=True):
            self.unpatch_model(self.offload_device, unpatch_weights=False)
            self.patch_model(load_weights=False)  # object patches (e.g. the sigma-shift model_sampling)
            placed = self._dit().ensure_loaded(extra_memory if extra_memory and extra_memory < 1e30 else None)
            self.load(device_to, lowvram_model_memory=extra_memory, force_patch_weights=force_patch_weights)
            return placed

    def partially_unload(self, device_to, memory_to_free=0, force_patch_weights=False):
        dit = self._dit()
        if memory_to_free and memory_to_free < dit.gpu_bytes():
            freed = dit.shrink(int(memory_to_free))
        else:
            freed = dit.unload()
        self.model.model_loaded_weight_memory = dit.gpu_bytes()
        return freed

    def detach(self, unpatch_all=True):
        if unpatch_all:  # detach(False) swaps this patcher for a clone sharing the same engine
            self._dit().unload()
        return super().detach(unpatch_all)


def unet_config(cfg) -> dict:
    """The dict ComfyUI's model detection derives from a curve-form H3 checkpoint."""
    return {
        "image_model": "minimax_h3", "num_layers": cfg.layers, "token_refiner_num_layers": cfg.refiner_layers,
        "hidden_size": cfg.hidden, "latents_dim": cfg.video_channels, "audio_latents_dim": cfg.audio_channels,
        "attention_head_dim": cfg.head_dim, "num_attention_heads": cfg.heads, "ffn_hidden_size": cfg.ffn,
        "text_dim": cfg.text_dim, "adaln_curve_grid": cfg.curve_grid, "time_embed_dim": cfg.t_dim,
        "rope_inv_freq_len": cfg.rope_inv_freq_len, "gate_compress": False,
    }


def build_model_patcher(path: str, precision: str = "a8", resident_blocks: int = 0, mlp_chunk: int = 0,
                        attention: str = "exact") -> H3TurboPatcher:
    load_device, offload_device = mm.get_torch_device(), mm.unet_offload_device()
    probe = comfy.supported_models.MiniMaxH3({"image_model": "minimax_h3"})
    # ComfyUI's own choice for H3 (bf16 or fp32); honours --fp32-unet
    dtype = mm.unet_dtype(load_device, supported_dtypes=list(probe.supported_inference_dtypes))
    if dtype not in (torch.bfloat16, torch.float32):
        dtype = torch.float32
    dit = H3TurboDiT(path, precision, resident_blocks, mlp_chunk, attention, dtype, host=ComfyMemoryHost())
    model_config = comfy.supported_models.MiniMaxH3(unet_config(dit.cfg))
    manual_cast = mm.unet_manual_cast(dtype, load_device, model_config.supported_inference_dtypes)
    model_config.set_inference_dtype(dtype, manual_cast, device=load_device)
    LOG.info("H3-Turbo Fast UNET Loader: compute dtype %s", dtype)
    model = H3TurboBaseModel(model_config, dit, device=offload_device)
    return H3TurboPatcher(model, load_device=load_device, offload_device=offload_device)


class H3TurboFastUNetLoader:
    CATEGORY = "H3-Turbo"
    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load"
    DESCRIPTION = ("Loads a converted official-H3 4-bit checkpoint (.h3t) and runs it on the MI355X H3-Turbo engine. Same "
                   "MODEL output as UNETLoader, with weight copies hidden behind compute. No run-time LoRAs.")

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {
            "h3t_name": (folder_paths.get_filename_list(FOLDER),),
            "precision": (["a8", "a16"], {"default": "a8", "tooltip": "a8 = the checkpoint's native int8 activations "
                                                                       "(fast). a16 = unquantised activations (slower)."}),
            "resident_blocks": ("INT", {"default": 0, "min": 0, "max": 200,
                                        "tooltip": "Blocks kept on the GPU. 0 = as many as ComfyUI's VRAM budget allows."}),
            "mlp_chunk": ("INT", {"default": 0, "min": 0, "max": 65536,
                                  "tooltip": "Rows per MLP pass. 0 = automatic (chunks only when a long clip would not fit)."}),
            "attention": (["exact"], {"default": "exact", "tooltip": "exact = the reference SDPA."}),
        }}

    def load(self, h3t_name, precision, resident_blocks, mlp_chunk, attention="exact"):
        path = folder_paths.get_full_path_or_raise(FOLDER, h3t_name)
        return (build_model_patcher(path, precision, resident_blocks, mlp_chunk, attention),)


NODE_CLASS_MAPPINGS = {"H3TurboFastUNetLoader": H3TurboFastUNetLoader}
NODE_DISPLAY_NAME_MAPPINGS = {"H3TurboFastUNetLoader": "H3-Turbo Fast UNET Loader (h3t)"}
