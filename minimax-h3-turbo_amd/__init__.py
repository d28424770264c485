"""ComfyUI custom-node entry point: ComfyUI imports this directory's __init__ and reads its node mappings
(install by linking this directory into ComfyUI/custom_nodes).  Nothing else imports it."""
from .comfy_h3_nodes import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
