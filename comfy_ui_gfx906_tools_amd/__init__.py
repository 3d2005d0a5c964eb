"""MI355X (gfx950) quantized-linear engine behind the reference's ComfyUI node API: ComfyUI loads
this package as a custom node pack through the two mappings below (the reference's
nodes/ComfyUI-Gfx906Int4/__init__.py exports the same names)."""
from .nodes import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
