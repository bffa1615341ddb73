"""ComfyUI custom-node entry (the repository cloned into ComfyUI's custom_nodes).

reference ``__init__.py:1-26``: exports the node mappings of
``rdna3_fastmm.comfyui`` from this checkout's ``rdna3-fastmm_amd`` directory,
and refuses to run next to a different ``rdna3_fastmm`` that is already
imported (two copies would register the same operators twice).
"""

from pathlib import Path
import sys

_source_root = Path(__file__).resolve().parent / "rdna3-fastmm_amd"
_loaded = sys.modules.get("rdna3_fastmm")
if _loaded is not None:
    _loaded_file = getattr(_loaded, "__file__", None)
    if _loaded_file is None or _source_root not in Path(_loaded_file).resolve().parents:
        raise RuntimeError(
            "A different rdna3_fastmm package is already loaded; restart ComfyUI after removing "
            "the conflicting installation"
        )

sys.path.insert(0, str(_source_root))
try:
    from rdna3_fastmm.comfyui import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS
finally:
    sys.path.remove(str(_source_root))

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
