"""ComfyUI custom node that compiles a diffusion model with the ``rdna3-fastmm`` backend.

Counterpart of the reference's node (``src/rdna3_fastmm/comfyui.py:76-119``;
custom-node entry ``__init__.py:1-26``, here the repository root's
``__init__.py``). Saved workflows reference a node by its class key, so the
key ``RDNA3FastMMCompile``, its single MODEL input and output, and the two
refusal messages stay as the reference has them; the rest is this package's.

What the node does to a MODEL: it resolves its toolchain first (the MI355X
runtime gate, ComfyUI's ``comfy_api.torch_helpers.set_torch_compile_wrapper``
from ComfyUI 0.19.0 on, and this package's Dynamo backend) and refuses with a
``RuntimeError`` before touching the model if any part is missing. It then
patches a clone of the model (dynamic shapes off) so that only the
``diffusion_model`` submodule is compiled with the backend, which rewrites
just the BF16 Linears in the MI355X dispatch table and leaves the rest to
standard Inductor. ComfyUI hands every call a new ``transformer_options``
dict; guards on it are dropped so that does not force recompiles.
"""

from __future__ import annotations

import importlib
import logging
from typing import Any, Callable, NamedTuple, Sequence

NODE_KEY = "RDNA3FastMMCompile"
COMPILED_SUBMODULES = ("diffusion_model",)
MINIMUM_COMFYUI = "0.19.0"
_LOG = logging.getLogger(__name__)


def skip_comfy_transformer_option_guards(guards: Sequence[Any]) -> list[bool]:
    """Dynamo guard filter (True keeps a guard): every guard except those on the
    per-call ``transformer_options`` dict ComfyUI passes to the model."""
    return ["transformer_options" not in str(getattr(guard, "name", "")) for guard in guards]


class Toolchain(NamedTuple):
    """What compiling needs from the environment."""

    wrap_model: Callable[..., None]  # ComfyUI's set_torch_compile_wrapper
    backend: Callable[..., object]  # rdna3_fastmm.inductor.compile_backend


def _runtime_problem() -> str | None:
    """Why this machine is not the tested MI355X stack (None when it is)."""
    try:
        from .runtime import unsupported_runtime_reason
    except ModuleNotFoundError as error:  # e.g. torch absent from ComfyUI's environment
        return f"missing Python dependency {error.name}"
    return unsupported_runtime_reason()


def toolchain() -> Toolchain:
    """Resolve the node's dependencies, or raise RuntimeError naming the missing one."""
    problem = _runtime_problem()
    if problem is not None:
        raise RuntimeError(f"Cannot enable RDNA3 FastMM: {problem}")
    try:
        helpers = importlib.import_module("comfy_api.torch_helpers")
    except ModuleNotFoundError as error:
        if (error.name or "").startswith("comfy_api"):
            raise RuntimeError(f"RDNA3 FastMM requires ComfyUI {MINIMUM_COMFYUI} or newer") from error
        raise
    backend = importlib.import_module(f"{__package__}.inductor").compile_backend
    return Toolchain(wrap_model=helpers.set_torch_compile_wrapper, backend=backend)


class RDNA3FastMMCompile:
    """MODEL -> MODEL whose diffusion model runs through the FastMM Linear rewrite."""

    RETURN_TYPES = ("MODEL",)
    RETURN_NAMES = ("model",)
    FUNCTION = "compile_model"
    CATEGORY = "model_patches/compile"
    EXPERIMENTAL = True
    DESCRIPTION = (
        "Compiles the diffusion model with FastMM on MI355X: BF16 Linear shapes with a measured "
        "win run reduced-multiplication HIP kernels, everything else stays ordinary Inductor code."
    )

    @classmethod
    def INPUT_TYPES(cls) -> dict[str, dict[str, tuple[str]]]:
        return {"required": {"model": ("MODEL",)}}

    def compile_model(self, model: Any) -> tuple[Any]:
        tools = toolchain()  # refuse before cloning anything
        patched = model.clone(disable_dynamic=True)
        tools.wrap_model(
            model=patched,
            backend=tools.backend,
            options={"guard_filter_fn": skip_comfy_transformer_option_guards},
            dynamic=False,
            keys=list(COMPILED_SUBMODULES),
        )
        _LOG.info("rdna3-fastmm: %s compiled with the FastMM backend", ", ".join(COMPILED_SUBMODULES))
        return (patched,)


NODE_CLASS_MAPPINGS = {NODE_KEY: RDNA3FastMMCompile}
NODE_DISPLAY_NAME_MAPPINGS = {NODE_KEY: "RDNA3 FastMM Compile"}
