"""ComfyUI node: compile a diffusion model with the ``rdna3-fastmm`` backend.

reference ``src/rdna3_fastmm/comfyui.py:76-119`` (and the custom-node entry
``__init__.py:1-26``, here the repository root's ``__init__.py``). The node
keeps the reference's class key ``RDNA3FastMMCompile``, so saved workflows
load unchanged. It clones the MODEL (dynamic shapes off) and asks ComfyUI's
``comfy_api.torch_helpers.set_torch_compile_wrapper`` (ComfyUI >= 0.19.0) to
wrap only ``diffusion_model`` with ``torch.compile`` on this package's Dynamo
backend. Guards on ComfyUI's per-call ``transformer_options`` are dropped,
as in the reference, so changing them does not recompile. The backend then
rewrites only the BF16 Linears in the MI355X dispatch table; everything else
compiles with standard Inductor.

The node refuses to run (``RuntimeError``, before cloning) when the runtime is
not the tested MI355X stack. There is no Python-version gate: this package
runs on Python 3.10+, unlike the reference's 3.12/3.13 requirement.
"""

from __future__ import annotations

from importlib import import_module
import logging
from typing import Any, Callable, Protocol, Sequence

BackendCompiler = Callable[..., object]
logger = logging.getLogger(__name__)


class ComfyModel(Protocol):
    def clone(self, disable_dynamic: bool = False) -> "ComfyModel": ...


class GuardEntry(Protocol):
    name: str


def skip_comfy_transformer_option_guards(guard_entries: Sequence[GuardEntry]) -> list[bool]:
    """Keep every Dynamo guard except those on ComfyUI's ``transformer_options``."""
    return ["transformer_options" not in entry.name for entry in guard_entries]


def _unsupported_reason() -> str | None:
    try:
        runtime = import_module("rdna3_fastmm.runtime")
    except ModuleNotFoundError as error:
        return f"missing Python dependency {error.name}"
    return runtime.unsupported_runtime_reason()


def _load_compile_backend() -> BackendCompiler:
    return import_module("rdna3_fastmm.inductor").compile_backend


def _load_compile_setter() -> Callable[..., None]:
    try:
        helpers = import_module("comfy_api.torch_helpers")
    except ModuleNotFoundError as error:
        if error.name is not None and error.name.startswith("comfy_api"):
            raise RuntimeError("RDNA3 FastMM requires ComfyUI 0.19.0 or newer") from error
        raise
    return helpers.set_torch_compile_wrapper


class RDNA3FastMMCompile:
    @classmethod
    def INPUT_TYPES(cls) -> dict[str, dict[str, tuple[str]]]:
        return {"required": {"model": ("MODEL",)}}

    RETURN_TYPES = ("MODEL",)
    RETURN_NAMES = ("model",)
    FUNCTION = "compile_model"
    CATEGORY = "model_patches/compile"
    DESCRIPTION = (
        "Compiles the diffusion model with FastMM on MI355X. BF16 Linear shapes with a "
        "measured win use reduced-multiplication HIP kernels; all other operations remain "
        "ordinary PyTorch Inductor operations."
    )
    EXPERIMENTAL = True

    def compile_model(self, model: ComfyModel) -> tuple[Any]:
        reason = _unsupported_reason()
        if reason is not None:
            raise RuntimeError(f"Cannot enable RDNA3 FastMM: {reason}")
        set_compile_wrapper = _load_compile_setter()
        backend = _load_compile_backend()
        compiled = model.clone(disable_dynamic=True)
        set_compile_wrapper(
            model=compiled,
            backend=backend,
            options={"guard_filter_fn": skip_comfy_transformer_option_guards},
            dynamic=False,
            keys=["diffusion_model"],
        )
        logger.info("Enabled RDNA3 FastMM for the ComfyUI diffusion model")
        return (compiled,)


NODE_CLASS_MAPPINGS = {"RDNA3FastMMCompile": RDNA3FastMMCompile}
NODE_DISPLAY_NAME_MAPPINGS = {"RDNA3FastMMCompile": "RDNA3 FastMM Compile"}
