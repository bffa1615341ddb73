"""ComfyUI node and custom-node entry (reference tests/test_comfyui.py), CPU only.

ComfyUI itself is not installed here: its compile helper is replaced by a
recording fake, as in the reference's tests.
"""

from __future__ import annotations

from pathlib import Path
import subprocess
import sys
from types import ModuleType

import pytest

from rdna3_fastmm import comfyui

REPO_ROOT = Path(__file__).resolve().parent.parent


class FakeGuard:
    def __init__(self, name: str) -> None:
        self.name = name


class FakeModel:
    def __init__(self) -> None:
        self.clone_arguments: list[bool] = []

    def clone(self, disable_dynamic: bool = False) -> "FakeModel":
        self.clone_arguments.append(disable_dynamic)
        return FakeModel()


def test_guard_filter_drops_only_transformer_options() -> None:
    guards = [FakeGuard("model.model_options['transformer_options']"), FakeGuard("model.model_options['x']"),
              FakeGuard("input")]
    assert comfyui.skip_comfy_transformer_option_guards(guards) == [False, True, True]


def test_node_clones_and_wraps_only_the_diffusion_model(monkeypatch) -> None:
    captured = {}

    def backend(*args, **kwargs):
        return object()

    def set_wrapper(**kwargs):
        captured.update(kwargs)

    monkeypatch.setattr(comfyui, "toolchain", lambda: comfyui.Toolchain(set_wrapper, backend))
    source = FakeModel()
    (compiled,) = comfyui.RDNA3FastMMCompile().compile_model(source)
    assert compiled is captured["model"] and compiled is not source
    assert source.clone_arguments == [True]
    assert captured["backend"] is backend
    assert captured["keys"] == ["diffusion_model"] and captured["dynamic"] is False
    assert captured["options"] == {"guard_filter_fn": comfyui.skip_comfy_transformer_option_guards}


def test_node_rejects_an_unsupported_runtime_before_cloning(monkeypatch) -> None:
    source = FakeModel()
    monkeypatch.setattr(comfyui, "_runtime_problem", lambda: "unsupported test runtime")
    with pytest.raises(RuntimeError, match="Cannot enable RDNA3 FastMM: unsupported test runtime"):
        comfyui.RDNA3FastMMCompile().compile_model(source)
    assert source.clone_arguments == []


def test_runtime_problem_is_the_runtime_gate() -> None:
    # the runtime gate's reason (None on the tested MI355X stack) comes through unchanged
    from rdna3_fastmm.runtime import unsupported_runtime_reason

    assert comfyui._runtime_problem() == unsupported_runtime_reason()


def test_toolchain_requires_current_comfyui(monkeypatch) -> None:
    def missing(name: str) -> ModuleType:
        raise ModuleNotFoundError(f"No module named {name!r}", name=name)

    monkeypatch.setattr(comfyui, "_runtime_problem", lambda: None)
    monkeypatch.setattr(comfyui.importlib, "import_module", missing)
    with pytest.raises(RuntimeError, match="requires ComfyUI 0.19.0 or newer"):
        comfyui.toolchain()


def test_toolchain_uses_comfyuis_helper_and_the_backend(monkeypatch) -> None:
    helpers = ModuleType("comfy_api.torch_helpers")
    helpers.set_torch_compile_wrapper = lambda **kwargs: None
    monkeypatch.setitem(sys.modules, "comfy_api", ModuleType("comfy_api"))
    monkeypatch.setitem(sys.modules, "comfy_api.torch_helpers", helpers)
    monkeypatch.setattr(comfyui, "_runtime_problem", lambda: None)
    tools = comfyui.toolchain()
    assert tools.wrap_model is helpers.set_torch_compile_wrapper
    assert tools.backend.__name__ == "compile_backend"


def test_node_contract_is_exported() -> None:
    node = comfyui.RDNA3FastMMCompile
    assert node.INPUT_TYPES() == {"required": {"model": ("MODEL",)}}
    assert (node.RETURN_TYPES, node.FUNCTION, node.EXPERIMENTAL) == (("MODEL",), "compile_model", True)
    assert comfyui.NODE_CLASS_MAPPINGS == {"RDNA3FastMMCompile": node}
    assert comfyui.NODE_DISPLAY_NAME_MAPPINGS == {"RDNA3FastMMCompile": "RDNA3 FastMM Compile"}


def _run_entry(code: str) -> subprocess.CompletedProcess:
    """Import the repository as a ComfyUI custom node does, in a fresh interpreter."""
    script = (
        "import importlib.util, sys\n"
        f"spec = importlib.util.spec_from_file_location('fastmm_node', {str(REPO_ROOT / '__init__.py')!r}, "
        f"submodule_search_locations=[{str(REPO_ROOT)!r}])\n"
        "module = importlib.util.module_from_spec(spec)\n" + code
    )
    return subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)


def test_custom_node_entry_exports_the_mappings() -> None:
    result = _run_entry(
        "spec.loader.exec_module(module)\n"
        "import rdna3_fastmm.comfyui as c\n"
        "assert module.NODE_CLASS_MAPPINGS is c.NODE_CLASS_MAPPINGS\n"
        f"assert {str(REPO_ROOT / 'rdna3-fastmm_amd')!r} not in sys.path\n"
        "print('ok')\n"
    )
    assert result.returncode == 0 and result.stdout.strip() == "ok", result.stderr


def test_custom_node_entry_refuses_another_loaded_package(tmp_path) -> None:
    stale = tmp_path / "rdna3_fastmm"
    stale.mkdir()
    (stale / "__init__.py").write_text("SOURCE = 'stale install'\n")
    result = _run_entry(
        f"sys.path.insert(0, {str(tmp_path)!r})\n"
        "import rdna3_fastmm\n"
        "try:\n"
        "    spec.loader.exec_module(module)\n"
        "except RuntimeError as error:\n"
        "    print(error)\n"
    )
    assert "A different rdna3_fastmm package is already loaded" in result.stdout, result.stderr


def test_package_metadata_ships_the_node_data() -> None:
    import tomli

    pyproject = tomli.loads((REPO_ROOT / "pyproject.toml").read_text())
    assert pyproject["tool"]["comfy"]["requires-comfyui"] == ">=0.19.0"
    data = pyproject["tool"]["setuptools"]["package-data"]["rdna3_fastmm"]
    assert {"corpora/*.json", "dispatch/*.json"} <= set(data)
