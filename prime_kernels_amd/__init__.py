"""prime_kernels_amd: MI355X (gfx950) build of the prime-kernels SmolLM2 decode path.

Registry surface mirrors the reference's prime_kernels/__init__.py:23-78 (`KERNELS`, `spec`,
`is_built`, `unavailable_reason`, `is_available`, `load`, `status`); availability is decided by
"library built?", then "requirements importable?", then "device is gfx950?".
"""

from __future__ import annotations

import importlib
import importlib.util
from pathlib import Path
from types import ModuleType

from prime_kernels_amd._spec import Arch, KernelSpec
from prime_kernels_amd._spec import load as _load_manifest

__all__ = ["Arch", "KernelSpec", "KERNELS", "is_available", "is_built", "load", "spec", "status",
           "unavailable_reason"]

_SPECS: dict[str, KernelSpec] = _load_manifest(Path(__file__).parent)
_LOADED_MODULES: dict[str, ModuleType] = {}

KERNELS: tuple[str, ...] = tuple(_SPECS)
LIB_DIR = Path(__file__).resolve().parent / "_lib"


def spec(name: str) -> KernelSpec:
    if name not in _SPECS:
        raise KeyError(f"unknown kernel {name!r}, have {', '.join(KERNELS) or '<none>'}")
    return _SPECS[name]


def is_built(name: str) -> bool:
    kernel = spec(name)
    return (kernel.path / "__init__.py").is_file() and (LIB_DIR / kernel.library).is_file()


def unavailable_reason(name: str, device: int | None = None) -> str | None:
    import torch

    kernel = spec(name)
    if not is_built(name):
        return f"{name} was not compiled into this install of prime_kernels_amd (run __graft_entry__.build())"
    missing = [r for r in kernel.requires if importlib.util.find_spec(r) is None]
    if missing:
        return f"{name} requires {', '.join(missing)}, which is not installed"
    if not torch.cuda.is_available():
        return f"{name} requires a HIP device ({kernel.arch_list}), none is available"
    arch = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device()).gcnArchName
    if not kernel.supports(arch):
        return f"{name} requires {kernel.arch_list}, this device is {arch}"
    return None


def is_available(name: str, device: int | None = None) -> bool:
    return unavailable_reason(name, device) is None


def load(name: str, device: int | None = None) -> ModuleType:
    try:
        return _LOADED_MODULES[name]
    except KeyError:
        pass
    reason = unavailable_reason(name, device)
    if reason is not None:
        raise RuntimeError(reason)
    module = importlib.import_module(spec(name).module)
    _LOADED_MODULES[name] = module
    return module


def status(device: int | None = None) -> dict[str, str]:
    return {name: unavailable_reason(name, device) or "available" for name in KERNELS}
