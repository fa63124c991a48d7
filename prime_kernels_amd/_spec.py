"""Parser for kernels.toml (reference: prime_kernels/_spec.py:1-96, re-targeted to AMD gfx ids)."""

from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import Path

try:  # Python >= 3.11
    import tomllib as _toml
except ModuleNotFoundError:  # this image runs Python 3.10; tomli is the same parser
    import tomli as _toml

MANIFEST = "kernels.toml"

_ARCH = re.compile(r"^gfx(\d+)([a-f0-9]*)$")


@dataclass(frozen=True)
class Arch:
    """An AMD GPU architecture a kernel is compiled for, e.g. `gfx950` (MI355X)."""

    name: str

    @classmethod
    def parse(cls, raw: str) -> "Arch":
        if not _ARCH.match(raw):
            raise ValueError(f"invalid arch {raw!r}, expected e.g. 'gfx950'")
        return cls(raw)

    def offload_flag(self) -> str:
        return f"--offload-arch={self.name}"

    def matches(self, gcn_arch_name: str) -> bool:
        # torch reports e.g. "gfx950:sramecc+:xnack-"; the base id must match exactly
        return gcn_arch_name.split(":")[0] == self.name

    def __str__(self) -> str:
        return self.name


@dataclass(frozen=True)
class KernelSpec:
    """Everything needed to build one kernel and to decide whether it can run here."""

    name: str
    path: Path
    description: str
    ops: str
    sources: tuple[Path, ...]
    library: str
    archs: tuple[Arch, ...]
    requires: tuple[str, ...]

    @property
    def module(self) -> str:
        return f"prime_kernels_amd.{self.name}"

    @property
    def arch_list(self) -> str:
        return ", ".join(str(a) for a in self.archs)

    def supports(self, gcn_arch_name: str) -> bool:
        return any(a.matches(gcn_arch_name) for a in self.archs)


def load(package_dir: Path) -> dict[str, KernelSpec]:
    """Parse kernels.toml into one spec per kernel, in manifest order."""
    package_dir = package_dir.resolve()
    manifest = _toml.loads((package_dir / MANIFEST).read_text())
    return {name: _kernel(name, package_dir, table) for name, table in manifest.items()}


def _kernel(name: str, package_dir: Path, table: dict) -> KernelSpec:
    return KernelSpec(
        name=name,
        path=package_dir / name,
        description=table["description"],
        ops=table.get("ops", ""),
        sources=tuple(package_dir / "csrc" / s for s in table.get("sources", [])),
        library=table.get("library", ""),
        archs=tuple(Arch.parse(a) for a in table["arch"]),
        requires=tuple(table.get("requires", [])),
    )
