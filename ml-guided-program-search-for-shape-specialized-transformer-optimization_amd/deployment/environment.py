"""Stable identity of the environment a deployed config was measured in.

Keeps the reference's fingerprint record (deployment/environment.py:150-296):
the same JSON field names, the canonical SHA-256 ``identity`` and the
``measurement_identity`` that ignores the source digests.  The facts behind
the fields are ROCm's instead of CUDA's:

  compute_capability    gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  driver_version        amdgpu kernel driver: the module's own version where
                        amdgpu is a loadable module (/sys/module/amdgpu/
                        version, e.g. a DKMS build), else the upstream release
                        of the kernel that carries it (the leading
                        major.minor.patch that ROCm SMI or uname reports),
                        replacing the nvidia-smi probe of the reference
                        (:99-124)
  cuda_runtime_version  torch.version.hip (the HIP runtime torch ships)
  cudnn_version         MIOpen version as torch reports it
"""

from __future__ import annotations

import hashlib
import importlib.metadata
import json
import platform
import re
import subprocess
from dataclasses import dataclass
from enum import Enum
from pathlib import Path
from typing import Any

import torch

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
_OFFICIAL_DEFINITION_PATHS = (
    Path("official/test_shapes.json"),
    Path("official/torch_transformer_benchmark.py"),
)
_IMPLEMENTATION_SUFFIXES = {".py", ".hip", ".hpp", ".h"}


class ImplementationScope(str, Enum):
    """Independent resident and long-sequence (streamed) lifecycles."""

    RESIDENT = "resident"
    SHAPE14 = "shape14"

    def __str__(self) -> str:
        return str(self.value)


def _stable_json(value: object) -> bytes:
    return json.dumps(
        value, ensure_ascii=False, sort_keys=True, separators=(",", ":"), allow_nan=False
    ).encode("utf-8")


def stable_digest(value: object) -> str:
    return hashlib.sha256(_stable_json(value)).hexdigest()


def _files_digest(root: Path, relative_paths: list[Path]) -> str:
    records = [
        {"path": path.as_posix(), "sha256": hashlib.sha256((root / path).read_bytes()).hexdigest()}
        for path in sorted(relative_paths, key=lambda item: item.as_posix())
    ]
    return stable_digest(records)


def official_definitions_digest(project_root: Path = PACKAGE_ROOT) -> str:
    """Digest of the official benchmark definitions when they are installed
    next to the solution (the reference's layout); "not-available" otherwise."""

    present = [path for path in _OFFICIAL_DEFINITION_PATHS if (project_root / path).exists()]
    if not present:
        return "not-available"
    return _files_digest(project_root, present)


def _scope_of(relative: Path) -> ImplementationScope | None:
    parts = relative.parts
    if len(parts) >= 2 and parts[0] == "solution" and parts[1] == "shape14":
        return ImplementationScope.SHAPE14
    if parts and parts[0] == "csrc":
        return None  # kernels serve both scopes
    if len(parts) >= 2 and parts[0] == "solution" and parts[1] == "kernels":
        return None
    return None


def solution_implementation_digest(
    project_root: Path = PACKAGE_ROOT,
    *,
    scope: ImplementationScope = ImplementationScope.RESIDENT,
) -> str:
    """Digest of the Python plan code and HIP sources serving ``scope``."""

    root = Path(project_root)
    wanted = ImplementationScope(scope)
    paths = [
        path.relative_to(root)
        for folder in ("solution", "csrc")
        for path in (root / folder).rglob("*")
        if path.is_file()
        and path.suffix in _IMPLEMENTATION_SUFFIXES
        and "_build" not in path.parts
        and _scope_of(path.relative_to(root)) in {None, wanted}
    ]
    if not paths:
        raise FileNotFoundError(f"no implementation files under {root}")
    return _files_digest(root, paths)


_KERNEL_RELEASE = re.compile(r"^(\d+\.\d+(?:\.\d+)?)")


def kernel_driver_release(release: str) -> str | None:
    """The upstream part of a kernel release string ("6.18.44" of
    "6.18.44-fc-v1045-amdproxy9"), or None when it does not start with one.
    The suffix names the distribution's build of the host kernel; machines of
    one pool run the same driver under different suffixes."""

    match = _KERNEL_RELEASE.match(release.strip())
    return match.group(1) if match else None


def amdgpu_driver_version() -> str:
    """Version of the amdgpu kernel driver: the loadable module's version
    when sysfs has it, else the upstream release of the kernel the driver is
    built into (as ROCm SMI reports it on such systems, or uname)."""

    sysfs = Path("/sys/module/amdgpu/version")
    try:
        text = sysfs.read_text(encoding="utf-8").strip()
        if text:
            return text
    except OSError:
        pass
    reported: str | None = None
    try:
        completed = subprocess.run(
            ["rocm-smi", "--showdriverversion", "--json"],
            check=True, capture_output=True, text=True, timeout=20,
        )
        document = json.loads(completed.stdout)
        for value in document.values():
            if isinstance(value, dict):
                for key, item in value.items():
                    if "driver" in key.lower():
                        reported = str(item)
                        break
            if reported is not None:
                break
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    for candidate in (reported, platform.release()):
        if candidate:
            return kernel_driver_release(candidate) or candidate
    raise RuntimeError("cannot determine the amdgpu driver version")


def installed_triton_version() -> str:
    for distribution in ("triton", "pytorch-triton-rocm", "triton-windows"):
        try:
            return importlib.metadata.version(distribution)
        except importlib.metadata.PackageNotFoundError:
            continue
    return "not-installed"


def _required_string(value: Any, name: str) -> str:
    if not isinstance(value, str) or not value:
        raise ValueError(f"environment fingerprint field {name!r} must be a string")
    return value


def configure_process_math_mode() -> None:
    """Full-precision accumulation for 16-bit matrix reductions (reference :144-147)."""

    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False


@dataclass(frozen=True, slots=True)
class EnvironmentFingerprint:
    device_name: str
    compute_capability: str
    driver_version: str
    torch_version: str
    cuda_runtime_version: str
    cudnn_version: str
    triton_version: str
    matmul_precision: str
    allow_tf32: bool
    allow_fp16_reduced_precision_reduction: bool
    cudnn_allow_tf32: bool | None
    official_definitions_digest: str
    solution_implementation_digest: str
    scope: ImplementationScope = ImplementationScope.RESIDENT

    @classmethod
    def detect(
        cls,
        device: str | torch.device,
        *,
        project_root: Path = PACKAGE_ROOT,
        scope: ImplementationScope = ImplementationScope.RESIDENT,
    ) -> EnvironmentFingerprint:
        resolved = torch.device(device)
        if resolved.type != "cuda" or not torch.cuda.is_available():
            raise ValueError("environment fingerprint detection requires a GPU")
        if torch.version.hip is None:
            raise RuntimeError("the ROCm fingerprint requires a ROCm build of torch")
        index = torch.cuda.current_device() if resolved.index is None else resolved.index
        properties = torch.cuda.get_device_properties(index)
        miopen = torch.backends.cudnn.version()
        return cls(
            device_name=torch.cuda.get_device_name(index),
            compute_capability=str(getattr(properties, "gcnArchName", "unknown")),
            driver_version=amdgpu_driver_version(),
            torch_version=str(torch.__version__),
            cuda_runtime_version=str(torch.version.hip),
            cudnn_version="not-available" if miopen is None else str(miopen),
            triton_version=installed_triton_version(),
            matmul_precision=str(torch.get_float32_matmul_precision()),
            allow_tf32=bool(torch.backends.cuda.matmul.allow_tf32),
            allow_fp16_reduced_precision_reduction=bool(
                torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction
            ),
            cudnn_allow_tf32=getattr(torch.backends.cudnn, "allow_tf32", None),
            official_definitions_digest=official_definitions_digest(project_root),
            solution_implementation_digest=solution_implementation_digest(project_root, scope=scope),
            scope=ImplementationScope(scope),
        )

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> EnvironmentFingerprint:
        for name in ("allow_tf32", "allow_fp16_reduced_precision_reduction"):
            if not isinstance(value[name], bool):
                raise TypeError(f"environment fingerprint field {name!r} must be boolean")
        if value["cudnn_allow_tf32"] is not None and not isinstance(value["cudnn_allow_tf32"], bool):
            raise TypeError("environment fingerprint field 'cudnn_allow_tf32' must be boolean or null")
        strings = {
            name: _required_string(value[name], name)
            for name in (
                "device_name", "compute_capability", "driver_version", "torch_version",
                "cuda_runtime_version", "cudnn_version", "triton_version", "matmul_precision",
                "official_definitions_digest", "solution_implementation_digest",
            )
        }
        return cls(
            **strings,
            allow_tf32=value["allow_tf32"],
            allow_fp16_reduced_precision_reduction=value["allow_fp16_reduced_precision_reduction"],
            cudnn_allow_tf32=value["cudnn_allow_tf32"],
            scope=ImplementationScope(_required_string(value["scope"], "scope")),
        )

    def to_dict(self) -> dict[str, str | bool | None]:
        return {
            "scope": self.scope.value,
            "device_name": self.device_name,
            "compute_capability": self.compute_capability,
            "driver_version": self.driver_version,
            "torch_version": self.torch_version,
            "cuda_runtime_version": self.cuda_runtime_version,
            "cudnn_version": self.cudnn_version,
            "triton_version": self.triton_version,
            "matmul_precision": self.matmul_precision,
            "allow_tf32": self.allow_tf32,
            "allow_fp16_reduced_precision_reduction": self.allow_fp16_reduced_precision_reduction,
            "cudnn_allow_tf32": self.cudnn_allow_tf32,
            "official_definitions_digest": self.official_definitions_digest,
            "solution_implementation_digest": self.solution_implementation_digest,
        }

    @property
    def identity(self) -> str:
        return stable_digest(self.to_dict())

    @property
    def measurement_identity(self) -> str:
        value = self.to_dict()
        value.pop("official_definitions_digest")
        value.pop("solution_implementation_digest")
        return stable_digest(value)


__all__ = [
    "EnvironmentFingerprint",
    "ImplementationScope",
    "amdgpu_driver_version",
    "configure_process_math_mode",
    "installed_triton_version",
    "kernel_driver_release",
    "official_definitions_digest",
    "solution_implementation_digest",
    "stable_digest",
]
