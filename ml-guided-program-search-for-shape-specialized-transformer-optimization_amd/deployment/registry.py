"""Exact-match registry of measured configurations.

The file keeps the reference's schema-3 document (deployment/registry.py:17,
:20-81 for the shape key): ``{"schema_version": 3, "bundles": [{"hardware":
<EnvironmentFingerprint>, "entries": [{"shape": <ShapeFingerprint>,
"config": <ConfigSpec>}]}]}``, so a registry written by either side reads on
the other.  Lookup semantics are the reference's: a bundle serves the running
environment when its fingerprint's ``measurement_identity`` equals the
environment's (the first such bundle wins), and an entry serves a model when
its shape fingerprint is equal field for field.

This module reads a document once into :class:`RegistryIndex`, a map from
``(measurement_identity, ShapeFingerprint)`` to the stored config, and
serves every query from that map.  Publishing edits the one bundle it
touches and writes the whole document back atomically; bundles of other
environments, and entries this code cannot parse, are written back as they
were read.
"""

from __future__ import annotations

import json
import os
import stat
import tempfile
from dataclasses import astuple, dataclass, fields
from pathlib import Path
from typing import Any, Iterator

from solution.config import ConfigSpec

from .environment import EnvironmentFingerprint

DEFAULT_DEPLOYED_CONFIGS_PATH = Path(__file__).resolve().parent / "deployed_configs.json"
DEPLOYMENT_SCHEMA_VERSION = 3


@dataclass(frozen=True, slots=True)
class ShapeFingerprint:
    """The workload a registry entry was measured on (schema-3 field names)."""

    batch_size: int
    qkv_dim: int
    heads: int
    seq_len: int
    layers: int
    causal: bool
    ffn_dim: int
    dtype: str
    padding_ratio: float
    input_scale: float

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> ShapeFingerprint:
        # Each field is coerced by its annotated type; a missing field raises
        # KeyError, as an incomplete key must never match.
        coerce = {"int": int, "bool": bool, "str": str, "float": float}
        return cls(**{f.name: coerce[f.type](value[f.name]) for f in fields(cls)})

    def to_dict(self) -> dict[str, Any]:
        return dict(zip((f.name for f in fields(self)), astuple(self)))


def _parse_shape(raw: Any) -> ShapeFingerprint | None:
    if not isinstance(raw, dict):
        return None
    try:
        return ShapeFingerprint.from_dict(raw)
    except (KeyError, TypeError, ValueError):
        return None


def _parse_identity(raw: Any) -> str | None:
    if not isinstance(raw, dict):
        return None
    try:
        return EnvironmentFingerprint.from_dict(raw).measurement_identity
    except (KeyError, TypeError, ValueError):
        return None


class RegistryIndex:
    """One registry document and its ``(identity, shape) -> config`` index."""

    def __init__(self, document: dict[str, Any] | None = None) -> None:
        usable = (
            isinstance(document, dict)
            and document.get("schema_version") == DEPLOYMENT_SCHEMA_VERSION
            and isinstance(document.get("bundles"), list)
        )
        self.document: dict[str, Any] = (
            document if usable else {"schema_version": DEPLOYMENT_SCHEMA_VERSION, "bundles": []}
        )
        # identity -> the bundle that serves it (the first one in the file)
        self._bundles: dict[str, dict[str, Any]] = {}
        # (identity, shape) -> raw config of the first entry for that shape
        self._configs: dict[tuple[str, ShapeFingerprint], dict[str, Any]] = {}
        for bundle in self.document["bundles"]:
            identity = _parse_identity(bundle.get("hardware")) if isinstance(bundle, dict) else None
            if identity is None or identity in self._bundles:
                continue
            self._bundles[identity] = bundle
            self._index_bundle(identity, bundle)

    def _index_bundle(self, identity: str, bundle: dict[str, Any]) -> None:
        entries = bundle.get("entries")
        for entry in entries if isinstance(entries, list) else ():
            if not isinstance(entry, dict) or not isinstance(entry.get("config"), dict):
                continue
            shape = _parse_shape(entry.get("shape"))
            if shape is not None:
                self._configs.setdefault((identity, shape), entry["config"])

    @classmethod
    def read(cls, path: str | Path) -> RegistryIndex:
        """The registry at ``path``; empty when the file does not exist or
        holds another schema version.  A file that is not a JSON object with a
        ``bundles`` array is an error."""

        try:
            text = Path(path).read_text(encoding="utf-8")
        except FileNotFoundError:
            return cls()
        document = json.loads(text)
        if not isinstance(document, dict) or not isinstance(document.get("bundles"), list):
            raise ValueError(f"{path}: a deployed-config file must hold a bundles array")
        return cls(document)

    def lookup(self, identity: str, shape: ShapeFingerprint) -> ConfigSpec | None:
        raw = self._configs.get((identity, shape))
        return None if raw is None else ConfigSpec.from_dict(raw)

    def items(self, identity: str) -> Iterator[tuple[ShapeFingerprint, ConfigSpec]]:
        for (owner, shape), raw in self._configs.items():
            if owner == identity:
                yield shape, ConfigSpec.from_dict(raw)

    def put(self, hardware: EnvironmentFingerprint, shape: ShapeFingerprint, config: ConfigSpec) -> None:
        """Record ``config`` for ``shape`` under ``hardware``'s bundle: the
        bundle's fingerprint becomes ``hardware``'s, and the entry for an equal
        shape is replaced in place (appended when there is none)."""

        identity = hardware.measurement_identity
        bundle = self._bundles.get(identity)
        if bundle is None:
            bundle = {"hardware": None, "entries": []}
            self.document["bundles"].append(bundle)
            self._bundles[identity] = bundle
        bundle["hardware"] = hardware.to_dict()
        if not isinstance(bundle.get("entries"), list):
            bundle["entries"] = []
        new_entry = {"shape": shape.to_dict(), "config": config.to_dict()}
        entries = bundle["entries"]
        slot = next(
            (i for i, entry in enumerate(entries) if isinstance(entry, dict) and _parse_shape(entry.get("shape")) == shape),
            None,
        )
        if slot is None:
            entries.append(new_entry)
        else:
            entries[slot] = new_entry
        self._configs[(identity, shape)] = new_entry["config"]

    def write(self, path: str | Path) -> Path:
        """Write the document to ``path`` through a temporary file in the same
        directory, so a reader sees the old file or the new one, never a part."""

        target = Path(path)
        target.parent.mkdir(parents=True, exist_ok=True)
        text = json.dumps(self.document, ensure_ascii=False, indent=2, allow_nan=False) + "\n"
        handle, temporary = tempfile.mkstemp(prefix=target.name + ".", suffix=".tmp", dir=target.parent)
        try:
            with os.fdopen(handle, "w", encoding="utf-8") as stream:
                stream.write(text)
            # mkstemp creates the file 0600; the published file keeps the
            # mode of the one it replaces, or a new file's default (0666 less
            # the umask), so readers under other uids still read it.
            os.chmod(temporary, _published_mode(target))
            os.replace(temporary, target)
        except BaseException:
            Path(temporary).unlink(missing_ok=True)
            raise
        return target


def _process_umask() -> int:
    # Read from /proc where it exists: setting and restoring os.umask would
    # briefly change it for every thread of the process.
    try:
        for line in Path("/proc/self/status").read_text(encoding="ascii").splitlines():
            if line.startswith("Umask:"):
                return int(line.split()[1], 8)
    except (OSError, ValueError):
        pass
    umask = os.umask(0o022)
    os.umask(umask)
    return umask


def _published_mode(target: Path) -> int:
    try:
        return stat.S_IMODE(target.stat().st_mode)
    except FileNotFoundError:
        return 0o666 & ~_process_umask()


def _fingerprint(hardware: EnvironmentFingerprint | dict[str, Any]) -> EnvironmentFingerprint:
    if isinstance(hardware, EnvironmentFingerprint):
        return hardware
    return EnvironmentFingerprint.from_dict(hardware)


def _shape(shape: ShapeFingerprint | dict[str, Any]) -> ShapeFingerprint:
    return shape if isinstance(shape, ShapeFingerprint) else ShapeFingerprint.from_dict(shape)


def resolve_deployed_config(
    *,
    hardware: EnvironmentFingerprint | dict[str, Any],
    shape: ShapeFingerprint | dict[str, Any],
    path: str | Path | None = None,
) -> ConfigSpec | None:
    """The config measured for exactly this environment and shape, or None.
    ``path`` defaults to DEFAULT_DEPLOYED_CONFIGS_PATH, read at call time."""

    registry = RegistryIndex.read(DEFAULT_DEPLOYED_CONFIGS_PATH if path is None else path)
    return registry.lookup(_fingerprint(hardware).measurement_identity, _shape(shape))


def iter_deployed_configs(
    *,
    hardware: EnvironmentFingerprint | dict[str, Any],
    path: str | Path = DEFAULT_DEPLOYED_CONFIGS_PATH,
) -> tuple[tuple[ShapeFingerprint, ConfigSpec], ...]:
    """Every (shape, config) published for this environment, in file order."""

    return tuple(RegistryIndex.read(path).items(_fingerprint(hardware).measurement_identity))


def publish_deployed_config(
    *,
    hardware: EnvironmentFingerprint | dict[str, Any],
    shape: ShapeFingerprint | dict[str, Any],
    config: ConfigSpec,
    path: str | Path = DEFAULT_DEPLOYED_CONFIGS_PATH,
) -> Path:
    """Insert or replace one exact winner and rewrite the file atomically."""

    registry = RegistryIndex.read(path)
    registry.put(_fingerprint(hardware), _shape(shape), config)
    return registry.write(path)


__all__ = [
    "DEFAULT_DEPLOYED_CONFIGS_PATH",
    "DEPLOYMENT_SCHEMA_VERSION",
    "RegistryIndex",
    "ShapeFingerprint",
    "iter_deployed_configs",
    "publish_deployed_config",
    "resolve_deployed_config",
]
