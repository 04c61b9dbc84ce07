"""The deployment registry (deployment/registry.py) on the CPU: schema-3
documents, exact-match lookup by measurement identity and shape, and
publication that leaves the rest of the file as it was."""

from __future__ import annotations

import copy
import dataclasses
import json

import pytest

from deployment.environment import EnvironmentFingerprint
from deployment.registry import (
    DEFAULT_DEPLOYED_CONFIGS_PATH,
    RegistryIndex,
    ShapeFingerprint,
    iter_deployed_configs,
    publish_deployed_config,
    resolve_deployed_config,
)
from solution.config import ConfigSpec, hip_config

COMMITTED = json.loads(DEFAULT_DEPLOYED_CONFIGS_PATH.read_text(encoding="utf-8"))


def _hardware(**changes) -> EnvironmentFingerprint:
    raw = dict(COMMITTED["bundles"][0]["hardware"])
    raw.update(changes)
    return EnvironmentFingerprint.from_dict(raw)


SHAPE = ShapeFingerprint(4, 512, 8, 256, 2, True, 2048, "bfloat16", 0.0, 1.0)


def test_committed_registry_resolves_every_entry_it_holds():
    for bundle in COMMITTED["bundles"]:
        hardware = bundle["hardware"]
        pairs = iter_deployed_configs(hardware=hardware)
        assert [shape.to_dict() for shape, _ in pairs] == [e["shape"] for e in bundle["entries"]]
        for entry in bundle["entries"]:
            config = resolve_deployed_config(hardware=hardware, shape=entry["shape"])
            assert config == ConfigSpec.from_dict(entry["config"])


def test_shape_fingerprint_round_trips_and_requires_every_field():
    assert ShapeFingerprint.from_dict(SHAPE.to_dict()) == SHAPE
    assert list(SHAPE.to_dict()) == [f.name for f in dataclasses.fields(ShapeFingerprint)]
    partial = SHAPE.to_dict()
    del partial["ffn_dim"]
    with pytest.raises(KeyError):
        ShapeFingerprint.from_dict(partial)


def test_lookup_ignores_source_digests_but_not_the_device(tmp_path):
    path = tmp_path / "registry.json"
    publish_deployed_config(hardware=_hardware(), shape=SHAPE, config=hip_config(), path=path)
    # a code change (new implementation digest) keeps the entry resolvable
    edited = _hardware(solution_implementation_digest="0" * 64)
    assert resolve_deployed_config(hardware=edited, shape=SHAPE, path=path) == hip_config()
    # another device, another shape or a missing file resolve nothing
    other = _hardware(compute_capability="gfx942:sramecc+:xnack-")
    assert resolve_deployed_config(hardware=other, shape=SHAPE, path=path) is None
    wider = dataclasses.replace(SHAPE, batch_size=8)
    assert resolve_deployed_config(hardware=_hardware(), shape=wider, path=path) is None
    assert resolve_deployed_config(hardware=_hardware(), shape=SHAPE, path=tmp_path / "none.json") is None


def test_publish_replaces_in_place_and_keeps_other_bundles(tmp_path):
    path = tmp_path / "registry.json"
    document = copy.deepcopy(COMMITTED)
    foreign = {"hardware": dict(_hardware(compute_capability="gfx942").to_dict()), "entries": [{"junk": 1}]}
    document["bundles"].insert(0, foreign)
    path.write_text(json.dumps(document), encoding="utf-8")
    hardware = EnvironmentFingerprint.from_dict(COMMITTED["bundles"][1]["hardware"])
    existing = ShapeFingerprint.from_dict(COMMITTED["bundles"][1]["entries"][0]["shape"])
    count = len(COMMITTED["bundles"][1]["entries"])
    replacement = hip_config(microbatch_size=4) if existing.seq_len >= 32768 else hip_config()
    publish_deployed_config(hardware=hardware, shape=existing, config=replacement, path=path)
    written = json.loads(path.read_text(encoding="utf-8"))
    assert written["bundles"][0] == foreign  # untouched, unparsable entry included
    bundle = written["bundles"][2]
    assert len(bundle["entries"]) == count
    assert bundle["entries"][0] == {"shape": existing.to_dict(), "config": replacement.to_dict()}
    assert bundle["entries"][1:] == COMMITTED["bundles"][1]["entries"][1:]
    assert resolve_deployed_config(hardware=hardware, shape=existing, path=path) == replacement
    # a new shape is appended to the same bundle; a new device gets a new bundle
    publish_deployed_config(hardware=hardware, shape=SHAPE, config=hip_config(), path=path)
    assert len(json.loads(path.read_text())["bundles"][2]["entries"]) == count + 1
    other = _hardware(compute_capability="gfx951")
    publish_deployed_config(hardware=other, shape=SHAPE, config=hip_config(), path=path)
    final = json.loads(path.read_text())
    assert len(final["bundles"]) == len(document["bundles"]) + 1
    assert final["bundles"][-1]["hardware"] == other.to_dict()
    assert not list(tmp_path.glob("*.tmp"))


def test_first_bundle_of_an_identity_serves_it(tmp_path):
    path = tmp_path / "registry.json"
    hardware = _hardware()
    first = {"hardware": hardware.to_dict(), "entries": [{"shape": SHAPE.to_dict(), "config": hip_config().to_dict()}]}
    second = copy.deepcopy(first)
    second["entries"][0]["config"] = hip_config(microbatch_size=2).to_dict()
    path.write_text(json.dumps({"schema_version": 3, "bundles": [first, second]}), encoding="utf-8")
    assert resolve_deployed_config(hardware=hardware, shape=SHAPE, path=path) == hip_config()
    publish_deployed_config(hardware=hardware, shape=SHAPE, config=hip_config(microbatch_size=4), path=path)
    written = json.loads(path.read_text())
    assert written["bundles"][1] == second
    assert resolve_deployed_config(hardware=hardware, shape=SHAPE, path=path) == hip_config(microbatch_size=4)


def test_other_schema_versions_and_malformed_files(tmp_path):
    path = tmp_path / "registry.json"
    old = {"schema_version": 2, "bundles": [{"hardware": _hardware().to_dict(), "entries": [
        {"shape": SHAPE.to_dict(), "config": hip_config().to_dict()}]}]}
    path.write_text(json.dumps(old), encoding="utf-8")
    assert resolve_deployed_config(hardware=_hardware(), shape=SHAPE, path=path) is None
    # publishing over another schema starts a schema-3 document
    publish_deployed_config(hardware=_hardware(), shape=SHAPE, config=hip_config(), path=path)
    written = json.loads(path.read_text())
    assert written["schema_version"] == 3 and len(written["bundles"]) == 1
    path.write_text("[1, 2]", encoding="utf-8")
    with pytest.raises(ValueError):
        RegistryIndex.read(path)


def test_publish_keeps_the_file_mode(tmp_path):
    """The atomic rewrite keeps the replaced file's mode (mkstemp's 0600 would
    lock out readers under other uids); a new file gets 0666 less the umask."""

    import os
    import stat

    path = tmp_path / "registry.json"
    path.write_text(json.dumps(COMMITTED), encoding="utf-8")
    os.chmod(path, 0o644)
    publish_deployed_config(hardware=_hardware(), shape=SHAPE, config=hip_config(), path=path)
    assert stat.S_IMODE(path.stat().st_mode) == 0o644
    os.chmod(path, 0o664)
    publish_deployed_config(hardware=_hardware(), shape=SHAPE, config=hip_config(microbatch_size=2), path=path)
    assert stat.S_IMODE(path.stat().st_mode) == 0o664
    fresh = tmp_path / "fresh.json"
    umask = os.umask(0o022)
    try:
        publish_deployed_config(hardware=_hardware(), shape=SHAPE, config=hip_config(), path=fresh)
    finally:
        os.umask(umask)
    assert stat.S_IMODE(fresh.stat().st_mode) == 0o644


def test_driver_version_is_the_kernel_release_without_its_build_suffix():
    """Boxes of one pool run one amdgpu driver under kernel releases that
    differ only in the distribution's build suffix; the fingerprint keeps the
    upstream release, so a measurement published on one box serves the others."""

    from deployment.environment import kernel_driver_release

    assert kernel_driver_release("6.18.44-fc-v1045-amdproxy9") == "6.18.44"
    assert kernel_driver_release("6.18.44-fc-v595-amdproxy8") == "6.18.44"
    assert kernel_driver_release("6.8.0-45-generic") == "6.8.0"
    assert kernel_driver_release("6.10") == "6.10"
    assert kernel_driver_release("unknown") is None
    for bundle in COMMITTED["bundles"]:
        assert bundle["hardware"]["driver_version"] == kernel_driver_release(bundle["hardware"]["driver_version"])
