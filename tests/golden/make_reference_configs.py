"""Extract the reference's deployed configs and published config ids as data.

Reads (as JSON data, no code) the reference's deployment registry
(deployment/deployed_configs.json) and the final report that lists the
config id of every official shape
(result/20260831T083857.848038Z/final_performance.json), and writes
reference_configs.json: one record per official shape with the shape
fingerprint, the full ConfigSpec document and the published config_id.

Run once in a container where the reference is mounted:
    python tests/golden/make_reference_configs.py /root/reference
"""

from __future__ import annotations

import json
import sys
from pathlib import Path


def main(reference_root: str) -> None:
    root = Path(reference_root)
    registry = json.loads((root / "deployment/deployed_configs.json").read_text())
    report = json.loads(
        (root / "result/20260831T083857.848038Z/final_performance.json").read_text()
    )
    entries = [entry for bundle in registry["bundles"] for entry in bundle["entries"]]
    shapes = json.loads((root / "official/test_shapes.json").read_text())["ordered_shapes"]
    records = []
    for index, (official, published) in enumerate(zip(shapes, report["shapes"])):
        key = {k: official[k] for k in ("batch_size", "qkv_dim", "heads", "seq_len", "layers", "causal", "ffn_dim")}
        match = [e for e in entries if all(e["shape"][k] == v for k, v in key.items())]
        assert len(match) == 1, (index, key)
        records.append(
            {
                "case_id": official["case_id"],
                "shape": match[0]["shape"],
                "config": match[0]["config"],
                "published_config_id": published["config_id"],
            }
        )
    out = Path(__file__).resolve().parent / "reference_configs.json"
    out.write_text(json.dumps({"source": "reference deployment registry + final report", "records": records}, indent=1) + "\n")
    print(out, len(records))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
