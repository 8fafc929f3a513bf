"""Regenerate the golden fixtures from data files of the reference repository.

Run in the build container only (the GPU box has no reference checkout):

    python tests/golden/make_golden.py /root/reference

* e4m3_lut.json      -- the 256 decode values of the reference's E4M3 table
                        (native_indexer_plan.metal:19-35, equal to fp8.py:37-39),
                        parsed as numbers from the table's float literals.
* sigmoid_sweep.json -- domain definition and SHA-256 hashes recorded by the
                        reference's exhaustive BF16 sigmoid sweep
                        (bench-results/m3ultra512-native-routed-sigmoid-
                        formula-sweep-20260907.json).
"""

from __future__ import annotations

import json
import re
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def lut(reference: Path) -> list[float]:
    text = (reference / "native_execution" / "native_indexer_plan.metal").read_text()
    start = text.index("kNativeE4M3[256] = {")
    body = text[start:text.index("};", start)]
    values = [float(v) for v in re.findall(r"(-?[0-9][0-9.e+-]*)f", body.split("{", 1)[1])]
    if len(values) != 256:
        raise RuntimeError(f"expected 256 table values, found {len(values)}")
    return values


def sweep(reference: Path) -> dict:
    d = json.loads((reference / "bench-results" /
                    "m3ultra512-native-routed-sigmoid-formula-sweep-20260907.json").read_text())
    return {
        "source": "bench-results/m3ultra512-native-routed-sigmoid-formula-sweep-20260907.json",
        "domain_definition": d["domain"]["definition"],
        "domain_elements": d["domain"]["elements"],
        "domain_bits_sha256": d["domain"]["bits_sha256"],
        "reference_sigmoid_sha256": d["reference"]["sigmoid_hash"],
        "reference_execution": d["reference"]["execution"],
        "formula_hashes": {k: v["actual_hash"] for k, v in d["results"].items()},
        "formula_first_difference": {k: v["first_difference"] for k, v in d["results"].items()},
        "hash_definition": "sha256 of the little-endian uint16 BF16 bit patterns, domain in ascending bit order",
    }


def main(reference: Path) -> None:
    (HERE / "e4m3_lut.json").write_text(json.dumps({
        "source": "native_execution/native_indexer_plan.metal:19-35 (kNativeE4M3)",
        "values": lut(reference),
    }, indent=1) + "\n")
    (HERE / "sigmoid_sweep.json").write_text(json.dumps(sweep(reference), indent=2, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
