"""Copy the routed-expert sections of the reference's operator fixture into tests/golden.

The reference pins its routing and clamped-SwiGLU operators with
tests/fixtures/deepseek_v4_operators.json (a pure-Python translation of the official model
equations, tolerance 3e-5). Only the sections on this path are kept: ``expert``,
``hash_route`` and ``learned_route``. Run where the reference tree is mounted:

    python tests/golden/extract_reference_fixtures.py /root/reference
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

KEEP = ("absolute_tolerance", "format", "official_revision", "expert", "hash_route",
        "learned_route")


def main(ref_root: str) -> None:
    src = Path(ref_root) / "tests" / "fixtures" / "deepseek_v4_operators.json"
    data = json.loads(src.read_text())
    out = {k: data[k] for k in KEEP}
    out["source"] = "reference tests/fixtures/deepseek_v4_operators.json (sections on the MoE path)"
    dst = Path(__file__).with_name("deepseek_v4_moe_operators.json")
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {dst}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
