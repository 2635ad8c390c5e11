"""Write reference_lines.json: the line count of every text file of the
reference checkout (default /root/reference), so that tests can check the
file:line citations in this repository without the checkout present.

    python tests/golden/make_reference_lines.py [/path/to/reference]
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

SUFFIXES = {".py", ".cu", ".cpp", ".md", ".toml", ".yml", ".yaml", ".txt", ".in", ".cfg"}


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    counts = {}
    for p in sorted(root.rglob("*")):
        if ".git" in p.parts or not p.is_file():
            continue
        if p.suffix not in SUFFIXES and p.name not in ("LICENSE", "MANIFEST.in"):
            continue
        counts[str(p.relative_to(root))] = len(p.read_text(errors="replace").splitlines())
    out = Path(__file__).with_name("reference_lines.json")
    out.write_text(json.dumps(counts, indent=1, sort_keys=True) + "\n")
    print(f"{len(counts)} files -> {out}")


if __name__ == "__main__":
    main()
