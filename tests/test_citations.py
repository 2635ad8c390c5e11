"""Every ``file:line`` citation of a reference file names lines that exist.

The reference's line counts come from ``tests/golden/reference_lines.json``
(written by ``tests/golden/make_reference_lines.py``), so the check needs no
reference checkout.  A citation is ``path.ext:N`` or ``path.ext:N-M`` whose
path is a reference file or a unique suffix of one; citations of this
repository's own files (names the reference does not have) are not checked.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
COUNTS = json.loads((ROOT / "tests" / "golden" / "reference_lines.json").read_text())
CITE = re.compile(r"([A-Za-z0-9_./-]+\.(?:py|cu|cpp|md|toml|yml|yaml)):(\d+)(?:-(\d+))?")
SOURCES = (".py", ".hip", ".hpp", ".h", ".c", ".md")
# review and survey notes quote the reference as it is discussed, not as code
NOT_CHECKED = {"SURVEY.md", "VERDICT.md", "ADVICE.md", "BASELINE.md"}
SKIP_DIRS = {"_work", "gpurun_out", ".git", "__pycache__", ".pytest_cache", "_build"}


def _files():
    for f in sorted(ROOT.rglob("*")):
        if not f.is_file() or SKIP_DIRS.intersection(f.relative_to(ROOT).parts):
            continue
        if f.name in NOT_CHECKED or not (f.suffix in SOURCES or f.name == "Makefile"):
            continue
        yield f


def _citations():
    for f in _files():
        for i, line in enumerate(f.read_text(errors="replace").splitlines(), 1):
            for m in CITE.finditer(line):
                path = m.group(1).lstrip("./")
                matches = [p for p in COUNTS if p == path or p.endswith("/" + path)]
                if matches:
                    yield f.relative_to(ROOT), i, m.group(0), matches, int(m.group(2)), int(m.group(3) or m.group(2))


def test_fixture_lists_the_reference_files_the_path_cites():
    for name in ("src/kvssd/backends/reference.py", "src/kvssd/quant.py", "csrc/fused_decode.cu"):
        assert COUNTS[name] > 0


def test_every_reference_citation_is_in_range_and_unambiguous():
    bad = []
    seen = 0
    for where, line, text, matches, first, last in _citations():
        seen += 1
        if len(matches) != 1:
            bad.append(f"{where}:{line}: {text} is ambiguous ({', '.join(matches)})")
            continue
        n = COUNTS[matches[0]]
        if not 1 <= first <= last <= n:
            bad.append(f"{where}:{line}: {text} but {matches[0]} has {n} lines")
    assert seen > 100, "the citation scan found suspiciously few citations"
    assert not bad, "\n".join(bad)
