"""Every ``file:line`` citation of a reference file names lines that exist,
and the function or class a citation's line names.

The reference's line counts and symbol spans come from
``tests/golden/reference_lines.json`` and ``reference_symbols.json`` (written
by ``tests/golden/make_reference_lines.py``), so the check needs no reference
checkout.  A citation is ``path.ext:N`` or ``path.ext:N-M`` whose path is a
reference file or a unique suffix of one, plus every bare ``:N`` / ``:N-M``
later on the same line, which continues the citation before it
(``format.py:14-16 and :104-131``).  Citations of this repository's own files
(names the reference does not have) are not checked.

A citation's line names a reference symbol of the cited file when the
symbol's qualified name (``CacheSpec.record_bytes``) appears on it, or its
own name does and is unmistakably an identifier (an underscore or a capital
letter, five characters or more: ``unpack_codes``, ``KVSSDPipeline``).  When
a line names symbols of the cited file, the cited range must overlap at
least one of them.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
COUNTS = json.loads((GOLDEN / "reference_lines.json").read_text())
SYMBOLS = json.loads((GOLDEN / "reference_symbols.json").read_text())
CITE = re.compile(r"([A-Za-z0-9_./-]+\.(?:py|cu|cpp|md|toml|yml|yaml)):(\d+)(?:-(\d+))?")
BARE = re.compile(r"(?<![\w./:-]):(\d+)(?:-(\d+))?(?!\w)(?!\.\w)")
SOURCES = (".py", ".hip", ".hpp", ".h", ".c", ".md")
# review and survey notes quote the reference as it is discussed, not as code
NOT_CHECKED = {"SURVEY.md", "VERDICT.md", "ADVICE.md", "BASELINE.md"}
# this file's own negative controls cite wrong lines on purpose
SELF = Path(__file__).resolve()
SKIP_DIRS = {"_work", "gpurun_out", ".git", "__pycache__", ".pytest_cache", "_build"}


def _files():
    for f in sorted(ROOT.rglob("*")):
        if not f.is_file() or SKIP_DIRS.intersection(f.relative_to(ROOT).parts):
            continue
        if f.name in NOT_CHECKED or f == SELF or not (f.suffix in SOURCES or f.name == "Makefile"):
            continue
        yield f


def line_citations(line: str):
    """(text, [reference files matching the path], first, last) of every
    citation on a line, bare continuations included."""
    out = []
    spans = []
    last = None
    events = [(m.start(), "cite", m) for m in CITE.finditer(line)] + [(m.start(), "bare", m) for m in BARE.finditer(line)]
    for _, kind, m in sorted(events, key=lambda e: e[0]):
        if kind == "cite":
            path = m.group(1).lstrip("./")
            matches = [p for p in COUNTS if p == path or p.endswith("/" + path)]
            last = matches or None
            spans.append((m.start(), m.end()))
            if matches:
                out.append((m.group(0), matches, int(m.group(2)), int(m.group(3) or m.group(2))))
        elif last and not any(a <= m.start() < b for a, b in spans):
            out.append((m.group(0), last, int(m.group(1)), int(m.group(2) or m.group(1))))
    return out


def named_symbols(line: str, ref_file: str) -> dict[str, list[int]]:
    named = {}
    for qual, span in SYMBOLS.get(ref_file, {}).items():
        own = qual.rsplit(".", 1)[-1]
        if re.search(rf"(?<![\w.]){re.escape(qual)}\b", line):
            named[qual] = span
        elif len(own) >= 5 and ("_" in own.strip("_") or own != own.lower()) and re.search(
            rf"(?<![\w]){re.escape(own)}\b", line
        ):
            named[qual] = span
    return named


def citation_problems(where: str, line: str) -> list[str]:
    bad = []
    for text, matches, first, last in line_citations(line):
        if len(matches) != 1:
            bad.append(f"{where}: {text} is ambiguous ({', '.join(matches)})")
            continue
        ref = matches[0]
        n = COUNTS[ref]
        if not 1 <= first <= last <= n:
            bad.append(f"{where}: {text} but {ref} has {n} lines")
            continue
        named = named_symbols(line, ref)
        if named and not any(first <= b and a <= last for a, b in named.values()):
            spans = ", ".join(f"{k} {a}-{b}" for k, (a, b) in named.items())
            bad.append(f"{where}: {text} misses what the line names ({spans})")
    return bad


def test_fixture_lists_the_reference_files_the_path_cites():
    for name in ("src/kvssd/backends/reference.py", "src/kvssd/quant.py", "csrc/fused_decode.cu"):
        assert COUNTS[name] > 0
    assert SYMBOLS["src/kvssd/quant.py"]["unpack_codes"] == [40, 46]
    assert SYMBOLS["csrc/fused_decode.cu"]["fused_decode_cuda"] == [92, 143]


def test_every_reference_citation_is_in_range_and_names_its_symbol():
    bad = []
    seen = 0
    for f in _files():
        for i, line in enumerate(f.read_text(errors="replace").splitlines(), 1):
            seen += len(line_citations(line))
            bad += citation_problems(f"{f.relative_to(ROOT)}:{i}", line)
    assert seen > 100, "the citation scan found suspiciously few citations"
    assert not bad, "\n".join(bad)


def test_checker_catches_the_kinds_of_mistake_it_is_for():
    # a range past the file's end in a bare continuation
    assert citation_problems("x", "layout: src/kvssd/format.py:14-16 and :203-230.")
    # a range that holds another function than the one named
    assert citation_problems("x", "unpack_codes: src/kvssd/quant.py:66-72")
    assert citation_problems("x", "`quantize_tensor` (src/kvssd/quant.py:68-73)")
    # and the right ones pass
    assert not citation_problems("x", "layout: src/kvssd/format.py:14-16 and :104-131")
    assert not citation_problems("x", "unpack_codes: src/kvssd/quant.py:40-46")
    assert not citation_problems("x", "`KVSSDPipeline.decode` src/kvssd/pipeline.py:167-187, chunks :56-116")
    # slices and times are not continuations without a citation before them
    assert line_citations("x[:4] at 07:51") == []
