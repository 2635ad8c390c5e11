"""Write reference_lines.json and reference_symbols.json from a reference
checkout (default /root/reference), so that tests can check the file:line
citations in this repository without the checkout present:

* reference_lines.json: the line count of every text file;
* reference_symbols.json: per Python / CUDA / C++ source, the line span
  [first, last] of every function, method and class, found by parsing the
  text (Python's ast for .py; brace matching for .cu / .cpp).  Nothing of the
  reference is imported or run.

    python tests/golden/make_reference_lines.py [/path/to/reference]
"""

from __future__ import annotations

import ast
import json
import re
import sys
from pathlib import Path

SUFFIXES = {".py", ".cu", ".cpp", ".md", ".toml", ".yml", ".yaml", ".txt", ".in", ".cfg"}
# a C/C++ function definition's head: return type(s), a name, an argument list
C_HEAD = re.compile(r"^[A-Za-z_][\w:<>,\s\*&]*?\b([A-Za-z_]\w*)\s*\(")


def python_symbols(text: str) -> dict[str, list[int]]:
    spans: dict[str, list[int]] = {}

    def visit(node, prefix: str) -> None:
        for child in ast.iter_child_nodes(node):
            if isinstance(child, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)):
                first = min([child.lineno] + [d.lineno for d in child.decorator_list])
                name = prefix + child.name
                spans[name] = [first, child.end_lineno]
                visit(child, name + ".")

    visit(ast.parse(text), "")
    return spans


def c_symbols(text: str) -> dict[str, list[int]]:
    """Functions defined at file scope: a head line at column 0, then a body
    from its first '{' to the matching '}' (strings and comments are rare
    enough in these files that braces inside them are not handled)."""
    lines = text.splitlines()
    spans: dict[str, list[int]] = {}
    i = 0
    while i < len(lines):
        m = C_HEAD.match(lines[i])
        if m and not lines[i].startswith((" ", "\t", "#", "//")) and m.group(1) not in ("if", "for", "while", "return"):
            first = i - 1 if i > 0 and lines[i - 1].startswith("template") else i
            depth, opened, j = 0, False, i
            while j < len(lines):
                code = lines[j].split("//")[0]
                if ";" in code and not opened and "{" not in code:
                    break  # a declaration
                depth += code.count("{") - code.count("}")
                opened = opened or "{" in code
                if opened and depth == 0:
                    spans[m.group(1)] = [first + 1, j + 1]
                    break
                j += 1
            i = j + 1
            continue
        i += 1
    return spans


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    counts, symbols = {}, {}
    for p in sorted(root.rglob("*")):
        if ".git" in p.parts or not p.is_file():
            continue
        if p.suffix not in SUFFIXES and p.name not in ("LICENSE", "MANIFEST.in"):
            continue
        rel = str(p.relative_to(root))
        text = p.read_text(errors="replace")
        counts[rel] = len(text.splitlines())
        if p.suffix == ".py":
            symbols[rel] = python_symbols(text)
        elif p.suffix in (".cu", ".cpp"):
            symbols[rel] = c_symbols(text)
    here = Path(__file__).parent
    (here / "reference_lines.json").write_text(json.dumps(counts, indent=1, sort_keys=True) + "\n")
    (here / "reference_symbols.json").write_text(json.dumps(symbols, indent=1, sort_keys=True) + "\n")
    print(f"{len(counts)} files, {sum(map(len, symbols.values()))} symbols -> {here}")


if __name__ == "__main__":
    main()
