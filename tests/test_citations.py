"""Every `file:line` citation in the public header, the docs and the sources points at lines that
exist.

A citation is a file name with a known extension followed by `:line`, `:first-last`, or a comma
list of those (`mx_gemm.c:25-108, 123-194`). The file is looked up under the reference tree first
(a path as written, else a unique file of that base name or path suffix), then in this repository
(the tests and modules that the documents cite). Skipped when the reference tree is absent (the GPU
box): the check needs the cited files.
"""

import re
from functools import lru_cache
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
REFERENCE = Path("/root/reference")

# Files whose citations are checked: the C-ABI header, the documents this build writes, and
# every source file of the package, the oracle, the tests and the bench.
SCANNED = (
    ["include/matricxon_amd.h", "DESIGN.md", "INTEGRATION.md", "README.md", "bench.py",
     "__graft_entry__.py"]
    + [str(p.relative_to(REPO)) for d in ("matricxon_amd", "oracle", "tests")
       for p in sorted((REPO / d).rglob("*"))
       if p.suffix in (".py", ".hip", ".hpp", ".c", ".h") and "_ref" not in p.parts
       and "__pycache__" not in p.parts]
)

CITE = re.compile(
    r"(?<![\w/.-])((?:[\w-]+/)*[\w-]+\.(?:c|h|py|toml|txt|json|cfg|ini))"
    r":(\d+(?:-\d+)?(?:,\s?\d+(?:-\d+)?)*)"
)


@lru_cache(maxsize=None)
def _reference_files() -> tuple[Path, ...]:
    return tuple(p for p in REFERENCE.rglob("*") if p.is_file() and ".git" not in p.parts)


@lru_cache(maxsize=None)
def _line_count(path: Path) -> int:
    with open(path, "rb") as f:
        return sum(1 for _ in f)


def _resolve(name: str) -> Path | None:
    direct = REFERENCE / name
    if direct.is_file():
        return direct
    suffix = "/" + name
    hits = [p for p in _reference_files() if str(p).endswith(suffix)]
    if len(hits) == 1:
        return hits[0]
    local = REPO / name
    if local.is_file():
        return local
    if len(hits) > 1:
        return max(hits, key=_line_count)  # ambiguous base name: the check is only an upper bound
    mine = [p for p in REPO.rglob(Path(name).name) if "_work" not in p.parts]
    return mine[0] if len(mine) == 1 else None


def _ranges(spec: str) -> list[tuple[int, int]]:
    out = []
    for part in spec.split(","):
        part = part.strip()
        a, _, b = part.partition("-")
        out.append((int(a), int(b or a)))
    return out


def _citations():
    for rel in SCANNED:
        text = (REPO / rel).read_text(errors="replace")
        for lineno, line in enumerate(text.splitlines(), 1):
            for m in CITE.finditer(line):
                yield rel, lineno, m.group(1), m.group(2)


@pytest.mark.skipif(not REFERENCE.is_dir(), reason="the reference tree is not present")
def test_every_citation_points_at_existing_lines():
    bad = []
    for rel, lineno, name, spec in _citations():
        target = _resolve(name)
        if target is None:
            bad.append(f"{rel}:{lineno}: {name}:{spec} (no such file)")
            continue
        n = _line_count(target)
        for a, b in _ranges(spec):
            if not (1 <= a <= b <= n):
                bad.append(f"{rel}:{lineno}: {name}:{spec} ({target} has {n} lines)")
                break
    assert not bad, "citations of missing lines:\n" + "\n".join(bad)


def test_citation_pattern():
    """The parser reads the forms the documents use."""
    found = [(m.group(1), m.group(2)) for m in CITE.finditer(
        "(app/native/src/mx_gemm.c:25-108, 123-194) and `kquants.py:10-23`; "
        "device_packed.py:41-46,74-79; not a citation: 3.5:1 or http://x.py")]
    assert found == [("app/native/src/mx_gemm.c", "25-108, 123-194"), ("kquants.py", "10-23"),
                     ("device_packed.py", "41-46,74-79")]
    assert _ranges("25-108, 123-194") == [(25, 108), (123, 194)]
