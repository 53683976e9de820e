"""Every `file.ext:L` / `file.ext:L-M` citation of a reference file must name
lines that exist.

Sources, headers, tests, the oracle and the design notes cite the reference
by path (often shortened to its last components, crates/rusticide-X/ to X/)
and line range. When the
reference checkout is mounted at its usual place, each citation must resolve
to a file there whose path ends with the cited one and that has at least M
lines. Without the checkout (as on a GPU box) the test is skipped.
"""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE = "/root/reference"

FILES = ["DESIGN.md", "INTEGRATION.md", "bench.py", "__graft_entry__.py"]
DIRS = ["include", "rusticide_amd", "oracle", "tests"]
EXTS = (".h", ".hip", ".c", ".py", ".md")

# path.ext:L[-M][,L[-M]]... with a reference extension
CITE = re.compile(r"([A-Za-z0-9_./-]+\.(?:rs|toml|json|md)):(\d+(?:-\d+)?(?:,\d+(?:-\d+)?)*)")


def repo_files():
    for f in FILES:
        yield os.path.join(ROOT, f)
    for d in DIRS:
        for dirpath, dirnames, names in os.walk(os.path.join(ROOT, d)):
            dirnames[:] = [n for n in dirnames if not n.startswith(("_", "."))]
            for n in names:
                if n.endswith(EXTS) and n != os.path.basename(__file__):
                    yield os.path.join(dirpath, n)


def reference_index():
    index = {}
    for dirpath, dirnames, names in os.walk(REFERENCE):
        dirnames[:] = [n for n in dirnames if n not in (".git", "target")]
        for n in names:
            full = os.path.join(dirpath, n)
            index.setdefault(n, []).append(full)
    return index


def line_count(path, cache={}):
    if path not in cache:
        with open(path, "rb") as f:
            cache[path] = sum(1 for _ in f)
    return cache[path]


@pytest.mark.skipif(not os.path.isdir(REFERENCE), reason="the reference checkout is not mounted")
def test_every_cited_line_range_exists():
    index = reference_index()
    bad, checked = [], 0
    for path in repo_files():
        with open(path, encoding="utf-8", errors="replace") as f:
            for lineno, text in enumerate(f, 1):
                for cited, ranges in CITE.findall(text):
                    name = os.path.basename(cited)
                    # crates/rusticide-X/src/... is often cited as X/src/...
                    tail = "/" + cited.lstrip("./")
                    candidates = [c for c in index.get(name, [])
                                  if c.endswith(tail) or c.replace("/rusticide-", "/").endswith(tail)]
                    if not candidates:
                        if name in ("DESIGN.md", "INTEGRATION.md", "SURVEY.md", "BASELINE.md", "README.md"):
                            continue  # this repository's own notes, not the reference
                        bad.append(f"{os.path.relpath(path, ROOT)}:{lineno}: {cited} not in the reference")
                        continue
                    top = max(int(r.split("-")[-1]) for r in ranges.split(","))
                    lows = [int(r.split("-")[0]) for r in ranges.split(",")]
                    checked += 1
                    if not any(line_count(c) >= top for c in candidates) or min(lows) < 1:
                        n = max(line_count(c) for c in candidates)
                        bad.append(f"{os.path.relpath(path, ROOT)}:{lineno}: {cited}:{ranges} "
                                   f"past the end ({n} lines)")
                    for r in ranges.split(","):
                        lo, _, hi = r.partition("-")
                        if hi and int(hi) < int(lo):
                            bad.append(f"{os.path.relpath(path, ROOT)}:{lineno}: {cited}:{r} is backwards")
    assert checked > 100
    assert not bad, "\n".join(bad)
