"""Every `path:line` citation in the sources and design notes points inside
the file it names.

Citations name the reference's files (relative to its repository root, or by
file name alone when that name is unique there) or this repository's own
files. A cited line past the end of its file, or a range that runs
backwards, is a stale citation. Skipped when the reference checkout is not
present (it is not on the GPU box).
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"

SCANNED = ["include", "oracle", os.path.join("wgblas_amd", "csrc"), os.path.join("wgblas_amd", "js"),
           "tests", "DESIGN.md", "INTEGRATION.md", "README.md", "bench.py", "__graft_entry__.py",
           os.path.join("wgblas_amd", "native.py"), os.path.join("wgblas_amd", "build.py")]
EXTS = (".h", ".c", ".cc", ".cpp", ".hip", ".py", ".mjs", ".md", ".js")
CITE = re.compile(r"([A-Za-z0-9_.\-/]+\.(?:mjs|wgsl|js|json|yml|yaml|h|c|cc|hip|py|md|mts|toml))"
                  r":(\d+(?:-\d+)?(?:,\s?\d+(?:-\d+)?)*)")


def _files():
    for entry in SCANNED:
        path = os.path.join(ROOT, entry)
        if os.path.isfile(path):
            yield path
        for dirpath, dirnames, filenames in os.walk(path):
            dirnames[:] = [d for d in dirnames if d not in ("golden", "lib", "__pycache__", "node_modules")]
            for f in filenames:
                if f.endswith(EXTS):
                    yield os.path.join(dirpath, f)


def _index(root):
    by_name = {}
    for dirpath, dirnames, filenames in os.walk(root):
        dirnames[:] = [d for d in dirnames if d not in (".git", "node_modules")]
        for f in filenames:
            by_name.setdefault(f, []).append(os.path.join(dirpath, f))
    return by_name


def _line_count(path, cache={}):
    if path not in cache:
        with open(path, "rb") as fh:
            data = fh.read()
            cache[path] = data.count(b"\n") + (0 if data.endswith(b"\n") else 1)
    return cache[path]


def _resolve(cited, ref_names, own_names):
    """Candidate files for a cited path: the reference's file at that path,
    else this repository's, else (a bare or partial path) every file of that
    name whose path ends with the cited one, reference first."""
    for root in (REF, ROOT):
        p = os.path.join(root, cited)
        if os.path.isfile(p):
            return [p]
    base = os.path.basename(cited)
    for names in (ref_names, own_names):
        hits = [p for p in names.get(base, []) if p.endswith("/" + cited) or cited == base]
        if hits:
            return hits
    return []


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout not present")
def test_every_citation_is_in_range():
    ref_names, own_names = _index(REF), _index(ROOT)
    bad = []
    for path in _files():
        text = open(path, encoding="utf-8", errors="replace").read()
        for m in CITE.finditer(text):
            cited, spans = m.group(1), m.group(2)
            where = f"{os.path.relpath(path, ROOT)}:{text.count(chr(10), 0, m.start()) + 1}"
            targets = _resolve(cited, ref_names, own_names)
            if not targets:
                bad.append(f"{where}: {cited} not found")
                continue
            for span in spans.split(","):
                lo, _, hi = span.strip().partition("-")
                lo, hi = int(lo), int(hi or lo)
                if hi < lo:
                    bad.append(f"{where}: {cited}:{span} runs backwards")
                elif not any(hi <= _line_count(t) for t in targets):
                    bad.append(f"{where}: {cited}:{span} past the end "
                               f"({', '.join(str(_line_count(t)) for t in targets)} lines)")
    assert not bad, "stale citations:\n" + "\n".join(bad)
