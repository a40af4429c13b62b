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


# A name in code form (`name`, a.b, camelCase, snake_case or name()) or a
# quoted message right before a parenthesised group of citations names what
# the group cites.
_CODE = (r"(?:`[A-Za-z_][\w.]*(?:\(\))?`|[A-Za-z_]\w*(?:\.\w+)+(?:\(\))?|[a-z]+[A-Z]\w*(?:\(\))?"
         r"|[A-Za-z]\w*_\w+(?:\(\))?|\w+\(\))")
_NAMED = re.compile(r"(" + _CODE + r")\s*$")
_MESSAGE = re.compile(r"\"([^\"]{8,})\"\s*$")
_GROUP = re.compile(r"\(([^()]*)\)")
# A comment block ending right above a definition names that definition.
_COMMENT = re.compile(r"^\s*(//|/\*|\*|#)")
_DEF = re.compile(r"^\s*(?:export\s+)?(?:async\s+)?(?:function\s+(\w+)|static\s+(?:async\s+)?(\w+)\s*\("
                  r"|class\s+(\w+)|def\s+(\w+)|(?:async\s+)?(\w+)\s*\([^)]*\)\s*\{)")


def _lines(path, cache={}):
    if path not in cache:
        cache[path] = open(path, encoding="utf-8", errors="replace").read().split("\n")
    return cache[path]


def _named_in_range(pattern, cites, ref_names, own_names):
    """(the name occurs in some cited file, it occurs inside a cited range
    there, give or take two lines)."""
    in_file = in_range = False
    for m in cites:
        targets = _resolve(m.group(1), ref_names, own_names)
        if not targets:
            continue
        lines = _lines(targets[0])
        if not any(re.search(pattern, line) for line in lines):
            continue
        in_file = True
        for span in m.group(2).split(","):
            lo, _, hi = span.strip().partition("-")
            lo, hi = int(lo), int(hi or lo)
            if re.search(pattern, "\n".join(lines[max(0, lo - 3):hi + 2])):
                in_range = True
    return in_file, in_range


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout not present")
def test_cited_range_holds_the_named_symbol():
    """Where a citation names what it cites — a symbol or a message right
    before the parenthesised citations, or the definition that a doc comment
    with citations sits on — the cited range (give or take two lines) holds
    that name, whenever the cited file holds it at all."""
    ref_names, own_names = _index(REF), _index(ROOT)
    bad, checked = [], 0
    for path in _files():
        text = open(path, encoding="utf-8", errors="replace").read()
        for g in _GROUP.finditer(text):
            cites = list(CITE.finditer(g.group(1)))
            if not cites:
                continue
            pre = text[max(0, g.start() - 120):g.start()].split("\n")[-1]
            sym, msg = _NAMED.search(pre), _MESSAGE.search(pre)
            if sym:
                name = sym.group(1).strip("`").replace("()", "").split(".")[-1]
                if any(name == os.path.splitext(os.path.basename(m.group(1)))[0] for m in cites):
                    continue  # the file's own name: the whole file is meant
                pattern = r"\b%s\b" % re.escape(name)
            elif msg:
                name = msg.group(1)
                pattern = re.escape(name[:30])
            else:
                continue
            in_file, in_range = _named_in_range(pattern, cites, ref_names, own_names)
            checked += in_file
            if in_file and not in_range:
                line = text.count("\n", 0, g.start()) + 1
                bad.append(f"{os.path.relpath(path, ROOT)}:{line}: {name} is not in ({g.group(1)[:90]})")
        if not path.endswith((".mjs", ".js", ".py")):
            continue
        lines = text.split("\n")
        i = 0
        while i < len(lines):
            if not (_COMMENT.match(lines[i]) and CITE.search(lines[i])):
                i += 1
                continue
            j = i
            while j < len(lines) and _COMMENT.match(lines[j]):
                j += 1
            d = _DEF.match(lines[j]) if j < len(lines) else None
            name = next((x for x in d.groups() if x), None) if d else None
            if name and name not in ("if", "for", "while", "switch", "catch", "return"):
                pattern = r"\b%s\b" % re.escape(name)
                for m in CITE.finditer("\n".join(lines[i:j])):
                    in_file, in_range = _named_in_range(pattern, [m], ref_names, own_names)
                    checked += in_file
                    if in_file and not in_range:
                        bad.append(f"{os.path.relpath(path, ROOT)}:{i + 1}: {name} (defined below) is not "
                                   f"in {m.group(0)}")
            i = max(j, i + 1)
    assert checked >= 5, f"only {checked} named citations found: the patterns stopped matching"
    assert not bad, "citations whose range does not hold what they name:\n" + "\n".join(bad)
