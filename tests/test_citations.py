"""Every reference citation in this repository points at real lines.

A citation is ``path.py:a`` or ``path.py:a-b`` (paths relative to the
reference package ``src/myvllm``, or a bare file name that is unique there),
and a continuation ``:a`` / ``:a-b`` in backticks right after one cites the
same file.  Each cited range must lie inside the cited file.  Runs where the
reference checkout is present (the build container); skipped elsewhere.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/src/myvllm"
SCANNED = ["oracle", "myvllm_amd", "include", "tests", "bench.py", "__graft_entry__.py", "DESIGN.md",
           "INTEGRATION.md"]
CITE = re.compile(r"(?P<file>[\w./]+\.py)?:(?P<a>\d+)(?:-(?P<b>\d+))?")
SOURCE_SUFFIXES = (".py", ".hip", ".cpp", ".h", ".md")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout not present")


def _reference_files():
    files = {}
    for d, _, names in os.walk(REF):
        for n in names:
            if n.endswith(".py"):
                p = os.path.join(d, n)
                files[os.path.relpath(p, REF)] = sum(1 for _ in open(p, encoding="utf-8"))
    return files


def _resolve(name, files):
    name = name.lstrip("./")
    for prefix in ("", "src/myvllm/"):
        if name.startswith(prefix) and name[len(prefix):] in files:
            return name[len(prefix):]
    hits = [f for f in files if f.endswith("/" + name) or f == name]
    return hits[0] if len(hits) == 1 else None


def _scanned_files():
    for entry in SCANNED:
        p = os.path.join(ROOT, entry)
        if os.path.isfile(p):
            yield p
        else:
            for d, _, names in os.walk(p):
                if "__pycache__" in d:
                    continue
                for n in names:
                    if n.endswith(SOURCE_SUFFIXES):
                        yield os.path.join(d, n)


def citations():
    files = _reference_files()
    own = {os.path.basename(p) for p in _scanned_files()}
    out = []
    for path in _scanned_files():
        text = open(path, encoding="utf-8").read()
        current = None
        for m in CITE.finditer(text):
            name = m.group("file")
            if name:
                if os.path.basename(name) in own and _resolve(name, files) is None:
                    current = None  # a file of this repository
                    continue
                current = _resolve(name, files)
                if current is None:
                    out.append((os.path.relpath(path, ROOT), m.group(0), None, None, None))
                    continue
            else:
                # a bare ":a" continues the last cited file only inside backticks
                if current is None or text[max(0, m.start() - 1)] != "`":
                    continue
            a = int(m.group("a"))
            b = int(m.group("b") or a)
            out.append((os.path.relpath(path, ROOT), m.group(0), current, a, b))
    return out, files


def test_every_citation_is_inside_its_file():
    cites, files = citations()
    assert len(cites) > 100
    bad = []
    for where, text, f, a, b in cites:
        if f is None:
            bad.append(f"{where}: {text} names no unique reference file")
        elif not (1 <= a <= b <= files[f]):
            bad.append(f"{where}: {text} -> {f} has {files[f]} lines")
    assert not bad, "\n".join(bad)
