"""Comments and code stand on their own: no committed source names the build's working
documents, its tooling or a phase of its development; reference files are cited by
their own paths.  Runs on any host."""

from __future__ import annotations

import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCE = re.compile(r"\.(py|hip|hpp|h|c)$|(^|/)Makefile$")
FORBIDDEN = [re.compile(p, re.I) for p in (
    r"this build", r"\b(design|survey|integration|verdict|advice)\.md\b", r"\bsurvey\s*§", r"\bbaseline\.(json|md)\b",
    r"north_star", r"gpu" + r"run", r"\bgpu (box|pool)\b", r"\bthe checker\b", r"\bround\s+\d", r"/root/reference",
)]


def test_no_source_names_the_working_documents_or_tooling():
    # tracked files and new ones not yet added (the ignored working area excluded)
    files = subprocess.run(["git", "ls-files", "--cached", "--others", "--exclude-standard"], cwd=ROOT,
                           capture_output=True, text=True, check=True).stdout.split()
    this = os.path.relpath(__file__, ROOT)
    hits = []
    for name in files:
        if not SOURCE.search(name) or name == this:
            continue
        with open(os.path.join(ROOT, name), encoding="utf-8", errors="replace") as f:
            for number, line in enumerate(f, 1):
                hits.extend(f"{name}:{number}: {line.strip()[:80]}" for p in FORBIDDEN if p.search(line))
    assert not hits, "\n".join(hits)
