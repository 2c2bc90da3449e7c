"""Every reference citation (``ie/....py:N`` or ``:N-M``) in the C-ABI header, the
design and integration notes and the package's sources names a file of the reference
and lines that file has (CPU; reads the reference's files as text where they are
present, and is skipped where they are not)."""
from __future__ import annotations

import re
from pathlib import Path

import pytest

from conftest import ROOT

REFERENCE = Path("/root/reference")
CITATION = re.compile(r"\b((?:ie|tests)/[\w/]+\.py):(\d+)(?:-(\d+))?((?:,\d+(?:-\d+)?)*)")


def sources():
    yield ROOT / "include" / "iekv.h"
    yield ROOT / "INTEGRATION.md"
    yield ROOT / "DESIGN.md"
    yield from sorted((ROOT / "inference-engine_amd" / "iekv").rglob("*.py"))
    yield from sorted((ROOT / "inference-engine_amd" / "csrc").glob("*.h*"))
    yield from sorted((ROOT / "oracle").glob("*.py"))


def test_reference_citations_name_existing_lines():
    if not (REFERENCE / "ie").is_dir():
        pytest.skip("the reference is not present here")
    checked = 0
    for path in sources():
        for m in CITATION.finditer(path.read_text()):
            cited = REFERENCE / m.group(1)
            assert cited.is_file(), f"{path.name}: {m.group(0)} names no reference file"
            length = len(cited.read_text().splitlines())
            spans = [(m.group(2), m.group(3))] + [
                tuple(part.split("-")) if "-" in part else (part, None)
                for part in m.group(4).split(",") if part]
            for first, last in spans:
                lo, hi = int(first), int(last or first)
                assert 1 <= lo <= hi <= length, \
                    f"{path.name}: {m.group(0)} cites lines past the end ({length} lines)"
            checked += 1
    assert checked > 50
