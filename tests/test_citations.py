"""Every `path:line` citation in this repository points at lines that exist.

Docstrings, comments, the C-ABI header and the documents cite the reference
repository as `path:a-b` (optionally `path:a-b, c-d`).  For each citation
this test checks that

- the path names exactly one file of the reference (by its path, or by a
  unique path suffix such as `triton/sgd.py`), or else one file of this
  repository;
- every cited range lies inside that file;
- where the citation directly follows a backquoted name (`` `name` (path:a-b) ``)
  and the file defines that name with `def` or `class`, the definition lies
  inside the cited lines; otherwise the name appears in them.

It reads the reference checkout, so it is skipped where that is absent (the
GPU box has none).
"""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
REFERENCE = Path("/root/reference")

pytestmark = pytest.mark.skipif(not REFERENCE.is_dir(), reason="needs the reference checkout")

# Documents written about this repository by others are not scanned.
NOT_SCANNED = {"VERDICT.md", "ADVICE.md", "SURVEY.md", "BASELINE.md"}
SUFFIXES = (".py", ".h", ".hip", ".cpp", ".c", ".md")

CITATION = re.compile(
    r"(?<![\w/.-])((?:/root/reference/)?(?:[\w.-]+/)*[\w-]+\.(?:py|md|toml|yml|sh|in|txt))"
    r":(\d+)(?:-(\d+))?((?:,\s?\d+(?:-\d+)?(?![\w.]))*)"
)
NAMED = re.compile(r"`([A-Za-z_][\w.]*)(?:\([^`]*\))?`\s*(?:\(|at\s+|in\s+)?$")


def _files(root, names):
    return {name: root / name for name in names}


def _reference_files():
    return _files(REFERENCE, sorted(
        p.relative_to(REFERENCE).as_posix()
        for p in REFERENCE.rglob("*")
        if p.is_file() and "__pycache__" not in p.parts and ".git" not in p.parts
    ))


def _repo_files():
    listed = subprocess.run(["git", "ls-files"], cwd=REPO, capture_output=True, text=True, check=True)
    return _files(REPO, listed.stdout.split())


def _resolve(path, files):
    if path in files:
        return [path]
    return [name for name in files if name.endswith("/" + path)]


def _ranges(match):
    ranges = [(int(match.group(2)), int(match.group(3) or match.group(2)))]
    for part in re.findall(r"\d+(?:-\d+)?", match.group(4) or ""):
        first, _, last = part.partition("-")
        ranges.append((int(first), int(last or first)))
    return ranges


def _citations():
    reference, repo = _reference_files(), _repo_files()
    for name, path in sorted(repo.items()):
        if name in NOT_SCANNED or not name.endswith(SUFFIXES) or not path.is_file():
            continue
        text = path.read_text(errors="replace")
        for match in CITATION.finditer(text):
            cited = match.group(1).removeprefix("/root/reference/")
            line = text.count("\n", 0, match.start()) + 1
            named = NAMED.search(text[max(0, match.start() - 120):match.start()])
            yield f"{name}:{line}", cited, _ranges(match), named and named.group(1).split(".")[-1], reference, repo


def _check(cited, ranges, symbol, reference, repo):
    found = _resolve(cited, reference)
    files = reference
    if not found:
        found, files = _resolve(cited, repo), repo
    if len(found) != 1:
        return [f"{cited} names {len(found)} files {found}"]
    lines = files[found[0]].read_text(errors="replace").splitlines()
    errors = [f"{cited}:{a}-{b} lies outside {found[0]} ({len(lines)} lines)"
              for a, b in ranges if not 1 <= a <= b <= len(lines)]
    if errors or not symbol:
        return errors
    cited_lines = [lines[i - 1] for a, b in ranges for i in range(a, b + 1)]
    definition = re.compile(rf"\s*(?:async\s+)?(?:def|class)\s+{re.escape(symbol)}\b")
    if any(definition.match(text) for text in lines):
        if not any(definition.match(text) for text in cited_lines):
            errors.append(f"`{symbol}` is defined outside {found[0]}:{ranges}")
    elif not any(re.search(rf"\b{re.escape(symbol)}\b", text) for text in cited_lines):
        errors.append(f"`{symbol}` does not appear in {found[0]}:{ranges}")
    return errors


def test_every_citation_names_existing_lines():
    problems, count = [], 0
    for where, cited, ranges, symbol, reference, repo in _citations():
        count += 1
        problems.extend(f"{where}: {error}" for error in _check(cited, ranges, symbol, reference, repo))
    assert count > 200, f"only {count} citations found: the scan is broken"
    assert not problems, "\n".join(problems)


def test_the_header_cites_each_replaced_entry_point():
    """Each C-ABI entry point that replaces a reference interface cites it."""
    header = (REPO / "include" / "sr_states_hip.h").read_text()
    expected = {
        "sr_update_key": "update_key",
        "sr_state_key": "state_key",
        "sr_cast": "_sr_cast_bf16_kernel",
        "sr_adamw_step": "_fused_adamw_kernel",
        "sr_adamw_multi": "_multi_adamw_kernel",
        "sr_sgdm_step": "_fused_sgdm_kernel",
        "sr_sgdm_multi": "_multi_sgdm_kernel",
    }
    reference = _reference_files()
    for entry, symbol in expected.items():
        declaration = re.search(rf"\n(?:int|uint32_t) {entry}\(", header)
        assert declaration, entry
        comment = header[header.rfind("/*", 0, declaration.start()):declaration.start()]
        cited = [m for m in CITATION.finditer(comment)]
        assert cited, f"{entry} cites nothing"
        hits = []
        for m in cited:
            path = _resolve(m.group(1), reference)
            assert len(path) == 1, m.group(0)
            lines = reference[path[0]].read_text().splitlines()
            for a, b in _ranges(m):
                hits += [text for text in lines[a - 1:b] if re.search(rf"\bdef {re.escape(symbol)}\b", text)]
        assert hits, f"{entry}: no cited range defines {symbol}"


def test_the_checker_catches_a_bad_citation():
    reference, repo = _reference_files(), _repo_files()
    assert _check("sr_states/triton/sgd.py", [(434, 490)], None, reference, repo)
    assert _check("sgd.py", [(12, 16)], None, reference, repo)  # three files match
    assert _check("sr_states/triton/adamw.py", [(160, 221)], "_fused_adamw_kernel", reference, repo)
    assert not _check("sr_states/triton/adamw.py", [(59, 100)], "_fused_adamw_kernel", reference, repo)
