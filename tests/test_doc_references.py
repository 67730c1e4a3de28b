"""The documents at the repository root point at files that exist: every
path under profiles/, tests/, include/, oracle/ or the package that they
quote in backticks names a file or folder of the tree, and a quoted line
number lies inside that file."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOCS = ("DESIGN.md", "README.md", "INTEGRATION.md")
PATH = re.compile(r"`((?:profiles|tests|include|oracle|tokamax-tpu-kernel-lab_amd)/[\w./-]+?)(?::(\d+)(?:-(\d+))?)?`")
# named as what is absent: the reference has no C source to build there
ABSENT_ON_PURPOSE = {"oracle/_ref"}


@pytest.mark.parametrize("doc", DOCS)
def test_quoted_paths_exist(doc):
  text = open(os.path.join(ROOT, doc)).read()
  quoted = PATH.findall(text)
  assert quoted, f"{doc} quotes no repository path"
  bad = []
  for path, lo, hi in quoted:
    path = path.rstrip(".")
    full = os.path.join(ROOT, path)
    if path in ABSENT_ON_PURPOSE:
      continue
    if not os.path.exists(full):
      bad.append(path)
    elif lo and os.path.isfile(full):
      n = sum(1 for _ in open(full, errors="replace"))
      if int(hi or lo) > n:
        bad.append(f"{path}:{lo}{'-' + hi if hi else ''} (file has {n} lines)")
  assert not bad, bad


def test_profiles_name_their_commands():
  """Each committed profile summary gives the command that made it, which
  runs committed files only (no working-folder script)."""
  folder = os.path.join(ROOT, "profiles")
  names = sorted(os.listdir(folder))
  assert names
  for name in names:
    text = open(os.path.join(folder, name), errors="replace").read()
    assert re.search(r"rocprofv3|python", text), f"{name}: no command"
    assert "_work/" not in text, f"{name}: names a working-folder file"
    for script in re.findall(r"python3? (?:-u )?([\w./-]+\.py)", text):
      assert os.path.exists(os.path.join(ROOT, script)), f"{name}: {script} is not in the tree"
