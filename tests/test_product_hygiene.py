"""What the shipped library and its Python layer must not contain, checked in
their sources (csrc/*.hip, csrc/*.h, lmoe/*.py; comments stripped):

* no environment switches: a caller's environment must not change which
  kernel runs (every variant the library can take is chosen by the problem
  shape alone);
* no device allocation or memset in the library: workspaces and outputs come
  from the caller, and a memset node recorded into a captured HIP graph has
  given wrong results on replays after the first (the layer forward is
  replayed as one graph);
* no stream priorities, no registration of existing host memory, no uncached
  device memory (each has hung or corrupted work on the target boxes);
* no CUDA compatibility layer (hipify output, platform switches);
* the product never imports the CPU oracle (test infrastructure only)."""
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tokamax-tpu-kernel-lab_amd")
CPP = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")) + glob.glob(os.path.join(PKG, "csrc", "*.h")))
PY = sorted(glob.glob(os.path.join(PKG, "lmoe", "*.py")))


def _cpp_code(path):
  text = open(path).read()
  text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
  return re.sub(r"//[^\n]*", " ", text)


def _py_code(path):
  text = open(path).read()
  text = re.sub(r'("""|\'\'\').*?\1', " ", text, flags=re.S)
  return re.sub(r"#[^\n]*", " ", text)


CPP_FORBIDDEN = {
    "environment read": r"\b(getenv|secure_getenv)\s*\(",
    "device allocation": r"\bhip(Malloc|MallocAsync|MallocManaged|ExtMallocWithFlags|Free|FreeAsync)\s*\(",
    "memset": r"\bhipMemset\w*\s*\(",
    "stream priority": r"\bhip(StreamCreateWithPriority|DeviceGetStreamPriorityRange)\s*\(",
    "host registration": r"\bhipHostRegister\s*\(",
    "uncached memory": r"\bhipDeviceMallocUncached\b",
    "CUDA compatibility layer": r"__HIP_PLATFORM_(AMD|NVIDIA|NVCC|HCC)__|#\s*include\s*<cuda|__CUDA_ARCH__|\bcuda[A-Z]\w*\s*\(",
}

PY_FORBIDDEN = {
    "environment read": r"\bos\.(environ|getenv)\b",
    "stream priority": r"\bStream\([^)]*priority|is_high_priority_stream\s*=\s*True",
    "host registration": r"\bcudaHostRegister\b|\bhipHostRegister\b",
    "oracle import": r"^\s*(from|import)\s+oracle\b",
    "working-file import": r"\b_work\b",
}


@pytest.mark.parametrize("what", sorted(CPP_FORBIDDEN))
def test_library_sources(what):
  assert len(CPP) >= 15
  hits = [f"{os.path.basename(p)}: {m.group(0)}" for p in CPP
          for m in re.finditer(CPP_FORBIDDEN[what], _cpp_code(p), re.M)]
  assert not hits, hits


@pytest.mark.parametrize("what", sorted(PY_FORBIDDEN))
def test_python_layer_sources(what):
  assert len(PY) >= 8
  hits = [f"{os.path.basename(p)}: {m.group(0)}" for p in PY
          for m in re.finditer(PY_FORBIDDEN[what], _py_code(p), re.M)]
  assert not hits, hits


def test_the_patterns_find_what_they_name(tmp_path):
  """Each pattern matches the form it forbids, and the comment stripping
  removes comments but leaves code alone."""
  samples = {
      "environment read": 'const char* v = getenv("LMOE_X");',
      "device allocation": "hipMalloc(&p, n);",
      "memset": "hipMemsetAsync(p, 0, n, st);",
      "stream priority": "hipStreamCreateWithPriority(&s, 0, -1);",
      "host registration": "hipHostRegister(p, n, 0);",
      "uncached memory": "hipExtMallocWithFlags(&p, n, hipDeviceMallocUncached);",
      "CUDA compatibility layer": "#ifdef __HIP_PLATFORM_AMD__",
  }
  for what, code in samples.items():
    assert re.search(CPP_FORBIDDEN[what], code), what
  py = {
      "environment read": 'x = os.environ.get("LMOE_DENSE")',
      "stream priority": "s = torch.cuda.Stream(priority=-1)",
      "oracle import": "from oracle import lmoe_oracle as O",
      "working-file import": "import _work.probe",
  }
  for what, code in py.items():
    assert re.search(PY_FORBIDDEN[what], code, re.M), what
  cpp = tmp_path / "x.hip"
  cpp.write_text('int a = 1;  // getenv("A")\n/* hipMalloc(&p, n); */ int b = getenv("B") != 0;\n')
  hits = re.findall(CPP_FORBIDDEN["environment read"], _cpp_code(cpp))
  assert len(hits) == 1 and not re.search(CPP_FORBIDDEN["device allocation"], _cpp_code(cpp))
  py_file = tmp_path / "x.py"
  py_file.write_text('"""os.environ in a docstring"""\nx = 1  # os.environ\ny = os.environ["B"]\n')
  assert len(re.findall(PY_FORBIDDEN["environment read"], _py_code(py_file))) == 1
