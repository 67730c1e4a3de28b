"""Register, scratch and LDS budgets of every kernel in the built liblmoe.so,
read from the AMDGPU metadata note the compiler writes into each gfx950 code
object (per kernel: VGPR and AGPR counts, scratch bytes per lane, spill
counts, static LDS).  A kernel that spills into scratch memory, or whose
registers no longer leave room for the waves per SIMD its schedule counts
on, loses time without changing a single output bit, so no parity test can
see it; here it fails on the CPU.

The same code objects, disassembled, show that the build's
``-packed-fp32-ops`` target feature holds: no packed FP32 add / multiply /
FMA anywhere (those have given silent wrong results on the target boxes).

The code objects come out of the library's .hip_fatbin section: one clang
offload bundle per source file, each holding a host entry and the gfx950 ELF
code object."""
import os
import re
import shutil
import struct
import subprocess

import pytest
import yaml

from lmoe import _lib

LLVM = "/opt/rocm/llvm/bin"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
LDS_PER_CU = 160 * 1024
REGS_PER_SIMD_LANE = 512  # unified VGPR + AGPR file of a CDNA4 SIMD, per lane of a wave64

# the only kernels allowed scratch memory, with the bytes per lane they may use
SCRATCH_ALLOWED = {
    # the build's own dense projection kernel, an A/B beside hipBLASLt and not
    # the layer's default (4 VGPRs spilled)
    r"dense_gemm_kernel": 32,
    # the fused MXFP4 gate/up + SiTU with one tile per block: launched only when
    # the streamed kernel's LDS tile table does not fit beside its 3-slot ring
    # (more than 481 groups); the config-5 layer takes the streamed kernel
    r"grouped_gemm_dma_kernelILi64ELi256ELi1ELi1ELi3E": 96,
}


def _code_objects(tmp_path):
  fatbin = tmp_path / "fatbin.bin"
  r = subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fatbin}", _lib.LIB_PATH,
                      str(tmp_path / "lib_copy.so")], capture_output=True, text=True, timeout=120)
  assert r.returncode == 0, r.stderr
  data = fatbin.read_bytes()
  objs, pos = [], 0
  while (start := data.find(BUNDLE_MAGIC, pos)) >= 0:
    (entries,) = struct.unpack_from("<Q", data, start + len(BUNDLE_MAGIC))
    p = start + len(BUNDLE_MAGIC) + 8
    for _ in range(entries):
      offset, size, triple_len = struct.unpack_from("<QQQ", data, p)
      triple = data[p + 24:p + 24 + triple_len].decode()
      p += 24 + triple_len
      if triple.endswith("gfx950") and size:
        objs.append(data[start + offset:start + offset + size])
    pos = start + len(BUNDLE_MAGIC)
  return objs


def _write_code_objects(tmp_path):
  paths = []
  for i, obj in enumerate(_code_objects(tmp_path)):
    path = tmp_path / f"co_{i}.o"
    path.write_bytes(obj)
    paths.append(path)
  return paths


def _kernels(paths):
  kernels = []
  for path in paths:
    notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", str(path)], capture_output=True, text=True,
                           timeout=120).stdout
    doc = notes[notes.index("---"):]
    end = re.search(r"^\s*\.\.\.\s*$", doc, re.M)
    meta = yaml.safe_load(doc[:end.start()] if end else doc)
    kernels += meta["amdhsa.kernels"]
  return kernels


def _demangle(names):
  if not shutil.which("c++filt"):
    return dict(zip(names, names))
  out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True).stdout.split("\n")
  return dict(zip(names, out))


def _waves_per_simd(k):
  regs = -(-k[".vgpr_count"] // 4) * 4 + k[".agpr_count"]
  return REGS_PER_SIMD_LANE // max(-(-regs // 8) * 8, 8)


@pytest.fixture(scope="module")
def code_objects(tmp_path_factory):
  if not os.path.exists(_lib.LIB_PATH):
    pytest.fail(f"{_lib.LIB_PATH} is not built")
  paths = _write_code_objects(tmp_path_factory.mktemp("codeobj"))
  assert len(paths) >= 10  # one per source file with device code
  return paths


@pytest.fixture(scope="module")
def kernels(code_objects):
  ks = _kernels(code_objects)
  assert len(ks) > 100
  return ks


def test_every_kernel_fits_a_cu(kernels):
  for k in kernels:
    name = k[".name"]
    assert k[".wavefront_size"] == 64, name
    assert not k[".uses_dynamic_stack"], name
    assert k[".group_segment_fixed_size"] <= LDS_PER_CU, name
    assert k[".max_flat_workgroup_size"] <= 1024, name
    assert _waves_per_simd(k) >= 1, name


def test_scratch_only_where_allowed(kernels):
  """No kernel but the two allowed above uses scratch memory: the layer's
  hot path (streamed MXFP4 GEMMs, skinny decode GEMMs, router, dispatch,
  combine, elementwise) keeps every value in registers or LDS."""
  names = _demangle([k[".name"] for k in kernels])
  users = {}
  for k in kernels:
    scratch = k[".private_segment_fixed_size"]
    if scratch == 0:
      continue
    limit = next((v for pat, v in SCRATCH_ALLOWED.items() if re.search(pat, k[".name"])), None)
    users[names[k[".name"]]] = scratch
    assert limit is not None, f"{names[k['.name']]} uses {scratch} B of scratch per lane"
    assert scratch <= limit, f"{names[k['.name']]} uses {scratch} B of scratch per lane (allowed {limit})"
  assert len(users) <= 3, users


def test_streamed_gemm_keeps_three_waves_per_simd(kernels):
  """The streamed grouped GEMM (the config-5 gate/up and down projections)
  runs three persistent blocks of four waves per CU, one wave from each
  block on every SIMD, so that one block's DMA waits overlap another's
  MFMAs: its registers must leave room for three waves per SIMD."""
  streamed = [k for k in kernels if "grouped_gemm_stream_kernel" in k[".name"]]
  assert len(streamed) >= 2  # without and with the SiTU epilogue
  for k in streamed:
    assert k[".private_segment_fixed_size"] == 0, k[".name"]
    assert _waves_per_simd(k) >= 3, (k[".name"], k[".vgpr_count"], k[".agpr_count"])


PACKED_FP32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")

AXPY2 = r"""
#include <hip/hip_runtime.h>
__global__ void axpy2(const float2* __restrict__ x, float2* __restrict__ y, float a, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) { float2 v = x[i], w = y[i]; w.x = a * v.x + w.x; w.y = a * v.y + w.y; y[i] = w; }
}
"""


def test_no_packed_fp32_in_the_library(code_objects, tmp_path):
  """The control first: the same compiler, without the feature switch, turns
  a float2 a*x + y into a packed FP32 FMA that this pattern finds; the
  library's code, built with the switch, holds none."""
  src = tmp_path / "axpy2.hip"
  src.write_text(AXPY2)
  r = subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S", str(src),
                      "-o", str(tmp_path / "axpy2.s")], capture_output=True, text=True, timeout=300)
  assert r.returncode == 0, r.stderr[-2000:]
  assert PACKED_FP32.search((tmp_path / "axpy2.s").read_text())
  instructions = 0
  for path in code_objects:
    dis = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", str(path)], capture_output=True, text=True,
                         timeout=300).stdout
    instructions += dis.count("\n")
    hit = PACKED_FP32.search(dis)
    assert hit is None, f"{path.name}: {hit.group(0)}"
  assert instructions > 100000  # the disassembly is the whole library
