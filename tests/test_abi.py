"""C-ABI checks that need no GPU: the library loads, exports every function
include/lmoe.h declares, and rejects bad arguments with the documented status
codes before touching the device."""
import ctypes

import pytest

from lmoe import _lib


@pytest.fixture(scope="module")
def L():
  return _lib.lib()


def test_every_declared_symbol_is_exported(L):
  declared = _lib.declared_functions()
  assert len(declared) >= 16
  missing = [n for n in declared if not hasattr(L, n)]
  assert not missing, missing
  assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)


def test_version_and_error_string(L):
  assert L.lmoe_version() >= 1
  rc = L.lmoe_router_topk(None, None, 4, 8, 9, 0, 1, 1.0, _lib.F32, None, None, None, None)
  assert rc == _lib.ERR_INVALID
  assert b"k=9" in L.lmoe_last_error()


@pytest.mark.parametrize("call,code", [
    (lambda L: L.lmoe_router_topk(None, None, 4, 8192, 2, 0, 1, 1.0, _lib.F32, None, None, None, None),
     _lib.ERR_UNSUPPORTED),
    (lambda L: L.lmoe_router_topk(None, None, 4, 8, 2, 7, 1, 1.0, _lib.F32, None, None, None, None),
     _lib.ERR_INVALID),
    (lambda L: L.lmoe_ragged_dot(None, _lib.BF16, None, 0, None, 16, 12, 16, 2, -1, None, _lib.BF16, None),
     _lib.ERR_INVALID),
    (lambda L: L.lmoe_ragged_dot(ctypes.c_void_p(16), _lib.BF16, ctypes.c_void_p(16), 0,
                                 ctypes.c_void_p(16), 16, 12, 16, 2, -1, ctypes.c_void_p(16), _lib.BF16,
                                 None), _lib.ERR_UNSUPPORTED),
    (lambda L: L.lmoe_ragged_dot(None, _lib.BF16, None, 0, None, 16, 16, 16, 2, 5, None, _lib.BF16, None),
     _lib.ERR_INVALID),
    (lambda L: L.lmoe_dispatch_local(None, None, 0, None, 1, 4, 2, 8, 0, 4, 128, None, None, None, None,
                                     None, None, None, None, 0, None), _lib.ERR_WORKSPACE),
    (lambda L: L.lmoe_ragged_dot_mxfp4(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                       ctypes.c_void_p(16), 16, 96, 16, 1, -1, 0, 0, 0.0, 0.0,
                                       ctypes.c_void_p(16), None), _lib.ERR_UNSUPPORTED),
    (lambda L: L.lmoe_mxfp4_dequant(None, None, 1, 4, 33, 32, None, 0, None), _lib.ERR_INVALID),
    # allocation-free dispatch: sizes beyond its static scratch are refused first
    (lambda L: L.lmoe_dispatch_local_noalloc(None, None, 0, None, 1, 1 << 20, 1, 8, 0, 4096, 128, None, None,
                                             None, None, None, None, None, None), _lib.ERR_WORKSPACE),
    # skinny MXFP4 GEMM: K % 128, group count, flags
    (lambda L: L.lmoe_ragged_dot_mxfp4_skinny(ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256),
                                              ctypes.c_void_p(256), 16, 192, 64, 1, -1, 0, 0, 0.0, 0.0, 0,
                                              ctypes.c_void_p(256), None), _lib.ERR_UNSUPPORTED),
    (lambda L: L.lmoe_ragged_dot_mxfp4_skinny(ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256),
                                              ctypes.c_void_p(256), 16, 128, 64, 1025, -1, 0, 0, 0.0, 0.0, 0,
                                              ctypes.c_void_p(256), None), _lib.ERR_UNSUPPORTED),
    (lambda L: L.lmoe_ragged_dot_mxfp4_skinny(ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256),
                                              ctypes.c_void_p(256), 16, 128, 64, 1, -1, 0x2, 0, 0.0, 0.0, 0,
                                              ctypes.c_void_p(256), None), _lib.ERR_INVALID),
])
def test_argument_validation(L, call, code):
  assert call(L) == code


def test_workspace_sizes(L):
  assert L.lmoe_dispatch_workspace_size(4096, 16, 112) >= 2 * 64 * 112 * 4
  assert L.lmoe_combine_workspace_size(16384, 4096) >= 16384 * 4


def test_ops_refuse_cpu_tensors():
  import torch
  from lmoe import ops
  with pytest.raises(ValueError):
    ops.ragged_dot(torch.zeros(4, 8), torch.zeros(1, 8, 8), torch.zeros(1, dtype=torch.int32))
  with pytest.raises(NotImplementedError):
    ops.ragged_dot(torch.zeros(4, 8), torch.zeros(1, 8, 8), torch.zeros(1, dtype=torch.int32),
                   implementation="xla")


def test_default_split_choice():
  """The split-K heuristic: a split only for one group with few tiles."""
  from lmoe.ops import mxfp4_k_split
  assert [mxfp4_k_split(m, 2048, 7168, 1) for m in (1, 128, 1024, 4096)] == [14, 8, 4, 1]
  assert mxfp4_k_split(8804, 4096, 1024, 113) == 1  # grouped: never
  assert mxfp4_k_split(64, 256, 256, 1) == 1        # too few K steps


@pytest.mark.parametrize("e,lat", [(64, 128), (896, 1024), (4, 4), (896, 2048), (128, 1028), (896, 1026),
                                   (898, 1024), (62, 128)])
def test_router_project_predicate_matches_library(L, e, lat):
  """The layer picks the one-launch router top-k + latent cast
  (lmoe_router_topk_proj) by ops.router_topk_project_supported; on the layout
  the layer passes -- logits and latent projection as the column blocks of one
  (T, E + lat) f32 GEMM output, the projection starting 4 E bytes in -- the
  predicate must agree with the library's own size checks (T = 0: the library
  returns after its checks without touching the device)."""
  from lmoe import ops
  base = 1 << 20
  rc = L.lmoe_router_topk_proj(ctypes.c_void_p(base), e + lat, None, 0, e, min(8, e), _lib.ACT_SIGMOID, 1, 1.0,
                               _lib.F32, None, None, ctypes.c_void_p(base + 4 * e), e + lat, lat,
                               ctypes.c_void_p(2 * base), None)
  want = _lib.OK if ops.router_topk_project_supported(e, lat) else _lib.ERR_UNSUPPORTED
  assert rc == want, L.lmoe_last_error()


@pytest.mark.parametrize("compiler,flags", [("gcc", ["-std=c99", "-pedantic"]), ("g++", ["-std=c++17", "-x", "c++"])])
def test_header_builds_a_c_host_that_links_and_runs(tmp_path, compiler, flags):
  """include/lmoe.h as a C (or C++) host uses it: a program that takes the
  address of every declared function compiles warning-free, links against
  liblmoe.so and runs the host-side calls (version, a refused call and its
  message, the workspace-size queries) without a device."""
  import os
  import re
  import subprocess
  root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
  inc = os.path.join(root, "include")
  libdir = os.path.dirname(_lib.LIB_PATH)
  names = sorted(set(re.findall(r"\b(lmoe_[a-z0-9_]+)\s*\(", open(os.path.join(inc, "lmoe.h")).read())))
  src = tmp_path / "host.c"
  src.write_text("\n".join(
      ["#include <stdio.h>", "#include <string.h>", '#include "lmoe.h"', "typedef void (*fn_t)(void);",
       "static fn_t all[] = {"] + [f"  (fn_t){n}," for n in names] +
      ["};", "int main(void) {",
       "  int rc = lmoe_router_topk(NULL, NULL, 4, 8, 9, LMOE_ACT_SIGMOID, 1, 1.0f, LMOE_F32, NULL, NULL, NULL, NULL);",
       '  printf("%d %d %d %lld %lld\\n", (int)(sizeof(all) / sizeof(all[0])), lmoe_version(), rc,',
       "         (long long)lmoe_dispatch_workspace_size(4096, 16, 112),",
       "         (long long)lmoe_dispatch_workspace_size(-1, 16, 112));",
       '  return rc == LMOE_ERR_INVALID && strstr(lmoe_last_error(), "k=9") != NULL ? 0 : 1;', "}"]) + "\n")
  exe = tmp_path / "host"
  cmd = [compiler, *flags, "-Wall", "-Wextra", "-Werror", f"-I{inc}", str(src), f"-L{libdir}", "-llmoe",
         f"-Wl,-rpath,{libdir}", "-Wl,-rpath-link,/opt/rocm/lib", "-o", str(exe)]
  r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
  assert r.returncode == 0, r.stderr
  r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
  assert r.returncode == 0, (r.stdout, r.stderr)
  count, version, rc, ws, ws_bad = (int(v) for v in r.stdout.split())
  assert count == len(names) == len(_lib.SIGNATURES) and version >= 1 and rc == _lib.ERR_INVALID
  assert ws == _lib.lib().lmoe_dispatch_workspace_size(4096, 16, 112) and ws_bad == -1


def test_integration_bindings_match_the_library():
  """The ctypes bindings the integration guide shows a maintainer (argtypes lists and
  example calls) agree with the library's signatures, so copying them binds
  the entry points correctly."""
  import os
  import re
  root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
  txt = open(os.path.join(root, "INTEGRATION.md")).read()
  kinds = {"P": _lib.P, "I64": _lib.I64, "I32": _lib.I32, "ctypes.c_float": _lib.F}
  bound = re.findall(r"lib\.(lmoe_\w+)\.argtypes = \[(.*?)\]", txt, re.S)
  assert len(bound) >= 5
  for name, body in bound:
    toks = [t.strip() for t in body.replace("\n", " ").split(",") if t.strip()]
    assert [kinds[t] for t in toks] == _lib.SIGNATURES[name][0], name
  calls = re.findall(r"rc = lib\.(lmoe_\w+)\((.*?)\)\n", txt, re.S)
  assert len(calls) >= 5
  for name, body in calls:
    depth, n = 0, 1
    for ch in body:
      depth += ch in "(["
      depth -= ch in ")]"
      n += ch == "," and depth == 0
    assert n == len(_lib.SIGNATURES[name][0]), (name, n)


def test_header_prototypes_match_the_ctypes_bindings():
  """Every prototype in include/lmoe.h has the parameter list and return
  type the ctypes binding declares (pointer / int64_t / int / float, in
  order): a binding that disagreed would pass its arguments in the wrong
  registers without any error."""
  import os
  import re
  root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
  hdr = re.sub(r"/\*.*?\*/", "", open(os.path.join(root, "include", "lmoe.h")).read(), flags=re.S)
  protos = re.findall(r"([\w\s\*]+?)\b(lmoe_\w+)\s*\(([^;{]*?)\)\s*;", hdr, re.S)
  scalar = {"int64_t": _lib.I64, "int": _lib.I32, "float": _lib.F}

  def kind(decl):
    decl = " ".join(decl.replace("const ", "").split())
    if "*" in decl:
      return _lib.P
    return scalar.get(decl.split(" ")[0], decl)

  assert len(protos) == len(_lib.SIGNATURES)
  for ret, name, params in protos:
    args = [kind(p) for p in params.split(",") if p.strip() and p.strip() != "void"]
    ret = " ".join(ret.split())
    ret_kind = ctypes.c_char_p if "char" in ret else scalar.get(ret.split(" ")[-1], ret)
    assert (args, ret_kind) == _lib.SIGNATURES[name], name
