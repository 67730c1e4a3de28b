"""ctypes binding of liblmoe.so (C-ABI declared in include/lmoe.h).

There is no fallback: if the library is missing, every GPU operator raises.
Status codes map to Python exceptions the way the reference's callers expect
(unsupported shape / backend -> NotImplementedError, bad argument ->
ValueError, runtime failure -> RuntimeError).
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblmoe.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                           "include", "lmoe.h")

# enum values (include/lmoe.h)
OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_WORKSPACE = -4
F32 = 0
BF16 = 1
RHS_GKN = 0
RHS_GNK = 1
ACT_SIGMOID = 0
ACT_SOFTMAX = 1
EPI_NONE = 0
EPI_SITU = 1
MXFP4_LDS_DEQUANT = 0
MXFP4_SCALED_MFMA = 1
MXFP4_LDS_DEQUANT_TILED = 2
MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS = 0x100
DISPATCH_FLAG_SKIP_PADDING_ROWS = 0x1
DISPATCH_FLAG_NO_ROWS = 0x2
COMBINE_SCATTER_ADD = 0
COMBINE_SLOT_SUM = 1

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F = ctypes.c_float

SIGNATURES = {
    "lmoe_last_error": ([], ctypes.c_char_p),
    "lmoe_version": ([], I32),
    "lmoe_device_arch_ok": ([], I32),
    "lmoe_ragged_dot": ([P, I32, P, I32, P, I64, I64, I64, I64, I32, P, I32, P], I32),
    "lmoe_ragged_dot_gateup_situ": ([P, P, I32, P, I64, I64, I64, I64, I32, F, F, I32, P, P], I32),
    "lmoe_ragged_dot_fp8_scaled": ([P, P, P, I64, P, I64, I64, I64, I64, I32, I32, F, F, P, P], I32),
    "lmoe_mxfp4_dequant": ([P, P, I64, I64, I64, I64, P, I32, P], I32),
    "lmoe_ragged_dot_mxfp4": ([P, P, P, P, I64, I64, I64, I64, I32, I32, I32, F, F, P, P], I32),
    "lmoe_ragged_dot_mxfp4_rows": ([P, I64, P, P, P, P, I64, I64, I64, I64, I32, I32, I32, F, F, P, P], I32),
    "lmoe_ragged_dot_mxfp4_splitk": ([P, P, P, P, I64, I64, I64, I64, I32, I64, P, I64, I32, F, F, P, P], I32),
    "lmoe_ragged_dot_mxfp4_skinny": ([P, P, P, P, I64, I64, I64, I64, I32, I32, I32, F, F, I64, P, P], I32),
    "lmoe_dispatch_mxfp4_skinny": ([P, P, I32, P, I64, I64, I64, I64, I64, I64, P, P, I64, I64, I32, F, F, I32,
                                    P, P, P, P, P, P, P, P], I32),
    "lmoe_mxfp4_tile": ([P, P, I64, I64, I64, P, P, P], I32),
    "lmoe_mxfp8_scale_bytes": ([I64, I64], I64),
    "lmoe_quantize_mxfp8": ([P, I32, I64, I64, P, P, P], I32),
    "lmoe_quantize_mxfp6": ([P, I32, I64, I64, P, P, P], I32),
    "lmoe_ragged_dot_mxfp6_mxfp4": ([P, P, P, P, P, I64, I64, I64, I64, I32, P, I32, P], I32),
    "lmoe_ragged_dot_mxfp8_mxfp4": ([P, P, P, P, P, I64, I64, I64, I64, I32, I32, F, F, P, I32, P], I32),
    "lmoe_router_topk": ([P, P, I64, I64, I64, I32, I32, F, I32, P, P, P, P], I32),
    "lmoe_router_topk_ld": ([P, I64, P, I64, I64, I64, I32, I32, F, I32, P, P, P, P], I32),
    "lmoe_router_topk_proj": ([P, I64, P, I64, I64, I64, I32, I32, F, I32, P, P, P, I64, I64, P, P], I32),
    "lmoe_dispatch_workspace_size": ([I64, I64, I64], I64),
    "lmoe_dispatch_local": ([P, P, I32, P, I32, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P,
                             I64, P], I32),
    "lmoe_dispatch_local_noalloc": ([P, P, I32, P, I32, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P],
                                    I32),
    "lmoe_dispatch_local_small": ([P, P, I32, P, I32, I64, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, I32, P], I32),
    "lmoe_dispatch_local_rows": ([P, P, I32, P, I32, I64, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, I32, P, I64, P], I32),
    "lmoe_combine_workspace_size": ([I64, I64], I64),
    "lmoe_combine_scatter_add": ([P, I32, P, P, I32, I64, I64, I64, P, I32, P, I64, P], I32),
    "lmoe_combine_slots": ([P, I32, P, P, I32, I64, I64, I64, I32, P, I32, P], I32),
    "lmoe_combine_slots_rms_norm": ([P, I32, P, P, I32, I64, I64, I64, I32, P, F, P, P, I32, P], I32),
    "lmoe_rms_norm": ([P, P, I64, I64, F, I32, P, P], I32),
    "lmoe_dense_blaslt": ([P, I32, P, I32, I64, I64, I64, P, I32, P], I32),
    "lmoe_dense": ([P, P, I64, I64, I64, P, I32, P], I32),
    "lmoe_dense_skinny": ([P, P, I64, I64, I64, P, I32, P], I32),
    "lmoe_situ_and_mul": ([P, P, I64, F, F, I32, P, P], I32),
    "lmoe_add": ([P, P, I64, I32, P, P], I32),
    "lmoe_cast_rows": ([P, I32, I64, I64, I64, P, I32, P], I32),
    "lmoe_transpose": ([P, I64, I64, I64, I32, P, P], I32),
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
  pass


def lib() -> ctypes.CDLL:
  """Load liblmoe.so once; raise LibraryMissing if it has not been built."""
  global _lib
  if _lib is not None:
    return _lib
  with _lock:
    if _lib is None:
      if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python build_lib.py` (or __graft_entry__.build()). "
            "There is no CPU fallback for the LatentMoE kernels.")
      handle = ctypes.CDLL(LIB_PATH)
      for name, (args, res) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = res
      _lib = handle
  return _lib


def check(rc: int, what: str) -> None:
  if rc == OK:
    return
  msg = lib().lmoe_last_error().decode(errors="replace")
  if rc == ERR_UNSUPPORTED:
    raise NotImplementedError(f"{what}: {msg}")
  if rc in (ERR_INVALID, ERR_WORKSPACE):
    raise ValueError(f"{what}: {msg}")
  raise RuntimeError(f"{what}: status {rc}: {msg}")


def declared_functions() -> list[str]:
  """Names of the functions declared in include/lmoe.h."""
  import re
  with open(HEADER_PATH) as f:
    text = f.read()
  return sorted(set(re.findall(r"\b(lmoe_[a-z0-9_]+)\s*\(", text)))
