"""A stand-in for liblmoe.so that computes, on the CPU, for the few entry
points the operators' host-side fallbacks reach: lmoe_ragged_dot (f32 and
bf16, both weight layouts, zero_group), lmoe_situ_and_mul and lmoe_add,
each reading and writing the host buffers behind the pointers the operators
pass, with the oracle's definitions.  Test infrastructure only: it lets the
Python layer's composition (which entry point, which views, dtypes and
casts) be checked for values on a machine without a GPU; the kernels
themselves are checked on the GPU.  Where no GPU is present each call is
first put to the real library, whose host checks run before any launch: a
call the library refuses is refused here too, with its status and message.
Any other entry point raises."""
import ctypes

import numpy as np
import torch

from lmoe import _lib, ops
from oracle import lmoe_oracle as O


# the real library's host checks, only where nothing can launch
_HOST_CHECKS = torch.cuda.device_count() == 0


def _read(ptr, count, dtype):
  """float32 values of `count` elements of `dtype` (F32 / BF16) at ptr."""
  if count == 0:
    return np.zeros(0, np.float32)
  if dtype == _lib.F32:
    return np.ctypeslib.as_array((ctypes.c_float * count).from_address(ptr)).copy()
  if dtype == _lib.BF16:
    return O.bits_to_f32(np.ctypeslib.as_array((ctypes.c_uint16 * count).from_address(ptr)).copy())
  raise ValueError(dtype)


def _write(ptr, values, dtype):
  values = np.ascontiguousarray(values, np.float32).ravel()
  if values.size == 0:
    return
  if dtype == _lib.F32:
    np.ctypeslib.as_array((ctypes.c_float * values.size).from_address(ptr))[:] = values
  elif dtype == _lib.BF16:
    np.ctypeslib.as_array((ctypes.c_uint16 * values.size).from_address(ptr))[:] = O.bf16_bits(values)
  else:
    raise ValueError(dtype)


def _dt(code):
  return "f32" if code == _lib.F32 else "bf16"


class EmulatedLib:
  def __init__(self):
    self.calls = []

  def __getattr__(self, name):
    if not name.startswith("lmoe_"):
      raise AttributeError(name)
    if name.endswith("workspace_size"):
      return getattr(_lib.lib(), name)
    impl = type(self).__dict__.get("_" + name)
    if impl is None:
      raise NotImplementedError(f"{name} is not emulated")
    impl = impl.__get__(self)

    def entry(*args):
      self.calls.append(name)
      if _HOST_CHECKS:
        rc = getattr(_lib.lib(), name)(*args)  # stops at its first HIP call (no device)
        if rc not in (_lib.OK, _lib.ERR_HIP):
          return rc
      return impl(*args)
    return entry

  def names(self):
    return list(self.calls)

  def _lmoe_ragged_dot(self, lhs, lhs_dt, rhs, layout, gs, M, K, N, G, zero_group, out, out_dt, stream):
    a = _read(lhs, M * K, lhs_dt).reshape(M, K)
    w = _read(rhs, G * K * N, lhs_dt)
    # (G, K, N) in memory order, so numpy sums each dot product as the oracle does
    w = w.reshape(G, K, N) if layout == _lib.RHS_GKN else np.ascontiguousarray(w.reshape(G, N, K).transpose(0, 2, 1))
    sizes = np.ctypeslib.as_array((ctypes.c_int32 * G).from_address(gs)).copy() if G else np.zeros(0, np.int32)
    res = O.ragged_dot(a, w, sizes, "f32")
    if 0 <= zero_group < G:
      start = int(sizes[:zero_group].sum())
      res[start:start + int(sizes[zero_group])] = 0
    _write(out, O.cast(res, _dt(out_dt)), out_dt)
    return _lib.OK

  def _lmoe_situ_and_mul(self, gate, up, count, beta, beta_lin, dt, out, stream):
    g, u = _read(gate, count, dt), _read(up, count, dt)
    _write(out, O.situ_and_mul(g, u, beta, beta_lin, _dt(dt)), dt)
    return _lib.OK

  def _lmoe_add(self, a, b, count, dt, out, stream):
    _write(out, O.cast(_read(a, count, dt) + _read(b, count, dt), _dt(dt)), dt)
    return _lib.OK


def install(monkeypatch) -> EmulatedLib:
  lib = EmulatedLib()

  def dev(*ts):
    for t in ts:
      if t is not None and not t.is_contiguous():
        raise ValueError("LatentMoE operators need contiguous tensors")

  monkeypatch.setattr(ops, "lib", lambda: lib)
  monkeypatch.setattr(ops, "_stream", lambda: 0)
  monkeypatch.setattr(ops, "_dev", dev)
  return lib
