"""The C-ABI under arbitrary arguments: every entry point, called with sizes
drawn from edge values (negative, zero, one, powers of two and their
neighbours, 2^31, 2^48, 2^62, INT64_MIN / MAX), enums and flags likewise,
floats including NaN and infinities, and each buffer either null or a small
valid host block, returns LMOE_OK or one of the four error codes, never
crashes, and every error leaves a message in lmoe_last_error; the size
queries return -1 or a size.  On a machine without a GPU a call that passes
the host checks stops at its first HIP call (LMOE_ERR_HIP), so this
exercises exactly the checks that stand between a caller and a launch.  It
never runs where a GPU is present: there a call that passes the checks would
launch on these host blocks."""
import ctypes
import math

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from lmoe import _lib

pytestmark = pytest.mark.skipif(torch.cuda.device_count() > 0,
                                reason="host-check fuzzing launches nothing only where no GPU is present")

STATUS = {_lib.OK, _lib.ERR_INVALID, _lib.ERR_UNSUPPORTED, _lib.ERR_HIP, _lib.ERR_WORKSPACE}
EDGE64 = [0, 1, 2, 3, 4, 7, 8, 15, 16, 31, 32, 63, 64, 65, 127, 128, 255, 256, 1000, 1024, 4096, 8192, 65535,
          65536, 65537, (1 << 31) - 1, 1 << 31, 1 << 32, (1 << 48) - 1, 1 << 48, 1 << 62, (1 << 63) - 1,
          -1, -2, -(1 << 31), -(1 << 63)]
EDGE32 = [v for v in EDGE64 if -(1 << 31) <= v < (1 << 31)] + [12345, -7]
FLOATS = [0.0, -0.0, 1.0, 4.0, 25.0, 1e-6, -1.0, 1e30, math.inf, -math.inf, math.nan]

_BLOCK = np.zeros(4096 + 256, dtype=np.uint8)
BLOCK = _BLOCK.ctypes.data + (-_BLOCK.ctypes.data) % 256  # 4 KiB, 256-byte aligned

ENTRY_POINTS = sorted(n for n, (args, ret) in _lib.SIGNATURES.items() if args)


def _arg(kind):
  if kind is _lib.P:
    return st.sampled_from([None, BLOCK])
  if kind is _lib.I64:
    return st.one_of(st.sampled_from(EDGE64), st.integers(-(1 << 63), (1 << 63) - 1))
  if kind is _lib.I32:
    return st.one_of(st.sampled_from(EDGE32), st.integers(-(1 << 31), (1 << 31) - 1))
  return st.one_of(st.sampled_from(FLOATS), st.floats(width=32))


@pytest.mark.parametrize("name", ENTRY_POINTS)
def test_entry_point_returns_a_status_for_any_arguments(name):
  L = _lib.lib()
  argtypes, restype = _lib.SIGNATURES[name]
  fn = getattr(L, name)
  strategy = st.tuples(*[_arg(t) for t in argtypes])

  @settings(max_examples=300, deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.too_slow])
  @given(strategy)
  def check(args):
    rc = fn(*args)
    if restype is _lib.I64:  # size queries
      assert rc == -1 or rc >= 0, (name, args, rc)
      return
    assert rc in STATUS, (name, args, rc)
    if rc != _lib.OK:
      assert L.lmoe_last_error(), (name, args, rc)

  check()


def test_the_buffer_is_what_the_alignment_checks_accept():
  assert BLOCK % 256 == 0 and BLOCK + 4096 <= _BLOCK.ctypes.data + _BLOCK.nbytes
  assert ctypes.sizeof(ctypes.c_void_p) == 8
