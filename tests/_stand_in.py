"""A stand-in for liblmoe.so that lets the layer's host logic run on CPU
tensors: every lmoe_* compute entry is recorded with its arguments and
returns LMOE_OK without touching memory (outputs keep whatever their
allocation held); workspace-size queries are answered by the real library,
which computes them on the host.  ``install`` also relaxes the operators'
GPU-tensor checks to contiguity / layout checks and pins the stream handle
to 0.  Only CPU tests use it, to check which entry points a configuration
reaches and with which sizes -- never results."""
from lmoe import _lib, ops


class RecordingLib:
  def __init__(self):
    self.calls = []

  def __getattr__(self, name):
    if not name.startswith("lmoe_"):
      raise AttributeError(name)
    if name.endswith("workspace_size"):
      return getattr(_lib.lib(), name)

    def entry(*args):
      self.calls.append((name, args))
      return _lib.OK
    return entry

  def names(self):
    return [n for n, _ in self.calls]


def install(monkeypatch) -> RecordingLib:
  lib = RecordingLib()

  def dev(*ts):
    for t in ts:
      if t is not None and not t.is_contiguous():
        raise ValueError("LatentMoE operators need contiguous tensors")

  def dev_rows(t):
    if t.dim() != 2:
      raise ValueError("expected a 2-D tensor")
    return t.contiguous() if t.stride(1) != 1 or t.stride(0) < t.shape[1] else t

  monkeypatch.setattr(ops, "lib", lambda: lib)
  monkeypatch.setattr(ops, "_stream", lambda: 0)
  monkeypatch.setattr(ops, "_dev", dev)
  monkeypatch.setattr(ops, "_dev_rows", dev_rows)
  return lib
