"""Helpers shared by the GPU parity tests: numpy <-> torch with bf16 handled
as exact bit patterns, and the reference's error metric."""
import numpy as np
import torch

from oracle import lmoe_oracle as O


def to_dev(a, dtype="f32", device="cuda"):
  """numpy (float32 values; bf16-exact when dtype == "bf16") -> torch on device."""
  a = np.asarray(a)
  if a.dtype.kind in "iub":
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)
  if dtype == "bf16":
    bits = O.bf16_bits(a).view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(bits)).to(device).view(torch.bfloat16)
  return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def to_np(t):
  """torch -> numpy float32 (bf16 converted exactly) or integer/bool arrays."""
  t = t.detach()
  if t.dtype == torch.bfloat16:
    return O.bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
  return t.cpu().numpy()


def agreement(out, ref):
  """Fraction of the elements of ``out`` bit-equal to ``ref`` (NaN never is)."""
  out, ref = np.asarray(out), np.asarray(ref)
  assert out.shape == ref.shape, (out.shape, ref.shape)
  return float(np.mean(out == ref)) if ref.size else 1.0


def max_rel(out, ref):
  """max|out - ref| / max|ref| (benchmark_harness.py:192-199)."""
  out = np.asarray(out, np.float64)
  ref = np.asarray(ref, np.float64)
  denom = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
  return float(np.max(np.abs(out - ref))) / denom if ref.size else 0.0


def banner(msg):
  print(f"[gpu-test] {msg}", flush=True)
