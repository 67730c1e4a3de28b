"""MXFP4 expert weights from a safetensors checkpoint, in this build's layout.

The checkpoint format follows the reference's fetcher
(05_ragged_dot_on_tpu/fetch_real_mxfp4_expert_weights.py:51-67, 78-112) and
its key table (README.md:303-318):

* a safetensors file is an 8-byte little-endian header length, a JSON header
  mapping each tensor name to {dtype, shape, data_offsets}, then the data
  section; ``data_offsets`` are relative to the start of the data section
  (byte ``8 + header_len``), not to the start of the file;
* routed expert e of layer l is
  ``<prefix>layers.{l}.block_sparse_moe.experts.{e}.{w1,w3,w2}.weight_{packed,scale}``
  with w1 = gate, w3 = up, w2 = down, all U8, in the checkpoint (out, in)
  orientation: packed (N, K/2) with the low nibble first, E8M0 scales
  (N, K/32);
* an expert's six tensors are usually stored back to back, so one read per
  expert fetches all of them (the reader checks this and otherwise reads
  tensor by tensor).

``load_mxfp4_experts`` returns the dict ``LocalShardLatentMoE(expert_format=
"mxfp4")`` takes: gate and up concatenated on N ([gate | up], the fused
gate/up layout), plus the trailing all-zero padding expert (the zero group of
the local-shard dispatch).  The layer re-tiles these once for its kernels.
Large files are memory-mapped, never read whole.
"""

from __future__ import annotations

import json
import os
import struct
from typing import Iterable

import numpy as np
import torch

EXPERT_KEY = "{prefix}layers.{layer}.block_sparse_moe.experts.{expert}.{w}.weight_{part}"
DEFAULT_PREFIX = "language_model.model."
_ROLES = {"gate": "w1", "up": "w3", "down": "w2"}
_DTYPES = {"U8": np.uint8, "I8": np.int8, "BF16": np.uint16, "F16": np.float16, "F32": np.float32,
           "I32": np.int32, "I64": np.int64}
# the safetensors format's limit on the JSON header
MAX_HEADER_BYTES = 100_000_000


def read_header(path: str) -> tuple[dict, int]:
  """(header without "__metadata__", absolute offset of the data section).
  Every entry is checked to be {dtype: str, shape: [int >= 0, ...],
  data_offsets: [lo, hi]} with 0 <= lo <= hi; the offsets are checked against
  the file when a tensor is read."""
  with open(path, "rb") as f:
    raw = f.read(8)
    if len(raw) != 8:
      raise ValueError(f"{path}: not a safetensors file (shorter than 8 bytes)")
    (n,) = struct.unpack("<Q", raw)
    size = os.fstat(f.fileno()).st_size
    if n > size - 8:
      raise ValueError(f"{path}: header length {n} exceeds the file size {size}")
    if n > MAX_HEADER_BYTES:
      raise ValueError(f"{path}: header length {n} exceeds the format's {MAX_HEADER_BYTES} bytes")
    try:
      header = json.loads(f.read(n))
    except RecursionError:
      raise ValueError(f"{path}: the header nests too deeply") from None
  if not isinstance(header, dict):
    raise ValueError(f"{path}: the header is not a JSON object")
  header.pop("__metadata__", None)
  is_int = lambda v: isinstance(v, int) and not isinstance(v, bool)
  for name, meta in header.items():
    ok = (isinstance(meta, dict) and isinstance(meta.get("dtype"), str) and isinstance(meta.get("shape"), list)
          and all(is_int(d) and d >= 0 for d in meta["shape"]) and isinstance(meta.get("data_offsets"), list)
          and len(meta["data_offsets"]) == 2 and all(is_int(o) for o in meta["data_offsets"])
          and 0 <= meta["data_offsets"][0] <= meta["data_offsets"][1])
    if not ok:
      raise ValueError(f"{path}: malformed header entry {name!r}: {meta!r}")
  return header, 8 + n


class _File:
  """One safetensors file: header plus a read-only memory map."""

  def __init__(self, path: str):
    self.path = path
    self.header, self.data_start = read_header(path)
    self.map = np.memmap(path, dtype=np.uint8, mode="r")

  def span(self, lo: int, hi: int) -> np.ndarray:
    a, b = self.data_start + lo, self.data_start + hi
    if lo < 0 or hi < lo or b > self.map.shape[0]:
      raise ValueError(f"{self.path}: data range [{lo}, {hi}) outside the file")
    return self.map[a:b]

  def tensor(self, name: str, raw: np.ndarray | None = None, base: int = 0) -> np.ndarray:
    meta = self.header[name]
    dt = _DTYPES.get(meta["dtype"])
    if dt is None:
      raise NotImplementedError(f"{name}: dtype {meta['dtype']}")
    lo, hi = meta["data_offsets"]
    buf = raw[lo - base:hi - base] if raw is not None else self.span(lo, hi)
    count = int(np.prod(meta["shape"])) if meta["shape"] else 1
    if buf.nbytes != count * np.dtype(dt).itemsize:
      raise ValueError(f"{name}: {buf.nbytes} bytes for shape {meta['shape']} {meta['dtype']}")
    return np.frombuffer(buf.tobytes(), dtype=dt).reshape(meta["shape"])


def _open_checkpoint(path: str) -> tuple[list[_File], dict[str, _File]]:
  """A .safetensors file, or a directory with model.safetensors.index.json
  (weight_map: name -> file) or with one or more .safetensors files."""
  files: list[str]
  if os.path.isdir(path):
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
      with open(index) as f:
        wm = json.load(f)["weight_map"]
      files = sorted({os.path.join(path, v) for v in wm.values()})
      root = os.path.realpath(path)
      for fp in files:
        if os.path.dirname(os.path.realpath(fp)) != root:
          raise ValueError(f"{index}: shard {fp!r} is not a file of the checkpoint directory")
    else:
      files = sorted(os.path.join(path, f) for f in os.listdir(path) if f.endswith(".safetensors"))
  else:
    files = [path]
  if not files:
    raise FileNotFoundError(f"no .safetensors files under {path}")
  opened = [_File(f) for f in files]
  owner = {}
  for fh in opened:
    for name in fh.header:
      owner[name] = fh
  return opened, owner


def _expert_tensors(owner: dict, layer: int, expert: int, prefix: str) -> dict[str, np.ndarray]:
  names = {(role, part): EXPERT_KEY.format(prefix=prefix, layer=layer, expert=expert, w=w, part=part)
           for role, w in _ROLES.items() for part in ("packed", "scale")}
  missing = [n for n in names.values() if n not in owner]
  if missing:
    raise KeyError(f"expert {expert} of layer {layer}: missing {missing}")
  fhs = {id(owner[n]): owner[n] for n in names.values()}
  out = {}
  if len(fhs) == 1:
    fh = next(iter(fhs.values()))
    offs = [fh.header[n]["data_offsets"] for n in names.values()]
    lo, hi = min(o[0] for o in offs), max(o[1] for o in offs)
    if hi - lo == sum(o[1] - o[0] for o in offs):  # contiguous: one read for the six tensors
      raw = np.asarray(fh.span(lo, hi))
      return {k: fh.tensor(n, raw, lo) for k, n in names.items()}
  for k, n in names.items():
    out[k] = owner[n].tensor(n)
  return out


def load_mxfp4_experts(path: str, layer: int, experts: Iterable[int], device="cuda",
                       prefix: str = DEFAULT_PREFIX, padding_expert: bool = True) -> dict:
  """Routed experts ``experts`` (e.g. range(local_start, local_start + L)) of
  ``layer`` as {"gu_packed" (L(+1), 2I, lat/2), "gu_scale" (L(+1), 2I,
  lat/32), "down_packed" (L(+1), lat, I/2), "down_scale" (L(+1), lat, I/32)},
  uint8 tensors on ``device``; with ``padding_expert`` a trailing zero expert
  (the local-shard padding bucket) is appended."""
  _, owner = _open_checkpoint(path)
  experts = list(experts)
  if not experts:
    raise ValueError("no experts requested")
  gu_p, gu_s, dn_p, dn_s = [], [], [], []
  shapes = None
  for e in experts:
    t = _expert_tensors(owner, layer, e, prefix)
    g_p, g_s, u_p, u_s = t["gate", "packed"], t["gate", "scale"], t["up", "packed"], t["up", "scale"]
    d_p, d_s = t["down", "packed"], t["down", "scale"]
    sh = (g_p.shape, g_s.shape, u_p.shape, u_s.shape, d_p.shape, d_s.shape)
    if shapes is None:
      shapes = sh
      i, half_lat = g_p.shape
      if u_p.shape != g_p.shape or g_s.shape != (i, half_lat * 2 // 32) or u_s.shape != g_s.shape:
        raise ValueError(f"expert {e}: gate/up shapes {sh[:4]} are not (I, lat/2) + (I, lat/32)")
      if d_p.shape != (half_lat * 2, i // 2) or d_s.shape != (half_lat * 2, i // 32):
        raise ValueError(f"expert {e}: down shapes {sh[4:]} are not (lat, I/2) + (lat, I/32)")
    elif sh != shapes:
      raise ValueError(f"expert {e}: shapes {sh} differ from expert {experts[0]}'s {shapes}")
    for arr in (g_p, g_s, u_p, u_s, d_p, d_s):
      if arr.dtype != np.uint8:
        raise ValueError(f"expert {e}: MXFP4 tensors are U8, got {arr.dtype}")
    gu_p.append(np.concatenate([g_p, u_p], 0))
    gu_s.append(np.concatenate([g_s, u_s], 0))
    dn_p.append(d_p)
    dn_s.append(d_s)
  if padding_expert:
    for lst in (gu_p, gu_s, dn_p, dn_s):
      lst.append(np.zeros_like(lst[0]))
  to = lambda lst: torch.from_numpy(np.ascontiguousarray(np.stack(lst))).to(device)
  return {"gu_packed": to(gu_p), "gu_scale": to(gu_s), "down_packed": to(dn_p), "down_scale": to(dn_s)}
