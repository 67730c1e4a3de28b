"""MXFP4 checkpoint loader (lmoe.loader) on CPU.

Checkpoints are written by the ``safetensors`` library itself, an independent
writer of the format the reference's fetcher parses
(05_ragged_dot_on_tpu/fetch_real_mxfp4_expert_weights.py:51-67): reading its
files back byte-exact pins the header-length / data-section offset rule and
the key table (README.md:303-318, w1 = gate, w3 = up, w2 = down).  The
tensor-by-tensor path (experts split over shards, non-contiguous spans) is
covered by a sharded checkpoint with an index file.
"""
import json
import os

import numpy as np
import pytest

from safetensors.numpy import save_file

from lmoe import loader

LAYER, I, LAT = 3, 64, 128


def _expert(rng):
  u8 = lambda *s: rng.integers(0, 256, s, dtype=np.uint8)
  return {"w1.weight_packed": u8(I, LAT // 2), "w1.weight_scale": u8(I, LAT // 32),
          "w3.weight_packed": u8(I, LAT // 2), "w3.weight_scale": u8(I, LAT // 32),
          "w2.weight_packed": u8(LAT, I // 2), "w2.weight_scale": u8(LAT, I // 32)}


def _key(e, name, layer=LAYER):
  return f"language_model.model.layers.{layer}.block_sparse_moe.experts.{e}.{name}"


def _checkpoint(rng, n_experts=24):
  tensors, experts = {}, {}
  for e in range(n_experts):
    experts[e] = _expert(rng)
    tensors.update({_key(e, k): v for k, v in experts[e].items()})
  # neighbours the loader must skip: another layer's expert, dense weights of
  # other dtypes that sort before the U8 tensors in the data section
  tensors.update({_key(0, k, LAYER + 1): v for k, v in _expert(rng).items()})
  tensors["language_model.model.layers.3.self_attn.q_proj.weight"] = rng.standard_normal((32, 48)).astype(np.float32)
  tensors["language_model.model.layers.3.block_sparse_moe.gate.weight"] = rng.standard_normal((24, 40)).astype(np.float16)
  return tensors, experts


def _check(got, experts, ids, padding=True):
  want_gu_p = np.stack([np.concatenate([experts[e]["w1.weight_packed"], experts[e]["w3.weight_packed"]]) for e in ids])
  want_gu_s = np.stack([np.concatenate([experts[e]["w1.weight_scale"], experts[e]["w3.weight_scale"]]) for e in ids])
  want_d_p = np.stack([experts[e]["w2.weight_packed"] for e in ids])
  want_d_s = np.stack([experts[e]["w2.weight_scale"] for e in ids])
  L = len(ids)
  for name, want in (("gu_packed", want_gu_p), ("gu_scale", want_gu_s), ("down_packed", want_d_p),
                     ("down_scale", want_d_s)):
    t = got[name].numpy()
    assert t.dtype == np.uint8
    assert t.shape == ((L + 1,) if padding else (L,)) + want.shape[1:], name
    assert np.array_equal(t[:L], want), name
    if padding:
      assert not t[L].any(), name


def test_single_file_local_range(tmp_path):
  rng = np.random.default_rng(0)
  tensors, experts = _checkpoint(rng)
  path = str(tmp_path / "model.safetensors")
  save_file(tensors, path, metadata={"format": "pt"})
  ids = list(range(16, 24))  # a local shard: experts [16, 24)
  got = loader.load_mxfp4_experts(path, LAYER, ids, device="cpu")
  _check(got, experts, ids)
  assert got["gu_packed"].shape == (9, 2 * I, LAT // 2)
  got = loader.load_mxfp4_experts(path, LAYER, [5, 2, 11], device="cpu", padding_expert=False)
  _check(got, experts, [5, 2, 11], padding=False)


def test_header_offsets_are_relative_to_the_data_section(tmp_path):
  rng = np.random.default_rng(1)
  tensors, experts = _checkpoint(rng, 4)
  path = str(tmp_path / "m.safetensors")
  save_file(tensors, path)
  header, start = loader.read_header(path)
  with open(path, "rb") as f:
    n = int.from_bytes(f.read(8), "little")
    f.seek(start + header[_key(2, "w2.weight_scale")]["data_offsets"][0])
    raw = f.read(LAT * I // 32)
  assert start == 8 + n
  assert np.array_equal(np.frombuffer(raw, np.uint8).reshape(LAT, I // 32), experts[2]["w2.weight_scale"])
  # an expert's six tensors lie back to back in this file: one span covers them
  offs = sorted(header[_key(2, k)]["data_offsets"] for k in experts[2])
  assert all(a[1] == b[0] for a, b in zip(offs, offs[1:]))


def test_sharded_checkpoint_with_index(tmp_path):
  """gate/up of every expert in one shard, down in another: the six tensors of
  an expert span two files, so they are read one by one."""
  rng = np.random.default_rng(2)
  tensors, experts = _checkpoint(rng, 8)
  a = {k: v for k, v in tensors.items() if ".w2." not in k}
  b = {k: v for k, v in tensors.items() if ".w2." in k}
  save_file(a, str(tmp_path / "model-00001-of-00002.safetensors"))
  save_file(b, str(tmp_path / "model-00002-of-00002.safetensors"))
  wm = {k: "model-00001-of-00002.safetensors" for k in a}
  wm.update({k: "model-00002-of-00002.safetensors" for k in b})
  with open(tmp_path / "model.safetensors.index.json", "w") as f:
    json.dump({"metadata": {}, "weight_map": wm}, f)
  got = loader.load_mxfp4_experts(str(tmp_path), LAYER, range(2, 6), device="cpu")
  _check(got, experts, [2, 3, 4, 5])
  os.remove(tmp_path / "model.safetensors.index.json")  # directory without an index
  got = loader.load_mxfp4_experts(str(tmp_path), LAYER, range(2, 6), device="cpu")
  _check(got, experts, [2, 3, 4, 5])


def test_non_contiguous_expert_in_one_file(tmp_path):
  """Interleaved experts (a writer that orders keys differently): the single
  span check fails and the reader falls back to per-tensor reads."""
  rng = np.random.default_rng(3)
  _, experts = _checkpoint(rng, 3)
  # hand-written file, tensors in the order w1(e0) w1(e1) ... so e0 is split
  order = [(e, k) for k in experts[0] for e in range(3)]
  header, blobs, off = {}, [], 0
  for e, k in order:
    v = experts[e][k]
    header[_key(e, k)] = {"dtype": "U8", "shape": list(v.shape), "data_offsets": [off, off + v.nbytes]}
    blobs.append(v.tobytes())
    off += v.nbytes
  hb = json.dumps(header).encode()
  hb += b" " * (-len(hb) % 8)
  path = tmp_path / "x.safetensors"
  path.write_bytes(len(hb).to_bytes(8, "little") + hb + b"".join(blobs))
  got = loader.load_mxfp4_experts(str(path), LAYER, [1, 0, 2], device="cpu")
  _check(got, experts, [1, 0, 2])


def test_errors(tmp_path):
  rng = np.random.default_rng(4)
  tensors, experts = _checkpoint(rng, 4)
  path = str(tmp_path / "m.safetensors")
  save_file(tensors, path)
  with pytest.raises(KeyError, match="expert 7"):
    loader.load_mxfp4_experts(path, LAYER, [1, 7], device="cpu")
  with pytest.raises(KeyError):
    loader.load_mxfp4_experts(path, LAYER + 2, [0], device="cpu")
  with pytest.raises(ValueError, match="no experts"):
    loader.load_mxfp4_experts(path, LAYER, [], device="cpu")
  # a shape that differs from the first expert's
  bad = dict(tensors)
  bad[_key(2, "w2.weight_scale")] = np.zeros((LAT, I // 16), np.uint8)
  save_file(bad, str(tmp_path / "bad.safetensors"))
  with pytest.raises(ValueError, match="expert 2"):
    loader.load_mxfp4_experts(str(tmp_path / "bad.safetensors"), LAYER, [0, 2], device="cpu")
  # gate scales inconsistent with the packed K
  bad = dict(tensors)
  bad[_key(0, "w1.weight_scale")] = np.zeros((I, LAT // 16), np.uint8)
  save_file(bad, str(tmp_path / "bad2.safetensors"))
  with pytest.raises(ValueError, match="gate/up shapes"):
    loader.load_mxfp4_experts(str(tmp_path / "bad2.safetensors"), LAYER, [0], device="cpu")
  # not U8
  bad = dict(tensors)
  bad[_key(1, "w3.weight_packed")] = experts[1]["w3.weight_packed"].astype(np.int8)
  save_file(bad, str(tmp_path / "bad3.safetensors"))
  with pytest.raises(ValueError, match="U8"):
    loader.load_mxfp4_experts(str(tmp_path / "bad3.safetensors"), LAYER, [1], device="cpu")
  # truncated file: the header is intact, the data section is short
  raw = open(path, "rb").read()
  (tmp_path / "trunc.safetensors").write_bytes(raw[:-100])
  with pytest.raises(ValueError, match="outside the file"):  # the other layer's expert is stored last
    loader.load_mxfp4_experts(str(tmp_path / "trunc.safetensors"), LAYER + 1, [0], device="cpu")
  (tmp_path / "short.safetensors").write_bytes(b"\x05\x00")
  with pytest.raises(ValueError, match="not a safetensors"):
    loader.read_header(str(tmp_path / "short.safetensors"))
  (tmp_path / "huge.safetensors").write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
  with pytest.raises(ValueError, match="exceeds"):
    loader.read_header(str(tmp_path / "huge.safetensors"))


def _raw_file(path, header, data=b""):
  h = json.dumps(header).encode()
  path.write_bytes(len(h).to_bytes(8, "little") + h + data)
  return str(path)


def test_malformed_headers_are_refused(tmp_path):
  """Headers that are valid JSON but not the safetensors layout are refused
  with ValueError naming the entry, before any tensor is read."""
  good = {"dtype": "U8", "shape": [2, 4], "data_offsets": [0, 8]}
  assert loader.read_header(_raw_file(tmp_path / "ok.safetensors", {"t": good}, bytes(8)))[0] == {"t": good}
  bad_entries = [
      [1, 2],                                               # not an object
      {"t": "U8"},                                          # entry not an object
      {"t": {"shape": [2, 4], "data_offsets": [0, 8]}},     # no dtype
      {"t": dict(good, shape=[2, -4])},                     # negative dim
      {"t": dict(good, shape=[2, 4.0])},                    # float dim
      {"t": dict(good, data_offsets=[8, 0])},               # hi < lo
      {"t": dict(good, data_offsets=[-8, 0])},              # negative offset
      {"t": dict(good, data_offsets=[0, 8, 16])},           # three offsets
      {"t": dict(good, data_offsets=[0, True])},            # bool offset
  ]
  for i, h in enumerate(bad_entries):
    with pytest.raises(ValueError, match="header"):
      loader.read_header(_raw_file(tmp_path / f"bad{i}.safetensors", h, bytes(8)))


def test_byte_count_must_match_the_shape(tmp_path):
  names = {f"{w}.weight_{p}": (n, m) for w, n, m in (("w1", I, LAT), ("w3", I, LAT), ("w2", LAT, I))
           for p in ("packed", "scale")}
  header, off, blob = {}, 0, b""
  for name, (n, m) in names.items():
    cols = m // 2 if name.endswith("packed") else m // 32
    nbytes = n * cols - (1 if name == "w2.weight_scale" else 0)  # one byte short
    header[_key(0, name)] = {"dtype": "U8", "shape": [n, cols], "data_offsets": [off, off + nbytes]}
    off += nbytes
    blob += bytes(nbytes)
  path = _raw_file(tmp_path / "short_tensor.safetensors", header, blob)
  with pytest.raises(ValueError, match="bytes for shape"):
    loader.load_mxfp4_experts(path, LAYER, [0], device="cpu")


def test_index_cannot_name_files_outside_the_checkpoint(tmp_path):
  rng = np.random.default_rng(5)
  tensors, _ = _checkpoint(rng, 1)
  (tmp_path / "elsewhere").mkdir()
  save_file(tensors, str(tmp_path / "elsewhere" / "x.safetensors"))
  ckpt = tmp_path / "ckpt"
  ckpt.mkdir()
  (ckpt / "model.safetensors.index.json").write_text(
      json.dumps({"weight_map": {k: "../elsewhere/x.safetensors" for k in tensors}}))
  with pytest.raises(ValueError, match="not a file of the checkpoint directory"):
    loader.load_mxfp4_experts(str(ckpt), LAYER, [0], device="cpu")


def test_hostile_headers_are_refused(tmp_path):
  """A header nested past the JSON parser's recursion limit, and a header
  longer than the format's 100 MB cap (a sparse file, so nothing that large
  is written or read), raise ValueError like any other malformed header."""
  import struct
  deep = tmp_path / "deep.safetensors"
  body = b"[" * 200000 + b"]" * 200000
  deep.write_bytes(struct.pack("<Q", len(body)) + body)
  with pytest.raises(ValueError, match="nests too deeply"):
    loader.read_header(str(deep))
  big = tmp_path / "big.safetensors"
  n = loader.MAX_HEADER_BYTES + 1
  with open(big, "wb") as f:
    f.write(struct.pack("<Q", n))
    f.seek(8 + n)
    f.write(b"\0")
  with pytest.raises(ValueError, match="exceeds the format's"):
    loader.read_header(str(big))


def test_arbitrary_headers_parse_or_raise_value_error(tmp_path):
  """Random header entries (dtype, shape, offsets inside and outside the
  data) over random data bytes: every file parses and every tensor reads, or
  the loader raises ValueError / NotImplementedError (an unknown dtype) --
  nothing else escapes."""
  import json
  import struct
  from hypothesis import HealthCheck, given, settings
  from hypothesis import strategies as st
  path = tmp_path / "f.safetensors"
  seen = {"ok": 0}
  size = {"U8": 1, "F32": 4, "BF16": 2, "I32": 4}
  shape = st.lists(st.integers(0, 6), max_size=3)

  @settings(max_examples=300, deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.function_scoped_fixture])
  @given(st.lists(st.tuples(st.sampled_from(["U8", "F32", "BF16", "I32", "U8", "F32", "F8_E4M3", 7]),
                            st.one_of(shape, shape, shape, st.integers(0, 3)),
                            st.integers(-2, 40), st.integers(-2, 40), st.sampled_from([True, True, True, False])),
                  max_size=4),
         st.binary(min_size=64, max_size=96), st.sampled_from([0, 0, 0, -1, 1, -3]))
  def run(entries, payload, skew):
    h = {}
    for i, (dt, sh, lo, hi, fits) in enumerate(entries):
      if fits and isinstance(sh, list) and dt in size and lo >= 0:  # offsets that match the shape
        hi = lo + int(np.prod(sh)) * size[dt]
      h[f"t{i}"] = {"dtype": dt, "shape": sh, "data_offsets": [lo, hi]}
    body = json.dumps(h).encode()
    path.write_bytes(struct.pack("<Q", max(len(body) + skew, 0)) + body + payload)
    try:
      f = loader._File(str(path))
    except ValueError:
      return
    for name in f.header:
      try:
        f.tensor(name)
        seen["ok"] += 1
      except (ValueError, NotImplementedError):
        pass

  run()
  assert seen["ok"] > 20
