"""GPU parity of the reference's block-scaled fp8 weight path (a19):
``PallasMosaicTpuV2RaggedDot()(lhs, rhs_q, group_sizes=..., rhs_scale=...)``
with rhs_q (G, K, N) float8_e4m3fn and rhs_scale (G, K/bs, 1, N) float32,
bs = K (rd.py:2789-2811) or 32 (rd.py:2836-2953).

* the in-kernel dequantisation bf16(f32(q) * scale) is bit-exact: with
  one-hot activations every output is a single weight;
* whole ragged_dots (multiple groups, an empty group, tail rows, the padding
  bucket, the SiTU epilogue) within the bf16 bar (2e-2 max-relative) of the
  oracle, which restates the reference's own check (dequantise, then
  ragged_dot);
* the op class dispatches by the scale dtype: f32 scales -> this fp8 path,
  uint8 E8M0 scales -> MXFP4; ``maybe_quantize_lhs`` -> the MXFP8 x MXFP4 path.
"""
import numpy as np
import pytest
import torch

from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


def _quantize_like_reference(w, bs):
  """The reference's fp8 quantisation (rd.py:2786-2795, 2900-2915):
  scale = amax / 448 per (group, block, column), q = clip(w / scale) cast to
  float8_e4m3fn (torch's cast: round to nearest even)."""
  g, k, n = w.shape
  blocks = w.reshape(g, k // bs, bs, n)
  scale = (np.abs(blocks).max(axis=2) / 448.0).astype(np.float32)  # (G, K/bs, N)
  scale = np.where(scale > 0, scale, np.float32(1.0))
  q = np.clip(blocks / scale[:, :, None, :], -448.0, 448.0).astype(np.float32)
  codes = torch.from_numpy(q).to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(g, k, n)
  return codes, scale[:, :, None, :]


@pytest.mark.parametrize("bs", [256, 32])
def test_fp8_dequant_bit_exact_one_hot(gpu_device, bs):
  """lhs row r = e_r: out[r, n] = bf16(f32(q[r, n]) * scale[r // bs, n]),
  every code except NaN in every column, scales spanning 1e-30..1e30 with
  subnormal products, negative and zero scales.  Values are compared (-0 ==
  +0): the one-hot f32 sum adds +0 products, which turns a -0 weight into +0."""
  from lmoe import ops
  rng = np.random.default_rng(bs)
  k, n = 256, 128
  codes = ((np.arange(k)[:, None] + 5 * np.arange(n)[None, :]) % 256).astype(np.uint8)[None]
  codes[(codes & 0x7F) == 0x7F] = 0x38  # NaN codes -> 1.0
  nb = k // bs
  scale = (rng.standard_normal((1, nb, 1, n)) * 10.0 ** rng.integers(-30, 30, (1, nb, 1, n))).astype(np.float32)
  scale[0, 0, 0, :3] = [0.0, -1.0, 2.0 ** -140]
  lhs = np.eye(k, dtype=np.float32)
  out = ops.ragged_dot_fp8_scaled(to_dev(lhs, "bf16"), to_dev(codes).view(torch.float8_e4m3fn), to_dev(scale),
                                  to_dev(np.array([k], np.int32)))
  want = O.dequantize_fp8_blockscaled(codes, scale)[0]
  got = to_np(out)
  bad = np.argwhere(got != want)
  for r, c in bad[:12]:
    print(f"  k={r} n={c} code=0x{codes[0, r, c]:02x} scale={scale[0, r // bs, 0, c]:.6e} "
          f"got={got[r, c]:.6e} want={want[r, c]:.6e}")
  print(f"  {len(bad)} of {got.size} differ")
  assert len(bad) == 0


FP8_CASES = [
    # m, k, n, g, bs, tail rows, situ, zero_group
    (300, 256, 128, 4, 32, 9, False, -1),
    (300, 256, 128, 4, 256, 0, False, 3),
    (148, 3584, 3072, 2, 32, 0, False, 1),     # the reference's probe shape (74 rows + padding bucket)
    (148, 3584, 3072, 2, 3584, 0, False, 1),
    (500, 1024, 1024, 9, 32, 11, True, -1),   # [gate | up] with the SiTU epilogue
    (77, 72, 40, 3, 8, 5, False, -1),         # partial tiles in every dimension
]


@pytest.mark.parametrize("m,k,n,g,bs,tail,situ,zg", FP8_CASES)
def test_fp8_scaled_ragged_dot_matches_oracle(gpu_device, m, k, n, g, bs, tail, situ, zg):
  from lmoe import ops
  banner(f"fp8 ragged_dot m={m} k={k} n={n} g={g} bs={bs} situ={situ} zero_group={zg}")
  rng = np.random.default_rng(m + k + n + bs)
  gs = rng.multinomial(m - tail, np.ones(g) / g).astype(np.int32)
  if g > 2:
    gs[1] = 0
  w = O.bf16_round(rng.standard_normal((g, k, n)) * 0.02)
  codes, scale = _quantize_like_reference(w, bs)
  lhs = O.bf16_round(rng.standard_normal((m, k)) * 0.02 * 50)
  if zg >= 0:
    start = int(gs[:zg].sum())
    lhs[start:start + gs[zg]] = 0.0
  spec = "situ:4.0:25.0" if situ else None
  out = ops.ragged_dot_fp8_scaled(to_dev(lhs, "bf16"), to_dev(codes).view(torch.float8_e4m3fn), to_dev(scale),
                                  to_dev(gs), fuse_gateup_activation=spec, zero_group=zg)
  ref = O.ragged_dot_fp8_scaled(lhs, codes, scale, gs, "bf16", situ=(4.0, 25.0) if situ else None)
  o = to_np(out)
  assert o.shape == ref.shape
  err = max_rel(o, ref)
  # the quantisation error of fp8 itself, for the record (rd.py:2843-2848 allows 0.05 abs)
  plain = O.ragged_dot(lhs, w, gs, "bf16") if not situ else None
  dev = max_rel(o, plain) if plain is not None else float("nan")
  banner(f"  max-rel vs oracle {err:.2e}; fp8 quantisation deviation from the bf16 weights {dev:.2e}")
  assert err <= 2e-2
  assert not o[int(gs.sum()):].any()


def test_op_class_dispatches_on_the_scale_dtype(gpu_device):
  """HipRaggedDot: f32 scales -> fp8 contract (bit-identical to
  ragged_dot_fp8_scaled); uint8 scales -> MXFP4; maybe_quantize_lhs on MXFP4
  -> MXFP8 x MXFP4, bit-identical to the explicit call; maybe_quantize_lhs on
  fp8 weights -> NotImplementedError."""
  from lmoe import ops
  rng = np.random.default_rng(3)
  m, k, n, g = 200, 256, 128, 3
  gs = to_dev(np.array([90, 0, 110], np.int32))
  lhs = to_dev(O.bf16_round(rng.standard_normal((m, k))), "bf16")
  codes, scale = _quantize_like_reference(O.bf16_round(rng.standard_normal((g, k, n)) * 0.02), 32)
  q8, s8 = to_dev(codes).view(torch.float8_e4m3fn), to_dev(scale)
  op = ops.HipRaggedDot()
  assert torch.equal(op(lhs, q8, group_sizes=gs, rhs_scale=s8), ops.ragged_dot_fp8_scaled(lhs, q8, s8, gs))
  with pytest.raises(NotImplementedError):
    op(lhs, q8, group_sizes=gs, rhs_scale=s8, maybe_quantize_lhs=True)
  packed = to_dev(rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8))
  e8 = to_dev(rng.integers(119, 130, (g, n, k // 32), dtype=np.uint8))
  assert torch.equal(op(lhs, packed, group_sizes=gs, rhs_scale=e8), ops.ragged_dot_mxfp4(lhs, packed, e8, gs))
  tpk, tsc = ops.mxfp4_tile_weights(packed, e8)
  q, qs = ops.quantize_mxfp8(lhs)
  want = ops.ragged_dot_mxfp8_mxfp4(q, qs, tpk, tsc, gs)
  assert torch.equal(op(lhs, packed, group_sizes=gs, rhs_scale=e8, maybe_quantize_lhs=True), want)
  assert torch.equal(op(lhs, tpk, group_sizes=gs, rhs_scale=tsc, maybe_quantize_lhs=True), want)
  with pytest.raises(ValueError):
    op(lhs, q8, group_sizes=gs, rhs_scale=s8.to(torch.float16))
