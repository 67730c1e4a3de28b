"""GPU parity of the skinny (decode-regime) MXFP4 grouped GEMM.

The kernel computes the same ragged_dot as the tile kernel (odq.py:65-172;
decode shapes rd.py:553-577) with another f32 summation order, so it is held
to the oracle at the bf16 bar (2e-2 max-rel, benchmark_harness.py:192-199),
plus properties of its own: results repeatable bit for bit (the waves'
partial sums are added in a fixed order), right for any pass size, rows of
the padding group zeroed or left alone, and exact dequantisation on one-hot
activations (every output is one weight, including the edge scales).
"""
import numpy as np
import pytest
import torch

from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _mx_weights(rng, g, n, k):
  packed = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  scale = rng.integers(119, 130, (g, n, k // 32), dtype=np.uint8)  # exponents -8..2
  return packed, scale


@pytest.mark.parametrize("m", [1, 5, 16, 100, 128])
def test_skinny_config4_matmul(gpu_device, m):
  """BASELINE config 4 (K=7168, N=2048, one group) at decode M (eight waves
  per 16-column item, 64-row passes above M=64): repeated calls are
  bit-identical, and right on fresh data each time."""
  from lmoe import ops
  banner(f"skinny cfg4 m={m}")
  rng = np.random.default_rng(100 + m)
  k, n = 7168, 2048
  packed, scale = _mx_weights(rng, 1, n, k)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  gs = np.array([m], np.int32)
  for rep in range(2):
    lhs = O.bf16_round(rng.standard_normal((m, k)))
    ref = O.ragged_dot_mxfp4(lhs, packed, scale, gs, "bf16")
    a = ops.ragged_dot_mxfp4(to_dev(lhs, "bf16"), tpk, tsc, to_dev(gs), weight_layout="tiled", mode="skinny")
    b = ops.ragged_dot_mxfp4(to_dev(lhs, "bf16"), tpk, tsc, to_dev(gs), weight_layout="tiled", mode="skinny")
    assert torch.equal(a, b)
    assert max_rel(to_np(a), ref) <= BF16_TOL, rep


@pytest.mark.parametrize("t,m_padded,situ", [(1, 128, True), (1, 128, False), (16, 128, True), (128, 512, True),
                                              (128, 512, False)])
def test_skinny_local_shard_groups(gpu_device, t, m_padded, situ):
  """Decode-shaped groups: 112 local experts + the padding bucket (zero group
  112) as the local-shard dispatch lays them out for T tokens; with and
  without the row bound hint (pass sizes 16..64 rows), padding rows zeroed or
  left unwritten."""
  from lmoe import ops
  banner(f"skinny groups t={t} m_padded={m_padded} situ={situ}")
  rng = np.random.default_rng(t * 3 + situ)
  L, k, n = 112, (256 if situ else 512), (512 if situ else 256)
  gs = np.zeros(L + 1, np.int32)
  slots = rng.choice(L, size=t * 2, replace=True)  # about two local rows per token, skewed
  np.add.at(gs, slots, 1)
  gs = np.minimum(gs, t)  # a token routes to an expert at most once
  gs[L] = m_padded - gs[:L].sum()
  lhs = O.bf16_round(rng.standard_normal((m_padded, k)))
  start = int(gs[:L].sum())
  lhs[start:] = 0.0
  packed, scale = _mx_weights(rng, L + 1, n, k)
  packed[L] = 0
  epi = (4.0, 25.0) if situ else None
  fa = "situ:4.0:25.0" if situ else None
  ref = O.ragged_dot_mxfp4(lhs, packed, scale, gs, "bf16", epi)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  x, g_d = to_dev(lhs, "bf16"), to_dev(gs)
  full = ops.ragged_dot_mxfp4(x, tpk, tsc, g_d, fuse_gateup_activation=fa, zero_group=L, weight_layout="tiled",
                              mode="skinny")
  hinted = ops.ragged_dot_mxfp4(x, tpk, tsc, g_d, fuse_gateup_activation=fa, zero_group=L, weight_layout="tiled",
                                mode="skinny", max_group_rows=t)
  o = to_np(full)
  assert max_rel(o, ref) <= BF16_TOL
  assert np.all(o[start:] == 0)
  assert max_rel(to_np(hinted), ref) <= BF16_TOL
  # skip flag: padding rows keep whatever was there, real rows are unchanged
  skip = ops.ragged_dot_mxfp4(x, tpk, tsc, g_d, fuse_gateup_activation=fa, zero_group=L, weight_layout="tiled",
                              mode="skinny", max_group_rows=t, skip_zero_group_rows=True)
  assert torch.equal(skip[:start], hinted[:start])
  # the tile kernel on the same data agrees at the bf16 bar
  tile = ops.ragged_dot_mxfp4(x, tpk, tsc, g_d, fuse_gateup_activation=fa, zero_group=L, weight_layout="tiled")
  assert max_rel(o, to_np(tile)) <= BF16_TOL


def test_skinny_large_groups_and_overrun(gpu_device):
  """Groups larger than one pass (300 rows with a 16-row hint: 19 passes),
  a group sizes sum past M (the rows beyond M are dropped) and an empty zero
  group."""
  from lmoe import ops
  rng = np.random.default_rng(5)
  m, k, n = 700, 256, 64
  gs = np.array([300, 0, 5, 200, 400], np.int32)  # sum 905 > 700
  lhs = O.bf16_round(rng.standard_normal((m, k)))
  packed, scale = _mx_weights(rng, 5, n, k)
  clipped = gs.copy()
  clipped[4] = m - gs[:4].sum()
  ref = O.ragged_dot_mxfp4(lhs, packed, scale, clipped, "bf16", (4.0, 25.0))
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  for hint in (16, 0):
    out = to_np(ops.ragged_dot_mxfp4(to_dev(lhs, "bf16"), tpk, tsc, to_dev(gs), fuse_gateup_activation="situ:4.0:25.0",
                                     zero_group=1, weight_layout="tiled", mode="skinny", max_group_rows=hint))
    assert max_rel(out, ref) <= BF16_TOL, hint


def test_skinny_one_hot_dequant_exact(gpu_device):
  """One-hot activation rows pick single weights: each output is one
  dequantised weight rounded to bf16 (exact: e2m1 x 2^e fits bf16) or NaN
  where the column holds an inf (0 x inf), for every scale byte including
  0..2 (denormal products) and 253..255 (overflow)."""
  from lmoe import ops
  rng = np.random.default_rng(9)
  k, n, g = 256, 64, 2
  m = 32
  gs = np.array([16, 16], np.int32)
  ks = rng.choice(k, m, replace=False)
  lhs = np.zeros((m, k), np.float32)
  lhs[np.arange(m), ks] = 1.0
  packed = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  scale = rng.integers(0, 256, (g, n, k // 32), dtype=np.uint8)
  scale[0, :8, :] = np.array([0, 1, 2, 3, 252, 253, 254, 255], np.uint8)[:, None]
  ref = O.ragged_dot_mxfp4(lhs, packed, scale, gs, "bf16")
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  out = to_np(ops.ragged_dot_mxfp4(to_dev(lhs, "bf16"), tpk, tsc, to_dev(gs), weight_layout="tiled", mode="skinny"))
  np.testing.assert_array_equal(np.isnan(out), np.isnan(ref))
  fin = ~np.isnan(ref)
  # a denormal product (scale bytes 0, 1) may leave the matrix core as the
  # value or as zero (input-denormal handling is the hardware's); every
  # normal, zero and infinite value is exact
  den = fin & (ref != 0) & (np.abs(ref) < 2.0 ** -126)
  exact = fin & ~den
  np.testing.assert_array_equal(out[exact], ref[exact])
  assert np.all((out[den] == ref[den]) | (out[den] == 0))


def test_skinny_alternating_layouts_repeatable(gpu_device):
  """The gate/up and down GEMMs of a decode step alternate (different
  column-tile counts and epilogues): every call of each stays bit-identical to
  its first one, i.e. no call leaves state that changes another's result."""
  from lmoe import ops
  rng = np.random.default_rng(12)
  L, lat, inter = 112, 256, 512
  gs = np.zeros(L + 1, np.int32)
  gs[[3, 40, 77]] = [1, 2, 1]
  gs[L] = 128 - gs.sum()
  x = to_dev(O.bf16_round(rng.standard_normal((128, lat))), "bf16")
  gu_p, gu_s = _mx_weights(rng, L + 1, 2 * inter, lat)
  dn_p, dn_s = _mx_weights(rng, L + 1, lat, inter)
  gu = ops.mxfp4_tile_weights(to_dev(gu_p), to_dev(gu_s))
  dn = ops.mxfp4_tile_weights(to_dev(dn_p), to_dev(dn_s))
  g_d = to_dev(gs)
  first = None
  for _ in range(4):
    act = ops.ragged_dot_mxfp4(x, *gu, g_d, fuse_gateup_activation="situ:4.0:25.0", zero_group=L,
                               weight_layout="tiled", mode="skinny", max_group_rows=2)
    out = ops.ragged_dot_mxfp4(act, *dn, g_d, zero_group=L, weight_layout="tiled", mode="skinny", max_group_rows=2)
    if first is None:
      first = (act.clone(), out.clone())
      ref = O.ragged_dot_mxfp4(to_np(x), gu_p, gu_s, gs, "bf16", (4.0, 25.0))
      assert max_rel(to_np(act)[:4], ref[:4]) <= BF16_TOL  # rows of the three hit groups
    else:
      assert torch.equal(act, first[0]) and torch.equal(out, first[1])


@pytest.mark.parametrize("m,k,n,odt", [(1, 7168, 1920, "f32"), (5, 7168, 1920, "f32"), (16, 1024, 7168, "bf16"),
                                       (40, 512, 384, "f32"), (100, 256, 96, "bf16")])
def test_dense_skinny_matches_fp32_reference(gpu_device, m, k, n, odt):
  """The few-row dense projection (decode step: fused router + down
  projection with f32 out, up-projection with bf16 out; 40 and 100 rows take
  several passes) against an fp32 torch matmul of the same bf16 operands
  (f32 out within 1e-5 relative, bf16 out within 2e-2) and against hipBLASLt;
  repeatable bit for bit."""
  from lmoe import ops
  g = torch.Generator(device="cuda").manual_seed(m * 7 + n)
  x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
  w = (torch.randn((n, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
  dt = torch.float32 if odt == "f32" else torch.bfloat16
  ref = x.float() @ w.float().t()
  a = ops.dense(x, w, out_dtype=dt, w_layout="nk", backend="skinny")
  b = ops.dense(x, w, out_dtype=dt, w_layout="nk", backend="skinny")
  lib = ops.dense(x, w, out_dtype=dt, w_layout="nk", backend="blaslt")
  assert torch.equal(a, b)
  tol = 1e-5 if odt == "f32" else 2e-2
  assert max_rel(to_np(a), to_np(ref)) <= tol
  assert max_rel(to_np(a), to_np(lib)) <= tol


def test_skinny_empty_and_all_padding(gpu_device):
  """M = 0 returns an empty result; groups that are all padding (only the
  zero group has rows) give all-zero rows, with nothing computed."""
  from lmoe import ops
  rng = np.random.default_rng(13)
  k, n, g = 256, 64, 3
  packed, scale = _mx_weights(rng, g, n, k)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  empty = ops.ragged_dot_mxfp4(torch.empty((0, k), dtype=torch.bfloat16, device="cuda"), tpk, tsc,
                               to_dev(np.zeros(g, np.int32)), weight_layout="tiled", mode="skinny")
  assert empty.shape == (0, n)
  x = to_dev(O.bf16_round(rng.standard_normal((40, k))), "bf16")
  out = ops.ragged_dot_mxfp4(x, tpk, tsc, to_dev(np.array([0, 0, 40], np.int32)), zero_group=2,
                             weight_layout="tiled", mode="skinny")
  assert out.shape == (40, n) and not out.any()


FUSED_CASES = [
    # T, E, k, start, L, lat, n, situ, capacity factor (m_padded), skip padding rows
    (1, 896, 16, 0, 112, 1024, 4096, True, 2.0, True),      # config 5, one decode token
    (16, 896, 16, 37, 112, 1024, 4096, True, 2.0, False),   # shard offset, padding rows zeroed
    (64, 896, 16, 0, 112, 1024, 4096, True, 2.0, True),     # T*k = 1024 (the limit)
    (40, 64, 8, 8, 48, 256, 512, False, 0.3, False),        # plain product; m_padded 128 < 240 local slots: tail truncation
    (3, 32, 4, 0, 32, 128, 96, False, 2.0, True),           # every expert local, N = 96
]


@pytest.mark.parametrize("t,e,k,start,L,lat,n,situ,cf,skip", FUSED_CASES)
def test_dispatch_skinny_fused_equals_two_launches(gpu_device, t, e, k, start, L, lat, n, situ, cf, skip):
  """dispatch_ragged_dot_mxfp4_skinny (one launch) == dispatch_local(path="small")
  followed by the skinny ragged_dot_mxfp4 on the sorted rows, bit for bit: every
  dispatch output and the expert GEMM's rows (ref.py:754-877, rd.py:610-723)."""
  from lmoe import ops
  banner(f"fused decode dispatch T={t} E={e} k={k} start={start} L={L} lat={lat} n={n} situ={situ} cf={cf}")
  gen = torch.Generator(device="cuda").manual_seed(t * 1000 + e)
  idx = torch.argsort(torch.rand((t, e), generator=gen, device="cuda"), dim=1)[:, :k].to(torch.int32).contiguous()
  w = torch.rand((t, k), generator=gen, device="cuda").to(torch.bfloat16)
  x = torch.randn((t, lat), generator=gen, device="cuda").to(torch.bfloat16)
  rng = np.random.default_rng(t + e + n)
  packed, scale = _mx_weights(rng, L + 1, n, lat)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  m_padded = ops.compute_m_padded(t, k, e, L, cf)
  fa = "situ:4.0:25.0" if situ else None
  d1, act1 = ops.dispatch_ragged_dot_mxfp4_skinny(idx, w, x, start, L, m_padded, tpk, tsc,
                                                  fuse_gateup_activation=fa, skip_zero_group_rows=skip)
  d0 = ops.dispatch_local(idx, w, x, start, L, m_padded, path="small")
  act0 = ops.ragged_dot_mxfp4(d0.sorted_tokens, tpk, tsc, d0.group_sizes, fuse_gateup_activation=fa, mode="skinny",
                              zero_group=L, weight_layout="tiled", skip_zero_group_rows=skip, max_group_rows=t)
  torch.cuda.synchronize()
  for name in ("group_sizes", "valid_mask", "per_expert_counts", "padded_token_idx", "padded_combine_weight",
               "slot_pos"):
    assert torch.equal(getattr(d1, name), getattr(d0, name)), name
  assert d1.sorted_tokens is None
  kept = int(d0.group_sizes[:L].sum())
  banner(f"  m_padded={m_padded} kept rows {kept} of {t * k} slots")
  if skip:
    assert torch.equal(act1[:kept], act0[:kept])
  else:
    assert torch.equal(act1, act0)
    assert bool((act1[kept:] == 0).all())
