"""GPU parity: router top-k, local-shard dispatch and combine vs the CPU oracle.

Integer / index outputs (top-k ids, group sizes, permutations, gathered rows,
masks) must be bit-exact.  The gate scores and routing weights are bit-exact
too: the kernel and the oracle evaluate the sigmoid / softmax by the same
binary64 operation sequence and renormalise in the same order.  The combine
reproduces the oracle's rounding sequence, so it is compared exactly too.
"""
import numpy as np
import pytest
import torch

from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


def _logits(rng, t, e, kind):
  if kind == "normal":
    return rng.standard_normal((t, e)).astype(np.float32)
  if kind == "ties":  # integer logits: many exactly tied scores
    return rng.integers(-3, 4, (t, e)).astype(np.float32)
  if kind == "skew":
    rank = rng.permutation(e)
    return (rng.standard_normal((t, e)) - 1.2 * np.log(rank + 1)).astype(np.float32)
  if kind == "extreme":  # saturation, subnormal sigmoids, +-0, huge magnitudes
    x = (rng.standard_normal((t, e)) * 40).astype(np.float32)
    x.flat[:12] = [0.0, -0.0, 88.7, -87.3, -100.0, -103.9, -150.0, 1e30, -1e30, 709.0, -745.0, 30.0]
    return x
  raise ValueError(kind)


@pytest.mark.parametrize("t,e,k,kind,act,wdt", [
    (2048, 896, 16, "normal", "sigmoid", "bf16"),  # config 3 router
    (512, 896, 16, "skew", "sigmoid", "f32"),
    (257, 8, 2, "normal", "sigmoid", "f32"),
    (300, 64, 16, "ties", "sigmoid", "f32"),
    (300, 64, 6, "ties", "softmax", "f32"),
    (128, 8, 2, "normal", "softmax", "f32"),  # config 1 router (BASELINE: softmax)
    (64, 4096, 64, "normal", "sigmoid", "f32"),
    (33, 5, 5, "normal", "sigmoid", "bf16"),
    (16, 896, 1, "normal", "sigmoid", "f32"),
    (64, 896, 16, "extreme", "sigmoid", "f32"),
    (64, 100, 8, "extreme", "softmax", "f32"),
])
def test_router_topk_matches_oracle(gpu_device, t, e, k, kind, act, wdt):
  from lmoe import ops
  banner(f"router t={t} e={e} k={k} {kind} {act} {wdt}")
  rng = np.random.default_rng(t * 7 + e)
  logits = _logits(rng, t, e, kind)
  bias = np.zeros(e, np.float32)
  if kind == "ties":
    bias[::7] = 0.25
  ref = O.router_from_logits(logits, bias, k, True, 1.0, act, wdt)
  idx, w, scores = ops.router_topk_from_logits(
      to_dev(logits), to_dev(bias), k, True, 1.0, act,
      torch.bfloat16 if wdt == "bf16" else torch.float32, return_scores=True)
  idx, w, scores = to_np(idx), to_np(w), to_np(scores)
  assert np.array_equal(scores.view(np.uint32), ref.scores.view(np.uint32))
  assert np.array_equal(idx, ref.topk_idx)
  assert np.array_equal(w.view(np.uint32), ref.topk_weight.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("t,e,k,kind,wdt", [
    (4096, 896, 16, "skew", "bf16"),     # config 5 router
    (2048, 896, 16, "normal", "f32"),
    (300, 64, 16, "ties", "f32"),        # integer logits: more than 64 candidates -> full path
    (257, 8, 2, "normal", "f32"),        # fewer experts than lanes
    (64, 4096, 64, "normal", "f32"),     # k = 64
    (100, 896, 1, "normal", "f32"),
    (64, 896, 16, "extreme", "f32"),
])
def test_router_candidate_path_equals_full_path(gpu_device, t, e, k, kind, wdt):
  """Without a full score output the sigmoid gate selects from approximate-
  score candidates; ids and weights are bit-identical to the exact full path
  (which runs when scores are requested) and match the oracle."""
  from lmoe import ops
  rng = np.random.default_rng(t + 3 * e + k)
  logits = _logits(rng, t, e, kind)
  bias = (0.05 * rng.standard_normal(e)).astype(np.float32)
  if kind == "ties":
    bias = np.where(np.arange(e) % 7 == 0, 0.25, 0.0).astype(np.float32)
  wt = torch.bfloat16 if wdt == "bf16" else torch.float32
  lg, bs = to_dev(logits), to_dev(bias)
  i1, w1 = ops.router_topk_from_logits(lg, bs, k, True, 2.5, "sigmoid", wt)
  i2, w2, _ = ops.router_topk_from_logits(lg, bs, k, True, 2.5, "sigmoid", wt, return_scores=True)
  assert torch.equal(i1, i2)
  assert torch.equal(w1, w2)
  ref = O.router_from_logits(logits, bias, k, True, 2.5, "sigmoid", wdt)
  assert np.array_equal(to_np(i1), ref.topk_idx)
  assert np.array_equal(to_np(w1), ref.topk_weight)


def test_router_topk_strided_logits(gpu_device):
  """Logits as the router columns of a wider GEMM output (row stride > E):
  identical results to the contiguous copy."""
  from lmoe import ops
  rng = np.random.default_rng(5)
  t, e, extra, k = 777, 896, 1024, 16
  wide = to_dev(rng.standard_normal((t, e + extra)).astype(np.float32))
  bias = to_dev((0.01 * rng.standard_normal(e)).astype(np.float32))
  view = wide[:, :e]
  assert view.stride(0) == e + extra
  a = ops.router_topk_from_logits(view, bias, k, True, 2.5, "sigmoid", torch.bfloat16, return_scores=True)
  b = ops.router_topk_from_logits(view.contiguous(), bias, k, True, 2.5, "sigmoid", torch.bfloat16,
                                  return_scores=True)
  for x, y in zip(a, b):
    assert torch.equal(x, y)


@pytest.mark.parametrize("rows,cols,ld", [(4096, 1024, 1920), (333, 96, 96), (17, 5, 9)])
def test_cast_rows_f32_to_bf16(gpu_device, rows, cols, ld):
  """Strided f32 -> bf16 rows: round-to-nearest-even, bit-identical to
  torch's conversion (incl. NaN, +-inf, -0, values that round up past the
  bf16 maximum)."""
  from lmoe import ops
  rng = np.random.default_rng(rows)
  x = (rng.standard_normal((rows, ld)) * 10.0 ** rng.integers(-30, 30, (rows, ld))).astype(np.float32)
  x.flat[:6] = [np.nan, np.inf, -np.inf, -0.0, 3.3961775e38, 1.0 + 2.0 ** -8]
  xd = to_dev(x)
  got = ops.cast_rows(xd[:, :cols], torch.bfloat16)
  want = xd[:, :cols].to(torch.bfloat16)
  assert got.is_contiguous() and got.shape == (rows, cols)
  assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("mode,t,k,lat,dt", [
    ("scatter_add", 4096, 16, 1024, "bf16"),   # the layer's shape
    ("scatter_add", 300, 6, 136, "f32"),       # partial lane pass
    ("slot_sum", 257, 16, 2048, "bf16"),       # four passes
    ("slot_sum", 64, 2, 8, "f32"),
])
def test_combine_rms_norm_fused_equals_two_kernels(gpu_device, mode, t, k, lat, dt):
  """The fused combine + RMSNorm is bit-identical to combine_slots on zeros
  followed by rms_norm, for both combine modes, and writes the same routed
  rows when asked."""
  from lmoe import ops
  rng = np.random.default_rng(t + lat)
  m = t * k // 2
  tdt = torch.bfloat16 if dt == "bf16" else torch.float32
  shard = to_dev(rng.standard_normal((m, lat)).astype(np.float32)).to(tdt)
  perm = rng.permutation(t * k)  # each row feeds at most one slot, about half the slots dropped
  slot_pos = to_dev(np.where(perm < m, perm, -1).reshape(t, k).astype(np.int32))
  if mode == "scatter_add":
    w = to_dev(rng.random(m).astype(np.float32)).to(tdt)
  else:
    w = to_dev(rng.random((t, k)).astype(np.float32))
  scale = to_dev((1.0 + 0.1 * rng.standard_normal(lat)).astype(np.float32)).to(tdt)
  routed = ops.combine_slots(shard, slot_pos, w, t, k, mode=mode, out_dtype=tdt)
  ref = ops._rms_norm(routed, scale, 1e-6)
  normed, routed2 = ops.combine_slots_rms_norm(shard, slot_pos, w, t, k, scale, 1e-6, mode=mode, out_dtype=tdt,
                                               return_routed=True)
  assert torch.equal(routed2, routed)
  assert torch.equal(normed, ref)
  assert torch.equal(ops.combine_slots_rms_norm(shard, slot_pos, w, t, k, scale, 1e-6, mode=mode, out_dtype=tdt),
                     ref)


def test_router_golden_bias(gpu_device):
  """The golden bundles' uninitialised bias (1.36e5, denormals) through the GPU gate."""
  import _golden
  from lmoe import ops
  config, dtype, hidden, w, golden = _golden.load("golden_bundle_small")
  idx, wt = ops.router_topk_from_logits(to_dev(golden["router_logits"]),
                                        to_dev(w["e_score_correction_bias"]), 2, True, 1.0)
  g = np.sort(golden["topk_indices"], axis=1)
  assert np.array_equal(np.sort(to_np(idx), axis=1), g)


DISPATCH_CASES = [
    # name, T, k, E, start, L, cf, tile, wdt
    ("config3", 2048, 16, 896, 0, 112, 2.0, 128, "bf16"),
    ("offset137", 256, 16, 896, 137, 64, 4.0, 128, "f32"),
    ("overflow", 256, 16, 896, 137, 64, 0.05, 1, "f32"),
    ("decode_t1", 1, 16, 896, 0, 112, 2.0, 128, "bf16"),
    ("all_local", 100, 4, 16, 0, 16, 1.0, 1, "f32"),
    ("last_shard", 64, 2, 24, 18, 6, 4.0, 128, "f32"),
    ("big_chunks", 4096, 16, 896, 448, 112, 2.0, 128, "bf16"),
    # the sort's one-block scan stages its histogram in 64 KB of LDS: 128 chunks
    # x 127 experts plus the bin starts fill it exactly; one more expert per
    # chunk no longer fits and is scanned in place
    ("scan_lds_full", 4096, 16, 896, 0, 127, 2.0, 128, "bf16"),
    ("scan_in_place", 4096, 16, 896, 0, 128, 2.0, 128, "f32"),
    # 128 chunks x 201 bins = 25728 counters: more than 16 per scan thread, so
    # each thread also runs its tail loop past the counts held in registers
    ("scan_thread_tail", 4096, 16, 896, 0, 200, 2.0, 128, "bf16"),
]


def _run_dispatch(topk_idx, topk_w, x, wdt, start, L, m_padded, path="sort"):
  from lmoe import ops
  t, k = topk_idx.shape
  assert path == "sort" or ops.small_dispatch_supported(t, k, x.shape[1], L, m_padded)
  return ops.dispatch_local(to_dev(topk_idx), to_dev(topk_w, wdt), to_dev(x, "bf16"), start, L, m_padded,
                            path=path)


def _dispatch_params():
  """Every case on the counting-sort path; the one-launch path only at the
  sizes it takes (it refuses larger ones with NotImplementedError)."""
  from lmoe import ops
  out = []
  for case in DISPATCH_CASES:
    name, t, k, e, start, L, cf, tile, wdt = case
    out.append((*case, "sort"))
    if ops.small_dispatch_supported(t, k, 64, L, O.compute_m_padded(t, k, e, L, cf, tile)):
      out.append((*case, "small"))
  return out


@pytest.mark.parametrize("name,t,k,e,start,L,cf,tile,wdt,path", _dispatch_params())
def test_dispatch_matches_oracle_bit_exact(gpu_device, name, t, k, e, start, L, cf, tile, wdt, path):
  """Both dispatch paths (multi-block counting sort; one launch for
  decode-sized batches) against the oracle, all six outputs and slot_pos."""
  banner(f"dispatch {name} {path}")
  rng = np.random.default_rng(len(name) * 31 + t)
  topk_idx = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
  topk_w = O.cast(rng.uniform(size=(t, k)), wdt)
  x = O.bf16_round(rng.standard_normal((t, 64)))
  m_padded = O.compute_m_padded(t, k, e, L, cf, tile)
  ref, slot_pos = O.filter_and_pad_to_shard_jittable(topk_idx, topk_w, x, k, e, start, L, cf, tile,
                                                     return_slot_pos=True)
  got = _run_dispatch(topk_idx, topk_w, x, wdt, start, L, m_padded, path)
  for field in ("sorted_tokens", "group_sizes", "valid_mask", "per_expert_counts", "padded_token_idx",
                "padded_combine_weight"):
    a, b = to_np(getattr(got, field)), getattr(ref, field)
    assert a.shape == b.shape, field
    assert np.array_equal(a, b), field
  assert np.array_equal(to_np(got.slot_pos), slot_pos)


@pytest.mark.parametrize("path", ["sort", "small"])
@pytest.mark.parametrize("case", ["empty_shard", "extreme_skew", "boundary"])
def test_dispatch_literal_kats(gpu_device, case, path):
  """test_sharded_routing_local.py literal inputs (62-99, 102-125, 232-266)."""
  if case == "empty_shard":
    ti = np.array([[0, 1], [1, 2], [6, 7], [7, 0], [2, 3]], np.int32)
    tw, start, L, e = np.full((5, 2), 0.5, np.float32), 4, 2, 8
  elif case == "extreme_skew":
    ti, tw, start, L, e = np.full((50, 1), 5, np.int32), np.full((50, 1), 0.7, np.float32), 3, 5, 16
  else:
    ti = np.array([[4], [5], [8], [9]], np.int32)
    tw, start, L, e = np.array([[0.1], [0.2], [0.3], [0.4]], np.float32), 5, 4, 20
  t, k = ti.shape
  x = O.bf16_round(np.random.default_rng(5).standard_normal((t, 32)))
  m_padded = O.compute_m_padded(t, k, e, L, 4.0, 1)
  ref = O.filter_and_pad_to_shard(ti, tw, x, k, e, start, L, 4.0, 1)
  got = _run_dispatch(ti, tw, x, "f32", start, L, m_padded, path)
  for a, b in zip(got[:6], ref):
    assert np.array_equal(to_np(a), b)


@pytest.mark.parametrize("t", [1, 37, 512])
def test_dispatch_small_from_strided_f32(gpu_device, t):
  """The one-launch dispatch reading the latent columns of the fused f32
  router + down-projection output (row stride E + lat) equals cast-to-bf16
  then the sort path; with the padding rows skipped every other output and
  the kept rows are unchanged."""
  from lmoe import ops
  rng = np.random.default_rng(40 + t)
  k, e, L, lat = 16, 896, 112, 256
  topk_idx = torch.tensor(np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32), device="cuda")
  topk_w = torch.tensor(rng.uniform(size=(t, k)).astype(np.float32), device="cuda")
  rd = torch.tensor(rng.standard_normal((t, e + lat)).astype(np.float32), device="cuda")
  m_padded = O.compute_m_padded(t, k, e, L, 2.0, 128)
  ref = ops.dispatch_local(topk_idx, topk_w, ops.cast_rows(rd[:, e:], torch.bfloat16), 0, L, m_padded, path="sort")
  got = ops.dispatch_local(topk_idx, topk_w, rd[:, e:], 0, L, m_padded, path="small")
  for a, b in zip(got, ref):
    assert torch.equal(a, b)
  skip = ops.dispatch_local(topk_idx, topk_w, rd[:, e:], 0, L, m_padded, path="small", skip_padding_rows=True)
  nk = int(ref.group_sizes[:L].sum())
  assert torch.equal(skip.sorted_tokens[:nk], ref.sorted_tokens[:nk])
  for a, b in zip(skip[1:], ref[1:]):
    assert torch.equal(a, b)


@pytest.mark.parametrize("odt", ["bf16", "f32"])
def test_combine_slots_scatter_add_bit_exact(gpu_device, odt):
  from lmoe import ops
  rng = np.random.default_rng(11)
  t, k, e, L = 512, 16, 896, 112
  topk_idx = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
  topk_w = O.cast(rng.uniform(size=(t, k)), odt)
  x = O.bf16_round(rng.standard_normal((t, 64)))
  d, slot_pos = O.filter_and_pad_to_shard_jittable(topk_idx, topk_w, x, k, e, 0, L, 2.0, 128,
                                                   return_slot_pos=True)
  shard_out = O.cast(rng.standard_normal(d.sorted_tokens.shape), odt)
  ref = O.combine_shard_contribution(np.zeros((t, 64), np.float32), shard_out, d.padded_token_idx,
                                     d.padded_combine_weight, odt, odt, odt)
  got = ops.combine_slots(to_dev(shard_out, odt), to_dev(slot_pos), to_dev(d.padded_combine_weight, odt),
                          t, k, mode="scatter_add",
                          out_dtype=torch.bfloat16 if odt == "bf16" else torch.float32)
  assert np.array_equal(to_np(got), ref)


def test_combine_slot_sum_bit_exact(gpu_device):
  from lmoe import ops
  rng = np.random.default_rng(12)
  t, k, e = 300, 4, 16
  topk_idx = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
  topk_w = rng.uniform(size=(t, k)).astype(np.float32)
  order, _, gs = O.unsharded_dispatch(topk_idx, np.zeros((t, 8), np.float32), e)
  outs = O.bf16_round(rng.standard_normal((t * k, 48)))
  ref, _ = O.unsharded_combine(outs, order, topk_w, t, k, "bf16")
  slot_pos = np.empty(t * k, np.int32)
  slot_pos[order] = np.arange(t * k, dtype=np.int32)
  got = ops.combine_slots(to_dev(outs, "bf16"), to_dev(slot_pos), to_dev(topk_w), t, k, mode="slot_sum",
                          out_dtype=torch.bfloat16)
  assert np.array_equal(to_np(got), ref)


@pytest.mark.parametrize("t,m,lat", [(40, 1000, 24), (4096, 16384, 64)])
@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_generic_combine_scatter_add(gpu_device, dt, t, m, lat):
  """_combine_shard_contribution on arbitrary indices: duplicates, -1 padding
  rows with non-zero content (test_sharded_routing_local.py:170-194), a
  non-zero running accumulator, and one token hit 300 times (> LDS batch).
  The config-5 sized case (4096 tokens, 16384 rows: 16 chunks of the sort by
  token, 65536 counters) runs the scan's per-thread tail loop."""
  from lmoe import ops
  rng = np.random.default_rng(13 + t)
  idx = rng.integers(-1, t, m).astype(np.int32)
  idx[:300] = 7
  w = O.cast(rng.uniform(size=m), dt)
  w[idx < 0] = 0
  shard = O.cast(rng.standard_normal((m, lat)), dt)
  routed0 = O.cast(rng.standard_normal((t, lat)), dt)
  ref = O.combine_shard_contribution(routed0, shard, idx, w, dt, dt, dt)
  got = ops._combine_shard_contribution(to_dev(routed0, dt), to_dev(shard, dt), to_dev(idx), to_dev(w, dt))
  assert np.array_equal(to_np(got), ref)  # value equality (-1 rows add +-0 in the reference)


def test_combine_padding_literal(gpu_device):
  from lmoe import ops
  shard = np.random.default_rng(3).standard_normal((6, 8)).astype(np.float32)
  idx = np.array([0, 1, 2, 3, -1, -1], np.int32)
  w = np.array([0.5, 0.5, 0.5, 0.5, 0.0, 0.0], np.float32)
  got = ops._combine_shard_contribution(to_dev(np.zeros((4, 8), np.float32)), to_dev(shard), to_dev(idx),
                                        to_dev(w))
  assert np.max(np.abs(to_np(got) - shard[:4] * 0.5)) < 1e-6


def test_dispatch_deterministic_rerun(gpu_device):
  """Same inputs twice -> identical bytes (no atomics in the ordering)."""
  rng = np.random.default_rng(14)
  t, k, e, L = 4096, 16, 896, 112
  ti = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
  tw = O.bf16_round(rng.uniform(size=(t, k)))
  x = O.bf16_round(rng.standard_normal((t, 128)))
  m = O.compute_m_padded(t, k, e, L)
  a = _run_dispatch(ti, tw, x, "bf16", 0, L, m)
  b = _run_dispatch(ti, tw, x, "bf16", 0, L, m)
  for u, v in zip(a, b):
    assert torch.equal(u, v)


def test_dispatch_rows_sort_path_from_strided_f32(gpu_device):
  """Prefill-sized dispatch (T*k = 32768 slots, past the one-launch kernel)
  from the f32 latent columns of the fused projection output: the counting
  sort with the converting gather equals cast-to-bf16 then the bf16 sort path
  bit for bit; with the padding rows skipped every other output and the kept
  rows are unchanged."""
  from lmoe import ops
  rng = np.random.default_rng(77)
  t, k, e, L, lat = 2048, 16, 896, 112, 128
  topk_idx = torch.tensor(np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32), device="cuda")
  topk_w = torch.tensor(rng.uniform(size=(t, k)).astype(np.float32), device="cuda")
  rd = torch.tensor(rng.standard_normal((t, e + lat)).astype(np.float32), device="cuda")
  m_padded = O.compute_m_padded(t, k, e, L, 2.0, 128)
  ref = ops.dispatch_local(topk_idx, topk_w, ops.cast_rows(rd[:, e:], torch.bfloat16), 0, L, m_padded, path="sort")
  got = ops.dispatch_local(topk_idx, topk_w, rd[:, e:], 0, L, m_padded, path="sort")
  for a, b in zip(got, ref):
    assert torch.equal(a, b)
  skip = ops.dispatch_local(topk_idx, topk_w, rd[:, e:], 0, L, m_padded, path="sort", skip_padding_rows=True)
  nk = int(ref.group_sizes[:L].sum())
  assert torch.equal(skip.sorted_tokens[:nk], ref.sorted_tokens[:nk])
  for a, b in zip(skip[1:], ref[1:]):
    assert torch.equal(a, b)


def test_dispatch_small_refuses_large_sizes(gpu_device):
  """The one-launch dispatch raises NotImplementedError beyond its sizes
  (T*k > 8192 slots here) instead of running."""
  from lmoe import ops
  t, k = 4096, 16
  idx = torch.zeros((t, k), dtype=torch.int32, device="cuda")
  w = torch.zeros((t, k), dtype=torch.float32, device="cuda")
  x = torch.zeros((t, 64), dtype=torch.bfloat16, device="cuda")
  with pytest.raises(NotImplementedError):
    ops.dispatch_local(idx, w, x, 0, 112, 16384, path="small")


@pytest.mark.parametrize("path", ["sort", "small"])
def test_dispatch_empty_batch(gpu_device, path):
  """T = 0 tokens: every row is padding (zero row, token -1, weight 0), the
  group sizes are all padding, on both dispatch paths."""
  from lmoe import ops
  L, lat, m_padded = 16, 64, 128
  idx = torch.empty((0, 4), dtype=torch.int32, device="cuda")
  w = torch.empty((0, 4), dtype=torch.float32, device="cuda")
  x = torch.empty((0, lat), dtype=torch.bfloat16, device="cuda")
  d = ops.dispatch_local(idx, w, x, 0, L, m_padded, path=path)
  assert d.sorted_tokens.shape == (m_padded, lat) and not d.sorted_tokens.any()
  assert d.group_sizes[:L].sum().item() == 0 and d.group_sizes[L].item() == m_padded
  assert not d.valid_mask.any() and bool((d.padded_token_idx == -1).all()) and not d.padded_combine_weight.any()


@pytest.mark.parametrize("name", ["route_and_filter_to_local_shard", "route_and_filter_to_local_shard_jittable"])
def test_route_and_filter_to_local_shard(gpu_device, name):
  """ref.py:1144-1187 / ref.py:1382-1416: _router_gate (logits GEMM, sigmoid,
  top-k, bf16 weights) composed with the shard dispatch; all six outputs
  bit-exact against the oracle's gate and dispatch on the same logits."""
  from lmoe import ops
  from lmoe.config import LatentMoEConfig
  cfg = LatentMoEConfig(hidden_size=512, latent_size=256, intermediate_size=256, num_experts=896, top_k=16,
                        num_shared_experts=0)
  rng = np.random.default_rng(77)
  t, start, L = 1024, 336, 112
  hidden = O.bf16_round(rng.standard_normal((t, cfg.hidden_size)))
  router_w = O.bf16_round(rng.standard_normal((cfg.hidden_size, cfg.num_experts)) * 0.02)
  bias = (0.01 * rng.standard_normal(cfg.num_experts)).astype(np.float32)
  x = O.bf16_round(rng.standard_normal((t, cfg.latent_size)))
  hd, rw, bd, xd = to_dev(hidden, "bf16"), to_dev(router_w, "bf16"), to_dev(bias), to_dev(x, "bf16")
  out = getattr(ops, name)(hd, xd, rw, bd, cfg, start, L, 2.0)
  assert len(out) == 6
  logits = to_np(ops.router_logits(hd, rw))  # the same GEMM the composition runs
  assert max_rel(logits, O.matmul(hidden, router_w, "f32")) <= 1e-5
  r = O.router_from_logits(logits, bias, cfg.top_k, True, 1.0, "sigmoid", "bf16")
  ref = O.filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, x, cfg.top_k, cfg.num_experts, start, L)
  for field, a, b in zip(ref._fields, out, ref):
    assert np.array_equal(to_np(a), b), field
