"""GPU parity of the layer's gathered-rows path (prefill, tiled MXFP4 experts):

* ``router_topk_project`` (router_and_projection's outputs, ref.py:634-655,
  from one GEMM output) equals ``router_topk_from_logits`` + ``cast_rows``
  bit for bit;
* ``dispatch_local(..., gather_rows=False)`` writes every metadata output of
  the full dispatch bit for bit (ref.py:754-877 without the row gather);
* ``ragged_dot_mxfp4(tokens, ..., lhs_row_index=padded_token_idx)`` equals
  ``ragged_dot_mxfp4(tokens[padded_token_idx], ...)`` bit for bit, and the
  oracle's ragged_dot on the gathered rows within the bf16 bar;
* sizes the streamed kernel cannot take are refused before any launch.
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
  scale = rng.integers(119, 130, (g, n, k // 32), dtype=np.uint8)
  return packed, scale


@pytest.mark.parametrize("t,e,k,lat", [(4096, 896, 16, 1024), (300, 64, 8, 128), (1, 896, 16, 1024)])
def test_router_topk_project_equals_router_then_cast(gpu_device, t, e, k, lat):
  from lmoe import ops
  banner(f"router_topk_project t={t} e={e} k={k} lat={lat}")
  rng = np.random.default_rng(t + e)
  rd = torch.tensor(rng.standard_normal((t, e + lat)).astype(np.float32), device="cuda")
  bias = torch.tensor(rng.standard_normal(e).astype(np.float32) * 0.1, device="cuda")
  idx, w, xb = ops.router_topk_project(rd[:, :e], rd[:, e:], bias, k, True, 1.0, "sigmoid", torch.bfloat16)
  ridx, rw = ops.router_topk_from_logits(rd[:, :e], bias, k, True, 1.0, "sigmoid", torch.bfloat16)
  assert torch.equal(idx, ridx) and torch.equal(w, rw)
  assert torch.equal(xb, ops.cast_rows(rd[:, e:], torch.bfloat16))
  # softmax gate (full path) with the same cast
  idx, w, xb = ops.router_topk_project(rd[:, :e], rd[:, e:], None, k, True, 1.0, "softmax", torch.float32)
  ridx, rw = ops.router_topk_from_logits(rd[:, :e], None, k, True, 1.0, "softmax", torch.float32)
  assert torch.equal(idx, ridx) and torch.equal(w, rw)
  assert torch.equal(xb, rd[:, e:].to(torch.bfloat16))


@pytest.mark.parametrize("t,k,e,start,L", [(4096, 16, 896, 0, 112), (2048, 16, 896, 37, 112), (40, 4, 32, 8, 8),
                                           (256, 8, 8192, 100, 4000)])
def test_dispatch_without_rows_equals_full_metadata(gpu_device, t, k, e, start, L):
  """Few bins: the place kernel writes the metadata itself; 4000 bins: the
  one-block scan path and a separate metadata kernel."""
  from lmoe import ops
  banner(f"dispatch without rows t={t} k={k} e={e} start={start} L={L}")
  rng = np.random.default_rng(5 + t)
  lat = 256
  topk_idx = torch.tensor(np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32), device="cuda")
  topk_w = torch.tensor(rng.uniform(size=(t, k)).astype(np.float32), device="cuda").to(torch.bfloat16)
  x = torch.tensor(rng.standard_normal((t, lat)).astype(np.float32), device="cuda").to(torch.bfloat16)
  m_padded = O.compute_m_padded(t, k, e, L, 2.0, 128)
  ref = ops.dispatch_local(topk_idx, topk_w, x, start, L, m_padded, path="sort")
  got = ops.dispatch_local(topk_idx, topk_w, None, start, L, m_padded, gather_rows=False, lat=lat)
  assert got.sorted_tokens is None
  for a, b in zip(got[1:], ref[1:]):
    assert torch.equal(a, b)


def _gathered_case(rng, t, m, g, zero_at, k, n):
  """Token rows (t, k) bf16 and a dispatch-like row index: groups of sizes
  gs over m rows, the zero group (padding bucket, index -1) at zero_at."""
  w = 1.0 / np.arange(1, g + 1) ** 1.2
  gs = rng.multinomial(m - 40, w / w.sum()).astype(np.int32)
  gs[[1, g // 2]] = 0
  gs[2] = 1
  if zero_at >= 0:
    gs[zero_at] = 0
    gs[zero_at] = m - 40 - int(gs.sum())
  idx = np.full(m, -1, np.int32)
  row = 0
  for gi, c in enumerate(gs):
    if gi != zero_at:
      idx[row:row + c] = rng.integers(0, t, c)
    row += c
  tokens = O.bf16_round(rng.standard_normal((t, k)))
  return gs, idx, tokens


@pytest.mark.parametrize("situ", [False, True])
@pytest.mark.parametrize("t,m,k,n,g,zero_at", [(4096, 16384, 1024, 4096, 113, 112),
                                               (700, 3000, 256, 512, 41, 40),
                                               (50, 600, 128, 256, 9, -1)])
def test_ragged_dot_mxfp4_gathered_rows(gpu_device, situ, t, m, k, n, g, zero_at):
  from lmoe import ops
  banner(f"mxfp4 gathered rows situ={situ} t={t} m={m} k={k} n={n} g={g} zero_at={zero_at}")
  rng = np.random.default_rng(m + n + situ)
  gs, idx, tokens = _gathered_case(rng, t, m, g, zero_at, k, n)
  packed, scale = _mx_weights(rng, g, n, k)
  fa = "situ:4.0:25.0" if situ else None
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  tok_d, idx_d, gs_d = to_dev(tokens, "bf16"), to_dev(idx), to_dev(gs)
  gathered = tok_d[torch.clamp(idx_d, min=0).long()]  # test-side gather (rows of -1 are never read)
  ref = ops.ragged_dot_mxfp4(gathered.contiguous(), tpk, tsc, gs_d, fuse_gateup_activation=fa, zero_group=zero_at,
                             weight_layout="tiled", k_split=1, skip_zero_group_rows=True)
  got = ops.ragged_dot_mxfp4(tok_d, tpk, tsc, gs_d, fuse_gateup_activation=fa, zero_group=zero_at,
                             weight_layout="tiled", skip_zero_group_rows=True, lhs_row_index=idx_d)
  rows = np.ones(m, bool)
  if zero_at >= 0:
    s0 = int(gs[:zero_at].sum())
    rows[s0:s0 + gs[zero_at]] = False
  rows[int(gs.sum()):] = False
  rows_d = torch.tensor(rows, device="cuda")
  assert torch.equal(got[rows_d], ref[rows_d])
  # against the oracle on the gathered rows (a sample of groups at full size)
  lhs = tokens[np.maximum(idx, 0)]
  lhs[~rows] = 0.0
  oref = O.ragged_dot_mxfp4(lhs, packed, scale, gs, "bf16", (4.0, 25.0) if situ else None)
  assert max_rel(to_np(got)[rows], oref[rows]) <= BF16_TOL


def test_ragged_dot_mxfp4_gathered_rows_refuses_large_grids(gpu_device):
  """More tiles per resident block than the kernel's LDS row table holds:
  NotImplementedError before anything is launched."""
  from lmoe import ops
  rng = np.random.default_rng(3)
  t, m, k, n, g = 64, 40000, 64, 4096, 2
  gs = np.array([m // 2, m - m // 2], np.int32)
  idx = rng.integers(0, t, m).astype(np.int32)
  packed, scale = _mx_weights(rng, g, n, k)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  with pytest.raises(NotImplementedError):
    ops.ragged_dot_mxfp4(to_dev(O.bf16_round(rng.standard_normal((t, k))), "bf16"), tpk, tsc, to_dev(gs),
                         fuse_gateup_activation="situ:4.0:25.0", weight_layout="tiled", lhs_row_index=to_dev(idx))
  torch.cuda.synchronize()
