"""Split-K MXFP4 grouped GEMM (lmoe_ragged_dot_mxfp4_splitk): the K steps of
every tile (64x128 up to M = 256, 64x256 above) are computed as k_split f32
partial planes and summed in order by a second kernel.

* parity with the oracle (dequantise, then ragged_dot; odq.py:65-172) within
  the bf16 bar, for one and several groups, a zero group and tail rows, the
  SiTU epilogue, one K step per range and ranges of unequal length;
* repeatable bit for bit, and within bf16 rounding of the unsplit kernel;
* bad k_split values and a short workspace are rejected before any launch.
"""
import ctypes

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


SPLIT_CASES = [
    # m, k, n, g, k_split, situ, zero_group, tail rows
    (300, 1024, 256, 1, 3, False, -1, 0),     # 64x256 tiles; 16 steps -> ranges 6, 6, 4
    (130, 1024, 512, 1, 16, True, -1, 0),     # one step per range, SiTU
    (200, 2048, 512, 3, 5, False, 1, 7),      # groups, a zero group, tail rows
    (77, 640, 136, 2, 4, False, -1, 5),       # partial tiles in M and N; 10 steps -> 3, 3, 3, 1
    (600, 640, 136, 2, 4, False, 0, 9),       # 64x256 tiles: partial n-tile, zero group, tail rows
    (520, 1024, 512, 1, 5, True, -1, 0),      # 64x256 tiles with the SiTU epilogue
    (128, 7168, 2048, 1, 8, False, -1, 0),    # config 4, M = 128 (the default split)
    (1024, 7168, 2048, 1, 4, False, -1, 0),   # config 4, M = 1024 (the default split, 64x256 tiles)
]


@pytest.mark.parametrize("m,k,n,g,ks,situ,zg,tail", SPLIT_CASES)
def test_splitk_matches_oracle(gpu_device, m, k, n, g, ks, situ, zg, tail):
  from lmoe import ops
  banner(f"split-K mxfp4 m={m} k={k} n={n} g={g} k_split={ks} situ={situ} zero_group={zg} tail={tail}")
  rng = np.random.default_rng(m + k + n + ks)
  gs = rng.multinomial(m - tail, np.ones(g) / g).astype(np.int32)
  lhs = O.bf16_round(rng.standard_normal((m, k)))
  if zg >= 0:
    start = int(gs[:zg].sum())
    lhs[start:start + gs[zg]] = 0.0
  packed, scale = _mx_weights(rng, g, n, k)
  epi = (4.0, 25.0) if situ else None
  ref = O.ragged_dot_mxfp4(lhs, packed, scale, gs, "bf16", epi)
  fa = "situ:4.0:25.0" if situ else None
  lhs_d, gs_d = to_dev(lhs, "bf16"), to_dev(gs)
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(scale))
  out = ops.ragged_dot_mxfp4(lhs_d, tpk, tsc, gs_d, fuse_gateup_activation=fa, zero_group=zg,
                             weight_layout="tiled", k_split=ks)
  again = ops.ragged_dot_mxfp4(lhs_d, tpk, tsc, gs_d, fuse_gateup_activation=fa, zero_group=zg,
                               weight_layout="tiled", k_split=ks)
  whole = ops.ragged_dot_mxfp4(lhs_d, tpk, tsc, gs_d, fuse_gateup_activation=fa, zero_group=zg,
                               weight_layout="tiled", k_split=1)
  o = to_np(out)
  err, err_whole = max_rel(o, ref), max_rel(o, to_np(whole))
  banner(f"  max-rel vs oracle {err:.2e}, vs unsplit kernel {err_whole:.2e}")
  assert o.shape == ref.shape
  assert err <= BF16_TOL
  assert err_whole <= BF16_TOL
  assert torch.equal(out, again)
  assert np.all(o[int(gs.sum()):] == 0)
  if zg >= 0:
    start = int(gs[:zg].sum())
    assert np.all(o[start:start + gs[zg]] == 0)


def test_splitk_rejects_bad_arguments(gpu_device):
  from lmoe import _lib
  lib = _lib.lib()
  m, k, n = 64, 512, 128
  lhs = torch.zeros((m, k), dtype=torch.bfloat16, device=gpu_device)
  pk = torch.zeros((1, k // 64, n, 32), dtype=torch.uint8, device=gpu_device)
  sc = torch.full((1, k // 64, n, 2), 127, dtype=torch.uint8, device=gpu_device)
  gs = torch.tensor([m], dtype=torch.int32, device=gpu_device)
  out = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
  ws = torch.empty((4 * m * n,), dtype=torch.float32, device=gpu_device)
  P = lambda t: ctypes.c_void_p(t.data_ptr())

  def call(ks, ws_bytes):
    return lib.lmoe_ragged_dot_mxfp4_splitk(P(lhs), P(pk), P(sc), P(gs), m, k, n, 1, -1, ks, P(ws), ws_bytes,
                                            _lib.EPI_NONE, 0.0, 0.0, P(out), None)

  assert call(0, ws.numel() * 4) == _lib.ERR_INVALID
  assert call(k // 64 + 1, ws.numel() * 4) == _lib.ERR_INVALID
  assert call(4, 4 * m * n * 4 - 16) == _lib.ERR_INVALID  # one plane short
  assert call(4, ws.numel() * 4) == _lib.OK
  torch.cuda.synchronize()
  assert not out.float().abs().max().item()
