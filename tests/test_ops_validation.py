"""The Python operators refuse inputs whose shapes or dtypes the kernels would
misread, before anything reaches the library: the C-ABI sees only pointers
and the sizes it is given, so a top-k weight array shorter than the ids, too
few token rows, a short norm scale, mismatched elementwise operands or a
group-size array of the wrong length would otherwise be read past its end on
the device.  Checked on CPU tensors against the recording stand-in library:
each bad call raises ValueError / NotImplementedError (the reference's error
kinds for bad arguments and unsupported cases) and records no library call."""
import pytest
import torch

import _stand_in
from lmoe import ops

bf = torch.bfloat16
R = lambda *s, dt=bf: torch.randn(*s, generator=torch.Generator().manual_seed(0)).to(dt)
U8 = lambda *s: torch.zeros(*s, dtype=torch.uint8)
I32 = lambda *s: torch.zeros(*s, dtype=torch.int32)
GS = torch.tensor([10, 0, 20, 34], dtype=torch.int32)

BAD = {
    "ragged_dot: lhs not 2-D": lambda: ops.ragged_dot(R(64), R(4, 128, 64), GS),
    "ragged_dot: K differs": lambda: ops.ragged_dot(R(64, 96), R(4, 128, 64), GS),
    "ragged_dot: int64 group sizes": lambda: ops.ragged_dot(R(64, 128), R(4, 128, 64), GS.long()),
    "ragged_dot: 3 group sizes for 4 groups": lambda: ops.ragged_dot(R(64, 128), R(4, 128, 64), GS[:3]),
    "ragged_dot: mixed dtypes": lambda: ops.ragged_dot(R(64, 128), R(4, 128, 64, dt=torch.float32), GS),
    "ragged_dot: unknown backend": lambda: ops.ragged_dot(R(64, 128), R(4, 128, 64), GS, implementation="xla"),
    "gate/up: odd 2I": lambda: ops.ragged_dot_gateup_situ(R(64, 128), R(4, 128, 63), GS, 4.0, 25.0),
    "gate/up: 3 group sizes": lambda: ops.ragged_dot_gateup_situ(R(64, 128), R(4, 128, 64), GS[:3], 4.0, 25.0),
    "mxfp4: scale shape": lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 64, 64), U8(4, 64, 3), GS),
    "mxfp4: 3 group sizes": lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 64, 64), U8(4, 64, 4), GS[:3]),
    "mxfp4 tiled: 5 group sizes": lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 2, 64, 32), U8(4, 2, 64, 2),
                                                                torch.cat([GS, GS[:1]]), weight_layout="tiled"),
    "mxfp4 rows: 3 group sizes": lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 2, 64, 32), U8(4, 2, 64, 2), GS[:3],
                                                               weight_layout="tiled", lhs_row_index=I32(64)),
    "mxfp4: unknown mode": lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 64, 64), U8(4, 64, 4), GS, mode="fast"),
    # K = 65 with weights for K = 64: K / 64 and K / 32 round down to the weights' shapes
    "mxfp4 tiled: K not a multiple of 64": lambda: ops.ragged_dot_mxfp4(R(64, 65), U8(4, 1, 64, 32), U8(4, 1, 64, 2),
                                                                         GS, weight_layout="tiled"),
    "mxfp4: K not a multiple of 64": lambda: ops.ragged_dot_mxfp4(R(64, 65), U8(4, 64, 32), U8(4, 64, 2), GS),
    "mxfp4 rows: K not a multiple of 64": lambda: ops.ragged_dot_mxfp4(R(64, 65), U8(4, 1, 64, 32), U8(4, 1, 64, 2),
                                                                        GS, weight_layout="tiled",
                                                                        lhs_row_index=I32(64)),
    "mxfp8 x mxfp4: K not a multiple of 128": lambda: ops.ragged_dot_mxfp8_mxfp4(U8(64, 130), U8(1, 64, 4),
                                                                                  U8(4, 2, 64, 32), U8(4, 2, 64, 2),
                                                                                  GS),
    "mxfp8 x mxfp4: 3 group sizes": lambda: ops.ragged_dot_mxfp8_mxfp4(U8(64, 128), U8(1, 64, 4), U8(4, 2, 64, 32),
                                                                        U8(4, 2, 64, 2), GS[:3]),
    "mxfp6 x mxfp4: 3 group sizes": lambda: ops.ragged_dot_mxfp6_mxfp4(U8(64, 96), U8(1, 64, 4), U8(4, 2, 64, 32),
                                                                        U8(4, 2, 64, 2), GS[:3]),
    "dequant: scale shape": lambda: ops.dequantize_mxfp4(U8(4, 64), U8(4, 3)),
    "router: bf16 logits": lambda: ops.router_topk_from_logits(R(8, 16), None, 4),
    "router: bias length": lambda: ops.router_topk_from_logits(R(8, 16, dt=torch.float32), torch.zeros(15), 4),
    "router+projection: bias length": lambda: ops.router_topk_project(R(8, 16, dt=torch.float32),
                                                                       R(8, 32, dt=torch.float32), torch.zeros(8), 4),
    "dispatch: int64 ids": lambda: ops.dispatch_local(torch.zeros(8, 4, dtype=torch.int64), torch.rand(8, 4),
                                                      R(8, 64), 0, 16, 128),
    "dispatch: weights (T, k-1)": lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 3), R(8, 64), 0, 16, 128),
    "dispatch: f16 weights": lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 4).half(), R(8, 64), 0, 16, 128),
    "dispatch: 7 token rows for T = 8": lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 4), R(7, 64), 0, 16, 128),
    "dispatch sort path: 7 token rows": lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 4), R(7, 64), 0, 16, 128,
                                                                   path="sort"),
    "dispatch without rows: weights (T, k-1)": lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 3), None, 0, 16,
                                                                          128, gather_rows=False, lat=64),
    "fused decode dispatch: 7 token rows": lambda: ops.dispatch_ragged_dot_mxfp4_skinny(
        I32(8, 4), torch.rand(8, 4), R(7, 128), 0, 16, 128, U8(17, 2, 64, 32), U8(17, 2, 64, 2)),
    "combine: unknown mode": lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(8, 4), 8, 4, mode="sum"),
    "combine: slot_pos length": lambda: ops.combine_slots(R(128, 64), I32(31), torch.rand(8, 4), 8, 4,
                                                          mode="slot_sum"),
    "combine: slot_sum weights length": lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(8, 3), 8, 4,
                                                                  mode="slot_sum"),
    "combine: scatter_add weights per row": lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(127), 8, 4,
                                                                      mode="scatter_add"),
    "combine: empty shard": lambda: ops.combine_slots(R(0, 64), I32(32), torch.rand(8, 4), 8, 4, mode="slot_sum"),
    "combine: routed_out shape": lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(128), 8, 4,
                                                           mode="scatter_add", routed_out=R(8, 32)),
    "combine + norm: scale length": lambda: ops.combine_slots_rms_norm(R(128, 64), I32(32), torch.rand(8, 4), 8, 4,
                                                                       torch.ones(32, dtype=bf), 1e-6,
                                                                       mode="slot_sum"),
    "scatter-add combine: index length": lambda: ops._combine_shard_contribution(R(8, 64), R(128, 64), I32(127),
                                                                                 torch.rand(128)),
    "scatter-add combine: width": lambda: ops._combine_shard_contribution(R(8, 32), R(128, 64), I32(128),
                                                                          torch.rand(128)),
    "rms_norm: scale length": lambda: ops._rms_norm(R(8, 64), torch.ones(32, dtype=bf), 1e-6),
    "situ: shapes": lambda: ops._situ_and_mul(R(8, 64), R(8, 32), 4.0, 25.0),
    "situ: dtypes": lambda: ops._situ_and_mul(R(8, 64), R(8, 64, dt=torch.float32), 4.0, 25.0),
    "add: shapes": lambda: ops.add(R(8, 64), R(8, 32)),
    "add: dtypes": lambda: ops.add(R(8, 64), R(8, 64, dt=torch.float32)),
    "dense: K differs": lambda: ops.dense(R(8, 64), R(32, 128), w_layout="nk", backend="blaslt"),
    "dense: unknown backend": lambda: ops.dense(R(8, 64), R(64, 32), backend="cublas"),
    "cast: int8 target": lambda: ops.cast_rows(R(8, 64, dt=torch.float32), torch.int8),
    "mxfp8 quantiser: K % 128": lambda: ops.quantize_mxfp8(R(8, 100)),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_bad_inputs_are_refused_before_the_library(monkeypatch, case):
  rec = _stand_in.install(monkeypatch)
  with pytest.raises((ValueError, NotImplementedError)):
    BAD[case]()
  assert not rec.calls, rec.names()


def test_the_same_calls_with_good_inputs_reach_the_library(monkeypatch):
  """The refusals above are the inputs' fault: corrected, each operator
  reaches its entry point."""
  rec = _stand_in.install(monkeypatch)
  good = [
      lambda: ops.ragged_dot(R(64, 128), R(4, 128, 64), GS),
      lambda: ops.ragged_dot_gateup_situ(R(64, 128), R(4, 128, 64), GS, 4.0, 25.0),
      lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 64, 64), U8(4, 64, 4), GS),
      lambda: ops.ragged_dot_mxfp4(R(64, 128), U8(4, 2, 64, 32), U8(4, 2, 64, 2), GS, weight_layout="tiled",
                                   lhs_row_index=I32(64)),
      lambda: ops.ragged_dot_mxfp8_mxfp4(U8(64, 128), U8(1, 64, 4), U8(4, 2, 64, 32), U8(4, 2, 64, 2), GS),
      lambda: ops.ragged_dot_mxfp6_mxfp4(U8(64, 96), U8(1, 64, 4), U8(4, 2, 64, 32), U8(4, 2, 64, 2), GS),
      lambda: ops.router_topk_from_logits(R(8, 16, dt=torch.float32), torch.zeros(16), 4),
      lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 4), R(8, 64), 0, 16, 128),
      lambda: ops.dispatch_local(I32(8, 4), torch.rand(8, 4), R(8, 64), 0, 16, 128, path="sort"),
      lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(8, 4), 8, 4, mode="slot_sum"),
      lambda: ops.combine_slots(R(128, 64), I32(32), torch.rand(128), 8, 4, mode="scatter_add"),
      lambda: ops._combine_shard_contribution(R(8, 64), R(128, 64), I32(128), torch.rand(128)),
      lambda: ops._rms_norm(R(8, 64), torch.ones(64, dtype=bf), 1e-6),
      lambda: ops._situ_and_mul(R(8, 64), R(8, 64), 4.0, 25.0),
      lambda: ops.add(R(8, 64), R(8, 64)),
  ]
  for i, fn in enumerate(good):
    rec.calls.clear()
    fn()
    assert rec.calls, i


@pytest.mark.parametrize("case", ["router E", "router hidden", "bias", "down_proj", "up_proj", "norm_scale",
                                  "local range past E", "no local experts"])
def test_layer_refuses_weights_that_disagree_with_its_config(monkeypatch, case):
  """LocalShardLatentMoE checks its dense weights against the config and its
  local expert range against the expert count when it is built."""
  from lmoe import forward
  from lmoe.workloads import Config5, make_config5
  rec = _stand_in.install(monkeypatch)
  c = Config5(tokens=16, hidden=256, latent=256, intermediate=256, experts=128, top_k=16, local_start=16,
              local_experts=16)
  hidden, w, ex = make_config5("cpu", c, "mxfp4")
  kw = dict(router_weight=w["router_weight"], e_score_correction_bias=w["e_score_correction_bias"],
            down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
            local_expert_start=c.local_start, local_num_experts=c.local_experts, expert_format="mxfp4", experts=ex)
  forward.LocalShardLatentMoE(c.config(), **kw)  # consistent: builds
  bad = {"router E": dict(router_weight=w["router_weight"][:, :120]),
         "router hidden": dict(router_weight=w["router_weight"][:200]),
         "bias": dict(e_score_correction_bias=w["e_score_correction_bias"][:100]),
         "down_proj": dict(down_proj=w["down_proj"][:, :128]), "up_proj": dict(up_proj=w["up_proj"][:128]),
         "norm_scale": dict(norm_scale=w["norm_scale"][:128]), "local range past E": dict(local_expert_start=120),
         "no local experts": dict(local_num_experts=0)}[case]
  rec.calls.clear()
  with pytest.raises(ValueError):
    forward.LocalShardLatentMoE(c.config(), **dict(kw, **bad))
  assert not rec.calls


@pytest.mark.parametrize("shape", [(0, 0), (5, 0), (0, 64)])
def test_empty_rms_norm_returns_its_empty_output(monkeypatch, shape):
  """Normalising no elements (no rows, or rows of width 0) gives an empty
  output of the input's shape without a library call (the library refuses
  a width of 0)."""
  rec = _stand_in.install(monkeypatch)
  out = ops._rms_norm(R(*shape), torch.ones(shape[1], dtype=bf), 1e-6)
  assert out.shape == shape and out.dtype == bf
  assert not rec.calls
