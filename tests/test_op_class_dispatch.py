"""``HipRaggedDot`` (the op-class form of the reference's
``PallasMosaicTpuV2RaggedDot()(...)`` calls, rd.py:713-720 and
rd.py:2804-2811) picks its path from the weights it is given: plain bf16
weights -> the grouped GEMM (with ``fuse_gateup_activation``, the fused
gate/up + SiTU); fp8 E4M3 weights with f32 ``rhs_scale`` -> the block-scaled
fp8 path; uint8 E8M0 scales -> the MXFP4 paths (``maybe_quantize_lhs`` ->
MXFP8 activations on the scaled MFMA, re-tiling checkpoint weights first).
Checked on the CPU against the recording stand-in library: the entry points
each combination reaches, and the combinations it refuses."""
import pytest
import torch

import _stand_in
from lmoe import ops

bf = torch.bfloat16
GS = torch.tensor([10, 0, 20, 34], dtype=torch.int32)
M, K, N, G = 64, 128, 64, 4


def _x():
  return torch.randn(M, K).to(bf)


CASES = {
    "bf16 weights": (lambda op: op(_x(), torch.randn(G, K, N).to(bf), group_sizes=GS), ["lmoe_ragged_dot"]),
    "bf16 weights, fused gate/up": (
        lambda op: op(_x(), torch.randn(G, K, 2 * N).to(bf), group_sizes=GS, fuse_gateup_activation="situ:4:25"),
        ["lmoe_ragged_dot_gateup_situ"]),
    "fp8 weights, f32 scale": (
        lambda op: op(_x(), torch.randn(G, K, N).to(torch.float8_e4m3fn), group_sizes=GS,
                      rhs_scale=torch.ones(G, K // 32, 1, N)), ["lmoe_ragged_dot_fp8_scaled"]),
    "mxfp4 checkpoint weights": (
        lambda op: op(_x(), torch.zeros(G, N, K // 2, dtype=torch.uint8), group_sizes=GS,
                      rhs_scale=torch.zeros(G, N, K // 32, dtype=torch.uint8)), ["lmoe_ragged_dot_mxfp4"]),
    "mxfp4 tiled weights, fused gate/up": (
        lambda op: op(_x(), torch.zeros(G, K // 64, 2 * N, 32, dtype=torch.uint8), group_sizes=GS,
                      rhs_scale=torch.zeros(G, K // 64, 2 * N, 2, dtype=torch.uint8),
                      fuse_gateup_activation="situ:4:25"), ["lmoe_ragged_dot_mxfp4"]),
    "mxfp4 checkpoint weights, quantised activations": (
        lambda op: op(_x(), torch.zeros(G, N, K // 2, dtype=torch.uint8), group_sizes=GS,
                      rhs_scale=torch.zeros(G, N, K // 32, dtype=torch.uint8), maybe_quantize_lhs=True),
        ["lmoe_mxfp4_tile", "lmoe_quantize_mxfp8", "lmoe_ragged_dot_mxfp8_mxfp4"]),
}

REFUSED = {
    "fp8 weights with quantised activations": (
        lambda op: op(_x(), torch.randn(G, K, N).to(torch.float8_e4m3fn), group_sizes=GS,
                      rhs_scale=torch.ones(G, K // 32, 1, N), maybe_quantize_lhs=True), NotImplementedError),
    "quantised activations without quantised weights": (
        lambda op: op(_x(), torch.randn(G, K, N).to(bf), group_sizes=GS, maybe_quantize_lhs=True),
        NotImplementedError),
    "f16 scales": (
        lambda op: op(_x(), torch.zeros(G, N, K // 2, dtype=torch.uint8), group_sizes=GS,
                      rhs_scale=torch.zeros(G, N, K // 32, dtype=torch.float16)), ValueError),
    "another activation": (
        lambda op: op(_x(), torch.randn(G, K, 2 * N).to(bf), group_sizes=GS, fuse_gateup_activation="gelu"),
        NotImplementedError),
    "non-numeric beta": (
        lambda op: op(_x(), torch.randn(G, K, 2 * N).to(bf), group_sizes=GS, fuse_gateup_activation="situ:x:25"),
        ValueError),
    "zero beta": (
        lambda op: op(_x(), torch.randn(G, K, 2 * N).to(bf), group_sizes=GS, fuse_gateup_activation="situ:0:25"),
        ValueError),
    "infinite linear beta": (
        lambda op: op(_x(), torch.randn(G, K, 2 * N).to(bf), group_sizes=GS,
                      fuse_gateup_activation="situ:4:inf"), ValueError),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_each_weight_kind_reaches_its_path(monkeypatch, case):
  rec = _stand_in.install(monkeypatch)
  fn, want = CASES[case]
  fn(ops.HipRaggedDot())
  assert rec.names() == want


@pytest.mark.parametrize("case", sorted(REFUSED))
def test_unsupported_combinations_are_refused(monkeypatch, case):
  rec = _stand_in.install(monkeypatch)
  fn, exc = REFUSED[case]
  with pytest.raises(exc):
    fn(ops.HipRaggedDot())
  assert not rec.calls


def test_mxfp4_mode_of_the_op_class(monkeypatch):
  """``HipRaggedDot(mxfp4_mode=...)`` selects the MXFP4 kernel family for
  every call: the skinny decode kernel here (tiled weights)."""
  rec = _stand_in.install(monkeypatch)
  ops.HipRaggedDot(mxfp4_mode="skinny")(_x(), torch.zeros(G, K // 64, N, 32, dtype=torch.uint8), group_sizes=GS,
                                        rhs_scale=torch.zeros(G, K // 64, N, 2, dtype=torch.uint8))
  assert rec.names() == ["lmoe_ragged_dot_mxfp4_skinny"]
