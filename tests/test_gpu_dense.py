"""GPU parity of the hand-written dense projection kernel (lmoe_dense), the
layer's router logits + down-projection (ref.py:620, ref.py:634-655) and
up-projection (ref.py:430): bf16 x @ w^T with f32 accumulation against a
float64 product of the same bf16 values (f32 output 1e-5, bf16 output 2e-2
max-relative, benchmark_harness.py:192-199); partial tiles in M and N,
a single K step, and the output rows and columns outside the product left
untouched."""
import numpy as np
import pytest
import torch

from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k,n,odt", [
    (4096, 7168, 1920, "f32"),   # config 5 router logits + down-projection
    (4096, 1024, 7168, "bf16"),  # config 5 up-projection
    (300, 64, 136, "f32"),       # one K step, partial tiles
    (257, 512, 1032, "bf16"),
    (1, 128, 8, "f32"),
])
def test_dense_kernel_matches_fp64_product(gpu_device, m, k, n, odt):
  from lmoe import ops
  banner(f"dense m={m} k={k} n={n} {odt}")
  rng = np.random.default_rng(m + k + n)
  x = O.bf16_round(rng.standard_normal((m, k)))
  w = O.bf16_round(rng.standard_normal((n, k)) * 0.02)
  ref = x.astype(np.float64) @ w.astype(np.float64).T
  tdt = torch.float32 if odt == "f32" else torch.bfloat16
  out = to_np(ops.dense(to_dev(x, "bf16"), to_dev(w, "bf16"), tdt, w_layout="nk", backend="dense"))
  err = max_rel(out, ref)
  banner(f"  max-rel {err:.2e}")
  assert out.shape == (m, n)
  assert err <= (1e-5 if odt == "f32" else 2e-2)
  if odt == "bf16":
    assert np.array_equal(out, O.bf16_round(out))


def test_dense_kernel_equals_blaslt_within_f32_rounding(gpu_device):
  """Same products, another summation order: the two backends agree to f32
  rounding on the layer's fused projection."""
  from lmoe import ops
  g = torch.Generator(device="cuda").manual_seed(5)
  x = torch.randn((512, 7168), generator=g, device="cuda").to(torch.bfloat16)
  w = (torch.randn((1920, 7168), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
  a = ops.dense(x, w, torch.float32, w_layout="nk", backend="dense")
  b = ops.dense(x, w, torch.float32, w_layout="nk", backend="blaslt")
  assert max_rel(to_np(a), to_np(b)) <= 1e-5
