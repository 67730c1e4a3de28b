"""The allocation-free dispatch entry point (lmoe_dispatch_local_noalloc)
through the C-ABI: every output bit-identical to lmoe_dispatch_local with a
caller workspace, on two calls in a row (the second smaller, so the static
scratch array still holds the first call's counters), and equal to the
oracle's jittable dispatch (ref.py:754-877)."""
import ctypes

import numpy as np
import pytest
import torch

from _util import banner, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


def _outputs(t, k, lat, m_padded, L, wdt, dev):
  return {
      "sorted_tokens": torch.full((m_padded, lat), 7, dtype=torch.int16, device=dev).view(torch.bfloat16),
      "group_sizes": torch.full((L + 1,), -5, dtype=torch.int32, device=dev),
      "valid": torch.full((m_padded,), 3, dtype=torch.uint8, device=dev),
      "per_expert_counts": torch.full((L,), -5, dtype=torch.int32, device=dev),
      "padded_token_idx": torch.full((m_padded,), -7, dtype=torch.int32, device=dev),
      "padded_w": torch.full((m_padded,), 9.0, dtype=wdt, device=dev),
      "slot_pos": torch.full((t * k,), -9, dtype=torch.int32, device=dev),
  }


def _call(name, idx, w, x, t, k, start, L, m_padded, out, workspace=None):
  from lmoe import _lib
  lib = _lib.lib()
  p = lambda a: ctypes.c_void_p(a.data_ptr())
  wdt = _lib.BF16 if w.dtype == torch.bfloat16 else _lib.F32
  args = [p(idx), p(w), wdt, p(x), _lib.BF16, t, k, x.shape[1], start, L, m_padded, p(out["sorted_tokens"]),
          p(out["group_sizes"]), p(out["valid"]), p(out["per_expert_counts"]), p(out["padded_token_idx"]),
          p(out["padded_w"]), p(out["slot_pos"])]
  if workspace is not None:
    args += [p(workspace), workspace.numel()]
  stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
  rc = getattr(lib, name)(*args, stream)
  assert rc == _lib.OK, lib.lmoe_last_error()


def test_noalloc_dispatch_equals_workspace_dispatch(gpu_device):
  from lmoe import _lib
  lib = _lib.lib()
  # config-5 sized (65536 slots, 128 chunks x 112 experts), then a smaller,
  # differently shaped call on the same scratch
  for case, (t, k, e, start, L, cf, wname) in enumerate([(4096, 16, 896, 0, 112, 2.0, "bf16"),
                                                         (300, 8, 64, 16, 16, 2.0, "f32")]):
    banner(f"noalloc dispatch call {case}: T={t} k={k} E={e} start={start} L={L}")
    rng = np.random.default_rng(900 + case)
    topk_idx = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    topk_w = O.cast(rng.uniform(size=(t, k)), wname)
    x = O.bf16_round(rng.standard_normal((t, 128)))
    m_padded = O.compute_m_padded(t, k, e, L, cf)
    wdt = torch.bfloat16 if wname == "bf16" else torch.float32
    idx_d, w_d, x_d = to_dev(topk_idx), to_dev(topk_w, wname), to_dev(x, "bf16")
    ref = _outputs(t, k, 128, m_padded, L, wdt, gpu_device)
    ws = torch.empty(lib.lmoe_dispatch_workspace_size(t, k, L), dtype=torch.uint8, device=gpu_device)
    _call("lmoe_dispatch_local", idx_d, w_d, x_d, t, k, start, L, m_padded, ref, workspace=ws)
    got = _outputs(t, k, 128, m_padded, L, wdt, gpu_device)
    _call("lmoe_dispatch_local_noalloc", idx_d, w_d, x_d, t, k, start, L, m_padded, got)
    torch.cuda.synchronize()
    for name in ref:
      assert torch.equal(got[name].view(torch.uint8), ref[name].view(torch.uint8)), (case, name)
    oracle, slot_pos = O.filter_and_pad_to_shard_jittable(topk_idx, topk_w, x, k, e, start, L, cf,
                                                          return_slot_pos=True)
    for field, key in zip(oracle._fields, ("sorted_tokens", "group_sizes", "valid", "per_expert_counts",
                                           "padded_token_idx", "padded_w")):
      assert np.array_equal(to_np(got[key]), getattr(oracle, field)), (case, field)
    assert np.array_equal(to_np(got["slot_pos"]), slot_pos)


def test_noalloc_dispatch_rejects_sizes_beyond_its_scratch(gpu_device):
  """T*k = 2^20 slots with L = 4096 needs 64 MiB of counters: refused with
  LMOE_ERR_WORKSPACE before anything runs."""
  from lmoe import _lib
  lib = _lib.lib()
  rc = lib.lmoe_dispatch_local_noalloc(None, None, 0, None, 1, 1 << 20, 1, 8, 0, 4096, 128, None, None, None,
                                       None, None, None, None, None)
  assert rc == _lib.ERR_WORKSPACE
  assert b"static array" in lib.lmoe_last_error()
