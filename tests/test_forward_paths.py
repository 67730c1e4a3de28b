"""The layer's path selection (LocalShardLatentMoE.forward) on the CPU: the
host logic runs on CPU tensors against a stand-in for liblmoe.so that records
every entry point it is asked for and launches nothing, so each configuration
is checked to reach only entry points whose size limits it meets -- e.g. a
decode step with more than 1024 latent columns must not ask the one-launch
router + latent cast (lmoe_router_topk_proj), which refuses it.  The recorded
calls are then re-issued to the real library, whose host-side argument and
size checks must all pass (without a device it stops at its first HIP call)."""
import pytest
import torch

import _stand_in
from lmoe import _lib, forward, ops
from lmoe.workloads import Config5, make_config5


@pytest.fixture
def rec(monkeypatch):
  return _stand_in.install(monkeypatch)


def _layer(lat, tokens, experts=128, mode="lds_dequant"):
  c = Config5(tokens=tokens, hidden=256, latent=lat, intermediate=256, experts=experts, top_k=16, local_start=16,
              local_experts=16)
  hidden, w, ex = make_config5("cpu", c, "mxfp4")
  layer = forward.LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                      e_score_correction_bias=w["e_score_correction_bias"],
                                      down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                                      local_expert_start=c.local_start, local_num_experts=c.local_experts,
                                      expert_format="mxfp4", experts=ex, capacity_factor=c.capacity_factor,
                                      mxfp4_mode=mode)
  return layer, hidden


def _proj_calls(rec):
  return [a for n, a in rec.calls if n == "lmoe_router_topk_proj"]


def test_decode_step_fuses_dispatch_into_the_skinny_gateup(rec):
  layer, hidden = _layer(256, 16)
  rec.calls.clear()
  layer.forward(hidden[:1].contiguous())
  assert rec.names() == ["lmoe_dense_blaslt", "lmoe_router_topk_proj", "lmoe_dispatch_mxfp4_skinny",
                         "lmoe_ragged_dot_mxfp4_skinny", "lmoe_combine_slots_rms_norm", "lmoe_dense_blaslt"]


@pytest.mark.parametrize("tokens", [1, 64, 512])
def test_latent_above_1024_never_asks_the_one_launch_projection(rec, tokens):
  """2048 latent columns: the router top-k reads the logits columns and the
  dispatch rounds the latent columns itself, at decode and prefill sizes."""
  layer, hidden = _layer(2048, max(tokens, 16))
  rec.calls.clear()
  layer.forward(hidden[:tokens].contiguous())
  names = rec.names()
  assert "lmoe_router_topk_proj" not in names and "lmoe_router_topk_ld" in names
  if tokens <= 64:
    assert "lmoe_dispatch_local_small" in names and names.count("lmoe_ragged_dot_mxfp4_skinny") == 2
  else:
    assert "lmoe_dispatch_local_rows" in names and names.count("lmoe_ragged_dot_mxfp4") == 2


def test_expert_count_not_a_multiple_of_4_never_asks_the_one_launch_projection(rec):
  """E % 4 != 0: the latent columns of the fused output start at 4 E bytes,
  off the 16-byte alignment the one-launch projection needs."""
  layer, hidden = _layer(256, 512, experts=126)
  rec.calls.clear()
  for t in (1, 512):
    layer.forward(hidden[:t].contiguous())
  assert not _proj_calls(rec)


def test_prefill_gathers_rows_in_the_gateup_kernel(rec):
  layer, hidden = _layer(256, 512)
  rec.calls.clear()
  layer.forward(hidden)
  assert rec.names() == ["lmoe_dense_blaslt", "lmoe_router_topk_proj", "lmoe_dispatch_local_rows",
                         "lmoe_ragged_dot_mxfp4_rows", "lmoe_ragged_dot_mxfp4", "lmoe_combine_slots_rms_norm",
                         "lmoe_dense_blaslt"]
  (args,) = _proj_calls(rec)
  # lmoe_router_topk_proj(logits, ld, bias, T, E, k, act, renorm, scale, wdt, idx, w, x_src, x_ld, lat, ...)
  x_ld, lat = args[13], args[14]
  assert lat == 256 and lat <= ops.ROUTER_PROJECT_MAX_LAT and x_ld % 4 == 0 and args[12] % 16 == 0


def test_stage_returning_forward_and_scaled_mode_take_the_sort_dispatch(rec):
  layer, hidden = _layer(256, 512)
  rec.calls.clear()
  layer.forward(hidden, return_stages=True)
  names = rec.names()
  assert "lmoe_router_topk_proj" not in names and "lmoe_cast_rows" in names
  assert "lmoe_ragged_dot_mxfp4_rows" not in names
  scaled, hidden = _layer(256, 512, mode="scaled_mfma")
  rec.calls.clear()
  scaled.forward(hidden)
  names = rec.names()
  assert names.count("lmoe_quantize_mxfp8") == 2 and names.count("lmoe_ragged_dot_mxfp8_mxfp4") == 2
  assert "lmoe_ragged_dot_mxfp4_rows" not in names and "lmoe_ragged_dot_mxfp4_skinny" not in names


@pytest.mark.parametrize("lat,tokens,mode,stages", [
    (256, 1, "lds_dequant", False), (256, 16, "lds_dequant", True), (256, 64, "lds_dequant", False),
    (256, 512, "lds_dequant", False), (256, 512, "lds_dequant", True), (256, 512, "scaled_mfma", False),
    (1024, 1, "lds_dequant", False), (1024, 512, "lds_dequant", False), (2048, 1, "lds_dequant", False),
    (2048, 512, "lds_dequant", False), (2048, 512, "lds_dequant", True)])
def test_every_call_passes_the_library_checks(rec, lat, tokens, mode, stages):
  """Each entry point the layer asks for, re-issued to the real library with
  the same arguments (host pointers of the CPU tensors), must get past the
  library's own argument and size checks: without a device the library then
  returns LMOE_ERR_HIP at its first HIP call, never LMOE_ERR_INVALID /
  UNSUPPORTED / WORKSPACE.  On a machine with a GPU the replay would launch
  kernels on host pointers, so it runs only where there is none."""
  if torch.cuda.device_count() > 0:
    return
  layer, hidden = _layer(lat, max(tokens, 16), mode=mode)
  rec.calls.clear()
  layer.forward(hidden[:tokens].contiguous(), return_stages=stages)
  real = _lib.lib()
  assert rec.calls
  for name, args in rec.calls:
    rc = getattr(real, name)(*args)
    assert rc in (_lib.OK, _lib.ERR_HIP), (name, rc, real.lmoe_last_error())


def test_the_replay_sees_a_refusal(rec):
  """The replay above can fail: the same recorded projection call with 2048
  latent columns is refused by the library's host check."""
  if torch.cuda.device_count() > 0:
    return
  layer, hidden = _layer(256, 16)
  rec.calls.clear()
  layer.forward(hidden[:1].contiguous())
  (args,) = _proj_calls(rec)
  real = _lib.lib()
  assert real.lmoe_router_topk_proj(*args) in (_lib.OK, _lib.ERR_HIP)
  bad = list(args)
  bad[14] = 2048
  assert real.lmoe_router_topk_proj(*bad) == _lib.ERR_INVALID
  assert b"latent" in real.lmoe_last_error()


@pytest.mark.parametrize("fused,shared", [(False, True), (True, True), (False, False), (True, False)])
def test_single_shard_functional_forward_path(rec, fused, shared):
  """latent_moe_forward_ragged_dot_single_shard_jittable (rd.py:1035-1137):
  down-projection, router logits, top-k, dispatch, the shard FFN (three
  grouped GEMMs, or the fused gate/up + SiTU and the down GEMM), combine,
  RMSNorm, up-projection, and the shared-expert MLP when given; every
  recorded call then passes the real library's host checks."""
  from lmoe import config as C
  cfg = C.mosaic_correctness_config()
  w = C.init_weights(cfg, 5, torch.bfloat16, device="cpu")
  start, L = 2, 4
  shard = lambda t: torch.cat([t[start:start + L], torch.zeros_like(t[:1])]).contiguous()
  hidden = torch.randn(32, cfg.hidden_size).to(torch.bfloat16)
  forward.latent_moe_forward_ragged_dot_single_shard_jittable(
      hidden, w.router_weight, w.e_score_correction_bias, w.down_proj, shard(w.expert_gate), shard(w.expert_up),
      shard(w.expert_down), w.norm_scale, w.up_proj, w.shared_gate if shared else None,
      w.shared_up if shared else None, w.shared_down if shared else None, cfg, start, L, fused_gateup=fused)
  names = rec.names()
  ffn = (["lmoe_ragged_dot_gateup_situ", "lmoe_ragged_dot"] if fused
         else ["lmoe_ragged_dot", "lmoe_ragged_dot", "lmoe_situ_and_mul", "lmoe_ragged_dot"])
  head = names[:4]
  assert set(head[:2]) <= {"lmoe_ragged_dot", "lmoe_dense_blaslt"} and head[2] == "lmoe_router_topk_ld"
  assert head[3].startswith("lmoe_dispatch_local")
  assert names[4:4 + len(ffn)] == ffn
  rest = names[4 + len(ffn):]
  assert rest[0] == "lmoe_combine_slots" and rest[1] == "lmoe_rms_norm"
  assert ("lmoe_add" in rest) == shared and ("lmoe_situ_and_mul" in rest) == shared
  if torch.cuda.device_count() == 0:
    real = _lib.lib()
    for name, args in rec.calls:
      assert getattr(real, name)(*args) in (_lib.OK, _lib.ERR_HIP), (name, real.lmoe_last_error())
