"""The Python layer's composition of the library, checked for values on the
CPU: the forwards run with the emulating stand-in library (each entry point
computed by the oracle's definition on the operators' host buffers, behind
the real library's host checks where no GPU is present), and their outputs
go through the same checks as the GPU suite's forward tests -- the six
golden bundles stage by stage at the reference's tolerances, the unsharded
and single-shard forwards against the oracle on their own logits (routing,
weights and every dispatch output bit for bit), and the prepared-weight
layer with bf16 experts at one token and larger batches.  A mistake in how
the operators chain the entry points (an argument order, a stride, a dtype,
a combine mode, a padding group) fails here without a GPU; the kernels
themselves are the GPU suite's."""
import numpy as np
import pytest
import torch

import _emulated_lib
import _golden
from _layer_check import check_single_shard, check_unsharded
from _util import to_dev, to_np
from lmoe.config import LatentMoEConfig, LatentMoEWeights
from oracle import lmoe_oracle as O


def _dev(a, dt="f32"):
  return to_dev(a, dt, device="cpu")


def _weights(w, dt):
  return LatentMoEWeights(**{k: _dev(O.cast(v, dt), dt) for k, v in w.items()})


@pytest.mark.parametrize("bundle", _golden.BUNDLES)
def test_unsharded_forward_on_golden_bundles(monkeypatch, bundle):
  from lmoe.forward import latent_moe_forward
  lib = _emulated_lib.install(monkeypatch)
  config, dtype, hidden, w, golden = _golden.load(bundle)
  final, inter = latent_moe_forward(_dev(O.cast(hidden, dtype), dtype), _weights(w, dtype), config,
                                    return_intermediates=True)
  ours = {k: to_np(v) for k, v in inter.items()}
  ours["sorted_token_indices"] = ours["sorted_token_indices"].astype(np.int64)
  atol, rtol = _golden.TOLERANCES[dtype]
  known = _golden.KNOWN_RESIDUALS.get(bundle, {})
  failures = []

  def check(name, g, o, exact):
    assert g.shape == o.shape, (name, g.shape, o.shape)
    if exact:
      if not np.array_equal(g, o):
        failures.append(f"{name}: exact mismatch")
      return
    max_abs = float(np.max(np.abs(g.astype(np.float64) - o))) if g.size else 0.0
    bound = known.get(name)
    if bound is not None:
      if max_abs > bound:
        failures.append(f"{name}: {max_abs:.3e} > documented {bound:.3e}")
    elif not np.allclose(g, o, atol=atol, rtol=rtol):
      failures.append(f"{name}: max_abs={max_abs:.3e}")

  _golden.compare_stages(golden, ours, config, dtype, check)
  assert not failures, failures
  wc = {k: O.cast(v, dtype) for k, v in w.items()}
  check_unsharded(f"emulated unsharded {bundle}", O.cast(hidden, dtype), wc, config, dtype, "sigmoid", final, inter)
  assert {"lmoe_router_topk_ld", "lmoe_ragged_dot", "lmoe_combine_slots", "lmoe_rms_norm"} <= set(lib.names())


def _shard_problem(rng, cfg, t, start, L):
  """The GPU suite's shard problem with the latent projection and the expert
  weights scaled by powers of two (bf16 values stay exact) so that gate and
  up are of order one: at the small sizes used here (hidden 64, latent 32)
  and N(0, 0.02^2) weights they are near 0.02, where SiTU-GLU is close to
  the symmetric g * u / 2 and a gate / up swap moves the output by less than
  the bf16 bound."""
  import test_gpu_forward as G
  hidden, w, gate, up, down = G._shard_problem(rng, cfg, t, start, L)
  w = dict(w, down_proj=w["down_proj"] * 8)
  return hidden, w, gate * 16, up * 16, down * 4


@pytest.mark.parametrize("fused", [False, True])
def test_single_shard_forward(monkeypatch, fused):
  from lmoe.forward import latent_moe_forward_ragged_dot_single_shard_jittable as fwd
  _emulated_lib.install(monkeypatch)
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48, num_experts=32, top_k=4,
                        num_shared_experts=1)
  t, start, L = 40, 8, 8
  hidden, w, gate, up, down = _shard_problem(np.random.default_rng(21), cfg, t, start, L)
  d = lambda a: _dev(a, "bf16")
  out, st = fwd(d(hidden), d(w["router_weight"]), _dev(w["e_score_correction_bias"]), d(w["down_proj"]), d(gate),
                d(up), d(down), d(w["norm_scale"]), d(w["up_proj"]), d(w["shared_gate"]), d(w["shared_up"]),
                d(w["shared_down"]), cfg, start, L, return_stages=True, fused_gateup=fused)
  check_single_shard(f"emulated single shard fused={fused}", hidden, w, gate, up, down, cfg, "bf16", start, L, 2.0,
                     True, out, st)


@pytest.mark.parametrize("t", [1, 5, 96])
def test_local_shard_layer_bf16_experts(monkeypatch, t):
  """The prepared-weight layer (fused router + down-projection GEMM, the
  dispatch rounding the f32 latent columns to bf16, the fused gate/up, the
  combine fused with the RMSNorm), one token included."""
  from lmoe import ops
  from lmoe.forward import LocalShardLatentMoE
  lib = _emulated_lib.install(monkeypatch)
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=32, num_experts=32, top_k=4,
                        num_shared_experts=0)
  start, L = 0, 8
  hidden, w, gate, up, down = _shard_problem(np.random.default_rng(22 + t), cfg, t, start, L)
  d = lambda a: _dev(a, "bf16")
  experts = {"gu_nk": ops.prefuse_gateup_weights_gnk(d(gate), d(up)), "down_nk": ops.to_gnk(d(down))}
  layer = LocalShardLatentMoE(cfg, router_weight=d(w["router_weight"]),
                              e_score_correction_bias=_dev(w["e_score_correction_bias"]), down_proj=d(w["down_proj"]),
                              up_proj=d(w["up_proj"]), norm_scale=d(w["norm_scale"]), local_expert_start=start,
                              local_num_experts=L, expert_format="bf16", experts=experts)
  out, st = layer.forward(d(hidden), return_stages=True)
  check_single_shard(f"emulated layer bf16 experts T={t}", hidden, w, gate, up, down, cfg, "bf16", start, L, 2.0,
                     False, out, st)
  assert "lmoe_ragged_dot_gateup_situ" in lib.names()
  assert torch.equal(layer.forward(d(hidden)), out)  # without the stages: the same output


def _mxfp4_layer(tokens, mode="lds_dequant"):
  """A small config-5-shaped layer with MXFP4 experts: each E8M0 scale byte
  raised by 4 (every dequantised weight times 16, exactly) and the latent
  projection times 8, so gate and up are of order one."""
  from lmoe.forward import LocalShardLatentMoE
  from lmoe.workloads import Config5, make_config5
  c = Config5(tokens=tokens, hidden=128, latent=128, intermediate=128, experts=32, top_k=4, local_start=8,
              local_experts=8)
  hidden, w, experts = make_config5("cpu", c, "mxfp4")
  for key in ("gu_scale", "down_scale"):
    experts[key] = experts[key] + 4
  w["down_proj"] = w["down_proj"] * 8
  w["norm_scale"] = _dev(O.bf16_round(np.random.default_rng(7).uniform(0.5, 2.0, c.latent)), "bf16")
  layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                              e_score_correction_bias=w["e_score_correction_bias"], down_proj=w["down_proj"],
                              up_proj=w["up_proj"], norm_scale=w["norm_scale"], local_expert_start=c.local_start,
                              local_num_experts=c.local_experts, expert_format="mxfp4", experts=experts,
                              capacity_factor=c.capacity_factor, mxfp4_mode=mode)
  return c, hidden, w, experts, layer


def _dequantized_shard(c, experts):
  inter = c.intermediate
  gu = O.dequantize_mxfp4(to_np(experts["gu_packed"]), to_np(experts["gu_scale"]))
  dn = O.dequantize_mxfp4(to_np(experts["down_packed"]), to_np(experts["down_scale"]))
  return gu[:, :inter, :].transpose(0, 2, 1), gu[:, inter:, :].transpose(0, 2, 1), dn.transpose(0, 2, 1)


# token counts: the decode step (fused dispatch + skinny expert GEMMs), the
# prefill step (rows gathered by the gate/up kernel), past the decode bound
@pytest.mark.parametrize("tokens,path", [(1, "lmoe_dispatch_mxfp4_skinny"), (16, "lmoe_dispatch_mxfp4_skinny"),
                                         (64, "lmoe_dispatch_mxfp4_skinny"), (65, "lmoe_ragged_dot_mxfp4_rows"),
                                         (200, "lmoe_ragged_dot_mxfp4_rows")])
def test_local_shard_layer_mxfp4(monkeypatch, tokens, path):
  """The benchmarked layer's composition at decode and prefill sizes against
  the oracle's single-shard forward on the dequantised experts; the
  stage-returning run (the sort dispatch, padding rows written) gives the
  same output bit for bit."""
  lib = _emulated_lib.install(monkeypatch)
  c, hidden, w, experts, layer = _mxfp4_layer(tokens)
  out = layer.forward(hidden)
  assert path in lib.names()
  lib.calls.clear()
  out_st, st = layer.forward(hidden, return_stages=True)
  assert path not in lib.names()  # the stages come from the sort dispatch
  assert torch.equal(out, out_st)
  gate, up, down = _dequantized_shard(c, experts)
  wn = {k: to_np(v) for k, v in w.items()}
  check_single_shard(f"emulated mxfp4 layer T={tokens}", to_np(hidden), wn, gate, up, down, c.config(), "bf16",
                     c.local_start, c.local_experts, c.capacity_factor, False, out, st)


def test_local_shard_layer_scaled_mfma(monkeypatch):
  from _layer_check import check_single_shard_mx8
  lib = _emulated_lib.install(monkeypatch)
  c, hidden, w, experts, layer = _mxfp4_layer(96, mode="scaled_mfma")
  out, st = layer.forward(hidden, return_stages=True)
  assert {"lmoe_quantize_mxfp8", "lmoe_ragged_dot_mxfp8_mxfp4"} <= set(lib.names())
  wn = {k: to_np(v) for k, v in w.items()}
  ex = {k: to_np(experts[k]) for k in ("gu_packed", "gu_scale", "down_packed", "down_scale")}
  check_single_shard_mx8("emulated scaled_mfma layer", to_np(hidden), wn, ex, c.config(), c.local_start,
                         c.local_experts, c.capacity_factor, out, st)


def test_mxfp4_layer_values_across_configurations(monkeypatch):
  """The MXFP4 layer over random configurations (expert count, shard size
  and position, top-k, token count, latent / intermediate / hidden sizes,
  capacity factors that truncate, lds_dequant or scaled mode): every forward
  equals its stage-returning run and passes the same oracle checks as above."""
  import contextlib
  import io
  from hypothesis import HealthCheck, given, settings
  from hypothesis import strategies as st
  from _layer_check import check_single_shard_mx8
  from lmoe.forward import LocalShardLatentMoE
  from lmoe.workloads import Config5, make_config5
  _emulated_lib.install(monkeypatch)
  stats = {"ran": 0}

  @settings(max_examples=30, deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
  @given(st.data())
  def run(data):
    pick = lambda xs: data.draw(st.sampled_from(xs))
    e = pick([8, 16, 60, 128])
    L = pick([n for n in (1, 4, 15, 16) if n <= e])
    c = Config5(tokens=pick([1, 2, 5, 16, 63, 64, 65, 130]), hidden=pick([64, 128]), latent=pick([64, 128, 256]),
                intermediate=pick([64, 128]), experts=e, top_k=pick([k for k in (1, 2, 4, 8) if k <= e]),
                local_start=pick(sorted({0, e - L})), local_experts=L, capacity_factor=pick([0.25, 1.0, 2.0]))
    mode = pick(["lds_dequant", "lds_dequant", "scaled_mfma"])
    hidden, w, ex = make_config5("cpu", c, "mxfp4")
    for key in ("gu_scale", "down_scale"):
      ex[key] = ex[key] + 4
    w["down_proj"] = w["down_proj"] * 8
    try:
      layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                  e_score_correction_bias=w["e_score_correction_bias"], down_proj=w["down_proj"],
                                  up_proj=w["up_proj"], norm_scale=w["norm_scale"], local_expert_start=c.local_start,
                                  local_num_experts=L, expert_format="mxfp4", experts=ex,
                                  capacity_factor=c.capacity_factor, mxfp4_mode=mode)
    except NotImplementedError:  # the scaled mode's sizes
      return
    out = layer.forward(hidden)
    out_st, st_ = layer.forward(hidden, return_stages=True)
    assert torch.equal(out, out_st), (c, mode)
    wn = {k: to_np(v) for k, v in w.items()}
    with contextlib.redirect_stdout(io.StringIO()):
      if mode == "scaled_mfma":
        exn = {k: to_np(ex[k]) for k in ("gu_packed", "gu_scale", "down_packed", "down_scale")}
        check_single_shard_mx8("sweep", to_np(hidden), wn, exn, c.config(), c.local_start, L, c.capacity_factor,
                               out_st, st_)
      else:
        gate, up, down = _dequantized_shard(c, ex)
        check_single_shard("sweep", to_np(hidden), wn, gate, up, down, c.config(), "bf16", c.local_start, L,
                           c.capacity_factor, False, out_st, st_)
    stats["ran"] += 1

  run()
  assert stats["ran"] >= 20, stats


@pytest.mark.parametrize("act,renorm,scaling,dt", [("softmax", True, 1.0, "bf16"), ("softmax", False, 2.5, "f32"),
                                                   ("sigmoid", False, 2.5, "bf16")])
def test_unsharded_forward_gate_options(monkeypatch, act, renorm, scaling, dt):
  """The unsharded forward's gate options the golden bundles do not hold
  (softmax, no renormalisation, a routed scaling factor): against the oracle
  on its own logits, routing bit for bit."""
  from lmoe.config import init_weights
  from lmoe.forward import latent_moe_forward
  _emulated_lib.install(monkeypatch)
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48, num_experts=16, top_k=4,
                        num_shared_experts=1, moe_renormalize=renorm, routed_scaling_factor=scaling)
  tdt = torch.float32 if dt == "f32" else torch.bfloat16
  import dataclasses
  W = init_weights(cfg, key=3, dtype=tdt, device="cpu")
  W = dataclasses.replace(W, router_weight=W.router_weight * 8)  # logits of order one: the gate's shape matters
  hidden = O.cast(np.random.default_rng(3).standard_normal((24, 64)), dt)
  final, inter = latent_moe_forward(_dev(hidden, dt), W, cfg, act=act, return_intermediates=True)
  wn = {k: to_np(v) for k, v in W.as_dict().items()}
  check_unsharded(f"emulated unsharded {act}", hidden, wn, cfg, dt, act, final, inter)


def _launch_free_log(monkeypatch):
  """Records, for each library call, the real library's own status on the
  same arguments: where no GPU is present any launch fails with ERR_HIP, so
  OK means the call returned before launching anything."""
  from lmoe import _lib
  real, log = _lib.lib(), []
  emulated = _emulated_lib.EmulatedLib.__getattr__

  def getattr_(self, name):
    entry = emulated(self, name)
    if not name.startswith("lmoe_") or name.endswith("workspace_size"):
      return entry

    def call(*args):
      log.append((name, getattr(real, name)(*args)))
      return entry(*args)
    return call
  monkeypatch.setattr(_emulated_lib.EmulatedLib, "__getattr__", getattr_)
  return log


@pytest.mark.skipif(torch.cuda.device_count() > 0, reason="reads the real library's status without a device")
def test_empty_batch(monkeypatch):
  """A batch of no tokens through every forward (unsharded, functional
  single shard with and without the fused gate/up, the prepared layer with
  bf16 experts and with MXFP4 experts in both modes, stages returned or
  not): an empty output of the hidden width and the input's dtype, the
  dispatch of no slots as the oracle gives it at m_padded = 0, and no call
  that launches a kernel (every entry point returns before its launch on
  empty sizes)."""
  from lmoe import _lib, forward
  from lmoe.config import init_weights
  from lmoe.workloads import Config5, make_config5
  _emulated_lib.install(monkeypatch)
  log = _launch_free_log(monkeypatch)
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48, num_experts=16, top_k=2,
                        num_shared_experts=1)
  want = O.filter_and_pad_to_shard_jittable(np.zeros((0, 2), np.int32), np.zeros((0, 2), np.float32),
                                            np.zeros((0, 32), np.float32), 2, 16, 0, 4, m_padded=0)
  outs = []
  for dt in (torch.float32, torch.bfloat16):
    W = init_weights(cfg, dtype=dt, device="cpu")
    h = torch.zeros(0, 64, dtype=dt)
    final, inter = forward.latent_moe_forward(h, W, cfg, return_intermediates=True)
    outs.append((final, dt, 64))
    assert all(v.shape[0] == 0 for k, v in inter.items() if k != "group_sizes")
    assert not inter["group_sizes"].any()
    pad = lambda w: torch.cat([w[0:4], torch.zeros_like(w[:1])])
    for fused in (False, True):
      final, st = forward.latent_moe_forward_ragged_dot_single_shard_jittable(
          h, W.router_weight, W.e_score_correction_bias, W.down_proj, pad(W.expert_gate), pad(W.expert_up),
          pad(W.expert_down), W.norm_scale, W.up_proj, W.shared_gate, W.shared_up, W.shared_down, cfg, 0, 4,
          fused_gateup=fused, return_stages=True)
      outs.append((final, dt, 64))
      for name, a, b in zip(want._fields, st["dispatch"], want):
        assert np.array_equal(to_np(a), b) and tuple(a.shape) == b.shape, name
      assert st["dispatch"].slot_pos.numel() == 0
  assert log and all(rc == _lib.OK for _, rc in log), log
  for fmt, mode in (("bf16", "lds_dequant"), ("mxfp4", "lds_dequant"), ("mxfp4", "scaled_mfma")):
    c = Config5(tokens=4, hidden=128, latent=128, intermediate=128, experts=16, top_k=2, local_start=0,
                local_experts=8)
    hidden, w, ex = make_config5("cpu", c, fmt)
    layer = forward.LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                        e_score_correction_bias=w["e_score_correction_bias"],
                                        down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                                        local_expert_start=0, local_num_experts=8, expert_format=fmt, experts=ex,
                                        capacity_factor=c.capacity_factor, mxfp4_mode=mode)
    log.clear()  # (re-tiling the MXFP4 weights at construction launches)
    outs.append((layer.forward(hidden[:0]), hidden.dtype, 128))
    out, st = layer.forward(hidden[:0], return_stages=True)
    outs.append((out, hidden.dtype, 128))
    assert st["dispatch"].group_sizes.tolist() == [0] * 9
    assert all(rc == _lib.OK for _, rc in log), log
  for out, dt, width in outs:
    assert tuple(out.shape) == (0, width) and out.dtype == dt
  assert len(outs) == 12


def test_no_capacity(monkeypatch):
  """capacity_factor 0: m_padded is 0 and every slot is dropped (ref.py:825-826
  rounds 0 up to 0), so the routed output is zero and the output is the
  shared experts' alone -- the oracle's single-shard forward at the same
  capacity, for the functional forward (fused gate/up or not) and the
  prepared layer with bf16 or MXFP4 experts."""
  from lmoe import forward
  from lmoe.config import init_weights
  from lmoe.workloads import Config5, make_config5
  _emulated_lib.install(monkeypatch)
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48, num_experts=16, top_k=2,
                        num_shared_experts=1)
  W = init_weights(cfg, dtype=torch.bfloat16, device="cpu")
  h = torch.randn(5, 64, generator=torch.Generator().manual_seed(0)).bfloat16()
  pad = lambda w: torch.cat([w[0:4], torch.zeros_like(w[:1])])
  wn = {k: to_np(v) for k, v in vars(W).items()}
  want, _ = O.single_shard_forward(to_np(h), wn, to_np(pad(W.expert_gate)), to_np(pad(W.expert_up)),
                                   to_np(pad(W.expert_down)), cfg, "bf16", 0, 4, capacity_factor=0.0)
  assert np.any(want != 0)
  for fused in (False, True):
    got, st = forward.latent_moe_forward_ragged_dot_single_shard_jittable(
        h, W.router_weight, W.e_score_correction_bias, W.down_proj, pad(W.expert_gate), pad(W.expert_up),
        pad(W.expert_down), W.norm_scale, W.up_proj, W.shared_gate, W.shared_up, W.shared_down, cfg, 0, 4,
        capacity_factor=0.0, fused_gateup=fused, return_stages=True)
    assert not st["routed_out"].any() and st["shard_out"].shape[0] == 0
    assert np.array_equal(to_np(got), want)
  for fmt in ("bf16", "mxfp4"):
    c = Config5(tokens=4, hidden=128, latent=128, intermediate=128, experts=16, top_k=2, local_start=0,
                local_experts=8, capacity_factor=0.0)
    hidden, w, ex = make_config5("cpu", c, fmt)
    layer = forward.LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                        e_score_correction_bias=w["e_score_correction_bias"],
                                        down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                                        local_expert_start=0, local_num_experts=8, expert_format=fmt, experts=ex,
                                        capacity_factor=0.0)
    out, st = layer.forward(hidden, return_stages=True)
    assert torch.equal(layer.forward(hidden), out)
    assert tuple(out.shape) == (4, 128) and not out.any() and not st["routed_out"].any()


@pytest.mark.parametrize("tokens", [16, 200])
def test_local_shard_layer_gate_options(monkeypatch, tokens):
  """The prepared MXFP4 layer with the softmax gate, no renormalisation and a
  routed scaling factor (ref.py:340-361) at a decode size (the one-launch
  router projection and fused dispatch) and a prefill size (gathered rows),
  stages returned and not: against the oracle's single-shard forward with the
  same options."""
  import dataclasses
  from lmoe.forward import LocalShardLatentMoE
  lib = _emulated_lib.install(monkeypatch)
  c, hidden, w, experts, _ = _mxfp4_layer(tokens)
  cfg = dataclasses.replace(c.config(), moe_renormalize=False, routed_scaling_factor=2.5)
  layer = LocalShardLatentMoE(cfg, router_weight=w["router_weight"], e_score_correction_bias=w["e_score_correction_bias"],
                              down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                              local_expert_start=c.local_start, local_num_experts=c.local_experts,
                              expert_format="mxfp4", experts=experts, capacity_factor=c.capacity_factor,
                              act="softmax")
  out = layer.forward(hidden)
  assert "lmoe_router_topk_proj" in lib.names()
  out_st, st = layer.forward(hidden, return_stages=True)
  assert torch.equal(out, out_st)
  gate, up, down = _dequantized_shard(c, experts)
  wn = {k: to_np(v) for k, v in w.items()}
  check_single_shard(f"emulated softmax layer T={tokens}", to_np(hidden), wn, gate, up, down, cfg, "bf16",
                     c.local_start, c.local_experts, c.capacity_factor, False, out, st, act="softmax")


@pytest.mark.parametrize("tokens", [16, 200])
def test_local_shard_layer_with_shared_experts(monkeypatch, tokens):
  """The prepared MXFP4 layer with its shared-expert MLP (ref.py:428-433,
  given in the layout its docstring states) against the oracle's
  single-shard forward with the shared experts included; a shared weight of
  the wrong shape is refused when the layer is built."""
  from lmoe import ops
  from lmoe.forward import LocalShardLatentMoE
  _emulated_lib.install(monkeypatch)
  c, hidden, w, experts, _ = _mxfp4_layer(tokens)
  rng = np.random.default_rng(tokens)
  si = 2 * c.intermediate
  sh = {k: O.bf16_round(rng.standard_normal(s) * 0.05) for k, s in
        (("shared_gate", (c.hidden, si)), ("shared_up", (c.hidden, si)), ("shared_down", (si, c.hidden)))}
  t = {k: _dev(v, "bf16") for k, v in sh.items()}
  shared = {"gu_nk": ops.prefuse_gateup_weights_gnk(t["shared_gate"][None], t["shared_up"][None]),
            "down_nk": t["shared_down"].t().contiguous()}
  kw = dict(router_weight=w["router_weight"], e_score_correction_bias=w["e_score_correction_bias"],
            down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
            local_expert_start=c.local_start, local_num_experts=c.local_experts, expert_format="mxfp4",
            experts=experts, capacity_factor=c.capacity_factor)
  layer = LocalShardLatentMoE(c.config(), shared=shared, **kw)
  out = layer.forward(hidden)
  out_st, st = layer.forward(hidden, return_stages=True)
  assert torch.equal(out, out_st)
  gate, up, down = _dequantized_shard(c, experts)
  wn = {k: to_np(v) for k, v in w.items()} | sh
  cfg = c.config()
  check_single_shard(f"emulated layer with shared experts T={tokens}", to_np(hidden), wn, gate, up, down, cfg,
                     "bf16", c.local_start, c.local_experts, c.capacity_factor, True, out, st)
  with pytest.raises(ValueError, match="shared"):
    LocalShardLatentMoE(c.config(), shared={"gu_nk": shared["gu_nk"], "down_nk": shared["down_nk"].t()}, **kw)
