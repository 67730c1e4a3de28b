"""Per-kernel benchmarks of the BASELINE configurations on one GPU.

Mirrors the reference's measurement protocol (hw_session_common.py:120-175:
warm-up, then rounds of back-to-back calls timed with device events, median
over rounds) and its metrics (bf16 TFLOP/s, GB/s, fraction of the binding
roofline: valid rows only, each weight byte counted once).

  python -m lmoe.kernel_bench [--only cfg2,cfg3,cfg4,cfg5,decode,prefill,dist,dense,copy] [--rounds 10] [--calls 20]

Prints one JSON object per measured kernel.
"""

from __future__ import annotations

import argparse
import json
import statistics

import numpy as np
import torch

from . import ops
from .workloads import Config5, make_config5, random_mxfp4, zipf_group_sizes

HBM_GBS = 8000.0
PEAK = {"bf16": 2500.0, "fp8": 5000.0, "mxfp4": 10100.0}


_FILTER = None  # substring: only kernels whose name contains it are run
_PROFILE = False  # run each selected kernel a few times, no timing


_DECODE_TOKENS = (1, 2, 4, 8, 16, 32, 64, 128)
_PREFILL_TOKENS = (128, 512, 2048, 4096)


def time_fn(fn, rounds=10, calls=20, name="", graph=True):
  """Median per-call ms over `rounds` rounds of `calls` back-to-back calls,
  each round one replay of the calls captured as a HIP graph (``graph=False``:
  eager launches, for a ``fn`` that already replays a graph)."""
  if _FILTER and _FILTER not in name:
    return None
  if _PROFILE:
    for _ in range(5):
      fn()
    torch.cuda.synchronize()
    return None
  fn()
  torch.cuda.synchronize()
  # the calls of one round captured as one HIP graph (no host launch cost in
  # the timing, as in the layer's graph replay); eager launches if a call
  # cannot be captured
  run = None
  try:
    if not graph:
      raise RuntimeError("eager launches requested")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
      fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
      for _ in range(calls):
        fn()
    torch.cuda.synchronize()
    run = g.replay
  except Exception:  # noqa: BLE001 -- fall back to eager launches
    torch.cuda.synchronize()
  per = []
  for _ in range(rounds):
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    if run is not None:
      run()
    else:
      for _ in range(calls):
        fn()
    b.record()
    b.synchronize()
    per.append(a.elapsed_time(b) / calls)
  return statistics.median(per)


def report(name, ms, flops, nbytes, peak_key="bf16", **extra):
  if ms is None:
    return None
  t = ms / 1000.0
  tf = flops / t / 1e12 if flops else 0.0
  gbs = nbytes / t / 1e9
  t_roof = max(flops / (PEAK[peak_key] * 1e12), nbytes / (HBM_GBS * 1e9))
  rec = {"kernel": name, "us": round(ms * 1000, 2), "tflops": round(tf, 2), "gbs": round(gbs, 1),
         "mfma_util": round(tf / PEAK[peak_key], 4), "roofline_frac": round(t_roof / t, 4),
         "bound": "hbm" if nbytes / (HBM_GBS * 1e9) >= flops / (PEAK[peak_key] * 1e12) else "mfma"}
  rec.update(extra)
  print(json.dumps(rec), flush=True)
  return rec


def bench_cfg2(dev, rounds, calls):
  gs = zipf_group_sizes(8192, 32, seed=2)
  gen = torch.Generator(device=dev).manual_seed(2)
  lhs = torch.randn((8192, 2048), generator=gen, device=dev).to(torch.bfloat16)
  rhs = (torch.randn((32, 2048, 1024), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
  g = torch.from_numpy(gs).to(dev)
  flops = 2.0 * 2048 * 1024 * gs.sum()
  nbytes = (gs > 0).sum() * 2048 * 1024 * 2 + 8192 * 2048 * 2 + 8192 * 1024 * 2
  ms = time_fn(lambda: ops.ragged_dot(lhs, rhs, g), rounds, calls, name="cfg2 ragged_dot bf16 (GKN reference layout)")
  report("cfg2 ragged_dot bf16 (GKN reference layout)", ms, flops, nbytes)
  rhs_nk = ops.to_gnk(rhs)
  ms = time_fn(lambda: ops.ragged_dot(lhs, rhs_nk, g, rhs_layout="gnk"), rounds, calls, name="cfg2 ragged_dot bf16 (GNK prepared layout)")
  report("cfg2 ragged_dot bf16 (GNK prepared layout)", ms, flops, nbytes)


def bench_cfg3(dev, rounds, calls):
  t, e, k, L, lat, inter = 2048, 896, 16, 112, 1024, 2048
  gen = torch.Generator(device=dev).manual_seed(3)
  logits = torch.randn((t, e), generator=gen, device=dev)
  x = torch.randn((t, lat), generator=gen, device=dev).to(torch.bfloat16)
  gu = (torch.randn((L + 1, 2 * inter, lat), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
  dn = (torch.randn((L + 1, lat, inter), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
  idx, w = ops.router_topk_from_logits(logits, None, k, True, 1.0, "sigmoid", torch.bfloat16)
  m_padded = ops.compute_m_padded(t, k, e, L)
  d = ops.dispatch_local(idx, w, x, 0, L, m_padded)
  gs = d.group_sizes.cpu().numpy()
  rows, hit = int(gs[:L].sum()), int((gs[:L] > 0).sum())
  ms = time_fn(lambda: ops.router_topk_from_logits(logits, None, k, True, 1.0, "sigmoid", torch.bfloat16),
               rounds, calls, name="cfg3 router_topk (2048x896, k=16)")
  report("cfg3 router_topk (2048x896, k=16)", ms, 0, t * e * 4 + t * k * 6)
  ms = time_fn(lambda: ops.dispatch_local(idx, w, x, 0, L, m_padded), rounds, calls, name="cfg3 dispatch (counting sort + gather)")
  report("cfg3 dispatch (counting sort + gather)", ms, 0,
         t * k * 4 + rows * lat * 2 * 2 + (m_padded - rows) * lat * 2 + m_padded * 11, rows=rows)
  f_gu = 2.0 * rows * lat * 2 * inter
  b_gu = hit * 2 * inter * lat * 2 + rows * lat * 2 + rows * inter * 2
  ms = time_fn(lambda: ops.ragged_dot_gateup_situ(d.sorted_tokens, gu, d.group_sizes, 4.0, 25.0,
                                                  rhs_layout="gnk", zero_group=L), rounds, calls, name="cfg3 gate/up+SiTU bf16 grouped GEMM")
  report("cfg3 gate/up+SiTU bf16 grouped GEMM", ms, f_gu, b_gu, rows=rows, experts_hit=hit)
  act = ops.ragged_dot_gateup_situ(d.sorted_tokens, gu, d.group_sizes, 4.0, 25.0, rhs_layout="gnk",
                                   zero_group=L)
  f_dn = 2.0 * rows * inter * lat
  b_dn = hit * inter * lat * 2 + rows * inter * 2 + rows * lat * 2
  ms = time_fn(lambda: ops.ragged_dot(act, dn, d.group_sizes, rhs_layout="gnk", zero_group=L), rounds,
               calls, name="cfg3 down bf16 grouped GEMM")
  report("cfg3 down bf16 grouped GEMM", ms, f_dn, b_dn, rows=rows)
  out = ops.ragged_dot(act, dn, d.group_sizes, rhs_layout="gnk", zero_group=L)
  ms = time_fn(lambda: ops.combine_slots(out, d.slot_pos, d.padded_combine_weight, t, k,
                                         mode="scatter_add", out_dtype=torch.bfloat16), rounds, calls, name="cfg3 combine (slot scatter-add)")
  report("cfg3 combine (slot scatter-add)", ms, 0, rows * lat * 2 + t * lat * 2 * 2 + t * k * 4)


def bench_cfg4(dev, rounds, calls):
  k_, n_ = 7168, 2048
  packed, scale = random_mxfp4(1, n_, k_, dev, seed=4)
  tpk, tsc = ops.mxfp4_tile_weights(packed, scale)
  for m in (1, 16, 128, 1024, 4096):
    gen = torch.Generator(device=dev).manual_seed(m)
    a = torch.randn((m, k_), generator=gen, device=dev).to(torch.bfloat16)
    g = torch.tensor([m], dtype=torch.int32, device=dev)
    flops = 2.0 * m * k_ * n_
    nbytes = n_ * k_ * (0.5 + 1 / 32) + m * k_ * 2 + m * n_ * 2
    ms = time_fn(lambda: ops.ragged_dot_mxfp4(a, packed, scale, g), rounds, calls, name=f"cfg4 mxfp4 matmul checkpoint scales M={m}")
    report(f"cfg4 mxfp4 matmul checkpoint scales M={m}", ms, flops, nbytes, peak_key="bf16", m=m)
    ks = ops.mxfp4_k_split(m, n_, k_, 1)
    nm = f"cfg4 mxfp4 matmul tiled weights M={m}" + (f" (split-K {ks})" if ks > 1 else "")
    ms = time_fn(lambda: ops.ragged_dot_mxfp4(a, tpk, tsc, g, weight_layout="tiled"), rounds, calls, name=nm)
    report(nm, ms, flops, nbytes, peak_key="bf16", m=m, k_split=ks)
    if ks > 1:
      nm = f"cfg4 mxfp4 matmul tiled weights M={m} (unsplit)"
      ms = time_fn(lambda: ops.ragged_dot_mxfp4(a, tpk, tsc, g, weight_layout="tiled", k_split=1), rounds, calls,
                   name=nm)
      report(nm, ms, flops, nbytes, peak_key="bf16", m=m)
    if m <= 128:
      ms = time_fn(lambda: ops.ragged_dot_mxfp4(a, tpk, tsc, g, weight_layout="tiled", mode="skinny"), rounds,
                   calls, name=f"cfg4 mxfp4 matmul skinny M={m}")
      report(f"cfg4 mxfp4 matmul skinny M={m}", ms, flops, nbytes, peak_key="bf16", m=m)
    ms = time_fn(lambda: ops.quantize_mxfp8(a), rounds, calls, name=f"cfg4 mxfp8 quantise M={m}")
    report(f"cfg4 mxfp8 quantise M={m}", ms, 0, m * k_ * (2 + 1 + 1 / 32), m=m)
    q, qs = ops.quantize_mxfp8(a)
    ms = time_fn(lambda: ops.ragged_dot_mxfp8_mxfp4(q, qs, tpk, tsc, g), rounds, calls,
                 name=f"cfg4 mxfp8 x mxfp4 scaled MFMA M={m}")
    report(f"cfg4 mxfp8 x mxfp4 scaled MFMA M={m}", ms, flops, nbytes - m * k_ * (1 - 1 / 32),
           peak_key="fp8", m=m)
    ms = time_fn(lambda: ops.quantize_mxfp6(a), rounds, calls, name=f"cfg4 mxfp6 quantise M={m}")
    report(f"cfg4 mxfp6 quantise M={m}", ms, 0, m * k_ * (2 + 0.75 + 1 / 32), m=m)
    q6, qs6 = ops.quantize_mxfp6(a)
    ms = time_fn(lambda: ops.ragged_dot_mxfp6_mxfp4(q6, qs6, tpk, tsc, g), rounds, calls,
                 name=f"cfg4 mxfp6 x mxfp4 scaled MFMA (FP4 rate) M={m}")
    report(f"cfg4 mxfp6 x mxfp4 scaled MFMA (FP4 rate) M={m}", ms, flops, nbytes - m * k_ * (1.25 - 1 / 32),
           peak_key="mxfp4", m=m)


def bench_cfg5(dev, rounds, calls):
  from .forward import LocalShardLatentMoE
  c = Config5()
  hidden, w, experts = make_config5(dev, c, "mxfp4")
  layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                              e_score_correction_bias=w["e_score_correction_bias"],
                              down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                              local_expert_start=0, local_num_experts=c.local_experts,
                              expert_format="mxfp4", experts=experts)
  _, st = layer.forward(hidden, return_stages=True)
  d = st["dispatch"]
  gs = d.group_sizes.cpu().numpy()
  L, lat, inter, H, T = c.local_experts, c.latent, c.intermediate, c.hidden, c.tokens
  rows, hit = int(gs[:L].sum()), int((gs[:L] > 0).sum())
  ms = time_fn(lambda: layer.forward(hidden), rounds, max(1, calls // 4), name="cfg5 full layer")
  report("cfg5 full layer", ms, 0, 0, tokens_per_s=round(T / (ms / 1000)) if ms else None, rows=rows)
  ms = time_fn(lambda: layer._dense(hidden, layer.router_nk, torch.float32), rounds, calls, name="cfg5 router logits GEMM 4096x7168x896 (f32 out)")
  report("cfg5 router logits GEMM 4096x7168x896 (f32 out)", ms, 2.0 * T * H * c.experts,
         T * H * 2 + H * c.experts * 2 + T * c.experts * 4)
  ms = time_fn(lambda: layer._dense(hidden, layer.down_nk), rounds, calls, name="cfg5 down-proj GEMM 4096x7168x1024")
  report("cfg5 down-proj GEMM 4096x7168x1024", ms, 2.0 * T * H * lat, T * H * 2 + H * lat * 2 + T * lat * 2)
  f_gu = 2.0 * rows * lat * 2 * inter
  b_gu = hit * 2 * inter * lat * (0.5 + 1 / 32) + rows * lat * 2 + rows * inter * 2
  E = layer.experts
  for lay, sfx in (("checkpoint", ""), ("tiled", "_tiled")):
    nm = f"cfg5 mxfp4 gate/up+SiTU grouped GEMM ({lay} weights)"
    ms = time_fn(lambda: ops.ragged_dot_mxfp4(d.sorted_tokens, E["gu_packed" + sfx], E["gu_scale" + sfx],
                                              d.group_sizes, fuse_gateup_activation="situ:4.0:25.0",
                                              zero_group=L, weight_layout=lay), rounds, calls, name=nm)
    report(nm, ms, f_gu, b_gu, rows=rows, experts_hit=hit)
  ms = time_fn(lambda: ops.quantize_mxfp8(d.sorted_tokens), rounds, calls, name="cfg5 mxfp8 quantise sorted tokens")
  report("cfg5 mxfp8 quantise sorted tokens", ms, 0, d.sorted_tokens.numel() * (3 + 1 / 32))
  q, qs = ops.quantize_mxfp8(d.sorted_tokens)
  nm = "cfg5 mxfp8 x mxfp4 gate/up+SiTU scaled MFMA"
  ms = time_fn(lambda: ops.ragged_dot_mxfp8_mxfp4(q, qs, E["gu_packed_tiled"], E["gu_scale_tiled"], d.group_sizes,
                                                  fuse_gateup_activation="situ:4.0:25.0", zero_group=L),
               rounds, calls, name=nm)
  report(nm, ms, f_gu, b_gu - rows * lat * (1 - 1 / 32), peak_key="fp8", rows=rows, experts_hit=hit)
  act = st["act"]
  f_dn = 2.0 * rows * inter * lat
  b_dn = hit * lat * inter * (0.5 + 1 / 32) + rows * inter * 2 + rows * lat * 2
  for lay, sfx in (("checkpoint", ""), ("tiled", "_tiled")):
    nm = f"cfg5 mxfp4 down grouped GEMM ({lay} weights)"
    ms = time_fn(lambda: ops.ragged_dot_mxfp4(act, E["down_packed" + sfx], E["down_scale" + sfx], d.group_sizes,
                                              zero_group=L, weight_layout=lay), rounds, calls, name=nm)
    report(nm, ms, f_dn, b_dn, rows=rows)
  q, qs = ops.quantize_mxfp8(act)
  nm = "cfg5 mxfp8 x mxfp4 down scaled MFMA"
  ms = time_fn(lambda: ops.ragged_dot_mxfp8_mxfp4(q, qs, E["down_packed_tiled"], E["down_scale_tiled"], d.group_sizes,
                                                  zero_group=L), rounds, calls, name=nm)
  report(nm, ms, f_dn, b_dn - rows * inter * (1 - 1 / 32), peak_key="fp8", rows=rows)
  normed = st["normed"]
  ms = time_fn(lambda: layer._dense(normed, layer.up_nk), rounds, calls, name="cfg5 up-proj GEMM 4096x1024x7168")
  report("cfg5 up-proj GEMM 4096x1024x7168", ms, 2.0 * T * lat * H, T * lat * 2 + lat * H * 2 + T * H * 2)


def _capture(layer, hidden):
  """The layer forward as one HIP graph (warm-up on a side stream of default
  priority, then capture); returns (replay, static output)."""
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    layer.forward(hidden)
  torch.cuda.current_stream().wait_stream(side)
  torch.cuda.synchronize()
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    out = layer.forward(hidden)
  torch.cuda.synchronize()
  return g.replay, out


def _layer_sweep(dev, rounds, calls, tokens, label):
  """The config-5 layer at each token count of ``tokens``: the first T of the
  4096 config-5 tokens through the full local-shard forward, timed as
  HIP-graph replays (the serving loop's launch mode).  Bytes per step = the
  dense projection weights (router, down, up) + the MXFP4 weights of the
  local experts that receive rows + the hidden rows in and out; FLOPs = the
  dense projections + the expert GEMMs on the routed rows."""
  from .forward import LocalShardLatentMoE
  c = Config5()
  hidden, w, experts = make_config5(dev, c, "mxfp4")
  layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                              e_score_correction_bias=w["e_score_correction_bias"],
                              down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                              local_expert_start=c.local_start, local_num_experts=c.local_experts,
                              expert_format="mxfp4", experts=experts, capacity_factor=c.capacity_factor)
  L, lat, inter, H = c.local_experts, c.latent, c.intermediate, c.hidden
  dense_bytes = 2 * H * (c.experts + 2 * lat)
  expert_bytes = (2 * inter * lat + lat * inter) * (0.5 + 1 / 32)
  for t in tokens:
    h = hidden[:t].contiguous()
    _, st = layer.forward(h, return_stages=True)
    gs = st["dispatch"].group_sizes.cpu().numpy()
    hit, rows = int((gs[:L] > 0).sum()), int(gs[:L].sum())
    replay, _ = _capture(layer, h)
    nm = f"{label} layer T={t}"
    ms = time_fn(replay, rounds, calls, name=nm, graph=False)
    flops = 2.0 * t * H * (c.experts + 2 * lat) + 2.0 * rows * 3 * inter * lat
    report(nm, ms, flops, dense_bytes + hit * expert_bytes + t * H * 4, tokens=t, experts_hit=hit,
           routed_rows=rows, skinny_expert_gemms=layer._decode_path(t),
           tokens_per_s=round(t / (ms / 1000)) if ms else None)


def bench_decode(dev, rounds, calls):
  """The decode half of the reference's latency sweep (rd.py:553-577:
  num_tokens 1..128 through the same layer)."""
  _layer_sweep(dev, rounds, calls, _DECODE_TOKENS, "decode")


def bench_prefill(dev, rounds, calls):
  """The prefill half of the reference's latency sweep (rd.py:553-577: batch
  1 at seq 128 / 512 / 2048 / 4096 through the same layer)."""
  _layer_sweep(dev, rounds, calls, _PREFILL_TOKENS, "prefill")


def bench_dist(dev, rounds, calls):
  """The reference's ragged_dot group-distribution matrix
  (benchmark_harness.py:100-153): three shapes x five distributions, in its
  call shape (rhs (G, K, N)), bf16 and f32 inputs."""
  from .workloads import HARNESS_DISTRIBUTIONS, HARNESS_SHAPES, harness_group_sizes
  gen = torch.Generator(device=dev).manual_seed(11)
  for shape, (m, k, n, g) in HARNESS_SHAPES.items():
    for dt, tdt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
      lhs = torch.randn((m, k), generator=gen, device=dev).to(tdt)
      rhs = torch.randn((g, k, n), generator=gen, device=dev).to(tdt)
      esz = 2 if dt == "bf16" else 4
      for dist in HARNESS_DISTRIBUTIONS:
        gs = harness_group_sizes(m, g, dist, seed=0)
        gsd = torch.from_numpy(gs).to(dev)
        nm = f"dist ragged_dot {shape} {m}x{k}x{n} G={g} {dist} {dt}"
        ms = time_fn(lambda: ops.ragged_dot(lhs, rhs, gsd), rounds, calls, name=nm)
        report(nm, ms, 2.0 * m * k * n, (int((gs > 0).sum()) * k * n + m * k + m * n) * esz,
               group_sizes=gs.tolist())


def bench_dense(dev, rounds, calls):
  """The layer's two dense projections at config 5 on each backend: the
  fused router + down-projection (4096 x 7168 -> 896 + 1024, f32 out) and the
  up-projection (4096 x 1024 -> 7168, bf16 out)."""
  gen = torch.Generator(device=dev).manual_seed(6)
  T, H, E, lat = 4096, 7168, 896, 1024
  for nm, m, k, n, odt in (("router+down", T, H, E + lat, torch.float32), ("up-proj", T, lat, H, torch.bfloat16)):
    x = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    flops = 2.0 * m * n * k
    nbytes = m * k * 2 + n * k * 2 + m * n * (4 if odt == torch.float32 else 2)
    for backend in ("blaslt", "dense", "hip"):
      name = f"dense {nm} {m}x{k}x{n} [{backend}]"
      ms = time_fn(lambda: ops.dense(x, w, odt, w_layout="nk", backend=backend), rounds, calls, name=name)
      report(name, ms, flops, nbytes)


def bench_copy(dev, rounds, calls):
  """Plain 256 MiB device copy: the calibration kernel for the HBM traffic
  counters (FETCH_SIZE / WRITE_SIZE should read 256 MiB each)."""
  n = 256 << 20
  a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
  b = torch.empty_like(a)
  ms = time_fn(lambda: b.copy_(a), rounds, calls, name="copy 256MiB")
  report("copy 256MiB", ms, 0, 2 * n)


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--only", default="cfg2,cfg3,cfg4,cfg5")
  ap.add_argument("--rounds", type=int, default=10)
  ap.add_argument("--calls", type=int, default=20)
  ap.add_argument("--kernel", default=None, help="only kernels whose name contains this")
  ap.add_argument("--profile", action="store_true", help="run the selected kernels 5x, untimed")
  ap.add_argument("--tokens", default="1,2,4,8,16,32,64,128", help="decode: token counts")
  a = ap.parse_args()
  global _FILTER, _PROFILE, _DECODE_TOKENS
  _FILTER, _PROFILE = a.kernel, a.profile
  _DECODE_TOKENS = tuple(int(x) for x in a.tokens.split(","))
  dev = torch.device("cuda:0")
  for name in a.only.split(","):
    globals()[f"bench_{name}"](dev, a.rounds, a.calls)


if __name__ == "__main__":
  main()
