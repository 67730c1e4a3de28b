"""numpy restatement of the reference LatentMoE hot path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may use this module, and only as the checker / the timed CPU baseline.
The product package never imports it.

Conventions
-----------
* bf16 tensors are carried as float32 arrays whose values are exactly
  representable in bf16 (``bf16_round`` is round-to-nearest-even, the rounding
  XLA applies on every ``astype(bfloat16)`` and after every bf16 op).
* ``dtype`` arguments are the strings ``"f32"`` or ``"bf16"``.
* Every function cites the reference ``file:line`` it restates; paths are
  relative to the reference repository root.  Short aliases:
    ref.py = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py
    rd.py  = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_ragged_dot.py
    deq.py = 05_ragged_dot_on_tpu/mxfp4_dequant.py
    odq.py = 05_ragged_dot_on_tpu/mxfp4_online_dequant_matmul_pallas.py
    gk.py  = 05_ragged_dot_on_tpu/own_gateup_situ_pallas_kernel.py

Pinning (what checks each function against something other than itself) is
listed in ``PINNING`` at the bottom of this file and exercised by
``tests/test_oracle_*.py``.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np

F32 = np.float32

# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
  """Round float32 values to the nearest bf16 (ties to even), returned as float32.

  Same rounding as XLA's f32->bf16 convert, which the reference applies on every
  ``.astype(jnp.bfloat16)`` (e.g. ref.py:293, ref.py:310, ref.py:630).
  NaN stays NaN (quietened); overflow past bf16 max rounds to inf.
  """
  x = np.ascontiguousarray(x, dtype=F32)
  u = x.view(np.uint32)
  bias = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
  r = (u + bias) & np.uint32(0xFFFF0000)
  nan = np.isnan(x)
  if nan.any():
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r)
  return r.astype(np.uint32).view(F32)


def bf16_bits(x) -> np.ndarray:
  """uint16 bit patterns of bf16-valued float32 data (rounds first)."""
  return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bits_to_f32(u16) -> np.ndarray:
  """bf16 bit patterns (uint16 / int16) -> float32 values."""
  u = np.asarray(u16).astype(np.uint16).astype(np.uint32) << np.uint32(16)
  return u.view(F32)


def cast(x, dtype: str) -> np.ndarray:
  x = np.asarray(x, dtype=F32)
  return bf16_round(x) if dtype == "bf16" else x


def promote(a: str, b: str) -> str:
  """JAX dtype promotion between bf16 and f32 (f32 wins)."""
  return "f32" if "f32" in (a, b) else "bf16"


def matmul(a, b, dtype: str) -> np.ndarray:
  """``a @ b`` the way XLA-CPU computes it for ``dtype`` operands: float32
  products and accumulation, one rounding of the result to ``dtype``."""
  out = np.matmul(np.asarray(a, F32), np.asarray(b, F32), dtype=F32)
  return cast(out, dtype)


# ---------------------------------------------------------------------------
# Elementwise math (float32 throughout, like XLA-CPU)
# ---------------------------------------------------------------------------


def sigmoid(x) -> np.ndarray:
  """``jax.nn.sigmoid`` in float32: 1 / (1 + exp(-x))."""
  x = np.asarray(x, F32)
  with np.errstate(over="ignore"):
    return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)


def softmax(x, axis=-1) -> np.ndarray:
  """Row softmax in float32 (the official gate's softmax branch, reference
  06_kimi_k3_golden_validation/generate_pytorch_golden.py:151-156)."""
  x = np.asarray(x, F32)
  m = np.max(x, axis=axis, keepdims=True)
  e = np.exp(x - m)
  return (e / np.sum(e, axis=axis, keepdims=True, dtype=F32)).astype(F32)


def situ_and_mul(gate, up, beta: float, linear_beta: float, dtype: str) -> np.ndarray:
  """Kimi SiTU-GLU, ref.py:296-310: compute in f32, cast back to ``dtype``.

  situ_gate = beta*tanh(g/beta)*sigmoid(g); bounded_up = lb*tanh(u/lb).
  """
  g = np.asarray(gate, F32)
  u = np.asarray(up, F32)
  situ_gate = F32(beta) * np.tanh(g / F32(beta)) * sigmoid(g)
  bounded_up = F32(linear_beta) * np.tanh(u / F32(linear_beta))
  return cast(situ_gate * bounded_up, dtype)


def rms_norm(x, scale, eps: float, dtype: str) -> np.ndarray:
  """ref.py:286-293: f32 mean-square, x*rsqrt(var+eps), cast to input dtype,
  then ``* scale`` in the input dtype."""
  xf = np.asarray(x, F32)
  var = np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32)
  normalized = xf * (F32(1.0) / np.sqrt(var + F32(eps)))
  normalized = cast(normalized, dtype)
  return cast(normalized * np.asarray(scale, F32), dtype)


# ---------------------------------------------------------------------------
# Router (a3)
# ---------------------------------------------------------------------------


# Gate scores: a fully specified binary64 evaluation (the router kernel runs
# the same operation sequence, so the device scores can be compared bit for
# bit).  exp(t): Cody & Waite argument reduction (W. J. Cody and W. Waite,
# "Software Manual for the Elementary Functions", 1980) with fdlibm's ln2
# split (e_exp.c: ln2_hi has 21 trailing zero bits, so n*ln2_hi is exact),
# then the degree-13 Taylor polynomial of e^r on |r| <= ln2/2 in Horner form,
# scaled by 2^n.  Only correctly rounded add/sub/mul/div, floor and ldexp are
# used (numpy evaluates each separately: no fused multiply-add).
GATE_INV_LN2 = float.fromhex("0x1.71547652b82fep+0")
GATE_LN2_HI = float.fromhex("0x1.62e42fee00000p-1")
GATE_LN2_LO = float.fromhex("0x1.a39ef35793c76p-33")
GATE_INV_FACT = tuple(1.0 / math.factorial(j) for j in range(14))  # each correctly rounded


def gate_exp64(t) -> np.ndarray:
  """binary64 e^t by the fixed sequence above; t > 709 -> inf, t < -708 -> 0."""
  t = np.asarray(t, np.float64)
  tc = np.clip(np.where(np.isnan(t), 0.0, t), -708.0, 709.0)
  n = np.floor(tc * GATE_INV_LN2 + 0.5)
  r = (tc - n * GATE_LN2_HI) - n * GATE_LN2_LO
  p = np.full(r.shape, GATE_INV_FACT[13])
  for j in range(12, -1, -1):
    p = p * r + GATE_INV_FACT[j]
  e = np.ldexp(p, n.astype(np.int32))
  e = np.where(t > 709.0, np.inf, np.where(t < -708.0, 0.0, e))
  return np.where(np.isnan(t), np.nan, e)


def gate_sigmoid(x) -> np.ndarray:
  """Router sigmoid (``jax.nn.sigmoid`` of ref.py:349 / ref.py:622) as
  f32(1 / (1 + exp(-x))) evaluated in binary64: the correctly rounded f32
  sigmoid except within ~2^-50 relative of an f32 rounding boundary."""
  x = np.asarray(x, F32)
  with np.errstate(over="ignore", invalid="ignore"):
    return (1.0 / (1.0 + gate_exp64(-x.astype(np.float64)))).astype(F32)


def gate_softmax(x) -> np.ndarray:
  """Row softmax of the official gate's softmax branch
  (06_kimi_k3_golden_validation/generate_pytorch_golden.py:151-156):
  d = f32(x - max), e = exp(d) in binary64, p = f32(e / sum e).  The sum runs
  in a fixed order: 64 partial sums, partial l adding experts l, l+64,
  l+128, ... in turn, then an xor butterfly over distances 32, 16, ..., 1."""
  x = np.asarray(x, F32)
  lead, e_n = x.shape[:-1], x.shape[-1]
  x2 = x.reshape(-1, e_n)
  d = (x2 - np.max(x2, axis=-1, keepdims=True)).astype(F32)
  with np.errstate(over="ignore", invalid="ignore"):
    ex = gate_exp64(d.astype(np.float64))
  chunks = -(-e_n // 64)
  pad = np.zeros((x2.shape[0], chunks * 64), np.float64)
  pad[:, :e_n] = ex
  acc = np.zeros((x2.shape[0], 64), np.float64)
  for c in range(chunks):
    acc = acc + pad[:, c * 64:(c + 1) * 64]
  lanes = np.arange(64)
  for off in (32, 16, 8, 4, 2, 1):
    acc = acc + acc[:, lanes ^ off]
  with np.errstate(invalid="ignore", divide="ignore"):
    return (ex / acc[:, :1]).astype(F32).reshape(*lead, e_n)


def top_k(values, k: int) -> np.ndarray:
  """``jax.lax.top_k`` index semantics: descending by value, equal values ordered
  by ascending index (stable).  Returns int32 (T, k)."""
  v = np.asarray(values, F32)
  order = np.argsort(-v, axis=-1, kind="stable")[..., :k]
  return order.astype(np.int32)


class RouterOut(NamedTuple):
  topk_idx: np.ndarray  # (T, k) int32, global expert ids
  topk_weight: np.ndarray  # (T, k) f32 (or bf16-valued if cast)
  scores: np.ndarray  # (T, E) f32, activation output (before bias)
  scores_for_choice: np.ndarray  # (T, E) f32


def router_from_logits(logits, bias, top_k_: int, renormalize: bool, scaling: float,
                       act: str = "sigmoid", weight_dtype: str = "f32") -> RouterOut:
  """Gate math of ref.py:347-361 (unsharded, weights stay f32) and
  ref.py:601-631 (``_router_gate``: weights cast to the compute dtype at 630).

  scores = act(logits) (``gate_sigmoid`` / ``gate_softmax``); choice =
  scores + bias; idx = top_k(choice);
  w = scores[idx]; if k>1 and renorm: w /= sum(w)+1e-20; w *= scaling.
  The softmax branch follows the official gate
  (06_kimi_k3_golden_validation/generate_pytorch_golden.py:151-156).
  """
  logits = np.asarray(logits, F32)
  if act == "sigmoid":
    scores = gate_sigmoid(logits)
  elif act == "softmax":
    scores = gate_softmax(logits)
  else:
    raise NotImplementedError(act)
  bias = np.zeros(logits.shape[-1], F32) if bias is None else np.asarray(bias, F32)
  choice = (scores + bias[None, :]).astype(F32)
  idx = top_k(choice, top_k_)
  w = np.take_along_axis(scores, idx.astype(np.int64), axis=-1).astype(F32)
  if top_k_ > 1 and renormalize:
    # f32 sum in top-k order (XLA's reduction order is unspecified; this one
    # is fixed so the device result can be compared bit for bit)
    denom = np.zeros(w.shape[:-1] + (1,), F32)
    for j in range(top_k_):
      denom = (denom + w[..., j:j + 1]).astype(F32)
    w = (w / (denom + F32(1e-20))).astype(F32)
  w = (w * F32(scaling)).astype(F32)
  return RouterOut(idx, cast(w, weight_dtype), scores, choice)


def router_gate(hidden, router_weight, bias, config, act: str = "sigmoid",
                weight_dtype: str = "f32") -> tuple[RouterOut, np.ndarray]:
  """``_router_gate`` ref.py:601-631 including the f32 logits matmul
  (ref.py:620): logits = f32(hidden) @ f32(router_weight)."""
  logits = matmul(hidden, router_weight, "f32")
  r = router_from_logits(logits, bias, config.top_k, config.moe_renormalize,
                         config.routed_scaling_factor, act, weight_dtype)
  return r, logits


# ---------------------------------------------------------------------------
# Dispatch (a5, a6, a7)
# ---------------------------------------------------------------------------

MOSAIC_TILE_SIZE = 128  # ref.py:149


def round_up_to_tile(value: int, tile_size: int = MOSAIC_TILE_SIZE) -> int:
  """ref.py:152-153."""
  return -(-value // tile_size) * tile_size


def compute_m_padded(num_tokens: int, top_k_: int, num_experts: int, local_num_experts: int,
                     capacity_factor: float = 2.0, tile_size: int = MOSAIC_TILE_SIZE) -> int:
  """ref.py:825-826 (the jittable form, ``math.ceil`` on the Python float)."""
  expected_total = num_tokens * top_k_ * local_num_experts / num_experts
  return round_up_to_tile(math.ceil(expected_total * capacity_factor), tile_size)


class ShardDispatch(NamedTuple):
  sorted_tokens: np.ndarray  # (m_padded, lat)
  group_sizes: np.ndarray  # (L+1,) int32
  valid_mask: np.ndarray  # (m_padded,) bool
  per_expert_counts: np.ndarray  # (L,) int32
  padded_token_idx: np.ndarray  # (m_padded,) int32, -1 on padding rows
  padded_combine_weight: np.ndarray  # (m_padded,) weight dtype, 0 on padding rows


def filter_and_pad_to_shard(topk_idx, topk_weight, x, top_k_: int, num_experts: int,
                            local_expert_start: int, local_num_experts: int,
                            capacity_factor: float = 2.0, tile_size: int = MOSAIC_TILE_SIZE,
                            m_padded: int | None = None) -> ShardDispatch:
  """Eager ``filter_and_pad_to_shard``, ref.py:658-751.

  Filter slots to [start, start+L), stable argsort by local id, truncate to
  ``m_padded`` (drop the tail), bincount, gather x rows, pad with zero rows /
  token -1 / weight 0.  Written filter-first exactly like the eager reference
  so that the jittable restatement below is checked against an independent
  formulation.
  """
  topk_idx = np.asarray(topk_idx)
  num_tokens = topk_idx.shape[0]
  flat_ids = topk_idx.reshape(-1).astype(np.int64)
  token_of_slot = np.arange(num_tokens * top_k_) // top_k_
  flat_w = np.asarray(topk_weight, F32).reshape(-1)
  local_end = local_expert_start + local_num_experts
  in_shard = (flat_ids >= local_expert_start) & (flat_ids < local_end)
  kept_local = flat_ids[in_shard] - local_expert_start
  kept_tok = token_of_slot[in_shard]
  kept_w = flat_w[in_shard]
  order = np.argsort(kept_local, kind="stable")
  s_local, s_tok, s_w = kept_local[order], kept_tok[order], kept_w[order]
  if m_padded is None:
    m_padded = compute_m_padded(num_tokens, top_k_, num_experts, local_num_experts,
                                capacity_factor, tile_size)
  keep = min(len(s_local), m_padded)
  counts = np.bincount(s_local[:keep], minlength=local_num_experts).astype(np.int32)
  pad = m_padded - keep
  group_sizes = np.concatenate([counts, np.array([pad], np.int32)]).astype(np.int32)
  x = np.asarray(x, F32)
  sorted_tokens = np.zeros((m_padded, x.shape[-1]), F32)
  sorted_tokens[:keep] = x[s_tok[:keep]]
  valid = np.zeros(m_padded, bool)
  valid[:keep] = True
  tok = np.full(m_padded, -1, np.int32)
  tok[:keep] = s_tok[:keep]
  w = np.zeros(m_padded, F32)
  w[:keep] = s_w[:keep]
  return ShardDispatch(sorted_tokens, group_sizes, valid, counts, tok, w)


def filter_and_pad_to_shard_jittable(topk_idx, topk_weight, x, top_k_: int, num_experts: int,
                                     local_expert_start: int, local_num_experts: int,
                                     capacity_factor: float = 2.0,
                                     tile_size: int = MOSAIC_TILE_SIZE,
                                     m_padded: int | None = None,
                                     return_slot_pos: bool = False):
  """Jittable dispatch, ref.py:754-877: sentinel key L for out-of-shard slots,
  pad keys to m_padded, stable argsort, take the first m_padded.

  With ``return_slot_pos`` also returns the inverse permutation ``slot_pos``
  (T*k,) int32: the sorted row of each (token, slot), or -1 when the slot is
  out of shard or truncated (not a reference output; the GPU combine uses it).
  """
  topk_idx = np.asarray(topk_idx)
  num_tokens = topk_idx.shape[0]
  total = num_tokens * top_k_
  flat_ids = topk_idx.reshape(-1).astype(np.int64)
  token_of_slot = np.arange(total) // top_k_
  flat_w = np.asarray(topk_weight, F32).reshape(-1)
  local_end = local_expert_start + local_num_experts
  in_shard = (flat_ids >= local_expert_start) & (flat_ids < local_end)
  key = np.where(in_shard, flat_ids - local_expert_start, local_num_experts)
  if m_padded is None:
    m_padded = compute_m_padded(num_tokens, top_k_, num_experts, local_num_experts,
                                capacity_factor, tile_size)
  pad_amount = max(0, m_padded - total)
  if pad_amount:
    key = np.concatenate([key, np.full(pad_amount, local_num_experts)])
    token_of_slot = np.concatenate([token_of_slot, np.zeros(pad_amount, np.int64)])
    flat_w = np.concatenate([flat_w, np.zeros(pad_amount, F32)])
  full_order = np.argsort(key, kind="stable")
  order = full_order[:m_padded]
  sorted_key = key[order]
  valid = sorted_key < local_num_experts
  tok_all = token_of_slot[order]
  tok = np.where(valid, tok_all, -1).astype(np.int32)
  w = np.where(valid, flat_w[order], F32(0)).astype(F32)
  counts = np.bincount(sorted_key[valid], minlength=local_num_experts).astype(np.int32)
  pad = m_padded - int(counts.sum())
  group_sizes = np.concatenate([counts, np.array([pad], np.int32)]).astype(np.int32)
  x = np.asarray(x, F32)
  sorted_tokens = np.where(valid[:, None], x[tok_all], F32(0)).astype(F32)
  out = ShardDispatch(sorted_tokens, group_sizes, valid, counts, tok, w)
  if not return_slot_pos:
    return out
  slot_pos = np.full(total, -1, np.int32)
  rows = np.nonzero(valid)[0]
  slot_pos[order[rows]] = rows.astype(np.int32)
  return out, slot_pos


def unsharded_dispatch(topk_idx, x, num_experts: int):
  """Unsharded dispatch in ``latent_moe_forward``, ref.py:369-379: stable
  argsort of the flat expert ids, gather, bincount."""
  topk_idx = np.asarray(topk_idx)
  t, k = topk_idx.shape
  flat = topk_idx.reshape(-1).astype(np.int64)
  order = np.argsort(flat, kind="stable")
  token_of_slot = np.arange(t * k) // k
  sorted_token_idx = token_of_slot[order]
  sorted_tokens = np.asarray(x, F32)[sorted_token_idx]
  group_sizes = np.bincount(flat, minlength=num_experts).astype(np.int32)
  return order.astype(np.int32), sorted_tokens, group_sizes


# ---------------------------------------------------------------------------
# Grouped GEMM (a9-a12)
# ---------------------------------------------------------------------------


def ragged_dot(lhs, rhs, group_sizes, dtype: str) -> np.ndarray:
  """Per-group textbook matmul (the semantics of ``tokamax.ragged_dot`` as used at
  rd.py:358-369): rows [cum_g, cum_g+n_g) of lhs times rhs[g]; rows past
  sum(group_sizes) are zero; output dtype = lhs dtype."""
  lhs = np.asarray(lhs, F32)
  rhs = np.asarray(rhs, F32)
  gs = np.asarray(group_sizes).astype(np.int64)
  out = np.zeros((lhs.shape[0], rhs.shape[-1]), F32)
  start = 0
  for g, n in enumerate(gs):
    n = int(n)
    if n > 0:
      out[start:start + n] = np.matmul(lhs[start:start + n], rhs[g], dtype=F32)
    start += n
  return cast(out, dtype)


def prefuse_gateup_weights(expert_gate, expert_up) -> np.ndarray:
  """rd.py:610-641: plain concatenation [gate | up] on the N axis."""
  return np.concatenate([np.asarray(expert_gate, F32), np.asarray(expert_up, F32)], axis=-1)


def ragged_dot_gateup_situ(lhs, rhs_gu, group_sizes, beta: float, linear_beta: float,
                           dtype: str, round_before_act: bool = True) -> np.ndarray:
  """Fused gate/up + SiTU-GLU (rd.py:644-723; epilogue convention gk.py:114-125):
  gate/up accumulators rounded to ``dtype`` before the f32 SiTU, output ``dtype``."""
  n2 = np.asarray(rhs_gu).shape[-1]
  inter = n2 // 2
  acc = ragged_dot(lhs, rhs_gu, group_sizes, "f32")
  g, u = acc[:, :inter], acc[:, inter:]
  if round_before_act:
    g, u = cast(g, dtype), cast(u, dtype)
  return situ_and_mul(g, u, beta, linear_beta, dtype)


def situ_glu_mlp(x, w_gate, w_up, w_down, beta, linear_beta, dtype: str) -> np.ndarray:
  """ref.py:313-327: situ_and_mul(x@Wg, x@Wu) @ Wd, each matmul rounded to dtype."""
  g = matmul(x, w_gate, dtype)
  u = matmul(x, w_up, dtype)
  return matmul(situ_and_mul(g, u, beta, linear_beta, dtype), w_down, dtype)


def local_shard_expert_ffn(sorted_tokens, expert_gate, expert_up, expert_down, group_sizes,
                           config, dtype: str) -> np.ndarray:
  """Naive per-expert loop, ref.py:1486-1528 (the padding bucket is just the
  last group).  Rows past sum(group_sizes) are returned as zero."""
  sorted_tokens = np.asarray(sorted_tokens, F32)
  out = np.zeros((sorted_tokens.shape[0], np.asarray(expert_down).shape[-1]), F32)
  start = 0
  for e, n in enumerate(np.asarray(group_sizes).astype(np.int64)):
    n = int(n)
    if n > 0:
      out[start:start + n] = situ_glu_mlp(
          sorted_tokens[start:start + n], expert_gate[e], expert_up[e], expert_down[e],
          config.activation_situ_beta, config.activation_situ_linear_beta, dtype)
    start += n
  return out


# ---------------------------------------------------------------------------
# Combine (a13)
# ---------------------------------------------------------------------------


def combine_shard_contribution(routed_out, shard_out, padded_token_idx, padded_combine_weight,
                               out_dtype: str, shard_dtype: str, weight_dtype: str) -> np.ndarray:
  """``_combine_shard_contribution``, ref.py:1113-1141:
  routed_out.at[idx].add((shard_out * w[:, None]).astype(routed_out.dtype)).

  Scatter-add semantics restated exactly: the product is formed in the
  promoted dtype of (shard_out, w) and cast to the output dtype; updates are
  applied one row at a time in ascending row order, each add rounded to the
  output dtype; negative indices wrap (numpy/JAX), out-of-range rows drop.
  """
  routed = np.array(routed_out, dtype=F32, copy=True)
  t = routed.shape[0]
  prod_dtype = promote(shard_dtype, weight_dtype)
  weighted = cast(np.asarray(shard_out, F32) * np.asarray(padded_combine_weight, F32)[:, None],
                  prod_dtype)
  weighted = cast(weighted, out_dtype)
  idx = np.asarray(padded_token_idx).astype(np.int64)
  idx = np.where(idx < 0, idx + t, idx)
  ok = (idx >= 0) & (idx < t)
  rows = np.nonzero(ok)[0]
  tok = idx[rows]
  # occurrence rank of each row among the rows of the same token (ascending row)
  o = np.lexsort((rows, tok))
  rows, tok = rows[o], tok[o]
  first = np.r_[True, tok[1:] != tok[:-1]]
  grp_start = np.maximum.accumulate(np.where(first, np.arange(len(tok)), 0))
  rank = np.arange(len(tok)) - grp_start
  for r in range(int(rank.max()) + 1 if len(rank) else 0):
    sel = rank == r
    tt, rr = tok[sel], rows[sel]
    routed[tt] = cast(routed[tt] + weighted[rr], out_dtype)
  return routed


def unsharded_combine(outs, order, topk_weight, num_tokens: int, top_k_: int,
                      compute_dtype: str) -> np.ndarray:
  """ref.py:413-416: inverse permutation, f32 weighted sum over the k slots,
  one cast to the compute dtype."""
  outs = np.asarray(outs, F32)
  unsorted = np.zeros_like(outs)
  unsorted[np.asarray(order)] = outs
  unsorted = unsorted.reshape(num_tokens, top_k_, -1)
  w = np.asarray(topk_weight, F32)
  acc = np.zeros((num_tokens, outs.shape[-1]), F32)
  for j in range(top_k_):
    acc = (acc + unsorted[:, j, :] * w[:, j:j + 1]).astype(F32)
  return cast(acc, compute_dtype), unsorted


# ---------------------------------------------------------------------------
# Full forwards (a15, a16)
# ---------------------------------------------------------------------------


def latent_moe_forward(hidden, w: dict, config, dtype: str, act: str = "sigmoid", logits=None,
                       x=None):
  """``latent_moe_forward``, ref.py:330-435, with the 18 intermediates of
  06_kimi_k3_golden_validation/test_jax_reference_against_pytorch_golden.py:173-275.

  ``w`` holds reference-layout (in, out) arrays with keys router_weight,
  e_score_correction_bias, down_proj, up_proj, expert_gate, expert_up,
  expert_down, norm_scale, shared_gate, shared_up, shared_down.
  ``logits`` / ``x``, when given, replace the router logits GEMM and the
  down-projection (a checker passes the device's own values, so every later
  stage is compared on identical routing and identical gathered rows).
  Returns (final_output, intermediates).
  """
  hidden = cast(hidden, dtype)
  inter: dict[str, np.ndarray] = {}
  t = hidden.shape[0]
  k = config.top_k
  if logits is None:
    r, logits = router_gate(hidden, w["router_weight"], w["e_score_correction_bias"], config,
                            act=act, weight_dtype="f32")
  else:
    logits = np.asarray(logits, F32)
    r = router_from_logits(logits, w["e_score_correction_bias"], config.top_k, config.moe_renormalize,
                           config.routed_scaling_factor, act, "f32")
  inter["router_logits"] = logits
  inter["router_scores_before_bias"] = r.scores
  inter["router_scores_for_choice"] = r.scores_for_choice
  inter["topk_indices"] = r.topk_idx
  inter["topk_weights"] = r.topk_weight
  x = matmul(hidden, w["down_proj"], dtype) if x is None else cast(x, dtype)
  inter["latent_projection"] = x
  order, sorted_tokens, group_sizes = unsharded_dispatch(r.topk_idx, x, config.num_experts)
  inter["sorted_token_indices"] = order
  inter["group_sizes"] = group_sizes
  lat = config.latent_size
  inter_sz = config.intermediate_size
  gate_o = np.zeros((t * k, inter_sz), F32)
  up_o = np.zeros((t * k, inter_sz), F32)
  situ_o = np.zeros((t * k, inter_sz), F32)
  down_o = np.zeros((t * k, lat), F32)
  start = 0
  for e in range(config.num_experts):
    n = int(group_sizes[e])
    if n:
      chunk = sorted_tokens[start:start + n]
      g = matmul(chunk, w["expert_gate"][e], dtype)
      u = matmul(chunk, w["expert_up"][e], dtype)
      s = situ_and_mul(g, u, config.activation_situ_beta, config.activation_situ_linear_beta, dtype)
      d = matmul(s, w["expert_down"][e], dtype)
      gate_o[start:start + n], up_o[start:start + n] = g, u
      situ_o[start:start + n], down_o[start:start + n] = s, d
    start += n
  inter["expert_gate_output"] = gate_o
  inter["expert_up_output"] = up_o
  inter["situ_output"] = situ_o
  inter["expert_down_output"] = down_o
  routed, unsorted = unsharded_combine(down_o, order, r.topk_weight, t, k, dtype)
  inter["routed_output_before_combine"] = unsorted.reshape(t * k, lat)
  inter["routed_output_after_combine"] = routed
  normed = rms_norm(routed, w["norm_scale"], config.rms_norm_eps, dtype)
  inter["normalized_output"] = normed
  up = matmul(normed, w["up_proj"], dtype)
  inter["up_projection_output"] = up
  shared = situ_glu_mlp(hidden, w["shared_gate"], w["shared_up"], w["shared_down"],
                        config.activation_situ_beta, config.activation_situ_linear_beta, dtype)
  inter["shared_expert_output"] = shared
  final = cast(up + shared, dtype)
  inter["final_output"] = final
  return final, inter


def single_shard_forward(hidden, w: dict, shard_gate, shard_up, shard_down, config, dtype: str,
                         local_expert_start: int, local_num_experts: int,
                         capacity_factor: float = 2.0, act: str = "sigmoid",
                         include_shared: bool = True, logits=None, x=None):
  """``latent_moe_forward_ragged_dot_single_shard_jittable``, rd.py:1035-1137,
  with the naive per-expert FFN as the ragged_dot oracle.  ``shard_*`` have
  L+1 experts (the last is the padding bucket).  ``logits`` / ``x``, when
  given, replace the router logits GEMM and the down-projection (see
  ``latent_moe_forward``).  Returns (final, stages)."""
  hidden = cast(hidden, dtype)
  stages: dict[str, np.ndarray] = {}
  x = matmul(hidden, w["down_proj"], dtype) if x is None else cast(x, dtype)
  stages["x"] = x
  if logits is None:
    r, logits = router_gate(hidden, w["router_weight"], w["e_score_correction_bias"], config,
                            act=act, weight_dtype=dtype)
  else:
    logits = np.asarray(logits, F32)
    r = router_from_logits(logits, w["e_score_correction_bias"], config.top_k, config.moe_renormalize,
                           config.routed_scaling_factor, act, dtype)
  stages["router_logits"] = logits
  stages["router_scores_for_choice"] = r.scores_for_choice
  stages["topk_idx"] = r.topk_idx
  stages["topk_weight"] = r.topk_weight
  d = filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, x, config.top_k,
                                       config.num_experts, local_expert_start,
                                       local_num_experts, capacity_factor)
  stages["dispatch"] = d
  shard_out = local_shard_expert_ffn(d.sorted_tokens, shard_gate, shard_up, shard_down,
                                     d.group_sizes, config, dtype)
  stages["shard_out"] = shard_out
  routed = np.zeros((hidden.shape[0], config.latent_size), F32)
  routed = combine_shard_contribution(routed, shard_out, d.padded_token_idx,
                                      d.padded_combine_weight, dtype, dtype, dtype)
  stages["routed_out"] = routed
  normed = rms_norm(routed, w["norm_scale"], config.rms_norm_eps, dtype)
  stages["normed"] = normed
  up = matmul(normed, w["up_proj"], dtype)
  stages["up"] = up
  if include_shared:
    shared = situ_glu_mlp(hidden, w["shared_gate"], w["shared_up"], w["shared_down"],
                          config.activation_situ_beta, config.activation_situ_linear_beta, dtype)
    stages["shared"] = shared
    final = cast(up + shared, dtype)
  else:
    final = up
  return final, stages


# ---------------------------------------------------------------------------
# MXFP4 (a17, a18)
# ---------------------------------------------------------------------------

FP4_E2M1_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], F32)  # deq.py:26


def e8m0_to_f32(scale_u8) -> np.ndarray:
  """E8M0 byte s -> 2^(s-127) as float32, deq.py:63-64 (exact for every byte:
  byte 0 is the f32 denormal 2^-127, byte 255 overflows to inf)."""
  s = np.asarray(scale_u8).astype(np.int64)
  with np.errstate(over="ignore"):
    return np.ldexp(np.float64(1.0), s - 127).astype(F32)


def fp4_e2m1_to_f32(nibble) -> np.ndarray:
  """deq.py:52-54: sign = bit 3, |v| = table[n & 7]; nibble 8 is -0.0."""
  n = np.asarray(nibble).astype(np.int64)
  mag = FP4_E2M1_TABLE[n & 7]
  return (mag * np.where((n & 8) != 0, F32(-1.0), F32(1.0))).astype(F32)


_BYTES = np.arange(256)
_MXFP4_PAIR_LUT = np.stack([fp4_e2m1_to_f32(_BYTES & 0x0F), fp4_e2m1_to_f32(_BYTES >> 4)], axis=-1)
_E8M0_LUT = e8m0_to_f32(_BYTES)


def dequantize_mxfp4(weight_packed, weight_scale) -> np.ndarray:
  """``dequantize_mxfp4``, deq.py:29-67.  packed (..., N, K/2) u8 (low nibble =
  element 2j, high = 2j+1), scale (..., N, K/gs) u8 -> (..., N, K) float32."""
  p = np.asarray(weight_packed, np.uint8)
  *lead, n_out, kh = p.shape
  k = kh * 2
  s = np.asarray(weight_scale, np.uint8)
  ng = s.shape[-1]
  gs = k // ng
  # byte -> (element 2j, element 2j+1) values, then one multiply by the
  # block's scale (the same products as decoding each nibble separately)
  values = _MXFP4_PAIR_LUT[p].reshape(*lead, n_out, ng, gs)
  scale = _E8M0_LUT[s][..., None]
  with np.errstate(invalid="ignore", over="ignore"):
    return (values * scale).astype(F32).reshape(*lead, n_out, k)


def mxfp4_matmul(x, weight_packed, weight_scale, dtype: str = "bf16") -> np.ndarray:
  """y = x @ dequant(W)^T (odq.py:1-36 orientation), bf16 weights exact,
  f32 accumulation, one rounding to ``dtype``."""
  wd = bf16_round(dequantize_mxfp4(weight_packed, weight_scale))
  return matmul(x, wd.T, dtype)


def ragged_dot_mxfp4(lhs, w_packed, w_scale, group_sizes, dtype: str = "bf16",
                     situ: tuple[float, float] | None = None) -> np.ndarray:
  """Grouped x @ deq(W_g)^T with W_g in checkpoint (N, K/2) layout; with
  ``situ=(beta, lb)`` the N axis is [gate | up] and the SiTU-GLU epilogue
  (rounded to ``dtype`` first) is applied."""
  lhs = np.asarray(lhs, F32)
  gs = np.asarray(group_sizes).astype(np.int64)
  n_out = np.asarray(w_packed).shape[1]
  acc = np.zeros((lhs.shape[0], n_out), F32)
  start = 0
  for g, n in enumerate(gs):
    n = int(n)
    if n:
      wd = bf16_round(dequantize_mxfp4(w_packed[g], w_scale[g]))
      acc[start:start + n] = np.matmul(lhs[start:start + n], wd.T, dtype=F32)
    start += n
  if situ is None:
    return cast(acc, dtype)
  inter = n_out // 2
  g_, u_ = cast(acc[:, :inter], dtype), cast(acc[:, inter:], dtype)
  return situ_and_mul(g_, u_, situ[0], situ[1], dtype)


# ---------------------------------------------------------------------------
# MXFP8 activations x MXFP4 weights: the native scaled-MFMA path
# ---------------------------------------------------------------------------
# The reference has no such path (its MXFP4 paths dequantise to bf16); this is
# the build's own definition, following the OCP Microscaling (MX) v1.0
# specification: E4M3 ("fn": no infinities, 0x7F/0xFF NaN, max 448) elements
# with one E8M0 scale per 32 consecutive elements along K; conversion picks the
# shared exponent floor(log2(amax)) - emax_elem (emax_elem = 8 for E4M3), then
# rounds each scaled element to nearest-even and saturates to +-448.

E4M3_MAX = 448.0


def fp8_e4m3_to_f32(code) -> np.ndarray:
  """OCP E4M3 (fn) byte -> float32: sign bit 7, exponent bits 6..3 (bias 7),
  mantissa bits 2..0; exponent 0 is subnormal (m/8 * 2^-6); 0x7F / 0xFF NaN."""
  c = np.asarray(code).astype(np.int64)
  e = (c >> 3) & 15
  m = c & 7
  mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.ldexp(1.0, e - 7))
  mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
  return (np.where((c & 0x80) != 0, -mag, mag)).astype(F32)


def f32_to_fp8_e4m3(x) -> np.ndarray:
  """float -> OCP E4M3 byte, round to nearest even, saturating to +-448
  (infinities saturate too); NaN -> 0x7F."""
  x = np.asarray(x, np.float64)
  sign = np.where(np.signbit(x), 0x80, 0).astype(np.int64)
  a = np.minimum(np.abs(np.nan_to_num(x, nan=0.0, posinf=E4M3_MAX, neginf=-E4M3_MAX)), E4M3_MAX)
  with np.errstate(divide="ignore"):
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
  e = np.maximum(e, -6.0)  # below 2^-6: subnormal grid of 2^-9
  quantum = np.ldexp(1.0, (e - 3).astype(np.int64))
  q = np.rint(a / quantum) * quantum  # numpy rint: ties to even
  q = np.minimum(q, E4M3_MAX)
  with np.errstate(divide="ignore"):
    qe = np.floor(np.log2(np.where(q > 0, q, 1.0))).astype(np.int64)
  normal = q >= 2.0 ** -6
  code_n = ((qe + 7) << 3) | np.rint((q / np.ldexp(1.0, qe) - 1.0) * 8.0).astype(np.int64)
  code_s = np.rint(q / 2.0 ** -9).astype(np.int64)
  code = np.where(normal, code_n, code_s) | sign
  code = np.where(np.isnan(x), 0x7F, code)
  return code.astype(np.uint8)


def quantize_mxfp8(x) -> tuple[np.ndarray, np.ndarray]:
  """(M, K) float -> (codes (M, K) u8 E4M3, scales (M, K/32) u8 E8M0), blocks of
  32 along K.  Shared exponent floor(log2(max|x|)) - 8 over the block's finite
  values, clamped to [-127, 127] (an all-zero block gets byte 0); elements are
  x * 2^-exp converted by ``f32_to_fp8_e4m3``."""
  x = np.asarray(x, np.float64)
  m, k = x.shape
  blocks = x.reshape(m, k // 32, 32)
  fin = np.where(np.isfinite(blocks), np.abs(blocks), 0.0)
  amax = fin.max(axis=-1)
  with np.errstate(divide="ignore"):
    ex = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - 8, -127)
  ex = np.clip(ex, -127, 127).astype(np.int64)
  scaled = blocks * np.ldexp(1.0, -ex)[..., None]
  codes = f32_to_fp8_e4m3(scaled).reshape(m, k)
  return codes, (ex + 127).astype(np.uint8)


def dequantize_mxfp8(codes, scales) -> np.ndarray:
  """E4M3 codes (M, K) x E8M0 scales (M, K/32) -> float64 values (exact)."""
  v = fp8_e4m3_to_f32(codes).astype(np.float64)
  s = np.ldexp(1.0, np.asarray(scales).astype(np.int64) - 127)
  return v * np.repeat(s, 32, axis=-1)


def ragged_dot_mxfp8_mxfp4(lhs_codes, lhs_scales, w_packed, w_scale, group_sizes, dtype: str = "f32",
                           situ: tuple[float, float] | None = None) -> np.ndarray:
  """Grouped deq(A) @ deq(W_g)^T with MXFP8 activations and MXFP4 weights in
  checkpoint (N, K/2) layout.  Every product is exact; the sums are taken in
  float64 and rounded once to ``dtype`` (``situ``: gate/up rounded to bf16,
  SiTU-GLU, output bf16, as in the bf16 fused epilogue).  Rows past
  sum(group_sizes) are zero."""
  a = dequantize_mxfp8(lhs_codes, lhs_scales)
  gs = np.asarray(group_sizes).astype(np.int64)
  n_out = np.asarray(w_packed).shape[1]
  acc = np.zeros((a.shape[0], n_out), np.float64)
  start = 0
  for g, n in enumerate(gs):
    n = int(n)
    if n:
      wd = dequantize_mxfp4(w_packed[g], w_scale[g]).astype(np.float64)
      acc[start:start + n] = a[start:start + n] @ wd.T
    start += n
  if situ is None:
    return cast(acc.astype(F32), dtype)
  inter = n_out // 2
  g_, u_ = bf16_round(acc[:, :inter].astype(F32)), bf16_round(acc[:, inter:].astype(F32))
  return situ_and_mul(g_, u_, situ[0], situ[1], "bf16")


# ---------------------------------------------------------------------------
# MXFP6 activations x MXFP4 weights: the scaled MFMA at the FP4/FP6 rate
# ---------------------------------------------------------------------------
# No reference counterpart either: OCP MX v1.0 FP6 E2M3 elements (sign, 2-bit
# exponent with bias 1, 3-bit mantissa; no infinities or NaN; max 7.5,
# subnormal spacing 1/8) with one E8M0 scale per 32 elements along K.  The
# shared exponent is floor(log2(amax)) - 2 (emax_elem = 2 for E2M3); scaled
# elements are rounded to nearest-even and saturate to +-7.5.  The packed
# layout (the build's own) puts element j of a 32-element block at bits
# 6j .. 6j+5 of the block's 24 little-endian bytes, i.e. (M, K) codes become
# (M, K*3/4) bytes.

E2M3_MAX = 7.5


def fp6_e2m3_to_f32(code) -> np.ndarray:
  """E2M3 code (6 bits) -> float32: sign bit 5, exponent bits 4..3 (bias 1),
  mantissa bits 2..0; exponent 0 is subnormal (m/8)."""
  c = np.asarray(code).astype(np.int64)
  e = (c >> 3) & 3
  m = c & 7
  mag = np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * np.ldexp(1.0, e - 1))
  return np.where((c & 0x20) != 0, -mag, mag).astype(F32)


def f32_to_fp6_e2m3(x) -> np.ndarray:
  """float -> E2M3 code, round to nearest even on the representable grid,
  saturating to +-7.5 (infinities too); NaN -> 0.  The grid spacing is 1/8
  below 2, 1/4 in [2, 4) and 1/2 in [4, 8), and the code of a magnitude is
  8 * binade + the rounded mantissa count, so a carry out of the mantissa
  moves into the next binade by itself."""
  x = np.asarray(x, np.float64)
  sign = np.where(np.signbit(x), 0x20, 0).astype(np.int64)
  a = np.minimum(np.abs(np.nan_to_num(x, nan=0.0, posinf=E2M3_MAX, neginf=-E2M3_MAX)), E2M3_MAX)
  code = np.where(a < 2.0, np.rint(a * 8.0),
                  np.where(a < 4.0, 8 + np.rint(a * 4.0), 16 + np.rint(a * 2.0))).astype(np.int64)
  return (code | sign).astype(np.uint8)


def quantize_mxfp6(x) -> tuple[np.ndarray, np.ndarray]:
  """(M, K) float -> (codes (M, K) u8 E2M3 (6 bits used), scales (M, K/32) u8
  E8M0): shared exponent floor(log2(max|x|)) - 2 over the block's finite
  values, clamped to [-127, 127] (an all-zero block gets byte 0)."""
  x = np.asarray(x, np.float64)
  m, k = x.shape
  blocks = x.reshape(m, k // 32, 32)
  fin = np.where(np.isfinite(blocks), np.abs(blocks), 0.0)
  amax = fin.max(axis=-1)
  with np.errstate(divide="ignore"):
    ex = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - 2, -127)
  ex = np.clip(ex, -127, 127).astype(np.int64)
  scaled = blocks * np.ldexp(1.0, -ex)[..., None]
  codes = f32_to_fp6_e2m3(scaled).reshape(m, k)
  return codes, (ex + 127).astype(np.uint8)


def pack_fp6(codes) -> np.ndarray:
  """(M, K) 6-bit codes -> (M, K*3/4) bytes: element j of each 32-element
  block at bits 6j .. 6j+5 of the block's 24 little-endian bytes."""
  c = np.asarray(codes).astype(np.uint64)
  m, k = c.shape
  blk = c.reshape(m, k // 32, 8, 4)  # 4 elements -> 3 bytes
  v = blk[..., 0] | (blk[..., 1] << 6) | (blk[..., 2] << 12) | (blk[..., 3] << 18)
  out = np.stack([(v >> (8 * b)) & 0xFF for b in range(3)], axis=-1).astype(np.uint8)
  return out.reshape(m, k * 3 // 4)


def unpack_fp6(packed, k: int) -> np.ndarray:
  """Inverse of ``pack_fp6``."""
  p = np.asarray(packed).astype(np.uint64)
  m = p.shape[0]
  t = p.reshape(m, k // 4, 3)
  v = t[..., 0] | (t[..., 1] << 8) | (t[..., 2] << 16)
  return np.stack([(v >> (6 * e)) & 0x3F for e in range(4)], axis=-1).reshape(m, k).astype(np.uint8)


def dequantize_mxfp6(codes, scales) -> np.ndarray:
  """E2M3 codes (M, K) x E8M0 scales (M, K/32) -> float64 values (exact)."""
  v = fp6_e2m3_to_f32(codes).astype(np.float64)
  s = np.ldexp(1.0, np.asarray(scales).astype(np.int64) - 127)
  return v * np.repeat(s, 32, axis=-1)


def ragged_dot_mxfp6_mxfp4(lhs_codes, lhs_scales, w_packed, w_scale, group_sizes, dtype: str = "f32"
                           ) -> np.ndarray:
  """Grouped deq(A) @ deq(W_g)^T with MXFP6 activations (unpacked codes) and
  MXFP4 weights in checkpoint (N, K/2) layout; float64 sums rounded once to
  ``dtype``.  Rows past sum(group_sizes) are zero."""
  a = dequantize_mxfp6(lhs_codes, lhs_scales)
  gs = np.asarray(group_sizes).astype(np.int64)
  n_out = np.asarray(w_packed).shape[1]
  acc = np.zeros((a.shape[0], n_out), np.float64)
  start = 0
  for g, n in enumerate(gs):
    n = int(n)
    if n:
      wd = dequantize_mxfp4(w_packed[g], w_scale[g]).astype(np.float64)
      acc[start:start + n] = a[start:start + n] @ wd.T
    start += n
  return cast(acc.astype(F32), dtype)


# ---------------------------------------------------------------------------
# Block-scaled fp8 weights (a19)
# ---------------------------------------------------------------------------


def dequantize_fp8_blockscaled(rhs_q, rhs_scale) -> np.ndarray:
  """The reference's dequantisation of fp8 weights with f32 block scales,
  rd.py:2815 (one block per column) and rd.py:2934-2935 (32-row blocks):
  (rhs_q.astype(f32) * scale).astype(bf16), with rhs_q (G, K, N) E4M3 codes
  and rhs_scale (G, K/bs, 1, N).  Returns bf16-valued float32 (G, K, N)."""
  q = fp8_e4m3_to_f32(np.asarray(rhs_q, np.uint8))
  g, k, n = q.shape
  sc = np.asarray(rhs_scale, F32)
  bs = k // sc.shape[1]
  with np.errstate(over="ignore", invalid="ignore"):
    deq = (q.reshape(g, k // bs, bs, n) * sc.reshape(g, k // bs, 1, n)).astype(F32)
  return bf16_round(deq.reshape(g, k, n))


def ragged_dot_fp8_scaled(lhs, rhs_q, rhs_scale, group_sizes, dtype: str = "bf16",
                          situ: tuple[float, float] | None = None) -> np.ndarray:
  """``PallasMosaicTpuV2RaggedDot()(lhs, rhs_q, rhs_scale=...)`` as the
  reference checks it (rd.py:2815-2821, rd.py:2934-2941): ragged_dot of lhs
  with the dequantised bf16 weights, f32 accumulation, one rounding to
  ``dtype`` (``situ``: the fused SiTU-GLU epilogue on [gate | up])."""
  w = dequantize_fp8_blockscaled(rhs_q, rhs_scale)
  if situ is None:
    return ragged_dot(lhs, w, group_sizes, dtype)
  return ragged_dot_gateup_situ(lhs, w, group_sizes, situ[0], situ[1], dtype)


PINNING = {
    # Keys name every public function of this module ("a / b" when one check
    # pins several); ``tests/test_oracle_basics.py`` asserts the coverage.
    "bf16_round / bf16_bits / bits_to_f32 / cast":
        "torch's bfloat16 cast over random, denormal and edge floats, ties to even; all 65536 bf16 bit "
        "patterns decoded against torch's bfloat16 view and round-tripped (test_oracle_basics.py)",
    "promote": "torch.promote_types over every bf16/f32 pair, which JAX's promotion lattice agrees with "
               "for these two types (test_oracle_basics.py)",
    "matmul": "a float64 product: the f32 result within f32 accumulation error, the bf16 result its "
              "single rounding, within half a bf16 ulp plus that error (test_oracle_basics.py)",
    "sigmoid / softmax / situ_and_mul / rms_norm": "float64 closed forms (test_oracle_basics.py)",
    "gate_exp64 / gate_sigmoid / gate_softmax":
        "libm exp within 1 ulp (planted ln2/Taylor mistakes fail), sigmoid correctly rounded vs extended "
        "precision, softmax within 1 ulp (test_oracle_basics.py)",
    "top_k": "brute-force sort by (-value, index) with ties (test_oracle_basics.py)",
    "router_from_logits / router_gate": "golden bundles router_* / topk_* (6 stages); renormalisation "
                                        "order KAT (test_oracle_golden.py, test_oracle_basics.py)",
    "round_up_to_tile / compute_m_padded":
        "literal values; the reference's m_padded table (expert_ffn_roofline.py:42-47) at its token sweep "
        "(rd.py:1843) (test_oracle_composites.py, test_oracle_dispatch.py)",
    "filter_and_pad_to_shard / filter_and_pad_to_shard_jittable":
        "literal KATs from test_sharded_routing_local.py, brute force, eager == jittable "
        "(test_oracle_dispatch.py)",
    "unsharded_dispatch / unsharded_combine / latent_moe_forward / situ_glu_mlp":
        "golden group_sizes, canonical sorted_token_indices and every stage of the six bundles "
        "(test_oracle_golden.py)",
    "ragged_dot / local_shard_expert_ffn": "golden expert_* / situ_output stages, brute-force per-row "
                                           "dot (test_oracle_basics.py, test_oracle_dispatch.py)",
    "combine_shard_contribution": "sharded sum == unsharded forward over 4 configs, literal padding KAT, "
                                  "rounding-order KAT (test_oracle_dispatch.py)",
    "single_shard_forward": "one shard holding every expert equals latent_moe_forward stage by stage; "
                            "the routed outputs of all shards sum to the unsharded one "
                            "(test_oracle_dispatch.py)",
    "prefuse_gateup_weights / ragged_dot_gateup_situ / mxfp4_matmul / ragged_dot_mxfp4":
        "explicit [gate | up] layout; float64 per-row brute force with the OCP E2M1 table, gate/up swap "
        "and nibble-order mistakes fail (test_oracle_composites.py)",
    "e8m0_to_f32 / fp4_e2m1_to_f32 / dequantize_mxfp4":
        "OCP MX v1.0 bit formulas over all 256 scale bytes and all 16 codes; exhaustive 256 bytes x edge "
        "scales; literal KAT (test_oracle_basics.py)",
    "fp8_e4m3_to_f32 / f32_to_fp8_e4m3":
        "all 256 codes and a dense sweep incl. ties and subnormals vs torch.float8_e4m3fn "
        "(test_oracle_mxfp8.py)",
    "quantize_mxfp8 / dequantize_mxfp8":
        "OCP MX closed form (exponent choice, saturation, zero block), grid values round-trip exactly, "
        "planted exponent mistake fails (test_oracle_mxfp8.py)",
    "ragged_dot_mxfp8_mxfp4": "brute-force triple loop on small inputs; equals the bf16 oracle when the "
                              "activations are on the E4M3 grid (test_oracle_mxfp8.py)",
    "dequantize_fp8_blockscaled / ragged_dot_fp8_scaled":
        "torch float8_e4m3fn -> f32 * scale -> bf16 casts, all 256 codes x block sizes K and 32 "
        "(test_oracle_mxfp8.py)",
    "fp6_e2m3_to_f32 / f32_to_fp6_e2m3 / quantize_mxfp6 / dequantize_mxfp6 / pack_fp6 / unpack_fp6":
        "the OCP E2M3 value table (monotone codes, spacing 1/8, 1/4, 1/2), brute-force nearest-even search "
        "over a dense sweep with every midpoint, the MX exponent closed form (amax / 2^X in [4, 8)), grid "
        "values round-trip, a planted emax mistake fails, one-hot bit placement of the packing "
        "(test_oracle_mxfp6.py)",
    "ragged_dot_mxfp6_mxfp4": "brute-force triple loop on small inputs (test_oracle_mxfp6.py)",
}
