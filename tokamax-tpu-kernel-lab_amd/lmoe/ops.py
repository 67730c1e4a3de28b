"""Reference-shaped operators of the LatentMoE expert hot path on the HIP kernels.

Each function keeps the name, argument meaning, output dtype and error
behaviour of the reference function it replaces (cited file:line, reference
paths relative to the reference repository; ref.py =
05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py, rd.py =
05_ragged_dot_on_tpu/kimi_k3_latent_moe_ragged_dot.py).  Tensors are torch
tensors on the GPU; outputs are new tensors (the reference's JAX arrays are
immutable).  Every operator runs a kernel of liblmoe.so on the current torch
stream; nothing falls back to torch or the CPU.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch

from . import _lib
from ._lib import check, lib

MOSAIC_TILE_SIZE = 128  # ref.py:149
_MOSAIC_TILE_SIZE = MOSAIC_TILE_SIZE  # the reference's name

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _dt(t: torch.Tensor) -> int:
  try:
    return _DT[t.dtype]
  except KeyError:
    raise NotImplementedError(f"dtype {t.dtype} is not supported (bf16 / f32 only)") from None


def _dev_rows(t: torch.Tensor) -> torch.Tensor:
  """A GPU 2-D tensor whose rows may be strided (unit column stride, row
  stride >= width); anything else is made contiguous."""
  if not t.is_cuda:
    raise ValueError("LatentMoE operators need GPU tensors (no CPU fallback)")
  if t.dim() != 2:
    raise ValueError("expected a 2-D tensor")
  if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
    t = t.contiguous()
  return t


def _dev(*ts: torch.Tensor) -> None:
  for t in ts:
    if t is None:
      continue
    if not t.is_cuda:
      raise ValueError("LatentMoE operators need GPU tensors (no CPU fallback)")
    if not t.is_contiguous():
      raise ValueError("LatentMoE operators need contiguous tensors")


def _p(t: torch.Tensor | None) -> int | None:
  return None if t is None else t.data_ptr()


def _stream() -> int:
  return torch.cuda.current_stream().cuda_stream


def _check_groups(group_sizes: torch.Tensor, g: int) -> None:
  """The kernels read exactly g group sizes."""
  if group_sizes.dtype != torch.int32:
    raise ValueError("group_sizes must be int32")
  if tuple(group_sizes.shape) != (g,):
    raise ValueError(f"group_sizes {tuple(group_sizes.shape)} for {g} groups")


def _check_topk(topk_idx: torch.Tensor, topk_weight: torch.Tensor) -> None:
  """The dispatch reads T*k ids and T*k weights."""
  if topk_idx.dtype != torch.int32 or topk_idx.dim() != 2:
    raise ValueError(f"topk_idx must be int32 (T, k), got {topk_idx.dtype} {tuple(topk_idx.shape)}")
  if tuple(topk_weight.shape) != tuple(topk_idx.shape):
    raise ValueError(f"topk_weight {tuple(topk_weight.shape)} vs topk_idx {tuple(topk_idx.shape)}")
  if topk_weight.dtype not in (torch.float32, torch.bfloat16):
    raise ValueError(f"topk_weight must be float32 or bfloat16, got {topk_weight.dtype}")


def _check_rows(x: torch.Tensor, t: int) -> None:
  """Token rows: one per token."""
  if x.dim() != 2 or x.shape[0] != t:
    raise ValueError(f"x {tuple(x.shape)}: want ({t}, lat) token rows")


def _row_strided(x: torch.Tensor) -> bool:
  """Rows further apart than their width (e.g. a column slice of a wider
  array), judged by the strides themselves: torch calls a single-row slice
  contiguous whatever its row stride, and a one-token batch must take the
  same path as a larger one."""
  return x.stride(-1) != 1 or (x.shape[0] > 0 and x.stride(0) != x.shape[-1])


def _workspace(nbytes: int, device) -> torch.Tensor:
  return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# a9 / a12: grouped GEMMs
# ---------------------------------------------------------------------------


def ragged_dot(lhs: torch.Tensor, rhs: torch.Tensor, group_sizes: torch.Tensor, precision=None,
               implementation: str | None = None, preferred_element_type: torch.dtype | None = None,
               *, rhs_layout: str = "gkn", zero_group: int = -1) -> torch.Tensor:
  """``tokamax.ragged_dot(lhs, rhs, group_sizes)`` (call shape rd.py:358-369).

  lhs (M, K); rhs (G, K, N) for ``rhs_layout="gkn"`` (the reference layout) or
  (G, N, K) for ``"gnk"`` (prepared, k-contiguous); group_sizes (G,) int32 on
  the device (never read on the host).  Output (M, N) in lhs dtype (or
  ``preferred_element_type``); rows past sum(group_sizes) are zero.
  ``implementation`` accepts only None / "hip": there is one backend.
  ``precision`` is accepted for signature compatibility: f32 operands are
  always computed at full f32 precision (the reference needs
  Precision.HIGHEST for that, trg.py:150-163).
  ``zero_group`` names a group computed as exact zeros without reading its
  weights (the padding bucket, whose rows are zero).
  """
  if implementation not in (None, "hip"):
    raise NotImplementedError(f"implementation={implementation!r}: only the HIP backend exists")
  _dev(lhs, rhs, group_sizes)
  if lhs.dim() != 2 or rhs.dim() != 3:
    raise ValueError(f"ragged_dot: lhs {tuple(lhs.shape)} / rhs {tuple(rhs.shape)} ranks")
  if group_sizes.dtype != torch.int32:
    raise ValueError("group_sizes must be int32")
  m, k = lhs.shape
  g = rhs.shape[0]
  if rhs_layout == "gkn":
    layout, kk, n = _lib.RHS_GKN, rhs.shape[1], rhs.shape[2]
  elif rhs_layout == "gnk":
    layout, n, kk = _lib.RHS_GNK, rhs.shape[1], rhs.shape[2]
  else:
    raise ValueError(f"rhs_layout {rhs_layout!r}")
  if kk != k or group_sizes.shape != (g,):
    raise ValueError(f"ragged_dot: shapes lhs {tuple(lhs.shape)} rhs {tuple(rhs.shape)} "
                     f"group_sizes {tuple(group_sizes.shape)}")
  if rhs.dtype != lhs.dtype:
    raise NotImplementedError(f"mixed lhs {lhs.dtype} / rhs {rhs.dtype}")
  out_dtype = preferred_element_type or lhs.dtype
  if m == 0 or n == 0 or k == 0:  # nothing to read: an empty sum is zero
    return torch.zeros((m, n), dtype=out_dtype, device=lhs.device)
  if lhs.dtype == torch.bfloat16 and (k % 8 or n % 8):
    # off the bf16 kernels' 8-element grid: the any-shape f32 kernel on the
    # same values (bf16 products are exact in f32, accumulated in f32 as on
    # the bf16 path), then one rounding to the output dtype
    out = ragged_dot(lhs.float(), rhs.float(), group_sizes, preferred_element_type=torch.float32,
                     rhs_layout=rhs_layout, zero_group=zero_group)
    return out if out_dtype == torch.float32 else out.to(out_dtype)
  # reference-layout (G, K, N) weights are read as they lie: the kernel
  # transposes each B tile in LDS (ds_read_b64_tr_b16), as fast as prepared
  # (G, N, K) weights and faster than transposing them first
  out = torch.empty((m, n), dtype=out_dtype, device=lhs.device)
  check(lib().lmoe_ragged_dot(_p(lhs), _dt(lhs), _p(rhs), layout, _p(group_sizes), m, k, n, g,
                              zero_group, _p(out), _dt(out), _stream()), "ragged_dot")
  return out


def parse_fused_activation(spec: str) -> tuple[float, float]:
  """"situ:<beta>:<linear_beta>" (the op-class string of rd.py:713-720)."""
  parts = spec.split(":")
  if len(parts) != 3 or parts[0] != "situ":
    raise NotImplementedError(f"fuse_gateup_activation={spec!r}: only 'situ:<beta>:<beta_lin>'")
  beta, beta_lin = float(parts[1]), float(parts[2])
  if not (0.0 < beta < math.inf and 0.0 < beta_lin < math.inf):
    raise ValueError(f"fuse_gateup_activation={spec!r}: beta and beta_lin must be positive and finite "
                     "(each divides a tanh argument)")
  return beta, beta_lin


def ragged_dot_gateup_situ(lhs: torch.Tensor, rhs_gu: torch.Tensor, group_sizes: torch.Tensor,
                           beta: float, linear_beta: float, *, rhs_layout: str = "gkn",
                           zero_group: int = -1, round_before_act: bool = True) -> torch.Tensor:
  """One grouped GEMM against the prefused [gate | up] weight with the SiTU-GLU
  epilogue in registers (rd.py:644-723; gate/up rounded to bf16 before SiTU as
  in gk.py:114-125).  rhs_gu (G, K, 2I) ("gkn") or (G, 2I, K) ("gnk"); out (M, I)."""
  _dev(lhs, rhs_gu, group_sizes)
  f32 = lhs.dtype == torch.float32 and rhs_gu.dtype == torch.float32
  if not f32 and (lhs.dtype != torch.bfloat16 or rhs_gu.dtype != torch.bfloat16):
    raise NotImplementedError("fused gate/up SiTU takes bf16 (or f32) lhs and weights of one dtype")
  if lhs.dim() != 2 or rhs_gu.dim() != 3:
    raise ValueError(f"gateup: lhs {tuple(lhs.shape)} / rhs {tuple(rhs_gu.shape)} ranks")
  m, k = lhs.shape
  g = rhs_gu.shape[0]
  if rhs_layout == "gkn":
    layout, kk, n2 = _lib.RHS_GKN, rhs_gu.shape[1], rhs_gu.shape[2]
  elif rhs_layout == "gnk":
    layout, n2, kk = _lib.RHS_GNK, rhs_gu.shape[1], rhs_gu.shape[2]
  else:
    raise ValueError(f"rhs_layout {rhs_layout!r}")
  if kk != k or n2 % 2:
    raise ValueError(f"gateup shapes lhs {tuple(lhs.shape)} rhs {tuple(rhs_gu.shape)}")
  _check_groups(group_sizes, g)
  inter = n2 // 2
  if f32 or m == 0 or k == 0 or inter == 0 or k % 8 or inter % 8:
    # f32 (rounding to f32 before the activation is the identity), empty or
    # off-grid problems: the two halves as ragged_dots, then the SiTU-GLU
    if rhs_layout == "gkn":
      gate, up = rhs_gu[:, :, :inter].contiguous(), rhs_gu[:, :, inter:].contiguous()
    else:
      gate, up = rhs_gu[:, :inter].contiguous(), rhs_gu[:, inter:].contiguous()
    # gate / up rounded to the lhs dtype before the activation, or kept f32
    pet = None if f32 or round_before_act else torch.float32
    gate_out = ragged_dot(lhs, gate, group_sizes, preferred_element_type=pet, rhs_layout=rhs_layout,
                          zero_group=zero_group)
    up_out = ragged_dot(lhs, up, group_sizes, preferred_element_type=pet, rhs_layout=rhs_layout,
                        zero_group=zero_group)
    act = _situ_and_mul(gate_out, up_out, beta, linear_beta)
    return act if act.dtype == lhs.dtype else act.to(lhs.dtype)
  out = torch.empty((m, inter), dtype=torch.bfloat16, device=lhs.device)
  check(lib().lmoe_ragged_dot_gateup_situ(_p(lhs), _p(rhs_gu), layout, _p(group_sizes), m, k, inter,
                                          g, zero_group, beta, linear_beta, int(round_before_act),
                                          _p(out), _stream()), "ragged_dot_gateup_situ")
  return out


def ragged_dot_fp8_scaled(lhs: torch.Tensor, rhs_q: torch.Tensor, rhs_scale: torch.Tensor,
                          group_sizes: torch.Tensor, *, fuse_gateup_activation: str | None = None,
                          zero_group: int = -1) -> torch.Tensor:
  """The reference's block-scaled fp8 weight path (rd.py:2789-2811, one scale
  per column: rhs_scale (G, 1, 1, N); rd.py:2836-2953, one per 32 rows of K:
  (G, K/32, 1, N)): rhs_q (G, K, N) float8_e4m3fn (or its uint8 codes),
  rhs_scale (G, K/bs, 1, N) float32.  Each weight is used as
  bf16(f32(q) * scale), the reference's dequantisation, then a bf16 ragged_dot
  with f32 accumulation; output (M, N) bf16, or (M, N/2) with the SiTU-GLU
  epilogue."""
  _dev(lhs, rhs_q, rhs_scale, group_sizes)
  if lhs.dtype != torch.bfloat16:
    raise NotImplementedError("the fp8-weight ragged_dot takes bf16 activations")
  if rhs_q.dtype not in (torch.float8_e4m3fn, torch.uint8):
    raise ValueError(f"rhs must be float8_e4m3fn (or its uint8 codes), got {rhs_q.dtype}")
  if rhs_scale.dtype != torch.float32:
    raise ValueError(f"rhs_scale must be float32, got {rhs_scale.dtype}")
  if group_sizes.dtype != torch.int32:
    raise ValueError("group_sizes must be int32")
  m, k = lhs.shape
  if rhs_q.dim() != 3 or rhs_q.shape[1] != k:
    raise ValueError(f"rhs {tuple(rhs_q.shape)} vs lhs {tuple(lhs.shape)}: want (G, K, N)")
  g, _, n = rhs_q.shape
  if (rhs_scale.dim() != 4 or rhs_scale.shape[0] != g or rhs_scale.shape[2] != 1 or rhs_scale.shape[3] != n
      or rhs_scale.shape[1] == 0 or k % rhs_scale.shape[1]):
    raise ValueError(f"rhs_scale {tuple(rhs_scale.shape)}: want (G, K/block_size, 1, N) for rhs {tuple(rhs_q.shape)}")
  if group_sizes.shape != (g,):
    raise ValueError(f"group_sizes {tuple(group_sizes.shape)} for {g} groups")
  bs = k // rhs_scale.shape[1]
  epi, b, bl, width = _lib.EPI_NONE, 0.0, 0.0, n
  if fuse_gateup_activation is not None:
    b, bl = parse_fused_activation(fuse_gateup_activation)
    epi, width = _lib.EPI_SITU, n // 2
  out = torch.empty((m, width), dtype=torch.bfloat16, device=lhs.device)
  check(lib().lmoe_ragged_dot_fp8_scaled(_p(lhs), _p(rhs_q), _p(rhs_scale), bs, _p(group_sizes), m, k, n, g,
                                         zero_group, epi, b, bl, _p(out), _stream()), "ragged_dot_fp8_scaled")
  return out


class HipRaggedDot:
  """Op-class form of the grouped GEMM, mirroring how the reference reaches
  the fused and scaled paths through ``PallasMosaicTpuV2RaggedDot()(...)``
  (rd.py:713-720, rd.py:2804-2811): ``op(lhs, rhs, group_sizes=...,
  fuse_gateup_activation="situ:b:bl", rhs_scale=..., maybe_quantize_lhs=...)``.

  ``rhs_scale`` follows the reference's contract when it is float32: rhs is
  (G, K, N) float8_e4m3fn and rhs_scale (G, K/bs, 1, N)
  (``ragged_dot_fp8_scaled``).  A uint8 ``rhs_scale`` selects this build's
  MXFP4 weights instead: rhs (G, N, K/2) packed E2M1 codes, rhs_scale
  (G, N, K/32) E8M0 bytes (``ragged_dot_mxfp4``).  ``maybe_quantize_lhs=True``
  quantises the activations to MXFP8 on the MXFP4 path (the native scaled
  MFMA, tiled weights from ``mxfp4_tile_weights``); the fp8 path has no
  activation quantisation and raises NotImplementedError for it."""

  def __init__(self, mxfp4_mode: str = "lds_dequant"):
    self.mxfp4_mode = mxfp4_mode

  def __call__(self, lhs, rhs, *, group_sizes, rhs_scale=None, fuse_gateup_activation=None,
               maybe_quantize_lhs=False, rhs_layout="gkn", zero_group=-1):
    if rhs_scale is not None and rhs_scale.dtype == torch.float32:
      if maybe_quantize_lhs:
        raise NotImplementedError("maybe_quantize_lhs with fp8 (E4M3 + f32 scale) weights")
      return ragged_dot_fp8_scaled(lhs, rhs, rhs_scale, group_sizes,
                                   fuse_gateup_activation=fuse_gateup_activation, zero_group=zero_group)
    if rhs_scale is not None:
      if rhs_scale.dtype != torch.uint8:
        raise ValueError(f"rhs_scale dtype {rhs_scale.dtype}: float32 (fp8 weights) or uint8 (MXFP4 E8M0)")
      if maybe_quantize_lhs:
        tiled = rhs.dim() == 4
        if not tiled:
          rhs, rhs_scale = mxfp4_tile_weights(rhs, rhs_scale)
        return ragged_dot_mxfp4(lhs, rhs, rhs_scale, group_sizes, fuse_gateup_activation=fuse_gateup_activation,
                                mode="scaled_mfma", zero_group=zero_group, weight_layout="tiled")
      return ragged_dot_mxfp4(lhs, rhs, rhs_scale, group_sizes,
                              fuse_gateup_activation=fuse_gateup_activation, mode=self.mxfp4_mode,
                              zero_group=zero_group, weight_layout="tiled" if rhs.dim() == 4 else "checkpoint")
    if maybe_quantize_lhs:
      raise NotImplementedError("maybe_quantize_lhs without quantised weights (rhs_scale)")
    if fuse_gateup_activation is not None:
      b, bl = parse_fused_activation(fuse_gateup_activation)
      return ragged_dot_gateup_situ(lhs, rhs, group_sizes, b, bl, rhs_layout=rhs_layout,
                                    zero_group=zero_group)
    return ragged_dot(lhs, rhs, group_sizes, rhs_layout=rhs_layout, zero_group=zero_group)


def prefuse_gateup_weights(expert_gate: torch.Tensor, expert_up: torch.Tensor) -> torch.Tensor:
  """rd.py:610-641: plain concatenation [gate | up] on the last (N) axis."""
  return torch.cat([expert_gate, expert_up], dim=-1).contiguous()


def prefuse_gateup_weights_gnk(expert_gate: torch.Tensor, expert_up: torch.Tensor) -> torch.Tensor:
  """The same prefused weight in the k-contiguous (G, 2I, K) layout the MFMA
  tiles read with plain 16-byte loads; done once at weight-load time."""
  return torch.cat([expert_gate, expert_up], dim=-1).transpose(1, 2).contiguous()


def to_gnk(w: torch.Tensor) -> torch.Tensor:
  """(G, K, N) -> (G, N, K) contiguous (weight preparation, outside timed regions)."""
  return w.transpose(1, 2).contiguous()


# ---------------------------------------------------------------------------
# a17 / a18: MXFP4
# ---------------------------------------------------------------------------


def dequantize_mxfp4(weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
  """``dequantize_mxfp4`` (mxfp4_dequant.py:29-67): packed (..., N, K/2) u8,
  scale (..., N, K/gs) u8 -> (..., N, K) float32 (bit-exact)."""
  _dev(weight_packed, weight_scale)
  if weight_packed.dtype != torch.uint8 or weight_scale.dtype != torch.uint8:
    raise ValueError("packed / scale must be uint8")
  *lead, n, kh = weight_packed.shape
  k = kh * 2
  ng = weight_scale.shape[-1]
  if tuple(weight_scale.shape[:-1]) != (*lead, n) or ng == 0 or k % ng:
    raise ValueError(f"scale shape {tuple(weight_scale.shape)} vs packed {tuple(weight_packed.shape)}")
  batch = math.prod(lead) if lead else 1
  out = torch.empty((*lead, n, k), dtype=out_dtype, device=weight_packed.device)
  check(lib().lmoe_mxfp4_dequant(_p(weight_packed), _p(weight_scale), batch, n, k, k // ng, _p(out),
                                 _dt(out), _stream()), "mxfp4_dequant")
  return out


_MX_MODES = {"lds_dequant": _lib.MXFP4_LDS_DEQUANT, "scaled_mfma": _lib.MXFP4_SCALED_MFMA, "skinny": -1, "scaled_mfma_fp6": -1}


def skinny_supported(k: int, n: int, g: int, situ: bool) -> bool:
  """Shapes the skinny (decode) MXFP4 kernel takes: K % 128 == 0, 16-column
  output tiles, at most 1024 groups."""
  return k % 128 == 0 and n % (32 if situ else 16) == 0 and g <= 1024


def mxfp4_tile_weights(w_packed: torch.Tensor, w_scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
  """One-time weight preparation (the MXFP4 counterpart of
  ``prefuse_gateup_weights``, rd.py:610-641): checkpoint-layout packed
  (G, N, K/2) and E8M0 scales (G, N, K/32) -> k-step-major (G, K/64, N, 32)
  and (G, K/64, N, 2), as ``ragged_dot_mxfp4(..., weight_layout="tiled")``
  streams them (one contiguous read per k step and column run).  Each 32-byte
  record keeps the checkpoint's eight 4-byte groups in the order
  0, 2, 4, 6, 1, 3, 5, 7."""
  _dev(w_packed, w_scale)
  if w_packed.dtype != torch.uint8 or w_scale.dtype != torch.uint8 or w_packed.dim() != 3:
    raise ValueError("packed / scale must be uint8 (G, N, K/2) / (G, N, K/32)")
  g, n, kh = w_packed.shape
  k = kh * 2
  if k % 64 or tuple(w_scale.shape) != (g, n, k // 32):
    raise ValueError(f"packed {tuple(w_packed.shape)} scale {tuple(w_scale.shape)}: need K % 64 == 0")
  w_packed, w_scale = w_packed.contiguous(), w_scale.contiguous()
  pk = torch.empty((g, k // 64, n, 32), dtype=torch.uint8, device=w_packed.device)
  sc = torch.empty((g, k // 64, n, 2), dtype=torch.uint8, device=w_packed.device)
  check(lib().lmoe_mxfp4_tile(_p(w_packed), _p(w_scale), g, n, k, _p(pk), _p(sc), _stream()), "mxfp4_tile")
  return pk, sc


def quantize_mxfp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
  """OCP MX E4M3 quantisation of activations (no reference counterpart; the
  native scaled-MFMA path): x (M, K) bf16/f32 -> codes (M, K) uint8 and E8M0
  scales (K/128, roundup(M, 4), 4) uint8 (the k-step-major layout the scaled
  GEMM streams).  One shared exponent floor(log2 max|x|) - 8 per 32 along K."""
  _dev(x)
  if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float32):
    raise ValueError(f"x must be (M, K) bf16/f32, got {tuple(x.shape)} {x.dtype}")
  m, k = x.shape
  if k % 128:
    raise NotImplementedError(f"MXFP8 quantisation needs K % 128 == 0 (K={k})")
  x = x.contiguous()
  m4 = (m + 3) // 4 * 4
  q = torch.empty((m, k), dtype=torch.uint8, device=x.device)
  sc = torch.empty((k // 128, m4, 4), dtype=torch.uint8, device=x.device)
  check(lib().lmoe_quantize_mxfp8(_p(x), _dt(x), m, k, _p(q), _p(sc), _stream()), "quantize_mxfp8")
  return q, sc


def ragged_dot_mxfp8_mxfp4(lhs_q: torch.Tensor, lhs_scale: torch.Tensor, w_packed: torch.Tensor,
                           w_scale: torch.Tensor, group_sizes: torch.Tensor, *,
                           fuse_gateup_activation: str | None = None, zero_group: int = -1,
                           out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
  """Grouped deq(A) @ deq(W_g)^T on the block-scaled MFMA: A from
  ``quantize_mxfp8``, W from ``mxfp4_tile_weights``.  With
  ``fuse_gateup_activation`` the N axis is [gate | up] and the SiTU-GLU epilogue
  is applied (bf16 output of width N/2)."""
  _dev(lhs_q, lhs_scale, w_packed, w_scale, group_sizes)
  m, k = lhs_q.shape
  if w_packed.dim() != 4 or w_packed.shape[3] != 32:
    raise ValueError(f"weights must be tiled (G, K/64, N, 32), got {tuple(w_packed.shape)}")
  g, _, n, _ = w_packed.shape
  m4 = (m + 3) // 4 * 4
  if (lhs_q.dtype != torch.uint8 or k % 128 or tuple(lhs_scale.shape) != (k // 128, m4, 4)
      or tuple(w_packed.shape) != (g, k // 64, n, 32) or tuple(w_scale.shape) != (g, k // 64, n, 2)):
    raise ValueError(f"shapes: lhs {tuple(lhs_q.shape)} scale {tuple(lhs_scale.shape)} "
                     f"w {tuple(w_packed.shape)} w_scale {tuple(w_scale.shape)}")
  _check_groups(group_sizes, g)
  epi, b, bl, width = _lib.EPI_NONE, 0.0, 0.0, n
  if fuse_gateup_activation is not None:
    b, bl = parse_fused_activation(fuse_gateup_activation)
    epi, width, out_dtype = _lib.EPI_SITU, n // 2, torch.bfloat16
  out = torch.empty((m, width), dtype=out_dtype, device=lhs_q.device)
  check(lib().lmoe_ragged_dot_mxfp8_mxfp4(_p(lhs_q), _p(lhs_scale), _p(w_packed), _p(w_scale), _p(group_sizes),
                                          m, k, n, g, zero_group, epi, b, bl, _p(out), _dt(out), _stream()),
        "ragged_dot_mxfp8_mxfp4")
  return out


def quantize_mxfp6(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
  """OCP MX FP6 E2M3 quantisation of activations (no reference counterpart;
  the scaled-MFMA path at the FP4/FP6 rate): x (M, K) bf16/f32 -> packed codes
  (M, K*3/4) uint8 (32 codes in 24 bytes, code j at bits 6j..6j+5) and E8M0
  scales (K/128, roundup(M, 4), 4) uint8.  One shared exponent
  floor(log2 max|x|) - 2 per 32 along K; elements round to nearest even and
  saturate to +-7.5."""
  _dev(x)
  if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float32):
    raise ValueError(f"x must be (M, K) bf16/f32, got {tuple(x.shape)} {x.dtype}")
  m, k = x.shape
  if k % 128:
    raise NotImplementedError(f"MXFP6 quantisation needs K % 128 == 0 (K={k})")
  x = x.contiguous()
  m4 = (m + 3) // 4 * 4
  q = torch.empty((m, k * 3 // 4), dtype=torch.uint8, device=x.device)
  sc = torch.empty((k // 128, m4, 4), dtype=torch.uint8, device=x.device)
  check(lib().lmoe_quantize_mxfp6(_p(x), _dt(x), m, k, _p(q), _p(sc), _stream()), "quantize_mxfp6")
  return q, sc


def ragged_dot_mxfp6_mxfp4(lhs_q: torch.Tensor, lhs_scale: torch.Tensor, w_packed: torch.Tensor,
                           w_scale: torch.Tensor, group_sizes: torch.Tensor, *, zero_group: int = -1,
                           out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
  """Grouped deq(A) @ deq(W_g)^T on the 32x32x64 block-scaled MFMA at the
  FP4/FP6 rate: A from ``quantize_mxfp6``, W from ``mxfp4_tile_weights``."""
  _dev(lhs_q, lhs_scale, w_packed, w_scale, group_sizes)
  m, kp = lhs_q.shape
  k = kp * 4 // 3
  if w_packed.dim() != 4 or w_packed.shape[3] != 32:
    raise ValueError(f"weights must be tiled (G, K/64, N, 32), got {tuple(w_packed.shape)}")
  g, _, n, _ = w_packed.shape
  m4 = (m + 3) // 4 * 4
  if (lhs_q.dtype != torch.uint8 or kp % 96 or tuple(lhs_scale.shape) != (k // 128, m4, 4)
      or tuple(w_packed.shape) != (g, k // 64, n, 32) or tuple(w_scale.shape) != (g, k // 64, n, 2)):
    raise ValueError(f"shapes: lhs {tuple(lhs_q.shape)} scale {tuple(lhs_scale.shape)} "
                     f"w {tuple(w_packed.shape)} w_scale {tuple(w_scale.shape)}")
  _check_groups(group_sizes, g)
  out = torch.empty((m, n), dtype=out_dtype, device=lhs_q.device)
  check(lib().lmoe_ragged_dot_mxfp6_mxfp4(_p(lhs_q), _p(lhs_scale), _p(w_packed), _p(w_scale), _p(group_sizes),
                                          m, k, n, g, zero_group, _p(out), _dt(out), _stream()),
        "ragged_dot_mxfp6_mxfp4")
  return out


def mxfp4_k_split(m: int, n: int, k: int, g: int) -> int:
  """K ranges for the split-K MXFP4 kernel (1: no split).  One group only
  (the tile count of a grouped problem depends on device-side group sizes).
  Up to M = 256 the kernel uses 64x128 tiles: split until the tiles times
  the ranges reach one per CU, keeping at least 8 K steps (512 of K) per
  range; above it 64x256 tiles: split until two per CU, at least 16 steps
  per range.  Measured at config 4 (K = 7168, N = 2048): M = 1 in 14 ranges
  12.9 us (7 ranges 14.2, unsplit 57), M = 128 in 8 ranges 20.4 us (7
  ranges 20.8, unsplit 73), M = 1024 in 4 ranges of 64x256 tiles 45.5 us
  (2 ranges of 64x128 tiles 48.7, unsplit 75)."""
  if g != 1 or k % 64 != 0:
    return 1
  steps = k // 64
  if m <= 256:
    tiles = -(-m // 64) * -(-n // 128)
    return max(1, min(-(-256 // max(tiles, 1)), steps // 8))
  tiles = -(-m // 64) * -(-n // 256)
  return max(1, min(-(-512 // max(tiles, 1)), steps // 16))


def ragged_dot_mxfp4(lhs: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                     group_sizes: torch.Tensor, *, fuse_gateup_activation: str | None = None,
                     mode: str = "lds_dequant", zero_group: int = -1,
                     weight_layout: str = "checkpoint", skip_zero_group_rows: bool = False,
                     max_group_rows: int = 0, k_split: int | None = None,
                     lhs_row_index: torch.Tensor | None = None) -> torch.Tensor:
  """Grouped lhs @ deq(W_g)^T with W_g in checkpoint (N, K/2) layout
  (orientation of mxfp4_online_dequant_matmul_pallas.py:1-36) and block-32
  E8M0 scales (G, N, K/32), or with ``weight_layout="tiled"`` the
  (G, K/64, N, 32) / (G, K/64, N, 2) pair from ``mxfp4_tile_weights`` (same
  result, faster kernel).  With ``fuse_gateup_activation`` the N axis is
  [gate | up] and the SiTU-GLU epilogue is applied (output width N/2).
  ``skip_zero_group_rows``: the rows of ``zero_group`` and those past
  sum(group_sizes) may be left unwritten (uninitialised) instead of zeroed,
  for callers that never read them.

  ``k_split`` (tiled weights, ``mode="lds_dequant"``): K ranges computed
  in parallel as f32 partial planes and summed in order by a second kernel;
  None picks ``mxfp4_k_split`` (a split only for one group with few tiles,
  e.g. the config-4 matmul at M <= 1024), 1 never splits.  A split result
  equals the unsplit one within bf16 rounding (another f32 summation order).

  ``mode="skinny"`` (tiled weights, K % 128 == 0): the decode-regime kernel
  for groups of a few rows -- each weight byte of a group with rows read once
  per pass of up to 16, 32, 64 or 128 rows, sized from min(M,
  ``max_group_rows``) (0: unknown).  Equal to the other modes within bf16
  rounding (another f32 summation order), not bit for bit.

  ``lhs_row_index`` (int32 (M,), tiled weights, ``mode="lds_dequant"``):
  the grouped lhs is gathered from ``lhs`` (rows, K) -- row r is
  ``lhs[lhs_row_index[r]]`` -- inside the kernel, i.e.
  ``ragged_dot(lhs[lhs_row_index], W, group_sizes)`` without the gathered copy
  (the dispatch's padded_token_idx over the token rows).  Raises
  NotImplementedError where the streamed kernel does not apply."""
  if lhs_row_index is not None:
    return _ragged_dot_mxfp4_rows(lhs, lhs_row_index, w_packed, w_scale, group_sizes,
                                  fuse_gateup_activation=fuse_gateup_activation, mode=mode,
                                  zero_group=zero_group, weight_layout=weight_layout,
                                  skip_zero_group_rows=skip_zero_group_rows)
  _dev(lhs, w_packed, w_scale, group_sizes)
  if lhs.dtype != torch.bfloat16:
    raise NotImplementedError("MXFP4 GEMM takes bf16 activations")
  if w_packed.dtype != torch.uint8 or w_scale.dtype != torch.uint8:
    raise ValueError(f"MXFP4 weights must be uint8 packed codes and E8M0 scale bytes, got "
                     f"{w_packed.dtype} / {w_scale.dtype}")
  if group_sizes.dtype != torch.int32:
    raise ValueError("group_sizes must be int32")
  m, k = lhs.shape
  if k % 64:  # the weight shapes below are formed with K / 64 and K / 32
    raise NotImplementedError(f"MXFP4 GEMM needs K % 64 == 0 (K={k})")
  if weight_layout == "tiled":
    if w_packed.dim() != 4 or w_packed.shape[3] != 32:
      raise ValueError(f"tiled packed weights must be (G, K/64, N, 32), got {tuple(w_packed.shape)}")
    g, _, n, _ = w_packed.shape
    want = ((g, k // 64, n, 32), (g, k // 64, n, 2))
  elif weight_layout == "checkpoint":
    g, n, _ = w_packed.shape
    want = ((g, n, k // 2), (g, n, k // 32))
  else:
    raise ValueError(f"weight_layout {weight_layout!r}")
  if (tuple(w_packed.shape), tuple(w_scale.shape)) != want:
    raise ValueError(f"mxfp4 shapes lhs {tuple(lhs.shape)} packed {tuple(w_packed.shape)} "
                     f"scale {tuple(w_scale.shape)} ({weight_layout} layout wants {want})")
  _check_groups(group_sizes, g)
  epi, b, bl = _lib.EPI_NONE, 0.0, 0.0
  width = n
  if fuse_gateup_activation is not None:
    b, bl = parse_fused_activation(fuse_gateup_activation)
    epi, width = _lib.EPI_SITU, n // 2
  if mode not in _MX_MODES:
    raise ValueError(f"mode {mode!r}")
  mode_id = _MX_MODES[mode]
  if mode == "scaled_mfma_fp6":
    if weight_layout != "tiled":
      raise NotImplementedError("the MXFP6 scaled-MFMA path streams weights from mxfp4_tile_weights (weight_layout='tiled')")
    if fuse_gateup_activation is not None:
      raise NotImplementedError("the MXFP6 scaled-MFMA path has no fused SiTU epilogue")
    q, qs = quantize_mxfp6(lhs)
    return ragged_dot_mxfp6_mxfp4(q, qs, w_packed, w_scale, group_sizes, zero_group=zero_group)
  if mode == "scaled_mfma":
    if weight_layout != "tiled":
      raise NotImplementedError("the scaled-MFMA path streams weights from mxfp4_tile_weights (weight_layout='tiled')")
    q, qs = quantize_mxfp8(lhs)
    return ragged_dot_mxfp8_mxfp4(q, qs, w_packed, w_scale, group_sizes,
                                  fuse_gateup_activation=fuse_gateup_activation, zero_group=zero_group)
  if mode == "skinny":
    if weight_layout != "tiled":
      raise NotImplementedError("the skinny kernel reads mxfp4_tile_weights output (weight_layout='tiled')")
    flags = _lib.MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS if skip_zero_group_rows else 0
    out = torch.empty((m, width), dtype=torch.bfloat16, device=lhs.device)
    check(lib().lmoe_ragged_dot_mxfp4_skinny(_p(lhs), _p(w_packed), _p(w_scale), _p(group_sizes), m, k, n, g,
                                             zero_group, flags, epi, b, bl, max_group_rows, _p(out), _stream()),
          "ragged_dot_mxfp4_skinny")
    return out
  if weight_layout == "tiled":
    mode_id = _lib.MXFP4_LDS_DEQUANT_TILED
    splits = mxfp4_k_split(m, n, k, g) if k_split is None else int(k_split)
    if splits > 1:
      steps = k // 64
      splits = -(-steps // -(-steps // splits)) if 1 <= splits <= steps else splits  # no empty range
      ws = torch.empty((splits * m * n,), dtype=torch.float32, device=lhs.device)
      out = torch.empty((m, width), dtype=torch.bfloat16, device=lhs.device)
      check(lib().lmoe_ragged_dot_mxfp4_splitk(_p(lhs), _p(w_packed), _p(w_scale), _p(group_sizes), m, k, n, g,
                                               zero_group, splits, _p(ws), ws.numel() * 4, epi, b, bl, _p(out),
                                               _stream()),
            "ragged_dot_mxfp4_splitk")
      return out
  if skip_zero_group_rows:
    mode_id |= _lib.MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS
  out = torch.empty((m, width), dtype=torch.bfloat16, device=lhs.device)
  check(lib().lmoe_ragged_dot_mxfp4(_p(lhs), _p(w_packed), _p(w_scale), _p(group_sizes), m, k, n, g,
                                    zero_group, mode_id, epi, b, bl, _p(out), _stream()),
        "ragged_dot_mxfp4")
  return out


def _ragged_dot_mxfp4_rows(lhs, row_index, w_packed, w_scale, group_sizes, *, fuse_gateup_activation, mode,
                           zero_group, weight_layout, skip_zero_group_rows):
  _dev(lhs, row_index, w_packed, w_scale, group_sizes)
  if lhs.dtype != torch.bfloat16 or lhs.dim() != 2 or not lhs.is_contiguous():
    raise NotImplementedError("gathered rows: lhs must be a contiguous bf16 (rows, K) array")
  if row_index.dtype != torch.int32 or row_index.dim() != 1:
    raise ValueError("lhs_row_index must be int32 (M,)")
  if w_packed.dtype != torch.uint8 or w_scale.dtype != torch.uint8:
    raise ValueError(f"MXFP4 weights must be uint8 packed codes and E8M0 scale bytes, got "
                     f"{w_packed.dtype} / {w_scale.dtype}")
  if group_sizes.dtype != torch.int32:
    raise ValueError("group_sizes must be int32")
  if weight_layout != "tiled" or mode != "lds_dequant":
    raise NotImplementedError("gathered rows: tiled weights on the lds_dequant streamed kernel only")
  rows, k = lhs.shape
  if k % 64:
    raise NotImplementedError(f"MXFP4 GEMM needs K % 64 == 0 (K={k})")
  m = row_index.shape[0]
  if w_packed.dim() != 4 or w_packed.shape[3] != 32:
    raise ValueError(f"tiled packed weights must be (G, K/64, N, 32), got {tuple(w_packed.shape)}")
  g, _, n, _ = w_packed.shape
  if (tuple(w_packed.shape), tuple(w_scale.shape)) != ((g, k // 64, n, 32), (g, k // 64, n, 2)):
    raise ValueError(f"mxfp4 shapes lhs {tuple(lhs.shape)} packed {tuple(w_packed.shape)} scale {tuple(w_scale.shape)}")
  _check_groups(group_sizes, g)
  epi, b, bl, width = _lib.EPI_NONE, 0.0, 0.0, n
  if fuse_gateup_activation is not None:
    b, bl = parse_fused_activation(fuse_gateup_activation)
    epi, width = _lib.EPI_SITU, n // 2
  mode_id = _lib.MXFP4_LDS_DEQUANT_TILED | (_lib.MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS if skip_zero_group_rows else 0)
  out = torch.empty((m, width), dtype=torch.bfloat16, device=lhs.device)
  check(lib().lmoe_ragged_dot_mxfp4_rows(_p(lhs), rows, _p(row_index), _p(w_packed), _p(w_scale), _p(group_sizes),
                                         m, k, n, g, zero_group, mode_id, epi, b, bl, _p(out), _stream()),
        "ragged_dot_mxfp4_rows")
  return out


# ---------------------------------------------------------------------------
# a3 / a4: router
# ---------------------------------------------------------------------------

_ACTS = {"sigmoid": _lib.ACT_SIGMOID, "softmax": _lib.ACT_SOFTMAX}


def router_topk_from_logits(logits: torch.Tensor, bias: torch.Tensor | None, top_k: int,
                            renormalize: bool = True, scaling: float = 1.0, act: str = "sigmoid",
                            weight_dtype: torch.dtype = torch.float32, return_scores: bool = False):
  """Gate math of ref.py:347-361 / ref.py:601-631 on given f32 logits (T, E):
  returns (topk_idx int32 (T, k), topk_weight (T, k) weight_dtype[, scores]).
  ``logits`` may be a row-strided view (unit column stride), e.g. the router
  columns of a wider GEMM output."""
  logits = _dev_rows(logits)
  _dev(bias)
  if logits.dtype != torch.float32:
    raise ValueError("router logits must be float32 (the reference's gate runs in f32)")
  if bias is not None and bias.dtype != torch.float32:
    bias = bias.float().contiguous()
  t, e = logits.shape
  if bias is not None and bias.numel() != e:
    raise ValueError(f"bias has {bias.numel()} entries for {e} experts")
  idx = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
  w = torch.empty((t, top_k), dtype=weight_dtype, device=logits.device)
  scores = torch.empty((t, e), dtype=torch.float32, device=logits.device) if return_scores else None
  check(lib().lmoe_router_topk_ld(_p(logits), max(logits.stride(0), e), _p(bias), t, e, top_k, _ACTS[act],
                                  int(renormalize), scaling, _dt(w), _p(idx), _p(w), _p(scores), _stream()),
        "router_topk")
  return (idx, w, scores) if return_scores else (idx, w)


ROUTER_PROJECT_MAX_LAT = 1024


def router_topk_project_supported(e: int, lat: int) -> bool:
  """Sizes ``router_topk_project`` takes when the router logits and the
  latent projection are the column blocks [0, E) and [E, E + lat) of one
  (T, E + lat) f32 GEMM output (the layer's fused router + down-projection):
  at most 1024 latent columns, lat % 4 == 0, and E % 4 == 0, so that the
  projection block starts 16-byte aligned and the row stride E + lat is a
  multiple of 4.  These are the size checks of lmoe_router_topk_proj."""
  return 0 < lat <= ROUTER_PROJECT_MAX_LAT and lat % 4 == 0 and e % 4 == 0


def router_topk_project(logits: torch.Tensor, x: torch.Tensor, bias: torch.Tensor | None, top_k: int,
                        renormalize: bool = True, scaling: float = 1.0, act: str = "sigmoid",
                        weight_dtype: torch.dtype = torch.float32):
  """router_and_projection's outputs (ref.py:634-655) from one GEMM that
  computed the router logits and the latent projection together: the gate of
  ``router_topk_from_logits`` on ``logits`` (T, E) f32 plus ``x`` (T, lat)
  f32 rounded to bf16 (nearest even), in one launch.  Both may be row-strided
  views (unit column stride).  Returns (topk_idx, topk_weight, x_bf16)."""
  logits, x = _dev_rows(logits), _dev_rows(x)
  _dev(bias)
  if logits.dtype != torch.float32 or x.dtype != torch.float32:
    raise ValueError("router logits and the projection must be float32 GEMM outputs")
  if bias is not None and bias.dtype != torch.float32:
    bias = bias.float().contiguous()
  t, e = logits.shape
  if bias is not None and bias.numel() != e:
    raise ValueError(f"bias has {bias.numel()} entries for {e} experts")
  lat = x.shape[1]
  if x.shape[0] != t:
    raise ValueError(f"logits {tuple(logits.shape)} and x {tuple(x.shape)} differ in rows")
  idx = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
  w = torch.empty((t, top_k), dtype=weight_dtype, device=logits.device)
  xb = torch.empty((t, lat), dtype=torch.bfloat16, device=logits.device)
  check(lib().lmoe_router_topk_proj(_p(logits), max(logits.stride(0), e), _p(bias), t, e, top_k, _ACTS[act],
                                    int(renormalize), scaling, _dt(w), _p(idx), _p(w), _p(x),
                                    max(x.stride(0), lat), lat, _p(xb), _stream()),
        "router_topk_proj")
  return idx, w, xb


def cast_rows(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
  """Contiguous ``x.to(dtype)`` of a 2-D, row-strided view (unit column
  stride); f32 -> bf16 rounds to nearest even."""
  x = _dev_rows(x)
  rows, cols = x.shape
  out = torch.empty((rows, cols), dtype=dtype, device=x.device)
  check(lib().lmoe_cast_rows(_p(x), _dt(x), rows, cols, max(x.stride(0), cols), _p(out), _dt(out), _stream()),
        "cast_rows")
  return out


_GROUP_CACHE: dict = {}


def _ones_group(m: int, device) -> torch.Tensor:
  """Cached one-group group_sizes tensor [m] (no per-call host->device copy)."""
  key = (m, str(device))
  t = _GROUP_CACHE.get(key)
  if t is None:
    if len(_GROUP_CACHE) > 256:
      _GROUP_CACHE.clear()
    t = torch.full((1,), m, dtype=torch.int32, device=device)
    _GROUP_CACHE[key] = t
  return t


_DENSE_BACKENDS = ("auto", "hip", "dense", "blaslt", "skinny")


# The skinny dense kernel's parallelism is one block per 16 output columns:
# measured against hipBLASLt at M = 1..16 it wins from N = 4096 on (the
# decode up-projection, 7168 columns: 5.4 vs 6.4 us) and loses below (the
# 1920-column router + down projection: 11.4 vs 10.4 us, half the CUs idle).
SKINNY_DENSE_ROWS = 16
SKINNY_DENSE_MIN_N = 4096


def dense(x: torch.Tensor, w: torch.Tensor, out_dtype: torch.dtype | None = None,
          w_layout: str = "kn", backend: str | None = None) -> torch.Tensor:
  """x @ w (w (K, N), or (N, K) with w_layout="nk").

  ``backend``: "hip" runs it as a one-group grouped GEMM on the hand-written
  kernels; "blaslt" calls hipBLASLt (the ROCm library GEMM; (N, K) weights
  only); "skinny" the hand-written few-row kernel (bf16 (N, K) weights,
  K % 128 == 0, N % 16 == 0).  "auto" (the default), for bf16
  (N, K) weights -- the layer's router logits (f32 out), down- and
  up-projections: the skinny kernel for at most SKINNY_DENSE_ROWS rows and
  N >= SKINNY_DENSE_MIN_N, else hipBLASLt; for other weights the hand-written
  grouped kernels.  All accumulate the exact bf16 products in f32; only the
  summation order differs."""
  backend = backend or "auto"
  if backend not in _DENSE_BACKENDS:
    raise ValueError(f"backend {backend!r}")
  out_dtype = out_dtype or x.dtype
  if x.dim() == 2 and w.dim() == 2 and x.shape[1] == w.shape[1 if w_layout == "nk" else 0]:
    n = w.shape[0 if w_layout == "nk" else 1]
    if x.shape[0] == 0 or x.shape[1] == 0 or n == 0:  # nothing to read: an empty sum is zero
      return torch.zeros((x.shape[0], n), dtype=out_dtype, device=x.device)
  nk_bf16 = w_layout == "nk" and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
  if backend == "auto" and nk_bf16 and x.dim() == 2 and x.shape[0] <= SKINNY_DENSE_ROWS \
     and x.shape[1] % 128 == 0 and w.shape[0] % 16 == 0 and w.shape[0] >= SKINNY_DENSE_MIN_N:
    backend = "skinny"
  if backend == "skinny":
    if not nk_bf16:
      raise NotImplementedError("the skinny dense kernel takes bf16 x and bf16 (N, K) weights")
    _dev(x, w)
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
      raise ValueError(f"dense: x {tuple(x.shape)} / w {tuple(w.shape)}")
    x, w = x.contiguous(), w.contiguous()
    m, k = x.shape
    n = w.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    check(lib().lmoe_dense_skinny(_p(x), _p(w), m, k, n, _p(out), _dt(out), _stream()), "dense_skinny")
    return out
  if backend == "dense":
    if not nk_bf16:
      raise NotImplementedError("the dense kernel takes bf16 x and bf16 (N, K) weights")
    _dev(x, w)
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
      raise ValueError(f"dense: x {tuple(x.shape)} / w {tuple(w.shape)}")
    x, w = x.contiguous(), w.contiguous()
    m, k = x.shape
    n = w.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    check(lib().lmoe_dense(_p(x), _p(w), m, k, n, _p(out), _dt(out), _stream()), "dense")
    return out
  use_blaslt = backend == "blaslt" or (backend == "auto" and nk_bf16)
  if use_blaslt:
    if w_layout != "nk":
      raise NotImplementedError("the hipBLASLt backend takes (N, K) weights")
    _dev(x, w)
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
      raise ValueError(f"dense: x {tuple(x.shape)} / w {tuple(w.shape)}")
    if w.dtype != x.dtype:
      raise NotImplementedError(f"mixed x {x.dtype} / w {w.dtype}")
    x, w = x.contiguous(), w.contiguous()
    m, k = x.shape
    n = w.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    check(lib().lmoe_dense_blaslt(_p(x), _dt(x), _p(w), _dt(w), m, k, n, _p(out), _dt(out), _stream()),
          "dense_blaslt")
    return out
  rhs = w.unsqueeze(0)
  return ragged_dot(x, rhs, _ones_group(x.shape[0], x.device), preferred_element_type=out_dtype,
                    rhs_layout="gkn" if w_layout == "kn" else "gnk")


def router_logits(hidden: torch.Tensor, router_weight: torch.Tensor) -> torch.Tensor:
  """``f32(hidden) @ f32(router_weight)`` (ref.py:620).  For bf16 operands the
  products are exact in f32, so the bf16 MFMA with f32 accumulation computes
  the same f32 matmul (up to summation order)."""
  if hidden.dtype == router_weight.dtype:
    return dense(hidden, router_weight, out_dtype=torch.float32)
  return dense(hidden.float(), router_weight.float(), out_dtype=torch.float32)


def _router_gate(hidden_states: torch.Tensor, router_weight: torch.Tensor,
                 e_score_correction_bias: torch.Tensor, config, act: str = "sigmoid"):
  """ref.py:601-631: f32 gate math, combine weight cast to the compute dtype."""
  logits = router_logits(hidden_states, router_weight)
  return router_topk_from_logits(logits, e_score_correction_bias, config.top_k,
                                 config.moe_renormalize, config.routed_scaling_factor, act,
                                 hidden_states.dtype)


def router_and_projection(hidden_states, router_weight, e_score_correction_bias, down_proj, config):
  """ref.py:634-655: _router_gate plus x = hidden @ down_proj."""
  topk_idx, topk_weight = _router_gate(hidden_states, router_weight, e_score_correction_bias, config)
  return topk_idx, topk_weight, dense(hidden_states, down_proj)


# ---------------------------------------------------------------------------
# a6 / a7: local-shard dispatch
# ---------------------------------------------------------------------------


def round_up_to_tile(value: int, tile_size: int = MOSAIC_TILE_SIZE) -> int:
  """ref.py:152-153."""
  return -(-value // tile_size) * tile_size


_round_up_to_tile = round_up_to_tile  # the reference's name (ref.py:152)


def compute_m_padded(num_tokens: int, top_k: int, num_experts: int, local_num_experts: int,
                     capacity_factor: float = 2.0, tile_size: int = MOSAIC_TILE_SIZE) -> int:
  """ref.py:825-826: round_up(ceil(T*k*L/E * cf), tile), static per config."""
  expected_total = num_tokens * top_k * local_num_experts / num_experts
  return round_up_to_tile(math.ceil(expected_total * capacity_factor), tile_size)


class Dispatch(NamedTuple):
  sorted_tokens: torch.Tensor
  group_sizes: torch.Tensor
  valid_mask: torch.Tensor
  per_expert_counts: torch.Tensor
  padded_token_idx: torch.Tensor
  padded_combine_weight: torch.Tensor
  slot_pos: torch.Tensor


SMALL_DISPATCH_SLOTS = 8192


def small_dispatch_supported(t: int, k: int, lat: int, L: int, m_padded: int) -> bool:
  """Sizes the one-launch dispatch takes (decode-sized batches)."""
  return t * k <= SMALL_DISPATCH_SLOTS and m_padded <= 8192 and L + 1 <= 1024 and lat % 8 == 0


def _no_slot_dispatch(t, k, L, lat, rows_dtype, w_dtype, dev, gather_rows=True) -> Dispatch:
  """m_padded == 0 (an empty batch, or a capacity factor of 0): no slot is
  kept, so every output is known without a launch -- zero group sizes and
  counts, every slot_pos -1, the per-row outputs empty (ref.py:816-868 at
  m_padded 0)."""
  empty = lambda dtype, *shape: torch.empty(shape or (0,), dtype=dtype, device=dev)
  return Dispatch(empty(rows_dtype, 0, lat) if gather_rows else None,
                  torch.zeros((L + 1,), dtype=torch.int32, device=dev), empty(torch.bool),
                  torch.zeros((L,), dtype=torch.int32, device=dev), empty(torch.int32), empty(w_dtype),
                  torch.full((t * k,), -1, dtype=torch.int32, device=dev))


def _dispatch_metadata(topk_idx, topk_weight, local_expert_start, L, m_padded, lat):
  _dev(topk_idx, topk_weight)
  if lat is None:
    raise ValueError("dispatch without rows: give x or lat")
  t, k = topk_idx.shape
  dev = topk_idx.device
  if m_padded == 0:
    return _no_slot_dispatch(t, k, L, lat, torch.bfloat16, topk_weight.dtype, dev, gather_rows=False)
  group_sizes = torch.empty((L + 1,), dtype=torch.int32, device=dev)
  valid = torch.empty((m_padded,), dtype=torch.bool, device=dev)
  counts = torch.empty((L,), dtype=torch.int32, device=dev)
  tok = torch.empty((m_padded,), dtype=torch.int32, device=dev)
  w = torch.empty((m_padded,), dtype=topk_weight.dtype, device=dev)
  slot_pos = torch.empty((t * k,), dtype=torch.int32, device=dev)
  ws = _workspace(lib().lmoe_dispatch_workspace_size(t, k, L), dev)
  check(lib().lmoe_dispatch_local_rows(_p(topk_idx), _p(topk_weight), _dt(topk_weight), None, _lib.BF16, lat, t, k,
                                       lat, local_expert_start, L, m_padded, None, _p(group_sizes), _p(valid),
                                       _p(counts), _p(tok), _p(w), _p(slot_pos), _lib.DISPATCH_FLAG_NO_ROWS, _p(ws),
                                       ws.numel(), _stream()), "dispatch_local_rows")
  return Dispatch(None, group_sizes, valid, counts, tok, w, slot_pos)


FUSED_DISPATCH_SLOTS, FUSED_DISPATCH_ROWS = 1024, 2048


def dispatch_skinny_supported(t: int, k: int, lat: int, n: int, L: int, m_padded: int, situ: bool) -> bool:
  """Sizes ``dispatch_ragged_dot_mxfp4_skinny`` takes (a decode step)."""
  return (t * k <= FUSED_DISPATCH_SLOTS and m_padded <= FUSED_DISPATCH_ROWS and L + 1 <= 1024
          and skinny_supported(lat, n, L + 1, situ))


def dispatch_ragged_dot_mxfp4_skinny(topk_idx: torch.Tensor, topk_weight: torch.Tensor, x: torch.Tensor,
                                     local_expert_start: int, local_num_experts: int, m_padded: int,
                                     w_tiled: torch.Tensor, s_tiled: torch.Tensor, *,
                                     fuse_gateup_activation: str | None = None,
                                     skip_zero_group_rows: bool = False) -> tuple[Dispatch, torch.Tensor]:
  """``dispatch_local(..., path="small")`` and ``ragged_dot_mxfp4(sorted_tokens,
  ..., mode="skinny", weight_layout="tiled", zero_group=L)`` in one launch (a
  decode step, ref.py:754-877 then rd.py:610-723): the same dispatch outputs
  except ``sorted_tokens`` (None: each block reads its rows' token rows of x
  itself) and the same expert GEMM output, bit for bit.  x: bf16 token rows
  (T, >= lat), unit column stride.  Sizes: ``dispatch_skinny_supported``."""
  _check_topk(topk_idx, topk_weight)
  _check_rows(x, topk_idx.shape[0])
  if x.dtype != torch.bfloat16:
    raise NotImplementedError("the fused decode dispatch reads bf16 token rows")
  if w_tiled.dtype != torch.uint8 or s_tiled.dtype != torch.uint8:
    raise ValueError("tiled MXFP4 weights and scales must be uint8")
  t, k = topk_idx.shape
  L = local_num_experts
  g, _, n, _ = w_tiled.shape
  lat = x.shape[-1]
  if g != L + 1 or tuple(w_tiled.shape) != (L + 1, lat // 64, n, 32) or tuple(s_tiled.shape) != (L + 1, lat // 64, n, 2):
    raise ValueError(f"tiled weights {tuple(w_tiled.shape)} / {tuple(s_tiled.shape)} for L + 1 = {L + 1} experts, K = {lat}")
  epi, b, bl, width = _lib.EPI_NONE, 0.0, 0.0, n
  if fuse_gateup_activation is not None:
    b, bl = parse_fused_activation(fuse_gateup_activation)
    epi, width = _lib.EPI_SITU, n // 2
  if not dispatch_skinny_supported(t, k, lat, n, L, m_padded, epi == _lib.EPI_SITU):
    raise NotImplementedError(f"fused decode dispatch: T*k={t * k}, m_padded={m_padded}, L={L}, K={lat}, N={n}")
  x = _dev_rows(x)
  _dev(topk_idx, topk_weight, w_tiled, s_tiled)
  dev = x.device
  if m_padded == 0:
    d = _no_slot_dispatch(t, k, L, lat, torch.bfloat16, topk_weight.dtype, dev, gather_rows=False)
    return d, torch.empty((0, width), dtype=torch.bfloat16, device=dev)
  group_sizes = torch.empty((L + 1,), dtype=torch.int32, device=dev)
  valid = torch.empty((m_padded,), dtype=torch.bool, device=dev)
  counts = torch.empty((L,), dtype=torch.int32, device=dev)
  tok = torch.empty((m_padded,), dtype=torch.int32, device=dev)
  w = torch.empty((m_padded,), dtype=topk_weight.dtype, device=dev)
  slot_pos = torch.empty((t * k,), dtype=torch.int32, device=dev)
  out = torch.empty((m_padded, width), dtype=torch.bfloat16, device=dev)
  flags = _lib.MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS if skip_zero_group_rows else 0
  check(lib().lmoe_dispatch_mxfp4_skinny(_p(topk_idx), _p(topk_weight), _dt(topk_weight), _p(x),
                                         x.stride(0) if t > 0 else lat, t, k, local_expert_start, L, m_padded,
                                         _p(w_tiled), _p(s_tiled), lat, n, epi, b, bl, flags, _p(group_sizes),
                                         _p(valid), _p(counts), _p(tok), _p(w), _p(slot_pos), _p(out), _stream()),
        "dispatch_mxfp4_skinny")
  return Dispatch(None, group_sizes, valid, counts, tok, w, slot_pos), out


def dispatch_local(topk_idx: torch.Tensor, topk_weight: torch.Tensor, x: torch.Tensor | None,
                   local_expert_start: int, local_num_experts: int, m_padded: int, *, path: str = "auto",
                   skip_padding_rows: bool = False, gather_rows: bool = True, lat: int | None = None) -> Dispatch:
  """The GPU dispatch with an explicit m_padded; also returns slot_pos (T*k,).

  ``path``: "sort" (the multi-block counting sort + gather), "small" (one
  launch for decode-sized batches, ``small_dispatch_supported``) or "auto"
  (small when supported and x is bf16).  Both give the same outputs bit for
  bit.  A contiguous x keeps its dtype in sorted_tokens; a row-strided view
  (unit column stride) of bf16 or f32 values, or ``skip_padding_rows``, gives
  bf16 sorted tokens (f32 rounded to nearest even), and ``skip_padding_rows``
  leaves their padding rows unwritten.

  ``gather_rows=False``: every output but the rows (``sorted_tokens`` is
  None; ``x`` may be None, then ``lat`` gives the row width), for an expert
  GEMM that gathers the token rows itself (``ragged_dot_mxfp4(...,
  lhs_row_index=padded_token_idx)``); the counting-sort path at every size."""
  _check_topk(topk_idx, topk_weight)
  t, k = topk_idx.shape
  if x is not None:
    _check_rows(x, t)
  if not gather_rows:
    return _dispatch_metadata(topk_idx, topk_weight, local_expert_start, local_num_experts, m_padded,
                              x.shape[-1] if x is not None else lat)
  if x is None:
    raise ValueError("dispatch with rows: x is required")
  lat = x.shape[-1]
  L = local_num_experts
  if m_padded == 0:
    _dev(topk_idx, topk_weight)
    _dev_rows(x)
    # the dtype the gather would write: bf16 for a row-strided view (judged
    # by its strides alone, the view having no rows) or skipped padding rows
    strided = x.stride(-1) != 1 or x.stride(0) != x.shape[-1]
    rows_dtype = torch.bfloat16 if skip_padding_rows or strided else x.dtype
    return _no_slot_dispatch(t, k, L, lat, rows_dtype, topk_weight.dtype, x.device)
  small_ok = small_dispatch_supported(t, k, lat, L, m_padded)
  if path == "auto":
    path = "small" if small_ok and x.dtype == torch.bfloat16 and not _row_strided(x) else "sort"
  if path == "small":
    if not small_ok:
      raise NotImplementedError(f"one-launch dispatch: T*k={t * k}, m_padded={m_padded}, L={L}, lat={lat}")
    x = _dev_rows(x)
    _dev(topk_idx, topk_weight)
    dev = x.device
    sorted_tokens = torch.empty((m_padded, lat), dtype=torch.bfloat16, device=dev)
    group_sizes = torch.empty((L + 1,), dtype=torch.int32, device=dev)
    valid = torch.empty((m_padded,), dtype=torch.bool, device=dev)
    counts = torch.empty((L,), dtype=torch.int32, device=dev)
    tok = torch.empty((m_padded,), dtype=torch.int32, device=dev)
    w = torch.empty((m_padded,), dtype=topk_weight.dtype, device=dev)
    slot_pos = torch.empty((t * k,), dtype=torch.int32, device=dev)
    flags = _lib.DISPATCH_FLAG_SKIP_PADDING_ROWS if skip_padding_rows else 0
    check(lib().lmoe_dispatch_local_small(_p(topk_idx), _p(topk_weight), _dt(topk_weight), _p(x), _dt(x),
                                          x.stride(0) if t > 0 else lat, t, k, lat, local_expert_start, L,
                                          m_padded, _p(sorted_tokens), _p(group_sizes), _p(valid), _p(counts),
                                          _p(tok), _p(w), _p(slot_pos), flags, _stream()), "dispatch_local_small")
    return Dispatch(sorted_tokens, group_sizes, valid, counts, tok, w, slot_pos)
  if path != "sort":
    raise ValueError(f"path {path!r}")
  if skip_padding_rows or _row_strided(x):
    # row-strided bf16 / f32 rows, written as bf16: the counting sort with a
    # converting gather (the one-launch kernel when the sizes fit it)
    x = _dev_rows(x)
    _dev(topk_idx, topk_weight)
    dev = x.device
    sorted_tokens = torch.empty((m_padded, lat), dtype=torch.bfloat16, device=dev)
    group_sizes = torch.empty((L + 1,), dtype=torch.int32, device=dev)
    valid = torch.empty((m_padded,), dtype=torch.bool, device=dev)
    counts = torch.empty((L,), dtype=torch.int32, device=dev)
    tok = torch.empty((m_padded,), dtype=torch.int32, device=dev)
    w = torch.empty((m_padded,), dtype=topk_weight.dtype, device=dev)
    slot_pos = torch.empty((t * k,), dtype=torch.int32, device=dev)
    ws = _workspace(lib().lmoe_dispatch_workspace_size(t, k, L), dev)
    flags = _lib.DISPATCH_FLAG_SKIP_PADDING_ROWS if skip_padding_rows else 0
    check(lib().lmoe_dispatch_local_rows(_p(topk_idx), _p(topk_weight), _dt(topk_weight), _p(x), _dt(x),
                                         x.stride(0) if t > 0 else lat, t, k, lat, local_expert_start, L, m_padded,
                                         _p(sorted_tokens), _p(group_sizes), _p(valid), _p(counts), _p(tok), _p(w),
                                         _p(slot_pos), flags, _p(ws), ws.numel(), _stream()), "dispatch_local_rows")
    return Dispatch(sorted_tokens, group_sizes, valid, counts, tok, w, slot_pos)
  _dev(topk_idx, topk_weight, x)
  dev = x.device
  sorted_tokens = torch.empty((m_padded, lat), dtype=x.dtype, device=dev)
  group_sizes = torch.empty((L + 1,), dtype=torch.int32, device=dev)
  valid = torch.empty((m_padded,), dtype=torch.bool, device=dev)
  counts = torch.empty((L,), dtype=torch.int32, device=dev)
  tok = torch.empty((m_padded,), dtype=torch.int32, device=dev)
  w = torch.empty((m_padded,), dtype=topk_weight.dtype, device=dev)
  slot_pos = torch.empty((t * k,), dtype=torch.int32, device=dev)
  ws_bytes = lib().lmoe_dispatch_workspace_size(t, k, L)
  ws = _workspace(ws_bytes, dev)
  check(lib().lmoe_dispatch_local(_p(topk_idx), _p(topk_weight), _dt(topk_weight), _p(x), _dt(x), t, k,
                                  lat, local_expert_start, L, m_padded, _p(sorted_tokens),
                                  _p(group_sizes), _p(valid), _p(counts), _p(tok), _p(w), _p(slot_pos),
                                  _p(ws), ws.numel(), _stream()), "dispatch_local")
  return Dispatch(sorted_tokens, group_sizes, valid, counts, tok, w, slot_pos)


def filter_and_pad_to_shard_jittable(topk_idx, topk_weight, x, config, local_expert_start: int,
                                     local_num_experts: int, capacity_factor: float = 2.0,
                                     tile_size: int = MOSAIC_TILE_SIZE):
  """ref.py:754-877: returns (sorted_tokens, group_sizes, valid_mask,
  per_expert_counts, padded_token_idx, padded_combine_weight)."""
  m_padded = compute_m_padded(topk_idx.shape[0], config.top_k, config.num_experts, local_num_experts,
                              capacity_factor, tile_size)
  return tuple(dispatch_local(topk_idx, topk_weight, x, local_expert_start, local_num_experts,
                              m_padded)[:6])


def filter_and_pad_to_shard(topk_idx, topk_weight, x, config, local_expert_start: int,
                            local_num_experts: int, capacity_factor: float = 2.0,
                            tile_size: int = MOSAIC_TILE_SIZE):
  """ref.py:658-751.  The reference proves its eager and jittable dispatches
  bit-identical (ref.py:880-939), so both names run the same fixed-shape GPU
  dispatch (no host sync); the eager overflow warning print is not emitted."""
  return filter_and_pad_to_shard_jittable(topk_idx, topk_weight, x, config, local_expert_start,
                                          local_num_experts, capacity_factor, tile_size)


def route_and_filter_to_local_shard_jittable(hidden_states, x, router_weight, e_score_correction_bias,
                                             config, local_expert_start, local_num_experts,
                                             capacity_factor=2.0, tile_size=MOSAIC_TILE_SIZE):
  """ref.py:1382-1416: _router_gate then the jittable dispatch."""
  topk_idx, topk_weight = _router_gate(hidden_states, router_weight, e_score_correction_bias, config)
  return filter_and_pad_to_shard_jittable(topk_idx, topk_weight, x, config, local_expert_start,
                                          local_num_experts, capacity_factor, tile_size)


route_and_filter_to_local_shard = route_and_filter_to_local_shard_jittable  # ref.py:1144-1187


# ---------------------------------------------------------------------------
# a13: combine
# ---------------------------------------------------------------------------


def _combine_shard_contribution(routed_out: torch.Tensor, shard_out: torch.Tensor,
                                padded_token_idx: torch.Tensor,
                                padded_combine_weight: torch.Tensor) -> torch.Tensor:
  """ref.py:1113-1141: routed_out.at[idx].add((shard_out * w).astype(routed_out.dtype)),
  returned as a new tensor.  Rows are added per token in ascending row order
  with the output dtype's rounding after every add (the reference's scatter
  order); idx -1 rows (padding, weight 0) are skipped."""
  _dev(routed_out, shard_out, padded_token_idx, padded_combine_weight)
  if shard_out.dim() != 2 or routed_out.dim() != 2 or routed_out.shape[1] != shard_out.shape[1]:
    raise ValueError(f"routed_out {tuple(routed_out.shape)} / shard_out {tuple(shard_out.shape)}: want (T, lat) / (m, lat)")
  m, lat = shard_out.shape
  if padded_token_idx.dtype != torch.int32 or padded_token_idx.numel() != m or padded_combine_weight.numel() != m:
    raise ValueError(f"padded_token_idx (int32) and padded_combine_weight need {m} entries, got "
                     f"{padded_token_idx.dtype} {padded_token_idx.numel()} / {padded_combine_weight.numel()}")
  out = routed_out.clone()
  t = routed_out.shape[0]
  ws = _workspace(lib().lmoe_combine_workspace_size(m, t), routed_out.device)
  check(lib().lmoe_combine_scatter_add(_p(shard_out), _dt(shard_out), _p(padded_token_idx),
                                       _p(padded_combine_weight), _dt(padded_combine_weight), m, lat, t,
                                       _p(out), _dt(out), _p(ws), ws.numel(), _stream()),
        "combine_scatter_add")
  return out


def _check_slots(shard_out, slot_pos, weights, num_tokens, top_k, mode):
  """The slot combine reads T*k slot positions, T*k weights (slot_sum) or one
  weight per shard row (scatter_add), and at least one shard row (dropped
  slots re-read row 0).  In scatter_add mode a shard of no rows (every slot
  dropped, m_padded == 0) adds nothing and is combined without a launch by
  the callers; slot_sum keeps every slot, so its rows cannot be missing."""
  if shard_out.dim() != 2 or (mode != "scatter_add" and num_tokens * top_k > 0 and shard_out.shape[0] == 0):
    raise ValueError(f"shard_out {tuple(shard_out.shape)}: want (m >= 1, lat)")
  if slot_pos.dtype != torch.int32 or slot_pos.numel() != num_tokens * top_k:
    raise ValueError(f"slot_pos must be int32 with T*k = {num_tokens * top_k} entries, got "
                     f"{slot_pos.dtype} {slot_pos.numel()}")
  want = num_tokens * top_k if mode == "slot_sum" else shard_out.shape[0]
  if mode in ("slot_sum", "scatter_add") and weights.numel() != want:
    raise ValueError(f"{mode} weights need {want} entries, got {weights.numel()}")


def combine_slots(shard_out: torch.Tensor, slot_pos: torch.Tensor, weights: torch.Tensor,
                  num_tokens: int, top_k: int, *, mode: str, routed_out: torch.Tensor | None = None,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
  """Combine driven by the dispatch's slot_pos.  mode="scatter_add": adds into a
  copy of routed_out exactly like _combine_shard_contribution (weights are the
  padded per-row weights); mode="slot_sum": the unsharded f32 weighted sum of
  ref.py:413-416 (weights are topk_weight (T, k) f32)."""
  _dev(shard_out, slot_pos, weights)
  _check_slots(shard_out, slot_pos, weights, num_tokens, top_k, mode)
  lat = shard_out.shape[-1]
  if mode == "scatter_add":
    if routed_out is None:
      routed_out = torch.zeros((num_tokens, lat), dtype=out_dtype or shard_out.dtype,
                               device=shard_out.device)
    if tuple(routed_out.shape) != (num_tokens, lat):
      raise ValueError(f"routed_out {tuple(routed_out.shape)}: want ({num_tokens}, {lat})")
    out = routed_out.clone()
    m = _lib.COMBINE_SCATTER_ADD
  elif mode == "slot_sum":
    out = torch.empty((num_tokens, lat), dtype=out_dtype or shard_out.dtype, device=shard_out.device)
    m = _lib.COMBINE_SLOT_SUM
  else:
    raise ValueError(mode)
  if shard_out.shape[0] == 0:  # no shard rows (no slots, or every one dropped): nothing to add
    return out if mode == "scatter_add" else out.zero_()
  check(lib().lmoe_combine_slots(_p(shard_out), _dt(shard_out), _p(slot_pos), _p(weights),
                                 _dt(weights), num_tokens, top_k, lat, m, _p(out), _dt(out),
                                 _stream()), "combine_slots")
  return out


def combine_slots_rms_norm(shard_out: torch.Tensor, slot_pos: torch.Tensor, weights: torch.Tensor,
                           num_tokens: int, top_k: int, norm_scale: torch.Tensor, eps: float, *, mode: str,
                           out_dtype: torch.dtype | None = None, return_routed: bool = False):
  """combine_slots into zeros followed by _rms_norm of the routed rows, in one
  kernel (bit-identical to the two calls): returns normed (T, lat), or
  (normed, routed) with ``return_routed``."""
  _dev(shard_out, slot_pos, weights, norm_scale)
  _check_slots(shard_out, slot_pos, weights, num_tokens, top_k, mode)
  lat = shard_out.shape[-1]
  if norm_scale.numel() != lat:
    raise ValueError(f"norm_scale has {norm_scale.numel()} entries for {lat} columns")
  dt = out_dtype or shard_out.dtype
  m = {"scatter_add": _lib.COMBINE_SCATTER_ADD, "slot_sum": _lib.COMBINE_SLOT_SUM}[mode]
  if shard_out.shape[0] == 0:  # no shard rows: the routed rows stay zero
    routed = torch.zeros((num_tokens, lat), dtype=dt, device=shard_out.device)
    normed = _rms_norm(routed, norm_scale.to(dt).contiguous(), eps)
    return (normed, routed) if return_routed else normed
  normed = torch.empty((num_tokens, lat), dtype=dt, device=shard_out.device)
  routed = torch.empty_like(normed) if return_routed else None
  check(lib().lmoe_combine_slots_rms_norm(_p(shard_out), _dt(shard_out), _p(slot_pos), _p(weights), _dt(weights),
                                          num_tokens, top_k, lat, m, _p(norm_scale.to(dt).contiguous()), eps,
                                          _p(routed), _p(normed), _dt(normed), _stream()), "combine_rms_norm")
  return (normed, routed) if return_routed else normed


def combine_rms_norm_supported(lat: int) -> bool:
  return lat % 8 == 0 and lat <= 2048


# ---------------------------------------------------------------------------
# a10 / a14: elementwise stages
# ---------------------------------------------------------------------------


def _rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
  """ref.py:286-293."""
  _dev(x, scale)
  n = x.shape[-1]
  if scale.numel() != n:
    raise ValueError(f"scale has {scale.numel()} entries for rows of {n}")
  out = torch.empty_like(x)
  if x.numel() == 0:  # no rows, or rows of width 0: nothing to normalise
    return out
  check(lib().lmoe_rms_norm(_p(x), _p(scale.to(x.dtype).contiguous()), x.numel() // n, n, eps, _dt(x),
                            _p(out), _stream()), "rms_norm")
  return out


def _situ_and_mul(gate: torch.Tensor, up: torch.Tensor, beta: float, linear_beta: float) -> torch.Tensor:
  """ref.py:296-310: f32 SiTU-GLU, cast back to the input dtype."""
  _dev(gate, up)
  if gate.shape != up.shape or gate.dtype != up.dtype:
    raise ValueError(f"gate {tuple(gate.shape)} {gate.dtype} / up {tuple(up.shape)} {up.dtype} differ")
  out = torch.empty_like(gate)
  check(lib().lmoe_situ_and_mul(_p(gate), _p(up), gate.numel(), beta, linear_beta, _dt(gate), _p(out),
                                _stream()), "situ_and_mul")
  return out


def add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
  """a + b rounded to the dtype (the residual add of ref.py:435)."""
  _dev(a, b)
  if a.shape != b.shape or a.dtype != b.dtype:
    raise ValueError(f"a {tuple(a.shape)} {a.dtype} / b {tuple(b.shape)} {b.dtype} differ")
  out = torch.empty_like(a)
  check(lib().lmoe_add(_p(a), _p(b), a.numel(), _dt(a), _p(out), _stream()), "add")
  return out


def _situ_glu_mlp(x, w_gate, w_up, w_down, beta, linear_beta):
  """ref.py:313-327 on dense weights (in, out): situ(x@Wg, x@Wu) @ Wd."""
  return dense(_situ_and_mul(dense(x, w_gate), dense(x, w_up), beta, linear_beta), w_down)


# ---------------------------------------------------------------------------
# a11: expert FFN over one shard
# ---------------------------------------------------------------------------


def _local_shard_expert_ffn(sorted_tokens, expert_gate, expert_up, expert_down, group_sizes, config):
  """ref.py:1486-1528, the reference's per-expert-loop form of the shard FFN
  (the oracle its ragged_dot form, rd.py:580-607, is checked against): the
  same function, so here both names run the grouped GEMMs -- gate / up,
  SiTU-GLU, down -- over the sorted rows, the trailing padding group included
  (its rows are zero, so are its outputs)."""
  return _local_shard_expert_ffn_ragged_dot(sorted_tokens, expert_gate, expert_up, expert_down, group_sizes,
                                            config)


def _local_shard_expert_ffn_ragged_dot(sorted_tokens, expert_gate, expert_up, expert_down,
                                       group_sizes, config, implementation=None, zero_group=-1):
  """rd.py:580-607: gate / up ragged_dots, SiTU-GLU, down ragged_dot."""
  b, bl = config.activation_situ_beta, config.activation_situ_linear_beta
  gate = ragged_dot(sorted_tokens, expert_gate, group_sizes, implementation=implementation,
                    zero_group=zero_group)
  up = ragged_dot(sorted_tokens, expert_up, group_sizes, implementation=implementation,
                  zero_group=zero_group)
  return ragged_dot(_situ_and_mul(gate, up, b, bl), expert_down, group_sizes,
                    implementation=implementation, zero_group=zero_group)


def _local_shard_expert_ffn_ragged_dot_fused_gateup(sorted_tokens, expert_gate, expert_up, expert_down,
                                                    group_sizes, config, zero_group=-1):
  """rd.py:726-748: prefuse then the fused gate/up + SiTU GEMM and the down GEMM."""
  fused = prefuse_gateup_weights(expert_gate, expert_up)
  return _fused_gateup_expert_ffn_from_prefused_weights(
      sorted_tokens, fused, expert_down, group_sizes, config.activation_situ_beta,
      config.activation_situ_linear_beta, zero_group=zero_group)


def _fused_gateup_expert_ffn_from_prefused_weights(sorted_tokens, fused_expert_gate_up, expert_down,
                                                   group_sizes, beta, linear_beta,
                                                   implementation=None, zero_group=-1,
                                                   rhs_layout="gkn"):
  """rd.py:644-723 on an already-prefused weight."""
  if implementation not in (None, "hip"):
    raise NotImplementedError(f"implementation={implementation!r}")
  act = ragged_dot_gateup_situ(sorted_tokens, fused_expert_gate_up, group_sizes, beta, linear_beta,
                               rhs_layout=rhs_layout, zero_group=zero_group)
  return ragged_dot(act, expert_down, group_sizes, rhs_layout=rhs_layout, zero_group=zero_group)
