"""A stand-in for liblmoe.so that computes, on the CPU, the entry points of
the bf16 / f32 forwards -- router top-k (with the projection's bf16 rows),
the four dispatch entry points, the three combines, the grouped GEMM and
fused gate/up, the dense projections, RMSNorm, SiTU-GLU, add and the row
cast -- and of the MXFP4 expert paths (weight tiling and dequantisation, the
grouped GEMM in both weight layouts and its gathered-rows, skinny and
split-K forms, the fused decode dispatch, MXFP8 / MXFP6 activation
quantisation and their scaled GEMMs) -- each reading and writing the host buffers behind the pointers the
operators pass, with the oracle's definitions (the slot-driven combine
restates the header's add order directly).  Test infrastructure only: it lets the
Python layer's composition (which entry point, which views, dtypes and
casts) be checked for values on a machine without a GPU; the kernels
themselves are checked on the GPU.  Where no GPU is present each call is
first put to the real library, whose host checks run before any launch: a
call the library refuses is refused here too, with its status and message.
Any other entry point raises."""
import ctypes

import numpy as np
import torch

from lmoe import _lib, ops
from oracle import lmoe_oracle as O


# the real library's host checks, only where nothing can launch
_HOST_CHECKS = torch.cuda.device_count() == 0


def _read(ptr, count, dtype):
  """float32 values of `count` elements of `dtype` (F32 / BF16) at ptr."""
  if count == 0:
    return np.zeros(0, np.float32)
  if dtype == _lib.F32:
    return np.ctypeslib.as_array((ctypes.c_float * count).from_address(ptr)).copy()
  if dtype == _lib.BF16:
    return O.bits_to_f32(np.ctypeslib.as_array((ctypes.c_uint16 * count).from_address(ptr)).copy())
  raise ValueError(dtype)


def _write(ptr, values, dtype):
  values = np.ascontiguousarray(values, np.float32).ravel()
  if values.size == 0:
    return
  if dtype == _lib.F32:
    np.ctypeslib.as_array((ctypes.c_float * values.size).from_address(ptr))[:] = values
  elif dtype == _lib.BF16:
    np.ctypeslib.as_array((ctypes.c_uint16 * values.size).from_address(ptr))[:] = O.bf16_bits(values)
  else:
    raise ValueError(dtype)


def _dt(code):
  return "f32" if code == _lib.F32 else "bf16"


def _ints(ptr, count, ctype=ctypes.c_int32):
  if count == 0 or not ptr:
    return np.zeros(0, np.int64)
  return np.ctypeslib.as_array((ctype * count).from_address(ptr)).astype(np.int64)


def _put_ints(ptr, values, ctype=ctypes.c_int32):
  v = np.asarray(values).ravel()
  if v.size and ptr:
    np.ctypeslib.as_array((ctype * v.size).from_address(ptr))[:] = v


def _rows(ptr, n, ld, width, dtype):
  """n rows of `width` elements, ld elements apart, as float32 (n, width)."""
  if n == 0 or width == 0:
    return np.zeros((n, width), np.float32)
  flat = _read(ptr, (n - 1) * ld + width, dtype)
  return np.stack([flat[i * ld:i * ld + width] for i in range(n)])


def _gkn(ptr, G, K, N, dtype, layout):
  """Grouped weights as (G, K, N) in memory order, whichever layout they have."""
  w = _read(ptr, G * K * N, dtype)
  return w.reshape(G, K, N) if layout == _lib.RHS_GKN else np.ascontiguousarray(w.reshape(G, N, K).transpose(0, 2, 1))


class EmulatedLib:
  def __init__(self):
    self.calls = []

  def __getattr__(self, name):
    if not name.startswith("lmoe_"):
      raise AttributeError(name)
    if name.endswith("workspace_size"):
      return getattr(_lib.lib(), name)
    impl = type(self).__dict__.get("_" + name)
    if impl is None:
      raise NotImplementedError(f"{name} is not emulated")
    impl = impl.__get__(self)

    def entry(*args):
      self.calls.append(name)
      if _HOST_CHECKS:
        rc = getattr(_lib.lib(), name)(*args)  # stops at its first HIP call (no device)
        if rc not in (_lib.OK, _lib.ERR_HIP):
          return rc
      return impl(*args)
    return entry

  def names(self):
    return list(self.calls)

  @staticmethod
  def _zero_group_rows(res, sizes, zero_group):
    if 0 <= zero_group < len(sizes):
      start = int(sizes[:zero_group].sum())
      res[start:start + int(sizes[zero_group])] = 0
    return res

  def _lmoe_ragged_dot(self, lhs, lhs_dt, rhs, layout, gs, M, K, N, G, zero_group, out, out_dt, stream):
    a = _read(lhs, M * K, lhs_dt).reshape(M, K)
    # (G, K, N) in memory order, so numpy sums each dot product as the oracle does
    w = _gkn(rhs, G, K, N, lhs_dt, layout)
    sizes = _ints(gs, G)
    res = self._zero_group_rows(O.ragged_dot(a, w, sizes, "f32"), sizes, zero_group)
    _write(out, O.cast(res, _dt(out_dt)), out_dt)
    return _lib.OK

  def _lmoe_ragged_dot_gateup_situ(self, lhs, rhs, layout, gs, M, K, I, G, zero_group, beta, beta_lin, rba, out,
                                   stream):
    a = _read(lhs, M * K, _lib.BF16).reshape(M, K)
    sizes = _ints(gs, G)
    res = O.ragged_dot_gateup_situ(a, _gkn(rhs, G, K, 2 * I, _lib.BF16, layout), sizes, beta, beta_lin, "bf16",
                                   round_before_act=bool(rba))
    _write(out, self._zero_group_rows(res, sizes, zero_group), _lib.BF16)
    return _lib.OK

  def _lmoe_ragged_dot_fp8_scaled(self, lhs, rhs_q, rhs_scale, block_size, gs, M, K, N, G, zero_group, epi, beta,
                                  beta_lin, out, stream):
    a = _read(lhs, M * K, _lib.BF16).reshape(M, K)
    q = _ints(rhs_q, G * K * N, ctypes.c_uint8).astype(np.uint8).reshape(G, K, N)
    sc = _read(rhs_scale, G * (K // block_size) * N, _lib.F32).reshape(G, K // block_size, 1, N)
    sizes = _ints(gs, G)
    res = O.ragged_dot_fp8_scaled(a, q, sc, sizes, "bf16", situ=(beta, beta_lin) if epi == _lib.EPI_SITU else None)
    _write(out, self._zero_group_rows(res, sizes, zero_group), _lib.BF16)
    return _lib.OK

  # ---- dense projections: x (M, K) @ w_nk^T, f32 accumulation
  def _lmoe_dense_blaslt(self, x, x_dt, w, w_dt, M, K, N, out, out_dt, stream):
    a = _read(x, M * K, x_dt).reshape(M, K)
    b = _read(w, N * K, w_dt).reshape(N, K)
    _write(out, O.matmul(a, np.ascontiguousarray(b.T), _dt(out_dt)), out_dt)
    return _lib.OK

  def _lmoe_dense(self, x, w, M, K, N, out, out_dt, stream):
    return self._lmoe_dense_blaslt(x, _lib.BF16, w, _lib.BF16, M, K, N, out, out_dt, stream)

  _lmoe_dense_skinny = _lmoe_dense

  # ---- router
  def _lmoe_router_topk_ld(self, logits, ld, bias, T, E, k, act, renorm, scale, w_dt, idx, w, scores, stream):
    if T == 0:
      return _lib.OK
    lg = _rows(logits, T, ld, E, _lib.F32)
    b = _read(bias, E, _lib.F32) if bias else None
    r = O.router_from_logits(lg, b, k, bool(renorm), scale, "sigmoid" if act == _lib.ACT_SIGMOID else "softmax",
                             _dt(w_dt))
    _put_ints(idx, r.topk_idx)
    _write(w, r.topk_weight, w_dt)
    if scores:
      _write(scores, r.scores, _lib.F32)
    return _lib.OK

  def _lmoe_router_topk(self, logits, bias, T, E, k, act, renorm, scale, w_dt, idx, w, scores, stream):
    return self._lmoe_router_topk_ld(logits, E, bias, T, E, k, act, renorm, scale, w_dt, idx, w, scores, stream)

  def _lmoe_router_topk_proj(self, logits, ld, bias, T, E, k, act, renorm, scale, w_dt, idx, w, x_src, x_ld, lat,
                             x_out, stream):
    self._lmoe_router_topk_ld(logits, ld, bias, T, E, k, act, renorm, scale, w_dt, idx, w, None, stream)
    _write(x_out, O.cast(_rows(x_src, T, x_ld, lat, _lib.F32), "bf16"), _lib.BF16)
    return _lib.OK

  # ---- dispatch (ref.py:754-877): the oracle's jittable dispatch
  def _dispatch(self, idx, w, w_dt, xrows, T, k, start, L, m_padded, sorted_tokens, sorted_dt, gs, valid, counts,
                tok, pw, slot, skip_padding):
    if T == 0:  # no slots: every row is padding
      width = xrows.shape[1] if xrows is not None else 1
      sorted_x, sizes = np.zeros((m_padded, width), np.float32), np.zeros(L + 1, np.int32)
      sizes[L] = m_padded
      ok, cnt = np.zeros(m_padded, bool), np.zeros(L, np.int32)
      tk, wk, slot_pos = np.full(m_padded, -1, np.int32), np.zeros(m_padded, np.float32), np.zeros(0, np.int32)
    else:
      ids = _ints(idx, T * k).reshape(T, k)
      wts = _read(w, T * k, w_dt).reshape(T, k)
      x = xrows if xrows is not None else np.zeros((T, 1), np.float32)
      d, slot_pos = O.filter_and_pad_to_shard_jittable(ids, wts, x, k, start + L, start, L, m_padded=m_padded,
                                                       return_slot_pos=True)
      sorted_x, sizes, ok, cnt, tk, wk = d
    if sorted_tokens and xrows is not None:
      rows = int(cnt.sum()) if skip_padding else m_padded
      _write(sorted_tokens, O.cast(sorted_x[:rows], _dt(sorted_dt)), sorted_dt)
    _put_ints(gs, sizes)
    _put_ints(valid, ok.astype(np.uint8), ctypes.c_uint8)
    _put_ints(counts, cnt)
    _put_ints(tok, tk)
    _write(pw, O.cast(wk, _dt(w_dt)), w_dt)
    _put_ints(slot, slot_pos)
    return _lib.OK

  def _lmoe_dispatch_local_noalloc(self, idx, w, w_dt, x, x_dt, T, k, lat, start, L, m_padded, sorted_tokens, gs,
                                   valid, counts, tok, pw, slot, stream):
    return self._dispatch(idx, w, w_dt, _rows(x, T, lat, lat, x_dt), T, k, start, L, m_padded, sorted_tokens,
                          x_dt, gs, valid, counts, tok, pw, slot, False)

  def _lmoe_dispatch_local(self, idx, w, w_dt, x, x_dt, T, k, lat, start, L, m_padded, sorted_tokens, gs, valid,
                           counts, tok, pw, slot, ws, ws_size, stream):
    return self._lmoe_dispatch_local_noalloc(idx, w, w_dt, x, x_dt, T, k, lat, start, L, m_padded, sorted_tokens,
                                             gs, valid, counts, tok, pw, slot, stream)

  def _lmoe_dispatch_local_small(self, idx, w, w_dt, x, x_dt, x_ld, T, k, lat, start, L, m_padded, sorted_tokens,
                                 gs, valid, counts, tok, pw, slot, flags, stream):
    if flags & _lib.DISPATCH_FLAG_NO_ROWS:
      xrows = None
    else:
      xrows = _rows(x, T, x_ld, lat, x_dt) if T else np.zeros((0, lat), np.float32)
    return self._dispatch(idx, w, w_dt, xrows, T, k, start, L, m_padded, sorted_tokens, _lib.BF16, gs, valid,
                          counts, tok, pw, slot, bool(flags & _lib.DISPATCH_FLAG_SKIP_PADDING_ROWS))

  def _lmoe_dispatch_local_rows(self, idx, w, w_dt, x, x_dt, x_ld, T, k, lat, start, L, m_padded, sorted_tokens,
                                gs, valid, counts, tok, pw, slot, flags, ws, ws_size, stream):
    return self._lmoe_dispatch_local_small(idx, w, w_dt, x, x_dt, x_ld, T, k, lat, start, L, m_padded,
                                           sorted_tokens, gs, valid, counts, tok, pw, slot, flags, stream)

  # ---- combine
  @staticmethod
  def _combine(shard, shard_dt, slot, w, w_dt, T, k, lat, mode, routed, out_dt):
    """routed (T, lat) float32 values before the combine -> after it."""
    sp = _ints(slot, T * k).reshape(T, k)
    kept = sp[sp >= 0]
    m = int(kept.max()) + 1 if kept.size else 1
    rows = _read(shard, m * lat, shard_dt).reshape(m, lat)
    if mode == _lib.COMBINE_SLOT_SUM:
      # ref.py:413-416: f32 weighted sum over the k slots in slot order, one cast
      wt = _read(w, T * k, w_dt).reshape(T, k)
      acc = np.zeros((T, lat), np.float32)
      for j in range(k):
        vals = np.where((sp[:, j] >= 0)[:, None], rows[np.maximum(sp[:, j], 0)], np.float32(0))
        acc = (acc + vals * wt[:, j:j + 1]).astype(np.float32)
      return O.cast(acc, _dt(out_dt))
    # ref.py:1113-1141: each token's kept rows added in ascending row order
    pw = _read(w, m, w_dt)
    pti = np.full(m, -1, np.int64)
    for t in range(T):
      for j in range(k):
        if sp[t, j] >= 0:
          pti[sp[t, j]] = t
    return O.combine_shard_contribution(routed, rows, pti, pw, _dt(out_dt), _dt(shard_dt), _dt(w_dt))

  def _lmoe_combine_slots(self, shard, shard_dt, slot, w, w_dt, T, k, lat, mode, routed, out_dt, stream):
    cur = _read(routed, T * lat, out_dt).reshape(T, lat) if mode == _lib.COMBINE_SCATTER_ADD else None
    _write(routed, self._combine(shard, shard_dt, slot, w, w_dt, T, k, lat, mode, cur, out_dt), out_dt)
    return _lib.OK

  def _lmoe_combine_slots_rms_norm(self, shard, shard_dt, slot, w, w_dt, T, k, lat, mode, scale, eps, routed,
                                   normed, dt, stream):
    res = self._combine(shard, shard_dt, slot, w, w_dt, T, k, lat, mode, np.zeros((T, lat), np.float32), dt)
    if routed:
      _write(routed, res, dt)
    _write(normed, O.rms_norm(res, _read(scale, lat, dt), eps, _dt(dt)), dt)
    return _lib.OK

  def _lmoe_combine_scatter_add(self, shard, shard_dt, pti, pw, w_dt, m, lat, T, routed, out_dt, ws, ws_size,
                                stream):
    cur = _read(routed, T * lat, out_dt).reshape(T, lat)
    res = O.combine_shard_contribution(cur, _read(shard, m * lat, shard_dt).reshape(m, lat), _ints(pti, m),
                                       _read(pw, m, w_dt), _dt(out_dt), _dt(shard_dt), _dt(w_dt))
    _write(routed, res, out_dt)
    return _lib.OK

  # ---- MXFP4 weights: checkpoint (G, N, K/2) + (G, N, K/32); tiled (G, K/64, N, 32) + (G, K/64, N, 2),
  # each 32-byte record holding the checkpoint's eight 4-byte groups in the order below
  _RECORD = np.array([0, 2, 4, 6, 1, 3, 5, 7])

  @classmethod
  def _untile(cls, wp, ws, G, N, K):
    tp = _ints(wp, G * (K // 64) * N * 32, ctypes.c_uint8).astype(np.uint8).reshape(G, K // 64, N, 8, 4)
    ts = _ints(ws, G * (K // 64) * N * 2, ctypes.c_uint8).astype(np.uint8).reshape(G, K // 64, N, 2)
    packed = np.empty_like(tp)
    packed[:, :, :, cls._RECORD] = tp
    packed = packed.transpose(0, 2, 1, 3, 4).reshape(G, N, K // 2)
    return packed, np.ascontiguousarray(ts.transpose(0, 2, 1, 3).reshape(G, N, K // 32))

  @staticmethod
  def _checkpoint(wp, ws, G, N, K):
    return (_ints(wp, G * N * (K // 2), ctypes.c_uint8).astype(np.uint8).reshape(G, N, K // 2),
            _ints(ws, G * N * (K // 32), ctypes.c_uint8).astype(np.uint8).reshape(G, N, K // 32))

  def _lmoe_mxfp4_tile(self, packed, scale, G, N, K, packed_out, scale_out, stream):
    pk, sc = self._checkpoint(packed, scale, G, N, K)
    rec = pk.reshape(G, N, K // 64, 8, 4)[:, :, :, self._RECORD].transpose(0, 2, 1, 3, 4)
    _put_ints(packed_out, rec.reshape(-1), ctypes.c_uint8)
    _put_ints(scale_out, sc.reshape(G, N, K // 64, 2).transpose(0, 2, 1, 3).reshape(-1), ctypes.c_uint8)
    return _lib.OK

  def _lmoe_mxfp4_dequant(self, packed, scale, batch, N, K, group_size, out, out_dt, stream):
    pk = _ints(packed, batch * N * (K // 2), ctypes.c_uint8).astype(np.uint8).reshape(batch, N, K // 2)
    sc = _ints(scale, batch * N * (K // group_size), ctypes.c_uint8).astype(np.uint8).reshape(batch, N, -1)
    _write(out, O.cast(O.dequantize_mxfp4(pk, sc), _dt(out_dt)), out_dt)
    return _lib.OK

  def _mx_gemm(self, a, pk, sc, sizes, zero_group, epi, beta, beta_lin, out):
    res = O.ragged_dot_mxfp4(a, pk, sc, sizes, "bf16", situ=(beta, beta_lin) if epi == _lib.EPI_SITU else None)
    _write(out, self._zero_group_rows(res, sizes, zero_group), _lib.BF16)
    return _lib.OK

  def _lmoe_ragged_dot_mxfp4(self, lhs, wp, ws, gs, M, K, N, G, zero_group, mode, epi, beta, beta_lin, out,
                             stream):
    mode &= ~_lib.MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS  # rows it lets go unwritten are written (as zeros)
    pk, sc = (self._untile if mode == _lib.MXFP4_LDS_DEQUANT_TILED else self._checkpoint)(wp, ws, G, N, K)
    return self._mx_gemm(_read(lhs, M * K, _lib.BF16).reshape(M, K), pk, sc, _ints(gs, G), zero_group, epi, beta,
                         beta_lin, out)

  def _lmoe_ragged_dot_mxfp4_rows(self, lhs, lhs_rows, row_index, wp, ws, gs, M, K, N, G, zero_group, mode, epi,
                                  beta, beta_lin, out, stream):
    tokens = _read(lhs, lhs_rows * K, _lib.BF16).reshape(lhs_rows, K)
    a = tokens[np.clip(_ints(row_index, M), 0, max(lhs_rows - 1, 0))] if lhs_rows else np.zeros((M, K), np.float32)
    pk, sc = self._untile(wp, ws, G, N, K)
    return self._mx_gemm(a, pk, sc, _ints(gs, G), zero_group, epi, beta, beta_lin, out)

  def _lmoe_ragged_dot_mxfp4_skinny(self, lhs, wt, st, gs, M, K, N, G, zero_group, flags, epi, beta, beta_lin,
                                    max_group_rows, out, stream):
    pk, sc = self._untile(wt, st, G, N, K)
    return self._mx_gemm(_read(lhs, M * K, _lib.BF16).reshape(M, K), pk, sc, _ints(gs, G), zero_group, epi, beta,
                         beta_lin, out)

  def _lmoe_ragged_dot_mxfp4_splitk(self, lhs, wp, ws, gs, M, K, N, G, zero_group, k_split, work, work_bytes, epi,
                                    beta, beta_lin, out, stream):
    return self._lmoe_ragged_dot_mxfp4_skinny(lhs, wp, ws, gs, M, K, N, G, zero_group, 0, epi, beta, beta_lin, 0,
                                              out, stream)

  def _lmoe_dispatch_mxfp4_skinny(self, idx, w, w_dt, x, x_ld, T, k, start, L, m_padded, wt, st, K, N, epi, beta,
                                  beta_lin, flags, gs, valid, counts, tok, pw, slot, out, stream):
    self._dispatch(idx, w, w_dt, None, T, k, start, L, m_padded, None, _lib.BF16, gs, valid, counts, tok, pw, slot,
                   False)
    rows = _rows(x, T, x_ld, K, _lib.BF16)
    t = _ints(tok, m_padded)
    a = np.where((t >= 0)[:, None], rows[np.maximum(t, 0)] if T else 0, np.float32(0)).astype(np.float32)
    pk, sc = self._untile(wt, st, L + 1, N, K)
    return self._mx_gemm(a, pk, sc, _ints(gs, L + 1), L, epi, beta, beta_lin, out)

  # ---- MXFP8 / MXFP6 activations: codes (M, K) / packed (M, K*3/4), E8M0 scales k-step-major
  # (K/128, roundup(M, 4), 4): scale_t[s, m, j] = scale[m, 4 s + j], pad rows 0
  @staticmethod
  def _put_scales(ptr, scales, M, K):
    m4 = -(-M // 4) * 4
    st = np.zeros((K // 128, m4, 4), np.uint8)
    st[:, :M, :] = np.asarray(scales, np.uint8).reshape(M, K // 128, 4).transpose(1, 0, 2)
    _put_ints(ptr, st.reshape(-1), ctypes.c_uint8)

  @staticmethod
  def _get_scales(ptr, M, K):
    m4 = -(-M // 4) * 4
    st = _ints(ptr, (K // 128) * m4 * 4, ctypes.c_uint8).astype(np.uint8).reshape(K // 128, m4, 4)
    return np.ascontiguousarray(st.transpose(1, 0, 2).reshape(m4, K // 32)[:M])

  def _lmoe_quantize_mxfp8(self, x, x_dt, M, K, q, scale_t, stream):
    codes, scales = O.quantize_mxfp8(_read(x, M * K, x_dt).reshape(M, K))
    _put_ints(q, codes.reshape(-1), ctypes.c_uint8)
    self._put_scales(scale_t, scales, M, K)
    return _lib.OK

  def _lmoe_quantize_mxfp6(self, x, x_dt, M, K, q, scale_t, stream):
    codes, scales = O.quantize_mxfp6(_read(x, M * K, x_dt).reshape(M, K))
    _put_ints(q, O.pack_fp6(codes).reshape(-1), ctypes.c_uint8)
    self._put_scales(scale_t, scales, M, K)
    return _lib.OK

  def _lmoe_ragged_dot_mxfp8_mxfp4(self, q, qs, wp, ws, gs, M, K, N, G, zero_group, epi, beta, beta_lin, out,
                                   out_dt, stream):
    codes = _ints(q, M * K, ctypes.c_uint8).astype(np.uint8).reshape(M, K)
    pk, sc = self._untile(wp, ws, G, N, K)
    sizes = _ints(gs, G)
    situ = epi == _lib.EPI_SITU
    dt = _lib.BF16 if situ else out_dt
    res = O.ragged_dot_mxfp8_mxfp4(codes, self._get_scales(qs, M, K), pk, sc, sizes, _dt(dt),
                                   situ=(beta, beta_lin) if situ else None)
    _write(out, self._zero_group_rows(res, sizes, zero_group), dt)
    return _lib.OK

  def _lmoe_ragged_dot_mxfp6_mxfp4(self, q, qs, wp, ws, gs, M, K, N, G, zero_group, out, out_dt, stream):
    codes = O.unpack_fp6(_ints(q, M * K * 3 // 4, ctypes.c_uint8).astype(np.uint8).reshape(M, K * 3 // 4), K)
    pk, sc = self._untile(wp, ws, G, N, K)
    sizes = _ints(gs, G)
    res = O.ragged_dot_mxfp6_mxfp4(codes, self._get_scales(qs, M, K), pk, sc, sizes, _dt(out_dt))
    _write(out, self._zero_group_rows(res, sizes, zero_group), out_dt)
    return _lib.OK

  # ---- elementwise
  def _lmoe_rms_norm(self, x, scale, rows, n, eps, dt, out, stream):
    _write(out, O.rms_norm(_read(x, rows * n, dt).reshape(rows, n), _read(scale, n, dt), eps, _dt(dt)), dt)
    return _lib.OK

  def _lmoe_cast_rows(self, x, x_dt, rows, cols, ld, out, out_dt, stream):
    _write(out, O.cast(_rows(x, rows, ld, cols, x_dt), _dt(out_dt)), out_dt)
    return _lib.OK

  def _lmoe_situ_and_mul(self, gate, up, count, beta, beta_lin, dt, out, stream):
    g, u = _read(gate, count, dt), _read(up, count, dt)
    _write(out, O.situ_and_mul(g, u, beta, beta_lin, _dt(dt)), dt)
    return _lib.OK

  def _lmoe_add(self, a, b, count, dt, out, stream):
    _write(out, O.cast(_read(a, count, dt) + _read(b, count, dt), _dt(dt)), dt)
    return _lib.OK


def install(monkeypatch) -> EmulatedLib:
  lib = EmulatedLib()

  def dev(*ts):
    for t in ts:
      if t is not None and not t.is_contiguous():
        raise ValueError("LatentMoE operators need contiguous tensors")

  def dev_rows(t):
    if t.dim() != 2:
      raise ValueError("expected a 2-D tensor")
    return t.contiguous() if t.stride(1) != 1 or t.stride(0) < t.shape[1] else t

  monkeypatch.setattr(ops, "lib", lambda: lib)
  monkeypatch.setattr(ops, "_stream", lambda: 0)
  monkeypatch.setattr(ops, "_dev", dev)
  monkeypatch.setattr(ops, "_dev_rows", dev_rows)
  return lib
