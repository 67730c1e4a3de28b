/*
 * lmoe.h -- C-ABI of liblmoe.so, the MI355X (gfx950) LatentMoE expert hot path.
 *
 * Every pointer argument is a DEVICE pointer owned by the caller (in the Python
 * host layer: torch tensors), except where marked "host".  Every call is
 * stream-ordered on `stream` (a hipStream_t passed as void*; NULL = the null
 * stream), allocates nothing, and returns an int status: LMOE_OK (0) or a
 * negative LMOE_ERR_* code, with a message retrievable from lmoe_last_error()
 * (thread-local).  Calls hold no global state and are safe to issue from
 * several host threads on different streams, with two exceptions stated at
 * their declarations: lmoe_dense_blaslt keeps library handles and plans, and
 * lmoe_dispatch_local_noalloc uses one static scratch array per GPU.
 *
 * Data types: bf16 is stored as its 16-bit pattern (torch.bfloat16 layout),
 * f32 as IEEE float.  Index arrays are int32.  Booleans are one byte.
 *
 * Sizes are int64.  A call whose buffers would hold more than 2^48 elements
 * (beyond any device's memory), or whose sizes exceed a limit stated at its
 * declaration, returns LMOE_ERR_UNSUPPORTED before anything is launched; the
 * size products are formed with overflow checks, so no size wraps around.
 * A null pointer for a buffer a call needs returns LMOE_ERR_INVALID.
 *
 * The reference interface each entry point replaces is cited as file:line
 * relative to the reference repository (Yog-Sothothftgn/tokamax-tpu-kernel-lab),
 * with these aliases:
 *   ref.py = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py
 *   rd.py  = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_ragged_dot.py
 *   deq.py = 05_ragged_dot_on_tpu/mxfp4_dequant.py
 *   odq.py = 05_ragged_dot_on_tpu/mxfp4_online_dequant_matmul_pallas.py
 *   gk.py  = 05_ragged_dot_on_tpu/own_gateup_situ_pallas_kernel.py
 */
#ifndef LMOE_H_
#define LMOE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------*/
#define LMOE_OK 0
#define LMOE_ERR_INVALID -1     /* bad shape / argument (Python: ValueError) */
#define LMOE_ERR_UNSUPPORTED -2 /* dtype / layout / size not implemented (NotImplementedError) */
#define LMOE_ERR_HIP -3         /* HIP runtime error */
#define LMOE_ERR_WORKSPACE -4   /* workspace missing or too small */

/* ---- dtypes and enums -----------------------------------------------------*/
#define LMOE_F32 0
#define LMOE_BF16 1

#define LMOE_RHS_GKN 0 /* rhs[g][k][n], n contiguous: the reference layout (x @ W) */
#define LMOE_RHS_GNK 1 /* rhs[g][n][k], k contiguous: prepared / checkpoint layout */

#define LMOE_ACT_SIGMOID 0
#define LMOE_ACT_SOFTMAX 1

#define LMOE_EPI_NONE 0
#define LMOE_EPI_SITU 1 /* rhs N axis is [gate | up]; out = SiTU-GLU(gate, up), width N/2 */

#define LMOE_MXFP4_LDS_DEQUANT 0 /* dequantise weight tiles to bf16 in LDS, bf16 MFMA */
#define LMOE_MXFP4_SCALED_MFMA 1 /* native scaled MFMA: use lmoe_quantize_mxfp8 + lmoe_ragged_dot_mxfp8_mxfp4 */
#define LMOE_MXFP4_LDS_DEQUANT_TILED 2 /* as LDS_DEQUANT, weights re-tiled by lmoe_mxfp4_tile */
/* OR-ed into the mode: the rows of zero_group and the rows past
 * sum(group_sizes) may be left unwritten instead of zeroed (for callers that
 * never read them, e.g. the padding bucket of a local-shard layer); honoured
 * by the tiled path, the others write zeros. */
#define LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS 0x100

#define LMOE_COMBINE_SCATTER_ADD 0 /* sharded: sequential adds rounded to out dtype (ref.py:1113-1141) */
#define LMOE_COMBINE_SLOT_SUM 1    /* unsharded: f32 sum over slots, one cast (ref.py:413-416) */

/* ---- library ----------------------------------------------------------------*/
const char* lmoe_last_error(void); /* host string, valid until the next call on this thread */
int lmoe_version(void);
int lmoe_device_arch_ok(void); /* 1 if device 0 is gfx950, else 0 (host-side query) */

/* ---- a9: grouped GEMM ----------------------------------------------------------
 * Replaces tokamax.ragged_dot(lhs, rhs, group_sizes) (call sites rd.py:358-369,
 * rd.py:604-607): rows [cum_g, cum_g + n_g) of lhs times
 * rhs[g]; rows past sum(group_sizes) are written as zero.  lhs (M, K) and out
 * (M, N) row-major; out dtype may differ from lhs dtype (f32 out = the logits
 * GEMM of ref.py:620).  group_sizes (G,) int32 is read on the device only.
 * `zero_group` >= 0 names one group whose rows are written as zero without
 * reading its weights (the trailing padding bucket, whose input rows are zero:
 * ref.py:1497-1500); pass -1 to compute every group.
 * bf16: K % 8 == 0, N % 8 == 0, 16-byte aligned lhs/rhs; f32: any shape.
 * M < 2^31 rows (also for every grouped GEMM below).
 */
int lmoe_ragged_dot(const void* lhs, int lhs_dtype, const void* rhs, int rhs_layout,
                    const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                    int zero_group, void* out, int out_dtype, void* stream);

/* ---- a12: fused gate/up + SiTU-GLU epilogue ------------------------------------
 * Replaces PallasMosaicTpuV2RaggedDot()(lhs, rhs_gu, group_sizes=...,
 * fuse_gateup_activation="situ:<beta>:<beta_lin>") (rd.py:713-720) over the
 * prefused [gate | up] weight of rd.py:610-641 (rhs_gu: (G, K, 2I) for GKN,
 * (G, 2I, K) for GNK).  out (M, I) = SiTU(gate, up) with the epilogue of
 * gk.py:114-125: accumulators rounded to bf16 first when round_before_act != 0.
 * bf16 only.
 */
int lmoe_ragged_dot_gateup_situ(const void* lhs, const void* rhs_gu, int rhs_layout,
                                const int32_t* group_sizes, int64_t M, int64_t K, int64_t I,
                                int64_t G, int zero_group, float beta, float beta_lin,
                                int round_before_act, void* out, void* stream);

/* ---- a19: block-scaled fp8 weights ---------------------------------------------
 * Replaces PallasMosaicTpuV2RaggedDot()(lhs, rhs_q, group_sizes=...,
 * rhs_scale=..., maybe_quantize_lhs=False) on fp8 weights (rd.py:2789-2811:
 * one scale per (group, column), rhs_scale (G, 1, 1, N); rd.py:2836-2953: one
 * per 32 rows of K, (G, K/32, 1, N)).  rhs_q (G, K, N) OCP E4M3 ("fn") codes,
 * rhs_scale (G, K/block_size, 1, N) f32; every weight is used as
 * bf16(f32(code) * scale) -- the reference's own check dequantises
 * (rhs_q.astype(f32) * scale).astype(bf16) and runs ragged_dot -- and the
 * products are accumulated in f32.  lhs (M, K) bf16, out (M, N) bf16, or
 * (M, N/2) with LMOE_EPI_SITU ([gate | up] on N, rounded to bf16 before the
 * activation).  block_size divides K and is a multiple of 4 (the reference
 * uses K and 32).  K % 8 == 0, N % 8 == 0 (N % 16 with SiTU); lhs 16-byte,
 * rhs_q 8-byte, rhs_scale 16-byte aligned.  Rows past sum(group_sizes) are zero.
 */
int lmoe_ragged_dot_fp8_scaled(const void* lhs, const uint8_t* rhs_q, const float* rhs_scale, int64_t block_size,
                               const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                               int zero_group, int epilogue, float beta, float beta_lin, void* out, void* stream);

/* ---- a17: MXFP4 dequantisation ---------------------------------------------------
 * Replaces dequantize_mxfp4(weight_packed, weight_scale) (deq.py:29-67):
 * packed (N, K/2) u8 (low nibble = element 2j), scale (N, K/gs) u8 E8M0 ->
 * out (N, K) in out_dtype (f32 or bf16), bit-exact (E2M1 * 2^(s-127)).
 * Batched over `batch` independent matrices laid out back to back.
 */
int lmoe_mxfp4_dequant(const uint8_t* packed, const uint8_t* scale, int64_t batch, int64_t N,
                       int64_t K, int64_t group_size, void* out, int out_dtype, void* stream);

/* ---- a18 (+a12): grouped GEMM on MXFP4 weights ------------------------------------
 * out = lhs @ deq(W_g)^T per group (orientation of odq.py:1-36 / odq.py:150-157,
 * checkpoint layout W_g (N, K/2) u8 + (N, K/32) u8, group size 32).  With
 * epilogue LMOE_EPI_SITU the N axis is [gate | up] and out is (M, N/2).
 * lhs bf16 (M, K), out bf16.  mode: LMOE_MXFP4_LDS_DEQUANT,
 * LMOE_MXFP4_LDS_DEQUANT_TILED (same result; w_packed (G, K/64, N, 32) and
 * w_scale (G, K/64, N, 2) from lmoe_mxfp4_tile, which lets each k step's
 * weight tile stream into LDS as one contiguous read) or
 * LMOE_MXFP4_SCALED_MFMA.
 */
int lmoe_ragged_dot_mxfp4(const void* lhs, const uint8_t* w_packed, const uint8_t* w_scale,
                          const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                          int zero_group, int mode, int epilogue, float beta, float beta_lin,
                          void* out, void* stream);

/* ---- a11/a12 + a18: the expert GEMM on gathered token rows --------------------------
 * lmoe_ragged_dot_mxfp4 (tiled weights, LMOE_MXFP4_LDS_DEQUANT_TILED) whose
 * grouped lhs is gathered from a token array: row r of the grouped problem is
 * row row_index[r] of lhs (lhs_rows, K) bf16 -- the composition
 * ragged_dot(x[padded_token_idx], W, group_sizes) that rd.py:604-607 (and the
 * fused gate/up of rd.py:644-723) run on the dispatch's sorted_tokens, without
 * materialising sorted_tokens.  row_index is the dispatch's padded_token_idx
 * (M entries; only rows inside the groups are read, indices are clamped into
 * [0, lhs_rows)).  Same results as gathering first, bit for bit.  The streamed
 * kernel only: LMOE_ERR_UNSUPPORTED when it does not apply (lhs_rows > 65536,
 * or more than 8 tiles per resident block).  Optional
 * LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS.
 */
int lmoe_ragged_dot_mxfp4_rows(const void* lhs, int64_t lhs_rows, const int32_t* row_index,
                               const uint8_t* w_packed, const uint8_t* w_scale, const int32_t* group_sizes,
                               int64_t M, int64_t K, int64_t N, int64_t G, int zero_group, int mode,
                               int epilogue, float beta, float beta_lin, void* out, void* stream);

/* ---- a18, few long-K tiles: split-K grouped GEMM on tiled MXFP4 weights ---------
 * Same operation as lmoe_ragged_dot_mxfp4 with LMOE_MXFP4_LDS_DEQUANT_TILED
 * (the config-4 matmul of odq.py:65-172 / mxfp4_online_dequant_matmul_pallas.py:94-157
 * at M <= ~1024, where the tile grid alone fills a fraction of the chip): the
 * K steps of every tile are dealt into k_split contiguous ranges (1 <= k_split
 * <= K/64; ranges of ceil(K/64 / k_split) steps, fewer ranges when that
 * leaves one empty), each range's f32 partial sums go to `workspace`
 * (k_split * M * N * 4 bytes, 16-byte aligned, caller-owned), and a second
 * kernel adds the ranges in order and applies the epilogue.  Repeatable bit
 * for bit; agrees with the unsplit kernel within bf16 rounding (another f32
 * summation order).  Rows of zero_group and past sum(group_sizes) are zero.
 * k_split == 1 runs the unsplit kernel (workspace unused).
 */
int lmoe_ragged_dot_mxfp4_splitk(const void* lhs, const uint8_t* w_packed, const uint8_t* w_scale,
                                 const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                 int zero_group, int64_t k_split, float* workspace, int64_t workspace_bytes,
                                 int epilogue, float beta, float beta_lin, void* out, void* stream);

/* ---- a18, decode regime: skinny-M grouped GEMM on tiled MXFP4 weights -------------
 * Same result contract as lmoe_ragged_dot_mxfp4 with LMOE_MXFP4_LDS_DEQUANT_TILED
 * (w_tiled / s_tiled from lmoe_mxfp4_tile, bf16 lhs and out, epilogue
 * LMOE_EPI_NONE or LMOE_EPI_SITU, flags 0 or LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS),
 * for the case the reference's decode sweep runs through the same ragged_dot
 * (rd.py:553-577: num_tokens 1..128, a few rows per local expert) and the
 * config-4 matmul at small M (odq.py:65-172).  Each weight byte of a group
 * with rows is read once per pass of 16 * c rows, c in {1, 2, 4} chosen from
 * min(M, max_group_rows) (max_group_rows <= 0: unknown; a bound that is too
 * small only costs extra passes).  Partial sums are added in a fixed order
 * (repeatable bit for bit) but not in the tile kernel's: the two agree within
 * bf16 rounding, not bit for bit.  K % 128 == 0, N % 16 == 0 (N % 32 with
 * SiTU), G <= 1024, M, K, N < 2^31; lhs, w_tiled and out 16-byte aligned.
 * No workspace.
 */
int lmoe_ragged_dot_mxfp4_skinny(const void* lhs, const uint8_t* w_tiled, const uint8_t* s_tiled,
                                 const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                 int zero_group, int flags, int epilogue, float beta, float beta_lin,
                                 int64_t max_group_rows, void* out, void* stream);

/* ---- f4, decode regime: the one-launch dispatch fused into the skinny gate/up --------
 * lmoe_dispatch_local_small (ref.py:754-877: stable expert-major order, tail
 * truncation at m_padded, padding bucket L) followed by
 * lmoe_ragged_dot_mxfp4_skinny on the sorted rows (rd.py:610-723, gate/up
 * with the SiTU epilogue, or a plain product) in one launch, for a decode
 * step (rd.py:553-577).  Every dispatch output but sorted_tokens is written
 * exactly as lmoe_dispatch_local_small writes it; out equals
 * lmoe_ragged_dot_mxfp4_skinny(sorted_tokens, ..., group_sizes, M = m_padded,
 * G = L + 1, zero_group = L, max_group_rows = T) bit for bit.  x: the (T, >= K)
 * bf16 token rows, row stride x_ld elements (x_ld % 8 == 0); each block reads
 * the row of its sorted row's token itself, so no sorted copy is written.
 * w_tiled / s_tiled: the L + 1 experts' weights from lmoe_mxfp4_tile, (N, K)
 * per expert.  T*k <= 1024, m_padded <= 2048, L <= 1023, K % 128 == 0,
 * N % 16 == 0 (N % 32 with SiTU); topk_w bf16 or f32.  flags: 0 or
 * LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS.  No workspace.
 */
int lmoe_dispatch_mxfp4_skinny(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                               int64_t x_ld, int64_t T, int64_t k, int64_t local_start, int64_t L,
                               int64_t m_padded, const uint8_t* w_tiled, const uint8_t* s_tiled, int64_t K,
                               int64_t N, int epilogue, float beta, float beta_lin, int flags,
                               int32_t* group_sizes, uint8_t* valid, int32_t* per_expert_counts,
                               int32_t* padded_token_idx, void* padded_w, int32_t* slot_pos, void* out,
                               void* stream);

/* ---- dense projections on hipBLASLt ------------------------------------------------
 * out (M, N) = x (M, K) @ w_nk^T, w_nk stored (N, K): the layer's plain dense
 * projections (x = hidden @ down_proj, ref.py:634-655; out = normed @ up_proj,
 * ref.py:430) as a library GEMM (ROCm hipBLASLt), f32 accumulation.  x and w
 * share a dtype (bf16 or f32); out bf16 or f32.  Uses only algorithms that
 * need no workspace; the first call per device creates a hipBLASLt handle and
 * the first call per shape a plan, both kept until the process ends.
 */
int lmoe_dense_blaslt(const void* x, int x_dtype, const void* w_nk, int w_dtype, int64_t M, int64_t K, int64_t N,
                      void* out, int out_dtype, void* stream);
/* The same dense projection on this library's own kernel: out (M, N) = x (M, K)
 * @ w_nk^T with bf16 x and bf16 w_nk (N, K), f32 accumulation, out bf16 or f32
 * (the layer's router logits + down-projection, ref.py:620 / ref.py:634-655,
 * and up-projection, ref.py:430).  256 x 128 output tiles on the bf16 MFMA
 * with a direct-to-LDS DMA pipeline; summation order differs from hipBLASLt's.
 * K % 64 == 0, N % 8 == 0, K < 2^23, M, N < 2^31, buffers 16-byte aligned.
 * No workspace.
 */
int lmoe_dense(const void* x, const void* w_nk, int64_t M, int64_t K, int64_t N, void* out, int out_dtype,
               void* stream);
/* The same dense projection for a few rows (a decode step's M = T tokens),
 * on a hand-written skinny kernel: x (M, K) bf16 @ w_nk^T with bf16 w_nk
 * (N, K), f32 accumulation, out bf16 or f32.  Each weight byte is read once
 * per 16/32/64 rows; the K axis is split over a block's waves and summed in a
 * fixed order (repeatable bit for bit, another order than hipBLASLt's).
 * K % 128 == 0, N % 16 == 0, M, K, N < 2^31, pointers 16-byte aligned.  No
 * workspace.
 */
int lmoe_dense_skinny(const void* x, const void* w_nk, int64_t M, int64_t K, int64_t N, void* out, int out_dtype,
                      void* stream);

/* ---- a18: MXFP4 weight preparation ------------------------------------------------
 * One-time weight preparation, the MXFP4 counterpart of prefuse_gateup_weights
 * (rd.py:610-641): k-step-major re-tiling of checkpoint-layout weights,
 * packed (G, N, K/2) -> packed_out (G, K/64, N, 32) and E8M0 scales
 * (G, N, K/32) -> scale_out (G, K/64, N, 2).  Each 32-byte record (one column,
 * 64 k values) holds the checkpoint's eight 4-byte groups in the order
 * 0, 2, 4, 6, 1, 3, 5, 7 (one 16-byte LDS read per MFMA lane and k step).
 * K % 64 == 0; outputs must not alias inputs; packed buffers 16-byte aligned.
 */
int lmoe_mxfp4_tile(const uint8_t* packed, const uint8_t* scale, int64_t G, int64_t N, int64_t K,
                    uint8_t* packed_out, uint8_t* scale_out, void* stream);

/* ---- a18 native: MXFP8 activations x MXFP4 weights on the block-scaled MFMA ----------
 * The reference has no counterpart (its MXFP4 paths dequantise to bf16,
 * odq.py:65-172); this is the native scaled-MFMA path of the north star, with
 * OCP MX semantics: E4M3 activations with one E8M0 scale per 32 along K.
 *
 * lmoe_quantize_mxfp8: x (M, K) bf16/f32 -> q (M, K) E4M3 codes, and scale_t,
 * the E8M0 scales in the k-step-major layout (K/128, roundup(M, 4), 4) of
 * lmoe_mxfp8_scale_bytes(M, K) bytes (pad rows 0).  Shared exponent
 * floor(log2 max|x|) - 8 per block of 32 (finite values; all-zero block -> 0),
 * elements round-to-nearest-even, saturating to +-448, NaN -> 0x7F.  K % 128 == 0.
 *
 * lmoe_ragged_dot_mxfp8_mxfp4: grouped deq(q) @ deq(W_g)^T with weights from
 * lmoe_mxfp4_tile ((G, K/64, N, 32) + (G, K/64, N, 2)); out (M, N) in out_dtype,
 * or (M, N/2) bf16 with LMOE_EPI_SITU (gate/up rounded to bf16 first).  Rows
 * past sum(group_sizes) are written as zero; zero_group as in lmoe_ragged_dot.
 * E8M0 byte 255 is NaN here (OCP MX), unlike dequantize_mxfp4's 2^128.
 */
int64_t lmoe_mxfp8_scale_bytes(int64_t M, int64_t K);
int lmoe_quantize_mxfp8(const void* x, int x_dtype, int64_t M, int64_t K, uint8_t* q, uint8_t* scale_t,
                        void* stream);
int lmoe_ragged_dot_mxfp8_mxfp4(const uint8_t* lhs_q, const uint8_t* lhs_scale_t, const uint8_t* w_packed_t,
                                const uint8_t* w_scale_t, const int32_t* group_sizes, int64_t M, int64_t K,
                                int64_t N, int64_t G, int zero_group, int epilogue, float beta, float beta_lin,
                                void* out, int out_dtype, void* stream);

/* ---- north star (c), FP4/FP6 rate: MXFP6 activations x MXFP4 weights ---------------
 * No counterpart in the reference (its MXFP4 paths dequantise to bf16).  The
 * 32x32x64 block-scaled MFMA runs at the FP4/FP6 rate only with both operands
 * 6 bits or narrower, so activations are quantised to OCP MX FP6 E2M3.
 * lmoe_quantize_mxfp6: x (M, K) bf16/f32 -> q (M, K*3/4) packed E2M3 codes (32
 * codes in 24 little-endian bytes, code j at bits 6j..6j+5; x 16-byte and q
 * 8-byte aligned), scale_t as lmoe_quantize_mxfp8 (lmoe_mxfp8_scale_bytes(M,
 * K) bytes).  Shared exponent floor(log2(max|x|)) - 2 over a block's finite
 * values, clamped to [-127, 127]; elements round to nearest even and
 * saturate to +-7.5; NaN -> +-0.  K % 128 == 0.
 * lmoe_ragged_dot_mxfp6_mxfp4: grouped deq(q) @ deq(W_g)^T with weights from
 * lmoe_mxfp4_tile; out (M, N) bf16 or f32; rows past sum(group_sizes) and of
 * zero_group are zero.  K % 128 == 0, N % 8 == 0; q and weights 16-byte
 * aligned.  The instruction's block dot is accumulated below fp32 precision,
 * as on the MXFP8 path.
 */
int lmoe_quantize_mxfp6(const void* x, int x_dtype, int64_t M, int64_t K, uint8_t* q, uint8_t* scale_t,
                        void* stream);
int lmoe_ragged_dot_mxfp6_mxfp4(const uint8_t* lhs_q, const uint8_t* lhs_scale_t, const uint8_t* w_packed_t,
                                const uint8_t* w_scale_t, const int32_t* group_sizes, int64_t M, int64_t K,
                                int64_t N, int64_t G, int zero_group, void* out, int out_dtype, void* stream);

/* ---- a3: router top-k --------------------------------------------------------------
 * Replaces the gate math of _router_gate (ref.py:601-631) / latent_moe_forward
 * step 1 (ref.py:347-361) given f32 logits (T, E): scores = act(logits);
 * idx = top_k(scores + bias) (descending, ties -> lower index); w = scores[idx];
 * renormalise when renorm != 0 and k > 1; w *= scale; w stored as
 * weight_dtype.  bias may be NULL (zeros).  scores_out (T, E) f32 is optional.
 * E <= 4096, k <= 64, k <= E.
 */
int lmoe_router_topk(const float* logits, const float* bias, int64_t T, int64_t E, int64_t k,
                     int act, int renorm, float scale, int weight_dtype, int32_t* topk_idx,
                     void* topk_w, float* scores_out, void* stream);
/* Same with the logits rows ld >= E floats apart (e.g. the router columns of
 * a GEMM that computes the router logits together with another projection of
 * the same hidden states). */
int lmoe_router_topk_ld(const float* logits, int64_t ld, const float* bias, int64_t T, int64_t E,
                        int64_t k, int act, int renorm, float scale, int weight_dtype,
                        int32_t* topk_idx, void* topk_w, float* scores_out, void* stream);
/* router_and_projection (ref.py:634-655) given the GEMM that computes the
 * router logits and the latent projection x = h @ down_proj together (f32
 * rows of ld floats: logits at columns [0, E), x at x_src = logits + E or any
 * rows of x_ld floats): lmoe_router_topk_ld's (topk_idx, topk_w) and x as bf16
 * (T, lat), rounded to nearest even -- the projection's output dtype -- by the
 * same launch.  lat <= 1024, lat % 4 == 0, x_ld % 4 == 0, x_src 16-byte and
 * x_out 8-byte aligned. */
int lmoe_router_topk_proj(const float* logits, int64_t ld, const float* bias, int64_t T, int64_t E,
                          int64_t k, int act, int renorm, float scale, int weight_dtype,
                          int32_t* topk_idx, void* topk_w, const float* x_src, int64_t x_ld,
                          int64_t lat, uint16_t* x_out, void* stream);

/* ---- a7: local-shard dispatch ------------------------------------------------------
 * Replaces filter_and_pad_to_shard_jittable (ref.py:754-877), bit-identical to
 * the eager filter_and_pad_to_shard (ref.py:658-751): slots whose expert is in
 * [local_start, local_start + L) are stable-sorted by local id, truncated to
 * m_padded, and the x rows gathered.  Outputs (all device):
 *   sorted_tokens (m_padded, lat) x_dtype, zero on padding rows
 *   group_sizes (L+1,) int32 [counts..., m_padded - sum]
 *   valid (m_padded,) u8, per_expert_counts (L,) int32
 *   padded_token_idx (m_padded,) int32 (-1 on padding), padded_w (m_padded,) w_dtype
 *   slot_pos (T*k,) int32 or NULL: sorted row of each (token, slot), -1 if not kept
 * T, k, T*k and m_padded < 2^31, L + 1 <= 12288, local_start + L < 2^31.
 * m_padded == 0 allows a NULL sorted_tokens; the other outputs must still be
 * non-NULL (a caller with no slots to keep can form the result itself: zero
 * group sizes and counts, every slot_pos -1).
 * Workspace: lmoe_dispatch_workspace_size(T, k, L) bytes, no initialisation needed
 * (-1 for sizes the dispatch refuses).
 */
int64_t lmoe_dispatch_workspace_size(int64_t T, int64_t k, int64_t L);
int lmoe_dispatch_local(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                        int x_dtype, int64_t T, int64_t k, int64_t lat, int64_t local_start,
                        int64_t L, int64_t m_padded, void* sorted_tokens, int32_t* group_sizes,
                        uint8_t* valid, int32_t* per_expert_counts, int32_t* padded_token_idx,
                        void* padded_w, int32_t* slot_pos, void* workspace,
                        int64_t workspace_size, void* stream);

/* lmoe_dispatch_local without a workspace argument: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * counting sort's workspace is a 4 MiB static device array (one per GPU, held
 * until the process ends), so lmoe_dispatch_workspace_size(T, k, L) must not
 * exceed 4 MiB (e.g. T*k = 65536 slots with L <= 4095): larger sizes return
 * LMOE_ERR_WORKSPACE without launching anything.  Outputs and semantics are
 * those of lmoe_dispatch_local, bit for bit.  Every call on one GPU uses the
 * same array: calls that overlap on one GPU (concurrent streams, host
 * threads) race; calls ordered on one stream do not.  Allocates nothing.
 */
int lmoe_dispatch_local_noalloc(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                                int x_dtype, int64_t T, int64_t k, int64_t lat, int64_t local_start,
                                int64_t L, int64_t m_padded, void* sorted_tokens, int32_t* group_sizes,
                                uint8_t* valid, int32_t* per_expert_counts, int32_t* padded_token_idx,
                                void* padded_w, int32_t* slot_pos, void* stream);

/* The same dispatch in one launch for decode-sized batches (T*k <= 8192,
 * m_padded <= 8192, L < 1024): every output as lmoe_dispatch_local, bit for
 * bit, except that x may be a row-strided (row stride x_ld elements) bf16 or
 * f32 array and sorted_tokens is bf16 (f32 rounded to nearest even, the same
 * rounding as lmoe_cast_rows).  lat % 8 == 0, x rows and sorted_tokens
 * 16-byte aligned.  With LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS the padding rows
 * of sorted_tokens (from sum(group_sizes[:L]) on) are left unwritten, for
 * callers that never read them.  No workspace.
 */
#define LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS 0x1
/* lmoe_dispatch_local_rows only: write every output but sorted_tokens (x and
 * sorted_tokens may be null), for callers whose expert GEMM gathers the token
 * rows itself (lmoe_ragged_dot_mxfp4_rows); the counting-sort path at every size. */
#define LMOE_DISPATCH_FLAG_NO_ROWS 0x2
int lmoe_dispatch_local_small(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                              int x_dtype, int64_t x_ld, int64_t T, int64_t k, int64_t lat,
                              int64_t local_start, int64_t L, int64_t m_padded, uint16_t* sorted_tokens,
                              int32_t* group_sizes, uint8_t* valid, int32_t* per_expert_counts,
                              int32_t* padded_token_idx, void* padded_w, int32_t* slot_pos, int flags,
                              void* stream);
/* The same contract as lmoe_dispatch_local_small (row-strided bf16 or f32 x,
 * bf16 sorted_tokens, optional skip of the padding rows) at any size: the
 * one-launch kernel when T*k, m_padded and L fit it, else the counting sort of
 * lmoe_dispatch_local and a gather that rounds f32 rows to bf16.  Workspace:
 * lmoe_dispatch_workspace_size(T, k, L) bytes (unused on the one-launch path).
 */
int lmoe_dispatch_local_rows(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x, int x_dtype,
                             int64_t x_ld, int64_t T, int64_t k, int64_t lat, int64_t local_start, int64_t L,
                             int64_t m_padded, uint16_t* sorted_tokens, int32_t* group_sizes, uint8_t* valid,
                             int32_t* per_expert_counts, int32_t* padded_token_idx, void* padded_w,
                             int32_t* slot_pos, int flags, void* workspace, int64_t workspace_size, void* stream);

/* ---- a13: combine -----------------------------------------------------------------
 * lmoe_combine_scatter_add replaces _combine_shard_contribution (ref.py:1113-1141):
 * routed_out.at[idx].add((shard_out * w[:, None]).astype(routed_out.dtype)),
 * in place on routed_out (T, lat).  Deterministic: each token's rows are added
 * in ascending row order, each add rounded to out_dtype (the scatter order of
 * the reference).  idx -1 rows (padding, weight 0) are skipped, other indices
 * outside [0, T) are dropped.  Workspace: lmoe_combine_workspace_size(m, T)
 * (-1 for sizes the combine refuses).
 *
 * lmoe_combine_slots is the same combine driven by the dispatch's slot_pos
 * (no sort needed): mode LMOE_COMBINE_SCATTER_ADD reproduces
 * _combine_shard_contribution (weights padded_w[row]); mode
 * LMOE_COMBINE_SLOT_SUM reproduces the unsharded f32 weighted sum of
 * ref.py:413-416 (weights topk_w[t, j], f32), writing routed_out.  With
 * T > 0, shard_out holds at least one row (slots that were not kept re-read
 * row 0, whose value they do not use; a dispatch's m_padded is at least one
 * tile).  The same holds for lmoe_combine_slots_rms_norm.
 */
int64_t lmoe_combine_workspace_size(int64_t m, int64_t T);
int lmoe_combine_scatter_add(const void* shard_out, int shard_dtype, const int32_t* padded_token_idx,
                             const void* padded_w, int w_dtype, int64_t m, int64_t lat, int64_t T,
                             void* routed_out, int out_dtype, void* workspace,
                             int64_t workspace_size, void* stream);
int lmoe_combine_slots(const void* shard_out, int shard_dtype, const int32_t* slot_pos,
                       const void* w, int w_dtype, int64_t T, int64_t k, int64_t lat, int mode,
                       void* routed_out, int out_dtype, void* stream);
/* lmoe_combine_slots into a zero routed_out, fused with lmoe_rms_norm of the
 * routed rows (the layer's combine -> _rms_norm, ref.py:413-427 /
 * ref.py:1113-1141 + 286-293): normed_out (T, lat) = rms_norm(routed) * scale.
 * routed_out (T, lat) is also written when not NULL.  Bit-identical to the
 * two calls.  dtype is the routed / normed / scale dtype; lat % 8 == 0,
 * lat <= 2048; bf16 buffers 16-byte aligned, f32 32-byte aligned. */
int lmoe_combine_slots_rms_norm(const void* shard_out, int shard_dtype, const int32_t* slot_pos,
                                const void* w, int w_dtype, int64_t T, int64_t k, int64_t lat, int mode,
                                const void* norm_scale, float eps, void* routed_out, void* normed_out,
                                int dtype, void* stream);

/* ---- a14 / a10: adjacent elementwise stages -----------------------------------------
 * lmoe_rms_norm: _rms_norm (ref.py:286-293): f32 mean square, x*rsqrt(var+eps)
 *   cast to dtype, then * scale in dtype.  x, out (rows, n); scale (n,).
 * lmoe_situ_and_mul: _situ_and_mul (ref.py:296-310) on separate gate/up (rows, n).
 * lmoe_add: out = cast(a + b) elementwise (the residual add of ref.py:435).
 */
int lmoe_rms_norm(const void* x, const void* scale, int64_t rows, int64_t n, float eps, int dtype,
                  void* out, void* stream);
int lmoe_situ_and_mul(const void* gate, const void* up, int64_t count, float beta, float beta_lin,
                      int dtype, void* out, void* stream);
int lmoe_add(const void* a, const void* b, int64_t count, int dtype, void* out, void* stream);
/* lmoe_cast_rows: out (rows, cols) contiguous = cast(x), x rows ld >= cols
 * elements apart; f32 -> bf16 rounds to nearest even (the rounding of a bf16
 * matmul output).  Used to split the layer's fused router + down-projection
 * GEMM (f32 out) into the f32 logits and the bf16 latent x (ref.py:358/371). */
int lmoe_cast_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld, void* out,
                   int out_dtype, void* stream);
/* lmoe_transpose: out (G, C, R) = in (G, R, C) transposed per batch, 2- or
 * 4-byte elements, out not aliasing in.  Turns the reference's (G, K, N)
 * ragged_dot weights (rd.py:358-369) into the k-contiguous (G, N, K) layout
 * the fast grouped GEMM kernels read. */
int lmoe_transpose(const void* in, int64_t G, int64_t R, int64_t C, int elem_bytes, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LMOE_H_ */
