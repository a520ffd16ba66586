/*
 * q3hip.h -- C ABI of libq3hip.so, the MI355X (gfx950) kernels behind the Qwen3 decoder
 * operator set.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts/shapes as int64_t, and the hipStream_t to
 *     launch on (the caller's current stream; NULL = legacy default stream);
 *   - never allocates device memory: outputs and workspaces are owned by the caller, and a
 *     `*_workspace_bytes` query states the size of any workspace;
 *   - returns 0 on success, a hipError_t value if a launch failed, or Q3_ERR_INVALID if the
 *     arguments were rejected before any launch (see q3_error_string).
 * Tensors are dense row-major unless a stride argument says otherwise.  `dtype` is one of
 * Q3_F32 / Q3_F16 / Q3_BF16 and applies to every floating tensor of the call unless noted.
 *
 * "Replaces" comments cite the reference entry (wuyii8941/qwen3-triton, file:line) whose
 * Triton launch(es) the function stands in for.
 */
#ifndef Q3HIP_H
#define Q3HIP_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3_OK 0
#define Q3_ERR_INVALID 100000 /* arguments rejected before launch */
#define Q3_ERR_SCRATCH 100001 /* request larger than a no-allocation entry point's fixed scratch */

enum { Q3_F32 = 0, Q3_F16 = 1, Q3_BF16 = 2 };

/* Human-readable text for a return code. */
const char* q3_error_string(int code);
/* ABI version of this header; bumped on any signature change. */
int q3_abi_version(void);

/* ------------------------------------------------------------------ RMSNorm
 * y[r,:] = x[r,:] * rsqrt(mean(x[r,:]^2) + eps) * w, fp32 internally, one rounding.
 * Replaces: qwen3_triton/kernels/norm.py:7-13 (_forward), kernels/math_precision.py:15-37,
 *           ops/triton/rms_norm.py:11-31,62-88; inference/kernels.py:176-185 (rms_norm). */
int q3_rmsnorm_fwd(int dtype, const void* x, const void* w, void* y, int64_t rows, int64_t h, float eps,
                   hipStream_t stream);
/* dx = (g*w - x*inv^2*mean(g*w*x))*inv ; dw = sum_rows g*x*inv (deterministic two-level sum).
 * Replaces: kernels/norm.py:16-37,53-63 (_backward + _reduce_rows), ops/triton/rms_norm.py:33-59,90-116. */
size_t q3_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t h);
int q3_rmsnorm_bwd(int dtype, const void* x, const void* w, const void* dy, void* dx, void* dw, void* workspace,
                   int64_t rows, int64_t h, float eps, hipStream_t stream);
/* dx = dres + (the RMSNorm input gradient), the backward of a residual block's input x that feeds
 * both the residual sum and the norm (y = x + f(norm(x))): the two gradients of x are summed in
 * the same pass instead of by a separate add.  dres [rows, h], same dtype; dw and the workspace as
 * q3_rmsnorm_bwd.  The norm's gradient is rounded to the storage type before the sum, as the
 * separate add would see it.
 * Replaces: kernels/norm.py:39-66 (_RMSNorm.backward) + kernels/residual.py:13-30 (_Residual.backward),
 *           whose two gradients of x the reference sums in autograd. */
int q3_rmsnorm_bwd_add(int dtype, const void* x, const void* w, const void* dy, const void* dres, void* dx, void* dw,
                       void* workspace, int64_t rows, int64_t h, float eps, hipStream_t stream);

/* ------------------------------------------------------------------ fused per-head RMSNorm + RoPE
 * x: [tokens, heads, d] (rows = tokens*heads); cos/sin: [tokens, d]; w: [d].
 * y = rope(rmsnorm(x)) with split-half rotation.
 * Replaces: kernels/norm_rope.py:12-28,53-71 (_norm_rope_forward), kernels/math_precision.py:39-64,
 *           ops/triton/fused_qk_norm_rope.py:11-66 (per tensor), inference/kernels.py:188-194. */
int q3_norm_rope_fwd(int dtype, const void* x, const void* w, const void* cos, const void* sin, void* y,
                     int64_t tokens, int64_t heads, int64_t d, float eps, hipStream_t stream);
/* Backward: inverse rotation, then RMSNorm backward; dw reduced deterministically.
 * Replaces: kernels/norm_rope.py:30-50,62-69, ops/triton/fused_qk_norm_rope.py:111-235. */
size_t q3_norm_rope_bwd_workspace_bytes(int64_t tokens, int64_t heads, int64_t d);
int q3_norm_rope_bwd(int dtype, const void* x, const void* w, const void* cos, const void* sin, const void* dy,
                     void* dx, void* dw, void* workspace, int64_t tokens, int64_t heads, int64_t d, float eps,
                     hipStream_t stream);
/* The query and key tensors of one layer in one launch per direction (same per-row arithmetic, so
 * yq / yk and dxq / dxk are bit-identical to two q3_norm_rope_fwd / _bwd calls): q [tokens, hq, d]
 * with weight wq, k [tokens, hk, d] with wk, shared cos/sin [tokens, d].  dw is [2, d]: dW_q, then
 * dW_k (deterministic; the fp32 summation order differs from the single-tensor call).  Vector path
 * only (d / 2 a multiple of 8 for 16-bit types, 4 for fp32, d / vector width in {8, 16, 32}); other
 * shapes return Q3_ERR_INVALID.
 * Replaces: ops/triton/fused_qk_norm_rope.py:237-273 (_FusedQKNormRoPEFunction, one launch per
 *           tensor there), its forward _fused_one (:68-109) and backward _fused_backward_one
 *           (:191-235) for the pair. */
int q3_norm_rope_qk_fwd(int dtype, const void* q, const void* k, const void* wq, const void* wk, const void* cos,
                        const void* sin, void* yq, void* yk, int64_t tokens, int64_t hq, int64_t hk, int64_t d,
                        float eps, hipStream_t stream);
/* Prefill form of q3_norm_rope_qk_fwd: q / k / v [B, S, h, d] (contiguous), yq [B, S, hq, d] as
 * there; the normed + rotated keys and the unchanged values are written straight into the
 * [B, hk, capacity, d] caches at positions start .. start + S - 1 (start + S <= capacity), so the
 * whole Q/K-norm + RoPE + cache append of a prefill chunk is one launch.  Bit-identical to
 * q3_norm_rope_qk_fwd followed by q3_kv_append.
 * Replaces: inference/model.py:122-124 (norm_rope on q and k, kernels.append). */
int q3_norm_rope_qk_cache_fwd(int dtype, const void* q, const void* k, const void* v, const void* wq, const void* wk,
                              const void* cos, const void* sin, void* yq, void* cache_k, void* cache_v, int64_t B,
                              int64_t S, int64_t hq, int64_t hk, int64_t d, int64_t capacity, int64_t start, float eps,
                              hipStream_t stream);
size_t q3_norm_rope_qk_bwd_workspace_bytes(int64_t tokens, int64_t hq, int64_t hk, int64_t d);
int q3_norm_rope_qk_bwd(int dtype, const void* q, const void* k, const void* wq, const void* wk, const void* cos,
                        const void* sin, const void* dyq, const void* dyk, void* dxq, void* dxk, void* dw,
                        void* workspace, int64_t tokens, int64_t hq, int64_t hk, int64_t d, float eps,
                        hipStream_t stream);

/* ------------------------------------------------------------------ RoPE
 * cos/sin[t, j] = cos/sin(fp32(pos[t]) * inv_freq[j mod d/2]) for j < d, stored in `dtype`.
 * Replaces: kernels/rotary.py:12-17,36-45 (_tables / rotary_tables). */
int q3_rope_tables(int dtype, const void* pos, int pos_is_int64, const float* inv_freq, void* cos, void* sin,
                   int64_t n_pos, int64_t d, hipStream_t stream);
/* y = x*cos + rotate_half(x)*sin (backward=0) or its transpose (backward=1).
 * layout 0: x is [B,S,H,D] (kernels/rotary.py:19-34,47-66); layout 1: x is [B,H,S,D]
 * (ops/triton/rope.py:11-148).  cos/sin: [B,S,D]. */
int q3_rope_apply(int dtype, const void* x, const void* cos, const void* sin, void* y, int64_t batch, int64_t seq,
                  int64_t heads, int64_t d, int layout, int backward, hipStream_t stream);

/* ------------------------------------------------------------------ SwiGLU
 * y = silu(g)*u ; backward dg = dy*u*s*(1+g*(1-s)), du = dy*silu(g), s = sigmoid(g).
 * Replaces: kernels/activation.py:6-36, kernels/math_precision.py:66-96, ops/triton/silu_and_mul.py:20-121. */
int q3_swiglu_fwd(int dtype, const void* g, const void* u, void* y, int64_t n, hipStream_t stream);
int q3_swiglu_bwd(int dtype, const void* g, const void* u, const void* dy, void* dg, void* du, int64_t n,
                  hipStream_t stream);

/* SwiGLU backward on [rows, cols] blocks at their own row strides (gate and up halves of one
 * [rows, 2*cols] buffer, as the reference's silu_and_mul input).  Same math as q3_swiglu_bwd.
 * Replaces: ops/triton/silu_and_mul.py:20-121 (strided [..., 2d] form), kernels/mlp_precision.py:36-48. */
int q3_swiglu_bwd_2d(int dtype, const void* g, int64_t ldg, const void* u, int64_t ldu, const void* dy, int64_t lddy,
                     void* dg, int64_t lddg, void* du, int64_t lddu, int64_t rows, int64_t cols, hipStream_t stream);

/* ------------------------------------------------------------------ elementwise / data movement */
/* y[r * ldy + c] = x[r * ldx + c] for r < rows, c < cols (bit copy between strided blocks).
 * No counterpart in the reference (it concatenates with torch); used to pack gradients side by side. */
int q3_copy2d(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols,
              hipStream_t stream);
/* y[c * ldy + r] = x[r * ldx + c] for r < rows, c < cols; writes nothing else (so it can fill a column
 * block of a wider matrix).  Replaces: the .t().contiguous() operand copies of kernels/linear.py:45-105. */
int q3_transpose2d(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols,
                   hipStream_t stream);
/* c = a + b (fp32 add).  Replaces kernels/residual.py:6-30. */
int q3_add(int dtype, const void* a, const void* b, void* c, int64_t n, hipStream_t stream);
/* y = convert(x).  Replaces kernels/attention.py:11-20 (cast_tensor). */
int q3_cast(int src_dtype, int dst_dtype, const void* x, void* y, int64_t n, hipStream_t stream);
/* x[:] = value (a kernel, never a memset, so it is safe inside captured graphs). */
int q3_fill(int dtype, void* x, float value, int64_t n, hipStream_t stream);
/* out[b, s] = start + s (+ *start_dev when non-NULL).  Replaces _model.py:29-32 (_positions),
 * inference/kernels.py:12-21. */
int q3_positions(int64_t* out, int64_t batch, int64_t seq, int64_t start, const int64_t* start_dev,
                 hipStream_t stream);
/* y[b][c][r] = x[b][r][c] for 16-bit or 32-bit elements (a layout change, not arithmetic); output rows
 * have stride ldy >= rows and the pad [rows, ldy) is zero-filled. */
int q3_transpose(int dtype, const void* x, void* y, int64_t batch, int64_t rows, int64_t cols, int64_t ldy,
                 hipStream_t stream);

/* ------------------------------------------------------------------ embedding
 * y[i,:] = w[ids[i],:].  Out-of-range ids produce zero rows and set *bad_ids (device int) to 1.
 * Replaces: kernels/embedding.py:12-26,49-64. */
int q3_embedding_fwd(int dtype, const void* ids, int ids_is_int64, const void* w, void* y, int* bad_ids,
                     int64_t n_ids, int64_t vocab, int64_t h, hipStream_t stream);
/* dw = scatter-sum of dy rows by id, deterministic (fixed summation order per token, no atomics).
 * dw is fully written (rows of unused tokens are zero).  Replaces kernels/embedding.py:29-46,66-77. */
size_t q3_embedding_bwd_workspace_bytes(int64_t n_ids);
int q3_embedding_bwd(int dtype, const void* ids, int ids_is_int64, const void* dy, void* dw, void* workspace,
                     int64_t n_ids, int64_t vocab, int64_t h, hipStream_t stream);


/* ------------------------------------------------------------------ GEMM
 * C[M,N] = alpha * A[M,K] . B[N,K]^T (+ C when accumulate != 0); A, B bf16/fp16 with K-contiguous
 * rows (strides lda, ldb elements; K, lda, ldb multiples of 8; 16-byte aligned bases); C in
 * out_dtype with row stride ldc; fp32 accumulation on the matrix cores.
 * Replaces: kernels/linear.py:13-42,45-77 (_gemm / matmul), kernels/gemm_experiments.py:12-101,
 *           ops/triton/gate_up_swiglu.py:151-176 (_matmul_kernel). */
int q3_gemm_nt(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
               int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int accumulate, hipStream_t stream);
/* Projection plus residual in one matrix-core GEMM: C = R + A B^T for A [M, K], B [N, K] (K-contiguous
 * rows) and the residual R [M, N] (row stride ldr); the GEMM output is rounded to dtype and then
 * added to R in fp32 and rounded again, so C is bit-identical to q3_gemm_nt followed by q3_add.
 * C may alias R.  M % 128 == 0, N % 128 == 0, K % 64 == 0 (256 x 256 tiles when M and N are multiples of
 * 256 and that grid has at least 192 tiles, else 128 x 128, as q3_gemm_nt plans them), strides % 8 == 0,
 * pointers 16-byte aligned.
 * Replaces: _model.py:60-108 / components.py (x = x + self_attn(...), x = x + mlp(...): the o_proj /
 * down_proj kernels/linear.py launch followed by kernels/residual.py:13-30). */
int q3_gemm_nt_residual(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                        int64_t ldr, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream);
/* q3_gemm_nt_residual with a caller workspace of q3_gemm_nt_residual_workspace_bytes(M, N, K) bytes
 * (16-byte aligned).  When that size is nonzero -- M, N multiples of 256 whose 256 x 256 grid has 96 to 128
 * tiles, i.e. would occupy at most half of the CUs, and K % 128 == 0 with K / 2 >= 4096, e.g. the
 * 2048-token prefill's down projection -- the GEMM runs as two K halves on 256 x 256 tiles into
 * fp32 partials in the workspace, and one pass forms C = R + (P0 + P1) with the same two roundings
 * (the product rounded, then the residual added and rounded): within the rounding of the unsplit
 * launch, not bit-identical to it.  With a null workspace, or a zero size, it is q3_gemm_nt_residual.
 * Replaces: the same reference launches as q3_gemm_nt_residual. */
size_t q3_gemm_nt_residual_workspace_bytes(int64_t M, int64_t N, int64_t K);
int q3_gemm_nt_residual_ws(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                           int64_t ldr, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);
/* q3_gemm_nt_residual_ws that also writes Y = RMSNorm(C) with weight norm_w [N] and eps (the norm of the
 * next block's input: Y = C rsqrt(mean(C^2) + eps) norm_w from the rounded C, q3_rmsnorm_fwd's
 * expression, row stride ldy), N <= 8192.  On the two-K-halves plan the combining pass forms both
 * (one row per workgroup: C is never re-read); otherwise the residual GEMM runs, then
 * q3_rmsnorm_fwd (contiguous C and Y required there).
 * Replaces: the o_proj / down_proj launch + residual add of components.py / _model.py followed by
 * the next RMSNorm (kernels/norm.py:39-66, inference/kernels.py:176). */
int q3_gemm_nt_residual_norm_ws(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                                int64_t ldr, void* C, int64_t ldc, const void* norm_w, float eps, void* Y,
                                int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);
/* Gate/up projections with the SwiGLU epilogue in one matrix-core GEMM: for x [M, K] and weights
 * wg, wu [N, K] (K-contiguous rows, row stride ldw), stores G = x wg^T, U = x wu^T (each rounded to
 * dtype) and Y = silu(G) * U computed from the rounded G and U (the same expression as
 * q3_swiglu_fwd on the stored G, U), all [M, N] at row stride ldo.  One launch reads x and both
 * weights once per tile.  g and u may both be null (inference: Y only, the same values).  M % 256 == 0,
 * N % 128 == 0, K % 64 == 0, ldo % 8 == 0; every pointer 16-byte aligned.
 * Replaces: kernels/mlp_precision.py:16-33 / kernels/mlp.py:14-33 (_gate_up: both K loops and the
 * G, U, Y stores in one kernel), ops/triton/gate_up_swiglu.py:178-288. */
int q3_gemm_gate_up_swiglu(int dtype, const void* x, int64_t ldx, const void* wg, const void* wu, int64_t ldw,
                           void* g, void* u, void* y, int64_t ldo, int64_t M, int64_t N, int64_t K,
                           hipStream_t stream);
/* q3_gemm_gate_up_swiglu that also stores Y^T [N, M] (row stride ldyt % 8 == 0, ldyt >= M) from the
 * same epilogue: the operand the down projection's weight-gradient GEMM reads, so the backward needs no
 * transpose pass over Y.  G, U, Y as q3_gemm_gate_up_swiglu (bit-identical); Y^T holds the same values.
 * Replaces: kernels/mlp_precision.py:16-33 (the forward that feeds the block's backward; the
 * reference's backward reads Y through a strided operand). */
int q3_gemm_gate_up_swiglu_t(int dtype, const void* x, int64_t ldx, const void* wg, const void* wu, int64_t ldw,
                             void* g, void* u, void* y, int64_t ldo, void* yt, int64_t ldyt, int64_t M, int64_t N,
                             int64_t K, hipStream_t stream);
/* Down-projection input gradient with the SwiGLU backward in its epilogue: dY = dy wt^T for
 * dy [M, K] and wt [N, K] (the transposed down weight: K-contiguous rows), rounded to dtype as a
 * standalone GEMM output, then dg = dY u s (1 + g (1 - s)), du = dY g s with s = sigmoid(g) for
 * the saved SwiGLU inputs g, u [M, N] (row stride ldgu) -- the q3_swiglu_bwd formula, so the result
 * is bit-identical to q3_gemm_nt + q3_swiglu_bwd.  Stores dg, du [M, N] at row stride ldd and, when
 * dgt / dut are non-null, their transposes [N, M] at row stride lddt (the operands of the gate/up
 * weight-gradient GEMM), so dY never reaches memory and no separate transpose pass runs.
 * M % 256 == 0, N % 256 == 0, K % 64 == 0, strides % 8 == 0, pointers 16-byte aligned.
 * Replaces: kernels/mlp_precision.py:36-63 (_GateUp.backward: the down-projection dX GEMM of
 * kernels/linear.py:92-100 followed by the SwiGLU backward of kernels/activation.py:22-36). */
int q3_gemm_swiglu_bwd(int dtype, const void* dy, int64_t lddy, const void* wt, int64_t ldw, const void* g,
                       const void* u, int64_t ldgu, void* dg, void* du, int64_t ldd, void* dgt, void* dut,
                       int64_t lddt, int64_t M, int64_t N, int64_t K, hipStream_t stream);
/* Several projections of one input in one matrix-core launch: for A [M, K] and nseg (1..3) weights
 * Bs[s] [Ns[s], K] (common row stride ldb), writes Cs[s] = A Bs[s]^T ([M, Ns[s]] at row stride
 * ldcs[s]), fp32 accumulation, one rounding, bit-identical to nseg separate q3_gemm_nt calls with
 * the same tile plan.  M % 128 == 0, every Ns[s] % 128 == 0, K % 64 == 0, ldcs[s] % 8 == 0,
 * pointers 16-byte aligned; 256 x 256 tiles when M and every Ns[s] are multiples of 256 and that grid
 * has at least 192 tiles, else 128 x 128.  The K and V projections of Qwen3-8B (N = 1024) alone fill
 * only part of the 256 CUs; side by side with Q they share one well-filled grid.
 * Replaces: components.py:19-21 / _model.py (q_proj, k_proj, v_proj: three kernels/linear.py
 * launches on the same input). */
int q3_gemm_nt_multi(int dtype, const void* A, int64_t lda, int nseg, const void* const* Bs, int64_t ldb,
                     void* const* Cs, const int64_t* Ns, const int64_t* ldcs, int64_t M, int64_t K,
                     hipStream_t stream);
/* Same product for arbitrary element strides: A(m,k) = A[m*sam + k*sak], B(k,n) = B[k*sbk + n*sbn];
 * any dtype (fp32 included).  SIMT path for shapes the matrix-core kernel does not take.
 * Replaces: kernels/linear.py:13-42 (_gemm with arbitrary strides). */
int q3_gemm_strided(int in_dtype, int out_dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                    int64_t sbn, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int accumulate,
                    hipStream_t stream);

/* ------------------------------------------------------------------ causal GQA flash attention
 * Q/O/dO/dQ are [B,Hq,Lq,D] and K/V/dK/dV [B,Hkv,Lk,D] with D contiguous and element strides
 * (qsb, qsh, qss) resp. (ksb, ksh, kss) for batch, head and position (so [B,S,H,D] and cache
 * layouts are taken in place).  Lk >= Lq; query i attends keys j <= i + (Lk - Lq); query head h
 * uses KV head h/(Hq/Hkv).  LSE and delta are [B,Hq,Lq] fp32 (natural-log LSE; delta =
 * rowsum(O*dO) is backward scratch).  On the matrix-core path (q3_attention_mfma_supported) the
 * caller also passes sequence-major copies [B,H,D,ld] (ld >= L, ld % 16 == 0, zero pad) made by
 * q3_attention_seq_major: vt of V (forward), qt of Q, kt of K and dot of dO (backward; at head_dim
 * 128 only kt is read -- Q and dO are read transposed in LDS -- and qt / dot may be null), and every
 * row must be 16-byte aligned.  Within every 16-position block of such a row the positions are
 * stored in the order 0-3, 8-11, 4-7, 12-15 (the operand order of the matrix-core kernels).
 * Other dtypes/head sizes run a SIMT path that ignores them.
 * Replaces: kernels/attention.py:20-50 + attention_kernels.py:9-253 (_attention_forward_kernel,
 *           _attention_delta_kernel, _attention_dq_kernel, _attention_dkdv_fused_kernel,
 *           _attention_kv_head_reduce_kernel), kernels/attention_precision.py:14-182,
 *           ops/triton/attention.py:29-292, ops/triton/attention_backward.py:21-236,
 *           inference/kernels.py:38-68 (_inference_cached_attention, prefill against the cache). */
int q3_attention_mfma_supported(int dtype, int64_t d);
int q3_attention_seq_major(int dtype, const void* x, int64_t sb, int64_t sh, int64_t ss, void* y, int64_t ldy,
                           int64_t B, int64_t H, int64_t L, int64_t D, hipStream_t stream);
int q3_attention_fwd(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k, const void* v,
                     int64_t ksb, int64_t ksh, int64_t kss, const void* vt, int64_t ldvt, void* o, float* lse,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D, float scale,
                     hipStream_t stream);
int q3_attention_bwd(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k, const void* v,
                     int64_t ksb, int64_t ksh, int64_t kss, const void* o, const void* dout, const float* lse,
                     const void* qt, int64_t ldqt, const void* kt, int64_t ldkt, const void* dot, float* delta,
                     void* dq, void* dk, void* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk,
                     int64_t D, float scale, hipStream_t stream);

/* ------------------------------------------------------------------ causal cross-entropy
 * Rows r = b*S + s of logits z (row stride ld).  tgt[r] = labels[b, s+1] for s < S-1, else
 * ignore_index (q3_ce_shift_labels).  For a vocabulary chunk z[:, 0:n] holding columns
 * [col0, col0+n) of the full logits, q3_ce_chunk_stats writes the row max m and sum exp(z - m) and,
 * where the target lies in the chunk, its logit into pick.  q3_ce_finish merges nchunks chunk-major
 * partials ([nchunks][rows]) into lse[r], per-row loss lse - z_target (0 when ignored), and
 * loss = sum / count over valid rows (fixed summation order); *bad is set to 1 for a target outside
 * [0, vocab) that is not ignore_index.  q3_ce_chunk_grad writes
 * dz = (exp(z - lse) - onehot(target - col0)) * (*up) / (*count) (0 for ignored rows) in out_dtype.
 * Replaces: kernels/loss.py:6-44,46-71 (_partials, _rows, _mean, _backward, _CausalCE); together with
 * q3_gemm_nt it is the fused LM-head + CE (no reference function; composes kernels/linear.py and
 * kernels/loss.py). */
int q3_ce_shift_labels(const int64_t* labels, int64_t* tgt, int64_t batch, int64_t seq, int64_t ignore_index,
                       hipStream_t stream);
int q3_ce_chunk_stats(int dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                      float* m_out, float* s_out, float* pick, int64_t rows, hipStream_t stream);
int q3_ce_finish(const float* m_part, const float* s_part, int nchunks, const float* pick, const int64_t* tgt,
                 float* lse, float* loss_rows, int* bad, float* loss, float* count, int64_t rows, int64_t vocab,
                 int64_t ignore_index, hipStream_t stream);
int q3_ce_chunk_grad(int dtype, int out_dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                     const float* lse, const float* count, const float* up, void* dz, int64_t ldo, int64_t rows,
                     int64_t vocab, int64_t ignore_index, hipStream_t stream);
/* q3_ce_chunk_grad for 16-bit logits with the transposed copy the weight gradient needs:
 * dz[r, c] (row stride ldo, out type = dtype; dz may be z itself with ldo == ld) and
 * dzt[c * lddzt + r] = dz[r, c] for the chunk's n columns (n and rows multiples of 8, 16-byte aligned
 * buffers, strides multiples of 8).  The backward of the fused LM-head + CE when the forward stored
 * the chunk's bf16 logits (q3_gemm_nt_ce_stats_store): dz comes from the stored logits, with no second
 * logits GEMM.
 * Replaces: kernels/loss.py:34-44,64-68 (_backward) on the reference's bf16 logits. */
int q3_ce_chunk_grad_t(int dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                       const float* lse, const float* count, const float* up, void* dz, int64_t ldo, void* dzt,
                       int64_t lddzt, int64_t rows, int64_t vocab, int64_t ignore_index, hipStream_t stream);
/* The logits GEMM and q3_ce_chunk_grad in one kernel: z = A . B^T (A [M, K] token rows, B [N, K] the
 * chunk's vocabulary rows starting at column col0; K % 64 == 0, 16-byte aligned K-contiguous rows) is
 * formed in fp32 on the matrix cores and only dz (dtype, row stride lddz) is written, with the same
 * expression as q3_ce_chunk_grad; up may be null (1).  With dzt non-NULL the same values are also
 * stored transposed, dzt[n * lddzt + m] = dz[m, n] (the operand of dW = dz^T . A), which needs
 * M % 256 == 0, N % 256 == 0, (M / 256) * (N / 256) >= 256, lddz and lddzt multiples of 8 and
 * 16-byte aligned dz, dzt.  The backward of the fused LM-head + CE.
 * Replaces: kernels/loss.py:34-44,64-68 (_backward) together with the logits matmul of
 * _model.py:131-132 (no single reference function). */
int q3_gemm_nt_ce_grad(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, void* dz, int64_t lddz,
                       void* dzt, int64_t lddzt, int64_t M, int64_t N, int64_t K, int64_t col0, const int64_t* tgt,
                       const float* lse, const float* count, const float* up, int64_t vocab, int64_t ignore_index,
                       hipStream_t stream);
/* The logits GEMM and q3_ce_chunk_stats in one kernel: z = A . B^T as above; per row and per group
 * of 128 logit columns g (g = 0 .. ceil(N / 128) - 1), m_part[(part0 + g) * ldp + row] and
 * s_part[...] receive the group's max and sum of exp(z - max), and pick[row] the logit of column
 * tgt[row] - col0 when it lies in [0, N).  q3_ce_finish then merges all groups of all chunks as
 * its nchunks partials.  The forward of the fused LM-head + CE.
 * Replaces: kernels/loss.py:6-33,55-61 (_partials, _rows) together with the logits matmul of
 * _model.py:131-132 (no single reference function). */
int q3_gemm_nt_ce_stats(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                        int64_t K, int64_t col0, const int64_t* tgt, float* m_part, float* s_part, float* pick,
                        int64_t part0, int64_t ldp, hipStream_t stream);
/* q3_gemm_nt_ce_stats that also stores the logits rounded to dtype, z[row * ldz + col] (ldz a multiple
 * of 8, 16-byte aligned z), and forms the statistics from those rounded values -- the bf16 logits of
 * the reference's lm_head output (_model.py:131-132), kept for the backward.
 * Replaces: the logits matmul of _model.py:131-132 with kernels/loss.py:6-33,55-61 (_partials, _rows). */
int q3_gemm_nt_ce_stats_store(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                              int64_t K, int64_t col0, const int64_t* tgt, float* m_part, float* s_part, float* pick,
                              int64_t part0, int64_t ldp, void* z, int64_t ldz, hipStream_t stream);

/* ------------------------------------------------------------------ greedy decode
 * y[m, n] = sum_k x[m, k] * W[n, k] for m < M <= 16 (x rows at stride ldx, y rows at stride ldy),
 * fp32 accumulation on the matrix cores, weights streamed once (q3_decode_linear, mode 0, no norm).
 * Replaces: inference/kernels.py:116-146 (_inference_gemv / linear for small M),
 * inference/accumulation.py:13-84. */
int q3_gemv(int dtype, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t m, int64_t n,
            int64_t k, hipStream_t stream);
/* Fused decode-step projection for M <= 16 token rows (K % 8 == 0, 16-byte aligned rows):
 *   with norm_w, xn W^T means rsqrt(mean_k x[m, k]^2 + eps) * (dtype(x[m, :] * norm_w) W^T), the
 *   RMSNorm's row scale applied to the fp32 dot product; without it, x W^T;
 *   mode 0: y_i[m, :n_i] = xn W_i^T for each of the nseg <= 3 segments (W_i [n_i, K], row-major);
 *   mode 1: y_0 = res + dtype(xn W_0^T)  (residual add; res rows at stride ldres, may alias y_0);
 *   mode 2: y_0 = silu(dtype(xn W_0^T)) * dtype(xn W_1^T)  (SwiGLU; nseg == 2, n_0 == n_1).
 * w, y, ldy and n are host arrays of nseg entries.  Deterministic (fixed-order reductions).
 * Replaces, in one launch each: inference/model.py:117-121 (rms_norm + q/k/v linear),
 * inference/model.py:126 (o_proj linear + residual_add), inference/model.py:127-130 (rms_norm +
 * gate/up linear + swiglu), inference/model.py:134 (down linear + residual_add). */
int q3_decode_linear(int dtype, const void* x, int64_t ldx, int64_t m, int64_t k, const void* norm_w, float eps,
                     int mode, int nseg, const void* const* w, void* const* y, const int64_t* ldy, const int64_t* n,
                     const void* res, int64_t ldres, hipStream_t stream);
/* cache_{k,v}[b, h, start + s, :] = {k,v}[b, s, h, :]; caches are [B,H,capacity,D].  When start_dev is
 * non-NULL the start position is read from that device int64 at run time (a graph-replayable decode
 * step); positions >= capacity are skipped.  Replaces: inference/kernels.py:24-35 (_inference_cache_append). */
int q3_kv_append(int dtype, const void* k, const void* v, void* cache_k, void* cache_v, int64_t B, int64_t S,
                 int64_t H, int64_t D, int64_t capacity, int64_t start, const int64_t* start_dev,
                 hipStream_t stream);
/* One query per (b, head) against the first T_len cached positions (D = 128, Hq/Hkv <= 8): one
 * workgroup per (b, kv head, 128-key split) serves the whole GQA group,
 * then a fixed-order merge of the split partials.  q/out element strides (batch, head);
 * cache strides (ksb, ksh) with position stride D.  With len_dev non-NULL, T_len = *len_dev + 1 is
 * read at run time and the launch covers the whole capacity (workspace sized for T_len = capacity).
 * The launched span (T_len, or capacity with len_dev) is at most 65536 positions.
 * Replaces: inference/kernels.py:71-113 (_inference_decode_partial, _inference_decode_merge,
 * attention with s == 1). */
size_t q3_decode_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t T_len);
int q3_decode_attention(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* cache_k, const void* cache_v,
                        int64_t ksb, int64_t ksh, void* out, int64_t osb, int64_t osh, void* workspace, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity, int64_t D,
                        float scale, hipStream_t stream);
/* Decode step attention with the per-token prologue fused in: q [B,Hq,D] and the new token's k, v
 * [B,Hkv,D] are raw projections.  Each workgroup applies QK-norm (q_norm_w / k_norm_w, eps) and RoPE
 * (cos/sin [B,D] rows of the token's position, batch stride csb) to its query heads; the workgroup
 * whose split holds the token's position writes the normed+roped k and raw v into the caches there and
 * uses them directly.  Same geometry, workspace and results (bit for bit) as q3_norm_rope_fwd on q and
 * k, then q3_kv_append, then q3_decode_attention.  Replaces, in one launch pair:
 * inference/model.py:122-125 (norm_rope q/k, cache append, attention for s == 1). */
int q3_decode_step_attention(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
                             int64_t kvsb, int64_t kvsh, const void* q_norm_w, const void* k_norm_w, float eps,
                             const void* cos, const void* sin, int64_t csb, void* cache_k, void* cache_v, int64_t ksb,
                             int64_t ksh, void* out, int64_t osb, int64_t osh, void* workspace, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity, int64_t D,
                             float scale, hipStream_t stream);
/* q3_decode_step_attention without a workspace argument: the split partials go to a fixed
 * Q3_NOALLOC_SCRATCH_BYTES (16 MiB) device array inside the library (one per GPU, kept until the
 * process ends), so the call allocates nothing.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid allocation).  The
 * limit is q3_decode_attention_workspace_bytes(B, Hq, Hkv, span) <= Q3_NOALLOC_SCRATCH_BYTES, span =
 * capacity when len_dev is given, else T_len (B 8 x Hq 32 fits a span of 16128 positions);
 * larger requests return Q3_ERR_SCRATCH before any launch.  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (concurrent streams or threads) race; calls in
 * one stream are ordered and safe.  Arguments and results otherwise as q3_decode_step_attention
 * (bit-identical outputs). */
#define Q3_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int q3_decode_step_attention_noalloc(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
                                     int64_t kvsb, int64_t kvsh, const void* q_norm_w, const void* k_norm_w, float eps,
                                     const void* cos, const void* sin, int64_t csb, void* cache_k, void* cache_v,
                                     int64_t ksb, int64_t ksh, void* out, int64_t osb, int64_t osh, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity,
                                     int64_t D, float scale, hipStream_t stream);
/* Greedy step: token[b] = argmax logits[b, :vocab] (lowest index on ties), pad if done[b]; writes
 * ids[b, p] (ids may be NULL; p = pos, plus *pos_dev when pos_dev is non-NULL), next[b],
 * done[b] |= token in eos[0:n_eos].
 * Replaces: inference/kernels.py:149-173 (_inference_argmax_parts, _inference_select, select). */
size_t q3_greedy_select_workspace_bytes(int64_t batch);
int q3_greedy_select(int dtype, const void* logits, int64_t ld, int64_t batch, int64_t vocab, void* workspace,
                     int64_t* ids, int64_t ld_ids, int64_t pos, const int64_t* pos_dev, int64_t* next, uint8_t* done,
                     const int64_t* eos, int n_eos, int64_t pad, hipStream_t stream);
/* *counter += by on the device (advances a device-resident cache length between graph replays).
 * No counterpart in the reference: it is what lets one captured decode step serve every position. */
int q3_advance(int64_t* counter, int64_t by, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* Q3HIP_H */
