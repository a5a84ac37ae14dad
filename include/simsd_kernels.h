/*
 * libsimsd_kernels.so -- C ABI of the SimSD matmul hot path on MI355X (gfx950).
 *
 * Plain C: raw device pointers, element strides, sizes, and the HIP stream as
 * an opaque pointer (hipStream_t, e.g. torch.cuda.current_stream().cuda_stream).
 * Every entry point is stream-ordered, never synchronises the host, never
 * allocates device memory, and returns 0 on success or -1 with a message left
 * in simsd_last_error_string() (per thread).  The caller owns every buffer,
 * workspaces included.  Launches go to the current HIP device: callers make
 * the tensors' device current first (the reference's device guard,
 * kernels/moe_dispatch_fused.py:145-151).
 *
 * Reference entry points each function replaces are cited as file:line in the
 * airevo2/SimSD-release tree.
 */
#ifndef SIMSD_KERNELS_H_
#define SIMSD_KERNELS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIMSD_ABI_VERSION 18

/* dtype codes */
#define SIMSD_DTYPE_BF16 0
#define SIMSD_DTYPE_F16 1
#define SIMSD_DTYPE_F32 2

/* routing scores */
#define SIMSD_SCORE_SOFTMAX 0
#define SIMSD_SCORE_SIGMOID 1

#define SIMSD_MOE_MAX_EXPERTS 1024
#define SIMSD_MOE_MAX_SLOTS 8192

/* ---- housekeeping ---------------------------------------------------- */
int simsd_abi_version(void);
const char* simsd_last_error_string(void);

/* ---- skinny linear ------------------------------------------------------
 * y[m, n] = dtype(sum_k x[m, k] * w[n, k])  (+ bias[n] in the dtype), fp32
 * accumulation, y in the input dtype: the bias goes onto the rounded product,
 * as the reference's `y += bias` after its kernel (thin_linear_fused.py:343-344).
 * Replaces the launch of _thin_gemv_kernel (+ _thin_gemv_reduce when
 * SPLIT_K > 1) in thin_linear, kernels/thin_linear_fused.py:321-344, and the
 * kernels themselves (67-171).
 *   strides are in elements; any stride works (non-unit K strides and
 *   unaligned rows take a slower element-wise path);
 *   block_n: weight rows per workgroup (4, 8, 16 or 32; 0 = automatic;
 *            above 8 tokens in bf16/fp16 also 24 -- two 16-row MFMA blocks,
 *            the second half-filled -- and 64, 96 or 128, the shared-activation
 *            tiles; 24 acts as 16 and 64-128 as 32 elsewhere);
 *   block_k: k elements of activations a wave holds at once in the M <= 8
 *            bf16/fp16 kernel (256 or 1024; 0 = 256; other kernels ignore it);
 *   split_k: workgroups along K (0 = automatic); with split_k > 1 fp32
 *            partial tiles go to the workspace and a second launch sums them
 *            in split order (deterministic);
 *   num_waves: waves per workgroup splitting K (2, 4 or 8; 0 = 4);
 *   workspace: needed only when split_k > 1 (size from
 *            simsd_thin_linear_workspace_bytes, 16-byte aligned, no
 *            initialisation needed).
 * Results are bit-identical across calls for the same shape and config.
 * K must be >= 1 (the caller handles K == 0). */
int simsd_thin_linear(const void* x, int64_t stride_xm, int64_t stride_xk,
                      const void* w, int64_t stride_wn, int64_t stride_wk,
                      const void* bias, int64_t stride_b,
                      void* y, int64_t stride_ym, int64_t stride_yn,
                      int64_t M, int64_t N, int64_t K, int dtype,
                      int block_n, int block_k, int split_k, int num_waves,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* simsd_thin_linear without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: its
 * thin_linear allocates its partials through _partials().  The split-K
 * partials go to a static per-GPU array of
 * simsd_thin_linear_noalloc_max_scratch_bytes() bytes (8 MiB) inside the
 * library; a call whose plan needs more returns -1 with an error.  Nothing is
 * allocated and nothing needs clearing (every partial is written before it
 * is read).  All calls on one GPU share that array: calls that overlap on one
 * GPU (two streams at once) race.  Results equal simsd_thin_linear's. */
int simsd_thin_linear_noalloc(const void* x, int64_t stride_xm, int64_t stride_xk,
                              const void* w, int64_t stride_wn, int64_t stride_wk,
                              const void* bias, int64_t stride_b,
                              void* y, int64_t stride_ym, int64_t stride_yn,
                              int64_t M, int64_t N, int64_t K, int dtype,
                              int block_n, int block_k, int split_k, int num_waves, void* stream);
int64_t simsd_thin_linear_noalloc_max_scratch_bytes(void);

/* Workspace bytes simsd_thin_linear needs for this shape/config (0 if none).
 * Plays the role of _partials(), kernels/thin_linear_fused.py:177-185. */
int64_t simsd_thin_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype,
                                          int block_n, int split_k, int num_waves);

/* The launch geometry simsd_thin_linear picks: out4 = {rows per workgroup,
 * columns per block, waves per workgroup, split_k}.  Counterpart of
 * pick_config / _heuristic_config, kernels/thin_linear_fused.py:217-262. */
int simsd_thin_linear_plan(int64_t M, int64_t N, int64_t K, int dtype, int block_n,
                           int split_k, int num_waves, int* out4);

/* ---- gated projection ----------------------------------------------------
 * h[m, i] = dtype( dtype(silu(dtype(g))) * dtype(u) ),
 *   g = sum_k x[m, k] w_gate[i, k],  u = sum_k x[m, k] w_up[i, k]  (fp32 sums)
 * -- the rounding points of a bf16/fp16 act_fn(gate_proj(x)) * up_proj(x) in
 * PyTorch -- in one pass over both weights, with no [M, 2I] intermediate.
 * Fuses the gate and up projections of an MLP block with its SiLU and
 * product, modeling_sdar.py:113-119 (SDARMLP.forward, a caller of
 * thin_linear); no single reference entry point.  A merged [2I, K] gate_up
 * weight is w_gate = its first I rows and w_up = the rest.
 *   bf16/fp16 only; x, w_gate and w_up K-contiguous, 16-byte aligned rows.
 *   block_n: gate + up rows per workgroup (8, 16 or 32; 0 = automatic), i.e.
 *            block_n / 2 output columns; other arguments as simsd_thin_linear;
 *   workspace (split_k > 1): simsd_thin_linear_workspace_bytes(M, 2*I, K, ...). */
int simsd_thin_linear_silu_mul(const void* x, int64_t stride_xm, int64_t stride_xk,
                               const void* w_gate, int64_t stride_gn, int64_t stride_gk,
                               const void* w_up, int64_t stride_un, int64_t stride_uk,
                               void* h, int64_t stride_hm, int64_t stride_hn,
                               int64_t M, int64_t I, int64_t K, int dtype,
                               int block_n, int block_k, int split_k, int num_waves,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* ---- RMSNorm and the RMSNorm prologue -------------------------------------
 * y[m, k] = dtype( gamma[k] * dtype( x[m, k] * r_m ) ),
 *   r_m = 1 / sqrt( sum_k x[m, k]^2 / K + eps )  (fp32)
 * -- the stock PyTorch RMSNorm the reference's runner installs
 * (sdar/run_native_tp2.py:34-51; SDARRMSNorm, modeling_sdar.py:74-92), in one
 * launch.  x and y K-contiguous (row strides in elements), gamma [K]
 * contiguous in the same dtype. */
int simsd_rmsnorm(const void* x, int64_t stride_xm, const void* gamma, float eps, void* y,
                  int64_t stride_ym, int64_t M, int64_t K, int dtype, void* stream);

/* RMSNorm(x) followed by simsd_thin_linear / simsd_thin_linear_silu_mul on
 * it.  At <= 8 tokens (bf16/fp16, vector-aligned operands, 16-byte aligned
 * gamma) the norm runs inside the GEMV: every workgroup derives its tokens'
 * scale and normalises the activations as it loads them, so the normalised
 * rows never go to memory.  Otherwise, or when the workgroups' statistics
 * reads (workgroups x M x K elements) would pass 32 MB, as for an lm_head,
 * the norm is written to the workspace and the linear reads it.  workspace: simsd_rmsnorm_linear_workspace_bytes
 * (N_rows = N, or 2*I for the gated form). */
int64_t simsd_rmsnorm_linear_workspace_bytes(int64_t M, int64_t N_rows, int64_t K, int dtype,
                                             int block_n, int split_k, int num_waves);
int simsd_rmsnorm_thin_linear(const void* x, int64_t stride_xm, int64_t stride_xk,
                              const void* gamma, float eps,
                              const void* w, int64_t stride_wn, int64_t stride_wk,
                              const void* bias, int64_t stride_b,
                              void* y, int64_t stride_ym, int64_t stride_yn,
                              int64_t M, int64_t N, int64_t K, int dtype,
                              int block_n, int block_k, int split_k, int num_waves,
                              void* workspace, int64_t workspace_bytes, void* stream);
int simsd_rmsnorm_thin_linear_silu_mul(const void* x, int64_t stride_xm, int64_t stride_xk,
                                       const void* gamma, float eps,
                                       const void* w_gate, int64_t stride_gn, int64_t stride_gk,
                                       const void* w_up, int64_t stride_un, int64_t stride_uk,
                                       void* h, int64_t stride_hm, int64_t stride_hn,
                                       int64_t M, int64_t I, int64_t K, int dtype,
                                       int block_n, int block_k, int split_k, int num_waves,
                                       void* workspace, int64_t workspace_bytes, void* stream);

/* ---- MoE: routing ------------------------------------------------------
 * ids_out[t, j] (int64) = index of the j-th largest logit of row t (ties to
 * the lower index); w_out[t, j] (fp32) = score of that expert, where score is
 * softmax over all E logits or sigmoid of the logit, renormalised over the k
 * picks when renorm != 0 and k > 1 (denominator + 1e-20), times scale.
 * Not part of the reference operator (the gate is remote LLaDA2 code); the
 * sigmoid/renorm/scale rule restates _routing,
 * kernels/workspace/moe_dispatch/build_oracle.py:71-90.  k <= 64, E <= 1024. */
int simsd_moe_route_topk(const float* logits, int64_t T, int64_t E, int64_t stride_t, int k,
                         int scoring, int renorm, float scale, int64_t* ids_out, float* w_out,
                         void* stream);

/* ---- MoE: align -------------------------------------------------------
 * Worst-case tile count min(E, M) + ceil(M / 16) for M = T*k slots.
 * _num_tiles, kernels/moe_dispatch_fused.py:135-137. */
int simsd_moe_num_tiles(int64_t M, int64_t E);

/* Sort the M = T*k flat slots by expert (stable) and lay each expert's group
 * out on 16-row boundaries.  Replaces _align, kernels/moe_dispatch_fused.py:93-132.
 *   counts[E]          slots per expert
 *   offsets[E+1]       exclusive scan of counts (offsets[E] = valid slots)
 *   pad_offsets[E+1]   exclusive scan of counts rounded up to 16
 *   perm[M]            slot ids in sorted order (argsort(ids, stable=True));
 *                      ids outside [0, E) sort last, in slot order
 *   slots[16*num_tiles] slot id per padded row, -1 for padding
 *   tile_expert[num_tiles] expert of each 16-row tile, E past the used range
 * One workgroup; E <= 1024, M <= 8192. */
int simsd_moe_align(const int64_t* ids, int64_t M, int64_t E, int num_tiles,
                    int32_t* counts, int32_t* offsets, int32_t* pad_offsets, int32_t* perm,
                    int32_t* slots, int32_t* tile_expert, void* stream);

/* Route and align in one launch (one workgroup): the outputs of
 * simsd_moe_route_topk (ids_out, w_out) followed by those of simsd_moe_align
 * on the same ids, identical to calling the two in sequence.  The picks stay
 * in LDS between the steps, which saves a launch and a round trip through
 * memory at small token counts.  Counterpart of the remote gate's top-k
 * followed by _align, kernels/moe_dispatch_fused.py:93-132.  T*k <= 8192,
 * E <= 1024, k <= 64; tokens are routed 16 at a time, so large T is better
 * served by the two separate calls. */
int simsd_moe_route_align(const float* logits, int64_t T, int64_t E, int64_t stride_t, int k,
                          int scoring, int renorm, float scale, int64_t* ids_out, float* w_out,
                          int num_tiles, int32_t* counts, int32_t* offsets, int32_t* pad_offsets,
                          int32_t* perm, int32_t* slots, int32_t* tile_expert, void* stream);

/* ---- MoE: grouped expert FFN + combine ----------------------------------
 * out[t] = dtype( sum_j fp32(down_e(silu(gate_e(x_t)) * up_e(x_t))) * w[t, j] )
 * with e = ids[t, j], then, when a shared expert is given,
 * out[t] = dtype(out[t] + shared(x_t)).  Rounding points follow the reference
 * (g, u, silu(g), h and each expert output rounded to the dtype; weighting and
 * the sum over j in fp32).  Replaces the three _gemm launches, the SiLU.mul and
 * the combine of moe_dispatch, kernels/moe_dispatch_fused.py:140-192; the
 * shared-expert addition is the remote LLaDA2 forward's, fused in.
 *   w_gate/w_up [E, I, H], w_down [E, H, I] (element strides per dim);
 *   sh_gate/sh_up [Is, H], sh_down [H, Is] or all NULL;
 *   slots/tile_expert/num_tiles from simsd_moe_align;
 *   ids with out-of-range experts contribute nothing;
 *   workspace: simsd_moe_workspace_bytes(T, k, H, I, Is, dtype) bytes. */
int64_t simsd_moe_workspace_bytes(int64_t T, int k, int64_t H, int64_t I, int64_t Is, int dtype);

int simsd_moe_grouped_ffn(const void* x, int64_t stride_xt, int64_t stride_xh,
                          const void* w_gate, int64_t sge, int64_t sgi, int64_t sgh,
                          const void* w_up, int64_t sue, int64_t sui, int64_t suh,
                          const void* w_down, int64_t sde, int64_t sdh, int64_t sdi,
                          const void* sh_gate, int64_t shg_i, int64_t shg_h,
                          const void* sh_up, int64_t shu_i, int64_t shu_h,
                          const void* sh_down, int64_t shd_h, int64_t shd_i, int64_t Is,
                          const int32_t* slots, const int32_t* tile_expert, int num_tiles,
                          const int64_t* topk_ids, int64_t stride_idt, int64_t stride_idk,
                          const float* topk_w, int64_t stride_wt, int64_t stride_wk,
                          void* out, int64_t stride_ot, int64_t stride_oh,
                          int64_t T, int k, int64_t E, int64_t H, int64_t I, int dtype,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* y[m, n] = residual[m, n] + dtype(sum_k x[m, k] * w[n, k]): the linear with
 * the decoder layer's residual add in its epilogue (the projection rounded to
 * the dtype, then the dtype add, as `hidden = residual + o_proj(attn)` and
 * `hidden = residual + mlp(...)` compute it, sdar/modeling_sdar.py's decoder
 * layer).  y may be the residual itself (in place).  Other arguments as
 * simsd_thin_linear; workspace from simsd_thin_linear_workspace_bytes. */
int simsd_thin_linear_residual(const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn, int64_t swk,
                               const void* residual, int64_t srm, int64_t srn, void* y, int64_t sym, int64_t syn,
                               int64_t M, int64_t N, int64_t K, int dtype, int block_n, int block_k, int split_k,
                               int num_waves, void* workspace, int64_t workspace_bytes, void* stream);

/* The split-K partials of x @ w^T without their reduce launch: part
 * [split_k][M][N] fp32 (16-byte aligned, part_bytes >= split_k * M * N * 4),
 * partial s summing k-chunk s of the plan (split_k 1..16, taken as given;
 * split_k 1 is the whole K in one partial).  For a consumer that sums them in
 * a launch it makes anyway -- simsd_reduce_residual_rmsnorm,
 * simsd_reduce_qkv_rope_cache -- so a projection can split K (every
 * workgroup reading 1/split of the activation rows) at no extra launch: the
 * reference's split-K GEMV writes the same staging and sums it in its own
 * launch, kernels/thin_linear_fused.py:139-171, 313-344.  Other arguments as
 * simsd_thin_linear (no bias). */
int simsd_thin_linear_partials(const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn, int64_t swk,
                               void* part, int64_t part_bytes, int64_t M, int64_t N, int64_t K, int dtype,
                               int block_n, int block_k, int split_k, int num_waves, void* stream);

/* The decoder layer's residual add and the next RMSNorm on a projection's
 * partials, one launch: for each row m,
 *   h[m, :]  = dtype(dtype(sum_s part[s, m, :]) + residual[m, :])
 *   xn[m, :] = dtype(gamma * dtype(h[m, :] * r)),  r = 1 / sqrt(mean(h^2) + eps)
 * (the partials summed in split order; the stock RMSNorm of
 * sdar/run_native_tp2.py:42-47 / SDARRMSNorm, modeling_sdar.py:74-92, on the
 * new residual stream -- `hidden = residual + proj(...)` followed by the next
 * norm of the decoder layer, modeling_sdar.py:305-366).  Bit-identical to
 * simsd_thin_linear_residual's reduce followed by simsd_rmsnorm on the same
 * partials.  bf16 or fp16; N % 8 == 0, N <= 8192; split 1..8; 16-byte
 * aligned rows (row strides srm, shm, sxn elements).  h may be residual (in
 * place). */
int simsd_reduce_residual_rmsnorm(const void* part, int split, int64_t part_bytes, const void* residual,
                                  int64_t srm, void* h, int64_t shm, const void* gamma, float eps, void* xn,
                                  int64_t sxn, int64_t M, int64_t N, int dtype, void* stream);

/* ---- logits epilogue: softmax statistics and the unmasking choice -------
 * For logits rows l[m, 0:V] (bf16, fp16 or fp32; row stride slm elements,
 * unit element stride):
 *   ids[m]  = the first index of the row maximum (int64),
 *   conf[m] = its softmax probability 1 / sum_v exp(l[m, v] - max) (fp32),
 *   probs[m, v] = exp(l[m, v] - max) / sum (fp32, row stride spm; NULL to skip),
 * i.e. probs = F.softmax(logits.float(), -1), ids = probs.argmax(-1),
 * conf = probs.gather(1, ids): the epilogue of the draft denoise step,
 * speculative_decoding/cache_aware.py:916-919, and the verify pass's
 * target_probs, cache_aware.py:1197-1198.  All sums run in a fixed order
 * (bit-reproducible).  Workspace: simsd_softmax_argmax_workspace_bytes(M, V),
 * 16-byte aligned, no initialisation needed. */
int64_t simsd_softmax_argmax_workspace_bytes(int64_t M, int64_t V);

int simsd_softmax_argmax(const void* logits, int64_t slm, int64_t M, int64_t V, int dtype, int64_t* ids,
                         float* conf, float* probs, int64_t spm, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* One unmasking step of the draft's block denoise loop, in place,
 * cache_aware.py:916-938: ids/conf as above for the M <= 64 rows of the
 * block; among the rows with cur_ids[m] == mask_id, the n_unmask with the
 * largest conf (ties: the lower row; rows not masked rank as -inf, as in the
 * reference's masked_conf.topk) get cur_ids[m] = ids[m], step_map[m] = step
 * (step_map may be NULL) and, when per_pos_probs is not NULL, their softmax
 * row written to per_pos_probs[m, :] (row stride spp).  Workspace as for
 * simsd_softmax_argmax. */
int simsd_denoise_select(const void* logits, int64_t slm, int64_t M, int64_t V, int dtype, int64_t* cur_ids,
                         int64_t mask_id, int n_unmask, int64_t* step_map, int64_t step, float* per_pos_probs,
                         int64_t spp, int64_t* ids, float* conf, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* ---- attention over a static KV cache ----------------------------------
 * Cache layout per layer (one sequence, head_dim D = 128, L slots, L a
 * multiple of 32): one block of L * D elements per KV head (head stride
 * kv_head_stride >= L * D elements) in each of two tile arrays, laid out in
 * the order the attention's MFMA operands read them:
 *   K: (slot s, dim d) at ((s/16 * 16 + d/8) * 16 + s%16) * 8 + d%8
 *   V: (slot s, dim d) at ((((s/32 * 8 + d/16) * 16 + d%16) * 4 + s/4%4) * 2
 *                          + s/16%2) * 4 + s%4
 * The KV heads are stored once per group, not replicated per query head.
 *
 * simsd_qkv_rope_cache: for each of the M tokens of qkv [M, (Hq + 2 Hkv) * D]
 * (q heads, then k heads, then v heads; row stride sqkv), the SDAR attention
 * prologue, sdar/modeling_sdar.py:250-262: q and k heads through their
 * RMSNorm (stock rounding points; weights q_norm_w / k_norm_w [D], NULL to
 * skip), then RoPE with the cos/sin rows of pos[m] (tables [n_pos, D], row
 * stride scs, as the rotary embedding returns them, in the dtype):
 *   out = dtype(dtype(x * cos) + dtype(rotate_half(x) * sin)),
 * q to q_out [M, Hq, D] (strides sqo_m, sqo_h), k and v into the cache at
 * slot slots[m] and, when slots2 is not NULL, also at slots2[m] -- the
 * index_copy_ writes of adapters/base.py:184-236.  Positions outside
 * [0, n_pos) give a zero q row and no k write; slots outside [0, L) are
 * skipped. */
int simsd_qkv_rope_cache(const void* qkv, int64_t sqkv, const void* q_norm_w, const void* k_norm_w, float eps,
                         const void* cos, const void* sin, int64_t scs, int64_t n_pos, const int64_t* pos,
                         const int64_t* slots, const int64_t* slots2, void* k_cache, void* v_cache,
                         int64_t kv_head_stride, int64_t L, void* q_out, int64_t sqo_m, int64_t sqo_h, int64_t M,
                         int64_t Hq, int64_t Hkv, int64_t head_dim, int dtype, void* stream);

/* simsd_qkv_rope_cache with the q/k/v projection given as its split-K
 * partials (part [split][M][(Hq + 2 Hkv) * D] fp32 from
 * simsd_thin_linear_partials, split 1..8): each value is the partials' sum
 * in split order rounded to the dtype -- the reduced projection's value --
 * then as simsd_qkv_rope_cache.  Bit-identical to the reduce followed by
 * simsd_qkv_rope_cache, in one launch. */
int simsd_reduce_qkv_rope_cache(const void* part, int split, int64_t part_bytes, const void* q_norm_w,
                                const void* k_norm_w, float eps, const void* cos, const void* sin, int64_t scs,
                                int64_t n_pos, const int64_t* pos, const int64_t* slots, const int64_t* slots2,
                                void* k_cache, void* v_cache, int64_t kv_head_stride, int64_t L, void* q_out,
                                int64_t sqo_m, int64_t sqo_h, int64_t M, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                int dtype, void* stream);

/* simsd_block_attention: out[m, hq] = softmax(scale * q[m, hq] . K[h]^T over
 * the visible slots) . V[h] with h = hq / (Hq / Hkv) -- the SDPA call of
 * adapters/base.py:245-262 with its bool mask (mask [M, >= L_valid] uint8,
 * row stride smask, nonzero = visible; NULL = all visible; 4-byte aligned
 * rows of at least L_valid rounded up to 4 bytes).  Slots
 * [0, L_valid) are considered, L_valid <= L_cap (the cache's slot count, a
 * multiple of 32); fp32 softmax, output rounded to the dtype; rows with no
 * visible slot give 0.  Every slot below L_cap must hold finite values (a
 * zero-initialised cache written only with finite K/V), since slots past a
 * row's visible range may enter the P.V product with weight 0.
 * valid_len_dev (nullable) points at a device int64
 * that lowers L_valid at run time (clamped to [0, L_valid]), so a captured
 * graph can follow a growing context.  q [M, Hq, D] and out [M, Hq, D] with
 * (row, head) strides.  Workspace: simsd_block_attention_workspace_bytes(M, Hq, Hkv,
 * L_valid), 16-byte aligned; its first bytes hold arrival counters that must
 * be zero before the first call on that workspace (allocate it zeroed and
 * keep it), and every completed call leaves them zero.  Calls that share a
 * workspace must run in stream order.  Deterministic. */
int64_t simsd_block_attention_workspace_bytes(int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid);

int simsd_block_attention(const void* q, int64_t sq_m, int64_t sq_h, const void* k_cache, const void* v_cache,
                          int64_t kv_head_stride, int64_t L_cap, const uint8_t* mask, int64_t smask, void* out,
                          int64_t so_m, int64_t so_h, int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid,
                          const int64_t* valid_len_dev, int64_t head_dim, float scale, int dtype, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* simsd_qkv_rope_attention: simsd_qkv_rope_cache followed by
 * simsd_block_attention in one launch, for a forward of M <= 16 rows whose
 * cache slots are the last M of the valid range, [lv - M, lv) with lv the
 * (device-lowered) valid length -- the layout of every forward of the
 * speculative runner.  Replaces, per layer, the q/k norm + RoPE of
 * sdar/modeling_sdar.py:250-262, the cache write of
 * adapters/base.py:186-236 (index_copy_) and the SDPA of
 * adapters/base.py:245-262.  qkv [M, (Hq + 2 Hkv) * D] is the merged
 * projection output (row stride sqkv); the other arguments are those of the
 * two calls it replaces (no q_out: the rotated queries stay in registers; no
 * second slots).  Writes the M rows' K (normed, rotated; rows with a
 * position outside [0, n_pos) leave their K slot unwritten and attend with
 * zero K) and V at their slots, and out.  Only the head form is fused: at
 * most 32 query rows per KV head and L_valid <= 4096 slots, else the call
 * fails (use the two calls).  16-byte aligned qkv rows, norm weights, cos /
 * sin rows and K / V tiles.  pos may be NULL: cos / sin then hold the rows'
 * own tables, row m's at m * scs (n_pos >= M), gathered once by the caller
 * for all layers of a forward, so the launch loads them without first
 * loading the positions.  Workspace: simsd_block_attention_workspace_bytes
 * with the same arguments, under the same rules.  Deterministic; the q/k
 * norm's fp32 sum of squares is ordered differently from
 * simsd_qkv_rope_cache's, so outputs may differ from the two calls' in the
 * last bit. */
int simsd_qkv_rope_attention(const void* qkv, int64_t sqkv, const void* q_norm_w, const void* k_norm_w, float eps,
                             const void* cos, const void* sin, int64_t scs, int64_t n_pos, const int64_t* pos,
                             void* k_cache, void* v_cache, int64_t kv_head_stride, int64_t L_cap,
                             const uint8_t* mask, int64_t smask, void* out, int64_t so_m, int64_t so_h, int64_t M,
                             int64_t Hq, int64_t Hkv, int64_t L_valid, const int64_t* valid_len_dev,
                             int64_t head_dim, float scale, int dtype, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* simsd_block_mask: the attention mask rows (uint8, 1 = visible; row stride
 * smask, n_cols slots) of a cached forward whose rows are n_prefix rows of a
 * committed block folded in (speculative_decoding/cache_aware.py:1062-1070),
 * n_free rows of the block being denoised, and K verify blocks of bl data
 * then bl mask rows (speculative_decoding/verify.py:350-418).  Slots
 * [0, ctx_len) are the committed context; the rows' own scratch slots start at
 * s0 in row order.  Verify visibility follows the multi-block rule of
 * sdar/new_attn_multi_block.py:22-183 with step_map [K, bl] (int64, device;
 * -1 = never drafted) and bs denoising steps per block; every row sees the
 * context and the prefix; the free block sees itself.  A prefix of several
 * committed blocks (n_prefix a multiple of bl) is block-causal among itself,
 * as the reference flushes them into the cache one block at a time
 * (cache_aware.py:2324-2336).  Replaces the torch
 * mask construction of cache_aware.py:1149-1180 and the multi-block mask
 * builder. */
int simsd_block_mask(uint8_t* mask, int64_t smask, int64_t n_cols, int64_t ctx_len, int64_t s0, int n_prefix,
                     int n_free, int K, int bl, int bs, const int64_t* step_map, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SIMSD_KERNELS_H_ */
