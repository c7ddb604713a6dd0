/*
 * specfold_amd — C ABI of the MI355X (gfx950) kernels for SpecFold's folded
 * multi-branch verify step.
 *
 * Every entry point takes raw device pointers, plain int/float sizes and a HIP
 * stream (passed as void*), launches asynchronously on that stream, allocates
 * nothing, and returns an int status (SF_OK or one of the SF_ERR_* codes).
 * Buffers are caller-owned; scratch comes in as a workspace argument whose size
 * the matching *_workspace_bytes() function returns.
 *
 * Layout conventions (one verify step of B1 branches x N block positions,
 * BN = B1*N "flat rows", flat row r = b*N + n):
 *   hidden   bf16 [BN, D]                 layer input, row-major
 *   q_buf    bf16 [BN+1, H*hd]            roped q per flat row (row BN = trash)
 *   kv_buf   bf16 [BN+1, 2*Hkv*hd]        roped k heads, then v heads
 *   o32      fp32 [BN, H*hd]   o_bf bf16 [BN, H*hd]   attention output
 *   m_tab, z_tab fp32 [BN, H]             softmax row max and sum exp(s - m)
 *   rows     int32 [bucket]               ascending flat ids of recomputed rows
 *   prefix K/V cache: element (head h, token t, dim d) lives at
 *     base + page_table[t / page_size] * page_stride + h * head_stride
 *          + (t % page_size) * hd + d
 *   or, with page_table == NULL, at base + h * head_stride + t * hd + d
 *   (the reference's contiguous [1, Hkv, P, hd] cache is head_stride = P*hd).
 *
 * Reference = chungen04/specfold; paths are relative to its root.
 */
#ifndef SPECFOLD_AMD_H
#define SPECFOLD_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF_OK 0
#define SF_ERR_SHAPE 1     /* a size outside what the kernels support */
#define SF_ERR_ARG 2       /* a required pointer is NULL or a value is invalid */
#define SF_ERR_WORKSPACE 3 /* workspace smaller than *_workspace_bytes() */
#define SF_ERR_HIP 4       /* a HIP launch failed */
#define SF_ERR_SCRATCH 5   /* larger than the fixed scratch of an allocation-free entry point */
#define SF_ERR_CAPTURE 6   /* an allocation-free entry point's first call on a device made
                              under stream capture (its set-up must run eagerly) */

/* Gate precision modes for sf_fold_gate. */
#define SF_GATE_MODEL_DTYPE 0 /* norms rounded to bf16 as the PyTorch reference
                                 does (specfold/generate/fastdllm_v2_folded.py:139-141) */
#define SF_GATE_FP32_SQUARED 1 /* dsq > delta^2 * psq in fp32, as the Triton gate
                                  (specfold/generate/triton_kernels.py:227-230) */
#define SF_GATE_ALL 2          /* every row recomputed: the dense block forward
                                  (specfold/generate/fastdllm_v2_generation.py:151-186) */
/* Flag OR-ed into a gate mode: the always-recomputed root branches are those that
   are their own parent (par[b] == b) instead of branch 0 alone, so one call gates
   several sequences' branch trees laid out one after another (a batched verify
   step; each sequence's main branch has par[b] == b).  No counterpart in the
   reference, whose verify step takes one sequence. */
#define SF_GATE_ROOTS_BY_PARENT 16
/* gate_mode flag: the gate entry points launch the row kernel only (rec, rstd, xn,
 * hidden_out); the compaction (f, src, rows, count, seg, segcnt, slot, which may
 * then be NULL here) is left to sf_qkv_rope_gated, which runs it in its GEMM's
 * prologue. */
#define SF_GATE_DEFER_COMPACT 32

const char* sf_status_string(int status);
/* 2: GEMM weights in the packed layout of sf_pack_weight; fused residual entries.
 * 3: sf_parent_map (the branch parent map on the device); sf_logit_stats.
 * 4: batched verify steps: SF_GATE_ROOTS_BY_PARENT, sf_qkv_rope_branches.
 * 5: GEMMs on 64-wide K chunks (K % 64, N % 128); sf_ffn_gate_up takes a workspace.
 * 6: sf_logit_stats_noalloc, SF_ERR_SCRATCH.
 * 7: sf_attn_rows; the attention workspace holds the merged prefix states.
 * 8: all-rows o_proj / lm_head: sf_o_proj_post_norm, sf_o_proj_workspace_bytes (the
 *    workspace of sf_o_proj_residual).
 * 9: SF_ERR_CAPTURE; attention entry points refuse bucket or B1*N above 1024.
 * 10: sf_head_logits (the head with the Fast-dLLM shift); sf_lm_head runs on it.
 * 11: attention merges each recomputed row's prefix partials in the kernel that
 *     attends its rows: the workspace holds the range partials only; B1 <= 64.
 * 12: SF_GATE_DEFER_COMPACT and sf_qkv_rope_gated (the compaction in the QKV GEMM).
 * 13: sf_head_logits_rows (the head for the rows a decode step reads).
 * 14: sf_decode_facts; sf_attn_rows / sf_attn_prefix_block take NULL o32, m_tab, z_tab. */
int sf_abi_version(void);

/*
 * Branch parent map on the device.  Replaces _build_parent_map
 * (specfold/generate/fastdllm_v2_folded.py:55-75), which computes the same map on
 * the host after one device-to-host copy.  tokens [B1, N] int64 (row 0 = main);
 * diff(i) = {n : tokens[i][n] != tokens[0][n]}; par[i] = the lowest j != i with
 * |diff(j)| = |diff(i)| - 1 and diff(j) a subset of diff(i), else 0 (par[0] = 0);
 * counts[i] = |diff(i)| (counts may be NULL).  Limits: B1 <= 64, N <= 64.
 */
int sf_parent_map(const int64_t* tokens, int B1, int N, int32_t* par, int32_t* counts,
                  void* stream);

/*
 * (1) Fold gate + deterministic compaction + src resolve + input RMSNorm.
 * Replaces residual_delta_gate_kernel and src_resolve_kernel
 * (specfold/generate/triton_kernels.py:199-239 and :18-26), i.e. the per-branch
 * gate of the reference (specfold/generate/fastdllm_v2_folded.py:136-144) and
 * the compaction it feeds (:141 nonzero; Triton launch :306-310).
 *
 * rec[r]    = 1 if flat row r is recomputed (branch 0 always), else 0
 * f[r]      = rec ? b : par[b]
 * src[r]    = nearest recomputing ancestor branch of (b, n) (fixed point of f)
 * rows      = ascending flat ids of recomputed rows, slots >= count hold BN
 * count[0]  = number of recomputed rows (may exceed bucket: overflow)
 * seg[b*N+k], segcnt[b] = the k-th recomputed flat row of branch b, and how many
 * slot[r]   = index of row r in rows, or -1 (folded or beyond bucket); may be NULL
 * rstd[r]   = 1 / sqrt(mean(x^2) + eps)
 * xn[r, :]  = bf16(ln_w * bf16(x * rstd)) for recomputed rows (the
 *             Qwen2RMSNorm output the QKV projection consumes)
 * Limits: B1*N <= 1024, B1 <= 64, D % 8 == 0, D <= 8192, 1 <= bucket <= B1*N.
 *
 * sf_fold_gate_residual is the same gate for layers after the first, with the
 * previous layer's folded residual update fused in: the layer input is
 * x[r] = bf16(hp[r] + ffn[src_prev[r]*N + r%N]) (fastdllm_v2_folded.py:218),
 * written to hidden_out (which must not alias hp).  src_prev is read before src
 * is written, so both may be the same buffer.
 *
 * sf_residual_rmsnorm, after the last layer: hidden_out[r] = x[r] as above and
 * out[r] = bf16(w * bf16(x[r] * rstd)) for every row (the final norm, :222).
 */
int sf_fold_gate(const uint16_t* hidden, const int32_t* par, const uint16_t* ln_w, int B1, int N,
                 int D, int bucket, float delta, float eps, int gate_mode, int8_t* rec, int32_t* f,
                 int32_t* src, int32_t* rows, int32_t* count, int32_t* seg, int32_t* segcnt,
                 int32_t* slot, float* rstd, uint16_t* xn, void* stream);
int sf_fold_gate_residual(const uint16_t* hp, const uint16_t* ffn, const int32_t* src_prev,
                          const int32_t* par, const uint16_t* ln_w, int B1, int N, int D,
                          int bucket, float delta, float eps, int gate_mode, uint16_t* hidden_out,
                          int8_t* rec, int32_t* f, int32_t* src, int32_t* rows, int32_t* count,
                          int32_t* seg, int32_t* segcnt, int32_t* slot, float* rstd, uint16_t* xn,
                          void* stream);
int sf_residual_rmsnorm(const uint16_t* hp, const uint16_t* ffn, const int32_t* src,
                        const uint16_t* w, int B1, int N, int D, float eps, uint16_t* hidden_out,
                        uint16_t* out, void* stream);

/*
 * (2) QKV projection (bf16 MFMA, fp32 accumulate) + bias + RoPE + scatter for
 * the compacted rows.  Replaces fused_ln_qkv_rope_scatter_kernel
 * (specfold/generate/triton_kernels.py:29-87), i.e. the reference's
 * q/k/v_proj + rotate_half RoPE on recomputed rows
 * (specfold/generate/fastdllm_v2_folded.py:151-161).  The RMSNorm is applied by
 * sf_fold_gate (xn).  w_qkv = cat(Wq, Wk, Wv) [(H+2Hkv)*hd, D] in the packed
 * layout of sf_pack_weight (:77-87 packing); b_qkv may be NULL (NLD: no bias).
 * The workspace (sf_qkv_workspace_bytes) holds the GEMM's fp32 partial slots
 * (section (6)).  cos/sin bf16: with
 * pos0 == NULL they are [N, hd] tables of the block; otherwise [table_rows, hd]
 * tables over absolute positions and block position n uses row *pos0 + n
 * (pos0 = the device-side prefix length; clamped to the table), so a captured
 * launch stays valid as the prefix grows.
 * q_scale (optional, fp32 [N]) multiplies roped q by bf16(q_scale[n]) — the
 * llama-4 attention scale of specfold/generate/nld_folded.py:37-53, 175-176.
 * Limits: hd == 128, D % 128 == 0, bucket <= 1024.
 */
size_t sf_qkv_workspace_bytes(int bucket, int D, int n_qkv);
int sf_qkv_rope(const uint16_t* xn, const int32_t* rows, const int32_t* count, int bucket, int BN,
                const uint16_t* w_qkv, const uint16_t* b_qkv, const uint16_t* cos_tab,
                const uint16_t* sin_tab, const int32_t* pos0, int table_rows,
                const float* q_scale, int N, int D, int H, int Hkv, int hd,
                uint16_t* q_buf, uint16_t* kv_buf, void* workspace, size_t workspace_bytes,
                void* stream);
/* sf_qkv_rope for a batched verify step: the branch trees of several sequences
 * laid out one after another (BN = total branches * N), each sequence at its own
 * prefix length.  pos0_branch: int32 [BN/N], the first absolute position of each
 * branch's block (its sequence's prefix length), required; cos/sin [table_rows, hd]
 * over absolute positions; q_scale_rows: optional fp32 [BN], the scale of each flat
 * row.  Same GEMM, workspace and limits as sf_qkv_rope, plus BN % N == 0.  No
 * counterpart in the reference (its verify step takes one sequence); a batch of
 * one sequence gives the results of sf_qkv_rope. */
int sf_qkv_rope_branches(const uint16_t* xn, const int32_t* rows, const int32_t* count, int bucket,
                         int BN, const uint16_t* w_qkv, const uint16_t* b_qkv,
                         const uint16_t* cos_tab, const uint16_t* sin_tab,
                         const int32_t* pos0_branch, int table_rows, const float* q_scale_rows,
                         int N, int D, int H, int Hkv, int hd, uint16_t* q_buf, uint16_t* kv_buf,
                         void* workspace, size_t workspace_bytes, void* stream);

/* (1)+(2) for a gate launched with SF_GATE_DEFER_COMPACT: the compaction of rec
 * runs in the prologue of every workgroup of the QKV GEMM (each needs the
 * compacted rows as its A rows), and workgroup 0 writes f, src, rows, count, seg,
 * segcnt and slot (may be NULL) exactly as sf_fold_gate documents them, so the
 * gate's separate compaction launch goes (fastdllm_v2_folded.py:141-152 and
 * :151-161; Triton src_resolve_kernel + fused_ln_qkv_rope_scatter_kernel,
 * specfold/generate/triton_kernels.py:18-87).  pos0_per_branch = 0: the rope and
 * q scale of sf_qkv_rope (pos0 [1] or NULL, q_scale [N] or NULL); 1: those of
 * sf_qkv_rope_branches (pos0 [B1], q_scale [B1*N] or NULL).  The q/kv outputs
 * equal those of sf_fold_gate + sf_qkv_rope bit for bit.  Same workspace as
 * sf_qkv_rope.  Limits: B1 <= 64, B1*N <= 1024, 1 <= bucket <= B1*N, and those of
 * sf_qkv_rope.  No counterpart in the reference. */
int sf_qkv_rope_gated(const uint16_t* xn, const int8_t* rec, const int32_t* par, int B1, int N,
                      int bucket, int32_t* f, int32_t* src, int32_t* rows, int32_t* count,
                      int32_t* seg, int32_t* segcnt, int32_t* slot, const uint16_t* w_qkv,
                      const uint16_t* b_qkv, const uint16_t* cos_tab, const uint16_t* sin_tab,
                      const int32_t* pos0, int pos0_per_branch, int table_rows,
                      const float* q_scale, int D, int H, int Hkv, int hd, uint16_t* q_buf,
                      uint16_t* kv_buf, void* workspace, size_t workspace_bytes, void* stream);

/*
 * (3) Attention of the recomputed rows over [shared prefix ; own branch block],
 * keeping the softmax state.  Replaces specfold_flash_attn_gqa_kernel
 * (specfold/generate/triton_kernels.py:301-361), i.e. the reference's fp32
 * attention of recomputed rows (specfold/generate/fastdllm_v2_folded.py:164-181).
 * Block key j of branch b is kv_buf row src[b*N+j]*N + j.  No mask, unless
 * block_causal != 0: then block position n sees the block keys j <= n (and the
 * whole prefix) — the causal forward the NLD generator commits blocks with
 * (specfold/generate/nld_generation.py:300-310, use_causal_mask=True); used
 * with every row recomputed.
 * Writes o32, o_bf, m_tab, z_tab for the rows listed in rows[0:min(count,bucket)];
 * o32, m_tab and z_tab may be NULL (not written: o_proj reads o_bf only).
 * prefix_len (optional, device int32[1]): the prefix length, read on the device;
 * P is then the capacity the grid and workspace are sized for (so one captured
 * graph serves a growing cache).  With prefix_len NULL, P is the length.
 * workspace: sf_attn_workspace_bytes(bucket, H, P) bytes, 16-byte aligned (scratch).
 * Limits: hd == 128, H % Hkv == 0, N <= 64, H/Hkv <= 8, B1 <= 64, B1*N <= 1024
 * and bucket <= 1024 (else SF_ERR_SHAPE), P <= 32768, a page size of 16, 32, 64
 * or 128 tokens (a page holds whole 16-key groups).
 */
size_t sf_attn_workspace_bytes(int bucket, int H, int P);
int sf_attn_prefix_block(const uint16_t* q_buf, const uint16_t* kv_buf, const uint16_t* prefix_k,
                         const uint16_t* prefix_v, const int32_t* page_table, int P, int page_size,
                         long long page_stride, long long head_stride, const int32_t* src,
                         const int32_t* rows, const int32_t* count, int bucket, int B1, int N,
                         int H, int Hkv, int hd, float scaling, const int32_t* prefix_len,
                         int block_causal, float* o32, uint16_t* o_bf, float* m_tab,
                         float* z_tab, void* workspace, size_t workspace_bytes, void* stream);

/*
 * (3)+(4) Attention of every row of branches [b_first, b_first + b_count): the
 * recomputed rows as sf_attn_prefix_block computes them, and each folded row
 * (b, n) from the query of its source row s = src[b*N+n]*N + n over the prefix
 * (s's merged prefix state, merged once for s and every row it serves) and
 * branch b's own block keys -- the exact softmax
 * over the branch's keys that the reference's chain correction reaches
 * incrementally (specfold/generate/fastdllm_v2_folded.py:164-204; Triton
 * specfold_flash_attn_gqa_kernel + specfold_chain_correction_gqa_kernel,
 * specfold/generate/triton_kernels.py:301-429), so one call replaces
 * sf_attn_prefix_block + sf_chain_correct.  rows / count: the recomputed rows of
 * those branches (ascending; every folded row's source row among them).  A batched
 * step calls it once per sequence with that sequence's branch range and rows.
 * Same workspace and limits as sf_attn_prefix_block (B1 <= 64, B1*N <= 1024,
 * bucket <= 1024); no causal mode.
 */
int sf_attn_rows(const uint16_t* q_buf, const uint16_t* kv_buf, const uint16_t* prefix_k,
                 const uint16_t* prefix_v, const int32_t* page_table, int P, int page_size,
                 long long page_stride, long long head_stride, const int32_t* src,
                 const int32_t* rows, const int32_t* count, int bucket, int B1, int N,
                 int b_first, int b_count, int H, int Hkv, int hd, float scaling,
                 const int32_t* prefix_len, float* o32, uint16_t* o_bf, float* m_tab,
                 float* z_tab, void* workspace, size_t workspace_bytes, void* stream);

/*
 * (4) Chain correction of folded rows: start from the state of the nearest
 * recomputing ancestor and apply the exact rank-|R| softmax update for every
 * key changed along the ancestor chain.  Replaces
 * specfold_chain_correction_gqa_kernel (specfold/generate/triton_kernels.py:364-429),
 * the order-free form of the reference's one-hop correction
 * (specfold/generate/fastdllm_v2_folded.py:183-204).
 * Reads o32/m_tab/z_tab of src rows; writes o32, o_bf, m_tab, z_tab of folded rows.
 * Limits: hd == 128, H/Hkv <= 8, B1*N <= 1024.
 */
int sf_chain_correct(const uint16_t* q_buf, const uint16_t* kv_buf, const int32_t* src,
                     const int32_t* par, const int8_t* rec, const int32_t* seg,
                     const int32_t* segcnt, int B1, int N, int H, int Hkv, int hd, float scaling,
                     float* o32, uint16_t* o_bf, float* m_tab, float* z_tab, void* stream);

/*
 * (5) In-place KV-cache append: copy the k and v heads of n_tok consecutive
 * kv_buf rows (starting at row0) to cache positions start_pos .. start_pos+n_tok-1.
 * Replaces the torch.cat growth of the prefix cache inside the block-commit
 * forward (specfold/model_cache/nemotron_labs_diffusion/modeling_ministral.py:154-162
 * via DynamicCache.update; called from specfold/generate/fastdllm_v2_generation.py:557-575).
 * Limits: hd == 128.
 */
int sf_kv_append(const uint16_t* kv_buf, int row0, int n_tok, int Hkv, int hd, uint16_t* k_cache,
                 uint16_t* v_cache, const int32_t* page_table, int page_size,
                 long long page_stride, long long head_stride, int start_pos, void* stream);

/*
 * (6) The rest of the layer on the compacted rows (reference:
 * specfold/generate/fastdllm_v2_folded.py:207-218; Triton
 * fused_ln_gateup_silu_kernel / fused_down_residual_scatter_kernel,
 * specfold/generate/triton_kernels.py:102-194, and the torch addmm/index ops of
 * the fused path, fastdllm_v2_folded.py:351-361).
 *
 * Weights.  Every GEMM entry point here and sf_qkv_rope take their weight
 * [N, K] in the PACKED fragment-major layout that sf_pack_weight writes from a
 * row-major bf16 matrix (16-byte word (t, c, l) = W[16t + l%16][32c + 8(l/16) ..
 * +8], t < N/16, c < K/32, l < 64): each wave's weight stream is then one
 * sequential read.  Packing is done once per model (the counterpart of the
 * reference's _pack_layer_weights, fastdllm_v2_folded.py:77-87).
 *
 * Workspace.  The weight is streamed once on bf16 MFMA with fp32 accumulation
 * for every row (up to 256 rows per pass), split stream-K over one workgroup per
 * CU: tiles computed by several workgroups go through fp32 partial slots in a
 * caller workspace of sf_gemm_workspace_bytes(M or bucket, N, K) bytes
 * (sf_ffn_gate_up_workspace_bytes for sf_ffn_gate_up, sf_qkv_workspace_bytes for
 * sf_qkv_rope), summed in a fixed order by a fix-up kernel (deterministic).
 * Calls sharing a workspace must not overlap.
 *
 * sf_o_proj_residual and sf_o_proj_post_norm apply the weight to every row
 * instead (M = B1·N): one pass over the weights for up to 256 rows, the
 * workgroups splitting the columns and K into up to 16 ranges whose fp32 sums go
 * to a caller workspace of sf_o_proj_workspace_bytes(M, N, K) bytes and are added
 * in range order by the residual kernel (deterministic).  sf_head_logits (and
 * sf_lm_head) too, each workgroup over the whole of K (no workspace).
 *
 * sf_pack_weight        out = packed(w), w row-major [N, K]; N % 16 == 0, K % 64 == 0
 * sf_o_proj_residual    hp[r] = bf16(x[r] + bf16(o_bf[r] . Wo^T)), r < M (all rows)
 * sf_o_proj_post_norm   the same for r < BN, and for recomputed rows (slot[r] >= 0)
 *                       zn[slot[r]] = bf16(w * bf16(hp[r] * rstd)): o_proj and
 *                       sf_residual_post_norm in one call, without the bf16 y round
 *                       trip (fastdllm_v2_folded.py:207-212)
 * sf_residual_post_norm hp[r] = bf16(x[r] + y[r]) for r < BN, and for recomputed rows
 *                       zn[slot[r]] = bf16(w * bf16(hp[r] * rstd)) (y = a bf16 o_proj
 *                       output computed elsewhere, e.g. by a library GEMM)
 * sf_rows_rmsnorm       out[m] = bf16(w * bf16(x[rows[m]] * rstd)), m < count
 * sf_ffn_gate_up        act[m] = bf16(bf16(silu(bf16(zn[m] . Wg^T))) * bf16(zn[m] . Wu^T))
 * sf_ffn_down_scatter   ffn[rows[m]] = bf16(act[m] . Wd^T), m < count
 * sf_residual_gather_add out[r] = bf16(hp[r] + ffn[src[r]*N + r%N]), r < B1*N
 *                       (folded rows take their nearest recomputing ancestor's FFN)
 * sf_lm_head            logits[m] = bf16(x[m] . Wlm^T), m < M
 * Limits: K % 64 == 0, N % 128 == 0 (gate/up: I % 128, lm_head: V % 128), M/bucket
 * <= 1024, D <= 8192.
 */
size_t sf_gemm_workspace_bytes(int mcap, int N, int K);
size_t sf_ffn_gate_up_workspace_bytes(int bucket, int D, int I);
int sf_pack_weight(const uint16_t* w, int N, int K, uint16_t* out, void* stream);
size_t sf_o_proj_workspace_bytes(int M, int N, int K);
int sf_o_proj_residual(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo, int M, int K,
                       int N, uint16_t* hp, void* workspace, size_t workspace_bytes, void* stream);
int sf_o_proj_post_norm(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo, int BN, int K,
                        int D, const int32_t* slot, const uint16_t* ln_w, float eps, uint16_t* hp,
                        uint16_t* zn, void* workspace, size_t workspace_bytes, void* stream);
int sf_residual_post_norm(const uint16_t* x, const uint16_t* y, const int32_t* slot, int BN,
                          int D, const uint16_t* w, float eps, uint16_t* hp, uint16_t* zn,
                          void* stream);
int sf_rows_rmsnorm(const uint16_t* x, const int32_t* rows, const int32_t* count, int bucket,
                    const uint16_t* w, int D, float eps, uint16_t* out, void* stream);
int sf_ffn_gate_up(const uint16_t* zn, const int32_t* count, int bucket, const uint16_t* wg,
                   const uint16_t* wu, int D, int I, uint16_t* act, void* workspace,
                   size_t workspace_bytes, void* stream);
int sf_ffn_down_scatter(const uint16_t* act, const int32_t* count, int bucket, const int32_t* rows,
                        const uint16_t* wd, int I, int D, uint16_t* ffn, void* workspace,
                        size_t workspace_bytes, void* stream);
int sf_residual_gather_add(const uint16_t* hp, const uint16_t* ffn, const int32_t* src, int B1,
                           int N, int D, uint16_t* out, void* stream);
int sf_lm_head(const uint16_t* x, int M, const uint16_t* w, int D, int V, uint16_t* logits,
               void* stream);

/*
 * (8) Output head of the verify step, with Fast-dLLM's logit shift in its stores.
 * logits = x . Wlm^T for the M rows of x (the final-norm hidden states of the
 * B1·N block rows), Wlm [V, D] packed by sf_pack_weight, bf16 out, fp32
 * accumulation over D in one fixed order (a row's logits do not depend on M or on
 * the other rows).  shift_n = 0: row m goes to logits row m (NLD,
 * specfold/generate/nld_folded.py:237; sf_lm_head is this with ld_out = V).
 * shift_n = N: x holds blocks of N rows and the output is the reference's
 * _shift_logits(lm_head(norm(h))) (specfold/generate/fastdllm_v2_generation.py:
 * 121-126 applied to specfold/generate/fastdllm_v2_folded.py:222-223): row (b, n)
 * is stored at (b, n + 1), row (b, 0) at (b, 0) and (b, 1), row (b, N - 1) not at
 * all.  Replaces lm_head + _shift_logits, a library GEMM and a copy of the logits.
 * ld_out: the logits row stride in elements (>= V, a multiple of 4).  No workspace.
 * Limits: 1 <= M <= 1024 (one pass over the weights per 256 rows), D % 64 == 0,
 * V % 128 == 0, shift_n == 0 or (shift_n >= 2 and M % shift_n == 0); x and w
 * 16-byte aligned, logits 8-byte aligned.
 */
int sf_head_logits(const uint16_t* x, int M, const uint16_t* w, int D, int V, int shift_n,
                   uint16_t* logits, long long ld_out, void* stream);
/* sf_head_logits for a row window: of every N-row block of x (M % N == 0), only the
 * logits rows of positions [row_lo, row_lo + row_n) are computed and written (the
 * other rows of logits are left as they are); shift != 0: position n's logits come
 * from x row n - 1 of its block (n > 0) or n itself (n = 0), as above.  The rows a
 * decode step reads (the reference loop slices the small block of the main
 * branch and, on a later draft hit, of a cached draft's logits,
 * specfold/generate/fastdllm_v2_generation.py:610-651), so the head does the work
 * of those rows only: at most 128 of them take a pass with half the X bytes and
 * MFMAs per column.  Each row's values equal the full call's bit for bit.
 * sf_head_logits(shift_n) is this with N = shift_n (M without shift), the whole
 * block.  Limits: as sf_head_logits, with 0 <= row_lo, row_n >= 1,
 * row_lo + row_n <= N. */
int sf_head_logits_rows(const uint16_t* x, int M, const uint16_t* w, int D, int V, int N,
                        int shift, int row_lo, int row_n, uint16_t* logits, long long ld_out,
                        void* stream);

/* ---- greedy decoding statistics of logits rows ----------------------------------
 * Replaces, at temperature 0, the top-p sampler of the reference decode loop
 * (specfold/generate/fastdllm_model_executor.py:109-155: sort, softmax, cumsum,
 * scatter, softmax, argmax; called from fastdllm_v2_generation.py:646-676) and the
 * softmax/topk calls of its draft construction (fastdllm_v2_generation.py:430-470,
 * nld_generation.py:105-151; nld transfer: modeling_nemotron_labs_diffusion.py:
 * 835-861).  For each of the M rows of bf16 logits (row stride ld elements), with
 * e_i = exp(l_i - l_max) (fp32) and Z = sum e_i:
 *   top_idx/top_val [M, 8]  the 8 largest logits, value descending then index
 *                           ascending (top_idx[m*8] is torch.argmax's token)
 *   zfull [M]   Z;   conf_full [M] = bf16(1/Z) (the bf16 softmax maximum)
 *   znuc  [M]   the top-p nucleus mass: e summed in descending order up to and
 *               including the first token that carries it past top_p * Z
 *   greedy_tok [M], conf [M]   the argmax of the bf16 nucleus probabilities
 *               bf16(e_i / znuc) (lowest index among equal) and bf16(1/znuc)
 * workspace: sf_logit_stats_workspace_bytes(M) bytes, zero before the first call:
 * its first M * 65536 32-bit counters are value histograms that every call leaves
 * zero again; the rest is scratch each call overwrites before reading.
 * Limits: 8 <= V <= 2096896 (32 slices of at most 8191 8-token vectors), V % 8 == 0,
 * ld % 8 == 0, 16-byte aligned logits, 0 < top_p (top_p >= 1 keeps every token).
 */
size_t sf_logit_stats_workspace_bytes(int M);
int sf_logit_stats(const uint16_t* logits, int M, int V, long long ld, float top_p,
                   int32_t* top_idx, float* top_val, float* zfull, float* znuc,
                   int32_t* greedy_tok, float* conf, float* conf_full, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * sf_logit_stats without a workspace argument: the same kernels and outputs
 * (bit-identical), with the histograms and candidates in a fixed array in device
 * memory that the library holds on each GPU it runs on until the process ends
 * (16 MiB + 32 KiB per GPU).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  It calls no allocating
 * routine; the first call on a device looks the array up, clears it on
 * `stream` and waits for the clear (the current device must be the stream's),
 * so that first call must not be made under stream capture: it returns
 * SF_ERR_CAPTURE there without launching anything.  Make one eager call per
 * device before capturing; later calls may be captured.
 * Limit: M <= sf_logit_stats_noalloc_max_rows() (64), else SF_ERR_SCRATCH.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other host threads) race and must be ordered by the caller.
 */
int sf_logit_stats_noalloc_max_rows(void);
int sf_logit_stats_noalloc(const uint16_t* logits, int M, int V, long long ld, float top_p,
                           int32_t* top_idx, float* top_val, float* zfull, float* znuc,
                           int32_t* greedy_tok, float* conf, float* conf_full, void* stream);

/* ---- one decode-loop iteration's decisions and loop facts -----------------------
 * Replaces, for one sequence, the Fast-dLLM loop's torch sequence after a small
 * block's sampling (specfold/generate/fastdllm_v2_generation.py:660-700: the
 * threshold-or-argmax unmask of the small block and its write into the token
 * state) and the loop's reads of the token state that follow (stop token with no
 * mask before it, masked counts, draft-cache hit, committed count), in one launch.
 * x_t: int64 [L] token state (batch one); the block is its last bl tokens and the
 * tail x_t[plen:] its last L - plen (1 .. bl).  conf (bf16 [sbs], the small
 * block's probabilities), x_1 (int64 [sbs], its sampled tokens), threshold (the
 * loop's threshold rounded to bf16, as torch compares a bf16 tensor with it):
 * with conf given, column k of the small block at block offset s0 is unmasked
 * when it is masked and conf[k] > threshold or k is the first maximum of conf over
 * the masked columns; unmask[k] = 1 then, and x_t takes x_1[k].  conf NULL: no
 * decision, the facts only.  states: n_states (<= 16) device pointers to cached
 * draft states (int64 [bl] each, host array).  facts (int64, out): [stop, block
 * masked count, each small block's masked count (bl / sbs of them), the first
 * state equal to the block or -1 (only when n_states > 0), the unmasked count
 * (only with conf)] -- the torch form's values exactly.
 * Limits: 1 <= bl <= 64, bl % sbs == 0, L - bl <= plen < L.  No counterpart in
 * the reference as a kernel (its loop runs these as separate torch ops).
 */
int sf_decode_facts(int64_t* x_t, int L, int plen, int bl, int sbs, int s0, long long mask_id,
                    long long stop_id, const uint16_t* conf, const int64_t* x_1, float threshold,
                    const int64_t* const* states, int n_states, int8_t* unmask, int64_t* facts,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECFOLD_AMD_H */
