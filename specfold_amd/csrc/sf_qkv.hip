// QKV projection of the compacted (recomputed) rows on bf16 MFMA, then bias,
// RoPE and the scatter into the per-flat-row q/kv tables.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:151-161
// (nn.Linear outputs rounded to bf16, RoPE as qf*c + rotate_half(qf)*s with each
// bf16 op rounded) and the Triton kernel specfold/generate/triton_kernels.py:29-87.
//
// GEMM: out[m, c] = sum_k xn[rows[m], k] * w[c, k]; M = count <= bucket,
// N = (H + 2*Hkv)*hd, K = D, on the stream-K weight-streaming core of
// sf_gemm_core.h with one head (128 columns) per tile, every piece to fp32
// partial slots; the epilogue kernel sums a head's slots in slot order
// (deterministic), adds the bias, rounds, ropes and scatters.
#include "sf_gemm_core.h"

using namespace sfg;

namespace {

// Wave w of workgroup (x, y) handles head 4y + w of compacted rows
// m = x, x + gridDim.x, ... < count; lane t owns dims t and t+64, exactly the pair
// rotate_half mixes.  BRANCHES: the first absolute position is pos0[branch] and
// the q scale q_scale[flat row] (a batched step: each sequence's branches at its
// own prefix length); otherwise *pos0 and q_scale[n] for every row.
template <bool BRANCHES>
__global__ __launch_bounds__(256) void sf_qkv_epilogue_kernel(
    const float* __restrict__ part, Plan plan, int bucket, int n_qkv,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ count_p,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, const int32_t* __restrict__ pos0, int table_rows,
    const float* __restrict__ q_scale, int N, int H, int Hkv, uint16_t* __restrict__ q_buf,
    uint16_t* __restrict__ kv_buf) {
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (head >= H + 2 * Hkv) return;
  const int t = threadIdx.x & 63;
  const int c0 = head * 128 + t;
  const int c1 = c0 + 64;
  const int nsl = tile_last(head, plan) - tile_first(head, plan) + 1;
  const size_t stride = (size_t)bucket * n_qkv;
  const float b0 = bias ? sf_bf2f(bias[c0]) : 0.f;
  const float b1 = bias ? sf_bf2f(bias[c1]) : 0.f;
  const int count = min(*count_p, bucket);
  const int p0 = (!BRANCHES && pos0) ? *pos0 : 0;
  for (int m = blockIdx.x; m < count; m += gridDim.x) {
    const int row = rows[m];
    const float* ps = part + (size_t)m * n_qkv;
    float y0 = sum_slots<float>(ps + c0, stride, nsl);
    float y1 = sum_slots<float>(ps + c1, stride, nsl);
    const int n = row % N;
    const int pb = BRANCHES ? pos0[row / N] : p0;
    if (bias) {  // (without a bias, a -0 sum stays -0 as in torch)
      y0 += b0;
      y1 += b1;
    }
    y0 = sf_rbf(y0);  // nn.Linear output is a bf16 tensor
    y1 = sf_rbf(y1);
    if (head < H + Hkv) {
      const size_t tr = (size_t)min(max(pb + n, 0), table_rows - 1) * 128;
      const float cs0 = sf_bf2f(cos_tab[tr + t]);
      const float cs1 = sf_bf2f(cos_tab[tr + t + 64]);
      const float sn0 = sf_bf2f(sin_tab[tr + t]);
      const float sn1 = sf_bf2f(sin_tab[tr + t + 64]);
      // rotate_half(y) = (-y1, y0): out = bf16(bf16(y*c) + bf16(rot*s))
      const float o0 = sf_rbf(sf_rbf(y0 * cs0) + sf_rbf(-y1 * sn0));
      const float o1 = sf_rbf(sf_rbf(y1 * cs1) + sf_rbf(y0 * sn1));
      y0 = o0;
      y1 = o1;
      if (head < H && q_scale) {
        const float qs = sf_rbf(q_scale[BRANCHES ? row : n]);
        y0 = sf_rbf(y0 * qs);
        y1 = sf_rbf(y1 * qs);
      }
    }
    uint16_t* dst;
    if (head < H)
      dst = q_buf + (size_t)row * H * 128 + head * 128;
    else
      dst = kv_buf + (size_t)row * 2 * Hkv * 128 + (head - H) * 128;
    dst[t] = sf_f2bf(y0);
    dst[t + 64] = sf_f2bf(y1);
  }
}

}  // namespace

extern "C" size_t sf_qkv_workspace_bytes(int bucket, int D, int n_qkv) {
  if (bucket < 1 || D < kKC || D % kKC || n_qkv < 128 || n_qkv % 128) return 0;
  return part_bytes(make_plan(n_qkv / 128, D / kKC), bucket, n_qkv);
}

extern "C" int sf_qkv_rope(const uint16_t* xn, const int32_t* rows, const int32_t* count,
                           int bucket, int BN, const uint16_t* w_qkv, const uint16_t* b_qkv,
                           const uint16_t* cos_tab, const uint16_t* sin_tab, const int32_t* pos0,
                           int table_rows, const float* q_scale, int N, int D, int H, int Hkv,
                           int hd, uint16_t* q_buf, uint16_t* kv_buf,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (!xn || !rows || !count || !w_qkv || !cos_tab || !sin_tab || !q_buf || !kv_buf || !workspace)
    return SF_ERR_ARG;
  if (hd != 128 || H < 1 || Hkv < 1 || H % Hkv != 0) return SF_ERR_SHAPE;
  if (D < kKC || D % kKC != 0) return SF_ERR_SHAPE;
  if (N < 1 || BN < 1 || bucket < 1 || bucket > BN || bucket > 1024) return SF_ERR_SHAPE;
  if (!pos0) table_rows = N;
  if (table_rows < N) return SF_ERR_SHAPE;
  const int n_qkv = (H + 2 * Hkv) * hd;
  if (workspace_bytes < sf_qkv_workspace_bytes(bucket, D, n_qkv)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan p = make_plan(n_qkv / 128, D / kKC);
  float* part = reinterpret_cast<float*>(workspace);
  launch_sk<1, kPart>(p, xn, rows, D, count, 0, bucket, w_qkv, nullptr, D, n_qkv, part, Epi{}, st);
  dim3 g2(min(bucket, 128), (H + 2 * Hkv + 3) / 4);
  hipLaunchKernelGGL(sf_qkv_epilogue_kernel<false>, g2, dim3(256), 0, st, part, p, bucket, n_qkv, rows,
                     count, b_qkv, cos_tab, sin_tab, pos0, table_rows, q_scale, N, H, Hkv, q_buf,
                     kv_buf);
  return sf_launch_status();
}

// The batched-step variant: one GEMM over the recomputed rows of several
// sequences laid out one after another, the rope and q scale of each branch at its
// own sequence's positions.  pos0_branch: int32 [BN / N], the first absolute
// position of each branch (its sequence's prefix length); q_scale_rows: fp32 [BN]
// or NULL.  No counterpart in the reference (one sequence per verify step).
extern "C" int sf_qkv_rope_branches(const uint16_t* xn, const int32_t* rows,
                                    const int32_t* count, int bucket, int BN,
                                    const uint16_t* w_qkv, const uint16_t* b_qkv,
                                    const uint16_t* cos_tab, const uint16_t* sin_tab,
                                    const int32_t* pos0_branch, int table_rows,
                                    const float* q_scale_rows, int N, int D, int H, int Hkv,
                                    int hd, uint16_t* q_buf, uint16_t* kv_buf, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!xn || !rows || !count || !w_qkv || !cos_tab || !sin_tab || !pos0_branch || !q_buf ||
      !kv_buf || !workspace)
    return SF_ERR_ARG;
  if (hd != 128 || H < 1 || Hkv < 1 || H % Hkv != 0) return SF_ERR_SHAPE;
  if (D < kKC || D % kKC != 0) return SF_ERR_SHAPE;
  if (N < 1 || BN < 1 || BN % N != 0 || bucket < 1 || bucket > BN || bucket > 1024)
    return SF_ERR_SHAPE;
  if (table_rows < N) return SF_ERR_SHAPE;
  const int n_qkv = (H + 2 * Hkv) * hd;
  if (workspace_bytes < sf_qkv_workspace_bytes(bucket, D, n_qkv)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan p = make_plan(n_qkv / 128, D / kKC);
  float* part = reinterpret_cast<float*>(workspace);
  launch_sk<1, kPart>(p, xn, rows, D, count, 0, bucket, w_qkv, nullptr, D, n_qkv, part, Epi{}, st);
  dim3 g2(min(bucket, 128), (H + 2 * Hkv + 3) / 4);
  hipLaunchKernelGGL(sf_qkv_epilogue_kernel<true>, g2, dim3(256), 0, st, part, p, bucket, n_qkv,
                     rows, count, b_qkv, cos_tab, sin_tab, pos0_branch, table_rows, q_scale_rows,
                     N, H, Hkv, q_buf, kv_buf);
  return sf_launch_status();
}

// sf_qkv_rope (pos0_per_branch = 0) or sf_qkv_rope_branches (1) with the fold
// gate's compaction in the GEMM's prologue, for a gate launched with
// SF_GATE_DEFER_COMPACT: every GEMM workgroup compacts rec for its own A rows (one
// launch fewer per layer), and workgroup 0 writes f, src, rows, count, seg, segcnt
// and slot (may be NULL) as sf_fold_gate documents them, for the epilogue and the
// kernels after it.  No counterpart in the reference (its gate and its QKV
// projection are separate launches).
extern "C" int sf_qkv_rope_gated(const uint16_t* xn, const int8_t* rec, const int32_t* par,
                                 int B1, int N, int bucket, int32_t* f, int32_t* src,
                                 int32_t* rows, int32_t* count, int32_t* seg, int32_t* segcnt,
                                 int32_t* slot, const uint16_t* w_qkv, const uint16_t* b_qkv,
                                 const uint16_t* cos_tab, const uint16_t* sin_tab,
                                 const int32_t* pos0, int pos0_per_branch, int table_rows,
                                 const float* q_scale, int D, int H, int Hkv, int hd,
                                 uint16_t* q_buf, uint16_t* kv_buf, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!xn || !rec || !par || !f || !src || !rows || !count || !seg || !segcnt || !w_qkv ||
      !cos_tab || !sin_tab || !q_buf || !kv_buf || !workspace || (pos0_per_branch && !pos0))
    return SF_ERR_ARG;
  if (hd != 128 || H < 1 || Hkv < 1 || H % Hkv != 0) return SF_ERR_SHAPE;
  if (D < kKC || D % kKC != 0) return SF_ERR_SHAPE;
  if (B1 < 1 || B1 > 64 || N < 1 || B1 * N > kGateMaxRows) return SF_ERR_SHAPE;
  if (bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  if (!pos0) table_rows = N;
  if (table_rows < N) return SF_ERR_SHAPE;
  const int n_qkv = (H + 2 * Hkv) * hd;
  if (workspace_bytes < sf_qkv_workspace_bytes(bucket, D, n_qkv)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan p = make_plan(n_qkv / 128, D / kKC);
  float* part = reinterpret_cast<float*>(workspace);
  const GateIn gate{rec, par, B1, N, GateOut{f, src, rows, count, seg, segcnt, slot}};
  launch_sk<1, kPart, true>(p, xn, nullptr, D, nullptr, 0, bucket, w_qkv, nullptr, D, n_qkv, part,
                            Epi{}, st, gate);
  dim3 g2(min(bucket, 128), (H + 2 * Hkv + 3) / 4);
  if (pos0_per_branch)
    hipLaunchKernelGGL(sf_qkv_epilogue_kernel<true>, g2, dim3(256), 0, st, part, p, bucket, n_qkv,
                       rows, count, b_qkv, cos_tab, sin_tab, pos0, table_rows, q_scale, N, H, Hkv,
                       q_buf, kv_buf);
  else
    hipLaunchKernelGGL(sf_qkv_epilogue_kernel<false>, g2, dim3(256), 0, st, part, p, bucket,
                       n_qkv, rows, count, b_qkv, cos_tab, sin_tab, pos0, table_rows, q_scale, N,
                       H, Hkv, q_buf, kv_buf);
  return sf_launch_status();
}
