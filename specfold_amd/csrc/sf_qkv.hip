// QKV projection of the compacted (recomputed) rows on bf16 MFMA, then bias,
// RoPE and the scatter into the per-flat-row q/kv tables.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:151-161
// (nn.Linear outputs rounded to bf16, RoPE as qf*c + rotate_half(qf)*s with each
// bf16 op rounded) and the Triton kernel specfold/generate/triton_kernels.py:29-87.
//
// GEMM: out[m, c] = sum_k xn[rows[m], k] * w[c, k]; M = count <= bucket,
// N = (H + 2*Hkv)*hd, K = D, on the weight-streaming core of sf_gemm_core.h
// (64 columns x one K range per workgroup, split-K so >= 256 workgroups stream
// the 33 MB weight once).  fp32 partials go to the workspace; a small epilogue
// sums the splits in a fixed order (deterministic), adds the bias, rounds and
// ropes.
#include "sf_gemm_core.h"

namespace {

using namespace sfg;

constexpr int kHD = 128;

// One 64-lane workgroup per (compacted row, head); lane t owns dims t and t+64,
// exactly the pair rotate_half mixes.
__global__ __launch_bounds__(64) void sf_qkv_epilogue_kernel(
    const float* __restrict__ part, int nsplit, int bucket, int n_qkv,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ count_p,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, const float* __restrict__ q_scale, int N, int H, int Hkv,
    uint16_t* __restrict__ q_buf, uint16_t* __restrict__ kv_buf) {
  const int m = blockIdx.x;
  const int head = blockIdx.y;
  const int t = threadIdx.x;
  const int count = min(*count_p, bucket);
  if (m >= count) return;
  const int row = rows[m];
  const int n = row % N;
  const int c0 = head * kHD + t;
  const int c1 = c0 + kHD / 2;
  float y0 = 0.f, y1 = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float* ps = part + ((size_t)s * bucket + m) * n_qkv;
    y0 += ps[c0];
    y1 += ps[c1];
  }
  if (bias) {
    y0 += sf_bf2f(bias[c0]);
    y1 += sf_bf2f(bias[c1]);
  }
  y0 = sf_rbf(y0);  // nn.Linear output is a bf16 tensor
  y1 = sf_rbf(y1);
  if (head < H + Hkv) {
    const float cs0 = sf_bf2f(cos_tab[n * kHD + t]);
    const float cs1 = sf_bf2f(cos_tab[n * kHD + t + kHD / 2]);
    const float sn0 = sf_bf2f(sin_tab[n * kHD + t]);
    const float sn1 = sf_bf2f(sin_tab[n * kHD + t + kHD / 2]);
    // rotate_half(y) = (-y1, y0): out = bf16(bf16(y*c) + bf16(rot*s))
    const float o0 = sf_rbf(sf_rbf(y0 * cs0) + sf_rbf(-y1 * sn0));
    const float o1 = sf_rbf(sf_rbf(y1 * cs1) + sf_rbf(y0 * sn1));
    y0 = o0;
    y1 = o1;
    if (head < H && q_scale) {
      const float qs = sf_rbf(q_scale[n]);
      y0 = sf_rbf(y0 * qs);
      y1 = sf_rbf(y1 * qs);
    }
  }
  uint16_t* dst;
  if (head < H)
    dst = q_buf + (size_t)row * H * kHD + head * kHD;
  else
    dst = kv_buf + (size_t)row * 2 * Hkv * kHD + (head - H) * kHD;
  dst[t] = sf_f2bf(y0);
  dst[t + kHD / 2] = sf_f2bf(y1);
}

}  // namespace

extern "C" size_t sf_qkv_workspace_bytes(int bucket, int D, int n_qkv) {
  if (bucket < 1 || D < kKC || n_qkv < 64) return 0;
  const int ns = pick_nsplit(n_qkv / 64, D, (bucket + kMB - 1) / kMB);
  return (size_t)ns * bucket * n_qkv * sizeof(float);
}

extern "C" int sf_qkv_rope(const uint16_t* xn, const int32_t* rows, const int32_t* count,
                           int bucket, int BN, const uint16_t* w_qkv, const uint16_t* b_qkv,
                           const uint16_t* cos_tab, const uint16_t* sin_tab, const float* q_scale,
                           int N, int D, int H, int Hkv, int hd, uint16_t* q_buf, uint16_t* kv_buf,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (!xn || !rows || !count || !w_qkv || !cos_tab || !sin_tab || !q_buf || !kv_buf || !workspace)
    return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0) return SF_ERR_SHAPE;
  if (D < kKC || D % kKC != 0) return SF_ERR_SHAPE;
  if (N < 1 || BN < 1 || bucket < 1 || bucket > BN || bucket > 1024) return SF_ERR_SHAPE;
  const int n_qkv = (H + 2 * Hkv) * hd;
  if (workspace_bytes < sf_qkv_workspace_bytes(bucket, D, n_qkv)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int nsplit = pick_nsplit(n_qkv / 64, D, (bucket + kMB - 1) / kMB);
  float* part = reinterpret_cast<float*>(workspace);
  launch_gemm<1, kPartial>(xn, rows, D, count, 0, bucket, w_qkv, nullptr, D, n_qkv, nsplit, part,
                           nullptr, 0, st);
  dim3 g2(bucket, H + 2 * Hkv);
  hipLaunchKernelGGL(sf_qkv_epilogue_kernel, g2, dim3(64), 0, st, part, nsplit, bucket, n_qkv, rows,
                     count, b_qkv, cos_tab, sin_tab, q_scale, N, H, Hkv, q_buf, kv_buf);
  return sf_launch_status();
}
