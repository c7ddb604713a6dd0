// The rest of the verify-step layer on the compacted rows: o_proj + residual,
// post-attention RMSNorm, gate/up with fused SiLU*mul, down with scatter to the
// per-row FFN table, the folded rows' residual update, and the lm_head.
//
// Reference semantics (specfold/generate/fastdllm_v2_folded.py):
//   :207-209  hp = x + bf16(O @ Wo^T)                (every row; residual never folded)
//   :211-218  ffn[rbar] = down(bf16(silu(bf16(z Wg^T))) * bf16(z Wu^T)),
//             z = post_attention_layernorm(hp[rbar]); folded rows reuse the parent's ffn
//   :218      h_next = hp + ffn                        (bf16 add)
//   :222-223  logits = lm_head(norm(h))
// Triton counterparts: fused_ln_gateup_silu_kernel and fused_down_residual_scatter_kernel
// (specfold/generate/triton_kernels.py:102-194).
#include <math.h>

#include "sf_gemm_core.h"

namespace {

using namespace sfg;

// hp[r, n] = bf16(x[r, n] + bf16(sum_s part[s, r, n])), 4 columns per thread
__global__ __launch_bounds__(256) void reduce_residual_kernel(
    const float* __restrict__ part, int nsplit, int mcap, int M, int N,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ out) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)M * N / 4;
  if (q >= total) return;
  const size_t e = q * 4;
  const size_t r = e / N, n = e - r * N;
  sf_f32x4 s = *reinterpret_cast<const sf_f32x4*>(part + r * N + n);
  for (int k = 1; k < nsplit; ++k)
    s += *reinterpret_cast<const sf_f32x4*>(part + ((size_t)k * mcap + r) * N + n);
  const sf_u32x2 xv = *reinterpret_cast<const sf_u32x2*>(x + e);
  const float x0 = __uint_as_float(xv[0] << 16), x1 = __uint_as_float(xv[0] & 0xffff0000u);
  const float x2 = __uint_as_float(xv[1] << 16), x3 = __uint_as_float(xv[1] & 0xffff0000u);
  sf_u32x2 o;
  o[0] = sf_pack2(x0 + sf_rbf(s[0]), x1 + sf_rbf(s[1]));
  o[1] = sf_pack2(x2 + sf_rbf(s[2]), x3 + sf_rbf(s[3]));
  *reinterpret_cast<sf_u32x2*>(out + e) = o;
}

// out[rows[m], n] = bf16(sum_s part[s, m, n]) for m < count
__global__ __launch_bounds__(256) void reduce_scatter_kernel(
    const float* __restrict__ part, int nsplit, int mcap, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int N, uint16_t* __restrict__ out) {
  const int M = min(*count_p, mcap);
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)M * N / 4;
  if (q >= total) return;
  const size_t e = q * 4;
  const size_t m = e / N, n = e - m * N;
  sf_f32x4 s = *reinterpret_cast<const sf_f32x4*>(part + m * N + n);
  for (int k = 1; k < nsplit; ++k)
    s += *reinterpret_cast<const sf_f32x4*>(part + ((size_t)k * mcap + m) * N + n);
  sf_u32x2 o;
  o[0] = sf_pack2(s[0], s[1]);
  o[1] = sf_pack2(s[2], s[3]);
  *reinterpret_cast<sf_u32x2*>(out + (size_t)rows[m] * N + n) = o;
}

// Qwen2RMSNorm of compacted rows: out[m] = bf16(w * bf16(x[rows[m]] * rstd)); one wave per row.
template <int VPL>
__global__ __launch_bounds__(256) void rows_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int mcap, const uint16_t* __restrict__ w, int D,
    float eps, uint16_t* __restrict__ out) {
  const int M = min(*count_p, mcap);
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  const int nvec = D >> 3;
  const sf_u32x4* xr = reinterpret_cast<const sf_u32x4*>(x + (size_t)rows[m] * D);
  sf_u32x4 xv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (lane + i * 64 < nvec) xv[i] = xr[lane + i * 64];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (lane + i * 64 < nvec) {
      float f[8];
      sf_unpack8(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(f[j], f[j], ss);
    }
  }
  ss = sf_wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  const sf_u32x4* wr = reinterpret_cast<const sf_u32x4*>(w);
  sf_u32x4* orow = reinterpret_cast<sf_u32x4*>(out + (size_t)m * D);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = lane + i * 64;
    if (idx < nvec) {
      float f[8], g[8];
      sf_unpack8(xv[i], f);
      sf_unpack8(wr[idx], g);
      sf_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = sf_pack2(g[2 * j] * sf_rbf(f[2 * j] * inv), g[2 * j + 1] * sf_rbf(f[2 * j + 1] * inv));
      orow[idx] = o;
    }
  }
}

// h[r, :] = bf16(hp[r, :] + ffn[src[r]*N + n, :]); 8 elements per thread
__global__ __launch_bounds__(256) void residual_gather_add_kernel(
    const uint16_t* __restrict__ hp, const uint16_t* __restrict__ ffn,
    const int32_t* __restrict__ src, int BN, int N, int D, uint16_t* __restrict__ out) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int per_row = D / 8;
  if (q >= (size_t)BN * per_row) return;
  const int r = (int)(q / per_row);
  const int c = (int)(q - (size_t)r * per_row) * 8;
  const int n = r % N;
  const int fr = src[r] * N + n;
  float a[8], b[8];
  sf_unpack8(*reinterpret_cast<const sf_u32x4*>(hp + (size_t)r * D + c), a);
  sf_unpack8(*reinterpret_cast<const sf_u32x4*>(ffn + (size_t)fr * D + c), b);
  sf_u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = sf_pack2(a[2 * j] + b[2 * j], a[2 * j + 1] + b[2 * j + 1]);
  *reinterpret_cast<sf_u32x4*>(out + (size_t)r * D + c) = o;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t sf_gemm_workspace_bytes(int mcap, int N, int K) {
  if (mcap < 1 || N < 64 || K < kKC) return 0;
  const int mblocks = (mcap + kMB - 1) / kMB;
  const int ns = pick_nsplit(N / 64, K, mblocks);
  return (size_t)ns * mcap * N * sizeof(float);
}

extern "C" int sf_o_proj_residual(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo,
                                  int M, int K, int N, uint16_t* hp, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (!o_bf || !x || !wo || !hp || !workspace) return SF_ERR_ARG;
  if (M < 1 || M > 1024 || K % kKC || N % 64 || !aligned16(o_bf) || !aligned16(wo))
    return SF_ERR_SHAPE;
  if (workspace_bytes < sf_gemm_workspace_bytes(M, N, K)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int mblocks = (M + kMB - 1) / kMB;
  const int ns = pick_nsplit(N / 64, K, mblocks);
  float* part = reinterpret_cast<float*>(workspace);
  launch_gemm<1, kPartial>(o_bf, nullptr, K, nullptr, M, M, wo, nullptr, K, N, ns, part, nullptr,
                           0, st);
  const size_t total = (size_t)M * N / 4;
  hipLaunchKernelGGL(reduce_residual_kernel, dim3((total + 255) / 256), dim3(256), 0, st, part, ns,
                     M, M, N, x, hp);
  return sf_launch_status();
}

extern "C" int sf_rows_rmsnorm(const uint16_t* x, const int32_t* rows, const int32_t* count,
                               int bucket, const uint16_t* w, int D, float eps, uint16_t* out,
                               void* stream) {
  if (!x || !rows || !count || !w || !out) return SF_ERR_ARG;
  if (bucket < 1 || D % 8 || D > 8192) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vpl = (D / 8 + 63) / 64;
  dim3 grid((bucket + 3) / 4);
  if (vpl <= 4)
    hipLaunchKernelGGL(rows_rmsnorm_kernel<4>, grid, dim3(256), 0, st, x, rows, count, bucket, w,
                       D, eps, out);
  else if (vpl <= 8)
    hipLaunchKernelGGL(rows_rmsnorm_kernel<8>, grid, dim3(256), 0, st, x, rows, count, bucket, w,
                       D, eps, out);
  else
    hipLaunchKernelGGL(rows_rmsnorm_kernel<16>, grid, dim3(256), 0, st, x, rows, count, bucket, w,
                       D, eps, out);
  return sf_launch_status();
}

extern "C" int sf_ffn_gate_up(const uint16_t* zn, const int32_t* count, int bucket,
                              const uint16_t* wg, const uint16_t* wu, int D, int I,
                              uint16_t* act, void* stream) {
  if (!zn || !count || !wg || !wu || !act) return SF_ERR_ARG;
  if (bucket < 1 || bucket > 1024 || D % kKC || I % 64) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  launch_gemm<2, kSiluMul>(zn, nullptr, D, count, 0, bucket, wg, wu, D, I, 1, nullptr, act, I, st);
  return sf_launch_status();
}

extern "C" int sf_ffn_down_scatter(const uint16_t* act, const int32_t* count, int bucket,
                                   const int32_t* rows, const uint16_t* wd, int I, int D,
                                   uint16_t* ffn, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (!act || !count || !rows || !wd || !ffn || !workspace) return SF_ERR_ARG;
  if (bucket < 1 || bucket > 1024 || I % kKC || D % 64) return SF_ERR_SHAPE;
  if (workspace_bytes < sf_gemm_workspace_bytes(bucket, D, I)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int mblocks = (bucket + kMB - 1) / kMB;
  const int ns = pick_nsplit(D / 64, I, mblocks);
  float* part = reinterpret_cast<float*>(workspace);
  launch_gemm<1, kPartial>(act, nullptr, I, count, 0, bucket, wd, nullptr, I, D, ns, part,
                           nullptr, 0, st);
  const size_t total = (size_t)bucket * D / 4;
  hipLaunchKernelGGL(reduce_scatter_kernel, dim3((total + 255) / 256), dim3(256), 0, st, part, ns,
                     bucket, rows, count, D, ffn);
  return sf_launch_status();
}

extern "C" int sf_residual_gather_add(const uint16_t* hp, const uint16_t* ffn, const int32_t* src,
                                      int B1, int N, int D, uint16_t* out, void* stream) {
  if (!hp || !ffn || !src || !out) return SF_ERR_ARG;
  if (B1 < 1 || N < 1 || D % 8) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t total = (size_t)B1 * N * D / 8;
  hipLaunchKernelGGL(residual_gather_add_kernel, dim3((total + 255) / 256), dim3(256), 0, st, hp,
                     ffn, src, B1 * N, N, D, out);
  return sf_launch_status();
}

extern "C" int sf_lm_head(const uint16_t* x, int M, const uint16_t* w, int D, int V,
                          uint16_t* logits, void* stream) {
  if (!x || !w || !logits) return SF_ERR_ARG;
  if (M < 1 || M > 1024 || D % kKC || V % 64) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (V % 128 == 0)
    launch_gemm<2, kBf16>(x, nullptr, D, nullptr, M, M, w, nullptr, D, V, 1, nullptr, logits, V,
                          st);
  else
    launch_gemm<1, kBf16>(x, nullptr, D, nullptr, M, M, w, nullptr, D, V, 1, nullptr, logits, V,
                          st);
  return sf_launch_status();
}
