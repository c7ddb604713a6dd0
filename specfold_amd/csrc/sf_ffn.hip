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
#include "sf_gemm_rows.h"

namespace {

using namespace sfg;

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
  const sf_u32x4* wr = reinterpret_cast<const sf_u32x4*>(w);
  // all loads first (clamped addresses, no branches): one memory latency per wave
  sf_u32x4 xv[VPL], wv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) wv[i] = wr[min(lane + i * 64, nvec - 1)];
#pragma unroll
  for (int i = 0; i < VPL; ++i) xv[i] = xr[min(lane + i * 64, nvec - 1)];
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
  sf_u32x4* orow = reinterpret_cast<sf_u32x4*>(out + (size_t)m * D);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = lane + i * 64;
    if (idx < nvec) {
      float f[8], g[8];
      sf_unpack8(xv[i], f);
      sf_unpack8(wv[i], g);
      sf_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = sf_pack2(g[2 * j] * sf_rbf(f[2 * j] * inv), g[2 * j + 1] * sf_rbf(f[2 * j + 1] * inv));
      orow[idx] = o;
    }
  }
}

// One wave per flat row r: hp[r] = bf16(x[r] + y[r]) (the attention residual,
// fastdllm_v2_folded.py:207-209, with y = bf16(O . Wo^T)), and for a recomputed
// row (slot[r] >= 0) its post-attention RMSNorm zn[slot[r]] = bf16(w * bf16(hp[r] *
// rstd)) (:211-212).  All loads are issued before the first use.
template <int VPL>
__global__ __launch_bounds__(256) void residual_post_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
    const int32_t* __restrict__ slot, int BN, int D, const uint16_t* __restrict__ w, float eps,
    uint16_t* __restrict__ hp, uint16_t* __restrict__ zn) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= BN) return;
  const int nvec = D >> 3;
  const sf_u32x4* xr = reinterpret_cast<const sf_u32x4*>(x + (size_t)r * D);
  const sf_u32x4* yr = reinterpret_cast<const sf_u32x4*>(y + (size_t)r * D);
  const sf_u32x4* wr = reinterpret_cast<const sf_u32x4*>(w);
  const int sl = slot[r];
  sf_u32x4 xv[VPL], yv[VPL], wv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) xv[i] = xr[min(lane + i * 64, nvec - 1)];
#pragma unroll
  for (int i = 0; i < VPL; ++i) yv[i] = yr[min(lane + i * 64, nvec - 1)];
#pragma unroll
  for (int i = 0; i < VPL; ++i) wv[i] = wr[min(lane + i * 64, nvec - 1)];
  sf_u32x4* hrow = reinterpret_cast<sf_u32x4*>(hp + (size_t)r * D);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float a[8], b[8];
    sf_unpack8(xv[i], a);
    sf_unpack8(yv[i], b);
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[i][j] = sf_pack2(a[2 * j] + b[2 * j], a[2 * j + 1] + b[2 * j + 1]);
    if (lane + i * 64 < nvec) {
      hrow[lane + i * 64] = xv[i];
      float h[8];
      sf_unpack8(xv[i], h);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(h[j], h[j], ss);
    }
  }
  if (sl < 0) return;  // wave-uniform
  ss = sf_wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  sf_u32x4* orow = reinterpret_cast<sf_u32x4*>(zn + (size_t)sl * D);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = lane + i * 64;
    if (idx < nvec) {
      float f[8], g[8];
      sf_unpack8(xv[i], f);
      sf_unpack8(wv[i], g);
      sf_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = sf_pack2(g[2 * j] * sf_rbf(f[2 * j] * inv), g[2 * j + 1] * sf_rbf(f[2 * j + 1] * inv));
      orow[idx] = o;
    }
  }
}

// The o_proj residual from the all-rows GEMM's KS fp32 partial slots, one
// 512-thread workgroup per flat row r: y = bf16(sum_s part[s][r]) in slot order,
// hp[r] = bf16(x[r] + y) (fastdllm_v2_folded.py:207-209), and with zn given, for a
// recomputed row (slot[r] >= 0), zn[slot[r]] = bf16(w * bf16(hp[r] * rstd))
// (:211-212).  Thread t takes vectors of 8 t, t + 512, ... (VPT of them: one at
// D = 3584, against two with 256 threads, which measured ~0.5 us slower per
// launch); every load of the row (x, the norm weights, up to 4 slots of partials)
// is in flight at once, so a row costs one memory round trip per 4 slots.  hp
// stays in registers for the norm; the sum of squares is reduced per wave, then
// over the 8 waves in wave order.
constexpr int kPrnThreads = 512;
template <int VPT>
__global__ __launch_bounds__(kPrnThreads) void part_residual_norm_kernel(
    const float* __restrict__ part, int ks, size_t stride, const uint16_t* __restrict__ x,
    const int32_t* __restrict__ slot, int D, const uint16_t* __restrict__ w, float eps,
    uint16_t* __restrict__ hp, uint16_t* __restrict__ zn) {
  __shared__ float s_ss[kPrnThreads / 64];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = D >> 3;
  const int sl = zn ? slot[r] : -1;  // workgroup-uniform
  const sf_u32x4* xr = reinterpret_cast<const sf_u32x4*>(x + (size_t)r * D);
  const sf_f32x4* pr = reinterpret_cast<const sf_f32x4*>(part + (size_t)r * D);
  const size_t st4 = stride / 4;  // slot stride in float4
  int v[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) v[i] = min(tid + i * kPrnThreads, nvec - 1);
  // the row's x, norm weights and its first four K-range slots in one round of
  // loads (clamped slots, added in slot order below), further slots four at a time
  constexpr int kSl = 4;
  sf_u32x4 xv[VPT], wv[VPT];
  sf_f32x4 y[VPT][2];
  sf_f32x4 a0[kSl][VPT][2];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    xv[i] = xr[v[i]];
    wv[i] = zn ? reinterpret_cast<const sf_u32x4*>(w)[v[i]] : sf_u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kSl; ++j) {
    const size_t o = (size_t)min(j, ks - 1) * st4;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      a0[j][i][0] = sf_handoff_load(pr + o + 2 * v[i]);
      a0[j][i][1] = sf_handoff_load(pr + o + 2 * v[i] + 1);
    }
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    y[i][0] = a0[0][i][0];
    y[i][1] = a0[0][i][1];
  }
#pragma unroll
  for (int j = 1; j < kSl; ++j)
    if (j < ks) {
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        y[i][0] += a0[j][i][0];
        y[i][1] += a0[j][i][1];
      }
    }
  for (int s0 = kSl; s0 < ks; s0 += 4) {
    sf_f32x4 a[4][VPT][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const size_t o = (size_t)min(s0 + j, ks - 1) * st4;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        a[j][i][0] = sf_handoff_load(pr + o + 2 * v[i]);
        a[j][i][1] = sf_handoff_load(pr + o + 2 * v[i] + 1);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (s0 + j < ks) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
          y[i][0] += a[j][i][0];
          y[i][1] += a[j][i][1];
        }
      }
  }
  sf_u32x4* hrow = reinterpret_cast<sf_u32x4*>(hp + (size_t)r * D);
  sf_u32x4 hv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    float a[8];
    sf_unpack8(xv[i], a);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float y0 = sf_rbf(y[i][j >> 1][(2 * j) & 3]);
      const float y1 = sf_rbf(y[i][j >> 1][(2 * j + 1) & 3]);
      hv[i][j] = sf_pack2(a[2 * j] + y0, a[2 * j + 1] + y1);
    }
    if (tid + i * kPrnThreads < nvec) {
      sf_handoff_store(&hrow[tid + i * kPrnThreads], hv[i]);
      float h[8];
      sf_unpack8(hv[i], h);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(h[j], h[j], ss);
    }
  }
  if (sl < 0) return;  // workgroup-uniform: no barrier is skipped by part of it
  ss = sf_wave_sum(ss);
  if ((tid & 63) == 0) s_ss[tid >> 6] = ss;
  __syncthreads();
  float tot = s_ss[0];
#pragma unroll
  for (int k = 1; k < kPrnThreads / 64; ++k) tot += s_ss[k];
  const float inv = 1.0f / sqrtf(tot / (float)D + eps);
  sf_u32x4* orow = reinterpret_cast<sf_u32x4*>(zn + (size_t)sl * D);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = tid + i * kPrnThreads;
    if (idx < nvec) {
      float f[8], g[8];
      sf_unpack8(hv[i], f);
      sf_unpack8(wv[i], g);
      sf_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = sf_pack2(g[2 * j] * sf_rbf(f[2 * j] * inv), g[2 * j + 1] * sf_rbf(f[2 * j + 1] * inv));
      sf_handoff_store(&orow[idx], o);
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

// The fix-ups below take 8 rows x 128 columns per workgroup (one 4-column group
// per thread): grid (column tiles, ceil(mcap / 8)); row blocks past the device-side
// row count exit at once.
constexpr int kFixRows = 8;

// Fix-up of the FFN down GEMM: tiles computed by several stream-K workgroups are
// summed from their partial slots in slot order and scattered as bf16 rows
// (tiles of a single workgroup were written by the GEMM itself).
__global__ __launch_bounds__(256) void down_fixup_kernel(const float* __restrict__ part, Plan plan,
                                                         int mcap, const int32_t* __restrict__ rows,
                                                         const int32_t* __restrict__ count_p, int N,
                                                         uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int first = tile_first(t, plan);
  const int nsl = tile_last(t, plan) - first + 1;
  if (nsl == 1) return;
  const int M = min(*count_p, mcap);
  const int m = blockIdx.y * kFixRows + (threadIdx.x >> 5);
  if (m >= M) return;
  const size_t stride = (size_t)mcap * N;
  const int c = t * 128 + (threadIdx.x & 31) * 4;
  const int row = rows[m];
  const sf_f32x4 y = sum_slots<sf_f32x4, 12>(part + (size_t)m * N + c, stride, nsl);
  sf_u32x2 o;
  o[0] = sf_pack2(y[0], y[1]);
  o[1] = sf_pack2(y[2], y[3]);
  sf_handoff_store(reinterpret_cast<sf_u32x2*>(out + (size_t)row * N + c), o);
}

// Fix-up of the gate/up GEMM: a 128-column tile computed by several workgroups has
// its gate and up sums in partial slot rows of 2I columns (gate, then up); they
// are summed in slot order and the SiLU*mul epilogue applied, with the same three
// bf16 roundings as the GEMM's own epilogue.
__global__ __launch_bounds__(256) void silu_fixup_kernel(const float* __restrict__ part, Plan plan,
                                                         int mcap, const int32_t* __restrict__ count_p,
                                                         int I, uint16_t* __restrict__ act) {
  const int t = blockIdx.x;
  const int first = tile_first(t, plan);
  const int nsl = tile_last(t, plan) - first + 1;
  if (nsl == 1) return;
  const int M = min(*count_p, mcap);
  const size_t stride = (size_t)mcap * 2 * I;
  {
    const int m = blockIdx.y * kFixRows + (threadIdx.x >> 5);
    if (m >= M) return;
    const int c = t * 128 + (threadIdx.x & 31) * 4;
    const float* p = part + (size_t)m * 2 * I + c;
    const sf_f32x4 g = sum_slots<sf_f32x4>(p, stride, nsl);
    const sf_f32x4 u = sum_slots<sf_f32x4>(p + I, stride, nsl);
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float gt = sf_rbf(g[i]);
      r[i] = sf_rbf(gt / (1.0f + expf(-gt))) * sf_rbf(u[i]);
    }
    sf_u32x2 o;
    o[0] = sf_pack2(r[0], r[1]);
    o[1] = sf_pack2(r[2], r[3]);
    sf_handoff_store(reinterpret_cast<sf_u32x2*>(act + (size_t)m * I + c), o);
  }
}

// Row-major W [N, K] -> the packed fragment-major layout of the GEMM core: 16-byte
// word (tile t, chunk c, lane l) = W[16t + l%16][32c + 8(l/16) .. +8].  One thread
// per 16-byte word, reads gathered, writes sequential.
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ w, int N,
                                                          int K, uint16_t* __restrict__ out) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t nwords = (size_t)N * K / 8;
  if (q >= nwords) return;
  const int l = (int)(q & 63);
  const size_t tc = q >> 6;                 // tile * (K/32) + chunk
  const int chunks = K / 32;
  const size_t t = tc / chunks;
  const int c = (int)(tc - t * chunks);
  const size_t row = t * 16 + (l & 15);
  const size_t k = (size_t)c * 32 + (l >> 4) * 8;
  *reinterpret_cast<sf_u32x4*>(out + q * 8) = *reinterpret_cast<const sf_u32x4*>(w + row * K + k);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The gate/up split.  With at least two 16-column units per workgroup of the
// grid (and at most eight), the column-spread plan: every workgroup streams its
// units over all of K (cfg3: 1184 units, 5 each over 237 workgroups), so no tile
// is shared -- no partial slots, no fix-up launch -- and every CU streams the same
// share of the weights.  Narrower outputs are dealt out stream-K.
// FFN down (128-column tiles over D, K = I): each tile cut into whole K ranges
// (split plan) while the tiles are fewer than the grid; stream-K otherwise.
Plan down_plan(int N, int K) {
  const int T = N / 128, S = K / kKC;
  return T < SFG_GRID ? make_plan_split(T, S) : make_plan(T, S);
}

Plan gate_up_plan(int I, int S) {
  const int nu = I / 16;
  if (nu >= 2 * SFG_GRID && nu <= 8 * SFG_GRID)
    return make_plan_spread(nu, S, spread_workgroups(nu, SFG_GRID));
  return make_plan(I / 128, S);
}

}  // namespace

extern "C" size_t sf_gemm_workspace_bytes(int mcap, int N, int K) {
  if (mcap < 1 || N < 128 || N % 128 || K < kKC || K % kKC) return 0;
  const size_t b = part_bytes(down_plan(N, K), mcap, N);
  return b < 256 ? 256 : b;
}

extern "C" size_t sf_ffn_gate_up_workspace_bytes(int bucket, int D, int I) {
  if (bucket < 1 || I < 128 || I % 128 || D < kKC || D % kKC) return 0;
  const size_t b = part_bytes(make_plan(I / 128, D / kKC), bucket, 2 * I);
  return b < 256 ? 256 : b;
}

extern "C" int sf_pack_weight(const uint16_t* w, int N, int K, uint16_t* out, void* stream) {
  if (!w || !out || w == out) return SF_ERR_ARG;
  if (N < 16 || N % 16 || K < kKC || K % kKC || !aligned16(w) || !aligned16(out))
    return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t words = (size_t)N * K / 8;
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st, w,
                     N, K, out);
  return sf_launch_status();
}

// K ranges of o_proj's all-rows GEMM (the partial slots its consumer adds)
constexpr int kOprojMaxSplits = 16;

extern "C" size_t sf_o_proj_workspace_bytes(int M, int N, int K) {
  if (M < 1 || M > 1024 || N < 128 || N % 128 || K < kKC || K % kKC) return 0;
  const int ks = rows_splits<1>(M, N, K, kOprojMaxSplits);
  const size_t b = (size_t)ks * M * N * sizeof(float);
  return b < 256 ? 256 : b;
}

namespace {
// o_proj over every row to the workspace's partial slots, then one wave per row
// adds them to the residual (and normalises the recomputed rows when zn is given)
int o_proj_launch(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo, int M, int K, int N,
                  const int32_t* slot, const uint16_t* ln_w, float eps, uint16_t* hp,
                  uint16_t* zn, void* workspace, hipStream_t st) {
  float* part = reinterpret_cast<float*>(workspace);
  launch_rows<1, kRowsPart>(o_bf, M, wo, K, N, kOprojMaxSplits, part, nullptr, st);
  const int ks = rows_splits<1>(M, N, K, kOprojMaxSplits);
  const size_t stride = (size_t)M * N;
  const int vpt = (N / 8 + kPrnThreads - 1) / kPrnThreads;
  const dim3 grid(M);
  if (vpt <= 1)
    hipLaunchKernelGGL(part_residual_norm_kernel<1>, grid, dim3(kPrnThreads), 0, st, part, ks,
                       stride, x, slot, N, ln_w, eps, hp, zn);
  else if (vpt <= 2)
    hipLaunchKernelGGL(part_residual_norm_kernel<2>, grid, dim3(kPrnThreads), 0, st, part, ks,
                       stride, x, slot, N, ln_w, eps, hp, zn);
  else
    hipLaunchKernelGGL(part_residual_norm_kernel<4>, grid, dim3(kPrnThreads), 0, st, part, ks,
                       stride, x, slot, N, ln_w, eps, hp, zn);
  return sf_launch_status();
}
}  // namespace

extern "C" int sf_o_proj_residual(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo,
                                  int M, int K, int N, uint16_t* hp, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (!o_bf || !x || !wo || !hp || !workspace) return SF_ERR_ARG;
  if (M < 1 || M > 1024 || K < kKC || K % kKC || N < 128 || N % 128 || N > 8192 ||
      !aligned16(o_bf) || !aligned16(wo) || !aligned16(x) || !aligned16(hp) ||
      !aligned16(workspace))
    return SF_ERR_SHAPE;
  if (workspace_bytes < sf_o_proj_workspace_bytes(M, N, K)) return SF_ERR_WORKSPACE;
  return o_proj_launch(o_bf, x, wo, M, K, N, nullptr, nullptr, 0.f, hp, nullptr, workspace,
                       reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sf_o_proj_post_norm(const uint16_t* o_bf, const uint16_t* x, const uint16_t* wo,
                                   int BN, int K, int D, const int32_t* slot, const uint16_t* ln_w,
                                   float eps, uint16_t* hp, uint16_t* zn, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!o_bf || !x || !wo || !slot || !ln_w || !hp || !zn || !workspace) return SF_ERR_ARG;
  if (BN < 1 || BN > 1024 || K < kKC || K % kKC || D < 128 || D % 128 || D > 8192 ||
      !aligned16(o_bf) || !aligned16(wo) || !aligned16(x) || !aligned16(hp) || !aligned16(zn) ||
      !aligned16(ln_w) || !aligned16(workspace))
    return SF_ERR_SHAPE;
  if (workspace_bytes < sf_o_proj_workspace_bytes(BN, D, K)) return SF_ERR_WORKSPACE;
  return o_proj_launch(o_bf, x, wo, BN, K, D, slot, ln_w, eps, hp, zn, workspace,
                       reinterpret_cast<hipStream_t>(stream));
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

extern "C" int sf_residual_post_norm(const uint16_t* x, const uint16_t* y, const int32_t* slot,
                                     int BN, int D, const uint16_t* w, float eps, uint16_t* hp,
                                     uint16_t* zn, void* stream) {
  if (!x || !y || !slot || !w || !hp || !zn) return SF_ERR_ARG;
  if (BN < 1 || BN > 1024 || D % 8 || D > 8192) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vpl = (D / 8 + 63) / 64;
  dim3 grid((BN + 3) / 4);
  if (vpl <= 4)
    hipLaunchKernelGGL(residual_post_norm_kernel<4>, grid, dim3(256), 0, st, x, y, slot, BN, D, w,
                       eps, hp, zn);
  else if (vpl <= 8)
    hipLaunchKernelGGL(residual_post_norm_kernel<8>, grid, dim3(256), 0, st, x, y, slot, BN, D, w,
                       eps, hp, zn);
  else
    hipLaunchKernelGGL(residual_post_norm_kernel<16>, grid, dim3(256), 0, st, x, y, slot, BN, D, w,
                       eps, hp, zn);
  return sf_launch_status();
}

extern "C" int sf_ffn_gate_up(const uint16_t* zn, const int32_t* count, int bucket,
                              const uint16_t* wg, const uint16_t* wu, int D, int I,
                              uint16_t* act, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!zn || !count || !wg || !wu || !act || !workspace) return SF_ERR_ARG;
  if (bucket < 1 || bucket > 1024 || D % kKC || I % 128) return SF_ERR_SHAPE;
  if (workspace_bytes < sf_ffn_gate_up_workspace_bytes(bucket, D, I)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan p = gate_up_plan(I, D / kKC);
  float* part = reinterpret_cast<float*>(workspace);
  Epi ep{};
  ep.out = act;
  ep.ldo = I;
  // whole tiles get SiLU*mul straight from registers, shared tiles in the fix-up
  launch_sk<2, kSilu>(p, zn, nullptr, D, count, 0, bucket, wg, wu, D, I, part, ep, st);
  if (p.U < p.S)
    hipLaunchKernelGGL(silu_fixup_kernel, dim3(p.T, (bucket + kFixRows - 1) / kFixRows), dim3(256),
                       0, st, part, p, bucket, count, I, act);
  return sf_launch_status();
}

extern "C" int sf_ffn_down_scatter(const uint16_t* act, const int32_t* count, int bucket,
                                   const int32_t* rows, const uint16_t* wd, int I, int D,
                                   uint16_t* ffn, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (!act || !count || !rows || !wd || !ffn || !workspace) return SF_ERR_ARG;
  if (bucket < 1 || bucket > 1024 || I % kKC || D % 128) return SF_ERR_SHAPE;
  if (workspace_bytes < sf_gemm_workspace_bytes(bucket, D, I)) return SF_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan p = down_plan(D, I);
  float* part = reinterpret_cast<float*>(workspace);
  Epi ep{};
  ep.rows = rows;
  ep.out = ffn;
  ep.ldo = D;
  launch_sk<1, kScatter>(p, act, nullptr, I, count, 0, bucket, wd, nullptr, I, D, part, ep, st);
  hipLaunchKernelGGL(down_fixup_kernel, dim3(p.T, (bucket + kFixRows - 1) / kFixRows), dim3(256), 0,
                     st, part, p, bucket, rows, count, D, ffn);
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

