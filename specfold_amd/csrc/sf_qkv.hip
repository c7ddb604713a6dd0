// QKV projection of the compacted (recomputed) rows on bf16 MFMA, then bias,
// RoPE and the scatter into the per-flat-row q/kv tables.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:151-161
// (nn.Linear outputs rounded to bf16, RoPE as qf*c + rotate_half(qf)*s with each
// bf16 op rounded) and the Triton kernel specfold/generate/triton_kernels.py:29-87.
//
// GEMM: out[m, c] = sum_k xn[rows[m], k] * w[c, k]; M = count <= bucket,
// N = (H + 2*Hkv)*hd, K = D.  The weight is the large operand (33 MB at the 7B
// shape) and is read exactly once: workgroups tile 64 output columns x one K
// range (split-K), every wave owns 16 columns and streams its weight slice
// straight into VGPRs, while the activation tile (all M rows) is shared
// through LDS.  fp32 partials go to the workspace; a small epilogue sums the
// splits in a fixed order (deterministic), adds the bias, rounds and ropes.
#include "sf_common.h"

namespace {

constexpr int kNT = 64;    // output columns per workgroup (4 waves x 16)
constexpr int kKC = 64;    // K elements per LDS stage
constexpr int kMB = 256;   // rows per M block
constexpr int kLds = 72;   // LDS row stride (bf16): 64 + 8 pad, keeps 16 B reads conflict-light
constexpr int kHD = 128;

int qkv_nsplit(int D, int n_qkv) {
  const int tiles = n_qkv / kNT;
  const int nch = D / kKC;
  int s = (256 + tiles - 1) / tiles;  // >= one workgroup per CU on 256 CUs
  if (s < 1) s = 1;
  if (s > nch) s = nch;
  return s;
}

__global__ __launch_bounds__(256) void sf_qkv_gemm_kernel(
    const uint16_t* __restrict__ xn, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, const uint16_t* __restrict__ w, int D,
    int n_qkv, int nsplit, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][kMB * kLds];
  __shared__ int s_rows[kMB];
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * kMB;
  const int count = min(*count_p, bucket);
  if (m0 >= count) return;
  const int mrows = min(kMB, count - m0);
  const int nmt = (mrows + 15) >> 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int nch = D / kKC;
  const int c0 = split * nch / nsplit;
  const int c1 = (split + 1) * nch / nsplit;

  for (int i = tid; i < mrows; i += 256) s_rows[i] = rows[m0 + i];
  __syncthreads();

  // activation loader: 8 threads x 16 B per row, 32 rows per pass
  const int a_seg = tid & 7;
  const int a_row0 = tid >> 3;
  sf_u32x4 areg[kMB / 32];
  auto load_a = [&](int c) {
#pragma unroll
    for (int ps = 0; ps < kMB / 32; ++ps) {
      const int rr = a_row0 + ps * 32;
      if (rr < mrows)
        areg[ps] = *reinterpret_cast<const sf_u32x4*>(xn + (size_t)s_rows[rr] * D + c * kKC +
                                                      a_seg * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int ps = 0; ps < kMB / 32; ++ps) {
      const int rr = a_row0 + ps * 32;
      if (rr < mrows) *reinterpret_cast<sf_u32x4*>(&sA[buf][rr * kLds + a_seg * 8]) = areg[ps];
    }
  };

  // weight operand: lane holds w[col][k .. k+8], k = chunk + ks*32 + (lane/16)*8
  const int col = tile * kNT + wv * 16 + (lane & 15);
  const int kq = (lane >> 4) * 8;
  const uint16_t* wrow = w + (size_t)col * D + kq;
  sf_u32x4 bcur[2], bnext[2];
  auto load_b = [&](int c, sf_u32x4* bb) {
    bb[0] = *reinterpret_cast<const sf_u32x4*>(wrow + c * kKC);
    bb[1] = *reinterpret_cast<const sf_u32x4*>(wrow + c * kKC + 32);
  };

  sf_f32x4 acc[kMB / 16];
#pragma unroll
  for (int i = 0; i < kMB / 16; ++i) acc[i] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  load_a(c0);
  store_a(0);
  load_b(c0, bcur);
  __syncthreads();
  int buf = 0;
  for (int c = c0; c < c1; ++c) {
    const bool more = c + 1 < c1;
    if (more) {
      load_a(c + 1);
      load_b(c + 1, bnext);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const sf_bf16x8 bfrag = sf_as_bf16x8(bcur[ks]);
      const uint16_t* abase = &sA[buf][(lane & 15) * kLds + ks * 32 + kq];
#pragma unroll
      for (int mt = 0; mt < kMB / 16; ++mt) {
        if (mt < nmt) {
          const sf_u32x4 af = *reinterpret_cast<const sf_u32x4*>(abase + mt * 16 * kLds);
          acc[mt] = sf_mfma16x16x32(sf_as_bf16x8(af), bfrag, acc[mt]);
        }
      }
    }
    if (more) {
      store_a(buf ^ 1);
      bcur[0] = bnext[0];
      bcur[1] = bnext[1];
    }
    __syncthreads();
    buf ^= 1;
  }

  // D layout of 16x16 MFMA: lane holds rows (lane/16)*4 + r, column lane%16
  float* pbase = part + ((size_t)split * bucket + m0) * n_qkv + col;
#pragma unroll
  for (int mt = 0; mt < kMB / 16; ++mt) {
    if (mt < nmt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + (lane >> 4) * 4 + r;
        if (m < mrows) pbase[(size_t)m * n_qkv] = acc[mt][r];
      }
    }
  }
}

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
  if (bucket < 1 || D < kKC || n_qkv < kNT) return 0;
  return (size_t)qkv_nsplit(D, n_qkv) * bucket * n_qkv * sizeof(float);
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
  const int nsplit = qkv_nsplit(D, n_qkv);
  float* part = reinterpret_cast<float*>(workspace);
  dim3 g1(n_qkv / kNT, nsplit, (bucket + kMB - 1) / kMB);
  hipLaunchKernelGGL(sf_qkv_gemm_kernel, g1, dim3(256), 0, st, xn, rows, count, bucket, w_qkv, D,
                     n_qkv, nsplit, part);
  dim3 g2(bucket, H + 2 * Hkv);
  hipLaunchKernelGGL(sf_qkv_epilogue_kernel, g2, dim3(64), 0, st, part, nsplit, bucket, n_qkv, rows,
                     count, b_qkv, cos_tab, sin_tab, q_scale, N, H, Hkv, q_buf, kv_buf);
  return sf_launch_status();
}
