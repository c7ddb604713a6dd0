// Chain correction of folded rows.
//
// A folded row (b, n) inherits the query of its nearest recomputing ancestor
// s = src[b*N+n] and that row's softmax state (m0, Z0, O0) over s's keys.  Its
// own keys differ from s's exactly at the entries recomputed by the branches on
// the chain b -> par(b) -> ... -> s (excluding s).  For every such entry e of
// branch c, the old key/value is the one branch par(c) sees at e
// (kv row src[par(c)*N+e]*N+e) and the new one is c's own.  Then
//   m  = max(m0, max_new q.k_new*scaling)
//   Z  = Z0*exp(m0-m) + sum (a_new - a_old),  a = exp(q.k*scaling - m)
//   O  = (O0*Z0*exp(m0-m) + sum (a_new v_new - a_old v_old)) / Z
// which is exact softmax attention over the branch's keys.  This is the
// telescoped, order-free form of the reference's per-branch one-hop update
// (specfold/generate/fastdllm_v2_folded.py:183-204); the entry loop order and
// accumulation follow specfold/generate/triton_kernels.py:364-429.
//
// One wave per (folded row, kv head); lane = g*8 + c owns dims c*16..c*16+15 of
// q-head g of that kv head (G <= 8), so the G dot products of an entry reduce
// over 8 lanes in parallel.  Entries of a chain are visited in hop order
// (b, par(b), ...) and, within a branch, in ascending position.
#include <math.h>

#include "sf_common.h"

namespace {

constexpr int kHD = 128;

SF_DEV void load16(const uint16_t* p, float out[16]) {
  sf_unpack8(*reinterpret_cast<const sf_u32x4*>(p), out);
  sf_unpack8(*reinterpret_cast<const sf_u32x4*>(p + 8), out + 8);
}

SF_DEV float dot16_group8(const float a[16], const float b[16]) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) d = fmaf(a[i], b[i], d);
  d += __shfl_xor(d, 1, 64);
  d += __shfl_xor(d, 2, 64);
  d += __shfl_xor(d, 4, 64);
  return d;
}

constexpr int kMaxBN = 1024;
constexpr int kMaxB1 = 64;
constexpr int kBatch1 = 8;  // chain entries whose new keys are loaded together (pass 1)
constexpr int kBatch2 = 4;  // chain entries whose old and new K/V are loaded together (pass 2)

SF_DEV void load16w(const uint16_t* p, sf_u32x4 w[2]) {
  w[0] = *reinterpret_cast<const sf_u32x4*>(p);
  w[1] = *reinterpret_cast<const sf_u32x4*>(p + 8);
}

SF_DEV void unpack16(const sf_u32x4 w[2], float out[16]) {
  sf_unpack8(w[0], out);
  sf_unpack8(w[1], out + 8);
}

// The fold tables (src, seg, par, segcnt) are staged in LDS by the whole
// workgroup in one round of loads; each wave then walks its chain from LDS and
// loads the K/V of its chain entries in batches (one memory latency per batch).
__global__ __launch_bounds__(256) void sf_chain_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
    const int32_t* __restrict__ src, const int32_t* __restrict__ par,
    const int8_t* __restrict__ rec, const int32_t* __restrict__ seg,
    const int32_t* __restrict__ segcnt, int B1, int N, int H, int Hkv, float scaling,
    float* __restrict__ o32, uint16_t* __restrict__ o_bf, float* __restrict__ m_tab,
    float* __restrict__ z_tab) {
  __shared__ int s_src[kMaxBN];
  __shared__ int s_seg[kMaxBN];
  __shared__ int s_par[kMaxB1];
  __shared__ int s_cnt[kMaxB1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int BN = B1 * N;
  const int idx = blockIdx.x * 4 + (tid >> 6);
  const bool item = idx < BN * Hkv;
  const int r = item ? idx / Hkv : 0;
  const int h = idx - r * Hkv;

  int tsrc[kMaxBN / 256], tseg[kMaxBN / 256];
#pragma unroll
  for (int k = 0; k < kMaxBN / 256; ++k) {
    const int i = min(tid + 256 * k, BN - 1);
    tsrc[k] = src[i];
    tseg[k] = seg[i];
  }
  const int tpar = par[min(tid, B1 - 1)];
  const int tcnt = segcnt[min(tid, B1 - 1)];
  const bool folded = rec[r] == 0;
#pragma unroll
  for (int k = 0; k < kMaxBN / 256; ++k) {
    if (tid + 256 * k < BN) {
      s_src[tid + 256 * k] = tsrc[k];
      s_seg[tid + 256 * k] = tseg[k];
    }
  }
  if (tid < B1) {
    s_par[tid] = tpar;
    s_cnt[tid] = tcnt;
  }
  __syncthreads();
  if (!item || !folded) return;

  const int G = H / Hkv;
  const int g = lane >> 3;
  const int c = lane & 7;
  const bool gv = g < G;
  const int gq = h * G + (gv ? g : 0);
  const int b = r / N;
  const int n = r - b * N;
  const int s = s_src[r];
  const int sflat = s * N + n;
  const int kvs = 2 * Hkv * kHD;
  const uint16_t* kbase = kv_buf + h * kHD + c * 16;
  const uint16_t* vbase = kv_buf + (Hkv + h) * kHD + c * 16;

  float q[16], o0[16];
  load16(q_buf + (size_t)sflat * H * kHD + gq * kHD + c * 16, q);
  const float* op = o32 + (size_t)sflat * H * kHD + gq * kHD + c * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) o0[i] = op[i];
  const float m0 = m_tab[(size_t)sflat * H + gq];
  const float z0 = z_tab[(size_t)sflat * H + gq];

  // pass 1: the new row max over every entry changed along the chain
  float mn = m0;
  int cur = b;
  for (int hop = 0; hop < B1 && cur != s; ++hop) {
    const int cnt = s_cnt[cur];
    const int* sg = s_seg + cur * N;
    for (int j0 = 0; j0 < cnt; j0 += kBatch1) {
      sf_u32x4 kw[kBatch1][2];
#pragma unroll
      for (int u = 0; u < kBatch1; ++u) load16w(kbase + (size_t)sg[min(j0 + u, cnt - 1)] * kvs, kw[u]);
#pragma unroll
      for (int u = 0; u < kBatch1; ++u) {
        if (j0 + u < cnt) {
          float kn[16];
          unpack16(kw[u], kn);
          mn = fmaxf(mn, dot16_group8(q, kn) * scaling);
        }
      }
    }
    cur = s_par[cur];
  }

  // pass 2: rescale the inherited state, then swap old entries for new ones
  float z = z0 * expf(m0 - mn);
  float num[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) num[i] = o0[i] * z;
  cur = b;
  for (int hop = 0; hop < B1 && cur != s; ++hop) {
    const int pc = s_par[cur];
    const int cnt = s_cnt[cur];
    const int* sg = s_seg + cur * N;
    for (int j0 = 0; j0 < cnt; j0 += kBatch2) {
      sf_u32x4 ko[kBatch2][2], vo[kBatch2][2], kn[kBatch2][2], vn[kBatch2][2];
#pragma unroll
      for (int u = 0; u < kBatch2; ++u) {
        const int rj = sg[min(j0 + u, cnt - 1)];
        const int e = rj % N;
        const size_t old = (size_t)(s_src[pc * N + e] * N + e) * kvs;
        const size_t nw = (size_t)rj * kvs;
        load16w(kbase + old, ko[u]);
        load16w(vbase + old, vo[u]);
        load16w(kbase + nw, kn[u]);
        load16w(vbase + nw, vn[u]);
      }
#pragma unroll
      for (int u = 0; u < kBatch2; ++u) {
        if (j0 + u < cnt) {
          float kof[16], knf[16];
          unpack16(ko[u], kof);
          unpack16(kn[u], knf);
          const float ao = expf(dot16_group8(q, kof) * scaling - mn);
          const float an = expf(dot16_group8(q, knf) * scaling - mn);
          z = z - ao + an;
          float vof[16], vnf[16];
          unpack16(vo[u], vof);
          unpack16(vn[u], vnf);
#pragma unroll
          for (int i = 0; i < 16; ++i) num[i] = num[i] - ao * vof[i] + an * vnf[i];
        }
      }
    }
    cur = pc;
  }

  if (!gv) return;
  const float inv = 1.0f / z;
  const size_t off = (size_t)r * H * kHD + gq * kHD + c * 16;
  float* o = o32 + off;
  sf_u32x4 w0, w1;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = num[i] * inv;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w0[i] = sf_pack2(num[2 * i] * inv, num[2 * i + 1] * inv);
    w1[i] = sf_pack2(num[8 + 2 * i] * inv, num[8 + 2 * i + 1] * inv);
  }
  *reinterpret_cast<sf_u32x4*>(o_bf + off) = w0;
  *reinterpret_cast<sf_u32x4*>(o_bf + off + 8) = w1;
  if (c == 0) {
    m_tab[(size_t)r * H + gq] = mn;
    z_tab[(size_t)r * H + gq] = z;
  }
}

}  // namespace

extern "C" int sf_chain_correct(const uint16_t* q_buf, const uint16_t* kv_buf, const int32_t* src,
                                const int32_t* par, const int8_t* rec, const int32_t* seg,
                                const int32_t* segcnt, int B1, int N, int H, int Hkv, int hd,
                                float scaling, float* o32, uint16_t* o_bf, float* m_tab,
                                float* z_tab, void* stream) {
  if (!q_buf || !kv_buf || !src || !par || !rec || !seg || !segcnt || !o32 || !o_bf || !m_tab ||
      !z_tab)
    return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > 8) return SF_ERR_SHAPE;
  if (B1 < 1 || B1 > 64 || N < 1 || B1 * N > 1024) return SF_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int waves = B1 * N * Hkv;
  hipLaunchKernelGGL(sf_chain_kernel, dim3((waves + 3) / 4), dim3(256), 0, st, q_buf, kv_buf, src,
                     par, rec, seg, segcnt, B1, N, H, Hkv, scaling, o32, o_bf, m_tab, z_tab);
  return sf_launch_status();
}
