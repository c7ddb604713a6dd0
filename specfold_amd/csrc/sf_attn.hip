// Attention of the recomputed rows over [shared prefix ; own branch block],
// emitting the softmax state (m, Z) next to O.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:164-181 (fp32
// scores = (q . k) * scaling, m = max, Z = sum exp(s - m), O = sum exp(s - m) v / Z,
// no mask) and the Triton kernel specfold/generate/triton_kernels.py:301-361.
//
// Two kernels (flash-decoding split over the prefix):
//  * prefix: grid (query tile, 128-key prefix chunk, kv head).  All recomputed
//    rows x the G q-heads of one kv head are flattened to queries qi = m*G + g
//    and tiled 64 per workgroup (16 per wave), so each prefix K/V element is
//    read by the few query tiles of its chunk instead of once per row.  The
//    chunk's page ids are read once into LDS, then every K/V load of the chunk
//    is issued at once (one memory latency per workgroup), K and V^T are staged
//    in LDS, and two 64-key MFMA stages run from LDS.  Scores are formed
//    transposed, S^T = K Q^T, so every lane holds 4 keys of ONE query: the
//    softmax rescale is per lane and P^T feeds the P.V MFMA straight from
//    registers (the 8 k-slots of a lane are keys {4g..4g+3} of two 16-key
//    tiles, and V^T is read in that same order).  P is split into bf16 hi + lo
//    halves (two MFMAs) so P.V keeps ~16 mantissa bits, close to the
//    reference's fp32 einsum.  Each chunk writes its (m, l, acc) partial.
//  * block + merge: one 256-thread workgroup per (recomputed row, kv head):
//    every load (q, the branch's N block keys/values gathered through src, all
//    chunk partials) is issued up front; block scores, the merged max, Z and O
//    follow from LDS.
// The prefix length may come from device memory (p_len), so a captured graph
// of the verify step stays valid while the cache grows; `P` is then the
// capacity the grid and the workspace are sized for.
#include <math.h>

#include "sf_common.h"

namespace {

constexpr int kHD = 128;
constexpr int kQT = 64;      // queries per workgroup
constexpr int kChunk = 128;  // prefix keys per workgroup
constexpr int kKStr = 136;   // K tile row stride (bf16)
constexpr int kVStr = 136;   // V^T tile row stride (bf16): 128 keys + 8 pad
constexpr int kMaxG = 8;
constexpr int kMaxN = 64;

SF_DEV uint32_t bf_at(const sf_u32x4& w, int j) {
  return (w[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

__global__ __launch_bounds__(256) void sf_attn_prefix_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table, int page_size,
    long long page_stride, long long head_stride, const int32_t* __restrict__ p_len, int P_host,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ count_p, int bucket, int H,
    int Hkv, float scaling, int qmax, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kChunk * kKStr];
  __shared__ __attribute__((aligned(16))) uint16_t sV[kHD * kVStr];
  __shared__ int s_page[kChunk];
  const int G = H / Hkv;
  const int qt = blockIdx.x;
  const int ci = blockIdx.y;
  const int h = blockIdx.z;
  const int nchunks = gridDim.y;
  const int P = p_len ? *p_len : P_host;
  const int k_begin = ci * kChunk;
  if (k_begin >= P) return;
  const int k_end = min(P, k_begin + kChunk);
  const int count = min(*count_p, bucket);
  const int nq = count * G;
  if (qt * kQT >= nq) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int grp = lane >> 4;  // 0..3
  const int ql = lane & 15;
  const int qi = qt * kQT + wv * 16 + ql;
  const bool qvalid = qi < nq;
  const long long head_off = (long long)h * head_stride;

  // page ids of the chunk's keys (one per key; pages must not straddle the chunk
  // unevenly, so page_size divides 128 — checked on the host)
  if (tid < kChunk) {
    const int t = k_begin + tid;
    s_page[tid] = (page_table && t < k_end) ? page_table[t / page_size] : 0;
  }
  // Q^T operand: lane holds q[qi][ds*32 + grp*8 .. +8]
  sf_u32x4 qf[4];
  if (qvalid) {
    const int m = qi / G;
    const int g = qi - m * G;
    const uint16_t* qp = q_buf + (size_t)rows[m] * H * kHD + (h * G + g) * kHD + grp * 8;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const sf_u32x4*>(qp + ds * 32);
  } else {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = sf_u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  auto key_ptr = [&](const uint16_t* base, int kl) -> const uint16_t* {
    const int t = k_begin + kl;
    if (page_table) {
      const int off = t % page_size;
      return base + (long long)s_page[kl] * page_stride + head_off + (long long)off * kHD;
    }
    return base + head_off + (long long)t * kHD;
  };

  // all K/V loads of the chunk at once: K thread->(key = (tid>>4) + 16i, seg = tid&15);
  // V thread->(keys 64p + 4*(tid>>4) + 0..3, seg = tid&15) so 4 consecutive keys pack
  // into one 8-byte V^T write
  const sf_u32x4 zero4 = {0u, 0u, 0u, 0u};
  const int sg = tid & 15;
  const int kr = tid >> 4;
  sf_u32x4 kreg[8], vreg[2][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int kl = kr + 16 * i;
    kreg[i] = (k_begin + kl < k_end)
                  ? *reinterpret_cast<const sf_u32x4*>(key_ptr(pk, kl) + sg * 8)
                  : zero4;
  }
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kl = 64 * p + 4 * kr + i;
      vreg[p][i] = (k_begin + kl < k_end)
                       ? *reinterpret_cast<const sf_u32x4*>(key_ptr(pv, kl) + sg * 8)
                       : zero4;
    }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<sf_u32x4*>(&sK[(kr + 16 * i) * kKStr + sg * 8]) = kreg[i];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t packed =
          (uint64_t)bf_at(vreg[p][0], j) | ((uint64_t)bf_at(vreg[p][1], j) << 16) |
          ((uint64_t)bf_at(vreg[p][2], j) << 32) | ((uint64_t)bf_at(vreg[p][3], j) << 48);
      *reinterpret_cast<uint64_t*>(&sV[(sg * 8 + j) * kVStr + 64 * p + 4 * kr]) = packed;
    }
  __syncthreads();

  float m_run = -INFINITY;
  float l_run = 0.f;
  sf_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int kbase = st * 64;
    if (k_begin + kbase >= k_end) break;
    float s[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      sf_f32x4 a = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* kb = &sK[(kbase + kt * 16 + ql) * kKStr + grp * 8];
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const sf_u32x4 kf = *reinterpret_cast<const sf_u32x4*>(kb + ds * 32);
        a = sf_mfma16x16x32(sf_as_bf16x8(kf), sf_as_bf16x8(qf[ds]), a);
      }
      const int key0 = k_begin + kbase + kt * 16 + grp * 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kt][r] = (key0 + r < k_end) ? a[r] * scaling : -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = expf(m_run - m_new);
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[kt][r] = expf(s[kt][r] - m_new);
        lsum += s[kt][r];
      }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;

#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kt0 = 2 * j, kt1 = 2 * j + 1;
      float ph[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ph[r] = s[kt0][r];
        ph[4 + r] = s[kt1][r];
      }
      sf_u32x4 hi, lo;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        const float a0 = ph[2 * w2], a1 = ph[2 * w2 + 1];
        hi[w2] = sf_pack2(a0, a1);
        lo[w2] = sf_pack2(a0 - sf_rbf(a0), a1 - sf_rbf(a1));
      }
      const sf_bf16x8 bhi = sf_as_bf16x8(hi);
      const sf_bf16x8 blo = sf_as_bf16x8(lo);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* vrow = &sV[(dt * 16 + ql) * kVStr + kbase + grp * 4];
        const uint64_t a0 = *reinterpret_cast<const uint64_t*>(vrow + kt0 * 16);
        const uint64_t a1 = *reinterpret_cast<const uint64_t*>(vrow + kt1 * 16);
        sf_u32x4 vf;
        vf[0] = (uint32_t)a0;
        vf[1] = (uint32_t)(a0 >> 32);
        vf[2] = (uint32_t)a1;
        vf[3] = (uint32_t)(a1 >> 32);
        const sf_bf16x8 va = sf_as_bf16x8(vf);
        acc[dt] = sf_mfma16x16x32(va, bhi, acc[dt]);
        acc[dt] = sf_mfma16x16x32(va, blo, acc[dt]);
      }
    }
  }

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (qvalid) {
    const size_t slot = ((size_t)h * nchunks + ci) * qmax + qi;
    if (grp == 0) {
      ws_ml[slot * 2] = m_run;
      ws_ml[slot * 2 + 1] = l_run;
    }
    float* op = ws_o + slot * kHD + grp * 4;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<sf_f32x4*>(op + dt * 16) = acc[dt];
  }
}

// One 512-thread workgroup per (recomputed row m, kv head h); thread t owns the
// output pair (q-head t/64, dims 2*(t%64) .. +1).
constexpr int kMaxChunks = 256;   // prefix <= 32768 keys
constexpr int kBatch = 16;        // chunk partials loaded per round

__global__ __launch_bounds__(512) void sf_attn_block_merge_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
    const int32_t* __restrict__ src, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, int N, int H, int Hkv, float scaling,
    const int32_t* __restrict__ p_len, int P_host, int nchunks_cap, int qmax,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, float* __restrict__ o32,
    uint16_t* __restrict__ o_bf, float* __restrict__ m_tab, float* __restrict__ z_tab) {
  __shared__ float sq[kMaxG][kHD];
  __shared__ __attribute__((aligned(16))) uint16_t sk[kMaxN][kHD];
  __shared__ __attribute__((aligned(16))) uint16_t sv[kMaxN][kHD];
  __shared__ float ss[kMaxG][kMaxN];
  __shared__ float sml[kMaxG][2 * kMaxChunks];   // per q-head: (m, l) of every chunk
  __shared__ float sM[kMaxG], sZ[kMaxG];
  const int m = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int count = min(*count_p, bucket);
  if (m >= count) return;
  const int G = H / Hkv;
  const int P = p_len ? *p_len : P_host;
  const int nch = min((P + kChunk - 1) / kChunk, nchunks_cap);
  const int row = rows[m];
  const int b = row / N;
  const int kvs = 2 * Hkv * kHD;

  // --- loads: q, the branch's block K/V (gathered through src), chunk (m, l) -------
  if (tid < G * 32) {
    const int g = tid >> 5, d = (tid & 31) * 4;
    const sf_u32x2 w = *reinterpret_cast<const sf_u32x2*>(
        q_buf + (size_t)row * H * kHD + (h * G + g) * kHD + d);
    sq[g][d] = __uint_as_float(w[0] << 16);
    sq[g][d + 1] = __uint_as_float(w[0] & 0xffff0000u);
    sq[g][d + 2] = __uint_as_float(w[1] << 16);
    sq[g][d + 3] = __uint_as_float(w[1] & 0xffff0000u);
  }
  for (int i = tid; i < N * 16; i += 512) {
    const int j = i >> 4, sgm = i & 15;
    const size_t kvrow = (size_t)(src[b * N + j] * N + j) * kvs;
    *reinterpret_cast<sf_u32x4*>(&sk[j][sgm * 8]) =
        *reinterpret_cast<const sf_u32x4*>(kv_buf + kvrow + h * kHD + sgm * 8);
    *reinterpret_cast<sf_u32x4*>(&sv[j][sgm * 8]) =
        *reinterpret_cast<const sf_u32x4*>(kv_buf + kvrow + (Hkv + h) * kHD + sgm * 8);
  }
  for (int i = tid; i < G * nch; i += 512) {
    const int g = i / nch, c = i - g * nch;
    const size_t sl = ((size_t)h * nchunks_cap + c) * qmax + (size_t)m * G + g;
    sml[g][2 * c] = ws_ml[sl * 2];
    sml[g][2 * c + 1] = ws_ml[sl * 2 + 1];
  }
  // this thread's first batch of chunk accumulators, in flight during the scores
  const int my_g = tid >> 6, dp = (tid & 63) * 2;
  const bool mine = my_g < G;
  const size_t my_slot0 = (size_t)h * nchunks_cap * qmax + (size_t)m * G + my_g;
  float2 accb[kBatch];
#pragma unroll
  for (int c = 0; c < kBatch; ++c)
    if (mine && c < nch)
      accb[c] = *reinterpret_cast<const float2*>(ws_o + (my_slot0 + (size_t)c * qmax) * kHD + dp);
  __syncthreads();

  // --- block scores: thread -> (g, j) ----------------------------------------------
  for (int i = tid; i < G * N; i += 512) {
    const int g = i / N, j = i - g * N;
    float d = 0.f;
#pragma unroll 4
    for (int e = 0; e < kHD; e += 8) {
      float kf[8];
      sf_unpack8(*reinterpret_cast<const sf_u32x4*>(&sk[j][e]), kf);
#pragma unroll
      for (int t = 0; t < 8; ++t) d = fmaf(sq[g][e + t], kf[t], d);
    }
    ss[g][j] = d * scaling;
  }
  __syncthreads();

  // --- per q-head: merged max, block probabilities, chunk weights, Z (wave w: head w)
  {
    const int lane = tid & 63, w = tid >> 6;
    if (w < G) {
      const int g = w;
      float mm = -INFINITY;
      for (int j = lane; j < N; j += 64) mm = fmaxf(mm, ss[g][j]);
      for (int c = lane; c < nch; c += 64) mm = fmaxf(mm, sml[g][2 * c]);
      mm = sf_wave_max(mm);
      float z = 0.f;
      for (int j = lane; j < N; j += 64) {
        const float p = expf(ss[g][j] - mm);
        ss[g][j] = p;
        z += p;
      }
      for (int c = lane; c < nch; c += 64) {
        const float wgt = expf(sml[g][2 * c] - mm);
        sml[g][2 * c] = wgt;
        z += sml[g][2 * c + 1] * wgt;
      }
      z = sf_wave_sum(z);
      if (lane == 0) {
        sM[g] = mm;
        sZ[g] = z;
      }
    }
  }
  __syncthreads();
  if (!mine) return;

  // --- O = (sum_j p_j v_j + sum_c w_c acc_c) / Z --------------------------------------
  float o0 = 0.f, o1 = 0.f;
  for (int j = 0; j < N; ++j) {
    const float p = ss[my_g][j];
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(&sv[j][dp]);
    o0 = fmaf(p, __uint_as_float(vv << 16), o0);
    o1 = fmaf(p, __uint_as_float(vv & 0xffff0000u), o1);
  }
  for (int cb = 0; cb < nch; cb += kBatch) {
    if (cb > 0) {
#pragma unroll
      for (int c = 0; c < kBatch; ++c)
        if (cb + c < nch)
          accb[c] = *reinterpret_cast<const float2*>(
              ws_o + (my_slot0 + (size_t)(cb + c) * qmax) * kHD + dp);
    }
#pragma unroll
    for (int c = 0; c < kBatch; ++c) {
      if (cb + c < nch) {
        const float wgt = sml[my_g][2 * (cb + c)];
        o0 = fmaf(wgt, accb[c].x, o0);
        o1 = fmaf(wgt, accb[c].y, o1);
      }
    }
  }
  const float inv = 1.0f / sZ[my_g];
  const float r0 = o0 * inv, r1 = o1 * inv;
  const size_t off = (size_t)row * H * kHD + (h * G + my_g) * kHD + dp;
  *reinterpret_cast<float2*>(o32 + off) = make_float2(r0, r1);
  *reinterpret_cast<uint32_t*>(o_bf + off) = sf_pack2(r0, r1);
  if (dp == 0) {
    m_tab[(size_t)row * H + h * G + my_g] = sM[my_g];
    z_tab[(size_t)row * H + h * G + my_g] = sZ[my_g];
  }
}

int nchunks_for(int P) { return (P + kChunk - 1) / kChunk; }

}  // namespace

extern "C" size_t sf_attn_workspace_bytes(int bucket, int H, int P) {
  if (bucket < 1 || H < 1 || P < 0) return 0;
  if (P == 0) return 16;
  // per (kv head, chunk, query): 128 fp32 acc + (m, l); queries per kv head = bucket*G,
  // so the total over kv heads is nchunks * bucket * H slots.
  return (size_t)nchunks_for(P) * bucket * H * (kHD + 2) * sizeof(float);
}

extern "C" int sf_attn_prefix_block(const uint16_t* q_buf, const uint16_t* kv_buf,
                                    const uint16_t* prefix_k, const uint16_t* prefix_v,
                                    const int32_t* page_table, int P, int page_size,
                                    long long page_stride, long long head_stride,
                                    const int32_t* src, const int32_t* rows, const int32_t* count,
                                    int bucket, int B1, int N, int H, int Hkv, int hd,
                                    float scaling, const int32_t* prefix_len, float* o32,
                                    uint16_t* o_bf, float* m_tab, float* z_tab, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!q_buf || !kv_buf || !src || !rows || !count || !o32 || !o_bf || !m_tab || !z_tab)
    return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > kMaxG) return SF_ERR_SHAPE;
  if (N < 1 || N > kMaxN || B1 < 1 || bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  if (P < 0 || nchunks_for(P) > kMaxChunks) return SF_ERR_SHAPE;
  if (P > 0) {
    if (!prefix_k || !prefix_v || !workspace) return SF_ERR_ARG;
    if (page_table && (page_size < 1 || kChunk % page_size != 0)) return SF_ERR_SHAPE;
    if (!page_table && head_stride < (long long)P * kHD) return SF_ERR_SHAPE;
    if (workspace_bytes < sf_attn_workspace_bytes(bucket, H, P)) return SF_ERR_WORKSPACE;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = H / Hkv;
  const int qmax = bucket * G;
  const int nch = P > 0 ? nchunks_for(P) : 0;
  float* ws_ml = nullptr;
  float* ws_o = nullptr;
  if (P > 0) {
    const size_t nslot = (size_t)nch * qmax * Hkv;
    ws_o = reinterpret_cast<float*>(workspace);
    ws_ml = ws_o + nslot * kHD;
    dim3 g1((qmax + kQT - 1) / kQT, nch, Hkv);
    hipLaunchKernelGGL(sf_attn_prefix_kernel, g1, dim3(256), 0, st, q_buf, prefix_k, prefix_v,
                       page_table, page_size, page_stride, head_stride, prefix_len, P, rows,
                       count, bucket, H, Hkv, scaling, qmax, ws_o, ws_ml);
  }
  dim3 g2(bucket, Hkv);
  hipLaunchKernelGGL(sf_attn_block_merge_kernel, g2, dim3(512), 0, st, q_buf, kv_buf, src, rows,
                     count, bucket, N, H, Hkv, scaling, P > 0 ? prefix_len : nullptr, P, nch, qmax,
                     ws_o, ws_ml, o32, o_bf, m_tab, z_tab);
  return sf_launch_status();
}
