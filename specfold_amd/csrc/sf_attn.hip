// Attention of the recomputed rows over [shared prefix ; own branch block],
// emitting the softmax state (m, Z) next to O.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:164-181 (fp32
// scores = (q . k) * scaling, m = max, Z = sum exp(s - m), O = sum exp(s - m) v / Z,
// no mask) and the Triton kernel specfold/generate/triton_kernels.py:301-361.
//
// Two kernels:
//  * prefix: grid (query tile, prefix chunk, kv head).  All recomputed rows x
//    the G q-heads of one kv head are flattened to queries qi = m*G + g and
//    tiled 64 per workgroup (16 per wave), so each prefix K/V element is read
//    by the few query tiles of its chunk instead of once per row.  K and V^T
//    tiles of 64 keys are staged in LDS (double buffered).  Scores are formed
//    transposed, S^T = K Q^T, so every lane holds 4 keys of ONE query: the
//    softmax rescale is per lane and P^T feeds the P.V MFMA straight from
//    registers (the 8 k-slots of a lane are keys {4g..4g+3} of two 16-key
//    tiles, and V^T is read in that same order).  P is split into
//    bf16 hi + lo halves (two MFMAs) so P.V keeps ~16 mantissa bits, close to
//    the reference's fp32 einsum.  Each chunk writes its (m, l, acc) partial.
//  * block+merge: one wave per (recomputed row, kv head): scores of the
//    branch's N block keys (gathered through src), merged with the prefix
//    partials into the final O (fp32 and bf16), m and Z.
#include <math.h>

#include "sf_common.h"

namespace {

constexpr int kHD = 128;
constexpr int kQT = 64;     // queries per workgroup
constexpr int kKT = 64;     // keys per LDS stage
constexpr int kKStr = 136;  // K tile row stride (bf16)
constexpr int kVStr = 72;   // V^T tile row stride (bf16)

int attn_chunk(int P) {
  int c = 256;
  while ((P + c - 1) / c > 32) c += kKT;
  return c;
}

SF_DEV const uint16_t* key_row(const uint16_t* base, const int32_t* page_table, int t,
                               int page_size, long long page_stride, long long head_off) {
  if (page_table) {
    const int lp = t / page_size;
    const int off = t - lp * page_size;
    return base + (long long)page_table[lp] * page_stride + head_off + (long long)off * kHD;
  }
  return base + head_off + (long long)t * kHD;
}

SF_DEV uint32_t bf_at(const sf_u32x4& w, int j) {
  return (w[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

__global__ __launch_bounds__(256) void sf_attn_prefix_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table, int P, int page_size,
    long long page_stride, long long head_stride, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, int H, int Hkv, float scaling, int chunk,
    int qmax, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKT * kKStr];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][kHD * kVStr];
  const int G = H / Hkv;
  const int qt = blockIdx.x;
  const int ci = blockIdx.y;
  const int h = blockIdx.z;
  const int nchunks = gridDim.y;
  const int count = min(*count_p, bucket);
  const int nq = count * G;
  if (qt * kQT >= nq) return;
  const int k_begin = ci * chunk;
  const int k_end = min(P, k_begin + chunk);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int grp = lane >> 4;  // 0..3
  const int ql = lane & 15;
  const int qi = qt * kQT + wv * 16 + ql;
  const bool qvalid = qi < nq;
  const long long head_off = (long long)h * head_stride;

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

  sf_u32x4 kreg[4], vreg[4];
  const sf_u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = i * 256 + tid;
      const int key = id >> 4;
      const int sg = id & 15;
      const int t = k0 + key;
      kreg[i] = (t < k_end) ? *reinterpret_cast<const sf_u32x4*>(
                                  key_row(pk, page_table, t, page_size, page_stride, head_off) +
                                  sg * 8)
                            : zero4;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 4 * (tid >> 4) + i;
      const int t = k0 + key;
      vreg[i] = (t < k_end) ? *reinterpret_cast<const sf_u32x4*>(
                                  key_row(pv, page_table, t, page_size, page_stride, head_off) +
                                  (tid & 15) * 8)
                            : zero4;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = i * 256 + tid;
      *reinterpret_cast<sf_u32x4*>(&sK[buf][(id >> 4) * kKStr + (id & 15) * 8]) = kreg[i];
    }
    const int kk = 4 * (tid >> 4);
    const int d0 = (tid & 15) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t packed = (uint64_t)bf_at(vreg[0], j) | ((uint64_t)bf_at(vreg[1], j) << 16) |
                              ((uint64_t)bf_at(vreg[2], j) << 32) |
                              ((uint64_t)bf_at(vreg[3], j) << 48);
      *reinterpret_cast<uint64_t*>(&sV[buf][(d0 + j) * kVStr + kk]) = packed;
    }
  };

  float m_run = -INFINITY;
  float l_run = 0.f;
  sf_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = (k_end - k_begin + kKT - 1) / kKT;
  load_tile(k_begin);
  store_tile(0);
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < nst;
    if (more) load_tile(k_begin + (st + 1) * kKT);

    float s[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      sf_f32x4 a = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* kb = &sK[buf][(kt * 16 + ql) * kKStr + grp * 8];
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const sf_u32x4 kf = *reinterpret_cast<const sf_u32x4*>(kb + ds * 32);
        a = sf_mfma16x16x32(sf_as_bf16x8(kf), sf_as_bf16x8(qf[ds]), a);
      }
      const int kbase = k_begin + st * kKT + kt * 16 + grp * 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kt][r] = (kbase + r < k_end) ? a[r] * scaling : -INFINITY;
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
        const uint16_t* vrow = &sV[buf][(dt * 16 + ql) * kVStr + grp * 4];
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
    if (more) store_tile(buf ^ 1);
    __syncthreads();
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

// One wave per (recomputed row m, kv head h): block scores for the G q-heads,
// merge with the prefix chunk partials, final O / m / Z.
__global__ __launch_bounds__(64) void sf_attn_block_merge_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
    const int32_t* __restrict__ src, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, int N, int H, int Hkv, float scaling,
    int nchunks, int qmax, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    float* __restrict__ o32, uint16_t* __restrict__ o_bf, float* __restrict__ m_tab,
    float* __restrict__ z_tab) {
  __shared__ float sq[8][kHD];
  __shared__ float sp[8][64];
  __shared__ int s_kvrow[64];
  const int m = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int count = min(*count_p, bucket);
  if (m >= count) return;
  const int G = H / Hkv;
  const int row = rows[m];
  const int b = row / N;
  const int kvs = 2 * Hkv * kHD;

#pragma unroll
  for (int g = 0; g < 8; ++g) {
    if (g < G) {
      const uint32_t pr = *reinterpret_cast<const uint32_t*>(
          q_buf + (size_t)row * H * kHD + (h * G + g) * kHD + 2 * lane);
      sq[g][2 * lane] = __uint_as_float(pr << 16);
      sq[g][2 * lane + 1] = __uint_as_float(pr & 0xffff0000u);
    }
  }
  if (lane < N) s_kvrow[lane] = src[b * N + lane] * N + lane;
  __syncthreads();

  // scores: lanes (2j, 2j+1) split the head dim of block key j
  for (int j0 = 0; j0 < N; j0 += 32) {
    const int j = j0 + (lane >> 1);
    const int half = lane & 1;
    float dot[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) dot[g] = 0.f;
    if (j < N) {
      const uint16_t* kp = kv_buf + (size_t)s_kvrow[j] * kvs + h * kHD + half * 64;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        float kf[8];
        sf_unpack8(*reinterpret_cast<const sf_u32x4*>(kp + v * 8), kf);
#pragma unroll
        for (int g = 0; g < 8; ++g)
          if (g < G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) dot[g] = fmaf(sq[g][half * 64 + v * 8 + e], kf[e], dot[g]);
          }
      }
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) dot[g] += __shfl_xor(dot[g], 1, 64);
    if (j < N && half == 0) {
#pragma unroll
      for (int g = 0; g < 8; ++g)
        if (g < G) sp[g][j] = dot[g] * scaling;
    }
  }
  __syncthreads();

  // per q-head: merged max, block probabilities, Z
  float mg[8], zg[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    mg[g] = 0.f;
    zg[g] = 1.f;
    if (g < G) {
      const size_t qi = (size_t)m * G + g;
      const float sv = lane < N ? sp[g][lane] : -INFINITY;
      float mm = sv;
      for (int c = lane; c < nchunks; c += 64)
        mm = fmaxf(mm, ws_ml[(((size_t)h * nchunks + c) * qmax + qi) * 2]);
      mm = sf_wave_max(mm);
      const float pv = lane < N ? expf(sv - mm) : 0.f;
      if (lane < N) sp[g][lane] = pv;
      float z = pv;
      for (int c = lane; c < nchunks; c += 64) {
        const size_t sl = ((size_t)h * nchunks + c) * qmax + qi;
        z += ws_ml[sl * 2 + 1] * expf(ws_ml[sl * 2] - mm);
      }
      zg[g] = sf_wave_sum(z);
      mg[g] = mm;
    }
  }
  __syncthreads();

  // O: lane owns dims 2*lane, 2*lane+1
  float o[8][2];
#pragma unroll
  for (int g = 0; g < 8; ++g) o[g][0] = o[g][1] = 0.f;
  for (int j = 0; j < N; ++j) {
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(
        kv_buf + (size_t)s_kvrow[j] * kvs + (Hkv + h) * kHD + 2 * lane);
    const float v0 = __uint_as_float(vv << 16), v1 = __uint_as_float(vv & 0xffff0000u);
#pragma unroll
    for (int g = 0; g < 8; ++g)
      if (g < G) {
        const float p = sp[g][j];
        o[g][0] = fmaf(p, v0, o[g][0]);
        o[g][1] = fmaf(p, v1, o[g][1]);
      }
  }
  for (int c = 0; c < nchunks; ++c) {
#pragma unroll
    for (int g = 0; g < 8; ++g)
      if (g < G) {
        const size_t sl = ((size_t)h * nchunks + c) * qmax + (size_t)m * G + g;
        const float wgt = expf(ws_ml[sl * 2] - mg[g]);
        const float2 a = *reinterpret_cast<const float2*>(ws_o + sl * kHD + 2 * lane);
        o[g][0] = fmaf(wgt, a.x, o[g][0]);
        o[g][1] = fmaf(wgt, a.y, o[g][1]);
      }
  }
#pragma unroll
  for (int g = 0; g < 8; ++g)
    if (g < G) {
      const float inv = 1.0f / zg[g];
      const float r0 = o[g][0] * inv, r1 = o[g][1] * inv;
      const size_t off = (size_t)row * H * kHD + (h * G + g) * kHD + 2 * lane;
      *reinterpret_cast<float2*>(o32 + off) = make_float2(r0, r1);
      *reinterpret_cast<uint32_t*>(o_bf + off) = sf_pack2(r0, r1);
      if (lane == 0) {
        m_tab[(size_t)row * H + h * G + g] = mg[g];
        z_tab[(size_t)row * H + h * G + g] = zg[g];
      }
    }
}

}  // namespace

extern "C" size_t sf_attn_workspace_bytes(int bucket, int H, int P) {
  if (bucket < 1 || H < 1 || P < 0) return 0;
  if (P == 0) return 16;
  const int nch = (P + attn_chunk(P) - 1) / attn_chunk(P);
  // per (kv head, chunk, query): 128 fp32 acc + (m, l); queries per kv head = bucket*G,
  // so the total over kv heads is nch * bucket * H slots.
  return (size_t)nch * bucket * H * (kHD + 2) * sizeof(float);
}

extern "C" int sf_attn_prefix_block(const uint16_t* q_buf, const uint16_t* kv_buf,
                                    const uint16_t* prefix_k, const uint16_t* prefix_v,
                                    const int32_t* page_table, int P, int page_size,
                                    long long page_stride, long long head_stride,
                                    const int32_t* src, const int32_t* rows, const int32_t* count,
                                    int bucket, int B1, int N, int H, int Hkv, int hd,
                                    float scaling, float* o32, uint16_t* o_bf, float* m_tab,
                                    float* z_tab, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (!q_buf || !kv_buf || !src || !rows || !count || !o32 || !o_bf || !m_tab || !z_tab)
    return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > 8) return SF_ERR_SHAPE;
  if (N < 1 || N > 64 || B1 < 1 || bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  if (P < 0) return SF_ERR_SHAPE;
  if (P > 0) {
    if (!prefix_k || !prefix_v || !workspace) return SF_ERR_ARG;
    if (page_table && page_size < 1) return SF_ERR_SHAPE;
    if (!page_table && head_stride < (long long)P * kHD) return SF_ERR_SHAPE;
    if (workspace_bytes < sf_attn_workspace_bytes(bucket, H, P)) return SF_ERR_WORKSPACE;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = H / Hkv;
  const int qmax = bucket * G;
  int nchunks = 0;
  float* ws_ml = nullptr;
  float* ws_o = nullptr;
  if (P > 0) {
    const int chunk = attn_chunk(P);
    nchunks = (P + chunk - 1) / chunk;
    const size_t nslot = (size_t)nchunks * qmax * Hkv;
    ws_o = reinterpret_cast<float*>(workspace);
    ws_ml = ws_o + nslot * kHD;
    dim3 g1((qmax + kQT - 1) / kQT, nchunks, Hkv);
    hipLaunchKernelGGL(sf_attn_prefix_kernel, g1, dim3(256), 0, st, q_buf, prefix_k, prefix_v,
                       page_table, P, page_size, page_stride, head_stride, rows, count, bucket, H,
                       Hkv, scaling, chunk, qmax, ws_o, ws_ml);
  }
  dim3 g2(bucket, Hkv);
  hipLaunchKernelGGL(sf_attn_block_merge_kernel, g2, dim3(64), 0, st, q_buf, kv_buf, src, rows,
                     count, bucket, N, H, Hkv, scaling, nchunks, qmax, ws_o, ws_ml, o32, o_bf,
                     m_tab, z_tab);
  return sf_launch_status();
}
