// Attention of the recomputed rows over [shared prefix ; own branch block],
// emitting the softmax state (m, Z) next to O.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:164-181 (fp32
// scores = (q . k) * scaling, m = max, Z = sum exp(s - m), O = sum exp(s - m) v / Z,
// no mask) and the Triton kernel specfold/generate/triton_kernels.py:301-361.
//
// Two kernels (flash-decoding split over the prefix):
//  * prefix: a persistent grid walks the active (query tile, range of 128-key
//    prefix chunks, kv head) items; the item count follows the device-side row
//    count and prefix length, so no workgroup is dispatched for an empty tile.
//    All recomputed rows x the G q-heads of one kv head are flattened to queries
//    qi = m*G + g and tiled 64 per item (16 per wave), so each prefix K/V
//    element is read by the few query tiles of its chunk instead of once per
//    row.  Items of one chunk range are consecutive and go to one XCD
//    (workgroup b runs on XCD b % 8), so the range's later reads hit that XCD's
//    L2.  A range is one chunk while one-chunk items fill about two rounds of
//    the grid and grows with the prefix beyond that (long contexts: fewer
//    partials, and chunk c+1's K/V loads are in flight while chunk c is
//    computed).  Per chunk, K is staged in LDS and V written transposed; scores
//    are formed transposed, S^T = K Q^T, so every lane holds keys of ONE query:
//    the softmax is per lane, rescaled across the range's chunks as in flash
//    attention, and P^T feeds the P.V MFMA straight from registers (the 8
//    k-slots of a lane are keys {4g..4g+3} of two 16-key tiles, and V^T is read
//    in that same order).  P is split into bf16 hi + lo halves (two MFMAs) so
//    P.V keeps ~16 mantissa bits, close to the reference's fp32 einsum.  Each
//    item writes its (m, l, acc) partial.
//  * block + merge: one 512-thread workgroup per active (recomputed row, kv
//    head): every load (q, the branch's N block keys/values gathered through src,
//    all range partials) is issued up front; block scores, the merged max, Z and
//    O follow from LDS.
// Softmax exponentials are exp2 of scores pre-scaled by log2(e) (one v_exp_f32
// each); partial maxima stay in that base-2 domain and the emitted m is converted
// back, so (m, Z) describe the natural-base softmax the reference computes.
// The prefix length may come from device memory (p_len), so a captured graph
// of the verify step stays valid while the cache grows; `P` is then the
// capacity the grid and the workspace are sized for.
#include <math.h>

#include "sf_common.h"
#include "sf_index.h"

namespace {

using namespace sfa;  // kHD, kQT, kChunk, kMaxChunks and the index maps

constexpr int kKStr = 136;   // K tile row stride (bf16)
constexpr int kVStr = 136;   // V^T tile row stride (bf16): 128 keys + 8 pad
constexpr int kMaxG = 8;
constexpr int kMaxN = 64;
constexpr int kCUs = 256;  // MI355X compute units

// V^T tile swizzle (vt_swz): keys of dim row d are stored in 4-key (8-byte)
// units, unit u at position u ^ vt_swz(d).  The transposing writes (16 lanes per
// key group hitting rows 8 apart) then spread over every bank, and the P.V reads
// (16 consecutive rows, one unit each) stay conflict-free: vt_swz is constant
// across the 16 rows one read instruction touches.
//
// Prefix chunks per work item (prefix_cpi): one while the one-chunk items fill
// about two rounds of the resident grid, longer ranges beyond (fewer partials to
// write and merge, and the next chunk's loads overlap this chunk's math).
//
// Keys of a chunk are held in a permuted slot order: load j (0..7) of thread row
// r = tid / 16 brings key 16j + r, which occupies slot key_slot(j, r) =
// 64(j/4) + 4r + j%4.  Every load instruction then reads 16 consecutive keys
// (one 4 KB stretch of a page, whose id is uniform: a scalar load), and the 4
// keys a thread transposes into V^T are 4 consecutive slots.  The softmax does
// not depend on key order; only the mask of a partial last chunk needs the key
// behind a slot (slot_key).

// One (query tile, range of prefix chunks, kv head) item of the prefix pass; all
// 256 threads take part (the LDS barriers are uniform).  K/V of chunk c+1 are
// loaded into registers while chunk c is scored and accumulated; the running
// (max, sum, acc) is rescaled per chunk as in flash attention.
SF_DEV void prefix_item(const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
                        const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table,
                        int page_size, long long page_stride, long long head_stride, int P,
                        const int32_t* __restrict__ rows, int nq, int G, int H, float scale_log2,
                        int qmax, int nch_cap, int qt, int r, int c0, int c1, int h, uint16_t* sK,
                        uint16_t* sV, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int grp = lane >> 4;  // 0..3
  const int ql = lane & 15;
  const int qi = qt * kQT + wv * 16 + ql;
  const bool qvalid = qi < nq;
  const long long head_off = (long long)h * head_stride;

  // Q^T operand: lane holds q[qi][ds*32 + grp*8 .. +8]; a padding query (qi >= nq)
  // repeats the last real one and its partial is never written
  sf_u32x4 qf[4];
  {
    const int qc = min(qi, nq - 1);
    const int m = qc / G;
    const int g = qc - m * G;
    const uint16_t* qp = q_buf + (size_t)rows[m] * H * kHD + (h * G + g) * kHD + grp * 8;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const sf_u32x4*>(qp + ds * 32);
  }

  // 16-key group j of chunk ci starts at key g0 (groups past the prefix end are
  // clamped to the last group holding keys, keys past the end to the last key);
  // with a page size that is a multiple of 16 a group never straddles pages.
  const int last_g0 = last_group_g0(P);
  const int sg = tid & 15;
  const int kr = tid >> 4;
  auto group_page = [&](int ci, int j) -> int {
    const int g0 = chunk_group_g0(ci, j, last_g0);
    return page_table ? page_table[g0 / page_size] : 0;
  };
  sf_u32x4 kreg[8], vreg[2][4];
  auto load_chunk = [&](int ci, const int* pg) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int g0 = chunk_group_g0(ci, j, last_g0);
      const long long grow = page_table
          ? (long long)pg[j] * page_stride + (long long)(g0 & (page_size - 1)) * kHD
          : (long long)g0 * kHD;
      const int off = group_key(kr, g0, P) * kHD + sg * 8;
      kreg[j] = *reinterpret_cast<const sf_u32x4*>(pk + head_off + grow + off);
      vreg[j >> 2][j & 3] = *reinterpret_cast<const sf_u32x4*>(pv + head_off + grow + off);
    }
  };
  int pg_next[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pg_next[j] = group_page(c0, j);
  load_chunk(c0, pg_next);
  if (c0 + 1 < c1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pg_next[j] = group_page(c0 + 1, j);
  }

  float m_run = -INFINITY, l_run = 0.f;
  sf_f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c = c0; c < c1; ++c) {
    const int nkeys = min(P - c * kChunk, kChunk);  // >= 1
    // stage K (slot order) and V^T of chunk c (V^T: dims (2w, 2w+1) of slots
    // 4kr + 64p .. +3 -> one word per dim, by byte permutes)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<sf_u32x4*>(&sK[key_slot(j, kr) * kKStr + sg * 8]) = kreg[j];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t x0 = vreg[p][0][w], x1 = vreg[p][1][w];
        const uint32_t x2 = vreg[p][2][w], x3 = vreg[p][3][w];
        sf_u32x2 lo, hi;
        lo[0] = (x0 & 0xffffu) | (x1 << 16);
        lo[1] = (x2 & 0xffffu) | (x3 << 16);
        hi[0] = (x0 >> 16) | (x1 & 0xffff0000u);
        hi[1] = (x2 >> 16) | (x3 & 0xffff0000u);
        const int d = sg * 8 + 2 * w;  // d and d + 1 share vt_swz
        const int col = ((16 * p + kr) ^ vt_swz(d)) * 4;
        *reinterpret_cast<sf_u32x2*>(&sV[d * kVStr + col]) = lo;
        *reinterpret_cast<sf_u32x2*>(&sV[(d + 1) * kVStr + col]) = hi;
      }
    __syncthreads();
    if (c + 1 < c1) {
      load_chunk(c + 1, pg_next);
      if (c + 2 < c1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) pg_next[j] = group_page(c + 2, j);
      }
    }

    // S^T = K Q^T (raw dot products) for the 8 slot tiles of the chunk
    float s[8][4];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      sf_f32x4 a = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* kb = &sK[(kt * 16 + ql) * kKStr + grp * 8];
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const sf_u32x4 kf = *reinterpret_cast<const sf_u32x4*>(kb + ds * 32);
        a = sf_mfma16x16x32(sf_as_bf16x8(kf), sf_as_bf16x8(qf[ds]), a);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) s[kt][rr] = a[rr];
    }
    if (nkeys < kChunk) {  // uniform: only a partial last chunk
#pragma unroll
      for (int kt = 0; kt < 8; ++kt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (slot_key(kt * 16 + grp * 4 + rr) >= nkeys) s[kt][rr] = -INFINITY;
    }

    // the 4 lane groups of a query hold its 128 keys; the max is taken on the raw
    // dot products (the scale is positive) and probabilities are
    // exp2(s * scale_log2 - m) with m in the scaled base-2 domain
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) mx = fmaxf(mx, s[kt][rr]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx * scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first chunk
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        s[kt][rr] = __builtin_amdgcn_exp2f(fmaf(s[kt][rr], scale_log2, -m_new));
        lsum += s[kt][rr];
      }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * alpha;

    // acc += V^T P^T; P split into three bf16 parts hi + mid + lo (24 bits: the
    // products P*V are those of the reference's fp32 einsum)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kt0 = 2 * j, kt1 = 2 * j + 1;
      sf_u32x4 hi, mid, lo;
#pragma unroll
      for (int w2 = 0; w2 < 2; ++w2) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int kt = t ? kt1 : kt0;
          const float a0 = s[kt][2 * w2], a1 = s[kt][2 * w2 + 1];
          const float r0 = a0 - sf_rbf(a0), r1 = a1 - sf_rbf(a1);
          hi[2 * t + w2] = sf_pack2(a0, a1);
          mid[2 * t + w2] = sf_pack2(r0, r1);
          lo[2 * t + w2] = sf_pack2(r0 - sf_rbf(r0), r1 - sf_rbf(r1));
        }
      }
      const sf_bf16x8 bhi = sf_as_bf16x8(hi);
      const sf_bf16x8 bmid = sf_as_bf16x8(mid);
      const sf_bf16x8 blo = sf_as_bf16x8(lo);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = dt * 16 + ql;
        const uint16_t* vrow = &sV[d * kVStr];
        const int sw = vt_swz(d);
        const sf_u32x2 a0 = *reinterpret_cast<const sf_u32x2*>(vrow + ((4 * kt0 + grp) ^ sw) * 4);
        const sf_u32x2 a1 = *reinterpret_cast<const sf_u32x2*>(vrow + ((4 * kt1 + grp) ^ sw) * 4);
        const sf_u32x4 vf = {a0[0], a0[1], a1[0], a1[1]};
        const sf_bf16x8 va = sf_as_bf16x8(vf);
        acc[dt] = sf_mfma16x16x32(va, blo, acc[dt]);
        acc[dt] = sf_mfma16x16x32(va, bmid, acc[dt]);
        acc[dt] = sf_mfma16x16x32(va, bhi, acc[dt]);
      }
    }
    __syncthreads();  // sK / sV are rewritten by the next chunk
  }

  if (qvalid) {
    const size_t slot = attn_slot(h, r, qi, nch_cap, qmax);
    if (grp == 0) {
      ws_ml[slot * 2] = m_run;
      ws_ml[slot * 2 + 1] = l_run;
    }
    float* op = ws_o + slot * kHD + grp * 4;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<sf_f32x4*>(op + dt * 16) = acc[dt];
  }
}

// gridDim.x is a multiple of 8; XCD x (workgroups b with b % 8 == x) takes the
// x-th eighth of the item list, so consecutive items (the query tiles of one
// chunk range) share an L2.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sf_attn_prefix_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table, int page_size,
    long long page_stride, long long head_stride, const int32_t* __restrict__ p_len, int P_cap,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ count_p, int bucket, int H,
    int Hkv, float scale_log2, int qmax, int nch_cap, float* __restrict__ ws_o,
    float* __restrict__ ws_ml) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kChunk * kKStr];
  __shared__ __attribute__((aligned(16))) uint16_t sV[kHD * kVStr];
  const int G = H / Hkv;
  const int P = p_len ? min(*p_len, P_cap) : P_cap;
  if (P <= 0) return;
  const int nq = min(*count_p, bucket) * G;
  const PrefixGrid pg = prefix_grid(P, nq, Hkv);
  const int n_qt = pg.n_qt;
  const int nch = pg.nch;
  const int cpi = pg.cpi;
  const int nr = pg.nr;
  const int items = n_qt * nr * Hkv;
  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int end = xcd_begin(items, xcd + 1);
  for (int it = xcd_begin(items, xcd) + (int)(blockIdx.x >> 3); it < end; it += per) {
    const AttnItem item = attn_item(it, n_qt, nr);
    const int c0 = item.r * cpi;
    prefix_item(q_buf, pk, pv, page_table, page_size, page_stride, head_stride, P, rows, nq, G, H,
                scale_log2, qmax, nch_cap, item.qt, item.r, c0, min(nch, c0 + cpi), item.h, sK, sV,
                ws_o, ws_ml);
    __syncthreads();  // LDS is reused by the next item
  }
}

// One 512-thread workgroup per active (recomputed row m, kv head h) item, walked
// by a persistent grid; thread t owns the output pair (q-head t/64, dims
// 2*(t%64) .. +1).
constexpr int kBatch = 16;        // chunk partials loaded per round

SF_DEV void merge_item(const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
                       const int32_t* __restrict__ src, const int32_t* __restrict__ rows, int m,
                       int h, int N, int H, int Hkv, int G, float scale_log2, int causal, int nch,
                       int nchunks_cap, int qmax, const float* __restrict__ ws_o,
                       const float* __restrict__ ws_ml, float* __restrict__ o32,
                       uint16_t* __restrict__ o_bf, float* __restrict__ m_tab,
                       float* __restrict__ z_tab, float (*sq)[kHD], uint16_t (*sk)[kHD],
                       uint16_t (*sv)[kHD], float (*ss)[kMaxN], float (*sml)[2 * kMaxChunks],
                       float* sM, float* sZ) {
  const int tid = threadIdx.x;
  const int my_g = tid >> 6, dp = (tid & 63) * 2;
  const bool mine = my_g < G;
  const size_t my_slot0 = (size_t)h * nchunks_cap * qmax + (size_t)m * G + my_g;
  // --- loads: chunk (m, l) and the first batch of chunk accumulators (independent
  // of the row id), then q and the branch's block K/V gathered through src --------
  for (int i = tid; i < G * nch; i += 512) {
    const int g = i / nch, c = i - g * nch;
    // attn_slot(h, c, m·G + g, ...) in 64-bit arithmetic (tests/cpp/index_check.cpp
    // checks that these reads are exactly the prefix pass's writes)
    const size_t sl = ((size_t)h * nchunks_cap + c) * qmax + (size_t)m * G + g;
    const float2 ml = *reinterpret_cast<const float2*>(ws_ml + sl * 2);
    sml[g][2 * c] = ml.x;
    sml[g][2 * c + 1] = ml.y;
  }
  float2 accb[kBatch];
#pragma unroll
  for (int c = 0; c < kBatch; ++c)
    if (mine && c < nch)
      accb[c] = *reinterpret_cast<const float2*>(ws_o + (my_slot0 + (size_t)c * qmax) * kHD + dp);
  const int row = rows[m];
  const int b = row / N;
  const int kvs = 2 * Hkv * kHD;
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
    const sf_u32x4 kk = *reinterpret_cast<const sf_u32x4*>(kv_buf + kvrow + h * kHD + sgm * 8);
    const sf_u32x4 vv =
        *reinterpret_cast<const sf_u32x4*>(kv_buf + kvrow + (Hkv + h) * kHD + sgm * 8);
    *reinterpret_cast<sf_u32x4*>(&sk[j][sgm * 8]) = kk;
    *reinterpret_cast<sf_u32x4*>(&sv[j][sgm * 8]) = vv;
  }
  __syncthreads();

  // --- block scores (base-2 domain): thread -> (g, j) ------------------------------
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
    // causal (a block commit of an AR forward): block position n sees keys j <= n
    ss[g][j] = (causal && j > row - b * N) ? -INFINITY : d * scale_log2;
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
        const float p = __builtin_amdgcn_exp2f(ss[g][j] - mm);
        ss[g][j] = p;
        z += p;
      }
      for (int c = lane; c < nch; c += 64) {
        const float wgt = __builtin_amdgcn_exp2f(sml[g][2 * c] - mm);
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

  // --- O = (sum_j p_j v_j + sum_c w_c acc_c) / Z --------------------------------------
  if (mine) {
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
          accb[c] = *reinterpret_cast<const float2*>(
              ws_o + (my_slot0 + (size_t)min(cb + c, nch - 1) * qmax) * kHD + dp);
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
      // the natural-base max the block scores and chunk maxima were measured from
      m_tab[(size_t)row * H + h * G + my_g] = sM[my_g] * 0.69314718055994530942f;
      z_tab[(size_t)row * H + h * G + my_g] = sZ[my_g];
    }
  }
}

__global__ __launch_bounds__(512) void sf_attn_block_merge_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
    const int32_t* __restrict__ src, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, int N, int H, int Hkv, float scale_log2,
    int causal, const int32_t* __restrict__ p_len, int P_cap, int nchunks_cap, int qmax,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, float* __restrict__ o32,
    uint16_t* __restrict__ o_bf, float* __restrict__ m_tab, float* __restrict__ z_tab) {
  __shared__ float sq[kMaxG][kHD];
  __shared__ __attribute__((aligned(16))) uint16_t sk[kMaxN][kHD];
  __shared__ __attribute__((aligned(16))) uint16_t sv[kMaxN][kHD];
  __shared__ float ss[kMaxG][kMaxN];
  __shared__ float sml[kMaxG][2 * kMaxChunks];   // per q-head: (m, l) of every chunk
  __shared__ float sM[kMaxG], sZ[kMaxG];
  const int count = min(*count_p, bucket);
  const int G = H / Hkv;
  const int P = p_len ? min(*p_len, P_cap) : P_cap;
  // number of prefix partials per query: the prefix kernel's chunk ranges
  const int nch = merge_ranges(P, count * G, Hkv, nchunks_cap);
  for (int it = blockIdx.x; it < count * Hkv; it += gridDim.x) {
    merge_item(q_buf, kv_buf, src, rows, it / Hkv, it % Hkv, N, H, Hkv, G, scale_log2, causal, nch,
               nchunks_cap, qmax, ws_o, ws_ml, o32, o_bf, m_tab, z_tab, sq, sk, sv, ss, sml, sM,
               sZ);
    __syncthreads();  // LDS is reused by the next item
  }
}

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
                                    float scaling, const int32_t* prefix_len, int block_causal,
                                    float* o32,
                                    uint16_t* o_bf, float* m_tab, float* z_tab, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!q_buf || !kv_buf || !src || !rows || !count || !o32 || !o_bf || !m_tab || !z_tab)
    return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > kMaxG) return SF_ERR_SHAPE;
  if (N < 1 || N > kMaxN || B1 < 1 || bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  if (P < 0 || nchunks_for(P) > kMaxChunks) return SF_ERR_SHAPE;
  if (P > 0) {
    if (!prefix_k || !prefix_v || !workspace) return SF_ERR_ARG;
    // a page holds whole 16-key groups and a chunk whole pages: 16, 32, 64 or 128
    if (page_table && (page_size < 16 || kChunk % page_size != 0)) return SF_ERR_SHAPE;
    if (!page_table && head_stride < (long long)P * kHD) return SF_ERR_SHAPE;
    if (workspace_bytes < sf_attn_workspace_bytes(bucket, H, P)) return SF_ERR_WORKSPACE;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = H / Hkv;
  const int qmax = bucket * G;
  const int nch = P > 0 ? nchunks_for(P) : 0;
  const float scale_log2 = scaling * 1.44269504088896340736f;
  float* ws_ml = nullptr;
  float* ws_o = nullptr;
  if (P > 0) {
    const size_t nslot = (size_t)nch * qmax * Hkv;
    ws_o = reinterpret_cast<float*>(workspace);
    ws_ml = ws_o + nslot * kHD;
    // persistent grid: at most two 70 KB-LDS workgroups fit a CU; a multiple of 8
    const int grid = prefix_launch_grid(qmax, nch, Hkv);
    hipLaunchKernelGGL(sf_attn_prefix_kernel, dim3(grid), dim3(256), 0, st, q_buf, prefix_k,
                       prefix_v, page_table, page_size, page_stride, head_stride, prefix_len, P,
                       rows, count, bucket, H, Hkv, scale_log2, qmax, nch, ws_o, ws_ml);
  }
  const int grid2 = min(bucket * Hkv, 2 * kCUs);
  hipLaunchKernelGGL(sf_attn_block_merge_kernel, dim3(grid2), dim3(512), 0, st, q_buf, kv_buf,
                     src, rows, count, bucket, N, H, Hkv, scale_log2, block_causal ? 1 : 0,
                     P > 0 ? prefix_len : nullptr,
                     P, nch, qmax, ws_o, ws_ml, o32, o_bf, m_tab, z_tab);
  return sf_launch_status();
}
