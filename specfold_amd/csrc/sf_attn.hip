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

using namespace sfa;  // kHD, kQT, kChunk, kMaxRanges and the index maps

constexpr int kMaxG = 8;
constexpr int kMaxN = 64;
constexpr int kCUs = 256;  // MI355X compute units

// ---- prefix pass ---------------------------------------------------------------------
// Work item = (query tile of 128 queries, range of 64-key prefix chunks, kv head),
// one 512-thread workgroup per CU walking items.  Wave w takes the 32 queries
// (w & 3) * 32 .. +32 of the tile (two 16-query MFMA tiles) against keys
// (w >> 2) * 32 .. +32 of every chunk, so the 8 waves share each staged chunk and
// each wave keeps its own running softmax state; the two key halves of a query
// are combined when the range is done.
//
// Staging: K and V rows of a chunk go straight from the cache to an LDS ring of
// kRing chunks (global_load_lds, 16 bytes per lane, 1 KB per instruction; rows
// swizzled by k_unit / v_unit on the copy side), kRing - 1 chunks ahead of the
// one being computed.  Waves 0-3 copy the K rows, waves 4-7 the V rows, wave w
// the 16-key group w & 3 (one page: a scalar page-table read per chunk).
// Scores are formed transposed, S^T = K Q^T (K fragments: one 16-byte read of a
// key row per lane; Q^T stays in registers), so each lane holds 4 keys of one
// query per 16-key tile: the softmax max / sum reduce over the 4 lane groups.
// P^T then feeds O^T += V^T P^T as the B operand straight from registers; the
// V^T operand comes from the row-major V rows by two transposing reads
// (ds_read_b64_tr_b16) per 32 keys x 16 dims.
// P is split into kPParts bf16 parts (hi, then the rounding residuals) so the
// products P.V keep 8 * kPParts mantissa bits.
#ifndef SFA_P_PARTS
#define SFA_P_PARTS 2
#endif
constexpr int kPParts = SFA_P_PARTS;
constexpr int kRing = 4;                          // chunks in the LDS ring
constexpr int kSlotBytes = 2 * kHalfBytes;        // K then V rows: 32 KB
constexpr int kPrefixThreads = 512;
constexpr int kCopiesPerChunk = 4;                // DMA instructions per wave per chunk

// softmax-weighted accumulation of one chunk for one wave (two query tiles)
template <int NP>
SF_DEV void pv_parts(const float (&p)[2][4], sf_bf16x8 (&b)[NP]) {
  // element j of the B operand: key 4*group + j of tile 0 (j < 4), of tile 1 (j >= 4)
  sf_u32x4 w[NP];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float a0 = p[u >> 1][2 * (u & 1)], a1 = p[u >> 1][2 * (u & 1) + 1];
    w[0][u] = sf_pack2(a0, a1);
    if (NP > 1) {
      const float r0 = a0 - sf_rbf(a0), r1 = a1 - sf_rbf(a1);
      w[NP > 1 ? 1 : 0][u] = sf_pack2(r0, r1);
      if (NP > 2) w[NP > 2 ? 2 : 0][u] = sf_pack2(r0 - sf_rbf(r0), r1 - sf_rbf(r1));
    }
  }
#pragma unroll
  for (int i = 0; i < NP; ++i) b[i] = sf_as_bf16x8(w[i]);
}

SF_DEV void prefix_item(const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
                        const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table,
                        int page_size, long long page_stride, long long head_stride, int P,
                        const int32_t* __restrict__ rows, int nq, int G, int H, float scale_log2,
                        int qmax, int nr_cap, int qt, int r, int c0, int c1, int h,
                        uint8_t* ring, int* s_pg, float* __restrict__ ws_o,
                        float* __restrict__ ws_ml) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int grp = lane >> 4;  // 0..3
  const int ql = lane & 15;
  const int qg = wv & 3;      // query group
  const int kh = wv >> 2;     // key half of every chunk
  const long long head_off = (long long)h * head_stride;

  // ---- item set-up, in two rounds of loads: (1) the query rows and the range's
  // page ids (to LDS); (2) the first kRing - 1 chunk copies, then q -------------------
  const int jg = wv & 3;
  const bool is_v = wv >= 4;
  const int last_g0 = last_group_g0(P);
  const int ngroups = 4 * (c1 - c0);
  if (page_table) {
    for (int i = tid; i < ngroups; i += kPrefixThreads)
      s_pg[i] = page_table[chunk_group_g0(c0 + (i >> 2), i & 3, last_g0) / page_size];
  }
  int qrow[2], qhead[2];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    // a padding query (qi >= nq) repeats the last real one; its partial is not written
    const int qc = min(qt * kQT + qg * 32 + qs * 16 + ql, nq - 1);
    const int m = qc / G;
    qrow[qs] = rows[m];
    qhead[qs] = h * G + (qc - m * G);
  }
  sf_wait_vm_loads();
  // the q rows' addresses, formed before any copy is in flight
  long long qoff[2];  // element offsets (a pinned pointer would lose its address space)
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    sf_pin(qrow[qs]);
    qoff[qs] = (long long)qrow[qs] * H * kHD + qhead[qs] * kHD + grp * 8;
    sf_pin(qoff[qs]);
  }
  __syncthreads();  // s_pg

  // copies: wave w fills rows 16(w&3) .. +16 of K (w < 4) or V (w >= 4) of a chunk;
  // the wave's 16-key group of chunk ci (past the range end: its last chunk again)
  // lies in one page
  const uint16_t* src_base = (is_v ? pv : pk) + head_off;
  int unit_off[kCopiesPerChunk];  // element offset of the logical unit this lane copies
#pragma unroll
  for (int i = 0; i < kCopiesPerChunk; ++i) {
    const int row = 16 * jg + 4 * i + (lane >> 4);
    const int p = lane & 15;
    unit_off[i] = (is_v ? v_unit(row, p) : k_unit(row, p)) * 8;
  }
  const int dst0 = (is_v ? kHalfBytes : 0) + 16 * jg * kRowBytes;
  const sf_lds_off pg_addr = sf_lds_addr(s_pg) + 4 * jg;
  auto issue = [&](int ci, uint8_t* slot) {
    const int cc = min(ci, c1 - 1);
    const int g0 = __builtin_amdgcn_readfirstlane(chunk_group_g0(cc, jg, last_g0));
    long long grow = (long long)g0 * kHD;
    if (page_table) {
      const int pg = __builtin_amdgcn_readfirstlane(
          (int)sf_lds_read4_now(pg_addr + 16 * (uint32_t)(cc - c0)));
      grow = (long long)pg * page_stride + (long long)(g0 & (page_size - 1)) * kHD;
    }
    const uint16_t* gsrc = src_base + grow;
#pragma unroll
    for (int i = 0; i < kCopiesPerChunk; ++i) {
      const int kr = group_key(4 * i + (lane >> 4), g0, P);
      sf_lds_dma16(gsrc + (size_t)kr * kHD + unit_off[i], slot + dst0 + 4 * i * kRowBytes);
    }
  };
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j) issue(c0 + j, ring + j * kSlotBytes);

  // Q^T operands: lane holds q[query][ds*32 + grp*8 .. +8] of its query in each of
  // the two 16-query tiles.  They complete (with the first copies) before the loop,
  // so its wait counts cover the copies alone.
  sf_u32x4 qf[2][4];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      qf[qs][ds] = *reinterpret_cast<const sf_u32x4*>(q_buf + qoff[qs] + ds * 32);
  sf_wait_vm_loads();
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) sf_pin(qf[qs][ds]);

  // ---- LDS read addresses (this lane, relative to a slot) ----------------------------
  // this wave's keys start at row 32 * kh of the chunk (a multiple of 16 rows: the
  // swizzles are unchanged)
  uint32_t koff[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = (uint32_t)(k_frag_off(lane, ds) + 32 * kh * kRowBytes);
  // v_tr_off(lane, dt) = v_tr_off(lane, 0) + 32 * ((dt ^ vsw) - vsw) with vsw the
  // row's v_unit term: the dim tile enters through v_unit's XOR only
  const int vrow = 4 * grp + (ql >> 2);
  const int vsw = vrow & 7;
  const uint32_t vlane = (uint32_t)(v_tr_off(lane, 0) - 32 * vsw + 32 * kh * kRowBytes);

  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  sf_f32x4 acc[2][8];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[qs][dt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int c, const uint8_t* slot) {
    const sf_lds_off base = sf_lds_addr(slot);
    sf_u32x4 kf[8];   // [t * 4 + ds]
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      kf[ds] = sf_lds_read16<0>(base + koff[ds]);
      kf[4 + ds] = sf_lds_read16<16 * kRowBytes>(base + koff[ds]);
    }
    sf_lds_reads_done(kf);

    // S^T tiles [t][qs] (raw dot products)
    float s[2][2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        sf_f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
          a = sf_mfma16x16x32(sf_as_bf16x8(kf[t * 4 + ds]), sf_as_bf16x8(qf[qs][ds]), a);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t][qs][i] = a[i];
      }
    const int kbase = c * kChunk + kh * 32 + grp * 4;  // key of s[0][.][0] of this lane
    if (kbase + 16 + 3 >= P) {  // a partial last chunk: keys past the prefix
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int qs = 0; qs < 2; ++qs)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kbase + 16 * t + i >= P) s[t][qs][i] = -INFINITY;
    }

    // online softmax per query (base 2, scores pre-scaled by log2(e) * scaling):
    // the max over the 4 lane groups first (lane shuffles go through the LDS
    // pipe), then the V^T operand reads, whose latency the exponentials cover
    float m_use[2], alpha[2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[t][qs][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[qs], mx * scale_log2);
      // a key half with no key yet (only past a short prefix's end) stays empty
      m_use[qs] = m_new == -INFINITY ? 0.f : m_new;
      alpha[qs] = __builtin_amdgcn_exp2f(m_run[qs] - m_use[qs]);
      m_run[qs] = m_new;
    }
    sf_u32x2 vf[16];  // [dt * 2 + t]
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const sf_lds_off va = base + vlane + (uint32_t)(((dt ^ vsw) & 7) * 32);
      vf[2 * dt] = sf_lds_read8_tr<0>(va);
      vf[2 * dt + 1] = sf_lds_read8_tr<16 * kRowBytes>(va);
    }
    float lsum[2] = {0.f, 0.f};
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[t][qs][i] = __builtin_amdgcn_exp2f(fmaf(s[t][qs][i], scale_log2, -m_use[qs]));
          lsum[qs] += s[t][qs][i];
        }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[qs][dt] = acc[qs][dt] * alpha[qs];
    }
    // the exponentials and rescales are done before the wait for the V^T reads
    // (an empty asm that takes them in keeps the compiler from sinking them past it)
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sf_pin(s[t][qs][i]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) sf_pin(acc[qs][dt]);
    }
    sf_lds_reads_done(vf);
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      lsum[qs] += __shfl_xor(lsum[qs], 16, 64);
      lsum[qs] += __shfl_xor(lsum[qs], 32, 64);
      l_run[qs] = l_run[qs] * alpha[qs] + lsum[qs];
    }

    // O^T += V^T P^T over the wave's 32 keys (smallest P part first)
    sf_bf16x8 pb[2][kPParts];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      float p2[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) p2[t][i] = s[t][qs][i];
      pv_parts<kPParts>(p2, pb[qs]);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const sf_u32x4 vw = {vf[2 * dt][0], vf[2 * dt][1], vf[2 * dt + 1][0], vf[2 * dt + 1][1]};
      const sf_bf16x8 va = sf_as_bf16x8(vw);
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int pp = kPParts - 1; pp >= 0; --pp)
          acc[qs][dt] = sf_mfma16x16x32(va, pb[qs][pp], acc[qs][dt]);
    }
  };

  // ---- the ring: chunk k of the range in slot k % kRing --------------------------------
  const int nck = c1 - c0;
#pragma unroll 1
  for (int k = 0; k < nck; ++k) {
    // chunk k has landed (each wave's copies complete in issue order), and every
    // wave is done with the slot the next issue overwrites (chunk k - 1's)
    sf_wait_vm_barrier<(kRing - 2) * kCopiesPerChunk>();
    issue(c0 + k + kRing - 1, ring + ((k + kRing - 1) % kRing) * kSlotBytes);
    compute(c0 + k, ring + (k % kRing) * kSlotBytes);
  }
  // drain the clamped re-issues past the range end before the ring is reused
  sf_wait_vm_barrier<0>();

  // ---- combine the two key halves of each query, write the partial -----------------
  float* xo = reinterpret_cast<float*>(ring);            // [qg][qs][dt][lane] x 4
  float* xml = xo + 4 * 2 * 8 * 64 * 4;                   // [qg][qs][ql] x (m, l)
  if (kh == 1) {
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<sf_f32x4*>(xo + (((qg * 2 + qs) * 8 + dt) * 64 + lane) * 4) = acc[qs][dt];
      if (grp == 0) {
        xml[((qg * 2 + qs) * 16 + ql) * 2] = m_run[qs];
        xml[((qg * 2 + qs) * 16 + ql) * 2 + 1] = l_run[qs];
      }
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const int qi = qt * kQT + qg * 32 + qs * 16 + ql;
      const float m1 = xml[((qg * 2 + qs) * 16 + ql) * 2];
      const float l1 = xml[((qg * 2 + qs) * 16 + ql) * 2 + 1];
      const float mm = fmaxf(m_run[qs], m1);  // finite: half 0 holds the range's first key
      const float w0 = __builtin_amdgcn_exp2f(m_run[qs] - mm);
      const float w1 = __builtin_amdgcn_exp2f(m1 - mm);
      if (qi < nq) {
        const size_t slot = attn_slot(h, r, qi, nr_cap, qmax);
        if (grp == 0) {
          ws_ml[slot * 2] = mm;
          ws_ml[slot * 2 + 1] = l_run[qs] * w0 + l1 * w1;
        }
        float* op = ws_o + slot * kHD + grp * 4;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const sf_f32x4 a1 =
              *reinterpret_cast<const sf_f32x4*>(xo + (((qg * 2 + qs) * 8 + dt) * 64 + lane) * 4);
          *reinterpret_cast<sf_f32x4*>(op + dt * 16) = acc[qs][dt] * w0 + a1 * w1;
        }
      }
    }
  }
}

// gridDim.x is a multiple of 8; XCD x (workgroups b with b % 8 == x) takes the
// x-th eighth of the item list, so consecutive items (the query tiles of one
// chunk range) share an L2.
__global__ __launch_bounds__(kPrefixThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sf_attn_prefix_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, const int32_t* __restrict__ page_table, int page_size,
    long long page_stride, long long head_stride, const int32_t* __restrict__ p_len, int P_cap,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ count_p, int bucket, int H,
    int Hkv, float scale_log2, int qmax, int nr_cap, float* __restrict__ ws_o,
    float* __restrict__ ws_ml) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRing * kSlotBytes];
  __shared__ int s_pg[4 * kMaxChunks];  // page of each 16-key group of the item's range
  const int G = H / Hkv;
  const int P = p_len ? min(*p_len, P_cap) : P_cap;
  if (P <= 0) return;
  const int nq = min(*count_p, bucket) * G;
  const PrefixGrid pg = prefix_grid(P, nq, Hkv);
  const int items = pg.n_qt * pg.nr * Hkv;
  const int xcd = blockIdx.x & 7;
  const int per = gridDim.x >> 3;
  const int end = xcd_begin(items, xcd + 1);
  for (int it = xcd_begin(items, xcd) + (int)(blockIdx.x >> 3); it < end; it += per) {
    const AttnItem item = attn_item(it, pg.n_qt, pg.nr);
    const int c0 = item.r * pg.cpi;
    prefix_item(q_buf, pk, pv, page_table, page_size, page_stride, head_stride, P, rows, nq, G, H,
                scale_log2, qmax, nr_cap, item.qt, item.r, c0, min(pg.nch, c0 + pg.cpi), item.h,
                ring, s_pg, ws_o, ws_ml);
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
                       uint16_t (*sv)[kHD], float (*ss)[kMaxN], float (*sml)[2 * kMaxRanges],
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
  __shared__ float sml[kMaxG][2 * kMaxRanges];   // per q-head: (m, l) of every range
  __shared__ float sM[kMaxG], sZ[kMaxG];
  const int count = min(*count_p, bucket);
  const int G = H / Hkv;
  const int P = p_len ? min(*p_len, P_cap) : P_cap;
  // number of prefix partials per query: the prefix kernel's chunk ranges
  const int nch = merge_ranges(P, count * G, Hkv);
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
  // per (kv head, chunk range, query): 128 fp32 acc + (m, l); queries per kv head =
  // bucket*G, so the total over kv heads is ranges * bucket * H slots.
  return (size_t)ranges_cap(P) * bucket * H * (kHD + 2) * sizeof(float);
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
    // a page holds whole 16-key groups: 16, 32, 64 or 128 keys
    if (page_table && (page_size < 16 || page_size > 128 || (page_size & (page_size - 1))))
      return SF_ERR_SHAPE;
    if (!page_table && head_stride < (long long)P * kHD) return SF_ERR_SHAPE;
    if (workspace_bytes < sf_attn_workspace_bytes(bucket, H, P)) return SF_ERR_WORKSPACE;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = H / Hkv;
  const int qmax = bucket * G;
  const int nch = P > 0 ? nchunks_for(P) : 0;
  const int nr_cap = P > 0 ? ranges_cap(P) : 0;
  const float scale_log2 = scaling * 1.44269504088896340736f;
  float* ws_ml = nullptr;
  float* ws_o = nullptr;
  if (P > 0) {
    const size_t nslot = (size_t)nr_cap * qmax * Hkv;
    ws_o = reinterpret_cast<float*>(workspace);
    ws_ml = ws_o + nslot * kHD;
    // persistent grid: one 128 KB-LDS workgroup per CU; a multiple of 8
    const int grid = prefix_launch_grid(qmax, nch, Hkv);
    hipLaunchKernelGGL(sf_attn_prefix_kernel, dim3(grid), dim3(kPrefixThreads), 0, st, q_buf,
                       prefix_k, prefix_v, page_table, page_size, page_stride, head_stride,
                       prefix_len, P, rows, count, bucket, H, Hkv, scale_log2, qmax, nr_cap, ws_o,
                       ws_ml);
  }
  const int grid2 = min(bucket * Hkv, 2 * kCUs);
  hipLaunchKernelGGL(sf_attn_block_merge_kernel, dim3(grid2), dim3(512), 0, st, q_buf, kv_buf,
                     src, rows, count, bucket, N, H, Hkv, scale_log2, block_causal ? 1 : 0,
                     P > 0 ? prefix_len : nullptr,
                     P, nr_cap, qmax, ws_o, ws_ml, o32, o_bf, m_tab, z_tab);
  return sf_launch_status();
}
