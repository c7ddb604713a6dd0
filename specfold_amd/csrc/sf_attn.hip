// Attention of the recomputed rows over [shared prefix ; own branch block],
// emitting the softmax state (m, Z) next to O.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:164-181 (fp32
// scores = (q . k) * scaling, m = max, Z = sum exp(s - m), O = sum exp(s - m) v / Z,
// no mask) and the Triton kernel specfold/generate/triton_kernels.py:301-361.
//
// Two kernels (flash-decoding split over the prefix, then the branch blocks):
//  * prefix (sf_attn_prefix_kernel): a persistent grid walks the active (query
//    tile, range of 64-key prefix chunks, kv head) items; the item count follows
//    the device-side row count and prefix length.  All recomputed rows x the G
//    q-heads of one kv head are flattened to queries qi = m*G + g and tiled 128
//    per item (32 per wave, against one key half of every chunk), so each prefix
//    K/V element is read by the few query tiles of its range instead of once per
//    row.  Items of one chunk range are consecutive and go to one XCD, so the
//    range's later reads hit that XCD's L2.  K/V chunks go straight to an LDS ring
//    by direct copies; scores are formed transposed, S^T = K Q^T, so every lane
//    holds keys of ONE query and the softmax is per lane; P^T feeds the P.V MFMA
//    from registers, V^T comes from transposing LDS reads.  P is split into bf16
//    hi + lo parts (two MFMAs), so P.V keeps ~16 mantissa bits, close to the
//    reference's fp32 einsum.  Each item writes its (m, l, acc) partial.
//  * rows (sf_attn_rows_kernel): one workgroup per (recomputed row, kv head)
//    merges the row's range partials into one prefix state per q-head and then
//    attends every row that takes this row's query -- itself and the folded rows
//    whose source it is -- over the prefix state and that row's own branch's N
//    block keys (gathered through src), on MFMA, writing O, m and Z.
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
constexpr float kLazy = 8.f;   // base-2 headroom of the softmax reference (exponentials <= 256)
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
  // the same offsets with the key row folded in, for a group of 16 keys in the prefix
  int lane_off[kCopiesPerChunk];
#pragma unroll
  for (int i = 0; i < kCopiesPerChunk; ++i) lane_off[i] = (4 * i + (lane >> 4)) * kHD + unit_off[i];
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
    if (g0 + 16 <= P) {  // wave-uniform: all 16 keys of the group exist
#pragma unroll
      for (int i = 0; i < kCopiesPerChunk; ++i)
        sf_lds_dma16(gsrc + lane_off[i], slot + dst0 + 4 * i * kRowBytes);
    } else {
#pragma unroll
      for (int i = 0; i < kCopiesPerChunk; ++i) {
        const int kr = group_key(4 * i + (lane >> 4), g0, P);
        sf_lds_dma16(gsrc + (size_t)kr * kHD + unit_off[i], slot + dst0 + 4 * i * kRowBytes);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < kRing - 2; ++j) issue(c0 + j, ring + j * kSlotBytes);

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

  // online softmax state per query: m_ref is the reference acc and l are kept
  // against (-inf: nothing accumulated yet), m_hi the running maximum.  The
  // reference is moved up to the maximum only when the maximum passes it by more
  // than kLazy (base 2), so most chunks skip the rescale of acc; every exponential
  // is then at most 2^kLazy.
  float m_ref[2] = {-INFINITY, -INFINITY}, m_hi[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  sf_f32x4 acc[2][8];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[qs][dt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  // Each chunk's P^T parts are carried into the next chunk's step, whose P.V MFMAs
  // for them (V^T read again from the carried chunk's slot, which the copies leave
  // alone until the step after) run beside that chunk's softmax arithmetic: the
  // wave's instruction stream interleaves them.  Before the first chunk the parts
  // are zero, so its step adds exact zeros.
  sf_bf16x8 pb[2][kPParts];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int pp = 0; pp < kPParts; ++pp) pb[qs][pp] = sf_as_bf16x8(sf_u32x4{0u, 0u, 0u, 0u});

  // the V^T operands of the slot at `base` (32 keys x 16 dims per dim tile: two
  // transposing reads each); complete after sf_lds_reads_done
  auto read_vt = [&](sf_lds_off base, sf_u32x2 (&vf)[16]) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const sf_lds_off va = base + vlane + (uint32_t)(((dt ^ vsw) & 7) * 32);
      vf[2 * dt] = sf_lds_read8_tr<0>(va);
      vf[2 * dt + 1] = sf_lds_read8_tr<16 * kRowBytes>(va);
    }
  };
  // O^T += V^T P^T over the wave's 32 keys of the carried chunk (each acc tile takes
  // the smallest P part first)
  auto add_pv = [&](const sf_u32x2 (&vf)[16]) {
#pragma unroll
    for (int pp = kPParts - 1; pp >= 0; --pp)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const sf_u32x4 vw = {vf[2 * dt][0], vf[2 * dt][1], vf[2 * dt + 1][0], vf[2 * dt + 1][1]};
#pragma unroll
        for (int qs = 0; qs < 2; ++qs)
          acc[qs][dt] = sf_mfma16x16x32(sf_as_bf16x8(vw), pb[qs][pp], acc[qs][dt]);
      }
  };

  // chunk c in the slot at `base`; the carried chunk's slot at `vbase`
  // a rescale of acc decided by a step, applied at the start of the next (after the
  // P.V that step added, before the one the next adds)
  bool resc_prev = false;
  float alpha_prev[2] = {1.f, 1.f};
  auto rescale = [&]() {
    if (resc_prev) {
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[qs][dt] = acc[qs][dt] * alpha_prev[qs];
    }
  };

  auto step = [&](int c, sf_lds_off base, sf_lds_off vbase) {
    rescale();
    sf_u32x4 kf[8];   // [t * 4 + ds]
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      kf[ds] = sf_lds_read16<0>(base + koff[ds]);
      kf[4 + ds] = sf_lds_read16<16 * kRowBytes>(base + koff[ds]);
    }
    sf_lds_reads_done(kf);

    // S^T tiles [t][qs] (raw dot products; four independent accumulations)
    sf_f32x4 sa[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) sa[t][qs] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int qs = 0; qs < 2; ++qs)
          sa[t][qs] = sf_mfma16x16x32(sf_as_bf16x8(kf[t * 4 + ds]), sf_as_bf16x8(qf[qs][ds]), sa[t][qs]);
    float s[2][2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t][qs][i] = sa[t][qs][i];
    // the carried chunk's V^T, once the K fragments are consumed (no scheduling
    // across this point: the two operand sets are never live together)
    __builtin_amdgcn_sched_barrier(0);
    sf_u32x2 vf[16];
    read_vt(vbase, vf);
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

    // online softmax per query (base 2, scores pre-scaled by log2(e) * scaling).
    // m_hi is kept per lane (the maximum of the lane's own keys) and checked against
    // the reference per lane; only a rescale takes the maximum over the query's four
    // lane groups (shuffles), so most chunks need no cross-lane step
    bool need = false;
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[t][qs][i]);
      mx *= scale_log2;
      m_hi[qs] = fmaxf(m_hi[qs], mx);
      need = need | (mx > m_ref[qs] + kLazy);   // m_ref -inf: any finite key
    }
    // wave-uniform: move every query of the wave's reference to its running
    // maximum.  acc is rescaled at the start of the next step, after the carried
    // chunk's P.V (its P is against the old reference) has been added: the same
    // acc * alpha + P.V sequence, one chunk later.
    const bool resc = __ballot(need) != 0;
    float alpha[2] = {1.f, 1.f};
    if (resc) {
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        float mx = m_hi[qs];
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        m_hi[qs] = mx;
        // a key half with no key yet (only past a short prefix's end) stays empty
        const float nr = mx == -INFINITY ? 0.f : mx;
        alpha[qs] = __builtin_amdgcn_exp2f(m_ref[qs] - nr);
        m_ref[qs] = mx;
      }
    }
    float m_use[2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) m_use[qs] = m_ref[qs] == -INFINITY ? 0.f : m_ref[qs];
    sf_lds_reads_done(vf);
    add_pv(vf);
    float lsum[2] = {0.f, 0.f};
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      float p2[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p2[t][i] = __builtin_amdgcn_exp2f(fmaf(s[t][qs][i], scale_log2, -m_use[qs]));
          lsum[qs] += p2[t][i];
        }
      pv_parts<kPParts>(p2, pb[qs]);
    }
    // l is kept per lane (its own keys' terms; alpha is the same for the query's
    // four lane groups) and summed over them when the range is done
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) l_run[qs] = l_run[qs] * alpha[qs] + lsum[qs];
    // one MFMA of the carried P.V, then three VALU operations (the exponentials and
    // the P parts of this chunk), and so on: the matrix core and the VALU work side
    // by side within the wave
#pragma unroll
    for (int i = 0; i < 16 * kPParts; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 3, 0);
    }
    resc_prev = resc;
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) alpha_prev[qs] = alpha[qs];
  };

  // ---- the ring: chunk k of the range in slot k % kRing, copied kAhead chunks
  // ahead; its slot is rewritten kRing - kAhead steps later (step k + 1 still reads
  // its V^T) --------------------------------------------------------------------------
  constexpr int kAhead = kRing - 2;
  const int nck = c1 - c0;
#pragma unroll 1
  for (int k = 0; k < nck; ++k) {
    // chunk k has landed (each wave's copies complete in issue order), and every
    // wave is done with the slot the next issue overwrites (chunk k - 2's)
    sf_wait_vm_barrier<(kAhead - 1) * kCopiesPerChunk>();
    issue(c0 + k + kAhead, ring + ((k + kAhead) % kRing) * kSlotBytes);
    // (the first step's zero P parts take chunk 0's own V^T: landed, finite values,
    // where the carried slot would hold stale LDS bytes, possibly NaN patterns)
    const sf_lds_off cur = sf_lds_addr(ring + (k % kRing) * kSlotBytes);
    step(c0 + k, cur, k == 0 ? cur : sf_lds_addr(ring + ((k + kRing - 1) % kRing) * kSlotBytes));
  }
  {  // the last chunk's P.V
    rescale();
    sf_u32x2 vf[16];
    read_vt(sf_lds_addr(ring + ((nck + kRing - 1) % kRing) * kSlotBytes), vf);
    sf_lds_reads_done(vf);
    add_pv(vf);
  }
  // drain the clamped re-issues past the range end before the ring is reused
  sf_wait_vm_barrier<0>();

  // ---- combine the two key halves of each query, write the partial -----------------
  // the query's maximum and l over its four lane groups
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    m_hi[qs] = fmaxf(m_hi[qs], __shfl_xor(m_hi[qs], 16, 64));
    m_hi[qs] = fmaxf(m_hi[qs], __shfl_xor(m_hi[qs], 32, 64));
    l_run[qs] += __shfl_xor(l_run[qs], 16, 64);
    l_run[qs] += __shfl_xor(l_run[qs], 32, 64);
  }
  float* xo = reinterpret_cast<float*>(ring);            // [qg][qs][dt][lane] x 4
  float* xml = xo + 4 * 2 * 8 * 64 * 4;   // [qg][qs][ql] x (m_ref, l, m_hi, -)
  if (kh == 1) {
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<sf_f32x4*>(xo + (((qg * 2 + qs) * 8 + dt) * 64 + lane) * 4) = acc[qs][dt];
      if (grp == 0) {
        xml[((qg * 2 + qs) * 16 + ql) * 4] = m_ref[qs];
        xml[((qg * 2 + qs) * 16 + ql) * 4 + 1] = l_run[qs];
        xml[((qg * 2 + qs) * 16 + ql) * 4 + 2] = m_hi[qs];
      }
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const int qi = qt * kQT + qg * 32 + qs * 16 + ql;
      // the partial is kept against the range's maximum mm: each half's (acc, l)
      // moves from its reference to mm (an empty half 1 has m_ref -inf: weight 0)
      const float m1 = xml[((qg * 2 + qs) * 16 + ql) * 4];
      const float l1 = xml[((qg * 2 + qs) * 16 + ql) * 4 + 1];
      const float h1 = xml[((qg * 2 + qs) * 16 + ql) * 4 + 2];
      const float mm = fmaxf(m_hi[qs], h1);  // finite: half 0 holds the range's first key
      const float w0 = __builtin_amdgcn_exp2f(m_ref[qs] - mm);
      const float w1 = __builtin_amdgcn_exp2f(m1 - mm);
      if (qi < nq) {
        const size_t slot = attn_slot(h, r, qi, nr_cap, qmax);
        if (grp == 0) {
          sf_handoff_store(reinterpret_cast<sf_f32x2*>(ws_ml + slot * 2),
                           sf_f32x2{mm, l_run[qs] * w0 + l1 * w1});
        }
        float* op = ws_o + slot * kHD + grp * 4;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const sf_f32x4 a1 =
              *reinterpret_cast<const sf_f32x4*>(xo + (((qg * 2 + qs) * 8 + dt) * 64 + lane) * 4);
          sf_handoff_store(reinterpret_cast<sf_f32x4*>(op + dt * 16), acc[qs][dt] * w0 + a1 * w1);
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

// ---- rows: the prefix merge and the block attention, per source row ---------------------
// One 8-wave workgroup per (compacted row m, kv head h).  Its row r = rows[m] = (b, n)
// was recomputed.  The nr range partials of its G q-heads are merged into one
// prefix state {acc[128], m, l} per q-head (m in the scaled base-2 domain of the
// partials), held in LDS: wave g merges q-head g, lane l dims 2l, 2l+1 and the
// (m, l) of range l (nr <= 64).  Every row of position n that takes r's query --
// r itself, and (FOLDED) each folded row (b', n) whose source is r, i.e.
// src[b'*N + n] == b -- then attends with that query over the merged prefix and
// over its own branch b''s N block keys (kv rows src[b'*N + j]*N + j).  For a
// folded row this is the softmax over its own keys that the reference reaches by
// chain correction (fastdllm_v2_folded.py:183-204: the old keys' terms swapped for
// the new ones); the prefix part is the same for all of them, so it is merged once.
// The waves deal those rows out (one each up to 8 branches): the G q-heads are the
// columns of one 16-query MFMA tile (columns past G repeat q-head G - 1; their
// results are dropped); block scores S^T = K Q^T with the K fragments read straight
// from the kv rows, O^T += V^T P^T with the branch's V rows copied to the wave's own
// LDS region for the transposing reads.
// Latency: the row, the src table and the count are one round of loads; the
// partials and the query go out as soon as the count is known; the first row's K
// and V once the src table is in LDS, before the merge arithmetic.
// FOLDED = false computes the listed rows only (each is its own and only row).
constexpr int kRowsWaves = 8;
constexpr int kRowsThreads = kRowsWaves * 64;
constexpr int kMaxBucket = 1024;  // compacted rows, B1 * N <= 1024
constexpr int kMaxB1 = 64;        // branches: one ballot covers them

// The block K fragments (S^T tiles t of 16 keys, MFMA A operand: lane l holds key
// 16t + l%16, dims 32 ds + 8 (l/16) .. +8) of kv head h for branch bd, straight from
// the kv rows (keys past N repeat key N - 1, finite under their zero weights), and
// the V rows of the branch by direct copies to the wave's LDS region sv (row r at
// r * kRowBytes, 16-byte unit p holding logical unit v_unit(r, p); rows padded to
// 64 rows the same way).  Lane L looks up the kv row of key L once;
// the other lanes' rows come by shuffles, so the loads are not held up by a chain
// of LDS reads.
template <int NB>
SF_DEV void row_kv_issue(const uint16_t* __restrict__ kv_buf, const int* s_src, int bd, int N,
                         int Hkv, int h, sf_u32x4 (&kf)[NB / 16][4], uint8_t* sv) {
  // every tile and copy of the NB-key block is issued whatever N is (keys past N
  // repeat key N - 1), so the loads carry no branches and the compiler's wait
  // counts after them stay exact
  constexpr int NT = NB / 16, NC = NB / 4;
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
  const size_t kvs = (size_t)2 * Hkv * kHD;
  const int jl = sf_imin(lane, N - 1);
  const int row_l = s_src[bd * N + jl] * N + jl;   // kv row of key lane (N <= 64)
  int krow[NT], vrow[NC];
#pragma unroll
  for (int t = 0; t < NT; ++t) krow[t] = __shfl(row_l, 16 * t + (lane & 15), 64);
#pragma unroll
  for (int i = 0; i < NC; ++i) vrow[i] = __shfl(row_l, 4 * i + (lane >> 4), 64);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint16_t* kp = kv_buf + (size_t)krow[t] * kvs + h * kHD + grp * 8;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) kf[t][ds] = *reinterpret_cast<const sf_u32x4*>(kp + ds * 32);
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int row = 4 * i + (lane >> 4);
    const uint16_t* vp = kv_buf + (size_t)vrow[i] * kvs + (Hkv + h) * kHD;
    sf_lds_dma16(vp + v_unit(row, lane & 15) * 8, sv + i * 1024);
  }
}

// NB = 32: two workgroups per CU (<= 128 VGPRs, 72 KB of LDS each), so a launch of
// more (row, kv head) items than CUs (cfg5: 39 x 8) runs in one round
template <bool FOLDED, int NB>
__global__ __launch_bounds__(kRowsThreads)
__attribute__((amdgpu_waves_per_eu(NB == 32 ? 4 : 2, NB == 32 ? 4 : 2))) void
sf_attn_rows_kernel(
    const uint16_t* __restrict__ q_buf, const uint16_t* __restrict__ kv_buf,
    const int32_t* __restrict__ src, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ count_p, int bucket, int B1, int N, int b_first, int b_count,
    int H, int Hkv, float scale_log2, int causal, const int32_t* __restrict__ p_len, int P_cap,
    int nr_cap, int qmax, const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
    float* __restrict__ o32, uint16_t* __restrict__ o_bf, float* __restrict__ m_tab,
    float* __restrict__ z_tab) {
  constexpr int NT = NB / 16;   // 16-key tiles of the block
  __shared__ __attribute__((aligned(16))) uint8_t sV[kRowsWaves][NB * kRowBytes];
  __shared__ __attribute__((aligned(16))) float sAcc[kMaxG][kHD];
  __shared__ float sM[kMaxG], sL[kMaxG];
  __shared__ int sSrc[kMaxBucket];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int grp = lane >> 4;
  const int ql = lane & 15;
  const int G = H / Hkv;
  const int m = blockIdx.x / Hkv;   // < bucket: the grid is bucket * Hkv
  const int h = blockIdx.x - m * Hkv;
  const int BN = B1 * N;

  // ---- round 1: the row, the src table, the count and the prefix length, as one
  // round of loads: the exit test reads all of them (r < BN and P >= 0 always hold),
  // so the compiler cannot sink any load past it, and the whole table is written
  // (entries past BN repeat the last) with no branch -------------------------------------
  const int r = rows[m];
  const int cnt_raw = *count_p;
  const int plen_raw = *(p_len ? p_len : count_p);   // a select, not a branch
  const int count = min(cnt_raw, bucket);
  const int P = P_cap > 0 ? (p_len ? min(plen_raw, P_cap) : P_cap) : 0;
  constexpr int kSrcPerThread = kMaxBucket / kRowsThreads;
  int srcv[kSrcPerThread];
#pragma unroll
  for (int k = 0; k < kSrcPerThread; ++k) srcv[k] = src[min(tid + k * kRowsThreads, BN - 1)];
#pragma unroll
  for (int k = 0; k < kSrcPerThread; ++k) sSrc[tid + k * kRowsThreads] = srcv[k];
  if ((m >= count) | (r >= BN) | (P < 0)) return;   // workgroup-uniform; no short circuit
  const int b = r / N;
  const int n = r - b * N;
  const int nr = P > 0 ? merge_ranges(P, count * G, Hkv) : 0;

  // ---- round 2: this wave's q-head's range partials and the query -------------------------
  // Branch-free: without a prefix (nr = 0) the loads re-read q (any valid address)
  // and are dropped; waves past G load q-head G - 1's and drop them.
  constexpr int kB = 16;  // range partials loaded per round (clamped addresses)
  const int gm = min(wv, G - 1);
  const int qi = m * G + gm;
  // range u of query qi sits at attn_slot(h, u, qi) = attn_slot(h, 0, qi) + u * qmax
  const bool pre = nr > 0;
  const size_t slot0 = pre ? attn_slot(h, 0, qi, nr_cap, qmax) : 0;
  const size_t rstride = pre ? (size_t)qmax : 0;
  const float* pw_o = pre ? ws_o + slot0 * kHD + 2 * lane : reinterpret_cast<const float*>(q_buf);
  const float* pw_ml = pre ? ws_ml + slot0 * 2 : reinterpret_cast<const float*>(q_buf);
  const int nr1 = max(nr, 1);
  sf_f32x2 ml = sf_handoff_load(
      reinterpret_cast<const sf_f32x2*>(pw_ml + (size_t)min(lane, nr1 - 1) * rstride * 2));
  sf_f32x2 a[kB];
#pragma unroll
  for (int u = 0; u < kB; ++u)
    a[u] = sf_handoff_load(
        reinterpret_cast<const sf_f32x2*>(pw_o + (size_t)min(u, nr1 - 1) * rstride * kHD));
  // Q^T operand: lane holds q[q-head ql][ds*32 + grp*8 .. +8] of row r
  sf_u32x4 qf[4];
  {
    const int hq = h * G + min(ql, G - 1);
    const uint16_t* qp = q_buf + (size_t)r * H * kHD + hq * kHD + grp * 8;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const sf_u32x4*>(qp + ds * 32);
  }
  sf_lds_barrier();  // sSrc (the partials and the query stay in flight)

  // ---- this wave's rows: every kRowsWaves-th of the rows that take r's query, in
  // branch order (one ballot: B1 <= 64); the first one's K and V go out now ----------------
  unsigned long long mine = 0;
  {
    const int bb = b_first + lane;
    const bool dep = lane < b_count && (FOLDED ? sSrc[bb * N + n] == b : bb == b);
    unsigned long long mask = __ballot(dep);
    for (int k = 0; mask; ++k) {
      const unsigned long long bit = mask & (0ull - mask);
      if ((k & (kRowsWaves - 1)) == wv) mine |= bit;
      mask ^= bit;
    }
  }
  uint8_t* sv = sV[wv];
  sf_u32x4 kf[NT][4];
  int bd = mine ? b_first + __builtin_ctzll(mine) : -1;   // wave-uniform
  // a wave without a row issues its own branch's copies too (dropped): no branch
  row_kv_issue<NB>(kv_buf, sSrc, bd >= 0 ? bd : b, N, Hkv, h, kf, sv);

  // ---- the merged prefix state of q-head wv ------------------------------------------------
  if (wv < G) {  // wave-uniform
    float2 acc = make_float2(0.f, 0.f);
    float mm = -INFINITY, l = 0.f;
    if (nr > 0) {
      ml = lane < nr ? ml : sf_f32x2{-INFINITY, 0.f};
      mm = sf_wave_max(ml.x);  // -inf only with no prefix key at all
      const float w = (lane < nr && mm > -INFINITY) ? __builtin_amdgcn_exp2f(ml.x - mm) : 0.f;
      l = sf_wave_sum(ml.y * w);
      for (int r0 = 0; r0 < nr; r0 += kB) {
        if (r0 > 0) {
#pragma unroll
          for (int u = 0; u < kB; ++u)
            a[u] = sf_handoff_load(reinterpret_cast<const sf_f32x2*>(
                pw_o + (size_t)min(r0 + u, nr - 1) * rstride * kHD));
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const float wr = __shfl(w, min(r0 + u, 63), 64);   // 0 past nr
          acc.x = fmaf(wr, a[u].x, acc.x);
          acc.y = fmaf(wr, a[u].y, acc.y);
        }
      }
    }
    *reinterpret_cast<float2*>(&sAcc[wv][2 * lane]) = acc;
    if (lane == 0) {
      sM[wv] = mm;
      sL[wv] = l;
    }
  }
  // the states are in LDS for every wave (the block copies stay in flight)
  sf_lds_barrier();

  const int gq = min(ql, G - 1);
  const float m_run = sM[gq], l_run = sL[gq];
  while (bd >= 0) {  // wave-uniform
    // ---- block scores S^T = K Q^T ----------------------------------------------------------
    float s_t[NT][4];  // [key tile][i]: key 16t + 4*grp + i of this lane's query
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      sf_f32x4 acc_s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds)
        acc_s = sf_mfma16x16x32(sf_as_bf16x8(kf[t][ds]), sf_as_bf16x8(qf[ds]), acc_s);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * t + 4 * grp + i;
        const bool keep = j < N && !(causal && j > n);
        s_t[t][i] = keep ? acc_s[i] : -INFINITY;   // exp2 gives 0
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s_t[t][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx * scale_log2);   // finite: key 0 is never masked
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float lsum = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s_t[t][i] = __builtin_amdgcn_exp2f(fmaf(s_t[t][i], scale_log2, -m_new));
        lsum += s_t[t][i];
      }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    const float l_new = l_run * alpha + lsum;
    // the prefix state's acc (O^T layout: dims 16 dt + 4 grp + i of q-head gq), rescaled
    sf_f32x4 acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      acc[dt] = *reinterpret_cast<const sf_f32x4*>(&sAcc[gq][dt * 16 + grp * 4]) * alpha;

    // ---- O^T += V^T P^T over 32-key blocks (the V copies landed) -------------------------------
    sf_wait_vm_loads();
#pragma unroll
    for (int kb = 0; kb < NB / 32; ++kb) {
      {
        float p2[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) p2[t][i] = s_t[2 * kb + t][i];   // 0 past key N - 1
        sf_bf16x8 pb[kPParts];
        pv_parts<kPParts>(p2, pb);
        sf_u32x2 vf[16];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          // v_tr_off counts from a staged chunk's K rows; the region holds V rows only
          const sf_lds_off va = sf_lds_addr(sv) - (uint32_t)kHalfBytes +
                                (uint32_t)(v_tr_off(lane, dt) + 32 * kb * kRowBytes);
          vf[2 * dt] = sf_lds_read8_tr<0>(va);
          vf[2 * dt + 1] = sf_lds_read8_tr<16 * kRowBytes>(va);
        }
        sf_lds_reads_done(vf);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const sf_u32x4 vw = {vf[2 * dt][0], vf[2 * dt][1], vf[2 * dt + 1][0], vf[2 * dt + 1][1]};
          const sf_bf16x8 va = sf_as_bf16x8(vw);
#pragma unroll
          for (int pp = kPParts - 1; pp >= 0; --pp) acc[dt] = sf_mfma16x16x32(va, pb[pp], acc[dt]);
        }
      }
    }

    // ---- outputs of row (bd, n) ---------------------------------------------------------------
    if (ql < G) {
      const int ro = bd * N + n;
      const int hq = h * G + ql;
      const float inv = 1.0f / l_new;
      const size_t off = (size_t)ro * H * kHD + hq * kHD + grp * 4;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const sf_f32x4 o = acc[dt] * inv;
        if (o32) *reinterpret_cast<sf_f32x4*>(o32 + off + dt * 16) = o;   // (kernel argument)
        sf_u32x2 w;
        w[0] = sf_pack2(o[0], o[1]);
        w[1] = sf_pack2(o[2], o[3]);
        sf_handoff_store(reinterpret_cast<sf_u32x2*>(o_bf + off + dt * 16), w);
      }
      if (grp == 0) {
        // the natural-base max the scores were measured from
        if (m_tab) m_tab[(size_t)ro * H + hq] = m_new * 0.69314718055994530942f;
        if (z_tab) z_tab[(size_t)ro * H + hq] = l_new;
      }
    }
    // the next row of this wave (its V copies overwrite the region: the reads of
    // this one are done)
    mine &= mine - 1;
    bd = mine ? b_first + __builtin_ctzll(mine) : -1;
    if (bd >= 0) row_kv_issue<NB>(kv_buf, sSrc, bd, N, Hkv, h, kf, sv);
  }
}

}  // namespace

namespace {

size_t partial_bytes(int bucket, int H, int P) {
  return (size_t)ranges_cap(P) * bucket * H * (kHD + 2) * sizeof(float);
}

// The prefix pass, then the merge + block attention for the rows of branches
// [b_first, b_first + b_count) (FOLDED: folded rows too).
int attention(bool folded, const uint16_t* q_buf, const uint16_t* kv_buf,
              const uint16_t* prefix_k, const uint16_t* prefix_v, const int32_t* page_table,
              int P, int page_size, long long page_stride, long long head_stride,
              const int32_t* src, const int32_t* rows, const int32_t* count, int bucket, int B1,
              int N, int b_first, int b_count, int H, int Hkv, int hd, float scaling,
              const int32_t* prefix_len, int block_causal, float* o32, uint16_t* o_bf,
              float* m_tab, float* z_tab, void* workspace, size_t workspace_bytes,
              hipStream_t st) {
  // o32, m_tab and z_tab may be NULL (not written): o_proj reads o_bf only
  if (!q_buf || !kv_buf || !src || !rows || !count || !o_bf) return SF_ERR_ARG;
  if (hd != kHD || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > kMaxG) return SF_ERR_SHAPE;
  if (N < 1 || N > kMaxN || B1 < 1 || bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  // the rows kernel stages src in a kMaxBucket-entry LDS table and finds a row's
  // branches with one 64-lane ballot
  if (bucket > kMaxBucket || B1 * N > kMaxBucket || B1 > kMaxB1) return SF_ERR_SHAPE;
  if (b_first < 0 || b_count < 1 || b_first + b_count > B1) return SF_ERR_SHAPE;
  if (P < 0 || nchunks_for(P) > kMaxChunks) return SF_ERR_SHAPE;
  if (P > 0) {
    if (!prefix_k || !prefix_v || !workspace) return SF_ERR_ARG;
    // a page holds whole 16-key groups: 16, 32, 64 or 128 keys
    if (page_table && (page_size < 16 || page_size > 128 || (page_size & (page_size - 1))))
      return SF_ERR_SHAPE;
    if (!page_table && head_stride < (long long)P * kHD) return SF_ERR_SHAPE;
    if (workspace_bytes < sf_attn_workspace_bytes(bucket, H, P)) return SF_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return SF_ERR_ARG;
  }
  const int G = H / Hkv;
  const int qmax = bucket * G;
  const float scale_log2 = scaling * 1.44269504088896340736f;
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
  int nr_cap = 0;
  if (P > 0) {
    const int nch = nchunks_for(P);
    nr_cap = ranges_cap(P);
    const size_t nslot = (size_t)nr_cap * qmax * Hkv;
    ws_o = reinterpret_cast<float*>(workspace);
    ws_ml = ws_o + nslot * kHD;
    // persistent grid: one 136 KB-LDS workgroup per CU; a multiple of 8
    const int grid = prefix_launch_grid(qmax, nch, Hkv);
    hipLaunchKernelGGL(sf_attn_prefix_kernel, dim3(grid), dim3(kPrefixThreads), 0, st, q_buf,
                       prefix_k, prefix_v, page_table, page_size, page_stride, head_stride,
                       prefix_len, P, rows, count, bucket, H, Hkv, scale_log2, qmax, nr_cap, ws_o,
                       ws_ml);
  }
  const dim3 grid2(bucket * Hkv);
  const int causal = block_causal ? 1 : 0;
#define SF_ATTN_ROWS(F, NB)                                                                      \
  hipLaunchKernelGGL((sf_attn_rows_kernel<F, NB>), grid2, dim3(kRowsThreads), 0, st, q_buf,     \
                     kv_buf, src, rows, count, bucket, B1, N, b_first, b_count, H, Hkv,          \
                     scale_log2, causal, prefix_len, P, nr_cap, qmax, ws_o, ws_ml, o32, o_bf,    \
                     m_tab, z_tab)
  if (folded) {
    if (N <= 32) SF_ATTN_ROWS(true, 32); else SF_ATTN_ROWS(true, 64);
  } else {
    if (N <= 32) SF_ATTN_ROWS(false, 32); else SF_ATTN_ROWS(false, 64);
  }
#undef SF_ATTN_ROWS
  return sf_launch_status();
}

}  // namespace

extern "C" size_t sf_attn_workspace_bytes(int bucket, int H, int P) {
  if (bucket < 1 || H < 1 || P < 0) return 0;
  if (P == 0) return 16;
  // the range partials: per (kv head, chunk range, query) 128 fp32 acc + (m, l), with
  // bucket*G queries per kv head: ranges * bucket * H slots
  return partial_bytes(bucket, H, P);
}

extern "C" int sf_attn_prefix_block(const uint16_t* q_buf, const uint16_t* kv_buf,
                                    const uint16_t* prefix_k, const uint16_t* prefix_v,
                                    const int32_t* page_table, int P, int page_size,
                                    long long page_stride, long long head_stride,
                                    const int32_t* src, const int32_t* rows, const int32_t* count,
                                    int bucket, int B1, int N, int H, int Hkv, int hd,
                                    float scaling, const int32_t* prefix_len, int block_causal,
                                    float* o32, uint16_t* o_bf, float* m_tab, float* z_tab,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  return attention(false, q_buf, kv_buf, prefix_k, prefix_v, page_table, P, page_size,
                   page_stride, head_stride, src, rows, count, bucket, B1, N, 0, B1, H, Hkv, hd,
                   scaling, prefix_len, block_causal, o32, o_bf, m_tab, z_tab, workspace,
                   workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sf_attn_rows(const uint16_t* q_buf, const uint16_t* kv_buf,
                            const uint16_t* prefix_k, const uint16_t* prefix_v,
                            const int32_t* page_table, int P, int page_size, long long page_stride,
                            long long head_stride, const int32_t* src, const int32_t* rows,
                            const int32_t* count, int bucket, int B1, int N, int b_first,
                            int b_count, int H, int Hkv, int hd, float scaling,
                            const int32_t* prefix_len, float* o32, uint16_t* o_bf, float* m_tab,
                            float* z_tab, void* workspace, size_t workspace_bytes, void* stream) {
  return attention(true, q_buf, kv_buf, prefix_k, prefix_v, page_table, P, page_size, page_stride,
                   head_stride, src, rows, count, bucket, B1, N, b_first, b_count, H, Hkv, hd,
                   scaling, prefix_len, 0, o32, o_bf, m_tab, z_tab, workspace, workspace_bytes,
                   reinterpret_cast<hipStream_t>(stream));
}
