// Weight-streaming GEMM core for skinny row blocks:  C[m, n] = sum_k A[arow(m), k] * W[n, k]
//
// Shapes on this path: M = recomputed rows (<= 256, often 30-120) or all BN rows,
// N and K = 1.5k-152k; W (bf16, [N, K], packed fragment-major) is the big operand
// and is read once from HBM.  One workgroup of 8 waves per CU; wave w owns WN
// column tiles of 16 (column group w), so the workgroup covers 128*WN columns.
// ALL rows of A (up to MB = 64 or 128 per pass: one pass over the weights for
// every row up to 128) are staged through a ring of LDS buffers, 64 K at a time,
// and shared by the 8 waves; the weights go to LDS too, each wave's own
// fragments.  Work is split stream-K: a grid of one workgroup per CU, each taking
// an equal share of the (tile, K stage) units; tiles shared by several workgroups
// are summed by a fix-up
// kernel.  MFMA: v_mfma_f32_16x16x32_bf16, fp32 accumulation.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (64 lanes): A 16x32 — lane l holds
// A[l%16][8*(l/16) .. +8]; B 32x16 — lane l holds B[8*(l/16) .. +8][l%16];
// D 16x16 — lane l holds D[4*(l/16) + i][l%16], i = 0..3.
#pragma once

#include "sf_common.h"
#include "sf_compact.h"
#include "sf_index.h"

namespace sfg {

constexpr int kThreads = 512; // 8 waves
// kKC (K per stage), kLdsBudget and SFG_RING_MAX: sf_index.h

// One ring stage of a workgroup of up to MB rows and WN weight tiles per wave:
// the two 32-K chunks of the MB/16 A m tiles (1 KB per (chunk, m tile)), then
// every wave's WN weight fragments of its chunk (1 KB each, in lane order: the
// packed layout).  Sizes in 16-byte words.  The ring holds as many stages as fit
// kLdsBudget, at most SFG_RING_MAX.
// kWReg (one weight tile per wave: down, QKV): the weights skip LDS -- each lane
// loads the 16-byte fragment its MFMA takes straight into a VGPR ring of the same
// depth -- and a stage in LDS is the A rows alone.  A direct global->LDS copy
// stream runs at ~5.5 TB/s on MI355X against ~6.5 TB/s for the same stream through
// VGPRs (measured with the A copies and the per-stage barrier kept).  gate/up (two
// tiles per wave) keeps its weights on the LDS path: the register ring (3 stages,
// all the VGPRs allow) measured faster at one shape and slower at three.
template <int MB, int WN>
struct Stage {
  static constexpr bool kWReg = WN == 1;
  static constexpr int kA = 2 * (MB / 16) * 64;   // words of A per stage
  static constexpr int kW = kWReg ? 0 : 8 * WN * 2 * 64;   // words of weights per stage
  static constexpr int kWords = kA + kW;
  // kWReg: 4 stages (3 in flight: the register stream's rate, and what the kernels'
  // scalar registers allow without spilling)
  static constexpr int kRingMax = kWReg ? 4 : SFG_RING_MAX;
  static constexpr int kRing =
      kLdsBudget / (kWords * 16) < kRingMax ? kLdsBudget / (kWords * 16) : kRingMax;
};

// The fragments are read from the ring by sf_lds_read16, which the compiler does
// not track, so it adds no wait for the copies in flight (the waits are
// sf_wait_vm_barrier's and sf_lds_reads_done's).  A rows are 64 bytes per
// tile row, whose four 16-byte units are XOR-swizzled — unit u of tile row r
// sits at position u ^ a_swz(r), so the 16 lanes of a fragment read that share
// a unit hit distinct banks.
template <int MB, int WN>
struct Ring {
  sf_u32x4* slot[8];
};

// Rows handled by one workgroup of a launch whose row count is at most mcap.
inline int row_block(int mcap) { return mcap <= 64 ? 64 : 128; }

// The A fragments (NMT m tiles, 1 KB apart) and weight fragments (WN tiles, CPS KB
// apart: a tile's CPS chunk blocks follow each other) of K chunk C of a stage, read
// from LDS without waiting (sf_lds_read16 with compile-time offsets).
template <int NMT, int WN, int CPS = 2, int I = 0>
SF_DEV void lds_fragments(sf_u32x4 (&f)[NMT + WN], sf_lds_off a_addr, sf_lds_off w_addr) {
  if constexpr (I < NMT) {
    f[I] = sf_lds_read16<I * 1024>(a_addr);
    lds_fragments<NMT, WN, CPS, I + 1>(f, a_addr, w_addr);
  } else if constexpr (I < NMT + WN) {
    f[I] = sf_lds_read16<(I - NMT) * CPS * 1024>(w_addr);
    lds_fragments<NMT, WN, CPS, I + 1>(f, a_addr, w_addr);
  }
}

// Main loop over stages [s0, s1) of K (64 each: two 32-wide MFMA chunks) for NMT
// m tiles of 16 rows.  `wsrc[t]` is this lane's weight stream for column tile t;
// `acc[mt][t]` accumulates rows mt*16.., column tile t; `rows` the workgroup's
// row table in LDS.
//
// Every operand goes to LDS by direct copies (global_load_lds, 16 bytes per lane,
// 1 KB per instruction): per stage the 2*NMT A tile copies (chunk, m tile) dealt
// out over the 8 waves (copy q to wave q % 8; a wave with fewer real copies
// repeats the last one — the same bytes to the same place — so every wave issues
// DPW per stage), and each wave's own 2*WN weight fragments (two chunks per
// tile).  Stage s + R - 1 is issued while stage s is computed; a wave's loads
// complete in issue order, so waiting for stage s (vmcnt <= (R - 2) * copies per
// stage) leaves the younger stages in flight.  Stage s + R - 1 goes into the slot
// of stage s - 1 after the barrier of stage s, when no wave reads that slot any
// more.  Copies past the last stage re-read it (clamped) and rows past mrows
// re-read the last row, which keeps every count exact; the loop drains them at
// its end.
// A wave with no columns of its own (wact false: a column-spread workgroup with
// fewer units than waves) issues only its share of the A copies (and waits for
// its own count of them), reads no fragments and issues no MFMAs (its results are
// dropped), which leaves the copy path, the LDS and the matrix cores of its CU to
// the others.
template <int WN, int NMT, int MB>
SF_DEV void mainloop(const uint16_t* __restrict__ A, int lda, int mrows, const int* rows,
                     const uint16_t* const (&wsrc)[WN], int s0, int s1, const Ring<MB, WN>& rg,
                     sf_f32x4 (&acc)[MB / 16][WN], bool wact = true) {
  using St = Stage<MB, WN>;
  constexpr int R = St::kRing;
  static_assert(R >= 3, "the ring needs three stages");
  constexpr int kMT = MB / 16;
  constexpr int DPW = (2 * NMT + 7) / 8;
  constexpr bool kWR = St::kWReg;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int slast = s1 - 1;
  // this lane's part of each A tile copy: tile row lane/4, stored unit lane%4
  // holding A unit a_copy_unit(lane) of the copy's 32-K chunk
  const uint16_t* asrc[DPW];
  int adst[DPW];   // first word of the copy in a slot
#pragma unroll
  for (int j = 0; j < DPW; ++j) {
    const int q = a_copy(wv, j, NMT);
    const int ch = q / NMT, mt = q - ch * NMT;
    const int r = sf_imin(mt * 16 + (lane >> 2), mrows - 1);
    asrc[j] = A + (size_t)rows[r] * lda + ch * 32 + a_copy_unit(lane) * 8;
    adst[j] = (ch * kMT + mt) * 64;
  }
  const int wdst = St::kA + wv * WN * 128;   // this wave's weights: [tile][chunk][1 KB]
  // kWR: this lane's weight fragments of the stages in flight, [ring slot][tile][chunk]
  sf_u32x4 wreg[kWR ? R : 1][WN][2];
  // stage s into ring slot j (j a constant once the loops below are unrolled)
  auto issue = [&](int s, int j) {
    const int sc = sf_imin(s, slast);
    sf_u32x4* slot = rg.slot[j];
#pragma unroll
    for (int d = 0; d < DPW; ++d) sf_lds_dma16(asrc[d] + sc * kKC, slot + adst[d]);
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if constexpr (kWR)
          wreg[j][t][c] = sf_stream_load16(wsrc[t] + (size_t)weight_chunk(sc, c) * kKsStride);
        else if (wact)   // wave-uniform: a wave with no unit copies no weights
          sf_lds_dma16(wsrc[t] + (size_t)weight_chunk(sc, c) * kKsStride,
                       slot + wdst + (t * 2 + c) * 64);
      }
  };
#pragma unroll
  for (int j = 0; j < R - 1; ++j) issue(s0 + j, j);

  // this lane's A fragment in chunk c of a stage: word a_read_word(lane) of tile
  // (c, mt); its weight fragment: word `lane` of block (tile t, chunk c)
  const sf_lds_off a_byte = (sf_lds_off)a_read_word(lane) * 16;
  const sf_lds_off w_byte = (sf_lds_off)(wdst + lane) * 16;
  // the fragment reads and MFMAs of the stage in ring slot j
  auto compute = [&](int j) {
    const sf_lds_off base = sf_lds_addr(rg.slot[j]);
    if (!kWR && !wact) return;   // wave-uniform: no operand reads or MFMAs for dropped results
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      constexpr int kLW = kWR ? 0 : WN;   // weight fragments read from LDS
      sf_u32x4 f[NMT + kLW];
      lds_fragments<NMT, kLW>(f, base + a_byte + c * kMT * 1024, base + w_byte + c * 1024);
      sf_lds_reads_done(f);
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int t = 0; t < WN; ++t) {
          const sf_u32x4 w = kWR ? wreg[kWR ? j : 0][t][c] : f[kWR ? 0 : NMT + t];
          acc[mt][t] = sf_mfma16x16x32(sf_as_bf16x8(f[mt]), sf_as_bf16x8(w), acc[mt][t]);
        }
    }
  };
  // whole groups of R stages with no branch inside (the compiler's own waits for
  // the weight registers then stay exact across the loop): stage sb + j in slot j
  // -- wait for it, issue stage sb + j + R - 1 into slot j - 1, compute.  The last
  // (s1 - s0) % R < R stages were all issued by then: one wait for every copy,
  // then their fragment reads and MFMAs.
  int sb = s0;
#pragma unroll 1
  for (; sb + R <= s1; sb += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      // a wave with no unit (column-spread plan) issues only its A copies
      if (kWR || wact)
        sf_wait_vm_barrier<(R - 2) * (DPW + 2 * WN)>();
      else
        sf_wait_vm_barrier<(R - 2) * DPW>();
      issue(sb + j + R - 1, (j + R - 1) % R);
      compute(j);
    }
  }
  sf_wait_vm_barrier<0>();
#pragma unroll
  for (int j = 0; j < R - 1; ++j)
    if (sb + j < s1) compute(j);   // wave-uniform
  // every wave is done with the ring before the LDS is reused (the copies past the
  // last stage -- clamped re-reads of it -- were waited for above)
  sf_wait_vm_barrier<0>();
}

// The finished piece goes to LDS as an fp32 tile [MB][TW] (after the main loop's
// drain, in the ring's memory).  Column of (wave w, tile t, lane): 16*(WN*w + t)
// + lane%16; for kSilu (TW = 256) the gate tile at w*16 + lane%16 and the up tile
// at 128 + w*16 + lane%16.
template <int WN, int MB, bool SILU>
struct TileLds {
  static constexpr int kTW = SILU ? 256 : 128 * WN;   // columns of a tile in LDS
  static constexpr int kFloats = MB * kTW;
};
template <int WN, int MB, bool SILU>
SF_DEV void tile_to_lds(float* x, const sf_f32x4 (&acc)[MB / 16][WN], int nmt) {
  constexpr int kMT = MB / 16;
  constexpr int kTW = TileLds<WN, MB, SILU>::kTW;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    if (mt >= nmt) continue;
#pragma unroll
    for (int t = 0; t < WN; ++t) {
      const int c = SILU ? t * 128 + wv * 16 + (lane & 15) : 16 * (WN * wv + t) + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[(mt * 16 + (lane >> 4) * 4 + i) * kTW + c] = acc[mt][t][i];
    }
  }
}

// ---------------------------------------------------------------------------
// Stream-K schedule.  The output columns are cut into T tiles of 64·WN columns
// and K into S stages of 64; the T*S (tile, stage) units are dealt out in
// tile-major order, U consecutive units per workgroup, so every workgroup streams
// the same number of weight bytes whatever T is (a fixed tile-per-workgroup grid
// leaves some CUs with twice the work of others).  A workgroup's range may end
// one tile and start the next.  A tile computed by one workgroup alone gets its
// epilogue straight from registers; the pieces of a tile shared by several
// workgroups go to fp32 partial slots (slot j = g - first(t)) that a fix-up kernel
// sums in slot order after the GEMM — deterministic, and no cross-workgroup
// synchronisation inside the kernel (an agent-scope fence costs a whole-L2
// write-back and invalidate on this multi-XCD part).
// (Plan, make_plan, make_plan_whole, plan_grid, plan_slots, tile_first,
// tile_last, plan_range_end, plan_piece and part_bytes: sf_index.h.)

// sum_{j < n} p[j * stride .. +T] in slot order (deterministic).  The first MAXN
// slots' loads all go out at once (clamped addresses, no branch in between: one
// round of loads for up to MAXN contributors), further ones four at a time.
template <typename T, int MAXN = 8>
SF_DEV T sum_slots(const float* p, size_t stride, int n) {
  T v0[MAXN];
#pragma unroll
  for (int j = 0; j < MAXN; ++j)
    v0[j] = sf_handoff_load(reinterpret_cast<const T*>(p + (size_t)min(j, n - 1) * stride));
  T acc = v0[0];
#pragma unroll
  for (int j = 1; j < MAXN; ++j)
    if (j < n) acc += v0[j];
  for (int s0 = MAXN; s0 < n; s0 += 4) {
    T v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = sf_handoff_load(reinterpret_cast<const T*>(p + (size_t)min(s0 + j, n - 1) * stride));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (s0 + j < n) acc += v[j];
  }
  return acc;
}

// Output modes.
enum Mode {
  kPart = 0,     // every tile piece to its partial slot (QKV: the fix-up adds bias + RoPE)
  kScatter = 1,  // out[rows[m]][c] = bf16(y); shared tiles to partial slots (FFN down)
  kSilu = 2,     // out[m][c] = bf16(bf16(silu(bf16 y_gate)) * bf16 y_up); shared tiles to
                 // partial slots of 2N columns (gate, then up) for the fix-up
  kResid = 3,    // out[m][c] = bf16(res[m][c] + bf16(y)); whole tiles only (o_proj)
  kPlain = 4,    // out[m][c] = bf16(y); whole tiles only (lm_head)
};

struct Epi {
  const int32_t* rows;  // output row of compacted row m (kScatter)
  uint16_t* out;        // bf16 output, row stride ldo
  int ldo;
  const uint16_t* res;  // residual (kResid), row stride ldo
};

// GATED: the A rows are the fold gate's compaction of rec (B1 x N flags), done
// by every workgroup in its prologue (gate_compact) instead of read from a rows
// table; workgroup 0 also writes the compaction's outputs `out` for the kernels
// after this one.
constexpr int kGateMaxRows = 1024;
struct GateIn {
  const int8_t* rec;
  const int32_t* par;
  int B1, N;
  GateOut out;
};

// C = A[rows] . W^T on packed weights, stream-K over (tile, stage) units; WN column
// tiles of 16 per wave (kSilu: WN = 2 = the gate and the up tile of the same 16
// output columns).  All M <= MB rows in one pass over the weights (more rows:
// one pass per MB rows).  Grid: plan_grid workgroups.
// part: fp32 partial slots [slot][mcap][N] ([slot][mcap][2N] for kSilu).
// GATED: rows and the count come from the compaction of gate.rec (mcap = bucket).
template <int WN, int MODE, int MB, bool GATED = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_sk_kernel(const uint16_t* __restrict__ A, const int32_t* __restrict__ a_rows, int lda,
                    const int32_t* __restrict__ count_p, int m_static, int mcap,
                    const uint16_t* __restrict__ W0, const uint16_t* __restrict__ W1, int K, int N,
                    Plan plan, float* __restrict__ part, Epi ep, GateIn gate) {
  constexpr int kMT = MB / 16;    // max m tiles of this kernel
  using St = Stage<MB, WN>;
  constexpr int R = St::kRing;
  // the ring, whose memory then holds each piece's fp32 tile for the epilogue
  constexpr int kTileWords = TileLds<WN, MB, MODE == kSilu>::kFloats / 4;
  constexpr int kRingWords = R * St::kWords > kTileWords ? R * St::kWords : kTileWords;
  __shared__ sf_u32x4 ring[kRingWords];
  __shared__ int rows_s[MB];
  __shared__ int s_grows[GATED ? kGateMaxRows : 1];      // the compacted rows
  __shared__ int s_gtot[GATED ? kGateMaxRows / 64 : 1];
  int M;
  if constexpr (GATED) {
    // the ring's memory is free until the main loop: the compaction's scratch
    static_assert(2 * kGateMaxRows * 4 <= kRingWords * 16, "gate scratch");
    int* s_f = reinterpret_cast<int*>(ring);
    const int total = gate_compact<kThreads, kGateMaxRows / kThreads>(
        gate.rec, gate.par, gate.B1, gate.N, mcap, s_f, s_f + kGateMaxRows, s_gtot, s_grows,
        blockIdx.x == 0, gate.out);
    M = sf_imin(total, mcap);
  } else {
    M = count_p ? sf_imin(*count_p, mcap) : m_static;
  }
  Ring<MB, WN> rg;
#pragma unroll
  for (int j = 0; j < 8; ++j) rg.slot[j] = ring + (j < R ? j : 0) * St::kWords;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const size_t stride = (size_t)mcap * N;
  const int g = blockIdx.x;
  const int u_end = plan_range_end(g, plan);
  // rows beyond MB (a launch whose mcap exceeds 256) take further passes
  for (int m0 = 0; m0 < M; m0 += MB) {
  const int mrows = sf_imin(MB, M - m0);
  const int nmt = (mrows + 15) >> 4;
  __syncthreads();  // the previous pass's last readers of the row table are done
  if (tid < MB) {
    const int r = m0 + sf_imin(tid, mrows - 1);
    rows_s[tid] = GATED ? s_grows[r] : (a_rows ? a_rows[r] : r);
  }
  __syncthreads();
  for (int u = plan_range_begin(g, plan); u < u_end;) {
    const Piece pc = plan_piece(u, u_end, plan);
    const int t = pc.t;
    const int sa = pc.sa;
    const int sb = pc.sb;
    const int cg = wv;  // column group
    int col[WN];
    const uint16_t* wrow[WN];  // this lane's weight stream of each column tile
    // column-spread plan: this workgroup's units [ub, ue); a wave past them keeps the
    // last one's column (in range) but streams no weights (mainloop's wact) and its
    // results are not written: only ue - ub column groups are
    const int ub = plan.NU ? spread_begin(t, plan) : 0;
    const int ue = plan.NU ? spread_begin(t + 1, plan) : 0;
    if (MODE == kSilu) {
      const int c = plan.NU ? 16 * sf_imin(ub + cg, ue - 1) + (lane & 15)
                            : gemm_col<WN, true>(t, cg, 0, lane);
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) col[tt] = c;
      wrow[0] = weight_lane_ptr(W0, c >> 4, K, lane);
      wrow[WN - 1] = weight_lane_ptr(W1, c >> 4, K, lane);
    } else {
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) {
        col[tt] = gemm_col<WN, false>(t, cg, tt, lane);
        wrow[tt] = weight_lane_ptr(W0, col[tt] >> 4, K, lane);
      }
    }
    sf_f32x4 acc[kMT][WN];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) acc[mt][tt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    // m tiles rounded up to 2, 3, 4 or 8 (fewer instantiations; the extra tiles
    // re-read the last row and their results are dropped)
    const bool wact = !plan.NU || cg < ue - ub;
    if (nmt <= 2)
      mainloop<WN, 2, MB>(A, lda, mrows, rows_s, wrow, sa, sb, rg, acc, wact);
    else if (nmt == 3)
      mainloop<WN, 3, MB>(A, lda, mrows, rows_s, wrow, sa, sb, rg, acc, wact);
    else if (nmt <= 4 || kMT < 8)
      mainloop<WN, (kMT < 4 ? kMT : 4), MB>(A, lda, mrows, rows_s, wrow, sa, sb, rg, acc, wact);
    else
      mainloop<WN, (kMT < 8 ? kMT : 8), MB>(A, lda, mrows, rows_s, wrow, sa, sb, rg, acc, wact);
    // the tile to LDS (the ring's memory), then every thread takes 4 consecutive
    // columns of a row: epilogue, vector stores
    constexpr bool kS = MODE == kSilu;
    float* tl = reinterpret_cast<float*>(ring);
    static_assert(TileLds<WN, MB, kS>::kFloats * 4 <= kRingWords * 16, "tile LDS");
    tile_to_lds<WN, MB, kS>(tl, acc, nmt);
    __syncthreads();
    u += sb - sa;
    const int first = tile_first(t, plan);
    const bool whole = MODE != kPart && tile_last(t, plan) == first;
    constexpr int kTW = TileLds<WN, MB, kS>::kTW;
    // partial slot rows: N columns (kSilu: 2N, the gate sums then the up sums)
    constexpr int kPW = kS ? 2 : 1;
    float* pw = part + ((size_t)(g - first) * stride + (size_t)m0 * N) * kPW;
    const int c0 = kS ? (plan.NU ? 16 * ub : t * 128) : t * kTW;   // first output column
    const int cw = kS && plan.NU ? 16 * (ue - ub) : 128;   // kSilu: columns of the tile
    for (int e = tid; e < mrows * (kTW / 4); e += kThreads) {
      const int m = e / (kTW / 4);
      const int c = (e - m * (kTW / 4)) * 4;          // column in the LDS tile
      const sf_f32x4 y = *reinterpret_cast<const sf_f32x4*>(tl + m * kTW + c);
      if (!whole) {
        // kSilu: LDS columns [0, 128) are gate sums -> pw[.. + c0 + c], [128, 256)
        // up sums -> pw[.. + N + c0 + c - 128]
        const size_t pc = kS ? (c < 128 ? (size_t)c0 + c : (size_t)N + c0 + c - 128)
                             : (size_t)c0 + c;
        sf_handoff_store(reinterpret_cast<sf_f32x4*>(pw + (size_t)m * N * kPW + pc), y);
      } else if (kS) {
        if (c < cw) {
          const sf_f32x4 up = *reinterpret_cast<const sf_f32x4*>(tl + m * kTW + 128 + c);
          float r[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gt = sf_rbf(y[i]);
            r[i] = sf_rbf(gt / (1.0f + expf(-gt))) * sf_rbf(up[i]);
          }
          sf_u32x2 o;
          o[0] = sf_pack2(r[0], r[1]);
          o[1] = sf_pack2(r[2], r[3]);
          sf_handoff_store(reinterpret_cast<sf_u32x2*>(ep.out + (size_t)(m0 + m) * ep.ldo + c0 + c), o);
        }
      } else {
        float r[4];
        const size_t orow = MODE == kScatter ? (size_t)ep.rows[m0 + m] : (size_t)(m0 + m);
        const size_t o = orow * ep.ldo + c0 + c;
        if (MODE == kResid) {
          float x[4];
          const sf_u32x2 rv = *reinterpret_cast<const sf_u32x2*>(ep.res + o);
          x[0] = __uint_as_float(rv[0] << 16);
          x[1] = __uint_as_float(rv[0] & 0xffff0000u);
          x[2] = __uint_as_float(rv[1] << 16);
          x[3] = __uint_as_float(rv[1] & 0xffff0000u);
#pragma unroll
          for (int i = 0; i < 4; ++i) r[i] = x[i] + sf_rbf(y[i]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) r[i] = y[i];
        }
        sf_u32x2 ov;
        ov[0] = sf_pack2(r[0], r[1]);
        ov[1] = sf_pack2(r[2], r[3]);
        sf_handoff_store(reinterpret_cast<sf_u32x2*>(ep.out + o), ov);
      }
    }
    __syncthreads();  // the tile LDS is the next piece's ring
  }
  }  // row passes
}

// One pass over the weights for every row: the row block MB is the smallest of
// 64 / 128 / 256 that holds mcap rows (A ring 8 / 8 / 4 stages, 64 / 128 / 128 KB).
template <int WN, int MODE, bool GATED = false>
inline void launch_sk(const Plan& p, const uint16_t* A, const int32_t* a_rows, int lda,
                      const int32_t* count_p, int m_static, int mcap, const uint16_t* W0,
                      const uint16_t* W1, int K, int N, float* part, const Epi& ep,
                      hipStream_t st, const GateIn& gate = GateIn{}) {
  const dim3 grid(plan_grid(p));
  if (row_block(mcap) == 64)
    hipLaunchKernelGGL((gemm_sk_kernel<WN, MODE, 64, GATED>), grid, dim3(kThreads), 0, st, A,
                       a_rows, lda, count_p, m_static, mcap, W0, W1, K, N, p, part, ep, gate);
  else
    hipLaunchKernelGGL((gemm_sk_kernel<WN, MODE, 128, GATED>), grid, dim3(kThreads), 0, st, A,
                       a_rows, lda, count_p, m_static, mcap, W0, W1, K, N, p, part, ep, gate);
}

}  // namespace sfg
