// Weight-streaming GEMM core for skinny row blocks:  C[m, n] = sum_k A[arow(m), k] * W[n, k]
//
// Shapes on this path: M = recomputed rows (<= 256, often 30-120) or all BN rows,
// N and K = 1.5k-38k; W (bf16, [N, K], packed fragment-major) is the big operand
// and is read once from HBM.  A workgroup is 4 waves; wave w owns WN column tiles
// of 16; a block of up to 64 rows of A is staged through LDS in 128-wide K stages
// (double buffered) and shared by the 4 waves; every wave streams its own weight
// tiles straight into VGPRs.  Work is split stream-K: a fixed grid of workgroups
// per m block, each taking an equal share of the (tile, K stage) units; tiles
// shared by several workgroups are summed by a fix-up kernel.
// MFMA: v_mfma_f32_16x16x32_bf16, fp32 accumulation.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (64 lanes): A 16x32 — lane l holds
// A[l%16][8*(l/16) .. +8]; B 32x16 — lane l holds B[8*(l/16) .. +8][l%16];
// D 16x16 — lane l holds D[4*(l/16) + i][l%16], i = 0..3.
#pragma once

#include "sf_common.h"
#include "sf_index.h"

namespace sfg {

#ifndef SFG_MB
#define SFG_MB 64
#endif
constexpr int kMB = SFG_MB;       // rows of A per workgroup (default of every kernel)
constexpr int kKC = 128;          // K per LDS stage
constexpr int kLdsStride = 136;   // bf16 per LDS row (128 + 8 pad: 272 B, spreads banks)
constexpr int kMT = kMB / 16;     // max m tiles per workgroup

// Shared memory of one workgroup of MB rows: two A stages + the row index table.
template <int MB>
struct SmemT {
  uint16_t a[2][MB * kLdsStride];
  int rows[MB];
};
using Smem = SmemT<kMB>;

// Prefetch depth: a ring of SFG_RING register slots per wave (A rows and weights
// of one K stage each), so every wave keeps SFG_RING-1 stages of loads
// (WN x 4 KB of weights each) outstanding.
#ifndef SFG_RING
#define SFG_RING 2
#endif
#ifndef SFG_WAVES
#define SFG_WAVES 2   // waves per SIMD the register allocation targets
#endif

// Weight layout (fragment-major, "packed"; weight_lane_ptr, kKsStride and
// kStageElems in sf_index.h): every wave's weight stream is a sequential read.
// sf_pack_weight produces it from row-major W.

// Main loop over stages [s0, s1) of K for NMT m tiles of 16 rows (NMT is a
// template parameter so the MFMA loop is straight-line).  `wrow[t]` is this
// lane's weight stream for column tile t; `acc[mt][t]` accumulates rows mt*16..,
// column tile t.
//
// Stage s's A rows and weights are issued together, SFG_RING-1 stages ahead, into
// a register ring of SFG_RING slots (A too, not only W).  A wave's vector-memory
// loads complete in issue order, so waiting for stage s then waits for nothing
// younger: the SFG_RING-1 later stages stay in flight.  A(s) goes to LDS (double
// buffered) only at the start of iteration s, followed by the one barrier of the
// stage.  Loads past the last stage re-read it and rows past mrows re-read the
// last row (clamped, no branches), which keeps the wait counts exact.
template <int WN, int NMT, int MB = kMB>
SF_DEV void mainloop(const uint16_t* __restrict__ A, int lda, int mrows,
                     const uint16_t* const (&wrow)[WN], int s0, int s1, SmemT<MB>& sm,
                     sf_f32x4 (&acc)[MB / 16][WN]) {
  constexpr int R = SFG_RING;
  static_assert(R % 2 == 0, "ring depth must be even (LDS double buffer parity)");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int kq = (lane >> 4) * 8;
  const int a_seg = tid & 15;      // 16 x 16 B per 128-wide row stage
  const int a_row0 = tid >> 4;     // 16 rows per pass, NMT passes
  const int slast = s1 - 1;
  const uint16_t* arow[NMT];
#pragma unroll
  for (int p = 0; p < NMT; ++p)
    arow[p] = A + (size_t)sm.rows[min(a_row0 + p * 16, mrows - 1)] * lda + a_seg * 8;
  sf_u32x4 areg[R][NMT];
  sf_u32x4 w[R][WN][4];

  auto issue = [&](int s, int slot) {
    const int sc = min(s, slast);
#pragma unroll
    for (int p = 0; p < NMT; ++p)
      areg[slot][p] = *reinterpret_cast<const sf_u32x4*>(arow[p] + sc * kKC);
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        w[slot][t][ks] =
            *reinterpret_cast<const sf_u32x4*>(wrow[t] + (size_t)sc * kStageElems + ks * kKsStride);
  };

#pragma unroll
  for (int j = 0; j < R - 1; ++j) issue(s0 + j, j);

#pragma unroll 1
  for (int sb = s0; sb < s1; sb += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int s = sb + j;
      if (s >= s1) break;
      issue(s + R - 1, (j + R - 1) % R);
#pragma unroll
      for (int p = 0; p < NMT; ++p)
        *reinterpret_cast<sf_u32x4*>(&sm.a[j & 1][(a_row0 + p * 16) * kLdsStride + a_seg * 8]) =
            areg[j][p];
      __syncthreads();
      const uint16_t* abase = &sm.a[j & 1][(lane & 15) * kLdsStride + kq];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) {
          const sf_bf16x8 af = sf_as_bf16x8(
              *reinterpret_cast<const sf_u32x4*>(abase + mt * 16 * kLdsStride + ks * 32));
#pragma unroll
          for (int t = 0; t < WN; ++t)
            acc[mt][t] = sf_mfma16x16x32(af, sf_as_bf16x8(w[j][t][ks]), acc[mt][t]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Stream-K schedule.  The output columns are cut into T tiles of TW columns and K
// into S stages of 128; the T*S (tile, stage) units are dealt out in tile-major
// order, U consecutive units per workgroup, so every workgroup streams the same
// number of weight bytes whatever T is (a fixed tile-per-workgroup grid leaves
// some CUs with twice the work of others).  A workgroup's range may end one tile
// and start the next.  A tile computed by one workgroup alone gets its epilogue
// straight from registers; the pieces of a tile shared by several workgroups go
// to fp32 partial slots (slot j = g - first(t)) that a fix-up kernel sums in slot
// order after the GEMM — deterministic, and no cross-workgroup synchronisation
// inside the kernel (an agent-scope fence costs a whole-L2 write-back and
// invalidate on this multi-XCD part).
// (Plan, make_plan, make_plan_whole, plan_grid, plan_slots, tile_first,
// tile_last, plan_range_end, plan_piece and part_bytes: sf_index.h.)

// sum_{j < n} p[j * stride .. +T] in slot order (deterministic).  Loads go out four
// at a time from clamped addresses with no branch in between.
template <typename T>
SF_DEV T sum_slots(const float* p, size_t stride, int n) {
  T acc = *reinterpret_cast<const T*>(p);
  for (int s0 = 1; s0 < n; s0 += 4) {
    T v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = *reinterpret_cast<const T*>(p + (size_t)min(s0 + j, n - 1) * stride);
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
  kSilu = 2,     // out[m][c] = bf16(bf16(silu(bf16 y_gate)) * bf16 y_up); whole tiles only
  kResid = 3,    // out[m][c] = bf16(res[m][c] + bf16(y)); whole tiles only (o_proj)
  kPlain = 4,    // out[m][c] = bf16(y); whole tiles only (lm_head)
};

struct Epi {
  const int32_t* rows;  // output row of compacted row m (kScatter)
  uint16_t* out;        // bf16 output, row stride ldo
  int ldo;
  const uint16_t* res;  // residual (kResid), row stride ldo
};

// C = A[rows] . W^T on packed weights, stream-K over (tile, stage) units; WN column
// tiles of 16 per wave (kSilu: WN = 2 = the gate and the up tile of the same 16
// output columns).  Grid: (plan_grid, 1, m blocks).  part: fp32 partial slots
// [slot][mcap][N].
template <int WN, int MODE, int MB = kMB, int WAVES = SFG_WAVES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES)))
void gemm_sk_kernel(const uint16_t* __restrict__ A, const int32_t* __restrict__ a_rows, int lda,
                    const int32_t* __restrict__ count_p, int m_static, int mcap,
                    const uint16_t* __restrict__ W0, const uint16_t* __restrict__ W1, int K, int N,
                    Plan plan, float* __restrict__ part, Epi ep) {
  constexpr int kMT = MB / 16;    // max m tiles of this kernel's row block
  __shared__ SmemT<MB> sm;
  const int M = count_p ? min(*count_p, mcap) : m_static;
  const int m0 = blockIdx.z * MB;
  if (m0 >= M) return;
  const int mrows = min(MB, M - m0);
  const int nmt = (mrows + 15) >> 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  if (tid < MB) {
    const int r = m0 + min(tid, mrows - 1);
    sm.rows[tid] = a_rows ? a_rows[r] : r;
  }
  __syncthreads();
  const size_t stride = (size_t)mcap * N;
  const int g = blockIdx.x;
  const int u_end = plan_range_end(g, plan);
  for (int u = g * plan.U; u < u_end;) {
    const Piece pc = plan_piece(u, u_end, plan);
    const int t = pc.t;
    const int sa = pc.sa;
    const int sb = pc.sb;
    int col[WN];
    const uint16_t* wrow[WN];
    if (MODE == kSilu) {
      const int c = gemm_col<WN, true>(t, wv, 0, lane);
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) col[tt] = c;
      wrow[0] = weight_lane_ptr(W0, c >> 4, K, lane);
      wrow[WN - 1] = weight_lane_ptr(W1, c >> 4, K, lane);
    } else {
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) {
        col[tt] = gemm_col<WN, false>(t, wv, tt, lane);
        wrow[tt] = weight_lane_ptr(W0, col[tt] >> 4, K, lane);
      }
    }
    sf_f32x4 acc[kMT][WN];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) acc[mt][tt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    switch (nmt) {
      case 1: mainloop<WN, 1, MB>(A, lda, mrows, wrow, sa, sb, sm, acc); break;
      case 2: mainloop<WN, 2, MB>(A, lda, mrows, wrow, sa, sb, sm, acc); break;
      case 3: mainloop<WN, 3, MB>(A, lda, mrows, wrow, sa, sb, sm, acc); break;
      default: mainloop<WN, kMT, MB>(A, lda, mrows, wrow, sa, sb, sm, acc); break;
    }
    const int first = tile_first(t, plan);
    const bool whole = MODE != kPart && tile_last(t, plan) == first;
    float* pw = part + (size_t)(g - first) * stride + (size_t)m0 * N;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
      if (mt >= nmt) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mt * 16 + (lane >> 4) * 4 + i;
        if (m >= mrows) continue;
        if (!whole) {
#pragma unroll
          for (int tt = 0; tt < WN; ++tt) pw[(size_t)m * N + col[tt]] = acc[mt][tt][i];
        } else if (MODE == kSilu) {
          const float gt = sf_rbf(acc[mt][0][i]);
          const float r = sf_rbf(gt / (1.0f + expf(-gt))) * sf_rbf(acc[mt][WN - 1][i]);
          ep.out[(size_t)(m0 + m) * ep.ldo + col[0]] = sf_f2bf(r);
        } else {
#pragma unroll
          for (int tt = 0; tt < WN; ++tt) {
            const float y = acc[mt][tt][i];
            if (MODE == kResid) {
              const size_t o = (size_t)(m0 + m) * ep.ldo + col[tt];
              ep.out[o] = sf_f2bf(sf_bf2f(ep.res[o]) + sf_rbf(y));
            } else {
              const size_t orow = MODE == kScatter ? (size_t)ep.rows[m0 + m] : (size_t)(m0 + m);
              ep.out[orow * ep.ldo + col[tt]] = sf_f2bf(y);
            }
          }
        }
      }
    }
    __syncthreads();  // the next piece's first A stage reuses LDS buffer 0
    u += sb - sa;
  }
}

// MB rows per workgroup (grid z = row blocks), register allocation for WAVES
// waves per SIMD; every launch here uses the defaults.
template <int WN, int MODE, int MB = kMB, int WAVES = SFG_WAVES>
inline void launch_sk(const Plan& p, const uint16_t* A, const int32_t* a_rows, int lda,
                      const int32_t* count_p, int m_static, int mcap, const uint16_t* W0,
                      const uint16_t* W1, int K, int N, float* part, const Epi& ep,
                      hipStream_t st) {
  static_assert(MB % 16 == 0 && MB >= 16 && MB <= 256, "row block: 16..256 rows, whole m tiles");
  dim3 grid(plan_grid(p), 1, (mcap + MB - 1) / MB);
  hipLaunchKernelGGL((gemm_sk_kernel<WN, MODE, MB, WAVES>), grid, dim3(256), 0, st, A, a_rows,
                     lda, count_p, m_static, mcap, W0, W1, K, N, p, part, ep);
}

}  // namespace sfg
