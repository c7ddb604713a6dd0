// Weight-streaming GEMM core for skinny row blocks:  C[m, n] = sum_k A[arow(m), k] * W[n, k]
//
// Shapes on this path: M = recomputed rows (<= 256, often 30-120) or all BN rows,
// N and K = 1.5k-38k; W (bf16, [N, K], K contiguous) is the big operand and is read
// once from HBM.  A workgroup is 4 waves; wave w owns WN column tiles of 16; a block
// of up to 128 rows of A is staged through LDS in 128-wide K stages (double
// buffered) and shared by the 4 waves; every wave streams its own weight rows
// straight into VGPRs one stage ahead (WN x 4 x 16 B per lane), so a workgroup keeps
// 16-32 KB of weight loads in flight.  MFMA: v_mfma_f32_16x16x32_bf16, fp32 acc.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (64 lanes): A 16x32 — lane l holds
// A[l%16][8*(l/16) .. +8]; B 32x16 — lane l holds B[8*(l/16) .. +8][l%16];
// D 16x16 — lane l holds D[4*(l/16) + i][l%16], i = 0..3.
#pragma once

#include "sf_common.h"

namespace sfg {

#ifndef SFG_MB
#define SFG_MB 64
#endif
constexpr int kMB = SFG_MB;       // rows of A per workgroup
constexpr int kKC = 128;          // K per LDS stage
constexpr int kLdsStride = 136;   // bf16 per LDS row (128 + 8 pad: 272 B, spreads banks)
constexpr int kMT = kMB / 16;     // max m tiles per workgroup

// Shared memory of one workgroup: two A stages + the row index table.
struct Smem {
  uint16_t a[2][kMB * kLdsStride];
  int rows[kMB];
};

// Weight prefetch depth: a ring of SFG_PF register slots per wave, so every wave
// keeps (SFG_PF-1) stages of weight loads (WN x 4 KB each) outstanding.
#ifndef SFG_PF
#define SFG_PF 2
#endif
#ifndef SFG_WAVES
#define SFG_WAVES 2   // waves per SIMD the register allocation targets
#endif

// Main loop over stages [s0, s1) of K for NMT m tiles of 16 rows (NMT is a
// template parameter so the MFMA loop is straight-line).  `wrow[t]` points at
// W[col_t][kq] for this lane (kq = 8*(lane/16)); `acc[mt][t]` accumulates rows
// mt*16.., column tile t.
//
// Load order matters: a wave's vector-memory loads complete in issue order, so
// waiting for one waits for every older one.  Each iteration therefore issues
// the A stage two ahead (s+2) BEFORE the weight stage PF-1 ahead; writing A(s+1)
// into LDS at the end of iteration s then waits only for loads issued before
// A(s+1), never for the weights still in flight.  The loop is unrolled by PF
// (a multiple of 2) so ring slots and LDS buffers are compile-time indices.
template <int WN, int NMT>
SF_DEV void mainloop(const uint16_t* __restrict__ A, int lda, int mrows,
                     const uint16_t* const (&wrow)[WN], int s0, int s1, Smem& sm,
                     sf_f32x4 (&acc)[kMT][WN]) {
  constexpr int PF = SFG_PF;
  static_assert(PF % 2 == 0, "ring depth must be even (LDS double buffer parity)");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int kq = (lane >> 4) * 8;
  const int a_seg = tid & 15;      // 16 x 16 B per 128-wide row stage
  const int a_row0 = tid >> 4;     // 16 rows per pass, NMT passes
  sf_u32x4 areg[2][NMT];
  sf_u32x4 w[PF][WN][4];

  auto load_a = [&](int s, sf_u32x4 (&ar)[NMT]) {
#pragma unroll
    for (int p = 0; p < NMT; ++p) {
      const int r = a_row0 + p * 16;
      if (r < mrows)
        ar[p] = *reinterpret_cast<const sf_u32x4*>(A + (size_t)sm.rows[r] * lda + s * kKC +
                                                   a_seg * 8);
    }
  };
  auto store_a = [&](int buf, const sf_u32x4 (&ar)[NMT]) {
#pragma unroll
    for (int p = 0; p < NMT; ++p) {
      const int r = a_row0 + p * 16;
      if (r < mrows)
        *reinterpret_cast<sf_u32x4*>(&sm.a[buf][r * kLdsStride + a_seg * 8]) = ar[p];
    }
  };
  auto load_w = [&](int s, sf_u32x4 (&ws)[WN][4]) {
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        ws[t][ks] = *reinterpret_cast<const sf_u32x4*>(wrow[t] + s * kKC + ks * 32);
  };

  // prologue: A(s0), A(s0+1) first, then weight stages s0 .. s0+PF-2
  load_a(s0, areg[0]);
  if (s0 + 1 < s1) load_a(s0 + 1, areg[1]);
#pragma unroll
  for (int j = 0; j < PF - 1; ++j)
    if (s0 + j < s1) load_w(s0 + j, w[j]);
  store_a(0, areg[0]);
  __syncthreads();

#pragma unroll 1
  for (int sb = s0; sb < s1; sb += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int s = sb + j;
      if (s < s1) {
        // slot parity: stage s's A is in LDS buffer j&1 and A(s+1) in areg[(j+1)&1]
        if (s + 2 < s1) load_a(s + 2, areg[j & 1]);
        if (s + PF - 1 < s1) load_w(s + PF - 1, w[(j + PF - 1) % PF]);
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
        if (s + 1 < s1) store_a((j + 1) & 1, areg[(j + 1) & 1]);
        __syncthreads();
      }
    }
  }
}

// Number of K splits so that (column tiles x splits) covers the 256 CUs with one
// active M block (the common case: the row count is known only on the device).
inline int pick_nsplit(int tiles, int K, int /*mblocks*/ = 1) {
  const int nst = K / kKC;
  int s = (256 + tiles - 1) / tiles;
  if (s < 1) s = 1;
  if (s > nst) s = nst;
  return s;
}

// Epilogue modes of gemm_rows_kernel.
enum Mode { kPartial = 0, kSiluMul = 1, kBf16 = 2 };

template <int WN, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(SFG_WAVES, SFG_WAVES)))
void gemm_rows_kernel(
    const uint16_t* __restrict__ A, const int32_t* __restrict__ a_rows, int lda,
    const int32_t* __restrict__ count_p, int m_static, int mcap, const uint16_t* __restrict__ W0,
    const uint16_t* __restrict__ W1, int K, int N, int nsplit, float* __restrict__ part,
    uint16_t* __restrict__ out, int ldo) {
  __shared__ Smem sm;
  const int M = count_p ? min(*count_p, mcap) : m_static;
  const int m0 = blockIdx.z * kMB;
  if (m0 >= M) return;
  const int mrows = min(kMB, M - m0);
  const int nmt = (mrows + 15) >> 4;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < mrows; i += 256) sm.rows[i] = a_rows ? a_rows[m0 + i] : m0 + i;
  __syncthreads();
  const int nst = K / kKC;
  const int s0 = blockIdx.y * nst / nsplit;
  const int s1 = (blockIdx.y + 1) * nst / nsplit;
  const int kq = (lane >> 4) * 8;
  int col[WN];
  const uint16_t* wrow[WN];
  if (MODE == kSiluMul) {
    // tile 0 = gate rows, tile 1 = up rows, same 16 output columns
    const int c = blockIdx.x * 64 + wv * 16 + (lane & 15);
#pragma unroll
    for (int t = 0; t < WN; ++t) col[t] = c;
    wrow[0] = W0 + (size_t)c * K + kq;
    wrow[WN - 1] = W1 + (size_t)c * K + kq;
  } else {
#pragma unroll
    for (int t = 0; t < WN; ++t) {
      col[t] = blockIdx.x * 64 * WN + wv * 16 * WN + t * 16 + (lane & 15);
      wrow[t] = W0 + (size_t)col[t] * K + kq;
    }
  }
  sf_f32x4 acc[kMT][WN];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int t = 0; t < WN; ++t) acc[mt][t] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  switch (nmt) {
    case 1: mainloop<WN, 1>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    case 2: mainloop<WN, 2>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    case 3: mainloop<WN, 3>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
#if SFG_MB > 64
    case 4: mainloop<WN, 4>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    case 5: mainloop<WN, 5>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    case 6: mainloop<WN, 6>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    case 7: mainloop<WN, 7>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
    default: mainloop<WN, kMT>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
#else
    default: mainloop<WN, kMT>(A, lda, mrows, wrow, s0, s1, sm, acc); break;
#endif
  }

#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    if (mt >= nmt) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = mt * 16 + (lane >> 4) * 4 + i;
      if (m >= mrows) continue;
      if (MODE == kPartial) {
        float* p = part + ((size_t)blockIdx.y * mcap + m0 + m) * N;
#pragma unroll
        for (int t = 0; t < WN; ++t) p[col[t]] = acc[mt][t][i];
      } else if (MODE == kBf16) {
#pragma unroll
        for (int t = 0; t < WN; ++t) out[(size_t)(m0 + m) * ldo + col[t]] = sf_f2bf(acc[mt][t][i]);
      } else {
        const float g = sf_rbf(acc[mt][0][i]);
        const float u = sf_rbf(acc[mt][WN - 1][i]);
        const float s = sf_rbf(g / (1.0f + expf(-g)));
        out[(size_t)(m0 + m) * ldo + col[0]] = sf_f2bf(s * u);
      }
    }
  }
}

template <int WN, int MODE>
inline void launch_gemm(const uint16_t* A, const int32_t* a_rows, int lda,
                        const int32_t* count_p, int m_static, int mcap, const uint16_t* W0,
                        const uint16_t* W1, int K, int N, int nsplit, float* part, uint16_t* out,
                        int ldo, hipStream_t st) {
  const int span = MODE == kSiluMul ? 64 : 64 * WN;
  dim3 grid(N / span, nsplit, (mcap + kMB - 1) / kMB);
  hipLaunchKernelGGL((gemm_rows_kernel<WN, MODE>), grid, dim3(256), 0, st, A, a_rows, lda,
                     count_p, m_static, mcap, W0, W1, K, N, nsplit, part, out, ldo);
}

}  // namespace sfg
