// All-rows GEMM:  C[m, n] = sum_k A[m, k] * W[n, k]  for every row m < M <= 256
//
// For the projections applied to every row of the verify block (o_proj, lm_head:
// M = B1·N = 256 at 7B), where the weights are read once for all rows.  The 8
// waves of a workgroup are RG row groups of 128 rows x CG = 8 / RG column groups
// of WN 16-column tiles; both operands go to LDS by direct copies (A: the
// workgroup's K range of every row, read from L2 by each tile's workgroups; W:
// each column tile's fragments once, shared by the row groups).  K is cut into KS
// ranges so that T·KS workgroups fill the machine (o_proj at 7B: 56 tiles of 64
// columns x 4 ranges); a range's fp32 sums go to partial slots [KS][M][N] that the
// consumer adds in range order (deterministic).  With KS = 1 the result is
// rounded to bf16 and stored directly.
//
// The MFMA takes the weight fragment as its first operand (v_mfma_f32_16x16x32_bf16
// computes C^T for the tile), so lane l ends with row l%16 of its m tile and the 4
// consecutive columns 4(l/16) .. +4 of its n tile: one 16-byte fp32 or 8-byte
// bf16 store per lane and tile.
// (RowsPlan, RowsStage, make_rows_plan, rows_item, rows_split_begin, rows_splits
// and the copy maps: sf_index.h.)
#pragma once

#include "sf_gemm_core.h"

namespace sfg {

enum RowsMode {
  kRowsPart = 0,  // fp32 sums of the workgroup's K range to part[s][m][n]
  kRowsBf16 = 1,  // out[m][n] = bf16(sum) (KS = 1)
};

// Grid: rows_grid(plan) workgroups of kThreads.  A: M rows of K (row stride K);
// W packed (sf_pack_weight); part: slot s at part + s * part_stride, row m at
// + m * N; out: row stride N.
template <int RG, int WN, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_rows_kernel(const uint16_t* __restrict__ A, int M, const uint16_t* __restrict__ W,
                      int K, int N, RowsPlan plan, float* __restrict__ part, size_t part_stride,
                      uint16_t* __restrict__ out) {
  using St = RowsStage<RG, WN>;
  constexpr int R = St::kRing;
  static_assert(R >= 3, "the ring needs three stages");
  constexpr int kMT = St::kMT;
  __shared__ sf_u32x4 ring[R * St::kWords];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int q = rows_item(blockIdx.x, rows_grid(plan));
  const int s = q / plan.T;
  const int t = q - s * plan.T;
  const int s0 = rows_split_begin(s, plan);
  const int s1 = rows_split_begin(s + 1, plan);
  const int slast = s1 - 1;
  const int rgrp = wv / St::kCG;
  const int cgrp = wv - rgrp * St::kCG;

  // this wave's copies: lane L of an A copy brings row L/4 of its m tile (rows
  // past M re-read row M - 1), A unit a_copy_unit(L) of the chunk; lane L of a
  // weight copy brings lane L's fragment of its (tile, chunk) block
  constexpr int CPS = St::kCPS;
  const uint16_t* asrc[St::kDA];
  int adst[St::kDA];
#pragma unroll
  for (int j = 0; j < St::kDA; ++j) {
    const int cq = rows_a_copy(wv + 8 * j, St::kNA);
    const int ch = rows_a_chunk(cq, kMT), mt = rows_a_mtile(cq, kMT);
    const int r = sf_imin(mt * 16 + (lane >> 2), M - 1);
    asrc[j] = A + (size_t)r * K + ch * 32 + a_copy_unit(lane) * 8;
    adst[j] = (ch * kMT + mt) * 64;
  }
  const uint16_t* wsrc[St::kDW];
  int wdst[St::kDW];
#pragma unroll
  for (int j = 0; j < St::kDW; ++j) {
    const int cq = rows_w_copy(wv + 8 * j, St::kNW);
    const int tw = rows_w_tile(cq, CPS), c = rows_w_chunk(cq, CPS);
    wsrc[j] = weight_lane_ptr(W, t * St::kTW + tw, K, lane) + (size_t)c * kKsStride;
    wdst[j] = St::kA + (tw * CPS + c) * 64;
  }
  auto slot = [&](int j) { return ring + j * St::kWords; };
  auto issue = [&](int sg, sf_u32x4* sl) {
    const int sc = sf_imin(sg, slast);
#pragma unroll
    for (int j = 0; j < St::kDA; ++j) sf_lds_dma16(asrc[j] + sc * St::kKS, sl + adst[j]);
#pragma unroll
    for (int j = 0; j < St::kDW; ++j)
      sf_lds_dma16(wsrc[j] + (size_t)sc * CPS * kKsStride, sl + wdst[j]);
  };
#pragma unroll
  for (int j = 0; j < R - 1; ++j) issue(s0 + j, slot(j));

  sf_f32x4 acc[8][WN];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int tt = 0; tt < WN; ++tt) acc[i][tt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  // this lane's A fragment of m tile rgrp*8 + i in chunk c: word a_read_word(lane)
  // of A tile (c, mt); its weight fragment of tile cgrp*WN + tt: word `lane` of
  // block (tile, c)
  const sf_lds_off a_byte = (sf_lds_off)(rgrp * 8 * 64 + a_read_word(lane)) * 16;
  const sf_lds_off w_byte = (sf_lds_off)(St::kA + cgrp * WN * CPS * 64 + lane) * 16;
#pragma unroll 1
  for (int sb = s0; sb < s1; sb += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (sb + j < s1) {  // wave-uniform; no break, so the ring indices stay static
        sf_wait_vm_barrier<(R - 2) * (St::kDA + St::kDW)>();
        issue(sb + j + R - 1, slot((j + R - 1) % R));
        const sf_lds_off base = sf_lds_addr(slot(j));
#pragma unroll
        for (int c = 0; c < CPS; ++c) {
          sf_u32x4 f[8 + WN];
          lds_fragments<8, WN, CPS>(f, base + a_byte + c * kMT * 1024, base + w_byte + c * 1024);
          sf_lds_reads_done(f);
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int tt = 0; tt < WN; ++tt)
              acc[i][tt] = sf_mfma16x16x32(sf_as_bf16x8(f[8 + tt]), sf_as_bf16x8(f[i]), acc[i][tt]);
        }
      }
    }
  }
  // drain the clamped re-issues past the last stage before the workgroup exits
  sf_wait_vm_barrier<0>();

  // lane: row rgrp*128 + 16 i + lane%16, columns col0 + 16 tt + 4 (lane/16) .. +4
  const int col0 = (t * St::kTW + cgrp * WN) * 16 + (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = rgrp * 128 + i * 16 + (lane & 15);
    if (row < M) {
#pragma unroll
      for (int tt = 0; tt < WN; ++tt) {
        const size_t o = (size_t)row * N + col0 + tt * 16;
        if (MODE == kRowsPart) {
          sf_handoff_store(reinterpret_cast<sf_f32x4*>(part + (size_t)s * part_stride + o),
                           acc[i][tt]);
        } else {
          sf_u32x2 v;
          v[0] = sf_pack2(acc[i][tt][0], acc[i][tt][1]);
          v[1] = sf_pack2(acc[i][tt][2], acc[i][tt][3]);
          *reinterpret_cast<sf_u32x2*>(out + o) = v;
        }
      }
    }
  }
}

// One launch per 256 rows: rows [m0, m0 + 256) of A, out and every partial slot
// (slot stride M·N).  N must be a multiple of 16·WN·4 and of 128·rows_wn(1).
template <int WN, int MODE>
inline void launch_rows(const uint16_t* A, int M, const uint16_t* W, int K, int N, int ks_max,
                        float* part, uint16_t* out, hipStream_t st) {
  const int ks = rows_splits<WN>(M, N, K, ks_max);
  for (int m0 = 0; m0 < M; m0 += 256) {
    const int mb = sf_imin(256, M - m0);
    const int rg = rows_rg(mb);
    const RowsPlan p{rows_tiles<WN>(N, rg), ks, rows_stages(K)};
    const dim3 grid(rows_grid(p));
    const uint16_t* a = A + (size_t)m0 * K;
    float* pp = part ? part + (size_t)m0 * N : nullptr;
    uint16_t* oo = out ? out + (size_t)m0 * N : nullptr;
    const size_t ps = (size_t)M * N;
    if (rg == 1)
      hipLaunchKernelGGL((gemm_rows_kernel<1, rows_wn<WN>(1), MODE>), grid, dim3(kThreads), 0, st,
                         a, mb, W, K, N, p, pp, ps, oo);
    else
      hipLaunchKernelGGL((gemm_rows_kernel<2, WN, MODE>), grid, dim3(kThreads), 0, st, a, mb, W, K,
                         N, p, pp, ps, oo);
  }
}

}  // namespace sfg
