// The verify step's output head: logits of every row of the block in one pass
// over the head weights, with Fast-dLLM's shift done by the stores.
//
// Reference semantics:
//   specfold/generate/fastdllm_v2_folded.py:222-223   logits = lm_head(norm(h))
//   specfold/generate/fastdllm_v2_generation.py:121-126  _shift_logits: position n
//       of a block takes position n-1's logits, position 0 keeps its own
//   specfold/generate/nld_folded.py:237                 NLD: unshifted
// (the Triton path, fastdllm_v2_folded.py:365-366, runs the same torch ops).
//
// logits[m, v] = sum_k X[m, k] W[v, k] for M <= 256 rows per pass (B1·N = 256 at
// B1 = 8) and V = 131k-152k columns: 256 flop per weight byte, so the head is
// bound by streaming W (1.09 GB at 7B) unless the MFMAs fall below ~60% of their
// peak.  Design (one 8-wave workgroup per CU, one 128-column tile per workgroup,
// the whole of K):
//   * the weights go from HBM straight into VGPRs: wave w = (row group rg, column
//     group cg) owns WN = 2 tiles of 16 columns; in the packed layout
//     (sf_pack_weight) a tile's 32-K chunk is one contiguous 1 KB block, so each
//     weight load is a fully used 1 KB read, and a wave's stream is sequential.
//     The two row groups load the same blocks (the second read hits L2).  Three
//     64-K stages of weights are in flight per wave (48 VGPRs);
//   * the rows X are shared by the 8 waves: each 64-K stage (256 rows x 64 K,
//     32 KB) goes to an LDS ring of 4 stages by direct global -> LDS copies (X is
//     1.8 MB and stays in L2), XOR-swizzled so the fragment reads are
//     conflict-free (the A-tile layout of the other GEMMs: sf_index.h);
//   * v_mfma_f32_16x16x32_bf16 with the weight fragment as the first operand, so
//     each lane ends with 4 consecutive columns of one row (8-byte stores);
//   * the store's row map does the shift: row (b, n) goes to output row
//     (b, n + 1), row (b, 0) also to (b, 0), row (b, N - 1) nowhere.
// Each 64-K stage per wave: 4 A copies + 4 weight loads issued, 16 A fragment
// reads, 32 MFMAs.  fp32 accumulation over the whole of K in one order (K
// ascending), so a row's logits do not depend on the other rows or on M.
#include <type_traits>

#include "sf_common.h"
#include "sf_index.h"

namespace {

using namespace sfg;

// Rows of a launch: output row r (r < Mo, the launch's rows in order) is row
// b*N + n of the logits, b = r / W, n = lo + r % W: every N-row block's positions
// [lo, lo + W); its input row is b*N + n - 1 under Fast-dLLM's shift (n > 0), else
// b*N + n.  The whole block (lo = 0, W = N) gives every row; N = Mo, no shift: the
// plain product.
struct HeadRows {
  int N, lo, W, shift;
};
SF_DEV int head_out_row(int r, const HeadRows& hr) {
  const int b = r / hr.W;
  return b * hr.N + hr.lo + (r - b * hr.W);
}
SF_DEV int head_in_row(int r, const HeadRows& hr) {
  const int b = r / hr.W;
  const int n = hr.lo + (r - b * hr.W);
  return b * hr.N + ((hr.shift && n > 0) ? n - 1 : n);
}

// A workgroup of NW waves = RG row groups x NW / RG column groups of WN 16-column
// tiles over a pass of HR rows (256 or 128); TN columns per workgroup tile; a ring
// of R 64-K stages (X in LDS, each wave's weight fragments in VGPRs), R - 1 of
// them in flight.
template <int NW, int RG, int WN, int R, int HR>
struct HeadShape {
  static constexpr int kNW = NW;
  static constexpr int kRG = RG;
  static constexpr int kWN = WN;
  static constexpr int kRing = R;
  static constexpr int kRows = HR;                 // rows per pass
  static constexpr int kMT = HR / 16;              // m tiles per pass
  static constexpr int kStageWords = 2 * kMT * 64; // 16-byte words of X per stage
  static constexpr int kCG = NW / RG;              // column groups
  static constexpr int kNMT = kMT / RG;            // m tiles per wave
  static constexpr int kTN = kCG * WN * 16;        // columns of a tile
  static constexpr int kDA = 2 * kMT / NW;         // X copies per wave per stage
  static constexpr int kDB = 2 * WN;               // weight loads per wave per stage
  static_assert(kDA * NW == 2 * kMT, "the X copies of a stage divide over the waves");
  // X fragments read (and waited for) FG m tiles at a time: 4 where the
  // accumulators leave no room for 8
  static constexpr int kFG = kNMT * WN >= 32 ? 4 : (kNMT < 8 ? kNMT : 8);
  static_assert(kNMT % kFG == 0, "whole fragment groups");
};
// Passes of 256 rows.  The whole rounds: 8 waves x 32 columns over all 256 rows
// -- each weight byte loaded by one wave, 64 KB of weights in flight per CU.
using HeadMain = HeadShape<8, 1, 2, 3, 256>;
// The partial last round: 8 waves = 2 row groups x 4 column groups of 32 columns
// (each weight block loaded by both row groups), 128-column tiles spread over
// twice as many CUs.
using HeadTail = HeadShape<8, 2, 2, 4, 256>;
// Passes of at most 128 rows (a row window of the block): the same tiles with half
// the X bytes and MFMAs per column, and a ring one stage deeper.
using HeadMain128 = HeadShape<8, 1, 2, 4, 128>;
using HeadTail128 = HeadShape<8, 2, 2, 4, 128>;

// The X fragments of FG consecutive m tiles (1 KB apart) from LDS byte address a,
// without waiting (sf_lds_read16 with compile-time offsets).
template <int FG, int I = 0>
SF_DEV void head_fragments(sf_u32x4 (&f)[FG], sf_lds_off a) {
  if constexpr (I < FG) {
    f[I] = sf_lds_read16<I * 1024>(a);
    head_fragments<FG, I + 1>(f, a);
  }
}

// Calls f(sb + J, J) for J = J0 .. R-1 (with J a compile-time constant, so every
// ring index below stays static), or only for sb + J < S when TAIL.
template <int J, int R, bool TAIL, class F>
SF_DEV void head_stages(int sb, int S, F& f) {
  if constexpr (J < R) {
    if (!TAIL || sb + J < S) f(sb + J, std::integral_constant<int, J>{});
    head_stages<J + 1, R, TAIL>(sb, S, f);
  }
}

// One pass of at most HR rows (the launch's output rows [m0, m0 + HR) of Mo, in
// the row map hr) over the column tiles t0 + blockIdx.x of TN columns.  X: the
// input rows (row stride K); W: packed [V, K]; out: row stride ldo.
template <int NW, int RG, int WN, int R, int HR>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(8 / NW, 8 / NW)))
void head_kernel(const uint16_t* __restrict__ X, int Mo, int m0, HeadRows hr,
                 const uint16_t* __restrict__ W, int K, int t0, uint16_t* __restrict__ out,
                 long long ldo) {
  using Sh = HeadShape<NW, RG, WN, R, HR>;
  constexpr int kHMT = Sh::kMT;
  constexpr int kHStageWords = Sh::kStageWords;
  constexpr int kHDA = Sh::kDA;
  constexpr int kHDB = Sh::kDB;
  constexpr int kHWN = WN;
  __shared__ sf_u32x4 ring[R * kHStageWords];
  constexpr int CG = Sh::kCG;
  constexpr int NMT = Sh::kNMT;
  constexpr int TN = Sh::kTN;
  constexpr int FG = Sh::kFG;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // the wave index in a scalar register: the copies' LDS bases (M0) are then
  // wave-uniform for the compiler too
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wv / CG;
  const int cg = wv - rg * CG;
  const int t = t0 + blockIdx.x;
  const int S = K / kKC;
  const int slast = S - 1;

  // X copies: copy q = wv + NW*j is (chunk q / kHMT, m tile q % kHMT); lane L
  // brings pass row L/4 of the tile (rows past Mo re-read the last one), unit
  // a_copy_unit(L), from its input row
  const uint16_t* asrc[kHDA];
  int adst[kHDA];
#pragma unroll
  for (int j = 0; j < kHDA; ++j) {
    const int q = wv + NW * j;
    const int ch = q / kHMT, mt = q - ch * kHMT;
    const int r = sf_imin(m0 + mt * 16 + (lane >> 2), Mo - 1);
    asrc[j] = X + (size_t)head_in_row(r, hr) * K + ch * 32 + a_copy_unit(lane) * 8;
    adst[j] = (ch * kHMT + mt) * 64;
  }
  // this lane's weight streams: 16-column tiles t*TN/16 + cg*WN + tt
  const uint16_t* wsrc[kHWN];
#pragma unroll
  for (int tt = 0; tt < kHWN; ++tt)
    wsrc[tt] = weight_lane_ptr(W, t * (TN / 16) + cg * kHWN + tt, K, lane);

  // Issues are made for consecutive stages s = 0, 1, ...; the stream pointers
  // advance one stage after each issue until they reach the last stage, so an
  // issue past it re-reads the last stage (clamped) and one pointer per stream
  // stays live (no per-issue address arithmetic).
  sf_u32x4 wreg[R][2][kHWN];   // the weight fragments of the R - 1 stages in flight
  auto issue = [&](int s, int j) {
    sf_u32x4* sl = ring + j * kHStageWords;
#pragma unroll
    for (int q = 0; q < kHDA; ++q) sf_lds_dma16(asrc[q], sl + adst[q]);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int tt = 0; tt < kHWN; ++tt)
        wreg[j][c][tt] = *reinterpret_cast<const sf_u32x4*>(wsrc[tt] + c * kKsStride);
    // advance unless this was the last stage (a select, not a branch)
    const int live = s < slast ? 1 : 0;
#pragma unroll
    for (int q = 0; q < kHDA; ++q) asrc[q] += live * kKC;
#pragma unroll
    for (int tt = 0; tt < kHWN; ++tt) wsrc[tt] += live * (2 * kKsStride);
  };
#pragma unroll
  for (int j = 0; j < R - 1; ++j) issue(j, j);

  sf_f32x4 acc[NMT][kHWN];
#pragma unroll
  for (int i = 0; i < NMT; ++i)
#pragma unroll
    for (int tt = 0; tt < kHWN; ++tt) acc[i][tt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  // this lane's X fragment of m tile rg*NMT + i in chunk c: word a_read_word(lane)
  // of tile (c, rg*NMT + i)
  const sf_lds_off a_byte = (sf_lds_off)((rg * NMT) * 64 + a_read_word(lane)) * 16;
  // stage s in ring slot j: wait for it (issued R - 1 stages ago: its X copies of
  // every wave -- the barrier -- and this wave's weights; no wave still reads slot
  // j - 1), issue stage s + R - 1 into slot j - 1, then its MFMAs, FG m tiles at
  // a time.  Every m tile is computed (rows past M are copies of row M - 1, never
  // stored): no branch in the loop, so the compiler's waits stay exact.
  auto stage = [&](int s, auto jc) {
    constexpr int j = decltype(jc)::value;
    sf_wait_vm_barrier<(R - 2) * (kHDA + kHDB)>();
    issue(s + R - 1, (j + R - 1) % R);
    const sf_lds_off base = sf_lds_addr(ring + j * kHStageWords);
    // the stage's NG = 2 chunks x NMT / FG fragment groups, software-pipelined:
    // group g + 1's reads are issued before group g's wait, so the LDS latency of
    // one group hides behind the MFMAs of the other
    constexpr int NH = NMT / FG;
    constexpr int NG = 2 * NH;
    sf_u32x4 fb[2][FG];
    auto group_addr = [&](int gi) {
      return base + a_byte + ((gi / NH) * kHMT + (gi % NH) * FG) * 1024;
    };
    head_fragments<FG>(fb[0], group_addr(0));
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      if (gi + 1 < NG) {
        head_fragments<FG>(fb[(gi + 1) & 1], group_addr(gi + 1));
        sf_lds_reads_done_but<FG>(fb[gi & 1]);
      } else {
        sf_lds_reads_done(fb[gi & 1]);
      }
      const int c = gi / NH, h = gi % NH;
#pragma unroll
      for (int i = 0; i < FG; ++i)
#pragma unroll
        for (int tt = 0; tt < kHWN; ++tt)
          acc[h * FG + i][tt] = sf_mfma16x16x32(sf_as_bf16x8(wreg[j][c][tt]),
                                                sf_as_bf16x8(fb[gi & 1][i]), acc[h * FG + i][tt]);
    }
  };
  int sb = 0;
#pragma unroll 1
  for (; sb + R <= S; sb += R)   // whole groups of R stages: no branch inside
    head_stages<0, R, false>(sb, S, stage);
  head_stages<0, R, true>(sb, S, stage);   // the last S % R (wave-uniform branches, once)
  // drain the clamped re-issues past the last stage before the workgroup exits
  sf_wait_vm_barrier<0>();

  // lane: row (rg*NMT + i)*16 + lane%16 of the pass, columns col0 + 16 tt .. +4
  const int col0 = t * TN + cg * kHWN * 16 + (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < NMT; ++i) {
    const int row = m0 + (rg * NMT + i) * 16 + (lane & 15);
    if (row < Mo) {
      sf_u32x2 v[kHWN];
#pragma unroll
      for (int tt = 0; tt < kHWN; ++tt) {
        v[tt][0] = sf_pack2(acc[i][tt][0], acc[i][tt][1]);
        v[tt][1] = sf_pack2(acc[i][tt][2], acc[i][tt][3]);
      }
      const size_t orow = (size_t)head_out_row(row, hr);
#pragma unroll
      for (int tt = 0; tt < kHWN; ++tt)
        sf_handoff_store(reinterpret_cast<sf_u32x2*>(out + orow * ldo + col0 + tt * 16), v[tt]);
    }
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

namespace {

// Whole rounds of the main shape's tiles (one per CU), the rest in the tail shape's
// (the partial last round spread over up to twice the CUs); passes of Main::kRows.
template <class Main, class Tail>
void head_launch(const uint16_t* x, int Mo, const HeadRows& hr, const uint16_t* w, int D, int V,
                 uint16_t* logits, long long ld_out, hipStream_t st) {
  constexpr int kCUs = 256;
  const int t_main = V / Main::kTN;
  const int n_main = (t_main / kCUs) * kCUs;
  const int n_rest = (V - n_main * Main::kTN) / Tail::kTN;
  for (int m0 = 0; m0 < Mo; m0 += Main::kRows) {
    if (n_main)
      hipLaunchKernelGGL((head_kernel<Main::kNW, Main::kRG, Main::kWN, Main::kRing, Main::kRows>),
                         dim3(n_main), dim3(Main::kNW * 64), 0, st, x, Mo, m0, hr, w, D, 0, logits,
                         ld_out);
    if (n_rest)
      hipLaunchKernelGGL((head_kernel<Tail::kNW, Tail::kRG, Tail::kWN, Tail::kRing, Tail::kRows>),
                         dim3(n_rest), dim3(Tail::kNW * 64), 0, st, x, Mo, m0, hr, w, D,
                         n_main * (Main::kTN / Tail::kTN), logits, ld_out);
  }
}

}  // namespace

extern "C" int sf_head_logits_rows(const uint16_t* x, int M, const uint16_t* w, int D, int V,
                                   int N, int shift, int row_lo, int row_n, uint16_t* logits,
                                   long long ld_out, void* stream) {
  if (!x || !w || !logits) return SF_ERR_ARG;
  if (M < 1 || M > 1024 || D < kKC || D % kKC || V < HeadTail::kTN || V % HeadTail::kTN ||
      ld_out < V || ld_out % 4 || !aligned16(x) || !aligned16(w) ||
      reinterpret_cast<uintptr_t>(logits) % 8)
    return SF_ERR_SHAPE;
  if (N < 1 || M % N || row_lo < 0 || row_n < 1 || row_lo + row_n > N) return SF_ERR_SHAPE;
  const HeadRows hr{N, row_lo, row_n, shift ? 1 : 0};
  const int Mo = (M / N) * row_n;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (Mo <= HeadMain128::kRows)
    head_launch<HeadMain128, HeadTail128>(x, Mo, hr, w, D, V, logits, ld_out, st);
  else
    head_launch<HeadMain, HeadTail>(x, Mo, hr, w, D, V, logits, ld_out, st);
  return sf_launch_status();
}

extern "C" int sf_head_logits(const uint16_t* x, int M, const uint16_t* w, int D, int V,
                              int shift_n, uint16_t* logits, long long ld_out, void* stream) {
  if (M < 1 || shift_n < 0 || shift_n == 1 || (shift_n > 0 && M % shift_n)) return SF_ERR_SHAPE;
  const int N = shift_n > 0 ? shift_n : M;
  return sf_head_logits_rows(x, M, w, D, V, N, shift_n > 0, 0, N, logits, ld_out, stream);
}

extern "C" int sf_lm_head(const uint16_t* x, int M, const uint16_t* w, int D, int V,
                          uint16_t* logits, void* stream) {
  return sf_head_logits(x, M, w, D, V, 0, logits, V, stream);
}
