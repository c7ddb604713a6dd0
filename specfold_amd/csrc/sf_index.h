// Integer index maps of the kernels, shared with their CPU checker.
//
// Plain integer functions: the stream-K schedule of the weight-streaming GEMMs
// and their output-column / packed-weight addressing, and the prefix attention's
// work decomposition, key-slot permutation, V^T swizzle and page-group
// addressing.  Under hipcc they are host+device functions used by the kernels
// and the launchers; under a plain C++ compiler they build on their own, so the
// CPU test tests/cpp/index_check.cpp walks them over the shapes the entry points
// accept and checks that every access lands inside its buffer, every unit of
// work is done exactly once and the kernels that pass work to each other agree
// on its layout.
#pragma once

#include <stddef.h>

#if defined(__HIPCC__)
#define SF_IDX __host__ __device__ __forceinline__
#else
#define SF_IDX inline
#endif

SF_IDX int sf_imin(int a, int b) { return a < b ? a : b; }
SF_IDX int sf_imax(int a, int b) { return a > b ? a : b; }

// ---------------------------------------------------------------------------
// Weight-streaming GEMM (sf_gemm_core.h)
// ---------------------------------------------------------------------------
namespace sfg {

// Packed ("fragment-major") weights: for each 16-row tile of W [N, K] and each
// 32-wide K chunk, the 64 lanes' MFMA B fragments (lane l holds
// W[16t + l%16][32c + 8(l/16) .. +8]) are one contiguous 1 KB block, and the
// chunks of a tile follow each other.
constexpr int kKsStride = 512;     // elements between 32-wide chunks of a tile
constexpr int kKC = 64;            // K per stage: two 32-wide MFMA chunks
constexpr int kLdsBudget = 152 * 1024;  // LDS of a stage ring
#ifndef SFG_RING_MAX
#define SFG_RING_MAX 6
#endif

// Lane `lane`'s first fragment of 16-row tile `tile16`, from base W (a pointer to
// the packed weights in the kernels; an integer 0 gives the element offset).
template <typename P>
SF_IDX P weight_lane_ptr(P W, int tile16, int K, int lane) {
  return W + (size_t)tile16 * (K / 32) * 512 + lane * 8;
}

// A stage of the GEMM core is 64 K, two 32-wide MFMA chunks; chunk c of stage sc:
SF_IDX int weight_chunk(int sc, int c) { return 2 * sc + c; }

// A operand in LDS: per (chunk, m tile) a 1 KB tile of 16 rows x 64 bytes whose
// four 16-byte units are XOR-swizzled (unit u of row r at position u ^ a_swz(r)).
// Direct copy j of wave wv brings (chunk, m tile) q = a_copy(wv, j, NMT) = ch*NMT
// + mt (waves with fewer real copies repeat the last one); its lane L writes word
// L of the tile (row L/4, position L%4) with A unit a_copy_unit(L) of that row.
// The MFMA reader lane l (row l%16, unit l/16) reads word a_read_word(l).
SF_IDX int a_swz(int r) { return (r >> 1) & 3; }
SF_IDX int a_copy(int wv, int j, int NMT) { return sf_imin(wv + 8 * j, 2 * NMT - 1); }
SF_IDX int a_copy_unit(int L) { return (L & 3) ^ a_swz(L >> 2); }
SF_IDX int a_read_word(int l) { return (l & 15) * 4 + ((l >> 4) ^ a_swz(l & 15)); }

// Output column held by lane `lane` of wave `wv` (its column group) in its column
// tile `tt` of 128·WN-column tile t (WN tiles of 16 per wave).  SILU: the gate and
// the up tile of one wave cover the same 16 columns of a 128-column tile.
template <int WN, bool SILU>
SF_IDX int gemm_col(int t, int wv, int tt, int lane) {
  return SILU ? t * 128 + wv * 16 + (lane & 15)
              : t * 128 * WN + wv * 16 * WN + tt * 16 + (lane & 15);
}

// Stream-K schedule.  The output columns are cut into T tiles and K into S
// stages of 64; the T*S (tile, stage) units are dealt out in tile-major order,
// U consecutive units per workgroup.
#ifndef SFG_GRID
#define SFG_GRID 256   // workgroups (MI355X: one 8-wave workgroup per CU)
#endif

struct Plan {
  int T;       // column tiles
  int S;       // K stages
  int U;       // units per workgroup
  int NU = 0;  // > 0: column-spread plan (below) over NU column units of 16
  int KS = 0;  // > 0: split plan (below), KS workgroups per tile
};

// Balanced plan over SFG_GRID workgroups.
inline Plan make_plan(int T, int S) {
  const long long units = (long long)T * S;
  const int U = (int)((units + SFG_GRID - 1) / SFG_GRID);
  return Plan{T, S, U < 1 ? 1 : U};
}
// One workgroup per whole tile: every tile has a single contributor.
inline Plan make_plan_whole(int T, int S) { return Plan{T, S, S}; }
// Column-spread plan (gate/up: kSilu only): the NU 16-column units of the output
// are dealt out over T workgroups, workgroup t taking units [spread_begin(t),
// spread_begin(t + 1)) -- between 1 and 8, one per wave -- over all S stages of K.
// Every tile (a workgroup's columns) is whole, so there are no partial slots, and
// every CU streams NU/T units instead of the 8 of a 128-column tile.
inline Plan make_plan_spread(int NU, int S, int T) { return Plan{T, S, S, NU}; }
SF_IDX int spread_begin(int t, const Plan& p) { return (int)((long long)t * p.NU / p.T); }
// Workgroups of a column-spread plan over nu units: the fewest that give none more
// than ceil(nu / grid) units, so all but a few carry the same count (a full grid
// of 4 and 5 units leaves the CUs with 4 idle through the last fifth of the
// stream, when the others no longer fill HBM).
SF_IDX int spread_workgroups(int nu, int grid) {
  const int k = (nu + grid - 1) / grid;
  return (nu + k - 1) / k;
}
// Split plan: each of the T tiles is cut into KS ranges of whole K stages (range
// j: [split_begin(j), split_begin(j + 1))), one workgroup each, so T·KS workgroups
// each hold a single piece -- no range crosses a tile, so no workgroup pays a
// second ring fill and epilogue (the stream-K ranges that straddle two tiles
// finish last) -- and range j of a tile goes to partial slot j.  KS is the most
// that keeps T·KS within the grid.
inline Plan make_plan_split(int T, int S) {
  int ks = SFG_GRID / T;
  ks = ks < 1 ? 1 : (ks > S ? S : ks);
  return Plan{T, S, (S + ks - 1) / ks, 0, ks};
}
SF_IDX int split_begin(int j, const Plan& p) { return (int)((long long)j * p.S / p.KS); }

inline int plan_grid(const Plan& p) {
  if (p.KS) return p.T * p.KS;
  return (int)(((long long)p.T * p.S + p.U - 1) / p.U);
}
// Upper bound of contributors (slots) per tile.
inline int plan_slots(const Plan& p) {
  if (p.KS) return p.KS;
  return p.U >= p.S ? 2 : (p.S + p.U - 1) / p.U + 1;
}

// First and last workgroup holding units of tile t; a piece of tile t computed by
// workgroup g goes to partial slot g - tile_first(t).
SF_IDX int tile_first(int t, const Plan& p) {
  if (p.KS) return t * p.KS;
  return (int)((long long)t * p.S / p.U);
}
SF_IDX int tile_last(int t, const Plan& p) {
  if (p.KS) return t * p.KS + p.KS - 1;
  return (int)(((long long)(t + 1) * p.S - 1) / p.U);
}

// Workgroup g's units are [plan_range_begin(g), plan_range_end(g)) in tile-major
// unit order (unit t·S + s): [g·U, min((g + 1)·U, T·S)) for stream-K and the
// spread plan, range g % KS of tile g / KS for a split plan.
SF_IDX int plan_range_begin(int g, const Plan& p) {
  if (p.KS) return (g / p.KS) * p.S + split_begin(g % p.KS, p);
  return g * p.U;
}
SF_IDX int plan_range_end(int g, const Plan& p) {
  if (p.KS) return (g / p.KS) * p.S + split_begin(g % p.KS + 1, p);
  const int total = p.T * p.S;
  return sf_imin((g + 1) * p.U, total);
}

// The piece of a workgroup's range that starts at unit u: tile t, stages [sa, sb).
struct Piece {
  int t, sa, sb;
};
SF_IDX Piece plan_piece(int u, int u_end, const Plan& p) {
  const int t = u / p.S;
  const int sa = u - t * p.S;
  return Piece{t, sa, sf_imin(p.S, sa + (u_end - u))};
}

// Partial slots of a plan: [plan_slots][mcap][N] fp32.
inline size_t part_bytes(const Plan& p, int mcap, int N) {
  return (size_t)plan_slots(p) * mcap * N * sizeof(float);
}

// ---------------------------------------------------------------------------
// All-rows GEMM (sf_gemm_rows.h): every row of A, up to 128·RG, in one pass over
// the weights.  The 8 waves are RG row groups (128 rows each) x CG = 8 / RG
// column groups (WN tiles of 16 columns each), so a workgroup tile is 16·WN·CG
// columns by all rows.  K (S stages of 64) is cut into KS ranges of whole stages;
// workgroup g computes range s of tile t, (s, t) = item rows_item(g) in split-major
// order.  KS > 1 leaves KS fp32 partial sums per output for the consumer to add
// in range order.
struct RowsPlan {
  int T;   // column tiles
  int KS;  // K ranges
  int S;   // K stages
};
// KS fills SFG_GRID workgroups without exceeding ks_max (1 where the caller has
// no partial buffer) or an eighth of the stages (a range of at least 8 stages
// keeps the partial traffic below the weight stream's).
inline RowsPlan make_rows_plan(int T, int S, int ks_max) {
  int ks = SFG_GRID / T;
  ks = sf_imin(ks, (S + 7) / 8);
  ks = sf_imin(ks, ks_max);
  return RowsPlan{T, ks < 1 ? 1 : ks, S};
}
SF_IDX int rows_grid(const RowsPlan& p) { return p.T * p.KS; }
// Workgroup g runs on XCD g % 8; the G items are numbered so that one XCD's
// workgroups take consecutive items (split-major: they share their K range of A,
// which stays in that XCD's L2).  A bijection of [0, G).
SF_IDX int rows_item(int g, int G) {
  const int x = g & 7;
  return x * (G >> 3) + sf_imin(x, G & 7) + (g >> 3);
}
SF_IDX int rows_split_begin(int s, const RowsPlan& p) {
  return (int)((long long)p.S * s / p.KS);
}
// Stage layout of a workgroup of RG row groups and WN 16-column tiles per wave,
// CPS 32-wide K chunks per stage.  The copies of a stage are dealt over the 8 waves
// (copy q = wv + 8j); a wave with fewer real copies repeats the last one (the same
// bytes to the same place), so every wave issues the same number per stage.
#ifndef SFG_ROWS_CPS
#define SFG_ROWS_CPS 2
#endif
template <int RG, int WN, int CPS = SFG_ROWS_CPS>
struct RowsStage {
  static constexpr int kMB = 128 * RG;       // rows per pass
  static constexpr int kMT = kMB / 16;       // m tiles
  static constexpr int kCG = 8 / RG;         // column groups
  static constexpr int kTW = kCG * WN;       // 16-column tiles of a workgroup tile
  static constexpr int kCPS = CPS;           // K chunks per stage
  static constexpr int kKS = 32 * CPS;       // K per stage
  static constexpr int kNA = CPS * kMT;      // A tile copies per stage
  static constexpr int kNW = CPS * kTW;      // weight block copies per stage
  static constexpr int kA = kNA * 64;        // 16-byte words of A per stage
  static constexpr int kW = kNW * 64;        // words of weights per stage
  static constexpr int kWords = kA + kW;
  static constexpr int kDA = (kNA + 7) / 8;  // A copies per wave per stage
  static constexpr int kDW = (kNW + 7) / 8;  // weight copies per wave per stage
  static constexpr int kRing =
      kLdsBudget / (kWords * 16) < SFG_RING_MAX ? kLdsBudget / (kWords * 16) : SFG_RING_MAX;
};
// A pass of at most 128 rows uses one row group (RG = 1, 8 column groups) with
// half the tiles per wave (at least one), a pass of up to 256 rows two; WN is
// the two-group configuration's.
inline int rows_rg(int mb) { return mb <= 128 ? 1 : 2; }
template <int WN>
constexpr int rows_wn(int rg) { return rg == 2 ? WN : (WN > 1 ? WN / 2 : 1); }
template <int WN>
inline int rows_tiles(int N, int rg) { return N / (16 * rows_wn<WN>(rg) * (8 / rg)); }
// K stages of an all-rows GEMM (32·CPS each).
inline int rows_stages(int K) { return K / (32 * SFG_ROWS_CPS); }
// K ranges of an all-rows GEMM over M rows: the first pass's plan, used by every
// pass (the consumer adds the same number of partial slots for every row).
template <int WN>
inline int rows_splits(int M, int N, int K, int ks_max) {
  const int rg = rows_rg(sf_imin(256, M));
  return make_rows_plan(rows_tiles<WN>(N, rg), rows_stages(K), ks_max).KS;
}
// Copy q of a stage (clamped to the last real copy): A tile (chunk q / MT, m tile
// q % MT, in the tile layout of a_copy); weight block (tile q / CPS, chunk q % CPS).
SF_IDX int rows_a_copy(int q, int NA) { return sf_imin(q, NA - 1); }
SF_IDX int rows_a_chunk(int q, int MT) { return q / MT; }
SF_IDX int rows_a_mtile(int q, int MT) { return q % MT; }
SF_IDX int rows_w_copy(int q, int NW) { return sf_imin(q, NW - 1); }
SF_IDX int rows_w_tile(int q, int CPS) { return q / CPS; }
SF_IDX int rows_w_chunk(int q, int CPS) { return q % CPS; }
// fp32 partials of a plan for M rows and N columns: [KS][M][N].
inline size_t rows_part_bytes(const RowsPlan& p, int M, int N) {
  return p.KS > 1 ? (size_t)p.KS * M * N * sizeof(float) : 0;
}

}  // namespace sfg

// ---------------------------------------------------------------------------
// Prefix attention (sf_attn.hip)
// ---------------------------------------------------------------------------
namespace sfa {

constexpr int kHD = 128;
constexpr int kQT = 128;       // queries per work item: 4 query groups of 32
constexpr int kChunk = 64;     // prefix keys per chunk (one LDS ring stage)
constexpr int kMaxChunks = 512;   // prefix <= 32768 keys
constexpr int kMaxRanges = 64;    // prefix partials per query at most
#ifndef SFA_ITEMS_TARGET
#define SFA_ITEMS_TARGET 256
#endif
constexpr int kItemsTarget = SFA_ITEMS_TARGET;

// LDS layout of a staged chunk: key rows of 256 bytes (16 units of 16 bytes =
// 8 dims each), K rows then V rows.  Unit u of key row r sits at unit
//  k_unit(r, u) = u ^ (r & 15)      in K: the 16 consecutive rows one MFMA
//                                   operand read takes at one unit hit 16
//                                   distinct units;
//  v_unit(r, u) = u ^ 2 * (r & 7)   in V: a transposing read takes 16
//                                   consecutive rows x one aligned unit pair;
//                                   rows 0-7 land on 8 distinct pairs, rows 8-15
//                                   on the same 8 (the read's second pass).
// Both are involutions, so the copy that fills physical unit p of row r reads
// logical unit k_unit(r, p) / v_unit(r, p).
SF_IDX int k_unit(int r, int u) { return u ^ (r & 15); }
SF_IDX int v_unit(int r, int u) { return u ^ (2 * (r & 7)); }
constexpr int kRowBytes = kHD * 2;               // one key row in LDS
constexpr int kHalfBytes = kChunk * kRowBytes;   // the K (or V) rows of a chunk

// Operand reads of a staged chunk, byte offsets from the chunk's K rows:
// * K fragment of MFMA A = K (16 keys of tile 0 x 32 dims ds*32..): lane l reads
//   key row l%16, logical unit ds*4 + l/16 (16 bytes); tile t adds 16 rows.
SF_IDX int k_frag_off(int lane, int ds) {
  const int row = lane & 15;
  return row * kRowBytes + k_unit(row, ds * 4 + (lane >> 4)) * 16;
}
// * V^T fragment of MFMA A = V^T (16 dims dt*16.. x 32 keys) by two transposing
//   reads (keys 4g..4g+3 of tiles 0 and 1, g = l/16): lane L of group g points at
//   row 4g + L/4, dims dt*16 + 4(L%4) .. +4 (8 bytes); tile 1 adds 16 rows.
SF_IDX int v_tr_off(int lane, int dt) {
  const int L = lane & 15;
  const int row = 4 * (lane >> 4) + (L >> 2);
  const int col = dt * 16 + 4 * (L & 3);  // first dim
  return kHalfBytes + row * kRowBytes + v_unit(row, col >> 3) * 16 + (col & 7) * 2;
}

// Chunks per work item: enough that the items fill about one round of the
// resident grid (longer ranges write fewer partials) and no query has more
// than kMaxRanges partials.  A pure function of device-side sizes, evaluated
// identically by the prefix and merge kernels.
SF_IDX int prefix_cpi(int nch, int n_qt, int Hkv) {
  const long long work = (long long)nch * n_qt * Hkv;
  int c = (int)((work + kItemsTarget - 1) / kItemsTarget);
  c = sf_imax(c, (nch + kMaxRanges - 1) / kMaxRanges);
  return sf_imax(1, sf_imin(c, nch));
}

// 16-key group j (0..3) of chunk ci starts at key chunk_group_g0 (groups past
// the prefix end are clamped to the last group holding keys, last_group_g0(P));
// row kr of the group holds key g0 + group_key(kr, g0, P) (keys past the end
// clamped to the last key).  With a page size that is a multiple of 16 a group
// never straddles pages.
SF_IDX int last_group_g0(int P) { return (P - 1) & ~15; }
SF_IDX int chunk_group_g0(int ci, int j, int last_g0) {
  return sf_imin(ci * kChunk + 16 * j, last_g0);
}
SF_IDX int group_key(int kr, int g0, int P) { return sf_imin(kr, P - 1 - g0); }

// Persistent prefix grid (a multiple of 8 workgroups; workgroup b runs on XCD
// b % 8): XCD x walks items [xcd_begin(items, x), xcd_begin(items, x + 1)).
SF_IDX int xcd_begin(int items, int xcd) { return (int)(((long long)items * xcd) >> 3); }

// Item it of the prefix pass: query tile qt, chunk range r, kv head h (the
// query tiles of one (range, head) are consecutive: one XCD, one L2).
struct AttnItem {
  int qt, r, h;
};
SF_IDX AttnItem attn_item(int it, int n_qt, int nr) {
  const int qt = it % n_qt;
  const int rest = it / n_qt;
  return AttnItem{qt, rest % nr, rest / nr};
}

// The prefix pass's decomposition for nq active queries per kv head and a prefix
// of P keys: n_qt query tiles, nch chunks, cpi chunks per range, nr ranges
// (= partials per query); items = n_qt · nr · Hkv ...
struct PrefixGrid {
  int n_qt, nch, cpi, nr;
};
SF_IDX PrefixGrid prefix_grid(int P, int nq, int Hkv) {
  const int n_qt = (nq + kQT - 1) / kQT;
  const int nch = (P + kChunk - 1) / kChunk;
  const int cpi = prefix_cpi(nch, n_qt, Hkv);
  return PrefixGrid{n_qt, nch, cpi, (nch + cpi - 1) / cpi};
}
// ... and the partials per query as the merge kernel derives them from its
// query count nq = rows · G.
SF_IDX int merge_ranges(int P, int nq, int Hkv) {
  return P > 0 ? prefix_grid(P, nq, Hkv).nr : 0;
}

inline int nchunks_for(int P) { return (P + kChunk - 1) / kChunk; }
// Range slots the workspace holds per (kv head, query) for a prefix capacity P.
inline int ranges_cap(int P) { return nchunks_for(P) < kMaxRanges ? nchunks_for(P) : kMaxRanges; }

// Partial slot of query qi of range r, kv head h: the workspace holds
// [Hkv][nr_cap][qmax] slots of kHD fp32 (acc), then the same count of (m, l).
SF_IDX size_t attn_slot(int h, int r, int qi, int nr_cap, int qmax) {
  return ((size_t)h * nr_cap + r) * qmax + qi;
}

// Persistent prefix grid for a capacity of qmax queries per kv head and a prefix
// capacity of nch chunks: enough workgroups for every item, at most one per CU
// (256 CUs), a multiple of 8.
inline int prefix_launch_grid(int qmax, int nch, int Hkv) {
  const int nr = nch < kMaxRanges ? nch : kMaxRanges;
  const long long items_cap = (long long)((qmax + kQT - 1) / kQT) * nr * Hkv;
  const long long g = ((items_cap + 7) / 8) * 8;
  return g < 256 ? (int)g : 256;
}

}  // namespace sfa

// ---------------------------------------------------------------------------
// Greedy statistics (sf_logits.hip): the slices of a logits row
// ---------------------------------------------------------------------------
namespace sfl {

constexpr int kMaxSlices = 32;          // slices per row: one wave merges their lists
constexpr int kMaxSliceVectors = 8191;  // 8-token vectors per slice: <= 65528 tokens,
                                        // so a slice's 16-bit counts and places fit
constexpr int kMaxVocab = kMaxSlices * kMaxSliceVectors * 8;   // 2,096,896 tokens

// Slices per row of V tokens (V % 8 == 0) for M rows: about 256 workgroups in
// all, at most kMaxSlices, and enough that no slice holds more than
// kMaxSliceVectors vectors (V <= kMaxVocab).
inline int slices_for(int M, int V) {
  const int nvec = V / 8;
  const int need = (nvec + kMaxSliceVectors - 1) / kMaxSliceVectors;
  return sf_imax(need, sf_imax(1, sf_imin(kMaxSlices, 256 / M)));
}
// Slice s of S holds the vectors [slice_begin(s), slice_begin(s + 1)) of nvec.
SF_IDX int slice_begin(int s, int nvec, int S) { return (int)((long long)nvec * s / S); }

}  // namespace sfl
