// CPU checker of the kernels' integer index maps (specfold_amd/csrc/sf_index.h),
// built with a plain C++ compiler and run by tests/test_index_maps.py.
//
//   index_check <libspecfold_amd.so>
//
// Walks the maps the kernels use over the shapes the entry points accept and
// checks what the kernels rely on:
//   * stream-K GEMM plans: every (tile, stage) unit done exactly once, every
//     workgroup's range non-empty, the partial slot of each piece inside the
//     plan's slot count and the library's workspace, whole-tile plans single-
//     contributor; the all-rows GEMM's (range, tile) items, K ranges, copies,
//     LDS reads and stores (each output element once per range, inside the
//     workspace); output columns of each mode inside N and covering each tile
//     once; every packed-weight load inside the N·K weights, and the fragment it
//     reads (under the packed layout) belonging to the column the lane writes;
//   * prefix attention: a staged chunk's LDS layout (the copies fill every cell
//     once; the K fragment and transposing V^T reads, emulated element by
//     element, deliver the operands the MFMAs expect; K reads bank-conflict free
//     per quarter-wave, V^T reads on distinct 32-byte pairs per 8 rows), the
//     page-group addressing (every load inside the prefix and inside its page;
//     every real key loaded exactly once; masked rows are exactly the clamped
//     loads), the persistent grid's item walk (each item once), the chunk
//     ranges (a partition of the chunks), and the partial slots (inside the
//     library's workspace; the merge reads exactly the slots the prefix pass
//     wrote, with the same range count).
// Prints one line per family and "OK"; exits 1 at the first failed check.
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "sf_index.h"

static long long g_checks = 0;
#define CHECK(cond, ...)                                              \
  do {                                                                \
    ++g_checks;                                                       \
    if (!(cond)) {                                                    \
      fprintf(stderr, "FAIL %s:%d: %s  ", __FILE__, __LINE__, #cond); \
      fprintf(stderr, __VA_ARGS__);                                   \
      fprintf(stderr, "\n");                                          \
      exit(1);                                                        \
    }                                                                 \
  } while (0)

typedef size_t (*ws3_fn)(int, int, int);
static ws3_fn f_gemm_ws, f_qkv_ws, f_attn_ws, f_gu_ws, f_oproj_ws;

// ---------------------------------------------------------------------------
// GEMM plans
// ---------------------------------------------------------------------------
// Walks plan p as the GEMM kernel does; returns the largest slot index used.
static int walk_plan(const sfg::Plan& p, bool whole) {
  const int grid = sfg::plan_grid(p);
  const long long total = (long long)p.T * p.S;
  std::vector<unsigned char> seen((size_t)total, 0);
  std::vector<int> lo(p.T, 1 << 30), hi(p.T, -1), cnt(p.T, 0);
  int max_slot = -1;
  for (int g = 0; g < grid; ++g) {
    const int u_end = sfg::plan_range_end(g, p);
    const int u_begin = sfg::plan_range_begin(g, p);
    CHECK(u_begin < u_end, "empty range g=%d T=%d S=%d U=%d KS=%d", g, p.T, p.S, p.U, p.KS);
    int last_t = -1, pieces = 0;
    for (int u = u_begin; u < u_end;) {
      ++pieces;
      const sfg::Piece pc = sfg::plan_piece(u, u_end, p);
      CHECK(pc.t >= 0 && pc.t < p.T && pc.sa >= 0 && pc.sa < pc.sb && pc.sb <= p.S,
            "piece t=%d sa=%d sb=%d", pc.t, pc.sa, pc.sb);
      CHECK(pc.t > last_t, "tile order g=%d", g);
      last_t = pc.t;
      for (int s = pc.sa; s < pc.sb; ++s) {
        const long long unit = (long long)pc.t * p.S + s;
        CHECK(unit == u + (s - pc.sa), "unit order");
        CHECK(!seen[unit], "unit %lld twice", unit);
        seen[unit] = 1;
      }
      const int first = sfg::tile_first(pc.t, p), last = sfg::tile_last(pc.t, p);
      CHECK(first <= g && g <= last, "g=%d outside [%d, %d] of tile %d", g, first, last, pc.t);
      const int slot = g - first;
      CHECK(slot < sfg::plan_slots(p), "slot %d >= %d", slot, sfg::plan_slots(p));
      if (slot > max_slot) max_slot = slot;
      lo[pc.t] = lo[pc.t] < g ? lo[pc.t] : g;
      hi[pc.t] = hi[pc.t] > g ? hi[pc.t] : g;
      ++cnt[pc.t];
      u += pc.sb - pc.sa;
    }
    // a split plan's workgroup holds exactly one piece
    if (p.KS) CHECK(pieces == 1, "split plan g=%d: %d pieces", g, pieces);
  }
  for (long long u = 0; u < total; ++u) CHECK(seen[u], "unit %lld never done", u);
  for (int t = 0; t < p.T; ++t) {
    // the contributors of a tile are exactly tile_first .. tile_last, one piece each
    CHECK(lo[t] == sfg::tile_first(t, p) && hi[t] == sfg::tile_last(t, p) &&
              cnt[t] == hi[t] - lo[t] + 1,
          "tile %d contributors [%d, %d] x%d vs [%d, %d]", t, lo[t], hi[t], cnt[t],
          sfg::tile_first(t, p), sfg::tile_last(t, p));
    if (whole) CHECK(lo[t] == hi[t], "whole plan shares tile %d", t);
  }
  return max_slot;
}

static void check_plans() {
  long long plans = 0;
  std::vector<int> Ss;
  for (int S = 1; S <= 96; ++S) Ss.push_back(S);
  for (int S = 97; S <= 640; S += 13) Ss.push_back(S);
  for (int T = 1; T <= 160; ++T)
    for (int S : Ss) {
      const sfg::Plan p = sfg::make_plan(T, S);
      CHECK(sfg::plan_grid(p) <= SFG_GRID, "grid %d", sfg::plan_grid(p));
      walk_plan(p, false);
      const sfg::Plan w = sfg::make_plan_whole(T, S);
      CHECK(sfg::plan_grid(w) == T, "whole grid");
      walk_plan(w, true);
      // split plan: T·KS workgroups within the grid, KS = min(S, grid / T) ranges per
      // tile (whole tiles once T reaches the grid's size / 2)
      const sfg::Plan sp = sfg::make_plan_split(T, S);
      CHECK(sfg::plan_grid(sp) <= SFG_GRID && sp.KS >= 1 && sp.KS <= S, "split grid %d",
            sfg::plan_grid(sp));
      const int ss = walk_plan(sp, sp.KS == 1);
      CHECK(ss == sp.KS - 1, "split plan slots %d of %d", ss + 1, sp.KS);
      plans += 3;
    }
  // column-spread plans (gate/up): over T workgroups, workgroup t's units
  // [spread_begin(t), spread_begin(t + 1)) -- 1..8 of them, one per wave, waves past
  // them repeating the last -- cover every 16-column unit exactly once, with whole
  // tiles (no partial slots) and T workgroups
  // (T, NU): a sweep of grids, then the grids gate/up picks (spread_workgroups) for
  // every unit count it takes the plan at on 256 CUs, with the unit counts per
  // workgroup all equal to ceil(NU / 256) but a few one lower
  std::vector<std::pair<int, int>> spread_cases;
  for (int T : {1, 3, 8, 64, 255, 256})
    for (int NU = T; NU <= 8 * T; NU += (NU < 3 * T ? 1 : 7)) spread_cases.push_back({T, NU});
  for (int NU = 2 * 256; NU <= 8 * 256; ++NU) {
    const int T = sfg::spread_workgroups(NU, 256);
    const int k = (NU + 255) / 256;
    CHECK(T <= 256 && T * k >= NU && (T - 1) * k < NU, "spread grid %d for %d units", T, NU);
    int fewer = 0;
    const sfg::Plan sp = sfg::make_plan_spread(NU, 56, T);
    for (int t = 0; t < T; ++t) {
      const int n = sfg::spread_begin(t + 1, sp) - sfg::spread_begin(t, sp);
      CHECK(n == k || n == k - 1, "spread units %d of %d", n, k);
      fewer += n < k;
    }
    CHECK(fewer < T, "spread: every workgroup short");
    spread_cases.push_back({T, NU});
  }
  for (const auto& tc : spread_cases) {
    const int T = tc.first, NU = tc.second;
    {
      const sfg::Plan sp = sfg::make_plan_spread(NU, 56, T);
      CHECK(sfg::plan_grid(sp) == T, "spread grid");
      std::vector<int> hit(NU, 0);
      for (int t = 0; t < T; ++t) {
        CHECK(sfg::tile_first(t, sp) == t && sfg::tile_last(t, sp) == t, "spread tile shared");
        const int ub = sfg::spread_begin(t, sp), ue = sfg::spread_begin(t + 1, sp);
        CHECK(ue - ub >= 1 && ue - ub <= 8, "spread units %d", ue - ub);
        for (int wv = 0; wv < 8; ++wv) {
          const int unit = std::min(ub + wv, ue - 1);   // the kernel's column unit
          CHECK(unit >= 0 && unit < NU, "spread unit %d", unit);
          if (wv < ue - ub) {
            CHECK(unit == ub + wv, "spread written unit");
            ++hit[unit];
          }
        }
      }
      for (int u = 0; u < NU; ++u) CHECK(hit[u] == 1, "spread unit %d written %d times", u, hit[u]);
      ++plans;
    }
  }
  // the shapes of the workloads (hidden D, q/k/v width, intermediate I, vocab V)
  struct Shape { int D, nqkv, I, V; };
  const Shape shapes[] = {{1536, 2048, 8960, 151936},  {3584, 4608, 18944, 152064},
                          {4096, 6144, 14336, 131072}, {5120, 7168, 17408, 131072},
                          {896, 1152, 4864, 151936}};
  for (const Shape& s : shapes) {
    for (int mcap : {1, 39, 64, 65, 128, 129, 256, 1024}) {
      // QKV: 128-column tiles, 64-K stages, stream-K, partial slots [slots][bucket][n_qkv]
      const sfg::Plan q = sfg::make_plan(s.nqkv / 128, s.D / 64);
      const int qs = walk_plan(q, false);
      const size_t need_q = (size_t)(qs + 1) * mcap * s.nqkv * sizeof(float);
      CHECK(f_qkv_ws(mcap, s.D, s.nqkv) >= need_q, "qkv workspace D=%d", s.D);
      // down: 128-column tiles over D, K = I, each tile cut into whole K ranges
      const sfg::Plan d = s.D / 128 < SFG_GRID ? sfg::make_plan_split(s.D / 128, s.I / 64)
                                                : sfg::make_plan(s.D / 128, s.I / 64);
      const int ds = walk_plan(d, false);
      CHECK(f_gemm_ws(mcap, s.D, s.I) >= (size_t)(ds + 1) * mcap * s.D * sizeof(float),
            "down workspace D=%d I=%d", s.D, s.I);
      // gate/up: 128 output columns per tile, partial rows of 2I (gate, then up)
      const sfg::Plan gu = sfg::make_plan(s.I / 128, s.D / 64);
      const int gs = walk_plan(gu, false);
      CHECK(f_gu_ws(mcap, s.D, s.I) >= (size_t)(gs + 1) * mcap * 2 * s.I * sizeof(float),
            "gate/up workspace D=%d I=%d", s.D, s.I);
      plans += 3;
    }
  }
  printf("gemm plans: %lld plans walked\n", plans);
}

// All-rows GEMM (o_proj: WN 1, up to 16 K ranges, partials in the library's
// workspace; lm_head: WN 2, one range, bf16 out), walked as launch_rows and
// gemm_rows_kernel do for M rows: every workgroup maps to a distinct (range,
// tile) item and every item is taken; the ranges partition the K stages; every A
// copy reads a row of its pass inside A, every weight copy lies inside the packed
// N·K weights and fills the LDS block the readers take; every LDS access lies
// inside the ring; every store lies inside its output (partial slots: inside the
// workspace) and each output element is written once per range.
template <int RG, int WN>
static void walk_rows_pass(const sfg::RowsPlan& p, int M, int m0, int mb, int N, int K,
                           int ks, size_t part_elems, std::vector<unsigned char>* hit) {
  using St = sfg::RowsStage<RG, WN>;
  CHECK(St::kRing >= 3 && St::kRing * St::kWords * 16 <= 160 * 1024, "ring");
  CHECK(p.T * St::kTW * 16 == N, "tiles cover N: T=%d N=%d", p.T, N);
  const int G = sfg::rows_grid(p);
  std::vector<int> seen(G, 0);
  for (int g = 0; g < G; ++g) {
    const int q = sfg::rows_item(g, G);
    CHECK(q >= 0 && q < G && !seen[q]++, "item %d of %d", q, G);
  }
  for (int s = 0; s < p.KS; ++s) {
    const int s0 = sfg::rows_split_begin(s, p), s1 = sfg::rows_split_begin(s + 1, p);
    CHECK(s1 > s0 && s0 >= 0 && s1 <= p.S, "range %d [%d, %d)", s, s0, s1);
    if (s == 0) CHECK(s0 == 0, "first range");
    if (s == p.KS - 1) CHECK(s1 == p.S, "last range");
  }
  // copies of one stage: each A tile (chunk, m tile) and weight block (tile, chunk)
  // at least once over the 8 waves (waves past the last copy repeat it)
  constexpr int CPS = St::kCPS;
  std::vector<int> acell(St::kNA, 0), wcell(St::kNW, 0);
  for (int wv = 0; wv < 8; ++wv) {
    for (int j = 0; j < St::kDA; ++j) {
      const int cq = sfg::rows_a_copy(wv + 8 * j, St::kNA);
      const int ch = sfg::rows_a_chunk(cq, St::kMT), mt = sfg::rows_a_mtile(cq, St::kMT);
      CHECK(ch < CPS && mt < St::kMT, "a copy");
      ++acell[ch * St::kMT + mt];
      for (int L = 0; L < 64; ++L) {
        const int r = sf_imin(mt * 16 + (L >> 2), mb - 1);
        CHECK(r >= 0 && r < mb && m0 + r < M, "a row");
        const size_t last = (size_t)(m0 + r) * K + (size_t)(p.S - 1) * St::kKS + ch * 32 +
                            sfg::a_copy_unit(L) * 8 + 8;
        CHECK(last <= (size_t)M * K, "a load");
      }
    }
    for (int j = 0; j < St::kDW; ++j) {
      const int cq = sfg::rows_w_copy(wv + 8 * j, St::kNW);
      const int tw = sfg::rows_w_tile(cq, CPS), c = sfg::rows_w_chunk(cq, CPS);
      CHECK(tw < St::kTW && c < CPS, "w copy");
      ++wcell[tw * CPS + c];
      for (int t : {0, p.T - 1})
        for (int L : {0, 63}) {
          const size_t e = sfg::weight_lane_ptr((size_t)0, t * St::kTW + tw, K, L) +
                           (size_t)c * sfg::kKsStride +
                           (size_t)(p.S - 1) * CPS * sfg::kKsStride + 8;
          CHECK(e <= (size_t)N * K, "w load");
        }
    }
  }
  for (int v : acell) CHECK(v >= 1, "a cell filled %d times", v);
  for (int v : wcell) CHECK(v >= 1, "w cell filled %d times", v);
  CHECK(p.S * St::kKS == K, "stages cover K");
  // fragment reads inside the stage's words
  for (int wv = 0; wv < 8; ++wv) {
    const int rgrp = wv / St::kCG, cgrp = wv % St::kCG;
    for (int lane = 0; lane < 64; ++lane)
      for (int c = 0; c < CPS; ++c) {
        for (int i = 0; i < 8; ++i) {
          const int w = (c * St::kMT + rgrp * 8 + i) * 64 + sfg::a_read_word(lane);
          CHECK(w >= 0 && w < St::kA, "a read word %d", w);
        }
        for (int tt = 0; tt < WN; ++tt) {
          const int w = St::kA + ((cgrp * WN + tt) * CPS + c) * 64 + lane;
          CHECK(w >= St::kA && w < St::kWords, "w read word %d", w);
        }
      }
  }
  // stores: lane (row rgrp*128 + 16 i + l%16, columns col0 + 16 tt + 4 (l/16) .. +4)
  for (int q = 0; q < G; ++q) {
    const int s = q / p.T, t = q % p.T;
    for (int wv = 0; wv < 8; ++wv) {
      const int rgrp = wv / St::kCG, cgrp = wv % St::kCG;
      for (int lane = 0; lane < 64; ++lane) {
        const int col0 = (t * St::kTW + cgrp * WN) * 16 + (lane >> 4) * 4;
        for (int i = 0; i < 8; ++i) {
          const int row = rgrp * 128 + i * 16 + (lane & 15);
          if (row >= mb) continue;
          for (int tt = 0; tt < WN; ++tt) {
            const size_t o = (size_t)(m0 + row) * N + col0 + tt * 16;
            CHECK(col0 + tt * 16 + 4 <= N && o + 4 <= (size_t)M * N, "store");
            const size_t e = (size_t)s * M * N + o;
            CHECK(e + 4 <= part_elems, "partial store %zu of %zu", e, part_elems);
            for (int k = 0; k < 4; ++k) CHECK(!(*hit)[e + k]++, "element written twice");
          }
        }
      }
    }
  }
  (void)ks;
}

template <int WN>
static void walk_rows(int M, int N, int K, int ks_max, size_t ws_bytes) {
  const int ks = sfg::rows_splits<WN>(M, N, K, ks_max);
  CHECK(ks >= 1 && ks <= ks_max, "ks %d", ks);
  const size_t part_elems = (size_t)ks * M * N;
  if (ks_max > 1) CHECK(ws_bytes >= part_elems * 4, "o_proj workspace %zu < %zu", ws_bytes, part_elems * 4);
  std::vector<unsigned char> hit(part_elems, 0);
  for (int m0 = 0; m0 < M; m0 += 256) {
    const int mb = sf_imin(256, M - m0);
    const int rg = sfg::rows_rg(mb);
    const sfg::RowsPlan p{sfg::rows_tiles<WN>(N, rg), ks, sfg::rows_stages(K)};
    if (rg == 1)
      walk_rows_pass<1, sfg::rows_wn<WN>(1)>(p, M, m0, mb, N, K, ks, part_elems, &hit);
    else
      walk_rows_pass<2, WN>(p, M, m0, mb, N, K, ks, part_elems, &hit);
  }
  for (unsigned char h : hit) CHECK(h == 1, "element not written");
}

static void check_rows_plans() {
  long long n = 0;
  const int dims[] = {1536, 3584, 4096, 5120, 896};
  for (int D : dims)
    for (int M : {1, 39, 128, 129, 256, 300}) {
      walk_rows<1>(M, D, D, 16, f_oproj_ws(M, D, D));
      ++n;
    }
  // lm_head at a reduced vocabulary of the same tile structure (the walk marks
  // every element); the full vocabularies' tile counts
  for (int D : {1536, 3584})
    for (int M : {1, 129, 256}) {
      walk_rows<2>(M, 2048, D, 1, 0);
      ++n;
    }
  for (int V : {151936, 152064, 131072})
    for (int rg : {1, 2}) {
      const int T = sfg::rows_tiles<2>(V, rg);
      CHECK(T * 16 * sfg::rows_wn<2>(rg) * (8 / rg) == V, "lm_head tiles V=%d", V);
    }
  printf("all-rows GEMM: %lld launches walked\n", n);
}

// Output columns and packed-weight addressing of one GEMM mode: N output
// columns in T tiles of 128·WN (SILU: 128), K = 64·S; each of the 8 waves owns
// one column group and takes both 32-K chunks of every stage.
template <int WN, bool SILU>
static void check_columns(int N, int K) {
  const int tw = SILU ? 128 : 128 * WN;
  CHECK(N % tw == 0, "N %% tile");
  const int T = N / tw, S = K / 64;
  const int ntile = SILU ? 1 : WN;
  for (int t = 0; t < T; ++t) {
    std::vector<int> hits(tw, 0);
    for (int wv = 0; wv < 8; ++wv)
      for (int tt = 0; tt < ntile; ++tt)
        for (int lane = 0; lane < 64; ++lane) {
          const int col = sfg::gemm_col<WN, SILU>(t, wv, tt, lane);
          CHECK(col >= t * tw && col < (t + 1) * tw && col < N, "col %d of tile %d", col, t);
          if (lane < 16) ++hits[col - t * tw];
          // the lane's weight stream: chunks weight_chunk(sc, c) of tile col/16
          for (int sc = 0; sc < S; ++sc)
            for (int c = 0; c < 2; ++c) {
              const size_t off = sfg::weight_lane_ptr<size_t>(0, col >> 4, K, lane) +
                                 (size_t)sfg::weight_chunk(sc, c) * sfg::kKsStride;
              CHECK(off + 8 <= (size_t)N * K, "weight load past the end");
              // packed layout: word (tile16 · K/32 + chunk) · 64 + l holds
              // W[16 tile16 + l%16][32 chunk + 8 (l/16) ..+8]
              CHECK(off % 8 == 0, "word alignment");
              const size_t word = off / 8;
              const size_t l = word & 63, tc = word >> 6;
              const size_t tile16 = tc / (K / 32), chunk = tc % (K / 32);
              CHECK(l == (size_t)lane, "a weight fragment is word `lane` of its 1 KB block");
              CHECK(tile16 * 16 + (l & 15) == (size_t)col, "B fragment column");
              CHECK(chunk * 32 + (l >> 4) * 8 == (size_t)sc * 64 + c * 32 + (lane >> 4) * 8,
                    "B fragment k");
            }
        }
    for (int c = 0; c < tw; ++c) CHECK(hits[c] == 1, "column %d of tile %d hit %d times", c, t, hits[c]);
  }
}

// The A operand's LDS tiles: the copies of a stage cover every (chunk, m tile)
// (extra copies only repeat the last), and the MFMA reader of every lane finds
// the A unit its fragment needs.
static void check_a_tiles() {
  for (int NMT : {1, 2, 3, 4, 5, 8, 16}) {
    const int DPW = (2 * NMT + 7) / 8;
    std::vector<int> got(2 * NMT, 0);
    for (int wv = 0; wv < 8; ++wv)
      for (int j = 0; j < DPW; ++j) {
        const int q = sfg::a_copy(wv, j, NMT);
        CHECK(q >= 0 && q < 2 * NMT, "copy %d out of range", q);
        ++got[q];
      }
    for (int q = 0; q < 2 * NMT - 1; ++q) CHECK(got[q] == 1, "tile %d copied %d times", q, got[q]);
    CHECK(got[2 * NMT - 1] >= 1, "last tile never copied");
  }
  // word w of a tile holds unit a_copy_unit(w) of row w/4
  int unit_at[64], row_at[64];
  std::vector<int> seen(64, 0);
  for (int L = 0; L < 64; ++L) {
    unit_at[L] = sfg::a_copy_unit(L);
    row_at[L] = L >> 2;
    ++seen[row_at[L] * 4 + unit_at[L]];
  }
  for (int i = 0; i < 64; ++i) CHECK(seen[i] == 1, "(row, unit) %d stored %d times", i, seen[i]);
  for (int l = 0; l < 64; ++l) {
    const int w = sfg::a_read_word(l);
    CHECK(w >= 0 && w < 64, "read word");
    CHECK(row_at[w] == (l & 15) && unit_at[w] == (l >> 4), "lane %d reads the wrong unit", l);
  }
  // the 8 lanes of each quarter-wave read distinct 16-byte bank groups
  for (int g = 0; g < 8; ++g) {
    int mask = 0;
    for (int l = 8 * g; l < 8 * g + 8; ++l) mask |= 1 << (sfg::a_read_word(l) & 7);
    CHECK(mask == 0xff, "bank groups of lanes %d..%d", 8 * g, 8 * g + 7);
  }
}

static void check_gemm_columns() {
  check_columns<1, false>(4608, 3584);    // QKV, 7B
  check_columns<1, false>(2048, 1536);    // QKV, 1.5B
  check_columns<1, false>(3584, 18944);   // down, 7B
  check_columns<1, false>(5120, 5120);    // o_proj, 14B
  check_columns<2, true>(18944, 3584);    // gate/up, 7B
  check_columns<2, true>(17408, 5120);    // gate/up, 14B
  check_columns<1, false>(1024, 896);     // lm_head-style 128-column tiles
  check_a_tiles();
  printf("gemm columns and weight fragments: ok\n");
}

// ---------------------------------------------------------------------------
// Prefix attention
// ---------------------------------------------------------------------------
// The LDS data path of one staged chunk: the copies (wave w fills rows 16(w&3)..
// of K for w < 4, of V for w >= 4; lane L of copy i writes 16 bytes at row
// 16(w&3) + 4i + L/16, physical unit L%16, reading logical unit k_unit / v_unit),
// then the K fragment reads and the transposing V^T reads of every wave,
// emulated element by element (the transposing read's layout: lane i of a
// 16-lane group gets element i%4 of the 8 bytes lane 4k + i/4 points at, k = 0..3).
static void check_lds_paths() {
  const int R = sfa::kChunk, D = sfa::kHD;
  auto logical = [&](int v, int row, int dim) { return (v ? 100000 : 0) + row * 1000 + dim; };
  std::vector<int> lds(2 * R * D, -1);  // element-granular model of the K then V rows
  for (int w = 0; w < 8; ++w)
    for (int i = 0; i < 4; ++i)
      for (int lane = 0; lane < 64; ++lane) {
        const int jg = w & 3, v = w >= 4;
        const int row = 16 * jg + 4 * i + lane / 16, p = lane & 15;
        const int u = v ? sfa::v_unit(row, p) : sfa::k_unit(row, p);
        CHECK((v ? sfa::v_unit(row, u) : sfa::k_unit(row, u)) == p, "unit map not an involution");
        for (int e = 0; e < 8; ++e) {
          int& cell = lds[(v * R + row) * D + p * 8 + e];
          CHECK(cell == -1, "LDS cell written twice");
          cell = logical(v, row, u * 8 + e);
        }
      }
  for (int c : lds) CHECK(c != -1, "LDS cell never written");
  auto at_byte = [&](int byte) {
    CHECK(byte >= 0 && byte % 2 == 0 && byte < 2 * sfa::kHalfBytes, "LDS byte %d", byte);
    return lds[byte / 2];
  };
  for (int kh = 0; kh < 2; ++kh)
    for (int t = 0; t < 2; ++t) {
      const int rows0 = 32 * kh + 16 * t;  // first key row of the 16-key tile
      for (int ds = 0; ds < 4; ++ds) {
        std::vector<int> units(64);
        for (int lane = 0; lane < 64; ++lane) {
          const int off = sfa::k_frag_off(lane, ds) + rows0 * sfa::kRowBytes;
          CHECK(off % 16 == 0, "K read alignment");
          units[lane] = (off % sfa::kRowBytes) / 16;
          for (int e = 0; e < 8; ++e)
            CHECK(at_byte(off + 2 * e) == logical(0, rows0 + lane % 16, ds * 32 + 8 * (lane / 16) + e),
                  "K fragment (kh=%d t=%d ds=%d lane=%d)", kh, t, ds, lane);
        }
        // 16 lanes of a quarter-wave read 16 distinct 16-byte units: no bank conflict
        for (int g = 0; g < 4; ++g) {
          std::vector<int> seen(16, 0);
          for (int i = 0; i < 16; ++i) ++seen[units[16 * g + i]];
          for (int u = 0; u < 16; ++u) CHECK(seen[u] == 1, "K read conflict");
        }
      }
      for (int dt = 0; dt < 8; ++dt) {
        std::vector<int> off(64);
        for (int lane = 0; lane < 64; ++lane) {
          off[lane] = sfa::v_tr_off(lane, dt) + rows0 * sfa::kRowBytes;
          CHECK(off[lane] % 8 == 0, "V^T read alignment");
        }
        for (int lane = 0; lane < 64; ++lane) {
          const int grp = lane / 16, i = lane % 16;
          for (int k = 0; k < 4; ++k) {
            const int srcl = 16 * grp + 4 * k + i / 4;
            const int got = at_byte(off[srcl] + 2 * (i % 4));
            // MFMA A operand element (dim row i, key 8*grp + k of the 32-key block):
            // key 4*grp + k of the tile
            CHECK(got == logical(1, rows0 + 4 * grp + k, dt * 16 + i),
                  "V^T fragment (kh=%d t=%d dt=%d lane=%d k=%d)", kh, t, dt, lane, k);
          }
        }
        // the 64 lanes' 8-byte pieces: 16 rows x 32 bytes; rows 0-7 of the tile on
        // 8 distinct aligned 32-byte pairs, rows 8-15 on the same 8 pairs
        std::vector<int> pairs(16, 0);
        for (int lane = 0; lane < 64; ++lane) {
          const int b = off[lane] - sfa::kHalfBytes - rows0 * sfa::kRowBytes;
          const int row = b / sfa::kRowBytes;
          if ((lane & 3) == 0) ++pairs[((b % sfa::kRowBytes) / 32) + 8 * (row >= 8)];
        }
        for (int q = 0; q < 16; ++q) CHECK(pairs[q] == 1, "V^T read pair %d used %d times", q, pairs[q]);
      }
    }
  printf("chunk LDS layout, K and V^T operand reads: ok\n");
}

// Copies of chunk ci for prefix length P and page size ps (ps = 0: contiguous).
static void check_chunk_loads(int P, int ps) {
  const int nch = sfa::nchunks_for(P);
  const int last_g0 = sfa::last_group_g0(P);
  const int npages = ps ? (P + ps - 1) / ps : 0;
  std::vector<unsigned char> loaded(P, 0);
  for (int ci = 0; ci < nch; ++ci) {
    for (int j = 0; j < 4; ++j) {
      const int g0 = sfa::chunk_group_g0(ci, j, last_g0);
      CHECK(g0 >= 0 && g0 % 16 == 0 && g0 < P, "group start %d (P=%d)", g0, P);
      if (ps) CHECK(g0 / ps < npages, "page index %d of %d", g0 / ps, npages);
      for (int kr = 0; kr < 16; ++kr) {
        const int kk = sfa::group_key(kr, g0, P);
        const int key = g0 + kk;
        CHECK(kk >= 0 && key < P, "key %d (P=%d)", key, P);
        if (ps) {
          CHECK((g0 & (ps - 1)) + kk < ps, "row %d past page of %d", (g0 & (ps - 1)) + kk, ps);
          CHECK(key / ps == g0 / ps, "group straddles pages");
        }
        // row 16j + kr of the chunk: the key the kernel's mask takes it for
        const int want = ci * sfa::kChunk + 16 * j + kr;
        if (want < P) {
          CHECK(key == want, "row holds key %d, not %d", key, want);
          CHECK(!loaded[key], "key %d loaded twice", key);
          loaded[key] = 1;
        } else {
          CHECK(ci == nch - 1, "masked row outside the last chunk");
        }
      }
    }
  }
  for (int k = 0; k < P; ++k) CHECK(loaded[k], "key %d never loaded (P=%d)", k, P);
}

static void check_page_addressing() {
  long long n = 0;
  for (int P = 1; P <= 2600; ++P)
    for (int ps : {0, 16, 32, 64, 128}) check_chunk_loads(P, ps), ++n;
  unsigned seed = 12345;
  for (int i = 0; i < 60; ++i) {
    seed = seed * 1103515245u + 12345u;
    const int P = 2600 + (int)(seed % (32768 - 2600 + 1));
    for (int ps : {0, 16, 128}) check_chunk_loads(P, ps), ++n;
  }
  for (int ps : {16, 32, 64, 128}) check_chunk_loads(32768, ps), ++n;
  printf("page-group addressing: %lld (P, page size) cases\n", n);
}

// The persistent prefix grid over one shape, and the merge's reads.
static void check_decomposition(int P, int P_cap, int count, int bucket, int G, int Hkv) {
  const int qmax = bucket * G;
  const int nch_cap = sfa::nchunks_for(P_cap);
  const int nr_cap = sfa::ranges_cap(P_cap);
  const int nq = count * G;
  const sfa::PrefixGrid pg = sfa::prefix_grid(P, nq, Hkv);
  const int nr_merge = sfa::merge_ranges(P, nq, Hkv);
  CHECK(pg.nr == nr_merge, "ranges: prefix %d merge %d (P=%d nq=%d Hkv=%d)", pg.nr, nr_merge, P,
        nq, Hkv);
  CHECK(nr_merge <= nr_cap && nr_cap <= sfa::kMaxRanges, "ranges %d > slots %d", nr_merge, nr_cap);
  // the ranges partition the chunks
  int next = 0;
  for (int r = 0; r < pg.nr; ++r) {
    const int c0 = r * pg.cpi;
    const int c1 = pg.nch < c0 + pg.cpi ? pg.nch : c0 + pg.cpi;
    CHECK(c0 == next && c1 > c0, "range %d = [%d, %d)", r, c0, c1);
    next = c1;
  }
  CHECK(next == pg.nch, "ranges end at %d of %d chunks", next, pg.nch);
  // the grid the host launches for the capacity walks every item once
  const int grid = sfa::prefix_launch_grid(qmax, nch_cap, Hkv);
  CHECK(grid >= 8 && grid % 8 == 0 && grid <= 256, "grid %d", grid);
  const int items = pg.n_qt * pg.nr * Hkv;
  std::vector<unsigned char> item_seen(items, 0);
  const size_t nslot = (size_t)nr_cap * qmax * Hkv;
  std::vector<unsigned char> written(nslot, 0);
  size_t n_written = 0;
  for (int b = 0; b < grid; ++b) {
    const int xcd = b & 7, per = grid >> 3;
    const int end = sfa::xcd_begin(items, xcd + 1);
    for (int it = sfa::xcd_begin(items, xcd) + (b >> 3); it < end; it += per) {
      CHECK(it >= 0 && it < items && !item_seen[it], "item %d", it);
      item_seen[it] = 1;
      const sfa::AttnItem a = sfa::attn_item(it, pg.n_qt, pg.nr);
      CHECK(a.qt < pg.n_qt && a.r < pg.nr && a.h < Hkv, "item decode");
      for (int qi = a.qt * sfa::kQT; qi < (a.qt + 1) * sfa::kQT && qi < nq; ++qi) {
        const size_t s = sfa::attn_slot(a.h, a.r, qi, nr_cap, qmax);
        CHECK(s < nslot, "slot %zu >= %zu", s, nslot);
        CHECK(!written[s], "slot written twice");
        written[s] = 1;
        ++n_written;
      }
    }
  }
  for (int it = 0; it < items; ++it) CHECK(item_seen[it], "item %d not walked", it);
  // the merge reads (row m, q-head g, range c) at h·nr_cap·qmax + c·qmax + m·G + g:
  // every read slot was written by the prefix pass, and nothing else was
  size_t reads = 0;
  for (int h = 0; h < Hkv; ++h)
    for (int m = 0; m < count; ++m)
      for (int g = 0; g < G; ++g)
        for (int c = 0; c < nr_merge; ++c) {
          const size_t s = ((size_t)h * nr_cap + c) * qmax + (size_t)m * G + g;
          CHECK(s < nslot && written[s], "merge reads unwritten slot (h=%d m=%d g=%d c=%d)", h, m, g, c);
          ++reads;
        }
  CHECK(reads == n_written, "prefix wrote %zu slots, merge reads %zu", n_written, reads);
  // (acc, then (m, l)) fit the library's workspace for this capacity
  const size_t need = nslot * (sfa::kHD + 2) * sizeof(float);
  CHECK(f_attn_ws(bucket, G * Hkv, P_cap) >= need, "attention workspace");
}

static void check_attention_grid() {
  long long n = 0;
  const int GH[][2] = {{1, 1}, {5, 8}, {7, 4}, {8, 8}, {6, 2}, {4, 8}};
  for (auto gh : GH) {
    const int G = gh[0], Hkv = gh[1];
    for (int bucket : {1, 8, 39, 64, 256}) {
      for (int count : {1, bucket / 2 + 1, bucket}) {
        if (count < 1 || count > bucket) continue;
        for (int P = 1; P <= 1100; P += 37) check_decomposition(P, P, count, bucket, G, Hkv), ++n;
        for (int P : {2047, 2048, 2112, 4096, 8191, 16384, 16448, 32768})
          check_decomposition(P, P, count, bucket, G, Hkv), ++n;
        // device length below the capacity the grid and workspace are sized for
        for (int P : {1, 100, 2049, 9000}) check_decomposition(P, 16448, count, bucket, G, Hkv), ++n;
      }
    }
  }
  // every chunk count with the north-star and the long-context heads
  for (int nch = 1; nch <= sfa::kMaxChunks; ++nch)
    for (int count : {1, 39, 256}) {
      check_decomposition(nch * sfa::kChunk, nch * sfa::kChunk, count, 256, 7, 4), ++n;
      check_decomposition(nch * sfa::kChunk - 5, nch * sfa::kChunk, count, 256, 5, 8), ++n;
    }
  printf("attention grids: %lld shapes\n", n);
}

// Greedy statistics: for every vector count a row can have (V <= kMaxVocab) and
// every minimum slice count M's share of 256 workgroups gives, the slices tile the
// row's vectors exactly, number at most kMaxSlices, and none holds more than
// kMaxSliceVectors vectors (its 16-bit counts and token places fit); V beyond
// kMaxVocab needs more slices than one wave merges.
static void check_logit_slices() {
  long long n = 0;
  const int nmax = sfl::kMaxVocab / 8;
  for (int M : {1, 2, 3, 5, 7, 8, 9, 16, 31, 32, 33, 64, 85, 86, 127, 128, 129, 255, 256, 257,
                512, 1024}) {
    for (int nvec = 1; nvec <= nmax; ++nvec) {
      const int S = sfl::slices_for(M, nvec * 8);
      CHECK(S >= 1 && S <= sfl::kMaxSlices, "slice count");
      CHECK(sfl::slice_begin(0, nvec, S) == 0 && sfl::slice_begin(S, nvec, S) == nvec,
            "slices cover the row");
      int big = 0;
      for (int s = 0; s < S; ++s) {
        const int len = sfl::slice_begin(s + 1, nvec, S) - sfl::slice_begin(s, nvec, S);
        CHECK(len >= 0, "slice order");
        big = len > big ? len : big;
      }
      CHECK(big <= sfl::kMaxSliceVectors, "M %d, %d vectors: a slice of %d", M, nvec, big);
      ++n;
    }
  }
  for (int M : {1, 64, 1024})
    CHECK(sfl::slices_for(M, sfl::kMaxVocab + 8) > sfl::kMaxSlices, "past the vocabulary cap");
  printf("logit slices: %lld shapes\n", n);
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: index_check <libspecfold_amd.so>\n");
    return 2;
  }
  void* lib = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!lib) {
    fprintf(stderr, "dlopen: %s\n", dlerror());
    return 2;
  }
  f_gemm_ws = (ws3_fn)dlsym(lib, "sf_gemm_workspace_bytes");
  f_qkv_ws = (ws3_fn)dlsym(lib, "sf_qkv_workspace_bytes");
  f_attn_ws = (ws3_fn)dlsym(lib, "sf_attn_workspace_bytes");
  f_gu_ws = (ws3_fn)dlsym(lib, "sf_ffn_gate_up_workspace_bytes");
  f_oproj_ws = (ws3_fn)dlsym(lib, "sf_o_proj_workspace_bytes");
  if (!f_gemm_ws || !f_qkv_ws || !f_attn_ws || !f_gu_ws || !f_oproj_ws) {
    fprintf(stderr, "missing workspace queries\n");
    return 2;
  }
  check_plans();
  check_rows_plans();
  check_gemm_columns();
  check_lds_paths();
  check_page_addressing();
  check_attention_grid();
  check_logit_slices();
  printf("OK (%lld checks)\n", g_checks);
  return 0;
}
