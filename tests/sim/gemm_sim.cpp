// Runs the weight-streaming GEMM entry points (kernel sources compiled for the
// CPU SIMT simulator in separate objects) on random bf16 inputs and checks them
// against float64 dot products rounded as each epilogue specifies:
//   sf_pack_weight      the packed layout word (t, c, l) = W[16t + l%16][32c + 8(l/16) .. +8]
//   sf_ffn_gate_up      act[m] = bf16(bf16(silu(bf16 g)) * bf16 u), m < count (stream-K, fix-up)
//   sf_ffn_down_scatter ffn[rows[m]] = bf16(act[m] . Wd^T), m < count (stream-K, fix-up);
//                       rows not in `rows` stay untouched
//   sf_o_proj_residual  hp[r] = bf16(x[r] + bf16(o[r] . Wo^T)), r < M (static M; all-rows
//                       GEMM, K ranges through fp32 partial slots)
//   sf_o_proj_post_norm the same hp, and zn[slot[r]] = bf16(w * bf16(hp[r] * rstd)) for
//                       the rows with slot[r] >= 0
//   sf_lm_head          logits[m] = bf16(x[m] . W^T), m < M
//   sf_head_logits      the same, shifted: row (b, n) of each block to (b, n + 1),
//                       (b, 0) kept, bit for bit the unshifted rows
//   sf_qkv_rope         q / k / v of the recomputed rows: bias, RoPE from absolute
//                       position tables, the optional q scale, scatter by flat row
// A result may differ from the rounded float64 value where the fp32 sum (another
// summation order) lies next to a rounding boundary, or where the sum cancels:
// the check allows two bf16 steps plus 1e-6 of the sum of the terms' magnitudes
// (plus one step of bf16(y) where a rounded product feeds a residual sum), on at
// most 2% of the outputs; everything else must match exactly.
//
//   gemm_sim D I count bucket M seed
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <cmath>
#include <random>
#include <vector>

#include "sf_common.h"

static uint16_t bf(double f) { return sim_f_to_bf16((float)f); }
static double fb(uint16_t b) { return (double)sim_bf16_to_f(b); }

struct Checker {
  const char* name;
  long n = 0, near = 0, bad = 0;
  // want: the float64 value before the final bf16 rounding; mag: sum of |terms|
  void add(uint16_t got, double want, double mag, double extra = 0) {
    const uint16_t w = bf(want);
    ++n;
    if (got == w) return;
    const double ulp = std::ldexp(1.0, std::ilogb(std::fabs(fb(w)) + 1e-30) - 7);
    if (std::fabs(fb(got) - want) <= 2 * ulp + 1e-6 * mag + extra) {
      ++near;
      return;
    }
    if (++bad <= 5) fprintf(stderr, "%s: got %g want %g (mag %g)\n", name, fb(got), want, mag);
  }
  bool report() {
    printf("  %-22s %7ld outputs: %ld within rounding, %ld wrong\n", name, n, near, bad);
    return bad == 0 && near * 50 <= n;
  }
};

static std::vector<uint16_t> pack(const std::vector<uint16_t>& w, int N, int K) {
  std::vector<uint16_t> out((size_t)N * K);
  if (const int st = sf_pack_weight(w.data(), N, K, out.data(), nullptr)) {
    fprintf(stderr, "sf_pack_weight(N=%d, K=%d) returned %d\n", N, K, st);
    exit(1);
  }
  return out;
}

int main(int argc, char** argv) {
  if (argc != 7) {
    fprintf(stderr, "usage: gemm_sim D I count bucket M seed\n");
    return 2;
  }
  const int D = atoi(argv[1]), I = atoi(argv[2]), count = atoi(argv[3]), bucket = atoi(argv[4]);
  const int M = atoi(argv[5]);
  std::mt19937 rng((unsigned)atoi(argv[6]));
  std::normal_distribution<float> nd(0.f, 1.f);
  auto rnd = [&](size_t n, float sd) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = bf(sd * nd(rng));
    return v;
  };
  bool ok = true;

  // ---- packing ----------------------------------------------------------------------
  {
    const int N = 64, K = 256;
    auto w = rnd((size_t)N * K, 1.f);
    auto p = pack(w, N, K);
    long bad = 0;
    for (int t = 0; t < N / 16; ++t)
      for (int c = 0; c < K / 32; ++c)
        for (int l = 0; l < 64; ++l)
          for (int e = 0; e < 8; ++e)
            bad += p[(((size_t)t * (K / 32) + c) * 64 + l) * 8 + e] !=
                   w[(size_t)(16 * t + l % 16) * K + 32 * c + 8 * (l / 16) + e];
    printf("  %-22s %s\n", "pack layout", bad ? "WRONG" : "exact");
    ok &= bad == 0;
  }

  // ---- gate/up and down over the recomputed rows ----------------------------------------
  {
    auto zn = rnd((size_t)bucket * D, 1.f);
    auto wg = rnd((size_t)I * D, 0.05f), wu = rnd((size_t)I * D, 0.05f);
    auto wd = rnd((size_t)D * I, 0.05f);
    const auto pg = pack(wg, I, D), pu = pack(wu, I, D), pd = pack(wd, D, I);
    std::vector<uint16_t> act((size_t)bucket * I, 0x7fc0);
    int32_t cnt = count;
    std::vector<float> gws(sf_ffn_gate_up_workspace_bytes(bucket, D, I) / 4 + 16);
    if (sf_ffn_gate_up(zn.data(), &cnt, bucket, pg.data(), pu.data(), D, I, act.data(), gws.data(),
                       gws.size() * 4, nullptr)) {
      fprintf(stderr, "sf_ffn_gate_up failed\n");
      return 1;
    }
    Checker cg{"ffn gate/up"};
    for (int m = 0; m < count; ++m)
      for (int c = 0; c < I; ++c) {
        double g = 0, u = 0, mg = 0, mu = 0;
        for (int k = 0; k < D; ++k) {
          g += fb(zn[(size_t)m * D + k]) * fb(wg[(size_t)c * D + k]);
          u += fb(zn[(size_t)m * D + k]) * fb(wu[(size_t)c * D + k]);
          mg += std::fabs(fb(zn[(size_t)m * D + k]) * fb(wg[(size_t)c * D + k]));
          mu += std::fabs(fb(zn[(size_t)m * D + k]) * fb(wu[(size_t)c * D + k]));
        }
        const double gt = fb(bf(g));
        const double s = fb(bf((float)gt / (1.0f + expf(-(float)gt))));
        // a one-step flip of bf16(g) or bf16(u) (their fp32 sums next to a rounding
        // boundary) carries through silu and the product
        const double sig = 1.0 / (1.0 + std::exp(-gt));
        const double dsilu = std::fabs(sig * (1.0 + gt * (1.0 - sig)));
        const double ug = std::ldexp(1.0, std::ilogb(std::fabs(gt) + 1e-30) - 7);
        const double uu = std::ldexp(1.0, std::ilogb(std::fabs(u) + 1e-30) - 7);
        const double flip = dsilu * ug * std::fabs(u) + std::fabs(s) * uu;
        cg.add(act[(size_t)m * I + c], (double)(float)(s * fb(bf(u))), mg + mu, flip);
      }
    ok &= cg.report();

    // down: rows[m] = a permutation of flat rows; act rows as computed above
    const int BN = bucket + 7;
    std::vector<int32_t> rows(bucket);
    {  // distinct destination rows in a scrambled order
      std::vector<int32_t> perm(BN);
      for (int i = 0; i < BN; ++i) perm[i] = i;
      std::shuffle(perm.begin(), perm.end(), rng);
      for (int m = 0; m < bucket; ++m) rows[m] = perm[m];
    }
    std::vector<uint16_t> ffn((size_t)BN * D, 0x1234);
    auto act_in = rnd((size_t)bucket * I, 1.f);
    std::vector<float> ws(sf_gemm_workspace_bytes(bucket, D, I) / 4 + 16);
    if (sf_ffn_down_scatter(act_in.data(), &cnt, bucket, rows.data(), pd.data(), I, D, ffn.data(),
                            ws.data(), ws.size() * 4, nullptr)) {
      fprintf(stderr, "sf_ffn_down_scatter failed\n");
      return 1;
    }
    Checker cd{"ffn down + scatter"};
    std::vector<char> written(BN, 0);
    for (int m = 0; m < count; ++m) {
      written[rows[m]] = 1;
      for (int c = 0; c < D; ++c) {
        double y = 0, mag = 0;
        for (int k = 0; k < I; ++k) {
          y += fb(act_in[(size_t)m * I + k]) * fb(wd[(size_t)c * I + k]);
          mag += std::fabs(fb(act_in[(size_t)m * I + k]) * fb(wd[(size_t)c * I + k]));
        }
        cd.add(ffn[(size_t)rows[m] * D + c], y, mag);
      }
    }
    long touched = 0;
    for (int r = 0; r < BN; ++r)
      if (!written[r])
        for (int c = 0; c < D; ++c) touched += ffn[(size_t)r * D + c] != 0x1234;
    printf("  %-22s %s\n", "down: other rows", touched ? "OVERWRITTEN" : "untouched");
    ok &= cd.report() && touched == 0;
    // the shared tiles' arrival counters are left zero: a second call on the same
    // workspace writes the same rows again, bit for bit
    std::vector<uint16_t> ffn2((size_t)BN * D, 0x1234);
    if (sf_ffn_down_scatter(act_in.data(), &cnt, bucket, rows.data(), pd.data(), I, D, ffn2.data(),
                            ws.data(), ws.size() * 4, nullptr)) {
      fprintf(stderr, "sf_ffn_down_scatter failed\n");
      return 1;
    }
    const bool same = ffn2 == ffn;
    printf("  %-22s %s\n", "down: repeat call", same ? "identical" : "DIFFERENT");
    ok &= same;
  }

  // ---- o_proj + residual and lm_head over M static rows -----------------------------------
  {
    auto o = rnd((size_t)M * D, 1.f), x = rnd((size_t)M * D, 1.f);
    auto wo = rnd((size_t)D * D, 0.05f);
    const auto po = pack(wo, D, D);
    std::vector<uint16_t> hp((size_t)M * D);
    std::vector<float> ws(sf_o_proj_workspace_bytes(M, D, D) / 4 + 16);
    if (sf_o_proj_residual(o.data(), x.data(), po.data(), M, D, D, hp.data(), ws.data(),
                           ws.size() * 4, nullptr)) {
      fprintf(stderr, "sf_o_proj_residual failed\n");
      return 1;
    }
    std::vector<double> yref((size_t)M * D), ymag((size_t)M * D);
    for (int r = 0; r < M; ++r)
      for (int c = 0; c < D; ++c) {
        double y = 0, mag = 0;
        for (int k = 0; k < D; ++k) {
          y += fb(o[(size_t)r * D + k]) * fb(wo[(size_t)c * D + k]);
          mag += std::fabs(fb(o[(size_t)r * D + k]) * fb(wo[(size_t)c * D + k]));
        }
        yref[(size_t)r * D + c] = y;
        ymag[(size_t)r * D + c] = mag;
      }
    auto check_hp = [&](const char* name, const std::vector<uint16_t>& h) {
      Checker co{name};
      for (int r = 0; r < M; ++r)
        for (int c = 0; c < D; ++c) {
          const double y = yref[(size_t)r * D + c];
          // a one-step flip of bf16(y) carries through the residual sum
          const double uy = std::ldexp(1.0, std::ilogb(std::fabs(y) + 1e-30) - 7);
          co.add(h[(size_t)r * D + c], (double)(float)(fb(x[(size_t)r * D + c]) + fb(bf(y))),
                 ymag[(size_t)r * D + c], uy);
        }
      return co.report();
    };
    ok &= check_hp("o_proj + residual", hp);
    printf("  o_proj K ranges: %zu\n", sf_o_proj_workspace_bytes(M, D, D) / (4 * (size_t)M * D));

    // o_proj + residual + post-attention RMSNorm of the recomputed rows (slot >= 0);
    // the norm is checked on the kernel's own hp
    {
      std::vector<int32_t> slot(M);
      int ns = 0;
      for (int r = 0; r < M; ++r) slot[r] = (rng() % 3 == 0) ? -1 : ns++;
      auto lw = rnd(D, 1.f);
      const float eps = 1e-6f;
      std::vector<uint16_t> hp2((size_t)M * D), zn((size_t)std::max(ns, 1) * D, 0x1234);
      if (sf_o_proj_post_norm(o.data(), x.data(), po.data(), M, D, D, slot.data(), lw.data(), eps,
                              hp2.data(), zn.data(), ws.data(), ws.size() * 4, nullptr)) {
        fprintf(stderr, "sf_o_proj_post_norm failed\n");
        return 1;
      }
      ok &= check_hp("o_proj + post norm: hp", hp2);
      const bool same = hp2 == hp;
      printf("  %-22s %s\n", "hp of both entries", same ? "identical" : "DIFFER");
      ok &= same;
      Checker cz{"o_proj + post norm: zn"};
      for (int r = 0; r < M; ++r) {
        if (slot[r] < 0) continue;
        float ss = 0.f;
        for (int c = 0; c < D; ++c) ss += fb(hp2[(size_t)r * D + c]) * fb(hp2[(size_t)r * D + c]);
        const float inv = 1.0f / std::sqrt(ss / (float)D + eps);
        for (int c = 0; c < D; ++c) {
          const double t = fb(bf((double)((float)fb(hp2[(size_t)r * D + c]) * inv)));
          const double ut = std::ldexp(1.0, std::ilogb(std::fabs(t) + 1e-30) - 7);
          cz.add(zn[(size_t)slot[r] * D + c], fb(lw[c]) * t, 0, std::fabs(fb(lw[c])) * ut);
        }
      }
      ok &= cz.report();
    }

    const int V = 384;
    auto wl = rnd((size_t)V * D, 0.05f);
    const auto pl = pack(wl, V, D);
    std::vector<uint16_t> logits((size_t)M * V);
    if (sf_lm_head(x.data(), M, pl.data(), D, V, logits.data(), nullptr)) {
      fprintf(stderr, "sf_lm_head failed\n");
      return 1;
    }
    Checker cl{"lm_head"};
    for (int m = 0; m < M; ++m)
      for (int v = 0; v < V; ++v) {
        double y = 0, mag = 0;
        for (int k = 0; k < D; ++k) {
          y += fb(x[(size_t)m * D + k]) * fb(wl[(size_t)v * D + k]);
          mag += std::fabs(fb(x[(size_t)m * D + k]) * fb(wl[(size_t)v * D + k]));
        }
        cl.add(logits[(size_t)m * V + v], y, mag);
      }
    ok &= cl.report();

    // the same head with Fast-dLLM's shift in the stores (sf_head_logits): blocks of
    // sn rows, output row (b, n + 1) = row (b, n) of the unshifted logits bit for
    // bit, row (b, 0) kept; into rows of stride V + 8 whose padding stays untouched
    int sn = 0;
    for (int c : {32, 16, 10, 8, 5, 4, 2})
      if (M % c == 0) {
        sn = c;
        break;
      }
    if (sn) {
      const int ld = V + 8;
      std::vector<uint16_t> sh((size_t)M * ld, 0xBEEF);
      if (sf_head_logits(x.data(), M, pl.data(), D, V, sn, sh.data(), ld, nullptr)) {
        fprintf(stderr, "sf_head_logits failed\n");
        return 1;
      }
      long bad = 0;
      for (int m = 0; m < M; ++m) {
        const int n = m % sn;
        const int srow = n == 0 ? m : m - 1;
        for (int v = 0; v < ld; ++v) {
          const uint16_t want = v < V ? logits[(size_t)srow * V + v] : 0xBEEF;
          bad += sh[(size_t)m * ld + v] != want;
        }
      }
      printf("  %-22s %7ld outputs: %ld wrong (blocks of %d rows)\n", "head_logits shifted",
             (long)M * ld, bad, sn);
      ok &= bad == 0;
    }
  }
  // ---- QKV projection + bias + RoPE (+ q scale) + scatter ----------------------------------
  // the reference's op sequence (fastdllm_v2_folded.py:151-161, nld_folded.py:173-174):
  // y = bf16(x . W^T + b); rope: bf16(bf16(y * cos) + bf16(rotate_half(y) * sin)) for q
  // and k heads, rotate_half(y)[d] = -y[d + 64] (d < 64), y[d - 64] (d >= 64); then
  // for q heads bf16(q * bf16(q_scale[n])); written to row `row` of q_buf / kv_buf
  for (int with_scale = 0; with_scale < 2; ++with_scale) {
    const int H = 4, Hkv = 2, hd = 128, N = 16, nq = (H + 2 * Hkv) * hd;
    const int BNq = std::max(bucket, count) + 5;
    auto xn = rnd((size_t)BNq * D, 1.f);
    auto w = rnd((size_t)nq * D, 0.05f), bias = rnd(nq, 0.5f);
    const auto pw = pack(w, nq, D);
    const int table_rows = 300;
    std::vector<uint16_t> cs((size_t)table_rows * hd), sn((size_t)table_rows * hd);
    for (int t = 0; t < table_rows; ++t)
      for (int d = 0; d < hd; ++d) {
        const double ang = t / std::pow(10000.0, (2.0 * (d % 64)) / hd);
        cs[(size_t)t * hd + d] = bf(std::cos(ang));
        sn[(size_t)t * hd + d] = bf(std::sin(ang));
      }
    std::vector<int32_t> rows(bucket);
    {
      std::vector<int32_t> perm(BNq);
      for (int i = 0; i < BNq; ++i) perm[i] = i;
      std::shuffle(perm.begin(), perm.end(), rng);
      std::sort(perm.begin(), perm.begin() + count);
      for (int m = 0; m < bucket; ++m) rows[m] = m < count ? perm[m] : BNq;
    }
    std::vector<float> qs(N);
    for (int n = 0; n < N; ++n) qs[n] = 1.0f + 0.03f * n;
    int32_t cnt = count, pos0 = 117;
    std::vector<uint16_t> qb((size_t)(BNq + 1) * H * hd, 0x1234), kvb((size_t)(BNq + 1) * 2 * Hkv * hd, 0x1234);
    std::vector<float> ws(sf_qkv_workspace_bytes(bucket, D, nq) / 4 + 16);
    const int st = sf_qkv_rope(xn.data(), rows.data(), &cnt, bucket, BNq, pw.data(), bias.data(),
                               cs.data(), sn.data(), &pos0, table_rows,
                               with_scale ? qs.data() : nullptr, N, D, H, Hkv, hd, qb.data(),
                               kvb.data(), ws.data(), ws.size() * 4, nullptr);
    if (st) {
      fprintf(stderr, "sf_qkv_rope returned %d\n", st);
      return 1;
    }
    Checker cq{with_scale ? "qkv + rope + q scale" : "qkv + rope"};
    std::vector<char> written(BNq + 1, 0);
    for (int m = 0; m < count; ++m) {
      const int row = rows[m], n = row % N, tr = std::min(pos0 + n, table_rows - 1);
      written[row] = 1;
      std::vector<double> y(nq), mag(nq);
      for (int c = 0; c < nq; ++c) {
        double a = 0, g = 0;
        for (int k = 0; k < D; ++k) {
          a += fb(xn[(size_t)row * D + k]) * fb(w[(size_t)c * D + k]);
          g += std::fabs(fb(xn[(size_t)row * D + k]) * fb(w[(size_t)c * D + k]));
        }
        y[c] = a + fb(bias[c]);
        mag[c] = g;
      }
      for (int hh = 0; hh < H + 2 * Hkv; ++hh)
        for (int d = 0; d < hd; ++d) {
          const int c = hh * hd + d;
          const double yb = fb(bf(y[c]));
          double out = yb;
          double slack = 0;
          if (hh < H + Hkv) {
            const double rot = d < 64 ? -fb(bf(y[c + 64])) : fb(bf(y[c - 64]));
            const double a1 = fb(bf((float)(yb * fb(cs[(size_t)tr * hd + d]))));
            const double a2 = fb(bf((float)(rot * fb(sn[(size_t)tr * hd + d]))));
            out = (double)(float)(a1 + a2);
            // a one-step flip of either rounded input carries through the rope sum
            slack = std::ldexp(1.0, std::ilogb(std::fabs(a1) + 1e-30) - 7) +
                    std::ldexp(1.0, std::ilogb(std::fabs(a2) + 1e-30) - 7);
            if (hh < H && with_scale) {
              const double q = fb(bf(out));
              out = (double)(float)(q * fb(bf(qs[n])));
              slack *= 2;
            }
          }
          const uint16_t got = hh < H ? qb[((size_t)row * H + hh) * hd + d]
                                      : kvb[((size_t)row * 2 * Hkv + (hh - H)) * hd + d];
          cq.add(got, out, mag[c], slack);
        }
    }
    long touched = 0;
    for (int r = 0; r <= BNq; ++r)
      if (!written[r]) {
        for (int e = 0; e < H * hd; ++e) touched += qb[(size_t)r * H * hd + e] != 0x1234;
        for (int e = 0; e < 2 * Hkv * hd; ++e) touched += kvb[(size_t)r * 2 * Hkv * hd + e] != 0x1234;
      }
    printf("  %-22s %s\n", "qkv: other rows", touched ? "OVERWRITTEN" : "untouched");
    ok &= cq.report() && touched == 0;
  }
  printf("D=%d I=%d count=%d bucket=%d M=%d: %s\n", D, I, count, bucket, M, ok ? "OK" : "FAIL");
  return ok ? 0 : 1;
}
