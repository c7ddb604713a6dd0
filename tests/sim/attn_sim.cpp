// Runs the attention entry points (kernel source given by KERNEL_SRC, compiled for
// the CPU SIMT simulator) on random inputs and checks O, m and Z against a float64
// restatement of the attention the kernels compute, with scores scaled by `scaling`:
//  * folded = 0: sf_attn_prefix_block.  R random recomputed rows; every q-head of
//    each attends over the P prefix keys (paged, shuffled pages) and its branch's N
//    block keys (gathered through src; causal within the block when asked).
//  * folded = 1: sf_attn_rows over a gate structure (random parents, branch 0 and
//    random draft rows recomputed, src = the nearest recomputing ancestor's
//    branch; R is then ignored): EVERY row (b, n) attends with the query of its
//    source row src[b*N + n]*N + n over the prefix and branch b's own block keys.
//
//   attn_sim P page_size B1 N H Hkv R causal seed [folded]
// Prints the error summary; exits 1 when beyond tolerance.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <cmath>
#include <random>
#include <vector>

#include KERNEL_SRC

static uint16_t bf(float f) { return sim_f_to_bf16(f); }
static double fb(uint16_t b) { return (double)sim_bf16_to_f(b); }

int main(int argc, char** argv) {
  if (argc < 10 || argc > 12) {
    fprintf(stderr, "usage: attn_sim P page_size B1 N H Hkv R causal seed [folded [ramp]]\n");
    return 2;
  }
  const int folded = argc >= 11 ? atoi(argv[10]) : 0;
  // ramp = 1: prefix keys scaled by 1 + 3 p / P, so the scores' maximum climbs along
  // the prefix and the online softmax moves its reference in later chunks too;
  // ramp = 2: the last 40 keys scaled 3x more, so it moves in the last chunk as well
  const int ramp = argc >= 12 ? atoi(argv[11]) : 0;
  const int P = atoi(argv[1]), ps = atoi(argv[2]), B1 = atoi(argv[3]), N = atoi(argv[4]);
  const int H = atoi(argv[5]), Hkv = atoi(argv[6]), causal = atoi(argv[8]);
  int R = atoi(argv[7]);
  const unsigned seed = (unsigned)atoi(argv[9]);
  const int hd = 128, G = H / Hkv, BN = B1 * N, bucket = BN;
  const float scaling = 1.0f / std::sqrt((float)hd);
  std::mt19937 rng(seed);
  std::normal_distribution<float> nd(0.f, 1.f);

  std::vector<uint16_t> q((size_t)BN * H * hd), kv((size_t)BN * 2 * Hkv * hd);
  for (auto& x : q) x = bf(nd(rng));
  for (auto& x : kv) x = bf(nd(rng));
  std::vector<int32_t> rows, src(BN);
  if (!folded) {
    // recomputed rows: R distinct flat rows, ascending
    std::vector<int> all(BN);
    for (int i = 0; i < BN; ++i) all[i] = i;
    std::shuffle(all.begin(), all.end(), rng);
    rows.assign(all.begin(), all.begin() + R);
    std::sort(rows.begin(), rows.end());
    // src: block position j of branch b reads branch src[b*N + j]'s K/V row (<= b)
    for (int b = 0; b < B1; ++b)
      for (int j = 0; j < N; ++j) src[b * N + j] = b == 0 ? 0 : (int)(rng() % (b + 1));
  } else {
    // the gate's structure: parent branches, recompute flags (branch 0 always),
    // f = own branch if recomputed else the parent's, src = f's fixed point
    std::vector<int> par(B1, 0), f(BN);
    for (int b = 1; b < B1; ++b) par[b] = (int)(rng() % b);
    for (int b = 0; b < B1; ++b)
      for (int n = 0; n < N; ++n) {
        const bool rec = b == 0 || (rng() % 10) < 3;
        f[b * N + n] = rec ? b : par[b];
        if (rec) rows.push_back(b * N + n);
      }
    for (int t = 0; t < BN; ++t) {
      int sb = f[t];
      for (int hop = 0; hop < B1; ++hop) sb = f[sb * N + t % N];
      src[t] = sb;
    }
    R = (int)rows.size();
  }
  rows.resize(bucket, BN);  // past the count: BN, as the gate's compaction leaves them
  int32_t count = R, plen = P;

  // prefix: pages of ps keys, [page][Hkv][ps][hd], page table shuffled
  const int npages = std::max(1, (P + ps - 1) / ps);
  const long long head_stride = (long long)ps * hd, page_stride = (long long)Hkv * ps * hd;
  std::vector<uint16_t> pk((size_t)npages * page_stride + 64), pv(pk.size());
  for (auto& x : pk) x = bf(nd(rng));
  for (auto& x : pv) x = bf(nd(rng));
  std::vector<int32_t> table(npages);
  for (int i = 0; i < npages; ++i) table[i] = i;
  std::shuffle(table.begin(), table.end(), rng);
  if (ramp)
    for (int p = 0; p < P; ++p)
      for (int h = 0; h < Hkv; ++h)
        for (int d = 0; d < hd; ++d) {
          uint16_t& x = pk[(size_t)table[p / ps] * page_stride + (size_t)h * head_stride +
                           (size_t)(p % ps) * hd + d];
          x = bf((float)(fb(x) * (1.0 + 3.0 * p / P) * (ramp == 2 && p >= P - 40 ? 3.0 : 1.0)));
        }
  auto pkey = [&](const std::vector<uint16_t>& a, int h, int p, int d) {
    return fb(a[(size_t)table[p / ps] * page_stride + (size_t)h * head_stride + (size_t)(p % ps) * hd + d]);
  };

  std::vector<float> o32((size_t)BN * H * hd, NAN), mt((size_t)BN * H, NAN), zt((size_t)BN * H, NAN);
  std::vector<uint16_t> obf((size_t)BN * H * hd);
  const size_t wsb = sf_attn_workspace_bytes(bucket, H, P);
  std::vector<float> ws_store(wsb / 4 + 128);  // the entry point wants 256-byte alignment
  float* ws_al = reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(ws_store.data()) + 255) &
                                          ~static_cast<uintptr_t>(255));
  const int st =
      folded ? sf_attn_rows(q.data(), kv.data(), pk.data(), pv.data(), table.data(), P, ps,
                            page_stride, head_stride, src.data(), rows.data(), &count, bucket, B1,
                            N, 0, B1, H, Hkv, hd, scaling, &plen, o32.data(), obf.data(), mt.data(),
                            zt.data(), ws_al, wsb, nullptr)
             : sf_attn_prefix_block(q.data(), kv.data(), pk.data(), pv.data(), table.data(), P,
                                    ps, page_stride, head_stride, src.data(), rows.data(), &count,
                                    bucket, B1, N, H, Hkv, hd, scaling, &plen, causal, o32.data(),
                                    obf.data(), mt.data(), zt.data(), ws_al, wsb, nullptr);
  if (st != 0) {
    fprintf(stderr, "attention entry point returned %d\n", st);
    return 1;
  }

  double max_o = 0, err_o = 0, err_m = 0, err_z = 0, ref_o = 0;
  const int kvs = 2 * Hkv * hd;
  // the rows to check: the recomputed ones, or (folded) every row with its query's row
  std::vector<int> out_rows, q_rows;
  for (int m = 0; m < R; ++m) out_rows.push_back(rows[m]), q_rows.push_back(rows[m]);
  if (folded) {
    out_rows.clear(), q_rows.clear();
    for (int t = 0; t < BN; ++t) out_rows.push_back(t), q_rows.push_back(src[t] * N + t % N);
  }
  for (size_t k = 0; k < out_rows.size(); ++k) {
    const int row = out_rows[k], b = row / N, n = row % N, qrow = q_rows[k];
    for (int hq = 0; hq < H; ++hq) {
      const int h = hq / G;
      std::vector<double> s, w;
      std::vector<std::vector<double>> vals;
      for (int p = 0; p < P; ++p) {
        double d = 0;
        for (int e = 0; e < hd; ++e) d += fb(q[((size_t)qrow * H + hq) * hd + e]) * pkey(pk, h, p, e);
        s.push_back(d * scaling);
        std::vector<double> v(hd);
        for (int e = 0; e < hd; ++e) v[e] = pkey(pv, h, p, e);
        vals.push_back(v);
      }
      for (int j = 0; j < N; ++j) {
        if (causal && j > n) continue;
        const size_t kr = (size_t)(src[b * N + j] * N + j) * kvs;
        double d = 0;
        for (int e = 0; e < hd; ++e) d += fb(q[((size_t)qrow * H + hq) * hd + e]) * fb(kv[kr + h * hd + e]);
        s.push_back(d * scaling);
        std::vector<double> v(hd);
        for (int e = 0; e < hd; ++e) v[e] = fb(kv[kr + (Hkv + h) * hd + e]);
        vals.push_back(v);
      }
      const double mx = *std::max_element(s.begin(), s.end());
      double z = 0;
      for (double x : s) z += std::exp(x - mx);
      for (int e = 0; e < hd; ++e) {
        double o = 0;
        for (size_t i = 0; i < s.size(); ++i) o += std::exp(s[i] - mx) * vals[i][e];
        o /= z;
        const double got = o32[((size_t)row * H + hq) * hd + e];
        err_o = std::max(err_o, std::fabs(got - o));
        ref_o = std::max(ref_o, std::fabs(o));
      }
      err_m = std::max(err_m, std::fabs(mt[(size_t)row * H + hq] - mx));
      err_z = std::max(err_z, std::fabs(zt[(size_t)row * H + hq] - z) / z);
      max_o = ref_o;
    }
  }
  printf("P=%d ps=%d B1=%d N=%d H=%d/%d R=%d causal=%d folded=%d: O max abs err %.3g (|O| max "
         "%.3g), m %.3g, Z rel %.3g\n", P, ps, B1, N, H, Hkv, R, causal, folded, err_o, max_o,
         err_m, err_z);
  bool ok = err_o <= 2e-4 * std::max(1.0, max_o) && err_m <= 1e-4 && err_z <= 1e-4 &&
            std::isfinite(err_o) && std::isfinite(err_m) && std::isfinite(err_z);
  // without the optional outputs (fp32 O, m, Z: NULL) the bf16 output is the same
  std::vector<uint16_t> obf2((size_t)BN * H * hd);
  const int st2 =
      folded ? sf_attn_rows(q.data(), kv.data(), pk.data(), pv.data(), table.data(), P, ps,
                            page_stride, head_stride, src.data(), rows.data(), &count, bucket, B1,
                            N, 0, B1, H, Hkv, hd, scaling, &plen, nullptr, obf2.data(), nullptr,
                            nullptr, ws_al, wsb, nullptr)
             : sf_attn_prefix_block(q.data(), kv.data(), pk.data(), pv.data(), table.data(), P,
                                    ps, page_stride, head_stride, src.data(), rows.data(), &count,
                                    bucket, B1, N, H, Hkv, hd, scaling, &plen, causal, nullptr,
                                    obf2.data(), nullptr, nullptr, ws_al, wsb, nullptr);
  bool same = st2 == 0;
  for (size_t k = 0; k < out_rows.size() && same; ++k)
    for (int e = 0; e < H * hd; ++e)
      same &= obf2[(size_t)out_rows[k] * H * hd + e] == obf[(size_t)out_rows[k] * H * hd + e];
  printf("  without fp32 O / m / Z: bf16 output %s\n", same ? "identical" : "DIFFERENT");
  ok &= same;
  if (!ok) printf("FAIL\n");
  return ok ? 0 : 1;
}
