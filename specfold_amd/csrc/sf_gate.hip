// Fold gate: per-row relative-residual test, deterministic compaction of the
// recomputed rows, src resolution and the input RMSNorm of recomputed rows.
//
// Reference semantics: specfold/generate/fastdllm_v2_folded.py:136-152
// (gate against the subset-parent, RMSNorm of recomputed rows) and the Triton
// gate/src kernels specfold/generate/triton_kernels.py:18-26, 199-239.
// Unlike the Triton gate (atomic slot order), rows[] is in ascending flat-row
// order, which equals the concatenation of the reference's per-branch
// nonzero() lists.
#include "sf_common.h"
#include "sf_compact.h"

namespace {

constexpr int kGateWaves = 1;  // one wave per flat row and workgroup (the rows spread over
                                // the CUs: 5.4-5.8 against 6.5-6.7 us with 4 rows per workgroup)
constexpr int kMaxVecPerLane = 16;  // 16 x 8 bf16 x 64 lanes = 8192 columns

// One wave per flat row r = b*N + n: three fp32 sums over D (x^2, residual^2,
// parent^2), the gate decision, rstd, and the normalized row for recomputed rows.
// RESID: the layer input is first formed from the previous layer's outputs,
// x[r] = bf16(hp[r] + ffn[src_prev[r]*N + n]) (the folded residual update of
// fastdllm_v2_folded.py:218), for the row and for its parent row, and x[r] is
// written to hidden_out.  `par` may be NULL (every row its own parent).
template <int VPL, bool RESID, bool ROOTS>
__global__ __launch_bounds__(kGateWaves * 64) void sf_gate_rows_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ ffn,
    const int32_t* __restrict__ src_prev, const int32_t* __restrict__ par,
    const uint16_t* __restrict__ ln_w, int B1, int N, int D, float delta, float eps, int mode,
    uint16_t* __restrict__ hidden_out, int8_t* __restrict__ rec, float* __restrict__ rstd,
    uint16_t* __restrict__ xn) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * kGateWaves + (threadIdx.x >> 6);
  const int BN = B1 * N;
  if (r >= BN) return;
  const int b = r / N;
  const int n = r - b * N;
  // Two rounds of loads.  (1) The parent, every branch's source at position n
  // (lane l: branch l; B1 <= 64), the row and the norm weights; (2) the parent row
  // and the FFN rows of the row's and the parent's sources, whose ids come from
  // round 1 by shuffles instead of a further round through memory.  Addresses are
  // clamped and nothing branches, so each round costs one memory latency.
  int p = par ? par[b] : b;
  const int src_n = RESID ? src_prev[min(lane, B1 - 1) * N + n] : 0;
  const int nvec = D >> 3;
  const sf_u32x4* xrow = reinterpret_cast<const sf_u32x4*>(hidden + (size_t)r * D);
  const sf_u32x4* wrow = reinterpret_cast<const sf_u32x4*>(ln_w);
  sf_u32x4 xv[VPL], pv[VPL], wv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) xv[i] = xrow[min(lane + i * 64, nvec - 1)];
#pragma unroll
  for (int i = 0; i < VPL; ++i) wv[i] = wrow[min(lane + i * 64, nvec - 1)];
  p = p < 0 ? 0 : (p >= B1 ? B1 - 1 : p);
  // a draft row is gated against its parent's; the root branch (branch 0, or with
  // ROOTS every branch that is its own parent: the main branch of each sequence
  // of a batched step) is always recomputed
  const bool draft = (ROOTS ? p != b : b > 0) && mode != SF_GATE_ALL;
  const int pr = p * N + n;
  const sf_u32x4* prow = reinterpret_cast<const sf_u32x4*>(hidden + (size_t)pr * D);
  sf_u32x4 fx[RESID ? VPL : 1], fp[RESID ? VPL : 1];
  if (RESID) {
    // src_prev[b*N + n] and src_prev[p*N + n]
    const int s_r = __shfl(src_n, b, 64);
    const int s_p = __shfl(src_n, p, 64);
    const sf_u32x4* fxrow = reinterpret_cast<const sf_u32x4*>(ffn + (size_t)(s_r * N + n) * D);
    const sf_u32x4* fprow = reinterpret_cast<const sf_u32x4*>(ffn + (size_t)(s_p * N + n) * D);
#pragma unroll
    for (int i = 0; i < VPL; ++i) fx[i] = fxrow[min(lane + i * 64, nvec - 1)];
#pragma unroll
    for (int i = 0; i < VPL; ++i) fp[i] = fprow[min(lane + i * 64, nvec - 1)];
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) pv[i] = prow[min(lane + i * 64, nvec - 1)];
  if (RESID) {
    // h = bf16(hp + ffn), the layer input, kept as packed bf16
    sf_u32x4* hout = reinterpret_cast<sf_u32x4*>(hidden_out + (size_t)r * D);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float a[8], c[8], e[8], g[8];
      sf_unpack8(xv[i], a);
      sf_unpack8(fx[i], c);
      sf_unpack8(pv[i], e);
      sf_unpack8(fp[i], g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[i][j] = sf_pack2(a[2 * j] + c[2 * j], a[2 * j + 1] + c[2 * j + 1]);
        pv[i][j] = sf_pack2(e[2 * j] + g[2 * j], e[2 * j + 1] + g[2 * j + 1]);
      }
      if (lane + i * 64 < nvec) sf_handoff_store(&hout[lane + i * 64], xv[i]);
    }
  }

  float ss = 0.f, ds = 0.f, ps = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (lane + i * 64 >= nvec) continue;
    float xf[8], pf[8];
    sf_unpack8(xv[i], xf);
    sf_unpack8(pv[i], pf);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss = fmaf(xf[j], xf[j], ss);
      float d = xf[j] - pf[j];
      if (mode == SF_GATE_MODEL_DTYPE) d = sf_rbf(d);  // x - x_par is a bf16 tensor op
      ds = fmaf(d, d, ds);
      ps = fmaf(pf[j], pf[j], ps);
    }
  }
  ss = sf_wave_sum(ss);
  ds = sf_wave_sum(ds);
  ps = sf_wave_sum(ps);

  // Qwen2RMSNorm: x * rsqrt(mean(x^2) + eps) in fp32 (torch CPU rsqrt is 1/sqrt).
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  bool is_rec = true;
  if (draft) {
    if (mode == SF_GATE_MODEL_DTYPE) {
      // bf16 norms: dn = bf16(|x - xp|), thr = bf16(delta * bf16(|xp|)), dn > thr.
      const float dn = sf_rbf(sqrtf(ds));
      const float pn = sf_rbf(sqrtf(ps));
      const float thr = sf_rbf(delta * pn);
      is_rec = dn > thr;
    } else {
      is_rec = ds > (delta * delta) * ps;
    }
  }
  if (lane == 0) {
    if (rec) rec[r] = is_rec ? 1 : 0;
    if (rstd) rstd[r] = inv;
  }
  if (!is_rec) return;

  // normalized row: bf16(w * bf16(x * rstd)), as Qwen2RMSNorm in bf16.
  sf_u32x4* out = reinterpret_cast<sf_u32x4*>(xn + (size_t)r * D);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = lane + i * 64;
    if (idx < nvec) {
      float xf[8], wf[8];
      sf_unpack8(xv[i], xf);
      sf_unpack8(wv[i], wf);
      sf_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = sf_rbf(wf[2 * j] * sf_rbf(xf[2 * j] * inv));
        const float c = sf_rbf(wf[2 * j + 1] * sf_rbf(xf[2 * j + 1] * inv));
        o[j] = sf_pack2(a, c);
      }
      sf_handoff_store(&out[idx], o);
    }
  }
}

// One workgroup of 1024 threads, thread t = flat row t (gate_compact, sf_compact.h).
__global__ __launch_bounds__(1024) void sf_gate_compact_kernel(
    const int8_t* __restrict__ rec, const int32_t* __restrict__ par, int B1, int N, int bucket,
    int32_t* __restrict__ f, int32_t* __restrict__ src, int32_t* __restrict__ rows,
    int32_t* __restrict__ count, int32_t* __restrict__ seg, int32_t* __restrict__ segcnt,
    int32_t* __restrict__ slot_out) {
  __shared__ int s_f[1024];
  __shared__ int s_slot[1024];
  __shared__ int s_tot[16];
  const GateOut out{f, src, rows, count, seg, segcnt, slot_out};
  gate_compact<1024, 1>(rec, par, B1, N, bucket, s_f, s_slot, s_tot, nullptr, true, out);
}

template <int VPL, bool RESID, bool ROOTS>
void launch_rows(const uint16_t* hidden, const uint16_t* ffn, const int32_t* src_prev,
                 const int32_t* par, const uint16_t* ln_w, int B1, int N, int D, float delta,
                 float eps, int mode, uint16_t* hidden_out, int8_t* rec, float* rstd,
                 uint16_t* xn, hipStream_t st) {
  const int BN = B1 * N;
  dim3 grid((BN + kGateWaves - 1) / kGateWaves);
  hipLaunchKernelGGL((sf_gate_rows_kernel<VPL, RESID, ROOTS>), grid, dim3(kGateWaves * 64), 0, st,
                     hidden, ffn, src_prev, par, ln_w, B1, N, D, delta, eps, mode, hidden_out, rec,
                     rstd, xn);
}

template <bool RESID, bool ROOTS>
void launch_rows_any(int D, const uint16_t* hidden, const uint16_t* ffn, const int32_t* src_prev,
                     const int32_t* par, const uint16_t* ln_w, int B1, int N, float delta,
                     float eps, int mode, uint16_t* hidden_out, int8_t* rec, float* rstd,
                     uint16_t* xn, hipStream_t st) {
  const int vpl = (D / 8 + 63) / 64;
  if (vpl <= 4)
    launch_rows<4, RESID, ROOTS>(hidden, ffn, src_prev, par, ln_w, B1, N, D, delta, eps, mode,
                                 hidden_out, rec, rstd, xn, st);
  else if (vpl <= 8)
    launch_rows<8, RESID, ROOTS>(hidden, ffn, src_prev, par, ln_w, B1, N, D, delta, eps, mode,
                                 hidden_out, rec, rstd, xn, st);
  else if (vpl <= 12)
    launch_rows<12, RESID, ROOTS>(hidden, ffn, src_prev, par, ln_w, B1, N, D, delta, eps, mode,
                                  hidden_out, rec, rstd, xn, st);
  else
    launch_rows<16, RESID, ROOTS>(hidden, ffn, src_prev, par, ln_w, B1, N, D, delta, eps, mode,
                                  hidden_out, rec, rstd, xn, st);
}

template <bool RESID>
void launch_rows_mode(int D, const uint16_t* hidden, const uint16_t* ffn, const int32_t* src_prev,
                      const int32_t* par, const uint16_t* ln_w, int B1, int N, float delta,
                      float eps, int gate_mode, uint16_t* hidden_out, int8_t* rec, float* rstd,
                      uint16_t* xn, hipStream_t st) {
  const int mode = gate_mode & ~(SF_GATE_ROOTS_BY_PARENT | SF_GATE_DEFER_COMPACT);
  if (gate_mode & SF_GATE_ROOTS_BY_PARENT)
    launch_rows_any<RESID, true>(D, hidden, ffn, src_prev, par, ln_w, B1, N, delta, eps, mode,
                                 hidden_out, rec, rstd, xn, st);
  else
    launch_rows_any<RESID, false>(D, hidden, ffn, src_prev, par, ln_w, B1, N, delta, eps, mode,
                                  hidden_out, rec, rstd, xn, st);
}

int check_gate_args(int B1, int N, int D, int bucket, int gate_mode) {
  const int mode = gate_mode & ~(SF_GATE_ROOTS_BY_PARENT | SF_GATE_DEFER_COMPACT);
  if (mode != SF_GATE_MODEL_DTYPE && mode != SF_GATE_FP32_SQUARED && mode != SF_GATE_ALL)
    return SF_ERR_ARG;
  if (B1 < 1 || B1 > 64 || N < 1 || B1 * N > 1024) return SF_ERR_SHAPE;
  if (D < 8 || D % 8 != 0 || D > 8 * 64 * kMaxVecPerLane) return SF_ERR_SHAPE;
  if (bucket < 1 || bucket > B1 * N) return SF_ERR_SHAPE;
  return SF_OK;
}

}  // namespace

extern "C" const char* sf_status_string(int status) {
  switch (status) {
    case SF_OK: return "ok";
    case SF_ERR_SHAPE: return "shape outside kernel limits";
    case SF_ERR_ARG: return "invalid argument";
    case SF_ERR_WORKSPACE: return "workspace too small";
    case SF_ERR_HIP: return "HIP launch failed";
    case SF_ERR_SCRATCH: return "size beyond the fixed scratch of an allocation-free entry point";
    case SF_ERR_CAPTURE:
      return "first call of an allocation-free entry point on this device made under stream "
             "capture (make one eager call first)";
    default: return "unknown status";
  }
}

namespace {

// Parent of every draft branch (specfold/generate/fastdllm_v2_folded.py:55-75):
// diff(i) = the positions where branch i's token differs from the main row's;
// parent(i) = the lowest j != i with |diff(j)| = |diff(i)| - 1 and diff(j) a
// subset of diff(i), else 0 (the main row).  One wave; diff sets as 64-bit masks.
__global__ __launch_bounds__(64) void sf_parent_map_kernel(const int64_t* __restrict__ tokens,
                                                           int B1, int N,
                                                           int32_t* __restrict__ par,
                                                           int32_t* __restrict__ counts) {
  __shared__ unsigned long long s_mask[64];
  __shared__ int s_cnt[64];
  const int i = threadIdx.x;
  if (i < B1) {
    unsigned long long m = 0ull;
    for (int n = 0; n < N; ++n)
      if (tokens[(size_t)i * N + n] != tokens[n]) m |= 1ull << n;
    s_mask[i] = m;
    s_cnt[i] = __popcll(m);
  }
  __syncthreads();
  if (i < B1) {
    int p = 0;
    for (int j = 0; i > 0 && j < B1; ++j)
      if (j != i && s_cnt[j] == s_cnt[i] - 1 && (s_mask[j] & ~s_mask[i]) == 0ull) {
        p = j;
        break;
      }
    par[i] = p;
    if (counts) counts[i] = s_cnt[i];
  }
}

}  // namespace

extern "C" int sf_abi_version(void) { return 14; }

extern "C" int sf_parent_map(const int64_t* tokens, int B1, int N, int32_t* par, int32_t* counts,
                             void* stream) {
  if (!tokens || !par) return SF_ERR_ARG;
  if (B1 < 1 || B1 > 64 || N < 1 || N > 64) return SF_ERR_SHAPE;
  hipLaunchKernelGGL(sf_parent_map_kernel, dim3(1), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), tokens, B1, N, par, counts);
  return sf_launch_status();
}

extern "C" int sf_fold_gate(const uint16_t* hidden, const int32_t* par, const uint16_t* ln_w,
                            int B1, int N, int D, int bucket, float delta, float eps, int gate_mode,
                            int8_t* rec, int32_t* f, int32_t* src, int32_t* rows, int32_t* count,
                            int32_t* seg, int32_t* segcnt, int32_t* slot, float* rstd, uint16_t* xn,
                            void* stream) {
  const bool defer = (gate_mode & SF_GATE_DEFER_COMPACT) != 0;
  if (!hidden || !par || !ln_w || !rec || !rstd || !xn) return SF_ERR_ARG;
  if (!defer && (!f || !src || !rows || !count || !seg || !segcnt)) return SF_ERR_ARG;
  const int chk = check_gate_args(B1, N, D, bucket, gate_mode);
  if (chk != SF_OK) return chk;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  launch_rows_mode<false>(D, hidden, nullptr, nullptr, par, ln_w, B1, N, delta, eps, gate_mode,
                         nullptr, rec, rstd, xn, st);
  if (!defer)
    hipLaunchKernelGGL(sf_gate_compact_kernel, dim3(1), dim3(1024), 0, st, rec, par, B1, N,
                       bucket, f, src, rows, count, seg, segcnt, slot);
  return sf_launch_status();
}

extern "C" int sf_fold_gate_residual(const uint16_t* hp, const uint16_t* ffn,
                                     const int32_t* src_prev, const int32_t* par,
                                     const uint16_t* ln_w, int B1, int N, int D, int bucket,
                                     float delta, float eps, int gate_mode, uint16_t* hidden_out,
                                     int8_t* rec, int32_t* f, int32_t* src, int32_t* rows,
                                     int32_t* count, int32_t* seg, int32_t* segcnt, int32_t* slot,
                                     float* rstd, uint16_t* xn, void* stream) {
  const bool defer = (gate_mode & SF_GATE_DEFER_COMPACT) != 0;
  if (!hp || !ffn || !src_prev || !par || !ln_w || !hidden_out || !rec || !rstd || !xn)
    return SF_ERR_ARG;
  if (!defer && (!f || !src || !rows || !count || !seg || !segcnt)) return SF_ERR_ARG;
  if (hidden_out == hp) return SF_ERR_ARG;
  const int chk = check_gate_args(B1, N, D, bucket, gate_mode);
  if (chk != SF_OK) return chk;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // the row kernel reads src_prev; only the compaction after it writes src
  launch_rows_mode<true>(D, hp, ffn, src_prev, par, ln_w, B1, N, delta, eps, gate_mode, hidden_out,
                        rec, rstd, xn, st);
  if (!defer)
    hipLaunchKernelGGL(sf_gate_compact_kernel, dim3(1), dim3(1024), 0, st, rec, par, B1, N,
                       bucket, f, src, rows, count, seg, segcnt, slot);
  return sf_launch_status();
}

extern "C" int sf_residual_rmsnorm(const uint16_t* hp, const uint16_t* ffn, const int32_t* src,
                                   const uint16_t* w, int B1, int N, int D, float eps,
                                   uint16_t* hidden_out, uint16_t* out, void* stream) {
  if (!hp || !ffn || !src || !w || !hidden_out || !out || hidden_out == hp) return SF_ERR_ARG;
  const int chk = check_gate_args(B1, N, D, 1, SF_GATE_ALL);
  if (chk != SF_OK) return chk;
  launch_rows_any<true, false>(D, hp, ffn, src, nullptr, w, B1, N, 0.f, eps, SF_GATE_ALL,
                               hidden_out, nullptr, nullptr, out,
                               reinterpret_cast<hipStream_t>(stream));
  return sf_launch_status();
}
