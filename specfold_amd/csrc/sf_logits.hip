// Per-position statistics of logits rows for greedy decoding: the top-8 tokens,
// the softmax normaliser, the top-p (nucleus) normaliser and the greedy token
// with its bf16 probability.  They replace the sort, softmax, cumulative-sum and
// scatter sequence of the reference's top-p sampler
// (specfold/generate/fastdllm_model_executor.py:129-155) and the softmax + topk
// calls of its draft construction (fastdllm_v2_generation.py:430-470,
// nld_generation.py:105-151) at temperature 0.
//
// Semantics, with e_i = exp(l_i - l_max) in fp32 and Z = sum_i e_i:
//  * top-8: (index, logit) ordered by logit descending, then index ascending.
//  * nucleus: with p_i = bf16(e_i / Z) (the bf16 softmax) in descending order,
//    keep every token up to and including the first one whose cumulative sum,
//    rounded to bf16, exceeds top_p (the reference keeps a sorted token while
//    bf16(cumsum of the probabilities before it) <= top_p); Zn = sum of e over the
//    kept tokens.  Tokens of equal value are interchangeable, so Zn depends only
//    on how many tied tokens at the cut are kept, not on which.
//  * greedy token: the reference's argmax over the bf16 nucleus probabilities
//    bf16(e_i / Zn): the lowest index whose bf16 probability equals the maximum,
//    bf16(1 / Zn) (near-equal logits can round to the same bf16 probability).
//  * conf = bf16(1 / Zn) (the greedy token's probability), conf_full =
//    bf16(1 / Z) (the maximum of the bf16 softmax).
//
// Two kernels.  Slice: several workgroups per row count their tokens into a
// 65536-bin histogram of the bf16 bit pattern in LDS (two 16-bit counts per
// 32-bit word), add its nonzero bins into the row's histogram in memory (integer
// atomics: one per distinct value of the slice instead of one per token, which on
// logits clustered over a few hundred bf16 values contended in L2), and reduce
// their slice's top-8.  Finish: one workgroup per row merges the slice candidates and
// walks the histogram in descending value order: masses are count(v) * e(v) and
// count(v) * p(v), summed in a fixed order (deterministic), which gives Z, the
// cut and Zn from exact counts; it then clears the histogram for the next call.
#include <math.h>

#include <mutex>

#include "sf_common.h"
#include "sf_index.h"

namespace {

constexpr int kTop = 8;
constexpr int kSliceThreads = 512;
constexpr int kFinishThreads = 1024;
constexpr int kKeys = 65536;
using sfl::kMaxSlices;
using sfl::slices_for;
static_assert(kMaxSlices <= 64, "one wave merges the slices' lists");
static_assert(sfl::kMaxSliceVectors * 8 <= 65535, "a slice's counts and token places fit 16 bits");

// order key of a bf16 bit pattern: larger value -> larger key
SF_DEV uint32_t bf16_key(uint32_t b) { return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u); }
SF_DEV float key_value(uint32_t k) {
  const uint32_t b = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
  return __uint_as_float(b << 16);
}

// (value desc, index asc)
SF_DEV bool better(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

// Block-wide best of one candidate per thread; every thread gets the winner.
template <int NT>
SF_DEV void block_best(float& v, int& i, float* s_v, int* s_i) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    const int j = __shfl_xor(i, o, 64);
    if (better(w, j, v, i)) {
      v = w;
      i = j;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = v;
    s_i[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  v = s_v[0];
  i = s_i[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w)
    if (better(s_v[w], s_i[w], v, i)) {
      v = s_v[w];
      i = s_i[w];
    }
  __syncthreads();
}

// Ordering key of a bf16 logit for the top-8: larger value -> larger key, both
// zeros equal (as in a float comparison), NaN 0 (below every value, equal to an
// empty slot, so never taken).
SF_DEV uint32_t rank_key(uint32_t b) {
  const uint32_t a = b & 0x7fffu;
  if (a > 0x7f80u) return 0u;
  return bf16_key(a == 0u ? 0u : b);
}

template <typename K>
SF_DEV K wave_max(K x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const K y = __shfl_xor(x, o, 64);
    x = x > y ? x : y;
  }
  return x;
}

// Top-8 of a wave from per-lane lists of L keys in descending order (nonzero keys
// distinct, 0 = empty): 8 rounds of a wave maximum, the winning lane popping its
// list's head.  Every lane gets the 8 in `out`, largest first.
template <int L, typename K>
SF_DEV void wave_top8(K (&l)[L], K (&out)[kTop]) {
#pragma unroll
  for (int r = 0; r < kTop; ++r) {
    const K w = wave_max(l[0]);
    out[r] = w;
    const bool pop = l[0] == w;
#pragma unroll
    for (int k = 0; k + 1 < L; ++k) l[k] = pop ? l[k + 1] : l[k];
    l[L - 1] = pop ? K(0) : l[L - 1];
  }
}

// Prefix sums over the workgroup's threads in thread order (a shuffle scan per
// wave, then the wave totals in order; deterministic): returns the exclusive
// prefix, with the inclusive one in `incl` (the next thread's exclusive prefix,
// bit for bit) and the workgroup total in `total`.  s_w: NT / 64 floats of LDS.
template <int NT>
SF_DEV float block_scan(float x, float* s_w, float& incl, float& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float in = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(in, o, 64);
    if (lane >= o) in += y;
  }
  float ex = __shfl_up(in, 1, 64);
  if (lane == 0) ex = 0.f;
  if (lane == 63) s_w[wv] = in;
  __syncthreads();
  float base = 0.f, tot = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (w < wv) base += s_w[w];
    tot += s_w[w];
  }
  __syncthreads();
  incl = base + in;
  total = tot;
  return base + ex;
}

// grid (S, M): slice s of row m counts its tokens into hist[m] and writes its
// top-8 as keys (rank_key(value) << 16 | 0xffff - token's place in the slice:
// larger = higher value, then lower index; 0 = none) to cand[m][s][0..7].
__global__ __launch_bounds__(kSliceThreads) void sf_logit_slice_kernel(
    const uint16_t* __restrict__ logits, long long ld, int V, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ cand) {
  static_assert(kSliceThreads / 64 * kTop == 64, "one wave merges the waves' lists");
  __shared__ sf_u32x4 s_hist4[kKeys / 8];   // key 2i: low half of word i, 2i + 1: high half
  __shared__ uint32_t s_top[kSliceThreads / 64 * kTop];
  uint32_t* s_hist = reinterpret_cast<uint32_t*>(s_hist4);
  for (int i = threadIdx.x; i < kKeys / 8; i += kSliceThreads) s_hist4[i] = sf_u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
  const int S = gridDim.x, s = blockIdx.x, row = blockIdx.y;
  const uint16_t* x = logits + (long long)row * ld;
  uint32_t* h = hist + (size_t)row * kKeys;
  const int nvec = V >> 3;
  const int v0 = sfl::slice_begin(s, nvec, S), v1 = sfl::slice_begin(s + 1, nvec, S);
  // the thread's top-8 keys in descending order: each token passes down the list
  // in a compare-exchange chain (branch-free; the slice has at most 65535 tokens)
  uint32_t top[kTop];
#pragma unroll
  for (int k = 0; k < kTop; ++k) top[k] = 0u;
  for (int vi = v0 + threadIdx.x; vi < v1; vi += kSliceThreads) {
    const sf_u32x4 w = *reinterpret_cast<const sf_u32x4*>(x + (size_t)vi * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t bits = (e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu);
      const uint32_t key = bf16_key(bits);
      atomicAdd(&s_hist[key >> 1], (key & 1u) ? 0x10000u : 1u);
      const uint32_t rk = rank_key(bits);
      uint32_t c = rk ? (rk << 16) | (0xffffu - (uint32_t)((vi - v0) * 8 + e)) : 0u;
#pragma unroll
      for (int k = 0; k < kTop; ++k) {
        const uint32_t hi = max(top[k], c);
        c = min(top[k], c);
        top[k] = hi;
      }
    }
  }
  // the slice's counts into the row's histogram: its nonzero bins only
  __syncthreads();
  for (int i = threadIdx.x; i < kKeys / 8; i += kSliceThreads) {
    const sf_u32x4 w = s_hist4[i];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (w[q] & 0xffffu) atomicAdd(&h[8 * i + 2 * q], w[q] & 0xffffu);
      if (w[q] >> 16) atomicAdd(&h[8 * i + 2 * q + 1], w[q] >> 16);
    }
  }
  // the slice's top-8: each wave's, then wave 0 merges the waves' 8 x 8
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t wt[kTop];
  wave_top8<kTop>(top, wt);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kTop; ++r) s_top[wv * kTop + r] = wt[r];
  }
  __syncthreads();
  if (wv == 0) {
    uint32_t one[1] = {s_top[lane]};
    uint32_t bt[kTop];
    wave_top8<1>(one, bt);
    if (lane < kTop) {
      uint32_t b = bt[0];
#pragma unroll
      for (int r = 1; r < kTop; ++r) b = r == lane ? bt[r] : b;
      cand[((size_t)row * S + s) * kTop + lane] = b;
    }
  }
}

// one workgroup per row
__global__ __launch_bounds__(kFinishThreads) void sf_logit_finish_kernel(
    const uint16_t* __restrict__ logits, long long ld, int V, int S, float top_p,
    uint32_t* __restrict__ hist, const uint32_t* __restrict__ cand, int32_t* __restrict__ top_idx,
    float* __restrict__ top_val, float* __restrict__ zfull, float* __restrict__ znuc,
    int32_t* __restrict__ greedy_tok, float* __restrict__ conf, float* __restrict__ conf_full) {
  __shared__ float s_v[kFinishThreads / 64];
  __shared__ int s_i[kFinishThreads / 64];
  __shared__ float s_bv[kTop];
  __shared__ int s_bi[kTop];
  __shared__ float s_cutf[2];  // Z, Zn
  const int tid = threadIdx.x, row = blockIdx.x;
  uint32_t* h = hist + (size_t)row * kKeys;

  // ---- merge the slices' top-8 lists (S <= 64): lane s of wave 0 takes slice s's ----
  // list, keyed (rank << 32 | 0xffff - s << 16 | 0xffff - place): ties go to the
  // lower slice, then the lower place, i.e. the lower token index
  if (tid < 64) {
    uint64_t l[kTop];
#pragma unroll
    for (int k = 0; k < kTop; ++k) {
      const uint32_t c = tid < S ? cand[((size_t)row * S + tid) * kTop + k] : 0u;
      l[k] = c ? ((uint64_t)(c >> 16) << 32) | ((uint64_t)(0xffffu - tid) << 16) | (c & 0xffffu)
               : 0ull;
    }
    uint64_t b[kTop];
    wave_top8<kTop>(l, b);
    if (tid < kTop) {
      uint64_t w = b[0];
#pragma unroll
      for (int r = 1; r < kTop; ++r) w = r == tid ? b[r] : w;
      float v = -INFINITY;
      int i = 0x7fffffff;
      if (w) {
        const int s = 0xffff - (int)((w >> 16) & 0xffffu);
        i = sfl::slice_begin(s, V >> 3, S) * 8 + (0xffff - (int)(w & 0xffffu));
        v = __uint_as_float((uint32_t)logits[(long long)row * ld + i] << 16);
      }
      s_bv[tid] = v;
      s_bi[tid] = i;
    }
  }
  __syncthreads();
  float bv[kTop];
  int bi[kTop];
#pragma unroll
  for (int r = 0; r < kTop; ++r) {
    bv[r] = s_bv[r];
    bi[r] = s_bi[r];
  }
  const float lmax = bv[0];

  // ---- histogram walk: thread t owns keys 65535 - 64t - j, j = 0..63 (descending) --
  // Two sums per stretch, each taken from the stretch's highest key down: the
  // softmax mass (e = exp(v - l_max)) and, once Z is known, the bf16 probability
  // mass the reference accumulates (p = bf16(e / Z): softmax of bf16 logits).
  const int kb = kKeys - 1 - 64 * tid;
  const sf_u32x4* hv = reinterpret_cast<const sf_u32x4*>(h + kb - 63);
  // sum over the stretch, highest key first, of count * f(value)
  auto stretch_sum = [&](auto f) {
    float acc = 0.f;
#pragma unroll
    for (int q = 15; q >= 0; --q) {
      const sf_u32x4 w = hv[q];
#pragma unroll
      for (int r = 3; r >= 0; --r)
        if (w[r]) acc += (float)w[r] * f(key_value(kb - 63 + 4 * q + r));
    }
    return acc;
  };
  const float part = stretch_sum([&](float v) { return expf(v - lmax); });
  // prefix over the stretches in descending key order (fixed order; Z is the total)
  float z, incl_e;
  const float excl_e = block_scan<kFinishThreads>(part, s_v, incl_e, z);
  const float part_p = stretch_sum([&](float v) { return sf_rbf(expf(v - lmax) / z); });
  float incl_p, tot_p;
  const float excl_p = block_scan<kFinishThreads>(part_p, s_v, incl_p, tot_p);
  if (tid == 0) s_cutf[1] = z;  // the nucleus mass when nothing is cut
  __syncthreads();
  // The reference drops sorted token i >= 1 when bf16(cumsum_{j<i} p_j) > top_p:
  // the kept tokens run up to and including the first one whose cumulative
  // probability crosses.  Exactly one stretch holds the crossing (monotone sums).
  auto crosses = [&](float cum) { return sf_rbf(cum) > top_p; };
  if (!crosses(excl_p) && crosses(incl_p)) {
    // the walk down the stretch to the first key whose mass crosses, in two halves
    // of 32 counts, each read in one round of loads (count of key kb - j in
    // cnt[j - 32 * half])
    float cp = excl_p, ce = excl_e;
    bool found = false;
    uint32_t cx = 0;
    float ex = 0.f, px = 0.f, cpx = 0.f, cex = 0.f;
    for (int half = 0; half < 2 && !found; ++half) {
      uint32_t cnt[32];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const sf_u32x4 w = hv[15 - 8 * half - q];
#pragma unroll
        for (int r = 0; r < 4; ++r) cnt[4 * q + 3 - r] = w[r];
      }
#pragma unroll
      for (int jj = 0; jj < 32; ++jj) {
        const int j = 32 * half + jj;
        const uint32_t c = cnt[jj];
        if (!found && c) {
          const float e = expf(key_value(kb - j) - lmax);
          const float pj = sf_rbf(e / z);
          if (crosses(cp + (float)c * pj)) {
            found = true;
            cx = c; ex = e; px = pj; cpx = cp; cex = ce;
          }
          cp += (float)c * pj;
          ce += (float)c * e;
        }
      }
    }
    float zc = ce;  // rounding kept the crossing out of reach: whole stretch
    if (found) {
      // fewest tokens of the crossing value whose cumulative probability crosses
      uint32_t lo = 1, hi = cx;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (crosses(cpx + (float)mid * px)) hi = mid; else lo = mid + 1;
      }
      zc = cex + (float)lo * ex;
    }
    s_cutf[1] = zc;
  }
  __syncthreads();
  const float zn = s_cutf[1];

  // ---- greedy token: lowest index whose bf16 probability equals the maximum -------
  const float cmax = sf_rbf(1.0f / zn);
  int g = 0x7fffffff;
  bool all_tied = true;
#pragma unroll
  for (int r = 0; r < kTop; ++r) {
    const bool tied = bv[r] > -INFINITY && sf_rbf(expf(bv[r] - lmax) / zn) == cmax;
    if (tied) g = min(g, bi[r]);
    all_tied = all_tied && tied;
  }
  if (all_tied) {
    // more than 8 tokens may share the maximum probability: every token whose
    // value is at least the smallest tied value is tied; scan the row
    // (probabilities are monotone in the logit)
    const float lo = bv[kTop - 1];
    float vmin = lo;
    for (uint32_t k = bf16_key(__float_as_uint(lo) >> 16); k > 0; --k) {
      const float v = key_value(k - 1);
      if (sf_rbf(expf(v - lmax) / zn) != cmax) break;
      vmin = v;
    }
    const uint16_t* x = logits + (long long)row * ld;
    int gi = 0x7fffffff;
    for (int vi = tid; vi < (V >> 3); vi += kFinishThreads) {
      const sf_u32x4 w = *reinterpret_cast<const sf_u32x4*>(x + (size_t)vi * 8);
      float f[8];
      sf_unpack8(w, f);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (f[e] >= vmin) gi = min(gi, vi * 8 + e);
    }
    float dummy = 0.f;
    block_best<kFinishThreads>(dummy, gi, s_v, s_i);
    g = gi;
  }

  // ---- outputs; clear this row's histogram for the next call ---------------------
  if (tid == 0) {
#pragma unroll
    for (int r = 0; r < kTop; ++r) {
      top_idx[row * kTop + r] = bi[r];
      top_val[row * kTop + r] = bv[r];
    }
    zfull[row] = z;
    znuc[row] = zn;
    greedy_tok[row] = g;
    conf[row] = cmax;
    conf_full[row] = sf_rbf(1.0f / z);
  }
  {
    sf_u32x4* hv = reinterpret_cast<sf_u32x4*>(h + kb - 63);
#pragma unroll
    for (int q = 0; q < 16; ++q) hv[q] = sf_u32x4{0u, 0u, 0u, 0u};
  }
}

// Rows the allocation-free entry point takes; with S = slices_for(M, V) slices per
// row (sf_index.h), M * S <= 256 for every M <= 64 and V <= 4 * 65528 (a call whose larger
// vocabulary needs more than the 512 candidate lists is refused), so the
// candidates fit in 512 * 8 keys.
constexpr int kNoAllocMaxRows = 64;
constexpr size_t kNoAllocHistBytes = (size_t)kNoAllocMaxRows * kKeys * 4;
constexpr size_t kNoAllocBytes = kNoAllocHistBytes + (size_t)512 * kTop * 4;

__global__ __launch_bounds__(256) void sf_zero_kernel(sf_u32x4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = sf_u32x4{0u, 0u, 0u, 0u};
}

int launch_stats(const uint16_t* logits, int M, int V, long long ld, float top_p, int32_t* top_idx,
                 float* top_val, float* zfull, float* znuc, int32_t* greedy_tok, float* conf,
                 float* conf_full, uint32_t* hist, void* cand, hipStream_t st) {
  const int S = slices_for(M, V);
  uint32_t* cand_k = reinterpret_cast<uint32_t*>(cand);
  hipLaunchKernelGGL(sf_logit_slice_kernel, dim3(S, M), dim3(kSliceThreads), 0, st, logits, ld, V,
                     hist, cand_k);
  hipLaunchKernelGGL(sf_logit_finish_kernel, dim3(M), dim3(kFinishThreads), 0, st, logits, ld, V,
                     S, top_p, hist, cand_k, top_idx, top_val, zfull, znuc, greedy_tok,
                     conf, conf_full);
  return sf_launch_status();
}

int check_stats_args(const uint16_t* logits, int M, int V, long long ld, float top_p,
                     const int32_t* top_idx, const float* top_val, const float* zfull,
                     const float* znuc, const int32_t* greedy_tok, const float* conf,
                     const float* conf_full) {
  if (!logits || !top_idx || !top_val || !zfull || !znuc || !greedy_tok || !conf || !conf_full)
    return SF_ERR_ARG;
  if (M < 1 || V < kTop || V % 8 != 0 || ld < V || ld % 8 != 0) return SF_ERR_SHAPE;
  if (V > sfl::kMaxVocab) return SF_ERR_SHAPE;
  if (reinterpret_cast<uintptr_t>(logits) % 16 != 0 || !(top_p > 0.0f)) return SF_ERR_ARG;
  return SF_OK;
}

}  // namespace

// The allocation-free entry point's workspace: the histograms of kNoAllocMaxRows
// rows (zero between calls), then the slice candidates (scratch).  Each GPU holds its own copy
// for the life of the process.  Host code never uses this name as an address (on
// the host it is only a stand-in for the symbol): it takes the device address
// from hipGetSymbolAddress, once per device.
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // scratch's device address per device; null until set up

// The current device's copy of scratch.  The first call on a device looks its
// address up and clears the histograms with a fill kernel on `st`, then waits for
// it, so the address is published only once the array is zero for every stream;
// that first call is refused under stream capture (the clear would become a node
// of the caller's graph, run again on every replay, and would not have run when
// the address is published).  Every call leaves the histograms zero again.
int scratch_for_current_device(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SF_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return SF_ERR_HIP;
    if (cs != hipStreamCaptureStatusNone) return SF_ERR_CAPTURE;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SF_ERR_HIP;
    hipLaunchKernelGGL(sf_zero_kernel, dim3(1024), dim3(256), 0, st,
                       reinterpret_cast<sf_u32x4*>(p), kNoAllocHistBytes / 16);
    if (sf_launch_status() != SF_OK || hipStreamSynchronize(st) != hipSuccess) return SF_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SF_OK;
}

}  // namespace

extern "C" size_t sf_logit_stats_workspace_bytes(int M) {
  if (M < 1) return 0;
  // candidates for the most slices any V takes (kMaxSlices)
  return (size_t)M * kKeys * 4 + (size_t)M * kMaxSlices * kTop * 4;
}

extern "C" int sf_logit_stats(const uint16_t* logits, int M, int V, long long ld, float top_p,
                              int32_t* top_idx, float* top_val, float* zfull, float* znuc,
                              int32_t* greedy_tok, float* conf, float* conf_full, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const int a = check_stats_args(logits, M, V, ld, top_p, top_idx, top_val, zfull, znuc,
                                 greedy_tok, conf, conf_full);
  if (a != SF_OK) return a;
  if (!workspace || reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return SF_ERR_ARG;
  if (workspace_bytes < sf_logit_stats_workspace_bytes(M)) return SF_ERR_WORKSPACE;
  uint32_t* hist = reinterpret_cast<uint32_t*>(workspace);
  return launch_stats(logits, M, V, ld, top_p, top_idx, top_val, zfull, znuc, greedy_tok, conf,
                      conf_full, hist, hist + (size_t)M * kKeys,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sf_logit_stats_noalloc_max_rows(void) { return kNoAllocMaxRows; }

extern "C" int sf_logit_stats_noalloc(const uint16_t* logits, int M, int V, long long ld,
                                      float top_p, int32_t* top_idx, float* top_val, float* zfull,
                                      float* znuc, int32_t* greedy_tok, float* conf,
                                      float* conf_full, void* stream) {
  const int a = check_stats_args(logits, M, V, ld, top_p, top_idx, top_val, zfull, znuc,
                                 greedy_tok, conf, conf_full);
  if (a != SF_OK) return a;
  if (M > kNoAllocMaxRows ||
      (size_t)M * slices_for(M, V) * kTop * 4 > kNoAllocBytes - kNoAllocHistBytes)
    return SF_ERR_SCRATCH;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int s = scratch_for_current_device(st, &ws);
  if (s != SF_OK) return s;
  // fixed layout whatever M is: the histograms of every row the array can take,
  // then the candidates, so that no call writes candidates over a histogram that
  // a later call with more rows counts into
  uint8_t* base = reinterpret_cast<uint8_t*>(ws);
  return launch_stats(logits, M, V, ld, top_p, top_idx, top_val, zfull, znuc, greedy_tok, conf,
                      conf_full, reinterpret_cast<uint32_t*>(base), base + kNoAllocHistBytes, st);
}
