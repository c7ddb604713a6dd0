// One decode-loop iteration's decisions and the facts its control flow reads, in
// one launch on one wave (the block is at most 64 tokens).
//
// Replaces, for a batch of one sequence, the torch sequence of the Fast-dLLM loop
// after a small block's sampling (specfold/generate/fastdllm_v2_generation.py:
// 660-700, restated op for op in specfold_amd/generate/fastdllm_v2_generation.py):
//   conf = where(small_mask, conf, -inf); best = argmax(conf) (first maximum)
//   unmask = ((conf > threshold) | (col == best)) & small_mask
//   x_t[small block] = where(unmask, x_1, x_t[small block])
// and then the loop's reads of the token state (stop token with no mask before
// it, the block's and each small block's masked counts, the first cached draft
// state equal to the block, the committed count), which the torch form computes
// with ~25 small kernels.  Integer and bool logic plus one bf16 comparison: the
// results are the torch sequence's exactly.
#include "sf_common.h"

namespace {

constexpr int kMaxStates = 16;   // cached draft states compared with the block

struct StatePtrs {
  const int64_t* p[kMaxStates];
};

__device__ __forceinline__ int wave_first_set(unsigned long long m) {
  return m ? __builtin_ctzll(m) : -1;
}

// One wave.  Lane j < bl holds block token j (flat position L - bl + j).
__global__ __launch_bounds__(64) void sf_decode_facts_kernel(
    int64_t* __restrict__ x_t, int L, int plen, int bl, int sbs, int s0, long long mask_id,
    long long stop_id, const uint16_t* __restrict__ conf, const int64_t* __restrict__ x_1,
    float threshold, StatePtrs states, int n_states, int8_t* __restrict__ unmask_out,
    int64_t* __restrict__ facts) {
  const int j = threadIdx.x;
  const bool in = j < bl;
  const long long pos = (long long)L - bl + (in ? j : 0);
  long long tok = in ? x_t[pos] : 0;

  // ---- the small block's decision (conf given) -----------------------------------
  int n_unmask = 0;
  if (conf) {
    const int k = j - s0;                               // column in the small block
    const bool col = in && k >= 0 && k < sbs;
    const bool masked = col && tok == mask_id;
    // bf16 confidences compare as floats (the torch ops run in bf16; the threshold
    // comes rounded to bf16)
    const float c = masked ? sf_bf2f(conf[k]) : -INFINITY;
    // argmax over the small block's columns, the first maximum (torch.argmax)
    float best = c;
    int bidx = col ? k : 0x7fffffff;
    for (int o = 32; o >= 1; o >>= 1) {
      const float ob = __shfl_xor(best, o, 64);
      const int oi = __shfl_xor(bidx, o, 64);
      if (ob > best || (ob == best && oi < bidx)) {
        best = ob;
        bidx = oi;
      }
    }
    const bool un = masked && (c > threshold || k == bidx);
    if (col) {
      unmask_out[k] = un ? 1 : 0;
      if (un) {
        tok = x_1[k];
        x_t[pos] = tok;
      }
    }
    n_unmask = __popcll(__ballot(un));
  }

  // ---- facts of the (updated) token state ------------------------------------------
  const bool is_mask = in && tok == mask_id;
  const unsigned long long mmask = __ballot(is_mask);
  // the tail x_t[plen:] is the block's last L - plen tokens
  const int t0 = bl - (L - plen);                       // block index of tail token 0
  const bool in_tail = in && j >= t0;
  const unsigned long long smask = __ballot(in_tail && tok == stop_id);
  const int first = wave_first_set(smask);             // block index of the first stop
  // masks before the first stop (none when there is no stop: torch's argmax of an
  // all-zero row is 0, so nothing is "ahead")
  const unsigned long long before =
      first >= 0 ? (mmask & ((1ull << first) - 1ull) & ~((1ull << t0) - 1ull)) : 0ull;
  // the first cached state equal to the block
  int hit = -1;
  for (int s = 0; s < n_states && hit < 0; ++s) {
    const bool eq = !in || states.p[s][j] == tok;
    if (__ballot(!eq) == 0ull) hit = s;
  }
  if (j == 0) {
    int o = 0;
    facts[o++] = (first >= 0 && before == 0ull) ? 1 : 0;
    facts[o++] = __popcll(mmask);
    for (int b = 0; b < bl / sbs; ++b) {
      const unsigned long long sb = ((sbs == 64) ? ~0ull : ((1ull << sbs) - 1ull)) << (b * sbs);
      facts[o++] = __popcll(mmask & sb);
    }
    if (n_states > 0) facts[o++] = hit;
    if (conf) facts[o++] = n_unmask;
  }
}

}  // namespace

extern "C" int sf_decode_facts(int64_t* x_t, int L, int plen, int bl, int sbs, int s0,
                               long long mask_id, long long stop_id, const uint16_t* conf,
                               const int64_t* x_1, float threshold,
                               const int64_t* const* states, int n_states, int8_t* unmask,
                               int64_t* facts, void* stream) {
  if (!x_t || !facts) return SF_ERR_ARG;
  // the tail x_t[plen:] is 1 .. bl of the block's tokens
  if (bl < 1 || bl > 64 || sbs < 1 || bl % sbs || L < bl || plen < L - bl || plen >= L)
    return SF_ERR_SHAPE;
  if (n_states < 0 || n_states > kMaxStates || (n_states > 0 && !states)) return SF_ERR_SHAPE;
  if (conf && (!x_1 || !unmask || s0 < 0 || s0 + sbs > bl)) return SF_ERR_ARG;
  StatePtrs sp{};
  for (int s = 0; s < n_states; ++s) {
    if (!states[s]) return SF_ERR_ARG;
    sp.p[s] = states[s];
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(sf_decode_facts_kernel, dim3(1), dim3(64), 0, st, x_t, L, plen, bl, sbs, s0,
                     mask_id, stop_id, conf, x_1, threshold, sp, n_states, unmask, facts);
  return sf_launch_status();
}
