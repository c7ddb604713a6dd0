// The fold gate's compaction as a workgroup-level device function: the standalone
// compaction kernel (sf_gate.hip) and the prologue of the gated QKV GEMM
// (sf_qkv.hip, every workgroup compacting for its own A rows) run the same code.
//
// Reference semantics: the compaction the per-branch gate feeds
// (specfold/generate/fastdllm_v2_folded.py:141 nonzero, :136-152) and the Triton
// src kernel (specfold/generate/triton_kernels.py:18-26), with rows in ascending
// flat-row order (the concatenation of the reference's per-branch nonzero()
// lists) instead of the Triton gate's atomic slot order.
#pragma once

#include "sf_common.h"

// Outputs of the compaction, as sf_fold_gate documents them (slot may be NULL).
struct GateOut {
  int32_t* f;
  int32_t* src;
  int32_t* rows;
  int32_t* count;
  int32_t* seg;
  int32_t* segcnt;
  int32_t* slot;
};

// Compaction of the recompute flags rec[0, BN), BN = B1*N <= NT*K, by one
// workgroup of NT threads (thread i takes rows i + k*NT, k < K; NT a multiple of
// 64).  A ballot/popcount scan gives row t its slot, the number of recomputed rows
// before it; the recomputed rows with a slot below bucket go to s_rows[slot] (LDS,
// may be NULL) in ascending order.  Returns the count (which may exceed bucket).
// s_f, s_slot: LDS scratch of BN ints each; s_tot: NT*K/64 ints.  With write_out
// (one workgroup of a launch) also writes f, src (the fixed point of f: chains
// strictly shorten towards branch 0, so B1 hops reach it), rows (BN past the
// count), count, seg, segcnt and slot.  Starts and ends with every thread of the
// workgroup; ends with a barrier, so the scratch may be reused.
template <int NT, int K>
SF_DEV int gate_compact(const int8_t* __restrict__ rec, const int32_t* __restrict__ par, int B1,
                        int N, int bucket, int* s_f, int* s_slot, int* s_tot, int* s_rows,
                        bool write_out, const GateOut& out) {
  static_assert(NT % 64 == 0, "whole waves");
  constexpr int kWaves = NT / 64;
  const int BN = B1 * N;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  bool flag[K];
  int pre[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int t = tid + k * NT;
    flag[k] = t < BN && rec[t] != 0;
    const unsigned long long bal = __ballot(flag[k]);
    pre[k] = __popcll(bal & ((1ull << lane) - 1ull));   // recomputed rows below, in the chunk
    if (lane == 0) s_tot[wv + k * kWaves] = __popcll(bal);
  }
  __syncthreads();
  int total = 0;
  int base[K];
#pragma unroll
  for (int k = 0; k < K; ++k) base[k] = 0;
  for (int c = 0; c < K * kWaves; ++c) {
    const int v = s_tot[c];
#pragma unroll
    for (int k = 0; k < K; ++k) base[k] += c < wv + k * kWaves ? v : 0;
    total += v;
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int t = tid + k * NT;
    if (t < BN) {
      const int b = t / N;
      const int slot = base[k] + pre[k];
      int p = par[b];
      p = p < 0 ? 0 : (p >= B1 ? B1 - 1 : p);
      const int fv = flag[k] ? b : p;
      s_f[t] = fv;
      s_slot[t] = slot;
      const bool listed = flag[k] && slot < bucket;
      if (listed && s_rows) s_rows[slot] = t;
      if (write_out) {
        out.f[t] = fv;
        if (listed) out.rows[slot] = t;
        if (out.slot) out.slot[t] = listed ? slot : -1;
      }
    }
  }
  if (write_out)
    for (int s = tid; s < bucket; s += NT)
      if (s >= total) out.rows[s] = BN;
  __syncthreads();
  if (write_out) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int t = tid + k * NT;
      if (t < BN) {
        const int b = t / N;
        const int n = t - b * N;
        const int first = s_slot[b * N];
        if (flag[k]) out.seg[b * N + (s_slot[t] - first)] = t;
        if (n == 0) out.segcnt[b] = ((b + 1 < B1) ? s_slot[(b + 1) * N] : total) - first;
        int s = s_f[t];
        for (int hop = 0; hop < B1; ++hop) s = s_f[s * N + n];
        out.src[t] = s;
      }
    }
    if (tid == 0) *out.count = total;
  }
  __syncthreads();
  return total;
}
