// Shared device helpers for the SpecFold gfx950 kernels.
//
// Storage type for bf16 is uint16_t (raw bits); arithmetic is done in fp32 and
// rounded back with round-to-nearest-even, which is what torch's bf16 ops do.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "specfold_amd.h"

#define SF_DEV __device__ __forceinline__
#define SF_HD __host__ __device__ __forceinline__

typedef __bf16 sf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sf_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sf_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sf_u32x2 __attribute__((ext_vector_type(2)));
typedef float sf_f32x2 __attribute__((ext_vector_type(2)));

SF_DEV float sf_bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// fp32 -> bf16, round to nearest even, NaN kept a NaN: gfx950's
// v_cvt_pk_bf16_f32 (checked bit-for-bit against the integer RNE formula
// bits + 0x7fff + lsb on all 2^32 inputs).
typedef __bf16 sf_bf16x2 __attribute__((ext_vector_type(2)));

SF_DEV uint16_t sf_f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Round an fp32 value through bf16 (the value a bf16 tensor op would store).
SF_DEV float sf_rbf(float f) { return sf_bf2f(sf_f2bf(f)); }

// Unpack 8 bf16 held in a 16-byte word.
SF_DEV void sf_unpack8(const sf_u32x4 w, float out[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

SF_DEV uint32_t sf_pack2(float lo, float hi) {
  sf_bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Full 64-lane butterfly reductions (result valid in every lane).
SF_DEV float sf_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

SF_DEV float sf_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Reinterpret 8 packed bf16 (u32x4) as the MFMA operand vector.
SF_DEV sf_bf16x8 sf_as_bf16x8(const sf_u32x4 w) {
  union {
    sf_u32x4 u;
    sf_bf16x8 b;
  } c;
  c.u = w;
  return c.b;
}

SF_DEV sf_f32x4 sf_mfma16x16x32(const sf_bf16x8 a, const sf_bf16x8 b, sf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---- direct global -> LDS loads (gfx950 global_load_lds_dwordx4) -------------------
// Every lane copies 16 bytes from its own global address `src` to LDS at
// lds_base + 16 * lane (lds_base: wave-uniform, 16-byte aligned).  The copy counts
// in the issuing wave's vmcnt like any load; the data may be read (by any wave)
// after that count has come down past it and a workgroup barrier.
typedef __attribute__((address_space(3))) void sf_lds_void;
SF_DEV void sf_lds_dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(const_cast<void*>(src), (sf_lds_void*)lds_base, 16, 0, 0);
}

// Wait until at most N vector-memory loads of this wave are outstanding (they
// complete in issue order) and all of its LDS accesses have completed, then a
// workgroup barrier: after it, every wave's loads older than its last N are in
// LDS / registers and no wave still reads LDS it read before the barrier.  No
// memory fence is implied; the signal fences keep the compiler from moving
// memory accesses across the pair.
template <int N>
SF_DEV void sf_wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A workgroup barrier once this wave's LDS accesses have completed; its vector
// memory loads (direct copies included) stay in flight.
SF_DEV void sf_lds_barrier() { sf_wait_vm_barrier<63>(); }

// LDS fragment reads the compiler does not track: 16 bytes at byte address
// `addr` + OFF of LDS into a register, no wait; sf_lds_reads_done makes the values
// usable (s_waitcnt lgkmcnt(0), with every value passed through it so that no use
// is scheduled above the wait).  Used where the compiler would otherwise wait for
// every direct global -> LDS copy in flight before any LDS read.
typedef uint32_t sf_lds_off;  // an LDS byte address
template <int OFF>
SF_DEV sf_u32x4 sf_lds_read16(sf_lds_off addr) {
  sf_u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
template <int N>
SF_DEV void sf_lds_reads_done(sf_u32x4 (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
// The same, leaving the LATER youngest LDS reads in flight (s_waitcnt
// lgkmcnt(LATER)): the reads of v were issued before those LATER.  Valid only where
// LDS operations are the wave's only lgkmcnt traffic (LDS operations complete in
// order; scalar memory loads would not).
template <int LATER, int N>
SF_DEV void sf_lds_reads_done_but(sf_u32x4 (&v)[N]) {
  static_assert(LATER >= 0 && LATER < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(LATER) : "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
// Transposing LDS read (ds_read_b64_tr_b16), untracked like sf_lds_read16: within
// each group of 16 lanes, lane i receives the 4 16-bit elements
//   out[i][k] = (8 bytes at the address of lane 4k + i/4)[i % 4],   k = 0..3,
// i.e. if lane L of the group points at 4 consecutive elements of row L/4,
// starting at column 4(L%4), lane i gets column i of rows 0..3: a 4x16 block
// read column-wise (layout checked on gfx950).
template <int OFF>
SF_DEV sf_u32x2 sf_lds_read8_tr(sf_lds_off addr) {
  sf_u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
template <int N>
SF_DEV void sf_lds_reads_done(sf_u32x2 (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
// One 32-bit LDS read, completed before the function returns (untracked by the
// compiler like sf_lds_read16; for tables read between direct copies).
SF_DEV uint32_t sf_lds_read4_now(sf_lds_off addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Scheduling pins: sf_pin(x) makes x an input and output of an empty volatile asm,
// so whatever computes x stays before the next volatile asm (such as a wait) and
// whatever uses x stays after it.  sf_wait_vm_loads() waits for every vector
// memory load of the wave (s_waitcnt vmcnt(0)).
template <typename T>
SF_DEV void sf_pin(T& x) {
  asm volatile("" : "+v"(x));
}
SF_DEV void sf_wait_vm_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
SF_DEV sf_lds_off sf_lds_addr(const void* p) {
  return (sf_lds_off)(uintptr_t)(const sf_lds_void*)p;
}

// 16 bytes of a read-once stream (weights) into a register, with the non-temporal
// hint: the lines are not kept in L2 for reuse.
SF_DEV sf_u32x4 sf_stream_load16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const sf_u32x4*>(p));
}

// fp32 hand-offs (partial sums one kernel writes and the next reads once) with the
// non-temporal (streaming) hint, so their lines are not kept dirty in L2 for reuse:
// left there, the next weight-streaming kernel pays their write-back while it
// streams (measured at cfg3: gate/up 53.4 against 55.7 us in the step, the verify
// step 5.21 against 5.31-5.35 ms).  SF_PLAIN_HANDOFF gives plain accesses.
template <typename T>
SF_DEV void sf_handoff_store(T* p, T v) {
#ifdef SF_PLAIN_HANDOFF
  *p = v;
#else
  __builtin_nontemporal_store(v, p);
#endif
}
template <typename T>
SF_DEV T sf_handoff_load(const T* p) {
#if defined(SF_PLAIN_HANDOFF) || defined(SF_PLAIN_HANDOFF_LOADS)
  return *p;
#else
  return __builtin_nontemporal_load(p);
#endif
}

// Launch-error check shared by every entry point.
static inline int sf_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SF_OK : SF_ERR_HIP;
}
