// Host stand-in for specfold_amd/csrc/sf_common.h in the CPU SIMT simulation
// (tests/sim/simt.h): the same names and semantics, built on the simulator.  The
// kernel sources are compiled unchanged against it (a copy of the kernel file is
// placed next to this header so its quoted include resolves here).
#pragma once

#include <stdint.h>

#include "simt.h"
#include "specfold_amd.h"

#define SF_DEV inline
#define SF_HD inline

typedef uint16_t sf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sf_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sf_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sf_u32x2 __attribute__((ext_vector_type(2)));
typedef float sf_f32x2 __attribute__((ext_vector_type(2)));

SF_DEV float sf_bf2f(uint16_t b) { return sim_bf16_to_f(b); }
SF_DEV uint16_t sf_f2bf(float f) { return sim_f_to_bf16(f); }
SF_DEV float sf_rbf(float f) { return sf_bf2f(sf_f2bf(f)); }

SF_DEV void sf_unpack8(const sf_u32x4 w, float out[8]) {
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

SF_DEV uint32_t sf_pack2(float lo, float hi) {
  return (uint32_t)sf_f2bf(lo) | ((uint32_t)sf_f2bf(hi) << 16);
}

SF_DEV float sf_wave_sum(float v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
SF_DEV float sf_wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

SF_DEV sf_bf16x8 sf_as_bf16x8(const sf_u32x4 w) { return __builtin_bit_cast(sf_bf16x8, w); }

SF_DEV sf_f32x4 sf_mfma16x16x32(const sf_bf16x8 a, const sf_bf16x8 b, sf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

static inline int sf_launch_status() { return hipGetLastError() == hipSuccess ? SF_OK : SF_ERR_HIP; }

// Direct global -> LDS copies: done at issue in the simulation (the waits that
// order them on the GPU are no-ops here; the barrier is a workgroup barrier).
typedef void sf_lds_void;
SF_DEV void sf_lds_dma16(const void* src, void* lds_base) {
  memcpy(static_cast<char*>(lds_base) + 16 * sim_lane(), src, 16);
}
template <int N>
SF_DEV void sf_wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __syncthreads();
}

SF_DEV void sf_lds_barrier() { __syncthreads(); }
SF_DEV sf_u32x4 sf_stream_load16(const void* p) { return *reinterpret_cast<const sf_u32x4*>(p); }
template <typename T>
SF_DEV void sf_handoff_store(T* p, T v) { *p = v; }
template <typename T>
SF_DEV T sf_handoff_load(const T* p) { return *p; }

// LDS fragment reads (the GPU issues them untracked and waits once): plain reads.
typedef uintptr_t sf_lds_off;
template <int OFF>
SF_DEV sf_u32x4 sf_lds_read16(sf_lds_off addr) {
  sf_u32x4 v;
  memcpy(&v, reinterpret_cast<const void*>(addr + OFF), 16);
  return v;
}
template <int N>
SF_DEV void sf_lds_reads_done(sf_u32x4 (&)[N]) {}
template <int LATER, int N>
SF_DEV void sf_lds_reads_done_but(sf_u32x4 (&)[N]) {}
SF_DEV sf_lds_off sf_lds_addr(const void* p) { return reinterpret_cast<uintptr_t>(p); }
SF_DEV uint32_t sf_lds_read4_now(sf_lds_off addr) {
  uint32_t v;
  memcpy(&v, reinterpret_cast<const void*>(addr), 4);
  return v;
}
// scheduling pins and waits: nothing to order in the simulation
template <typename T>
SF_DEV void sf_pin(T&) {}
SF_DEV void sf_wait_vm_loads() {}
// ds_read_b64_tr_b16: lane i of each 16-lane group gets element i % 4 of the
// 8 bytes lane 4k + i/4 points at, k = 0..3 (the layout measured on gfx950).
template <int OFF>
SF_DEV sf_u32x2 sf_lds_read8_tr(sf_lds_off addr) {
  uint16_t mine[4];
  memcpy(mine, reinterpret_cast<const void*>(addr + OFF), 8);
  uint16_t got[4];
  sim_wave_exchange(mine, 8, [&](const uint8_t* buf) {
    const int l = sim_lane(), grp = l & ~15, i = l & 15;
    for (int k = 0; k < 4; ++k) {
      uint16_t e[4];
      memcpy(e, buf + (grp + 4 * k + i / 4) * 128, 8);
      got[k] = e[i % 4];
    }
  });
  sf_u32x2 v;
  memcpy(&v, got, 8);
  return v;
}
template <int N>
SF_DEV void sf_lds_reads_done(sf_u32x2 (&)[N]) {}
