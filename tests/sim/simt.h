// A small SIMT simulator that runs HIP kernel source on the CPU, for tests only.
//
// A workgroup runs as one fiber per work-item on one OS thread, switched at
// barriers; workgroups are shared out over a small pool of OS threads.
// __syncthreads is a barrier over the workgroup, wave-collective operations
// (shuffles, MFMA) exchange operands through a per-wave buffer between two
// barriers over the wave's 64 lanes.  __shared__ variables become function-local
// thread_local statics (one workgroup per pool thread is alive at a time).
// MFMA results are computed from the operand layouts the AMD matrix instruction
// documentation gives for each instruction (see mfma_* below), with fp32
// accumulation of exact products.  Only what the kernels under test use is here.
#pragma once

#include <stdint.h>
#include <string.h>

#include <ucontext.h>

#include <atomic>
#include <cmath>
#include <functional>
#include <thread>
#include <vector>

// ---- launch geometry ---------------------------------------------------------------
struct sim_dim3 {
  unsigned x = 1, y = 1, z = 1;
  sim_dim3() = default;
  sim_dim3(unsigned a, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
typedef sim_dim3 dim3;

// One work-item: a fiber with its own stack and geometry.
struct SimFiber {
  ucontext_t ctx;
  std::vector<char> stack;
  sim_dim3 tid, bid, bdim, gdim;
  int flat = 0;
  bool done = false;
  const unsigned* wait_gen = nullptr;  // waiting until *wait_gen != wait_val
  unsigned wait_val = 0;
};

// A barrier of n fibers: the last to arrive starts a new generation.
struct SimBarrier {
  int n = 0, arrived = 0;
  unsigned gen = 0;
};

// The workgroup a pool thread is running.
struct SimBlock {
  std::vector<SimFiber> fibers;
  ucontext_t sched;
  SimFiber* cur = nullptr;
  SimBarrier block;
  std::vector<SimBarrier> wave;
  std::vector<std::vector<uint8_t>> xch;  // per wave: 64 lanes x 128 bytes
};
inline thread_local SimBlock* sim_blk = nullptr;
#define threadIdx (sim_blk->cur->tid)
#define blockIdx (sim_blk->cur->bid)
#define blockDim (sim_blk->cur->bdim)
#define gridDim (sim_blk->cur->gdim)

inline void sim_arrive(SimBarrier& b) {
  SimFiber* f = sim_blk->cur;
  if (++b.arrived == b.n) {
    b.arrived = 0;
    ++b.gen;
    return;
  }
  f->wait_gen = &b.gen;
  f->wait_val = b.gen;
  swapcontext(&f->ctx, &sim_blk->sched);
}

inline void __syncthreads() { sim_arrive(sim_blk->block); }

// ---- wave collectives --------------------------------------------------------------
inline int sim_lane() { return sim_blk->cur->flat & 63; }
inline int sim_wave() { return sim_blk->cur->flat >> 6; }

// Deposit `bytes` of this lane's value, wait for the wave, run `use` on the
// wave's deposits, wait again before the buffer is reused.
template <typename F>
inline void sim_wave_exchange(const void* mine, size_t bytes, F use) {
  const int w = sim_wave();
  auto& buf = sim_blk->xch[w];
  memcpy(&buf[sim_lane() * 128], mine, bytes);
  sim_arrive(sim_blk->wave[w]);
  use(buf.data());
  sim_arrive(sim_blk->wave[w]);
}

// v_readfirstlane: the value of the wave's first lane (every lane is active here)
inline int sim_readfirstlane(int v) {
  int out;
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b, 4); });
  return out;
}
#define __builtin_amdgcn_readfirstlane(x) sim_readfirstlane(x)

inline float __shfl(float v, int src, int width = 64) {
  (void)width;
  float out;
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b + (src & 63) * 128, 4); });
  return out;
}

inline int __shfl(int v, int src, int width = 64) {
  (void)width;
  int out;
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b + (src & 63) * 128, 4); });
  return out;
}

inline float __shfl_xor(float v, int mask, int width = 64) {
  (void)width;
  float out;
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b + ((sim_lane() ^ mask) & 63) * 128, 4); });
  return out;
}

inline unsigned __shfl_xor(unsigned v, int mask, int width = 64) {
  (void)width;
  unsigned out;
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b + ((sim_lane() ^ mask) & 63) * 128, 4); });
  return out;
}

template <typename T>
inline T sim_shfl_xor(T v, int mask) {
  T out;
  sim_wave_exchange(&v, sizeof(T), [&](const uint8_t* b) {
    memcpy(&out, b + ((sim_lane() ^ mask) & 63) * 128, sizeof(T));
  });
  return out;
}
inline int __shfl_xor(int v, int mask, int width = 64) { (void)width; return sim_shfl_xor(v, mask); }
inline unsigned long __shfl_xor(unsigned long v, int mask, int width = 64) {
  (void)width;
  return sim_shfl_xor(v, mask);
}
inline unsigned long long __shfl_xor(unsigned long long v, int mask, int width = 64) {
  (void)width;
  return sim_shfl_xor(v, mask);
}

// __shfl_up: lane l reads lane l - delta; lanes below delta keep their own value
inline float __shfl_up(float v, unsigned delta, int width = 64) {
  (void)width;
  float out;
  const int src = sim_lane() >= (int)delta ? sim_lane() - (int)delta : sim_lane();
  sim_wave_exchange(&v, 4, [&](const uint8_t* b) { memcpy(&out, b + src * 128, 4); });
  return out;
}

inline unsigned long long __ballot(int pred) {
  const int mine = pred != 0;
  unsigned long long m = 0;
  sim_wave_exchange(&mine, 4, [&](const uint8_t* b) {
    for (int l = 0; l < 64; ++l) {
      int v;
      memcpy(&v, b + l * 128, 4);
      if (v) m |= 1ull << l;
    }
  });
  return m;
}
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }

// device-scope atomics: workgroups run concurrently on the pool threads
inline unsigned atomicAdd(unsigned* p, unsigned v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
inline int atomicAdd(int* p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }

// ---- scalar helpers ------------------------------------------------------------------
inline float __uint_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float sim_bf16_to_f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
inline uint16_t sim_f_to_bf16(float f) {  // round to nearest even, NaN stays NaN
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
inline float sim_f16_to_f(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) return (s ? -1.f : 1.f) * std::ldexp((float)m, -24);
  if (e == 31) return __uint_as_float(s | 0x7f800000u | (m << 13));
  return __uint_as_float(s | ((e + 112) << 23) | (m << 13));
}
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline float sim_exp2f(float x) { return std::exp2(x); }
#define __builtin_amdgcn_exp2f(x) sim_exp2f(x)
// scheduling hints: no effect on what a kernel computes
#define __builtin_amdgcn_sched_group_barrier(mask, size, id) ((void)0)
#define __builtin_amdgcn_sched_barrier(mask) ((void)0)

// fp32 -> fp16 rounded toward zero (v_cvt_pkrtz_f16_f32), two at a time
typedef _Float16 sim_half2 __attribute__((ext_vector_type(2)));
inline uint16_t sim_f_to_f16_rtz(float f) {
  const uint32_t u = __float_as_uint(f), s = (u >> 16) & 0x8000u;
  const int e = (int)((u >> 23) & 255) - 127 + 15;
  const uint32_t m = u & 0x7fffffu;
  if (((u >> 23) & 255) == 255) return (uint16_t)(s | 0x7c00u | (m ? 0x200u : 0));
  if (e >= 31) return (uint16_t)(s | 0x7bffu);                  // toward zero: largest finite
  if (e <= 0) {                                                  // subnormal or zero
    if (e < -10) return (uint16_t)s;
    return (uint16_t)(s | ((m | 0x800000u) >> (14 - e)));
  }
  return (uint16_t)(s | (e << 10) | (m >> 13));
}
inline sim_half2 sim_cvt_pkrtz(float a, float b) {
  const uint32_t w = (uint32_t)sim_f_to_f16_rtz(a) | ((uint32_t)sim_f_to_f16_rtz(b) << 16);
  return __builtin_bit_cast(sim_half2, w);
}
#define __builtin_amdgcn_cvt_pkrtz(a, b) sim_cvt_pkrtz(a, b)

// ---- MFMA ----------------------------------------------------------------------------
// Operands are 8 16-bit values per lane (bf16 or fp16 bit patterns).
typedef uint16_t sim_h8 __attribute__((ext_vector_type(8)));
typedef float sim_f4 __attribute__((ext_vector_type(4)));
typedef float sim_f16v __attribute__((ext_vector_type(16)));

struct SimMfmaIn {
  uint16_t a[8], b[8];
};

// v_mfma_f32_16x16x32_{bf16,f16}: A 16x32, lane l holds A[l%16][8(l/16) .. +8];
// B 32x16, lane l holds B[8(l/16) .. +8][l%16]; D 16x16, lane l holds
// D[4(l/16) + i][l%16], i = 0..3.
template <bool F16>
inline sim_f4 sim_mfma16(sim_h8 a, sim_h8 b, sim_f4 c) {
  SimMfmaIn in;
  for (int i = 0; i < 8; ++i) in.a[i] = a[i], in.b[i] = b[i];
  sim_f4 d = c;
  sim_wave_exchange(&in, sizeof in, [&](const uint8_t* buf) {
    auto lane_in = [&](int l) { return reinterpret_cast<const SimMfmaIn*>(buf + l * 128); };
    const int l = sim_lane(), col = l & 15;
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * (l >> 4) + i;
      float acc = c[i];
      for (int k = 0; k < 32; ++k) {
        const uint16_t av = lane_in(row + 16 * (k >> 3))->a[k & 7];
        const uint16_t bv = lane_in(col + 16 * (k >> 3))->b[k & 7];
        acc += F16 ? sim_f16_to_f(av) * sim_f16_to_f(bv) : sim_bf16_to_f(av) * sim_bf16_to_f(bv);
      }
      d[i] = acc;
    }
  });
  return d;
}

// v_mfma_f32_32x32x16_{bf16,f16}: A 32x16, lane l holds A[l%32][8(l/32) .. +8];
// B 16x32, lane l holds B[8(l/32) .. +8][l%32]; D 32x32, lane l holds
// D[8(i/4) + 4(l/32) + i%4][l%32], i = 0..15.
template <bool F16>
inline sim_f16v sim_mfma32(sim_h8 a, sim_h8 b, sim_f16v c) {
  SimMfmaIn in;
  for (int i = 0; i < 8; ++i) in.a[i] = a[i], in.b[i] = b[i];
  sim_f16v d = c;
  sim_wave_exchange(&in, sizeof in, [&](const uint8_t* buf) {
    auto lane_in = [&](int l) { return reinterpret_cast<const SimMfmaIn*>(buf + l * 128); };
    const int l = sim_lane(), col = l & 31;
    for (int i = 0; i < 16; ++i) {
      const int row = 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
      float acc = c[i];
      for (int k = 0; k < 16; ++k) {
        const uint16_t av = lane_in(row + 32 * (k >> 3))->a[k & 7];
        const uint16_t bv = lane_in(col + 32 * (k >> 3))->b[k & 7];
        acc += F16 ? sim_f16_to_f(av) * sim_f16_to_f(bv) : sim_bf16_to_f(av) * sim_bf16_to_f(bv);
      }
      d[i] = acc;
    }
  });
  return d;
}

template <typename T>
inline sim_h8 sim_as_h8(T v) { return __builtin_bit_cast(sim_h8, v); }
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, x, y, z) sim_mfma16<false>(sim_as_h8(a), sim_as_h8(b), c)
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, x, y, z) sim_mfma16<true>(sim_as_h8(a), sim_as_h8(b), c)
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) sim_mfma32<false>(sim_as_h8(a), sim_as_h8(b), c)
#define __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, x, y, z) sim_mfma32<true>(sim_as_h8(a), sim_as_h8(b), c)

// ---- vector types ---------------------------------------------------------------------
struct float2 {
  float x, y;
};
inline float2 make_float2(float x, float y) { return float2{x, y}; }

// ---- kernels and launches ------------------------------------------------------------
#define amdgpu_waves_per_eu(...)
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
// LDS objects start 16-byte aligned on the GPU (a kernel's first object at offset
// 0); the simulator gives its thread_local stand-ins the same alignment, which the
// host's 16-byte vector loads and stores need.
#define __shared__ static thread_local __attribute__((aligned(16)))
typedef void* hipStream_t;
typedef int hipError_t;
#define hipSuccess 0
inline int sim_launch_error = 0;
inline hipError_t hipGetLastError() { int e = sim_launch_error; sim_launch_error = 0; return e; }
// Device globals are ordinary host arrays here: one "device", whose symbol
// address is the array's own.
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(sym) (&(sym))
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
  *p = const_cast<void*>(sym);
  return hipSuccess;
}
// Launches run to completion when they are made and nothing is ever captured.
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* s) {
  *s = hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }

// Runs grid x block work-items: the workgroups are shared out over a pool of OS
// threads; a workgroup runs as blockDim fibers on one of them (its __shared__
// statics are thread_local), scheduled round-robin between barriers.
inline void sim_fiber_entry(unsigned lo, unsigned hi) {
  auto* fn = reinterpret_cast<std::function<void()>*>(((uintptr_t)hi << 32) | lo);
  (*fn)();
  sim_blk->cur->done = true;
  swapcontext(&sim_blk->cur->ctx, &sim_blk->sched);
}

template <typename K, typename... A>
inline void sim_launch(K kernel, sim_dim3 grid, sim_dim3 block, A... args) {
  const int nt = (int)(block.x * block.y * block.z);
  if (nt % 64 != 0 || nt > 1024) { sim_launch_error = 1; return; }
  const long long nblocks = (long long)grid.x * grid.y * grid.z;
  std::atomic<long long> next{0};
  auto worker = [&]() {
    SimBlock sb;
    sim_blk = &sb;
    sb.fibers.resize(nt);
    sb.wave.assign(nt / 64, SimBarrier{64, 0, 0});
    sb.xch.assign(nt / 64, std::vector<uint8_t>(64 * 128));
    sb.block = SimBarrier{nt, 0, 0};
    std::function<void()> body = [&]() { kernel(args...); };
    for (long long b; (b = next.fetch_add(1)) < nblocks;) {
      const sim_dim3 bid((unsigned)(b % grid.x), (unsigned)((b / grid.x) % grid.y),
                         (unsigned)(b / ((long long)grid.x * grid.y)));
      for (int t = 0; t < nt; ++t) {
        SimFiber& f = sb.fibers[t];
        f.flat = t;
        f.tid = sim_dim3(t % block.x, (t / block.x) % block.y, t / (block.x * block.y));
        f.bid = bid;
        f.bdim = block;
        f.gdim = grid;
        f.done = false;
        f.wait_gen = nullptr;
        f.stack.resize(256 << 10);
        getcontext(&f.ctx);
        f.ctx.uc_stack.ss_sp = f.stack.data();
        f.ctx.uc_stack.ss_size = f.stack.size();
        f.ctx.uc_link = nullptr;
        const uintptr_t p = reinterpret_cast<uintptr_t>(&body);
        makecontext(&f.ctx, (void (*)())sim_fiber_entry, 2, (unsigned)(p & 0xffffffffu),
                    (unsigned)(p >> 32));
      }
      for (int alive = nt; alive > 0;) {
        alive = 0;
        for (int t = 0; t < nt; ++t) {
          SimFiber& f = sb.fibers[t];
          if (f.done) continue;
          ++alive;
          if (f.wait_gen && *f.wait_gen == f.wait_val) continue;
          f.wait_gen = nullptr;
          sb.cur = &f;
          swapcontext(&sb.sched, &f.ctx);
        }
      }
    }
    sim_blk = nullptr;
  };
  const int nthreads = (int)std::min<long long>(nblocks, 8);
  std::vector<std::thread> th;
  for (int i = 0; i < nthreads; ++i) th.emplace_back(worker);
  for (auto& x : th) x.join();
}
#define hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ...) \
  sim_launch(kernel, sim_dim3(grid), sim_dim3(block), __VA_ARGS__)
