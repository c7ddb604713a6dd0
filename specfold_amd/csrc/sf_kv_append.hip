// In-place KV-cache append: copy the roped k heads and the v heads of n_tok
// consecutive kv_buf rows into cache positions start_pos.., through a page
// table (or a contiguous [Hkv, capacity, hd] cache when page_table is NULL).
//
// Replaces the torch.cat growth DynamicCache.update does in the block-commit
// forward (specfold/model_cache/nemotron_labs_diffusion/modeling_ministral.py:154-162;
// specfold/generate/fastdllm_v2_generation.py:557-575): the result is byte-equal
// to cat(cache, new_rows, dim=-2) read back in logical order, with no O(P) copy.
#include "sf_common.h"

namespace {

constexpr int kHD = 128;

// one thread per 16-byte segment; 16 consecutive threads cover one 256-byte
// (token, head) row, so reads and writes are both full 256 B runs.
__global__ __launch_bounds__(256) void sf_kv_append_kernel(
    const uint16_t* __restrict__ kv_buf, int row0, int n_tok, int Hkv,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ page_table, int page_size, long long page_stride,
    long long head_stride, int start_pos) {
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int total = n_tok * 2 * Hkv * 16;
  if (id >= total) return;
  const int sg = id & 15;
  int rest = id >> 4;
  const int h = rest % Hkv;
  rest /= Hkv;
  const int kv = rest & 1;
  const int t = rest >> 1;
  const sf_u32x4 v = *reinterpret_cast<const sf_u32x4*>(
      kv_buf + (size_t)(row0 + t) * 2 * Hkv * kHD + (kv * Hkv + h) * kHD + sg * 8);
  const int pos = start_pos + t;
  uint16_t* base = kv ? v_cache : k_cache;
  long long off;
  if (page_table) {
    const int lp = pos / page_size;
    off = (long long)page_table[lp] * page_stride + (long long)h * head_stride +
          (long long)(pos - lp * page_size) * kHD;
  } else {
    off = (long long)h * head_stride + (long long)pos * kHD;
  }
  *reinterpret_cast<sf_u32x4*>(base + off + sg * 8) = v;
}

}  // namespace

extern "C" int sf_kv_append(const uint16_t* kv_buf, int row0, int n_tok, int Hkv, int hd,
                            uint16_t* k_cache, uint16_t* v_cache, const int32_t* page_table,
                            int page_size, long long page_stride, long long head_stride,
                            int start_pos, void* stream) {
  if (!kv_buf || !k_cache || !v_cache) return SF_ERR_ARG;
  if (hd != kHD || Hkv < 1 || n_tok < 0 || row0 < 0 || start_pos < 0) return SF_ERR_SHAPE;
  if (page_table && page_size < 1) return SF_ERR_SHAPE;
  if (n_tok == 0) return SF_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int total = n_tok * 2 * Hkv * 16;
  hipLaunchKernelGGL(sf_kv_append_kernel, dim3((total + 255) / 256), dim3(256), 0, st, kv_buf,
                     row0, n_tok, Hkv, k_cache, v_cache, page_table, page_size, page_stride,
                     head_stride, start_pos);
  return sf_launch_status();
}
