// KV-cache store for gfx950: store_kvcache of mini_vllm/layers/attention.py:59-90
// (one token per slot_mapping entry, slot -1 skipped) for bf16 caches, and the
// FP8 e4m3fn store with a per-tensor scale that the reference loads from an
// external package (attention.py:17-56): code = sat_e4m3fn(x / scale).
//
// One wave per (token, kv head): 64 lanes x 2 elements = 128 head dims, so
// every row is one fully coalesced 256-byte (bf16) or 128-byte (fp8) store.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"
#include "hs_fp8.h"

namespace hs {

struct StoreArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_st, k_sh, v_st, v_sh;
  uint8_t* kc;
  uint8_t* vc;
  int fp8;
  int64_t c_sb, c_st, c_sh;
  float k_scale, v_scale;
  const int32_t* slots;
  int N, Hkv, block_size, num_blocks;
};

template <bool kFp8>
__global__ __launch_bounds__(256) void k_store_kv(StoreArgs a) {
  const int wave = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  if (wave >= a.N * a.Hkv) return;
  const int tok = wave / a.Hkv, h = wave % a.Hkv;
  const int slot = a.slots[tok];
  if (slot < 0) return;
  const int blk = slot / a.block_size, off = slot % a.block_size;
  if (blk >= a.num_blocks) return;
  const int64_t dst = (int64_t)blk * a.c_sb + (int64_t)off * a.c_st + (int64_t)h * a.c_sh + lane * 2;
  const uint32_t kk = *reinterpret_cast<const uint32_t*>(a.k + tok * a.k_st + h * a.k_sh + lane * 2);
  const uint32_t vv = *reinterpret_cast<const uint32_t*>(a.v + tok * a.v_st + h * a.v_sh + lane * 2);
  if constexpr (kFp8) {
    const float k0 = __uint_as_float(kk << 16), k1 = __uint_as_float(kk & 0xffff0000u);
    const float v0 = __uint_as_float(vv << 16), v1 = __uint_as_float(vv & 0xffff0000u);
    const uint16_t kq = (uint16_t)f32_to_e4m3fn_sat(k0 / a.k_scale) |
                        ((uint16_t)f32_to_e4m3fn_sat(k1 / a.k_scale) << 8);
    const uint16_t vq = (uint16_t)f32_to_e4m3fn_sat(v0 / a.v_scale) |
                        ((uint16_t)f32_to_e4m3fn_sat(v1 / a.v_scale) << 8);
    *reinterpret_cast<uint16_t*>(a.kc + dst) = kq;
    *reinterpret_cast<uint16_t*>(a.vc + dst) = vq;
  } else {
    *reinterpret_cast<uint32_t*>(a.kc + dst * 2) = kk;
    *reinterpret_cast<uint32_t*>(a.vc + dst * 2) = vv;
  }
}

}  // namespace hs

using namespace hs;

extern "C" int hs_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                                const void* value, int64_t value_stride_tok,
                                int64_t value_stride_head, void* k_cache, void* v_cache,
                                int kv_dtype, int64_t cache_stride_block,
                                int64_t cache_stride_tok, int64_t cache_stride_head,
                                float k_scale, float v_scale, const int32_t* slot_mapping,
                                int num_tokens, int num_kv_heads, int head_dim, int block_size,
                                int num_blocks, void* stream) {
  if (num_tokens == 0) return HS_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return HS_ERR_INVALID;
  if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || num_blocks <= 0)
    return HS_ERR_INVALID;
  if (head_dim != 128) return HS_ERR_UNSUPPORTED;
  if (kv_dtype != HS_BF16 && kv_dtype != HS_FP8_E4M3) return HS_ERR_INVALID;
  if (kv_dtype == HS_FP8_E4M3 && !(k_scale > 0.0f && v_scale > 0.0f)) return HS_ERR_INVALID;
  if ((key_stride_tok | key_stride_head | value_stride_tok | value_stride_head) & 1)
    return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)key | (uintptr_t)value) & 3) return HS_ERR_UNSUPPORTED;
  if ((cache_stride_block | cache_stride_tok | cache_stride_head) & 1) return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 3) return HS_ERR_UNSUPPORTED;
  StoreArgs a;
  a.k = static_cast<const uint16_t*>(key);
  a.v = static_cast<const uint16_t*>(value);
  a.k_st = key_stride_tok;
  a.k_sh = key_stride_head;
  a.v_st = value_stride_tok;
  a.v_sh = value_stride_head;
  a.kc = static_cast<uint8_t*>(k_cache);
  a.vc = static_cast<uint8_t*>(v_cache);
  a.fp8 = (kv_dtype == HS_FP8_E4M3);
  a.c_sb = cache_stride_block;
  a.c_st = cache_stride_tok;
  a.c_sh = cache_stride_head;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.slots = slot_mapping;
  a.N = num_tokens;
  a.Hkv = num_kv_heads;
  a.block_size = block_size;
  a.num_blocks = num_blocks;
  const int waves = num_tokens * num_kv_heads;
  dim3 grid((waves + 3) / 4);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.fp8)
    hipLaunchKernelGGL(k_store_kv<true>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_store_kv<false>, grid, dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}
