// Fused elementwise kernels of the Qwen3 decoder layer around the verify path.
//
// The reference fuses these with torch.compile (mini_vllm/layers/
// layernorm.py:18-36, rotary_embedding.py:8-50, activation.py:8-16); eager
// PyTorch would launch ~45 tiny kernels per layer for them, which at batch 1
// costs more than the layer's GEMMs. One launch each here:
//   hs_rmsnorm       (optional residual add) + RMSNorm, one workgroup per row;
//   hs_qk_norm_rope  per-head RMSNorm of q and k + neox RoPE, one 16-lane row
//                    per (token, head): lane j holds dims 8j .. 8j + 7, all
//                    lane exchanges in DPP;
//   hs_qk_norm_rope_store  the same, with k written straight into its paged
//                    cache slot and v copied there (bf16, or FP8 e4m3fn with a
//                    per-tensor scale), replacing the separate store_kvcache
//                    launch (attention.py:59-90, :145);
//   hs_silu_mul      silu(gate) * up.
// Numerics follow the reference: the residual sum and the normalisation are
// fp32, the normalised value is rounded to bf16 before the weight multiply.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"
#include "hs_fp8.h"
#include "hs_model_dev.h"

namespace hs {

constexpr int kNT = 256;

__device__ __forceinline__ void load4(const uint16_t* p, float (&a)[4]) {
  const uint2 raw = *reinterpret_cast<const uint2*>(p);
  a[0] = bf((uint16_t)raw.x);
  a[1] = bf((uint16_t)(raw.x >> 16));
  a[2] = bf((uint16_t)raw.y);
  a[3] = bf((uint16_t)(raw.y >> 16));
}

// x [rows, H] (row stride xs), residual [rows, H] (rs; may be null), w [H].
// Pass 1 accumulates the sum of squares of the fp32 (x + residual); pass 2
// re-reads the row (cache-resident), stores the bf16 residual and the output.
__global__ __launch_bounds__(kNT) void k_rmsnorm(const uint16_t* __restrict__ x, int64_t xs,
                                                 uint16_t* __restrict__ res, int64_t rs,
                                                 const uint16_t* __restrict__ w,
                                                 uint16_t* __restrict__ out, int64_t os, int H,
                                                 float eps) {
  __shared__ float s_sum[kNT / 64];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const uint16_t* xr = x + row * xs;
  uint16_t* rr = res ? res + row * rs : nullptr;
  uint16_t* orow = out + row * os;
  float ss = 0.0f;
  for (int i = tid * 4; i < H; i += kNT * 4) {
    float a[4], r[4];
    load4(xr + i, a);
    if (rr) {
      load4(rr + i, r);
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] += r[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) ss += a[k] * a[k];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (lane == 0) s_sum[wid] = ss;
  __syncthreads();
  ss = 0.0f;
#pragma unroll
  for (int k = 0; k < kNT / 64; ++k) ss += s_sum[k];
  const float inv = rsqrtf(ss / (float)H + eps);
  for (int i = tid * 4; i < H; i += kNT * 4) {
    float a[4], r[4], wf[4];
    load4(xr + i, a);
    if (rr) {
      load4(rr + i, r);
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] += r[k];
      uint2 nr;
      nr.x = (uint32_t)to_bf(a[0]) | ((uint32_t)to_bf(a[1]) << 16);
      nr.y = (uint32_t)to_bf(a[2]) | ((uint32_t)to_bf(a[3]) << 16);
      *reinterpret_cast<uint2*>(rr + i) = nr;
    }
    load4(w + i, wf);
    uint16_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = to_bf(bf(to_bf(a[k] * inv)) * wf[k]);
    uint2 ov;
    ov.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
    ov.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
    *reinterpret_cast<uint2*>(orow + i) = ov;
  }
}

// One 16-lane row per (token, head), four heads per wave (norm_rope_row's
// layout: lane j of a row holds dims 8j .. 8j + 7, read and written with one
// 16-byte access); heads [0, Hq) are q, [Hq, Hq+Hkv) are k.
__global__ __launch_bounds__(kNT) void k_qk_norm_rope(const uint16_t* __restrict__ qkv, int64_t ts,
                                                      int Hq, int Hkv,
                                                      const uint16_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ kw,
                                                      const float* __restrict__ cos_sin,
                                                      const int64_t* __restrict__ positions,
                                                      float eps, uint16_t* __restrict__ qo,
                                                      uint16_t* __restrict__ ko, int N) {
  const int H = Hq + Hkv;
  const int64_t row = ((int64_t)blockIdx.x * kNT + threadIdx.x) >> 4;
  const int j = threadIdx.x & 15;
  if (row >= (int64_t)N * H) return;  // whole rows: the row's DPP partners are here
  const int tok = (int)(row / H), h = (int)(row % H);
  const bool isq = h < Hq;
  uint16_t xh[8], w[8], y[8];
  unpack8(*reinterpret_cast<const uint4*>(qkv + tok * ts + h * 128 + 8 * j), xh);
  unpack8(*reinterpret_cast<const uint4*>((isq ? qw : kw) + 8 * j), w);
  float x[8], c[8], sn[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = bf(xh[k]);
  load_rot8(cos_sin + positions[tok] * 128, j, c, sn);
  norm_rope_row(x, w, c, sn, eps, j, y);
  uint16_t* dst = isq ? qo + ((int64_t)tok * Hq + h) * 128 : ko + ((int64_t)tok * Hkv + (h - Hq)) * 128;
  *reinterpret_cast<uint4*>(dst + 8 * j) = pack8(y);
}

struct NormRopeStoreArgs {
  const uint16_t* qkv;
  int64_t ts;
  int Hq, Hkv;
  const uint16_t* qw;
  const uint16_t* kw;
  const float* cos_sin;
  const int64_t* positions;
  float eps;
  uint16_t* qo;
  uint8_t* kc;
  uint8_t* vc;
  int64_t c_sb, c_st, c_sh;  // cache strides in elements
  float k_scale, v_scale;
  const int32_t* slots;
  int block_size, num_blocks, N;
};

// One 16-lane row per (token, head) over the q, k and v heads of the fused qkv
// row (four heads per wave, norm_rope_row's layout): q heads are normalised,
// rotated and written to qo; k heads are normalised, rotated and stored at
// the token's cache slot; v heads are stored unchanged. Slots < 0 (and blocks
// beyond num_blocks) store nothing, as store_kvcache.
template <bool kFp8>
__global__ __launch_bounds__(kNT) void k_qk_norm_rope_store(NormRopeStoreArgs a) {
  // the argument block's three 64-byte lines requested together (latency-bound
  // at decode sizes)
  asm volatile("" ::"s"(a.qkv), "s"(a.qo), "s"(a.block_size));
  const int H = a.Hq + 2 * a.Hkv;
  const int64_t row = ((int64_t)blockIdx.x * kNT + threadIdx.x) >> 4;
  const int j = threadIdx.x & 15;
  if (row >= (int64_t)a.N * H) return;  // whole rows: the row's DPP partners are here
  const int tok = (int)(row / H), h = (int)(row % H);
  uint16_t xh[8];
  unpack8(*reinterpret_cast<const uint4*>(a.qkv + tok * a.ts + h * 128 + 8 * j), xh);
  const bool isv = h >= a.Hq + a.Hkv;
  if (isv) {  // v: stored as it is
    const int slot = a.slots[tok];
    if (slot < 0) return;
    const int blk = slot / a.block_size, off = slot % a.block_size;
    if (blk >= a.num_blocks) return;
    const int64_t elem = (int64_t)blk * a.c_sb + (int64_t)off * a.c_st +
                         (int64_t)(h - a.Hq - a.Hkv) * a.c_sh;
    store_row8<kFp8>(a.vc, elem, j, xh, a.v_scale);
    return;
  }
  const bool isq = h < a.Hq;
  uint16_t w[8], y[8];
  unpack8(*reinterpret_cast<const uint4*>((isq ? a.qw : a.kw) + 8 * j), w);
  float x[8], c[8], sn[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = bf(xh[k]);
  load_rot8(a.cos_sin + a.positions[tok] * 128, j, c, sn);
  norm_rope_row(x, w, c, sn, a.eps, j, y);
  if (isq) {
    *reinterpret_cast<uint4*>(a.qo + ((int64_t)tok * a.Hq + h) * 128 + 8 * j) = pack8(y);
    return;
  }
  const int slot = a.slots[tok];
  if (slot < 0) return;
  const int blk = slot / a.block_size, off = slot % a.block_size;
  if (blk >= a.num_blocks) return;
  const int64_t elem = (int64_t)blk * a.c_sb + (int64_t)off * a.c_st + (int64_t)(h - a.Hq) * a.c_sh;
  store_row8<kFp8>(a.kc, elem, j, y, a.k_scale);
}

__global__ __launch_bounds__(kNT) void k_silu_mul(const uint16_t* __restrict__ gu, int64_t gs,
                                                  int F, uint16_t* __restrict__ out, int64_t os,
                                                  int N) {
  const int64_t total = (int64_t)N * (F / 4);
  for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kNT) {
    const int64_t row = i / (F / 4);
    const int c = (int)(i % (F / 4)) * 4;
    const uint2 g = *reinterpret_cast<const uint2*>(gu + row * gs + c);
    const uint2 u = *reinterpret_cast<const uint2*>(gu + row * gs + F + c);
    const uint16_t gv[4] = {(uint16_t)g.x, (uint16_t)(g.x >> 16), (uint16_t)g.y,
                            (uint16_t)(g.y >> 16)};
    const uint16_t uv[4] = {(uint16_t)u.x, (uint16_t)(u.x >> 16), (uint16_t)u.y,
                            (uint16_t)(u.y >> 16)};
    uint16_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = bf(gv[k]);
      const uint16_t sl = to_bf(a / (1.0f + __expf(-a)));  // F.silu in fp32, rounded
      o[k] = bf_mul(sl, uv[k]);
    }
    uint2 ov;
    ov.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
    ov.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
    *reinterpret_cast<uint2*>(out + row * os + c) = ov;
  }
}

}  // namespace hs

using namespace hs;

extern "C" {

int hs_rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
               const void* weight, void* out, int64_t out_stride, int rows, int hidden,
               float eps, void* stream) {
  if (rows == 0) return HS_OK;
  if (!x || !weight || !out || rows < 0 || hidden <= 0) return HS_ERR_INVALID;
  if (hidden % 4) return HS_ERR_UNSUPPORTED;
  if ((x_stride | out_stride | (residual ? residual_stride : 0)) & 3) return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)x | (uintptr_t)out | (uintptr_t)weight | (uintptr_t)residual) & 7)
    return HS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kNT), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), x_stride, static_cast<uint16_t*>(residual),
                     residual_stride, static_cast<const uint16_t*>(weight),
                     static_cast<uint16_t*>(out), out_stride, hidden, eps);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_qk_norm_rope(const void* qkv, int64_t token_stride, int num_q_heads, int num_kv_heads,
                    int head_dim, const void* q_weight, const void* k_weight,
                    const float* cos_sin, const int64_t* positions, float eps, void* q_out,
                    void* k_out, int num_tokens, void* stream) {
  if (num_tokens == 0) return HS_OK;
  if (!qkv || !q_weight || !k_weight || !cos_sin || !positions || !q_out || !k_out ||
      num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0)
    return HS_ERR_INVALID;
  if (head_dim != 128) return HS_ERR_UNSUPPORTED;
  // 16-byte rows: every 8-element piece of a head is one load or store
  if ((token_stride % 8) || (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_out |
                             (uintptr_t)q_weight | (uintptr_t)k_weight | (uintptr_t)cos_sin) & 15))
    return HS_ERR_UNSUPPORTED;
  const int64_t rows = (int64_t)num_tokens * (num_q_heads + num_kv_heads);
  hipLaunchKernelGGL(k_qk_norm_rope, dim3((unsigned)((rows + kNT / 16 - 1) / (kNT / 16))), dim3(kNT), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv),
                     token_stride, num_q_heads, num_kv_heads,
                     static_cast<const uint16_t*>(q_weight),
                     static_cast<const uint16_t*>(k_weight), cos_sin, positions, eps,
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), num_tokens);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_qk_norm_rope_store(const void* qkv, int64_t token_stride, int num_q_heads,
                          int num_kv_heads, int head_dim, const void* q_weight,
                          const void* k_weight, const float* cos_sin, const int64_t* positions,
                          float eps, void* q_out, void* k_cache, void* v_cache, int kv_dtype,
                          int64_t cache_stride_block, int64_t cache_stride_tok,
                          int64_t cache_stride_head, float k_scale, float v_scale,
                          const int32_t* slot_mapping, int block_size, int num_blocks,
                          int num_tokens, void* stream) {
  if (num_tokens == 0) return HS_OK;
  if (!qkv || !q_weight || !k_weight || !cos_sin || !positions || !q_out || !k_cache ||
      !v_cache || !slot_mapping || num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      block_size <= 0 || num_blocks <= 0)
    return HS_ERR_INVALID;
  if (head_dim != 128) return HS_ERR_UNSUPPORTED;
  if (kv_dtype != HS_BF16 && kv_dtype != HS_FP8_E4M3) return HS_ERR_INVALID;
  if (kv_dtype == HS_FP8_E4M3 && !(k_scale > 0.0f && v_scale > 0.0f)) return HS_ERR_INVALID;
  if (token_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * 128) return HS_ERR_INVALID;
  // 16-byte rows (8-byte fp8 rows): every 8-element piece of a head is one load or store
  if ((token_stride % 8) || (cache_stride_block % 8) || (cache_stride_tok % 8) ||
      (cache_stride_head % 8) ||
      (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)q_weight | (uintptr_t)k_weight |
        (uintptr_t)cos_sin) & 15) ||
      (((uintptr_t)k_cache | (uintptr_t)v_cache) & (kv_dtype == HS_BF16 ? 15 : 7)))
    return HS_ERR_UNSUPPORTED;
  NormRopeStoreArgs a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.ts = token_stride;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.cos_sin = cos_sin;
  a.positions = positions;
  a.eps = eps;
  a.qo = static_cast<uint16_t*>(q_out);
  a.kc = static_cast<uint8_t*>(k_cache);
  a.vc = static_cast<uint8_t*>(v_cache);
  a.c_sb = cache_stride_block;
  a.c_st = cache_stride_tok;
  a.c_sh = cache_stride_head;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.slots = slot_mapping;
  a.block_size = block_size;
  a.num_blocks = num_blocks;
  a.N = num_tokens;
  const int64_t rows = (int64_t)num_tokens * (num_q_heads + 2 * num_kv_heads);
  const dim3 grid((unsigned)((rows + kNT / 16 - 1) / (kNT / 16)));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kv_dtype == HS_FP8_E4M3)
    hipLaunchKernelGGL(k_qk_norm_rope_store<true>, grid, dim3(kNT), 0, s, a);
  else
    hipLaunchKernelGGL(k_qk_norm_rope_store<false>, grid, dim3(kNT), 0, s, a);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_silu_mul(const void* gate_up, int64_t gate_up_stride, int ffn, void* out,
                int64_t out_stride, int rows, void* stream) {
  if (rows == 0) return HS_OK;
  if (!gate_up || !out || rows < 0 || ffn <= 0) return HS_ERR_INVALID;
  if (ffn % 4 || (gate_up_stride | out_stride) & 3) return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)gate_up | (uintptr_t)out) & 7) return HS_ERR_UNSUPPORTED;
  const int64_t total = (int64_t)rows * (ffn / 4);
  int64_t blocks = (total + kNT - 1) / kNT;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)blocks), dim3(kNT), 0,
                     reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(gate_up), gate_up_stride, ffn,
                     static_cast<uint16_t*>(out), out_stride, rows);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

}  // extern "C"
