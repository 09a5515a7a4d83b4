// gamma+1-query paged-attention verify kernel for gfx950 (MFMA 16x16x32 bf16).
//
// Replaces the verify branch of Attention.forward,
// mini_vllm/layers/attention.py:145-160 (flash_attn_varlen_func over the
// paged cache with block_table, causal=True, softmax_scale = D^-0.5), and is
// also usable for decode (q_len 1) and prefill (q_len > gamma+1).
//
// Work decomposition: a workgroup (8 waves) owns one (sequence, kv head,
// 16-row query tile, key split). The query tile holds the G = Hq/Hkv query
// heads of up to 16/G consecutive query tokens, so one K/V head is streamed
// once for all of them (GQA). Each wave walks 32-key windows of the split:
//   S^T[32 keys x 16 rows] = K (A operand, 16-byte loads straight from the
//                             paged cache) x Q^T (B operand, registers)
//   online softmax in the S^T layout (one query row per lane column),
//   O^T[128 x 16] += V^T (A operand, from a per-wave transposed LDS tile)
//                    x P^T (B operand: the exp2'd S^T values of the lane),
// so P never leaves registers. Causal alignment is bottom-right: query token
// i of a sequence with Lq queries and Lk keys sees keys 0 .. Lk - Lq + i.
// FP8 (e4m3fn) caches are decoded exactly to bf16 in registers; the per-tensor
// k/v scales are folded into the softmax scale and the output.
// Splits of one query tile are merged by k_attn_combine.
//
// Large launches (enough 32-key windows for every CU) run instead as the
// balanced launch k_verify_attn_sk: one workgroup per CU, each streaming an
// equal share of all windows (the hardware dispatcher left a third of the
// CUs idle between workgroups of the grid above), with 8 kv heads as one
// head per wave over the same windows so each window reads whole cached
// token rows; pieces of tiles shared by two workgroups are merged by
// k_attn_combine_sk.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/hilda_spec.h"
#include "hs_model_dev.h"

namespace hs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kAW = 8;          // waves per workgroup
constexpr int kAT = kAW * 64;   // threads per workgroup
constexpr int kD = 128;         // head dim
constexpr int kWin = 32;        // keys per window
constexpr int kRows = 16;       // query rows per tile
constexpr int kMaxSplit = 4096; // keys per split (block-table prefetch capacity)
constexpr int kBtCap = kMaxSplit / kWin + 2;

struct AttnArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint8_t* kc;
  const uint8_t* vc;
  int fp8;
  int64_t c_sb, c_st, c_sh;  // element strides of the caches
  float v_scale;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_width;   // entries per block-table row
  int num_blocks;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B, Hkv, G, block_size, qtiles, nsplit, split_len;
  int bs_shift;               // log2(block_size) for power-of-two block sizes, else -1
  float scale_log2;          // softmax_scale * k_scale * log2(e)
  uint16_t* out;
  int64_t o_st, o_sh;
  float* part_o;             // [slots, 16, 128]: key splits, or two per balanced workgroup
  float* part_ml;            // [slots, 16, 2]
  int* sk_pre;               // balanced launch: window prefix over the tiles [tiles + 1]
  int* sk_w0;                // balanced launch: first window of each workgroup [nwg + 1]
  int sk_nwg;                // balanced launch: workgroups
  int xcd_pack;              // per-tile grid: only workgroups x % xcd_pack == 0 work
  unsigned* tickets;         // fused kernel: split-merge tickets per (sequence, kv head)
  int contig;                // keys are the call's own unpaged rows (no block table)
};

// The q/k-norm + RoPE + KV-store step run inside the per-tile kernel
// (k_verify_attn_qkv): the fused qkv rows of the call's tokens (token-major,
// the sequences' query tokens in cu_seqlens_q order), the norm weights, the
// RoPE table and the tokens' positions and cache slots.
struct QkvArgs {
  const uint16_t* qkv;
  int64_t ts;                // qkv token stride (elements)
  const uint16_t* qw;
  const uint16_t* kw;
  const float* cos_sin;      // [max_position, 128]: cos | sin
  const int64_t* positions;
  const int32_t* slots;
  float eps;
  float k_scale, v_scale;    // store scales (fp8 caches)
  int Hq;
  int cs_rows;               // rows of cos_sin
};

// block of a key position: a shift for power-of-two block sizes, a division
// (several dependent scalar and VALU steps) otherwise
__device__ __forceinline__ int key_block(int key, int bs_shift, int block_size) {
  return bs_shift >= 0 ? key >> bs_shift : key / block_size;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));  // v_cvt_pk_bf16_f32
}

// 8 fp8 e4m3fn bytes -> 8 bf16 (exact: every e4m3fn value is a bf16 value)
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16(uint2 raw) {
  union {
    uint32_t u[4];
    bf16x8_t v;
  } r;
  const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw.x, false);
  const auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw.x, true);
  const auto c = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw.y, false);
  const auto d = __builtin_amdgcn_cvt_pk_f32_fp8((int)raw.y, true);
  r.u[0] = (__float_as_uint(a[0]) >> 16) | (__float_as_uint(a[1]) & 0xffff0000u);
  r.u[1] = (__float_as_uint(b[0]) >> 16) | (__float_as_uint(b[1]) & 0xffff0000u);
  r.u[2] = (__float_as_uint(c[0]) >> 16) | (__float_as_uint(c[1]) & 0xffff0000u);
  r.u[3] = (__float_as_uint(d[0]) >> 16) | (__float_as_uint(d[1]) & 0xffff0000u);
  return r.v;
}

__device__ __forceinline__ bf16x8_t u4_to_bf16x8(uint4 u) {
  union {
    uint4 u;
    bf16x8_t v;
  } r;
  r.u = u;
  return r.v;
}

// 8 consecutive head-dim elements of one cached token as bf16x8
template <bool kFp8>
__device__ __forceinline__ bf16x8_t load_kv8(const uint8_t* base, int64_t elem_off) {
  if constexpr (kFp8) {
    const uint2 raw = *reinterpret_cast<const uint2*>(base + elem_off);
    return fp8x8_to_bf16(raw);
  } else {
    const uint4 raw = *reinterpret_cast<const uint4*>(base + elem_off * 2);
    return u4_to_bf16x8(raw);
  }
}

// LDS layout of one window tile: kWin cached head rows, one row per key, with
// the 16-byte chunks of row kk stored at chunk index (c ^ swz(kk)) so that the
// MFMA operand reads below are free of bank conflicts.
//   bf16 rows (256 B, 16 chunks): K reads touch keys 8a+4kb+c (a, c = 0..3)
//     at one chunk; V transpose reads touch keys 8g+4h+q (q = 0..3) at two
//     adjacent chunks.
//   fp8 rows (128 B, 8 chunks): rows of equal parity share a bank half; K
//     reads touch keys 8a+4kb+{c, c+2}, V transpose reads keys 8g+{0,2,4,6}.
__device__ __forceinline__ int swz16(int kk) {
  return ((kk & 3) << 1) | ((kk >> 3) & 1) | (((kk >> 4) & 1) << 3);
}
__device__ __forceinline__ int swz8(int kk) {
  return ((kk >> 1) & 1) | ((((kk >> 2) ^ (kk >> 3)) & 1) << 1) | (((kk >> 4) & 1) << 2);
}

// Max / sum over the four lanes n, n+16, n+32, n+48 of a row with the gfx950
// lane-swap moves (v_permlane16_swap / v_permlane32_swap: each returns the
// register with one 16- or 32-lane half exchanged, so the pair holds both
// partners' values) instead of LDS-routed shuffles.
__device__ __forceinline__ float row4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef int v2i32_t __attribute__((ext_vector_type(2)));
#define HS_LDS __attribute__((address_space(3)))

// Per-lane byte offsets of a wave's window loads, the same for every window
// of the wave (computed once): instruction i of a tile covers rows kk = i * R
// + lane / L (R rows of L lanes each, 16 bytes per lane); `off` is the
// lane's chunk of row kk (its swizzled position in the tile) and `off0` the
// same chunk of row 0, the stand-in for rows past `hi`. The host keeps 32
// token rows of the cache within 2 GiB.
template <bool kFp8>
struct WinOffs {
  static constexpr int kLanesPerRow = (kFp8 ? 128 : 256) / 16;
  static constexpr int kRowsPerInst = 64 / kLanesPerRow;
  static constexpr int kInst = kWin / kRowsPerInst;
  uint32_t off[kInst], off0[kInst];
  int lrow;  // lane / kLanesPerRow
};

template <bool kFp8>
__device__ __forceinline__ WinOffs<kFp8> win_offs(const AttnArgs& a, int lane) {
  using W = WinOffs<kFp8>;
  const int esz = kFp8 ? 1 : 2;
  W w;
  w.lrow = lane / W::kLanesPerRow;
  const int sl = lane % W::kLanesPerRow;
#pragma unroll
  for (int i = 0; i < W::kInst; ++i) {
    const int kk = i * W::kRowsPerInst + w.lrow;
    const uint32_t c16 = (uint32_t)(sl ^ (kFp8 ? swz8(kk) : swz16(kk))) * 16u;
    w.off[i] = (uint32_t)(kk * a.c_st * esz) + c16;
    w.off0[i] = c16;
  }
  return w;
}

// Copies the K and V rows of one 32-key window into the wave's LDS tiles with
// global->LDS loads (16 bytes per lane, each instruction covering whole rows).
// Keys at or past `hi` re-read key ws (always valid) so every tile row holds
// finite cache data; their scores are masked to -inf.
template <bool kFp8>
__device__ __forceinline__ void issue_window(const uint8_t* kbase, const uint8_t* vbase, int ws,
                                             int hi, uint8_t* tile_k, uint8_t* tile_v,
                                             const WinOffs<kFp8>& wo) {
  using W = WinOffs<kFp8>;
  const int lim = hi - ws;  // rows of the window below hi
#pragma unroll
  for (int i = 0; i < W::kInst; ++i) {
    const uint32_t off = (i * W::kRowsPerInst + wo.lrow < lim) ? wo.off[i] : wo.off0[i];
    __builtin_amdgcn_global_load_lds(kbase + off, (HS_LDS void*)(tile_k + i * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(vbase + off, (HS_LDS void*)(tile_v + i * 1024), 16, 0, 0);
  }
}

// One tile (K or V) of issue_window: its 8 (bf16) or 4 (fp8) loads.
template <bool kFp8>
__device__ __forceinline__ void issue_tile(const uint8_t* base, int ws, int hi, uint8_t* tile,
                                           const WinOffs<kFp8>& wo) {
  using W = WinOffs<kFp8>;
  const int lim = hi - ws;
#pragma unroll
  for (int i = 0; i < W::kInst; ++i) {
    const uint32_t off = (i * W::kRowsPerInst + wo.lrow < lim) ? wo.off[i] : wo.off0[i];
    __builtin_amdgcn_global_load_lds(base + off, (HS_LDS void*)(tile + i * 1024), 16, 0, 0);
  }
}

// 8 fp8 e4m3fn values held as two dwords -> bf16x8
__device__ __forceinline__ bf16x8_t fp8x8w_to_bf16(uint32_t lo, uint32_t hi) {
  return fp8x8_to_bf16(make_uint2(lo, hi));
}

// One query tile: sequence b, kv head kvh, query tile qt (rows qt*16 ..
// qt*16 + 15 of the sequence's Lq * G (token, head) rows), with the
// sequence's query start qs and lengths.
struct TileRef {
  int b, kvh, qt, qs, Lq, Lk, rows;
  int ks;  // first key row of the sequence (unpaged keys, AttnArgs::contig)
};

// from the sequence's bounds cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
__device__ __forceinline__ TileRef tile_ref_of(int b, int kvh, int qt, int G, int q0, int q1,
                                               int k0, int k1) {
  TileRef t;
  t.b = b;
  t.kvh = kvh;
  t.qt = qt;
  t.qs = q0;
  t.Lq = q1 - q0;
  t.Lk = k1 - k0;
  t.rows = t.Lq * G;
  t.ks = k0;
  return t;
}
__device__ __forceinline__ TileRef tile_ref(const AttnArgs& a, int b, int kvh, int qt, int G) {
  return tile_ref_of(b, kvh, qt, G, a.cu_q[b], a.cu_q[b + 1], a.cu_k[b], a.cu_k[b + 1]);
}

// keys of the sequence visible to the tile's last row (0 for an empty tile)
__device__ __forceinline__ int tile_keys(const TileRef& t, int G) {
  const int r0 = t.qt * kRows;
  if (r0 >= t.rows || t.Lk <= 0) return 0;
  const int last_row = (r0 + kRows - 1 < t.rows - 1) ? r0 + kRows - 1 : t.rows - 1;
  const int lim = t.Lk - t.Lq + last_row / G + 1;
  const int hi = lim < t.Lk ? lim : t.Lk;
  return hi > 0 ? hi : 0;
}

// LDS of the per-wave window tiles: the K tiles of the 8 waves in one array,
// their V tiles in another (so the compiler tells a wave's K loads from its V
// loads and waits for each on its own). After the key loop a wave's partial
// output (16 rows x 128 floats, 8 KB) goes into its K tile (bf16), or into
// 8 KB slots over both arrays (fp8 tiles are 4 KB).
template <bool kFp8>
struct AttnLds {
  static constexpr int kRowB = kFp8 ? 128 : 256;
  static constexpr int kTileB = kWin * kRowB;
  static constexpr int kArrB = kAW * kTileB;  // bytes of each of the K and V arrays
};

// wave w's partial output in the tile arrays
template <bool kFp8>
__device__ __forceinline__ float* wave_part(uint8_t* s_kt, uint8_t* s_vt, int w) {
  constexpr int kTileB = AttnLds<kFp8>::kTileB;
  constexpr int kPartB = kRows * kD * 4;
  if constexpr (kTileB >= kPartB)
    return reinterpret_cast<float*>(s_kt + w * kTileB);
  else
    return reinterpret_cast<float*>(w < kAW / 2 ? s_kt + w * kPartB : s_vt + (w - kAW / 2) * kPartB);
}
// float offset of (row, 4-float group c4) in a partial: groups XOR-swizzled by
// the row, so the MFMA-layout writes (16 rows at one group) and the merge's
// row reads hit distinct banks
__device__ __forceinline__ int part_off(int row, int c4) { return row * kD + ((c4 ^ row) << 2); }

// Running softmax state of one wave: per query row (lane column n) the max
// (log2 domain) and the sum of the lane's exp2 terms, and O^T in the MFMA
// accumulator layout (lane holds O[row n][d = db*16 + 4g + j]).
struct WaveAcc {
  float m, lsum;
  f32x4_t oacc[8];
};

// The q/k-norm + RoPE of the fused kernel's (sequence, kv head) tile, in
// norm_rope_row's layout (one 16-lane row per head, lane j holding dims 8j ..
// 8j + 7, so the bits equal hs_qk_norm_rope_store's): the tile's q rows go to
// s_q (16 rows x 128 bf16), the kv head's k and v rows of the sequence's query
// tokens to s_new (token i's rows laid out as the tile row of key Lk - Lq + i,
// the cache's bytes: bf16, or the e4m3fn codes the store writes) and to the
// registers from which kv_store_all writes them to their cache slots (slots <
// 0 and blocks past num_blocks store nothing). The host runs this only when
// one workgroup holds every query row of the (sequence, kv head), so no other
// workgroup of the split reads these rows.
// Heads are wave items of 4 rows: the q rows first, then the k rows, then the
// v rows of the query tokens, each kind from a wave boundary on; prologue
// wave p takes items p, p + 4 and p + 8 (three rounds cover 16 q rows and the
// k and v rows of 16 tokens). qkv_load issues every load of the wave's rows as
// soon as the sequence bounds are known, each piece of a head one 16-byte
// load; the cos/sin row is fetched at
// the position the token holds in its sequence (Lk - Lq + i, clamped into the
// table) together with positions[], and fetched again in qkv_compute where
// positions[] says otherwise.
constexpr int kPW = 4;  // prologue waves of the fused kernel
constexpr int kQkvRounds = 3;
constexpr int kQkvT = (kAW + kPW) * 64;  // threads of a fused workgroup
struct QkvRow {
  int kind;  // 0: q row, 1: k of a token, 2: v of a token, -1: none
  int idx;   // q row of the tile, or query token
  int tok;   // token of the call
};
struct QkvLoads {
  QkvRow row[kQkvRounds];
  int64_t pos[kQkvRounds];
  int guess[kQkvRounds], slot[kQkvRounds];
  uint4 x[kQkvRounds];
  uint4 wq, wk;  // the lane's pieces of the q and k norm weights
  float c[kQkvRounds][8], sn[kQkvRounds][8];
};

// the row of lane `lane` in wave item wi (4 rows per item)
__device__ __forceinline__ QkvRow qkv_row(const TileRef& t, int nrows, int wi, int lane) {
  const int wq = (nrows + 3) / 4, wk = (t.Lq + 3) / 4;
  QkvRow r;
  r.kind = -1;
  r.idx = 0;
  r.tok = t.qs;
  int k, base, count;
  if (wi < wq) {
    k = 0, base = 0, count = nrows;
  } else if (wi < wq + wk) {
    k = 1, base = wq, count = t.Lq;
  } else if (wi < wq + 2 * wk) {
    k = 2, base = wq + wk, count = t.Lq;
  } else {
    return r;
  }
  const int i = 4 * (wi - base) + (lane >> 4);
  if (i >= count) return r;
  r.kind = k;
  r.idx = i;
  return r;
}

__device__ __forceinline__ void qkv_load(const AttnArgs& a, const QkvArgs& qa, const TileRef& t,
                                         int kvh, int G, int pw, QkvLoads& L) {
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int nrows = t.rows < kRows ? t.rows : kRows;
  const int items = (nrows + 3) / 4 + 2 * ((t.Lq + 3) / 4);
  // the norm weights' pieces of this lane, once for every round
  L.wq = *reinterpret_cast<const uint4*>(qa.qw + 8 * j);
  L.wk = *reinterpret_cast<const uint4*>(qa.kw + 8 * j);
  // An item holds rows of one kind, so the round's branches are the wave's;
  // within an item a lane without a row loads the item's first row, so every
  // load of the round goes out before the first wait.
#pragma unroll
  for (int i = 0; i < kQkvRounds; ++i) {
    QkvRow r = qkv_row(t, nrows, pw + kPW * i, lane);
    L.row[i] = r;
    if (pw + kPW * i >= items) continue;
    // lane 0 holds the item's first row
    const int kind = __builtin_amdgcn_readfirstlane(r.kind);
    const int idx = r.kind < 0 ? 0 : r.idx;
    const int qi = kind == 0 ? idx / G : idx;
    const int tok = t.qs + qi;
    L.row[i].tok = tok;
    const int head = kind == 0 ? kvh * G + idx % G : qa.Hq + (kind == 2 ? a.Hkv : 0) + kvh;
    L.x[i] = *reinterpret_cast<const uint4*>(qa.qkv + (int64_t)tok * qa.ts + (int64_t)head * kD + 8 * j);
    if (kind != 0) L.slot[i] = qa.slots[tok];
    if (kind != 2) {
      L.pos[i] = qa.positions[tok];
      int g = t.Lk - t.Lq + qi;
      g = g < 0 ? 0 : (g >= qa.cs_rows ? qa.cs_rows - 1 : g);
      L.guess[i] = g;
      load_rot8(qa.cos_sin + (int64_t)g * kD, j, L.c[i], L.sn[i]);
    }
  }
}

// The cache stores of the wave's k/v rows: element offset of the row (-1:
// nothing to store), the cache, and the lane's 8 bf16 values.
struct KvStores {
  int64_t elem[kQkvRounds];
  bool isv[kQkvRounds];
  uint16_t h[kQkvRounds][8];
};

// byte offset of dims 8j .. 8j + 7 of a tile row for window row kk (the
// tile's 16-byte chunk swizzle; 8 fp8 codes are half a chunk)
template <bool kFp8>
__device__ __forceinline__ int tile_piece(int kk, int j) {
  if constexpr (kFp8)
    return (((j >> 1) ^ swz8(kk)) << 4) | ((j & 1) << 3);
  else
    return (j ^ swz16(kk)) << 4;
}

template <bool kFp8>
__device__ __forceinline__ void qkv_compute(const AttnArgs& a, const QkvArgs& qa, const TileRef& t,
                                            int kvh, QkvLoads& L, uint16_t* s_q, uint8_t* s_new,
                                            KvStores& S) {
  constexpr int kRowB = AttnLds<kFp8>::kRowB;
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int knew = t.Lk - t.Lq;
  // nothing computed from the loaded positions moves above this point (the
  // compiler would otherwise compare them with the guesses right after the
  // loads and wait there, before the next round's loads go out)
#pragma unroll
  for (int i = 0; i < kQkvRounds; ++i) asm volatile("" : "+v"(L.pos[i]), "+v"(L.guess[i]));
#pragma unroll
  for (int i = 0; i < kQkvRounds; ++i) {
    S.elem[i] = -1;
    S.isv[i] = false;
    const QkvRow r = L.row[i];
    if (r.kind < 0) continue;
    uint16_t xh[8], y[8];
    unpack8(L.x[i], xh);
    if (r.kind != 2) {
      if (L.pos[i] != L.guess[i])  // the token sits elsewhere than its key index
        load_rot8(qa.cos_sin + L.pos[i] * kD, j, L.c[i], L.sn[i]);
      uint16_t w[8];
      unpack8(r.kind == 0 ? L.wq : L.wk, w);
      float x[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = bf(xh[k]);
      norm_rope_row(x, w, L.c[i], L.sn[i], qa.eps, j, y);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) y[k] = xh[k];
    }
    if (r.kind == 0) {
      *reinterpret_cast<uint4*>(s_q + r.idx * kD + 8 * j) = pack8(y);
      continue;
    }
    // token r.idx's k or v row as the tile row of key knew + r.idx (the fast
    // case needs Lq <= kRows)
    if (r.idx < kRows) {
      const int kk = (knew + r.idx) & (kWin - 1);
      uint8_t* dst = s_new + (r.kind == 2 ? kRows * kRowB : 0) + r.idx * kRowB + tile_piece<kFp8>(kk, j);
      if constexpr (kFp8)
        *reinterpret_cast<uint2*>(dst) = e4m3x8_of_bf16(y, r.kind == 2 ? qa.v_scale : qa.k_scale);
      else
        *reinterpret_cast<uint4*>(dst) = pack8(y);
    }
    // store_kvcache semantics: slots < 0 and blocks past num_blocks store nothing
    if (L.slot[i] >= 0) {
      const int blk = L.slot[i] / a.block_size, off = L.slot[i] % a.block_size;
      if (blk < a.num_blocks)
        S.elem[i] = (int64_t)blk * a.c_sb + (int64_t)off * a.c_st + (int64_t)kvh * a.c_sh;
    }
    S.isv[i] = r.kind == 2;
#pragma unroll
    for (int k = 0; k < 8; ++k) S.h[i][k] = y[k];
  }
}

template <bool kFp8>
__device__ __forceinline__ void kv_store_all(const AttnArgs& a, const QkvArgs& qa,
                                             const KvStores& S) {
  const int j = threadIdx.x & 15;
#pragma unroll
  for (int i = 0; i < kQkvRounds; ++i) {
    if (S.elem[i] >= 0)
      store_row8<kFp8>(const_cast<uint8_t*>(S.isv[i] ? a.vc : a.kc), S.elem[i], j, S.h[i],
                       S.isv[i] ? qa.v_scale : qa.k_scale);
  }
}

// Workgroup barrier that orders LDS only: global loads and stores in flight
// stay in flight (a plain __syncthreads waits for all of them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool kFp8, bool kNew>
__device__ __forceinline__ const uint8_t* window_row(const uint8_t* tile, const uint8_t* nrow, int ws,
                                                     int knew, int nlast, int kk) {
  constexpr int kRowB = AttnLds<kFp8>::kRowB;
  if constexpr (kNew) {
    const int r = ws + kk - knew;
    return r >= 0 ? nrow + (r < nlast ? r : nlast) * kRowB : tile + kk * kRowB;
  } else {
    return tile + kk * kRowB;
  }
}

// K of window ws as the A operand of S^T (row rho = n holds key ws + 8*(n/4)
// + 4*kb + (n%4)), from the wave's K tile or, kNew, the new-key rows.
template <bool kFp8, bool kNew>
__device__ __forceinline__ void read_k(const uint8_t* tile_k, const uint8_t* nk, int ws, int knew,
                                       int nlast, int lane, bf16x8_t (&ka)[2][4]) {
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int kk = 8 * (n >> 2) + 4 * kb + (n & 3);
    const uint8_t* row = window_row<kFp8, kNew>(tile_k, nk, ws, knew, nlast, kk);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      if constexpr (kFp8) {
        const int u = g + 4 * ds;  // 8-byte unit of dims 8g + 32ds
        const int ph = (((u >> 1) ^ swz8(kk)) << 4) | ((u & 1) << 3);
        const uint2 raw = *reinterpret_cast<const uint2*>(row + ph);
        ka[kb][ds] = fp8x8w_to_bf16(raw.x, raw.y);
      } else {
        const int ph = ((g + 4 * ds) ^ swz16(kk)) << 4;
        ka[kb][ds] = u4_to_bf16x8(*reinterpret_cast<const uint4*>(row + ph));
      }
    }
  }
}

// V^T of window ws as the A operand of d-block db (lane (n, g) holds
// V[8g .. 8g+7][16db + n]), gathered with transposing LDS reads.
template <bool kFp8, bool kNew>
__device__ __forceinline__ void read_v(const uint8_t* tile_v, const uint8_t* nv, int ws, int knew,
                                       int nlast, int lane, bf16x8_t (&va)[8]) {
  constexpr int kRowB = AttnLds<kFp8>::kRowB;
  (void)kRowB;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    if constexpr (kFp8) {
      const int kk = 8 * g + (n >> 1);
      const int ph = ((db ^ swz8(kk)) << 4) | ((n & 1) << 3);
      const v2i32_t t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (HS_LDS v2i32_t*)(window_row<kFp8, kNew>(tile_v, nv, ws, knew, nlast, kk) + ph));
      va[db] = fp8x8w_to_bf16((uint32_t)t[0], (uint32_t)t[1]);
    } else {
      union {
        v4i16_t h[2];
        bf16x8_t v;
      } u;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kk = 8 * g + 4 * h + (n >> 2);
        const int ph = (((2 * db + ((n & 3) >> 1)) ^ swz16(kk)) << 4) | ((n & 1) << 3);
        u.h[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (HS_LDS v4i16_t*)(window_row<kFp8, kNew>(tile_v, nv, ws, knew, nlast, kk) + ph));
      }
      va[db] = u.v;
    }
  }
}

// Reads window ws (keys ws .. ws + 31) from the wave's LDS tiles into the
// MFMA operand registers (read_k and read_v). kNew: the rows of keys at or
// past knew come from the new-key rows nk / nv instead (row key - knew, laid
// out as the tile row of that key; masked keys past the last new row nlast
// read that row: finite data weighted 0).
template <bool kFp8, bool kNew>
__device__ __forceinline__ void window_read(const uint8_t* tile_k, const uint8_t* tile_v,
                                            const uint8_t* nk, const uint8_t* nv, int ws,
                                            int knew, int nlast, int lane, bf16x8_t (&ka)[2][4],
                                            bf16x8_t (&va)[8]) {
  read_k<kFp8, kNew>(tile_k, nk, ws, knew, nlast, lane, ka);
  read_v<kFp8, kNew>(tile_v, nv, ws, knew, nlast, lane, va);
}

// A row's scores are exponentiated against a reference that trails its
// running max by at most 2^kRefSlack (log2 units): O and the sum are rescaled
// only when some row's max passes its reference by more, which after the
// first window is rare. The normalised output is the same softmax.
constexpr float kRefSlack = 8.0f;

// One window's contribution to the wave's running softmax state, in two
// steps: mma_s, S^T = K Q^T for the two 16-key blocks, the keys at or past
// hi, past the row's last visible key lim_r and the rows past the tile
// masked, the reference update (m, the row's reference in scaled log2 units)
// and P^T = exp2(S^T scale - m) in bf16; mma_pv, O^T += V^T P^T with P^T from
// registers.
__device__ __forceinline__ bf16x8_t mma_s(const AttnArgs& a, int ws, int hi, int lim_r, bool r_ok,
                                          int kfull, int lane, const bf16x8_t (&ka)[2][4],
                                          const bf16x8_t (&qv)[4], float& m, float& lsum,
                                          f32x4_t (&oacc)[8]) {
  const int g = lane >> 4;
  // keys below kfull are below hi and visible to every row of the tile: a
  // window of such keys needs no mask (rows past the tile hold zero queries,
  // finite scores, and are never written out)
  const bool full = ws + kWin <= kfull;
  f32x4_t st[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kb][ds], qv[ds], acc, 0, 0, 0);
    st[kb] = acc;
  }
  // lane holds row n, keys ws + 8g + 4kb + j (raw scores)
  float sv[8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 4; ++j) sv[kb * 4 + j] = st[kb][j];
  if (!full) {
    // a branch of its own (the empty asm keeps the compiler from computing
    // the mask for every window and selecting)
    asm volatile("; masked window");
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = ws + 8 * g + 4 * kb + j;
        if (!r_ok || key >= hi || key > lim_r) sv[kb * 4 + j] = -INFINITY;
      }
  }
  float mloc = -INFINITY;
#pragma unroll
  for (int t = 0; t < 8; ++t) mloc = fmaxf(mloc, sv[t]);
  mloc = row4_max(mloc) * a.scale_log2;  // the softmax scale is positive
  const bool up = mloc > m + kRefSlack;
  if (__builtin_amdgcn_ballot_w64(up)) {
    const float m_new = up ? mloc : m;
    // a row whose reference is still -inf has seen no key: its sums are exact
    // zeros and need no rescale (the first window of every wave)
    if (__builtin_amdgcn_ballot_w64(up && m != -INFINITY)) {
      const float alpha = (m_new == m) ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 8; ++db) oacc[db] *= alpha;
    }
    m = m_new;
  }
  const float base = (m == -INFINITY) ? 0.0f : m;
  float psum = 0.0f;
  union {
    uint16_t h[8];
    bf16x8_t v;
  } pb;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[t], a.scale_log2, -base));
    psum += p;
    pb.h[t] = f32_to_bf16_rne(p);
  }
  lsum += psum;
  return pb.v;
}

// O^T[d][row] += V^T[d][keys 8g..8g+7] * P^T
__device__ __forceinline__ void mma_pv(const bf16x8_t (&va)[8], bf16x8_t pb, f32x4_t (&oacc)[8]) {
#pragma unroll
  for (int db = 0; db < 8; ++db)
    oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db], pb, oacc[db], 0, 0, 0);
}

__device__ __forceinline__ void window_mma(const AttnArgs& a, int ws, int hi, int lim_r, bool r_ok,
                                           int kfull, int lane, const bf16x8_t (&ka)[2][4],
                                           const bf16x8_t (&va)[8], const bf16x8_t (&qv)[4],
                                           float& m, float& lsum, f32x4_t (&oacc)[8]) {
  const bf16x8_t pb = mma_s(a, ws, hi, lim_r, r_ok, kfull, lane, ka, qv, m, lsum, oacc);
  mma_pv(va, pb, oacc);
}

// Walks keys [lo, hi) of query tile t (hi clipped to the keys the tile's
// last row sees) against kv head kvh in this wave: 32-key windows ws0,
// ws0 + step, ... below hi, the next window's K/V rows in flight while the
// current one is multiplied. Loads the wave's query rows, then waits at a
// workgroup barrier for s_bt: the block-table entries of the sequence from
// block lo / block_size on, up to bt_cap of them, filled by the caller.
// kG: query heads per KV head as a compile-time constant (2, 4 or 8), or 0 to
// read it from the arguments (any other group size).
template <bool kFp8, int kG>
__device__ __forceinline__ void wave_walk(const AttnArgs& a, const TileRef& t, int kvh, int lo,
                                          int hi, int ws0, int step, const int* s_bt, int bt_cap,
                                          uint8_t* tile_k, uint8_t* tile_v, WaveAcc& acc) {
  const int G = kG ? kG : a.G;
  const int qs = t.qs, Lq = t.Lq, Lk = t.Lk, rows = t.rows;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;  // query row of this lane (B-operand column)
  const int g = lane >> 4;  // k-group of this lane
  const int r0 = t.qt * kRows;
  const int bt0 = key_block(lo, a.bs_shift, a.block_size);
  const int nbt_used = (hi > lo) ? key_block(hi - 1, a.bs_shift, a.block_size) - bt0 + 1 : 0;

  // query row of this lane
  const int r = r0 + n;
  const bool r_ok = r < rows;
  const int qi = r_ok ? r / G : 0;
  const int qh = kvh * G + (r_ok ? r % G : 0);
  const int lim_r = Lk - Lq + qi;  // last visible key of this row
  // keys below kfull: visible to every row of the tile, below hi
  const int kfull = min(hi, Lk - Lq + r0 / G + 1);
  bf16x8_t qv[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    if (r_ok) {
      const uint16_t* qp =
          a.q + (int64_t)(qs + qi) * a.q_st + (int64_t)qh * a.q_sh + ds * 32 + g * 8;
      qv[ds] = u4_to_bf16x8(*reinterpret_cast<const uint4*>(qp));
    } else {
      qv[ds] = u4_to_bf16x8(make_uint4(0, 0, 0, 0));
    }
  }

  float m = -INFINITY, lsum = 0.0f;
  f32x4_t oacc[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) oacc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int esz = kFp8 ? 1 : 2;
  __syncthreads();  // s_bt ready

  // window ws of this wave -> cache row bases (bytes) of its K and V head rows;
  // false when its block is not a valid cache block (the window is skipped)
  auto window_base = [&](int ws, const uint8_t*& kb, const uint8_t*& vb) -> bool {
    if (a.contig) {  // unpaged keys: row ks + key of the [tokens, Hkv, 128] k / v
      const int64_t off = ((int64_t)(t.ks + ws) * a.c_st + (int64_t)kvh * a.c_sh) * esz;
      kb = a.kc + off;
      vb = a.vc + off;
      return true;
    }
    const int blk_idx = key_block(ws, a.bs_shift, a.block_size);
    const int bi = blk_idx - bt0;
    const int blk = (bi < nbt_used && bi < bt_cap && bt0 + bi < a.bt_width) ? s_bt[bi] : -1;
    if (blk < 0 || blk >= a.num_blocks) return false;
    const int64_t off = ((int64_t)blk * a.c_sb + (int64_t)(ws - blk_idx * a.block_size) * a.c_st +
                         (int64_t)kvh * a.c_sh) * esz;
    kb = a.kc + off;
    vb = a.vc + off;
    return true;
  };

  const WinOffs<kFp8> wo = win_offs<kFp8>(a, lane);
  int ws = ws0;
  bool have = false;
  if (ws < hi) {
    const uint8_t *kb, *vb;
    have = window_base(ws, kb, vb);
    if (have) issue_window<kFp8>(kb, vb, ws, hi, tile_k, tile_v, wo);
  }
  while (ws < hi) {
    const int ws_next = ws + step;
    const bool cur = have;
    bf16x8_t ka[2][4], va[8];
    if (cur) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      window_read<kFp8, false>(tile_k, tile_v, nullptr, nullptr, ws, 0, 0, lane, ka, va);
      // every LDS read of the tiles has returned before the next window overwrites them
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    have = false;
    if (ws_next < hi) {
      const uint8_t *kb, *vb;
      have = window_base(ws_next, kb, vb);
      if (have) issue_window<kFp8>(kb, vb, ws_next, hi, tile_k, tile_v, wo);
    }
    if (cur) window_mma(a, ws, hi, lim_r, r_ok, kfull, lane, ka, va, qv, m, lsum, oacc);
    ws = ws_next;
  }
  // per-row totals of this wave
  lsum = row4_sum(lsum);
  acc.m = m;
  acc.lsum = lsum;
#pragma unroll
  for (int db = 0; db < 8; ++db) acc.oacc[db] = oacc[db];
}

// Merge of the 8 waves' partials for one query row and dims d0 .. d0 + 3:
// running max M, sum L and unnormalised output o. Every wave's state is
// there: a wave that held no keys has max -inf, sum 0 and output 0, so its
// weight exp2(-inf - M) is 0. Waves in order, so every kernel sharing it
// gives the same bits. s_m / s_l: [row][wave]; wave w's partial at wave_part.
template <bool kFp8>
__device__ __forceinline__ void merge_waves(const float (*s_m)[kAW], const float (*s_l)[kAW],
                                            uint8_t* s_kt, uint8_t* s_vt, int row, int c4,
                                            float& M, float& L, float (&o)[4]) {
  const float4 m0 = *reinterpret_cast<const float4*>(&s_m[row][0]);
  const float4 m1 = *reinterpret_cast<const float4*>(&s_m[row][4]);
  const float4 l0 = *reinterpret_cast<const float4*>(&s_l[row][0]);
  const float4 l1 = *reinterpret_cast<const float4*>(&s_l[row][4]);
  float4 x[kAW];
#pragma unroll
  for (int w = 0; w < kAW; ++w)
    x[w] = *reinterpret_cast<const float4*>(wave_part<kFp8>(s_kt, s_vt, w) + part_off(row, c4));
  const float mw[kAW] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
  const float lw[kAW] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
  M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAW; ++w) M = fmaxf(M, mw[w]);
  const float Mb = (M == -INFINITY) ? 0.0f : M;
  L = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = 0.0f;
#pragma unroll
  for (int w = 0; w < kAW; ++w) {
    const float f = __builtin_amdgcn_exp2f(mw[w] - Mb);
    L += lw[w] * f;
    o[0] += x[w].x * f; o[1] += x[w].y * f; o[2] += x[w].z * f; o[3] += x[w].w * f;
  }
}

// Merges the ns key-split partials of query row rr = qt*16 + row of tile
// (b, kvh, qt) (query start qs) and writes its normalised output, dims d0 ..
// d0 + 7: k_attn_combine's arithmetic, shared with the fused kernel's
// in-kernel merge so that both give the same bits.
// Partials read by another workgroup of the same launch (the fused kernel's
// in-kernel split merge) move with agent-scope atomic stores and loads: the
// stores write through to the coherent level before the writer's ticket is
// taken, the loads do not hit a stale line of another XCD's L2, and no
// fence has to write back or invalidate a whole L2 (an agent-scope fence on
// this GPU does both, ~17 us per launch measured). Partials merged by a
// later launch use plain accesses.
template <bool kCoherent>
__device__ __forceinline__ void part_store4(float* p, float x, float y, float z, float w) {
  if constexpr (kCoherent) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p),
                       (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p + 2),
                       (uint64_t)__float_as_uint(z) | ((uint64_t)__float_as_uint(w) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(x, y, z, w);
  }
}
template <bool kCoherent>
__device__ __forceinline__ void part_store2(float* p, float x, float y) {
  if constexpr (kCoherent)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p),
                       (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *reinterpret_cast<float2*>(p) = make_float2(x, y);
}
template <bool kCoherent>
__device__ __forceinline__ float2 part_load2(const float* p) {
  if constexpr (kCoherent) {
    const uint64_t u = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
  } else {
    return *reinterpret_cast<const float2*>(p);
  }
}

// merges the ns key splits of row `row` (query row rr) of one (sequence, kv
// head, query tile), dims d0 .. d0 + 7, and writes the normalised output
template <bool kCoherent>
__device__ __forceinline__ void combine_splits(const AttnArgs& a, int b, int kvh, int qt, int qs,
                                               int ns, int row, int rr, int d0) {
  const int64_t base = (((int64_t)b * a.Hkv + kvh) * a.qtiles + qt) * a.nsplit;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s)
    M = fmaxf(M, part_load2<kCoherent>(a.part_ml + ((base + s) * kRows + row) * 2).x);
  const float Mb = (M == -INFINITY) ? 0.0f : M;
  float L = 0.0f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int s = 0; s < ns; ++s) {
    const int64_t pidx = (base + s) * kRows + row;
    const float2 ml = part_load2<kCoherent>(a.part_ml + pidx * 2);
    const float f = __builtin_amdgcn_exp2f(ml.x - Mb);
    L += ml.y * f;
    float x[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float2 v = part_load2<kCoherent>(a.part_o + pidx * kD + d0 + 2 * k);
      x[2 * k] = v.x;
      x[2 * k + 1] = v.y;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] += x[k] * f;
  }
  const float inv = (L > 0.0f) ? a.v_scale / L : 0.0f;
  const int oi = rr / a.G, oh = kvh * a.G + rr % a.G;
  union {
    uint16_t h[8];
    uint4 u;
  } ob;
#pragma unroll
  for (int t = 0; t < 8; ++t) ob.h[t] = f32_to_bf16_rne(o[t] * inv);
  *reinterpret_cast<uint4*>(a.out + (int64_t)(qs + oi) * a.o_st + (int64_t)oh * a.o_sh + d0) = ob.u;
}

// Merges the 8 waves' running states (acc) of query tile t, whose keys were
// [klo, khi) with wave w on windows w, w + 8, ..., and writes the normalised
// output (pslot < 0) or the unnormalised partial (o, running max, sum) at
// partial slot pslot. The per-wave K and V window tiles (s_kt, s_vt) take the
// per-wave partial outputs here. kSplitMerge (the fused kernel): a
// partial (the tile's keys span ns > 1 splits) is merged in the kernel: the
// last of the tile's ns workgroups to take its ticket (a.tickets[b * Hkv +
// kvh], zero between calls) merges them all.
template <bool kFp8, int kG, bool kSplitMerge>
__device__ __forceinline__ void merge_tile(const AttnArgs& a, const TileRef& t, int64_t pslot,
                                           uint8_t* s_kt, uint8_t* s_vt, float (*s_m)[kAW],
                                           float (*s_l)[kAW],
                                           const WaveAcc& acc, int ns) {
  const int G = kG ? kG : a.G;
  constexpr int kTileB = AttnLds<kFp8>::kTileB;
  const int kvh = t.kvh, qs = t.qs, rows = t.rows;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int r0 = t.qt * kRows;
  // bf16 tiles: a wave's partial output fits its own K tile, which it has
  // finished reading (its last window's reads were waited on), so it needs no
  // barrier before writing it; fp8 tiles are smaller and the partials go over
  // both tile arrays after every wave is done with its tiles
  constexpr bool kOwn = AttnLds<kFp8>::kTileB >= kRows * kD * 4;
  if (g == 0) {
    s_m[n][wid] = acc.m;
    s_l[n][wid] = acc.lsum;
  }
  if constexpr (!kOwn) lds_barrier();  // every wave is done with its tiles
  float* part = wave_part<kFp8>(s_kt, s_vt, wid);
#pragma unroll
  for (int db = 0; db < 8; ++db)
    *reinterpret_cast<float4*>(part + part_off(n, db * 4 + g)) =
        make_float4(acc.oacc[db][0], acc.oacc[db][1], acc.oacc[db][2], acc.oacc[db][3]);
  lds_barrier();
  // merge the waves: thread handles row tid / 32, dims 4 (tid % 32) .. + 3
  {
    const int row = tid >> 5;
    const int rr = r0 + row;
    if (rr < rows) {
      const int c4 = tid & 31, d0 = c4 * 4;
      float M, L, o[4];
      merge_waves<kFp8>(s_m, s_l, s_kt, s_vt, row, c4, M, L, o);
      const int oi = rr / G, oh = kvh * G + rr % G;
      if (pslot < 0) {
        const float inv = (L > 0.0f) ? a.v_scale / L : 0.0f;
        union {
          uint16_t h[4];
          uint2 u;
        } ob;
#pragma unroll
        for (int t = 0; t < 4; ++t) ob.h[t] = f32_to_bf16_rne(o[t] * inv);
        *reinterpret_cast<uint2*>(a.out + (int64_t)(qs + oi) * a.o_st + (int64_t)oh * a.o_sh +
                                  d0) = ob.u;
      } else {
        const int64_t pidx = pslot * kRows + row;
        part_store4<kSplitMerge>(a.part_o + pidx * kD + d0, o[0], o[1], o[2], o[3]);
        if ((tid & 31) == 0) part_store2<kSplitMerge>(a.part_ml + pidx * 2, M, L);
      }
    }
  }
  if constexpr (kSplitMerge) {
    if (pslot >= 0) {
      // in-kernel merge of the ns splits: every thread's partial stores
      // (agent-scope, written through) have completed before the workgroup
      // takes its ticket; the last workgroup reads them all at agent scope
      // and merges
      __shared__ int s_last;
      unsigned* ticket = a.tickets + (int64_t)t.b * a.Hkv + kvh;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev + 1 == (unsigned)ns;
      }
      __syncthreads();
      if (!s_last) return;
      if (tid == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int row = tid >> 4, rr = r0 + row;
      if (tid < kRows * 16 && rr < rows)
        combine_splits<true>(a, t.b, kvh, t.qt, qs, ns, row, rr, (tid & 15) * 8);
    }
  }
}

// Attends query tile t over keys [klo, khi) with the 8 waves of the workgroup
// (wave w takes windows w, w + 8, ...), merges the waves and writes the
// normalised output (pslot < 0) or the unnormalised partial at partial slot
// pslot (merge_tile). s_bt as for wave_walk.
template <bool kFp8, int kG>
__device__ __forceinline__ void attend_keys(const AttnArgs& a, const TileRef& t, int klo, int khi,
                                            int64_t pslot, uint8_t* s_kt, uint8_t* s_vt,
                                            float (*s_m)[kAW],
                                            float (*s_l)[kAW], const int* s_bt, int bt_cap) {
  constexpr int kTileB = AttnLds<kFp8>::kTileB;
  const int wid = threadIdx.x >> 6;
  uint8_t* tile_k = s_kt + wid * kTileB;
  uint8_t* tile_v = s_vt + wid * kTileB;
  WaveAcc acc;
  wave_walk<kFp8, kG>(a, t, t.kvh, klo, khi, klo + wid * kWin, kAW * kWin, s_bt, bt_cap, tile_k,
                      tile_v, acc);
  merge_tile<kFp8, kG, false>(a, t, pslot, s_kt, s_vt, s_m, s_l, acc, 1);
}

// One launch = one workgroup per (kv head x query tile, split, sequence).
// The grid's fastest dimension is not the split: consecutive workgroups go to
// the 8 XCDs in turn and the later splits of short sequences are empty, so
// split-fastest would leave the same XCDs idle; with 8 KV heads every XCD
// gets one head of every sequence and split.
// A small grid (at most one XCD's worth of workgroups) is packed onto one
// XCD: the host launches xcd_pack = 8 times the x dimension and only the
// workgroups with x % 8 == 0, which the dispatcher places on the same XCD,
// do the work; otherwise the workgroups of the XCDs dispatched last start up
// to ~2 us after the first (measured on an idle GPU; ~0.25 us in a graph).
// Small calls are latency-bound: every memory round trip and every long
// dependent computation before the first K/V window is issued adds to the
// kernel. The fields the prologue needs come ahead of the argument block as
// scalar arguments, which the dispatcher preloads into SGPRs (this file is built
// with -amdgpu-kernarg-preload-count covering them), so the first loads go out
// without waiting for the argument block; the prologue has no integer division
// for power-of-two block sizes and a single query tile (the host passes shifts
// and the block-table entries one split can touch).
template <bool kFp8, int kG>
__global__ __launch_bounds__(kAT) void k_verify_attn(const int32_t* cu_q, const int32_t* cu_k,
                                                     const int32_t* bt, int bt_stride,
                                                     int xcd_shift, int qtiles, int split_len,
                                                     int bs_shift, int bt_width, int nbt_split,
                                                     AttnArgs a) {
  const int G = kG ? kG : a.G;
  __shared__ __attribute__((aligned(16))) uint8_t s_kt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) uint8_t s_vt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) float s_m[kRows][kAW], s_l[kRows][kAW];
  __shared__ int s_bt[kBtCap];
  if (blockIdx.x & ((1u << xcd_shift) - 1)) return;
  const int bx = blockIdx.x >> xcd_shift;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;

  // The sequence bounds and the block-table entries this split can touch
  // (they only depend on the split) are requested before either is waited on.
  const int cq0 = cu_q[b], cq1 = cu_q[b + 1], ck0 = cu_k[b], ck1 = cu_k[b + 1];
  const int lo = split * split_len;
  const int bt0 = split == 0 ? 0 : key_block(lo, bs_shift, a.block_size);
  int nbt = nbt_split;
  if (nbt > bt_width - bt0) nbt = bt_width - bt0;
  const int32_t* btrow = bt + (int64_t)b * bt_stride;
  // branchless (a branch here would wait for the bounds first): entry
  // bt0 + tid clamped into the row (bt_width >= 1, checked by the host)
  const int bi = bt0 + tid < bt_width ? bt0 + tid : bt_width - 1;
  const int bt_mine = btrow[bi];
  // the argument block's four 64-byte lines are requested now, together (one
  // field of each), while the loads above are in flight
  asm volatile("" ::"s"(a.q), "s"(a.c_sh), "s"(a.scale_log2), "s"(a.sk_pre));
  const int kvh = qtiles == 1 ? bx : bx / qtiles;
  const int qt = bx - kvh * qtiles;
  // one wait for all five loads (otherwise the compiler sinks the table load
  // into the store below, behind the wait for the bounds)
  asm volatile("" ::"v"(bt_mine), "v"(cq0), "v"(cq1), "v"(ck0), "v"(ck1));
  const TileRef t = tile_ref_of(b, kvh, qt, G, cq0, cq1, ck0, ck1);
  if (tid < nbt) s_bt[tid] = bt_mine;
  for (int i = tid + kAT; i < nbt; i += kAT) s_bt[i] = btrow[bt0 + i];
  // this split holds keys [lo, lo + split_len) of the sequence's Lk; a tile
  // with more than split_len keys is split and writes partials
  if (qt * kRows >= t.rows || lo >= t.Lk) return;
  int hi = lo + split_len;
  const int vis = tile_keys(t, G);
  if (vis < hi) hi = vis;
  const int64_t pslot =
      t.Lk <= split_len ? -1 : (((int64_t)b * a.Hkv + kvh) * qtiles + qt) * a.nsplit + split;
  attend_keys<kFp8, kG>(a, t, lo, hi, pslot, s_kt, s_vt, s_m, s_l, s_bt, kBtCap);
}

// k_verify_attn with the q/k-norm + RoPE + KV-store step of its tile's
// tokens in the prologue: the host launches it where one query tile holds
// every query row of each (sequence, kv head). The grid is (kv head x xcd
// pack, key split, sequence); split s holds keys [s * split_len, (s + 1) *
// split_len) of the sequence, so a sequence whose keys fit one split is one
// workgroup per kv head and the other splits' workgroups return at once;
// longer sequences write partials that the last of their workgroups merges
// (merge_tile). With xcd_shift = 3 the workgroups that work are those with
// x % 8 == split % 8, so the kv heads of one split are dispatched to one XCD
// and consecutive splits to different XCDs (placement only). Replaces
// hs_qk_norm_rope_store + hs_verify_attention (+ the split combine) for
// decode and verify steps.
// Waves 0-7 walk windows w, w + 8, ... of the split as in k_verify_attn (the
// same keys in the same order: bit-identical outputs); waves 8-11 run the
// q/k-norm + RoPE prologue. Nothing waits for a workgroup barrier before the
// first window is in flight: each attention wave loads the block-table
// entries of its own windows (lane j: window j) with the sequence bounds and
// issues its first window as soon as they arrive. The prologue waves load and
// compute the query rows and the query tokens' own keys (Lk - Lq .. Lk - 1)
// meanwhile; their waits are for their own loads (a wave with window loads
// into LDS in flight could only wait for all of them). Where every token's
// cache slot is the one the block table gives its key (the fast case, every
// decode and verify step of the engine), the windows read those rows from
// s_new, and the cache stores go out unwaited. Otherwise (a padding slot, a
// token stored elsewhere) the stores are waited for and a window reaching
// those keys reads them back from the cache, as the two launches do.
template <bool kFp8, int kG>
__global__ __launch_bounds__(kQkvT) void k_verify_attn_qkv(const int32_t* cu_q, const int32_t* cu_k,
                                                         const int32_t* bt, int bt_stride,
                                                         int xcd_shift, int bs_shift,
                                                         int bt_width, int nbt_split, int split_len,
                                                         AttnArgs a, QkvArgs qa) {
  constexpr int kRowB = AttnLds<kFp8>::kRowB;
  constexpr int kTileB = AttnLds<kFp8>::kTileB;
  __shared__ __attribute__((aligned(16))) uint8_t s_kt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) uint8_t s_vt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) float s_m[kRows][kAW], s_l[kRows][kAW];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[kRows * kD];
  // the query tokens' k rows, then their v rows (at most kRows tokens)
  __shared__ __attribute__((aligned(16))) uint8_t s_new[2 * kRows * kRowB];
  __shared__ int s_fast;
  (void)nbt_split;
  const int G = kG ? kG : a.G;
  const unsigned xm = (1u << xcd_shift) - 1;
  if ((blockIdx.x & xm) != (blockIdx.y & xm)) return;
  const int kvh = blockIdx.x >> xcd_shift;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cq0 = cu_q[b], cq1 = cu_q[b + 1], ck0 = cu_k[b], ck1 = cu_k[b + 1];
  const int lo = split * split_len;
  const int32_t* btrow = bt + (int64_t)b * bt_stride;
  // block-table entry of this wave's window j (keys lo + 32 wid + 256 j) in
  // lane j, clamped into the row (a window past the row is skipped below)
  const int wbi = key_block(lo + kWin * wid + kAW * kWin * lane, bs_shift, a.block_size);
  const int wbt = btrow[wbi < bt_width ? wbi : bt_width - 1];
  // the argument block's lines are requested now, together (one field of each)
  asm volatile("" ::"s"(a.q), "s"(a.c_sh), "s"(a.scale_log2), "s"(a.sk_pre), "s"(qa.qkv),
               "s"(qa.cs_rows));
  // one wait for the bounds and the table entries
  asm volatile("" ::"v"(wbt), "v"(cq0), "v"(cq1), "v"(ck0), "v"(ck1));
  const TileRef t = tile_ref_of(b, kvh, 0, G, cq0, cq1, ck0, ck1);
  // no query token or no key of this split: nothing to store or attend
  if (t.rows <= 0 || t.Lk <= 0 || lo >= t.Lk) return;
  int hi = lo + split_len;
  const int vis = tile_keys(t, G);
  if (vis < hi) hi = vis;
  const int knew = t.Lk - t.Lq;  // first key of the query tokens
  if (wid >= kAW) {
    // prologue wave: q/k-norm + RoPE of its rows into s_q and s_new, the
    // fast-case check (every query token's slot is its key's table entry),
    // and the cache stores. It has no window loads in flight, so its waits
    // are for its own loads only. It ends after the barrier: the attention
    // waves' later barriers count the surviving waves.
    const int pw = wid - kAW;
    QkvLoads ql;
    qkv_load(a, qa, t, kvh, G, pw, ql);
    const int fi = lane < t.Lq ? lane : t.Lq - 1;
    const int fkey = knew + fi;
    const int fbi = key_block(fkey, bs_shift, a.block_size);
    const int fblk = btrow[fbi < bt_width ? fbi : bt_width - 1];
    const int fslot = qa.slots[t.qs + fi];
    // the attention waves issue their first windows after this barrier, so
    // these loads are ahead of the windows in the CU's memory pipeline
    lds_barrier();
    KvStores S;
    qkv_compute<kFp8>(a, qa, t, kvh, ql, s_q, s_new, S);
    const bool ok = t.Lq <= kRows && fslot >= 0 && fbi < bt_width && fblk >= 0 &&
                    fblk < a.num_blocks && fslot == fblk * a.block_size + (fkey - fbi * a.block_size);
    const bool fast = __builtin_amdgcn_ballot_w64(!ok) == 0;  // the same in every wave
    if (!fast) {
      // the stores reach the L2 before any attention wave loads those rows
      kv_store_all<kFp8>(a, qa, S);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    if (pw == 0 && lane == 0) s_fast = fast ? 1 : 0;
    lds_barrier();  // s_q, s_new and s_fast written
    // fast: nothing in this kernel reads the stored rows
    if (fast) kv_store_all<kFp8>(a, qa, S);
    return;
  }
  const int esz = kFp8 ? 1 : 2;
  uint8_t* tile_k = s_kt + wid * kTileB;
  uint8_t* tile_v = s_vt + wid * kTileB;
  // window j of this wave (first key wsj) -> its cache row bases; false when
  // its block is not a valid cache block (the window is skipped)
  auto window_base = [&](int j, int wsj, const uint8_t*& kb, const uint8_t*& vb) -> bool {
    const int bi = key_block(wsj, bs_shift, a.block_size);
    if (bi >= bt_width) return false;
    const int blk = __builtin_amdgcn_readlane(wbt, j);
    if (blk < 0 || blk >= a.num_blocks) return false;
    const int64_t off = ((int64_t)blk * a.c_sb + (int64_t)(wsj - bi * a.block_size) * a.c_st +
                         (int64_t)kvh * a.c_sh) * esz;
    kb = a.kc + off;
    vb = a.vc + off;
    return true;
  };
  // the first window goes out as soon as the bounds and table entries are in
  // and the prologue waves have issued their loads
  const WinOffs<kFp8> wo = win_offs<kFp8>(a, lane);
  lds_barrier();
  int ws = lo + kWin * wid;
  const uint8_t* kb0 = a.kc;
  const uint8_t* vb0 = a.vc;
  bool have = ws < hi && window_base(0, ws, kb0, vb0);
  if (have) {  // K first, so that its scores can start while V lands
    issue_tile<kFp8>(kb0, ws, hi, tile_k, wo);
    issue_tile<kFp8>(vb0, ws, hi, tile_v, wo);
  }
  // the prologue waves wrote s_q, s_new and s_fast. A barrier that orders LDS
  // only: the compiler's LDS release would first wait for this wave's window
  // loads into LDS, so the barrier would open when the last wave's first window
  // had landed; here each wave waits for its own window after it (the first
  // read below and the loop wait for its loads), and the waves whose windows
  // land first start first.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const bool fast = __builtin_amdgcn_readfirstlane(s_fast) != 0;
  if (!fast && have) {
    // the first window was loaded before the stores, which may have written
    // any of its rows: load it again past this CU's L1
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint8_t *kb, *vb;
    window_base(0, ws, kb, vb);
    issue_tile<kFp8>(kb, ws, hi, tile_k, wo);
    issue_tile<kFp8>(vb, ws, hi, tile_v, wo);
  }
  const int n = lane & 15, g = lane >> 4;
  const int r = n;
  const bool r_ok = r < t.rows;
  const int lim_r = knew + (r_ok ? r / G : 0);  // last visible key of this row
  const int kfull = min(hi, knew + 1);  // keys every row sees, below hi
  bf16x8_t qv[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
    qv[ds] = r_ok ? u4_to_bf16x8(*reinterpret_cast<const uint4*>(s_q + n * kD + ds * 32 + g * 8))
                  : u4_to_bf16x8(make_uint4(0, 0, 0, 0));
  float m = -INFINITY, lsum = 0.0f;
  f32x4_t oacc[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) oacc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // fast: keys from knew on read s_new
  const int kn = fast ? knew : INT32_MAX;
  const uint8_t* nk = s_new;
  const uint8_t* nv = s_new + kRows * kRowB;
  // Each window streams its K tile, then its V tile; window j + 1's K goes
  // out as soon as K_j is in registers and its V as soon as V_j is, so the
  // next window's loads overlap this window's scores, softmax and P V. Every
  // tile read waits for all loads in flight (loads into LDS cannot be waited
  // for one by one across the loop: the compiler would wait for all anyway).
  for (int j = 0; ws < hi; ++j) {
    const int ws_next = ws + kAW * kWin;
    const bool cur = have;
    const uint8_t *kbn = nullptr, *vbn = nullptr;
    const bool have_next = ws_next < hi && window_base(j + 1, ws_next, kbn, vbn);
    // a window of query-token keys only reads s_new: nothing to load
    const bool load_next = have_next && ws_next < kn;
    if (cur) {
      bf16x8_t ka[2][4], va[8];
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      read_k<kFp8, true>(tile_k, nk, ws, kn, t.Lq - 1, lane, ka);
      // every LDS read of the tile has returned before the next window overwrites it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (load_next) issue_tile<kFp8>(kbn, ws_next, hi, tile_k, wo);
      const bf16x8_t pb = mma_s(a, ws, hi, lim_r, r_ok, kfull, lane, ka, qv, m, lsum, oacc);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      read_v<kFp8, true>(tile_v, nv, ws, kn, t.Lq - 1, lane, va);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (load_next) issue_tile<kFp8>(vbn, ws_next, hi, tile_v, wo);
      mma_pv(va, pb, oacc);
    } else if (load_next) {
      issue_tile<kFp8>(kbn, ws_next, hi, tile_k, wo);
      issue_tile<kFp8>(vbn, ws_next, hi, tile_v, wo);
    }
    have = have_next;
    ws = ws_next;
  }
  WaveAcc acc;
  acc.m = m;
  acc.lsum = row4_sum(lsum);
#pragma unroll
  for (int db = 0; db < 8; ++db) acc.oacc[db] = oacc[db];
  // splits holding keys (at most the launched ones: keys past the declared
  // maximum are not attended, as in the per-tile kernel)
  int ns = (t.Lk + split_len - 1) / split_len;
  if (ns > (int)gridDim.y) ns = (int)gridDim.y;
  const int64_t pslot = ns <= 1 ? -1 : ((int64_t)b * a.Hkv + kvh) * a.nsplit + split;
  merge_tile<kFp8, kG, true>(a, t, pslot, s_kt, s_vt, s_m, s_l, acc, ns);
}

// Balanced launch: one workgroup per CU. The 32-key windows of all tiles
// form one list; workgroup k of N takes windows [W*k/N, W*(k+1)/N) of the W
// in all, so every workgroup streams the same number of windows whatever the
// sequence lengths, and no workgroup waits on the hardware dispatcher after
// the start. Its range covers whole tiles (written as final outputs) and at
// most two pieces of tiles shared with its neighbours: its first piece goes
// to partial slot 2k, its last to 2k + 1, merged by k_attn_combine_sk.
// Two tile kinds:
//   kHeads = false: tile = (kv head, sequence, query tile), kv-head-major;
//     the 8 waves take alternate windows of one kv head and merge in LDS.
//     Workgroups k, k + N/Hkv, ... walk the same sequences at the same
//     offsets for different heads, so the heads' 256-byte pieces of each
//     cached token row are read close together in time.
//   kHeads = true (8 kv heads): tile = (sequence, query tile); wave w takes
//     kv head w over the same windows, so each window reads whole cached
//     token rows (all heads) at once, and the waves need no merge. A slot
//     then holds the pieces of all 8 heads.
constexpr int kSkMaxTiles = 4096;
constexpr int kSkBtCap = 1024 + 2;

// tile j of the balanced launch's list
template <bool kHeads>
__device__ __forceinline__ void sk_tile(const AttnArgs& a, int j, int& b, int& kvh, int& qt) {
  if constexpr (kHeads) {
    kvh = 0;
    b = j / a.qtiles;
    qt = j % a.qtiles;
  } else {
    const int per_head = a.B * a.qtiles;
    kvh = j / per_head;
    const int rem = j % per_head;
    b = rem / a.qtiles;
    qt = rem % a.qtiles;
  }
}

template <bool kHeads>
__device__ __forceinline__ int sk_tiles(const AttnArgs& a) {
  return kHeads ? a.B * a.qtiles : a.B * a.Hkv * a.qtiles;
}

// Attends query tile t over keys [klo, khi) with wave w on kv head w (all
// waves walk the same windows) and writes each wave's rows: normalised
// output (pslot < 0) or the unnormalised partial at partial slot pslot.
template <bool kFp8, int kG>
__device__ __forceinline__ void attend_heads(const AttnArgs& a, const TileRef& t, int klo, int khi,
                                             int64_t pslot, uint8_t* s_kt, uint8_t* s_vt,
                                             const int* s_bt,
                                             int bt_cap) {
  const int G = kG ? kG : a.G;
  constexpr int kTileB = AttnLds<kFp8>::kTileB;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int kvh = wid;
  uint8_t* tile_k = s_kt + wid * kTileB;
  uint8_t* tile_v = s_vt + wid * kTileB;
  WaveAcc acc;
  wave_walk<kFp8, kG>(a, t, kvh, klo, khi, klo, kWin, s_bt, bt_cap, tile_k, tile_v, acc);
  const int r = t.qt * kRows + n;
  if (r >= t.rows) return;
  const int qi = r / G, qh = kvh * G + r % G;
  if (pslot < 0) {
    const float inv = (acc.lsum > 0.0f) ? a.v_scale / acc.lsum : 0.0f;
    uint16_t* op = a.out + (int64_t)(t.qs + qi) * a.o_st + (int64_t)qh * a.o_sh + 4 * g;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t w0 = (uint32_t)f32_to_bf16_rne(acc.oacc[db][0] * inv) |
                          ((uint32_t)f32_to_bf16_rne(acc.oacc[db][1] * inv) << 16);
      const uint32_t w1 = (uint32_t)f32_to_bf16_rne(acc.oacc[db][2] * inv) |
                          ((uint32_t)f32_to_bf16_rne(acc.oacc[db][3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + db * 16) = make_uint2(w0, w1);
    }
  } else {
    const int64_t pidx = (pslot * a.Hkv + kvh) * kRows + n;
    float* po = a.part_o + pidx * kD + 4 * g;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<float4*>(po + db * 16) =
          make_float4(acc.oacc[db][0], acc.oacc[db][1], acc.oacc[db][2], acc.oacc[db][3]);
    if (g == 0) {
      a.part_ml[pidx * 2] = acc.m;
      a.part_ml[pidx * 2 + 1] = acc.lsum;
    }
  }
}

template <bool kFp8, int kG, bool kHeads>
__global__ __launch_bounds__(kAT) void k_verify_attn_sk(AttnArgs a) {
  const int G = kG ? kG : a.G;
  __shared__ __attribute__((aligned(16))) uint8_t s_kt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) uint8_t s_vt[AttnLds<kFp8>::kArrB];
  __shared__ __attribute__((aligned(16))) float s_m[kHeads ? 1 : kRows][kAW],
      s_l[kHeads ? 1 : kRows][kAW];
  __shared__ int s_bt[kSkBtCap];
  __shared__ int s_pre[kSkMaxTiles + 1];
  __shared__ int s_wsum[kAW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int ntiles = sk_tiles<kHeads>(a);

  // window count of every tile, then their prefix sums (s_pre[j] = windows
  // before tile j); thread tid owns tiles [tid * per, tid * per + per)
  const int per = (ntiles + kAT - 1) / kAT;
  int tsum = 0;
  for (int i = 0; i < per; ++i) {
    const int j = tid * per + i;
    if (j >= ntiles) break;
    int b, kvh, qt;
    sk_tile<kHeads>(a, j, b, kvh, qt);
    const TileRef t = tile_ref(a, b, kvh, qt, G);
    const int nw = (tile_keys(t, G) + kWin - 1) / kWin;
    s_pre[j + 1] = nw;
    tsum += nw;
  }
  int incl = tsum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  if (lane == 63) s_wsum[wid] = incl;
  __syncthreads();
  int run = incl - tsum;
  for (int w = 0; w < wid; ++w) run += s_wsum[w];
  for (int i = 0; i < per; ++i) {
    const int j = tid * per + i;
    if (j >= ntiles) break;
    run += s_pre[j + 1];
    s_pre[j + 1] = run;
  }
  if (tid == 0) s_pre[0] = 0;
  __syncthreads();

  const int64_t W = s_pre[ntiles];
  const int64_t N = gridDim.x, k = blockIdx.x;
  if (k == 0)
    for (int j = tid; j <= ntiles; j += kAT) a.sk_pre[j] = s_pre[j];
  const int w_begin = (int)(W * k / N), w_end = (int)(W * (k + 1) / N);
  if (tid == 0) {
    a.sk_w0[k] = w_begin;
    if (k == N - 1) a.sk_w0[N] = w_end;
  }
  if (w_begin >= w_end) return;
  // tile holding window w_begin: the last j with s_pre[j] <= w_begin
  int jl = 0, jh = ntiles - 1;
  while (jl < jh) {
    const int mid = (jl + jh + 1) >> 1;
    if (s_pre[mid] <= w_begin) jl = mid; else jh = mid - 1;
  }
  int j = jl, w = w_begin, seg = 0;
  while (w < w_end) {
    while (s_pre[j + 1] <= w) ++j;  // tiles without windows
    const int s0 = s_pre[j], s1 = s_pre[j + 1];
    const int seg_end = s1 < w_end ? s1 : w_end;
    int b, kvh, qt;
    sk_tile<kHeads>(a, j, b, kvh, qt);
    const TileRef t = tile_ref(a, b, kvh, qt, G);
    const int klo = (w - s0) * kWin;
    int khi = (seg_end - s0) * kWin;
    const int vis = tile_keys(t, G);
    if (vis < khi) khi = vis;
    const int64_t pslot = (w == s0 && seg_end == s1) ? -1 : 2 * k + (seg > 0 ? 1 : 0);
    __syncthreads();  // the previous piece's readers of s_bt and the tiles are done
    const int bt0 = key_block(klo, a.bs_shift, a.block_size);
    const int nbt = key_block(khi - 1, a.bs_shift, a.block_size) - bt0 + 1;
    for (int i = tid; i < nbt && i < kSkBtCap && bt0 + i < a.bt_width; i += kAT)
      s_bt[i] = a.bt[(int64_t)b * a.bt_stride + bt0 + i];
    if constexpr (kHeads)
      attend_heads<kFp8, kG>(a, t, klo, khi, pslot, s_kt, s_vt, s_bt, kSkBtCap);
    else
      attend_keys<kFp8, kG>(a, t, klo, khi, pslot, s_kt, s_vt, s_m, s_l, s_bt, kSkBtCap);
    w = seg_end;
    ++seg;
  }
}

// merges the pieces of the tiles that the balanced launch split between
// workgroups: one workgroup per (tile, kv head of the tile); whole tiles
// return at once. The pieces' loads go out 8 at a time and merge online.
template <bool kHeads>
__global__ __launch_bounds__(kRows * 16) void k_attn_combine_sk(AttnArgs a) {
  constexpr int kU = 8;
  const int j = blockIdx.x;
  const int ntiles = sk_tiles<kHeads>(a);
  const int64_t W = a.sk_pre[ntiles], N = a.sk_nwg;
  const int s0 = a.sk_pre[j], s1 = a.sk_pre[j + 1];
  if (s0 == s1) return;
  // first and last workgroups whose window range [W*k/N, W*(k+1)/N) meets [s0, s1)
  const int kf = (int)((N * (s0 + 1) + W - 1) / W - 1);
  const int kl = (int)((N * s1 + W - 1) / W - 1);
  if (kf == kl) return;
  int b, kvh, qt;
  sk_tile<kHeads>(a, j, b, kvh, qt);
  if (kHeads) kvh = blockIdx.y;
  const int tid = threadIdx.x;
  const int qs = a.cu_q[b];
  const int rows = (a.cu_q[b + 1] - qs) * a.G;
  const int row = tid >> 4;
  const int d0 = (tid & 15) * 8;
  const int rr = qt * kRows + row;
  if (rr >= rows) return;
  float M = -INFINITY, L = 0.0f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int kb = kf; kb <= kl; kb += kU) {
    float mp[kU], lp[kU];
    float4 x0[kU], x1[kU];
    bool use[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = kb + u <= kl ? kb + u : kl;
      const int wk = a.sk_w0[k];
      use[u] = (kb + u <= kl) && wk != a.sk_w0[k + 1];  // empty ranges hold no piece
      const int64_t slot = 2 * (int64_t)k + ((k == kf && wk < s0) ? 1 : 0);
      const int64_t pidx = (kHeads ? slot * a.Hkv + kvh : slot) * kRows + row;
      mp[u] = a.part_ml[pidx * 2];
      lp[u] = a.part_ml[pidx * 2 + 1];
      x0[u] = *reinterpret_cast<const float4*>(a.part_o + pidx * kD + d0);
      x1[u] = *reinterpret_cast<const float4*>(a.part_o + pidx * kD + d0 + 4);
    }
    float Mg = M;
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (use[u]) Mg = fmaxf(Mg, mp[u]);
    const float Mb = (Mg == -INFINITY) ? 0.0f : Mg;
    const float sc = __builtin_amdgcn_exp2f(M - Mb);
    L *= sc;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] *= sc;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (!use[u]) continue;  // (its loads read a stale slot; none of it is used)
      const float f = __builtin_amdgcn_exp2f(mp[u] - Mb);
      L += lp[u] * f;
      o[0] += x0[u].x * f; o[1] += x0[u].y * f; o[2] += x0[u].z * f; o[3] += x0[u].w * f;
      o[4] += x1[u].x * f; o[5] += x1[u].y * f; o[6] += x1[u].z * f; o[7] += x1[u].w * f;
    }
    M = Mg;
  }
  const float inv = (L > 0.0f) ? a.v_scale / L : 0.0f;
  const int oi = rr / a.G, oh = kvh * a.G + rr % a.G;
  union {
    uint16_t h[8];
    uint4 u;
  } ob;
#pragma unroll
  for (int t = 0; t < 8; ++t) ob.h[t] = f32_to_bf16_rne(o[t] * inv);
  *reinterpret_cast<uint4*>(a.out + (int64_t)(qs + oi) * a.o_st + (int64_t)oh * a.o_sh + d0) = ob.u;
}

// merges the key splits of every (sequence, kv head, query tile)
__global__ __launch_bounds__(kRows * 16) void k_attn_combine(AttnArgs a) {
  const int kvh = blockIdx.y / a.qtiles;
  const int qt = blockIdx.y % a.qtiles;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int qs = a.cu_q[b];
  const int Lq = a.cu_q[b + 1] - qs;
  const int Lk = a.cu_k[b + 1] - a.cu_k[b];
  const int rows = Lq * a.G;
  const int r0 = qt * kRows;
  if (r0 >= rows || Lk <= 0) return;
  const int ns = (Lk + a.split_len - 1) / a.split_len;
  if (ns <= 1) return;
  const int row = tid >> 4;
  const int rr = r0 + row;
  if (rr >= rows) return;
  combine_splits<false>(a, b, kvh, qt, qs, ns, row, rr, (tid & 15) * 8);
}

template <bool kFp8>
static void launch_attn(int G, dim3 grid, hipStream_t s, const AttnArgs& a) {
  const int bts = (int)a.bt_stride;
  const int xs = a.xcd_pack == 8 ? 3 : 0;
  // block-table entries one split can touch (it may start inside a block)
  int nbt = (a.split_len + a.block_size - 1) / a.block_size + 1;
  if (nbt > kBtCap) nbt = kBtCap;
  switch (G) {
    case 2: hipLaunchKernelGGL((k_verify_attn<kFp8, 2>), grid, dim3(kAT), 0, s, a.cu_q, a.cu_k, a.bt, bts,
                                 xs, a.qtiles, a.split_len, a.bs_shift, a.bt_width, nbt, a); break;
    case 4: hipLaunchKernelGGL((k_verify_attn<kFp8, 4>), grid, dim3(kAT), 0, s, a.cu_q, a.cu_k, a.bt, bts,
                                 xs, a.qtiles, a.split_len, a.bs_shift, a.bt_width, nbt, a); break;
    case 8: hipLaunchKernelGGL((k_verify_attn<kFp8, 8>), grid, dim3(kAT), 0, s, a.cu_q, a.cu_k, a.bt, bts,
                                 xs, a.qtiles, a.split_len, a.bs_shift, a.bt_width, nbt, a); break;
    default: hipLaunchKernelGGL((k_verify_attn<kFp8, 0>), grid, dim3(kAT), 0, s, a.cu_q, a.cu_k, a.bt, bts,
                                 xs, a.qtiles, a.split_len, a.bs_shift, a.bt_width, nbt, a); break;
  }
}

template <bool kFp8>
static void launch_attn_qkv(int G, dim3 grid, hipStream_t s, const AttnArgs& a,
                            const QkvArgs& qa) {
  const int bts = (int)a.bt_stride;
  const int xs = a.xcd_pack == 8 ? 3 : 0;
  int nbt = (a.split_len + a.block_size - 1) / a.block_size + 1;
  if (nbt > kBtCap) nbt = kBtCap;
  const int sl = a.split_len;
  switch (G) {
    case 2: hipLaunchKernelGGL((k_verify_attn_qkv<kFp8, 2>), grid, dim3(kQkvT), 0, s, a.cu_q, a.cu_k, a.bt,
                                 bts, xs, a.bs_shift, a.bt_width, nbt, sl, a, qa); break;
    case 4: hipLaunchKernelGGL((k_verify_attn_qkv<kFp8, 4>), grid, dim3(kQkvT), 0, s, a.cu_q, a.cu_k, a.bt,
                                 bts, xs, a.bs_shift, a.bt_width, nbt, sl, a, qa); break;
    case 8: hipLaunchKernelGGL((k_verify_attn_qkv<kFp8, 8>), grid, dim3(kQkvT), 0, s, a.cu_q, a.cu_k, a.bt,
                                 bts, xs, a.bs_shift, a.bt_width, nbt, sl, a, qa); break;
    default: hipLaunchKernelGGL((k_verify_attn_qkv<kFp8, 0>), grid, dim3(kQkvT), 0, s, a.cu_q, a.cu_k, a.bt,
                                  bts, xs, a.bs_shift, a.bt_width, nbt, sl, a, qa); break;
  }
}

template <bool kFp8, bool kHeads>
static void launch_attn_sk(int G, int nwg, hipStream_t s, const AttnArgs& a) {
  switch (G) {
    case 2: hipLaunchKernelGGL((k_verify_attn_sk<kFp8, 2, kHeads>), dim3(nwg), dim3(kAT), 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_verify_attn_sk<kFp8, 4, kHeads>), dim3(nwg), dim3(kAT), 0, s, a); break;
    case 8: hipLaunchKernelGGL((k_verify_attn_sk<kFp8, 8, kHeads>), dim3(nwg), dim3(kAT), 0, s, a); break;
    default: hipLaunchKernelGGL((k_verify_attn_sk<kFp8, 0, kHeads>), dim3(nwg), dim3(kAT), 0, s, a); break;
  }
}

static int g_attn_cus[64];  // CUs per device, filled on first use

static int attn_num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!g_attn_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    g_attn_cus[dev] = n;
  }
  return g_attn_cus[dev];
}

// Balanced launch (one workgroup per CU) when the tiles fit its prefix table
// and the longest length gives enough windows per workgroup (below that the
// classic grid is one short wave of workgroups anyway): with 8 kv heads the
// heads-in-waves kind (tiles without the head, each wave one head: at least
// 4 windows per workgroup), otherwise the kv-head-major kind (at least 16
// windows per workgroup, 2 per wave). Returns the workgroup count, or 0 for
// the classic grid; *heads tells the kind.
static int attn_sk_plan(int B, int Hkv, int qtiles, int max_seqlen_k, bool* heads) {
  const int cus = attn_num_cus();
  const int64_t wins = (max_seqlen_k + kWin - 1) / kWin;
  *heads = (Hkv == kAW);
  const int64_t tiles = (int64_t)B * qtiles * (*heads ? 1 : Hkv);
  if (tiles > kSkMaxTiles) return 0;
  if (tiles * wins < (*heads ? 4LL : 16LL) * cus) return 0;
  return cus;
}

static size_t attn_sk_workspace(int B, int Hkv, int qtiles, int nwg, bool heads) {
  const size_t slots = 2 * (size_t)nwg * kRows * (heads ? Hkv : 1);
  const size_t tiles = (size_t)B * qtiles * (heads ? 1 : Hkv);
  return slots * kD * sizeof(float) + slots * 2 * sizeof(float) +
         (tiles + 1 + nwg + 1) * sizeof(int) + 256;
}

static void attn_plan(int B, int Hkv, int qtiles, int max_seqlen_k, int* nsplit, int* split_len) {
  const int64_t tiles = (int64_t)B * Hkv * qtiles;
  const int64_t target = 1024;  // workgroups in flight across 256 CUs
  int64_t want = (target + tiles - 1) / tiles;
  if (want < 1) want = 1;
  int64_t len = (max_seqlen_k + want - 1) / want;
  len = (len + 127) / 128 * 128;
  // a split below 1024 keys costs more in the extra combine launch (~3.5 us)
  // than it gains in parallelism (each wave already prefetches its next
  // window); splits are also capped by the block-table prefetch
  if (len < 1024) len = 1024;
  if (len > kMaxSplit) len = kMaxSplit;
  *split_len = (int)len;
  *nsplit = (int)((max_seqlen_k + len - 1) / len);
  if (*nsplit < 1) *nsplit = 1;
}

// The first kTicketBytes of an attention workspace hold the fused kernel's
// split-merge tickets (one 32-bit counter per (sequence, kv head), zero
// between calls: the workgroup that merges a tile resets its counter); the
// partial results follow. Fused calls with more (sequence, kv head) pairs
// than tickets run as the store and attention launches.
constexpr size_t kTicketBytes = 16384;
constexpr int kTicketSlots = (int)(kTicketBytes / sizeof(unsigned));

// Scratch of hs_verify_attention_noalloc: the partial results of key splits
// or of the balanced launch's shared tile pieces, which hs_verify_attention
// keeps in the caller's workspace. 34 MiB holds the largest layout the
// balanced launch uses on a 256-CU device (two pieces of 8 heads x 16 rows x
// 128 floats per workgroup, 32.5 MiB). Every GPU the library runs on holds
// its own copy until the process ends; host code must never use the array's
// name as an address (it is a host-side stand-in): the per-device address
// comes from hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = (size_t)34 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of this device's scratch, looked up once per device with that
// device current; null on failure.
static void* scratch_of_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace hs

using namespace hs;

// Argument checks and the launch plan shared by hs_verify_attention and
// hs_qk_norm_rope_attend: fills *pa (everything but the partial-result
// pointers) and *pneed (the workspace size of the call).
static int attn_prepare(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        int64_t cache_stride_block, int64_t cache_stride_tok,
                        int64_t cache_stride_head, float k_scale, float v_scale,
                        const int32_t* block_tables, int64_t block_table_stride,
                        int block_table_width, int num_blocks, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int num_seqs, int max_seqlen_q,
                        int max_seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                        int block_size, float softmax_scale, void* out, int64_t out_stride_tok,
                        int64_t out_stride_head, void* workspace, size_t workspace_bytes,
                        AttnArgs* pa, size_t* pneed) {
  if (!q || !k_cache || !v_cache || !block_tables || !cu_seqlens_q || !cu_seqlens_k || !out)
    return HS_ERR_INVALID;
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_seqlen_q <= 0 ||
      max_seqlen_k <= 0 || num_blocks <= 0 || block_size <= 0 || block_table_width <= 0 ||
      block_table_stride < block_table_width || block_table_stride > INT32_MAX)
    return HS_ERR_INVALID;
  if (num_q_heads % num_kv_heads) return HS_ERR_INVALID;
  if (head_dim != kD) return HS_ERR_UNSUPPORTED;
  if (block_size % kWin) return HS_ERR_UNSUPPORTED;
  if (kv_dtype != HS_BF16 && kv_dtype != HS_FP8_E4M3) return HS_ERR_INVALID;
  const int G = num_q_heads / num_kv_heads;
  if (G > kRows) return HS_ERR_UNSUPPORTED;
  // 16-byte alignment of every row the kernel loads or stores
  const int esz = (kv_dtype == HS_BF16) ? 2 : 1;
  if ((q_stride_tok % 8) || (q_stride_head % 8) || (out_stride_tok % 8) || (out_stride_head % 8))
    return HS_ERR_UNSUPPORTED;
  if (((cache_stride_block * esz) % 16) || ((cache_stride_tok * esz) % 16) ||
      ((cache_stride_head * esz) % 16))
    return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15)
    return HS_ERR_UNSUPPORTED;
  // a window's 32 token rows lie within 2 GiB of its first (32-bit load offsets)
  if (cache_stride_tok * esz * kWin > INT32_MAX) return HS_ERR_UNSUPPORTED;
  const size_t need = *pneed = hs_verify_attention_workspace_size(num_seqs, num_q_heads, num_kv_heads,
                                                         max_seqlen_q, max_seqlen_k);
  AttnArgs& a = *pa;
  a.qtiles = (max_seqlen_q * G + kRows - 1) / kRows;
  attn_plan(num_seqs, num_kv_heads, a.qtiles, max_seqlen_k, &a.nsplit, &a.split_len);
  if (a.nsplit > 1 && (!workspace || workspace_bytes < need)) return HS_ERR_WORKSPACE;
  if ((int64_t)num_kv_heads * a.qtiles > 65535 || a.nsplit > 65535 || num_seqs > 65535)
    return HS_ERR_UNSUPPORTED;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint8_t*>(k_cache);
  a.vc = static_cast<const uint8_t*>(v_cache);
  a.fp8 = (kv_dtype == HS_FP8_E4M3);
  a.c_sb = cache_stride_block;
  a.c_st = cache_stride_tok;
  a.c_sh = cache_stride_head;
  a.v_scale = a.fp8 ? v_scale : 1.0f;
  a.bt = block_tables;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.num_blocks = num_blocks;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.B = num_seqs;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.scale_log2 = softmax_scale * (a.fp8 ? k_scale : 1.0f) * 1.4426950408889634f;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  a.tickets = static_cast<unsigned*>(workspace);
  a.contig = 0;
  return HS_OK;
}

extern "C" {

size_t hs_verify_attention_workspace_size(int num_seqs, int num_q_heads, int num_kv_heads,
                                          int max_seqlen_q, int max_seqlen_k) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_seqlen_q <= 0 ||
      max_seqlen_k <= 0 || num_q_heads % num_kv_heads)
    return 0;
  const int G = num_q_heads / num_kv_heads;
  const int qtiles = (max_seqlen_q * G + kRows - 1) / kRows;
  int nsplit, split_len;
  attn_plan(num_seqs, num_kv_heads, qtiles, max_seqlen_k, &nsplit, &split_len);
  const size_t parts = (size_t)num_seqs * num_kv_heads * qtiles * nsplit * kRows;
  const size_t classic = parts * kD * sizeof(float) + parts * 2 * sizeof(float) + 256;
  bool heads = false;
  const int nwg = attn_sk_plan(num_seqs, num_kv_heads, qtiles, max_seqlen_k, &heads);
  const size_t sk = nwg ? attn_sk_workspace(num_seqs, num_kv_heads, qtiles, nwg, heads) : 0;
  return kTicketBytes + (classic > sk ? classic : sk);
}

int hs_verify_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        int64_t cache_stride_block, int64_t cache_stride_tok,
                        int64_t cache_stride_head, float k_scale, float v_scale,
                        const int32_t* block_tables, int64_t block_table_stride,
                        int block_table_width, int num_blocks,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int num_seqs,
                        int max_seqlen_q, int max_seqlen_k, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, float softmax_scale, void* out,
                        int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                        size_t workspace_bytes, void* stream) {
  // no block table: the keys are the call's own unpaged rows
  // (flash_attn_varlen_func without block_table, attention.py:147-160):
  // k_cache / v_cache are [tokens, num_kv_heads, 128] with sequence b's keys
  // at rows cu_seqlens_k[b] .. cu_seqlens_k[b + 1] - 1, and the block
  // arguments are ignored (the kernel's table prefetch reads cu_seqlens_k,
  // whose values it does not use)
  const bool contig = block_tables == nullptr;
  if (contig) {
    block_tables = cu_seqlens_k;
    block_table_stride = 1;
    block_table_width = 1;
    num_blocks = 1;
    block_size = kWin;
    cache_stride_block = 0;
  }
  AttnArgs a;
  size_t need = 0;
  const int prc = attn_prepare(q, q_stride_tok, q_stride_head, k_cache, v_cache, kv_dtype,
                               cache_stride_block, cache_stride_tok, cache_stride_head, k_scale,
                               v_scale, block_tables, block_table_stride, block_table_width,
                               num_blocks, cu_seqlens_q, cu_seqlens_k, num_seqs, max_seqlen_q,
                               max_seqlen_k, num_q_heads, num_kv_heads, head_dim, block_size,
                               softmax_scale, out, out_stride_tok, out_stride_head, workspace,
                               workspace_bytes, &a, &need);
  if (prc != HS_OK) return prc;
  a.contig = contig ? 1 : 0;
  const int G = a.G;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  bool heads = false;
  const int nwg = contig ? 0 : attn_sk_plan(num_seqs, num_kv_heads, a.qtiles, max_seqlen_k, &heads);
  if (nwg && workspace && workspace_bytes >= need &&
      (max_seqlen_k + block_size - 1) / block_size + 1 <= kSkBtCap) {
    const size_t slots = 2 * (size_t)nwg * kRows * (heads ? num_kv_heads : 1);
    a.part_o = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kTicketBytes);
    a.part_ml = a.part_o + slots * kD;
    const int ntiles = num_seqs * a.qtiles * (heads ? 1 : num_kv_heads);
    a.sk_pre = reinterpret_cast<int*>(a.part_ml + slots * 2);
    a.sk_w0 = a.sk_pre + ntiles + 1;
    a.sk_nwg = nwg;
    a.xcd_pack = 1;
    if (heads) {
      if (a.fp8)
        launch_attn_sk<true, true>(G, nwg, s, a);
      else
        launch_attn_sk<false, true>(G, nwg, s, a);
      hipLaunchKernelGGL(k_attn_combine_sk<true>, dim3(ntiles, num_kv_heads), dim3(kRows * 16), 0,
                         s, a);
    } else {
      if (a.fp8)
        launch_attn_sk<true, false>(G, nwg, s, a);
      else
        launch_attn_sk<false, false>(G, nwg, s, a);
      hipLaunchKernelGGL(k_attn_combine_sk<false>, dim3(ntiles), dim3(kRows * 16), 0, s, a);
    }
    return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
  }
  const size_t parts = (size_t)num_seqs * num_kv_heads * a.qtiles * a.nsplit * kRows;
  a.part_o = workspace ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kTicketBytes)
                       : nullptr;
  a.part_ml = workspace ? a.part_o + parts * kD : nullptr;
  a.sk_pre = nullptr;
  a.sk_w0 = nullptr;
  a.sk_nwg = 0;
  const int64_t wgs = (int64_t)num_kv_heads * a.qtiles * a.nsplit * num_seqs;
  a.xcd_pack = (wgs <= 32) ? 8 : 1;  // 8 XCDs of 32 CUs; workgroup i runs on XCD i % 8
  dim3 grid(a.xcd_pack * num_kv_heads * a.qtiles, a.nsplit, num_seqs);
  if (a.fp8)
    launch_attn<true>(G, grid, s, a);
  else
    launch_attn<false>(G, grid, s, a);
  if (a.nsplit > 1)
    hipLaunchKernelGGL(k_attn_combine, dim3(num_seqs, num_kv_heads * a.qtiles),
                       dim3(kRows * 16), 0, s, a);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_qk_norm_rope_attend(const void* qkv, int64_t token_stride, int num_tokens,
                           const void* q_weight, const void* k_weight, const float* cos_sin,
                           int cos_sin_rows, const int64_t* positions, float eps,
                           const int32_t* slot_mapping,
                           void* q_out, void* k_cache, void* v_cache, int kv_dtype,
                           int64_t cache_stride_block, int64_t cache_stride_tok,
                           int64_t cache_stride_head, float k_scale, float v_scale,
                           const int32_t* block_tables, int64_t block_table_stride,
                           int block_table_width, int num_blocks, const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int num_seqs, int max_seqlen_q,
                           int max_seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                           int block_size, float softmax_scale, void* out,
                           int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (num_tokens <= 0) return num_tokens == 0 ? HS_OK : HS_ERR_INVALID;
  if (!qkv || !q_weight || !k_weight || !cos_sin || !positions || !slot_mapping || !q_out ||
      cos_sin_rows <= 0 || !block_tables)
    return HS_ERR_INVALID;
  if (num_q_heads <= 0 || num_kv_heads <= 0) return HS_ERR_INVALID;
  if (head_dim != kD) return HS_ERR_UNSUPPORTED;
  if (kv_dtype != HS_BF16 && kv_dtype != HS_FP8_E4M3) return HS_ERR_INVALID;
  if (token_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * kD) return HS_ERR_INVALID;
  if (kv_dtype == HS_FP8_E4M3 && !(k_scale > 0.0f && v_scale > 0.0f)) return HS_ERR_INVALID;
  // 16-byte pieces of every head (q/k-norm + RoPE rows of 16 lanes)
  if ((token_stride % 8) || (((uintptr_t)qkv | (uintptr_t)q_weight | (uintptr_t)k_weight |
                              (uintptr_t)cos_sin) & 15))
    return HS_ERR_UNSUPPORTED;
  // q_out [num_tokens, Hq, 128]: the two-launch path's q, and the argument
  // checks' stand-in for q (the fused kernel does not write it)
  AttnArgs a;
  size_t need = 0;
  const int prc = attn_prepare(q_out, (int64_t)num_q_heads * kD, kD, k_cache, v_cache, kv_dtype,
                               cache_stride_block, cache_stride_tok, cache_stride_head, k_scale,
                               v_scale, block_tables, block_table_stride, block_table_width,
                               num_blocks, cu_seqlens_q, cu_seqlens_k, num_seqs, max_seqlen_q,
                               max_seqlen_k, num_q_heads, num_kv_heads, head_dim, block_size,
                               softmax_scale, out, out_stride_tok, out_stride_head, workspace,
                               workspace_bytes, &a, &need);
  if (prc != HS_OK) return prc;
  bool heads = false;
  const int nwg = attn_sk_plan(num_seqs, num_kv_heads, a.qtiles, max_seqlen_k, &heads);
  const bool sk = nwg && workspace && workspace_bytes >= need &&
                  (max_seqlen_k + block_size - 1) / block_size + 1 <= kSkBtCap;
  const int64_t pairs = (int64_t)num_kv_heads * num_seqs;
  // one launch where one query tile holds every query row of a (sequence, kv
  // head) and the classic grid serves the call; key splits need the
  // workspace (partials and tickets)
  const bool fused = !sk && a.qtiles == 1 && max_seqlen_q * a.G <= kRows &&
                     (a.nsplit == 1 || (workspace && workspace_bytes >= need &&
                                        pairs <= kTicketSlots));
  if (!fused) {
    // a (sequence, kv head) over several workgroups: the store first, then the
    // attention over the stored cache
    const int rc = hs_qk_norm_rope_store(
        qkv, token_stride, num_q_heads, num_kv_heads, head_dim, q_weight, k_weight, cos_sin,
        positions, eps, q_out, k_cache, v_cache, kv_dtype, cache_stride_block, cache_stride_tok,
        cache_stride_head, k_scale, v_scale, slot_mapping, block_size, num_blocks, num_tokens,
        stream);
    if (rc != HS_OK) return rc;
    return hs_verify_attention(q_out, (int64_t)num_q_heads * kD, kD, k_cache, v_cache, kv_dtype,
                               cache_stride_block, cache_stride_tok, cache_stride_head, k_scale,
                               v_scale, block_tables, block_table_stride, block_table_width,
                               num_blocks, cu_seqlens_q, cu_seqlens_k, num_seqs, max_seqlen_q,
                               max_seqlen_k, num_q_heads, num_kv_heads, head_dim, block_size,
                               softmax_scale, out, out_stride_tok, out_stride_head, workspace,
                               workspace_bytes, stream);
  }
  QkvArgs qa;
  qa.qkv = static_cast<const uint16_t*>(qkv);
  qa.ts = token_stride;
  qa.qw = static_cast<const uint16_t*>(q_weight);
  qa.kw = static_cast<const uint16_t*>(k_weight);
  qa.cos_sin = cos_sin;
  qa.positions = positions;
  qa.slots = slot_mapping;
  qa.eps = eps;
  qa.k_scale = k_scale;
  qa.v_scale = v_scale;
  qa.Hq = num_q_heads;
  qa.cs_rows = cos_sin_rows;
  if (a.nsplit > 1) {
    const size_t parts = (size_t)num_seqs * num_kv_heads * a.nsplit * kRows;
    a.part_o = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kTicketBytes);
    a.part_ml = a.part_o + parts * kD;
  } else {
    a.part_o = nullptr;
    a.part_ml = nullptr;
  }
  a.sk_pre = nullptr;
  a.sk_w0 = nullptr;
  a.sk_nwg = 0;
  // kv heads of one split packed onto one XCD when they fit its 32 CUs
  a.xcd_pack = (pairs <= 32) ? 8 : 1;
  const dim3 grid(a.xcd_pack * num_kv_heads, a.nsplit, num_seqs);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.fp8)
    launch_attn_qkv<true>(a.G, grid, s, a, qa);
  else
    launch_attn_qkv<false>(a.G, grid, s, a, qa);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_verify_attention_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache, int kv_dtype,
                                int64_t cache_stride_block, int64_t cache_stride_tok,
                                int64_t cache_stride_head, float k_scale, float v_scale,
                                const int32_t* block_tables, int64_t block_table_stride,
                                int block_table_width, int num_blocks,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int num_seqs, int max_seqlen_q, int max_seqlen_k,
                                int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                float softmax_scale, void* out, int64_t out_stride_tok,
                                int64_t out_stride_head, void* stream) {
  void* ws = scratch_of_current_device();
  if (!ws) return HS_ERR_LAUNCH;
  // same kernels and launch choice as hs_verify_attention with a workspace of
  // the scratch's size: a call whose layout does not fit runs the per-tile
  // grid when that needs no partials, and is rejected otherwise
  const int rc = hs_verify_attention(
      q, q_stride_tok, q_stride_head, k_cache, v_cache, kv_dtype, cache_stride_block,
      cache_stride_tok, cache_stride_head, k_scale, v_scale, block_tables, block_table_stride,
      block_table_width, num_blocks, cu_seqlens_q, cu_seqlens_k, num_seqs, max_seqlen_q,
      max_seqlen_k, num_q_heads, num_kv_heads, head_dim, block_size, softmax_scale, out,
      out_stride_tok, out_stride_head, ws, kNoAllocScratchBytes, stream);
  return rc == HS_ERR_WORKSPACE ? HS_ERR_SCRATCH_LIMIT : rc;
}

size_t hs_verify_attention_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

}  // extern "C"
