/*
 * spec_oracle.c - CPU restatement of the speculative-decoding acceptance path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP kernels in
 * hilda-vllm_amd/csrc; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it. The product path never calls it.
 *
 * It restates, sequentially and with a full sort instead of radix selection:
 *   - the acceptance loop of ModelRunner.run_verify,
 *     mini_vllm/engine/model_runner.py:391-428 (softmax at :398, gathers at
 *     :403-404, ratio and clamp at :406, strict u < a at :408, bonus draw at
 *     :410-414, residual max(P-Q,0) with the 1e-10 fallback at :415-426),
 *     with torch.rand / torch.multinomial replaced by explicit uniforms;
 *   - Sampler._apply_top_k / _apply_top_p, mini_vllm/layers/sampler.py:27-49
 *     (descending order, ties by lower index; strict cumsum < p; keep rank 0);
 *   - Sampler.forward's temperature division, sampler.py:20.
 * Number formats (shared contract with the kernels, written independently):
 *   exp        Cody-Waite reduction + degree-7 Taylor with fmaf, 0 below -86;
 *   fx44(v)    floor(v * 2^44), computed here through double;
 *   f32(n)     C's (float) conversion of a uint64 (round to nearest even);
 *   f32rz(n)   the same rounded toward zero (every softmax normaliser);
 *   softmax normaliser over the whole row: per 2048-element chunk c,
 *              m_c = max x, E_c = sum fx44(exp(x - m_c)); M = max m_c;
 *              S = f32rz(sum_c fx40(f32rz(E_c) 2^-44 * exp(m_c - M))) 2^-40;
 *   normaliser over a strict subset K: f32rz(sum_{i in K} fx44(exp(x_i-M)))2^-44;
 *   top-p cumulative sum: f32(exact sum of fx44(p_r)) 2^-44 compared with p;
 *   draw with uniform u: U = floor(u 2^24) (clamped to 2^24-1),
 *              t = floor(U * W / 2^24), token = min{i : sum_{j<=i} w_j > t}
 *              with w_j = fx44(weight_j) and W = sum_j w_j.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_CHUNK 2048

static float or_exp(float y) {
  if (!(y >= -86.0f)) return 0.0f;
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.428606765330187e-06f;
  float t = y * log2e;
  float k = rintf(t);
  float r = fmaf(-k, ln2_hi, y);
  r = fmaf(-k, ln2_lo, r);
  float p = 1.98412698e-04f;
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

/* exported for the unit tests of the number formats */
float or_exp_f32(float y) { return or_exp(y); }

static uint64_t or_fx(float v, int bits) {
  if (!(v > 0.0f) || isinf(v)) return 0;
  double d = ldexp((double)v, bits); /* exact: 24-bit significand */
  return (uint64_t)floor(d);
}
uint64_t or_fx44(float v) { return or_fx(v, 44); }
static float or_f32(uint64_t n) { return (float)n; }
float or_f32_of_u64(uint64_t n) { return or_f32(n); }
/* toward zero: used for every softmax normaliser */
static float or_f32_rz(uint64_t n) {
  float f = (float)n;
  if ((uint64_t)f > n) f = nextafterf(f, 0.0f);
  return f;
}
float or_f32_rz_of_u64(uint64_t n) { return or_f32_rz(n); }

static uint32_t or_key(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
uint32_t or_key_f32(float x) { return or_key(x); }

/* ---- per-row distribution ------------------------------------------------ */

typedef struct {
  uint32_t key;
  int32_t idx;
} rank_t;

static int rank_cmp(const void* a, const void* b) {
  const rank_t* x = (const rank_t*)a;
  const rank_t* y = (const rank_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

/* x[V] already divided by T. Computes M, the kept mask and its normaliser. */
static void row_dist(const float* x, int V, int topk, float topp, int filtered, float* outM,
                     float* outS, uint8_t* keep) {
  const int nch = (V + OR_CHUNK - 1) / OR_CHUNK;
  float* mc = (float*)malloc(sizeof(float) * nch);
  uint64_t* ec = (uint64_t*)malloc(sizeof(uint64_t) * nch);
  float M = -INFINITY;
  for (int c = 0; c < nch; ++c) {
    int lo = c * OR_CHUNK, hi = lo + OR_CHUNK < V ? lo + OR_CHUNK : V;
    float m = -INFINITY;
    for (int i = lo; i < hi; ++i) m = fmaxf(m, x[i]);
    uint64_t e = 0;
    for (int i = lo; i < hi; ++i) e += or_fx(or_exp(x[i] - m), 44);
    mc[c] = m;
    ec[c] = e;
    if (m > M) M = m;
  }
  uint64_t S = 0;
  for (int c = 0; c < nch; ++c) S += or_fx(ldexpf(or_f32_rz(ec[c]), -44) * or_exp(mc[c] - M), 40);
  float Sfull = ldexpf(or_f32_rz(S), -40);
  free(mc);
  free(ec);

  for (int i = 0; i < V; ++i) keep[i] = 1;
  const int k_on = filtered && topk > 0 && topk < V;
  const int p_on = filtered && topp < 1.0f;
  float Sk = Sfull;
  if (k_on || p_on) {
    rank_t* rk = (rank_t*)malloc(sizeof(rank_t) * V);
    for (int i = 0; i < V; ++i) {
      rk[i].key = or_key(x[i]);
      rk[i].idx = i;
    }
    qsort(rk, V, sizeof(rank_t), rank_cmp);
    int nA = k_on ? topk : V;
    float SA = Sfull;
    if (k_on) {
      uint64_t s = 0;
      for (int r = 0; r < nA; ++r) s += or_fx(or_exp(x[rk[r].idx] - M), 44);
      SA = ldexpf(or_f32_rz(s), -44);
    }
    int nB = nA;
    if (p_on) {
      uint64_t cum = 0;
      nB = 0;
      for (int r = 0; r < nA; ++r) {
        float m = or_exp(x[rk[r].idx] - M) / SA;
        cum += or_fx(m, 44);
        float c = ldexpf(or_f32(cum), -44);
        if (r == 0 || c < topp) nB = r + 1;
        else break;
      }
    }
    for (int i = 0; i < V; ++i) keep[i] = 0;
    for (int r = 0; r < nB; ++r) keep[rk[r].idx] = 1;
    if (nB == V) {
      Sk = Sfull;
    } else if (nB == nA && k_on) {
      Sk = SA;
    } else {
      uint64_t s = 0;
      for (int r = 0; r < nB; ++r) s += or_fx(or_exp(x[rk[r].idx] - M), 44);
      Sk = ldexpf(or_f32_rz(s), -44);
    }
    free(rk);
  }
  *outM = M;
  *outS = Sk;
}

static float prob_of(const float* x, const uint8_t* keep, float M, float S, int i) {
  return keep[i] ? or_exp(x[i] - M) / S : 0.0f;
}

static uint32_t or_u24(float u) {
  if (!(u > 0.0f)) return 0u;
  float s = u * 16777216.0f;
  if (s >= 16777215.0f) return 16777215u;
  return (uint32_t)s;
}

/* inverse-CDF draw over integer weights w[V] */
static int64_t draw(const uint64_t* w, int V, float u) {
  unsigned __int128 W = 0;
  for (int i = 0; i < V; ++i) W += w[i];
  unsigned __int128 t = ((unsigned __int128)or_u24(u) * W) >> 24;
  unsigned __int128 acc = 0;
  for (int i = 0; i < V; ++i) {
    acc += w[i];
    if (acc > t) return i;
  }
  return -1;
}

static int64_t argmax_row(const float* v, int V) {
  int64_t best = 0;
  uint32_t bk = or_key(v[0]);
  for (int i = 1; i < V; ++i) {
    uint32_t k = or_key(v[i]);
    if (k > bk) {
      bk = k;
      best = i;
    }
  }
  return best;
}

/* mode: 0 reference, 1 filtered, 2 greedy (same values as the C ABI) */
int or_spec_accept(const float* logits, int B, int gamma, int V, const float* q,
                   const int64_t* dtok, const float* temps, const int32_t* top_ks,
                   const float* top_ps, const float* u_acc, const float* u_res, int mode,
                   int32_t* nacc, int64_t* out_tokens, int32_t* out_len, float* row_stats,
                   float* probs_out) {
  const int R = gamma + 1;
  float* x = (float*)malloc(sizeof(float) * (size_t)R * V);
  uint8_t* keep = (uint8_t*)malloc((size_t)R * V);
  float* Ms = (float*)malloc(sizeof(float) * R);
  float* Ss = (float*)malloc(sizeof(float) * R);
  uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * V);
  for (int b = 0; b < B; ++b) {
    const float* lb = logits + (size_t)b * R * V;
    int64_t* ob = out_tokens + (size_t)b * R;
    for (int j = 0; j < R; ++j) ob[j] = -1;
    if (mode == 2) {
      int r = gamma;
      for (int j = 0; j < gamma; ++j) {
        if (dtok[(size_t)b * gamma + j] != argmax_row(lb + (size_t)j * V, V)) {
          r = j;
          break;
        }
      }
      for (int j = 0; j < r; ++j) ob[j] = dtok[(size_t)b * gamma + j];
      ob[r] = argmax_row(lb + (size_t)r * V, V);
      nacc[b] = r;
      out_len[b] = r + 1;
      continue;
    }
    const float T = temps[b];
    for (int j = 0; j < R; ++j) {
      float* xj = x + (size_t)j * V;
      for (int i = 0; i < V; ++i) xj[i] = (T == 1.0f) ? lb[(size_t)j * V + i] : lb[(size_t)j * V + i] / T;
      row_dist(xj, V, top_ks ? top_ks[b] : 0, top_ps ? top_ps[b] : 1.0f, mode == 1, &Ms[j], &Ss[j],
               keep + (size_t)j * V);
      if (row_stats) {
        row_stats[2 * ((size_t)b * R + j)] = Ms[j];
        row_stats[2 * ((size_t)b * R + j) + 1] = Ss[j];
      }
      if (probs_out)
        for (int i = 0; i < V; ++i)
          probs_out[((size_t)b * R + j) * V + i] =
              prob_of(xj, keep + (size_t)j * V, Ms[j], Ss[j], i);
    }
    int r = gamma;
    for (int j = 0; j < gamma; ++j) {
      int64_t d = dtok[(size_t)b * gamma + j];
      float pt = 0.0f, pd = 0.0f;
      if (d >= 0 && d < V) {
        pt = prob_of(x + (size_t)j * V, keep + (size_t)j * V, Ms[j], Ss[j], (int)d);
        pd = q[((size_t)b * gamma + j) * V + d];
      }
      float ratio = pt / fmaxf(pd, 1e-10f);
      float a = fminf(ratio, 1.0f);
      if (!(u_acc[(size_t)b * gamma + j] < a)) {
        r = j;
        break;
      }
    }
    const float* xr = x + (size_t)r * V;
    const uint8_t* kr = keep + (size_t)r * V;
    int use_res = 0;
    if (r < gamma) {
      const float* qr = q + ((size_t)b * gamma + r) * V;
      uint64_t W = 0;
      for (int i = 0; i < V; ++i) {
        float p = prob_of(xr, kr, Ms[r], Ss[r], i);
        w[i] = or_fx(fmaxf(p - qr[i], 0.0f), 44);
        W += w[i];
      }
      use_res = ldexpf(or_f32(W), -44) > 1e-10f;
    }
    if (!use_res)
      for (int i = 0; i < V; ++i) w[i] = or_fx(prob_of(xr, kr, Ms[r], Ss[r], i), 44);
    for (int j = 0; j < r; ++j) ob[j] = dtok[(size_t)b * gamma + j];
    ob[r] = draw(w, V, u_res[b]);
    nacc[b] = r;
    out_len[b] = r + 1;
  }
  free(x);
  free(keep);
  free(Ms);
  free(Ss);
  free(w);
  return 0;
}

int or_sampler(const float* logits, int rows, int V, const float* temps, const int32_t* top_ks,
               const float* top_ps, int mode, float* probs_out, const float* uniforms,
               int64_t* tokens_out, float* row_stats) {
  float* x = (float*)malloc(sizeof(float) * V);
  uint8_t* keep = (uint8_t*)malloc(V);
  uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * V);
  for (int r = 0; r < rows; ++r) {
    const float* lr = logits + (size_t)r * V;
    if (mode == 2) {
      tokens_out[r] = argmax_row(lr, V);
      continue;
    }
    const float T = temps[r];
    for (int i = 0; i < V; ++i) x[i] = (T == 1.0f) ? lr[i] : lr[i] / T;
    float M, S;
    row_dist(x, V, top_ks ? top_ks[r] : 0, top_ps ? top_ps[r] : 1.0f, mode == 1, &M, &S, keep);
    if (row_stats) {
      row_stats[2 * (size_t)r] = M;
      row_stats[2 * (size_t)r + 1] = S;
    }
    for (int i = 0; i < V; ++i) {
      float p = prob_of(x, keep, M, S, i);
      if (probs_out) probs_out[(size_t)r * V + i] = p;
      w[i] = or_fx(p, 44);
    }
    if (uniforms && tokens_out) tokens_out[r] = draw(w, V, uniforms[r]);
  }
  free(x);
  free(keep);
  free(w);
  return 0;
}

/* kept-set size of one row (for tests of the filter) */
int or_filter_keep(const float* logits_row, int V, float T, int topk, float topp, uint8_t* keep,
                   float* M, float* S) {
  if (V <= 0) return 0;
  float* x = (float*)malloc(sizeof(float) * V);
  for (int i = 0; i < V; ++i) x[i] = (T == 1.0f) ? logits_row[i] : logits_row[i] / T;
  row_dist(x, V, topk, topp, 1, M, S, keep);
  int n = 0;
  for (int i = 0; i < V; ++i) n += keep[i];
  free(x);
  return n;
}
