/*
 * dsmoe oracle — TEST INFRASTRUCTURE ONLY (see dsmoe_oracle.h).
 *
 * CPU restatement of the reference MoE-FFN path.  Build with
 * -O2 -ffp-contract=off (oracle/Makefile): the reference's Rust source has
 * IEEE semantics without FMA contraction, and so does this file.
 *
 * Reductions follow the reference thread structure, written as the same
 * sums in the same order:
 *   - matmul_f16 (matmul.rs:57-105): 256 strided partial sums, then the
 *     halving tree 128..1 in shared memory;
 *   - 8-lane xor butterfly (moe.rs:35-41) over lane-strided block sums,
 *     which for lane 0 equals the halving tree 4,2,1;
 *   - 32-lane shuffle_down sum (matmul.rs:10-17): halving tree 16..1.
 *
 * Pinning (what checks each function besides the GPU comparison):
 *   or_f16_to_f32                  exhaustive over all 65536 inputs vs numpy f16 + FTZ rule
 *   or_expf/or_logf/or_softplus    float64 numpy within a few ulp; quant_cpu.rs:453-501 known answers
 *   or_dot_iq2_xxs_q8k / bsum      quant_cpu.rs:304-364 known answers; brute-force int64
 *                                  dequantised dot; closed form single sub-block
 *   or_dot_q2k_q8k                 quant_cpu.rs:393-429 known answers; brute-force int64
 *   or_q8k_quantize                kernels_smoke.rs:518-610-style answers; bsums == sum(qs);
 *                                  signed-amax maps to -127; zero block
 *   or_q8_0_quantize/or_q8_0_matvec kernels_smoke.rs:150-302, 518-610 known answers
 *   or_router_select               brute-force full sort by (score desc, index asc);
 *                                  weights sum to route_scale; ratio preservation
 *   grouped routing (n_group > 1)  brute force over all group subsets (no reference
 *                                  counterpart: the reference has no group-limited top-k)
 *   or_router_select_hash          hand-computed weights on a tiny table (logits > 20 are their
 *                                  own softplus: probabilities 6, 8, 10; an id of -1 weighs 0;
 *                                  the 2^-14 floor); out-of-range tokens take row 0
 *                                  (moe.rs:92-159)
 *   or_dispatch                    numpy stable argsort; prefix sums
 *   or_moe_sum                     f32 values whose sum depends on the slot order
 *   or_rms_norm_plain              float64 within f32 rounding; exact on dyadic rows with eps 0
 *   or_hc4_split / or_hc_split_norm closed forms: sigmoid(+-ln 3) per section scale; uniform comb
 *                                  logits with eps = 0.5 follow x <- x / (eps + 4x) once per
 *                                  column pass and twice per round (pins eps placement and the
 *                                  round count); a permutation-pattern comb with eps = 0 is
 *                                  already doubly stochastic (pins the indexing); plus float64
 *                                  (weighted sum, norm) and Sinkhorn invariants; exp bits as
 *                                  or_expf (parity unpinned against the reference GPU's exp)
 *   or_hc_expand                   dyadic inputs (exact in f32) vs the float64 formula, with
 *                                  a non-symmetric comb; numpy f32 in the reference's order
 *   or_moe_forward                 float64 dequantise-then-GEMM closed form through the same
 *                                  activation quantizers, within 1e-3, with the SwiGLU clamp
 *                                  active on ~18 % of the products
 */
#include "dsmoe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* small parallel-for over [0, n)                                      */
/* ------------------------------------------------------------------ */
typedef void (*range_fn)(void* ctx, int lo, int hi);
typedef struct { range_fn fn; void* ctx; int lo, hi; } pf_job;
static void* pf_run(void* p) { pf_job* j = (pf_job*)p; j->fn(j->ctx, j->lo, j->hi); return NULL; }
static void parallel_for(int n, int nthreads, range_fn fn, void* ctx) {
  if (nthreads <= 1 || n < 2) { fn(ctx, 0, n); return; }
  if (nthreads > n) nthreads = n;
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  pf_job jobs[256];
  for (int i = 0; i < nthreads; i++) {
    jobs[i].fn = fn; jobs[i].ctx = ctx;
    jobs[i].lo = (int)((long long)n * i / nthreads);
    jobs[i].hi = (int)((long long)n * (i + 1) / nthreads);
  }
  for (int i = 1; i < nthreads; i++) pthread_create(&th[i], NULL, pf_run, &jobs[i]);
  pf_run(&jobs[0]);
  for (int i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------ */
/* scalar helpers                                                      */
/* ------------------------------------------------------------------ */
static const uint64_t kGrid[256] = {
#include "iq2xxs_grid.inc"
};

static inline float bits2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rdf32(const uint8_t* p) {
  return bits2f((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}
static inline int16_t rdi16(const uint8_t* p) { return (int16_t)rd16(p); }

/* utils.rs:16-29 — subnormal halves flush to zero */
float or_f16_to_f32(uint16_t h) {
  uint32_t u = h, sign = (u & 0x8000u) << 16, ex = (u >> 10) & 0x1Fu, man = u & 0x3FFu, b;
  if (ex == 0) b = sign;
  else if (ex == 31) b = sign | 0x7F800000u | (man << 13);
  else b = sign | ((ex + 112u) << 23) | (man << 13);
  return bits2f(b);
}

uint64_t or_iq2_grid(uint32_t idx) { return kGrid[idx & 255]; }

/* quantize.rs:693-709: table entry = index with bit 7 set to make popcount even */
uint8_t or_iq2_sign(uint32_t idx7) {
  uint32_t p = 0;
  for (int i = 0; i < 7; i++) p ^= (idx7 >> i) & 1u;
  return (uint8_t)(idx7 | (p << 7));
}

/* exp / log: the build's fixed method (the reference's device math is not
 * reproducible off its toolchain).  Cody-Waite + degree-7 Taylor; log via
 * 2*atanh series.  Same steps as deepseek-rs_amd/csrc/dsmoe_math.h. */
static inline float p2i(int n) { return bits2f((uint32_t)(n + 127) << 23); }
float or_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return bits2f(0x7F800000u);
  if (x < -103.97208404541015625f) return 0.0f;
  float t = x * 1.44269502162933349609375f;
  int n = (int)(t >= 0.0f ? t + 0.5f : t - 0.5f);
  float fn = (float)n;
  float r = (x - fn * 0.693145751953125f) - fn * 1.428606765330187045e-06f;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  if (n > 127) return (p * 2.0f) * p2i(n - 1);
  if (n < -126) return (p * p2i(n + 64)) * p2i(-64);
  return p * p2i(n);
}
float or_logf(float y) {
  if (y != y || y < 0.0f) return bits2f(0x7FC00000u);
  if (y == 0.0f) return bits2f(0xFF800000u);
  if (y == bits2f(0x7F800000u)) return y;
  int e = 0;
  if (y < 1.17549435e-38f) { y = y * 8388608.0f; e = -23; }
  uint32_t b = f2bits(y);
  e += (int)(b >> 23) - 127;
  float m = bits2f((b & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421353816986083984375f) { m = m * 0.5f; e += 1; }
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float z = s * s;
  float q = 2.0f / 11.0f;
  q = q * z + 2.0f / 9.0f;
  q = q * z + 2.0f / 7.0f;
  q = q * z + 2.0f / 5.0f;
  q = q * z + 2.0f / 3.0f;
  float lm = 2.0f * s + s * (z * q);
  float fe = (float)e;
  return fe * 0.693145751953125f + (fe * 1.428606765330187045e-06f + lm);
}
/* moe.rs:12-24 */
float or_softplus(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return or_expf(x);
  return or_logf(1.0f + or_expf(x));
}
/* moe.rs:706 / utils.rs:160 */
float or_silu(float g) { return g / (1.0f + or_expf(-g)); }

/* Rust `(v) as i32` followed by the [-128, 127] clamp of quantize.rs:389-401 */
static inline int8_t sat_i8_trunc(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)(int)v;
}

/* ------------------------------------------------------------------ */
/* block dots                                                          */
/* ------------------------------------------------------------------ */
/* quantize.rs:711-724 dot_iq2_dp8 */
static int32_t iq2_dp8(uint64_t grid, uint8_t sign_byte, const int8_t* q8) {
  uint32_t p = 0;
  for (int i = 0; i < 8; i++) p ^= (sign_byte >> i) & 1u;
  uint8_t sb = (uint8_t)(sign_byte ^ (p << 7));
  int32_t acc = 0;
  for (int i = 0; i < 8; i++) {
    int8_t g = (int8_t)((grid >> (8 * i)) & 0xFF);
    int8_t w = ((sb >> i) & 1) ? (int8_t)(-g) : g;
    acc += (int32_t)w * (int32_t)q8[i];
  }
  return acc;
}

/* quantize.rs:763-812 integer part */
int32_t or_iq2_xxs_bsum(const uint8_t* iq2, const uint8_t* q8k) {
  const int8_t* q8 = (const int8_t*)(q8k + 4);
  const uint8_t* qs = iq2 + 2;
  int32_t bsum = 0;
  for (int ib = 0; ib < 8; ib++) {
    const uint8_t* q2 = qs + ib * 8;
    uint32_t aux0 = (uint32_t)rd16(q2) | ((uint32_t)rd16(q2 + 2) << 16);
    uint32_t aux1 = (uint32_t)rd16(q2 + 4) | ((uint32_t)rd16(q2 + 6) << 16);
    int32_t ls = (int32_t)(2 * (aux1 >> 28) + 1);
    int32_t sumi = 0;
    for (int g = 0; g < 4; g++) {
      uint64_t gr = kGrid[(aux0 >> (8 * g)) & 0xFF];
      uint8_t s = or_iq2_sign((aux1 >> (7 * g)) & 127);
      sumi += iq2_dp8(gr, s, q8 + ib * 32 + g * 8);
    }
    bsum += sumi * ls;
  }
  return bsum;
}

/* quantize.rs:763-812: 0.125 * xd * yd * bsum, evaluated left to right */
float or_dot_iq2_xxs_q8k(const uint8_t* iq2, const uint8_t* q8k) {
  float xd = or_f16_to_f32(rd16(iq2));
  float yd = rdf32(q8k);
  int32_t bsum = or_iq2_xxs_bsum(iq2, q8k);
  return 0.125f * xd * yd * (float)bsum;
}

/* quantize.rs:818-843 dot_q2_16 */
static int32_t q2_16(const uint8_t* q2, const int8_t* q8, int shift) {
  int32_t sum = 0;
  for (int i = 0; i < 16; i++) sum += (int32_t)((q2[i] >> shift) & 3) * (int32_t)q8[i];
  return sum;
}

/* quantize.rs:846-901 integer parts */
void or_q2k_isum_summs(const uint8_t* q2k, const uint8_t* q8k, int32_t* isum_out, int32_t* summs_out) {
  const uint8_t* sc = q2k;
  const uint8_t* q2 = q2k + 16;
  const int8_t* q8 = (const int8_t*)(q8k + 4);
  int32_t summs = 0;
  for (int j = 0; j < 16; j++) summs += (int32_t)rdi16(q8k + 260 + 2 * j) * (int32_t)(sc[j] >> 4);
  int32_t isum = 0;
  int is = 0, q2o = 0, q8o = 0;
  for (int k = 0; k < 2; k++) {
    int shift = 0;
    for (int j = 0; j < 4; j++) {
      isum += (int32_t)(sc[is++] & 0xF) * q2_16(q2 + q2o, q8 + q8o, shift);
      isum += (int32_t)(sc[is++] & 0xF) * q2_16(q2 + q2o + 16, q8 + q8o + 16, shift);
      shift += 2;
      q8o += 32;
    }
    q2o += 32;
  }
  *isum_out = isum;
  *summs_out = summs;
}

/* quantize.rs:846-901: dall*isum - dmin*summs with dall = yd*d, dmin = yd*dmin */
float or_dot_q2k_q8k(const uint8_t* q2k, const uint8_t* q8k) {
  float yd = rdf32(q8k);
  float dall = yd * or_f16_to_f32(rd16(q2k + 80));
  float dmin = yd * or_f16_to_f32(rd16(q2k + 82));
  int32_t isum, summs;
  or_q2k_isum_summs(q2k, q8k, &isum, &summs);
  return dall * (float)isum - dmin * (float)summs;
}

/* ------------------------------------------------------------------ */
/* activation quantizers                                               */
/* ------------------------------------------------------------------ */
/* quantize.rs:309-417 q8k_quantize: signed-amax tree (strict >), iscale =
 * -127/max, d = 1/iscale, q = trunc(iscale*x +- 0.5) saturated, bsums */
void or_q8k_quantize(const float* x, uint8_t* out, int in_dim, int rows) {
  int nb = in_dim / 256;
  for (int r = 0; r < rows; r++) {
    for (int b = 0; b < nb; b++) {
      const float* xb = x + (size_t)r * in_dim + (size_t)b * 256;
      uint8_t* yb = out + ((size_t)r * nb + b) * 292;
      float ab[256], vv[256];
      for (int t = 0; t < 256; t++) { float v = xb[t]; ab[t] = v < 0.0f ? -v : v; vv[t] = v; }
      for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; t++)
          if (ab[t + s] > ab[t]) { ab[t] = ab[t + s]; vv[t] = vv[t + s]; }
      if (ab[0] == 0.0f) { memset(yb, 0, 292); continue; }
      float iscale = -127.0f / vv[0];
      float d = 1.0f / iscale;
      memcpy(yb, &d, 4);
      int8_t* qs = (int8_t*)(yb + 4);
      for (int t = 0; t < 256; t++) {
        float raw = iscale * xb[t];
        qs[t] = sat_i8_trunc(raw >= 0.0f ? raw + 0.5f : raw - 0.5f);
      }
      for (int j = 0; j < 16; j++) {
        int32_t s = 0;
        for (int k = 0; k < 16; k++) s += qs[j * 16 + k];
        int16_t s16 = (int16_t)s;
        memcpy(yb + 260 + 2 * j, &s16, 2);
      }
    }
  }
}

/* quantize.rs:147-225 quantize_q8_0: abs-max 16-way tree, d = amax/127,
 * id = 1/d (0 if d == 0), q = trunc(v*id +- 0.5) saturated */
void or_q8_0_quantize(const float* x, int8_t* xq, float* xscale, int in_dim, int rows) {
  int nb = (in_dim + 31) / 32;
  for (int r = 0; r < rows; r++) {
    for (int b = 0; b < nb; b++) {
      int i0 = b * 32, bn = in_dim - i0 < 32 ? in_dim - i0 : 32;
      const float* xb = x + (size_t)r * in_dim + i0;
      float v[32], a[32];
      for (int t = 0; t < 32; t++) { v[t] = t < bn ? xb[t] : 0.0f; a[t] = v[t] < 0.0f ? -v[t] : v[t]; }
      for (int s = 16; s > 0; s >>= 1)
        for (int t = 0; t < s; t++)
          if (a[t + s] > a[t]) a[t] = a[t + s];
      float d = a[0] / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      xscale[(size_t)r * nb + b] = d;
      for (int t = 0; t < 32; t++) {
        int8_t q = 0;
        if (t < bn) { float raw = v[t] * id; q = sat_i8_trunc(raw >= 0.0f ? raw + 0.5f : raw - 0.5f); }
        xq[((size_t)r * nb + b) * 32 + t] = q;
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* router                                                              */
/* ------------------------------------------------------------------ */
typedef struct { const uint16_t* w; const float* x; float* out; int d, E, T; } rl_ctx;
static void rl_range(void* p, int lo, int hi) {
  rl_ctx* c = (rl_ctx*)p;
  float part[256];
  for (int idx = lo; idx < hi; idx++) {
    int tok = idx / c->E, row = idx % c->E;
    const uint16_t* wr = c->w + (size_t)row * c->d;
    const float* xr = c->x + (size_t)tok * c->d;
    for (int tx = 0; tx < 256; tx++) {
      float s = 0.0f;
      for (int i = tx; i < c->d; i += 256) s += or_f16_to_f32(wr[i]) * xr[i];
      part[tx] = s;
    }
    for (int s = 128; s > 0; s >>= 1)
      for (int tx = 0; tx < s; tx++) part[tx] += part[tx + s];
    c->out[(size_t)tok * c->E + row] = part[0];
  }
}
/* matmul.rs:57-105 matmul_f16, block 256 */
void or_router_logits(const uint16_t* w, const float* x, float* out, int d, int E, int T, int nthreads) {
  rl_ctx c = {w, x, out, d, E, T};
  parallel_for(E * T, nthreads, rl_range, &c);
}

/* insertion of (score, index) into a descending list of length n with
 * strict-greater comparison (moe.rs:243-262): ties keep the earlier index */
static void insert_topk(int32_t* sel, int n, const float* score, int e) {
  float s = score[e];
  for (int j = 0; j < n; j++) {
    float cur = sel[j] < 0 ? -INFINITY : score[sel[j]];
    if (s > cur) {
      for (int k = n - 1; k > j; k--) sel[k] = sel[k - 1];
      sel[j] = e;
      return;
    }
  }
}

/* moe.rs:177-287 router_select_parallel (n_group == 1), generalised to
 * E experts / top-k / route_scale; n_group > 1 adds group-limited
 * selection (group score = best + second best biased score). */
/* Hash routing (moe.rs:92-109 with the weights of :143-159): the token id
 * picks the k experts from the table (token ids outside [0, hash_rows) use
 * row 0; no token array = token_scalar for every token); probs are
 * sqrt(softplus(logit)) as in top-k routing; weight j = probs[e_j] (0 for an
 * id outside [0, E)) / (max(sum in slot order, 2^-14) / route_scale). */
void or_router_select_hash(const or_config* c, const float* logits, const int32_t* hash, int hash_rows,
                           const int32_t* tokens, int token_scalar, int T, float* probs, int32_t* selected,
                           float* weights) {
  const int E = c->n_expert, K = c->top_k;
  for (int t = 0; t < T; t++) {
    if (probs)
      for (int e = 0; e < E; e++) probs[(size_t)t * E + e] = sqrtf(or_softplus(logits[(size_t)t * E + e]));
    int tok = tokens ? tokens[t] : token_scalar;
    if (tok < 0 || tok >= hash_rows) tok = 0;
    float sum = 0.0f;
    for (int j = 0; j < K; j++) {
      const int e = hash[(size_t)tok * K + j];
      selected[(size_t)t * K + j] = e;
      const float v = (e >= 0 && e < E) ? sqrtf(or_softplus(logits[(size_t)t * E + e])) : 0.0f;
      weights[(size_t)t * K + j] = v;
      sum += v;
    }
    if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
    for (int j = 0; j < K; j++) weights[(size_t)t * K + j] /= sum / c->route_scale;
  }
}

void or_router_select(const or_config* c, const float* logits, const float* bias, int T,
                      float* probs, int32_t* selected, float* weights) {
  int E = c->n_expert, K = c->top_k;
  float* p = (float*)malloc(sizeof(float) * E);
  float* sc = (float*)malloc(sizeof(float) * E);
  float* gs = (float*)malloc(sizeof(float) * (c->n_group > 0 ? c->n_group : 1));
  int32_t* gsel = (int32_t*)malloc(sizeof(int32_t) * (c->n_group > 0 ? c->n_group : 1));
  for (int t = 0; t < T; t++) {
    for (int e = 0; e < E; e++) {
      p[e] = sqrtf(or_softplus(logits[(size_t)t * E + e]));
      if (probs) probs[(size_t)t * E + e] = p[e];
      sc[e] = c->has_bias ? p[e] + bias[e] : p[e];
    }
    int32_t* sel = selected + (size_t)t * K;
    for (int j = 0; j < K; j++) sel[j] = -1;
    if (c->n_group <= 1) {
      for (int e = 0; e < E; e++) insert_topk(sel, K, sc, e);
    } else {
      int G = c->n_group, gsz = E / G, TG = c->topk_group;
      for (int g = 0; g < G; g++) {
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int e = g * gsz; e < (g + 1) * gsz; e++) {
          float s = sc[e];
          if (s > b1) { b2 = b1; b1 = s; } else if (s > b2) { b2 = s; }
        }
        gs[g] = gsz >= 2 ? b1 + b2 : b1;
      }
      for (int j = 0; j < TG; j++) gsel[j] = -1;
      for (int g = 0; g < G; g++) insert_topk(gsel, TG, gs, g);
      for (int e = 0; e < E; e++) {
        int g = e / gsz, ok = 0;
        for (int j = 0; j < TG; j++) ok |= (gsel[j] == g);
        if (ok) insert_topk(sel, K, sc, e);
      }
    }
    float* w = weights + (size_t)t * K;
    float sum = 0.0f;
    for (int j = 0; j < K; j++) {
      int e = sel[j];
      float v = (e >= 0 && e < E) ? p[e] : 0.0f;
      w[j] = v;
      sum += v;
    }
    if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
    for (int j = 0; j < K; j++) w[j] /= sum / c->route_scale;
  }
  free(p); free(sc); free(gs); free(gsel);
}

/* ------------------------------------------------------------------ */
/* Q8_0 matvec + swiglu (shared expert)                                */
/* ------------------------------------------------------------------ */
typedef struct { const uint8_t* w; const int8_t* xq; const float* xs; float* out; int in_dim, out_dim, T; } qm_ctx;
static void qm_range(void* p, int lo, int hi) {
  qm_ctx* c = (qm_ctx*)p;
  int nb = (c->in_dim + 31) / 32;
  for (int idx = lo; idx < hi; idx++) {
    int tok = idx / c->out_dim, row = idx % c->out_dim;
    const uint8_t* wr = c->w + (size_t)row * nb * 34;
    const int8_t* xq = c->xq + (size_t)tok * nb * 32;
    const float* xs = c->xs + (size_t)tok * nb;
    float lane[32];
    for (int l = 0; l < 32; l++) {
      float acc = 0.0f;
      for (int b = l; b < nb; b += 32) {
        int i0 = b * 32, bn = c->in_dim - i0 < 32 ? c->in_dim - i0 : 32;
        const uint8_t* blk = wr + (size_t)b * 34;
        float scale = or_f16_to_f32(rd16(blk));
        int32_t dot = 0;
        for (int i = 0; i < bn; i++) dot += (int32_t)(int8_t)blk[2 + i] * (int32_t)xq[b * 32 + i];
        acc += scale * xs[b] * (float)dot;
      }
      lane[l] = acc;
    }
    for (int s = 16; s > 0; s >>= 1)
      for (int l = 0; l < s; l++) lane[l] += lane[l + s];
    c->out[(size_t)tok * c->out_dim + row] = lane[0];
  }
}
/* matmul.rs:357-458 matmul_q8_0_preq_warp8 / _batch_warp8 */
void or_q8_0_matvec(const uint8_t* w, const int8_t* xq, const float* xscale, float* out,
                    int in_dim, int out_dim, int T, int nthreads) {
  qm_ctx c = {w, xq, xscale, out, in_dim, out_dim, T};
  parallel_for(out_dim * T, nthreads, qm_range, &c);
}

/* utils.rs:141-163 */
void or_swiglu(const float* gate, const float* up, float* out, int n, float clamp, float weight) {
  for (int i = 0; i < n; i++) {
    float g = gate[i], u = up[i];
    if (clamp > 1.0e-6f) {
      if (g > clamp) g = clamp;
      if (u > clamp) u = clamp;
      if (u < -clamp) u = -clamp;
    }
    float s = g / (1.0f + or_expf(-g));
    out[i] = s * u * weight;
  }
}

/* ------------------------------------------------------------------ */
/* routed experts                                                      */
/* ------------------------------------------------------------------ */
typedef struct {
  const uint8_t *gate, *up, *xq; const int32_t* sel; const float* wts;
  float *g_out, *u_out, *m_out; int d, I, T, k; float clamp;
} gu_ctx;
static void gu_range(void* p, int lo, int hi) {
  gu_ctx* c = (gu_ctx*)p;
  int nb = c->d / 256;
  size_t row_bytes = (size_t)nb * 66, exp_bytes = (size_t)c->I * row_bytes;
  for (int idx = lo; idx < hi; idx++) {
    int pair = idx / c->I, row = idx % c->I;
    int tok = pair / c->k;
    int e = c->sel[pair]; if (e < 0) e = 0;
    const uint8_t* gr = c->gate + (size_t)e * exp_bytes + (size_t)row * row_bytes;
    const uint8_t* ur = c->up + (size_t)e * exp_bytes + (size_t)row * row_bytes;
    const uint8_t* xq = c->xq + (size_t)tok * nb * 292;
    float lg[8], lu[8];
    for (int l = 0; l < 8; l++) {
      float ga = 0.0f, ua = 0.0f;
      for (int b = l; b < nb; b += 8) {
        ga += or_dot_iq2_xxs_q8k(gr + (size_t)b * 66, xq + (size_t)b * 292);
        ua += or_dot_iq2_xxs_q8k(ur + (size_t)b * 66, xq + (size_t)b * 292);
      }
      lg[l] = ga; lu[l] = ua;
    }
    for (int s = 4; s > 0; s >>= 1)
      for (int l = 0; l < s; l++) { lg[l] += lg[l + s]; lu[l] += lu[l + s]; }
    float g = lg[0], u = lu[0];
    if (c->clamp > 1.0e-6f) {
      if (g > c->clamp) g = c->clamp;
      if (u > c->clamp) u = c->clamp;
      if (u < -c->clamp) u = -c->clamp;
    }
    size_t off = (size_t)pair * c->I + row;
    if (c->g_out) c->g_out[off] = g;
    if (c->u_out) c->u_out[off] = u;
    c->m_out[off] = (g / (1.0f + or_expf(-g))) * u * c->wts[pair];
  }
}
/* moe.rs:622-715 moe_gate_up_mid_qwarp32 (pair = tok*k + slot) */
void or_gate_up_mid(const uint8_t* gate, const uint8_t* up, const uint8_t* xq,
                    const int32_t* selected, const float* weights,
                    float* gate_out, float* up_out, float* mid_out,
                    int d, int I, int T, int k, float clamp, int nthreads) {
  gu_ctx c = {gate, up, xq, selected, weights, gate_out, up_out, mid_out, d, I, T, k, clamp};
  parallel_for(T * k * I, nthreads, gu_range, &c);
}

typedef struct { const uint8_t *down, *midq; const int32_t* sel; float* out; int d, I, T, k; } dn_ctx;
static void dn_range(void* p, int lo, int hi) {
  dn_ctx* c = (dn_ctx*)p;
  int nb = c->I / 256;
  size_t row_bytes = (size_t)nb * 84, exp_bytes = (size_t)c->d * row_bytes;
  for (int idx = lo; idx < hi; idx++) {
    int pair = idx / c->d, row = idx % c->d;
    int e = c->sel[pair]; if (e < 0) e = 0;
    const uint8_t* wr = c->down + (size_t)e * exp_bytes + (size_t)row * row_bytes;
    const uint8_t* mq = c->midq + (size_t)pair * nb * 292;
    float lane[8];
    for (int l = 0; l < 8; l++) {
      float a = 0.0f;
      for (int b = l; b < nb; b += 8) a += or_dot_q2k_q8k(wr + (size_t)b * 84, mq + (size_t)b * 292);
      lane[l] = a;
    }
    for (int s = 4; s > 0; s >>= 1)
      for (int l = 0; l < s; l++) lane[l] += lane[l + s];
    c->out[(size_t)pair * c->d + row] = lane[0];
  }
}
/* moe.rs:821-866 moe_down_qwarp32 -> down_out[pair, d] */
void or_down(const uint8_t* down, const uint8_t* midq, const int32_t* selected,
             float* down_out, int d, int I, int T, int k, int nthreads) {
  dn_ctx c = {down, midq, selected, down_out, d, I, T, k};
  parallel_for(T * k * d, nthreads, dn_range, &c);
}

/* moe.rs:983-1005 moe_sum (slot order; equals moe_down_sum6 :922-970) */
void or_moe_sum(const float* down, float* out, int d, int k, int T) {
  for (int t = 0; t < T; t++)
    for (int r = 0; r < d; r++) {
      float acc = 0.0f;
      for (int s = 0; s < k; s++) acc += down[((size_t)t * k + s) * d + r];
      out[(size_t)t * d + r] = acc;
    }
}

/* rms_norm_plain (engine/src/kernels/norm.rs:14-63): 256 lane-strided sums
 * of squares, the halving tree 128..1, scale = 1 / sqrt(sum / n + eps),
 * out = x * scale. */
void or_rms_norm_plain(const float* x, float* out, int n, int rows, float eps) {
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * n;
    float part[256];
    for (int l = 0; l < 256; l++) {
      float s = 0.0f;
      for (int i = l; i < n; i += 256) s += xr[i] * xr[i];
      part[l] = s;
    }
    for (int st = 128; st > 0; st >>= 1)
      for (int l = 0; l < st; l++) part[l] += part[l + st];
    const float scale = 1.0f / sqrtf(part[0] / (float)n + eps);
    for (int i = 0; i < n; i++) out[(size_t)r * n + i] = xr[i] * scale;
  }
}

/* hc4_split_one (engine/src/kernels/hc.rs:17-99): out[0..4) = sigmoid(mix *
 * s0 + base) + eps, out[4..8) = 2 sigmoid(mix * s1 + base), out[8..24) =
 * the 4x4 comb: row softmax of mix * s2 + base (+ eps), a column
 * normalisation, then iters - 1 Sinkhorn rounds (rows, then columns; every
 * sum starts at eps). */
void or_hc4_split(const float* mix, const float* scale, const float* base, int iters, float eps, float* out) {
  for (int i = 0; i < 4; i++) {
    const float z = mix[i] * scale[0] + base[i];
    out[i] = 1.0f / (1.0f + or_expf(-z)) + eps;
  }
  for (int i = 0; i < 4; i++) {
    const float z = mix[4 + i] * scale[1] + base[4 + i];
    out[4 + i] = 2.0f / (1.0f + or_expf(-z));
  }
  float c[16];
  for (int r = 0; r < 4; r++) {
    float m = -INFINITY;
    for (int col = 0; col < 4; col++) {
      const float v = mix[8 + r * 4 + col] * scale[2] + base[8 + r * 4 + col];
      c[r * 4 + col] = v;
      if (v > m) m = v;
    }
    float s = 0.0f;
    for (int col = 0; col < 4; col++) {
      const float v = or_expf(c[r * 4 + col] - m);
      c[r * 4 + col] = v;
      s += v;
    }
    for (int col = 0; col < 4; col++) c[r * 4 + col] = c[r * 4 + col] / s + eps;
  }
  for (int col = 0; col < 4; col++) {
    float s = eps;
    for (int r = 0; r < 4; r++) s += c[r * 4 + col];
    for (int r = 0; r < 4; r++) c[r * 4 + col] /= s;
  }
  for (int it = 1; it < iters; it++) {
    for (int r = 0; r < 4; r++) {
      float s = eps;
      for (int col = 0; col < 4; col++) s += c[r * 4 + col];
      for (int col = 0; col < 4; col++) c[r * 4 + col] /= s;
    }
    for (int col = 0; col < 4; col++) {
      float s = eps;
      for (int r = 0; r < 4; r++) s += c[r * 4 + col];
      for (int r = 0; r < 4; r++) c[r * 4 + col] /= s;
    }
  }
  for (int i = 0; i < 16; i++) out[8 + i] = c[i];
}

/* hc_split_weighted_sum_norm_fused (engine/src/kernels/hc.rs:313-398), n_hc
 * = 4, a 256-thread row: the row's split (24 values, written to split),
 * out[i] = sum over h in order of residual[h][i] * pre[h], its sum of squares
 * over 256 lane-strided partials and the halving tree 128..1, then
 * norm_out[i] = out[i] * (1 / sqrt(sumsq / n + norm_eps)) * norm_w[i]. */
void or_hc_split_norm(const float* mix, const float* scale, const float* base, const float* residual_hc,
                      const float* norm_w, float* split, float* out, float* norm_out, int n_embd, int n_rows,
                      int iters, float eps, float norm_eps) {
  for (int t = 0; t < n_rows; t++) {
    float* sp = split + (size_t)t * 24;
    or_hc4_split(mix + (size_t)t * 24, scale, base, iters, eps, sp);
    const float* res = residual_hc + (size_t)t * 4 * n_embd;
    float* o = out + (size_t)t * n_embd;
    float part[256];
    for (int l = 0; l < 256; l++) {
      float s = 0.0f;
      for (int i = l; i < n_embd; i += 256) {
        float acc = 0.0f;
        for (int h = 0; h < 4; h++) acc += res[(size_t)h * n_embd + i] * sp[h];
        o[i] = acc;
        s += acc * acc;
      }
      part[l] = s;
    }
    for (int st = 128; st > 0; st >>= 1)
      for (int l = 0; l < st; l++) part[l] += part[l + st];
    const float ns = 1.0f / sqrtf(part[0] / (float)n_embd + norm_eps);
    for (int i = 0; i < n_embd; i++) norm_out[(size_t)t * n_embd + i] = o[i] * ns * norm_w[i];
  }
}

/* hc_expand (engine/src/kernels/hc.rs:212-259): the FFN residual merge
 * after the layer (session.rs:2157-2175).  out[t][dst][i] =
 * (block_out + block_add)[t][i] * post[dst] + sum over src in order of
 * comb[dst + src*n_hc] * residual[t][src][i], where post and comb are the
 * token's split row at offsets n_hc and 2*n_hc.  f32, no fused multiply-add. */
void or_hc_expand(const float* block_out, const float* block_add, const float* residual_hc, const float* split,
                  float* out_hc, int n_embd, int n_hc, int n_tokens, int mix_hc, int has_add) {
  for (int t = 0; t < n_tokens; t++)
    for (int dst = 0; dst < n_hc; dst++)
      for (int i = 0; i < n_embd; i++) {
        float v = block_out[(size_t)t * n_embd + i];
        if (has_add) v += block_add[(size_t)t * n_embd + i];
        const float* row = split + (size_t)t * mix_hc;
        float acc = v * row[n_hc + dst];
        for (int src = 0; src < n_hc; src++)
          acc += row[2 * n_hc + dst + src * n_hc] * residual_hc[((size_t)t * n_hc + src) * n_embd + i];
        out_hc[((size_t)t * n_hc + dst) * n_embd + i] = acc;
      }
}

/* ------------------------------------------------------------------ */
/* dispatch: moe.rs:299-362 count/prefix/scatter and :547-596 tiles.   */
/* The scatter is restated as a stable counting sort: within an expert  */
/* the pairs keep ascending pair order (the reference's atomic cursor   */
/* leaves that order unspecified).                                      */
/* ------------------------------------------------------------------ */
void or_dispatch(const int32_t* selected, int pairs, int E, int block_m,
                 uint32_t* counts, uint32_t* offsets, uint32_t* sorted_pairs,
                 uint32_t* tile_offsets, uint32_t* tile_experts, uint32_t* tile_starts) {
  for (int e = 0; e < E; e++) counts[e] = 0;
  for (int p = 0; p < pairs; p++) { int e = selected[p] < 0 ? 0 : selected[p]; counts[e]++; }
  uint32_t sum = 0;
  for (int e = 0; e < E; e++) { offsets[e] = sum; sum += counts[e]; }
  offsets[E] = sum;
  uint32_t* cur = (uint32_t*)malloc(sizeof(uint32_t) * (E > 0 ? E : 1));
  for (int e = 0; e < E; e++) cur[e] = offsets[e];
  for (int p = 0; p < pairs; p++) { int e = selected[p] < 0 ? 0 : selected[p]; sorted_pairs[cur[e]++] = (uint32_t)p; }
  free(cur);
  if (tile_offsets) {
    uint32_t ts = 0;
    for (int e = 0; e < E; e++) { tile_offsets[e] = ts; ts += (counts[e] + block_m - 1) / block_m; }
    tile_offsets[E] = ts;
    for (int e = 0; e < E; e++) {
      uint32_t n = (counts[e] + block_m - 1) / block_m;
      for (uint32_t t = 0; t < n; t++) {
        tile_experts[tile_offsets[e] + t] = (uint32_t)e;
        tile_starts[tile_offsets[e] + t] = t * (uint32_t)block_m;
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* whole layer: session.rs:1894-2155                                   */
/* ------------------------------------------------------------------ */
int or_moe_forward(const or_config* c,
                   const uint16_t* w_router, const float* bias,
                   const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                   const uint8_t* w_sh_gate, const uint8_t* w_sh_up, const uint8_t* w_sh_down,
                   const float* x, int T, float* shared_out, float* routed_out,
                   int32_t* selected_out, float* weights_out, int nthreads) {
  int d = c->d_model, I = c->d_ff, E = c->n_expert, K = c->top_k;
  if (d % 256 || I % 256 || K > E || K < 1 || T < 0) return 1;
  size_t P = (size_t)T * K;
  float* logits = (float*)malloc(sizeof(float) * (size_t)T * E + 4);
  int32_t* sel = (int32_t*)malloc(sizeof(int32_t) * P + 4);
  float* wts = (float*)malloc(sizeof(float) * P + 4);
  uint8_t* xq = (uint8_t*)malloc((size_t)T * (d / 256) * 292 + 4);
  float* mid = (float*)malloc(sizeof(float) * P * I + 4);
  uint8_t* midq = (uint8_t*)malloc(P * (I / 256) * 292 + 4);
  float* down = (float*)malloc(sizeof(float) * P * d + 4);

  /* (h) router + routed experts */
  or_router_logits(w_router, x, logits, d, E, T, nthreads);
  or_router_select(c, logits, bias, T, NULL, sel, wts);
  or_q8k_quantize(x, xq, d, T);
  or_gate_up_mid(w_gate, w_up, xq, sel, wts, NULL, NULL, mid, d, I, T, K, c->swiglu_clamp, nthreads);
  or_q8k_quantize(mid, midq, I, (int)P);
  or_down(w_down, midq, sel, down, d, I, T, K, nthreads);
  or_moe_sum(down, routed_out, d, K, T);
  if (selected_out) memcpy(selected_out, sel, sizeof(int32_t) * P);
  if (weights_out) memcpy(weights_out, wts, sizeof(float) * P);

  /* (g) shared expert */
  int Is = c->d_ff_shared;
  if (c->shared_fmt == 0) {
    int nb = (d + 31) / 32, nbm = (Is + 31) / 32;
    int8_t* q = (int8_t*)malloc((size_t)T * (nb > nbm ? nb : nbm) * 32 + 4);
    float* qs = (float*)malloc(sizeof(float) * (size_t)T * (nb > nbm ? nb : nbm) + 4);
    float* g = (float*)malloc(sizeof(float) * (size_t)T * Is + 4);
    float* u = (float*)malloc(sizeof(float) * (size_t)T * Is + 4);
    float* m = (float*)malloc(sizeof(float) * (size_t)T * Is + 4);
    or_q8_0_quantize(x, q, qs, d, T);
    or_q8_0_matvec(w_sh_gate, q, qs, g, d, Is, T, nthreads);
    or_q8_0_matvec(w_sh_up, q, qs, u, d, Is, T, nthreads);
    or_swiglu(g, u, m, T * Is, c->swiglu_clamp, 1.0f);
    or_q8_0_quantize(m, q, qs, Is, T);
    or_q8_0_matvec(w_sh_down, q, qs, shared_out, Is, d, T, nthreads);
    free(q); free(qs); free(g); free(u); free(m);
  } else if (c->shared_fmt == 1) {
    /* IQ2_XXS / Q2_K shared expert: one slot with weight 1 per token */
    int32_t* s0 = (int32_t*)calloc((size_t)T, sizeof(int32_t));
    float* w1 = (float*)malloc(sizeof(float) * (size_t)T + 4);
    for (int t = 0; t < T; t++) w1[t] = 1.0f;
    float* m = (float*)malloc(sizeof(float) * (size_t)T * Is + 4);
    uint8_t* mq = (uint8_t*)malloc((size_t)T * (Is / 256) * 292 + 4);
    or_gate_up_mid(w_sh_gate, w_sh_up, xq, s0, w1, NULL, NULL, m, d, Is, T, 1, c->swiglu_clamp, nthreads);
    or_q8k_quantize(m, mq, Is, T);
    or_down(w_sh_down, mq, s0, shared_out, d, Is, T, 1, nthreads);
    free(s0); free(w1); free(m); free(mq);
  } else {
    memset(shared_out, 0, sizeof(float) * (size_t)T * d);
  }
  free(logits); free(sel); free(wts); free(xq); free(mid); free(midq); free(down);
  return 0;
}
