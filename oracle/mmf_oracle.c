/* mmf_oracle.c -- CPU restatement of the reference HGRN-Bit engine (see mmf_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker; never part of the product path).
 * Compiled with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() standing for an FMA that g++ 11.4 emits for the reference source under its
 * GNU-mode default -ffp-contract=fast. Each function cites the reference lines it follows.
 */
#include "mmf_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------- */
/* primitives                                                                           */
/* ---------------------------------------------------------------------------------- */

/* hsum_ps (simd.hpp:48-57): lo+hi, then movehdup/movehl adds ->
 * ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)). */
float mo_hsum8(const float a[8]) {
  float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  return (s0 + s1) + (s2 + s3);
}

/* sumsq (simd.hpp:69-89): 8 lane accumulators over k = j (mod 8), _mm256_fmadd_ps, then
 * hsum; the scalar tail `s += x*x` is contracted to an FMA. */
float mo_sumsq(const float* x, size_t n) {
  float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t c = 0;
  for (; c + 8 <= n; c += 8)
    for (int j = 0; j < 8; ++j) a[j] = fmaf(x[c + j], x[c + j], a[j]);
  float s = mo_hsum8(a);
  for (; c < n; ++c) s = fmaf(x[c], x[c], s);
  return s;
}

/* ternary_dot_f32 (simd.hpp:92-122): 8 lanes acc = fma(y, (float)w, acc), hsum, then the
 * scalar tail as signed adds. The 8 lane chains are one 8-wide vector: each lane is the
 * same single-rounding fma as fmaf, the vector form only converts the weights 8 at a time. */
float mo_ternary_dot_f32(const float* y, const int8_t* w, size_t n) {
  float a[8];
  size_t k = 0;
  __m256 acc = _mm256_setzero_ps();
  for (; k + 8 <= n; k += 8) {
    const __m256 wv = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(w + k))));
    acc = _mm256_fmadd_ps(_mm256_loadu_ps(y + k), wv, acc);
  }
  _mm256_storeu_ps(a, acc);
  float s = mo_hsum8(a);
  for (; k < n; ++k) {
    if (w[k] > 0) s += y[k];
    else if (w[k] < 0) s -= y[k];
  }
  return s;
}

/* ternary_dot_i32 (simd.hpp:125-154): exact integer sum (32-bit wrap, as the SIMD adds). */
int32_t mo_ternary_dot_i32(const int32_t* q, const int8_t* w, size_t n) {
  uint32_t s = 0;
  for (size_t k = 0; k < n; ++k) s += (uint32_t)q[k] * (uint32_t)(int32_t)w[k];
  return (int32_t)s;
}

/* quant_q510 (simd.hpp:162-187). SIMD body: _mm256_cvtps_epi32 (round-half-even; any
 * value outside int32 or NaN -> INT32_MIN) then clamp to [-32768, 32767]. Scalar tail:
 * nearbyintf, clamp in float, then convert. */
void mo_quant_q510(int32_t* q, const float* y, float qs, size_t n) {
  size_t c = 0;
  for (; c + 8 <= n; c += 8)
    for (int j = 0; j < 8; ++j) {
      float v = y[c + j] * qs;
      int32_t r = (fabsf(v) < 2147483648.0f) ? (int32_t)nearbyintf(v) : INT32_MIN;
      q[c + j] = r < -32768 ? -32768 : (r > 32767 ? 32767 : r);
    }
  for (; c < n; ++c) {
    float v = nearbyintf(y[c] * qs);
    if (v > 32767.0f) v = 32767.0f;
    else if (v < -32768.0f) v = -32768.0f;
    q[c] = isnan(v) ? INT32_MIN : (int32_t)v;
  }
}

/* Cephes exp constants (simd.hpp:212-249). */
#define EXP_HI 88.3762626647949f
#define EXP_LO -88.3762626647949f
#define LOG2EF 1.44269504088896341f
#define C1 0.693359375f
#define C2 -2.12194440e-4f
#define P0 1.9875691500E-4f
#define P1 1.3981999507E-3f
#define P2 8.3334519073E-3f
#define P3 4.1665795894E-2f
#define P4 1.6666665459E-1f
#define P5 5.0000001201E-1f

static float pow2i(float fx) {
  int32_t e = (int32_t)(((uint32_t)((int32_t)fx + 127)) << 23);
  float r;
  memcpy(&r, &e, 4);
  return r;
}

/* exp8_ps lane (simd.hpp:232-249): clamp by max/min (NaN -> the low bound), then the
 * explicit FMAs of the AVX2 code. Returns the polynomial p and 2^n separately: the
 * callers' `1 + p*2^n` is fused by g++ into fma(p, 2^n, 1). */
static void exp_body_parts(float x, float* p_out, float* pow2n) {
  x = (x > EXP_LO) ? x : EXP_LO; /* _mm256_max_ps(x, lo) */
  x = (x < EXP_HI) ? x : EXP_HI; /* _mm256_min_ps(x, hi) */
  float fx = floorf(fmaf(x, LOG2EF, 0.5f));
  float r = fmaf(-fx, C1, x);
  r = fmaf(-fx, C2, r);
  float p = P0;
  p = fmaf(p, r, P1);
  p = fmaf(p, r, P2);
  p = fmaf(p, r, P3);
  p = fmaf(p, r, P4);
  p = fmaf(p, r, P5);
  p = fmaf(p, r * r, r + 1.0f);
  *p_out = p;
  *pow2n = pow2i(fx);
}

/* expf_poly (simd.hpp:212-229) as g++ contracts it in the scalar tails: the clamp keeps
 * NaN, `x*log2e + 0.5` and the range reduction fuse, and `p*(r*r) + r + 1` becomes
 * fma(p, r*r, r) + 1. */
static void exp_tail_parts(float x, float* p_out, float* pow2n) {
  if (x > EXP_HI) x = EXP_HI;
  else if (x < EXP_LO) x = EXP_LO;
  float fx = floorf(fmaf(x, LOG2EF, 0.5f));
  float r = fmaf(-fx, C1, x);
  r = fmaf(-fx, C2, r);
  float p = P0;
  p = fmaf(p, r, P1);
  p = fmaf(p, r, P2);
  p = fmaf(p, r, P3);
  p = fmaf(p, r, P4);
  p = fmaf(p, r, P5);
  p = fmaf(p, r * r, r) + 1.0f;
  *p_out = p;
  *pow2n = pow2i(fx);
}

float mo_exp_body(float x) {
  float p, e;
  exp_body_parts(x, &p, &e);
  return p * e;
}

float mo_exp_tail(float x) {
  float p, e;
  exp_tail_parts(x, &p, &e);
  return p * e;
}

/* 1 + exp(-a) as the callers compute it: fma(p, 2^n, 1). */
static float den_body(float a) {
  float p, e;
  exp_body_parts(-a, &p, &e);
  return fmaf(p, e, 1.0f);
}
static float den_tail(float a) {
  float p, e;
  exp_tail_parts(-a, &p, &e);
  return fmaf(p, e, 1.0f);
}

/* sigmoid / silu / swiglu (simd.hpp:270-330): 8-wide body, scalar tail. */
void mo_sigmoid(float* out, const float* x, size_t n) {
  size_t body = n & ~(size_t)7;
  for (size_t i = 0; i < body; ++i) out[i] = 1.0f / den_body(x[i]);
  for (size_t i = body; i < n; ++i) out[i] = 1.0f / den_tail(x[i]);
}

void mo_silu(float* out, const float* x, size_t n) {
  size_t body = n & ~(size_t)7;
  for (size_t i = 0; i < body; ++i) out[i] = x[i] / den_body(x[i]);
  for (size_t i = body; i < n; ++i) out[i] = x[i] / den_tail(x[i]);
}

void mo_swiglu(float* out, const float* a, const float* b, size_t n) {
  size_t body = n & ~(size_t)7;
  for (size_t i = 0; i < body; ++i) out[i] = (a[i] / den_body(a[i])) * b[i];
  for (size_t i = body; i < n; ++i) out[i] = (a[i] / den_tail(a[i])) * b[i];
}

/* parallel_chunks (parallel.hpp:30-37, chunk 8192): each chunk is one SIMD call, so the
 * body/tail split restarts at every chunk. */
static void chunked_swiglu(float* out, const float* a, const float* b, size_t n) {
  for (size_t off = 0; off < n; off += 8192) {
    size_t len = (n - off < 8192) ? n - off : 8192;
    mo_swiglu(out + off, a + off, b + off, len);
  }
}
static void chunked_sigmoid(float* f, size_t n) {
  for (size_t off = 0; off < n; off += 8192) {
    size_t len = (n - off < 8192) ? n - off : 8192;
    mo_sigmoid(f + off, f + off, len);
  }
}

/* ---------------------------------------------------------------------------------- */
/* kernels                                                                              */
/* ---------------------------------------------------------------------------------- */

/* rstd = 1 / sqrt(sumsq / n + eps), each step correctly rounded (bitlinear.cpp:69,
 * rmsnorm.cpp:19). */
float mo_rstd(float sumsq, size_t n, float eps) {
  return 1.0f / sqrtf(sumsq / (float)n + eps);
}

/* rmsnorm (rmsnorm.cpp:11-22): y = (x * rstd) * w. */
void mo_rmsnorm(float* y, const float* x, const float* w, size_t rows, size_t cols, float eps) {
#pragma omp parallel for schedule(static) if (rows > 1)
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    float rstd = mo_rstd(mo_sumsq(xr, cols), cols, eps);
    for (size_t c = 0; c < cols; ++c) yr[c] = (xr[c] * rstd) * w[c];
  }
}

/* rmsnorm_swishgate (rmsnorm_swishgate.cpp:13-30): out = ((g*rstd)*w) * silu(o). */
void mo_rmsnorm_swishgate(float* out, const float* g, const float* o, const float* w,
                          size_t rows, size_t cols, float eps) {
#pragma omp parallel for schedule(static) if (rows > 1)
  for (size_t r = 0; r < rows; ++r) {
    const float* gr = g + r * cols;
    float* so = (float*)malloc(cols * sizeof(float));
    float rstd = mo_rstd(mo_sumsq(gr, cols), cols, eps);
    mo_silu(so, o + r * cols, cols);
    for (size_t c = 0; c < cols; ++c) out[r * cols + c] = ((gr[c] * rstd) * w[c]) * so[c];
    free(so);
  }
}

/* hgrn_scan / hgrn_step (hgrn_scan.cpp:11-19, simd.hpp:335-357): state = fma(f, state, i)
 * (g++ fuses the mul+add), out_t = state. */
void mo_hgrn_scan(float* out, const float* i, const float* f, size_t T, size_t D,
                  float* state_io) {
  float* st = state_io ? state_io : (float*)calloc(D, sizeof(float));
  for (size_t t = 0; t < T; ++t)
    for (size_t d = 0; d < D; ++d) {
      st[d] = fmaf(f[t * D + d], st[d], i[t * D + d]);
      out[t * D + d] = st[d];
    }
  if (!state_io) free(st);
}

/* Fused BitLinear (bitlinear.cpp:21-117) plus the int8 absmax mode. */
void mo_bitlinear(float* out, const float* x, const float* normw, const int8_t* wq,
                  float scale_w, size_t rows, size_t K, size_t N, float eps, int mode,
                  int frac_bits, float* norm_out, int32_t* acc_out, int32_t* codes_out,
                  float* scale_a_out) {
  const float inv_scale_w = 1.0f / scale_w;
  const float qs = (float)(1u << frac_bits);
  const float inv_fixed = 1.0f / (qs * scale_w);
  float* y = (float*)malloc(K * sizeof(float));
  int32_t* q = (int32_t*)malloc(K * sizeof(int32_t));
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * K;
    float rstd = mo_rstd(mo_sumsq(xr, K), K, eps);
    for (size_t c = 0; c < K; ++c) y[c] = (xr[c] * rstd) * normw[c];
    if (norm_out) memcpy(norm_out + r * K, y, K * sizeof(float));
    float* outr = out + r * N;
    if (mode == MO_FLOAT) {
#pragma omp parallel for schedule(static)
      for (size_t o = 0; o < N; ++o) outr[o] = mo_ternary_dot_f32(y, wq + o * K, K) * inv_scale_w;
      continue;
    }
    float deq = inv_fixed;
    float sa = 0.0f;
    if (mode == MO_FIXED) {
      mo_quant_q510(q, y, qs, K);
    } else {
      /* reference.py:131-135: scale = 127 / max(max|y|, 1e-5); q = clamp(round(y*scale)) */
      float amax = 0.0f;
      for (size_t c = 0; c < K; ++c) amax = fmaxf(amax, fabsf(y[c]));
      sa = 127.0f / (amax > 1e-5f ? amax : 1e-5f);
      for (size_t c = 0; c < K; ++c) {
        float v = nearbyintf(y[c] * sa);
        v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
        q[c] = (int32_t)v;
      }
      if (scale_a_out) scale_a_out[r] = sa;
    }
    if (codes_out) memcpy(codes_out + r * K, q, K * sizeof(int32_t));
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < N; ++o) {
      int32_t acc = mo_ternary_dot_i32(q, wq + o * K, K);
      if (acc_out) acc_out[r * N + o] = acc;
      /* FixedQ510: dequant_scale (simd.hpp:191-206) = (float)acc * inv_fixed.
       * Int8: reference.py:184 out = acc / (scale_w * scale_a). */
      outr[o] = (mode == MO_FIXED) ? (float)acc * deq : (float)acc / (scale_w * sa);
    }
  }
  free(y);
  free(q);
}

void mo_ternary_matmul(const int32_t* x, int32_t* acc, const int8_t* wq, size_t N, size_t M,
                       size_t b) {
  for (size_t i = 0; i < b; ++i) {
#pragma omp parallel for schedule(static)
    for (size_t m = 0; m < M; ++m) acc[i * M + m] = mo_ternary_dot_i32(x + i * N, wq + m * N, N);
  }
}

size_t mo_argmax(const float* v, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (v[i] > v[best]) best = i;
  return best;
}

/* ---------------------------------------------------------------------------------- */
/* model                                                                                */
/* ---------------------------------------------------------------------------------- */

/* Model::block (hgrn_model.cpp:80-195). */
void mo_block(const mo_model* m, int mode, int frac, float* h, size_t T, size_t layer,
              float* state, int stream_state, float* trace) {
  const size_t H = m->H, I = m->I, TH = T * H;
  const mo_layer* Ly = &m->layers[layer];
  const float eps = m->eps;
  float* resid = (float*)malloc(TH * sizeof(float));
  float* hs = (float*)malloc(TH * sizeof(float));
  float* ib = (float*)malloc(TH * sizeof(float));
  float* fb = (float*)malloc(TH * sizeof(float));
  float* gb = (float*)malloc(TH * sizeof(float));
  float* scan = (float*)malloc(TH * sizeof(float));
  float* recur = (float*)malloc(TH * sizeof(float));
  float* onemf = (float*)malloc(T * (H > I ? H : I) * sizeof(float));
  float* oin = (float*)malloc(T * (H > I ? H : I) * sizeof(float));
  float* oout = (float*)malloc(TH * sizeof(float));
  float* y = (float*)malloc(T * 2 * I * sizeof(float));
  float* gate = (float*)malloc(T * I * sizeof(float));

  memcpy(resid, h, TH * sizeof(float));
  mo_rmsnorm(hs, h, Ly->attn_norm, T, H, eps);
  /* i/f/g share hs; the FixedQ510 cluster path is bit-identical to three bitlinear calls
   * (bitlinear.cpp:119-160, kernels.hpp:46-50). */
  mo_bitlinear(ib, hs, Ly->normw[0], Ly->wq[0], Ly->scale_w[0], T, H, H, eps, mode, frac, 0, 0, 0, 0);
  mo_bitlinear(fb, hs, Ly->normw[1], Ly->wq[1], Ly->scale_w[1], T, H, H, eps, mode, frac, 0, 0, 0, 0);
  mo_bitlinear(gb, hs, Ly->normw[2], Ly->wq[2], Ly->scale_w[2], T, H, H, eps, mode, frac, 0, 0, 0, 0);

  /* gate: f = sigmoid(f); f = fma(1 - lb, f, lb) for layer > 0 (hgrn_model.cpp:113-124) */
  chunked_sigmoid(fb, TH);
  if (m->use_lower_bound && layer > 0 && m->lower_bounds) {
    const float* lb = m->lower_bounds + layer * H;
    for (size_t t = 0; t < T; ++t)
      for (size_t c = 0; c < H; ++c) fb[t * H + c] = fmaf(1.0f - lb[c], fb[t * H + c], lb[c]);
  }
  /* scan input = silu(i) * (1 - f) (hgrn_model.cpp:128-134) */
  for (size_t n = 0; n < TH; ++n) onemf[n] = 1.0f - fb[n];
  chunked_swiglu(scan, ib, onemf, TH);
  /* recurrence (hgrn_model.cpp:138-150) */
  if (stream_state) {
    for (size_t b = 0; b < T; ++b)
      for (size_t d = 0; d < H; ++d) {
        float s = fmaf(fb[b * H + d], state[b * H + d], scan[b * H + d]);
        state[b * H + d] = s;
        recur[b * H + d] = s;
      }
  } else {
    mo_hgrn_scan(recur, scan, fb, T, H, state);
  }
  if (trace) {
    memcpy(trace + 0 * TH, ib, TH * sizeof(float));
    memcpy(trace + 1 * TH, fb, TH * sizeof(float));
    memcpy(trace + 2 * TH, gb, TH * sizeof(float));
    memcpy(trace + 3 * TH, scan, TH * sizeof(float));
    memcpy(trace + 4 * TH, recur, TH * sizeof(float));
  }
  /* g_norm, o_proj, residual (hgrn_model.cpp:153-166) */
  mo_rmsnorm_swishgate(oin, gb, recur, Ly->g_norm, T, H, eps);
  mo_bitlinear(oout, oin, Ly->normw[3], Ly->wq[3], Ly->scale_w[3], T, H, H, eps, mode, frac, 0, 0, 0, 0);
  for (size_t n = 0; n < TH; ++n) resid[n] += oout[n];
  /* MLP (hgrn_model.cpp:167-194) */
  mo_rmsnorm(hs, resid, Ly->mlp_norm, T, H, eps);
  mo_bitlinear(y, hs, Ly->normw[4], Ly->wq[4], Ly->scale_w[4], T, H, 2 * I, eps, mode, frac, 0, 0, 0, 0);
  for (size_t t = 0; t < T; ++t)
    for (size_t c = 0; c < I; ++c) {
      gate[t * I + c] = y[t * 2 * I + c];
      onemf[t * I + c] = y[t * 2 * I + I + c];
    }
  chunked_swiglu(oin, gate, onemf, T * I);
  mo_bitlinear(oout, oin, Ly->normw[5], Ly->wq[5], Ly->scale_w[5], T, I, H, eps, mode, frac, 0, 0, 0, 0);
  for (size_t n = 0; n < TH; ++n) h[n] = resid[n] + oout[n];

  free(resid); free(hs); free(ib); free(fb); free(gb); free(scan); free(recur);
  free(onemf); free(oin); free(oout); free(y); free(gate);
}

static void embed(const mo_model* m, const int64_t* ids, size_t T, float* h) {
  for (size_t t = 0; t < T; ++t) memcpy(h + t * m->H, m->emb + (size_t)ids[t] * m->H, m->H * sizeof(float));
}

/* head: final RMSNorm on `rows` rows then lm_head (hgrn_model.cpp:305-310, 440-441) */
static void head(const mo_model* m, int mode, int frac, const float* h, size_t rows, float* logits) {
  float* fn = (float*)malloc(rows * m->H * sizeof(float));
  mo_rmsnorm(fn, h, m->norm_w, rows, m->H, m->eps);
  mo_bitlinear(logits, fn, m->lm_normw, m->lm_wq, m->lm_scale_w, rows, m->H, m->V, m->eps, mode,
               frac, 0, 0, 0, 0);
  free(fn);
}

size_t mo_generate(const mo_model* m, int mode, int frac, const int64_t* ids, size_t n,
                   size_t new_tokens, int64_t eos_id, int64_t* out, float* state_out,
                   float* last_logits) {
  const size_t H = m->H, L = m->L, V = m->V;
  float* st = (float*)calloc(L * H, sizeof(float));
  float* h = (float*)malloc(n * H * sizeof(float));
  float* lg = (float*)malloc(V * sizeof(float));
  size_t len = n;
  memcpy(out, ids, n * sizeof(int64_t));
  embed(m, ids, n, h);
  for (size_t l = 0; l < L; ++l) mo_block(m, mode, frac, h, n, l, st + l * H, 0, NULL);
  if (new_tokens > 0) {
    head(m, mode, frac, h + (n - 1) * H, 1, lg);
    int64_t t = (int64_t)mo_argmax(lg, V);
    out[len++] = t;
    for (size_t step = 1; step < new_tokens && t != eos_id; ++step) {
      embed(m, &out[len - 1], 1, h);
      for (size_t l = 0; l < L; ++l) mo_block(m, mode, frac, h, 1, l, st + l * H, 0, NULL);
      head(m, mode, frac, h, 1, lg);
      t = (int64_t)mo_argmax(lg, V);
      out[len++] = t;
    }
    if (last_logits) memcpy(last_logits, lg, V * sizeof(float));
  }
  if (state_out) memcpy(state_out, st, L * H * sizeof(float));
  free(st); free(h); free(lg);
  return len;
}

void mo_forward(const mo_model* m, int mode, int frac, const int64_t* ids, size_t T,
                float* logits) {
  float* h = (float*)malloc(T * m->H * sizeof(float));
  embed(m, ids, T, h);
  for (size_t l = 0; l < m->L; ++l) mo_block(m, mode, frac, h, T, l, NULL, 0, NULL);
  head(m, mode, frac, h, T, logits);
  free(h);
}

void mo_generate_serve(const mo_model* m, int mode, int frac, const int64_t* flat,
                       const size_t* lens, size_t B, size_t new_tokens, int64_t eos_id,
                       int64_t* out, size_t cap_per, size_t* out_len, float* state_out) {
  const size_t H = m->H, L = m->L, V = m->V;
  float* st = (float*)calloc(L * B * H, sizeof(float));
  char* done = (char*)calloc(B, 1);
  float* lg = (float*)malloc(B * V * sizeof(float));
  size_t maxT = B, off = 0;
  for (size_t b = 0; b < B; ++b) maxT = lens[b] > maxT ? lens[b] : maxT;
  float* h = (float*)malloc(maxT * H * sizeof(float));
  for (size_t b = 0; b < B; ++b) {
    const size_t T = lens[b];
    memcpy(out + b * cap_per, flat + off, T * sizeof(int64_t));
    out_len[b] = T;
    embed(m, flat + off, T, h);
    off += T;
    for (size_t l = 0; l < L; ++l) mo_block(m, mode, frac, h, T, l, st + (l * B + b) * H, 0, NULL);
    head(m, mode, frac, h + (T - 1) * H, 1, lg);
    int64_t t0 = (int64_t)mo_argmax(lg, V);
    out[b * cap_per + out_len[b]++] = t0;
    if (t0 == eos_id) done[b] = 1;
  }
  for (size_t step = 1; step < new_tokens; ++step) {
    for (size_t b = 0; b < B; ++b) embed(m, &out[b * cap_per + out_len[b] - 1], 1, h + b * H);
    for (size_t l = 0; l < L; ++l) mo_block(m, mode, frac, h, B, l, st + l * B * H, 1, NULL);
    head(m, mode, frac, h, B, lg);
    int all_done = 1;
    for (size_t b = 0; b < B; ++b) {
      if (done[b]) continue;
      int64_t t = (int64_t)mo_argmax(lg + b * V, V);
      out[b * cap_per + out_len[b]++] = t;
      if (t == eos_id) done[b] = 1;
      else all_done = 0;
    }
    if (all_done) break;
  }
  if (state_out) memcpy(state_out, st, L * B * H * sizeof(float));
  free(st); free(done); free(lg); free(h);
}
