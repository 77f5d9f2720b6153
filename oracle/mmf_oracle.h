/* mmf_oracle.h -- CPU restatement of the reference HGRN-Bit engine's numerics.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker for the parity tests: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and never as the
 * thing measured or shipped. The product (libmmfree_hip.so) does not link it.
 *
 * Every function restates the arithmetic of the reference as compiled by g++ 11.4 with
 * its own flags (-O2 -std=gnu++17 -mavx2 -mfma, i.e. -ffp-contract=fast): each place
 * where that build fuses a multiply and an add is written here as an explicit fmaf(),
 * and this file is compiled with -ffp-contract=off so nothing else fuses. Citations are
 * to the reference sources (cpp/...). Pinning: see tests/test_oracle.py -- every function
 * is checked against the compiled reference (oracle/_ref) and against committed golden
 * vectors; closed forms pin the integer paths.
 */
#ifndef MMF_ORACLE_H
#define MMF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation modes: 0 Float, 1 FixedQ510 (kernels.hpp:21-26), 2 Int8Absmax (the
 * per-row int8 "bitnet" mode of tools/reference.py:131-135,180-184, added as a third
 * mode of the C++ engine). */
enum { MO_FLOAT = 0, MO_FIXED = 1, MO_INT8 = 2 };

/* ---- primitives (simd.hpp) ---- */
float mo_hsum8(const float a[8]);                            /* simd.hpp:48-57 */
float mo_sumsq(const float* x, size_t n);                    /* simd.hpp:69-89 */
float mo_ternary_dot_f32(const float* y, const int8_t* w, size_t n); /* simd.hpp:92-122 */
int32_t mo_ternary_dot_i32(const int32_t* q, const int8_t* w, size_t n); /* simd.hpp:125-154 */
void mo_quant_q510(int32_t* q, const float* y, float qs, size_t n);    /* simd.hpp:162-187 */
float mo_exp_body(float x);      /* exp8_ps lane (simd.hpp:232-249), product p*2^n rounded */
float mo_exp_tail(float x);      /* expf_poly (simd.hpp:212-229) as contracted by g++ */
void mo_sigmoid(float* out, const float* x, size_t n);       /* simd.hpp:270-287 */
void mo_silu(float* out, const float* x, size_t n);          /* simd.hpp:289-308 */
void mo_swiglu(float* out, const float* a, const float* b, size_t n); /* simd.hpp:310-330 */

/* ---- kernels (kernels.hpp) ---- */
float mo_rstd(float sumsq, size_t n, float eps);             /* bitlinear.cpp:69 */
void mo_rmsnorm(float* y, const float* x, const float* w, size_t rows, size_t cols, float eps);
void mo_rmsnorm_swishgate(float* out, const float* g, const float* o, const float* w,
                          size_t rows, size_t cols, float eps);
void mo_hgrn_scan(float* out, const float* i, const float* f, size_t T, size_t D,
                  float* state_io);
/* Fused BitLinear (bitlinear.cpp:21-117; Int8Absmax per reference.py:131-135,180-184).
 * Optional debug outputs (NULL to skip): norm_out [rows,K] the RMSNorm y; acc_out
 * [rows,N] the int32 accumulators (modes 1, 2); codes_out [rows,K] the integer
 * activation codes (modes 1, 2); scale_a_out [rows] the int8 activation scale (mode 2). */
void mo_bitlinear(float* out, const float* x, const float* normw, const int8_t* wq,
                  float scale_w, size_t rows, size_t K, size_t N, float eps, int mode,
                  int frac_bits, float* norm_out, int32_t* acc_out, int32_t* codes_out,
                  float* scale_a_out);
/* CpuBackend::matmul_batch (ternary_backend.hpp:43-48,96-103): acc[i*M+m] = sum_n x[i*N+n]*wq[m*N+n] */
void mo_ternary_matmul(const int32_t* x, int32_t* acc, const int8_t* wq, size_t N, size_t M,
                       size_t b);

/* ---- model (hgrn_model.cpp) ---- */
typedef struct {
  const float *attn_norm, *mlp_norm, *g_norm;
  const int8_t* wq[6];      /* i, f, g, o, gate, down */
  float scale_w[6];
  const float* normw[6];
} mo_layer;

typedef struct {
  size_t V, H, L, I;
  float eps;
  int use_lower_bound;
  const float* emb;          /* [V, H] */
  const float* norm_w;       /* [H] */
  const int8_t* lm_wq;       /* [V, H] */
  float lm_scale_w;
  const float* lm_normw;     /* [H] */
  const float* lower_bounds; /* [L, H] or NULL */
  const mo_layer* layers;    /* [L] */
} mo_model;

/* One layer over T rows (Model::block, hgrn_model.cpp:80-195). state: [H] carried across
 * time (stream_state = 0) or [T, H], one per row (stream_state = 1). If trace is not
 * NULL it receives the block's internals, each [T, H]: i, f (gated), g, scan input,
 * recurrence output (5 * T * H floats). */
void mo_block(const mo_model* m, int mode, int frac_bits, float* h, size_t T, size_t layer,
              float* state, int stream_state, float* trace);

/* Greedy Model::generate (hgrn_model.cpp:249-347): writes the id stream (prompt + up to
 * new_tokens) to out (capacity n + new_tokens) and returns its length. state_out
 * ([L, H], may be NULL) receives the final recurrent state; last_logits ([V], may be
 * NULL) the logits of the last emitted token. */
size_t mo_generate(const mo_model* m, int mode, int frac_bits, const int64_t* ids, size_t n,
                   size_t new_tokens, int64_t eos_id, int64_t* out, float* state_out,
                   float* last_logits);

/* Model::forward (hgrn_model.cpp:239-247): stateless, logits [T, V]. */
void mo_forward(const mo_model* m, int mode, int frac_bits, const int64_t* ids, size_t T,
                float* logits);

/* Greedy Model::generate_serve (hgrn_model.cpp:349-454). prompts flattened with lens[B];
 * out[b * cap_per + j]; out_len[b]. */
void mo_generate_serve(const mo_model* m, int mode, int frac_bits, const int64_t* flat,
                       const size_t* lens, size_t B, size_t new_tokens, int64_t eos_id,
                       int64_t* out, size_t cap_per, size_t* out_len, float* state_out);

/* Greedy argmax, first index wins ties (hgrn_model.cpp:270-273). */
size_t mo_argmax(const float* v, size_t n);

#ifdef __cplusplus
}
#endif
#endif
