/* mmfree_hip.h -- C ABI of the MI355X (gfx950) HGRN-Bit engine, libmmfree_hip.so.
 *
 * The drop-in boundary between the host engine (the mmfree C++17 API: Model, Weights,
 * TernaryBackend, the kernels.hpp free functions) and the HIP kernels. Plain C types only:
 * no HIP or torch types cross it. Each entry point names the reference interface it
 * replaces (files of aebarthyi/matmulfreellmCPU, cpp/...).
 *
 * Conventions
 *   - Every function returns MMF_OK (0) or an MMF_ERR_* code; mmf_last_error(ctx) then
 *     holds a message. The C++ layer turns a non-zero status into std::runtime_error,
 *     which is the reference's error channel (weights.cpp:193-209, weights.hpp:49).
 *   - "dev" pointers are device memory (from mmf_malloc or any HIP allocation on the
 *     context's device); work on them is enqueued on the context's stream and is complete
 *     after mmf_sync. "host" pointers are read or written before the call returns.
 *   - A context is single-threaded, like the reference Model (bitlinear.cpp:47-53 shares
 *     static staging buffers): calls on one context must not overlap.
 *   - Activation modes (kernels.hpp:21-26): MMF_FLOAT (fp32 activations), MMF_FIXED_Q510
 *     (static Q(15-f).f codes, int32 accumulation), and MMF_INT8_ABSMAX, a third mode with
 *     per-row int8 absmax codes (tools/reference.py:131-135,180-184).
 */
#ifndef MMFREE_HIP_H
#define MMFREE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mmf_ctx mmf_ctx;

enum {
  MMF_OK = 0,
  MMF_ERR_ARG = 1,      /* invalid argument (shape, id, pointer, mode) */
  MMF_ERR_HIP = 2,      /* HIP runtime error */
  MMF_ERR_STATE = 3,    /* call out of order (e.g. no model loaded) */
  MMF_ERR_NODEV = 4,    /* no usable gfx950 device */
  MMF_ERR_MISSING = 5   /* a required tensor is missing (weights.hpp:47-50) */
};

enum { MMF_FLOAT = 0, MMF_FIXED_Q510 = 1, MMF_INT8_ABSMAX = 2 };

/* ---- context ------------------------------------------------------------------------ */
/* Open device `device` (must be gfx950); creates the context's stream. */
int mmf_create(mmf_ctx** out, int device);
void mmf_destroy(mmf_ctx* ctx);
/* Message of the last failed call on ctx (or of the last failed mmf_create if ctx is NULL). */
const char* mmf_last_error(const mmf_ctx* ctx);
/* Wait for all work enqueued on the context's stream. */
int mmf_sync(mmf_ctx* ctx);
/* The context's hipStream_t, as an opaque pointer (for timing with events). */
void* mmf_stream(mmf_ctx* ctx);
/* Device name and compute-unit count, for reports. */
int mmf_device_info(mmf_ctx* ctx, char* name, size_t name_cap, int* cus);

/* ---- device memory (so callers need no HIP headers) ----------------------------------- */
int mmf_malloc(mmf_ctx* ctx, void** dev, size_t bytes);
int mmf_free(mmf_ctx* ctx, void* dev);
int mmf_upload(mmf_ctx* ctx, void* dev, const void* host, size_t bytes);
int mmf_download(mmf_ctx* ctx, void* host, const void* dev, size_t bytes);

/* ---- resident projections: the TernaryBackend seam ------------------------------------ */
/* Register a ternary projection wq [N, K] (int8 in {-1, 0, +1}, nn.Linear layout, host
 * memory, as the blob stores it: tools/provision.py:98-99,122) with its per-tensor
 * scale_w and BitLinear norm weight normw [K] (may be NULL if only the integer matmul is
 * used). The weights are repacked on the device to 2 bits per weight. Returns the
 * proj_id that the calls below and TernaryBackend::matmul take
 * (ternary_backend.hpp:26-31: proj_id addresses resident weights). */
int mmf_proj_register(mmf_ctx* ctx, const int8_t* wq, size_t N, size_t K, float scale_w,
                      const float* normw, int* proj_id);
/* Replace the weights of a registered projection with wq [N, K] of its registered shape
 * (host memory, ternary int8): the seam's "the weights at wq now" contract of proj_id -1
 * (ternary_backend.hpp:26-31) for a caller whose buffer now holds other weights. Scale and
 * norm weight are kept. On MMF_ERR_ARG (a weight outside {-1, 0, +1}) the projection's
 * weights are undefined until the next successful update. */
int mmf_proj_update(mmf_ctx* ctx, int proj_id, const int8_t* wq);
/* Shape of a registered projection. */
int mmf_proj_shape(mmf_ctx* ctx, int proj_id, size_t* N, size_t* K);
/* Free a registered projection's device memory; proj_id is invalid afterwards (calls that
 * pass it fail with MMF_ERR_ARG). For callers that re-register a buffer whose weights, scale
 * or norm weight changed (the host operator functions of kernels.hpp:29-68, which cache
 * projections by host pointer), so that replaced projections do not accumulate. */
int mmf_proj_release(mmf_ctx* ctx, int proj_id);

/* TernaryBackend::matmul_batch (ternary_backend.hpp:43-48, 96-103):
 * acc[i*N + o] = sum_k x[i*K + k] * wq[o, k] for b rows; x holds int16-range Q5.10 codes
 * stored as int32 (ternary_backend.hpp:8-13). dev pointers. */
int mmf_ternary_matmul(mmf_ctx* ctx, int proj_id, const int32_t* x, int32_t* acc, size_t b);
/* The same for k projections on host buffers in one round trip: x[z] holds b rows of K_z
 * codes and acc[z] receives b rows of N_z accumulators for proj_ids[z] (host memory). All
 * codes go to the device in one copy through pinned staging the context keeps, the k matmuls
 * run back to back, and all accumulators return in one copy before the call returns (one
 * synchronisation). TernaryBackend::matmul_batch and matmul_seq (ternary_backend.hpp:43-90)
 * on host buffers, as HipTernaryBackend calls it. */
int mmf_ternary_matmul_host(mmf_ctx* ctx, int k, const int* proj_ids, const int32_t* const* x,
                            int32_t* const* acc, size_t b);

/* ---- operators (kernels.hpp:29-68), dev pointers ----------------------------------------- */
/* bitlinear (kernels.hpp:41-44, bitlinear.cpp:21-117) with the projection's registered
 * weights, scale and norm: x [rows, K] -> out [rows, N]. acc (may be NULL) receives the
 * int32 accumulators in the integer modes. */
int mmf_bitlinear(mmf_ctx* ctx, int proj_id, int mode, int frac_bits, float eps, const float* x,
                  float* out, size_t rows, int32_t* acc);
/* bitlinear_cluster (kernels.hpp:46-50, bitlinear.cpp:119-160): k (<= 3) projections with
 * equal shapes sharing the input x; bit-identical to k mmf_bitlinear calls. */
int mmf_bitlinear_cluster(mmf_ctx* ctx, const int* proj_ids, int k, int mode, int frac_bits,
                          float eps, const float* x, float* const* outs, size_t rows);
/* mmf_bitlinear without any device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Same arguments, results and errors as mmf_bitlinear; its
 * scratch (the activation codes and split-K partials of the call) lives in a static device
 * array of MMF_NOALLOC_SCRATCH_BYTES bytes, one per GPU, held until the process ends. A call
 * whose scratch would exceed it fails with MMF_ERR_ARG before launching anything (split the
 * rows over several calls). Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (from contexts with different streams, or other threads) race. */
#define MMF_NOALLOC_SCRATCH_BYTES (64u << 20)
int mmf_bitlinear_noalloc(mmf_ctx* ctx, int proj_id, int mode, int frac_bits, float eps, const float* x,
                          float* out, size_t rows, int32_t* acc);
/* Device bytes of the grow-only workspace this context holds for the operator entry points
 * (activation codes and split-K partials of mmf_bitlinear and its kin). It grows with the
 * largest call and is freed by mmf_destroy; mmf_bitlinear_noalloc adds nothing to it. No
 * counterpart in the reference: for callers that budget device memory. */
int mmf_workspace_bytes(mmf_ctx* ctx, size_t* bytes);
/* The integer input of a FixedQ510 BitLinear, for an external TernaryBackend: the RMSNorm
 * y = (x * rstd) * normw (bitlinear.cpp:62-70) and its Q5.10 codes (simd.hpp:162-187) as int32
 * codes [rows, K] (frac_bits fractional bits). dev pointers. */
int mmf_bitlinear_codes(mmf_ctx* ctx, const float* x, const float* normw, int32_t* codes, size_t rows,
                        size_t K, float eps, int frac_bits);
/* rmsnorm (kernels.hpp:29-31, rmsnorm.cpp:11-22) */
int mmf_rmsnorm(mmf_ctx* ctx, float* y, const float* x, const float* w, size_t rows, size_t cols,
                float eps);
/* swiglu: out = silu(a) * b (kernels.hpp:52-53, activations.cpp:9-15) */
int mmf_swiglu(mmf_ctx* ctx, float* out, const float* a, const float* b, size_t n);
/* hgrn_scan (kernels.hpp:55-59, hgrn_scan.cpp:11-19): state may be NULL (zeros) */
int mmf_hgrn_scan(mmf_ctx* ctx, float* out, const float* i, const float* f, size_t T, size_t D,
                  float* state);
/* rmsnorm_swishgate (kernels.hpp:61-63, rmsnorm_swishgate.cpp:13-30) */
int mmf_rmsnorm_swishgate(mmf_ctx* ctx, float* out, const float* g, const float* o,
                          const float* w, size_t rows, size_t cols, float eps);

/* ---- model (model.hpp:33-120) ----------------------------------------------------------- */
typedef struct {
  size_t vocab_size, hidden_size, num_hidden_layers, intermediate_size; /* config.hpp:8-21 */
  int use_lower_bound;
  float rms_norm_eps;
} mmf_config;

/* Begin a model (replaces Model::Model + the Weights tensor table, model.hpp:37,
 * weights.cpp:191-254): the tensors of the MMFREE1 blob are then handed over one by one
 * with mmf_model_tensor (names and shapes of tools/provision.py:101-124), and
 * mmf_model_finalize checks that every tensor is present, repacks the projections and
 * prepares the decode plan for (mode, frac_bits). */
int mmf_model_begin(mmf_ctx* ctx, const mmf_config* cfg);
/* dtype: 0 = f32, 1 = i8. host data, numel = product of shape. */
int mmf_model_tensor(mmf_ctx* ctx, const char* name, int dtype, const size_t* shape, int ndim,
                     const void* data);
int mmf_model_finalize(mmf_ctx* ctx, int mode, int frac_bits);
int mmf_model_config(mmf_ctx* ctx, mmf_config* cfg);

/* External integer matmul of the model's FixedQ510 projections: Model::set_backend with a
 * TernaryBackend that is not this engine's (model.hpp:74-79, hgrn_model.cpp:40-78; the split
 * of bitlinear.cpp:39-94 and bitlinear_cluster, :119-160). While fn is set (NULL clears it),
 * every FixedQ510 projection of the model -- prefill, serving steps, generate, forward, trace
 * -- computes its RMSNorm and Q5.10 codes on the device and calls
 *     fn(user, layer, proj, k, codes, acc, K, N, rows)
 * on the calling thread with host arrays: codes [k][rows][K] (int16-range codes as int32, in
 * element order), to be answered with acc [k][rows][N], acc[j][r][o] = sum_n
 * codes[j][r][n] * wq_j[o][n] (wrapping int32). proj is 0..5 for i, f, g, o, gate (N = 2I,
 * the gate and up halves), down of `layer`, or 6 with layer -1 for the lm_head; k is 3 for
 * the i/f/g cluster (proj 0, 1, 2), else 1. A non-zero return fails the model call with
 * MMF_ERR_ARG. The accumulators are dequantised and consumed on the device as the built-in
 * matmul's would be, so the results equal the built-in path's for a correct fn. Float and
 * Int8Absmax projections ignore fn (the reference's float path has no backend, kernels.hpp
 * :37-40). The timing entry points refuse to run while fn is set. */
typedef int (*mmf_matmul_fn)(void* user, int layer, int proj, int k, const int32_t* codes, int32_t* acc,
                             size_t K, size_t N, size_t rows);
int mmf_model_set_matmul(mmf_ctx* ctx, mmf_matmul_fn fn, void* user);

/* The prefill recurrence of float mode. chunked = 0 (the default): the time-ordered scan,
 * state = fma(f, state, in) step by step as the reference runs it (hgrn_scan.cpp:11-19,
 * simd.hpp:335-357), bit-exact. chunked = 1: a chunked parallel scan (chunks of 16 steps
 * scanned from zero with the product of their gates, the chunks' starting states combined
 * in time order, then each chunk re-run from its starting state), which rounds differently:
 * logits agree within fp32 rounding, not bit for bit. It has no counterpart in the reference;
 * it applies to float-mode prefills of one sequence with hidden % 64 == 0 (everything else
 * keeps the time-ordered scan). */
int mmf_model_set_scan(mmf_ctx* ctx, int chunked);

/* Device-time op profile of the model's kernels, for the Profiler / --profile breakdown
 * (the reference times each op on the host: hgrn_model.cpp:88-189, bench.cpp:16-40).
 * While on, every model launch is bracketed by events on the context's stream, the decode
 * steps run launch by launch instead of from their captured graphs, and the timing entry
 * points refuse to run. _read adds up the device time (microseconds) and launch count per
 * op since the last read: MMF_PROF_NORM the row prologues (the model's RMSNorms and g_norm
 * with each BitLinear's own norm and activation codes), MMF_PROF_MATMUL the BitLinear GEMMs
 * and the fused single-row BitLinear kernels (norms, GEMV and epilogue), MMF_PROF_MIXER the
 * gate math and recurrence of the row path, MMF_PROF_LM_HEAD the final norm and lm_head,
 * MMF_PROF_EMBED the embedding gather. Measurement only. */
enum { MMF_PROF_NORM = 0, MMF_PROF_MATMUL = 1, MMF_PROF_MIXER = 2, MMF_PROF_LM_HEAD = 3, MMF_PROF_EMBED = 4,
       MMF_PROF_KINDS = 5 };
int mmf_model_profile(mmf_ctx* ctx, int on);
int mmf_model_profile_read(mmf_ctx* ctx, double* us, uint64_t* launches);

/* Greedy Model::generate (model.hpp:44-50, hgrn_model.cpp:249-347), decode loop on the
 * device. Writes the id stream (prompt + generated) to out (capacity cap) and its length to
 * out_len. on_token (may be NULL) is called with each generated id, in order; eos_id < 0
 * disables the stop. The recurrent state is reset at entry. */
typedef void (*mmf_token_cb)(void* user, int64_t id);
int mmf_model_generate(mmf_ctx* ctx, const int64_t* ids, size_t n, size_t new_tokens,
                       int64_t eos_id, int64_t* out, size_t cap, size_t* out_len,
                       mmf_token_cb on_token, void* user);

/* Step-wise interface for sampling and serving (Model::generate with temperature > 0,
 * Model::generate_serve, hgrn_model.cpp:263-303,349-454):
 *   mmf_model_reset(B)      zero the recurrent state of B streams ([L][B][H])
 *   mmf_model_prefill(b)    run the prompt of stream b through all layers (time scan)
 *   mmf_model_step(tokens)  one batched decode step of all B streams
 * logits (host [rows, V], may be NULL) and argmax (host [rows], may be NULL) receive the
 * result for the last prompt position / each stream. */
int mmf_model_reset(mmf_ctx* ctx, size_t streams);
int mmf_model_prefill(mmf_ctx* ctx, size_t stream, const int64_t* ids, size_t n, float* logits,
                      int64_t* argmax);
int mmf_model_step(mmf_ctx* ctx, const int64_t* tokens, float* logits, int64_t* argmax);
/* The prompts of streams 0..n-1 (n <= the mmf_model_reset count), concatenated in ids with
 * lens[b] ids each, prefilled together: the same states, logits [n, V] and argmax [n] as n
 * mmf_model_prefill calls in stream order (the reference prefills stream by stream in
 * generate_serve, hgrn_model.cpp:412-428). The prompts run as one stack of rows through
 * every BitLinear, the recurrence scans each stream's rows from its own state. */
int mmf_model_prefill_streams(mmf_ctx* ctx, size_t n, const int64_t* ids, const size_t* lens,
                              float* logits, int64_t* argmax);
/* Recurrent state [L][B][H] after the last generate / prefill / step (host out). */
int mmf_model_state(mmf_ctx* ctx, float* out);

/* Model::forward (model.hpp:40-41, hgrn_model.cpp:239-247): stateless, logits [T, V] host. */
int mmf_model_forward(mmf_ctx* ctx, const int64_t* ids, size_t T, float* logits);

/* Layer-by-layer prefill trace for parity checks: after each layer l, h [L][T][H], the
 * state [L][H] and the block internals [L][5][T][H] (i, gated f, g, scan input,
 * recurrence output). host outputs; internals may be NULL. */
int mmf_model_trace(mmf_ctx* ctx, const int64_t* ids, size_t T, float* h, float* state,
                    float* internals);

/* Timing of the single-row decode kernels on the context's stream (HIP events around
 * `reps` decode steps, after `warmup` untimed ones): average microseconds per step and
 * per launch of the kernel kinds {IFG, O, GATE, DOWN, LM} (kind_us[5], may be NULL; each
 * kind's launches for all layers are replayed back to back from a captured HIP graph, so
 * the figure is the kernels' execution time). No counterpart in the reference engine:
 * measurement only. */
int mmf_model_time_decode(mmf_ctx* ctx, int warmup, int reps, double* step_us, double* kind_us);

/* Timing of the prefill (prompt of T ids through all layers, then the final norm, lm_head
 * and argmax of the last position -- the reference bench's time to the first token,
 * bench.cpp:47-63) on the context's stream: average microseconds per prefill over `reps`
 * runs after `warmup` (one HIP event pair around the runs), and, if kind_us (8 doubles) is
 * not NULL, the microseconds per prefill spent in each launch kind {BitLinear prologues,
 * i/f/g GEMM, mixer/recurrence, o GEMM, gate GEMM (+swiglu), down GEMM, final norm +
 * lm_head, embedding} from an event pair around every launch (a second set of runs).
 * No counterpart in the reference engine: measurement only. */
int mmf_model_time_prefill(mmf_ctx* ctx, const int64_t* ids, size_t T, int warmup, int reps,
                           double* total_us, double* kind_us);

/* Timing of one lockstep serving step of the context's streams (mmf_model_reset(ctx, B)),
 * launched kernel by kernel with an HIP event pair around every launch: after `warmup`
 * steps, kind_us (8 doubles, the kinds of mmf_model_time_prefill; the embedding is counted
 * under "embedding", the argmax with the lm_head) receives the microseconds per step spent
 * in each kind over `reps` steps. The steps advance the streams' states like mmf_model_step.
 * No counterpart in the reference engine: measurement only. */
int mmf_model_time_step(mmf_ctx* ctx, const int64_t* tokens, int warmup, int reps, double* kind_us);

/* Timing of mmf_bitlinear on device buffers (same arguments): average microseconds per call
 * with `reps` calls back to back in one HIP graph (device time; launched one by one when
 * MMF_GRAPH=0), and of its two launches (prologue: RMSNorm + activation codes; GEMM) from an
 * event pair around each launch. Measurement only. */
int mmf_time_bitlinear(mmf_ctx* ctx, int proj_id, int mode, int frac_bits, float eps, const float* x,
                       float* out, size_t rows, int warmup, int reps, double* total_us,
                       double* prologue_us, double* gemm_us);

/* Device calibration for the rooflines: sustained HBM read bandwidth (GB/s, a 2 GiB buffer),
 * Infinity Cache read bandwidth (GB/s, a 128 MiB buffer read 8 times), int8 matrix-core rate
 * (TOP/s, independent v_mfma_i32_32x32x32_i8) and non-packed fp32 FMA rate (TFLOP/s), into
 * out[0..3]. Each comes from a kernel that does only that work; the context's stream is
 * synchronized. No counterpart in the reference engine: measurement only. */
int mmf_measure_peaks(mmf_ctx* ctx, double* out4);

#ifdef __cplusplus
}
#endif
#endif
