// mmf_internal.hpp -- layouts and kernel launchers shared by the HIP sources.
//
// Device layout of a ternary projection wq [N, K] (int8 in the blob, nn.Linear layout):
//   K8 = K & ~7 elements are split into 8 "chains" j = 0..7, chain j holding k = j + 8t
//   for t < nb = K8/8 -- exactly the 8 AVX2 lanes of the reference dot products
//   (simd.hpp:92-154), so a chain summed in t order is one reference lane. Chains are
//   padded to Lc = roundup(nb, 16) codes (Wc = Lc/16 words, zero codes in the padding).
//   Outputs are grouped by 16; group og's slab is contiguous:
//       pk[((og * Wc + m) * 16 + ol) * 8 + j]   (word m of chain j of output og*16+ol)
//   so a 128-thread block (16 outputs x 8 chains) streams one contiguous slab, 512 bytes
//   per step. The K - K8 < 8 tail codes are kept as int8 tail[o * 8 + t]; rowsum[o] is the
//   sum of the chain part of row o (for the split Q5.10 product).
// Activations for one row use the same chain-transposed order: element k < K8 sits at
// j * Lc + t (k = j + 8t), the tail after 8 * Lc.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mmf {

constexpr int kGroup = 16;  // outputs per slab
constexpr int kBlock = 128; // threads of a GEMV block: 16 outputs x 8 chains

enum Mode : int { kFloat = 0, kFixed = 1, kInt8 = 2 };

struct Geom {
  int N, K, K8, nb, ntail, Lc, Wc, ngroups;
};

__host__ __device__ inline Geom make_geom(int N, int K) {
  Geom g;
  g.N = N;
  g.K = K;
  g.K8 = K & ~7;
  g.nb = g.K8 / 8;
  g.ntail = K - g.K8;
  g.Lc = (g.nb + 15) / 16 * 16;
  if (g.Lc == 0) g.Lc = 16;
  g.Wc = g.Lc / 16;
  g.ngroups = (N + kGroup - 1) / kGroup;
  return g;
}

// Device view of one resident projection.
struct ProjDev {
  const uint32_t* pk = nullptr;
  const uint32_t* pkm = nullptr;  // the same words in the matrix-core tile order (mmf_mfma.hip)
  const uint32_t* pk4 = nullptr;  // float-mode decode: the slab with fp4 codes (launch_pack4), or null
  int pair = 0;                   // pkm interleaves the two halves (MLP gate/up) by 32-column group
  const int8_t* tail = nullptr;
  const int32_t* rowsum = nullptr;
  const float* normw = nullptr;   // BitLinear norm weight [K]
  const float* normwT = nullptr;  // the same, chain-transposed [8*Lc + 8] (decode kernels)
  Geom g{};
  float scale_w = 1.0f;
  float inv_scale_w = 1.0f;  // 1.0f / scale_w (bitlinear.cpp:28)
  float inv_fixed = 1.0f;    // 1.0f / (2^frac * scale_w) (bitlinear.cpp:30), for the model frac
};

// ---- fused single-row decode kernels (mmf_decode.hip) -------------------------------
// kOp: one BitLinear of the operator API on one natural-layout row (no stage-1 norm, the
// outputs stored in natural order, optional int32 accumulators)
enum DecKind : int { kIFG = 0, kO = 1, kGate = 2, kDown = 3, kLM = 4, kOp = 5 };

struct DecArgs {
  ProjDev p[3];
  int H, I, vocab, layer, use_lb;
  float eps, qs, inv_fixed[3];
  // Vectors below are chain-transposed ([8*Lc + 8], zero padding) unless noted.
  const float* x;         // input vector; nullptr for layer 0 (embedding row of *key,
                          // a cleared key or one outside [0, vocab) reads row 0)
  const float* embT;      // chain-transposed embedding rows [V][8*Lc_H + 8]
  const float* x2;        // kO: silu of the recurrence output (written by kIFG)
  const float* pre_w;     // stage-1 norm weight (attn / g / mlp / final norm), or nullptr
  const float* lb;        // lower bound row of this layer (kIFG; natural order), or nullptr
  const float* hin;       // kO: layer input h; kDown: resid
  int oLc, oK8;           // chain geometry of the output vector
  float* state;           // kIFG: this layer's recurrent state [H] (natural order)
  float* recur;           // kIFG out: silu(recurrence output)
  float* gout;            // kIFG out
  float* out;             // kIFG layer 0: copy of the embedding row (h); kO: resid;
                          // kGate: z; kDown: next h; kLM: logits (natural, may be null)
  unsigned long long* keys;  // argmax keys: one per kLM block; reduced by layer-0 kIFG
  int nkeys;
  int64_t* hist;          // kIFG layer 0: token history, hist[*hist_pos]++ (below hist_cap)
  int32_t* hist_pos;
  int hist_cap;
  int wgroups;            // set by launch_decode: output groups per block whose weight words
                          // are copied into LDS at entry (0: read from global in the GEMV)
  int32_t* acc;           // kOp, integer modes: the int32 accumulators [N] (tails and the
                          // Q5.10 bias included), or null
};

// Bytes of dynamic LDS one block may allocate on the current device.
int lds_limit();

constexpr int kLMBlocks = 2048;  // most lm_head blocks (argmax key slots)
// lm_head grid for `groups` output groups over hidden size K: every block recomputes the
// final norms over K, so wide rows take fewer blocks, each striding over several groups
// (measured: one group per block at K = 1024, 512 blocks at K = 2048 and 2560).
inline int lm_blocks(int groups, int K) {
  const int cap = K <= 1024 ? kLMBlocks : 512;
  return groups < cap ? groups : cap;
}
hipError_t launch_decode(DecKind kind, Mode mode, const DecArgs& a, hipStream_t s);
// Timing runs: while both events are set, launch_decode records them at its kernel's own start
// and end (hipExtLaunchKernelGGL), the timestamps a profiler's kernel trace reports, instead of
// around the launch on the stream.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;
// rows of x [rows, K] -> chain-transposed rows out [rows, 8*Lc + 8]
hipError_t launch_to_chain(const float* x, float* out, int rows, int K, int Lc, hipStream_t s);

// Argmax key: (orderable float bits << 32) | (0xFFFFFFFF - index): the max key is the first
// index of the largest value (the reference's strict `>` scan, hgrn_model.cpp:270-273).
__host__ __device__ inline int64_t key_index(unsigned long long k) {
  return static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFull));
}

// ---- generic row kernels (mmf_ops.hip) ------------------------------------------------
// Chain-transposed activations of `rows` rows for NA projections:
//   float: y  [NA][rows][8*Lc + 8]
//   int:   q  [NA][2 planes][fragment tiles] int8 codes (plane 1 unused in kInt8),
//          ct [NA][rows][8] int32 tail codes, sa [NA][rows] int8 scales
// The integer planes are stored in the matrix cores' operand order: rows in groups of 32,
// chain positions in chunks of 32, and each (group, chunk) fragment one contiguous 1 KB in
// which lane l = row % 32 + 32 * (pos / 16 % 2) holds 16 consecutive positions. A fragment
// then moves to LDS as one linear 1 KB transfer. Each plane holds rows rounded up to 32.
struct ActBuf {
  float* y = nullptr;
  int8_t* q = nullptr;
  int32_t* ct = nullptr;
  float* sa = nullptr;
  int Lc = 0, K = 0, K8 = 0, nb = 0, ntail = 0, rows = 0, na = 0;
  __host__ __device__ size_t ystride() const { return static_cast<size_t>(8 * Lc + 8); }
  __host__ __device__ int rows32() const { return (rows + 31) & ~31; }
  // bytes of one plane of one projection
  __host__ __device__ size_t qplane() const { return static_cast<size_t>(rows32()) * 8 * Lc; }
  // byte offset of the row's first fragment within a plane (position 0)
  __host__ __device__ size_t qrow(int row) const {
    return static_cast<size_t>(row >> 5) * (Lc / 4) * 1024 + (row & 31) * 16;
  }
  // byte offset of chain position pos from the row's base
  __host__ __device__ static size_t qpos(int pos) {
    return static_cast<size_t>(pos >> 5) * 1024 + ((pos >> 4) & 1) * 512 + (pos & 15);
  }
  __host__ __device__ size_t qoff(int proj, int plane, int row, int pos) const {
    return (2 * static_cast<size_t>(proj) + plane) * qplane() + qrow(row) + qpos(pos);
  }
};

// Stage kinds of the row prologue (what happens before the BitLinear's own RMSNorm).
// kPreMixSwish: kPreSwish whose x2 is computed in the prologue by the recurrence step of
// independent streams (launch_mixer's stream_state form, hgrn_model.cpp:109-150): x2 holds
// the i projection, mix_f the f projection, and mix_state [rows, K] is updated in place.
enum PreKind : int { kPreNone = 0, kPreNorm = 1, kPreSwish = 2, kPreMixSwish = 3 };

struct PrologueArgs {
  const float* x;      // [rows, K]
  const float* x2;     // kPreSwish: recurrence output rows [rows, K]; kPreMixSwish: i rows
  const float* pre_w;  // stage-1 norm weight
  const float* pre_wT; // the same, chain-transposed [8*Lc + 8] (null: not for k_rowseg)
  const float* normw[3];
  const float* normwT[3];  // the same, chain-transposed [8*Lc + 8] (null: the general kernel)
  int na;
  PreKind pre;
  float eps, qs;
  const float* mix_f;  // kPreMixSwish: f projection rows [rows, K]
  float* mix_state;    // kPreMixSwish: recurrent state [rows, K], read and updated
  const float* mix_lb; // kPreMixSwish: lower bounds [K] or null
};
// kPreMixSwish runs only in the float4 prologue: it returns hipErrorNotSupported, launching
// nothing, where that does not apply (the caller then runs launch_mixer and kPreSwish).
hipError_t launch_prologue(Mode mode, const PrologueArgs& a, ActBuf& act, hipStream_t s);

// Integer codes [rows, K] (int16-range, as int32) -> planes (TernaryBackend path).
hipError_t launch_codes_to_planes(const int32_t* x, ActBuf& act, hipStream_t s);
// The inverse: planes (and tail codes) of act's na projections -> int32 codes
// [na][rows][K] in natural element order, for an external integer matmul.
hipError_t launch_planes_to_codes(const ActBuf& act, Mode mode, int32_t* codes, hipStream_t s);

enum EpiKind : int { kEpiStore = 0, kEpiAdd = 1, kEpiSwigluPair = 2 };

struct GemmArgs {
  ProjDev p[3];
  int nmat;            // matrices (grid.z)
  int rows;
  Mode mode;
  float inv_fixed[3];
  bool raw_acc;        // int modes: write integer accumulators only (TernaryBackend)
  EpiKind epi;
  const float* add;    // kEpiAdd: out = add + val (same shape as out)
  float* out[3];       // [rows, N] per matrix (kEpiSwigluPair: out[0] = z [rows, N/2])
  int32_t* acc[3];     // optional int32 accumulators [rows, N]
  int swiglu_n;        // kEpiSwigluPair: rows * (N/2), for the tail rule
  // matrix-core split-K (set by launch_gemm): ksplit partial tiles [ksplit][nmat][rows][N]
  // of exact int32 sums in ws, reduced in split order by a second kernel
  int ksplit;
  int32_t* ws;
  // launch_acc_epilogue: ws holds complete accumulators [nmat][rows][N] (tails and the
  // Q5.10 bias included, as an external integer matmul returns them)
  bool ext_acc;
};
// Dispatches the integer modes to the matrix-core kernel (mmf_mfma.hip) from
// mfma_min_rows() rows on, everything else to the dot-product kernel.
hipError_t launch_gemm(const GemmArgs& a, const ActBuf& act, hipStream_t s);
hipError_t launch_gemm_mfma(const GemmArgs& a, const ActBuf& act, hipStream_t s);
// Dequantisation and output stage (a.epi) of complete integer accumulators a.ws
// [nmat][rows][N] (integer modes): what the GEMM's epilogue does after its own matmul.
hipError_t launch_acc_epilogue(const GemmArgs& a, const ActBuf& act, hipStream_t s);
// Float mode on the fp32 matrix cores (mmf_mfma_f.hip), bit-exact with the FMA chains;
// used from float_mfma_min_rows() rows on when mfma_f_ok(a).
bool mfma_f_ok(const GemmArgs& a);
hipError_t launch_gemm_mfma_f(const GemmArgs& a, const ActBuf& act, hipStream_t s);

// The TernaryBackend seam's few-row integer matmul (mmf_ternary_matmul_host): k projections of
// one shape g, b rows each (b <= seam_max_rows()); x [k][b][K] int32 codes and acc [k][b][N]
// int32 in memory the device reads and writes directly (the caller's pinned host staging).
constexpr int kSeamMaxProj = 8;
struct SeamArgs {
  const uint32_t* pk[kSeamMaxProj];
  const int8_t* tail[kSeamMaxProj];
  const int32_t* rowsum[kSeamMaxProj];
  const int32_t* x;
  int32_t* acc;
  Geom g;
  int b;
};
int seam_max_rows();
hipError_t launch_seam_dot(const SeamArgs& a, int k, hipStream_t s);

// ---- device calibration (mmf_peaks.hip) ----------------------------------------------------
// out = {HBM read GB/s, Infinity Cache read GB/s, int8 MFMA TOP/s, fp32 FMA TFLOP/s}; allocates
// and frees 2 GiB of scratch, synchronizes the stream.
hipError_t measure_peaks(int cus, hipStream_t s, double out[4]);
// Bytes of int32 workspace launch_gemm needs for `a` (0 when it will not split K); the
// caller passes at least that much in a.ws.
size_t gemm_workspace_bytes(const GemmArgs& a);
// Rows from which the integer modes use the matrix cores (MMF_MFMA_MIN_ROWS, default 8;
// 0 disables them).
int mfma_min_rows();
// Rows from which float mode uses the fp32 matrix cores (MMF_FLOAT_MFMA_MIN_ROWS, default
// 16; 0 disables them).
int float_mfma_min_rows();

// HGRN gate + recurrence over rows (hgrn_model.cpp:109-150). i, f, g: [rows, H].
// stream_state = false: rows are time steps of one sequence, state [H] carried in order.
// stream_state = true: rows are independent streams, state [rows, H].
// keep_gates: f is overwritten with the gated forget values and scan_out receives the
// recurrence input ([rows, H]; required for a time scan of more than one row). Without it,
// a time scan with H % 16 == 0 computes the gates inside the scan kernel and leaves f and
// scan_out untouched.
hipError_t launch_mixer(const float* i, float* f, float* scan_out, float* recur, float* state,
                        const float* lb, int rows, int H, bool stream_state, bool keep_gates, hipStream_t s);
// The chunked parallel scan of a prefill (float mode, opt-in): the gate math of the raw i
// and f rows [rows, H] and the recurrence from state [H] (updated), with chunk summaries in
// ws (scan_chunked_ws_floats floats). Results are within fp32 rounding of the time-ordered
// scan, not equal to it. Needs H % 64 == 0.
size_t scan_chunked_ws_floats(int rows, int H);
hipError_t launch_scan_chunked(const float* i, const float* f, const float* lb, float* recur, float* state,
                               float* ws, int rows, int H, hipStream_t s);
// The same over nseg sequences stacked as row segments [off[b], off[b + 1]) (device array of
// nseg + 1 offsets), segment b scanning from and into state + b * H. Needs H % 8 == 0, so
// that no element of any segment is a SIMD tail element of the gate math. keep_gates as
// for launch_mixer (without it the gate math runs inside the segment scan).
hipError_t launch_mixer_segs(const float* i, float* f, float* scan, float* recur, float* state, const float* lb,
                             const int* off, int nseg, int rows, int H, bool keep_gates, hipStream_t s);
// rows idx[r] (device) of x [*, K] -> out [n, K]
hipError_t launch_gather_rows(const float* x, const int* idx, float* out, int n, int K, hipStream_t s);

// Embedding gather rows (hgrn_model.cpp:321-326).
hipError_t launch_embed(const float* emb, const int64_t* ids, float* h, int rows, int H,
                        hipStream_t s);
// Final RMSNorm rows (hgrn_model.cpp:235,440): plain rmsnorm kernel.
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int cols, float eps,
                          hipStream_t s);
// Q5.10 codes of rows y [rows, K] (SIMD body / scalar tail per row).
hipError_t launch_quant_rows(const float* y, int32_t* q, int rows, int K, float qs, hipStream_t s);
// Row argmax over [rows, V] logits -> ids.
hipError_t launch_argmax_rows(const float* logits, int rows, int V, int64_t* ids, hipStream_t s);
// Elementwise ops for the op-level API (kernels.hpp:54-68).
hipError_t launch_swiglu(const float* a, const float* b, float* out, size_t n, hipStream_t s);
hipError_t launch_swishgate(const float* g, const float* o, const float* w, float* out, int rows,
                            int cols, float eps, hipStream_t s);
hipError_t launch_scan(const float* i, const float* f, float* out, float* state, int T, int D,
                       hipStream_t s);

// ---- weight repack (mmf_ops.hip) ----------------------------------------------------------
hipError_t launch_pack(const int8_t* wq, const Geom& g, uint32_t* pk, int8_t* tail, int32_t* rowsum,
                       hipStream_t s);
// slab words -> matrix-core tile order (pair: interleave the two halves by 32-column group,
// which needs N % 64 == 0); pkm holds pkm_words(g) words.
size_t pkm_words(const Geom& g);
bool pkm_pairable(const Geom& g);
hipError_t launch_pack_mfma(const uint32_t* pk, const Geom& g, bool pair, uint32_t* pkm, hipStream_t s);
// slab words -> the fp4 slab of the float-mode decode GEMV: the same groups and lanes with 8 codes
// per word (2 Wc words per chain, code t of a word in nibble t: 0 -> 0x0, +1 -> 0x2, -1 -> 0xA,
// E2M1 values that v_cvt_scalef32_pk_f32_fp4 converts exactly); pk4 holds pk4_words(g) words.
size_t pk4_words(const Geom& g);
hipError_t launch_pack4(const uint32_t* pk, const Geom& g, uint32_t* pk4, hipStream_t s);

}  // namespace mmf
