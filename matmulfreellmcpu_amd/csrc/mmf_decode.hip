// mmf_decode.hip -- fused single-row decode kernels, one launch per BitLinear group of a
// layer (Model::block at T = 1, hgrn_model.cpp:80-195):
//   kIFG  : [embed] -> attn_norm -> BitLinear norm -> i/f/g GEMVs -> sigmoid, lower bound,
//           swiglu, recurrence step (hgrn_model.cpp:95-150)
//   kO    : g_norm (RMSNorm(g) * silu(recur)) -> BitLinear norm -> o GEMV -> resid = h + o
//   kGate : mlp_norm -> BitLinear norm -> gate/up GEMV (rows c and I + c) -> swiglu
//   kDown : BitLinear norm -> down GEMV -> h = resid + d
//   kLM   : final norm -> BitLinear norm -> lm_head GEMV -> logits, one argmax key per block
//           (reduced by the next step's layer-0 kIFG or by the host)
//
// Latency is what bounds a batch-1 decode step, so each kernel is organised around it:
//  * all vectors passed between these kernels, and all norm weights, are stored in the
//    chain-transposed order (mmf_internal.hpp) with zero padding, so a block's prologue is
//    a contiguous float4 copy into LDS and the reference's 8-lane reductions run over LDS
//    rows without index arithmetic or bounds checks (zero padding adds exact zeros);
//  * every global load that does not depend on the prologue -- the block's first 16 weight
//    words per matrix, the epilogue operands, the prologue inputs -- is issued at entry;
//  * every block recomputes the (order-exact) row norms of its input vector, so no
//    grid-wide synchronisation is needed inside a launch.
// Thread (ol, j) of a matrix's 128 threads sums chain j of output og*16+ol, which is the
// reference's AVX2 lane j (16 outputs x 8 chains per output group).
#include <hip/hip_ext.h>

#include <cstdlib>

#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

thread_local LaunchEvents g_launch_events;

namespace {

// kernel<<<grid, block, lds, s>>>(args...), or with g_launch_events recorded at the kernel's
// start and end
template <class K, class... A>
hipError_t launch_k(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, A... args) {
  const LaunchEvents ev = g_launch_events;
  if (ev.start && ev.stop) hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s, ev.start, ev.stop, 0, args...);
  else kernel<<<grid, block, lds, s>>>(args...);
  return hipGetLastError();
}

template <int KIND> struct KindTraits;
// NM matrices (one wave pair each), NA activation vectors, NP prologue source vectors
template <> struct KindTraits<kIFG> { static constexpr int NM = 3, NA = 3, NP = 5; };
template <> struct KindTraits<kO> { static constexpr int NM = 1, NA = 1, NP = 4; };
template <> struct KindTraits<kGate> { static constexpr int NM = 2, NA = 1, NP = 3; };
template <> struct KindTraits<kDown> { static constexpr int NM = 1, NA = 1, NP = 2; };
template <> struct KindTraits<kLM> { static constexpr int NM = 1, NA = 1, NP = 3; };
template <> struct KindTraits<kOp> { static constexpr int NM = 1, NA = 1, NP = 2; };

typedef __attribute__((address_space(3))) void lds_void;

// Lane l's segment of a chain-transposed vector of chain length 32 RC: floats
// [4 RC l, 4 RC (l + 1)), i.e. segment l % 8 of chain l / 8, plus the 8 tail floats after
// the 8 rows (the same for every lane).
template <int RC>
__device__ __forceinline__ void load_seg(const float* p, int l, float4 (&d)[RC], float (&t)[8]) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int c = 0; c < RC; ++c) d[c] = q[l * RC + c];
  const float4 t0 = q[64 * RC], t1 = q[64 * RC + 1];
  t[0] = t0.x; t[1] = t0.y; t[2] = t0.z; t[3] = t0.w;
  t[4] = t1.x; t[5] = t1.y; t[6] = t1.z; t[7] = t1.w;
}

// A block is KS parts of NM * 128 threads. In every part, thread (mi, ol, j) sums chain j of
// output ol of the block's group for matrix mi. What the parts do:
//   kLM             part p takes the block's p-th output group (the groups a block strides
//                   over run side by side);
//   integer modes   part p sums words [p Wc / KS, (p + 1) Wc / KS) of every chain; the int32
//                   partials meet in LDS (integer sums do not depend on their order);
//   float           only part 0 runs the GEMV (a chain is one reference lane, in order); the
//                   other parts share the loads, the normalisation and the encoding.
//
// W4 (float mode, not kLM): the GEMV reads the fp4 slab pk4 (8 codes per word, one conversion
// per two codes) instead of the 2-bit slab (a byte permute per two codes into fp16 pairs).
//
// RC > 0 (the chain length Lc is 32 RC, no row padding): wave 0 runs both norm chains from
// registers. Lane 8j + s holds segment s (4 RC consecutive steps) of chain j of the input
// row and of the stage-1 weights; each chain runs segment by segment, every lane summing its
// own segment and a DPP row shift handing the running sum to the next segment's lane, so a
// step costs one dependent FMA (about 6.4 cycles) instead of an LDS round trip. Wave 0 then
// writes the stage-1 output to LDS for the encoding pass; the row norm needs no barrier of
// its own. RC == 0 runs the same chains over LDS rows (any Lc).
// Integer gate/up launches 352 to 432 blocks of 512 threads: two must share a CU (4 waves per
// SIMD, at most 128 VGPRs) or the grid runs in two rounds (hidden 2560 needed 129 VGPRs and
// took 13.3 us per launch). At the register-chain widths the cap costs a few spilled pointers.
template <int MODE, int KIND, int RC>
constexpr int kDecMinWaves = (MODE != kFloat && KIND == kGate && RC > 0) ? 4 : 1;

template <int MODE, int KIND, int NV, int KS, int RC, bool W4>
__global__ __launch_bounds__(kBlock * KindTraits<KIND>::NM * KS) __attribute__((amdgpu_waves_per_eu(kDecMinWaves<MODE, KIND, RC>)))
void k_decode(DecArgs a) {
  static_assert(!W4 || (MODE == kFloat && KIND != kLM), "fp4 words are for the float layer GEMVs");
  constexpr int NM = KindTraits<KIND>::NM, NA = KindTraits<KIND>::NA, NP = KindTraits<KIND>::NP;
  constexpr int BM = kBlock * NM;  // threads of one part
  constexpr int BS = BM * KS;
  constexpr bool LMG = (KIND == kLM);                         // parts = output groups
  constexpr bool KSPLIT = (MODE != kFloat) && !LMG && KS > 1;  // parts = word ranges
  extern __shared__ float smem[];
  // ---- kernel arguments ---------------------------------------------------------------------
  // Every field the launch uses is read here and pinned in scalar registers: the scalar loads
  // then issue back to back at entry and cost one round trip, instead of one dependent round
  // trip each where a field is first used (the compiler otherwise sinks them to their uses).
  const int mis = __builtin_amdgcn_readfirstlane((static_cast<int>(threadIdx.x) >> 6) % (2 * NM) >> 1);  // wave's matrix
  const ProjDev& Pa = a.p[KIND == kIFG ? mis : 0];
  const Geom& g0 = a.p[0].g;
  const int gN = g0.N, gK = g0.K, Lc = g0.Lc, nt = g0.ntail, Wc = g0.Wc, gng = g0.ngroups;
  const uint32_t* const pk = W4 ? Pa.pk4 : Pa.pk;
  const int8_t* const ptail = Pa.tail;
  const int32_t* const prowsum = Pa.rowsum;
  const float pscale = Pa.scale_w, pinv = Pa.inv_scale_w, invfx = a.inv_fixed[KIND == kIFG ? mis : 0];
  const float* const nw0 = a.p[0].normwT;
  const float* const nw1 = a.p[1].normwT;
  const float* const nw2 = a.p[2].normwT;
  const float* const ax = a.x;
  const float* const aembT = a.embT;
  const float* const ax2 = a.x2;
  const float* const apre = a.pre_w;
  const float* const alb = a.lb;
  const float* const ahin = a.hin;
  float* const astate = a.state;
  float* const arecur = a.recur;
  float* const agout = a.gout;
  float* const aout = a.out;
  unsigned long long* const akeys = a.keys;
  int64_t* const ahist = a.hist;
  int32_t* const ahist_pos = a.hist_pos;
  const int awg = a.wgroups, aoLc = a.oLc, aoK8 = a.oK8, aH = a.H, avocab = a.vocab, ankeys = a.nkeys,
            ahist_cap = a.hist_cap;
  const float aeps = a.eps, aqs = a.qs;
#define MMF_PIN_BASE                                                                           \
  "s"(gN), "s"(gK), "s"(Lc), "s"(nt), "s"(Wc), "s"(pk), "s"(ptail), "s"(prowsum), "s"(pscale),  \
      "s"(pinv), "s"(invfx), "s"(nw0), "s"(ax), "s"(aout), "s"(awg), "s"(aeps), "s"(aqs)
  // one statement per kind, so that all the loads precede it (layer 0's token-gather fields
  // are left to load where used)
  if constexpr (KIND == kIFG)
    MMF_PIN(MMF_PIN_BASE, "s"(nw1), "s"(nw2), "s"(alb), "s"(astate), "s"(arecur), "s"(agout), "s"(aH), "s"(apre),
            "s"(aoLc), "s"(aoK8));
  else if constexpr (KIND == kO)
    MMF_PIN(MMF_PIN_BASE, "s"(apre), "s"(ax2), "s"(ahin), "s"(aoLc), "s"(aoK8));
  else if constexpr (KIND == kGate)
    MMF_PIN(MMF_PIN_BASE, "s"(gng), "s"(apre), "s"(aoLc), "s"(aoK8));
  else if constexpr (KIND == kDown)
    MMF_PIN(MMF_PIN_BASE, "s"(ahin), "s"(aoLc), "s"(aoK8));
  else
    MMF_PIN(MMF_PIN_BASE, "s"(apre), "s"(akeys));
#undef MMF_PIN_BASE
  const int Ww = W4 ? 2 * Wc : Wc;  // slab words per chain
  const int W = 8 * Lc + 8;  // floats of a chain-transposed vector in global memory
  const int F4 = W / 4;  // float4s of a chain-transposed vector
  // LDS copies pad each chain row by 16 bytes so that the 8 chain lanes of a wave read
  // different banks: float rows LS floats apart, int8 plane rows LQ bytes apart.
  const int L32 = (Lc + 31) / 32 * 32;  // rows zero-filled to whole 32-value chain batches
  const int LS = L32 + 4, WL = 8 * LS + 8, LQ = Lc + 16;
  const int tid = threadIdx.x, part = tid / BM, mi = (tid % BM) >> 7, lt = tid & 127, ol = lt >> 3, j = lt & 7;
  const int ai = (NA > 1) ? mi : 0;  // this thread's activation vector
  const int nout = (KIND == kGate) ? gN / 2 : gN;
  const int ngroups_out = (nout + kGroup - 1) / kGroup;

  float* X = smem;           // [WL] input row
  float* S = X + WL;         // [WL] kO: silu(recur)
  float* red = S + WL;       // [32] chain partials, per-wave maxima and argmax keys
  float* vals = red + 32;    // [KS][NM][16] per-part, per-matrix results of the block's outputs
  float* Y = vals + 48 * KS; // float: NA x [WL]; int: NA x 2 planes x [8 LQ] bytes + tails + scales
  int8_t* Q = reinterpret_cast<int8_t*>(Y);
  int32_t* CT = reinterpret_cast<int32_t*>(Q + NA * 16 * LQ);
  float* SA = reinterpret_cast<float*>(CT + NA * 8);
  // [NM][G][Wc][128] all weight words of the block's G output groups, slab row layout
  // (16-byte aligned: the weight copies write 16 bytes per lane)
  uint32_t* WX = (MODE == kFloat) ? reinterpret_cast<uint32_t*>(Y + NA * WL)
                                  : reinterpret_cast<uint32_t*>(SA + ((NA + 3) & ~3));
  const int G = awg;

  // ---- entry: issue every load that does not depend on the prologue --------------------
  const int mrow = (KIND == kGate && mi == 1) ? gng / 2 : 0;  // gate: the up half
  // epilogue owners of the single-group kinds: part 0, matrix 0, lane j == 0
  const int o0 = static_cast<int>(blockIdx.x) * kGroup + ol;
  const bool epi = !LMG && part == 0 && mi == 0 && j == 0 && o0 < nout;
  const int po = epi ? ((o0 < aoK8) ? (o0 & 7) * aoLc + (o0 >> 3) : 8 * aoLc + (o0 - aoK8)) : 0;
  float e_lb = 0.0f, e_st = 0.0f, e_hin = 0.0f;
  if (epi) {
    if (KIND == kIFG) {
      if (alb) e_lb = alb[o0];
      e_st = astate[o0];
    }
    if (KIND == kO || KIND == kDown) e_hin = ahin[po];
  }
  // FixedQ510 with one group per block: the 128 * rowsum term of lane j == 0's output, now
  const int32_t e_rs =
      (MODE == kFixed && !LMG && j == 0 && o0 < nout) ? 128 * prowsum[o0 + ((KIND == kGate && mi == 1) ? nout : 0)] : 0;

  // layer 0: the token is the argmax over the previous lm_head's per-block keys
  int64_t tok = 0;
  if (KIND == kIFG && ax == nullptr) {
    unsigned long long best = 0ull;
    for (int e0 = tid; e0 < ankeys; e0 += 8 * BS) {  // 8 keys per thread in flight at once
      unsigned long long k[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) k[u] = e0 + u * BS < ankeys ? akeys[e0 + u * BS] : 0ull;
#pragma unroll
      for (int u = 0; u < 8; ++u) best = k[u] > best ? k[u] : best;
    }
    best = wave_max_u64(best);
    unsigned long long* r64 = reinterpret_cast<unsigned long long*>(vals);
    if ((tid & 63) == 0) r64[tid >> 6] = best;
    __syncthreads();
    best = r64[0];
    for (int w = 1; w < BS / 64; ++w) best = r64[w] > best ? r64[w] : best;
    tok = key_index(best);
    if (tok < 0 || tok >= avocab) tok = 0;
    if (blockIdx.x == 0 && tid == 0 && ahist) {
      const int pos = *ahist_pos;
      if (pos < ahist_cap) ahist[pos] = tok;
      *ahist_pos = pos + 1;
    }
  }

  // prologue sources (all chain-transposed, zero-padded, W floats):
  //   0: input row   1: stage-1 weight (kO: recur)   then the BitLinear norm weights
  const float* src[NP];
  src[0] = (KIND == kIFG && ax == nullptr) ? aembT + static_cast<size_t>(tok) * W : ax;
  if (KIND == kIFG) { src[1] = apre; src[2] = nw0; src[3] = nw1; src[4] = nw2; }
  if (KIND == kO) { src[1] = ax2; src[2] = apre; src[3] = nw0; }
  if (KIND == kGate || KIND == kLM) { src[1] = apre; src[2] = nw0; }
  if (KIND == kDown) { src[1] = nw0; }
  constexpr int NW0 = NP - NA;              // first BitLinear norm-weight source
  constexpr int PW = (KIND == kO) ? 2 : 1;  // which source holds the stage-1 weight
  // RC > 0: wave 0 loads its segments of the input row, the stage-1 weight and kO's gate first
  constexpr int RX = RC > 0 ? RC : 1;
  float4 xs[RX], ws[RX], gs[RX];
  float xt[8], wt[8], gt[8];
  if constexpr (RC > 0) {
    if (tid < 64) {
      load_seg<RC>(src[0], tid, xs, xt);
      if constexpr (KIND != kDown) load_seg<RC>(src[PW], tid, ws, wt);
      if constexpr (KIND == kO) load_seg<RC>(src[1], tid, gs, gt);
    }
  }
  // the rest in the block layout (RC > 0: only the BitLinear norm weights)
  constexpr int S0 = RC > 0 ? NW0 : 0;
  float4 v[NP][NV];
#pragma unroll
  for (int s = S0; s < NP; ++s)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + i * BS;
      v[s][i] = (e < F4) ? reinterpret_cast<const float4*>(src[s])[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  // the weight words of the block's output groups (after the input, which the norms need
  // first): straight into LDS in the slab order, 16 bytes per lane, so one instruction of a
  // wave moves 1 KB (two slab rows); the 2 KS waves of a matrix take every 2 KS-th KB. A slab
  // of an odd number of rows ends in half a KB, which lanes 32..63 skip. With register chains
  // wave 0 issues none of them: its chains wait for every load the wave has in flight (the
  // copy loops' counts are not known at compile time), and behind its share of the copies
  // the 2.7B lm_head's first chain waited 3.3 us for the launch's whole weight stream; the
  // other waves of matrix 0 take its share (2.7B float decode 819 -> 862 tok/s). The wave
  // indices are scalars (one value per wave).
  {
    const int w64 = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wmi = (w64 % (2 * NM)) >> 1, wv = (w64 / (2 * NM)) * 2 + (w64 & 1), lane = lt & 63;
    const int nwords = Ww * 128;
    constexpr bool SKIP0 = RC > 0;
    const int nwv = 2 * KS - ((SKIP0 && wmi == 0) ? 1 : 0);  // copying waves of this matrix
    const int cw = (SKIP0 && wmi == 0) ? wv - 1 : wv;        // this wave's index among them
    if (cw >= 0) {
      for (int gi = 0; gi < G; ++gi) {
        const int og_i = static_cast<int>(blockIdx.x) + gi * static_cast<int>(gridDim.x);
        if (og_i >= ngroups_out) break;
        const uint32_t* sx = pk + static_cast<size_t>(og_i + mrow) * nwords;
        uint32_t* dx = WX + (wmi * G + gi) * nwords;
        for (int c = cw * 256; c < nwords; c += 256 * nwv)
          if (c + 4 * lane < nwords) __builtin_amdgcn_global_load_lds(sx + c + 4 * lane, (lds_void*)(dx + c), 16, 0, 0);
      }
    }
  }
  // LDS float4 index of each of this thread's global float4s
  int li[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int p = 4 * (tid + i * BS);
    const int jj = p / Lc;
    li[i] = (p < 8 * Lc) ? (jj * LS + (p - jj * Lc)) / 4 : (8 * LS + (p - 8 * Lc)) / 4;
  }
  float r2;
  if constexpr (RC > 0) {
    // ---- both norm chains on wave 0, from registers (no barrier until the row is in LDS) ----
    if (tid < 64) {
      if constexpr (KIND != kDown) {
        const float r1 = rstd_of(seg_sumsq<RC>(xs, xt, nt), gK, aeps);
#pragma unroll
        for (int c = 0; c < RC; ++c) {
          float4 x = xs[c];
          const float4 w = ws[c];
          x.x = (x.x * r1) * w.x; x.y = (x.y * r1) * w.y; x.z = (x.z * r1) * w.z; x.w = (x.w * r1) * w.w;
          if (KIND == kO) {
            const float4 sg = gs[c];
            x.x = x.x * sg.x; x.y = x.y * sg.y; x.z = x.z * sg.z; x.w = x.w * sg.w;
          }
          xs[c] = x;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          xt[t] = (xt[t] * r1) * wt[t];
          if (KIND == kO) xt[t] = xt[t] * gt[t];
        }
      }
      const float ss2 = seg_sumsq<RC>(xs, xt, nt);
      // the stage-1 output into the LDS rows: lane 8j + s -> row j, floats [4 RC s, 4 RC (s + 1))
      float4* xr = reinterpret_cast<float4*>(X + (tid >> 3) * LS + 4 * RC * (tid & 7));
#pragma unroll
      for (int c = 0; c < RC; ++c) xr[c] = xs[c];
      if (tid == 0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) X[8 * LS + t] = xt[t];
        red[0] = rstd_of(ss2, gK, aeps);
      }
    }
    __syncthreads();
    r2 = red[0];
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + i * BS;
      if (e < F4) {
        reinterpret_cast<float4*>(X)[li[i]] = v[0][i];
        if (KIND == kO) reinterpret_cast<float4*>(S)[li[i]] = v[1][i];
      }
    }
    for (int z = tid; z < 8 * (L32 - Lc); z += BS) {  // zeros past Lc in each row
      const int jj = z / (L32 - Lc);
      X[jj * LS + Lc + (z - jj * (L32 - Lc))] = 0.0f;
    }
    __syncthreads();
    // ---- stage 1: the kernel's own pre-norm -----------------------------------------------
    if (KIND != kDown) {
      chain_begin(X, Lc, LS, red);
      __syncthreads();
      const float r1 = rstd_of(chain_end(X, LS, nt, red), gK, aeps);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = tid + i * BS;
        if (e < F4) {
          float4 x = reinterpret_cast<float4*>(X)[li[i]];
          const float4 w = v[PW][i];
          x.x = (x.x * r1) * w.x; x.y = (x.y * r1) * w.y; x.z = (x.z * r1) * w.z; x.w = (x.w * r1) * w.w;
          if (KIND == kO) {
            const float4 sg = reinterpret_cast<float4*>(S)[li[i]];
            x.x = x.x * sg.x; x.y = x.y * sg.y; x.z = x.z * sg.z; x.w = x.w * sg.w;
          }
          reinterpret_cast<float4*>(X)[li[i]] = x;
        }
      }
      __syncthreads();
    }
    // ---- stage 2: BitLinear RMSNorm -------------------------------------------------------
    chain_begin(X, Lc, LS, red);
    __syncthreads();
    r2 = rstd_of(chain_end(X, LS, nt, red), gK, aeps);
  }
  // ---- activation encoding -------------------------------------------------------------------
#pragma unroll
  for (int aa = 0; aa < NA; ++aa) {
    if (MODE == kFloat) {
      float4* yo = reinterpret_cast<float4*>(Y + aa * WL);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = tid + i * BS;
        if (e < F4) {
          const float4 x = reinterpret_cast<float4*>(X)[li[i]];
          const float4 w = v[NW0 + aa][i];
          yo[li[i]] = make_float4((x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w);
        }
      }
    } else {
      float sa = 0.0f;
      if (MODE == kInt8) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int e = tid + i * BS;
          if (e < F4) {
            const float4 x = reinterpret_cast<float4*>(X)[li[i]];
            const float4 w = v[NW0 + aa][i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf((x.x * r2) * w.x), fabsf((x.y * r2) * w.y)),
                               fmaxf(fabsf((x.z * r2) * w.z), fabsf((x.w * r2) * w.w))));
          }
        }
        m = wave_max(m);
        if ((tid & 63) == 0) red[8 + (tid >> 6)] = m;
        __syncthreads();
        m = red[8];
        for (int w = 1; w < BS / 64; ++w) m = fmaxf(m, red[8 + w]);
        sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
        if (tid == 0) SA[aa] = sa;
      }
      int8_t* q = Q + aa * 16 * LQ;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = tid + i * BS;
        if (e < F4) {
          const float4 x = reinterpret_cast<float4*>(X)[li[i]];
          const float4 w = v[NW0 + aa][i];
          const float y[4] = {(x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w};
          if (4 * e < 8 * Lc) {
            uint32_t hi = 0, lo = 0;
            int32_t cd[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) cd[u] = (MODE == kFixed) ? q510_body(y[u], aqs) : q8_of(y[u], sa);
            if (MODE == kFixed) pack_split4(cd, hi, lo);
            else hi = pack_low4(cd);
            const int jj = (4 * e) / Lc, qp = jj * LQ + (4 * e - jj * Lc);  // byte position
            *reinterpret_cast<uint32_t*>(q + qp) = hi;
            if (MODE == kFixed) *reinterpret_cast<uint32_t*>(q + 8 * LQ + qp) = lo;
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int t = 4 * e - 8 * Lc + u;
              CT[aa * 8 + t] = (t < nt) ? ((MODE == kFixed) ? q510_tail(y[u], aqs) : q8_of(y[u], sa)) : 0;
            }
          }
        }
      }
      if (MODE == kInt8) __syncthreads();  // red[8..] reused by the next vector's max
    }
  }
  if (G > 0) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS copies landed
  __syncthreads();

  // ---- GEMV: each thread one chain (or one chain's word range) of one matrix ----------------
  // One word = 16 codes of chain j against 16 activations: act_of reads the activations from
  // LDS, word_of runs the chain over them.
  struct Act {
    float4 f[MODE == kFloat ? (W4 ? 2 : 4) : 1];
    uint4 h, l;
  };
  auto act_of = [&](int m) {
    Act r;
    if (MODE == kFloat) {
      constexpr int NF = W4 ? 2 : 4;  // float4s of one word's activations
      const float4* yl = reinterpret_cast<const float4*>(Y + ai * WL + j * LS + 4 * NF * m);
#pragma unroll
      for (int q = 0; q < NF; ++q) r.f[q] = yl[q];
    } else {
      const int8_t* ql = Q + ai * 16 * LQ + j * LQ + 16 * m;
      r.h = *reinterpret_cast<const uint4*>(ql);
      if (MODE == kFixed) r.l = *reinterpret_cast<const uint4*>(ql + 8 * LQ);
    }
    return r;
  };
  // The chain sums of this thread over words [m0, m1) of group og (slot gi of the LDS copy):
  // float in facc, integer planes in hacc / lacc.
  auto gemv = [&](int og, int gi, int m0, int m1, float& facc, int32_t& hacc, int32_t& lacc) {
    auto word_of = [&](uint32_t w, const Act& x) {
      if constexpr (W4) {
        facc = word_dot_f4(w, x.f[0], x.f[W4 ? 1 : 0], facc);
      } else if (MODE == kFloat) {
        const float y[16] = {x.f[0].x, x.f[0].y, x.f[0].z, x.f[0].w, x.f[1].x, x.f[1].y, x.f[1].z, x.f[1].w,
                             x.f[2].x, x.f[2].y, x.f[2].z, x.f[2].w, x.f[3].x, x.f[3].y, x.f[3].z, x.f[3].w};
        facc = word_dot_f(w, y, facc);
      } else {
        const uint32_t w0 = w4_i8(w, 0), w1 = w4_i8(w, 1), w2 = w4_i8(w, 2), w3 = w4_i8(w, 3);
        hacc = dot4(w3, x.h.w, dot4(w2, x.h.z, dot4(w1, x.h.y, dot4(w0, x.h.x, hacc))));
        if (MODE == kFixed) lacc = dot4(w3, x.l.w, dot4(w2, x.l.z, dot4(w1, x.l.y, dot4(w0, x.l.x, lacc))));
      }
    };
    if (W4 && G > 0 && RC > 0) {
      // fp4 words in LDS at a model width: the chain's 4 RC words fully unrolled, so the
      // compiler issues each word's reads (one word, two float4 of activations) well ahead
      // of its FMAs and the chain waits on no LDS round trip
      constexpr int NC4 = RC > 0 ? RC : 1;  // chunks of 4 words (32 codes); Ww = 4 RC
      const uint32_t* wl = WX + (mi * G + gi) * 4 * NC4 * 128 + lt;
      const float4* yl = reinterpret_cast<const float4*>(Y + ai * WL + j * LS);
      // chunk c + 1's reads are issued before chunk c's FMAs; the scheduling barriers keep the
      // compiler from sinking them to their uses (it otherwise reads one float4 ahead)
      uint32_t wa[4];
      float4 xa[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        wa[u] = wl[u * 128];
        xa[2 * u] = yl[2 * u];
        xa[2 * u + 1] = yl[2 * u + 1];
      }
#pragma unroll
      for (int c = 0; c < NC4; ++c) {
        uint32_t wb[4];
        float4 xb[8];
        if (c + 1 < NC4) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int m = 4 * (c + 1) + u;
            wb[u] = wl[m * 128];
            xb[2 * u] = yl[2 * m];
            xb[2 * u + 1] = yl[2 * m + 1];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) facc = word_dot_f4(wa[u], xa[2 * u], xa[2 * u + 1], facc);
        __builtin_amdgcn_sched_barrier(0);
        if (c + 1 < NC4) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            wa[u] = wb[u];
            xa[2 * u] = xb[2 * u];
            xa[2 * u + 1] = xb[2 * u + 1];
          }
        }
      }
    } else if (W4 && G > 0) {  // any other width: 4 words at a time
      const uint32_t* wl = WX + (mi * G + gi) * Ww * 128 + lt;
      const float4* yl = reinterpret_cast<const float4*>(Y + ai * WL + j * LS);
      int m = m0;
      for (; m + 4 <= m1; m += 4) {
        const uint32_t w0 = wl[m * 128], w1 = wl[(m + 1) * 128], w2 = wl[(m + 2) * 128], w3 = wl[(m + 3) * 128];
        const float4 a0 = yl[2 * m], a1 = yl[2 * m + 1], a2 = yl[2 * m + 2], a3 = yl[2 * m + 3];
        const float4 a4 = yl[2 * m + 4], a5 = yl[2 * m + 5], a6 = yl[2 * m + 6], a7 = yl[2 * m + 7];
        facc = word_dot_f4(w0, a0, a1, facc);
        facc = word_dot_f4(w1, a2, a3, facc);
        facc = word_dot_f4(w2, a4, a5, facc);
        facc = word_dot_f4(w3, a6, a7, facc);
      }
      for (; m < m1; ++m) facc = word_dot_f4(wl[m * 128], yl[2 * m], yl[2 * m + 1], facc);
    } else if (G > 0) {  // words in LDS: 4 at a time, all their reads issued before the chain
      const uint32_t* wl = WX + (mi * G + gi) * Ww * 128 + lt;
      int m = m0;
      for (; m + 4 <= m1; m += 4) {
        const uint32_t w0 = wl[m * 128], w1 = wl[(m + 1) * 128], w2 = wl[(m + 2) * 128], w3 = wl[(m + 3) * 128];
        const Act x0 = act_of(m), x1 = act_of(m + 1), x2 = act_of(m + 2), x3 = act_of(m + 3);
        word_of(w0, x0);
        word_of(w1, x1);
        word_of(w2, x2);
        word_of(w3, x3);
      }
      for (; m < m1; ++m) word_of(wl[m * 128], act_of(m));
    } else {  // LDS too small for the words: read them from global memory, 8 at a time
      const uint32_t* slab = pk + static_cast<size_t>(og + mrow) * Ww * 128 + lt;
      constexpr int U = 8;
      for (int mb = m0; mb < m1; mb += U) {
        uint32_t w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) w[u] = (mb + u < m1) ? slab[static_cast<size_t>(mb + u) * 128] : 0u;
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (mb + u < m1) word_of(w[u], act_of(mb + u));
      }
    }
  };
  // The output value of output o of matrix mi (lane j == 0) from its chain sums: reduce the 8
  // chains, add the tail, scale.
  auto finish = [&](int o, float facc, int32_t sum) {
    const int oo = o + ((KIND == kGate && mi == 1) ? nout : 0);
    float val = 0.0f;
    if (MODE == kFloat) {
      float s = facc;
      if (j == 0 && o < nout) {
        const float* yt = Y + ai * WL + 8 * LS;
        for (int t = 0; t < nt; ++t) {
          const int8_t wt = ptail[oo * 8 + t];
          if (wt > 0) s += yt[t];
          else if (wt < 0) s -= yt[t];
        }
      }
      val = s * pinv;
    } else if (j == 0 && o < nout) {
      int32_t s = sum;
      if (MODE == kFixed) s += LMG ? 128 * prowsum[oo] : e_rs;
      for (int t = 0; t < nt; ++t) s += static_cast<int32_t>(ptail[oo * 8 + t]) * CT[ai * 8 + t];
      val = (MODE == kFixed) ? static_cast<float>(s) * invfx : static_cast<float>(s) / (pscale * SA[ai]);
    }
    return val;
  };

  if constexpr (LMG) {
    // ---- lm_head: part p runs the block's groups p, p + KS, ... (slot gi); logits and keys
    unsigned long long best = 0ull;
    for (int gi = part, og = static_cast<int>(blockIdx.x) + part * static_cast<int>(gridDim.x); og < ngroups_out;
         gi += KS, og += KS * static_cast<int>(gridDim.x)) {
      float facc = 0.0f;
      int32_t hacc = 0, lacc = 0;
      gemv(og, gi, 0, Ww, facc, hacc, lacc);
      const int o = og * kGroup + ol;
      int32_t sum = 0;
      if (MODE == kFloat) {
        facc = hsum8_lanes(facc);
      } else {
        sum = isum8_lanes(MODE == kFixed ? hacc * 256 + lacc : hacc);  // one reduction of both planes
      }
      const float val = finish(o, facc, sum);
      if (j != 0 || o >= nout) continue;
      if (aout) aout[o] = val;
      const unsigned long long kk = amax_key(val, o);
      best = kk > best ? kk : best;
    }
    if (akeys) {  // one partial key per block, reduced by the consumer
      best = wave_max_u64(best);
      unsigned long long* r64 = reinterpret_cast<unsigned long long*>(red);
      if ((tid & 63) == 0) r64[tid >> 6] = best;
      __syncthreads();
      if (tid == 0) {
        unsigned long long b = r64[0];
        for (int w = 1; w < BS / 64; ++w) b = r64[w] > b ? r64[w] : b;
        akeys[blockIdx.x] = b;
      }
    }
    return;
  } else {
    // ---- one output group per block ----------------------------------------------------------
    const int og = static_cast<int>(blockIdx.x);
    float facc = 0.0f;
    int32_t hacc = 0, lacc = 0;
    if (KSPLIT) gemv(og, 0, part * Wc / KS, (part + 1) * Wc / KS, facc, hacc, lacc);
    else if (part == 0) gemv(og, 0, 0, Ww, facc, hacc, lacc);
    int32_t sum = 0;
    if (MODE == kFloat) {
      facc = hsum8_lanes(facc);
    } else {
      sum = isum8_lanes(MODE == kFixed ? hacc * 256 + lacc : hacc);  // one reduction of both planes
      if (KSPLIT) {  // the parts' partial sums meet in LDS, added by part 0
        int32_t* ps = reinterpret_cast<int32_t*>(vals);
        if (j == 0) ps[(part * NM + mi) * 16 + ol] = sum;
        __syncthreads();
        if (part == 0) {
          sum = ps[mi * 16 + ol];
          for (int p = 1; p < KS; ++p) sum += ps[(p * NM + mi) * 16 + ol];
        }
        __syncthreads();  // vals is reused below
      }
    }
    const int o = og * kGroup + ol;
    const float val = (part == 0) ? finish(o, facc, sum) : 0.0f;
    float v1 = 0.0f, v2 = 0.0f;
    if (NM > 1) {  // gather the other matrices' results for the same outputs
      if (part == 0 && j == 0) vals[mi * 16 + ol] = val;
      __syncthreads();
      v1 = vals[16 + ol];
      if (NM > 2) v2 = vals[32 + ol];
    }
    if (!epi) return;

    // ---- epilogues -------------------------------------------------------------------
    const int p = po;
    if (KIND == kIFG) {
      const bool tl = o >= (aH & ~7);  // sigmoid / swiglu over T*H = H elements
      float f = sigmoid_of(v1, tl);
      if (alb) f = __builtin_fmaf(1.0f - e_lb, f, e_lb);
      const float in = swiglu_of(val, 1.0f - f, tl);
      const float s = __builtin_fmaf(f, e_st, in);
      astate[o] = s;
      // silu of the recurrence output, the gate of the next kO's g_norm (one SIMD call of
      // H elements, rmsnorm_swishgate.cpp:24: the same tail rule as above)
      arecur[p] = silu_of(s, tl);
      agout[p] = v2;
      if (aout) aout[p] = src[0][p];  // layer 0: the embedding row becomes h
    } else if (KIND == kO || KIND == kDown) {
      aout[p] = e_hin + val;
    } else {  // kGate
      aout[p] = swiglu_of(val, v1, o >= (nout & ~7));
    }
  }
}

// Batch-1 layer kinds (kIFG, kO, kDown; kGate stays on k_decode) at the model widths (chain
// length Lc = 32 RC), with no barrier before the GEMV. A block is NM waves, wave mi holding
// matrix mi for the 8 outputs 8 blockIdx.x + ol (half of a 16-output slab group): lane 8 ol + j
// runs the reference's lane chain j of output ol. Every wave works on its own:
//  * it loads its lane segments of the input row, the stage-1 weight (kO: and silu of the
//    recurrence) and its matrix's BitLinear norm weight (lane 8c + s: segment s of chain c);
//    the pointers of these first loads are the leading kernel parameters, which the launch
//    preloads into scalar registers, so the loads do not wait for the argument block;
//  * it copies its own slab words (64 per word row; float: the fp4 slab, integer modes: the
//    2-bit slab) into its own LDS slice by DMA;
//  * it runs both norm chains from registers (a DPP row shift hands each running sum to the
//    next segment's lane), the same sums in the same order in every wave, and encodes its
//    activation row into its own LDS slice from registers: float y = (x * r2) * w; FixedQ510
//    the Q5.10 code split into a high and a biased low int8 plane (q = 256 h + l + 128);
//    Int8Absmax the int8 code at 127 / max|y| (the maximum reduced over the wave);
//  * it waits for its own DMA and runs its 64 chains: float as in-order fp32 FMAs over fp4
//    codes; the integer modes as v_dot4 sums (exact, so in any order) of the planes.
// Only the epilogue of the multi-matrix kinds meets in LDS (one barrier). Outputs, epilogues
// and the layer-0 token gather are k_decode's.
template <int MODE, int KIND, int RC>
struct DecfShape {
  static constexpr int NM = KindTraits<KIND>::NM;
  static constexpr int Lc = 32 * RC, LS = Lc + 4, WL = 8 * LS + 8;  // float rows
  static constexpr int LQ = Lc + 16;                                   // int8 plane rows (bytes)
  static constexpr int NW = (MODE == kFloat) ? 4 * RC : 2 * RC;        // slab words per chain
  // floats of a wave's activation area: float Y; integer: 2 planes, 8 tail codes, the scale
  static constexpr int ACT = (MODE == kFloat) ? WL : (16 * LQ) / 4 + 8 + 4;
  // kOp: + the natural row turned into the chain-transposed layout (8 rows of LS floats)
  static constexpr int TR = (KIND == kOp) ? 8 * LS : 0;
  static constexpr int SLICE = ACT + NW * 64 + TR;  // + the wave's words (+ the staging)
};

template <int MODE, int KIND, int RC>
__global__ __launch_bounds__(64 * KindTraits<KIND>::NM) void k_decf(const float* __restrict__ xin,
                                                                   const float* __restrict__ prew,
                                                                   const float* __restrict__ xg,
                                                                   const float* __restrict__ nwa,
                                                                   const float* __restrict__ nwb,
                                                                   const float* __restrict__ nwc, DecArgs a) {
  static_assert(KIND != kLM && KIND != kGate, "the lm_head and gate/up run k_decode");
  constexpr bool ST1 = KIND != kDown && KIND != kOp;  // a stage-1 norm before the BitLinear
  using S = DecfShape<MODE, KIND, RC>;
  constexpr int NM = S::NM, LS = S::LS, LQ = S::LQ, NW = S::NW, SLICE = S::SLICE;
  extern __shared__ float smem[];
  const int mi = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // wave = matrix
  const int lane = threadIdx.x & 63, ol = lane >> 3, j = lane & 7;
  float* Y = smem + mi * SLICE;                                          // float activations
  int8_t* Q = reinterpret_cast<int8_t*>(Y);                              // integer: [2][8][LQ] planes
  int32_t* CT = reinterpret_cast<int32_t*>(Q + 16 * LQ);                 // integer: [8] tail codes
  float* SA = reinterpret_cast<float*>(CT + 8);                          // Int8Absmax: the row scale
  uint32_t* WXw = reinterpret_cast<uint32_t*>(Y + S::ACT);
  float* vals = smem + NM * SLICE;  // [NM][8]
  const ProjDev& Pa = a.p[KIND == kIFG ? mi : 0];
  const Geom& g0 = a.p[0].g;
  const int gK = g0.K, nt = g0.ntail, gN = g0.N;
  const uint32_t* const pk = (MODE == kFloat) ? Pa.pk4 : Pa.pk;
  const int8_t* const ptail = Pa.tail;
  const float pinv = Pa.inv_scale_w;
  const float aeps = a.eps;
  const int nout = gN;
  const int W = 8 * S::Lc + 8;

  // layer 0: the token is the argmax over the previous lm_head's per-block keys (every wave
  // reduces all keys itself)
  const float* src0 = xin;
  if (KIND == kIFG && xin == nullptr) {
    const unsigned long long* keys = a.keys;
    const int nkeys = a.nkeys;
    unsigned long long best = 0ull;
    for (int e0 = lane; e0 < nkeys; e0 += 8 * 64) {
      unsigned long long k[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) k[u] = e0 + u * 64 < nkeys ? keys[e0 + u * 64] : 0ull;
#pragma unroll
      for (int u = 0; u < 8; ++u) best = k[u] > best ? k[u] : best;
    }
    best = wave_max_u64(best);
    int64_t tok = key_index(best);
    if (tok < 0 || tok >= a.vocab) tok = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.hist) {
      const int pos = *a.hist_pos;
      if (pos < a.hist_cap) a.hist[pos] = tok;
      *a.hist_pos = pos + 1;
    }
    src0 = a.embT + static_cast<size_t>(tok) * W;
  }
  // ---- this wave's lane segments (independent of the argument block except at layer 0) ------
  float4 xs[RC], ws[RC], gs[RC], ns[RC];
  float xt[8], wt[8], gt[8], nt8[8];
  if constexpr (KIND == kOp) {
    // the operator's row in natural order (K = 8 Lc: no tail): float4 q of lane l is
    // q = l + 64 k, elements 4q .. 4q+3 = step q / 2 of chains 4 (q % 2) .. + 3; through this
    // wave's staging rows into the lane segments
    float* T = Y + S::ACT + NW * 64;
    float4 nx[RC];
#pragma unroll
    for (int k = 0; k < RC; ++k) nx[k] = reinterpret_cast<const float4*>(src0)[lane + 64 * k];
#pragma unroll
    for (int k = 0; k < RC; ++k) {
      const int q = lane + 64 * k, t = q >> 1, j0 = 4 * (q & 1);
      T[(j0 + 0) * LS + t] = nx[k].x;
      T[(j0 + 1) * LS + t] = nx[k].y;
      T[(j0 + 2) * LS + t] = nx[k].z;
      T[(j0 + 3) * LS + t] = nx[k].w;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int c = 0; c < RC; ++c) xs[c] = reinterpret_cast<const float4*>(T + (lane >> 3) * LS + 4 * RC * (lane & 7))[c];
#pragma unroll
    for (int t = 0; t < 8; ++t) xt[t] = 0.0f;
  } else {
    load_seg<RC>(src0, lane, xs, xt);
  }
  if constexpr (ST1) load_seg<RC>(prew, lane, ws, wt);
  if constexpr (KIND == kO) load_seg<RC>(xg, lane, gs, gt);
  // kDown at RC >= 22: row, norm weight and slab words would be 3 RC > 63 loads in flight,
  // and the wave would stall issuing them until the first ones return; the norm weight's
  // loads are issued in the middle of the norm chain instead (they are needed after it)
  constexpr bool DEFER_NW = !ST1 && 3 * RC > 60;
  // kO at hidden 2048 and 2560: row, stage-1 weight, gate and norm weight are 4 (RC + 2)
  // float4 per lane, and issuing them took 1.4 us at RC = 10 before the first chain could
  // start; the norm weight's loads go into the middle of the first chain instead
  constexpr bool DEFER_NW1 = KIND == kO && RC >= 8;
  if constexpr (!DEFER_NW && !DEFER_NW1)
    load_seg<RC>(KIND == kIFG ? (mi == 0 ? nwa : (mi == 1 ? nwb : nwc)) : nwa, lane, ns, nt8);
  // these loads issue first: nothing below (the DMA addresses need argument-block fields) may
  // move above them
  __builtin_amdgcn_sched_barrier(0);
  // ---- this wave's slab words: rows m of the half group, 4 rows of 64 words per DMA ---------
  {
    const int og = static_cast<int>(blockIdx.x) >> 1, h = static_cast<int>(blockIdx.x) & 1;
    const uint32_t* sw = pk + static_cast<size_t>(og) * NW * 128 + 64 * h;
#pragma unroll
    for (int c = 0; c < (NW + 3) / 4; ++c) {
      const int m = 4 * c + (lane >> 4);
      if (m < NW)
        __builtin_amdgcn_global_load_lds(sw + m * 128 + 4 * (lane & 15), (lds_void*)(WXw + 4 * c * 64), 16, 0, 0);
    }
  }
  // ---- epilogue operands (lanes j == 0 of wave 0) ---------------------------------------------
  const int o = 8 * static_cast<int>(blockIdx.x) + ol;
  const bool epi = mi == 0 && j == 0 && o < nout;
  const int po = epi ? (KIND == kOp ? o : ((o < a.oK8) ? (o & 7) * a.oLc + (o >> 3) : 8 * a.oLc + (o - a.oK8))) : 0;
  float e_lb = 0.0f, e_st = 0.0f, e_hin = 0.0f;
  if (epi) {
    if (KIND == kIFG) {
      if (a.lb) e_lb = a.lb[o];
      e_st = a.state[o];
    }
    if (KIND == kO || KIND == kDown) e_hin = a.hin[po];
  }
  // FixedQ510: the output's 128 * rowsum term (lane j == 0 of every matrix), fetched now
  const int32_t e_rs = (MODE == kFixed && j == 0 && o < nout) ? 128 * Pa.rowsum[o] : 0;
  // ---- both norm chains in every wave, then this wave's activation row -----------------------
  if constexpr (ST1) {
    float ss1;
    if constexpr (DEFER_NW1) ss1 = seg_sumsq_at<RC, 3>(xs, xt, nt, [&] { load_seg<RC>(nwa, lane, ns, nt8); });
    else ss1 = seg_sumsq<RC>(xs, xt, nt);
    const float r1 = rstd_of(ss1, gK, aeps);
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      float4 x = xs[c];
      const float4 w = ws[c];
      x.x = (x.x * r1) * w.x; x.y = (x.y * r1) * w.y; x.z = (x.z * r1) * w.z; x.w = (x.w * r1) * w.w;
      if (KIND == kO) {
        const float4 sg = gs[c];
        x.x = x.x * sg.x; x.y = x.y * sg.y; x.z = x.z * sg.z; x.w = x.w * sg.w;
      }
      xs[c] = x;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xt[t] = (xt[t] * r1) * wt[t];
      if (KIND == kO) xt[t] = xt[t] * gt[t];
    }
  }
  float r2;
  if constexpr (DEFER_NW) r2 = rstd_of(seg_sumsq_at<RC, 3>(xs, xt, nt, [&] { load_seg<RC>(nwa, lane, ns, nt8); }), gK, aeps);
  else r2 = rstd_of(seg_sumsq<RC>(xs, xt, nt), gK, aeps);
  // the BitLinear input y = (x * r2) * w of the lane's segment (lane 8c + s: chain c, floats
  // [4 RC s, 4 RC (s + 1))) and of the tail
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const float4 x = xs[c], w = ns[c];
    xs[c] = make_float4((x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w);
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) xt[t] = (xt[t] * r2) * nt8[t];
  float sa = 0.0f;
  if constexpr (MODE == kFloat) {
    float4* yr = reinterpret_cast<float4*>(Y + (lane >> 3) * LS + 4 * RC * (lane & 7));
#pragma unroll
    for (int c = 0; c < RC; ++c) yr[c] = xs[c];
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < 8; ++t) Y[8 * LS + t] = xt[t];
    }
  } else {
    if constexpr (MODE == kInt8) {  // 127 / max|y| over the row (body and tail), any order
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < RC; ++c)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xs[c].x), fabsf(xs[c].y)), fmaxf(fabsf(xs[c].z), fabsf(xs[c].w))));
#pragma unroll
      for (int t = 0; t < 8; ++t) m = fmaxf(m, fabsf(xt[t]));
      m = wave_max(m);
      sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
    }
    // the lane's 4 RC codes as RC words per plane: row (lane >> 3), bytes [4 RC s, 4 RC (s + 1))
    uint32_t* qh = reinterpret_cast<uint32_t*>(Q + (lane >> 3) * LQ + 4 * RC * (lane & 7));
    uint32_t* ql = reinterpret_cast<uint32_t*>(Q + 8 * LQ + (lane >> 3) * LQ + 4 * RC * (lane & 7));
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const float y[4] = {xs[c].x, xs[c].y, xs[c].z, xs[c].w};
      int32_t cd[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) cd[u] = (MODE == kFixed) ? q510_body(y[u], a.qs) : q8_of(y[u], sa);
      if constexpr (MODE == kFixed) {
        uint32_t hi, lo;
        pack_split4(cd, hi, lo);
        qh[c] = hi;
        ql[c] = lo;
      } else {
        qh[c] = pack_low4(cd);
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < 8; ++t) CT[t] = (t < nt) ? ((MODE == kFixed) ? q510_tail(xt[t], a.qs) : q8_of(xt[t], sa)) : 0;
    }
  }
  // the wave's own DMA and LDS writes are complete before any of its lanes reads them
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  float val = 0.0f;
  int32_t stot = 0;  // integer modes: the output's exact accumulator
  if constexpr (MODE == kFloat) {
    // ---- GEMV: chunks of 4 fp4 words, the reads of chunk c + 1 issued before chunk c's FMAs
    float facc = 0.0f;
    const uint32_t* wl = WXw + lane;
    const float4* yl = reinterpret_cast<const float4*>(Y + j * LS);
    uint32_t wa[4];
    float4 xa[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      wa[u] = wl[u * 64];
      xa[2 * u] = yl[2 * u];
      xa[2 * u + 1] = yl[2 * u + 1];
    }
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      uint32_t wb[4];
      float4 xb[8];
      if (c + 1 < RC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int m = 4 * (c + 1) + u;
          wb[u] = wl[m * 64];
          xb[2 * u] = yl[2 * m];
          xb[2 * u + 1] = yl[2 * m + 1];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) facc = word_dot_f4(wa[u], xa[2 * u], xa[2 * u + 1], facc);
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < RC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          wa[u] = wb[u];
          xa[2 * u] = xb[2 * u];
          xa[2 * u + 1] = xb[2 * u + 1];
        }
      }
    }
    facc = hsum8_lanes(facc);  // lane j == 0: the 8 chains of output ol in the hsum_ps order
    if (j == 0 && o < nout) {
      float s = facc;
      const float* yt = Y + 8 * LS;
      for (int t = 0; t < nt; ++t) {
        const int8_t w8 = ptail[o * 8 + t];
        if (w8 > 0) s += yt[t];
        else if (w8 < 0) s -= yt[t];
      }
      val = s * pinv;
    }
  } else {
    // ---- GEMV: 2-bit words two at a time (32 codes), v_dot4 on each plane; two independent
    // accumulators per plane (exact integer sums), the next pair's reads issued first
    const uint32_t* wl = WXw + lane;
    const uint4* qh = reinterpret_cast<const uint4*>(Q + j * LQ);
    const uint4* ql = reinterpret_cast<const uint4*>(Q + 8 * LQ + j * LQ);
    int32_t h0 = 0, h1 = 0, l0 = 0, l1 = 0;
    auto pair = [&](uint32_t wv, const uint4& xh, const uint4& xl, int32_t& hh, int32_t& ll) {
      const uint32_t w0 = w4_i8(wv, 0), w1 = w4_i8(wv, 1), w2 = w4_i8(wv, 2), w3 = w4_i8(wv, 3);
      hh = dot4(w3, xh.w, dot4(w2, xh.z, dot4(w1, xh.y, dot4(w0, xh.x, hh))));
      if (MODE == kFixed) ll = dot4(w3, xl.w, dot4(w2, xl.z, dot4(w1, xl.y, dot4(w0, xl.x, ll))));
    };
    uint32_t wa[2];
    uint4 ha[2], la[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      wa[u] = wl[u * 64];
      ha[u] = qh[u];
      if (MODE == kFixed) la[u] = ql[u];
    }
#pragma unroll
    for (int c = 0; c < RC; ++c) {  // NW = 2 RC words: RC pairs
      uint32_t wb[2];
      uint4 hb[2], lb[2];
      if (c + 1 < RC) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int m = 2 * (c + 1) + u;
          wb[u] = wl[m * 64];
          hb[u] = qh[m];
          if (MODE == kFixed) lb[u] = ql[m];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      pair(wa[0], ha[0], la[0], h0, l0);
      pair(wa[1], ha[1], la[1], h1, l1);
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < RC) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          wa[u] = wb[u];
          ha[u] = hb[u];
          if (MODE == kFixed) la[u] = lb[u];
        }
      }
    }
    // both planes in one reduction (per-lane partials stay far inside int32: |hi sum| <= 128 Lc)
    const int32_t sum = isum8_lanes(MODE == kFixed ? (h0 + h1) * 256 + (l0 + l1) : h0 + h1);
    if (j == 0 && o < nout) {
      int32_t s = sum;
      if (MODE == kFixed) s += e_rs;
      for (int t = 0; t < nt; ++t) s += static_cast<int32_t>(ptail[o * 8 + t]) * CT[t];
      stot = s;
      val = (MODE == kFixed) ? static_cast<float>(s) * a.inv_fixed[KIND == kIFG ? mi : 0]
                             : static_cast<float>(s) / (Pa.scale_w * sa);
    }
  }
  float v1 = 0.0f, v2 = 0.0f;
  if constexpr (NM > 1) {  // the other matrices' results for the same outputs
    if (j == 0) vals[mi * 8 + ol] = val;
    __syncthreads();
    v1 = vals[8 + ol];
    if (NM > 2) v2 = vals[16 + ol];
  }
  if (!epi) return;
  const int p = po;
  if (KIND == kIFG) {
    const int aH = a.H;
    const bool tl = o >= (aH & ~7);
    float f = sigmoid_of(v1, tl);
    if (a.lb) f = __builtin_fmaf(1.0f - e_lb, f, e_lb);
    const float in = swiglu_of(val, 1.0f - f, tl);
    const float s = __builtin_fmaf(f, e_st, in);
    a.state[o] = s;
    a.recur[p] = silu_of(s, tl);
    a.gout[p] = v2;
    if (a.out) a.out[p] = src0[p];  // layer 0: the embedding row becomes h
  } else if (KIND == kOp) {
    a.out[p] = val;
    if (MODE != kFloat && a.acc) a.acc[p] = stot;
  } else {  // kO, kDown
    a.out[p] = e_hin + val;
  }
}

template <int MODE, int KIND, int RC>
hipError_t decf_rc(const DecArgs& a, hipStream_t s) {
  using S = DecfShape<MODE, KIND, RC>;
  const size_t lds = (static_cast<size_t>(S::NM) * S::SLICE + S::NM * 8) * sizeof(float);
  const int grid = (a.p[0].g.N + 7) / 8;
  const float* prew = (KIND == kDown || KIND == kOp) ? nullptr : a.pre_w;
  const float* xg = (KIND == kO) ? a.x2 : nullptr;
  return launch_k(k_decf<MODE, KIND, RC>, grid, 64 * S::NM, lds, s, a.x, prew, xg, a.p[0].normwT, a.p[1].normwT,
                  a.p[2].normwT, a);
}

// k_decf for a layer kind when every matrix has its slab (float: the fp4 one) and a chain-
// transposed norm weight and the width is a model width; hipErrorNotSupported (nothing
// launched) otherwise. Where it runs, by measurement (per-launch microseconds, k_decode ->
// k_decf):
//  * float: o and down at every width; i/f/g up to hidden 2048 (at 2560 its three waves' own
//    loads of three 10 KB vectors over 320 blocks cost more than k_decode's barriers: 9.3 ->
//    10.1 us);
//  * FixedQ510 and Int8Absmax: i/f/g and o up to hidden 2048 (370M FixedQ510 i/f/g 5.9 -> 4.8,
//    o 4.2 -> 3.8 us);
//  * gate/up never: with 2I outputs it takes 352 to 864 blocks, and their own loads cost more
//    than the barriers saved (float 370M 4.9 -> 5.0, 2.7B 10.0 -> 13.7 us).
template <int MODE, int KIND>
hipError_t decf_kind(const DecArgs& a, hipStream_t s) {
  if constexpr (KIND == kGate || KIND == kLM) {
    return hipErrorNotSupported;
  } else {
    constexpr int NP = (KIND == kIFG) ? 3 : 1;
    for (int z = 0; z < NP; ++z)
      if (!((MODE == kFloat) ? a.p[z].pk4 : a.p[z].pk) || !a.p[z].normwT) return hipErrorNotSupported;
    const int Lc = a.p[0].g.Lc;
    if (Lc % 32 != 0 || a.p[0].g.Wc * 2 != Lc / 8) return hipErrorNotSupported;
    if (MODE == kFloat && KIND == kIFG && Lc > 256) return hipErrorNotSupported;
    // the integer modes: i/f/g and o up to hidden 2048 only; down and the 2560-wide kinds keep
    // k_decode, whose 2 to 4 parts per block split each chain's words (370M FixedQ510 down
    // 4.77 -> 4.94 us, 2.7B i/f/g 9.1 -> 10.1, o 6.5 -> 7.0, down 8.3 -> 10.8 on k_decf)
    if constexpr (KIND == kOp) {
      // one row of the operator API: the natural row must fill the chains exactly
      if (a.p[0].g.ntail != 0 || a.p[0].g.nb != Lc) return hipErrorNotSupported;
      switch (Lc / 32) {
        case 4: return decf_rc<MODE, KIND, 4>(a, s);
        case 8: return decf_rc<MODE, KIND, 8>(a, s);
        case 10: return decf_rc<MODE, KIND, 10>(a, s);
        case 11: return decf_rc<MODE, KIND, 11>(a, s);
        case 22: return decf_rc<MODE, KIND, 22>(a, s);
        case 27: return decf_rc<MODE, KIND, 27>(a, s);
        default: return hipErrorNotSupported;
      }
    }
    if (MODE != kFloat && (KIND == kDown || Lc > 256)) return hipErrorNotSupported;
    if constexpr (KIND == kDown) {
      switch (Lc / 32) {
        case 11: return decf_rc<MODE, KIND, 11>(a, s);
        case 22: return decf_rc<MODE, KIND, 22>(a, s);
        case 27: return decf_rc<MODE, KIND, 27>(a, s);
        default: return hipErrorNotSupported;
      }
    } else {
      switch (Lc / 32) {
        case 4: return decf_rc<MODE, KIND, 4>(a, s);
        case 8: return decf_rc<MODE, KIND, 8>(a, s);
        case 10: return decf_rc<MODE, KIND, 10>(a, s);
        default: return hipErrorNotSupported;
      }
    }
  }
}

// Parts per block (see k_decode): integer modes split each chain's words over 2 (i/f/g,
// gate/up) or 4 (o, down) parts; float keeps one part, except that the lm_head runs its groups
// side by side in every mode.
template <int MODE, int KIND>
constexpr int kParts = (MODE == kFloat) ? 1 : ((KIND == kO || KIND == kDown) ? 4 : 2);

constexpr int nv_for(int F4, int BS) { return F4 <= 2 * BS ? 2 : (F4 <= 4 * BS ? 4 : (F4 <= 8 * BS ? 8 : 16)); }

template <int MODE, int KIND, int KS, int RC, bool W4>
hipError_t dec_rc(const DecArgs& a, size_t lds, int grid, hipStream_t s) {
  constexpr int BS = kBlock * KindTraits<KIND>::NM * KS;
  constexpr int F4 = (8 * 32 * RC + 8) / 4;  // float4s of a chain-transposed vector
  static_assert(F4 <= 16 * BS, "row too long for the block layout");
  return launch_k(k_decode<MODE, KIND, nv_for(F4, BS), KS, RC, W4>, grid, BS, lds, s, a);
}

template <int MODE, int KIND, int KS, bool W4>
hipError_t dec_ks(const DecArgs& a, size_t lds, int grid, hipStream_t s) {
  constexpr int BS = kBlock * KindTraits<KIND>::NM * KS;
  const int Lc = a.p[0].g.Lc;
  if (Lc % 32 == 0) {  // register chains at the model widths: H 1024/2048/2560, I 2816/5632/6912
    if constexpr (KIND == kDown) {
      switch (Lc / 32) {
        case 11: return dec_rc<MODE, KIND, KS, 11, W4>(a, lds, grid, s);
        case 22: return dec_rc<MODE, KIND, KS, 22, W4>(a, lds, grid, s);
        case 27: return dec_rc<MODE, KIND, KS, 27, W4>(a, lds, grid, s);
        default: break;
      }
    } else {
      switch (Lc / 32) {
        case 4: return dec_rc<MODE, KIND, KS, 4, W4>(a, lds, grid, s);
        case 8: return dec_rc<MODE, KIND, KS, 8, W4>(a, lds, grid, s);
        case 10: return dec_rc<MODE, KIND, KS, 10, W4>(a, lds, grid, s);
        default: break;
      }
    }
  }
  const int F4 = (8 * Lc + 8) / 4;
  if (F4 <= 2 * BS) return launch_k(k_decode<MODE, KIND, 2, KS, 0, W4>, grid, BS, lds, s, a);
  if (F4 <= 4 * BS) return launch_k(k_decode<MODE, KIND, 4, KS, 0, W4>, grid, BS, lds, s, a);
  if (F4 <= 8 * BS) return launch_k(k_decode<MODE, KIND, 8, KS, 0, W4>, grid, BS, lds, s, a);
  if (F4 <= 16 * BS) return launch_k(k_decode<MODE, KIND, 16, KS, 0, W4>, grid, BS, lds, s, a);
  return hipErrorInvalidValue;
}

template <int MODE, int KIND>
hipError_t dec_kind(const DecArgs& a, size_t lds, int grid, bool w4, hipStream_t s) {
  if constexpr (KIND == kLM) {
    switch (a.wgroups) {  // one part per group held in LDS, at most 4
      case 0:
      case 1: return dec_ks<MODE, KIND, 1, false>(a, lds, grid, s);
      case 2: return dec_ks<MODE, KIND, 2, false>(a, lds, grid, s);
      case 3: return dec_ks<MODE, KIND, 3, false>(a, lds, grid, s);
      default: return dec_ks<MODE, KIND, 4, false>(a, lds, grid, s);
    }
  } else if constexpr (MODE == kFloat) {
    if (w4) return dec_ks<MODE, KIND, kParts<MODE, KIND>, true>(a, lds, grid, s);
    return dec_ks<MODE, KIND, kParts<MODE, KIND>, false>(a, lds, grid, s);
  } else {
    return dec_ks<MODE, KIND, kParts<MODE, KIND>, false>(a, lds, grid, s);
  }
}

// MMF_DECF=0 keeps every layer kind on k_decode (for comparisons); default on.
bool decf_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("MMF_DECF");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <int MODE>
hipError_t dec_mode(DecKind kind, const DecArgs& a, hipStream_t s) {
  if (kind == kOp) return decf_kind<MODE, kOp>(a, s);
  if (kind != kLM && decf_enabled()) {
    hipError_t e = hipErrorNotSupported;
    switch (kind) {
      case kIFG: e = decf_kind<MODE, kIFG>(a, s); break;
      case kO: e = decf_kind<MODE, kO>(a, s); break;
      case kGate: e = decf_kind<MODE, kGate>(a, s); break;
      default: e = decf_kind<MODE, kDown>(a, s); break;
    }
    if (e != hipErrorNotSupported) return e;
  }
  const Geom& g = a.p[0].g;
  const int Lc = g.Lc;
  const int na = kind == kIFG ? 3 : 1;
  const size_t WL = 8 * static_cast<size_t>((Lc + 31) / 32 * 32 + 4) + 8, LQ = Lc + 16;
  // X, S, red[32], vals[4 parts x 48]: sized for the most parts any kind takes
  size_t lds = (2 * WL + 32 + 4 * 48) * sizeof(float);
  lds += (MODE == kFloat) ? na * WL * sizeof(float) : na * (16 * LQ + 8 * sizeof(int32_t)) + 4 * sizeof(float);
  const int nout = (kind == kGate) ? g.N / 2 : g.N;
  int grid = (nout + kGroup - 1) / kGroup;
  if (kind == kLM) grid = lm_blocks(grid, g.K);
  // all weight words of the block's output groups go to LDS at entry when they fit (the
  // lm_head's blocks stride over several groups)
  DecArgs b = a;
  b.wgroups = 0;
  const int nm = kind == kIFG ? 3 : (kind == kGate ? 2 : 1);
  const int G = (kind == kLM) ? (((nout + kGroup - 1) / kGroup) + grid - 1) / grid : 1;
  const size_t wx = static_cast<size_t>(nm) * G * g.Wc * 128 * sizeof(uint32_t);
  // float layer GEMVs: the fp4 slab (twice the words) when every matrix has one and its words
  // fit in LDS beside the rest; otherwise the 2-bit slab
  // (gate/up keeps the 2-bit slab: its four GEMV waves per CU are bound by the LDS reads of the
  // activations, not by the code conversion -- 4.88 us per 370M launch either way)
  bool w4 = MODE == kFloat && (kind == kIFG || kind == kO || kind == kDown);
  for (int z = 0; z < (kind == kIFG ? 3 : 1); ++z) w4 = w4 && a.p[z].pk4 != nullptr;
  w4 = w4 && lds + 2 * wx <= static_cast<size_t>(lds_limit());
  if (w4) {
    b.wgroups = G;
    lds += 2 * wx;
  } else if (lds + wx <= static_cast<size_t>(lds_limit())) {
    b.wgroups = G;
    lds += wx;
  }
  switch (kind) {
    case kIFG: return dec_kind<MODE, kIFG>(b, lds, grid, w4, s);
    case kO: return dec_kind<MODE, kO>(b, lds, grid, w4, s);
    case kGate: return dec_kind<MODE, kGate>(b, lds, grid, w4, s);
    case kDown: return dec_kind<MODE, kDown>(b, lds, grid, w4, s);
    default: return dec_kind<MODE, kLM>(b, lds, grid, false, s);
  }
}

// Chain-transposed copy of rows: out[r][act_pos(k)] = x[r][k], zero padding.
__global__ void k_to_chain(const float* __restrict__ x, float* __restrict__ out, int K, int Lc) {
  const int K8 = K & ~7, nb = K8 / 8, W = 8 * Lc + 8;
  const float* xr = x + static_cast<size_t>(blockIdx.x) * K;
  float* orow = out + static_cast<size_t>(blockIdx.x) * W;
  for (int p = threadIdx.x; p < W; p += blockDim.x) {
    float v = 0.0f;
    if (p < 8 * Lc) {
      const int jj = p / Lc, t = p - jj * Lc;
      if (t < nb) v = xr[jj + 8 * t];
    } else if (p - 8 * Lc < K - K8) {
      v = xr[K8 + p - 8 * Lc];
    }
    orow[p] = v;
  }
}

}  // namespace

hipError_t launch_decode(DecKind kind, Mode mode, const DecArgs& a, hipStream_t s) {
  switch (mode) {
    case kFloat: return dec_mode<kFloat>(kind, a, s);
    case kFixed: return dec_mode<kFixed>(kind, a, s);
    default: return dec_mode<kInt8>(kind, a, s);
  }
}

hipError_t launch_to_chain(const float* x, float* out, int rows, int K, int Lc, hipStream_t s) {
  k_to_chain<<<rows, 256, 0, s>>>(x, out, K, Lc);
  return hipGetLastError();
}

}  // namespace mmf
