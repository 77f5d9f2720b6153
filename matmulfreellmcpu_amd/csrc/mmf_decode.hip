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
// A block is 16 outputs x 8 chains; thread (ol, j) sums chain j of output og*16+ol, which
// is the reference's AVX2 lane j.
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

// MMF_PHASE_TRACE (off by default): thread 0 of block 0 records wall_clock64() at the phase
// boundaries of the decode kernel into mmf_phase_trace[kind][0..7]; thread 0 of the last
// block records its entry and exit in [kind][8], [kind][9]. Read with mmf_debug_phase_trace.
#ifdef MMF_PHASE_TRACE
__device__ unsigned long long mmf_phase_trace[5][10];
#define MMF_MARK(k, i)                                                                  \
  do {                                                                                  \
    if (blockIdx.x == 0 && threadIdx.x == 0) mmf_phase_trace[k][i] = wall_clock64();    \
  } while (0)
#define MMF_SPAN(k, first)                                                              \
  do {                                                                                  \
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0)                                \
      mmf_phase_trace[k][(first) ? 8 : 9] = wall_clock64();                             \
  } while (0)
#else
#define MMF_MARK(k, i) do {} while (0)
#define MMF_SPAN(k, first) do {} while (0)
#endif

namespace mmf {

namespace {

template <int KIND> struct KindTraits;
// NM matrices (one wave pair each), NA activation vectors, NP prologue source vectors
template <> struct KindTraits<kIFG> { static constexpr int NM = 3, NA = 3, NP = 5; };
template <> struct KindTraits<kO> { static constexpr int NM = 1, NA = 1, NP = 4; };
template <> struct KindTraits<kGate> { static constexpr int NM = 2, NA = 1, NP = 3; };
template <> struct KindTraits<kDown> { static constexpr int NM = 1, NA = 1, NP = 2; };
template <> struct KindTraits<kLM> { static constexpr int NM = 1, NA = 1, NP = 3; };

constexpr int kPF = 16;  // weight words prefetched at entry

template <int MODE, int KIND, int NV>
__global__ __launch_bounds__(kBlock * KindTraits<KIND>::NM) void k_decode(DecArgs a) {
  constexpr int NM = KindTraits<KIND>::NM, NA = KindTraits<KIND>::NA, NP = KindTraits<KIND>::NP;
  constexpr int BS = kBlock * NM;
  extern __shared__ float smem[];
  const Geom& g = a.p[0].g;
  const int Lc = g.Lc, nt = g.ntail, Wc = g.Wc;
  const int W = 8 * Lc + 8;  // floats of a chain-transposed vector in global memory
  const int W4 = W / 4;
  // LDS copies pad each chain row by 16 bytes so that the 8 chain lanes of a wave read
  // different banks: float rows LS floats apart, int8 plane rows LQ bytes apart.
  const int L32 = (Lc + 31) / 32 * 32;  // rows zero-filled to whole 32-value chain batches
  const int LS = L32 + 4, WL = 8 * LS + 8, LQ = Lc + 16;
  const int tid = threadIdx.x, mi = tid >> 7, lt = tid & 127, ol = lt >> 3, j = lt & 7;
  const int ai = (NA > 1) ? mi : 0;  // this thread's activation vector
  const int nout = (KIND == kGate) ? g.N / 2 : g.N;
  const int ngroups_out = (nout + kGroup - 1) / kGroup;
  const ProjDev& P = a.p[KIND == kIFG ? mi : 0];

  float* X = smem;           // [WL] input row
  float* S = X + WL;         // [WL] kO: silu(recur)
  float* red = S + WL;       // [16]
  float* vals = red + 16;    // [NM][16] per-matrix results of the block's outputs
  float* Y = vals + 48;      // float: NA x [WL]; int: NA x 2 planes x [8 LQ] bytes + tails + scales
  int8_t* Q = reinterpret_cast<int8_t*>(Y);
  int32_t* CT = reinterpret_cast<int32_t*>(Q + NA * 16 * LQ);
  float* SA = reinterpret_cast<float*>(CT + NA * 8);

  // ---- entry: issue every load that does not depend on the prologue --------------------
  MMF_MARK(KIND, 0);
  MMF_SPAN(KIND, true);
  int og = blockIdx.x;
  const int o0 = og * kGroup + ol;
  const int mrow = (KIND == kGate && mi == 1) ? g.ngroups / 2 : 0;  // gate: the up half
  uint32_t wpf[kPF];
  {
    const uint32_t* s0 = P.pk + static_cast<size_t>(og + mrow) * Wc * 128 + ol * 8 + j;
#pragma unroll
    for (int u = 0; u < kPF; ++u) wpf[u] = (u < Wc && og < ngroups_out) ? s0[static_cast<size_t>(u) * 128] : 0u;
  }
  const bool epi = (mi == 0 && j == 0 && og < ngroups_out && o0 < nout);
  const int po = epi ? ((o0 < a.oK8) ? (o0 & 7) * a.oLc + (o0 >> 3) : 8 * a.oLc + (o0 - a.oK8)) : 0;
  float e_lb = 0.0f, e_st = 0.0f, e_hin = 0.0f;
  if (epi) {
    if (KIND == kIFG) {
      if (a.lb) e_lb = a.lb[o0];
      e_st = a.state[o0];
    }
    if (KIND == kO || KIND == kDown) e_hin = a.hin[po];
  }

  // layer 0: the token is the argmax over the previous lm_head's per-block keys
  int64_t tok = 0;
  if (KIND == kIFG && a.x == nullptr) {
    unsigned long long best = 0ull;
    for (int e = tid; e < a.nkeys; e += BS) {
      const unsigned long long k = a.keys[e];
      best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
      const unsigned long long other = __shfl_xor(best, off);
      best = other > best ? other : best;
    }
    unsigned long long* r64 = reinterpret_cast<unsigned long long*>(vals);
    if ((tid & 63) == 0) r64[tid >> 6] = best;
    __syncthreads();
    best = r64[0];
    for (int w = 1; w < BS / 64; ++w) best = r64[w] > best ? r64[w] : best;
    tok = key_index(best);
    if (tok < 0 || tok >= a.vocab) tok = 0;
    if (blockIdx.x == 0 && tid == 0 && a.hist) {
      const int pos = *a.hist_pos;
      if (pos < a.hist_cap) a.hist[pos] = tok;
      *a.hist_pos = pos + 1;
    }
  }

  // prologue sources (all chain-transposed, zero-padded, W floats):
  //   0: input row   1: stage-1 weight (kO: recur)   then the BitLinear norm weights
  const float* src[NP];
  src[0] = (KIND == kIFG && a.x == nullptr) ? a.embT + static_cast<size_t>(tok) * W : a.x;
  if (KIND == kIFG) { src[1] = a.pre_w; src[2] = a.p[0].normwT; src[3] = a.p[1].normwT; src[4] = a.p[2].normwT; }
  if (KIND == kO) { src[1] = a.x2; src[2] = a.pre_w; src[3] = a.p[0].normwT; }
  if (KIND == kGate || KIND == kLM) { src[1] = a.pre_w; src[2] = a.p[0].normwT; }
  if (KIND == kDown) { src[1] = a.p[0].normwT; }
  float4 v[NP][NV];
#pragma unroll
  for (int s = 0; s < NP; ++s)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + i * BS;
      v[s][i] = (e < W4) ? reinterpret_cast<const float4*>(src[s])[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  // LDS float4 index of each of this thread's global float4s
  int li[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int p = 4 * (tid + i * BS);
    const int jj = p / Lc;
    li[i] = (p < 8 * Lc) ? (jj * LS + (p - jj * Lc)) / 4 : (8 * LS + (p - 8 * Lc)) / 4;
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + i * BS;
    if (e < W4) {
      reinterpret_cast<float4*>(X)[li[i]] = v[0][i];
      if (KIND == kO) reinterpret_cast<float4*>(S)[li[i]] = v[1][i];
    }
  }
  for (int z = tid; z < 8 * (L32 - Lc); z += BS) {  // zeros past Lc in each row
    const int jj = z / (L32 - Lc);
    X[jj * LS + Lc + (z - jj * (L32 - Lc))] = 0.0f;
  }
  __syncthreads();
  MMF_MARK(KIND, 1);

  // ---- stage 1: the kernel's own pre-norm -------------------------------------------------
  if (KIND != kDown) {
    chain_begin(X, Lc, LS, red);
    if (KIND == kO && tid >= 64) {
      // silu(recur) on wave 1 while wave 0 runs the chains (one SIMD call of H elements,
      // rmsnorm_swishgate.cpp:24: tail elements sit after the 8 rows)
      const int WL4 = WL / 4;
      for (int e = tid - 64; e < WL4; e += BS - 64) {
        float4 r = reinterpret_cast<float4*>(S)[e];
        const bool tl = 4 * e >= 8 * LS;
        r.x = silu_of(r.x, tl); r.y = silu_of(r.y, tl); r.z = silu_of(r.z, tl); r.w = silu_of(r.w, tl);
        reinterpret_cast<float4*>(S)[e] = r;
      }
    }
    __syncthreads();
    const float r1 = rstd_of(chain_end(X, LS, nt, red), g.K, a.eps);
    constexpr int PW = (KIND == kO) ? 2 : 1;  // which source holds the stage-1 weight
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + i * BS;
      if (e < W4) {
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
  // ---- stage 2: BitLinear RMSNorm, activation encoding ------------------------------------
  MMF_MARK(KIND, 2);
  chain_begin(X, Lc, LS, red);
  __syncthreads();
  const float r2 = rstd_of(chain_end(X, LS, nt, red), g.K, a.eps);
  MMF_MARK(KIND, 3);
  constexpr int NW0 = NP - NA;  // first norm-weight source
#pragma unroll
  for (int aa = 0; aa < NA; ++aa) {
    if (MODE == kFloat) {
      float4* yo = reinterpret_cast<float4*>(Y + aa * WL);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = tid + i * BS;
        if (e < W4) {
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
          if (e < W4) {
            const float4 x = reinterpret_cast<float4*>(X)[li[i]];
            const float4 w = v[NW0 + aa][i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf((x.x * r2) * w.x), fabsf((x.y * r2) * w.y)),
                               fmaxf(fabsf((x.z * r2) * w.z), fabsf((x.w * r2) * w.w))));
          }
        }
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
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
        if (e < W4) {
          const float4 x = reinterpret_cast<float4*>(X)[li[i]];
          const float4 w = v[NW0 + aa][i];
          const float y[4] = {(x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w};
          if (4 * e < 8 * Lc) {
            uint32_t hi = 0, lo = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (MODE == kFixed) {
                const int32_t c = q510_body(y[u], a.qs);
                hi |= static_cast<uint32_t>((c >> 8) & 0xFF) << (8 * u);
                lo |= static_cast<uint32_t>(((c & 0xFF) - 128) & 0xFF) << (8 * u);
              } else {
                hi |= static_cast<uint32_t>(q8_of(y[u], sa) & 0xFF) << (8 * u);
              }
            }
            const int jj = (4 * e) / Lc, qp = jj * LQ + (4 * e - jj * Lc);  // byte position
            *reinterpret_cast<uint32_t*>(q + qp) = hi;
            if (MODE == kFixed) *reinterpret_cast<uint32_t*>(q + 8 * LQ + qp) = lo;
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int t = 4 * e - 8 * Lc + u;
              CT[aa * 8 + t] = (t < nt) ? ((MODE == kFixed) ? q510_tail(y[u], a.qs) : q8_of(y[u], sa)) : 0;
            }
          }
        }
      }
      if (MODE == kInt8) __syncthreads();  // red[8..] reused by the next vector's max
    }
  }
  __syncthreads();

  // ---- GEMV: each thread one chain of one matrix --------------------------------------------
  MMF_MARK(KIND, 4);
  unsigned long long best = 0ull;
  for (; og < ngroups_out; og += gridDim.x) {
    const uint32_t* slab = P.pk + static_cast<size_t>(og + mrow) * Wc * 128 + ol * 8 + j;
    if (og != static_cast<int>(blockIdx.x)) {  // later groups (kLM grid-stride): reload
#pragma unroll
      for (int u = 0; u < kPF; ++u) wpf[u] = (u < Wc) ? slab[static_cast<size_t>(u) * 128] : 0u;
    }
    float facc = 0.0f;
    int32_t hacc = 0, lacc = 0;
    auto word = [&](uint32_t w, int m) {
      if (MODE == kFloat) {
        const float4* yl = reinterpret_cast<const float4*>(Y + ai * WL + j * LS + 16 * m);
        const float4 y0 = yl[0], y1 = yl[1], y2 = yl[2], y3 = yl[3];
        const float y[16] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w,
                             y2.x, y2.y, y2.z, y2.w, y3.x, y3.y, y3.z, y3.w};
#pragma unroll
        for (int t = 0; t < 16; ++t) facc = __builtin_fmaf(y[t], code_f(w, t), facc);
      } else {
        const int8_t* ql = Q + ai * 16 * LQ + j * LQ + 16 * m;
        const uint4 h = *reinterpret_cast<const uint4*>(ql);
        const uint32_t w0 = w4_i8(w, 0), w1 = w4_i8(w, 1), w2 = w4_i8(w, 2), w3 = w4_i8(w, 3);
        hacc = dot4(w3, h.w, dot4(w2, h.z, dot4(w1, h.y, dot4(w0, h.x, hacc))));
        if (MODE == kFixed) {
          const uint4 l = *reinterpret_cast<const uint4*>(ql + 8 * LQ);
          lacc = dot4(w3, l.w, dot4(w2, l.z, dot4(w1, l.y, dot4(w0, l.x, lacc))));
        }
      }
    };
#pragma unroll
    for (int u = 0; u < kPF; ++u)
      if (u < Wc) word(wpf[u], u);
    constexpr int U = 8;
    for (int m0 = kPF; m0 < Wc; m0 += U) {
      uint32_t w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) w[u] = (m0 + u < Wc) ? slab[static_cast<size_t>(m0 + u) * 128] : 0u;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (m0 + u < Wc) word(w[u], m0 + u);
    }

    // reduce the 8 chains, add the tail, scale
    MMF_MARK(KIND, 5);
    const int o = og * kGroup + ol;
    const int oo = o + ((KIND == kGate && mi == 1) ? nout : 0);
    float val = 0.0f;
    if (MODE == kFloat) {
      float s = hsum8_lanes(facc);
      if (j == 0 && o < nout) {
        const float* yt = Y + ai * WL + 8 * LS;
        for (int t = 0; t < nt; ++t) {
          const int8_t wt = P.tail[oo * 8 + t];
          if (wt > 0) s += yt[t];
          else if (wt < 0) s -= yt[t];
        }
      }
      val = s * P.inv_scale_w;
    } else {
      int32_t s = isum8_lanes(hacc);
      if (MODE == kFixed) s = s * 256 + isum8_lanes(lacc);
      if (j == 0 && o < nout) {
        if (MODE == kFixed) s += 128 * P.rowsum[oo];
        for (int t = 0; t < nt; ++t) s += static_cast<int32_t>(P.tail[oo * 8 + t]) * CT[ai * 8 + t];
        val = (MODE == kFixed) ? static_cast<float>(s) * a.inv_fixed[KIND == kIFG ? mi : 0]
                               : static_cast<float>(s) / (P.scale_w * SA[ai]);
      }
    }
    float v1 = 0.0f, v2 = 0.0f;
    if (NM > 1) {  // gather the other matrices' results for the same outputs
      if (j == 0) vals[mi * 16 + ol] = val;
      __syncthreads();
      v1 = vals[16 + ol];
      if (NM > 2) v2 = vals[32 + ol];
      __syncthreads();
    }
    if (mi != 0 || j != 0 || o >= nout) continue;

    // ---- epilogues -------------------------------------------------------------------
    const int p = (og == static_cast<int>(blockIdx.x))
                      ? po
                      : ((o < a.oK8) ? (o & 7) * a.oLc + (o >> 3) : 8 * a.oLc + (o - a.oK8));
    if (KIND == kIFG) {
      const bool tl = o >= (a.H & ~7);  // sigmoid / swiglu over T*H = H elements
      float f = sigmoid_of(v1, tl);
      if (a.lb) f = __builtin_fmaf(1.0f - e_lb, f, e_lb);
      const float in = swiglu_of(val, 1.0f - f, tl);
      const float s = __builtin_fmaf(f, e_st, in);
      a.state[o] = s;
      a.recur[p] = s;
      a.gout[p] = v2;
      if (a.out) a.out[p] = src[0][p];  // layer 0: the embedding row becomes h
    } else if (KIND == kO || KIND == kDown) {
      a.out[p] = e_hin + val;
    } else if (KIND == kGate) {
      a.out[p] = swiglu_of(val, v1, o >= (nout & ~7));
    } else {  // kLM
      if (a.out) a.out[o] = val;
      const unsigned long long kk = amax_key(val, o);
      best = kk > best ? kk : best;
    }
  }

  MMF_MARK(KIND, 6);
  if (KIND == kLM && a.keys) {  // one partial key per block, reduced by the consumer
    for (int off = 32; off > 0; off >>= 1) {
      const unsigned long long other = __shfl_xor(best, off);
      best = other > best ? other : best;
    }
    unsigned long long* r64 = reinterpret_cast<unsigned long long*>(red);
    if ((tid & 63) == 0) r64[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) a.keys[blockIdx.x] = r64[0] > r64[1] ? r64[0] : r64[1];
  }
  MMF_MARK(KIND, 7);
  MMF_SPAN(KIND, false);
}

template <int MODE, int KIND>
hipError_t dec_kind(const DecArgs& a, size_t lds, int grid, hipStream_t s) {
  constexpr int BS = kBlock * KindTraits<KIND>::NM;
  const int W4 = (8 * a.p[0].g.Lc + 8) / 4;
  if (W4 <= 2 * BS) k_decode<MODE, KIND, 2><<<grid, BS, lds, s>>>(a);
  else if (W4 <= 4 * BS) k_decode<MODE, KIND, 4><<<grid, BS, lds, s>>>(a);
  else if (W4 <= 8 * BS) k_decode<MODE, KIND, 8><<<grid, BS, lds, s>>>(a);
  else if (W4 <= 16 * BS) k_decode<MODE, KIND, 16><<<grid, BS, lds, s>>>(a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int MODE>
hipError_t dec_mode(DecKind kind, const DecArgs& a, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int Lc = g.Lc;
  const int na = kind == kIFG ? 3 : 1;
  const size_t WL = 8 * static_cast<size_t>((Lc + 31) / 32 * 32 + 4) + 8, LQ = Lc + 16;
  size_t lds = (2 * WL + 16 + 48) * sizeof(float);
  lds += (MODE == kFloat) ? na * WL * sizeof(float) : na * (16 * LQ + 8 * sizeof(int32_t) + sizeof(float));
  const int nout = (kind == kGate) ? g.N / 2 : g.N;
  int grid = (nout + kGroup - 1) / kGroup;
  if (kind == kLM && grid > kLMBlocks) grid = kLMBlocks;
  switch (kind) {
    case kIFG: return dec_kind<MODE, kIFG>(a, lds, grid, s);
    case kO: return dec_kind<MODE, kO>(a, lds, grid, s);
    case kGate: return dec_kind<MODE, kGate>(a, lds, grid, s);
    case kDown: return dec_kind<MODE, kDown>(a, lds, grid, s);
    default: return dec_kind<MODE, kLM>(a, lds, grid, s);
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

#ifdef MMF_PHASE_TRACE
extern "C" int mmf_debug_phase_trace(unsigned long long* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(mmf_phase_trace), sizeof(unsigned long long) * 50) == hipSuccess ? 0 : 2;
}
#endif
