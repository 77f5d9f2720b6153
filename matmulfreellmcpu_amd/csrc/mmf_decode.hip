// mmf_decode.hip -- fused single-row decode kernels, one launch per BitLinear group of a
// layer (Model::block at T = 1, hgrn_model.cpp:80-195):
//   kIFG  : [embed] -> attn_norm -> BitLinear norm -> i/f/g GEMVs -> sigmoid, lower bound,
//           swiglu, recurrence step (hgrn_model.cpp:95-150)
//   kO    : g_norm (RMSNorm(g) * silu(recur)) -> BitLinear norm -> o GEMV -> resid = h + o
//   kGate : mlp_norm -> BitLinear norm -> gate/up GEMV (rows c and I + c) -> swiglu
//   kDown : BitLinear norm -> down GEMV -> h = resid + d
//   kLM   : final norm -> BitLinear norm -> lm_head GEMV -> logits, argmax key (atomicMax)
// Every block recomputes the (cheap, order-exact) row norms of its input vector in LDS, so
// no grid-wide synchronisation is needed inside a launch. A block is 16 outputs x 8 chains;
// thread (ol, j) sums chain j of output og*16+ol, the reference's AVX2 lane j.
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

__device__ __forceinline__ int act_pos(int k, int K8, int Lc) {
  return k < K8 ? (k & 7) * Lc + (k >> 3) : 8 * Lc + (k - K8);
}

__device__ float dec_sumsq(const float* X, int Lc, int nb, int ntail, float* red) {
  if (threadIdx.x < 8) {
    const float* c = X + threadIdx.x * Lc;
    float a = 0.0f;
    int t = 0;
    for (; t + 4 <= nb; t += 4) {
      float4 v = *reinterpret_cast<const float4*>(c + t);
      a = __builtin_fmaf(v.x, v.x, a);
      a = __builtin_fmaf(v.y, v.y, a);
      a = __builtin_fmaf(v.z, v.z, a);
      a = __builtin_fmaf(v.w, v.w, a);
    }
    for (; t < nb; ++t) a = __builtin_fmaf(c[t], c[t], a);
    red[threadIdx.x] = a;
  }
  __syncthreads();
  float s = hsum8(red);
  for (int t = 0; t < ntail; ++t) {
    const float v = X[8 * Lc + t];
    s = __builtin_fmaf(v, v, s);
  }
  __syncthreads();
  return s;
}

__device__ float dec_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float m = fmaxf(red[0], red[1]);
  __syncthreads();
  return m;
}

template <int KIND> struct KindTraits;
template <> struct KindTraits<kIFG> { static constexpr int NM = 3, NA = 3; };
template <> struct KindTraits<kO> { static constexpr int NM = 1, NA = 1; };
template <> struct KindTraits<kGate> { static constexpr int NM = 2, NA = 1; };
template <> struct KindTraits<kDown> { static constexpr int NM = 1, NA = 1; };
template <> struct KindTraits<kLM> { static constexpr int NM = 1, NA = 1; };

template <int MODE, int KIND>
__global__ __launch_bounds__(kBlock) void k_decode(DecArgs a) {
  constexpr int NM = KindTraits<KIND>::NM, NA = KindTraits<KIND>::NA;
  extern __shared__ float smem[];
  const Geom& g = a.p[0].g;
  const int K = g.K, K8 = g.K8, nb = g.nb, nt = g.ntail, Lc = g.Lc;
  const int tid = threadIdx.x, ol = tid >> 3, j = tid & 7;

  float* X = smem;                 // [8Lc + 8] input row, chain-transposed
  float* S = X + 8 * Lc + 8;       // [8Lc + 8] silu(recur) (kO)
  float* red = S + 8 * Lc + 8;     // [16]
  float* Y = red + 16;             // float: NA x [8Lc + 8]
  int8_t* Q = reinterpret_cast<int8_t*>(red + 16);      // int: NA x [2 x 8Lc]
  int32_t* CT = reinterpret_cast<int32_t*>(Q + NA * 16 * Lc);  // NA x 8 tail codes
  float* SA = reinterpret_cast<float*>(CT + NA * 8);           // NA int8 scales

  // ---- input row -------------------------------------------------------------------
  const float* xsrc = a.x;
  if (KIND == kIFG && xsrc == nullptr) {
    int64_t tok = key_index(*a.key);
    if (tok < 0 || tok >= a.vocab) tok = 0;
    xsrc = a.emb + static_cast<size_t>(tok) * K;
    if (blockIdx.x == 0 && tid == 0 && a.hist) {
      const int pos = *a.hist_pos;
      if (pos < a.hist_cap) a.hist[pos] = tok;
      *a.hist_pos = pos + 1;
    }
  }
  if (KIND == kO && a.key_reset && blockIdx.x == 0 && tid == 0) *a.key_reset = 0ull;
  for (int k = tid; k < K; k += kBlock) X[act_pos(k, K8, Lc)] = xsrc[k];
  for (int jj = 0; jj < 8; ++jj)
    for (int t = nb + tid; t < Lc; t += kBlock) X[jj * Lc + t] = 0.0f;
  if (tid < 8 && tid >= nt) X[8 * Lc + tid] = 0.0f;
  if (KIND == kO)
    for (int k = tid; k < K; k += kBlock) S[act_pos(k, K8, Lc)] = silu_of(a.x2[k], k >= (K & ~7));
  __syncthreads();

  // ---- stage 1: the block's own pre-norm -----------------------------------------------
  if (KIND != kDown) {
    const float r1 = rstd_of(dec_sumsq(X, Lc, nb, nt, red), K, a.eps);
    for (int k = tid; k < K; k += kBlock) {
      const int p = act_pos(k, K8, Lc);
      float v = (X[p] * r1) * a.pre_w[k];
      if (KIND == kO) v = v * S[p];
      X[p] = v;
    }
    __syncthreads();
  }
  // ---- stage 2: the BitLinear RMSNorm and activation encoding ---------------------------
  const float r2 = rstd_of(dec_sumsq(X, Lc, nb, nt, red), K, a.eps);
#pragma unroll
  for (int ai = 0; ai < NA; ++ai) {
    const float* nw = a.p[ai].normw;
    if (MODE == kFloat) {
      float* yo = Y + ai * (8 * Lc + 8);
      for (int p = tid; p < 8 * Lc + 8; p += kBlock) {
        float v = 0.0f;
        if (p < 8 * Lc) {
          const int jj = p / Lc, t = p - jj * Lc;
          if (t < nb) v = (X[p] * r2) * nw[jj + 8 * t];
        } else if (p - 8 * Lc < nt) {
          v = (X[p] * r2) * nw[K8 + p - 8 * Lc];
        }
        yo[p] = v;
      }
    } else {
      float sa = 0.0f;
      if (MODE == kInt8) {
        float m = 0.0f;
        for (int k = tid; k < K; k += kBlock) m = fmaxf(m, fabsf((X[act_pos(k, K8, Lc)] * r2) * nw[k]));
        m = dec_max(m, red);
        sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
        if (tid == 0) SA[ai] = sa;
      }
      int8_t* q = Q + ai * 16 * Lc;
      for (int p4 = tid * 4; p4 < 8 * Lc; p4 += kBlock * 4) {
        const int jj = p4 / Lc, t0 = p4 - jj * Lc;
        uint32_t hi = 0, lo = 0;
        for (int u = 0; u < 4; ++u) {
          const int t = t0 + u;
          if (t < nb) {
            const float y = (X[p4 + u] * r2) * nw[jj + 8 * t];
            if (MODE == kFixed) {
              const int32_t c = q510_body(y, a.qs);
              hi |= static_cast<uint32_t>((c >> 8) & 0xFF) << (8 * u);
              lo |= static_cast<uint32_t>(((c & 0xFF) - 128) & 0xFF) << (8 * u);
            } else {
              hi |= static_cast<uint32_t>(q8_of(y, sa) & 0xFF) << (8 * u);
            }
          }
        }
        *reinterpret_cast<uint32_t*>(q + p4) = hi;
        if (MODE == kFixed) *reinterpret_cast<uint32_t*>(q + 8 * Lc + p4) = lo;
      }
      if (tid < 8) {
        int32_t c = 0;
        if (tid < nt) {
          const float y = (X[8 * Lc + tid] * r2) * nw[K8 + tid];
          c = (MODE == kFixed) ? q510_tail(y, a.qs) : q8_of(y, sa);
        }
        CT[ai * 8 + tid] = c;
      }
    }
  }
  __syncthreads();

  // ---- GEMV over this block's output groups ---------------------------------------------
  const int nout = (KIND == kGate) ? g.N / 2 : g.N;
  const int ngroups_out = (nout + kGroup - 1) / kGroup;
  unsigned long long best = 0ull;
  for (int og = blockIdx.x; og < ngroups_out; og += gridDim.x) {
    const uint32_t* slab[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const ProjDev& P = a.p[KIND == kIFG ? mi : 0];
      const int gg = og + ((KIND == kGate && mi == 1) ? g.ngroups / 2 : 0);
      slab[mi] = P.pk + static_cast<size_t>(gg) * g.Wc * 128 + ol * 8 + j;
    }
    float facc[NM];
    int32_t hacc[NM], lacc[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) { facc[mi] = 0.0f; hacc[mi] = 0; lacc[mi] = 0; }

    constexpr int U = 4;  // words in flight per matrix
    for (int m0 = 0; m0 < g.Wc; m0 += U) {
      uint32_t w[U][NM];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
          w[u][mi] = (m0 + u < g.Wc) ? slab[mi][static_cast<size_t>(m0 + u) * 128] : 0u;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int m = m0 + u;
        if (m >= g.Wc) break;
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) {
          const int ai = (NA > 1) ? mi : 0;
          if (MODE == kFloat) {
            const float* yl = Y + ai * (8 * Lc + 8) + j * Lc + 16 * m;
            float y[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const float4 v = *reinterpret_cast<const float4*>(yl + 4 * q4);
              y[4 * q4] = v.x; y[4 * q4 + 1] = v.y; y[4 * q4 + 2] = v.z; y[4 * q4 + 3] = v.w;
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) facc[mi] = __builtin_fmaf(y[t], code_f(w[u][mi], t), facc[mi]);
          } else {
            const int8_t* ql = Q + ai * 16 * Lc + j * Lc + 16 * m;
            const uint4 h = *reinterpret_cast<const uint4*>(ql);
            const uint32_t w0 = w4_i8(w[u][mi], 0), w1 = w4_i8(w[u][mi], 1), w2 = w4_i8(w[u][mi], 2),
                           w3 = w4_i8(w[u][mi], 3);
            hacc[mi] = dot4(w0, h.x, hacc[mi]);
            hacc[mi] = dot4(w1, h.y, hacc[mi]);
            hacc[mi] = dot4(w2, h.z, hacc[mi]);
            hacc[mi] = dot4(w3, h.w, hacc[mi]);
            if (MODE == kFixed) {
              const uint4 l = *reinterpret_cast<const uint4*>(ql + 8 * Lc);
              lacc[mi] = dot4(w0, l.x, lacc[mi]);
              lacc[mi] = dot4(w1, l.y, lacc[mi]);
              lacc[mi] = dot4(w2, l.z, lacc[mi]);
              lacc[mi] = dot4(w3, l.w, lacc[mi]);
            }
          }
        }
      }
    }

    // reduce the 8 chains, add the tail, scale
    const int o = og * kGroup + ol;
    float val[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const ProjDev& P = a.p[KIND == kIFG ? mi : 0];
      const int oo = o + ((KIND == kGate && mi == 1) ? nout : 0);
      const int ai = (NA > 1) ? mi : 0;
      if (MODE == kFloat) {
        float s = hsum8_lanes(facc[mi]);
        if (j == 0 && o < nout) {
          const float* yt = Y + ai * (8 * Lc + 8) + 8 * Lc;
          for (int t = 0; t < nt; ++t) {
            const int8_t wt = P.tail[oo * 8 + t];
            if (wt > 0) s += yt[t];
            else if (wt < 0) s -= yt[t];
          }
        }
        val[mi] = s * P.inv_scale_w;
      } else {
        int32_t s = isum8_lanes(hacc[mi]);
        if (MODE == kFixed) s = s * 256 + isum8_lanes(lacc[mi]);
        val[mi] = 0.0f;
        if (j == 0 && o < nout) {
          if (MODE == kFixed) s += 128 * P.rowsum[oo];
          for (int t = 0; t < nt; ++t) s += static_cast<int32_t>(P.tail[oo * 8 + t]) * CT[ai * 8 + t];
          val[mi] = (MODE == kFixed) ? static_cast<float>(s) * a.inv_fixed[KIND == kIFG ? mi : 0]
                                     : static_cast<float>(s) / (P.scale_w * SA[ai]);
        }
      }
    }
    if (j != 0 || o >= nout) continue;

    // ---- epilogues -------------------------------------------------------------------
    if (KIND == kIFG) {
      const bool tl = o >= (a.H & ~7);  // sigmoid / swiglu over T*H = H elements
      float f = sigmoid_of(val[1], tl);
      if (a.lb) f = __builtin_fmaf(1.0f - a.lb[o], f, a.lb[o]);
      const float in = swiglu_of(val[0], 1.0f - f, tl);
      const float s = __builtin_fmaf(f, a.state[o], in);
      a.state[o] = s;
      a.recur[o] = s;
      a.gout[o] = val[2];
      if (a.out) a.out[o] = xsrc[o];
    } else if (KIND == kO || KIND == kDown) {
      a.out[o] = a.hin[o] + val[0];
    } else if (KIND == kGate) {
      a.out[o] = swiglu_of(val[0], val[1], o >= (nout & ~7));
    } else {  // kLM
      if (a.out) a.out[o] = val[0];
      const unsigned long long kk = amax_key(val[0], o);
      best = kk > best ? kk : best;
    }
  }

  if (KIND == kLM && a.key) {
    for (int off = 32; off > 0; off >>= 1) {
      const unsigned long long other = __shfl_xor(best, off);
      best = other > best ? other : best;
    }
    __syncthreads();
    unsigned long long* r64 = reinterpret_cast<unsigned long long*>(red);
    if ((tid & 63) == 0) r64[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
      const unsigned long long b = r64[0] > r64[1] ? r64[0] : r64[1];
      atomicMax(a.key, b);
    }
  }
}

template <int MODE>
hipError_t dec_mode(DecKind kind, const DecArgs& a, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int Lc = g.Lc;
  const int na = kind == kIFG ? 3 : 1;
  size_t lds = (2 * static_cast<size_t>(8 * Lc + 8) + 16) * sizeof(float);
  lds += (MODE == kFloat) ? na * static_cast<size_t>(8 * Lc + 8) * sizeof(float)
                          : na * (16 * static_cast<size_t>(Lc) + 8 * sizeof(int32_t) + sizeof(float));
  const int nout = (kind == kGate) ? g.N / 2 : g.N;
  int grid = (nout + kGroup - 1) / kGroup;
  if (kind == kLM && grid > 2048) grid = 2048;
  switch (kind) {
    case kIFG: k_decode<MODE, kIFG><<<grid, kBlock, lds, s>>>(a); break;
    case kO: k_decode<MODE, kO><<<grid, kBlock, lds, s>>>(a); break;
    case kGate: k_decode<MODE, kGate><<<grid, kBlock, lds, s>>>(a); break;
    case kDown: k_decode<MODE, kDown><<<grid, kBlock, lds, s>>>(a); break;
    default: k_decode<MODE, kLM><<<grid, kBlock, lds, s>>>(a); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(DecKind kind, Mode mode, const DecArgs& a, hipStream_t s) {
  switch (mode) {
    case kFloat: return dec_mode<kFloat>(kind, a, s);
    case kFixed: return dec_mode<kFixed>(kind, a, s);
    default: return dec_mode<kInt8>(kind, a, s);
  }
}

}  // namespace mmf
