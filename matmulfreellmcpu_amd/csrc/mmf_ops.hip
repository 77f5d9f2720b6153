// mmf_ops.hip -- multi-row kernels: weight repack, BitLinear prologue (norms + activation
// quantisation), the ternary GEMM over row tiles, the HGRN mixer/recurrence and the
// elementwise ops. These serve prefill, batched (serving) decode, the stateless forward
// and the op-level entry points; single-row decode has fused kernels in mmf_decode.hip.
//
// Numerics follow the reference engine exactly (see mmf_device.hpp): every fp32
// reduction keeps the 8-lane order of the AVX2 code, every int32 sum is exact.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

// Chain-transposed LDS copy of one row for the order-exact row norms: chain j at
// X[j * LS ...], LS = roundup(Lc, 32) + 4 (the +4 spreads the 8 chain rows over distinct
// LDS banks), zeros from nb up to roundup(Lc, 32), the tail at X[8 * LS ...].
__device__ __forceinline__ int lds_stride(int Lc) { return (Lc + 31) / 32 * 32 + 4; }

__device__ __forceinline__ int act_pos(int k, int K8, int LS) {
  return k < K8 ? (k & 7) * LS + (k >> 3) : 8 * LS + (k - K8);
}

// Reference sumsq (simd.hpp:69-89) of a padded chain-transposed vector in LDS: every
// thread gets the result. `red` is 8 floats of LDS.
template <int U = 8>
__device__ float block_sumsq(const float* X, int Lc, int LS, int ntail, float* red) {
  chain_begin<U>(X, Lc, LS, red);
  __syncthreads();
  const float s = chain_end(X, LS, ntail, red);
  __syncthreads();
  return s;
}
// The same with the ring-buffered chains (rows zero to a multiple of 32).
__device__ float block_sumsq_ring(const float* X, int Lc, int LS, int ntail, float* red) {
  chain_ring(X, Lc, LS, red);
  __syncthreads();
  const float s = chain_end(X, LS, ntail, red);
  __syncthreads();
  return s;
}

// Maximum over a block of NW full waves, one barrier: a DPP butterfly within each 16-lane
// row, the four row maxima read out of lanes 0/16/32/48, one slot per wave in red[0 .. NW).
// The result is uniform. red must not be written again before every thread has read it:
// callers alternate between two areas with a barrier between their uses of either.
template <int NW>
__device__ float block_max1(float v, float* red) {
  auto dpp_max = [](float x, auto ctrl) {
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value, 0xf, 0xf, false);
    return fmaxf(x, __builtin_bit_cast(float, y));
  };
  v = dpp_max(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  v = dpp_max(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  v = dpp_max(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  v = dpp_max(v, std::integral_constant<int, 0x140>{});  // row_mirror
  const auto lane = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
  const float m = fmaxf(fmaxf(lane(0), lane(16)), fmaxf(lane(32), lane(48)));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

// for k = threadIdx.x, + blockDim.x, ... < n: fetch(k) for kU elements first, then use(k,
// value) -- kU global loads in flight per thread instead of one round trip per element.
constexpr int kU = 8;
template <class Fetch, class Use>
__device__ __forceinline__ void batched_loop(int n, Fetch fetch, Use use) {
  for (int k0 = threadIdx.x; k0 < n; k0 += kU * blockDim.x) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = k0 + u * blockDim.x;
      v[u] = k < n ? fetch(k) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = k0 + u * blockDim.x;
      if (k < n) use(k, v[u]);
    }
  }
}

// Load row x[0..K) into the padded chain-transposed LDS layout (zeros in the padding).
__device__ void load_T(float* X, const float* x, int K, int K8, int Lc, int LS, int nb) {
  batched_loop(K, [&](int k) { return x[k]; }, [&](int k, float v) { X[act_pos(k, K8, LS)] = v; });
  const int L32 = (Lc + 31) / 32 * 32;
  for (int j = 0; j < 8; ++j)
    for (int t = nb + threadIdx.x; t < L32; t += blockDim.x) X[j * LS + t] = 0.0f;
  for (int t = (K - K8) + threadIdx.x; t < 8; t += blockDim.x) X[8 * LS + t] = 0.0f;
}

// ------------------------------------------------------------------------------------
// weight repack
// ------------------------------------------------------------------------------------
__global__ void k_pack(const int8_t* __restrict__ wq, Geom g, uint32_t* __restrict__ pk,
                       int* __restrict__ bad) {
  const size_t nwords = static_cast<size_t>(g.ngroups) * g.Wc * kGroup * 8;
  for (size_t w = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; w < nwords;
       w += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int j = static_cast<int>(w & 7);
    const int ol = static_cast<int>((w >> 3) & 15);
    const size_t gm = w >> 7;  // og * Wc + m
    const int m = static_cast<int>(gm % g.Wc);
    const int og = static_cast<int>(gm / g.Wc);
    const int o = og * kGroup + ol;
    uint32_t word = 0;
    if (o < g.N) {
      const int8_t* row = wq + static_cast<size_t>(o) * g.K;
      for (int t = 0; t < 16; ++t) {
        const int tt = 16 * m + t;
        if (tt < g.nb) {
          const int v = row[j + 8 * tt];
          if (v < -1 || v > 1) atomicOr(bad, 1);
          word |= static_cast<uint32_t>(v & 3) << code_shift(t);
        }
      }
    }
    pk[w] = word;
  }
}

// The TernaryBackend seam's few-row matmul (mmf_ternary_matmul_host): acc[z][r][o] =
// sum_k x[z][r][k] * wq_z[o][k] in int32 for B <= kSeamRows rows, one launch for k projections
// of one shape (blockIdx.y = z). x and acc are the caller's pinned host staging. A block issues
// its first slab words, then reads its projection's rows of codes from host memory once and
// stores each row's body as two int8 planes in the slab's chain order (x = 256 hi + lo + 128
// with hi = x >> 8 and lo = (x & 255) - 128, the split of the Q5.10 GEMMs) and its tail as
// int32. It runs two 16-output groups at a time: thread (ol, j) sums chain j of output ol with
// v_dot4 on each plane (words read 8 at a time), the 8 chains are added across lanes, then
// 256 hi + lo + 128 rowsum + tail. All sums are exact integers (the reference's int32 lanes),
// so their order is free.
constexpr int kSeamRows = 4;
template <int B>
__global__ __launch_bounds__(256) void k_seam_dot(SeamArgs a) {
  extern __shared__ int32_t seam_lds[];
  const int z = blockIdx.y;
  const Geom& g = a.g;
  const int K = g.K, LQ = g.Lc + 16;        // plane row stride in bytes (16 bytes of padding)
  int8_t* hp = reinterpret_cast<int8_t*>(seam_lds);  // [B][2][8][LQ]: hi plane, lo plane
  int32_t* tl = seam_lds + B * 4 * LQ;                 // [B][8] tail codes
  const int lt = threadIdx.x & 127, ol = lt >> 3, j = lt & 7, sub = threadIdx.x >> 7;
  const uint32_t* pk = a.pk[z];
  int og = 2 * blockIdx.x + sub;
  uint32_t w[8];
  auto words = [&](int og_, int m0) {
    const uint32_t* wp = pk + static_cast<size_t>(og_) * g.Wc * 128 + lt;
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = (m0 + u < g.Wc) ? wp[(m0 + u) * 128] : 0u;  // zero words add nothing
  };
  if (og < g.ngroups) words(og, 0);
  const int32_t* x = a.x + static_cast<size_t>(z) * B * K;
  for (int r = 0; r < B; ++r) {
    int8_t* hr = hp + r * 16 * LQ;
    for (int e = threadIdx.x; e < 8 * LQ; e += 256) {  // chain position order: element j + 8t at row j, byte t
      const int jj = e / LQ, t = e - jj * LQ, k = jj + 8 * t;
      const int32_t v = (t < g.nb) ? x[static_cast<size_t>(r) * K + k] : 0;  // past the body: 0 = 256*0 + (-128) + 128
      hr[e] = static_cast<int8_t>(v >> 8);
      hr[8 * LQ + e] = static_cast<int8_t>((v & 255) - 128);
    }
    if (threadIdx.x < 8) tl[r * 8 + threadIdx.x] = (static_cast<int>(threadIdx.x) < g.ntail) ? x[static_cast<size_t>(r) * K + g.K8 + threadIdx.x] : 0;
  }
  __syncthreads();
  for (; og < g.ngroups; og += 2 * gridDim.x) {
    int32_t sh[B], sl[B];
#pragma unroll
    for (int r = 0; r < B; ++r) sh[r] = sl[r] = 0;
    for (int m0 = 0; m0 < g.Wc; m0 += 8) {
      if (m0 > 0) words(og, m0);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (m0 + q >= g.Wc) break;
        const uint32_t w0 = w4_i8(w[q], 0), w1 = w4_i8(w[q], 1), w2 = w4_i8(w[q], 2), w3 = w4_i8(w[q], 3);
#pragma unroll
        for (int r = 0; r < B; ++r) {
          const int8_t* hr = hp + r * 16 * LQ + j * LQ + 16 * (m0 + q);
          const uint4 xh = *reinterpret_cast<const uint4*>(hr);
          const uint4 xl = *reinterpret_cast<const uint4*>(hr + 8 * LQ);
          sh[r] = dot4(w3, xh.w, dot4(w2, xh.z, dot4(w1, xh.y, dot4(w0, xh.x, sh[r]))));
          sl[r] = dot4(w3, xl.w, dot4(w2, xl.z, dot4(w1, xl.y, dot4(w0, xl.x, sl[r]))));
        }
      }
    }
    const int o = og * kGroup + ol;
    const bool live = o < g.N;
    const int32_t rs = live ? a.rowsum[z][o] : 0;
#pragma unroll
    for (int r = 0; r < B; ++r) {
      const int32_t h = isum8_lanes(sh[r]), l = isum8_lanes(sl[r]);
      if (j == 0 && live) {
        uint32_t v = static_cast<uint32_t>(h) * 256u + static_cast<uint32_t>(l) + 128u * static_cast<uint32_t>(rs);
        for (int t = 0; t < g.ntail; ++t)
          v += static_cast<uint32_t>(static_cast<int32_t>(a.tail[z][o * 8 + t]) * tl[r * 8 + t]);
        a.acc[(static_cast<size_t>(z) * B + r) * g.N + o] = static_cast<int32_t>(v);
      }
    }
    if (og + 2 * static_cast<int>(gridDim.x) < g.ngroups) words(og + 2 * gridDim.x, 0);
  }
}

// 2-bit slab -> fp4 slab (float-mode decode): word m of a chain in pk (16 codes) becomes words
// 2m and 2m + 1 of pk4 (codes 0..7 and 8..15), code t of a word in nibble t as an E2M1 value
// (0 -> 0x0, +1 -> 0x2, -1 -> 0xA; all exact), so one v_cvt_scalef32_pk_f32_fp4 turns byte b
// into the fp32 codes 2b and 2b + 1.
__global__ void k_pack4(const uint32_t* __restrict__ pk, size_t nwords, int Wc, uint32_t* __restrict__ pk4) {
  for (size_t w = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; w < nwords;
       w += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint32_t src = pk[w];
    const size_t gm = w >> 7;  // og * Wc + m
    const size_t og = gm / Wc, m = gm % Wc;
    const size_t lane = w & 127;
    uint32_t half[2] = {0u, 0u};
    for (int t = 0; t < 16; ++t) {
      const uint32_t c = (src >> code_shift(t)) & 3u;
      const uint32_t n = c == 1u ? 0x2u : (c == 3u ? 0xAu : 0x0u);
      half[t >> 3] |= n << (4 * (t & 7));
    }
    const size_t base = ((og * 2 * Wc + 2 * m) << 7) + lane;
    pk4[base] = half[0];
    pk4[base + 128] = half[1];
  }
}

// Per output row (one block each, rows padded to whole groups): the exact int32 sum of the
// body codes (order-free) and the tail codes. One thread per row walking K codes in turn
// took 0.7 ms for a 5632 x 1024 matrix; a block reads the row in 256-byte steps.
__global__ __launch_bounds__(256) void k_pack_rows(const int8_t* __restrict__ wq, Geom g,
                                                   int8_t* __restrict__ tail,
                                                   int32_t* __restrict__ rowsum, int* __restrict__ bad) {
  __shared__ int32_t part[4];
  const int o = blockIdx.x;
  int32_t s = 0;
  if (o < g.N) {
    const int8_t* row = wq + static_cast<size_t>(o) * g.K;
    for (int k = threadIdx.x; k < g.K8; k += 256) s += row[k];
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) rowsum[o] = (part[0] + part[1]) + (part[2] + part[3]);
  if (threadIdx.x < 8) {
    const int t = threadIdx.x;
    const int8_t v = (o < g.N && t < g.ntail) ? wq[static_cast<size_t>(o) * g.K + g.K8 + t] : 0;
    if (v < -1 || v > 1) atomicOr(bad, 1);
    tail[o * 8 + t] = v;
  }
}

// Row of block b in the row kernels that write the fragment-tiled integer codes. A 128-byte
// line of those codes holds 16 bytes of each of 8 consecutive rows; blocks go to the 8 XCDs
// in turn (block b on XCD b % 8), so XCD x takes the 8-row groups x, x + 8, x + 16, ... and
// the partial lines of one group merge in one L2 instead of meeting in memory from several.
// The grid is the row count rounded up to 64; blocks past the last row exit at once.
__device__ __forceinline__ int xcd_row(int b) {
  const int x = b & 7, i = b >> 3;
  return (((i >> 3) << 3) + x) * 8 + (i & 7);
}
static int row_grid(int rows) { return (rows + 63) / 64 * 64; }

// ------------------------------------------------------------------------------------
// BitLinear prologue over rows: optional stage-1 norm, the BitLinear RMSNorm
// (bitlinear.cpp:62-78, 99-107) and the activation encoding of each of na projections.
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ void k_prologue(PrologueArgs a, ActBuf act) {
  extern __shared__ float smem[];
  const int row = xcd_row(blockIdx.x);
  if (row >= act.rows) return;
  const int Lc = act.Lc, K = act.K, K8 = act.K8, nb = act.nb, nt = act.ntail;
  const int LS = lds_stride(Lc);
  float* X = smem;                   // [8*LS + 8]
  float* S = X + 8 * LS + 8;         // [8*LS + 8] silu(x2) for kPreSwish
  float* red = S + 8 * LS + 8;       // [16]
  load_T(X, a.x + static_cast<size_t>(row) * K, K, K8, Lc, LS, nb);
  if (a.pre == kPreSwish) {
    // silu over one row of `cols` = K elements (rmsnorm_swishgate.cpp:24): tail k >= K & ~7
    const float* o = a.x2 + static_cast<size_t>(row) * K;
    batched_loop(K, [&](int k) { return o[k]; },
                 [&](int k, float v) { S[act_pos(k, K8, LS)] = silu_of(v, k >= (K & ~7)); });
  }
  __syncthreads();
  if (a.pre != kPreNone) {
    const float r1 = rstd_of(block_sumsq(X, Lc, LS, nt, red), K, a.eps);
    batched_loop(K, [&](int k) { return a.pre_w[k]; }, [&](int k, float w) {
      const int p = act_pos(k, K8, LS);
      float v = (X[p] * r1) * w;
      if (a.pre == kPreSwish) v = v * S[p];
      X[p] = v;
    });
    __syncthreads();
  }
  const float r2 = rstd_of(block_sumsq(X, Lc, LS, nt, red), K, a.eps);
  // Per projection: y = (x * rstd) * normw (bitlinear.cpp:62-70) for every element in one
  // parallel pass into LDS (S is free after stage 1), then the encoding reads only LDS.
  float* Y = S;
  for (int ai = 0; ai < a.na; ++ai) {
    const float* __restrict__ nw = a.normw[ai];
    const size_t ar = static_cast<size_t>(ai) * act.rows + row;
    float m = 0.0f;
    batched_loop(K, [&](int k) { return nw[k]; }, [&](int k, float w) {
      const int p = act_pos(k, K8, LS);
      const float y = (X[p] * r2) * w;
      Y[p] = y;
      if (MODE == kInt8) m = fmaxf(m, fabsf(y));
    });
    float sa = 0.0f;
    if (MODE == kInt8) {
      m = block_max(m, red);  // includes the barrier that publishes Y
      sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
      if (threadIdx.x == 0) act.sa[ar] = sa;
    } else {
      __syncthreads();
    }
    if (MODE == kFloat) {
      float* yo = act.y + ar * act.ystride();
      for (int j = 0; j < 8; ++j)
        for (int t = threadIdx.x; t < Lc; t += blockDim.x) yo[j * Lc + t] = (t < nb) ? Y[j * LS + t] : 0.0f;
      for (int t = threadIdx.x; t < 8; t += blockDim.x) yo[8 * Lc + t] = (t < nt) ? Y[8 * LS + t] : 0.0f;
    } else {
      int8_t* q = act.q + act.qoff(ai, 0, row, 0);
      const size_t lop = act.qplane();
      // 4 consecutive chain positions per thread -> one 32-bit store per plane (4 consecutive
      // positions from a multiple of 4 stay in one 16-byte run of the fragment layout)
      const int n4 = Lc / 4;
      for (int w = threadIdx.x; w < 8 * n4; w += blockDim.x) {
        const int j = w / n4, t4 = (w - j * n4) * 4;
        uint32_t hi = 0, lo = 0;
        for (int u = 0; u < 4; ++u) {
          const int t = t4 + u;
          if (t < nb) {
            const float y = Y[j * LS + t];
            if (MODE == kFixed) {
              const int32_t c = q510_body(y, a.qs);
              hi |= static_cast<uint32_t>((c >> 8) & 0xFF) << (8 * u);
              lo |= static_cast<uint32_t>(((c & 0xFF) - 128) & 0xFF) << (8 * u);
            } else {
              hi |= static_cast<uint32_t>(q8_of(y, sa) & 0xFF) << (8 * u);
            }
          }
        }
        *reinterpret_cast<uint32_t*>(q + ActBuf::qpos(j * Lc + t4)) = hi;
        if (MODE == kFixed) *reinterpret_cast<uint32_t*>(q + lop + ActBuf::qpos(j * Lc + t4)) = lo;
      }
      for (int t = threadIdx.x; t < 8; t += blockDim.x) {
        int32_t c = 0;
        if (t < nt) {
          const float y = Y[8 * LS + t];
          c = (MODE == kFixed) ? q510_tail(y, a.qs) : q8_of(y, sa);
        }
        act.ct[ar * 8 + t] = c;
      }
    }
    __syncthreads();  // Y is rewritten for the next projection
  }
}

__device__ __forceinline__ float f4el(const float4& f, int c) {
  return c == 0 ? f.x : (c == 1 ? f.y : (c == 2 ? f.z : f.w));
}

// Waves per SIMD of the row prologue: 8 (64 VGPRs; 8 rows resident per CU, so 2048 rows run
// in one round; chains through a ring of 8 float4) where what a thread keeps -- the row inputs
// and stage-1 weight through the first chain, two sets of norm weights (and the Int8
// values, through the absmax) in the encoding -- fits without spilling, else the compiler's
// choice.
template <int MODE, int PRE, int NA, int MAXG, int BT>
constexpr int rowpro_waves() {
  constexpr int nx = PRE == kPreSwish ? 2 : (PRE == kPreMixSwish ? 5 : 1);
  constexpr int entry = 8 * MAXG * (nx + (PRE != kPreNone ? 1 : 0));               // row inputs
  constexpr int encode = 8 * MAXG * ((NA > 1 ? 2 : 1) + (MODE == kInt8 ? 1 : 0));  // weights, values
  return (BT == 256 && entry <= 24 && encode <= 40) ? 8 : 1;
}

// The row prologue for K % 4 == 0 with 16-byte aligned inputs and the chain-transposed norm
// weights normwT. One block per row; each thread owns
//  - groups (the loads and the element-wise stage 1): group t < G = nb + (ntail > 0) is the
//    eight elements 8t .. 8t+7, chain position t of every chain (two float4 loads), or for
//    t = nb the ntail (= 4) tail elements. Its values go to the chain-transposed LDS row
//    X[c * LS + t] (tail: X[8 * LS + c]) that the order-fixed norm chains read;
//  - units (the BitLinear norm and the encoding): unit u < Lc is positions t0 .. t0+7 of
//    chain j (u = j * Lc/8 + t0/8). Its eight normed values come from two LDS reads and two
//    float4 reads of normwT and leave as one 8-byte store per int8 plane (positions
//    t0 .. t0+7 are contiguous in the fragment layout) or as two float4 stores.
// Every global input of a group, the stage-1 weight included, is loaded at entry (one
// memory round trip); the BitLinear norm weights of the thread's units are loaded before the
// second norm chain (projection 0) or while the previous projection is encoded, so their
// latency hides behind work -- or, with PW (a few rows per launch: a launch is one row's
// latency), at entry too. Arithmetic and order are those of k_prologue.
template <int MODE, int PRE, int NA, int MAXG, bool PW, int BT>
__global__ __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(rowpro_waves<MODE, PRE, NA, MAXG, BT>())))
void k_rowpro(PrologueArgs a, ActBuf act) {
  extern __shared__ float smem[];
  constexpr bool SW = PRE == kPreSwish || PRE == kPreMixSwish, MIX = PRE == kPreMixSwish;
  constexpr int NX = SW ? 2 : 1;  // x, and x2 for the swish gate
  constexpr bool PWG = PRE != kPreNone;  // the stage-1 weight is loaded at entry with the row
  const int row = xcd_row(blockIdx.x);
  if (row >= act.rows) return;
  const int Lc = act.Lc, K = act.K, K8 = act.K8, nb = act.nb, nt = act.ntail, L8 = Lc / 8;
  const int G = nb + (nt > 0 ? 1 : 0);
  const int LS = lds_stride(Lc);
  const int tid = threadIdx.x;
  float* X = smem;
  float* S = SW ? X + 8 * LS + 8 : X;  // silu(x2), g_norm only
  float* red = S + 8 * LS + 8;         // 32 floats: the chain partials, then two block-max areas
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  // unit u -> chain j = u / L8 and first position t0: j by a multiply-high with
  // mL8 = ceil(2^32 / L8), exact while u * L8 < 2^32 (here u < Lc <= 2048, L8 >= 2)
  const uint32_t mL8 = 0xFFFFFFFFu / static_cast<uint32_t>(L8) + 1u;
  auto unit_jt = [&](int u, int& j, int& t0) {
    j = static_cast<int>(__umulhi(static_cast<uint32_t>(u), mL8));
    t0 = 8 * (u - j * L8);
  };
  // elements 8t .. 8t+7 of a K-long vector: two float4, or for the tail group one and zeros
  // (the tail group's second load repeats its first, an address in bounds, and is replaced by
  // zeros: a select of values, not of addresses)
  auto ld8 = [&](const float* p, int t, float4* o) {
    const float4* p4 = reinterpret_cast<const float4*>(p) + 2 * t;
    const float4 h = p4[t < nb ? 1 : 0];
    o[0] = p4[0];
    o[1] = t < nb ? h : z4;
  };
  const size_t rK = static_cast<size_t>(row) * K;

  float4 v[NX][MAXG][2];
  float4 pw[PWG ? MAXG : 1][2];
  float4 fv[MIX ? MAXG : 1][2], sv[MIX ? MAXG : 1][2], lv[MIX ? MAXG : 1][2];
  float4 nwv[PW ? NA : 1][PW ? MAXG : 1][2];
#pragma unroll
  for (int g = 0; g < MAXG; ++g) {
    const int t = tid + g * BT;
    if (t < G) {
#pragma unroll
      for (int vi = 0; vi < NX; ++vi) ld8((vi ? a.x2 : a.x) + rK, t, v[vi][g]);
      if constexpr (PWG) ld8(a.pre_w, t, pw[g]);
      if constexpr (MIX) {
        ld8(a.mix_f + rK, t, fv[g]);
        ld8(a.mix_state + rK, t, sv[g]);
        if (a.mix_lb) ld8(a.mix_lb, t, lv[g]);
        else lv[g][0] = lv[g][1] = z4;
      }
    }
    if constexpr (PW) {
      const int u = tid + g * BT;
      if (u < Lc) {
        int j, t0;
        unit_jt(u, j, t0);
#pragma unroll
        for (int ai = 0; ai < NA; ++ai) {
          const float4* wp = reinterpret_cast<const float4*>(a.normwT[ai] + j * Lc + t0);
          nwv[ai][g][0] = wp[0];
          nwv[ai][g][1] = wp[1];
        }
      }
    }
  }

  // the groups into the chain-transposed LDS rows (and silu(x2) for the swish gate)
#pragma unroll
  for (int g = 0; g < MAXG; ++g) {
    const int t = tid + g * BT;
    if (t >= G) continue;
    float xs[8], x2s[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      xs[c] = f4el(v[0][g][c >> 2], c & 3);
      x2s[c] = f4el(v[NX - 1][g][c >> 2], c & 3);
    }
    if constexpr (MIX) {
      // the recurrence step of k_mixer (stream_state), element for element; the swiglu and
      // sigmoid tail rule counts over all rows x K elements
      const size_t e0 = rK + 8 * static_cast<size_t>(t);
      const size_t body = (static_cast<size_t>(act.rows) * K) & ~static_cast<size_t>(7);
      float st[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const bool tail = e0 + c >= body;
        const float lb = f4el(lv[g][c >> 2], c & 3);
        float f = sigmoid_of(f4el(fv[g][c >> 2], c & 3), tail);
        if (a.mix_lb) f = __builtin_fmaf(1.0f - lb, f, lb);
        const float in = swiglu_of(x2s[c], 1.0f - f, tail);
        st[c] = __builtin_fmaf(f, f4el(sv[g][c >> 2], c & 3), in);
      }
      float4* so = reinterpret_cast<float4*>(a.mix_state + rK) + 2 * t;
      so[0] = make_float4(st[0], st[1], st[2], st[3]);
      if (t < nb) so[1] = make_float4(st[4], st[5], st[6], st[7]);
#pragma unroll
      for (int c = 0; c < 8; ++c) x2s[c] = st[c];
    }
    if (t < nb) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        X[c * LS + t] = xs[c];
        if (SW) S[c * LS + t] = silu_of(x2s[c], false);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (c < nt) {
          X[8 * LS + c] = xs[c];
          if (SW) S[8 * LS + c] = silu_of(x2s[c], true);
        }
      }
    }
  }
  const int L32 = (Lc + 31) / 32 * 32;
  for (int jr = 0; jr < 8; ++jr)
    for (int t = nb + tid; t < L32; t += BT) X[jr * LS + t] = 0.0f;
  for (int t = nt + tid; t < 8; t += BT) X[8 * LS + t] = 0.0f;
  __syncthreads();

  // the chain wave (wave 0) issues ahead of the other rows' waves on its SIMD until both
  // norms are known
  if (tid < 64) __builtin_amdgcn_s_setprio(3);
  if (PRE != kPreNone) {
    const float r1 = rstd_of(block_sumsq_ring(X, Lc, LS, nt, red), K, a.eps);
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const int t = tid + g * BT;
      if (t >= G) continue;
      const float4* w = pw[g];
      const int nc = t < nb ? 8 : nt;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (c < nc) {
          const int p = t < nb ? c * LS + t : 8 * LS + c;
          float x = (f4el(v[0][g][c >> 2], c & 3) * r1) * f4el(w[c >> 2], c & 3);
          if (SW) x = x * S[p];
          X[p] = x;
        }
      }
    }
    __syncthreads();
  }
  // the norm weights of the units: projection ai into set ai % 2 (not PW)
  float4 wq[PW ? 1 : 2][PW ? 1 : MAXG][2];
  auto load_w = [&](int ai, int set) {
    if constexpr (!PW) {
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        const int u = tid + g * BT;
        if (u >= Lc) continue;
        int j, t0;
        unit_jt(u, j, t0);
        const float4* wp = reinterpret_cast<const float4*>(a.normwT[ai] + j * Lc + t0);
        wq[set][g][0] = wp[0];
        wq[set][g][1] = wp[1];
      }
    }
  };
  load_w(0, 0);
  const float r2 = rstd_of(block_sumsq_ring(X, Lc, LS, nt, red), K, a.eps);
  if (tid < 64) __builtin_amdgcn_s_setprio(0);

  // the BitLinear norm of unit g: y = (x * rstd) * normw (bitlinear.cpp:62-70)
  auto unit_y = [&](int ai, int g, float* y) {
    const int u = tid + g * BT;
    int j, t0;
    unit_jt(u, j, t0);
    const float4* xp = reinterpret_cast<const float4*>(X + j * LS + t0);
    const float4 x0 = xp[0], x1 = xp[1];
    float4 w0, w1;
    if constexpr (PW) {
      w0 = nwv[ai][g][0];
      w1 = nwv[ai][g][1];
    } else {
      w0 = wq[ai & 1][g][0];
      w1 = wq[ai & 1][g][1];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      y[c] = (f4el(x0, c) * r2) * f4el(w0, c);
      y[4 + c] = (f4el(x1, c) * r2) * f4el(w1, c);
    }
  };
#pragma unroll
  for (int ai = 0; ai < NA; ++ai) {
    if (ai + 1 < NA) load_w(ai + 1, (ai + 1) & 1);
    const size_t ar = static_cast<size_t>(ai) * act.rows + row;
    float* yo = act.y + ar * act.ystride();
    int8_t* q = act.q + act.qoff(ai, 0, row, 0);  // plane 0 of this row; plane 1 at + qplane
    const size_t lop = act.qplane();
    // unit g's eight values out: padding positions (t >= nb) as zeros in every plane
    auto unit_out = [&](int g, const float* y, float sa) {
      const int u = tid + g * BT;
      int j, t0;
      unit_jt(u, j, t0);
      const int nv = nb - t0;
      if (MODE == kFloat) {
        float o[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = c < nv ? y[c] : 0.0f;
        float4* yp = reinterpret_cast<float4*>(yo + j * Lc + t0);
        yp[0] = make_float4(o[0], o[1], o[2], o[3]);
        yp[1] = make_float4(o[4], o[5], o[6], o[7]);
      } else {
        int32_t cd[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) cd[c] = (MODE == kFixed) ? q510_body(y[c], a.qs) : q8_of(y[c], sa);
        uint32_t h0, h1, l0 = 0, l1 = 0;
        if (MODE == kFixed) {
          pack_split4(cd, h0, l0);
          pack_split4(cd + 4, h1, l1);
        } else {
          h0 = pack_low4(cd);
          h1 = pack_low4(cd + 4);
        }
        // (Int8Absmax padding codes are 0 already: zero x and normw give y = 0, or NaN -> 0)
        if (MODE == kFixed && nv < 8) {
          const uint32_t m0 = nv >= 4 ? ~0u : (nv <= 0 ? 0u : (1u << (8 * nv)) - 1u);
          const uint32_t m1 = nv <= 4 ? 0u : (1u << (8 * (nv - 4))) - 1u;
          h0 &= m0;
          h1 &= m1;
          l0 &= m0;
          l1 &= m1;
        }
        const size_t o = ActBuf::qpos(j * Lc + t0);
        *reinterpret_cast<uint2*>(q + o) = make_uint2(h0, h1);
        if (MODE == kFixed) *reinterpret_cast<uint2*>(q + lop + o) = make_uint2(l0, l1);
      }
    };
    // the tail elements, one per lane c < ntail
    float yt = 0.0f;
    if (tid < nt) yt = (X[8 * LS + tid] * r2) * a.normw[ai][K8 + tid];
    float sa = 0.0f;
    if constexpr (MODE == kInt8) {
      // absmax over the row first (the padding contributes zeros)
      float y[MAXG][8];
      float m = tid < nt ? fabsf(yt) : 0.0f;
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        if (tid + g * BT >= Lc) continue;
        unit_y(ai, g, y[g]);
#pragma unroll
        for (int c = 0; c < 8; ++c) m = fmaxf(m, fabsf(y[g][c]));
      }
      m = block_max1<BT / 64>(m, red + 16 * (ai & 1));
      sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
      if (tid == 0) act.sa[ar] = sa;
#pragma unroll
      for (int g = 0; g < MAXG; ++g)
        if (tid + g * BT < Lc) unit_out(g, y[g], sa);
    } else {
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        if (tid + g * BT >= Lc) continue;
        float y[8];
        unit_y(ai, g, y);
        unit_out(g, y, 0.0f);
      }
    }
    if (tid < 8) {
      if (MODE == kFloat) yo[8 * Lc + tid] = tid < nt ? yt : 0.0f;
      else act.ct[ar * 8 + tid] = tid < nt ? ((MODE == kFixed) ? q510_tail(yt, a.qs) : q8_of(yt, sa)) : 0;
    }
  }
}

// The row prologue of long rows without a stage-1 norm (the MLP down projection's input,
// K = 5632 or 6912: 3 or 4 groups per thread), with half of the row in LDS at a time. The
// whole chain-transposed row takes 8 * (Lc + 4) floats (22.7 KB at K = 5632): 7 rows per CU,
// so 2048 rows need two rounds. Here LDS holds positions [0, 512) (pass A: groups g < 2) and
// then positions [512, Lc) (pass B): 16.7 KB, 8 rows per CU, one round. Each thread keeps its
// groups in registers from the entry loads:
//  - thread j < 8 sums chain j over pass A, and after the LDS holds pass B continues from the
//    same running sum (the reference's order and rounding, as in k_rowpro);
//  - the units of pass B are encoded from LDS, then pass A goes back into LDS and its units
//    are encoded.
// Unit, group and output layouts and the arithmetic are k_rowpro's (kPreNone, one
// projection). Needs nb >= 512 and 256 * MAXG >= max(Lc, G). Float and FixedQ510 only:
// 20.6 / 21.2 us against k_rowpro's 23.2 / 23.5 us at 2048 x 5632. (Int8Absmax, whose row
// maximum must precede every code, measured 23.5 us against 20.7: a second pass over both
// halves or the maximum from registers with spills.)
template <int MODE, int MAXG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MAXG == 3 ? 8 : 1)))
void k_rowpro_split(PrologueArgs a, ActBuf act) {
  static_assert(MODE == kFloat || MODE == kFixed, "Int8Absmax needs the row maximum first: k_rowpro");
  constexpr int BT = 256, P = 2 * BT;  // pass B starts at position P
  extern __shared__ float smem[];
  const int row = xcd_row(blockIdx.x);
  if (row >= act.rows) return;
  const int Lc = act.Lc, K = act.K, K8 = act.K8, nb = act.nb, nt = act.ntail, L8 = Lc / 8;
  const int G = nb + (nt > 0 ? 1 : 0);
  const int LS = lds_stride(P > Lc - P ? P : Lc - P);
  const int tid = threadIdx.x;
  float* X = smem;
  float* red = X + 8 * LS + 8;  // chain partials [0, 8); block maximum [16, 32)
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  auto ld8 = [&](const float* p, int t, float4* o) {
    const float4* p4 = reinterpret_cast<const float4*>(p) + 2 * t;
    const float4 h = p4[t < nb ? 1 : 0];
    o[0] = p4[0];
    o[1] = t < nb ? h : z4;
  };
  const uint32_t mL8 = 0xFFFFFFFFu / static_cast<uint32_t>(L8) + 1u;  // as in k_rowpro
  auto unit_jt = [&](int u, int& j, int& t0) {
    j = static_cast<int>(__umulhi(static_cast<uint32_t>(u), mL8));
    t0 = 8 * (u - j * L8);
  };

  float4 v[MAXG][2];
#pragma unroll
  for (int g = 0; g < MAXG; ++g)
    if (tid + g * BT < G) ld8(a.x + static_cast<size_t>(row) * K, tid + g * BT, v[g]);
  // groups [g0, g1) into the LDS rows at position t - base (the tail group to the tail slots)
  auto put = [&](int g0, int g1, int base) {
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const int t = tid + g * BT;
      if (g < g0 || g >= g1 || t >= G) continue;
      if (t < nb) {
#pragma unroll
        for (int c = 0; c < 8; ++c) X[c * LS + t - base] = f4el(v[g][c >> 2], c & 3);
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (c < nt) X[8 * LS + c] = f4el(v[g][c >> 2], c & 3);
      }
    }
  };
  put(0, 2, 0);
  __syncthreads();
  if (tid < 64) __builtin_amdgcn_s_setprio(3);
  float acc = 0.0f;
  if (tid < 8) acc = chain_ring_part(X, P, LS, 0.0f);
  __syncthreads();
  // pass B into LDS: its groups, rows zero from nb - P to a multiple of 32, the tail slots
  auto fill_b = [&]() {
    put(2, MAXG, P);
    const int LB = (Lc - P + 31) / 32 * 32;
    for (int jr = 0; jr < 8; ++jr)
      for (int t = nb - P + tid; t < LB; t += BT) X[jr * LS + t] = 0.0f;
    for (int t = nt + tid; t < 8; t += BT) X[8 * LS + t] = 0.0f;
  };
  fill_b();
  __syncthreads();
  if (tid < 8) red[tid] = chain_ring_part(X, Lc - P, LS, acc);
  __syncthreads();
  const float r2 = rstd_of(chain_end(X, LS, nt, red), K, a.eps);
  if (tid < 64) __builtin_amdgcn_s_setprio(0);

  // the norm weights of the thread's units (chain-transposed)
  float4 wq[MAXG][2];
  auto load_w = [&]() {
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const int u = tid + g * BT;
      if (u >= Lc) continue;
      int j, t0;
      unit_jt(u, j, t0);
      const float4* wp = reinterpret_cast<const float4*>(a.normwT[0] + j * Lc + t0);
      wq[g][0] = wp[0];
      wq[g][1] = wp[1];
    }
  };
  load_w();
  float* yo = act.y + static_cast<size_t>(row) * act.ystride();
  int8_t* q = act.q + act.qoff(0, 0, row, 0);  // plane 0 of this row; plane 1 at + qplane
  const size_t lop = act.qplane();
  // unit g's normed values y = (x * rstd) * normw (bitlinear.cpp:62-70) from LDS position
  // t0 - base of row j
  auto unit_y = [&](int g, int j, int t0, int base, float* y) {
    const float4* xp = reinterpret_cast<const float4*>(X + j * LS + t0 - base);
    const float4 x0 = xp[0], x1 = xp[1];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      y[c] = (f4el(x0, c) * r2) * f4el(wq[g][0], c);
      y[4 + c] = (f4el(x1, c) * r2) * f4el(wq[g][1], c);
    }
  };
  // the units whose positions lie in [lo, hi), read from LDS at position t0 - base
  auto encode = [&](int lo, int hi, int base) {
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const int u = tid + g * BT;
      if (u >= Lc) continue;
      int j, t0;
      unit_jt(u, j, t0);
      if (t0 < lo || t0 >= hi) continue;
      float y[8];
      unit_y(g, j, t0, base, y);
      const int nv = nb - t0;
      if (MODE == kFloat) {
        float o[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = c < nv ? y[c] : 0.0f;
        float4* yp = reinterpret_cast<float4*>(yo + j * Lc + t0);
        yp[0] = make_float4(o[0], o[1], o[2], o[3]);
        yp[1] = make_float4(o[4], o[5], o[6], o[7]);
      } else {
        int32_t cd[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) cd[c] = q510_body(y[c], a.qs);
        uint32_t h0, h1, l0, l1;
        pack_split4(cd, h0, l0);
        pack_split4(cd + 4, h1, l1);
        if (nv < 8) {
          const uint32_t m0 = nv >= 4 ? ~0u : (nv <= 0 ? 0u : (1u << (8 * nv)) - 1u);
          const uint32_t m1 = nv <= 4 ? 0u : (1u << (8 * (nv - 4))) - 1u;
          h0 &= m0;
          h1 &= m1;
          l0 &= m0;
          l1 &= m1;
        }
        const size_t o = ActBuf::qpos(j * Lc + t0);
        *reinterpret_cast<uint2*>(q + o) = make_uint2(h0, h1);
        *reinterpret_cast<uint2*>(q + lop + o) = make_uint2(l0, l1);
      }
    }
  };
  // the tail elements, one per lane c < ntail (in the LDS tail slots from pass B on)
  if (tid < 8) {
    const float yt = tid < nt ? (X[8 * LS + tid] * r2) * a.normw[0][K8 + tid] : 0.0f;
    if (MODE == kFloat) yo[8 * Lc + tid] = yt;
    else act.ct[static_cast<size_t>(row) * 8 + tid] = tid < nt ? q510_tail(yt, a.qs) : 0;
  }
  encode(P, Lc, P);
  __syncthreads();
  put(0, 2, 0);
  __syncthreads();
  encode(0, P, 0);
}

// The row prologue of a few rows at the model widths (K = 256 RC: no tail, no padding) for
// the stage kinds without element-wise work (kPreNorm, kPreNone): one wave per projection
// (NA waves per row) and no wait on other blocks. The waves load the row coalesced (float4
// q = l + 64 k, a share of the k each) and turn it through LDS into the lane-segment layout
// of the register chains: lane 8j + s holds steps [4 RC s, 4 RC (s + 1)) of chain j, i.e.
// chain-transposed floats [4 RC l, 4 RC (l + 1)), the layout in which the stage-1 weight
// pre_wT and the norm weights normwT are stored. Every wave then runs both order-fixed norm
// chains from registers (seg_sumsq: one dependent FMA per step and a DPP shift between
// segments; the same chains in every wave, side by side on the CU's SIMDs) and encodes its
// own projection, whose norm weights it loads at entry. Arithmetic and order are those of
// k_rowpro. (One wave encoding all three i/f/g projections: 6.9 us per launch at hidden
// 2560 and 64 rows, against 6.0 us with a wave each; splitting one projection's steps over
// two waves measured no faster. The swish-gate kinds run in k_rowseg_sw: their silu, sigmoid
// and swiglu per element on one wave per row measured 13.8 us against k_rowpro's 10.7 us for
// 64 rows at K = 2560.)
template <int MODE, int PRE, int NA, int RC>
__global__ __launch_bounds__(64 * NA) void k_rowseg(PrologueArgs a, ActBuf act) {
  static_assert(PRE == kPreNorm || PRE == kPreNone, "element-wise stage kinds run in k_rowpro");
  constexpr int W = NA;
  constexpr int Lc = 32 * RC, K = 8 * Lc, LS = Lc + 4;
  constexpr int KW = (RC + W - 1) / W;  // row float4 per lane per wave at entry
  __shared__ float X[8 * LS];
  const int row = xcd_row(blockIdx.x);
  if (row >= act.rows) return;
  const int lane = threadIdx.x & 63;
  // this wave's projection (a compile-time 0 with one projection: no run-time guards)
  const int ai = (NA > 1) ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6) : 0;
  const int wv = ai;
  const float4* xr = reinterpret_cast<const float4*>(a.x + static_cast<size_t>(row) * K);

  // entry loads: this wave's share of the row (natural layout), the stage-1 weight and,
  // with several projections, the norm weights of its own (segment layout; one projection
  // loads them after the chains: at entry, 40 more registers in flight measured 0.5 us
  // slower)
  float4 nx[KW];
#pragma unroll
  for (int k = 0; k < KW; ++k)
    if (wv * KW + k < RC) nx[k] = xr[lane + 64 * (wv * KW + k)];
  float4 ws[PRE != kPreNone ? RC : 1];
  if constexpr (PRE != kPreNone) {
#pragma unroll
    for (int c = 0; c < RC; ++c) ws[c] = reinterpret_cast<const float4*>(a.pre_wT)[lane * RC + c];
  }
  float4 nw[NA > 1 ? RC : 1];
  if constexpr (NA > 1) {
#pragma unroll
    for (int c = 0; c < RC; ++c) nw[c] = reinterpret_cast<const float4*>(a.normwT[ai])[lane * RC + c];
  }
  // natural float4 q holds elements 4q .. 4q+3: step q / 2 of chains 4 (q % 2) .. 4 (q % 2) + 3
#pragma unroll
  for (int k = 0; k < KW; ++k) {
    if (wv * KW + k < RC) {
      const int q = lane + 64 * (wv * KW + k), t = q >> 1, j0 = 4 * (q & 1);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[(j0 + c) * LS + t] = f4el(nx[k], c);
    }
  }
  __syncthreads();
  const int j = lane >> 3, sg = lane & 7;
  float4 xs[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c) xs[c] = reinterpret_cast<const float4*>(X + j * LS + 4 * RC * sg)[c];
  const float zt[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (PRE != kPreNone) {
    const float r1 = rstd_of(seg_sumsq<RC>(xs, zt, 0), K, a.eps);
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      float4 x = xs[c];
      const float4 w = ws[c];
      x.x = (x.x * r1) * w.x; x.y = (x.y * r1) * w.y; x.z = (x.z * r1) * w.z; x.w = (x.w * r1) * w.w;
      xs[c] = x;
    }
  }
  const float r2 = rstd_of(seg_sumsq<RC>(xs, zt, 0), K, a.eps);

  const size_t ar = static_cast<size_t>(ai) * act.rows + row;
  float4 y[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const float4 w = (NA > 1) ? nw[c] : reinterpret_cast<const float4*>(a.normwT[ai])[lane * RC + c];
    const float4 x = xs[c];
    y[c] = make_float4((x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w);
  }
  if constexpr (MODE == kFloat) {
    float* yo = act.y + ar * act.ystride();
#pragma unroll
    for (int c = 0; c < RC; ++c) reinterpret_cast<float4*>(yo)[lane * RC + c] = y[c];
    if (lane < 8) yo[8 * Lc + lane] = 0.0f;
  } else {
    float sa = 0.0f;
    if constexpr (MODE == kInt8) {
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < RC; ++c)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(y[c].x), fabsf(y[c].y)), fmaxf(fabsf(y[c].z), fabsf(y[c].w))));
      m = wave_max(m);
      sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
      if (lane == 0) act.sa[ar] = sa;
    }
    int8_t* q = act.q + act.qoff(ai, 0, row, 0);
    const size_t lop = act.qplane();
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      int32_t cd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) cd[e] = (MODE == kFixed) ? q510_body(f4el(y[c], e), a.qs) : q8_of(f4el(y[c], e), sa);
      const size_t o = ActBuf::qpos(4 * (lane * RC + c));
      if constexpr (MODE == kFixed) {
        uint32_t h, l;
        pack_split4(cd, h, l);
        *reinterpret_cast<uint32_t*>(q + o) = h;
        *reinterpret_cast<uint32_t*>(q + lop + o) = l;
      } else {
        *reinterpret_cast<uint32_t*>(q + o) = pack_low4(cd);
      }
    }
    if (lane < 8) act.ct[ar * 8 + lane] = 0;
  }
}

// The swish-gate row prologues (kPreSwish, and kPreMixSwish with the recurrence step of
// independent streams) of a few rows at the model widths, one 1024-thread block per row: all
// 16 waves do the element-wise work in natural layout, one float4 per thread (the step's
// sigmoid, swiglu and state update, then silu of the gate input), and write the row and the
// gate into LDS in the lane-segment layout of the register chains; wave 0 then runs both
// order-fixed norm chains from registers (seg_sumsq) and encodes its segments, as k_rowseg.
// Arithmetic and order are those of k_rowpro (K % 8 == 0: no element is in the reference's
// scalar tail).
template <int MODE, int PRE, int RC>
__global__ __launch_bounds__(1024) void k_rowseg_sw(PrologueArgs a, ActBuf act) {
  static_assert(PRE == kPreSwish || PRE == kPreMixSwish, "the swish-gate kinds");
  constexpr bool MIX = PRE == kPreMixSwish;
  constexpr int Lc = 32 * RC, K = 8 * Lc, LS = Lc + 4, NQ = K / 4;
  __shared__ float X[8 * LS], S[8 * LS];
  const int row = xcd_row(blockIdx.x);
  if (row >= act.rows) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const size_t rK = static_cast<size_t>(row) * K;
  // wave 0: the stage-1 weight's segments (needed after the LDS round)
  float4 ws[RC];
  if (tid < 64) {
#pragma unroll
    for (int c = 0; c < RC; ++c) ws[c] = reinterpret_cast<const float4*>(a.pre_wT)[lane * RC + c];
  }
  for (int q = tid; q < NQ; q += 1024) {
    const float4 xv = reinterpret_cast<const float4*>(a.x + rK)[q];
    float4 gv = reinterpret_cast<const float4*>(a.x2 + rK)[q];
    if constexpr (MIX) {
      const float4 fv = reinterpret_cast<const float4*>(a.mix_f + rK)[q];
      const float4 sv = reinterpret_cast<const float4*>(a.mix_state + rK)[q];
      const float4 lv = a.mix_lb ? reinterpret_cast<const float4*>(a.mix_lb)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      float st[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float f = sigmoid_of(f4el(fv, c), false);
        if (a.mix_lb) {
          const float lb = f4el(lv, c);
          f = __builtin_fmaf(1.0f - lb, f, lb);
        }
        const float in = swiglu_of(f4el(gv, c), 1.0f - f, false);
        st[c] = __builtin_fmaf(f, f4el(sv, c), in);
      }
      gv = make_float4(st[0], st[1], st[2], st[3]);
      reinterpret_cast<float4*>(a.mix_state + rK)[q] = gv;
    }
    // natural float4 q holds elements 4q .. 4q+3: step q / 2 of chains 4 (q % 2) .. + 3
    const int t = q >> 1, j0 = 4 * (q & 1);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      X[(j0 + c) * LS + t] = f4el(xv, c);
      S[(j0 + c) * LS + t] = silu_of(f4el(gv, c), false);
    }
  }
  __syncthreads();
  if (tid >= 64) return;
  const int j = lane >> 3, sg = lane & 7;
  float4 xs[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c) xs[c] = reinterpret_cast<const float4*>(X + j * LS + 4 * RC * sg)[c];
  const float zt[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const float r1 = rstd_of(seg_sumsq<RC>(xs, zt, 0), K, a.eps);
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    float4 x = xs[c];
    const float4 w = ws[c];
    const float4 g = reinterpret_cast<const float4*>(S + j * LS + 4 * RC * sg)[c];
    x.x = ((x.x * r1) * w.x) * g.x; x.y = ((x.y * r1) * w.y) * g.y;
    x.z = ((x.z * r1) * w.z) * g.z; x.w = ((x.w * r1) * w.w) * g.w;
    xs[c] = x;
  }
  const float r2 = rstd_of(seg_sumsq<RC>(xs, zt, 0), K, a.eps);
  const size_t ar = row;  // one projection
  float4 y[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const float4 w = reinterpret_cast<const float4*>(a.normwT[0])[lane * RC + c];
    const float4 x = xs[c];
    y[c] = make_float4((x.x * r2) * w.x, (x.y * r2) * w.y, (x.z * r2) * w.z, (x.w * r2) * w.w);
  }
  if constexpr (MODE == kFloat) {
    float* yo = act.y + ar * act.ystride();
#pragma unroll
    for (int c = 0; c < RC; ++c) reinterpret_cast<float4*>(yo)[lane * RC + c] = y[c];
    if (lane < 8) yo[8 * Lc + lane] = 0.0f;
  } else {
    float sa = 0.0f;
    if constexpr (MODE == kInt8) {
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < RC; ++c)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(y[c].x), fabsf(y[c].y)), fmaxf(fabsf(y[c].z), fabsf(y[c].w))));
      m = wave_max(m);
      sa = 127.0f / (m > 1e-5f ? m : 1e-5f);
      if (lane == 0) act.sa[ar] = sa;
    }
    int8_t* q = act.q + act.qoff(0, 0, row, 0);
    const size_t lop = act.qplane();
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      int32_t cd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) cd[e] = (MODE == kFixed) ? q510_body(f4el(y[c], e), a.qs) : q8_of(f4el(y[c], e), sa);
      const size_t o = ActBuf::qpos(4 * (lane * RC + c));
      if constexpr (MODE == kFixed) {
        uint32_t h, l;
        pack_split4(cd, h, l);
        *reinterpret_cast<uint32_t*>(q + o) = h;
        *reinterpret_cast<uint32_t*>(q + lop + o) = l;
      } else {
        *reinterpret_cast<uint32_t*>(q + o) = pack_low4(cd);
      }
    }
    if (lane < 8) act.ct[ar * 8 + lane] = 0;
  }
}

// int16-range codes -> split planes (the TernaryBackend path: codes arrive quantised)
__global__ void k_codes(const int32_t* __restrict__ x, ActBuf act) {
  const int row = xcd_row(blockIdx.x), Lc = act.Lc, nb = act.nb;
  if (row >= act.rows) return;
  const int32_t* xr = x + static_cast<size_t>(row) * act.K;
  int8_t* q = act.q + act.qoff(0, 0, row, 0);
  const size_t lop = act.qplane();
  for (int j = 0; j < 8; ++j)
    for (int t4 = threadIdx.x * 4; t4 < Lc; t4 += blockDim.x * 4) {
      uint32_t hi = 0, lo = 0;
      for (int u = 0; u < 4; ++u) {
        const int t = t4 + u;
        if (t < nb) {
          const int32_t c = xr[j + 8 * t];
          hi |= static_cast<uint32_t>((c >> 8) & 0xFF) << (8 * u);
          lo |= static_cast<uint32_t>(((c & 0xFF) - 128) & 0xFF) << (8 * u);
        }
      }
      *reinterpret_cast<uint32_t*>(q + ActBuf::qpos(j * Lc + t4)) = hi;
      *reinterpret_cast<uint32_t*>(q + lop + ActBuf::qpos(j * Lc + t4)) = lo;
    }
  for (int t = threadIdx.x; t < 8; t += blockDim.x)
    act.ct[static_cast<size_t>(row) * 8 + t] = (t < act.ntail) ? xr[act.K8 + t] : 0;
}

// planes -> int32 codes [na][rows][K] in natural element order (the inverse of k_codes, for
// an external TernaryBackend): FixedQ510 code = 256 * hi + lo + 128, Int8Absmax code = the
// plane-0 byte; the tail codes come from ct. One block per (row, projection).
__global__ void k_planes_to_codes(ActBuf act, int mode, int32_t* __restrict__ codes) {
  const int row = xcd_row(blockIdx.x), ai = blockIdx.y, Lc = act.Lc;
  if (row >= act.rows) return;
  const int8_t* q = act.q + act.qoff(ai, 0, row, 0);
  const size_t lop = act.qplane();
  const size_t ar = static_cast<size_t>(ai) * act.rows + row;
  int32_t* out = codes + ar * act.K;
  for (int k = threadIdx.x; k < act.K8; k += blockDim.x) {
    const size_t o = ActBuf::qpos((k & 7) * Lc + (k >> 3));
    const int hi = q[o];
    out[k] = mode == kFixed ? hi * 256 + static_cast<int>(q[lop + o]) + 128 : hi;
  }
  for (int t = threadIdx.x; t < act.ntail; t += blockDim.x) out[act.K8 + t] = act.ct[ar * 8 + t];
}

// ------------------------------------------------------------------------------------
// Ternary GEMM over row tiles. Block = 16 outputs x 8 chains; R rows per block; the
// activations of one chunk of MW words per chain are staged in LDS for all R rows.
// PAIR: the block computes rows o and o + N/2 of one matrix (the MLP gate/up halves,
// hgrn_model.cpp:171-185) and applies swiglu in the epilogue.
// ------------------------------------------------------------------------------------
constexpr int kMW = 8;  // words per chain per LDS chunk

template <int MODE, int R, bool PAIR>
__global__ __launch_bounds__(kBlock) void k_gemm(GemmArgs a, ActBuf act) {
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc;
  const int tid = threadIdx.x, ol = tid >> 3, j = tid & 7;
  const int og = blockIdx.x;
  const int row0 = blockIdx.y * R;
  const int nrows = min(R, a.rows - row0);
  const int ai = (act.na > 1) ? z : 0;
  constexpr int NM = PAIR ? 2 : 1;
  const int half_groups = g.ngroups / 2;  // PAIR: N/2 is a multiple of 16
  const uint32_t* slab[NM];
  slab[0] = P.pk + static_cast<size_t>(og) * g.Wc * 128 + ol * 8 + j;
  if (PAIR) slab[NM - 1] = P.pk + static_cast<size_t>(og + half_groups) * g.Wc * 128 + ol * 8 + j;

  float facc[NM][R];
  int32_t iacc[NM][R], lacc[NM][R];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int r = 0; r < R; ++r) { facc[mi][r] = 0.0f; iacc[mi][r] = 0; lacc[mi][r] = 0; }

  for (int m0 = 0; m0 < g.Wc; m0 += kMW) {
    const int mw = min(kMW, g.Wc - m0);
    __syncthreads();
    // stage activations [r][chain][mw*16] of this chunk
    if (MODE == kFloat) {
      float* L = smem;
      const int per_row = 8 * mw * 16;
      for (int e = tid * 4; e < R * per_row; e += kBlock * 4) {
        const int r = e / per_row, rem = e - r * per_row, jj = rem / (mw * 16), t = rem - jj * mw * 16;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nrows)
          v = *reinterpret_cast<const float4*>(
              act.y + (static_cast<size_t>(ai) * act.rows + row0 + r) * act.ystride() + jj * Lc + m0 * 16 + t);
        *reinterpret_cast<float4*>(L + r * per_row + jj * mw * 16 + t) = v;
      }
    } else {
      uint32_t* L = reinterpret_cast<uint32_t*>(smem);
      const int np = (MODE == kFixed) ? 2 : 1;
      const int per_row = np * 8 * mw * 4;  // dwords
      for (int e = tid; e < R * per_row; e += kBlock) {
        const int r = e / per_row, rem = e - r * per_row, pl = rem / (8 * mw * 4),
                  rem2 = rem - pl * 8 * mw * 4, jj = rem2 / (mw * 4), d = rem2 - jj * mw * 4;
        uint32_t v = 0;
        if (r < nrows)
          v = *reinterpret_cast<const uint32_t*>(act.q + act.qoff(ai, pl, row0 + r, jj * Lc + m0 * 16 + d * 4));
        L[e] = v;
      }
    }
    __syncthreads();
    for (int mm = 0; mm < mw; ++mm) {
      const int m = m0 + mm;
      uint32_t w[NM];
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) w[mi] = slab[mi][static_cast<size_t>(m) * 128];
      if (MODE == kFloat) {
        const float* L = smem;
        const int per_row = 8 * mw * 16;
        float wf[NM][16];
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
#pragma unroll
          for (int t = 0; t < 16; ++t) wf[mi][t] = code_f(w[mi], t);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float* yl = L + r * per_row + j * mw * 16 + mm * 16;
          float y[16];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            float4 v = *reinterpret_cast<const float4*>(yl + 4 * q4);
            y[4 * q4] = v.x; y[4 * q4 + 1] = v.y; y[4 * q4 + 2] = v.z; y[4 * q4 + 3] = v.w;
          }
#pragma unroll
          for (int mi = 0; mi < NM; ++mi)
#pragma unroll
            for (int t = 0; t < 16; ++t) facc[mi][r] = __builtin_fmaf(y[t], wf[mi][t], facc[mi][r]);
        }
      } else {
        const uint32_t* L = reinterpret_cast<const uint32_t*>(smem);
        const int np = (MODE == kFixed) ? 2 : 1;
        const int per_row = np * 8 * mw * 4;
        uint32_t wv[NM][4];
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[mi][i] = w4_i8(w[mi], i);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint4 h = *reinterpret_cast<const uint4*>(L + r * per_row + j * mw * 4 + mm * 4);
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) {
            iacc[mi][r] = dot4(wv[mi][0], h.x, iacc[mi][r]);
            iacc[mi][r] = dot4(wv[mi][1], h.y, iacc[mi][r]);
            iacc[mi][r] = dot4(wv[mi][2], h.z, iacc[mi][r]);
            iacc[mi][r] = dot4(wv[mi][3], h.w, iacc[mi][r]);
          }
          if (MODE == kFixed) {
            const uint4 l = *reinterpret_cast<const uint4*>(L + r * per_row + 8 * mw * 4 + j * mw * 4 + mm * 4);
#pragma unroll
            for (int mi = 0; mi < NM; ++mi) {
              lacc[mi][r] = dot4(wv[mi][0], l.x, lacc[mi][r]);
              lacc[mi][r] = dot4(wv[mi][1], l.y, lacc[mi][r]);
              lacc[mi][r] = dot4(wv[mi][2], l.z, lacc[mi][r]);
              lacc[mi][r] = dot4(wv[mi][3], l.w, lacc[mi][r]);
            }
          }
        }
      }
    }
  }

  // reduce the 8 chains of each output and apply the epilogue
  const int Nout = PAIR ? g.N / 2 : g.N;
  const int o = og * kGroup + ol;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float val[NM];
    int32_t tot[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int oo = o + (mi ? Nout : 0);
      const size_t ar = static_cast<size_t>(ai) * act.rows + row0 + r;
      if (MODE == kFloat) {
        float s = hsum8_lanes(facc[mi][r]);
        if (j == 0 && r < nrows && oo < g.N) {
          const float* yt = act.y + ar * act.ystride() + 8 * Lc;
          for (int t = 0; t < g.ntail; ++t) {
            const int8_t wt = P.tail[oo * 8 + t];
            if (wt > 0) s += yt[t];
            else if (wt < 0) s -= yt[t];
          }
        }
        val[mi] = s * P.inv_scale_w;
        tot[mi] = 0;
      } else {
        int32_t s = isum8_lanes(iacc[mi][r]);
        if (MODE == kFixed) s = s * 256 + isum8_lanes(lacc[mi][r]);
        if (j == 0 && r < nrows && oo < g.N) {
          if (MODE == kFixed) s += 128 * P.rowsum[oo];
          const int32_t* ct = act.ct + ar * 8;
          for (int t = 0; t < g.ntail; ++t) s += static_cast<int32_t>(P.tail[oo * 8 + t]) * ct[t];
        }
        tot[mi] = s;
        if (MODE == kFixed) val[mi] = static_cast<float>(s) * a.inv_fixed[z];
        else if (j == 0 && r < nrows) val[mi] = static_cast<float>(s) / (P.scale_w * act.sa[ar]);
        else val[mi] = 0.0f;
      }
    }
    if (j != 0 || r >= nrows || o >= Nout) continue;
    const size_t grow = static_cast<size_t>(row0 + r);
    if (MODE != kFloat && a.acc[z]) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) a.acc[z][grow * g.N + o + (mi ? Nout : 0)] = tot[mi];
    }
    if (MODE != kFloat && a.raw_acc) continue;
    if (PAIR) {
      const size_t e = grow * Nout + o;
      a.out[0][e] = swiglu_of(val[0], val[NM - 1], static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
    } else if (a.epi == kEpiAdd) {
      const size_t e = grow * g.N + o;
      a.out[z][e] = a.add[e] + val[0];
    } else {
      a.out[z][grow * g.N + o] = val[0];
    }
  }
}

// ------------------------------------------------------------------------------------
// Float-mode ternary GEMM over row tiles, register-blocked over outputs. Block = 128 threads
// = 16 output lanes x 8 chains; thread (ol, j) runs chain j (the reference's AVX2 lane j,
// simd.hpp:92-122: fma(y_k, w_k, a) over k = j + 8t in t order) of NO outputs from NO
// slabs, for R rows. Activations of kFW words per chain are staged in LDS for the R rows,
// chain rows padded by 4 floats so the 8 chains of a wave hit distinct banks; each value
// read feeds NO FMAs and each weight word R x 16. PAIR: the first half of the slabs are
// gate outputs, the second half their up partners N/2 later (swiglu epilogue).
// ------------------------------------------------------------------------------------
constexpr int kFW = 4;                // words per chain per LDS chunk
constexpr int kFCS = kFW * 16 + 4;    // floats per staged chain row

template <int R, int NO, bool PAIR>
__global__ __launch_bounds__(128) void k_gemm_f(GemmArgs a, ActBuf act) {
  static_assert(!PAIR || NO % 2 == 0, "gate/up pairs need an even output count");
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc, Wc = g.Wc;
  const int tid = threadIdx.x, ol = tid >> 3, j = tid & 7;
  const int row0 = blockIdx.y * R;
  const int nrows = min(R, a.rows - row0);
  const int am = (act.na > 1) ? z : 0;
  const int half = g.ngroups / 2;
  int grp[NO];
  bool gok[NO];
#pragma unroll
  for (int s = 0; s < NO; ++s) {
    if (PAIR) {
      const int gg = blockIdx.x * (NO / 2) + (s % (NO / 2));
      gok[s] = gg < half;
      grp[s] = (s < NO / 2) ? gg : half + gg;
    } else {
      grp[s] = blockIdx.x * NO + s;
      gok[s] = grp[s] < g.ngroups;
    }
    if (!gok[s]) grp[s] = 0;
  }
  const uint32_t* slab[NO];
#pragma unroll
  for (int s = 0; s < NO; ++s) slab[s] = P.pk + static_cast<size_t>(grp[s]) * Wc * 128 + ol * 8 + j;
  float acc[NO][R];
#pragma unroll
  for (int s = 0; s < NO; ++s)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[s][r] = 0.0f;
  constexpr int PR = 8 * kFCS;  // LDS floats per staged row
  const float* ybase = act.y + (static_cast<size_t>(am) * act.rows + row0) * act.ystride();
  for (int m0 = 0; m0 < Wc; m0 += kFW) {
    const int mw = min(kFW, Wc - m0);
    uint32_t w[kFW][NO];
#pragma unroll
    for (int mm = 0; mm < kFW; ++mm)
#pragma unroll
      for (int s = 0; s < NO; ++s)
        w[mm][s] = (mm < mw && gok[s]) ? slab[s][static_cast<size_t>(m0 + mm) * 128] : 0u;
    __syncthreads();
    const int n4 = mw * 4;
    for (int e = tid; e < R * 8 * n4; e += 128) {
      const int r = e / (8 * n4), rem = e - r * 8 * n4, jj = rem / n4, q = rem - jj * n4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r < nrows)
        v = *reinterpret_cast<const float4*>(ybase + static_cast<size_t>(r) * act.ystride() + jj * Lc + m0 * 16 + q * 4);
      *reinterpret_cast<float4*>(smem + r * PR + jj * kFCS + q * 4) = v;
    }
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < kFW; ++mm) {
      if (mm >= mw) break;
      float wf[NO][16];
#pragma unroll
      for (int s = 0; s < NO; ++s)
#pragma unroll
        for (int t = 0; t < 16; ++t) wf[s][t] = code_f(w[mm][s], t);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float* yl = smem + r * PR + j * kFCS + mm * 16;
        float y[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 v = *reinterpret_cast<const float4*>(yl + 4 * q4);
          y[4 * q4] = v.x;
          y[4 * q4 + 1] = v.y;
          y[4 * q4 + 2] = v.z;
          y[4 * q4 + 3] = v.w;
        }
#pragma unroll
        for (int s = 0; s < NO; ++s)
#pragma unroll
          for (int t = 0; t < 16; ++t) acc[s][r] = __builtin_fmaf(y[t], wf[s][t], acc[s][r]);
      }
    }
  }
  // reduce the 8 chains of each output (hsum_ps order), tails, scale, epilogue
  const int Nout = PAIR ? g.N / 2 : g.N;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const size_t ar = static_cast<size_t>(am) * act.rows + row0 + r;
    float val[NO];
#pragma unroll
    for (int s = 0; s < NO; ++s) {
      float sum = hsum8_lanes(acc[s][r]);
      const int o = grp[s] * 16 + ol;
      if (j == 0 && r < nrows && gok[s] && o < g.N) {
        const float* yt = act.y + ar * act.ystride() + 8 * Lc;
        for (int t = 0; t < g.ntail; ++t) {
          const int8_t wt = P.tail[o * 8 + t];
          if (wt > 0) sum += yt[t];
          else if (wt < 0) sum -= yt[t];
        }
      }
      val[s] = sum * P.inv_scale_w;
    }
    if (j != 0 || r >= nrows) continue;
    const size_t grow = static_cast<size_t>(row0 + r);
    if (PAIR) {
#pragma unroll
      for (int s = 0; s < NO / 2; ++s) {
        const int o = grp[s] * 16 + ol;
        if (!gok[s] || o >= Nout) continue;
        const size_t e = grow * Nout + o;
        a.out[0][e] = swiglu_of(val[s], val[s + NO / 2], static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
      }
    } else {
#pragma unroll
      for (int s = 0; s < NO; ++s) {
        const int o = grp[s] * 16 + ol;
        if (!gok[s] || o >= g.N) continue;
        const size_t e = grow * g.N + o;
        a.out[z][e] = (a.epi == kEpiAdd) ? a.add[e] + val[s] : val[s];
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// HGRN gate + recurrence (hgrn_model.cpp:109-150)
// ------------------------------------------------------------------------------------
__global__ void k_mixer(const float* __restrict__ i, float* __restrict__ f, float* __restrict__ scan_out,
                        float* __restrict__ recur, float* __restrict__ state,
                        const float* __restrict__ lb, int rows, int H, int stream_state) {
  const int n = rows * H;  // the sigmoid / swiglu element count (tail rule)
  const int body = n & ~7;
  if (stream_state) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int c = e % H;
    float fv = sigmoid_of(f[e], e >= body);
    if (lb) fv = __builtin_fmaf(1.0f - lb[c], fv, lb[c]);
    const float in = swiglu_of(i[e], 1.0f - fv, e >= body);
    const float s = __builtin_fmaf(fv, state[e], in);
    state[e] = s;
    recur[e] = s;
    f[e] = fv;
    if (scan_out) scan_out[e] = in;
    return;
  }
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  float s = state[c];
  const float lbc = lb ? lb[c] : 0.0f;
  constexpr int U = 8;
  int t = 0;
  for (; t + U <= rows; t += U) {
    float iv[U], fv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      iv[u] = i[static_cast<size_t>(t + u) * H + c];
      fv[u] = f[static_cast<size_t>(t + u) * H + c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = (t + u) * H + c;
      float g = sigmoid_of(fv[u], e >= body);
      if (lb) g = __builtin_fmaf(1.0f - lbc, g, lbc);
      const float in = swiglu_of(iv[u], 1.0f - g, e >= body);
      s = __builtin_fmaf(g, s, in);
      recur[e] = s;
      f[e] = g;
      if (scan_out) scan_out[e] = in;
    }
  }
  for (; t < rows; ++t) {
    const int e = t * H + c;
    float g = sigmoid_of(f[e], e >= body);
    if (lb) g = __builtin_fmaf(1.0f - lbc, g, lbc);
    const float in = swiglu_of(i[e], 1.0f - g, e >= body);
    s = __builtin_fmaf(g, s, in);
    recur[e] = s;
    f[e] = g;
    if (scan_out) scan_out[e] = in;
  }
  state[c] = s;
}

// Time-scan prefill split in two: the gate math of every element in parallel, then the
// recurrence alone. k_gate: g = sigmoid(f) (then the lower bound), in = swiglu(i, 1 - g)
// over the whole [rows, H] buffer, whose element count sets the tail rule
// (hgrn_model.cpp:113-131). f is overwritten with g.
__global__ void k_gate(const float* __restrict__ i, float* __restrict__ f, float* __restrict__ scan_in,
                       const float* __restrict__ lb, int rows, int H) {
  const size_t n = static_cast<size_t>(rows) * H;
  const size_t body = n & ~static_cast<size_t>(7);
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    float g = sigmoid_of(f[e], e >= body);
    if (lb) {
      const float l = lb[e % H];
      g = __builtin_fmaf(1.0f - l, g, l);
    }
    scan_in[e] = swiglu_of(i[e], 1.0f - g, e >= body);
    f[e] = g;
  }
}

// The recurrence state = fma(g, state, in) (simd.hpp:335-357) down each column, in time
// order. One thread per column; the g and in values of the next kScanU steps are loaded
// while the current kScanU steps are computed.
constexpr int kScanU = 64;

__global__ __launch_bounds__(64) void k_scan_seq(const float* __restrict__ g, const float* __restrict__ in,
                                                 float* __restrict__ recur, float* __restrict__ state, int rows,
                                                 int H) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  float s = state[c];
  float gc[kScanU], ic[kScanU], gn[kScanU], inx[kScanU];
  auto load = [&](int t0, float* gd, float* id) {
#pragma unroll
    for (int u = 0; u < kScanU; ++u) {
      const int t = t0 + u < rows ? t0 + u : rows - 1;
      gd[u] = g[static_cast<size_t>(t) * H + c];
      id[u] = in[static_cast<size_t>(t) * H + c];
    }
  };
  load(0, gc, ic);
  for (int t0 = 0; t0 < rows; t0 += kScanU) {
    if (t0 + kScanU < rows) load(t0 + kScanU, gn, inx);
#pragma unroll
    for (int u = 0; u < kScanU; ++u) {
      if (t0 + u < rows) {
        s = __builtin_fmaf(gc[u], s, ic[u]);
        recur[static_cast<size_t>(t0 + u) * H + c] = s;
      }
    }
#pragma unroll
    for (int u = 0; u < kScanU; ++u) {
      gc[u] = gn[u];
      ic[u] = inx[u];
    }
  }
  state[c] = s;
}

// The recurrence of several independent sequences stacked as row segments (the prompts of
// the serving streams): segment b = rows [off[b], off[b + 1]) starts from state b
// (state + b * H) and leaves its last value there. One thread per (column, segment); each
// segment is scanned in time order exactly as k_scan_seq scans one sequence.
// GATE: g and in are the raw f and i projections and the gate math (k_gate's arithmetic,
// no element tail since H % 8 == 0) runs on each step beside the chain.
template <bool GATE>
__global__ __launch_bounds__(64) void k_scan_segs(const float* __restrict__ g, const float* __restrict__ in,
                                                  const float* __restrict__ lb, float* __restrict__ recur,
                                                  float* __restrict__ state, const int* __restrict__ off, int H) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  const int b = blockIdx.y, t0 = off[b], t1 = off[b + 1];
  float* st = state + static_cast<size_t>(b) * H;
  float s = st[c];
  const float lbc = (GATE && lb) ? lb[c] : 0.0f;
  constexpr int U = 16;
  for (int t = t0; t < t1; t += U) {
    float gc[U], ic[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tt = t + u < t1 ? t + u : t1 - 1;
      gc[u] = g[static_cast<size_t>(tt) * H + c];
      ic[u] = in[static_cast<size_t>(tt) * H + c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t + u < t1) {
        float gg = gc[u], xin = ic[u];
        if (GATE) {
          gg = sigmoid_of(gg, false);
          if (lb) gg = __builtin_fmaf(1.0f - lbc, gg, lbc);
          xin = swiglu_of(xin, 1.0f - gg, false);
        }
        s = __builtin_fmaf(gg, s, xin);
        recur[static_cast<size_t>(t + u) * H + c] = s;
      }
    }
  }
  st[c] = s;
}

// rows idx[r] of x [*, K] -> out [n, K]
__global__ void k_gather_rows(const float* __restrict__ x, const int* __restrict__ idx, float* __restrict__ out,
                              int K) {
  const float* src = x + static_cast<size_t>(idx[blockIdx.x]) * K;
  float* dst = out + static_cast<size_t>(blockIdx.x) * K;
  for (int k = threadIdx.x; k < K; k += blockDim.x) dst[k] = src[k];
}

// The recurrence for H % C == 0 (C = 4, 8 or 16 columns per block), staged through LDS so
// that enough bytes are in flight: a block owns C columns and walks time in tiles of kScTT
// steps. Waves by role: wave 0 runs the C column chains (state = fma(g, state, in), in
// time order) at raised issue priority; waves 1-4 fill a ring of kScNR tiles of g and in by
// direct global-to-LDS DMA (lane l's 16 bytes land at LDS base + 16 l: 256 / C steps x C
// columns per transfer); waves 1-14 convert each tile into column-major rows for the chain,
// and the last wave stores the previous tile. One barrier per tile. (Launches use C = 8: at
// 2048 x 2048 16 columns per block, half the blocks, measured 15% slower and 4 columns per
// block 60% slower.) The column groups of one line go to blocks of the same XCD (blocks are
// dealt to the 8 XCDs round-robin).
constexpr int kScTT = 128;
constexpr int kScWaves = 16, kScStoreWaves = 1;  // the last kScStoreWaves waves store
// Ring depth (tiles): the loads of a tile are in flight for NR - 2 tile iterations (about
// 1 us each).
template <int C>
constexpr int scan_ring_depth() {
  return C == 4 ? 16 : (C == 8 ? 8 : 4);
}

typedef __attribute__((address_space(3))) void lds_void_t;

template <int C>
__device__ __forceinline__ void scan_issue(const float* g, const float* in, float* ring, int tile, int slot,
                                           int T, int H, int c0, int lw, int lane) {
  constexpr int TA = kScTT * C / 256;  // transfers per array per tile
  constexpr int LPW = 2 * TA / 4;      // transfers per loader wave per tile
  constexpr int SPT = 256 / C;         // steps per transfer
  constexpr int LPR = C / 4;           // lanes per step row
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int idx = lw * LPW + i, arr = idx / TA, q = idx % TA;
    int t = tile * kScTT + SPT * q + lane / LPR;
    t = t < T ? t : T - 1;
    const float* src = (arr ? in : g) + static_cast<size_t>(t) * H + c0 + 4 * (lane % LPR);
    float* dst = ring + ((slot * 2 + arr) * kScTT + SPT * q) * C;
    __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
  }
}

// GATE: g and in are the raw f and i projections, and the conversion applies the gate math
// (sigmoid, lower bound, swiglu; hgrn_model.cpp:113-124, the same functions as k_gate), so
// the gated values never go through memory. Element tail rules do not arise: this kernel
// requires H % 16 == 0.
//
// Each iteration k: the loaders issue the transfers of tile k + kScNR - 1; waves 1 .. 14
// convert tile k + 1 from the ring (step-major, as loaded) into column-major rows GT / IT
// (three tile buffers, one row per column); wave 0 chains tile k; wave 15 stores tile k - 1.
// Cycles per tile at 2048 x 2048 (timing copy, medians): chain 1370, gate math 990, store
// wave 1850 with its stores drained, iteration 2350 (the chain alone took 2300 when it
// wrote its results).
//  * The chain: lane (cl, sg) = NSEG cl + sg holds segment sg (SL = kScTT / NSEG steps) of
//    column cl, read once per tile. Round r runs segment r's steps in every lane (only the
//    lanes of segment r hold the running state; the others compute values nobody uses), and
//    a DPP row shift hands each running state to the next segment's lane (after the last
//    round, back to segment 0). The lanes of segment r keep the state they start it from,
//    and these starting states are the chain's only LDS write (a result write costs the
//    issuing wave some 25-30 cycles; one per 4 steps doubled the chain's time).
//  * The store wave recomputes each segment of tile k - 1 from its starting state, with the
//    same FMAs in the same order (so the same values), and stores the states step by step.
// Tile k + 1 must then be in LDS at the barrier of iteration k, and an extra first iteration
// converts tile 0. A partial last tile is chained one step at a time by the segment-0 lanes,
// which store it themselves.
template <bool GATE, int C, int kScNR = scan_ring_depth<C>()>
__global__ __launch_bounds__(64 * kScWaves) void k_scan_ring(const float* __restrict__ g, const float* __restrict__ in,
                                                             const float* __restrict__ lb, float* __restrict__ recur,
                                                             float* __restrict__ state, int T, int H) {
  static_assert(C == 4 || C == 8 || C == 16, "4, 8 or 16 columns per block");
  constexpr int NCONV = kScWaves - 1 - kScStoreWaves;  // converting waves 1 .. NCONV
  static_assert((64 * NCONV) % C == 0, "a converting lane keeps its column");
  static_assert((kScNR - 2) * kScTT * C / 512 < 64, "outstanding transfers per loader wave");
  constexpr int LPW = kScTT * C / 512;  // transfers per loader wave per tile
  constexpr int NSEG = 64 / C, SL = kScTT / NSEG;
  constexpr int LT = kScTT + 36;  // column row: the tile and a pad against bank conflicts
  extern __shared__ __align__(16) float sm[];
  float* ring = sm;                          // [kScNR][2][kScTT][C], as loaded
  float* GT = ring + kScNR * 2 * kScTT * C;  // [3][C][LT] converted g (tile % 3)
  float* IT = GT + 3 * C * LT;               // [3][C][LT] converted in
  float* ST = IT + 3 * C * LT;               // [2][64] starting states of the segments (tile & 1)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // column group: XCD-contiguous when the groups split evenly over the 8 XCDs
  const int ngrp = H / C, b = blockIdx.x;
  const int grp = (ngrp % 8 == 0) ? (b & 7) * (ngrp / 8) + (b >> 3) : b;
  const int c0 = grp * C;
  const int ntiles = (T + kScTT - 1) / kScTT;
  const bool loader = wave >= 1 && wave <= 4;
  const bool conv = wave >= 1 && wave <= NCONV;
  const bool storer = wave >= kScWaves - kScStoreWaves;
  constexpr int SQ = SL / kScStoreWaves;  // steps of a segment each store wave stores
  const int sq0 = (wave - (kScWaves - kScStoreWaves)) * SQ;
  // chain and store waves: lane (cl, sg)
  const int cl = lane / NSEG, sg = lane % NSEG;
  float s = (wave == 0 && sg == 0) ? state[c0 + cl] : 0.0f;
  // the chain is the block's critical path: its instructions issue ahead of the conversion
  // sharing its SIMD
  if (wave == 0) __builtin_amdgcn_s_setprio(3);
  // the column a converting lane handles is fixed (64 x NCONV lanes, C columns per step row)
  const int ccol = (threadIdx.x - 64) % C;
  const float lbc = (GATE && conv && lb) ? lb[c0 + ccol] : 0.0f;
  if (loader)
    for (int t = 0; t < kScNR - 1 && t < ntiles; ++t) scan_issue<C>(g, in, ring, t, t, T, H, c0, wave - 1, lane);
  for (int k = -1; k <= ntiles; ++k) {
    // this wave's LDS writes (converted tiles, starting states) have landed before the
    // barrier publishes them
    __builtin_amdgcn_s_waitcnt(0xC07F);
    if (loader) {
      // this wave's transfers of tile k + 1 are done once only later tiles' are outstanding
      if (k >= 0 && k + kScNR - 2 < ntiles)
        __builtin_amdgcn_s_waitcnt(((kScNR - 3) * LPW & 0xF) | (((kScNR - 3) * LPW >> 4) << 14) | 0x0F70);
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (loader && k >= 0 && k + kScNR - 1 < ntiles)
      scan_issue<C>(g, in, ring, k + kScNR - 1, (k + kScNR - 1) % kScNR, T, H, c0, wave - 1, lane);
    if (conv && k + 1 < ntiles) {
      // tile k + 1 into column-major rows (GATE: g' = sigmoid(f), then the lower bound;
      // in' = swiglu(i, 1 - g'))
      const float* Gr = ring + (((k + 1) % kScNR) * 2 + 0) * kScTT * C;
      const float* Ir = ring + (((k + 1) % kScNR) * 2 + 1) * kScTT * C;
      float* Gc = GT + ((k + 1) % 3) * C * LT + ccol * LT;
      float* Ic = IT + ((k + 1) % 3) * C * LT + ccol * LT;
      const int n = min(kScTT, T - (k + 1) * kScTT);
      for (int e = threadIdx.x - 64; e < n * C; e += 64 * NCONV) {
        float gg = Gr[e], ii = Ir[e];
        if (GATE) {
          gg = sigmoid_of(gg, false);
          if (lb) gg = __builtin_fmaf(1.0f - lbc, gg, lbc);
          ii = swiglu_of(ii, 1.0f - gg, false);
        }
        const int st = e / C;
        Gc[st] = gg;
        Ic[st] = ii;
      }
    }
    if (wave == 0 && k >= 0 && k < ntiles) {
      const float* Gc = GT + (k % 3) * C * LT + cl * LT;
      const float* Ic = IT + (k % 3) * C * LT + cl * LT;
      const int n = min(kScTT, T - k * kScTT);
      if (n == kScTT) {
        const float4* G4 = reinterpret_cast<const float4*>(Gc + sg * SL);
        const float4* I4 = reinterpret_cast<const float4*>(Ic + sg * SL);
        float4 gv[SL / 4], iv[SL / 4];
#pragma unroll
        for (int u = 0; u < SL / 4; ++u) {
          gv[u] = G4[u];
          iv[u] = I4[u];
        }
        float s0 = s;  // the state this lane's segment starts from (segment 0: the tile's)
#pragma unroll
        for (int r = 0; r < NSEG; ++r) {
          if (r > 0) s0 = (sg == r) ? s : s0;
#pragma unroll
          for (int u = 0; u < SL / 4; ++u) {
            s = __builtin_fmaf(gv[u].x, s, iv[u].x);
            s = __builtin_fmaf(gv[u].y, s, iv[u].y);
            s = __builtin_fmaf(gv[u].z, s, iv[u].z);
            s = __builtin_fmaf(gv[u].w, s, iv[u].w);
          }
          // row_shr:1, after the last round row_shl:NSEG-1 (within rows of 16 lanes; a
          // column's NSEG lanes never straddle a row)
          const int si = __builtin_bit_cast(int, s);
          s = __builtin_bit_cast(float, r + 1 < NSEG ? __builtin_amdgcn_update_dpp(0, si, 0x111, 0xf, 0xf, false)
                                                     : __builtin_amdgcn_update_dpp(0, si, 0x100 + NSEG - 1, 0xf, 0xf, false));
        }
        ST[(k & 1) * 64 + lane] = s0;
      } else if (sg == 0) {
        // the last, partial tile: one step at a time, stored here
        float* out = recur + static_cast<size_t>(k) * kScTT * H + c0 + cl;
        for (int t = 0; t < n; ++t) {
          s = __builtin_fmaf(Gc[t], s, Ic[t]);
          out[static_cast<size_t>(t) * H] = s;
        }
      }
    }
    if (storer && k >= 1 && k * kScTT <= T) {
      // tile k - 1 (whole): segment sg of column cl again from its starting state
      const int kk = k - 1;
      const float4* G4 = reinterpret_cast<const float4*>(GT + (kk % 3) * C * LT + cl * LT + sg * SL);
      const float4* I4 = reinterpret_cast<const float4*>(IT + (kk % 3) * C * LT + cl * LT + sg * SL);
      float r = ST[(kk & 1) * 64 + lane];
      float4 gv[SL / 4], iv[SL / 4];
#pragma unroll
      for (int u = 0; u < SL / 4; ++u) {
        gv[u] = G4[u];
        iv[u] = I4[u];
      }
      float* out = recur + static_cast<size_t>(kk * kScTT + sg * SL) * H + c0 + cl;
      // every store wave recomputes the segment from its start and stores steps
      // [sq0, sq0 + SQ) (two store waves measured no faster than one)
#pragma unroll
      for (int u = 0; u < SL / 4; ++u) {
        float v[4];
        r = __builtin_fmaf(gv[u].x, r, iv[u].x);
        v[0] = r;
        r = __builtin_fmaf(gv[u].y, r, iv[u].y);
        v[1] = r;
        r = __builtin_fmaf(gv[u].z, r, iv[u].z);
        v[2] = r;
        r = __builtin_fmaf(gv[u].w, r, iv[u].w);
        v[3] = r;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (4 * u + c >= sq0 && 4 * u + c < sq0 + SQ) out[static_cast<size_t>(4 * u + c) * H] = v[c];
      }
    }
  }
  if (wave == 0 && sg == 0) state[c0 + cl] = s;
}

__global__ void k_embed(const float* __restrict__ emb, const int64_t* __restrict__ ids,
                        float* __restrict__ h, int rows, int H) {
  const size_t n = static_cast<size_t>(rows) * H;
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t r = e / H, c = e - r * H;
    h[e] = emb[static_cast<size_t>(ids[r]) * H + c];
  }
}

// rmsnorm / swishgate rows: one block per row, padded chain-transposed copy in LDS for the
// order-exact sumsq
__global__ void k_rownorm(const float* __restrict__ x, const float* __restrict__ o,
                          const float* __restrict__ w, float* __restrict__ y, int cols, float eps) {
  extern __shared__ float smem[];
  const int K = cols, K8 = K & ~7, nb = K8 / 8, Lc = nb > 0 ? (nb + 15) / 16 * 16 : 16;
  const int LS = lds_stride(Lc);
  float* X = smem;
  float* red = X + 8 * LS + 8;
  const float* xr = x + static_cast<size_t>(blockIdx.x) * K;
  load_T(X, xr, K, K8, Lc, LS, nb);
  __syncthreads();
  const float r = rstd_of(block_sumsq(X, Lc, LS, K - K8, red), K, eps);
  float* yr = y + static_cast<size_t>(blockIdx.x) * K;
  const float* orow = o ? o + static_cast<size_t>(blockIdx.x) * K : nullptr;
  for (int k0 = threadIdx.x; k0 < K; k0 += kU * blockDim.x) {
    float xv[kU], wv[kU], ov[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = k0 + u * blockDim.x;
      xv[u] = k < K ? xr[k] : 0.0f;
      wv[u] = k < K ? w[k] : 0.0f;
      ov[u] = (orow && k < K) ? orow[k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = k0 + u * blockDim.x;
      if (k >= K) continue;
      float v = (xv[u] * r) * wv[u];
      if (orow) v = v * silu_of(ov[u], k >= K8);
      yr[k] = v;
    }
  }
}

__global__ void k_argmax_rows(const float* __restrict__ lg, int V, int64_t* __restrict__ ids) {
  __shared__ unsigned long long red[16];
  const float* r = lg + static_cast<size_t>(blockIdx.x) * V;
  unsigned long long best = 0;
  // 16 logits per thread loaded before any is compared: one memory round trip per 16
  // instead of one per logit
  constexpr int U = 16;
  for (int v0 = threadIdx.x; v0 < V; v0 += U * blockDim.x) {
    float x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x;
      x[u] = v < V ? r[v] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x;
      const unsigned long long k = v < V ? amax_key(x[u], v) : 0ull;
      best = k > best ? k : best;
    }
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) best = red[i] > best ? red[i] : best;
    best = red[0] > best ? red[0] : best;
    ids[blockIdx.x] = key_index(best);
  }
}

__global__ void k_quant_rows(const float* __restrict__ y, int32_t* __restrict__ q, int rows, int K, float qs) {
  const size_t n = static_cast<size_t>(rows) * K;
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int k = static_cast<int>(e % K);
    q[e] = (k < (K & ~7)) ? q510_body(y[e], qs) : q510_tail(y[e], qs);
  }
}

__global__ void k_swiglu(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                         size_t n) {
  const size_t body = n & ~static_cast<size_t>(7);
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[e] = swiglu_of(a[e], b[e], e >= body);
}

__global__ void k_scan(const float* __restrict__ i, const float* __restrict__ f, float* __restrict__ out,
                       float* __restrict__ state, int T, int D) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  float s = state ? state[d] : 0.0f;
  for (int t = 0; t < T; ++t) {
    const size_t e = static_cast<size_t>(t) * D + d;
    s = __builtin_fmaf(f[e], s, i[e]);
    out[e] = s;
  }
  if (state) state[d] = s;
}

}  // namespace

// ------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------
hipError_t launch_pack(const int8_t* wq, const Geom& g, uint32_t* pk, int8_t* tail, int32_t* rowsum,
                       hipStream_t s) {
  int* bad = nullptr;
  hipError_t e = hipMalloc(&bad, sizeof(int));
  if (e != hipSuccess) return e;
  e = hipMemsetAsync(bad, 0, sizeof(int), s);
  if (e != hipSuccess) { (void)hipFree(bad); return e; }
  const size_t nwords = static_cast<size_t>(g.ngroups) * g.Wc * kGroup * 8;
  const int blocks = static_cast<int>(std::min<size_t>((nwords + 255) / 256, 65536));
  k_pack<<<blocks, 256, 0, s>>>(wq, g, pk, bad);
  k_pack_rows<<<g.ngroups * kGroup, 256, 0, s>>>(wq, g, tail, rowsum, bad);
  e = hipGetLastError();
  int hbad = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&hbad, bad, sizeof(int), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(bad);
  if (e == hipSuccess && hbad) return hipErrorInvalidValue;
  return e;
}

int seam_max_rows() { return kSeamRows; }

hipError_t launch_seam_dot(const SeamArgs& a, int k, hipStream_t s) {
  if (a.b < 1 || a.b > kSeamRows || k < 1 || k > kSeamMaxProj) return hipErrorInvalidValue;
  const size_t lds = static_cast<size_t>(a.b) * (16 * (a.g.Lc + 16) + 8 * sizeof(int32_t));
  if (lds > static_cast<size_t>(lds_limit())) return hipErrorInvalidValue;
  // each block reads the rows from host memory once (cheap: 64 blocks x 4 KB measured +0.7 us)
  const dim3 grid(std::min((a.g.ngroups + 1) / 2, 256), k);
  switch (a.b) {
    case 1: k_seam_dot<1><<<grid, 256, lds, s>>>(a); break;
    case 2: k_seam_dot<2><<<grid, 256, lds, s>>>(a); break;
    case 3: k_seam_dot<3><<<grid, 256, lds, s>>>(a); break;
    default: k_seam_dot<4><<<grid, 256, lds, s>>>(a); break;
  }
  return hipGetLastError();
}

size_t pk4_words(const Geom& g) { return static_cast<size_t>(g.ngroups) * 2 * g.Wc * kGroup * 8; }

hipError_t launch_pack4(const uint32_t* pk, const Geom& g, uint32_t* pk4, hipStream_t s) {
  const size_t nwords = static_cast<size_t>(g.ngroups) * g.Wc * kGroup * 8;
  const int blocks = static_cast<int>(std::min<size_t>((nwords + 255) / 256, 65536));
  k_pack4<<<blocks, 256, 0, s>>>(pk, nwords, g.Wc, pk4);
  return hipGetLastError();
}

static int host_lds_stride(int Lc) { return (Lc + 31) / 32 * 32 + 4; }

// Up to kPrologueFewRows rows (two per CU, the CUs otherwise idle) a row gets a 1024-thread
// block (k_rowpro) with every input, the norm weights included, loaded at entry: each thread
// then works on one group and one unit, with four waves per SIMD to hide each other's
// latency. Above it, 256-thread blocks keep more rows resident per CU. (One wave per row with
// one chain wave for 8 rows measured slower: every row of a block then waits for the
// slowest row's loads, and a single wave per row serialises the encoding.)
constexpr int kPrologueFewRows = 512;

// groups or units per row, whichever is more (k_rowpro)
static int rowpro_need(const ActBuf& act) { return std::max(act.Lc, act.nb + (act.ntail > 0 ? 1 : 0)); }
static bool rowpro_fits(const ActBuf& act) {
  return rowpro_need(act) <= (act.rows <= kPrologueFewRows ? 2048 : 1024);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// MMF_ROWSEG=0 keeps few-row prologues on k_rowpro (for comparisons); default on.
static bool rowseg_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("MMF_ROWSEG");
    return !(e && e[0] == '0');
  }();
  return on;
}

// k_rowseg at the model widths (K = 256 RC: hidden 1024/2048/2560, and without a stage-1
// norm also 2816/5632/6912), one wave per row: kPreNorm up to kSegRows rows (64 rows at
// K = 2560: 5.5 us against k_rowpro's 7.1 us), kPreNone (the operator API's BitLinear) up to
// kSegRowsNone rows (the MLP down projection's 64-row input at K = 6912 measured 8.9 us
// against k_rowpro's 8.1 us); the swish-gate kinds (one projection) on k_rowseg_sw up to
// kSegRows rows.
constexpr int kSegRows = 512, kSegRowsNone = 16;

template <int MODE, int PRE, int NA, int RC>
static hipError_t rowseg_inst(const PrologueArgs& a, ActBuf& act, hipStream_t s) {
  if constexpr (PRE == kPreNorm || PRE == kPreNone) {
    k_rowseg<MODE, PRE, NA, RC><<<row_grid(act.rows), 64 * NA, 0, s>>>(a, act);
    return hipGetLastError();
  } else if constexpr (NA == 1) {
    k_rowseg_sw<MODE, PRE, RC><<<row_grid(act.rows), 1024, 0, s>>>(a, act);
    return hipGetLastError();
  } else {
    return hipErrorNotSupported;
  }
}

template <int MODE, int PRE, int NA>
static hipError_t rowseg_launch(const PrologueArgs& a, ActBuf& act, hipStream_t s) {
  if (act.rows > (PRE == kPreNone ? kSegRowsNone : kSegRows) || act.Lc % 32 != 0 || act.K != 8 * act.Lc ||
      act.nb != act.Lc || act.ntail != 0)
    return hipErrorNotSupported;
  if (PRE != kPreNone && !(a.pre_wT && aligned16(a.pre_wT))) return hipErrorNotSupported;
  switch (act.Lc / 32) {
    case 4: return rowseg_inst<MODE, PRE, NA, 4>(a, act, s);
    case 8: return rowseg_inst<MODE, PRE, NA, 8>(a, act, s);
    case 10: return rowseg_inst<MODE, PRE, NA, 10>(a, act, s);
    default: break;
  }
  if constexpr (PRE == kPreNone) {
    switch (act.Lc / 32) {
      case 11: return rowseg_inst<MODE, PRE, NA, 11>(a, act, s);
      case 22: return rowseg_inst<MODE, PRE, NA, 22>(a, act, s);
      case 27: return rowseg_inst<MODE, PRE, NA, 27>(a, act, s);
      default: break;
    }
  }
  return hipErrorNotSupported;
}

template <int MODE, int PRE, int NA>
static hipError_t rowpro_inst(const PrologueArgs& a, ActBuf& act, size_t lds, hipStream_t s) {
  if (rowseg_enabled()) {
    const hipError_t e = rowseg_launch<MODE, PRE, NA>(a, act, s);
    if (e != hipErrorNotSupported) return e;
  }
  const int need = rowpro_need(act), grid = row_grid(act.rows);
  if constexpr (PRE == kPreNone && NA == 1 && MODE != kInt8) {
    // long rows of many-row launches: half of the row in LDS at a time (k_rowpro_split)
    if (act.rows > kPrologueFewRows && need > 512 && need <= 1024 && act.nb >= 512 && aligned16(a.normw[0])) {
      const size_t lds_split = (8 * static_cast<size_t>(host_lds_stride(std::max(512, act.Lc - 512))) + 8 + 32) * sizeof(float);
      if (need <= 768) k_rowpro_split<MODE, 3><<<grid, 256, lds_split, s>>>(a, act);
      else k_rowpro_split<MODE, 4><<<grid, 256, lds_split, s>>>(a, act);
      return hipGetLastError();
    }
  }
  if (act.rows <= kPrologueFewRows) {
    if (need <= 1024) k_rowpro<MODE, PRE, NA, 1, true, 1024><<<grid, 1024, lds, s>>>(a, act);
    else k_rowpro<MODE, PRE, NA, 2, true, 1024><<<grid, 1024, lds, s>>>(a, act);
  } else if (need <= 256) {
    k_rowpro<MODE, PRE, NA, 1, false, 256><<<grid, 256, lds, s>>>(a, act);
  } else if (need <= 512) {
    k_rowpro<MODE, PRE, NA, 2, false, 256><<<grid, 256, lds, s>>>(a, act);
  } else if (need <= 768) {
    k_rowpro<MODE, PRE, NA, 3, false, 256><<<grid, 256, lds, s>>>(a, act);
  } else {
    k_rowpro<MODE, PRE, NA, 4, false, 256><<<grid, 256, lds, s>>>(a, act);
  }
  return hipGetLastError();
}

template <int MODE>
static hipError_t rowpro_mode(const PrologueArgs& a, ActBuf& act, size_t lds, hipStream_t s) {
  if (a.pre == kPreNorm && a.na == 3) return rowpro_inst<MODE, kPreNorm, 3>(a, act, lds, s);
  if (a.pre == kPreNorm && a.na == 1) return rowpro_inst<MODE, kPreNorm, 1>(a, act, lds, s);
  if (a.pre == kPreSwish && a.na == 1) return rowpro_inst<MODE, kPreSwish, 1>(a, act, lds, s);
  if (a.pre == kPreMixSwish && a.na == 1) return rowpro_inst<MODE, kPreMixSwish, 1>(a, act, lds, s);
  if (a.pre == kPreNone && a.na == 1) return rowpro_inst<MODE, kPreNone, 1>(a, act, lds, s);
  if (a.pre == kPreNone && a.na == 3) return rowpro_inst<MODE, kPreNone, 3>(a, act, lds, s);
  return hipErrorNotSupported;
}

hipError_t launch_prologue(Mode mode, const PrologueArgs& a, ActBuf& act, hipStream_t s) {
  const size_t rowf = static_cast<size_t>(8 * host_lds_stride(act.Lc) + 8);
  const size_t lds = (2 * rowf + 16) * sizeof(float);
  const bool sw = a.pre == kPreSwish || a.pre == kPreMixSwish;
  const size_t lds4 = ((sw ? 2 : 1) * rowf + 32) * sizeof(float);  // k_rowpro
  bool fast = act.K % 4 == 0 && rowpro_fits(act) && aligned16(a.x) && (a.na == 1 || a.na == 3);
  if (a.pre != kPreNone) fast = fast && aligned16(a.pre_w);
  if (sw) fast = fast && aligned16(a.x2);
  for (int i = 0; i < a.na; ++i) fast = fast && a.normwT[i] && aligned16(a.normwT[i]);
  if (a.pre == kPreMixSwish) {
    fast = fast && a.na == 1 && aligned16(a.mix_f) && aligned16(a.mix_state) && (!a.mix_lb || aligned16(a.mix_lb));
    if (!fast) return hipErrorNotSupported;
  }
  if (fast) {
    hipError_t e = hipErrorNotSupported;
    switch (mode) {
      case kFloat: e = rowpro_mode<kFloat>(a, act, lds4, s); break;
      case kFixed: e = rowpro_mode<kFixed>(a, act, lds4, s); break;
      default: e = rowpro_mode<kInt8>(a, act, lds4, s); break;
    }
    if (e != hipErrorNotSupported) return e;
  }
  const int threads = 256;
  switch (mode) {
    case kFloat: k_prologue<kFloat><<<row_grid(act.rows), threads, lds, s>>>(a, act); break;
    case kFixed: k_prologue<kFixed><<<row_grid(act.rows), threads, lds, s>>>(a, act); break;
    default: k_prologue<kInt8><<<row_grid(act.rows), threads, lds, s>>>(a, act); break;
  }
  return hipGetLastError();
}

hipError_t launch_codes_to_planes(const int32_t* x, ActBuf& act, hipStream_t s) {
  k_codes<<<row_grid(act.rows), 256, 0, s>>>(x, act);
  return hipGetLastError();
}

hipError_t launch_planes_to_codes(const ActBuf& act, Mode mode, int32_t* codes, hipStream_t s) {
  if (mode == kFloat || act.na < 1 || act.na > 3) return hipErrorInvalidValue;
  k_planes_to_codes<<<dim3(row_grid(act.rows), act.na), 256, 0, s>>>(act, mode, codes);
  return hipGetLastError();
}

template <int MODE, int R, bool PAIR>
static hipError_t gemm_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int np = (MODE == kFixed) ? 2 : 1;
  const size_t lds = (MODE == kFloat) ? static_cast<size_t>(R) * 8 * kMW * 16 * sizeof(float)
                                      : static_cast<size_t>(R) * np * 8 * kMW * 16;
  dim3 grid(PAIR ? g.ngroups / 2 : g.ngroups, (a.rows + R - 1) / R, PAIR ? 1 : a.nmat);
  k_gemm<MODE, R, PAIR><<<grid, kBlock, lds, s>>>(a, act);
  return hipGetLastError();
}

template <int R, int NO, bool PAIR>
static int gemm_f_blocks(const GemmArgs& a) {
  const Geom& g = a.p[0].g;
  const int gx = PAIR ? (g.ngroups / 2 + NO / 2 - 1) / (NO / 2) : (g.ngroups + NO - 1) / NO;
  return gx * ((a.rows + R - 1) / R) * (PAIR ? 1 : a.nmat);
}

template <int R, int NO, bool PAIR>
static hipError_t gemm_f_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const size_t lds = static_cast<size_t>(R) * 8 * kFCS * sizeof(float);
  const int gx = PAIR ? (g.ngroups / 2 + NO / 2 - 1) / (NO / 2) : (g.ngroups + NO - 1) / NO;
  dim3 grid(gx, (a.rows + R - 1) / R, PAIR ? 1 : a.nmat);
  k_gemm_f<R, NO, PAIR><<<grid, 128, lds, s>>>(a, act);
  return hipGetLastError();
}

// Four outputs per thread while that leaves at least 1024 blocks (two waves per SIMD),
// else two, else one: a small launch is latency-bound and wants more waves more than
// fewer LDS reads.
template <int R, bool PAIR>
static hipError_t gemm_f_rows(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (gemm_f_blocks<R, 4, PAIR>(a) >= 1024) return gemm_f_inst<R, 4, PAIR>(a, act, s);
  if constexpr (PAIR) {  // a block holds gate/up pairs: at least two outputs per thread
    return gemm_f_inst<R, 2, PAIR>(a, act, s);
  } else {
    if (gemm_f_blocks<R, 2, PAIR>(a) >= 1024) return gemm_f_inst<R, 2, PAIR>(a, act, s);
    return gemm_f_inst<R, 1, PAIR>(a, act, s);
  }
}

template <int MODE>
static hipError_t gemm_mode(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (MODE == kFloat && float_mfma_min_rows() > 0 && a.rows >= float_mfma_min_rows() && mfma_f_ok(a))
    return launch_gemm_mfma_f(a, act, s);
  if (MODE == kFloat && a.rows > 4) {
    const bool pair = a.epi == kEpiSwigluPair;
    // up to 64 rows (serving steps): 4-row tiles, so that the >= 1024-block rule keeps two
    // outputs per thread (half the LDS reads per FMA of one) on the 2560-column GEMMs;
    // 64-stream 2.7B float step 10.9 -> 9.4 ms against 8-row tiles
    if (a.rows <= 64) return pair ? gemm_f_rows<4, true>(a, act, s) : gemm_f_rows<4, false>(a, act, s);
    return pair ? gemm_f_rows<16, true>(a, act, s) : gemm_f_rows<16, false>(a, act, s);
  }
  const bool pair = a.epi == kEpiSwigluPair;
  if (a.rows <= 1) return pair ? gemm_inst<MODE, 1, true>(a, act, s) : gemm_inst<MODE, 1, false>(a, act, s);
  if (a.rows <= 4) return pair ? gemm_inst<MODE, 4, true>(a, act, s) : gemm_inst<MODE, 4, false>(a, act, s);
  return pair ? gemm_inst<MODE, 8, true>(a, act, s) : gemm_inst<MODE, 8, false>(a, act, s);
}

int float_mfma_min_rows() {
  static const int v = [] {
    const char* e = std::getenv("MMF_FLOAT_MFMA_MIN_ROWS");
    return e ? std::atoi(e) : 16;
  }();
  return v;
}

int mfma_min_rows() {
  static const int v = [] {
    const char* e = std::getenv("MMF_MFMA_MIN_ROWS");
    return e ? std::atoi(e) : 8;
  }();
  return v;
}

hipError_t launch_gemm(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (a.mode != kFloat && mfma_min_rows() > 0 && a.rows >= mfma_min_rows()) {
    // (the matrix-core kernel addresses a matrix's planes and weights with 31-bit offsets)
    bool ok = 2 * act.qplane() <= 0x7FFFFFFFu;
    for (int z = 0; z < (a.epi == kEpiSwigluPair ? 1 : a.nmat); ++z)
      ok = ok && a.p[z].pkm && (a.p[z].pair != 0) == (a.epi == kEpiSwigluPair) &&
           pkm_words(a.p[z].g) * 4 <= 0x7FFFFFFFu;
    if (ok) return launch_gemm_mfma(a, act, s);
  }
  switch (a.mode) {
    case kFloat: return gemm_mode<kFloat>(a, act, s);
    case kFixed: return gemm_mode<kFixed>(a, act, s);
    default: return gemm_mode<kInt8>(a, act, s);
  }
}

// Columns per k_scan_ring block: 8, so that H / 8 blocks (256 at H = 2048) cover the CUs;
// the two blocks of a 64-byte line sit on one XCD and share its L2.
template <bool GATE>
static hipError_t scan_ring_launch(const float* g, const float* in, const float* lb, float* recur, float* state,
                                   int rows, int H, hipStream_t s) {
  auto go = [&](auto cc) {
    constexpr int C = decltype(cc)::value;
    const size_t lds =
        (static_cast<size_t>(scan_ring_depth<C>()) * 2 * kScTT * C + 6 * static_cast<size_t>(C) * (kScTT + 36) +
         128) *
        sizeof(float);
    k_scan_ring<GATE, C><<<H / C, 64 * kScWaves, lds, s>>>(g, in, lb, recur, state, rows, H);
    return hipGetLastError();
  };
  return go(std::integral_constant<int, 8>{});
}

// Chunked parallel scan of the prefill recurrence (float mode, opt-in; not the reference's
// rounding). Time is cut into chunks of kChunkT steps (16: at T = 2048, H = 2048 that is 4096
// waves, four per SIMD, to hide the loads), and three launches run:
//   1. k_chunk_sum, per (chunk, column): the gate math of k_gate and the chunk's scan from a
//      zero state, l = fma(g, l, in), with the product of its gates, p = g * p;
//   2. k_chunk_carry, per column: the chunks' starting states in time order,
//      S_c = fma(p_{c-1}, S_{c-1}, l_{c-1}), S_0 = the layer's state;
//   3. k_chunk_apply, per (chunk, column): the chunk again from its starting state with the
//      reference's own steps, state = fma(g, state, in); the last chunk stores the state.
// In real arithmetic S_c is the state the time-ordered scan reaches; in fp32 it differs by
// the rounding of the products and of the combination, so the result is within tolerance of
// the reference rather than equal to it. The chunks and columns run in parallel (one wave
// per 64 columns of a chunk); the gate math runs twice, in launches 1 and 3.
constexpr int kChunkT = 16;

__device__ __forceinline__ void gate_pair(float f, float i, float lbv, bool has_lb, float& g, float& in) {
  g = sigmoid_of(f, false);
  if (has_lb) g = __builtin_fmaf(1.0f - lbv, g, lbv);
  in = swiglu_of(i, 1.0f - g, false);
}

__global__ __launch_bounds__(64) void k_chunk_sum(const float* __restrict__ fr, const float* __restrict__ ir,
                                                  const float* __restrict__ lb, float* __restrict__ lsum,
                                                  float* __restrict__ prod, int T, int H) {
  const int h = blockIdx.x * 64 + threadIdx.x, c = blockIdx.y;
  const int t0 = c * kChunkT, n = min(kChunkT, T - t0);
  float fv[kChunkT], iv[kChunkT];
#pragma unroll
  for (int u = 0; u < kChunkT; ++u) {
    const size_t e = static_cast<size_t>(t0 + (u < n ? u : 0)) * H + h;
    fv[u] = fr[e];
    iv[u] = ir[e];
  }
  const float lbv = lb ? lb[h] : 0.0f;
  float l = 0.0f, p = 1.0f;
#pragma unroll
  for (int u = 0; u < kChunkT; ++u) {
    if (u < n) {
      float g, in;
      gate_pair(fv[u], iv[u], lbv, lb != nullptr, g, in);
      l = __builtin_fmaf(g, l, in);
      p = p * g;
    }
  }
  lsum[static_cast<size_t>(c) * H + h] = l;
  prod[static_cast<size_t>(c) * H + h] = p;
}

__global__ __launch_bounds__(64) void k_chunk_carry(const float* __restrict__ lsum, const float* __restrict__ prod,
                                                    const float* __restrict__ state, float* __restrict__ start,
                                                    int nchunks, int H) {
  const int h = blockIdx.x * 64 + threadIdx.x;
  float S = state[h];
  constexpr int B = 64;  // chunks' summaries in flight at once (one memory round trip per 64 chunks)
  for (int c0 = 0; c0 < nchunks; c0 += B) {
    float lv[B], pv[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int c = c0 + u < nchunks ? c0 + u : nchunks - 1;
      lv[u] = lsum[static_cast<size_t>(c) * H + h];
      pv[u] = prod[static_cast<size_t>(c) * H + h];
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (c0 + u < nchunks) {
        start[static_cast<size_t>(c0 + u) * H + h] = S;
        S = __builtin_fmaf(pv[u], S, lv[u]);
      }
    }
  }
}

__global__ __launch_bounds__(64) void k_chunk_apply(const float* __restrict__ fr, const float* __restrict__ ir,
                                                    const float* __restrict__ lb, const float* __restrict__ start,
                                                    float* __restrict__ recur, float* __restrict__ state, int T,
                                                    int H) {
  const int h = blockIdx.x * 64 + threadIdx.x, c = blockIdx.y;
  const int t0 = c * kChunkT, n = min(kChunkT, T - t0);
  float fv[kChunkT], iv[kChunkT];
#pragma unroll
  for (int u = 0; u < kChunkT; ++u) {
    const size_t e = static_cast<size_t>(t0 + (u < n ? u : 0)) * H + h;
    fv[u] = fr[e];
    iv[u] = ir[e];
  }
  const float lbv = lb ? lb[h] : 0.0f;
  float s = start[static_cast<size_t>(c) * H + h];
#pragma unroll
  for (int u = 0; u < kChunkT; ++u) {
    if (u < n) {
      float g, in;
      gate_pair(fv[u], iv[u], lbv, lb != nullptr, g, in);
      s = __builtin_fmaf(g, s, in);
      recur[static_cast<size_t>(t0 + u) * H + h] = s;
    }
  }
  if (c == static_cast<int>(gridDim.y) - 1) state[h] = s;
}

size_t scan_chunked_ws_floats(int rows, int H) {
  return 3 * static_cast<size_t>((rows + kChunkT - 1) / kChunkT) * H;
}

hipError_t launch_scan_chunked(const float* i, const float* f, const float* lb, float* recur, float* state,
                               float* ws, int rows, int H, hipStream_t s) {
  if (rows < 1 || H % 64 != 0) return hipErrorInvalidValue;
  const int nch = (rows + kChunkT - 1) / kChunkT;
  float* lsum = ws;
  float* prod = lsum + static_cast<size_t>(nch) * H;
  float* start = prod + static_cast<size_t>(nch) * H;
  k_chunk_sum<<<dim3(H / 64, nch), 64, 0, s>>>(f, i, lb, lsum, prod, rows, H);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_chunk_carry<<<H / 64, 64, 0, s>>>(lsum, prod, state, start, nch, H);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_chunk_apply<<<dim3(H / 64, nch), 64, 0, s>>>(f, i, lb, start, recur, state, rows, H);
  return hipGetLastError();
}

hipError_t launch_mixer(const float* i, float* f, float* scan_out, float* recur, float* state,
                        const float* lb, int rows, int H, bool stream_state, bool keep_gates, hipStream_t s) {
  if (!stream_state && !keep_gates && rows > 1 && H % 16 == 0 &&
      ((reinterpret_cast<uintptr_t>(i) | reinterpret_cast<uintptr_t>(f) | reinterpret_cast<uintptr_t>(recur)) & 15) == 0) {
    // one kernel: the gate math runs inside the scan on each tile (k_scan_ring<true, C>)
    return scan_ring_launch<true>(f, i, lb, recur, state, rows, H, s);
  }
  if (!stream_state && scan_out && rows > 1) {
    const size_t n = static_cast<size_t>(rows) * H;
    const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 16384));
    k_gate<<<blocks, 256, 0, s>>>(i, f, scan_out, lb, rows, H);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool aligned = ((reinterpret_cast<uintptr_t>(f) | reinterpret_cast<uintptr_t>(scan_out) |
                           reinterpret_cast<uintptr_t>(recur)) & 15) == 0;
    if (H % 16 == 0 && aligned) {
      return scan_ring_launch<false>(f, scan_out, nullptr, recur, state, rows, H, s);
    } else {
      k_scan_seq<<<(H + 63) / 64, 64, 0, s>>>(f, scan_out, recur, state, rows, H);
    }
    return hipGetLastError();
  }
  const int n = stream_state ? rows * H : H;
  k_mixer<<<(n + 255) / 256, 256, 0, s>>>(i, f, scan_out, recur, state, lb, rows, H, stream_state ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_mixer_segs(const float* i, float* f, float* scan, float* recur, float* state, const float* lb,
                             const int* off, int nseg, int rows, int H, bool keep_gates, hipStream_t s) {
  if (H % 8 != 0) return hipErrorInvalidValue;  // a SIMD tail per segment would differ
  if (!keep_gates) {  // one kernel: the gate math beside each segment's chain
    k_scan_segs<true><<<dim3((H + 63) / 64, nseg), 64, 0, s>>>(f, i, lb, recur, state, off, H);
    return hipGetLastError();
  }
  const size_t n = static_cast<size_t>(rows) * H;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 16384));
  k_gate<<<blocks, 256, 0, s>>>(i, f, scan, lb, rows, H);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_scan_segs<false><<<dim3((H + 63) / 64, nseg), 64, 0, s>>>(f, scan, nullptr, recur, state, off, H);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const float* x, const int* idx, float* out, int n, int K, hipStream_t s) {
  k_gather_rows<<<n, 256, 0, s>>>(x, idx, out, K);
  return hipGetLastError();
}

hipError_t launch_embed(const float* emb, const int64_t* ids, float* h, int rows, int H, hipStream_t s) {
  const size_t n = static_cast<size_t>(rows) * H;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 16384));
  k_embed<<<blocks, 256, 0, s>>>(emb, ids, h, rows, H);
  return hipGetLastError();
}

static size_t rownorm_lds(int cols) {
  const int nb = (cols & ~7) / 8, Lc = nb > 0 ? (nb + 15) / 16 * 16 : 16;
  return (static_cast<size_t>(8 * host_lds_stride(Lc) + 8) + 16) * sizeof(float);
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int cols, float eps,
                          hipStream_t s) {
  k_rownorm<<<rows, 256, rownorm_lds(cols), s>>>(x, nullptr, w, y, cols, eps);
  return hipGetLastError();
}

hipError_t launch_swishgate(const float* g, const float* o, const float* w, float* out, int rows, int cols,
                            float eps, hipStream_t s) {
  k_rownorm<<<rows, 256, rownorm_lds(cols), s>>>(g, o, w, out, cols, eps);
  return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* logits, int rows, int V, int64_t* ids, hipStream_t s) {
  k_argmax_rows<<<rows, 1024, 0, s>>>(logits, V, ids);
  return hipGetLastError();
}

hipError_t launch_quant_rows(const float* y, int32_t* q, int rows, int K, float qs, hipStream_t s) {
  const size_t n = static_cast<size_t>(rows) * K;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 16384));
  k_quant_rows<<<blocks > 0 ? blocks : 1, 256, 0, s>>>(y, q, rows, K, qs);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* a, const float* b, float* out, size_t n, hipStream_t s) {
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 16384));
  k_swiglu<<<blocks > 0 ? blocks : 1, 256, 0, s>>>(a, b, out, n);
  return hipGetLastError();
}

hipError_t launch_scan(const float* i, const float* f, float* out, float* state, int T, int D, hipStream_t s) {
  k_scan<<<(D + 255) / 256, 256, 0, s>>>(i, f, out, state, T, D);
  return hipGetLastError();
}

}  // namespace mmf
