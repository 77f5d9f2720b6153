// mmf_device.hpp -- device-side numerics shared by the HIP kernels (gfx950).
//
// Every function reproduces, operation for operation and rounding for rounding, the
// reference engine's arithmetic as g++ compiles it (-O2 -mavx2 -mfma, GNU mode, so each
// mul+add pair in cpp/include/mmfree/simd.hpp that is not an explicit intrinsic FMA is
// fused). All HIP sources are compiled with -ffp-contract=off and every FMA below is an
// explicit __builtin_fmaf; division and sqrt are the correctly rounded IEEE forms
// (-fhip-fp32-correctly-rounded-divide-sqrt).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include <cstdint>

namespace mmf {

// Makes the listed uniform values (kernel arguments) live in scalar registers at this point:
// their scalar loads issue together before it, instead of one dependent load at each use,
// which the compiler otherwise repeats inside loops that store to global memory. No
// instruction is emitted.
#define MMF_PIN(...) asm volatile("" ::__VA_ARGS__)

// ---- packed ternary weights --------------------------------------------------------
// A 32-bit word holds 16 two-bit two's-complement codes (00 = 0, 01 = +1, 11 = -1). Code
// t (0..15) sits at bit 8*(t%4) + 2*(t/4), so (word >> 2i) & 0x03030303 puts the codes
// of t = 4i..4i+3 in the low bits of bytes 0..3 (a v_perm_b32 selector).
__device__ __forceinline__ constexpr int code_shift(int t) { return 8 * (t & 3) + 2 * (t >> 2); }

// signed code of position t as float (-1, 0, +1): one v_bfe_i32 + v_cvt_f32_i32
__device__ __forceinline__ float code_f(uint32_t w, int t) {
  return static_cast<float>(static_cast<int32_t>(w << (30 - code_shift(t))) >> 30);
}

// Codes of a word as fp16 pairs (+1 = 0x3C00, -1 = 0xBC00, 0 = 0x0000; all exact): pair (i,
// odd) holds codes 4i + odd (low half) and 4i + 2 + odd (high half). One v_perm_b32 takes
// each byte from the table {0x00, 0x3C, 0x00, 0xBC} by its selector byte: the two codes sit
// in selector bytes 1 and 3 (the halves' high bytes), and bytes 0 and 2 are 0, which selects
// the table's zero byte. The even codes reach bytes 1 and 3 by one funnel shift.
typedef _Float16 mmf_half2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ mmf_half2 code_pair_h(uint32_t w, int i, bool odd) {
  const uint32_t src = odd ? (w >> (2 * i)) : __builtin_amdgcn_alignbit(w, 0u, 24 + 2 * i);  // even: w << (8 - 2i)
  return __builtin_bit_cast(mmf_half2, __builtin_amdgcn_perm(0u, 0xBC003C00u, src & 0x03000300u));
}

// The 16-code word against 16 activations in the reference's order, acc = fma(y_t, w_t, acc)
// for t = 0..15 with one rounding each: the fp16 code converts exactly inside the FMA
// (v_fma_mix_f32), so this is the fp32 FMA of the code as float, with about 2.4
// instructions per code instead of 3 (extract, convert, FMA).
__device__ __forceinline__ float word_dot_f(uint32_t w, const float (&y)[16], float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const mmf_half2 e = code_pair_h(w, i, false), o = code_pair_h(w, i, true);
    acc = __builtin_fmaf(y[4 * i], static_cast<float>(e.x), acc);
    acc = __builtin_fmaf(y[4 * i + 1], static_cast<float>(o.x), acc);
    acc = __builtin_fmaf(y[4 * i + 2], static_cast<float>(e.y), acc);
    acc = __builtin_fmaf(y[4 * i + 3], static_cast<float>(o.y), acc);
  }
  return acc;
}

// An fp4 word (8 codes, code t in nibble t as an E2M1 value: 0x0 = 0, 0x2 = +1, 0xA = -1)
// against 8 activations, acc = fma(y_t, w_t, acc) for t = 0..7: each
// v_cvt_scalef32_pk_f32_fp4 (scale 1) turns byte b into the exact fp32 codes 2b and 2b + 1,
// so a code costs one FMA and half a conversion. The product y_t * w_t is exact and each step
// rounds once, as the reference's fmadd lane does.
typedef float mmf_float2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float word_dot_f4(uint32_t w, const float4& a, const float4& b, float acc) {
  const mmf_float2 c0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const mmf_float2 c1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const mmf_float2 c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const mmf_float2 c3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  acc = __builtin_fmaf(a.x, c0.x, acc);
  acc = __builtin_fmaf(a.y, c0.y, acc);
  acc = __builtin_fmaf(a.z, c1.x, acc);
  acc = __builtin_fmaf(a.w, c1.y, acc);
  acc = __builtin_fmaf(b.x, c2.x, acc);
  acc = __builtin_fmaf(b.y, c2.y, acc);
  acc = __builtin_fmaf(b.z, c3.x, acc);
  acc = __builtin_fmaf(b.w, c3.y, acc);
  return acc;
}

// weights t = 4i..4i+3 as four int8 lanes: v_perm_b32 with the byte table {0, +1, 0, -1}
__device__ __forceinline__ uint32_t w4_i8(uint32_t w, int i) {
  return __builtin_amdgcn_perm(0u, 0xFF000100u, (w >> (2 * i)) & 0x03030303u);
}

__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4(static_cast<int32_t>(a), static_cast<int32_t>(b), c, false);
}

// ---- reductions in the reference order ---------------------------------------------
// hsum_ps (simd.hpp:48-57): ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
__device__ __forceinline__ float hsum8(const float* a) {
  float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  return (s0 + s1) + (s2 + s3);
}

// Lane i + N's value in lane i within each row of 16 lanes (DPP row_shl:N, no memory
// round trip); lanes whose source lies past their row get zero.
template <int N>
__device__ __forceinline__ int dpp_shl(int v) {
  static_assert(N >= 1 && N <= 15, "row shift");
  return __builtin_amdgcn_update_dpp(0, v, 0x100 + N, 0xf, 0xf, false);
}
template <int N>
__device__ __forceinline__ float dpp_shl(float v) {
  return __builtin_bit_cast(float, dpp_shl<N>(__builtin_bit_cast(int, v)));
}

// Wave-wide maxima, in every lane, without a memory round trip: butterflies inside each row
// of 16 lanes (DPP quad_perm [1,0,3,2] and [2,3,0,1], then row_ror 4 and 8), then the four
// row maxima by readlane. Call from all 64 lanes of a wave. (Any order gives the same
// maximum; fmaxf ignores a NaN unless every value is one.)
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float wave_max(float v) {
  auto step = [](float x, auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    return fmaxf(x, __builtin_bit_cast(float, dpp_mov<C>(__builtin_bit_cast(int, x))));
  };
  v = step(v, std::integral_constant<int, 0xB1>{});
  v = step(v, std::integral_constant<int, 0x4E>{});
  v = step(v, std::integral_constant<int, 0x124>{});
  v = step(v, std::integral_constant<int, 0x128>{});
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  auto step = [](unsigned long long x, auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    const unsigned lo = static_cast<unsigned>(dpp_mov<C>(static_cast<int>(x)));
    const unsigned hi = static_cast<unsigned>(dpp_mov<C>(static_cast<int>(x >> 32)));
    const unsigned long long y = (static_cast<unsigned long long>(hi) << 32) | lo;
    return y > x ? y : x;
  };
  v = step(v, std::integral_constant<int, 0xB1>{});
  v = step(v, std::integral_constant<int, 0x4E>{});
  v = step(v, std::integral_constant<int, 0x124>{});
  v = step(v, std::integral_constant<int, 0x128>{});
  unsigned long long best = 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v), 16 * r));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), 16 * r));
    const unsigned long long y = (static_cast<unsigned long long>(hi) << 32) | lo;
    best = y > best ? y : best;
  }
  return best;
}

// The same tree across the 8 consecutive lanes that hold the 8 chain partials of one
// output (lane j holds a_j). Valid in lane j == 0 of each group of 8 (the groups of 8 lie
// inside the DPP rows of 16, so every source of such a lane is in its row).
__device__ __forceinline__ float hsum8_lanes(float a) {
  float s = a + dpp_shl<4>(a);  // lanes 0..3: a_j + a_{j+4}
  s = s + dpp_shl<1>(s);        // lane 0: s0+s1, lane 2: s2+s3
  return s + dpp_shl<2>(s);     // lane 0: (s0+s1)+(s2+s3)
}

__device__ __forceinline__ int32_t isum8_lanes(int32_t a) {
  a += dpp_shl<4>(a);
  a += dpp_shl<2>(a);
  return a + dpp_shl<1>(a);
}

// rstd = 1 / sqrt(sumsq / n + eps) (bitlinear.cpp:69, rmsnorm.cpp:19)
__device__ __forceinline__ float rstd_of(float ss, int n, float eps) {
  return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

// Sequential reference lane sums (simd.hpp:69-89) over a zero-padded chain-transposed LDS
// vector whose rows are LS floats apart and zero up to a multiple of 32, in two halves so
// other waves can work while wave 0 runs the chains: chain_begin -- thread j < 8 sums row j
// with FMAs in order, 4U values per batch, the next batch loading while the current one is
// summed (the zeros add exact zeros); chain_end (after a barrier) -- hsum + the tail.
// U float4 per batch (4U values; rows are zero to a multiple of 32, so U = 4 or 8).
template <int U = 8>
__device__ inline void chain_begin(const float* X, int Lc, int LS, float* red) {
  static_assert(U == 4 || U == 8, "batches of 16 or 32 values");
  if (threadIdx.x < 8) {
    const float4* c = reinterpret_cast<const float4*>(X + threadIdx.x * LS);
    const int nbat = (Lc + 4 * U - 1) / (4 * U);
    float a = 0.0f;
    float4 A[U], B[U];
#pragma unroll
    for (int u = 0; u < U; ++u) A[u] = c[u];
    for (int b = 0; b < nbat; b += 2) {
      const bool more = b + 1 < nbat;
      if (more)
#pragma unroll
        for (int u = 0; u < U; ++u) B[u] = c[U * (b + 1) + u];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        a = __builtin_fmaf(A[u].x, A[u].x, a);
        a = __builtin_fmaf(A[u].y, A[u].y, a);
        a = __builtin_fmaf(A[u].z, A[u].z, a);
        a = __builtin_fmaf(A[u].w, A[u].w, a);
      }
      if (more) {
        if (b + 2 < nbat)
#pragma unroll
          for (int u = 0; u < U; ++u) A[u] = c[U * (b + 2) + u];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          a = __builtin_fmaf(B[u].x, B[u].x, a);
          a = __builtin_fmaf(B[u].y, B[u].y, a);
          a = __builtin_fmaf(B[u].z, B[u].z, a);
          a = __builtin_fmaf(B[u].w, B[u].w, a);
        }
      }
    }
    red[threadIdx.x] = a;
  }
}

// chain_begin through a ring of 8 float4 registers: a slot is refilled as soon as its four
// values are summed, so seven LDS reads stay in flight ahead of the FMAs instead of the two
// register sets' one batch. chain_ring_part sums positions [0, n) of row j (thread j < 8)
// onto a and returns it, reading whole rounds of 32 values (rows are zero from n to a
// multiple of 32); the last round's refills read up to 32 floats past that (row j + 1, or
// for row 7 the tail and the 32 floats after it, which the LDS area must hold) and are never
// used. The sums and their order are chain_begin's.
__device__ inline float chain_ring_part(const float* X, int n, int LS, float a) {
  constexpr int R = 8;
  const float4* c = reinterpret_cast<const float4*>(X + threadIdx.x * LS);
  const int n4 = (n + 4 * R - 1) / (4 * R) * R;
  float4 V[R];
#pragma unroll
  for (int k = 0; k < R; ++k) V[k] = c[k];
  for (int b = 0; b < n4; b += R) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      a = __builtin_fmaf(V[k].x, V[k].x, a);
      a = __builtin_fmaf(V[k].y, V[k].y, a);
      a = __builtin_fmaf(V[k].z, V[k].z, a);
      a = __builtin_fmaf(V[k].w, V[k].w, a);
      V[k] = c[b + R + k];
    }
  }
  return a;
}
__device__ inline void chain_ring(const float* X, int Lc, int LS, float* red) {
  if (threadIdx.x < 8) red[threadIdx.x] = chain_ring_part(X, Lc, LS, 0.0f);
}

__device__ inline float chain_end(const float* X, int LS, int nt, const float* red) {
  float s = hsum8(red);
  for (int t = 0; t < nt; ++t) {
    const float v = X[8 * LS + t];
    s = __builtin_fmaf(v, v, s);
  }
  return s;
}

// The same sums from registers across one wave: lane 8j + s holds steps [4 RC s, 4 RC (s+1))
// of chain j in v. Segment s of every chain is summed in round s, and a DPP row shift by
// one lane (within rows of 16 lanes, so never across chains j) hands each running sum to
// the lane of the next segment; after round 7 lane 8j + 7 holds chain j. Lanes outside
// their round sum data that the next shift overwrites. Returns hsum_ps of the 8 chains plus
// the tail tv[0..nt) (uniform over the wave). Call from all 64 lanes of one wave.
// seg_sumsq_at runs hook() between rounds HR and HR + 1 (HR < 0: never), fenced against
// scheduling so that what it issues (loads deferred so as not to fill the wave's 63
// outstanding memory requests at entry) stays there.
struct NoHook {
  __device__ void operator()() const {}
};
template <int RC>
__device__ __forceinline__ float seg_sumsq(const float4 (&v)[RC], const float (&tv)[8], int nt);
template <int RC, int HR, class F>
__device__ __forceinline__ float seg_sumsq_at(const float4 (&v)[RC], const float (&tv)[8], int nt, F&& hook) {
  float a = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      a = __builtin_fmaf(v[c].x, v[c].x, a);
      a = __builtin_fmaf(v[c].y, v[c].y, a);
      a = __builtin_fmaf(v[c].z, v[c].z, a);
      a = __builtin_fmaf(v[c].w, v[c].w, a);
    }
    if (s == HR) {
      __builtin_amdgcn_sched_barrier(0);
      hook();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s < 7)
      a = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0x111 /* row_shr:1 */,
                                                                  0xf, 0xf, false));
  }
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 8 * j + 7));
  float s = hsum8(p);
#pragma unroll
  for (int t = 0; t < 7; ++t)
    if (t < nt) s = __builtin_fmaf(tv[t], tv[t], s);
  return s;
}
template <int RC>
__device__ __forceinline__ float seg_sumsq(const float4 (&v)[RC], const float (&tv)[8], int nt) {
  return seg_sumsq_at<RC, -1>(v, tv, nt, NoHook{});
}

// ---- Cephes exp (simd.hpp:212-249) ----------------------------------------------------
constexpr float kExpHi = 88.3762626647949f;
constexpr float kExpLo = -88.3762626647949f;

__device__ __forceinline__ float pow2_of(float fx) {
  return __int_as_float((static_cast<int32_t>(fx) + 127) << 23);
}

__device__ __forceinline__ float exp_poly(float r) {
  float p = 1.9875691500E-4f;
  p = __builtin_fmaf(p, r, 1.3981999507E-3f);
  p = __builtin_fmaf(p, r, 8.3334519073E-3f);
  p = __builtin_fmaf(p, r, 4.1665795894E-2f);
  p = __builtin_fmaf(p, r, 1.6666665459E-1f);
  return __builtin_fmaf(p, r, 5.0000001201E-1f);
}

// 1 + exp(-a), the denominator of sigmoid/silu/swiglu. Body = one lane of the AVX2 path
// (exp8_ps with max/min clamp, p = fma(p, r*r, r+1)); tail = the scalar expf_poly as g++
// contracts it (p = fma(p, r*r, r) + 1). Callers fuse 1 + p*2^n into fma(p, 2^n, 1).
__device__ __forceinline__ float den_body(float a) {
  float x = -a;
  x = (x > kExpLo) ? x : kExpLo;
  x = (x < kExpHi) ? x : kExpHi;
  float fx = floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
  float r = __builtin_fmaf(-fx, 0.693359375f, x);
  r = __builtin_fmaf(-fx, -2.12194440e-4f, r);
  float p = __builtin_fmaf(exp_poly(r), r * r, r + 1.0f);
  return __builtin_fmaf(p, pow2_of(fx), 1.0f);
}

__device__ __noinline__ float den_tail(float a) {
  float x = -a;
  if (x > kExpHi) x = kExpHi;
  else if (x < kExpLo) x = kExpLo;
  float fx = floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
  float r = __builtin_fmaf(-fx, 0.693359375f, x);
  r = __builtin_fmaf(-fx, -2.12194440e-4f, r);
  float p = __builtin_fmaf(exp_poly(r), r * r, r) + 1.0f;
  return __builtin_fmaf(p, pow2_of(fx), 1.0f);
}

// `tail` selects the scalar-tail form: element e of an n-element SIMD call is a tail
// element iff e >= (n & ~7).
__device__ __forceinline__ float den_of(float a, bool tail) { return tail ? den_tail(a) : den_body(a); }
__device__ __forceinline__ float sigmoid_of(float x, bool tail) { return 1.0f / den_of(x, tail); }
__device__ __forceinline__ float silu_of(float x, bool tail) { return x / den_of(x, tail); }
__device__ __forceinline__ float swiglu_of(float a, float b, bool tail) { return (a / den_of(a, tail)) * b; }

// ---- activation quantisers --------------------------------------------------------------
// Q5.10 (simd.hpp:162-187). Body: _mm256_cvtps_epi32 semantics (out of int32 range or
// NaN -> INT32_MIN) then clamp. Tail: nearbyintf, clamp in float, convert.
__device__ __forceinline__ int32_t q510_body(float y, float qs) {
  float v = y * qs;
  int32_t r = (fabsf(v) < 2147483648.0f) ? static_cast<int32_t>(rintf(v)) : INT32_MIN;
  return r < -32768 ? -32768 : (r > 32767 ? 32767 : r);
}
__device__ __forceinline__ int32_t q510_tail(float y, float qs) {
  float v = rintf(y * qs);
  if (v > 32767.0f) v = 32767.0f;
  else if (v < -32768.0f) v = -32768.0f;
  return (v != v) ? INT32_MIN : static_cast<int32_t>(v);
}
// v_cvt_i32_f32: rounds toward zero, saturates out-of-range inputs and gives 0 for NaN (the
// hardware conversion, written out so that its out-of-range result is defined here).
__device__ __forceinline__ int32_t cvt_i32_sat(float v) {
  int32_t r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
  return r;
}
// int8 absmax (tools/reference.py:131-135): q = clamp(round_half_even(y * scale_a), -128, 127).
// The clamp runs on the saturated integer (one v_med3_i32): the same value as a float clamp
// before the conversion for every input, NaN (0) included.
__device__ __forceinline__ int32_t q8_of(float y, float sa) {
  const int32_t c = cvt_i32_sat(rintf(y * sa));
  return c < -128 ? -128 : (c > 127 ? 127 : c);
}

// Byte packing of four codes (code 0 in byte 0) for the int8 planes: FixedQ510 hi = bits
// 8..15 of each code, lo = bits 0..7 minus 128 (the top bit flipped); Int8 the low byte.
// __builtin_amdgcn_perm(a, b, sel) is v_perm_b32: result byte i = byte sel[i] of the
// eight bytes b[0..3], a[0..3] (selector 0x0c gives zero).
__device__ __forceinline__ void pack_split4(const int32_t* c, uint32_t& hi, uint32_t& lo) {
  const uint32_t p01 = __builtin_amdgcn_perm(static_cast<uint32_t>(c[1]), static_cast<uint32_t>(c[0]), 0x04000501u);
  const uint32_t p23 = __builtin_amdgcn_perm(static_cast<uint32_t>(c[3]), static_cast<uint32_t>(c[2]), 0x04000501u);
  hi = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
  lo = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
}
__device__ __forceinline__ uint32_t pack_low4(const int32_t* c) {
  const uint32_t p01 = __builtin_amdgcn_perm(static_cast<uint32_t>(c[1]), static_cast<uint32_t>(c[0]), 0x0c0c0400u);
  const uint32_t p23 = __builtin_amdgcn_perm(static_cast<uint32_t>(c[3]), static_cast<uint32_t>(c[2]), 0x0c0c0400u);
  return __builtin_amdgcn_perm(p23, p01, 0x05040100u);
}

// a / d, correctly rounded, from y = RN(1/d) (Markstein's correction: a first quotient
// RN(a * y), then q + r * y with the exact remainder r = fma(-d, q, a); two corrections).
// Used for the Int8Absmax dequantisation acc / (scale_w * scale_a), where a is an integer
// with |a| <= 2^21 and d, 1/d are normal: for 2000 divisors (the scales' range and random
// ones over 2^-60 .. 2^60) every such a gave the quotient of the division, bit for bit,
// already after one correction.
__device__ __forceinline__ float div_by_recip(float a, float d, float y) {
  float q = a * y;
  float r = __builtin_fmaf(-d, q, a);
  q = __builtin_fmaf(r, y, q);
  r = __builtin_fmaf(-d, q, a);
  return __builtin_fmaf(r, y, q);
}

// Argmax key: order-preserving float bits in the high word (-0 folded onto +0, which the
// reference's `>` cannot tell apart), 0xFFFFFFFF - index in the low word, so the largest key
// is the first index of the largest value (hgrn_model.cpp:270-273).
__device__ __forceinline__ unsigned long long amax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(idx));
}

}  // namespace mmf
