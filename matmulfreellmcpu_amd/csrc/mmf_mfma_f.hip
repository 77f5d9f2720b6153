// mmf_mfma_f.hip -- the float-mode ternary GEMM on the CDNA4 matrix cores, bit-exact.
//
// The reference's float BitLinear (simd.hpp:92-122) keeps 8 AVX2 lanes per output: lane j
// runs acc_j = fma(y_k, w_k, acc_j) over k = j + 8t in t order, the lanes are summed in the
// hsum_ps order ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), and the K % 8 tail is added after.
// With w_k in {-1, 0, +1} the product y_k * w_k is exact, so fma(y, w, acc) is the single
// rounding of acc + y*w. v_mfma_f32_16x16x1_4b_f32 computes D = C + A*B per element with
// one product (K = 1), so a chain of these instructions on one accumulator, fed the chain's
// positions in t order, reproduces acc_j bit for bit (denormals included). Each chain is
// its own accumulator tile, so the instruction order across chains is free, and the 8
// chains give 8 independent accumulators to keep the matrix core busy.
//
// Instruction layout (4 blocks of 16 x 16 x 1): lane l supplies A = y[row l % 16] and
// B = w[column l] of block l / 16; accumulator r of lane l is block r / 4, row
// 4 * (l / 16) + r % 4, column l % 16. Here all four blocks take the same 16 rows and
// lane l's B is column n0 + l (four 16-column blocks side by side), so a wave computes a
// 16-row x 64-column tile per instruction and position.
//
// Operands. Activations are the fp32 chain rows of the prologue (row r, chain j, position
// t at y[r * (8 Lc + 8) + j * Lc + t]); a block stages the 16 rows x 8 chains x 16 positions
// of one chunk in one of two LDS slots (loaded several chunks ahead into register sets), and each
// lane reads 4 positions of one chain per ds_read_b128. Weights are the 2-bit slabs of the
// GEMV path: the word (group n / 16, chunk c, output n % 16, chain j) holds the 16 codes of
// chain j at t = 16c .. 16c + 15, one v_bfe_i32 + v_cvt_f32_i32 per code.
//
// Three tilings, chosen by how many tiles a launch has (mfma_f_epi):
//   k_mfma_f (long row ranges, prefill): a block is 32 rows x 128 columns. Each wave has two
//     16-row subtiles that share each decoded weight, and 4 of the 8 chains: the wave pair of
//     a column group runs chains {0, 4, 1, 5} and {2, 6, 3, 7}, 128 accumulator registers,
//     two waves per SIMD. The activation tile is staged through LDS.
//   k_mfma_f32w (mid-size launches: the serving steps' i/f/g and gate/up GEMMs): 32 x 64
//     tiles of the 32x32x1 instruction, one chain per wave, operands straight to registers.
//   k_mfma_f1 (narrow launches: the serving steps' o/down GEMMs): 16 x 64 tiles, one chain
//     per wave, 8 waves per tile, operands straight to registers.
// The waves add their chains in the hsum_ps order, through LDS across waves.
// Epilogues: store, residual add, and the MLP pair (wave columns 0..31 gate outputs c0 ..
// c0+31, columns 32..63 their up partners N/2 later: swiglu in registers).
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int kFRS = 8 * 16 + 4;  // LDS floats per staged row (8 chains x 16 positions, padded)

template <int EPI, int RM, int CW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_mfma_f(GemmArgs a, ActBuf act) {
  static_assert(RM == 2 && CW == 4, "32 x 128 block tiles: two 16-row subtiles, 4 chains per wave");
  constexpr bool PAIR = EPI == kEpiSwigluPair;
  constexpr int NC = CW, TR = 16 * RM, S = 2, BUFF = TR * kFRS, WH = 8 / CW, WCOL = 4 / WH;
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc, Wc = g.Wc;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wh = wv % WH, wc = wv / WH;
  const int row0 = blockIdx.y * TR;
  const int am = (act.na > 1) ? z : 0;
  const int N = g.N, Nh = N / 2;
  // this lane's B column (weight row) and the wave's first output column
  int n, cbase;
  bool nok;
  if (PAIR) {
    cbase = (blockIdx.x * WCOL + wc) * 32;
    const int c = cbase + (lane & 31);
    nok = c < Nh;
    n = (lane < 32) ? c : Nh + c;
  } else {
    cbase = (blockIdx.x * WCOL + wc) * 64;
    n = cbase + lane;
    nok = n < N;
  }
  int jc[NC];
#pragma unroll
  for (int q = 0; q < NC; ++q) jc[q] = 2 * wh + (q >> 1) + 4 * (q & 1);  // {2wh, 2wh+4, 2wh+1, 2wh+5}
  const uint32_t* wrow = P.pk + static_cast<size_t>(nok ? (n >> 4) : 0) * Wc * 128 + (n & 15) * 8;
  auto load_w = [&](int c, uint32_t (&w)[NC]) {
#pragma unroll
    for (int q = 0; q < NC; ++q) w[q] = nok ? wrow[static_cast<size_t>(c) * 128 + jc[q]] : 0u;
  };
  // activation tile loads: TR rows x 8 chains x 4 float4 per chunk, 2 RM per thread
  const float* ybase = act.y + (static_cast<size_t>(am) * act.rows + row0) * act.ystride();
  const int nrows = min(TR, a.rows - row0);
  constexpr int NL = 2 * RM;
  int ge_off[NL], ls_off[NL];
  bool ge_ok[NL];
#pragma unroll
  for (int h = 0; h < NL; ++h) {
    const int e = tid + 256 * h, r = e >> 5, ch = (e >> 2) & 7, f4 = e & 3;
    ge_ok[h] = r < nrows;
    ge_off[h] = r * static_cast<int>(act.ystride()) + ch * Lc + 4 * f4;
    ls_off[h] = r * kFRS + ch * 16 + 4 * f4;
  }
  auto load_y = [&](int c, float4 (&v)[NL]) {
#pragma unroll
    for (int h = 0; h < NL; ++h)
      v[h] = ge_ok[h] ? *reinterpret_cast<const float4*>(ybase + ge_off[h] + 16 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  v16f acc[RM][NC];
#pragma unroll
  for (int m = 0; m < RM; ++m)
#pragma unroll
    for (int q = 0; q < NC; ++q) acc[m][q] = v16f{};
  const int ri = lane & 15;  // this lane's A row within a subtile
  // S register sets in flight: set u holds the activations and weights of the chunks
  // c = u (mod S). Chunk c's activations are loaded at the top of iteration c - S, written to
  // LDS slot (c & 1) at the bottom of iteration c - 1; its weights are loaded at the bottom of
  // iteration c - S and used in iteration c. The loop body is unrolled S times so that every
  // set index is a compile-time constant.
  float4 yr[S][NL];
  uint32_t wr[S][NC];
#pragma unroll
  for (int u = 0; u < S; ++u)
    if (u < Wc) {
      load_y(u, yr[u]);
      load_w(u, wr[u]);
    }
#pragma unroll
  for (int h = 0; h < NL; ++h) *reinterpret_cast<float4*>(smem + ls_off[h]) = yr[0][h];
  __syncthreads();
  for (int c0 = 0; c0 < Wc; c0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int c = c0 + u;
      if (c >= Wc) break;
      const float* yb = smem + (c & 1) * BUFF + ri * kFRS;
      if (c + S < Wc) load_y(c + S, yr[u]);
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        float4 av[RM][NC];
#pragma unroll
        for (int m = 0; m < RM; ++m)
#pragma unroll
          for (int q = 0; q < NC; ++q) av[m][q] = *reinterpret_cast<const float4*>(yb + 16 * m * kFRS + jc[q] * 16 + 4 * tq);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
          for (int q = 0; q < NC; ++q) {
            const float b = code_f(wr[u][q], 4 * tq + tt);
#pragma unroll
            for (int m = 0; m < RM; ++m) {
              const float y = tt == 0 ? av[m][q].x : tt == 1 ? av[m][q].y : tt == 2 ? av[m][q].z : av[m][q].w;
              acc[m][q] = __builtin_amdgcn_mfma_f32_16x16x1f32(y, b, acc[m][q], 0, 0, 0);
            }
          }
        }
      }
      if (c + 1 < Wc) {
#pragma unroll
        for (int h = 0; h < NL; ++h)
          *reinterpret_cast<float4*>(smem + ((c + 1) & 1) * BUFF + ls_off[h]) = yr[(u + 1) % S][h];
      }
      if (c + S < Wc) load_w(c + S, wr[u]);
      __syncthreads();
    }
  }
  // ---- chain reduction in the hsum_ps order --------------------------------------------
  float val[RM][16];
  {
    // partial tiles in LDS [wc][wh][m][r][lane]: s_{2wh} + s_{2wh+1} (s_j = a_j + a_{j+4})
    constexpr int PS = RM * 16 * 64;  // floats of one wave's partial tile
#pragma unroll
    for (int m = 0; m < RM; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = (acc[m][0][r] + acc[m][1][r]) + (acc[m][2][r] + acc[m][3][r]);
        smem[(wc * WH + wh) * PS + (m * 16 + r) * 64 + lane] = p;
      }
    __syncthreads();
    if (wh != 0) return;
    const float* rp = smem + wc * WH * PS + lane;
#pragma unroll
    for (int m = 0; m < RM; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = (m * 16 + r) * 64;
        val[m][r] = rp[o] + rp[PS + o];
      }
  }
  // ---- tails, scale, epilogue ----------------------------------------------------------
  const int col = lane & 15, rq = 4 * (lane >> 4);
  auto finish = [&](float s, int o, int row) {
    const float* yt = act.y + (static_cast<size_t>(am) * act.rows + row) * act.ystride() + 8 * Lc;
    for (int t = 0; t < g.ntail; ++t) {
      const int8_t wt = P.tail[o * 8 + t];
      if (wt > 0) s += yt[t];
      else if (wt < 0) s -= yt[t];
    }
    return s * P.inv_scale_w;
  };
#pragma unroll
  for (int m = 0; m < RM; ++m) {
    if (PAIR) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int row = row0 + 16 * m + rq + (r & 3);
        const int c = cbase + 16 * (r >> 2) + col;
        if (row >= a.rows || c >= Nh) continue;
        const float vg = finish(val[m][r], c, row), vu = finish(val[m][r + 8], Nh + c, row);
        const size_t e = static_cast<size_t>(row) * Nh + c;
        a.out[0][e] = swiglu_of(vg, vu, static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + 16 * m + rq + (r & 3);
        const int o = cbase + 16 * (r >> 2) + col;
        if (row >= a.rows || o >= N) continue;
        const float v = finish(val[m][r], o, row);
        const size_t e = static_cast<size_t>(row) * N + o;
        a.out[z][e] = (EPI == kEpiAdd) ? a.add[e] + v : v;
      }
    }
  }
}

// 32-row x 64-column tiles on v_mfma_f32_32x32x1_2b_f32 (the two blocks are the two 32-column
// halves; accumulator r of lane l is block r / 16, row 8 ((r % 16) / 4) + 4 (l / 32) + r % 4,
// column l % 32), one chain per wave, 8 waves (512 threads) per tile, operands straight to
// registers: for launches with enough 16-row tiles that each wave's longer instructions pay
// (the serving steps' i/f/g and gate/up GEMMs: 64 x 2560 x 7680 in 33 us, 64 x 2560 x 13824
// in 58 us, against 42 and 76 us on 16-row tiles with two chains per wave).
template <int EPI>
__global__ __launch_bounds__(512) void k_mfma_f32w(GemmArgs a, ActBuf act) {
  constexpr bool PAIR = EPI == kEpiSwigluPair;
  constexpr int S = 3;
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc, Wc = g.Wc;
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's chain
  const int row0 = blockIdx.y * 32;
  const int am = (act.na > 1) ? z : 0;
  const int N = g.N, Nh = N / 2;
  int n, cbase;
  bool nok;
  if (PAIR) {
    cbase = blockIdx.x * 32;  // gate columns cbase + lane % 32 (block 0), up partners N/2 later (block 1)
    const int c = cbase + (lane & 31);
    nok = c < Nh;
    n = (lane < 32) ? c : Nh + c;
  } else {
    cbase = blockIdx.x * 64;
    n = cbase + lane;
    nok = n < N;
  }
  const uint32_t* wrow = P.pk + static_cast<size_t>(nok ? (n >> 4) : 0) * Wc * 128 + (n & 15) * 8 + j;
  const int ri = lane & 31;
  const bool rok = row0 + ri < a.rows;
  const float* yrow = act.y + (static_cast<size_t>(am) * act.rows + row0 + ri) * act.ystride() + j * Lc;
  auto load = [&](int c, float4 (&v)[4], uint32_t& w) {
#pragma unroll
    for (int tq = 0; tq < 4; ++tq)
      v[tq] = rok ? *reinterpret_cast<const float4*>(yrow + 16 * c + 4 * tq) : make_float4(0.f, 0.f, 0.f, 0.f);
    w = nok ? wrow[static_cast<size_t>(c) * 128] : 0u;
  };
  v32f acc = v32f{};
  float4 ar[S][4];
  uint32_t wr[S];
#pragma unroll
  for (int u = 0; u < S; ++u)
    if (u < Wc) load(u, ar[u], wr[u]);
  for (int c0 = 0; c0 < Wc; c0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int c = c0 + u;
      if (c >= Wc) break;
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const float4 v = ar[u][tq];
          const float y = tt == 0 ? v.x : tt == 1 ? v.y : tt == 2 ? v.z : v.w;
          acc = __builtin_amdgcn_mfma_f32_32x32x1f32(y, code_f(wr[u], 4 * tq + tt), acc, 0, 0, 0);
        }
      if (c + S < Wc) load(c + S, ar[u], wr[u]);
    }
  }
  // chain tiles through LDS [j][r][lane]; wave 0 adds them in the hsum_ps order
  constexpr int PS = 32 * 64;
#pragma unroll
  for (int r = 0; r < 32; ++r) smem[j * PS + r * 64 + lane] = acc[r];
  __syncthreads();
  if (j != 0) return;
  // each output's 8 chain values are added where it is stored (no 32-value array live)
  auto hsum = [&](int r) {
    const float* p = smem + r * 64 + lane;
    return ((p[0] + p[4 * PS]) + (p[PS] + p[5 * PS])) + ((p[2 * PS] + p[6 * PS]) + (p[3 * PS] + p[7 * PS]));
  };
  auto finish = [&](float sum, int o, int row) {
    const float* yt = act.y + (static_cast<size_t>(am) * act.rows + row) * act.ystride() + 8 * Lc;
    for (int t = 0; t < g.ntail; ++t) {
      const int8_t wt = P.tail[o * 8 + t];
      if (wt > 0) sum += yt[t];
      else if (wt < 0) sum -= yt[t];
    }
    return sum * P.inv_scale_w;
  };
  const int col = lane & 31, rq = 4 * (lane >> 5);
  if (PAIR) {
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + 8 * (r >> 2) + rq + (r & 3);
      const int c = cbase + col;
      if (row >= a.rows || c >= Nh) continue;
      const float vg = finish(hsum(r), c, row), vu = finish(hsum(r + 16), Nh + c, row);
      const size_t e = static_cast<size_t>(row) * Nh + c;
      a.out[0][e] = swiglu_of(vg, vu, static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
    }
  } else {
    for (int r = 0; r < 32; ++r) {
      const int rr = r & 15;
      const int row = row0 + 8 * (rr >> 2) + rq + (rr & 3);
      const int o = cbase + 32 * (r >> 4) + col;
      if (row >= a.rows || o >= N) continue;
      const float v = finish(hsum(r), o, row);
      const size_t e = static_cast<size_t>(row) * N + o;
      a.out[z][e] = (EPI == kEpiAdd) ? a.add[e] + v : v;
    }
  }
}

template <int EPI>
__global__ __launch_bounds__(512) void k_mfma_f1(GemmArgs a, ActBuf act) {
  constexpr bool PAIR = EPI == kEpiSwigluPair;
  constexpr int S = 3;
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc, Wc = g.Wc;
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's chain
  const int row0 = blockIdx.y * 16;
  const int am = (act.na > 1) ? z : 0;
  const int N = g.N, Nh = N / 2;
  int n, cbase;
  bool nok;
  if (PAIR) {
    cbase = blockIdx.x * 32;
    const int c = cbase + (lane & 31);
    nok = c < Nh;
    n = (lane < 32) ? c : Nh + c;
  } else {
    cbase = blockIdx.x * 64;
    n = cbase + lane;
    nok = n < N;
  }
  const uint32_t* wrow = P.pk + static_cast<size_t>(nok ? (n >> 4) : 0) * Wc * 128 + (n & 15) * 8 + j;
  const int ri = lane & 15;
  const bool rok = row0 + ri < a.rows;
  const float* yrow = act.y + (static_cast<size_t>(am) * act.rows + row0 + ri) * act.ystride() + j * Lc;
  auto load = [&](int c, float4 (&v)[4], uint32_t& w) {
#pragma unroll
    for (int tq = 0; tq < 4; ++tq)
      v[tq] = rok ? *reinterpret_cast<const float4*>(yrow + 16 * c + 4 * tq) : make_float4(0.f, 0.f, 0.f, 0.f);
    w = nok ? wrow[static_cast<size_t>(c) * 128] : 0u;
  };
  v16f acc = v16f{};
  float4 ar[S][4];
  uint32_t wr[S];
#pragma unroll
  for (int u = 0; u < S; ++u)
    if (u < Wc) load(u, ar[u], wr[u]);
  for (int c0 = 0; c0 < Wc; c0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int c = c0 + u;
      if (c >= Wc) break;
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const float4 v = ar[u][tq];
          const float y = tt == 0 ? v.x : tt == 1 ? v.y : tt == 2 ? v.z : v.w;
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(y, code_f(wr[u], 4 * tq + tt), acc, 0, 0, 0);
        }
      if (c + S < Wc) load(c + S, ar[u], wr[u]);
    }
  }
  constexpr int PS = 16 * 64;  // floats of one chain's tile in LDS [j][r][lane]
#pragma unroll
  for (int r = 0; r < 16; ++r) smem[j * PS + r * 64 + lane] = acc[r];
  __syncthreads();
  if (j != 0) return;
  float val[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float* p = smem + r * 64 + lane;
    val[r] = ((p[0] + p[4 * PS]) + (p[PS] + p[5 * PS])) + ((p[2 * PS] + p[6 * PS]) + (p[3 * PS] + p[7 * PS]));
  }
  auto finish = [&](float sum, int o, int row) {
    const float* yt = act.y + (static_cast<size_t>(am) * act.rows + row) * act.ystride() + 8 * Lc;
    for (int t = 0; t < g.ntail; ++t) {
      const int8_t wt = P.tail[o * 8 + t];
      if (wt > 0) sum += yt[t];
      else if (wt < 0) sum -= yt[t];
    }
    return sum * P.inv_scale_w;
  };
  const int col = lane & 15, rq = 4 * (lane >> 4);
  if (PAIR) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = row0 + rq + (r & 3);
      const int c = cbase + 16 * (r >> 2) + col;
      if (row >= a.rows || c >= Nh) continue;
      const float vg = finish(val[r], c, row), vu = finish(val[r + 8], Nh + c, row);
      const size_t e = static_cast<size_t>(row) * Nh + c;
      a.out[0][e] = swiglu_of(vg, vu, static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + rq + (r & 3);
      const int o = cbase + 16 * (r >> 2) + col;
      if (row >= a.rows || o >= N) continue;
      const float v = finish(val[r], o, row);
      const size_t e = static_cast<size_t>(row) * N + o;
      a.out[z][e] = (EPI == kEpiAdd) ? a.add[e] + v : v;
    }
  }
}

template <int EPI>
hipError_t mfma_f1_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int per = EPI == kEpiSwigluPair ? 32 : 64;
  const int cols = EPI == kEpiSwigluPair ? g.N / 2 : g.N;
  dim3 grid((cols + per - 1) / per, (a.rows + 15) / 16, EPI == kEpiSwigluPair ? 1 : a.nmat);
  k_mfma_f1<EPI><<<grid, 512, 8 * 16 * 64 * sizeof(float), s>>>(a, act);
  return hipGetLastError();
}

template <int EPI>
hipError_t mfma_f32w_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int per = EPI == kEpiSwigluPair ? 32 : 64;
  const int cols = EPI == kEpiSwigluPair ? g.N / 2 : g.N;
  dim3 grid((cols + per - 1) / per, (a.rows + 31) / 32, EPI == kEpiSwigluPair ? 1 : a.nmat);
  k_mfma_f32w<EPI><<<grid, 512, 8 * 32 * 64 * sizeof(float), s>>>(a, act);
  return hipGetLastError();
}

template <int EPI, int RM, int CW>
long mfma_f_blocks(const GemmArgs& a) {
  const int per = (EPI == kEpiSwigluPair ? 32 : 64) * (CW / 2);
  const int cols = EPI == kEpiSwigluPair ? a.p[0].g.N / 2 : a.p[0].g.N;
  return static_cast<long>((cols + per - 1) / per) * ((a.rows + 16 * RM - 1) / (16 * RM)) *
         (EPI == kEpiSwigluPair ? 1 : a.nmat);
}

template <int EPI, int RM, int CW>
hipError_t mfma_f_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int per = (EPI == kEpiSwigluPair ? 32 : 64) * (CW / 2);
  const int cols = EPI == kEpiSwigluPair ? g.N / 2 : g.N;
  dim3 grid((cols + per - 1) / per, (a.rows + 16 * RM - 1) / (16 * RM), EPI == kEpiSwigluPair ? 1 : a.nmat);
  const size_t ring = static_cast<size_t>(2) * 16 * RM * kFRS * sizeof(float);
  const size_t red = static_cast<size_t>(4) * RM * 16 * 64 * sizeof(float);
  k_mfma_f<EPI, RM, CW><<<grid, 256, ring > red ? ring : red, s>>>(a, act);
  return hipGetLastError();
}

// 32 x 128 block tiles while that leaves at least 1024 blocks (four per CU); else 32 x 64
// tiles of the 32x32 instruction while there would be at least 384 16-row tiles (1.5 per
// CU: 64 x 2560 x 7680 37 against 42 us, 64 x 2560 x 13824 58 against 76 us), else 16 x 64
// tiles with one chain per wave
template <int EPI>
hipError_t mfma_f_epi(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (mfma_f_blocks<EPI, 2, 4>(a) >= 1024) return mfma_f_inst<EPI, 2, 4>(a, act, s);
  if (mfma_f_blocks<EPI, 1, 2>(a) >= 384) return mfma_f32w_inst<EPI>(a, act, s);
  return mfma_f1_inst<EPI>(a, act, s);
}

}  // namespace

bool mfma_f_ok(const GemmArgs& a) {
  if (a.mode != kFloat) return false;
  const Geom& g = a.p[0].g;
  if (a.epi == kEpiSwigluPair && (g.N % 32) != 0) return false;  // gate/up halves of whole 16-col groups
  return true;
}

hipError_t launch_gemm_mfma_f(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  switch (a.epi) {
    case kEpiSwigluPair: return mfma_f_epi<kEpiSwigluPair>(a, act, s);
    case kEpiAdd: return mfma_f_epi<kEpiAdd>(a, act, s);
    default: return mfma_f_epi<kEpiStore>(a, act, s);
  }
}

}  // namespace mmf
