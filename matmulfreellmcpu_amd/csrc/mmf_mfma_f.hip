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
// of one chunk in LDS (double-buffered, loaded a chunk ahead through registers), and each
// lane reads 4 positions of one chain per ds_read_b128. Weights are the 2-bit slabs of the
// GEMV path: the word (group n / 16, chunk c, output n % 16, chain j) holds the 16 codes of
// chain j at t = 16c .. 16c + 15, one v_bfe_i32 + v_cvt_f32_i32 per code.
//
// Chains per wave (CW):
//   CW = 8: each of the 4 waves owns 64 columns and all 8 chains (128 accumulator
//           registers) and reduces them in registers: a 16 x 256 block tile;
//   CW = 2: the 4 waves share one 16 x 64 tile, wave w running chains w and w + 4, for
//           launches with too few tiles to fill the chip (serving steps). Each wave adds
//           its two chains (a_w + a_{w+4}, the first level of hsum_ps) and wave 0 adds the
//           four partial tiles through LDS in the remaining order.
// Epilogues: store, residual add, and the MLP pair (wave columns 0..31 gate outputs c0 ..
// c0+31, columns 32..63 their up partners N/2 later: swiglu in registers).
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kFT = 16;                   // rows of a tile
constexpr int kFRS = 8 * 16 + 4;          // LDS floats per staged row (8 chains x 16, padded)
constexpr int kFBuf = kFT * kFRS;         // LDS floats per chunk buffer

template <int EPI, int CW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_mfma_f(GemmArgs a, ActBuf act) {
  constexpr bool PAIR = EPI == kEpiSwigluPair;
  constexpr int NC = CW;                  // accumulators (chains) per wave
  extern __shared__ float smem[];
  const int z = blockIdx.z;
  const ProjDev& P = a.p[z];
  const Geom& g = P.g;
  const int Lc = act.Lc, Wc = g.Wc;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row0 = blockIdx.y * kFT;
  const int am = (act.na > 1) ? z : 0;
  const int N = g.N, Nh = N / 2;
  // this lane's B column (weight row) and the tile's column base
  int n;
  bool nok;
  int cbase;  // PAIR: first gate column of the wave; else first column of the wave
  if (PAIR) {
    cbase = (blockIdx.x * (CW == 8 ? 4 : 1) + (CW == 8 ? wv : 0)) * 32;
    const int c = cbase + (lane & 31);
    nok = c < Nh;
    n = (lane < 32) ? c : Nh + c;
  } else {
    cbase = (blockIdx.x * (CW == 8 ? 4 : 1) + (CW == 8 ? wv : 0)) * 64;
    n = cbase + lane;
    nok = n < N;
  }
  // chains of this wave
  int jc[NC];
#pragma unroll
  for (int q = 0; q < NC; ++q) jc[q] = (CW == 8) ? q : wv + 4 * q;
  const uint32_t* wrow = P.pk + static_cast<size_t>(nok ? (n >> 4) : 0) * Wc * 128 + (n & 15) * 8;
  auto load_w = [&](int c, uint32_t (&w)[NC]) {
    if constexpr (CW == 8) {
      const uint4* p4 = reinterpret_cast<const uint4*>(wrow + static_cast<size_t>(c) * 128);
      uint4 lo = nok ? p4[0] : make_uint4(0, 0, 0, 0), hi = nok ? p4[1] : make_uint4(0, 0, 0, 0);
      w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w;
      w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
    } else {
#pragma unroll
      for (int q = 0; q < NC; ++q) w[q] = nok ? wrow[static_cast<size_t>(c) * 128 + jc[q]] : 0u;
    }
  };
  // activation tile loads: 512 float4 per chunk, two per thread
  const float* ybase = act.y + (static_cast<size_t>(am) * act.rows + row0) * act.ystride();
  const int nrows = min(kFT, a.rows - row0);
  int ge_off[2], ls_off[2];
  bool ge_ok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = tid + 256 * h, r = e >> 5, ch = (e >> 2) & 7, f4 = e & 3;
    ge_ok[h] = r < nrows;
    ge_off[h] = r * static_cast<int>(act.ystride()) + ch * Lc + 4 * f4;
    ls_off[h] = r * kFRS + ch * 16 + 4 * f4;
  }
  auto load_y = [&](int c, float4 (&v)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v[h] = ge_ok[h] ? *reinterpret_cast<const float4*>(ybase + ge_off[h] + 16 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  v16f acc[NC];
#pragma unroll
  for (int q = 0; q < NC; ++q) acc[q] = v16f{};
  uint32_t wcur[NC], wnext[NC];
  float4 ynext[2];
  load_w(0, wcur);
  load_y(0, ynext);
#pragma unroll
  for (int h = 0; h < 2; ++h) *reinterpret_cast<float4*>(smem + ls_off[h]) = ynext[h];
  __syncthreads();
  const int ri = lane & 15;  // this lane's A row within the tile
  for (int c = 0; c < Wc; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < Wc;
    if (more) {
      load_w(c + 1, wnext);
      load_y(c + 1, ynext);
    }
    const float* yl = smem + buf * kFBuf + ri * kFRS;
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) {
      float4 av[NC];
#pragma unroll
      for (int q = 0; q < NC; ++q) av[q] = *reinterpret_cast<const float4*>(yl + jc[q] * 16 + 4 * tq);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
        for (int q = 0; q < NC; ++q) {
          const float y = tt == 0 ? av[q].x : tt == 1 ? av[q].y : tt == 2 ? av[q].z : av[q].w;
          acc[q] = __builtin_amdgcn_mfma_f32_16x16x1f32(y, code_f(wcur[q], 4 * tq + tt), acc[q], 0, 0, 0);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int h = 0; h < 2; ++h) *reinterpret_cast<float4*>(smem + (buf ^ 1) * kFBuf + ls_off[h]) = ynext[h];
#pragma unroll
      for (int q = 0; q < NC; ++q) wcur[q] = wnext[q];
    }
    __syncthreads();
  }
  // ---- chain reduction in the hsum_ps order --------------------------------------------
  float val[16];
  if constexpr (CW == 8) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      val[r] = ((acc[0][r] + acc[4][r]) + (acc[1][r] + acc[5][r])) + ((acc[2][r] + acc[6][r]) + (acc[3][r] + acc[7][r]));
  } else {
    // partial s_w = a_w + a_{w+4}; LDS [w][r][lane]; wave 0 finishes (s0 + s1) + (s2 + s3)
#pragma unroll
    for (int r = 0; r < 16; ++r) smem[(wv * 16 + r) * 64 + lane] = acc[0][r] + acc[1][r];
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      val[r] = (smem[(0 * 16 + r) * 64 + lane] + smem[(1 * 16 + r) * 64 + lane]) +
               (smem[(2 * 16 + r) * 64 + lane] + smem[(3 * 16 + r) * 64 + lane]);
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

template <int EPI, int CW>
hipError_t mfma_f_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int per = (EPI == kEpiSwigluPair ? 32 : 64) * (CW == 8 ? 4 : 1);
  const int cols = EPI == kEpiSwigluPair ? g.N / 2 : g.N;
  dim3 grid((cols + per - 1) / per, (a.rows + kFT - 1) / kFT, EPI == kEpiSwigluPair ? 1 : a.nmat);
  const size_t lds = 2 * kFBuf * sizeof(float);  // also holds CW = 2's 4 x 16 x 64 partials
  static_assert(2 * kFBuf >= 4 * 16 * 64, "reduction buffer");
  k_mfma_f<EPI, CW><<<grid, 256, lds, s>>>(a, act);
  return hipGetLastError();
}

template <int EPI>
hipError_t mfma_f_epi(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Geom& g = a.p[0].g;
  const int cols = EPI == kEpiSwigluPair ? g.N / 2 : g.N;
  const int per8 = (EPI == kEpiSwigluPair ? 32 : 64) * 4;
  const long blocks8 = static_cast<long>((cols + per8 - 1) / per8) * ((a.rows + kFT - 1) / kFT) *
                       (EPI == kEpiSwigluPair ? 1 : a.nmat);
  // all 8 chains per wave while that gives at least two blocks per CU
  if (blocks8 >= 512) return mfma_f_inst<EPI, 8>(a, act, s);
  return mfma_f_inst<EPI, 2>(a, act, s);
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
