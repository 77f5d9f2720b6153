// mmf_mfma_f.hip -- the float-mode ternary GEMM on the CDNA4 matrix cores, bit-exact.
//
// The reference's float BitLinear (simd.hpp:92-122) keeps 8 AVX2 lanes per output: lane j
// runs acc_j = fma(y_k, w_k, acc_j) over k = j + 8t in t order, the lanes are summed in the
// hsum_ps order ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), and the K % 8 tail is added after.
// With w_k in {-1, 0, +1} the product y_k * w_k is exact, so fma(y, w, acc) is the single
// rounding of acc + y*w. The fp32 matrix ops with one product per element (K = 1:
// v_mfma_f32_32x32x1_2b_f32, v_mfma_f32_16x16x1_4b_f32) compute D = C + A*B, so a chain of
// them on one accumulator, fed the chain's positions in t order, reproduces acc_j bit for bit
// (denormals included). Each chain is its own accumulator tile, run by its own wave: 8 waves
// per tile, wave j running chain j; the 8 chain tiles meet in LDS, and each wave adds an
// eighth of the outputs in the hsum_ps order where it stores them.
//
// Operands go straight to registers, 3 chunks of 16 chain positions in flight per wave (no
// wave shares another's activations, so there is no LDS staging and no barrier until the
// reduction): lane l reads 4 positions of its row's chain per float4 load. Activations are
// the fp32 chain rows of the prologue (row r, chain j, position t at y[r * (8 Lc + 8) +
// j * Lc + t]). Weights are the 2-bit slabs of the GEMV path: the word (group n / 16, chunk
// c, output n % 16, chain j) holds the 16 codes of chain j at t = 16c .. 16c + 15, one
// v_bfe_i32 + v_cvt_f32_i32 per code. A wave issues a matrix op only about every 70 cycles
// whatever its number of accumulators, so one chain per wave (the most waves per tile)
// measured fastest at every size.
//
// Two tilings, chosen by how many tiles a launch has (mfma_f_epi):
//   k_mfma_f32w: 32 x 64 tiles of the 32x32x1 instruction (2048 MACs per op: half the ops
//     per wave of two 16-row tiles), from 384 16-row tiles on (prefill, the serving steps'
//     i/f/g and gate/up GEMMs);
//   k_mfma_f1: 16 x 64 tiles of the 16x16x1 instruction (4 blocks of 16 columns side by
//     side, all with the same 16 rows) for narrower launches (the serving steps' o/down).
// Epilogues: store, residual add, and the MLP pair (B columns 0..31 gate outputs c0 ..
// c0+31, columns 32..63 their up partners N/2 later: swiglu in registers).
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

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
  // every lane loads from an in-range row and chunk (rows past the last are multiplied but
  // never stored; a column past the last multiplies zero codes), so every chunk issues the
  // same five loads unconditionally and the compiler waits for each chunk with a constant
  // count, S - 1 chunks of loads still in flight (a conditional load made it wait for all)
  const int ri = lane & 31;
  const int rl = min(row0 + ri, a.rows - 1);
  const float* yrow = act.y + (static_cast<size_t>(am) * act.rows + rl) * act.ystride() + j * Lc;
  auto load = [&](int c, float4 (&v)[4], uint32_t& w) {
    c = min(c, Wc - 1);
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) v[tq] = *reinterpret_cast<const float4*>(yrow + 16 * c + 4 * tq);
    w = wrow[static_cast<size_t>(c) * 128];
  };
  v32f acc = v32f{};
  float4 ar[S][4];
  uint32_t wr[S];
  // (issued in chunk order, which the scheduler must keep: the first chunk's loads issued
  // last would make every wait count zero)
#pragma unroll
  for (int u = 0; u < S; ++u) {
    load(u, ar[u], wr[u]);
    __builtin_amdgcn_sched_barrier(0);
  }
  auto chunk = [&](int u) {  // the 16 positions of the chunk in ring slot u, in t order
#pragma unroll
    for (int tq = 0; tq < 4; ++tq)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float4 v = ar[u][tq];
        const float y = tt == 0 ? v.x : tt == 1 ? v.y : tt == 2 ? v.z : v.w;
        acc = __builtin_amdgcn_mfma_f32_32x32x1f32(y, code_f(nok ? wr[u] : 0u, 4 * tq + tt), acc, 0, 0, 0);
      }
  };
  // whole runs of S chunks (no exit inside a run: the same loads and waits in every run),
  // then the last Wc % S chunks, which load nothing
  int c0 = 0;
  for (; c0 + S <= Wc; c0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      chunk(u);
      load(c0 + u + S, ar[u], wr[u]);  // refilled as soon as its chunk has used it
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (c0 + u < Wc) chunk(u);
  // chain tiles through LDS [j][r][lane]; then every wave adds, in the hsum_ps order, and
  // stores the outputs of accumulator rows r = j (mod 8): an eighth of the tile each
  // (wave 0 alone took 10.7k cycles for a 32 x 64 tile)
  constexpr int PS = 32 * 64;
#pragma unroll
  for (int r = 0; r < 32; ++r) smem[j * PS + r * 64 + lane] = acc[r];
  __syncthreads();
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
    for (int r = j; r < 16; r += 8) {
      const int row = row0 + 8 * (r >> 2) + rq + (r & 3);
      const int c = cbase + col;
      if (row >= a.rows || c >= Nh) continue;
      const float vg = finish(hsum(r), c, row), vu = finish(hsum(r + 16), Nh + c, row);
      const size_t e = static_cast<size_t>(row) * Nh + c;
      a.out[0][e] = swiglu_of(vg, vu, static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
    }
  } else {
    for (int r = j; r < 32; r += 8) {
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
  const int rl = min(row0 + ri, a.rows - 1);  // in-range loads only, as in k_mfma_f32w
  const float* yrow = act.y + (static_cast<size_t>(am) * act.rows + rl) * act.ystride() + j * Lc;
  auto load = [&](int c, float4 (&v)[4], uint32_t& w) {
    c = min(c, Wc - 1);
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) v[tq] = *reinterpret_cast<const float4*>(yrow + 16 * c + 4 * tq);
    w = wrow[static_cast<size_t>(c) * 128];
  };
  v16f acc = v16f{};
  float4 ar[S][4];
  uint32_t wr[S];
  // (issued in chunk order, which the scheduler must keep: the first chunk's loads issued
  // last would make every wait count zero)
#pragma unroll
  for (int u = 0; u < S; ++u) {
    load(u, ar[u], wr[u]);
    __builtin_amdgcn_sched_barrier(0);
  }
  auto chunk = [&](int u) {  // the 16 positions of the chunk in ring slot u, in t order
#pragma unroll
    for (int tq = 0; tq < 4; ++tq)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float4 v = ar[u][tq];
        const float y = tt == 0 ? v.x : tt == 1 ? v.y : tt == 2 ? v.z : v.w;
        acc = __builtin_amdgcn_mfma_f32_16x16x1f32(y, code_f(nok ? wr[u] : 0u, 4 * tq + tt), acc, 0, 0, 0);
      }
  };
  // whole runs of S chunks (no exit inside a run: the same loads and waits in every run),
  // then the last Wc % S chunks, which load nothing
  int c0 = 0;
  for (; c0 + S <= Wc; c0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      chunk(u);
      load(c0 + u + S, ar[u], wr[u]);  // refilled as soon as its chunk has used it
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (c0 + u < Wc) chunk(u);
  constexpr int PS = 16 * 64;  // floats of one chain's tile in LDS [j][r][lane]
#pragma unroll
  for (int r = 0; r < 16; ++r) smem[j * PS + r * 64 + lane] = acc[r];
  __syncthreads();
  // each output's 8 chain values are added where it is stored, wave j taking accumulator
  // rows r = j (mod 8), as in k_mfma_f32w
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
  const int col = lane & 15, rq = 4 * (lane >> 4);
  if (PAIR) {
    for (int r = j; r < 8; r += 8) {
      const int row = row0 + rq + (r & 3);
      const int c = cbase + 16 * (r >> 2) + col;
      if (row >= a.rows || c >= Nh) continue;
      const float vg = finish(hsum(r), c, row), vu = finish(hsum(r + 8), Nh + c, row);
      const size_t e = static_cast<size_t>(row) * Nh + c;
      a.out[0][e] = swiglu_of(vg, vu, static_cast<int64_t>(e) >= (a.swiglu_n & ~7));
    }
  } else {
    for (int r = j; r < 16; r += 8) {
      const int row = row0 + rq + (r & 3);
      const int o = cbase + 16 * (r >> 2) + col;
      if (row >= a.rows || o >= N) continue;
      const float v = finish(hsum(r), o, row);
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

// 16 x 64 tiles of a launch (16 x 32 gate columns with their up partners for the pair)
template <int EPI>
long mfma_f_tiles16(const GemmArgs& a) {
  const int per = EPI == kEpiSwigluPair ? 32 : 64;
  const int cols = EPI == kEpiSwigluPair ? a.p[0].g.N / 2 : a.p[0].g.N;
  return static_cast<long>((cols + per - 1) / per) * ((a.rows + 15) / 16) * (EPI == kEpiSwigluPair ? 1 : a.nmat);
}


// 32 x 64 tiles of the 32x32 instruction while there would be at least 384 16-row tiles (1.5
// per CU), else 16 x 64 tiles
template <int EPI>
hipError_t mfma_f_epi(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (mfma_f_tiles16<EPI>(a) >= 384) return mfma_f32w_inst<EPI>(a, act, s);
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
