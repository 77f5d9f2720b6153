// mmf_mfma.hip -- the ternary GEMM of the integer modes on the CDNA4 matrix cores.
//
// C[row, o] = sum_p A[row, p] * W[o, p] over the chain-permuted positions p < 8*Lc, with
// A the int8 activation planes (FixedQ510: hi and lo planes of the split Q5.10 code; Int8:
// one plane) and W the ternary weights. Every product and sum is exact in int32, so the
// order in which the matrix cores add them does not matter: the result equals the
// reference's integer dot products (simd.hpp:125-154) bit for bit.
//
// Instruction: v_mfma_i32_32x32x32_i8 (on gfx950 it issues at about 1.6x the int8 rate of
// the 16x16x64 form). Lane l supplies row (l % 32) of A and column (l % 32) of B, 16 int8
// values each, for position group l / 32; the output tile puts C[8*(i/4) + 4*(l/32) + i%4]
// [l % 32] in accumulator i of lane l. A and B use the same (lane group, byte) -> position
// map, so any assignment of positions to bytes that is the same for both gives the exact
// dot product.
//
// Weights ("pkm" layout): for physical 32-column group cg and 32-position block kb, the 64
// words of lanes l = 32*kq + ol are contiguous: pkm[(cg * nK32 + kb) * 64 + l] holds the 16
// codes of column 32*cg + ol at positions 32*kb + 16*kq + [0, 16) -- one word of the slab
// layout with -1 stored as 10 instead of 11 -- so a wave reads 256 contiguous bytes per
// fragment and expands each word to its 16-byte B operand with four v_perm_b32 (expand_w). For the MLP gate matrix the groups are interleaved
// (gate group c at cg = 2c, its up partner N/2 + 32c at cg = 2c + 1) so that one wave holds
// both halves of swiglu(gate, up) (hgrn_model.cpp:171-185) in registers.
//
// Activations: the prologues store the int8 planes already in fragment order (32 rows x 32
// positions per contiguous 1 KB, lanes as the matrix cores take them), so an A transfer is
// one linear 1 KB read.
//
// Block: WM x WN waves (2 x 4 for long row ranges and wide matrices: 128 x 256 tiles, so
// the activations are re-read once per 256 columns), each wave a 64 x 64 tile (2 x 2
// fragments).
// The operands of each 64-position stage move from global memory straight into a ring of
// LDS slots (buffer loads into LDS, up to 6 slots, 5 stages ahead), each wave moving its
// share of every stage (16 bytes or one word per lane, in the matrix cores' lane order);
// one barrier per stage publishes a slot to the block. Every fragment read is one linear
// 1 KB (A) or 256 B (B) LDS access. (Against staging the same loads through registers two
// stages ahead, this measured 10% faster on the long-prefill shapes; most of the remaining
// gap to the matrix-core peak is the stage barriers' LDS-read bubble, the output stores
// after the loop, and whole-chip rounds of tiles.)
// Split-K: when a GEMM has too few tiles to occupy the chip (a few dozen rows, or narrow
// matrices), blockIdx.y selects a contiguous range of stages; each block stores its exact
// int32 partial tile, and k_splitk_epi adds the partials in split order and applies the
// epilogue (integer sums: the order does not change the result).
//
// K-groups (KW > 1): the split can also live inside one block. Its waves form KW groups of
// WM x WN waves that take equal runs of the stages of the same tile, each through its own
// LDS slots; group 0 adds the others' int32 tiles from LDS and runs the epilogue. That
// gives more waves per SIMD (or no partials through memory) with the same tile traffic.
#include <cstdlib>
#include <type_traits>

#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__global__ void k_pack_mfma(const uint32_t* __restrict__ pk, Geom g, int pair, uint32_t* __restrict__ pkm) {
  const int nK32 = g.Lc / 4;
  const int ng32 = (g.N + 31) / 32;
  const size_t total = static_cast<size_t>(ng32) * nK32 * 64;
  for (size_t w = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; w < total;
       w += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int l = static_cast<int>(w & 63);
    const size_t t = w >> 6;
    const int kb = static_cast<int>(t % nK32);
    const int cg = static_cast<int>(t / nK32);
    const int lcg = pair ? ((cg & 1) ? ng32 / 2 + (cg >> 1) : (cg >> 1)) : cg;
    const int col = lcg * 32 + (l & 31), kq = l >> 5;
    const int p0 = kb * 32 + kq * 16;
    const int j = p0 / g.Lc, m = (p0 % g.Lc) >> 4;
    // -1 (11) becomes 10, so that expand_w selects every byte with a single permute
    const uint32_t x = col < g.N ? pk[(static_cast<size_t>((col >> 4) * g.Wc + m) * 16 + (col & 15)) * 8 + j] : 0u;
    pkm[w] = x ^ ((x >> 1) & 0x55555555u);
  }
}

// A matrix-core slab word (codes 00 = 0, 01 = +1, 10 = -1; code t of the word at bit
// 8 (t % 4) + 2 (t / 4)) as the 16 int8 weights of one operand, four per dword. Each dword is
// one AND and one v_perm_b32 over the byte array {S0, S1}: with the codes at bits 0-1 of each
// selector byte (values 0, 1, 2) the selector picks byte 0, 1 or 2 of S1 = {0x00, 0x01, 0xFF};
// at bits 2-3 (values 0, 4, 8) it picks byte 0 of S1 (0x00), byte 0 of S0 (0x01), or with 8
// the sign of S1's byte 1 (0x80) replicated (0xFF). The upper two dwords share one shift.
__device__ __forceinline__ v4i expand_w(uint32_t w) {
  const uint32_t h = w >> 4;
  v4i b;
  b[0] = static_cast<int>(__builtin_amdgcn_perm(0u, 0x00FF0100u, w & 0x03030303u));
  b[1] = static_cast<int>(__builtin_amdgcn_perm(0x01u, 0x00008000u, w & 0x0C0C0C0Cu));
  b[2] = static_cast<int>(__builtin_amdgcn_perm(0u, 0x00FF0100u, h & 0x03030303u));
  b[3] = static_cast<int>(__builtin_amdgcn_perm(0x01u, 0x00008000u, h & 0x0C0C0C0Cu));
  return b;
}

// s_waitcnt with only the vector-memory counter constrained (vmcnt <= N).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}
// s_waitcnt lgkmcnt(0): this wave's LDS reads and writes have returned.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

template <int V>
using ic = std::integral_constant<int, V>;

typedef __attribute__((address_space(3))) void* lds_ptr;

// Buffer loads straight into LDS (buffer_load ... lds) of 16 (or 4) bytes per lane from
// byte offset voff (per lane) + soff (uniform) of a raw buffer (base, num_records bytes;
// offsets past it read zeros): lane l's bytes land at LDS address m0 + 16 l (4 l).
// Written as inline assembly so that the compiler, which cannot tell which LDS bytes such a
// transfer writes, adds no waits of its own: it made every LDS read after a transfer wait
// for all transfers in flight (or, for global_load_lds, for all earlier LDS reads), which
// undid the ring. The kernel orders the transfers itself: it waits for a stage's transfers
// (vmcnt) and passes a barrier before any wave reads that stage's slot, and a slot is
// refilled only after every wave has passed the barrier that follows its last reads. M0 is
// set by each of these statements (one wait state before the load reads it) and used by
// nothing else in the kernel.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 raw_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return u32x4{static_cast<uint32_t>(b), static_cast<uint32_t>(b >> 32) & 0xFFFFu, bytes, 0x00020000u};
}
// the 32-bit LDS address of a pointer into a __shared__ array
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}
__device__ __forceinline__ void lds_dma16(u32x4 r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "s"(lds)
               : "memory");
}
__device__ __forceinline__ void lds_dma4(u32x4 r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "s"(lds)
               : "memory");
}

// Bytes of one stage of one K-group: the activation fragments [plane][frag][k-chunk] of
// 1 KB, then the weight fragments [group][k-chunk] of 256 B.
template <int MODE, int WM, int WN, int FM, int FN, int KQ>
__host__ __device__ constexpr int stage_bytes() {
  return ((MODE == kFixed) ? 2 : 1) * FM * WM * KQ * 1024 + FN * WN * KQ * 256;
}
// LDS bytes of a block beside its stage ring: the int8 row divisors and their reciprocals.
template <int MODE, int WM, int FM>
__host__ __device__ constexpr int row_scale_bytes() {
  return (MODE == kInt8 ? 2 : 1) * 32 * FM * WM * 4;
}
// Depth of the stage ring: as many slots (at most 6) as fit the LDS of the blocks a CU
// holds (two for blocks of at most four waves, else one), with the int8 row scales.
template <int MODE, int WM, int WN, int FM, int FN, int KQ, int KW>
__host__ __device__ constexpr int ring_depth() {
  constexpr int per_cu = 160 * 1024, blocks = (WM * WN * KW > 4) ? 1 : 2;
  constexpr int d = (per_cu / blocks - row_scale_bytes<MODE, WM, FM>() - 256) / (KW * stage_bytes<MODE, WM, WN, FM, FN, KQ>());
  return d > 6 ? 6 : d;
}

// Minimum waves per SIMD the compiler must fit (the second launch bound): 2 for blocks of
// up to four waves; 4 for the Int8Absmax 8-wave 128 x 256 tiles without a residual (at most
// 128 VGPRs, so two blocks share a CU: they measured 7% slower at 136 VGPRs, one block per
// CU); else 1.
template <int MODE, int EPI, int WM, int WN, int KW>
constexpr int mfma_min_waves() {
  if (MODE == kInt8 && EPI != kEpiAdd && WM * WN == 8 && KW == 1) return 4;
  return (WM * WN * KW > 4) ? 1 : 2;
}

template <int MODE, int EPI, int WM, int WN, int FM, int FN, int KQ, int KW>
__global__ __launch_bounds__(64 * WM * WN * KW, (mfma_min_waves<MODE, EPI, WM, WN, KW>())) void k_mfma(GemmArgs a, ActBuf act) {
  constexpr int P = (MODE == kFixed) ? 2 : 1;  // activation planes
  constexpr int NW = WM * WN;                   // waves per K-group (one tile)
  constexpr int BM = 32 * FM * WM;              // rows per block
  constexpr int BG = FN * WN;                   // physical 32-column groups per block
  constexpr int FR = FM * WM;                   // 32-row fragments per block
  constexpr int SA = P * FR * KQ * 1024;        // A bytes per stage: [plane][frag][k-chunk]
  constexpr int SS = SA + BG * KQ * 256;        // stage bytes (A, then B: [group][k-chunk])
  constexpr int DA = P * FR * KQ / NW;          // A transfers per wave per stage
  constexpr int DB = BG * KQ / NW;              // B transfers per wave per stage
  static_assert(DA * NW == P * FR * KQ && DB * NW == BG * KQ, "transfers must split evenly over the waves");
  static_assert(EPI != kEpiSwigluPair || FN % 2 == 0, "a swiglu pair needs both its column groups in one wave");
  static_assert(SS == stage_bytes<MODE, WM, WN, FM, FN, KQ>(), "stage layout");

  const int z = blockIdx.z;
  const ProjDev& W = a.p[z];
  const int N = W.g.N, Lc = act.Lc;
  // every argument the block reads, in one batch of scalar loads before the first branch
  // (a load placed after a branch waits for its own round trip)
  float* const outz = a.out[EPI == kEpiSwigluPair ? 0 : z];
  int32_t* const accz = a.acc[z];
  int32_t* const wsp = a.ws;
  const float* const addp = a.add;
  const int8_t* const tailp = W.tail;
  const int rawacc = a.raw_acc ? 1 : 0, swn = a.swiglu_n, ntail = W.g.ntail;
  const float invf = a.inv_fixed[z], scw = W.scale_w;
  const int8_t* const aq = act.q;
  const uint32_t* const pkm = W.pkm;
  const int32_t* const rsum = W.rowsum;
  const float* const asa = act.sa;
  const int32_t* const act_ct = act.ct;
  const int arows = act.rows, ana = act.na, ksp = gridDim.y;
  MMF_PIN("s"(outz), "s"(accz), "s"(wsp), "s"(addp), "s"(tailp), "s"(rawacc), "s"(swn), "s"(ntail), "s"(invf),
          "s"(scw), "s"(aq), "s"(pkm), "s"(rsum), "s"(asa), "s"(act_ct), "s"(arows), "s"(ana), "s"(ksp), "s"(Lc));
  const int ng32 = (N + 31) / 32;
  // XCD-aware tile order: blocks are dealt to the 8 XCDs round-robin by block index, so
  // block i runs on XCD i % 8; that XCD takes the i / 8-th tile of its own contiguous
  // share of the row-major tile list. Concurrent blocks of one XCD then walk the column
  // tiles of the same row tiles, and their activation rows stay in that XCD's L2.
  const int nct = (ng32 + BG - 1) / BG, nrt = (arows + BM - 1) / BM;
  const int ntile = nct * nrt, share = (ntile + 7) / 8;
  const int tile = (blockIdx.x & 7) * share + (blockIdx.x >> 3);
  if (tile >= ntile) return;
  const int tid = threadIdx.x, lane = tid & 63;
  // K-groups: with KW > 1 the block's waves form KW groups of NW waves; group kg multiplies
  // the kg-th of KW equal runs of the block's stages through its own LDS slots, and the
  // groups' partial tiles are added in LDS before the epilogue (exact int32 sums)
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar stage offsets
  const int kg = (KW > 1) ? wid / NW : 0, wave = (KW > 1) ? wid % NW : wid;
  const int wm = wave / WN, wn = wave % WN;  // this wave: row fragments wm*FM.., groups wn*FN..
  const int row0 = (tile / nct) * BM;
  const int cgb = (tile % nct) * BG;
  const int am = (ana > 1) ? z : 0;
  // stage range of this block's split (all stages without split-K)
  const int nall = Lc / (4 * KQ), ks = blockIdx.y;
  // (nall * ksp < 2^31: 32-bit quotients; none without a split)
  const int st0 = ksp == 1 ? 0 : static_cast<int>(static_cast<unsigned>(nall * ks) / static_cast<unsigned>(ksp));
  const int nst = ksp == 1 ? nall
                           : static_cast<int>(static_cast<unsigned>(nall * (ks + 1)) / static_cast<unsigned>(ksp)) - st0;
  const int cnt = (nst + KW - 1) / KW;           // loop stages of every group
  const int gb = kg * cnt;                       // the group's first stage (from st0)
  const int ng = max(0, min(cnt, nst - gb));     // stages the group multiplies
  const int8_t* qbase = aq + 2 * static_cast<size_t>(am) * act.qplane();

  // per-lane sources of this wave's transfers (advanced by KQ fragments = KQ KB of the
  // fragment-tiled activations / KQ x 256 B of weights per stage). Row groups past the last
  // 32-row group of the activations (a row tile that overhangs it) read that last group
  // again; their products are never stored. (Byte offsets from the matrix's planes and
  // from its weights: both below 2^31, which launch_gemm checks.)
  const u32x4 arsrc = raw_rsrc(qbase, static_cast<uint32_t>(P * act.qplane()));
  const u32x4 brsrc = raw_rsrc(pkm, static_cast<uint32_t>(ng32 * (Lc / 4) * 256));
  uint32_t aoff[DA];
  const int lastg = act.rows32() / 32 - 1;
#pragma unroll
  for (int i = 0; i < DA; ++i) {
    const int f = wave * DA + i;  // = (plane * FR + frag) * KQ + k-chunk
    const int kh = f % KQ, pl = (f / KQ) / FR, rf = (f / KQ) % FR;
    int g = (row0 >> 5) + rf;
    g = g < lastg ? g : lastg;
    aoff[i] = static_cast<uint32_t>(pl * act.qplane() + (static_cast<size_t>(g) * (Lc / 4) + kh) * 1024 + lane * 16);
  }
  uint32_t boff[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) {
    const int f = wave * DB + i;  // = group * KQ + k-chunk
    int cg = cgb + f / KQ;
    cg = cg < ng32 ? cg : ng32 - 1;
    boff[i] = static_cast<uint32_t>(((static_cast<size_t>(cg) * (Lc / 4) + f % KQ) * 64 + lane) * 4);
  }

  // epilogue operands that do not depend on the accumulators, fetched before the main loop
  // so their latency hides behind it: per-row int8 scales (one per lane, to LDS after the
  // loop), per-column Q5.10 offsets (128 * rowsum). Every wave loads them, from clamped
  // (in-range) indices, and selects afterwards: a load inside a branch is waited for at
  // the branch's end, a memory round trip before the first transfer is issued.
  float sv = 0.0f;
  if constexpr (MODE == kInt8) {
    int row = row0 + (wave * 64 + lane) % BM;
    row = row < arows ? row : arows - 1;
    sv = asa[static_cast<size_t>(am) * arows + row];
  }
  const int Nout = (EPI == kEpiSwigluPair) ? N / 2 : N;
  const int ol = lane & 31;
  // column (in N) of each of the wave's groups; a swiglu pair's gate group is even and its
  // up partner follows it: gate column (cg/2)*32 + ol, up column Nout + the same
  int col[FN];
  int32_t csum[FN];
#pragma unroll
  for (int bj = 0; bj < FN; ++bj) {
    const int cg = cgb + wn * FN + bj;
    col[bj] = (EPI == kEpiSwigluPair) ? (cg >> 1) * 32 + ol + ((bj & 1) ? Nout : 0) : cg * 32 + ol;
    csum[bj] = 0;
    if constexpr (MODE == kFixed) {
      const int32_t rs = rsum[col[bj] < N ? col[bj] : N - 1];
      csum[bj] = (ksp == 1 && col[bj] < N) ? 128 * rs : 0;
    }
  }

  v16i acc[P][FM][FN];
#pragma unroll
  for (int pl = 0; pl < P; ++pl)
#pragma unroll
    for (int ai = 0; ai < FM; ++ai)
#pragma unroll
      for (int bj = 0; bj < FN; ++bj) acc[pl][ai][bj] = v16i{};

  // The stage ring: D slots, each its own LDS array (so that the compiler tells the slot
  // being filled from the slot being read and waits for nothing it need not), each holding
  // one stage of every K-group ([KW][SS] bytes). Every wave moves its share of a stage (DA
  // activation transfers of 1 KB, DB weight transfers of 256 B) from global memory straight
  // into a slot with buffer loads into LDS (lds_dma16/4: lane l's bytes land at the
  // transfer's base + l * size), D - 1 stages ahead: no registers and no LDS stores on the
  // way. Before stage st a wave waits until only the later stages' transfers are
  // outstanding, and one barrier per stage publishes slot st % D to the block and frees the
  // slot of stage st - 1 for stage st + D - 1. Nothing is issued past the loop's last stage
  // (the wait counts shrink over the last D - 2 stages): repeated loads there took a third
  // of the transfers of a 10-stage loop through the CU's memory pipeline, which bounds
  // these loops.
  constexpr int D = ring_depth<MODE, WM, WN, FM, FN, KQ, KW>();
  constexpr int NT = DA + DB;  // transfers per wave per stage
  static_assert(D >= 3 && D <= 6 && (D - 2) * NT < 64, "ring depth");
  constexpr int QB = KW * SS;
  // two-group split of the sum and the epilogue (see after the main loop): each group's four
  // waves send one fragment pair (FN x 4 KB) through two ring slots
  constexpr bool KW2S = KW == 2 && FM == 2 && NW == 4 && D >= 4 && 2 * FN * 4096 <= QB;
  __shared__ __align__(16) unsigned char q0[QB], q1[QB], q2[QB], q3[D > 3 ? QB : 16], q4[D > 4 ? QB : 16],
      q5[D > 5 ? QB : 16];
  __shared__ float srow[BM];  // Int8: the divisor of each row, scale_w * scale_a
  __shared__ float srcp[MODE == kInt8 ? BM : 1];  // Int8: its correctly rounded reciprocal
  auto slot = [&](auto sc) -> unsigned char* {
    constexpr int S = decltype(sc)::value;
    if constexpr (S == 0) return q0;
    else if constexpr (S == 1) return q1;
    else if constexpr (S == 2) return q2;
    else if constexpr (S == 3) return q3;
    else if constexpr (S == 4) return q4;
    else return q5;
  };
  auto issue = [&](auto sc, int s2) {
    unsigned char* sb = slot(sc) + kg * SS;
    const int sg = st0 + min(gb + s2, nst - 1);
#pragma unroll
    for (int i = 0; i < DA; ++i) lds_dma16(arsrc, aoff[i], sg * 1024 * KQ, lds_addr(sb + (wave * DA + i) * 1024));
#pragma unroll
    for (int i = 0; i < DB; ++i) lds_dma4(brsrc, boff[i], sg * 256 * KQ, lds_addr(sb + SA + (wave * DB + i) * 256));
  };
  auto stage = [&](auto sc, int st) {
    constexpr int S = decltype(sc)::value;
    // this wave's reads of the previous stage have returned and its transfers of stage st
    // have landed: only the transfers of the later stages already issued (up to D - 2 of
    // them; fewer in the last stages, which issue nothing past the run) may be outstanding
    wait_lds();
    const int ahead = min(D - 2, cnt - 1 - st);
    if (ahead >= D - 2) {
      wait_vm<(D - 2) * NT>();
    } else if (ahead == 0) {
      wait_vm<0>();
    } else if (ahead == 1) {
      wait_vm<NT>();
    } else if (ahead == 2) {
      wait_vm<2 * NT>();
    } else {
      wait_vm<3 * NT>();
    }
    // one barrier per stage where a K-group's slots are shared by several waves; a one-wave
    // group owns its slots (the waits above order its own reads and transfers)
    if constexpr (NW > 1) {
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    if (st + D - 1 < cnt) issue(ic<(S + D - 1) % D>{}, st + D - 1);
    const unsigned char* sb = slot(sc) + kg * SS;
    uint32_t bw[KQ][FN];
    v4i av[KQ][P][FM];
#pragma unroll
    for (int kh = 0; kh < KQ; ++kh)
#pragma unroll
      for (int bj = 0; bj < FN; ++bj)
        bw[kh][bj] = *reinterpret_cast<const uint32_t*>(sb + SA + ((wn * FN + bj) * KQ + kh) * 256 + lane * 4);
#pragma unroll
    for (int kh = 0; kh < KQ; ++kh)
#pragma unroll
      for (int pl = 0; pl < P; ++pl)
#pragma unroll
        for (int ai = 0; ai < FM; ++ai)
          av[kh][pl][ai] = *reinterpret_cast<const v4i*>(sb + ((pl * FR + wm * FM + ai) * KQ + kh) * 1024 + lane * 16);
    // all LDS reads of the stage first, then the matrix-core work: each product waits only
    // for its own operands while the later reads are in flight. A group past its run (an
    // uneven split) multiplies zero weights instead of branching around the products: a
    // branch would make the first product wait for every read of the stage.
    __builtin_amdgcn_sched_barrier(0);
    const bool run = !(KW > 1 && st >= ng);
#pragma unroll
    for (int kh = 0; kh < KQ; ++kh) {
      v4i bop[FN];
#pragma unroll
      for (int bj = 0; bj < FN; ++bj) bop[bj] = expand_w(run ? bw[kh][bj] : 0u);
#pragma unroll
      for (int pl = 0; pl < P; ++pl)
#pragma unroll
        for (int ai = 0; ai < FM; ++ai)
#pragma unroll
          for (int bj = 0; bj < FN; ++bj)
            acc[pl][ai][bj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[kh][pl][ai], bop[bj], acc[pl][ai][bj], 0, 0, 0);
    }
  };
  if (cnt > 0) {
    issue(ic<0>{}, 0);
    if (cnt > 1) issue(ic<1>{}, 1);
    if constexpr (D > 3) if (cnt > 2) issue(ic<2>{}, 2);
    if constexpr (D > 4) if (cnt > 3) issue(ic<3>{}, 3);
    if constexpr (D > 5) if (cnt > 4) issue(ic<4>{}, 4);
    int st = 0;
    for (; st + D <= cnt; st += D) {  // straight-line runs of D stages: compile-time slots
      stage(ic<0>{}, st);
      stage(ic<1>{}, st + 1);
      stage(ic<2>{}, st + 2);
      if constexpr (D > 3) stage(ic<3>{}, st + 3);
      if constexpr (D > 4) stage(ic<4>{}, st + 4);
      if constexpr (D > 5) stage(ic<5>{}, st + 5);
    }
    if (st < cnt) stage(ic<0>{}, st);
    if (st + 1 < cnt) stage(ic<1>{}, st + 1);
    if constexpr (D > 3) if (st + 2 < cnt) stage(ic<2>{}, st + 2);
    if constexpr (D > 4) if (st + 3 < cnt) stage(ic<3>{}, st + 3);
    if constexpr (D > 5) if (st + 4 < cnt) stage(ic<4>{}, st + 4);
  }
  // every transfer (the repeats past the last stage included) has landed before the LDS is
  // reused or the block ends
  wait_lds();
  wait_vm<0>();
  // Int8: the rows' divisors and their reciprocals. The fast epilogue divides through the
  // reciprocal (div_by_recip: the same quotient) when the whole block allows it: |acc| <=
  // 2^21 (K < 16384) and every divisor and reciprocal normal.
  bool rcp_ok = false;
  if (MODE == kInt8) {
    bool ok = true;
    if (kg == 0 && wave * 64 + lane < BM) {  // one lane per row of the block (BM may be 32)
      const float dn = scw * sv, y = 1.0f / dn;
      srow[wave * 64 + lane] = dn;
      srcp[wave * 64 + lane] = y;
      ok = dn >= 0x1p-100f && dn <= 0x1p100f;
    }
    rcp_ok = __syncthreads_and(ok) && act.K < 16384;
  }
  if constexpr (KW > 1) {
    // K-group reduction: FixedQ510 folds its planes first (hi * 256 + lo into plane 1, as
    // the split-K partials do); then in each round groups 1..KW-1 store as many fragments as
    // a ring slot holds (all of them for the FixedQ510 few-row tiles), group r into slot
    // r - 1 (free once every wave has passed the barrier that precedes the stores), and after
    // one more barrier group 0 adds them: 16 bytes per lane per access
    if constexpr (MODE == kFixed) {
#pragma unroll
      for (int ai = 0; ai < FM; ++ai)
#pragma unroll
        for (int bj = 0; bj < FN; ++bj)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            acc[1][ai][bj][i] = acc[0][ai][bj][i] * 256 + acc[1][ai][bj][i];
            acc[0][ai][bj][i] = 0;
          }
    }
    // Eight one-wave groups on a whole in-range tile: the sums and the epilogue are shared.
    // Every group stores its fragments (GPS8 groups per ring slot); then group g < 4 FM adds
    // row quad g % 4 of row fragment g / 4 (both column groups) over all eight groups and
    // runs the epilogue for those rows -- up to eight waves instead of one reading and storing.
    constexpr int GR = FM * FN * 4096;  // bytes of one group's fragments
    constexpr int GPS8 = QB / GR;       // groups per ring slot
    if constexpr (KW == 8 && NW == 1 && FN == 2 && (FM == 1 || FM == 2) && GPS8 >= 2 &&
                  (8 + GPS8 - 1) / GPS8 <= (D < 4 ? D : 4)) {
      const bool whole = row0 + BM <= act.rows && (cgb + BG) * 32 <= N && !accz && !rawacc && ntail == 0 &&
                         (EPI != kEpiSwigluPair ||
                          static_cast<size_t>(row0 + BM) * Nout <= static_cast<size_t>(swn & ~7));
      if (whole) {
        auto grp = [&](int g) -> v4i* {  // [fragment][quad][lane] as int4, GR bytes per group
          const int sl = g / GPS8;
          return reinterpret_cast<v4i*>((sl == 0 ? q0 : (sl == 1 ? q1 : (sl == 2 ? q2 : q3))) + (g % GPS8) * GR);
        };
        __syncthreads();
        {
          v4i* my = grp(kg);
#pragma unroll
          for (int f = 0; f < FM * FN; ++f)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const v16i& v = acc[P - 1][f / FN][f % FN];
              my[(f * 4 + q) * 64 + lane] = v4i{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            }
        }
        __syncthreads();
        if (kg >= FM * 4) return;  // 32-row tiles: four row quads, four waves
        const int ai = kg >> 2, q = kg & 3;
        v4i tot[FN];
#pragma unroll
        for (int bj = 0; bj < FN; ++bj) tot[bj] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const v4i* src = grp(g);
#pragma unroll
          for (int bj = 0; bj < FN; ++bj) {
            const v4i t = src[((ai * FN + bj) * 4 + q) * 64 + lane];
            tot[bj] = tot[bj] + t;
          }
        }
        // rows rbase + e of this quad (fragment row 8 q + 4 (lane / 32) + e), columns col[bj]
        const int rb = row0 + ai * 32 + 4 * (lane >> 5) + 8 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rb + e;
          const size_t grow = static_cast<size_t>(r);
          float val[FN];
#pragma unroll
          for (int bj = 0; bj < FN; ++bj) {
            const int32_t sacc = tot[bj][e] + csum[bj];
            if constexpr (MODE == kFixed) {
              val[bj] = static_cast<float>(sacc) * invf;
            } else {
              const float den = srow[r - row0];
              val[bj] = rcp_ok ? div_by_recip(static_cast<float>(sacc), den, srcp[r - row0])
                               : static_cast<float>(sacc) / den;
            }
          }
          if constexpr (EPI == kEpiSwigluPair) {
            outz[grow * Nout + col[0]] = swiglu_of(val[0], val[1], false);
          } else {
#pragma unroll
            for (int bj = 0; bj < FN; ++bj) {
              const size_t o = grow * N + col[bj];
              outz[o] = (EPI == kEpiAdd) ? addp[o] + val[bj] : val[bj];
            }
          }
        }
        return;
      }
    }
    // Two K-groups of two row fragments each (the long-prefill 128 x 128 tiles): the groups
    // split the sum and the epilogue by row fragment. Group g keeps fragment g, sends its
    // fragment 1 - g to the same wave of the other group through LDS and adds the one it
    // receives (exact int32 sums: any order), then stores its own 32-row half of the tile.
    if constexpr (KW2S) {
      // (kept and sent fragments as compile-time indices: a run-time index into the
      // accumulator array would put it in scratch memory)
      auto exch = [&](auto keepc) {
        constexpr int KEEP = decltype(keepc)::value, SEND = 1 - KEEP;
        __syncthreads();
        {
          v4i* out = reinterpret_cast<v4i*>((KEEP == 0 ? (wave < 2 ? q0 : q1) : (wave < 2 ? q2 : q3)) +
                                            (wave & 1) * (FN * 4 * 64 * 16));
#pragma unroll
          for (int bj = 0; bj < FN; ++bj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const v16i& v = acc[P - 1][SEND][bj];
              out[(bj * 4 + q) * 64 + lane] = v4i{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            }
        }
        __syncthreads();
        {
          const v4i* in = reinterpret_cast<const v4i*>((KEEP == 1 ? (wave < 2 ? q0 : q1) : (wave < 2 ? q2 : q3)) +
                                                       (wave & 1) * (FN * 4 * 64 * 16));
#pragma unroll
          for (int bj = 0; bj < FN; ++bj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const v4i t = in[(bj * 4 + q) * 64 + lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[P - 1][KEEP][bj][4 * q + e] += t[e];
            }
        }
        if constexpr (KEEP == 1) {  // the kept fragment to slot 0: the epilogue runs on slot 0
#pragma unroll
          for (int bj = 0; bj < FN; ++bj) acc[P - 1][0][bj] = acc[P - 1][1][bj];
        }
      };
      if (kg == 0) exch(std::integral_constant<int, 0>{});
      else exch(std::integral_constant<int, 1>{});
    } else {
    // fragments per round: the most (up to all of them) for which every wave's fragments of
    // groups 1..KW-1 fit the first min(D, 4) ring slots, GPS groups sharing a slot
    constexpr int NS = D < 4 ? D : 4;
    constexpr int FB = [] {
      for (int fb = FM * FN; fb >= 1; --fb) {
        const int gps = QB / (NW * fb * 4096);
        if (gps >= 1 && (KW - 1 + gps - 1) / gps <= NS) return fb;
      }
      return 0;
    }();
    static_assert(FB >= 1, "the reduced groups fit the ring slots");
    constexpr int GB = NW * FB * 4096;  // bytes of one group's round
    constexpr int GPS = QB / GB;
    auto red_slot = [&](int r) -> v4i* {  // [wave][fragment of the round][quad][lane] as int4
      const int sl = (r - 1) / GPS, off = ((r - 1) % GPS) * GB;
      return reinterpret_cast<v4i*>((sl == 0 ? q0 : (sl == 1 ? q1 : (sl == 2 ? q2 : q3))) + off);
    };
#pragma unroll
    for (int f0 = 0; f0 < FM * FN; f0 += FB) {
      __syncthreads();
      if (kg != 0) {
        v4i* red = red_slot(kg);
#pragma unroll
        for (int f = f0; f < f0 + FB && f < FM * FN; ++f)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const v16i& v = acc[P - 1][f / FN][f % FN];
            red[((wave * FB + f - f0) * 4 + q) * 64 + lane] = v4i{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          }
      }
      __syncthreads();
      if (kg == 0) {
#pragma unroll
        for (int r = 1; r < KW; ++r) {
          const v4i* red = red_slot(r);
#pragma unroll
          for (int f = f0; f < f0 + FB && f < FM * FN; ++f)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const v4i t = red[((wave * FB + f - f0) * 4 + q) * 64 + lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[P - 1][f / FN][f % FN][4 * q + e] += t[e];
            }
        }
      }
    }
    if (kg != 0) return;
    }
  }

  // with the two-group split each group stores one row fragment, held in slot 0, whose rows
  // are shifted by its group index
  constexpr int FME = KW2S ? 1 : FM;
  const int ash = KW2S ? kg : 0;
  if (ksp > 1) {
    // split-K: exact partial sums of this stage range, logical column order
    int32_t* wp = wsp + (static_cast<size_t>(ks) * a.nmat + z) * act.rows * static_cast<size_t>(N);
    const int Nh = N / 2;
#pragma unroll
    for (int bj = 0; bj < FN; ++bj) {
      const int cg = cgb + wn * FN + bj;
      const int o = (EPI == kEpiSwigluPair) ? ((cg & 1) ? Nh : 0) + (cg >> 1) * 32 + ol : cg * 32 + ol;
      if (cg >= ng32 || o >= N) continue;
#pragma unroll
      for (int ai = 0; ai < FME; ++ai)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = row0 + (wm * FM + ai + ash) * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
          if (row >= act.rows) continue;
          wp[static_cast<size_t>(row) * N + o] =
              (MODE == kFixed) ? acc[0][ai][bj][i] * 256 + acc[P - 1][ai][bj][i] : acc[0][ai][bj][i];
        }
    }
    return;
  }

  // epilogue: exact integer totals, dequantisation, output stage. The residual rows of
  // all fragments are loaded in one batch before any store. Stored columns of this lane:
  // one per group (NB = FN), or one per swiglu pair (its gate column; NB = FN / 2).
  constexpr int NB = (EPI == kEpiSwigluPair) ? FN / 2 : FN;
  constexpr int GS = (EPI == kEpiSwigluPair) ? 2 : 1;  // groups per stored column
  bool cok[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) cok[b] = col[GS * b] < Nout;
  float addv[FM][16][NB];
  if (EPI == kEpiAdd) {
#pragma unroll
    for (int ai = 0; ai < FME; ++ai)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        int row = row0 + (wm * FM + ai + ash) * 32 + 4 * (lane >> 5) + 8 * (i >> 2) + (i & 3);
        row = row < act.rows ? row : act.rows - 1;
#pragma unroll
        for (int b = 0; b < NB; ++b) addv[ai][i][b] = cok[b] ? addp[static_cast<size_t>(row) * N + col[b]] : 0.0f;
      }
  }
  // Whole tile in range, no tail weights, no integer accumulator output, below the swiglu
  // tail rule: one straight store per output with no per-element tests (the general path
  // below measured several times slower per tile).
  const bool fast = row0 + BM <= act.rows && (cgb + BG) * 32 <= N && !accz && !rawacc && ntail == 0 &&
                    (EPI != kEpiSwigluPair || static_cast<size_t>(row0 + BM) * Nout <= static_cast<size_t>(swn & ~7));
  auto fast_epi = [&](auto use_rcp) {
#pragma unroll
    for (int ai = 0; ai < FME; ++ai) {
      const int rbase = row0 + (wm * FM + ai + ash) * 32 + 4 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = rbase + 8 * (i >> 2) + (i & 3);
        const size_t grow = static_cast<size_t>(r);
        const float den = (MODE == kInt8) ? srow[r - row0] : 1.0f;
        const float rcp = (MODE == kInt8 && decltype(use_rcp)::value) ? srcp[r - row0] : 1.0f;
        float val[FN];
#pragma unroll
        for (int bj = 0; bj < FN; ++bj) {
          const int32_t s = (MODE == kFixed) ? acc[0][ai][bj][i] * 256 + acc[P - 1][ai][bj][i] + csum[bj] : acc[0][ai][bj][i];
          if constexpr (MODE == kFixed) val[bj] = static_cast<float>(s) * invf;
          else if constexpr (decltype(use_rcp)::value) val[bj] = div_by_recip(static_cast<float>(s), den, rcp);
          else val[bj] = static_cast<float>(s) / den;
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if (EPI == kEpiSwigluPair)
            outz[grow * Nout + col[2 * b]] = swiglu_of(val[2 * b], val[2 * b + 1], false);
          else
            outz[grow * N + col[b]] = (EPI == kEpiAdd) ? addv[ai][i][b] + val[b] : val[b];
        }
      }
    }
  };
  if (fast) {
    if (MODE == kInt8 && rcp_ok) fast_epi(std::true_type{});
    else fast_epi(std::false_type{});
    return;
  }
#pragma unroll
  for (int ai = 0; ai < FME; ++ai) {
    const int rbase = row0 + (wm * FM + ai + ash) * 32 + 4 * (lane >> 5);
    float den[16];
    if (MODE == kInt8) {
#pragma unroll
      for (int i = 0; i < 16; ++i) den[i] = srow[rbase - row0 + 8 * (i >> 2) + (i & 3)];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = rbase + 8 * (i >> 2) + (i & 3);
      if (row >= act.rows) continue;
      const size_t grow = static_cast<size_t>(row);
      const int32_t* ct = act.ct + (static_cast<size_t>(am) * act.rows + row) * 8;
      int32_t tot[FN];
      float val[FN];
#pragma unroll
      for (int bj = 0; bj < FN; ++bj) {
        int32_t s = (MODE == kFixed) ? acc[0][ai][bj][i] * 256 + acc[P - 1][ai][bj][i] + csum[bj] : acc[0][ai][bj][i];
        if (ntail && col[bj] < N)
          for (int t = 0; t < ntail; ++t) s += static_cast<int32_t>(tailp[col[bj] * 8 + t]) * ct[t];
        tot[bj] = s;
        val[bj] = (MODE == kFixed) ? static_cast<float>(s) * invf : static_cast<float>(s) / den[i];
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (!cok[b]) continue;
        if (EPI == kEpiSwigluPair) {
          if (accz) {
            accz[grow * N + col[2 * b]] = tot[2 * b];
            accz[grow * N + col[2 * b + 1]] = tot[2 * b + 1];
          }
          if (rawacc) continue;
          const size_t e = grow * Nout + col[2 * b];
          outz[e] = swiglu_of(val[2 * b], val[2 * b + 1], static_cast<int64_t>(e) >= (swn & ~7));
        } else {
          const size_t e = grow * N + col[b];
          if (accz) accz[e] = tot[b];
          if (rawacc) continue;
          outz[e] = (EPI == kEpiAdd) ? addv[ai][i][b] + val[b] : val[b];
        }
      }
    }
  }
}

// Split-K epilogue: one thread per output element (per pair for swiglu), the partials of
// every split added in split order, then the same bias / tail / dequantisation / output
// stage as the single-pass epilogue.
template <int MODE, int EPI>
__global__ void k_splitk_epi(GemmArgs a, ActBuf act) {
  const int z = blockIdx.z;
  const ProjDev& W = a.p[z];
  const int N = W.g.N;
  const int Nout = (EPI == kEpiSwigluPair) ? N / 2 : N;
  const size_t n = static_cast<size_t>(act.rows) * Nout;
  const size_t plane = static_cast<size_t>(act.rows) * N;  // one split of one matrix
  const int am = (act.na > 1) ? z : 0;
  constexpr int NM = (EPI == kEpiSwigluPair) ? 2 : 1;
  float* const outz = a.out[EPI == kEpiSwigluPair ? 0 : z];
  int32_t* const accz = a.acc[z];
  const int32_t* const wsp = a.ws;
  const float* const addp = a.add;
  const int8_t* const tailp = W.tail;
  const int32_t* const rsum = W.rowsum;
  // complete accumulators (ext_acc) already hold the tail products and the Q5.10 bias
  const int bias = a.ext_acc ? 0 : 1;
  const int rawacc = a.raw_acc ? 1 : 0, swn = a.swiglu_n, ntail = bias ? W.g.ntail : 0, ksplit = a.ksplit,
            nmat = a.nmat;
  const float invf = a.inv_fixed[z], scw = W.scale_w;
  MMF_PIN("s"(outz), "s"(accz), "s"(wsp), "s"(addp), "s"(tailp), "s"(rsum), "s"(rawacc), "s"(swn), "s"(ntail),
          "s"(ksplit), "s"(nmat), "s"(invf), "s"(scw), "s"(bias));
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int row = static_cast<int>(e / Nout), o0 = static_cast<int>(e % Nout);
    const size_t ar = static_cast<size_t>(am) * act.rows + row;
    float val[NM];
    int32_t tot[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int o = o0 + (mi ? Nout : 0);
      // the partials of 8 splits at a time are all loaded before any is added: one memory
      // round trip per 8 splits instead of one per split
      int32_t s = 0;
      const int32_t* wo = wsp + static_cast<size_t>(z) * plane + static_cast<size_t>(row) * N + o;
      for (int k0 = 0; k0 < ksplit; k0 += 8) {
        int32_t pv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) pv[u] = (k0 + u < ksplit) ? wo[static_cast<size_t>(k0 + u) * nmat * plane] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) s += pv[u];
      }
      if (MODE == kFixed && bias) s += 128 * rsum[o];
      if (ntail) {
        const int32_t* ct = act.ct + ar * 8;
        int32_t tw[8], tc[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          tw[t] = (t < ntail) ? static_cast<int32_t>(tailp[o * 8 + t]) : 0;
          tc[t] = (t < ntail) ? ct[t] : 0;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) s += tw[t] * tc[t];
      }
      tot[mi] = s;
      val[mi] = (MODE == kFixed) ? static_cast<float>(s) * invf : static_cast<float>(s) / (scw * act.sa[ar]);
    }
    const size_t grow = static_cast<size_t>(row);
    if (accz) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) accz[grow * N + o0 + (mi ? Nout : 0)] = tot[mi];
    }
    if (rawacc) continue;
    if (EPI == kEpiSwigluPair) {
      outz[e] = swiglu_of(val[0], val[NM - 1], static_cast<int64_t>(e) >= (swn & ~7));
    } else if (EPI == kEpiAdd) {
      outz[e] = addp[e] + val[0];
    } else {
      outz[e] = val[0];
    }
  }
}

template <int WM, int WN, int FM = 2>
int tiles_of(const GemmArgs& a) {
  const int ng32 = (a.p[0].g.N + 31) / 32;
  return ((ng32 + 2 * WN - 1) / (2 * WN)) * ((a.rows + 32 * FM * WM - 1) / (32 * FM * WM));
}

// 32-position k-chunks per stage (one barrier per stage). 128-position stages measured
// slower for Int8Absmax (one block per CU instead of two).
constexpr int kStageKQ = 2;

// A tile of 64 TM rows and 64 TN columns: TM x TN waves of 64 x 64 (2 x 2 fragments) per
// K-group. (Waves of 32 x 128, one row fragment by four column groups, read 40% fewer
// operand bytes from LDS per product but measured 10-20% slower on every long-prefill
// shape: twice the weight expansion per product, for no fewer stalls.)
template <int MODE, int EPI, int TM, int TN, int KQ, int KW, int FM = 2>
bool mfma_launch(const GemmArgs& a, const ActBuf& act, dim3 grid, hipStream_t s) {
  constexpr int WM = TM, WN = TN, FN = 2;
  constexpr int bytes =
      ring_depth<MODE, WM, WN, FM, FN, KQ, KW>() * KW * stage_bytes<MODE, WM, WN, FM, FN, KQ>() + row_scale_bytes<MODE, WM, FM>();
  if (bytes > lds_limit()) return false;
  k_mfma<MODE, EPI, WM, WN, FM, FN, KQ, KW><<<grid, dim3(64 * WM * WN * KW), 0, s>>>(a, act);
  return true;
}

// Tile shape: 64 rows for short row ranges (batched decode), else 128; 256 columns when
// that still gives every CU a block (all blocks of all matrices), else 128. Then K is
// split in powers of two until there are 128 blocks (each split >= 4 stages). A split GEMM
// of 49-64 rows with K <= 6912 and enough tiles (at least kKGroupTiles 64 x 128 tiles, or
// at least 64 32 x 64 tiles, or at most 64 stages) runs instead on tiles of eight K-groups
// in one block (kw), whose partial tiles meet in LDS: no partials through memory and no
// split-K epilogue launch; 8-32 rows take 32 x 64 such tiles (K <= 4096, or K <= 6912
// with at least 32 tiles).
struct Plan {
  int wm, wn, ksplit, kw;
  int fm = 2;  // 32-row fragments per wave (1: 32-row tiles)
};
static bool kw8_rows32() {
  static const bool on = [] {
    const char* e = std::getenv("MMF_KW8_32");
    return !(e && e[0] == '0');
  }();
  return on;
}
constexpr int kKGroupTiles = 48;

Plan plan_of(const GemmArgs& a) {
  const int nz = (a.epi == kEpiSwigluPair) ? 1 : a.nmat;
  Plan p{a.rows <= 64 ? 1 : 2, 4, 1, 1};
  if (p.wm == 1 ? tiles_of<1, 4>(a) * nz < 256 : tiles_of<2, 4>(a) * nz < 256) p.wn = 2;
  // FixedQ510 (two int8 passes per tile) over 128-row tiles: 128 x 128 tiles throughout.
  // Finer tiles balance the CUs (the 1.3B i/f/g GEMM: 768 tiles, three per CU, instead of
  // 384, one or two per CU): i/f/g 1.57 -> 1.30 ms and gate/up 2.43 -> 2.31 ms per 2048-token
  // prefill. Int8Absmax gained nothing on i/f/g and lost 5% on gate/up.
  if (a.mode == kFixed && p.wm == 2) p.wn = 2;
  // Int8Absmax: 64 x 256 tiles where 128 x 256 tiles would give the 256 CUs between one and
  // two tiles each: the 1.3B i/f/g GEMM (384 tiles) 1.00 -> 0.90 ms per 2048-token prefill
  // as 768 tiles, 2048 x 5632 x 1024 (352 tiles) 26.5 -> 24.8 us. At 704 tiles (2048 x 11264
  // x 2048) the halving measured 8% slower.
  if (a.mode == kInt8 && p.wm == 2 && p.wn == 4) {
    const int t = tiles_of<2, 4>(a) * nz;
    if (t > 256 && t < 512) p.wm = 1;
  }
  const int tiles = (p.wm == 1 ? (p.wn == 4 ? tiles_of<1, 4>(a) : tiles_of<1, 2>(a))
                               : (p.wn == 4 ? tiles_of<2, 4>(a) : tiles_of<2, 2>(a))) * nz;
  // split K until there are 128 blocks (one per two CUs; more splits measured slower, the
  // partial traffic growing with the split count), keeping >= 4 stages per split
  const int nst = a.p[0].g.Lc / 8;
  while (tiles * p.ksplit < 128 && nst / (2 * p.ksplit) >= 4 && p.ksplit < 16) p.ksplit *= 2;
  const int t32 = tiles_of<1, 1, 1>(a) * nz;  // 32 x 64 tiles
  // 8-32 rows: 32 x 64 tiles of eight K-groups where K <= 4096 (16-row op calls: 2048 x
  // 11264 15.8 -> 11.6 us, 1024 x 1024 10.5 -> 9.6 us per call), or over 16 rows K <= 6912
  // with at least 32 tiles (the 1.3B down projection, K = 5632: 12.2 us per launch against
  // 9.4 us for the split plus 2.0 us for its epilogue launch, whose writes also delayed the
  // next launch by 2.4 us; at 16 rows the split stays faster, 15.5 against 17.2 us)
  if (kw8_rows32() && a.rows >= 8 && a.rows <= 32 && p.ksplit > 1 && nst >= 16 &&
      (nst <= 64 || (nst <= 216 && t32 >= 32 && a.rows > 16))) {
    p = Plan{1, 1, 1, 8, 1};
    return p;
  }
  if (p.wm == 1 && a.rows > 48 && p.ksplit > 1 && nst >= 16 && nst <= 216 &&
      (tiles >= kKGroupTiles || nst <= 64 || t32 >= 64)) {
    // (a 4-wave-wide tile never splits: it has >= 256 tiles) tiles of eight K-groups, one
    // wave each, 32-position stages: twice the blocks of 64 x 128 tiles with four K-groups
    // of two waves, each wave a quarter of the chain of stages (64 rows, FixedQ510: i/f/g
    // 2560 x 3 x 2560 18.1 -> 16.3 us, gate/up 2560 x 13824 20.1 -> 18.6 us per launch in a
    // step, before the shared epilogue below). 32 x 64 tiles where they still fit one block
    // per CU: twice the blocks, half the activation rows streamed through each CU (2.7B x 64
    // FixedQ510 step, per launch: i/f/g 11.0 -> 8.2 us, o 12.9 -> 9.8 us; the down
    // projection, K = 6912, 14.5 us against 10.7 us for the split plus 5.1 us for its
    // epilogue launch, whose writes also delayed the next launch by 3.5 us); else 64 x 64
    // (gate/up: 432 32 x 64 tiles would take two rounds, 18.0 against 11.8 us).
    p.kw = 8;
    p.wn = 1;
    p.ksplit = 1;
    if (t32 <= 256) p.fm = 1;
  }
  // 128 x 128 tiles at one block per CU (the 2048-column o/down GEMMs of a long prefill):
  // two K-groups per block give each SIMD two waves instead of one, with the same tile
  // and operand traffic
  if (p.wm == 2 && p.wn == 2 && p.ksplit == 1 && tiles <= 256 && nst >= 8) p.kw = 2;
  return p;
}

template <int MODE, int EPI, int WM, int WN, int KW, int KQ = kStageKQ, int FM = 2>
hipError_t mfma_inst(const GemmArgs& a, const ActBuf& act, int ksplit, hipStream_t s) {
  const int ntile = tiles_of<WM, WN, FM>(a);
  const int nz = EPI == kEpiSwigluPair ? 1 : a.nmat;
  dim3 grid(8 * ((ntile + 7) / 8), ksplit, nz);
  if (!mfma_launch<MODE, EPI, WM, WN, KQ, KW, FM>(a, act, grid, s)) return hipErrorInvalidConfiguration;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ksplit == 1) return e;
  GemmArgs b = a;
  b.ksplit = ksplit;
  const int Nout = EPI == kEpiSwigluPair ? a.p[0].g.N / 2 : a.p[0].g.N;
  const size_t n = static_cast<size_t>(a.rows) * Nout;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
  k_splitk_epi<MODE, EPI><<<dim3(blocks, 1, nz), 256, 0, s>>>(b, act);
  return hipGetLastError();
}

template <int MODE, int EPI>
hipError_t mfma_epi(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  const Plan p = plan_of(a);
  const int ks = a.ws ? p.ksplit : 1;
  if (p.kw == 8)
    return p.fm == 1 ? mfma_inst<MODE, EPI, 1, 1, 8, 1, 1>(a, act, ks, s) : mfma_inst<MODE, EPI, 1, 1, 8, 1>(a, act, ks, s);
  if (p.kw == 2) return mfma_inst<MODE, EPI, 2, 2, 2>(a, act, ks, s);
  if (p.wm == 1)
    return p.wn == 4 ? mfma_inst<MODE, EPI, 1, 4, 1>(a, act, ks, s) : mfma_inst<MODE, EPI, 1, 2, 1>(a, act, ks, s);
  return p.wn == 4 ? mfma_inst<MODE, EPI, 2, 4, 1>(a, act, ks, s) : mfma_inst<MODE, EPI, 2, 2, 1>(a, act, ks, s);
}

template <int MODE>
hipError_t mfma_mode(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  switch (a.epi) {
    case kEpiSwigluPair: return mfma_epi<MODE, kEpiSwigluPair>(a, act, s);
    case kEpiAdd: return mfma_epi<MODE, kEpiAdd>(a, act, s);
    default: return mfma_epi<MODE, kEpiStore>(a, act, s);
  }
}

}  // namespace

// The device's LDS limit per block (160 KB on gfx950).
int lds_limit() {
  static int v = [] {
    int dev = 0, lim = 65536;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      lim = 65536;
    return lim;
  }();
  return v;
}

size_t pkm_words(const Geom& g) { return static_cast<size_t>((g.N + 31) / 32) * 16 * g.Lc; }

bool pkm_pairable(const Geom& g) { return g.N % 64 == 0; }

hipError_t launch_pack_mfma(const uint32_t* pk, const Geom& g, bool pair, uint32_t* pkm, hipStream_t s) {
  if (pair && !pkm_pairable(g)) return hipErrorInvalidValue;
  const size_t total = pkm_words(g);
  const int blocks = static_cast<int>(std::min<size_t>((total + 255) / 256, 65536));
  k_pack_mfma<<<blocks, 256, 0, s>>>(pk, g, pair ? 1 : 0, pkm);
  return hipGetLastError();
}

size_t gemm_workspace_bytes(const GemmArgs& a) {
  if (a.mode == kFloat || mfma_min_rows() <= 0 || a.rows < mfma_min_rows()) return 0;
  const Plan p = plan_of(a);
  if (p.ksplit == 1) return 0;
  return static_cast<size_t>(p.ksplit) * a.nmat * a.rows * static_cast<size_t>(a.p[0].g.N) * sizeof(int32_t);
}
hipError_t launch_gemm_mfma(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  return a.mode == kFixed ? mfma_mode<kFixed>(a, act, s) : mfma_mode<kInt8>(a, act, s);
}

template <int MODE, int EPI>
static hipError_t acc_epi_inst(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  GemmArgs b = a;
  b.ksplit = 1;
  b.ext_acc = true;
  const int Nout = EPI == kEpiSwigluPair ? a.p[0].g.N / 2 : a.p[0].g.N;
  const size_t n = static_cast<size_t>(a.rows) * Nout;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
  k_splitk_epi<MODE, EPI><<<dim3(blocks, 1, EPI == kEpiSwigluPair ? 1 : a.nmat), 256, 0, s>>>(b, act);
  return hipGetLastError();
}

template <int MODE>
static hipError_t acc_epi_mode(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  switch (a.epi) {
    case kEpiSwigluPair: return acc_epi_inst<MODE, kEpiSwigluPair>(a, act, s);
    case kEpiAdd: return acc_epi_inst<MODE, kEpiAdd>(a, act, s);
    default: return acc_epi_inst<MODE, kEpiStore>(a, act, s);
  }
}

hipError_t launch_acc_epilogue(const GemmArgs& a, const ActBuf& act, hipStream_t s) {
  if (a.mode == kFloat || !a.ws || a.rows <= 0) return hipErrorInvalidValue;
  return a.mode == kFixed ? acc_epi_mode<kFixed>(a, act, s) : acc_epi_mode<kInt8>(a, act, s);
}

}  // namespace mmf
