// mmf_peaks.hip -- device calibration for the rooflines. Each kernel does one kind of work
// and nothing else, so its rate is the sustained ceiling of that resource on this device:
//   - HBM read: a 2 GiB buffer (far beyond the 256 MB Infinity Cache) read once per pass,
//     nontemporal, in contiguous per-block chunks;
//   - Infinity Cache (MALL) read: a 128 MiB buffer (beyond the 8 x 4 MB of L2, within the
//     MALL) read repeatedly;
//   - int8 matrix cores: independent v_mfma_i32_32x32x32_i8 on register operands;
//   - fp32 vector FMA: independent v_fma_f32 chains (non-packed, as every kernel here is
//     built without packed fp32).
// The published figures the rooflines are priced against (8 TB/s, 5.0 POP/s int8 dense) are
// reported beside these measured ones; neither replaces the other.
#include "mmf_device.hpp"
#include "mmf_internal.hpp"

namespace mmf {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Reads of n4 float4 elements, `passes` times: each pass a block reads one contiguous chunk
// (n4 / gridDim.x elements, a multiple of 2048), eight 16-byte loads in flight per thread;
// NT marks them nontemporal (streamed past the caches: the HBM pass). Each thread's sum is
// stored so the loads cannot be dropped.
template <bool NT>
__global__ __launch_bounds__(256) void k_peak_read(const float4* __restrict__ p, size_t n4, int passes,
                                                   float* __restrict__ sink) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  constexpr int U = 8;
  float acc = 0.0f;
  const size_t per = n4 / gridDim.x;
  for (int r = 0; r < passes; ++r) {
    // pass r reads the chunk gridDim.x / 8 blocks further on (the same XCD under round-robin
    // dispatch, so a chunk is re-read only after the XCD's L2 has seen the whole buffer's
    // eighth)
    const size_t c = (blockIdx.x + static_cast<size_t>(r) * (gridDim.x / 8)) % gridDim.x;
    const f4v* q = reinterpret_cast<const f4v*>(p) + c * per;
    for (size_t i = threadIdx.x; i < per; i += 256 * U) {
      f4v v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(q + i + u * 256) : q[i + u * 256];
#pragma unroll
      for (int u = 0; u < U; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
  }
  sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// Four independent accumulators per wave, so consecutive MFMAs never wait on each other.
__global__ __launch_bounds__(256) void k_peak_mfma(int iters, int* __restrict__ sink) {
  const int t = static_cast<int>(threadIdx.x);
  const v4i a = {t, t + 1, t + 2, t + 3}, b = {3 * t, 5, 7 - t, 11};
  v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) s += c0[k] ^ c1[k] ^ c2[k] ^ c3[k];
  sink[blockIdx.x * blockDim.x + t] = s;
}

// Eight independent fp32 FMA chains per thread.
__global__ __launch_bounds__(256) void k_peak_fma(int iters, float x, float* __restrict__ sink) {
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = static_cast<float>(threadIdx.x + k);
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = __builtin_fmaf(a[k], x, 0.5f);
  }
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += a[k];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Milliseconds of the fastest of `reps` timed runs of f (after two untimed runs).
template <class F>
float best_ms(hipStream_t s, int reps, F f) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1.0f;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return -1.0f;
  }
  float best = -1.0f;
  f();
  f();
  for (int r = 0; r < reps; ++r) {
    if (hipEventRecord(e0, s) != hipSuccess) break;
    f();
    if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) break;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) break;
    if (best < 0.0f || ms < best) best = ms;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return best;
}

}  // namespace

hipError_t measure_peaks(int cus, hipStream_t s, double out[4]) {
  constexpr size_t kHbm = size_t(2) << 30, kMall = size_t(128) << 20;
  constexpr int kMallPasses = 8;
  // 4096 blocks: chunks of 32768 (HBM) and 2048 (MALL) float4, whole multiples of a block's
  // 2048-element step
  constexpr int blocks = 4096;
  static_assert((kHbm / 16) % (blocks * 2048) == 0 && (kMall / 16) % (blocks * 2048) == 0, "whole steps");
  void* buf = nullptr;
  float* sink = nullptr;
  hipError_t e = hipMalloc(&buf, kHbm);
  if (e != hipSuccess) return e;
  e = hipMalloc(&sink, static_cast<size_t>(blocks) * 256 * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(buf);
    return e;
  }
  e = hipMemsetAsync(buf, 0, kHbm, s);
  const float4* p = static_cast<const float4*>(buf);
  if (e == hipSuccess) {
    const float ms = best_ms(s, 10, [&] { k_peak_read<true><<<blocks, 256, 0, s>>>(p, kHbm / 16, 1, sink); });
    out[0] = ms > 0.0f ? kHbm / (ms * 1e-3) / 1e9 : 0.0;
    const float mm = best_ms(s, 5, [&] { k_peak_read<false><<<blocks, 256, 0, s>>>(p, kMall / 16, kMallPasses, sink); });
    out[1] = mm > 0.0f ? static_cast<double>(kMall) * kMallPasses / (mm * 1e-3) / 1e9 : 0.0;
    constexpr int kIters = 4096;
    const int mb = 2 * (cus > 0 ? cus : 256);  // two 4-wave blocks per CU: two waves per SIMD
    const float mf = best_ms(s, 3, [&] {
      k_peak_mfma<<<mb, 256, 0, s>>>(kIters, reinterpret_cast<int*>(sink));
    });
    out[2] = mf > 0.0f ? static_cast<double>(mb) * 4 * kIters * 4 * 65536.0 / (mf * 1e-3) / 1e12 : 0.0;
    const int fb = 8 * (cus > 0 ? cus : 256);
    const float ff = best_ms(s, 3, [&] { k_peak_fma<<<fb, 256, 0, s>>>(kIters, 0.999f, sink); });
    out[3] = ff > 0.0f ? static_cast<double>(fb) * 256 * kIters * 8 * 2.0 / (ff * 1e-3) / 1e12 : 0.0;
    e = hipGetLastError();
  }
  const hipError_t e2 = hipStreamSynchronize(s);
  (void)hipFree(sink);
  (void)hipFree(buf);
  return e != hipSuccess ? e : e2;
}

}  // namespace mmf
