// grid_barrier.hip -- mmfree-grid-barrier: the latency of a grid-wide synchronisation inside
// one kernel on this GPU, against which a persistent (one launch per decode step) design of
// the batch-1 decode is weighed: such a kernel needs four grid-wide syncs per layer.
//
// Every block of a co-resident grid (checked with the occupancy API) runs `iters` rounds; in
// each round it publishes one value and then needs every other block's value of that round:
//   counter   one device-scope atomic counter; thread 0 of each block adds 1 and spins
//             (device-scope loads) until it reaches the round's target; values go through
//             device-scope stores and loads;
//   fence     the same with plain stores and loads and __threadfence() on both sides (L2
//             writeback and invalidate);
//   stamped   no counter: each block stores (value, round) as one 64-bit device-scope word in
//             one of two slot arrays (by round parity), and wave 0 of every block loads all
//             slots until each carries the round; the sync and the data load are one poll.
// Each round checks that the value read for the next block is that block's value of that
// round (visibility errors). Every wait is bounded (1 << 16 polls): a round that runs out
// sets a flag, every block leaves its loop, and the run reports timeouts instead of hanging.
// Measurement only; prints microseconds per round, the best of 4 runs.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

constexpr long kPollLimit = 1L << 16;

#define CK(x)                                                                                \
  do {                                                                                       \
    hipError_t e_ = (x);                                                                     \
    if (e_ != hipSuccess) {                                                                  \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
      std::exit(1);                                                                          \
    }                                                                                        \
  } while (0)

template <typename T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned value_of(int round, int block) {
  return static_cast<unsigned>(round) * 4096u + static_cast<unsigned>(block);
}

// FENCE = false: the counter protocol; true: the fence protocol.
template <bool FENCE>
__global__ void k_counter(unsigned* counter, unsigned* data, int iters, unsigned* errs, unsigned* timeouts) {
  const int nb = gridDim.x, b = blockIdx.x;
  __shared__ unsigned stop;
  unsigned bad = 0;
  for (int it = 0; it < iters; ++it) {
    unsigned* slot = data + (it & 1) * nb;
    if (threadIdx.x == 0) {
      if (FENCE) {
        slot[b] = value_of(it, b);
        __threadfence();
      } else {
        st_dev(&slot[b], value_of(it, b));
        __builtin_amdgcn_s_waitcnt(0);  // the store has completed before the arrival
      }
      __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned target = static_cast<unsigned>(it + 1) * nb;
      long polls = 0;
      unsigned st = 0;
      while (ld_dev(counter) < target) {
        if (++polls > kPollLimit) {
          atomicAdd(timeouts, 1u);
          break;
        }
      }
      if (ld_dev(timeouts) != 0) st = 1;
      if (FENCE) __threadfence();
      stop = st;
    }
    __syncthreads();
    if (stop) break;
    if (threadIdx.x == 0) {
      const int nbr = (b + 1) % nb;
      const unsigned got = FENCE ? slot[nbr] : ld_dev(&slot[nbr]);
      if (got != value_of(it, nbr)) ++bad;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && bad) atomicAdd(errs, bad);
}

__global__ void k_stamped(unsigned long long* slots, int iters, unsigned* errs, unsigned* timeouts) {
  const int nb = gridDim.x, b = blockIdx.x;
  __shared__ unsigned stop;
  __shared__ unsigned vals[1024];
  unsigned bad = 0;
  for (int it = 0; it < iters; ++it) {
    unsigned long long* slot = slots + (it & 1) * nb;
    const unsigned round = static_cast<unsigned>(it + 1);
    if (threadIdx.x == 0) st_dev(&slot[b], (static_cast<unsigned long long>(round) << 32) | value_of(it, b));
    if (threadIdx.x < 64) {
      long polls = 0;
      bool done = false;
      while (!done) {
        unsigned long long w[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {  // all of this lane's loads in flight at once
          const int e = threadIdx.x + 64 * u;
          w[u] = e < nb ? ld_dev(&slot[e]) : (static_cast<unsigned long long>(round) << 32);
        }
        bool mine = true;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int e = threadIdx.x + 64 * u;
          if (static_cast<unsigned>(w[u] >> 32) != round) mine = false;
          else if (e < nb) vals[e] = static_cast<unsigned>(w[u]);
        }
        done = __all(mine);
        if (!done && ++polls > kPollLimit) {
          if (threadIdx.x == 0) atomicAdd(timeouts, 1u);
          break;
        }
      }
      if (threadIdx.x == 0) stop = done ? 0u : 1u;
    }
    __syncthreads();
    if (stop) break;
    if (threadIdx.x == 0) {
      const int nbr = (b + 1) % nb;
      if (vals[nbr] != value_of(it, nbr)) ++bad;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && bad) atomicAdd(errs, bad);
}

template <class K, class Launch>
void measure(const char* name, K kernel, int blocks, int threads, int iters, int cus, Launch launch) {
  int occ = 0;
  CK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, 0));
  if (occ * cus < blocks) {
    std::printf("%-8s blocks %4d: not co-resident (%d per CU), skipped\n", name, blocks, occ);
    return;
  }
  unsigned *errs, *tmo;
  CK(hipMalloc(&errs, 4));
  CK(hipMalloc(&tmo, 4));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  float best = 1e30f;
  unsigned he = 0, ht = 0;
  for (int rep = 0; rep < 4; ++rep) {
    CK(hipMemset(errs, 0, 4));
    CK(hipMemset(tmo, 0, 4));
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    launch(errs, tmo);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    unsigned re = 0, rt = 0;
    CK(hipMemcpy(&re, errs, 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(&rt, tmo, 4, hipMemcpyDeviceToHost));
    he += re;
    ht += rt;
    if (ms < best) best = ms;
  }
  std::printf("%-8s blocks %4d threads %d: %7.3f us per round (best of 4 runs of %d rounds), visibility errors %u, "
              "timeouts %u\n",
              name, blocks, threads, 1000.0f * best / iters, iters, he, ht);
  CK(hipFree(errs));
  CK(hipFree(tmo));
  CK(hipEventDestroy(e0));
  CK(hipEventDestroy(e1));
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 1000;
  hipDeviceProp_t p;
  CK(hipGetDeviceProperties(&p, 0));
  std::printf("device %s, %d CUs\n", p.gcnArchName, p.multiProcessorCount);
  const int cus = p.multiProcessorCount, threads = 256;
  for (int blocks : {64, 128, 256, 512, 1024}) {
    unsigned *counter, *data;
    unsigned long long* slots;
    CK(hipMalloc(&counter, 4));
    CK(hipMalloc(&data, 2 * sizeof(unsigned) * blocks));
    CK(hipMalloc(&slots, 2 * sizeof(unsigned long long) * blocks));
    measure("counter", k_counter<false>, blocks, threads, iters, cus, [&](unsigned* e, unsigned* t) {
      CK(hipMemsetAsync(counter, 0, 4));
      k_counter<false><<<blocks, threads>>>(counter, data, iters, e, t);
    });
    measure("fence", k_counter<true>, blocks, threads, iters, cus, [&](unsigned* e, unsigned* t) {
      CK(hipMemsetAsync(counter, 0, 4));
      k_counter<true><<<blocks, threads>>>(counter, data, iters, e, t);
    });
    measure("stamped", k_stamped, blocks, threads, iters, cus, [&](unsigned* e, unsigned* t) {
      CK(hipMemsetAsync(slots, 0, 2 * sizeof(unsigned long long) * blocks));
      k_stamped<<<blocks, threads>>>(slots, iters, e, t);
    });
    CK(hipFree(counter));
    CK(hipFree(data));
    CK(hipFree(slots));
  }
  return 0;
}
