// mmfree/ternary_backend.hpp -- the pluggable ternary-matmul seam of the BitLinear.
//
// Same virtual interface, default behaviour and contracts as the reference's seam
// (cpp/include/mmfree/ternary_backend.hpp:26-91), so a backend written for either engine
// plugs into both:
//   acc[o] = sum_{n<N} x[n] * wq[o*N + n] for o < M, wq int8 in {-1, 0, +1} ([M, N]);
//   x carries int16-range Q5.10 codes stored as int32; proj_id addresses resident weights
//   (-1 = use the wq pointer); matmul_batch_chunked reports every column exactly once;
//   matmul_seq's default is serial and bit-identical to k matmul_batch calls.
// The MI355X implementation is HipTernaryBackend (mmfree/hip_backend.hpp); CpuBackend
// below is the host-CPU one.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace mmfree {

struct TernaryBackend {
  // acc[0..M) for one activation vector x[0..N).
  virtual void matmul(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                      std::size_t N, std::size_t M) = 0;

  // Preferred number of activation vectors per call.
  virtual std::size_t batch_size() const { return 1; }

  // acc[i*M + m] for b vectors x[i*N + n]; default: one matmul per row.
  virtual void matmul_batch(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                            std::size_t N, std::size_t M, std::size_t b) {
    for (std::size_t i = 0; i < b; ++i) matmul(proj_id, x + i * N, acc + i * M, wq, N, M);
  }

  // As matmul_batch, reporting finished column ranges through on_cols(col0, ncols); every
  // column exactly once, in any order. Default: one call covering [0, M) at the end.
  virtual void matmul_batch_chunked(int proj_id, const std::int32_t* x, std::int32_t* acc,
                                    const std::int8_t* wq, std::size_t N, std::size_t M, std::size_t b,
                                    const std::function<void(std::size_t, std::size_t)>& on_cols) {
    matmul_batch(proj_id, x, acc, wq, N, M, b);
    if (on_cols) on_cols(0, M);
  }

  // k projections sharing (N, M, b): produce(j, xq) fills b*N codes, the backend fills
  // acc[b*M], consume(j, acc) takes it. Default: strictly serial.
  virtual void matmul_seq(const int* proj_ids, const std::int8_t* const* wqs, int k,
                          const std::function<void(int, std::int32_t*)>& produce,
                          const std::function<void(int, const std::int32_t*)>& consume, std::size_t N,
                          std::size_t M, std::size_t b) {
    std::vector<std::int32_t> xq(b * N), acc(b * M);
    for (int j = 0; j < k; ++j) {
      produce(j, xq.data());
      matmul_batch(proj_ids[j], xq.data(), acc.data(), wqs[j], N, M, b);
      consume(j, acc.data());
    }
  }

  virtual ~TernaryBackend() = default;
};

// The host-CPU backend (reference: ternary_backend.hpp:96-103): each output is the exact
// integer sum of its row, outputs spread over OpenMP threads when the program is built
// with OpenMP. Integer sums do not depend on their order, so the accumulators are the
// same for any thread count. Sums wrap at 32 bits like the reference's SIMD adds (real
// shapes never reach that: |code| <= 32768 and N <= 65536).
struct CpuBackend final : TernaryBackend {
  void matmul(int /*proj_id*/, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq, std::size_t N,
              std::size_t M) override {
    const std::ptrdiff_t outs = static_cast<std::ptrdiff_t>(M);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (std::ptrdiff_t o = 0; o < outs; ++o) {
      const std::int8_t* w = wq + static_cast<std::size_t>(o) * N;
      std::uint32_t s = 0;
      for (std::size_t n = 0; n < N; ++n)
        s += static_cast<std::uint32_t>(x[n]) * static_cast<std::uint32_t>(static_cast<std::int32_t>(w[n]));
      acc[o] = static_cast<std::int32_t>(s);
    }
  }
};

}  // namespace mmfree
