// mmfree/kernels.hpp -- the BitLinear / HGRN operators, run on the MI355X.
//
// Same free functions, argument order and meaning as the reference's CPU kernels
// (cpp/include/mmfree/kernels.hpp:29-68); pointers are host memory, as there. Each call
// copies its operands to the process's default device context (device MMFREE_DEVICE or 0),
// runs the gfx950 kernel and copies the result back; results are bit-identical to the
// reference engine's. For resident weights and device pointers use mmfree_hip.h or Model.
// Errors (no device, bad arguments) are thrown as std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>

namespace mmfree {

struct TernaryBackend;  // mmfree/ternary_backend.hpp

// Activation handling of the BitLinear input (post-RMSNorm y):
//   Float      fp32 activations (kernels.hpp:21-26 of the reference)
//   FixedQ510  static Q(15-f).f int16 codes, int32 accumulation, acc / (2^f * scale_w)
//   Int8Absmax per-row int8 codes, scale_a = 127 / max|y|, acc / (scale_w * scale_a)
//              (tools/reference.py:131-135,180-184; an addition to the reference's two)
enum class ActQuant { Float, FixedQ510, Int8Absmax };

void rmsnorm(float* y, const float* x, const float* weight, std::size_t rows, std::size_t cols,
             float eps);

void bitlinear(float* out, const float* x, const float* norm_weight, const int8_t* wq, float scale_w,
               std::size_t rows, std::size_t in_dim, std::size_t out_dim, float eps,
               float* norm_out = nullptr, ActQuant aq = ActQuant::Float, int frac_bits = 10,
               TernaryBackend* be = nullptr, int proj_id = -1);

void bitlinear_cluster(float* const* outs, const float* x, const float* const* norm_weights,
                       const int8_t* const* wqs, const float* scale_w, int k, std::size_t rows,
                       std::size_t in_dim, std::size_t out_dim, float eps, int frac_bits,
                       TernaryBackend* be, const int* proj_ids);

void swiglu(float* out, const float* a, const float* b, std::size_t n);

void hgrn_scan(float* out, const float* i, const float* f, std::size_t T, std::size_t D,
               float* state_io = nullptr);

void rmsnorm_swishgate(float* out, const float* g, const float* o, const float* weight,
                       std::size_t rows, std::size_t cols, float eps);

}  // namespace mmfree
