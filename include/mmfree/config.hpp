// mmfree/config.hpp -- HGRN-Bit model configuration, read from the blob header.
// Same fields and defaults as the reference engine's Config (cpp/include/mmfree/config.hpp:8-21).
#pragma once

#include <cstddef>

namespace mmfree {

struct Config {
  std::size_t vocab_size = 32000;
  std::size_t hidden_size = 1024;
  std::size_t num_hidden_layers = 24;
  std::size_t num_heads = 1;           // parsed, unused (the recurrence is elementwise)
  std::size_t expand_ratio = 1;        // parsed, unused
  std::size_t intermediate_size = 2816;  // gate_proj out = 2 * this; down_proj in = this
  bool use_lower_bound = true;
  bool use_short_conv = false;         // parsed, unused
  float rms_norm_eps = 1e-6f;

  std::size_t input_dim() const { return hidden_size * expand_ratio; }
  std::size_t head_dim() const { return input_dim() / num_heads; }
};

}  // namespace mmfree
