// weight.hpp -- the object behind an opaque ullm_linear_weight_t handle.
#pragma once

#include <stdint.h>

#include "layout.hpp"

struct ullm_linear_weight_t {
  uint32_t encoding = 0;
  int device = 0;
  uint64_t n = 0, k = 0;
  uint64_t gate = 0;  // F of a gated-pair weight (N = 2F), 0 for a plain one
  ullm::Fp8Layout fp8{};
  ullm::Aq4Layout aq4{};
  void *tiles = nullptr;  // FP8: u8 wave tiles; AQ4: u32 wave tiles
  void *aux = nullptr;    // FP8: f32 scales [n16]; AQ4: u32 scale|zero words
  uint64_t tile_bytes = 0, aux_bytes = 0;
};
