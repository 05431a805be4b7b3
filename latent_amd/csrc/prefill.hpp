// Host interface of the grouped-MFMA prefill path.
#pragma once

#include <stddef.h>

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace latent {
namespace prefill {

// Token->expert grouping written by the general path's prep kernel.
struct Grouping {
  int* meta;              // [0] active experts, [3] routed pairs; [2] M tiles (written by the tile kernel)
  const int* act_expert;  // [A]
  const int* act_start;   // [A]
  const int* act_count;   // [A]
  const int* pair_tok;    // [P]
  const int* pair_slot;   // [P]
  const float* pair_w;    // [P]
};

// Scratch of the prefill path inside the caller's workspace.
struct Layout {
  size_t tile_a, tile_r0, xexp, xh, gu, gu_exp, h, h_exp, dl, dl_exp, pos_of, y, y_exp, units, part, total;
};

// Routed pairs per active expert needed before the MFMA path pays off.
constexpr int kMinPairsPerExpert = 16;

bool supported(const latent_moe_args& a);
Layout layout_for(const latent_moe_args& a);
// Runs after the prep kernel on the same stream.
int forward(const latent_moe_args& a, const Factor* fac, const Grouping& g, char* scratch, hipStream_t s);

}  // namespace prefill
}  // namespace latent
