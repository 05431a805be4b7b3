// Host interface of the MFMA phases over the row layout (rows.hip).
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace latent {
namespace rows {

// Everything the three phase kernels read: the six factors (INT8 word offsets
// set), the grouping of the general path's prep kernel, x as fp16 rows with a
// power-of-two exponent per token, and the zeroed fp32 accumulators.
struct Params {
  Factor fac[6];
  const int32_t* ranks;  // [E][3] per-expert ranks of gate, up, down (NULL: max_rank)
  const int* meta;       // [0] active experts
  const int* act_expert;
  const int* act_start;
  const int* act_count;
  const int* pair_tok;
  const int* pair_slot;
  const float* pair_w;
  const _Float16* xh;  // [T][d] x * 2^xexp
  const int* xexp;     // [T]
  float* gu;           // [P][2R] gate and up latents (accumulated)
  float* dl;           // [P][R] down latents (accumulated)
  float* out;
  int T, d, ff, K, R, wbd, out_mode;
  int a_max;     // upper bound of the active experts (grid)
  int na_split;  // phase A: K ranges per factor
  int n_a, n_bc, n_d;  // items per active expert
};

// The row-layout shapes the kernels take (d, ff multiples of 32, max_rank at
// most 512, x 16-byte aligned for the fp16 conversion).
bool supported(const latent_moe_args& a);
// Sets the work split (na_split, n_a, n_bc, n_d) of p from its shape.
void plan(Params& p);
int launch(const Params& p, bool int8, hipStream_t s);

}  // namespace rows
}  // namespace latent
