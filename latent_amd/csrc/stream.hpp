// Host interface of the streaming MFMA decode path (stream.hip).
#pragma once

#include "common.hpp"

namespace latent {
namespace stream {

constexpr int kMaxM = 16;  // routed pairs per work unit (the MFMA row count)
constexpr int64_t kMaxPairs = 4096;  // routed pairs the decode launches take

// The layer's shape and format can take the tile layout (latent_tiles_supported).
bool tiles_shape_ok(const latent_moe_args& a);

// Token grouping produced by the prep kernel (moe.hip), all device pointers.
// Pairs are grouped by expert; a work unit is a run of at most kMaxM
// consecutive grouped pairs of one expert.
struct Grouping {
  const int* meta;         // [3] routed pairs, [4] work units
  const int4* unit_info;   // [units] {expert, first grouped pair, pairs (1..kMaxM), 0}
  const int* unit_tok;     // [units][kMaxM] token of each row (0 past the unit's pairs)
  const int* pair_tok;     // [P] token, slot and router weight of each grouped pair
  const int* pair_slot;
  const float* pair_w;
  int* err;                // word a timed-out bounded wait sets
};

// Scratch of the path inside the caller's workspace.  xh / xexp (x as fp16
// rows * 2^xexp, one exponent per token) and pos_of (grouped pair of each
// routed slot) are written by the prep kernel.
struct Layout {
  size_t xh, xexp, partA, lath, lexp, partC, dlath, dexp, ybuf, pos_of, total;
};

// Batches of at most 32 routed pairs: the whole chain in one launch in which
// every workgroup issues all its tile loads first (lite_kernel), grouping and
// x conversion included, so the prep kernel is not launched.  Taken by default
// wherever a grid of at most four resident grids gives every workgroup tiles
// that fit its registers; LATENT_STREAM_LAUNCH=phases
// selects the per-phase launches instead.  Its counters live in the
// workspace control block at kLiteCtrlOffset (zero between calls).
constexpr size_t kLiteCtrlOffset = 192 * 1024;
constexpr size_t kLiteCtrlBytes = 64 * 1024;
bool lite_applies(const latent_moe_args& a);
// ctrl: the workspace's control block; scratch: the decode layout (layout_for).
int lite_forward(const latent_moe_args& a, char* ctrl, char* scratch, int* err, hipStream_t s);

// The call can take this path: the factors are in the tile layout
// (latent_tiles_repack) and the batch has at most kMaxPairs routed pairs.
bool supported(const latent_moe_args& a);
// Upper bound of work units: every active expert contributes ceil(n_e / kMaxM).
int64_t max_units(int64_t pairs, int64_t experts);
Layout layout_for(const latent_moe_args& a);
int forward(const latent_moe_args& a, const Grouping& g, char* scratch, hipStream_t s);

// Prefill-sized batches on the same tile layout: units of up to kBulkM
// grouped pairs of one expert, two workgroups per CU.
constexpr int kBulkM = 64;

// Inputs and intermediates of the bulk chain, all device pointers.
struct BulkArgs {
  const int* nunits;     // number of units
  const int4* units;     // [units] {expert, first grouped pair, pairs (1..kBulkM), 0}
  const int* pair_tok;   // [P] token, slot and router weight of each grouped pair
  const int* pair_slot;
  const float* pair_w;
  const _Float16* xh;    // [T][d] x as fp16 rows * 2^xexp
  const int* xexp;       // [T]
  _Float16* lat;         // [2][P][256] gate / up latents * 2^lexp
  int* lexp;             // [2][P]
  _Float16* hh;          // [P][ff] h * 2^hexp
  int* hexp;             // [P][ff / 32]: one exponent per 32 columns
  _Float16* dlat;        // [P][256] down latent * 2^dexp
  int* dexp;             // [P]
  _Float16* y;           // reduced output: [P][d] y * 2^yexp (the caller's combine sums w * y per token)
  int* yexp;             // [P][d / 64]: one exponent per 64 columns
  float* part;           // partial sums, bulk_part_bytes
};

// The layer has a tile layout this chain can stream (rank 256, pure NF4).
bool bulk_supported(const latent_moe_args& a);
size_t bulk_part_bytes(const latent_moe_args& a, int64_t max_units);
// Per-slot output: writes out's routed rows (times w when the weight goes
// before the down projection); reduced output: writes y and yexp.
int bulk_forward(const latent_moe_args& a, const BulkArgs& b, int64_t max_units, hipStream_t s);

}  // namespace stream
}  // namespace latent
