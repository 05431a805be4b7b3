// Host interface of the fused (persistent, one-launch) decode path.
#pragma once

#include <stddef.h>

#include <hip/hip_runtime.h>

#include "../../include/latent_ffn.h"

namespace latent {

struct Factor;

namespace fused {

// Workspace bytes at the start of every workspace that the fused path keeps
// zero between calls (queue tickets, per-expert counters, combine counters).
constexpr size_t kReserved = 256 * 1024;
// Byte offset, inside that region, of the int error word a timed-out bounded
// wait sets (read and cleared by latent_moe_check).
constexpr size_t kErrorOffset = 36;

struct Plan {
  int ra, nca, cb, ncb, cd, ncd;
  size_t off_sync, off_ycnt;  // inside the reserved region
  size_t off_partA, off_glat, off_partB, off_dlat, off_ybuf, scratch_bytes;  // after it
};

bool supported(const latent_moe_args& a);
bool make_plan(const latent_moe_args& a, Plan& plan);
// fac: the six factors (make_factor) with their INT8 word offsets set.
int forward(const latent_moe_args& a, hipStream_t s, char* workspace, const Plan& plan, const Factor (&fac)[6]);

}  // namespace fused
}  // namespace latent
