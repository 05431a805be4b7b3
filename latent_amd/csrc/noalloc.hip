// latent_moe_ffn_forward for callers that cannot allocate device memory.
//
// The scratch of every call comes from one library-owned device array per GPU
// (`scratch`, LATENT_NOALLOC_SCRATCH_BYTES), allocated by the HIP runtime with
// this file's code object and held until the process ends.  Host code never
// passes the array's name to a kernel: its device address is looked up once
// per device with hipGetSymbolAddress and that pointer is used everywhere.
// The first LATENT_NOALLOC_CONTROL_BYTES are the workspace control block,
// whose counters every call leaves zero; it is cleared once per device, by a
// fill kernel, before the first call uses it.  Its error word, set only by a
// timed-out bounded wait, is read (and after a timeout the whole control block
// re-zeroed) by latent_moe_check with a NULL workspace.  All calls on one GPU share the
// array, so calls that overlap on one GPU (several streams or host threads)
// race; calls issued in order on one stream do not.
#include "common.hpp"
#include "fused.hpp"

#include <mutex>

namespace latent {
namespace {

static_assert(LATENT_NOALLOC_CONTROL_BYTES == fused::kReserved, "control block size");

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[LATENT_NOALLOC_SCRATCH_BYTES];

__global__ void clear_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

std::mutex g_mutex;
void* g_ptr[kMaxDevices] = {};

}  // namespace

// The device address of `scratch` on the current device, set up on the first
// call there (symbol lookup, control block cleared on `s`).
int noalloc_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return LATENT_E_HIP;
  if (dev < 0 || dev >= kMaxDevices) return LATENT_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LATENT_E_HIP;
    const size_t n16 = LATENT_NOALLOC_CONTROL_BYTES / 16;
    (void)hipGetLastError();  // clear a stale error so the check below sees only this launch's
    hipLaunchKernelGGL(clear_kernel, dim3(static_cast<unsigned>((n16 + 255) / 256)), dim3(256), 0, s,
                       static_cast<uint4*>(p), n16);
    if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return LATENT_OK;
}

}  // namespace latent

extern "C" int latent_moe_ffn_forward_noalloc(const latent_moe_args* args, latent_stream_t stream) {
  if (!args) return LATENT_E_INVALID;
  latent_moe_args a = *args;
  a.workspace = nullptr;
  a.workspace_bytes = 0;
  size_t need = 0;
  const int st = latent_moe_workspace_size(&a, &need);
  if (st != LATENT_OK) return st;
  if (need > LATENT_NOALLOC_SCRATCH_BYTES) return LATENT_E_WORKSPACE;
  if (a.n_tokens == 0) return LATENT_OK;
  void* p = nullptr;
  const int sp = latent::noalloc_scratch(reinterpret_cast<hipStream_t>(stream), &p);
  if (sp != LATENT_OK) return sp;
  a.workspace = p;
  a.workspace_bytes = LATENT_NOALLOC_SCRATCH_BYTES;
  return latent_moe_ffn_forward(&a, stream);
}
