// NF4 / INT8 codec kernels: bit-exact unpack and byte-exact pack.
//
// unpack  : loader/latent_loader.py:133-145 (NF4), :161-170 (INT8) -- one fp32
//           multiply `level * f32(scale_f16)` per element.
// pack    : loader/latent_loader.py:111-130 (NF4) and :148-158 (INT8) applied per
//           row as loader/write_latent_gguf.py:227-257 does.
#include "common.hpp"

namespace latent {
namespace {

__constant__ float kLevels[16] = {
    nf4_level(0),  nf4_level(1),  nf4_level(2),  nf4_level(3),  nf4_level(4),  nf4_level(5),
    nf4_level(6),  nf4_level(7),  nf4_level(8),  nf4_level(9),  nf4_level(10), nf4_level(11),
    nf4_level(12), nf4_level(13), nf4_level(14), nf4_level(15),
};

template <bool kHasInt8>
__global__ void __launch_bounds__(256) unpack_kernel(Factor f, int64_t e, float* __restrict__ out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = kLevels[threadIdx.x];
  __syncthreads();
  const int64_t groups = f.cols / kGroup;
  const int64_t total = f.rows * groups;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / groups;
    const int g = static_cast<int>(i - row * groups);
    float v[kGroup];
    decode_group<kHasInt8>(f, e, row, g, lut, v);
    const float s = group_scale(f, e, row, g);
    float4* dst = reinterpret_cast<float4*>(out + row * f.cols + static_cast<int64_t>(g) * kGroup);
#pragma unroll
    for (int j = 0; j < kGroup / 4; ++j) {
      dst[j] = make_float4(__fmul_rn(v[4 * j], s), __fmul_rn(v[4 * j + 1], s), __fmul_rn(v[4 * j + 2], s),
                           __fmul_rn(v[4 * j + 3], s));
    }
  }
}

// One thread per 32-value group.  Scale = fp32 absmax (0 -> 1), normalise with a
// correctly rounded fp32 division, nearest level by |n - level| in fp32 with the
// first index winning ties (np.argmin), fp16 scale by round-to-nearest-even.
__global__ void __launch_bounds__(256) pack_nf4_kernel(const float* __restrict__ in, int64_t n_groups,
                                                       uint8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
  for (int64_t gi = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; gi < n_groups;
       gi += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float4* src = reinterpret_cast<const float4*>(in + gi * kGroup);
    float v[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup / 4; ++j) {
      const float4 q = src[j];
      v[4 * j] = q.x;
      v[4 * j + 1] = q.y;
      v[4 * j + 2] = q.z;
      v[4 * j + 3] = q.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float scale = (amax == 0.0f) ? 1.0f : amax;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const float n = __fdiv_rn(v[j], scale);
      int best = 0;
      float bestd = fabsf(__fsub_rn(n, kLevels[0]));
#pragma unroll
      for (int c = 1; c < 16; ++c) {
        const float dd = fabsf(__fsub_rn(n, kLevels[c]));
        if (dd < bestd) {
          bestd = dd;
          best = c;
        }
      }
      w[j >> 3] |= static_cast<uint32_t>(best) << (4 * (j & 7));
    }
    *reinterpret_cast<uint4*>(codes + gi * kGroupBytes) = make_uint4(w[0], w[1], w[2], w[3]);
    scales[gi] = __half_as_ushort(__float2half_rn(scale));
  }
}

__global__ void __launch_bounds__(256) pack_int8_kernel(const float* __restrict__ in, int64_t n_groups,
                                                        int8_t* __restrict__ q, uint16_t* __restrict__ scales) {
  for (int64_t gi = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; gi < n_groups;
       gi += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float* src = in + gi * kGroup;
    float amax = 0.0f;
    for (int j = 0; j < kGroup; ++j) amax = fmaxf(amax, fabsf(src[j]));
    float s = __fdiv_rn(amax, 127.0f);
    if (s == 0.0f) s = 1.0f;
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    for (int j = 0; j < kGroup; ++j) {
      float r = rintf(__fdiv_rn(src[j], s));
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const int8_t b = static_cast<int8_t>(static_cast<int>(r));
      w[j >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(b)) << (8 * (j & 3));
    }
    uint4* dst = reinterpret_cast<uint4*>(q + gi * kGroup);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    scales[gi] = __half_as_ushort(__float2half_rn(s));
  }
}

inline unsigned grid_for(int64_t items, int block) {
  const int64_t blocks = (items + block - 1) / block;
  return static_cast<unsigned>(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

Factor make_factor(const latent_factor& f) {
  Factor r;
  r.codes = f.codes;
  r.scales = f.scales;
  r.ext.bitmap = f.int8_bitmap;
  r.ext.row_offset = f.int8_row_offset;
  r.ext.data = f.int8_data;
  r.ext.word_offset = nullptr;
  r.rows = f.rows;
  r.cols = f.cols;
  return r;
}

int check_factor(const latent_factor& f) {
  if (!f.codes || !f.scales || f.rows <= 0 || f.cols <= 0 || (f.cols % kGroup) != 0) return LATENT_E_INVALID;
  const bool any = f.int8_bitmap || f.int8_row_offset || f.int8_data;
  const bool all = f.int8_bitmap && f.int8_row_offset && f.int8_data;
  if (any && !all) return LATENT_E_INVALID;
  if (!aligned16(f.codes) || (f.int8_data && !aligned16(f.int8_data))) return LATENT_E_INVALID;
  return LATENT_OK;
}

}  // namespace latent

using namespace latent;

extern "C" int latent_unpack(const latent_factor* factor, int64_t expert, float* out, latent_stream_t stream) {
  if (!factor || !out || expert < 0) return LATENT_E_INVALID;
  const int st = check_factor(*factor);
  if (st != LATENT_OK) return st;
  if (!aligned16(out)) return LATENT_E_INVALID;
  const Factor f = make_factor(*factor);
  const int64_t groups = f.rows * (f.cols / kGroup);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (f.ext.bitmap)
    hipLaunchKernelGGL(unpack_kernel<true>, dim3(grid_for(groups, 256)), dim3(256), 0, s, f, expert, out);
  else
    hipLaunchKernelGGL(unpack_kernel<false>, dim3(grid_for(groups, 256)), dim3(256), 0, s, f, expert, out);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

extern "C" int latent_pack_nf4(const float* values, int64_t rows, int64_t cols, uint8_t* codes, uint16_t* scales,
                               latent_stream_t stream) {
  if (!values || !codes || !scales || rows <= 0 || cols <= 0 || (cols % kGroup) != 0) return LATENT_E_INVALID;
  if (!aligned16(values) || !aligned16(codes)) return LATENT_E_INVALID;
  const int64_t n_groups = rows * (cols / kGroup);
  hipLaunchKernelGGL(pack_nf4_kernel, dim3(grid_for(n_groups, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), values, n_groups, codes, scales);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

extern "C" int latent_pack_int8(const float* values, int64_t n_groups, int8_t* q, uint16_t* scales,
                                latent_stream_t stream) {
  if (!values || !q || !scales || n_groups <= 0) return LATENT_E_INVALID;
  if (!aligned16(q)) return LATENT_E_INVALID;
  hipLaunchKernelGGL(pack_int8_kernel, dim3(grid_for(n_groups, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), values, n_groups, q, scales);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}
