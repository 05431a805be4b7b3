// Shared device helpers for the gfx950 LATENT kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/latent_ffn.h"

namespace latent {

constexpr int kGroup = 32;     // elements per quantization group (one row segment)
constexpr int kGroupBytes = 16; // NF4 bytes of a group: one 128-bit load
constexpr int kWave = 64;

// The 16 NF4 levels, loader/latent_loader.py:28-48.  Identical float literals,
// so each rounds to the same binary32 value as np.float32(literal).
__host__ __device__ constexpr float nf4_level(int c) {
  constexpr float t[16] = {
      -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f,
      -0.09105004f, 0.0f,         0.0795803f,   0.1609302f,  0.2461123f,   0.33791524f,
      0.44070983f,  0.562617f,    0.72295684f,  1.0f,
  };
  return t[c & 15];
}

// Exponent e that brings a row maximum m into [2^14, 2^15) (0 for m == 0 or
// not finite): rows of tiny latents are stored as fp16 * 2^e so they keep
// fp16's full precision; powers of two scale exactly.
__device__ __forceinline__ int pow2_row_exponent(float m) {
  if (!(m > 0.f) || !(m < 3.0e38f)) return 0;
  const int ilog = static_cast<int>((__float_as_uint(m) >> 23) & 0xFFu) - 127;
  return min(120, max(-120, 14 - ilog));
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ float load_act(const void* p, int dtype, int64_t i) {
  if (dtype == LATENT_F32) return static_cast<const float*>(p)[i];
  uint16_t b = static_cast<const uint16_t*>(p)[i];
  if (dtype == LATENT_F16) return half_bits_to_float(b);
  return __uint_as_float(static_cast<uint32_t>(b) << 16);  // bf16
}

// Elements i .. i+7 of an activation array (i % 8 == 0, 16-byte aligned base).
__device__ __forceinline__ void load_act8(const void* p, int dtype, int64_t i, float v[8]) {
  if (dtype == LATENT_F32) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    return;
  }
  const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t lo = static_cast<uint16_t>(u[j] & 0xFFFFu), hi = static_cast<uint16_t>(u[j] >> 16);
    if (dtype == LATENT_F16) {
      v[2 * j] = half_bits_to_float(lo);
      v[2 * j + 1] = half_bits_to_float(hi);
    } else {  // bf16
      v[2 * j] = __uint_as_float(static_cast<uint32_t>(lo) << 16);
      v[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
    }
  }
}

// Cross-lane reductions without LDS traffic (__shfl_xor compiles to
// ds_bpermute): DPP inside 16-lane rows, lane-half swaps across rows.
// op_over(v, lo, hi) combines v over the lanes l ^ b for the b in [lo, hi)
// that are multiples of lo (lo, hi powers of two, 1 <= lo <= hi <= 64, and
// hi >= 16 when lo <= 4), every lane ending with the group's result.  The 4-
// and 8-lane steps use row rotations, which cover the same lane sets as xor 4
// and xor 8 once both are applied.
template <typename Op>
__device__ __forceinline__ float op_over(float v, int lo, int hi, Op op) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  if (lo <= 1 && hi > 1) v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));  // quad_perm [1,0,3,2]: lane ^ 1
  if (lo <= 2 && hi > 2) v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));  // quad_perm [2,3,0,1]: lane ^ 2
  if (lo <= 4 && hi > 4) v = op(v, dpp(v, std::integral_constant<int, 0x124>{})); // row_ror:4
  if (lo <= 8 && hi > 8) v = op(v, dpp(v, std::integral_constant<int, 0x128>{})); // row_ror:8 (lane ^ 8)
  if (lo <= 16 && hi > 16) {  // rows r and r ^ 1
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  if (lo <= 32 && hi > 32) {  // lane halves
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  return v;
}
struct OpAdd {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Lookup of an expert's per-group INT8 extension (see latent_factor).
struct Int8Ext {
  const uint32_t* bitmap;      // [E][rows][words]
  const int32_t* row_offset;   // [E][rows]
  const int8_t* data;          // [n][32]
  const int32_t* word_offset;  // [E][rows][words]: index of each bitmap word's first INT8
                               // group (row_offset itself when words == 1); NULL: not built
};

// One stacked factor with the expert strides resolved.
struct Factor {
  const uint8_t* codes;
  const uint16_t* scales;
  Int8Ext ext;
  int64_t rows, cols;
  __host__ __device__ int64_t code_stride() const { return cols / 2; }      // bytes per row
  __host__ __device__ int64_t scale_stride() const { return cols / kGroup; } // groups per row
  __host__ __device__ int words() const { return static_cast<int>((cols / kGroup + 31) / 32); }
};

__device__ __forceinline__ int popc(uint32_t v) { return __builtin_popcount(v); }

// Decode one 32-element group of row `row` of expert `e` into fp32 codebook
// values (not yet scaled).  NF4: 16 bytes, low nibble first.  INT8: 32 bytes
// of the side buffer.  The group's scale is returned separately by the caller.
template <bool kHasInt8>
__device__ __forceinline__ void decode_group(const Factor& f, int64_t e, int64_t row, int g, const float* lut,
                                             float v[kGroup]) {
  const int64_t erow = e * f.rows + row;
  // kHasInt8 selects the code path for a layer in which some factor carries the
  // extension; factors without it (bitmap == nullptr) are pure NF4.
  if (kHasInt8 && f.ext.bitmap != nullptr) {
    const uint32_t* bm = f.ext.bitmap + erow * f.words();
    const uint32_t word = bm[g >> 5];
    if ((word >> (g & 31)) & 1u) {
      int64_t idx = popc(word & ((1u << (g & 31)) - 1u));
      if (f.ext.word_offset) {
        idx += f.ext.word_offset[erow * f.words() + (g >> 5)];
      } else {
        for (int w = 0; w < (g >> 5); ++w) idx += popc(bm[w]);
        idx += f.ext.row_offset[erow];
      }
      const uint4* q = reinterpret_cast<const uint4*>(f.ext.data + idx * kGroup);
      const uint4 q0 = q[0], q1 = q[1];
      const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) v[i * 4 + b] = static_cast<float>(static_cast<int8_t>((qw[i] >> (8 * b)) & 0xFF));
      }
      return;
    }
  }
  const uint4 c = *reinterpret_cast<const uint4*>(f.codes + erow * f.code_stride() + static_cast<int64_t>(g) * kGroupBytes);
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int n = 0; n < 8; ++n) v[i * 8 + n] = lut[(cw[i] >> (4 * n)) & 15u];
  }
}

__device__ __forceinline__ float group_scale(const Factor& f, int64_t e, int64_t row, int g) {
  return half_bits_to_float(f.scales[(e * f.rows + row) * f.scale_stride() + g]);
}

__device__ __forceinline__ void atomic_add_f32(float* p, float v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace latent
