// Streaming MFMA decode path of the LATENT MoE-layer expert FFN (gfx950).
//
// Replaces, for decode-sized batches, the per-(token, slot) dispatch of
// kernels/latent_fused_expert_ffn.cu:27-108 and its launch loop (:255-289).
//
// The layer is a chain of grouped GEMVs over the routed experts.  Tokens are
// grouped by expert (prep kernel, moe.hip) and cut into work units of at most
// 16 pairs of one expert; every unit is one 16-row MFMA tile, so the work per
// factor byte does not grow with the number of tokens an expert receives.
//
//   A   x . A_g | A_u      K slices of 256 rows   -> partial latents  (reduce_a)
//   B   g_lat . B_g, u_lat . B_u  N slices of 256 -> g, u [pair][ff]
//   C   h . A_d, h = SiLU(g)*u     K slices of 256 -> partial d latent (reduce_c)
//   D   d_lat . B_d               N slices of 256 -> y rows, then the combine
//
// Each item (unit, 256 x 256 slice of one factor) is one 256-thread workgroup:
//   * the slice's NF4 codes (32 KB) and fp16 scales (4 KB) go global -> LDS by
//     direct loads (global_load_lds_dwordx4), 16-byte chunks XOR-swizzled so
//     the fragment reads below are free of bank conflicts;
//   * the unit's activation rows are scaled by a power of two per row (row
//     maximum in [2^14, 2^15)) and stored as fp16 [16][256];
//   * wave w owns 128 columns (w & 1) and 128 K rows (w >> 1).  Lane l reads
//     one code dword (8 columns) from each of 8 consecutive rows, interleaves
//     the nibbles of row pairs (k, k+1) into bytes, and looks each byte up in
//     a 256-entry table of (level, level) fp16 pairs: that dword, times the
//     two rows' fp16 scales (one v_pk_mul_f16), is one K pair of an MFMA B
//     fragment.  The 8 columns of the dword feed 8 v_mfma_f32_16x16x32_f16
//     whose N blocks are the columns 8n + j, so a lane's accumulators hold 8
//     adjacent output columns;
//   * the two K halves are added through LDS, rows are unscaled (2^-e) and
//     stored in fp32.
//
// Arithmetic: fp16 operands (levels and scales exact in fp16 up to one
// rounding of level * scale and of the scaled activation), fp32 accumulation.
// Every sum runs in a fixed order, so results are bit-reproducible.
#include "stream.hpp"

#include <algorithm>

namespace latent {
namespace stream {
namespace {

constexpr int kT = 256;                       // threads per workgroup
constexpr int kK = 256;                       // K rows per item slice
constexpr int kN = 256;                       // N columns per item slice
constexpr int kChunks = kN / kGroup;          // 16-byte code chunks (= scale groups) per slice row
constexpr int kActPitch = kK + 8;             // fp16 per LDS activation row (16-byte pad)
constexpr int kLutCopies = 8;
constexpr int kExpMin = -120, kExpMax = 120;
enum { F_GATE_A = 0, F_GATE_B, F_UP_A, F_UP_B, F_DOWN_A, F_DOWN_B };
enum Phase { kPhaseA = 0, kPhaseB, kPhaseC, kPhaseD };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

struct Params {
  Factor fac[6];
  Grouping g;
  const void* x;
  const int32_t* ids;
  float* out;
  float* partA;  // [2][nks][P][256]
  float* lat;    // [2][P][256]
  float* gu;     // [2][P][ff]
  float* partC;  // [nkc][P][256]
  float* dlat;   // [P][256]
  float* ybuf;   // [T*K][d]
  int x_dtype, T, K, E, d, ff, P, wbd, out_mode;
  int umax;  // units the unit tables hold
  int nks, nbs, nkc, nds;  // slices: A (d/256), B (ff/256), C (ff/256), D (d/256)
};

// LDS byte address of a __shared__ object and raw LDS loads.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T& obj) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)(&obj)));
}
template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr));
}

// A wave-uniform 64-bit address in scalar registers.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Direct global -> LDS load of 16 bytes at base + off (base wave-uniform, off
// per lane): lane l's bytes land at LDS byte lds + 16 l (lds wave-uniform).
// Inline assembly keeps the compiler from making later LDS reads wait on it;
// the kernel waits itself (vmcnt) before its barrier.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "m0", "memory");
}

// Chunk (row r, chunk c) of a slice sits in LDS slot r * 8 + (c ^ 4 * bit3(r)):
// rows r and r + 8, read by the two K quarters of one half-wave, use opposite
// chunk halves, so a half-wave's 32 dword reads hit 32 distinct banks.  The
// map is an involution, so the load side uses the same formula.

// Exponent e with m * 2^e in [2^14, 2^15) (0 for m == 0 or not finite).
__device__ __forceinline__ int row_exponent(float m) {
  if (!(m > 0.f) || !(m < 3.0e38f)) return 0;
  const int ilog = static_cast<int>((__float_as_uint(m) >> 23) & 0xFFu) - 127;
  return min(kExpMax, max(kExpMin, 14 - ilog));
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// s_waitcnt vmcnt(n) (n < 64) with lgkmcnt and expcnt left alone.
template <int kCount>
__device__ __forceinline__ void wait_vm() {
  static_assert(kCount >= 0 && kCount < 64, "vmcnt field");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((kCount & 15) | (7 << 4) | (15 << 8) | ((kCount >> 4) << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Barrier for LDS data: lgkmcnt(0) + s_barrier; direct loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Shared memory of one item.  After the K loop the whole block is reused as
// the fold buffer of the two K halves ([2 column halves][16 rows][128] fp32).
struct alignas(16) ItemSmem {
  union {
    struct {
      uint16_t scales[kK * kChunks];     // [row][group] fp16 bits
      _Float16 act[kMaxM * kActPitch];   // [row][k] fp16, row scaled by 2^rexp
      uint32_t lut[256 * kLutCopies];    // [byte][copy]: half2(level(lo nibble), level(hi nibble))
    } in;
    float fold[2 * kMaxM * 128];
  } u;
  int rexp[kMaxM];
};

template <int kPhase>
__device__ __forceinline__ int items_per_unit(const Params& p) {
  return kPhase == kPhaseA ? 2 * p.nks : kPhase == kPhaseB ? 2 * p.nbs : kPhase == kPhaseC ? p.nkc : p.nds;
}

// One workgroup per (unit, slice) item.  Loads are issued in the order
// activations, scales (direct to LDS), codes (to VGPRs, 8 rows per K step), so
// that waiting for the activations leaves the code loads in flight and each K
// step waits only for its own rows.
template <int kPhase>
__global__ void __launch_bounds__(kT, 5) item_kernel(Params p) {
  __shared__ ItemSmem sm;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Items of a unit are numbered in blocks of 8 (padded); block g runs on XCD
  // g % 8 (workgroup b runs on XCD b % 8), so the 8 column slices that share
  // each 128-byte line of scales (phases B and D) are read through one L2.
  const int per = items_per_unit<kPhase>(p);
  const int per_pad = (per + 7) & ~7;
  const int b = blockIdx.x, k = b >> 3;
  const int item = (((k >> 3) << 3) + (b & 7)) * 8 + (k & 7);
  const int unit = item / per_pad;
  const int sub = item - unit * per_pad;
  if (sub >= per || unit >= p.umax) return;
  // Row tables do not depend on unit_info: load them alongside it.
  const int arow = tid >> 4;  // activation row of this thread (16 columns each)
  int atok = 0;
  if (kPhase == kPhaseA) atok = p.g.unit_tok[unit * kMaxM + arow];
  float aw = 1.0f;
  if (kPhase == kPhaseC && p.wbd) aw = p.g.unit_w[unit * kMaxM + arow];
  if (unit >= p.g.meta[4]) return;
  const int4 info = p.g.unit_info[unit];
  const int e = __builtin_amdgcn_readfirstlane(info.x);
  const int start = __builtin_amdgcn_readfirstlane(info.y);
  const int m = __builtin_amdgcn_readfirstlane(info.z);

  int f = 0, slice, fi, row0 = 0, col0 = 0;
  if (kPhase == kPhaseA) {
    f = sub / p.nks;
    slice = sub - f * p.nks;
    fi = f ? F_UP_A : F_GATE_A;
    row0 = slice * kK;
  } else if (kPhase == kPhaseB) {
    f = sub / p.nbs;
    slice = sub - f * p.nbs;
    fi = f ? F_UP_B : F_GATE_B;
    col0 = slice * kN;
  } else if (kPhase == kPhaseC) {
    slice = sub;
    fi = F_DOWN_A;
    row0 = slice * kK;
  } else {
    slice = sub;
    fi = F_DOWN_B;
    col0 = slice * kN;
  }
  const Factor& F = p.fac[fi];
  const int64_t frow = static_cast<int64_t>(e) * F.rows + row0;
  const uint8_t* codes = F.codes + frow * F.code_stride() + col0 / 2;
  const uint16_t* scales = F.scales + frow * F.scale_stride() + col0 / kGroup;
  const int64_t code_row = F.code_stride();

  // 1. Raw activation chunks (16 values per thread), converted after the code
  //    loads are in flight.  Rows past the unit's pairs load a valid row and
  //    are zeroed later.
  const int kk = (tid & 15) * 16;
  const bool live = arow < m;
  const int pair = start + min(arow, m - 1);
  uint4 raw[8];
  if (kPhase == kPhaseA) {
    const int64_t base = static_cast<int64_t>(atok) * p.d + row0 + kk;
    if (p.x_dtype == LATENT_F32) {
      const uint4* s4 = reinterpret_cast<const uint4*>(static_cast<const float*>(p.x) + base);
#pragma unroll
      for (int q = 0; q < 4; ++q) raw[q] = s4[q];
    } else {
      const uint4* s4 = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.x) + base);
#pragma unroll
      for (int q = 0; q < 2; ++q) raw[q] = s4[q];
    }
  } else if (kPhase == kPhaseC) {
    const int64_t base = static_cast<int64_t>(pair) * p.ff + row0 + kk;
    const uint4* g4 = reinterpret_cast<const uint4*>(p.gu + base);
    const uint4* u4 = reinterpret_cast<const uint4*>(p.gu + static_cast<int64_t>(p.P) * p.ff + base);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      raw[q] = g4[q];
      raw[4 + q] = u4[q];
    }
  } else {
    const float* src = kPhase == kPhaseB ? p.lat + (static_cast<int64_t>(f) * p.P + pair) * kK
                                         : p.dlat + static_cast<int64_t>(pair) * kK;
    const uint4* s4 = reinterpret_cast<const uint4*>(src + kk);
#pragma unroll
    for (int q = 0; q < 4; ++q) raw[q] = s4[q];
  }

  // 2. Scales: 256 rows x 16 bytes, direct to LDS (one load per thread).
  dma16(scales, static_cast<uint32_t>(tid * F.scale_stride() * 2), lds_addr(sm.u.in.scales[0]) + wave * kWave * 16);

  // 3. Codes: wave -> (column half ch, K half kh); lane -> (dword cq, K quarter
  //    kq).  Rows kh*128 + s*32 + kq*8 + i, dword ch*16 + cq of the slice row.
  const int ch = wave & 1, kh = wave >> 1;
  const int cq = lane & 15, kq = lane >> 4;
  uint32_t d[4][8];
  {
    const uint8_t* cbase = codes + (ch * 16 + cq) * 4;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        d[s][i] = *reinterpret_cast<const uint32_t*>(cbase + (kh * 128 + s * 32 + kq * 8 + i) * code_row);
  }

  // 4. Level-pair table (one entry per thread, kLutCopies copies).
  {
    const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
    const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
    uint4* dstv = reinterpret_cast<uint4*>(&sm.u.in.lut[tid * kLutCopies]);
    dstv[0] = make_uint4(bits, bits, bits, bits);
    dstv[1] = make_uint4(bits, bits, bits, bits);
  }

  // 5. Activation rows -> fp16 scaled by 2^rexp (row maximum over its 16 threads).
  {
    float v[16];
    if (kPhase == kPhaseA && p.x_dtype != LATENT_F32) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t w[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t lo = w[i] & 0xFFFFu, hi = w[i] >> 16;
          if (p.x_dtype == LATENT_BF16) {
            v[8 * q + 2 * i] = __uint_as_float(lo << 16);
            v[8 * q + 2 * i + 1] = __uint_as_float(hi << 16);
          } else {
            v[8 * q + 2 * i] = half_bits_to_float(static_cast<uint16_t>(lo));
            v[8 * q + 2 * i + 1] = half_bits_to_float(static_cast<uint16_t>(hi));
          }
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 t = __builtin_bit_cast(float4, raw[q]);
        v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
      }
      if (kPhase == kPhaseC) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 u = __builtin_bit_cast(float4, raw[4 + q]);
          v[4 * q] = silu(v[4 * q]) * u.x * aw;
          v[4 * q + 1] = silu(v[4 * q + 1]) * u.y * aw;
          v[4 * q + 2] = silu(v[4 * q + 2]) * u.z * aw;
          v[4 * q + 3] = silu(v[4 * q + 3]) * u.w * aw;
        }
      }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = live ? v[i] : 0.f;
      mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = op_over(mx, 1, 16, OpMax{});
    const int ex = row_exponent(mx);
    half8 h0, h1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      h0[i] = static_cast<_Float16>(ldexpf(v[i], ex));
      h1[i] = static_cast<_Float16>(ldexpf(v[8 + i], ex));
    }
    half8* dst = reinterpret_cast<half8*>(&sm.u.in.act[arow * kActPitch + kk]);
    dst[0] = h0;
    dst[1] = h1;
    if ((tid & 15) == 0) sm.rexp[arow] = ex;
  }
  // The scale loads precede the 32 code loads: at most 32 outstanding => scales landed.
  wait_vm<32>();
  lds_barrier();

  // 6. K loop.
  const int c = ch * 4 + (cq >> 2);
  const uint32_t lut_lane = lds_addr(sm.u.in.lut[0]) + ((lane & (kLutCopies - 1)) << 2);
  const uint32_t scale_base = lds_addr(sm.u.in.scales[0]) + c * 2;
  float4v acc[8];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) acc[jj] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int k0 = kh * 128 + s * 32 + kq * 8;
    const half8 a = *reinterpret_cast<const half8*>(&sm.u.in.act[cq * kActPitch + k0]);
    uint32_t sp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t s0 = lds_ld<uint16_t>(scale_base + (k0 + 2 * q) * (kChunks * 2));
      const uint32_t s1 = lds_ld<uint16_t>(scale_base + (k0 + 2 * q + 1) * (kChunks * 2));
      sp[q] = s0 | (s1 << 16);
    }
    uint32_t frag[8][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = (d[s][2 * q] & 0x0F0F0F0Fu) | ((d[s][2 * q + 1] << 4) & 0xF0F0F0F0u);
      const uint32_t hi = ((d[s][2 * q] >> 4) & 0x0F0F0F0Fu) | (d[s][2 * q + 1] & 0xF0F0F0F0u);
      const half2v sc = __builtin_bit_cast(half2v, sp[q]);
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const uint32_t pe = lds_ld<uint32_t>(lut_lane + (((lo >> (8 * bb)) & 0xFFu) << 5));
        const uint32_t po = lds_ld<uint32_t>(lut_lane + (((hi >> (8 * bb)) & 0xFFu) << 5));
        frag[2 * bb][q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pe) * sc);
        frag[2 * bb + 1][q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, po) * sc);
      }
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint4 fv = make_uint4(frag[jj][0], frag[jj][1], frag[jj][2], frag[jj][3]);
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, fv), acc[jj], 0, 0, 0);
    }
  }

  // 7. Add the K halves through LDS (the inputs are dead now), unscale, store.
  lds_barrier();
  if (kh == 1) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int row = kq * 4 + vv;
      if (row >= m) continue;
      float4* dst = reinterpret_cast<float4*>(&sm.u.fold[(ch * kMaxM + row) * 128 + cq * 8]);
      dst[0] = make_float4(acc[0][vv], acc[1][vv], acc[2][vv], acc[3][vv]);
      dst[1] = make_float4(acc[4][vv], acc[5][vv], acc[6][vv], acc[7][vv]);
    }
  }
  lds_barrier();
  if (kh == 1) return;
  int ddst[4];
  float dw[4];
  if (kPhase == kPhaseD) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      ddst[vv] = p.g.unit_dst[unit * kMaxM + kq * 4 + vv];
      dw[vv] = p.g.unit_w[unit * kMaxM + kq * 4 + vv];
    }
  }
#pragma unroll
  for (int vv = 0; vv < 4; ++vv) {
    const int row = kq * 4 + vv;
    if (row >= m) continue;
    const float4* src = reinterpret_cast<const float4*>(&sm.u.fold[(ch * kMaxM + row) * 128 + cq * 8]);
    const float4 f0 = src[0], f1 = src[1];
    float sc = ldexpf(1.0f, -sm.rexp[row]);
    const int prow = start + row;
    const int col = ch * 128 + cq * 8;
    float* dst;
    if (kPhase == kPhaseA) {
      dst = p.partA + ((static_cast<int64_t>(f) * p.nks + slice) * p.P + prow) * kN + col;
    } else if (kPhase == kPhaseB) {
      dst = p.gu + (static_cast<int64_t>(f) * p.P + prow) * p.ff + col0 + col;
    } else if (kPhase == kPhaseC) {
      dst = p.partC + (static_cast<int64_t>(slice) * p.P + prow) * kN + col;
    } else {
      if (p.out_mode == LATENT_OUT_REDUCED && !p.wbd) sc *= dw[vv];
      dst = (p.out_mode == LATENT_OUT_REDUCED ? p.ybuf : p.out) + static_cast<int64_t>(ddst[vv]) * p.d + col0 + col;
    }
    reinterpret_cast<float4*>(dst)[0] = make_float4((acc[0][vv] + f0.x) * sc, (acc[1][vv] + f0.y) * sc,
                                                    (acc[2][vv] + f0.z) * sc, (acc[3][vv] + f0.w) * sc);
    reinterpret_cast<float4*>(dst)[1] = make_float4((acc[4][vv] + f1.x) * sc, (acc[5][vv] + f1.y) * sc,
                                                    (acc[6][vv] + f1.z) * sc, (acc[7][vv] + f1.w) * sc);
  }
}

constexpr int kSumBatch = 8;

__device__ __forceinline__ void add4(float4& s, const float4& v) {
  s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
}

// sum_{j < n} src[j * stride], added in j order; the loads of a batch of
// kBatch terms are all issued before the first add.  Adding the +0 fill of
// a partial batch leaves the sum unchanged.
template <int kBatch>
__device__ __forceinline__ float4 sum_strided(const float4* src, int64_t stride, int n) {
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < n; k0 += kBatch) {
    float4 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      v[j] = k0 + j < n ? src[static_cast<int64_t>(k0 + j) * stride] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) add4(s, v[j]);
  }
  return s;
}

// lat[f][pair][:] = sum over K slices of partA[f][ks][pair][:], slices in order.
__global__ void __launch_bounds__(kT) reduce_a_kernel(Params p) {
  const int routed = p.g.meta[3];
  const int64_t n4 = 2LL * routed * (kN / 4);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; i < n4; i += static_cast<int64_t>(gridDim.x) * kT) {
    const int64_t f = i / (static_cast<int64_t>(routed) * (kN / 4));
    const int64_t rem = i - f * routed * (kN / 4);
    const int64_t pair = rem / (kN / 4), c4 = rem - pair * (kN / 4);
    const float4* src = reinterpret_cast<const float4*>(p.partA + (f * p.nks * p.P + pair) * kN) + c4;
    reinterpret_cast<float4*>(p.lat + (f * p.P + pair) * kN)[c4] =
        sum_strided<32>(src, static_cast<int64_t>(p.P) * (kN / 4), p.nks);
  }
}

// dlat[pair][:] = sum over K slices of partC[ks][pair][:], slices in order.
__global__ void __launch_bounds__(kT) reduce_c_kernel(Params p) {
  const int routed = p.g.meta[3];
  const int64_t n4 = static_cast<int64_t>(routed) * (kN / 4);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; i < n4; i += static_cast<int64_t>(gridDim.x) * kT) {
    const int64_t pair = i / (kN / 4), c4 = i - pair * (kN / 4);
    const float4* src = reinterpret_cast<const float4*>(p.partC + pair * kN) + c4;
    reinterpret_cast<float4*>(p.dlat + pair * kN)[c4] = sum_strided<kSumBatch>(src, static_cast<int64_t>(p.P) * (kN / 4), p.nkc);
  }
}

// out[t][:] = sum over the token's valid slots, in slot order, of ybuf[t*K + slot][:].
__global__ void __launch_bounds__(kT) combine_kernel(Params p) {
  const int64_t d4 = p.d / 4;
  const int64_t n4 = static_cast<int64_t>(p.T) * d4;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; i < n4; i += static_cast<int64_t>(gridDim.x) * kT) {
    const int64_t t = i / d4, c4 = i - t * d4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < p.K; k0 += kSumBatch) {
      float4 v[kSumBatch];
#pragma unroll
      for (int j = 0; j < kSumBatch; ++j) {
        const int k = k0 + j;
        const int e = k < p.K ? p.ids[t * p.K + k] : -1;
        v[j] = (e >= 0 && e < p.E) ? reinterpret_cast<const float4*>(p.ybuf + (t * p.K + k) * p.d)[c4]
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int j = 0; j < kSumBatch; ++j) add4(s, v[j]);
    }
    reinterpret_cast<float4*>(p.out)[i] = s;
  }
}

}  // namespace
}  // namespace stream
}  // namespace latent

// ===========================================================================
// Host side
// ===========================================================================
namespace latent {
namespace stream {

static bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

bool supported(const latent_moe_args& a) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs) {
    if (f->int8_bitmap || f->int8_row_offset || f->int8_data) return false;
    if (!aligned16(f->codes) || !aligned16(f->scales)) return false;
  }
  const int64_t P = a.n_tokens * a.n_expert_used;
  return a.max_rank == kK && a.n_embd % kK == 0 && a.n_ff % kK == 0 && P >= 1 && P <= 4096 && aligned16(a.x) &&
         a.n_expert <= 4096;
}

int64_t max_units(int64_t pairs, int64_t experts) { return std::min(pairs, experts) + pairs / kMaxM; }

Layout layout_for(const latent_moe_args& a) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const int64_t P = a.n_tokens * a.n_expert_used, d = a.n_embd, ff = a.n_ff;
  Layout L{};
  size_t off = 0;
  L.partA = off; off = al(off + 2ull * (d / kK) * P * kN * 4);
  L.lat = off;   off = al(off + 2ull * P * kN * 4);
  L.gu = off;    off = al(off + 2ull * P * ff * 4);
  L.partC = off; off = al(off + static_cast<size_t>(ff / kK) * P * kN * 4);
  L.dlat = off;  off = al(off + static_cast<size_t>(P) * kN * 4);
  L.ybuf = off;  off = al(off + static_cast<size_t>(P) * d * 4);
  L.total = off;
  return L;
}

int forward(const latent_moe_args& a, const Factor* fac, const Grouping& g, char* scratch, hipStream_t s) {
  const Layout L = layout_for(a);
  Params p{};
  for (int i = 0; i < 6; ++i) p.fac[i] = fac[i];
  p.g = g;
  p.x = a.x;
  p.ids = a.ids;
  p.out = static_cast<float*>(a.out);
  p.partA = reinterpret_cast<float*>(scratch + L.partA);
  p.lat = reinterpret_cast<float*>(scratch + L.lat);
  p.gu = reinterpret_cast<float*>(scratch + L.gu);
  p.partC = reinterpret_cast<float*>(scratch + L.partC);
  p.dlat = reinterpret_cast<float*>(scratch + L.dlat);
  p.ybuf = reinterpret_cast<float*>(scratch + L.ybuf);
  p.x_dtype = a.x_dtype;
  p.T = static_cast<int>(a.n_tokens);
  p.K = static_cast<int>(a.n_expert_used);
  p.E = static_cast<int>(a.n_expert);
  p.d = static_cast<int>(a.n_embd);
  p.ff = static_cast<int>(a.n_ff);
  p.P = p.T * p.K;
  p.wbd = a.weight_before_down ? 1 : 0;
  p.out_mode = a.out_mode;
  p.nks = p.d / kK;
  p.nbs = p.ff / kN;
  p.nkc = p.ff / kK;
  p.nds = p.d / kN;
  const unsigned U = static_cast<unsigned>(max_units(p.P, a.n_expert));
  p.umax = static_cast<int>(U);
  auto red_grid = [](int64_t n4) { return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(2048, (n4 + kT - 1) / kT))); };
  // Grids cover every unit's items padded to blocks of 8, rounded to 64
  // workgroups (a whole block of 8 per XCD).
  auto item_grid = [&](int64_t per) { return static_cast<unsigned>((U * ((per + 7) / 8 * 8) + 63) / 64 * 64); };
  hipLaunchKernelGGL(item_kernel<kPhaseA>, dim3(item_grid(2 * p.nks)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(reduce_a_kernel, dim3(red_grid(2LL * p.P * (kN / 4))), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseB>, dim3(item_grid(2 * p.nbs)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseC>, dim3(item_grid(p.nkc)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(reduce_c_kernel, dim3(red_grid(static_cast<int64_t>(p.P) * (kN / 4))), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseD>, dim3(item_grid(p.nds)), dim3(kT), 0, s, p);
  if (a.out_mode == LATENT_OUT_REDUCED)
    hipLaunchKernelGGL(combine_kernel, dim3(red_grid(static_cast<int64_t>(p.T) * p.d / 4)), dim3(kT), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace stream
}  // namespace latent
