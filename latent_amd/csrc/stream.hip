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
//   A   x . A_g | A_u               K slices of 256 rows -> partial latents (reduce_a)
//   B   g = g_lat . B_g, u = u_lat . B_u, h = SiLU(g) * u [* w]
//                                   N slices of 256, gate and up paired
//   C   h . A_d                     K slices of 256 rows -> partial d latent (reduce_c)
//   D   d_lat . B_d                 N slices of 256      -> y rows, then the combine
//
// Every activation a phase reads is an fp16 row with one power-of-two
// exponent per row and 256-column slice (row maximum in [2^14, 2^15)): the
// prep kernel writes x that way, reduce_a / reduce_c the latents and phase B
// h, so the latents of a LATENT chain (1e-3 ... 1e-9 here) keep fp16's full
// precision.
//
// One 256-thread workgroup runs a group of consecutive slices of one unit.
// Per slice (a 256 x 256 block of a factor):
//   * wave w owns column half ch = w & 1 and K half kh = w >> 1; lane
//     (cq = lane & 15, kq = lane >> 4) loads one code dword (columns
//     ch*128 + 8cq .. +7) of rows kq*8 .. kq*8+7 of each 32-row step: 32
//     buffer loads per slice into registers, issued one slice ahead;
//   * the slice's fp16 scales (4 KB) and, for K slices, its activation rows
//     (8 KB) and their exponents go global -> LDS by direct loads
//     (global_load_lds), issued two slices ahead into double buffers;
//   * the nibbles of row pairs (k, k+1) are interleaved into bytes, each byte
//     is looked up in a 256-entry table of (level, level) fp16 pairs in LDS,
//     and one v_pk_mul_f16 by the two rows' fp16 scales gives one K pair of an
//     MFMA B fragment: column j of the dword feeds v_mfma_f32_16x16x32_f16
//     number j, whose N block is the columns 8n + j of the half;
//   * the two K halves are added through LDS.
// K-sliced phases (A, C) accumulate a group's slices in registers (rescaled
// when the next slice's row exponents differ) and write one partial sum per
// group; N-sliced phases (B, D) write every slice.
//
// Units run on XCD (unit mod 8) -- workgroup b runs on XCD b mod 8 -- so all
// slices of a unit, which share activation rows and 128-byte lines of scales,
// are read through one L2.
//
// Arithmetic: fp16 operands (levels and scales exact in fp16 up to one
// rounding of level * scale and of the scaled activation), fp32 accumulation.
// Every sum runs in a fixed order, so results are bit-reproducible.
#include "stream.hpp"

#include <algorithm>
#include <type_traits>

namespace latent {
namespace stream {
namespace {

constexpr int kT = 256;                    // threads per workgroup
constexpr int kK = 256;                    // K rows per slice
constexpr int kN = 256;                    // N columns per slice
constexpr int kSliceGroups = kN / kGroup;  // scale groups per slice row
constexpr int kActChunks = kK / 8;         // 16-byte chunks of an fp16 activation row
constexpr int kLutCopies = 32;            // one table copy per LDS bank
constexpr int kMaxNB = 8;                  // N (or K) slices per workgroup
enum { F_GATE_A = 0, F_GATE_B, F_UP_A, F_UP_B, F_DOWN_A, F_DOWN_B };
enum Phase { kPhaseA = 0, kPhaseB, kPhaseC, kPhaseD };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

struct Params {
  Factor fac[6];
  Grouping g;
  const int32_t* ids;
  float* out;
  const _Float16* xh;  // [T][d] fp16 x * 2^xexp
  const int* xexp;     // [T]
  float* partA;        // [2][gA][P][256]
  _Float16* lath;      // [2][P][256]
  int* lexp;           // [2][P]
  _Float16* hh;        // [P][ff]
  int* hexp;           // [P][ff/256]
  float* partC;        // [gC][P][256]
  _Float16* dlath;     // [P][256]
  int* dexp;           // [P]
  float* ybuf;         // [T*K][d]
  int T, K, E, d, ff, P, wbd, out_mode;
  int umax;                // units the unit tables hold
  int nks, nbs, nkc, nds;  // slices: A (d/256), B (ff/256), C (ff/256), D (d/256)
  int nb[4];               // slices per group, per phase (B: N slices, each run for gate and up)
  int gA, gB, gC, gD;      // groups: A per factor, B/C/D per unit
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

// Direct global -> LDS loads.  Lane l's bytes land at LDS byte lds + 16 l
// (dwordx4) or lds + 4 l (dword); lds is wave-uniform.  Inline assembly keeps
// the compiler from making later LDS reads wait on them: the kernel counts
// them itself (vmcnt) before the barrier that publishes the data.
// Uniform base + per-lane 32-bit offset:
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "m0", "memory");
}

// Raw (byte-addressed) buffer resource over `bytes` bytes from `base`
// (wave-uniform); loads beyond them return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(base)), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// SiLU with the hardware exponential and reciprocal (each within about 1 ulp);
// g -> -inf gives -0, g -> +inf gives g.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// s_waitcnt vmcnt(n): at most n vector memory operations of this wave left
// outstanding.  Inline assembly: the compiler does not see the direct loads
// this wait is for, so it would drop a wait it thinks satisfied.
template <int kCount>
__device__ __forceinline__ void wait_vm() {
  static_assert(kCount >= 0 && kCount < 63, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCount) : "memory");
}
// Barrier for LDS data: lgkmcnt(0) + s_barrier; direct loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Shared memory of one workgroup (about 73 KB: two resident per CU).
struct alignas(16) ItemSmem {
  uint32_t lut[256 * kLutCopies];         // [byte][copy]: half2(level(lo nibble), level(hi nibble))
  uint16_t scales[2][kK * kSliceGroups];  // [buffer][row][group] fp16 bits
  uint4 act[2][kMaxM * kActChunks];       // [buffer][row][chunk ^ row]: fp16 rows * 2^rexp
  float fold[2 * kMaxM * 128];            // K half 1 of both column halves ([ch][row][128])
  int rexp[2][kMaxM];                     // row exponents of act[buffer]
  float hmax[2][kMaxM];                   // phase B: row maxima of h per column half
  uint32_t row_dst[kMaxM];                // phase D: output row offset of each row
  float row_w[kMaxM];                     // router weight applied to each row (1 if none)
};

// Chunk c of activation row r sits at chunk (c ^ (r & 15)) of the row: the 16
// rows an MFMA fragment read touches then hit 16 different bank groups.
__device__ __forceinline__ int act_slot(int row, int chunk) { return row * kActChunks + (chunk ^ (row & 15)); }

template <int kPhase>
__device__ __forceinline__ int groups_per_unit(const Params& p) {
  return kPhase == kPhaseA ? 2 * p.gA : kPhase == kPhaseB ? p.gB : kPhase == kPhaseC ? p.gC : p.gD;
}

// Direct loads per run: scales, plus for K slices 2 activation loads and the exponents.
template <int kPhase>
constexpr int run_dma() {
  return kPhase == kPhaseA || kPhase == kPhaseC ? 4 : 1;
}

// Direct load of 4 bytes at base + off (base wave-uniform, off per lane):
// lane l's bytes land at LDS byte lds + 4 l.
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "m0", "memory");
}

// A 256-wide fp16 activation block of the unit's 16 rows into act buffer
// `buf`: thread tid loads chunk (tid % 32) of rows tid / 32 and 8 + tid / 32,
// at byte offsets off0 and off1 from `base` (the chunk position is added here).
__device__ __forceinline__ void dma_act(ItemSmem& sm, int buf, int tid, int wave, const void* base, uint32_t off0,
                                        uint32_t off1) {
  const int r0 = tid / kActChunks;
  const uint32_t c0 = (tid % kActChunks) ^ (r0 & 15), c1 = (tid % kActChunks) ^ ((r0 + 8) & 15);
  dma16(base, off0 + c0 * 16, lds_addr(sm.act[buf][0]) + wave * kWave * 16);
  dma16(base, off1 + c1 * 16, lds_addr(sm.act[buf][0]) + (kT + wave * kWave) * 16);
}

// The 16 row exponents into rexp[buf]: lane l < 16 loads row l's, at byte
// offset `off` from `base`.  Every wave loads the same values, so every wave
// counts the same loads.
__device__ __forceinline__ void dma_exp(ItemSmem& sm, int buf, int lane, const void* base, uint32_t off) {
  if (lane < kMaxM) dma4(base, off, lds_addr(sm.rexp[buf][0]));
}

// Issue the code loads of a slice: rows kh*128 + s*32 + kq*8 + i, dword
// ch*16 + cq of the slice row.  Buffer loads: one lane offset register, the
// row offset (s*32 + i) * code_row in a scalar register.
__device__ __forceinline__ void load_codes(uint32_t (&d)[4][8], const uint8_t* codes, uint32_t code_row, int ch, int kh,
                                           int cq, int kq) {
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(codes, kK * code_row);
  const uint32_t lane_off = (kh * 128 + kq * 8) * code_row + (ch * 16 + cq) * 4;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < 8; ++i) d[s][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, lane_off, (s * 32 + i) * code_row, 0);
}

// Decode + MFMA of one slice for this wave's four 32-row steps.
__device__ __forceinline__ void k_loop(const ItemSmem& sm, int sbuf, int abuf, const uint32_t (&d)[4][8], int ch,
                                       int kh, int cq, int kq, uint32_t lut_lane, float4v (&acc)[8]) {
  const int c = ch * 4 + (cq >> 2);
  const uint32_t scale_base = lds_addr(const_cast<ItemSmem&>(sm).scales[sbuf][0]) + c * 2;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int k0 = kh * 128 + s * 32 + kq * 8;
    const half8 a = __builtin_bit_cast(half8, sm.act[abuf][act_slot(cq, k0 / 8)]);
    uint32_t sp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t s0 = lds_ld<uint16_t>(scale_base + (k0 + 2 * q) * (kSliceGroups * 2));
      const uint32_t s1 = lds_ld<uint16_t>(scale_base + (k0 + 2 * q + 1) * (kSliceGroups * 2));
      sp[q] = s0 | (s1 << 16);
    }
    // Byte t of lo[q] holds column 2t of rows (2q, 2q+1), byte t of hi[q] column 2t+1.
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lo[q] = (d[s][2 * q] & 0x0F0F0F0Fu) | ((d[s][2 * q + 1] << 4) & 0xF0F0F0F0u);
      hi[q] = ((d[s][2 * q] >> 4) & 0x0F0F0F0Fu) | (d[s][2 * q + 1] & 0xF0F0F0F0u);
    }
    // Columns 2bb and 2bb + 1: their four K pairs, then their two MFMAs.
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      uint32_t fe[4], fo[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const half2v sc = __builtin_bit_cast(half2v, sp[q]);
        const uint32_t pe = lds_ld<uint32_t>(lut_lane + (((lo[q] >> (8 * bb)) & 0xFFu) << 7));
        const uint32_t po = lds_ld<uint32_t>(lut_lane + (((hi[q] >> (8 * bb)) & 0xFFu) << 7));
        fe[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pe) * sc);
        fo[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, po) * sc);
      }
      acc[2 * bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          a, __builtin_bit_cast(half8, make_uint4(fe[0], fe[1], fe[2], fe[3])), acc[2 * bb], 0, 0, 0);
      acc[2 * bb + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          a, __builtin_bit_cast(half8, make_uint4(fo[0], fo[1], fo[2], fo[3])), acc[2 * bb + 1], 0, 0, 0);
    }
  }
}

// Add the K halves: K-half-1 waves write rows < m to LDS, K-half-0 waves add
// them (after the call they hold the slice sums; the others are consumed).
__device__ __forceinline__ void fold_halves(ItemSmem& sm, float4v (&acc)[8], int ch, int kh, int cq, int kq, int m) {
  if (kh == 1) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int row = kq * 4 + vv;
      if (row >= m) continue;
      float4* dst = reinterpret_cast<float4*>(&sm.fold[(ch * kMaxM + row) * 128 + cq * 8]);
      dst[0] = make_float4(acc[0][vv], acc[1][vv], acc[2][vv], acc[3][vv]);
      dst[1] = make_float4(acc[4][vv], acc[5][vv], acc[6][vv], acc[7][vv]);
    }
  }
  lds_barrier();
  if (kh == 0) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int row = kq * 4 + vv;
      if (row >= m) continue;
      const float4* src = reinterpret_cast<const float4*>(&sm.fold[(ch * kMaxM + row) * 128 + cq * 8]);
      const float4 f0 = src[0], f1 = src[1];
      acc[0][vv] += f0.x; acc[1][vv] += f0.y; acc[2][vv] += f0.z; acc[3][vv] += f0.w;
      acc[4][vv] += f1.x; acc[5][vv] += f1.y; acc[6][vv] += f1.z; acc[7][vv] += f1.w;
    }
  }
}

// K-half-0 waves store rows < m of the sums scaled by 2^-rexp[buf][row] times
// scale(row) to dst_row(row) + the wave's 8 columns.
template <typename DstRow, typename RowScale>
__device__ __forceinline__ void store_rows(const ItemSmem& sm, int buf, const float4v (&acc)[8], int ch, int cq, int kq,
                                           int m, DstRow dst_row, RowScale scale) {
#pragma unroll
  for (int vv = 0; vv < 4; ++vv) {
    const int row = kq * 4 + vv;
    if (row >= m) continue;
    float* dst = dst_row(row) + ch * 128 + cq * 8;
    const float sc = scale(row) * ldexpf(1.0f, -sm.rexp[buf][row]);
    reinterpret_cast<float4*>(dst)[0] = make_float4(acc[0][vv] * sc, acc[1][vv] * sc, acc[2][vv] * sc, acc[3][vv] * sc);
    reinterpret_cast<float4*>(dst)[1] = make_float4(acc[4][vv] * sc, acc[5][vv] * sc, acc[6][vv] * sc, acc[7][vv] * sc);
  }
}

// One workgroup per (unit, group of consecutive slices).
template <int kPhase>
__global__ void __launch_bounds__(kT, 2) item_kernel(Params p) {
  __shared__ ItemSmem sm;
  constexpr bool kSliceK = kPhase == kPhaseA || kPhase == kPhaseC;  // slices along K (else along N)
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = wave & 1, kh = wave >> 1;
  const int cq = lane & 15, kq = lane >> 4;
  // Workgroup b runs on XCD b % 8 and takes units u == b (mod 8) in order.
  const int gpu = groups_per_unit<kPhase>(p);
  const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
  const int unit = xcd + 8 * (j / gpu);
  const int grp = j - (j / gpu) * gpu;
  if (unit >= p.umax || unit >= p.g.meta[4]) return;
  const int4 info = p.g.unit_info[unit];
  const int e = __builtin_amdgcn_readfirstlane(info.x);
  const int start = __builtin_amdgcn_readfirstlane(info.y);
  const int m = __builtin_amdgcn_readfirstlane(info.z);
  // Pair (grouped order) of activation row r; rows past the unit's pairs read
  // the last pair's row (their products are never stored).
  auto pair_of = [&](int r) { return start + min(r, m - 1); };
  // Per-row values this thread needs, read before any streaming load so that
  // no wait for them lands among the streaming loads: its two activation rows
  // (tid / 32, 8 + tid / 32), its exponent row (lane & 15) and the 4 output
  // rows kq*4 + vv it stores.
  const int ar0 = tid / kActChunks, ar1 = ar0 + kT / kActChunks, er = lane & 15;
  // Byte offsets of the activation rows (from the block's base) and of the
  // exponent row: A rows are tokens, the other phases' rows are pairs.
  uint32_t aoff0, aoff1, eoff;
  if constexpr (kPhase == kPhaseA) {
    aoff0 = static_cast<uint32_t>(p.g.unit_tok[unit * kMaxM + ar0]) * p.d * 2;
    aoff1 = static_cast<uint32_t>(p.g.unit_tok[unit * kMaxM + ar1]) * p.d * 2;
    eoff = static_cast<uint32_t>(p.g.unit_tok[unit * kMaxM + er]) * 4;
  } else {
    const uint32_t apitch = kPhase == kPhaseC ? p.ff * 2 : kK * 2;
    aoff0 = static_cast<uint32_t>(pair_of(ar0)) * apitch;
    aoff1 = static_cast<uint32_t>(pair_of(ar1)) * apitch;
    eoff = static_cast<uint32_t>(pair_of(er)) * (kPhase == kPhaseC ? p.nkc * 4 : 4);
  }
  // Output row offsets (D, floats) and weights (D reduced, B with the weight
  // before down) of the unit's rows, kept in LDS.
  if (tid < kMaxM) {
    const int row = min(tid, m - 1);
    sm.row_dst[tid] = kPhase == kPhaseD ? static_cast<uint32_t>(p.g.unit_dst[unit * kMaxM + row]) * p.d : 0u;
    const bool weighted =
        (kPhase == kPhaseD && !p.wbd && p.out_mode == LATENT_OUT_REDUCED) || (kPhase == kPhaseB && p.wbd);
    sm.row_w[tid] = weighted ? p.g.unit_w[unit * kMaxM + row] : 1.0f;
  }

  // The group: factor(s) and slices [s0, s0 + ns) of the factor's nsl slices.
  int f = 0, gi, nsl;
  if (kPhase == kPhaseA) {
    f = grp / p.gA;
    gi = grp - f * p.gA;
    nsl = p.nks;
  } else {
    gi = grp;
    nsl = kPhase == kPhaseB ? p.nbs : kPhase == kPhaseC ? p.nkc : p.nds;
  }
  const int nb = p.nb[kPhase];
  const int s0 = gi * nb;
  const int ns = min(nb, nsl - s0);
  const int nrun = kPhase == kPhaseB ? 2 * ns : ns;  // B runs (gate, up) per N slice
  const int fi0 = kPhase == kPhaseA ? (f ? F_UP_A : F_GATE_A) : kPhase == kPhaseB ? F_GATE_B
                  : kPhase == kPhaseC ? F_DOWN_A : F_DOWN_B;
  // Run q reads factor fi(q), slice sl(q): B alternates gate and up.
  auto fi_of = [&](int q) { return kPhase == kPhaseB ? ((q & 1) ? F_UP_B : F_GATE_B) : fi0; };
  auto sl_of = [&](int q) { return s0 + (kPhase == kPhaseB ? q >> 1 : q); };
  const uint32_t code_row = static_cast<uint32_t>(p.fac[fi0].code_stride());  // gate and up share shapes
  const uint32_t srow_bytes = static_cast<uint32_t>(p.fac[fi0].scale_stride() * 2);

  // Direct loads of run q: scales into buffer q & 1; K slices also their
  // activation rows and exponents.
  auto issue_dma = [&](int q) __attribute__((always_inline)) {
    const Factor& F = p.fac[fi_of(q)];
    const int sl = sl_of(q);
    const int64_t frow = static_cast<int64_t>(e) * F.rows + (kSliceK ? sl * kK : 0);
    const uint16_t* scales = F.scales + frow * F.scale_stride() + (kSliceK ? 0 : sl * kN / kGroup);
    dma16(scales, tid * srow_bytes, lds_addr(sm.scales[q & 1][0]) + wave * kWave * 16);
    if constexpr (kPhase == kPhaseA) {
      dma_act(sm, q & 1, tid, wave, p.xh + sl * kK, aoff0, aoff1);
      dma_exp(sm, q & 1, lane, p.xexp, eoff);
    } else if constexpr (kPhase == kPhaseC) {
      dma_act(sm, q & 1, tid, wave, p.hh + sl * kK, aoff0, aoff1);
      dma_exp(sm, q & 1, lane, p.hexp + sl, eoff);
    }
  };
  auto codes_of = [&](int q) {
    const Factor& F = p.fac[fi_of(q)];
    const int sl = sl_of(q);
    const int64_t frow = static_cast<int64_t>(e) * F.rows + (kSliceK ? sl * kK : 0);
    return F.codes + frow * F.code_stride() + (kSliceK ? 0 : sl * kN / 2);
  };

  // Level-pair table (one entry per thread, kLutCopies copies), built before
  // the streaming loads: its level lookups would otherwise wait for them.
  {
    const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
    const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
    uint4* dstv = reinterpret_cast<uint4*>(&sm.lut[tid * kLutCopies]);
    // Rotated start: the lanes of one store spread over the banks.
#pragma unroll
    for (int j = 0; j < kLutCopies / 4; ++j) dstv[(j + tid) & (kLutCopies / 4 - 1)] = make_uint4(bits, bits, bits, bits);
  }
  const uint32_t lut_lane = lds_addr(sm.lut[0]) + ((lane & (kLutCopies - 1)) << 2);

  // Prologue.  N-sliced phases read one activation block for the whole group
  // (B: the gate latent into buffer 0, the up latent into buffer 1).
  if constexpr (kPhase == kPhaseB) {
#pragma unroll
    for (int fb = 0; fb < 2; ++fb) {
      dma_act(sm, fb, tid, wave, p.lath + static_cast<int64_t>(fb) * p.P * kK, aoff0, aoff1);
      dma_exp(sm, fb, lane, p.lexp + static_cast<int64_t>(fb) * p.P, eoff);
    }
  } else if constexpr (kPhase == kPhaseD) {
    dma_act(sm, 0, tid, wave, p.dlath, aoff0, aoff1);
    dma_exp(sm, 0, lane, p.dexp, eoff);
  }
  uint32_t d0[4][8], d1[4][8];
  issue_dma(0);
  load_codes(d0, codes_of(0), code_row, ch, kh, cq, kq);
  if (nrun > 1) issue_dma(1);

  float4v acc[8];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) acc[jj] = float4v{0.f, 0.f, 0.f, 0.f};
  int prev_exp[4] = {0, 0, 0, 0};  // K slices: row exponent of the running sums (rows kq*4 + vv)
  float4v gkeep[8];                // B: the gate product of the current N slice (K-half-0 waves)

  // Run q (parity kOdd = q & 1, known where each copy is expanded): `cur`
  // holds its codes, `nxt` receives run q + 1's.
  auto run = [&](int q, auto odd, uint32_t (&cur)[4][8], uint32_t (&nxt)[4][8]) __attribute__((always_inline)) {
    constexpr int kOdd = decltype(odd)::value;
    // Loads complete in issue order.  After run q's direct loads come its 32
    // code loads (issued one run earlier) and run q + 1's direct loads, if
    // any (issued at the end of run q - 1): wait until no more are outstanding.
    if (q + 1 < nrun)
      wait_vm<32 + run_dma<kPhase>()>();
    else
      wait_vm<32>();
    lds_barrier();
    // Run q + 1's code loads; the last run loads its own codes again (an L2
    // hit), so that every run issues the same loads and the compiler's waits
    // for run q's codes never reach the ones issued here.
    load_codes(nxt, codes_of(min(q + 1, nrun - 1)), code_row, ch, kh, cq, kq);
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the slice's MFMAs
    constexpr int abuf = (kPhase == kPhaseB || kSliceK) ? kOdd : 0;
    if constexpr (kPhase == kPhaseC) {
      // Bring the running sums to this slice's row exponents (phase A's rows
      // are tokens, whose one exponent holds for every slice).
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
        const int ex = sm.rexp[kOdd][kq * 4 + vv];
        if (q > 0) {
          const float sc = ldexpf(1.0f, ex - prev_exp[vv]);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) acc[jj][vv] *= sc;
        }
        prev_exp[vv] = ex;
      }
    }
    k_loop(sm, kOdd, abuf, cur, ch, kh, cq, kq, lut_lane, acc);
    if constexpr (kPhase == kPhaseB) {
      fold_halves(sm, acc, ch, kh, cq, kq, m);
      if constexpr (!kOdd) {
        // Gate: keep g = acc * 2^-rexp_g for the up run of this N slice (the
        // K-half-1 waves keep values they never use).
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) {
          const float sc = ldexpf(1.0f, -sm.rexp[0][kq * 4 + vv]);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) gkeep[jj][vv] = acc[jj][vv] * sc;
        }
      } else {
        // Up: h = SiLU(g) * u [* w] with u = acc * 2^-rexp_u, stored fp16 with
        // one exponent per row and slice; the row maximum spans both column
        // halves and is exchanged through LDS.  Only the K-half-0 waves hold
        // the folded sums.
        const int sl = sl_of(q);
        float hv[8][4];
        if (kh == 0) {
#pragma unroll
          for (int vv = 0; vv < 4; ++vv) {
            const int row = kq * 4 + vv;
            const float rs = ldexpf(1.0f, -sm.rexp[1][row]) * sm.row_w[row];
            float mx = 0.f;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              hv[jj][vv] = silu(gkeep[jj][vv]) * (acc[jj][vv] * rs);
              mx = fmaxf(mx, fabsf(hv[jj][vv]));
            }
            mx = op_over(mx, 1, 16, OpMax{});
            if (cq == 0) sm.hmax[ch][row] = mx;
          }
        }
        lds_barrier();
        if (kh == 0) {
#pragma unroll
          for (int vv = 0; vv < 4; ++vv) {
            const int row = kq * 4 + vv;
            if (row >= m) continue;
            const int ex = pow2_row_exponent(fmaxf(sm.hmax[0][row], sm.hmax[1][row]));
            half8 hb;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) hb[jj] = static_cast<_Float16>(ldexpf(hv[jj][vv], ex));
            const int64_t prow = start + row;
            *reinterpret_cast<half8*>(p.hh + prow * p.ff + sl * kN + ch * 128 + cq * 8) = hb;
            if (ch == 0 && cq == 0) p.hexp[prow * p.nkc + sl] = ex;
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) acc[jj] = float4v{0.f, 0.f, 0.f, 0.f};
    } else if constexpr (kPhase == kPhaseD) {
      const int col0 = sl_of(q) * kN;
      fold_halves(sm, acc, ch, kh, cq, kq, m);
      if (kh == 0) {
        float* base = p.out_mode == LATENT_OUT_REDUCED ? p.ybuf : p.out;
        store_rows(
            sm, 0, acc, ch, cq, kq, m, [&](int row) { return base + sm.row_dst[row] + col0; },
            [&](int row) { return sm.row_w[row]; });
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) acc[jj] = float4v{0.f, 0.f, 0.f, 0.f};
    }
    lds_barrier();  // run q's LDS buffers are free for run q + 2
    if (q + 2 < nrun) issue_dma(q + 2);
  };
  for (int q = 0; q < nrun; q += 2) {
    run(q, std::integral_constant<int, 0>{}, d0, d1);
    if (q + 1 < nrun) run(q + 1, std::integral_constant<int, 1>{}, d1, d0);
  }
  if constexpr (kSliceK) {
    // K-sliced: fold the group's sum and store it as one partial.
    fold_halves(sm, acc, ch, kh, cq, kq, m);
    if (kh == 0) {
      const int lb = (nrun - 1) & 1;  // exponents of the last slice
      float* part = kPhase == kPhaseA ? p.partA + (static_cast<int64_t>(f) * p.gA + gi) * p.P * kN
                                      : p.partC + static_cast<int64_t>(gi) * p.P * kN;
      store_rows(
          sm, lb, acc, ch, cq, kq, m, [&](int row) { return part + static_cast<int64_t>(start + row) * kN; },
          [](int) { return 1.0f; });
    }
  }
}

// Sum of n partial rows [j][pair][256] (j in order) -> fp16 row * 2^e and e.
// One wave per (factor, pair) row, 4 columns per lane.
__device__ __forceinline__ void reduce_row(const float* part, int64_t stride, int n, _Float16* dst, int* dexp, int lane) {
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr int kBatch = 8;
  for (int k0 = 0; k0 < n; k0 += kBatch) {
    float4 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      v[j] = k0 + j < n ? reinterpret_cast<const float4*>(part + (k0 + j) * stride)[lane] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      s.x += v[j].x; s.y += v[j].y; s.z += v[j].z; s.w += v[j].w;
    }
  }
  const float mx = op_over(fmaxf(fmaxf(fabsf(s.x), fabsf(s.y)), fmaxf(fabsf(s.z), fabsf(s.w))), 1, kWave, OpMax{});
  const int ex = pow2_row_exponent(mx);
  half4v h;
  h[0] = static_cast<_Float16>(ldexpf(s.x, ex));
  h[1] = static_cast<_Float16>(ldexpf(s.y, ex));
  h[2] = static_cast<_Float16>(ldexpf(s.z, ex));
  h[3] = static_cast<_Float16>(ldexpf(s.w, ex));
  reinterpret_cast<half4v*>(dst)[lane] = h;
  if (lane == 0) *dexp = ex;
}

// lat[f][pair] = sum over the K groups of partA[f][g][pair], in group order.
__global__ void __launch_bounds__(kT) reduce_a_kernel(Params p) {
  const int routed = p.g.meta[3];
  const int lane = threadIdx.x & (kWave - 1);
  for (int64_t row = blockIdx.x * (kT / kWave) + (threadIdx.x >> 6); row < 2LL * routed;
       row += static_cast<int64_t>(gridDim.x) * (kT / kWave)) {
    const int64_t f = row / routed, pair = row - f * routed;
    reduce_row(p.partA + (f * p.gA * p.P + pair) * kN, static_cast<int64_t>(p.P) * kN, p.gA,
               p.lath + (f * p.P + pair) * kN, p.lexp + f * p.P + pair, lane);
  }
}

// dlat[pair] = sum over the K groups of partC[g][pair], in group order.
__global__ void __launch_bounds__(kT) reduce_c_kernel(Params p) {
  const int routed = p.g.meta[3];
  const int lane = threadIdx.x & (kWave - 1);
  for (int64_t pair = blockIdx.x * (kT / kWave) + (threadIdx.x >> 6); pair < routed;
       pair += static_cast<int64_t>(gridDim.x) * (kT / kWave))
    reduce_row(p.partC + pair * kN, static_cast<int64_t>(p.P) * kN, p.gC, p.dlath + pair * kN, p.dexp + pair, lane);
}

constexpr int kSumBatch = 8;

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
      for (int j = 0; j < kSumBatch; ++j) {
        s.x += v[j].x; s.y += v[j].y; s.z += v[j].z; s.w += v[j].w;
      }
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
         a.n_expert <= 4096 && a.n_embd <= (1 << 16) && a.n_ff <= (1 << 16);
}

int64_t max_units(int64_t pairs, int64_t experts) { return std::min(pairs, experts) + pairs / kMaxM; }

// Slices per workgroup for a phase with `per_unit` slices in each of `units`
// units: about four rounds of the 512 workgroups resident on the chip.
static int pick_nb(int64_t units, int64_t per_unit) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kMaxNB, units * per_unit / 2048)));
}

struct Split {
  int nb[4], gA, gB, gC, gD;
};

static Split split_for(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  const int64_t U = max_units(P, a.n_expert);
  const int nks = static_cast<int>(a.n_embd / kK), nbs = static_cast<int>(a.n_ff / kN);
  const int nkc = static_cast<int>(a.n_ff / kK), nds = static_cast<int>(a.n_embd / kN);
  Split s{};
  s.nb[kPhaseA] = pick_nb(U, 2 * nks);
  s.nb[kPhaseB] = std::max(1, pick_nb(U, 2 * nbs) / 2);  // each B slice is a gate and an up run
  s.nb[kPhaseC] = pick_nb(U, nkc);
  s.nb[kPhaseD] = pick_nb(U, nds);
  s.gA = (nks + s.nb[kPhaseA] - 1) / s.nb[kPhaseA];
  s.gB = (nbs + s.nb[kPhaseB] - 1) / s.nb[kPhaseB];
  s.gC = (nkc + s.nb[kPhaseC] - 1) / s.nb[kPhaseC];
  s.gD = (nds + s.nb[kPhaseD] - 1) / s.nb[kPhaseD];
  return s;
}

Layout layout_for(const latent_moe_args& a) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const int64_t T = a.n_tokens, P = a.n_tokens * a.n_expert_used, d = a.n_embd, ff = a.n_ff;
  const Split sp = split_for(a);
  Layout L{};
  size_t off = 0;
  L.xh = off;    off = al(off + static_cast<size_t>(T) * d * 2);
  L.xexp = off;  off = al(off + static_cast<size_t>(T) * 4);
  L.partA = off; off = al(off + 2ull * sp.gA * P * kN * 4);
  L.lath = off;  off = al(off + 2ull * P * kN * 2);
  L.lexp = off;  off = al(off + 2ull * P * 4);
  L.hh = off;    off = al(off + static_cast<size_t>(P) * ff * 2);
  L.hexp = off;  off = al(off + static_cast<size_t>(P) * (ff / kN) * 4);
  L.partC = off; off = al(off + static_cast<size_t>(sp.gC) * P * kN * 4);
  L.dlath = off; off = al(off + static_cast<size_t>(P) * kN * 2);
  L.dexp = off;  off = al(off + static_cast<size_t>(P) * 4);
  L.ybuf = off;  off = al(off + static_cast<size_t>(P) * d * 4);
  L.total = off;
  return L;
}

int forward(const latent_moe_args& a, const Factor* fac, const Grouping& g, char* scratch, hipStream_t s) {
  const Layout L = layout_for(a);
  const Split sp = split_for(a);
  Params p{};
  for (int i = 0; i < 6; ++i) p.fac[i] = fac[i];
  p.g = g;
  p.ids = a.ids;
  p.out = static_cast<float*>(a.out);
  p.xh = reinterpret_cast<const _Float16*>(scratch + L.xh);
  p.xexp = reinterpret_cast<const int*>(scratch + L.xexp);
  p.partA = reinterpret_cast<float*>(scratch + L.partA);
  p.lath = reinterpret_cast<_Float16*>(scratch + L.lath);
  p.lexp = reinterpret_cast<int*>(scratch + L.lexp);
  p.hh = reinterpret_cast<_Float16*>(scratch + L.hh);
  p.hexp = reinterpret_cast<int*>(scratch + L.hexp);
  p.partC = reinterpret_cast<float*>(scratch + L.partC);
  p.dlath = reinterpret_cast<_Float16*>(scratch + L.dlath);
  p.dexp = reinterpret_cast<int*>(scratch + L.dexp);
  p.ybuf = reinterpret_cast<float*>(scratch + L.ybuf);
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
  for (int i = 0; i < 4; ++i) p.nb[i] = sp.nb[i];
  p.gA = sp.gA;
  p.gB = sp.gB;
  p.gC = sp.gC;
  p.gD = sp.gD;
  const unsigned U = static_cast<unsigned>(max_units(p.P, a.n_expert));
  p.umax = static_cast<int>(U);
  auto blocks = [](int64_t n) { return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(2048, n))); };
  // Workgroup b takes unit (b mod 8) + 8 (b / 8 / groups) and that unit's
  // group (b / 8) mod groups: 8 * ceil(U / 8) * groups workgroups.
  auto item_grid = [&](int64_t groups) { return static_cast<unsigned>(8 * ((U + 7) / 8) * groups); };
  const int rows_per_block = kT / kWave;
  hipLaunchKernelGGL(item_kernel<kPhaseA>, dim3(item_grid(2 * p.gA)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(reduce_a_kernel, dim3(blocks((2LL * p.P + rows_per_block - 1) / rows_per_block)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseB>, dim3(item_grid(p.gB)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseC>, dim3(item_grid(p.gC)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(reduce_c_kernel, dim3(blocks((static_cast<int64_t>(p.P) + rows_per_block - 1) / rows_per_block)),
                     dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseD>, dim3(item_grid(p.gD)), dim3(kT), 0, s, p);
  if (a.out_mode == LATENT_OUT_REDUCED)
    hipLaunchKernelGGL(combine_kernel, dim3(blocks((static_cast<int64_t>(p.T) * p.d / 4 + kT - 1) / kT)), dim3(kT), 0, s,
                       p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace stream
}  // namespace latent
