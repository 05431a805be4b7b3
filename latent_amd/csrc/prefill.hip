// Grouped-MFMA prefill path: the LATENT factor chain as four grouped GEMMs over
// the expert-sorted (token, slot) pairs.
//
// Replaces, for prefill-sized batches, the per-token launch loop of
// kernels/latent_fused_expert_ffn.cu:255-289; restates project /
// swiglu_expert (loader/latent_runtime.py:35-59) per expert:
//
//   A    gu[p]  = x[tok(p)] . [A_g | A_u]                 K = d,  N = 2R
//   BC1  h[p]   = SiLU(gu[p][:R] . B_g) * (gu[p][R:] . B_u)  K = R,  N = ff
//   BC2  dl[p]  = h[p] . A_d                               K = ff, N = R
//   D    y[p]   = dl[p] . B_d                              K = R,  N = d
//   out[t] = sum over the token's slots of w * y (reduced), or y per slot
//
// BC1 runs as two GEMMs: SiLU of the gate product is stored (fp16, exponent
// blocks) into the h buffer, and the up GEMM's epilogue reads it back in place
// and stores h = SiLU(g) * u.
//
// A workgroup (4 waves) owns one M tile of up to 128 pairs of one expert and a
// run of column tiles.  Per 32-row K slice it dequantizes 256 factor columns
// (two halves of 128; NF4 level in fp16 times the group scale, packed fp16)
// into LDS as [column][k] and multiplies them on v_mfma_f32_32x32x16_f16 with
// fp32 accumulation; each wave owns 64 pairs x 128 columns, one exponent
// block of the output.  Activation rows, NF4
// codes and scales reach LDS by direct global->LDS loads through a ring of
// kStages slices, so the next slices are in flight while one is decoded and
// another multiplied; the ring runs on across the column tiles of a work item.
// Intermediates (gu, h, dl, y) are stored in fp16 per pair; a per-token
// combine kernel sums the weighted slot rows in slot order (reduced mode), or
// the last GEMM stores fp32 rows per slot.
//
// fp16 range: the latents of a LATENT chain are small (about 1e-3 .. 1e-9 at
// the DeepSeek-V3 shape), far below fp16's normal range.  Every fp16 operand
// row therefore carries a power-of-two exponent: a producer tile stores
// v * 2^e with e chosen per (row, 128-column block) so that the block's
// largest |v| lands in [2^14, 2^15), and records e; a consumer rescales each
// block of its row to the row's smallest exponent c (exact ldexp on fp16) and
// multiplies its fp32 accumulators by 2^-c.  x is converted once per call to
// fp16 rows scaled the same way (one exponent per token).  Scaling by powers
// of two adds no rounding.
#include "prefill.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "stream.hpp"

namespace latent {
namespace prefill {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;   // 4 waves: 2 row halves x 2 column halves of a tile
constexpr int kMT = 128;        // pairs per tile
constexpr int kHalf = 128;      // factor columns per decoded half
constexpr int kNT = 2 * kHalf;  // decoded columns per K slice
constexpr int kKS = 32;         // K rows per slice
constexpr int kBlk = 128;       // columns per exponent block of an intermediate row
constexpr int kStages = 3;      // raw K slices in the load ring
constexpr int kMaxBlocks = 16;  // exponent blocks in one K range (K <= 2048)
constexpr int kTileThreads = 1024;
constexpr int kExpMin = -120, kExpMax = 120;

enum ASrc { kFromX = 0, kFromPairs = 1 };
// kStoreSiLU stores SiLU of the product; kSwiGLU multiplies the product into
// what dst holds on entry (SiLU of the gate product) and stores the result.
enum Epi { kStoreHalf = 0, kSwiGLU = 1, kToOutput = 2, kStoreSiLU = 3 };

struct Params {
  Grouping g;
  const int* tile_a;
  const int* tile_r0;
  const _Float16* xh;  // kFromX: scaled fp16 x [T][d], row tok(p)
  int d;
  const _Float16* a;  // kFromPairs: a[p * lda + col], scaled by 2^a_exp[p][col / kBlk]
  int64_t lda;
  int a_col;           // first A column read
  const int* a_exp;    // kFromPairs: [P][a_exp_ld] block exponents; kFromX: [T] row exponents of x
  int a_exp_ld;
  int K;
  Factor f0, f1;  // the output columns are [f0 | f1] (nfac factors)
  int ncols;      // columns of one factor, a multiple of kHalf
  int nfac;       // 1 or 2
  int nsub;       // column tiles (kNT output columns) per M tile
  int spc;        // column tiles per work item
  _Float16* dst;  // kStoreHalf / kSwiGLU: dst[p * ldd + col]
  int64_t ldd;
  int* dst_exp;  // [P][dst_exp_ld] exponents of the stored blocks
  int dst_exp_ld;
  float* out;  // kToOutput: per-slot rows out[(tok * k + slot) * ncols + col]
  int wbd, n_expert_used;
};

// LDS placements, free of bank conflicts for the access patterns below (64
// lanes against 32 or 64 banks of 4 bytes):
//   activation chunk c (8 halfs) of tile row r  -> 16-byte slot r*4 + (c ^ a_swz(r))
//   decoded chunk c (8 k) of column n            -> 16-byte slot n*4 + (c ^ b_swz(n))
//   NF4 code row r of a half                     -> 64-byte slot r ^ ((r >> 2) & 3),
//     its 16-byte segment s                      -> position s ^ ((r >> 3) & 3)
__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
__device__ __forceinline__ int b_swz(int n) { return ((n >> 1) ^ (n >> 2)) & 3; }

// One raw K slice: the activation slice, the codes of both decoded halves,
// and their scales as [32 rows][4 groups] fp16; scale[2], scale[3] receive the
// balancing loads that keep every wave's direct-load count per slice equal.
struct alignas(16) Stage {
  _Float16 a[kMT * kKS];
  uint32_t code[2][kKS * kHalf / 8];
  uint32_t scale[4][kKS * kHalf / kGroup / 2];
};

struct alignas(16) Decoded {
  _Float16 b[kNT * kKS];
};

template <bool kShift>
struct Smem {
  uint32_t lut2[256];  // entry a | b << 4: half2(level a, level b) (two K rows of one column)
  int cexp[kMT];                                     // row exponent of each operand row
  int8_t shift[kShift ? kMT : 1][kMaxBlocks];        // per-block change to reach cexp
  int tok[kMT];
  int slot[kMT];
  float w[kMT];
  int dro[kMT];  // (p0 + row) * ldd: output row offsets
  int dxo[kMT];  // (p0 + row) * dst_exp_ld: exponent row offsets
};

// Direct global -> LDS loads: lane l's 16 (4) bytes land at LDS byte address
// lds + 16 l (4 l); lds is wave-uniform.  Inline assembly, so that the
// compiler does not make every later LDS read wait for them (vmcnt(0)); the
// pipeline waits for them itself (slice_barrier).  The scalar-base forms take
// a 32-bit lane offset.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "m0");
}
// A wave-uniform 64-bit address in scalar registers (the scalar-base forms
// need it there).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(lds)
               : "m0");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(uniform_ptr(base)),
               "s"(lds)
               : "m0");
}

// LDS access by byte address.
template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr));
}

// LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T& obj) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)(&obj)));
}

// Workgroup barrier of the slice pipeline: each wave waits until at most n of
// its direct loads are in flight and its LDS accesses are done (s_waitcnt
// vmcnt(n) lgkmcnt(0)), then meets the others.  __syncthreads() would wait for
// every direct load.  The signal fences keep the compiler from moving LDS
// accesses across it.
template <int kN>
__device__ __forceinline__ void slice_barrier() {
  static_assert(kN >= 0 && kN < 16, "vmcnt field");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0070 | kN);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Barrier for LDS data only; direct loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// SiLU with the hardware exp2 and reciprocal (relative error near 1e-7, far
// below the fp16 storage of h); exp overflow gives g * 0 for very negative g.
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// Exponent e with m * 2^e in [2^14, 2^15) (0 for m == 0 or not finite).
__device__ __forceinline__ int block_exponent(float m) {
  if (!(m > 0.f) || !(m < 3.0e38f)) return 0;
  const int ilog = static_cast<int>((__float_as_uint(m) >> 23) & 0xFFu) - 127;  // floor(log2 m), normal m
  return min(kExpMax, max(kExpMin, 14 - ilog));
}

// Maximum over the 32 lanes that hold one row of an MFMA result (lanes l and
// l ^ 32 hold different rows).
__device__ __forceinline__ float max32(float m) { return op_over(m, 1, 32, OpMax{}); }

template <int kA, int kEpi>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(Params p) {
  constexpr bool kShift = kA == kFromPairs;
  constexpr int kDma = 4;  // direct loads per wave per slice
  __shared__ Smem<kShift> s;
  __shared__ Stage ring[kStages];
  __shared__ Decoded dec[2];

  // Work items (M tile, run of column tiles) in expert order, cut into 8
  // contiguous runs, one per XCD (workgroup b runs on XCD b % 8): a tile's
  // column runs share its activation rows, an expert's tiles share its factor
  // slices, both in one L2.
  const int nchunk = (p.nsub + p.spc - 1) / p.spc;
  const int total_items = p.g.meta[2] * nchunk;
  const int per_xcd = (total_items + 7) / 8;
  const int jb = blockIdx.x >> 3, item = (blockIdx.x & 7) * per_xcd + jb;
  if (jb >= per_xcd || item >= total_items) return;
  const int tile = item / nchunk, chunk = item - tile * nchunk;
  const int u0 = chunk * p.spc, nu = min(p.spc, p.nsub - u0);
  const int ta = p.tile_a[tile], r0 = p.tile_r0[tile];
  const int rows = min(kMT, p.g.act_count[ta] - r0);
  const int p0 = p.g.act_start[ta] + r0;
  const int64_t e = p.g.act_expert[ta];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w & 1, wn = w >> 1;

  {
    half2v v;
    v[0] = static_cast<_Float16>(nf4_level(tid & 15));
    v[1] = static_cast<_Float16>(nf4_level(tid >> 4));
    s.lut2[tid] = __builtin_bit_cast(uint32_t, v);
  }
  static_assert(kThreads == 256, "one level-pair entry per thread");
  if (tid < kMT) {
    const bool ok = tid < rows;
    s.tok[tid] = ok ? p.g.pair_tok[p0 + tid] : 0;
    s.slot[tid] = ok ? p.g.pair_slot[p0 + tid] : 0;
    s.w[tid] = ok ? p.g.pair_w[p0 + tid] : 0.f;
    s.dro[tid] = static_cast<int>((p0 + tid) * p.ldd);
    s.dxo[tid] = (p0 + tid) * p.dst_exp_ld;
    // Operand row exponents: x rows carry one; intermediate rows are rescaled
    // to the smallest block exponent over the K range they are read in.
    int c = 0;
    if constexpr (kA == kFromX) {
      if (ok) c = p.a_exp[s.tok[tid]];
    } else {
      const int nb = p.K / kBlk;
      if (ok) {
        const int* ex = p.a_exp + static_cast<int64_t>(p0 + tid) * p.a_exp_ld + p.a_col / kBlk;
        c = kExpMax;
        for (int b = 0; b < nb; ++b) c = min(c, ex[b]);
        for (int b = 0; b < nb; ++b) s.shift[tid][b] = static_cast<int8_t>(max(-128, c - ex[b]));
      } else {
        for (int b = 0; b < nb; ++b) s.shift[tid][b] = 0;
      }
    }
    s.cexp[tid] = c;
  }
  __syncthreads();

  // ---- direct-load sources (per lane) ----
  const int nk = p.K / kKS;   // K slices per column tile (a multiple of 4)
  const int total = nu * nk;  // slices of this item
  const char* asrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int qp = (2 * w + i) * 64 + lane;  // 16-byte slot
    const int r = qp >> 2, c = (qp & 3) ^ a_swz(r);
    const int rr = r < rows ? r : 0;  // pad rows re-read row 0 (finite; never stored)
    asrc[i] = kA == kFromX
                  ? reinterpret_cast<const char*>(p.xh + static_cast<int64_t>(s.tok[rr]) * p.d + 8 * c)
                  : reinterpret_cast<const char*>(p.a + static_cast<int64_t>(p0 + rr) * p.lda + p.a_col + 8 * c);
  }
  const int hw = w >> 1;  // the half whose codes and scales this wave loads and decodes
  const uint32_t cstride = static_cast<uint32_t>(p.ncols / 2), sstride = static_cast<uint32_t>(p.ncols / kGroup) * 2;
  uint32_t code_off, scale_off;
  {
    const int sg = (w & 1) * 64 + lane;  // 16-byte segment of the half slice
    const int rs = sg >> 2, r = rs ^ ((rs >> 2) & 3), seg = (sg & 3) ^ ((r >> 3) & 3);
    code_off = r * cstride + 16 * seg;
    scale_off = (lane >> 1) * sstride + 4 * (lane & 1);
  }
  const int64_t cstep = static_cast<int64_t>(kKS) * cstride, sstep = static_cast<int64_t>(kKS) * sstride;
  // Source of this wave's half of the item's first slice.  Column tiles of an
  // item are adjacent tiles of one factor (the host sets one tile per item
  // when the output columns span two factors or end in a half tile), so the
  // next tile starts kNT / 2 code bytes to the right.
  const char* cptr;
  const char* sptr;
  {
    int v = u0 * kNT + hw * kHalf;
    v = v >= p.nfac * p.ncols ? u0 * kNT : v;  // empty half: load the first (never stored)
    const bool second = v >= p.ncols;
    const Factor& f = second ? p.f1 : p.f0;
    const int col = second ? v - p.ncols : v;
    cptr = reinterpret_cast<const char*>(f.codes) + e * f.rows * cstride + col / 2;
    sptr = reinterpret_cast<const char*>(f.scales) + e * f.rows * sstride + (col / kGroup) * 2;
  }
  const int64_t cwrap = kNT / 2 - (nk - 1) * cstep, swrap = (kNT / kGroup) * 2 - (nk - 1) * sstep;
  int ik = 0, aoff = 0, left = total;  // K slice of the next issue, its activation byte offset, slices to issue
  const uint32_t ring_lds = lds_addr(ring[0]);
  // Every step issues exactly one slice (uniform vmcnt bookkeeping, no
  // branches in the step): past the item's last slice, that slice is loaded
  // again into the free stage and never used.  Scalar selects only.
  auto issue = [&](int stg) __attribute__((always_inline)) {
    const uint32_t base = ring_lds + stg * static_cast<uint32_t>(sizeof(Stage));
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(asrc[i] + aoff, base + offsetof(Stage, a) + (2 * w + i) * 1024);
    dma16s(cptr, code_off, base + offsetof(Stage, code) + (hw * 512 + (w & 1) * 256) * 4);
    dma4s(sptr, scale_off, base + offsetof(Stage, scale) + (hw + 2 * (w & 1)) * 256);
    const bool adv = --left > 0;
    const bool wrap = ++ik == nk;
    ik = wrap ? 0 : ik;
    cptr += adv ? (wrap ? cwrap : cstep) : 0;
    sptr += adv ? (wrap ? swrap : sstep) : 0;
    aoff = adv ? (wrap ? 0 : aoff + kKS * 2) : aoff;
  };

  // ---- decode (per thread: K rows 4kq .. 4kq+3, factor columns 8cg .. 8cg+7) ----
  // Decoded column n of a half holds factor column 4 (n % 32) + n / 32 of it,
  // so that the 4 accumulators of a lane for one row are 4 adjacent output
  // columns.  The thread mapping and the rotation rot of the write order keep
  // the code reads and decoded writes free of bank conflicts.
  const int kq = (tid & 1) | (((tid >> 5) & 1) << 1) | (((tid >> 1) & 1) << 2);
  const int cg = ((tid >> 2) & 7) | ((tid >> 6) << 3), wd = cg & 15, seg = wd >> 2, rot = kq;
  uint32_t code_word[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) code_word[i] = (4 * kq + (i ^ (kq & 3))) * 16 + 4 * (seg ^ ((kq >> 1) & 3)) + (wd & 3);
  uint32_t woff[8];  // byte offset of factor column 8cg + ((j + rot) & 7), k 4kq .. 4kq+3
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int fc = 8 * wd + ((j + rot) & 7);                 // factor column in the half
    const int n = kHalf * (cg >> 4) + 32 * (fc & 3) + (fc >> 2);  // its decoded column
    woff[j] = n * 64 + 16 * ((kq >> 1) ^ b_swz(n)) + 8 * (kq & 1);
  }
  // Ring stages are addressed through a base taken with readfirstlane, opaque
  // to the compiler: with a visible stage index it keeps a copy of every
  // per-lane address for each of the kStages stages in registers.
  uint32_t code_addr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) code_addr[i] = ring_lds + offsetof(Stage, code) + hw * 2048 + code_word[i] * 4;
  const uint32_t scale_addr = ring_lds + offsetof(Stage, scale) + hw * 256 + ((4 * kq) * 4 + seg) * 2;
  auto stage_off = [&](int stg) __attribute__((always_inline)) {
    return __builtin_amdgcn_readfirstlane(stg * static_cast<uint32_t>(sizeof(Stage)));
  };
  auto prepare = [&](int stg, int db) __attribute__((always_inline)) {
    const uint32_t so = stage_off(stg);
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = lds_ld<uint32_t>(code_addr[i] + so);
    half2v s01, s23;
    s01[0] = lds_ld<_Float16>(scale_addr + so);
    s01[1] = lds_ld<_Float16>(scale_addr + so + 8);
    s23[0] = lds_ld<_Float16>(scale_addr + so + 16);
    s23[1] = lds_ld<_Float16>(scale_addr + so + 24);
    // Code pairs of K rows (4kq, 4kq+1) and (4kq+2, 4kq+3): per byte, the
    // nibble of the first row | the nibble of the second row << 4, the index
    // of the level pair; even columns in ev, odd columns in od.
    uint32_t ev[2], od[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t a = __builtin_amdgcn_alignbit(c[2 * q], c[2 * q], 4 * rot);  // nibble j <- column (j + rot) & 7
      const uint32_t b = __builtin_amdgcn_alignbit(c[2 * q + 1], c[2 * q + 1], 4 * rot);
      ev[q] = (a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u);
      od[q] = ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u);
    }
    char* D = reinterpret_cast<char*>(dec[db].b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sh = 8 * (j >> 1);
      const uint32_t* src = (j & 1) ? od : ev;
      half2v v01 = __builtin_bit_cast(half2v, s.lut2[(src[0] >> sh) & 0xFFu]);
      half2v v23 = __builtin_bit_cast(half2v, s.lut2[(src[1] >> sh) & 0xFFu]);
      v01 *= s01;
      v23 *= s23;
      uint2 o;
      o.x = __builtin_bit_cast(uint32_t, v01);
      o.y = __builtin_bit_cast(uint32_t, v23);
      *reinterpret_cast<uint2*>(D + woff[j]) = o;
    }
  };

  // ---- multiply ----
  f32x16 acc[2][4];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  };
  zero_acc();
  half2v amul[2];  // 2^shift of the lane's A rows for the current exponent block
#pragma unroll
  for (int i = 0; i < 2; ++i) amul[i] = half2v{1.f, 1.f};
  uint32_t a_addr[2][2];  // [ks / 16][i]
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 64 * wm + 32 * i + (lane & 31), c = 2 * k2 + (lane >> 5);
      a_addr[k2][i] = ring_lds + offsetof(Stage, a) + (r * 4 + (c ^ a_swz(r))) * 16;
    }
  // Fragments of one slice: A rows (2 row blocks) and decoded B columns (4
  // column blocks) for both 16-deep K steps.
  half8 af[2][2], bf[2][4];
  auto load_frags = [&](int stg, int db) __attribute__((always_inline)) {
    const uint32_t so = stage_off(stg);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int c = 2 * k2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[k2][i] = lds_ld<half8>(a_addr[k2][i] + so);
        if constexpr (kShift) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            half2v v{af[k2][i][2 * t], af[k2][i][2 * t + 1]};
            v *= amul[i];
            af[k2][i][2 * t] = v[0];
            af[k2][i][2 * t + 1] = v[1];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = kHalf * wn + 32 * j + (lane & 31);
        bf[k2][j] = *reinterpret_cast<const half8*>(&dec[db].b[(n * 4 + (c ^ b_swz(n))) * 8]);
      }
    }
  };
  auto run_mfma = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[k2][i], bf[k2][j], acc[i][j], 0, 0, 0);
  };

  // ---- epilogue of column tile ut: this wave's 64 rows x 128 columns ----
  auto epilogue = [&](int ut) __attribute__((always_inline)) {
    const int vcol = ut * kNT + wn * kHalf;  // first output column of this wave
    if (vcol >= p.nfac * p.ncols) return;    // empty half
    // The lane index, opaque to the compiler, so that the epilogue's row
    // addresses are formed here instead of being hoisted out of the K loop
    // into registers the loop needs.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    auto row_of = [&](int i, int r) __attribute__((always_inline)) {
      return 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
    };
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ce = s.cexp[row_of(i, r)];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j][r] = __builtin_ldexpf(acc[i][j][r], -ce);
      }
    if constexpr (kEpi == kToOutput) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row_of(i, r);
          if (row >= rows) continue;
          float* o = p.out + (static_cast<int64_t>(s.tok[row]) * p.n_expert_used + s.slot[row]) * p.ncols + vcol +
                     4 * (ln & 31);
          *reinterpret_cast<float4*>(o) = make_float4(acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]);
        }
      return;
    }
    const int blk = vcol / kBlk;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (kEpi == kStoreSiLU) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j][r] = silu_f32(acc[i][j][r]);
      }
      if constexpr (kEpi == kSwiGLU) {
        // dst holds SiLU(g) * 2^sexp in fp16.  Loads of 8 rows first (pad rows read row 0).
#pragma unroll
        for (int r0 = 0; r0 < 16; r0 += 8) {
          uint2 gw[8];
          int gx[8];
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const int row = row_of(i, r0 + r), rr = row < rows ? row : 0;
            gw[r] = *reinterpret_cast<const uint2*>(p.dst + s.dro[rr] + vcol + 4 * (ln & 31));
            gx[r] = p.dst_exp[s.dxo[rr] + blk];
          }
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const float wr = __builtin_ldexpf(p.wbd ? s.w[row_of(i, r0 + r)] : 1.f, -gx[r]);
            const uint32_t q[4] = {gw[r].x & 0xFFFFu, gw[r].x >> 16, gw[r].y & 0xFFFFu, gw[r].y >> 16};
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j][r0 + r] *= half_bits_to_float(static_cast<uint16_t>(q[j])) * wr;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) m = fmaxf(m, fabsf(acc[i][j][r]));
        m = max32(m);
        const int row = row_of(i, r);
        if (row >= rows) continue;
        const int ex = block_exponent(m);
        half2v h01, h23;
        h01[0] = static_cast<_Float16>(__builtin_ldexpf(acc[i][0][r], ex));
        h01[1] = static_cast<_Float16>(__builtin_ldexpf(acc[i][1][r], ex));
        h23[0] = static_cast<_Float16>(__builtin_ldexpf(acc[i][2][r], ex));
        h23[1] = static_cast<_Float16>(__builtin_ldexpf(acc[i][3][r], ex));
        *reinterpret_cast<uint2*>(p.dst + s.dro[row] + vcol + 4 * (ln & 31)) =
            make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
        if ((ln & 31) == 0) p.dst_exp[s.dxo[row] + blk] = ex;
      }
    }
  };

  // ---- pipeline ----
  // Step s: wait until slice s + 1 has landed (and every wave is done with
  // step s - 1), refill the stage slice s - 1 used with slice s + kAhead,
  // multiply slice s while decoding slice s + 1 into the free decode buffer.
  constexpr int kAhead = kStages - 1;  // slices issued ahead of the one multiplied
  static_assert((kAhead - 2) * kDma < 16, "vmcnt field");
#pragma unroll
  for (int i = 0; i < kAhead; ++i) issue(i);
  slice_barrier<(kAhead - 1) * kDma>();  // slice 0 landed
  prepare(0, 0);
  auto next_stage = [](int x) __attribute__((always_inline)) { return x + 1 == kStages ? 0 : x + 1; };
  int st_mul = 0, st_prep = 1 % kStages, st_issue = kAhead % kStages;  // ring stages of slices sl, sl + 1, sl + kAhead
  int kk0 = 0;  // K slice of the group's first step
  for (int s0 = 0; s0 < total; s0 += 4) {
    if constexpr (kShift) {
      // One exponent block per 4 slices (kBlk = 4 * kKS; operand columns start on a block).
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int sft = s.shift[64 * wm + 32 * i + (lane & 31)][kk0 >> 2];
        const _Float16 m = sft < -24 ? static_cast<_Float16>(0.f) : static_cast<_Float16>(__builtin_ldexpf(1.f, sft));
        amul[i] = half2v{m, m};
      }
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      // Issued so far: slices 0 .. sl + kAhead - 1 (sl = s0 + I); slice sl + 1 must land.
      slice_barrier<(kAhead - 2) * kDma>();
      issue(st_issue);
      load_frags(st_mul, I & 1);
      run_mfma();
      prepare(st_prep, (I + 1) & 1);  // past the last slice: decodes a stage never used
      st_mul = next_stage(st_mul);
      st_prep = next_stage(st_prep);
      st_issue = next_stage(st_issue);
      // Interleave the decode of slice sl + 1 with the 16 MFMAs of slice sl.
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
      }
    }
    kk0 += 4;
    if (kk0 == nk) {
      epilogue(u0 + s0 / nk);
      zero_acc();
      kk0 = 0;
    }
  }
  // Past-the-end loads must land before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0070);
}

// x rows to fp16: xh[t] = fp16(x[t] * 2^e[t]) with 2^e * max|x[t]| in [2^14, 2^15).
// One wave per token, four tokens per workgroup: no barrier, and every
// token of a 4096-token call is resident at once (a workgroup per token,
// with two barriers around the maximum, ran in two residency rounds).  Lane
// l holds the 8-element chunks l, l + 64, ... of the row (raw, up to
// kXPrepChunks of them: rows of up to 8192 elements are read once; longer
// rows twice); d % 8 == 0 and x 16-byte aligned.
// Also clears the token's slot entries of pos_of and, when per_slot_out is
// given (per-slot output mode), writes the zero rows of the token's dropped
// slots (id outside [0, E)): the GEMMs write routed rows only.
constexpr int kXPrepChunks = 16;
template <bool kF32>
__global__ void __launch_bounds__(kThreads) x_prep_kernel(const void* x, int x_dtype, int T, int d, _Float16* xh,
                                                          int* xexp, int* pos_of, int k, const int32_t* ids, int E,
                                                          float* per_slot_out) {
  constexpr int kW = kF32 ? 2 : 1;  // 16-byte words per chunk of 8 elements
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * (kThreads / kWave) + static_cast<int>(threadIdx.x >> 6);
  if (t >= T) return;
  for (int sl = lane; sl < k; sl += kWave) pos_of[static_cast<int64_t>(t) * k + sl] = -1;
  if (per_slot_out) {
    for (int sl = 0; sl < k; ++sl) {
      const int e = ids[static_cast<int64_t>(t) * k + sl];
      if (e >= 0 && e < E) continue;
      float4* row = reinterpret_cast<float4*>(per_slot_out + (static_cast<int64_t>(t) * k + sl) * d);
      for (int c = lane; c < d / 4; c += kWave) row[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const int64_t base = static_cast<int64_t>(t) * d;
  auto load = [&](int c, uint4 (&r)[kW]) __attribute__((always_inline)) {
    if constexpr (kF32) {
      const uint4* q = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + base + c * 8);
      r[0] = q[0];
      r[kW - 1] = q[1];
    } else {
      r[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base + c * 8);
    }
  };
  auto vals = [&](const uint4 (&r)[kW], float (&v)[8]) __attribute__((always_inline)) {
    if constexpr (kF32) {
      const uint32_t w[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[kW - 1].x, r[kW - 1].y, r[kW - 1].z, r[kW - 1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
    } else {
      const uint32_t w[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (x_dtype == LATENT_BF16) {
          v[2 * i] = __uint_as_float(w[i] << 16);
          v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        } else {
          v[2 * i] = half_bits_to_float(static_cast<uint16_t>(w[i] & 0xFFFFu));
          v[2 * i + 1] = half_bits_to_float(static_cast<uint16_t>(w[i] >> 16));
        }
      }
    }
  };
  const int nc = d / 8;
  const bool cached = nc <= kXPrepChunks * kWave;
  uint4 raw[kXPrepChunks][kW];
  float m = 0.f;
  if (cached) {
#pragma unroll
    for (int r = 0; r < kXPrepChunks; ++r)
      if (lane + r * kWave < nc) load(lane + r * kWave, raw[r]);
#pragma unroll
    for (int r = 0; r < kXPrepChunks; ++r) {
      if (lane + r * kWave < nc) {
        float v[8];
        vals(raw[r], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
      }
    }
  } else {
    for (int c = lane; c < nc; c += kWave) {
      uint4 rr[kW];
      float v[8];
      load(c, rr);
      vals(rr, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
  }
  const int e = block_exponent(op_over(m, 1, kWave, OpMax{}));
  if (lane == 0) xexp[t] = e;
  auto store = [&](int c, const float (&v)[8]) __attribute__((always_inline)) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(__builtin_ldexpf(v[i], e));
    *reinterpret_cast<half8*>(xh + base + c * 8) = h;
  };
  if (cached) {
#pragma unroll
    for (int r = 0; r < kXPrepChunks; ++r) {
      if (lane + r * kWave < nc) {
        float v[8];
        vals(raw[r], v);
        store(lane + r * kWave, v);
      }
    }
    return;
  }
  for (int c = lane; c < nc; c += kWave) {
    uint4 rr[kW];
    float v[8];
    load(c, rr);
    vals(rr, v);
    store(c, v);
  }
}


// out[t] = sum over slots (in slot order) of w * y[pos_of[t][slot]] * 2^-exp,
// y rows in fp16 with one exponent per 2^blk_log2 columns (row stride
// yexp_ld).  One workgroup per token.  The token's grouped positions and
// weights are read once into LDS (the output stores could alias them, so
// they would otherwise be reloaded for every column chunk); then each thread
// takes 8-column chunks tid, tid + 256, ... two at a time, with the y rows and
// exponents of both chunks and kCombineSlots slots loaded before any is
// added (32 loads in flight per thread).  k <= kCombineMaxK.
constexpr int kCombineSlots = 8;
constexpr int kCombineMaxK = 64;
constexpr int kCombineChunks = 2;
__global__ void __launch_bounds__(kThreads) combine_kernel(const _Float16* y, const int* yexp, int yexp_ld, int blk_log2,
                                                           const int* pos_of, const float* pair_w, int k, int d, int wbd,
                                                           float* out) {
  __shared__ int spos[kCombineMaxK];
  __shared__ float sw[kCombineMaxK];
  const int t = blockIdx.x, tid = threadIdx.x;
  if (tid < k) {
    // A dropped slot (-1) adds an exact zero; its (unwritten) row is not read.
    const int pos = pos_of[t * k + tid];
    spos[tid] = pos;
    sw[tid] = pos >= 0 ? (wbd ? 1.f : pair_w[pos]) : 0.f;
  }
  __syncthreads();
  const int nc = d / 8;
  for (int c0 = tid; c0 < nc; c0 += kThreads * kCombineChunks) {
    float acc[kCombineChunks][8] = {};
    for (int s0 = 0; s0 < k; s0 += kCombineSlots) {
      half8 h[kCombineChunks][kCombineSlots];
      int ex[kCombineChunks][kCombineSlots];
#pragma unroll
      for (int i = 0; i < kCombineSlots; ++i) {
        const int sl = s0 + i;
        const int pos = sl < k ? spos[sl] : -1;
#pragma unroll
        for (int r = 0; r < kCombineChunks; ++r) {
          const int c = (c0 + r * kThreads) * 8;
          h[r][i] = half8{};
          ex[r][i] = 0;
          if (pos >= 0 && c < d) {
            h[r][i] = *reinterpret_cast<const half8*>(y + static_cast<int64_t>(pos) * d + c);
            ex[r][i] = yexp[static_cast<int64_t>(pos) * yexp_ld + (c >> blk_log2)];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kCombineSlots; ++i) {
        const float wi = s0 + i < k ? sw[s0 + i] : 0.f;
#pragma unroll
        for (int r = 0; r < kCombineChunks; ++r) {
          const float w = __builtin_ldexpf(wi, -ex[r][i]);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(w, static_cast<float>(h[r][i][j]), acc[r][j]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kCombineChunks; ++r) {
      const int c = (c0 + r * kThreads) * 8;
      if (c < d) {
        float4* o = reinterpret_cast<float4*>(out + static_cast<int64_t>(t) * d + c);
        o[0] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        o[1] = make_float4(acc[r][4], acc[r][5], acc[r][6], acc[r][7]);
      }
    }
  }
}

// Workgroup 0: M tiles of `rows` pairs (kMT for the GEMMs) for every active
// expert, in expert order; with `units`, also each tile as {expert, first
// grouped pair, pairs, 0}.  The other workgroups: pos_of[tok * k + slot] =
// pair for the routed pairs, kTileThreads pairs each (x_prep_kernel cleared
// pos_of to -1).  Both read only the grouping, so they share one launch.
__global__ void __launch_bounds__(kTileThreads) tiles_kernel(Grouping g, int rows, int* tile_a, int* tile_r0,
                                                             int4* units, int* pos_of, int P, int k) {
  __shared__ int scan[kTileThreads];
  const int tid = threadIdx.x;
  if (blockIdx.x > 0) {
    const int i = (blockIdx.x - 1) * kTileThreads + tid;
    if (i < P && i < g.meta[3]) pos_of[g.pair_tok[i] * k + g.pair_slot[i]] = i;
    return;
  }
  const int n_active = g.meta[0];
  const int per = (n_active + kTileThreads - 1) / kTileThreads;
  const int a0 = min(n_active, tid * per), a1 = min(n_active, a0 + per);
  int mine = 0;
  for (int a = a0; a < a1; ++a) mine += (g.act_count[a] + rows - 1) / rows;
  scan[tid] = mine;
  __syncthreads();
  for (int off = 1; off < kTileThreads; off <<= 1) {
    const int v = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  int t = scan[tid] - mine;
  for (int a = a0; a < a1; ++a) {
    for (int r = 0; r < g.act_count[a]; r += rows) {
      tile_a[t] = a;
      tile_r0[t] = r;
      if (units) units[t] = make_int4(g.act_expert[a], g.act_start[a] + r, min(rows, g.act_count[a] - r), 0);
      ++t;
    }
  }
  if (tid == kTileThreads - 1) g.meta[2] = scan[tid];
}


size_t align_up(size_t v) { return (v + 255) / 256 * 256; }

// A layer in the tile layout runs the streaming-tile engine; one in the row
// layout the grouped GEMMs.
bool use_bulk(const latent_moe_args& a) { return a.layout == LATENT_LAYOUT_TILES; }

// M tiles (units of the streaming-tile engine) of `rows` pairs: at most
// ceil(n_e / rows) per active expert.
int64_t max_tiles(const latent_moe_args& a, int rows) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  return (P + rows - 1) / rows + std::min<int64_t>(a.n_expert, P);
}

// Column tiles per work item: about 32 K slices of work per item, so short-K
// GEMMs keep the load ring running across several column tiles.
int tiles_per_item(int K, int nsub) { return std::max(1, std::min({nsub, 4, (32 * kKS) / K})); }

template <int kA, int kEpi>
int launch(Params p, int64_t tiles, hipStream_t s) {
  p.nsub = (p.nfac * p.ncols + kNT - 1) / kNT;
  // Several tiles per item only within one factor and whole tiles.
  p.spc = (p.nfac == 1 && p.ncols % kNT == 0) ? tiles_per_item(p.K, p.nsub) : 1;
  const int64_t items = tiles * ((p.nsub + p.spc - 1) / p.spc);
  const dim3 grid(static_cast<unsigned>(8 * ((items + 7) / 8)));
  hipLaunchKernelGGL((gemm_kernel<kA, kEpi>), grid, dim3(kThreads), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace

bool supported(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  const int64_t active = std::max<int64_t>(1, std::min<int64_t>(a.n_expert, P));
  // In the tile layout, calls beyond the decode launches' pairs come here at
  // any number of pairs per expert (the row-layout paths cannot read tiles).
  const bool beyond_decode = a.layout == LATENT_LAYOUT_TILES && P > stream::kMaxPairs;
  if (P < static_cast<int64_t>(kMinPairsPerExpert) * active && !beyond_decode) return false;
  if (a.n_expert_used > kCombineMaxK) return false;
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs)
    if (f->int8_bitmap != nullptr) return false;  // per-group INT8 layers take the general path
  if ((reinterpret_cast<uintptr_t>(a.x) & 15u) != 0) return false;
  if (a.layout == LATENT_LAYOUT_TILES) return stream::bulk_supported(a);
  // Whole 128-column halves and exponent blocks, whole 4-slice groups of K;
  // at most kMaxBlocks exponent blocks in a K range; 16-byte code rows and
  // 4-byte scale pairs for the direct loads.
  if (a.n_embd % kBlk || a.n_ff % kBlk || a.max_rank % kBlk) return false;
  if (a.n_ff > kMaxBlocks * kBlk || a.max_rank > kMaxBlocks * kBlk) return false;
  for (const latent_factor* f : fs)
    if ((reinterpret_cast<uintptr_t>(f->codes) & 15u) || (reinterpret_cast<uintptr_t>(f->scales) & 3u)) return false;
  return true;
}

Layout layout_for(const latent_moe_args& a) {
  const bool bulk = use_bulk(a);
  const int64_t P = a.n_tokens * a.n_expert_used, R = a.max_rank, T = max_tiles(a, bulk ? stream::kBulkM : kMT);
  Layout L{};
  size_t off = 0;
  L.tile_a = off;  off = align_up(off + T * sizeof(int));
  L.tile_r0 = off; off = align_up(off + T * sizeof(int));
  const int64_t rb = R / kBlk, fb = a.n_ff / kBlk, db = a.n_embd / kBlk;
  L.xexp = off;    off = align_up(off + a.n_tokens * sizeof(int));
  L.xh = off;      off = align_up(off + a.n_tokens * a.n_embd * sizeof(_Float16));
  L.gu = off;      off = align_up(off + P * 2 * R * sizeof(_Float16));
  L.gu_exp = off;  off = align_up(off + P * 2 * rb * sizeof(int));
  // The streaming-tile engine keeps finer exponent blocks: 32 h and 64 y columns.
  const int64_t hb = bulk ? a.n_ff / 32 : fb, yb = bulk ? a.n_embd / 64 : db;
  L.h = off;       off = align_up(off + P * a.n_ff * sizeof(_Float16));
  L.h_exp = off;   off = align_up(off + P * hb * sizeof(int));
  L.dl = off;      off = align_up(off + P * R * sizeof(_Float16));
  L.dl_exp = off;  off = align_up(off + P * rb * sizeof(int));
  L.pos_of = off;  off = align_up(off + P * sizeof(int));
  L.y = off;       off = align_up(off + (a.out_mode == LATENT_OUT_REDUCED ? P * a.n_embd * sizeof(_Float16) : 0));
  L.y_exp = off;   off = align_up(off + (a.out_mode == LATENT_OUT_REDUCED ? P * yb * sizeof(int) : 0));
  L.units = off;   off = align_up(off + (bulk ? T * sizeof(int4) : 0));
  L.part = off;    off = align_up(off + (bulk ? stream::bulk_part_bytes(a, T) : 0));
  L.total = off;
  return L;
}

int forward(const latent_moe_args& a, const Factor* fac, const Grouping& g, char* scratch, hipStream_t s) {
  const Layout L = layout_for(a);
  const bool bulk = use_bulk(a);
  const int64_t tiles = max_tiles(a, bulk ? stream::kBulkM : kMT);
  int* tile_a = reinterpret_cast<int*>(scratch + L.tile_a);
  int* tile_r0 = reinterpret_cast<int*>(scratch + L.tile_r0);
  _Float16* gu = reinterpret_cast<_Float16*>(scratch + L.gu);
  _Float16* h = reinterpret_cast<_Float16*>(scratch + L.h);
  _Float16* dl = reinterpret_cast<_Float16*>(scratch + L.dl);
  int* xexp = reinterpret_cast<int*>(scratch + L.xexp);
  _Float16* xh = reinterpret_cast<_Float16*>(scratch + L.xh);
  int* gu_exp = reinterpret_cast<int*>(scratch + L.gu_exp);
  int* h_exp = reinterpret_cast<int*>(scratch + L.h_exp);
  int* dl_exp = reinterpret_cast<int*>(scratch + L.dl_exp);
  int* pos_of = reinterpret_cast<int*>(scratch + L.pos_of);
  _Float16* y = reinterpret_cast<_Float16*>(scratch + L.y);
  int* y_exp = reinterpret_cast<int*>(scratch + L.y_exp);
  const int K = static_cast<int>(a.n_expert_used);
  const int P = static_cast<int>(a.n_tokens * a.n_expert_used);
  const int R = static_cast<int>(a.max_rank), d = static_cast<int>(a.n_embd), ff = static_cast<int>(a.n_ff);
  const int rb = R / kBlk, fb = ff / kBlk, db = d / kBlk;
  {
    const dim3 xg(static_cast<unsigned>((a.n_tokens + kThreads / kWave - 1) / (kThreads / kWave)));
    float* pso = a.out_mode == LATENT_OUT_PER_SLOT ? static_cast<float*>(a.out) : nullptr;
    const int T = static_cast<int>(a.n_tokens), E = static_cast<int>(a.n_expert);
    if (a.x_dtype == LATENT_F32)
      hipLaunchKernelGGL(x_prep_kernel<true>, xg, dim3(kThreads), 0, s, a.x, a.x_dtype, T, d, xh, xexp, pos_of, K, a.ids,
                         E, pso);
    else
      hipLaunchKernelGGL(x_prep_kernel<false>, xg, dim3(kThreads), 0, s, a.x, a.x_dtype, T, d, xh, xexp, pos_of, K,
                         a.ids, E, pso);
  }
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  int4* units = reinterpret_cast<int4*>(scratch + L.units);
  hipLaunchKernelGGL(tiles_kernel, dim3(static_cast<unsigned>(1 + (P + kTileThreads - 1) / kTileThreads)),
                     dim3(kTileThreads), 0, s, g, bulk ? stream::kBulkM : kMT, tile_a, tile_r0, bulk ? units : nullptr,
                     pos_of, P, K);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;

  if (bulk) {
    // The streaming tile layout with 128-pair units: x -> latents -> h ->
    // d latent -> y (or the per-slot rows), then the per-token combine.
    stream::BulkArgs bk{};
    bk.nunits = g.meta + 2;
    bk.units = units;
    bk.pair_tok = g.pair_tok;
    bk.pair_slot = g.pair_slot;
    bk.pair_w = g.pair_w;
    bk.xh = xh;
    bk.xexp = xexp;
    bk.lat = gu;       // [2][P][256]: the gu buffer's size at rank 256
    bk.lexp = gu_exp;
    bk.hh = h;
    bk.hexp = h_exp;
    bk.dlat = dl;
    bk.dexp = dl_exp;
    bk.y = y;
    bk.yexp = y_exp;
    bk.part = reinterpret_cast<float*>(scratch + L.part);
    const int st = stream::bulk_forward(a, bk, tiles, s);
    if (st != LATENT_OK || a.out_mode == LATENT_OUT_PER_SLOT) return st;
    // The router weight is applied here in both weighting modes (y is linear in h).
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(a.n_tokens)), dim3(kThreads), 0, s, y, y_exp, d / 64, 6,
                       pos_of, g.pair_w, K, d, 0, static_cast<float*>(a.out));
    return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
  }

  Params p{};
  p.g = g;
  p.tile_a = tile_a;
  p.tile_r0 = tile_r0;
  p.xh = xh;
  p.d = d;
  p.out = static_cast<float*>(a.out);
  p.wbd = a.weight_before_down ? 1 : 0;
  p.n_expert_used = static_cast<int>(a.n_expert_used);

  // A: gu = x . [A_g | A_u]
  p.K = d;
  p.a_exp = xexp;
  p.f0 = fac[0];
  p.f1 = fac[2];
  p.ncols = R;
  p.nfac = 2;
  p.dst = gu;
  p.ldd = 2 * R;
  p.dst_exp = gu_exp;
  p.dst_exp_ld = 2 * rb;
  int st = launch<kFromX, kStoreHalf>(p, tiles, s);
  if (st != LATENT_OK) return st;
  // BC1: h = SiLU(g . B_g) * (u . B_u): the gate product into h, then the up
  // product, whose epilogue reads it back.
  p.K = R;
  p.a = gu;
  p.lda = 2 * R;
  p.a_col = 0;
  p.a_exp = gu_exp;
  p.a_exp_ld = 2 * rb;
  p.f0 = p.f1 = fac[1];
  p.ncols = ff;
  p.nfac = 1;
  p.dst = h;
  p.ldd = ff;
  p.dst_exp = h_exp;
  p.dst_exp_ld = fb;
  st = launch<kFromPairs, kStoreSiLU>(p, tiles, s);
  if (st != LATENT_OK) return st;
  p.a_col = R;
  p.f0 = p.f1 = fac[3];
  st = launch<kFromPairs, kSwiGLU>(p, tiles, s);
  if (st != LATENT_OK) return st;
  // BC2: dl = h . A_d
  p.K = ff;
  p.a = h;
  p.lda = ff;
  p.a_col = 0;
  p.a_exp = h_exp;
  p.a_exp_ld = fb;
  p.f0 = p.f1 = fac[4];
  p.ncols = R;
  p.dst = dl;
  p.ldd = R;
  p.dst_exp = dl_exp;
  p.dst_exp_ld = rb;
  st = launch<kFromPairs, kStoreHalf>(p, tiles, s);
  if (st != LATENT_OK) return st;
  // D: y = dl . B_d
  p.K = R;
  p.a = dl;
  p.lda = R;
  p.a_exp = dl_exp;
  p.a_exp_ld = rb;
  p.f0 = p.f1 = fac[5];
  p.ncols = d;
  if (a.out_mode == LATENT_OUT_PER_SLOT) return launch<kFromPairs, kToOutput>(p, tiles, s);
  // Reduced: y rows in fp16, then the per-token weighted sum.
  p.dst = y;
  p.ldd = d;
  p.dst_exp = y_exp;
  p.dst_exp_ld = db;
  st = launch<kFromPairs, kStoreHalf>(p, tiles, s);
  if (st != LATENT_OK) return st;
  hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(a.n_tokens)), dim3(kThreads), 0, s, y, y_exp, db, 7,
                     pos_of, g.pair_w, K, d, p.wbd, static_cast<float*>(a.out));
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace prefill
}  // namespace latent
