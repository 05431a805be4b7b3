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
// Each GEMM tile is 128 pairs x 128 columns on 4 waves (2 x 2 of 64 x 64,
// v_mfma_f32_32x32x16_f16, fp32 accumulation).  Per 32-row K slice the NF4
// factor slice is dequantized (level * scale in fp32, rounded to fp16) into
// LDS transposed to [column][k], the activation slice is gathered and
// converted to fp16 into LDS as [pair][k]; both are double-buffered and the
// next slice's global loads are in flight while the current one multiplies.
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

namespace latent {
namespace prefill {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kMT = 128;       // pairs per tile
constexpr int kNT = 128;       // output columns per tile
constexpr int kKS = 32;        // K rows staged per slice
constexpr int kLds = 40;       // halfs per LDS row: 32 + 8 pad keeps 16-byte fragment reads conflict-free
constexpr int kTileThreads = 1024;
constexpr int kExpMin = -120, kExpMax = 120;

enum ASrc { kFromX = 0, kFromPairs = 1 };
enum Epi { kStoreHalf = 0, kSwiGLU = 1, kToOutput = 2 };

struct Params {
  Grouping g;
  const int* tile_a;
  const int* tile_r0;
  const _Float16* xh;  // kFromX: scaled fp16 x [T][d], row tok(p)
  int d;
  const _Float16* a;  // kFromPairs: a[p * lda + col], scaled by 2^a_exp[p][col / 128]
  int64_t lda;
  int a_col0, a_col1;  // A columns of the first / second product
  const int* a_exp;    // kFromPairs: [P][a_exp_ld] block exponents; kFromX: [T] row exponents of x
  int a_exp_ld;
  int a_part, a_part_blocks;  // the A rows were written as parts of a_part columns, ceil(a_part / 128) blocks each
  int K;
  Factor f0, f1;  // second factor: the u side of SwiGLU, or the blockIdx.z == 1 factor
  int ncols;      // output columns of one factor
  int zdim;       // products per tile: 2 for [A_g | A_u], else 1
  _Float16* dst;  // kStoreHalf / kSwiGLU: dst[p * ldd + col]
  int64_t ldd;
  int dst_col1;   // column offset of the blockIdx.z == 1 product
  int* dst_exp;   // [P][dst_exp_ld] exponents of the stored blocks
  int dst_exp_ld;
  float* out;     // kToOutput: per-slot rows out[(tok * k + slot) * ncols + col]
  int wbd, n_expert_used;
};

// LDS: a ring of kStages raw K slices filled by direct global->LDS loads
// (activations as fp16 16-byte chunks, NF4 codes, fp16 scales), and the
// decoded factor slice, double-buffered, as fp16 [column][k].  Every ring
// stage and decode buffer is its own __shared__ variable and is indexed at
// compile time, so the compiler can tell which direct loads an LDS read
// depends on (one shared object would make every LDS read wait for all of
// them).
constexpr int kStages = 4;
constexpr int kMaxBlocks = 16;  // 128-column exponent blocks per operand row (K <= 2048)

// Bank-conflict-free placements (checked for 32 and 64 banks of 4 bytes):
//   activation chunk c (8 halfs) of row r  -> 16-byte slot r*4 + (c ^ a_swz(r))
//   code chunk c (16 bytes) of factor row r -> 16-byte slot code_row(r)*4 + (c ^ code_swz(r))
__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
__device__ __forceinline__ int code_row(int r) { return (r >> 1) + 16 * (r & 1); }
__device__ __forceinline__ int code_swz(int r) { return (r >> 3) & 3; }

struct Stage {
  _Float16 a[kMT * kKS];       // activations [row][4 chunks of 8 halfs], swizzled
  uint32_t bc[kKS * kNT / 8];  // NF4 codes [32 rows][4 chunks of 16 bytes], rows and chunks permuted
  uint32_t bs[2 * 64];         // scales: [32 rows][4 fp16]; the second half takes a balancing load
};

struct Decoded {
  _Float16 b[kNT * kLds];      // decoded factor slice [column][k]
};

struct Smem {
  float lut[16];
  int cexp[2][kMT];                  // per-row exponent of the operand rows (both products)
  int8_t shift[2][kMT][kMaxBlocks];  // per-row, per-block exponent change to reach cexp
  float rmax[2][kMT];                // row maxima of the two column halves of the output tile
  int tok[kMT];
  int slot[kMT];
  float w[kMT];
};

struct Lds {
  Smem& m;
  Stage &s0, &s1, &s2, &s3;
  Decoded &d0, &d1;
  template <int I>
  __device__ __forceinline__ Stage& stage() const {
    if constexpr (I % kStages == 0) return s0;
    else if constexpr (I % kStages == 1) return s1;
    else if constexpr (I % kStages == 2) return s2;
    else return s3;
  }
  template <int I>
  __device__ __forceinline__ Decoded& dec() const {
    if constexpr (I % 2 == 0) return d0;
    else return d1;
  }
};

// Exponent block of column `col` of an intermediate row.
__device__ __forceinline__ int a_block(const Params& p, int col) {
  return (col / p.a_part) * p.a_part_blocks + (col % p.a_part) / kNT;
}

// Direct global -> LDS loads: lane l's 16 (4) bytes land at lds + 16 l (4 l).
// Written as inline assembly so the compiler does not treat every later LDS
// read as dependent on them (it would wait for all of them, vmcnt(0)); the
// pipeline waits for them itself (slice_barrier).  lds must be wave-uniform.
__device__ __forceinline__ uint32_t lds_u32(void* lds) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)(lds))));
}
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_u32(lds))
               : "m0");
}
__device__ __forceinline__ void dma4(const void* src, void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_u32(lds))
               : "m0");
}

// Issue K slice sl into ring stage st: every wave issues exactly three direct
// loads (two groups of activation rows, then codes or scales), so one vmcnt
// value covers a whole slice.
template <int kA>
__device__ __forceinline__ void issue_slice(const Params& p, const Smem& m, Stage& st, const Factor& f, int64_t e,
                                            int p0, int rows, int n0, int acol, int sl) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int k0 = sl * kKS;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (2 * w + i) * 64 + lane;  // LDS chunk position
    const int r = q >> 2, c = (q & 3) ^ a_swz(r);  // holds chunk c of row r
    const int rr = r < rows ? r : 0;                     // pad rows re-read row 0 (finite; never stored)
    const _Float16* src = kA == kFromX ? p.xh + static_cast<int64_t>(m.tok[rr]) * p.d + k0 + 8 * c
                                       : p.a + static_cast<int64_t>(p0 + rr) * p.lda + acol + k0 + 8 * c;
    dma16(src, &st.a[(2 * w + i) * 512]);
  }
  const int64_t cstride = f.cols / 2, sstride = f.cols / kGroup;
  if (w < 2) {
    const int pr = 16 * w + (lane >> 2);                 // LDS row position
    const int row = 2 * (pr & 15) + (pr >> 4);           // factor row held there
    const int col = n0 + 32 * ((lane & 3) ^ code_swz(row));
    const int colc = col < p.ncols ? col : n0;  // chunks past the factor's columns re-read chunk 0 (decoded as zero)
    dma16(f.codes + (e * f.rows + k0 + row) * cstride + colc / 2, &st.bc[w * 256]);
  } else {
    const int row = lane >> 1, g0 = n0 / kGroup + 2 * (lane & 1);
    const int g = g0 * kGroup < p.ncols ? g0 : n0 / kGroup;
    dma4(f.scales + (e * f.rows + k0 + row) * sstride + g, &st.bs[(w - 2) * 64]);
  }
}

// Workgroup barrier for the slice pipeline.  __syncthreads() would fence
// every outstanding direct load (vmcnt(0)); instead each wave waits until at
// most c slices (3 direct loads each) are in flight and its LDS writes are
// done (s_waitcnt vmcnt(3c) lgkmcnt(0)), then meets the others at s_barrier.
// The signal fences keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void slice_barrier(int c) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (c >= 2)
    __builtin_amdgcn_s_waitcnt(0x0070 | 6);
  else if (c == 1)
    __builtin_amdgcn_s_waitcnt(0x0070 | 3);
  else
    __builtin_amdgcn_s_waitcnt(0x0070);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Decode a ring stage into a decode buffer (thread: rows 2rp, 2rp+1; columns
// 8cg .. 8cg+7) and, for intermediate operands, bring each activation chunk of
// the stage to its row exponent (multiply by 2^shift, exact).
template <int kA>
__device__ __forceinline__ void prepare_slice(const Params& p, const Smem& m, Stage& st, Decoded& d, int n0, int acol,
                                              int q, int sl) {
  const int tid = threadIdx.x, rp = tid & 15, cg = tid >> 4;
  {
    const int r0 = 2 * rp, r1 = 2 * rp + 1;
    const uint32_t c0 = st.bc[4 * (4 * code_row(r0) + ((cg >> 2) ^ code_swz(r0))) + (cg & 3)];
    const uint32_t c1 = st.bc[4 * (4 * code_row(r1) + ((cg >> 2) ^ code_swz(r1))) + (cg & 3)];
    const uint16_t* sh = reinterpret_cast<const uint16_t*>(st.bs);
    const bool ok = n0 + 8 * cg < p.ncols;
    const float s0 = ok ? half_bits_to_float(sh[(2 * rp) * 4 + (cg >> 2)]) : 0.f;
    const float s1 = ok ? half_bits_to_float(sh[(2 * rp + 1) * 4 + (cg >> 2)]) : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half2v v;
      v[0] = static_cast<_Float16>(m.lut[(c0 >> (4 * j)) & 15u] * s0);
      v[1] = static_cast<_Float16>(m.lut[(c1 >> (4 * j)) & 15u] * s1);
      *reinterpret_cast<half2v*>(&d.b[(8 * cg + j) * kLds + 2 * rp]) = v;
    }
  }
  if constexpr (kA == kFromPairs) {
    const int r = tid >> 1;
    const int sft = m.shift[q][r][a_block(p, acol + sl * kKS) - a_block(p, acol)];
    if (sft != 0) {
      const _Float16 mul = sft < -24 ? static_cast<_Float16>(0.f) : static_cast<_Float16>(__builtin_ldexpf(1.f, sft));
#pragma unroll
      for (int c = 2 * (tid & 1); c < 2 * (tid & 1) + 2; ++c) {
        half8* v = reinterpret_cast<half8*>(&st.a[(r * 4 + (c ^ a_swz(r))) * 8]);
        *v = *v * mul;
      }
    }
  }
}

__device__ __forceinline__ void mfma_slice(const Stage& st, const Decoded& d, f32x16 (&acc)[2][2]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w & 1, wn = w >> 1;
#pragma unroll
  for (int ks = 0; ks < kKS; ks += 16) {
    half8 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 64 * wm + 32 * i + (lane & 31), c = (ks >> 3) + (lane >> 5);
      af[i] = *reinterpret_cast<const half8*>(&st.a[(r * 4 + (c ^ a_swz(r))) * 8]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      bf[j] = *reinterpret_cast<const half8*>(&d.b[(64 * wn + 32 * j + (lane & 31)) * kLds + ks + 8 * (lane >> 5)]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
  }
}

// One pipeline step for slice sl = sl0 + I (stage I % kStages, decode buffer
// I % 2): wait for slice sl + 1, refill the stage slice sl - 1 used, prepare
// slice sl + 1, multiply slice sl.
template <int kA, int I>
__device__ __forceinline__ void k_step(const Params& p, const Lds& L, const Factor& f, int64_t e, int p0, int rows,
                                       int n0, int acol, int q, int sl0, int n, f32x16 (&acc)[2][2]) {
  const int sl = sl0 + I;
  if (sl >= n) return;
  // Slices issued so far: 0 .. min(n - 1, sl + kStages - 2); slice sl + 1 must have landed.
  slice_barrier(sl + 1 < n ? min(n - 1, sl + kStages - 2) - (sl + 1) : 0);
  if (sl + kStages - 1 < n)
    issue_slice<kA>(p, L.m, L.template stage<I + kStages - 1>(), f, e, p0, rows, n0, acol, sl + kStages - 1);
  if (sl + 1 < n)
    prepare_slice<kA>(p, L.m, L.template stage<I + 1>(), L.template dec<I + 1>(), n0, acol, q, sl + 1);
  mfma_slice(L.template stage<I>(), L.template dec<I>(), acc);
}

// acc[i][j] += A[rows 64*wm + 32*i ..][K] . B[K][cols 64*wn + 32*j ..] over the
// whole K of the tile, for factor f (expert e) and activation column acol.
template <int kA>
__device__ __forceinline__ void run_k(const Params& p, const Lds& L, const Factor& f, int64_t e, int p0, int rows,
                                      int n0, int acol, int q, f32x16 (&acc)[2][2]) {
  const int n = p.K / kKS;  // >= 1
  issue_slice<kA>(p, L.m, L.s0, f, e, p0, rows, n0, acol, 0);
  if (n > 1) issue_slice<kA>(p, L.m, L.s1, f, e, p0, rows, n0, acol, 1);
  if (n > 2) issue_slice<kA>(p, L.m, L.s2, f, e, p0, rows, n0, acol, 2);
  slice_barrier(min(n - 1, kStages - 2));  // slice 0 landed
  prepare_slice<kA>(p, L.m, L.s0, L.d0, n0, acol, q, 0);
  for (int sl0 = 0; sl0 < n; sl0 += kStages) {
    k_step<kA, 0>(p, L, f, e, p0, rows, n0, acol, q, sl0, n, acc);
    k_step<kA, 1>(p, L, f, e, p0, rows, n0, acol, q, sl0, n, acc);
    k_step<kA, 2>(p, L, f, e, p0, rows, n0, acol, q, sl0, n, acc);
    k_step<kA, 3>(p, L, f, e, p0, rows, n0, acol, q, sl0, n, acc);
  }
  __syncthreads();
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// Exponent e with m * 2^e in [2^14, 2^15) (0 for m == 0 or not finite).
__device__ __forceinline__ int block_exponent(float m) {
  if (!(m > 0.f) || !(m < 3.0e38f)) return 0;
  const int ilog = static_cast<int>((__float_as_uint(m) >> 23) & 0xFFu) - 127;  // floor(log2 m), normal m
  return min(kExpMax, max(kExpMin, 14 - ilog));
}

template <int kA, int kEpi>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(Params p) {  // two workgroups per CU
  __shared__ Smem s;
  __shared__ Stage st0, st1, st2, st3;
  __shared__ Decoded dc0, dc1;
  const Lds L{s, st0, st1, st2, st3, dc0, dc1};
  // Work items (tile, product z, column tile) in expert order, cut into 8
  // contiguous runs, one per XCD (workgroup b runs on XCD b % 8): a tile's
  // column tiles share its activation rows, an expert's tiles share its factor
  // slices, both in one L2.
  const int nn = (p.ncols + kNT - 1) / kNT, per_tile = nn * p.zdim;
  const int total = p.g.meta[2] * per_tile;
  const int per_xcd = (total + 7) / 8;
  const int j = blockIdx.x >> 3, item = (blockIdx.x & 7) * per_xcd + j;
  if (j >= per_xcd || item >= total) return;
  const int tile = item / per_tile, rem = item - tile * per_tile;
  const int a = p.tile_a[tile], r0 = p.tile_r0[tile];
  const int rows = min(kMT, p.g.act_count[a] - r0);
  const int p0 = p.g.act_start[a] + r0;
  const int64_t e = p.g.act_expert[a];
  const int z = rem / nn;
  const int n0 = (rem - z * nn) * kNT;
  const int tid = threadIdx.x;
  if (tid < 16) s.lut[tid] = nf4_level(tid);
  if (tid < kMT) {
    const bool ok = tid < rows;
    s.tok[tid] = ok ? p.g.pair_tok[p0 + tid] : 0;
    s.slot[tid] = ok ? p.g.pair_slot[p0 + tid] : 0;
    s.w[tid] = ok ? p.g.pair_w[p0 + tid] : 0.f;
  }
  __syncthreads();
  // Operand row exponents: x rows carry one; intermediate rows are rescaled to
  // the smallest block exponent over the K range each product reads.
  constexpr int kProducts = kEpi == kSwiGLU ? 2 : 1;
  for (int i = tid; i < kProducts * kMT; i += kThreads) {
    const int q = i / kMT, r = i % kMT;
    int c = 0;
    if (r < rows) {
      if constexpr (kA == kFromX) {
        c = p.a_exp[s.tok[r]];
      } else {
        const int acol = q ? p.a_col1 : p.a_col0;
        const int b0 = a_block(p, acol), b1 = a_block(p, acol + p.K - 1);
        const int* ex = p.a_exp + static_cast<int64_t>(p0 + r) * p.a_exp_ld;
        c = kExpMax;
        for (int b = b0; b <= b1; ++b) c = min(c, ex[b]);
        for (int b = b0; b <= b1; ++b) s.shift[q][r][b - b0] = static_cast<int8_t>(max(-128, c - ex[b]));
      }
    } else if constexpr (kA == kFromPairs) {
      for (int b = 0; b < kMaxBlocks; ++b) s.shift[q][r][b] = 0;
    }
    s.cexp[q][r] = c;
  }
  __syncthreads();

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  run_k<kA>(p, L, z ? p.f1 : p.f0, e, p0, rows, n0, z ? p.a_col1 : p.a_col0, 0, acc);

  const int lane = tid & 63, w = tid >> 6, wm = w & 1, wn = w >> 1;
  if constexpr (kEpi == kSwiGLU) {
    f32x16 acc_u[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_u[i][j][r] = 0.f;
    run_k<kA>(p, L, p.f1, e, p0, rows, n0, p.a_col1, 1, acc_u);
    // h = SiLU(g) * u (* w), in place of g.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const float g = __builtin_ldexpf(acc[i][j][r], -s.cexp[0][row]);
          const float u = __builtin_ldexpf(acc_u[i][j][r], -s.cexp[1][row]);
          float h = silu_f32(g) * u;
          if (p.wbd) h *= s.w[row];
          acc[i][j][r] = h;
        }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          acc[i][j][r] = __builtin_ldexpf(acc[i][j][r], -s.cexp[0][row]);
        }
  }

  if constexpr (kEpi == kToOutput) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = n0 + 64 * wn + 32 * j + (lane & 31);
        if (col >= p.ncols) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row >= rows) continue;
          p.out[(static_cast<int64_t>(s.tok[row]) * p.n_expert_used + s.slot[row]) * p.ncols + col] = acc[i][j][r];
        }
      }
    return;
  }

  // fp16 store with a per-(row, 128-column block) exponent.  Row maxima: over
  // the lane's two column blocks, the 32 lanes of a row, then the two waves
  // that share the rows.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (n0 + 64 * wn + 32 * j + (lane & 31) < p.ncols) m = fmaxf(m, fabsf(acc[i][j][r]));
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      if ((lane & 31) == 0) s.rmax[wn][64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] = m;
    }
  __syncthreads();
  const int blk = z * nn + n0 / kNT;
  if (tid < rows) p.dst_exp[static_cast<int64_t>(p0 + tid) * p.dst_exp_ld + blk] = block_exponent(fmaxf(s.rmax[0][tid], s.rmax[1][tid]));
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 64 * wn + 32 * j + (lane & 31);
      if (col >= p.ncols) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= rows) continue;
        const int ex = block_exponent(fmaxf(s.rmax[0][row], s.rmax[1][row]));
        p.dst[static_cast<int64_t>(p0 + row) * p.ldd + (z ? p.dst_col1 : 0) + col] =
            static_cast<_Float16>(__builtin_ldexpf(acc[i][j][r], ex));
      }
    }
}

// x rows to fp16: xh[t] = fp16(x[t] * 2^e[t]) with 2^e * max|x[t]| in [2^14, 2^15).
// One workgroup per token; d % 8 == 0 and x 16-byte aligned.
// Also clears the token's slot entries of pos_of.
__global__ void __launch_bounds__(kThreads) x_prep_kernel(const void* x, int x_dtype, int d, _Float16* xh, int* xexp,
                                                          int* pos_of, int k) {
  __shared__ float red[kThreads / kWave];
  __shared__ int ex;
  const int t = blockIdx.x, tid = threadIdx.x;
  if (tid < k) pos_of[t * k + tid] = -1;
  const int64_t base = static_cast<int64_t>(t) * d;
  auto load8 = [&](int c, float (&v)[8]) {
    if (x_dtype == LATENT_F32) {
      const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base + c);
      const float4 a = q[0], b = q[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const uint4 h = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base + c);
      const uint32_t w[4] = {h.x, h.y, h.z, h.w};
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
  float m = 0.f;
  for (int c = tid * 8; c < d; c += kThreads * 8) {
    float v[8];
    load8(c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
  }
  for (int off = 1; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = m;
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < kThreads / kWave; ++i) m = fmaxf(m, red[i]);
    ex = block_exponent(m);
    xexp[t] = ex;
  }
  __syncthreads();
  const int e = ex;
  for (int c = tid * 8; c < d; c += kThreads * 8) {
    float v[8];
    load8(c, v);
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(__builtin_ldexpf(v[i], e));
    *reinterpret_cast<half8*>(xh + base + c) = h;
  }
}

// pos_of[tok * k + slot] = pair for the routed pairs (x_prep_kernel cleared it to -1).
__global__ void __launch_bounds__(kThreads) slots_kernel(Grouping g, int* pos_of, int P, int k) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < P && i < g.meta[3]) pos_of[g.pair_tok[i] * k + g.pair_slot[i]] = i;
}

// out[t] = sum over slots (in slot order) of w * y[pos_of[t][slot]] * 2^-exp,
// y rows in fp16 with one exponent per 128 columns.  One workgroup per token.
__global__ void __launch_bounds__(kThreads) combine_kernel(const _Float16* y, const int* yexp, int yexp_ld,
                                                           const int* pos_of, const float* pair_w, int k, int d, int wbd,
                                                           float* out) {
  const int t = blockIdx.x;
  for (int c = threadIdx.x * 8; c < d; c += kThreads * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sl = 0; sl < k; ++sl) {
      const int pos = pos_of[t * k + sl];
      if (pos < 0) continue;
      const half8 h = *reinterpret_cast<const half8*>(y + static_cast<int64_t>(pos) * d + c);
      const float w = __builtin_ldexpf(wbd ? 1.f : pair_w[pos], -yexp[static_cast<int64_t>(pos) * yexp_ld + c / kNT]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, static_cast<float>(h[i]), acc[i]);
    }
    float4* o = reinterpret_cast<float4*>(out + static_cast<int64_t>(t) * d + c);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// M tiles of kMT pairs for every active expert, in expert order.
__global__ void __launch_bounds__(kTileThreads) tiles_kernel(Grouping g, int* tile_a, int* tile_r0) {
  __shared__ int scan[kTileThreads];
  const int tid = threadIdx.x;
  const int n_active = g.meta[0];
  const int per = (n_active + kTileThreads - 1) / kTileThreads;
  const int a0 = min(n_active, tid * per), a1 = min(n_active, a0 + per);
  int mine = 0;
  for (int a = a0; a < a1; ++a) mine += (g.act_count[a] + kMT - 1) / kMT;
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
    for (int r = 0; r < g.act_count[a]; r += kMT) {
      tile_a[t] = a;
      tile_r0[t] = r;
      ++t;
    }
  }
  if (tid == kTileThreads - 1) g.meta[2] = scan[tid];
}

size_t align_up(size_t v) { return (v + 255) / 256 * 256; }

int64_t max_tiles(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  return (P + kMT - 1) / kMT + std::min<int64_t>(a.n_expert, P);
}

template <int kA, int kEpi>
int launch(Params p, int64_t tiles, int ncols, int zdim, hipStream_t s) {
  p.zdim = zdim;
  const int64_t items = tiles * ((ncols + kNT - 1) / kNT) * zdim;
  const dim3 grid(static_cast<unsigned>(8 * ((items + 7) / 8)));
  hipLaunchKernelGGL((gemm_kernel<kA, kEpi>), grid, dim3(kThreads), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace

bool supported(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  const int64_t active = std::max<int64_t>(1, std::min<int64_t>(a.n_expert, P));
  if (P < static_cast<int64_t>(kMinPairsPerExpert) * active) return false;
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs)
    if (f->int8_bitmap != nullptr) return false;  // per-group INT8 layers take the general path
  if ((reinterpret_cast<uintptr_t>(a.x) & 15u) != 0) return false;
  // Direct 16-byte code loads and 4-byte scale-pair loads: 64-column multiples
  // and aligned factor arrays; at most kMaxBlocks exponent blocks per row.
  if (a.n_embd % 64 || a.n_ff % 64 || a.max_rank % 64) return false;
  if (a.n_ff > kMaxBlocks * kNT || a.max_rank > kMaxBlocks * kNT) return false;
  for (const latent_factor* f : fs)
    if ((reinterpret_cast<uintptr_t>(f->codes) & 15u) || (reinterpret_cast<uintptr_t>(f->scales) & 3u)) return false;
  return true;
}

Layout layout_for(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used, R = a.max_rank, T = max_tiles(a);
  Layout L{};
  size_t off = 0;
  L.tile_a = off;  off = align_up(off + T * sizeof(int));
  L.tile_r0 = off; off = align_up(off + T * sizeof(int));
  const int64_t rb = (R + kNT - 1) / kNT, fb = (a.n_ff + kNT - 1) / kNT;
  L.xexp = off;    off = align_up(off + a.n_tokens * sizeof(int));
  L.xh = off;      off = align_up(off + a.n_tokens * a.n_embd * sizeof(_Float16));
  L.gu = off;      off = align_up(off + P * 2 * R * sizeof(_Float16));
  L.gu_exp = off;  off = align_up(off + P * 2 * rb * sizeof(int));
  L.h = off;       off = align_up(off + P * a.n_ff * sizeof(_Float16));
  L.h_exp = off;   off = align_up(off + P * fb * sizeof(int));
  L.dl = off;      off = align_up(off + P * R * sizeof(_Float16));
  L.dl_exp = off;  off = align_up(off + P * rb * sizeof(int));
  const int64_t db = (a.n_embd + kNT - 1) / kNT;
  L.pos_of = off;  off = align_up(off + P * sizeof(int));
  L.y = off;       off = align_up(off + (a.out_mode == LATENT_OUT_REDUCED ? P * a.n_embd * sizeof(_Float16) : 0));
  L.y_exp = off;   off = align_up(off + (a.out_mode == LATENT_OUT_REDUCED ? P * db * sizeof(int) : 0));
  L.total = off;
  return L;
}

int forward(const latent_moe_args& a, const Factor* fac, const Grouping& g, char* scratch, hipStream_t s) {
  const Layout L = layout_for(a);
  const int64_t tiles = max_tiles(a);
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
  const int rb = (R + kNT - 1) / kNT, fb = (ff + kNT - 1) / kNT;
  hipLaunchKernelGGL(x_prep_kernel, dim3(static_cast<unsigned>(a.n_tokens)), dim3(kThreads), 0, s, a.x, a.x_dtype, d,
                     xh, xexp, pos_of, K);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  hipLaunchKernelGGL(tiles_kernel, dim3(1), dim3(kTileThreads), 0, s, g, tile_a, tile_r0);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  hipLaunchKernelGGL(slots_kernel, dim3(static_cast<unsigned>((P + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, g,
                     pos_of, P, K);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;

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
  p.dst = gu;
  p.ldd = 2 * R;
  p.dst_col1 = R;
  p.dst_exp = gu_exp;
  p.dst_exp_ld = 2 * rb;
  int st = launch<kFromX, kStoreHalf>(p, tiles, R, 2, s);
  if (st != LATENT_OK) return st;
  // BC1: h = SiLU(g . B_g) * (u . B_u)
  p.K = R;
  p.a = gu;
  p.lda = 2 * R;
  p.a_col0 = 0;
  p.a_col1 = R;
  p.a_exp = gu_exp;
  p.a_exp_ld = 2 * rb;
  p.a_part = R;
  p.a_part_blocks = rb;
  p.f0 = fac[1];
  p.f1 = fac[3];
  p.ncols = ff;
  p.dst = h;
  p.ldd = ff;
  p.dst_col1 = 0;
  p.dst_exp = h_exp;
  p.dst_exp_ld = fb;
  st = launch<kFromPairs, kSwiGLU>(p, tiles, ff, 1, s);
  if (st != LATENT_OK) return st;
  // BC2: dl = h . A_d
  p.K = ff;
  p.a = h;
  p.lda = ff;
  p.a_col0 = p.a_col1 = 0;
  p.a_exp = h_exp;
  p.a_exp_ld = fb;
  p.a_part = ff;
  p.a_part_blocks = fb;
  p.f0 = p.f1 = fac[4];
  p.ncols = R;
  p.dst = dl;
  p.ldd = R;
  p.dst_exp = dl_exp;
  p.dst_exp_ld = rb;
  st = launch<kFromPairs, kStoreHalf>(p, tiles, R, 1, s);
  if (st != LATENT_OK) return st;
  // D: out += w * (dl . B_d)
  p.K = R;
  p.a = dl;
  p.lda = R;
  p.a_exp = dl_exp;
  p.a_exp_ld = rb;
  p.a_part = R;
  p.a_part_blocks = rb;
  p.f0 = p.f1 = fac[5];
  p.ncols = d;
  if (a.out_mode == LATENT_OUT_PER_SLOT) return launch<kFromPairs, kToOutput>(p, tiles, d, 1, s);
  // Reduced: y rows in fp16, then the per-token weighted sum.
  const int db = (d + kNT - 1) / kNT;
  p.dst = y;
  p.ldd = d;
  p.dst_col1 = 0;
  p.dst_exp = y_exp;
  p.dst_exp_ld = db;
  st = launch<kFromPairs, kStoreHalf>(p, tiles, d, 1, s);
  if (st != LATENT_OK) return st;
  hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(a.n_tokens)), dim3(kThreads), 0, s, y, y_exp, db, pos_of,
                     g.pair_w, K, d, p.wbd, static_cast<float*>(a.out));
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace prefill
}  // namespace latent
