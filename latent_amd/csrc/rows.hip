// MoE-layer LATENT expert FFN over the row layout with fp16 MFMA.
//
// The three phases of the multi-kernel path (moe.hip) for layers held in the
// row layout -- per-expert ranks up to 512, INT8 groups allowed -- with the
// products on v_mfma_f32_16x16x32_f16 instead of fp32 FMAs:
//   A   xh . A_g | A_u -> gu     items (expert, factor, range of d rows)
//   BC  g . B_g, u . B_u -> h = SiLU(g) u (in LDS); h . A_d -> dl
//                                items (expert, 256 columns of ff)
//   D   dl . B_d -> out          items (expert, 512 columns of d)
// Replaces, like moe.hip, the per-(token, slot) chain of
// kernels/latent_fused_expert_ffn.cu:27-108 for the routed pairs of each
// active expert; only an expert's true-rank rows and columns are read.
//
// Every factor is row-major [K][N] with 32-column groups along N (16 bytes
// of NF4 codes, low nibble first, or 32 INT8 bytes, and one fp16 scale),
// while an MFMA operand holds 8 consecutive K values per lane.  So a
// workgroup decodes a chunk of rows at a time into LDS, transposed: thread
// (group, row pair) turns its two rows' groups into fp16 values (level x
// scale or q x scale, one rounding) and stores each column's pair of rows as
// one dword; the MFMA then reads 16 bytes of one column per lane.  A chunk is
// 256 such units: ngp groups (the item's groups rounded up to a power of
// two, 2..16) by 512 / ngp rows, so a chunk is about 8 KB of codes whatever
// the rank.  The codes, scales, bitmap words and word offsets of chunk c + 2
// are in flight in registers while chunk c is decoded, and the INT8 bytes of
// chunk c + 1 (their offsets known one chunk earlier).
//
// Activations (x rows, latents, h) enter the MFMA as fp16 rows scaled by a
// power of two per row (the row maximum into [2^14, 2^15)); products are
// scaled back in fp32 and summed into the fp32 accumulators of the
// multi-kernel path with atomics (gu, dl; out for the reduced output), which
// its prep kernel zeroes.  A pass takes 16 pairs of one expert (one MFMA row
// block); an expert with more pairs takes several passes.
#include "common.hpp"
#include "rows.hpp"

#include <algorithm>

namespace latent {
namespace rows {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

enum { F_GATE_A = 0, F_GATE_B, F_UP_A, F_UP_B, F_DOWN_A, F_DOWN_B };

constexpr int kT = 256;            // threads per workgroup (4 waves)
constexpr int kPass = 16;          // pairs per pass: one MFMA row block
constexpr int kMaxGroups = 16;     // groups per chunk (512 columns)
constexpr int kCB = 256;           // BC: ff columns per item
constexpr int kCD = 512;           // D: d columns per item
constexpr int kHDw = kCB / 2 + 4;  // BC: dwords per h row (256 halves + 8 pad)
// Decoded chunk: group blocks of 32 columns of (rows / 2 + 4) dwords; at
// most 16 x (32 x 20 + 4) dwords (ngp = 16, 32 rows).
constexpr int kBtDw = kMaxGroups * (32 * 20 + 4);
constexpr int kActDw = kPass * (256 / 2 + 4);  // activation rows of a chunk of at most 256 rows

// LDS byte address of a __shared__ object and raw LDS accesses.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T& obj) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)(&obj)));
}
template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr));
}
template <typename T>
__device__ __forceinline__ void lds_st(uint32_t addr, const T& v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr)) = v;
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Workgroup barrier over LDS only: waits for this wave's LDS accesses, then
// s_barrier.  (__syncthreads() would also wait for every outstanding global
// load and drain the chunks loaded ahead.)  Workgroups of these kernels
// share data through LDS only.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Raw buffer resource over `bytes` bytes (loads beyond them return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

__device__ __forceinline__ int rank_of(const Params& p, int e, int kind) {
  if (!p.ranks) return p.R;
  const int r = p.ranks[e * 3 + kind];
  return r < 0 ? 0 : (r > p.R ? p.R : r);
}

// Workgroup b -> (active expert a, item i): an expert's items on one XCD
// (workgroups go to the 8 XCDs round robin), so its activations stay in one L2.
__device__ __forceinline__ bool map_item(int b, int n_items, int n_active, int& a, int& i) {
  const int x = b & 7, j = b >> 3;
  a = x + 8 * (j / n_items);
  i = j - (j / n_items) * n_items;
  return a < n_active;
}

// Level-pair table: entry b = (level(b & 15), level(b >> 4)) as two fp16.
__device__ __forceinline__ void lut_fill(uint32_t* lut, int tid) {
  const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
  lut[tid] = __builtin_bit_cast(uint32_t, lv);
}

// Chunk shape for ng groups (a compile-time type, so every LDS offset of a
// chunk is an immediate): ngp = ng rounded up to a power of two in [2, 16],
// rows = 512 / ngp; dwords per decoded column cstr = rows / 2 + 4 (16-byte
// MFMA reads of 8 consecutive columns fall on distinct banks), per group
// block gstr = 32 cstr + 64 / ngp (the 64 stores of a wave, 64 / ngp row
// pairs of ngp groups, fall on distinct banks).
template <int NGP>
struct Shape {
  static constexpr int ngp = NGP, rows = 512 / NGP, cstr = rows / 2 + 4, gstr = 32 * cstr + 64 / NGP;
};
// The same shape as run-time values (one code path for every shape).
struct DynShape {
  int ngp, rows, cstr, gstr;
};
__device__ __forceinline__ DynShape dyn_shape(int ng) {
  int ngp = 2;
  while (ngp < ng) ngp <<= 1;
  const int rows = 512 / ngp, cstr = rows / 2 + 4;
  return DynShape{ngp, rows, cstr, 32 * cstr + 64 / ngp};
}
// f(Shape<ngp>{}) for the chunk shape of ng groups.
template <typename F>
__device__ __forceinline__ void with_shape(int ng, F&& f) {
  if (ng <= 2)
    f(Shape<2>{});
  else if (ng <= 4)
    f(Shape<4>{});
  else if (ng <= 8)
    f(Shape<8>{});
  else
    f(Shape<16>{});
}

// One thread's decode unit of a chunk: rows r, r + 1 of one group.
struct Unit {
  u32x4 c[2];     // codes
  uint32_t s;     // scales (fp16 bits; row r in the low half)
  uint32_t w[2];  // INT8 bitmap words
  int o[2];       // their word offsets
};
struct Q {  // the INT8 bytes of the unit's rows (zero where NF4)
  u32x4 v[2][2];
};

// One thread's view of a decode source: rows below row_end of groups
// [g0, g0 + ng) of one expert's factor, in chunks of sh.rows rows from row
// `base`; the thread's unit is group gi and row pair rp of each chunk.  The
// expert's codes, scales, bitmap words and word offsets through buffer
// resources (wave-uniform; 32-bit offsets, zeros past the expert's rows or
// for a factor without INT8 groups), the INT8 bytes through one over the
// factor's side buffer.
struct Src {
  __amdgpu_buffer_rsrc_t rc, rs, rb, ro, rd;
  int cs, ss, words;
  int base, row_end, g0, ng, gi, rp;
};
__device__ __forceinline__ Src make_src(const Factor& f, int e, int base, int row_end, int g0, int ng, int gi,
                                        int rp) {
  const int64_t er = static_cast<int64_t>(e) * f.rows;
  const int cs = static_cast<int>(f.code_stride()), ss = static_cast<int>(f.scale_stride()), words = f.words();
  const bool has8 = f.ext.bitmap != nullptr;
  const uint32_t rows = static_cast<uint32_t>(f.rows);
  Src s;
  s.rc = buffer_rsrc(f.codes + er * cs, rows * cs);
  s.rs = buffer_rsrc(f.scales + er * ss, rows * ss * 2u);
  s.rb = buffer_rsrc(has8 ? f.ext.bitmap + er * words : nullptr, has8 ? rows * words * 4u : 0u);
  s.ro = buffer_rsrc(has8 ? f.ext.word_offset + er * words : nullptr, has8 ? rows * words * 4u : 0u);
  s.rd = buffer_rsrc(f.ext.data, has8 ? 0x7FFFFFF0u : 0u);
  s.cs = cs;
  s.ss = ss;
  s.words = words;
  s.base = base;
  s.row_end = row_end;
  s.g0 = g0;
  s.ng = ng;
  s.gi = gi;
  s.rp = rp;
  return s;
}

// Loads of rows r, r + 1 of group g.
template <bool kInt8>
__device__ __forceinline__ void unit_load(const Src& s, int r, int g, Unit& u) {
  const uint32_t r0 = static_cast<uint32_t>(r), r1 = r0 + 1u;
  u.c[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.rc, r0 * s.cs + g * kGroupBytes, 0, 0));
  u.c[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.rc, r1 * s.cs + g * kGroupBytes, 0, 0));
  const uint32_t s0 = __builtin_amdgcn_raw_buffer_load_b16(s.rs, (r0 * s.ss + g) * 2u, 0, 0);
  const uint32_t s1 = __builtin_amdgcn_raw_buffer_load_b16(s.rs, (r1 * s.ss + g) * 2u, 0, 0);
  u.s = s0 | (s1 << 16);
  if (kInt8) {
    const uint32_t ws = static_cast<uint32_t>(g >> 5);
    u.w[0] = __builtin_amdgcn_raw_buffer_load_b32(s.rb, (r0 * s.words + ws) * 4u, 0, 0);
    u.w[1] = __builtin_amdgcn_raw_buffer_load_b32(s.rb, (r1 * s.words + ws) * 4u, 0, 0);
    u.o[0] = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(s.ro, (r0 * s.words + ws) * 4u, 0, 0));
    u.o[1] = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(s.ro, (r1 * s.words + ws) * 4u, 0, 0));
  }
}

// The INT8 bytes of a unit's flagged rows (an unflagged row reads past the
// range and gets zeros: no branch).
template <bool kInt8>
__device__ __forceinline__ void q_load(const Src& s, const Unit& u, int g, Q& q) {
  if (!kInt8) return;
  const uint32_t bit = 1u << (g & 31);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bool is8 = (u.w[h] & bit) != 0u;
    const uint32_t off = is8 ? static_cast<uint32_t>(u.o[h] + popc(u.w[h] & (bit - 1u))) * kGroup : 0x80000000u;
    q.v[h][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.rd, off, 0, 0));
    q.v[h][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.rd, off + 16u, 0, 0));
  }
}

// Row h of a unit as 16 fp16 pairs (columns 2i, 2i + 1): level x scale or
// q x scale, rounded once; zeros for a dead row (scale 0: every level and q
// is finite).  INT8 bytes become fp16 exactly through 0x6400 | (q ^ 0x80) =
// 1024 + q + 128, less 1152.
template <bool kInt8>
__device__ __forceinline__ void unit_row(const Unit& u, const Q& q, int h, int g, bool live, uint32_t lut,
                                         half2v (&v)[16]) {
  const _Float16 s = live ? __builtin_bit_cast(_Float16, static_cast<uint16_t>(u.s >> (16 * h)))
                          : static_cast<_Float16>(0.f);
  const half2v s2 = {s, s};
  const bool is8 = kInt8 && ((u.w[h] >> (g & 31)) & 1u);
  if (is8) {
    const half2v bias = {static_cast<_Float16>(-1152.f), static_cast<_Float16>(-1152.f)};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t d = q.v[h][i >> 2][i & 3] ^ 0x80808080u;
      const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, d, 0x04010400u);  // bytes (d0, 0x64, d1, 0x64)
      const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, d, 0x04030402u);  // bytes (d2, 0x64, d3, 0x64)
      v[2 * i] = (__builtin_bit_cast(half2v, lo) + bias) * s2;
      v[2 * i + 1] = (__builtin_bit_cast(half2v, hi) + bias) * s2;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t b = (u.c[h][i >> 2] >> (8 * (i & 3))) & 0xFFu;
      v[i] = __builtin_bit_cast(half2v, lds_ld<uint32_t>(lut + b * 4)) * s2;
    }
  }
}

// Decode a unit and store it transposed: column j's dword at dst + j cstr
// holds (row r, row r + 1).
template <bool kInt8>
__device__ __forceinline__ void unit_store(const Unit& u, const Q& q, int g, bool live0, bool live1, uint32_t lut,
                                           uint32_t dst, int cstr) {
  half2v v0[16], v1[16];
  unit_row<kInt8>(u, q, 0, g, live0, lut, v0);
  unit_row<kInt8>(u, q, 1, g, live1, lut, v1);
  const uint32_t step = static_cast<uint32_t>(cstr) * 4u;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t a = __builtin_bit_cast(uint32_t, v0[i]), b = __builtin_bit_cast(uint32_t, v1[i]);
    lds_st<uint32_t>(dst + (2 * i) * step, __builtin_amdgcn_perm(b, a, 0x05040100u));
    lds_st<uint32_t>(dst + (2 * i + 1) * step, __builtin_amdgcn_perm(b, a, 0x07060302u));
  }
}

// The decode ring: units of chunks c .. c + 3 (slots c % 4) and INT8 bytes
// of chunks c, c + 1 (slots c % 2).  Every chunk issues the same loads
// (clamped past the last chunk), so the compiler's wait counts hold on every
// path.
template <bool kInt8>
struct Ring {
  Unit u[4];
  Q q[2];
};

template <bool kInt8, class SH>
__device__ __forceinline__ void ring_issue(const Src& s, SH sh, int c, int nc, Unit& u) {
  const int g = s.g0 + min(s.gi, s.ng - 1);
  unit_load<kInt8>(s, s.base + min(c, nc - 1) * sh.rows + 2 * s.rp, g, u);
}
template <bool kInt8, class SH>
__device__ __forceinline__ void ring_store(const Src& s, SH sh, int c, const Unit& u, const Q& q,
                                           uint32_t lut, uint32_t bt, int block) {
  if (s.gi >= s.ng) return;
  const int r = s.base + c * sh.rows + 2 * s.rp;
  const uint32_t dst = bt + static_cast<uint32_t>(block * sh.gstr + s.rp) * 4u;
  unit_store<kInt8>(u, q, s.g0 + s.gi, r < s.row_end, r + 1 < s.row_end, lut, dst, sh.cstr);
}

// MFMA steps of a chunk: acc[j] += act rows . decoded columns of column block
// cb = cb0 + j * cbs (j < kNcb, cb < ncb), rows / 32 steps of K.  act: LDS
// byte address of the activation rows (astr dwords apart) at the chunk's
// first K value.
template <int kNcb, class SH>
__device__ __forceinline__ void chunk_mfma(uint32_t act, int astr, uint32_t bt, SH sh, int cb0, int cbs,
                                           int ncb, int n, int kq, float4v (&acc)[kNcb]) {
  const int steps = sh.rows / 32;
  for (int s = 0; s < steps; ++s) {
    const half8 a = lds_ld<half8>(act + static_cast<uint32_t>(n * astr + s * 16 + kq * 4) * 4u);
#pragma unroll
    for (int j = 0; j < kNcb; ++j) {
      const int cb = cb0 + j * cbs;
      if (cb < ncb) {
        const uint32_t col = (cb & 1) * 16 + n;
        const half8 b = lds_ld<half8>(bt + static_cast<uint32_t>((cb >> 1) * sh.gstr + col * sh.cstr + s * 16 + kq * 4) * 4u);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
      }
    }
  }
}

// The chunk loop of one decode source.  Step c issues the activation loads
// of chunk c + 1 (issue(c + 1, slot)), the INT8 bytes of chunk c + 1 (whose
// units were issued two steps earlier) and the units of chunk c + 3, then
// stores chunk c's activations (store(c, slot)) and decoded units to LDS
// and runs its MFMA steps (mfma(c)).  Loads complete in issue order, so the
// decode of chunk c leaves the units of chunks c + 2 and c + 3 in flight.
// Two barriers per chunk: the decoded chunk and the activations are
// complete, then every wave is done with them (LDS barriers: the loads
// issued ahead stay in flight).  block: the thread's group block in the
// decoded chunk.
template <bool kInt8, class SH, typename Issue, typename Store, typename Mfma>
__device__ __forceinline__ void run_chunks(const Src& s, SH sh, int nc, int block, uint32_t lut,
                                           uint32_t bt, Ring<kInt8>& rg, Issue&& issue, Store&& store,
                                           Mfma&& mfma) {
  const int g = s.g0 + min(s.gi, s.ng - 1);
  ring_issue<kInt8>(s, sh, 0, nc, rg.u[0]);
  ring_issue<kInt8>(s, sh, 1, nc, rg.u[1]);
  ring_issue<kInt8>(s, sh, 2, nc, rg.u[2]);
  q_load<kInt8>(s, rg.u[0], g, rg.q[0]);
  issue(0, std::integral_constant<int, 0>{});
  auto step = [&](int c, auto us) __attribute__((always_inline)) {
    constexpr int U = decltype(us)::value, Qs = U & 1;
    issue(c + 1, std::integral_constant<int, Qs ^ 1>{});
    q_load<kInt8>(s, rg.u[(U + 1) & 3], g, rg.q[Qs ^ 1]);
    ring_issue<kInt8>(s, sh, c + 3, nc, rg.u[(U + 3) & 3]);
    store(c, std::integral_constant<int, Qs>{});
    ring_store<kInt8>(s, sh, c, rg.u[U], rg.q[Qs], lut, bt, block);
    lds_barrier();
    mfma(c);
    lds_barrier();
  };
  for (int c = 0; c < nc; c += 4) {
    step(c, std::integral_constant<int, 0>{});
    if (c + 1 >= nc) break;
    step(c + 1, std::integral_constant<int, 1>{});
    if (c + 2 >= nc) break;
    step(c + 2, std::integral_constant<int, 2>{});
    if (c + 3 >= nc) break;
    step(c + 3, std::integral_constant<int, 3>{});
  }
}

__device__ __forceinline__ half2v to_h2(float a, float b, int ex) {
  return half2v{static_cast<_Float16>(ldexpf(a, ex)), static_cast<_Float16>(ldexpf(b, ex))};
}

// ---------------------------------------------------------------------------
// Phase A: x . A_g, x . A_u over a range of d rows
// ---------------------------------------------------------------------------
struct alignas(16) SmemA {
  uint32_t bt[kBtDw];
  uint32_t act[2][kActDw];  // x rows of the chunk (by ring slot parity of the stage)
  uint32_t lut[256];
  int rtok[kPass];
  int rexp[kPass];
};

template <bool kInt8>
__global__ void __launch_bounds__(kT, 2) a_kernel(Params p) {
  __shared__ SmemA sm;
  int a, item;
  if (!map_item(blockIdx.x, p.n_a, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int kind = item & 1, split = item >> 1;
  const Factor& f = p.fac[kind ? F_UP_A : F_GATE_A];
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int rank = rank_of(p, e, kind), ng = (rank + kGroup - 1) / kGroup;
  if (ng == 0 || mtot == 0) return;
  with_shape(ng, [&](auto sh) __attribute__((always_inline)) {
    // The item's share of the expert's chunks of d (chunks of sh.rows rows:
    // about 8 KB of codes each, so an expert's chunk count grows with its rank).
    const int nct = (p.d + sh.rows - 1) / sh.rows;
    const int c_lo = split * nct / p.na_split, c_hi = (split + 1) * nct / p.na_split;
    const int nc = c_hi - c_lo;
    if (nc <= 0) return;
    const int r_lo = c_lo * sh.rows, r_end = min(p.d, c_hi * sh.rows);
    lut_fill(sm.lut, tid);
    const uint32_t L_lut = lds_addr(sm.lut), L_bt = lds_addr(sm.bt);
    const uint32_t L_act[2] = {lds_addr(sm.act[0]), lds_addr(sm.act[1])};
    const Src src = make_src(f, e, r_lo, r_end, 0, ng, tid & (sh.ngp - 1), tid / sh.ngp);
    const int ncb = 2 * ng;  // 16-column blocks of the rank
    const int astr = sh.cstr;
    // x staging: 16 rows x sh.rows halves in 16-byte pieces; piece i of this
    // thread is tid + 256 i (i < 2; sh.rows <= 256).
    const int pieces = kPass * sh.rows / 8, ppr = sh.rows / 8;
    for (int tb = 0; tb < mtot; tb += kPass) {
      const int m = min(kPass, mtot - tb);
      if (tid < kPass) {
        const int tok = tid < m ? p.pair_tok[s0 + tb + tid] : -1;
        sm.rtok[tid] = tok;
        sm.rexp[tid] = tok >= 0 ? p.xexp[tok] : 0;
      }
      lds_barrier();
      u32x4 xr[2][2];
      auto load_x = [&](int c, u32x4 (&x)[2]) __attribute__((always_inline)) {
  #pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int pc = tid + kT * i;
          const int row = min(pc / ppr, kPass - 1), k8 = pc % ppr;
          const int tok = sm.rtok[row];
          const int col = r_lo + min(c, nc - 1) * sh.rows + k8 * 8;
          const bool ok = pc < pieces && tok >= 0 && col < r_end;
          const int64_t off = static_cast<int64_t>(max(tok, 0)) * p.d + min(col, p.d - 8);
          const u32x4 v = *reinterpret_cast<const u32x4*>(p.xh + off);
          x[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
        }
      };
      float4v acc[8];
  #pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
      Ring<kInt8> rg;
      auto issue = [&](int c, auto slot) __attribute__((always_inline)) { load_x(c, xr[decltype(slot)::value]); };
      auto store = [&](int c, auto slot) __attribute__((always_inline)) {
        constexpr int S = decltype(slot)::value;
  #pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int pc = tid + kT * i;
          if (pc < pieces)
            lds_st<u32x4>(L_act[S] + static_cast<uint32_t>((pc / ppr) * astr + (pc % ppr) * 4) * 4u, xr[S][i]);
        }
      };
      auto mfma = [&](int c) __attribute__((always_inline)) {
        // The stage of chunk c wrote act[c % 2] (the ring's slot order).
        chunk_mfma<8>(L_act[c & 1], astr, L_bt, sh, wave, 4, ncb, n, kq, acc);
      };
      run_chunks<kInt8>(src, sh, nc, src.gi, L_lut, L_bt, rg, issue, store, mfma);
      // Partial latents of the pass: scaled back, summed into gu.
  #pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int cb = wave + 4 * j;
        const int col = cb * 16 + n;
        if (cb < ncb && col < rank) {
  #pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = kq * 4 + v;
            if (row < m) {
              const float sc = ldexpf(1.0f, -sm.rexp[row]);
              atomic_add_f32(p.gu + static_cast<int64_t>(s0 + tb + row) * (2 * p.R) + kind * p.R + col, acc[j][v] * sc);
            }
          }
        }
      }
      lds_barrier();  // rtok / rexp of the next pass
    }
  });
}

// ---------------------------------------------------------------------------
// Phase BC: g . B_g and u . B_u over 256 columns of ff, h = SiLU(g) u in
// LDS, then h . A_d (those 256 rows of A_d)
// ---------------------------------------------------------------------------
struct alignas(16) SmemBC {
  uint32_t bt[kBtDw];
  uint32_t act[2][2][kPass * 20];  // [slot][gate, up] latent rows of a 32-row chunk
  uint32_t h[kPass * kHDw];        // h rows (fp16 x 2^hexp)
  uint32_t lut[256];
  int rexp[2][kPass];              // gate, up latent exponents
  int hexp[kPass];
  float hmax[4][kPass];
};

template <bool kInt8>
__global__ void __launch_bounds__(kT, 2) bc_kernel(Params p) {
  __shared__ SmemBC sm;
  int a, item;
  if (!map_item(blockIdx.x, p.n_bc, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int rg_ = rank_of(p, e, 0), ru = rank_of(p, e, 1), rd = rank_of(p, e, 2);
  const int c0 = item * kCB, ncol = min(kCB, p.ff - c0), ngc = ncol / kGroup;
  if (mtot == 0) return;
  lut_fill(sm.lut, tid);
  const uint32_t L_lut = lds_addr(sm.lut), L_bt = lds_addr(sm.bt), L_h = lds_addr(sm.h);
  const Factor& fbg = p.fac[F_GATE_B];
  const Factor& fbu = p.fac[F_UP_B];
  const Factor& fad = p.fac[F_DOWN_A];
  // Stage 1: 16 groups per chunk (8 of B_g, 8 of B_u), 32 rows of the rank.
  constexpr Shape<16> sh1{};
  const int kb = max(rg_, ru);
  const int nc1 = (kb + 31) / 32;
  // Stage 2: the 256 rows of A_d at c0, rd columns.
  const int ngd = (rd + kGroup - 1) / kGroup;
  for (int tb = 0; tb < mtot; tb += kPass) {
    const int m = min(kPass, mtot - tb);
    // Latent row exponents: max |g|, then max |u|, over the rank (16 lanes per row).
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int r = tid >> 4, t = tid & 15;
      const int rk = k ? ru : rg_;
      float mx = 0.f;
      if (r < m) {
        const float* row = p.gu + static_cast<int64_t>(s0 + tb + r) * (2 * p.R) + k * p.R;
        for (int c = t; c < rk; c += 16) mx = fmaxf(mx, fabsf(row[c]));
      }
      mx = op_over(mx, 1, 16, OpMax{});
      if (t == 0) sm.rexp[k][r] = pow2_row_exponent(mx);
    }
    lds_barrier();
    float4v accg[4], accu[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) accg[j] = accu[j] = float4v{0.f, 0.f, 0.f, 0.f};
    if (nc1 > 0) {
      // Two sources in one chunk: waves 0-1 decode the item's groups of B_g
      // into group blocks 0-7, waves 2-3 those of B_u into blocks 8-15
      // (thread: group tid % 8, row pair (tid % 128) / 8).  Rows past a
      // factor's own rank decode as zeros.
      const bool up = uniform(tid >> 7) != 0;
      const Src mine = make_src(up ? fbu : fbg, e, 0, up ? ru : rg_, c0 / kGroup, ngc, tid & 7, (tid & 127) >> 3);
      const int block = (up ? 8 : 0) + (tid & 7);
      // act staging: gate and up latent rows of chunk c (32 rank rows), fp16 x 2^rexp.
      u32x4 lr[2];
      auto load_l = [&](int c, u32x4& x) __attribute__((always_inline)) {
        // Thread: row r = tid >> 4, factor k = (tid >> 3) & 1, 4 values at 4 (tid & 7).
        const int r = tid >> 4, k = (tid >> 3) & 1, q4 = (tid & 7) * 4;
        const int col = min(c, nc1 - 1) * 32 + q4;
        const int rk = k ? ru : rg_;
        const bool ok = r < m && col < rk;
        const float* src = p.gu + static_cast<int64_t>(s0 + tb + min(r, m - 1)) * (2 * p.R) + k * p.R + min(col, p.R - 4);
        const float4 v = *reinterpret_cast<const float4*>(src);
        x = ok ? u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)}
               : u32x4{0u, 0u, 0u, 0u};
      };
      auto issue = [&](int c, auto slot) __attribute__((always_inline)) { load_l(c, lr[decltype(slot)::value]); };
      auto store = [&](int c, auto slot) __attribute__((always_inline)) {
        constexpr int S = decltype(slot)::value;
        const int r = tid >> 4, k = (tid >> 3) & 1, q4 = (tid & 7) * 4;
        const int ex = sm.rexp[k][r];
        const half2v h0 = to_h2(__uint_as_float(lr[S][0]), __uint_as_float(lr[S][1]), ex);
        const half2v h1 = to_h2(__uint_as_float(lr[S][2]), __uint_as_float(lr[S][3]), ex);
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 w = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
        lds_st<u32x2>(lds_addr(sm.act[S][k]) + static_cast<uint32_t>(r * 20 + q4 / 2) * 4u, w);
      };
      Ring<kInt8> rg;
      auto mfma = [&](int c) __attribute__((always_inline)) {
        const int S = c & 1;
        // Wave w: columns [64w, 64w + 64) of the item for both factors
        // (groups 2w, 2w + 1 of B_g and 8 + 2w, 9 + 2w of B_u).
        chunk_mfma<4>(lds_addr(sm.act[S][0]), 20, L_bt, sh1, 4 * wave, 1, 2 * ngc, n, kq, accg);
        chunk_mfma<4>(lds_addr(sm.act[S][1]), 20, L_bt, sh1, 16 + 4 * wave, 1, 16 + 2 * ngc, n, kq, accu);
      };
      run_chunks<kInt8>(mine, sh1, nc1, block, L_lut, L_bt, rg, issue, store, mfma);
    }
    // h = SiLU(g) u (x router weight before down) of the wave's 64 columns,
    // fp16 with one exponent per row (the maximum over the item's columns).
    float hv[4][4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = kq * 4 + v;
      const float sg = ldexpf(1.0f, -sm.rexp[0][row]), su = ldexpf(1.0f, -sm.rexp[1][row]);
      const float wr = p.wbd && row < m ? p.pair_w[s0 + tb + row] : 1.0f;
      float mx = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = 64 * wave + 16 * j + n;
        const float g = accg[j][v] * sg, u = accu[j][v] * su;
        hv[j][v] = col < ncol && row < m ? g / (1.0f + expf(-g)) * u * wr : 0.f;
        mx = fmaxf(mx, fabsf(hv[j][v]));
      }
      mx = op_over(mx, 1, 16, OpMax{});
      if (n == 0) sm.hmax[wave][row] = mx;
    }
    lds_barrier();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = kq * 4 + v;
      const float mx = fmaxf(fmaxf(sm.hmax[0][row], sm.hmax[1][row]), fmaxf(sm.hmax[2][row], sm.hmax[3][row]));
      const int ex = pow2_row_exponent(mx);
      if (wave == 0 && n == 0) sm.hexp[row] = ex;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = 64 * wave + 16 * j + n;
        const _Float16 hh = static_cast<_Float16>(ldexpf(hv[j][v], ex));
        lds_st<_Float16>(L_h + static_cast<uint32_t>(row * kHDw * 4 + col * 2), hh);
      }
    }
    lds_barrier();
    // Stage 2: d latent partial of these 256 rows of A_d.
    // (One run-time shape: a compile-time one per group count spilled.)
    if (ngd > 0) {
      const DynShape sh2 = dyn_shape(ngd);
      const int nc2 = (ncol + sh2.rows - 1) / sh2.rows;
      float4v accd[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) accd[j] = float4v{0.f, 0.f, 0.f, 0.f};
      const Src sd = make_src(fad, e, c0, c0 + ncol, 0, ngd, tid & (sh2.ngp - 1), tid / sh2.ngp);
      auto none = [&](int, auto) __attribute__((always_inline)) {};
      Ring<kInt8> rg;
      auto mfma = [&](int c) __attribute__((always_inline)) {
        chunk_mfma<8>(L_h + static_cast<uint32_t>(c * sh2.rows) * 2u, kHDw, L_bt, sh2, wave, 4, 2 * ngd, n, kq, accd);
      };
      run_chunks<kInt8>(sd, sh2, nc2, sd.gi, L_lut, L_bt, rg, none, none, mfma);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int cb = wave + 4 * j;
        const int col = cb * 16 + n;
        if (cb < 2 * ngd && col < rd) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = kq * 4 + v;
            if (row < m)
              atomic_add_f32(p.dl + static_cast<int64_t>(s0 + tb + row) * p.R + col,
                             accd[j][v] * ldexpf(1.0f, -sm.hexp[row]));
          }
        }
      }
    }
    lds_barrier();
  }
}

// ---------------------------------------------------------------------------
// Phase D: d_lat . B_d over 512 columns of d, weighted into out
// ---------------------------------------------------------------------------
struct alignas(16) SmemD {
  uint32_t bt[kBtDw];
  uint32_t act[2][kPass * 20];  // d latent rows of a 32-row chunk
  uint32_t lut[256];
  int rexp[kPass];
  int rtok[kPass];
  float rw[kPass];
};

template <bool kInt8>
__global__ void __launch_bounds__(kT, 2) d_kernel(Params p) {
  __shared__ SmemD sm;
  int a, item;
  if (!map_item(blockIdx.x, p.n_d, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int rd = rank_of(p, e, 2);
  const int c0 = item * kCD, ncol = min(kCD, p.d - c0), ngc = ncol / kGroup;
  const Factor& f = p.fac[F_DOWN_B];
  if (mtot == 0) return;
  lut_fill(sm.lut, tid);
  const uint32_t L_lut = lds_addr(sm.lut), L_bt = lds_addr(sm.bt);
  constexpr Shape<16> sh{};  // 32 rows of the rank per chunk
  const int nc = (rd + 31) / 32;
  const Src src = make_src(f, e, 0, rd, c0 / kGroup, ngc, tid & (sh.ngp - 1), tid / sh.ngp);
  for (int tb = 0; tb < mtot; tb += kPass) {
    const int m = min(kPass, mtot - tb);
    {
      const int r = tid >> 4, t = tid & 15;
      float mx = 0.f;
      if (r < m) {
        const float* row = p.dl + static_cast<int64_t>(s0 + tb + r) * p.R;
        for (int c = t; c < rd; c += 16) mx = fmaxf(mx, fabsf(row[c]));
      }
      mx = op_over(mx, 1, 16, OpMax{});
      if (t == 0) {
        sm.rexp[r] = pow2_row_exponent(mx);
        const int pair = s0 + tb + min(r, m - 1);
        sm.rtok[r] = r < m ? p.pair_tok[pair] * p.K + p.pair_slot[pair] : -1;
        sm.rw[r] = p.wbd ? 1.0f : p.pair_w[pair];
      }
    }
    lds_barrier();
    float4v acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
    if (nc > 0) {
      u32x4 lr[2];
      // Thread: row r = tid >> 4 (16 rows), 2 values at 2 (tid & 15) of the chunk's 32.
      auto load_l = [&](int c, u32x4& x) __attribute__((always_inline)) {
        const int r = tid >> 4, q2 = (tid & 15) * 2;
        const int col = min(c, nc - 1) * 32 + q2;
        const bool ok = r < m && col < rd;
        const float* s = p.dl + static_cast<int64_t>(s0 + tb + min(r, m - 1)) * p.R + min(col, p.R - 2);
        const float2 v = *reinterpret_cast<const float2*>(s);
        x = ok ? u32x4{__float_as_uint(v.x), __float_as_uint(v.y), 0u, 0u} : u32x4{0u, 0u, 0u, 0u};
      };
      auto issue = [&](int c, auto slot) __attribute__((always_inline)) { load_l(c, lr[decltype(slot)::value]); };
      auto store = [&](int c, auto slot) __attribute__((always_inline)) {
        constexpr int S = decltype(slot)::value;
        const int r = tid >> 4, q2 = (tid & 15) * 2;
        const half2v h = to_h2(__uint_as_float(lr[S][0]), __uint_as_float(lr[S][1]), sm.rexp[r]);
        lds_st<uint32_t>(lds_addr(sm.act[S]) + static_cast<uint32_t>(r * 20 + q2 / 2) * 4u,
                         __builtin_bit_cast(uint32_t, h));
      };
      Ring<kInt8> rg;
      auto mfma = [&](int c) __attribute__((always_inline)) {
        chunk_mfma<8>(lds_addr(sm.act[c & 1]), 20, L_bt, sh, wave, 4, 2 * ngc, n, kq, acc);
      };
      run_chunks<kInt8>(src, sh, nc, src.gi, L_lut, L_bt, rg, issue, store, mfma);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int cb = wave + 4 * j;
      const int col = cb * 16 + n;
      if (cb < 2 * ngc) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = kq * 4 + v;
          if (row < m) {
            const float y = acc[j][v] * ldexpf(1.0f, -sm.rexp[row]);
            const int ts = sm.rtok[row];  // token * K + slot
            if (p.out_mode == LATENT_OUT_REDUCED)
              atomic_add_f32(p.out + static_cast<int64_t>(ts / p.K) * p.d + c0 + col, sm.rw[row] * y);
            else
              p.out[static_cast<int64_t>(ts) * p.d + c0 + col] = y;
          }
        }
      }
    }
    lds_barrier();
  }
}

}  // namespace

bool supported(const latent_moe_args& a) {
  if (a.layout != LATENT_LAYOUT_ROWS || a.max_rank > 512) return false;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15u) != 0) return false;  // 16-byte loads of x (prep's fp16 rows)
  // INT8 bytes are read through 32-bit buffer offsets: even an all-INT8 side
  // buffer of a factor must stay below 2^31 bytes.
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs) {
    if (!f->int8_bitmap) continue;
    if (a.n_expert * f->rows * f->cols >= (int64_t{1} << 31)) return false;
  }
  return true;
}

void plan(Params& p) {
  // Phase A items per expert and factor: about 4096 items in all, 4 to 16
  // per factor (measured at the DeepSeek-V3 shape with ranks 64..512: 8 at
  // 16, 64 and 256 tokens within 3 % of the best; 2 took 17 % longer, 32 up
  // to 14 %).
  int s = 4;
  while (s < 16 && 2ll * p.a_max * s < 4096) s *= 2;
  p.na_split = s;
  p.n_a = 2 * s;
  p.n_bc = (p.ff + kCB - 1) / kCB;
  p.n_d = (p.d + kCD - 1) / kCD;
}

int launch(const Params& p, bool int8, hipStream_t s) {
  const unsigned groups = static_cast<unsigned>((p.a_max + 7) / 8);
  if (int8) {
    hipLaunchKernelGGL(a_kernel<true>, dim3(8 * groups * p.n_a), dim3(kT), 0, s, p);
    hipLaunchKernelGGL(bc_kernel<true>, dim3(8 * groups * p.n_bc), dim3(kT), 0, s, p);
    hipLaunchKernelGGL(d_kernel<true>, dim3(8 * groups * p.n_d), dim3(kT), 0, s, p);
  } else {
    hipLaunchKernelGGL(a_kernel<false>, dim3(8 * groups * p.n_a), dim3(kT), 0, s, p);
    hipLaunchKernelGGL(bc_kernel<false>, dim3(8 * groups * p.n_bc), dim3(kT), 0, s, p);
    hipLaunchKernelGGL(d_kernel<false>, dim3(8 * groups * p.n_d), dim3(kT), 0, s, p);
  }
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace rows
}  // namespace latent
