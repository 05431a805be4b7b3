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
//   A   x . A_g | A_u              K tiles of 256 rows -> partial latents (reduce A)
//   B   [g | u] = lat . [B_g | B_u], h = SiLU(g) * u
//                                  tiles of 128 gate + 128 up columns, h formed in-lane
//   C   h . A_d                    K tiles of 256 rows -> partial d latent (reduce C)
//   D   d_lat . B_d                N tiles of 256 columns -> y rows, then the combine
//
// The factors are read in the tile layout (latent_tiles_repack, which
// reorders each of the twelve factor tensors in place of the row layout at
// load time): every 256 x 256 block of a factor is 32 KB of NF4 codes in the
// order the lanes consume them, plus its 4 KB of fp16 scales in the factor's
// scale tensor, so each lane reads its MFMA operand bytes with one 128-bit
// load per 32-row step and every tile is one contiguous stream:
//   * wave w owns tile columns 64w .. 64w+63 over all 256 rows; lane
//     (n = lane & 15, kq = lane >> 4) holds, per 32-row step s, the code
//     pairs of rows s*32 + kq*8 + (2q, 2q+1), q = 0..3, for columns
//     64w + 4n + j, j = 0..3 (byte 4j + q, low nibble = even row): dword j
//     is the B operand of v_mfma_f32_16x16x32_f16 number j, whose N block is
//     the columns 4n + j of the wave;
//   * scales: half2 (scale(2P, G), scale(2P + 1, G)) for group G = 0..7 and
//     row pair P at dword G * 128 + (P ^ 8 (G & 1)) (the xor spreads the
//     lanes of one LDS read over all banks);
//   * a phase-B tile is a 128-column half tile of gate_b and the same columns
//     of up_b: for lane n of wave w the columns j = 0, 1 are gate columns
//     32w + 2n + j of the 128-column block and j = 2, 3 the up columns of the
//     same outputs, so each lane forms h = SiLU(g) * u of its two columns
//     itself; each half tile keeps a lane's 16 bytes per K step pair, and its
//     four scale groups become groups 0..3 (gate) and 4..7 (up) in LDS.
// A byte (two rows of one column) is looked up in a 256-entry table of
// (level, level) fp16 pairs in LDS, one copy per LDS bank, and one
// v_pk_mul_f16 by the two rows' scales gives one K pair of the B operand.
//
// Every activation a phase reads is an fp16 row with a power-of-two exponent
// (row maximum in [2^14, 2^15)): the prep kernel writes x that way (one
// exponent per token), the reduce kernels the latents (one per row) and
// phase B h (one per row and 128-column block, in LDS), so the small latents
// of a LATENT chain keep fp16's full precision.
//
// Work split: phase A, phases B and C together (bc_kernel: h never leaves
// LDS) and phase D are each one persistent launch of two workgroups per CU;
// workgroup b takes the contiguous range [b*chunk, (b+1)*chunk) of the
// launch's work list (unit-major), so every workgroup streams the same number
// of tiles.  Tile i + 2's loads are issued while tile i is computed: its codes
// into registers, its scales, activations and exponents into registers that
// are stored to LDS at the end of tile i + 1.  All are ordinary buffer loads,
// so the compiler places every wait.  Phase A accumulates consecutive tiles
// of one (unit, factor) in registers and writes one partial sum per segment;
// phase C writes one per item; the reduce kernels add a row's partials in
// workgroup (item) order.
//
// Arithmetic: fp16 operands (levels and scales exact in fp16 up to one
// rounding of level * scale and of the scaled activation), fp32 accumulation.
// Every sum runs in a fixed order, so results are bit-reproducible.
#include "stream.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace latent {
namespace stream {
namespace {

constexpr int kT = 256;                               // threads per workgroup
constexpr int kK = 256;                               // rows of a tile
constexpr int kN = 256;                               // columns of a tile
constexpr int kSteps = kK / 32;                       // MFMA K steps per tile
constexpr int kCodeBytes = kK * kN / 2;               // 32 KB of a 256 x 256 tile's codes
constexpr int kScaleBytes = kK * kN / kGroup * 2;     // 4 KB of its scales
constexpr int kHBlock = kN / 2;                       // h columns of a phase-B tile
constexpr int kHalfCodeBytes = kCodeBytes / 2;        // a gate_b / up_b half tile: 256 x 128
constexpr int kHalfScaleBytes = kScaleBytes / 2;
constexpr int kLutCopies = 32;                        // one table copy per LDS bank
constexpr int kActChunks = kK / 8;                    // 16-byte chunks of an fp16 activation row
constexpr int kGroupsPerCU = 2;                       // resident workgroups per CU of the item kernels
constexpr int64_t kSpinTicks = 100000000;             // bounded waits: 1 s of s_memrealtime (100 MHz)
constexpr int kCombineBatch = 8;                      // slots' rows in flight per output float4 (combine)
constexpr int kMaxKTiles = 64;                        // small-batch chain: d / 256 at most
constexpr int kRedLoads = 8;                          // partial rows in flight per reduce step
enum Phase { kPhaseA = 0, kPhaseB, kPhaseC, kPhaseD };
// Factor order of latent_moe_args (src3..src14 of the ggml op).
enum { F_GATE_A = 0, F_GATE_B, F_UP_A, F_UP_B, F_DOWN_A, F_DOWN_B, kFactors };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct Params {
  const uint8_t* codes[kFactors];   // the six factors' codes in the tile layout
  const uint8_t* scales[kFactors];  // and their scales (fp16 bits), same order
  const int* meta;        // [4] work units
  const int4* unit_info;  // [units] {expert, first grouped pair, pairs, 0}
  const int* unit_tok;    // [units][16] token of each row
  const int* pos_of;      // [T*K] grouped pair of each routed slot
  const int32_t* ids;
  const void* weights;
  int w_dtype;
  float* out;
  const _Float16* xh;  // [T][d] fp16 x * 2^xexp
  const int* xexp;     // [T]
  float* partA;        // [slots][16][256]
  _Float16* lat;       // [2][P][256]
  int* lexp;           // [2][P]
  _Float16* hh;        // bulk launches: [P][ff] h * 2^hexp
  int* hexp;           // bulk launches: [P][ff/32]
  float* partC;        // decode: [P][nkc][256] by grouped pair; bulk launches: [slots][64][256]
  _Float16* dlat;      // [P][256]
  int* dexp;           // [P]
  float* ybuf;         // [P][d]
  int T, K, E, d, ff, P, wbd, out_mode;
  int nka, nb, nkc, nd;  // tiles per unit and factor: A (d/256), B (ff/128), C (ff/256), D (d/256)
  int G;                 // workgroups the tile ranges are cut for
  // Bulk (prefill) launches only.
  const int* pair_tok;    // [P] token of each grouped pair
  const int* pair_slot;   // [P] slot of each grouped pair
  const float* pair_w;    // [P] router weight of each grouped pair
  const int* nunits;      // number of units (reduce kernels; the decode launches set meta + 4)
  _Float16* yh;           // reduced output: [P][d] fp16 y rows * 2^yexp
  int* yexp;              // [P][d / 128]
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
template <typename T>
__device__ __forceinline__ void lds_st(uint32_t addr, const T& v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr)) = v;
}

// Loads through the scalar unit: the address must be the same in every lane.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int sload(const int* p) { return *(const __attribute__((address_space(4))) int*)(p); }
__device__ __forceinline__ i32x4 sload4(const int4* p) {
  return *(const __attribute__((address_space(4))) i32x4*)(p);
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Raw (byte-addressed) buffer resource over `bytes` bytes from `base`
// (wave-uniform); loads beyond them return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
// Factor tile loads: non-temporal (nt), since a decode step streams each tile
// once; the caches then favour the rows, latents and partial sums that are
// read again (measured: batch 64 250 -> 242 us, batch 8 96 -> 92 us).
constexpr int kTilePolicy = 2;  // cache-policy operand: nt
__device__ __forceinline__ u32x4 ld128_tile(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kTilePolicy);
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
}

// Barrier for LDS data only: this wave's LDS operations complete, then
// s_barrier.  (__syncthreads() would also wait for every outstanding global
// load, which would drain the loads issued ahead for later tiles.)
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// SiLU with the hardware exponential and reciprocal (each within about 1 ulp);
// g -> -inf gives -0, g -> +inf gives g.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Chunk c of activation row r sits at chunk (c ^ (r & 15)) of the row.
__device__ __forceinline__ int act_slot(int row, int chunk) { return row * kActChunks + (chunk ^ (row & 15)); }

// LDS byte offset of the lane's scale dwords of K step 0 in scale group G of a
// tile's scale block; K step s adds 64 s.  (Row pair P of group G sits at
// dword G * 128 + (P ^ 8 (G & 1)), the lane's first pair of step s is
// P = 16 s + 4 kq, and the xor only touches bit 3, below 16 s.)
__device__ __forceinline__ uint32_t scale_lane(int G, int kq) {
  return static_cast<uint32_t>(G * 128 + ((kq * 4) ^ ((G & 1) << 3))) * 4;
}

// ---------------------------------------------------------------------------
// Per-phase shape of the work
// ---------------------------------------------------------------------------
template <int kPhase>
struct Shape {
  static constexpr bool kSliceK = kPhase == kPhaseA || kPhase == kPhaseC;  // tiles along K (partial sums)
  static constexpr int kActBlocks = kPhase == kPhaseB ? 2 : 1;  // activation blocks per tile (B: gate and up latents)
  static constexpr int kActLoads = 2 * kActBlocks;              // 16-byte activation chunks per thread
  static constexpr int kExps = kPhase == kPhaseB || kPhase == kPhaseC ? 32 : 16;
};

// Tiles per unit, and per key (a K-tiled phase's segment: one unit and factor).
template <int kPhase>
__device__ __forceinline__ int tiles_per_unit(const Params& p) {
  return kPhase == kPhaseA ? 2 * p.nka : kPhase == kPhaseB ? p.nb : kPhase == kPhaseC ? p.nkc : p.nd;
}
template <int kPhase>
__device__ __forceinline__ int tiles_per_key(const Params& p) {
  return kPhase == kPhaseA ? p.nka : kPhase == kPhaseC ? p.nkc : 1;
}
// Tiles of a key of the bulk (prefill) launches, the unit of work a
// workgroup takes whole: A a (unit, factor), B, C and D a unit.
template <int kPhase>
__device__ __forceinline__ int bulk_key_tiles(const Params& p) {
  return kPhase == kPhaseA ? p.nka : tiles_per_unit<kPhase>(p);
}

// LDS of the per-phase item kernels (phases A and D), 64 KB in 256 rows of
// 256 bytes.  The first 128 bytes of row b hold the level pair of code byte b
// in 32 copies (copy c at 4 c), so the table address of a code byte is one
// byte permute of the byte and the lane's copy offset (row = byte << 8).  The
// rows' other halves, 32 KB in all, hold the staging of a tile, addressed by
// staging offset o (item_st): the scale blocks [2][4 KB], the activation rows
// [2][16][32 chunks of 16 B] and the row exponents [2][16].  No 16-byte access
// straddles a half row.
struct alignas(16) ItemLds {
  uint32_t w[256 * 64];
};
constexpr uint32_t kStScales = 0;
constexpr uint32_t kStAct = kStScales + 2 * kScaleBytes;
constexpr uint32_t kStExp = kStAct + 2 * kMaxM * kActChunks * 16;
static_assert(kStExp + 2 * 16 * 4 <= 256 * 128, "a tile's staging fits the table rows' second halves");
__device__ __forceinline__ uint32_t item_st(uint32_t o) { return o + (o & ~127u) + 128u; }
// Table address of byte q of code dword x, for the lane's copy offset lc
// (< 128): (byte << 8) | lc.
__device__ __forceinline__ uint32_t lut_addr(uint32_t x, int q, uint32_t lc) {
  return __builtin_amdgcn_perm(x, lc, 0x0C0C0000u | ((4u + q) << 8));
}

// Registers a tile's non-code loads land in before they are stored to LDS.
template <int kPhase>
struct StageAct {
  u32x4 act[Shape<kPhase>::kActLoads];
  int ex;
};

// Phase A's per-lane token rows of a tile: the rows of the thread's two
// activation chunks and of exponent row lane & 15.
struct Toks {
  int a0, a1, e;
};

// Scalar description of a tile: its unit and position in the unit.
struct TileRef {
  int e, start, m, r;  // expert, first grouped pair, pairs, tile index within the unit
};

template <int kPhase>
__device__ __forceinline__ TileRef tile_ref(const Params& p, int t) {
  const int per = tiles_per_unit<kPhase>(p);
  const int u = uniform(t / per);
  const i32x4 info = sload4(p.unit_info + u);
  return TileRef{uniform(info[0]), uniform(info[1]), uniform(info[2]), t - u * per};
}

// The loads below take `valid`: when false they are issued against empty
// buffer ranges, fetch nothing and return zeros, so every step issues the same
// loads and the compiler's wait counts hold on every path.

// Scales and codes of tile idx of factor f (a 256 x 256 tile of gate_a, up_a,
// down_a or down_b): the scale block into `sc` (the dwords of the threads
// `sc_on` selects, zeros elsewhere), K steps [s0, s0 + ns) into cb[0 .. ns).
template <int ns, typename Prm>
__device__ __forceinline__ void load_full(const Prm& p, int f, int idx, bool valid, bool sc_on, int s0, int tid,
                                          int lane, int wave, u32x4& sc, u32x4 (&cb)[kSteps]) {
  const __amdgpu_buffer_rsrc_t rs =
      buffer_rsrc(p.scales[f] + static_cast<int64_t>(idx) * kScaleBytes, valid ? kScaleBytes : 0);
  sc = ld128_tile(rs, sc_on ? tid * 16 : 0x40000000u, 0);
  const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(p.codes[f] + static_cast<int64_t>(idx) * kCodeBytes, valid ? kCodeBytes : 0);
  const uint32_t cbase = wave * (kSteps * kWave * 16) + lane * 16;
#pragma unroll
  for (int s = 0; s < ns; ++s) cb[s] = ld128_tile(rc, cbase, (s0 + s) * kWave * 16);
}

// A phase-B tile, h block idx (expert-major): gate_b's and up_b's half tiles
// of those 128 columns.  Waves 0 and 1 load the gate half tile's 2 KB of
// scales, waves 2 and 3 the up half tile's, so the block in LDS is the gate
// groups 0..3 followed by the up groups 4..7.  cb[0..3] hold the gate half
// tile's K step pairs, cb[4..7] the up half tile's (see code_dword).
template <typename Prm>
__device__ __forceinline__ void load_btile(const Prm& p, int idx, bool valid, int tid, int lane, int wave, u32x4& sc,
                                           u32x4 (&cb)[kSteps]) {
  const int64_t so = static_cast<int64_t>(idx) * kHalfScaleBytes, co = static_cast<int64_t>(idx) * kHalfCodeBytes;
  const __amdgpu_buffer_rsrc_t rs =
      buffer_rsrc((wave < 2 ? p.scales[F_GATE_B] : p.scales[F_UP_B]) + so, valid ? kHalfScaleBytes : 0);
  sc = ld128_tile(rs, (tid & 127) * 16, 0);
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(p.codes[F_GATE_B] + co, valid ? kHalfCodeBytes : 0);
  const __amdgpu_buffer_rsrc_t ru = buffer_rsrc(p.codes[F_UP_B] + co, valid ? kHalfCodeBytes : 0);
  const uint32_t cbase = wave * (kSteps / 2 * kWave * 16) + lane * 16;
#pragma unroll
  for (int sp = 0; sp < kSteps / 2; ++sp) {
    cb[sp] = ld128_tile(rg, cbase, sp * kWave * 16);
    cb[kSteps / 2 + sp] = ld128_tile(ru, cbase, sp * kWave * 16);
  }
}

// Code dword j (the B operand of MFMA j) of K step s of a register tile.  A
// phase-B tile (kB) keeps, per lane, 16 bytes per K step pair of each half
// tile: dwords (s even, j), (s even, j + 1), (s odd, j), (s odd, j + 1) of the
// gate columns (j = 0, 1) in cb[s / 2] and of the up columns (j = 2, 3) in
// cb[4 + s / 2].  Compile-time indices: no register moves.
template <bool kB>
__device__ __forceinline__ uint32_t code_dword(const u32x4 (&cb)[kSteps], int s, int j) {
  if constexpr (kB) return j < 2 ? cb[s >> 1][(s & 1) * 2 + j] : cb[kSteps / 2 + (s >> 1)][(s & 1) * 2 + j - 2];
  else return cb[s][j];
}

// A tile's scale block into `sc`, then its codes into `cb`.
template <int kPhase>
__device__ __forceinline__ void issue_codes(const Params& p, const TileRef& tr, int tid, int lane, int wave, bool valid,
                                            u32x4& sc, u32x4 (&cb)[kSteps]) {
  if constexpr (kPhase == kPhaseA) {
    const int f = tr.r >= p.nka;
    load_full<kSteps>(p, f ? F_UP_A : F_GATE_A, tr.e * p.nka + tr.r - f * p.nka, valid, true, 0, tid, lane, wave, sc, cb);
  } else if constexpr (kPhase == kPhaseB) {
    load_btile(p, tr.e * p.nb + tr.r, valid, tid, lane, wave, sc, cb);
  } else if constexpr (kPhase == kPhaseC) {
    load_full<kSteps>(p, F_DOWN_A, tr.e * p.nkc + tr.r, valid, true, 0, tid, lane, wave, sc, cb);
  } else {
    load_full<kSteps>(p, F_DOWN_B, tr.e * p.nd + tr.r, valid, true, 0, tid, lane, wave, sc, cb);
  }
}

// A tile's activation chunks and row exponents.  Chunk tid + 256 h is 16-byte
// chunk tid % 32 of row (tid / 32 + 8 h) % 16 of activation block h / 2;
// exponent lane l is row l & 15 (of block (l >> 4) & 1 where there are two).
template <int kPhase>
__device__ __forceinline__ void issue_act(const Params& p, const TileRef& tr, const Toks& tk, int tid, int lane,
                                          bool valid, StageAct<kPhase>& st) {
  static_assert(kPhase == kPhaseA || kPhase == kPhaseD, "phases B and C run in bc_kernel");
  const uint32_t live = valid ? 0xFFFFFFFFu : 0u;  // masks every buffer range
  auto pair_of = [&](int r) { return tr.start + min(r, tr.m - 1); };
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
  if constexpr (kPhase == kPhaseA) {
    const int ks = tr.r >= p.nka ? tr.r - p.nka : tr.r;
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(p.xh, (static_cast<uint32_t>(p.T) * p.d * 2) & live);
    const uint32_t col = ks * kK * 2 + chunk * 16;
    st.act[0] = ld128(rx, static_cast<uint32_t>(tk.a0) * p.d * 2 + col, 0);
    st.act[1] = ld128(rx, static_cast<uint32_t>(tk.a1) * p.d * 2 + col, 0);
    const __amdgpu_buffer_rsrc_t re = buffer_rsrc(p.xexp, (p.T * 4) & live);
    st.ex = static_cast<int>(ld32(re, tk.e * 4));
  } else {
    const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(p.dlat, (static_cast<uint32_t>(p.P) * kK * 2) & live);
    st.act[0] = ld128(rl, static_cast<uint32_t>(pair_of(r0)) * kK * 2 + chunk * 16, 0);
    st.act[1] = ld128(rl, static_cast<uint32_t>(pair_of(r0 + 8)) * kK * 2 + chunk * 16, 0);
    const __amdgpu_buffer_rsrc_t re = buffer_rsrc(p.dexp, (p.P * 4) & live);
    st.ex = static_cast<int>(ld32(re, pair_of(lane & 15) * 4));
  }
}

// Store a staged tile into LDS buffer `buf` (L: the item kernel's LDS).
template <int kPhase>
__device__ __forceinline__ void store_stage(uint32_t L, int buf, const u32x4& sc, const StageAct<kPhase>& st, int tid,
                                            int lane, int wave) {
  static_assert(Shape<kPhase>::kActBlocks == 1 && Shape<kPhase>::kExps == 16, "phases A and D");
  lds_st<u32x4>(L + item_st(kStScales + buf * kScaleBytes + tid * 16), sc);
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
#pragma unroll
  for (int h = 0; h < Shape<kPhase>::kActLoads; ++h) {
    const int row = (r0 + 8 * h) % kMaxM;
    lds_st<u32x4>(L + item_st(kStAct + (buf * kMaxM * kActChunks + act_slot(row, chunk)) * 16), st.act[h]);
  }
  if (wave == 0 && lane < 16) lds_st<int>(L + item_st(kStExp + (buf * 16 + lane) * 4), st.ex);
}

// The MFMA steps of a tile: acc[j] += act . (codes dword j, decoded and
// scaled).  L: the item kernel's LDS; lc: the lane's table copy offset.
__device__ __forceinline__ void mfma_steps(uint32_t L, int buf, const u32x4 (&cb)[kSteps], int n, int kq, int wave,
                                           uint32_t lc, float4v (&acc)[4]) {
  // The lane's scale dwords of step s sit 64 s bytes after those of step 0
  // (fewer than 64 bytes into a half row), 128 more per step pair in LDS.
  const uint32_t sc0 = L + item_st(kStScales + buf * kScaleBytes + scale_lane(2 * wave + (n >> 3), kq));
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int chunk = s * 4 + kq;
    const half8 a0 = lds_ld<half8>(L + item_st(kStAct + (buf * kMaxM * kActChunks + act_slot(n, chunk)) * 16));
    const u32x4 sc = lds_ld<u32x4>(sc0 + s * 64 + (s >> 1) * 128);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = cb[s][j];
      uint32_t f[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pr = lds_ld<uint32_t>(L + lut_addr(x, q, lc));
        // Through a scalar: __builtin_bit_cast of a vector element reads element 0.
        const uint32_t sq = sc[q];
        f[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pr) * __builtin_bit_cast(half2v, sq));
      }
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(half8, make_uint4(f[0], f[1], f[2], f[3])),
                                                      acc[j], 0, 0, 0);
    }
  }
}

// Partial-sum slot of segment key `key` in workgroup b's range (K-tiled phases).
__device__ __forceinline__ int part_slot(int b, int key, int chunk, int per_key, int maxj) {
  return b * maxj + key - (b * chunk) / per_key;
}

template <int kPhase>
__global__ void __launch_bounds__(kT, kGroupsPerCU) item_kernel(Params p) {
  static_assert(kPhase == kPhaseA || kPhase == kPhaseD, "phases B and C run in bc_kernel");
  __shared__ ItemLds sm;
  const uint32_t L = lds_addr(sm);
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int per_unit = tiles_per_unit<kPhase>(p), per_key = tiles_per_key<kPhase>(p);
  const int U = uniform(sload(p.meta + 4));
  const int total = U * per_unit;
  const int b = blockIdx.x;
  const int chunk = (total + p.G - 1) / p.G;
  const int lo = b * chunk, hi = min(total, lo + chunk);
  if (lo >= hi) return;
  const int ntile = hi - lo;
  const int maxj = (chunk + per_key - 1) / per_key + 1;

  // Level-pair table: thread tid fills row tid's 32 copies (rotated start, so
  // the lanes of one store spread over the banks).
  {
    const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
    const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_st<u32x4>(L + tid * 256 + ((j + tid) & 7) * 16, u32x4{bits, bits, bits, bits});
  }
  static_assert(kLutCopies == 32, "one table copy per bank of a 32-lane half wave");
  const uint32_t lc = (lane & 31) << 2;

  // Phase A's token rows of tile t (loaded one tile before the tile's loads).
  const int ar0 = tid / kActChunks, ar1 = ar0 + 8;
  auto load_toks = [&](int t, bool valid, Toks& tk) __attribute__((always_inline)) {
    if constexpr (kPhase == kPhaseA) {
      const int u = uniform(min(t, hi - 1) / per_unit);
      const __amdgpu_buffer_rsrc_t ru = buffer_rsrc(p.unit_tok + static_cast<int64_t>(u) * kMaxM, valid ? kMaxM * 4 : 0);
      tk.a0 = static_cast<int>(ld32(ru, ar0 * 4));
      tk.a1 = static_cast<int>(ld32(ru, ar1 * 4));
      tk.e = static_cast<int>(ld32(ru, (lane & 15) * 4));
    }
  };

  u32x4 cb[3][kSteps];
  u32x4 sc[3];
  StageAct<kPhase> sa[3];
  Toks tk[3] = {};
  TileRef ref[3];
  float4v acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};

  // Prologue: tiles 0 and 1 in flight, tile 0 staged in LDS buffer 0.  Tiles
  // past the range (here and in the steps) issue empty loads.
  load_toks(lo, true, tk[0]);
  load_toks(lo + 1, ntile > 1, tk[1]);
  load_toks(lo + 2, ntile > 2, tk[2]);
  ref[0] = tile_ref<kPhase>(p, lo);
  ref[1] = tile_ref<kPhase>(p, min(lo + 1, hi - 1));
  issue_act<kPhase>(p, ref[0], tk[0], tid, lane, true, sa[0]);
  issue_codes<kPhase>(p, ref[0], tid, lane, wave, true, sc[0], cb[0]);
  issue_act<kPhase>(p, ref[1], tk[1], tid, lane, ntile > 1, sa[1]);
  issue_codes<kPhase>(p, ref[1], tid, lane, wave, ntile > 1, sc[1], cb[1]);
  store_stage<kPhase>(L, 0, sc[0], sa[0], tid, lane, wave);

  // Tile i sits in slot c = i % 3; tiles i + 1 and i + 2 in the other two.
  auto step = [&](int i, auto cs) __attribute__((always_inline)) {
    constexpr int c = decltype(cs)::value, c1 = (c + 1) % 3, c2 = (c + 2) % 3;
    const int buf = i & 1;
    lds_barrier();  // LDS buffer `buf` holds tile i; every wave is done with tile i - 1
    // Loads of tile i + 2.
    load_toks(lo + i + 3, i + 3 < ntile, tk[c]);
    ref[c2] = tile_ref<kPhase>(p, min(lo + i + 2, hi - 1));
    issue_act<kPhase>(p, ref[c2], tk[c2], tid, lane, i + 2 < ntile, sa[c2]);
    issue_codes<kPhase>(p, ref[c2], tid, lane, wave, i + 2 < ntile, sc[c2], cb[c2]);
    const TileRef& tr = ref[c];
    mfma_steps(L, buf, cb[c], n, kq, wave, lc, acc);
    const int t = lo + i;
    if constexpr (kPhase == kPhaseA) {
      // End of a segment (last tile of the range or of this key): one partial.
      if (i + 1 == ntile || (t + 1) % per_key == 0) {
        const int key = t / per_key;
        float* part = p.partA + static_cast<int64_t>(part_slot(b, key, chunk, per_key, maxj)) * kMaxM * kN;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = kq * 4 + v;
          if (row < tr.m) {
            // x's one exponent per token is the same in every tile.
            const float sc = ldexpf(1.0f, -lds_ld<int>(L + item_st(kStExp + (buf * 16 + row) * 4)));
            *reinterpret_cast<float4*>(part + row * kN + wave * 64 + n * 4) =
                make_float4(acc[0][v] * sc, acc[1][v] * sc, acc[2][v] * sc, acc[3][v] * sc);
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
      }
    } else {
      // D: the y rows of the tile's 256 columns, by grouped pair.
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = kq * 4 + v;
        if (row < tr.m) {
          const float sc = ldexpf(1.0f, -lds_ld<int>(L + item_st(kStExp + (buf * 16 + row) * 4)));
          float* dst = p.ybuf + static_cast<int64_t>(tr.start + row) * p.d + tr.r * kN + wave * 64 + n * 4;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[0][v] * sc, acc[1][v] * sc, acc[2][v] * sc, acc[3][v] * sc);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
    }
    // Tile i + 1's scales and activations into the other LDS buffer (last
    // read by tile i - 1, which every wave finished before this step's barrier).
    store_stage<kPhase>(L, buf ^ 1, sc[c1], sa[c1], tid, lane, wave);
  };
  // Whole triples without branches between the steps, then the last one or two.
  int i = 0;
  for (; i + 3 <= ntile; i += 3) {
    step(i, std::integral_constant<int, 0>{});
    step(i + 1, std::integral_constant<int, 1>{});
    step(i + 2, std::integral_constant<int, 2>{});
  }
  if (i < ntile) step(i, std::integral_constant<int, 0>{});
  if (i + 1 < ntile) step(i + 1, std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// Phases B and C in one launch (bc_kernel)
// ---------------------------------------------------------------------------
// Item (unit, j), j < ff / 256: B tiles 2j and 2j + 1 (h for ff columns
// 256 j .. 256 j + 255, two 128-column blocks with one exponent per row each,
// kept in LDS) and C tile j (those h columns times A_d's rows 256 j ..).  A
// workgroup's range is whole items, so its tile sequence is B, B, C, B, B, C,
// ...: tile i sits in register slot i % 3 and its kind is i % 3 (0, 1: the
// item's B tiles, 2: its C tile).  The gate / up latents of an item's unit are
// staged during the previous item's C tile.  Every C tile writes its own
// partial d latent (slot = item), which reduce_kernel<kPhaseC, .., true> sums
// in item order.
// LDS: the item kernels' 64 KB of table rows (ItemLds) whose second halves
// hold the gate / up latents of the current item's unit (staging offset
// kBcAct, [2][16][32 chunks]) and h of the item's two 128-column blocks
// (kBcHb, [2][16][16 chunks], a row's chunks at its first 16 slots), then the
// scale blocks and the row exponents.
struct alignas(16) BcSmem {
  ItemLds rows;
  u32x4 scales[2][kScaleBytes / 16];   // [buffer]: the tile's scale block
  int lexp[2][kMaxM];                  // latent exponents
  int hexp[2][kMaxM];                  // h exponents per block
  float hmax[4][kMaxM];                // per-wave row maxima of h
};
constexpr uint32_t kBcAct = 0;
constexpr uint32_t kBcHb = kBcAct + 2 * kMaxM * kActChunks * 16;
static_assert(kBcHb + 2 * kMaxM * kActChunks * 16 <= 256 * 128, "latents and h fit the table rows' second halves");

// MFMA steps [s0, s0 + ns) of a register tile: activation chunk 4 (s - s0) + kq
// of act0 (and act1 for the up columns of a B tile), scale rows of step s.
template <bool kTwo, int s0, int ns>
__device__ __forceinline__ void bc_mfma(uint32_t L, uint32_t act0, uint32_t act1, uint32_t sbase,
                                        const u32x4 (&cb)[kSteps], int n, int kq, int wave, uint32_t lc,
                                        float4v (&acc)[4]) {
#pragma unroll
  for (int r = 0; r < ns; ++r) {
    const int s = s0 + r;
    const int chunk = r * 4 + kq;
    const half8 a0 = lds_ld<half8>(L + item_st(act0 + act_slot(n, chunk) * 16));
    const int S0 = s;  // K step (scale rows)
    u32x4 sc0, sc1;
    half8 a1;
    if constexpr (kTwo) {
      a1 = lds_ld<half8>(L + item_st(act1 + act_slot(n, chunk) * 16));
      const int Gg = wave, Gu = 4 + wave;
      sc0 = lds_ld<u32x4>(sbase + scale_lane(Gg, kq) + S0 * 64);
      sc1 = lds_ld<u32x4>(sbase + scale_lane(Gu, kq) + S0 * 64);
    } else {
      const int G = 2 * wave + (n >> 3);
      sc0 = lds_ld<u32x4>(sbase + scale_lane(G, kq) + S0 * 64);
      sc1 = sc0;
      a1 = a0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = code_dword<kTwo>(cb, s, j);
      const u32x4 sc = j < 2 ? sc0 : sc1;
      uint32_t f[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pr = lds_ld<uint32_t>(L + lut_addr(x, q, lc));
        const uint32_t sq = sc[q];  // through a scalar: a bit_cast of a vector element reads element 0
        f[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pr) * __builtin_bit_cast(half2v, sq));
      }
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(j < 2 ? a0 : a1,
                                                      __builtin_bit_cast(half8, make_uint4(f[0], f[1], f[2], f[3])),
                                                      acc[j], 0, 0, 0);
    }
  }
}

__global__ void __launch_bounds__(kT, kGroupsPerCU) bc_kernel(Params p) {
  __shared__ BcSmem sm;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int U = uniform(sload(p.meta + 4));
  const int total = U * p.nkc;
  const int b = blockIdx.x;
  const int chunk = (total + p.G - 1) / p.G;
  const int lo = b * chunk, hi = min(total, lo + chunk);
  if (lo >= hi) return;
  const int ntile = 3 * (hi - lo);
  const uint32_t L = lds_addr(sm.rows);
  {
    const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
    const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_st<u32x4>(L + tid * 256 + ((j + tid) & 7) * 16, u32x4{bits, bits, bits, bits});
  }
  const uint32_t lc = (lane & 31) << 2;
  const int r0 = tid / kActChunks, ch = tid % kActChunks;

  // Codes and scales of tile t of the range (loads past the range fetch
  // nothing): a B tile (kind 0, 1) is the gate_b and up_b half tiles of h
  // block 2 j + kind (as load_btile lays them out), a C tile (kind 2) down_a's
  // tile j (as load_full).  Both kinds issue the same loads, one scale block
  // and eight code quads, and the kind selects only their bases and offsets:
  // with a branch between two load sequences the compiler's wait counts,
  // merged over both paths, waited for every load, including those just
  // issued for the tile two steps ahead.
  auto issue_codes = [&](int t, u32x4& sc, u32x4 (&cb)[kSteps]) __attribute__((always_inline)) {
    const int tt = min(t, ntile - 1);
    const int it = lo + tt / 3, kind = tt % 3;
    const int u = it / p.nkc, j = it - u * p.nkc;
    const int e = uniform(sload4(p.unit_info + u)[0]);
    const bool bt = kind < 2, valid = t < ntile;
    const int64_t hb = static_cast<int64_t>(e) * p.nb + 2 * j + kind;  // B: half tile of gate_b / up_b
    const int64_t ct = static_cast<int64_t>(e) * p.nkc + j;            // C: tile of down_a
    const uint8_t* sbase = bt ? (wave < 2 ? p.scales[F_GATE_B] : p.scales[F_UP_B]) + hb * kHalfScaleBytes
                              : p.scales[F_DOWN_A] + ct * kScaleBytes;
    const uint8_t* c0 = bt ? p.codes[F_GATE_B] + hb * kHalfCodeBytes : p.codes[F_DOWN_A] + ct * kCodeBytes;
    const uint8_t* c1 = bt ? p.codes[F_UP_B] + hb * kHalfCodeBytes : c0;
    const uint32_t cbytes = valid ? (bt ? kHalfCodeBytes : kCodeBytes) : 0u;
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sbase, valid ? (bt ? kHalfScaleBytes : kScaleBytes) : 0u);
    sc = ld128_tile(rs, bt ? (tid & 127) * 16 : tid * 16, 0);
    const __amdgpu_buffer_rsrc_t r0 = buffer_rsrc(c0, cbytes), r1 = buffer_rsrc(c1, cbytes);
    const uint32_t cbase = (bt ? wave * (kSteps / 2 * kWave * 16) : wave * (kSteps * kWave * 16)) + lane * 16;
#pragma unroll
    for (int q = 0; q < kSteps; ++q)
      cb[q] = ld128_tile(q < kSteps / 2 ? r0 : r1, cbase, (bt ? q % (kSteps / 2) : q) * kWave * 16);
  };
  // Gate / up latent rows (rows past the unit's pairs repeat its last pair)
  // and exponents of item it's unit.
  u32x4 st[4];
  int stex = 0;
  auto issue_lat = [&](int it, bool valid) __attribute__((always_inline)) {
    const int u = min(it, hi - 1) / p.nkc;
    const i32x4 info = sload4(p.unit_info + u);
    const int start = uniform(info[1]), m = uniform(info[2]);
    const uint32_t live = valid ? 0xFFFFFFFFu : 0u;
    const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(p.lat, (2u * p.P * kK * 2) & live);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int row = (r0 + 8 * h) % kMaxM, f = h / 2;
      st[h] = ld128(rl, (static_cast<uint32_t>(f) * p.P + start + min(row, m - 1)) * kK * 2 + ch * 16, 0);
    }
    const __amdgpu_buffer_rsrc_t re = buffer_rsrc(p.lexp, (2u * p.P * 4) & live);
    stex = static_cast<int>(ld32(re, (((lane >> 4) & 1) * p.P + start + min(lane & 15, m - 1)) * 4));
  };
  auto store_lat = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
      lds_st<u32x4>(L + item_st(kBcAct + ((h / 2) * kMaxM * kActChunks + act_slot((r0 + 8 * h) % kMaxM, ch)) * 16), st[h]);
    if (wave == 0 && lane < 32) sm.lexp[lane >> 4][lane & 15] = stex;
  };

  u32x4 cb[3][kSteps], sc[3];
  issue_lat(lo, true);
  issue_codes(0, sc[0], cb[0]);
  issue_codes(1, sc[1], cb[1]);
  sm.scales[0][tid] = sc[0];
  store_lat();

  auto step = [&](int i, auto cs) __attribute__((always_inline)) {
    constexpr int c = decltype(cs)::value, c1 = (c + 1) % 3, c2 = (c + 2) % 3;
    const int buf = i & 1;
    const int it = lo + i / 3;
    const int m = uniform(sload4(p.unit_info + it / p.nkc)[2]);
    lds_barrier();  // LDS buffer `buf` holds tile i; every wave is done with tile i - 1
    // C tile: the next item's latents first (loads complete in order, so the
    // wait for them at the end of this step leaves tile i + 2's in flight).
    if constexpr (c == 2) issue_lat(it + 1, i + 1 < ntile);
    issue_codes(i + 2, sc[c2], cb[c2]);
    const uint32_t sbase = lds_addr(sm.scales[buf][0]);
    if constexpr (c < 2) {
      float4v accB[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) accB[j] = float4v{0.f, 0.f, 0.f, 0.f};
      bc_mfma<true, 0, kSteps>(L, kBcAct, kBcAct + kMaxM * kActChunks * 16, sbase, cb[c], n, kq, wave, lc, accB);
      // h = SiLU(g) * u of columns 32w + 2n + jj of block c, fp16 with one exponent per row.
      float hv[2][4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = kq * 4 + v;
        const float sg = ldexpf(1.0f, -sm.lexp[0][row]), su = ldexpf(1.0f, -sm.lexp[1][row]);
        float mx = 0.f;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          hv[jj][v] = silu(accB[jj][v] * sg) * (accB[jj + 2][v] * su);
          mx = fmaxf(mx, fabsf(hv[jj][v]));
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
        half2v h2;
        h2[0] = static_cast<_Float16>(ldexpf(hv[0][v], ex));
        h2[1] = static_cast<_Float16>(ldexpf(hv[1][v], ex));
        lds_st<half2v>(L + item_st(kBcHb + (c * kMaxM * kActChunks + act_slot(row, 4 * wave + (n >> 2))) * 16 + (n & 3) * 4),
                       h2);
        if (wave == 0 && n == 0) sm.hexp[c][row] = ex;
      }
    } else {
      // K rows 0..127 of the C tile take h block 0, rows 128..255 block 1;
      // each half's products are scaled back before they join the sum.
      float4v accC[4], part[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) accC[j] = part[j] = float4v{0.f, 0.f, 0.f, 0.f};
      constexpr uint32_t kHb1 = kBcHb + kMaxM * kActChunks * 16;
      bc_mfma<false, 0, kSteps / 2>(L, kBcHb, kBcHb, sbase, cb[c], n, kq, wave, lc, accC);
      bc_mfma<false, kSteps / 2, kSteps / 2>(L, kHb1, kHb1, sbase, cb[c], n, kq, wave, lc, part);
      // The item's partial rows by grouped pair: row (pair * nkc + j).
      const int iu = it / p.nkc, ij = it - iu * p.nkc;
      const int istart = uniform(sload4(p.unit_info + iu)[1]);
      float* dst = p.partC + (static_cast<int64_t>(istart) * p.nkc + ij) * kN;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = kq * 4 + v;
        const float s0 = ldexpf(1.0f, -sm.hexp[0][row]), s1 = ldexpf(1.0f, -sm.hexp[1][row]);
        if (row < m)
          *reinterpret_cast<float4*>(dst + static_cast<int64_t>(row) * p.nkc * kN + wave * 64 + n * 4) =
              make_float4(fmaf(part[0][v], s1, accC[0][v] * s0), fmaf(part[1][v], s1, accC[1][v] * s0),
                          fmaf(part[2][v], s1, accC[2][v] * s0), fmaf(part[3][v], s1, accC[3][v] * s0));
      }
      // The next item's latents (the B tiles that read the old ones are done).
      store_lat();
    }
    // Tile i + 1's scales into the other buffer (last read by tile i - 1).
    sm.scales[buf ^ 1][tid] = sc[c1];
  };
  for (int i = 0; i < ntile; i += 3) {
    step(i, std::integral_constant<int, 0>{});
    step(i + 1, std::integral_constant<int, 1>{});
    step(i + 2, std::integral_constant<int, 2>{});
  }
}

// A row of 256 sums -> fp16 row * 2^e and e (one wave, 4 columns per lane).
__device__ __forceinline__ void finish_row(float4 s, _Float16* dst, int* dexp, int lane) {
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

// How a bulk launch deals its keys (runs of `per_key` consecutive tiles that
// share activations: A a (unit, factor), B, C and D a unit) to workgroups.
// Workgroup b runs on XCD x = b % 8 (workgroups go to the XCDs round robin),
// as the j = b / 8-th of that XCD's J = G / 8.  XCD x takes the contiguous
// block [K x / 8, K (x + 1) / 8) of the key list (unit-major, so an expert's
// keys are neighbours, and a unit's gate and up keys too):
//   * F = (its keys) / J full rounds: workgroup j takes keys j, j + J, ...
//     whole, so the XCD's workgroups that run at the same time work on the
//     keys of one expert, reading the same factor tile at the same K step
//     and the same unit's activation slices: all but the first read of each
//     hit that XCD's L2;
//   * the rest (fewer than J keys) as even tile ranges of c tiles, so every
//     workgroup ends within one tile of the others.
// A partial sum of a K-tiled phase (A, C) belongs to a whole key (slot =
// key) or to a piece of a rest key: slot 2 U + (x J + j) * kRemPieces + the
// piece's key ordinal in workgroup j's range (a range of at most per_key
// tiles meets at most two keys).
struct Deal {
  int kx0, F, J, rest0, T_rem, c;  // XCD's first key, full rounds, workgroups, first rest key, rest tiles, range
};
__host__ __device__ inline Deal deal_for(int nkey, int per_key, int G, int xcd) {
  Deal d;
  d.J = G >> 3;
  d.kx0 = static_cast<int>(static_cast<int64_t>(nkey) * xcd / 8);
  const int kx1 = static_cast<int>(static_cast<int64_t>(nkey) * (xcd + 1) / 8);
  d.F = (kx1 - d.kx0) / d.J;
  d.rest0 = d.kx0 + d.F * d.J;
  d.T_rem = (kx1 - d.rest0) * per_key;
  d.c = (d.T_rem + d.J - 1) / d.J;
  return d;
}
constexpr int kRemPieces = 2;  // rest pieces per workgroup range (<= per_key tiles)

// lat (phase A) / dlat (phase C) rows: the partial sums of each (unit,
// factor, row) added in workgroup order.  One wave per (key, row); units of
// at most kRows pairs (partial blocks of kRows rows).
// kPerItem: phase C's partials are one per item (bc_kernel), row (pair * nkc
// + j) for item j of a unit, summed in item order.  kByKey: the bulk launches' slots (Deal): a whole
// key's one partial, or a rest key's pieces in workgroup order.
template <int kPhase, int kRows, bool kPerItem = false, bool kByKey = false>
__global__ void __launch_bounds__(kT) reduce_kernel(Params p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int per_unit = tiles_per_unit<kPhase>(p), per_key = tiles_per_key<kPhase>(p);
  const int keys_per_unit = per_unit / per_key;
  const int U = *p.nunits;
  const int total = U * per_unit;
  const int chunk = (total + p.G - 1) / p.G;
  const int maxj = (chunk + per_key - 1) / per_key + 1;
  float* part = kPhase == kPhaseA ? p.partA : p.partC;
  const int nkey = U * keys_per_unit;
  const int J = p.G >> 3;
  // kByKey, phase C: the rest keys only (fewer than J per XCD).  A whole
  // key's workgroup left its sum in the key's slot; a rest key's pieces are
  // summed into that slot here, and phase D finishes both as it stages them.
  // Phase A: every key, finished here (phase B stages two latent blocks per
  // unit, and finishing them there measured slower).
  constexpr bool kRestOnly = kByKey && kPhase == kPhaseC;
  if constexpr (kByKey) {
    // A wave takes kRowsPerWave rows of one key, so the key's dealing and
    // unit are looked up once and those rows' partials are in flight together
    // (one row per wave left each wave with about ten rows in turn, two
    // dependent round trips each).  Pieces in workgroup order.
    constexpr int kRowsPerWave = 8;
    constexpr int kGroups = kRows / kRowsPerWave;
    static_assert(kRows % kRowsPerWave == 0, "whole row groups");
    const int nw = (kRestOnly ? 8 * J : nkey) * kGroups;
    for (int w = blockIdx.x * (kT / kWave) + static_cast<int>(threadIdx.x >> 6); w < nw;
         w += gridDim.x * (kT / kWave)) {
      int key, row0, xcd = 0;
      Deal dl;
      if constexpr (kRestOnly) {
        xcd = uniform(w / (J * kGroups));
        dl = deal_for(nkey, per_key, p.G, xcd);
        key = dl.rest0 + uniform(w / kGroups) % J;
        row0 = (w % kGroups) * kRowsPerWave;
        if (key >= static_cast<int>(static_cast<int64_t>(nkey) * (xcd + 1) / 8)) continue;
      } else {
        key = uniform(w / kGroups);
        row0 = (w - key * kGroups) * kRowsPerWave;
        while (xcd < 7 && key >= static_cast<int>(static_cast<int64_t>(nkey) * (xcd + 1) / 8)) ++xcd;
        dl = deal_for(nkey, per_key, p.G, xcd);
      }
      const int u = key / keys_per_unit, f = key - u * keys_per_unit;
      const int4 info = p.unit_info[u];
      if (row0 >= info.z) continue;
      const int rk = key - dl.rest0;
      const int b0 = rk < 0 ? -1 : rk * per_key / dl.c, b1 = rk < 0 ? -1 : ((rk + 1) * per_key - 1) / dl.c;
      float4 s[kRowsPerWave];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) s[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int b = b0; b <= b1; ++b) {
        const int64_t slot =
            b < 0 ? key : 2 * U + (xcd + 8 * b) * kRemPieces + key - (dl.rest0 * per_key + b * dl.c) / per_key;
        float4 v[kRowsPerWave];
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r)
          v[r] = row0 + r < info.z ? reinterpret_cast<const float4*>(part + (slot * kRows + row0 + r) * kN)[lane]
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
          s[r].x += v[r].x; s[r].y += v[r].y; s[r].z += v[r].z; s[r].w += v[r].w;
        }
      }
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) {
        if (row0 + r < info.z) {
          const int64_t pair = info.y + row0 + r;
          if constexpr (kRestOnly)
            reinterpret_cast<float4*>(part + (static_cast<int64_t>(key) * kRows + row0 + r) * kN)[lane] = s[r];
          else
            finish_row(s[r], p.lat + (static_cast<int64_t>(f) * p.P + pair) * kK, p.lexp + f * p.P + pair, lane);
        }
      }
    }
    return;
  }
  for (int w = blockIdx.x * (kT / kWave) + static_cast<int>(threadIdx.x >> 6); w < nkey * kRows;
       w += gridDim.x * (kT / kWave)) {
    const int row = w % kRows;
    const int key = w / kRows;
    const int u = key / keys_per_unit, f = key - u * keys_per_unit;
    const int4 info = p.unit_info[u];
    if (row >= info.z) continue;
    const int b0 = kPerItem ? key * per_key : (key * per_key) / chunk;
    const int b1 = kPerItem ? key * per_key + per_key - 1 : (key * per_key + per_key - 1) / chunk;
    // Batches of kRedLoads partials in flight, summed in workgroup (item) order.
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int bb = b0; bb <= b1; bb += kRedLoads) {
      float4 v[kRedLoads];
#pragma unroll
      for (int q = 0; q < kRedLoads; ++q) {
        const int b = min(bb + q, b1);
        int64_t rowoff;  // float offset of the partial row
        if constexpr (kPerItem)
          rowoff = (static_cast<int64_t>(info.y + row) * per_key + (b - key * per_key)) * kN;  // by grouped pair
        else
          rowoff = (static_cast<int64_t>(part_slot(b, key, chunk, per_key, maxj)) * kRows + row) * kN;
        // Only the batch's live partials are read (b1 is wave-uniform).
        v[q] = bb + q <= b1 ? reinterpret_cast<const float4*>(part + rowoff)[lane] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int q = 0; q < kRedLoads; ++q) {
        if (bb + q <= b1) {
          s.x += v[q].x; s.y += v[q].y; s.z += v[q].z; s.w += v[q].w;
        }
      }
    }
    const int64_t pair = info.y + row;
    if (kPhase == kPhaseA)
      finish_row(s, p.lat + (static_cast<int64_t>(f) * p.P + pair) * kK, p.lexp + f * p.P + pair, lane);
    else
      finish_row(s, p.dlat + pair * kK, p.dexp + pair, lane);
  }
}

// out from the y rows of the routed slots, in slot order: reduced mode sums
// w * y over the token's slots; per-slot mode writes y (times w when the weight
// goes before the down projection: y is linear in h) and zero for a dropped slot.
// d % 256 == 0, so the 64 float4 columns of a wave lie in one output row: the
// slot's id, weight and grouped position are wave-uniform (scalar loads), and
// the y rows of kCombineBatch slots are loaded before any is added.
__global__ void __launch_bounds__(kT) combine_kernel(Params p) {
  const int64_t d4 = p.d / 4;
  const int64_t rows = p.out_mode == LATENT_OUT_REDUCED ? p.T : static_cast<int64_t>(p.T) * p.K;
  const int64_t n4 = rows * d4;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; i < n4; i += static_cast<int64_t>(gridDim.x) * kT) {
    const int r = uniform(static_cast<int>(i / d4));
    const int64_t c4 = i - static_cast<int64_t>(r) * d4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p.out_mode == LATENT_OUT_REDUCED) {
      for (int k0 = 0; k0 < p.K; k0 += kCombineBatch) {
        float4 v[kCombineBatch];
        float w[kCombineBatch];
        bool ok[kCombineBatch];
#pragma unroll
        for (int q = 0; q < kCombineBatch; ++q) {
          const int slot = r * p.K + min(k0 + q, p.K - 1);
          const int e = p.ids[slot];
          ok[q] = k0 + q < p.K && e >= 0 && e < p.E;
          w[q] = load_act(p.weights, p.w_dtype, slot);
          const int pos = ok[q] ? p.pos_of[slot] : 0;
          v[q] = reinterpret_cast<const float4*>(p.ybuf + static_cast<int64_t>(pos) * p.d)[c4];
        }
#pragma unroll
        for (int q = 0; q < kCombineBatch; ++q) {
          if (ok[q]) {
            s.x += w[q] * v[q].x; s.y += w[q] * v[q].y; s.z += w[q] * v[q].z; s.w += w[q] * v[q].w;
          }
        }
      }
    } else {
      const int e = p.ids[r];
      if (e >= 0 && e < p.E) {
        s = reinterpret_cast<const float4*>(p.ybuf + static_cast<int64_t>(p.pos_of[r]) * p.d)[c4];
        if (p.wbd) {
          const float w = load_act(p.weights, p.w_dtype, r);
          s.x *= w; s.y *= w; s.z *= w; s.w *= w;
        }
      }
    }
    reinterpret_cast<float4*>(p.out)[i] = s;
  }
}

// ---------------------------------------------------------------------------
// Helpers of the small-batch chain (lite_kernel)
// ---------------------------------------------------------------------------
// Coherent (sc1) 128-bit load and store: agent-scope, seen across XCDs.
__device__ __forceinline__ float4 ld_coh4(const float* base, uint32_t voff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(base, 0x7FFFFFFF), voff, 0, 16);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ void st_coh4(float* base, uint32_t voff, float4 v) {
  const u32x4 w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(w, buffer_rsrc(base, 0x7FFFFFFF), voff, 0, 16);
}
__device__ __forceinline__ void add4(float4& a, const float4& b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

// Balanced split of N items over G workgroups (N * G < 2^32).
__device__ __forceinline__ int range_lo(int N, int b, int G) {
  return static_cast<int>(static_cast<uint32_t>(N) * static_cast<uint32_t>(b) / static_cast<uint32_t>(G));
}

// MFMA steps over code registers cb[0 .. ns): register step r is K step
// srow0 + r of the tile (its scale rows) and activation chunk step r.
// acc[j] += act . (codes dword j, decoded and scaled); act1 feeds the up
// columns of a B tile (kTwo).
// L: the workgroup's table rows (ItemLds); act0 / act1: staging offsets of
// the activation blocks; lc: the lane's table copy offset.
template <bool kTwo, int ns>
__device__ __forceinline__ void reg_mfma(uint32_t L, uint32_t act0, uint32_t act1, uint32_t sbase,
                                          const u32x4 (&cb)[kSteps], int srow0, int n, int kq, int wave,
                                          uint32_t lc, float4v (&acc)[4]) {
#pragma unroll
  for (int r = 0; r < ns; ++r) {
    const int chunk = r * 4 + kq;
    const half8 a0 = lds_ld<half8>(L + item_st(act0 + act_slot(n, chunk) * 16));
    const int S0 = srow0 + r;  // K step (scale rows)
    u32x4 sc0, sc1;
    half8 a1;
    if constexpr (kTwo) {
      a1 = lds_ld<half8>(L + item_st(act1 + act_slot(n, chunk) * 16));
      const int Gg = wave, Gu = 4 + wave;
      sc0 = lds_ld<u32x4>(sbase + scale_lane(Gg, kq) + S0 * 64);
      sc1 = lds_ld<u32x4>(sbase + scale_lane(Gu, kq) + S0 * 64);
    } else {
      const int G = 2 * wave + (n >> 3);
      sc0 = lds_ld<u32x4>(sbase + scale_lane(G, kq) + S0 * 64);
      sc1 = sc0;
      a1 = a0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = code_dword<kTwo>(cb, r, j);
      const u32x4 sc = j < 2 ? sc0 : sc1;
      uint32_t f[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pr = lds_ld<uint32_t>(L + lut_addr(x, q, lc));
        const uint32_t sq = sc[q];
        f[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pr) * __builtin_bit_cast(half2v, sq));
      }
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(j < 2 ? a0 : a1,
                                                      __builtin_bit_cast(half8, make_uint4(f[0], f[1], f[2], f[3])),
                                                      acc[j], 0, 0, 0);
    }
  }
}

// A row of 256 sums (four per lane) -> fp16 row * 2^e in an LDS activation
// block (chunk layout of act_slot, at staging offset blk of the table rows L)
// and its exponent.
__device__ __forceinline__ void finish_row_lds(float4 s, uint32_t L, uint32_t blk, int* exps, int r, int lane) {
  const float mx = op_over(fmaxf(fmaxf(fabsf(s.x), fabsf(s.y)), fmaxf(fabsf(s.z), fabsf(s.w))), 1, kWave, OpMax{});
  const int ex = pow2_row_exponent(mx);
  half4v h;
  h[0] = static_cast<_Float16>(ldexpf(s.x, ex));
  h[1] = static_cast<_Float16>(ldexpf(s.y, ex));
  h[2] = static_cast<_Float16>(ldexpf(s.z, ex));
  h[3] = static_cast<_Float16>(ldexpf(s.w, ex));
  lds_st<half4v>(L + item_st(blk + act_slot(r, lane >> 1) * 16 + (lane & 1) * 8), h);
  if (lane == 0) exps[r] = ex;
}

// Every wave's stores (and loads) complete, then a barrier: the workgroup's
// partial sums are visible before its counter adds.
__device__ __forceinline__ void drain_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr int kLiteMaxP = 32;  // routed pairs the small-batch chain takes
constexpr int kLiteSlots = 3;  // tiles a workgroup holds in registers
constexpr int kLiteRed = 16;   // partial rows in flight per lane in the latent sums
// Counters sit on their own cache lines (a line shared by every unit's
// counter serialises all publishes and polls: ~5 us per dependency step).
constexpr int kLiteUnitStride = 32;  // ints between per-unit counters (128 B)
constexpr int kLiteKeyStride = 16;   // ints between (token, tile) counters (64 B)
constexpr int kLiteTicketInts = 32;  // the start-order ticket's line (128 B) before the counters
constexpr int kLiteMaxGrid = 4;      // largest grid, in resident grids
// B, C and D tiles are needed only after A's results: their workgroups issue
// their loads this long after grouping, so A's tiles come first from HBM.
constexpr int64_t kLiteLateTicks = 300;  // 3 us of s_memrealtime (100 MHz)

struct LiteParams {
  const uint8_t* codes[kFactors];   // the six factors in the tile layout (Params' order)
  const uint8_t* scales[kFactors];
  const void* x;
  int x_dtype;
  const int32_t* ids;
  const void* weights;
  int w_dtype;
  float* out;
  float* partA;  // [2][nka][P][256]
  float* partC;  // [nb][P][256]
  float* ybuf;   // [P][d] (reduced output)
  int* cntA;     // [kLiteMaxP][kLiteUnitStride] A tiles done per unit
  int* cntC;     // [kLiteMaxP][kLiteUnitStride] BC items done per unit
  int* cntD;     // [kLiteMaxP][kLiteUnitStride] D tiles done per unit
  int* cntY;     // [T][nd][kLiteKeyStride] routed rows stored per (token, column tile)
  int* ticket;   // start-order ticket (grids beyond the resident workgroups), else null
  int* err;      // set when a bounded wait times out
  int T, K, E, d, P, wbd;
  int nka, nb, nkc, nd;
  int resident;  // workgroups resident at once (two per CU)
};

// Workgroups per role: gB = the BC items, the rest split between A and D in
// proportion to their tiles.
struct LiteSplit {
  int gA, gB, gD;
};
__host__ __device__ inline LiteSplit lite_split(int U, int nka, int nb, int nd, int G) {
  const int64_t NA = 2ll * U * nka, ND = static_cast<int64_t>(U) * nd;
  const int gB = U * nb, R = G - gB;
  int gA = NA + ND > 0 ? static_cast<int>(R * NA / (NA + ND)) : 1;
  gA = gA < 1 ? 1 : (gA > R - 1 ? R - 1 : gA);
  return LiteSplit{gA, gB, R - gA};
}
// Every workgroup's tiles fit its registers (at most kLiteSlots A or D tiles).
__host__ __device__ inline bool lite_fits(int U, int nka, int nb, int nd, int G) {
  if (U < 1) return true;
  if (G - U * nb < 2) return false;
  const LiteSplit s = lite_split(U, nka, nb, nd, G);
  const int64_t NA = 2ll * U * nka, ND = static_cast<int64_t>(U) * nd;
  return (NA + s.gA - 1) / s.gA <= kLiteSlots && (ND + s.gD - 1) / s.gD <= kLiteSlots;
}

// The table rows (ItemLds) hold in their second halves the activation
// blocks (staging offset kLtAct, [2][16][32 chunks]; A: x rows; BC: gate / up
// latents; D: down latent in block 0), h (kLtHb, [16][32 chunks], 128
// columns) and the latent sums (kLtRed, [row of 2][wave][lane] float4).
constexpr uint32_t kLtAct = 0;
constexpr uint32_t kLtHb = kLtAct + 2 * kMaxM * kActChunks * 16;
constexpr uint32_t kLtRed = kLtHb + kMaxM * kActChunks * 16;
static_assert(kLtRed + 2 * 4 * kWave * 16 <= 256 * 128, "the chain's staging fits the table rows' second halves");
constexpr uint32_t lt_act(int blk) { return kLtAct + blk * kMaxM * kActChunks * 16; }
struct alignas(16) LiteSmem {
  ItemLds rows;
  u32x4 scales[2][kScaleBytes / 16];    // scale blocks of the one or two tiles being computed
  int rexp[2][kMaxM];                   // exponents of act's rows
  int hexp[kMaxM];                      // h exponents
  float hmax[4][kMaxM];                 // per-wave row maxima of h
  int ue[kLiteMaxP], ustart[kLiteMaxP], um[kLiteMaxP];  // units: expert, first grouped pair, pairs
  int pos_pair[kLiteMaxP];              // routed pair (token * K + slot) at each grouped position
  int pos_of[kLiteMaxP];                // grouped position of each routed pair (-1: dropped)
  float w[kLiteMaxP];                   // router weight of each routed pair
  int last[kLiteSlots * kMaxM];         // D: (token, tile) sums this workgroup completes
  int nunits, nlast, ticket;
};

// Level-pair table: thread tid fills row tid's 32 copies (rotated start, so
// the lanes of one store spread over the banks).
__device__ __forceinline__ void lut_fill(uint32_t L, int tid) {
  const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
  const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
#pragma unroll
  for (int j = 0; j < 8; ++j) lds_st<u32x4>(L + tid * 256 + ((j + tid) & 7) * 16, u32x4{bits, bits, bits, bits});
}

// Wave 0: the grouping of the call's routed pairs (lane i holds pair i).
__device__ __forceinline__ void lite_group(const LiteParams& p, LiteSmem& sm, int lane) {
  const bool in = lane < p.P;
  const int e = in ? p.ids[lane] : -1;
  const bool valid = e >= 0 && e < p.E;
  if (in) sm.w[lane] = load_act(p.weights, p.w_dtype, lane);
  uint64_t todo = __ballot(valid);
  int u = 0, start = 0, pos = -1;
  while (todo) {
    const int leader = __ffsll(static_cast<unsigned long long>(todo)) - 1;
    const int el = __shfl(e, leader, kWave);
    const uint64_t same = __ballot(valid && e == el);
    if (valid && e == el) pos = start + __popcll(same & ((1ull << lane) - 1ull));
    const int c = __popcll(same);
    // An expert's pairs beyond kMaxM start further units of the expert.
    for (int q = 0; q < c; q += kMaxM, ++u) {
      if (lane == 0) {
        sm.ue[u] = el;
        sm.ustart[u] = start + q;
        sm.um[u] = min(kMaxM, c - q);
      }
    }
    start += c;
    todo &= ~same;
  }
  if (in) sm.pos_of[lane] = pos;
  if (pos >= 0) sm.pos_pair[pos] = lane;
  if (lane == 0) {
    sm.nunits = u;
    sm.nlast = 0;
  }
}

// Routed slots of token t with a valid expert.
__device__ __forceinline__ int lite_routed(const LiteParams& p, const LiteSmem& sm, int t) {
  int c = 0;
  for (int q = 0; q < p.K; ++q) c += sm.pos_of[t * p.K + q] >= 0;
  return c;
}

// Bounded wait (thread 0) until *c >= target, then a workgroup barrier.
__device__ __forceinline__ void lite_wait(int* err, const int* c, int target) {
  if (threadIdx.x == 0) {
    const int64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(2);
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  lds_barrier();
}

// Sleep until `ticks` of s_memrealtime have passed since t0.
__device__ __forceinline__ void lite_sleep_until(int64_t t0, int64_t ticks) {
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// 8 x elements (dtype f32: a then b; f16 / bf16: a) as floats.
__device__ __forceinline__ void lite_x8(const u32x4& a, const u32x4& b, int dtype, float v[8]) {
  if (dtype == LATENT_F32) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = __uint_as_float(a[j]);
      v[4 + j] = __uint_as_float(b[j]);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (dtype == LATENT_F16) {
      v[2 * j] = half_bits_to_float(static_cast<uint16_t>(a[j] & 0xFFFFu));
      v[2 * j + 1] = half_bits_to_float(static_cast<uint16_t>(a[j] >> 16));
    } else {
      v[2 * j] = __uint_as_float(a[j] << 16);
      v[2 * j + 1] = __uint_as_float(a[j] & 0xFFFF0000u);
    }
  }
}



// Sums of partial rows into fp16 latent rows (act block k, exponents rexp[k])
// for the rows [0, m) of a unit whose first grouped pair is `start`.  Block i
// of key k holds P rows of 256 floats at byte ((k * nblocks + i) * P) * 1 KB of
// `base`.  kKeys = 2 (gate and up latents, two chains per key) or 1 (down
// latent, four chains): wave w runs chain c = w % chains of key w / chains,
// adding blocks c, c + chains, ... in order; a row is the chains' sums added
// in chain order.
template <int kKeys>
__device__ __forceinline__ void lite_latents(LiteSmem& sm, const float* base, int P, int nblocks, int start, int m,
                                             int lane, int wave) {
  const uint32_t L = lds_addr(sm.rows);
  constexpr int kChains = 4 / kKeys;
  const int key = wave / kChains, chain = wave % kChains;
  const int nk = (nblocks - chain + kChains - 1) / kChains;
  for (int r0 = 0; r0 < m; r0 += 2) {
    const int rows = min(2, m - r0);
    for (int rr = 0; rr < rows; ++rr) {
      const uint32_t roff = static_cast<uint32_t>(start + r0 + rr) * (kN * 4) + lane * 16;
      float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int i0 = 0; i0 < nk; i0 += kLiteRed) {
        float4 v[kLiteRed];
#pragma unroll
        for (int q = 0; q < kLiteRed; ++q) {
          const uint32_t blk = static_cast<uint32_t>(key * nblocks + chain + kChains * (i0 + q));
          v[q] = i0 + q < nk ? ld_coh4(base, blk * P * (kN * 4) + roff) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int q = 0; q < kLiteRed; ++q) add4(s, v[q]);
      }
      lds_st<float4v>(L + item_st(kLtRed + ((rr * 4 + wave) * kWave + lane) * 16), float4v{s.x, s.y, s.z, s.w});
    }
    lds_barrier();
    for (int c = wave; c < rows * kKeys; c += 4) {
      const int rr = c / kKeys, k = c % kKeys;
      auto red = [&](int w) __attribute__((always_inline)) {
        const float4v v = lds_ld<float4v>(L + item_st(kLtRed + ((rr * 4 + w) * kWave + lane) * 16));
        return make_float4(v[0], v[1], v[2], v[3]);
      };
      float4 t = red(k * kChains);
#pragma unroll
      for (int ch = 1; ch < kChains; ++ch) add4(t, red(k * kChains + ch));
      finish_row_lds(t, L, lt_act(k), sm.rexp[k], r0 + rr, lane);
    }
    lds_barrier();
  }
}

// Two register tiles' MFMA steps interleaved (two independent chains per
// wave): accA += actA . tile A, accB += actB . tile B (non-interleaved
// columns: phases A and D).
__device__ __forceinline__ void lite_mfma2(uint32_t L, uint32_t actA, uint32_t actB, uint32_t sbaseA, uint32_t sbaseB,
                                           const u32x4 (&cbA)[kSteps], const u32x4 (&cbB)[kSteps], int n, int kq,
                                           int wave, uint32_t lc, float4v (&accA)[4], float4v (&accB)[4]) {
  const int G = 2 * wave + (n >> 3);
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int chunk = s * 4 + kq;
    const uint32_t sd = scale_lane(G, kq) + s * 64;
    const half8 a[2] = {lds_ld<half8>(L + item_st(actA + act_slot(n, chunk) * 16)),
                        lds_ld<half8>(L + item_st(actB + act_slot(n, chunk) * 16))};
    const u32x4 sc[2] = {lds_ld<u32x4>(sbaseA + sd), lds_ld<u32x4>(sbaseB + sd)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const uint32_t x = tt ? cbB[s][j] : cbA[s][j];
        uint32_t f[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t pr = lds_ld<uint32_t>(L + lut_addr(x, q, lc));
          const uint32_t sq = sc[tt][q];  // through a scalar: a bit_cast of a vector element reads element 0
          f[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pr) * __builtin_bit_cast(half2v, sq));
        }
        const half8 b = __builtin_bit_cast(half8, make_uint4(f[0], f[1], f[2], f[3]));
        if (tt)
          accB[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], b, accB[j], 0, 0, 0);
        else
          accA[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], b, accA[j], 0, 0, 0);
      }
    }
  }
}

// Role A: K tiles [j0, j0 + nj) of the list (unit, gate/up, k).
__device__ __forceinline__ void lite_role_a(const LiteParams& p, LiteSmem& sm, int j0, int nj, int tid, int lane,
                                            int wave, uint32_t lc) {
  const uint32_t L = lds_addr(sm.rows);
  const int n = lane & 15, kq = lane >> 4;
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
  const int per = 2 * p.nka;
  const uint32_t esz = p.x_dtype == LATENT_F32 ? 4u : 2u;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(p.x, static_cast<uint32_t>(p.T) * p.d * esz);
  u32x4 cb[kLiteSlots][kSteps], sc[kLiteSlots], xr[2][2][2];
  // x slices of tile j (rows r0, r0 + 8 of its unit; f32 x takes both dwords of a chunk pair).
  auto load_x = [&](int j, bool valid, u32x4 (&xj)[2][2]) __attribute__((always_inline)) {
    const int t = j0 + min(j, nj - 1);
    const int u = t / per, r = t - u * per, f = r >= p.nka ? 1 : 0, k = r - f * p.nka;
    const int start = uniform(sm.ustart[u]), m = uniform(sm.um[u]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = r0 + 8 * h;
      const bool live = valid && row < m;
      const int tok = live ? sm.pos_pair[start + row] / p.K : 0;
      const uint32_t off = (static_cast<uint32_t>(tok) * p.d + k * kK + chunk * 8) * esz;
      xj[h][0] = ld128(rx, live ? off : 0x80000000u, 0);
      xj[h][1] = ld128(rx, live && esz == 4 ? off + 16 : 0x80000000u, 0);
    }
  };
  // Every tile's scales and codes, tile by tile, with the x slices of tiles 0 and 1.
#pragma unroll
  for (int j = 0; j < kLiteSlots; ++j) {
    const bool valid = j < nj;
    const int t = j0 + min(j, nj - 1);
    const int u = t / per, r = t - u * per, f = r >= p.nka ? 1 : 0, k = r - f * p.nka;
    const int e = uniform(sm.ue[u]), start = uniform(sm.ustart[u]), m = uniform(sm.um[u]);
    load_full<kSteps>(p, f ? F_UP_A : F_GATE_A, e * p.nka + k, valid, true, 0, tid, lane, wave, sc[j], cb[j]);
    if (j < 2) load_x(j, valid, xr[j]);
  }
  // Tile j into LDS buffer `buf`: its scales, and its x rows as fp16 * 2^e
  // with one exponent per row of this 256-column slice.
  auto stage = [&](int j, int buf, const u32x4 (&xj)[2][2]) __attribute__((always_inline)) {
    sm.scales[buf][tid] = sc[j];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = r0 + 8 * h;
      float v[8];
      lite_x8(xj[h][0], xj[h][1], p.x_dtype, v);
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
      mx = op_over(mx, 1, 32, OpMax{});
      const int ex = pow2_row_exponent(mx);
      half8 hv;
#pragma unroll
      for (int i = 0; i < 8; ++i) hv[i] = static_cast<_Float16>(ldexpf(v[i], ex));
      lds_st<u32x4>(L + item_st(lt_act(buf) + act_slot(row, chunk) * 16), __builtin_bit_cast(u32x4, hv));
      if (chunk == 0) sm.rexp[buf][row] = ex;
    }
  };
  // Tile j's partial rows (the products of buffer buf's rows, scaled back).
  auto store_part = [&](int j, int buf, float4v (&acc)[4]) __attribute__((always_inline)) {
    const int t = j0 + j;
    const int u = t / per, r = t - u * per, f = r >= p.nka ? 1 : 0, k = r - f * p.nka;
    const int start = uniform(sm.ustart[u]), m = uniform(sm.um[u]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = kq * 4 + v;
      if (row < m) {
        const float s = ldexpf(1.0f, -sm.rexp[buf][row]);
        const uint32_t off = ((static_cast<uint32_t>(f * p.nka + k) * p.P + start + row) * kN + wave * 64 + n * 4) * 4;
        st_coh4(p.partA, off, make_float4(acc[0][v] * s, acc[1][v] * s, acc[2][v] * s, acc[3][v] * s));
      }
    }
  };
  float4v acc0[4], acc1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc0[j] = acc1[j] = float4v{0.f, 0.f, 0.f, 0.f};
  // Tiles 0 and 1 together (two independent MFMA chains per wave), then tile 2.
  stage(0, 0, xr[0]);
  if (nj > 1) stage(1, 1, xr[1]);
  lds_barrier();
  if (nj > 1) {
    lite_mfma2(L, lt_act(0), lt_act(1), lds_addr(sm.scales[0][0]), lds_addr(sm.scales[1][0]), cb[0], cb[1], n, kq,
               wave, lc, acc0, acc1);
    store_part(1, 1, acc1);
  } else {
    reg_mfma<false, kSteps>(L, lt_act(0), lt_act(0), lds_addr(sm.scales[0][0]), cb[0], 0, n, kq, wave, lc, acc0);
  }
  store_part(0, 0, acc0);
  if (nj > 2) {
    lds_barrier();  // every wave is done with buffer 0
#pragma unroll
    for (int j = 0; j < 4; ++j) acc0[j] = float4v{0.f, 0.f, 0.f, 0.f};
    load_x(2, true, xr[0]);  // only workgroups with three tiles get here
    stage(2, 0, xr[0]);
    lds_barrier();
    reg_mfma<false, kSteps>(L, lt_act(0), lt_act(0), lds_addr(sm.scales[0][0]), cb[2], 0, n, kq, wave, lc, acc0);
    store_part(2, 0, acc0);
  }
  // Publish once every partial is stored.
  drain_barrier();
  if (tid < nj)
    __hip_atomic_fetch_add(p.cntA + (j0 + tid) / per * kLiteUnitStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Role BC: item (unit u, h block kb).
__device__ __forceinline__ void lite_role_bc(const LiteParams& p, LiteSmem& sm, int item, int64_t t0, int tid, int lane,
                                             int wave, uint32_t lc) {
  const uint32_t L = lds_addr(sm.rows);
  const int n = lane & 15, kq = lane >> 4;
  const int u = item / p.nb, kb = item - u * p.nb, hh = kb & 1;
  const int e = uniform(sm.ue[u]), start = uniform(sm.ustart[u]), m = uniform(sm.um[u]);
  u32x4 cbB[kSteps], cbC[kSteps], scB, scC;
  lite_sleep_until(t0, kLiteLateTicks);
  load_btile(p, e * p.nb + kb, true, tid, lane, wave, scB, cbB);
  // C tile kb / 2, K half hh: steps 4hh .. 4hh + 3 and the scales of row pairs 64hh .. 64hh + 63.
  load_full<kSteps / 2>(p, F_DOWN_A, e * p.nkc + (kb >> 1), true, ((tid & 31) >= 16) == (hh != 0), 4 * hh, tid, lane,
                        wave, scC, cbC);
  lite_wait(p.err, p.cntA + u * kLiteUnitStride, 2 * p.nka);
  lite_latents<2>(sm, p.partA, p.P, p.nka, start, m, lane, wave);
  sm.scales[0][tid] = scB;
  sm.scales[1][tid] = scC;
  lds_barrier();
  float4v acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
  reg_mfma<true, kSteps>(L, lt_act(0), lt_act(1), lds_addr(sm.scales[0][0]), cbB, 0, n, kq, wave, lc, acc);
  // h = SiLU(g) * u of columns 32w + 2n + jj of the block, fp16 with one exponent per row.
  float hv[2][4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = kq * 4 + v;
    const float sg = ldexpf(1.0f, -sm.rexp[0][row]), su = ldexpf(1.0f, -sm.rexp[1][row]);
    float mx = 0.f;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      hv[jj][v] = silu(acc[jj][v] * sg) * (acc[jj + 2][v] * su);
      mx = fmaxf(mx, fabsf(hv[jj][v]));
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
    half2v h2;
    h2[0] = static_cast<_Float16>(ldexpf(hv[0][v], ex));
    h2[1] = static_cast<_Float16>(ldexpf(hv[1][v], ex));
    lds_st<half2v>(L + item_st(kLtHb + act_slot(row, 4 * wave + (n >> 2)) * 16 + (n & 3) * 4), h2);
    if (wave == 0 && n == 0) sm.hexp[row] = ex;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4v{0.f, 0.f, 0.f, 0.f};
  lds_barrier();
  reg_mfma<false, kSteps / 2>(L, kLtHb, kLtHb, lds_addr(sm.scales[1][0]), cbC, 4 * hh, n, kq, wave, lc, acc);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = kq * 4 + v;
    if (row < m) {
      const float s = ldexpf(1.0f, -sm.hexp[row]);
      const uint32_t off = ((static_cast<uint32_t>(kb) * p.P + start + row) * kN + wave * 64 + n * 4) * 4;
      st_coh4(p.partC, off, make_float4(acc[0][v] * s, acc[1][v] * s, acc[2][v] * s, acc[3][v] * s));
    }
  }
  drain_barrier();
  if (tid == 0) __hip_atomic_fetch_add(p.cntC + u * kLiteUnitStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Role D: column tiles [j0, j0 + nj) of the list (unit, n).
template <int kOutMode>
__device__ __forceinline__ void lite_role_d(const LiteParams& p, LiteSmem& sm, int j0, int nj, int64_t t0, int tid,
                                            int lane, int wave, uint32_t lc) {
  const uint32_t L = lds_addr(sm.rows);
  const int n = lane & 15, kq = lane >> 4;
  u32x4 cb[kLiteSlots][kSteps], sc[kLiteSlots];
  lite_sleep_until(t0, kLiteLateTicks);
#pragma unroll
  for (int j = 0; j < kLiteSlots; ++j) {
    const int t = j0 + min(j, nj - 1);
    const int u = t / p.nd, s = t - u * p.nd;
    const int e = uniform(sm.ue[u]);
    load_full<kSteps>(p, F_DOWN_B, e * p.nd + s, j < nj, true, 0, tid, lane, wave, sc[j], cb[j]);
  }
  // Wait for unit u's C partials and sum them into the down latent (act
  // block 0); the workgroup holding D tile (u, 0) resets cntA[u] (every BC
  // item of the unit is past its wait for it).
  auto unit_latent = [&](int u, int s) __attribute__((always_inline)) {
    lite_wait(p.err, p.cntC + u * kLiteUnitStride, p.nb);
    if (s == 0 && tid == 0) __hip_atomic_store(p.cntA + u * kLiteUnitStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lite_latents<1>(sm, p.partC, p.P, p.nb, uniform(sm.ustart[u]), uniform(sm.um[u]), lane, wave);
  };
  // Tile j's y rows (the products of the down latent's rows, scaled back).
  auto store_y = [&](int j, float4v (&acc)[4]) __attribute__((always_inline)) {
    const int t = j0 + j;
    const int u = t / p.nd, s = t - u * p.nd;
    const int start = uniform(sm.ustart[u]), m = uniform(sm.um[u]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = kq * 4 + v;
      if (row < m) {
        const float sy = ldexpf(1.0f, -sm.rexp[0][row]);
        const int pos = start + row, col = s * kN + wave * 64 + n * 4;
        if constexpr (kOutMode == LATENT_OUT_PER_SLOT) {
          const int i = sm.pos_pair[pos];
          const float sw = p.wbd ? sy * sm.w[i] : sy;
          *reinterpret_cast<float4*>(p.out + static_cast<int64_t>(i) * p.d + col) =
              make_float4(acc[0][v] * sw, acc[1][v] * sw, acc[2][v] * sw, acc[3][v] * sw);
        } else {
          st_coh4(p.ybuf, (static_cast<uint32_t>(pos) * p.d + col) * 4,
                  make_float4(acc[0][v] * sy, acc[1][v] * sy, acc[2][v] * sy, acc[3][v] * sy));
        }
      }
    }
  };
  const int u0 = j0 / p.nd;
  if (nj == 2 && (j0 + 1) / p.nd == u0) {
    // Two tiles of one unit together (two independent MFMA chains per wave).
    unit_latent(u0, j0 - u0 * p.nd);
    float4v acc0[4], acc1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc0[j] = acc1[j] = float4v{0.f, 0.f, 0.f, 0.f};
    sm.scales[0][tid] = sc[0];
    sm.scales[1][tid] = sc[1];
    lds_barrier();
    lite_mfma2(L, lt_act(0), lt_act(0), lds_addr(sm.scales[0][0]), lds_addr(sm.scales[1][0]), cb[0], cb[1], n, kq,
               wave, lc, acc0, acc1);
    store_y(0, acc0);
    store_y(1, acc1);
  } else {
    // One tile at a time, each after its unit's latent.
    int cur = -1;
#pragma unroll
    for (int j = 0; j < kLiteSlots; ++j) {
      if (j < nj) {
        const int t = j0 + j;
        const int u = t / p.nd;
        lds_barrier();  // every wave is done with the previous tile's LDS
        if (u != cur) {
          cur = u;
          unit_latent(u, t - u * p.nd);
        }
        sm.scales[0][tid] = sc[j];
        lds_barrier();
        float4v acc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = float4v{0.f, 0.f, 0.f, 0.f};
        reg_mfma<false, kSteps>(L, lt_act(0), lt_act(0), lds_addr(sm.scales[0][0]), cb[j], 0, n, kq, wave, lc, acc);
        store_y(j, acc);
      }
    }
  }
  drain_barrier();
  // The unit's last D tile resets its BC and D counts.
  if (tid < nj) {
    const int u = (j0 + tid) / p.nd * kLiteUnitStride;
    if (__hip_atomic_fetch_add(p.cntD + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == p.nd) {
      __hip_atomic_store(p.cntC + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.cntD + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (kOutMode == LATENT_OUT_REDUCED) {
    // Thread 64 + 16 j + r counts row r of tile j into its (token, tile).
    const int q = tid - kWave;
    if (q >= 0 && q < kLiteSlots * kMaxM && (q >> 4) < nj) {
      const int t = j0 + (q >> 4), row = q & 15;
      const int u = t / p.nd, s = t - u * p.nd;
      if (row < sm.um[u]) {
        const int tok = sm.pos_pair[sm.ustart[u] + row] / p.K;
        const int key = tok * p.nd + s;
        if (__hip_atomic_fetch_add(p.cntY + key * kLiteKeyStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 ==
            lite_routed(p, sm, tok))
          sm.last[atomicAdd(&sm.nlast, 1)] = key;
      }
    }
    lds_barrier();
    // Completed (token, tile)s: the token's y rows in slot order, times w.
    const int nl = uniform(sm.nlast);
    for (int c = wave; c < nl; c += 4) {
      const int key = uniform(sm.last[c]);
      const int tok = key / p.nd, s = key - tok * p.nd;
      const uint32_t col = static_cast<uint32_t>(s * kN + lane * 4) * 4;
      float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int k0 = 0; k0 < p.K; k0 += kCombineBatch) {
        float4 v[kCombineBatch];
        float w[kCombineBatch];
        bool ok[kCombineBatch];
#pragma unroll
        for (int q2 = 0; q2 < kCombineBatch; ++q2) {
          const int i = tok * p.K + min(k0 + q2, p.K - 1);
          const int pos = k0 + q2 < p.K ? sm.pos_of[i] : -1;
          ok[q2] = pos >= 0;
          w[q2] = sm.w[i];
          v[q2] = ok[q2] ? ld_coh4(p.ybuf, static_cast<uint32_t>(pos) * p.d * 4 + col) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int q2 = 0; q2 < kCombineBatch; ++q2) {
          if (ok[q2]) {
            sum.x += w[q2] * v[q2].x;
            sum.y += w[q2] * v[q2].y;
            sum.z += w[q2] * v[q2].z;
            sum.w += w[q2] * v[q2].w;
          }
        }
      }
      *reinterpret_cast<float4*>(p.out + static_cast<int64_t>(tok) * p.d + s * kN + lane * 4) = sum;
      if (lane == 0) __hip_atomic_store(p.cntY + key * kLiteKeyStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int kOutMode>
__global__ void __launch_bounds__(kT, kGroupsPerCU) lite_kernel(LiteParams p) {
  __shared__ LiteSmem sm;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = uniform(tid >> 6);
  const int G = static_cast<int>(gridDim.x);
  // A grid larger than the resident workgroups takes roles in start order:
  // every workgroup a role waits for holds a lower ticket, so it is already
  // running.  The last ticket's holder resets the counter for the next call.
  int tk = 0;
  if (p.ticket && tid == 0) tk = __hip_atomic_fetch_add(p.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  lut_fill(lds_addr(sm.rows), tid);
  const uint32_t lc = (lane & 31) << 2;  // the lane's table copy offset
  if (wave == 0) lite_group(p, sm, lane);
  if (p.ticket && tid == 0) {
    sm.ticket = tk;
    if (tk == G - 1) __hip_atomic_store(p.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  lds_barrier();
  const int b = p.ticket ? uniform(sm.ticket) : static_cast<int>(blockIdx.x);
  // Workgroups that start once others have finished skip the B, C and D load delay.
  const int64_t t0 = __builtin_amdgcn_s_memrealtime() - (b < p.resident ? 0 : kLiteLateTicks);
  const int U = uniform(sm.nunits);
  // Rows no D tile writes (reduced output: tokens without a routed slot;
  // per-slot output: dropped slots), one row per workgroup from the last.
  {
    const int z = G - 1 - b;
    if constexpr (kOutMode == LATENT_OUT_REDUCED) {
      if (z < p.T && lite_routed(p, sm, z) == 0)
        for (int c = tid; c < p.d / 4; c += kT)
          reinterpret_cast<float4*>(p.out + static_cast<int64_t>(z) * p.d)[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      if (z < p.P && sm.pos_of[z] < 0)
        for (int c = tid; c < p.d / 4; c += kT)
          reinterpret_cast<float4*>(p.out + static_cast<int64_t>(z) * p.d)[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if (U == 0) return;
  const LiteSplit sp = lite_split(U, p.nka, p.nb, p.nd, G);
  if (b < sp.gA) {
    const int N = 2 * U * p.nka;
    const int j0 = range_lo(N, b, sp.gA), nj = range_lo(N, b + 1, sp.gA) - j0;
    if (nj > kLiteSlots) {
      if (tid == 0) __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (nj > 0) lite_role_a(p, sm, j0, nj, tid, lane, wave, lc);
  } else if (b < sp.gA + sp.gB) {
    lite_role_bc(p, sm, b - sp.gA, t0, tid, lane, wave, lc);
  } else {
    const int N = U * p.nd, jd = b - sp.gA - sp.gB;
    const int j0 = range_lo(N, jd, sp.gD), nj = range_lo(N, jd + 1, sp.gD) - j0;
    if (nj > kLiteSlots) {
      if (tid == 0) __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (nj > 0) lite_role_d<kOutMode>(p, sm, j0, nj, t0, tid, lane, wave, lc);
  }
}

// ---------------------------------------------------------------------------
// Prefill-sized batches: bulk units of up to 128 pairs (bulk_kernel)
// ---------------------------------------------------------------------------
// The same tile layout and phases as the decode launches, with units of up
// to kBulkM = 64 grouped pairs of one expert: a decoded B operand feeds four
// 16-row MFMA blocks (the unit's blocks, rounded up to 1, 2 or 4), so an
// expert's factor stream is read ceil(n_e / 64) times instead of
// ceil(n_e / 16).  An expert with fewer than 16 pairs runs one 16-row block
// per tile, the work shape of the decode path.  Two workgroups per CU, so a
// SIMD holds two waves and one's decode and LDS waits overlap the other's
// MFMAs; the unit's activation rows sit in LDS, 33 KB per 64 x 256 block
// (phase B: the gate and up latents).  Phases A and C load the next tile's
// block into registers while a tile is computed (their K slice changes every
// tile); phases B and D load a unit's block once, when the unit changes.
//
// Exponents: A's rows are x rows (one exponent per token), B's the gate and
// up latents and D's the d latent (one per row).  B writes h with one
// exponent per row and 32 columns (a wave's columns of a tile, so no wave
// waits for another).  C's K slices are eight such blocks: a unit's rows are
// rescaled while they are staged to the smallest exponent c of the row's
// blocks (exact powers of two; only the row's smaller blocks lose low bits),
// and the partial sums are scaled by 2^-c.  Reduced output stores y in fp16
// with one exponent per row and 64 columns (again a wave's own) for the
// per-token combine; per-slot output stores fp32 rows.

constexpr int kBulkBlocks = kBulkM / 16;
constexpr int kBulkRing = 2;  // code ring depth (tiles)
constexpr int kBulkHBlock = 32;  // h columns per exponent (phase B: a wave's columns of a tile)
constexpr int kBulkYBlock = 64;  // y columns per exponent (phase D: a wave's columns of a tile)
constexpr int kBulkRounds = kBulkM * kActChunks / kT;  // 16-byte activation chunks per thread and block
constexpr uint32_t kNoRow = 0x80000000u;               // offset of a padding row: beyond every buffer range
// Activation rows in LDS are 33 chunks apart: the 16 rows x 4 chunks of one
// MFMA operand read fall on distinct banks, and every fragment address of a
// tile is one base register plus an immediate offset.
constexpr int kBulkStride = kActChunks + 1;
__device__ __forceinline__ int bulk_slot(int row, int chunk) { return row * kBulkStride + chunk; }

template <int kPhase>
struct BulkShape {
  static constexpr int kActBlocks = kPhase == kPhaseB ? 2 : 1;
  // Level table copies: B keeps two activation blocks in LDS, and two
  // workgroups share a CU's 160 KB.
  static constexpr int kLut = kPhase == kPhaseB ? 8 : 32;
  static constexpr int kLutShift = kPhase == kPhaseB ? 5 : 7;
  static constexpr bool kStaged = kPhase == kPhaseA || kPhase == kPhaseC;
};

// D: 256 table rows of 256 bytes, as the item kernels' (ItemLds): row b's
// first half holds code byte b's level pair in 32 copies, so a lookup
// address is one byte permute (lut_addr), and the rows' second halves hold
// the unit's activation block: activation row r's chunks 8 j .. 8 j + 7 in
// table row 4 r + j, chunk c at position (c ^ r) & 7 of the 128 bytes (the 8
// rows an MFMA read takes at once meet 8 distinct bank groups, and every
// operand address of a K step is one of two lane bases plus an immediate).
// Measured D 297 -> 284 us; the same layout in A and C (and its address
// arithmetic next to B's) tipped them into spills: A 428 -> 487 us, C 110 ->
// 125 us.  A, B and C: a table of 32 (B: 8) copies per byte and the
// activation block(s) beside it, rows 33 chunks apart.
template <int kPhase>
struct alignas(16) BulkSmem {
  static constexpr bool kTableRows = kPhase == kPhaseD;
  static_assert(!kTableRows || kBulkM * kActChunks * 16 == 256 * 128, "the block fills the rows' second halves");
  uint32_t lut[kTableRows ? 256 * 64 : 256 * BulkShape<kPhase>::kLut];  // [byte][copy]: half2(level(lo), level(hi))
  u32x4 scales[kScaleBytes / 16];                                        // the tile's scale block
  u32x4 act[kTableRows ? 1 : BulkShape<kPhase>::kActBlocks][kTableRows ? 1 : kBulkM * kBulkStride];
  int rexp[2][kBulkM];     // A: x exponent, C: row exponent c (by unit parity); B: gate / up latent; D: d latent
  uint32_t rowoff[2][kBulkM];  // A: byte offset of each row's x row (by unit parity); D: output row
  int texp[kPhase == kPhaseC ? kK / kBulkHBlock : 1][kBulkM];  // C: the staged tile's h block exponents of each row
  float pw[kBulkM];        // D, per-slot output: router weight of each row
  // D: floor(log2) of each row's L1 norm (y scale), clamped; B: the sum of
  // those of the row's gate and up latents (fp16 scale)
  int il1[kPhase == kPhaseD || kPhase == kPhaseB ? kBulkM : 1];
};

// LDS byte address of chunk `chunk` of row `row` of activation block blk.
template <int kPhase>
__device__ __forceinline__ uint32_t bulk_act(const BulkSmem<kPhase>& sm, int blk, int row, int chunk) {
  BulkSmem<kPhase>& m = const_cast<BulkSmem<kPhase>&>(sm);
  if constexpr (BulkSmem<kPhase>::kTableRows)
    return lds_addr(m.lut[0]) + static_cast<uint32_t>(row * 1024 + (chunk >> 3) * 256 + 128 + (((chunk ^ row) & 7) << 4));
  else return lds_addr(m.act[blk][0]) + bulk_slot(row, chunk) * 16;
}

// MFMA steps of a tile over the unit's first kRb 16-row blocks: per 32-row
// step the four B operands of the wave's columns are decoded once and
// multiplied into every block.  Rows past the unit's pairs hold zeros.
template <int kPhase, int kRb>
__device__ __forceinline__ void bulk_steps(const BulkSmem<kPhase>& sm, const u32x4 (&cb)[kSteps], int n, int kq,
                                           int wave, uint32_t lut_lane, float4v (&acc)[kBulkBlocks][4]) {
  const uint32_t sbase = lds_addr(const_cast<BulkSmem<kPhase>&>(sm).scales[0]);
  // Table rows: the lane's activation bases of even and odd K steps.
  const uint32_t abase0 = BulkSmem<kPhase>::kTableRows ? bulk_act(sm, 0, n, kq) : 0u, abase1 = abase0 ^ 64u;
  // Phase C: the lane base of the scale rows, of which each step takes an
  // opaque copy, so the compiler neither keeps eight per-step addresses live
  // across the tile loop (they spilled, and every reload waited for the tile
  // loads in flight) nor hoists later steps' scale reads.
  const uint32_t slc = kPhase == kPhaseC ? sbase + scale_lane(2 * wave + (n >> 3), kq) : 0u;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int chunk = s * 4 + kq;
    const int P0 = s * 16 + kq * 4;
    u32x4 sc0, sc1;
    if constexpr (kPhase == kPhaseB) {
      const int Gg = wave, Gu = 4 + wave;
      sc0 = lds_ld<u32x4>(sbase + (Gg * 128 + (P0 ^ ((Gg & 1) << 3))) * 4);
      sc1 = lds_ld<u32x4>(sbase + (Gu * 128 + (P0 ^ ((Gu & 1) << 3))) * 4);
    } else if constexpr (kPhase == kPhaseC) {
      uint32_t a0 = slc;
      asm volatile("" : "+v"(a0));
      sc0 = lds_ld<u32x4>(a0 + s * 64);
      sc1 = sc0;
    } else {
      const int G = 2 * wave + (n >> 3);
      sc0 = lds_ld<u32x4>(sbase + (G * 128 + (P0 ^ ((G & 1) << 3))) * 4);
      sc1 = sc0;
    }
    half8 bf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = code_dword<kPhase == kPhaseB>(cb, s, j);
      const u32x4 sc = j < 2 ? sc0 : sc1;
      uint32_t f[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pr =
            BulkSmem<kPhase>::kTableRows
                ? lds_ld<uint32_t>(lds_addr(const_cast<BulkSmem<kPhase>&>(sm).lut[0]) + lut_addr(x, q, lut_lane))
                : lds_ld<uint32_t>(lut_lane + (((x >> (8 * q)) & 0xFFu) << BulkShape<kPhase>::kLutShift));
        const uint32_t sq = sc[q];
        f[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, pr) * __builtin_bit_cast(half2v, sq));
      }
      bf[j] = __builtin_bit_cast(half8, make_uint4(f[0], f[1], f[2], f[3]));
    }
#pragma unroll
    for (int rb = 0; rb < kRb; ++rb) {
      const int row = rb * 16 + n;
      half8 a0, a1;
      if constexpr (BulkSmem<kPhase>::kTableRows) {
        // Row rb * 16 + n, chunk 4 s + kq: table row 4 row + s / 2, position
        // ((s & 1) * 4 + kq) ^ (n & 7).
        a0 = lds_ld<half8>((s & 1 ? abase1 : abase0) + rb * 16384 + (s >> 1) * 256);
        a1 = a0;
      } else {
        a0 = __builtin_bit_cast(half8, sm.act[0][bulk_slot(row, chunk)]);
        a1 = kPhase == kPhaseB ? __builtin_bit_cast(half8, sm.act[BulkShape<kPhase>::kActBlocks - 1][bulk_slot(row, chunk)])
                               : a0;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(j < 2 ? a0 : a1, bf[j], acc[rb][j], 0, 0, 0);
    }
  }
}

// Phase D's y exponents come from a bound instead of each row's maximum over
// the wave's 64 columns (a 16-lane reduction per row and tile): a staged row's
// fp16 values a_k times the decoded tile b_kj (|b_kj| <= the largest scale of
// the wave's two groups, |level| <= 1) give |y_j| <= 2^-e sum_k |a_k| * maxsc
// < 2^(il1 + 1) * 2^(ilog(maxsc) + 1), so y * 2^(13 - il1 - ilog(maxsc)) stays
// below 2^15 and fp16 keeps its full relative precision down to 2^-28 of the
// bound.  il1 = floor(log2(sum |a_k| * 2^-e)), clamped so that the exponent
// stays within [-122, 120] (a clamp from below only loosens the bound).
__device__ __forceinline__ int bulk_y_ilog(float l1, int e) {
  const int il = static_cast<int>((__float_as_uint(l1) >> 23) & 0xFFu) - 127 - e;
  return min(120, max(-83, il));
}
// floor(log2) of the largest |scale| of the scale groups wave w reads in a
// tile's scale block in LDS (group G at dwords 128 G..; fp16 bit patterns of
// non-negative values order as integers).  D: groups 2w and 2w + 1 (its 64
// columns).  B: the sum over gate group w and up group 4 + w (its 32 h
// columns' g and u).
template <bool kB, class Smem>
__device__ __forceinline__ int bulk_scale_ilog(const Smem& sm, int wave, int lane) {
  const u32x4 q = sm.scales[kB ? 32 * wave + (lane & 31) + (lane >> 5) * 128 : 64 * wave + lane];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = q[i] & 0x7FFF7FFFu;
    m = max(m, max(v & 0xFFFFu, v >> 16));
  }
  const float mx = op_over(static_cast<float>(m), 1, kB ? 32 : kWave, OpMax{});
  const int il = static_cast<int>(static_cast<uint32_t>(mx) >> 10) - 15;
  if constexpr (kB) return __builtin_amdgcn_readlane(il, 0) + __builtin_amdgcn_readlane(il, 32);
  return il;
}

// Per-unit tables of the bulk phases (all threads; a barrier must follow).
//   A: rowoff[buf][r] = byte offset of the row's x row, rexp[buf][r] = its exponent;
//   C: rexp[buf][r] = smallest exponent of the row's h blocks.
template <int kPhase>
__device__ __forceinline__ void bulk_unit_tables(const Params& p, BulkSmem<kPhase>& sm, const TileRef& tr, int buf,
                                                 int tid) {
  if (tid >= kBulkM) return;
  const bool live = tid < tr.m;
  const int pair = tr.start + min(tid, tr.m - 1);
  if constexpr (kPhase == kPhaseA) {
    const int tok = p.pair_tok[pair];
    sm.rowoff[buf][tid] = live ? static_cast<uint32_t>(tok) * p.d * 2u : kNoRow;
    sm.rexp[buf][tid] = live ? p.xexp[tok] : 0;
  } else if constexpr (kPhase == kPhaseC) {
    const int nh = p.ff / kBulkHBlock;
    const __amdgpu_buffer_rsrc_t re = buffer_rsrc(p.hexp, static_cast<uint32_t>(p.P) * nh * 4);
    int c = 0x7FFFFFFF;
    for (int b0 = 0; b0 < nh; b0 += 8) {  // eight loads in flight
      int e[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) e[q] = static_cast<int>(ld32(re, (static_cast<uint32_t>(pair) * nh + min(b0 + q, nh - 1)) * 4));
#pragma unroll
      for (int q = 0; q < 8; ++q) c = min(c, e[q]);
    }
    sm.rexp[buf][tid] = live ? c : 0;
  }
}

// Phases B and D: the unit's activation block(s) into LDS (blocking), with
// their row exponents and, for D's per-slot output, each row's output row and
// weight.  Runs between barriers.
//   B: the gate and up latents, finished by A's reduce launch (fp16 rows and
//      exponents, by grouped pair).
//   D: the fp32 sum of C's key u, left in the key's partial slot by its
//      workgroup (or, for a rest key, by the reduce launch), finished here
//      as finish_row does: fp16 row * 2^e, e from the row's maximum over its
//      256 columns (a row's 32 chunks are 32 lanes of one wave); four rounds
//      of rows at a time, two 16-byte loads per chunk of 8 values.
template <int kPhase>
__device__ __forceinline__ void bulk_unit_act(const Params& p, BulkSmem<kPhase>& sm, const TileRef& tr, int u,
                                              int tid) {
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
  if constexpr (kPhase == kPhaseB) {
    const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(p.lat, 2u * p.P * kK * 2);
    u32x4 st[2][kBulkRounds];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int h = 0; h < kBulkRounds; ++h) {
        const int r = r0 + 8 * h;
        const uint32_t off =
            r < tr.m ? (static_cast<uint32_t>(blk) * p.P + tr.start + r) * kK * 2 + chunk * 16 : kNoRow;
        st[blk][h] = ld128(rl, off, 0);
      }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int h = 0; h < kBulkRounds; ++h) sm.act[blk][bulk_slot(r0 + 8 * h, chunk)] = st[blk][h];
    // floor(log2) of each row's L1 norm, gate plus up (fp16 scale; the row
    // exponents are applied where they are used).  Row slots through one
    // opaque lane base plus immediates.
    uint32_t rowl = lds_addr(sm.il1[0]) + r0 * 4;
    asm volatile("" : "+v"(rowl));
#pragma unroll
    for (int h = 0; h < kBulkRounds; ++h) {
      int il = 0;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        float l1 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w = st[blk][h][q];  // through a scalar: a bit_cast of a vector element reads element 0
          const half2v hv = __builtin_bit_cast(half2v, w);
          l1 += fabsf(static_cast<float>(hv[0])) + fabsf(static_cast<float>(hv[1]));
        }
        l1 = op_over(l1, 1, 32, OpAdd{});
        il += static_cast<int>((__float_as_uint(l1) >> 23) & 0xFFu) - 127;
      }
      if (chunk == 0) lds_st<int>(rowl + 32 * h, il);
    }
    if (tid < 2 * kBulkM) {
      const int blk = tid / kBulkM, r = tid % kBulkM;
      sm.rexp[blk][r] = p.lexp[blk * p.P + tr.start + min(r, tr.m - 1)];
    }
  } else {
    constexpr int kBatch = 4;
    const float* src = p.partC + static_cast<int64_t>(u) * kBulkM * kN;
    // The rows' exponent and L1 slots as one opaque lane base plus immediates
    // (per-row addresses hoisted out of the tile loop spilled).
    uint32_t rowx = lds_addr(sm.rexp[0][0]) + r0 * 4, rowl = lds_addr(sm.il1[0]) + r0 * 4;
    asm volatile("" : "+v"(rowx), "+v"(rowl));
    const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(src, kBulkM * kN * 4);
#pragma unroll
    for (int h0 = 0; h0 < kBulkRounds; h0 += kBatch) {
      u32x4 v[kBatch][2];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int r = r0 + 8 * (h0 + q);
        const uint32_t off = r < tr.m ? static_cast<uint32_t>(r * kN + chunk * 8) * 4 : kNoRow;
        v[q][0] = ld128(rl, off, 0);
        v[q][1] = ld128(rl, off + 16, 0);
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int r = r0 + 8 * (h0 + q);
        float x[8], mx = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t bits = v[q][i >> 2][i & 3];  // through a scalar: a bit_cast of a vector element reads element 0
          x[i] = __uint_as_float(bits);
          mx = fmaxf(mx, fabsf(x[i]));
        }
        const int ex = pow2_row_exponent(op_over(mx, 1, 32, OpMax{}));
        half8 hv;
        float l1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          hv[i] = static_cast<_Float16>(ldexpf(x[i], ex));
          l1 += fabsf(static_cast<float>(hv[i]));
        }
        l1 = op_over(l1, 1, 32, OpAdd{});
        lds_st<u32x4>(bulk_act(sm, 0, r, chunk), __builtin_bit_cast(u32x4, hv));
        if (chunk == 0) {
          lds_st<int>(rowx + 32 * (h0 + q), ex);
          lds_st<int>(rowl + 32 * (h0 + q), bulk_y_ilog(l1, ex));
        }
      }
    }
    if (tid < kBulkM) {
      const int pair = tr.start + min(tid, tr.m - 1);
      sm.rowoff[0][tid] = static_cast<uint32_t>(p.pair_tok[pair] * p.K + p.pair_slot[pair]);
      sm.pw[tid] = p.pair_w[pair];
    }
  }
}

// Phases A and C: issue the loads of a tile's activation block (and C's block
// exponents) into registers.
constexpr int kBulkTex = kK / kBulkHBlock * kBulkM / kT;  // C: h block exponents per thread and tile

template <int kPhase>
__device__ __forceinline__ void bulk_issue_act(const Params& p, BulkSmem<kPhase>& sm, const TileRef& tr, int ubuf,
                                               int tid, bool valid, u32x4 (&st)[kBulkRounds], int (&tex)[kBulkTex]) {
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
  if constexpr (kPhase == kPhaseA) {
    const int ks = tr.r >= p.nka ? tr.r - p.nka : tr.r;
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(p.xh, valid ? static_cast<uint32_t>(p.T) * p.d * 2 : 0u);
    const uint32_t col = ks * kK * 2 + chunk * 16;
#pragma unroll
    for (int h = 0; h < kBulkRounds; ++h) st[h] = ld128(rx, sm.rowoff[ubuf][r0 + 8 * h] + col, 0);
  } else {
    const int ks = tr.r;
    const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(p.hh, valid ? static_cast<uint32_t>(p.P) * p.ff * 2 : 0u);
    const uint32_t col = ks * kK * 2 + chunk * 16;
#pragma unroll
    for (int h = 0; h < kBulkRounds; ++h) {
      const int r = r0 + 8 * h;
      st[h] = ld128(rh, r < tr.m ? static_cast<uint32_t>(tr.start + r) * p.ff * 2 + col : kNoRow, 0);
    }
    // Exponent of h block q of row r: thread tid loads block tid % 8 of rows
    // tid / 8 + 32 j.
    const int nh = p.ff / kBulkHBlock, nq = kK / kBulkHBlock;
    const __amdgpu_buffer_rsrc_t re = buffer_rsrc(p.hexp, valid ? static_cast<uint32_t>(p.P) * nh * 4 : 0u);
#pragma unroll
    for (int j = 0; j < kBulkTex; ++j) {
      const int r = tid / nq + (kT / nq) * j;
      tex[j] = static_cast<int>(
          ld32(re, r < tr.m ? (static_cast<uint32_t>(tr.start + r) * nh + ks * nq + tid % nq) * 4 : kNoRow));
    }
  }
}

// Phases A and C: store a staged activation block (C: rescaled to the unit's
// row exponents; the block exponents go through LDS, so this takes one more
// barrier).
template <int kPhase>
__device__ __forceinline__ void bulk_store_act(BulkSmem<kPhase>& sm, int ubuf, int tid, const u32x4 (&st)[kBulkRounds],
                                               const int (&tex)[kBulkTex]) {
  const int r0 = tid / kActChunks, chunk = tid % kActChunks;
  if constexpr (kPhase == kPhaseC) {
    constexpr int nq = kK / kBulkHBlock;
#pragma unroll
    for (int j = 0; j < kBulkTex; ++j) sm.texp[tid % nq][tid / nq + (kT / nq) * j] = tex[j];
    lds_barrier();
    const int q = chunk / (kBulkHBlock / 8);  // the chunk's h block within the tile
#pragma unroll
    for (int h = 0; h < kBulkRounds; ++h) {
      const int r = r0 + 8 * h;
      const int sh = max(-30, sm.rexp[ubuf][r] - sm.texp[q][r]);
      const _Float16 m = static_cast<_Float16>(ldexpf(1.0f, sh));
      const half2v m2 = {m, m};
      u32x4 v = st[h];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t vq = v[q];  // through a scalar: a bit_cast of a vector element reads element 0
        v[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, vq) * m2);
      }
      sm.act[0][bulk_slot(r, chunk)] = v;
    }
  } else {
#pragma unroll
    for (int h = 0; h < kBulkRounds; ++h) sm.act[0][bulk_slot(r0 + 8 * h, chunk)] = st[h];
  }
}

template <int kPhase>
__global__ void __launch_bounds__(kT, kGroupsPerCU) bulk_kernel(Params p) {
  using BS = BulkShape<kPhase>;
  __shared__ BulkSmem<kPhase> sm;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = uniform(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int per_unit = tiles_per_unit<kPhase>(p), per_key = bulk_key_tiles<kPhase>(p);
  const int U = uniform(sload(p.nunits));
  // Whole keys per workgroup, dealt XCD by XCD: workgroup b runs on XCD
  // b % 8, which takes the contiguous block [K x / 8, K (x + 1) / 8) of the
  // key list (unit-major, so an expert's keys are neighbours); its
  // workgroups take the block's keys round robin.  Workgroups of one XCD
  // that run at the same time then work on the keys of one expert, the same
  // factor tile at the same K step, and the same unit's activation slices
  // (gate and up keys of a unit are neighbours): all but the first read hit
  // that XCD's L2.
  const int nkey = U * (per_unit / per_key);
  const int b = blockIdx.x, xcd = b & 7, jw = b >> 3;
  const Deal dl = deal_for(nkey, per_key, p.G, xcd);
  const int nfull = dl.F * per_key;                          // tiles of the whole keys
  const int r0 = jw * dl.c;                                  // first rest tile of the range
  const int nrest = max(0, min(dl.c, dl.T_rem - r0));
  const int ntile = nfull + nrest;
  if (ntile == 0) return;
  // Flat tile index (unit-major, as tile_ref reads it) of the workgroup's tile i.
  auto vt = [&](int i) __attribute__((always_inline)) {
    if (i < nfull) {
      const int r = i / per_key;
      return (dl.kx0 + jw + r * dl.J) * per_key + (i - r * per_key);
    }
    return dl.rest0 * per_key + r0 + (i - nfull);
  };
  const int key_rest0 = (dl.rest0 * per_key + r0) / per_key;  // key of the first rest tile
  // Segment (run of one key's tiles) ordinal of tile i in the workgroup, and
  // the LDS table buffer it uses (segments alternate).
  auto seg = [&](int i) __attribute__((always_inline)) {
    return i < nfull ? i / per_key : dl.F + vt(i) / per_key - key_rest0;
  };
  auto kbuf = [&](int i) __attribute__((always_inline)) { return seg(i) & 1; };
  // Tile i1 starts another segment than tile i1 - 1.
  auto new_seg = [&](int i1) __attribute__((always_inline)) { return seg(i1) != seg(i1 - 1); };

  {
    const half2v lv = {static_cast<_Float16>(nf4_level(tid & 15)), static_cast<_Float16>(nf4_level(tid >> 4))};
    const uint32_t bits = __builtin_bit_cast(uint32_t, lv);
    if constexpr (BulkSmem<kPhase>::kTableRows) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        lds_st<u32x4>(lds_addr(sm.lut[0]) + tid * 256 + ((j + tid) & 7) * 16, u32x4{bits, bits, bits, bits});
    } else {
      uint4* dstv = reinterpret_cast<uint4*>(&sm.lut[tid * BS::kLut]);
#pragma unroll
      for (int j = 0; j < BS::kLut / 4; ++j) dstv[(j + tid) & (BS::kLut / 4 - 1)] = make_uint4(bits, bits, bits, bits);
    }
  }
  // Table rows: the lane's copy offset (lut_addr); otherwise the lane's copy's address.
  const uint32_t lut_lane = BulkSmem<kPhase>::kTableRows ? static_cast<uint32_t>(lane & 31) << 2
                                                         : lds_addr(sm.lut[0]) + ((lane & (BS::kLut - 1)) << 2);

  // Code ring of kBulkRing tiles: tile i + kBulkRing - 1's loads are issued
  // while tile i is computed.
  u32x4 cb[kBulkRing][kSteps];
  u32x4 sc[kBulkRing];
  TileRef ref[kBulkRing];
  u32x4 st[kBulkRounds];
  int tex[kBulkTex] = {};
  float4v acc[kBulkBlocks][4];
#pragma unroll
  for (int rb = 0; rb < kBulkBlocks; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[rb][j] = float4v{0.f, 0.f, 0.f, 0.f};

  // Prologue: per-unit tables of tiles 0 and 1 (A, C) or the first unit's
  // activations (B, D); tile 0's activations and scales in LDS; the ring's
  // first tiles in flight.
#pragma unroll
  for (int r = 0; r + 1 < kBulkRing; ++r) ref[r] = tile_ref<kPhase>(p, vt(min(r, ntile - 1)));
  const TileRef ref1 = tile_ref<kPhase>(p, vt(min(1, ntile - 1)));
  if constexpr (BS::kStaged) {
    bulk_unit_tables<kPhase>(p, sm, ref[0], 0, tid);
    if (ntile > 1 && new_seg(1)) bulk_unit_tables<kPhase>(p, sm, ref1, 1, tid);
    lds_barrier();
    bulk_issue_act<kPhase>(p, sm, ref[0], 0, tid, true, st, tex);
  } else {
    bulk_unit_act<kPhase>(p, sm, ref[0], vt(0) / per_unit, tid);
  }
#pragma unroll
  for (int r = 0; r + 1 < kBulkRing; ++r) issue_codes<kPhase>(p, ref[r], tid, lane, wave, r < ntile, sc[r], cb[r]);
  if constexpr (BS::kStaged) bulk_store_act<kPhase>(sm, 0, tid, st, tex);
  sm.scales[tid] = sc[0];

  auto step = [&](int i, auto cs) __attribute__((always_inline)) {
    // Slots: c holds tile i, c1 tile i + 1, cl the tile issued now (i + kBulkRing - 1).
    constexpr int c = decltype(cs)::value, c1 = (c + 1) % kBulkRing, cl = (c + kBulkRing - 1) % kBulkRing;
    const int t = vt(i);
    const int ubuf = kbuf(i);
    lds_barrier();  // tile i's activations and scales are in LDS
    // Tile i + 1's activations first (A, C), then tile i + 2's codes: loads
    // complete in order, so the wait for the activations at the end of this
    // step leaves the codes in flight.
    ref[cl] = tile_ref<kPhase>(p, vt(min(i + kBulkRing - 1, ntile - 1)));
    if constexpr (BS::kStaged)
      bulk_issue_act<kPhase>(p, sm, ref[c1], kbuf(min(i + 1, ntile - 1)), tid, i + 1 < ntile, st, tex);
    issue_codes<kPhase>(p, ref[cl], tid, lane, wave, i + kBulkRing - 1 < ntile, sc[cl], cb[cl]);
    const TileRef& tr = ref[c];
    const int nrb = (tr.m + 15) >> 4;
    // Row tables from the lane's first row (kq * 4): entry rb * 16 + v is the
    // lane's row v of block rb (immediate offsets).
    const int* rx0 = &sm.rexp[0][kq * 4];
    const int* rx1 = &sm.rexp[1][kq * 4];
    // Branch-free MFMA sections for 1, 2 or 4 blocks (the unit's blocks
    // rounded up): a branch per block would expose every operand read.
    if (nrb > 2)
      bulk_steps<kPhase, 4>(sm, cb[c], n, kq, wave, lut_lane, acc);
    else if (nrb > 1)
      bulk_steps<kPhase, 2>(sm, cb[c], n, kq, wave, lut_lane, acc);
    else
      bulk_steps<kPhase, 1>(sm, cb[c], n, kq, wave, lut_lane, acc);

    if constexpr (Shape<kPhase>::kSliceK) {
      if (i + 1 == ntile || new_seg(i + 1)) {
        // End of a segment: a whole key's sum (slot = key) or a rest piece
        // (slot in the workgroup's rest range, see Deal).  Through a buffer
        // resource: one lane offset, and each row's offset a constant in
        // the scalar operand (no per-row 64-bit addresses to keep live
        // across the loop).
        const int key = t / per_key;
        const int slot = i < nfull ? key : 2 * U + ((xcd + 8 * jw) * kRemPieces + key - key_rest0);
        const float* part = (kPhase == kPhaseA ? p.partA : p.partC) + static_cast<int64_t>(slot) * kBulkM * kN;
        const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(part, kBulkM * kN * 4);
        const uint32_t lane_off = static_cast<uint32_t>(kq * 4 * kN + wave * 64 + n * 4) * 4;
#pragma unroll
        for (int rb = 0; rb < kBulkBlocks; ++rb) {
          if (rb < nrb) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int row = rb * 16 + kq * 4 + v;
              if (row < tr.m) {
                const float s = ldexpf(1.0f, -(ubuf ? rx1 : rx0)[rb * 16 + v]);
                const u32x4 w = {__float_as_uint(acc[rb][0][v] * s), __float_as_uint(acc[rb][1][v] * s),
                                 __float_as_uint(acc[rb][2][v] * s), __float_as_uint(acc[rb][3][v] * s)};
                __builtin_amdgcn_raw_buffer_store_b128(w, rp, lane_off, (rb * 16 + v) * kN * 4, 0);
              }
            }
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[rb][j] = float4v{0.f, 0.f, 0.f, 0.f};
        }
      }
    } else if constexpr (kPhase == kPhaseB) {
      // h = SiLU(g) * u of the wave's 32 h columns, fp16 with one exponent
      // per row and 32-column block (the wave's own: no exchange).
      // The exponent comes from a bound, as D's does: |SiLU(g)| <= |g|, and
      // |g| < 2^(il_g + 1 - e_g) 2^(ilog(maxsc_g) + 1) with il_g = floor(log2)
      // of the staged gate latent row's L1 norm (u alike), so h * 2^ex stays
      // below 2^15 for ex = 11 - il_g - il_u - ilog(maxsc_g) - ilog(maxsc_u)
      // + e_g + e_u.
      const int nh = p.ff / kBulkHBlock;
      const int hex0 = 11 - bulk_scale_ilog<true>(sm, wave, lane);
#pragma unroll
      for (int rb = 0; rb < kBulkBlocks; ++rb) {
        if (rb < nrb) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = rb * 16 + kq * 4 + v;
            const int eg = rx0[rb * 16 + v], eu = rx1[rb * 16 + v];
            const float sg = ldexpf(1.0f, -eg), su = ldexpf(1.0f, -eu);
            const float h0 = silu(acc[rb][0][v] * sg) * (acc[rb][2][v] * su);
            const float h1 = silu(acc[rb][1][v] * sg) * (acc[rb][3][v] * su);
            const int ex = min(120, max(-120, hex0 - (&sm.il1[kq * 4])[rb * 16 + v] + eg + eu));
            if (row < tr.m) {
              half2v hb;
              hb[0] = static_cast<_Float16>(ldexpf(h0, ex));
              hb[1] = static_cast<_Float16>(ldexpf(h1, ex));
              const int64_t prow = tr.start + row;
              *reinterpret_cast<half2v*>(p.hh + prow * p.ff + tr.r * kHBlock + wave * 32 + n * 2) = hb;
              if (n == 0) p.hexp[prow * nh + tr.r * 4 + wave] = ex;
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rb][j] = float4v{0.f, 0.f, 0.f, 0.f};
      }
    } else {
      // D: y rows of the tile's 256 columns; reduced output in fp16 with one
      // exponent per row and 64-column block (the wave's own).
      const bool reduced = p.out_mode == LATENT_OUT_REDUCED;
      const int ny = p.d / kBulkYBlock;
      const int yex0 = reduced ? 13 - bulk_scale_ilog<false>(sm, wave, lane) : 0;
#pragma unroll
      for (int rb = 0; rb < kBulkBlocks; ++rb) {
        if (rb < nrb) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = rb * 16 + kq * 4 + v;
            const int64_t prow = tr.start + row;
            const int col = tr.r * kN + wave * 64 + n * 4;
            if (reduced) {
              const int ex = yex0 - (&sm.il1[kq * 4])[rb * 16 + v];
              const int ea = ex - rx0[rb * 16 + v];  // y = acc * 2^-rexp
              if (row < tr.m) {
                half4v hv;
#pragma unroll
                for (int j = 0; j < 4; ++j) hv[j] = static_cast<_Float16>(ldexpf(acc[rb][j][v], ea));
                *reinterpret_cast<half4v*>(p.yh + prow * p.d + col) = hv;
                if (n == 0) p.yexp[prow * ny + tr.r * 4 + wave] = ex;
              }
            } else if (row < tr.m) {
              const float w = ldexpf(p.wbd ? (&sm.pw[kq * 4])[rb * 16 + v] : 1.0f, -rx0[rb * 16 + v]);
              *reinterpret_cast<float4*>(p.out + static_cast<int64_t>((&sm.rowoff[0][kq * 4])[rb * 16 + v]) * p.d + col) =
                  make_float4(acc[rb][0][v] * w, acc[rb][1][v] * w, acc[rb][2][v] * w, acc[rb][3][v] * w);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rb][j] = float4v{0.f, 0.f, 0.f, 0.f};
      }
    }

    lds_barrier();  // every wave is done with tile i's activations and scales
    if constexpr (BS::kStaged) {
      bulk_store_act<kPhase>(sm, kbuf(min(i + 1, ntile - 1)), tid, st, tex);
      // Tables of tile i + 2's segment, when it starts one (tile i + 1's
      // segment, in the other buffer, is the one in use).
      if (i + 2 < ntile && new_seg(i + 2))
        bulk_unit_tables<kPhase>(p, sm, tile_ref<kPhase>(p, vt(i + 2)), kbuf(i + 2), tid);
    } else {
      if (i + 1 < ntile && new_seg(i + 1)) bulk_unit_act<kPhase>(p, sm, ref[c1], vt(i + 1) / per_unit, tid);
    }
    sm.scales[tid] = sc[c1];
  };
  int i = 0;
  if constexpr (kBulkRing == 2) {
    for (; i + 2 <= ntile; i += 2) {
      step(i, std::integral_constant<int, 0>{});
      step(i + 1, std::integral_constant<int, 1>{});
    }
    if (i < ntile) step(i, std::integral_constant<int, 0>{});
  } else {
    for (; i + 3 <= ntile; i += 3) {
      step(i, std::integral_constant<int, 0>{});
      step(i + 1, std::integral_constant<int, 1>{});
      step(i + 2, std::integral_constant<int, 2>{});
    }
    if (i < ntile) step(i, std::integral_constant<int, 0>{});
    if (i + 1 < ntile) step(i + 1, std::integral_constant<int, 1>{});
  }
}

// ---------------------------------------------------------------------------
// Tile layout (latent_tiles_repack)
// ---------------------------------------------------------------------------
// Each factor tensor holds its own tiles, expert-major (expert e's tiles are
// the same byte range of the tensor as its rows in the row layout):
//   K tiles  gate_a, up_a, down_a: 256-row K slices (all 256 columns), tile t
//            = rows 256 t ..; 32 KB of codes, 4 KB of scales;
//   N tiles  down_b: 256-column slices (all 256 rows), tile t = columns 256 t ..;
//   H tiles  gate_b, up_b: 128-column half tiles (all 256 rows), 16 KB + 2 KB.
// A tile's codes are 16-byte units, one per (wave w, K step s or step pair
// sp, lane): unit (w * 8 + s) * 64 + lane of a K / N tile holds, in dword j,
// the code pairs of rows 32 s + 8 kq + (2q, 2q + 1) (byte q, low nibble = even
// row) of column 64 w + 4 n + j (n = lane & 15, kq = lane >> 4); unit
// (w * 4 + sp) * 64 + lane of an H tile holds in dword 2 h + jj the code pairs
// of K step s = 2 sp + h, column 32 w + 2 n + jj.  Scales: dword G * 128 + (P
// ^ 8 (G & 1)) holds the fp16 scales of rows 2P and 2P + 1 of the tile's
// 32-column group G (8 groups in a K / N tile, 4 in an H tile).
enum TileKind { kKindK = 0, kKindN, kKindH };

__host__ __device__ inline int tile_kind(int f) {
  return f == F_GATE_B || f == F_UP_B ? kKindH : f == F_DOWN_B ? kKindN : kKindK;
}

struct RepackParams {
  uint8_t* rcodes;    // row layout: u8 [E][rows][cols / 2]
  uint16_t* rscales;  //             u16 [E][rows][cols / 32]
  uint8_t* tcodes;    // tile layout, same sizes
  uint16_t* tscales;
  int kind;
  int64_t rows, cols;
  int64_t code_units;    // 16-byte units over all experts (0: codes not repacked)
  int64_t scale_dwords;  // scale dwords over all experts (0: scales not repacked)
};

// Row base and column (within the expert) of dword dw of code unit u of an
// expert's tile-layout codes: byte q of the dword holds rows rbase + 2q
// (low nibble) and rbase + 2q + 1 of that column.
__device__ __forceinline__ void unit_coords(int kind, int64_t u, int dw, int64_t& rbase, int64_t& col) {
  const int per = kind == kKindH ? kHalfCodeBytes / 16 : kCodeBytes / 16;
  const int64_t t = u / per;
  const int k16 = static_cast<int>(u - t * per);
  const int lane = k16 % kWave, nn = lane & 15, kq = lane >> 4;
  if (kind == kKindH) {
    const int w = k16 / (kSteps / 2 * kWave), sp = (k16 / kWave) % (kSteps / 2);
    rbase = (2 * sp + (dw >> 1)) * 32 + kq * 8;
    col = t * kHBlock + 32 * w + 2 * nn + (dw & 1);
  } else {
    const int w = k16 / (kSteps * kWave), s = (k16 / kWave) % kSteps;
    rbase = (kind == kKindK ? t * kK : 0) + s * 32 + kq * 8;
    col = (kind == kKindN ? t * kN : 0) + 64 * w + 4 * nn + dw;
  }
}

// Row pair and group (within the expert) of scale dword i of an expert's
// tile-layout scales: the scales of rows `row` and row + 1.
__device__ __forceinline__ void scale_coords(int kind, int64_t i, int64_t& row, int64_t& grp) {
  const int per = kind == kKindH ? kHalfScaleBytes / 4 : kScaleBytes / 4;
  const int64_t t = i / per;
  const int dw = static_cast<int>(i - t * per);
  const int G = dw / 128, P = (dw % 128) ^ ((G & 1) << 3);
  row = (kind == kKindK ? t * kK : 0) + 2 * P;
  grp = kind == kKindK ? G : t * (kind == kKindN ? kN / kGroup : kHBlock / kGroup) + G;
}

// One direction of the repack, grid-stride over the code units, then the
// scale dwords: kToTiles gathers each tile unit's 32 nibbles from the row
// layout; the inverse scatters them back as whole row bytes (the columns of a
// row byte, 2c and 2c + 1, are dwords (0, 1) or (2, 3) of one unit).
template <bool kToTiles>
__global__ void __launch_bounds__(kT) repack_kernel(RepackParams rp) {
  const int64_t upe = rp.rows * rp.cols / 32;            // code units per expert
  const int64_t dpe = rp.rows * rp.cols / kGroup / 2;    // scale dwords per expert
  const int64_t rstride = rp.cols / 2, sstride = rp.cols / kGroup;
  const int64_t n = rp.code_units + rp.scale_dwords;
  for (int64_t g = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; g < n; g += static_cast<int64_t>(gridDim.x) * kT) {
    if (g < rp.code_units) {
      const int64_t e = g / upe, u = g - e * upe;
      uint8_t* rbytes = rp.rcodes + e * rp.rows * rstride;
      uint4* tunit = reinterpret_cast<uint4*>(rp.tcodes) + g;
      if constexpr (kToTiles) {
        uint32_t out[4];
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
          int64_t rb, c;
          unit_coords(rp.kind, u, dw, rb, c);
          uint32_t word = 0;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const uint8_t v = rbytes[(rb + q) * rstride + c / 2];
            word |= static_cast<uint32_t>((v >> ((c & 1) * 4)) & 15u) << (4 * q);
          }
          out[dw] = word;
        }
        *tunit = make_uint4(out[0], out[1], out[2], out[3]);
      } else {
        const uint4 in = *tunit;
        const uint32_t w[4] = {in.x, in.y, in.z, in.w};
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          int64_t rb, c;
          unit_coords(rp.kind, u, 2 * pr, rb, c);  // dword 2 pr + 1: column c + 1, same rows
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const uint32_t lo = (w[2 * pr] >> (4 * q)) & 15u, hi = (w[2 * pr + 1] >> (4 * q)) & 15u;
            rbytes[(rb + q) * rstride + c / 2] = static_cast<uint8_t>(lo | (hi << 4));
          }
        }
      }
    } else {
      const int64_t i = g - rp.code_units;
      const int64_t e = i / dpe, k = i - e * dpe;
      int64_t row, grp;
      scale_coords(rp.kind, k, row, grp);
      uint16_t* rs = rp.rscales + e * rp.rows * sstride;
      uint32_t* ts = reinterpret_cast<uint32_t*>(rp.tscales) + i;
      if constexpr (kToTiles) {
        *ts = static_cast<uint32_t>(rs[row * sstride + grp]) | (static_cast<uint32_t>(rs[(row + 1) * sstride + grp]) << 16);
      } else {
        const uint32_t v = *ts;
        rs[row * sstride + grp] = static_cast<uint16_t>(v & 0xFFFFu);
        rs[(row + 1) * sstride + grp] = static_cast<uint16_t>(v >> 16);
      }
    }
  }
}

}  // namespace
}  // namespace stream
}  // namespace latent

// ===========================================================================
// Host side
// ===========================================================================
namespace latent {

Factor make_factor(const latent_factor& f);

namespace stream {

static bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Layers the tile layout exists for: pure NF4, rank 256, d and ff multiples of 256.
bool tiles_shape_ok(const latent_moe_args& a) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs)
    if (f->int8_bitmap || f->int8_row_offset || f->int8_data) return false;
  return a.max_rank == kK && a.n_embd % kK == 0 && a.n_ff % kK == 0 && a.n_expert >= 1 && a.n_expert <= 4096 &&
         a.n_embd <= (1 << 16) && a.n_ff <= (1 << 16);
}

// A call whose factors are in the tile layout: the shapes it exists for and
// 16-byte aligned code and scale tensors (the kernels' 128-bit loads).
static bool tiles_given(const latent_moe_args& a) {
  if (a.layout != LATENT_LAYOUT_TILES || !tiles_shape_ok(a)) return false;
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs)
    if (!f->codes || !f->scales || !aligned16(f->codes) || !aligned16(f->scales)) return false;
  return true;
}

template <typename Prm>
static void set_tiles(const latent_moe_args& a, Prm& p) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (int i = 0; i < kFactors; ++i) {
    p.codes[i] = fs[i]->codes;
    p.scales[i] = reinterpret_cast<const uint8_t*>(fs[i]->scales);
  }
}

bool supported(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  return tiles_given(a) && P >= 1 && P <= kMaxPairs && aligned16(a.x);
}

int64_t max_units(int64_t pairs, int64_t experts) { return std::min(pairs, experts) + pairs / kMaxM; }

// Workgroups the item kernels' tile ranges are cut for: two per CU.
static int grid_size() {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kGroupsPerCU * 256;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = kGroupsPerCU * cus;
  }
  return cache[dev];
}

// Partial-sum slots of a K-tiled phase (per_unit tiles per unit, per_key per
// segment key) for at most `units` units on G workgroups.
static int64_t part_slots(int64_t units, int per_unit, int per_key, int G) {
  const int64_t total = units * per_unit;
  const int64_t chunk = (total + G - 1) / G;
  const int64_t maxj = (chunk + per_key - 1) / per_key + 1;
  return static_cast<int64_t>(G) * maxj;
}

bool bulk_supported(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  // 32-bit byte offsets into x, h and the latents.
  return tiles_given(a) && P >= 1 && a.n_tokens * a.n_embd * 2 < (1ll << 31) && P * a.n_ff * 2 < (1ll << 31) &&
         P * kK * 4 < (1ll << 31);
}

size_t bulk_part_bytes(const latent_moe_args& a, int64_t max_units) {
  (void)a;
  // One partial per whole key (A's (unit, factor) keys outnumber C's units)
  // and kRemPieces per workgroup for the pieces of the rest keys (Deal).
  return static_cast<size_t>(2 * max_units + kRemPieces * (grid_size() & ~7)) * kBulkM * kN * 4;
}

int bulk_forward(const latent_moe_args& a, const BulkArgs& bk, int64_t max_units, hipStream_t s) {
  Params p{};
  set_tiles(a, p);
  p.nunits = bk.nunits;
  p.unit_info = bk.units;
  p.pair_tok = bk.pair_tok;
  p.pair_slot = bk.pair_slot;
  p.pair_w = bk.pair_w;
  p.xh = bk.xh;
  p.xexp = bk.xexp;
  p.partA = p.partC = bk.part;  // A's partials are summed before C writes its own
  p.lat = bk.lat;
  p.lexp = bk.lexp;
  p.hh = bk.hh;
  p.hexp = bk.hexp;
  p.dlat = bk.dlat;
  p.dexp = bk.dexp;
  p.yh = bk.y;
  p.yexp = bk.yexp;
  p.out = static_cast<float*>(a.out);
  p.T = static_cast<int>(a.n_tokens);
  p.K = static_cast<int>(a.n_expert_used);
  p.E = static_cast<int>(a.n_expert);
  p.d = static_cast<int>(a.n_embd);
  p.ff = static_cast<int>(a.n_ff);
  p.P = p.T * p.K;
  p.wbd = a.weight_before_down ? 1 : 0;
  p.out_mode = a.out_mode;
  p.nka = p.d / kK;
  p.nb = p.ff / kHBlock;
  p.nkc = p.ff / kK;
  p.nd = p.d / kN;
  p.G = grid_size() & ~7;  // whole XCDs: the bulk kernels deal keys XCD by XCD (b % 8)
  const int64_t U = max_units;
  auto rblocks = [](int64_t rows) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(2048, (rows + kT / kWave - 1) / (kT / kWave))));
  };
  // Every workgroup is launched (those the dealing leaves without a key
  // return at once), so each XCD's block of keys is covered.
  hipLaunchKernelGGL(bulk_kernel<kPhaseA>, dim3(p.G), dim3(kT), 0, s, p);
  hipLaunchKernelGGL((reduce_kernel<kPhaseA, kBulkM, false, true>), dim3(rblocks(U * 2 * kBulkM / 8)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(bulk_kernel<kPhaseB>, dim3(p.G), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(bulk_kernel<kPhaseC>, dim3(p.G), dim3(kT), 0, s, p);
  // C's reduce sums only the rest keys' pieces (a whole key's sum is in its
  // slot); D finishes the rows as it stages them.
  hipLaunchKernelGGL((reduce_kernel<kPhaseC, kBulkM, false, true>), dim3(rblocks(p.G * kBulkM / 8)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL(bulk_kernel<kPhaseD>, dim3(p.G), dim3(kT), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

// Workgroups of the small-batch chain for a call: the resident count (two
// per CU) when every unit count up to the call's maximum fits it, else the
// fewest beyond it (a multiple of 8, at most kLiteMaxGrid times the resident count) with
// which they all fit; 0 when the call does not take the chain.
static int lite_grid(const latent_moe_args& a) {
  const char* env = std::getenv("LATENT_STREAM_LAUNCH");
  if (env && !std::strcmp(env, "phases")) return 0;
  if (!supported(a)) return 0;
  const int64_t P = a.n_tokens * a.n_expert_used;
  if (P < 1 || P > kLiteMaxP || a.n_embd / kK > kMaxKTiles) return 0;
  if (a.n_tokens * a.n_embd * 4 >= (1ll << 31)) return 0;  // 32-bit byte offsets into x
  const int nka = static_cast<int>(a.n_embd / kK), nb = static_cast<int>(a.n_ff / kHBlock);
  const int nd = static_cast<int>(a.n_embd / kN);
  if ((kLiteTicketInts + 3 * kLiteMaxP * kLiteUnitStride + a.n_tokens * nd * kLiteKeyStride) * 4 >
      static_cast<int64_t>(kLiteCtrlBytes))
    return 0;
  // Partial sums in the decode layout's regions: A's 2 nka blocks of P rows.
  if (2ll * nka * P > part_slots(max_units(P, a.n_expert), 2 * nka, nka, grid_size()) * kMaxM) return 0;
  const int G0 = grid_size();
  const int umax = static_cast<int>(std::min<int64_t>(P, max_units(P, a.n_expert)));
  auto all_fit = [&](int G) {
    for (int U = 1; U <= umax; ++U)
      if (!lite_fits(U, nka, nb, nd, G)) return false;
    return true;
  };
  if (all_fit(G0)) return G0;
  // Lower bound: every unit's BC items plus A and D tiles in full slots.
  int G = G0;
  for (int U = 1; U <= umax; ++U) {
    const int need = U * nb + (2 * U * nka + kLiteSlots - 1) / kLiteSlots + (U * nd + kLiteSlots - 1) / kLiteSlots;
    G = std::max(G, (need + 7) / 8 * 8);
  }
  for (; G <= kLiteMaxGrid * G0; G += 8)
    if (all_fit(G)) return G;
  return 0;
}

bool lite_applies(const latent_moe_args& a) { return lite_grid(a) > 0; }

int lite_forward(const latent_moe_args& a, char* ctrl, char* scratch, int* err, hipStream_t s) {
  const Layout L = layout_for(a);
  LiteParams p{};
  set_tiles(a, p);
  p.x = a.x;
  p.x_dtype = a.x_dtype;
  p.ids = a.ids;
  p.weights = a.weights;
  p.w_dtype = a.weights_dtype;
  p.out = static_cast<float*>(a.out);
  // The partial sums sit in the decode layout's partial regions: A's 2 nka
  // blocks of P rows (lite_grid checks they fit A's slots) and C's nb blocks
  // of P rows (the size of C's region).
  p.partA = reinterpret_cast<float*>(scratch + L.partA);
  p.partC = reinterpret_cast<float*>(scratch + L.partC);
  p.ybuf = reinterpret_cast<float*>(scratch + L.ybuf);
  const int G = lite_grid(a);
  if (G <= 0) return LATENT_E_UNSUPPORTED;
  int* c = reinterpret_cast<int*>(ctrl + kLiteCtrlOffset);
  p.ticket = G > grid_size() ? c : nullptr;
  p.resident = grid_size();
  c += kLiteTicketInts;
  p.cntA = c;
  p.cntC = c + kLiteMaxP * kLiteUnitStride;
  p.cntD = c + 2 * kLiteMaxP * kLiteUnitStride;
  p.cntY = c + 3 * kLiteMaxP * kLiteUnitStride;
  p.err = err;
  p.T = static_cast<int>(a.n_tokens);
  p.K = static_cast<int>(a.n_expert_used);
  p.E = static_cast<int>(a.n_expert);
  p.d = static_cast<int>(a.n_embd);
  p.P = p.T * p.K;
  p.wbd = a.weight_before_down ? 1 : 0;
  p.nka = p.d / kK;
  p.nb = static_cast<int>(a.n_ff / kHBlock);
  p.nkc = static_cast<int>(a.n_ff / kK);
  p.nd = p.d / kN;
  if (a.out_mode == LATENT_OUT_REDUCED)
    hipLaunchKernelGGL(lite_kernel<LATENT_OUT_REDUCED>, dim3(G), dim3(kT), 0, s, p);
  else
    hipLaunchKernelGGL(lite_kernel<LATENT_OUT_PER_SLOT>, dim3(G), dim3(kT), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

Layout layout_for(const latent_moe_args& a) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const int64_t T = a.n_tokens, P = a.n_tokens * a.n_expert_used, d = a.n_embd, ff = a.n_ff;
  const int64_t U = max_units(P, a.n_expert);
  const int G = grid_size();
  const int nka = static_cast<int>(d / kK);
  // Partial blocks of 16 rows: A per workgroup range and segment.  C's
  // partials are rows by grouped pair, nkc per pair (bc_kernel: one per item
  // and row).  The small-batch chain (at most 32 routed pairs) keeps its
  // partials in the same regions as [factor block][pair] rows: 2 nka blocks
  // of A (fewer than A's slots here) and nb blocks of P rows of C.
  const int64_t blocksA = part_slots(U, 2 * nka, nka, G);
  const int64_t rowsC = P * (ff / kHBlock);
  Layout L{};
  size_t off = 0;
  L.xh = off;     off = al(off + static_cast<size_t>(T) * d * 2);
  L.xexp = off;   off = al(off + static_cast<size_t>(T) * 4);
  L.partA = off;  off = al(off + static_cast<size_t>(blocksA) * kMaxM * kN * 4);
  L.lath = off;   off = al(off + 2ull * P * kK * 2);
  L.lexp = off;   off = al(off + 2ull * P * 4);
  L.partC = off;  off = al(off + static_cast<size_t>(rowsC) * kN * 4);
  L.dlath = off;  off = al(off + static_cast<size_t>(P) * kK * 2);
  L.dexp = off;   off = al(off + static_cast<size_t>(P) * 4);
  L.ybuf = off;   off = al(off + static_cast<size_t>(P) * d * 4);
  L.pos_of = off; off = al(off + static_cast<size_t>(P) * 4);
  L.total = off;
  return L;
}

int forward(const latent_moe_args& a, const Grouping& g, char* scratch, hipStream_t s) {
  const Layout L = layout_for(a);
  Params p{};
  set_tiles(a, p);
  p.meta = g.meta;
  p.nunits = g.meta + 4;
  p.unit_info = g.unit_info;
  p.unit_tok = g.unit_tok;
  p.pos_of = reinterpret_cast<const int*>(scratch + L.pos_of);
  p.ids = a.ids;
  p.weights = a.weights;
  p.w_dtype = a.weights_dtype;
  p.out = static_cast<float*>(a.out);
  p.xh = reinterpret_cast<const _Float16*>(scratch + L.xh);
  p.xexp = reinterpret_cast<const int*>(scratch + L.xexp);
  p.partA = reinterpret_cast<float*>(scratch + L.partA);
  p.lat = reinterpret_cast<_Float16*>(scratch + L.lath);
  p.lexp = reinterpret_cast<int*>(scratch + L.lexp);
  p.partC = reinterpret_cast<float*>(scratch + L.partC);
  p.dlat = reinterpret_cast<_Float16*>(scratch + L.dlath);
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
  p.nka = p.d / kK;
  p.nb = p.ff / kHBlock;
  p.nkc = p.ff / kK;
  p.nd = p.d / kN;
  p.G = grid_size();
  const int64_t U = max_units(p.P, a.n_expert);
  auto blocks = [](int64_t n) { return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(2048, n))); };
  // At most G workgroups; fewer when the phase has fewer tiles than that even
  // at the largest unit count (the others would find an empty range).
  auto item_grid = [&](int64_t per_unit) { return static_cast<unsigned>(std::min<int64_t>(p.G, U * per_unit)); };
  const int rows_per_block = kT / kWave;
  hipLaunchKernelGGL(item_kernel<kPhaseA>, dim3(item_grid(2 * p.nka)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL((reduce_kernel<kPhaseA, kMaxM>), dim3(blocks((U * 2 * kMaxM + rows_per_block - 1) / rows_per_block)),
                     dim3(kT), 0, s, p);
  hipLaunchKernelGGL(bc_kernel, dim3(item_grid(p.nkc)), dim3(kT), 0, s, p);
  hipLaunchKernelGGL((reduce_kernel<kPhaseC, kMaxM, true>), dim3(blocks((U * kMaxM + rows_per_block - 1) / rows_per_block)),
                     dim3(kT), 0, s, p);
  hipLaunchKernelGGL(item_kernel<kPhaseD>, dim3(item_grid(p.nd)), dim3(kT), 0, s, p);
  const int64_t out4 = (a.out_mode == LATENT_OUT_REDUCED ? p.T : static_cast<int64_t>(p.P)) * p.d / 4;
  hipLaunchKernelGGL(combine_kernel, dim3(blocks((out4 + kT - 1) / kT)), dim3(kT), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace stream
}  // namespace latent

extern "C" int latent_tiles_supported(const latent_moe_args* args) {
  if (!args) return LATENT_E_INVALID;
  return latent::stream::tiles_shape_ok(*args) ? 1 : 0;
}

extern "C" int latent_tiles_repack(int32_t factor, const latent_factor* src, latent_factor* dst, int64_t n_expert,
                                   int32_t to_tiles, latent_stream_t stream) {
  using namespace latent;
  using namespace latent::stream;
  if (!src || !dst || factor < 0 || factor >= kFactors || n_expert < 1) return LATENT_E_INVALID;
  if (src->rows != dst->rows || src->cols != dst->cols) return LATENT_E_INVALID;
  if (src->int8_bitmap || src->int8_row_offset || src->int8_data || dst->int8_bitmap || dst->int8_row_offset ||
      dst->int8_data)
    return LATENT_E_UNSUPPORTED;  // the tile layout is pure NF4
  if (!src->codes != !dst->codes || !src->scales != !dst->scales || (!src->codes && !src->scales))
    return LATENT_E_INVALID;
  const int kind = tile_kind(factor);
  const int64_t rows = src->rows, cols = src->cols;
  const bool ok = kind == kKindK ? cols == kN && rows > 0 && rows % kK == 0
                : kind == kKindN ? rows == kK && cols > 0 && cols % kN == 0
                                 : rows == kK && cols > 0 && cols % kHBlock == 0;
  if (!ok) return LATENT_E_UNSUPPORTED;
  const latent_factor* tile_side = to_tiles ? dst : src;
  if ((tile_side->codes && !aligned16(tile_side->codes)) || (tile_side->scales && !aligned16(tile_side->scales)))
    return LATENT_E_INVALID;
  RepackParams rp{};
  const latent_factor* rows_side = to_tiles ? src : dst;
  rp.rcodes = const_cast<uint8_t*>(rows_side->codes);
  rp.rscales = const_cast<uint16_t*>(rows_side->scales);
  rp.tcodes = const_cast<uint8_t*>(tile_side->codes);
  rp.tscales = const_cast<uint16_t*>(tile_side->scales);
  rp.kind = kind;
  rp.rows = rows;
  rp.cols = cols;
  rp.code_units = src->codes ? n_expert * rows * cols / 32 : 0;
  rp.scale_dwords = src->scales ? n_expert * rows * cols / kGroup / 2 : 0;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const int64_t n = rp.code_units + rp.scale_dwords;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(8192, (n + kT - 1) / kT));
  if (to_tiles)
    hipLaunchKernelGGL(repack_kernel<true>, dim3(blocks), dim3(kT), 0, s, rp);
  else
    hipLaunchKernelGGL(repack_kernel<false>, dim3(blocks), dim3(kT), 0, s, rp);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}
