// Fused decode path: the whole MoE-layer expert FFN in ONE persistent kernel.
//
// Replaces kernels/latent_fused_expert_ffn.cu:27-132 and its per-token launch
// loop (:255-289) for decode-sized batches (T*k <= 512 routed pairs).
//
// Structure
//   * Every workgroup (two per CU, 8 waves each) builds a 16 KB codebook table in LDS
//     and computes the token->expert grouping of all T*k pairs itself (cheap at
//     decode sizes), so no grid-wide step precedes the work.
//   * Work items, per active expert:  A  rows of A_g / A_u      -> g_lat, u_lat
//                                      BC ff slice of B_g, B_u -> h -> h . A_d rows
//                                      D  d slice of B_d       -> y -> output
//     Experts are spread over 8 queues, one per XCD (workgroup b runs on XCD
//     b % 8), so one expert's partial sums stay in one L2.  Workgroups take
//     tickets from their queue; a queue lists all A items, then BC, then D, so a
//     waiting item only ever waits on items already taken by running workgroups.
//   * A and BC items write partial sums; the last item of an expert to finish
//     (per-expert counter) adds them in a fixed order and publishes a ready
//     flag; cross-workgroup data moves through coherent (sc1) loads and stores.
//     Results are deterministic.
//   * Counters are reset by their last user, so the control block is zero again
//     when the kernel ends; it must be zero before the first call.
//
// Dequant: a code byte b (two NF4 codes) indexes lut[b] = (level[b & 15],
// level[b >> 4]) as a float2; the table is replicated for 8 lanes to spread
// LDS banks, and the address is (b << 6) | (lane % 8) * 8.
// The group scale is folded into the activation: acc += (x * s) * level, fp32.
#include "common.hpp"
#include "fused.hpp"
#include "stream.hpp"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <type_traits>

namespace latent {

Factor make_factor(const latent_factor& f);

namespace fused {
namespace {

constexpr int kW = 8;            // waves per workgroup (two workgroups per CU)
constexpr int kNT = kW * kWave;  // 512 threads
constexpr int kMB = 4;           // tokens per pass
constexpr int kLutCopies = 8;
constexpr int kLutEntries = 256 * kLutCopies;
constexpr int64_t kSpinTicks = 100000000;  // 1 s of s_memrealtime (100 MHz)
constexpr int kFactorArgsBytes = 6 * 64;   // LDS table of the six factor descriptors

struct Ctrl {
  int ticket[8];
  int exit_count;
  int error;
  int pad[6];
};

static_assert(offsetof(Ctrl, error) == kErrorOffset, "error word offset");

struct ExpertSync {
  int cA, rA, cB, rB, cD, pad[3];
};

struct Params {
  Factor fac[6];
  const void* x;
  const int32_t* ids;
  const void* weights;
  const int32_t* ranks;
  float* out;
  Ctrl* ctrl;
  ExpertSync* sync;  // [a_max]
  int* ycnt;         // [T][ncd]
  float* partA;      // [2][nca][P][R]
  float* glat;       // [P][2R]
  float* partB;      // [ncb][P][R]
  float* dlat;       // [P][R]
  float* ybuf;       // [P][d]
  int x_dtype, w_dtype;
  int T, d, ff, E, K, R, P;
  int wbd, out_mode;
  int ra, nca;  // phase A: rows per item, items per expert and factor
  int cb, ncb;  // phase BC: ff columns per item, items per expert
  int cd, ncd;  // phase D: d columns per item, items per expert
};

__device__ __forceinline__ int next_pow2(int v) { return v <= 1 ? 1 : 1 << (32 - __builtin_clz(v - 1)); }
__device__ __forceinline__ int ilog2(int v) { return 31 - __builtin_clz(v); }

__device__ __forceinline__ int rank_of(const Params& p, int e, int kind) {
  if (!p.ranks) return p.R;
  const int r = p.ranks[e * 3 + kind];
  return r < 0 ? 0 : (r > p.R ? p.R : r);
}

// ---------------------------------------------------------------------------
// LDS layout
// ---------------------------------------------------------------------------
struct FactorArgs;

// Fixed LDS layout (compile-time offsets: every LDS access uses an immediate
// address, so no scalar registers hold array bases).  The routing scratch
// (w, cnt, start, whist) is only live inside route() and shares its space with
// the activation / slice / cross-wave buffers used afterwards.
constexpr int kMaxP = 512;                    // routed pairs (T * k)
static_assert(kMaxP <= kNT, "route() ranks the active experts with one thread each");
constexpr int kMaxEx = 512;                   // experts
constexpr int kVMax = 1024;                   // staged activation floats per token
constexpr int kCbMax = 512;                   // ff columns of a BC slice
constexpr int kRedFloats = kMB * (kW / 2) * 256;  // cross-wave partial slots: (wr / 2) * M * ncols

struct SmemLayout {
  alignas(16) char fac[kFactorArgsBytes];
  float2 lut[kLutEntries];
  int act_e[kMaxP], act_s[kMaxP], act_c[kMaxP];
  int pr_tok[kMaxP], pr_slot[kMaxP];
  float pr_w[kMaxP];
  int pos_of[kMaxP];
  int nvalid[kMaxP];
  int misc[16];
  alignas(16) char emit[64];
  union alignas(16) {
    struct {
      float w[kMaxP];
      int cnt[kMaxEx];
      int start[kMaxEx];
      int whist[kW][kMaxEx];  // pairs of each expert per wave
    } route;
    struct {
      float vin[kMB * kVMax];
      float hs[kMB * kCbMax];
      float red[kRedFloats];
    } work;
  } u;
};

struct EmitArgs;

struct Smem {
  FactorArgs* fac; // [6] factor descriptors (kept in LDS, not in scalar registers)
  float2* lut;     // [256][kLutCopies]
  float* w;        // [P]
  int* cnt;        // [E]
  int* start;      // [E]
  int* whist;      // [kW][kMaxEx]
  int* act_e;      // [A]
  int* act_s;      // [A]
  int* act_c;      // [A]
  int* pr_tok;     // [P] pairs grouped by expert
  int* pr_slot;    // [P]
  float* pr_w;     // [P]
  int* pos_of;     // [P] position of pair t*K+slot, -1 if dropped
  int* nvalid;     // [T]
  int* misc;       // [16]: 0 n_active, 1 broadcast, 2 ticket
  float* vin;      // [kMB][kVMax]
  float* hs;       // [kMB][cb]  (g of the BC slice, then h)
  float* red;      // cross-wave partials
  EmitArgs* emit;  // the current tile's output description
};

__device__ __forceinline__ Smem carve(SmemLayout& m) {
  Smem s;
  s.fac = reinterpret_cast<FactorArgs*>(m.fac);
  s.lut = m.lut;
  s.w = m.u.route.w;
  s.cnt = m.u.route.cnt;
  s.start = m.u.route.start;
  s.whist = &m.u.route.whist[0][0];
  s.act_e = m.act_e;
  s.act_s = m.act_s;
  s.act_c = m.act_c;
  s.pr_tok = m.pr_tok;
  s.pr_slot = m.pr_slot;
  s.pr_w = m.pr_w;
  s.pos_of = m.pos_of;
  s.nvalid = m.nvalid;
  s.misc = m.misc;
  s.emit = reinterpret_cast<EmitArgs*>(m.emit);
  s.vin = m.u.work.vin;
  s.hs = m.u.work.hs;
  s.red = m.u.work.red;
  return s;
}

// ---------------------------------------------------------------------------
// Routing, computed identically by every workgroup (deterministic order:
// experts ascending, pairs of one expert in increasing t*K + slot).
// ---------------------------------------------------------------------------
__device__ void route(const Params& p, const Smem& s) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  // One routed pair per thread (P <= kMaxP <= kNT).
  const int i = tid;
  int e = -1;
  if (i < p.P) {
    e = p.ids[i];
    s.w[i] = load_act(p.weights, p.w_dtype, i);
    s.pos_of[i] = -1;
  }
  const bool valid = e >= 0 && e < p.E;
  for (int k = tid; k < kW * p.E; k += kNT) s.whist[(k / p.E) * kMaxEx + k % p.E] = 0;
  for (int t = tid; t < p.T; t += kNT) s.nvalid[t] = 0;
  __syncthreads();
  if (valid) atomicAdd(&s.nvalid[i / p.K], 1);
  // Within each wave, group the lanes by expert (one ballot per distinct
  // expert of the wave): a pair's rank among the wave's earlier pairs of its
  // expert, and the wave's count of each expert.
  int my_rank = 0;
  uint64_t rem = __ballot(valid);
  while (rem != 0) {
    const int leader = __ffsll(static_cast<unsigned long long>(rem)) - 1;
    const int e0 = __shfl(e, leader);
    const uint64_t m = __ballot(valid && e == e0);
    if (valid && e == e0) my_rank = __popcll(m & ((uint64_t{1} << lane) - 1));
    if (lane == leader) s.whist[wave * kMaxEx + e0] = __popcll(m);
    rem &= ~m;
  }
  __syncthreads();
  for (int ee = tid; ee < p.E; ee += kNT) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) c += s.whist[w * kMaxEx + ee];
    s.cnt[ee] = c;
  }
  __syncthreads();
  if (tid < kWave) {
    // One wave scans the expert counts (E <= kMaxE).  An expert with more than
    // kMB pairs is split into work units ("active entries") of at most kMB
    // pairs each, so no item runs a second batch and the units of one expert
    // run side by side.
    int run = 0, act = 0;
    for (int base = 0; base < p.E; base += kWave) {
      const int e = base + tid;
      const int c = e < p.E ? s.cnt[e] : 0;
      const int nu = (c + kMB - 1) / kMB;
      int incl = c, ai = nu;
      for (int off = 1; off < kWave; off <<= 1) {
        const int v = __shfl_up(incl, off);
        const int va = __shfl_up(ai, off);
        if (tid >= off) {
          incl += v;
          ai += va;
        }
      }
      if (e < p.E) {
        s.start[e] = run + incl - c;
        for (int u = 0; u < nu; ++u) {
          const int a = act + ai - nu + u;
          s.act_e[a] = e;
          s.act_s[a] = run + incl - c + u * kMB;
          s.act_c[a] = min(kMB, c - u * kMB);
        }
      }
      run += __shfl(incl, kWave - 1);
      act += __shfl(ai, kWave - 1);
    }
    if (tid == 0) s.misc[0] = act;
  }
  __syncthreads();
  // Placement: pair i goes to start[e] + (pairs of e in earlier waves) + (its
  // rank in its wave), so the pairs of one expert keep their order.
  if (valid) {
    int pos = s.start[e] + my_rank;
    for (int w = 0; w < wave; ++w) pos += s.whist[w * kMaxEx + e];
    const int tok = i / p.K;
    s.pr_tok[pos] = tok;
    s.pr_slot[pos] = i - tok * p.K;
    s.pr_w[pos] = s.w[i];
    s.pos_of[i] = pos;
  }
  // Active entries by pair count, largest first (ties by index), so each queue
  // starts its longest items first.  Counts are 1..kMB: the rank is the number
  // of entries with a larger count plus the earlier entries with the same one
  // (wave ballots within a wave, per-wave totals through LDS across waves).
  __syncthreads();
  const int n_active = s.misc[0];
  int my_e = 0, my_s = 0, my_c = 0;
  if (tid < n_active) {
    my_e = s.act_e[tid];
    my_s = s.act_s[tid];
    my_c = s.act_c[tid];
  }
  int below = 0;
#pragma unroll
  for (int v = 1; v <= kMB; ++v) {
    const uint64_t mask = __ballot(my_c == v);
    if (my_c == v) below = __popcll(mask & ((uint64_t{1} << lane) - 1));
    if (lane == 0) s.cnt[wave * kMB + v - 1] = __popcll(mask);
  }
  __syncthreads();
  int rank = below;
  if (tid < n_active) {
    for (int w = 0; w < kW; ++w) {
#pragma unroll
      for (int v = 1; v <= kMB; ++v) {
        const int n = s.cnt[w * kMB + v - 1];
        rank += (v > my_c || (v == my_c && w < wave)) ? n : 0;
      }
    }
  }
  __syncthreads();
  if (tid < n_active) {
    s.act_e[rank] = my_e;
    s.act_s[rank] = my_s;
    s.act_c[rank] = my_c;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Item bookkeeping.  Queue q holds active experts queue_expert(q, k), k = 0, 1, ...
// Items of a queue: [A: nq*2*nca][BC: nq*ncb][D: nq*ncd][Z: zero rows]
// ---------------------------------------------------------------------------
// Active experts are ranked by token count (largest first) and dealt to the
// queues in a snake order: ranks 8k .. 8k+7 go to queues 0..7 for even k and
// 7..0 for odd k, so every queue gets a like mix of heavy and light experts.
__device__ __forceinline__ int queue_expert(int q, int k) { return 8 * k + ((k & 1) ? 7 - q : q); }
__device__ __forceinline__ int experts_in_queue(int n_active, int q) {
  const int full = n_active / 8, r = n_active % 8;
  const bool extra = (full & 1) ? (7 - q) < r : q < r;
  return full + (extra ? 1 : 0);
}

// Zero work for outputs no D item writes: tokens with no valid slot (reduced
// mode) or dropped slots (per-slot mode); one item per (row, d slice).
__device__ __forceinline__ int zero_rows(const Params& p, const Smem& s, int q, int idx, bool count_only) {
  // Rows are enumerated in order; row r belongs to queue r % 8.
  int n = 0;
  const int rows = p.out_mode == LATENT_OUT_REDUCED ? p.T : p.P;
  for (int r = q; r < rows; r += 8) {
    const bool need = p.out_mode == LATENT_OUT_REDUCED ? (s.nvalid[r] == 0) : (s.pos_of[r] < 0);
    if (need) {
      if (!count_only && n == idx) return r;
      ++n;
    }
  }
  return count_only ? n : -1;
}

// ---------------------------------------------------------------------------
// Cross-workgroup signalling.  Data that another workgroup reads is written and
// read with agent-scope relaxed atomics (single sc1 loads / stores, coherent
// across XCDs without L2 write-back or invalidate).  A producer's waves drain
// their stores (s_waitcnt) before the barrier that precedes the counter
// update; counters and flags are relaxed agent-scope atomics.  No release or
// acquire fences: on gfx950 those write back / invalidate the whole L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void drain_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Bounded spin on a flag.  On timeout the error word is set and the workgroup
// proceeds, so the kernel always terminates.
__device__ void wait_flag(const Params& p, int* flag) {
  if (threadIdx.x == 0) {
    const int64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      __builtin_amdgcn_s_sleep(1);
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
        __hip_atomic_store(&p.ctrl->error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// Arrive on a counter; true in every thread of the workgroup that is the last
// of `total` arrivals.
__device__ bool arrive_last(int* counter, int total, int* bcast) {
  drain_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *bcast = (old == total - 1);
  }
  __syncthreads();
  return *bcast != 0;
}

__device__ void publish(int* flag) {
  drain_stores();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Tile GEMV.  y[t][j] = sum_{rows r} vin[t][r] * scale(r, g0 + j/32) * level(code(r, 32*g0 + j))
// for rows [r0, r1), groups [g0, g0 + G) (G a power of two), t < M.
// Lane layout: lpr lanes along groups x rpw lanes along rows in each wave;
// wg waves along groups x wr waves along rows.  Every argument is a plain
// value so the kernel-argument block never needs an address.
// ---------------------------------------------------------------------------
// Global-address-space pointers: keep loads as global_load_* across calls.
#define LATENT_GLOBAL_AS __attribute__((address_space(1)))
template <typename T>
using gptr = const T LATENT_GLOBAL_AS*;
template <typename T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
  return (gptr<T>)(p);
}
// The same global address in every lane, made visibly uniform so the compiler
// keeps it in scalar registers (loads then use scalar base + 32-bit offset).
template <typename T>
__device__ __forceinline__ gptr<T> uniform(gptr<T> p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<gptr<T>>((static_cast<uint64_t>(hi) << 32) | lo);
}
#define LATENT_LDS_AS __attribute__((address_space(3)))
template <typename T>
using lptr = T LATENT_LDS_AS*;
template <typename T>
__device__ __forceinline__ lptr<T> as_lds(T* p) {
  return (lptr<T>)(p);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

struct FactorArgs {
  gptr<uint8_t> codes;
  gptr<uint16_t> scales;
  gptr<uint32_t> bitmap;
  gptr<int32_t> word_offset;  // [E][rows][words]: first INT8 group index of each bitmap word
  gptr<int8_t> data;
  int64_t rows, cols;
};

static_assert(sizeof(FactorArgs) <= kFactorArgsBytes / 6, "factor table slot");

// The six factor descriptors are copied to LDS once per workgroup: held in
// scalar registers for the whole kernel they would crowd out everything else.
__device__ __forceinline__ void stage_factors(const Params& p, const Smem& s) {
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const Factor& f = p.fac[i];
      s.fac[i] = FactorArgs{as_global(f.codes), as_global(f.scales), as_global(f.ext.bitmap),
                            as_global(f.ext.word_offset), as_global(f.ext.data), f.rows, f.cols};
    }
  }
}

__device__ __forceinline__ FactorArgs fargs(const Smem& s, int i) { return s.fac[i]; }

// One tile GEMV of a workgroup:
//   y[t][j] = sum_{r0 <= r < r1} vin[t][r - vbase] * scale(r, g0 + j/32) * level(code(r, 32*g0 + j))
// for the g_valid groups starting at g0 (G = next power of two >= g_valid),
// t < m, written as dst[rowoff[t] + j] = y * scale[t], or with swiglu set as
// dst[...] = SiLU(dst[...]) * y * scale[t] (dst then holds the gate).
struct Job {
  FactorArgs f;
  int64_t e;
  int r0, r1, g0, G, g_valid;
  lptr<const float> vin;
  int vstride, vbase;
  float* dst;
  int64_t rowoff[kMB];
  float scale[kMB];
  int swiglu;
  int coherent;  // dst is read by another workgroup: store with st_coh
};

template <typename T>
__device__ __forceinline__ T pick_t(int t, const T (&a)[kMB]) {
  return t == 0 ? a[0] : t == 1 ? a[1] : t == 2 ? a[2] : a[3];
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// What a tile's final pass needs to write its rows.  It is staged in LDS by
// thread 0 when the tile starts and read back after the tile's fold barriers,
// so none of it stays in registers through the streaming loop.
struct EmitArgs {
  float* dst;
  int64_t rowoff[kMB];
  float scale[kMB];
  int swiglu;
  int coherent;
};

static_assert(sizeof(EmitArgs) <= 64, "LDS slot of the emit arguments");

__device__ __forceinline__ void stage_emit(const Job& j, lptr<EmitArgs> ea) {
  if (threadIdx.x == 0) {
    ea->dst = j.dst;
#pragma unroll
    for (int t = 0; t < kMB; ++t) {
      ea->rowoff[t] = j.rowoff[t];
      ea->scale[t] = j.scale[t];
    }
    ea->swiglu = j.swiglu;
    ea->coherent = j.coherent;
  }
}

__device__ __forceinline__ void emit_one(lptr<const EmitArgs> ea, int t, int col, float v) {
  const float scale = ea->scale[t];
  float* q = ea->dst + ea->rowoff[t] + col;
  if (ea->coherent)
    st_coh(q, v * scale);
  else
    *q = ea->swiglu ? silu_f32(*q) * v * scale : v * scale;
}

// A lane owns half a group: 16 columns (8 code bytes) of one row per step.
constexpr int kHalf = kGroup / 2;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// acc[t][j] += xs[t] * level(code j) for the 16 columns of one half group.
template <int M>
__device__ __forceinline__ void fma_half_nf4(const u32x2& c, const float (&xs)[M], lptr<const char> lut,
                                             uint32_t lanebase, float (&acc)[M][kHalf]) {
  f32x2 v[8];
  const uint32_t cw[2] = {c.x, c.y};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t addr = (((cw[i] >> (8 * b)) & 0xFFu) << 6) | lanebase;  // entry stride kLutCopies x 8 B
      v[i * 4 + b] = *reinterpret_cast<lptr<const f32x2>>(lut + addr);
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
#pragma unroll
    for (int t = 0; t < M; ++t) {
      acc[t][2 * k] = fmaf(xs[t], v[k].x, acc[t][2 * k]);
      acc[t][2 * k + 1] = fmaf(xs[t], v[k].y, acc[t][2 * k + 1]);
    }
  }
}

// Same for a half group stored as INT8: its 16 values, in q.
template <int M>
__device__ __forceinline__ void fma_half_int8(const u32x4& q, const float (&xs)[M], float (&acc)[M][kHalf]) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float v = static_cast<float>(static_cast<int8_t>((qw[i] >> (8 * b)) & 0xFFu));
#pragma unroll
      for (int t = 0; t < M; ++t) acc[t][i * 4 + b] = fmaf(xs[t], v, acc[t][i * 4 + b]);
    }
  }
}

// Raw buffer over a whole array (on: kFbufBytes of range; off: an empty
// range), and its loads.  A load at kFbufBytes or beyond (or from an empty
// range) returns zero without touching memory.
constexpr uint32_t kFbufBytes = 0x7FFFFF00u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fbuf(const void* base, bool on) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           on ? static_cast<int>(kFbufBytes) : 0, 0x00020000);
}
__device__ __forceinline__ uint32_t fld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ u32x4 fld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return u32x4{v[0], v[1], v[2], v[3]};
}

// Row-lane reduction + cross-wave fold of a tile's accumulators.
//
// Lanes of one half group h are spread over rpw row lanes (lane = ro * lph + hl).
// With rpw == 4 (lph == 16) the row lanes are reduced by a transposing
// butterfly of lane-half swaps (permlane32 pairs ro with ro ^ 2, permlane16 ro
// with ro ^ 1): each step adds two accumulators of a lane pair and keeps one of
// them per lane, so the values a lane holds halve per step and every lane ends
// with a distinct quarter of the reduced half group: value i is acc[t][c] with
// t * 16 + c = 4 i + 2 (ro & 1) + (ro >> 1).  The shares then go to an LDS slot
// per row wave, and the caller sums the wr slots in order and emits whole rows.
__device__ __forceinline__ float2 swap32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 swap16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int M>
__device__ __forceinline__ void fold_rows(float (&acc)[M][kHalf], lptr<float> red, int h, int ro, bool hvalid, int wri,
                                          int ncols) {
  constexpr int N = M * kHalf, NV = N / 4;
  float w[N / 2], v[NV];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float2 r = swap32(acc[(2 * i) / kHalf][(2 * i) % kHalf], acc[(2 * i + 1) / kHalf][(2 * i + 1) % kHalf]);
    w[i] = r.x + r.y;
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float2 r = swap16(w[2 * i], w[2 * i + 1]);
    v[i] = r.x + r.y;
  }
  // Every row wave stores its own slot (wr * M * ncols = kW * 16 * kHalf * M
  // <= kRedFloats floats for M <= 2), so one barrier ends the fold.
  static_assert(M <= 2, "one fold slot per row wave");
  const int sel = 2 * (ro & 1) + (ro >> 1);
  if (hvalid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int n = 4 * i + sel, t = n / kHalf, c = n % kHalf;
      red[(wri * M + t) * ncols + h * kHalf + c] = v[i];
    }
  }
  __syncthreads();
}

// Same for rpw >= 8 (tiles narrower than 16 half groups): xor shuffles over the
// row lanes, then row lane 0 holds the whole half group.
template <int M>
__device__ __forceinline__ void fold_rows_shfl(float (&acc)[M][kHalf], lptr<float> red, int h, int ro, bool hvalid,
                                               int wri, int wr, int ncols, int lph) {
  for (int off = lph; off < kWave; off <<= 1) {
#pragma unroll
    for (int t = 0; t < M; ++t)
#pragma unroll
      for (int c = 0; c < kHalf; ++c) acc[t][c] += __shfl_xor(acc[t][c], off);
  }
  const bool writer = ro == 0 && hvalid;
  const int slots = wr > 1 ? wr / 2 : 1;
  if (writer && wri < slots) {
#pragma unroll
    for (int t = 0; t < M; ++t) {
      lptr<float> dst = red + (wri * M + t) * ncols + h * kHalf;
#pragma unroll
      for (int c = 0; c < kHalf; ++c) dst[c] = acc[t][c];
    }
  }
  __syncthreads();
  if (wr == 1) return;
  if (writer && wri >= slots) {
#pragma unroll
    for (int t = 0; t < M; ++t) {
      lptr<float> dst = red + ((wri - slots) * M + t) * ncols + h * kHalf;
#pragma unroll
      for (int c = 0; c < kHalf; ++c) dst[c] += acc[t][c];
    }
  }
  __syncthreads();
}

// Tile GEMV over half groups: H = 2G half groups, lanes along half groups (lph
// per row; 16 lanes = one 128-byte row segment) x rows; waves along half
// groups (wg) x rows (wr).  The in-wave sum runs over the row lanes; the
// cross-wave sum folds the upper half of the row slices onto the lower half,
// then adds the lower slices in order (fixed order, deterministic).  M is the
// token capacity of the accumulators, m <= M the tokens present.
template <int M, bool kInt8>
__device__ __forceinline__ void tile_gemv(const Job& j, int m, lptr<const char> lut, lptr<float> red,
                                          lptr<EmitArgs> ea) {
  stage_emit(j, ea);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int H = 2 * j.G, h_valid = 2 * j.g_valid;
  int lph, wg;
  if (H <= 16) {
    lph = H;
    wg = 1;
  } else {
    lph = max(16, H / kW);
    wg = H / lph;
  }
  const int wr = kW / wg;
  const int rpw = kWave / lph;
  const int hl = lane & (lph - 1);             // half group within the wave's slice
  const int ro = lane >> ilog2(lph);           // row lane
  const int wgi = wave % wg, wri = wave / wg;  // wave's half-group slice / row slice
  const int h = wgi * lph + hl;                // half group within the tile
  const int rstep = wr * rpw;
  const uint32_t lanebase = static_cast<uint32_t>(lane & (kLutCopies - 1)) << 3;
  const FactorArgs& f = j.f;
  const int64_t cstride = f.cols / 2, sstride = f.cols / kGroup;

  float acc[M][kHalf];
#pragma unroll
  for (int t = 0; t < M; ++t)
#pragma unroll
    for (int c = 0; c < kHalf; ++c) acc[t][c] = 0.f;

  // Rows of this lane: row_l + k*rstep for k < nsteps (nsteps uniform across
  // the wave); the lane's valid rows are those below r1 (nv of them).  Loads
  // past them re-read the lane's last valid row (or r0 for none) and are
  // masked by a zero scale, so every access stays inside the expert.
  const int r0 = j.r0, r1 = j.r1;
  const int row_w = r0 + wri * rpw;
  const int nsteps = row_w < r1 ? (r1 - 1 - row_w) / rstep + 1 : 0;
  const int row_l = row_w + ro;
  const bool hvalid = h < h_valid;
  const int nv = (hvalid && row_l < r1) ? (r1 - 1 - row_l) / rstep + 1 : 0;
  const int row0 = max(r0, min(row_l, r1 - 1));
  const int rowz = nv > 0 ? row_l + (nv - 1) * rstep : row0;
  const int hh = hvalid ? h : 0;
  const int gg = j.g0 + (hh >> 1), half = hh & 1;
  // Expert bases are uniform (scalar registers); lanes address with 32-bit
  // offsets from them, clamped to the lane's last valid row.
  const gptr<uint8_t> cexp = uniform(f.codes + j.e * f.rows * cstride);
  const gptr<uint8_t> sexp = uniform(reinterpret_cast<gptr<uint8_t>>(f.scales + j.e * f.rows * sstride));
  const uint32_t ccol = static_cast<uint32_t>(gg * kGroupBytes + half * (kGroupBytes / 2));
  const uint32_t c_first = static_cast<uint32_t>(row0) * static_cast<uint32_t>(cstride) + ccol;
  const uint32_t c_last = static_cast<uint32_t>(rowz) * static_cast<uint32_t>(cstride) + ccol;
  // Scale offsets in bytes.
  const uint32_t s_first = 2u * (static_cast<uint32_t>(row0) * static_cast<uint32_t>(sstride) + gg);
  const uint32_t s_last = 2u * (static_cast<uint32_t>(rowz) * static_cast<uint32_t>(sstride) + gg);
  const uint32_t cdelta = static_cast<uint32_t>(rstep) * static_cast<uint32_t>(cstride);
  const uint32_t sdelta = 2u * static_cast<uint32_t>(rstep) * static_cast<uint32_t>(sstride);
  const int v_first = row0 - j.vbase, v_last = rowz - j.vbase;
  // Ring of kRing rows in flight per lane; slot u is refilled with the row
  // kRing steps ahead right after it is consumed.  Four-token tiles spend
  // their registers on accumulators and do 4x the arithmetic per row, so a
  // shallower ring keeps them inside 128 VGPRs without starving the loads.
  // Layers with INT8 groups run a second, earlier stage: each row's bitmap
  // word and word offset are loaded two rings ahead, and the group's INT8
  // values (an empty load for an NF4 group) one ring ahead, with the codes --
  // so no load waits on another inside the loop.
  constexpr int kRing = (M >= 3 || kInt8) ? 4 : 8;
  // Scales stay raw fp16 bits in the ring: converting at load time would make
  // the refill wait for its own load.
  u32x2 ring[kRing];
  uint32_t sring[kRing];  // one register per scale (16-bit packing would force a wait per refill)
  // INT8 stage (kInt8 only; every load issued, against empty ranges for an NF4 factor).
  uint32_t bring[kInt8 ? kRing : 1], fring[kInt8 ? kRing : 1];
  int32_t pring[kInt8 ? kRing : 1];
  u32x4 qring[kInt8 ? kRing : 1];
  const bool has8 = kInt8 && f.bitmap != nullptr;
  const int words = static_cast<int>((f.cols / kGroup + 31) / 32);
  const uint32_t bit = static_cast<uint32_t>(gg & 31), below = (1u << bit) - 1u;
  const uint32_t b_first = 4u * (static_cast<uint32_t>(row0) * words + (gg >> 5));
  const uint32_t b_last = 4u * (static_cast<uint32_t>(rowz) * words + (gg >> 5));
  const uint32_t bdelta = 4u * static_cast<uint32_t>(rstep) * words;
  const int64_t eb = j.e * f.rows * words;
  auto generic = [](auto q) { return reinterpret_cast<const void*>(reinterpret_cast<uintptr_t>(q)); };
  const __amdgpu_buffer_rsrc_t rbm = fbuf(has8 ? generic(f.bitmap + eb) : nullptr, has8);
  const __amdgpu_buffer_rsrc_t rwo = fbuf(has8 ? generic(f.word_offset + eb) : nullptr, has8);
  const __amdgpu_buffer_rsrc_t rdt = fbuf(has8 ? generic(f.data) : nullptr, has8);
  auto stage_a = [&](int slot, uint32_t boff) __attribute__((always_inline)) {
    if constexpr (kInt8) {
      bring[slot] = fld32(rbm, boff);
      pring[slot] = static_cast<int32_t>(fld32(rwo, boff));
    }
  };
  auto stage_b = [&](int slot) __attribute__((always_inline)) {
    if constexpr (kInt8) {
      const uint32_t flag = (bring[slot] >> bit) & 1u;
      const uint32_t idx = static_cast<uint32_t>(pring[slot]) + static_cast<uint32_t>(popc(bring[slot] & below));
      qring[slot] = fld128(rdt, flag ? idx * kGroup + half * kHalf : kFbufBytes);
      fring[slot] = flag;
    }
  };
#pragma unroll
  for (int u = 0; u < kRing; ++u) stage_a(u, min(b_first + u * bdelta, b_last));
#pragma unroll
  for (int u = 0; u < kRing; ++u) {
    stage_b(u);
    ring[u] = *reinterpret_cast<gptr<u32x2>>(cexp + min(c_first + u * cdelta, c_last));
    sring[u] = *reinterpret_cast<gptr<uint16_t>>(sexp + min(s_first + u * sdelta, s_last));
    stage_a(u, min(b_first + (u + kRing) * bdelta, b_last));
    __builtin_amdgcn_sched_barrier(0);  // issue in consumption order
  }
  uint32_t ck = c_first, sk = s_first, bk = b_first;
  int vk = v_first;
  // One block of kRing steps; with kRefill each consumed slot is reloaded with
  // the row kRing steps ahead.  The last block runs without refills, so no
  // load is left in flight when the tile ends (a dangling load would make the
  // next tile wait for it, and for every store before it, once its register
  // is reused).
  auto block = [&](int k0, auto refill) {
#pragma unroll
    for (int u = 0; u < kRing; ++u) {
      const int k = k0 + u;
      const float sm = k < nv ? half_bits_to_float(sring[u]) : 0.f;
      const int vr = min(vk + u * rstep, v_last);
      float xs[M];
#pragma unroll
      for (int t = 0; t < M; ++t) xs[t] = j.vin[t * j.vstride + vr] * sm;
      // A branch on the group's format: the lanes of a wave diverge only where
      // INT8 and NF4 groups meet (a select over both decodes measured 3x slower).
      if (kInt8 && fring[u] != 0) {
        if constexpr (kInt8) fma_half_int8<M>(qring[u], xs, acc);
      } else {
        fma_half_nf4<M>(ring[u], xs, lut, lanebase, acc);
      }
      if constexpr (decltype(refill)::value) {
        // Pin the refill between this step and the next.  Hoisted above the
        // step, its load would need a fresh register and a copy at the loop
        // latch, and that copy waits for every load in flight; sunk below, it
        // loses the distance to its use.  Either way the ring stops hiding the
        // memory latency.
        __builtin_amdgcn_sched_barrier(0);
        stage_b(u);  // row k + kRing, from the bitmap word loaded a ring ago
        ring[u] = *reinterpret_cast<gptr<u32x2>>(cexp + min(ck + (u + kRing) * cdelta, c_last));
        sring[u] = *reinterpret_cast<gptr<uint16_t>>(sexp + min(sk + (u + kRing) * sdelta, s_last));
        stage_a(u, min(bk + (u + 2 * kRing) * bdelta, b_last));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    ck += kRing * cdelta;
    sk += kRing * sdelta;
    bk += kRing * bdelta;
    vk += kRing * rstep;
  };
  int k0 = 0;
  for (; k0 + kRing < nsteps; k0 += kRing) block(k0, std::true_type{});
  if (k0 < nsteps) block(k0, std::false_type{});
  const int ncols = H * kHalf;
  // lph = 16 whenever H >= 16 (at most 64 half groups per tile), so the row
  // lanes are 4 there; narrower tiles have 8 or more.
  int slots;
  if constexpr (M <= 2) {
    if (rpw == 4) {
      fold_rows<M>(acc, red, h, ro, hvalid, wri, ncols);
      slots = wr;
    } else {
      fold_rows_shfl<M>(acc, red, h, ro, hvalid, wri, wr, ncols, lph);
      slots = wr > 1 ? wr / 2 : 1;
    }
  } else {
    fold_rows_shfl<M>(acc, red, h, ro, hvalid, wri, wr, ncols, lph);
    slots = wr > 1 ? wr / 2 : 1;
  }
  const int nvalid_cols = h_valid * kHalf;
  for (int i = tid; i < m * nvalid_cols; i += kNT) {
    const int t = i / nvalid_cols, col = i - t * nvalid_cols;
    float v = 0.f;
    for (int w = 0; w < slots; ++w) v += red[(w * M + t) * ncols + col];
    emit_one(ea, t, col, v);
  }
  __syncthreads();
}

// The one place the tile is expanded (accumulator capacities 1 to 4 tokens).
template <bool kInt8>
__device__ __forceinline__ void run_tile(const Job& j, int m, const Smem& s) {
  const lptr<const char> lut = reinterpret_cast<lptr<const char>>(as_lds(static_cast<const float2*>(s.lut)));
  const lptr<float> red = as_lds(s.red);
  const lptr<EmitArgs> ea = as_lds(s.emit);
  if (m == 1)
    tile_gemv<1, kInt8>(j, 1, lut, red, ea);
  else if (m == 2)
    tile_gemv<2, kInt8>(j, 2, lut, red, ea);
  else if (m == 3)
    tile_gemv<3, kInt8>(j, 3, lut, red, ea);
  else
    tile_gemv<4, kInt8>(j, m, lut, red, ea);
}

// ---------------------------------------------------------------------------
// Staging and reduction helpers.  Loads are issued in batches before any use
// so one item pays one memory round trip per batch, not one per element.
// ---------------------------------------------------------------------------
// x rows of up to kMB tokens, columns [c0, c0 + n) (n % 8 == 0, c0 % 8 == 0),
// converted to fp32 into dst[t * dstride + j].
__device__ __forceinline__ void stage_x(const Params& p, const int* toks, int m, int c0, int n, float* dst,
                                        int dstride) {
  const int tid = threadIdx.x;
  for (int j0 = tid * 8; j0 < n; j0 += kNT * 8) {
    float v[kMB][8];
#pragma unroll
    for (int t = 0; t < kMB; ++t) {
      if (t < m) {
        const int64_t base = static_cast<int64_t>(toks[t]) * p.d + c0 + j0;
        if (p.x_dtype == LATENT_F32) {
          const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + base);
          const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + base + 4);
          v[t][0] = a.x; v[t][1] = a.y; v[t][2] = a.z; v[t][3] = a.w;
          v[t][4] = b.x; v[t][5] = b.y; v[t][6] = b.z; v[t][7] = b.w;
        } else {
          const uint4 hv = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.x) + base);
          const uint32_t w[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (p.x_dtype == LATENT_BF16) {
              v[t][2 * i] = __uint_as_float(w[i] << 16);
              v[t][2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            } else {
              v[t][2 * i] = half_bits_to_float(static_cast<uint16_t>(w[i] & 0xFFFFu));
              v[t][2 * i + 1] = half_bits_to_float(static_cast<uint16_t>(w[i] >> 16));
            }
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kMB; ++t) {
      if (t < m) {
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[t * dstride + j0 + i] = v[t][i];
      }
    }
  }
}

// Coherent rows src[t * sstride + j] (j < n) of up to kMB tokens into LDS.
__device__ __forceinline__ void stage_coh(const float* src, int64_t sstride, int m, int n, float* dst, int dstride) {
  for (int j = threadIdx.x; j < n; j += kNT) {
    float v[kMB];
#pragma unroll
    for (int t = 0; t < kMB; ++t) v[t] = t < m ? ld_coh(src + t * sstride + j) : 0.f;
#pragma unroll
    for (int t = 0; t < kMB; ++t)
      if (t < m) dst[t * dstride + j] = v[t];
  }
}

// sum_{c < n} src[c * cstride], loads batched 8 at a time, summed in c order.
__device__ __forceinline__ float sum_coh(const float* src, int64_t cstride, int n) {
  float acc = 0.f;
  for (int c0 = 0; c0 < n; c0 += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = c0 + i < n ? ld_coh(src + (c0 + i) * cstride) : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += v[i];
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Items.  An item is a list of tile jobs per batch of up to kMB of the
// expert's pairs, bracketed by a prologue (wait for its inputs) and an
// epilogue (partial-sum reduction / output combine / counter reset):
//   A  (kind, chunk): rows [chunk*ra, +ra) of A_g (kind 0) or A_u (kind 1)
//                     x -> partA[kind][chunk]
//   BC (chunk):       ff columns [chunk*cb, +cb):  g_lat . B_g -> hs,
//                     hs = SiLU(hs) * (u_lat . B_u), hs . A_d rows -> partB[chunk]
//   D  (chunk):       d columns [chunk*cd, +cd) of d_lat . B_d -> out / ybuf
// ---------------------------------------------------------------------------
enum ItemType { kItemA = 0, kItemBC = 1, kItemD = 2, kItemZ = 3 };

struct Item {
  int type, a, kind, chunk;
  int e, s0, mtot;
};

__device__ __forceinline__ int groups_of(int rank) { return (rank + kGroup - 1) / kGroup; }

// Stage the batch's activations (tokens tb.., m of them) into LDS.
__device__ __forceinline__ void stage_batch(const Params& p, const Smem& s, const Item& it, int tb, int m) {
  if (it.type == kItemA) {
    const int r0 = it.chunk * p.ra, nrows = min(p.d, r0 + p.ra) - r0;
    stage_x(p, s.pr_tok + it.s0 + tb, m, r0, nrows, s.vin, kVMax);
  } else if (it.type == kItemBC) {
    stage_coh(p.glat + static_cast<int64_t>(it.s0 + tb) * 2 * p.R, 2 * p.R, m, 2 * p.R, s.vin, kVMax);
  } else {
    const int n = groups_of(rank_of(p, it.e, 2)) * kGroup;
    stage_coh(p.dlat + static_cast<int64_t>(it.s0 + tb) * p.R, p.R, m, n, s.vin, kVMax);
  }
}

// Tile job `sub` of the batch at tb; false if there is nothing to compute.
__device__ __forceinline__ bool make_job(const Params& p, const Smem& s, const Item& it, int sub, int tb, int m,
                                         Job& j) {
  j.e = it.e;
  j.swiglu = 0;
  j.coherent = 0;
  j.vin = as_lds(static_cast<const float*>(s.vin));
  j.vstride = kVMax;
  j.vbase = 0;
  j.g0 = 0;
#pragma unroll
  for (int t = 0; t < kMB; ++t) j.scale[t] = 1.0f;
  if (it.type == kItemA) {
    const int ng = groups_of(rank_of(p, it.e, it.kind));
    j.f = fargs(s, it.kind == 0 ? 0 : 2);
    j.r0 = it.chunk * p.ra;
    j.r1 = min(p.d, j.r0 + p.ra);
    j.G = next_pow2(ng);
    j.g_valid = ng;
    j.vbase = j.r0;
    j.dst = p.partA + ((static_cast<int64_t>(it.kind) * p.nca + it.chunk) * p.P + it.s0 + tb) * p.R;
#pragma unroll
    for (int t = 0; t < kMB; ++t) j.rowoff[t] = static_cast<int64_t>(t) * p.R;
    j.coherent = 1;
    return ng > 0 && j.r1 > j.r0;
  }
  if (it.type == kItemBC) {
    const int c0 = it.chunk * p.cb, ncol = min(p.cb, p.ff - c0);
    if (ncol <= 0) return false;
    if (sub < 2) {
      // g = g_lat . B_g (sub 0) into hs, then hs = SiLU(hs) * (u_lat . B_u) (sub 1).
      j.f = fargs(s, sub == 0 ? 1 : 3);
      j.r0 = 0;
      j.r1 = rank_of(p, it.e, sub);  // an empty row range yields zeros
      j.g0 = c0 / kGroup;
      j.G = next_pow2(p.cb / kGroup);
      j.g_valid = ncol / kGroup;
      j.vin = as_lds(static_cast<const float*>(s.vin + sub * p.R));
      j.dst = s.hs;
#pragma unroll
      for (int t = 0; t < kMB; ++t) j.rowoff[t] = static_cast<int64_t>(t) * p.cb;
      if (sub == 1) {
        j.swiglu = 1;
        if (p.wbd) {
#pragma unroll
          for (int t = 0; t < kMB; ++t) j.scale[t] = s.pr_w[it.s0 + tb + min(t, m - 1)];
        }
      }
      return true;
    }
    // hs . A_d rows [c0, c0 + ncol) -> partial d_lat.
    const int ngd = groups_of(rank_of(p, it.e, 2));
    j.f = fargs(s, 4);
    j.r0 = c0;
    j.r1 = c0 + ncol;
    j.G = next_pow2(ngd);
    j.g_valid = ngd;
    j.vin = as_lds(static_cast<const float*>(s.hs));
    j.vstride = p.cb;
    j.vbase = c0;
    j.dst = p.partB + (static_cast<int64_t>(it.chunk) * p.P + it.s0 + tb) * p.R;
#pragma unroll
    for (int t = 0; t < kMB; ++t) j.rowoff[t] = static_cast<int64_t>(t) * p.R;
    j.coherent = 1;
    return ngd > 0;
  }
  // D: d_lat . B_d, columns [c0, c0 + ncol).
  const int c0 = it.chunk * p.cd, ncol = min(p.cd, p.d - c0);
  j.f = fargs(s, 5);
  j.r0 = 0;
  j.r1 = rank_of(p, it.e, 2);
  j.g0 = c0 / kGroup;
  j.G = next_pow2(p.cd / kGroup);
  j.g_valid = ncol / kGroup;
  const bool per_slot = p.out_mode == LATENT_OUT_PER_SLOT;
  j.coherent = per_slot ? 0 : 1;
  j.dst = (per_slot ? p.out : p.ybuf) + c0;
#pragma unroll
  for (int t = 0; t < kMB; ++t) {
    const int pair = it.s0 + tb + min(t, m - 1);
    if (per_slot) {
      j.rowoff[t] = (static_cast<int64_t>(s.pr_tok[pair]) * p.K + s.pr_slot[pair]) * p.d;
    } else {
      j.rowoff[t] = static_cast<int64_t>(pair) * p.d;
      j.scale[t] = p.wbd ? 1.0f : s.pr_w[pair];
    }
  }
  return ncol > 0;
}

// A: the last A item of the expert sums the partials into g_lat | u_lat.
__device__ __forceinline__ void finish_a(const Params& p, const Smem& s, const Item& it) {
  if (!arrive_last(&p.sync[it.a].cA, 2 * p.nca, &s.misc[1])) return;
  const int ng0 = groups_of(rank_of(p, it.e, 0)) * kGroup;
  const int ng1 = groups_of(rank_of(p, it.e, 1)) * kGroup;
  const int width = ng0 + ng1;
  for (int t = 0; t < it.mtot; ++t) {
    for (int cc = threadIdx.x; cc < width; cc += kNT) {
      const int k = cc < ng0 ? 0 : 1, col = cc < ng0 ? cc : cc - ng0;
      const float v = sum_coh(p.partA + ((static_cast<int64_t>(k) * p.nca) * p.P + it.s0 + t) * p.R + col,
                              static_cast<int64_t>(p.P) * p.R, p.nca);
      st_coh(p.glat + static_cast<int64_t>(it.s0 + t) * 2 * p.R + k * p.R + col, v);
    }
  }
  publish(&p.sync[it.a].rA);
}

// BC: the last BC item of the expert sums the partials into d_lat.
__device__ __forceinline__ void finish_bc(const Params& p, const Smem& s, const Item& it) {
  if (!arrive_last(&p.sync[it.a].cB, p.ncb, &s.misc[1])) return;
  const int width = groups_of(rank_of(p, it.e, 2)) * kGroup;
  for (int t = 0; t < it.mtot; ++t) {
    for (int col = threadIdx.x; col < width; col += kNT) {
      const float v =
          sum_coh(p.partB + static_cast<int64_t>(it.s0 + t) * p.R + col, static_cast<int64_t>(p.P) * p.R, p.ncb);
      st_coh(p.dlat + static_cast<int64_t>(it.s0 + t) * p.R + col, v);
    }
  }
  publish(&p.sync[it.a].rB);
}

// D: in reduced mode the last of a token's valid slots to finish this d slice
// sums them in slot order; the last D item of the expert resets its counters.
__device__ __forceinline__ void finish_d(const Params& p, const Smem& s, const Item& it) {
  const int c0 = it.chunk * p.cd, ncol = min(p.cd, p.d - c0);
  if (p.out_mode == LATENT_OUT_REDUCED && ncol > 0) {
    drain_stores();
    __syncthreads();
    for (int t = 0; t < it.mtot; ++t) {
      const int tok = s.pr_tok[it.s0 + t];
      if (threadIdx.x == 0) {
        int* cnt = &p.ycnt[tok * p.ncd + it.chunk];
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s.misc[1] = (old == s.nvalid[tok] - 1);
        if (old == s.nvalid[tok] - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (s.misc[1]) {
        for (int col = threadIdx.x; col < ncol; col += kNT) {
          float v = 0.f;
          for (int k0 = 0; k0 < p.K; k0 += 8) {
            float y[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int pos = k0 + i < p.K ? s.pos_of[tok * p.K + k0 + i] : -1;
              y[i] = pos >= 0 ? ld_coh(p.ybuf + static_cast<int64_t>(pos) * p.d + c0 + col) : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) v += y[i];
          }
          p.out[static_cast<int64_t>(tok) * p.d + c0 + col] = v;
        }
      }
      __syncthreads();
    }
  }
  if (arrive_last(&p.sync[it.a].cD, p.ncd, &s.misc[1])) {
    if (threadIdx.x == 0) {
      ExpertSync* es = &p.sync[it.a];
      __hip_atomic_store(&es->cA, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&es->rA, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&es->cB, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&es->rB, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&es->cD, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

__device__ __forceinline__ void item_zero(const Params& p, int row, int chunk) {
  const int c0 = chunk * p.cd, ncol = min(p.cd, p.d - c0);
  float* dst = p.out + static_cast<int64_t>(row) * p.d + c0;
  for (int col = threadIdx.x; col < ncol; col += kNT) dst[col] = 0.f;
}

// Waves per SIMD: two workgroups per CU (128 VGPRs) for pure-NF4 layers; one
// workgroup per CU (256 VGPRs) with INT8 groups, whose second decode stage
// spilled 321 VGPRs (372 bytes per lane) at 128.
template <bool kInt8>
constexpr int waves_per_simd() { return kInt8 ? 2 : 4; }

template <bool kInt8>
__global__ void __launch_bounds__(kNT, waves_per_simd<kInt8>()) fused_kernel(Params p) {
  __shared__ SmemLayout smem;
  const Smem s = carve(smem);
  const int tid = threadIdx.x;
  // Codebook table: entry b holds (level[b & 15], level[b >> 4]), one copy per
  // lane of a 16-lane LDS cycle.
  for (int i = tid; i < kLutEntries; i += kNT) {
    const int b = i / kLutCopies;
    s.lut[i] = make_float2(nf4_level(b & 15), nf4_level(b >> 4));
  }
  stage_factors(p, s);
  route(p, s);
  const int n_active = s.misc[0];
  const int q = blockIdx.x & 7;
  const int nq = experts_in_queue(n_active, q);
  const int nA = nq * 2 * p.nca, nB = nq * p.ncb, nD = nq * p.ncd;
  const int nZ = zero_rows(p, s, q, 0, true) * p.ncd;
  const int total = nA + nB + nD + nZ;
  // The next ticket is fetched while the current item runs; thread 0 holds it
  // in a register until the item is done, so no wave waits on the atomic.
  int next_ticket = 0;
  if (tid == 0) next_ticket = __hip_atomic_fetch_add(&p.ctrl->ticket[q], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    if (tid == 0) s.misc[2] = next_ticket;
    __syncthreads();
    int t = s.misc[2];
    __syncthreads();
    if (t >= total) break;
    if (tid == 0) next_ticket = __hip_atomic_fetch_add(&p.ctrl->ticket[q], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Item it;
    it.kind = 0;
    if (t < nA) {
      const int per = 2 * p.nca, r = t % per;
      it.type = kItemA;
      it.a = queue_expert(q, t / per);
      it.kind = r / p.nca;
      it.chunk = r % p.nca;
    } else if ((t -= nA) < nB) {
      it.type = kItemBC;
      it.a = queue_expert(q, t / p.ncb);
      it.chunk = t % p.ncb;
    } else if ((t -= nB) < nD) {
      it.type = kItemD;
      it.a = queue_expert(q, t / p.ncd);
      it.chunk = t % p.ncd;
    } else {
      t -= nD;
      item_zero(p, zero_rows(p, s, q, t / p.ncd, false), t % p.ncd);
      continue;
    }
    it.e = s.act_e[it.a];
    it.s0 = s.act_s[it.a];
    it.mtot = s.act_c[it.a];
    if (it.type == kItemBC) wait_flag(p, &p.sync[it.a].rA);
    if (it.type == kItemD) wait_flag(p, &p.sync[it.a].rB);
    const int nsub = it.type == kItemBC ? 3 : 1;
    for (int tb = 0; tb < it.mtot; tb += kMB) {
      const int m = min(kMB, it.mtot - tb);
      stage_batch(p, s, it, tb, m);
      __syncthreads();
      for (int sub = 0; sub < nsub; ++sub) {
        Job j;
        if (make_job(p, s, it, sub, tb, m, j)) run_tile<kInt8>(j, m, s);
      }
    }
    if (it.type == kItemA)
      finish_a(p, s, it);
    else if (it.type == kItemBC)
      finish_bc(p, s, it);
    else
      finish_d(p, s, it);
  }
  // The last workgroup out resets the queues.
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(&p.ctrl->exit_count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == static_cast<int>(gridDim.x) - 1) {
      for (int i = 0; i < 8; ++i) __hip_atomic_store(&p.ctrl->ticket[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&p.ctrl->exit_count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}
}  // namespace
}  // namespace fused
}  // namespace latent

// ===========================================================================
// Host side
// ===========================================================================
namespace latent {
namespace fused {

// Below kMinPairs routed pairs (one or two tokens at top-8) the multi-kernel
// path is faster: its per-workgroup items are larger than this kernel's.
constexpr int kMinPairs = 32;
constexpr int kMaxPairs = kMaxP;
constexpr int kMaxE = kMaxEx;
constexpr int kWgPerCu = 2;  // two 512-thread workgroups per CU (<= 80 KB of LDS each)
static_assert(sizeof(SmemLayout) <= 80 * 1024, "two workgroups per CU");

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// INT8 groups are read through a buffer resource of kFbufBytes with a 32-bit
// byte offset (group index * 32): a factor qualifies only when even an
// all-INT8 side buffer (every group of every expert) stays below that range.
bool int8_fits(const latent_moe_args& a) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  for (const latent_factor* f : fs) {
    if (!f->int8_bitmap) continue;
    const int64_t groups = a.n_expert * f->rows * (f->cols / kGroup);
    if (groups * kGroup >= static_cast<int64_t>(kFbufBytes)) return false;
  }
  return true;
}

bool supported(const latent_moe_args& a) {
  const int64_t P = a.n_tokens * a.n_expert_used;
  const bool x_aligned = (reinterpret_cast<uintptr_t>(a.x) & 15u) == 0;  // 16-byte vector staging of x
  return P >= kMinPairs && P <= kMaxPairs && a.n_expert <= kMaxE && 2 * a.max_rank <= kVMax && x_aligned &&
         int8_fits(a);
}

static int pick_cols(int64_t extent, double per_xcd, int target, int lo, int hi) {
  int c = hi;
  while (c > lo && static_cast<double>((extent + c - 1) / c) * per_xcd < target) c /= 2;
  return c;
}

bool make_plan(const latent_moe_args& a, Plan& pl) {
  const int64_t T = a.n_tokens, K = a.n_expert_used, E = a.n_expert, R = a.max_rank, d = a.n_embd, ff = a.n_ff;
  const int64_t P = T * K, A = P;  // active entries: at most one per routed pair
  const double est = static_cast<double>(E) * (1.0 - std::pow(1.0 - static_cast<double>(K) / E, static_cast<double>(T)));
  const double per_xcd = std::max(1.0, std::ceil(est / 8.0));
  const double wgs_per_xcd = 32.0 * kWgPerCu;
  pl.cb = pick_cols(ff, per_xcd, 1.5 * wgs_per_xcd, 64, kCbMax);
  pl.ncb = static_cast<int>((ff + pl.cb - 1) / pl.cb);
  // At most 1024 columns (32 groups): the tile then folds its row slices
  // through LDS and stores whole rows (coalesced), never 16-column lane runs.
  pl.cd = pick_cols(d, per_xcd, 1.5 * wgs_per_xcd, 128, 1024);
  pl.ncd = static_cast<int>((d + pl.cd - 1) / pl.cd);
  // One round of A items per queue where the activations fit: 2 * nca items per expert.
  int nca = std::max<int>(1, static_cast<int>(std::floor(wgs_per_xcd / (2.0 * per_xcd))));
  nca = std::max<int>(nca, static_cast<int>((d + 1023) / 1024));
  // Rows per A item: whole groups of rows, at most kVMax (the staged x slice).
  nca = std::min<int>(nca, static_cast<int>(std::max<int64_t>(1, d / kGroup)));
  pl.ra = static_cast<int>(((d + nca - 1) / nca + kGroup - 1) / kGroup * kGroup);
  pl.nca = static_cast<int>((d + pl.ra - 1) / pl.ra);
  if (pl.ra > kVMax || 2 * R > kVMax || pl.cb > kCbMax) return false;
  size_t off = 256;
  pl.off_sync = off;
  off = align256(off + A * sizeof(ExpertSync));
  pl.off_ycnt = off;
  off = align256(off + T * pl.ncd * sizeof(int));
  if (off > stream::kLiteCtrlOffset) return false;  // the small-batch chain's counters follow
  off = 0;
  pl.off_partA = off; off = align256(off + 2ull * pl.nca * P * R * 4);
  pl.off_glat = off;  off = align256(off + P * 2 * R * 4);
  pl.off_partB = off; off = align256(off + static_cast<size_t>(pl.ncb) * P * R * 4);
  pl.off_dlat = off;  off = align256(off + P * R * 4);
  pl.off_ybuf = off;  off = align256(off + P * d * 4);
  pl.scratch_bytes = off;
  return true;
}

// Workgroups that are resident at once: whole XCDs of CUs times the
// workgroups per CU (fewer CUs when the kernel holds more registers).
static int grid_size(int per_cu) {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = std::max(8, n / 8 * 8);
  }
  return cached[dev] * per_cu;
}

template <bool kInt8>
static int launch(const Params& p, hipStream_t s) {
  // 512 threads = 2 waves per SIMD per workgroup.
  const int grid = grid_size(waves_per_simd<kInt8>() / 2);
  if (grid <= 0) return LATENT_E_HIP;
  hipLaunchKernelGGL(fused_kernel<kInt8>, dim3(grid), dim3(kNT), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

int forward(const latent_moe_args& a, hipStream_t s, char* ws, const Plan& pl, const Factor (&fac)[6]) {
  Params p{};
  bool any_int8 = false;
  for (int i = 0; i < 6; ++i) {
    p.fac[i] = fac[i];
    any_int8 = any_int8 || fac[i].ext.bitmap != nullptr;
  }
  char* scratch = ws + kReserved;
  p.x = a.x;
  p.ids = a.ids;
  p.weights = a.weights;
  p.ranks = a.ranks;
  p.out = static_cast<float*>(a.out);
  p.ctrl = reinterpret_cast<Ctrl*>(ws);
  p.sync = reinterpret_cast<ExpertSync*>(ws + pl.off_sync);
  p.ycnt = reinterpret_cast<int*>(ws + pl.off_ycnt);
  p.partA = reinterpret_cast<float*>(scratch + pl.off_partA);
  p.glat = reinterpret_cast<float*>(scratch + pl.off_glat);
  p.partB = reinterpret_cast<float*>(scratch + pl.off_partB);
  p.dlat = reinterpret_cast<float*>(scratch + pl.off_dlat);
  p.ybuf = reinterpret_cast<float*>(scratch + pl.off_ybuf);
  p.x_dtype = a.x_dtype;
  p.w_dtype = a.weights_dtype;
  p.T = static_cast<int>(a.n_tokens);
  p.d = static_cast<int>(a.n_embd);
  p.ff = static_cast<int>(a.n_ff);
  p.E = static_cast<int>(a.n_expert);
  p.K = static_cast<int>(a.n_expert_used);
  p.R = static_cast<int>(a.max_rank);
  p.P = p.T * p.K;
  p.wbd = a.weight_before_down ? 1 : 0;
  p.out_mode = a.out_mode;
  p.ra = pl.ra;
  p.nca = pl.nca;
  p.cb = pl.cb;
  p.ncb = pl.ncb;
  p.cd = pl.cd;
  p.ncd = pl.ncd;
  return any_int8 ? launch<true>(p, s) : launch<false>(p, s);
}

}  // namespace fused
}  // namespace latent
