// MoE-layer LATENT expert FFN on gfx950: routed-token gather + wave64 NF4 GEMV chain.
//
// Replaces kernels/latent_fused_expert_ffn.cu:27-132 (dispatch / per-slot copy /
// reduce kernels) and its host launcher :134-292.  The reference launches one
// 128-thread block per (token, slot) and re-reads every factor per token; here
// tokens are grouped by expert on the device so each routed expert's packed
// factors stream from HBM once per call, split over many workgroups:
//
//   prep     group (token, slot) pairs by expert (histogram, scan, scatter) and
//            clear the fp32 accumulators.
//   phase A  [x]           . A_g | A_u  -> g_lat, u_lat   (split over rows of A)
//   phase BC [g_lat,u_lat] . B_g , B_u  -> h = SiLU(g)*u  (split over ff columns)
//            h[cols]       . A_d[cols]  -> d_lat           (same ff slice)
//   phase D  d_lat         . B_d        -> y, weighted into out (split over d)
//
// Every phase is a GEMV over a row-major [K][N] factor whose 32-column groups
// are one 128-bit load of NF4 codes + one fp16 scale.  A lane owns one group
// (32 output columns) and walks rows; the activation for the row is multiplied
// by the group scale once and then by 32 codebook levels read from a 16-entry
// LDS table.  Lanes sharing a group are combined with wave shuffles, waves
// through LDS, workgroups with fp32 atomics.  All arithmetic is fp32.
#include "common.hpp"
#include "fused.hpp"
#include "prefill.hpp"
#include "rows.hpp"
#include "stream.hpp"

#include <cstdlib>
#include <cstring>

#include <algorithm>

namespace latent {

Factor make_factor(const latent_factor& f);
int check_factor(const latent_factor& f);

namespace {

__constant__ float kLevelsMoe[16] = {
    nf4_level(0),  nf4_level(1),  nf4_level(2),  nf4_level(3),  nf4_level(4),  nf4_level(5),
    nf4_level(6),  nf4_level(7),  nf4_level(8),  nf4_level(9),  nf4_level(10), nf4_level(11),
    nf4_level(12), nf4_level(13), nf4_level(14), nf4_level(15),
};

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxExperts = 4096;  // LDS histogram of the prep kernel
constexpr int kMaxExpertUsed = 64;  // slots per token (the router's limit)
constexpr int kMaxRank = 512;
constexpr int kRouteThreads = 1024;
enum { F_GATE_A = 0, F_GATE_B, F_UP_A, F_UP_B, F_DOWN_A, F_DOWN_B };

struct MoeParams {
  Factor fac[6];
  const void* x;
  const int32_t* ids;
  const void* weights;
  const int32_t* ranks;
  float* out;
  int* meta;  // [0] active experts, [1] invalid ids seen
  int* act_expert;
  int* act_start;
  int* act_count;
  int* pair_tok;
  int* pair_slot;
  float* pair_w;
  float* gu;  // [P][2R]
  float* dl;  // [P][R]
  int4* unit_info;  // streaming path work units {expert, first pair, pairs, 0} (NULL: not built)
  int* unit_tok;    // [units][16] token of each unit row (0 past the unit's pairs)
  int* pos_of;      // [T*K] grouped position of each routed slot (streaming path)
  _Float16* xh;     // streaming path: x as fp16 rows * 2^xexp (NULL: not converted)
  int* xexp;        // [T] row exponents
  int x_dtype, w_dtype;
  int T, d, ff, E, K, R;
  int wbd, out_mode;
  int a_max;             // upper bound of active experts (grid sizing)
  int ra, n_a;           // phase A: rows per item, items per expert (2 * ceil(d/ra))
  int cb, n_bc;          // phase BC: ff columns per item, items per expert
  int cd, n_d;           // phase D: d columns per item, items per expert
  int64_t zero_floats;   // accumulator floats cleared by prep
  int zero_out;          // reduced mode: prep clears out (the phase kernels accumulate into it)
  int clear;             // prep clears the accumulators (and out) also where it converts x
};

__device__ __forceinline__ int ilog2(int v) { return 31 - __builtin_clz(v); }
__device__ __forceinline__ int next_pow2(int v) { return v <= 1 ? 1 : 1 << (32 - __builtin_clz(v - 1)); }

__device__ __forceinline__ int rank_of(const MoeParams& p, int e, int kind) {
  if (!p.ranks) return p.R;
  const int r = p.ranks[e * 3 + kind];
  return r < 0 ? 0 : (r > p.R ? p.R : r);
}

// Workgroup b -> (active expert a, item i) so that all items of one expert land
// on the same XCD (workgroups are dispatched to the 8 XCDs round-robin): their
// shared activations and atomics then stay in one L2.
__device__ __forceinline__ bool map_item(int b, int n_items, int n_active, int& a, int& i) {
  const int x = b & 7;
  const int j = b >> 3;
  a = x + 8 * (j / n_items);
  i = j - (j / n_items) * n_items;
  return a < n_active;
}

// ---------------------------------------------------------------------------
// prep: workgroup 0 groups pairs by expert; the others clear accumulators.
// ---------------------------------------------------------------------------
constexpr int kCached = 4;  // pairs per thread held in registers by route_block
constexpr int kOrderedExperts = 1024;  // route_block places pairs in index order up to this many experts

// Place routed pair i (expert e, weight w) at the expert's next position and
// in its streaming unit's row tables.  start[e] is the expert's first
// position; fill[e] its running insert position.
__device__ __forceinline__ void place_pair(const MoeParams& p, const int* start, const int* ubase, int i, int e,
                                           float w, int pos) {
  const int tok = i / p.K, slot = i - tok * p.K;
  p.pair_tok[pos] = tok;
  p.pair_slot[pos] = slot;
  p.pair_w[pos] = w;
  if (p.unit_info) {
    const int rel = pos - start[e];
    const int row = (ubase[e] + rel / stream::kMaxM) * stream::kMaxM + rel % stream::kMaxM;
    p.unit_tok[row] = tok;
    p.pos_of[i] = pos;
  }
}

// Same, at the expert's next free position (the order among one expert's
// pairs then depends on timing).
__device__ __forceinline__ void scatter_pair(const MoeParams& p, const int* start, int* fill, const int* ubase, int i,
                                             int e, float w) {
  if (e < 0 || e >= p.E) return;
  place_pair(p, start, ubase, i, e, w, atomicAdd(&fill[e], 1));
}

__device__ void route_block(const MoeParams& p) {
  __shared__ int cnt[kMaxExperts];  // pairs per expert, then the expert's first position
  __shared__ int fill[kMaxExperts];
  __shared__ int ubase[kMaxExperts];  // first streaming unit of each expert
  constexpr int kRouteWaves = kRouteThreads / kWave;
  __shared__ int ordered_counts[kRouteWaves * kOrderedExperts];
  __shared__ int wave_sum[3][kRouteWaves];
  __shared__ int bad;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int P = p.T * p.K;
  for (int e = tid; e < p.E; e += kRouteThreads) {
    cnt[e] = 0;
    fill[e] = 0;
  }
  if (tid == 0) bad = 0;
  // The first kCached pairs of each thread stay in registers for the scatter.
  int my_e[kCached];
  float my_w[kCached];
#pragma unroll
  for (int j = 0; j < kCached; ++j) {
    const int i = tid + j * kRouteThreads;
    my_e[j] = i < P ? p.ids[i] : -1;
    my_w[j] = i < P ? load_act(p.weights, p.w_dtype, i) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kCached; ++j) {
    const int e = my_e[j];
    if (e >= 0 && e < p.E)
      atomicAdd(&cnt[e], 1);
    else if (e >= p.E)
      atomicAdd(&bad, 1);
  }
  for (int i = tid + kCached * kRouteThreads; i < P; i += kRouteThreads) {
    const int e = p.ids[i];
    if (e >= 0 && e < p.E)
      atomicAdd(&cnt[e], 1);
    else if (e >= p.E)
      atomicAdd(&bad, 1);
  }
  __syncthreads();
  // Block scan over experts: each thread owns a contiguous run of experts.
  const int per = (p.E + kRouteThreads - 1) / kRouteThreads;
  const int e0 = min(p.E, tid * per), e1 = min(p.E, e0 + per);
  int sc = 0, sa = 0, su = 0;
  for (int e = e0; e < e1; ++e) {
    sc += cnt[e];
    sa += cnt[e] > 0;
    su += (cnt[e] + stream::kMaxM - 1) / stream::kMaxM;
  }
  // Inclusive scan: within the wave by shuffles, then across the waves'
  // totals.
  int ic = sc, ia = sa, iu = su;
  for (int off = 1; off < kWave; off <<= 1) {
    const int vc = __shfl_up(ic, off, kWave), va = __shfl_up(ia, off, kWave), vu = __shfl_up(iu, off, kWave);
    if (lane >= off) {
      ic += vc;
      ia += va;
      iu += vu;
    }
  }
  if (lane == kWave - 1) {
    wave_sum[0][wave] = ic;
    wave_sum[1][wave] = ia;
    wave_sum[2][wave] = iu;
  }
  __syncthreads();
  for (int w = 0; w < wave; ++w) {
    ic += wave_sum[0][w];
    ia += wave_sum[1][w];
    iu += wave_sum[2][w];
  }
  int start = ic - sc;
  int act = ia - sa;
  int unit = iu - su;
  for (int e = e0; e < e1; ++e) {
    const int c = cnt[e];
    fill[e] = start;  // reuse as the running insert position
    cnt[e] = start;
    ubase[e] = unit;
    if (c > 0) {
      p.act_expert[act] = e;
      p.act_start[act] = start;
      p.act_count[act] = c;
      if (p.unit_info) {  // units of at most kMaxM pairs of one expert; rows past the pairs are padding
        for (int j = 0; j < c; j += stream::kMaxM, ++unit) {
          const int m = min(stream::kMaxM, c - j);
          p.unit_info[unit] = make_int4(e, start + j, m, 0);
          for (int r = m; r < stream::kMaxM; ++r) {
            p.unit_tok[unit * stream::kMaxM + r] = 0;
          }
        }
      }
      ++act;
    }
    start += c;
  }
  if (tid == kRouteThreads - 1) {
    p.meta[0] = ia;
    p.meta[1] = bad;
    p.meta[3] = ic;  // routed pairs
    p.meta[4] = iu;  // streaming work units
  }
  __syncthreads();
  const int words = (P + 31) / 32;
  if (p.E * words <= kRouteWaves * kOrderedExperts) {
    // Pairs of one expert land in pair-index order, so the work units (and
    // every sum over them) are the same on every call: a bit mask of each
    // expert's pairs, and a pair's rank is the number of its expert's bits
    // below its own.
    uint32_t* mask = reinterpret_cast<uint32_t*>(ordered_counts);  // [E][words]
    for (int x = tid; x < p.E * words; x += kRouteThreads) mask[x] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kCached; ++j) {
      const int i = tid + j * kRouteThreads, e = my_e[j];
      if (e >= 0 && e < p.E) atomicOr(&mask[e * words + (i >> 5)], 1u << (i & 31));
    }
    for (int i = tid + kCached * kRouteThreads; i < P; i += kRouteThreads) {
      const int e = p.ids[i];
      if (e >= 0 && e < p.E) atomicOr(&mask[e * words + (i >> 5)], 1u << (i & 31));
    }
    __syncthreads();
    auto rank_of = [&](int i, int e) {
      const uint32_t* m = mask + e * words;
      int rank = __builtin_popcount(m[i >> 5] & ((1u << (i & 31)) - 1u));
      for (int x = 0; x < (i >> 5); ++x) rank += __builtin_popcount(m[x]);
      return rank;
    };
#pragma unroll
    for (int j = 0; j < kCached; ++j) {
      const int i = tid + j * kRouteThreads, e = my_e[j];
      if (e >= 0 && e < p.E) place_pair(p, cnt, ubase, i, e, my_w[j], cnt[e] + rank_of(i, e));
    }
    for (int i = tid + kCached * kRouteThreads; i < P; i += kRouteThreads) {
      const int e = p.ids[i];
      if (e >= 0 && e < p.E) place_pair(p, cnt, ubase, i, e, load_act(p.weights, p.w_dtype, i), cnt[e] + rank_of(i, e));
    }
    return;
  }
  if (p.E <= kOrderedExperts) {
    // Same order for layers whose masks do not fit, in rounds of
    // kRouteThreads pairs: within a wave, ballots rank the pairs of each
    // expert and count them; a scan over the waves' counts (per expert, in
    // wave order, after the earlier rounds) gives each wave's insert base.
    int* wcnt = ordered_counts;  // [waves][E]
    const int rounds = (P + kRouteThreads - 1) / kRouteThreads;
    for (int r = 0; r < rounds; ++r) {
      const int i = r * kRouteThreads + tid;
      int e = -1;
      float w = 0.f;
      if (r < kCached) {
#pragma unroll
        for (int j = 0; j < kCached; ++j) {
          if (j == r) {
            e = my_e[j];
            w = my_w[j];
          }
        }
      } else if (i < P) {
        e = p.ids[i];
        w = load_act(p.weights, p.w_dtype, i);
      }
      const int key = e >= 0 && e < p.E ? e : -1;
      for (int x = tid; x < kRouteWaves * p.E; x += kRouteThreads) wcnt[x] = 0;
      __syncthreads();
      int rank = 0;
      uint64_t todo = __ballot(1);
      while (todo) {
        const int leader = __ffsll(static_cast<unsigned long long>(todo)) - 1;
        const int kl = __shfl(key, leader, kWave);
        const uint64_t same = __ballot(key == kl);
        if (key == kl) {
          rank = __popcll(same & ((1ull << lane) - 1ull));
          if (lane == leader && kl >= 0) wcnt[wave * p.E + kl] = __popcll(same);
        }
        todo &= ~same;
      }
      __syncthreads();
      for (int x = tid; x < p.E; x += kRouteThreads) {
        int run = fill[x];
        for (int v = 0; v < kRouteWaves; ++v) {
          const int c = wcnt[v * p.E + x];
          wcnt[v * p.E + x] = run;
          run += c;
        }
        fill[x] = run;
      }
      __syncthreads();
      if (key >= 0) place_pair(p, cnt, ubase, i, key, w, wcnt[wave * p.E + key] + rank);
      __syncthreads();
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kCached; ++j) scatter_pair(p, cnt, fill, ubase, tid + j * kRouteThreads, my_e[j], my_w[j]);
  for (int i = tid + kCached * kRouteThreads; i < P; i += kRouteThreads) {
    const int e = p.ids[i];
    if (e >= 0 && e < p.E) scatter_pair(p, cnt, fill, ubase, i, e, load_act(p.weights, p.w_dtype, i));
  }
}

// Multi-workgroup grouping for large batches (the single-workgroup route_block
// serializes on its LDS counters): per-chunk histograms, one scan over
// (expert, chunk), then a scatter.  hist is [E + 1][nchunk] (the last row
// counts invalid ids); the scan turns it into each chunk's insert positions.
// Pairs of one expert land in an order that can vary from call to call; every
// consumer of the grouping computes each pair independently of the others in
// its expert, so results do not depend on it.
constexpr int kHistInts = 16384;  // (E + 1) * nchunk bound: the scan holds the histograms in LDS

__global__ void __launch_bounds__(kRouteThreads) group_count_kernel(MoeParams p, int* hist, int chunk) {
  __shared__ int cnt[kMaxExperts + 1];
  const int tid = threadIdx.x, E = p.E, P = p.T * p.K;
  for (int e = tid; e <= E; e += kRouteThreads) cnt[e] = 0;
  __syncthreads();
  const int i0 = blockIdx.x * chunk, i1 = min(P, i0 + chunk);
  for (int i = i0 + tid; i < i1; i += kRouteThreads) {
    const int e = p.ids[i];
    if (e >= 0 && e < E)
      atomicAdd(&cnt[e], 1);
    else if (e >= E)
      atomicAdd(&cnt[E], 1);
  }
  __syncthreads();
  for (int e = tid; e <= E; e += kRouteThreads) hist[e * gridDim.x + blockIdx.x] = cnt[e];
}

__global__ void __launch_bounds__(kRouteThreads) group_scan_kernel(MoeParams p, int* hist, int nchunk) {
  __shared__ int h[kHistInts];
  __shared__ int scan_c[kRouteThreads];
  __shared__ int scan_a[kRouteThreads];
  const int tid = threadIdx.x, E = p.E, n = (E + 1) * nchunk, E1 = E + 1;
  // Chunk-major in LDS (h[k * E1 + e]): the threads of one expert range then
  // read consecutive words (expert-major, a stride of nchunk words put a
  // wave's reads on one bank).
  for (int i = tid; i < n; i += kRouteThreads) h[(i % nchunk) * E1 + i / nchunk] = hist[i];
  __syncthreads();
  const int per = (E + kRouteThreads - 1) / kRouteThreads;
  const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
  int sc = 0, sa = 0;
  for (int e = e0; e < e1; ++e) {
    int c = 0;
    for (int k = 0; k < nchunk; ++k) c += h[k * E1 + e];
    sc += c;
    sa += c > 0;
  }
  scan_c[tid] = sc;
  scan_a[tid] = sa;
  __syncthreads();
  for (int off = 1; off < kRouteThreads; off <<= 1) {
    const int vc = tid >= off ? scan_c[tid - off] : 0;
    const int va = tid >= off ? scan_a[tid - off] : 0;
    __syncthreads();
    scan_c[tid] += vc;
    scan_a[tid] += va;
    __syncthreads();
  }
  int start = scan_c[tid] - sc;
  int act = scan_a[tid] - sa;
  for (int e = e0; e < e1; ++e) {
    const int s0 = start;
    for (int k = 0; k < nchunk; ++k) {  // chunk insert positions, in chunk order
      const int c = h[k * E1 + e];
      h[k * E1 + e] = start;
      start += c;
    }
    if (start > s0) {
      p.act_expert[act] = e;
      p.act_start[act] = s0;
      p.act_count[act] = start - s0;
      ++act;
    }
  }
  __syncthreads();
  for (int i = tid; i < E * nchunk; i += kRouteThreads) hist[i] = h[(i % nchunk) * E1 + i / nchunk];
  if (tid == kRouteThreads - 1) {
    int bad = 0;
    for (int k = 0; k < nchunk; ++k) bad += h[E * nchunk + k];
    p.meta[0] = scan_a[kRouteThreads - 1];
    p.meta[1] = bad;
    p.meta[3] = scan_c[kRouteThreads - 1];  // routed pairs
  }
}

__global__ void __launch_bounds__(kRouteThreads) group_scatter_kernel(MoeParams p, const int* hist, int chunk) {
  __shared__ int fill[kMaxExperts];
  const int tid = threadIdx.x, E = p.E, P = p.T * p.K;
  for (int e = tid; e < E; e += kRouteThreads) fill[e] = hist[e * gridDim.x + blockIdx.x];
  __syncthreads();
  const int i0 = blockIdx.x * chunk, i1 = min(P, i0 + chunk);
  for (int i = i0 + tid; i < i1; i += kRouteThreads) {
    const int e = p.ids[i];
    if (e >= 0 && e < E) {
      const int pos = atomicAdd(&fill[e], 1);
      p.pair_tok[pos] = i / p.K;
      p.pair_slot[pos] = i - (i / p.K) * p.K;
      p.pair_w[pos] = load_act(p.weights, p.w_dtype, i);
    }
  }
}

__global__ void __launch_bounds__(kRouteThreads) prep_kernel(MoeParams p) {
  if (blockIdx.x == 0) {
    route_block(p);
    return;
  }
  const int64_t nblk = gridDim.x - 1;
  const int64_t t0 = (blockIdx.x - 1) * static_cast<int64_t>(kRouteThreads) + threadIdx.x;
  const int64_t stride = nblk * kRouteThreads;
  if (p.xh) {
    // One workgroup per token, 8 elements per thread and step: the row maximum
    // picks the exponent that brings it into [2^14, 2^15), then the row is
    // stored as fp16 * 2^exponent (the streaming path requires d % 8 == 0 and
    // a 16-byte aligned x).
    __shared__ float wmax[kRouteThreads / kWave];
    for (int64_t t = blockIdx.x - 1; t < p.T; t += nblk) {
      const int64_t row = t * p.d;
      float mx = 0.f;
      for (int i = threadIdx.x * 8; i < p.d; i += kRouteThreads * 8) {
        float v[8];
        load_act8(p.x, p.x_dtype, row + i, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
      }
      mx = op_over(mx, 1, kWave, OpMax{});
      if (threadIdx.x % kWave == 0) wmax[threadIdx.x / kWave] = mx;
      __syncthreads();
#pragma unroll
      for (int w = 0; w < kRouteThreads / kWave; ++w) mx = fmaxf(mx, wmax[w]);
      __syncthreads();  // wmax is reused by the next token
      const int ex = pow2_row_exponent(mx);
      for (int i = threadIdx.x * 8; i < p.d; i += kRouteThreads * 8) {
        float v[8];
        load_act8(p.x, p.x_dtype, row + i, v);
        typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
        half8_t h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = static_cast<_Float16>(ldexpf(v[j], ex));
        *reinterpret_cast<half8_t*>(p.xh + row + i) = h;
      }
      if (threadIdx.x == 0) p.xexp[t] = ex;
    }
    // The streaming path clears nothing (its kernels write every output); the
    // row-layout MFMA phases accumulate like the fp32 ones.
    if (!p.clear) return;
  }
  // Accumulators gu and dl are contiguous: zero_floats covers both.
  float4* acc4 = reinterpret_cast<float4*>(p.gu);
  const int64_t n4 = p.zero_floats / 4;
  for (int64_t i = t0; i < n4; i += stride) acc4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (p.out_mode == LATENT_OUT_REDUCED) {
    if (!p.zero_out) return;
    float4* o4 = reinterpret_cast<float4*>(p.out);
    const int64_t no = static_cast<int64_t>(p.T) * p.d / 4;
    for (int64_t i = t0; i < no; i += stride) o4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    // Per-slot output: only dropped slots are never written by phase D.
    const int64_t rows = static_cast<int64_t>(p.T) * p.K;
    const int64_t d4 = p.d / 4;
    for (int64_t i = t0; i < rows * d4; i += stride) {
      const int64_t r = i / d4;
      const int e = p.ids[r];
      if (e < 0 || e >= p.E) reinterpret_cast<float4*>(p.out)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMV building blocks
// ---------------------------------------------------------------------------
// acc[t][j] += sum over this lane's rows of vin[t][row] * scale(row, g) * level(code(row, g*32+j))
// Rows: row_begin, row_begin + step, ... < row_end.  vin[t][row] = vin[t*vstride + row - vbase].
// kInt8Rows: rows per pass of a factor with INT8 groups, their loads in
// flight together; 0: one row at a time through decode_group (phase BC, which
// the prefetching form pushes to 256 VGPRs and one wave per SIMD).
template <int MB, bool kInt8, int kInt8Rows = 2>
__device__ __forceinline__ void accumulate_rows(const Factor& f, int64_t e, int row_begin, int row_end, int step, int g,
                                                const float* lut, const float* vin, int vstride, int vbase, int m,
                                                float (&acc)[MB][kGroup]) {
  if (kInt8 && kInt8Rows == 0) {
    for (int row = row_begin; row < row_end; row += step) {
      float v[kGroup];
      decode_group<true>(f, e, row, g, lut, v);
      const float s = group_scale(f, e, row, g);
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        if (t < m) {
          const float xs = vin[t * vstride + row - vbase] * s;
#pragma unroll
          for (int j = 0; j < kGroup; ++j) acc[t][j] = fmaf(xs, v[j], acc[t][j]);
        }
      }
    }
  } else if (kInt8 && f.ext.bitmap != nullptr) {
    // U rows per pass, every load of a row independent of the others: the
    // codes, the scale, the group's bitmap word and its word offset (the
    // side-buffer index of the word's first INT8 group), then, for the lanes
    // whose group is INT8, its 32 bytes.  (The chain bitmap -> offset ->
    // data paid three dependent round trips per row.)
    constexpr int U = kInt8Rows > 0 ? kInt8Rows : 1;
    const int words = f.words(), wsel = g >> 5;
    const uint32_t bit = 1u << (g & 31);
    const int64_t cstride = f.code_stride(), sstride = f.scale_stride(), erow0 = e * f.rows;
    for (int row = row_begin; row < row_end; row += U * step) {
      uint4 c[U], q[U][2];
      float s[U];
      uint32_t wd[U];
      int64_t wo[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = min(row + u * step, row_end - 1);  // past the end: row_end - 1 again, never used
        const int64_t er = erow0 + r;
        c[u] = *reinterpret_cast<const uint4*>(f.codes + er * cstride + static_cast<int64_t>(g) * kGroupBytes);
        s[u] = half_bits_to_float(f.scales[er * sstride + g]);
        wd[u] = f.ext.bitmap[er * words + wsel];
        wo[u] = words == 1 ? f.ext.row_offset[er]
                           : (f.ext.word_offset ? f.ext.word_offset[er * words + wsel] : int64_t{-1});
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        q[u][0] = q[u][1] = make_uint4(0u, 0u, 0u, 0u);
        if (wd[u] & bit) {
          int64_t idx = wo[u];
          if (idx < 0) {  // no word offsets built: count the row's earlier words
            const int r = min(row + u * step, row_end - 1);
            const uint32_t* bm = f.ext.bitmap + (erow0 + r) * words;
            idx = f.ext.row_offset[erow0 + r];
            for (int w = 0; w < wsel; ++w) idx += popc(bm[w]);
          }
          idx += popc(wd[u] & (bit - 1u));
          const uint4* qp = reinterpret_cast<const uint4*>(f.ext.data + idx * kGroup);
          q[u][0] = qp[0];
          q[u][1] = qp[1];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = row + u * step;
        if (r >= row_end) break;
        float v[kGroup];
        if (wd[u] & bit) {
          const uint32_t qw[8] = {q[u][0].x, q[u][0].y, q[u][0].z, q[u][0].w,
                                  q[u][1].x, q[u][1].y, q[u][1].z, q[u][1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[i * 4 + b] = static_cast<float>(static_cast<int8_t>((qw[i] >> (8 * b)) & 0xFF));
        } else {
          const uint32_t cw[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int n = 0; n < 8; ++n) v[i * 8 + n] = lut[(cw[i] >> (4 * n)) & 15u];
        }
#pragma unroll
        for (int t = 0; t < MB; ++t) {
          if (t < m) {
            const float xs = vin[t * vstride + r - vbase] * s[u];
#pragma unroll
            for (int j = 0; j < kGroup; ++j) acc[t][j] = fmaf(xs, v[j], acc[t][j]);
          }
        }
      }
    }
  } else {
    constexpr int U = MB == 1 ? 4 : 2;
    const int64_t cstride = f.code_stride();
    const int64_t sstride = f.scale_stride();
    const uint8_t* cbase = f.codes + e * f.rows * cstride + static_cast<int64_t>(g) * kGroupBytes;
    const uint16_t* sbase = f.scales + e * f.rows * sstride + g;
    int row = row_begin;
    for (; row + (U - 1) * step < row_end; row += U * step) {
      uint4 c[U];
      float s[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        c[u] = *reinterpret_cast<const uint4*>(cbase + static_cast<int64_t>(row + u * step) * cstride);
        s[u] = half_bits_to_float(sbase[static_cast<int64_t>(row + u * step) * sstride]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float v[kGroup];
        const uint32_t cw[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int n = 0; n < 8; ++n) v[i * 8 + n] = lut[(cw[i] >> (4 * n)) & 15u];
        }
#pragma unroll
        for (int t = 0; t < MB; ++t) {
          if (t < m) {
            const float xs = vin[t * vstride + row + u * step - vbase] * s[u];
#pragma unroll
            for (int j = 0; j < kGroup; ++j) acc[t][j] = fmaf(xs, v[j], acc[t][j]);
          }
        }
      }
    }
    for (; row < row_end; row += step) {
      const uint4 c = *reinterpret_cast<const uint4*>(cbase + static_cast<int64_t>(row) * cstride);
      const float s = half_bits_to_float(sbase[static_cast<int64_t>(row) * sstride]);
      float v[kGroup];
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int n = 0; n < 8; ++n) v[i * 8 + n] = lut[(cw[i] >> (4 * n)) & 15u];
      }
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        if (t < m) {
          const float xs = vin[t * vstride + row - vbase] * s;
#pragma unroll
          for (int j = 0; j < kGroup; ++j) acc[t][j] = fmaf(xs, v[j], acc[t][j]);
        }
      }
    }
  }
}

// Sum acc over the lanes of a wave that share group g (lanes differing in the
// bits at and above log2(lpr)), then the first lpr lanes store the wave's
// partial to red[wave][t][g*32 + j] (red row length ncols).
template <int MB>
__device__ __forceinline__ void wave_reduce_store(float (&acc)[MB][kGroup], int lpr, int lane, int wave, int ngroups,
                                                  int m, float* red, int ncols) {
#pragma unroll
  for (int t = 0; t < MB; ++t) {
    if (t < m) {
#pragma unroll
      for (int j = 0; j < kGroup; ++j) acc[t][j] = op_over(acc[t][j], lpr, kWave, OpAdd{});
    }
  }
  if (lane < lpr && lane < ngroups) {
#pragma unroll
    for (int t = 0; t < MB; ++t) {
      if (t < m) {
        float* dst = red + (wave * MB + t) * ncols + lane * kGroup;
#pragma unroll
        for (int j = 0; j < kGroup; ++j) dst[j] = acc[t][j];
      }
    }
  }
}

template <int MB>
__device__ __forceinline__ void zero_acc(float (&acc)[MB][kGroup]) {
#pragma unroll
  for (int t = 0; t < MB; ++t)
#pragma unroll
    for (int j = 0; j < kGroup; ++j) acc[t][j] = 0.f;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// phase A: x . A_g and x . A_u over a slice of rows of A
// ---------------------------------------------------------------------------
template <int MB, bool kInt8>
__global__ void __launch_bounds__(kThreads) phase_a_kernel(MoeParams p) {
  extern __shared__ float smem[];
  float* lut = smem;                 // 16
  float* xin = smem + 16;            // [MB][ra]
  float* red = xin + MB * p.ra;      // [kWaves][MB][R]
  int a, item;
  if (!map_item(blockIdx.x, p.n_a, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  if (tid < 16) lut[tid] = kLevelsMoe[tid];
  const int kind = item & 1;  // 0 gate, 1 up
  const int chunk = item >> 1;
  const Factor f = kind == 0 ? p.fac[F_GATE_A] : p.fac[F_UP_A];
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int ng = (rank_of(p, e, kind) + kGroup - 1) / kGroup;
  if (ng == 0) return;
  const int lpr = next_pow2(ng), rpw = kWave / lpr;
  const int g = lane & (lpr - 1), ro = lane >> ilog2(lpr);
  const int r0 = chunk * p.ra, r1 = min(p.d, r0 + p.ra), nrows = r1 - r0;
  const int ncols = ng * kGroup;
  for (int tb = 0; tb < mtot; tb += MB) {
    const int m = min(MB, mtot - tb);
    for (int i = tid; i < m * nrows; i += kThreads) {
      const int t = i / nrows, rr = i - t * nrows;
      const int tok = p.pair_tok[s0 + tb + t];
      xin[t * p.ra + rr] = load_act(p.x, p.x_dtype, static_cast<int64_t>(tok) * p.d + r0 + rr);
    }
    __syncthreads();
    float acc[MB][kGroup];
    zero_acc(acc);
    if (g < ng)
      accumulate_rows<MB, kInt8>(f, e, r0 + wave * rpw + ro, r1, kWaves * rpw, g, lut, xin, p.ra, r0, m, acc);
    wave_reduce_store<MB>(acc, lpr, lane, wave, ng, m, red, p.R);
    __syncthreads();
    for (int i = tid; i < m * ncols; i += kThreads) {
      const int t = i / ncols, col = i - t * ncols;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += red[(w * MB + t) * p.R + col];
      atomic_add_f32(p.gu + static_cast<int64_t>(s0 + tb + t) * (2 * p.R) + kind * p.R + col, v);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// phase BC: g,u over a slice of ff columns, h = SiLU(g)*u, then h . A_d[slice]
// ---------------------------------------------------------------------------
template <int MB, bool kInt8>
__global__ void __launch_bounds__(kThreads) phase_bc_kernel(MoeParams p) {
  extern __shared__ float smem[];
  float* lut = smem;                      // 16
  float* lat = smem + 16;                 // [MB][2R]
  float* hs = lat + MB * 2 * p.R;         // [2][MB][cb]
  float* red = hs + 2 * MB * p.cb;        // [kWaves][MB][max(cb, R)]
  const int redw = max(p.cb, p.R);
  int a, item;
  if (!map_item(blockIdx.x, p.n_bc, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  if (tid < 16) lut[tid] = kLevelsMoe[tid];
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int c0 = item * p.cb, ncol = min(p.cb, p.ff - c0), gpc = ncol / kGroup;
  const int lpr_b = next_pow2(p.cb / kGroup), rpw_b = kWave / lpr_b;
  const int gb = lane & (lpr_b - 1), rob = lane >> ilog2(lpr_b);
  const int rank_d = rank_of(p, e, 2);
  const int ngd = (rank_d + kGroup - 1) / kGroup;
  const int lpr_d = next_pow2(max(ngd, 1)), rpw_d = kWave / lpr_d;
  const int gd = lane & (lpr_d - 1), rod = lane >> ilog2(lpr_d);
  for (int tb = 0; tb < mtot; tb += MB) {
    const int m = min(MB, mtot - tb);
    for (int i = tid; i < m * 2 * p.R; i += kThreads) {
      const int t = i / (2 * p.R), col = i - t * 2 * p.R;
      lat[t * 2 * p.R + col] = p.gu[static_cast<int64_t>(s0 + tb + t) * 2 * p.R + col];
    }
    __syncthreads();
    for (int kind = 0; kind < 2; ++kind) {
      const Factor f = kind == 0 ? p.fac[F_GATE_B] : p.fac[F_UP_B];
      const int rk = rank_of(p, e, kind);
      float acc[MB][kGroup];
      zero_acc(acc);
      if (gb < gpc)
        accumulate_rows<MB, kInt8, 0>(f, e, wave * rpw_b + rob, rk, kWaves * rpw_b, c0 / kGroup + gb, lut,
                                   lat + kind * p.R, 2 * p.R, 0, m, acc);
      wave_reduce_store<MB>(acc, lpr_b, lane, wave, gpc, m, red, redw);
      __syncthreads();
      for (int i = tid; i < m * ncol; i += kThreads) {
        const int t = i / ncol, col = i - t * ncol;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += red[(w * MB + t) * redw + col];
        hs[(kind * MB + t) * p.cb + col] = v;
      }
      __syncthreads();
    }
    // h = SiLU(g) * u  (x router weight when weighting before down), in hs[0]
    for (int i = tid; i < m * ncol; i += kThreads) {
      const int t = i / ncol, col = i - t * ncol;
      float h = silu_f32(hs[t * p.cb + col]) * hs[(MB + t) * p.cb + col];
      if (p.wbd) h *= p.pair_w[s0 + tb + t];
      hs[t * p.cb + col] = h;
    }
    __syncthreads();
    if (ngd > 0) {
      float acc[MB][kGroup];
      zero_acc(acc);
      if (gd < ngd)
        accumulate_rows<MB, kInt8, 0>(p.fac[F_DOWN_A], e, c0 + wave * rpw_d + rod, c0 + ncol, kWaves * rpw_d, gd, lut, hs,
                                   p.cb, c0, m, acc);
      wave_reduce_store<MB>(acc, lpr_d, lane, wave, ngd, m, red, redw);
      __syncthreads();
      const int ncols_d = ngd * kGroup;
      for (int i = tid; i < m * ncols_d; i += kThreads) {
        const int t = i / ncols_d, col = i - t * ncols_d;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += red[(w * MB + t) * redw + col];
        atomic_add_f32(p.dl + static_cast<int64_t>(s0 + tb + t) * p.R + col, v);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// phase D: y = d_lat . B_d over a slice of d columns, then the combine
// ---------------------------------------------------------------------------
template <int MB, bool kInt8>
__global__ void __launch_bounds__(kThreads) phase_d_kernel(MoeParams p) {
  extern __shared__ float smem[];
  float* lut = smem;             // 16
  float* lat = smem + 16;        // [MB][R]
  float* red = lat + MB * p.R;   // [kWaves][MB][cd]
  int a, item;
  if (!map_item(blockIdx.x, p.n_d, p.meta[0], a, item)) return;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  if (tid < 16) lut[tid] = kLevelsMoe[tid];
  const int e = p.act_expert[a], s0 = p.act_start[a], mtot = p.act_count[a];
  const int c0 = item * p.cd, ncol = min(p.cd, p.d - c0), gpc = ncol / kGroup;
  const int lpr = next_pow2(p.cd / kGroup), rpw = kWave / lpr;
  const int g = lane & (lpr - 1), ro = lane >> ilog2(lpr);
  const int rk = rank_of(p, e, 2);
  for (int tb = 0; tb < mtot; tb += MB) {
    const int m = min(MB, mtot - tb);
    for (int i = tid; i < m * p.R; i += kThreads) {
      const int t = i / p.R, col = i - t * p.R;
      lat[t * p.R + col] = p.dl[static_cast<int64_t>(s0 + tb + t) * p.R + col];
    }
    __syncthreads();
    float acc[MB][kGroup];
    zero_acc(acc);
    if (g < gpc)
      accumulate_rows<MB, kInt8>(p.fac[F_DOWN_B], e, wave * rpw + ro, rk, kWaves * rpw, c0 / kGroup + g, lut, lat, p.R,
                                 0, m, acc);
    wave_reduce_store<MB>(acc, lpr, lane, wave, gpc, m, red, p.cd);
    __syncthreads();
    for (int i = tid; i < m * ncol; i += kThreads) {
      const int t = i / ncol, col = i - t * ncol;
      float y = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) y += red[(w * MB + t) * p.cd + col];
      const int pair = s0 + tb + t;
      const int tok = p.pair_tok[pair];
      if (p.out_mode == LATENT_OUT_REDUCED) {
        const float wgt = p.wbd ? 1.0f : p.pair_w[pair];
        atomic_add_f32(p.out + static_cast<int64_t>(tok) * p.d + c0 + col, wgt * y);
      } else {
        p.out[(static_cast<int64_t>(tok) * p.K + p.pair_slot[pair]) * p.d + c0 + col] = y;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Layout {
  size_t meta, act_expert, act_start, act_count, pair_tok, pair_slot, pair_w, hist, units, gu, dl, xh, xexp, total;
};

// Pairs per chunk of the multi-workgroup grouping: multiples of the block
// size, few enough chunks for the scan's LDS copy of the histograms.
int64_t group_chunk(int64_t P, int64_t E) {
  const int64_t max_chunks = std::max<int64_t>(1, kHistInts / (E + 1));
  int64_t chunk = kRouteThreads;
  while ((P + chunk - 1) / chunk > max_chunks) chunk += kRouteThreads;
  return chunk;
}
int64_t group_chunks(int64_t P, int64_t E) { const int64_t c = group_chunk(P, E); return (P + c - 1) / c; }

// Columns of the fp16 x rows the row-layout MFMA phases read (0: the call's
// shape never takes them).
int64_t xh_cols(const latent_moe_args& a) {
  return a.layout == LATENT_LAYOUT_ROWS && a.max_rank <= 512 ? a.n_embd : 0;
}

Layout layout_for(int64_t T, int64_t K, int64_t E, int64_t R, int64_t d) {
  Layout L{};
  const int64_t P = T * K;
  const int64_t amax = std::max<int64_t>(1, std::min(E, P));
  size_t off = 0;
  L.meta = off;       off = align_up(off + 64 * sizeof(int));
  L.act_expert = off; off = align_up(off + amax * sizeof(int));
  L.act_start = off;  off = align_up(off + amax * sizeof(int));
  L.act_count = off;  off = align_up(off + amax * sizeof(int));
  L.pair_tok = off;   off = align_up(off + P * sizeof(int));
  L.pair_slot = off;  off = align_up(off + P * sizeof(int));
  L.pair_w = off;     off = align_up(off + P * sizeof(float));
  L.hist = off;       off = align_up(off + group_chunks(P, E) * (E + 1) * sizeof(int));
  L.units = off;      off = align_up(off + (4 + stream::kMaxM) * stream::max_units(P, E) * sizeof(int));
  L.gu = off;         off += P * 2 * R * sizeof(float);  // gu and dl contiguous (one clear)
  L.dl = off;         off = align_up(off + P * R * sizeof(float));
  // x as fp16 rows x 2^xexp for the row-layout MFMA phases (d = 0: none).
  L.xh = off;         off = align_up(off + T * d * 2);
  L.xexp = off;       off = align_up(off + T * sizeof(int));
  L.total = off;
  return L;
}

int validate(const latent_moe_args& a) {
  if (a.n_tokens < 0 || a.n_embd <= 0 || a.n_ff <= 0 || a.n_expert <= 0 || a.n_expert_used <= 0 || a.max_rank <= 0)
    return LATENT_E_INVALID;
  if (a.n_embd % kGroup || a.n_ff % kGroup || a.max_rank % kGroup) return LATENT_E_INVALID;
  if (a.x_dtype < LATENT_F32 || a.x_dtype > LATENT_BF16) return LATENT_E_INVALID;
  if (a.weights_dtype != LATENT_F32 && a.weights_dtype != LATENT_F16) return LATENT_E_INVALID;
  if (a.out_mode != LATENT_OUT_REDUCED && a.out_mode != LATENT_OUT_PER_SLOT) return LATENT_E_INVALID;
  if (a.layout != LATENT_LAYOUT_ROWS && a.layout != LATENT_LAYOUT_TILES) return LATENT_E_INVALID;
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  const int64_t rows[6] = {a.n_embd, a.max_rank, a.n_embd, a.max_rank, a.n_ff, a.max_rank};
  const int64_t cols[6] = {a.max_rank, a.n_ff, a.max_rank, a.n_ff, a.max_rank, a.n_embd};
  for (int i = 0; i < 6; ++i) {
    const int st = check_factor(*fs[i]);
    if (st != LATENT_OK) return st;
    if (fs[i]->rows != rows[i] || fs[i]->cols != cols[i]) return LATENT_E_INVALID;
  }
  if (a.n_expert > kMaxExperts || a.max_rank > kMaxRank || a.n_expert_used > kMaxExpertUsed) return LATENT_E_UNSUPPORTED;
  const int64_t P = a.n_tokens * a.n_expert_used;
  if (a.n_tokens > (1 << 24) || P > (1 << 26) || a.n_embd > (1 << 20) || a.n_ff > (1 << 20)) return LATENT_E_UNSUPPORTED;
  if (a.layout == LATENT_LAYOUT_TILES && !stream::tiles_shape_ok(a)) return LATENT_E_UNSUPPORTED;
  return LATENT_OK;
}

int pick_pow2_chunk(int64_t per_expert_extent, int64_t experts, int64_t target_items, int lo, int hi) {
  int c = hi;
  while (c > lo && experts * ((per_expert_extent + c - 1) / c) < target_items) c /= 2;
  return c;
}

enum { kPathGeneral = 0, kPathFused = 1, kPathPrefill = 2, kPathStream = 3, kPathRows = 4 };

// The implementation for one call shape.  LATENT_MOE_PATH (general | fused |
// prefill | stream | rows) selects another path that supports the call, for
// comparisons; the default is the measured fastest supported path.  A layer
// in the tile layout has only the two MFMA paths (LATENT_E_UNSUPPORTED when
// neither takes the call).
int choose_path(const latent_moe_args& a, fused::Plan& pl) {
  if (a.layout == LATENT_LAYOUT_TILES) {
    const bool prefill_ok = prefill::supported(a), stream_ok = stream::supported(a);
    const char* env = std::getenv("LATENT_MOE_PATH");
    if (env && !std::strcmp(env, "stream") && stream_ok) return kPathStream;
    if (prefill_ok) return kPathPrefill;
    if (stream_ok) return kPathStream;
    return LATENT_E_UNSUPPORTED;
  }
  const bool fused_ok = fused::supported(a) && fused::make_plan(a, pl);
  const bool prefill_ok = prefill::supported(a);
  const bool stream_ok = stream::supported(a);
  const bool rows_ok = rows::supported(a);
  const char* env = std::getenv("LATENT_MOE_PATH");
  if (env && *env) {
    if (!std::strcmp(env, "rows") && rows_ok) return kPathRows;
    if (!std::strcmp(env, "stream") && stream_ok) return kPathStream;
    if (!std::strcmp(env, "fused") && fused_ok) return kPathFused;
    if (!std::strcmp(env, "prefill") && prefill_ok) return kPathPrefill;
    if (!std::strcmp(env, "general")) return kPathGeneral;
  }
  // Measured on MI355X at the DeepSeek-V3 shape (d 7168, ff 2048, 256
  // experts, top-8): below the prefill threshold the streaming MFMA path is
  // the fastest wherever it applies (batch 1: 49 vs 52 us for the
  // multi-kernel path; batch 8: 100 vs 144 us and batch 64: 270 vs 370 us
  // for the persistent kernel).  On the row layout:
  //   * with INT8 groups (ranks 64..512, 10 % INT8 groups): the row-layout
  //     MFMA phases from 16 routed pairs (batch 16 / 32 / 64 / 256: 382 /
  //     567 / 704 / 840 us against 400 / 577 / 830 us for the persistent
  //     fp32 kernel and 632 / 977 / 1,549 / 3,633 us for the multi-kernel
  //     path; batch 1: 160 against 134 us, so below 16 pairs the latter);
  //   * pure NF4 (rank 256): the persistent fp32 kernel where it applies
  //     (batch 16 / 32 / 64: 189 / 268 / 381 us against 246 / 362 / 495 us
  //     for the row-layout MFMA phases; batch 8 151 against 154 us).
  const bool int8 = a.gate_a.int8_bitmap || a.gate_b.int8_bitmap || a.up_a.int8_bitmap || a.up_b.int8_bitmap ||
                    a.down_a.int8_bitmap || a.down_b.int8_bitmap;
  const bool rows_pairs = rows_ok && a.n_tokens * a.n_expert_used >= 16;
  if (prefill_ok) return kPathPrefill;
  if (stream_ok) return kPathStream;
  if (int8 && rows_pairs) return kPathRows;
  if (fused_ok) return kPathFused;
  if (rows_pairs) return kPathRows;
  return kPathGeneral;
}

template <int MB, bool kInt8>
int launch_phases(const MoeParams& p, hipStream_t s) {
  const unsigned a_groups = static_cast<unsigned>((p.a_max + 7) / 8);
  const size_t lds_a = (16 + MB * p.ra + kWaves * MB * p.R) * sizeof(float);
  hipLaunchKernelGGL((phase_a_kernel<MB, kInt8>), dim3(8 * a_groups * p.n_a), dim3(kThreads), lds_a, s, p);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  const size_t lds_bc = (16 + MB * 2 * p.R + 2 * MB * p.cb + kWaves * MB * std::max(p.cb, p.R)) * sizeof(float);
  hipLaunchKernelGGL((phase_bc_kernel<MB, kInt8>), dim3(8 * a_groups * p.n_bc), dim3(kThreads), lds_bc, s, p);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  const size_t lds_d = (16 + MB * p.R + kWaves * MB * p.cd) * sizeof(float);
  hipLaunchKernelGGL((phase_d_kernel<MB, kInt8>), dim3(8 * a_groups * p.n_d), dim3(kThreads), lds_d, s, p);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  return LATENT_OK;
}

// Index of each bitmap word's first INT8 group: row_offset plus the set bits
// of the row's earlier words (one thread per expert row).
__global__ void __launch_bounds__(kThreads) int8_word_offset_kernel(const uint32_t* bitmap, const int32_t* row_offset,
                                                                   int32_t* out, int64_t rows_total, int words) {
  for (int64_t r = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; r < rows_total;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    int run = row_offset[r];
    for (int w = 0; w < words; ++w) {
      out[r * words + w] = run;
      run += popc(bitmap[r * words + w]);
    }
  }
}

// Workspace tail holding the per-word INT8 offsets of the factors whose rows
// span more than one bitmap word (factors of one word use row_offset).
size_t int8_word_offset_bytes(const latent_moe_args& a) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  size_t n = 0;
  for (const latent_factor* f : fs) {
    const int64_t words = (f->cols / kGroup + 31) / 32;
    if (f->int8_bitmap && words > 1) n += align_up(static_cast<size_t>(a.n_expert * f->rows * words) * sizeof(int32_t));
  }
  return n;
}

// Fill `word_offset` of every INT8 factor: the workspace tail for factors of
// more than one bitmap word (a kernel per factor), row_offset for the others.
int set_int8_word_offsets(const latent_moe_args& a, char* tail, Factor (&fac)[6], hipStream_t s) {
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  size_t off = 0;
  for (int i = 0; i < 6; ++i) {
    const latent_factor& f = *fs[i];
    if (!f.int8_bitmap) continue;
    const int64_t words = (f.cols / kGroup + 31) / 32;
    if (words == 1) {
      fac[i].ext.word_offset = f.int8_row_offset;
      continue;
    }
    int32_t* dst = reinterpret_cast<int32_t*>(tail + off);
    const int64_t rows_total = a.n_expert * f.rows;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(1024, (rows_total + kThreads - 1) / kThreads));
    hipLaunchKernelGGL(int8_word_offset_kernel, dim3(blocks), dim3(kThreads), 0, s, f.int8_bitmap, f.int8_row_offset,
                       dst, rows_total, static_cast<int>(words));
    fac[i].ext.word_offset = dst;
    off += align_up(static_cast<size_t>(rows_total * words) * sizeof(int32_t));
  }
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}

}  // namespace
}  // namespace latent

using namespace latent;

extern "C" int latent_version(void) { return 100; }

extern "C" const char* latent_status_string(int status) {
  switch (status) {
    case LATENT_OK: return "ok";
    case LATENT_E_INVALID: return "invalid argument";
    case LATENT_E_UNSUPPORTED: return "unsupported configuration";
    case LATENT_E_WORKSPACE: return "workspace missing or too small";
    case LATENT_E_HIP: return "HIP runtime error";
    case LATENT_E_TIMEOUT: return "a bounded wait between workgroups timed out (output undefined)";
    default: return "unknown status";
  }
}

// Workspace: [fused control block, zero between calls][scratch shared by both paths]
extern "C" int latent_moe_workspace_size(const latent_moe_args* args, size_t* bytes) {
  if (!args || !bytes) return LATENT_E_INVALID;
  const int st = validate(*args);
  if (st != LATENT_OK) return st;
  const Layout L = layout_for(args->n_tokens, args->n_expert_used, args->n_expert, args->max_rank, xh_cols(*args));
  size_t scratch = L.total;
  if (prefill::supported(*args)) scratch = std::max(scratch, L.gu + prefill::layout_for(*args).total);
  fused::Plan pl;
  if (args->layout == LATENT_LAYOUT_ROWS && fused::supported(*args) && fused::make_plan(*args, pl))
    scratch = std::max(scratch, pl.scratch_bytes);
  if (stream::supported(*args)) scratch = std::max(scratch, L.gu + stream::layout_for(*args).total);
  *bytes = fused::kReserved + align_up(scratch) + int8_word_offset_bytes(*args);
  return LATENT_OK;
}

namespace latent {
// The calling device's noalloc scratch array (noalloc.hip), set up on first use.
int noalloc_scratch(hipStream_t s, void** out);
namespace {
__global__ void clear_control_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}
}  // namespace
}  // namespace latent

// A set error word means a bounded wait expired: the chain that timed out
// finished on whatever data it had, and a producer's late counter update may
// have landed after its consumer reset that counter.  Once the stream has
// drained, every kernel of that call has ended, so re-zeroing the whole
// control block (counters, tickets and the error word) restores the state
// every call expects on entry.
extern "C" int latent_moe_check(void* workspace, size_t workspace_bytes, latent_stream_t stream) {
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!workspace) {
    if (workspace_bytes != 0) return LATENT_E_WORKSPACE;
    (void)hipGetLastError();
    const int st = noalloc_scratch(s, &workspace);
    if (st != LATENT_OK) return st;
  } else if (workspace_bytes < fused::kReserved) {
    return LATENT_E_WORKSPACE;
  }
  int* word = reinterpret_cast<int*>(static_cast<char*>(workspace) + fused::kErrorOffset);
  int h = 0;
  if (hipMemcpyAsync(&h, word, sizeof h, hipMemcpyDeviceToHost, s) != hipSuccess) return LATENT_E_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return LATENT_E_HIP;
  if (h == 0) return LATENT_OK;
  const size_t n16 = fused::kReserved / 16;
  hipLaunchKernelGGL(clear_control_kernel, dim3(static_cast<unsigned>((n16 + 255) / 256)), dim3(256), 0, s,
                     static_cast<uint4*>(workspace), n16);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) return LATENT_E_HIP;
  return LATENT_E_TIMEOUT;
}

extern "C" int latent_moe_path(const latent_moe_args* args) {
  if (!args) return LATENT_E_INVALID;
  const int st = validate(*args);
  if (st != LATENT_OK) return st;
  fused::Plan pl;
  return choose_path(*args, pl);
}

extern "C" int latent_stream_launch(const latent_moe_args* args) {
  if (!args) return LATENT_E_INVALID;
  const int st = validate(*args);
  if (st != LATENT_OK) return st;
  fused::Plan pl;
  if (choose_path(*args, pl) != kPathStream) return LATENT_E_UNSUPPORTED;
  return stream::lite_applies(*args) ? 2 : 0;
}

extern "C" int latent_moe_ffn_forward(const latent_moe_args* args, latent_stream_t stream) {
  if (!args) return LATENT_E_INVALID;
  const latent_moe_args& a = *args;
  int st = validate(a);
  if (st != LATENT_OK) return st;
  if (a.n_tokens == 0) return LATENT_OK;
  if (!a.x || !a.ids || !a.weights || !a.out) return LATENT_E_INVALID;
  if ((reinterpret_cast<uintptr_t>(a.out) & 15u) != 0) return LATENT_E_INVALID;
  size_t need = 0;
  latent_moe_workspace_size(&a, &need);
  if (!a.workspace || a.workspace_bytes < need) return LATENT_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(a.workspace) & (kAlign - 1)) != 0) return LATENT_E_WORKSPACE;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();  // clear a stale error so the checks below see only ours
  fused::Plan pl;
  const int path = choose_path(a, pl);
  if (path < 0) return path;
  MoeParams p{};
  const latent_factor* fs[6] = {&a.gate_a, &a.gate_b, &a.up_a, &a.up_b, &a.down_a, &a.down_b};
  bool any_int8 = false;
  for (int i = 0; i < 6; ++i) {
    p.fac[i] = make_factor(*fs[i]);
    any_int8 = any_int8 || fs[i]->int8_bitmap != nullptr;
  }
  if (any_int8) {
    // The tail of the workspace (after the largest path's scratch).
    size_t total = 0;
    latent_moe_workspace_size(&a, &total);
    char* tail = static_cast<char*>(a.workspace) + total - int8_word_offset_bytes(a);
    st = set_int8_word_offsets(a, tail, p.fac, s);
    if (st != LATENT_OK) return st;
  }
  if (path == kPathFused) return fused::forward(a, s, static_cast<char*>(a.workspace), pl, p.fac);
  const Layout L = layout_for(a.n_tokens, a.n_expert_used, a.n_expert, a.max_rank, xh_cols(a));
  char* ws = static_cast<char*>(a.workspace) + fused::kReserved;
  p.x = a.x;
  p.ids = a.ids;
  p.weights = a.weights;
  p.ranks = a.ranks;
  p.out = static_cast<float*>(a.out);
  p.meta = reinterpret_cast<int*>(ws + L.meta);
  p.act_expert = reinterpret_cast<int*>(ws + L.act_expert);
  p.act_start = reinterpret_cast<int*>(ws + L.act_start);
  p.act_count = reinterpret_cast<int*>(ws + L.act_count);
  p.pair_tok = reinterpret_cast<int*>(ws + L.pair_tok);
  p.pair_slot = reinterpret_cast<int*>(ws + L.pair_slot);
  p.pair_w = reinterpret_cast<float*>(ws + L.pair_w);
  p.gu = reinterpret_cast<float*>(ws + L.gu);
  p.dl = reinterpret_cast<float*>(ws + L.dl);
  p.x_dtype = a.x_dtype;
  p.w_dtype = a.weights_dtype;
  p.T = static_cast<int>(a.n_tokens);
  p.d = static_cast<int>(a.n_embd);
  p.ff = static_cast<int>(a.n_ff);
  p.E = static_cast<int>(a.n_expert);
  p.K = static_cast<int>(a.n_expert_used);
  p.R = static_cast<int>(a.max_rank);
  p.wbd = a.weight_before_down ? 1 : 0;
  p.out_mode = a.out_mode;
  const int64_t P = a.n_tokens * a.n_expert_used;
  p.a_max = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(a.n_expert, P)));
  const bool use_prefill = path == kPathPrefill;
  const bool use_stream = path == kPathStream;
  if (use_stream && stream::lite_applies(a)) {
    static_assert(stream::kLiteCtrlOffset + stream::kLiteCtrlBytes <= fused::kReserved, "control block");
    return stream::lite_forward(a, static_cast<char*>(a.workspace), ws + L.gu,
                                reinterpret_cast<int*>(static_cast<char*>(a.workspace) + fused::kErrorOffset), s);
  }
  if (use_stream) {
    const int64_t mu = stream::max_units(P, a.n_expert);
    p.unit_info = reinterpret_cast<int4*>(ws + L.units);
    p.unit_tok = reinterpret_cast<int*>(p.unit_info + mu);
    const stream::Layout SL = stream::layout_for(a);
    p.pos_of = reinterpret_cast<int*>(ws + L.gu + SL.pos_of);
    p.xh = reinterpret_cast<_Float16*>(ws + L.gu + SL.xh);
    p.xexp = reinterpret_cast<int*>(ws + L.gu + SL.xexp);
  }
  const bool use_rows = path == kPathRows;
  if (use_rows) {
    p.xh = reinterpret_cast<_Float16*>(ws + L.xh);
    p.xexp = reinterpret_cast<int*>(ws + L.xexp);
  }
  // The MFMA paths write their intermediates whole, and every output row
  // (per-token combine); the row-layout MFMA phases accumulate like the fp32 ones.
  p.zero_floats = use_prefill || use_stream ? 0 : P * 3 * a.max_rank;
  p.zero_out = use_prefill || use_stream ? 0 : 1;
  p.clear = use_stream ? 0 : 1;

  // Work split: enough items to fill 256 CUs even when few experts are routed.
  const int MB = a.n_tokens == 1 ? 1 : 4;
  const int ra_hi = std::max(128, std::min(2048, static_cast<int>((48 * 1024 / 4 - 16 - 4 * MB * p.R) / MB) & ~127));
  p.ra = pick_pow2_chunk(p.d, 2LL * p.a_max, 2048, 128, ra_hi);
  p.n_a = 2 * ((p.d + p.ra - 1) / p.ra);
  p.cb = pick_pow2_chunk(p.ff, p.a_max, 1024, 128, 256);
  p.n_bc = (p.ff + p.cb - 1) / p.cb;
  p.cd = pick_pow2_chunk(p.d, p.a_max, 2048, 128, 512);
  p.n_d = (p.d + p.cd - 1) / p.cd;

  const int64_t zero_work =
      use_stream ? 0
                 : p.zero_floats / 4 + (a.out_mode == LATENT_OUT_REDUCED ? p.zero_out * P / a.n_expert_used * a.n_embd / 4
                                                                         : P * a.n_embd / 4);
  // The streaming path and the row-layout MFMA phases also convert x, one
  // workgroup per token.
  const int64_t conv_blocks = use_stream || use_rows ? a.n_tokens : 1;
  const int zero_blocks = static_cast<int>(
      std::min<int64_t>(512, std::max<int64_t>(conv_blocks, zero_work / (kRouteThreads * 8))));
  if (use_prefill) {
    // Large batch: the multi-workgroup grouping; nothing to clear.
    int* hist = reinterpret_cast<int*>(ws + L.hist);
    const int chunk = static_cast<int>(group_chunk(P, a.n_expert));
    const int nchunk = static_cast<int>(group_chunks(P, a.n_expert));
    hipLaunchKernelGGL(group_count_kernel, dim3(nchunk), dim3(kRouteThreads), 0, s, p, hist, chunk);
    hipLaunchKernelGGL(group_scan_kernel, dim3(1), dim3(kRouteThreads), 0, s, p, hist, nchunk);
    hipLaunchKernelGGL(group_scatter_kernel, dim3(nchunk), dim3(kRouteThreads), 0, s, p, hist, chunk);
  } else {
    hipLaunchKernelGGL(prep_kernel, dim3(1 + zero_blocks), dim3(kRouteThreads), 0, s, p);
  }
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  if (use_prefill) {
    const prefill::Grouping g{p.meta, p.act_expert, p.act_start, p.act_count, p.pair_tok, p.pair_slot, p.pair_w};
    return prefill::forward(a, p.fac, g, ws + L.gu, s);
  }
  if (use_stream) {
    const stream::Grouping g{p.meta,      p.unit_info, p.unit_tok, p.pair_tok, p.pair_slot, p.pair_w,
                             reinterpret_cast<int*>(static_cast<char*>(a.workspace) + fused::kErrorOffset)};
    return stream::forward(a, g, ws + L.gu, s);
  }
  if (use_rows) {
    rows::Params rp{};
    for (int i = 0; i < 6; ++i) rp.fac[i] = p.fac[i];
    rp.ranks = p.ranks;
    rp.meta = p.meta;
    rp.act_expert = p.act_expert;
    rp.act_start = p.act_start;
    rp.act_count = p.act_count;
    rp.pair_tok = p.pair_tok;
    rp.pair_slot = p.pair_slot;
    rp.pair_w = p.pair_w;
    rp.xh = p.xh;
    rp.xexp = p.xexp;
    rp.gu = p.gu;
    rp.dl = p.dl;
    rp.out = p.out;
    rp.T = p.T;
    rp.d = p.d;
    rp.ff = p.ff;
    rp.K = p.K;
    rp.R = p.R;
    rp.wbd = p.wbd;
    rp.out_mode = p.out_mode;
    rp.a_max = p.a_max;
    rows::plan(rp);
    return rows::launch(rp, any_int8, s);
  }
  if (MB == 1)
    st = any_int8 ? launch_phases<1, true>(p, s) : launch_phases<1, false>(p, s);
  else
    st = any_int8 ? launch_phases<4, true>(p, s) : launch_phases<4, false>(p, s);
  return st;
}
