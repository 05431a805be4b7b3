// Router front end of a LATENT MoE layer on gfx950: logits, softmax, top-k,
// renormalisation and the optional drop rules, producing the (ids, weights)
// operands of latent_moe_ffn_forward on the device.
//
// The reference leaves routing to the graph builder (build_moe_ffn_latent,
// README.md:111-113, patch 004 empty) and restates the adaptive drop on the
// host (loader/adaptive_topk.py:29-90).  Here it is two kernels, so a whole
// decode layer (route + expert FFN) is stream-ordered device work that a HIP
// graph can hold:
//
//   logits_kernel  partial logits of x . W_r over one 64-row slice of d for a
//                  64-expert x 32-token tile; slices go to their own slot of the
//                  workspace (no atomics, fixed summation order).
//   topk_kernel    one wave per token: sum the slices in slice order (or read
//                  caller logits), top-k by repeated wave arg-max (ties -> the
//                  lower expert id), weights exp(l - max) renormalised over the
//                  kept k, then the drop rule.
//
// Work per call: the router matrix is read once per 32-token block (d*E*4 B in
// fp32 = 7.3 MB at d=7168, E=256) and is HBM-bound; top-k is latency-bound.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace latent {
namespace route {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 64;      // rows of d per logits workgroup
constexpr int kCols = 64;      // experts per logits workgroup
constexpr int kTok = 32;       // tokens per logits workgroup
constexpr int kMaxE = 1024;    // experts: 16 per lane in topk_kernel
constexpr int kPerLane = kMaxE / kWave;
constexpr int kMaxK = kWave;  // slot s lives in lane s
constexpr int kSliceBatch = 128;  // logit slices a topk thread loads at once

struct Params {
  const void* x;
  int x_dtype;
  const void* router;
  int router_dtype;
  const float* logits_in;
  float* logits_out;
  int32_t* ids;
  float* weights;
  float* partial;  // [nslice][T][E]
  int T, d, E, K, nslice, drop_rule;
  float drop_param;
  bool vec_router, vec_x;  // 4-element vector loads allowed (alignment, row length)
};

// Four consecutive elements [i, i+4) of a row of `n` elements (f32 / f16 /
// bf16), zero beyond n.  `vec`: the row start and i are 4-element aligned and
// the base is 16-byte (f32) or 8-byte (16-bit types) aligned.
__device__ __forceinline__ float4 load4(const void* base, int dtype, int64_t row_off, int i, int n, bool vec) {
  float v[4];
  if (vec && i + 4 <= n) {
    if (dtype == LATENT_F32) return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + row_off + i);
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + row_off + i);
    const uint32_t h[4] = {u.x & 0xFFFFu, u.x >> 16, u.y & 0xFFFFu, u.y >> 16};
#pragma unroll
    for (int q = 0; q < 4; ++q)
      v[q] = dtype == LATENT_BF16 ? __uint_as_float(h[q] << 16) : half_bits_to_float(static_cast<uint16_t>(h[q]));
    return make_float4(v[0], v[1], v[2], v[3]);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = i + q < n ? load_act(base, dtype, row_off + i + q) : 0.f;
  return make_float4(v[0], v[1], v[2], v[3]);
}

// grid (ceil(E/64), nslice, ceil(T/32)); 256 threads.  Every thread issues its
// 4 router chunks and 2 activation chunks (4 elements each) before the first
// LDS store, so a workgroup costs about one memory round trip.  The 32 x 64
// tile is then computed on fp32 matrix cores (v_mfma_f32_16x16x4_f32: fp32
// products and accumulation): wave w owns experts 16w..16w+15 and both
// 16-token halves, 16 steps of 4 rows (64-row slices: the dependent MFMA
// chains of 128-row slices took 9.7 us against 7.2 at d = 7168, batch 32).
typedef float float4v __attribute__((ext_vector_type(4)));
constexpr int kWPitch = kCols + 4;  // router tile row pitch (floats): fewer bank conflicts
__global__ void __launch_bounds__(kThreads) logits_kernel(Params p) {
  __shared__ float xs[kTok][kRows + 4];
  __shared__ float ws[kRows][kWPitch];
  const int tid = threadIdx.x;
  const int e0 = blockIdx.x * kCols, r0 = blockIdx.y * kRows, t0 = blockIdx.z * kTok;
  const int nr = min(kRows, p.d - r0), nt = min(kTok, p.T - t0), ne = min(kCols, p.E - e0);
  constexpr int kWChunks = kRows * kCols / 4 / kThreads;  // 8
  constexpr int kXChunks = kTok * kRows / 4 / kThreads;   // 4
  float4 wv[kWChunks], xv[kXChunks];
#pragma unroll
  for (int u = 0; u < kWChunks; ++u) {
    const int i = tid + u * kThreads, r = i / (kCols / 4), c = (i % (kCols / 4)) * 4;
    wv[u] = r < nr ? load4(p.router, p.router_dtype, static_cast<int64_t>(r0 + r) * p.E + e0, c, ne, p.vec_router)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int u = 0; u < kXChunks; ++u) {
    const int i = tid + u * kThreads, t = i / (kRows / 4), r = (i % (kRows / 4)) * 4;
    xv[u] = t < nt ? load4(p.x, p.x_dtype, static_cast<int64_t>(t0 + t) * p.d + r0, r, nr, p.vec_x)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int u = 0; u < kWChunks; ++u) {
    const int i = tid + u * kThreads, r = i / (kCols / 4), c = (i % (kCols / 4)) * 4;
    *reinterpret_cast<float4*>(&ws[r][c]) = wv[u];
  }
#pragma unroll
  for (int u = 0; u < kXChunks; ++u) {
    const int i = tid + u * kThreads, t = i / (kRows / 4), r = (i % (kRows / 4)) * 4;
    *reinterpret_cast<float4*>(&xs[t][r]) = xv[u];
  }
  __syncthreads();
  // Lane l: A = x[16h + l % 16][k + l / 16], B = W[k + l / 16][16w + l % 16];
  // C lane l holds rows 4 (l / 16) .. + 3 of column l % 16.
  const int lane = tid & (kWave - 1), w = tid >> 6;
  const int lr = lane & 15, lk = lane >> 4;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
#pragma unroll 8
  for (int k = 0; k < kRows; k += 4) {  // rows beyond nr hold zeros
    const float b = ws[k + lk][w * 16 + lr];
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[lr][k + lk], b, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[16 + lr][k + lk], b, acc[1], 0, 0, 0);
  }
  const int c = w * 16 + lr;
  if (c < ne) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = h * 16 + lk * 4 + i;
        if (t < nt) p.partial[(static_cast<int64_t>(blockIdx.y) * p.T + t0 + t) * p.E + e0 + c] = acc[h][i];
      }
  }
}

// Wave arg-max of (v, idx) pairs: larger v wins, equal v -> smaller idx.
// Each pair is one 64-bit key whose unsigned order is that order (the
// float's bits made monotonic above, the complemented index below; -0 is
// +0 first, so equal values tie), reduced over the wave with DPP row
// permutations and the permlane swaps (no LDS round trips).
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  uint32_t lo = ~static_cast<uint32_t>(idx);
  auto take = [&](uint32_t ohi, uint32_t olo) __attribute__((always_inline)) {
    const bool gt = ohi > hi || (ohi == hi && olo > lo);
    hi = gt ? ohi : hi;
    lo = gt ? olo : lo;
  };
  auto dpp = [&](auto ctrl) __attribute__((always_inline)) {
    constexpr int c = decltype(ctrl)::value;
    take(static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(hi), c, 0xF, 0xF, false)),
         static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(lo), c, 0xF, 0xF, false)));
  };
  dpp(std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]: lane ^ 1
  dpp(std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]: lane ^ 2
  dpp(std::integral_constant<int, 0x124>{});  // row_ror:4
  dpp(std::integral_constant<int, 0x128>{});  // row_ror:8
  {  // rows r and r ^ 1
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const uint32_t h0 = h[0], h1 = h[1], l0 = l[0], l1 = l[1];
    hi = h0; lo = l0;
    take(h1, l1);
  }
  {  // lane halves
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const uint32_t h0 = h[0], h1 = h[1], l0 = l[0], l1 = l[1];
    hi = h0; lo = l0;
    take(h1, l1);
  }
  v = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
  idx = static_cast<int>(~lo);
}

// One token per 256-thread workgroup.  Thread e sums the slices of expert e
// (all loads in flight at once, added in slice order) into LDS; wave 0 then
// selects the top k.
__global__ void __launch_bounds__(kThreads) topk_kernel(Params p) {
  __shared__ float lg[kMaxE];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int t = blockIdx.x;
  const int nj = (p.E + kWave - 1) / kWave;
  for (int e = threadIdx.x; e < p.E; e += kThreads) {
    float v;
    if (p.logits_in) {
      v = p.logits_in[static_cast<int64_t>(t) * p.E + e];
    } else {
      const float* src = p.partial + static_cast<int64_t>(t) * p.E + e;
      const int64_t stride = static_cast<int64_t>(p.T) * p.E;
      // Up to kSliceBatch slices in flight (d = 7168: all 112 in one round
      // trip), added in slice order.
      float part[kSliceBatch];
      v = 0.f;
      for (int s0 = 0; s0 < p.nslice; s0 += kSliceBatch) {
        // One pointer stepped by the slice stride (indexed loads kept one
        // scalar offset per slice and spilled them).
        typedef const __attribute__((address_space(1))) float* gptr;
        uintptr_t q = reinterpret_cast<uintptr_t>(src + s0 * stride);
#pragma unroll
        for (int i = 0; i < kSliceBatch; ++i) {
          part[i] = s0 + i < p.nslice ? *reinterpret_cast<gptr>(q) : 0.f;
          q += static_cast<uintptr_t>(stride) * sizeof(float);
          asm volatile("" : "+v"(q));
        }
#pragma unroll
        for (int i = 0; i < kSliceBatch; ++i) v += part[i];
      }
    }
    if (p.logits_out) p.logits_out[static_cast<int64_t>(t) * p.E + e] = v;
    lg[e] = v != v ? -INFINITY : v;  // NaN never wins a slot
  }
  __syncthreads();
  if (wave != 0) return;
  float l[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = j * kWave + lane;
    l[j] = (j < nj && e < p.E) ? lg[e] : -INFINITY;
  }
  // Top-k: k rounds of wave arg-max; a chosen expert is retired with a bit
  // of `taken`, so it cannot be chosen again even if every logit is -inf.
  // Lane s keeps the logit and id of slot s.
  uint32_t taken = 0;
  float my_l = -INFINITY;
  int my_e = -1;
  for (int s = 0; s < p.K; ++s) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      if (j >= nj) break;  // wave-uniform: the layer's experts only
      const int e = j * kWave + lane;
      const bool ok = e < p.E && !((taken >> j) & 1u);
      if (ok && (l[j] > bv || bi == 0x7FFFFFFF)) {
        bv = l[j];
        bi = e;
      }
    }
    wave_argmax(bv, bi);
    if (lane == s) {
      my_l = bv;
      my_e = bi;
    }
    if (bi != 0x7FFFFFFF && (bi & (kWave - 1)) == lane) taken |= 1u << (bi / kWave);
  }
  // Renormalised softmax over the kept k (the full softmax denominator
  // cancels); sums run serially in slot order.
  const float m = __shfl(my_l, 0, kWave);
  float w = lane < p.K ? expf(my_l - m) : 0.f;
  float wsum = 0.f;
  for (int s = 0; s < p.K; ++s) wsum += __shfl(w, s, kWave);
  w = w / wsum;
  int keep = p.K;
  if (p.drop_rule == LATENT_DROP_INCLUSIVE) {
    // loader/adaptive_topk.py:29-55 on the descending top-k scores.
    float total = 0.f;
    for (int s = 0; s < p.K; ++s) total += __shfl(w, s, kWave);
    const float target = p.drop_param * total;
    float cum = 0.f;
    for (int s = 0; s < p.K; ++s) {
      const float ws = __shfl(w, s, kWave);
      if (cum + ws > target) {
        keep = s;
        break;
      }
      cum += ws;
    }
  }
  if (lane < p.K) {
    bool drop = lane >= keep;
    if (p.drop_rule == LATENT_DROP_BELOW && w < p.drop_param) drop = true;
    const int64_t o = static_cast<int64_t>(t) * p.K + lane;
    p.ids[o] = drop ? -1 : my_e;
    p.weights[o] = drop ? 0.f : w;
  }
}

int64_t n_slices(int64_t d) { return (d + kRows - 1) / kRows; }

int validate(const latent_route_args& a) {
  if (a.n_tokens < 0 || a.n_expert <= 0 || a.n_expert_used <= 0) return LATENT_E_INVALID;
  if (a.n_expert_used > a.n_expert) return LATENT_E_INVALID;
  if (a.drop_rule < LATENT_DROP_NONE || a.drop_rule > LATENT_DROP_INCLUSIVE) return LATENT_E_INVALID;
  if (a.drop_rule == LATENT_DROP_INCLUSIVE && !(a.drop_param > 0.f && a.drop_param <= 1.f)) return LATENT_E_INVALID;
  if (!a.logits_in) {
    if (a.n_embd <= 0) return LATENT_E_INVALID;
    if (a.x_dtype < LATENT_F32 || a.x_dtype > LATENT_BF16) return LATENT_E_INVALID;
    if (a.router_dtype != LATENT_F32 && a.router_dtype != LATENT_BF16) return LATENT_E_INVALID;
  }
  if (a.n_expert > kMaxE || a.n_expert_used > kMaxK) return LATENT_E_UNSUPPORTED;
  if (a.n_tokens > (1 << 24) || a.n_embd > (1 << 20)) return LATENT_E_UNSUPPORTED;
  return LATENT_OK;
}

size_t workspace_bytes(const latent_route_args& a) {
  if (a.logits_in) return 0;
  return static_cast<size_t>(n_slices(a.n_embd)) * a.n_tokens * a.n_expert * sizeof(float);
}

}  // namespace
}  // namespace route
}  // namespace latent

using namespace latent;

extern "C" int latent_route_workspace_size(const latent_route_args* args, size_t* bytes) {
  if (!args || !bytes) return LATENT_E_INVALID;
  const int st = route::validate(*args);
  if (st != LATENT_OK) return st;
  *bytes = route::workspace_bytes(*args);
  return LATENT_OK;
}

extern "C" int latent_route(const latent_route_args* args, latent_stream_t stream) {
  if (!args) return LATENT_E_INVALID;
  const latent_route_args& a = *args;
  const int st = route::validate(a);
  if (st != LATENT_OK) return st;
  if (a.n_tokens == 0) return LATENT_OK;
  if (!a.ids || !a.weights) return LATENT_E_INVALID;
  if (!a.logits_in && (!a.x || !a.router)) return LATENT_E_INVALID;
  const size_t need = route::workspace_bytes(a);
  if (need && (!a.workspace || a.workspace_bytes < need)) return LATENT_E_WORKSPACE;
  route::Params p{};
  p.x = a.x;
  p.x_dtype = a.x_dtype;
  p.router = a.router;
  p.router_dtype = a.router_dtype;
  p.logits_in = a.logits_in;
  p.logits_out = a.logits_out;
  p.ids = a.ids;
  p.weights = a.weights;
  p.partial = static_cast<float*>(a.workspace);
  p.T = static_cast<int>(a.n_tokens);
  p.d = static_cast<int>(a.n_embd);
  p.E = static_cast<int>(a.n_expert);
  p.K = static_cast<int>(a.n_expert_used);
  p.nslice = a.logits_in ? 0 : static_cast<int>(route::n_slices(a.n_embd));
  p.drop_rule = a.drop_rule;
  p.drop_param = a.drop_param;
  auto aligned = [](const void* q, int dtype) {
    return (reinterpret_cast<uintptr_t>(q) & (dtype == LATENT_F32 ? 15u : 7u)) == 0;
  };
  p.vec_router = a.router && a.n_expert % 4 == 0 && aligned(a.router, a.router_dtype);
  p.vec_x = a.x && a.n_embd % 4 == 0 && aligned(a.x, a.x_dtype);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (!a.logits_in) {
    const dim3 grid(static_cast<unsigned>((a.n_expert + route::kCols - 1) / route::kCols), static_cast<unsigned>(p.nslice),
                    static_cast<unsigned>((a.n_tokens + route::kTok - 1) / route::kTok));
    hipLaunchKernelGGL(route::logits_kernel, grid, dim3(route::kThreads), 0, s, p);
    if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  }
  hipLaunchKernelGGL(route::topk_kernel, dim3(static_cast<unsigned>(a.n_tokens)), dim3(route::kThreads), 0, s, p);
  return hipGetLastError() == hipSuccess ? LATENT_OK : LATENT_E_HIP;
}
