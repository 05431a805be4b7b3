// Single-expert LATENT SwiGLU FFN on the factor artifacts exactly as
// loader/latent_loader.py writes them (flat quantization groups).
//
// Replaces swiglu_expert / _load_factor of loader/latent_runtime.py:19-59 for
// one expert: the six factors stay in their packed artifact form on the device
// and are dequantized on the fly.  Unlike the stacked per-row layout of the
// MoE-layer path, an artifact quantizes each factor as one flat row-major
// array: group g covers flat elements [g*G, (g+1)*G) whatever the row length
// (quantize_nf4 / quantize_int8, loader/latent_loader.py:111-158), so groups
// straddle rows whenever cols % G != 0 (odd ranks such as 37 from the
// energy-based rank choice, or INT8 group 64 on any shape).  Element (k, n) of
// a [rows][cols] factor is flat index i = k*cols + n:
//   NF4   code = nibble (i & 1) of byte i >> 1 (low nibble = even index),
//         value = level[code] * f32(scale_f16[i / G])
//   INT8  value = f32(q[i]) * f32(scale_f16[i / G])
// one fp32 multiply each, as dequantize_nf4 / dequantize_int8
// (loader/latent_loader.py:133-145, 161-170) compute it.
//
// The chain (loader/latent_runtime.py:35-59), all fp32:
//   gl = x . A_g, ul = x . A_u            K = d
//   g  = gl . B_g, u = ul . B_u           K = rank
//   dl = (SiLU(g) * u [* w]) . A_d        K = ff   (SwiGLU folded into staging)
//   y  = dl . B_d                         K = rank
// Each product is one launch of proj_kernel over (256-column tile, K slice,
// 8-token tile); with several K slices the fp32 partials are summed in slice
// order by reduce_kernel, so results are reproducible call to call.
#include "common.hpp"

#include <algorithm>

namespace latent {
namespace expert {
namespace {

constexpr int kT = 256;      // threads = output columns per workgroup
constexpr int kMT = 8;       // tokens per workgroup
constexpr int kStage = 512;  // K rows of activations staged in LDS at a time
constexpr int kTargetBlocks = 2048;
constexpr int kMinKSlice = 64;

struct Flat {
  const uint8_t* data;
  const uint16_t* scales;
  int kind;    // LATENT_Q_NF4 | LATENT_Q_INT8
  int gshift;  // log2(group size)
};

struct Proj {
  Flat f;
  const float* act;   // [T][K] (the gate product g for the SwiGLU prologue)
  const float* act2;  // [T][K] the up product u (SwiGLU prologue only)
  float wmul;         // router weight applied before A_d (1 otherwise)
  float* dst;         // [S][T][N] partials, or the result when S == 1
  int T, K, N, ks;    // ks: K rows per slice
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <bool kSwiGLU>
__global__ void __launch_bounds__(kT) proj_kernel(Proj p) {
  __shared__ float act[kMT][kStage];
  __shared__ float lv[16];
  const int tid = threadIdx.x;
  const int n = blockIdx.x * kT + tid;
  const int s = blockIdx.y;
  const int t0 = blockIdx.z * kMT;
  const int mt = min(kMT, p.T - t0);
  const int k0 = s * p.ks, k1 = min(p.K, k0 + p.ks);
  if (tid < 16) lv[tid] = nf4_level(tid);
  float acc[kMT];
#pragma unroll
  for (int t = 0; t < kMT; ++t) acc[t] = 0.f;
  int64_t idx = static_cast<int64_t>(k0) * p.N + n;
  for (int kc = k0; kc < k1; kc += kStage) {
    const int kn = min(kStage, k1 - kc);
    __syncthreads();  // the previous chunk's readers are done
    for (int i = tid; i < kMT * kStage; i += kT) {
      const int t = i / kStage, k = i - t * kStage;
      float v = 0.f;
      if (t < mt && k < kn) {
        const int64_t o = static_cast<int64_t>(t0 + t) * p.K + kc + k;
        v = p.act[o];
        if (kSwiGLU) v = silu(v) * p.act2[o] * p.wmul;
      }
      act[t][k] = v;
    }
    __syncthreads();
    if (n < p.N) {
      for (int k = 0; k < kn; ++k, idx += p.N) {
        const float sc = half_bits_to_float(p.f.scales[idx >> p.f.gshift]);
        float w;
        if (p.f.kind == LATENT_Q_NF4) {
          const uint32_t b = p.f.data[idx >> 1];
          w = __fmul_rn(lv[(idx & 1) ? (b >> 4) : (b & 15u)], sc);
        } else {
          w = __fmul_rn(static_cast<float>(reinterpret_cast<const int8_t*>(p.f.data)[idx]), sc);
        }
#pragma unroll
        for (int t = 0; t < kMT; ++t) acc[t] = fmaf(act[t][k], w, acc[t]);
      }
    }
  }
  if (n >= p.N) return;
  for (int t = 0; t < mt; ++t) p.dst[(static_cast<int64_t>(s) * p.T + t0 + t) * p.N + n] = acc[t];
}

// dst[t][n] = sum over slices s (in order) of part[s][t][n].
__global__ void __launch_bounds__(kT) reduce_kernel(const float* part, float* dst, int64_t tn, int S) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; i < tn; i += static_cast<int64_t>(gridDim.x) * kT) {
    float v = 0.f;
    for (int s = 0; s < S; ++s) v += part[s * tn + i];
    dst[i] = v;
  }
}

struct Plan {
  int S, ks;
};

Plan plan_for(int64_t T, int64_t K, int64_t N) {
  const int64_t tiles = ((N + kT - 1) / kT) * ((T + kMT - 1) / kMT);
  int64_t S = std::max<int64_t>(1, (kTargetBlocks + tiles - 1) / tiles);
  S = std::min<int64_t>(S, std::max<int64_t>(1, K / kMinKSlice));
  S = std::min<int64_t>(S, 65535);
  const int64_t ks = (K + S - 1) / S;
  return {static_cast<int>((K + ks - 1) / ks), static_cast<int>(ks)};
}

int group_shift(int g) {
  if (g < 2 || (g & (g - 1))) return -1;
  int s = 0;
  while ((1 << s) < g) ++s;
  return s;
}

int check(const latent_flat_factor& f, int64_t rows, int64_t cols) {
  if (!f.data || !f.scales) return LATENT_E_INVALID;
  if (f.kind != LATENT_Q_NF4 && f.kind != LATENT_Q_INT8) return LATENT_E_INVALID;
  if (f.rows != rows || f.cols != cols || rows <= 0 || cols <= 0) return LATENT_E_INVALID;
  if (group_shift(f.group_size) < 0) return LATENT_E_UNSUPPORTED;  // power-of-two groups only
  if (rows > (1 << 24) || cols > (1 << 24) || rows * cols > (int64_t{1} << 40)) return LATENT_E_UNSUPPORTED;
  return LATENT_OK;
}

struct Dims {
  int64_t T, d, rg, ru, rd, ff;
};

int validate(const latent_expert_args& a, Dims& m) {
  m.T = a.n_tokens;
  m.d = a.gate_a.rows;
  m.rg = a.gate_a.cols;
  m.ff = a.gate_b.cols;
  m.ru = a.up_a.cols;
  m.rd = a.down_a.cols;
  if (m.T < 0 || m.T > (1 << 24)) return LATENT_E_INVALID;
  const struct {
    const latent_flat_factor* f;
    int64_t rows, cols;
  } want[6] = {{&a.gate_a, m.d, m.rg}, {&a.gate_b, m.rg, m.ff}, {&a.up_a, m.d, m.ru},
               {&a.up_b, m.ru, m.ff},   {&a.down_a, m.ff, m.rd}, {&a.down_b, m.rd, m.d}};
  for (const auto& w : want) {
    const int st = check(*w.f, w.rows, w.cols);
    if (st != LATENT_OK) return st;
  }
  return LATENT_OK;
}

size_t al(size_t v) { return (v + 255) / 256 * 256; }

struct Layout {
  size_t gl, ul, g, u, dl, part, total;
};

size_t part_floats(const Dims& m, int64_t K, int64_t N) {
  const Plan pl = plan_for(m.T, K, N);
  return pl.S > 1 ? static_cast<size_t>(pl.S) * m.T * N : 0;
}

Layout layout_for(const Dims& m) {
  Layout L{};
  size_t off = 0;
  L.gl = off; off = al(off + m.T * m.rg * 4);
  L.ul = off; off = al(off + m.T * m.ru * 4);
  L.g = off;  off = al(off + m.T * m.ff * 4);
  L.u = off;  off = al(off + m.T * m.ff * 4);
  L.dl = off; off = al(off + m.T * m.rd * 4);
  size_t part = 0;
  part = std::max(part, part_floats(m, m.d, m.rg));
  part = std::max(part, part_floats(m, m.d, m.ru));
  part = std::max(part, part_floats(m, m.rg, m.ff));
  part = std::max(part, part_floats(m, m.ru, m.ff));
  part = std::max(part, part_floats(m, m.ff, m.rd));
  part = std::max(part, part_floats(m, m.rd, m.d));
  L.part = off; off = al(off + part * 4);
  L.total = std::max<size_t>(off, 256);
  return L;
}

Flat flat(const latent_flat_factor& f) {
  return {static_cast<const uint8_t*>(f.data), f.scales, f.kind, group_shift(f.group_size)};
}

// dst[T][N] = act[T][K] . W[K][N] (SwiGLU prologue: act = SiLU(act) * act2 * w).
int project(const Dims& m, const latent_flat_factor& f, const float* act, const float* act2, float wmul, bool swiglu,
            float* dst, float* part, hipStream_t s) {
  const int64_t K = f.rows, N = f.cols;
  const Plan pl = plan_for(m.T, K, N);
  Proj p{};
  p.f = flat(f);
  p.act = act;
  p.act2 = act2;
  p.wmul = wmul;
  p.dst = pl.S > 1 ? part : dst;
  p.T = static_cast<int>(m.T);
  p.K = static_cast<int>(K);
  p.N = static_cast<int>(N);
  p.ks = pl.ks;
  const dim3 grid(static_cast<unsigned>((N + kT - 1) / kT), static_cast<unsigned>(pl.S),
                  static_cast<unsigned>((m.T + kMT - 1) / kMT));
  if (grid.z > 65535) return LATENT_E_UNSUPPORTED;
  if (swiglu)
    hipLaunchKernelGGL(proj_kernel<true>, grid, dim3(kT), 0, s, p);
  else
    hipLaunchKernelGGL(proj_kernel<false>, grid, dim3(kT), 0, s, p);
  if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  if (pl.S > 1) {
    const int64_t tn = m.T * N;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(4096, (tn + kT - 1) / kT));
    hipLaunchKernelGGL(reduce_kernel, dim3(blocks), dim3(kT), 0, s, part, dst, tn, pl.S);
    if (hipGetLastError() != hipSuccess) return LATENT_E_HIP;
  }
  return LATENT_OK;
}

}  // namespace
}  // namespace expert
}  // namespace latent

using namespace latent;

extern "C" int latent_expert_workspace_size(const latent_expert_args* args, size_t* bytes) {
  if (!args || !bytes) return LATENT_E_INVALID;
  expert::Dims m;
  const int st = expert::validate(*args, m);
  if (st != LATENT_OK) return st;
  *bytes = expert::layout_for(m).total;
  return LATENT_OK;
}

extern "C" int latent_expert_forward(const latent_expert_args* args, latent_stream_t stream) {
  if (!args) return LATENT_E_INVALID;
  const latent_expert_args& a = *args;
  expert::Dims m;
  int st = expert::validate(a, m);
  if (st != LATENT_OK) return st;
  if (m.T == 0) return LATENT_OK;
  if (!a.x || !a.out) return LATENT_E_INVALID;
  const expert::Layout L = expert::layout_for(m);
  if (!a.workspace || a.workspace_bytes < L.total) return LATENT_E_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(a.workspace) & 255u) return LATENT_E_WORKSPACE;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  char* ws = static_cast<char*>(a.workspace);
  float* gl = reinterpret_cast<float*>(ws + L.gl);
  float* ul = reinterpret_cast<float*>(ws + L.ul);
  float* g = reinterpret_cast<float*>(ws + L.g);
  float* u = reinterpret_cast<float*>(ws + L.u);
  float* dl = reinterpret_cast<float*>(ws + L.dl);
  float* part = reinterpret_cast<float*>(ws + L.part);
  const float w = a.weight_before_down ? a.weight : 1.0f;
  if ((st = expert::project(m, a.gate_a, a.x, nullptr, 1.f, false, gl, part, s)) != LATENT_OK) return st;
  if ((st = expert::project(m, a.up_a, a.x, nullptr, 1.f, false, ul, part, s)) != LATENT_OK) return st;
  if ((st = expert::project(m, a.gate_b, gl, nullptr, 1.f, false, g, part, s)) != LATENT_OK) return st;
  if ((st = expert::project(m, a.up_b, ul, nullptr, 1.f, false, u, part, s)) != LATENT_OK) return st;
  if ((st = expert::project(m, a.down_a, g, u, w, true, dl, part, s)) != LATENT_OK) return st;
  return expert::project(m, a.down_b, dl, nullptr, 1.f, false, a.out, part, s);
}
