// Host-side argument handling of liblatent_hip.so under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/test_host_sanitizers.py from the
// library's host code only).  Every call below returns before any kernel
// launch: the checks of shapes, enums, pointers and workspaces, the workspace
// sizes of the DeepSeek-V3-shaped decode, prefill and heterogeneous layers,
// the path and layout queries, and the codec, router, single-expert and
// repack entry points.  Exit status = number of failed expectations.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "latent_ffn.h"

static int failures = 0;
#define EXPECT(cond)                                                    \
  do {                                                                  \
    if (!(cond)) {                                                      \
      std::fprintf(stderr, "%s:%d: expectation failed: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                       \
    }                                                                   \
  } while (0)

namespace {

// Host buffers standing in for the twelve factor tensors (never read: every
// call returns before a launch).
struct Layer {
  std::vector<uint8_t> bytes;
  latent_moe_args a{};
  Layer(int64_t T, int64_t d, int64_t ff, int64_t E, int64_t k, int64_t R) : bytes(1 << 16) {
    uint8_t* base = bytes.data() + ((16 - reinterpret_cast<uintptr_t>(bytes.data()) % 16) % 16);
    auto fac = [&](int64_t rows, int64_t cols) {
      latent_factor f{};
      f.codes = base;
      f.scales = reinterpret_cast<const uint16_t*>(base);
      f.rows = rows;
      f.cols = cols;
      return f;
    };
    a.gate_a = fac(d, R);
    a.gate_b = fac(R, ff);
    a.up_a = fac(d, R);
    a.up_b = fac(R, ff);
    a.down_a = fac(ff, R);
    a.down_b = fac(R, d);
    a.n_tokens = T;
    a.n_embd = d;
    a.n_ff = ff;
    a.n_expert = E;
    a.n_expert_used = k;
    a.max_rank = R;
    a.x_dtype = LATENT_BF16;
    a.weights_dtype = LATENT_F32;
    a.out_mode = LATENT_OUT_REDUCED;
  }
};

size_t workspace(const latent_moe_args& a, int* status) {
  size_t n = 0;
  *status = latent_moe_workspace_size(&a, &n);
  return n;
}

void status_strings() {
  EXPECT(latent_version() >= 100);
  for (int s = -6; s <= 1; ++s) EXPECT(latent_status_string(s) != nullptr);
  EXPECT(std::strcmp(latent_status_string(12345), "unknown status") == 0);
}

void workspace_sizes() {
  // DeepSeek-V3 shape: decode batches, prefill, and the heterogeneous layer
  // (per-expert ranks up to 512, INT8 groups).
  for (int64_t T : {1, 8, 64, 4096}) {
    Layer L(T, 7168, 2048, 256, 8, 256);
    int st = 0;
    const size_t rows = workspace(L.a, &st);
    EXPECT(st == LATENT_OK && rows > 0);
    L.a.layout = LATENT_LAYOUT_TILES;
    EXPECT(latent_tiles_supported(&L.a) == 1);
    const size_t tiles = workspace(L.a, &st);
    EXPECT(st == LATENT_OK && tiles > 0);
  }
  std::vector<int32_t> ranks(256 * 3, 64);
  std::vector<uint32_t> bitmap(16);
  std::vector<int32_t> offsets(16);
  std::vector<int8_t> data(64);
  for (int64_t T : {16, 256}) {
    Layer L(T, 7168, 2048, 256, 8, 512);
    L.a.ranks = ranks.data();
    L.a.up_a.int8_bitmap = bitmap.data();
    L.a.up_a.int8_row_offset = offsets.data();
    L.a.up_a.int8_data = data.data();
    int st = 0;
    EXPECT(workspace(L.a, &st) > 0 && st == LATENT_OK);
    EXPECT(latent_tiles_supported(&L.a) == 0);
    L.a.layout = LATENT_LAYOUT_TILES;
    workspace(L.a, &st);
    EXPECT(st == LATENT_E_UNSUPPORTED);
    EXPECT(latent_moe_path(&L.a) == LATENT_E_UNSUPPORTED);
  }
  // The workspace grows with the routed pairs.
  Layer small(8, 256, 512, 16, 4, 64), big(64, 256, 512, 16, 4, 64);
  int s1 = 0, s2 = 0;
  EXPECT(workspace(small.a, &s1) < workspace(big.a, &s2) && s1 == LATENT_OK && s2 == LATENT_OK);
}

void invalid_arguments() {
  struct Case {
    void (*mutate)(latent_moe_args&);
    int status;
  };
  const Case cases[] = {
      {[](latent_moe_args& a) { a.n_embd = 250; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.max_rank = 48; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.x_dtype = 9; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.out_mode = 2; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.weights_dtype = 2; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.gate_b.cols = 256; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.down_a.codes = nullptr; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.layout = 3; }, LATENT_E_INVALID},
      {[](latent_moe_args& a) { a.n_expert = 5000; }, LATENT_E_UNSUPPORTED},
      {[](latent_moe_args& a) { a.n_expert_used = 65; }, LATENT_E_UNSUPPORTED},
  };
  for (const Case& c : cases) {
    Layer L(8, 256, 512, 16, 4, 64);
    c.mutate(L.a);
    int st = 0;
    workspace(L.a, &st);
    EXPECT(st == c.status);
    EXPECT(latent_moe_ffn_forward(&L.a, nullptr) == c.status);
  }
  EXPECT(latent_moe_workspace_size(nullptr, nullptr) == LATENT_E_INVALID);
  EXPECT(latent_moe_ffn_forward(nullptr, nullptr) == LATENT_E_INVALID);
  // Missing activations, then a missing workspace, then the empty call.
  Layer L(8, 256, 512, 16, 4, 64);
  EXPECT(latent_moe_ffn_forward(&L.a, nullptr) == LATENT_E_INVALID);
  alignas(16) static float io[64];
  static int32_t ids[64];
  L.a.x = io;
  L.a.ids = ids;
  L.a.weights = io;
  L.a.out = io;
  EXPECT(latent_moe_ffn_forward(&L.a, nullptr) == LATENT_E_WORKSPACE);
  L.a.n_tokens = 0;
  EXPECT(latent_moe_ffn_forward(&L.a, nullptr) == LATENT_OK);
  uint8_t small_ws[64];
  EXPECT(latent_moe_check(small_ws, sizeof small_ws, nullptr) == LATENT_E_WORKSPACE);
}

void codec_route_expert_repack() {
  latent_factor f{};
  f.rows = 4;
  f.cols = 64;
  alignas(16) static float buf[1024];
  EXPECT(latent_unpack(&f, 0, buf, nullptr) == LATENT_E_INVALID);
  EXPECT(latent_pack_nf4(nullptr, 4, 64, nullptr, nullptr, nullptr) == LATENT_E_INVALID);
  EXPECT(latent_pack_nf4(buf, 4, 48, reinterpret_cast<uint8_t*>(buf), reinterpret_cast<uint16_t*>(buf), nullptr) ==
         LATENT_E_INVALID);
  EXPECT(latent_pack_int8(buf, 0, reinterpret_cast<int8_t*>(buf), reinterpret_cast<uint16_t*>(buf), nullptr) ==
         LATENT_E_INVALID);

  latent_route_args r{};
  r.n_tokens = 4;
  r.n_embd = 7168;
  r.n_expert = 256;
  r.n_expert_used = 8;
  r.x_dtype = LATENT_BF16;
  r.router_dtype = LATENT_F32;
  size_t n = 0;
  EXPECT(latent_route_workspace_size(&r, &n) == LATENT_OK && n == 112u * 4 * 256 * 4);
  latent_route_args b = r;
  b.n_expert_used = 257;
  EXPECT(latent_route_workspace_size(&b, &n) == LATENT_E_INVALID);
  b = r;
  b.n_expert = 2048;
  EXPECT(latent_route_workspace_size(&b, &n) == LATENT_E_UNSUPPORTED);
  b = r;
  b.drop_rule = 7;
  EXPECT(latent_route_workspace_size(&b, &n) == LATENT_E_INVALID);
  b = r;
  b.drop_rule = LATENT_DROP_INCLUSIVE;
  b.drop_param = 1.5f;
  EXPECT(latent_route(&b, nullptr) == LATENT_E_INVALID);

  static uint8_t data[4096];
  static uint16_t scales[256];
  latent_expert_args e{};
  const int64_t shapes[6][2] = {{16, 4}, {4, 12}, {16, 4}, {4, 12}, {12, 4}, {4, 16}};
  latent_flat_factor* fs[6] = {&e.gate_a, &e.gate_b, &e.up_a, &e.up_b, &e.down_a, &e.down_b};
  for (int i = 0; i < 6; ++i) {
    fs[i]->data = data;
    fs[i]->scales = scales;
    fs[i]->kind = LATENT_Q_NF4;
    fs[i]->group_size = 32;
    fs[i]->rows = shapes[i][0];
    fs[i]->cols = shapes[i][1];
  }
  e.n_tokens = 3;
  EXPECT(latent_expert_workspace_size(&e, &n) == LATENT_OK && n > 0);
  latent_expert_args eb = e;
  eb.gate_b.rows = 5;
  EXPECT(latent_expert_workspace_size(&eb, &n) == LATENT_E_INVALID);
  eb = e;
  eb.up_a.group_size = 48;
  EXPECT(latent_expert_forward(&eb, nullptr) == LATENT_E_UNSUPPORTED);
  EXPECT(latent_expert_forward(&e, nullptr) == LATENT_E_INVALID);  // no x / out

  latent_factor src{}, dst{};
  src.codes = data;
  src.scales = scales;
  dst.codes = data + 32;
  dst.scales = scales + 16;
  src.rows = dst.rows = 512;
  src.cols = dst.cols = 256;
  EXPECT(latent_tiles_repack(LATENT_GATE_B, &src, &dst, 4, 1, nullptr) == LATENT_E_UNSUPPORTED);
  EXPECT(latent_tiles_repack(6, &src, &dst, 4, 1, nullptr) == LATENT_E_INVALID);
  EXPECT(latent_tiles_repack(LATENT_GATE_A, nullptr, &dst, 4, 1, nullptr) == LATENT_E_INVALID);
  src.rows = 384;
  dst.rows = 384;
  EXPECT(latent_tiles_repack(LATENT_GATE_A, &src, &dst, 4, 1, nullptr) == LATENT_E_UNSUPPORTED);
}

}  // namespace

int main() {
  status_strings();
  workspace_sizes();
  invalid_arguments();
  codec_route_expert_repack();
  std::printf("host ABI checks: %d failed\n", failures);
  return failures;
}
