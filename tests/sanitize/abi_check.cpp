// Host-side AddressSanitizer / UndefinedBehaviorSanitizer check of the C ABI's argument
// validation and of the oracle's C expert MLP.  Built by tests/sanitize/Makefile with the
// library's sources compiled for the host only (no device code, no GPU needed): every call here
// is refused or answered before anything would be launched.  Exit status 0 = all checks passed
// and no sanitizer report (the sanitizers abort on their first finding).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/kandiga_amd.h"

extern "C" {
typedef struct {
  const void* w;
  const uint16_t* s;
  const uint16_t* b;
  int64_t w_stride;
  int64_t s_stride;
} oracle_proj;
typedef struct {
  int hidden, inter, bits, scale_bf16, act;
  oracle_proj gate, up, down;
} oracle_layer;
int oracle_switch_mlp(const oracle_layer* L, const uint16_t* x_f16, const int32_t* idx, int T, int K, float* y,
                      int nthreads);
int oracle_switch_mlp_f32(const oracle_layer* L, const float* x_f32, const int32_t* idx, int T, int K, float* y,
                          int nthreads);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
}

static int g_fail = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "check failed line %d: %s\n", __LINE__, #cond); \
      g_fail = 1;                                                     \
    }                                                                 \
  } while (0)

static kmoe_layer_desc desc(int H, int I, int E, int K, int bits) {
  kmoe_layer_desc d;
  std::memset(&d, 0, sizeof d);
  d.hidden = H;
  d.intermediate = I;
  d.num_experts = E;
  d.top_k = K;
  d.bits = bits;
  d.group_size = 64;
  d.scale_dtype = KMOE_SCALE_F16;
  d.activation = KMOE_ACT_SWIGLU;
  const uintptr_t fake = 1u << 20;  // aligned, never dereferenced by the validation
  kmoe_qproj* ps[3] = {&d.gate, &d.up, &d.down};
  for (int p = 0; p < 3; ++p) {
    const int rows = p < 2 ? I : H, cols = p < 2 ? H : I;
    ps[p]->weight = ps[p]->scales = ps[p]->biases = reinterpret_cast<const void*>(fake);
    ps[p]->weight_expert_stride = (int64_t)rows * cols * bits / 8;
    ps[p]->scale_expert_stride = (int64_t)rows * cols / 64 * 2;
  }
  return d;
}

static void abi_checks() {
  void* const fake = reinterpret_cast<void*>(uintptr_t(1) << 20);
  const float* const flog = static_cast<const float*>(fake);
  kmoe_layer* L = nullptr;
  kmoe_layer_desc d = desc(2048, 512, 256, 8, 3);
  CHECK(kmoe_layer_create(&d, &L) == KMOE_OK && L);
  size_t n1 = 0, n2 = 0;
  CHECK(kmoe_workspace_size(L, 1, &n1) == KMOE_OK && kmoe_workspace_size(L, 4096, &n2) == KMOE_OK && n1 < n2);
  // bad descriptors
  kmoe_layer* bad = nullptr;
  kmoe_layer_desc b = d;
  b.bits = 5;
  CHECK(kmoe_layer_create(&b, &bad) == KMOE_ERR_UNSUPPORTED && !bad);
  b = d;
  b.top_k = 17;
  CHECK(kmoe_layer_create(&b, &bad) == KMOE_ERR_INVALID_ARG);
  b = d;
  b.gate.weight_expert_stride = 5;
  CHECK(kmoe_layer_create(&b, &bad) != KMOE_OK);
  CHECK(kmoe_layer_create(nullptr, &bad) == KMOE_ERR_INVALID_ARG);
  // calls refused before launch
  CHECK(kmoe_forward(L, fake, flog, 1, fake, 5, nullptr, nullptr, fake, 1 << 30, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_forward(L, (char*)fake + 2, flog, 1, fake, 0, nullptr, nullptr, fake, 1 << 30, nullptr) ==
        KMOE_ERR_ALIGNMENT);
  CHECK(kmoe_forward(L, fake, flog, 4, fake, 0, nullptr, nullptr, fake, 512, nullptr) == KMOE_ERR_WORKSPACE);
  CHECK(kmoe_forward_x(L, fake, 9, flog, 1, fake, 0, nullptr, nullptr, fake, 1 << 30, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_expert_mlp_x(L, fake, -1, (const int32_t*)fake, 1, fake, fake, 1 << 30, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_forward(L, nullptr, nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr) == KMOE_OK);
  CHECK(kmoe_route(nullptr, 4, 256, 0, nullptr, nullptr, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_combine(nullptr, nullptr, 3, 0, 64, nullptr, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_dequantize(L, 3, 0, 0, 1, (uint8_t*)fake, (uint16_t*)fake, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_dequantize(L, 2, 0, 2040, 9, (uint8_t*)fake, (uint16_t*)fake, nullptr) == KMOE_ERR_INVALID_ARG);
  size_t np = 0;
  CHECK(kmoe_permute_workspace_size(4096, 8, 256, &np) == KMOE_OK && np > 4096 * 8 * 8);
  CHECK(kmoe_permute(nullptr, 4, 8, 2000, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr) ==
        KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_prefill_pack_size(&d, &np) == KMOE_OK && np > 0);
  CHECK(kmoe_tq3_gemv(fake, 64, 48, fake, 0, 1, (float*)fake, nullptr) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_tq3_gemv(fake, 64, 64, (char*)fake + 4, 0, 1, (float*)fake, nullptr) == KMOE_ERR_ALIGNMENT);
  CHECK(kmoe_tq3_workspace_size(1, 0, 512, &np) == KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_tq3_expert_mlp(fake, 3 * 2048 * 512 / 32 * 20, 4, 2048, 512, fake, (const int32_t*)fake, 2, 8, fake, fake,
                            1024, nullptr) == KMOE_ERR_WORKSPACE);
  CHECK(kmoe_tq3_expert_mlp(fake, 100, 4, 2048, 512, fake, (const int32_t*)fake, 1, 8, fake, fake, 1 << 20, nullptr) ==
        KMOE_ERR_INVALID_ARG);
  CHECK(kmoe_profile_begin(0) == KMOE_ERR_INVALID_ARG);
  CHECK(std::strlen(kmoe_strerror(KMOE_ERR_WORKSPACE)) > 0 && std::strlen(kmoe_last_error()) > 0);
  // block: a shared-expert gate without a shared expert is refused
  kmoe_block_desc bd;
  std::memset(&bd, 0, sizeof bd);
  bd.routed = L;
  bd.bits = 4;
  bd.scale_dtype = KMOE_SCALE_BF16;
  kmoe_block* blk = nullptr;
  CHECK(kmoe_block_create(&bd, &blk) != KMOE_OK && !blk);
  CHECK(kmoe_layer_destroy(L) == KMOE_OK);
}

// The oracle's C expert MLP on a small seeded layer: both activation entries, single- and
// multi-threaded, agree bit for bit on fp16-representable activations.
static void oracle_checks() {
  const int H = 128, I = 64, E = 5, K = 3, T = 3;
  for (int bits = 3; bits <= 4; ++bits) {
    std::vector<uint8_t> w[3];
    std::vector<uint16_t> s[3], bb[3];
    uint32_t st = 12345u + bits;
    auto rnd = [&]() { st = st * 1664525u + 1013904223u; return st >> 8; };
    oracle_layer L;
    std::memset(&L, 0, sizeof L);
    L.hidden = H;
    L.inter = I;
    L.bits = bits;
    oracle_proj* ps[3] = {&L.gate, &L.up, &L.down};
    for (int p = 0; p < 3; ++p) {
      const int rows = p < 2 ? I : H, cols = p < 2 ? H : I;
      const size_t wb = (size_t)rows * cols * bits / 8, sb = (size_t)rows * cols / 64;
      w[p].resize(wb * E);
      s[p].resize(sb * E);
      bb[p].resize(sb * E);
      for (auto& v : w[p]) v = (uint8_t)rnd();
      for (size_t i = 0; i < s[p].size(); ++i) {
        const float sc = 0.001f + (rnd() % 1000) * 1e-5f;
        s[p][i] = oracle_f32_to_f16(sc);
        bb[p][i] = oracle_f32_to_f16(-(float)(1 << (bits - 1)) * oracle_f16_to_f32(s[p][i]));
      }
      *ps[p] = oracle_proj{w[p].data(), s[p].data(), bb[p].data(), (int64_t)wb, (int64_t)sb};
    }
    std::vector<uint16_t> x16(T * H);
    std::vector<float> x32(T * H);
    for (int i = 0; i < T * H; ++i) {
      x16[i] = oracle_f32_to_f16(((int)(rnd() % 2001) - 1000) * 1e-3f);
      x32[i] = oracle_f16_to_f32(x16[i]);
    }
    std::vector<int32_t> idx(T * K);
    for (int i = 0; i < T * K; ++i) idx[i] = (i * 7 + bits) % E;
    std::vector<float> y1(T * K * H), y2(T * K * H), y3(T * K * H);
    CHECK(oracle_switch_mlp(&L, x16.data(), idx.data(), T, K, y1.data(), 1) == 0);
    CHECK(oracle_switch_mlp(&L, x16.data(), idx.data(), T, K, y2.data(), 3) == 0);
    CHECK(oracle_switch_mlp_f32(&L, x32.data(), idx.data(), T, K, y3.data(), 2) == 0);
    CHECK(std::memcmp(y1.data(), y2.data(), y1.size() * 4) == 0);
    CHECK(std::memcmp(y1.data(), y3.data(), y1.size() * 4) == 0);
    CHECK(oracle_switch_mlp(&L, nullptr, idx.data(), T, K, y1.data(), 1) != 0);
  }
}

int main() {
  abi_checks();
  oracle_checks();
  std::printf(g_fail ? "FAILED\n" : "OK\n");
  return g_fail;
}
