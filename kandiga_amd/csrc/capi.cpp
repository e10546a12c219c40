// C ABI of libkandiga_amd.so: argument validation, workspace carve-up and dispatch.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/kandiga_amd.h"
#include "kmoe_internal.h"

using namespace kmoe;

struct kmoe_layer {
  LayerConfig cfg;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return KMOE_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(KMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// Per-thread kernel timing state (kmoe_profile_begin / kmoe_profile_end).
struct ProfRec {
  const char* name;
  hipEvent_t e0, e1;
};
struct Prof {
  bool on = false;
  hipError_t failed = hipSuccess;
  std::vector<hipEvent_t> events;
  std::vector<ProfRec> recs;
};
thread_local Prof g_prof;

Prof& prof() { return g_prof; }
bool prof_on() { return g_prof.on; }
void prof_reset() {
  for (hipEvent_t ev : g_prof.events)
    if (ev) (void)hipEventDestroy(ev);
  g_prof = Prof{};
}

// m-tiles of TK assignments over E experts at bm rows per tile, at most (workspace sizing uses the
// shorter tiles).
int max_mtiles_for(int TK, int E, int bm = GEMM_BM_PACK) { return (TK + bm - 1) / bm + (E < TK ? E : TK); }

// Carve the workspace for `T` tokens.  base == nullptr computes the size only.
Work carve(char* base, int T, int K, int E, int H, int I, int Is, bool need_y, size_t* total) {
  Work w{};
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += up256(bytes);
    return p;
  };
  const size_t TK = (size_t)T * K;
  const int ntiles = (int)((TK + PERM_TILE - 1) / PERM_TILE);
  const int mmt = max_mtiles_for((int)TK, E);
  w.scalars = reinterpret_cast<int32_t*>(take(64 * sizeof(int32_t)));
  w.idx = reinterpret_cast<int32_t*>(take(TK * 4));
  w.wts = reinterpret_cast<float*>(take(TK * 4));
  w.perm = reinterpret_cast<int32_t*>(take(TK * 4));
  w.local_rank = reinterpret_cast<int32_t*>(take(TK * 4));
  w.tile_hist = reinterpret_cast<int32_t*>(take((size_t)ntiles * E * 4));
  w.counts = reinterpret_cast<int32_t*>(take((size_t)E * 4));
  w.offsets = reinterpret_cast<int32_t*>(take((size_t)(E + 1) * 4));
  w.unique = reinterpret_cast<int32_t*>(take((size_t)E * 4));
  w.ustart = reinterpret_cast<int32_t*>(take((size_t)(E + 1) * 4));
  w.mt_expert = reinterpret_cast<int32_t*>(take((size_t)mmt * 4));
  w.mt_row0 = reinterpret_cast<int32_t*>(take((size_t)mmt * 4));
  w.mt_rows = reinterpret_cast<int32_t*>(take((size_t)mmt * 4));
  w.act = reinterpret_cast<uint16_t*>(take(TK * I * 2 * 2));  // hi and lo planes
  w.xinv = reinterpret_cast<float*>(take((size_t)T * 4));
  if (need_y) {
    w.y32 = reinterpret_cast<float*>(take(TK * H * 4));
    w.xpp = reinterpret_cast<uint16_t*>(take((size_t)T * H * 2 * 2));  // hi and lo planes
  }
  if (Is > 0) {
    w.shared_out = reinterpret_cast<float*>(take((size_t)T * H * 4));
    w.shared_act = reinterpret_cast<uint16_t*>(take((size_t)T * Is * 4));  // two fp16 planes (decode)
  }
  *total = off;
  return w;
}

// GEMV decode kernels: up to 8 tokens, 128 assignments, hidden <= 4096 (two x chunks per lane).
bool is_decode(int T, int K, int H) { return T <= DEC_MAX_TOKENS && T * K <= DEC_STAGE2_ASSIGN && H <= 4096; }

Work layer_work(const kmoe_layer* L, char* base, int T, size_t* total) {
  const LayerArgs& a = L->cfg.args;
  return carve(base, T, L->cfg.top_k, a.E, a.H, a.I, a.sh_gate ? a.Is : 0, !is_decode(T, L->cfg.top_k, L->cfg.args.H), total);
}

int check_qproj(const kmoe_qproj& q, const char* name, int rows, int in, int bits, int E) {
  if (!q.weight || !q.scales || !q.biases) return fail(KMOE_ERR_INVALID_ARG, "%s: null pointer", name);
  const int64_t wbytes = (int64_t)rows * in * bits / 8;
  const int64_t sbytes = (int64_t)rows * (in / 64) * 2;
  const size_t walign = bits == 4 ? 16 : 4;
  if (!aligned(q.weight, walign) || q.weight_expert_stride % (int64_t)walign)
    return fail(KMOE_ERR_ALIGNMENT, "%s.weight must be %zu-byte aligned (pointer and expert stride)", name, walign);
  if (!aligned(q.scales, 2) || !aligned(q.biases, 2) || q.scale_expert_stride % 2)
    return fail(KMOE_ERR_ALIGNMENT, "%s scales/biases must be 2-byte aligned", name);
  if (E > 1 && (q.weight_expert_stride < wbytes || q.scale_expert_stride < sbytes))
    return fail(KMOE_ERR_INVALID_ARG, "%s: expert stride smaller than one expert's tensor", name);
  if (q.weight_expert_stride < 0 || q.scale_expert_stride < 0)
    return fail(KMOE_ERR_INVALID_ARG, "%s: negative expert stride", name);
  return KMOE_OK;
}

}  // namespace

extern "C" {

int kmoe_version(void) { return 100; }

const char* kmoe_strerror(int status) {
  switch (status) {
    case KMOE_OK: return "ok";
    case KMOE_ERR_INVALID_ARG: return "invalid argument";
    case KMOE_ERR_UNSUPPORTED: return "unsupported configuration";
    case KMOE_ERR_ALIGNMENT: return "misaligned pointer or stride";
    case KMOE_ERR_WORKSPACE: return "workspace too small";
    case KMOE_ERR_HIP: return "HIP runtime error";
    case KMOE_ERR_IO: return "I/O error";
    case KMOE_ERR_FORMAT: return "bad file format";
    case KMOE_ERR_DEVICE: return "device-side check failed";
    case KMOE_ERR_NO_MEMORY: return "out of memory";
    default: return "unknown status";
  }
}

const char* kmoe_last_error(void) { return g_last_error.c_str(); }

// Validates a layer description and fills `cfg` from it (the prefill copy fields aside).
static int config_from_desc(const kmoe_layer_desc* d, LayerConfig* cfg) {
  if (d->bits != 3 && d->bits != 4) return fail(KMOE_ERR_UNSUPPORTED, "bits must be 3 or 4 (got %d)", d->bits);
  if (d->group_size != 64) return fail(KMOE_ERR_UNSUPPORTED, "group_size must be 64 (got %d)", d->group_size);
  if (d->hidden <= 0 || d->hidden % 64 || d->hidden > 65536)
    return fail(KMOE_ERR_UNSUPPORTED, "hidden must be a positive multiple of 64 up to 65536 (got %d)", d->hidden);
  if (d->intermediate <= 0 || d->intermediate % 64 || d->intermediate > 65536)
    return fail(KMOE_ERR_UNSUPPORTED, "intermediate must be a positive multiple of 64 (got %d)", d->intermediate);
  if (d->num_experts < 1 || d->num_experts > 1024)
    return fail(KMOE_ERR_UNSUPPORTED, "num_experts must be in [1, 1024] (got %d)", d->num_experts);
  if (d->top_k < 1 || d->top_k > 16 || d->top_k > d->num_experts)
    return fail(KMOE_ERR_INVALID_ARG, "top_k must be in [1, min(16, num_experts)] (got %d)", d->top_k);
  if (d->scale_dtype != KMOE_SCALE_F16 && d->scale_dtype != KMOE_SCALE_BF16)
    return fail(KMOE_ERR_INVALID_ARG, "unknown scale_dtype %d", d->scale_dtype);
  if (d->activation != KMOE_ACT_SWIGLU && d->activation != KMOE_ACT_GELU_TANH)
    return fail(KMOE_ERR_INVALID_ARG, "unknown activation %d", d->activation);
  // decode stage-1 LDS: 8 tokens x H fp16 + chunk sums must fit in 160 KiB
  if ((size_t)8 * (d->hidden / 32) * 68 > 160 * 1024)
    return fail(KMOE_ERR_UNSUPPORTED, "hidden %d too large for the decode kernels", d->hidden);
  int rc;
  if ((rc = check_qproj(d->gate, "gate", d->intermediate, d->hidden, d->bits, d->num_experts))) return rc;
  if ((rc = check_qproj(d->up, "up", d->intermediate, d->hidden, d->bits, d->num_experts))) return rc;
  if ((rc = check_qproj(d->down, "down", d->hidden, d->intermediate, d->bits, d->num_experts))) return rc;
  const bool any_shared = d->shared_gate || d->shared_up || d->shared_down;
  if (any_shared) {
    if (!d->shared_gate || !d->shared_up || !d->shared_down)
      return fail(KMOE_ERR_INVALID_ARG, "shared expert needs gate, up and down pointers");
    if (d->shared_intermediate <= 0 || d->shared_intermediate % 64)
      return fail(KMOE_ERR_INVALID_ARG, "shared_intermediate must be a positive multiple of 64");
    if (!aligned(d->shared_gate, 16) || !aligned(d->shared_up, 16) || !aligned(d->shared_down, 16))
      return fail(KMOE_ERR_ALIGNMENT, "shared expert weights must be 16-byte aligned");
  }
  LayerArgs& a = cfg->args;
  a = LayerArgs{};
  auto qp = [](const kmoe_qproj& q) {
    return QProj{static_cast<const uint8_t*>(q.weight), static_cast<const uint16_t*>(q.scales),
                 static_cast<const uint16_t*>(q.biases), q.weight_expert_stride, q.scale_expert_stride / 2};
  };
  a.gate = qp(d->gate);
  a.up = qp(d->up);
  a.down = qp(d->down);
  a.sh_gate = static_cast<const uint16_t*>(d->shared_gate);
  a.sh_up = static_cast<const uint16_t*>(d->shared_up);
  a.sh_down = static_cast<const uint16_t*>(d->shared_down);
  a.H = d->hidden;
  a.I = d->intermediate;
  a.E = d->num_experts;
  a.Is = any_shared ? d->shared_intermediate : 0;
  cfg->top_k = d->top_k;
  cfg->bits = d->bits;
  cfg->bf16_scales = d->scale_dtype == KMOE_SCALE_BF16;
  cfg->act = d->activation;
  return KMOE_OK;
}

int kmoe_layer_create(const kmoe_layer_desc* d, kmoe_layer** out) {
  if (!d || !out) return fail(KMOE_ERR_INVALID_ARG, "null descriptor or output pointer");
  *out = nullptr;
  LayerConfig cfg{};
  int rc;
  if ((rc = config_from_desc(d, &cfg))) return rc;
  if (d->prefill_pack) {
    const PackLayout pl = pack_layout(cfg.args.H, cfg.args.I, cfg.args.E, cfg.bits);
    if (!aligned(d->prefill_pack, 256)) return fail(KMOE_ERR_ALIGNMENT, "prefill_pack must be 256-byte aligned");
    if (d->prefill_pack_bytes < pl.total)
      return fail(KMOE_ERR_INVALID_ARG, "prefill_pack_bytes %lld below the %lld bytes of the copy",
                  (long long)d->prefill_pack_bytes, (long long)pl.total);
    const uint8_t* base = static_cast<const uint8_t*>(d->prefill_pack);
    for (int q = 0; q < 3; ++q)
      cfg.args.pk[q] = PackProj{base + pl.codes[q], base + pl.sb[q], pl.codes_expert[q], pl.sb_expert[q]};
  }
  kmoe_layer* L = new (std::nothrow) kmoe_layer;
  if (!L) return fail(KMOE_ERR_NO_MEMORY, "out of host memory");
  L->cfg = cfg;
  *out = L;
  return ok();
}

int kmoe_prefill_pack_size(const kmoe_layer_desc* d, size_t* bytes) {
  if (!d || !bytes) return fail(KMOE_ERR_INVALID_ARG, "null descriptor or output pointer");
  LayerConfig cfg{};
  int rc;
  if ((rc = config_from_desc(d, &cfg))) return rc;
  *bytes = (size_t)pack_layout(cfg.args.H, cfg.args.I, cfg.args.E, cfg.bits).total;
  return ok();
}

int kmoe_prefill_pack(const kmoe_layer_desc* d, void* pack, size_t bytes, void* stream) {
  if (!d || !pack) return fail(KMOE_ERR_INVALID_ARG, "null descriptor or pack pointer");
  LayerConfig cfg{};
  int rc;
  if ((rc = config_from_desc(d, &cfg))) return rc;
  const PackLayout pl = pack_layout(cfg.args.H, cfg.args.I, cfg.args.E, cfg.bits);
  if (!aligned(pack, 256)) return fail(KMOE_ERR_ALIGNMENT, "pack must be 256-byte aligned");
  if (bytes < (size_t)pl.total)
    return fail(KMOE_ERR_INVALID_ARG, "pack holds %zu bytes, the copy needs %lld", bytes, (long long)pl.total);
  const hipError_t e = launch_prefill_pack(cfg, static_cast<uint8_t*>(pack), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "prefill pack launch");
}

int kmoe_layer_destroy(kmoe_layer* layer) {
  delete layer;
  return ok();
}

int kmoe_workspace_size(const kmoe_layer* layer, int32_t max_tokens, size_t* bytes) {
  if (!layer || !bytes) return fail(KMOE_ERR_INVALID_ARG, "null layer or output pointer");
  if (max_tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "max_tokens must be >= 0");
  size_t total = 0, t2 = 0;
  layer_work(layer, nullptr, max_tokens, &total);
  // a call with fewer tokens may take the other path; size for both
  if (max_tokens > 0) {
    const int t_small = max_tokens < DEC_MAX_TOKENS ? max_tokens : DEC_MAX_TOKENS;
    layer_work(layer, nullptr, t_small, &t2);
    const LayerArgs& a = layer->cfg.args;
    size_t t3 = 0;
    carve(nullptr, max_tokens, layer->cfg.top_k, a.E, a.H, a.I, a.sh_gate ? a.Is : 0, true, &t3);
    total = total > t3 ? total : t3;
  }
  *bytes = total > t2 ? total : t2;
  return ok();
}

int kmoe_route(const float* logits, int32_t tokens, int32_t num_experts, int32_t top_k, int32_t* idx, float* weights,
               void* stream) {
  if (tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "tokens must be >= 0");
  if (num_experts < 1 || num_experts > 1024) return fail(KMOE_ERR_UNSUPPORTED, "num_experts must be in [1, 1024]");
  if (top_k < 1 || top_k > 16 || top_k > num_experts)
    return fail(KMOE_ERR_INVALID_ARG, "top_k must be in [1, min(16, num_experts)]");
  if (tokens == 0) return ok();
  if (!logits || !idx || !weights) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(logits, 4) || !aligned(idx, 4) || !aligned(weights, 4))
    return fail(KMOE_ERR_ALIGNMENT, "logits/idx/weights must be 4-byte aligned");
  hipError_t e = launch_route(logits, tokens, num_experts, top_k, idx, weights, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "route launch");
}

int kmoe_permute_workspace_size(int32_t tokens, int32_t top_k, int32_t num_experts, size_t* bytes) {
  if (!bytes || tokens < 0 || top_k < 1 || num_experts < 1 || num_experts > 1024)
    return fail(KMOE_ERR_INVALID_ARG, "bad permutation size arguments");
  size_t total = 0;
  carve(nullptr, tokens, top_k, num_experts, 0, 0, 0, false, &total);
  *bytes = total;
  return ok();
}

int kmoe_permute(const int32_t* idx, int32_t tokens, int32_t top_k, int32_t num_experts, int32_t* perm,
                 int32_t* counts, int32_t* offsets, int32_t* unique, int32_t* num_unique, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (tokens < 0 || top_k < 1 || top_k > 16 || num_experts < 1 || num_experts > 1024)
    return fail(KMOE_ERR_INVALID_ARG, "bad permutation size arguments");
  if (!counts || !offsets || !unique || !num_unique || !workspace)
    return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (tokens > 0 && (!idx || !perm)) return fail(KMOE_ERR_INVALID_ARG, "null idx or perm");
  size_t need = 0;
  Work w = carve(static_cast<char*>(workspace), tokens, top_k, num_experts, 0, 0, 0, false, &need);
  if (workspace_bytes < need)
    return fail(KMOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  w.perm = perm;
  w.counts = counts;
  w.offsets = offsets;
  w.unique = unique;
  const int TK = tokens * top_k;
  hipError_t e;
  if (TK == 0) {
    e = hipMemsetAsync(counts, 0, (size_t)num_experts * 4, s);
    if (e == hipSuccess) e = hipMemsetAsync(offsets, 0, (size_t)(num_experts + 1) * 4, s);
    if (e == hipSuccess) e = hipMemsetAsync(num_unique, 0, 4, s);
    return e == hipSuccess ? ok() : hip_fail(e, "permute (empty)");
  }
  e = launch_permute(idx, TK, top_k, num_experts, w, max_mtiles_for(TK, num_experts, GEMM_BM), GEMM_BM, s);
  if (e == hipSuccess) e = hipMemcpyAsync(num_unique, w.scalars, 4, hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? ok() : hip_fail(e, "permute launch");
}

int kmoe_expert_mlp(const kmoe_layer* layer, const void* x, const int32_t* idx, int32_t tokens, void* y,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return kmoe_expert_mlp_x(layer, x, KMOE_X_F16, idx, tokens, y, workspace, workspace_bytes, stream);
}

int kmoe_expert_mlp_x(const kmoe_layer* layer, const void* x, int32_t x_dtype, const int32_t* idx, int32_t tokens,
                      void* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (!layer) return fail(KMOE_ERR_INVALID_ARG, "null layer");
  if (x_dtype < KMOE_X_F16 || x_dtype > KMOE_X_F32) return fail(KMOE_ERR_INVALID_ARG, "unknown x_dtype %d", x_dtype);
  if (tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "tokens must be >= 0");
  if (tokens == 0) return ok();
  if (!x || !idx || !y || !workspace) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(x, 16) || !aligned(y, 16) || !aligned(idx, 4))
    return fail(KMOE_ERR_ALIGNMENT, "x and y must be 16-byte aligned, idx 4-byte aligned");
  size_t need = 0;
  Work w = layer_work(layer, static_cast<char*>(workspace), tokens, &need);
  if (workspace_bytes < need) return fail(KMOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const LayerConfig& c = layer->cfg;
  const int K = c.top_k;
  uint16_t* yy = static_cast<uint16_t*>(y);
  hipError_t e;
  if (is_decode(tokens, K, c.args.H)) {
    DecodeCall d{x, nullptr, idx, tokens, nullptr, nullptr, nullptr, &w, yy, 0, false, nullptr, x_dtype};
    e = launch_decode(c, d, s);
  } else {
    const int bm = gemm_bm(c.args, x_dtype, tokens * K), mmt = max_mtiles_for(tokens * K, c.args.E, bm);
    e = launch_permute(idx, tokens * K, K, c.args.E, w, mmt, bm, s);
    if (e == hipSuccess) e = launch_xpair(c, x, x_dtype, tokens, w.xpp, w.xinv, s);
    if (e == hipSuccess)
      e = launch_gemm(c, w.xpp, tokens, w, mmt, yy, nullptr, s, x_dtype, x_dtype == KMOE_X_F16 ? nullptr : w.xinv);
    if (e == hipSuccess) e = launch_zero_bad_rows(idx, tokens * K, c.args.E, c.args.H, yy, s);
  }
  return e == hipSuccess ? ok() : hip_fail(e, "expert_mlp launch");
}

int kmoe_combine(const void* y, const float* weights, int32_t tokens, int32_t top_k, int32_t hidden, void* out,
                 void* stream) {
  if (tokens < 0 || top_k < 1 || top_k > 16 || hidden <= 0 || hidden % 64)
    return fail(KMOE_ERR_INVALID_ARG, "bad combine sizes");
  if (tokens == 0) return ok();
  if (!y || !weights || !out) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(y, 8) || !aligned(out, 8) || !aligned(weights, 4))
    return fail(KMOE_ERR_ALIGNMENT, "y/out must be 8-byte aligned, weights 4-byte aligned");
  hipError_t e = launch_combine(nullptr, static_cast<const uint16_t*>(y), weights, tokens, top_k, hidden, nullptr,
                                out, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "combine launch");
}

int kmoe_forward(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens, void* out,
                 int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace, size_t workspace_bytes,
                 void* stream) {
  return kmoe::forward_impl(layer, x, logits, tokens, out, out_dtype, idx_out, weights_out, workspace,
                            workspace_bytes, stream);
}

int kmoe_forward_x(const kmoe_layer* layer, const void* x, int32_t x_dtype, const float* logits, int32_t tokens,
                   void* out, int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (x_dtype < KMOE_X_F16 || x_dtype > KMOE_X_F32) return fail(KMOE_ERR_INVALID_ARG, "unknown x_dtype %d", x_dtype);
  return kmoe::forward_impl(layer, x, logits, tokens, out, out_dtype, idx_out, weights_out, workspace,
                            workspace_bytes, stream, nullptr, x_dtype);
}

}  // extern "C"

// The routed layer on a caller-provided workspace (kmoe_forward, and kmoe_forward_noalloc with the
// library's static scratch).
int kmoe::forward_impl(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens, void* out,
                       int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace,
                       size_t workspace_bytes, void* stream, const float* extra, int xdt, const Blend* blend,
                       const QDown* qd) {
  if (!layer) return fail(KMOE_ERR_INVALID_ARG, "null layer");
  if (tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "tokens must be >= 0");
  if (out_dtype != KMOE_OUT_F16 && out_dtype != KMOE_OUT_F32) return fail(KMOE_ERR_INVALID_ARG, "unknown out_dtype");
  const int out32 = out_dtype == KMOE_OUT_F32;
  if (tokens == 0) return ok();
  if (!x || !logits || !out || !workspace) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(logits, 4))
    return fail(KMOE_ERR_ALIGNMENT, "x and out must be 16-byte aligned, logits 4-byte aligned");
  if ((idx_out && !aligned(idx_out, 4)) || (weights_out && !aligned(weights_out, 4)))
    return fail(KMOE_ERR_ALIGNMENT, "idx_out/weights_out must be 4-byte aligned");
  size_t need = 0;
  Work w = layer_work(layer, static_cast<char*>(workspace), tokens, &need);
  if (workspace_bytes < need) return fail(KMOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const LayerConfig& c = layer->cfg;
  const LayerArgs& a = c.args;
  const int K = c.top_k;
  if (a.sh_gate && xdt != KMOE_X_F16)
    return fail(KMOE_ERR_UNSUPPORTED, "the dense shared expert takes fp16 activations only");
  if (idx_out) w.idx = idx_out;
  if (weights_out) w.wts = weights_out;
  hipError_t e = hipSuccess;
  const bool decode = is_decode(tokens, K, a.H);
  // decode runs the dense shared expert inside its two stages
  if (a.sh_gate && !decode) e = launch_shared(c, static_cast<const uint16_t*>(x), tokens, w, s);
  if (e != hipSuccess) return hip_fail(e, "shared expert launch");
  if (decode) {
    DecodeCall d{x, logits, nullptr, tokens, w.idx, w.wts, w.wts, &w, out, out32, true, extra, xdt};
    if (blend) d.blend = *blend;
    d.qd = qd;
    e = launch_decode(c, d, s);
  } else {
    const int bm = gemm_bm(a, xdt, tokens * K), mmt = max_mtiles_for(tokens * K, a.E, bm);
    e = launch_route_xpair(logits, tokens, a.E, K, w.idx, w.wts, x, xdt, a.H, c.bits, w.xpp, w.xinv, s);
    if (e == hipSuccess) e = launch_permute(w.idx, tokens * K, K, a.E, w, mmt, bm, s);
    if (e == hipSuccess)
      e = launch_gemm(c, w.xpp, tokens, w, mmt, nullptr, w.wts, s, xdt, xdt == KMOE_X_F16 ? nullptr : w.xinv);
    if (e == hipSuccess)
      e = launch_combine(w.y32, nullptr, nullptr, tokens, K, a.H, extra ? extra : a.sh_gate ? w.shared_out : nullptr,
                         out, out32, s);
  }
  return e == hipSuccess ? ok() : hip_fail(e, "forward launch");
}

int kmoe::workspace_bytes_for(const kmoe_layer* layer, int32_t tokens, size_t* bytes) {
  return kmoe_workspace_size(layer, tokens, bytes);
}

int kmoe::report_error(int code, const char* msg) { return fail(code, "%s", msg); }

extern "C" {

int kmoe_dequantize(const kmoe_layer* layer, int32_t proj, int32_t expert, int32_t row0, int32_t nrows,
                    uint8_t* codes, uint16_t* weights_f16, void* stream) {
  if (!layer || !codes || !weights_f16) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (proj < 0 || proj > 2) return fail(KMOE_ERR_INVALID_ARG, "proj must be 0 (gate), 1 (up) or 2 (down)");
  const LayerArgs& a = layer->cfg.args;
  const int rows = proj == 2 ? a.H : a.I;
  if (expert < 0 || expert >= a.E) return fail(KMOE_ERR_INVALID_ARG, "expert %d out of range", expert);
  if (row0 < 0 || nrows < 0 || row0 + nrows > rows) return fail(KMOE_ERR_INVALID_ARG, "row range out of bounds");
  hipError_t e = launch_dequantize(layer->cfg, proj, expert, row0, nrows, codes, weights_f16,
                                   static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "dequantize launch");
}

int kmoe_device_status(void* workspace, size_t workspace_bytes, int32_t* flags, void* stream) {
  if (!workspace || !flags || workspace_bytes < 256) return fail(KMOE_ERR_INVALID_ARG, "bad workspace or flags");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* sc = static_cast<int32_t*>(workspace);
  hipError_t e = hipMemcpyAsync(flags, sc + 2, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e == hipSuccess) e = hipMemsetAsync(sc + 2, 0, 4, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return e == hipSuccess ? ok() : hip_fail(e, "device status");
}

int kmoe_profile_begin(int32_t max_launches) {
  if (max_launches < 1 || max_launches > 16384) return fail(KMOE_ERR_INVALID_ARG, "max_launches must be 1..16384");
  if (prof_on()) return fail(KMOE_ERR_INVALID_ARG, "kernel timing already on for this thread");
  prof_reset();
  Prof& p = prof();
  p.events.resize(2 * (size_t)max_launches, nullptr);
  for (auto& ev : p.events) {
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) {
      ev = nullptr;
      prof_reset();
      return hip_fail(e, "hipEventCreate");
    }
  }
  p.recs.reserve((size_t)max_launches);
  p.on = true;
  return ok();
}

int kmoe_profile_end(kmoe_kernel_time* entries, int32_t max_entries, int32_t* n_entries) {
  if (!prof_on()) return fail(KMOE_ERR_INVALID_ARG, "kernel timing is not on for this thread");
  if (!n_entries || max_entries < 0 || (max_entries > 0 && !entries)) {
    prof_reset();
    return fail(KMOE_ERR_INVALID_ARG, "bad output arguments");
  }
  Prof& p = prof();
  std::vector<kmoe_kernel_time> agg;
  hipError_t err = p.failed;
  for (const ProfRec& r : p.recs) {
    if (err != hipSuccess) break;
    float ms = 0.f;
    err = hipEventSynchronize(r.e1);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, r.e0, r.e1);
    if (err != hipSuccess) break;
    kmoe_kernel_time* t = nullptr;
    for (auto& a : agg)
      if (std::strncmp(a.name, r.name, sizeof a.name) == 0) t = &a;
    if (!t) {
      kmoe_kernel_time z{};
      std::snprintf(z.name, sizeof z.name, "%s", r.name);
      z.min_ms = 1e30;
      agg.push_back(z);
      t = &agg.back();
    }
    t->launches += 1;
    t->total_ms += ms;
    t->min_ms = ms < t->min_ms ? ms : t->min_ms;
    t->max_ms = ms > t->max_ms ? ms : t->max_ms;
  }
  prof_reset();
  if (err != hipSuccess) return hip_fail(err, "kernel timing events");
  *n_entries = (int32_t)agg.size();
  for (int32_t i = 0; i < (int32_t)agg.size() && i < max_entries; ++i) entries[i] = agg[i];
  return ok();
}

}  // extern "C"

// ---- TQ3 codebook experts ------------------------------------------------------------------
extern "C" {

int kmoe_tq3_gemv(const void* blocks, int32_t rows, int32_t cols, const void* x, int32_t x_f32, int32_t tokens,
                  float* out, void* stream) {
  if (rows < 0 || tokens < 0 || cols <= 0 || cols % 32 || cols > 4096)
    return fail(KMOE_ERR_INVALID_ARG, "rows/tokens must be >= 0 and cols a multiple of 32 up to 4096");
  if (rows == 0 || tokens == 0) return ok();
  if (!blocks || !x || !out) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(blocks, 4) || !aligned(x, 16) || !aligned(out, 4))
    return fail(KMOE_ERR_ALIGNMENT, "blocks and out must be 4-byte aligned, x 16-byte aligned");
  Tq3Params p{static_cast<const uint8_t*>(blocks), 0, 0, nullptr, 1, x, 1, tokens, rows, cols, out, nullptr};
  hipError_t e = launch_tq3_gemv(p, x_f32 != 0, false, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "tq3 gemv launch");
}

int kmoe_tq3_workspace_size(int32_t tokens, int32_t top_k, int32_t intermediate, size_t* bytes) {
  if (!bytes || tokens < 0 || top_k < 1 || intermediate <= 0) return fail(KMOE_ERR_INVALID_ARG, "bad sizes");
  *bytes = up256((size_t)tokens * top_k * intermediate * sizeof(float));
  return ok();
}

int kmoe_tq3_expert_mlp(const void* experts, int64_t expert_bytes, int32_t num_experts, int32_t hidden,
                        int32_t intermediate, const void* x, const int32_t* idx, int32_t tokens, int32_t top_k, void* y,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (num_experts < 1 || top_k < 1 || tokens < 0 || hidden <= 0 || intermediate <= 0 || hidden % 32 ||
      intermediate % 32 || hidden > 4096 || intermediate > 4096)
    return fail(KMOE_ERR_INVALID_ARG, "hidden/intermediate must be multiples of 32 up to 4096; E, K >= 1");
  const int64_t mat = (int64_t)hidden * intermediate / 32 * 20;
  if (expert_bytes < 3 * mat) return fail(KMOE_ERR_INVALID_ARG, "expert_bytes below the three TQ3 matrices");
  if (tokens == 0) return ok();
  if (!experts || !x || !idx || !y || !workspace) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(experts, 4) || expert_bytes % 4 || !aligned(x, 16) || !aligned(y, 4) || !aligned(idx, 4) ||
      !aligned(workspace, 16))
    return fail(KMOE_ERR_ALIGNMENT, "experts/expert_bytes/y/idx 4-byte aligned, x and workspace 16-byte aligned");
  size_t need = 0;
  kmoe_tq3_workspace_size(tokens, top_k, intermediate, &need);
  if (workspace_bytes < need) return fail(KMOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int V = tokens * top_k;
  float* act = static_cast<float*>(workspace);
  const uint8_t* w = static_cast<const uint8_t*>(experts);
  // gate/up pairs with the SwiGLU output act [V][I] fp32, then down to fp16 y [V][H]
  Tq3Params a{w, expert_bytes, mat, idx, num_experts, x, top_k, V, intermediate, hidden, act, nullptr};
  hipError_t e = launch_tq3_gemv(a, false, true, s);
  Tq3Params d{w + 2 * mat, expert_bytes, 0, idx, num_experts, act, 1, V, hidden, intermediate, nullptr,
              static_cast<uint16_t*>(y)};
  if (e == hipSuccess) e = launch_tq3_gemv(d, true, false, s);
  return e == hipSuccess ? ok() : hip_fail(e, "tq3 expert mlp launch");
}

}  // extern "C"

// ---- the MoE block around the routed experts ------------------------------------------------
struct kmoe_block {
  const kmoe_layer* routed;
  LayerConfig shared;  // one-expert layer of the quantized shared expert (when has_shared)
  QProj router, sgate;
  int bits, bf16, has_shared, gated;
};

namespace {

struct BlockWork {
  char* routed;
  size_t routed_bytes;
  Work sh;           // the shared layer's carve
  float* logits;     // [T][E]
  float* gate;       // [T]
  int32_t* idx0;     // [T] zeros
  uint16_t* ysh;     // [T][H] fp16 shared-expert output
  float* extra;      // [T][H] residual + gated shared term
};

// Carve a block workspace for T tokens (base == nullptr: size only).
BlockWork block_carve(const kmoe_block* b, char* base, int T, size_t* total) {
  BlockWork w{};
  const LayerArgs& ra = b->routed->cfg.args;
  size_t routed = 0;
  kmoe_workspace_size(b->routed, T, &routed);
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += up256(bytes);
    return p;
  };
  w.routed = take(routed);
  w.routed_bytes = routed;
  if (b->has_shared) {
    const LayerArgs& sa = b->shared.args;
    size_t s1 = 0, s2 = 0;
    carve(nullptr, T, 1, 1, sa.H, sa.I, 0, false, &s1);
    carve(nullptr, T, 1, 1, sa.H, sa.I, 0, true, &s2);
    char* shb = take(s1 > s2 ? s1 : s2);
    size_t dummy = 0;
    w.sh = carve(shb, T, 1, 1, sa.H, sa.I, 0, !is_decode(T, 1, sa.H), &dummy);
  }
  w.logits = reinterpret_cast<float*>(take((size_t)T * ra.E * 4));
  w.gate = reinterpret_cast<float*>(take((size_t)T * 4));
  w.idx0 = reinterpret_cast<int32_t*>(take((size_t)T * 4));
  w.ysh = reinterpret_cast<uint16_t*>(take((size_t)T * ra.H * 2));
  w.extra = reinterpret_cast<float*>(take((size_t)T * ra.H * 4));
  *total = off;
  return w;
}

}  // namespace

extern "C" {

int kmoe_block_create(const kmoe_block_desc* d, kmoe_block** out) {
  if (!d || !out || !d->routed) return fail(KMOE_ERR_INVALID_ARG, "null descriptor, output pointer or routed layer");
  *out = nullptr;
  const LayerArgs& ra = d->routed->cfg.args;
  if (ra.sh_gate) return fail(KMOE_ERR_INVALID_ARG, "the routed layer of a block must not carry a dense shared expert");
  if (d->bits != 3 && d->bits != 4) return fail(KMOE_ERR_UNSUPPORTED, "block bits must be 3 or 4 (got %d)", d->bits);
  if (d->scale_dtype != KMOE_SCALE_F16 && d->scale_dtype != KMOE_SCALE_BF16)
    return fail(KMOE_ERR_INVALID_ARG, "unknown scale_dtype %d", d->scale_dtype);
  int rc;
  kmoe_qproj r = d->router;
  r.weight_expert_stride = r.scale_expert_stride = 0;
  if ((rc = check_qproj(r, "router", ra.E, ra.H, d->bits, 1))) return rc;
  kmoe_block tmp{};
  tmp.routed = d->routed;
  tmp.bits = d->bits;
  tmp.bf16 = d->scale_dtype == KMOE_SCALE_BF16;
  auto qp = [](const kmoe_qproj& q) {
    return QProj{static_cast<const uint8_t*>(q.weight), static_cast<const uint16_t*>(q.scales),
                 static_cast<const uint16_t*>(q.biases), 0, 0};
  };
  tmp.router = qp(r);
  tmp.gated = d->shared_expert_gate.weight != nullptr;
  if (tmp.gated) {
    kmoe_qproj g = d->shared_expert_gate;
    g.weight_expert_stride = g.scale_expert_stride = 0;
    if ((rc = check_qproj(g, "shared_expert_gate", 1, ra.H, d->bits, 1))) return rc;
    tmp.sgate = qp(g);
  }
  tmp.has_shared = d->shared_gate_proj.weight != nullptr;
  if (tmp.has_shared) {
    kmoe_layer_desc sd{};
    sd.hidden = ra.H;
    sd.intermediate = d->shared_intermediate;
    sd.num_experts = 1;
    sd.top_k = 1;
    sd.bits = d->bits;
    sd.group_size = 64;
    sd.scale_dtype = d->scale_dtype;
    sd.activation = KMOE_ACT_SWIGLU;
    sd.gate = d->shared_gate_proj;
    sd.up = d->shared_up_proj;
    sd.down = d->shared_down_proj;
    if ((rc = config_from_desc(&sd, &tmp.shared))) return rc;
  } else if (tmp.gated) {
    return fail(KMOE_ERR_INVALID_ARG, "a shared expert gate needs a shared expert");
  }
  kmoe_block* b = new (std::nothrow) kmoe_block(tmp);
  if (!b) return fail(KMOE_ERR_NO_MEMORY, "out of host memory");
  *out = b;
  return ok();
}

int kmoe_block_destroy(kmoe_block* block) {
  delete block;
  return ok();
}

int kmoe_block_workspace_size(const kmoe_block* block, int32_t max_tokens, size_t* bytes) {
  if (!block || !bytes) return fail(KMOE_ERR_INVALID_ARG, "null block or output pointer");
  if (max_tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "max_tokens must be >= 0");
  size_t a = 0, b = 0;
  block_carve(block, nullptr, max_tokens, &a);
  block_carve(block, nullptr, max_tokens < DEC_MAX_TOKENS ? max_tokens : DEC_MAX_TOKENS, &b);
  *bytes = a > b ? a : b;
  return ok();
}

int kmoe_block_forward(const kmoe_block* block, const void* x, const void* residual, int32_t tokens, void* out,
                       int32_t out_dtype, int32_t* idx_out, float* weights_out, float* logits_out, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (!block) return fail(KMOE_ERR_INVALID_ARG, "null block");
  if (tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "tokens must be >= 0");
  if (out_dtype != KMOE_OUT_F16 && out_dtype != KMOE_OUT_F32) return fail(KMOE_ERR_INVALID_ARG, "unknown out_dtype");
  if (tokens == 0) return ok();
  if (!x || !out || !workspace) return fail(KMOE_ERR_INVALID_ARG, "null pointer");
  if (!aligned(x, 16) || !aligned(out, 16) || (residual && !aligned(residual, 16)))
    return fail(KMOE_ERR_ALIGNMENT, "x, residual and out must be 16-byte aligned");
  if (logits_out && !aligned(logits_out, 4)) return fail(KMOE_ERR_ALIGNMENT, "logits_out must be 4-byte aligned");
  size_t need = 0;
  BlockWork w = block_carve(block, static_cast<char*>(workspace), tokens, &need);
  if (workspace_bytes < need) return fail(KMOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const LayerArgs& ra = block->routed->cfg.args;
  const uint16_t* xx = static_cast<const uint16_t*>(x);
  float* logits = logits_out ? logits_out : w.logits;
  // In decode the router projection rides along the shared layer's stage 1 as extra workgroups
  // (same bits and scale dtype); otherwise it is a launch of its own.
  const bool ql_ride = block->has_shared && is_decode(tokens, 1, ra.H) && block->shared.bits == block->bits &&
                       (block->shared.bf16_scales != 0) == (block->bf16 != 0);
  // ... and the shared expert's down rows ride along the routed layer's stage 1 (its stage-1 act
  // being ready by then), so decode makes three launches
  const bool qd_ride = ql_ride && is_decode(tokens, block->routed->cfg.top_k, ra.H);
  QDown qd;
  if (qd_ride) {
    qd.d = block->shared.args.down;
    qd.bits = block->shared.bits;
    qd.bf16 = block->shared.bf16_scales;
    qd.I = block->shared.args.I;
    qd.act = w.sh.act;
    qd.plane = (size_t)tokens * block->shared.args.I;
    qd.y = w.ysh;
  }
  QLin ql;
  ql.a = block->router;
  ql.ra = ra.E;
  ql.b = block->sgate;
  ql.rb = block->gated ? 1 : 0;
  ql.out_a = logits;
  ql.out_b = w.gate;
  hipError_t e = hipSuccess;
  if (!ql_ride)
    e = launch_qlinear(block->router, ra.E, block->sgate, block->gated ? 1 : 0, block->bits, block->bf16, xx, tokens,
                       ra.H, logits, w.gate, s);
  if (e == hipSuccess && block->has_shared) {
    const LayerConfig& sc = block->shared;
    // expert index 0 of every token for the one-expert shared layer: the library's constant zeros
    // in decode, else filled into the workspace
    const int32_t* zi = is_decode(tokens, 1, ra.H) ? zero_index() : nullptr;
    if (!zi) e = launch_fill_i32(w.idx0, tokens, 0, s);
    if (e == hipSuccess && is_decode(tokens, 1, ra.H)) {
      DecodeCall d{xx, nullptr, zi ? zi : w.idx0, tokens, nullptr, nullptr, nullptr, &w.sh, w.ysh, 0, false, nullptr};
      if (ql_ride) d.ql = &ql;
      d.stage1_only = qd_ride;  // its down rows ride along the routed layer's stage 1
      e = launch_decode(sc, d, s);
    } else if (e == hipSuccess) {
      const int bm = gemm_bm(sc.args, XDT_F16, tokens), mmt = max_mtiles_for(tokens, 1, bm);
      e = launch_permute(w.idx0, tokens, 1, 1, w.sh, mmt, bm, s);
      if (e == hipSuccess) e = launch_xpair(sc, xx, KMOE_X_F16, tokens, w.sh.xpp, nullptr, s);
      if (e == hipSuccess) e = launch_gemm(sc, w.sh.xpp, tokens, w.sh, mmt, w.ysh, nullptr, s);
    }
  }
  const bool need_extra = block->has_shared || residual;
  // decode adds residual + fp16 shared * sigmoid(gate) inside its combine; prefill's combine adds
  // the fp32 term prepared here
  const bool fused = is_decode(tokens, block->routed->cfg.top_k, ra.H);
  Blend bl;
  if (fused) {
    bl.res = static_cast<const uint16_t*>(residual);
    bl.sh = block->has_shared ? w.ysh : nullptr;
    bl.gate = block->has_shared && block->gated ? w.gate : nullptr;
  } else if (e == hipSuccess && need_extra) {
    e = launch_blend_prep(block->has_shared ? w.ysh : nullptr, block->gated ? w.gate : nullptr,
                          static_cast<const uint16_t*>(residual), tokens, ra.H, w.extra, s);
  }
  if (e != hipSuccess) return hip_fail(e, "block launch");
  return kmoe::forward_impl(block->routed, x, logits, tokens, out, out_dtype, idx_out, weights_out, w.routed,
                            w.routed_bytes, stream, !fused && need_extra ? w.extra : nullptr, KMOE_X_F16, &bl,
                            qd_ride ? &qd : nullptr);
}

}  // extern "C"

namespace kmoe {

void prof_events(const char* kernel_name, hipStream_t s, hipEvent_t* start, hipEvent_t* stop) {
  *start = *stop = nullptr;
  if (!prof_on()) return;
  Prof& p = prof();
  if (p.failed != hipSuccess || p.recs.size() * 2 >= p.events.size()) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  const size_t i = p.recs.size();
  p.recs.push_back(ProfRec{kernel_name, p.events[2 * i], p.events[2 * i + 1]});
  *start = p.events[2 * i];
  *stop = p.events[2 * i + 1];
}

}  // namespace kmoe
