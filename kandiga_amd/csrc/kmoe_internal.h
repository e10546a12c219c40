// Internal host/device interface between the C ABI (capi.cpp) and the kernel files.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kmoe {

// One quantized projection stack: expert e, row r starts at
//   w + e*w_stride + r*(in*bits/8)  and  s/b + e*s_stride + r*(in/64)  (strides in elements / bytes).
struct QProj {
  const uint8_t* w;
  const uint16_t* s;
  const uint16_t* b;
  int64_t w_stride;  // bytes
  int64_t s_stride;  // uint16 elements
};

// One projection of the prefill weight copy (kmoe_prefill_pack): codes of expert e at
// codes + e*codes_expert, laid out [32-row block][group][lane][chunk]; scales and biases at
// sb + e*sb_expert, [32-row block][group pair][row][s0 s1 b0 b1].  Null codes: no copy.
struct PackProj {
  const uint8_t* codes;
  const uint8_t* sb;
  int64_t codes_expert;  // bytes per expert
  int64_t sb_expert;     // bytes per expert
};

// Byte offsets of the six regions of a prefill copy (gate/up/down codes, then gate/up/down
// scale-bias pairs, each 256-byte aligned) and its total size.
struct PackLayout {
  int64_t codes[3], sb[3], codes_expert[3], sb_expert[3], total;
};
PackLayout pack_layout(int H, int I, int E, int bits);

struct LayerArgs {
  QProj gate, up, down;
  PackProj pk[3];  // gate, up, down of the prefill copy (codes null when absent)
  const uint16_t* sh_gate;  // dense fp16 shared expert [Is][H] (or null)
  const uint16_t* sh_up;    // [Is][H]
  const uint16_t* sh_down;  // [H][Is]
  int H, I, E, Is;
};

struct LayerConfig {
  LayerArgs args;
  int top_k;
  int bits;
  int bf16_scales;
  int act;  // 0 SwiGLU, 1 GELU-tanh gate
};

// Workspace carve-up for one call (all pointers device memory, null when unused).
struct Work {
  int32_t* idx;        // [T*K]
  float* wts;          // [T*K]
  int32_t* perm;       // [T*K]   assignment ids sorted by (expert, id)
  int32_t* local_rank; // [T*K]
  int32_t* tile_hist;  // [ntiles][E]
  int32_t* counts;     // [E]
  int32_t* offsets;    // [E+1]
  int32_t* unique;     // [E]
  int32_t* ustart;     // [E+1]   group starts of the unique experts
  int32_t* scalars;    // [0]=num_unique [1]=num GEMM m-tiles [2]=device error flags [4,5]=decode sync
  int32_t* mt_expert;  // [max_mtiles]
  int32_t* mt_row0;    // [max_mtiles]
  int32_t* mt_rows;    // [max_mtiles]
  uint16_t* act;       // 2 planes [T*K][I] fp16 (hi, lo), pair order; rows by assignment
                       // (decode) or by expert-sorted position (grouped GEMM)
  float* y32;          // [T*K][H] fp32 weighted per-assignment outputs (grouped-GEMM path of forward)
  uint16_t* xpp;       // x in pair order (grouped-GEMM path): hi plane [T][H], then the lo plane
                       // (fp32 activations)
  float* xinv;         // [T] 2^-s of each token's activation scaling (bf16 / fp32 activations)
  float* shared_out;     // [T][H] fp32 dense shared-expert output
  uint16_t* shared_act;  // shared-expert SwiGLU output: 2 fp16 planes [T][Is] (decode) or 1 (prefill)
};

constexpr int PERM_TILE = 1024;   // assignments per permutation tile
constexpr int GEMM_BM = 128;      // assignment rows per grouped-GEMM tile (MLX-layout weights)
constexpr int GEMM_BM_PACK = 64;  // rows per tile from the prefill copy at hidden <= 2048: half
                                  // the accumulators, three or four workgroups per CU
constexpr int DEC_MAX_TOKENS = 8; // largest batch served by the GEMV path
constexpr int DEC_STAGE2_ASSIGN = 128; // assignments held in two lane slots by decode stage 2

// Device error flag bits (Work::scalars[2]).
constexpr int DEVERR_BAD_EXPERT = 1;

// Activation dtypes of the C ABI (KMOE_X_*): rows [T][H] of fp16, bf16 or fp32.  bf16 and fp32
// rows are taken per token as fp16 planes of x * 2^s (kmoe_device.h, scaled activations).
constexpr int XDT_F16 = 0, XDT_BF16 = 1, XDT_F32 = 2;

// One decode-path call (1..DEC_MAX_TOKENS tokens): routing from logits, or given indices.
// The MoE block's term after the routed combine, out = routed + (residual + fp16 shared * gate'):
// res [T][H] fp16 or null, sh [T][H] fp16 (the block's shared-expert output) or null, gate [T]
// fp32 pre-sigmoid or null (ungated).  Decode adds it inside its combine.
struct Blend {
  const uint16_t* res = nullptr;
  const uint16_t* sh = nullptr;
  const float* gate = nullptr;
};

// A router projection (qlinear_kernel's work: out_a [T][ra] = A x, out_b [T][rb] = B x) run by
// extra workgroups of a decode stage 1 that takes given indices (the MoE block's shared layer).
struct QLin {
  QProj a, b;
  int ra = 0, rb = 0;
  float* out_a = nullptr;
  float* out_b = nullptr;
};

// The down projection of a one-expert layer (the MoE block's quantized shared expert) run by
// extra workgroups of another layer's decode stage 1: y [T][H] fp16 from act (two fp16 planes
// [T][I], the one-expert layer's stage-1 output in its pair order).
struct QDown {
  QProj d;
  int bits = 0, bf16 = 0, I = 0;
  const uint16_t* act = nullptr;
  size_t plane = 0;
  uint16_t* y = nullptr;
};

struct DecodeCall {
  const void* x;           // [T][H] of dtype xdt
  const float* logits;     // [T][E], or null when idx_in is given
  const int32_t* idx_in;   // [T][K], or null when routing
  int T;
  int32_t* idx_out;        // routing outputs written by stage 1 (routing mode)
  float* w_out;
  const float* wts;        // combine weights read by stage 2 (= w_out in routing mode)
  const Work* w;
  void* out;               // combined [T][H] (combine) or per-assignment y [T*K][H] fp16
  int out32;
  bool combine;
  const float* extra;      // [T][H] fp32 added after the combine (block residual + gated shared
                           // expert), or null: then the layer's dense shared expert output, if any
  int xdt;                 // XDT_* of x
  Blend blend;             // block term added in the combine (decode only)
  const QLin* ql = nullptr; // router projection riding along stage 1 (given-indices mode only)
  const QDown* qd = nullptr;  // one-expert down projection riding along stage 1 (routing mode)
  bool stage1_only = false;   // launch stage 1 only (its act is consumed by a QDown elsewhere)
};

// Kernel timing hook (kmoe_profile_begin/end).  prof_events hands out the next event pair of
// the calling thread's timing session for a launch of `kernel_name` on `s`, or two nulls when
// timing is off or `s` is being captured.  KMOE_LAUNCH passes a pair to hipExtLaunchKernelGGL,
// which stamps the kernel's own start and end into the events; untimed launches are plain.
void prof_events(const char* kernel_name, hipStream_t s, hipEvent_t* start, hipEvent_t* stop);

#define KMOE_LAUNCH(NAME, KERNEL, GRID, BLOCK, SHMEM, STREAM, ...)                                  \
  do {                                                                                             \
    hipEvent_t kmoe_e0_ = nullptr, kmoe_e1_ = nullptr;                                             \
    ::kmoe::prof_events(NAME, STREAM, &kmoe_e0_, &kmoe_e1_);                                       \
    if (kmoe_e0_)                                                                                  \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, kmoe_e0_, kmoe_e1_, 0, __VA_ARGS__); \
    else                                                                                           \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, __VA_ARGS__);                         \
  } while (0)

}  // namespace kmoe

struct kmoe_layer;

namespace kmoe {

// The routed layer (kmoe_forward's body) on the given workspace; the status and last error are
// those of kmoe_forward.
int forward_impl(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens, void* out,
                 int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace, size_t workspace_bytes,
                 void* stream, const float* extra = nullptr, int xdt = XDT_F16, const Blend* blend = nullptr,
                 const QDown* qd = nullptr);
// kmoe_workspace_size for `tokens` tokens of `layer`.
int workspace_bytes_for(const kmoe_layer* layer, int32_t tokens, size_t* bytes);
// Records `msg` as the calling thread's last error and returns `code`.
int report_error(int code, const char* msg);

// ---- launchers (return hipError_t of the launch) ----------------------------------------
hipError_t launch_route(const float* logits, int T, int E, int K, int32_t* idx, float* wts, hipStream_t s);
// launch_route plus xpp = x [T][H] in pair order for `bits`-bit codes (one launch); bf16 / fp32
// rows go in scaled (xinv[t] = 2^-s), fp32 rows as two planes (lo plane at xpp + T*H).
hipError_t launch_route_xpair(const float* logits, int T, int E, int K, int32_t* idx, float* wts, const void* x,
                              int xdt, int H, int bits, uint16_t* xpp, float* xinv, hipStream_t s);
// bm: rows per grouped-GEMM tile of the m-tile list (GEMM_BM, or GEMM_BM_PACK for a layer with
// the prefill copy; launch_gemm must be called for the same layer).
hipError_t launch_permute(const int32_t* idx, int TK, int K, int E, const Work& w, int max_mtiles, int bm,
                          hipStream_t s);
// Tiles of 64 rows pay off with the prefill copy's cheap weight loads, up to a gate/up k loop of
// 2048; past that the 128-row tile's weight reuse wins.  From the MLX layout they pay off for
// batches of at most 8192 assignments (most experts then hold under 64 rows, and the two-plane
// down GEMM runs half the padding; measured at 512 and 1024 tokens, top-8) when both projections hold an
// even number of groups per row.  fp32 activations (two A planes in the gate/up GEMM) always use
// 128-row tiles.  tk = tokens * top_k of the call.
inline int gemm_bm(const LayerArgs& a, int xdt = XDT_F16, int tk = 0) {
  if (xdt == XDT_F32 || a.H > 2048) return GEMM_BM;
  if (a.pk[0].codes) return GEMM_BM_PACK;
  const bool even = a.H % 128 == 0 && a.I % 128 == 0;  // two 64-wide groups per pair
  return even && tk > 0 && tk <= 8192 ? GEMM_BM_PACK : GEMM_BM;
}
hipError_t launch_decode(const LayerConfig& c, const DecodeCall& d, hipStream_t s);
// x [T][H] -> xpp in pair order (per 32-wide chunk), the gate/up GEMM's A layout (bf16 / fp32
// rows scaled and split as for launch_route_xpair).
hipError_t launch_xpair(const LayerConfig& c, const void* x, int xdt, int T, uint16_t* xpp, float* xinv, hipStream_t s);
// Per-assignment outputs: y16 (fp16, unweighted: the switch_mlp contract) or, when y16 is
// null, Work::y32 (fp32, each row scaled by its routing weight in wscale for the combine).
hipError_t launch_gemm(const LayerConfig& c, const uint16_t* x, int T, const Work& w, int max_mtiles,
                       uint16_t* y16, const float* wscale, hipStream_t s, int xdt = XDT_F16,
                       const float* xinv = nullptr);
// y[a] (fp16 [TK][H]) = 0 for every assignment a whose idx[a] lies outside [0, E).
hipError_t launch_zero_bad_rows(const int32_t* idx, int TK, int E, int H, uint16_t* y, hipStream_t s);
// out[t] = sum_k (wts ? wts[t,k] : 1) * y[t,k] (+ shared[t]); y is fp32 (y32) or fp16 bits (y16).
hipError_t launch_combine(const float* y32, const uint16_t* y16, const float* wts, int T, int K, int H,
                          const float* shared, void* out, int out32, hipStream_t s);
hipError_t launch_shared(const LayerConfig& c, const uint16_t* x, int T, const Work& w, hipStream_t s);
// MoE block (block.hip): out_a[t][r] (r < ra) and out_b[t][r] (r < rb) = rows of the quantized
// projections a and b (expert 0 of each, `bits`-bit codes) applied to x [T][H]; fp32.
hipError_t launch_qlinear(const QProj& a, int ra, const QProj& b, int rb, int bits, bool bf16, const uint16_t* x,
                          int T, int H, float* out_a, float* out_b, hipStream_t s);
// extra[t][h] = residual[t][h] + fp16 shared16[t][h] * sigmoid(gate[t]) (each term optional; no gate: 1).
hipError_t launch_blend_prep(const uint16_t* shared16, const float* gate, const uint16_t* residual, int T, int H,
                             float* extra, hipStream_t s);
hipError_t launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t s);
// DEC_MAX_TOKENS constant zeros in device memory of the current device (expert index 0 of every
// token of a one-expert layer in decode), or null if its address could not be obtained.
const int32_t* zero_index();
// TQ3 GEMV (tq3.hip): out[v][r] = row r of the TQ3 matrix of expert vexp[v] (at w + e * wstride;
// null vexp: expert 0) dotted with input row v / in_div (fp16, or fp32 when in32; rotated by the
// kernel); pair: r indexes gate/up row pairs (up matrix at + up_off) and out = silu(gate) * up.
// fp32 or fp16 out; experts outside [0, E) give zeros.  C a multiple of 32 up to 4096.
struct Tq3Params {
  const uint8_t* w;
  int64_t wstride, up_off;
  const int32_t* vexp;
  int E;
  const void* in;
  int in_div, V, R, C;
  float* out32;
  uint16_t* out16;
};
hipError_t launch_tq3_gemv(const Tq3Params& p, bool in32, bool pair, hipStream_t s);
// Writes the prefill copy of c's experts into `pack` (laid out by pack_layout).
hipError_t launch_prefill_pack(const LayerConfig& c, uint8_t* pack, hipStream_t s);
hipError_t launch_dequantize(const LayerConfig& c, int proj, int expert, int row0, int nrows, uint8_t* codes,
                             uint16_t* wf16, hipStream_t s);


}  // namespace kmoe
