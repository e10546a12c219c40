/*
 * kandiga_amd.h -- C ABI of the MI355X routed-expert MoE layer (libkandiga_amd.so).
 *
 * Plain pointers and sizes only.  "device" pointers are HIP device memory; `stream` is a
 * hipStream_t (NULL = default stream).  Calls are asynchronous on `stream` and return a
 * status (0 = KMOE_OK, negative = error; kmoe_strerror / kmoe_last_error describe it).
 * Arguments are validated on the host before anything is launched.  Every entry point is
 * re-entrant: layer handles are immutable after creation, and all scratch memory is a
 * caller-provided workspace (calls that overlap on one workspace race).
 *
 * Weight layout (MLX affine quantization, group size 64), per projection stack:
 *   weight  uint32 [E][rows][in*bits/32]  codes as a little-endian bit stream
 *   scales  fp16|bf16 [E][rows][in/64]
 *   biases  fp16|bf16 [E][rows][in/64]      w = q*scale + bias
 * with gate/up rows = intermediate, in = hidden, and down rows = hidden, in = intermediate.
 * The expert strides are explicit, so both mlx_lm's stacked SwitchGLU tensors and a
 * BKEX file body uploaded as-is (kandiga/_pack_experts.py:6-20) can be described.
 */
#ifndef KANDIGA_AMD_H
#define KANDIGA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum kmoe_status {
  KMOE_OK = 0,
  KMOE_ERR_INVALID_ARG = -1,
  KMOE_ERR_UNSUPPORTED = -2,
  KMOE_ERR_ALIGNMENT = -3,
  KMOE_ERR_WORKSPACE = -4,
  KMOE_ERR_HIP = -5,
  KMOE_ERR_IO = -6,
  KMOE_ERR_FORMAT = -7,
  KMOE_ERR_DEVICE = -8,
  KMOE_ERR_NO_MEMORY = -9
};

enum { KMOE_SCALE_F16 = 0, KMOE_SCALE_BF16 = 1 };
enum { KMOE_ACT_SWIGLU = 0, KMOE_ACT_GELU_TANH = 1 };
enum { KMOE_PROJ_GATE = 0, KMOE_PROJ_UP = 1, KMOE_PROJ_DOWN = 2 };
enum { KMOE_OUT_F16 = 0, KMOE_OUT_F32 = 1 };
/* Activation dtypes of kmoe_expert_mlp_x / kmoe_forward_x. */
enum { KMOE_X_F16 = 0, KMOE_X_BF16 = 1, KMOE_X_F32 = 2 };
/* Device error flags reported by kmoe_device_status (other bits are reserved and read 0: no
   kernel waits on another workgroup, so there is no time-out to report). */
enum {
  KMOE_DEVERR_BAD_EXPERT = 1 /* an expert index outside [0, num_experts) was dropped */
};

typedef struct {
  const void* weight;            /* device, 16-byte aligned (4-bit) / 4-byte aligned (3-bit) */
  const void* scales;            /* device, 2-byte aligned */
  const void* biases;            /* device, 2-byte aligned */
  int64_t weight_expert_stride;  /* bytes between consecutive experts' codes */
  int64_t scale_expert_stride;   /* bytes between consecutive experts' scales (same for biases) */
} kmoe_qproj;

typedef struct {
  int32_t hidden;        /* H, multiple of 64 */
  int32_t intermediate;  /* I, multiple of 64 */
  int32_t num_experts;   /* E, 1..1024 */
  int32_t top_k;         /* K, 1..min(E, 16) */
  int32_t bits;          /* 3 or 4 */
  int32_t group_size;    /* must be 64 */
  int32_t scale_dtype;   /* KMOE_SCALE_F16 or KMOE_SCALE_BF16 */
  int32_t activation;    /* KMOE_ACT_SWIGLU (silu(g)*u) or KMOE_ACT_GELU_TANH */
  kmoe_qproj gate, up, down;
  /* Optional always-on dense fp16 shared expert added after the routed combine
     (ungated): gate/up [Is][H], down [H][Is].  All NULL when absent. */
  const void* shared_gate;
  const void* shared_up;
  const void* shared_down;
  int32_t shared_intermediate;
  int32_t reserved;
  /* Optional prefill copy of the routed experts made by kmoe_prefill_pack from this same
     description (device, 256-byte aligned, kmoe_prefill_pack_size bytes), or NULL.  When set,
     the grouped GEMMs of calls with more than 8 tokens read the weights from it; decode and the
     dequantization check keep reading the MLX-layout tensors above. */
  const void* prefill_pack;
  int64_t prefill_pack_bytes;
} kmoe_layer_desc;

typedef struct kmoe_layer kmoe_layer;

/* Library version (major*10000 + minor*100 + patch). */
int kmoe_version(void);
const char* kmoe_strerror(int status);
/* Message of the last failing call on this thread ("" if none). */
const char* kmoe_last_error(void);

/* Validate a layer description and keep a copy (no device memory is allocated). */
int kmoe_layer_create(const kmoe_layer_desc* desc, kmoe_layer** out);
int kmoe_layer_destroy(kmoe_layer* layer);

/* Bytes of workspace needed for calls of up to max_tokens tokens on this layer.
 * The first 256 bytes hold device status words: zero the workspace once after allocating it. */
int kmoe_workspace_size(const kmoe_layer* layer, int32_t max_tokens, size_t* bytes);

/*
 * Router: per token the top_k experts by router logit (ties -> lower index) and their
 * softmax probabilities renormalised over the selected experts.
 * Replaces router_softmax_topk (kandiga/metal/moe_block.metal:419-505) and mlx_lm's
 * softmax -> argpartition -> renorm feeding switch_mlp (kandiga/engine.py:1090-1139).
 *   logits  device fp32 [tokens][num_experts];  idx device int32 [tokens][top_k];
 *   weights device fp32 [tokens][top_k].
 */
int kmoe_route(const float* logits, int32_t tokens, int32_t num_experts, int32_t top_k, int32_t* idx,
               float* weights, void* stream);

/*
 * Stable token -> expert permutation (kandiga/engine.py:407-418, the grouping of
 * _gpu_prefill_experts): perm lists the assignment ids a = t*top_k + k sorted by
 * (expert, a); counts/offsets are the per-expert histogram and its exclusive scan;
 * unique lists the experts with a nonzero count in ascending order, num_unique[0] their
 * number.  All output pointers are device memory:
 *   perm [tokens*top_k], counts [num_experts], offsets [num_experts+1],
 *   unique [num_experts], num_unique [1].
 */
int kmoe_permute_workspace_size(int32_t tokens, int32_t top_k, int32_t num_experts, size_t* bytes);
int kmoe_permute(const int32_t* idx, int32_t tokens, int32_t top_k, int32_t num_experts, int32_t* perm,
                 int32_t* counts, int32_t* offsets, int32_t* unique, int32_t* num_unique, void* workspace,
                 size_t workspace_bytes, void* stream);

/*
 * switch_mlp contract: y[t][k] = expert idx[t][k] applied to x[t] (SwiGLU gate/up/down over
 * the quantized experts), not combined.  Replaces _CPUSwitchGLU.__call__ (kandiga/engine.py:
 * 670-739) and, per token, bakan_cpu_expert_mlp_f16 (kandiga/metal/kandiga_cpu_expert.h:61-68).
 *   x device fp16 [tokens][H]; idx device int32 [tokens][top_k]; y device fp16 [tokens][top_k][H].
 */
int kmoe_expert_mlp(const kmoe_layer* layer, const void* x, const int32_t* idx, int32_t tokens, void* y,
                    void* workspace, size_t workspace_bytes, void* stream);
/*
 * kmoe_expert_mlp with the activations in the caller's dtype: x_dtype KMOE_X_F16, KMOE_X_BF16 or
 * KMOE_X_F32 (rows [tokens][H]).  Replaces bakan_cpu_expert_mlp_bf16 (bf16 x) and
 * bakan_cpu_expert_mlp (fp32 x) (kandiga/metal/kandiga_cpu_expert.h:51-89,
 * kandiga_cpu_expert.m:471-552, 690-719), which widen x to fp32.  Each token's row is taken as
 * fp16 planes of x * 2^s: s = 0 when its largest magnitude m lies in [2^-4, 2^4), else the power
 * of two that puts m in [1, 2).  A bf16 row is then exact in the hi plane (elements down to
 * 2^-14 m), an fp32 row carries ~22 bits (hi + lo planes); gate/up are multiplied by 2^-s and
 * the SwiGLU output is carried times 2^2s and taken back after the down projection, all exact
 * in fp32, so rows far outside fp16's range stay in range.  Rows of fp16-representable values
 * with m in the window give the fp16 path's result bit for bit.
 */
int kmoe_expert_mlp_x(const kmoe_layer* layer, const void* x, int32_t x_dtype, const int32_t* idx, int32_t tokens,
                      void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Weighted combine of switch_mlp outputs: out[t] = sum_k weights[t][k] * y[t][k], fp32
 * accumulation in k order, one fp16 rounding (moe_block.metal:515-539, blend_kernel).
 *   y device fp16 [tokens][top_k][hidden]; weights device fp32 [tokens][top_k];
 *   out device fp16 [tokens][hidden].
 */
int kmoe_combine(const void* y, const float* weights, int32_t tokens, int32_t top_k, int32_t hidden, void* out,
                 void* stream);

/*
 * Whole routed layer: route -> permute -> expert MLP -> weighted combine (+ shared expert).
 * The block the reference assembles from mlx_lm's SparseMoeBlock router and combine around
 * _CPUSwitchGLU (kandiga/engine.py:1090-1139, 670-739); its all-in-one restatement is the
 * MoE step of the unwired C/Metal engine (kandiga/metal/full_forward_lg.m:1316-1350,
 * 1635-1735: router_softmax_topk, expert_mlp_fused, blend_kernel).
 *   x device fp16 [tokens][H]; logits device fp32 [tokens][E];
 *   out device [tokens][H], fp16 (out_dtype KMOE_OUT_F16) or fp32 (KMOE_OUT_F32);
 *   idx_out / weights_out (device, optional, may be NULL) receive the routing.
 * 1..8 tokens run the GEMV decode kernels, larger batches the grouped MFMA GEMM.
 */
int kmoe_forward(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens, void* out,
                 int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace, size_t workspace_bytes,
                 void* stream);
/* kmoe_forward with the activations in the caller's dtype (as kmoe_expert_mlp_x).  A layer with
 * the dense fp16 shared expert takes KMOE_X_F16 only (KMOE_ERR_UNSUPPORTED otherwise). */
int kmoe_forward_x(const kmoe_layer* layer, const void* x, int32_t x_dtype, const float* logits, int32_t tokens,
                   void* out, int32_t out_dtype, int32_t* idx_out, float* weights_out, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * The whole MoE block mlp(x) of the decoder layer: router projection over the quantized
 * mlp.gate (fp32 logits), softmax -> top-K -> renorm, the routed experts, the quantized shared
 * expert mlp.shared_expert gated by sigmoid(mlp.shared_expert_gate . x), and an optional
 * residual:  out = (residual + sum_k w_k y_k) + fp16(shared(x)) * sigmoid(gate . x).
 * Replaces mlx_lm's Qwen MoE block as driven by kandiga/engine.py:1090-1139, restated in
 * kandiga/metal/moe_block.metal:194-227 (router_matmul_kernel), :240-336 (shared expert and its
 * gate), :419-505 (router_softmax_topk), :515-584 (blend_kernel / blend_residual_kernel), the
 * MoE step of kandiga/metal/full_forward_lg.m:1316-1350, 1635-1735 (bakan_forward_moe_block,
 * kandiga/metal/bakan_forward.h:111-140).
 * The router, shared expert and shared gate share one bit width (3 or 4, group 64) and scale
 * dtype, which may differ from the routed experts' (a 3-bit routed stack beside 4-bit
 * projections).  The routed layer must not carry a dense shared expert.
 */
typedef struct {
  const kmoe_layer* routed;        /* the routed experts (kmoe_layer_create); must outlive the block */
  kmoe_qproj router;               /* mlp.gate: [num_experts][hidden]; expert strides ignored */
  kmoe_qproj shared_gate_proj;     /* mlp.shared_expert.gate_proj [Is][hidden]; weight NULL: no shared expert */
  kmoe_qproj shared_up_proj;       /* mlp.shared_expert.up_proj [Is][hidden] */
  kmoe_qproj shared_down_proj;     /* mlp.shared_expert.down_proj [hidden][Is] */
  kmoe_qproj shared_expert_gate;   /* mlp.shared_expert_gate [1][hidden]; weight NULL: ungated shared expert */
  int32_t bits;                    /* codes of the four projections above: 3 or 4 */
  int32_t scale_dtype;             /* KMOE_SCALE_F16 or KMOE_SCALE_BF16 */
  int32_t shared_intermediate;     /* Is, multiple of 64 */
  int32_t reserved;
} kmoe_block_desc;

typedef struct kmoe_block kmoe_block;

int kmoe_block_create(const kmoe_block_desc* desc, kmoe_block** out);
int kmoe_block_destroy(kmoe_block* block);
/* Workspace bytes for block calls of up to max_tokens tokens (zero it once after allocating). */
int kmoe_block_workspace_size(const kmoe_block* block, int32_t max_tokens, size_t* bytes);
/*
 *   x device fp16 [tokens][hidden] (the post-attention-norm input of mlp); residual device fp16
 *   [tokens][hidden] or NULL; out device [tokens][hidden] fp16 or fp32 (out_dtype);
 *   idx_out / weights_out / logits_out (device, optional) receive the routing and the fp32 router
 *   logits [tokens][num_experts].
 */
int kmoe_block_forward(const kmoe_block* block, const void* x, const void* residual, int32_t tokens, void* out,
                       int32_t out_dtype, int32_t* idx_out, float* weights_out, float* logits_out, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * TQ3 codebook weights (kandiga/tq3/quantize.py:120-143, 390-486): 32 weights per 20-byte block
 * (fp16 d0 d1 m0 m1, 12 bytes of 3-bit Lloyd-Max indices), w = iWHT(C[q]*d + m) per block; a
 * matrix [rows][cols] is its rows' blocks in order.
 *
 * kmoe_tq3_gemv: out[t][r] = sum_c W[r][c] x[t][c], fp32, the input rotated into the transform
 * domain once per 32-block (replaces tq3_gemv, kandiga/tq3/fused_kernel.py:170-251, and
 * tq3_matvec / tq3_rotate_activations, kandiga/tq3/tq3_metal.metal:55-141).
 *   blocks device [rows*cols/32][20]; x device [tokens][cols] fp16 (x_f32 = 0) or fp32 (1);
 *   out device fp32 [tokens][rows]; cols a multiple of 32 up to 4096.
 *
 * kmoe_tq3_expert_mlp: the switch_mlp contract over TQ3 experts (a TQ3X file body,
 * kandiga/tq3/convert_experts.py:140-200: per expert the gate [I][H], up [I][H] and down [H][I]
 * matrices in turn, expert_bytes apart): y[t][k] = down(silu(gate x_t) * (up x_t)) of expert
 * idx[t][k], fp16.  Experts outside [0, num_experts) give zero rows.  The workspace holds the
 * SwiGLU outputs (kmoe_tq3_workspace_size).
 */
int kmoe_tq3_gemv(const void* blocks, int32_t rows, int32_t cols, const void* x, int32_t x_f32, int32_t tokens,
                  float* out, void* stream);
int kmoe_tq3_workspace_size(int32_t tokens, int32_t top_k, int32_t intermediate, size_t* bytes);
int kmoe_tq3_expert_mlp(const void* experts, int64_t expert_bytes, int32_t num_experts, int32_t hidden,
                        int32_t intermediate, const void* x, const int32_t* idx, int32_t tokens, int32_t top_k, void* y,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * kmoe_forward without a workspace argument: the library's own static device scratch of
 * KMOE_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends) serves as the workspace, and
 * the call allocates nothing (no hipMalloc, no allocating library routine).  No counterpart in
 * the reference; for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  Calls whose kmoe_workspace_size exceeds
 * the scratch fail with KMOE_ERR_WORKSPACE before anything is launched (every decode batch fits;
 * prefill up to about T*K*H*4 + T*K*I*4 bytes).  All calls on one GPU share its scratch: calls
 * that overlap on one GPU race.  Device error flags are not readable through this entry point.
 */
#define KMOE_NOALLOC_SCRATCH_BYTES (16u << 20)
int kmoe_forward_noalloc(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens, void* out,
                         int32_t out_dtype, int32_t* idx_out, float* weights_out, void* stream);

/*
 * Prefill weight copy.  No counterpart in the reference, whose routed experts exist only in
 * the MLX layout; for callers that run prefill and can hold a second copy of the experts (about
 * the size of the codes plus scales).  kmoe_prefill_pack rewrites every expert of `desc` into a
 * layout in which one wavefront load of the grouped GEMMs reads whole cache lines:
 *   codes  [expert][32-row block][group][lane n + 32h][chunk h of row n]   (12 or 16 bytes)
 *   scales/biases [expert][32-row block][group pair][row n][s0 s1 b0 b1]   (fp16/bf16 bits)
 * for gate, up and down in turn (each region 256-byte aligned).  Results do not depend on
 * whether a layer has the copy.  `pack` is device memory of kmoe_prefill_pack_size bytes;
 * the call is asynchronous on `stream` and reads the tensors `desc` points to.
 */
int kmoe_prefill_pack_size(const kmoe_layer_desc* desc, size_t* bytes);
int kmoe_prefill_pack(const kmoe_layer_desc* desc, void* pack, size_t bytes, void* stream);

/*
 * Dequantization check: codes (uint8 [nrows][in]) and fp16 weights round(q*s + b)
 * (uint16 bits [nrows][in]) of rows row0.. of one expert's projection, as the kernels
 * unpack them.  Device output pointers.
 */
int kmoe_dequantize(const kmoe_layer* layer, int32_t proj, int32_t expert, int32_t row0, int32_t nrows,
                    uint8_t* codes, uint16_t* weights_f16, void* stream);

/* Synchronise `stream`, then read and clear the device error flags kept in `workspace`. */
int kmoe_device_status(void* workspace, size_t workspace_bytes, int32_t* flags, void* stream);

/*
 * Kernel timing.  No counterpart in the reference, whose engine times whole calls on the host;
 * for benchmarks and profilers.  After kmoe_profile_begin(max_launches), every kernel this
 * library launches from the calling thread (up to max_launches, at most 16384) is bracketed by
 * a pair of HIP events recorded on the launch stream; launches into a stream under graph
 * capture are not timed.  kmoe_profile_end synchronises those events and fills one entry per
 * kernel name (launch count, total / min / max event time in ms), then stops timing.
 */
typedef struct kmoe_kernel_time {
  char name[48];
  int32_t launches;
  int32_t reserved;
  double total_ms;
  double min_ms;
  double max_ms;
} kmoe_kernel_time;

int kmoe_profile_begin(int32_t max_launches);
int kmoe_profile_end(kmoe_kernel_time* entries, int32_t max_entries, int32_t* n_entries);

#ifdef __cplusplus
}
#endif

#endif /* KANDIGA_AMD_H */
