// The rest of the MoE block around the routed experts: the router projection, the sigmoid gate
// of the shared expert and the residual blend (kandiga/metal/moe_block.metal:194-227
// router_matmul_kernel, :300-336 shared_gate_kernel, :515-584 blend_kernel / blend_residual_kernel).
// The shared expert itself runs through the routed-expert kernels as a one-expert layer.
//
//   qlinear_kernel: out[t][r] = sum_h W[r][h] x[t][h] for the rows of the router (the block's
//     num_experts logits) followed by the shared gate's one row, over MLX group-quantized
//     weights.  A workgroup takes 8 rows (2 per wave) and 4 tokens; each lane one 32-code
//     chunk at a time, with the raw-code dot of the decode kernels (codes as fp16 subnormals,
//     v_dot2_f32_f16, then s*2^24*dot + b*sum(x) per chunk); the 8 (row, token) totals of a wave
//     are reduced in one pass.  fp32 throughout.
//   blend_prep_kernel: extra[t][h] = residual[t][h] + fp16(shared[t][h]) * sigmoid(gate[t]), the
//     term the routed layer's combine adds after the weighted expert sum (moe_block.metal:
//     556-584 keeps the shared output in fp16 and gates it in fp32).
//   fill_i32_kernel: the expert index 0 of every token for the one-expert shared layer.
#include <mutex>

#include "kmoe_device.h"
#include "kmoe_internal.h"
#include "qlinear.h"

namespace kmoe {

template <int BITS, bool BF16, int RPW>
__global__ __launch_bounds__(256) void qlinear_kernel(const QProj A, int ra, const QProj B, int rb, int T, int H,
                                                      const uint16_t* __restrict__ x, float* __restrict__ out_a,
                                                      float* __restrict__ out_b) {
  qlinear_rows<BITS, BF16, RPW>(A, ra, B, rb, T, H, x, out_a, out_b, (int)blockIdx.x, (int)blockIdx.y);
}

__global__ __launch_bounds__(256) void blend_prep_kernel(const uint16_t* __restrict__ shared16,
                                                         const float* __restrict__ gate,
                                                         const uint16_t* __restrict__ residual, int T, int H,
                                                         float* __restrict__ extra) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * H) return;
  const int t = (int)(i / H);
  float v = residual ? f16_bits_to_f32(residual[i]) : 0.f;
  if (shared16) {
    const float g = gate ? 1.0f / (1.0f + expf(-gate[t])) : 1.0f;
    v += f16_bits_to_f32(shared16[i]) * g;
  }
  extra[i] = v;
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int n, int32_t v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// Never written: the loader places it, zeroed, on every device the library runs on.
__device__ int32_t g_zero_index[DEC_MAX_TOKENS] = {};

const int32_t* zero_index() {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static const int32_t* ptr[kMaxDev] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_zero_index)) != hipSuccess) return nullptr;
    ptr[dev] = static_cast<const int32_t*>(p);
  }
  return ptr[dev];
}

hipError_t launch_qlinear(const QProj& a, int ra, const QProj& b, int rb, int bits, bool bf16, const uint16_t* x,
                          int T, int H, float* out_a, float* out_b, hipStream_t s) {
  const int R = ra + rb;
  if (T == 0 || R == 0) return hipSuccess;
  // eight rows per wave once the batch outgrows decode (the token blocks then fill the GPU)
  const bool wide = T > DEC_MAX_TOKENS;
  const dim3 grid(qlinear_row_blocks(R, wide ? 8 : QL_RPW), qlinear_token_blocks(T));
#define KMOE_QL(BB, FF)                                                                                          \
  do {                                                                                                           \
    if (wide)                                                                                                    \
      KMOE_LAUNCH("qlinear_kernel", (qlinear_kernel<BB, FF, 8>), grid, dim3(256), 0, s, a, ra, b, rb, T, H, x,      \
                  out_a, out_b);                                                                                 \
    else                                                                                                         \
      KMOE_LAUNCH("qlinear_kernel", (qlinear_kernel<BB, FF, QL_RPW>), grid, dim3(256), 0, s, a, ra, b, rb, T, H, x, \
                  out_a, out_b);                                                                                 \
  } while (0)
  if (bits == 3) {
    if (bf16) KMOE_QL(3, true); else KMOE_QL(3, false);
  } else {
    if (bf16) KMOE_QL(4, true); else KMOE_QL(4, false);
  }
#undef KMOE_QL
  return hipGetLastError();
}

hipError_t launch_blend_prep(const uint16_t* shared16, const float* gate, const uint16_t* residual, int T, int H,
                             float* extra, hipStream_t s) {
  const size_t n = (size_t)T * H;
  if (n == 0) return hipSuccess;
  KMOE_LAUNCH("blend_prep_kernel", blend_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, shared16,
              gate, residual, T, H, extra);
  return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  KMOE_LAUNCH("fill_i32_kernel", fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace kmoe
