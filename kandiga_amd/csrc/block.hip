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

namespace kmoe {

constexpr int QL_TB = 4;    // tokens per workgroup
constexpr int QL_RPW = 2;   // rows per wave
constexpr uint32_t QL_ONE2 = 0x3C003C00u;
constexpr float QL_TWO24 = 16777216.0f;

template <int BITS, bool BF16>
__global__ __launch_bounds__(256) void qlinear_kernel(const QProj A, int ra, const QProj B, int rb, int T, int H,
                                                      const uint16_t* __restrict__ x, float* __restrict__ out_a,
                                                      float* __restrict__ out_b) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int R = ra + rb;
  const int t0 = blockIdx.y * QL_TB;
  const int r0 = (blockIdx.x * 4 + wave) * QL_RPW;
  const int nch = H / CHUNK, ng = H / GROUP;
  const size_t rbytes = (size_t)H * BITS / 8;
  float acc[QL_RPW * QL_TB];
#pragma unroll
  for (int v = 0; v < QL_RPW * QL_TB; ++v) acc[v] = 0.f;
  for (int c = lane; c < nch; c += 64) {
    uint32_t xp[QL_TB][16];
    float xs[QL_TB];
#pragma unroll
    for (int t = 0; t < QL_TB; ++t) {
      uint32_t nat[16];
      const int tt = min(t0 + t, T - 1);  // tokens past T reload the last one (never stored)
      load16g(x + (size_t)tt * H + (size_t)c * CHUNK, nat);
      float sm = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) sm = fdot2(nat[m], QL_ONE2, sm);
      xs[t] = sm;
      to_pair_order<BITS>(nat, xp[t]);
    }
#pragma unroll
    for (int r = 0; r < QL_RPW; ++r) {
      const int row = min(r0 + r, R - 1);  // rows past R recompute the last one (never stored)
      const QProj& P = row < ra ? A : B;
      const int pr = row < ra ? row : row - ra;
      uint32_t d[4], cp[16];
      load_chunk<BITS>(P.w + (size_t)pr * rbytes, c, d);
      unpack_chunk<BITS, false>(d, cp);
      const float sf = scale_to_f32<BF16>(P.s[(size_t)pr * ng + (c >> 1)]) * QL_TWO24;
      const float bf = scale_to_f32<BF16>(P.b[(size_t)pr * ng + (c >> 1)]);
#pragma unroll
      for (int t = 0; t < QL_TB; ++t) acc[r * QL_TB + t] += sf * chunk_dot(cp, xp[t]) + bf * xs[t];
    }
  }
  const float tot = wave_sum_multi<8>(acc);  // value v = r*QL_TB + t lands in lanes 8v..8v+7
  if ((lane & 7) == 0) {
    const int v = lane >> 3, r = v / QL_TB, t = v - r * QL_TB;
    const int row = r0 + r, tok = t0 + t;
    if (row < R && tok < T) {
      if (row < ra)
        out_a[(size_t)tok * ra + row] = tot;
      else
        out_b[(size_t)tok * rb + (row - ra)] = tot;
    }
  }
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
  const dim3 grid((R + 4 * QL_RPW - 1) / (4 * QL_RPW), (T + QL_TB - 1) / QL_TB);
#define KMOE_QL(BB, FF) \
  KMOE_LAUNCH("qlinear_kernel", (qlinear_kernel<BB, FF>), grid, dim3(256), 0, s, a, ra, b, rb, T, H, x, out_a, out_b)
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
