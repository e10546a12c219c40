// Prefill path: grouped GEMM over the expert-sorted assignments with fp16 MFMA.
//
// Replaces the reference's 4-bit prefill (kandiga/engine.py:386-516: permutation, one
// Metal dispatch for gate+up+SiLU over every (assignment, row), one for down, then a
// scatter back to [T, K, H]) and its 3-bit fallback (engine.py:720-735: T sequential
// CPU calls).
//
//   gemm_gateup_kernel: one workgroup per (m-tile of <= 128 sorted assignments of one
//     expert, 64 intermediate columns).  Per 64-wide k step the workgroup gathers the
//     tile's x rows (token = assignment / K) into LDS in pair order, dequantizes the 64
//     gate rows and 64 up rows of that k step into LDS as fp16 (one quant group per row,
//     round(q*s + b) by one fp16 fma), and runs v_mfma_f32_32x32x16_f16.  Each wave owns
//     64 rows x 32 columns of both gate and up, so SwiGLU is applied in registers and
//     act is written once (fp16, pair order for the down projection's k dimension).
//   gemm_down_kernel: one workgroup per (m-tile, 128 output columns); A = act rows of the
//     tile (already contiguous and in pair order), B = dequantized down rows.  The output
//     row of sorted position p is written to assignment perm[p], as fp32 for the fused
//     layer or fp16 for the switch_mlp contract.
//   combine_kernel: out[t] = sum_k w[t,k] * y[t,k] (+ shared expert), fp32 accumulate in
//     k order, one fp16 rounding (moe_block.metal:515-539).
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

template <int BITS>
struct PairPosTableP {
  uint8_t v[32];
};
template <int BITS>
constexpr PairPosTableP<BITS> make_pair_pos_p() {
  PairPosTableP<BITS> t{};
  for (int e = 0; e < 32; ++e) t.v[e] = (uint8_t)pair_pos(BITS, e);
  return t;
}
__constant__ PairPosTableP<3> p_pairpos3 = make_pair_pos_p<3>();
__constant__ PairPosTableP<4> p_pairpos4 = make_pair_pos_p<4>();

template <int BITS>
__device__ __forceinline__ int pairpos_p(int e) {
  if constexpr (BITS == 3) {
    return p_pairpos3.v[e];
  } else {
    return p_pairpos4.v[e];
  }
}

template <int ACT>
__device__ __forceinline__ float activate_p(float g, float u) {
  if constexpr (ACT == 0) {
    return silu_f32(g) * u;
  } else {
    return gelu_tanh_f32(g) * u;
  }
}

constexpr int BK = 64;   // k step = one quantization group
constexpr int LDH = 72;  // LDS row stride in halves (64 + 8 pad: 144 bytes)

__device__ __forceinline__ void load16g(const void* p, uint32_t (&v)[16]) {
  const uint4* s = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 t = s[q];
    v[4 * q] = t.x;
    v[4 * q + 1] = t.y;
    v[4 * q + 2] = t.z;
    v[4 * q + 3] = t.w;
  }
}

__device__ __forceinline__ void store16s(_Float16* dst, const uint32_t (&v)[16]) {
  uint4* d = reinterpret_cast<uint4*>(dst);
#pragma unroll
  for (int q = 0; q < 4; ++q) d[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

// Dequantize one 32-code chunk of a quantized row into 16 fp16 pairs (pair order).
template <int BITS, bool BF16>
__device__ __forceinline__ void dequant_chunk(const uint8_t* row, int chunk, uint16_t sbits, uint16_t bbits,
                                              uint32_t (&out)[16]) {
  uint32_t d[4];
  load_chunk<BITS>(row, chunk, d);
  const float sf = scale_to_f32<BF16>(sbits), bf = scale_to_f32<BF16>(bbits);
  const half2_t s2 = {(_Float16)sf, (_Float16)sf}, b2 = {(_Float16)bf, (_Float16)bf};
  unpack_chunk<BITS, true>(d, out);
#pragma unroll
  for (int p = 0; p < 16; ++p) out[p] = dequant_pair(out[p], s2, b2);
}

__device__ __forceinline__ float16_t mfma32(const half8_t a, const half8_t b, const float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int BITS, bool BF16, int ACT>
__global__ __launch_bounds__(256, 2) void gemm_gateup_kernel(const LayerArgs L, const uint16_t* __restrict__ x,
                                                             int K, const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ scalars,
                                                             const int32_t* __restrict__ mt_expert,
                                                             const int32_t* __restrict__ mt_row0,
                                                             const int32_t* __restrict__ mt_rows,
                                                             uint16_t* __restrict__ act) {
  constexpr int BNI = 64;  // intermediate columns per tile (gate and up each)
  __shared__ __attribute__((aligned(16))) _Float16 sA[GEMM_BM * LDH];
  __shared__ __attribute__((aligned(16))) _Float16 sB[2 * BNI * LDH];
  const int H = L.H, I = L.I;
  const int n_it = I / BNI;
  const int mt = blockIdx.x / n_it, it = blockIdx.x - mt * n_it;
  if (mt >= scalars[1]) return;
  const int e = mt_expert[mt], row0 = mt_row0[mt], nrows = mt_rows[mt];
  const int i0 = it * BNI;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  const int lr = tid >> 1, lc = tid & 1;  // loader: tile row 0..127, chunk 0..1 of the k step
  const bool a_ok = lr < nrows;
  const int tok = a_ok ? perm[row0 + lr] / K : 0;
  const uint16_t* xrow = x + (size_t)tok * H;
  const bool is_up = lr >= BNI;
  const uint8_t* wbase = is_up ? L.up.w : L.gate.w;
  const uint16_t* sbase = is_up ? L.up.s : L.gate.s;
  const uint16_t* bbase = is_up ? L.up.b : L.gate.b;
  const int64_t wst = is_up ? L.up.w_stride : L.gate.w_stride;
  const int64_t sst = is_up ? L.up.s_stride : L.gate.s_stride;
  const int brow = i0 + (lr & (BNI - 1));
  const size_t rbytes = (size_t)H * BITS / 8;
  const int ng = H / GROUP;
  const uint8_t* wrow = wbase + (size_t)e * wst + (size_t)brow * rbytes;
  const uint16_t* srow = sbase + (size_t)e * sst + (size_t)brow * ng;
  const uint16_t* bsrow = bbase + (size_t)e * sst + (size_t)brow * ng;

  float16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  for (int k0 = 0; k0 < H; k0 += BK) {
    uint32_t nat[16], pa[16];
    if (a_ok) {
      load16g(xrow + k0 + lc * CHUNK, nat);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) nat[q] = 0u;
    }
    to_pair_order<BITS>(nat, pa);
    uint32_t pb[16];
    dequant_chunk<BITS, BF16>(wrow, (k0 >> 5) + lc, srow[k0 >> 6], bsrow[k0 >> 6], pb);
    store16s(sA + lr * LDH + lc * CHUNK, pa);
    store16s(sB + lr * LDH + lc * CHUNK, pb);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int koff = ks * 16 + (lane >> 5) * 8;
      const half8_t a0 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + (lane & 31)) * LDH + koff);
      const half8_t a1 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + 32 + (lane & 31)) * LDH + koff);
      const half8_t bg = *reinterpret_cast<const half8_t*>(sB + (32 * wn + (lane & 31)) * LDH + koff);
      const half8_t bu = *reinterpret_cast<const half8_t*>(sB + (BNI + 32 * wn + (lane & 31)) * LDH + koff);
      acc[0][0] = mfma32(a0, bg, acc[0][0]);
      acc[0][1] = mfma32(a0, bu, acc[0][1]);
      acc[1][0] = mfma32(a1, bg, acc[1][0]);
      acc[1][1] = mfma32(a1, bu, acc[1][1]);
    }
    __syncthreads();
  }
  const int col = lane & 31;
  const int cbase = i0 + 32 * wn;
  const int cpos = pairpos_p<BITS>(col);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 64 * wm + 32 * mb + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
      if (r < nrows)
        act[(size_t)(row0 + r) * I + cbase + cpos] = f32_to_f16_bits(activate_p<ACT>(acc[mb][0][j], acc[mb][1][j]));
    }
  }
}

template <int BITS, bool BF16, bool OUT16>
__global__ __launch_bounds__(256, 2) void gemm_down_kernel(const LayerArgs L, const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ scalars,
                                                           const int32_t* __restrict__ mt_expert,
                                                           const int32_t* __restrict__ mt_row0,
                                                           const int32_t* __restrict__ mt_rows,
                                                           const uint16_t* __restrict__ act,
                                                           float* __restrict__ y32, uint16_t* __restrict__ y16) {
  constexpr int BN = 128;
  __shared__ __attribute__((aligned(16))) _Float16 sA[GEMM_BM * LDH];
  __shared__ __attribute__((aligned(16))) _Float16 sB[BN * LDH];
  const int H = L.H, I = L.I;
  const int n_ht = (H + BN - 1) / BN;
  const int mt = blockIdx.x / n_ht, ht = blockIdx.x - mt * n_ht;
  if (mt >= scalars[1]) return;
  const int e = mt_expert[mt], row0 = mt_row0[mt], nrows = mt_rows[mt];
  const int h0 = ht * BN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  const int lr = tid >> 1, lc = tid & 1;
  const bool a_ok = lr < nrows;
  const uint16_t* arow = act + (size_t)(row0 + (a_ok ? lr : 0)) * I;
  const int brow = h0 + lr;
  const bool b_ok = brow < H;
  const size_t rbytes = (size_t)I * BITS / 8;
  const int ng = I / GROUP;
  const int brow_c = b_ok ? brow : 0;
  const uint8_t* wrow = L.down.w + (size_t)e * L.down.w_stride + (size_t)brow_c * rbytes;
  const uint16_t* srow = L.down.s + (size_t)e * L.down.s_stride + (size_t)brow_c * ng;
  const uint16_t* bsrow = L.down.b + (size_t)e * L.down.s_stride + (size_t)brow_c * ng;

  float16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  for (int k0 = 0; k0 < I; k0 += BK) {
    uint32_t pa[16], pb[16];
    if (a_ok) {
      load16g(arow + k0 + lc * CHUNK, pa);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) pa[q] = 0u;
    }
    if (b_ok) {
      dequant_chunk<BITS, BF16>(wrow, (k0 >> 5) + lc, srow[k0 >> 6], bsrow[k0 >> 6], pb);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) pb[q] = 0u;
    }
    store16s(sA + lr * LDH + lc * CHUNK, pa);
    store16s(sB + lr * LDH + lc * CHUNK, pb);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int koff = ks * 16 + (lane >> 5) * 8;
      const half8_t a0 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + (lane & 31)) * LDH + koff);
      const half8_t a1 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + 32 + (lane & 31)) * LDH + koff);
      const half8_t b0 = *reinterpret_cast<const half8_t*>(sB + (64 * wn + (lane & 31)) * LDH + koff);
      const half8_t b1 = *reinterpret_cast<const half8_t*>(sB + (64 * wn + 32 + (lane & 31)) * LDH + koff);
      acc[0][0] = mfma32(a0, b0, acc[0][0]);
      acc[0][1] = mfma32(a0, b1, acc[0][1]);
      acc[1][0] = mfma32(a1, b0, acc[1][0]);
      acc[1][1] = mfma32(a1, b1, acc[1][1]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 64 * wm + 32 * mb + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
      if (r < nrows) {
        const size_t ybase = (size_t)perm[row0 + r] * H;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int h = h0 + 64 * wn + 32 * nb + (lane & 31);
          if (h < H) {
            if constexpr (OUT16) {
              y16[ybase + h] = f32_to_f16_bits(acc[mb][nb][j]);
            } else {
              y32[ybase + h] = acc[mb][nb][j];
            }
          }
        }
      }
    }
  }
}

// out[t, h] = sum_k w[t,k] * y[t*K + k, h] (+ shared[t, h]); Y is float or fp16 bits.
template <typename Y>
__global__ __launch_bounds__(256) void combine_kernel(const Y* __restrict__ y, const float* __restrict__ wts, int K,
                                                      int H, const float* __restrict__ shared,
                                                      void* __restrict__ out, int out32) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int k = 0; k < K; ++k) {
    const float wv = wts[(size_t)t * K + k];
    const size_t base = ((size_t)t * K + k) * H + h;
    float v0, v1, v2, v3;
    if constexpr (sizeof(Y) == 4) {
      const float4 v = *reinterpret_cast<const float4*>(y + base);
      v0 = v.x; v1 = v.y; v2 = v.z; v3 = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(y + base);
      v0 = f16_bits_to_f32((uint16_t)(v.x & 0xFFFFu));
      v1 = f16_bits_to_f32((uint16_t)(v.x >> 16));
      v2 = f16_bits_to_f32((uint16_t)(v.y & 0xFFFFu));
      v3 = f16_bits_to_f32((uint16_t)(v.y >> 16));
    }
    a0 += v0 * wv;
    a1 += v1 * wv;
    a2 += v2 * wv;
    a3 += v3 * wv;
  }
  if (shared) {
    const float4 s = *reinterpret_cast<const float4*>(shared + (size_t)t * H + h);
    a0 += s.x; a1 += s.y; a2 += s.z; a3 += s.w;
  }
  if (out32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + (size_t)t * H + h) = make_float4(a0, a1, a2, a3);
  } else {
    const uint32_t lo = (uint32_t)f32_to_f16_bits(a0) | ((uint32_t)f32_to_f16_bits(a1) << 16);
    const uint32_t hi = (uint32_t)f32_to_f16_bits(a2) | ((uint32_t)f32_to_f16_bits(a3) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + (size_t)t * H + h) = make_uint2(lo, hi);
  }
}

// ---- launchers --------------------------------------------------------------------------
template <int BITS, bool BF16, int ACT>
static hipError_t gemm_impl(const LayerConfig& c, const uint16_t* x, int T, const Work& w, int max_mtiles,
                            uint16_t* y16, hipStream_t s) {
  const LayerArgs& L = c.args;
  (void)T;
  KMOE_LAUNCH("gemm_gateup_kernel", (gemm_gateup_kernel<BITS, BF16, ACT>), dim3(max_mtiles * (L.I / 64)), dim3(256),
              0, s, L, x, c.top_k, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, w.act);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int n_ht = (L.H + 127) / 128;
  if (y16) {
    KMOE_LAUNCH("gemm_down_kernel", (gemm_down_kernel<BITS, BF16, true>), dim3(max_mtiles * n_ht), dim3(256), 0, s,
                L, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, w.act, (float*)nullptr, y16);
  } else {
    KMOE_LAUNCH("gemm_down_kernel", (gemm_down_kernel<BITS, BF16, false>), dim3(max_mtiles * n_ht), dim3(256), 0, s,
                L, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, w.act, w.y32, (uint16_t*)nullptr);
  }
  return hipGetLastError();
}

hipError_t launch_gemm(const LayerConfig& c, const uint16_t* x, int T, const Work& w, int max_mtiles, uint16_t* y16,
                       hipStream_t s) {
  if (max_mtiles == 0) return hipSuccess;
  if (c.bits == 3) {
    if (c.bf16_scales)
      return c.act ? gemm_impl<3, true, 1>(c, x, T, w, max_mtiles, y16, s) : gemm_impl<3, true, 0>(c, x, T, w, max_mtiles, y16, s);
    return c.act ? gemm_impl<3, false, 1>(c, x, T, w, max_mtiles, y16, s) : gemm_impl<3, false, 0>(c, x, T, w, max_mtiles, y16, s);
  }
  if (c.bf16_scales)
    return c.act ? gemm_impl<4, true, 1>(c, x, T, w, max_mtiles, y16, s) : gemm_impl<4, true, 0>(c, x, T, w, max_mtiles, y16, s);
  return c.act ? gemm_impl<4, false, 1>(c, x, T, w, max_mtiles, y16, s) : gemm_impl<4, false, 0>(c, x, T, w, max_mtiles, y16, s);
}

hipError_t launch_combine(const float* y32, const float* wts, int T, int K, int H, const float* shared,
                          void* out, int out32, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const dim3 grid((H / 4 + 255) / 256, T);
  KMOE_LAUNCH("combine_kernel", combine_kernel<float>, grid, dim3(256), 0, s, y32, wts, K, H, shared, out, out32);
  return hipGetLastError();
}

hipError_t launch_combine16(const uint16_t* y16, const float* wts, int T, int K, int H, uint16_t* out, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const dim3 grid((H / 4 + 255) / 256, T);
  KMOE_LAUNCH("combine_kernel", combine_kernel<uint16_t>, grid, dim3(256), 0, s, y16, wts, K, H, (const float*)nullptr,
                     (void*)out, 0);
  return hipGetLastError();
}

}  // namespace kmoe
