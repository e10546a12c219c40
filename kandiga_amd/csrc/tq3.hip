// TQ3 codebook GEMV (kandiga/tq3/fused_kernel.py:170-251 tq3_gemv, kandiga/tq3/tq3_metal.metal:55-141
// tq3_matvec / tq3_rotate_activations) and the switch_mlp contract over TQ3 experts.
//
// A TQ3 block is 32 weights in 20 bytes: fp16 d0 d1 m0 m1, then 12 bytes of 3-bit codebook
// indices (index r of 3-byte group g at bits 3r..3r+2 of b0 | b1<<8 | b2<<16).  The weights are
// w = S (H (C[q]*d + m)) / sqrt(32) per block (d, m of the block's half), so a row's dot with x is
//   sum_b  d0 * sum_{j<16} C[q_j] xr_j + m0 * sum_{j<16} xr_j + (the same for the upper half),
// with xr = H (S x_b) / sqrt(32) the rotated activation block.  Each workgroup rotates its input
// vector once into LDS (a 5-stage butterfly per 32-element block, in registers), then its waves
// take rows: LPR lanes per row (the row's block count rounded up to a power of two, at most 64),
// each lane its blocks' rotated values in registers, one 20-byte block per lane per row, the
// codebook in LDS; the lanes of a row are summed with DPP.
//
//   tq3_gemv_kernel<MODE>: out[v][r] = row r of the expert vexp[v]'s matrix applied to input
//     vector v.  MODE 0: fp16 input rows; 1: fp32 input rows; 2: the SwiGLU activation
//     silu(g) * u of an fp32 gate/up pair row [g | u] (the down projection of the expert MLP).
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

constexpr int TQ3_BLOCK = 32, TQ3_BYTES = 20;

__constant__ float c_tq3_cent[8] = {-1.996684f, -1.291398f, -0.740341f, -0.247508f,
                                    0.230106f,  0.725222f,  1.277503f,  1.988943f};
__constant__ float c_tq3_sign[32] = {+1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1,
                                     -1, -1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1};

struct Tq3Gemv {
  const uint8_t* w;     // expert 0's body
  int64_t wstride;      // bytes between experts
  int64_t moff0, moff1; // offsets of the matrices inside a body: rows < rsplit use moff0, others
                        // moff1 (row - rsplit)
  int rsplit;
  const int32_t* vexp;  // expert of each input vector (null: expert 0)
  int E;
  const void* in;       // input rows; vector v reads row v / in_div
  int in_div;
  int V, R, C;
  int rows_per_wg;
  float* out32;         // [V][R] fp32, or
  uint16_t* out16;      // [V][R] fp16
};

template <int MODE>
__device__ __forceinline__ float tq3_in(const Tq3Gemv& P, int row, int c) {
  if constexpr (MODE == 0) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(P.in)[(size_t)row * P.C + c]);
  } else if constexpr (MODE == 1) {
    return static_cast<const float*>(P.in)[(size_t)row * P.C + c];
  } else {
    const float* gu = static_cast<const float*>(P.in) + (size_t)row * 2 * P.C;
    return silu_f32(gu[c]) * gu[P.C + c];
  }
}

template <int MODE, int CPL>
__global__ __launch_bounds__(256) void tq3_gemv_kernel(const Tq3Gemv P) {
  extern __shared__ float lds[];  // [C] rotated input, [C/16] half sums, [8] codebook
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int v = blockIdx.y;
  const int nb = P.C / TQ3_BLOCK;
  float* s_xr = lds;
  float* s_hs = lds + P.C;
  float* s_cent = s_hs + 2 * nb;
  const int e = P.vexp ? P.vexp[v] : 0;
  const bool valid = e >= 0 && e < P.E;
  const int irow = v / P.in_div;
  if (tid < 8) s_cent[tid] = c_tq3_cent[tid];
  for (int b = tid; b < nb; b += 256) {
    float r[TQ3_BLOCK];
#pragma unroll
    for (int j = 0; j < TQ3_BLOCK; ++j) r[j] = tq3_in<MODE>(P, irow, b * TQ3_BLOCK + j) * c_tq3_sign[j];
#pragma unroll
    for (int st = 1; st < TQ3_BLOCK; st <<= 1) {
#pragma unroll
      for (int j = 0; j < TQ3_BLOCK; ++j) {
        if ((j & st) == 0) {
          const float a = r[j], c = r[j + st];
          r[j] = a + c;
          r[j + st] = a - c;
        }
      }
    }
    float h0 = 0.f, h1 = 0.f;
#pragma unroll
    for (int j = 0; j < TQ3_BLOCK; ++j) {
      r[j] *= 0.17677669529663688f;  // 1/sqrt(32)
      s_xr[b * TQ3_BLOCK + j] = r[j];
      if (j < 16) h0 += r[j]; else h1 += r[j];
    }
    s_hs[2 * b] = h0;
    s_hs[2 * b + 1] = h1;
  }
  __syncthreads();
  int lpr = 1;
  while (lpr < nb && lpr < 64) lpr <<= 1;
  const int rpw = 64 / lpr;  // rows per wave at a time
  const int cl = lane & (lpr - 1), rl = lane / lpr;
  float xr[CPL][TQ3_BLOCK], hs[CPL][2];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int b = min(cl + k * lpr, nb - 1);
#pragma unroll
    for (int j = 0; j < TQ3_BLOCK; ++j) xr[k][j] = s_xr[b * TQ3_BLOCK + j];
    hs[k][0] = s_hs[2 * b];
    hs[k][1] = s_hs[2 * b + 1];
  }
  const uint8_t* body = P.w + (valid ? (size_t)e * P.wstride : 0);
  const int r0 = blockIdx.x * P.rows_per_wg;
  for (int rr = wave * rpw; rr < P.rows_per_wg; rr += 4 * rpw) {
    const int row = r0 + rr + rl;
    float acc = 0.f;
    if (row < P.R && valid) {
      const uint8_t* m = body + (row < P.rsplit ? P.moff0 + (int64_t)row * nb * TQ3_BYTES
                                                : P.moff1 + (int64_t)(row - P.rsplit) * nb * TQ3_BYTES);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const int b = cl + k * lpr;
        if (b < nb) {
          const uint32_t* q = reinterpret_cast<const uint32_t*>(m + (size_t)b * TQ3_BYTES);
          const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
          const float d0 = f16_bits_to_f32((uint16_t)(w0 & 0xFFFFu)), d1 = f16_bits_to_f32((uint16_t)(w0 >> 16));
          const float m0 = f16_bits_to_f32((uint16_t)(w1 & 0xFFFFu)), m1 = f16_bits_to_f32((uint16_t)(w1 >> 16));
          // the 12 index bytes: groups g = 0..3 at bits 24g of the 96-bit word w2 | w3<<32 | w4<<64
          const uint32_t g0 = w2 & 0xFFFFFFu, g1 = (w2 >> 24) | ((w3 & 0xFFFFu) << 8);
          const uint32_t g2 = (w3 >> 16) | ((w4 & 0xFFu) << 16), g3 = w4 >> 8;
          const uint32_t grp[4] = {g0, g1, g2, g3};
          float s0 = 0.f, s1 = 0.f;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float c = s_cent[(grp[g] >> (3 * i)) & 7u];
              if (g < 2) s0 = fmaf(c, xr[k][8 * g + i], s0);
              else s1 = fmaf(c, xr[k][8 * g + i], s1);
            }
          }
          acc += d0 * s0 + m0 * hs[k][0] + d1 * s1 + m1 * hs[k][1];
        }
      }
    }
    const float tot = group_sum_last(acc, lpr);
    if (cl == lpr - 1 && rr + rl < P.rows_per_wg && row < P.R) {
      if (P.out16)
        P.out16[(size_t)v * P.R + row] = f32_to_f16_bits(tot);
      else
        P.out32[(size_t)v * P.R + row] = tot;
    }
  }
}

hipError_t launch_tq3_gemv(const Tq3Params& a, int mode, hipStream_t s) {
  if (a.V == 0 || a.R == 0) return hipSuccess;
  if (a.C % TQ3_BLOCK || a.C > 4096) return hipErrorInvalidValue;
  Tq3Gemv P{a.w, a.wstride, a.moff0, a.moff1, a.rsplit, a.vexp, a.E, a.in, a.in_div, a.V, a.R, a.C, 0,
            a.out32, a.out16};
  const int nb = a.C / TQ3_BLOCK;
  int lpr = 1;
  while (lpr < nb && lpr < 64) lpr <<= 1;
  const int rows_step = 4 * (64 / lpr);  // rows a workgroup covers per pass of its waves
  // enough workgroups to cover the chip, each reusing its rotated input over a few passes
  int passes = 1;
  while (passes < 8 && (long long)a.V * ((a.R + rows_step * passes * 2 - 1) / (rows_step * passes * 2)) >= 1024)
    passes *= 2;
  P.rows_per_wg = rows_step * passes;
  const dim3 grid((a.R + P.rows_per_wg - 1) / P.rows_per_wg, a.V);
  const size_t lds = ((size_t)a.C + 2 * nb + 8) * sizeof(float);
  const bool two = nb > 64;
#define KMOE_TQ(M, CPLV) \
  KMOE_LAUNCH("tq3_gemv_kernel", (tq3_gemv_kernel<M, CPLV>), grid, dim3(256), (uint32_t)lds, s, P)
  if (mode == 0) {
    if (two) KMOE_TQ(0, 2); else KMOE_TQ(0, 1);
  } else if (mode == 1) {
    if (two) KMOE_TQ(1, 2); else KMOE_TQ(1, 1);
  } else {
    if (two) KMOE_TQ(2, 2); else KMOE_TQ(2, 1);
  }
#undef KMOE_TQ
  return hipGetLastError();
}

}  // namespace kmoe
