// TQ3 codebook GEMV (kandiga/tq3/fused_kernel.py:170-251 tq3_gemv, kandiga/tq3/tq3_metal.metal:55-141
// tq3_matvec / tq3_rotate_activations) and the switch_mlp contract over TQ3 experts.
//
// A TQ3 block is 32 weights in 20 bytes: fp16 d0 d1 m0 m1, then 12 bytes of 3-bit codebook
// indices (index r of 3-byte group g at bits 3r..3r+2 of b0 | b1<<8 | b2<<16).  The weights are
// w = S (H (C[q]*d + m)) / sqrt(32) per block (d, m of the block's half), so a row's dot with x is
//   sum_b  d0 * sum_{j<16} C[q_j] xr_j + m0 * sum_{j<16} xr_j + (the same for the upper half),
// with xr = H (S x_b) / sqrt(32) the rotated activation block.
//
//   tq3_gemv_kernel: rows of one TQ3 matrix (or gate/up row pairs with the SwiGLU output) against
//     one input vector per grid row.  Each workgroup issues its weight loads, then rotates the
//     input into LDS (a thread per 32-block, in registers; tq3_rotate_activations does this once
//     per token) while they are in flight.  LPR lanes per row (the row's block count rounded up to
//     a power of two, at most 64), each lane its blocks' rotated values in registers, one 20-byte
//     block per lane per row, UR rows of the wave loaded together; codebook in LDS; the lanes of a
//     row are summed with DPP.
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

constexpr int TQ3_BLOCK = 32, TQ3_BYTES = 20;

__constant__ float c_tq3_cent[8] = {-1.996684f, -1.291398f, -0.740341f, -0.247508f,
                                    0.230106f,  0.725222f,  1.277503f,  1.988943f};
__constant__ float c_tq3_sign[32] = {+1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1,
                                     -1, -1, +1, -1, +1, -1, -1, +1, -1, +1, +1, -1, +1, -1, -1, +1};

// r <- H (S r) / sqrt(32): sign flips, the 5-stage butterfly, the normalisation.
__device__ __forceinline__ void tq3_rotate32(float (&r)[32]) {
#pragma unroll
  for (int j = 0; j < TQ3_BLOCK; ++j) r[j] *= c_tq3_sign[j];
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
#pragma unroll
  for (int j = 0; j < TQ3_BLOCK; ++j) r[j] *= 0.17677669529663688f;  // 1/sqrt(32)
}

__device__ __forceinline__ void store_rotated(const float (&r)[32], float* xr, float* hs) {
  float h0 = 0.f, h1 = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    h0 += r[j];
    h1 += r[16 + j];
  }
  float4* o = reinterpret_cast<float4*>(xr);
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
  hs[0] = h0;
  hs[1] = h1;
}

// The rotated blocks a lane multiplies: blocks cl + LPR*k of one input vector.
template <int CPL>
struct Tq3X {
  float x[CPL][32];
  float h[CPL][2];
};

template <int CPL>
__device__ __forceinline__ void load_lane_x(const float* __restrict__ xr, const float* __restrict__ hs, int cl,
                                            int lpr, int nb, Tq3X<CPL>& X) {
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int b = min(cl + k * lpr, nb - 1);  // lanes past the row's end reload its last block (unused)
    const float4* p = reinterpret_cast<const float4*>(xr + (size_t)b * TQ3_BLOCK);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = p[q];
      X.x[k][4 * q] = t.x;
      X.x[k][4 * q + 1] = t.y;
      X.x[k][4 * q + 2] = t.z;
      X.x[k][4 * q + 3] = t.w;
    }
    X.h[k][0] = hs[2 * b];
    X.h[k][1] = hs[2 * b + 1];
  }
}

// One lane's blocks of one row: raw 20-byte blocks (5 dwords each).
template <int CPL>
struct Tq3W {
  uint32_t w[CPL][5];
};

template <int CPL>
__device__ __forceinline__ void load_lane_w(const uint8_t* __restrict__ row, int cl, int lpr, int nb, bool on,
                                            Tq3W<CPL>& W) {
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int b = cl + k * lpr;
    if (on && b < nb) {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(row + (size_t)b * TQ3_BYTES);
#pragma unroll
      for (int i = 0; i < 5; ++i) W.w[k][i] = q[i];
    } else {
#pragma unroll
      for (int i = 0; i < 5; ++i) W.w[k][i] = 0u;  // d = m = 0: contributes nothing
    }
  }
}

// The lane's part of the row's dot: sum over its blocks of d0 s0 + m0 h0 + d1 s1 + m1 h1.
template <int CPL>
__device__ __forceinline__ float lane_dot(const Tq3W<CPL>& W, const Tq3X<CPL>& X, const float* s_cent) {
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const uint32_t w0 = W.w[k][0], w1 = W.w[k][1], w2 = W.w[k][2], w3 = W.w[k][3], w4 = W.w[k][4];
    const float d0 = f16_bits_to_f32((uint16_t)(w0 & 0xFFFFu)), d1 = f16_bits_to_f32((uint16_t)(w0 >> 16));
    const float m0 = f16_bits_to_f32((uint16_t)(w1 & 0xFFFFu)), m1 = f16_bits_to_f32((uint16_t)(w1 >> 16));
    // the 12 index bytes: groups g = 0..3 at bits 24g of the 96-bit word w2 | w3<<32 | w4<<64
    const uint32_t grp[4] = {w2 & 0xFFFFFFu, (w2 >> 24) | ((w3 & 0xFFFFu) << 8), (w3 >> 16) | ((w4 & 0xFFu) << 16),
                             w4 >> 8};
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float c = s_cent[(grp[g] >> (3 * i)) & 7u];
        if (g < 2) s0 = fmaf(c, X.x[k][8 * g + i], s0);
        else s1 = fmaf(c, X.x[k][8 * g + i], s1);
      }
    }
    acc += d0 * s0 + m0 * X.h[k][0] + d1 * s1 + m1 * X.h[k][1];
  }
  return acc;
}

// One block of input (32 values of an fp16 or fp32 row) rotated into LDS: xr and its half sums.
template <bool IN32>
__device__ __forceinline__ void rotate_block_to_lds(const void* in, size_t off, float* s_xr, float* s_hs, int b) {
  float r[32];
  if constexpr (IN32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(in) + off);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = p[q];
      r[4 * q] = t.x;
      r[4 * q + 1] = t.y;
      r[4 * q + 2] = t.z;
      r[4 * q + 3] = t.w;
    }
  } else {
    uint32_t w[16];
    load16g(static_cast<const uint16_t*>(in) + off, w);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      r[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xFFFFu));
      r[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
    }
  }
  tq3_rotate32(r);
  store_rotated(r, s_xr + b * TQ3_BLOCK, s_hs + 2 * b);
}

struct Tq3Gemv {
  const uint8_t* w;     // expert 0's matrix (expert e at w + e * wstride)
  int64_t wstride;
  int64_t up_off;       // PAIR: the up matrix's offset inside an expert
  const int32_t* vexp;  // expert of each input vector (null: expert 0)
  int E;
  const void* in;       // input rows [*][C] (fp16, or fp32 when IN32); vector v reads row v / in_div
  int in_div;
  int V, R, C;          // R output rows (PAIR: intermediate rows, two row dots each)
  int rows_per_wg;
  float* out32;         // [V][R] fp32 (PAIR: silu(gate) * up), or
  uint16_t* out16;      // [V][R] fp16
};

// out[v][r] for rows r of one workgroup: row r of expert vexp[v]'s matrix dotted with input row
// v / in_div, rotated into LDS by the workgroup (experts outside [0, E) give zeros).  PAIR: output
// r is silu(gate row r . x) * (up row r . x), the two dots in the same lanes.  Wave w takes row
// groups r0 + RPI*(w + 4j) (RPI = 64 / LPR rows at a time), UR groups per pass whose weight
// loads are in flight together: every weight load of the pass is issued before the input's
// rotation, so the rotation runs while they are in flight.
// The fields the first loads need lead the arguments as scalars, so gfx950 preloads them into
// SGPRs at wave launch (the library is built with kernel-argument preload).
template <int CPL, bool IN32, bool PAIR, int UR>
__global__ __launch_bounds__(256) void tq3_gemv_kernel(const uint8_t* __restrict__ w, const int32_t* __restrict__ vexp,
                                                       const void* __restrict__ in, int64_t wstride, int64_t up_off,
                                                       int E, int in_div, int R, int C, int rows_per_wg,
                                                       const Tq3Gemv P) {
  extern __shared__ float lds[];  // [C] rotated input, [C/16] half sums
  __shared__ float s_cent[8];
  constexpr int ND = PAIR ? 2 : 1;  // row dots per output row
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int v = blockIdx.y;
  const int nb = C / TQ3_BLOCK;
  float* s_xr = lds;
  float* s_hs = lds + C;
  if (tid < 8) s_cent[tid] = c_tq3_cent[tid];
  int lpr = 1;
  while (lpr < nb && lpr < 64) lpr <<= 1;
  const int rpi = 64 / lpr;
  const int cl = lane & (lpr - 1), rl = lane / lpr;
  const int e = vexp ? vexp[v] : 0;
  const bool valid = e >= 0 && e < E;
  const uint8_t* body = w + (valid ? (size_t)e * wstride : 0);
  const size_t rbytes = (size_t)nb * TQ3_BYTES;
  const int r0 = blockIdx.x * rows_per_wg;
  const int ir = v / in_div;
  bool first = true;
  for (int base = wave * rpi; base < rows_per_wg; base += 4 * rpi * UR) {
    Tq3W<CPL> W[UR][ND];
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int rr = base + 4 * rpi * u + rl, row = r0 + rr;
      const bool on = valid && rr < rows_per_wg && row < R;
#pragma unroll
      for (int q = 0; q < ND; ++q)
        load_lane_w<CPL>(body + (q ? up_off : 0) + (size_t)row * rbytes, cl, lpr, nb, on, W[u][q]);
    }
    if (first) {  // uniform: every wave takes at least one pass (rows_per_wg >= 4 * rpi)
      for (int b = tid; b < nb; b += 256)
        rotate_block_to_lds<IN32>(in, (size_t)ir * C + (size_t)b * TQ3_BLOCK, s_xr, s_hs, b);
      __syncthreads();
      first = false;
    }
    Tq3X<CPL> X;
    load_lane_x<CPL>(s_xr, s_hs, cl, lpr, nb, X);
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int rr = base + 4 * rpi * u + rl, row = r0 + rr;
      float tot = group_sum_last(lane_dot<CPL>(W[u][0], X, s_cent), lpr);
      if constexpr (PAIR) tot = silu_f32(tot) * group_sum_last(lane_dot<CPL>(W[u][1], X, s_cent), lpr);
      if (cl == lpr - 1 && rr < rows_per_wg && row < R) {
        if (P.out16)
          P.out16[(size_t)v * R + row] = f32_to_f16_bits(tot);
        else
          P.out32[(size_t)v * R + row] = tot;
      }
    }
  }
}

// ---- launchers ----------------------------------------------------------------------------
static int tq3_lpr(int nb) {
  int l = 1;
  while (l < nb && l < 64) l <<= 1;
  return l;
}

// in32: fp32 input rows; pair: gate/up pairs (P.up_off) with the SwiGLU output.
hipError_t launch_tq3_gemv(const Tq3Params& a, bool in32, bool pair, hipStream_t s) {
  if (a.V == 0 || a.R == 0) return hipSuccess;
  if (a.C % TQ3_BLOCK || a.C > 4096) return hipErrorInvalidValue;
  Tq3Gemv P{a.w, a.wstride, a.up_off, a.vexp, a.E, a.in, a.in_div, a.V, a.R, a.C, 0, a.out32, a.out16};
  const int nb = a.C / TQ3_BLOCK;
  // One pass of the four waves per workgroup, UR row groups each.  A grid that would stay under
  // 512 workgroups with four groups per wave takes two (twice the workgroups: one token's gate/up
  // 10.6 -> 8.8 us); a grid that stays at 1024 workgroups or more takes two or more passes.
  const int rpi = 64 / tq3_lpr(nb);
  auto wgs = [&](int rows) { return (long long)a.V * ((a.R + rows - 1) / rows); };
  const bool ur2 = wgs(16 * rpi) < 512;
  const int step = 4 * rpi * (ur2 ? 2 : 4);
  P.rows_per_wg = step;
  while (!ur2 && P.rows_per_wg < 8 * step && wgs(2 * P.rows_per_wg) >= 1024) P.rows_per_wg *= 2;
  const dim3 grid((a.R + P.rows_per_wg - 1) / P.rows_per_wg, a.V);
  const uint32_t lds = (uint32_t)(a.C + a.C / 16) * sizeof(float);
  // profiler names: the expert MLP's two launches apart
  const char* name = pair ? "tq3_gemv_kernel:gate_up" : in32 ? "tq3_gemv_kernel:down" : "tq3_gemv_kernel";
#define KMOE_TQ(CPLV, IN32V, PAIRV)                                                                 \
  do {                                                                                             \
    if (ur2)                                                                                       \
      KMOE_LAUNCH(name, (tq3_gemv_kernel<CPLV, IN32V, PAIRV, 2>), grid, dim3(256), lds, s, P.w, P.vexp, P.in, \
                  P.wstride, P.up_off, P.E, P.in_div, P.R, P.C, P.rows_per_wg, P);                        \
    else                                                                                                  \
      KMOE_LAUNCH(name, (tq3_gemv_kernel<CPLV, IN32V, PAIRV, 4>), grid, dim3(256), lds, s, P.w, P.vexp, P.in, \
                  P.wstride, P.up_off, P.E, P.in_div, P.R, P.C, P.rows_per_wg, P);                        \
  } while (0)
  if (nb > 64) {
    if (pair) KMOE_TQ(2, false, true);
    else if (in32) KMOE_TQ(2, true, false);
    else KMOE_TQ(2, false, false);
  } else {
    if (pair) KMOE_TQ(1, false, true);
    else if (in32) KMOE_TQ(1, true, false);
    else KMOE_TQ(1, false, false);
  }
#undef KMOE_TQ
  return hipGetLastError();
}

}  // namespace kmoe
