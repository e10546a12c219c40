// Dense fp16 shared expert of a MoE layer: shared_out[t] = down (silu(gate x_t) * (up x_t)),
// ungated, added to the routed combine (the always-on expert of the hidden-2560 layer; the
// reference adds it after the routed experts, moe_block.metal:515-539 blend_kernel with the
// shared term, full_forward_lg.m:1635-1735).  Weights: gate/up [Is][H], down [H][Is], fp16.
//
// Decode (1..8 tokens): bandwidth-bound GEMVs.
//   sh_gateup_gemv_kernel: x of all tokens staged in LDS; each wave streams SH_RW gate rows
//     and the same up rows (one 32-wide chunk per lane per step), v_dot2_f32_f16 against x,
//     DPP wave sums, act = silu(g)*u written as two fp16 planes (hi, lo).
//   sh_down_gemv_kernel: LPR lanes per down row (the chunk count rounded up to a power of
//     two), each lane dots its chunk with act hi + lo of every token; fp32 shared_out.
// Prefill: sh_gemm_kernel, a dense fp16 MFMA GEMM (128x128 tiles, 64-wide k steps, two k
//   steps of loads in flight), once for gate/up with the SwiGLU epilogue (act fp16 [T][Is])
//   and once for down (fp32 shared_out [T][H]).
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

constexpr int SH_RW = 2;  // gate/up rows per wave in the decode GEMV

template <int ACT>
__device__ __forceinline__ float sh_activate(float g, float u) {
  if constexpr (ACT == 0) {
    return silu_f32(g) * u;
  } else {
    return gelu_tanh_f32(g) * u;
  }
}

__device__ __forceinline__ void ld16(const void* p, uint32_t (&v)[16]) {
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

__device__ __forceinline__ float dot32(const uint32_t (&w)[16], const uint32_t (&x)[16], float acc) {
#pragma unroll
  for (int m = 0; m < 16; ++m) acc = fdot2(w[m], x[m], acc);
  return acc;
}

template <int ACT, int NT>
__global__ __launch_bounds__(256) void sh_gateup_gemv_kernel(const uint16_t* __restrict__ x, int T, int H, int Is,
                                                             const uint16_t* __restrict__ gate,
                                                             const uint16_t* __restrict__ up,
                                                             uint16_t* __restrict__ act, size_t plane) {
  extern __shared__ uint32_t xs[];  // [T][H/2] dwords (fp16 pairs, natural order)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int hw = H / 2;
  for (int i = tid; i < T * hw / 4; i += 256)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(x)[i];
  __syncthreads();
  const int i0 = (blockIdx.x * 4 + wave) * SH_RW;
  const int nch = H / CHUNK;
  float ag[SH_RW][NT], au[SH_RW][NT];
#pragma unroll
  for (int r = 0; r < SH_RW; ++r)
#pragma unroll
    for (int j = 0; j < NT; ++j) ag[r][j] = au[r][j] = 0.f;
  for (int c = lane; c < nch; c += 64) {
    uint32_t g[SH_RW][16], u[SH_RW][16];
#pragma unroll
    for (int r = 0; r < SH_RW; ++r) {
      ld16(gate + (size_t)(i0 + r) * H + (size_t)c * CHUNK, g[r]);
      ld16(up + (size_t)(i0 + r) * H + (size_t)c * CHUNK, u[r]);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if (j < T) {
        uint32_t xv[16];
        const uint4* src = reinterpret_cast<const uint4*>(xs + (size_t)j * hw + (size_t)c * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint4 t4 = src[q];
          xv[4 * q] = t4.x;
          xv[4 * q + 1] = t4.y;
          xv[4 * q + 2] = t4.z;
          xv[4 * q + 3] = t4.w;
        }
#pragma unroll
        for (int r = 0; r < SH_RW; ++r) {
          ag[r][j] = dot32(g[r], xv, ag[r][j]);
          au[r][j] = dot32(u[r], xv, au[r][j]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < SH_RW; ++r) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if (j < T) {
        const float gs = wave_sum_dpp(ag[r][j]);
        const float us = wave_sum_dpp(au[r][j]);
        if (lane == 0) {
          const float a = sh_activate<ACT>(gs, us);
          const _Float16 hi = (_Float16)a;
          const _Float16 lo = (_Float16)(a - (float)hi);
          const size_t o = (size_t)j * Is + i0 + r;
          act[o] = __builtin_bit_cast(uint16_t, hi);
          act[plane + o] = __builtin_bit_cast(uint16_t, lo);
        }
      }
    }
  }
}

template <int NT>
__global__ __launch_bounds__(256) void sh_down_gemv_kernel(const uint16_t* __restrict__ act, size_t plane, int T,
                                                           int H, int Is, const uint16_t* __restrict__ down,
                                                           float* __restrict__ out, int lpr_log2) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int LPR = 1 << lpr_log2, RPW = 64 >> lpr_log2;
  const int h = (blockIdx.x * 4 + wave) * RPW + (lane >> lpr_log2);
  const int cl = lane & (LPR - 1);
  const int nch = Is / CHUNK;
  float acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = 0.f;
  if (h < H) {
    for (int c = cl; c < nch; c += LPR) {
      uint32_t d[16];
      ld16(down + (size_t)h * Is + (size_t)c * CHUNK, d);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < T) {
          uint32_t ah[16], al[16];
          ld16(act + (size_t)j * Is + (size_t)c * CHUNK, ah);
          ld16(act + plane + (size_t)j * Is + (size_t)c * CHUNK, al);
          acc[j] = dot32(d, al, dot32(d, ah, acc[j]));
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const float v = group_sum_last(acc[j], LPR);
    if (h < H && j < T && cl == LPR - 1) out[(size_t)j * H + h] = v;
  }
}

// ---- prefill: dense fp16 GEMM -------------------------------------------------------------
constexpr int SBM = 128, SBK = 64, SLD = 72;

__device__ __forceinline__ float16_t sh_mfma(const half8_t a, const half8_t b, const float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// C[m][n] = sum_k A[m][k] * B[n][k] over a 128 x 128 tile.  GATEUP: B rows 0..63 are gate
// rows i0.., 64..127 the same up rows, and the epilogue writes act[m][i] = act(g, u) as fp16;
// otherwise B = down rows n0.. and the epilogue writes fp32 out[m][n].
template <bool GATEUP, int ACT>
__global__ __launch_bounds__(256, 3) void sh_gemm_kernel(const uint16_t* __restrict__ A, int M, int Kd,
                                                         const uint16_t* __restrict__ B0,
                                                         const uint16_t* __restrict__ B1, int N,
                                                         uint16_t* __restrict__ act_out, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) _Float16 sA[SBM * SLD];
  __shared__ __attribute__((aligned(16))) _Float16 sB[128 * SLD];
  const int ncol = GATEUP ? N / 64 : (N + 127) / 128;  // N = Is (GATEUP) or H
  const int mt = blockIdx.x / ncol, ct = blockIdx.x - mt * ncol;
  const int m0 = mt * SBM;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = tid >> 1, lc = tid & 1;
  const int arow_i = min(m0 + lr, M - 1);  // rows past M load row M-1 (never stored)
  const uint16_t* arow = A + (size_t)arow_i * Kd;
  int brow_i;
  const uint16_t* bsrc;
  if constexpr (GATEUP) {
    brow_i = ct * 64 + (lr & 63);
    bsrc = lr < 64 ? B0 : B1;
  } else {
    brow_i = min(ct * 128 + lr, N - 1);
    bsrc = B0;
  }
  const uint16_t* brow = bsrc + (size_t)brow_i * Kd;

  float16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  struct Stg {
    uint32_t a[16], b[16];
  };
  auto load = [&](Stg& S, int k0) {
    ld16(arow + k0 + lc * CHUNK, S.a);
    ld16(brow + k0 + lc * CHUNK, S.b);
  };
  auto store = [&](const Stg& S) {
    uint4* da = reinterpret_cast<uint4*>(sA + lr * SLD + lc * CHUNK);
    uint4* db = reinterpret_cast<uint4*>(sB + lr * SLD + lc * CHUNK);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      da[q] = make_uint4(S.a[4 * q], S.a[4 * q + 1], S.a[4 * q + 2], S.a[4 * q + 3]);
      db[q] = make_uint4(S.b[4 * q], S.b[4 * q + 1], S.b[4 * q + 2], S.b[4 * q + 3]);
    }
  };
  auto mma = [&]() {
#pragma unroll
    for (int ks = 0; ks < SBK / 16; ++ks) {
      const int koff = ks * 16 + (lane >> 5) * 8;
      const half8_t a0 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + (lane & 31)) * SLD + koff);
      const half8_t a1 = *reinterpret_cast<const half8_t*>(sA + (64 * wm + 32 + (lane & 31)) * SLD + koff);
      half8_t b0, b1;
      if constexpr (GATEUP) {  // wave wn: gate cols 32wn.., up cols 32wn..
        b0 = *reinterpret_cast<const half8_t*>(sB + (32 * wn + (lane & 31)) * SLD + koff);
        b1 = *reinterpret_cast<const half8_t*>(sB + (64 + 32 * wn + (lane & 31)) * SLD + koff);
      } else {
        b0 = *reinterpret_cast<const half8_t*>(sB + (64 * wn + (lane & 31)) * SLD + koff);
        b1 = *reinterpret_cast<const half8_t*>(sB + (64 * wn + 32 + (lane & 31)) * SLD + koff);
      }
      acc[0][0] = sh_mfma(a0, b0, acc[0][0]);
      acc[0][1] = sh_mfma(a0, b1, acc[0][1]);
      acc[1][0] = sh_mfma(a1, b0, acc[1][0]);
      acc[1][1] = sh_mfma(a1, b1, acc[1][1]);
    }
  };
  const int nk = Kd / SBK;
  Stg S0, S1;
  load(S0, 0);
  if (nk > 1) load(S1, SBK);
  for (int kk = 0; kk < nk; kk += 2) {
    store(S0);
    __syncthreads();
    if (kk + 2 < nk) load(S0, (kk + 2) * SBK);
    mma();
    __syncthreads();
    if (kk + 1 < nk) {
      store(S1);
      __syncthreads();
      if (kk + 3 < nk) load(S1, (kk + 3) * SBK);
      mma();
      __syncthreads();
    }
  }
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int m = m0 + 64 * wm + 32 * mb + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
      if (m < M) {
        if constexpr (GATEUP) {
          const int i = ct * 64 + 32 * wn + (lane & 31);
          act_out[(size_t)m * N + i] = f32_to_f16_bits(sh_activate<ACT>(acc[mb][0][j], acc[mb][1][j]));
        } else {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const int n = ct * 128 + 64 * wn + 32 * nb + (lane & 31);
            if (n < N) out[(size_t)m * N + n] = acc[mb][nb][j];
          }
        }
      }
    }
  }
}

// ---- launcher -----------------------------------------------------------------------------
template <int ACT, int NT>
static hipError_t shared_decode(const LayerConfig& c, const uint16_t* x, int T, const Work& w, hipStream_t s) {
  const LayerArgs& L = c.args;
  const size_t plane = (size_t)T * L.Is;
  const size_t lds = (size_t)T * L.H * 2;
  const void* k1 = reinterpret_cast<const void*>(&sh_gateup_gemv_kernel<ACT, NT>);
  if (lds > 65536) {
    hipError_t ae = hipFuncSetAttribute(k1, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (ae != hipSuccess) return ae;
  }
  KMOE_LAUNCH("sh_gateup_gemv_kernel", (sh_gateup_gemv_kernel<ACT, NT>), dim3(L.Is / (4 * SH_RW)), dim3(256),
              (uint32_t)lds, s, x, T, L.H, L.Is, L.sh_gate, L.sh_up, w.shared_act, plane);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  int l2 = 0;
  while ((1 << l2) < L.Is / CHUNK && l2 < 6) ++l2;
  const int rows_per_wg = 4 * (64 >> l2);
  KMOE_LAUNCH("sh_down_gemv_kernel", (sh_down_gemv_kernel<NT>), dim3((L.H + rows_per_wg - 1) / rows_per_wg),
              dim3(256), 0, s, (const uint16_t*)w.shared_act, plane, T, L.H, L.Is, L.sh_down, w.shared_out, l2);
  return hipGetLastError();
}

template <int ACT>
static hipError_t shared_prefill(const LayerConfig& c, const uint16_t* x, int T, const Work& w, hipStream_t s) {
  const LayerArgs& L = c.args;
  const int nmt = (T + SBM - 1) / SBM;
  KMOE_LAUNCH("sh_gemm_kernel", (sh_gemm_kernel<true, ACT>), dim3(nmt * (L.Is / 64)), dim3(256), 0, s, x, T, L.H,
              L.sh_gate, L.sh_up, L.Is, w.shared_act, (float*)nullptr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  KMOE_LAUNCH("sh_gemm_kernel", (sh_gemm_kernel<false, ACT>), dim3(nmt * ((L.H + 127) / 128)), dim3(256), 0, s,
              (const uint16_t*)w.shared_act, T, L.Is, L.sh_down, (const uint16_t*)nullptr, L.H, (uint16_t*)nullptr,
              w.shared_out);
  return hipGetLastError();
}

hipError_t launch_shared(const LayerConfig& c, const uint16_t* x, int T, const Work& w, hipStream_t s) {
  if (T == 0) return hipSuccess;
  if (T <= DEC_MAX_TOKENS) {
    const int nt = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8;
    if (c.act) {
      switch (nt) {
        case 1: return shared_decode<1, 1>(c, x, T, w, s);
        case 2: return shared_decode<1, 2>(c, x, T, w, s);
        case 4: return shared_decode<1, 4>(c, x, T, w, s);
        default: return shared_decode<1, 8>(c, x, T, w, s);
      }
    }
    switch (nt) {
      case 1: return shared_decode<0, 1>(c, x, T, w, s);
      case 2: return shared_decode<0, 2>(c, x, T, w, s);
      case 4: return shared_decode<0, 4>(c, x, T, w, s);
      default: return shared_decode<0, 8>(c, x, T, w, s);
    }
  }
  return c.act ? shared_prefill<1>(c, x, T, w, s) : shared_prefill<0>(c, x, T, w, s);
}

}  // namespace kmoe
