// Prefill path: grouped GEMM over the expert-sorted assignments with fp16 MFMA.
//
// Replaces the reference's 4-bit prefill (kandiga/engine.py:386-516: permutation, one
// Metal dispatch for gate+up+SiLU over every (assignment, row), one for down, then a
// scatter back to [T, K, H]) and its 3-bit fallback (engine.py:720-735: T sequential
// CPU calls).
//
//   xpair_kernel: x into pair order once per call (the k order the dequantized weights have).
//   gemm_gateup_kernel: one workgroup per (m-tile of <= 128 sorted assignments of one
//     expert, 64 intermediate columns).  Per 64-wide k step the workgroup gathers the
//     tile's x rows (token = assignment / K, already in pair order) into LDS, dequantizes the 64
//     gate rows and 64 up rows of that k step into LDS as fp16 (one quant group per row,
//     round(q*s + b) by one fp16 fma), and runs v_mfma_f32_32x32x16_f16.  Each wave owns
//     64 rows x 32 columns of both gate and up, so SwiGLU is applied in registers and
//     act is written once (fp16, pair order for the down projection's k dimension).
//     Every loader thread keeps two further k steps of global loads in flight in
//     registers while the current step is multiplied out of LDS.
//   gemm_down_kernel: one workgroup per (m-tile, 128 output columns); A = act rows of the
//     tile (already contiguous and in pair order), B = dequantized down rows, same
//     pipeline.  The output row of sorted position p is written, as fp16, to assignment
//     perm[p]: fp16 for the switch_mlp contract, or fp32 scaled by that assignment's routing
//     weight for the fused layer (an fp16 intermediate would add up to half an fp16 ulp of
//     each term before the combine, which the 2e-2 bound cannot absorb when terms cancel).
//   Tiles are ordered so that the column tiles of one m-tile, and the m-tiles of one
//   expert, run on the same XCD and share its L2.
//   combine_kernel: out[t] = sum_k w[t,k] * y[t,k] (+ shared expert), fp32 accumulate in
//     k order, one rounding to the output type (moe_block.metal:515-539).
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

// Load one chunk of packed codes through the caches (weights of one expert are read by every
// m-tile of that expert, so prefill keeps them in L2; decode streams them nontemporally).
template <int BITS>
__device__ __forceinline__ void load_chunk_c(const uint8_t* __restrict__ row, int chunk, uint32_t (&d)[4]) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(row + (size_t)chunk * Bits<BITS>::chunk_bytes);
  if constexpr (BITS == 3) {
    d[0] = src[0];
    d[1] = src[1];
    d[2] = src[2];
    d[3] = 0;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(src);
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
  }
}

// Dequantize loaded codes of one 32-code chunk into 16 fp16 pairs (pair order).
template <int BITS, bool BF16>
__device__ __forceinline__ void dequant_regs(const uint32_t (&d)[4], uint16_t sbits, uint16_t bbits,
                                             uint32_t (&out)[16]) {
  const float sf = scale_to_f32<BF16>(sbits), bf = scale_to_f32<BF16>(bbits);
  const half2_t s2 = {(_Float16)sf, (_Float16)sf}, b2 = {(_Float16)bf, (_Float16)bf};
  unpack_chunk<BITS, true>(d, out);
#pragma unroll
  for (int p = 0; p < 16; ++p) out[p] = dequant_pair(out[p], s2, b2);
}

__device__ __forceinline__ float16_t mfma32(const half8_t a, const half8_t b, const float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Tile index (m-tile * ncol + column tile) of workgroup b.  Workgroups are dealt to the 8 XCDs
// round-robin (XCD x runs b = x, x+8, ...); XCD x takes m-tiles x, x+8, ... and runs all column
// tiles of one m-tile back to back, so the gathered rows of an m-tile are fetched into one L2
// and the valid m-tiles (a prefix of the grid) are spread evenly over the XCDs.  The grid
// holds a multiple of 8 m-tiles.
__device__ __forceinline__ int xcd_tile(int b, int ncol) {
  const int x = b & 7, j = b >> 3;
  return ((j / ncol) * 8 + x) * ncol + (j % ncol);
}

// Registers of one k step (64 wide) of one loader thread: an A chunk and a B chunk.
struct KStage {
  uint32_t a[16];
  uint32_t w[4];
  uint16_t s, b;
};

// x [T][H] -> pair order within each 32-wide chunk (the k order of the dequantized weights).
template <int BITS>
__global__ __launch_bounds__(256) void xpair_kernel(const uint16_t* __restrict__ x, size_t nchunks,
                                                    uint16_t* __restrict__ xpp) {
  const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= nchunks) return;
  uint32_t nat[16], pr[16];
  load16g(x + c * CHUNK, nat);
  to_pair_order<BITS>(nat, pr);
  store16s(reinterpret_cast<_Float16*>(xpp + c * CHUNK), pr);
}

template <int BITS, bool BF16, int ACT>
__global__ __launch_bounds__(256, 3) void gemm_gateup_kernel(const LayerArgs L, const uint16_t* __restrict__ x,
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
  const int q = xcd_tile(blockIdx.x, n_it);
  const int mt = q / n_it, it = q - mt * n_it;
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
      for (int qq = 0; qq < 16; ++qq) acc[i][j][qq] = 0.f;

  // rows past the end of the tile read token 0's x (their results are never stored)
  auto load = [&](KStage& S, int k0) {
    load16g(xrow + k0 + lc * CHUNK, S.a);
    load_chunk_c<BITS>(wrow, (k0 >> 5) + lc, S.w);
    S.s = srow[k0 >> 6];
    S.b = bsrow[k0 >> 6];
  };
  auto store = [&](const KStage& S) {
    uint32_t pb[16];
    dequant_regs<BITS, BF16>(S.w, S.s, S.b, pb);
    store16s(sA + lr * LDH + lc * CHUNK, S.a);
    store16s(sB + lr * LDH + lc * CHUNK, pb);
  };
  auto mma = [&]() {
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
  };
  // two k steps of loads in flight: while step k is multiplied out of LDS, the registers of
  // steps k+1 and k+2 are being filled (unrolled by two so no stage register is copied)
  const int nk = H / BK;
  KStage S0, S1;
  load(S0, 0);
  if (nk > 1) load(S1, BK);
  for (int kk = 0; kk < nk; kk += 2) {
    store(S0);
    __syncthreads();
    if (kk + 2 < nk) load(S0, (kk + 2) * BK);
    mma();
    __syncthreads();
    if (kk + 1 < nk) {
      store(S1);
      __syncthreads();
      if (kk + 3 < nk) load(S1, (kk + 3) * BK);
      mma();
      __syncthreads();
    }
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
__global__ __launch_bounds__(256, 3) void gemm_down_kernel(const LayerArgs L, const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ scalars,
                                                           const int32_t* __restrict__ mt_expert,
                                                           const int32_t* __restrict__ mt_row0,
                                                           const int32_t* __restrict__ mt_rows,
                                                           const uint16_t* __restrict__ act,
                                                           const float* __restrict__ wscale,
                                                           float* __restrict__ y32, uint16_t* __restrict__ y16) {
  constexpr int BN = 128;
  __shared__ __attribute__((aligned(16))) _Float16 sA[GEMM_BM * LDH];
  __shared__ __attribute__((aligned(16))) _Float16 sB[BN * LDH];
  __shared__ int32_t s_asg[GEMM_BM];  // assignment of each tile row, and its routing weight
  __shared__ float s_wa[GEMM_BM];
  const int H = L.H, I = L.I;
  const int n_ht = (H + BN - 1) / BN;
  const int q = xcd_tile(blockIdx.x, n_ht);
  const int mt = q / n_ht, ht = q - mt * n_ht;
  if (mt >= scalars[1]) return;
  const int e = mt_expert[mt], row0 = mt_row0[mt], nrows = mt_rows[mt];
  const int h0 = ht * BN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  const int lr = tid >> 1, lc = tid & 1;
  const bool a_ok = lr < nrows;
  const uint16_t* arow = act + (size_t)(row0 + (a_ok ? lr : 0)) * I;
  if (tid < GEMM_BM) {  // epilogue metadata, fetched while the k loop runs (read after its barriers)
    const int a = tid < nrows ? perm[row0 + tid] : 0;
    s_asg[tid] = a;
    s_wa[tid] = wscale && tid < nrows ? wscale[a] : 1.0f;
  }
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
      for (int qq = 0; qq < 16; ++qq) acc[i][j][qq] = 0.f;

  // rows past the end of the tile read the tile's first act row (their results are never stored)
  auto load = [&](KStage& S, int k0) {
    load16g(arow + k0 + lc * CHUNK, S.a);
    load_chunk_c<BITS>(wrow, (k0 >> 5) + lc, S.w);
    S.s = srow[k0 >> 6];
    S.b = bsrow[k0 >> 6];
  };
  auto store = [&](const KStage& S) {
    uint32_t pb[16];
    if (b_ok) {
      dequant_regs<BITS, BF16>(S.w, S.s, S.b, pb);
    } else {
#pragma unroll
      for (int qq = 0; qq < 16; ++qq) pb[qq] = 0u;
    }
    store16s(sA + lr * LDH + lc * CHUNK, S.a);
    store16s(sB + lr * LDH + lc * CHUNK, pb);
  };
  auto mma = [&]() {
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
  };
  const int nk = I / BK;
  KStage S0, S1;
  load(S0, 0);
  if (nk > 1) load(S1, BK);
  for (int kk = 0; kk < nk; kk += 2) {
    store(S0);
    __syncthreads();
    if (kk + 2 < nk) load(S0, (kk + 2) * BK);
    mma();
    __syncthreads();
    if (kk + 1 < nk) {
      store(S1);
      __syncthreads();
      if (kk + 3 < nk) load(S1, (kk + 3) * BK);
      mma();
      __syncthreads();
    }
  }
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 64 * wm + 32 * mb + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
      if (r < nrows) {
        const size_t ybase = (size_t)s_asg[r] * H;
        const float wa = s_wa[r];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int h = h0 + 64 * wn + 32 * nb + (lane & 31);
          if (h < H) {
            if constexpr (OUT16) {
              y16[ybase + h] = f32_to_f16_bits(acc[mb][nb][j] * wa);
            } else {
              y32[ybase + h] = acc[mb][nb][j] * wa;
            }
          }
        }
      }
    }
  }
}

// out[t, h] = sum_k w[t,k] * y[t*K + k, h] (+ shared[t, h]), fp32 accumulation in k order.
// Y = float (the fused layer's fp32 rows, already scaled by their routing weights: wts is null)
// or uint16_t (fp16 bits of switch_mlp outputs, weighted here).
template <typename Y>
__global__ __launch_bounds__(256) void combine_kernel(const Y* __restrict__ y, const float* __restrict__ wts, int K,
                                                      int H, const float* __restrict__ shared,
                                                      void* __restrict__ out, int out32) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int k = 0; k < K; ++k) {
    const float wv = wts ? wts[(size_t)t * K + k] : 1.0f;
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
    const float4 sv = *reinterpret_cast<const float4*>(shared + (size_t)t * H + h);
    a0 += sv.x; a1 += sv.y; a2 += sv.z; a3 += sv.w;
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
                            uint16_t* y16, const float* wscale, hipStream_t s) {
  const LayerArgs& L = c.args;
  (void)T;
  const int gmt = (max_mtiles + 7) & ~7;  // m-tiles of the grid: a multiple of 8 (see xcd_tile)
  KMOE_LAUNCH("gemm_gateup_kernel", (gemm_gateup_kernel<BITS, BF16, ACT>), dim3(gmt * (L.I / 64)), dim3(256),
              0, s, L, x, c.top_k, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, w.act);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int n_ht = (L.H + 127) / 128;
  if (y16) {
    KMOE_LAUNCH("gemm_down_kernel", (gemm_down_kernel<BITS, BF16, true>), dim3(gmt * n_ht), dim3(256), 0, s,
                L, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, (const uint16_t*)w.act, wscale,
                (float*)nullptr, y16);
  } else {
    KMOE_LAUNCH("gemm_down_kernel", (gemm_down_kernel<BITS, BF16, false>), dim3(gmt * n_ht), dim3(256), 0, s,
                L, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, (const uint16_t*)w.act, wscale, w.y32,
                (uint16_t*)nullptr);
  }
  return hipGetLastError();
}

hipError_t launch_gemm(const LayerConfig& c, const uint16_t* x, int T, const Work& w, int max_mtiles, uint16_t* y16,
                       const float* wscale, hipStream_t s) {
  if (max_mtiles == 0) return hipSuccess;
  if (c.bits == 3) {
    if (c.bf16_scales)
      return c.act ? gemm_impl<3, true, 1>(c, x, T, w, max_mtiles, y16, wscale, s) : gemm_impl<3, true, 0>(c, x, T, w, max_mtiles, y16, wscale, s);
    return c.act ? gemm_impl<3, false, 1>(c, x, T, w, max_mtiles, y16, wscale, s) : gemm_impl<3, false, 0>(c, x, T, w, max_mtiles, y16, wscale, s);
  }
  if (c.bf16_scales)
    return c.act ? gemm_impl<4, true, 1>(c, x, T, w, max_mtiles, y16, wscale, s) : gemm_impl<4, true, 0>(c, x, T, w, max_mtiles, y16, wscale, s);
  return c.act ? gemm_impl<4, false, 1>(c, x, T, w, max_mtiles, y16, wscale, s) : gemm_impl<4, false, 0>(c, x, T, w, max_mtiles, y16, wscale, s);
}

hipError_t launch_xpair(const LayerConfig& c, const uint16_t* x, int T, uint16_t* xpp, hipStream_t s) {
  const size_t nchunks = (size_t)T * c.args.H / CHUNK;
  if (nchunks == 0) return hipSuccess;
  const dim3 grid((unsigned)((nchunks + 255) / 256));
  if (c.bits == 3) {
    KMOE_LAUNCH("xpair_kernel", xpair_kernel<3>, grid, dim3(256), 0, s, x, nchunks, xpp);
  } else {
    KMOE_LAUNCH("xpair_kernel", xpair_kernel<4>, grid, dim3(256), 0, s, x, nchunks, xpp);
  }
  return hipGetLastError();
}

hipError_t launch_combine(const float* y32, const uint16_t* y16, const float* wts, int T, int K, int H,
                          const float* shared, void* out, int out32, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const dim3 grid((H / 4 + 255) / 256, T);
  if (y32) {
    KMOE_LAUNCH("combine_kernel", combine_kernel<float>, grid, dim3(256), 0, s, y32, wts, K, H, shared, out, out32);
  } else {
    KMOE_LAUNCH("combine_kernel", combine_kernel<uint16_t>, grid, dim3(256), 0, s, y16, wts, K, H, shared, out,
                out32);
  }
  return hipGetLastError();
}

}  // namespace kmoe
