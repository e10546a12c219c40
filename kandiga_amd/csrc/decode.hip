// Decode path (1..8 tokens): bandwidth-bound dequant GEMVs over the distinct selected experts.
//
// Replaces the reference's per-token CPU expert MLP (kandiga/metal/kandiga_cpu_expert.m:
// 355-401 per expert, :471-552 for the K-way fan-out; kandiga/engine.py:727-735 loops it
// over tokens).  Every distinct expert selected by any token is read from HBM once per
// layer and applied to all tokens routed to it.
//
//   dec_gateup_kernel: grid = (distinct-expert slot, block of 4*RW intermediate rows).
//     x of the expert's tokens is staged in LDS in pair order with per-chunk sums; each
//     wave streams RW gate rows and the same RW up rows (one 32-code chunk per lane per
//     step, 12/16-byte loads), accumulates q*x with v_dot2_f32_f16 on raw codes and
//     applies s*2^24*dot + b*sum(x) per chunk, reduces across the wave and writes
//     act = silu(gate) * up (fp16, pair order) for every (expert, token) row.
//   dec_down_kernel: grid = blocks of 64/LPR output rows (LPR lanes per row).  The four
//     waves split the distinct experts; each lane accumulates w[t,k] * (down row . act)
//     per token, and the waves' partials are added in a fixed order in LDS, so the
//     combine (moe_block.metal:515-539) is fused and deterministic.  The per-assignment
//     variant writes y[t,k,:] instead (the switch_mlp contract, engine.py:670-739).
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

template <int BITS>
struct PairPosTable {
  uint8_t v[32];
};
template <int BITS>
constexpr PairPosTable<BITS> make_pair_pos() {
  PairPosTable<BITS> t{};
  for (int e = 0; e < 32; ++e) t.v[e] = (uint8_t)pair_pos(BITS, e);
  return t;
}
__constant__ PairPosTable<3> c_pairpos3 = make_pair_pos<3>();
__constant__ PairPosTable<4> c_pairpos4 = make_pair_pos<4>();

template <int BITS>
__device__ __forceinline__ int pairpos(int e) {
  if constexpr (BITS == 3) {
    return c_pairpos3.v[e];
  } else {
    return c_pairpos4.v[e];
  }
}

constexpr float TWO24 = 16777216.0f;
constexpr uint32_t ONE2 = 0x3C003C00u;  // fp16 pair (1, 1)

template <int ACT>
__device__ __forceinline__ float activate(float g, float u) {
  if constexpr (ACT == 0) {
    return silu_f32(g) * u;
  } else {
    return gelu_tanh_f32(g) * u;
  }
}

__device__ __forceinline__ void load16(const void* p, uint32_t (&v)[16]) {
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

template <int BITS, bool BF16, int ACT, int NT, int RW>
__global__ __launch_bounds__(256) void dec_gateup_kernel(const LayerArgs L, const uint16_t* __restrict__ x, int K,
                                                         const int32_t* __restrict__ perm,
                                                         const int32_t* __restrict__ ustart,
                                                         const int32_t* __restrict__ unique,
                                                         const int32_t* __restrict__ scalars,
                                                         uint16_t* __restrict__ act, size_t act_plane,
                                                         int wgs_per_expert) {
  extern __shared__ uint32_t smem[];
  const int u = blockIdx.x / wgs_per_expert;
  const int rb = blockIdx.x - u * wgs_per_expert;
  if (u >= scalars[0]) return;
  const int e = unique[u];
  const int p0 = ustart[u];
  const int na = min(ustart[u + 1] - p0, NT);
  const int H = L.H, I = L.I, nch = H / CHUNK;
  uint32_t* xs = smem;                                               // [NT][nch][16]
  float* xsum = reinterpret_cast<float*>(smem + (size_t)NT * nch * 16);  // [NT][nch]
  for (int task = threadIdx.x; task < na * nch; task += blockDim.x) {
    const int j = task / nch, c = task - j * nch;
    const int t = perm[p0 + j] / K;
    uint32_t nat[16], pr[16];
    load16(x + (size_t)t * H + (size_t)c * CHUNK, nat);
    to_pair_order<BITS>(nat, pr);
    uint4* dst = reinterpret_cast<uint4*>(xs + ((size_t)j * nch + c) * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(pr[4 * q], pr[4 * q + 1], pr[4 * q + 2], pr[4 * q + 3]);
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) s = fdot2(nat[m], ONE2, s);
    xsum[j * nch + c] = s;
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ib = rb * (4 * RW) + wave * RW;
  const size_t rbytes = (size_t)H * BITS / 8;
  const int ng = H / GROUP;
  const uint8_t* gw = L.gate.w + (size_t)e * L.gate.w_stride + (size_t)ib * rbytes;
  const uint8_t* uw = L.up.w + (size_t)e * L.up.w_stride + (size_t)ib * rbytes;
  const size_t gso = (size_t)e * L.gate.s_stride + (size_t)ib * ng;
  const size_t uso = (size_t)e * L.up.s_stride + (size_t)ib * ng;
  const uint16_t* gs = L.gate.s + gso;
  const uint16_t* gb = L.gate.b + gso;
  const uint16_t* us = L.up.s + uso;
  const uint16_t* ub = L.up.b + uso;

  float ag[RW][NT], au[RW][NT];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int j = 0; j < NT; ++j) ag[r][j] = au[r][j] = 0.f;

  for (int c = lane; c < nch; c += 64) {
    uint32_t gd[RW][4], ud[RW][4];
    uint16_t gsc[RW], gbi[RW], usc[RW], ubi[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      load_chunk<BITS>(gw + r * rbytes, c, gd[r]);
      load_chunk<BITS>(uw + r * rbytes, c, ud[r]);
      gsc[r] = gs[r * ng + (c >> 1)];
      gbi[r] = gb[r * ng + (c >> 1)];
      usc[r] = us[r * ng + (c >> 1)];
      ubi[r] = ub[r * ng + (c >> 1)];
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      uint32_t cg[16], cu[16];
      unpack_chunk<BITS, false>(gd[r], cg);
      unpack_chunk<BITS, false>(ud[r], cu);
      const float sg = scale_to_f32<BF16>(gsc[r]) * TWO24, bg = scale_to_f32<BF16>(gbi[r]);
      const float su = scale_to_f32<BF16>(usc[r]) * TWO24, bu = scale_to_f32<BF16>(ubi[r]);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < na) {
          uint32_t xv[16];
          load16(xs + ((size_t)j * nch + c) * 16, xv);
          const float xsm = xsum[j * nch + c];
          ag[r][j] += sg * chunk_dot(cg, xv) + bg * xsm;
          au[r][j] += su * chunk_dot(cu, xv) + bu * xsm;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if (j < na) {
        const float g = wave_sum(ag[r][j]);
        const float uu = wave_sum(au[r][j]);
        if (lane == 0) {
          const int i = ib + r;
          const float a = activate<ACT>(g, uu);
          const _Float16 hi = (_Float16)a;
          const _Float16 lo = (_Float16)(a - (float)hi);
          const size_t o = (size_t)(p0 + j) * I + (i & ~31) + pairpos<BITS>(i & 31);
          act[o] = __builtin_bit_cast(uint16_t, hi);
          act[act_plane + o] = __builtin_bit_cast(uint16_t, lo);
        }
      }
    }
  }
}

template <int BITS, bool BF16, int NT, bool COMBINE>
__global__ __launch_bounds__(256) void dec_down_kernel(const LayerArgs L, int T, int K,
                                                       const int32_t* __restrict__ perm,
                                                       const int32_t* __restrict__ ustart,
                                                       const int32_t* __restrict__ unique,
                                                       const int32_t* __restrict__ scalars,
                                                       const float* __restrict__ wts,
                                                       const uint16_t* __restrict__ act, size_t act_plane,
                                                       void* __restrict__ out, int out32,
                                                       const float* __restrict__ shared_out, int lpr_log2) {
  extern __shared__ float sm2[];
  const int H = L.H, I = L.I, nchI = I / CHUNK;
  const int U = scalars[0];
  const int npos = ustart[U];
  const int LPR = 1 << lpr_log2, RPS = 64 >> lpr_log2;
  float* asum = sm2;                              // [T*K][nchI]
  float* red = sm2 + (size_t)T * K * nchI;        // [4][RPS][NT]
  for (int task = threadIdx.x; task < npos * nchI; task += blockDim.x) {
    const int pos = task / nchI, c = task - pos * nchI;
    uint32_t v[16], vl[16];
    load16(act + (size_t)pos * I + (size_t)c * CHUNK, v);
    load16(act + act_plane + (size_t)pos * I + (size_t)c * CHUNK, vl);
    float s = 0.f, sl = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      s = fdot2(v[m], ONE2, s);
      sl = fdot2(vl[m], ONE2, sl);
    }
    asum[task] = s + sl;
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rl = lane >> lpr_log2;
  const int cl = lane & (LPR - 1);
  const int h = blockIdx.x * RPS + rl;
  const size_t rbytes = (size_t)I * BITS / 8;
  const int ng = I / GROUP;
  float acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = 0.f;

  for (int uu = wave; uu < U; uu += 4) {
    const int e = unique[uu], p0 = ustart[uu];
    const int na = min(ustart[uu + 1] - p0, NT);
    const uint8_t* dw = L.down.w + (size_t)e * L.down.w_stride + (size_t)h * rbytes;
    const size_t dso = (size_t)e * L.down.s_stride + (size_t)h * ng;
    const uint16_t* ds = L.down.s + dso;
    const uint16_t* db = L.down.b + dso;
    float accj[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) accj[j] = 0.f;
    for (int c = cl; c < nchI; c += LPR) {
      uint32_t d[4];
      load_chunk<BITS>(dw, c, d);
      const float sc = scale_to_f32<BF16>(ds[c >> 1]) * TWO24, bi = scale_to_f32<BF16>(db[c >> 1]);
      uint32_t cp[16];
      unpack_chunk<BITS, false>(d, cp);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < na) {
          const int pos = p0 + j;
          uint32_t xv[16], xl[16];
          load16(act + (size_t)pos * I + (size_t)c * CHUNK, xv);
          load16(act + act_plane + (size_t)pos * I + (size_t)c * CHUNK, xl);
          const float part = sc * (chunk_dot(cp, xv) + chunk_dot(cp, xl)) + bi * asum[pos * nchI + c];
          if constexpr (COMBINE) {
            const int a = perm[pos];
            const int t = a / K;
            const float wv = wts[a] * part;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) acc[tt] += tt == t ? wv : 0.f;
          } else {
            accj[j] += part;
          }
        }
      }
    }
    if constexpr (!COMBINE) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < na) {
          const float v = group_sum(accj[j], LPR);
          if (cl == 0) static_cast<uint16_t*>(out)[(size_t)perm[p0 + j] * H + h] = f32_to_f16_bits(v);
        }
      }
    }
  }
  if constexpr (COMBINE) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const float v = group_sum(acc[tt], LPR);
      if (cl == 0) red[(wave * RPS + rl) * NT + tt] = v;
    }
    __syncthreads();
    if (wave == 0 && cl == 0) {
      for (int tt = 0; tt < T; ++tt) {
        float v = red[(0 * RPS + rl) * NT + tt];
        v += red[(1 * RPS + rl) * NT + tt];
        v += red[(2 * RPS + rl) * NT + tt];
        v += red[(3 * RPS + rl) * NT + tt];
        if (shared_out) v += shared_out[(size_t)tt * H + h];
        if (out32)
          static_cast<float*>(out)[(size_t)tt * H + h] = v;
        else
          static_cast<uint16_t*>(out)[(size_t)tt * H + h] = f32_to_f16_bits(v);
      }
    }
  }
}

// ---- dequantization check kernel (codes and fp16 weights of a few rows) ------------------
template <int BITS, bool BF16>
__global__ void dequant_kernel(const QProj P, int in_dim, int expert, int row0, int nrows,
                               uint8_t* __restrict__ codes, uint16_t* __restrict__ wf16) {
  const int nch = in_dim / CHUNK;
  const int task = blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= nrows * nch) return;
  const int r = task / nch, c = task - r * nch;
  const int row = row0 + r;
  const size_t rbytes = (size_t)in_dim * BITS / 8;
  const int ng = in_dim / GROUP;
  const uint8_t* w = P.w + (size_t)expert * P.w_stride + (size_t)row * rbytes;
  uint32_t d[4];
  load_chunk<BITS>(w, c, d);
  uint32_t raw[16], mag[16];
  unpack_chunk<BITS, false>(d, raw);
  unpack_chunk<BITS, true>(d, mag);
  const size_t so = (size_t)expert * P.s_stride + (size_t)row * ng + (c >> 1);
  const float sf = scale_to_f32<BF16>(P.s[so]), bf = scale_to_f32<BF16>(P.b[so]);
  const half2_t s2 = {(_Float16)sf, (_Float16)sf}, b2 = {(_Float16)bf, (_Float16)bf};
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int lo = c * CHUNK + pair_lo(BITS, p), hi = c * CHUNK + pair_hi(BITS, p);
    codes[(size_t)r * in_dim + lo] = (uint8_t)(raw[p] & 0xFFFFu);
    codes[(size_t)r * in_dim + hi] = (uint8_t)(raw[p] >> 16);
    const uint32_t wp = dequant_pair(mag[p], s2, b2);
    wf16[(size_t)r * in_dim + lo] = (uint16_t)(wp & 0xFFFFu);
    wf16[(size_t)r * in_dim + hi] = (uint16_t)(wp >> 16);
  }
}

// ---- launchers --------------------------------------------------------------------------
static int nt_for(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }
constexpr int DEC_RW = 2;

size_t decode_lds_bytes(const LayerConfig& c, int T) {
  const int nt = nt_for(T);
  const size_t nch = (size_t)c.args.H / CHUNK;
  return (size_t)nt * nch * 16 * 4 + (size_t)nt * nch * 4;
}

static int lpr_log2_for(int I) {
  const int nchI = I / CHUNK;
  int l = 0;
  while ((1 << l) < nchI && l < 6) ++l;
  return l;
}

template <int BITS, bool BF16, int ACT, int NT>
static hipError_t decode_impl(const LayerConfig& c, const uint16_t* x, int T, const Work& w, void* out,
                              int out32, bool combine, hipStream_t s) {
  const LayerArgs& L = c.args;
  const int K = c.top_k;
  const int max_u = min(T * K, L.E);
  const size_t act_plane = (size_t)T * K * L.I;
  const int wgs_per_expert = L.I / (4 * DEC_RW);
  const size_t lds1 = decode_lds_bytes(c, T);
  if (lds1 > 65536) {
    hipError_t ae = hipFuncSetAttribute(reinterpret_cast<const void*>(&dec_gateup_kernel<BITS, BF16, ACT, NT, DEC_RW>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
    if (ae != hipSuccess) return ae;
  }
  hipLaunchKernelGGL((dec_gateup_kernel<BITS, BF16, ACT, NT, DEC_RW>), dim3(max_u * wgs_per_expert), dim3(256), lds1,
                     s, L, x, K, w.perm, w.ustart, w.unique, w.scalars, w.act, act_plane, wgs_per_expert);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int l2 = lpr_log2_for(L.I);
  const int rps = 64 >> l2;
  const size_t lds2 = ((size_t)T * K * (L.I / CHUNK) + (size_t)4 * rps * NT) * sizeof(float);
  if (combine) {
    hipLaunchKernelGGL((dec_down_kernel<BITS, BF16, NT, true>), dim3(L.H / rps), dim3(256), lds2, s, L, T, K, w.perm,
                       w.ustart, w.unique, w.scalars, w.wts, w.act, act_plane, out, out32,
                       c.args.sh_gate ? (const float*)w.shared_out : nullptr, l2);
  } else {
    hipLaunchKernelGGL((dec_down_kernel<BITS, BF16, NT, false>), dim3(L.H / rps), dim3(256), lds2, s, L, T, K,
                       w.perm, w.ustart, w.unique, w.scalars, w.wts, w.act, act_plane, out, 0, (const float*)nullptr, l2);
  }
  return hipGetLastError();
}

template <int BITS, bool BF16, int ACT>
static hipError_t decode_nt(const LayerConfig& c, const uint16_t* x, int T, const Work& w, void* out, int out32,
                            bool comb, hipStream_t s) {
  switch (nt_for(T)) {
    case 1: return decode_impl<BITS, BF16, ACT, 1>(c, x, T, w, out, out32, comb, s);
    case 2: return decode_impl<BITS, BF16, ACT, 2>(c, x, T, w, out, out32, comb, s);
    case 4: return decode_impl<BITS, BF16, ACT, 4>(c, x, T, w, out, out32, comb, s);
    default: return decode_impl<BITS, BF16, ACT, 8>(c, x, T, w, out, out32, comb, s);
  }
}

hipError_t launch_decode(const LayerConfig& c, const uint16_t* x, int T, const Work& w, void* out, int out32,
                         bool combine, hipStream_t s) {
#define KMOE_DEC(B, F, A) decode_nt<B, F, A>(c, x, T, w, out, out32, combine, s)
  if (c.bits == 3) {
    if (c.bf16_scales) return c.act ? KMOE_DEC(3, true, 1) : KMOE_DEC(3, true, 0);
    return c.act ? KMOE_DEC(3, false, 1) : KMOE_DEC(3, false, 0);
  }
  if (c.bf16_scales) return c.act ? KMOE_DEC(4, true, 1) : KMOE_DEC(4, true, 0);
  return c.act ? KMOE_DEC(4, false, 1) : KMOE_DEC(4, false, 0);
#undef KMOE_DEC
}

hipError_t launch_dequantize(const LayerConfig& c, int proj, int expert, int row0, int nrows, uint8_t* codes,
                             uint16_t* wf16, hipStream_t s) {
  const QProj& P = proj == 0 ? c.args.gate : proj == 1 ? c.args.up : c.args.down;
  const int in_dim = proj == 2 ? c.args.I : c.args.H;
  const int tasks = nrows * (in_dim / CHUNK);
  const dim3 grid((tasks + 255) / 256), block(256);
  if (tasks == 0) return hipSuccess;
  if (c.bits == 3) {
    if (c.bf16_scales)
      hipLaunchKernelGGL((dequant_kernel<3, true>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
    else
      hipLaunchKernelGGL((dequant_kernel<3, false>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
  } else {
    if (c.bf16_scales)
      hipLaunchKernelGGL((dequant_kernel<4, true>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
    else
      hipLaunchKernelGGL((dequant_kernel<4, false>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
  }
  return hipGetLastError();
}

}  // namespace kmoe
