// Decode path (1..8 tokens): bandwidth-bound dequant GEMVs over the distinct selected experts.
//
// Replaces the reference's per-token CPU expert MLP (kandiga/metal/kandiga_cpu_expert.m:
// 355-401 per expert, :471-552 for the K-way fan-out; kandiga/engine.py:727-735 loops it over
// tokens) and the router/combine around it (moe_block.metal:419-539).  Each token's distinct
// selected experts are streamed from HBM once per layer.
//
// Two launches per layer.  On MI355X a kernel boundary (~1.6 us) is the cheapest grid-wide
// barrier: measured agent-scope counter or flag barriers cost 6-28 us for 256-512 workgroups.
//
//   dec_stage1_kernel: grid = tokens x workgroups per token.  Every workgroup routes its token
//     (DPP arg-max rounds) or reads its given indices, keeps the token's x in registers (pair
//     order, with per-chunk sums) and loops over (distinct expert, block of 4*RW intermediate
//     rows) items.  Each wave streams RW gate rows and the same RW up rows of the expert (one
//     32-code chunk per lane per row), accumulates q*x with v_dot2_f32_f16 on raw codes,
//     applies s*2^24*dot + b*sum(x) per chunk, reduces all 2*RW values across the wave in one
//     pass and writes act = silu(gate) * up as two fp16 planes (hi, lo: hi + lo carries ~22
//     bits) in pair order.
//   dec_stage2_kernel: grid = blocks of S2_ROWS output rows x groups of tokens.  Lanes are
//     (assignment, 32-wide chunk of the intermediate dimension) over RPW rows of the down
//     projection; each lane
//     dots its act chunk (hi and lo planes) with the rows' codes, the per-assignment row totals
//     go to LDS and are combined in k order with the routing weights (moe_block.metal:515-539),
//     so the fused combine is deterministic.  The per-assignment variant writes y[t,k,:]
//     instead (the switch_mlp contract, engine.py:670-739).
// No implicit multiply-add contraction in this file (explicit fmaf where a fused product is
// meant): the fp16 and the scaled-activation instantiations of stage 1 inline the same
// expressions into different code, and fp16-representable rows must give the same bits in both.
#pragma clang fp contract(off)

#include "kmoe_device.h"
#include "kmoe_internal.h"
#include "qlinear.h"

#include <type_traits>

namespace kmoe {

// Phase trace, compiled in only with -DKMOE_PHASE_TRACE: thread 0 of each workgroup stores the
// 100 MHz s_memrealtime clock at the marked points of the two decode kernels, read back with
// kmoe_phase_trace_dump().  Marks, stage 1: 0 entry, 1 routed (wave 0), 2 x permuted, 3 experts known,
// 4 item computed, 5 end; stage 2: 0 entry, 1 metadata, 2 experts done, 3 end.
#ifdef KMOE_PHASE_TRACE
constexpr int TRACE_WGS = 4096;
__device__ uint64_t g_phase_trace[2][TRACE_WGS][8];
#define KMOE_MARK(k, i)                                                  \
  do {                                                                   \
    if (threadIdx.x == 0 && blockIdx.x < TRACE_WGS)                      \
      g_phase_trace[k][blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define KMOE_MARK(k, i) \
  do {                  \
  } while (0)
#endif

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
constexpr int DEC_RW = 2;               // gate/up rows per wave per item of the single-token stage 1
// Gate/up rows per wave per item of the multi-token stage 1: more rows per item keep more
// weight bytes in flight per wave once several experts are selected.
constexpr int stage1_rw(int nt) { return nt >= 4 ? 4 : 2; }

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

struct Stage1Args {
  LayerArgs L;
  const void* x;            // [T][H] of dtype xdt (fp16, bf16, fp32)
  int xdt;
  const float* logits;      // [T][E] (routing mode) or null
  const int32_t* idx_in;    // [T][K] (given-indices mode) or null
  int T, K;
  int32_t* idx_out;         // [T][K] routing (first workgroup of each token), may be null
  float* w_out;             // [T][K]
  int32_t* scalars;         // [2] = device error flags
  uint16_t* act;            // [2][T*K][I], row a = assignment t*K + k
  size_t act_plane;
  float* xinv;              // [T] 2^-s of scaled activations (bf16 / fp32), or null
  int wgs_per_expert;       // row blocks (items) per expert: I / (4*RW)
  int wgs_per_token;        // workgroups working on each token
  uint16_t* sh_act;         // dense shared expert's SwiGLU output, 2 fp16 planes [T][Is] (or null)
  size_t sh_plane;          // T*Is
  QLin ql;                  // router projection of extra workgroups (EX_QL instantiations)
  int ql_row_blocks;        // its workgroups: row blocks x token blocks
  QDown qd;                 // one-expert down projection of extra workgroups (EX_QD instantiations)
};

// Down rows of a one-expert layer for workgroup b of the extra workgroups: LPR lanes per row (the
// chunk count rounded up to a power of two), 64/LPR rows per wave, every token's act chunk (hi
// and lo planes) dotted with the row's raw codes, s*2^24*dot + b*sum(act) per chunk, fp16 out
// (the arithmetic of stage 2's per-assignment form).
template <int BITS, bool BF16>
__device__ __forceinline__ void qdown_rows(const QDown& Q, int H, int T, int b) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int I = Q.I, nch = I / CHUNK, ng = I / GROUP;
  int lpr = 1;
  while (lpr < nch && lpr < 64) lpr <<= 1;
  const int rpw = 64 / lpr, cl = lane & (lpr - 1);
  const int h = (b * 4 + wave) * rpw + lane / lpr;
  const size_t rbytes = (size_t)I * BITS / 8;
  float acc[DEC_MAX_TOKENS];
#pragma unroll
  for (int j = 0; j < DEC_MAX_TOKENS; ++j) acc[j] = 0.f;
  if (h < H) {
    for (int c = cl; c < nch; c += lpr) {
      uint32_t d[4], cp[16];
      load_chunk<BITS>(Q.d.w + (size_t)h * rbytes, c, d);
      unpack_chunk<BITS, false>(d, cp);
      const float sf = scale_to_f32<BF16>(Q.d.s[(size_t)h * ng + (c >> 1)]) * TWO24;
      const float bf = scale_to_f32<BF16>(Q.d.b[(size_t)h * ng + (c >> 1)]);
#pragma unroll
      for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
        if (j < T) {
          uint32_t xh[16], xl[16];
          load16(Q.act + (size_t)j * I + (size_t)c * CHUNK, xh);
          load16(Q.act + Q.plane + (size_t)j * I + (size_t)c * CHUNK, xl);
          float sh = 0.f, sl = 0.f;
#pragma unroll
          for (int m = 0; m < 16; ++m) {
            sh = fdot2(xh[m], ONE2, sh);
            sl = fdot2(xl[m], ONE2, sl);
          }
          acc[j] += fmaf(sf, chunk_dot(cp, xh) + chunk_dot(cp, xl), bf * (sh + sl));
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
    const float v = group_sum_last(acc[j], lpr);
    if (cl == lpr - 1 && h < H && j < T) Q.y[(size_t)j * H + h] = f32_to_f16_bits(v);
  }
}

__device__ __forceinline__ void dec_qdown_rows(const QDown& Q, int H, int T, int b) {
  if (Q.bits == 3) {
    if (Q.bf16) qdown_rows<3, true>(Q, H, T, b);
    else qdown_rows<3, false>(Q, H, T, b);
  } else {
    if (Q.bf16) qdown_rows<4, true>(Q, H, T, b);
    else qdown_rows<4, false>(Q, H, T, b);
  }
}

// Extra workgroups of EX_QD: rows of H in blocks of 4 waves x 64/LPR rows.
inline int qdown_workgroups(const QDown& Q, int H) {
  int lpr = 1;
  while (lpr < Q.I / CHUNK && lpr < 64) lpr <<= 1;
  const int rows = 4 * (64 / lpr);
  return (H + rows - 1) / rows;
}

// Rows of the dense fp16 shared expert per wave in the decode stages.
constexpr int DEC_SH_RW = 2;

// The dense fp16 shared expert's gate/up rows for workgroup b of the workgroups that follow the
// routed ones in stage 1: DEC_SH_RW gate rows and the same up rows per wave against every
// token's x (fp16, natural order, read from L2), act = act(g)*u as two fp16 planes.  These rows
// need no routing, so they stream while the routed workgroups route.  Afterwards the workgroup
// touches one dword per 128-byte line of its share of the shared down matrix, so stage 2 finds
// those lines in the caches.
template <int ACT>
__device__ __forceinline__ void dec_shared_gateup(const uint16_t* __restrict__ x, int T, int H, const LayerArgs& L,
                                                  uint16_t* __restrict__ act, size_t plane, int b, int nb) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int i0 = (b * 4 + wave) * DEC_SH_RW;
  const int nch = H / CHUNK, Is = L.Is;
  float ag[DEC_SH_RW][DEC_MAX_TOKENS], au[DEC_SH_RW][DEC_MAX_TOKENS];
#pragma unroll
  for (int r = 0; r < DEC_SH_RW; ++r)
#pragma unroll
    for (int j = 0; j < DEC_MAX_TOKENS; ++j) ag[r][j] = au[r][j] = 0.f;
  for (int c = lane; c < nch; c += 64) {
    uint32_t g[DEC_SH_RW][16], u[DEC_SH_RW][16];
#pragma unroll
    for (int r = 0; r < DEC_SH_RW; ++r) {
      load16(L.sh_gate + (size_t)(i0 + r) * H + (size_t)c * CHUNK, g[r]);
      load16(L.sh_up + (size_t)(i0 + r) * H + (size_t)c * CHUNK, u[r]);
    }
#pragma unroll
    for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
      if (j < T) {
        uint32_t xv[16];
        load16(x + (size_t)j * H + (size_t)c * CHUNK, xv);
#pragma unroll
        for (int r = 0; r < DEC_SH_RW; ++r) {
          ag[r][j] += chunk_dot(g[r], xv);
          au[r][j] += chunk_dot(u[r], xv);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < DEC_SH_RW; ++r) {
#pragma unroll
    for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
      if (j < T) {
        const float gs = wave_sum_dpp(ag[r][j]);
        const float us = wave_sum_dpp(au[r][j]);
        if (lane == 0) {
          const float a = activate<ACT>(gs, us);
          const _Float16 hi = (_Float16)a;
          const _Float16 lo = (_Float16)(a - (float)hi);
          const size_t o = (size_t)j * Is + i0 + r;
          act[o] = __builtin_bit_cast(uint16_t, hi);
          act[plane + o] = __builtin_bit_cast(uint16_t, lo);
        }
      }
    }
  }
  const size_t lines = (size_t)H * Is * 2 / 128;
  const uint32_t* dn = reinterpret_cast<const uint32_t*>(L.sh_down);
  uint32_t sink = 0u;
  for (size_t ln = (size_t)b * 256 + tid; ln < lines; ln += (size_t)nb * 256) sink ^= dn[ln * 32];
  asm volatile("" ::"v"(sink));
}

// Stage 1.  Workgroup b works on token t = b / wgs_per_token only: wave 0 routes the token (or
// every wave reads its given indices) and shares the K experts through LDS behind the kernel's one
// barrier; every wave keeps the x chunks its lanes multiply in registers (pair order, with chunk
// sums).  Lane k < K of each wave holds assignment k's expert; the distinct experts are the lanes
// whose expert no lower lane also holds (routing never repeats one; given indices may).  Items are
// (distinct expert, block of 4*RW rows), strided over the token's workgroups; each writes act for
// every assignment of that expert.  The next item's weights are loaded while the current one is
// computed (two register stages, unrolled by two so no stage is copied while its loads are in
// flight).  Weights come through buffer resources made per expert, so the row offset is a scalar
// and the lane's chunk offset a constant.  Tokens are not grouped by expert: routing one token per
// workgroup keeps the prologue as short as a single token's, and an expert that two tokens share
// is read twice (the second read mostly from the memory-side cache).  CPL = x chunks per lane
// (H <= 64*32*CPL).  bf16 and fp32 activations are scaled per token (kmoe_device.h, scaled
// activations): the dots run on the scaled hi plane (and, for fp32, the lo plane as a second
// dot), the gate/up totals are multiplied by 2^-s before the activation, act is stored times
// 2^2s, and 2^-s goes to xinv[t] for stage 2.
//
// The values the first loads need (logits, x, the sizes) come as leading scalar arguments: gfx950
// preloads those into SGPRs at wave launch (the library is built with kernel-argument preload),
// so the x and logits loads issue without waiting for the kernel-argument fetch.
// EX: the work of the workgroups past the routed ones: 0 none, EX_SH the dense shared expert's
// gate/up rows, EX_QL the block's router projection, EX_QD the block's quantized shared expert's
// down rows (its act from the shared layer's stage 1).
constexpr int EX_SH = 1, EX_QL = 2, EX_QD = 3;
template <int BITS, bool BF16, int ACT, int CPL, int RW, bool ROUTE, bool XS, int EX>
__global__ __launch_bounds__(256) void dec_stage1_kernel(const float* __restrict__ logits,
                                                         const void* __restrict__ x, int H, int E, int K, int I,
                                                         int wgs_per_token, int nrouted, const Stage1Args A) {
  const LayerArgs& L = A.L;
  static_assert(!(EX && XS), "the extra workgroups serve fp16 activations only");
  static_assert(EX != EX_QL || !ROUTE, "the router projection rides along the block's shared layer only");
  if constexpr (EX == EX_QD) {  // workgroups past the routed ones: the block's shared down rows
    if ((int)blockIdx.x >= nrouted) {
      dec_qdown_rows(A.qd, H, A.T, (int)blockIdx.x - nrouted);
      return;
    }
  }
  if constexpr (EX == EX_QL) {  // workgroups past the shared layer's: the block's router projection
    if ((int)blockIdx.x >= nrouted) {
      const int bid = (int)blockIdx.x - nrouted;
      qlinear_rows<BITS, BF16>(A.ql.a, A.ql.ra, A.ql.b, A.ql.rb, A.T, H, static_cast<const uint16_t*>(x), A.ql.out_a,
                               A.ql.out_b, bid % A.ql_row_blocks, bid / A.ql_row_blocks);
      return;
    }
  }
  if constexpr (EX == EX_SH) {  // workgroups past the routed ones: the dense shared expert's gate/up rows
    if ((int)blockIdx.x >= nrouted) {
      dec_shared_gateup<ACT>(static_cast<const uint16_t*>(x), A.T, H, L, A.sh_act, A.sh_plane,
                             (int)blockIdx.x - nrouted, (int)gridDim.x - nrouted);
      return;
    }
  }
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nch = H / CHUNK;
  const int t = blockIdx.x / wgs_per_token;
  const int lb = blockIdx.x - t * wgs_per_token;
  KMOE_MARK(0, 0);
  // the lane's activation chunks as stored: 16 words per chunk (fp16, bf16) or 32 (fp32); XS
  // instantiates the scaled (bf16 / fp32) form, the fp16 form keeps none of its work
  const int xdt = XS ? A.xdt : XDT_F16;
  const bool has_lo = XS && xdt == XDT_F32;
  const int eb = has_lo ? 4 : 2;
  const char* const xrow = static_cast<const char*>(x) + (size_t)t * H * eb;
  uint32_t xw[CPL][32];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int m = 0; m < 32; ++m) xw[j][m] = 0u;
    if (c < nch) {
      const uint4* q = reinterpret_cast<const uint4*>(xrow + (size_t)c * CHUNK * eb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = q[i];
        xw[j][4 * i] = v.x;
        xw[j][4 * i + 1] = v.y;
        xw[j][4 * i + 2] = v.z;
        xw[j][4 * i + 3] = v.w;
      }
      if (has_lo) {
#pragma unroll
        for (int i = 4; i < 8; ++i) {
          const uint4 v = q[i];
          xw[j][4 * i] = v.x;
          xw[j][4 * i + 1] = v.y;
          xw[j][4 * i + 2] = v.z;
          xw[j][4 * i + 3] = v.w;
        }
      }
    }
  }
  int my = -1;
  float myl = 0.f;  // routing wave: the selected logits (lane k < K)
  // one routing wave per workgroup: redundant copies in the other waves would share SIMDs with
  // it and stretch its latency; they permute their x chunks and wait at the barrier instead.
  // Only the selection is on the path to the barrier; the weights come after it.
  // With routing the token's K experts are distinct and in slot order, and its K * wpe items
  // (slot item / wpe) are strided over its workgroups: a workgroup runs only the selection
  // rounds up to the slot of its last item, so the workgroups of the early slots start their
  // weight loads while the later slots are still being selected.  The workgroup holding the
  // token's last item runs all K rounds and writes the routing outputs.
  // Items are taken in reverse workgroup order: the first-dispatched workgroups (older waves,
  // which win issue on a shared CU) get the last slots, whose selection runs longest.
  const int li = wgs_per_token - 1 - lb;
  int kneed = K;
  bool writer = lb == 0;
  if constexpr (ROUTE) {
    const int ni = K * A.wgs_per_expert, per = (ni + wgs_per_token - 1) / wgs_per_token;
    const int last = min(ni, (li + 1) * per) - 1;
    kneed = last >= li * per ? last / A.wgs_per_expert + 1 : 0;
    writer = li == (ni - 1) / per;
  }
  __shared__ int32_t s_sel[16];
  if (ROUTE && wave == 0) {
    KMOE_TOPK_DISPATCH(E, (wave_topk_select_regs<EPL_>(logits + (size_t)t * E, E, kneed, my, myl)));
    if (lane < K) s_sel[lane] = my;  // -1 past the rounds run
  }
  KMOE_MARK(0, 1);
  // fp16 planes of the activations: as loaded (fp16), or scaled per token (bf16, fp32).  With
  // scaled activations and routing, the routing wave leaves that work to wave 1, which hands it
  // the finished planes through LDS behind the barrier: the scaling (a wave max, the split) would
  // otherwise add to the routing wave's path to the barrier, which every wave waits on.
  constexpr bool HAND = XS && ROUTE;
  const bool handed = HAND && wave == 0;
  uint32_t xr[CPL][16], xq[CPL][16];
  float xinv = 1.f, asc = 1.f;  // 2^-s, and 2^2s for act
  if (handed) {
  } else if (!XS) {
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        xr[j][m] = xw[j][m];
        xq[j][m] = 0u;
      }
  } else {
    float v[CPL][32];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (has_lo) {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[j][i] = __uint_as_float(xw[j][i]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          v[j][2 * i] = __uint_as_float(xw[j][i] << 16);
          v[j][2 * i + 1] = __uint_as_float(xw[j][i] & 0xFFFF0000u);
        }
      }
      amax = fmaxf(amax, chunk_amax(v[j]));
    }
    const int sx = row_scale_exp(__uint_as_float(wave_max_u32_dpp(__float_as_uint(amax))));
    xinv = exp2i(-sx);
    asc = exp2i(2 * sx);
    if (lb == 0 && wave == (HAND ? 1 : 0) && lane == 0 && A.xinv) A.xinv[t] = xinv;
#pragma unroll
    for (int j = 0; j < CPL; ++j) split_chunk(v[j], exp2i(sx), xr[j], xq[j]);
  }
  uint32_t xp[CPL][16], xlp[CPL][16];
  float xs[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (handed) break;
    to_pair_order<BITS>(xr[j], xp[j]);
    float sm = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) sm = fdot2(xr[j][m], ONE2, sm);
    if (has_lo) {
      to_pair_order<BITS>(xq[j], xlp[j]);
      float sl = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) sl = fdot2(xq[j][m], ONE2, sl);
      sm += sl;
    } else {
#pragma unroll
      for (int m = 0; m < 16; ++m) xlp[j][m] = 0u;
    }
    xs[j] = sm;
    // keep this work ahead of the barrier: sunk into the item loop it would wait behind the
    // first item's weight loads
#pragma unroll
    for (int m = 0; m < 16; ++m) asm volatile("" : "+v"(xp[j][m]));
    asm volatile("" : "+v"(xs[j]));
  }
  // lane-major hand-off slots: [chunk][pair word 0..15 | lo word 0..15 | chunk sum][lane]
  __shared__ uint32_t s_hand[HAND ? CPL * 33 * 64 + 2 : 1];
  if constexpr (HAND) {
    if (wave == 1) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          s_hand[(j * 33 + m) * 64 + lane] = xp[j][m];
          s_hand[(j * 33 + 16 + m) * 64 + lane] = xlp[j][m];
        }
        s_hand[(j * 33 + 32) * 64 + lane] = __float_as_uint(xs[j]);
      }
      if (lane == 0) {
        s_hand[CPL * 33 * 64] = __float_as_uint(xinv);
        s_hand[CPL * 33 * 64 + 1] = __float_as_uint(asc);
      }
    }
  }
  if constexpr (ROUTE) {
    __syncthreads();
    my = lane < K ? s_sel[lane] : -1;
  } else {
    if (lane < K) {
      const int e = A.idx_in[t * K + lane];
      my = (e >= 0 && e < E) ? e : -1;
    }
  }
  if constexpr (HAND) {
    if (handed) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          xp[j][m] = s_hand[(j * 33 + m) * 64 + lane];
          xlp[j][m] = s_hand[(j * 33 + 16 + m) * 64 + lane];
        }
        xs[j] = __uint_as_float(s_hand[(j * 33 + 32) * 64 + lane]);
      }
      xinv = __uint_as_float(s_hand[CPL * 33 * 64]);
      asc = __uint_as_float(s_hand[CPL * 33 * 64 + 1]);
    }
  }
  KMOE_MARK(0, 2);
  const uint64_t valid_m = __ballot(my >= 0);
  bool first = my >= 0;
  if constexpr (!ROUTE) {
    for (int j = 0; j < K; ++j) {
      const int ej = __builtin_amdgcn_readlane(my, j);
      first = first && !(j < lane && ej == my);
    }
  }
  const uint64_t first_m = __ballot(first);
  const int nu = ROUTE ? K : __popcll(first_m);
  if (!ROUTE && lb == 0 && tid == 0 && __popcll(valid_m) != K) atomicOr(&A.scalars[2], DEVERR_BAD_EXPERT);
  KMOE_MARK(0, 3);

  constexpr int V = 2 * RW;  // reduced values per item: gate then up, of RW rows
  const int wpe = A.wgs_per_expert;
  const int nitems = nu * wpe;
  const uint32_t rbytes = (uint32_t)H * BITS / 8;
  const int ng = H / GROUP;
  const uint32_t wbytes = (uint32_t)I * rbytes, sbytes = (uint32_t)I * ng * 2;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  uint32_t cvo[CPL], svo[CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    const int c = min(lane + 64 * q, nch - 1);  // lanes past the row's end reload its last chunk
    cvo[q] = (uint32_t)c * Bits<BITS>::chunk_bytes;
    svo[q] = (uint32_t)(c >> 1) * 2u;
  }
  // expert of the token's u-th distinct expert (uniform); with routing, slot u
  auto item_expert = [&](int u) {
    if constexpr (ROUTE) return __builtin_amdgcn_readlane(my, u);
    uint64_t fm = first_m;
    for (int q = 0; q < u; ++q) fm &= fm - 1ull;
    return __builtin_amdgcn_readlane(my, (int)__builtin_ctzll(fm));
  };
  struct WStage {
    uint32_t gd[CPL][RW][4], ud[CPL][RW][4];
    uint16_t gsc[CPL][RW], gbi[CPL][RW], usc[CPL][RW], ubi[CPL][RW];
  };
  auto load_item = [&](int item, WStage& W) {
    const int u = item / wpe;
    const int rb = item - u * wpe;
    const int e = item_expert(u);
    const int ib = rb * (4 * RW) + wv * RW;
    const auto gw = make_rsrc(L.gate.w + (size_t)e * L.gate.w_stride, wbytes);
    const auto uw = make_rsrc(L.up.w + (size_t)e * L.up.w_stride, wbytes);
    const auto gs = make_rsrc(L.gate.s + (size_t)e * L.gate.s_stride, sbytes);
    const auto gb = make_rsrc(L.gate.b + (size_t)e * L.gate.s_stride, sbytes);
    const auto us = make_rsrc(L.up.s + (size_t)e * L.up.s_stride, sbytes);
    const auto ub = make_rsrc(L.up.b + (size_t)e * L.up.s_stride, sbytes);
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const uint32_t wo = (uint32_t)(ib + r) * rbytes, so = (uint32_t)(ib + r) * ng * 2u;
        buf_chunk<BITS>(gw, cvo[q], wo, W.gd[q][r]);
        buf_chunk<BITS>(uw, cvo[q], wo, W.ud[q][r]);
        W.gsc[q][r] = buf_u16(gs, svo[q], so);
        W.gbi[q][r] = buf_u16(gb, svo[q], so);
        W.usc[q][r] = buf_u16(us, svo[q], so);
        W.ubi[q][r] = buf_u16(ub, svo[q], so);
      }
    }
  };
  const bool store_lane = lane < 32 && (lane & (64 / V - 1)) == 0;
  auto compute_item = [&](int item, const WStage& W) {
    const int u = item / wpe;
    const int rb = item - u * wpe;
    const int e = item_expert(u);
    const uint64_t amask = __ballot(my == e);
    const int ib = rb * (4 * RW) + wv * RW;
    // act column of the row this lane stores after the reduction (row r sits in lane group r)
    int col = 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = ib + r;
      const int cr = (i & ~31) + pairpos<BITS>(i & 31);
      col = (lane >> (V == 8 ? 3 : 4)) == r ? cr : col;
    }
    // acc[gu * RW + r]: gate (gu = 0) or up (gu = 1) partial of row r
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      if (lane + 64 * q < nch) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          uint32_t cg[16], cu[16];
          unpack_chunk<BITS, false>(W.gd[q][r], cg);
          unpack_chunk<BITS, false>(W.ud[q][r], cu);
          float dg = chunk_dot(cg, xp[q]), du = chunk_dot(cu, xp[q]);
          if (has_lo) {
            dg += chunk_dot(cg, xlp[q]);
            du += chunk_dot(cu, xlp[q]);
          }
          acc[r] += fmaf(scale_to_f32<BF16>(W.gsc[q][r]) * TWO24, dg, scale_to_f32<BF16>(W.gbi[q][r]) * xs[q]);
          acc[RW + r] += fmaf(scale_to_f32<BF16>(W.usc[q][r]) * TWO24, du, scale_to_f32<BF16>(W.ubi[q][r]) * xs[q]);
        }
      }
    }
    // lane groups 0..RW-1 hold the gate totals and RW..2RW-1 the up totals: one swap of the
    // wave halves puts each row's up total beside its gate total
    const float g = wave_sum_multi<V>(acc);
    const float uu =
        __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(g), __float_as_uint(g), false, false)[1]);
    if (store_lane) {
      const float a = activate<ACT>(g * xinv, uu * xinv) * asc;
      const _Float16 hi = (_Float16)a;
      const _Float16 lo = (_Float16)(a - (float)hi);
      for (uint64_t m = amask; m; m &= m - 1ull) {  // every assignment of this expert (repeats are rare)
        const size_t o = (size_t)(t * K + __builtin_ctzll(m)) * I + col;
        A.act[o] = __builtin_bit_cast(uint16_t, hi);
        A.act[A.act_plane + o] = __builtin_bit_cast(uint16_t, lo);
      }
    }
    KMOE_MARK(0, 4);
  };
  WStage W0, W1;
  // the workgroup's items: a contiguous range (consecutive row blocks, early slots first)
  const int per = (nitems + wgs_per_token - 1) / wgs_per_token;
  const int iend = min(nitems, (li + 1) * per);
  int item = li * per;
  if (item < iend) load_item(item, W0);
  // the routing outputs: the routing wave of the workgroup that ran all K rounds computes the
  // weights while its first item's loads are in flight
  if (ROUTE && writer && wave == 0) {
    const float wv = topk_weight(myl, K);
    if (lane < K) {
      if (A.idx_out) A.idx_out[t * K + lane] = my;
      if (A.w_out) A.w_out[t * K + lane] = wv;
    }
  }
  for (; item < iend; item += 2) {
    if (item + 1 < iend) load_item(item + 1, W1);
    prio_by_work_left(iend - item);
    compute_item(item, W0);
    if (item + 1 >= iend) break;
    if (item + 2 < iend) load_item(item + 2, W0);
    prio_by_work_left(iend - item - 1);
    compute_item(item + 1, W1);
  }
  KMOE_MARK(0, 5);
}

// Stage 2.  Lane (g, c) of a wave works on assignment g of its unit and 32-wide chunk c of the
// intermediate dimension, for RPW consecutive output rows: each act chunk is loaded once per
// workgroup and reused across the rows.  A unit is (group of 64/LPA assignments, RPW-row
// subset of the workgroup's S2_ROWS rows); the four waves take units round-robin.  With one
// chunk per lane (intermediate <= 2048) a wave's units form a two-stage pipeline (the next
// unit's loads in flight while the current one is computed); otherwise UF units at a time
// have all their loads in flight.  Per-assignment row results go to LDS and the combine
// sums them in k order (moe_block.metal:515-539), so the result does not depend on timing.
// The routing pointers and the sizes lead the arguments (preloaded into SGPRs, as for stage 1).
template <int BITS, bool BF16, int S2_ROWS, int RPW, int UF, bool COMBINE, bool SH>
__global__ __launch_bounds__(256) void dec_stage2_kernel(const int32_t* __restrict__ idx,
                                                         const float* __restrict__ wts, int T, int K, int TG,
                                                         int lpa_log2, const LayerArgs L,
                                                         const uint16_t* __restrict__ act, size_t act_plane,
                                                         void* __restrict__ out, int out32,
                                                         const float* __restrict__ shared_out,
                                                         const float* __restrict__ xinv,
                                                         const uint16_t* __restrict__ sh_act, size_t sh_plane,
                                                         Blend B) {
  __shared__ float red[DEC_STAGE2_ASSIGN * S2_ROWS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Token group blockIdx.y: tokens [t0, t0 + TG) are handled as a call of their own, so a
  // workgroup loads the act rows of only TG*K assignments for its output rows.
  {
    const int t0 = blockIdx.y * TG;
    T = min(TG, T - t0);
    idx += t0 * K;
    if (COMBINE) wts += t0 * K;
    act += (size_t)t0 * K * L.I;
    if (xinv) xinv += t0;
    if (COMBINE) {
      out = out32 ? static_cast<void*>(static_cast<float*>(out) + (size_t)t0 * L.H)
                  : static_cast<void*>(static_cast<uint16_t*>(out) + (size_t)t0 * L.H);
      if (shared_out) shared_out += (size_t)t0 * L.H;
      if (B.res) B.res += (size_t)t0 * L.H;
      if (B.sh) B.sh += (size_t)t0 * L.H;
      if (B.gate) B.gate += t0;
      if constexpr (SH) sh_act += (size_t)t0 * L.Is;
    } else {
      out = static_cast<uint16_t*>(out) + (size_t)t0 * K * L.H;
    }
  }
  const int H = L.H, I = L.I, E = L.E, nchI = I / CHUNK, TK = T * K;
  KMOE_MARK(1, 0);
  // routing of assignment a = t*K + k sits in lane a % 64 of slot a / 64 (T*K <= 128)
  int32_t ev0 = -1, ev1 = -1;
  float wv0 = 0.f, wv1 = 0.f;
  if (lane < TK) {
    ev0 = idx[lane];
    if (COMBINE) wv0 = wts[lane];
  }
  if (lane + 64 < TK) {
    ev1 = idx[lane + 64];
    if (COMBINE) wv1 = wts[lane + 64];
  }
  // 2^-s of scaled activations, token t in lane t (loaded with the routing, not after the dots)
  const float xv = xinv && lane < T ? xinv[lane] : 1.f;
  // the term this thread's combine output adds after the routed sum, loaded now rather than
  // after the dots: the fp32 extra row, or the block's residual + fp16 shared * sigmoid(gate)
  const bool add_term = COMBINE && (shared_out || B.res || B.sh);
  float term = 0.f;
  if (add_term && tid < T * S2_ROWS) {
    const int tt = tid / S2_ROWS, hh = blockIdx.x * S2_ROWS + (tid - tt * S2_ROWS);
    const size_t o = (size_t)tt * L.H + hh;
    if (shared_out) {
      term = shared_out[o];
    } else {
      term = B.res ? f16_bits_to_f32(B.res[o]) : 0.f;
      if (B.sh) term += f16_bits_to_f32(B.sh[o]) * (B.gate ? 1.0f / (1.0f + expf(-B.gate[tt])) : 1.0f);
    }
  }
  KMOE_MARK(1, 1);

  const int LPA = 1 << lpa_log2, AG = 64 >> lpa_log2;
  const int g = lane >> lpa_log2;
  const int cl = lane & (LPA - 1);
  const int h0 = blockIdx.x * S2_ROWS;
  const size_t rbytes = (size_t)I * BITS / 8;
  const int ng = I / GROUP;
  constexpr int NSUB = S2_ROWS / RPW;
  const int nunits = ((TK + AG - 1) / AG) * NSUB;

  if (nchI <= LPA) {
    // One chunk per lane (intermediate <= 2048): the wave's units (u = wave + 4j) run as a
    // two-stage pipeline, the loads of unit j+1 in flight while unit j is computed.
    struct S2Unit {
      int a, e, hb;
      bool v;
    };
    struct S2Load {
      uint32_t d[RPW][4], xh[16], xl[16];
      uint16_t sc[RPW], bi[RPW];
    };
    const int c = cl;
    const bool cv = c < nchI;
    auto unit_of = [&](int u) {  // uniform control flow (the shuffle needs every lane)
      S2Unit U;
      const int grp = u / NSUB;
      U.hb = h0 + (u - grp * NSUB) * RPW;
      U.a = grp * AG + g;
      // the assignment group never straddles the two slots (AG divides 64)
      const int e = __shfl(grp * AG < 64 ? ev0 : ev1, U.a & 63, 64);
      U.v = u < nunits && U.a < TK && e >= 0 && e < E;
      U.e = U.v ? e : 0;
      return U;
    };
    auto load_unit = [&](const S2Unit& U, S2Load& S) {
      if (U.v && cv) {
        const uint8_t* wrow = L.down.w + (size_t)U.e * L.down.w_stride + (size_t)U.hb * rbytes;
        const size_t so = (size_t)U.e * L.down.s_stride + (size_t)U.hb * ng + (c >> 1);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          load_chunk<BITS>(wrow + r * rbytes, c, S.d[r]);
          S.sc[r] = L.down.s[so + r * ng];
          S.bi[r] = L.down.b[so + r * ng];
        }
        load16(act + (size_t)U.a * I + (size_t)c * CHUNK, S.xh);
        load16(act + act_plane + (size_t)U.a * I + (size_t)c * CHUNK, S.xl);
      }
    };
    auto finish_unit = [&](int u, const S2Unit& U, const S2Load& S) {
      float part[RPW];
#pragma unroll
      for (int r = 0; r < RPW; ++r) part[r] = 0.f;
      const float xq = __shfl(xv, min(U.a, TK - 1) / K, 64);  // every lane: the shuffle is uniform
      if (U.v && cv) {
        float sh = 0.f, sl = 0.f;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          sh = fdot2(S.xh[m], ONE2, sh);
          sl = fdot2(S.xl[m], ONE2, sl);
        }
        const float xs = sh + sl;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          uint32_t cp[16];
          unpack_chunk<BITS, false>(S.d[r], cp);
          const float sf = scale_to_f32<BF16>(S.sc[r]) * TWO24, bf = scale_to_f32<BF16>(S.bi[r]);
          part[r] = fmaf(sf, chunk_dot(cp, S.xh) + chunk_dot(cp, S.xl), bf * xs);
        }
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float v = group_sum_last(part[r], LPA);  // 0 for an assignment with an invalid expert
        if (cl == LPA - 1 && u < nunits && U.a < TK) {
          if (xinv) v *= xq * xq;  // act was stored times 2^2s
          if constexpr (COMBINE) {
            red[U.a * S2_ROWS + (U.hb - h0) + r] = v;
          } else {
            static_cast<uint16_t*>(out)[(size_t)U.a * H + U.hb + r] = f32_to_f16_bits(v);
          }
        }
      }
    };
    const int nw = wave < nunits ? (nunits - wave + 3) / 4 : 0;  // this wave's units
    S2Load S0, S1;
    S2Unit U0 = unit_of(wave), U1;
    load_unit(U0, S0);
    for (int j = 0; j < nw; j += 2) {
      const int u = wave + 4 * j;
      if (j + 1 < nw) {
        U1 = unit_of(u + 4);
        load_unit(U1, S1);
      }
      prio_by_work_left(nw - j);
      finish_unit(u, U0, S0);
      if (j + 1 >= nw) break;
      if (j + 2 < nw) {
        U0 = unit_of(u + 8);
        load_unit(U0, S0);
      }
      prio_by_work_left(nw - j - 1);
      finish_unit(u + 4, U1, S1);
    }
  } else {
    for (int u0 = wave; u0 < nunits; u0 += 4 * UF) {
      int av[UF], ea[UF], hb[UF];
      bool va[UF];
#pragma unroll
      for (int i = 0; i < UF; ++i) {
        const int u = u0 + 4 * i;  // uniform
        const int grp = u / NSUB;
        hb[i] = h0 + (u - grp * NSUB) * RPW;
        const int a = grp * AG + g;
        // the assignment group never straddles the two slots (AG divides 64)
        const int e = __shfl(grp * AG < 64 ? ev0 : ev1, a & 63, 64);
        av[i] = a;
        va[i] = u < nunits && a < TK && e >= 0 && e < E;
        ea[i] = va[i] ? e : 0;
      }
      float part[UF][RPW];
#pragma unroll
      for (int i = 0; i < UF; ++i)
#pragma unroll
        for (int r = 0; r < RPW; ++r) part[i][r] = 0.f;
      for (int c = cl; c < nchI; c += LPA) {
        uint32_t d[UF][RPW][4], xh[UF][16], xl[UF][16];
        uint16_t sc[UF][RPW], bi[UF][RPW];
#pragma unroll
        for (int i = 0; i < UF; ++i) {
          if (va[i]) {
            const uint8_t* wrow = L.down.w + (size_t)ea[i] * L.down.w_stride + (size_t)hb[i] * rbytes;
            const size_t so = (size_t)ea[i] * L.down.s_stride + (size_t)hb[i] * ng + (c >> 1);
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
              load_chunk<BITS>(wrow + r * rbytes, c, d[i][r]);
              sc[i][r] = L.down.s[so + r * ng];
              bi[i][r] = L.down.b[so + r * ng];
            }
            load16(act + (size_t)av[i] * I + (size_t)c * CHUNK, xh[i]);
            load16(act + act_plane + (size_t)av[i] * I + (size_t)c * CHUNK, xl[i]);
          }
        }
#pragma unroll
        for (int i = 0; i < UF; ++i) {
          if (va[i]) {
            float sh = 0.f, sl = 0.f;
#pragma unroll
            for (int m = 0; m < 16; ++m) {
              sh = fdot2(xh[i][m], ONE2, sh);
              sl = fdot2(xl[i][m], ONE2, sl);
            }
            const float xs = sh + sl;
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
              uint32_t cp[16];
              unpack_chunk<BITS, false>(d[i][r], cp);
              const float sf = scale_to_f32<BF16>(sc[i][r]) * TWO24, bf = scale_to_f32<BF16>(bi[i][r]);
              part[i][r] += fmaf(sf, chunk_dot(cp, xh[i]) + chunk_dot(cp, xl[i]), bf * xs);
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < UF; ++i) {
        const int a = av[i];
        const float xq = __shfl(xv, min(a, TK - 1) / K, 64);  // every lane: the shuffle is uniform
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float v = group_sum_last(part[i][r], LPA);  // 0 for an assignment with an invalid expert
          if (cl == LPA - 1 && u0 + 4 * i < nunits && a < TK) {
            if (xinv) v *= xq * xq;  // act was stored times 2^2s
            if constexpr (COMBINE) {
              red[a * S2_ROWS + (hb[i] - h0) + r] = v;
            } else {
              static_cast<uint16_t*>(out)[(size_t)a * H + hb[i] + r] = f32_to_f16_bits(v);
            }
          }
        }
      }
    }
  }
  KMOE_MARK(1, 2);
  if constexpr (COMBINE) {
    // The dense fp16 shared expert's down rows of this workgroup (its act came from stage 1's
    // extra workgroups): LPS lanes per row, every token's act hi + lo planes, results to LDS for
    // the combine below, which adds them after the routed sum.
    __shared__ float s_sh[SH ? DEC_MAX_TOKENS * S2_ROWS : 1];
    if constexpr (SH) {
      const int nchs = L.Is / CHUNK;
      int lps = 1;
      while (lps < nchs && lps < 64) lps <<= 1;
      const int rpws = 64 / lps, cs = lane & (lps - 1);
      for (int rb = wave * rpws; rb < S2_ROWS; rb += 4 * rpws) {
        const int r = rb + lane / lps;
        float acc[DEC_MAX_TOKENS];
#pragma unroll
        for (int j = 0; j < DEC_MAX_TOKENS; ++j) acc[j] = 0.f;
        if (r < S2_ROWS) {
          const uint16_t* drow = L.sh_down + (size_t)(h0 + r) * L.Is;
          for (int c = cs; c < nchs; c += lps) {
            uint32_t d[16];
            load16(drow + (size_t)c * CHUNK, d);
#pragma unroll
            for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
              if (j < T) {
                uint32_t ah[16], al[16];
                load16(sh_act + (size_t)j * L.Is + (size_t)c * CHUNK, ah);
                load16(sh_act + sh_plane + (size_t)j * L.Is + (size_t)c * CHUNK, al);
                acc[j] += chunk_dot(d, ah) + chunk_dot(d, al);
              }
            }
          }
        }
#pragma unroll
        for (int j = 0; j < DEC_MAX_TOKENS; ++j) {
          const float v = group_sum_last(acc[j], lps);
          if (j < T && r < S2_ROWS && cs == lps - 1) s_sh[j * S2_ROWS + r] = v;
        }
      }
    }
    __shared__ float s_wt[DEC_STAGE2_ASSIGN];
    if (wave == 0) {
      if (lane < TK) s_wt[lane] = wv0;
      if (lane + 64 < TK) s_wt[lane + 64] = wv1;
    }
    __syncthreads();
    if (tid < T * S2_ROWS) {
      const int t = tid / S2_ROWS, r = tid - t * S2_ROWS;
      float v = 0.f;
      for (int k = 0; k < K; ++k) {
        const int a = t * K + k;
        v = fmaf(s_wt[a], red[a * S2_ROWS + r], v);
      }
      const int h = h0 + r;
      if constexpr (SH) v += s_sh[t * S2_ROWS + r];
      if (add_term) v += term;
      if (out32)
        static_cast<float*>(out)[(size_t)t * H + h] = v;
      else
        static_cast<uint16_t*>(out)[(size_t)t * H + h] = f32_to_f16_bits(v);
    }
  }
  KMOE_MARK(1, 3);
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
// Compute units of the current device (queried once per device).
static int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

static int nt_for(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }

// log2 of the lanes that share one assignment in stage 2: the chunk count rounded up, <= 64.
static int lpa_log2_for(int I) {
  const int nchI = I / CHUNK;
  int l = 0;
  while ((1 << l) < nchI && l < 6) ++l;
  return l;
}

template <typename KERN>
static hipError_t launch_stage1(KERN k1, int grid, hipStream_t s, const Stage1Args& A) {
  // extra workgroups after the routed ones: the dense shared expert's gate/up rows (fp16
  // activations only) or the block's router projection
  const int nsh = A.sh_act     ? A.L.Is / (4 * DEC_SH_RW)
                 : A.ql.out_a ? A.ql_row_blocks * qlinear_token_blocks(A.T)
                 : A.qd.y     ? qdown_workgroups(A.qd, A.L.H)
                              : 0;
  KMOE_LAUNCH("dec_stage1_kernel", k1, dim3(grid + nsh), dim3(256), 0, s, A.logits, A.x, A.L.H, A.L.E, A.K,
              A.L.I, A.wgs_per_token, grid, A);
  return hipGetLastError();
}

template <int BITS, bool BF16, int ACT, int NT>
static hipError_t decode_impl(const LayerConfig& c, const DecodeCall& d, hipStream_t s) {
  const LayerArgs& L = c.args;
  const int K = c.top_k, T = d.T;
  const Work& w = *d.w;
  const int nch = L.H / CHUNK;
  if (nch > 128) return hipErrorInvalidValue;  // x chunks of a token live in two registers per lane at most
  constexpr int RW = NT == 1 ? DEC_RW : stage1_rw(NT);
  Stage1Args A;
  A.L = L;
  A.x = d.x;
  A.xdt = d.xdt;
  A.logits = d.logits;
  A.idx_in = d.idx_in;
  A.T = T;
  A.K = K;
  A.idx_out = d.idx_out;
  A.w_out = d.w_out;
  A.scalars = w.scalars;
  A.act = w.act;
  A.act_plane = (size_t)T * K * L.I;
  A.xinv = d.xdt == XDT_F16 ? nullptr : w.xinv;
  A.sh_act = L.sh_gate && d.xdt == XDT_F16 ? w.shared_act : nullptr;
  A.sh_plane = (size_t)T * L.Is;
  A.ql = d.ql ? *d.ql : QLin{};
  A.ql_row_blocks = qlinear_row_blocks(A.ql.ra + A.ql.rb);
  if (d.ql && (d.logits || d.xdt != XDT_F16)) return hipErrorInvalidValue;
  A.qd = d.qd ? *d.qd : QDown{};
  if (d.qd && (!d.logits || d.xdt != XDT_F16 || L.sh_gate || d.ql)) return hipErrorInvalidValue;
  A.wgs_per_expert = L.I / (4 * RW);
  // at most two workgroups per CU in all: every workgroup repeats its token's routing, so the
  // grid stays resident and loops over the token's (expert, row block) items instead
  A.wgs_per_token = max(1, min(min(K, L.E) * A.wgs_per_expert, 2 * cu_count() / T));
  const int grid1 = T * A.wgs_per_token;
  hipError_t err;
  auto stage1 = [&](auto xs) {
    constexpr bool XSV = decltype(xs)::value;
    if constexpr (!XSV) {
      if (A.qd.y) {  // the block's shared down rows ride along (routing, fp16)
        if (nch <= 64) return launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, true, false, EX_QD>, grid1, s, A);
        return launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, true, false, EX_QD>, grid1, s, A);
      }
      if (A.ql.out_a) {  // the block's router projection rides along (given indices, fp16)
        if (nch <= 64)
          return launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, false, false, EX_QL>, grid1, s, A);
        return launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, false, false, EX_QL>, grid1, s, A);
      }
      // the dense shared expert's gate/up rows ride along (fp16 activations)
      if (A.sh_act) {
        if (nch <= 64)
          return d.logits ? launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, true, false, EX_SH>, grid1, s, A)
                          : launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, false, false, EX_SH>, grid1, s, A);
        return d.logits ? launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, true, false, EX_SH>, grid1, s, A)
                        : launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, false, false, EX_SH>, grid1, s, A);
      }
    }
    if (nch <= 64)
      return d.logits ? launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, true, XSV, 0>, grid1, s, A)
                      : launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 1, RW, false, XSV, 0>, grid1, s, A);
    return d.logits ? launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, true, XSV, 0>, grid1, s, A)
                    : launch_stage1(&dec_stage1_kernel<BITS, BF16, ACT, 2, RW, false, XSV, 0>, grid1, s, A);
  };
  err = d.xdt == XDT_F16 ? stage1(std::false_type{}) : stage1(std::true_type{});
  if (err != hipSuccess || d.stage1_only) return err;
  const int l2 = lpa_log2_for(L.I);
  // Output rows per workgroup (S2_ROWS) and per lane (RPW), and tokens per workgroup (TG).  Every
  // workgroup re-reads the act rows of its tokens' assignments, so taller row blocks cut that
  // traffic; the tokens are then split into groups over a second grid dimension, sized for about
  // two workgroups per CU (measured best at hidden 2048 and 4096, 4 and 8 tokens) with at least
  // 8 assignments per workgroup.  Below 32 assignments short row blocks over all tokens are
  // faster.
  const int32_t* idx = d.idx_in ? d.idx_in : d.idx_out;
  // the dense shared expert runs inside the two stages (fp16 activations, the only ones it takes)
  uint16_t* const sh_act = L.sh_gate && d.xdt == XDT_F16 ? w.shared_act : nullptr;
  const size_t sh_plane = (size_t)T * L.Is;
  const float* sho = d.extra;
  auto stage2 = [&](auto srows, auto rpw, int TG) {
    constexpr int SR = decltype(srows)::value, RP = decltype(rpw)::value, UF = 2;
    const dim3 grid2(L.H / SR, (T + TG - 1) / TG);
    if (d.combine && sh_act) {
      KMOE_LAUNCH("dec_stage2_kernel", (dec_stage2_kernel<BITS, BF16, SR, RP, UF, true, true>), grid2, dim3(256), 0, s,
                  idx, d.wts, T, K, TG, l2, L, (const uint16_t*)w.act, A.act_plane, d.out, d.out32, sho, A.xinv,
                  (const uint16_t*)sh_act, sh_plane, d.blend);
    } else if (d.combine) {
      KMOE_LAUNCH("dec_stage2_kernel", (dec_stage2_kernel<BITS, BF16, SR, RP, UF, true, false>), grid2, dim3(256), 0, s,
                  idx, d.wts, T, K, TG, l2, L, (const uint16_t*)w.act, A.act_plane, d.out, d.out32, sho, A.xinv,
                  (const uint16_t*)nullptr, (size_t)0, d.blend);
    } else {
      KMOE_LAUNCH("dec_stage2_kernel", (dec_stage2_kernel<BITS, BF16, SR, RP, UF, false, false>), grid2, dim3(256), 0, s,
                  idx, (const float*)nullptr, T, K, TG, l2, L, (const uint16_t*)w.act, A.act_plane, d.out, 0,
                  (const float*)nullptr, A.xinv, (const uint16_t*)nullptr, (size_t)0, Blend{});
    }
  };
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  using I16 = std::integral_constant<int, 16>;
  if constexpr (NT == 1) {
    // top-4 or fewer: two rows per lane give each wave two units in flight (measured 2% faster
    // at top-4; four rows per lane stay faster at top-8)
    if (K <= 4)
      stage2(I8{}, std::integral_constant<int, 2>{}, T);
    else
      stage2(I8{}, I4{}, T);
  } else if constexpr (NT == 2) {
    stage2(I4{}, I4{}, T);
  } else {
    if (T * K >= 32) {
      const int tg = T * (L.H / 16) / (2 * cu_count());
      stage2(I16{}, I8{}, min(T, max(tg, (8 + K - 1) / K)));
    } else
      stage2(I4{}, I4{}, T);
  }
  return hipGetLastError();
}

template <int BITS, bool BF16, int ACT>
static hipError_t decode_nt(const LayerConfig& c, const DecodeCall& d, hipStream_t s) {
  switch (nt_for(d.T)) {
    case 1: return decode_impl<BITS, BF16, ACT, 1>(c, d, s);
    case 2: return decode_impl<BITS, BF16, ACT, 2>(c, d, s);
    case 4: return decode_impl<BITS, BF16, ACT, 4>(c, d, s);
    default: return decode_impl<BITS, BF16, ACT, 8>(c, d, s);
  }
}

hipError_t launch_decode(const LayerConfig& c, const DecodeCall& d, hipStream_t s) {
  if (d.T < 1 || d.T > DEC_MAX_TOKENS || d.T * c.top_k > DEC_STAGE2_ASSIGN) return hipErrorInvalidValue;
#define KMOE_DEC(B, F, A) decode_nt<B, F, A>(c, d, s)
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
      KMOE_LAUNCH("dequant_kernel", (dequant_kernel<3, true>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
    else
      KMOE_LAUNCH("dequant_kernel", (dequant_kernel<3, false>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
  } else {
    if (c.bf16_scales)
      KMOE_LAUNCH("dequant_kernel", (dequant_kernel<4, true>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
    else
      KMOE_LAUNCH("dequant_kernel", (dequant_kernel<4, false>), grid, block, 0, s, P, in_dim, expert, row0, nrows, codes, wf16);
  }
  return hipGetLastError();
}

}  // namespace kmoe

#ifdef KMOE_PHASE_TRACE
extern "C" int kmoe_phase_trace_dump(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(kmoe::g_phase_trace), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int kmoe_phase_trace_clear(void) {
  static uint64_t zero[2 * kmoe::TRACE_WGS * 8];
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(kmoe::g_phase_trace), zero, sizeof zero, 0, hipMemcpyHostToDevice);
}
#endif
