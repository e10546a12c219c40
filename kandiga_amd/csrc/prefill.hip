// Prefill path: grouped GEMM over the expert-sorted assignments with fp16 MFMA.
//
// Replaces the reference's 4-bit prefill (kandiga/engine.py:386-516: permutation, one
// Metal dispatch for gate+up+SiLU over every (assignment, row), one for down, then a
// scatter back to [T, K, H]) and its 3-bit fallback (engine.py:720-735: T sequential
// CPU calls).
//
//   xpair_kernel: x into pair order once per call (the k order the dequantized weights have).
//   gemm_gateup_kernel: one workgroup per (m-tile of <= 128 sorted assignments of one expert,
//     256 intermediate columns of both gate and up); SwiGLU in registers, act written once as
//     two fp16 planes, hi = fp16(a) and lo = fp16(a - hi) (about 22 significant bits; pair order
//     for the down projection's k dimension).
//   gemm_down_kernel: one workgroup per (m-tile, 512 output columns); A = act rows of the tile
//     (contiguous, pair order), both planes: each dequantized weight fragment meets the hi and
//     the lo fragment of the rows, so the down projection sees fp32-quality activations (one
//     fp16 plane alone is off by up to 2^-12 of |act| per element, which reached 2.7e-2 of
//     output on 4-bit layers).  The output row of sorted position p is written to assignment
//     perm[p]: fp16 for the switch_mlp contract, or fp32 scaled by that assignment's routing
//     weight for the fused layer (an fp16 intermediate would add up to half an fp16 ulp of
//     each term before the combine).
//   Both run v_mfma_f32_32x32x16_f16 with the weights dequantized in registers (see the grouped
//   GEMM section below).
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

// N dwords (2N halves) of an A row between memory and registers, as 16-byte accesses.
template <int N>
__device__ __forceinline__ void stage_load(const void* p, uint32_t (&v)[N]) {
  const uint4* s = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int q = 0; q < N / 4; ++q) {
    const uint4 t = s[q];
    v[4 * q] = t.x;
    v[4 * q + 1] = t.y;
    v[4 * q + 2] = t.z;
    v[4 * q + 3] = t.w;
  }
}
template <int N>
__device__ __forceinline__ void stage_store(_Float16* dst, const uint32_t (&v)[N]) {
  uint4* d = reinterpret_cast<uint4*>(dst);
#pragma unroll
  for (int q = 0; q < N / 4; ++q) d[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

__device__ __forceinline__ float16_t mfma32(const half8_t a, const half8_t b, const float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

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

// ---- grouped GEMMs ----------------------------------------------------------------------
// Shared structure of both GEMMs.  A workgroup (4 waves) owns one m-tile: up to GEMM_BM = 128
// expert-sorted assignment rows of one expert, as four 32-row blocks (64 rows, two blocks, from
// the prefill copy).  Each wave owns two 32-column blocks of the output for all of the tile's
// rows, so its 8 accumulator blocks of v_mfma_f32_32x32x16_f16 hold 128 x 64 fp32 values, and
// two workgroups fit on a CU (three or four with 64-row tiles): while one waits at its k-step
// barrier or for loads, the others' waves issue.
//
//   * A (x rows for gate/up, act rows for down) is shared by the four waves: per 64-wide k step
//     (one quantization group) the tile's rows are loaded once into an LDS slab (double
//     buffered, one barrier per k step).  Rows are already in pair order, the k order in which
//     the weight codes unpack.
//   * B (the weights) never goes through LDS: no other wave needs a wave's columns, so each
//     lane dequantizes its own fragments in registers.  Lane (n, h) = (lane & 31, lane >> 5)
//     of a column block holds weight row n; for one quantization group it loads code chunk h
//     (codes 32h..32h+31, 12 or 16 bytes) and that row's scale and bias, and the four k16
//     steps of the group take pairs 4s..4s+3 of the chunk as their 8 fp16 values: exactly the
//     MFMA B layout (k = 8h..8h+7 of each step), with the A fragment read at the same pair-order
//     positions.  round(q*s + b) is one packed subtract and one packed fma per two weights.
//   * Only the 32-row blocks that hold assignments are multiplied (the kernel body is
//     instantiated for 1..4 blocks), so a ragged expert costs its rows rounded up to 32, not
//     to 128.
//   * Weights and scales come through per-projection buffer resources, so a weight row past
//     the projection's end reads zeros (such columns are computed but never stored).
// The codes of the group after next and the A rows of the next group are loaded while a group
// is multiplied.

constexpr int LDA = 72;                      // halves per row of the A slab (64 + 8 pad: 144 B)
constexpr int EPI_LD = 68;                   // floats per row of a wave's down epilogue staging (64 + 4)
constexpr int EPA_LD = 40;                   // halves per row of a wave's gate/up epilogue staging (32 + 8)
// LDS of a GEMM workgroup in halves: two stages of A slabs (np planes for gate/up: one, or the hi
// and lo planes of fp32 activations; the hi and lo planes of act for down), or the epilogue
// staging if larger
constexpr int lds_halves(int bm, bool down, int np = 1) {
  return 2 * (down ? 2 : np) * bm * LDA > (down ? 4 * 32 * EPI_LD * 2 : 4 * 32 * EPA_LD)
             ? 2 * (down ? 2 : np) * bm * LDA
             : (down ? 4 * 32 * EPI_LD * 2 : 4 * 32 * EPA_LD);
}

// Workgroup b -> (m-tile, column tile).  Workgroups are dealt to the 8 XCDs round-robin (XCD x
// runs b = x, x+8, ...).  XCD x takes a contiguous share of the m-tile list (the m-tiles of one
// expert are consecutive there, so the expert's weights stay in that XCD's L2) and runs the
// column tiles of one m-tile back to back (they share its A rows).  The grid holds
// 8 * ceil(max_mtiles / 8) * ncol workgroups; the actual count nmt is read on the device.
__device__ __forceinline__ bool xcd_mtile(int b, int ncol, int nmt, int& mt, int& ct) {
  const int x = b & 7, j = b >> 3;
  const int lm = j / ncol;
  ct = j - lm * ncol;
  const int share = (nmt + 7) >> 3;
  mt = x * share + lm;
  return lm < share && mt < nmt;
}

// A value every lane of the wave holds, moved to a scalar register (buffer resources and
// branches built from it stay uniform).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// One quantization group of a lane's JB weight rows: codes and (per-group scale path) the
// row's scale and bias.
template <int JB>
struct BGroup {
  uint32_t d[JB][4];
  uint16_t s[JB], b[JB];
};

// Scales and biases of two consecutive groups (2p: low half, 2p+1: high half) of a lane's rows,
// one 4-byte load each; used when a row holds an even number of groups (4-byte aligned rows).
template <int JB>
struct BScalePair {
  uint32_t s[JB], b[JB];
};

// Weight rows of a lane: row j's codes/scales/biases through resources rw/rs/rb[j] at lane
// offsets vw/vs[j] (bytes).  Group g adds the uniform offsets 2g chunks / 2g bytes.
template <int JB>
struct BRows {
  __amdgpu_buffer_rsrc_t rw[JB], rs[JB], rb[JB];
  uint32_t vw[JB], vs[JB];
  uint32_t gstride;  // code bytes from one group to the next at the same lane offset
  uint32_t pstride;  // scale bytes from one group pair to the next
};

template <int BITS, int JB, bool SCALES>
__device__ __forceinline__ void load_group(const BRows<JB>& R, int g, BGroup<JB>& G) {
  const uint32_t sw = (uint32_t)uniform(g * (int)R.gstride), ss = (uint32_t)uniform(g * 2);
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    buf_chunk_cached<BITS>(R.rw[j], R.vw[j], sw, G.d[j]);
    if constexpr (SCALES) {
      G.s[j] = buf_u16(R.rs[j], R.vs[j], ss);
      G.b[j] = buf_u16(R.rb[j], R.vs[j], ss);
    }
  }
}

// PK: the prefill copy holds s0 s1 b0 b1 of a row side by side (one 8-byte load).
template <int JB, bool PK>
__device__ __forceinline__ void load_scale_pair(const BRows<JB>& R, int p, BScalePair<JB>& S) {
  const uint32_t ss = (uint32_t)uniform(p * (int)R.pstride);
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    if constexpr (PK) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(R.rs[j], R.vs[j], ss, 0);
      S.s[j] = v[0];
      S.b[j] = v[1];
    } else {
      S.s[j] = __builtin_amdgcn_raw_buffer_load_b32(R.rs[j], R.vs[j], ss, 0);
      S.b[j] = __builtin_amdgcn_raw_buffer_load_b32(R.rb[j], R.vs[j], ss, 0);
    }
  }
}

// k16 step ST of one group: A fragments of the NB active row blocks from the slab (NP planes,
// plane p at slab + p*BM*LDA), B fragments of the JB column blocks dequantized from the group's
// codes; each B fragment is multiplied by every plane's A fragment.
template <int BITS, int NB, int JB, int ST, int NP, int BM>
__device__ __forceinline__ void gemm_step(float16_t (&acc)[4][JB], const _Float16* __restrict__ slab, int lane,
                                          const BGroup<JB>& G, const half2_t (&s2)[JB], const half2_t (&b2)[JB]) {
  const _Float16* ap = slab + (lane & 31) * LDA + 32 * (lane >> 5) + 8 * ST;
  if constexpr (NP == 1) {
    half8_t af[NB];
#pragma unroll
    for (int mb = 0; mb < NB; ++mb) af[mb] = *reinterpret_cast<const half8_t*>(ap + 32 * mb * LDA);
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const u32x4_t q = {dequant_pair(chunk_pair<BITS, 4 * ST + 0, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 1, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 2, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 3, true>(G.d[j]), s2[j], b2[j])};
      const half8_t bf = __builtin_bit_cast(half8_t, q);
#pragma unroll
      for (int mb = 0; mb < NB; ++mb) acc[mb][j] = mfma32(af[mb], bf, acc[mb][j]);
    }
  } else {
    // the JB B fragments are dequantized once, then each plane's A fragments are read and
    // multiplied in turn (one plane's fragments live at a time)
    half8_t bf[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const u32x4_t q = {dequant_pair(chunk_pair<BITS, 4 * ST + 0, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 1, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 2, true>(G.d[j]), s2[j], b2[j]),
                         dequant_pair(chunk_pair<BITS, 4 * ST + 3, true>(G.d[j]), s2[j], b2[j])};
      bf[j] = __builtin_bit_cast(half8_t, q);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      half8_t af[NB];
#pragma unroll
      for (int mb = 0; mb < NB; ++mb) af[mb] = *reinterpret_cast<const half8_t*>(ap + p * BM * LDA + 32 * mb * LDA);
#pragma unroll
      for (int j = 0; j < JB; ++j)
#pragma unroll
        for (int mb = 0; mb < NB; ++mb) acc[mb][j] = mfma32(af[mb], bf[j], acc[mb][j]);
    }
  }
}

// One group: sc/bi are the rows' scale and bias bits.
template <int BITS, bool BF16, int NB, int JB, int NP, int BM>
__device__ __forceinline__ void gemm_group(float16_t (&acc)[4][JB], const _Float16* __restrict__ slab, int lane,
                                           const BGroup<JB>& G, const uint16_t (&sc)[JB], const uint16_t (&bi)[JB]) {
  half2_t s2[JB], b2[JB];
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const _Float16 sf = (_Float16)scale_to_f32<BF16>(sc[j]), bf = (_Float16)scale_to_f32<BF16>(bi[j]);
    s2[j] = (half2_t){sf, sf};
    b2[j] = (half2_t){bf, bf};
  }
  gemm_step<BITS, NB, JB, 0, NP, BM>(acc, slab, lane, G, s2, b2);
  gemm_step<BITS, NB, JB, 1, NP, BM>(acc, slab, lane, G, s2, b2);
  gemm_step<BITS, NB, JB, 2, NP, BM>(acc, slab, lane, G, s2, b2);
  gemm_step<BITS, NB, JB, 3, NP, BM>(acc, slab, lane, G, s2, b2);
}

template <int JB>
__device__ __forceinline__ void pair_half(const BScalePair<JB>& S, int hi, uint16_t (&sc)[JB], uint16_t (&bi)[JB]) {
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    sc[j] = (uint16_t)(hi ? S.s[j] >> 16 : S.s[j] & 0xFFFFu);
    bi[j] = (uint16_t)(hi ? S.b[j] >> 16 : S.b[j] & 0xFFFFu);
  }
}

// Workgroup barrier for the LDS slabs only: waits for this wave's LDS writes, not for its
// global loads, so the prefetched groups stay in flight across it (__syncthreads would wait for
// every outstanding load).  The memory clobber keeps the compiler from moving LDS accesses
// across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The k loop over ng groups.  Thread t stages part of slab row t / TPR from arow (a row of
// ng*64 halves; with NP = 2 planes also from arow + plane, into the second plane slab).  Every
// load is unconditional (past the last group the index is clamped, re-reading that group), so
// the wait counts before each use are exact.  BL selects where the weights come from: 0 the MLX
// tensors with per-group scales; 1 the MLX tensors with scales and biases in pairs of groups
// (one pair per loop iteration, loaded an iteration ahead; ng even); 2 the prefill copy (pairs
// padded to even, so ng may be odd).
template <int BITS, bool BF16, int NB, int JB, int BL, int BM, int NP>
__device__ __forceinline__ void gemm_mainloop(float16_t (&acc)[4][JB], _Float16* __restrict__ sA,
                                              const uint16_t* __restrict__ arow, size_t plane, const BRows<JB>& R,
                                              int ng) {
  constexpr bool SP = BL >= 1, PK = BL == 2;
  // thread t stages part t % TPR (HPT halves) of slab row t / TPR
  constexpr int SLAB = NP * BM * LDA, TPR = 256 / BM, HPT = 64 / TPR;
  const int tid = threadIdx.x, lane = tid & 63;
  _Float16* const st = sA + (tid / TPR) * LDA + HPT * (tid % TPR);
  const uint16_t* const ag = arow + HPT * (tid % TPR);
  const int last = ng - 1;
  uint32_t ar[NP][HPT / 2];
  auto a_load = [&](int g) {
#pragma unroll
    for (int p = 0; p < NP; ++p) stage_load(ag + p * plane + (size_t)g * 64, ar[p]);
  };
  auto a_store = [&](_Float16* dst) {
#pragma unroll
    for (int p = 0; p < NP; ++p) stage_store(dst + p * BM * LDA, ar[p]);
  };
  BGroup<JB> G0, G1;
  BScalePair<JB> S, Sn;
  uint16_t sc[JB], bi[JB];
  load_group<BITS, JB, !SP>(R, 0, G0);
  load_group<BITS, JB, !SP>(R, min(1, last), G1);
  if constexpr (SP) {
    load_scale_pair<JB, PK>(R, 0, S);
    load_scale_pair<JB, PK>(R, min(1, last >> 1), Sn);
  }
  a_load(0);
  a_store(st);
  a_load(min(1, last));
  lds_barrier();
  // pairs of groups (slab 0, then slab 1), so the loop has one exit; an odd last group follows
  int g = 0;
  for (; g + 1 < ng; g += 2) {
    if constexpr (SP) {
      pair_half(S, 0, sc, bi);
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA, lane, G0, sc, bi);
    } else {
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA, lane, G0, G0.s, G0.b);
    }
    load_group<BITS, JB, !SP>(R, min(g + 2, last), G0);
    a_store(st + SLAB);
    a_load(min(g + 2, last));
    lds_barrier();
    if constexpr (SP) {
      pair_half(S, 1, sc, bi);
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA + SLAB, lane, G1, sc, bi);
    } else {
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA + SLAB, lane, G1, G1.s, G1.b);
    }
    load_group<BITS, JB, !SP>(R, min(g + 3, last), G1);
    if constexpr (SP) {
      S = Sn;
      load_scale_pair<JB, PK>(R, min((g >> 1) + 2, last >> 1), Sn);
    }
    a_store(st);
    a_load(min(g + 3, last));
    lds_barrier();
  }
  if (g < ng) {  // an odd last group (scale pairs: the low half of the last, padded pair)
    if constexpr (SP) {
      pair_half(S, 0, sc, bi);
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA, lane, G0, sc, bi);
    } else {
      gemm_group<BITS, BF16, NB, JB, NP, BM>(acc, sA, lane, G0, G0.s, G0.b);
    }
  }
}

template <int JB>
__device__ __forceinline__ void zero_acc(float16_t (&acc)[4][JB]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;
}

// Columns per workgroup: gate/up waves own 32 intermediate columns of both gate and up (column
// block 0 = gate rows c0 + n, block 1 = the same up rows); down waves own 64 output columns.
constexpr int GU_COLS = 4 * 32;  // intermediate columns per gate/up workgroup
constexpr int DN_COLS = 4 * 64;  // output columns per down workgroup

// gate/up GEMM + SwiGLU.  Column tile ct covers intermediate columns [128ct, 128ct + 128); wave w
// the 32 columns c0 = 128ct + 32w + n.  Each lane holds matching gate and up values and writes
// act = silu(gate) * up (fp16, pair order within each 32-column chunk, the down projection's k
// order) for the sorted position of each row.  Scaled activations (bf16 / fp32 rows): s_xs[r]
// holds 2^-s of row r's token, applied to gate and up before the activation, and act is stored
// times 2^2s (the down GEMM takes it back); NPX = 2 multiplies each weight fragment by the hi
// and the lo plane of fp32 rows (lo plane at x + xplane).
template <int BITS, bool BF16, int ACT, int NB, int BL, int BM, int NPX>
__device__ __forceinline__ void gateup_tile(const LayerArgs& L, const uint16_t* __restrict__ x, size_t xplane,
                                            int K, const int32_t* __restrict__ perm, int e, int row0, int nrows,
                                            int ct, _Float16* sA, const float* s_xs, uint16_t* __restrict__ act,
                                            size_t plane) {
  const int H = L.H, I = L.I;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int lr = tid / (256 / BM);
  const int tok = perm[row0 + min(lr, nrows - 1)] / K;  // rows past the tile's end reload its last row
  const int c0 = ct * GU_COLS + wave * 32;
  const uint32_t rbytes = (uint32_t)H * BITS / 8, ng = (uint32_t)H / GROUP;
  BRows<2> R;
  if constexpr (BL == 2) {
    const PackProj &pg = L.pk[0], &pu = L.pk[1];
    const uint32_t rbk = (uint32_t)(c0 >> 5), npair = (ng + 1) / 2;
    R.rw[0] = make_rsrc(pg.codes + (size_t)e * pg.codes_expert, (uint32_t)pg.codes_expert);
    R.rw[1] = make_rsrc(pu.codes + (size_t)e * pu.codes_expert, (uint32_t)pu.codes_expert);
    R.rs[0] = make_rsrc(pg.sb + (size_t)e * pg.sb_expert, (uint32_t)pg.sb_expert);
    R.rs[1] = make_rsrc(pu.sb + (size_t)e * pu.sb_expert, (uint32_t)pu.sb_expert);
    R.rb[0] = R.rs[0];
    R.rb[1] = R.rs[1];
    R.vw[0] = R.vw[1] = (rbk * ng * 64u + (uint32_t)lane) * Bits<BITS>::chunk_bytes;
    R.vs[0] = R.vs[1] = (rbk * npair * 32u + (uint32_t)(lane & 31)) * 8u;
    R.gstride = 64u * Bits<BITS>::chunk_bytes;
    R.pstride = 256u;
  } else {
    const uint32_t row = (uint32_t)(c0 + (lane & 31));
    R.rw[0] = make_rsrc(L.gate.w + (size_t)e * L.gate.w_stride, (uint32_t)I * rbytes);
    R.rw[1] = make_rsrc(L.up.w + (size_t)e * L.up.w_stride, (uint32_t)I * rbytes);
    R.rs[0] = make_rsrc(L.gate.s + (size_t)e * L.gate.s_stride, (uint32_t)I * ng * 2u);
    R.rb[0] = make_rsrc(L.gate.b + (size_t)e * L.gate.s_stride, (uint32_t)I * ng * 2u);
    R.rs[1] = make_rsrc(L.up.s + (size_t)e * L.up.s_stride, (uint32_t)I * ng * 2u);
    R.rb[1] = make_rsrc(L.up.b + (size_t)e * L.up.s_stride, (uint32_t)I * ng * 2u);
    R.vw[0] = R.vw[1] = row * rbytes + (uint32_t)(lane >> 5) * Bits<BITS>::chunk_bytes;
    R.vs[0] = R.vs[1] = row * ng * 2u;
    R.gstride = 2u * Bits<BITS>::chunk_bytes;
    R.pstride = 4u;
  }
  float16_t acc[4][2];
  zero_acc(acc);
  gemm_mainloop<BITS, BF16, NB, 2, BL, BM, NPX>(acc, sA, x + (size_t)tok * H, xplane, R, (int)ng);
  // Epilogue through LDS (the slabs are free once every wave is past the k loop): per 32-row
  // block and plane (hi, then lo) the wave writes its 32 x 32 act values at their pair-order
  // columns, then each lane stores 8 consecutive columns (16 bytes) of a row.
  lds_barrier();
  uint16_t* const wst = reinterpret_cast<uint16_t*>(sA) + wave * (32 * EPA_LD);
  const int h = lane >> 5, pc = pairpos_p<BITS>(lane & 31), c8 = 8 * (lane & 3);
#pragma unroll
  for (int mb = 0; mb < NB; ++mb) {
    float a[16];
    if (s_xs) {  // gate and up times 2^-s; act stored times 2^2s
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float xs = s_xs[32 * mb + 8 * (v >> 2) + 4 * h + (v & 3)];
        a[v] = activate_p<ACT>(acc[mb][0][v] * xs, acc[mb][1][v] * xs) * (1.0f / (xs * xs));
      }
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) a[v] = activate_p<ACT>(acc[mb][0][v], acc[mb][1][v]);
    }
#pragma unroll
    for (int pl = 0; pl < 2; ++pl) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rr = 8 * (v >> 2) + 4 * h + (v & 3);
        const _Float16 hi = (_Float16)a[v];
        wst[rr * EPA_LD + pc] = pl == 0 ? __builtin_bit_cast(uint16_t, hi) : f32_to_f16_bits(a[v] - (float)hi);
      }
      asm volatile("" ::: "memory");  // one wave's LDS accesses run in order; keep them in order
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int rr = (lane >> 2) + 16 * i, r = 32 * mb + rr;
        const uint4 q = *reinterpret_cast<const uint4*>(wst + rr * EPA_LD + c8);
        if (r < nrows && c0 < I) *reinterpret_cast<uint4*>(act + pl * plane + (size_t)(row0 + r) * I + c0 + c8) = q;
      }
      asm volatile("" ::: "memory");
    }
  }
}

// BM rows per tile: 128, or 64 where the shorter tile's 64 accumulators let three gate/up or
// (down_wgs) up to four down workgroups share a CU.
template <int BITS, bool BF16, int ACT, int BL, int BM, int NPX>
__global__ __launch_bounds__(256, BM == 64 ? 3 : 2) void gemm_gateup_kernel(const LayerArgs L, const uint16_t* __restrict__ x,
                                                             size_t xplane, const float* __restrict__ xinv,
                                                             int K, const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ scalars,
                                                             const int32_t* __restrict__ mt_expert,
                                                             const int32_t* __restrict__ mt_row0,
                                                             const int32_t* __restrict__ mt_rows,
                                                             uint16_t* __restrict__ act, size_t plane) {
  __shared__ __attribute__((aligned(16))) _Float16 sA[lds_halves(BM, false, NPX)];
  __shared__ float s_xs[BM];
  int mt, ct;
  if (!xcd_mtile(blockIdx.x, (L.I + GU_COLS - 1) / GU_COLS, uniform(scalars[1]), mt, ct)) return;
  const int e = uniform(mt_expert[mt]), row0 = uniform(mt_row0[mt]), nrows = uniform(mt_rows[mt]);
  // per-row 2^-s of scaled activations (written before the k loop's first barrier)
  if (xinv) {
    for (int r = threadIdx.x; r < BM; r += 256) s_xs[r] = xinv[perm[row0 + min(r, nrows - 1)] / K];
  }
  const float* xs = xinv ? s_xs : nullptr;
#define KMOE_GUT(NBV) gateup_tile<BITS, BF16, ACT, NBV, BL, BM, NPX>(L, x, xplane, K, perm, e, row0, nrows, ct, sA, xs, act, plane)
  if constexpr (BM == 64) {
    if (nrows <= 32) KMOE_GUT(1);
    else KMOE_GUT(2);
  } else {
    switch ((nrows + 31) >> 5) {
      case 1: KMOE_GUT(1); break;
      case 2: KMOE_GUT(2); break;
      case 3: KMOE_GUT(3); break;
      default: KMOE_GUT(4); break;
    }
  }
#undef KMOE_GUT
}

// down GEMM.  Column tile ct covers output columns [256ct, 256ct + 256); wave w the 64 columns
// c0 + 32j + n with c0 = 256ct + 64w (j = 0, 1).  Row r of the tile (sorted position row0 + r)
// is written to its assignment perm[row0 + r]: fp16 unweighted (the switch_mlp contract) or fp32
// scaled by the assignment's routing weight (the fused layer, summed by combine_kernel).
template <int BITS, bool BF16, bool OUT16, int NB, int BL, int BM>
__device__ __forceinline__ void down_tile(const LayerArgs& L, int e, int row0, int nrows, int ct, _Float16* sA,
                                          const int32_t* s_asg, const float* s_wa,
                                          const uint16_t* __restrict__ act, size_t plane, float* __restrict__ y32,
                                          uint16_t* __restrict__ y16) {
  const int H = L.H, I = L.I;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int lr = tid / (256 / BM);
  const int c0 = ct * DN_COLS + wave * 64;
  const uint32_t rbytes = (uint32_t)I * BITS / 8, ng = (uint32_t)I / GROUP;
  BRows<2> R;
  if constexpr (BL == 2) {
    const PackProj& pd = L.pk[2];
    const uint32_t npair = (ng + 1) / 2;
    const auto dw = make_rsrc(pd.codes + (size_t)e * pd.codes_expert, (uint32_t)pd.codes_expert);
    const auto dsb = make_rsrc(pd.sb + (size_t)e * pd.sb_expert, (uint32_t)pd.sb_expert);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t rbk = (uint32_t)(c0 >> 5) + (uint32_t)j;
      R.rw[j] = dw;
      R.rs[j] = dsb;
      R.rb[j] = dsb;
      R.vw[j] = (rbk * ng * 64u + (uint32_t)lane) * Bits<BITS>::chunk_bytes;
      R.vs[j] = (rbk * npair * 32u + (uint32_t)(lane & 31)) * 8u;
    }
    R.gstride = 64u * Bits<BITS>::chunk_bytes;
    R.pstride = 256u;
  } else {
    const auto dw = make_rsrc(L.down.w + (size_t)e * L.down.w_stride, (uint32_t)H * rbytes);
    const auto ds = make_rsrc(L.down.s + (size_t)e * L.down.s_stride, (uint32_t)H * ng * 2u);
    const auto db = make_rsrc(L.down.b + (size_t)e * L.down.s_stride, (uint32_t)H * ng * 2u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t row = (uint32_t)(c0 + 32 * j + (lane & 31));
      R.rw[j] = dw;
      R.rs[j] = ds;
      R.rb[j] = db;
      R.vw[j] = row * rbytes + (uint32_t)(lane >> 5) * Bits<BITS>::chunk_bytes;
      R.vs[j] = row * ng * 2u;
    }
    R.gstride = 2u * Bits<BITS>::chunk_bytes;
    R.pstride = 4u;
  }
  float16_t acc[4][2];
  zero_acc(acc);
  gemm_mainloop<BITS, BF16, NB, 2, BL, BM, 2>(acc, sA, act + (size_t)(row0 + min(lr, nrows - 1)) * I, plane, R,
                                              (int)ng);
  // Epilogue through LDS (the slabs are free once every wave is past the k loop): per 32-row
  // block the wave writes its 32 x 64 results in the MFMA layout, then reads them back as rows,
  // so each lane stores 4 consecutive columns of one row (16 bytes fp32, 8 bytes fp16).
  lds_barrier();
  float* const wst = reinterpret_cast<float*>(sA) + wave * (32 * EPI_LD);
  const int h = lane >> 5, n = lane & 31, c4 = 4 * (lane & 15);
#pragma unroll
  for (int mb = 0; mb < NB; ++mb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int rr = 8 * (v >> 2) + 4 * h + (v & 3);
      wst[rr * EPI_LD + n] = acc[mb][0][v];
      wst[rr * EPI_LD + 32 + n] = acc[mb][1][v];
    }
    asm volatile("" ::: "memory");  // one wave's LDS accesses run in order; keep them in order
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = (lane >> 4) + 4 * i, r = 32 * mb + rr;
      const float4 q = *reinterpret_cast<const float4*>(wst + rr * EPI_LD + c4);
      if (r < nrows && c0 < H) {
        const size_t yo = (size_t)s_asg[r] * H + c0 + c4;
        const float wa = s_wa[r];
        if constexpr (OUT16) {
          const uint32_t lo = (uint32_t)f32_to_f16_bits(q.x * wa) | ((uint32_t)f32_to_f16_bits(q.y * wa) << 16);
          const uint32_t hi = (uint32_t)f32_to_f16_bits(q.z * wa) | ((uint32_t)f32_to_f16_bits(q.w * wa) << 16);
          *reinterpret_cast<uint2*>(y16 + yo) = make_uint2(lo, hi);
        } else {
          *reinterpret_cast<float4*>(y32 + yo) = make_float4(q.x * wa, q.y * wa, q.z * wa, q.w * wa);
        }
      }
    }
    asm volatile("" ::: "memory");
  }
}

// Workgroups per CU of the down GEMM: with 64-row tiles as many as the kernel's registers allow
// without spilling (3: the hi and lo A fragments need more than a quarter of the register file),
// two with 128-row tiles.
constexpr int down_wgs(int bits, bool bf16, int bm) {
  return bm != 64 ? 2 : 3;
}
template <int BITS, bool BF16, bool OUT16, int BL, int BM>
__global__ __launch_bounds__(256, down_wgs(BITS, BF16, BM)) void gemm_down_kernel(const LayerArgs L, const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ scalars,
                                                           const int32_t* __restrict__ mt_expert,
                                                           const int32_t* __restrict__ mt_row0,
                                                           const int32_t* __restrict__ mt_rows,
                                                           const uint16_t* __restrict__ act, size_t plane,
                                                           const float* __restrict__ wscale,
                                                           float* __restrict__ y32, uint16_t* __restrict__ y16,
                                                           const float* __restrict__ xinv, int K) {
  __shared__ __attribute__((aligned(16))) _Float16 sA[lds_halves(BM, true)];
  __shared__ int32_t s_asg[BM];  // assignment of each tile row, and its output scale: the routing
  __shared__ float s_wa[BM];     // weight, times 2^-2s of scaled activations
  int mt, ct;
  if (!xcd_mtile(blockIdx.x, (L.H + DN_COLS - 1) / DN_COLS, uniform(scalars[1]), mt, ct)) return;
  const int e = uniform(mt_expert[mt]), row0 = uniform(mt_row0[mt]), nrows = uniform(mt_rows[mt]);
  const int tid = threadIdx.x;
  if (tid < BM) {  // read after the k loop's barriers
    const int a = tid < nrows ? perm[row0 + tid] : 0;
    s_asg[tid] = a;
    float wa = wscale && tid < nrows ? wscale[a] : 1.0f;
    if (xinv) wa *= xinv[a / K] * xinv[a / K];
    s_wa[tid] = wa;
  }
  if constexpr (BM == 64) {
    if (nrows <= 32) down_tile<BITS, BF16, OUT16, 1, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16);
    else down_tile<BITS, BF16, OUT16, 2, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16);
  } else {
    switch ((nrows + 31) >> 5) {
      case 1: down_tile<BITS, BF16, OUT16, 1, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16); break;
      case 2: down_tile<BITS, BF16, OUT16, 2, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16); break;
      case 3: down_tile<BITS, BF16, OUT16, 3, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16); break;
      default: down_tile<BITS, BF16, OUT16, 4, BL, BM>(L, e, row0, nrows, ct, sA, s_asg, s_wa, act, plane, y32, y16); break;
    }
  }
}
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
                            uint16_t* y16, const float* wscale, hipStream_t s, int xdt, const float* xinv) {
  const LayerArgs& L = c.args;
  const size_t plane = (size_t)T * c.top_k * L.I;  // act lo plane offset (the workspace holds both planes)
  const int per_xcd = (max_mtiles + 7) / 8;  // m-tiles of one XCD's share at most (see xcd_mtile)
  const dim3 grid_gu(8 * per_xcd * ((L.I + GU_COLS - 1) / GU_COLS));
  // weights from the prefill copy when the layer has one, else the MLX tensors with scales in
  // pairs of groups when the rows hold an even number of groups
  const bool pk = L.pk[0].codes != nullptr;
  const int bm = gemm_bm(L, xdt, T * c.top_k);  // the m-tile list was built with this many rows per tile
  const size_t xplane = (size_t)T * L.H;  // lo plane of fp32 activations
  const int bl_gu = pk ? 2 : (L.H / GROUP) % 2 == 0 ? 1 : 0;
  const int bl_dn = pk ? 2 : (L.I / GROUP) % 2 == 0 ? 1 : 0;
#define KMOE_GU(BLV, BMV, NPXV)                                                                                \
  KMOE_LAUNCH("gemm_gateup_kernel", (gemm_gateup_kernel<BITS, BF16, ACT, BLV, BMV, NPXV>), grid_gu, dim3(256), 0, s, \
              L, x, xplane, xinv, c.top_k, w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, w.act, plane)
  if (xdt == XDT_F32) {  // two activation planes, 128-row tiles
    if (bl_gu == 2) KMOE_GU(2, 128, 2); else if (bl_gu == 1) KMOE_GU(1, 128, 2); else KMOE_GU(0, 128, 2);
  } else if (bl_gu == 2) {
    if (bm == 64) KMOE_GU(2, 64, 1); else KMOE_GU(2, 128, 1);
  } else if (bl_gu == 1) {
    if (bm == 64) KMOE_GU(1, 64, 1); else KMOE_GU(1, 128, 1);
  } else KMOE_GU(0, 128, 1);
#undef KMOE_GU
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const dim3 grid_dn(8 * per_xcd * ((L.H + DN_COLS - 1) / DN_COLS));
#define KMOE_DOWN(OUT16, BLV, BMV)                                                                              \
  KMOE_LAUNCH("gemm_down_kernel", (gemm_down_kernel<BITS, BF16, OUT16, BLV, BMV>), grid_dn, dim3(256), 0, s, L,   \
              w.perm, w.scalars, w.mt_expert, w.mt_row0, w.mt_rows, (const uint16_t*)w.act, plane, wscale,      \
              OUT16 ? (float*)nullptr : w.y32, OUT16 ? y16 : (uint16_t*)nullptr, xinv, c.top_k)
  if (y16) {
    if (bl_dn == 2) {
      if (bm == 64) KMOE_DOWN(true, 2, 64); else KMOE_DOWN(true, 2, 128);
    } else if (bl_dn == 1) {
      if (bm == 64) KMOE_DOWN(true, 1, 64); else KMOE_DOWN(true, 1, 128);
    } else KMOE_DOWN(true, 0, 128);
  } else {
    if (bl_dn == 2) {
      if (bm == 64) KMOE_DOWN(false, 2, 64); else KMOE_DOWN(false, 2, 128);
    } else if (bl_dn == 1) {
      if (bm == 64) KMOE_DOWN(false, 1, 64); else KMOE_DOWN(false, 1, 128);
    } else KMOE_DOWN(false, 0, 128);
  }
#undef KMOE_DOWN
  return hipGetLastError();
}

hipError_t launch_gemm(const LayerConfig& c, const uint16_t* x, int T, const Work& w, int max_mtiles, uint16_t* y16,
                       const float* wscale, hipStream_t s, int xdt, const float* xinv) {
  if (max_mtiles == 0) return hipSuccess;
#define KMOE_GI(B, F, A) gemm_impl<B, F, A>(c, x, T, w, max_mtiles, y16, wscale, s, xdt, xinv)
  if (c.bits == 3) {
    if (c.bf16_scales) return c.act ? KMOE_GI(3, true, 1) : KMOE_GI(3, true, 0);
    return c.act ? KMOE_GI(3, false, 1) : KMOE_GI(3, false, 0);
  }
  if (c.bf16_scales) return c.act ? KMOE_GI(4, true, 1) : KMOE_GI(4, true, 0);
  return c.act ? KMOE_GI(4, false, 1) : KMOE_GI(4, false, 0);
#undef KMOE_GI
}

// y[a] = 0 for the assignments whose expert index lies outside [0, E).  The permutation drops
// them (and sets DEVERR_BAD_EXPERT), so the grouped GEMMs never write their rows; the decode path
// writes zeros for them, and this gives the grouped path the same result.  One thread per
// assignment; only the rare bad rows store anything.
__global__ __launch_bounds__(256) void zero_bad_rows_kernel(const int32_t* __restrict__ idx, int TK, int E, int H,
                                                            uint16_t* __restrict__ y) {
  const int a = blockIdx.x * 256 + threadIdx.x;
  if (a >= TK) return;
  const int e = idx[a];
  if (e >= 0 && e < E) return;
  uint4* row = reinterpret_cast<uint4*>(y + (size_t)a * H);
  for (int q = 0; q < H / 8; ++q) row[q] = make_uint4(0u, 0u, 0u, 0u);
}

hipError_t launch_zero_bad_rows(const int32_t* idx, int TK, int E, int H, uint16_t* y, hipStream_t s) {
  if (TK == 0) return hipSuccess;
  KMOE_LAUNCH("zero_bad_rows_kernel", zero_bad_rows_kernel, dim3((TK + 255) / 256), dim3(256), 0, s, idx, TK, E, H, y);
  return hipGetLastError();
}

// One wave per token: bf16 / fp32 activations into the A layout (token_to_pairs).
template <int BITS>
__global__ __launch_bounds__(256) void xprep_kernel(const void* __restrict__ x, int xdt, int T, int H,
                                                    uint16_t* __restrict__ xpp, size_t plane,
                                                    float* __restrict__ xinv) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  token_to_pairs<BITS>(x, xdt, t, H, threadIdx.x & 63, xpp, plane, xinv);
}

hipError_t launch_xpair(const LayerConfig& c, const void* x, int xdt, int T, uint16_t* xpp, float* xinv,
                        hipStream_t s) {
  if (T == 0) return hipSuccess;
  if (xdt != XDT_F16) {
    const dim3 grid((T + 3) / 4);
    const size_t plane = (size_t)T * c.args.H;
    if (c.bits == 3)
      KMOE_LAUNCH("xprep_kernel", xprep_kernel<3>, grid, dim3(256), 0, s, x, xdt, T, c.args.H, xpp, plane, xinv);
    else
      KMOE_LAUNCH("xprep_kernel", xprep_kernel<4>, grid, dim3(256), 0, s, x, xdt, T, c.args.H, xpp, plane, xinv);
    return hipGetLastError();
  }
  const size_t nchunks = (size_t)T * c.args.H / CHUNK;
  const dim3 grid((unsigned)((nchunks + 255) / 256));
  const uint16_t* x16 = static_cast<const uint16_t*>(x);
  if (c.bits == 3) {
    KMOE_LAUNCH("xpair_kernel", xpair_kernel<3>, grid, dim3(256), 0, s, x16, nchunks, xpp);
  } else {
    KMOE_LAUNCH("xpair_kernel", xpair_kernel<4>, grid, dim3(256), 0, s, x16, nchunks, xpp);
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

// ---------------------------------------------------------------------------------------------
// Prefill weight copy.  One wavefront load of the grouped GEMMs reads, per 32-row block and
// group, the two chunks of each of the 32 rows; in the MLX layout those are 32 separate
// row-strided pieces, in the copy one contiguous 64-chunk run.  Scales and biases of a group
// pair of a row sit side by side (s0 s1 b0 b1), one 8-byte load, with an odd last group padded.
// ---------------------------------------------------------------------------------------------

PackLayout pack_layout(int H, int I, int E, int bits) {
  PackLayout p{};
  const int64_t rows[3] = {I, I, H}, in[3] = {H, H, I};
  auto up256 = [](int64_t v) { return (v + 255) & ~(int64_t)255; };
  int64_t off = 0;
  for (int q = 0; q < 3; ++q) {
    p.codes_expert[q] = rows[q] * in[q] * bits / 8;
    p.codes[q] = off;
    off = up256(off + p.codes_expert[q] * E);
  }
  for (int q = 0; q < 3; ++q) {
    const int64_t ng = in[q] / GROUP, npair = (ng + 1) / 2;
    p.sb_expert[q] = rows[q] * npair * 8;
    p.sb[q] = off;
    off = up256(off + p.sb_expert[q] * E);
  }
  p.total = off;
  return p;
}

// One thread per output chunk o = ((e*nrb + rb)*ng + g)*64 + n + 32h: chunk 2g+h of row 32rb+n.
template <int BITS>
__global__ __launch_bounds__(256) void pack_codes_kernel(const QProj P, int rows, int in, int E,
                                                         uint8_t* __restrict__ dst) {
  constexpr int CB = Bits<BITS>::chunk_bytes, CD = Bits<BITS>::chunk_dwords;
  const int ng = in / GROUP, nrb = rows / 32;
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= (size_t)E * nrb * ng * 64) return;
  const int lane = (int)(o & 63);
  size_t r = o >> 6;
  const int g = (int)(r % ng);
  r /= ng;
  const int rb = (int)(r % nrb), e = (int)(r / nrb);
  const int row = rb * 32 + (lane & 31), chunk = 2 * g + (lane >> 5);
  const size_t rbytes = (size_t)in * BITS / 8;
  const uint32_t* src =
      reinterpret_cast<const uint32_t*>(P.w + (size_t)e * P.w_stride + row * rbytes + (size_t)chunk * CB);
  uint32_t* out = reinterpret_cast<uint32_t*>(dst + o * CB);
#pragma unroll
  for (int i = 0; i < CD; ++i) out[i] = src[i];
}

// One thread per (e, rb, pair, n): s[2p] s[2p+1] b[2p] b[2p+1] of row 32rb+n (zeros past ng).
__global__ __launch_bounds__(256) void pack_sb_kernel(const QProj P, int rows, int in, int E,
                                                      uint2* __restrict__ dst) {
  const int ng = in / GROUP, npair = (ng + 1) / 2, nrb = rows / 32;
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= (size_t)E * nrb * npair * 32) return;
  const int n = (int)(o & 31);
  size_t r = o >> 5;
  const int pr = (int)(r % npair);
  r /= npair;
  const int rb = (int)(r % nrb), e = (int)(r / nrb);
  const size_t base = (size_t)e * P.s_stride + (size_t)(rb * 32 + n) * ng;
  const int g0 = 2 * pr, g1 = 2 * pr + 1;
  const uint32_t s0 = P.s[base + g0], b0 = P.b[base + g0];
  const uint32_t s1 = g1 < ng ? P.s[base + g1] : 0u, b1 = g1 < ng ? P.b[base + g1] : 0u;
  dst[o] = make_uint2(s0 | (s1 << 16), b0 | (b1 << 16));
}

hipError_t launch_prefill_pack(const LayerConfig& c, uint8_t* pack, hipStream_t s) {
  const LayerArgs& L = c.args;
  const PackLayout pl = pack_layout(L.H, L.I, L.E, c.bits);
  const QProj* proj[3] = {&L.gate, &L.up, &L.down};
  const int rows[3] = {L.I, L.I, L.H}, in[3] = {L.H, L.H, L.I};
  for (int q = 0; q < 3; ++q) {
    const size_t nc = (size_t)L.E * (rows[q] / 32) * (in[q] / GROUP) * 64;
    const dim3 gc((unsigned)((nc + 255) / 256));
    if (c.bits == 3)
      KMOE_LAUNCH("pack_codes_kernel", pack_codes_kernel<3>, gc, dim3(256), 0, s, *proj[q], rows[q], in[q], L.E,
                  pack + pl.codes[q]);
    else
      KMOE_LAUNCH("pack_codes_kernel", pack_codes_kernel<4>, gc, dim3(256), 0, s, *proj[q], rows[q], in[q], L.E,
                  pack + pl.codes[q]);
    const size_t ns = (size_t)L.E * (rows[q] / 32) * ((in[q] / GROUP + 1) / 2) * 32;
    KMOE_LAUNCH("pack_sb_kernel", pack_sb_kernel, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, s, *proj[q],
                rows[q], in[q], L.E, reinterpret_cast<uint2*>(pack + pl.sb[q]));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace kmoe
