// Router projection of the MoE block over MLX group-quantized weights (the body of the qlinear
// launch, also run by extra workgroups of the shared layer's decode stage 1).  Included by the
// kernel sources after kmoe_device.h and kmoe_internal.h.
#pragma once

namespace kmoe {

constexpr int QL_TB = 4;    // tokens per workgroup
constexpr int QL_RPW = 2;   // rows per wave
constexpr uint32_t QL_ONE2 = 0x3C003C00u;
constexpr float QL_TWO24 = 16777216.0f;

// Rows [8 bx, 8 bx + 8) of the stacked projections A (ra rows) then B (rb rows) against tokens
// [4 by, 4 by + 4): one workgroup of the qlinear launch (block index (bx, by)).
// RPW rows per wave: 2 for a few tokens (more workgroups, shorter chains), 8 for many tokens
// (each token's pair-order conversion then serves 8 rows instead of 2).
template <int BITS, bool BF16, int RPW = QL_RPW>
__device__ __forceinline__ void qlinear_rows(const QProj& A, int ra, const QProj& B, int rb, int T, int H,
                                             const uint16_t* __restrict__ x, float* __restrict__ out_a,
                                             float* __restrict__ out_b, int bx, int by) {
  static_assert((RPW * QL_TB) % 8 == 0, "values reduce eight at a time");
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int R = ra + rb;
  const int t0 = by * QL_TB;
  const int r0 = (bx * 4 + wave) * RPW;
  const int nch = H / CHUNK, ng = H / GROUP;
  const size_t rbytes = (size_t)H * BITS / 8;
  float acc[RPW * QL_TB];
#pragma unroll
  for (int v = 0; v < RPW * QL_TB; ++v) acc[v] = 0.f;
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
    for (int r = 0; r < RPW; ++r) {
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
#pragma unroll
  for (int gv = 0; gv < RPW * QL_TB; gv += 8) {
    // value v = gv + k (v = r*QL_TB + t) lands in lanes 8k..8k+7
    const float tot = wave_sum_multi<8>(*reinterpret_cast<const float(*)[8]>(acc + gv));
    if ((lane & 7) == 0) {
      const int v = gv + (lane >> 3), r = v / QL_TB, t = v - r * QL_TB;
      const int row = r0 + r, tok = t0 + t;
      if (row < R && tok < T) {
        if (row < ra)
          out_a[(size_t)tok * ra + row] = tot;
        else
          out_b[(size_t)tok * rb + (row - ra)] = tot;
      }
    }
  }
}

// Workgroups of a qlinear launch over R rows and T tokens: row blocks x token blocks.
inline int qlinear_row_blocks(int R, int rpw = QL_RPW) { return (R + 4 * rpw - 1) / (4 * rpw); }
inline int qlinear_token_blocks(int T) { return (T + QL_TB - 1) / QL_TB; }

}  // namespace kmoe
