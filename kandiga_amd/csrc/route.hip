// Router top-K and the token -> expert permutation.
//
// Router (kandiga/metal/moe_block.metal:419-505, router_softmax_topk): per token the K
// experts with the largest router logits, ties going to the lower expert index, and
// weights w_k = p_k / sum_{j in top-K} p_j with p = softmax(logits).  The full-softmax
// denominator cancels, so w_k = exp(l_k - l_max) / sum_j exp(l_j - l_max) over the K
// selected logits.  Softmax is monotone in the logit, so selecting on the logit gives the
// probability ranking without evaluating a transcendental in the comparison: indices are
// reproducible bit for bit on any device.
//
// Permutation (kandiga/engine.py:407-418): the T*K assignments a = t*K + k are grouped
// by expert in a stable order (expert ascending, then a ascending), with group boundaries
// and the ascending list of distinct experts.  The multi-tile version ranks each tile of
// 1024 assignments with wave ballots (no atomics, so the order is deterministic) and then
// scatters with per-tile expert offsets.
#include "kmoe_device.h"
#include "kmoe_internal.h"

namespace kmoe {

template <int UNUSED = 0>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                    int32_t* __restrict__ idx, float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  int32_t* io = idx + (size_t)t * K;
  float* wo = wts + (size_t)t * K;
  KMOE_TOPK_DISPATCH(E, (wave_topk<EPL_>(row, E, K, io, wo, nullptr, nullptr)));
}

// ---- multi-tile permutation ---------------------------------------------------------------
// Pass 1: per tile of PERM_TILE assignments, the stable rank of each assignment among the
// tile's assignments of the same expert, and the tile's expert histogram.
// Routing plus the pair-order copy of x that the grouped GEMMs read (the GEMM path of the
// fused layer): the wave that routes token t also rewrites its H/32 chunks of x.
template <int BITS>
__global__ __launch_bounds__(256) void route_xpair_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                          int32_t* __restrict__ idx, float* __restrict__ wts,
                                                          const void* __restrict__ x, int xdt, int H,
                                                          uint16_t* __restrict__ xpp, size_t plane,
                                                          float* __restrict__ xinv) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  int32_t* io = idx + (size_t)t * K;
  float* wo = wts + (size_t)t * K;
  KMOE_TOPK_DISPATCH(E, (wave_topk<EPL_>(row, E, K, io, wo, nullptr, nullptr)));
  token_to_pairs<BITS>(x, xdt, t, H, lane, xpp, plane, xinv);
}

__global__ __launch_bounds__(256) void permute_rank_kernel(const int32_t* __restrict__ idx, int TK, int E,
                                                           int32_t* __restrict__ local_rank,
                                                           int32_t* __restrict__ tile_hist,
                                                           int32_t* __restrict__ scalars) {
  // Per round of 256 assignments, lane l of wave w sets bit l of lanes[w][e] for its expert e;
  // its stable rank in the tile is then the count of its expert so far in earlier rounds, in
  // waves before w, and in lanes of w below l.
  extern __shared__ unsigned long long sm64[];
  unsigned long long* lanes = sm64;                          // [4][E]
  int32_t* running = reinterpret_cast<int32_t*>(sm64 + 4 * E);  // [E]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int base = blockIdx.x * PERM_TILE;
  // every round's expert id is loaded up front: one memory round trip instead of one per round
  constexpr int ROUNDS = PERM_TILE / 256;
  int32_t ev[ROUNDS];
#pragma unroll
  for (int round = 0; round < ROUNDS; ++round) {
    const int a = base + round * 256 + tid;
    ev[round] = a < TK ? idx[a] : -1;
  }
  for (int q = tid; q < 4 * E; q += 256) lanes[q] = 0;
  for (int e = tid; e < E; e += 256) running[e] = 0;
  __syncthreads();
  bool bad = false;
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int round = 0; round < ROUNDS; ++round) {
    const int a = base + round * 256 + tid;
    int e = ev[round];
    if (a < TK && (e < 0 || e >= E)) { bad = true; e = -1; }
    const bool valid = e >= 0;
    if (valid) atomicOr(&lanes[wave * E + e], 1ull << lane);
    __syncthreads();
    if (valid) {
      int pre = running[e] + __popcll(lanes[wave * E + e] & below);
      for (int w = 0; w < wave; ++w) pre += __popcll(lanes[w * E + e]);
      local_rank[a] = pre;
    }
    __syncthreads();
    for (int q = tid; q < E; q += 256) {
      running[q] += __popcll(lanes[q]) + __popcll(lanes[E + q]) + __popcll(lanes[2 * E + q]) +
                    __popcll(lanes[3 * E + q]);
      lanes[q] = lanes[E + q] = lanes[2 * E + q] = lanes[3 * E + q] = 0;
    }
    __syncthreads();
  }
  for (int e = tid; e < E; e += 256) tile_hist[(size_t)blockIdx.x * E + e] = running[e];
  if (bad) atomicOr(&scalars[2], DEVERR_BAD_EXPERT);
}

// In-place exclusive scan of n <= 1024 ints in LDS by a 256-thread block; returns the total.
__device__ int block_exclusive_scan(int32_t* v, int n, int32_t* tmp) {
  // n <= 1024: thread t owns entries 4t..4t+3; a shuffle scan per wave, then the four wave
  // totals through tmp (two barriers in all)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int loc[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid * 4 + j;
    loc[j] = i < n ? v[i] : 0;
    s += loc[j];
  }
  int incl = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off, 64);
    if (lane >= off) incl += t;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int run = incl - s;
  for (int w = 0; w < wave; ++w) run += tmp[w];
  const int total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid * 4 + j;
    if (i < n) v[i] = run;
    run += loc[j];
  }
  __syncthreads();
  return total;
}

// Pass 2: expert offsets, scatter, and (block 0) counts / unique experts / GEMM tile list.
__global__ __launch_bounds__(256) void permute_scatter_kernel(
    const int32_t* __restrict__ idx, int TK, int E, int ntiles, const int32_t* __restrict__ local_rank,
    const int32_t* __restrict__ tile_hist, int32_t* __restrict__ perm, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ unique, int32_t* __restrict__ ustart,
    int32_t* __restrict__ scalars, int32_t* __restrict__ mt_expert, int32_t* __restrict__ mt_row0,
    int32_t* __restrict__ mt_rows, int bm) {
  __shared__ int32_t s_off[1024], s_before[1024], s_tot[1024], s_tmp[256];
  const int tid = threadIdx.x, tile = blockIdx.x;
  const int base = tile * PERM_TILE;
  // the tile's expert ids and ranks are loaded first, in flight with the histogram loads below
  constexpr int PER_THREAD = PERM_TILE / 256;
  int32_t ev[PER_THREAD], rk[PER_THREAD];
#pragma unroll
  for (int j = 0; j < PER_THREAD; ++j) {
    const int a = base + tid + 256 * j;
    ev[j] = a < TK ? idx[a] : -1;
    rk[j] = a < TK ? local_rank[a] : 0;
  }
  for (int e = tid; e < E; e += 256) {
    // eight independent partial sums, so the tile counts are loaded back to back
    int tot8[8] = {}, bef8[8] = {};
    int tt = 0;
    for (; tt + 8 <= ntiles; tt += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int h = tile_hist[(size_t)(tt + u) * E + e];
        bef8[u] += tt + u < tile ? h : 0;
        tot8[u] += h;
      }
    }
    for (; tt < ntiles; ++tt) {
      const int h = tile_hist[(size_t)tt * E + e];
      bef8[0] += tt < tile ? h : 0;
      tot8[0] += h;
    }
    int tot = 0, before = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      tot += tot8[u];
      before += bef8[u];
    }
    s_tot[e] = tot;
    s_off[e] = tot;
    s_before[e] = before;
  }
  __syncthreads();
  const int total = block_exclusive_scan(s_off, E, s_tmp);
#pragma unroll
  for (int j = 0; j < PER_THREAD; ++j) {
    const int a = base + tid + 256 * j, e = ev[j];
    if (a < TK && e >= 0 && e < E) perm[s_off[e] + s_before[e] + rk[j]] = a;
  }
  if (tile != 0) return;
  for (int e = tid; e < E; e += 256) {
    counts[e] = s_tot[e];
    offsets[e] = s_off[e];
  }
  if (tid == 0) offsets[E] = total;
  // unique experts (ascending) and their group starts
  __syncthreads();
  for (int e = tid; e < E; e += 256) s_before[e] = s_tot[e] > 0;
  __syncthreads();
  const int nu = block_exclusive_scan(s_before, E, s_tmp);
  for (int e = tid; e < E; e += 256) {
    if (s_tot[e] > 0) {
      unique[s_before[e]] = e;
      ustart[s_before[e]] = s_off[e];
    }
  }
  // grouped-GEMM m-tiles: ceil(count / bm) per expert
  __syncthreads();
  for (int e = tid; e < E; e += 256) s_before[e] = (s_tot[e] + bm - 1) / bm;
  __syncthreads();
  const int nmt = block_exclusive_scan(s_before, E, s_tmp);
  for (int e = tid; e < E; e += 256) {
    const int n = (s_tot[e] + bm - 1) / bm;
    for (int j = 0; j < n; ++j) {
      const int m = s_before[e] + j;
      mt_expert[m] = e;
      mt_row0[m] = s_off[e] + j * bm;
      mt_rows[m] = min(bm, s_tot[e] - j * bm);
    }
  }
  if (tid == 0) {
    scalars[0] = nu;
    scalars[1] = nmt;
    ustart[nu] = total;
  }
}

// ---- launchers --------------------------------------------------------------------------
hipError_t launch_route(const float* logits, int T, int E, int K, int32_t* idx, float* wts, hipStream_t s) {
  if (T == 0) return hipSuccess;
  KMOE_LAUNCH("route_kernel", route_kernel<0>, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, K, idx, wts);
  return hipGetLastError();
}

hipError_t launch_route_xpair(const float* logits, int T, int E, int K, int32_t* idx, float* wts, const void* x,
                              int xdt, int H, int bits, uint16_t* xpp, float* xinv, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const dim3 grid((T + 3) / 4);
  const size_t plane = (size_t)T * H;
  if (bits == 3)
    KMOE_LAUNCH("route_xpair_kernel", route_xpair_kernel<3>, grid, dim3(256), 0, s, logits, T, E, K, idx, wts, x, xdt,
                H, xpp, plane, xinv);
  else
    KMOE_LAUNCH("route_xpair_kernel", route_xpair_kernel<4>, grid, dim3(256), 0, s, logits, T, E, K, idx, wts, x, xdt,
                H, xpp, plane, xinv);
  return hipGetLastError();
}

hipError_t launch_permute(const int32_t* idx, int TK, int K, int E, const Work& w, int max_mtiles, int bm,
                          hipStream_t s) {
  (void)K;
  (void)max_mtiles;
  const int ntiles = (TK + PERM_TILE - 1) / PERM_TILE;
  if (ntiles == 0) return hipSuccess;
  KMOE_LAUNCH("permute_rank_kernel", permute_rank_kernel, dim3(ntiles), dim3(256),
              (size_t)4 * E * sizeof(unsigned long long) + (size_t)E * sizeof(int32_t), s, idx, TK, E,
                     w.local_rank, w.tile_hist, w.scalars);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  KMOE_LAUNCH("permute_scatter_kernel", permute_scatter_kernel, dim3(ntiles), dim3(256), 0, s, idx, TK, E, ntiles, w.local_rank,
                     w.tile_hist, w.perm, w.counts, w.offsets, w.unique, w.ustart, w.scalars, w.mt_expert,
                     w.mt_row0, w.mt_rows, bm);
  return hipGetLastError();
}

}  // namespace kmoe
