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

// Orderable key of a logit: larger logit -> larger key; +0 and -0 equal; NaN below all.
__device__ __forceinline__ uint32_t logit_key(float v) {
  if (v != v) return 0u;
  if (v == 0.0f) v = 0.0f;
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// One wave: top-K of one logits row.  Composite key (logit key << 32 | ~index) makes the
// maximum unique and puts the lower index first among equal logits.
template <int EPL>
__device__ void wave_topk(const float* __restrict__ row, int E, int K, int32_t* __restrict__ idx_out,
                          float* __restrict__ w_out, int32_t* __restrict__ sel_lds) {
  const int lane = threadIdx.x & 63;
  uint64_t keys[EPL];
#pragma unroll
  for (int m = 0; m < EPL; ++m) {
    const int e = lane + 64 * m;
    keys[m] = e < E ? (((uint64_t)logit_key(row[e]) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e)) : 0ull;
  }
  int my_sel = 0;
  for (int k = 0; k < K; ++k) {
    uint64_t best = 0;
#pragma unroll
    for (int m = 0; m < EPL; ++m) best = keys[m] > best ? keys[m] : best;
    const uint64_t wb = wave_max_u64(best);
#pragma unroll
    for (int m = 0; m < EPL; ++m) keys[m] = keys[m] == wb ? 0ull : keys[m];
    const int e = (int)(0xFFFFFFFFu - (uint32_t)wb);
    if (lane == k) my_sel = e;
  }
  // weights: lane k < K owns selection k
  const float l0 = row[__shfl(my_sel, 0, 64)];
  float ex = 0.0f;
  if (lane < K) ex = expf(row[my_sel] - l0);
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum += __shfl(ex, k, 64);  // k order, as the reference sums
  if (lane < K) {
    idx_out[lane] = my_sel;
    w_out[lane] = ex / sum;
    if (sel_lds) sel_lds[lane] = my_sel;
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                    int32_t* __restrict__ idx, float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  wave_topk<EPL>(logits + (size_t)t * E, E, K, idx + (size_t)t * K, wts + (size_t)t * K, nullptr);
}

// Stable grouping of up to DEC_MAX_ASSIGN assignments whose experts are in LDS (one block).
__device__ void group_assignments(const int32_t* __restrict__ sh_e, int TK, int E, int32_t* __restrict__ sh_first,
                                  int32_t* __restrict__ perm, int32_t* __restrict__ ustart,
                                  int32_t* __restrict__ unique, int32_t* __restrict__ scalars) {
  for (int a = threadIdx.x; a < TK; a += blockDim.x) {
    const int e = sh_e[a];
    int before_same = 0;
    for (int b = 0; b < a; ++b) before_same += sh_e[b] == e;
    sh_first[a] = before_same == 0 && e >= 0;
  }
  __syncthreads();
  int nu_local = 0;
  for (int a = threadIdx.x; a < TK; a += blockDim.x) {
    const int e = sh_e[a];
    if (e < 0) continue;  // invalid expert index: dropped, flagged by the caller
    int less = 0, before_same = 0, uniq_less = 0;
    for (int b = 0; b < TK; ++b) {
      const int eb = sh_e[b];
      less += (eb >= 0) & (eb < e);
      before_same += (b < a) & (eb == e);
      uniq_less += sh_first[b] & (eb >= 0) & (eb < e);
    }
    perm[less + before_same] = a;
    if (sh_first[a]) {
      unique[uniq_less] = e;
      ustart[uniq_less] = less;
      nu_local++;
    }
  }
  // number of valid assignments closes the last group
  __shared__ int s_nu, s_valid;
  if (threadIdx.x == 0) { s_nu = 0; s_valid = 0; }
  __syncthreads();
  if (nu_local) atomicAdd(&s_nu, nu_local);
  int v = 0;
  for (int a = threadIdx.x; a < TK; a += blockDim.x) v += sh_e[a] >= 0;
  if (v) atomicAdd(&s_valid, v);
  __syncthreads();
  if (threadIdx.x == 0) {
    scalars[0] = s_nu;
    ustart[s_nu] = s_valid;
    if (s_valid != TK) atomicOr(&scalars[2], DEVERR_BAD_EXPERT);
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void route_group_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                          int32_t* __restrict__ idx, float* __restrict__ wts,
                                                          int32_t* __restrict__ perm, int32_t* __restrict__ ustart,
                                                          int32_t* __restrict__ unique,
                                                          int32_t* __restrict__ scalars) {
  __shared__ int32_t sh_e[DEC_MAX_ASSIGN];
  __shared__ int32_t sh_first[DEC_MAX_ASSIGN];
  for (int t = threadIdx.x >> 6; t < T; t += 4)
    wave_topk<EPL>(logits + (size_t)t * E, E, K, idx + (size_t)t * K, wts + (size_t)t * K, sh_e + t * K);
  __syncthreads();
  group_assignments(sh_e, T * K, E, sh_first, perm, ustart, unique, scalars);
}

__global__ __launch_bounds__(256) void group_small_kernel(const int32_t* __restrict__ idx, int TK, int E,
                                                          int32_t* __restrict__ perm, int32_t* __restrict__ ustart,
                                                          int32_t* __restrict__ unique,
                                                          int32_t* __restrict__ scalars) {
  __shared__ int32_t sh_e[DEC_MAX_ASSIGN];
  __shared__ int32_t sh_first[DEC_MAX_ASSIGN];
  for (int a = threadIdx.x; a < TK; a += blockDim.x) {
    const int e = idx[a];
    sh_e[a] = (e >= 0 && e < E) ? e : -1;
  }
  __syncthreads();
  group_assignments(sh_e, TK, E, sh_first, perm, ustart, unique, scalars);
}

// ---- multi-tile permutation ---------------------------------------------------------------
// Pass 1: per tile of PERM_TILE assignments, the stable rank of each assignment among the
// tile's assignments of the same expert, and the tile's expert histogram.
__global__ __launch_bounds__(256) void permute_rank_kernel(const int32_t* __restrict__ idx, int TK, int E,
                                                           int32_t* __restrict__ local_rank,
                                                           int32_t* __restrict__ tile_hist,
                                                           int32_t* __restrict__ scalars) {
  extern __shared__ int32_t sm[];
  int32_t* running = sm;       // [E]
  int32_t* cnt = sm + E;       // [4][E]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int base = blockIdx.x * PERM_TILE;
  for (int e = tid; e < E; e += 256) running[e] = 0;
  bool bad = false;
  for (int round = 0; round < PERM_TILE / 256; ++round) {
    for (int q = tid; q < 4 * E; q += 256) cnt[q] = 0;
    __syncthreads();
    const int a = base + round * 256 + tid;
    int e = a < TK ? idx[a] : -1;
    if (a < TK && (e < 0 || e >= E)) { bad = true; e = -1; }
    const bool valid = e >= 0;
    uint64_t active = __ballot(valid);
    int rank_w = 0;
    while (active) {
      const int leader = __ffsll((unsigned long long)active) - 1;
      const int el = __shfl(e, leader, 64);
      const uint64_t m = __ballot(e == el) & active;
      if (valid && e == el) rank_w = __popcll(m & ((1ull << lane) - 1ull));
      if (lane == leader) cnt[wave * E + el] = __popcll(m);
      active &= ~m;
    }
    __syncthreads();
    if (valid) {
      int pre = running[e];
      for (int w = 0; w < wave; ++w) pre += cnt[w * E + e];
      local_rank[a] = pre + rank_w;
    }
    __syncthreads();
    for (int q = tid; q < E; q += 256) running[q] += cnt[q] + cnt[E + q] + cnt[2 * E + q] + cnt[3 * E + q];
    __syncthreads();
  }
  for (int e = tid; e < E; e += 256) tile_hist[(size_t)blockIdx.x * E + e] = running[e];
  if (bad) atomicOr(&scalars[2], DEVERR_BAD_EXPERT);
}

// In-place exclusive scan of n <= 1024 ints in LDS by a 256-thread block; returns the total.
__device__ int block_exclusive_scan(int32_t* v, int n, int32_t* tmp) {
  const int tid = threadIdx.x;
  // each thread owns up to 4 consecutive entries
  int loc[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = tid * 4 + j;
    loc[j] = i < n ? v[i] : 0;
    s += loc[j];
  }
  tmp[tid] = s;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int add = tid >= off ? tmp[tid - off] : 0;
    __syncthreads();
    tmp[tid] += add;
    __syncthreads();
  }
  const int total = tmp[255];
  int run = tid > 0 ? tmp[tid - 1] : 0;
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
    int32_t* __restrict__ mt_rows) {
  __shared__ int32_t s_off[1024], s_before[1024], s_tot[1024], s_tmp[256];
  const int tid = threadIdx.x, tile = blockIdx.x;
  for (int e = tid; e < E; e += 256) {
    int tot = 0, before = 0;
    for (int tt = 0; tt < ntiles; ++tt) {
      const int h = tile_hist[(size_t)tt * E + e];
      before += tt < tile ? h : 0;
      tot += h;
    }
    s_tot[e] = tot;
    s_off[e] = tot;
    s_before[e] = before;
  }
  __syncthreads();
  const int total = block_exclusive_scan(s_off, E, s_tmp);
  const int base = tile * PERM_TILE;
  for (int i = tid; i < PERM_TILE; i += 256) {
    const int a = base + i;
    if (a < TK) {
      const int e = idx[a];
      if (e >= 0 && e < E) perm[s_off[e] + s_before[e] + local_rank[a]] = a;
    }
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
  // grouped-GEMM m-tiles: ceil(count / GEMM_BM) per expert
  __syncthreads();
  for (int e = tid; e < E; e += 256) s_before[e] = (s_tot[e] + GEMM_BM - 1) / GEMM_BM;
  __syncthreads();
  const int nmt = block_exclusive_scan(s_before, E, s_tmp);
  for (int e = tid; e < E; e += 256) {
    const int n = (s_tot[e] + GEMM_BM - 1) / GEMM_BM;
    for (int j = 0; j < n; ++j) {
      const int m = s_before[e] + j;
      mt_expert[m] = e;
      mt_row0[m] = s_off[e] + j * GEMM_BM;
      mt_rows[m] = min(GEMM_BM, s_tot[e] - j * GEMM_BM);
    }
  }
  if (tid == 0) {
    scalars[0] = nu;
    scalars[1] = nmt;
    ustart[nu] = total;
  }
}

// ---- launchers --------------------------------------------------------------------------
static int epl_for(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16; }

template <int EPL>
static void route_launch(const float* logits, int T, int E, int K, int32_t* idx, float* wts, hipStream_t s) {
  hipLaunchKernelGGL(route_kernel<EPL>, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, K, idx, wts);
}

template <int EPL>
static void route_group_launch(const float* logits, int T, int E, int K, int32_t* idx, float* wts, int32_t* perm,
                               int32_t* ustart, int32_t* unique, int32_t* scalars, hipStream_t s) {
  hipLaunchKernelGGL(route_group_kernel<EPL>, dim3(1), dim3(256), 0, s, logits, T, E, K, idx, wts, perm, ustart,
                     unique, scalars);
}

hipError_t launch_route(const float* logits, int T, int E, int K, int32_t* idx, float* wts, hipStream_t s) {
  if (T == 0) return hipSuccess;
  switch (epl_for(E)) {
    case 1: route_launch<1>(logits, T, E, K, idx, wts, s); break;
    case 2: route_launch<2>(logits, T, E, K, idx, wts, s); break;
    case 4: route_launch<4>(logits, T, E, K, idx, wts, s); break;
    case 8: route_launch<8>(logits, T, E, K, idx, wts, s); break;
    default: route_launch<16>(logits, T, E, K, idx, wts, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_route_group(const float* logits, int T, int E, int K, int32_t* idx, float* wts, int32_t* perm,
                              int32_t* ustart, int32_t* unique, int32_t* scalars, hipStream_t s) {
  switch (epl_for(E)) {
    case 1: route_group_launch<1>(logits, T, E, K, idx, wts, perm, ustart, unique, scalars, s); break;
    case 2: route_group_launch<2>(logits, T, E, K, idx, wts, perm, ustart, unique, scalars, s); break;
    case 4: route_group_launch<4>(logits, T, E, K, idx, wts, perm, ustart, unique, scalars, s); break;
    case 8: route_group_launch<8>(logits, T, E, K, idx, wts, perm, ustart, unique, scalars, s); break;
    default: route_group_launch<16>(logits, T, E, K, idx, wts, perm, ustart, unique, scalars, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_group_small(const int32_t* idx, int T, int K, int E, int32_t* perm, int32_t* ustart,
                              int32_t* unique, int32_t* scalars, hipStream_t s) {
  hipLaunchKernelGGL(group_small_kernel, dim3(1), dim3(256), 0, s, idx, T * K, E, perm, ustart, unique, scalars);
  return hipGetLastError();
}

hipError_t launch_permute(const int32_t* idx, int TK, int K, int E, const Work& w, int max_mtiles, hipStream_t s) {
  (void)K;
  (void)max_mtiles;
  const int ntiles = (TK + PERM_TILE - 1) / PERM_TILE;
  if (ntiles == 0) return hipSuccess;
  hipLaunchKernelGGL(permute_rank_kernel, dim3(ntiles), dim3(256), (size_t)5 * E * sizeof(int32_t), s, idx, TK, E,
                     w.local_rank, w.tile_hist, w.scalars);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(permute_scatter_kernel, dim3(ntiles), dim3(256), 0, s, idx, TK, E, ntiles, w.local_rank,
                     w.tile_hist, w.perm, w.counts, w.offsets, w.unique, w.ustart, w.scalars, w.mt_expert,
                     w.mt_row0, w.mt_rows);
  return hipGetLastError();
}

}  // namespace kmoe
