// Device-side building blocks shared by every kernel of the routed-expert layer (gfx950).
//
// Chunks and pair order
// ---------------------
// Quantized rows are processed in chunks of 32 codes: 12 bytes (3 dwords) for 3-bit
// codes, 16 bytes (4 dwords) for 4-bit codes, both dword aligned.  A chunk is unpacked
// into 16 "pairs": a 32-bit word whose low half holds one code and whose high half
// holds another, each in bits 0..2 (3-bit) / 0..3 (4-bit) of its half.  The pair order
// is chosen so that unpacking is a packed 16-bit shift plus one mask per pair (see
// unpack3/unpack4 below); since a dot product is a sum, the activations only have to be
// stored in the same order ("pair order") for the products to line up.  Activation
// vectors handed between kernels (x staged in LDS, the SwiGLU output `act`) are stored
// per 32-element chunk in pair order: position 2p holds element pair_lo(p) and
// position 2p+1 holds element pair_hi(p).
//
// A pair word is used in one of two ways:
//   * raw:   the half-words are fp16 subnormals q * 2^-24; v_dot2_f32_f16 against fp16
//            activations accumulates exact products q*x*2^-24 in fp32, and the group
//            scale/bias are applied once per 32 columns: s*2^24*dot + b*sum(x).
//   * magic: OR 0x6400 gives the fp16 value 1024+q; subtracting 1024 gives q exactly and
//            one fp16 fma gives the dequantized weight round(q*s + b) (MFMA operands).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace kmoe {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int GROUP = 64;
constexpr int CHUNK = 32;  // codes per chunk

template <int BITS>
struct Bits {
  static constexpr int chunk_bytes = BITS * 4;       // 12 or 16
  static constexpr int chunk_dwords = BITS;           // 3 or 4
  static constexpr uint32_t mask = BITS == 3 ? 0x00070007u : 0x000F000Fu;
};

// Pair tables: element index (0..31 within the chunk) of the low / high half of pair p.
//   3-bit: (0,6)(1,7)(2,8)(3,9)(11,16)(12,17)(13,18)(14,19)(15,20)(22,27)(23,28)(24,29)
//          (25,30)(4,31)(5,26)(10,21)
//   4-bit: (8j+i, 8j+i+4) for j = 0..3, i = 0..3
__host__ __device__ constexpr int pair_lo(int bits, int p) {
  return bits == 3 ? (p < 4 ? p : p < 9 ? p + 7 : p < 13 ? p + 13 : p == 13 ? 4 : p == 14 ? 5 : 10)
                   : 8 * (p >> 2) + (p & 3);
}
__host__ __device__ constexpr int pair_hi(int bits, int p) {
  return bits == 3 ? (p < 4 ? p + 6 : p < 9 ? p + 12 : p < 13 ? p + 18 : p == 13 ? 31 : p == 14 ? 26 : 21)
                   : 8 * (p >> 2) + (p & 3) + 4;
}
// Storage position (0..31) of element e of a chunk in pair order.
__host__ __device__ constexpr int pair_pos(int bits, int e) {
  int pos = 0;
  for (int p = 0; p < 16; ++p) {
    if (pair_lo(bits, p) == e) pos = 2 * p;
    if (pair_hi(bits, p) == e) pos = 2 * p + 1;
  }
  return pos;
}

__device__ __forceinline__ uint32_t pk_shr(uint32_t v, unsigned lo, unsigned hi) {
  u16x2_t x = __builtin_bit_cast(u16x2_t, v);
  u16x2_t s = {(unsigned short)lo, (unsigned short)hi};
  return __builtin_bit_cast(uint32_t, x >> s);
}

// v_perm_b32: result byte i = byte sel_i of {S1 bytes 0..3, S0 bytes 4..7}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// 3-bit chunk (dwords d0..d2, codes c_j at bits 3j of the 96-bit stream) -> 16 pairs.
// (v & M) | O in one v_and_or_b32 when O != 0.  gfx9 VOP3 encodes no literal and reads at most
// one SGPR, so M goes in an SGPR and O in a VGPR (both loop-invariant).
template <uint32_t M, uint32_t O>
__device__ __forceinline__ uint32_t mask_or(uint32_t v) {
  if constexpr (O == 0u) {
    return v & M;
  } else {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(M), "v"(O));
    return r;
  }
}

// Pair P (0..15) of a 3-bit chunk.  Pairs 0-3 come from d0, 4-8 from d1, 9-12 from d2 (one
// packed shift each); 13-15 hold the codes that straddle dword boundaries or sit in the other
// half-word.
template <int P, bool MAGIC>
__device__ __forceinline__ uint32_t pair3(uint32_t d0, uint32_t d1, uint32_t d2) {
  constexpr uint32_t M = 0x00070007u, O = MAGIC ? 0x64006400u : 0u;
  if constexpr (P < 4) {
    return mask_or<M, O>(pk_shr(d0, 3 * P, 3 * P + 2));
  } else if constexpr (P < 9) {
    return mask_or<M, O>(pk_shr(d1, 3 * (P - 4) + 1, 3 * (P - 4)));
  } else if constexpr (P < 13) {
    return mask_or<M, O>(pk_shr(d2, 3 * (P - 9) + 2, 3 * (P - 9) + 1));
  } else if constexpr (P == 13) {
    // c4: d0 bits 12..14 (low half); c31: d2 bits 29..31 (high half, relative 13)
    return mask_or<M, O>(pk_shr((d0 & 0xFFFFu) | (d2 & 0xFFFF0000u), 12, 13));
  } else if constexpr (P == 14) {
    // c5: d0 bits 15..17; c26: d2 bits 14..16.  Bytes [d0.b1 d0.b2 | d2.b1 d2.b2] put them at 7 / 6.
    return mask_or<M, O>(pk_shr(perm_b32(d2, d0, 0x06050201u), 7, 6));
  } else {
    // c10: stream bits 30..32; c21: stream bits 63..65.
    const uint32_t c10 = __builtin_amdgcn_alignbit(d1, d0, 30);
    const uint32_t c21 = __builtin_amdgcn_alignbit(d2, d1, 31);
    return mask_or<M, O>(perm_b32(c21, c10, 0x05040100u));
  }
}

template <bool MAGIC>
__device__ __forceinline__ void unpack3(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t (&p)[16]) {
  p[0] = pair3<0, MAGIC>(d0, d1, d2);
  p[1] = pair3<1, MAGIC>(d0, d1, d2);
  p[2] = pair3<2, MAGIC>(d0, d1, d2);
  p[3] = pair3<3, MAGIC>(d0, d1, d2);
  p[4] = pair3<4, MAGIC>(d0, d1, d2);
  p[5] = pair3<5, MAGIC>(d0, d1, d2);
  p[6] = pair3<6, MAGIC>(d0, d1, d2);
  p[7] = pair3<7, MAGIC>(d0, d1, d2);
  p[8] = pair3<8, MAGIC>(d0, d1, d2);
  p[9] = pair3<9, MAGIC>(d0, d1, d2);
  p[10] = pair3<10, MAGIC>(d0, d1, d2);
  p[11] = pair3<11, MAGIC>(d0, d1, d2);
  p[12] = pair3<12, MAGIC>(d0, d1, d2);
  p[13] = pair3<13, MAGIC>(d0, d1, d2);
  p[14] = pair3<14, MAGIC>(d0, d1, d2);
  p[15] = pair3<15, MAGIC>(d0, d1, d2);
}

// 4-bit chunk (dwords d0..d3, nibble n of dword j = code 8j+n) -> 16 pairs.
template <bool MAGIC>
__device__ __forceinline__ void unpack4(const uint32_t (&d)[4], uint32_t (&p)[16]) {
  constexpr uint32_t M = 0x000F000Fu, O = MAGIC ? 0x64006400u : 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p[4 * j + i] = mask_or<M, O>(d[j] >> (4 * i));
  }
}

// Pair P of a chunk of either width.
template <int BITS, int P, bool MAGIC>
__device__ __forceinline__ uint32_t chunk_pair(const uint32_t (&d)[4]) {
  if constexpr (BITS == 3) {
    return pair3<P, MAGIC>(d[0], d[1], d[2]);
  } else {
    constexpr uint32_t M = 0x000F000Fu, O = MAGIC ? 0x64006400u : 0u;
    return mask_or<M, O>(d[P >> 2] >> (4 * (P & 3)));
  }
}

template <int BITS, bool MAGIC>
__device__ __forceinline__ void unpack_chunk(const uint32_t (&d)[4], uint32_t (&p)[16]) {
  if constexpr (BITS == 3) {
    unpack3<MAGIC>(d[0], d[1], d[2], p);
  } else {
    unpack4<MAGIC>(d, p);
  }
}

// Load one chunk of packed codes (3 or 4 dwords; the address is dword aligned).
template <int BITS>
__device__ __forceinline__ void load_chunk(const uint8_t* __restrict__ row, int chunk, uint32_t (&d)[4]) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(row + (size_t)chunk * Bits<BITS>::chunk_bytes);
  if constexpr (BITS == 3) {
    d[0] = __builtin_nontemporal_load(src + 0);
    d[1] = __builtin_nontemporal_load(src + 1);
    d[2] = __builtin_nontemporal_load(src + 2);
    d[3] = 0;
  } else {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
  }
}

// Permute 32 natural-order fp16 values (16 dwords, dword m = elements 2m, 2m+1) into pair order.
// 32 fp16 values (64 bytes) between memory and registers, as four 16-byte accesses.
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

template <int BITS>
__device__ __forceinline__ void to_pair_order(const uint32_t (&nat)[16], uint32_t (&out)[16]) {
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int lo = pair_lo(BITS, p), hi = pair_hi(BITS, p);
    const uint32_t sel_lo = (lo & 1) ? 0x0302u : 0x0100u;        // bytes of S1 (low half source)
    const uint32_t sel_hi = (hi & 1) ? 0x07060000u : 0x05040000u; // bytes of S0 (high half source)
    out[p] = perm_b32(nat[hi >> 1], nat[lo >> 1], sel_hi | sel_lo);
  }
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

// Sum of the 16 pair-dot products of a raw code chunk with an activation chunk (both pair order).
__device__ __forceinline__ float chunk_dot(const uint32_t (&codes)[16], const uint32_t (&x)[16]) {
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int p = 0; p < 16; p += 2) {
    a0 = fdot2(codes[p], x[p], a0);
    a1 = fdot2(codes[p + 1], x[p + 1], a1);
  }
  return a0 + a1;
}

template <bool BF16>
__device__ __forceinline__ float scale_to_f32(uint16_t v) {
  if constexpr (BF16) {
    return __uint_as_float((uint32_t)v << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, v);
  }
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t v) {
  return (float)__builtin_bit_cast(_Float16, v);
}

// Dequantize a magic pair word (each half 0x6400|q) to fp16 weights round(q*s + b).
__device__ __forceinline__ uint32_t dequant_pair(uint32_t magic_pair, half2_t s2, half2_t b2) {
  const half2_t q = __builtin_bit_cast(half2_t, magic_pair) - (half2_t){(_Float16)1024.0f, (_Float16)1024.0f};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s2, b2));  // one rounding: round(q*s + b)
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// DPP move of a 32-bit value (lanes whose source is masked off receive 0).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL, ROW_MASK>(__float_as_uint(v)));
}

// Sum over aligned groups of `width` consecutive lanes (a power of two <= 64) with DPP; the
// group's last lane holds the total (every lane of the group does for width <= 16).
__device__ __forceinline__ float group_sum_last(float v, int width) {
  if (width >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  if (width >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  if (width == 8) v += dpp_f32<0x141>(v);  // row_half_mirror: quad q meets quad q^1
  if (width >= 16) {
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
  }
  if (width >= 32) v += dpp_f32<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  if (width >= 64) v += dpp_f32<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// Wave64 sum with DPP: quad_perm [1,0,3,2], [2,3,0,1], row_ror 4, 8 give every lane its row
// sum; row_bcast 15 (rows 1,3) and row_bcast 31 (rows 2,3) accumulate rows into lane 63.
// Returns the total in every lane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x124>(v);
  v += dpp_f32<0x128>(v);
  v += dpp_f32<0x142, 0xA>(v);
  v += dpp_f32<0x143, 0xC>(v);
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
}

// Sums V per-lane values (V = 4 or 8) over the wave in one pass.  Each step halves the values a
// lane carries: v_permlane32_swap / v_permlane16_swap (gfx950) hand one value of every pair to
// the partner half, so each half sums a different value, then DPP finishes inside 16-lane rows.
// The total of value v ends in every lane of lane group v: lanes 8v..8v+7 for V = 8 and
// 16v..16v+15 for V = 4.  About 3V/2 + 6 instructions, against 7V for V separate reductions.
template <int V>
__device__ __forceinline__ float wave_sum_multi(const float (&v)[V]) {
  static_assert(V == 4 || V == 8, "V must be 4 or 8");
  float w[V / 2];
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {
    // lanes 0-31 end with v[i] of lanes l and l+32, lanes 32-63 with v[i + V/2] of l-32 and l
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + V / 2]), false,
                                                    false);
    w[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float x[V / 4];
#pragma unroll
  for (int i = 0; i < V / 4; ++i) {
    // rows 0 and 2 end with w[i] of rows (0,1) and (2,3); rows 1 and 3 with w[i + V/4]
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[i]), __float_as_uint(w[i + V / 4]), false,
                                                    false);
    x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float y;
  if constexpr (V == 8) {
    // lanes with bit 3 clear keep x[0] and lanes with it set keep x[1], each adding lane l ^ 8's
    const bool b3 = (__lane_id() & 8) != 0;
    const float keep = b3 ? x[1] : x[0], give = b3 ? x[0] : x[1];
    y = keep + dpp_f32<0x128>(give);  // row_ror:8
    y += dpp_f32<0xB1>(y);            // quad_perm [1,0,3,2]
    y += dpp_f32<0x4E>(y);            // quad_perm [2,3,0,1]
    y += dpp_f32<0x141>(y);           // row_half_mirror
  } else {
    y = x[0];
    y += dpp_f32<0x128>(y);
    y += dpp_f32<0x141>(y);
    y += dpp_f32<0xB1>(y);
    y += dpp_f32<0x4E>(y);
  }
  return y;
}

// Buffer resource over `bytes` bytes at `base` (raw, untyped dword access; loads past the end
// return zero).  Built in scalar registers when its arguments are uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int BUF_NT = 2;  // cache-policy bit of a buffer load: non-temporal (streamed once)

// One chunk of packed codes through a buffer resource: byte offset voff (per lane) + soff (uniform).
template <int BITS>
__device__ __forceinline__ void buf_chunk(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t (&d)[4]) {
  if constexpr (BITS == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, BUF_NT);
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = 0;
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, BUF_NT);
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
  }
}

__device__ __forceinline__ uint16_t buf_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// One chunk of packed codes through a buffer resource with the default (cached) policy: the
// grouped GEMMs read each expert's weights once per m-tile, so they are kept in L2.
template <int BITS>
__device__ __forceinline__ void buf_chunk_cached(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                 uint32_t (&d)[4]) {
  if constexpr (BITS == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = 0;
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
  }
}

// ---- scaled activations (bf16 and fp32 rows) ---------------------------------------------
// A bf16 or fp32 activation row is taken as fp16 planes of x * 2^s: hi = fp16(x 2^s), and for
// fp32 rows lo = fp16(x 2^s - hi) (hi + lo carries ~22 bits).  s = 0 when the row's largest
// magnitude m lies in [2^-4, 2^4) (the rows a normalised model feeds the layer); otherwise 2^s is
// the power of two that puts m in [1, 2).  Every bf16 element of magnitude at least 2^-14 m is
// then exact in hi (8 mantissa bits inside fp16's 11, no overflow) and smaller ones keep 2^-24 m
// absolute precision, so bf16's whole range is usable.  The gate/up products are taken on the
// scaled row and multiplied by 2^-s in fp32 (exact); the SwiGLU output, which grows with the
// square of the row, is stored times 2^2s, and the down projection's result is multiplied by
// 2^-2s, so the fp16 act planes stay in range for rows far outside fp16's.  With s = 0 the
// arithmetic is the fp16 path's, so fp16-representable rows in that window give its results bit
// for bit.  A row that is all zero or holds an infinity keeps s = 0 (non-finite values propagate).

// s for a row whose largest magnitude is amax (NaN elements do not take part).
__device__ __forceinline__ int row_scale_exp(float amax) {
  if (!(amax > 0.f) || !__builtin_isfinite(amax)) return 0;
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127;  // floor(log2 amax) (normal amax)
  if (e >= -4 && e < 4) return 0;
  return min(60, max(-60, -e));
}
__device__ __forceinline__ float exp2i(int s) { return __uint_as_float((uint32_t)(127 + s) << 23); }

// 32 consecutive activations of a bf16 (xdt 1) or fp32 (xdt 2) row, as fp32.
__device__ __forceinline__ void load_chunk_vals(const void* p, int xdt, float (&v)[32]) {
  if (xdt == 1) {
    uint32_t w[16];
    load16g(p, w);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 t = q[i];
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
  }
}

__device__ __forceinline__ float chunk_amax(const float (&v)[32]) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(v[i]));
  return m;
}

// hi and lo planes of v * k as fp16 pairs in natural order (element 2i low, 2i+1 high).
__device__ __forceinline__ void split_chunk(const float (&v)[32], float k, uint32_t (&hi)[16], uint32_t (&lo)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float a = v[2 * i] * k, b = v[2 * i + 1] * k;
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    const _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
    hi[i] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    lo[i] = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
  }
}

// Issue priority of the calling wave by its work left (wave-uniform `left`, capped at 3).  Two
// workgroups share each CU in the decode stages; by default the older one's waves win issue and
// finish first, leaving the younger one to run its tail alone.  Waves with more work left take
// precedence instead, so the two keep pace.
__device__ __forceinline__ void prio_by_work_left(int left) {
  if (left >= 3)
    __builtin_amdgcn_s_setprio(3);
  else if (left == 2)
    __builtin_amdgcn_s_setprio(2);
  else if (left == 1)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

// Orderable key of a router logit: larger logit -> larger key, +0 == -0, NaN below all.
__device__ __forceinline__ uint32_t logit_key(float v) {
  if (v != v) return 0u;
  if (v == 0.0f) v = 0.0f;
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Inverse of logit_key (the NaN key 0 maps back to a NaN).
__device__ __forceinline__ float logit_from_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Wave64 maximum of unsigned 32-bit values (0 is the identity), same DPP pattern.
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x124>(v));
  v = max(v, dpp_u32<0x128>(v));
  v = max(v, dpp_u32<0x142, 0xA>(v));
  v = max(v, dpp_u32<0x143, 0xC>(v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Top-K of one token's router logits by one wave (moe_block.metal:479-503 semantics): order by
// logit descending, equal logits to the lower index; weights exp(l_k - l_max) / sum_j
// exp(l_j - l_max), summed in k order.  Each lane holds EPL logits (EPL * 64 >= E), sorted once
// by (key desc, index asc).  A round is a 32-bit DPP max over the lanes' head keys; a ballot
// finds the lanes holding it, and only when two lanes hold the same logit does a second max
// over the inverted indices pick the lower index.  The winning lane then pops its head.
// Index e lives in lane e % 64, so the winner's lane follows from its index.
// Lane k < K returns the k-th expert in `sel` and its weight in `selw`; other lanes get -1, 0.
constexpr int TOPK_MAX_EPL = 16;  // logits per lane for up to 1024 experts

// Loads lane l's logits row[l + 64m] (m < ceil(E/64), zero past E) for wave_topk_vals, so the
// loads can be issued early and other work done while they are in flight.
__device__ __forceinline__ void wave_load_logits(const float* __restrict__ row, int E, float (&lv)[TOPK_MAX_EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < TOPK_MAX_EPL; ++m) {
    const int e = lane + 64 * m;
    lv[m] = 64 * m < E && e < E ? row[e] : 0.0f;
  }
}

// The selection half of the top-K: lane k < K gets the k-th expert in `sel` and its logit in
// `sel_l`; other lanes get -1 and 0.
template <int EPL>
__device__ __forceinline__ void wave_topk_select(const float (&lv)[TOPK_MAX_EPL], int E, int K, int& sel,
                                                 float& sel_l) {
  const int lane = threadIdx.x & 63;
  uint32_t kh[EPL], ke[EPL];  // key, ~index (larger ~index = lower index); padding: key 0, ~index 0
#pragma unroll
  for (int m = 0; m < EPL; ++m) {
    const int e = lane + 64 * m;
    kh[m] = e < E ? logit_key(lv[m]) : 0u;
    ke[m] = e < E ? ~(uint32_t)e : 0u;
  }
  // odd-even transposition sort, descending by key.  It swaps only on a strictly larger key,
  // so equal keys keep their order, which is ascending index (padding, at the largest m, last).
#pragma unroll
  for (int pass = 0; pass < EPL; ++pass) {
#pragma unroll
    for (int j = pass & 1; j + 1 < EPL; j += 2) {
      const bool sw = kh[j + 1] > kh[j];
      const uint32_t h0 = kh[j], e0 = ke[j];
      kh[j] = sw ? kh[j + 1] : h0;
      ke[j] = sw ? ke[j + 1] : e0;
      kh[j + 1] = sw ? h0 : kh[j + 1];
      ke[j + 1] = sw ? e0 : ke[j + 1];
    }
  }
  int my = -1;
  float my_l = 0.0f;
  for (int k = 0; k < K; ++k) {
    const uint32_t m = wave_max_u32_dpp(kh[0]);
    const bool hold = kh[0] == m;
    const uint64_t holders = __ballot(hold);
    int e;
    bool pop;
    if (__popcll(holders) == 1) {
      // the one holder pops; the index it held is only needed for the output
      e = (int)~(uint32_t)__builtin_amdgcn_readlane((int)ke[0], (int)__builtin_ctzll(holders));
      pop = hold;
    } else {
      e = (int)~wave_max_u32_dpp(hold ? ke[0] : 0u);
      pop = lane == (e & 63);
    }
    if (pop) {
#pragma unroll
      for (int j = 0; j + 1 < EPL; ++j) {
        kh[j] = kh[j + 1];
        ke[j] = ke[j + 1];
      }
      kh[EPL - 1] = 0u;
      ke[EPL - 1] = 0u;
    }
    if (lane == k) {
      my = e;
      my_l = logit_from_key(m);
    }
  }
  sel = my;
  sel_l = my_l;
}

// The weights half: lanes k < K hold the selected logits l_k (l_0 the largest); returns
// exp(l_k - l_0) / sum_j exp(l_j - l_0), the sum taken in k order, in lane k and 0 elsewhere.
__device__ __forceinline__ float topk_weight(float sel_l, int K) {
  const int lane = threadIdx.x & 63;
  const float l0 = __uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(sel_l)));
  const float ex = lane < K ? expf(sel_l - l0) : 0.0f;
  float sum = 0.0f;
  for (int k = 0; k < K; ++k)
    sum += __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(ex), k));
  return lane < K ? ex / sum : 0.0f;
}

template <int EPL>
__device__ __forceinline__ void wave_topk_vals(const float (&lv)[TOPK_MAX_EPL], int E, int K, int& sel, float& selw) {
  float sel_l;
  wave_topk_select<EPL>(lv, E, K, sel, sel_l);
  selw = topk_weight(sel_l, K);
}

template <int EPL>
__device__ __forceinline__ void wave_topk_regs(const float* __restrict__ row, int E, int K, int& sel, float& selw) {
  float lv[TOPK_MAX_EPL];
  wave_load_logits(row, E, lv);
  wave_topk_vals<EPL>(lv, E, K, sel, selw);
}

template <int EPL>
__device__ __forceinline__ void wave_topk_select_regs(const float* __restrict__ row, int E, int K, int& sel,
                                                      float& sel_l) {
  float lv[TOPK_MAX_EPL];
  wave_load_logits(row, E, lv);
  wave_topk_select<EPL>(lv, E, K, sel, sel_l);
}

// wave_topk_regs with the results stored: lanes k < K write idx_out[k] / w_out[k] (either may
// be null) and sel[k] / selw[k] (may be null).
template <int EPL>
__device__ __forceinline__ void wave_topk(const float* __restrict__ row, int E, int K, int32_t* idx_out,
                                          float* w_out, int32_t* sel, float* selw) {
  const int lane = threadIdx.x & 63;
  int e;
  float w;
  wave_topk_regs<EPL>(row, E, K, e, w);
  if (lane < K) {
    if (idx_out) idx_out[lane] = e;
    if (w_out) w_out[lane] = w;
    if (sel) sel[lane] = e;
    if (selw) selw[lane] = w;
  }
}

// Runtime E -> EPL dispatch helper for callers.
#define KMOE_TOPK_DISPATCH(E, CALL)      \
  do {                                   \
    if ((E) <= 64) {                     \
      constexpr int EPL_ = 1;            \
      CALL;                              \
    } else if ((E) <= 128) {             \
      constexpr int EPL_ = 2;            \
      CALL;                              \
    } else if ((E) <= 256) {             \
      constexpr int EPL_ = 4;            \
      CALL;                              \
    } else if ((E) <= 512) {             \
      constexpr int EPL_ = 8;            \
      CALL;                              \
    } else {                             \
      constexpr int EPL_ = 16;           \
      CALL;                              \
    }                                    \
  } while (0)

// Exclusive prefix count of `flag` over the threads of a 256-thread block, plus the total.
// Uses ballots and a 4-entry LDS array `tmp`; every thread must call it.
__device__ __forceinline__ int block_prefix_count(bool flag, int32_t* tmp, int* total) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint64_t m = __ballot(flag);
  if (lane == 0) tmp[wave] = __popcll(m);
  __syncthreads();
  int before = __popcll(m & ((1ull << lane) - 1ull));
  int tot = 0;
  for (int w = 0; w < 4; ++w) {
    const int c = tmp[w];
    before += w < wave ? c : 0;
    tot += c;
  }
  __syncthreads();
  *total = tot;
  return before;
}

// One wave writes token t's activations into the grouped GEMM's A layout: xpp row t in pair
// order (per 32-wide chunk).  fp16 rows (xdt 0) are permuted as they are; bf16 (1) and fp32 (2)
// rows are scaled (see the scaled activations above: xinv[t] = 2^-s), the hi plane going to xpp
// and, for fp32, the lo plane to xpp + plane.  Two passes over the row for bf16/fp32 (the largest
// magnitude first, the second pass mostly from L2).
template <int BITS>
__device__ __forceinline__ void token_to_pairs(const void* x, int xdt, int t, int H, int lane, uint16_t* xpp,
                                               size_t plane, float* xinv) {
  const int nch = H / CHUNK;
  if (xdt == 0) {
    const uint16_t* xr = static_cast<const uint16_t*>(x) + (size_t)t * H;
    for (int c = lane; c < nch; c += 64) {
      uint32_t nat[16], pr[16];
      load16g(xr + c * CHUNK, nat);
      to_pair_order<BITS>(nat, pr);
      store16s(reinterpret_cast<_Float16*>(xpp + (size_t)t * H + c * CHUNK), pr);
    }
    return;
  }
  const int eb = xdt == 2 ? 4 : 2;
  const char* xr = static_cast<const char*>(x) + (size_t)t * H * eb;
  float amax = 0.f;
  for (int c = lane; c < nch; c += 64) {
    float v[32];
    load_chunk_vals(xr + (size_t)c * CHUNK * eb, xdt, v);
    amax = fmaxf(amax, chunk_amax(v));
  }
  const int sx = row_scale_exp(__uint_as_float(wave_max_u32_dpp(__float_as_uint(amax))));
  if (lane == 0) xinv[t] = exp2i(-sx);
  const float k = exp2i(sx);
  for (int c = lane; c < nch; c += 64) {
    float v[32];
    uint32_t hi[16], lo[16], pr[16];
    load_chunk_vals(xr + (size_t)c * CHUNK * eb, xdt, v);
    split_chunk(v, k, hi, lo);
    to_pair_order<BITS>(hi, pr);
    store16s(reinterpret_cast<_Float16*>(xpp + (size_t)t * H + c * CHUNK), pr);
    if (xdt == 2) {
      to_pair_order<BITS>(lo, pr);
      store16s(reinterpret_cast<_Float16*>(xpp + plane + (size_t)t * H + c * CHUNK), pr);
    }
  }
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float gelu_tanh_f32(float g) {
  const float t = 0.7978845608f * (g + 0.044715f * g * g * g);
  return 0.5f * g * (1.0f + tanhf(t));
}

}  // namespace kmoe
