// Q4_K expert rows dotted with activations on the int8 dot instruction
// (v_dot4c_i32_i8: four int8 products summed into an int32 per lane op).
//
// Activation terms ("a8"). Each 16-element block b of an fp32 vector x is
// written as two int8 terms on one scale:
//   s_b = max_j |x_j| / 127,  hi_j = rint(x_j / s_b),  r_j = x_j - hi_j s_b,
//   lo_j = rint(254 r_j / s_b),  x~_j = s_b (hi_j + lo_j / 254),  e_j = x_j - x~_j
// with |e_j| <= s_b / 508 = max|x| / 64516 (|r_j| <= s_b / 2 keeps lo_j in
// [-127, 127]); a block of zeros, or of values below 1e-30, has s_b = 0.
// A Q4_K sub-block of 32 elements meets two x-blocks: for codes q_j, scale
// d*sc and min dmin*m (compute/quant.py:24-56 dequant_q4_k)
//   sum_j (d sc q_j - dmin m) x_j = sum over its two x-blocks b of
//     d sc (s_b / 254) (254 sum q hi + sum q lo)  +  d sc sum_j q_j e_j  -  dmin m sum_j x_j
// The integer sums are exact (|254 sum q hi + sum q lo| < 2^23, so their
// conversion to float is exact too) and sum_j x_j is the fp32 sum of the
// block. The error term d sc sum q_j e_j is taken at the codes' midpoint,
// 8 d sc E_b with E_b = sum_j e_j (kept with the terms), which leaves
// d sc sum (q_j - 8) e_j: codes are 0..15, so the part that every row of a
// matrix shares -- the codes' mean times E_b -- drops out (a Qwen3-shaped
// layer: ~2e-5 of max|y| against ~1e-4 without it, numpy model). Blocks of 16
// rather than 32 let a producer that holds 16 consecutive elements -- a
// gate/up workgroup's 48 rows -- write finished terms.
//
// Layout of a vector's terms. nq = K / 64 block pairs; pair q holds
// elements 64 q .. 64 q + 63, the two Q4_K sub-blocks whose codes share the
// bytes 32 g .. 32 g + 31 of a super-block (g = q & 3; low nibbles: sub-block
// 2g, high nibbles: 2g + 1), and x-blocks 4q .. 4q + 3 (x-block 4q + 2 s + h:
// elements 16 h .. 16 h + 15 of sub-block 2g + s). Pair q's 176 bytes are 11
// chunks of 16 bytes, chunk c at byte (c * nq + q) * 16, so that lanes q, q +
// 1, ... read consecutive chunks:
//   c 2 s + h:      hi terms of x-block 4q + 2 s + h     (s, h in 0..1)
//   c 4 + 2 s + h:  lo terms of x-block 4q + 2 s + h
//   c 8:  float s_b / 254 for x-blocks 4q .. 4q + 3
//   c 9:  float sum x over x-blocks 4q .. 4q + 3
//   c 10: float 8 E_b for x-blocks 4q .. 4q + 3
// Every kernel that reads terms gets them from a8_pair16 below, so kernels
// that share a row's arithmetic give identical bits.
#pragma once

#include "nsx_common.h"

constexpr int A8_PAIR_BYTES = 176;  // terms of one 64-element block pair

__host__ __device__ constexpr int64_t a8_bytes(int64_t K) { return (K / 64) * A8_PAIR_BYTES; }

// DPP quad permutations (lane xor 1, lane xor 2) and row mirrors
constexpr int A8_DPP_XOR1 = 0xB1, A8_DPP_XOR2 = 0x4E, A8_DPP_HALF_MIRROR = 0x141, A8_DPP_MIRROR = 0x140;

__device__ __forceinline__ int a8_i8(float v) { return (int)fminf(fmaxf(v, -127.f), 127.f) & 0xff; }

// Terms of x-block xb (16 elements) of a vector: the two lanes 2i, 2i + 1
// (both active) hold its elements, lane 2i + h elements 8 h .. 8 h + 7 in v.
// Writes them into the vector's terms at dst. (Multiplications by constants
// stand in for the divisions by 127 and 254: every producer runs this same
// function, so the terms are the same bits everywhere.)
__device__ __forceinline__ void a8_pair16(const float (&v)[8], int xb, int nq, uint8_t* dst) {
  const int hl = __lane_id() & 1;
  float amax = 0.f, sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    amax = fmaxf(amax, fabsf(v[j]));
    sum += v[j];
  }
  amax = fmaxf(amax, nsx_dpp_f<A8_DPP_XOR1>(amax));
  sum += nsx_dpp_f<A8_DPP_XOR1>(sum);  // a + b == b + a: both lanes hold the same bits
  const bool live = amax >= 1e-30f;
  const float s = live ? amax * (1.f / 127.f) : 0.f;
  const float inv = live ? 127.f * __builtin_amdgcn_rcpf(amax) : 0.f;
  const float s254 = s * (1.f / 254.f), inv254 = inv * 254.f;
  uint32_t hi[2] = {0u, 0u}, lo[2] = {0u, 0u};
  float err = 0.f;  // sum of x_j - s (hi_j + lo_j / 254) over the lane's elements
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = fminf(fmaxf(rintf(v[j] * inv), -127.f), 127.f);
    const float r = fmaf(-a, s, v[j]);
    const float b = fminf(fmaxf(rintf(r * inv254), -127.f), 127.f);
    err += fmaf(-b, s254, r);
    hi[j >> 2] |= (uint32_t)a8_i8(a) << (8 * (j & 3));
    lo[j >> 2] |= (uint32_t)a8_i8(b) << (8 * (j & 3));
  }
  err += nsx_dpp_f<A8_DPP_XOR1>(err);
  const int q = xb >> 2, c = xb & 3;  // chunk of the hi terms; lo terms: c + 4
  *(v2u*)(dst + ((int64_t)c * nq + q) * 16 + 8 * hl) = v2u{hi[0], hi[1]};
  *(v2u*)(dst + ((int64_t)(c + 4) * nq + q) * 16 + 8 * hl) = v2u{lo[0], lo[1]};
  if (hl == 0) {
    ((float*)(dst + ((int64_t)8 * nq + q) * 16))[c] = s254;
    ((float*)(dst + ((int64_t)9 * nq + q) * 16))[c] = sum;
    ((float*)(dst + ((int64_t)10 * nq + q) * 16))[c] = 8.f * err;
  }
}

// The terms of one block pair, as a lane holds them.
struct A8Pair {
  v4u t[8];  // chunks 0-7
  v4f s;     // chunk 8: s_b / 254 of the four x-blocks
  v2f sum;   // sum x over each sub-block (x-blocks 4q + 0 + 1, 4q + 2 + 3)
  v2f e8;    // 8 E over each sub-block
};

template <typename P>
__device__ __forceinline__ void a8_load(const P* base, int q, int nq, A8Pair& X) {
  const uint8_t* b = (const uint8_t*)base;
#pragma unroll
  for (int c = 0; c < 8; ++c) X.t[c] = *(const v4u*)(b + ((int64_t)c * nq + q) * 16);
  X.s = *(const v4f*)(b + ((int64_t)8 * nq + q) * 16);
  const v4f sm = *(const v4f*)(b + ((int64_t)9 * nq + q) * 16), e8 = *(const v4f*)(b + ((int64_t)10 * nq + q) * 16);
  X.sum = v2f{sm.x + sm.y, sm.z + sm.w};
  X.e8 = v2f{e8.x + e8.y, e8.z + e8.w};
}

// Dot product of block pair g = q & 3 of a Q4_K super-block (c0, c1: its 32
// code bytes 32 g .. 32 g + 31; hd: the super-block's d | dmin << 16 and 12
// scale bytes) with the pair's activation terms.
__device__ __forceinline__ float q4k_a8_dot(const v4u& c0, const v4u& c1, const v4u& hd, int g, const A8Pair& X) {
  int a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};  // per x-block: sum q hi, sum q lo
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = i < 4 ? c0[i & 3] : c1[i & 3];
    const int lo = (int)(w & 0x0f0f0f0fu), hi = (int)((w >> 4) & 0x0f0f0f0fu);
    const int h = i >> 2, di = i & 3;  // elements 16 h + 4 di .. of sub-blocks 2g (lo) and 2g + 1 (hi)
    a[h] = __builtin_amdgcn_sdot4(lo, (int)X.t[h][di], a[h], false);
    b[h] = __builtin_amdgcn_sdot4(lo, (int)X.t[4 + h][di], b[h], false);
    a[2 + h] = __builtin_amdgcn_sdot4(hi, (int)X.t[2 + h][di], a[2 + h], false);
    b[2 + h] = __builtin_amdgcn_sdot4(hi, (int)X.t[6 + h][di], b[2 + h], false);
  }
  float t[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) t[j] = (float)(a[j] * 254 + b[j]);
  // get_scale_min_k4 (compute/quant.py:24-40) of sub-blocks 2g and 2g + 1, both
  // at once: bytes 2 (g & 1) and 2 (g & 1) + 1 of the scale words, as 16 bits
  const uint32_t sh = 16u * (uint32_t)(g & 1);
  const uint32_t y = hd.y >> sh, z = hd.z >> sh, w = hd.w >> sh;
  const bool upper = g >= 2;  // sub-blocks 4..7: low bits in w, top two bits in y / z
  const uint32_t sc = upper ? ((w & 0x0f0fu) | ((y >> 2) & 0x3030u)) : (y & 0x3f3fu);
  const uint32_t mn = upper ? (((w >> 4) & 0x0f0fu) | ((z >> 2) & 0x3030u)) : (z & 0x3f3fu);
  const float d = nsx_h2f(hd.x & 0xffffu), dmin = nsx_h2f(hd.x >> 16);
  const float dsc0 = d * nsx_ub<0>(sc), dsc1 = d * nsx_ub<1>(sc);  // exact: 11-bit x 6-bit
  const float m0 = fmaf(dsc0, X.e8.x, -(dmin * nsx_ub<0>(mn)) * X.sum.x);
  const float m1 = fmaf(dsc1, X.e8.y, -(dmin * nsx_ub<1>(mn)) * X.sum.y);
  const float r0 = fmaf(dsc0 * X.s.x, t[0], fmaf(dsc0 * X.s.y, t[1], m0));
  const float r1 = fmaf(dsc1 * X.s.z, t[2], fmaf(dsc1 * X.s.w, t[3], m1));
  return r0 + r1;
}

// Sum over each group of LPR consecutive lanes (LPR in 4, 8, 16, 32, 64; every
// lane active). Every lane of a group gets the same bits.
template <int LPR>
__device__ __forceinline__ float a8_group_sum(float v) {
  static_assert(LPR == 4 || LPR == 8 || LPR == 16 || LPR == 32 || LPR == 64, "group of 4..64 lanes");
  v += nsx_dpp_f<A8_DPP_XOR1>(v);
  v += nsx_dpp_f<A8_DPP_XOR2>(v);
  if constexpr (LPR >= 8) v += nsx_dpp_f<A8_DPP_HALF_MIRROR>(v);
  if constexpr (LPR >= 16) v += nsx_dpp_f<A8_DPP_MIRROR>(v);
  if constexpr (LPR >= 32) {
    auto rl = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
    const float s01 = rl(0) + rl(16), s23 = rl(32) + rl(48);
    if constexpr (LPR == 32) return (__lane_id() & 32) ? s23 : s01;
    return s01 + s23;
  }
  return v;
}

// lanes per row for a dot of K elements: K / 64 block pairs rounded up to a power of two (>= 4)
__host__ __device__ constexpr int q4k_lpr(int K) {
  const int nq = K / 64;
  return nq <= 4 ? 4 : nq <= 8 ? 8 : nq <= 16 ? 16 : nq <= 32 ? 32 : 64;
}

// Producer of a whole vector's terms: 8-element slices over `threads` lanes
// starting at thread index `tid` (an even number apart).
__device__ __forceinline__ void a8_vector(const float* __restrict__ x, int K, uint8_t* dst, int tid, int threads) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  const int nq = K / 64;
  for (int i = tid; i < K / 8; i += threads) {  // K / 8 and threads are even: lane pairs stay whole
    const v4f lo = *(gv4f*)(x + 8 * i), hi = *(gv4f*)(x + 8 * i + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    a8_pair16(v, i >> 1, nq, dst);
  }
}
