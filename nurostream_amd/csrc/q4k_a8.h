// Q4_K expert rows dotted with activations on the int8 dot instruction
// (v_dot4c_i32_i8: four int8 products summed into an int32 per lane op).
//
// Activation terms ("a8"). Each 32-element block b of an fp32 vector x is
// written as two int8 terms on one scale:
//   s_b = max_j |x_j| / 127,  hi_j = rint(x_j / s_b),  r_j = x_j - hi_j s_b,
//   lo_j = rint(254 r_j / s_b),  x~_j = s_b (hi_j + lo_j / 254),  e_j = x_j - x~_j
// with |e_j| <= s_b / 508 = max|x| / 64516 (|r_j| <= s_b / 2 keeps lo_j in
// [-127, 127]); a block of zeros, or of values below 1e-30, has s_b = 0.
// A Q4_K sub-block is 32 elements, so one sub-block meets one x-block: for
// codes q_j, scale d*sc and min dmin*m (compute/quant.py:24-56 dequant_q4_k)
//   sum_j (d sc q_j - dmin m) x_j
//     = d sc (s_b / 254) (254 sum q hi + sum q lo)  +  d sc sum_j q_j e_j  -  dmin m sum_j x_j
// The integer sums are exact (|254 sum q hi + sum q lo| < 2^24, so their
// conversion to float is exact too) and sum_j x_j is the fp32 sum of the
// block. The error term d sc sum q_j e_j is taken at the codes' midpoint,
// 8 d sc E_b with E_b = sum_j e_j (kept with the terms), which leaves
// d sc sum (q_j - 8) e_j: codes are 0..15, so the part that every row of a
// matrix shares -- the codes' mean times E_b -- drops out (a Qwen3-shaped
// layer: ~2e-5 of max|y| against ~1e-4 without it, numpy model).
//
// Layout of a vector's terms. nq = K / 64 block pairs; pair q holds blocks
// 2q and 2q + 1 (the two sub-blocks whose codes share the bytes 32 g .. 32 g
// + 31 of a super-block, g = q & 3: low nibbles block 2q, high nibbles block
// 2q + 1). Pair q's 160 bytes are 10 chunks of 16 bytes, chunk c at byte
// (c * nq + q) * 16, so that lanes q, q + 1, ... read consecutive chunks:
//   c 0, 1: hi terms of block 2q (elements 0-15, 16-31)   c 2, 3: of block 2q + 1
//   c 4, 5: lo terms of block 2q                            c 6, 7: of block 2q + 1
//   c 8:    float {s_2q / 254, s_2q+1 / 254, sum x over block 2q, over block 2q + 1}
//   c 9:    float {8 E_2q, 8 E_2q+1, 0, 0}
// Every kernel that reads terms gets them from a8_quad below, so kernels
// that share a row's arithmetic give identical bits.
#pragma once

#include "nsx_common.h"

constexpr int A8_PAIR_BYTES = 160;  // terms of one 64-element block pair

__host__ __device__ constexpr int64_t a8_bytes(int64_t K) { return (K / 64) * A8_PAIR_BYTES; }

// DPP quad permutations (lane xor 1, lane xor 2) and row mirrors
constexpr int A8_DPP_XOR1 = 0xB1, A8_DPP_XOR2 = 0x4E, A8_DPP_HALF_MIRROR = 0x141, A8_DPP_MIRROR = 0x140;

__device__ __forceinline__ int a8_i8(float v) { return (int)fminf(fmaxf(v, -127.f), 127.f) & 0xff; }

// Terms of block `blk` of a vector: the four lanes of a DPP quad (lanes 4i ..
// 4i + 3, all active) hold its elements, quad lane ql = lane & 3 elements
// 8 ql .. 8 ql + 7 in v. Writes them into the vector's terms at dst.
__device__ __forceinline__ void a8_quad(const float (&v)[8], int blk, int nq, uint8_t* dst) {
  const int ql = __lane_id() & 3;
  float amax = 0.f, sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    amax = fmaxf(amax, fabsf(v[j]));
    sum += v[j];
  }
  amax = fmaxf(amax, nsx_dpp_f<A8_DPP_XOR1>(amax));
  amax = fmaxf(amax, nsx_dpp_f<A8_DPP_XOR2>(amax));
  sum += nsx_dpp_f<A8_DPP_XOR1>(sum);  // a + b == b + a: every quad lane holds the same bits
  sum += nsx_dpp_f<A8_DPP_XOR2>(sum);
  const bool live = amax >= 1e-30f;
  const float s = live ? amax / 127.f : 0.f;
  const float inv = live ? 127.f / amax : 0.f;
  const float s254 = s / 254.f;
  uint32_t hi[2] = {0u, 0u}, lo[2] = {0u, 0u};
  float err = 0.f;  // sum of x_j - s (hi_j + lo_j / 254) over the lane's elements
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = fminf(fmaxf(rintf(v[j] * inv), -127.f), 127.f);
    const float r = fmaf(-a, s, v[j]);
    const float b = fminf(fmaxf(rintf(r * inv * 254.f), -127.f), 127.f);
    err += fmaf(-b, s254, r);
    hi[j >> 2] |= (uint32_t)a8_i8(a) << (8 * (j & 3));
    lo[j >> 2] |= (uint32_t)a8_i8(b) << (8 * (j & 3));
  }
  err += nsx_dpp_f<A8_DPP_XOR1>(err);
  err += nsx_dpp_f<A8_DPP_XOR2>(err);
  const int q = blk >> 1, hb = blk & 1;
  const int c = 2 * hb + (ql >> 1);  // chunk of the hi terms; lo terms: c + 4
  *(v2u*)(dst + ((int64_t)c * nq + q) * 16 + 8 * (ql & 1)) = v2u{hi[0], hi[1]};
  *(v2u*)(dst + ((int64_t)(c + 4) * nq + q) * 16 + 8 * (ql & 1)) = v2u{lo[0], lo[1]};
  if (ql == 0) {
    float* sc = (float*)(dst + ((int64_t)8 * nq + q) * 16);
    sc[hb] = s254;
    sc[2 + hb] = sum;
    float* ec = (float*)(dst + ((int64_t)9 * nq + q) * 16);
    ec[hb] = 8.f * err;
    ec[2 + hb] = 0.f;
  }
}

// The terms of one block pair, as a lane holds them.
struct A8Pair {
  v4u t[8];  // chunks 0-7
  v4f s;     // chunk 8
  v2f e;     // chunk 9 (its first half)
};

template <typename P>
__device__ __forceinline__ void a8_load(const P* base, int q, int nq, A8Pair& X) {
#pragma unroll
  for (int c = 0; c < 8; ++c) X.t[c] = *(const v4u*)((const uint8_t*)base + ((int64_t)c * nq + q) * 16);
  X.s = *(const v4f*)((const uint8_t*)base + ((int64_t)8 * nq + q) * 16);
  X.e = *(const v2f*)((const uint8_t*)base + ((int64_t)9 * nq + q) * 16);
}

// Dot product of block pair g = q & 3 of a Q4_K super-block (c0, c1: its 32
// code bytes 32 g .. 32 g + 31; hd: the super-block's d | dmin << 16 and 12
// scale bytes) with the pair's activation terms.
__device__ __forceinline__ float q4k_a8_dot(const v4u& c0, const v4u& c1, const v4u& hd, int g, const A8Pair& X) {
  int a0 = 0, b0 = 0, a1 = 0, b1 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = i < 4 ? c0[i & 3] : c1[i & 3];
    const int lo = (int)(w & 0x0f0f0f0fu), hi = (int)((w >> 4) & 0x0f0f0f0fu);
    const int ci = i >> 2, di = i & 3;
    a0 = __builtin_amdgcn_sdot4(lo, (int)X.t[ci][di], a0, false);
    b0 = __builtin_amdgcn_sdot4(lo, (int)X.t[4 + ci][di], b0, false);
    a1 = __builtin_amdgcn_sdot4(hi, (int)X.t[2 + ci][di], a1, false);
    b1 = __builtin_amdgcn_sdot4(hi, (int)X.t[6 + ci][di], b1, false);
  }
  const float t0 = (float)(a0 * 254 + b0), t1 = (float)(a1 * 254 + b1);
  // get_scale_min_k4 (compute/quant.py:24-40) of sub-blocks 2g and 2g + 1, both
  // at once: bytes 2 (g & 1) and 2 (g & 1) + 1 of the scale words, as 16 bits
  const uint32_t sh = 16u * (uint32_t)(g & 1);
  const uint32_t y = hd.y >> sh, z = hd.z >> sh, w = hd.w >> sh;
  const bool upper = g >= 2;  // sub-blocks 4..7: low bits in w, top two bits in y / z
  const uint32_t sc = upper ? ((w & 0x0f0fu) | ((y >> 2) & 0x3030u)) : (y & 0x3f3fu);
  const uint32_t mn = upper ? (((w >> 4) & 0x0f0fu) | ((z >> 2) & 0x3030u)) : (z & 0x3f3fu);
  const float d = nsx_h2f(hd.x & 0xffffu), dmin = nsx_h2f(hd.x >> 16);
  const float dsc0 = d * nsx_ub<0>(sc), dsc1 = d * nsx_ub<1>(sc);  // exact: 11-bit x 6-bit
  const float r0 = fmaf(dsc0 * X.s.x, t0, fmaf(dsc0, X.e.x, -(dmin * nsx_ub<0>(mn)) * X.s.z));
  const float r1 = fmaf(dsc1 * X.s.y, t1, fmaf(dsc1, X.e.y, -(dmin * nsx_ub<1>(mn)) * X.s.w));
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

// Producer of a whole vector's terms: block quads over `threads` lanes
// starting at thread index `tid` (a multiple of 4 apart).
__device__ __forceinline__ void a8_vector(const float* __restrict__ x, int K, uint8_t* dst, int tid, int threads) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  const int nq = K / 64;
  for (int i = tid; i < K / 8; i += threads) {  // K / 8 and threads are multiples of 4: quads stay whole
    const v4f lo = *(gv4f*)(x + 8 * i), hi = *(gv4f*)(x + 8 * i + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    a8_quad(v, i >> 2, nq, dst);
  }
}
