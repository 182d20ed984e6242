// Row dot products over raw GGUF rows, shared by the fused GEMV seam and the
// raw-layout MoE kernels. One wave computes one row for NT tokens: lanes take
// 32-element units (a whole block for MXFP4/Q4_0/Q8_0, one sub-block for
// Q4_K, an eighth of a block for Q6_K), fetch them with range-checked dword
// buffer loads from the aligned address below and realign in registers, then
// the wave reduces.
//
// Each format's unit is split into raw_unit_fetch (the loads only, into a
// RawUnit of registers) and raw_unit_math (realignment and arithmetic), so a
// kernel can issue the loads of several units, or of the next row, before it
// waits on any of them. raw_unit_dot is the two back to back.
//
// Activations come from LDS as fp32, token stride K, together with per-32
// element sums (xsum, token stride K/32) for the formats whose codes carry an
// offset (Q4_0: q-8; Q4_K: -dmin*m).
#pragma once

#include "nsx_common.h"

template <int FMT>
struct RawUnit;
// MXFP4 / Q4_0: the 17 / 18-byte block from its aligned dword, shift s
template <> struct RawUnit<NSX_MXFP4> { uint32_t D[6]; uint32_t s; };
template <> struct RawUnit<NSX_Q4_0> { uint32_t D[6]; uint32_t s; };
// Q8_0: the 34-byte block
template <> struct RawUnit<NSX_Q8_0> { uint32_t D[10]; uint32_t s; };
// Q4_K: the block's 16-byte header and the sub-block's 32 code bytes (aligned)
template <> struct RawUnit<NSX_Q4_K> { uint32_t H[4]; uint32_t Q[8]; };
// Q6_K: 12 bytes around each of ql (lanes 0, 2), ql (lanes 1, 3), qh and the
// half's 8 scales, then the 8 bytes around d
template <> struct RawUnit<NSX_Q6_K> { uint32_t D[14]; uint32_t s; };

// Byte sources for raw_unit_fetch: 4-byte aligned dword reads at a byte
// offset, from a buffer resource (range-checked: past the range reads zero)
// or from an LDS copy of the bytes that keeps their offsets modulo 4.
struct RawBufSrc {
  __amdgpu_buffer_rsrc_t rs;
  __device__ __forceinline__ uint32_t operator()(uint32_t off) const { return nsx_bload32(rs, off); }
};
struct RawLdsSrc {
  const uint8_t* base;
  __device__ __forceinline__ uint32_t operator()(uint32_t off) const { return *(const uint32_t*)(base + off); }
};

// Loads of unit `u` of the row starting at byte `o_row` of `ld`.
template <int FMT, class Src>
__device__ __forceinline__ RawUnit<FMT> raw_unit_fetch(const Src& ld, uint32_t o_row, int u) {
  RawUnit<FMT> r;
  if constexpr (FMT == NSX_MXFP4 || FMT == NSX_Q4_0) {
    constexpr uint32_t BB = FMT == NSX_MXFP4 ? 17 : 18;
    const uint32_t o = o_row + (uint32_t)u * BB;
    r.s = o & 3u;
    const uint32_t oa = o & ~3u;
#pragma unroll
    for (int i = 0; i < 6; ++i) r.D[i] = ld(oa + 4u * i);
  } else if constexpr (FMT == NSX_Q8_0) {
    const uint32_t o = o_row + (uint32_t)u * 34u;
    r.s = o & 3u;
    const uint32_t oa = o & ~3u;
#pragma unroll
    for (int i = 0; i < 10; ++i) r.D[i] = ld(oa + 4u * i);
  } else if constexpr (FMT == NSX_Q6_K) {
    // Unit u = block b (u / 8), part j (u % 8): half h = j / 4 of the block,
    // positions l0 .. l0 + 7 (l0 = 8 (j % 4)) of its four 32-element lanes.
    // Every field offset below is a multiple of 4 from the block start, so
    // one byte shift realigns them all (any row alignment).
    const int b = u >> 3, j = u & 7, h = j >> 2, l0 = (j & 3) * 8;
    const uint32_t o = o_row + (uint32_t)b * 210u;
    r.s = o & 3u;
    const uint32_t oa = o & ~3u;
    const uint32_t off[4] = {64u * h + l0, 64u * h + 32u + l0, 128u + 32u * h + l0, 192u + 8u * h};
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 3; ++i) r.D[3 * f + i] = ld(oa + off[f] + 4u * i);
    r.D[12] = ld(oa + 208u);
    r.D[13] = ld(oa + 212u);
  } else {  // Q4_K (rows 4-byte aligned)
    const int b = u >> 3, s = u & 7;
    const uint32_t o = o_row + (uint32_t)b * 144u;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.H[i] = ld(o + 4u * i);
    const uint32_t qo = o + 16u + 32u * (uint32_t)(s >> 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) r.Q[i] = ld(qo + 4u * i);
  }
  return r;
}

// acc[t] += dot(unit u, x[t]) for the fetched unit. The unit's activations
// come through `xa4(t, k4)`: elements 4 k4 .. 4 k4 + 3 of the unit, in unit
// order (raw_unit_elem), of token t; `xsum(t)` is the sum of the unit's 32
// activations of token t (used by Q4_0 and Q4_K only). An accessor with
// kRegSums (one token, held in registers) also gives the unit's sum and its
// four 8-element group sums, so Q8_0 and Q6_K convert unsigned codes
// (q + 128, q) and take the offset off per unit / group instead of per
// element.
template <int FMT, int NT, class XA, class XS>
__device__ __forceinline__ void raw_unit_math(const RawUnit<FMT>& r, int u, const XA& xa4, const XS& xsum,
                                              float (&acc)[NT]) {
  if constexpr (FMT == NSX_MXFP4 || FMT == NSX_Q4_0) {
    uint32_t E[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) E[i] = nsx_alignbyte(r.D[i + 1], r.D[i], r.s);
    float part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = 0.f;
    if constexpr (FMT == NSX_MXFP4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = nsx_alignbyte(E[i + 1], E[i], 1);
        const v2f c0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
        const v2f c1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
        const v2f c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
        const v2f c3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = xa4(t, i);
          const v4f xh = xa4(t, 4 + i);
          float p = part[t];
          p = fmaf(c0.x, xa.x, p); p = fmaf(c0.y, xh.x, p);
          p = fmaf(c1.x, xa.y, p); p = fmaf(c1.y, xh.y, p);
          p = fmaf(c2.x, xa.z, p); p = fmaf(c2.y, xh.z, p);
          p = fmaf(c3.x, xa.w, p); p = fmaf(c3.y, xh.w, p);
          part[t] = p;
        }
      }
      // ggml value = 2^(e-128) * (2*e2m1) = 2^(e-127) * e2m1
      const int e = (int)(E[0] & 0xffu);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += __builtin_amdgcn_ldexpf(part[t], e - 127);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = nsx_alignbyte(E[i + 1], E[i], 2);
        uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
        // keep the masked dwords: the compiler would otherwise extract every
        // nibble with its own bit-field op ahead of the byte conversion
        asm volatile("" : "+v"(lo), "+v"(hi));
        const float l0 = nsx_ub<0>(lo), l1 = nsx_ub<1>(lo);
        const float l2 = nsx_ub<2>(lo), l3 = nsx_ub<3>(lo);
        const float h0 = nsx_ub<0>(hi), h1 = nsx_ub<1>(hi);
        const float h2 = nsx_ub<2>(hi), h3 = nsx_ub<3>(hi);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = xa4(t, i);
          const v4f xh = xa4(t, 4 + i);
          float p = part[t];
          p = fmaf(l0, xa.x, p); p = fmaf(l1, xa.y, p); p = fmaf(l2, xa.z, p); p = fmaf(l3, xa.w, p);
          p = fmaf(h0, xh.x, p); p = fmaf(h1, xh.y, p); p = fmaf(h2, xh.z, p); p = fmaf(h3, xh.w, p);
          part[t] = p;
        }
      }
      // d * sum((q - 8) x) = d * (sum(q x) - 8 sum(x))
      const float d = nsx_h2f(E[0] & 0xffffu);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = fmaf(d, fmaf(-8.f, xsum(t), part[t]), acc[t]);
    }
  } else if constexpr (FMT == NSX_Q8_0) {
    uint32_t E[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) E[i] = nsx_alignbyte(r.D[i + 1], r.D[i], r.s);
    const float d = nsx_h2f(E[0] & 0xffffu);
    float part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = nsx_alignbyte(E[i + 1], E[i], 2);
      if constexpr (XA::kRegSums) {
        // q + 128 as unsigned bytes (one conversion each); the 128 comes off
        // through the unit's activation sum below
        const uint32_t wu = w ^ 0x80808080u;
        const float q0 = nsx_ub<0>(wu), q1 = nsx_ub<1>(wu), q2 = nsx_ub<2>(wu), q3 = nsx_ub<3>(wu);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = xa4(t, i);
          float p = part[t];
          p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
          part[t] = p;
        }
      } else {
        const float q0 = (float)(int8_t)(w & 0xffu), q1 = (float)(int8_t)((w >> 8) & 0xffu);
        const float q2 = (float)(int8_t)((w >> 16) & 0xffu), q3 = (float)(int8_t)(w >> 24);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = xa4(t, i);
          float p = part[t];
          p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
          part[t] = p;
        }
      }
    }
    if constexpr (XA::kRegSums) {
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = fmaf(d, fmaf(-128.f, xa4.sum(), part[t]), acc[t]);
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = fmaf(d, part[t], acc[t]);
    }
  } else if constexpr (FMT == NSX_Q6_K) {
    // Element 128 h + 32 L + l0 + i takes its low 4 bits from ql[64 h + 32 (L & 1)
    // + l0 + i] (nibble L >> 1), its high 2 bits from qh[32 h + l0 + i] >> 2L,
    // and its int8 scale from sc[8 h + l0 / 16 + 2 L].
    const int l0 = (u & 3) * 8;
    uint32_t F[4][2];  // ql (lanes 0, 2), ql (lanes 1, 3), qh, scales
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      F[f][0] = nsx_alignbyte(r.D[3 * f + 1], r.D[3 * f], r.s);
      F[f][1] = nsx_alignbyte(r.D[3 * f + 2], r.D[3 * f + 1], r.s);
    }
    const float d = nsx_h2f(nsx_alignbyte(r.D[13], r.D[12], r.s) & 0xffffu);
    const int is = l0 >> 4;
    float dsc[4];
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      const int k = is + 2 * L;  // scale byte within the half's 8
      dsc[L] = d * (float)(int8_t)((F[3][k >> 2] >> (8 * (k & 3))) & 0xffu);  // exact
    }
    float part[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int L = 0; L < 4; ++L) part[t][L] = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // 4 positions per dword
      const uint32_t qa = F[0][i], qb = F[1][i], qc = F[2][i];
      const uint32_t q[4] = {(qa & 0x0f0f0f0fu) | ((qc << 4) & 0x30303030u),
                             (qb & 0x0f0f0f0fu) | ((qc << 2) & 0x30303030u),
                             ((qa >> 4) & 0x0f0f0f0fu) | (qc & 0x30303030u),
                             ((qb >> 4) & 0x0f0f0f0fu) | ((qc >> 2) & 0x30303030u)};
#pragma unroll
      for (int L = 0; L < 4; ++L) {
        // with register sums the 32 comes off per 8-element group below
        constexpr float off = XA::kRegSums ? 0.f : 32.f;
        const float q0 = nsx_ub<0>(q[L]) - off, q1 = nsx_ub<1>(q[L]) - off;  // exact
        const float q2 = nsx_ub<2>(q[L]) - off, q3 = nsx_ub<3>(q[L]) - off;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = xa4(t, 2 * L + i);  // elements 32 L + 4 i .. of the part
          float p = part[t][L];
          p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
          part[t][L] = p;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a = acc[t];
#pragma unroll
      for (int L = 0; L < 4; ++L) {
        if constexpr (XA::kRegSums) a = fmaf(dsc[L], fmaf(-32.f, xa4.gsum(L), part[t][L]), a);
        else a = fmaf(dsc[L], part[t][L], a);
      }
      acc[t] = a;
    }
  } else {  // Q4_K sub-block unit: block b = u/8, sub-block s = u%8
    const int s = u & 7;
    // get_scale_min_k4 on the 12 scale bytes H1..H3
    const uint32_t sb[3] = {r.H[1], r.H[2], r.H[3]};
    auto byte = [&](int i) -> uint32_t { return (sb[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    uint32_t sc, m;
    if (s < 4) {
      sc = byte(s) & 63u;
      m = byte(s + 4) & 63u;
    } else {
      sc = (byte(s + 4) & 0x0fu) | ((byte(s - 4) >> 6) << 4);
      m = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
    const float d = nsx_h2f(r.H[0] & 0xffffu), dmin = nsx_h2f(r.H[0] >> 16);
    const uint32_t sh = 4u * (uint32_t)(s & 1);
    float part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q = (r.Q[i] >> sh) & 0x0f0f0f0fu;
      asm volatile("" : "+v"(q));  // one mask per dword, not one bit-field op per nibble
      const float q0 = nsx_ub<0>(q), q1 = nsx_ub<1>(q);
      const float q2 = nsx_ub<2>(q), q3 = nsx_ub<3>(q);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const v4f xa = xa4(t, i);
        float p = part[t];
        p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
        part[t] = p;
      }
    }
    const float dsc = d * (float)sc;   // exact
    const float dmm = dmin * (float)m; // exact
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += fmaf(dsc, part[t], -dmm * xsum(t));
  }
}

// Row element of element k (0..31, unit order) of unit u. Units are 32
// consecutive elements except Q6_K's parts: four runs of 8, one in each of
// the half's 32-element lanes (elements 128 h + 32 L + l0 .. + 7).
template <int FMT>
__device__ __forceinline__ int raw_unit_elem(int u, int k) {
  if constexpr (FMT == NSX_Q6_K) {
    return (u >> 3) * 256 + ((u >> 2) & 1) * 128 + (u & 3) * 8 + 32 * (k >> 3) + (k & 7);
  } else {
    return u * 32 + k;
  }
}

// Activations of unit u from LDS rows (token stride K) and per-32 sums
// (token stride K/32; Q6_K units are not 32 consecutive elements and take no
// sums).
template <int FMT>
struct RawXLds {
  static constexpr bool kRegSums = false;  // no per-unit / per-8 sums on hand
  const float* xs;
  int K, u;
  __device__ __forceinline__ v4f operator()(int t, int k4) const {
    return *(const v4f*)(xs + t * K + raw_unit_elem<FMT>(u, 4 * k4));
  }
};
struct RawXSumLds {
  const float* xsum;
  int nsb, u;
  __device__ __forceinline__ float operator()(int t) const { return xsum[t * nsb + u]; }
};

// Partial dot of one 32-element unit `u` of the row starting at byte `o_row`
// (relative to the buffer resource base) with NT activation rows.
template <int FMT, int NT>
__device__ __forceinline__ void raw_unit_dot(__amdgpu_buffer_rsrc_t rs, uint32_t o_row, int u,
                                             const float* __restrict__ xs, int K,
                                             const float* __restrict__ xsum, float (&acc)[NT]) {
  const RawUnit<FMT> r = raw_unit_fetch<FMT>(RawBufSrc{rs}, o_row, u);
  raw_unit_math<FMT, NT>(r, u, RawXLds<FMT>{xs, K, u}, RawXSumLds{xsum, K >> 5, u}, acc);
}

// Four consecutive activations from element offset `i` (a multiple of 4) as
// fp32; `vec` says the address is aligned for one vector load.
__device__ __forceinline__ v4f nsx_load_act4(const void* __restrict__ p, int dtype, int64_t i, bool vec) {
  if (vec) {
    if (dtype == NSX_DT_F32) return *(const v4f*)((const float*)p + i);
    const v2u w = *(const v2u*)((const uint16_t*)p + i);
    if (dtype == NSX_DT_F16)
      return v4f{nsx_h2f(w.x & 0xffffu), nsx_h2f(w.x >> 16), nsx_h2f(w.y & 0xffffu), nsx_h2f(w.y >> 16)};
    return v4f{nsx_bf2f(w.x & 0xffffu), nsx_bf2f(w.x >> 16), nsx_bf2f(w.y & 0xffffu), nsx_bf2f(w.y >> 16)};
  }
  return v4f{nsx_load_act(p, dtype, i), nsx_load_act(p, dtype, i + 1), nsx_load_act(p, dtype, i + 2),
             nsx_load_act(p, dtype, i + 3)};
}

// G independent nsx_load_act4 loads at element offsets idx[g], with the
// dtype / alignment branch taken once outside them: inside one branch the
// loads have no control flow between them, so they are all in flight
// together (a branch per load makes each one wait for the last).
template <int G>
__device__ __forceinline__ void nsx_load_act4_n(const void* __restrict__ p, int dtype, const int64_t (&idx)[G],
                                                bool vec, v4f (&out)[G]) {
  if (vec && dtype == NSX_DT_F32) {
#pragma unroll
    for (int g = 0; g < G; ++g) out[g] = *(const v4f*)((const float*)p + idx[g]);
  } else if (vec) {
    v2u w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) w[g] = *(const v2u*)((const uint16_t*)p + idx[g]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (dtype == NSX_DT_F16)
        out[g] = v4f{nsx_h2f(w[g].x & 0xffffu), nsx_h2f(w[g].x >> 16), nsx_h2f(w[g].y & 0xffffu),
                     nsx_h2f(w[g].y >> 16)};
      else
        out[g] = v4f{nsx_bf2f(w[g].x & 0xffffu), nsx_bf2f(w[g].x >> 16), nsx_bf2f(w[g].y & 0xffffu),
                     nsx_bf2f(w[g].y >> 16)};
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) out[g] = nsx_load_act4(p, dtype, idx[g], false);
  }
}

// Stage NT activation rows (token stride `xstride` elements, dtype `xdt`) into
// LDS as fp32 [NT][K] followed by per-32 sums [NT][K/32]. Rows >= T are zero.
// K is a multiple of 32. Each thread issues its loads in groups of four
// before writing any of them. Must be called by the whole workgroup; ends
// with a barrier.
template <int NT>
__device__ __forceinline__ void stage_x(float* __restrict__ xs, const void* __restrict__ x, int xdt,
                                        int64_t xstride, int T, int K, bool sums) {
  const int kq = K >> 2;  // quads per token
  const int nq = NT * kq;
  const uint32_t align = xdt == NSX_DT_F32 ? 15u : 7u;
  const bool vec = ((uintptr_t)x & align) == 0 && (xstride & 3) == 0;
  constexpr int G = 4;
  for (int q0 = threadIdx.x; q0 < nq; q0 += G * blockDim.x) {
    v4f v[G];
    int64_t idx[G];
    bool live[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {  // addresses clamped to a valid element, values masked after the loads
      const int q = q0 + g * blockDim.x;
      const int t = q / kq;
      live[g] = q < nq && t < T;
      const int qc = live[g] ? q : 0;
      const int tc = qc / kq;
      idx[g] = (int64_t)tc * xstride + 4 * (qc - tc * kq);
    }
    nsx_load_act4_n<G>(x, xdt, idx, vec, v);
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (!live[g]) v[g] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int q = q0 + g * blockDim.x;
      if (q < nq) *(v4f*)(xs + 4 * q) = v[g];
    }
  }
  __syncthreads();
  if (sums) {
    const int nsb = K >> 5;
    float* xsum = xs + NT * K;
    for (int i = threadIdx.x; i < NT * nsb; i += blockDim.x) {
      const v4f* s = (const v4f*)(xs + (i / nsb) * K + (i % nsb) * 32);
      v4f w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = s[j];
      float a = 0.f;  // sequential order over the 32 elements
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a += w[j].x; a += w[j].y; a += w[j].z; a += w[j].w;
      }
      xsum[i] = a;
    }
    __syncthreads();
  }
}

// Block geometry: elements and bytes per ggml block.
template <int FMT>
struct RawBlock {
  static constexpr int BE = (FMT == NSX_Q4_K || FMT == NSX_Q6_K) ? 256 : 32;
  static constexpr int BB = FMT == NSX_MXFP4 ? 17 : FMT == NSX_Q4_0 ? 18 : FMT == NSX_Q8_0 ? 34
                          : FMT == NSX_Q4_K ? 144 : 210;
};

template <int FMT>
__device__ __host__ constexpr int raw_units(int K) {
  return K / 32;  // 32-element units; Q4_K sub-blocks and Q6_K parts are 32 elements too
}

template <int FMT>
__device__ __host__ constexpr uint32_t raw_row_bytes(int K) {
  return FMT == NSX_MXFP4 ? (uint32_t)(K / 32) * 17u
       : FMT == NSX_Q4_0  ? (uint32_t)(K / 32) * 18u
       : FMT == NSX_Q8_0  ? (uint32_t)(K / 32) * 34u
       : FMT == NSX_Q6_K  ? (uint32_t)(K / 256) * 210u
                          : (uint32_t)(K / 256) * 144u;
}
