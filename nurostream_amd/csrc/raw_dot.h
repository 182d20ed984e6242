// Row dot products over raw GGUF rows, shared by the fused GEMV seam and the
// raw-layout MoE kernels. One wave computes one row for NT tokens: lanes take
// 32-element units (a whole block for MXFP4/Q4_0/Q8_0, one sub-block for
// Q4_K, an eighth of a block for Q6_K), fetch them with range-checked dword buffer loads from the aligned
// address below and realign in registers, then the wave reduces.
//
// Activations come from LDS as fp32, token stride K, together with per-32
// element sums (xsum, token stride K/32) for the formats whose codes carry an
// offset (Q4_0: q-8; Q4_K: -dmin*m).
#pragma once

#include "nsx_common.h"

// Partial dot of one 32-element unit `u` of the row starting at byte `o_row`
// (relative to the buffer resource base) with NT activation rows.
template <int FMT, int NT>
__device__ __forceinline__ void raw_unit_dot(__amdgpu_buffer_rsrc_t rs, uint32_t o_row, int u,
                                             const float* __restrict__ xs, int K,
                                             const float* __restrict__ xsum, float (&acc)[NT]) {
  const int nsb = K >> 5;
  if constexpr (FMT == NSX_MXFP4 || FMT == NSX_Q4_0) {
    constexpr uint32_t BB = FMT == NSX_MXFP4 ? 17 : 18;
    const uint32_t o = o_row + (uint32_t)u * BB;
    const uint32_t s = o & 3u, oa = o & ~3u;
    uint32_t D[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) D[i] = nsx_bload32(rs, oa + 4u * i);
    uint32_t E[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) E[i] = nsx_alignbyte(D[i + 1], D[i], s);
    const float* xb0 = xs + u * 32;
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
          const v4f xa = *(const v4f*)(xb0 + t * K + 4 * i);
          const v4f xh = *(const v4f*)(xb0 + t * K + 16 + 4 * i);
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
        const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
        const float l0 = nsx_ub<0>(lo), l1 = nsx_ub<1>(lo);
        const float l2 = nsx_ub<2>(lo), l3 = nsx_ub<3>(lo);
        const float h0 = nsx_ub<0>(hi), h1 = nsx_ub<1>(hi);
        const float h2 = nsx_ub<2>(hi), h3 = nsx_ub<3>(hi);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = *(const v4f*)(xb0 + t * K + 4 * i);
          const v4f xh = *(const v4f*)(xb0 + t * K + 16 + 4 * i);
          float p = part[t];
          p = fmaf(l0, xa.x, p); p = fmaf(l1, xa.y, p); p = fmaf(l2, xa.z, p); p = fmaf(l3, xa.w, p);
          p = fmaf(h0, xh.x, p); p = fmaf(h1, xh.y, p); p = fmaf(h2, xh.z, p); p = fmaf(h3, xh.w, p);
          part[t] = p;
        }
      }
      // d * sum((q - 8) x) = d * (sum(q x) - 8 sum(x))
      const float d = nsx_h2f(E[0] & 0xffffu);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = fmaf(d, fmaf(-8.f, xsum[t * nsb + u], part[t]), acc[t]);
    }
  } else if constexpr (FMT == NSX_Q8_0) {
    const uint32_t o = o_row + (uint32_t)u * 34u;
    const uint32_t s = o & 3u, oa = o & ~3u;
    uint32_t D[10];
#pragma unroll
    for (int i = 0; i < 10; ++i) D[i] = nsx_bload32(rs, oa + 4u * i);
    uint32_t E[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) E[i] = nsx_alignbyte(D[i + 1], D[i], s);
    const float d = nsx_h2f(E[0] & 0xffffu);
    const float* xb0 = xs + u * 32;
    float part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = nsx_alignbyte(E[i + 1], E[i], 2);
      const float q0 = (float)(int8_t)(w & 0xffu), q1 = (float)(int8_t)((w >> 8) & 0xffu);
      const float q2 = (float)(int8_t)((w >> 16) & 0xffu), q3 = (float)(int8_t)(w >> 24);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const v4f xa = *(const v4f*)(xb0 + t * K + 4 * i);
        float p = part[t];
        p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
        part[t] = p;
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = fmaf(d, part[t], acc[t]);
  } else if constexpr (FMT == NSX_Q6_K) {
    // Unit u = block b (u / 8), part j (u % 8): half h = j / 4 of the block,
    // positions l0 .. l0 + 7 (l0 = 8 (j % 4)) of its four 32-element lanes
    // L = 0..3, i.e. elements 128 h + 32 L + l0 + i. The part's 8 bytes of
    // ql[64 h + l0 ..] (lanes 0, 2), ql[64 h + 32 + l0 ..] (lanes 1, 3) and
    // qh[32 h + l0 ..] are each read once; its four int8 scales are
    // sc[8 h + l0 / 16 + 2 L]. Every field offset is a multiple of 4 from the
    // block start, so one byte shift realigns them all (any row alignment).
    const int b = u >> 3, j = u & 7, h = j >> 2, l0 = (j & 3) * 8;
    const uint32_t o = o_row + (uint32_t)b * 210u;
    const uint32_t sft = o & 3u, oa = o & ~3u;
    auto ld8 = [&](uint32_t off, uint32_t& w0, uint32_t& w1) {
      const uint32_t D0 = nsx_bload32(rs, oa + off), D1 = nsx_bload32(rs, oa + off + 4),
                     D2 = nsx_bload32(rs, oa + off + 8);
      w0 = nsx_alignbyte(D1, D0, sft);
      w1 = nsx_alignbyte(D2, D1, sft);
    };
    uint32_t A[2], B[2], C[2], S[2], dw, dw1;
    ld8(64u * h + l0, A[0], A[1]);
    ld8(64u * h + 32u + l0, B[0], B[1]);
    ld8(128u + 32u * h + l0, C[0], C[1]);
    ld8(192u + 8u * h, S[0], S[1]);
    dw = nsx_bload32(rs, oa + 208u);
    dw1 = nsx_bload32(rs, oa + 212u);
    const float d = nsx_h2f(nsx_alignbyte(dw1, dw, sft) & 0xffffu);
    const int is = l0 >> 4;
    float dsc[4];
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      const int k = is + 2 * L;  // scale byte within the half's 8
      dsc[L] = d * (float)(int8_t)((S[k >> 2] >> (8 * (k & 3))) & 0xffu);  // exact
    }
    const float* xb0 = xs + b * 256 + h * 128 + l0;
    float part[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int L = 0; L < 4; ++L) part[t][L] = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // 4 positions per dword
      const uint32_t qa = A[i], qb = B[i], qc = C[i];
      const uint32_t q[4] = {(qa & 0x0f0f0f0fu) | ((qc << 4) & 0x30303030u),
                             (qb & 0x0f0f0f0fu) | ((qc << 2) & 0x30303030u),
                             ((qa >> 4) & 0x0f0f0f0fu) | (qc & 0x30303030u),
                             ((qb >> 4) & 0x0f0f0f0fu) | ((qc >> 2) & 0x30303030u)};
#pragma unroll
      for (int L = 0; L < 4; ++L) {
        const float q0 = nsx_ub<0>(q[L]) - 32.f, q1 = nsx_ub<1>(q[L]) - 32.f;  // exact
        const float q2 = nsx_ub<2>(q[L]) - 32.f, q3 = nsx_ub<3>(q[L]) - 32.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const v4f xa = *(const v4f*)(xb0 + t * K + 32 * L + 4 * i);
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
      for (int L = 0; L < 4; ++L) a = fmaf(dsc[L], part[t][L], a);
      acc[t] = a;
    }
  } else {  // Q4_K sub-block unit: block b = u/8, sub-block s = u%8 (rows 4-byte aligned)
    const int b = u >> 3, s = u & 7;
    const uint32_t o = o_row + (uint32_t)b * 144u;
    const uint32_t H0 = nsx_bload32(rs, o), H1 = nsx_bload32(rs, o + 4), H2 = nsx_bload32(rs, o + 8),
                   H3 = nsx_bload32(rs, o + 12);
    // get_scale_min_k4 on the 12 scale bytes H1..H3
    const uint32_t sb[3] = {H1, H2, H3};
    auto byte = [&](int i) -> uint32_t { return (sb[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    uint32_t sc, m;
    if (s < 4) {
      sc = byte(s) & 63u;
      m = byte(s + 4) & 63u;
    } else {
      sc = (byte(s + 4) & 0x0fu) | ((byte(s - 4) >> 6) << 4);
      m = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
    const float d = nsx_h2f(H0 & 0xffffu), dmin = nsx_h2f(H0 >> 16);
    const uint32_t qo = o + 16u + 32u * (uint32_t)(s >> 1);
    const uint32_t sh = 4u * (uint32_t)(s & 1);
    const float* xb0 = xs + b * 256 + s * 32;
    float part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = (nsx_bload32(rs, qo + 4u * i) >> sh) & 0x0f0f0f0fu;
      const float q0 = nsx_ub<0>(q), q1 = nsx_ub<1>(q);
      const float q2 = nsx_ub<2>(q), q3 = nsx_ub<3>(q);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const v4f xa = *(const v4f*)(xb0 + t * K + 4 * i);
        float p = part[t];
        p = fmaf(q0, xa.x, p); p = fmaf(q1, xa.y, p); p = fmaf(q2, xa.z, p); p = fmaf(q3, xa.w, p);
        part[t] = p;
      }
    }
    const float dsc = d * (float)sc;   // exact
    const float dmm = dmin * (float)m; // exact
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += fmaf(dsc, part[t], -dmm * xsum[t * nsb + u]);
  }
}

// Stage NT activation rows (token stride `xstride` elements, dtype `xdt`) into
// LDS as fp32 [NT][K] followed by per-32 sums [NT][K/32]. Rows >= T are zero.
// Must be called by the whole workgroup; ends with a barrier.
template <int NT>
__device__ __forceinline__ void stage_x(float* __restrict__ xs, const void* __restrict__ x, int xdt,
                                        int64_t xstride, int T, int K, bool sums) {
  const int n = NT * K;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int t = i / K;
    xs[i] = t < T ? nsx_load_act(x, xdt, (int64_t)t * xstride + (i - t * K)) : 0.f;
  }
  __syncthreads();
  if (sums) {
    const int nsb = K >> 5;
    float* xsum = xs + n;
    for (int i = threadIdx.x; i < NT * nsb; i += blockDim.x) {
      const float* s = xs + (i / nsb) * K + (i % nsb) * 32;
      float a = 0.f;
#pragma unroll 8
      for (int j = 0; j < 32; ++j) a += s[j];
      xsum[i] = a;
    }
    __syncthreads();
  }
}

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
