// MoE expert path for gfx950: router logits, top-k, routed expert products
// (MFMA over t64 tiles, or VALU over raw GGUF rows), activation and the
// weighted combine -- with expert ids never leaving the device.
//
// Reference semantics (neurostream/): model/gpt_oss.py:61-70,116-177 and
// moe/router.py:59-69,173-219. The row-window products of
// compute/blockffn.py:396-449 (stream_expert_ffn) are computed per expert
// window; a row's dot product does not depend on the block decomposition.
//
// No kernel here synchronises across workgroups: every global dependency is
// a kernel boundary (agent-scope fences cost an L2 write-back/invalidate per
// wave on gfx950), and reductions stay inside one workgroup's LDS.
#include "nsx_common.h"
#include "raw_dot.h"

#include <algorithm>
#include <stdlib.h>

static inline hipStream_t S(void* s) { return (hipStream_t)s; }

constexpr int MAX_TOPK = 16;
constexpr int MAX_EXPERTS = 256;

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// activation fragments ("xfrag")
//
// The MFMA kernels compute y = W x with W's MXFP4 blocks converted exactly to
// bf16 (pre-scaled by their e8m0 scale) and x split into three bf16 terms
// hi + mid + lo (|x - hi - mid - lo| <= 2^-24 |x|) that occupy B columns 0..2
// of v_mfma_f32_16x16x32_bf16. A lane (col c = l%16, group q = l/16) supplies
// 8 K-slots: for K-step s (blocks 4s..4s+3) and sub-step j, slot 2u / 2u+1
// hold elements 4j+u / 16+4j+u of block 4s+q -- exactly the order in which
// v_cvt_scalef32_pk_bf16_fp4 expands byte u of qs dword j.
// Storage per token (or per expert pair): [s][j][q][c:3][u:4] dwords, each
// dword = (bf16 of element 4j+u) | (bf16 of element 16+4j+u) << 16.
constexpr int XF_SPLIT = 3;
constexpr int XF_STEP_BYTES = 4 * 4 * XF_SPLIT * 16;  // 768 B per 4-block step

__device__ __forceinline__ void split3(float v, uint32_t (&o)[3]) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const uint32_t hi = b & 0xffff0000u;
  const float r1 = v - __builtin_bit_cast(float, hi);  // exact
  const uint32_t mid = __builtin_bit_cast(uint32_t, r1) & 0xffff0000u;
  const float r2 = r1 - __builtin_bit_cast(float, mid);  // exact
  o[0] = hi >> 16;
  o[1] = mid >> 16;
  o[2] = nsx_f2bf(r2);
}

// byte offset of (element n, split c) inside one activation's xfrag
__device__ __forceinline__ uint32_t xfrag_offset(int n, int c) {
  const int b = n >> 5, ee = n & 31;
  const int s = b >> 2, q = b & 3;
  const int half = ee >> 4, e2 = ee & 15;
  const int j = e2 >> 2, u = e2 & 3;
  return ((((uint32_t)(s * 4 + j) * 4 + q) * XF_SPLIT + c) * 4 + u) * 4 + half * 2;
}

// Fill xfrag entries for T activation rows of length K (grid-stride over all
// dwords, zero for blocks past K). Called from the router kernel.
__device__ __forceinline__ void build_xfrag(const float* __restrict__ x, int T, int K, uint8_t* __restrict__ xf,
                                            int64_t gtid, int64_t gstride) {
  const int nb = K / 32, nb4 = (nb + 3) / 4;
  const int64_t per_tok = (int64_t)nb4 * (XF_STEP_BYTES / 4);
  for (int64_t d = gtid; d < per_tok * T; d += gstride) {
    const int t = (int)(d / per_tok);
    int rem = (int)(d - (int64_t)t * per_tok);
    const int u = rem & 3;
    rem >>= 2;
    const int c = rem % XF_SPLIT;
    rem /= XF_SPLIT;
    const int q = rem & 3;
    rem >>= 2;
    const int j = rem & 3;
    const int s = rem >> 2;
    const int b = 4 * s + q;
    uint32_t lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
    if (b < nb) {
      const float* xb = x + (int64_t)t * K + b * 32;
      split3(xb[4 * j + u], lo);
      split3(xb[16 + 4 * j + u], hi);
    }
    ((uint32_t*)xf)[d] = lo[c] | (hi[c] << 16);
  }
}

// ---------------------------------------------------------------------------
// router logits: one wave per expert row, TT tokens per workgroup row

constexpr int RT_TT = 8;

__device__ __forceinline__ void load8_w(const void* W, int wdt, int64_t off, float (&w)[8]) {
  if (wdt == NSX_F32) {
    const v4f a = *(const v4f*)((const float*)W + off);
    const v4f b = *(const v4f*)((const float*)W + off + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    const v4u q = *(const v4u*)((const uint16_t*)W + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = q[i] & 0xffffu, hi = q[i] >> 16;
      w[2 * i] = wdt == NSX_BF16 ? nsx_bf2f(lo) : nsx_h2f(lo);
      w[2 * i + 1] = wdt == NSX_BF16 ? nsx_bf2f(hi) : nsx_h2f(hi);
    }
  }
}

constexpr int RT_MAXC = 8;  // 512-element chunks per lane and pass (K <= 4096 in one pass)

__global__ __launch_bounds__(256) void router_logits_kernel(const float* __restrict__ h, int T, int K,
                                                            const void* __restrict__ W, int wdt,
                                                            const float* __restrict__ bias, int E,
                                                            float* __restrict__ logits, uint8_t* __restrict__ xfrag) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  if (xfrag) {
    const int64_t nthreads = (int64_t)gridDim.x * gridDim.y * blockDim.x;
    const int64_t tid = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
    build_xfrag(h, T, K, xfrag, tid, nthreads);
  }
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * RT_TT;
  const int nt = min(RT_TT, T - t0);
  if (e >= E) return;
  float acc[RT_TT];
#pragma unroll
  for (int i = 0; i < RT_TT; ++i) acc[i] = 0.f;
  for (int k0 = 0; k0 < K; k0 += RT_MAXC * 512) {
    // every weight and activation load of the pass is issued before the arithmetic
    float w[RT_MAXC][8];
#pragma unroll
    for (int c = 0; c < RT_MAXC; ++c) {
      const int k = k0 + c * 512 + lane * 8;
      if (k < K) {
        load8_w(W, wdt, (int64_t)e * K + k, w[c]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) w[c][u] = 0.f;
      }
    }
    for (int i = 0; i < nt; ++i) {
      const float* hp = h + (int64_t)(t0 + i) * K;
      v4f ha[RT_MAXC], hb[RT_MAXC];
#pragma unroll
      for (int c = 0; c < RT_MAXC; ++c) {
        const int k = k0 + c * 512 + lane * 8;
        if (k < K) {
          ha[c] = *(const v4f*)(hp + k);
          hb[c] = *(const v4f*)(hp + k + 4);
        } else {
          ha[c] = hb[c] = v4f{0.f, 0.f, 0.f, 0.f};
        }
      }
      float s = acc[i];
#pragma unroll
      for (int c = 0; c < RT_MAXC; ++c) {
        s = fmaf(w[c][0], ha[c].x, s); s = fmaf(w[c][1], ha[c].y, s);
        s = fmaf(w[c][2], ha[c].z, s); s = fmaf(w[c][3], ha[c].w, s);
        s = fmaf(w[c][4], hb[c].x, s); s = fmaf(w[c][5], hb[c].y, s);
        s = fmaf(w[c][6], hb[c].z, s); s = fmaf(w[c][7], hb[c].w, s);
      }
      acc[i] = s;
    }
  }
#pragma unroll
  for (int i = 0; i < RT_TT; ++i) {
    const float s = nsx_wave_sum(acc[i]);
    if (lane == 0 && i < nt) logits[(int64_t)(t0 + i) * E + e] = bias ? s + bias[e] : s;
  }
}

// ---------------------------------------------------------------------------
// top-k over one token's logits, computed by one wave; results are uniform
// across the wave. Order: larger value first, ties to the lower index.

// float -> uint32 with the same order (NaNs aside), and back
__device__ __forceinline__ uint32_t f2key(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  return b & 0x80000000u ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  return __builtin_bit_cast(float, k & 0x80000000u ? (k ^ 0x80000000u) : ~k);
}

// Each round takes the wave maximum of the lanes' best keys, then the
// minimum index holding it (wave reductions run on DPP, not LDS permutes).
__device__ void topk_regs(const float* __restrict__ lg, int E, int k, int mode, int (&sel_i)[MAX_TOPK],
                          float (&sel_w)[MAX_TOPK]) {
  const int lane = __lane_id();
  constexpr int NV = MAX_EXPERTS / 64;
  float v[NV];
  bool ok[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    ok[i] = e < E;
    v[i] = ok[i] ? lg[e] : 0.f;
  }
  if (mode == NSX_ROUTE_QWEN3) {  // probs = softmax(logits) over all experts, float32 (router.py:65)
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (ok[i]) m = fmaxf(m, v[i]);
    m = key2f(__reduce_max_sync(~0ull, f2key(m)));
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (ok[i]) {
        v[i] = expf(v[i] - m);
        s += v[i];
      }
    s = nsx_wave_sum(s);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (ok[i]) v[i] = v[i] / s;
  }
  uint32_t key[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) key[i] = f2key(v[i]);
  float sel_v[MAX_TOPK];
#pragma unroll
  for (int j = 0; j < MAX_TOPK; ++j) {
    if (j >= k) break;
    uint32_t lk = 0, li = 0xffffu;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (ok[i] && (key[i] > lk || li == 0xffffu)) {  // i ascending: ties keep the lower index
        lk = key[i];
        li = lane + 64 * i;
      }
    const uint32_t mk = __reduce_max_sync(~0ull, li == 0xffffu ? 0u : lk);
    const uint32_t wi = __reduce_min_sync(~0ull, (li != 0xffffu && lk == mk) ? li : 0xffffu);
    sel_i[j] = wi == 0xffffu ? 0 : (int)wi;
    sel_v[j] = key2f(mk);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i == (int)wi) ok[i] = false;
  }
  if (mode == NSX_ROUTE_GPTOSS) {  // softmax over the selected logits in float32 (gpt_oss.py:120)
    float s = 0.f;
    for (int j = 0; j < k; ++j) {
      sel_w[j] = expf(sel_v[j] - sel_v[0]);
      s += sel_w[j];
    }
    for (int j = 0; j < k; ++j) sel_w[j] = sel_w[j] / s;
  } else {  // renormalise the selected probabilities (router.py:68)
    float s = 0.f;
    for (int j = 0; j < k; ++j) s += sel_v[j];
    for (int j = 0; j < k; ++j) sel_w[j] = sel_v[j] / s;
  }
}

__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int T, int E, int k, int mode,
                                                   int32_t* __restrict__ ids, float* __restrict__ wts) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  int si[MAX_TOPK];
  float sw[MAX_TOPK];
  topk_regs(logits + (int64_t)t * E, E, k, mode, si, sw);
  if (__lane_id() == 0)
    for (int j = 0; j < k; ++j) {
      ids[(int64_t)t * k + j] = si[j];
      wts[(int64_t)t * k + j] = sw[j];
    }
}

static int check_router(int64_t T, int64_t K, int wdt, int64_t E, int k, int mode) {
  NSX_REQUIRE(T >= 1 && T <= (1 << 20), NSX_EINVAL, "T=%lld", (long long)T);
  NSX_REQUIRE(K > 0 && K % 8 == 0 && K < (1 << 24), NSX_EINVAL, "router K=%lld must be a multiple of 8",
              (long long)K);
  NSX_REQUIRE(wdt == NSX_F32 || wdt == NSX_BF16 || wdt == NSX_F16, NSX_ETYPE, "router weight type %d", wdt);
  NSX_REQUIRE(E >= 1 && E <= MAX_EXPERTS, NSX_EINVAL, "n_expert=%lld outside 1..%d", (long long)E, MAX_EXPERTS);
  NSX_REQUIRE(k >= 1 && k <= MAX_TOPK && k <= E, NSX_EINVAL, "top_k=%d", k);
  NSX_REQUIRE(mode == NSX_ROUTE_GPTOSS || mode == NSX_ROUTE_QWEN3, NSX_EINVAL, "router mode %d", mode);
  return NSX_OK;
}

static int launch_logits(const float* h, int64_t T, int64_t K, const void* w, int wdt, const float* bias, int64_t E,
                         float* logits, uint8_t* xfrag, hipStream_t st) {
  const dim3 grid((unsigned)nsx_cdiv(E, 4), (unsigned)nsx_cdiv(T, RT_TT));
  return nsx_launch(router_logits_kernel, grid, dim3(256), 0, st, h, (int)T, (int)K, w, wdt, bias, (int)E, logits,
                    xfrag);
}

static int launch_topk(const float* logits, int64_t T, int64_t E, int k, int mode, int32_t* ids, float* wts,
                       hipStream_t st) {
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)nsx_cdiv(T, 4)), dim3(256), 0, st, logits, (int)T, (int)E, k, mode,
                     ids, wts);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int nsx_router_topk(const float* h, int64_t T, int64_t K, const void* w, int w_dtype, const float* bias,
                               int64_t n_expert, int top_k, int mode, int32_t* ids, float* weights, float* logits,
                               void* stream) {
  int rc = check_router(T, K, w_dtype, n_expert, top_k, mode);
  if (rc) return rc;
  NSX_REQUIRE(h && w && ids && weights && logits, NSX_EINVAL, "null buffer");
  rc = launch_logits(h, T, K, w, w_dtype, bias, n_expert, logits, nullptr, S(stream));
  if (rc) return rc;
  return launch_topk(logits, T, n_expert, top_k, mode, ids, weights, S(stream));
}

// ---------------------------------------------------------------------------
// t64 tile partial dot on the VALU (the lane owns one row of a 64-row tile);
// used by nsx_t64_gemv (stream_linear over resident t64 slabs).

template <int NT, int GMAX>
__device__ __forceinline__ void mx_t64_partial(const uint8_t* __restrict__ mat, int64_t qs_bytes, int nb, int nb4,
                                               int tile, int g0, int g1, const float* __restrict__ x,
                                               int64_t xstride, float (&acc)[NT]) {
  const int lane = __lane_id();
  typedef const __attribute__((address_space(1))) v4u gv4u;
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  gv4u* qs = (gv4u*)(mat + (int64_t)tile * nb * 1024 + lane * 16);
  gu32* sc = (gu32*)(mat + qs_bytes + (int64_t)tile * nb4 * 256) + lane;
  for (int gs = g0; gs < g1; gs += GMAX) {
    v4u q[GMAX * 4];
    uint32_t s[GMAX];
#pragma unroll
    for (int gi = 0; gi < GMAX; ++gi) {
      const int g = gs + gi;
      if (g < g1) {
        s[gi] = sc[(int64_t)g * 64];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int b = g * 4 + j;
          q[gi * 4 + j] = b < nb ? qs[(int64_t)b * 64] : v4u{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int gi = 0; gi < GMAX; ++gi) {
      const int g = gs + gi;
      if (g >= g1) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = g * 4 + j;
        if (b >= nb) break;
        const int e = (int)((s[gi] >> (8 * j)) & 0xffu);
        float p0[NT], p1[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) p0[t] = p1[t] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = q[gi * 4 + j][i];
          const v2f c0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
          const v2f c1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
          const v2f c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
          const v2f c3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            // constant address space: x is uniform and read-only here (scalar loads)
            const __attribute__((address_space(4))) float* xb =
                (const __attribute__((address_space(4))) float*)(x + t * xstride + b * 32 + 4 * i);
            p0[t] = fmaf(c0.x, xb[0], p0[t]);
            p1[t] = fmaf(c0.y, xb[16], p1[t]);
            p0[t] = fmaf(c1.x, xb[1], p0[t]);
            p1[t] = fmaf(c1.y, xb[17], p1[t]);
            p0[t] = fmaf(c2.x, xb[2], p0[t]);
            p1[t] = fmaf(c2.y, xb[18], p1[t]);
            p0[t] = fmaf(c3.x, xb[3], p0[t]);
            p1[t] = fmaf(c3.y, xb[19], p1[t]);
          }
        }
        // ggml value = 2^(e-128) * (2*e2m1) = 2^(e-127) * e2m1
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] += __builtin_amdgcn_ldexpf(p0[t] + p1[t], e - 127);
      }
    }
  }
}

constexpr int T64_GMAX = 8;

template <int NT>
__global__ __launch_bounds__(256) void t64_gemv_kernel(const uint8_t* __restrict__ mat, int64_t qs_bytes, int nb,
                                                       int nb4, int64_t row_lo, int64_t row_hi, int tile0,
                                                       const float* __restrict__ x, int64_t xstride, int T,
                                                       float* __restrict__ y, int64_t ystride) {
  __shared__ float red[4][NT][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int tile = tile0 + blockIdx.x;
  const int gper = (nb4 + 3) / 4;
  const int g0 = wave * gper, g1 = min(nb4, g0 + gper);
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  mx_t64_partial<NT, T64_GMAX>(mat, qs_bytes, nb, nb4, tile, g0, g1, x, xstride, acc);
#pragma unroll
  for (int t = 0; t < NT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  if (wave == 0) {
    const int64_t row = (int64_t)tile * 64 + lane;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float v = red[0][t][lane] + red[1][t][lane] + red[2][t][lane] + red[3][t][lane];
      if (t < T && row >= row_lo && row < row_hi) y[(int64_t)t * ystride + (row - row_lo)] = v;
    }
  }
}

template <int NT>
static int launch_t64_gemv(const void* t64, int64_t n_rows, int64_t K, int64_t lo, int64_t hi, const float* x,
                           int64_t T, float* y, hipStream_t st) {
  const int64_t nb = K / 32, nb4 = nsx_cdiv(nb, 4), tiles = nsx_cdiv(n_rows, 64);
  const int64_t qsb = tiles * nb * 1024;
  const int64_t tile0 = lo / 64, tile1 = nsx_cdiv(hi, 64);
  hipLaunchKernelGGL((t64_gemv_kernel<NT>), dim3((unsigned)(tile1 - tile0)), dim3(256), 0, st, (const uint8_t*)t64,
                     qsb, (int)nb, (int)nb4, lo, hi, (int)tile0, x, K, (int)T, y, hi - lo);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int nsx_t64_gemv(int t, const void* t64, int64_t n_rows, int64_t K, int64_t row_lo, int64_t row_hi,
                            const void* x, int x_dtype, int64_t T, float* y, void* stream) {
  NSX_REQUIRE(t == NSX_MXFP4, NSX_ENOTIMPL, "t64 GEMV is implemented for MXFP4 only (type %d)", t);
  NSX_REQUIRE(K > 0 && K % 32 == 0 && K < (1 << 24), NSX_EINVAL, "K=%lld", (long long)K);
  NSX_REQUIRE(0 <= row_lo && row_lo <= row_hi && row_hi <= n_rows, NSX_EINVAL, "row window [%lld, %lld) of %lld",
              (long long)row_lo, (long long)row_hi, (long long)n_rows);
  NSX_REQUIRE(T >= 1 && T <= 4, NSX_EINVAL, "t64 GEMV takes T in 1..4 (T=%lld)", (long long)T);
  NSX_REQUIRE(x_dtype == NSX_DT_F32, NSX_ETYPE, "t64 GEMV takes fp32 activations");
  if (row_hi == row_lo) return NSX_OK;
  NSX_REQUIRE(t64 && x && y, NSX_EINVAL, "null buffer");
  hipStream_t st = S(stream);
  const float* xf = (const float*)x;
  if (T == 1) return launch_t64_gemv<1>(t64, n_rows, K, row_lo, row_hi, xf, T, y, st);
  if (T == 2) return launch_t64_gemv<2>(t64, n_rows, K, row_lo, row_hi, xf, T, y, st);
  return launch_t64_gemv<4>(t64, n_rows, K, row_lo, row_hi, xf, T, y, st);
}

// ---------------------------------------------------------------------------
// MoE layer state shared by the kernels

struct MoeDev {
  const float* logits;
  int32_t* ids;
  float* wts;
  int T, top_k, E, mode;
  const uint64_t* gate_ptrs;
  const uint64_t* up_ptrs;
  const uint64_t* down_ptrs;
  const void* gate_base;
  const void* up_base;
  const void* down_base;
  int64_t gate_stride, up_stride, down_stride;
  const float* gate_bias;
  const float* up_bias;
  const float* down_bias;
  const float* h;
  float* out;
  float* act;             // (pairs, n_ff) fp32 activations
  float* ypair;           // (pairs, n_embd) fp32 per-expert down outputs (t64 path)
  const uint8_t* xf_h;    // xfrag of h, per token
  uint8_t* xf_a;          // xfrag of act, per pair
  int n_embd, n_ff;
  int nb_gu, nb4_gu;      // blocks / steps of K = n_embd
  int nb_d, nb4_d;        // blocks / steps of K = n_ff
  int64_t qsb_gu, qsb_d;  // t64 qs-plane bytes of one expert matrix
  int act_kind;
  float alpha, limit;
};

__device__ __forceinline__ float moe_act(int kind, float g, float u, float alpha, float limit) {
  if (kind == NSX_ACT_CLAMPED_SWIGLU) {  // gpt_oss.py:61-70
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
    const float sig = 1.f / (1.f + expf(-(g * alpha)));
    return (u + 1.f) * (g * sig);
  }
  const float sig = 1.f / (1.f + expf(-g));  // F.silu(gate) * up
  return g * sig * u;
}

__device__ __forceinline__ int clamp_expert(int e, int E) { return e < 0 ? 0 : (e >= E ? E - 1 : e); }

// ascending-expert order of a token's top-k slots (uniform across the wave)
__device__ __forceinline__ void slot_order(const int (&ids)[MAX_TOPK], int k, int (&order)[MAX_TOPK]) {
  for (int j = 0; j < k; ++j) order[j] = j;
  for (int i = 1; i < k; ++i) {
    const int oi = order[i], ei = ids[oi];
    int j = i - 1;
    while (j >= 0 && ids[order[j]] > ei) {
      order[j + 1] = order[j];
      --j;
    }
    order[j + 1] = oi;
  }
}

// out[rows] += w * y in the reference rounds the product and the sum separately
__device__ __forceinline__ float combine_one(float acc, float w, float y) { return __fadd_rn(acc, __fmul_rn(w, y)); }

// ---------------------------------------------------------------------------
// MFMA expert kernels over t64 tiles (MXFP4)

// e8m0 byte -> fp32 scale 2^(e-127) for v_cvt_scalef32_pk_bf16_fp4, exact for
// e in 0..254 (e=0 a denormal); e=255 runs with 2^127 and mx_bf16_double.
__device__ __forceinline__ float mx_scale_f32(uint32_t e) {
  return __builtin_bit_cast(float, e == 0 ? 0x00400000u : (e == 255 ? (254u << 23) : (e << 23)));
}

// ggml's e=255 scale is 2^127 on the doubled table, i.e. 2^128 * e2m1. The
// conversion ran with 2^127, so double each bf16: normal values gain one in
// the exponent (2^127-magnitudes overflow to inf, like the fp32 reference);
// zeros stay zero. (Denormals cannot occur at this scale.)
__device__ __forceinline__ uint32_t mx_bf16_double(uint32_t w2) {
  uint32_t r = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t v = (w2 >> (16 * h)) & 0xffffu;
    const uint32_t ex = v & 0x7f80u;
    if ((v & 0x7fffu) != 0 && ex != 0x7f80u) v = ex == 0x7f00u ? ((v & 0x8000u) | 0x7f80u) : v + 0x80u;
    r |= v << (16 * h);
  }
  return r;
}

__device__ __forceinline__ v8bf mx_a_operand(uint32_t w, float scale, bool dbl) {
  uint32_t p[4];
  p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
  if (__builtin_expect(dbl, 0)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = mx_bf16_double(p[i]);
  }
  v4u pv = {p[0], p[1], p[2], p[3]};
  return __builtin_bit_cast(v8bf, pv);
}

constexpr int MX_CH = 6;  // K-steps (4 blocks each) whose loads one wave holds in flight

// One wave: a whole 64-row t64 tile times an xfrag (global memory) over
// K-steps [s0, s1). Rows are four MFMA row groups g (rows 16g..16g+15) that
// share every B operand; lane (i = l%16, q = l/16) loads row 16g+i of block
// 4s+q (four 256-byte runs per instruction). Each pass issues all of its
// weight, scale and activation loads before any arithmetic.
template <int CH>
struct MxTile {
  v4u A[CH][4];
  uint32_t SC[CH][4];
  v4u B[CH][4];
};

template <int CH>
__device__ __forceinline__ void mx_tile_load(MxTile<CH>& r, const uint8_t* __restrict__ mat, int64_t qs_bytes,
                                             int nb, int nb4, int tile, int s0, int s1,
                                             const uint8_t* __restrict__ xf) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  const int lane = __lane_id();
  const int i = lane & 15, q = lane >> 4;
  const uint8_t* qs = mat + (int64_t)tile * nb * 1024 + i * 16;
  const uint8_t* sc = mat + qs_bytes + (int64_t)tile * nb4 * 256 + i * 4;
  const bool bcol = i < XF_SPLIT;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int s = s0 + u;
    if (s < s1) {
      const int b = min(4 * s + q, nb - 1);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        r.A[u][g] = *(gv4u*)(qs + (int64_t)b * 1024 + g * 256);
        r.SC[u][g] = *(gu32*)(sc + (int64_t)s * 256 + g * 64);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        r.B[u][jj] = bcol ? *(gv4u*)(xf + (((s * 4 + jj) * 4 + q) * XF_SPLIT + i) * 16) : v4u{0u, 0u, 0u, 0u};
    }
  }
}

template <int CH>
__device__ __forceinline__ void mx_tile_compute(const MxTile<CH>& r, int nb, int s0, int s1, v4f (&D)[4]) {
  const int q = __lane_id() >> 4;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int s = s0 + u;
    if (s >= s1) break;
    const bool valid = 4 * s + q < nb;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t e = (r.SC[u][g] >> (8 * q)) & 0xffu;
      const float scale = valid ? mx_scale_f32(e) : 0.f;
      const bool dbl = valid && e == 255u;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        D[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mx_a_operand(r.A[u][g][jj], scale, dbl),
                                                      __builtin_bit_cast(v8bf, r.B[u][jj]), D[g], 0, 0, 0);
    }
  }
}

// y for the tile's 64 rows over K-steps [s0, s1), written to red[64] (rows in
// tile order). D columns 0..2 (the three activation terms) are summed.
__device__ __forceinline__ void mx_tile_rows(const uint8_t* __restrict__ mat, int64_t qs_bytes, int nb, int nb4,
                                             int tile, int s0, int s1, const uint8_t* __restrict__ xf,
                                             float* __restrict__ red) {
  v4f D[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) D[g] = v4f{0.f, 0.f, 0.f, 0.f};
  MxTile<MX_CH> r;
  for (int p0 = s0; p0 < s1; p0 += MX_CH) {
    const int p1 = min(s1, p0 + MX_CH);
    mx_tile_load<MX_CH>(r, mat, qs_bytes, nb, nb4, tile, p0, p1, xf);
    mx_tile_compute<MX_CH>(r, nb, p0, p1, D);
  }
  const int lane = __lane_id();
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float d = D[g][k];
      const float y = d + __shfl_down(d, 1, 64) + __shfl_down(d, 2, 64);
      if ((lane & 15) == 0) red[g * 16 + (lane >> 4) * 4 + k] = y;
    }
  }
}

__device__ __forceinline__ const uint8_t* expert_base(const void* base, int64_t stride, const uint64_t* ptrs, int e) {
  return base ? (const uint8_t*)base + (int64_t)e * stride : (const uint8_t*)ptrs[e];
}

constexpr int GU_CHUNKS = 4;  // K chunks per gate/up tile (one wave each, per matrix)
constexpr int DN_CHUNKS = 4;  // K chunks per down tile

// phase 1: workgroup = (pair p, 64-row tile); wave = (matrix m, K chunk c).
// Writes the activation (fp32 and as an xfrag) and, from tile 0, the pair's
// expert id and routing weight.
__global__ __launch_bounds__(512) void moe_gu_mfma_kernel(MoeDev a) {
  __shared__ float red[2][GU_CHUNKS][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int tiles = a.n_ff >> 6;
  const int p = blockIdx.x / tiles, tile = blockIdx.x - p * tiles;
  const int t = p / a.top_k, j = p - t * a.top_k;
  int si[MAX_TOPK];
  float sw[MAX_TOPK];
  topk_regs(a.logits + (int64_t)t * a.E, a.E, a.top_k, a.mode, si, sw);
  const int e = clamp_expert(si[j], a.E);
  if (tile == 0 && wave == 0 && lane == 0) {
    a.ids[p] = e;
    a.wts[p] = sw[j];
  }
  const int m = wave & 1, c = wave >> 1;
  const uint8_t* mat = m == 0 ? expert_base(a.gate_base, a.gate_stride, a.gate_ptrs, e)
                              : expert_base(a.up_base, a.up_stride, a.up_ptrs, e);
  const int per = (a.nb4_gu + GU_CHUNKS - 1) / GU_CHUNKS;
  const int s0 = c * per, s1 = min(a.nb4_gu, s0 + per);
  mx_tile_rows(mat, a.qsb_gu, a.nb_gu, a.nb4_gu, tile, s0, s1,
               a.xf_h + (int64_t)t * a.nb4_gu * XF_STEP_BYTES, red[m][c]);
  __syncthreads();
  if (wave == 0) {
    const int row = tile * 64 + lane;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int k = 0; k < GU_CHUNKS; ++k) {
      g += red[0][k][lane];
      u += red[1][k][lane];
    }
    if (a.gate_bias) g += a.gate_bias[(int64_t)e * a.n_ff + row];
    if (a.up_bias) u += a.up_bias[(int64_t)e * a.n_ff + row];
    const float av = moe_act(a.act_kind, g, u, a.alpha, a.limit);
    a.act[(int64_t)p * a.n_ff + row] = av;
    uint32_t sp[3];
    split3(av, sp);
    uint8_t* xf = a.xf_a + (int64_t)p * a.nb4_d * XF_STEP_BYTES;
#pragma unroll
    for (int cc = 0; cc < XF_SPLIT; ++cc) *(uint16_t*)(xf + xfrag_offset(row, cc)) = (uint16_t)sp[cc];
  }
}

// phase 2: workgroup = (pair p, 64-row output tile); wave = K chunk.
// y[p] = down_e a_p + bias_e, combined across the token's experts later.
__global__ __launch_bounds__(256) void moe_down_mfma_kernel(MoeDev a) {
  __shared__ float red[DN_CHUNKS][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int tiles = a.n_embd >> 6;
  const int p = blockIdx.x / tiles, tile = blockIdx.x - p * tiles;
  const int e = clamp_expert(a.ids[p], a.E);
  const uint8_t* mat = expert_base(a.down_base, a.down_stride, a.down_ptrs, e);
  const int per = (a.nb4_d + DN_CHUNKS - 1) / DN_CHUNKS;
  const int s0 = wave * per, s1 = min(a.nb4_d, s0 + per);
  mx_tile_rows(mat, a.qsb_d, a.nb_d, a.nb4_d, tile, s0, s1, a.xf_a + (int64_t)p * a.nb4_d * XF_STEP_BYTES,
               red[wave]);
  __syncthreads();
  if (wave == 0) {
    const int row = tile * 64 + lane;
    float y = 0.f;
#pragma unroll
    for (int k = 0; k < DN_CHUNKS; ++k) y += red[k][lane];
    if (a.down_bias) y += a.down_bias[(int64_t)e * a.n_embd + row];
    a.ypair[(int64_t)p * a.n_embd + row] = y;
  }
}

// out[t] = sum over the token's experts in ascending id of w * y (thread per element)
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeDev a) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (n >= a.n_embd) return;
  const int k = a.top_k;
  int si[MAX_TOPK], order[MAX_TOPK];
  for (int jj = 0; jj < k; ++jj) si[jj] = a.ids[(int64_t)t * k + jj];
  slot_order(si, k, order);
  float o = 0.f;
  for (int jj = 0; jj < k; ++jj) {
    const int64_t q = (int64_t)t * k + order[jj];
    o = combine_one(o, a.wts[q], a.ypair[q * a.n_embd + n]);
  }
  a.out[(int64_t)t * a.n_embd + n] = o;
}

// ---------------------------------------------------------------------------
// raw GGUF rows (any format): phase 1 workgroup = (pair p, 32 rows), each wave
// computes whole gate and up rows; phase 2 workgroup = (token t, 32 output
// rows) with the token's top_k activation vectors staged in LDS.

constexpr int RAW_ROWS_PER_WG = 32;

template <int FMT>
__global__ __launch_bounds__(256) void moe_gu_raw_kernel(MoeDev a) {
  extern __shared__ float xs[];
  const int groups = (a.n_ff + RAW_ROWS_PER_WG - 1) / RAW_ROWS_PER_WG;
  const int p = blockIdx.x / groups;
  const int r0 = (blockIdx.x % groups) * RAW_ROWS_PER_WG;
  if (p >= a.T * a.top_k) return;
  const int e = clamp_expert(a.ids[p], a.E);
  const int t = p / a.top_k;
  const int K = a.n_embd;
  stage_x<1>(xs, a.h + (int64_t)t * K, NSX_DT_F32, K, 1, K, FMT == NSX_Q4_0 || FMT == NSX_Q4_K);
  const float* xsum = xs + K;
  const uint32_t rb = raw_row_bytes<FMT>(K);
  const uint8_t* gp = expert_base(a.gate_base, a.gate_stride, a.gate_ptrs, e);
  const uint8_t* up = expert_base(a.up_base, a.up_stride, a.up_ptrs, e);
  const uintptr_t ga = (uintptr_t)gp & ~(uintptr_t)3, ua = (uintptr_t)up & ~(uintptr_t)3;
  const uint32_t gh = (uint32_t)((uintptr_t)gp - ga), uh = (uint32_t)((uintptr_t)up - ua);
  const __amdgpu_buffer_rsrc_t rg = nsx_rsrc((const void*)ga, (gh + rb * (uint32_t)a.n_ff + 3u) & ~3u);
  const __amdgpu_buffer_rsrc_t ru = nsx_rsrc((const void*)ua, (uh + rb * (uint32_t)a.n_ff + 3u) & ~3u);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int nu = raw_units<FMT>(K);
  for (int r = r0 + wave; r < min(a.n_ff, r0 + RAW_ROWS_PER_WG); r += 4) {
    float g[1] = {0.f}, u[1] = {0.f};
    for (int k = lane; k < nu; k += 64) {
      raw_unit_dot<FMT, 1>(rg, gh + (uint32_t)r * rb, k, xs, K, xsum, g);
      raw_unit_dot<FMT, 1>(ru, uh + (uint32_t)r * rb, k, xs, K, xsum, u);
    }
    float gv = nsx_wave_sum(g[0]), uv = nsx_wave_sum(u[0]);
    if (lane == 0) {
      if (a.gate_bias) gv += a.gate_bias[(int64_t)e * a.n_ff + r];
      if (a.up_bias) uv += a.up_bias[(int64_t)e * a.n_ff + r];
      a.act[(int64_t)p * a.n_ff + r] = moe_act(a.act_kind, gv, uv, a.alpha, a.limit);
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(256) void moe_down_raw_kernel(MoeDev a) {
  extern __shared__ float xs[];  // [top_k][n_ff] then [top_k][n_ff/32]
  const int groups = (a.n_embd + RAW_ROWS_PER_WG - 1) / RAW_ROWS_PER_WG;
  const int t = blockIdx.x / groups;
  const int r0 = (blockIdx.x % groups) * RAW_ROWS_PER_WG;
  if (t >= a.T) return;
  const int K = a.n_ff, k = a.top_k;
  const bool sums = FMT == NSX_Q4_0 || FMT == NSX_Q4_K;
  for (int i = threadIdx.x; i < k * K; i += blockDim.x) xs[i] = a.act[(int64_t)t * k * K + i];
  __syncthreads();
  const int nsb = K / 32;
  float* xsum = xs + k * K;
  if (sums) {
    for (int i = threadIdx.x; i < k * nsb; i += blockDim.x) {
      const float* s = xs + (i / nsb) * K + (i % nsb) * 32;
      float v = 0.f;
      for (int jj = 0; jj < 32; ++jj) v += s[jj];
      xsum[i] = v;
    }
    __syncthreads();
  }
  int si[MAX_TOPK];
  for (int jj = 0; jj < k; ++jj) si[jj] = clamp_expert(a.ids[(int64_t)t * k + jj], a.E);
  int order[MAX_TOPK];
  slot_order(si, k, order);
  const uint32_t rb = raw_row_bytes<FMT>(K);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int nu = raw_units<FMT>(K);
  for (int r = r0 + wave; r < min(a.n_embd, r0 + RAW_ROWS_PER_WG); r += 4) {
    float o = 0.f;
    for (int jj = 0; jj < k; ++jj) {
      const int j = order[jj];
      const int eq = si[j];
      const uint8_t* dp = expert_base(a.down_base, a.down_stride, a.down_ptrs, eq);
      const uintptr_t da = (uintptr_t)dp & ~(uintptr_t)3;
      const uint32_t dh = (uint32_t)((uintptr_t)dp - da);
      const __amdgpu_buffer_rsrc_t rd = nsx_rsrc((const void*)da, (dh + rb * (uint32_t)a.n_embd + 3u) & ~3u);
      float acc[1] = {0.f};
      for (int u = lane; u < nu; u += 64)
        raw_unit_dot<FMT, 1>(rd, dh + (uint32_t)r * rb, u, xs + j * K, K, xsum + j * nsb, acc);
      float y = nsx_wave_sum(acc[0]);
      if (a.down_bias) y += a.down_bias[(int64_t)eq * a.n_embd + r];
      o = combine_one(o, a.wts[(int64_t)t * k + j], y);
    }
    if (lane == 0) a.out[(int64_t)t * a.n_embd + r] = o;
  }
}

// ---------------------------------------------------------------------------
// host side

struct MoePlan {
  int64_t off_logits, off_act, off_xfh, off_xfa, off_y, total;
  int nb4_gu, nb4_d;
};

static MoePlan moe_plan(const nsx_moe_layer* L, int64_t T) {
  MoePlan p{};
  const int64_t P = T * L->top_k;
  const bool t64 = L->layout == NSX_LAYOUT_T64;
  p.nb4_gu = (int)nsx_cdiv(L->n_embd / 32, 4);
  p.nb4_d = (int)nsx_cdiv(L->n_ff / 32, 4);
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  int64_t o = 0;
  p.off_logits = o;
  o = al(o + T * L->n_expert * 4);
  p.off_act = o;
  o = al(o + P * L->n_ff * 4);
  p.off_xfh = o;
  o = al(o + (t64 ? T * p.nb4_gu * XF_STEP_BYTES : 0));
  p.off_xfa = o;
  o = al(o + (t64 ? P * p.nb4_d * XF_STEP_BYTES : 0));
  p.off_y = o;
  o = al(o + (t64 ? P * L->n_embd * 4 : 0));
  p.total = o;
  return p;
}

static int check_layer(const nsx_moe_layer* L, int64_t T);

extern "C" int64_t nsx_moe_workspace_bytes(const nsx_moe_layer* L, int64_t T) {
  if (check_layer(L, T) != NSX_OK) return -1;
  return moe_plan(L, T).total;
}

static int check_layer(const nsx_moe_layer* L, int64_t T) {
  NSX_REQUIRE(L, NSX_EINVAL, "null layer");
  int rc = check_router(T, L->n_embd, L->router_dtype, L->n_expert, L->top_k, L->router_mode);
  if (rc) return rc;
  const int t = L->ggml_type;
  NSX_REQUIRE(t == NSX_MXFP4 || t == NSX_Q4_K || t == NSX_Q4_0 || t == NSX_Q8_0, NSX_ENOTIMPL,
              "expert weight type %d", t);
  NSX_REQUIRE(L->layout == NSX_LAYOUT_GGUF || (L->layout == NSX_LAYOUT_T64 && t == NSX_MXFP4), NSX_ENOTIMPL,
              "layout %d for type %d", L->layout, t);
  const int be = nsx_block_elems(t);
  NSX_REQUIRE(L->n_embd > 0 && L->n_ff > 0 && L->n_embd % be == 0 && L->n_ff % be == 0, NSX_EINVAL,
              "n_embd=%d n_ff=%d must be multiples of %d", L->n_embd, L->n_ff, be);
  NSX_REQUIRE(L->act == NSX_ACT_CLAMPED_SWIGLU || L->act == NSX_ACT_SILU_MUL, NSX_EINVAL, "act %d", L->act);
  NSX_REQUIRE(L->router_w && (L->gate_ptrs || L->gate_base) && (L->up_ptrs || L->up_base) &&
                  (L->down_ptrs || L->down_base),
              NSX_EINVAL, "null weights");
  const int64_t mx = std::max(L->n_embd, L->n_ff);
  NSX_REQUIRE((int64_t)raw_row_bytes<NSX_Q8_0>((int)mx) * mx < (1ll << 31), NSX_EINVAL, "expert matrix above 2 GiB");
  if (L->layout == NSX_LAYOUT_GGUF) {
    NSX_REQUIRE((int64_t)(L->n_embd + L->n_embd / 32) * 4 <= 64 * 1024, NSX_EINVAL, "n_embd too large for LDS");
    NSX_REQUIRE((int64_t)L->top_k * (L->n_ff + L->n_ff / 32) * 4 <= 160 * 1024, NSX_EINVAL,
                "top_k * n_ff too large for LDS");
  } else {
    NSX_REQUIRE(L->n_embd % 64 == 0 && L->n_ff % 64 == 0, NSX_EINVAL, "t64 layers need n_embd, n_ff % 64 == 0");

  }
  return NSX_OK;
}

template <int FMT>
static int launch_raw_phases(const MoeDev& d, int64_t T, hipStream_t st, bool gate_up, bool down) {
  const int64_t P = T * d.top_k;
  const size_t lds1 = (size_t)(d.n_embd + d.n_embd / 32) * 4;
  const unsigned g1 = (unsigned)(P * nsx_cdiv(d.n_ff, RAW_ROWS_PER_WG));
  if (gate_up) {
    int rc = nsx_launch(moe_gu_raw_kernel<FMT>, dim3(g1), dim3(256), lds1, st, d);
    if (rc) return rc;
  }
  if (!down) return NSX_OK;
  const size_t lds2 = (size_t)d.top_k * (d.n_ff + d.n_ff / 32) * 4;
  if (lds2 > 64 * 1024)
    NSX_HIP(hipFuncSetAttribute((const void*)moe_down_raw_kernel<FMT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds2));
  const unsigned g2 = (unsigned)(T * nsx_cdiv(d.n_embd, RAW_ROWS_PER_WG));
  return nsx_launch(moe_down_raw_kernel<FMT>, dim3(g2), dim3(256), lds2, st, d);
}

// Phases ph0..ph1 of one layer (NSX_PHASE_*); each later phase reads what
// the earlier ones left in the workspace.
static int moe_run(const nsx_moe_layer* L, const float* h, int64_t T, float* out, int32_t* ids, float* weights,
                   void* workspace, int64_t workspace_bytes, void* stream, int ph0, int ph1) {
  int rc = check_layer(L, T);
  if (rc) return rc;
  NSX_REQUIRE(h && out && ids && weights && workspace, NSX_EINVAL, "null buffer");
  const MoePlan p = moe_plan(L, T);
  NSX_REQUIRE(workspace_bytes >= p.total, NSX_EINVAL, "workspace of %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)p.total);
  NSX_REQUIRE(T * L->top_k < (1ll << 24), NSX_EINVAL, "too many (token, expert) pairs");
  hipStream_t st = S(stream);
  char* ws = (char*)workspace;
  const bool t64 = L->layout == NSX_LAYOUT_T64;

  MoeDev d{};
  d.logits = (const float*)(ws + p.off_logits);
  d.ids = ids;
  d.wts = weights;
  d.T = (int)T;
  d.top_k = L->top_k;
  d.E = L->n_expert;
  d.mode = L->router_mode;
  d.gate_ptrs = L->gate_ptrs;
  d.up_ptrs = L->up_ptrs;
  d.down_ptrs = L->down_ptrs;
  d.gate_base = L->gate_base;
  d.up_base = L->up_base;
  d.down_base = L->down_base;
  d.gate_stride = L->gate_stride;
  d.up_stride = L->up_stride;
  d.down_stride = L->down_stride;
  d.ypair = (float*)(ws + p.off_y);
  d.gate_bias = L->gate_bias;
  d.up_bias = L->up_bias;
  d.down_bias = L->down_bias;
  d.h = h;
  d.out = out;
  d.act = (float*)(ws + p.off_act);
  d.xf_h = (const uint8_t*)(ws + p.off_xfh);
  d.xf_a = (uint8_t*)(ws + p.off_xfa);
  d.n_embd = L->n_embd;
  d.n_ff = L->n_ff;
  d.act_kind = L->act;
  d.alpha = L->alpha;
  d.limit = L->limit;

  auto on = [&](int ph) { return ph0 <= ph && ph <= ph1; };
  if (on(NSX_PHASE_ROUTER)) {
    rc = launch_logits(h, T, L->n_embd, L->router_w, L->router_dtype, L->router_bias, L->n_expert,
                       (float*)(ws + p.off_logits), t64 ? (uint8_t*)(ws + p.off_xfh) : nullptr, st);
    if (rc) return rc;
    if (!t64 && (rc = launch_topk(d.logits, T, L->n_expert, L->top_k, L->router_mode, ids, weights, st))) return rc;
  }
  const int64_t P = T * L->top_k;

  if (t64) {
    d.nb_gu = L->n_embd / 32;
    d.nb4_gu = p.nb4_gu;
    d.nb_d = L->n_ff / 32;
    d.nb4_d = p.nb4_d;
    d.qsb_gu = nsx_cdiv(L->n_ff, 64) * d.nb_gu * 1024;
    d.qsb_d = nsx_cdiv(L->n_embd, 64) * d.nb_d * 1024;
    if (on(NSX_PHASE_GATE_UP) &&
        (rc = nsx_launch(moe_gu_mfma_kernel, dim3((unsigned)(P * (L->n_ff / 64))), dim3(128 * GU_CHUNKS), 0, st,
                         d)))
      return rc;
    if (on(NSX_PHASE_DOWN) &&
        (rc = nsx_launch(moe_down_mfma_kernel, dim3((unsigned)(P * (L->n_embd / 64))), dim3(64 * DN_CHUNKS), 0, st,
                         d)))
      return rc;
    if (on(NSX_PHASE_COMBINE) &&
        (rc = nsx_launch(moe_combine_kernel, dim3((unsigned)nsx_cdiv(L->n_embd, 256), (unsigned)T), dim3(256), 0, st,
                         d)))
      return rc;
    return NSX_OK;
  }
  switch (L->ggml_type) {  // the GGUF-layout down kernel also combines
    case NSX_MXFP4: return launch_raw_phases<NSX_MXFP4>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q4_K: return launch_raw_phases<NSX_Q4_K>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q4_0: return launch_raw_phases<NSX_Q4_0>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q8_0: return launch_raw_phases<NSX_Q8_0>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
  }
  return nsx_fail(NSX_ENOTIMPL, "expert weight type %d", L->ggml_type);
}

extern "C" int nsx_moe_forward(const nsx_moe_layer* L, const float* h, int64_t T, float* out, int32_t* ids,
                               float* weights, void* workspace, int64_t workspace_bytes, void* stream) {
  return moe_run(L, h, T, out, ids, weights, workspace, workspace_bytes, stream, NSX_PHASE_ROUTER,
                 NSX_PHASE_COMBINE);
}

extern "C" int nsx_moe_phase(const nsx_moe_layer* L, int phase, const float* h, int64_t T, float* out, int32_t* ids,
                             float* weights, void* workspace, int64_t workspace_bytes, void* stream) {
  NSX_REQUIRE(phase >= NSX_PHASE_ROUTER && phase <= NSX_PHASE_COMBINE, NSX_EINVAL, "phase %d", phase);
  return moe_run(L, h, T, out, ids, weights, workspace, workspace_bytes, stream, phase, phase);
}
