// MoE expert path for gfx950: router logits, top-k, routed expert products
// (block-scaled MFMA over t64 tiles, or VALU over raw GGUF rows), activation
// and the weighted combine -- with expert ids never leaving the device.
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
#include "mx.h"
#include "raw_dot.h"
#include "q4k_a8.h"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <stdlib.h>

static inline hipStream_t S(void* s) { return (hipStream_t)s; }

constexpr int MAX_TOPK = 8;
constexpr int MAX_EXPERTS = 256;

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int RT_TT = 8;

// 8 consecutive router weights (f32 / bf16 / f16) as floats, from global memory
template <int WDT>
__device__ __forceinline__ void load8_w(const void* W, int64_t off, float (&w)[8]) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  typedef const __attribute__((address_space(1))) v4u gv4u;
  if (WDT == NSX_F32) {
    const v4f a = *(gv4f*)((const float*)W + off);
    const v4f b = *(gv4f*)((const float*)W + off + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    const v4u q = *(gv4u*)((const uint16_t*)W + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = q[i] & 0xffffu, hi = q[i] >> 16;
      w[2 * i] = WDT == NSX_BF16 ? nsx_bf2f(lo) : nsx_h2f(lo);
      w[2 * i + 1] = WDT == NSX_BF16 ? nsx_bf2f(hi) : nsx_h2f(hi);
    }
  }
}

constexpr int RT_U = 2;      // 8-element chunks per thread and pass of the router (K <= 4096 in one pass)
constexpr int RT_XQ_WGS = 16;  // extra workgroups that quantize h for the t64 expert kernels

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

constexpr int TOPK_NV = MAX_EXPERTS / 64;  // logits per lane at most

// Issue the loads of one token's logits: lane l holds experts l + 64 i (i < NV).
// Unpredicated (index clamped); topk_select masks experts >= E.
template <int NV>
__device__ __forceinline__ void topk_load(const float* __restrict__ lg, int E, float (&v)[NV]) {
  const int lane = __lane_id();
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    v[i] = lg[e < E ? e : E - 1];
  }
}

// Top-k of the E <= 64 NV logits held as by topk_load, largest first, ties to
// the lower expert index. The lanes' remaining experts are lane masks per
// slot (slot i holds experts 64 i .. 64 i + 63); each round takes the wave
// maximum of the remaining keys (DPP), and the expert holding it with the
// lowest index is the lowest set bit of the first slot's ballot of "remaining
// and equal to the maximum". Results are wave-uniform. With weights false the
// softmax is skipped (sel_w is left zero), and only the first `rounds`
// experts are selected (the rest of sel_i is left zero).
template <int NV>
__device__ __forceinline__ void topk_select(float (&v)[NV], int E, int k, int mode, int (&sel_i)[MAX_TOPK],
                                            float (&sel_w)[MAX_TOPK], bool weights = true, int rounds = MAX_TOPK) {
  const int nr = weights ? k : min(k, rounds);
  const int lane = __lane_id();
  bool ok[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) ok[i] = lane + 64 * i < E;
  if (mode == NSX_ROUTE_QWEN3) {  // probs = softmax(logits) over all experts, float32 (router.py:65)
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (ok[i]) m = fmaxf(m, v[i]);
    m = key2f(nsx_wave_max_u32(f2key(m)));
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
    sel_v[j] = 0.f;
    sel_i[j] = 0;
    sel_w[j] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < MAX_TOPK; ++j) {
    if (j >= nr) break;
    uint32_t lk = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) lk = max(lk, ok[i] ? key[i] : 0u);
    const uint32_t mk = nsx_wave_max_u32(lk);
    int wi = 0;  // no expert left (E < k): index 0
    bool found = false;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint64_t b = __builtin_amdgcn_ballot_w64(ok[i] && key[i] == mk);
      if (!found && b != 0) {
        wi = 64 * i + (int)__builtin_ctzll(b);
        found = true;
      }
    }
    sel_i[j] = wi;
    sel_v[j] = key2f(mk);
#pragma unroll
    for (int i = 0; i < NV; ++i) ok[i] = ok[i] && lane + 64 * i != wi;
  }
  if (!weights) return;
  // static loop bounds (guards on k) keep sel_v / sel_w in registers
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAX_TOPK; ++j) {
    if (j < k) {
      // GPT-OSS: softmax over the selected logits in float32 (gpt_oss.py:120);
      // Qwen3: renormalise the selected probabilities (router.py:68)
      sel_w[j] = mode == NSX_ROUTE_GPTOSS ? expf(sel_v[j] - sel_v[0]) : sel_v[j];
      s += sel_w[j];
    }
  }
#pragma unroll
  for (int j = 0; j < MAX_TOPK; ++j)
    if (j < k) sel_w[j] = sel_w[j] / s;
}

// One token's top-k from its logits row (loads and selection), any E <= MAX_EXPERTS.
__device__ __forceinline__ void topk_regs(const float* __restrict__ lg, int E, int k, int mode,
                                          int (&sel_i)[MAX_TOPK], float (&sel_w)[MAX_TOPK], bool weights = true,
                                          int rounds = MAX_TOPK) {
  if (E <= 128) {
    float v[2];
    topk_load<2>(lg, E, v);
    topk_select<2>(v, E, k, mode, sel_i, sel_w, weights, rounds);
  } else {
    float v[TOPK_NV];
    topk_load<TOPK_NV>(lg, E, v);
    topk_select<TOPK_NV>(v, E, k, mode, sel_i, sel_w, weights, rounds);
  }
}

// The router's input as the residual stream of a stacked layer: h = rms_norm(x
// + r) * w (gpt_oss.py:126,177 -- the block's input norm), computed where it
// is read instead of by a launch of its own. `on` false: h is the input.
struct RtNorm {
  int on;
  const float* r;  // the previous block's output, added to x
  const float* w;  // norm weight (null: none)
  float eps;
  float* x_out;    // x + r, written by the first logit workgroup of each grid row
};

constexpr int NORM_MAXV = 16;  // values per thread of 256 (rows of n <= 4096)

// The residual add of a row (length n) in add_rmsnorm_kernel's layout --
// thread i of 256 holds elements i, i + 256, ... -- written to LDS row s when
// s is set; returns the thread's partial sum of squares in that kernel's
// order, so that a norm folded elsewhere gives its bits.
__device__ __forceinline__ float norm_stride(const float* __restrict__ x, const float* __restrict__ r, int n,
                                             float* s) {
  float v[NORM_MAXV];
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    const int c = min((int)threadIdx.x + i * 256, n - 1);
    v[i] = x[c] + r[c];
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    if ((int)threadIdx.x + i * 256 >= n) v[i] = 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  if (s) {
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
      const int c = threadIdx.x + i * 256;
      if (c < n) s[c] = v[i];
    }
  }
  return ss;
}

// 1 / rms from the threads' partial sums (wave sums, then the four waves in
// order, through part[wave][slot]); every thread of the 256 calls it
__device__ __forceinline__ float norm_inv(float ss, int n, float eps, float (*part)[RT_TT], int slot) {
  ss = nsx_wave_sum(ss);
  __syncthreads();  // an earlier call's readers of part are done
  if (__lane_id() == 0) part[threadIdx.x >> 6][slot] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) tot += part[i][slot];
  return 1.f / sqrtf(tot / (float)n + eps);
}

// Router logits (model/gpt_oss.py:97-99,116-121; moe/router.py:59-69).
// Workgroup e < E of grid row y computes expert e's logits for tokens 8y ..
// 8y + 7: its 256 threads split K into 8-element chunks (thread i: chunks i,
// i + 256, ...), so that a small batch spreads the router matrix over E
// compute units, and the four waves' partial sums meet in LDS in a fixed
// order. With xq set, RT_XQ_WGS more workgroups per grid row build the
// tokens' activation terms. Loads are unpredicated (addresses clamped, tails
// zeroed after the load) so that they are all in flight together. With the
// norm on, h is rms_norm(h + nm.r) * nm.w, as add_rmsnorm_kernel computes it.
template <int WDT>
__global__ __launch_bounds__(256) void router_logits_kernel(const float* __restrict__ h, int T, int K,
                                                            const void* __restrict__ W,
                                                            const float* __restrict__ bias, int E,
                                                            float* __restrict__ logits, uint8_t* __restrict__ xq,
                                                            RtNorm nm) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  __shared__ float part[4][RT_TT];
  __shared__ __align__(16) float s_rows[2][256 * NORM_MAXV];  // norm on: rows of x + r (or x + r and the weights)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int t0 = blockIdx.y * RT_TT;
  const int nt = min(RT_TT, T - t0);
  if ((int)blockIdx.x >= E) {  // activation terms of h, two blocks per wave task
    const int nb = K / 32, ns = (nb + 3) / 4, pairs = 2 * ns;
    if (!nm.on) {
      const int64_t tasks = (int64_t)T * pairs;
      const int64_t nwaves = (int64_t)gridDim.y * RT_XQ_WGS * 4;
      for (int64_t task = ((int64_t)blockIdx.y * RT_XQ_WGS + (blockIdx.x - E)) * 4 + wave; task < tasks;
           task += nwaves) {
        const int t = (int)(task / pairs), b = (int)(task % pairs) * 2 + (lane >> 5);
        const float r = h[(int64_t)t * K + (b < nb ? b : nb - 1) * 32 + (lane & 31)];
        xq_block(b < nb ? r : 0.f, b, xq + (int64_t)t * ns * XQ_STEP);
      }
      return;
    }
    // norm on: workgroup j of the row takes token j % nt and every (RT_XQ_WGS / nt)-th task of it
    const int j = blockIdx.x - E, slices = RT_XQ_WGS / nt;
    if (j >= slices * nt) return;
    const int t = t0 + j % nt, sl = j / nt;
    // x + r and the norm weights go through LDS (one round trip; the terms take one element per lane)
    float* s_v = s_rows[0];
    float* s_w = s_rows[1];
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
      const int c = threadIdx.x + i * 256;
      if (c < K) s_w[c] = nm.w ? nm.w[c] : 1.f;  // a unit weight multiplies exactly
    }
    const float ssq = norm_stride(h + (int64_t)t * K, nm.r + (int64_t)t * K, K, s_v);
    const float inv = norm_inv(ssq, K, nm.eps, part, 0);  // (its barriers publish s_v, s_w)
    for (int task = sl * 4 + wave; task < pairs; task += slices * 4) {
      const int b = task * 2 + (lane >> 5);
      const int c = (b < nb ? b : nb - 1) * 32 + (lane & 31);
      const float hn = (s_v[c] * inv) * s_w[c];  // a unit weight multiplies exactly
      xq_block(b < nb ? hn : 0.f, b, xq + (int64_t)t * ns * XQ_STEP);
    }
    return;
  }
  const int e = blockIdx.x;
  const int nc = K / 8;  // 8-element chunks
  // norm on: h = ((x + r) * inv) * w, x + r of the first RT_KEEP tokens kept in
  // LDS from the norm pass (add_rmsnorm_kernel's layout) for the dot's chunks
  constexpr int RT_KEEP = 2;
  float inv[RT_TT];
  float w0[RT_U][8], nw0[RT_U][8];  // norm on (K <= 4096, one pass): the router row and the norm weights,
  if (nm.on) {                       // loaded ahead of the norm pass so that one round trip covers both
#pragma unroll
    for (int u = 0; u < RT_U; ++u) {
      const int c = min(u * 256 + (int)threadIdx.x, nc - 1);
      load8_w<WDT>(W, (int64_t)e * K + 8 * (int64_t)c, w0[u]);
      const v4f a = nm.w ? *(gv4f*)(nm.w + 8 * c) : v4f{1.f, 1.f, 1.f, 1.f};
      const v4f b = nm.w ? *(gv4f*)(nm.w + 8 * c + 4) : v4f{1.f, 1.f, 1.f, 1.f};
      nw0[u][0] = a.x; nw0[u][1] = a.y; nw0[u][2] = a.z; nw0[u][3] = a.w;
      nw0[u][4] = b.x; nw0[u][5] = b.y; nw0[u][6] = b.z; nw0[u][7] = b.w;
    }
  }
#pragma unroll
  for (int i = 0; i < RT_TT; ++i) inv[i] = 1.f;
  if (nm.on) {
    float ss[RT_TT];
#pragma unroll
    for (int i = 0; i < RT_TT; ++i) {
      ss[i] = 0.f;
      if (i >= nt) continue;
      const float* xr = h + (int64_t)(t0 + i) * K;
      const float* rr = nm.r + (int64_t)(t0 + i) * K;
      ss[i] = norm_stride(xr, rr, K, i < RT_KEEP ? s_rows[i] : nullptr);
      // x + r for the next layer: elements 256 j .. 256 j + 255 written by workgroup j % E
      float* xo = nm.x_out + (int64_t)(t0 + i) * K;
      for (int j = e; 256 * j < K; j += E) {
        const int c = 256 * j + (int)threadIdx.x;
        if (c < K) xo[c] = xr[c] + rr[c];
      }
    }
#pragma unroll
    for (int i = 0; i < RT_TT; ++i) {
      const float sw = nsx_wave_sum(ss[i]);
      if (lane == 0 && i < nt) part[wave][i] = sw;
    }
    __syncthreads();  // (also publishes the kept rows)
#pragma unroll
    for (int i = 0; i < RT_TT; ++i) {
      float tot = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) tot += part[wv][i];
      inv[i] = i < nt ? 1.f / sqrtf(tot / (float)K + nm.eps) : 1.f;
    }
  }
  float acc[RT_TT];
#pragma unroll
  for (int i = 0; i < RT_TT; ++i) acc[i] = 0.f;
  for (int c0 = 0; c0 < nc; c0 += RT_U * 256) {
    float w[RT_U][8];
    if (nm.on) {
#pragma unroll
      for (int u = 0; u < RT_U; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) w[u][j] = w0[u][j];
    } else {
#pragma unroll
      for (int u = 0; u < RT_U; ++u) {
        const int c = c0 + u * 256 + (int)threadIdx.x;
        load8_w<WDT>(W, (int64_t)e * K + 8 * (int64_t)min(c, nc - 1), w[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < RT_U; ++u) {
      const bool in = c0 + u * 256 + (int)threadIdx.x < nc;
#pragma unroll
      for (int j = 0; j < 8; ++j) w[u][j] = in ? w[u][j] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < RT_TT; ++i) {
      if (i >= nt) break;
      const float* hp = h + (int64_t)(t0 + i) * K;
      float hv[RT_U][8];
#pragma unroll
      for (int u = 0; u < RT_U; ++u) {
        const int c = min(c0 + u * 256 + (int)threadIdx.x, nc - 1);
        if (!nm.on) {
          const v4f ha = *(gv4f*)(hp + 8 * c), hb = *(gv4f*)(hp + 8 * c + 4);
          hv[u][0] = ha.x; hv[u][1] = ha.y; hv[u][2] = ha.z; hv[u][3] = ha.w;
          hv[u][4] = hb.x; hv[u][5] = hb.y; hv[u][6] = hb.z; hv[u][7] = hb.w;
        } else {  // h = ((x + r) * inv) * w, as add_rmsnorm_kernel (K <= 4096: one pass, c0 = 0)
          float v[8];
          if (i < RT_KEEP) {
            const v4f a = *(const v4f*)(s_rows[i < RT_KEEP ? i : 0] + 8 * c);
            const v4f b = *(const v4f*)(s_rows[i < RT_KEEP ? i : 0] + 8 * c + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
          } else {
            const float* rp = nm.r + (int64_t)(t0 + i) * K;
            const v4f xa = *(gv4f*)(hp + 8 * c), xb = *(gv4f*)(hp + 8 * c + 4);
            const v4f ra = *(gv4f*)(rp + 8 * c), rb = *(gv4f*)(rp + 8 * c + 4);
            v[0] = xa.x + ra.x; v[1] = xa.y + ra.y; v[2] = xa.z + ra.z; v[3] = xa.w + ra.w;
            v[4] = xb.x + rb.x; v[5] = xb.y + rb.y; v[6] = xb.z + rb.z; v[7] = xb.w + rb.w;
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) hv[u][j] = (v[j] * inv[i]) * nw0[u][j];  // a unit weight multiplies exactly
        }
      }
      float sacc = acc[i];
#pragma unroll
      for (int u = 0; u < RT_U; ++u)  // w is zero past K
#pragma unroll
        for (int j = 0; j < 8; ++j) sacc = fmaf(w[u][j], hv[u][j], sacc);
      acc[i] = sacc;
    }
  }
  __shared__ float red[4][RT_TT];
#pragma unroll
  for (int i = 0; i < RT_TT; ++i) {
    if (i >= nt) break;
    const float sum = nsx_wave_sum(acc[i]);
    if (lane == 0) red[wave][i] = sum;
  }
  __syncthreads();
  if ((int)threadIdx.x < nt) {
    const int i = threadIdx.x;
    const float sum = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
    logits[(int64_t)(t0 + i) * E + e] = bias ? sum + bias[e] : sum;
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
                         float* logits, uint8_t* xq, hipStream_t st, RtNorm nm = RtNorm{0, nullptr, nullptr, 0.f, nullptr}) {
  const dim3 grid((unsigned)(E + (xq ? RT_XQ_WGS : 0)), (unsigned)nsx_cdiv(T, RT_TT));
  if (wdt == NSX_BF16)
    return nsx_launch(router_logits_kernel<NSX_BF16>, grid, dim3(256), 0, st, h, (int)T, (int)K, w, bias, (int)E,
                      logits, xq, nm);
  if (wdt == NSX_F16)
    return nsx_launch(router_logits_kernel<NSX_F16>, grid, dim3(256), 0, st, h, (int)T, (int)K, w, bias, (int)E,
                      logits, xq, nm);
  return nsx_launch(router_logits_kernel<NSX_F32>, grid, dim3(256), 0, st, h, (int)T, (int)K, w, bias, (int)E, logits,
                    xq, nm);
}

static int launch_topk(const float* logits, int64_t T, int64_t E, int k, int mode, int32_t* ids, float* wts,
                       hipStream_t st) {
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)nsx_cdiv(T, 4)), dim3(256), 0, st, logits, (int)T, (int)E, k, mode,
                     ids, wts);
  NSX_LAUNCHED();
  return NSX_OK;
}


// Bytes of one row of the Q4_K matrix-core kernels' activation terms for K
// columns (K a multiple of 256): hi[K], lo[K] (f16), sub-block sums hi[K/32],
// lo[K/32] (f16), 2^e (f32), padding to 16 bytes.
__host__ __device__ constexpr int64_t mq_row_bytes(int64_t K) { return 4 * K + K / 8 + 16; }

// One row x of K columns as those terms, by a workgroup of 256 threads (red:
// 4 floats of LDS): x' = x * 2^-e with max |x'| < 512, hi = f16(x'), lo =
// f16(x' - hi); the 32-element sums of x' likewise (< 2^14, inside f16's
// range); then 2^e.
// K <= MQ_TR_MAXK; 256 threads; sx: K floats of LDS. Each thread's elements (k = thread + 256 i) are loaded
// once, all in flight together (a loop with one load per pass waits a round trip per pass), then the max,
// the terms and, from the scaled values staged in sx, the sub-block sums in element order.
constexpr int MQ_TR_MAXK = 4096;
__device__ __forceinline__ void mq_terms_row(const float* __restrict__ xr, int K, uint8_t* __restrict__ row,
                                             float* red, float* sx) {
  constexpr int NV = MQ_TR_MAXK / 256;
  _Float16* hi = (_Float16*)row;
  _Float16* lo = hi + K;
  _Float16* shi = lo + K;
  _Float16* slo = shi + K / 32;
  const int tid = (int)threadIdx.x;
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = xr[min(tid + 256 * i, K - 1)];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (tid + 256 * i < K) mx = fmaxf(mx, fabsf(v[i]));
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  if (mx > 0.f && mx <= 3.4e38f) (void)frexpf(mx, &ex);  // mx < 2^ex
  const int e = ex - 9;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = tid + 256 * i;
    if (k < K) {
      const float vs = ldexpf(v[i], -e);
      const _Float16 h = (_Float16)vs;
      hi[k] = h;
      lo[k] = (_Float16)(vs - (float)h);
      sx[k] = vs;
    }
  }
  __syncthreads();
  for (int sidx = tid; sidx < K / 32; sidx += 256) {
    float acc = 0.f;
    for (int i = 0; i < 32; ++i) acc += sx[32 * sidx + i];
    const _Float16 h = (_Float16)acc;
    shi[sidx] = h;
    slo[sidx] = (_Float16)(acc - (float)h);
  }
  if (tid == 0) *(float*)(slo + K / 32) = ldexpf(1.f, e);
}

// ---------------------------------------------------------------------------
// Router logits for several tokens (T >= RM_MIN_T) as fp32 MFMA tiles.
//
// logits = h W^T is a small GEMM; the one-wave-per-expert kernel above
// re-reads each token group's h per expert. Here a wave computes a 16-token x
// 16-expert tile over one K-chunk of RM_KC with v_mfma_f32_16x16x4f32 (fp32
// products, fp32 accumulation; all of the chunk's loads in flight at once),
// and writes the tile's partial sums; router_reduce_kernel adds the chunks in
// a fixed order, adds the bias, writes the logits and selects the top-k. A
// workgroup is 4 waves: one token tile, 4 adjacent expert tiles (their h
// loads hit the same lines). Extra workgroups past the tiles build h's
// activation terms: the t64 layers' blocks, as in router_logits_kernel, or
// (xq_mq) the Q4_K matrix-core kernels' term rows, a workgroup per token.
//
// Operand layout of v_mfma_f32_16x16x4f32: A[i][k] in lane i + 16 k, B[k][j]
// in lane j + 16 k, D[i][j] in lane j + 16 (i / 4), register i % 4. Lane
// (i, q) loads 4 consecutive elements k0 + 4q .. k0 + 4q + 3 of its token's
// h and of its expert's row; MFMA u (0..3) takes element u of both, so the
// four MFMAs of a 16-wide step cover it in full.

constexpr int RM_MIN_T = 16;  // tokens from which the MFMA router runs
constexpr int RM_KC = 128;    // K per chunk (8 steps of 16)
constexpr int RM_EW = 4;      // expert tiles (waves) per workgroup
constexpr int RM_XQ = 2;      // h block pairs quantized per wave
constexpr int RM_RB = 32;     // partials per expert slot loaded at once in router_reduce_kernel (K <= 4096: one round)

// (the dtype known at compile time: a run-time branch around the load converts inside the branch, and each
// such load is waited for before the next one goes out)
template <int WDT>
__device__ __forceinline__ void load4_w(const void* W, int64_t off, float (&w)[4]) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  typedef const __attribute__((address_space(1))) u32x2 gu2;
  if constexpr (WDT == NSX_F32) {
    const v4f a = *(gv4f*)((const float*)W + off);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else {
    const u32x2 q = *(gu2*)((const uint16_t*)W + off);
    const uint32_t v[4] = {q.x & 0xffffu, q.x >> 16, q.y & 0xffffu, q.y >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = WDT == NSX_BF16 ? nsx_bf2f(v[i]) : nsx_h2f(v[i]);
  }
}

template <int WDT>
__global__ __launch_bounds__(64 * RM_EW) void router_mfma_kernel(const float* __restrict__ h, int T, int K,
                                                                 const void* __restrict__ W, int E,
                                                                 float* __restrict__ part, int ntile,
                                                                 uint8_t* __restrict__ xq, int xq_mq) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  if (xq_mq && (int)blockIdx.x >= ntile) {  // token blockIdx.x - ntile's term row
    __shared__ float red[4];
    __shared__ float sx[MQ_TR_MAXK];
    const int t = (int)blockIdx.x - ntile;
    mq_terms_row(h + (int64_t)t * K, K, xq + (int64_t)t * mq_row_bytes(K), red, sx);
    return;
  }
  if ((int)blockIdx.x >= ntile) {  // activation terms of h: RM_XQ tasks (two blocks each) per wave
    const int nb = K / 32, ns = (nb + 3) / 4, pairs = 2 * ns;
    const int64_t tasks = (int64_t)T * pairs;
    const int64_t task0 = ((int64_t)(blockIdx.x - ntile) * RM_EW + wave) * RM_XQ;
    float r[RM_XQ];
#pragma unroll
    for (int u = 0; u < RM_XQ; ++u) {  // loads first
      const int64_t task = min(task0 + u, tasks - 1);
      const int t = (int)(task / pairs), b = (int)(task % pairs) * 2 + (lane >> 5);
      r[u] = h[(int64_t)t * K + (b < nb ? b : nb - 1) * 32 + (lane & 31)];
    }
#pragma unroll
    for (int u = 0; u < RM_XQ; ++u) {
      const int64_t task = task0 + u;
      if (task >= tasks) break;
      const int t = (int)(task / pairs), b = (int)(task % pairs) * 2 + (lane >> 5);
      xq_block(b < nb ? r[u] : 0.f, b, xq + (int64_t)t * ns * XQ_STEP);
    }
    return;
  }
  const int ET = (E + 16 * RM_EW - 1) / (16 * RM_EW), TT = (T + 15) / 16;
  int b = (int)blockIdx.x;
  const int eg = b % ET;
  b /= ET;
  const int tt = b % TT, kc = b / TT;
  const int t0 = tt * 16, e0 = (eg * RM_EW + wave) * 16;
  const int ti = min(t0 + (lane & 15), T - 1), ei = min(e0 + (lane & 15), E - 1);
  const int q = lane >> 4;
  const int k_lo = kc * RM_KC, k_hi = min(K, k_lo + RM_KC);
  v4f a[RM_KC / 16];
  float w[RM_KC / 16][4];
#pragma unroll
  for (int s = 0; s < RM_KC / 16; ++s) {
    const int k = k_lo + 16 * s + 4 * q;
    const int kk = k < k_hi ? k : k_hi - 4;  // (K is a multiple of 16: a chunk ends on a whole step)
    a[s] = *(gv4f*)(h + (int64_t)ti * K + kk);
    load4_w<WDT>(W, (int64_t)ei * K + kk, w[s]);
  }
  // every step computed, those past the chunk's end on zeros (both operands: a weight may be infinite): a
  // loop exit at the end would sink each step's loads into its own block, a round trip per step
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < RM_KC / 16; ++s) {
    const bool on = k_lo + 16 * s < k_hi;
    const v4f as = on ? a[s] : v4f{0.f, 0.f, 0.f, 0.f};
    float ws[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ws[i] = on ? w[s][i] : 0.f;
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(as.x, ws[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(as.y, ws[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(as.z, ws[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(as.w, ws[3], acc, 0, 0, 0);
  }
  const int e = e0 + (lane & 15);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * q + r;
    if (t < T && e < E) part[((int64_t)kc * T + t) * E + e] = acc[r];
  }
}

// one wave per token: logits = sum of the K-chunk partials in chunk order +
// bias (written out), then the top-k as topk_kernel
template <int NV>
__device__ __forceinline__ void router_reduce_token(const float* __restrict__ part, int nkc, int T, int E, int t,
                                                    const float* __restrict__ bias, int k, int mode,
                                                    float* __restrict__ logits, int32_t* __restrict__ ids,
                                                    float* __restrict__ wts) {
  const int lane = __lane_id();
  float acc[NV], bv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    acc[i] = 0.f;
    // the bias first, unpredicated (no bias: a partial, not used): behind a branch after the partials it
    // would be one more round trip
    bv[i] = *(bias ? bias + min(lane + 64 * i, E - 1) : part);
  }
  for (int c0 = 0; c0 < nkc; c0 += RM_RB) {  // NV x RM_RB loads in flight, then the adds in chunk order
    float pv[NV][RM_RB];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int u = 0; u < RM_RB; ++u)
        pv[i][u] = part[((int64_t)min(c0 + u, nkc - 1) * T + t) * E + min(lane + 64 * i, E - 1)];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int u = 0; u < RM_RB; ++u) acc[i] = c0 + u < nkc ? acc[i] + pv[i][u] : acc[i];
  }
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = bias ? acc[i] + bv[i] : acc[i];
    if (lane + 64 * i < E) logits[(int64_t)t * E + lane + 64 * i] = v[i];
  }
  int si[MAX_TOPK];
  float sw[MAX_TOPK];
  topk_select<NV>(v, E, k, mode, si, sw);
  if (lane == 0)
    for (int j = 0; j < k; ++j) {
      ids[(int64_t)t * k + j] = si[j];
      wts[(int64_t)t * k + j] = sw[j];
    }
}

__global__ __launch_bounds__(256) void router_reduce_kernel(const float* __restrict__ part, int nkc, int T, int E,
                                                            const float* __restrict__ bias, int k, int mode,
                                                            float* __restrict__ logits, int32_t* __restrict__ ids,
                                                            float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= T) return;
  if (E <= 128)
    router_reduce_token<2>(part, nkc, T, E, t, bias, k, mode, logits, ids, wts);
  else
    router_reduce_token<TOPK_NV>(part, nkc, T, E, t, bias, k, mode, logits, ids, wts);
}

static int rm_chunks(int64_t K) { return (int)nsx_cdiv(K, RM_KC); }

static int launch_router_mfma(const float* h, int64_t T, int64_t K, const void* w, int wdt, const float* bias,
                              int64_t E, int k, int mode, float* part, float* logits, int32_t* ids, float* wts,
                              uint8_t* xq, bool xq_mq, hipStream_t st) {
  const int64_t ntile = nsx_cdiv(E, 16 * RM_EW) * nsx_cdiv(T, 16) * rm_chunks(K);
  const int64_t xq_tasks = T * 2 * nsx_cdiv(K / 32, 4);
  const int64_t grid = ntile + (xq ? (xq_mq ? T : nsx_cdiv(xq_tasks, (int64_t)RM_EW * RM_XQ)) : 0);
  const dim3 g((unsigned)grid), b(64 * RM_EW);
  int rc = wdt == NSX_F32    ? nsx_launch(router_mfma_kernel<NSX_F32>, g, b, 0, st, h, (int)T, (int)K, w, (int)E, part,
                                          (int)ntile, xq, (int)xq_mq)
           : wdt == NSX_BF16 ? nsx_launch(router_mfma_kernel<NSX_BF16>, g, b, 0, st, h, (int)T, (int)K, w, (int)E, part,
                                          (int)ntile, xq, (int)xq_mq)
                             : nsx_launch(router_mfma_kernel<NSX_F16>, g, b, 0, st, h, (int)T, (int)K, w, (int)E, part,
                                          (int)ntile, xq, (int)xq_mq);
  if (rc) return rc;
  return nsx_launch(router_reduce_kernel, dim3((unsigned)nsx_cdiv(T, 4)), dim3(256), 0, st, (const float*)part,
                    rm_chunks(K), (int)T, (int)E, bias, k, mode, logits, ids, wts);
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
// t64 GEMV over a row window (stream_linear over resident t64 slabs): one
// workgroup per tile; the window's tokens (up to 4) are first quantized into
// activation terms in LDS, then the four waves split the K-steps and meet in
// LDS.

constexpr int T64_S = 3;  // K-steps in flight per wave

__global__ __launch_bounds__(256) void t64_gemv_kernel(const uint8_t* __restrict__ mat, MxGeom G, int64_t row_lo,
                                                       int64_t row_hi, int tile0, const float* __restrict__ x, int K,
                                                       int T, float* __restrict__ y, int64_t ystride) {
  extern __shared__ __align__(16) uint8_t smem[];
  float* red = (float*)smem;                 // [wave 4][token 4][row 64]
  uint8_t* xq = smem + 4 * 4 * 64 * 4;       // [token][ns][XQ_STEP]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int64_t xstride = (int64_t)G.ns * XQ_STEP;
  const int pairs = 2 * G.ns;  // block pairs per token, padding blocks of the last step included
  for (int task = wave; task < T * pairs; task += 4) {
    const int t = task / pairs, b = (task % pairs) * 2 + (lane >> 5);
    const float r = b < G.nb ? x[(int64_t)t * K + b * 32 + (lane & 31)] : 0.f;
    xq_block(r, b, xq + t * xstride);
  }
  __syncthreads();
  const int tile = tile0 + blockIdx.x;
  const int per = (G.ns + 3) / 4;
  const int s0 = wave * per, s1 = min(G.ns, s0 + per);
  v4f D[4] = {};
  mx_tile_mfma<T64_S, true>(mat + (int64_t)tile * G.tile_bytes, G, s0, s1, xq, 0, xstride, T, D);
  mx_sum_terms(D);
  if ((lane & 3) == 0) {
    const int tok = (lane & 15) >> 2, r0 = 4 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 4; ++g) *(v4f*)(red + (wave * 4 + tok) * 64 + 16 * g + r0) = D[g];
  }
  __syncthreads();
  if (wave < T) {
    const int64_t row = (int64_t)tile * 64 + lane;
    const float v = red[(0 * 4 + wave) * 64 + lane] + red[(1 * 4 + wave) * 64 + lane] +
                    red[(2 * 4 + wave) * 64 + lane] + red[(3 * 4 + wave) * 64 + lane];
    if (row >= row_lo && row < row_hi) y[(int64_t)wave * ystride + (row - row_lo)] = v;
  }
}

extern "C" int nsx_t64_gemv(int t, const void* t64, int64_t n_rows, int64_t K, int64_t row_lo, int64_t row_hi,
                            const void* x, int x_dtype, int64_t T, float* y, void* stream) {
  NSX_REQUIRE(t == NSX_MXFP4, NSX_ENOTIMPL, "t64 GEMV is implemented for MXFP4 only (type %d)", t);
  NSX_REQUIRE(K > 0 && K % 32 == 0 && K <= 8192, NSX_EINVAL, "t64 GEMV takes K in 32..8192, a multiple of 32 "
              "(K=%lld)", (long long)K);
  NSX_REQUIRE(0 <= row_lo && row_lo <= row_hi && row_hi <= n_rows, NSX_EINVAL, "row window [%lld, %lld) of %lld",
              (long long)row_lo, (long long)row_hi, (long long)n_rows);
  NSX_REQUIRE(T >= 1 && T <= 4, NSX_EINVAL, "t64 GEMV takes T in 1..4 (T=%lld)", (long long)T);
  NSX_REQUIRE(x_dtype == NSX_DT_F32, NSX_ETYPE, "t64 GEMV takes fp32 activations");
  if (row_hi == row_lo) return NSX_OK;
  NSX_REQUIRE(t64 && x && y, NSX_EINVAL, "null buffer");
  const MxGeom G = mx_geom(n_rows, K);
  const int64_t tile0 = row_lo / 64, tile1 = nsx_cdiv(row_hi, 64);
  const size_t lds = 4 * 4 * 64 * 4 + (size_t)T * G.ns * XQ_STEP;
  if (lds > 64 * 1024)
    NSX_HIP(hipFuncSetAttribute((const void*)t64_gemv_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  return nsx_launch(t64_gemv_kernel, dim3((unsigned)(tile1 - tile0)), dim3(256), lds, S(stream),
                    (const uint8_t*)t64, G, row_lo, row_hi, (int)tile0, (const float*)x, (int)K, (int)T, y,
                    row_hi - row_lo);
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
  const uint64_t* gate_tiles;  // t64: tile t of expert e at X_tiles[e * tiles + t] (when set)
  const uint64_t* up_tiles;
  const uint64_t* down_tiles;
  const void* gate_base;
  const void* up_base;
  const void* down_base;
  int64_t gate_stride, up_stride, down_stride;
  const float* gate_bias;
  const float* up_bias;
  const float* down_bias;
  const float* h;
  float* out;
  float* act;            // (pairs, n_ff) fp32 activations (GGUF-layout path)
  const uint8_t* xq_h;   // activation terms of h, per token (t64, Q4_K matrix-core and grouped Q4_K paths)
  uint8_t* xq_a;         // activation terms of the expert activation, per pair (same paths)
  int n_embd, n_ff;
  MxGeom ggu, gdn;       // t64 geometry of a gate/up and of a down matrix
  int cg, sg;            // gate/up K-chunks and K-steps per chunk
  int cd, sd;            // down K-chunks per expert and K-steps per chunk
  int act_kind;
  float alpha, limit;
  // grouped dispatch (pairs sorted by expert)
  int4* items;           // work items: (expert, first sorted position, tokens, q | pairs of the expert << 16)
  int* n_items;
  int4* gu_items;        // the MXFP4 gate/up kernel's work items: (expert, first sorted position, tokens, 0)
  int* gu_bounds;        // [9]: XCD x runs gate/up units [gu_bounds[x], gu_bounds[x + 1])
  int* dn_bounds;        // [9]: the same for the down kernel's units (same items, its own tiles)
  int* gu_ctr;           // [8]: XCD x's gate/up units taken past its first two rounds (the sort zeroes them)
  int* dn_ctr;           // [9]: the same for the persistent down kernel, then its workgroups done (the last resets all)
  int32_t* sorted;       // pair ids, ascending expert, ascending pair id inside
  int32_t* corder;       // per token: its pair ids in ascending expert id
  float* y;              // (pairs, n_embd) expert outputs, bias included
  int max_items;
  int cdg, sdg;          // grouped down: K-chunks and K-steps per chunk
  int topk_in_gu;        // per-pair GGUF-layout paths: the gate/up kernel selects the top-k (no top-k launch)
  int topk_in_sort;      // grouped, T < RM_MIN_T: the sort kernel selects the top-k (no top-k launch)
  // decode chain of stacked layers (T = 1; moe_gu_chain_kernel, moe_down_chain_kernel)
  float* cx;             // the token's residual stream, updated in place by the down kernel
  const float* cnorm_w;  // this layer's norm weight (null: unit)
  float ceps;
  const float* crouter_b;  // this layer's router bias (null: none)
  const float* cp_in;    // this layer's router shares: [cp_groups][E] partial logits, then [cp_groups] sums of squares
  int cp_groups;         // shares per layer: the down kernel's work items of one token
  const void* cn_w;      // the next layer's router matrix (null: last layer, no shares written)
  int cn_wdt, cn_E;
  const float* cn_norm_w;  // the next layer's norm weight (null: unit)
  float* cp_out;         // the next layer's router shares
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

// The activation terms of K-blocks [2 * tiles, 4 * ns) -- the padding of the
// down matrix's last K-step, past n_ff -- are zero; the workgroup of the last
// gate/up tile writes them, so no call relies on what a workspace held before.
__device__ __forceinline__ void xq_zero_tail(int tile, const MxGeom& ggu, const MxGeom& gdn, uint8_t* dst) {
  if (tile != (int)ggu.tiles - 1) return;
  for (int b0 = 2 * (int)ggu.tiles; b0 < 4 * gdn.ns; b0 += 2) xq_block(0.f, b0 + (__lane_id() >> 5), dst);
}

// out[rows] += w * y in the reference rounds the product and the sum separately
__device__ __forceinline__ float combine_one(float acc, float w, float y) { return __fadd_rn(acc, __fmul_rn(w, y)); }

// ---------------------------------------------------------------------------
// expert kernels over t64 tiles (MXFP4, block-scaled MFMA)
//
// Every kernel finds its pair's expert with the same wave-level top-k over
// the token's logits, so no kernel waits on another's small outputs. Split-K
// partial sums go to separate slots and are added in a fixed order by the
// next kernel: results do not depend on scheduling.

// (the table is read as constant memory: for a wave-uniform e that is a scalar
// load, whose wait does not hold up the wave's vector loads in flight)
// (the pointer tables are read as constants: scalar loads, whose waits do not
// wait on the vector loads in flight, such as the pair list read just before)
typedef const __attribute__((address_space(4))) uint64_t nsx_cu64;
__device__ __forceinline__ const uint8_t* expert_base(const void* base, int64_t stride, const uint64_t* ptrs, int e) {
  return base ? (const uint8_t*)base + (int64_t)e * stride : (const uint8_t*)*((nsx_cu64*)ptrs + e);
}

// tile `tile` of expert e's t64 matrix: from the tile table when there is one
// (tiles may then sit anywhere the device can read, pinned host memory
// included), else at its offset in the expert
__device__ __forceinline__ const uint8_t* tile_base(const void* base, int64_t stride, const uint64_t* ptrs,
                                                    const uint64_t* tiles, const MxGeom& G, int e, int tile) {
  if (tiles) return (const uint8_t*)*((nsx_cu64*)tiles + (int64_t)e * G.tiles + tile);
  return expert_base(base, stride, ptrs, e) + (int64_t)tile * G.tile_bytes;
}

constexpr int GU_S = 3;         // K-steps per gate/up wave (one chunk)
constexpr int DC_S = 6;         // K-steps per down wave (one chunk, one row group)
constexpr int MAX_CHUNKS = 8;   // gate/up K-chunks (waves per matrix) of a workgroup (K <= 3072)

// Rows of D (after mx_sum_terms) for token column 0 go to dst[row] for rows < n.
__device__ __forceinline__ void mx_store_rows(const v4f (&D)[4], int tile, int n, float* __restrict__ dst) {
  const int lane = __lane_id();
  if ((lane & 15) != 0) return;
  const int r0 = tile * 64 + 4 * (lane >> 4);
#pragma unroll
  for (int g = 0; g < 4; ++g)
    if (r0 + 16 * g < n) *(v4f*)(dst + r0 + 16 * g) = D[g];
}

// gate/up of one (pair, 64-row tile) work item, by a whole workgroup: one
// wave per (gate|up, K-chunk), each a single pass over its chunk's steps. The
// waves meet in LDS (fixed order); wave 0 adds the biases, applies the
// activation and writes the activation's terms for the down phase -- the
// tile's 64 rows are exactly two 32-element blocks of the down matrix's K.
__device__ __forceinline__ void gu_item(const MoeDev& a, int p, int tile, float (&red)[2][MAX_CHUNKS][64],
                                        int& s_e) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int m = wave / a.cg, c = wave - m * a.cg;
  const int s0 = c * a.sg, s1 = min(a.ggu.ns, s0 + a.sg);
  const int k = a.top_k, t = p / k, j = p - t * k;
  MxRegs<GU_S> R;
  // the top-k by wave 0 alone (sixteen waves selecting at once would share each SIMD four ways);
  // the token's first item also writes the ids/weights outputs, which the down phase reads. Its
  // logits load is the critical path, so no other load of the CU queues ahead of it: the
  // activation terms (L2 hits after the first workgroups) are requested with the weights, step by
  // step.
  if (wave == 0) {
    int si[MAX_TOPK];
    float sw[MAX_TOPK];
    const bool writes = j == 0 && tile == 0;  // the token's first item writes the ids and weights
    topk_regs(a.logits + (int64_t)t * a.E, a.E, k, a.mode, si, sw, writes, j + 1);
    int my_e = 0, e = 0;
    float my_w = 0.f;
#pragma unroll
    for (int jj = 0; jj < MAX_TOPK; ++jj) {
      e = jj == j ? si[jj] : e;
      my_e = lane == jj ? si[jj] : my_e;
      my_w = lane == jj ? sw[jj] : my_w;
    }
    if (writes && lane < k) {
      a.ids[(int64_t)t * k + lane] = clamp_expert(my_e, a.E);
      a.wts[(int64_t)t * k + lane] = my_w;
    }
    if (lane == 0) s_e = clamp_expert(e, a.E);
  }
  __syncthreads();
  const int e = s_e;
  const uint8_t* mat = m == 0 ? tile_base(a.gate_base, a.gate_stride, a.gate_ptrs, a.gate_tiles, a.ggu, e, tile)
                              : tile_base(a.up_base, a.up_stride, a.up_ptrs, a.up_tiles, a.ggu, e, tile);
  mx_load_ab<GU_S>(R, mat, a.ggu, s0, s1, a.xq_h + (int64_t)t * a.ggu.ns * XQ_STEP, 0, 0, 1);
  const int row = tile * 64 + lane;
  const int rowc = min(row, a.n_ff - 1);
  float gb = 0.f, ub = 0.f;  // wave 0's biases, requested while the weights stream
  if (wave == 0) {
    if (a.gate_bias) gb = a.gate_bias[(int64_t)e * a.n_ff + rowc];
    if (a.up_bias) ub = a.up_bias[(int64_t)e * a.n_ff + rowc];
  }
  v4f D[4] = {};
  mx_compute<GU_S>(R, a.ggu, s0, s1, D);
  mx_sum_terms(D);
  if ((lane & 15) == 0) {  // (one item per workgroup: `red` is not in use yet)
    const int r0 = 4 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 4; ++g) *(v4f*)(&red[m][c][16 * g + r0]) = D[g];
  }
  __syncthreads();
  if (wave != 0) return;
  float gs = 0.f, us = 0.f;
  for (int cc = 0; cc < a.cg; ++cc) {
    gs += red[0][cc][lane];
    us += red[1][cc][lane];
  }
  const float av = row < a.n_ff ? moe_act(a.act_kind, gs + gb, us + ub, a.alpha, a.limit) : 0.f;
  xq_block(av, 2 * tile + (lane >> 5), a.xq_a + (int64_t)p * a.gdn.ns * XQ_STEP);
  xq_zero_tail(tile, a.ggu, a.gdn, a.xq_a + (int64_t)p * a.gdn.ns * XQ_STEP);
}

// the arguments of the per-pair t64 kernels, loaded in one batch
__device__ __forceinline__ void hoist_gu_args(const MoeDev& a) {
  nsx_hoist(a.top_k, a.E, a.mode, (const void*)a.logits, (const void*)a.ids, (const void*)a.wts,
            (const void*)a.xq_h, (const void*)a.xq_a, a.gate_base, a.up_base, (const void*)a.gate_ptrs,
            (const void*)a.up_ptrs, (const void*)a.gate_tiles, (const void*)a.up_tiles, a.gate_stride, a.up_stride,
            (const void*)a.gate_bias, (const void*)a.up_bias,
            a.n_ff, a.cg, a.sg, a.ggu.nb, a.ggu.ns, a.ggu.rlast, a.ggu.tile_bytes, a.ggu.tiles, a.gdn.ns, a.act_kind,
            a.alpha, a.limit);
}
__device__ __forceinline__ void hoist_down_args(const MoeDev& a) {
  nsx_hoist(a.T, a.top_k, a.E, (const void*)a.ids, (const void*)a.wts, a.down_base, (const void*)a.down_ptrs,
            (const void*)a.down_tiles,
            a.down_stride, (const void*)a.down_bias, (const void*)a.xq_a, (const void*)a.out, a.n_embd, a.cd, a.sd,
            a.gdn.nb, a.gdn.ns, a.gdn.rlast, a.gdn.tile_bytes, a.gdn.tiles, (int)gridDim.x);
}

// phase 1 on its own: workgroup = (pair, tile)
__global__ __launch_bounds__(1024) void moe_gu_kernel(MoeDev a) {
  __shared__ float red[2][MAX_CHUNKS][64];
  __shared__ int s_e;
  hoist_gu_args(a);
  const int tiles = (int)a.ggu.tiles;
  const int p = blockIdx.x / tiles;
  gu_item(a, p, blockIdx.x - p * tiles, red, s_e);
}

// down and combine of one (token, 16-row group of a 64-row output tile) work
// item, by a whole workgroup: one wave per (expert slot, K-chunk), each a
// single pass over its steps. down_begin stages the wave's activation terms
// in LDS (they do not depend on the expert, so their loads go first), reads
// the token's ids and weights (written by the gate/up phase) and requests the
// weights and biases; down_end runs the MFMAs and, in wave 0, sums each
// expert's chunks in a fixed order (chunk 0 carries the bias) and combines
// the experts in ascending id: out[rows] = sum of w_e * y_e.
constexpr int DC_PIECES = DC_S * XQ_STEP / 16;  // 16-byte pieces of one wave's activation terms
constexpr int DC_STAGE = (DC_PIECES + 63) / 64;  // of them per lane

struct DownItem {
  MxRegs<DC_S, 1> R;
  v4f bias;  // as loaded; used where bias_on
  int item, t, hh, tile, rg, p, s0, s1, id_l;
  float my_w;
  bool bias_on;
};

// Decode chain (T = 1): what the down kernel's lanes need past the combine --
// the residual stream at the lane's row (lane & 15 of the item's 16 rows),
// and for the waves computing the next layer's router shares the next norm
// weight at that row and expert e's router weights over the item's rows.
struct DownChain {
  float x, w;
  float W[16];
};

__device__ __forceinline__ void down_begin(const MoeDev& a, int item, DownItem& d, uint8_t* xs) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int groups = 4 * (int)a.gdn.tiles;
  d.item = item;
  d.t = item / groups;
  d.hh = item - d.t * groups;
  d.tile = d.hh >> 2;
  d.rg = d.hh & 3;
  const int k = a.top_k;
  const int j = wave / a.cd, c = wave - j * a.cd;
  d.p = d.t * k + j;
  d.s0 = c * a.sd;
  d.s1 = min(a.gdn.ns, d.s0 + a.sd);
  // the token's ids and weights, then this wave's activation terms (steps s0 .. s1 - 1), in one round
  // trip; the ids go first, so the weights' addresses wait on them alone (loads retire in issue order)
  const int npc = (d.s1 - d.s0) * (XQ_STEP / 16);
  const uint8_t* xsrc = a.xq_a + ((int64_t)d.p * a.gdn.ns + d.s0) * XQ_STEP;
  const int id_raw = a.ids[(int64_t)d.t * k + min(lane, k - 1)];  // lane jj < k: slot jj
  d.my_w = a.wts[(int64_t)d.t * k + min(lane, k - 1)];
  v4u stage[DC_STAGE];
#pragma unroll
  for (int i = 0; i < DC_STAGE; ++i) stage[i] = *(gv4u*)(xsrc + (int64_t)min(lane + 64 * i, npc - 1) * 16);
  d.id_l = clamp_expert(id_raw, a.E);
  const int e = __builtin_amdgcn_readlane(d.id_l, j);
  mx_load_a_flat<DC_S, 1>(d.R, tile_base(a.down_base, a.down_stride, a.down_ptrs, a.down_tiles, a.gdn, e, d.tile),
                          a.gdn, d.s0, d.s1, d.rg);
  const int r0 = d.tile * 64 + 16 * d.rg + 4 * (lane >> 4);
  // chunk 0's bias rows, requested while the weights stream: loaded on every lane (a lane without a bias row
  // reads the activation terms' first bytes) and selected where used -- a load under a branch merges into
  // a copy that waits for it, and for every weight load before it
  d.bias_on = c == 0 && a.down_bias && (lane & 15) == 0 && r0 < a.n_embd;
  d.bias = *(const v4f*)(d.bias_on ? a.down_bias + (int64_t)e * a.n_embd + r0 : (const float*)a.xq_a);
#pragma unroll
  for (int i = 0; i < DC_STAGE; ++i) {  // (clamped duplicates rewrite the same bytes)
    const int pc = min(lane + 64 * i, npc - 1);
    *(v4u*)(xs + pc * 16) = stage[i];
  }
}

template <bool CHAIN = false>
__device__ __forceinline__ void down_end(const MoeDev& a, DownItem& d, float (&red)[16][16], const uint8_t* xs,
                                         const DownChain* ch = nullptr) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int k = a.top_k;
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes land before its reads
  __builtin_amdgcn_wave_barrier();
  mx_load_b<DC_S, true, 1>(d.R, xs, d.s0, 0, 1, d.s0, d.s1);
  v4f D[1] = {};
  mx_compute<DC_S, 1>(d.R, a.gdn, d.s0, d.s1, D, d.rg);
  mx_sum_terms<1>(D);
  if ((lane & 15) == 0) *(v4f*)(&red[wave][4 * (lane >> 4)]) = d.bias_on ? D[0] + d.bias : D[0];
  // chain: waves 1 .. nlg compute the next layer's router shares from this item's rows (each combines them too)
  const int nlg = CHAIN && a.cn_w ? (a.cn_E + 63) >> 6 : 0;
  // wave 0 (and the share waves), while the others finish: the slots in ascending expert id
  // (ties: lower slot) -- lane jj < k's rank, then rank r's slot jx[r] by ballot
  int jx[MAX_TOPK];
  if (wave <= nlg) {
    int my_rank = 0;
#pragma unroll
    for (int jj = 0; jj < MAX_TOPK; ++jj) {
      const int ej = __builtin_amdgcn_readlane(d.id_l, jj < k ? jj : k - 1);
      my_rank += (jj < k && (ej < d.id_l || (ej == d.id_l && jj < lane))) ? 1 : 0;
    }
#pragma unroll
    for (int r = 0; r < MAX_TOPK; ++r) {
      const uint64_t b = __builtin_amdgcn_ballot_w64(lane < k && my_rank == r);
      jx[r] = b ? (int)__builtin_ctzll(b) : 0;
    }
  }
  __syncthreads();
  if (wave > nlg) return;
  const int row = d.tile * 64 + 16 * d.rg + (lane & 15);
  float o = 0.f;
  if (k <= 4 && a.cd == 4) {  // the usual shape (top-4, four K-chunks): every read issued at once
    float v[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) v[r][cc] = red[(r < k ? jx[r] : 0) * 4 + cc][lane & 15];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r >= k) break;
      const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d.my_w), jx[r]));
      float y = 0.f;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) y += v[r][cc];
      o = combine_one(o, w, y);
    }
  } else {
#pragma unroll
    for (int r = 0; r < MAX_TOPK; ++r) {
      if (r >= k) break;
      const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d.my_w), jx[r]));
      float y = 0.f;
      for (int cc = 0; cc < a.cd; ++cc) y += red[jx[r] * a.cd + cc][lane & 15];
      o = combine_one(o, w, y);
    }
  }
  if (wave == 0 && lane < 16 && row < a.n_embd) a.out[(int64_t)d.t * a.n_embd + row] = o;
  if constexpr (CHAIN) {
    // x + out, the residual add of gpt_oss.py:177 (the bits of x + r in add_rmsnorm_kernel), in place; and the
    // next block's router shares over these rows: sum of x^2, and sum of (x * w) * W[e] per expert, rows in order
    const bool live = row < a.n_embd;
    const float xn = ch->x + o;
    if (wave == 0) {
      if (lane < 16 && live) a.cx[(int64_t)d.t * a.n_embd + row] = xn;
      if (a.cn_w) {
        const float q = nsx_wave_sum(lane < 16 && live ? xn * xn : 0.f);
        if (lane == 0) a.cp_out[(int64_t)a.cp_groups * a.cn_E + d.item] = q;
      }
    } else {
      const float xw = live ? (a.cn_norm_w ? xn * ch->w : xn) : 0.f;
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, xw), i)), ch->W[i], acc);
      const int e = 64 * (wave - 1) + lane;
      if (e < a.cn_E) a.cp_out[(int64_t)d.item * a.cn_E + e] = acc;
    }
  }
}

// phase 2 on its own: XCD-aware order -- workgroup b runs on XCD b % 8, so
// item = (b % 8) * per + b / 8 keeps the four row groups of a tile (which read
// the same scale lines) on one L2
__global__ __launch_bounds__(1024) void moe_down_kernel(MoeDev a) {
  __shared__ float red[16][16];  // [wave = slot * cd + chunk][row of the group]
  __shared__ __align__(16) uint8_t xs[16][DC_S * XQ_STEP];  // each wave's activation terms, staged
  hoist_down_args(a);
  const int per = (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (item >= a.T * 4 * (int)a.gdn.tiles) return;  // padding workgroups of the 8-way split
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  DownItem d;
  down_begin(a, item, d, xs[wave]);
  down_end(a, d, red, xs[wave]);
}

// ---------------------------------------------------------------------------
// Stacked layers at decode (T = 1) without a router launch after the first
// layer: model/gpt_oss.py:123-177 layer after layer, x = x + moe(rms_norm(x)
// * w), with the router (gpt_oss.py:116-121) regrouped across the kernel
// boundary. The down kernel of layer l, besides its rows of out, adds them to
// the residual stream in place and writes, per work item (16 rows of the
// token), its share of layer l + 1's router: the partial dot of x * w_{l+1}
// over those rows with each expert's router row, and their partial sum of
// squares. Layer l + 1's gate/up kernel adds the shares in a fixed order --
// every workgroup the same way, so all of them select the same top-k -- and
// forms logits = (sum of the dot shares) / rms + bias, which is h . W^T + b
// for h = rms_norm(x) * w with the 1 / rms factored out of the dot; each
// workgroup quantizes h = (x / rms) * w (add_rmsnorm_kernel's formula) into
// LDS for its own MFMAs. Only the rms's summation order differs from the
// separate norm, so results match it to rounding, not bit for bit.

constexpr int CH_MAX_NS = 24;    // K-steps of h one gate/up workgroup holds in LDS (n_embd <= 3072)
constexpr int CH_XQ_PASSES = 4;  // h blocks per lane half: 15 waves x 2 halves x 4 passes >= 4 * CH_MAX_NS
constexpr int CH_SHARE_UNROLL = 8;  // share loads in flight per thread at once
constexpr int CH_SUB = 32;          // subsets of the items summed apart (at most), then in subset order

// 16 consecutive router weights as floats (dtype known at run time, wave-uniform)
__device__ __forceinline__ void load16_w(const void* W, int wdt, int64_t off, float (&w)[16]) {
  float a[8], b[8];
  if (wdt == NSX_F32) {
    load8_w<NSX_F32>(W, off, a);
    load8_w<NSX_F32>(W, off + 8, b);
  } else if (wdt == NSX_BF16) {
    load8_w<NSX_BF16>(W, off, a);
    load8_w<NSX_BF16>(W, off + 8, b);
  } else {
    load8_w<NSX_F16>(W, off, a);
    load8_w<NSX_F16>(W, off + 8, b);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w[i] = a[i];
    w[8 + i] = b[i];
  }
}

// down + combine (as moe_down_kernel), then the residual add and the next layer's router shares
__global__ __launch_bounds__(1024) void moe_down_chain_kernel(MoeDev a) {
  __shared__ float red[16][16];
  __shared__ __align__(16) uint8_t xs[16][DC_S * XQ_STEP];
  hoist_down_args(a);
  nsx_hoist((const void*)a.cx, (const void*)a.cn_w, (const void*)a.cn_norm_w, (const void*)a.cp_out, a.cn_wdt,
            a.cn_E, a.cp_groups);
  const int per = (int)(gridDim.x >> 3);
  const int item = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (item >= a.T * 4 * (int)a.gdn.tiles) return;  // padding workgroups of the 8-way split
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  DownItem d;
  down_begin(a, item, d, xs[wave]);
  // issued behind the weights (loads retire in order: the MFMAs do not wait for these)
  DownChain ch;
  const int r0 = d.tile * 64 + 16 * d.rg;
  const int row = min(r0 + (lane & 15), a.n_embd - 1);
  ch.x = a.cx[(int64_t)d.t * a.n_embd + row];
  ch.w = (a.cn_norm_w ? a.cn_norm_w : a.cx)[row];  // (no norm weight: unused, read from x)
  const int nlg = a.cn_w ? (a.cn_E + 63) >> 6 : 0;
  if (wave >= 1 && wave <= nlg) {  // router row e over the item's rows (n_embd % 16 == 0: all 16 inside the row,
                                    // or none: a group of the last tile past n_embd)
    const int e = min(64 * (wave - 1) + lane, a.cn_E - 1);
    if (r0 < a.n_embd) {
      load16_w(a.cn_w, a.cn_wdt, (int64_t)e * a.n_embd + r0, ch.W);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) ch.W[i] = 0.f;
    }
  }
  down_end<true>(a, d, red, xs[wave], &ch);
}

// gate/up of one (pair, tile) of a chained layer: the router shares summed in
// a fixed order, the top-k by wave 0 while waves 1.. quantize h into LDS, then
// gu_item's gate/up with the activation terms read from LDS.
__global__ __launch_bounds__(1024) void moe_gu_chain_kernel(MoeDev a) {
  __shared__ float red[2][MAX_CHUNKS][64];
  __shared__ __align__(16) float s_part[4096];  // [subset][E] sums of the dot shares (nsub * E <= 4096, E <= 128)
  __shared__ int s_e;
  __shared__ __align__(16) uint8_t s_xq[CH_MAX_NS * XQ_STEP];
  typedef const __attribute__((address_space(1))) v4f gv4f;
  hoist_gu_args(a);
  nsx_hoist((const void*)a.cx, (const void*)a.cnorm_w, a.ceps, (const void*)a.cp_in, a.cp_groups);
  const int tiles = (int)a.ggu.tiles;
  const int p = blockIdx.x / tiles, tile = blockIdx.x - p * tiles;  // T = 1: pair p is slot p
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = __lane_id();
  const int E = a.E, G = a.cp_groups, K = a.n_embd, nb = K / 32, nblk = 4 * a.ggu.ns;
  // 1. every load of the prologue in one round, with no control flow between them (a branch makes the compiler
  //    wait for every load before it): the items' sums of squares (every wave), x and w at this lane's h
  //    elements, the router bias, then the dot shares -- thread (sub, col) sums 4 experts over items sub,
  //    sub + nsub, ... in order (G <= CH_SHARE_UNROLL * nsub: one load each; indices clamped, extras masked)
  const float* ss_sh = a.cp_in + (int64_t)G * E;
  float ssv[4];  // G <= 256
#pragma unroll
  for (int i = 0; i < 4; ++i) ssv[i] = ss_sh[min(lane + 64 * i, G - 1)];
  float hx[CH_XQ_PASSES], hw[CH_XQ_PASSES];  // waves 1..: block 2 (wave - 1 + 15 i) + (lane >> 5)
#pragma unroll
  for (int i = 0; i < CH_XQ_PASSES; ++i) {
    const int b = 2 * (max(wave - 1, 0) + 15 * i) + (lane >> 5);
    const int c = min(b * 32 + (lane & 31), K - 1);
    hx[i] = a.cx[c];
    hw[i] = a.cnorm_w ? a.cnorm_w[c] : 1.f;
  }
  float rbias[2];  // wave 0: the router bias of experts lane + 64 i (E <= 128)
#pragma unroll
  for (int i = 0; i < 2; ++i) rbias[i] = a.crouter_b ? a.crouter_b[min(lane + 64 * i, E - 1)] : 0.f;
  const int ncol = E >> 2, nsub = min(CH_SUB, 1024 / ncol), col = tid % ncol, sub = tid / ncol;
  const int subc = min(sub, nsub - 1);
  const float* dot_sh = a.cp_in;
  v4f v[CH_SHARE_UNROLL];
#pragma unroll
  for (int i = 0; i < CH_SHARE_UNROLL; ++i)
    v[i] = *(gv4f*)(dot_sh + (int64_t)min(subc + i * nsub, G - 1) * E + 4 * col);
  // 2. the subsets' dot shares meet in LDS; every wave takes 1 / rms from the sums of squares (items in order: the
  //    same bits in every wave)
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CH_SHARE_UNROLL; ++i)
    if (subc + i * nsub < G) acc += v[i];
  if (sub < nsub) *(v4f*)(s_part + sub * E + 4 * col) = acc;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += lane + 64 * i < G ? ssv[i] : 0.f;
  ss = nsx_wave_sum(ss);
  const float inv = 1.f / sqrtf(ss / (float)K + a.ceps);
  __syncthreads();
  // 3. wave 0: each lane the logits of experts lane + 64 i (the subsets' sums in order, / rms, + bias), then the
  //    top-k from registers (the token's first item writes the ids and weights); meanwhile waves 1..15 put h's
  //    activation terms into LDS (two blocks a pass: h = (x / rms) * w, add_rmsnorm_kernel's formula) -- before
  //    any weight load goes out, since a wave's loads stall at issue once HBM is saturated
  const int k = a.top_k, j = p;
  if (wave != 0) {
#pragma unroll
    for (int i = 0; i < CH_XQ_PASSES; ++i) {
      const int b0 = 2 * (wave - 1 + 15 * i);  // wave-uniform: both halves' blocks b0, b0 + 1 are < nblk or not
      if (b0 < nblk) {
        const int b = b0 + (lane >> 5);
        xq_block(b < nb ? (hx[i] * inv) * hw[i] : 0.f, b, s_xq);  // (a unit weight multiplies exactly)
      }
    }
  } else {
    float lv[2];  // E <= 128
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ee = min(lane + 64 * i, E - 1);
      float sv[CH_SUB];  // every read at once (unpredicated: subsets past nsub read subset 0, then drop out)
#pragma unroll
      for (int sb = 0; sb < CH_SUB; ++sb) sv[sb] = s_part[(sb < nsub ? sb : 0) * E + ee];
      float l = 0.f;
#pragma unroll
      for (int sb = 0; sb < CH_SUB; ++sb) l += sb < nsub ? sv[sb] : 0.f;
      lv[i] = l * inv + rbias[i];
    }
    int si[MAX_TOPK];
    float sw[MAX_TOPK];
    const bool writes = j == 0 && tile == 0;
    topk_select<2>(lv, E, k, a.mode, si, sw, writes, j + 1);
    int my_e = 0, e = 0;
    float my_w = 0.f;
#pragma unroll
    for (int jj = 0; jj < MAX_TOPK; ++jj) {
      e = jj == j ? si[jj] : e;
      my_e = lane == jj ? si[jj] : my_e;
      my_w = lane == jj ? sw[jj] : my_w;
    }
    if (writes && lane < k) {
      a.ids[lane] = clamp_expert(my_e, E);
      a.wts[lane] = my_w;
    }
    if (lane == 0) s_e = clamp_expert(e, E);
  }
  __syncthreads();
  // 4. gu_item's gate/up: the weights' loads with no control flow between the steps, the activation terms from LDS
  const int e = s_e;
  const bool on = wave < 2 * a.cg;  // (waves past the gate/up chunks load a chunk too, and drop it)
  const int m = on ? wave / a.cg : 0, c = on ? wave - m * a.cg : 0;
  const int s0 = c * a.sg, s1 = min(a.ggu.ns, s0 + a.sg);
  const int row = tile * 64 + lane;
  const int rowc = min(row, a.n_ff - 1);
  MxRegs<GU_S> R;
  const uint8_t* mat = m == 0 ? tile_base(a.gate_base, a.gate_stride, a.gate_ptrs, a.gate_tiles, a.ggu, e, tile)
                              : tile_base(a.up_base, a.up_stride, a.up_ptrs, a.up_tiles, a.ggu, e, tile);
  mx_load_a_flat<GU_S>(R, mat, a.ggu, s0, s1);
  float gb = 0.f, ub = 0.f;
  if (wave == 0) {  // the biases, requested behind the weights
    if (a.gate_bias) gb = a.gate_bias[(int64_t)e * a.n_ff + rowc];
    if (a.up_bias) ub = a.up_bias[(int64_t)e * a.n_ff + rowc];
  }
  v4f D[4] = {};
  if (on) {
    mx_load_b<GU_S, true>(R, s_xq, 0, 0, 1, s0, s1);
    mx_compute<GU_S>(R, a.ggu, s0, s1, D);
    mx_sum_terms(D);
    if ((lane & 15) == 0) {
      const int r0 = 4 * (lane >> 4);
#pragma unroll
      for (int g = 0; g < 4; ++g) *(v4f*)(&red[m][c][16 * g + r0]) = D[g];
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float gs = 0.f, us = 0.f;
  for (int cc = 0; cc < a.cg; ++cc) {
    gs += red[0][cc][lane];
    us += red[1][cc][lane];
  }
  const float av = row < a.n_ff ? moe_act(a.act_kind, gs + gb, us + ub, a.alpha, a.limit) : 0.f;
  xq_block(av, 2 * tile + (lane >> 5), a.xq_a + (int64_t)p * a.gdn.ns * XQ_STEP);
  xq_zero_tail(tile, a.ggu, a.gdn, a.xq_a + (int64_t)p * a.gdn.ns * XQ_STEP);
}

// ---------------------------------------------------------------------------
// grouped dispatch (several tokens): the (token, expert) pairs are sorted by
// expert; a work item is up to GRP_TPI tokens of one expert, and a workgroup
// is (item, 64-row tile), so an expert's tile is requested once per item
// rather than once per pair, and the items of one tile run side by side on
// one XCD, so HBM serves it once (grp_unit). Each token's columns are computed exactly as the
// per-pair kernels compute them (same K-chunks, same summation order), and
// the combine adds the experts in ascending id: the outputs do not depend on
// the dispatch.

constexpr int GRP_TPI = 16;          // tokens per work item
constexpr int GRP_GU_T = 64;         // tokens per MXFP4 gate/up work item (GRP_TPI at a time)
// the grouped MXFP4 down runs persistent (moe_down_persistent_kernel) when its units can number this many times
// the resident workgroups (the 36-layer GPT-OSS stack at T = 8, at most 1485 units on 512 workgroups: 23.7 us per
// layer one workgroup per unit, 25.8 persistent; config 3, T = 128: 89.7 -> 84.5 us persistent)
constexpr int GRP_DN_PERSIST = 8;
constexpr int GRP_MAX_PAIRS = 4096;  // pairs per sort (nsx_moe_forward splits larger T)
constexpr int GRP_CHUNKS = GRP_MAX_PAIRS / 64;

__host__ __device__ __forceinline__ int grp_max_items(int E, int P, int tpi = GRP_TPI) {
  return (E < P ? E : P) + (P + tpi - 1) / tpi;
}

// Item q of expert e, whose cnt pairs start at sorted position bc: (e, first
// sorted position, tokens, q | cnt << 16). The last word lets a unit index
// find any item of the expert from the record of one of them (grp_unit).
__device__ __forceinline__ int4 grp_item(int e, int bc, int cnt, int q) {
  return make_int4(e, bc + q * GRP_TPI, min(GRP_TPI, cnt - q * GRP_TPI), q | (cnt << 16));
}

// Unit L of a dispatch whose items have `units` units each, given rec = the
// record of item s = L / units. An expert of m items owns the units
// [f * units, (f + m) * units), f its first item; they run tile-major -- unit
// u of the range is unit u / m of item f + u % m -- so the m items that need
// one weight tile are adjacent on one XCD and share its fetch in L2 (item-major,
// the XCD streams the expert's other tiles in between and each item re-reads
// it from HBM). Returns the item; `unit` gets its unit.
__device__ __forceinline__ int4 grp_unit(int4 rec, int s, int L, int units, int& unit) {
  const int q = rec.w & 0xffff, cnt = rec.w >> 16, m = (cnt + GRP_TPI - 1) / GRP_TPI;
  const int u = L - (s - q) * units;
  unit = u / m;
  const int qq = u - unit * m;
  return make_int4(rec.x, rec.y + (qq - q) * GRP_TPI, min(GRP_TPI, cnt - qq * GRP_TPI), 0);
}

// Relative time of a gate/up unit of z tokens, m = ceil(z / GRP_TPI) passes,
// fitted to per-unit timestamps of config 3 (T = 128): about 3.8 + 0.31 z +
// 2.6 m us. A pass past the first is not hidden under the next unit's weight
// stream, so a unit of 64 tokens costs about four of one token.
__host__ __device__ __forceinline__ int grp_gu_cost(int z) { return 12 + z + 8 * ((z + GRP_TPI - 1) / GRP_TPI); }
// The same for a down unit (half the weight bytes of a gate/up unit; a token's
// activation terms, 4.5 bytes per element, outweigh them): per-unit stamps of
// config 3 fit about 7.3 + 0.51 z - 2.3 m us (a pass past the first costs less
// per token), and of the forms 10 + z + 3m, 12 + z, 14 + z - 4m, 18 + z - 6m and
// 22 + z - 9m the third gave the shortest step (0.5 us below the first; the last
// two put too much on the XCD of the heavy items)
__host__ __device__ __forceinline__ int grp_dn_cost(int z) { return 14 + z - 4 * ((z + GRP_TPI - 1) / GRP_TPI); }

// lanes of this wave whose (valid) expert equals this lane's
__device__ __forceinline__ uint64_t grp_match(bool valid, int e) {
  uint64_t m = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(valid && bit);
    m &= bit ? bal : ~bal;
  }
  return valid ? m : 0ull;
}

// One workgroup, after the router phase's top-k: a stable counting sort of
// the pairs by expert (64-pair chunks, per-chunk counts, prefix over chunks),
// the work items and the per-token combine order.
__global__ __launch_bounds__(1024) void moe_sort_kernel(MoeDev a) {
  __shared__ uint16_t s_run[GRP_CHUNKS][MAX_EXPERTS];  // chunk counts, then exclusive prefix over chunks
  __shared__ int s_cnt[MAX_EXPERTS], s_off[MAX_EXPERTS];
  __shared__ int s_pc[2][MAX_EXPERTS + GRP_MAX_PAIRS / GRP_GU_T + 1];  // cost prefixes of the gate/up items: gate/up, down
  __shared__ uint8_t s_exp[GRP_MAX_PAIRS];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = __lane_id();
  const int T = a.T, k = a.top_k, E = a.E, P = T * k;
  const int nch = (P + 63) / 64;
  for (int i = tid; i < GRP_CHUNKS * MAX_EXPERTS; i += 1024) (&s_run[0][0])[i] = 0;
  if (a.topk_in_sort) {  // (T < 16: a wave per token) the top-k from the router's logits, as topk_kernel
    for (int t = wave; t < T; t += 16) {
      int si[MAX_TOPK];
      float sw[MAX_TOPK];
      topk_regs(a.logits + (int64_t)t * E, E, k, a.mode, si, sw);
      int my_e = 0;
      float my_w = 0.f;
#pragma unroll
      for (int jj = 0; jj < MAX_TOPK; ++jj) {  // lane jj < k: slot jj
        my_e = lane == jj ? si[jj] : my_e;
        my_w = lane == jj ? sw[jj] : my_w;
      }
      if (lane < k) {
        a.ids[(int64_t)t * k + lane] = my_e;
        a.wts[(int64_t)t * k + lane] = my_w;
        s_exp[t * k + lane] = (uint8_t)clamp_expert(my_e, E);
      }
    }
    __syncthreads();
  }
  // each pair's expert (one round of loads) into LDS, then its token's combine slot from there
  int pe[(GRP_MAX_PAIRS + 1023) / 1024], idv[(GRP_MAX_PAIRS + 1023) / 1024];
#pragma unroll
  for (int i = 0; i < (GRP_MAX_PAIRS + 1023) / 1024; ++i)  // every id load at once (clamped, unpredicated: under
    idv[i] = a.ids[min(tid + 1024 * i, P - 1)];             // the branches below each would be a round trip)
#pragma unroll
  for (int i = 0; i < (GRP_MAX_PAIRS + 1023) / 1024; ++i) {
    const int p = tid + 1024 * i;
    pe[i] = p < P ? (a.topk_in_sort ? (int)s_exp[p] : clamp_expert(idv[i], E)) : 0;
  }
  __syncthreads();  // (every read of s_exp above is done before it is written)
#pragma unroll
  for (int i = 0; i < (GRP_MAX_PAIRS + 1023) / 1024; ++i)
    if (tid + 1024 * i < P) s_exp[tid + 1024 * i] = (uint8_t)pe[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < (GRP_MAX_PAIRS + 1023) / 1024; ++i) {
    const int p = tid + 1024 * i;
    if (p >= P) break;
    const int t = p / k, j = p - t * k;
    const int e = pe[i];
    int rank = 0;
    for (int jj = 0; jj < k; ++jj) {
      const int ej = s_exp[t * k + jj];
      rank += (ej < e || (ej == e && jj < j)) ? 1 : 0;
    }
    a.corder[t * k + rank] = p;
  }
  for (int c = wave; c < nch; c += 16) {  // per-chunk counts (one lane per expert present writes)
    const int p = c * 64 + lane;
    const int e = p < P ? s_exp[p] : 0;
    const uint64_t m = grp_match(p < P, e);
    if (p < P && (m & ((1ull << lane) - 1ull)) == 0ull) s_run[c][e] = (uint16_t)__popcll(m);
  }
  __syncthreads();
  for (int e = tid; e < E; e += 1024) {
    int run = 0;
    for (int c = 0; c < nch; ++c) {
      const int v = s_run[c][e];
      s_run[c][e] = (uint16_t)run;
      run += v;
    }
    s_cnt[e] = run;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scans over experts (4 per lane) of the pair and item counts, and the gate/up items
    constexpr int EPL = MAX_EXPERTS / 64;
    const int tiles = (int)a.ggu.tiles;
    int cn[EPL], ni[EPL];
    int sc = 0, sn = 0;
    // gate/up items heavy first, in four buckets by passes (GRP_TPI tokens each): bucket 3 holds the full items
    // (GRP_GU_T tokens) and the partial ones of more than 3 passes, expert by expert; bucket b < 3 the partial
    // items of b + 1 passes. Per bucket and lane: (gate/up cost << 12) | items, and the down cost.
    int acc[4] = {0, 0, 0, 0}, acd[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      cn[i] = e < E ? s_cnt[e] : 0;
      ni[i] = (cn[i] + GRP_TPI - 1) / GRP_TPI;
      sc += cn[i];
      sn += ni[i];
      const int nf = cn[i] / GRP_GU_T, zr = cn[i] - nf * GRP_GU_T;
      acc[3] += nf * ((grp_gu_cost(GRP_GU_T) << 12) | 1);
      acd[3] += nf * grp_dn_cost(GRP_GU_T);
      if (zr > 0) {
        acc[(zr - 1) / GRP_TPI] += (grp_gu_cost(zr) << 12) | 1;
        acd[(zr - 1) / GRP_TPI] += grp_dn_cost(zr);
      }
    }
    int isc = sc, isn = sn, ia[4] = {acc[0], acc[1], acc[2], acc[3]}, id[4] = {acd[0], acd[1], acd[2], acd[3]};
    for (int d = 1; d < 64; d <<= 1) {
      const int oc = __shfl_up(isc, d, 64), on = __shfl_up(isn, d, 64);
      if (lane >= d) {
        isc += oc;
        isn += on;
      }
    }
    const bool gi = a.gu_items != nullptr;  // (t64 layers only: the MXFP4 grouped kernels' items and XCD runs)
    if (gi) {
      for (int d = 1; d < 64; d <<= 1) {
        int oa[4], od[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          oa[b] = __shfl_up(ia[b], d, 64);
          od[b] = __shfl_up(id[b], d, 64);
        }
        if (lane >= d) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            ia[b] += oa[b];
            id[b] += od[b];
          }
        }
      }
    }
    // bucket bases (items, gate/up cost, down cost): bucket 3 first
    int base_n[4], base_c[4], base_d[4], tn = 0, tc = 0, td = 0;
#pragma unroll
    for (int b = 3; b >= 0; --b) {
      const int tot = __shfl(ia[b], 63, 64), totd = __shfl(id[b], 63, 64);
      base_n[b] = tn + ((ia[b] - acc[b]) & 4095);
      base_c[b] = tc + ((ia[b] - acc[b]) >> 12);
      base_d[b] = td + (id[b] - acd[b]);
      tn += tot & 4095;
      tc += tot >> 12;
      td += totd;
    }
    int bc = isc - sc, bn = isn - sn;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      if (e < E) {
        s_off[e] = bc;
        for (int q = 0; q < ni[i]; ++q) a.items[bn + q] = grp_item(e, bc, cn[i], q);
        const int nf = gi ? cn[i] / GRP_GU_T : 0, zr = gi ? cn[i] - nf * GRP_GU_T : 0;
        const int cf = grp_gu_cost(GRP_GU_T), df = grp_dn_cost(GRP_GU_T);
        for (int q = 0; q < nf; ++q) {
          a.gu_items[base_n[3] + q] = make_int4(e, bc + q * GRP_GU_T, GRP_GU_T, 0);
          s_pc[0][base_n[3] + q] = base_c[3] + q * cf;
          s_pc[1][base_n[3] + q] = base_d[3] + q * df;
        }
        base_n[3] += nf;
        base_c[3] += nf * cf;
        base_d[3] += nf * df;
        if (zr > 0) {
          const int b = (zr - 1) / GRP_TPI;
          a.gu_items[base_n[b]] = make_int4(e, bc + nf * GRP_GU_T, zr, 0);
          s_pc[0][base_n[b]] = base_c[b];
          s_pc[1][base_n[b]] = base_d[b];
          ++base_n[b];
          base_c[b] += grp_gu_cost(zr);
          base_d[b] += grp_dn_cost(zr);
        }
      }
      bc += cn[i];
      bn += ni[i];
    }
    if (gi && lane == 0) {
      s_pc[0][tn] = tc;
      s_pc[1][tn] = td;
    }
    if (lane == 63) *a.n_items = isn;
    // XCD x of kernel g (0: gate/up, 1: down; lane 8 g + x) starts at the first unit whose cost prefix reaches x / 8
    // of the total: unit t of item k (cost prefix P_k, unit cost q_k = P_k+1 - P_k) starts at nt P_k + t q_k for
    // nt units per item. The item is the last one with 8 P_k <= x total, found by bisection over the prefixes
    // (ascending; LDS operations of one wave complete in order).
    if (gi && lane < 16) {
      const int g = lane >> 3, x = lane & 7;
      const int nt = g ? (int)a.gdn.tiles : tiles, tot = g ? td : tc;
      int L = x == 0 || tn == 0 ? 0 : tn * nt;  // (x = 0: 0; an empty sort: 0)
      if (x > 0 && tn > 0) {
        const int tx = x * tot;  // target, in eighths of a cost unit
        int k0 = 0, k1 = tn - 1;  // 8 P_k0 <= tx (P_0 = 0); find the largest such k
        while (k0 < k1) {
          const int m = (k0 + k1 + 1) >> 1;
          if (8 * s_pc[g][m] <= tx) k0 = m; else k1 = m - 1;
        }
        const int P = s_pc[g][k0], q = s_pc[g][k0 + 1] - P;
        const int t = (nt * (tx - 8 * P) + 8 * q - 1) / (8 * q);  // ceil: the first unit of item k0 at or past tx
        L = k0 * nt + min(t, nt);
      }
      (g ? a.dn_bounds : a.gu_bounds)[x] = L;
      if (x == 7) (g ? a.dn_bounds : a.gu_bounds)[8] = tn * nt;
      (g ? a.dn_ctr : a.gu_ctr)[x] = 0;
      if (lane == 15) a.dn_ctr[8] = 0;
    }
  }
  __syncthreads();
  for (int c = wave; c < nch; c += 16) {  // stable scatter
    const int p = c * 64 + lane;
    const int e = p < P ? s_exp[p] : 0;
    const uint64_t m = grp_match(p < P, e);
    if (p < P) a.sorted[s_off[e] + s_run[c][e] + __popcll(m & ((1ull << lane) - 1ull))] = p;
  }
}

// Workgroup index -> (unit, item), where an item has `units` work units
// (its tiles, or tile x row group). Workgroup b runs on XCD b % 8; the
// units x n_items live work units are cut into 8 contiguous runs, one per
// XCD, expert by expert (tile-major within an expert, grp_unit), so that an
// XCD's L2 holds the weight tile and activation terms of the few items it is
// working on while the grid, sized for the most items a sort can make, idles
// evenly on every XCD.
__device__ __forceinline__ bool grp_work(const MoeDev& a, int units, int& unit, int4& item) {
  const int live = units * *a.n_items, per = (live + 7) / 8;
  const int j = (int)(blockIdx.x >> 3);
  if (j >= per) return false;
  const int L = (int)(blockIdx.x & 7) * per + j;
  if (L >= live) return false;
  const int it = L / units;
  item = grp_unit(a.items[it], it, L, units, unit);
  return true;
}

// Pairs up to which the grouped gate/up kernel selects the top-k and sorts
// the pairs itself (one 64-lane chunk), with no sort launch before it.
constexpr int GRP_SMALL_P = 64;
static_assert(GRP_SMALL_P <= GRP_GU_T, "a small sort makes one gate/up item per expert");

// LDS-only workgroup barrier: waits on the wave's LDS operations, not on its
// loads and stores to memory still in flight
__device__ __forceinline__ void grp_lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

// moe_sort_kernel's results for P = T * top_k <= GRP_SMALL_P pairs, computed
// by a workgroup of the gate/up kernel into its LDS: each token's top-k from
// the router's logits (a wave per token, as the sort kernel), then wave 0
// sorts the pairs -- a single chunk, so the chunk prefix of the sort kernel
// is zero and the items, sorted list and combine order are the same values.
// Every workgroup computes them, the gate/up items (s_items, one per expert
// present: at most GRP_SMALL_P <= GRP_GU_T pairs) for itself; the writer also
// stores ids, weights, the gate/up items and the down kernel's XCD runs, the
// GRP_TPI-token items, n_items, sorted and corder for the down and combine
// phases and the caller. Every thread of the workgroup calls it.
__device__ void grp_small_sort(const MoeDev& a, int4* s_items, int* s_sorted, int* s_nitems, uint8_t* s_exp,
                               int* s_cnt, int* s_off, bool writer) {
  const int tid = threadIdx.x, nt = blockDim.x, nw = nt >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = __lane_id();
  const int T = a.T, k = a.top_k, E = a.E, P = T * k;
  for (int e = tid; e < E; e += nt) s_cnt[e] = 0;
  for (int t = wave; t < T; t += nw) {
    int si[MAX_TOPK];
    float sw[MAX_TOPK];
    topk_regs(a.logits + (int64_t)t * E, E, k, a.mode, si, sw);
    int my_e = 0;
    float my_w = 0.f;
#pragma unroll
    for (int jj = 0; jj < MAX_TOPK; ++jj) {  // lane jj < k: slot jj
      my_e = lane == jj ? si[jj] : my_e;
      my_w = lane == jj ? sw[jj] : my_w;
    }
    if (lane < k) {
      s_exp[t * k + lane] = (uint8_t)clamp_expert(my_e, E);
      if (writer) {
        a.ids[(int64_t)t * k + lane] = my_e;
        a.wts[(int64_t)t * k + lane] = my_w;
      }
    }
  }
  grp_lds_barrier();
  if (writer) {
    for (int p = tid; p < P; p += nt) {  // the token's combine order: its slots by (expert, slot)
      const int t = p / k, j = p - t * k, e = s_exp[p];
      int rank = 0;
      for (int jj = 0; jj < k; ++jj) {
        const int ej = s_exp[t * k + jj];
        rank += (ej < e || (ej == e && jj < j)) ? 1 : 0;
      }
      a.corder[t * k + rank] = p;
    }
  }
  const uint64_t below = (1ull << lane) - 1ull;
  const int e_l = lane < P ? s_exp[lane] : 0;  // pair `lane`'s expert
  const uint64_t m = grp_match(lane < P, e_l);
  if (wave == 0 && lane < P && (m & below) == 0ull) s_cnt[e_l] = (int)__popcll(m);
  grp_lds_barrier();
  if (wave == 0) {  // exclusive scans over experts (4 per lane) of the pair, item and expert counts
    int cn[MAX_EXPERTS / 64], ni[MAX_EXPERTS / 64];
    int sc = 0, sn = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < MAX_EXPERTS / 64; ++i) {
      const int e = lane * (MAX_EXPERTS / 64) + i;
      cn[i] = e < E ? s_cnt[e] : 0;
      ni[i] = (cn[i] + GRP_TPI - 1) / GRP_TPI;
      sc += cn[i];
      sn += ni[i];
      sb += cn[i] > 0;
    }
    int isc = sc, isn = sn, isb = sb;
    for (int d = 1; d < 64; d <<= 1) {
      const int oc = __shfl_up(isc, d, 64), on = __shfl_up(isn, d, 64), ob = __shfl_up(isb, d, 64);
      if (lane >= d) {
        isc += oc;
        isn += on;
        isb += ob;
      }
    }
    int bc = isc - sc, bn = isn - sn, bb = isb - sb;
#pragma unroll
    for (int i = 0; i < MAX_EXPERTS / 64; ++i) {
      const int e = lane * (MAX_EXPERTS / 64) + i;
      if (e < E) {
        s_off[e] = bc;
        if (cn[i] > 0) {
          s_items[bb] = make_int4(e, bc, cn[i], 0);
          if (writer) a.gu_items[bb] = s_items[bb];
        }
        if (writer)
          for (int q = 0; q < ni[i]; ++q) a.items[bn + q] = grp_item(e, bc, cn[i], q);
      }
      bc += cn[i];
      bn += ni[i];
      bb += cn[i] > 0;
    }
    if (lane == 63) {
      *s_nitems = isb;
      if (writer) *a.n_items = isn;
    }
    const int live_d = __shfl(isb, 63, 64) * (int)a.gdn.tiles, per_d = (live_d + 7) / 8;
    if (writer && lane <= 8) {  // the down kernel's runs (equal counts) and its counters
      a.dn_bounds[lane] = min(live_d, lane * per_d);
      a.dn_ctr[lane] = 0;
    }
  }
  grp_lds_barrier();
  if (wave == 0 && lane < P) {  // stable scatter
    const int pos = s_off[e_l] + (int)__popcll(m & below);
    s_sorted[pos] = lane;
    if (writer) a.sorted[pos] = lane;
  }
  grp_lds_barrier();
}

// gate/up for (item, tile) units, an item being up to GRP_GU_T tokens of one
// expert: one wave per K-chunk, computing that chunk of both the gate and the
// up tile, so a token's activation terms are read once per (item, tile,
// chunk) rather than once per matrix. A wave's gate (up) chunk is the (gate
// (up), chunk) wave of moe_gu_kernel: same steps, same accumulation order, so
// the activations are bit-identical to the per-pair path. The item's tokens
// go GRP_TPI at a time (one pass through the LDS reduction and epilogue each),
// four at a time inside (16 MFMA columns = 4 tokens x 4 terms), with the
// tile's weights held in registers throughout: HBM serves each tile once per
// item, and the XCD's workgroups, on the tiles of one item together, share its
// tokens' activation terms in L2. Persistent: the launch is the resident
// workgroups, 8 groups of nx (group x on XCD x: workgroup b runs on XCD b %
// 8), and group x works through XCD x's contiguous item-major run of units in
// rounds of nx (the sort lists the items heavy first and cuts the runs by
// grp_gu_cost, so the XCDs finish together), so no workgroup is dispatched per
// unit; the next unit's weights are requested before this unit's last
// epilogue, into the registers its MFMAs have finished with. SIN:
// every workgroup first selects the top-k and sorts the pairs itself
// (grp_small_sort; workgroup 0 stores the results), so small batches launch
// no sort kernel.
template <bool SIN>
__global__ __launch_bounds__(64 * MAX_CHUNKS) void moe_gu_grouped_kernel(MoeDev a) {
  __shared__ float red[2][MAX_CHUNKS][GRP_TPI][64];
  __shared__ int4 s_items[SIN ? GRP_SMALL_P : 1];
  __shared__ int s_sorted[SIN ? GRP_SMALL_P : 1], s_cnt[SIN ? MAX_EXPERTS : 1], s_off[SIN ? MAX_EXPERTS : 1];
  __shared__ int s_nitems, s_next;
  __shared__ uint8_t s_exp[SIN ? GRP_SMALL_P : 1];
  if constexpr (SIN) grp_small_sort(a, s_items, s_sorted, &s_nitems, s_exp, s_cnt, s_off, blockIdx.x == 0);
  auto item_at = [&](int i) { return SIN ? s_items[i] : a.gu_items[i]; };
  auto item_word = [&](int i, int w) {
    return SIN ? ((const int*)s_items)[4 * i + w] : ((const int*)a.gu_items)[4 * i + w];
  };
  auto sorted_at = [&](int i) { return SIN ? s_sorted[i] : a.sorted[i]; };
  const int tiles = (int)a.ggu.tiles;
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), j = (int)(blockIdx.x >> 3);
  // XCD xcd's run of units [lo, hi): cost-weighted bounds from the sort (a small sort: equal counts); round r of
  // the run is units lo + r nx .. + nx - 1, taken in alternating directions, so that a workgroup given a costly
  // unit in one round is given a cheap one in the next. Past round 1 (not for a small sort, which launches no sort
  // kernel to zero the counters), each workgroup takes units from the XCD's counter, one unit ahead: the run's
  // heavy-first units go to whichever workgroups are free first. A workgroup's units ascend (a later take returns
  // more), so it leaves the run at its first unit >= hi with no unit below hi still taken.
  int lo, hi;
  if constexpr (SIN) {
    const int live = tiles * s_nitems, per = (live + 7) / 8;
    lo = min(live, xcd * per);
    hi = min(live, lo + per);
  } else {
    lo = a.gu_bounds[xcd];
    hi = a.gu_bounds[xcd + 1];
  }
  int round = 0;
  int L = lo + j, Ln = lo + nx + (nx - 1 - j);
  if (L >= hi) return;
  const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int s0 = c * a.sg, s1 = min(a.ggu.ns, s0 + a.sg);
  const int64_t xs = (int64_t)a.ggu.ns * XQ_STEP;
  MxRegs<GU_S> Rg, Ru;
  int4 item = item_at(L / tiles);
  int tile = L - (L / tiles) * tiles;
  int e = clamp_expert(item.x, a.E);
  // the pair list goes out ahead of the weights: loads return in order, and the first token group's
  // activation loads wait on it (behind the weights, they would wait for every weight byte)
  int my_pair = sorted_at(item.y + min(lane, item.z - 1));  // lane i: the item's token i
  {  // both tiles' addresses before any load: a pointer-table read between the two load groups would wait on the first
    const uint8_t* gt = tile_base(a.gate_base, a.gate_stride, a.gate_ptrs, a.gate_tiles, a.ggu, e, tile);
    const uint8_t* ut = tile_base(a.up_base, a.up_stride, a.up_ptrs, a.up_tiles, a.ggu, e, tile);
    mx_load_a_flat<GU_S>(Rg, gt, a.ggu, s0, s1);
    mx_load_a_flat<GU_S>(Ru, ut, a.ggu, s0, s1);
  }
  // LDS-only barriers below: a memory-counter wait would hold the epilogue until the next unit's weights land
  auto lds_barrier = []() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
  };
  for (;;) {
    const int z = item.z;
    if (SIN) Ln = lo + (round + 1) * nx + ((round & 1) ? j : nx - 1 - j);
    // the next unit's item, requested now so that it is at hand when this unit's MFMAs are done (the last unit
    // re-reads its own); lane i holds word i & 3 -- a lane-varying load stays in VGPRs, where nothing waits on
    // it before its fields are read after the token loop
    const int iw_n = item_word(min(Ln, hi - 1) / tiles, lane & 3);
    int take = 0;  // the unit after the next one, from the counter (its answer lands with this unit's loads)
    if (!SIN && threadIdx.x == 0) take = atomicAdd(a.gu_ctr + xcd, 1);
    const int row = tile * 64 + lane;
    const int rowc = min(row, a.n_ff - 1);
    // the biases go out with the first token group's activation terms, with no branch before any load (a branch
    // between loads costs a wait on every load before it: here, the unit's weights); a layer without biases
    // reads a word of xq_h in their place. The token loops run at least once and wait on every load they issue,
    // so the biases have landed on every path into an epilogue -- the epilogue after the next unit's loads must
    // not wait on a load (the compiler, unsure of one, would wait on them all)
    const int64_t bo = (int64_t)e * a.n_ff + rowc;
    const float gbv = *(a.gate_bias ? a.gate_bias + bo : (const float*)a.xq_h);
    const float ubv = *(a.up_bias ? a.up_bias + bo : (const float*)a.xq_h);
    const int my_tok = my_pair / a.top_k;  // (after the loads above: it waits on the pair list)
    for (int q0 = 0;; q0 += GRP_TPI) {  // the item's tokens q0 .. q0 + n - 1
      const int n = min(GRP_TPI, z - q0);
      // token groups of 4; the loop runs at least once and waits on every load it issues
      int tg = 0;
      do {
        const int tok = tg * 4 + ((lane & 15) >> 2);
        MxB<GU_S> B;
        mx_load_bb<GU_S>(B, a.xq_h + (int64_t)__shfl(my_tok, q0 + min(tok, n - 1), 64) * xs, 0, s0, s1);
        asm volatile("" ::: "memory");  // all steps' loads go out before the first step's MFMAs wait on one
        mx_take_b(Rg, B);  // the gate and the up tile take the same activation operands
        mx_take_b(Ru, B);
        v4f Dg[4] = {}, Du[4] = {};
        mx_compute<GU_S>(Rg, a.ggu, s0, s1, Dg);
        mx_compute<GU_S>(Ru, a.ggu, s0, s1, Du);
        mx_sum_terms(Dg);
        mx_sum_terms(Du);
        if ((lane & 3) == 0 && tok < n) {
          const int r0 = 4 * (lane >> 4);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            *(v4f*)(&red[0][c][tok][16 * g + r0]) = Dg[g];
            *(v4f*)(&red[1][c][tok][16 * g + r0]) = Du[g];
          }
        }
      } while (++tg * 4 < n);
      // the biases are first used here, after the token loop's waits: an opaque copy, so that the compiler does not
      // hoist their use to the unit's start, where a wait on them is a wait on the weights issued before them
      float gb = gbv, ub = ubv;
      asm volatile("" : "+v"(gb), "+v"(ub));
      gb = a.gate_bias ? gb : 0.f;
      ub = a.up_bias ? ub : 0.f;
      auto epilogue = [&]() {
        if (c >= n) return;
        for (int w = c; w < n; w += a.cg) {  // token q0 + w of the item
          float gs = 0.f, us = 0.f;
          for (int cc = 0; cc < a.cg; ++cc) {
            gs += red[0][cc][w][lane];
            us += red[1][cc][w][lane];
          }
          const float av = row < a.n_ff ? moe_act(a.act_kind, gs + gb, us + ub, a.alpha, a.limit) : 0.f;
          const int pr = __builtin_amdgcn_readlane(my_pair, q0 + w);
          xq_block(av, 2 * tile + (lane >> 5), a.xq_a + (int64_t)pr * a.gdn.ns * XQ_STEP);
          xq_zero_tail(tile, a.ggu, a.gdn, a.xq_a + (int64_t)pr * a.gdn.ns * XQ_STEP);
        }
      };
      const bool more = q0 + GRP_TPI < z;  // more tokens: the weights stay
      if (!more && Ln >= hi) {  // (a path of its own: the weight registers are not live into a merge with reloaded ones)
        lds_barrier();
        epilogue();
        return;
      }
      if (!SIN && !more && threadIdx.x == 0) s_next = take;  // read after the barrier below; rewritten after the next
      int4 item_n;
      int tile_n = 0, e_n = 0, pair_n = 0;
      if (!more) {  // the next unit's weights and pair list go out before this unit's last epilogue
        item_n = int4{__builtin_amdgcn_readlane(iw_n, 0), __builtin_amdgcn_readlane(iw_n, 1),
                      __builtin_amdgcn_readlane(iw_n, 2), 0};
        tile_n = Ln - (Ln / tiles) * tiles;
        e_n = clamp_expert(item_n.x, a.E);
        pair_n = sorted_at(item_n.y + min(lane, item_n.z - 1));  // (ahead of the weights, as above)
        const uint8_t* gt = tile_base(a.gate_base, a.gate_stride, a.gate_ptrs, a.gate_tiles, a.ggu, e_n, tile_n);
        const uint8_t* ut = tile_base(a.up_base, a.up_stride, a.up_ptrs, a.up_tiles, a.ggu, e_n, tile_n);
        mx_load_a_flat<GU_S>(Rg, gt, a.ggu, s0, s1);
        mx_load_a_flat<GU_S>(Ru, ut, a.ggu, s0, s1);
      }
      lds_barrier();
      const int Lnn = SIN || more ? 0 : lo + 2 * nx + __builtin_amdgcn_readfirstlane(s_next);
      epilogue();
      lds_barrier();  // the epilogue's reads of red come before the next tokens' (unit's) writes
      if (more) continue;
      L = Ln;
      if (!SIN) Ln = Lnn;
      ++round;
      item = item_n;
      tile = tile_n;
      e = e_n;
      my_pair = pair_n;
      break;
    }
  }
}

// down for one (item, tile), an item being up to GRP_TPI tokens of one expert
// (the sort's GRP_TPI-token items, tile-major within an expert): one wave per
// K-chunk over all four 16-row
// groups, so each token's activation terms are read once per (item, tile)
// rather than once per row group (they are 4.5 bytes per element and token,
// more than the weights' 0.53 per element and row). A wave's chunk, row group
// by row group, is the (chunk, row group) wave of moe_down_kernel: same steps,
// same accumulation order, so y is bit-identical to the per-pair path.
// y[pair, rows] = the expert's down product plus its bias (chunk 0 carries it).
__global__ __launch_bounds__(256, 2) void moe_down_grouped_kernel(MoeDev a) {
  __shared__ float red[4][GRP_TPI][64];  // [wave = chunk][token][row of the tile]
  int tile;
  int4 item;
  if (!grp_work(a, (int)a.gdn.tiles, tile, item)) return;
  const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int e = clamp_expert(item.x, a.E), pos0 = item.y, n = item.z;
  const int s0 = c * a.sdg, s1 = min(a.gdn.ns, s0 + a.sdg);
  MxRegs<DC_S> R;
  // the pair list goes out ahead of the weights: loads return in order, and the first token group's
  // activation loads wait on it (behind the weights, they would wait for every weight byte)
  const int my_pair = a.sorted[pos0 + min(lane & 15, n - 1)];
  mx_load_a_flat<DC_S>(R, tile_base(a.down_base, a.down_stride, a.down_ptrs, a.down_tiles, a.gdn, e, tile), a.gdn, s0,
                       s1);
  const int r0 = tile * 64 + 4 * (lane >> 4);
  v4f bias[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    bias[g] = v4f{0.f, 0.f, 0.f, 0.f};
    if (c == 0 && a.down_bias && r0 + 16 * g < a.n_embd)
      bias[g] = *(const v4f*)(a.down_bias + (int64_t)e * a.n_embd + r0 + 16 * g);
  }
  const int64_t xs = (int64_t)a.gdn.ns * XQ_STEP;
  for (int tg = 0; tg * 4 < n; ++tg) {
    const int tok = tg * 4 + ((lane & 15) >> 2);
    const int pr = __shfl(my_pair, min(tok, n - 1), 64);
    mx_load_b_at<DC_S, false, 4, true>(R, a.xq_a + (int64_t)pr * xs, 0, s0, s1);
    asm volatile("" ::: "memory");  // all steps' loads go out before the first step's MFMAs wait on one
    v4f D[4] = {};
    mx_compute<DC_S>(R, a.gdn, s0, s1, D);
    mx_sum_terms<4>(D);
    if ((lane & 3) == 0 && tok < n) {
#pragma unroll
      for (int g = 0; g < 4; ++g) *(v4f*)(&red[c][tok][16 * g + 4 * (lane >> 4)]) = D[g] + bias[g];
    }
  }
  __syncthreads();
  const int row = tile * 64 + lane;
  for (int w = c; w < n; w += a.cdg) {  // token w of the item: chunks in order
    float y = 0.f;
    for (int cc = 0; cc < a.cdg; ++cc) y += red[cc][w][lane];
    const int pr = __builtin_amdgcn_readlane(my_pair, w);
    if (row < a.n_embd) a.y[(int64_t)pr * a.n_embd + row] = y;
  }
}

// down for (item, tile) units, an item being up to GRP_GU_T tokens of one
// expert (the gate/up kernel's items): one wave per K-chunk over all four
// 16-row groups, so each token's activation terms are read once per (item,
// tile) rather than once per row group (they are 4.5 bytes per element and
// token, more than the weights' 0.53 per element and row). A wave's chunk, row
// group by row group, is the (chunk, row group) wave of moe_down_kernel: same
// steps, same accumulation order, and the bias joins chunk 0's partial first,
// so y is bit-identical to the per-pair path. The tile's weights stay in
// registers over the item's tokens, GRP_TPI at a time. Persistent as the
// gate/up kernel: 8 groups of nx workgroups, group x on XCD x taking rounds of
// nx units of its run (cost-weighted by the sort), in alternating directions;
// the next unit's weights are requested before this unit's last epilogue.
// y[pair, rows] = the expert's down product plus its bias.
__global__ __launch_bounds__(256, 2) void moe_down_persistent_kernel(MoeDev a) {
  __shared__ float red[4][GRP_TPI][64];  // [wave = chunk][token][row of the tile]
  __shared__ int s_next;
  const int tiles = (int)a.gdn.tiles;
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), j = (int)(blockIdx.x >> 3);
  const int lo = a.dn_bounds[xcd], hi = a.dn_bounds[xcd + 1];
  // a workgroup leaving counts itself out; the last one to leave zeroes the counters for the next launch (no
  // workgroup takes a unit after it has counted itself out, so none is in use then). A down phase may run again
  // without a sort, so the kernel leaves its counters as it found them.
  auto leave = [&]() {
    if (threadIdx.x == 0 && atomicAdd(a.dn_ctr + 8, 1) == (int)gridDim.x - 1) {
      for (int i = 0; i < 9; ++i) atomicExch(a.dn_ctr + i, 0);
    }
  };
  int L = lo + j, Ln = lo + nx + (nx - 1 - j);
  if (L >= hi) {
    leave();
    return;
  }
  const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int s0 = c * a.sdg, s1 = min(a.gdn.ns, s0 + a.sdg);
  const int64_t xs = (int64_t)a.gdn.ns * XQ_STEP;
  MxRegs<DC_S> R;
  int4 item = a.gu_items[L / tiles];
  int tile = L - (L / tiles) * tiles;
  int e = clamp_expert(item.x, a.E);
  // the pair list goes out ahead of the weights: loads return in order, and the first token group's
  // activation loads wait on it (behind the weights, they would wait for every weight byte)
  int my_pair = a.sorted[item.y + min(lane, item.z - 1)];  // lane i: the item's token i
  mx_load_a_flat<DC_S>(R, tile_base(a.down_base, a.down_stride, a.down_ptrs, a.down_tiles, a.gdn, e, tile), a.gdn, s0,
                       s1);
  // LDS-only barriers below: a memory-counter wait would hold the epilogue until the next unit's weights land
  auto lds_barrier = []() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
  };
  for (;;) {
    const int z = item.z;
    // the next unit's item (lane i: word i & 3), requested now so that it is at hand after the token loop
    const int iw_n = ((const int*)a.gu_items)[4 * (min(Ln, hi - 1) / tiles) + (lane & 3)];
    int take = 0;  // the unit after the next one, from the XCD's counter (its answer lands with this unit's loads)
    if (threadIdx.x == 0) take = atomicAdd(a.dn_ctr + xcd, 1);
    const int row = tile * 64 + lane;
    // this lane's bias, with no branch before any load (a layer without biases reads a word of xq_a instead);
    // the token loops run at least once and wait on every load before their last, so it has landed before the
    // epilogue on every path
    const float bv = *(a.down_bias ? a.down_bias + (int64_t)e * a.n_embd + min(row, a.n_embd - 1)
                                   : (const float*)a.xq_a);
    for (int q0 = 0;; q0 += GRP_TPI) {  // the item's tokens q0 .. q0 + n - 1
      const int n = min(GRP_TPI, z - q0);
      int tg = 0;
      do {
        const int tok = tg * 4 + ((lane & 15) >> 2);
        const int pr = __shfl(my_pair, q0 + min(tok, n - 1), 64);
        mx_load_b_at<DC_S, false, 4, true>(R, a.xq_a + (int64_t)pr * xs, 0, s0, s1);
        asm volatile("" ::: "memory");  // all steps' loads go out before the first step's MFMAs wait on one
        v4f D[4] = {};
        mx_compute<DC_S>(R, a.gdn, s0, s1, D);
        mx_sum_terms<4>(D);
        if ((lane & 3) == 0 && tok < n) {
#pragma unroll
          for (int g = 0; g < 4; ++g) *(v4f*)(&red[c][tok][16 * g + 4 * (lane >> 4)]) = D[g];
        }
      } while (++tg * 4 < n);
      // an opaque copy: the compiler does not hoist the bias's first use to the unit's start, where a wait on it
      // is a wait on the weights issued before it
      float b = bv;
      asm volatile("" : "+v"(b));
      b = a.down_bias ? b : 0.f;
      auto epilogue = [&]() {
        for (int w = c; w < n; w += a.cdg) {  // token q0 + w of the item: chunk 0 with the bias, then the others
          float y = red[0][w][lane] + b;
          for (int cc = 1; cc < a.cdg; ++cc) y += red[cc][w][lane];
          const int pr = __builtin_amdgcn_readlane(my_pair, q0 + w);
          if (row < a.n_embd) a.y[(int64_t)pr * a.n_embd + row] = y;
        }
      };
      const bool more = q0 + GRP_TPI < z;  // more tokens: the weights stay
      if (!more && Ln >= hi) {  // (a path of its own: the weight registers are not live into a merge with reloaded ones)
        lds_barrier();
        epilogue();
        leave();
        return;
      }
      if (!more && threadIdx.x == 0) s_next = take;  // read after the barrier below; rewritten after the next
      int4 item_n;
      int tile_n = 0, e_n = 0, pair_n = 0;
      if (!more) {  // the next unit's weights and pair list go out before this unit's last epilogue
        item_n = int4{__builtin_amdgcn_readlane(iw_n, 0), __builtin_amdgcn_readlane(iw_n, 1),
                      __builtin_amdgcn_readlane(iw_n, 2), 0};
        tile_n = Ln - (Ln / tiles) * tiles;
        e_n = clamp_expert(item_n.x, a.E);
        pair_n = a.sorted[item_n.y + min(lane, item_n.z - 1)];  // (ahead of the weights, as above)
        mx_load_a_flat<DC_S>(R, tile_base(a.down_base, a.down_stride, a.down_ptrs, a.down_tiles, a.gdn, e_n, tile_n),
                             a.gdn, s0, s1);
      }
      lds_barrier();
      const int Lnn = more ? 0 : lo + 2 * nx + __builtin_amdgcn_readfirstlane(s_next);
      epilogue();
      lds_barrier();  // the epilogue's reads of red come before the next tokens' (unit's) writes
      if (more) continue;
      L = Ln;
      Ln = Lnn;
      item = item_n;
      tile = tile_n;
      e = e_n;
      my_pair = pair_n;
      break;
    }
  }
}

// out[t, row] = sum over t's pairs in ascending expert id of w * y (grid: rows/256 x T)
template <int KMAX>  // top_k <= KMAX: the token's pair indices in one round of loads, then their weights and rows
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeDev a) {
  const int t = blockIdx.y, row = min((int)(blockIdx.x * 256 + threadIdx.x), a.n_embd - 1), k = a.top_k;
  int pj[KMAX];
  float wj[KMAX], yj[KMAX];
#pragma unroll
  for (int jj = 0; jj < KMAX; ++jj) pj[jj] = a.corder[t * k + min(jj, k - 1)];
#pragma unroll
  for (int jj = 0; jj < KMAX; ++jj) {
    wj[jj] = a.wts[pj[jj]];
    yj[jj] = a.y[(int64_t)pj[jj] * a.n_embd + row];
  }
  float o = 0.f;
#pragma unroll
  for (int jj = 0; jj < KMAX; ++jj)
    if (jj < k) o = combine_one(o, wj[jj], yj[jj]);
  if ((int)(blockIdx.x * 256 + threadIdx.x) < a.n_embd) a.out[(int64_t)t * a.n_embd + row] = o;
}

// The combine fused with the next block's residual add and norm (a stacked
// layer's output goes nowhere else): for token t, o = the combine above, then
// x_out = x + o and h_out = rms_norm(x + o) * w in add_rmsnorm_kernel's layout
// and order -- the bits of moe_combine_kernel followed by that kernel, one
// launch instead of two. One workgroup per token; x_out may be x (each thread
// reads its elements before writing them).
struct AddNorm {
  const float* x;
  const float* w;  // norm weight (null: none)
  float eps;
  float* x_out;
  float* h_out;
};
template <int KMAX>  // top_k <= KMAX
__global__ __launch_bounds__(1024) void moe_combine_norm_kernel(MoeDev a, AddNorm an) {
  __shared__ float part[4];
  __shared__ __align__(16) float s_row[256 * NORM_MAXV];  // x + o of the token
  const int t = blockIdx.x, n = a.n_embd, k = a.top_k, tid = threadIdx.x;
  int pj[KMAX];
  float wj[KMAX];
#pragma unroll
  for (int jj = 0; jj < KMAX; ++jj) {
    pj[jj] = a.corder[t * k + min(jj, k - 1)];
    wj[jj] = a.wts[pj[jj]];
  }
  // x + o over the whole row by all 1024 threads, every load unpredicated and in flight together
  constexpr int EPT = 256 * NORM_MAXV / 1024;
  const float* xr = an.x + (int64_t)t * n;
  float wv[NORM_MAXV];  // the norm weights of the norm threads' elements, requested with the rest
  if (tid < 256) {
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) wv[i] = an.w ? an.w[min(tid + i * 256, n - 1)] : 1.f;
  }
  float yv[EPT][KMAX], xv[EPT];
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int c = min(tid + q * 1024, n - 1);
    xv[q] = xr[c];
#pragma unroll
    for (int jj = 0; jj < KMAX; ++jj) yv[q][jj] = a.y[(int64_t)pj[jj] * n + c];
  }
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    float o = 0.f;  // moe_combine_kernel's sum, in its order
#pragma unroll
    for (int jj = 0; jj < KMAX; ++jj) o = jj < k ? combine_one(o, wj[jj], yv[q][jj]) : o;
    const int c = tid + q * 1024;
    if (c < n) s_row[c] = xv[q] + o;
  }
  __syncthreads();  // every read of x is done before any write below
  // the norm in add_rmsnorm_kernel's layout and order: 256 threads, thread i holding i, i + 256, ...
  float v[NORM_MAXV];
  float ss = 0.f;
  if (tid < 256) {
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) {
      const int c = tid + i * 256;
      v[i] = c < n ? s_row[c] : 0.f;
      ss = fmaf(v[i], v[i], ss);
    }
    ss = nsx_wave_sum(ss);
    if (__lane_id() == 0) part[tid >> 6] = ss;
  }
  __syncthreads();
  if (tid >= 256) return;
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) tot += part[i];
  const float inv = 1.f / sqrtf(tot / (float)n + an.eps);
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    const int c = tid + i * 256;
    if (c < n) {
      an.x_out[(int64_t)t * n + c] = v[i];
      an.h_out[(int64_t)t * n + c] = an.w ? (v[i] * inv) * wv[i] : v[i] * inv;
    }
  }
}

// ---------------------------------------------------------------------------
// Raw GGUF rows (any format), one row per wave: the row's units are fetched
// with range-checked dword buffer loads (any byte alignment) and realigned in
// registers, every load of a wave in flight before its arithmetic.
// gate/up: workgroup = (pair p, RAW_WAVES rows); a wave loads its row of gate
// and of up, the workgroup stages the token's h in LDS meanwhile, then each
// wave adds its units in the order of the former row loop (units lane, lane +
// 64, ...), reduces over the wave and writes act = activation(gate, up).
// down: workgroup = (token t, RAW_WAVES output rows) with the token's k
// activation vectors staged in LDS; a wave loads its row of every routed
// expert (RAW_EB experts at a time) before any arithmetic, then combines the
// experts' results in ascending id.
constexpr int RAW_WAVES = 16;
constexpr int RAW_UPL = 2;  // units per lane in flight (128 units = K of 4096 at a time)

// x rows in LDS as 32-element chunks RAW_XPAD floats apart (row j's chunk c at
// j * (K / 32) * RAW_XPAD + RAW_XPAD * c), so that the lanes' 16-byte reads of
// their own units (lane l, chunk u0 + l) fall on distinct banks; then, for the
// formats whose codes carry an offset, the per-32 sums (row j's at
// nrows * (K / 32) * RAW_XPAD + j * (K / 32)), added in element order. The
// whole workgroup calls it; it ends with a barrier.
constexpr int RAW_XPAD = 36;
__host__ __device__ constexpr int64_t raw_xpad_bytes(int64_t nrows, int64_t K) {
  return nrows * (K / 32) * (RAW_XPAD + 1) * 4;
}
__device__ __forceinline__ void stage_rows_pad(float* __restrict__ xs, const float* __restrict__ src, int nrows,
                                               int K, bool sums) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  const int q4 = K / 4, n4 = nrows * q4, nc = K / 32, nt = (int)blockDim.x;
  for (int i0 = (int)threadIdx.x; i0 < n4; i0 += 4 * nt) {
    v4f v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = *(gv4f*)(src + 4 * min(i0 + q * nt, n4 - 1));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = i0 + q * nt;
      if (i < n4) {
        const int j = i / q4, c4 = i - j * q4;
        *(v4f*)(xs + (j * nc + (c4 >> 3)) * RAW_XPAD + 4 * (c4 & 7)) = v[q];
      }
    }
  }
  __syncthreads();
  if (!sums) return;
  float* xsum = xs + nrows * nc * RAW_XPAD;
  for (int i = (int)threadIdx.x; i < nrows * nc; i += nt) {
    const float* c = xs + i * RAW_XPAD;
    float a = 0.f;
    for (int k = 0; k < 32; ++k) a += c[k];
    xsum[i] = a;
  }
  __syncthreads();
}

// one token's unit, read once into registers (shared by the gate and up rows)
struct RawXArr {
  static constexpr bool kRegSums = false;
  const v4f (&x)[8];
  __device__ __forceinline__ v4f operator()(int, int k4) const { return x[k4]; }
};

// one token's unit u from the padded rows above (row base xr)
template <int FMT>
struct RawXLdsPad {
  static constexpr bool kRegSums = false;
  const float* xr;
  int u;
  __device__ __forceinline__ v4f operator()(int, int k4) const { return *(const v4f*)(xr + RAW_XPAD * u + 4 * k4); }
};
// experts whose row loads are in flight together (down; Q4_K's and Q8_0's 40-48-byte units take two, within
// 128 VGPRs)
template <int FMT>
constexpr int raw_eb() { return FMT == NSX_Q4_K || FMT == NSX_Q8_0 ? 2 : 4; }

// Rows staged through LDS (L16 > 0: formats whose unit fetch realigns any
// byte offset): a wave reads the aligned span holding its row with coalesced
// 16-byte loads, L16 per lane (each instruction 1 KiB of consecutive bytes,
// against ~9 cache lines per dword instruction when every lane loads its own
// 17-byte block), writes them into its own LDS buffer at their offsets from
// the span start (offsets modulo 4 kept), and fetches its units from there.
// A slot past the row repeats its last slot; one that would cross the end of
// the buffer range is moved back to end there (its bytes land at their own
// offsets), so every load is in range.
template <int FMT>
constexpr bool raw_stageable() { return FMT == NSX_MXFP4 || FMT == NSX_Q4_0 || FMT == NSX_Q8_0; }
constexpr int RAW_L16_MAX = 4;  // rows staged up to 64 x 4 slots (4096 bytes)
__host__ __device__ constexpr int raw_slots(uint32_t rb) { return (int)((rb + 3u + 15u) >> 4); }

template <int L16>
__device__ __forceinline__ void raw_row_issue(__amdgpu_buffer_rsrc_t rs, uint32_t s0, uint32_t rend, int n16,
                                              v4u (&V)[L16 > 0 ? L16 : 1], uint32_t (&D)[L16 > 0 ? L16 : 1]) {
  const int lane = __lane_id();
#pragma unroll
  for (int i = 0; i < L16; ++i) {
    const uint32_t sl = (uint32_t)min(lane + 64 * i, n16 - 1);
    const uint32_t off = min(s0 + 16u * sl, rend - 16u);
    V[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    D[i] = off - s0;
  }
}
template <int L16>
__device__ __forceinline__ void raw_row_put(uint8_t* buf, const v4u (&V)[L16 > 0 ? L16 : 1],
                                            const uint32_t (&D)[L16 > 0 ? L16 : 1]) {
#pragma unroll
  for (int i = 0; i < L16; ++i) {  // (4-byte aligned: dword writes)
    uint32_t* w = (uint32_t*)(buf + D[i]);
    w[0] = V[i].x;
    w[1] = V[i].y;
    w[2] = V[i].z;
    w[3] = V[i].w;
  }
}

template <int FMT, int L16>
__global__ __launch_bounds__(64 * RAW_WAVES) void moe_gu_raw_kernel(MoeDev a) {
  extern __shared__ __align__(16) float xs[];  // padded h (stage_rows_pad), then with L16 > 0 two row buffers per wave
  __shared__ int s_e;
  const int groups = (a.n_ff + RAW_WAVES - 1) / RAW_WAVES;
  const int p = blockIdx.x / groups;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int rg0 = blockIdx.x - p * groups;
  const int r = rg0 * RAW_WAVES + wave;
  if (p >= a.T * a.top_k) return;
  const int t = p / a.top_k;
  int e;
  if (a.topk_in_gu) {  // (forward below RM_MIN_T tokens) the pair's expert from the router's logits, as moe_gu_kernel
    if (wave == 0) {
      const int k = a.top_k, j = p - t * k;
      int si[MAX_TOPK];
      float sw[MAX_TOPK];
      const bool writes = j == 0 && rg0 == 0;  // the token's first workgroup writes the ids / weights down reads
      topk_regs(a.logits + (int64_t)t * a.E, a.E, k, a.mode, si, sw, writes, j + 1);
      int my_e = 0, ej = 0;
      float my_w = 0.f;
#pragma unroll
      for (int jj = 0; jj < MAX_TOPK; ++jj) {
        ej = jj == j ? si[jj] : ej;
        my_e = lane == jj ? si[jj] : my_e;
        my_w = lane == jj ? sw[jj] : my_w;
      }
      if (writes && lane < k) {
        a.ids[(int64_t)t * k + lane] = clamp_expert(my_e, a.E);
        a.wts[(int64_t)t * k + lane] = my_w;
      }
      if (lane == 0) s_e = clamp_expert(ej, a.E);
    }
    __syncthreads();
    e = s_e;
  } else {
    e = clamp_expert(a.ids[p], a.E);
  }
  const int K = a.n_embd;
  const uint32_t rb = raw_row_bytes<FMT>(K);
  const uint8_t* gp = expert_base(a.gate_base, a.gate_stride, a.gate_ptrs, e);
  const uint8_t* up = expert_base(a.up_base, a.up_stride, a.up_ptrs, e);
  const uintptr_t ga = (uintptr_t)gp & ~(uintptr_t)3, ua = (uintptr_t)up & ~(uintptr_t)3;
  const uint32_t gh = (uint32_t)((uintptr_t)gp - ga), uh = (uint32_t)((uintptr_t)up - ua);
  const uint32_t gend = (gh + rb * (uint32_t)a.n_ff + 3u) & ~3u, uend = (uh + rb * (uint32_t)a.n_ff + 3u) & ~3u;
  const __amdgpu_buffer_rsrc_t rg = nsx_rsrc((const void*)ga, gend);
  const __amdgpu_buffer_rsrc_t ru = nsx_rsrc((const void*)ua, uend);
  const int nu = raw_units<FMT>(K);
  const uint32_t orow = (uint32_t)min(r, a.n_ff - 1) * rb;
  const bool sums = FMT == NSX_Q4_0 || FMT == NSX_Q4_K;
  const float* xsum = xs + (K / 32) * RAW_XPAD;
  float g[1] = {0.f}, u[1] = {0.f};
  if constexpr (L16 > 0) {
    const int n16 = raw_slots(rb);
    uint8_t* wg = (uint8_t*)xs + raw_xpad_bytes(1, K) + (size_t)wave * 2 * n16 * 16;
    uint8_t* wu = wg + n16 * 16;
    const uint32_t gs = gh + orow, us = uh + orow;
    v4u GV[L16], UV[L16];
    uint32_t GD[L16], UD[L16];
    raw_row_issue<L16>(rg, gs & ~3u, gend, n16, GV, GD);
    raw_row_issue<L16>(ru, us & ~3u, uend, n16, UV, UD);
    stage_rows_pad(xs, a.h + (int64_t)t * K, 1, K, sums);  // the token's h (ends with a barrier)
    raw_row_put<L16>(wg, GV, GD);
    raw_row_put<L16>(wu, UV, UD);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's row bytes are in LDS before its reads
    __builtin_amdgcn_wave_barrier();
    for (int u0 = 0; u0 < nu; u0 += 64) {
      const int uu = u0 + lane;
      if (uu < nu) {
        v4f xv[8];  // the unit's activations, once for both rows
#pragma unroll
        for (int k4 = 0; k4 < 8; ++k4) xv[k4] = RawXLdsPad<FMT>{xs, uu}(0, k4);
        raw_unit_math<FMT, 1>(raw_unit_fetch<FMT>(RawLdsSrc{wg}, gs & 3u, uu), uu, RawXArr{xv},
                              RawXSumLds{xsum, K >> 5, uu}, g);
        raw_unit_math<FMT, 1>(raw_unit_fetch<FMT>(RawLdsSrc{wu}, us & 3u, uu), uu, RawXArr{xv},
                              RawXSumLds{xsum, K >> 5, uu}, u);
      }
    }
  } else {
    for (int u0 = 0; u0 < nu; u0 += 64 * RAW_UPL) {
      RawUnit<FMT> G[RAW_UPL], U[RAW_UPL];
#pragma unroll
      for (int i = 0; i < RAW_UPL; ++i) {  // (units past the row read its last unit again; not added)
        const int uu = min(u0 + lane + 64 * i, nu - 1);
        G[i] = raw_unit_fetch<FMT>(RawBufSrc{rg}, gh + orow, uu);
        U[i] = raw_unit_fetch<FMT>(RawBufSrc{ru}, uh + orow, uu);
      }
      if (u0 == 0)  // the token's h into LDS while the first units stream (ends with a barrier)
        stage_rows_pad(xs, a.h + (int64_t)t * K, 1, K, sums);
#pragma unroll
      for (int i = 0; i < RAW_UPL; ++i) {
        const int uu = u0 + lane + 64 * i;
        if (uu < nu) {
          raw_unit_math<FMT, 1>(G[i], uu, RawXLdsPad<FMT>{xs, uu}, RawXSumLds{xsum, K >> 5, uu}, g);
          raw_unit_math<FMT, 1>(U[i], uu, RawXLdsPad<FMT>{xs, uu}, RawXSumLds{xsum, K >> 5, uu}, u);
        }
      }
    }
  }
  float gv = nsx_wave_sum(g[0]), uv = nsx_wave_sum(u[0]);
  if (lane == 0 && r < a.n_ff) {
    if (a.gate_bias) gv += a.gate_bias[(int64_t)e * a.n_ff + r];
    if (a.up_bias) uv += a.up_bias[(int64_t)e * a.n_ff + r];
    a.act[(int64_t)p * a.n_ff + r] = moe_act(a.act_kind, gv, uv, a.alpha, a.limit);
  }
}

template <int FMT>
__global__ __launch_bounds__(64 * RAW_WAVES) void moe_down_raw_kernel(MoeDev a) {
  extern __shared__ __align__(16) float xs[];  // the token's top_k activation rows, padded (stage_rows_pad)
  const int groups = (a.n_embd + RAW_WAVES - 1) / RAW_WAVES;
  const int t = blockIdx.x / groups;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int r = (blockIdx.x - t * groups) * RAW_WAVES + wave;
  if (t >= a.T) return;
  const int K = a.n_ff, k = a.top_k;
  const int id_l = clamp_expert(a.ids[(int64_t)t * k + min(lane, k - 1)], a.E);  // lane jj < k: slot jj
  int si[MAX_TOPK];
#pragma unroll
  for (int jj = 0; jj < MAX_TOPK; ++jj) si[jj] = __builtin_amdgcn_readlane(id_l, jj < k ? jj : k - 1);
  int order[MAX_TOPK];
  slot_order(si, k, order);
  const uint32_t rb = raw_row_bytes<FMT>(K);
  const int nu = raw_units<FMT>(K), nsb = K / 32;
  const uint32_t orow = (uint32_t)min(r, a.n_embd - 1) * rb;
  constexpr int RAW_EB = raw_eb<FMT>();
  float y[MAX_TOPK];
  for (int b0 = 0; b0 < k; b0 += RAW_EB) {  // RAW_EB experts (ascending id) at a time
    float acc[RAW_EB];
#pragma unroll
    for (int q = 0; q < RAW_EB; ++q) acc[q] = 0.f;
    for (int u0 = 0; u0 < nu; u0 += 64 * RAW_UPL) {
      RawUnit<FMT> R[RAW_EB][RAW_UPL];
#pragma unroll
      for (int q = 0; q < RAW_EB; ++q) {
        const int eq = si[order[min(b0 + q, k - 1)]];
        const uint8_t* dp = expert_base(a.down_base, a.down_stride, a.down_ptrs, eq);
        const uintptr_t da = (uintptr_t)dp & ~(uintptr_t)3;
        const uint32_t dh = (uint32_t)((uintptr_t)dp - da);
        const __amdgpu_buffer_rsrc_t rd = nsx_rsrc((const void*)da, (dh + rb * (uint32_t)a.n_embd + 3u) & ~3u);
#pragma unroll
        for (int i = 0; i < RAW_UPL; ++i)
          R[q][i] = raw_unit_fetch<FMT>(RawBufSrc{rd}, dh + orow, min(u0 + lane + 64 * i, nu - 1));
      }
      if (b0 == 0 && u0 == 0)  // the k activation vectors (and per-32 sums) into LDS while the rows stream
        stage_rows_pad(xs, a.act + (int64_t)t * k * K, k, K, FMT == NSX_Q4_0 || FMT == NSX_Q4_K);
      const float* xsum = xs + k * nsb * RAW_XPAD;
#pragma unroll
      for (int q = 0; q < RAW_EB; ++q) {
        if (b0 + q >= k) break;
        const int j = order[b0 + q];
#pragma unroll
        for (int i = 0; i < RAW_UPL; ++i) {
          const int uu = u0 + lane + 64 * i;
          float one[1] = {acc[q]};
          if (uu < nu)
            raw_unit_math<FMT, 1>(R[q][i], uu, RawXLdsPad<FMT>{xs + j * nsb * RAW_XPAD, uu},
                                  RawXSumLds{xsum + j * nsb, K >> 5, uu}, one);
          acc[q] = one[0];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < RAW_EB; ++q)
      if (b0 + q < k) y[b0 + q] = nsx_wave_sum(acc[q]);
  }
  float o = 0.f;
  for (int jj = 0; jj < k; ++jj) {  // ascending expert id
    const int j = order[jj];
    float v = y[jj];
    if (a.down_bias) v += a.down_bias[(int64_t)si[j] * a.n_embd + min(r, a.n_embd - 1)];
    o = combine_one(o, a.wts[(int64_t)t * k + j], v);
  }
  if (lane == 0 && r < a.n_embd) a.out[(int64_t)t * a.n_embd + r] = o;
}

// ---------------------------------------------------------------------------
// Q4_K experts over raw GGUF rows, on the int8 dot instruction with the
// activations as two int8 terms per element (q4k_a8.h). A row of K elements
// is K/256 super-blocks of 144 B (d, dmin, 12 scale bytes, 128 code bytes;
// compute/quant.py:24-56), so rows and super-blocks are 16-byte aligned.
// Lane q of a row's LPR = q4k_lpr(K) lanes takes block pair q of the row
// (nq = K / 64 pairs; a lane with q >= nq loads pair nq - 1 and adds zero):
// code bytes 32 g .. 32 g + 31 (g = q & 3) of super-block q / 4 and that
// super-block's 16-byte header, three 128-bit loads. A wave covers 64 / LPR
// rows per step, and a row's partial sums meet in a8_group_sum. Every kernel
// below runs this arithmetic per (pair, row), so the per-pair and grouped
// kernels give identical bits.

constexpr int Q4K_KMAX = 4096;   // K of the Q4_K kernels (nq <= 64)
static_assert(Q4K_KMAX <= MQ_TR_MAXK, "mq_terms_row holds a row of K <= MQ_TR_MAXK");
constexpr int Q4K_GU_WAVES = 16;
constexpr int Q4K_GU_STEPS = 3;  // row steps of gate and of up per wave (per-pair kernel)
constexpr int Q4K_GU_AHEAD = 2;  // steps whose loads are in flight before the first compute
constexpr int Q4K_GG_WAVES = 8, Q4K_GG_STEPS = 2;  // grouped kernel (rows held while the tokens go by)
constexpr int Q4K_DN_STEPS = 4;  // row steps per down wave (per-pair kernel, two waves per expert slot)
constexpr int Q4K_DN_AHEAD = 2;  // steps whose loads are in flight before the first compute
constexpr int Q4K_DG_WAVES = 4, Q4K_DG_STEPS = 2;  // grouped down

struct Q4kRow {
  v4u c0, c1, hd;
};

// this lane's block pair q of `row` (rb: bytes per row)
__device__ __forceinline__ void q4k_row_load(const uint8_t* __restrict__ mat, int row, uint32_t rb, int q, Q4kRow& r) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  const uint8_t* sb = mat + (int64_t)row * rb + (q >> 2) * 144;
  // (plain loads: a non-temporal hint on the codes, whose cache lines the
  // header loads also touch, measured 25% slower)
  r.hd = *(gv4u*)sb;  // the four lanes of a super-block share it
  r.c0 = *(gv4u*)(sb + 16 + 32 * (q & 3));
  r.c1 = *(gv4u*)(sb + 32 + 32 * (q & 3));
}

// LDS barrier that leaves the memory counter alone: lgkmcnt(0) (this wave's
// LDS writes have landed), then s_barrier; the memory clobber keeps the
// compiler from moving LDS accesses across it. Row loads stay in flight.
__device__ __forceinline__ void q4k_lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  asm volatile("s_barrier" ::: "memory");
}

// Prologue of a gate/up work item of pair p (rows r0 ..): the token's h as
// activation terms in xs, and the pair's expert -- from the ids, or
// (topk_in_gu) from the top-k of the token's logits by wave 0 (through s_e),
// which in the token's first workgroup also writes the ids / weights the down
// phase reads. The terms are in
// LDS before any row load goes out: a wave's loads can stall at issue once the
// memory system is saturated, and a barrier behind them would keep every wave
// of the workgroup from computing until the last one had issued its last load.
__device__ __forceinline__ int q4k_gu_prologue(const MoeDev& a, int p, int r0, uint8_t* xs, int* s_e) {
  typedef const __attribute__((address_space(1))) v4f gv4f;
  const int K = a.n_embd, nq = K / 64, t = p / a.top_k;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  // loads first: the 8 activations of h of each thread past wave 0 (K <= 8 x 960; wave 0 selects
  // the top-k meanwhile), the pair's expert id (issued together with the top-k's logits load: one
  // round trip)
  const int i8 = min(max((int)threadIdx.x - 64, 0), K / 8 - 1);
  const v4f hlo = *(gv4f*)(a.h + (int64_t)t * K + 8 * i8), hhi = *(gv4f*)(a.h + (int64_t)t * K + 8 * i8 + 4);
  const int e_in = a.topk_in_gu ? 0 : a.ids[p];
  if (a.topk_in_gu && wave == 0) {
    // the top-k from the router's logits by wave 0 (as moe_gu_kernel): the first j + 1 experts,
    // all k (and their weights) in the token's first workgroup, which writes the ids / weights
    const int k = a.top_k, j = p - t * k;
    int si[MAX_TOPK];
    float sw[MAX_TOPK];
    const bool writes = j == 0 && r0 == 0;
    topk_regs(a.logits + (int64_t)t * a.E, a.E, k, a.mode, si, sw, writes, j + 1);
    int my_e = 0, ej = 0;
    float my_w = 0.f;
#pragma unroll
    for (int jj = 0; jj < MAX_TOPK; ++jj) {
      ej = jj == j ? si[jj] : ej;
      my_e = lane == jj ? si[jj] : my_e;
      my_w = lane == jj ? sw[jj] : my_w;
    }
    if (writes && lane < k) {
      a.ids[(int64_t)t * k + lane] = clamp_expert(my_e, a.E);
      a.wts[(int64_t)t * k + lane] = my_w;
    }
    if (lane == 0) *s_e = clamp_expert(ej, a.E);
  }
  if (wave > 0 && (int)threadIdx.x - 64 < K / 8) {  // K / 8 is even: lane pairs stay whole
    const float v[8] = {hlo.x, hlo.y, hlo.z, hlo.w, hhi.x, hhi.y, hhi.z, hhi.w};
    a8_pair16(v, ((int)threadIdx.x - 64) >> 1, nq, xs);
  }
  __syncthreads();
  return a.topk_in_gu ? *s_e : clamp_expert(e_in, a.E);
}

// The rows of a gate/up work item: pair p, expert e, rows r0 .. r0 + RPG - 1
// (wave = Q4K_GU_STEPS steps of 64 / LPR rows of gate and of up), activation
// terms in xs. The item's activations (RPG of them, whole 16-element blocks)
// meet in s_act, and the pair's activation terms for the down phase go out
// from there.
template <int LPR, bool BIAS>
__device__ __forceinline__ void q4k_gu_rows(const MoeDev& a, int p, int r0, int e, const uint8_t* xs,
                                            float* s_act) {
  constexpr int RPG = Q4K_GU_WAVES * Q4K_GU_STEPS * (64 / LPR);
  constexpr int RS = 64 / LPR;
  const int K = a.n_embd, nq = K / 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const uint32_t rb = (uint32_t)(K / 256) * 144u;
  const uint8_t* gm = expert_base(a.gate_base, a.gate_stride, a.gate_ptrs, e);
  const uint8_t* um = expert_base(a.up_base, a.up_stride, a.up_ptrs, e);
  const int q = min(lane % LPR, nq - 1), sub = lane / LPR;
  const bool live = lane % LPR < nq;
  const int rw = r0 + wave * Q4K_GU_STEPS * RS + sub;  // this lane's row at step 0
  Q4kRow G[Q4K_GU_STEPS], U[Q4K_GU_STEPS];
  auto load = [&](int j) {
    const int row = min(rw + j * RS, a.n_ff - 1);
    q4k_row_load(gm, row, rb, q, G[j]);
    q4k_row_load(um, row, rb, q, U[j]);
  };
#pragma unroll
  for (int j = 0; j < Q4K_GU_AHEAD; ++j) load(j);
  // BIAS (a layer with a gate or up bias): the rows' biases, behind the first rows' loads and unpredicated
  // (a missing one reads the logits' first float, not used) -- a load under a branch, inside the loop or
  // merging into it, waits for every row load before it
  float gbv[Q4K_GU_STEPS], ubv[Q4K_GU_STEPS];
  if constexpr (BIAS) {
#pragma unroll
    for (int j = 0; j < Q4K_GU_STEPS; ++j) {
      const int64_t o = (int64_t)e * a.n_ff + min(rw + j * RS, a.n_ff - 1);
      gbv[j] = *(a.gate_bias ? a.gate_bias + o : a.logits);
      ubv[j] = *(a.up_bias ? a.up_bias + o : a.logits);
    }
  }
  A8Pair X;
  a8_load(xs, q, nq, X);
#pragma unroll
  for (int j = 0; j < Q4K_GU_STEPS; ++j) {
    if (j > 0 && j + Q4K_GU_AHEAD - 1 < Q4K_GU_STEPS) {
      // the next step's loads go out once this wave has computed a step: a wave whose loads
      // stall at issue still computes what has arrived (the clobber keeps them here)
      asm volatile("" ::: "memory");
      load(j + Q4K_GU_AHEAD - 1);
    }
    float gs = q4k_a8_dot(G[j].c0, G[j].c1, G[j].hd, q & 3, X);
    float us = q4k_a8_dot(U[j].c0, U[j].c1, U[j].hd, q & 3, X);
    gs = a8_group_sum<LPR>(live ? gs : 0.f);
    us = a8_group_sum<LPR>(live ? us : 0.f);
    const int row = rw + j * RS;
    if (lane % LPR == 0 && row < a.n_ff) {
      if constexpr (BIAS) {
        if (a.gate_bias) gs += gbv[j];
        if (a.up_bias) us += ubv[j];
      }
      s_act[row - r0] = moe_act(a.act_kind, gs, us, a.alpha, a.limit);
    }
  }
  __syncthreads();
  // r0 and n_ff are multiples of 16: a lane pair's x-block lies inside or past n_ff as a whole
  const int i8 = threadIdx.x;
  if (i8 < RPG / 8 && r0 + 8 * i8 < a.n_ff) {
    const v4f lo = *(const v4f*)(s_act + 8 * i8), hi = *(const v4f*)(s_act + 8 * i8 + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    a8_pair16(v, (r0 >> 4) + (i8 >> 1), a.n_ff / 64, a.xq_a + (int64_t)p * a8_bytes(a.n_ff));
  }
}

#define Q4K_GU_HOIST(a)                                                                                          \
  nsx_hoist(a.n_ff, a.n_embd, a.top_k, a.E, (const void*)a.ids, (const void*)a.h, a.gate_base, a.up_base,       \
            (const void*)a.gate_ptrs, (const void*)a.up_ptrs, a.gate_stride, a.up_stride, (const void*)a.gate_bias, \
            (const void*)a.up_bias, (const void*)a.act, a.act_kind, a.alpha, a.limit)

// gate/up: workgroup = (pair, RPG rows); it writes the pair's activation terms
// for those rows (the down kernel reads terms, not activations)
template <int LPR, bool BIAS>  // (16 waves: one workgroup per compute unit, VGPRs <= 128)
__global__ __launch_bounds__(1024) void moe_gu_q4k_kernel(MoeDev a) {
  constexpr int RPG = Q4K_GU_WAVES * Q4K_GU_STEPS * (64 / LPR);
  __shared__ __align__(16) uint8_t xs[a8_bytes(Q4K_KMAX)];
  __shared__ __align__(16) float s_act[RPG];
  __shared__ int s_e;
  Q4K_GU_HOIST(a);
  const int groups = (a.n_ff + RPG - 1) / RPG;
  const int p = blockIdx.x / groups, r0 = (blockIdx.x - p * groups) * RPG;
  const int e = q4k_gu_prologue(a, p, r0, xs, &s_e);
  q4k_gu_rows<LPR, BIAS>(a, p, r0, e, xs, s_act);
}

// down and combine: workgroup = (token, RPG output rows), two waves per
// expert slot, each Q4K_DN_STEPS steps of 64 / LPR rows. The workgroup copies
// the activation terms of the token's k pairs into LDS, then issues its row
// loads; the slots' outputs are added in ascending expert id.
constexpr int Q4K_DN_SLICES = (int)((a8_bytes(Q4K_KMAX) / 16 + 127) / 128);  // 16-byte term chunks per thread (k pairs, 128 k threads)

template <int LPR, bool BIAS>
__global__ __launch_bounds__(1024) void moe_down_q4k_kernel(MoeDev a) {
  constexpr int RS = 64 / LPR, RPW = Q4K_DN_STEPS * RS, RPG = 2 * RPW;
  extern __shared__ __align__(16) uint8_t q4k_xa[];  // k vectors of terms
  __shared__ float red[MAX_TOPK][RPG];
  __shared__ int s_slot[MAX_TOPK];
  typedef const __attribute__((address_space(1))) v4f gv4f;
  nsx_hoist(a.n_embd, a.n_ff, a.top_k, a.E, (const void*)a.ids, (const void*)a.wts, (const void*)a.act,
            a.down_base, (const void*)a.down_ptrs, a.down_stride, (const void*)a.down_bias, (const void*)a.out);
  const int groups = (a.n_embd + RPG - 1) / RPG;
  const int t = blockIdx.x / groups, r0 = (blockIdx.x - t * groups) * RPG;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int k = a.top_k, K = a.n_ff, nq = K / 64, slot = wave >> 1;
  // loads first: the token's slot ids, then the activation terms of its k pairs (written by
  // the gate/up kernel, one contiguous run) into LDS
  const int id_l = clamp_expert(a.ids[(int64_t)t * k + min(lane, k - 1)], a.E);  // lane jj < k: slot jj
  {
    const int n16 = k * (int)(a8_bytes(K) / 16);
    const v4u* src = (const v4u*)(a.xq_a + (int64_t)t * k * a8_bytes(K));
    v4u buf[Q4K_DN_SLICES];
#pragma unroll
    for (int i = 0; i < Q4K_DN_SLICES; ++i) {
      const int c = (int)threadIdx.x + i * (int)blockDim.x;
      if (c < n16) buf[i] = src[c];
    }
#pragma unroll
    for (int i = 0; i < Q4K_DN_SLICES; ++i) {
      const int c = (int)threadIdx.x + i * (int)blockDim.x;
      if (c < n16) ((v4u*)q4k_xa)[c] = buf[i];
    }
  }
  const int e = __builtin_amdgcn_readlane(id_l, slot);
  if ((wave & 1) == 0) {  // this slot's rank in ascending expert id (ties: lower slot)
    const uint64_t before = __builtin_amdgcn_ballot_w64(lane < k && (id_l < e || (id_l == e && lane < slot)));
    if (lane == 0) s_slot[__builtin_popcountll(before)] = slot;
  }
  __syncthreads();  // the terms are in LDS before the row loads go out (see the gate/up kernel)
  const uint32_t rb = (uint32_t)(K / 256) * 144u;
  const uint8_t* dm = expert_base(a.down_base, a.down_stride, a.down_ptrs, e);
  const int q = min(lane % LPR, nq - 1), sub = lane / LPR;
  const bool live = lane % LPR < nq;
  const int rw = r0 + (wave & 1) * RPW + sub;
  Q4kRow R[Q4K_DN_STEPS];
#pragma unroll
  for (int j = 0; j < Q4K_DN_AHEAD; ++j) q4k_row_load(dm, min(rw + j * RS, a.n_embd - 1), rb, q, R[j]);
  float bv[Q4K_DN_STEPS];  // BIAS: the rows' biases, as in the gate/up kernel
  if constexpr (BIAS) {
#pragma unroll
    for (int j = 0; j < Q4K_DN_STEPS; ++j) bv[j] = a.down_bias[(int64_t)e * a.n_embd + min(rw + j * RS, a.n_embd - 1)];
  }
  A8Pair X;
  a8_load(q4k_xa + slot * a8_bytes(K), q, nq, X);
#pragma unroll
  for (int j = 0; j < Q4K_DN_STEPS; ++j) {
    if (j > 0 && j + Q4K_DN_AHEAD - 1 < Q4K_DN_STEPS) {  // as in the gate/up kernel
      asm volatile("" ::: "memory");
      const int jn = j + Q4K_DN_AHEAD - 1;
      q4k_row_load(dm, min(rw + jn * RS, a.n_embd - 1), rb, q, R[jn]);
    }
    float y = q4k_a8_dot(R[j].c0, R[j].c1, R[j].hd, q & 3, X);
    y = a8_group_sum<LPR>(live ? y : 0.f);
    const int row = rw + j * RS;
    if (lane % LPR == 0) {
      if constexpr (BIAS) {
        if (row < a.n_embd) y += bv[j];
      }
      red[slot][row - r0] = y;
    }
  }
  __syncthreads();
  if (threadIdx.x >= RPG) return;
  const int row = r0 + (int)threadIdx.x;
  float o = 0.f;
  for (int jj = 0; jj < k; ++jj) {
    const int jx = s_slot[jj];
    o = combine_one(o, a.wts[(int64_t)t * k + jx], red[jx][threadIdx.x]);
  }
  if (row < a.n_embd) a.out[(int64_t)t * a.n_embd + row] = o;
}

// Grouped Q4_K (several tokens per expert): the same per-(pair, row)
// arithmetic as the kernels above, with the rows' codes and headers held in
// registers while the work item's tokens go by one at a time, so an expert's
// rows are read from HBM once per item. The tokens' activation terms
// (a8_terms_kernel) are staged in LDS, Q4K_GROUP_NT tokens at a time, by the
// whole workgroup with one copy: every wave then reads them from LDS rather
// than each making its own dependent L2 round trip per token.

constexpr int Q4K_GROUP_NT = 4;  // tokens whose terms are in LDS at a time

// activation terms of the vectors x[v * K .. v * K + K), one workgroup per vector
__global__ __launch_bounds__(256) void a8_terms_kernel(const float* __restrict__ x, int K, uint8_t* __restrict__ dst) {
  a8_vector(x + (int64_t)blockIdx.x * K, K, dst + (int64_t)blockIdx.x * a8_bytes(K), (int)threadIdx.x, 256);
}

// The terms of tokens w0 .. w0 + nt - 1 of a work item into xs (xp 16-byte
// pieces per token, xps pieces apart in LDS), the token of item position w at
// src(w): all of the workgroup's threads, four pieces each in flight at a time.
template <typename Src>
__device__ __forceinline__ void q4k_stage_terms(uint8_t* __restrict__ xs, int w0, int nt, int xp, Src src,
                                                int xps = 0) {  // xps: LDS pieces per token (>= xp; 0: xp)
  constexpr int B = 4;
  const int tid = (int)threadIdx.x, nthr = (int)blockDim.x, total = nt * xp;
  xps = xps > 0 ? xps : xp;
  for (int c0 = 0; c0 < total; c0 += B * nthr) {
    v4u buf[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {  // (unpredicated: pieces past the end re-read the last one)
      const int c = min(c0 + tid + i * nthr, total - 1);
      const int tk = c / xp;
      buf[i] = *(const v4u*)(src(w0 + tk) + (int64_t)(c - tk * xp) * 16);
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int c = c0 + tid + i * nthr;
      const int tk = c / xp;
      if (c < total) ((v4u*)xs)[tk * xps + (c - tk * xp)] = buf[i];
    }
  }
}

// gate/up: workgroup = (item, RPG rows); wave = Q4K_GG_STEPS steps of 64 / LPR rows of gate and of up
template <int LPR>
__global__ __launch_bounds__(64 * Q4K_GG_WAVES, 4) void moe_gu_q4k_grouped_kernel(MoeDev a) {  // (4 waves per SIMD: two workgroups per CU)
  constexpr int RS = 64 / LPR, RPG = Q4K_GG_WAVES * Q4K_GG_STEPS * RS;
  __shared__ __align__(16) uint8_t xs[Q4K_GROUP_NT * a8_bytes(Q4K_KMAX)];
  int grp;
  int4 item;
  if (!grp_work(a, (a.n_ff + RPG - 1) / RPG, grp, item)) return;
  const int e = clamp_expert(item.x, a.E), pos0 = item.y, n = item.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int K = a.n_embd, nq = K / 64;
  const uint32_t rb = (uint32_t)(K / 256) * 144u;
  // the pair list ahead of the rows: loads return in order, and the staging below waits on it
  const int my_pair = a.sorted[pos0 + min(lane & 15, n - 1)];  // lane i < 16: the item's token i
  const uint8_t* gm = expert_base(a.gate_base, a.gate_stride, a.gate_ptrs, e);
  const uint8_t* um = expert_base(a.up_base, a.up_stride, a.up_ptrs, e);
  const int q = min(lane % LPR, nq - 1), sub = lane / LPR;
  const bool live = lane % LPR < nq;
  const int rw = grp * RPG + wave * Q4K_GG_STEPS * RS + sub;
  Q4kRow G[Q4K_GG_STEPS], U[Q4K_GG_STEPS];
  float gb[Q4K_GG_STEPS], ub[Q4K_GG_STEPS];
#pragma unroll
  for (int j = 0; j < Q4K_GG_STEPS; ++j) {
    const int row = min(rw + j * RS, a.n_ff - 1);
    q4k_row_load(gm, row, rb, q, G[j]);
    q4k_row_load(um, row, rb, q, U[j]);
    gb[j] = a.gate_bias ? a.gate_bias[(int64_t)e * a.n_ff + row] : 0.f;
    ub[j] = a.up_bias ? a.up_bias[(int64_t)e * a.n_ff + row] : 0.f;
  }
  const int64_t xb = a8_bytes(K);
  auto src = [&](int w) { return a.xq_h + (int64_t)(__shfl(my_pair, w, 64) / a.top_k) * xb; };
  for (int w0 = 0; w0 < n; w0 += Q4K_GROUP_NT) {
    const int nt = min(Q4K_GROUP_NT, n - w0);
    if (w0 > 0) __syncthreads();  // every wave is done with the previous tokens' terms
    q4k_stage_terms(xs, w0, nt, (int)(xb / 16), src);
    __syncthreads();
#pragma nounroll
    for (int w = 0; w < nt; ++w) {
      // unpack the codes per token (unpacked codes held across tokens would double
      // their registers): the empty asm marks them as changed
#pragma unroll
      for (int j = 0; j < Q4K_GG_STEPS; ++j)
        asm volatile("" : "+v"(G[j].c0), "+v"(G[j].c1), "+v"(G[j].hd), "+v"(U[j].c0), "+v"(U[j].c1), "+v"(U[j].hd));
      const int pr = __builtin_amdgcn_readlane(my_pair, w0 + w);
      A8Pair X;
      a8_load(xs + w * xb, q, nq, X);
#pragma unroll
      for (int j = 0; j < Q4K_GG_STEPS; ++j) {
        float gs = q4k_a8_dot(G[j].c0, G[j].c1, G[j].hd, q & 3, X);
        float us = q4k_a8_dot(U[j].c0, U[j].c1, U[j].hd, q & 3, X);
        gs = a8_group_sum<LPR>(live ? gs : 0.f);
        us = a8_group_sum<LPR>(live ? us : 0.f);
        const int row = rw + j * RS;
        if (lane % LPR == 0 && row < a.n_ff)
          a.act[(int64_t)pr * a.n_ff + row] = moe_act(a.act_kind, gs + gb[j], us + ub[j], a.alpha, a.limit);
      }
    }
  }
}

// down: workgroup = (item, RPG output rows); y[pair, rows] = the expert's
// down rows . activation(pair) + bias (moe_combine_kernel adds the pairs of a
// token in ascending expert id)
template <int LPR>
__global__ __launch_bounds__(256) void moe_down_q4k_grouped_kernel(MoeDev a) {
  constexpr int RS = 64 / LPR, RPG = Q4K_DG_WAVES * Q4K_DG_STEPS * RS;
  extern __shared__ __align__(16) uint8_t q4k_xg[];  // Q4K_GROUP_NT * a8_bytes(n_ff): sized at launch
  uint8_t* xs = q4k_xg;
  int grp;
  int4 item;
  if (!grp_work(a, (a.n_embd + RPG - 1) / RPG, grp, item)) return;
  const int e = clamp_expert(item.x, a.E), pos0 = item.y, n = item.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int K = a.n_ff, nq = K / 64;
  const uint32_t rb = (uint32_t)(K / 256) * 144u;
  const int my_pair = a.sorted[pos0 + min(lane & 15, n - 1)];  // (ahead of the rows, as in the gate/up kernel)
  const uint8_t* dm = expert_base(a.down_base, a.down_stride, a.down_ptrs, e);
  const int q = min(lane % LPR, nq - 1), sub = lane / LPR;
  const bool live = lane % LPR < nq;
  const int rw = grp * RPG + wave * Q4K_DG_STEPS * RS + sub;
  Q4kRow R[Q4K_DG_STEPS];
  float bias[Q4K_DG_STEPS];
#pragma unroll
  for (int j = 0; j < Q4K_DG_STEPS; ++j) {
    const int row = min(rw + j * RS, a.n_embd - 1);
    q4k_row_load(dm, row, rb, q, R[j]);
    bias[j] = a.down_bias ? a.down_bias[(int64_t)e * a.n_embd + row] : 0.f;
  }
  const int64_t xb = a8_bytes(K);
  auto src = [&](int w) { return a.xq_a + (int64_t)__shfl(my_pair, w, 64) * xb; };
  for (int w0 = 0; w0 < n; w0 += Q4K_GROUP_NT) {
    const int nt = min(Q4K_GROUP_NT, n - w0);
    if (w0 > 0) __syncthreads();
    q4k_stage_terms(xs, w0, nt, (int)(xb / 16), src);
    __syncthreads();
#pragma nounroll
    for (int w = 0; w < nt; ++w) {
#pragma unroll
      for (int j = 0; j < Q4K_DG_STEPS; ++j) asm volatile("" : "+v"(R[j].c0), "+v"(R[j].c1), "+v"(R[j].hd));
      const int pr = __builtin_amdgcn_readlane(my_pair, w0 + w);
      A8Pair X;
      a8_load(xs + w * xb, q, nq, X);
#pragma unroll
      for (int j = 0; j < Q4K_DG_STEPS; ++j) {
        float y = q4k_a8_dot(R[j].c0, R[j].c1, R[j].hd, q & 3, X);
        y = a8_group_sum<LPR>(live ? y : 0.f);
        const int row = rw + j * RS;
        if (lane % LPR == 0 && row < a.n_embd) a.y[(int64_t)pr * a.n_embd + row] = y + bias[j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped Q4_K on the matrix cores (NSX_DISPATCH_MFMA). For an expert's work
// item (up to 16 tokens) a wave computes 16 rows x the item's tokens with
// v_mfma_f32_16x16x32_f16, one 32-element sub-block per instruction:
//   A (16 rows x 32 k) = sc * q: integers <= 945, exact in f16, built from the
//     nibbles as the f16 bit patterns 0x6400 | q (= 1024 + q) and one packed
//     fma (x sc - 1024 sc, exact);
//   B (32 k x 16 tokens) = the activations as two f16 terms (hi + lo) of a
//     copy scaled by a power of two per token (mq_terms_kernel): about 22
//     significant bits per element, every product exact in the fp32 sum;
//   per 256-element super-block: y += d * acc - dmin * acc_min, where acc_min
//     = m (the sub-block mins) x the sub-blocks' activation sums, a second
//     MFMA over k = the super-block's 8 sub-blocks.
// The decode of each weight is shared by the item's tokens (the per-pair
// kernels decode an expert once per routed token) and the products run on
// the matrix cores, so the kernels are bound by the expert bytes.
// Operand layouts (16x16x32 f16): A lane l = row l % 16, k = 8 (l / 16) + v;
// B lane l = column l % 16, same k; D lane l = column l % 16, rows
// 4 (l / 16) + i.

constexpr int MQ_ROWS = 16;  // rows per wave (one MFMA tile)
constexpr int MQ_WG_ROWS = 64;
constexpr int MQ_LDS_NT = 4;  // items of up to this many tokens keep their activation terms in LDS

typedef _Float16 mq_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mq_h2 __attribute__((ext_vector_type(2)));
typedef float mq_f4 __attribute__((ext_vector_type(4)));

// LDS bytes per staged row: whole 1 KB pieces (a direct load's 64 lanes x 16 bytes) and 16 bytes of padding, so
// that consecutive rows do not start in the same bank
__host__ __device__ constexpr int64_t mq_lds_row(int64_t K) { return (mq_row_bytes(K) + 1023) / 1024 * 1024 + 16; }

// The term rows of n tokens (n <= MQ_LDS_NT; row w at src(w), tb bytes, a multiple of 16) into LDS at xs + w * tsb
// by direct loads, each wave instruction one 1 KB piece (lane i: bytes 16 i of it); lanes past the row's end re-read
// its last 16 bytes into the row's padding. The loads write LDS without registers and are counted by vmcnt: a wave
// waits on its own, then the workgroup meets at a barrier.
template <class Src>
__device__ __forceinline__ void mq_stage_lds(uint8_t* xs, int tsb, int n, int tb, Src src) {
  typedef const void __attribute__((address_space(1)))* gptr;
  typedef void __attribute__((address_space(3)))* lptr;
  const int wave = (int)(threadIdx.x >> 6), lane = __lane_id(), nw = (int)(blockDim.x >> 6);
  const int nc = (tb + 1023) >> 10;
  for (int c = wave; c < n * nc; c += nw) {
    const int w = c / nc, k = c - w * nc;
    const int off = min(k * 1024 + lane * 16, tb - 16);
    __builtin_amdgcn_global_load_lds((gptr)(src(w) + off), (lptr)(xs + w * tsb + k * 1024), 16, 0, 0);
  }
}

// One workgroup per row of x (K columns): the row's activation terms (mq_terms_row)
__global__ __launch_bounds__(256) void mq_terms_kernel(const float* __restrict__ x, int K,
                                                       uint8_t* __restrict__ terms) {
  __shared__ float red[4];
  __shared__ float sx[MQ_TR_MAXK];
  mq_terms_row(x + (int64_t)blockIdx.x * K, K, terms + (int64_t)blockIdx.x * mq_row_bytes(K), red, sx);
}

// A operands of one sub-block pair from its 8 code bytes (elements
// 8 g .. 8 g + 7): low nibbles -> sub-block 2j (x sc_lo), high nibbles ->
// sub-block 2j + 1 (x sc_hi). Each code byte b becomes the f16 bit pattern
// 0x64 : b (v_perm against a register of 0x64 bytes) after masking one
// nibble: 1024 + q for the low one; 1024 + 16 q for the high one, left in
// place, so its multiplier is sc / 16 (exact in f16).
// ml = (sc_lo, sc_lo), cl = -1024 ml, mh = (sc_hi / 16, sc_hi / 16), ch = -1024 mh.
__device__ __forceinline__ void mq_a_pair(uint2 q, mq_h2 ml, mq_h2 cl, mq_h2 mh, mq_h2 ch, mq_h8& alo, mq_h8& ahi) {
  const uint32_t w[2] = {q.x, q.y};
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t wl = w[h] & 0x0F0F0F0Fu, wh = w[h] & 0xF0F0F0F0u;
    // selector bytes 0-3 pick the second operand's bytes, 4 the first's (0x64)
    const uint32_t l01 = __builtin_amdgcn_perm(0x64646464u, wl, 0x04010400u);
    const uint32_t l23 = __builtin_amdgcn_perm(0x64646464u, wl, 0x04030402u);
    const uint32_t h01 = __builtin_amdgcn_perm(0x64646464u, wh, 0x04010400u);
    const uint32_t h23 = __builtin_amdgcn_perm(0x64646464u, wh, 0x04030402u);
    lo[2 * h] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(mq_h2, l01), ml, cl));
    lo[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(mq_h2, l23), ml, cl));
    hi[2 * h] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(mq_h2, h01), mh, ch));
    hi[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(mq_h2, h23), mh, ch));
  }
  alo = __builtin_bit_cast(mq_h8, v4u{lo[0], lo[1], lo[2], lo[3]});
  ahi = __builtin_bit_cast(mq_h8, v4u{hi[0], hi[1], hi[2], hi[3]});
}

// The A-operand scale factors of one super-block for lane group g (header H:
// d | dmin, scales[12]): get_scale_min_k4 for all 8 sub-blocks at once, then
// per half u (sub-block pairs g / 2 and 2 + g / 2) the multipliers of the low
// (ml, cl) and high (mh, ch) nibbles, and the scales' min words (MN03, MN47).
struct MqScales {
  mq_h2 ml[2], mh[2], cl[2], ch[2];
  uint32_t MN03, MN47;
};
__device__ __forceinline__ mq_h2 mq_biased(uint32_t w, uint32_t sel) {  // a byte b under 0x64 is the f16 1024 + b
  return __builtin_bit_cast(mq_h2, __builtin_amdgcn_perm(0x64646464u, w, sel));
}
__device__ __forceinline__ MqScales mq_scales(const v4u& H, int g) {
  // scales bytes 0-3 = H.y, 4-7 = H.z, 8-11 = H.w
  const uint32_t SC03 = H.y & 0x3F3F3F3Fu;
  const uint32_t SC47 = (H.w & 0x0F0F0F0Fu) | ((H.y >> 2) & 0x30303030u);
  MqScales S;
  S.MN03 = H.z & 0x3F3F3F3Fu;
  S.MN47 = ((H.w >> 4) & 0x0F0F0F0Fu) | ((H.z >> 2) & 0x30303030u);
  const mq_h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f}, km1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
  const mq_h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f}, km64 = {(_Float16)-64.f, (_Float16)-64.f};
  // lane group g holds half (g & 1) of sub-block pairs g / 2 (QA) and
  // 2 + g / 2 (QB): their scales (pair p = sub-blocks 2p, 2p + 1)
  const uint32_t blo = 2u * (uint32_t)(g >> 1), bhi = blo + 1u;  // bytes of pair g / 2 in SC03, of pair 2 + g / 2 in SC47
  const uint32_t sel_lo = 0x04000400u | (blo << 16) | blo, sel_hi = 0x04000400u | (bhi << 16) | bhi;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t SCW = u == 0 ? SC03 : SC47;
    S.ml[u] = mq_biased(SCW, sel_lo) - k1024;
    S.mh[u] = __builtin_elementwise_fma(mq_biased(SCW, sel_hi), k16, km64);
    S.cl[u] = S.ml[u] * km1024;
    S.ch[u] = S.mh[u] * km1024;
  }
  return S;
}

// code bytes 8t .. 8t + 7 of the lane's 32 (t < 2: QA's, else QB's)
__device__ __forceinline__ uint2 mq_codes(const v4u& QA, const v4u& QB, int t) {
  return t == 0 ? uint2{QA.x, QA.y} : t == 1 ? uint2{QA.z, QA.w} : t == 2 ? uint2{QB.x, QB.y} : uint2{QB.z, QB.w};
}

// the sub-block mins' MFMA (A2 row = the 8 mins at k 0..7, group 0; zero elsewhere) and y += d acc - dmin am
__device__ __forceinline__ void mq_finish(const v4u& H, const MqScales& S, const mq_f4& acc, const mq_h8& SH,
                                          const mq_h8& SL, int g, mq_f4& y) {
  const mq_h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f};
  const uint32_t m01 = __builtin_bit_cast(uint32_t, mq_biased(S.MN03, 0x04010400u) - k1024);
  const uint32_t m23 = __builtin_bit_cast(uint32_t, mq_biased(S.MN03, 0x04030402u) - k1024);
  const uint32_t m45 = __builtin_bit_cast(uint32_t, mq_biased(S.MN47, 0x04010400u) - k1024);
  const uint32_t m67 = __builtin_bit_cast(uint32_t, mq_biased(S.MN47, 0x04030402u) - k1024);
  const mq_h8 A2 = __builtin_bit_cast(mq_h8, g == 0 ? v4u{m01, m23, m45, m67} : v4u{0u, 0u, 0u, 0u});
  mq_f4 am = {0.f, 0.f, 0.f, 0.f};
  am = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2, SH, am, 0, 0, 0);
  am = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2, SL, am, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // d, dmin of row 4 g + i: the header lane (4 g + i) loaded
    const uint32_t dw = (uint32_t)__shfl((int)H.x, 4 * g + i, 64);
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw >> 16));
    y[i] = fmaf(d, acc[i], y[i]);
    y[i] = fmaf(-dmin, am[i], y[i]);
  }
}

// One super-block of one matrix: header H (d | dmin, scales[12]) and the
// lane's code bytes Q[j] (sub-block pair j) -> y (rows 4 g + i, the lane's
// token) += d * (sc q . x) - dmin * (m . xsum).
__device__ __forceinline__ void mq_superblock(const v4u& H, const v4u& QA, const v4u& QB, const mq_h8 (&BH)[8],
                                              const mq_h8 (&BL)[8], const mq_h8& SH, const mq_h8& SL, int g,
                                              mq_f4& y) {
  const MqScales S = mq_scales(H, g);
  mq_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {  // t < 2: QA's bytes 8t .., t >= 2: QB's bytes 8 (t - 2) ..
    const int u = t >> 1;
    mq_h8 alo, ahi;
    mq_a_pair(mq_codes(QA, QB, t), S.ml[u], S.cl[u], S.mh[u], S.ch[u], alo, ahi);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, BH[t], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, BL[t], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, BH[4 + t], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, BL[4 + t], acc, 0, 0, 0);
  }
  mq_finish(H, S, acc, SH, SL, g, y);
}

// The same for two matrices (gate and up, or two row tiles) over activation
// terms in LDS: each quarter t's four term operands are read just before its
// MFMAs (xb: the lane's terms of this super-block, hi at xb, lo at xb + lo_off;
// xs: the super-block's sub-block sums, lo at xs + slo_off), so 16 term
// registers are live rather than 72. Each matrix's MFMAs run in the order of
// mq_superblock: the results are the same bits.
__device__ __forceinline__ void mq_superblock2_lds(const v4u& H0, const v4u& QA0, const v4u& QB0, const v4u& H1,
                                                   const v4u& QA1, const v4u& QB1, const uint8_t* xb, int lo_off,
                                                   const uint8_t* xs, int slo_off, int g, mq_f4& y0, mq_f4& y1) {
  const MqScales S0 = mq_scales(H0, g), S1 = mq_scales(H1, g);
  mq_f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int u = t >> 1;
    const int o = 2 * (128 * (t >> 1) + 8 * (t & 1));  // element offset of s8 = t (hi: + 32 elements)
    const mq_h8 bh = *(const mq_h8*)(xb + o), bl = *(const mq_h8*)(xb + lo_off + o);
    const mq_h8 bh4 = *(const mq_h8*)(xb + o + 64), bl4 = *(const mq_h8*)(xb + lo_off + o + 64);
    mq_h8 alo, ahi;
    mq_a_pair(mq_codes(QA0, QB0, t), S0.ml[u], S0.cl[u], S0.mh[u], S0.ch[u], alo, ahi);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bh, acc0, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bl, acc0, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bh4, acc0, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bl4, acc0, 0, 0, 0);
    mq_a_pair(mq_codes(QA1, QB1, t), S1.ml[u], S1.cl[u], S1.mh[u], S1.ch[u], alo, ahi);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bh, acc1, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bl, acc1, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bh4, acc1, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bl4, acc1, 0, 0, 0);
  }
  const mq_h8 SH = *(const mq_h8*)xs, SL = *(const mq_h8*)(xs + slo_off);
  mq_finish(H0, S0, acc0, SH, SL, g, y0);
  mq_finish(H1, S1, acc1, SH, SL, g, y1);
}

// GU: gate and up rows (n_ff) over h's terms, then the activation into act;
// else: down rows (n_embd) over the pairs' activation terms, plus the bias,
// into y (moe_combine_kernel adds a token's pairs in ascending expert id).
// Workgroup = (item, 64 rows), wave = 16 rows over all of K.
template <bool GU>
__global__ __launch_bounds__(256, GU ? 2 : 3) void moe_q4k_mfma_kernel(MoeDev a) {
  // (waves per SIMD: gate/up's staged rows allow two workgroups per CU, so it takes the registers of two waves per
  // SIMD; down three)
  extern __shared__ __align__(16) uint8_t mq_xs[];  // MQ_LDS_NT * mq_lds_row(K): sized at launch
  const int NR = GU ? a.n_ff : a.n_embd, K = GU ? a.n_embd : a.n_ff;
  int tile;
  int4 item;
  // down: two 16-row tiles per wave (the second in the H1/A1/B1, y1 slots
  // that gate/up uses for the up matrix), so a wave's activation-term loads
  // serve twice the weight bytes
  constexpr int TILES = GU ? 1 : 2;
  if (!grp_work(a, (NR + TILES * MQ_WG_ROWS - 1) / (TILES * MQ_WG_ROWS), tile, item)) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = __lane_id();
  const int lr = lane & 15, g = lane >> 4;
  const int r0 = (tile * MQ_WG_ROWS + wave * MQ_ROWS) * TILES;
  const int e = clamp_expert(item.x, a.E), pos0 = item.y, n = item.z;
  // (a wave past the last row still takes part in the LDS staging and its barrier)
  if (r0 >= NR && n > MQ_LDS_NT) return;
  const int nsb = K / 256;
  const int64_t rb = (int64_t)nsb * 144;
  // weights through buffer loads (an expert matrix: NR rows of rb bytes), so
  // they are tracked by the vector-memory counter alone
  const uint32_t arow_off = (uint32_t)(min(r0 + lr, NR - 1) * rb);
  const uint32_t arow1_off = GU ? arow_off : (uint32_t)(min(r0 + MQ_ROWS + lr, NR - 1) * rb);
  const __amdgpu_buffer_rsrc_t rs0 = nsx_rsrc(expert_base(GU ? a.gate_base : a.down_base, GU ? a.gate_stride : a.down_stride,
                                                          GU ? a.gate_ptrs : a.down_ptrs, e),
                                              (uint32_t)(NR * rb));
  const __amdgpu_buffer_rsrc_t rs1 =
      GU ? nsx_rsrc(expert_base(a.up_base, a.up_stride, a.up_ptrs, e), (uint32_t)(NR * rb)) : rs0;
  // Columns past the item's tokens compute on zero terms (below); their
  // results are never stored, and MFMA columns are independent.
  const bool tv = lr < n;
  const int pr = a.sorted[pos0 + min(lr, n - 1)];
  const int64_t brow = GU ? pr / a.top_k : pr;
  const int64_t tb = mq_row_bytes(K);
  const uint8_t* tbase = GU ? a.xq_h : (const uint8_t*)a.xq_a;
  // terms rows: GU one per token (T), else one per pair (T * top_k)
  const __amdgpu_buffer_rsrc_t rt = nsx_rsrc(tbase, (uint32_t)((int64_t)(GU ? a.T : a.T * a.top_k) * tb));
  // the lane's token row; lane group g takes, in each super-block, elements
  // 64 p + 32 hi + 16 (g & 1) + 0..15 of pairs p = g / 2 and 2 + g / 2.
  // Lanes of columns past the item's tokens get an offset past the buffer's
  // end: their term loads return zeros without a memory access (an item
  // averages a few tokens, and the terms of all 16 columns would otherwise
  // be several times the weight bytes through the load path).
  const uint32_t oob = 0x80000000u;
  const uint32_t tv_off = tv ? (uint32_t)(brow * tb) + 2u * (64u * (uint32_t)(g >> 1) + 16u * (uint32_t)(g & 1)) : oob;
  const uint32_t ts_off = tv ? (uint32_t)(brow * tb) : oob;
  // Weights are requested AHEAD super-blocks ahead of the one computed,
  // after that super-block's activation terms, so waiting for the terms does
  // not wait for the prefetch (loads complete in order); several super-blocks
  // in flight per wave keep enough bytes in flight per CU at the two waves per
  // SIMD these registers allow.
  // lane group g reads code bytes 16 g .. + 15 and 64 + 16 g .. + 15, so each
  // load instruction covers 64 contiguous bytes of a row
  struct W {
    v4u H0, H1, A0, B0, A1, B1;
  };
  // The lane's offsets stay in registers for the whole loop and a super-block
  // goes in the scalar offset, so no address register is rewritten while an
  // earlier prefetch is in flight (rewriting one waits for that load). The
  // prefetches past the last super-block go through a zero-length resource:
  // they return zeros without a memory access, and the loop needs no branch.
  const uint32_t qa_off = arow_off + 16u + 16u * (uint32_t)g, qa1_off = arow1_off + 16u + 16u * (uint32_t)g;
  const __amdgpu_buffer_rsrc_t rnull = nsx_rsrc(tbase, 0u);
  auto load_w = [&](int sb, W& o) {
    const bool in = sb < nsb;
    const __amdgpu_buffer_rsrc_t r0 = in ? rs0 : rnull, r1 = in ? rs1 : rnull;
    const int so = in ? sb * 144 : 0;
    o.H0 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, arow_off, so, 0));
    o.A0 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, qa_off, so, 0));
    o.B0 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, qa_off + 64u, so, 0));
    if constexpr (GU) {
      o.H1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r1, arow_off, so, 0));
      o.A1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r1, qa_off, so, 0));
      o.B1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r1, qa_off + 64u, so, 0));
    } else {  // the second row tile
      o.H1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, arow1_off, so, 0));
      o.A1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, qa1_off, so, 0));
      o.B1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r0, qa1_off + 64u, so, 0));
    }
  };
  mq_f4 y0 = {0.f, 0.f, 0.f, 0.f}, y1 = {0.f, 0.f, 0.f, 0.f};
  // Items of up to MQ_LDS_NT tokens (the common case at a few tokens per
  // expert): the workgroup copies the tokens' whole term rows into LDS once,
  // and the super-block loop reads its terms from there -- LDS reads are
  // tracked apart from the weight loads, so nothing waits on a prefetch.
  // Larger items read each super-block's terms from L2 (through the buffer
  // loads above).
  const int tsb = (int)mq_lds_row(K);  // LDS bytes per token row
  const uint8_t* xrow = mq_xs + min(lr, n - 1) * tsb;
  const int lane_off = 2 * (64 * (g >> 1) + 16 * (g & 1));
  auto run = [&](auto blds) {
    constexpr bool BLDS = decltype(blds)::value;
    // weights requested AHEAD super-blocks ahead: two from LDS terms; one for the larger items, whose 72
    // registers of terms per super-block leave no room for more at three waves per SIMD
    constexpr int AHEAD = BLDS ? 2 : 1;
    auto step = [&](int sb, const W& cur, W& nxt) {
      if constexpr (BLDS) {
        // the terms from LDS inside the compute (their waits are LDS waits, apart from the weights')
        load_w(sb + AHEAD, nxt);
        __builtin_amdgcn_sched_barrier(0);
        if (sb < nsb)  // (the loop below runs whole rounds of steps)
          mq_superblock2_lds(cur.H0, cur.A0, cur.B0, cur.H1, cur.A1, cur.B1, xrow + lane_off + sb * 512, 2 * K,
                             xrow + 4 * K + 16 * sb, K / 16, g, y0, y1);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        mq_h8 BH[8], BL[8];
        const int sh_off = sb * 512, sl_off = 2 * K + sb * 512;  // hi[K] then lo[K], f16
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {  // s8 = 4 hi + t: pair (t >> 1) * 2 + g / 2, elements + 32 hi + 8 (t & 1)
          const int t = s8 & 3;
          const uint32_t o = 2u * (128u * (uint32_t)(t >> 1) + 32u * (uint32_t)(s8 >> 2) + 8u * (uint32_t)(t & 1));
          BH[s8] = __builtin_bit_cast(mq_h8, __builtin_amdgcn_raw_buffer_load_b128(rt, tv_off + o, sh_off, 0));
          BL[s8] = __builtin_bit_cast(mq_h8, __builtin_amdgcn_raw_buffer_load_b128(rt, tv_off + o, sl_off, 0));
        }
        // sub-block sums after the terms; the min term's A operand is zero outside
        // k < 8 (g == 0), so every group may load the same sums
        const mq_h8 SH = __builtin_bit_cast(mq_h8, __builtin_amdgcn_raw_buffer_load_b128(rt, ts_off, 4 * K + 16 * sb, 0));
        const mq_h8 SL =
            __builtin_bit_cast(mq_h8, __builtin_amdgcn_raw_buffer_load_b128(rt, ts_off, 4 * K + K / 16 + 16 * sb, 0));
        load_w(sb + AHEAD, nxt);
        // every load of the step goes out before the first MFMA waits on one, and the
        // step's compute stays between its loads and the next step's (left to itself
        // the scheduler spreads the term loads among the MFMAs, each wait then an L2
        // round trip, and issues the prefetch after most of the step's compute)
        __builtin_amdgcn_sched_barrier(0);
        if (sb < nsb) {  // (the loop below runs whole rounds of steps)
          mq_superblock(cur.H0, cur.A0, cur.B0, BH, BL, SH, SL, g, y0);
          mq_superblock(cur.H1, cur.A1, cur.B1, BH, BL, SH, SL, g, y1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    W w[AHEAD + 1];
    // the staged rows go out first (in flight together, no registers), then the weight prefetch. A wave then
    // waits on all of them, the first weights included: until a vmcnt(0) retires the direct-to-LDS loads, the
    // compiler counts them as loads of another kind whose order against the weight loads it does not know, and
    // waits vmcnt(0) at each use of a weight register in the loop below -- one drain of the prefetch per round
    // of steps instead of one per workgroup (config 4 T=32: 0.346 -> 0.337 ms per step)
    if constexpr (BLDS)
      mq_stage_lds(mq_xs, tsb, n, (int)tb, [&](int w) { return tbase + (int64_t)__shfl(brow, w, 64) * tb; });
    if (r0 < NR) {
#pragma unroll
      for (int j = 0; j < AHEAD; ++j) load_w(j, w[j]);
    }
    if constexpr (BLDS) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt not waited on
      grp_lds_barrier();
    }
    if (r0 >= NR) return;
    // step sb computes super-block sb and requests sb + AHEAD into the buffer sb - 1 used; one exit, and
    // every step's loads unconditional, so the wait counts stay exact around the loop
    for (int sb = 0; sb < nsb; sb += AHEAD + 1) {
#pragma unroll
      for (int j = 0; j <= AHEAD; ++j) step(sb + j, w[j], w[(j + AHEAD) % (AHEAD + 1)]);
    }
  };
  if (n <= MQ_LDS_NT)
    run(std::true_type{});
  else
    run(std::false_type{});
  if (r0 >= NR) return;
  const float scale = *(const float*)(tbase + brow * tb + 4 * K + K / 8);  // 2^e of this column's terms
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r0 + 4 * g + i;
    if (!tv || row >= NR) continue;
    if constexpr (GU) {
      float gv = y0[i] * scale, uv = y1[i] * scale;
      if (a.gate_bias) gv += a.gate_bias[(int64_t)e * a.n_ff + row];
      if (a.up_bias) uv += a.up_bias[(int64_t)e * a.n_ff + row];
      a.act[(int64_t)pr * a.n_ff + row] = moe_act(a.act_kind, gv, uv, a.alpha, a.limit);
    } else {
      float v = y0[i] * scale;
      if (a.down_bias) v += a.down_bias[(int64_t)e * a.n_embd + row];
      a.y[(int64_t)pr * a.n_embd + row] = v;
    }
  }
  if constexpr (!GU) {  // the second row tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = r0 + MQ_ROWS + 4 * g + i;
      if (!tv || row >= NR) continue;
      float v = y1[i] * scale;
      if (a.down_bias) v += a.down_bias[(int64_t)e * a.n_embd + row];
      a.y[(int64_t)pr * a.n_embd + row] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// host side

struct MoePlan {
  int64_t off_logits, off_act, off_xqh, off_xqa, total;
  int64_t off_items, off_nitems, off_gu_items, off_gu_bounds, off_sorted, off_corder, off_y, off_rpart;
  MxGeom ggu, gdn;
  int cg, cd, sd;
  bool grouped;
  int max_items, max_gu_items, cdg, sdg;
  bool mq;  // grouped Q4_K on the matrix cores: xqh / xqa hold activation terms (mq_row_bytes per row)
};

// NSX_DISPATCH_AUTO groups t64 layers from GRP_AUTO_MIN_T tokens (the 36-layer GPT-OSS stack at T = 2 / 3 / 5 / 7:
// 455 / 620 / 832 / 1034 us per pair, 520 / 591 / 778 / 939 us grouped), and takes the Q4_K matrix-core
// kernels from MQ_AUTO_MIN_PAIRS (token, expert) pairs: a Qwen3-235B-shaped layer (top-8 of 128) at T = 8 /
// 12 / 14 / 16 / 24 took 169 / 237 / 276 / 303 / 431 us per pair against 191 / 247 / 262 / 284 / 339 us on the
// matrix cores, whose lead grows with the tokens per expert
constexpr int GRP_AUTO_MIN_T = 3;
constexpr int MQ_AUTO_MIN_PAIRS = 104;

// The Q4_K kernels take K <= 4096 and 16-byte aligned expert rows.
static bool q4k_fast(const nsx_moe_layer* L) {
  if (L->ggml_type != NSX_Q4_K || L->n_embd > Q4K_KMAX || L->n_ff > Q4K_KMAX) return false;
  if (L->gate_base) {
    const uintptr_t m = (uintptr_t)L->gate_base | (uintptr_t)L->up_base | (uintptr_t)L->down_base |
                        (uintptr_t)L->gate_stride | (uintptr_t)L->up_stride | (uintptr_t)L->down_stride;
    return (m & 15u) == 0;
  }
  return false;  // address tables: alignment unknown on the host
}

// Grouped Q4_K on the matrix cores (moe_q4k_mfma_kernel): on request, and by
// AUTO from MQ_AUTO_MIN_PAIRS pairs (config 4, T=32: 0.37 ms against 0.56 ms per pair).
static bool use_mq(const nsx_moe_layer* L, int64_t T) {
  const bool want = L->dispatch == NSX_DISPATCH_MFMA || (L->dispatch == NSX_DISPATCH_AUTO && T * L->top_k >= MQ_AUTO_MIN_PAIRS);
  return want && L->layout == NSX_LAYOUT_GGUF && q4k_fast(L);
}

static bool use_grouped(const nsx_moe_layer* L, int64_t T) {
  if (L->dispatch == NSX_DISPATCH_GROUPED || use_mq(L, T)) return true;
  // Q4_K: AUTO groups through use_mq (the VALU grouped kernels measure slower than the per-pair ones)
  return L->dispatch == NSX_DISPATCH_AUTO && L->layout == NSX_LAYOUT_T64 && T >= GRP_AUTO_MIN_T;
}

// tokens per grouped pass (the sort handles GRP_MAX_PAIRS pairs)
static int64_t grp_chunk_tokens(const nsx_moe_layer* L) { return GRP_MAX_PAIRS / std::max(1, (int)L->top_k); }

static MoePlan moe_plan(const nsx_moe_layer* L, int64_t T) {
  MoePlan p{};
  p.grouped = use_grouped(L, T);
  p.mq = use_mq(L, T);
  if (p.grouped) T = std::min(T, grp_chunk_tokens(L));
  const int64_t P = T * L->top_k;
  const bool t64 = L->layout == NSX_LAYOUT_T64;
  p.ggu = mx_geom(L->n_ff, L->n_embd);
  p.gdn = mx_geom(L->n_embd, L->n_ff);
  p.cg = (int)nsx_cdiv(p.ggu.ns, GU_S);
  const int kk = std::max(1, std::min(L->top_k, 16));
  p.cd = std::max(1, std::min(p.gdn.ns, 16 / kk));  // top_k * cd waves per down workgroup
  p.sd = (int)nsx_cdiv(p.gdn.ns, p.cd);
  p.cdg = std::max(1, std::min(p.gdn.ns, 4));  // grouped down: 4 row groups x cdg chunks
  p.sdg = (int)nsx_cdiv(p.gdn.ns, p.cdg);
  p.max_items = p.grouped ? grp_max_items(L->n_expert, (int)P) : 0;
  p.max_gu_items = p.grouped && t64 ? grp_max_items(L->n_expert, (int)P, GRP_GU_T) : 0;
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  int64_t o = 0;
  p.off_logits = o;
  o = al(o + T * L->n_expert * 4);
  p.off_act = o;
  o = al(o + (t64 ? 0 : P * L->n_ff * 4));
  // Q4_K on the int8 dot: activation terms of h per token (grouped) and of the activations per pair
  const bool a8 = !p.mq && !t64 && q4k_fast(L);
  p.off_xqh = o;
  o = al(o + (t64 ? T * p.ggu.ns * XQ_STEP
                  : (p.mq ? T * mq_row_bytes(L->n_embd) : (a8 && p.grouped ? T * a8_bytes(L->n_embd) : 0))));
  p.off_xqa = o;
  o = al(o + (t64 ? P * p.gdn.ns * XQ_STEP : (p.mq ? P * mq_row_bytes(L->n_ff) : (a8 ? P * a8_bytes(L->n_ff) : 0))));
  p.off_items = o;
  o = al(o + (int64_t)p.max_items * 16);
  p.off_nitems = o;
  o = al(o + (p.grouped ? 4 : 0));
  p.off_gu_items = o;
  o = al(o + (int64_t)p.max_gu_items * 16);
  p.off_gu_bounds = o;
  o = al(o + (p.max_gu_items ? 35 * 4 : 0));  // bounds: gate/up, down; then the gate/up and down counters
  p.off_sorted = o;
  o = al(o + (p.grouped ? P * 4 : 0));
  p.off_corder = o;
  o = al(o + (p.grouped ? P * 4 : 0));
  p.off_y = o;
  o = al(o + (p.grouped ? P * L->n_embd * 4 : 0));
  p.off_rpart = o;  // router K-chunk partials (MFMA router)
  o = al(o + (T >= RM_MIN_T ? (int64_t)rm_chunks(L->n_embd) * T * L->n_expert * 4 : 0));
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
  NSX_REQUIRE(L->router_w && (L->gate_ptrs || L->gate_base || L->gate_tiles) &&
                  (L->up_ptrs || L->up_base || L->up_tiles) && (L->down_ptrs || L->down_base || L->down_tiles),
              NSX_EINVAL, "null weights");
  NSX_REQUIRE(L->layout == NSX_LAYOUT_T64 || !(L->gate_tiles || L->up_tiles || L->down_tiles), NSX_EINVAL,
              "tile tables need the t64 layout");
  const int64_t mx = std::max(L->n_embd, L->n_ff);
  NSX_REQUIRE((int64_t)raw_row_bytes<NSX_Q8_0>((int)mx) * mx < (1ll << 31), NSX_EINVAL, "expert matrix above 2 GiB");
  if (L->layout == NSX_LAYOUT_GGUF) {
    NSX_REQUIRE((int64_t)(L->n_embd + L->n_embd / 32) * 4 <= 64 * 1024, NSX_EINVAL, "n_embd too large for LDS");
    NSX_REQUIRE((int64_t)L->top_k * (L->n_ff + L->n_ff / 32) * 4 <= 160 * 1024, NSX_EINVAL,
                "top_k * n_ff too large for LDS");
  } else {
    const MoePlan pl = moe_plan(L, T);
    NSX_REQUIRE(pl.cg <= MAX_CHUNKS, NSX_EINVAL, "t64 layers take n_embd <= %d", MAX_CHUNKS * GU_S * 128);
    if (pl.grouped) {
      NSX_REQUIRE(pl.sdg <= DC_S, NSX_EINVAL, "grouped t64 layers take n_ff <= %d", DC_S * 4 * 128);
    } else {
      NSX_REQUIRE(pl.sd <= DC_S, NSX_EINVAL, "t64 layers take n_ff <= %d at top_k=%d",
                  DC_S * (16 / std::max(1, L->top_k)) * 128, L->top_k);
    }
  }
  NSX_REQUIRE(L->dispatch == NSX_DISPATCH_AUTO || L->dispatch == NSX_DISPATCH_PAIRS ||
                  L->dispatch == NSX_DISPATCH_GROUPED || L->dispatch == NSX_DISPATCH_MFMA,
              NSX_EINVAL, "dispatch %d", L->dispatch);
  NSX_REQUIRE(L->dispatch != NSX_DISPATCH_MFMA || (L->layout == NSX_LAYOUT_GGUF && q4k_fast(L)), NSX_ENOTIMPL,
              "NSX_DISPATCH_MFMA is implemented for stacked, 16-byte aligned Q4_K experts with K <= 4096");
  NSX_REQUIRE(!use_grouped(L, T) || L->layout == NSX_LAYOUT_T64 || q4k_fast(L), NSX_ENOTIMPL,
              "grouped dispatch is implemented for the t64 layout and for stacked, 16-byte aligned Q4_K "
              "experts with K <= 4096");
  return NSX_OK;
}


// f(std::integral_constant<int, LPR>) for the lanes per row of a Q4_K dot of K elements
template <typename F>
static int with_q4k_lpr(int K, F&& f) {
  switch (q4k_lpr(K)) {
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    default: return f(std::integral_constant<int, 64>{});
  }
}

static int launch_q4k(const MoeDev& d, int64_t T, hipStream_t st, bool gate_up, bool down) {
  const int64_t P = T * d.top_k;
  if (gate_up) {
    const bool bias = d.gate_bias || d.up_bias;
    const int rc = with_q4k_lpr(d.n_embd, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value, RPG = Q4K_GU_WAVES * Q4K_GU_STEPS * (64 / LPR);
      const dim3 g((unsigned)(P * nsx_cdiv(d.n_ff, RPG))), b(64 * Q4K_GU_WAVES);
      return bias ? nsx_launch(moe_gu_q4k_kernel<LPR, true>, g, b, 0, st, d)
                  : nsx_launch(moe_gu_q4k_kernel<LPR, false>, g, b, 0, st, d);
    });
    if (rc) return rc;
  }
  if (!down) return NSX_OK;
  return with_q4k_lpr(d.n_ff, [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value, RPG = 2 * Q4K_DN_STEPS * (64 / LPR);
    const size_t lds = (size_t)d.top_k * (size_t)a8_bytes(d.n_ff);
    const void* k = d.down_bias ? (const void*)moe_down_q4k_kernel<LPR, true> : (const void*)moe_down_q4k_kernel<LPR, false>;
    if (lds > 64 * 1024) NSX_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const dim3 g((unsigned)(T * nsx_cdiv(d.n_embd, RPG))), b(128 * d.top_k);
    return d.down_bias ? nsx_launch(moe_down_q4k_kernel<LPR, true>, g, b, lds, st, d)
                       : nsx_launch(moe_down_q4k_kernel<LPR, false>, g, b, lds, st, d);
  });
}

template <int FMT>
static int launch_raw_phases(const MoeDev& d, int64_t T, hipStream_t st, bool gate_up, bool down) {
  const int64_t P = T * d.top_k;
  const int n16 = raw_slots(raw_row_bytes<FMT>(d.n_embd));
  const int l16 = raw_stageable<FMT>() ? (n16 + 63) / 64 : 0;
  const size_t lds1 = (size_t)raw_xpad_bytes(1, d.n_embd) +
                      (l16 >= 1 && l16 <= RAW_L16_MAX ? (size_t)RAW_WAVES * 2 * n16 * 16 : 0);
  const unsigned g1 = (unsigned)(P * nsx_cdiv(d.n_ff, RAW_WAVES));
  if (gate_up) {
    auto go = [&](auto kern) {
      if (lds1 > 64 * 1024)
        NSX_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1));
      return nsx_launch(kern, dim3(g1), dim3(64 * RAW_WAVES), lds1, st, d);
    };
    int rc;
    if constexpr (raw_stageable<FMT>()) {
      rc = l16 == 1 ? go(moe_gu_raw_kernel<FMT, 1>) : l16 == 2 ? go(moe_gu_raw_kernel<FMT, 2>)
         : l16 == 3 ? go(moe_gu_raw_kernel<FMT, 3>) : l16 == 4 ? go(moe_gu_raw_kernel<FMT, 4>)
         : go(moe_gu_raw_kernel<FMT, 0>);
    } else {
      rc = go(moe_gu_raw_kernel<FMT, 0>);
    }
    if (rc) return rc;
  }
  if (!down) return NSX_OK;
  const size_t lds2 = (size_t)raw_xpad_bytes(d.top_k, d.n_ff);
  if (lds2 > 64 * 1024)
    NSX_HIP(hipFuncSetAttribute((const void*)moe_down_raw_kernel<FMT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds2));
  const unsigned g2 = (unsigned)(T * nsx_cdiv(d.n_embd, RAW_WAVES));
  return nsx_launch(moe_down_raw_kernel<FMT>, dim3(g2), dim3(64 * RAW_WAVES), lds2, st, d);
}

// The device view of a layer call: T tokens h -> out, ids, weights over the
// workspace laid out by moe_plan.
static MoeDev make_dev(const nsx_moe_layer* L, const MoePlan& p, char* ws, const float* h, int64_t T, float* out,
                       int32_t* ids, float* weights) {
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
  d.gate_tiles = L->gate_tiles;
  d.up_tiles = L->up_tiles;
  d.down_tiles = L->down_tiles;
  d.gate_base = L->gate_base;
  d.up_base = L->up_base;
  d.down_base = L->down_base;
  d.gate_stride = L->gate_stride;
  d.up_stride = L->up_stride;
  d.down_stride = L->down_stride;
  d.gate_bias = L->gate_bias;
  d.up_bias = L->up_bias;
  d.down_bias = L->down_bias;
  d.h = h;
  d.out = out;
  d.act = (float*)(ws + p.off_act);
  d.xq_h = (const uint8_t*)(ws + p.off_xqh);
  d.xq_a = (uint8_t*)(ws + p.off_xqa);
  d.n_embd = L->n_embd;
  d.n_ff = L->n_ff;
  d.ggu = p.ggu;
  d.gdn = p.gdn;
  d.cg = p.cg;
  d.sg = GU_S;
  d.cd = p.cd;
  d.sd = p.sd;
  d.act_kind = L->act;
  d.alpha = L->alpha;
  d.limit = L->limit;
  d.items = (int4*)(ws + p.off_items);
  d.n_items = (int*)(ws + p.off_nitems);
  d.gu_items = p.max_gu_items ? (int4*)(ws + p.off_gu_items) : nullptr;  // (null: the sort makes no such items)
  d.gu_bounds = p.max_gu_items ? (int*)(ws + p.off_gu_bounds) : nullptr;
  d.dn_bounds = p.max_gu_items ? d.gu_bounds + 9 : nullptr;
  d.gu_ctr = p.max_gu_items ? d.gu_bounds + 18 : nullptr;
  d.dn_ctr = p.max_gu_items ? d.gu_bounds + 26 : nullptr;
  d.sorted = (int32_t*)(ws + p.off_sorted);
  d.corder = (int32_t*)(ws + p.off_corder);
  d.y = (float*)(ws + p.off_y);
  d.max_items = p.max_items;
  d.cdg = p.cdg;
  d.sdg = p.sdg;
  return d;
}

// Phases ph0..ph1 of one layer (NSX_PHASE_*); each later phase reads what
// the earlier ones left in the workspace.
static int moe_run(const nsx_moe_layer* L, const float* h, int64_t T, float* out, int32_t* ids, float* weights,
                   void* workspace, int64_t workspace_bytes, void* stream, int ph0, int ph1,
                   RtNorm nm = RtNorm{0, nullptr, nullptr, 0.f, nullptr}, const AddNorm* an = nullptr) {
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
  MoeDev d = make_dev(L, p, ws, h, T, out, ids, weights);
  // Per-pair Q4_K below RM_MIN_T tokens: the gate/up kernel selects the top-k itself (no top-k launch), but only
  // when this call runs both phases -- a router phase run on its own always leaves the ids and weights written.
  // (the raw-row kernels of the other GGUF layouts likewise)
  d.topk_in_gu = !t64 && !p.grouped && T < RM_MIN_T && ph0 <= NSX_PHASE_ROUTER && ph1 >= NSX_PHASE_GATE_UP;
  // Grouped below RM_MIN_T tokens: the sort kernel selects the top-k itself, under the same condition.
  d.topk_in_sort = p.grouped && T < RM_MIN_T && ph0 <= NSX_PHASE_ROUTER && ph1 >= NSX_PHASE_GATE_UP;
  // The per-pair t64 gate/up kernel always selects the top-k itself; a router phase that ends the call launches
  // the top-k too, so that phase-by-phase callers read the ids after it.
  const bool router_alone = ph1 == NSX_PHASE_ROUTER;

  auto on = [&](int ph) { return ph0 <= ph && ph <= ph1; };
  if (on(NSX_PHASE_ROUTER)) {
    if (T >= RM_MIN_T) {  // logits as MFMA tiles, then chunk sums + top-k
      rc = launch_router_mfma(h, T, L->n_embd, L->router_w, L->router_dtype, L->router_bias, L->n_expert, L->top_k,
                              L->router_mode, (float*)(ws + p.off_rpart), (float*)(ws + p.off_logits), ids, weights,
                              t64 || p.mq ? (uint8_t*)(ws + p.off_xqh) : nullptr, !t64 && p.mq, st);
      if (rc) return rc;
    } else {
      rc = launch_logits(h, T, L->n_embd, L->router_w, L->router_dtype, L->router_bias, L->n_expert,
                         (float*)(ws + p.off_logits), t64 ? (uint8_t*)(ws + p.off_xqh) : nullptr, st, nm);
      if (rc) return rc;
      if ((!t64 || p.grouped || router_alone) && !d.topk_in_gu && !d.topk_in_sort &&  // else gate/up or sort selects it
          (rc = launch_topk(d.logits, T, L->n_expert, L->top_k, L->router_mode, ids, weights, st)))
        return rc;
    }
  }
  const int64_t P = T * L->top_k;

  if (p.grouped) {
    const int64_t items = (int64_t)p.max_items;
    auto grid8 = [&](int64_t groups) { return dim3((unsigned)(8 * nsx_cdiv(items * groups, 8))); };
    if (on(NSX_PHASE_GATE_UP)) {
      // a small batch whose top-k the sort would select: the t64 gate/up workgroups sort the pairs themselves
      const bool sin = t64 && d.topk_in_sort && P <= GRP_SMALL_P;
      if (!sin && (rc = nsx_launch(moe_sort_kernel, dim3(1), dim3(1024), 0, st, d))) return rc;
      if (t64) {
        // persistent: the resident workgroups (a multiple of 8), no more than the units can use
        const void* kern = sin ? (const void*)moe_gu_grouped_kernel<true> : (const void*)moe_gu_grouped_kernel<false>;
        const int64_t r = std::max<int64_t>(8, nsx_resident_workgroups(kern, 0, 64 * p.cg) / 8 * 8);
        const dim3 grid((unsigned)std::min<int64_t>(r, 8 * nsx_cdiv((int64_t)p.max_gu_items * p.ggu.tiles, 8)));
        rc = sin ? nsx_launch(moe_gu_grouped_kernel<true>, grid, dim3(64 * p.cg), 0, st, d)
                 : nsx_launch(moe_gu_grouped_kernel<false>, grid, dim3(64 * p.cg), 0, st, d);
      } else if (p.mq) {
        // h's term rows: from the matrix-core router's extra workgroups when it ran in this call
        if (!(on(NSX_PHASE_ROUTER) && T >= RM_MIN_T) &&
            (rc = nsx_launch(mq_terms_kernel, dim3((unsigned)T), dim3(256), 0, st, h, (int)L->n_embd,
                             (uint8_t*)(ws + p.off_xqh))))
          return rc;
        rc = nsx_launch(moe_q4k_mfma_kernel<true>, grid8(nsx_cdiv(L->n_ff, MQ_WG_ROWS)), dim3(256),
                        (size_t)(MQ_LDS_NT * mq_lds_row(L->n_embd)), st, d);
      } else {  // Q4_K on the int8 dot: the tokens' activation terms, then the rows
        if ((rc = nsx_launch(a8_terms_kernel, dim3((unsigned)T), dim3(256), 0, st, h, (int)L->n_embd,
                             (uint8_t*)(ws + p.off_xqh))))
          return rc;
        rc = with_q4k_lpr(L->n_embd, [&](auto lpr) {
          constexpr int LPR = decltype(lpr)::value;
          const int64_t g = nsx_cdiv(L->n_ff, Q4K_GG_WAVES * Q4K_GG_STEPS * (64 / LPR));
          return nsx_launch(moe_gu_q4k_grouped_kernel<LPR>, grid8(g), dim3(64 * Q4K_GG_WAVES), 0, st, d);
        });
      }
      if (rc) return rc;
    }
    if (on(NSX_PHASE_DOWN)) {
      if (t64) {
        // persistent (the resident workgroups, a multiple of 8) when its units can number GRP_DN_PERSIST times
        // the resident workgroups, else one workgroup per (GRP_TPI-token item, tile)
        const int64_t r = std::max<int64_t>(
            8, nsx_resident_workgroups((const void*)moe_down_persistent_kernel, 0, 64 * p.cdg) / 8 * 8);
        rc = (int64_t)p.max_gu_items * p.gdn.tiles >= GRP_DN_PERSIST * r
                 ? nsx_launch(moe_down_persistent_kernel, dim3((unsigned)r), dim3(64 * p.cdg), 0, st, d)
                 : nsx_launch(moe_down_grouped_kernel, grid8(p.gdn.tiles), dim3(64 * p.cdg), 0, st, d);
      } else if (p.mq) {
        if ((rc = nsx_launch(mq_terms_kernel, dim3((unsigned)P), dim3(256), 0, st, (const float*)d.act,
                             (int)L->n_ff, d.xq_a)))
          return rc;
        rc = nsx_launch(moe_q4k_mfma_kernel<false>, grid8(nsx_cdiv(L->n_embd, 2 * MQ_WG_ROWS)), dim3(256),
                        (size_t)(MQ_LDS_NT * mq_lds_row(L->n_ff)), st, d);
      } else {
        if ((rc = nsx_launch(a8_terms_kernel, dim3((unsigned)P), dim3(256), 0, st, (const float*)d.act,
                             (int)L->n_ff, d.xq_a)))
          return rc;
        rc = with_q4k_lpr(L->n_ff, [&](auto lpr) {
          constexpr int LPR = decltype(lpr)::value;
          const int64_t g = nsx_cdiv(L->n_embd, Q4K_DG_WAVES * Q4K_DG_STEPS * (64 / LPR));
          return nsx_launch(moe_down_q4k_grouped_kernel<LPR>, grid8(g), dim3(64 * Q4K_DG_WAVES),
                            (size_t)(Q4K_GROUP_NT * a8_bytes(L->n_ff)), st, d);
        });
      }
      if (rc) return rc;
    }
    if (on(NSX_PHASE_COMBINE)) {
      if (an)
        rc = L->top_k <= 4 ? nsx_launch(moe_combine_norm_kernel<4>, dim3((unsigned)T), dim3(1024), 0, st, d, *an)
                           : nsx_launch(moe_combine_norm_kernel<MAX_TOPK>, dim3((unsigned)T), dim3(1024), 0, st, d, *an);
      else
        rc = L->top_k <= 4 ? nsx_launch(moe_combine_kernel<4>, dim3((unsigned)nsx_cdiv(L->n_embd, 256), (unsigned)T),
                                        dim3(256), 0, st, d)
                           : nsx_launch(moe_combine_kernel<MAX_TOPK>, dim3((unsigned)nsx_cdiv(L->n_embd, 256),
                                        (unsigned)T), dim3(256), 0, st, d);
      if (rc) return rc;
    }
    return NSX_OK;
  }
  if (t64) {
    if (on(NSX_PHASE_GATE_UP) &&
        (rc = nsx_launch(moe_gu_kernel, dim3((unsigned)(P * p.ggu.tiles)), dim3(128 * p.cg), 0, st, d)))
      return rc;
    if (on(NSX_PHASE_DOWN) &&
        (rc = nsx_launch(moe_down_kernel, dim3((unsigned)(8 * nsx_cdiv(T * 4 * p.gdn.tiles, 8))),
                         dim3(64 * L->top_k * p.cd), 0, st, d)))
      return rc;
    return NSX_OK;  // the down kernel also combines
  }
  switch (L->ggml_type) {  // the GGUF-layout down kernel also combines
    case NSX_MXFP4: return launch_raw_phases<NSX_MXFP4>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q4_K:
      if (q4k_fast(L)) return launch_q4k(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
      return launch_raw_phases<NSX_Q4_K>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q4_0: return launch_raw_phases<NSX_Q4_0>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
    case NSX_Q8_0: return launch_raw_phases<NSX_Q8_0>(d, T, st, on(NSX_PHASE_GATE_UP), on(NSX_PHASE_DOWN));
  }
  return nsx_fail(NSX_ENOTIMPL, "expert weight type %d", L->ggml_type);
}

extern "C" int nsx_moe_forward(const nsx_moe_layer* L, const float* h, int64_t T, float* out, int32_t* ids,
                               float* weights, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_layer(L, T);
  if (rc) return rc;
  const int64_t tc = use_grouped(L, T) ? grp_chunk_tokens(L) : T;
  for (int64_t t0 = 0; t0 < T; t0 += tc) {  // grouped passes of at most GRP_MAX_PAIRS pairs, in token order
    const int64_t n = std::min(tc, T - t0);
    const int64_t k = L->top_k;
    if (h == nullptr || out == nullptr || ids == nullptr || weights == nullptr)
      return nsx_fail(NSX_EINVAL, "null buffer");
    rc = moe_run(L, h + t0 * L->n_embd, n, out + t0 * L->n_embd, ids + t0 * k, weights + t0 * k, workspace,
                 workspace_bytes, stream, NSX_PHASE_ROUTER, NSX_PHASE_COMBINE);
    if (rc) return rc;
  }
  return NSX_OK;
}

extern "C" int nsx_moe_forward_norm(const nsx_moe_layer* L, const float* x, const float* r, const float* norm_w,
                                    float eps, int64_t T, float* x_out, float* out, int32_t* ids, float* weights,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_layer(L, T);
  if (rc) return rc;
  NSX_REQUIRE(L->layout == NSX_LAYOUT_T64 && T < RM_MIN_T && L->n_embd <= 256 * NORM_MAXV, NSX_ENOTIMPL,
              "the norm runs in the router for t64 layers below %d tokens with n_embd <= %d", RM_MIN_T,
              256 * NORM_MAXV);
  NSX_REQUIRE(x && r && x_out && out && ids && weights, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(eps >= 0.f, NSX_EINVAL, "eps %g", (double)eps);
  const uintptr_t bytes = (uintptr_t)(T * L->n_embd * 4);
  auto overlap = [&](const void* p, const void* q) {
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return a < b + bytes && b < a + bytes;
  };
  NSX_REQUIRE(!overlap(x_out, x) && !overlap(x_out, r), NSX_EINVAL, "x_out overlaps x or r");
  return moe_run(L, x, T, out, ids, weights, workspace, workspace_bytes, stream, NSX_PHASE_ROUTER, NSX_PHASE_COMBINE,
                 RtNorm{1, r, norm_w, eps, x_out});
}

extern "C" int nsx_moe_forward_addnorm(const nsx_moe_layer* L, const float* h, int64_t T, const float* x,
                                       const float* norm_w, float eps, float* x_out, float* h_out, int32_t* ids,
                                       float* weights, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_layer(L, T);
  if (rc) return rc;
  NSX_REQUIRE(h && x && x_out && h_out && ids && weights, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(eps >= 0.f, NSX_EINVAL, "eps %g", (double)eps);
  NSX_REQUIRE(L->n_embd <= 256 * NORM_MAXV, NSX_EINVAL, "n_embd %d above %d", L->n_embd, 256 * NORM_MAXV);
  const uintptr_t bytes = (uintptr_t)(T * L->n_embd * 4);
  auto overlap = [&](const void* p, const void* q) {
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return a < b + bytes && b < a + bytes;
  };
  NSX_REQUIRE((x_out == x || !overlap(x_out, x)) && !overlap(h_out, x) && !overlap(h_out, x_out), NSX_EINVAL,
              "x_out must be x or apart from it, h_out apart from both");
  if (!use_grouped(L, T)) {  // the per-pair kernels combine in their down kernel: into h_out, then the norm
    if ((rc = nsx_moe_forward(L, h, T, h_out, ids, weights, workspace, workspace_bytes, stream))) return rc;
    return nsx_add_rmsnorm(x, h_out, T, L->n_embd, eps, norm_w, x_out, h_out, stream);
  }
  const int64_t tc = grp_chunk_tokens(L), k = L->top_k, ne = L->n_embd;
  for (int64_t t0 = 0; t0 < T; t0 += tc) {  // grouped passes in token order, as nsx_moe_forward
    const int64_t nt = std::min(tc, T - t0);
    // moe_run plans each pass for its own token count: a short last pass (AUTO: t64 below GRP_AUTO_MIN_T tokens,
    // Q4_K below MQ_AUTO_MIN_PAIRS pairs) runs the per-pair kernels, whose down kernel combines and which take no
    // fused add + norm -- that pass gets the separate norm, as the ungrouped branch above
    if (!use_grouped(L, nt)) {
      if ((rc = moe_run(L, h + t0 * ne, nt, h_out + t0 * ne, ids + t0 * k, weights + t0 * k, workspace,
                        workspace_bytes, stream, NSX_PHASE_ROUTER, NSX_PHASE_COMBINE)))
        return rc;
      if ((rc = nsx_add_rmsnorm(x + t0 * ne, h_out + t0 * ne, nt, ne, eps, norm_w, x_out + t0 * ne, h_out + t0 * ne,
                                stream)))
        return rc;
      continue;
    }
    const AddNorm an{x + t0 * ne, norm_w, eps, x_out + t0 * ne, h_out + t0 * ne};
    // (no combine output: h_out stands in for `out`, which the grouped phases before the combine never touch)
    rc = moe_run(L, h + t0 * ne, nt, h_out + t0 * ne, ids + t0 * k, weights + t0 * k, workspace, workspace_bytes,
                 stream, NSX_PHASE_ROUTER, NSX_PHASE_COMBINE, RtNorm{0, nullptr, nullptr, 0.f, nullptr}, &an);
    if (rc) return rc;
  }
  return NSX_OK;
}

// ---------------------------------------------------------------------------
// One layer of a stacked FFN chain at decode (T = 1): x += moe(rms_norm(x) *
// norm_w) in place, the router of every layer after the first regrouped
// across the kernel boundary (moe_gu_chain_kernel, moe_down_chain_kernel).

// the down kernel's work items of one token: one router share each
static int64_t chain_groups(const nsx_moe_layer* L) { return 4 * mx_geom(L->n_embd, L->n_ff).tiles; }

static int check_chain_layer(const nsx_moe_layer* L) {
  int rc = check_layer(L, 1);
  if (rc) return rc;
  NSX_REQUIRE(L->layout == NSX_LAYOUT_T64 && !use_grouped(L, 1), NSX_ENOTIMPL,
              "the decode chain runs t64 layers on the per-pair kernels");
  const MoePlan p = moe_plan(L, 1);
  NSX_REQUIRE(L->n_embd % 16 == 0 && p.ggu.ns <= CH_MAX_NS && L->n_expert % 4 == 0 && L->n_expert <= 128 &&
                  chain_groups(L) <= 256 && p.cg <= MAX_CHUNKS,
              NSX_ENOTIMPL,
              "the decode chain takes n_embd a multiple of 16 up to %d and a multiple of 4 experts up to 128",
              CH_MAX_NS * 128);
  return NSX_OK;
}

extern "C" int64_t nsx_moe_chain_share_bytes(const nsx_moe_layer* L) {
  if (check_chain_layer(L) != NSX_OK) return -1;
  return chain_groups(L) * (L->n_expert + 1) * 4;
}

extern "C" int nsx_moe_chain_t1(const nsx_moe_layer* L, float* x, const float* norm_w, float eps,
                                const float* share_in, const nsx_moe_layer* next, const float* next_norm_w,
                                float* share_out, float* out, int32_t* ids, float* weights, void* workspace,
                                int64_t workspace_bytes, int phases, void* stream) {
  int rc = check_chain_layer(L);
  if (rc) return rc;
  NSX_REQUIRE(x && out && ids && weights && workspace, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(eps >= 0.f, NSX_EINVAL, "eps %g", (double)eps);
  NSX_REQUIRE(phases >= 1 && phases <= 3, NSX_EINVAL, "phases %d: NSX_CHAIN_GATE_UP | NSX_CHAIN_DOWN", phases);
  const MoePlan p = moe_plan(L, 1);
  NSX_REQUIRE(workspace_bytes >= p.total, NSX_EINVAL, "workspace of %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)p.total);
  const int64_t G = chain_groups(L);
  if (next) {
    if ((rc = check_chain_layer(next))) return rc;
    NSX_REQUIRE(next->n_embd == L->n_embd, NSX_EINVAL, "the next layer has n_embd %d, this one %d", next->n_embd,
                L->n_embd);
    NSX_REQUIRE(share_out, NSX_EINVAL, "a next layer needs share_out");
    NSX_REQUIRE(L->top_k * p.cd >= 1 + nsx_cdiv(next->n_expert, 64), NSX_ENOTIMPL,
                "the down workgroup has %d waves, the next router's shares need %d", L->top_k * p.cd,
                1 + (int)nsx_cdiv(next->n_expert, 64));
  }
  // x and out are n_embd floats; a share buffer G * (E + 1) floats (share_in may be share_out: the gate/up
  // kernel has read it before the down kernel writes)
  auto overlap = [](const void* a, int64_t an, const void* b, int64_t bn) {
    const uintptr_t u = (uintptr_t)a, v = (uintptr_t)b;
    return a && b && u < v + (uintptr_t)(bn * 4) && v < u + (uintptr_t)(an * 4);
  };
  const int64_t n = L->n_embd;
  NSX_REQUIRE(!overlap(x, n, out, n) && !overlap(x, n, share_in, G * (L->n_expert + 1)) &&
                  !overlap(x, n, share_out, next ? G * (next->n_expert + 1) : 0) &&
                  !overlap(out, n, share_out, next ? G * (next->n_expert + 1) : 0) &&
                  !overlap(out, n, share_in, G * (L->n_expert + 1)),
              NSX_EINVAL, "x, out and the share buffers must not overlap");
  hipStream_t st = S(stream);
  char* ws = (char*)workspace;
  MoeDev d = make_dev(L, p, ws, out, 1, out, ids, weights);
  d.cx = x;
  d.cnorm_w = norm_w;
  d.ceps = eps;
  d.crouter_b = L->router_bias;
  d.cp_in = share_in;
  d.cp_groups = (int)G;
  d.cn_w = next ? next->router_w : nullptr;
  d.cn_wdt = next ? next->router_dtype : 0;
  d.cn_E = next ? next->n_expert : 0;
  d.cn_norm_w = next_norm_w;
  d.cp_out = share_out;
  if (phases & NSX_CHAIN_GATE_UP) {
    if (share_in == nullptr) {  // the first layer routes from x: h = rms_norm(x) * w into out (scratch until the
                                // down kernel writes the layer's output there), the router, the per-pair gate/up
      if ((rc = nsx_add_rmsnorm(x, nullptr, 1, n, eps, norm_w, nullptr, out, stream))) return rc;
      if ((rc = launch_logits(out, 1, n, L->router_w, L->router_dtype, L->router_bias, L->n_expert,
                              (float*)(ws + p.off_logits), (uint8_t*)(ws + p.off_xqh), st,
                              RtNorm{0, nullptr, nullptr, 0.f, nullptr})))
        return rc;
      if ((rc = nsx_launch(moe_gu_kernel, dim3((unsigned)(L->top_k * p.ggu.tiles)), dim3(128 * p.cg), 0, st, d)))
        return rc;
    } else if ((rc = nsx_launch(moe_gu_chain_kernel, dim3((unsigned)(L->top_k * p.ggu.tiles)), dim3(1024), 0, st,
                                d))) {
      return rc;
    }
  }
  if (phases & NSX_CHAIN_DOWN)
    return nsx_launch(moe_down_chain_kernel, dim3((unsigned)(8 * nsx_cdiv(4 * p.gdn.tiles, 8))),
                      dim3(64 * L->top_k * p.cd), 0, st, d);
  return NSX_OK;
}

extern "C" int nsx_moe_phase(const nsx_moe_layer* L, int phase, const float* h, int64_t T, float* out, int32_t* ids,
                             float* weights, void* workspace, int64_t workspace_bytes, void* stream) {
  NSX_REQUIRE(phase >= NSX_PHASE_ROUTER && phase <= NSX_PHASE_COMBINE, NSX_EINVAL, "phase %d", phase);
  NSX_REQUIRE(L == nullptr || !use_grouped(L, T) || T <= grp_chunk_tokens(L), NSX_EINVAL,
              "grouped phases take at most %d pairs (T=%lld)", GRP_MAX_PAIRS, (long long)T);
  return moe_run(L, h, T, out, ids, weights, workspace, workspace_bytes, stream, phase, phase);
}

// ---------------------------------------------------------------------------
// nsx_moe_forward without a caller workspace and without any allocation: the
// workspace is `scratch`, a file-scope device array (one copy per GPU, held
// until the process ends). Host code never passes the array's name to a
// kernel -- on the host it is only a stand-in for the symbol -- but the
// address hipGetSymbolAddress reports for the current device, looked up once
// per device and kept in scratch_addr. Each call clears the part of the array
// it uses with a fill kernel (not hipMemsetAsync, so the call can be captured
// into a graph), then runs nsx_moe_forward's kernels on it. Calls on one GPU
// share the array: calls that overlap (different streams, or host threads)
// race on it.

constexpr int MAX_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[NSX_STATIC_WORKSPACE_BYTES];
static std::mutex scratch_mu;
static void* scratch_addr[MAX_DEVICES];

static int scratch_for_current_device(void** out) {
  int dev = -1;
  NSX_HIP(hipGetDevice(&dev));
  NSX_REQUIRE(dev >= 0 && dev < MAX_DEVICES, NSX_EINVAL, "device %d outside 0..%d", dev, MAX_DEVICES - 1);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    NSX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    NSX_REQUIRE(p != nullptr, NSX_EHIP, "hipGetSymbolAddress returned a null address for the scratch array");
    scratch_addr[dev] = p;
  }
  *out = scratch_addr[dev];
  return NSX_OK;
}

__global__ __launch_bounds__(256) void ws_zero_kernel(uint4* __restrict__ p, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) p[i] = uint4{0u, 0u, 0u, 0u};
}

extern "C" int nsx_moe_forward_static(const nsx_moe_layer* L, const float* h, int64_t T, float* out, int32_t* ids,
                                      float* weights, void* stream) {
  int rc = check_layer(L, T);
  if (rc) return rc;
  NSX_REQUIRE(h && out && ids && weights, NSX_EINVAL, "null buffer");
  // nsx_moe_forward runs grouped passes of at most grp_chunk_tokens tokens, each planned for its own size
  const int64_t tc = use_grouped(L, T) ? std::min(T, grp_chunk_tokens(L)) : T;
  const int64_t need = moe_plan(L, tc).total;
  NSX_REQUIRE(need <= NSX_STATIC_WORKSPACE_BYTES, NSX_EINVAL,
              "T=%lld needs a %lld-byte workspace; the static workspace holds %lld bytes (use nsx_moe_forward "
              "with a caller workspace, or fewer tokens per call)",
              (long long)T, (long long)need, (long long)NSX_STATIC_WORKSPACE_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(&ws))) return rc;
  const int64_t n16 = nsx_cdiv(need, 16);
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(1024, nsx_cdiv(n16, 256)));
  if ((rc = nsx_launch(ws_zero_kernel, dim3(grid), dim3(256), 0, S(stream), (uint4*)ws, n16))) return rc;
  return nsx_moe_forward(L, h, T, out, ids, weights, ws, need, stream);
}

// ---------------------------------------------------------------------------
// s = x + r and y = rms_norm(s) * w over rows of n (compute/ops.py:14-20
// rms_norm, fp32: v * rsqrt(mean(v^2) + eps) * w), the link between stacked
// MoE layers (model/gpt_oss.py:126,177: the residual add, then the next
// layer's norm). One workgroup per row; r, w, s and y may each be NULL (no
// residual, unit weight, no sum or no norm output); s and y may alias x or r.

constexpr int NORM_THREADS = 256;

__global__ __launch_bounds__(NORM_THREADS) void add_rmsnorm_kernel(const float* x, const float* r, int n, float eps,
                                                                   const float* __restrict__ w, float* sum,
                                                                   float* y) {
  __shared__ float part[NORM_THREADS / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * n;
  const float* rr = r ? r + row * n : nullptr;
  // Every load is issued unconditionally (addresses clamped into the row,
  // tails zeroed at use), so all of them are in flight together: predicated
  // loads would each wait behind the last.
  float v[NORM_MAXV], wv[NORM_MAXV];
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    const int c = min((int)threadIdx.x + i * NORM_THREADS, n - 1);
    v[i] = xr[c];
    wv[i] = w ? w[c] : 1.f;
  }
  if (rr) {
#pragma unroll
    for (int i = 0; i < NORM_MAXV; ++i) v[i] += rr[min((int)threadIdx.x + i * NORM_THREADS, n - 1)];
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    if ((int)threadIdx.x + i * NORM_THREADS >= n) v[i] = 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  ss = nsx_wave_sum(ss);
  if (__lane_id() == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();  // every read of x and r is done before any write below
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += part[i];
  const float inv = 1.f / sqrtf(tot / (float)n + eps);
#pragma unroll
  for (int i = 0; i < NORM_MAXV; ++i) {
    const int c = threadIdx.x + i * NORM_THREADS;
    if (c < n) {
      if (sum) sum[row * n + c] = v[i];
      if (y) y[row * n + c] = w ? (v[i] * inv) * wv[i] : v[i] * inv;
    }
  }
}

extern "C" int nsx_add_rmsnorm(const float* x, const float* r, int64_t T, int64_t n, float eps, const float* w,
                               float* sum, float* y, void* stream) {
  NSX_REQUIRE(T >= 0 && T <= (1ll << 31) - 1, NSX_EINVAL, "T=%lld", (long long)T);
  NSX_REQUIRE(n >= 1 && n <= NORM_THREADS * NORM_MAXV, NSX_EINVAL, "row length %lld outside 1..%d", (long long)n,
              NORM_THREADS * NORM_MAXV);
  NSX_REQUIRE(eps >= 0.f, NSX_EINVAL, "eps %g", (double)eps);
  if (T == 0) return NSX_OK;
  NSX_REQUIRE(x && (sum || y), NSX_EINVAL, "null buffer");
  return nsx_launch(add_rmsnorm_kernel, dim3((unsigned)T), dim3(NORM_THREADS), 0, S(stream), x, r, (int)n, eps, w, sum,
                    y);
}

// ---------------------------------------------------------------------------
// Staging expert matrices whose blocks are split between HBM and pinned host
// RAM (BASELINE config 5b): host blocks go device-ward as DMA copies
// (nsx_copy_blocks_async, the block prefetcher's host-to-device step,
// compute/blockffn.py:278-393 + io/stream.py:200-216), HBM-resident blocks
// as one gather kernel (nsx_gather_copy). Every destination range is checked
// on the host against its device allocation before anything is queued.

constexpr int GATHER_CHUNK = 16384;  // bytes per workgroup
constexpr int GATHER_MAX = 128;      // segments per launch (kernel arguments: 2.5 KB)

struct GatherList {
  uint64_t src[GATHER_MAX], dst[GATHER_MAX];
  uint32_t n16[GATHER_MAX];  // 16-byte units
  int n;
};

__global__ __launch_bounds__(256) void gather_copy_kernel(GatherList L) {
  const int s = blockIdx.y;
  if (s >= L.n) return;
  const uint4* src = (const uint4*)L.src[s];
  uint4* dst = (uint4*)L.dst[s];
  const int64_t n16 = L.n16[s];
  const int64_t c0 = (int64_t)blockIdx.x * (GATHER_CHUNK / 16);
#pragma unroll
  for (int i = 0; i < GATHER_CHUNK / 16 / 256; ++i) {
    const int64_t j = c0 + i * 256 + threadIdx.x;
    if (j < n16) dst[j] = src[j];
  }
}

// [p, p + bytes) inside one device allocation
static int check_dev_range(const void* p, int64_t bytes, const char* what, int64_t i) {
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (void*)p) != hipSuccess || base == nullptr) {
    (void)hipGetLastError();
    return nsx_fail(NSX_EINVAL, "%s of segment %lld is not device memory", what, (long long)i);
  }
  NSX_REQUIRE((const char*)p + bytes <= (const char*)base + size, NSX_EINVAL,
              "%s of segment %lld runs past its allocation", what, (long long)i);
  return NSX_OK;
}

extern "C" int nsx_copy_blocks_async(int64_t n, const uint64_t* src, const uint64_t* dst, const int64_t* bytes,
                                     void* stream, void* event) {
  NSX_REQUIRE(n >= 0 && (n == 0 || (src && dst && bytes)), NSX_EINVAL, "bad segment list");
  for (int64_t i = 0; i < n; ++i) {
    NSX_REQUIRE(bytes[i] >= 0 && src[i] && dst[i], NSX_EINVAL, "segment %lld", (long long)i);
    if (bytes[i] == 0) continue;
    int rc = check_dev_range((const void*)dst[i], bytes[i], "destination", i);
    if (rc) return rc;
    NSX_HIP(hipMemcpyAsync((void*)dst[i], (const void*)src[i], (size_t)bytes[i], hipMemcpyDefault, S(stream)));
  }
  if (event) NSX_HIP(hipEventRecord((hipEvent_t)event, S(stream)));
  return NSX_OK;
}

extern "C" int nsx_gather_copy(int64_t n, const uint64_t* src, const uint64_t* dst, const int64_t* bytes,
                               void* stream) {
  NSX_REQUIRE(n >= 0 && (n == 0 || (src && dst && bytes)), NSX_EINVAL, "bad segment list");
  for (int64_t i0 = 0; i0 < n; i0 += GATHER_MAX) {
    GatherList L{};
    int64_t max_chunks = 1;
    for (int64_t i = i0; i < std::min(n, i0 + GATHER_MAX); ++i) {
      NSX_REQUIRE(bytes[i] >= 0 && bytes[i] % 16 == 0 && bytes[i] < (16ll << 32) && src[i] % 16 == 0 &&
                      dst[i] % 16 == 0,
                  NSX_EINVAL, "segment %lld: 16-byte aligned addresses and sizes required", (long long)i);
      if (bytes[i] > 0) {
        int rc = check_dev_range((const void*)src[i], bytes[i], "source", i);
        if (rc) return rc;
        if ((rc = check_dev_range((const void*)dst[i], bytes[i], "destination", i))) return rc;
      }
      L.src[L.n] = src[i];
      L.dst[L.n] = dst[i];
      L.n16[L.n] = (uint32_t)(bytes[i] >> 4);
      ++L.n;
      max_chunks = std::max<int64_t>(max_chunks, nsx_cdiv(bytes[i], GATHER_CHUNK));
    }
    int rc = nsx_launch(gather_copy_kernel, dim3((unsigned)max_chunks, (unsigned)L.n), dim3(256), 0, S(stream), L);
    if (rc) return rc;
  }
  return NSX_OK;
}

extern "C" int nsx_host_device_address(const void* host, uint64_t* device_address) {
  NSX_REQUIRE(host && device_address, NSX_EINVAL, "null pointer");
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host), 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reported here: do not leave it for the caller's next HIP call
    return nsx_fail(NSX_EHIP, "hipHostGetDevicePointer: %s (not device-mapped pinned memory?)", hipGetErrorString(e));
  }
  *device_address = (uint64_t)(uintptr_t)d;
  return NSX_OK;
}
