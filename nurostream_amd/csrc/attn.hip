// The step either side of the MoE FFN in a GPT-OSS decode token (gfx950):
// YaRN rotary embedding + KV-cache append, and sink attention with the
// alternating sliding window, for one query token.
//
// Semantics follow the reference's model/gpt_oss.py: yarn_tables (42-58),
// the attention block (101-114) and sink_attention (73-85); compute in fp32
// like its torch path. The position of the token is read from device memory
// (`pos`), so a captured graph of a whole decode token can be replayed token
// after token; nsx_pos_advance moves it on inside the graph.
//
// KV cache layout: K and V each [n_kv][ctx_max][head_dim] fp32.
// Attention is split over chunks of ATTN_CHUNK keys (one workgroup per kv
// head and chunk, each handling the kv head's n_rep query heads), and a
// combine kernel merges the chunks in chunk order together with the sink; a
// layer whose keys always fit one chunk (a 128-key sliding window) finishes
// in the chunk kernel.
// Both grids are sized for ctx_max, so their shape does not depend on the
// position; chunks past the current length return at once.
#include "nsx_common.h"

#include <algorithm>
#include <type_traits>
#include <math.h>

namespace {

constexpr int ATTN_D = 64;        // head_dim (GPT-OSS)
constexpr int ATTN_CHUNK = 128;   // keys per attention workgroup (two rounds of 64)
constexpr int ATTN_THREADS = 256;
constexpr int ATTN_MAX_REP = 16;  // query heads per kv head

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Rotary of element d of a 64-element head row at position p: x = the
// element, partner = element d ^ 32 (both with bias), rotate_half pairing
// (gpt_oss.py:42-58, ops.py:95-104). Explicit fmaf so that every kernel that
// applies it rounds the same way.
__device__ __forceinline__ float rope_elem(float x, float partner, int d, int p, const float* __restrict__ inv_freq,
                                           float amp) {
  const float ang = (float)p * inv_freq[d & (ATTN_D / 2 - 1)];  // fp32, as positions.float() * inv
  float s, c;
  sincosf(ang, &s, &c);
  c *= amp;
  s *= amp;
  const float ps = partner * s;
  return d < ATTN_D / 2 ? fmaf(x, c, -ps) : fmaf(x, c, ps);
}

// One wave per row of the q | k | v block: bias, then rotary for q and k
// rows; k and v rows go into the cache at the token's position.
__global__ __launch_bounds__(64) void rope_kv_append_kernel(
    float* __restrict__ qkv, const float* __restrict__ bq, const float* __restrict__ bk,
    const float* __restrict__ bv, int n_head, int n_kv, const float* __restrict__ inv_freq, float amp,
    const int32_t* __restrict__ pos_ptr, float* __restrict__ k_cache, float* __restrict__ v_cache,
    int64_t ctx_max) {
  const int r = blockIdx.x, lane = threadIdx.x;
  const int p = *pos_ptr;
  if (p < 0 || p >= ctx_max) return;  // the host keeps p < ctx_max; never write outside the cache
  float x = qkv[(int64_t)r * ATTN_D + lane];
  if (r < n_head) {
    if (bq) x += bq[(int64_t)r * ATTN_D + lane];
  } else if (r < n_head + n_kv) {
    if (bk) x += bk[(int64_t)(r - n_head) * ATTN_D + lane];
  } else {
    if (bv) x += bv[(int64_t)(r - n_head - n_kv) * ATTN_D + lane];
    const int g = r - n_head - n_kv;
    v_cache[((int64_t)g * ctx_max + p) * ATTN_D + lane] = x;
    return;
  }
  const float y = rope_elem(x, __shfl_xor(x, ATTN_D / 2, 64), lane, p, inv_freq, amp);
  if (r < n_head) {
    qkv[(int64_t)r * ATTN_D + lane] = y;
  } else {
    const int g = r - n_head;
    k_cache[((int64_t)g * ctx_max + p) * ATTN_D + lane] = y;
  }
}

__device__ __forceinline__ void attn_span(int p, int window, int& lo, int& total) {
  lo = window > 0 ? max(0, p + 1 - window) : 0;
  total = p + 1 - lo;
}

// Workgroup (kv head g, chunk c of ATTN_CHUNK keys): the chunk's attention
// for the kv head's n_rep query heads. Wave w takes query heads w, w + 4,
// ... (HPW = ceil(n_rep / 4) of them) and walks the chunk in rounds of 64
// keys: the scores with one key per lane, a running softmax per head in
// registers (wave max / sum), then the value sums with lane = (key group
// kg = lane / 16, dimensions 4 * (lane % 16) ..+3) over keys kg, kg + 4, ...,
// so a round's 64 value rows are 16 coalesced 16-byte loads per lane. The
// four key groups are summed with two shuffles at the end.
// part[(h * nchunk + c) * (D + 2)] = {m, l, acc[D]} for query head h.
// FINAL (only ever one chunk: a sliding window or a cache of at most
// ATTN_CHUNK keys): the workgroup also merges the sink and writes out[h].
// ROPE: q is the token's raw q | k | v block; each workgroup adds the bias
// and applies the rotary to its query heads itself, and the workgroup whose
// chunk holds the token's position does the same for the token's k row, adds
// v's bias and appends both to the cache before it reads any key (no other
// workgroup reads that row), so no separate rotary + append launch is needed.
struct RopeArgs {
  const float *bq, *bk, *bv, *inv_freq;
  float amp;
};
template <bool FINAL, int HPW, bool ROPE>
__global__ __launch_bounds__(ATTN_THREADS) void attn_chunk_kernel(
    const float* __restrict__ q, float* k_cache, float* v_cache, const int32_t* __restrict__ pos_ptr,
    int64_t ctx_max, int window, float scale, int n_rep, int n_head, int nchunk, float* __restrict__ part,
    const float* __restrict__ sinks, float* __restrict__ out, RopeArgs ra) {
  constexpr int NW = ATTN_THREADS / 64;
  __shared__ float qs[ATTN_MAX_REP][ATTN_D];
  // each wave's key weights, key j at (j % 4) * 16 + j / 4: key group kg reads its 16 as 4 vectors
  __shared__ float wl[NW][HPW][64];
  const int g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  const int p = *pos_ptr;
  if (p < 0 || p >= ctx_max) return;
  int lo, total;
  attn_span(p, window, lo, total);
  const int k0 = c * ATTN_CHUNK;
  if (k0 >= total) return;  // past the current length
  const int nk = min(ATTN_CHUNK, total - k0);
  if constexpr (ROPE) {
    for (int i = t; i < n_rep * ATTN_D; i += ATTN_THREADS) {
      const int64_t r = (int64_t)g * n_rep + i / ATTN_D;
      const int d = i % ATTN_D, dp = d ^ (ATTN_D / 2);
      float x = q[r * ATTN_D + d], xp = q[r * ATTN_D + dp];
      if (ra.bq) {
        x += ra.bq[r * ATTN_D + d];
        xp += ra.bq[r * ATTN_D + dp];
      }
      qs[i / ATTN_D][d] = rope_elem(x, xp, d, p, ra.inv_freq, ra.amp);
    }
    if (c == (total - 1) / ATTN_CHUNK && t < 2 * ATTN_D) {  // this chunk holds the token's own key
      const int d = t & (ATTN_D - 1);
      const int64_t at = ((int64_t)g * ctx_max + p) * ATTN_D + d;
      if (t < ATTN_D) {
        const float* kr = q + ((int64_t)n_head + g) * ATTN_D;
        const int dp = d ^ (ATTN_D / 2);
        float x = kr[d], xp = kr[dp];
        if (ra.bk) {
          x += ra.bk[(int64_t)g * ATTN_D + d];
          xp += ra.bk[(int64_t)g * ATTN_D + dp];
        }
        k_cache[at] = rope_elem(x, xp, d, p, ra.inv_freq, ra.amp);
      } else {
        float x = q[((int64_t)n_head + n_head / n_rep + g) * ATTN_D + d];  // v rows follow the n_kv k rows
        if (ra.bv) x += ra.bv[(int64_t)g * ATTN_D + d];
        v_cache[at] = x;
      }
    }
  } else {
    for (int i = t; i < n_rep * ATTN_D; i += ATTN_THREADS)
      qs[i / ATTN_D][i % ATTN_D] = q[((int64_t)g * n_rep + i / ATTN_D) * ATTN_D + i % ATTN_D];
  }
  __syncthreads();  // q staged; the appended k / v rows visible to the workgroup's loads
  const int wave = t >> 6, lane = t & 63, kg = lane >> 4, dq = lane & 15;
  const float* kb = k_cache + ((int64_t)g * ctx_max + lo + k0) * ATTN_D;
  const float* vb = v_cache + ((int64_t)g * ctx_max + lo + k0) * ATTN_D + 4 * dq;
  float m[HPW], l[HPW];
  v4f acc[HPW];
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
    acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  for (int r0 = 0; r0 < nk; r0 += 64) {
    const int n = min(64, nk - r0);
    const bool valid = lane < n;
    // All of the round's loads go out together; rows past the round's keys
    // are clamped to its last key and get weight 0.
    const v4f* kr = (const v4f*)(kb + (int64_t)(r0 + (valid ? lane : n - 1)) * ATTN_D);
    v4f kv[ATTN_D / 4];
#pragma unroll
    for (int d4 = 0; d4 < ATTN_D / 4; ++d4) kv[d4] = kr[d4];
    v4f vd[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) vd[u] = *(const v4f*)(vb + (int64_t)(r0 + min(kg + 4 * u, n - 1)) * ATTN_D);
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int h = wave + i * NW;
      float e = 0.f, corr = 1.f;
      if (h < n_rep) {
        float a = 0.f;
#pragma unroll
        for (int d4 = 0; d4 < ATTN_D / 4; ++d4) {
          const v4f qv = *(const v4f*)&qs[h][4 * d4];
          a = fmaf(qv.x, kv[d4].x, a); a = fmaf(qv.y, kv[d4].y, a);
          a = fmaf(qv.z, kv[d4].z, a); a = fmaf(qv.w, kv[d4].w, a);
        }
        const float sc = valid ? a * scale : -INFINITY;
        const float mn = fmaxf(m[i], wave_max(sc));  // finite: lane 0 holds a key
        e = valid ? expf(sc - mn) : 0.f;
        corr = expf(m[i] - mn);  // 0 on the first round (m = -inf)
        l[i] = fmaf(l[i], corr, wave_sum(e));
        m[i] = mn;
      }
      acc[i] *= corr;
      wl[wave][i][(lane & 3) * 16 + (lane >> 2)] = e;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
#pragma unroll
      for (int u4 = 0; u4 < 4; ++u4) {
        const v4f e = *(const v4f*)&wl[wave][i][kg * 16 + 4 * u4];  // keys kg + 4 * (4 * u4 + 0..3)
        acc[i] += e.x * vd[4 * u4];
        acc[i] += e.y * vd[4 * u4 + 1];
        acc[i] += e.z * vd[4 * u4 + 2];
        acc[i] += e.w * vd[4 * u4 + 3];
      }
    }
    __builtin_amdgcn_wave_barrier();  // reads done before the next round's writes
  }
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const int h = wave + i * NW;
    if (h >= n_rep) continue;
    v4f a = acc[i];
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
      a.x += __shfl_xor(a.x, o, 64);
      a.y += __shfl_xor(a.y, o, 64);
      a.z += __shfl_xor(a.z, o, 64);
      a.w += __shfl_xor(a.w, o, 64);
    }
    if (kg != 0) continue;
    const int hq = g * n_rep + h;
    if constexpr (FINAL) {  // the combine kernel's arithmetic for a single chunk
      const float sink = sinks ? sinks[hq] : -INFINITY;
      const float M = fmaxf(sink, m[i]);
      const float w = expf(m[i] - M);
      const float Z = fmaf(w, l[i], sinks ? expf(sink - M) : 0.f);
      *(v4f*)(out + (int64_t)hq * ATTN_D + 4 * dq) =
          v4f{(w * a.x) / Z, (w * a.y) / Z, (w * a.z) / Z, (w * a.w) / Z};
    } else {
      float* o = part + ((int64_t)hq * nchunk + c) * (ATTN_D + 2);
      if (dq == 0) {
        o[0] = m[i];
        o[1] = l[i];
      }
      float* od = o + 2 + 4 * dq;  // 8-byte aligned only: scalar stores
      od[0] = a.x;
      od[1] = a.y;
      od[2] = a.z;
      od[3] = a.w;
    }
  }
}

// One wave per query head: merge the chunks in order with the sink
// (softmax over [scores, sink], the sink column dropped).
__global__ __launch_bounds__(64) void attn_combine_kernel(
    const float* __restrict__ part, const float* __restrict__ sinks, const int32_t* __restrict__ pos_ptr,
    int64_t ctx_max, int window, int nchunk, float* __restrict__ out) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int p = *pos_ptr;
  if (p < 0 || p >= ctx_max) return;
  int lo, total;
  attn_span(p, window, lo, total);
  const int nc = (total + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const float* ph = part + (int64_t)h * nchunk * (ATTN_D + 2);
  const float sink = sinks ? sinks[h] : -INFINITY;
  float M = sink;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, ph[(int64_t)c * (ATTN_D + 2)]);
  float Z = sinks ? expf(sink - M) : 0.f, acc = 0.f;
  for (int c = 0; c < nc; ++c) {
    const float* pc = ph + (int64_t)c * (ATTN_D + 2);
    const float w = expf(pc[0] - M);
    Z = fmaf(w, pc[1], Z);
    acc = fmaf(w, pc[2 + d], acc);
  }
  out[(int64_t)h * ATTN_D + d] = acc / Z;
}

__global__ void pos_advance_kernel(int32_t* pos, int32_t n) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *pos += n;
}

}  // namespace

static inline hipStream_t S(void* s) { return (hipStream_t)s; }

extern "C" int nsx_rope_kv_append(float* qkv, const float* q_bias, const float* k_bias, const float* v_bias,
                                  int n_head, int n_kv, int head_dim, const float* inv_freq, float amplitude,
                                  const int32_t* pos, float* k_cache, float* v_cache, int64_t ctx_max,
                                  void* stream) {
  NSX_REQUIRE(head_dim == ATTN_D, NSX_ENOTIMPL, "head_dim %d (the kernels are written for 64)", head_dim);
  NSX_REQUIRE(n_head > 0 && n_kv > 0 && n_head % n_kv == 0 && n_head / n_kv <= ATTN_MAX_REP, NSX_EINVAL,
              "n_head=%d, n_kv=%d: n_head must be a multiple of n_kv, at most %d per kv head", n_head, n_kv,
              ATTN_MAX_REP);
  NSX_REQUIRE(ctx_max > 0 && ctx_max < (1ll << 31), NSX_EINVAL, "ctx_max=%lld", (long long)ctx_max);
  NSX_REQUIRE(qkv && inv_freq && pos && k_cache && v_cache, NSX_EINVAL, "null buffer");
  hipLaunchKernelGGL(rope_kv_append_kernel, dim3(n_head + 2 * n_kv), dim3(64), 0, S(stream), qkv, q_bias, k_bias,
                     v_bias, n_head, n_kv, inv_freq, amplitude, pos, k_cache, v_cache, ctx_max);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int64_t nsx_attn_workspace_bytes(int n_head, int head_dim, int64_t ctx_max) {
  if (head_dim != ATTN_D || n_head <= 0 || ctx_max <= 0) return -1;
  const int64_t nchunk = nsx_cdiv(ctx_max, ATTN_CHUNK);
  return (int64_t)n_head * nchunk * (ATTN_D + 2) * (int64_t)sizeof(float);
}

// Checks shared by both attention entry points, then the chunk launches
// (and the combine unless one chunk covers every position).
static int attn_launch(const float* q, float* k_cache, float* v_cache, const float* sinks, int n_head, int n_kv,
                       int head_dim, const int32_t* pos, int64_t ctx_max, int window, float scale,
                       void* workspace, float* out, bool rope, const RopeArgs& ra, hipStream_t st) {
  NSX_REQUIRE(head_dim == ATTN_D, NSX_ENOTIMPL, "head_dim %d (the kernels are written for 64)", head_dim);
  NSX_REQUIRE(n_head > 0 && n_kv > 0 && n_head % n_kv == 0 && n_head / n_kv <= ATTN_MAX_REP, NSX_EINVAL,
              "n_head=%d, n_kv=%d: n_head must be a multiple of n_kv, at most %d per kv head", n_head, n_kv,
              ATTN_MAX_REP);
  NSX_REQUIRE(ctx_max > 0 && ctx_max < (1ll << 31) && window >= 0, NSX_EINVAL, "ctx_max=%lld window=%d",
              (long long)ctx_max, window);
  NSX_REQUIRE(q && k_cache && v_cache && pos && workspace && out, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) % 16 == 0, NSX_EINVAL,
              "q, the caches and out must be 16-byte aligned");
  const int nchunk = (int)nsx_cdiv(ctx_max, ATTN_CHUNK);
  // a sliding window bounds the keys: only its chunks can be live
  const int live = window > 0 ? (int)std::min<int64_t>(nchunk, nsx_cdiv(window, ATTN_CHUNK)) : nchunk;
  const int n_rep = n_head / n_kv;
  const int hpw = (n_rep + ATTN_THREADS / 64 - 1) / (ATTN_THREADS / 64);
  auto chunks = [&](auto final_tag, auto hpw_tag, auto rope_tag) {
    constexpr bool F = decltype(final_tag)::value;
    hipLaunchKernelGGL((attn_chunk_kernel<F, decltype(hpw_tag)::value, decltype(rope_tag)::value>),
                       dim3(n_kv, F ? 1 : live), dim3(ATTN_THREADS), 0, st, q, k_cache, v_cache, pos, ctx_max,
                       window, scale, n_rep, n_head, nchunk, (float*)workspace, sinks, out, ra);
  };
  auto by_rope = [&](auto final_tag, auto hpw_tag) {
    if (rope) chunks(final_tag, hpw_tag, std::true_type{});
    else chunks(final_tag, hpw_tag, std::false_type{});
  };
  auto by_hpw = [&](auto final_tag) {
    switch (hpw) {
      case 1: by_rope(final_tag, std::integral_constant<int, 1>{}); break;
      case 2: by_rope(final_tag, std::integral_constant<int, 2>{}); break;
      case 3: by_rope(final_tag, std::integral_constant<int, 3>{}); break;
      default: by_rope(final_tag, std::integral_constant<int, 4>{}); break;
    }
  };
  if (live == 1) {  // one chunk at any position: no partials, no combine launch
    by_hpw(std::true_type{});
    NSX_LAUNCHED();
    return NSX_OK;
  }
  by_hpw(std::false_type{});
  NSX_LAUNCHED();
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_head), dim3(64), 0, st, (const float*)workspace, sinks, pos,
                     ctx_max, window, nchunk, out);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int nsx_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* sinks,
                               int n_head, int n_kv, int head_dim, const int32_t* pos, int64_t ctx_max,
                               int window, float scale, void* workspace, float* out, void* stream) {
  // the caches are only read on this path
  return attn_launch(q, const_cast<float*>(k_cache), const_cast<float*>(v_cache), sinks, n_head, n_kv, head_dim,
                     pos, ctx_max, window, scale, workspace, out, false, RopeArgs{}, S(stream));
}

extern "C" int nsx_attn_decode_qkv(const float* qkv, const float* q_bias, const float* k_bias, const float* v_bias,
                                   const float* inv_freq, float amplitude, const float* sinks, int n_head, int n_kv,
                                   int head_dim, const int32_t* pos, float* k_cache, float* v_cache,
                                   int64_t ctx_max, int window, float scale, void* workspace, float* out,
                                   void* stream) {
  NSX_REQUIRE(inv_freq, NSX_EINVAL, "null inv_freq");
  return attn_launch(qkv, k_cache, v_cache, sinks, n_head, n_kv, head_dim, pos, ctx_max, window, scale, workspace,
                     out, true, RopeArgs{q_bias, k_bias, v_bias, inv_freq, amplitude}, S(stream));
}

extern "C" int nsx_pos_advance(int32_t* pos, int32_t n, void* stream) {
  NSX_REQUIRE(pos, NSX_EINVAL, "null position");
  hipLaunchKernelGGL(pos_advance_kernel, dim3(1), dim3(64), 0, S(stream), pos, n);
  NSX_LAUNCHED();
  return NSX_OK;
}
