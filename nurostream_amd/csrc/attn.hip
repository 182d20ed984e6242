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
// combine kernel merges the chunks in chunk order together with the sink.
// Both grids are sized for ctx_max, so their shape does not depend on the
// position; chunks past the current length return at once.
#include "nsx_common.h"

#include <algorithm>
#include <math.h>

namespace {

constexpr int ATTN_D = 64;        // head_dim (GPT-OSS)
constexpr int ATTN_CHUNK = 256;   // keys per attention workgroup
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
  // rotate_half pairing: element i with i + D/2 (gpt_oss.py:42-58, ops.py:95-104)
  const int i = lane & (ATTN_D / 2 - 1);
  const float ang = (float)p * inv_freq[i];  // fp32, as positions.float() * inv
  float s, c;
  sincosf(ang, &s, &c);
  c *= amp;
  s *= amp;
  const float partner = __shfl_xor(x, ATTN_D / 2, 64);
  const float y = lane < ATTN_D / 2 ? x * c - partner * s : x * c + partner * s;
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

// Workgroup (kv head g, chunk c): scores of its n_rep query heads against
// the chunk's keys, the chunk's softmax statistics, and the value sums.
// part[(h * nchunk + c) * (D + 2)] = {m, l, acc[D]} for query head h.
__global__ __launch_bounds__(ATTN_THREADS) void attn_chunk_kernel(
    const float* __restrict__ q, const float* __restrict__ k_cache, const float* __restrict__ v_cache,
    const int32_t* __restrict__ pos_ptr, int64_t ctx_max, int window, float scale, int n_rep, int nchunk,
    float* __restrict__ part) {
  __shared__ float qs[ATTN_MAX_REP][ATTN_D];
  __shared__ float sc[ATTN_MAX_REP][ATTN_CHUNK];
  __shared__ float ml[ATTN_MAX_REP][2];
  const int g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  const int p = *pos_ptr;
  if (p < 0 || p >= ctx_max) return;
  int lo, total;
  attn_span(p, window, lo, total);
  const int k0 = c * ATTN_CHUNK;
  if (k0 >= total) return;  // past the current length
  const int nk = min(ATTN_CHUNK, total - k0);
  for (int i = t; i < n_rep * ATTN_D; i += ATTN_THREADS)
    qs[i / ATTN_D][i % ATTN_D] = q[((int64_t)g * n_rep + i / ATTN_D) * ATTN_D + i % ATTN_D];
  __syncthreads();
  // scores: one key per thread, all of its query heads
  {
    float acc[ATTN_MAX_REP];
#pragma unroll
    for (int h = 0; h < ATTN_MAX_REP; ++h) acc[h] = 0.f;
    if (t < nk) {
      const v4f* kr = (const v4f*)(k_cache + ((int64_t)g * ctx_max + lo + k0 + t) * ATTN_D);
#pragma unroll 4
      for (int d4 = 0; d4 < ATTN_D / 4; ++d4) {
        const v4f kv = kr[d4];
#pragma unroll
        for (int h = 0; h < ATTN_MAX_REP; ++h) {
          if (h < n_rep) {
            const v4f qv = *(const v4f*)&qs[h][4 * d4];
            float a = acc[h];
            a = fmaf(qv.x, kv.x, a); a = fmaf(qv.y, kv.y, a); a = fmaf(qv.z, kv.z, a); a = fmaf(qv.w, kv.w, a);
            acc[h] = a;
          }
        }
      }
    }
    for (int h = 0; h < n_rep; ++h) sc[h][t] = t < nk ? acc[h] * scale : -INFINITY;
  }
  __syncthreads();
  // softmax statistics of the chunk: wave w takes heads w, w + 4, ...
  const int wave = t >> 6, lane = t & 63;
  for (int h = wave; h < n_rep; h += ATTN_THREADS / 64) {
    float m = -INFINITY;
    for (int j = lane; j < ATTN_CHUNK; j += 64) m = fmaxf(m, sc[h][j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < ATTN_CHUNK; j += 64) {
      const float e = j < nk ? expf(sc[h][j] - m) : 0.f;
      sc[h][j] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml[h][0] = m;
      ml[h][1] = l;
    }
  }
  __syncthreads();
  // value sums: thread (head slot, d), keys in order
  const int d = t & (ATTN_D - 1);
  for (int h = t / ATTN_D; h < n_rep; h += ATTN_THREADS / ATTN_D) {
    float a = 0.f;
    const float* vr = v_cache + ((int64_t)g * ctx_max + lo + k0) * ATTN_D + d;
    for (int j = 0; j < nk; ++j) a = fmaf(sc[h][j], vr[(int64_t)j * ATTN_D], a);
    float* o = part + ((int64_t)(g * n_rep + h) * nchunk + c) * (ATTN_D + 2);
    if (d == 0) {
      o[0] = ml[h][0];
      o[1] = ml[h][1];
    }
    o[2 + d] = a;
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

extern "C" int nsx_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* sinks,
                               int n_head, int n_kv, int head_dim, const int32_t* pos, int64_t ctx_max,
                               int window, float scale, void* workspace, float* out, void* stream) {
  NSX_REQUIRE(head_dim == ATTN_D, NSX_ENOTIMPL, "head_dim %d (the kernels are written for 64)", head_dim);
  NSX_REQUIRE(n_head > 0 && n_kv > 0 && n_head % n_kv == 0 && n_head / n_kv <= ATTN_MAX_REP, NSX_EINVAL,
              "n_head=%d, n_kv=%d: n_head must be a multiple of n_kv, at most %d per kv head", n_head, n_kv,
              ATTN_MAX_REP);
  NSX_REQUIRE(ctx_max > 0 && ctx_max < (1ll << 31) && window >= 0, NSX_EINVAL, "ctx_max=%lld window=%d",
              (long long)ctx_max, window);
  NSX_REQUIRE(q && k_cache && v_cache && pos && workspace && out, NSX_EINVAL, "null buffer");
  const int nchunk = (int)nsx_cdiv(ctx_max, ATTN_CHUNK);
  // a sliding window bounds the keys: only its chunks can be live
  const int live = window > 0 ? (int)std::min<int64_t>(nchunk, nsx_cdiv(window, ATTN_CHUNK)) : nchunk;
  const int n_rep = n_head / n_kv;
  hipLaunchKernelGGL(attn_chunk_kernel, dim3(n_kv, live), dim3(ATTN_THREADS), 0, S(stream), q, k_cache, v_cache,
                     pos, ctx_max, window, scale, n_rep, nchunk, (float*)workspace);
  NSX_LAUNCHED();
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_head), dim3(64), 0, S(stream), (const float*)workspace, sinks, pos,
                     ctx_max, window, nchunk, out);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int nsx_pos_advance(int32_t* pos, int32_t n, void* stream) {
  NSX_REQUIRE(pos, NSX_EINVAL, "null position");
  hipLaunchKernelGGL(pos_advance_kernel, dim3(1), dim3(64), 0, S(stream), pos, n);
  NSX_LAUNCHED();
  return NSX_OK;
}
