// Dequantization, raw-GGUF fused GEMV, and the t64 tile layout (gfx950).
//
// Semantics follow the reference's compute/quant.py (dequantize, bit-exact)
// and compute/triton_kernels.py fused_gemv (fp32 accumulate); the kernels
// themselves are written for CDNA4: wave64, buffer loads with hardware range
// checking, the gfx950 FP4 conversion instruction, and wave reductions.
#include "nsx_common.h"
#include "mx.h"
#include "raw_dot.h"

#include <algorithm>
#include <mutex>
#include <string.h>

// ---------------------------------------------------------------------------
// error state

static thread_local char g_err[512] = "";

int nsx_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* nsx_last_error(void) { return g_err; }
extern "C" int nsx_abi_version(void) { return NSX_ABI_VERSION; }

static inline hipStream_t S(void* s) { return (hipStream_t)s; }

// ---------------------------------------------------------------------------
// FP4 conversion self test: v_cvt_scalef32_pk_f32_fp4 with scale 1.0 must give
// the e2m1 value of the low nibble in .x and of the high nibble in .y for the
// byte selected by the third operand.

__global__ void selftest_zero_kernel(uint32_t* bad) { *bad = 0; }

__global__ void selftest_kernel(uint32_t* bad) {
  const uint32_t b = threadIdx.x;  // 256 threads, one byte value each
  const uint32_t word = b << 16;   // byte 2
  v2f c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 2);
  const float lo = kE2M1x2[b & 15] * 0.5f, hi = kE2M1x2[b >> 4] * 0.5f;
  // code 8 may decode to -0.0; compare values, not bits
  if (c.x != lo || c.y != hi) atomicAdd(bad, 1u);
}

extern "C" int nsx_selftest(uint32_t* scratch, void* stream) {
  NSX_REQUIRE(scratch, NSX_EINVAL, "null scratch word");
  hipLaunchKernelGGL(selftest_zero_kernel, dim3(1), dim3(1), 0, S(stream), scratch);
  NSX_LAUNCHED();
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(256), 0, S(stream), scratch);
  NSX_LAUNCHED();
  uint32_t bad = 0;
  NSX_HIP(hipMemcpyAsync(&bad, scratch, sizeof bad, hipMemcpyDeviceToHost, S(stream)));
  NSX_HIP(hipStreamSynchronize(S(stream)));
  NSX_REQUIRE(bad == 0, NSX_EKERNEL, "fp4 conversion self test: %u byte values decoded wrongly", bad);
  return NSX_OK;
}

// ---------------------------------------------------------------------------
// Read-bandwidth probe: the denominator the expert kernels' HBM fractions are
// read against on the same box. Workgroup b reads bytes [b * per, (b + 1) *
// per) of src with 16-byte nontemporal loads, PROBE_U per thread in flight
// at once (as the expert kernels issue their weight loads), and folds them
// into one word that is stored only if it equals a constant no input of
// interest produces -- so the loads cannot be dropped and nothing is written.

constexpr int PROBE_U = 8;

__global__ __launch_bounds__(1024) void read_probe_kernel(const v4u* __restrict__ src, int64_t n16, int64_t per16,
                                                          uint32_t* __restrict__ sink) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  const int64_t lo = (int64_t)blockIdx.x * per16;
  const int64_t hi = min(lo + per16, n16);
  const int64_t step = (int64_t)blockDim.x * PROBE_U;
  uint32_t acc = 0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += step) {
    v4u v[PROBE_U];
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) {
      const int64_t j = min(i + (int64_t)u * blockDim.x, hi - 1);  // in bounds; duplicates past hi are discarded
      v[u] = __builtin_nontemporal_load((gv4u*)(src + j));
    }
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u)
      acc ^= i + (int64_t)u * blockDim.x < hi ? (v[u].x ^ v[u].y ^ v[u].z ^ v[u].w) : 0u;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

extern "C" int nsx_read_probe(const void* src, int64_t bytes, int workgroups, int threads, uint32_t* sink,
                              void* stream) {
  NSX_REQUIRE(src && sink, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(bytes >= 16 && bytes % 16 == 0 && ((uintptr_t)src & 15u) == 0, NSX_EINVAL,
              "the probe reads 16-byte aligned whole 16-byte units (%lld bytes)", (long long)bytes);
  NSX_REQUIRE(workgroups >= 1 && workgroups <= (1 << 20), NSX_EINVAL, "workgroups=%d", workgroups);
  NSX_REQUIRE(threads >= 64 && threads <= 1024 && threads % 64 == 0, NSX_EINVAL, "threads=%d", threads);
  const int64_t n16 = bytes / 16;
  const int64_t per16 = nsx_cdiv(n16, workgroups);
  return nsx_launch(read_probe_kernel, dim3((unsigned)workgroups), dim3((unsigned)threads), 0, S(stream),
                    (const v4u*)src, n16, per16, sink);
}

// ---------------------------------------------------------------------------
// dequantize (quant.py:118-140, 24-56, 84-107, 110-115)
//
// A workgroup stages BPW consecutive blocks into LDS with range-checked dword
// buffer loads (the source may start at any byte), then each thread expands
// four consecutive elements and writes them with one vector store.

constexpr int DQ_THREADS = 256;

template <int FMT>
struct Fmt;
template <> struct Fmt<NSX_MXFP4> { static constexpr int BE = 32, BB = 17, BPW = 32; };
template <> struct Fmt<NSX_Q4_0> { static constexpr int BE = 32, BB = 18, BPW = 32; };
template <> struct Fmt<NSX_Q8_0> { static constexpr int BE = 32, BB = 34, BPW = 32; };
template <> struct Fmt<NSX_Q4_K> { static constexpr int BE = 256, BB = 144, BPW = 4; };
template <> struct Fmt<NSX_Q6_K> { static constexpr int BE = 256, BB = 210, BPW = 4; };

template <int FMT>
__device__ __forceinline__ float dq_elem(const uint8_t* B, int blk, int j) {
  constexpr int BB = Fmt<FMT>::BB;
  const uint8_t* p = B + blk * BB;
  if constexpr (FMT == NSX_MXFP4) {
    const float scale = nsx_mx_scale_half(p[0]);
    const uint32_t q = p[1 + (j & 15)];
    const uint32_t code = j < 16 ? (q & 15u) : (q >> 4);
    return __fmul_rn(scale, kE2M1x2[code]);
  } else if constexpr (FMT == NSX_Q4_0) {
    const float d = nsx_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    const uint32_t q = p[2 + (j & 15)];
    const int v = (int)(j < 16 ? (q & 15u) : (q >> 4)) - 8;
    return __fmul_rn(d, (float)v);
  } else if constexpr (FMT == NSX_Q8_0) {
    const float d = nsx_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    const int v = (int)(int8_t)p[2 + j];
    return __fmul_rn(d, (float)v);
  } else if constexpr (FMT == NSX_Q6_K) {
    // element j = 128 h + 32 L + l: low 4 bits from ql[64 h + 32 (L & 1) + l]
    // (nibble L >> 1), high 2 bits from qh[32 h + l] >> 2L, scale int8
    // sc[j / 16], d fp16 at byte 208. d * sc * (q - 32) is exact in fp32
    // (11 + 7 + 5 significant bits), so the product order does not matter.
    const int h = j >> 7, L = (j >> 5) & 3, l = j & 31;
    const uint32_t lo = (p[64 * h + 32 * (L & 1) + l] >> (4 * (L >> 1))) & 15u;
    const uint32_t hi = (p[128 + 32 * h + l] >> (2 * L)) & 3u;
    const float d = nsx_h2f((uint32_t)p[208] | ((uint32_t)p[209] << 8));
    const float sc = (float)(int8_t)p[192 + (j >> 4)];
    return __fmul_rn(__fmul_rn(d, sc), (float)((int)(lo | (hi << 4)) - 32));
  } else {  // Q4_K
    const float d = nsx_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    const float dmin = nsx_h2f((uint32_t)p[2] | ((uint32_t)p[3] << 8));
    const int s = j >> 5, l = j & 31;
    uint32_t sc, m;
    nsx_q4k_scale_min(p + 4, s, sc, m);
    const uint32_t q = (p[16 + (s >> 1) * 32 + l] >> (4 * (s & 1))) & 15u;
    const float scale = __fmul_rn(d, (float)sc);   // exact
    const float off = __fmul_rn(dmin, (float)m);   // exact
    return __fsub_rn(__fmul_rn(scale, (float)q), off);  // one rounding
  }
}

template <int FMT, int OUT>
__global__ __launch_bounds__(DQ_THREADS) void dequant_kernel(
    const uint8_t* __restrict__ base, uint32_t head, uint32_t range, int64_t n_blocks,
    int64_t n_elements, void* __restrict__ out) {
  constexpr int BE = Fmt<FMT>::BE, BB = Fmt<FMT>::BB, BPW = Fmt<FMT>::BPW;
  constexpr int CHUNK = BPW * BB;
  constexpr int NDW = (CHUNK + 3) / 4 + 1;
  __shared__ uint32_t smem[NDW];

  const int64_t blk0 = (int64_t)blockIdx.x * BPW;
  if (blk0 >= n_blocks) return;
  const __amdgpu_buffer_rsrc_t rs = nsx_rsrc(base, range);
  const uint32_t c0 = head + (uint32_t)(blk0 * BB);  // byte offset of the chunk from `base`
  const uint32_t c0a = c0 & ~3u;
  for (int i = threadIdx.x; i < NDW; i += DQ_THREADS) smem[i] = nsx_bload32(rs, c0a + 4u * i);
  __syncthreads();
  const uint8_t* B = (const uint8_t*)smem + (c0 - c0a);

  const int nblk = (int)(n_blocks - blk0 < BPW ? n_blocks - blk0 : BPW);
  const int64_t e0 = blk0 * BE;
  for (int q = threadIdx.x; q < nblk * BE / 4; q += DQ_THREADS) {
    const int i = q * 4;
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = dq_elem<FMT>(B, (i + u) / BE, (i + u) % BE);
    const int64_t g = e0 + i;
    if (g >= n_elements) break;
    if (OUT == NSX_DT_F32) {
      float* o = (float*)out + g;
      if (g + 4 <= n_elements) {
        *(v4f*)o = v4f{v[0], v[1], v[2], v[3]};
      } else {
        for (int u = 0; u < 4 && g + u < n_elements; ++u) o[u] = v[u];
      }
    } else {
      uint16_t h[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        // round to fp32 first, exactly as the reference's `.to(out_dtype)` on a
        // float32 tensor: the barrier stops a fused multiply-to-half (v_fma_mix)
        float f = v[u];
        asm volatile("" : "+v"(f));
        h[u] = (uint16_t)(OUT == NSX_DT_F16 ? nsx_f2h(f) : nsx_f2bf(f));
      }
      uint16_t* o = (uint16_t*)out + g;
      if (g + 4 <= n_elements) {
        *(v2u*)o = v2u{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
      } else {
        for (int u = 0; u < 4 && g + u < n_elements; ++u) o[u] = h[u];
      }
    }
  }
}

template <int FMT, int OUT>
static int launch_dequant(const void* raw, int64_t n_blocks, int64_t n_elements, void* out,
                          hipStream_t st) {
  constexpr int BB = Fmt<FMT>::BB, BPW = Fmt<FMT>::BPW, BE = Fmt<FMT>::BE;
  // Split so that every launch's byte range fits a 32-bit buffer range.
  const int64_t max_blocks = ((int64_t)1 << 30) / BB / BPW * BPW;
  for (int64_t b0 = 0; b0 < n_blocks; b0 += max_blocks) {
    const int64_t nb = std::min(max_blocks, n_blocks - b0);
    const uint8_t* p = (const uint8_t*)raw + b0 * BB;
    const uintptr_t a = (uintptr_t)p & ~(uintptr_t)3;
    const uint32_t head = (uint32_t)((uintptr_t)p - a);
    const uint32_t range = head + (uint32_t)(nb * BB);
    const int64_t ne = std::min(n_elements - b0 * BE, nb * BE);
    if (ne <= 0) break;
    const size_t esz = OUT == NSX_DT_F32 ? 4 : 2;
    void* o = (char*)out + b0 * BE * esz;
    hipLaunchKernelGGL((dequant_kernel<FMT, OUT>), dim3((unsigned)nsx_cdiv(nb, BPW)), dim3(DQ_THREADS), 0,
                       st, (const uint8_t*)a, head, range, nb, ne, o);
    NSX_LAUNCHED();
  }
  return NSX_OK;
}

template <int FMT>
static int dequant_fmt(const void* raw, int64_t nb, int64_t ne, void* out, int odt, hipStream_t st) {
  switch (odt) {
    case NSX_DT_F32: return launch_dequant<FMT, NSX_DT_F32>(raw, nb, ne, out, st);
    case NSX_DT_F16: return launch_dequant<FMT, NSX_DT_F16>(raw, nb, ne, out, st);
    case NSX_DT_BF16: return launch_dequant<FMT, NSX_DT_BF16>(raw, nb, ne, out, st);
  }
  return nsx_fail(NSX_EINVAL, "unsupported output dtype %d", odt);
}

extern "C" int nsx_dequantize(int t, const void* raw, int64_t raw_bytes, int64_t n_elements,
                              void* out, int out_dtype, void* stream) {
  const int BE = nsx_block_elems(t), BB = nsx_block_bytes(t);
  NSX_REQUIRE(BB > 0, NSX_ENOTIMPL, "no dequant kernel for ggml type %d; supported: Q4_0 Q8_0 Q4_K Q6_K MXFP4", t);
  NSX_REQUIRE(raw_bytes >= 0 && n_elements >= 0, NSX_EINVAL, "negative size");
  const int64_t nb = raw_bytes / BB;
  NSX_REQUIRE(n_elements <= nb * BE, NSX_EINVAL, "%lld elements requested from %lld blocks",
              (long long)n_elements, (long long)nb);
  if (n_elements == 0) return NSX_OK;
  NSX_REQUIRE(raw && out, NSX_EINVAL, "null buffer");
  const int64_t need = nsx_cdiv(n_elements, BE);
  hipStream_t st = S(stream);
  switch (t) {
    case NSX_MXFP4: return dequant_fmt<NSX_MXFP4>(raw, need, n_elements, out, out_dtype, st);
    case NSX_Q4_0: return dequant_fmt<NSX_Q4_0>(raw, need, n_elements, out, out_dtype, st);
    case NSX_Q8_0: return dequant_fmt<NSX_Q8_0>(raw, need, n_elements, out, out_dtype, st);
    case NSX_Q4_K: return dequant_fmt<NSX_Q4_K>(raw, need, n_elements, out, out_dtype, st);
    case NSX_Q6_K: return dequant_fmt<NSX_Q6_K>(raw, need, n_elements, out, out_dtype, st);
  }
  return nsx_fail(NSX_ENOTIMPL, "ggml type %d", t);
}

// ---------------------------------------------------------------------------
// row gather + dequantize (compute/blockffn.py:470-487 gather_embeddings):
// one workgroup per requested row, the row id read from device memory so a
// captured decode step can take the next token from a device buffer. An id
// outside [0, n_rows) gives a row of zeros.

template <int FMT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ raw, int64_t row_bytes,
                                                           int64_t n_rows, const int32_t* __restrict__ ids, int K,
                                                           float* __restrict__ out) {
  const int64_t i = blockIdx.x;
  const int id = ids[i];
  const bool valid = id >= 0 && id < n_rows;
  const uint8_t* p = raw + (valid ? (int64_t)id : 0) * row_bytes;
  for (int j = threadIdx.x; j < K; j += blockDim.x) {
    float v = 0.f;
    if (valid) {
      if constexpr (FMT == NSX_F32) {
        v = ((const float*)p)[j];
      } else if constexpr (FMT == NSX_F16) {
        v = nsx_h2f(((const uint16_t*)p)[j]);
      } else if constexpr (FMT == NSX_BF16) {
        v = nsx_bf2f(((const uint16_t*)p)[j]);
      } else {
        constexpr int BE = Fmt<FMT>::BE;
        v = dq_elem<FMT>(p, j / BE, j % BE);
      }
    }
    out[i * K + j] = v;
  }
}

extern "C" int nsx_dequantize_rows(int t, const void* raw, int64_t n_rows, int64_t K, const int32_t* ids,
                                   int64_t n_ids, float* out, void* stream) {
  NSX_REQUIRE(n_rows >= 0 && K > 0 && n_ids >= 0 && n_ids < (1ll << 31) && K < (1ll << 30), NSX_EINVAL,
              "bad shape");
  int64_t row_bytes = 0;
  if (t == NSX_F32) row_bytes = K * 4;
  else if (t == NSX_F16 || t == NSX_BF16) row_bytes = K * 2;
  else {
    const int BE = nsx_block_elems(t), BB = nsx_block_bytes(t);
    NSX_REQUIRE(BB > 0, NSX_ENOTIMPL, "no dequant kernel for ggml type %d", t);
    NSX_REQUIRE(K % BE == 0, NSX_EINVAL, "K=%lld is not a multiple of the %d-element block", (long long)K, BE);
    row_bytes = K / BE * BB;
  }
  if (n_ids == 0) return NSX_OK;
  NSX_REQUIRE(raw && ids && out, NSX_EINVAL, "null buffer");
  if ((t == NSX_F32 && ((uintptr_t)raw & 3)) || ((t == NSX_F16 || t == NSX_BF16) && ((uintptr_t)raw & 1)))
    return nsx_fail(NSX_EINVAL, "float rows must be aligned to their element size");
  const dim3 g((unsigned)n_ids), b(256);
  const uint8_t* r = (const uint8_t*)raw;
  hipStream_t st = S(stream);
  switch (t) {
    case NSX_F32: hipLaunchKernelGGL(dequant_rows_kernel<NSX_F32>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_F16: hipLaunchKernelGGL(dequant_rows_kernel<NSX_F16>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_BF16: hipLaunchKernelGGL(dequant_rows_kernel<NSX_BF16>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_MXFP4: hipLaunchKernelGGL(dequant_rows_kernel<NSX_MXFP4>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_Q4_0: hipLaunchKernelGGL(dequant_rows_kernel<NSX_Q4_0>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_Q8_0: hipLaunchKernelGGL(dequant_rows_kernel<NSX_Q8_0>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_Q4_K: hipLaunchKernelGGL(dequant_rows_kernel<NSX_Q4_K>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    case NSX_Q6_K: hipLaunchKernelGGL(dequant_rows_kernel<NSX_Q6_K>, g, b, 0, st, r, row_bytes, n_rows, ids, (int)K, out); break;
    default: return nsx_fail(NSX_ENOTIMPL, "ggml type %d", t);
  }
  NSX_LAUNCHED();
  return NSX_OK;
}

// ---------------------------------------------------------------------------
// fused GEMV on raw GGUF rows (triton_kernels.py:199-228 seam)
//
// One wave per row; lanes take the row's 32-element units (raw_dot.h) and the
// wave reduces. A row is processed in chunks of up to 128 units (4096
// elements). Each chunk's bytes are read with coalesced 16-byte buffer loads
// (lane i takes bytes 16 i .., so one load instruction covers 1 KiB of
// consecutive bytes) into registers, written to a wave-private LDS buffer,
// and the lanes then read their units' fields from LDS: unit-per-lane global
// loads would touch many cache lines per instruction and revisit each line
// once per field. The loads of the wave's next chunk are issued before the
// arithmetic of the current one, so they overlap it. The grid is persistent
// (as many workgroups as fit at once): x is staged into LDS once per
// workgroup.

constexpr int GV_THREADS = 256;
constexpr int GV_WAVES = GV_THREADS / 64;
constexpr int GV_MAXT = 16;
constexpr int GV_CHUNK_UNITS = 128;
#ifndef GV_DEPTH_OVERRIDE
constexpr int GV_DEPTH = 2;  // chunks whose loads are in flight per wave
#else
constexpr int GV_DEPTH = GV_DEPTH_OVERRIDE;
#endif

template <int FMT>
struct GvChunk {
  static constexpr int BLOCKS = GV_CHUNK_UNITS * 32 / RawBlock<FMT>::BE;  // blocks per chunk
  static constexpr int BYTES = BLOCKS * RawBlock<FMT>::BB;
  static constexpr int LOADS = (BYTES + 3 + 1023) / 1024;  // 16-byte loads per lane
  // wave buffer: the loaded span plus the fetch's reads past the last unit
  static constexpr int WAVE_BYTES = LOADS * 1024 + 64;
};

template <int NT>
__host__ __device__ constexpr int gv_x_bytes(int K) {
  return ((NT * (K + K / 32) * 4) + 15) & ~15;
}
// XREG: x staged once per workgroup, 32-element chunks GV_XPAD floats apart
constexpr int GV_XPAD = 36;
constexpr int GV_XQ = 4;  // float4s of x per thread when staging (K <= 4 * GV_XQ * GV_THREADS)
__host__ __device__ constexpr int gv_xreg_bytes(int K) { return (K / 32) * GV_XPAD * 4; }

// Activations of one unit held in registers (unit order), one token, with
// the unit's sum and its four 8-element group sums.
struct RawXReg {
  static constexpr bool kRegSums = true;
  const float (&x)[32];
  float s;
  const float (&g)[4];
  __device__ __forceinline__ v4f operator()(int, int k4) const {
    return v4f{x[4 * k4], x[4 * k4 + 1], x[4 * k4 + 2], x[4 * k4 + 3]};
  }
  __device__ __forceinline__ float sum() const { return s; }
  __device__ __forceinline__ float gsum(int L) const { return g[L]; }
};
struct RawXSumReg {
  float s;
  __device__ __forceinline__ float operator()(int) const { return s; }
};

// XREG (one token, K <= 4096, so one chunk per row): each lane's two units
// are the same for every row, so their activations are read from LDS once
// into registers instead of once per row.
// The one-token GEMV's input as the residual stream of a block (NORM):
// h = rms_norm(x + r) * w (compute/ops.py:14-20), computed in the prologue the
// way add_rmsnorm_kernel computes it -- 256 threads, thread i holding elements
// i, i + 256, ..., the same sum order -- so h has the bits of that launch,
// which this replaces. The first workgroup writes x + r to s (when r and s are
// set).
struct GvNorm {
  const float* r;  // added to x (null: none)
  const float* w;  // norm weight (null: none)
  float eps;
  float* s;        // x + r out (null: not written); must not overlap x or r
};
constexpr int GV_NORM_MAXV = 16;  // values per thread (K <= 4096)

template <int FMT, int NT, bool XREG, int WAVES = GV_WAVES, bool NORM = false>
__global__ __launch_bounds__(64 * WAVES) void gemv_raw_kernel(
    const uint8_t* __restrict__ base, uint32_t head, uint32_t range, int n_rows, int K,
    const void* __restrict__ x, int x_dtype, int T, float* __restrict__ y, int64_t ystride,
    const float* __restrict__ bias, const float* resid,  // resid may be y (read, then written, per element)
    GvNorm nm = GvNorm{}) {
  static_assert(!NORM || (XREG && WAVES * 64 == 256), "the norm prologue is the one-token 256-thread path's");
  __shared__ float gv_part[NORM ? WAVES : 1];
  using C = GvChunk<FMT>;
  constexpr int BE = RawBlock<FMT>::BE, BB = RawBlock<FMT>::BB;
  extern __shared__ __align__(16) uint8_t gv_smem[];
  // LDS: without XREG, [NT][K] activations and [NT][K/32] block sums; with
  // XREG, x in 32-element chunks at a GV_XPAD-float stride; then one chunk
  // buffer per wave
  float* xs = (float*)gv_smem;
  constexpr bool SUMS = FMT == NSX_Q4_0 || FMT == NSX_Q4_K;
  if constexpr (!XREG) stage_x<NT>(xs, x, x_dtype, K, T, K, SUMS);
  const float* xsum = xs + NT * K;
  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // with XREG the wave buffers overlay the x staging area (x is in registers before any row bytes land)
  uint8_t* wbuf = gv_smem + (XREG ? 0 : gv_x_bytes<NT>(K)) + wave * C::WAVE_BYTES;
  constexpr int THREADS = 64 * WAVES;
  constexpr int XQ = (GV_XQ * GV_THREADS + THREADS - 1) / THREADS;  // float4s of x per thread (K <= 4096)
  const __amdgpu_buffer_rsrc_t rs = nsx_rsrc(base, range);
  const int nwaves = gridDim.x * WAVES;
  const uint32_t rb = raw_row_bytes<FMT>(K);
  const int nblk = K / BE;                        // blocks per row
  const int nch = (nblk + C::BLOCKS - 1) / C::BLOCKS;  // chunks per row

  // Work items of this wave: (row r0 + (k / nch) * nwaves, chunk k % nch).
  const int r0 = blockIdx.x * WAVES + wave;
  if (!XREG && r0 >= n_rows) return;  // (with XREG every wave takes part in staging x first)
  const int nitems = r0 < n_rows ? ((n_rows - 1 - r0) / nwaves + 1) * nch : 0;
  auto item_row = [&](int k) { return r0 + (k / nch) * nwaves; };
  auto chunk_start = [&](int k) {
    return head + (uint32_t)item_row(k) * rb + (uint32_t)((k % nch) * C::BLOCKS * BB);
  };
  auto chunk_loads = [&](int k) {  // 16-byte loads covering the chunk from its aligned start
    const int nb = min(C::BLOCKS, nblk - (k % nch) * C::BLOCKS);
    return (int)((nb * BB + 3 + 15) >> 4);
  };
  // Every 16-byte load lies inside the range: slots past the chunk repeat its
  // last slot, and a slot that would cross the range's end (the final row's
  // tail) is moved back to end there. Such a slot lands in LDS at its own
  // (4-byte aligned) position, so repeated bytes are written with their own
  // values. The range is at least one block (>= 17 bytes) long.
  const uint32_t rend = (range + 3u) & ~3u;
  struct Slot { v4u V[C::LOADS]; uint32_t D[C::LOADS]; };  // loaded bytes, LDS byte offsets
  auto issue = [&](int k, Slot& S) {
    const uint32_t s0 = chunk_start(k) & ~3u;
    const int n16 = chunk_loads(k);
#pragma unroll
    for (int g = 0; g < C::LOADS; ++g) {
      const uint32_t i = (uint32_t)min(lane + 64 * g, n16 - 1);
      const uint32_t off = min(s0 + 16u * i, rend - 16u);
      S.V[g] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      S.D[g] = off - s0;
    }
  };
  float xra[XREG ? 32 : 1], xrb[XREG ? 32 : 1], xsa = 0.f, xsb = 0.f, xga[4], xgb[4];
  Slot S0, S1;
  if constexpr (!XREG) {
    if (nitems > 0) issue(0, S0);
    if (GV_DEPTH > 1 && nitems > 1) issue(1, S1);
  } else {  // fp32 x, 16-byte aligned (the host's condition for XREG)
    // x into LDS with coalesced loads (consecutive threads, consecutive 16
    // bytes), 32-element chunk c at float offset GV_XPAD * c: with that
    // padding the lanes' 16-byte reads of their own units below (lane l,
    // chunk l) hit distinct banks. The x loads go out first and the first
    // rows' loads right behind them, so the rows stream while x is staged
    // (the memory counter retires loads in issue order). Then each lane keeps
    // its two units of x in registers for every row (K <= 4096: one chunk of
    // units per row), with the unit sums in the same sequential order as
    // stage_x.
    // No control flow between these loads and the rows' (a branch makes the
    // compiler wait for every load before it): the rows' first item is
    // always issued (a wave past the last row reads clamped, in-range bytes
    // it never uses) and the second one repeats the first when there is none.
    // LDS barrier without a memory-counter wait: lgkmcnt(0) (this wave's LDS
    // writes are done), then s_barrier; the memory clobber keeps the compiler
    // from moving the LDS reads above it. The row loads stay in flight.
    auto lds_barrier = []() {
      __builtin_amdgcn_s_waitcnt(0xc07f);
      asm volatile("s_barrier" ::: "memory");
    };
    if constexpr (NORM) {
      // x (+ r) and the norm weights in add_rmsnorm_kernel's layout, every load unpredicated (clamped, tails
      // zeroed at use); the rows go out behind them
      const float* xf = (const float*)x;
      float v[GV_NORM_MAXV], wv[GV_NORM_MAXV];
#pragma unroll
      for (int i = 0; i < GV_NORM_MAXV; ++i) {
        const int c = min((int)threadIdx.x + i * 256, K - 1);
        v[i] = xf[c];
        wv[i] = nm.w ? nm.w[c] : 1.f;
      }
      if (nm.r) {
#pragma unroll
        for (int i = 0; i < GV_NORM_MAXV; ++i) v[i] += nm.r[min((int)threadIdx.x + i * 256, K - 1)];
      }
      issue(0, S0);
      if constexpr (GV_DEPTH > 1) issue(nitems > 1 ? 1 : 0, S1);
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < GV_NORM_MAXV; ++i) {
        if ((int)threadIdx.x + i * 256 >= K) v[i] = 0.f;
        ss = fmaf(v[i], v[i], ss);
      }
      ss = nsx_wave_sum(ss);
      if (lane == 0) gv_part[wave] = ss;
      lds_barrier();
      float tot = 0.f;
#pragma unroll
      for (int i = 0; i < WAVES; ++i) tot += gv_part[i];
      const float inv = 1.f / sqrtf(tot / (float)K + nm.eps);
      const bool wr = nm.s && blockIdx.x == 0;
#pragma unroll
      for (int i = 0; i < GV_NORM_MAXV; ++i) {
        const int c = (int)threadIdx.x + i * 256;
        if (c < K) {
          xs[GV_XPAD * (c >> 5) + (c & 31)] = nm.w ? (v[i] * inv) * wv[i] : v[i] * inv;
          if (wr) nm.s[c] = v[i];
        }
      }
    } else {
      const int nq = K >> 2;  // <= XQ * THREADS
      v4f xv[XQ];
#pragma unroll
      for (int g = 0; g < XQ; ++g) xv[g] = ((const v4f*)x)[min((int)threadIdx.x + g * THREADS, nq - 1)];
      issue(0, S0);
      if constexpr (GV_DEPTH > 1) issue(nitems > 1 ? 1 : 0, S1);
      // the write is unpredicated (a thread past the end rewrites the last float4 with its own value): under
      // a branch, x's load sinks into the branch, behind the rows' loads, and its wait then waits on every
      // row byte
#pragma unroll
      for (int g = 0; g < XQ; ++g) {
        const int q = min((int)threadIdx.x + g * THREADS, nq - 1);
        *(v4f*)(xs + GV_XPAD * (q >> 3) + 4 * (q & 7)) = xv[g];
      }
    }
    lds_barrier();
    const int nu0 = K / 32;
    auto gather = [&](int u, float (&xr)[32], float& sum, float (&gs)[4]) {
      const bool on = u < nu0;
      const int uu = on ? u : 0;
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4) {
        const int e = raw_unit_elem<FMT>(uu, 4 * k4);
        const v4f v = *(const v4f*)(xs + GV_XPAD * (e >> 5) + (e & 31));
        xr[4 * k4] = on ? v.x : 0.f;
        xr[4 * k4 + 1] = on ? v.y : 0.f;
        xr[4 * k4 + 2] = on ? v.z : 0.f;
        xr[4 * k4 + 3] = on ? v.w : 0.f;
      }
      if constexpr (SUMS || FMT == NSX_Q8_0) {
        float a = 0.f;
#pragma unroll
        for (int k = 0; k < 32; ++k) a += xr[k];
        sum = a;
      }
      if constexpr (FMT == NSX_Q6_K) {
#pragma unroll
        for (int L = 0; L < 4; ++L) {
          float a = 0.f;
#pragma unroll
          for (int k = 0; k < 8; ++k) a += xr[8 * L + k];
          gs[L] = a;
        }
      }
    };
    gather(lane, xra, xsa, xga);
    gather(lane + 64, xrb, xsb, xgb);
    // every wave has its x in registers before any wave overwrites the area with row bytes
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
  }
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  // Item k: its bytes (slot k % GV_DEPTH, loaded GV_DEPTH items earlier) ->
  // LDS, the loads of item k + GV_DEPTH into the freed slot, then item k's
  // arithmetic.
  auto step = [&](int k, Slot& S) {
#pragma unroll
    for (int g = 0; g < C::LOADS; ++g) {  // in order with this wave's earlier LDS reads
      uint32_t* w = (uint32_t*)(wbuf + S.D[g]);
      w[0] = S.V[g].x; w[1] = S.V[g].y; w[2] = S.V[g].z; w[3] = S.V[g].w;
    }
    const uint32_t rel = chunk_start(k) & 3u;  // offset of the chunk's first byte in wbuf
    if (k + GV_DEPTH < nitems) issue(k + GV_DEPTH, S);
    const int c = k % nch;
    const int nu = min(GV_CHUNK_UNITS, (nblk - c * C::BLOCKS) * BE / 32);
    const int u0 = c * GV_CHUNK_UNITS;
    const RawLdsSrc src{wbuf};
    const RawUnit<FMT> A = raw_unit_fetch<FMT>(src, rel, lane);
    const RawUnit<FMT> B = raw_unit_fetch<FMT>(src, rel, lane + 64);
    if constexpr (XREG) {
      if (lane < nu) raw_unit_math<FMT, NT>(A, u0 + lane, RawXReg{xra, xsa, xga}, RawXSumReg{xsa}, acc);
      if (lane + 64 < nu) raw_unit_math<FMT, NT>(B, u0 + lane + 64, RawXReg{xrb, xsb, xgb}, RawXSumReg{xsb}, acc);
    } else {
      const int ua = u0 + lane, ub = ua + 64;
      if (lane < nu) raw_unit_math<FMT, NT>(A, ua, RawXLds<FMT>{xs, K, ua}, RawXSumLds{xsum, K >> 5, ua}, acc);
      if (lane + 64 < nu) raw_unit_math<FMT, NT>(B, ub, RawXLds<FMT>{xs, K, ub}, RawXSumLds{xsum, K >> 5, ub}, acc);
    }
    if (c == nch - 1) {
      const int r = item_row(k);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float v = nsx_wave_sum(acc[t]);
        if (lane == 0 && t < T && r < n_rows) {  // (r >= n_rows: a wave past the last row, below)
          // epilogue in the reference's order: resid + (x @ W.T + bias)
          if (bias) v += bias[r];
          if (resid) v = resid[(int64_t)t * ystride + r] + v;
          y[(int64_t)t * ystride + r] = v;
        }
        acc[t] = 0.f;
      }
    }
  };
  if constexpr (GV_DEPTH == 1) {
    for (int k = 0; k < nitems; ++k) step(k, S0);
  } else if constexpr (XREG) {
    // the first item outside any branch, so its loads (issued before x's staging) are used on every path:
    // under a branch, the compiler sinks them past the LDS barriers into it, behind x's round trip. A wave
    // past the last row runs it on the clamped in-range bytes it loaded and stores nothing.
    step(0, S0);
    for (int k = 1; k < nitems; k += 2) {
      step(k, S1);
      if (k + 1 < nitems) step(k + 1, S0);
    }
  } else {
    for (int k = 0; k < nitems; k += 2) {
      step(k, S0);
      if (k + 1 < nitems) step(k + 1, S1);
    }
  }
}

// Workgroups of `kernel` (`threads` threads, `lds` bytes) resident on the
// current device at once: CUs x blocks per CU, cached per kernel and LDS size.
int nsx_resident_workgroups(const void* kernel, size_t lds, int threads) {
  struct Entry { const void* k; size_t lds; int threads, dev, n; };
  static std::mutex mu;
  static Entry cache[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == kernel && cache[i].lds == lds && cache[i].threads == threads && cache[i].dev == dev)
      return cache[i].n;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (lds > 64 * 1024) (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) != hipSuccess || per <= 0) per = 1;
  (void)hipGetLastError();
  const int n = cus * per;
  if (used < 64) cache[used++] = Entry{kernel, lds, threads, dev, n};
  return n;
}

template <int FMT, int NT>
static int launch_gemv_raw(const void* raw, int64_t n_rows, int64_t K, const void* x, int xdt,
                           int64_t T, float* y, const float* bias, const float* resid, hipStream_t st,
                           const GvNorm* nm = nullptr) {
  const int64_t row_bytes = raw_row_bytes<FMT>((int)K);
  const int64_t rows_per_launch = std::max<int64_t>(1, ((int64_t)1 << 31) / row_bytes);
  constexpr bool XR = NT == 1;  // the register path exists for one token only (fp32 x, 16-byte aligned)
  const bool xreg = XR && K <= GV_CHUNK_UNITS * 32 && xdt == NSX_DT_F32 && ((uintptr_t)x & 15u) == 0;
  NSX_REQUIRE(!nm || (xreg && K <= 256 * GV_NORM_MAXV), NSX_EINVAL,
              "the norm prologue takes one fp32 token, 16-byte aligned, K <= %d", 256 * GV_NORM_MAXV);
  const size_t bufs = (size_t)GV_WAVES * GvChunk<FMT>::WAVE_BYTES;
  const size_t lds = xreg ? std::max((size_t)gv_xreg_bytes((int)K), bufs) : (size_t)gv_x_bytes<NT>((int)K) + bufs;
  const void* kern = xreg ? (const void*)gemv_raw_kernel<FMT, NT, XR> : (const void*)gemv_raw_kernel<FMT, NT, false>;
  if (lds > 64 * 1024) NSX_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  const int64_t resident = nsx_resident_workgroups(kern, lds, GV_THREADS);
  // Small one-token matrices (a row per wave fits the machine in one pass of
  // 16-wave workgroups): every row's loads go out at once and x is staged
  // once per workgroup. For the formats whose unit arithmetic fits the
  // 128-VGPR budget of a 1024-thread workgroup (Q4_0, MXFP4; the others would
  // spill and keep the 4-wave persistent grid).
  constexpr int BIG = 16;
  constexpr bool BIG_OK = XR && (FMT == NSX_Q4_0 || FMT == NSX_MXFP4);
  const size_t lds_big = std::max((size_t)gv_xreg_bytes((int)K), (size_t)BIG * GvChunk<FMT>::WAVE_BYTES);
  int64_t big_resident = 0;
  if constexpr (BIG_OK)
    big_resident = nsx_resident_workgroups((const void*)gemv_raw_kernel<FMT, NT, XR, BIG>, lds_big, 64 * BIG);
  for (int64_t r0 = 0; r0 < n_rows; r0 += rows_per_launch) {
    const int64_t nr = std::min(rows_per_launch, n_rows - r0);
    const uint8_t* p = (const uint8_t*)raw + r0 * row_bytes;
    const uintptr_t a = (uintptr_t)p & ~(uintptr_t)3;
    const uint32_t head = (uint32_t)((uintptr_t)p - a);
    const uint32_t range = head + (uint32_t)(nr * row_bytes);
    const float* b = bias ? bias + r0 : nullptr;
    const float* rr = resid ? resid + r0 : nullptr;
    if constexpr (BIG_OK) {
      if (xreg && !nm && nr <= BIG * big_resident) {
        if (lds_big > 64 * 1024)
          NSX_HIP(hipFuncSetAttribute((const void*)gemv_raw_kernel<FMT, NT, XR, BIG>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_big));
        hipLaunchKernelGGL((gemv_raw_kernel<FMT, NT, XR, BIG>), dim3((unsigned)nsx_cdiv(nr, BIG)), dim3(64 * BIG),
                           lds_big, st, (const uint8_t*)a, head, range, (int)nr, (int)K, x, xdt, (int)T, y + r0,
                           n_rows, b, rr);
        NSX_LAUNCHED();
        continue;
      }
    }
    // Persistent: the resident workgroups for large matrices; for small ones
    // (under two rounds of that grid) half of them, so each wave has several
    // rows and overlaps their loads (a large matrix on half the grid is slower).
    const int64_t per_row = nsx_cdiv(nr, GV_WAVES);
    const int64_t cap = per_row <= 2 * resident ? std::max<int64_t>(1, resident / 2) : resident;
    const unsigned grid = (unsigned)std::min<int64_t>(per_row, cap);
    if constexpr (XR) {
      if (nm) {  // (a later launch of a split matrix sees the normed input again, without writing s twice)
        GvNorm n1 = *nm;
        if (r0 > 0) n1.s = nullptr;
        hipLaunchKernelGGL((gemv_raw_kernel<FMT, NT, XR, GV_WAVES, true>), dim3(grid), dim3(GV_THREADS), lds, st,
                           (const uint8_t*)a, head, range, (int)nr, (int)K, x, xdt, (int)T, y + r0, n_rows, b, rr,
                           n1);
        NSX_LAUNCHED();
        continue;
      }
    }
    if (xreg)
      hipLaunchKernelGGL((gemv_raw_kernel<FMT, NT, XR>), dim3(grid), dim3(GV_THREADS), lds, st,
                         (const uint8_t*)a, head, range, (int)nr, (int)K, x, xdt, (int)T, y + r0, n_rows, b, rr);
    else
      hipLaunchKernelGGL((gemv_raw_kernel<FMT, NT, false>), dim3(grid), dim3(GV_THREADS), lds, st,
                         (const uint8_t*)a, head, range, (int)nr, (int)K, x, xdt, (int)T, y + r0, n_rows, b, rr);
    NSX_LAUNCHED();
  }
  return NSX_OK;
}

template <int FMT>
static int gemv_raw_fmt(const void* raw, int64_t n_rows, int64_t K, const void* x, int xdt, int64_t T,
                        float* y, const float* bias, const float* resid, hipStream_t st) {
  if (T == 1) return launch_gemv_raw<FMT, 1>(raw, n_rows, K, x, xdt, T, y, bias, resid, st);
  if (T == 2) return launch_gemv_raw<FMT, 2>(raw, n_rows, K, x, xdt, T, y, bias, resid, st);
  if (T <= 4) return launch_gemv_raw<FMT, 4>(raw, n_rows, K, x, xdt, T, y, bias, resid, st);
  if (T <= 8) return launch_gemv_raw<FMT, 8>(raw, n_rows, K, x, xdt, T, y, bias, resid, st);
  return launch_gemv_raw<FMT, 16>(raw, n_rows, K, x, xdt, T, y, bias, resid, st);
}

static inline int64_t pad_tokens(int64_t T) { return T == 1 ? 1 : T == 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 16; }

extern "C" int nsx_fused_gemv_ex(int t, const void* raw, int64_t n_rows, int64_t K, const void* x,
                                 int x_dtype, int64_t T, float* y, const float* bias, const float* resid,
                                 void* stream);

extern "C" int nsx_fused_gemv(int t, const void* raw, int64_t n_rows, int64_t K, const void* x,
                              int x_dtype, int64_t T, float* y, void* stream) {
  return nsx_fused_gemv_ex(t, raw, n_rows, K, x, x_dtype, T, y, nullptr, nullptr, stream);
}

extern "C" int nsx_fused_gemv_ex(int t, const void* raw, int64_t n_rows, int64_t K, const void* x,
                                 int x_dtype, int64_t T, float* y, const float* bias, const float* resid,
                                 void* stream) {
  const int BE = nsx_block_elems(t), BB = nsx_block_bytes(t);
  NSX_REQUIRE(BB > 0, NSX_ENOTIMPL, "no fused kernel for ggml type %d", t);
  NSX_REQUIRE(n_rows >= 0 && K > 0 && K % BE == 0, NSX_EINVAL,
              "K=%lld is not a positive multiple of the %d-element block", (long long)K, BE);
  NSX_REQUIRE(T >= 1 && T <= GV_MAXT, NSX_EINVAL, "T=%lld outside 1..%d", (long long)T, GV_MAXT);
  NSX_REQUIRE(x_dtype == NSX_DT_F32 || x_dtype == NSX_DT_F16 || x_dtype == NSX_DT_BF16, NSX_EINVAL,
              "x dtype %d", x_dtype);
  NSX_REQUIRE(n_rows < (1ll << 31) && K < (1ll << 20), NSX_EINVAL, "shape too large");
  if (n_rows == 0) return NSX_OK;
  NSX_REQUIRE(raw && x && y, NSX_EINVAL, "null buffer");
  NSX_REQUIRE((K + K / 32) * 4 <= 64 * 1024, NSX_EINVAL, "K=%lld too large for one workgroup's LDS", (long long)K);
  if (t == NSX_Q4_K)
    NSX_REQUIRE(((uintptr_t)raw & 3) == 0, NSX_EINVAL, "Q4_K rows must be 4-byte aligned");
  hipStream_t st = S(stream);
  // tokens per launch: as many as one workgroup's LDS holds (<= 64 KiB staged)
  int64_t chunk = 16;
  while (chunk > 1 && chunk * (K + K / 32) * 4 > 64 * 1024) chunk /= 2;
  const size_t xsz = x_dtype == NSX_DT_F32 ? 4 : 2;
  for (int64_t t0 = 0; t0 < T; t0 += chunk) {
    const int64_t nt = std::min(chunk, T - t0);
    const void* xc = (const char*)x + t0 * K * xsz;
    float* yc = y + t0 * n_rows;
    const float* rc_ = resid ? resid + t0 * n_rows : nullptr;
    int rc = NSX_ENOTIMPL;
    switch (t) {
      case NSX_MXFP4: rc = gemv_raw_fmt<NSX_MXFP4>(raw, n_rows, K, xc, x_dtype, nt, yc, bias, rc_, st); break;
      case NSX_Q4_0: rc = gemv_raw_fmt<NSX_Q4_0>(raw, n_rows, K, xc, x_dtype, nt, yc, bias, rc_, st); break;
      case NSX_Q8_0: rc = gemv_raw_fmt<NSX_Q8_0>(raw, n_rows, K, xc, x_dtype, nt, yc, bias, rc_, st); break;
      case NSX_Q4_K: rc = gemv_raw_fmt<NSX_Q4_K>(raw, n_rows, K, xc, x_dtype, nt, yc, bias, rc_, st); break;
      case NSX_Q6_K: rc = gemv_raw_fmt<NSX_Q6_K>(raw, n_rows, K, xc, x_dtype, nt, yc, bias, rc_, st); break;
    }
    if (rc) return rc;
  }
  return NSX_OK;
}

extern "C" int nsx_fused_gemv_norm(int t, const void* raw, int64_t n_rows, int64_t K, const float* x,
                                   const float* r, const float* w, float eps, float* s, float* y,
                                   const float* bias, const float* resid, void* stream) {
  const int BE = nsx_block_elems(t), BB = nsx_block_bytes(t);
  NSX_REQUIRE(BB > 0, NSX_ENOTIMPL, "no fused kernel for ggml type %d", t);
  NSX_REQUIRE(n_rows >= 0 && K > 0 && K % BE == 0, NSX_EINVAL,
              "K=%lld is not a positive multiple of the %d-element block", (long long)K, BE);
  NSX_REQUIRE(n_rows < (1ll << 31) && K <= 256 * GV_NORM_MAXV, NSX_EINVAL, "shape too large");
  if (n_rows == 0) return NSX_OK;
  NSX_REQUIRE(raw && x && y, NSX_EINVAL, "null buffer");
  NSX_REQUIRE(((uintptr_t)x & 15) == 0, NSX_EINVAL, "x must be 16-byte aligned");
  // Workgroup 0 writes s and every workgroup writes its rows of y while the others still read x, r and
  // resid in the norm prologue and epilogue: no output may overlap an input another workgroup reads (y may be
  // resid exactly: each element of y is read from resid by the thread that writes it)
  auto overlap = [](const void* p, int64_t pn, const void* q, int64_t qn) {
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return p && q && a < b + (uintptr_t)(qn * 4) && b < a + (uintptr_t)(pn * 4);
  };
  NSX_REQUIRE(!overlap(s, K, x, K) && !overlap(s, K, r, K) && !overlap(s, K, resid, n_rows) &&
                  !overlap(s, K, y, n_rows),
              NSX_EINVAL, "s must not overlap x, r, resid or y");
  NSX_REQUIRE(!overlap(y, n_rows, x, K) && !overlap(y, n_rows, r, K), NSX_EINVAL, "y must not overlap x or r");
  NSX_REQUIRE(resid == y || !overlap(y, n_rows, resid, n_rows), NSX_EINVAL,
              "y must be resid or apart from it");
  if (t == NSX_Q4_K)
    NSX_REQUIRE(((uintptr_t)raw & 3) == 0, NSX_EINVAL, "Q4_K rows must be 4-byte aligned");
  const GvNorm nm{r, w, eps, s};
  hipStream_t st = S(stream);
  switch (t) {
    case NSX_MXFP4: return launch_gemv_raw<NSX_MXFP4, 1>(raw, n_rows, K, x, NSX_DT_F32, 1, y, bias, resid, st, &nm);
    case NSX_Q4_0: return launch_gemv_raw<NSX_Q4_0, 1>(raw, n_rows, K, x, NSX_DT_F32, 1, y, bias, resid, st, &nm);
    case NSX_Q8_0: return launch_gemv_raw<NSX_Q8_0, 1>(raw, n_rows, K, x, NSX_DT_F32, 1, y, bias, resid, st, &nm);
    case NSX_Q4_K: return launch_gemv_raw<NSX_Q4_K, 1>(raw, n_rows, K, x, NSX_DT_F32, 1, y, bias, resid, st, &nm);
    case NSX_Q6_K: return launch_gemv_raw<NSX_Q6_K, 1>(raw, n_rows, K, x, NSX_DT_F32, 1, y, bias, resid, st, &nm);
  }
  return NSX_ENOTIMPL;
}

// ---------------------------------------------------------------------------
// t64 layout (MXFP4): 64-row tiles; qs plane [tile][block][row][16 B] then
// scale plane [tile][block/4][row][4 B]. Rows beyond n_rows and blocks beyond
// nb inside the last scale group are zero.

// ---------------------------------------------------------------------------
// t64 tiles (layout in mx.h): pack from / unpack to GGUF MXFP4 rows

extern "C" int64_t nsx_t64_bytes(int t, int64_t n_rows, int64_t K) {
  if (t != NSX_MXFP4 || K <= 0 || K % 32 || n_rows < 0) return -1;
  const MxGeom g = mx_geom(n_rows, K);
  return g.tiles * g.tile_bytes;
}

// 16 code bytes in GGUF order (byte j = element j | element j + 16 << 4) ->
// element order (byte m = element 2m | element 2m + 1 << 4), and back
__device__ __forceinline__ uint32_t mx_pair_nibbles(uint32_t x) {  // 4 nibble-bytes -> 2 bytes
  const uint32_t y = x | (x >> 4);
  return (y & 0xffu) | ((y >> 8) & 0xff00u);
}
__device__ __forceinline__ v4u mx_gguf_to_elem(const uint32_t (&q)[4]) {
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    lo[d] = q[d] & 0x0f0f0f0fu;         // elements 4d .. 4d + 3
    hi[d] = (q[d] >> 4) & 0x0f0f0f0fu;  // elements 16 + 4d .. 16 + 4d + 3
  }
  return v4u{mx_pair_nibbles(lo[0]) | (mx_pair_nibbles(lo[1]) << 16),
             mx_pair_nibbles(lo[2]) | (mx_pair_nibbles(lo[3]) << 16),
             mx_pair_nibbles(hi[0]) | (mx_pair_nibbles(hi[1]) << 16),
             mx_pair_nibbles(hi[2]) | (mx_pair_nibbles(hi[3]) << 16)};
}
__device__ __forceinline__ uint32_t mx_spread_nibbles(uint32_t x16) {  // 2 bytes -> 4 nibble-bytes
  const uint32_t b0 = x16 & 0xffu, b1 = (x16 >> 8) & 0xffu;
  return (b0 & 15u) | ((b0 >> 4) << 8) | ((b1 & 15u) << 16) | ((b1 >> 4) << 24);
}
__device__ __forceinline__ void mx_elem_to_gguf(v4u w, uint32_t (&q)[4]) {
  uint32_t el[8];  // nibble-bytes: el[d] = elements 4d .. 4d + 3
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    el[2 * d] = mx_spread_nibbles(w[d] & 0xffffu);
    el[2 * d + 1] = mx_spread_nibbles(w[d] >> 16);
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) q[d] = el[d] | (el[d + 4] << 4);
}

// one thread per (tile, step, g, lane) slot that exists in the layout
__global__ void t64_pack_kernel(const uint8_t* __restrict__ base, uint32_t head, uint32_t range, int64_t n_rows,
                                MxGeom G, uint8_t* __restrict__ dst) {
  const int64_t slot = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // over tiles * ns * 4 * 64
  if (slot >= G.tiles * G.ns * 256) return;
  const int lane = (int)(slot & 63), g = (int)((slot >> 6) & 3);
  const int64_t ts = slot >> 8;
  const int s = (int)(ts % G.ns);
  const int64_t tile = ts / G.ns;
  const int rs = s < G.ns - 1 ? 4 : G.rlast;
  const int q = lane >> 4, i = lane & 15;
  if (q >= rs) return;
  const int64_t row = tile * 64 + 16 * g + i;
  const int b = 4 * s + q;
  uint32_t Q[4] = {0u, 0u, 0u, 0u};
  uint32_t e = 0u;
  if (row < n_rows) {
    const __amdgpu_buffer_rsrc_t rs_ = nsx_rsrc(base, range);
    const uint32_t o = head + (uint32_t)((row * G.nb + b) * 17);
    const uint32_t sh = o & 3u, oa = o & ~3u;
    uint32_t Dw[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) Dw[k] = nsx_bload32(rs_, oa + 4u * k);
    uint32_t E[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) E[k] = nsx_alignbyte(Dw[k + 1], Dw[k], sh);
    e = E[0] & 0xffu;
#pragma unroll
    for (int k = 0; k < 4; ++k) Q[k] = nsx_alignbyte(E[k + 1], E[k], 1);
  }
  uint8_t* ch = dst + tile * G.tile_bytes + (int64_t)s * MX_STEP_BYTES;
  *(v4u*)(ch + g * rs * 256 + lane * 16) = mx_gguf_to_elem(Q);
  ch[rs * 1024 + lane * 4 + g] = (uint8_t)e;
}

// one thread per (row, block) of the matrix
__global__ void t64_unpack_kernel(const uint8_t* __restrict__ src, int64_t n_rows, MxGeom G,
                                  uint8_t* __restrict__ raw) {
  const int64_t slot = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (slot >= n_rows * G.nb) return;
  const int64_t row = slot / G.nb;
  const int b = (int)(slot % G.nb);
  const int64_t tile = row >> 6;
  const int r = (int)(row & 63), g = r >> 4, i = r & 15;
  const int s = b >> 2, q = b & 3;
  const int rs = s < G.ns - 1 ? 4 : G.rlast;
  const int lane = 16 * q + i;
  const uint8_t* ch = src + tile * G.tile_bytes + (int64_t)s * MX_STEP_BYTES;
  uint32_t Q[4];
  mx_elem_to_gguf(*(const v4u*)(ch + g * rs * 256 + lane * 16), Q);
  uint8_t* o = raw + slot * 17;
  o[0] = ch[rs * 1024 + lane * 4 + g];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) o[1 + 4 * k + j] = (uint8_t)(Q[k] >> (8 * j));
  }
}

extern "C" int nsx_t64_pack(int t, const void* raw, int64_t n_rows, int64_t K, void* t64, void* stream) {
  NSX_REQUIRE(t == NSX_MXFP4, NSX_ENOTIMPL, "t64 layout is implemented for MXFP4 only (type %d)", t);
  NSX_REQUIRE(K > 0 && K % 32 == 0 && n_rows >= 0, NSX_EINVAL, "bad shape %lld x %lld",
              (long long)n_rows, (long long)K);
  const MxGeom g = mx_geom(n_rows, K);
  if (n_rows == 0) return NSX_OK;
  NSX_REQUIRE(raw && t64, NSX_EINVAL, "null buffer");
  const int64_t raw_bytes = n_rows * g.nb * 17;
  NSX_REQUIRE(raw_bytes < (1ll << 32) - 8, NSX_EINVAL, "pack source above 4 GiB: pack per expert");
  const uint8_t* p = (const uint8_t*)raw;
  const uintptr_t a = (uintptr_t)p & ~(uintptr_t)3;
  const uint32_t head = (uint32_t)((uintptr_t)p - a);
  const int64_t total = g.tiles * g.ns * 256;
  hipLaunchKernelGGL(t64_pack_kernel, dim3((unsigned)nsx_cdiv(total, 256)), dim3(256), 0, S(stream),
                     (const uint8_t*)a, head, (uint32_t)(head + raw_bytes), n_rows, g, (uint8_t*)t64);
  NSX_LAUNCHED();
  return NSX_OK;
}

extern "C" int nsx_t64_unpack(int t, const void* t64, int64_t n_rows, int64_t K, void* raw, void* stream) {
  NSX_REQUIRE(t == NSX_MXFP4, NSX_ENOTIMPL, "t64 layout is implemented for MXFP4 only (type %d)", t);
  NSX_REQUIRE(K > 0 && K % 32 == 0 && n_rows >= 0, NSX_EINVAL, "bad shape");
  const MxGeom g = mx_geom(n_rows, K);
  if (n_rows == 0) return NSX_OK;
  NSX_REQUIRE(raw && t64, NSX_EINVAL, "null buffer");
  const int64_t total = n_rows * g.nb;
  hipLaunchKernelGGL(t64_unpack_kernel, dim3((unsigned)nsx_cdiv(total, 256)), dim3(256), 0, S(stream),
                     (const uint8_t*)t64, n_rows, g, (uint8_t*)raw);
  NSX_LAUNCHED();
  return NSX_OK;
}
