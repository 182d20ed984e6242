// Shared device/host helpers for the nurostream_amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/nurostream_amd.h"

#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "nurostream_amd kernels are written for gfx950 (MI355X) only"
#endif

// ---------------------------------------------------------------------------
// host-side error reporting

int nsx_fail(int code, const char* fmt, ...);
// Workgroups of `kernel` (`threads` threads, `lds` dynamic bytes) resident on the current device at once
// (CUs x blocks per CU), cached per kernel, LDS size and device.
int nsx_resident_workgroups(const void* kernel, size_t lds, int threads);

#define NSX_HIP(call)                                                           \
  do {                                                                          \
    hipError_t e_ = (call);                                                     \
    if (e_ != hipSuccess)                                                       \
      return nsx_fail(NSX_EHIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

#define NSX_REQUIRE(cond, code, ...)          \
  do {                                        \
    if (!(cond)) return nsx_fail(code, __VA_ARGS__); \
  } while (0)

#define NSX_LAUNCHED()                                                             \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess)                                                          \
      return nsx_fail(NSX_EHIP, "kernel launch failed: %s", hipGetErrorString(e_)); \
  } while (0)

// Launch `kernel` on `st` and report a failed launch.
template <typename... KA, typename... A>
static inline int nsx_launch(void (*kernel)(KA...), dim3 grid, dim3 block, size_t lds, hipStream_t st, A... args) {
  hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
  NSX_LAUNCHED();
  return NSX_OK;
}

static inline int64_t nsx_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// (elements per block, bytes per block) for the block formats the kernels handle.
static inline int nsx_block_elems(int t) {
  switch (t) {
    case NSX_Q4_0: case NSX_Q8_0: case NSX_MXFP4: return 32;
    case NSX_Q4_K: case NSX_Q6_K: return 256;
    default: return 0;
  }
}
static inline int nsx_block_bytes(int t) {
  switch (t) {
    case NSX_Q4_0: return 18;
    case NSX_Q8_0: return 34;
    case NSX_MXFP4: return 17;
    case NSX_Q4_K: return 144;
    case NSX_Q6_K: return 210;
    default: return 0;
  }
}

// ---------------------------------------------------------------------------
// device helpers

typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float nsx_h2f(uint32_t bits16) {
  // exact fp16 -> fp32, subnormal halves included (denormals are preserved
  // in this library's kernels: no -ffast-math, no denormal flushing)
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ float nsx_bf2f(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even, NaN -> quiet NaN (torch's rule)
__device__ __forceinline__ uint32_t nsx_f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t nsx_f2h(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// byte k of a dword as float (v_cvt_f32_ubyteK)
template <int k>
__device__ __forceinline__ float nsx_ub(uint32_t x) {
  return (float)((x >> (8 * k)) & 0xffu);
}

// byte-granular funnel: bytes [s, s+4) of the 8-byte little-endian pair (lo, hi)
__device__ __forceinline__ uint32_t nsx_alignbyte(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// Load element i of an activation vector stored as f32 / f16 / bf16.
__device__ __forceinline__ float nsx_load_act(const void* p, int dtype, int64_t i) {
  if (dtype == NSX_DT_F32) return ((const float*)p)[i];
  uint32_t b = ((const uint16_t*)p)[i];
  return dtype == NSX_DT_F16 ? nsx_h2f(b) : nsx_bf2f(b);
}

// Kernel arguments are read through the scalar cache where first used; a
// kernel whose first uses are spread over its prologue waits on one cache
// miss after another. nsx_hoist ties wave-uniform values to an empty asm
// statement, so their loads are issued together (one wait) where it stands.
__device__ __forceinline__ void nsx_hoist1(int v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void nsx_hoist1(int64_t v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void nsx_hoist1(float v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void nsx_hoist1(const void* v) { asm volatile("" ::"s"(v)); }
template <typename... A>
__device__ __forceinline__ void nsx_hoist(const A&... v) {
  (nsx_hoist1(v), ...);
}

// Wave64 reductions on DPP row rotations (within each 16-lane row, no LDS
// round trip) plus four readlanes; the result is wave-uniform. Every lane of
// the wave must be active.
#define NSX_DPP_ROR(n) (0x120 + (n))
template <typename Op>
__device__ __forceinline__ uint32_t nsx_row_reduce_u32(uint32_t v, Op op) {
  // update_dpp with bound_ctrl lets the compiler fold each move into the op
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, NSX_DPP_ROR(8), 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, NSX_DPP_ROR(4), 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, NSX_DPP_ROR(2), 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, NSX_DPP_ROR(1), 0xf, 0xf, true));
  return v;
}
__device__ __forceinline__ uint32_t nsx_wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = nsx_row_reduce_u32(v, mx);
  return mx(mx(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
            mx(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ uint32_t nsx_wave_min_u32(uint32_t v) {
  auto mn = [](uint32_t a, uint32_t b) { return a < b ? a : b; };
  v = nsx_row_reduce_u32(v, mn);
  return mn(mn(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
            mn(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
template <int CTRL>
__device__ __forceinline__ float nsx_dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// the same with bound_ctrl, so that the compiler can fold the move into its user
template <int CTRL>
__device__ __forceinline__ float nsx_dpp_fold(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
// max over the lane's 16-lane row of values >= 0 (or +inf): their bit patterns
// order as unsigned integers, and the integer max folds with its DPP move
__device__ __forceinline__ float nsx_row_max_nonneg(float v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  return __builtin_bit_cast(float, nsx_row_reduce_u32(__builtin_bit_cast(uint32_t, v), mx));
}
__device__ __forceinline__ float nsx_row_fmax(float v) {  // max over the lane's 16-lane row
  v = fmaxf(v, nsx_dpp_fold<NSX_DPP_ROR(8)>(v));
  v = fmaxf(v, nsx_dpp_fold<NSX_DPP_ROR(4)>(v));
  v = fmaxf(v, nsx_dpp_fold<NSX_DPP_ROR(2)>(v));
  return fmaxf(v, nsx_dpp_fold<NSX_DPP_ROR(1)>(v));
}
// Wave64 sum (wave-uniform): rows by rotation, then rows 0 + 1 + 2 + 3.
__device__ __forceinline__ float nsx_wave_sum(float v) {
  v += nsx_dpp_f<NSX_DPP_ROR(8)>(v);
  v += nsx_dpp_f<NSX_DPP_ROR(4)>(v);
  v += nsx_dpp_f<NSX_DPP_ROR(2)>(v);
  v += nsx_dpp_f<NSX_DPP_ROR(1)>(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Raw buffer resource over [p, p + nbytes) with p 4-byte aligned: stride 0,
// num_records in bytes, rounded up to whole dwords because the range check
// is per access (a dword straddling num_records would read as zero). The
// rounded tail stays inside the allocation: it lies in the same aligned dword
// as the last valid byte. Loads past the range return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t nsx_rsrc(const void* p, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)((nbytes + 3u) & ~3u), 0x00020000);
}

__device__ __forceinline__ uint32_t nsx_bload32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// OCP e2m1 magnitudes (true values, x1): used where a float table is needed.
__device__ __constant__ static const float kE2M1x2[16] = {
    0.f, 1.f, 2.f, 3.f, 4.f, 6.f, 8.f, 12.f, 0.f, -1.f, -2.f, -3.f, -4.f, -6.f, -8.f, -12.f};

// GGUF/ggml MXFP4 scale: 2^(e-128) from raw float bits, e<2 give denormals,
// e=255 gives 2^127 (not NaN).
__device__ __forceinline__ float nsx_mx_scale_half(uint32_t e) {
  uint32_t bits = e < 2 ? (0x00200000u << e) : ((e - 1u) << 23);
  return __builtin_bit_cast(float, bits);
}

// Q4_K get_scale_min_k4 for sub-block s (0..7) from the 12-byte field.
__device__ __forceinline__ void nsx_q4k_scale_min(const uint8_t* q, int s, uint32_t& sc, uint32_t& m) {
  if (s < 4) {
    sc = q[s] & 63u;
    m = q[s + 4] & 63u;
  } else {
    sc = (q[s + 4] & 0x0Fu) | ((q[s - 4] >> 6) << 4);
    m = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
  }
}
