// MXFP4 x activation products on gfx950's block-scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4, A = FP4 weights with their e8m0
// scales, B = FP8 E4M3 activation terms with e8m0 scales).
//
// Operand model (established with in-bounds one-hot probes on gfx950):
//   A (FP4, 4 VGPRs): lane l = 16 q + i holds row i and K = 32 q .. 32 q + 31
//     of the instruction's 128-wide K slice, element order: byte m = element
//     2m (low nibble) | element 2m + 1 (high nibble). Its scale byte (opsel
//     selects a byte of the scale VGPR) applies to those 32 K values.
//   B (FP8, 8 VGPRs): lane l = 16 g + c holds column c and K = 16 g .. 16 g +
//     15 (bytes 0..15) and 64 + 16 g .. 64 + 16 g + 15 (bytes 16..31); the
//     scale byte of lane 16 q + c applies to K = 32 q .. 32 q + 31.
//   D (4 VGPRs): lane l holds column l % 16, rows 4 (l / 16) .. + 3.
// Products are exact; the hardware sums groups of 8 of them aligned to the
// group's largest with about 12 kept bits, so results are good to ~4e-6 of
// max|y| on GEMV-like data (measured), inside the path's 1e-3 parity bar.
#pragma once

#include "nsx_common.h"

typedef int v8i __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// t64 tile layout (resident MXFP4 expert slabs)
//
// An n_rows x K MXFP4 matrix (nb = K / 32 blocks per row) is stored as
// ceil(n_rows / 64) tiles of nb * 1088 bytes -- the GGUF byte count, rows
// padded to 64. A tile is a run of K-steps s = 0 .. ns - 1 of r_s = min(4,
// nb - 4 s) blocks; step s starts at byte s * 4352 and holds
//   codes : [g 0..3][lane 0 .. 16 r_s - 1][16 B]   at g * r_s * 256 + lane * 16
//   scales: [lane 0 .. 16 r_s - 1][4 B]            at r_s * 1024 + lane * 4
// where lane = 16 q + i stands for row 16 g + i of the tile and block 4 s + q:
// its 16 code bytes are that block's codes in A-operand order and byte g of
// its scale dword is the block's e8m0. Padding rows are zero codes, scale 0.

constexpr int MX_STEP_BYTES = 4352;  // 64 rows x 4 blocks x 17 B
constexpr int MX_TILE_ROWS = 64;

struct MxGeom {
  int nb;              // blocks per row
  int ns;              // K-steps
  int rlast;           // blocks in the last step (1..4)
  int64_t tile_bytes;  // nb * 1088
  int64_t tiles;
};

__host__ __device__ __forceinline__ MxGeom mx_geom(int64_t n_rows, int64_t K) {
  MxGeom g;
  g.nb = (int)(K / 32);
  g.ns = (g.nb + 3) / 4;
  g.rlast = g.nb - 4 * (g.ns - 1);
  g.tile_bytes = (int64_t)g.nb * 1088;
  g.tiles = (n_rows + 63) / 64;
  return g;
}

// ---------------------------------------------------------------------------
// activation terms ("xq")
//
// x ~ sum over t < XQ_NT of 2^(s_t - 127) q_t, with q_t FP8 E4M3 and one e8m0
// s_t per 32-element block and term; term t + 1 encodes what term t left
// (round to nearest even, exact residuals), so each term adds 4 bits: the
// block's error is at most 2^-16 of its largest |x|. NaN or infinite inputs
// give a scale byte of 255 (NaN) in term 0, so they surface as NaN outputs.
// Storage per token and K-step (128 elements), in B-operand order:
//   codes : [g 0..3][t][32 B]   byte j of (g, t) is element 16 g + j (j < 16)
//                               or 64 + 16 g + j - 16 of the step
//   scales: [q 0..3][t][4 B]    e8m0 of block 4 s + q in byte 0
constexpr int XQ_NT = 4;
constexpr int XQ_CODES = 4 * XQ_NT * 32;
constexpr int XQ_STEP = XQ_CODES + 4 * XQ_NT * 4;  // 576 B

// Quantize one 32-element block into XQ_NT terms: lanes 32h .. 32h + 31 hold
// element (lane & 31) of their block in r; step is the token's xq record of
// the block's K-step and q the block's place in it (0..3). Both 32-lane
// halves run in lock step (each its own block).
//
// Term 0's e8m0 scale 2^s0 comes from the block's largest |r|, so that
// |r| / 2^s0 <= 448; term t uses 2^(s0 - 4t). v_cvt_pk_fp8_f32 rounds
// r / 2^s to nearest even on the OCP E4M3 grid (subnormals included; checked
// on gfx950 against a software rounding over every code, every tie and its
// neighbours and 16M random values -- the only difference is the sign of
// zero, so a value that rounds to zero stores +0), and the exact residual
// r - code * 2^s is the next term's input. A residual is at most half the
// grid spacing at the top binade, 16 * 2^s, which 2^(s - 4) still holds
// (16 * 2^s = 256 * 2^(s - 4) <= 448 * 2^(s - 4)): every term adds 4 bits,
// and the block's error after XQ_NT terms is at most 2^-16 of its largest
// |r|. Only term 0 needs a reduction over the block.
__device__ __forceinline__ void xq_block_step(float r, int q, uint8_t* step) {
  const int e = __lane_id() & 31;
  const int gp = (q & 1) * 2 + (e >> 4);
  const int j = (e & 15) + 16 * (q >> 1);
  float m = fabsf(r);
  if (!(m <= 3.4028235e38f)) m = __builtin_inff();  // NaN counts as the largest
  m = nsx_row_max_nonneg(m);
  {  // the block's two 16-lane rows: permlane16_swap pairs row 2i with row 2i + 1 (no LDS)
    const uint32_t mb = __builtin_bit_cast(uint32_t, m);
    const auto sw = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
    m = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
  }
  const bool fin = m <= 3.4028235e38f;  // else e8m0 NaN: the outputs of this token become NaN
  const bool nz = m != 0.f;
  const uint32_t mb = __builtin_bit_cast(uint32_t, m);
  const int s0 = (int)((mb >> 23) & 0xffu) - 127 - 8 + ((mb & 0x7fffffu) > 0x600000u ? 1 : 0);
  if (!fin) r = 0.f;
  uint32_t codes = 0;  // byte t: term t's code of this lane's element
  v4u sc;
#pragma unroll
  for (int t = 0; t < XQ_NT; ++t) {
    int sx = s0 - 4 * t;
    sx = sx < -127 ? -127 : sx;
    sc[t] = !fin ? (t == 0 ? 255u : 0u) : (nz ? (uint32_t)(sx + 127) : 0u);
    const uint32_t raw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_ldexpf(r, -sx), 0.f, 0, false) & 0xffu;
    r -= __builtin_amdgcn_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)raw, 0), sx);  // exact
    codes |= ((raw & 0x7fu) != 0u ? raw : 0u) << (8 * t);
  }
  // The four lanes of a quad hold consecutive elements (one dword of each
  // term's code row): a 4 x 4 byte transpose over the quad (DPP broadcasts,
  // byte selects) gives lane i of the quad term i's four codes, so each lane
  // stores one dword instead of a byte per term.
  static_assert(XQ_NT == 4, "one term per lane of a quad");
  const uint32_t i = __lane_id() & 3u;
  const uint32_t q0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)codes, 0x00, 0xf, 0xf, false);
  const uint32_t q1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)codes, 0x55, 0xf, 0xf, false);
  const uint32_t q2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)codes, 0xaa, 0xf, 0xf, false);
  const uint32_t q3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)codes, 0xff, 0xf, 0xf, false);
  // v_perm_b32 selectors: 0..3 bytes of the second operand, 4..7 of the first, 0x0c zero
  const uint32_t lo = __builtin_amdgcn_perm(q1, q0, i | (4u + i) << 8 | 0x0c0c0000u);
  const uint32_t hi = __builtin_amdgcn_perm(q3, q2, 0x0c0cu | i << 16 | (4u + i) << 24);
  *(uint32_t*)(step + (gp * XQ_NT + i) * 32 + (j & ~3)) = lo | hi;
  if (e == 0) *(v4u*)(step + XQ_CODES + q * XQ_NT * 4) = sc;  // the block's four term scales
}
__device__ __forceinline__ void xq_block(float r, int b, uint8_t* dst) {
  xq_block_step(r, b & 3, dst + (int64_t)(b >> 2) * XQ_STEP);
}

// ---------------------------------------------------------------------------
// one wave: a 64-row tile times up to 4 tokens' xq over K-steps [s0, s1)

#define NSX_MFMA_SCALE(A, B, C, G, SA, SB) \
  __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((A), (B), (C), 4, 0, (G), (SA), 0, (SB))

// Operands of up to S K-steps of one wave (G of the tile's four 16-row
// groups), held in registers.
template <int S, int G = 4>
struct MxRegs {
  v4u A[S][G], B0[S], B1[S];
  uint32_t SA[S], SB[S];
};

// A zero scale word for the lanes past a partial last step. It is writable
// memory on purpose: a load the compiler cannot fold stays a load, so no VALU
// select on the loaded scales is left to hoist out of a caller's token loop
// (such a select waits for every weight load before the loop's first
// activation load can go out).
static __device__ uint32_t nsx_mx_zero_scale[1];

// The scale operand of this lane for step chunk ch (rs live lane groups): the
// word of groups g0.. for G = 4, the byte of group g0 for G = 1 (in the low
// byte either way); the zero word for lanes past the step.
template <int G>
__device__ __forceinline__ uint32_t mx_load_sa(const uint8_t* ch, int rs, int lane, int g0) {
  static_assert(G == 1 || G == 4, "one or all four row groups");
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  typedef const __attribute__((address_space(1))) uint8_t gu8;
  const bool live = (lane >> 4) < rs;
  if constexpr (G == 4) {
    const uint8_t* p = live ? ch + rs * 1024 + lane * 4 : (const uint8_t*)nsx_mx_zero_scale;
    return __builtin_nontemporal_load((gu32*)p);
  } else {
    const uint8_t* p = live ? ch + rs * 1024 + lane * 4 + g0 : (const uint8_t*)nsx_mx_zero_scale;
    return __builtin_nontemporal_load((gu8*)p);
  }
}

// Weight operands of steps [s0, min(s1, s0 + S)) of a 64-row tile, read once
// per call (nontemporal: streamed weights do not displace cached data). Loads
// are unpredicated so that their waits retire step by step: lanes past a partial
// last step read an in-bounds stand-in with scale 0 (the activation there is
// zero). A weight e8m0 of 255 is NaN to the hardware: the row's result is
// non-finite, as in the reference, whose fp32 dequant makes such a block
// +-inf (2^127 times ggml's doubled table).
template <int S, int G = 4>
__device__ __forceinline__ void mx_load_a(MxRegs<S, G>& R, const uint8_t* __restrict__ tile, const MxGeom& G_,
                                          int s0, int s1, int g0 = 0) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  const int lane = __lane_id(), grp = lane >> 4;
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int s = s0 + u;
    if (s < s1) {
      const int rs = s < G_.ns - 1 ? 4 : G_.rlast;
      const uint8_t* ch = tile + (int64_t)s * MX_STEP_BYTES;
      const int la = grp < rs ? lane : 16 * rs - 1;
#pragma unroll
      for (int g = 0; g < G; ++g) R.A[u][g] = __builtin_nontemporal_load((gv4u*)(ch + (g0 + g) * rs * 256 + la * 16));
      R.SA[u] = mx_load_sa<G>(ch, rs, lane, g0);
    }
  }
}

// mx_load_a without control flow between the loads: steps past s1 (s1 > s0)
// reload step s1 - 1 (mx_compute skips them), so the loads of every step go out
// back to back even where the registers already hold earlier values.
template <int S, int G = 4>
__device__ __forceinline__ void mx_load_a_flat(MxRegs<S, G>& R, const uint8_t* __restrict__ tile, const MxGeom& G_,
                                               int s0, int s1, int g0 = 0) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  const int lane = __lane_id(), grp = lane >> 4;
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int s = min(s0 + u, s1 - 1);
    const int rs = s < G_.ns - 1 ? 4 : G_.rlast;
    const uint8_t* ch = tile + (int64_t)s * MX_STEP_BYTES;
    const int la = grp < rs ? lane : 16 * rs - 1;
#pragma unroll
    for (int g = 0; g < G; ++g) R.A[u][g] = __builtin_nontemporal_load((gv4u*)(ch + (g0 + g) * rs * 256 + la * 16));
    R.SA[u] = mx_load_sa<G>(ch, rs, lane, g0);
  }
}

// Activation operands of the same steps for this lane's column, whose token's
// terms start at xtok (step xs0 of that token; in LDS when BLDS): column
// c = lane % 16 is term c % XQ_NT of the lane's token. FLAT (s1 > s0): no
// branch between the steps' loads -- steps past s1 reload step s1 - 1 -- so a
// wait for one step's operands need not wait for the later steps'.
template <int S, bool BLDS, int G = 4, bool FLAT = false>
__device__ __forceinline__ void mx_load_b_at(MxRegs<S, G>& R, const uint8_t* __restrict__ xtok, int xs0, int s0,
                                             int s1) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  typedef const __attribute__((address_space(3))) v4u lv4u;
  typedef const __attribute__((address_space(3))) uint32_t lu32;
  const int lane = __lane_id();
  const int grp = lane >> 4, term = lane & (XQ_NT - 1);
  const uint8_t* xt = xtok + (grp * XQ_NT + term) * 32;
  const uint8_t* xst = xtok + XQ_CODES + (grp * XQ_NT + term) * 4;
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int s = FLAT ? min(s0 + u, s1 - 1) : s0 + u;
    if (FLAT || s < s1) {
      const int64_t xo = (int64_t)(s - xs0) * XQ_STEP;
      if (BLDS) {
        R.B0[u] = *(lv4u*)(xt + xo);
        R.B1[u] = *(lv4u*)(xt + xo + 16);
        R.SB[u] = *(lu32*)(xst + xo);
      } else {
        R.B0[u] = *(gv4u*)(xt + xo);
        R.B1[u] = *(gv4u*)(xt + xo + 16);
        R.SB[u] = *(gu32*)(xst + xo);
      }
    }
  }
}

// Activation operands of S K-steps held apart from the weights: with two of
// them a token loop requests the next token group's operands before the MFMAs
// of this one wait on theirs.
template <int S>
struct MxB {
  v4u B0[S], B1[S];
  uint32_t SB[S];
};

// mx_load_b_at<S, false, G, true> into an MxB (global terms, no branch between the steps' loads).
template <int S>
__device__ __forceinline__ void mx_load_bb(MxB<S>& B, const uint8_t* __restrict__ xtok, int xs0, int s0, int s1) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  const int lane = __lane_id();
  const int grp = lane >> 4, term = lane & (XQ_NT - 1);
  const uint8_t* xt = xtok + (grp * XQ_NT + term) * 32;
  const uint8_t* xst = xtok + XQ_CODES + (grp * XQ_NT + term) * 4;
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int64_t xo = (int64_t)(min(s0 + u, s1 - 1) - xs0) * XQ_STEP;
    B.B0[u] = *(gv4u*)(xt + xo);
    B.B1[u] = *(gv4u*)(xt + xo + 16);
    B.SB[u] = *(gu32*)(xst + xo);
  }
}

template <int S, int G>
__device__ __forceinline__ void mx_take_b(MxRegs<S, G>& R, const MxB<S>& B) {
#pragma unroll
  for (int u = 0; u < S; ++u) {
    R.B0[u] = B.B0[u];
    R.B1[u] = B.B1[u];
    R.SB[u] = B.SB[u];
  }
}

// The same for tokens laid out xq_stride bytes apart from xq (token 0):
// column c = token * XQ_NT + term for tokens < ntok; columns of tokens >=
// ntok repeat token ntok - 1 and are not read back.
template <int S, bool BLDS, int G = 4>
__device__ __forceinline__ void mx_load_b(MxRegs<S, G>& R, const uint8_t* __restrict__ xq, int xs0, int64_t xq_stride,
                                          int ntok, int s0, int s1) {
  const int tok0 = (__lane_id() & 15) / XQ_NT;
  const int tok = tok0 < ntok ? tok0 : ntok - 1;
  mx_load_b_at<S, BLDS, G>(R, xq + (int64_t)tok * xq_stride, xs0, s0, s1);
}

// mx_load_a and mx_load_b (global activation terms) of the same steps,
// interleaved step by step: the loads retire in issue order, so step u's
// MFMAs wait only for steps 0..u, weights and activations alike. No branch
// between the steps' loads (s1 > s0): steps past s1 reload step s1 - 1, which
// mx_compute skips -- with a branch per step the compiler waits at each merge
// for the loads before it, and the steps' loads go out one round trip apart.
template <int S, int G = 4>
__device__ __forceinline__ void mx_load_ab(MxRegs<S, G>& R, const uint8_t* __restrict__ tile, const MxGeom& G_,
                                           int s0, int s1, const uint8_t* __restrict__ xq, int xs0,
                                           int64_t xq_stride, int ntok, int g0 = 0) {
  typedef const __attribute__((address_space(1))) v4u gv4u;
  typedef const __attribute__((address_space(1))) uint32_t gu32;
  const int lane = __lane_id(), grp = lane >> 4;
  const int tok0 = (lane & 15) / XQ_NT;
  const int tok = tok0 < ntok ? tok0 : ntok - 1;
  const uint8_t* xtok = xq + (int64_t)tok * xq_stride;
  const int term = lane & (XQ_NT - 1);
  const uint8_t* xt = xtok + (grp * XQ_NT + term) * 32;
  const uint8_t* xst = xtok + XQ_CODES + (grp * XQ_NT + term) * 4;
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int s = min(s0 + u, s1 - 1);
    const int rs = s < G_.ns - 1 ? 4 : G_.rlast;
    const uint8_t* ch = tile + (int64_t)s * MX_STEP_BYTES;
    const int la = grp < rs ? lane : 16 * rs - 1;
#pragma unroll
    for (int g = 0; g < G; ++g) R.A[u][g] = __builtin_nontemporal_load((gv4u*)(ch + (g0 + g) * rs * 256 + la * 16));
    R.SA[u] = mx_load_sa<G>(ch, rs, lane, g0);
    const int64_t xo = (int64_t)(s - xs0) * XQ_STEP;
    R.B0[u] = *(gv4u*)(xt + xo);
    R.B1[u] = *(gv4u*)(xt + xo + 16);
    R.SB[u] = *(gu32*)(xst + xo);
  }
}

// D[g] (rows 16 (g0 + g) .. + 15 of the tile, 16 columns) += the loaded steps
// (the same G_, s0, s1, g0 as mx_load_a).
template <int S, int G = 4>
__device__ __forceinline__ void mx_compute(const MxRegs<S, G>& R, const MxGeom& G_, int s0, int s1, v4f (&D)[G],
                                           int g0 = 0) {
#pragma unroll
  for (int u = 0; u < S; ++u) {
    const int s = s0 + u;
    if (s >= s1) break;
    const uint32_t sa = R.SA[u];  // byte g: group g0 + g (stand-in lanes: 0)
    const uint32_t sb = R.SB[u];
    const v8i b = {(int)R.B0[u].x, (int)R.B0[u].y, (int)R.B0[u].z, (int)R.B0[u].w,
                   (int)R.B1[u].x, (int)R.B1[u].y, (int)R.B1[u].z, (int)R.B1[u].w};
    const v8i a0 = {(int)R.A[u][0].x, (int)R.A[u][0].y, (int)R.A[u][0].z, (int)R.A[u][0].w, 0, 0, 0, 0};
    D[0] = NSX_MFMA_SCALE(a0, b, D[0], 0, sa, sb);
    if constexpr (G >= 2) {
      const v8i a1 = {(int)R.A[u][1].x, (int)R.A[u][1].y, (int)R.A[u][1].z, (int)R.A[u][1].w, 0, 0, 0, 0};
      D[1] = NSX_MFMA_SCALE(a1, b, D[1], 1, sa, sb);
    }
    if constexpr (G == 4) {
      const v8i a2 = {(int)R.A[u][2].x, (int)R.A[u][2].y, (int)R.A[u][2].z, (int)R.A[u][2].w, 0, 0, 0, 0};
      const v8i a3 = {(int)R.A[u][3].x, (int)R.A[u][3].y, (int)R.A[u][3].z, (int)R.A[u][3].w, 0, 0, 0, 0};
      D[2] = NSX_MFMA_SCALE(a2, b, D[2], 2, sa, sb);
      D[3] = NSX_MFMA_SCALE(a3, b, D[3], 3, sa, sb);
    }
  }
}

// A whole K range [s0, s1) in passes of S steps.
template <int S, bool BLDS>
__device__ __forceinline__ void mx_tile_mfma(const uint8_t* __restrict__ tile, const MxGeom& G, int s0, int s1,
                                             const uint8_t* __restrict__ xq, int xs0, int64_t xq_stride, int ntok,
                                             v4f (&D)[4]) {
  for (int p0 = s0; p0 < s1; p0 += S) {
    MxRegs<S> R;
    mx_load_a<S>(R, tile, G, p0, s1);
    mx_load_b<S, BLDS>(R, xq, xs0, xq_stride, ntok, p0, s1);
    mx_compute<S>(R, G, p0, s1, D);
  }
}

// Sum the XQ_NT term columns of D: afterwards lane l with (l & 3) == 0 holds,
// for token (l & 15) / 4, rows 16 g + 4 (l / 16) + i (relative to the first
// row group) in D[g][i].
template <int G>
__device__ __forceinline__ void mx_sum_terms(v4f (&D)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = D[g][i];
      v += nsx_dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]: lane ^ 1
      v += nsx_dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]: lane ^ 2
      D[g][i] = v;
    }
  }
}
