/*
 * nurostream_amd -- C ABI of the MI355X (gfx950) MoE expert hot path.
 *
 * Every entry point takes plain device pointers, element/byte counts and a
 * HIP stream handle (`void *stream`, a hipStream_t; NULL = the null stream),
 * returns an NSX_* status code, and never allocates device memory. The
 * message of the last failure on the calling thread is nsx_last_error().
 *
 * The reference (hareramray/nurostream, Python + Triton) has no C ABI; each
 * function below names the Python seam it replaces (paths relative to the
 * reference's neurostream/ package).
 */
#ifndef NUROSTREAM_AMD_H
#define NUROSTREAM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSX_ABI_VERSION 3

/* status codes; the Python shim maps them onto the reference's exceptions */
enum {
  NSX_OK = 0,
  NSX_EINVAL = 1,   /* ValueError: shapes, sizes, windows */
  NSX_ETYPE = 2,    /* TypeError: wrong buffer element type */
  NSX_ENOTIMPL = 3, /* NotImplementedError: unsupported ggml type */
  NSX_EHIP = 4,     /* RuntimeError: HIP runtime failure */
  NSX_EKERNEL = 5,  /* RuntimeError: a kernel's own bounded check failed */
  NSX_EIO = 6,      /* OSError (EOFError for a short read): a file read failed */
  NSX_ETIMEDOUT = 7 /* TimeoutError: a wait ran out of time */
};

/* ggml type ids (format/gguf.py:19-35) */
enum {
  NSX_F32 = 0, NSX_F16 = 1, NSX_Q4_0 = 2, NSX_Q8_0 = 8, NSX_Q4_K = 12,
  NSX_Q6_K = 14, NSX_BF16 = 30, NSX_MXFP4 = 39
};

/* activation / output element types */
enum { NSX_DT_F32 = 0, NSX_DT_F16 = 1, NSX_DT_BF16 = 2 };

/* expert weight layouts */
enum {
  NSX_LAYOUT_GGUF = 0, /* raw GGUF rows, as read from the file */
  NSX_LAYOUT_T64 = 1   /* 64-row interleaved tiles (nsx_t64_pack) */
};

/* routers and activations */
enum { NSX_ROUTE_GPTOSS = 0, NSX_ROUTE_QWEN3 = 1 };
enum { NSX_ACT_CLAMPED_SWIGLU = 0, NSX_ACT_SILU_MUL = 1 };
/* How nsx_moe_forward runs the routed experts: per (token, expert) pair, or
 * grouped (pairs sorted by expert; each active expert's weights read once per
 * work item of up to 16 of its tokens; t64 MXFP4 layers, and stacked 16-byte
 * aligned Q4_K rows with K <= 4096). MFMA: grouped stacked Q4_K on the
 * matrix cores (f16 products of the exact sc * q codes and a two-term split
 * of the activations; outputs within 1e-5 of the per-pair kernels' rather
 * than identical to them). AUTO groups t64 layers from T >= 3 and takes MFMA
 * for stacked aligned Q4_K layers from T * top_k >= 104; below that it runs
 * pairs. */
enum { NSX_DISPATCH_AUTO = 0, NSX_DISPATCH_PAIRS = 1, NSX_DISPATCH_GROUPED = 2, NSX_DISPATCH_MFMA = 3 };

const char *nsx_last_error(void);
int nsx_abi_version(void);

/* Checks, on the current device, that the gfx950 FP4 conversion instruction
 * decodes all 256 byte values exactly as the MXFP4 table does; `scratch` is
 * one device uint32. No reference counterpart (a load-time self test). */
int nsx_selftest(uint32_t *scratch, void *stream);

/* No reference counterpart: a read-bandwidth probe, the same-box denominator
 * the expert kernels' HBM fractions are set beside. `workgroups` workgroups of
 * `threads` threads (a multiple of 64, <= 1024) read `bytes` (a multiple of
 * 16, src 16-byte aligned) in equal contiguous shares with 16-byte
 * nontemporal loads, 8 per thread in flight; nothing is written unless the
 * bytes fold to one fixed word (then one word of sink). */
int nsx_read_probe(const void *src, int64_t bytes, int workgroups, int threads,
                   uint32_t *sink, void *stream);

/* compute/quant.py:153-184 dequantize(raw, dtype, n_elements, out_dtype).
 * raw: `raw_bytes` bytes of ggml blocks (any alignment); out: n_elements of
 * out_dtype. Bit-exact with the reference for Q4_0, Q8_0, Q4_K, Q6_K, MXFP4
 * (Q6_K: compute/quant.py:84-107). */
int nsx_dequantize(int ggml_type, const void *raw, int64_t raw_bytes,
                   int64_t n_elements, void *out, int out_dtype, void *stream);

/* compute/triton_kernels.py:199-228 fused_gemv(raw, dtype, x, n_rows, K).
 * y[t, r] = sum_k x[t, k] * dequant(raw)[r, k] for t < T, fp32 accumulate.
 * raw: n_rows * row_bytes GGUF bytes (any alignment for Q4_0, Q8_0, Q6_K and
 * MXFP4, 4-byte aligned for Q4_K); x: (T, K) row-major in x_dtype; y:
 * (T, n_rows) fp32. The reference fuses only T == 1 (Q6_K:
 * triton_kernels.py:97-143); here T <= 16. */
int nsx_fused_gemv(int ggml_type, const void *raw, int64_t n_rows, int64_t K,
                   const void *x, int x_dtype, int64_t T, float *y, void *stream);
/* nsx_fused_gemv with the epilogue of model/gpt_oss.py:97-99,114
 * (x + _biased_linear(...)): y[t, r] = resid[t, r] + (dot + bias[r]);
 * bias (n_rows) and resid ((T, n_rows), may be y) are optional (NULL). */
int nsx_fused_gemv_ex(int ggml_type, const void *raw, int64_t n_rows, int64_t K,
                      const void *x, int x_dtype, int64_t T, float *y, const float *bias,
                      const float *resid, void *stream);
/* nsx_fused_gemv_ex for one token whose input is the block norm of the
 * residual stream: y = resid + (W . h + bias) with h = rms_norm(x + r) * w,
 * the rms_norm of compute/ops.py:14-20 ahead of the QKV linear
 * (model/gpt_oss.py:101-114) or the LM head (model/gpt_oss.py:207-228), in
 * the bits nsx_add_rmsnorm gives h -- one launch instead of two. x, r, w: K
 * floats (r, w optional), x 16-byte aligned, K <= 4096; s (optional) receives
 * x + r. Other workgroups still read x, r and resid while s and y are
 * written, so s must not overlap x, r, resid or y, and y must not overlap x
 * or r and is either resid itself or apart from it (NSX_EINVAL otherwise). */
int nsx_fused_gemv_norm(int ggml_type, const void *raw, int64_t n_rows, int64_t K,
                        const float *x, const float *r, const float *w, float eps, float *s,
                        float *y, const float *bias, const float *resid, void *stream);

/* 64-row interleaved tiles for VRAM-resident expert slabs. No reference
 * counterpart: residency/cache.py:369-389 admit_slab keeps the raw bytes;
 * here admission re-lays the same bits out so one 128-bit load per lane
 * covers one row's block (MXFP4 only). pack/unpack are exact inverses. */
int64_t nsx_t64_bytes(int ggml_type, int64_t n_rows, int64_t K);
int nsx_t64_pack(int ggml_type, const void *raw, int64_t n_rows, int64_t K,
                 void *t64, void *stream);
int nsx_t64_unpack(int ggml_type, const void *t64, int64_t n_rows, int64_t K,
                   void *raw, void *stream);
/* fused_gemv over rows [row_lo, row_hi) of a t64 matrix; y: (T, row_hi-row_lo) */
int nsx_t64_gemv(int ggml_type, const void *t64, int64_t n_rows, int64_t K,
                 int64_t row_lo, int64_t row_hi, const void *x, int x_dtype,
                 int64_t T, float *y, void *stream);

/* moe/router.py:59-69 route() (mode NSX_ROUTE_QWEN3) and
 * model/gpt_oss.py:116-121 _route() (mode NSX_ROUTE_GPTOSS).
 * h: (T, K) fp32; w: (n_expert, K) in w_dtype (NSX_F32 / NSX_BF16 / NSX_F16);
 * bias: (n_expert,) fp32 or NULL. ids/weights: (T, top_k), ordered by
 * descending value with ties to the lower expert index; logits: (T, n_expert)
 * fp32 output. */
int nsx_router_topk(const float *h, int64_t T, int64_t K, const void *w,
                    int w_dtype, const float *bias, int64_t n_expert, int top_k,
                    int mode, int32_t *ids, float *weights, float *logits,
                    void *stream);

/* One MoE FFN layer: router -> routed experts -> weighted combine.
 * model/gpt_oss.py:123-177 _ffn_block (neuron path, without the residual)
 * and moe/router.py:173-219 moe_ffn. Expert tensors are given per expert as
 * device arrays of device addresses (n_expert entries each). */
typedef struct nsx_moe_layer {
  int32_t ggml_type;    /* expert weight format (NSX_MXFP4 / NSX_Q4_K / NSX_Q4_0) */
  int32_t layout;       /* NSX_LAYOUT_GGUF or NSX_LAYOUT_T64 */
  int32_t n_expert;
  int32_t top_k;
  int32_t n_embd;       /* hidden size: K of gate/up, rows of down */
  int32_t n_ff;         /* expert width: rows of gate/up, K of down */
  int32_t router_mode;  /* NSX_ROUTE_* */
  int32_t act;          /* NSX_ACT_* */
  float alpha;          /* clamped SwiGLU alpha (1.702) */
  float limit;          /* clamped SwiGLU limit (7.0) */
  const void *router_w; /* (n_expert, n_embd) */
  int32_t router_dtype; /* NSX_F32 / NSX_BF16 / NSX_F16 */
  int32_t dispatch;     /* NSX_DISPATCH_* */
  const float *router_bias;  /* (n_expert,) or NULL */
  /* Expert e of a projection lives at base + e * stride when base is not
   * NULL, else at ptrs[e] (a device array of n_expert device addresses). */
  const uint64_t *gate_ptrs;
  const uint64_t *up_ptrs;
  const uint64_t *down_ptrs;
  const float *gate_bias; /* (n_expert, n_ff) or NULL */
  const float *up_bias;   /* (n_expert, n_ff) or NULL */
  const float *down_bias; /* (n_expert, n_embd) or NULL */
  const void *gate_base;
  const void *up_base;
  const void *down_base;
  int64_t gate_stride;
  int64_t up_stride;
  int64_t down_stride;
  /* t64 layout only, optional: per projection a device array of n_expert x
   * ceil(rows / 64) tile addresses, tile t of expert e at X_tiles[e * tiles +
   * t]; when set it takes precedence over base/ptrs. A tile may sit anywhere
   * the device can read, pinned host memory included (see
   * nsx_host_device_address): the kernels then read it over PCIe. */
  const uint64_t *gate_tiles;
  const uint64_t *up_tiles;
  const uint64_t *down_tiles;
} nsx_moe_layer;

/* Bytes of caller-provided workspace for T tokens. The caller zeroes the
 * workspace once before its first use (padding inside it must read as zero);
 * calls that share one workspace must not overlap. */
int64_t nsx_moe_workspace_bytes(const nsx_moe_layer *L, int64_t T);

/* out: (T, n_embd) fp32 = sum over the token's experts, in ascending expert
 * id, of weight * expert_ffn(h). ids/weights: (T, top_k) outputs. */
int nsx_moe_forward(const nsx_moe_layer *L, const float *h, int64_t T,
                    float *out, int32_t *ids, float *weights, void *workspace,
                    int64_t workspace_bytes, void *stream);

/* One block of a stacked GPT-OSS FFN (model/gpt_oss.py:123-177: the block's
 * input norm, then the routed experts): x_out = x + r, and out, ids, weights
 * as nsx_moe_forward of h = rms_norm(x + r) * norm_w (eps; norm_w may be
 * NULL), h being what nsx_add_rmsnorm(x, r, ...) computes, bit for bit. The
 * norm runs inside the router kernel, which is the only reader of h in the
 * t64 layout: no separate launch and no h in memory. For t64 layers below
 * 16 tokens with n_embd <= 4096 (NSX_ENOTIMPL otherwise: callers then run
 * nsx_add_rmsnorm and nsx_moe_forward). x_out must not overlap x or r; out
 * may be r (the router is done with r before any expert kernel writes out).
 * Same workspace as nsx_moe_forward. */
int nsx_moe_forward_norm(const nsx_moe_layer *L, const float *x, const float *r,
                         const float *norm_w, float eps, int64_t T, float *x_out,
                         float *out, int32_t *ids, float *weights, void *workspace,
                         int64_t workspace_bytes, void *stream);

/* One block of a stacked GPT-OSS FFN whose output feeds the next block
 * (model/gpt_oss.py:123-177, x_{l+1} = x_l + moe(h_l), then the next block's
 * input norm, compute/ops.py:14-20): nsx_moe_forward of h, then x_out =
 * x + out and h_out = rms_norm(x_out) * norm_w (eps; norm_w may be NULL) --
 * the bits of nsx_moe_forward followed by nsx_add_rmsnorm(x, out, ...). On the
 * grouped path the combine and the add + norm are one launch; the MoE output
 * itself is not written. x_out may be x; h_out must not overlap x or x_out
 * (it may be h). n_embd <= 4096. Same workspace as nsx_moe_forward. */
int nsx_moe_forward_addnorm(const nsx_moe_layer *L, const float *h, int64_t T,
                            const float *x, const float *norm_w, float eps, float *x_out,
                            float *h_out, int32_t *ids, float *weights, void *workspace,
                            int64_t workspace_bytes, void *stream);

/* The decode chain of stacked GPT-OSS FFN blocks at T = 1
 * (model/gpt_oss.py:123-177 layer after layer; the router of
 * model/gpt_oss.py:116-121 regrouped): x += moe(rms_norm(x) * norm_w), in
 * place (x: n_embd floats, the token's residual stream). out, ids, weights
 * as nsx_moe_forward of h = rms_norm(x) * norm_w.
 * share_in NULL: this block routes from x itself (a norm, a router and the
 * per-pair gate/up launch). Otherwise share_in holds this block's router
 * shares, written by the previous block's call: per work item of that call's
 * down kernel the partial dot of x * norm_w with each router row and the
 * partial sum of x^2; the gate/up kernel adds them in a fixed order, so
 * logits = (dot) / rms + bias and the top-k need no router launch, and each
 * of its workgroups quantizes h = (x / rms) * norm_w itself. With `next`
 * (the next block, and its norm weight next_norm_w, may be NULL) the down
 * kernel writes the next block's shares to share_out (which may be
 * share_in). h equals nsx_add_rmsnorm's but for the rms's summation order, so
 * outputs match the separate norm to rounding, not bit for bit. t64 layers on
 * the per-pair kernels (not NSX_DISPATCH_GROUPED), n_embd a multiple of 16 up
 * to 3072, experts a multiple of 4 up to 128 (NSX_ENOTIMPL otherwise). x, out and the
 * share buffers must not overlap. Same workspace as nsx_moe_forward(T = 1).
 * phases: NSX_CHAIN_GATE_UP (the gate/up launch, with the norm and router
 * before it when share_in is NULL), NSX_CHAIN_DOWN (the down launch: out, the
 * residual add, the next block's shares), or both -- one launch alone reads
 * what the other left, for timing one of them. No reference counterpart as
 * one call: the reference runs the same steps as separate torch calls. */
#define NSX_CHAIN_GATE_UP 1
#define NSX_CHAIN_DOWN 2
int64_t nsx_moe_chain_share_bytes(const nsx_moe_layer *L);
int nsx_moe_chain_t1(const nsx_moe_layer *L, float *x, const float *norm_w, float eps,
                     const float *share_in, const nsx_moe_layer *next,
                     const float *next_norm_w, float *share_out, float *out,
                     int32_t *ids, float *weights, void *workspace,
                     int64_t workspace_bytes, int phases, void *stream);

/* One phase of nsx_moe_forward: NSX_PHASE_ROUTER (logits, the top-k and the
 * ids/weights outputs, for every layout and dispatch; in the t64 layout also
 * the activation terms of h), NSX_PHASE_GATE_UP (grouped dispatch: the sort
 * by expert; expert gate/up GEMVs + activation; the per-pair t64 kernel
 * selects the top-k again from the logits and rewrites the same ids/weights),
 * NSX_PHASE_DOWN (expert down GEMVs; per-pair dispatch also the weighted
 * combine into out)
 * and NSX_PHASE_COMBINE (grouped dispatch: the ascending-expert combine;
 * otherwise nothing). A phase reads what the earlier phases of the same call
 * sequence left in the workspace; running the four in order is
 * nsx_moe_forward (which skips the top-k launch where a later kernel selects
 * the top-k itself: the per-pair t64 gate/up kernel, per-pair Q4_K below 16
 * tokens, and below 16 tokens on the grouped path the sort kernel -- or, for
 * t64 layers with at most 64 (token, expert) pairs, the grouped gate/up
 * kernel, which then sorts the pairs itself and launches no sort kernel).
 * Only a call that runs the router and gate/up phases together does this: a
 * call that ends with the router phase always writes ids/weights. Callers
 * use it to interleave other work (block reads, another layer's router)
 * between phases or to time one phase; the
 * reference runs these steps as separate torch calls
 * (model/gpt_oss.py:123-177). */
#define NSX_PHASE_ROUTER 0
#define NSX_PHASE_GATE_UP 1
#define NSX_PHASE_DOWN 2
#define NSX_PHASE_COMBINE 3
int nsx_moe_phase(const nsx_moe_layer *L, int phase, const float *h, int64_t T,
                  float *out, int32_t *ids, float *weights, void *workspace,
                  int64_t workspace_bytes, void *stream);

/* No counterpart in the reference. nsx_moe_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): it allocates nothing and takes no
 * workspace. Its workspace is a library-owned device array of
 * NSX_STATIC_WORKSPACE_BYTES per GPU (each GPU the library runs on holds its
 * own copy until the process ends); a call whose workspace
 * (nsx_moe_workspace_bytes, for at most one grouped pass of tokens) exceeds
 * it fails with NSX_EINVAL. Each call first clears the part it uses, on the
 * stream, with a fill kernel. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other host threads) race on
 * it. Outputs are those of nsx_moe_forward. */
#define NSX_STATIC_WORKSPACE_BYTES (32ll << 20)
int nsx_moe_forward_static(const nsx_moe_layer *L, const float *h, int64_t T,
                           float *out, int32_t *ids, float *weights,
                           void *stream);

/* compute/ops.py:14-20 rms_norm in fp32 over rows of n (n <= 4096), with the
 * residual add of model/gpt_oss.py:177 folded in: sum = x + r and
 * y = sum * rsqrt(mean(sum^2) + eps) * w. r, w, sum and y may each be NULL
 * (no residual, unit weight, no sum or no norm output; not both outputs);
 * sum and y may alias x or r. */
int nsx_add_rmsnorm(const float *x, const float *r, int64_t T, int64_t n,
                    float eps, const float *w, float *sum, float *y,
                    void *stream);

/* Expert blocks split between HBM and pinned host RAM (BASELINE config 5b).
 * nsx_copy_blocks_async: dst[i] <- src[i] (bytes[i]) for n segments, each a
 * DMA copy on `stream` (host-to-device from pinned memory, or any direct
 * copy), then `event` (a hipEvent_t, may be NULL) is recorded on the stream.
 * The block prefetcher's host-to-device step: io/stream.py:200-216
 * submit_rows and the block copy of compute/blockffn.py:341-378.
 * nsx_gather_copy: the same for device-to-device segments (16-byte aligned
 * addresses and sizes), as one kernel per 128 segments. Every destination
 * (and gather source) range is checked to lie inside one device allocation
 * (hipMemGetAddressRange: for memory from a caching allocator that is the
 * allocator's segment, so staying inside the intended buffer is the
 * caller's contract). The segment arrays are host arrays, read during the
 * call. */
int nsx_copy_blocks_async(int64_t n, const uint64_t *src, const uint64_t *dst,
                          const int64_t *bytes, void *stream, void *event);
int nsx_gather_copy(int64_t n, const uint64_t *src, const uint64_t *dst,
                    const int64_t *bytes, void *stream);

/* The device address of pinned host memory (allocated pinned, e.g. by
 * hipHostMalloc or torch's pin_memory), for tile tables that point into it.
 * Fails (NSX_EHIP) if host is not device-mapped pinned memory. */
int nsx_host_device_address(const void *host, uint64_t *device_address);

/* ---- the step either side of the FFN in a GPT-OSS decode token ----
 * The token's position is read from device memory (`pos`, an int32), so a
 * captured graph of a whole decode token replays token after token;
 * nsx_pos_advance moves it on. KV cache: K and V each
 * [n_kv][ctx_max][head_dim] fp32. head_dim is 64 (GPT-OSS). */

/* compute/blockffn.py:470-487 gather_embeddings: out[i] = dequant(row
 * ids[i]) as fp32 (K elements), ids in device memory; an id outside
 * [0, n_rows) gives zeros. Types: F32, F16, BF16 and the block types. */
int nsx_dequantize_rows(int ggml_type, const void *raw, int64_t n_rows, int64_t K, const int32_t *ids,
                        int64_t n_ids, float *out, void *stream);

/* model/gpt_oss.py:42-58 (yarn_tables), 101-110 (q/k/v bias, rotary,
 * KVCache.append) for one token: qkv holds the q (n_head rows), k and v
 * (n_kv rows each) projections, head_dim each; biases are added (NULL:
 * none); q and k rows are rotated by angle pos * inv_freq[i] (fp32) with
 * cos and sin scaled by amplitude, q in place; k and v go into the caches at
 * row pos. Nothing is written unless 0 <= pos < ctx_max. */
int nsx_rope_kv_append(float *qkv, const float *q_bias, const float *k_bias, const float *v_bias, int n_head,
                       int n_kv, int head_dim, const float *inv_freq, float amplitude, const int32_t *pos,
                       float *k_cache, float *v_cache, int64_t ctx_max, void *stream);
/* Workspace bytes of nsx_attn_decode for this cache length. */
int64_t nsx_attn_workspace_bytes(int n_head, int head_dim, int64_t ctx_max);
/* model/gpt_oss.py:73-85 sink_attention for the query token at position
 * pos: keys 0..pos (the last `window` of them when window > 0), query head h
 * reading kv head h / (n_head / n_kv), scores times `scale`, softmax over
 * [scores, sinks[h]] with the sink column dropped (sinks NULL: no sink).
 * out: [n_head][head_dim] fp32. */
int nsx_attn_decode(const float *q, const float *k_cache, const float *v_cache, const float *sinks, int n_head,
                    int n_kv, int head_dim, const int32_t *pos, int64_t ctx_max, int window, float scale,
                    void *workspace, float *out, void *stream);
/* nsx_rope_kv_append followed by nsx_attn_decode in one launch (two with the
 * chunk combine): qkv is the token's raw [n_head + 2 n_kv][head_dim] block
 * (the QKV projection without its bias), left unchanged; the token's k (with
 * bias and rotary) and v (with bias) rows are appended to the caches at pos,
 * and out is the attention of the rotated q. Results are bit-identical to the
 * two calls. Replaces the same reference lines: model/gpt_oss.py:42-58,
 * 73-85, 101-114. */
int nsx_attn_decode_qkv(const float *qkv, const float *q_bias, const float *k_bias, const float *v_bias,
                        const float *inv_freq, float amplitude, const float *sinks, int n_head, int n_kv,
                        int head_dim, const int32_t *pos, float *k_cache, float *v_cache, int64_t ctx_max,
                        int window, float scale, void *workspace, float *out, void *stream);
/* *pos += n on the stream (one thread). */
int nsx_pos_advance(int32_t *pos, int32_t n, void *stream);

/* ---- disk reader: GGUF bytes from a file into device (or host) memory ----
 * Replaces the reference's thread-pool reader and the disk side of its
 * streaming source (io/reader.py AsyncReader, io/stream.py StreamingSource):
 * n_workers threads issue positional reads (O_DIRECT where the file system
 * allows it) into staging buffers, and a read into device memory is copied
 * from its pinned staging buffer on the reader's copy stream as soon as it
 * lands, with no host thread in between. Reads larger than a staging buffer
 * are split across buffers and workers. */
typedef struct nsx_reader nsx_reader;

enum { NSX_READ_DIRECT = 1 }; /* try O_DIRECT (page-cache bypass); buffered where refused */

typedef struct {
  int64_t requests;     /* reads submitted */
  int64_t bytes_read;   /* bytes delivered */
  double read_seconds;  /* time spent inside reads, summed over the workers */
  double first_read;    /* CLOCK_MONOTONIC seconds: start of the first read */
  double last_read;     /* end of the latest read */
  int32_t direct;       /* 1 while reads bypass the page cache */
  int32_t n_workers;
} nsx_reader_stats;

/* io/reader.py:72-92 AsyncReader(path, n_workers). n_slots staging buffers
 * of slot_bytes each (>= 3 x 4096); pinned host memory when device >= 0 (the
 * device whose memory reads land in, copied on copy_stream, a hipStream_t of
 * that device), plain host memory when device < 0 (host destinations only).
 * n_workers == 0 gives a reader that never reads: a wait can only time out
 * (for tests of that path). */
int nsx_reader_open(const char *path, int n_workers, int flags, int n_slots, int64_t slot_bytes,
                    int device, void *copy_stream, nsx_reader **out);
/* io/reader.py:116-118 submit(offset, nbytes), the read under
 * io/stream.py:200-216 submit_rows: queue file bytes [offset, offset +
 * nbytes) into dst -- device memory when dst_on_device (the copy stream
 * first waits for the work already queued on `stream`, the stream dst was
 * allocated on), else host memory. A read past the end of the file fails
 * at wait. */
int nsx_reader_submit(nsx_reader *r, int64_t offset, int64_t nbytes, void *dst, int dst_on_device,
                      void *stream, uint64_t *ticket);
/* 1 once the ticket's bytes are read and their copies queued, 0 while
 * pending (the fut.done() of io/reader.py:129); NSX_EINVAL (< 0 as
 * -NSX_EINVAL) for an unknown ticket. */
int nsx_reader_poll(nsx_reader *r, uint64_t ticket);
/* io/reader.py:127-139 wait(fut): block up to timeout_us (< 0: no limit)
 * until the ticket's reads are done, then order `stream` after their device
 * copies (host destinations are complete on return), and retire the ticket.
 * NSX_EIO if a read failed or came up short (the ticket is retired),
 * NSX_ETIMEDOUT if the time ran out (the ticket stays pending). */
int nsx_reader_wait(nsx_reader *r, uint64_t ticket, int64_t timeout_us, void *stream);
/* io/reader.py:31-69 IOStats (the reader-side counters). */
int nsx_reader_get_stats(nsx_reader *r, nsx_reader_stats *out);
/* io/reader.py:141-148 close(): drop queued reads (their tickets fail), join
 * the workers, wait for copies out of staging, free everything. */
int nsx_reader_close(nsx_reader *r);

#ifdef __cplusplus
}
#endif

#endif /* NUROSTREAM_AMD_H */
