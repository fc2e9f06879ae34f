/*
 * e4b.h -- C ABI of libe4b.so, the MI355X (gfx950) batch-1 decode library.
 *
 * Plain C: pointers, sizes, return codes.  No C++ exceptions cross this ABI.
 * Return codes: 0 = ok, negative = error (see E4B_E*); e4b_last_error() gives
 * the message of the last failure on the calling thread.
 *
 * Ownership: input buffers are borrowed for the duration of a call; output
 * buffers are caller-allocated.  Device pointers are HIP device addresses
 * (from e4b_dev_alloc or any other HIP allocation on the current device).
 * `stream` arguments are hipStream_t values passed as void*; NULL means the
 * library's default stream (the HIP null stream).  Kernel-level entry points
 * are asynchronous on that stream; engine calls that return results are
 * synchronous.
 *
 * Workspace: kernel-level entry points that need scratch (split-K and argmax
 * partials, f16 staging of an f32 x) share one grow-only buffer per device.
 * A call that needs more than it holds allocates a larger one (hipMalloc,
 * no device synchronisation; the outgrown buffer is kept until the process
 * ends, so queued or captured work that holds it stays valid).  Inside a
 * stream capture such a call fails with E4B_EINVAL instead: make the same
 * call once before capturing.  Calls on one device that use the workspace
 * must be ordered (one stream at a time).
 *
 * Citations name the reference interface each entry point replaces
 * (paths relative to the Verilean/e4b-webgpu checkout).
 */
#ifndef E4B_H
#define E4B_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define E4B_OK 0
#define E4B_EINVAL (-1)   /* bad argument / shape                        */
#define E4B_ENOMEM (-2)   /* device or host allocation failed             */
#define E4B_EHIP (-3)     /* HIP runtime error                            */
#define E4B_ESTATE (-4)   /* call out of order (e.g. step before finalize) */
#define E4B_ENOTENSOR (-5) /* required tensor missing at finalize          */
#define E4B_ERANGE (-6)   /* position / token / size beyond capacity       */

/* ggml tensor type ids, as src/gguf.js:3 GGML */
#define E4B_GGML_F32 0
#define E4B_GGML_F16 1
#define E4B_GGML_Q4_0 2
#define E4B_GGML_Q6_K 14

/* activation dtypes for kernel-level entry points */
#define E4B_DT_F32 0     /* f32[n]                                              */
#define E4B_DT_F16 1     /* f16[n]                                              */
#define E4B_DT_F32_HL 2  /* an f32 vector pre-split as f16 hi[n] then f16 lo[n]   */
                         /* (e4b_split_f32): hi + lo is within                   */
                         /* max(2^-22 |x|, 2^-25) of x, |x| < 65520              */

/* ---------------------------------------------------------------------------
 * Library / device plumbing (replaces src/gpu.js:4-50 initDevice, upload,
 * alloc, readback).
 * ------------------------------------------------------------------------- */
const char* e4b_version(void);
const char* e4b_last_error(void);
int   e4b_device_count(int* n);
int   e4b_set_device(int device);
void* e4b_dev_alloc(size_t bytes);                           /* NULL on failure */
int   e4b_dev_free(void* p);
int   e4b_memcpy_h2d(void* dst_dev, const void* src_host, size_t bytes);
int   e4b_memcpy_d2h(void* dst_host, const void* src_dev, size_t bytes);
int   e4b_memset_dev(void* dst_dev, int value, size_t bytes);
int   e4b_memcpy_d2d(void* dst_dev, const void* src_dev, size_t bytes, void* stream);
int   e4b_sync(void);                                        /* device-wide */
int   e4b_stream_sync(void* stream);

/* HIP events for timing on a stream (replaces the timestamp-query profiling of
 * src/engine-a4b.js:707-740) */
void* e4b_event_create(void);
int   e4b_event_record(void* event, void* stream);
int   e4b_event_elapsed_ms(void* start, void* end, float* ms); /* waits for end */
int   e4b_event_destroy(void* event);

/* f32 -> (hi, lo) f16 split on the device: hi = f16(x), lo = f16(x - hi) (both
 * round to nearest even; x - hi is exact in f32).  |x - (hi + lo)| <=
 * max(2^-22 |x|, 2^-25): 22 of f32's 24 significant bits, and lo is an f16
 * subnormal (absolute step 2^-24) below |x| = 2^-3.  |x| must be < 65520. */
int   e4b_split_f32(const float* x, int64_t n, void* hl_out, void* stream);

/* ---------------------------------------------------------------------------
 * Seeded synthetic data (portable counter-based splitmix64; identical bytes
 * from any caller).  Distributions follow benchmark configs: q4_0 d =
 * f16(|N(0,sigma)|/8), nibbles U{0..15}; Q6_K d = f16(|N(0,sigma)|), scales
 * U{-32..31}, quants U{0..63}.
 * ------------------------------------------------------------------------- */
uint64_t e4b_synth_u64(uint64_t seed, uint64_t index);
int e4b_synth_normal_f32(uint64_t seed, int64_t n, float mean, float std, float* out);
int e4b_synth_uniform_u32(uint64_t seed, int64_t n, uint32_t lo, uint32_t hi_exclusive, uint32_t* out);
int e4b_synth_q40(uint64_t seed, int64_t rows, int64_t cols, float sigma, void* out_ggml);
int e4b_synth_q6k(uint64_t seed, int64_t rows, int64_t cols, float sigma, void* out_ggml);

/* ---------------------------------------------------------------------------
 * Weight formats.  Replaces repackQ40 / repackQ6K / q40cat
 * (src/engine-a4b.js:29-73, 126-138): raw ggml blocks in, the library's
 * device layout out.  Packing is a host-to-host transform; the caller uploads
 * the result (or uses e4b_*_upload which packs and copies in one call).
 * ------------------------------------------------------------------------- */
size_t e4b_q40_packed_bytes(int64_t rows, int64_t cols);
int    e4b_q40_pack(const void* ggml, int64_t rows, int64_t cols, void* packed_host);
size_t e4b_q6k_packed_bytes(int64_t rows, int64_t cols);
int    e4b_q6k_pack(const void* ggml, int64_t rows, int64_t cols, void* packed_host);

/* ---------------------------------------------------------------------------
 * Kernel-level entry points (parity + per-config benches).  All pointers are
 * device pointers; weights are in the packed layout above.
 * ------------------------------------------------------------------------- */

/* q4_0 GEMV y[rows] = W[rows x cols] . x  (kernels/q40mv.wgsl:56-89).
 * x_dtype E4B_DT_F32 (x is f32[cols]) or E4B_DT_F16 (x is f16[cols]).
 * cols % 32 == 0. */
int e4b_k_q40_gemv(const void* w_packed, int64_t rows, int64_t cols, const void* x,
                   int x_dtype, float* y, void* stream);

/* Fused gate/up q4_0 GEMV + GeGLU (kernels/q40gu.wgsl:62-119, dense role):
 * w_packed is [2*ff][cols] with gate rows [0,ff) then up rows [ff,2ff); x f16;
 * out f16[ff] = f16(gelu_tanh(gate) * up), tanh argument clamped to +-20. */
int e4b_k_q40_gemv_geglu(const void* w_packed, int64_t ff, int64_t cols, const void* x_f16,
                         void* out_f16, void* stream);

/* Batched q4_0 GEMM on the matrix cores, the prefill counterpart of the
 * GEMV (replaces the multi-column GEMVs of the reference's prefill,
 * kernels/q40mm.wgsl and kernels/q40sg.wgsl driven by
 * src/engine-a4b.js:465-585): x is f16[m][cols] row-major (m tokens),
 * y is f32[m][rows] row-major, y[t][r] = W[r] . x[t].  cols % 32 == 0. */
int e4b_k_q40_gemm(const void* w_packed, int64_t rows, int64_t cols, const void* x_f16, int m, float* y,
                   void* stream);

/* Batched gate/up + GeGLU: w_packed is [2*ff][cols] (gate rows then up
 * rows), x f16[m][cols], out f16[m][ff] = f16(gelu_tanh(gate) * up)
 * (kernels/q40gu.wgsl:62-119 per token). */
int e4b_k_q40_gemm_geglu(const void* w_packed, int64_t ff, int64_t cols, const void* x_f16, int m, void* out_f16,
                         void* stream);

/* The FFN input GEMV as the decode step runs it: a fused residual + RMSNorm
 * prologue, then gate/up + GeGLU (kernels/rmsacc3.wgsl:36-53 folded into
 * kernels/q40gu.wgsl:62-119):
 *   h = (h_in + rms(resid) * w_resid) * scale      (resid may be NULL: h = h_in * scale)
 *   x = f16(rms(h) * w_in);  out f16[ff] = f16(gelu_tanh(W_gate x) * (W_up x))
 * h_out (may be NULL) receives h.  cols (the hidden size) must be 256, 512,
 * 1024 or 2048; rms(v) = v * (mean(v^2) + eps)^-1/2. */
int e4b_k_q40_geglu_prenorm(const void* w_packed, int64_t ff, int64_t cols, const float* h_in,
                            const float* resid, const float* w_resid, const float* w_in, float scale,
                            float eps, float* h_out, void* out_f16, void* stream);

/* Q6_K GEMV + softcap + argmax (kernels/q6k.wgsl:75-130 MODE 1, then
 * kernels/argmax2.wgsl:8-48).  logits f32[rows] (may be NULL), amax u32[2] =
 * {index, f32 bits of the max}; ties -> lowest index; NaN never wins.
 * cols % 256 == 0.  softcap 0 disables the cap. */
int e4b_k_q6k_gemv_argmax(const void* w_packed, int64_t rows, int64_t cols, const float* x,
                          float softcap, float* logits, uint32_t* amax, void* stream);

/* e4b_k_q6k_gemv_argmax without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as e4b_k_q6k_gemv_argmax; its scratch
 * (f16 halves of x and the argmax partials) is a fixed 32 KiB device array
 * per GPU, held until the process ends, so cols must be <= 4096 (E4B_ERANGE
 * otherwise).  It calls no hipMalloc/hipFree.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (other streams, other threads)
 * race and must be ordered by the caller. */
int e4b_k_q6k_gemv_argmax_noalloc(const void* w_packed, int64_t rows, int64_t cols, const float* x,
                                  float softcap, float* logits, uint32_t* amax, void* stream);

/* Q6_K row dequant * mult (kernels/q6k.wgsl:37-73 MODE 0): out f32[cols]. */
int e4b_k_q6k_row(const void* w_packed, int64_t rows, int64_t cols, int64_t row, float mult,
                  float* out, void* stream);

/* argmax over f32[n] (kernels/argmax2.wgsl:8-48): amax u32[2]. */
int e4b_k_argmax(const float* x, int64_t n, uint32_t* amax, void* stream);

/* RoPE inverse frequencies out[p] = f32(theta^(-2p/head_dim)), p < angles
 * (host; the table headprep uses, kernels/headprep.wgsl:19-87). */
int e4b_rope_inv_freq(float theta, int head_dim, int angles, float* out_host);

/* One layer's decode attention for the token at `pos` (kernels/headprep.wgsl
 * :19-87, kernels/attsplit.wgsl:16-76 + kernels/attcomb.wgsl:10-36; one launch).
 *   qkv       f32[(q_heads + 2 kv_heads) * 256]: raw q heads, then k, then v
 *   q_norm, k_norm  f32[256] head-RMS weights (v gets a scale-less RMS)
 *   inv_freq  f32[rope_angles] (e4b_rope_inv_freq), NeoX pairs (p, p + 128)
 *   k_cache, v_cache  f16 [kv_heads][slots][256]; position p lives in slot
 *             p % slots when window > 0 (sliding ring, slots >= window), in
 *             slot p when window == 0 (global, pos < slots).  The new k/v is
 *             written to the slot of `pos`; live positions are
 *             (pos - window, pos] (sliding) or [0, pos] (global).
 *   chunk     positions per split-K chunk: 32 or 64 (0 = 64)
 *   out_f16   [q_heads][256] attention output, f16.
 * head_dim must be 256 and q_heads = 4 * kv_heads.  Uses the per-device
 * workspace: calls on one device must be ordered (one stream). */
int e4b_k_attn_decode(const float* qkv, const float* q_norm, const float* k_norm,
                      const float* inv_freq, int rope_angles, void* k_cache, void* v_cache,
                      int q_heads, int kv_heads, int head_dim, int slots, int window,
                      uint32_t pos, float eps, int chunk, void* out_f16, void* stream);

/* MoE FFN half-layer of an A4B-style decoder (src/engine-a4b.js:438-462):
 * all pointers are device pointers; the q4_0 matrices are in the packed
 * layout (e4b_q40_pack of the ggml rows).  Expert e's gate rows are
 * [2 ff e, 2 ff e + ff) and its up rows [2 ff e + ff, 2 ff (e+1)) of
 * exp_gate_up; its down rows are [hidden e, hidden (e+1)) of exp_down. */
typedef struct e4b_moe_weights {
  int32_t hidden;             /* 2816 (multiple of 256, <= 3072) */
  int32_t n_experts;          /* 128 (8..256) */
  int32_t expert_ffn;         /* 704 (multiple of 32, <= 768) */
  int32_t dense_ffn;          /* 2112 (multiple of 32, <= 3072) */
  float eps;                  /* 1e-6 */
  float layer_scale;          /* layer output scalar */
  const float* ffn_norm;      /* [hidden] dense-branch input norm */
  const float* router_scale;  /* [hidden] ffn_gate_inp.scale (raw; the kernel applies hidden^-1/2) */
  const float* pre_ffw2;      /* [hidden] expert-branch input norm */
  const float* router_w;      /* [n_experts][hidden] f32 */
  const float* pes;           /* [n_experts] per-expert output scale */
  const void* dense_gate_up;  /* q4_0 [2 dense_ffn][hidden]: gate rows then up rows */
  const void* exp_gate_up;    /* q4_0 [n_experts 2 expert_ffn][hidden] */
  const void* dense_down;     /* q4_0 [hidden][dense_ffn] */
  const void* exp_down;       /* q4_0 [n_experts hidden][expert_ffn] */
  const float* post_ffw1;     /* [hidden] dense-branch post norm */
  const float* post_ffw2;     /* [hidden] expert-branch post norm */
  const float* post_ffw;      /* [hidden] combined post norm */
} e4b_moe_weights;

/* Router + top-8 (kernels/routertop.wgsl:19-71): x = rms(h) * router_scale *
 * hidden^-1/2, scores = router_w . x, softmax, top-8 by a strict '>' scan
 * (ties -> lowest index), w_k = p_k / sum_top(p) * pes[idx_k].
 * topk_idx u32[8], topk_w f32[8] (device). */
int e4b_k_router_top8(const e4b_moe_weights* w, const float* h, uint32_t* topk_idx, float* topk_w,
                      void* stream);

/* The whole half-layer (rmsacc3 outputs -> routertop -> q40gu dense + 8 expert
 * slots -> dense down + q40moedown -> a4btail, kernels/rmsacc3.wgsl:36-53,
 * kernels/q40gu.wgsl:62-119, kernels/q40moedown.wgsl:42-75,
 * kernels/a4btail.wgsl:26-71):
 *   dense = W_down,d . f16(gelu(G x_d) * (U x_d)),  x_d = f16(rms(h) ffn_norm)
 *   moe   = sum_k w_k W_down,e_k . f16(gelu(G_e_k x_m) * (U_e_k x_m)),  x_m = f16(rms(h) pre_ffw2)
 *   comb  = rms(dense) post_ffw1 + rms(moe) post_ffw2
 *   h_out = (h + rms(comb) post_ffw) * layer_scale
 * Every output pointer except h_out may be NULL. */
int e4b_k_moe_layer(const e4b_moe_weights* w, const float* h, float* h_out, uint32_t* topk_idx,
                    float* topk_w, float* dense_out, float* moe_out, void* stream);

/* The half-layer over m prompt tokens (the reference's batched prefill of
 * the MoE layer, src/engine-a4b.js:478-549: routerTopB, expGroup +
 * guGsg32 / downGsg32 + waccB, kernels/expgroup.wgsl:15-50,
 * kernels/q40gugrp.wgsl:47-103): per token the e4b_k_moe_layer arithmetic;
 * the m*8 expert draws are sorted by expert and each expert's weight rows
 * are read once per tile of up to 32 draws (MFMA GEMMs).  h, h_out
 * f32[m][hidden]; topk_idx u32[m][8], topk_w f32[m][8], dense_out /
 * moe_out f32[m][hidden] may be NULL.  1 <= m <= 1024. */
int e4b_k_moe_prefill(const e4b_moe_weights* w, const float* h, int m, float* h_out, uint32_t* topk_idx,
                      float* topk_w, float* dense_out, float* moe_out, void* stream);

/* Causal attention of a prefill chunk (attnB / attnOSB of the reference's
 * batched prefill, src/engine-a4b.js:476-477; per query the arithmetic of
 * kernels/attnf32.wgsl:21-105 and kernels/attnos.wgsl:22-98, scale 1.0):
 *   q    f32[m][q_heads][256], prepped queries of positions p0 .. p0 + m - 1
 *   kc/vc f16[kv_heads][slots][256] caches already holding every key the
 *        queries attend to (position p in slot p % slots when window > 0)
 *   out  f16[m][q_heads * 256]
 * window > 0: keys (p - window, p] of a ring with slots >= window + m - 1;
 * window == 0: keys [0, p], p0 + m <= slots.  q_heads = 1, 2 or 4 x kv_heads. */
int e4b_k_attn_prefill(const float* q, const void* kc, const void* vc, void* out, int m, int q_heads, int kv_heads,
                       int slots, int window, uint32_t p0, void* stream);

/* ---------------------------------------------------------------------------
 * Engine: the per-token batch-1 decode step of an E4B-shaped decoder
 * (35 layers, 4 sliding : 1 global, GeGLU FFN, per-layer embeddings, q4_0
 * linears, Q6_K tied embedding / lm-head, f16 KV ring).  Replaces the engine
 * object of loadEngineA4B (src/engine-a4b.js:75, returned at :854-856): load
 * (openGGUF fetch + upload, src/gguf.js:74-81), step (:695-705), the GPU-fed
 * decodeChunk / generateFast loop (:786-848), argmaxFast (:781-784) and
 * readHidden (:850-852).  One context = one HIP stream; not reentrant.
 * ------------------------------------------------------------------------- */
typedef struct e4b_ctx e4b_ctx;

typedef struct e4b_config {
  int32_t hidden;         /* 2048 */
  int32_t layers;         /* 35 */
  int32_t q_heads;        /* 8 */
  int32_t kv_heads;       /* 2 (head_dim 256, 4 q heads per kv head) */
  int32_t head_dim;       /* 256 */
  int32_t ffn;            /* 16384 */
  int32_t ple_dim;        /* 256, or 0 = no per-layer embeddings */
  int32_t vocab;          /* 262144 */
  int32_t window;         /* sliding window, 512 */
  int32_t ring;           /* sliding-layer ring slots (>= window), 1024 */
  int32_t max_seq;        /* global-layer cache capacity (entries; see e4b_kv_count) */
  int32_t rope_angles;    /* rotated pairs per head, 128 */
  float theta_local;      /* 1e4 */
  float theta_global;     /* 1e6 */
  float eps;              /* 1e-6 */
  float softcap;          /* 30 (0 = none) */
  const uint8_t* layer_global; /* [layers] 1 = global; NULL = (i % 5 == 4) */
  int32_t attn_chunk;     /* E4B recipe: positions per split-K attention chunk of the full layers, 32 or
                           * 64 (0 = 64); the sliding layers use 32 unless attn_chunk is 64 */
  int32_t max_prompt;     /* prompt buffer capacity, 0 = max_seq */
  uint32_t flags;         /* E4B_FLAG_* */
  /* E4B_RECIPE_A4B (src/engine-a4b.js:100-116): the model loadEngineA4B
   * loads -- no per-layer embeddings, a MoE FFN half per layer, full layers
   * with their own head dim and rotated pairs and V = K.  Supported: hidden
   * a multiple of 256 up to 3072, head_dim 256, head_dim_full 256 or 512,
   * 1, 2, 4 or 8 q heads per KV head on every layer, ffn and expert_ffn
   * multiples of 32 (<= 3072, <= 768), 8..256 experts, ple_dim 0, and
   * max_seq <= 16384 (the full layers' merge holds 256 chunks of 64
   * positions).  e4b_prefill runs the
   * batched prefill of src/engine-a4b.js:465-584 (chunks of up to 512
   * tokens, ring - window + 1 at most). */
  int32_t recipe;              /* E4B_RECIPE_E4B (0) or E4B_RECIPE_A4B (1) */
  int32_t head_dim_full;       /* A4B: full layers' head dim (512), 0 = head_dim */
  int32_t rope_angles_full;    /* A4B: full layers' rotated pairs (64 = 0.25 * 512 / 2), 0 = rope_angles */
  int32_t n_experts;           /* A4B: 128 */
  int32_t expert_ffn;          /* A4B: 704 (ffn above is the dense branch, 2112) */
  const int32_t* layer_kv_heads; /* A4B: [layers] KV heads per layer; NULL = kv_heads */
} e4b_config;

/* the layer recipe of e4b_config.recipe */
#define E4B_RECIPE_E4B 0  /* dense GeGLU FFN + per-layer embeddings (benchmark config c4) */
#define E4B_RECIPE_A4B 1  /* MoE FFN half (benchmark config c3's layer), src/engine-a4b.js:424-463 */

/* launch the step's kernels directly each token instead of replaying the
 * captured hipGraph (same kernels; for profilers that do not follow graphs) */
#define E4B_FLAG_NO_GRAPH 1u
/* prefill token by token through the decode step (one graph replay per
 * prompt token) instead of the batched prefill */
#define E4B_FLAG_STEP_PREFILL 2u
/* full-layer KV budget (src/engine-a4b.js:587-657): every decode step adds
 * each live full-layer slot's normalised attention weight to a per-head
 * score (attnos SCORE = 1, kernels/attnos.wgsl:78-92), which e4b_kv_compact
 * ranks; costs one small kernel per full layer and token */
#define E4B_FLAG_KV_SCORE 4u
/* keep the residual stream after every layer of the last decode step for
 * e4b_read_layer_hidden (one extra store of the hidden state per layer) */
#define E4B_FLAG_LAYER_HIDDEN 16u
/* the flags e4b_create accepts; any other bit is an error (bit 8 named a
 * persistent layer loop that measured slower than the kernel chain and was
 * removed) */
#define E4B_FLAGS_KNOWN (E4B_FLAG_NO_GRAPH | E4B_FLAG_STEP_PREFILL | E4B_FLAG_KV_SCORE | E4B_FLAG_LAYER_HIDDEN)

/* tensor names follow the GGUF naming of the E4B family:
 *   token_embd.weight (Q6_K [vocab][hidden], tied lm-head), output_norm.weight,
 *   per_layer_token_embd.weight (Q6_K [vocab][layers*ple_dim]),
 *   per_layer_model_proj.weight (q4_0 [layers*ple_dim][hidden]),
 *   per_layer_proj_norm.weight, and per layer blk.N.{attn_norm, attn_q, attn_k,
 *   attn_v, attn_q_norm, attn_k_norm, attn_output, post_attention_norm,
 *   ffn_norm, ffn_gate, ffn_up, ffn_down, post_ffw_norm, inp_gate, proj,
 *   post_norm, layer_output_scale}.weight.  dims are ggml order (ne0 = row
 *   length).  Linear weights must be q4_0, norms f32. */
e4b_ctx* e4b_create(const e4b_config* cfg);   /* NULL on error (e4b_last_error) */
int  e4b_set_tensor(e4b_ctx* ctx, const char* name, int ggml_type, const int64_t* dims, int nd,
                    const void* bytes, size_t nbytes);
int  e4b_finalize(e4b_ctx* ctx);              /* allocates KV/activations, captures the step graph */
/* one token at `pos` (positions must be fed in order from 0); logits may be
 * NULL; argmax_out may be NULL */
int  e4b_step(e4b_ctx* ctx, uint32_t token, uint32_t pos, float* logits_or_null, uint32_t* argmax_out);
/* prefill of ids[0..n) from position 0 (prefill, src/engine-a4b.js:550-584):
 * chunks of up to 512 tokens (and at most ring - window + 1, rounded down
 * to a multiple of 128 above 128, so every key a
 * chunk's queries need keeps its ring slot), each layer as batched q4_0
 * GEMMs on the matrix cores plus per-token head prep, causal attention and
 * norms (E4B_RECIPE_A4B: the MoE half over the chunk's tokens with
 * expert-grouped GEMMs, src/engine-a4b.js:478-549); the lm-head runs once,
 * for the last token.  argmax_out = greedy
 * continuation of the last prompt token, which is also fed back as the next
 * e4b_decode input.  E4B_FLAG_STEP_PREFILL runs the prompt through the decode
 * step instead. */
int  e4b_prefill(e4b_ctx* ctx, const uint32_t* ids, uint32_t n, uint32_t* argmax_out);
/* the prompt token by token through the decode step (the prompt loop of
 * generateFast, src/engine-a4b.js:826-829: step(t, pos) per prompt token,
 * then argmaxFast), with no host round trip between tokens; the same state
 * and result as e4b_prefill under E4B_FLAG_STEP_PREFILL */
int  e4b_prefill_steps(e4b_ctx* ctx, const uint32_t* ids, uint32_t n, uint32_t* argmax_out);
/* GPU-fed greedy decode of `count` tokens starting at start_pos, fed with the
 * previous step's argmax; tokens_out[count] */
int  e4b_decode(e4b_ctx* ctx, uint32_t start_pos, uint32_t count, uint32_t* tokens_out);
int  e4b_argmax(e4b_ctx* ctx, uint32_t* token_out);     /* argmaxFast: last step's argmax */
int  e4b_read_hidden(e4b_ctx* ctx, float* out);         /* hidden state after the last layer */
/* The residual stream after `layer` in the last decode step (e4b_step, or
 * the last token of e4b_decode; readHidden, src/engine-a4b.js:850-852, per
 * layer: the per-layer state the resident harness's `stats` mode reports,
 * resident-a4b.html:96-101).  f32 [hidden]; the last layer's equals
 * e4b_read_hidden.  Needs E4B_FLAG_LAYER_HIDDEN for the layers before the
 * last (E4B_ESTATE otherwise); a batched prefill does not update it. */
int  e4b_read_layer_hidden(e4b_ctx* ctx, int layer, float* out);
/* A4B recipe: the top-8 experts (in slot order) and their router weights
 * (softmax over the layer's experts, renormalised over the 8, times the
 * per-expert scale; kernels/routertop.wgsl:19-71) that `layer` used in the
 * last decode step.  E4B_EINVAL on the E4B recipe. */
int  e4b_read_topk(e4b_ctx* ctx, int layer, uint32_t* idx, float* w);
int  e4b_read_logits(e4b_ctx* ctx, float* out);         /* last step's logits [vocab] */
int  e4b_read_kv(e4b_ctx* ctx, int layer, uint16_t* k_out, uint16_t* v_out); /* [kvh][slots][hd] f16 */
int  e4b_kv_slots(e4b_ctx* ctx, int layer);             /* slots of that layer's cache */
int  e4b_reset(e4b_ctx* ctx);                           /* zero KV caches and state */
void e4b_destroy(e4b_ctx* ctx);
/* timing: run `count` GPU-fed steps and return the elapsed device ms */
int  e4b_time_decode(e4b_ctx* ctx, uint32_t start_pos, uint32_t count, float* ms_out);

/* Per-dispatch GPU time of one step or one prefill chunk, summed per kernel
 * role (profileStep, src/engine-a4b.js:707-741, and profilePrefill,
 * :743-779: one timed pass per dispatch, for ranking).  The step's kernels
 * (or the first min(n, 512) prompt tokens' prefill chunk, without its
 * lm-head) are launched directly with a HIP event after each; an entry's time
 * is the span between the events around its launches.  Writes up to `cap`
 * entries in order of first launch and returns the number of roles, or a
 * negative error.  Both run a real step / chunk: e4b_profile_step is
 * e4b_step(token, pos); e4b_profile_prefill leaves the caches holding the
 * chunk's rows and the full layers' count at the chunk's length (decode
 * from a fresh e4b_prefill). */
typedef struct e4b_prof_entry {
  char name[40];  /* kernel role, e.g. "gate_up_geglu", "attn_sliding", "gemm_qkv" */
  float us;       /* summed microseconds */
  int32_t n;      /* dispatches */
} e4b_prof_entry;
int  e4b_profile_step(e4b_ctx* ctx, uint32_t token, uint32_t pos, e4b_prof_entry* out, int cap);
int  e4b_profile_prefill(e4b_ctx* ctx, const uint32_t* ids, uint32_t n, e4b_prof_entry* out, int cap);

/* Device-side timeline (the same per-dispatch ranking as profileStep,
 * src/engine-a4b.js:707-741, taken inside a captured hipGraph replay, which
 * event-based timing cannot see).  Only a library built with E4B_TRACE
 * (libe4b_trace.so, make target `trace`) records; the product library
 * returns E4B_EINVAL from e4b_trace_start.  While a trace runs, every
 * workgroup of every decode-step kernel writes one record: the chip's
 * real-time counter (e4b_trace_clock_khz ticks per ms) at its first
 * instruction and when its wave 0 exits, the kernel tag (family << 16 |
 * variant), its linear workgroup index, wave 0's HW_ID and XCC_ID
 * registers, and up to four phase marks inside the kernel (the GEMV: weight
 * loads issued, input vector ready, dot products done, rows reduced; the
 * attention: loads issued, head prep done, scores done, P.V done).  e4b_trace_start(cap) allocates room for cap records (cap / 8
 * per XCD) and clears the counts; e4b_trace_read copies up to `cap` records
 * (device-synchronising first; grouped by XCD, not in time order) and
 * returns the number recorded, which may exceed what fit (the excess is
 * dropped); e4b_trace_stop detaches and frees the buffer. */
typedef struct e4b_trace_rec {
  uint64_t t0, t1;
  uint32_t tag, blk;
  uint32_t hw_id, xcc;
  uint32_t mark[4];  /* wave 0's phase marks (ticks after t0; 0 = none) */
  uint32_t pad[4];
} e4b_trace_rec;
int  e4b_trace_start(size_t cap);
int  e4b_trace_read(e4b_trace_rec* out, size_t cap, size_t* recorded);
int  e4b_trace_stop(void);
int  e4b_trace_clock_khz(int* khz);

/* Full-layer KV budget.  Full (global) layers count their cache entries
 * apart from positions (kvCount, src/engine-a4b.js:217; CACHEMODE 2): the
 * token of a step goes to slot kvCount and attends to slots [0, kvCount];
 * e4b_step at position 0 and e4b_prefill restart the count, e4b_decode
 * continues it.  Until a compaction the count equals the position.
 *   e4b_kv_count: entries of the full layers (>= 0), or a negative error.
 *   e4b_read_scores: the accumulated mass of full layer `layer`, [q_heads]
 *     [max_seq] f32 (E4B_FLAG_KV_SCORE; zeroed by e4b_prefill, e4b_reset and
 *     compaction).
 *   e4b_kv_compact: compactAll (src/engine-a4b.js:587-617): per full layer,
 *     mass[t] = sum over heads of score[h][t]; keep the budget - protect
 *     older entries of largest mass (ties: lower slot first) and the
 *     min(protect, n) newest, in slot order; gather their K/V rows to slots
 *     0.. (kernels/kvgather.wgsl); zero the scores.  Returns the new count
 *     (min(n, budget) when protect <= budget), or a negative error; needs
 *     E4B_FLAG_KV_SCORE. */
int  e4b_kv_count(e4b_ctx* ctx);
int  e4b_read_scores(e4b_ctx* ctx, int layer, float* out);
int  e4b_kv_compact(e4b_ctx* ctx, int budget, int protect);
/* the selection e4b_kv_compact applies to one full layer (host only, no
 * device): score [q_heads][stride] over slots [0, n); writes the kept slots,
 * ascending, to keep_out[n] and returns their number, or a negative error */
int64_t e4b_kv_select(const float* score, int q_heads, int64_t stride, int64_t n, int budget, int protect,
                      uint32_t* keep_out);

/* GGUF loading on the C ABI (openGGUF, src/gguf.js:17-83, and the tensor
 * loop of loadEngineA4B, src/engine-a4b.js:121-214): the file is
 * memory-mapped; tokenizer.* metadata is skipped; the data start is aligned
 * to general.alignment (default 32).
 *   e4b_gguf_config: reads <arch>.embedding_length, block_count,
 *     attention.head_count(_kv), attention.key_length, feed_forward_length,
 *     embedding_length_per_layer_input, vocab_size, attention.sliding_window,
 *     rope.dimension_count_half, rope.freq_base(_swa),
 *     attention.layer_norm_rms_epsilon, final_logit_softcapping and
 *     attention.sliding_window_pattern (true = sliding) into cfg; fields the
 *     file lacks keep the caller's values (ring, max_seq, attn_chunk,
 *     max_prompt and flags are never in the file); a file without
 *     vocab_size takes the row count of token_embd.weight; the layer
 *     pattern is written to layer_global[cap] and cfg->layer_global points
 *     to it.  A file with <arch>.expert_count (the gemma4 26B-A4B MoE that
 *     loadEngineA4B loads, src/engine-a4b.js:100-116) selects
 *     E4B_RECIPE_A4B: head_dim = attention.key_length_swa, head_dim_full =
 *     attention.key_length, rope_angles = head_dim / 2, rope_angles_full =
 *     floor(0.25 * head_dim_full / 2), theta 1e4 / 1e6 whatever the file
 *     says (the recipe fixes them, src/engine-a4b.js:329), n_experts /
 *     expert_ffn from expert_count / expert_feed_forward_length
 *     (expert_used_count must be 8), ple_dim 0, ring >= window + 512, and
 *     the per-layer attention.head_count_kv array into layer_kv_heads[cap]
 *     (cfg->layer_kv_heads points to it).
 *   e4b_load_gguf: e4b_set_tensor for every tensor of the file (call
 *     e4b_finalize afterwards).
 *   e4b_open_gguf: config (from `base`, or ring 1024 / max_seq 4096 when
 *     NULL) + create + load + finalize in one call; NULL on error. */
int  e4b_gguf_config(const char* path, e4b_config* cfg, uint8_t* layer_global, int32_t* layer_kv_heads, int cap);
int  e4b_load_gguf(e4b_ctx* ctx, const char* path);
e4b_ctx* e4b_open_gguf(const char* path, const e4b_config* base);

#ifdef __cplusplus
}
#endif
#endif
