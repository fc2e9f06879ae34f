/*
 * oracle.h -- CPU restatement of the reference's batch-1 decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * e4b-webgpu_amd/) links, loads or calls this code.  Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py use it, and
 * only as the checker (or as the timed CPU baseline), never as the thing that
 * is measured or shipped.
 *
 * Every function restates one piece of the reference's WGSL/JS semantics and
 * cites the file:line it follows (paths relative to the reference checkout).
 * Arithmetic is carried in double and rounded to f32 / f16 exactly where the
 * reference stores an f32 / f16 value, so the oracle is the "truth" the GPU
 * path is compared against within a stated tolerance; integer outputs (argmax,
 * top-k indices, ring slots) are compared bit-exactly.
 *
 * Weight tensors are passed in raw ggml block layout (block_q4_0: 18 B / 32
 * weights; block_q6_K: 210 B / 256 weights), independent of any GPU repack.
 */
#ifndef E4B_ORACLE_H
#define E4B_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ---------------------------------------------------- */
float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f); /* round-to-nearest-even, IEEE binary16 */
void     orc_h2f_n(const uint16_t* h, int64_t n, float* out);
void     orc_f2h_n(const float* f, int64_t n, uint16_t* out);

/* ---- q4_0 -------------------------------------------------------------- */
void orc_q40_dequant(const uint8_t* blocks, int64_t nblocks, float* out);
void orc_q40_gemv(const uint8_t* w, int64_t rows, int64_t cols, const float* x, float* y);
/* expert-indexed GEMV: rows of expert e start at w + e*rows*cols/32*18 */
void orc_q40_gemv_expert(const uint8_t* w, int expert, int64_t rows, int64_t cols,
                         const float* x, float* y);

/* ---- Q6_K -------------------------------------------------------------- */
void orc_q6k_dequant(const uint8_t* blocks, int64_t nblocks, float mult, float* out);
void orc_q6k_dequant_row(const uint8_t* w, int64_t cols, int64_t row, float mult, float* out);
void orc_q6k_gemv(const uint8_t* w, int64_t rows, int64_t cols, const float* x,
                  float softcap, float* y);
void orc_argmax(const float* x, int64_t n, uint32_t out[2]);

/* ---- elementwise / norms ----------------------------------------------- */
void  orc_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y);
float orc_gelu_tanh(float g);

/* ---- router ------------------------------------------------------------ */
void orc_router_topk(const float* x, const float* W, const float* pes, int H, int E, int K,
                     uint32_t* idx, float* wts, float* scores);

/* ---- RoPE / head prep -------------------------------------------------- */
void orc_rope_inv_freq(float theta, int head_dim, int angles, float* inv);
void orc_headprep(const float* qkv, int qh, int kvh, int hd, int angles, const float* inv_freq,
                  const float* qw, const float* kw, float eps, uint32_t pos,
                  float* q_out, uint16_t* k_out, uint16_t* v_out);

/* ---- attention (cache layout [slot][kvh][hd] f16) ----------------------- */
void orc_attn_ring(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                   int hd, int ring, int window, uint32_t pos, uint16_t* out);
void orc_attn_linear(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                     int hd, uint32_t len, uint16_t* out);
void orc_attn_split(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                    int hd, uint32_t len, int window, int chunks, int cs,
                    float* part_o, float* part_me);
void orc_attn_combine(const float* part_o, const float* part_me, int qh, int hd, int n_chunks,
                      int chunks, uint16_t* out);

/* ---- KV ring protocol (specs/KVRing.tla) -------------------------------- */
int64_t orc_kvring_recover(int64_t t, int64_t mw, int64_t ring);
int     orc_kvring_check(int W, int C, int RING, int NCHUNKS, int GEN);

/* ---- MoE FFN half-layer (A4B style) ------------------------------------ */
typedef struct {
  int hidden, n_experts, top_k, expert_ffn, dense_ffn;
  float eps, layer_scale;
  const float* ffn_norm;      /* [H]  dense-branch input norm            */
  const float* router_scale;  /* [H]  ffn_gate_inp.scale (raw, unscaled)  */
  const float* pre_ffw2;      /* [H]  expert-branch input norm           */
  const float* router_w;      /* [E][H] f32                               */
  const float* pes;           /* [E]  per-expert output scale            */
  const uint8_t* dense_gate;  /* q4_0 [FF2][H] */
  const uint8_t* dense_up;    /* q4_0 [FF2][H] */
  const uint8_t* dense_down;  /* q4_0 [H][FF2] */
  const uint8_t* exp_gate_up; /* q4_0 [E][2*FF][H] (gate rows then up rows) */
  const uint8_t* exp_down;    /* q4_0 [E][H][FF] */
  const float* post_ffw1;     /* [H] */
  const float* post_ffw2;     /* [H] */
  const float* post_ffw;      /* [H] */
} orc_moe;
void orc_moe_ffn(const orc_moe* m, const float* h, uint32_t* topk_idx, float* topk_w,
                 float* dense_out, float* moe_out, float* h_out);
/* the same, also returning the selection's decision margin (K-th minus
 * (K+1)-th largest router score, over max |score|) when margin != NULL */
void orc_moe_ffn_m(const orc_moe* m, const float* h, uint32_t* topk_idx, float* topk_w,
                   float* dense_out, float* moe_out, float* h_out, double* margin);
void orc_moe_ffn_f(const orc_moe* m, const float* h, const uint32_t* force_idx, uint32_t* own_idx,
                   uint32_t* topk_idx, float* topk_w, float* dense_out, float* moe_out, float* h_out,
                   double* margin);

/* ---- full E4B-shaped decode step --------------------------------------- */
typedef struct {
  const float* attn_norm;
  const float* q_norm;
  const float* k_norm;
  const float* post_attn_norm;
  const float* ffn_norm;
  const float* post_ffw_norm;
  const float* post_norm;     /* post per-layer-input norm (PLE) */
  float layer_scale;
  const uint8_t *wq, *wk, *wv, *wo;          /* q4_0 */
  const uint8_t *wgate, *wup, *wdown;        /* q4_0 */
  const uint8_t *inp_gate, *proj;            /* q4_0 PLE gate [PD][H], proj [H][PD] */
  orc_moe moe;  /* A4B recipe: the layer's MoE FFN half (wgate/wup/wdown are the dense branch) */
} orc_layer;

typedef struct {
  int hidden, layers, q_heads, kv_heads, head_dim, ffn, ple_dim, vocab;
  int window, ring, max_seq, rope_angles;
  float theta_local, theta_global, eps, softcap;
  const uint8_t* layer_global; /* [layers] 1 = global (linear cache) */
  const uint8_t* tok_embd;     /* Q6_K [vocab][hidden], tied lm-head */
  const float* out_norm;       /* [hidden] */
  const uint8_t* ple_tab;      /* Q6_K [vocab][layers*ple_dim] */
  const uint8_t* ple_proj;     /* q4_0 [layers*ple_dim][hidden] */
  const float* ple_proj_norm;  /* [ple_dim] */
  const orc_layer* L;          /* [layers] */
  /* recipe 1 = the A4B engine's layer (src/engine-a4b.js:424-463): no PLE, */
  /* MoE FFN half (orc_moe_ffn); full layers use head_dim_full, rotate     */
  /* rope_angles_full pairs and take V from the raw K projection (KEQV);   */
  /* layer_kv_heads (may be NULL) gives each layer's KV heads               */
  int recipe, head_dim_full, rope_angles_full;
  const int* layer_kv_heads;
} orc_model;

typedef struct orc_state orc_state;
orc_state* orc_state_new(const orc_model* m);
void       orc_state_free(orc_state* s);
/* one decode step; logits may be NULL; returns the argmax token */
uint32_t   orc_step(const orc_model* m, orc_state* s, uint32_t token, uint32_t pos,
                    float* logits, float* hidden_out);
/* ring slot index the step at `pos` writes for layer type (0 sliding, 1 global) */
int64_t    orc_kv_slot(const orc_model* m, int is_global, uint32_t pos);
const uint16_t* orc_state_kcache(const orc_state* s, int layer);
void       orc_state_set_kv(const orc_model* m, orc_state* s, int layer, const uint16_t* k, const uint16_t* v);
const uint16_t* orc_state_vcache(const orc_state* s, int layer);
/* full-layer KV budget (src/engine-a4b.js:587-617) */
void       orc_state_set_scoring(orc_state* s, int on);
/* keep_rows: the step attends to the cache row handed over for the current */
/* token instead of writing its own; its own rows are kept apart           */
void       orc_state_set_keep_rows(orc_state* s, int on);
const uint16_t* orc_state_krow(const orc_state* s, int layer);  /* [layer's kv_heads][head_dim] */
const uint16_t* orc_state_vrow(const orc_state* s, int layer);
int64_t    orc_state_kv_count(const orc_state* s);
/* A4B recipe: the smallest top-8 decision margin over the last step's layers */
double     orc_state_route_margin(const orc_state* s);
/* per layer of the last step: the residual stream after the layer; A4B: the */
/* oracle's own top-8 and decision margin; force_topk(idx) makes the layer's */
/* expert slots use idx[8] (NULL: the oracle's own picks again)             */
const float*    orc_state_layer_hidden(const orc_state* s, int layer);
const uint32_t* orc_state_layer_topk(const orc_state* s, int layer);
double          orc_state_layer_margin(const orc_state* s, int layer);
void            orc_state_force_topk(orc_state* s, int layer, const uint32_t* idx);
const float* orc_state_score(const orc_state* s, int layer);
int64_t    orc_kv_keep(const float* score, int qh, int64_t scap, int64_t n, int budget, int protect,
                       uint32_t* keep);
int64_t    orc_kv_compact(const orc_model* m, orc_state* s, int budget, int protect);
void       orc_kv_gather_layer(const orc_model* m, orc_state* s, int layer, const uint32_t* keep, int64_t cnt);
void       orc_state_set_kv_count(orc_state* s, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
