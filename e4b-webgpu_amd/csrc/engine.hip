// engine.hip -- the batch-1 decode engine behind the e4b_* context ABI.
//
// Host orchestration of one token (the A4B engine's encodeForward /
// encodeLayer order, src/engine-a4b.js:424-463, 683-693, with the E4B per-layer
// embedding dataflow of src/engine.js:282-323), captured once into a hipGraph
// and replayed per token.  Every kernel reads the position / token from the
// device-side params block, and the last kernel feeds the argmax back as the
// next input token, so GPU-fed decode needs no host work between tokens.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <algorithm>
#include <vector>

#include "../../include/e4b.h"
#include "a4b.h"

// decode attention split of the E4B recipe (compile-time, for A/B builds):
// sliding layers' chunk and V slices, full layers' V slices
#ifndef E4B_TUNE_CHUNK_SW
#define E4B_TUNE_CHUNK_SW 32
#endif
#ifndef E4B_TUNE_VS_SW
#define E4B_TUNE_VS_SW 4
#endif
#ifndef E4B_TUNE_VS_GL
#define E4B_TUNE_VS_GL 4
#endif
// column slices of the o projection with the attention-combine prologue (1
// or 2; the consumer's prologue adds the slices)
#ifndef E4B_TUNE_OKS
#define E4B_TUNE_OKS 2
#endif
#include "kernels.h"
#include "moe.h"
#include "step.h"
#include "util.h"

namespace {

// per-layer tensors: the E4B recipe's, then the A4B recipe's MoE half
// (src/engine-a4b.js:150-199)
enum LayerPart {
  P_ATTN_NORM, P_Q, P_K, P_V, P_Q_NORM, P_K_NORM, P_O, P_POST_ATTN, P_FFN_NORM, P_GATE, P_UP, P_DOWN,
  P_POST_FFW, P_INP_GATE, P_PROJ, P_POST_NORM, P_SCALE,
  P_PRE_FFW2, P_POST_FFW1, P_POST_FFW2, P_ROUTER_W, P_ROUTER_SCALE, P_PES, P_EXP_GU, P_EXP_DOWN, P_COUNT
};
const char* kPartNames[P_COUNT] = {
    "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q_norm.weight",
    "attn_k_norm.weight", "attn_output.weight", "post_attention_norm.weight", "ffn_norm.weight", "ffn_gate.weight",
    "ffn_up.weight", "ffn_down.weight", "post_ffw_norm.weight", "inp_gate.weight", "proj.weight",
    "post_norm.weight", "layer_output_scale.weight", "pre_ffw_norm_2.weight", "post_ffw_norm_1.weight",
    "post_ffw_norm_2.weight", "ffn_gate_inp.weight", "ffn_gate_inp.scale", "ffn_down_exps.scale",
    "ffn_gate_up_exps.weight", "ffn_down_exps.weight"};
constexpr uint32_t bit(int p) { return 1u << p; }
// the parts each recipe needs (attn_v only on layers with their own V)
constexpr uint32_t kNeedE4B = (bit(P_SCALE) - 1u) & ~(bit(P_INP_GATE) | bit(P_PROJ) | bit(P_POST_NORM));
constexpr uint32_t kPleParts = bit(P_INP_GATE) | bit(P_PROJ) | bit(P_POST_NORM);
constexpr uint32_t kNeedA4B = ((bit(P_POST_FFW) << 1) - 1u) | bit(P_PRE_FFW2) | bit(P_POST_FFW1) | bit(P_POST_FFW2) |
                              bit(P_ROUTER_W) | bit(P_ROUTER_SCALE) | bit(P_PES) | bit(P_EXP_GU) | bit(P_EXP_DOWN);

struct Layer {
  bool global = false;
  uint8_t* qkv = nullptr;  // packed q4_0 [(QH + 2 KVH) HD][H]: q rows, k rows, v rows
  uint8_t* o = nullptr;    // [H][QH HD]
  uint8_t* gu = nullptr;   // [2 FF][H]: gate rows, then up rows
  uint8_t* down = nullptr; // [H][FF]
  uint8_t* pg = nullptr;   // PLE gate [PD][H]
  uint8_t* pp = nullptr;   // PLE proj [H][PD], block-transposed (decode PLE branch)
  uint8_t* pp_rm = nullptr; // the same matrix row-major (prefill GEMM)
  float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *post_attn = nullptr, *ffn_norm = nullptr,
        *post_ffw = nullptr, *post_norm = nullptr;
  float scale = 1.0f;
  uint16_t *kc = nullptr, *vc = nullptr;
  int slots = 0;
  uint32_t have = 0;
  float* score = nullptr;  // full layers with E4B_FLAG_KV_SCORE: [QH][slots] attention mass
  // attention shape of the layer: KV heads, head dim, rotated pairs, V = K
  // (the A4B recipe's full layers), rows of the q|k(|v) matrix, split-K
  // chunks its partials hold
  int kvh = 0, hd = 0, angles = 0, gch = 0;
  bool keqv = false;
  int64_t qkv_rows = 0;
  // A4B recipe: the MoE half (gu / down above hold the dense branch)
  float *pre_ffw2 = nullptr, *post_ffw1 = nullptr, *post_ffw2 = nullptr, *router_w = nullptr,
        *router_scale = nullptr, *pes = nullptr;
  uint8_t *exp_gu = nullptr, *exp_down = nullptr;  // q4_0 [E 2 FE][H], [E H][FE]
};

}  // namespace

struct e4b_ctx {
  e4b_config cfg;
  std::vector<uint8_t> lglobal;
  hipStream_t st = nullptr;
  std::vector<void*> allocs;
  // weights
  uint8_t* embd = nullptr;      // packed Q6_K [V][H] (embedding + tied lm-head)
  float* out_norm = nullptr;
  uint8_t* ple_tab = nullptr;   // ggml Q6_K blocks [V][L PD]
  uint8_t* ple_proj = nullptr;  // packed q4_0 [L PD][H]
  float* ple_norm = nullptr;    // [PD]
  std::vector<Layer> L;
  float* inv_local = nullptr;
  float* inv_global = nullptr;
  // state / activations
  uint32_t *params = nullptr, *prompt = nullptr, *tok_ring = nullptr, *amax = nullptr, *status = nullptr;
  float *h = nullptr, *hb = nullptr, *h_final = nullptr, *proj = nullptr, *ple = nullptr, *qkv = nullptr,
        *part_o = nullptr, *part_ml = nullptr;
  float2* rope = nullptr;        // [2][head_dim/2] (cos, sin) at the current position: local, global
  float *o = nullptr, *dn = nullptr, *pp = nullptr, *logits = nullptr;
  uint16_t *h_hl = nullptr, *xn = nullptr, *attn = nullptr, *xf = nullptr, *gg = nullptr, *xg = nullptr,
           *gp = nullptr, *xo_hl = nullptr;
  uint2* amax_part = nullptr;
  // full-layer entry count (host mirror of params[4]) and the scoring /
  // compaction buffers (E4B_FLAG_KV_SCORE)
  uint32_t kv_count = 0;
  float* raw = nullptr;                     // [QH][max_seq] raw scores of the current layer
  uint32_t* keep = nullptr;                 // [max_seq] compaction keep list
  uint16_t *kv_sk = nullptr, *kv_sv = nullptr;  // [KVH][max_seq][HD] gather scratch
  int nch = 0, chunk = 64, ring_cap = 0, max_prompt = 0, amax_parts = 0;
  // E4B recipe decode attention: split-K chunk and V slices of the sliding
  // and of the full layers (chunk = the full layers' chunk)
  int chunk_sw = 32, vs_sw = E4B_TUNE_VS_SW, vs_gl = E4B_TUNE_VS_GL;
  // E4B_FLAG_LAYER_HIDDEN: the residual stream after each layer of the last
  // decode step ([layers][hidden]; the last layer's is h_final)
  float* lh = nullptr;
  int64_t qkv_rows = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool finalized = false;
  // batched prefill: chunks of up to pf_cap tokens
  int pf_cap = 0;
  uint32_t* pf_ids = nullptr;  // [cap]
  float *pf_h = nullptr, *pf_proj = nullptr, *pf_ple = nullptr, *pf_qkv = nullptr, *pf_q = nullptr,
        *pf_y = nullptr;       // [cap][H], [2][cap][L PD], [cap][L PD], [cap][QKV], [cap][QH HD], [kPfKs][cap][H]
  uint16_t *pf_xhl = nullptr, *pf_xn = nullptr, *pf_attn = nullptr, *pf_gg = nullptr,
           *pf_gp = nullptr;   // [2][cap][H], [cap][H], [cap][QH HD], [cap][FF], [cap][PD]
  float* pf_apart = nullptr;   // split-key attention partials (attn_prefill_part_bytes)
  size_t pf_apart_bytes = 0;
  // per-dispatch profiling (e4b_profile_step / e4b_profile_prefill): while
  // prof_on, every launch of a directly launched step or prefill chunk is
  // followed by an event on the context stream, labelled by the kernel role
  // A4B recipe: the MoE half's scratch; the batched prefill's MoE scratch
  MoeArgs moe{};
  MoePrefillBufs pf_mb{};
  uint8_t* pf_moe = nullptr;
  bool prof_on = false;
  std::vector<hipEvent_t> prof_ev;       // event pool, grown on first use
  std::vector<const char*> prof_label;   // label of the dispatch ending at event i (i >= 1)
};

namespace {

int dalloc(e4b_ctx* c, void** p, size_t bytes) {
  hipError_t e = hipMalloc(p, bytes ? bytes : 16);
  if (e != hipSuccess) return e4b_fail(E4B_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  c->allocs.push_back(*p);
  return E4B_OK;
}
template <typename T>
int dalloc_t(e4b_ctx* c, T** p, size_t count) {
  return dalloc(c, reinterpret_cast<void**>(p), count * sizeof(T));
}

// profiling mark after a launch (no-op unless a profile call is running;
// never active during graph capture)
int tick(e4b_ctx* c, const char* label) {
  if (!c->prof_on) return E4B_OK;
  const size_t i = c->prof_label.size();
  if (i >= c->prof_ev.size()) {
    hipEvent_t e;
    E4B_HIP(hipEventCreate(&e));
    c->prof_ev.push_back(e);
  }
  E4B_HIP(hipEventRecord(c->prof_ev[i], c->st));
  c->prof_label.push_back(label);
  return E4B_OK;
}

// pack `rows` q4_0 rows and place them at row offset `row_off` of a packed
// matrix with `total_rows` rows (row-concatenation of same-width linears, the
// q40cat of src/engine-a4b.js:126-138)
int upload_q40_rows(uint8_t* dst, int64_t total_rows, int64_t cols, int64_t row_off, const void* ggml,
                    int64_t rows) {
  std::vector<uint8_t> tmp(e4b_q40_packed_bytes(rows, cols));
  int rc = e4b_q40_pack(ggml, rows, cols, tmp.data());
  if (rc) return rc;
  const size_t nb = (size_t)(cols / 32);
  const size_t nib_bytes = (size_t)rows * nb * 16, sc_bytes = (size_t)rows * nb * 2;
  const size_t dst_sc = E4B_ALIGN256((size_t)total_rows * nb * 16);
  E4B_HIP(hipMemcpy(dst + (size_t)row_off * nb * 16, tmp.data(), nib_bytes, hipMemcpyHostToDevice));
  E4B_HIP(hipMemcpy(dst + dst_sc + (size_t)row_off * nb * 2, tmp.data() + E4B_ALIGN256(nib_bytes), sc_bytes,
                    hipMemcpyHostToDevice));
  return E4B_OK;
}

// q4_0 matrix stored block-transposed: block j of row r at index j * rows + r
// in both planes, so a kernel that walks one block column over all rows
// streams contiguous memory (the fused PLE branch's projection)
int upload_q40_block_t(uint8_t* dst, int64_t rows, int64_t cols, const void* ggml) {
  std::vector<uint8_t> tmp(e4b_q40_packed_bytes(rows, cols)), out(tmp.size());
  int rc = e4b_q40_pack(ggml, rows, cols, tmp.data());
  if (rc) return rc;
  const int64_t nb = cols / 32;
  const size_t sc_off = E4B_ALIGN256((size_t)rows * nb * 16);
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < nb; ++j) {
      memcpy(&out[(size_t)(j * rows + r) * 16], &tmp[(size_t)(r * nb + j) * 16], 16);
      memcpy(&out[sc_off + (size_t)(j * rows + r) * 2], &tmp[sc_off + (size_t)(r * nb + j) * 2], 2);
    }
  E4B_HIP(hipMemcpy(dst, out.data(), out.size(), hipMemcpyHostToDevice));
  return E4B_OK;
}

int upload_f32(e4b_ctx* c, float** dst, const void* bytes, int64_t n) {
  if (!*dst) {
    int rc = dalloc_t(c, dst, (size_t)n);
    if (rc) return rc;
  }
  E4B_HIP(hipMemcpy(*dst, bytes, (size_t)n * 4, hipMemcpyHostToDevice));
  return E4B_OK;
}

int64_t nelems(const int64_t* dims, int nd) {
  int64_t n = 1;
  for (int i = 0; i < nd; ++i) n *= dims[i];
  return n;
}

int expect(const char* name, int type, int want_type, const int64_t* dims, int nd, int64_t cols, int64_t rows,
           int64_t mats = 1) {
  if (type != want_type) return e4b_fail(E4B_EINVAL, "%s: ggml type %d, expected %d", name, type, want_type);
  const int64_t d0 = nd > 0 ? dims[0] : 1, d1 = nd > 1 ? dims[1] : 1, d2 = nd > 2 ? dims[2] : 1;
  if (d0 != cols || d1 != rows || d2 != mats || nd > 3)
    return e4b_fail(E4B_EINVAL, "%s: dims [%lld, %lld, %lld], expected [%lld, %lld, %lld]", name, (long long)d0,
                    (long long)d1, (long long)d2, (long long)cols, (long long)rows, (long long)mats);
  return E4B_OK;
}

int record_step(e4b_ctx* c);

// batched prefill: tokens per chunk at most, and split-K slices of the
// o and down projection GEMMs (their consumers sum the slices)
constexpr int kPfMaxChunk = 512;
constexpr int kPfKsO = 4;    // o projection
constexpr int kPfKs = 8;     // down projection (the most slices; sizes the partial buffer)
constexpr int kPfKsQkv = 2;  // qkv (the head prep sums the slices)
constexpr int kPfKsPle = 8;  // PLE gate (256 rows; the GELU-multiply kernel sums the slices)
constexpr int kPfA4bOKs = 4;
constexpr int kPfA4bQkvKs = 2;  // A4B q|k|v projection (the head prep sums the slices)  // A4B o projection (the attention-residual row norm sums the slices)

}  // namespace

// ---------------------------------------------------------------------------
// The A4B recipe's shape limits: the MoE kernels (hidden a multiple of 256
// up to 3072, experts 8..256, expert FFN up to 768, dense FFN up to 3072),
// the general head prep / attention (head dims 256 and 512, any KV heads
// dividing the q heads)
// A4B prefill layers whose attention runs on the matrix cores (the prefill
// kernel: head dim 256 with 1, 2 or 4 q heads per KV head, or 512 with 8)
static bool a4b_pf_mfma_attn(const Layer& ly, int qh) {
  const int gqa = ly.kvh > 0 && qh % ly.kvh == 0 ? qh / ly.kvh : 0;
  return (ly.hd == 256 && (gqa == 1 || gqa == 2 || gqa == 4)) || (ly.hd == 512 && gqa == 8);
}

static bool a4b_config_ok(const e4b_config& k, char* why, size_t n) {
  auto bad = [&](const char* m) {
    snprintf(why, n, "%s", m);
    return false;
  };
  if (k.hidden <= 0 || k.hidden % 256 || k.hidden > 3072) return bad("hidden must be a multiple of 256 up to 3072");
  if (k.head_dim != 256) return bad("head_dim (sliding layers) must be 256");
  const int hdf = k.head_dim_full ? k.head_dim_full : k.head_dim;
  if (hdf != 256 && hdf != 512) return bad("head_dim_full must be 256 or 512");
  if (k.q_heads <= 0) return bad("q_heads must be positive");
  for (int l = 0; l < k.layers; ++l) {
    const int kvh = k.layer_kv_heads ? k.layer_kv_heads[l] : k.kv_heads;
    if (kvh <= 0 || k.q_heads % kvh) return bad("every layer's KV heads must divide q_heads");
    const int gqa = k.q_heads / kvh;
    if (gqa != 1 && gqa != 2 && gqa != 4 && gqa != 8) return bad("q heads per KV head must be 1, 2, 4 or 8");
  }
  if (k.ple_dim != 0) return bad("ple_dim must be 0 (no per-layer embeddings)");
  if (k.max_seq > kAttnGenMaxChunks * kAttnGenChunk)
    return bad("max_seq beyond 16384: the full layers' attention merge holds 256 chunks of 64 positions");
  if (k.ffn <= 0 || k.ffn % 32 || k.ffn > 3072) return bad("ffn (the dense branch) must be a multiple of 32 up to 3072");
  if (k.n_experts < 8 || k.n_experts > 256) return bad("n_experts must be 8..256");
  if (k.expert_ffn <= 0 || k.expert_ffn % 32 || k.expert_ffn > 768)
    return bad("expert_ffn must be a multiple of 32 up to 768");
  const int af = k.rope_angles_full ? k.rope_angles_full : k.rope_angles;
  if (k.rope_angles < 0 || k.rope_angles > k.head_dim / 2 || af < 0 || af > hdf / 2)
    return bad("rotated pairs beyond half the head dim");
  return true;
}

extern "C" e4b_ctx* e4b_create(const e4b_config* cfg) {
  if (!cfg) {
    e4b_fail(E4B_EINVAL, "e4b_create: null config");
    return nullptr;
  }
  const e4b_config& k = *cfg;
  if (k.recipe != E4B_RECIPE_E4B && k.recipe != E4B_RECIPE_A4B) {
    e4b_fail(E4B_EINVAL, "e4b_create: unknown recipe %d", k.recipe);
    return nullptr;
  }
  if (k.flags & ~E4B_FLAGS_KNOWN) {
    e4b_fail(E4B_EINVAL, "e4b_create: unknown flags 0x%x", k.flags & ~E4B_FLAGS_KNOWN);
    return nullptr;
  }
  if (k.layers <= 0 || k.vocab <= 0 || k.window <= 0 || k.ring < k.window || k.max_seq <= 0 || k.max_prompt < 0 ||
      (k.attn_chunk != 0 && k.attn_chunk != 32 && k.attn_chunk != 64)) {
    e4b_fail(E4B_EINVAL, "e4b_create: unsupported config (layers, vocab, window <= ring, max_seq, attn_chunk 32/64)");
    return nullptr;
  }
  if (k.recipe == E4B_RECIPE_A4B) {
    char why[160];
    if (!a4b_config_ok(k, why, sizeof(why))) {
      e4b_fail(E4B_EINVAL, "e4b_create: unsupported A4B config: %s", why);
      return nullptr;
    }
  } else if (!q40_prologue_supported(k.hidden) || k.head_dim != 256 || k.kv_heads <= 0 ||
             k.q_heads != 4 * k.kv_heads || k.ffn <= 0 || k.ffn % 32 || (k.ple_dim != 0 && k.ple_dim != 256) ||
             k.rope_angles < 0 || k.rope_angles > k.head_dim / 2) {
    e4b_fail(E4B_EINVAL,
             "e4b_create: unsupported config (hidden %d not 256, 512, 1024 or 2048, or: head_dim 256, q_heads = 4 * "
             "kv_heads, ple_dim 0 or 256, ring >= window)",
             k.hidden);
    return nullptr;
  }
  e4b_ctx* c = new e4b_ctx();
  c->cfg = k;
  c->lglobal.resize(k.layers);
  for (int i = 0; i < k.layers; ++i) c->lglobal[i] = k.layer_global ? (k.layer_global[i] != 0) : (i % 5 == 4);
  c->cfg.layer_global = nullptr;
  c->cfg.layer_kv_heads = nullptr;
  c->L.resize(k.layers);
  const bool a4b = k.recipe == E4B_RECIPE_A4B;
  for (int i = 0; i < k.layers; ++i) {
    Layer& ly = c->L[i];
    ly.global = c->lglobal[i] != 0;
    ly.kvh = (a4b && k.layer_kv_heads) ? k.layer_kv_heads[i] : k.kv_heads;
    const bool full = a4b && ly.global;
    ly.hd = (full && k.head_dim_full) ? k.head_dim_full : k.head_dim;
    ly.angles = (full && k.rope_angles_full) ? k.rope_angles_full : k.rope_angles;
    ly.keqv = full;  // src/engine-a4b.js:155 (full layers: V = K projection)
    ly.qkv_rows = (int64_t)(k.q_heads + (ly.keqv ? 1 : 2) * ly.kvh) * ly.hd;
    if (ly.qkv_rows > c->qkv_rows) c->qkv_rows = ly.qkv_rows;
  }
  hipError_t e = hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking);
  if (e != hipSuccess) {
    e4b_fail(E4B_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
    delete c;
    return nullptr;
  }
  return c;
}

extern "C" int e4b_set_tensor(e4b_ctx* c, const char* name, int type, const int64_t* dims, int nd,
                              const void* bytes, size_t nbytes) {
  if (!c || !name || !bytes || (nd > 0 && !dims)) return e4b_fail(E4B_EINVAL, "e4b_set_tensor: null argument");
  if (c->finalized) return e4b_fail(E4B_ESTATE, "e4b_set_tensor(%s) after e4b_finalize", name);
  const e4b_config& k = c->cfg;
  const int64_t H = k.hidden, V = k.vocab, PD = k.ple_dim, LPD = (int64_t)k.layers * k.ple_dim;
  const int64_t n = nelems(dims, nd);
  int rc;
  auto check_bytes = [&](size_t want) -> int {
    if (nbytes != want)
      return e4b_fail(E4B_EINVAL, "%s: %zu bytes, expected %zu", name, nbytes, want);
    return E4B_OK;
  };
  const std::string nm(name);
  if (nm == "token_embd.weight") {
    if ((rc = expect(name, type, E4B_GGML_Q6_K, dims, nd, H, V)) || (rc = check_bytes((size_t)(V * H / 256) * 210)))
      return rc;
    const size_t pb = e4b_q6k_packed_bytes(V, H);
    if (!c->embd && (rc = dalloc(c, (void**)&c->embd, pb))) return rc;
    std::vector<uint8_t> tmp(pb);
    if ((rc = e4b_q6k_pack(bytes, V, H, tmp.data()))) return rc;
    E4B_HIP(hipMemcpy(c->embd, tmp.data(), pb, hipMemcpyHostToDevice));
    return E4B_OK;
  }
  if (nm == "output_norm.weight") {
    if ((rc = expect(name, type, E4B_GGML_F32, dims, nd, H, 1)) || (rc = check_bytes((size_t)H * 4))) return rc;
    return upload_f32(c, &c->out_norm, bytes, H);
  }
  if (nm == "per_layer_token_embd.weight") {
    if (!PD) return e4b_fail(E4B_EINVAL, "%s given but ple_dim is 0", name);
    if ((rc = expect(name, type, E4B_GGML_Q6_K, dims, nd, LPD, V)) || (rc = check_bytes((size_t)(V * LPD / 256) * 210)))
      return rc;
    if (!c->ple_tab && (rc = dalloc(c, (void**)&c->ple_tab, nbytes))) return rc;
    E4B_HIP(hipMemcpy(c->ple_tab, bytes, nbytes, hipMemcpyHostToDevice));
    return E4B_OK;
  }
  if (nm == "per_layer_model_proj.weight") {
    if (!PD) return e4b_fail(E4B_EINVAL, "%s given but ple_dim is 0", name);
    if ((rc = expect(name, type, E4B_GGML_Q4_0, dims, nd, H, LPD)) || (rc = check_bytes((size_t)(LPD * H / 32) * 18)))
      return rc;
    if (!c->ple_proj && (rc = dalloc(c, (void**)&c->ple_proj, e4b_q40_packed_bytes(LPD, H)))) return rc;
    return upload_q40_rows(c->ple_proj, LPD, H, 0, bytes, LPD);
  }
  if (nm == "per_layer_proj_norm.weight") {
    if (!PD) return e4b_fail(E4B_EINVAL, "%s given but ple_dim is 0", name);
    if ((rc = expect(name, type, E4B_GGML_F32, dims, nd, PD, 1)) || (rc = check_bytes((size_t)PD * 4))) return rc;
    return upload_f32(c, &c->ple_norm, bytes, PD);
  }
  // blk.N.<part>.weight / blk.N.<part>.scale
  int li = -1, used = 0;
  if (sscanf(name, "blk.%d.%n", &li, &used) != 1 || used <= 0 || li < 0 || li >= k.layers)
    return e4b_fail(E4B_EINVAL, "e4b_set_tensor: unknown tensor '%s'", name);
  int pi = -1;
  for (int i = 0; i < P_COUNT; ++i)
    if (strcmp(name + used, kPartNames[i]) == 0) pi = i;
  if (pi < 0) return e4b_fail(E4B_EINVAL, "e4b_set_tensor: unknown tensor '%s'", name);
  const bool a4b = k.recipe == E4B_RECIPE_A4B;
  if (a4b && (bit(pi) & kPleParts))
    return e4b_fail(E4B_EINVAL, "e4b_set_tensor: '%s' is not part of the A4B recipe (no per-layer embeddings)", name);
  if (!a4b && pi >= P_PRE_FFW2)
    return e4b_fail(E4B_EINVAL, "e4b_set_tensor: '%s' belongs to the A4B recipe's MoE half (recipe is E4B)", name);
  Layer& ly = c->L[li];
  const int64_t QH = k.q_heads, KVH = ly.kvh, HD = ly.hd, FF = k.ffn, E = k.n_experts, FE = k.expert_ffn;
  auto q40 = [&](uint8_t** dst, int64_t total_rows, int64_t cols, int64_t row_off, int64_t rows) -> int {
    int r2;
    if ((r2 = expect(name, type, E4B_GGML_Q4_0, dims, nd, cols, rows)) ||
        (r2 = check_bytes((size_t)(rows * cols / 32) * 18)))
      return r2;
    if (!*dst && (r2 = dalloc(c, (void**)dst, e4b_q40_packed_bytes(total_rows, cols)))) return r2;
    return upload_q40_rows(*dst, total_rows, cols, row_off, bytes, rows);
  };
  auto f32v = [&](float** dst, int64_t len) -> int {
    int r2;
    if ((r2 = expect(name, type, E4B_GGML_F32, dims, nd, len, 1)) || (r2 = check_bytes((size_t)len * 4))) return r2;
    return upload_f32(c, dst, bytes, len);
  };
  switch (pi) {
    case P_ATTN_NORM: rc = f32v(&ly.attn_norm, H); break;
    case P_Q: rc = q40(&ly.qkv, ly.qkv_rows, H, 0, QH * HD); break;
    case P_K: rc = q40(&ly.qkv, ly.qkv_rows, H, QH * HD, KVH * HD); break;
    case P_V:
      // a V = K layer reads V from the K rows; the reference does not load
      // this tensor there (src/engine-a4b.js:202), nor does the library
      if (ly.keqv) return E4B_OK;
      rc = q40(&ly.qkv, ly.qkv_rows, H, (QH + KVH) * HD, KVH * HD);
      break;
    case P_Q_NORM: rc = f32v(&ly.q_norm, HD); break;
    case P_K_NORM: rc = f32v(&ly.k_norm, HD); break;
    case P_O: rc = q40(&ly.o, H, QH * HD, 0, H); break;
    case P_POST_ATTN: rc = f32v(&ly.post_attn, H); break;
    case P_FFN_NORM: rc = f32v(&ly.ffn_norm, H); break;
    case P_GATE: rc = q40(&ly.gu, 2 * FF, H, 0, FF); break;
    case P_UP: rc = q40(&ly.gu, 2 * FF, H, FF, FF); break;
    case P_DOWN: rc = q40(&ly.down, H, FF, 0, H); break;
    case P_POST_FFW: rc = f32v(&ly.post_ffw, H); break;
    case P_INP_GATE:
      if (!PD) return e4b_fail(E4B_EINVAL, "%s given but ple_dim is 0", name);
      rc = q40(&ly.pg, PD, H, 0, PD);
      break;
    case P_PROJ:  // stored block-transposed for the fused PLE branch
      if (!PD) return e4b_fail(E4B_EINVAL, "%s given but ple_dim is 0", name);
      if ((rc = expect(name, type, E4B_GGML_Q4_0, dims, nd, PD, H)) || (rc = check_bytes((size_t)(H * PD / 32) * 18)))
        return rc;
      if (!ly.pp && (rc = dalloc(c, (void**)&ly.pp, e4b_q40_packed_bytes(H, PD)))) return rc;
      if (!ly.pp_rm && (rc = dalloc(c, (void**)&ly.pp_rm, e4b_q40_packed_bytes(H, PD)))) return rc;
      if ((rc = upload_q40_block_t(ly.pp, H, PD, bytes))) return rc;
      rc = upload_q40_rows(ly.pp_rm, H, PD, 0, bytes, H);
      break;
    case P_POST_NORM: rc = f32v(&ly.post_norm, H); break;
    case P_SCALE:
      if (type != E4B_GGML_F32 || n != 1 || nbytes != 4) return e4b_fail(E4B_EINVAL, "%s: expected one f32", name);
      memcpy(&ly.scale, bytes, 4);
      rc = E4B_OK;
      break;
    case P_PRE_FFW2: rc = f32v(&ly.pre_ffw2, H); break;
    case P_POST_FFW1: rc = f32v(&ly.post_ffw1, H); break;
    case P_POST_FFW2: rc = f32v(&ly.post_ffw2, H); break;
    case P_ROUTER_SCALE: rc = f32v(&ly.router_scale, H); break;
    case P_PES: rc = f32v(&ly.pes, E); break;
    case P_ROUTER_W:  // f32 [E][H]
      if ((rc = expect(name, type, E4B_GGML_F32, dims, nd, H, E)) || (rc = check_bytes((size_t)(E * H) * 4))) return rc;
      rc = upload_f32(c, &ly.router_w, bytes, E * H);
      break;
    case P_EXP_GU:  // q4_0 [E][2 FE][H]: per expert the gate rows, then the up rows
      if ((rc = expect(name, type, E4B_GGML_Q4_0, dims, nd, H, 2 * FE, E)) ||
          (rc = check_bytes((size_t)(E * 2 * FE * H / 32) * 18)))
        return rc;
      if (!ly.exp_gu && (rc = dalloc(c, (void**)&ly.exp_gu, e4b_q40_packed_bytes(E * 2 * FE, H)))) return rc;
      rc = upload_q40_rows(ly.exp_gu, E * 2 * FE, H, 0, bytes, E * 2 * FE);
      break;
    case P_EXP_DOWN:  // q4_0 [E][H][FE]
      if ((rc = expect(name, type, E4B_GGML_Q4_0, dims, nd, FE, H, E)) ||
          (rc = check_bytes((size_t)(E * H * FE / 32) * 18)))
        return rc;
      if (!ly.exp_down && (rc = dalloc(c, (void**)&ly.exp_down, e4b_q40_packed_bytes(E * H, FE)))) return rc;
      rc = upload_q40_rows(ly.exp_down, E * H, FE, 0, bytes, E * H);
      break;
    default: rc = e4b_fail(E4B_EINVAL, "unhandled part %d", pi);
  }
  if (rc == E4B_OK) ly.have |= 1u << pi;
  return rc;
}

namespace {

int missing_parts(const e4b_ctx* c, int l, uint32_t need) {
  const uint32_t miss = need & ~c->L[l].have;
  for (int i = 0; i < P_COUNT; ++i)
    if (miss & bit(i)) return e4b_fail(E4B_ENOTENSOR, "missing blk.%d.%s", l, kPartNames[i]);
  return E4B_OK;
}

// The A4B recipe's device state: per-layer caches of the layer's KV heads and
// head dim, the split-K partials of the widest layer, the MoE half's scratch.
// Prompts run through the decode step (no batched prefill buffers).
int finalize_a4b(e4b_ctx* c) {
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, FF = k.ffn, E = k.n_experts, FE = k.expert_ffn;
  int rc;
  for (int l = 0; l < k.layers; ++l)
    if ((rc = missing_parts(c, l, kNeedA4B & ~(c->L[l].keqv ? bit(P_V) : 0u)))) return rc;
  // RoPE inverse frequencies THETA^(-2p/hd) with each layer type's head dim
  const int hd_s = k.head_dim, hd_f = k.head_dim_full ? k.head_dim_full : k.head_dim;
  {
    std::vector<float> il(hd_s / 2), ig(hd_f / 2);
    rope_inv_freq(k.theta_local, hd_s, hd_s / 2, il.data());
    rope_inv_freq(k.theta_global, hd_f, hd_f / 2, ig.data());
    if ((rc = upload_f32(c, &c->inv_local, il.data(), hd_s / 2)) ||
        (rc = upload_f32(c, &c->inv_global, ig.data(), hd_f / 2)))
      return rc;
  }
  c->chunk = kAttnGenChunk;
  c->ring_cap = k.max_seq;
  c->max_prompt = k.max_prompt > 0 ? k.max_prompt : k.max_seq;
  c->amax_parts = q6k_gemv_grid(k.vocab, k.hidden / 32);
  c->pf_cap = 0;
  size_t part = 0, ml = 0;
  int hd_max = 0;
  for (int l = 0; l < k.layers; ++l) {
    Layer& ly = c->L[l];
    ly.slots = ly.global ? k.max_seq : k.ring;
    ly.gch = attn_chunks(ly.global ? k.max_seq : k.window, kAttnGenChunk);
    const size_t n = (size_t)ly.kvh * ly.slots * ly.hd;
    if ((rc = dalloc_t(c, &ly.kc, n)) || (rc = dalloc_t(c, &ly.vc, n))) return rc;
    part = std::max(part, (size_t)QH * ly.gch * ly.hd);
    ml = std::max(ml, (size_t)QH * ly.gch * 2);
    hd_max = std::max(hd_max, ly.hd);
  }
  MoeArgs& m = c->moe;
  if ((rc = dalloc_t(c, &c->params, 16)) || (rc = dalloc_t(c, &c->prompt, (size_t)c->max_prompt)) ||
      (rc = dalloc_t(c, &c->tok_ring, (size_t)c->ring_cap)) || (rc = dalloc_t(c, &c->amax, 4)) ||
      (rc = dalloc_t(c, &c->status, 4)) || (rc = dalloc_t(c, &c->h, (size_t)H)) ||
      (rc = dalloc_t(c, &c->hb, (size_t)H)) || (rc = dalloc_t(c, &c->rope, (size_t)hd_s)) ||
      (rc = dalloc_t(c, &c->h_hl, (size_t)2 * H)) || (rc = dalloc_t(c, &c->xn, (size_t)H)) ||
      (rc = dalloc_t(c, &c->qkv, (size_t)c->qkv_rows)) ||
      (rc = dalloc_t(c, &c->part_o, part)) || (rc = dalloc_t(c, &c->part_ml, ml)) ||
      (rc = dalloc_t(c, &c->attn, (size_t)QH * hd_max)) || (rc = dalloc_t(c, &c->o, (size_t)4 * H)) ||
      (rc = dalloc_t(c, &c->xo_hl, (size_t)2 * H)) || (rc = dalloc_t(c, &c->logits, (size_t)k.vocab)) ||
      (rc = dalloc_t(c, &c->amax_part, (size_t)c->amax_parts)) || (rc = dalloc_t(c, &m.scores, (size_t)E)) ||
      (rc = dalloc_t(c, &m.xd, (size_t)H)) || (rc = dalloc_t(c, &m.xm, (size_t)H)) ||
      (rc = dalloc_t(c, &m.topk_idx, (size_t)kMoeTopK * k.layers)) ||
      (rc = dalloc_t(c, &m.topk_w, (size_t)kMoeTopK * k.layers)) ||
      ((k.flags & E4B_FLAG_LAYER_HIDDEN) && (rc = dalloc_t(c, &c->lh, (size_t)k.layers * H))) ||
      (rc = dalloc_t(c, &m.g_dense, (size_t)FF)) || (rc = dalloc_t(c, &m.g_slots, (size_t)kMoeTopK * FE)) ||
      (rc = dalloc_t(c, &m.dense_out, (size_t)H)) || (rc = dalloc_t(c, &m.moe_out, (size_t)H)))
    return rc;
  // full-layer KV budget (src/engine-a4b.js:587-657): accumulated attention
  // mass per full layer, the step's raw scores, the keep list and the gather
  // scratch
  if (k.flags & E4B_FLAG_KV_SCORE) {
    const size_t S = (size_t)k.max_seq;
    size_t rows = 1;
    for (Layer& ly : c->L)
      if (ly.global) {
        if ((rc = dalloc_t(c, &ly.score, (size_t)QH * S))) return rc;
        rows = std::max(rows, (size_t)ly.kvh * ly.slots * ly.hd);
      }
    if ((rc = dalloc_t(c, &c->raw, (size_t)QH * S)) || (rc = dalloc_t(c, &c->keep, S)) ||
        (rc = dalloc_t(c, &c->kv_sk, rows)) || (rc = dalloc_t(c, &c->kv_sv, rows)))
      return rc;
  }
  // batched prefill (src/engine-a4b.js:259-295, 465-584): chunks of up to 512
  // tokens; a chunk must leave every key its queries need in the sliding
  // rings (ring >= window + M - 1, the Complete condition of
  // specs/KVRing.tla with C = M), and the MoE prefill takes <= 1024 tokens
  {
    int cap = kPfMaxChunk;
    bool any_sliding = false;
    for (int l = 0; l < k.layers; ++l) any_sliding |= !c->L[l].global;
    if (cap > c->max_prompt) cap = c->max_prompt;
    if (cap > k.max_seq) cap = k.max_seq;
    if (any_sliding && cap > k.ring - k.window + 1) cap = k.ring - k.window + 1;
    if (cap > 128) cap = cap / 128 * 128;
    if (cap >= 1) {
      const size_t M = (size_t)cap;
      MoeArgs shape = m;
      shape.H = H;
      shape.E = E;
      shape.FF = FE;
      shape.FF2 = FF;
      const size_t moe_bytes = moe_prefill_scratch(shape, cap, nullptr, nullptr);
      // split-key partials of the matrix-core attention (sliding layers of
      // head dim 256 with 1, 2 or 4 q heads per KV head)
      size_t apart = 0;
      for (int l = 0; l < k.layers; ++l)
        if (a4b_pf_mfma_attn(c->L[l], QH))
          apart = std::max(apart, attn_prefill_part_bytes(cap, c->L[l].kvh, QH / c->L[l].kvh, c->L[l].hd));
      if ((rc = dalloc_t(c, &c->pf_ids, M)) || (rc = dalloc_t(c, &c->pf_h, M * H)) ||
          (rc = dalloc_t(c, &c->pf_xn, M * H)) || (rc = dalloc_t(c, &c->pf_qkv, (size_t)kPfA4bQkvKs * M * c->qkv_rows)) ||
          (rc = dalloc_t(c, &c->pf_q, M * QH * hd_max)) || (rc = dalloc_t(c, &c->pf_attn, M * QH * hd_max)) ||
          (rc = dalloc_t(c, &c->pf_y, (size_t)kPfA4bOKs * M * H)) || (rc = dalloc_t(c, &c->pf_xhl, 2 * M * H)) ||
          (rc = dalloc(c, (void**)&c->pf_moe, moe_bytes)) ||
          (apart && (rc = dalloc(c, (void**)&c->pf_apart, apart))))
        return rc;
      c->pf_apart_bytes = apart;
      moe_prefill_scratch(shape, cap, &c->pf_mb, c->pf_moe);
      c->pf_cap = cap;
    }
  }
  return E4B_OK;
}

}  // namespace

extern "C" int e4b_finalize(e4b_ctx* c) {
  if (!c) return e4b_fail(E4B_EINVAL, "e4b_finalize: null");
  if (c->finalized) return E4B_OK;
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, KVH = k.kv_heads, HD = k.head_dim, FF = k.ffn, PD = k.ple_dim;
  if (!c->embd) return e4b_fail(E4B_ENOTENSOR, "missing token_embd.weight");
  if (!c->out_norm) return e4b_fail(E4B_ENOTENSOR, "missing output_norm.weight");
  int rc;
  if (k.recipe == E4B_RECIPE_A4B) {
    if ((rc = finalize_a4b(c))) return rc;
  } else {
  if (PD && (!c->ple_tab || !c->ple_proj || !c->ple_norm))
    return e4b_fail(E4B_ENOTENSOR, "missing per_layer_token_embd / per_layer_model_proj / per_layer_proj_norm");
  for (int l = 0; l < k.layers; ++l)
    if ((rc = missing_parts(c, l, kNeedE4B | (PD ? kPleParts : 0u)))) return rc;
  // RoPE inverse frequencies THETA^(-2p/HD), rounded once to f32
  {
    std::vector<float> il(HD / 2), ig(HD / 2);
    rope_inv_freq(k.theta_local, HD, HD / 2, il.data());
    rope_inv_freq(k.theta_global, HD, HD / 2, ig.data());
    if ((rc = upload_f32(c, &c->inv_local, il.data(), HD / 2)) || (rc = upload_f32(c, &c->inv_global, ig.data(), HD / 2)))
      return rc;
  }
  // split-K attention: chunks of `chunk` positions; partials sized for the
  // layer with the most live positions
  // The sliding layers use 32-position chunks (16 for a 512 window) in 4 V
  // slices, so a window's K/V rows are spread over 128 blocks, and the o
  // projection's prologue merges their 16 chunks in one pass; the full
  // layers use attn_chunk (default 64) in 4 V slices.
  c->chunk = k.attn_chunk ? k.attn_chunk : 64;
  c->chunk_sw = k.attn_chunk == 64 ? 64 : E4B_TUNE_CHUNK_SW;
  c->nch = std::max(attn_chunks(k.max_seq, c->chunk), attn_chunks(k.window, c->chunk_sw));
  if (c->nch > kAttnMaxChunks)
    return e4b_fail(E4B_EINVAL, "max_seq %d needs %d attention chunks (max %d)", k.max_seq, c->nch, kAttnMaxChunks);
  c->ring_cap = k.max_seq;
  c->max_prompt = k.max_prompt > 0 ? k.max_prompt : k.max_seq;
  c->amax_parts = q6k_gemv_grid(k.vocab, k.hidden / 32);
  // caches
  for (int l = 0; l < k.layers; ++l) {
    Layer& ly = c->L[l];
    ly.slots = ly.global ? k.max_seq : k.ring;
    const size_t n = (size_t)KVH * ly.slots * HD;
    if ((rc = dalloc_t(c, &ly.kc, n)) || (rc = dalloc_t(c, &ly.vc, n))) return rc;
  }
  // activations
  const int NP = PD ? k.layers * PD : 1;
  if ((rc = dalloc_t(c, &c->params, 16)) || (rc = dalloc_t(c, &c->prompt, (size_t)c->max_prompt)) ||
      (rc = dalloc_t(c, &c->tok_ring, (size_t)c->ring_cap)) || (rc = dalloc_t(c, &c->amax, 4)) ||
      (rc = dalloc_t(c, &c->status, 4)) || (rc = dalloc_t(c, &c->h, (size_t)H)) ||
      (rc = dalloc_t(c, &c->hb, (size_t)H)) || (rc = dalloc_t(c, &c->rope, (size_t)HD)) ||
      (rc = dalloc_t(c, &c->h_hl, (size_t)2 * H)) || (rc = dalloc_t(c, &c->proj, (size_t)NP)) ||
      (rc = dalloc_t(c, &c->ple, (size_t)NP)) || (rc = dalloc_t(c, &c->xn, (size_t)H)) ||
      (rc = dalloc_t(c, &c->qkv, (size_t)c->qkv_rows)) ||
      (rc = dalloc_t(c, &c->part_o, (size_t)QH * c->nch * HD)) ||
      (rc = dalloc_t(c, &c->part_ml, (size_t)QH * c->nch * 2)) || (rc = dalloc_t(c, &c->attn, (size_t)QH * HD)) ||
      (rc = dalloc_t(c, &c->o, (size_t)2 * H)) || (rc = dalloc_t(c, &c->xf, (size_t)H)) ||
      (rc = dalloc_t(c, &c->gg, (size_t)FF)) || (rc = dalloc_t(c, &c->dn, (size_t)2 * H)) ||
      (rc = dalloc_t(c, &c->xg, (size_t)H)) || (rc = dalloc_t(c, &c->gp, (size_t)(PD ? PD : 1))) ||
      (rc = dalloc_t(c, &c->pp, (size_t)(PD ? PD / 32 : 1) * H)) || (rc = dalloc_t(c, &c->xo_hl, (size_t)2 * H)) ||
      (rc = dalloc_t(c, &c->logits, (size_t)k.vocab)) || (rc = dalloc_t(c, &c->amax_part, (size_t)c->amax_parts)) ||
      ((k.flags & E4B_FLAG_LAYER_HIDDEN) && (rc = dalloc_t(c, &c->lh, (size_t)k.layers * H))))
    return rc;
  // batched prefill buffers: a chunk of M tokens must leave every key its
  // queries need in the sliding rings (ring >= window + M - 1, the Complete
  // condition of specs/KVRing.tla with C = M)
  {
    bool any_sliding = false;
    for (int l = 0; l < k.layers; ++l) any_sliding |= !c->L[l].global;
    int cap = kPfMaxChunk;
    if (cap > c->max_prompt) cap = c->max_prompt;
    if (cap > k.max_seq) cap = k.max_seq;
    if (any_sliding && cap > k.ring - k.window + 1) cap = k.ring - k.window + 1;
    // whole 128-token GEMM tiles: a 513-token chunk (ring 1024, window 512)
    // would run a fifth token tile for one token
    if (cap > 128) cap = cap / 128 * 128;
    c->pf_cap = cap;
    const size_t M = (size_t)cap, NPs = (size_t)NP;
    if ((rc = dalloc_t(c, &c->pf_ids, M)) || (rc = dalloc_t(c, &c->pf_h, M * H)) ||
        (rc = dalloc_t(c, &c->pf_proj, 2 * M * NPs)) || (rc = dalloc_t(c, &c->pf_ple, M * NPs)) ||
        (rc = dalloc_t(c, &c->pf_qkv, kPfKsQkv * M * (size_t)c->qkv_rows)) || (rc = dalloc_t(c, &c->pf_q, M * QH * HD)) ||
        (rc = dalloc_t(c, &c->pf_y, (size_t)kPfKs * M * H)) || (rc = dalloc_t(c, &c->pf_xhl, 2 * M * H)) ||
        (rc = dalloc_t(c, &c->pf_xn, M * H)) || (rc = dalloc_t(c, &c->pf_attn, M * QH * HD)) ||
        (rc = dalloc_t(c, &c->pf_gg, M * FF)) || (rc = dalloc_t(c, &c->pf_gp, M * (size_t)(PD ? PD : 1))))
      return rc;
    c->pf_apart_bytes = attn_prefill_part_bytes(cap, KVH, QH / KVH);
    if ((rc = dalloc(c, (void**)&c->pf_apart, c->pf_apart_bytes))) return rc;
  }
  if (k.flags & E4B_FLAG_KV_SCORE) {
    const size_t S = (size_t)k.max_seq;
    for (Layer& ly : c->L)
      if (ly.global && (rc = dalloc_t(c, &ly.score, (size_t)QH * S))) return rc;
    if ((rc = dalloc_t(c, &c->raw, (size_t)QH * S)) || (rc = dalloc_t(c, &c->keep, S)) ||
        (rc = dalloc_t(c, &c->kv_sk, (size_t)KVH * S * HD)) || (rc = dalloc_t(c, &c->kv_sv, (size_t)KVH * S * HD)))
      return rc;
  }
  }  // E4B recipe
  c->finalized = true;
  if ((rc = e4b_reset(c))) return rc;
  if (k.flags & E4B_FLAG_NO_GRAPH) return E4B_OK;
  // capture one token
  E4B_HIP(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
  rc = record_step(c);
  hipGraph_t g = nullptr;
  hipError_t ce = hipStreamEndCapture(c->st, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    c->finalized = false;
    return rc;
  }
  if (ce != hipSuccess) {
    c->finalized = false;
    return e4b_fail(E4B_EHIP, "hipStreamEndCapture: %s", hipGetErrorString(ce));
  }
  c->graph = g;
  E4B_HIP(hipGraphInstantiate(&c->exec, c->graph, nullptr, nullptr, 0));
  return E4B_OK;
}

namespace {


// One token of the A4B recipe (the reference's encodeForward / encodeLayer,
// src/engine-a4b.js:424-463, 683-693): embedding; per layer the q|k(|v)
// GEMV (whose prologue runs the previous layer's MoE tail and this layer's
// input norm), head prep with the K/V write, split-K attention and its
// merge, o, then the MoE half (router with the attention residual, top-8,
// dense and expert gate/up + GeGLU, dense and expert down); after the last
// layer its tail, the final norm, lm-head + argmax, feedback.  The residual
// stream is c->h at layer boundaries and c->hb (h1) after the attention
// residual.
int record_step_a4b(e4b_ctx* c) {
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, E = k.n_experts, FE = k.expert_ffn, FF = k.ffn;
  hipStream_t st = c->st;
  int rc;
  const Q6Mat Em = q6_view(c->embd, k.vocab, H);
  if ((rc = launch_embed(Em, c->params, c->prompt, sqrtf((float)H), c->h, c->h_hl, c->status, c->inv_local,
                         c->inv_global, k.head_dim / 2, c->rope, st)) ||
      (rc = tick(c, "embed")))
    return rc;
  for (int l = 0; l < k.layers; ++l) {
    const Layer& ly = c->L[l];
    const int window = ly.global ? 0 : k.window;
    // 1. q|k(|v) GEMV; its prologue finishes the previous layer (the MoE
    //    tail over h1 in hb, written to h) and applies this layer's input norm
    GemvOut oq = {c->qkv, nullptr, nullptr, 0};
    ProArgs pq{};
    pq.tail = 1;
    pq.H = H;
    pq.eps = k.eps;
    pq.w2 = ly.attn_norm;
    pq.scale = 1.f;
    if (l == 0) {
      pq.hin = c->h;
    } else {
      const Layer& pv = c->L[l - 1];
      pq.hin = c->hb;
      pq.hout = c->h;
      pq.a = c->moe.dense_out;
      pq.a2 = c->moe.moe_out;
      pq.w1 = pv.post_ffw1;
      pq.w1b = pv.post_ffw2;
      pq.wp = pv.post_ffw;
      pq.scale = pv.scale;
      if (c->lh) pq.hsnap = c->lh + (size_t)(l - 1) * H;  // E4B_FLAG_LAYER_HIDDEN: the stream after layer l - 1
    }
    if ((rc = launch_q40(q40_view(ly.qkv, ly.qkv_rows, H), nullptr, nullptr, EPI_F32, oq, 1, st, &pq)) ||
        (rc = tick(c, "qkv")))
      return rc;
    AttnGen ag{};
    ag.qkv = c->qkv;
    ag.qw = ly.q_norm;
    ag.kw = ly.k_norm;
    ag.inv_freq = ly.global ? c->inv_global : c->inv_local;
    // the step's (cos, sin) table (k_embed) holds head_dim / 2 pairs per layer type
    ag.rope = ly.angles <= k.head_dim / 2 ? c->rope + (ly.global ? k.head_dim / 2 : 0) : nullptr;
    ag.params = c->params;
    ag.kc = ly.kc;
    ag.vc = ly.vc;
    ag.part_o = c->part_o;
    ag.part_ml = c->part_ml;
    ag.out = c->attn;
    ag.qh = QH;
    ag.kvh = ly.kvh;
    ag.hd = ly.hd;
    ag.angles = ly.angles;
    ag.slots = ly.slots;
    ag.window = window;
    ag.kv_idx = 4;  // full layers: params[4] = the token's slot
    ag.gch = ly.gch;
    ag.keqv = ly.keqv;
    ag.eps = k.eps;
    ag.raw = ly.score ? c->raw : nullptr;
    // the o projection merges the split-K partials in its prologue, in
    // column slices of 4 heads (2 or 4 slices, their partial outputs summed
    // by the router), when the layer's chunks fit the prologue's lanes;
    // else the merge launch writes the f16 attention output
    static_assert(kAttnGenChunk == 64, "the prologue's chunk_shift below");
    const int oks = QH / 4;
#ifdef E4B_TUNE_A4B_MERGE_LAUNCH  // A/B builds: the merge as its own launch
    const bool fuse = false;
#else
    const bool fuse = QH % 4 == 0 && (oks == 2 || oks == 4) && ly.gch <= kProAttnMaxChunks;
#endif
    ag.no_merge = fuse;
    GemvOut oo = {c->o, nullptr, nullptr, 0};
    const Q40Mat Wo = q40_view(ly.o, H, (int64_t)QH * ly.hd);
    if ((rc = launch_attn_gen(ag, st)) || (rc = tick(c, ly.global ? "attn_global" : "attn_sliding")) ||
        (ly.score && ((rc = launch_attn_score(c->part_ml, c->raw, c->params, 4, QH, ly.slots, kAttnGenChunk, ly.score,
                                              st)) ||
                      (rc = tick(c, "attn_score")))))
      return rc;
    if (fuse) {
      ProArgs pa{};
      pa.part_o = c->part_o;
      pa.part_ml = c->part_ml;
      pa.params = c->params;
      pa.kv_idx = 4;
      pa.window = window;
      pa.chunk_shift = 6;  // kAttnGenChunk = 64 positions
      pa.gch = ly.gch;
      pa.head_dim = ly.hd;
      rc = launch_q40(Wo, nullptr, nullptr, EPI_F32, oo, oks, st, &pa);
    } else {
      rc = launch_q40(Wo, (const uint32_t*)c->attn, nullptr, EPI_F32, oo, 1, st);
    }
    if (rc || (rc = tick(c, "o_proj"))) return rc;
    // 2. MoE half; its router forms the attention residual h1 = h +
    //    rms(o) post_attn into hb; the tail runs in the next layer's qkv
    //    prologue, after the last layer in its own launch (h = the output)
    MoeArgs a = c->moe;
    a.h = c->h;
    a.attn_o = c->o;
    a.attn_o_slices = fuse ? oks : 1;
    a.post_attn = ly.post_attn;
    a.h1 = c->hb;
    a.ffn_norm = ly.ffn_norm;
    a.router_scale = ly.router_scale;
    a.router_mult = 1.0f / sqrtf((float)H);
    a.pre_ffw2 = ly.pre_ffw2;
    a.router_w = ly.router_w;
    a.pes = ly.pes;
    a.dense_gu = q40_view(ly.gu, 2 * (int64_t)FF, H);
    a.exp_gu = q40_view(ly.exp_gu, (int64_t)E * 2 * FE, H);
    a.dense_down = q40_view(ly.down, H, FF);
    a.exp_down = q40_view(ly.exp_down, (int64_t)E * H, FE);
    a.post_ffw1 = ly.post_ffw1;
    a.post_ffw2 = ly.post_ffw2;
    a.post_ffw = ly.post_ffw;
    a.layer_scale = ly.scale;
    a.eps = k.eps;
    a.H = H;
    a.E = E;
    a.FF = FE;
    a.FF2 = FF;
    a.h_out = l == k.layers - 1 ? c->h : nullptr;
    a.topk_idx = c->moe.topk_idx + (size_t)kMoeTopK * l;  // each layer's picks stay readable (e4b_read_topk)
    a.topk_w = c->moe.topk_w + (size_t)kMoeTopK * l;
    if ((rc = launch_moe_ffn(a, st)) || (rc = tick(c, "moe_ffn"))) return rc;
  }
  c->h_final = c->h;
  if ((rc = launch_rownorm(c->h, nullptr, nullptr, nullptr, 1.f, c->out_norm, c->xo_hl, c->xo_hl + H, H, k.eps, st)) ||
      (rc = tick(c, "final_norm")) ||
      (rc = launch_q6k_gemv_argmax(Em, (const uint32_t*)c->xo_hl, (const uint32_t*)(c->xo_hl + H), k.softcap,
                                   c->logits, nullptr, c->amax_part, st)) ||
      (rc = tick(c, "lm_head")) ||
      (rc = launch_feedback(c->amax_part, c->amax_parts, c->amax, c->params, c->tok_ring, c->ring_cap, st)))
    return rc;
  return tick(c, "argmax_feedback");
}

int record_step(e4b_ctx* c) {
  if (c->cfg.recipe == E4B_RECIPE_A4B) return record_step_a4b(c);
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, KVH = k.kv_heads, HD = k.head_dim, FF = k.ffn, PD = k.ple_dim;
  const int Lc = k.layers;
  hipStream_t st = c->st;
  int rc;
  const Q6Mat E = q6_view(c->embd, k.vocab, H);
  // the hidden state ping-pongs between two buffers: a fused prologue reads
  // `hcur` in every block while block (0,0) writes the updated state to `hnext`
  float* hcur = c->h;
  float* hnext = c->hb;
  auto swap_h = [&]() {
    float* t = hcur;
    hcur = hnext;
    hnext = t;
  };
  auto pro = [&](float* hout, const float* a, const float* w1, const float* w2, float scale) {
    ProArgs p{};
    p.hin = hcur;
    p.hout = hout;
    p.a = a;
    p.w1 = w1;
    p.w2 = w2;
    p.scale = scale;
    p.H = H;
    p.eps = k.eps;
    return p;
  };
  if ((rc = launch_embed(E, c->params, c->prompt, sqrtf((float)H), c->h, c->h_hl, c->status, c->inv_local,
                         c->inv_global, HD / 2, c->rope, st)) ||
      (rc = tick(c, "embed")))
    return rc;
  if (PD) {
    GemvOut po = {c->proj, nullptr, nullptr, 0};
    if ((rc = launch_q40(q40_view(c->ple_proj, (int64_t)Lc * PD, H), (const uint32_t*)c->h_hl,
                         (const uint32_t*)(c->h_hl + H), EPI_F32, po, 1, st)) ||
        (rc = tick(c, "ple_model_proj")))
      return rc;
    if ((rc = launch_ple_prep(c->proj, c->ple_tab, c->ple_norm, c->params, c->prompt, Lc, k.vocab,
                              1.0f / sqrtf((float)H), c->ple, c->h, c->L[0].attn_norm, c->xn, H, k.eps, st)) ||
        (rc = tick(c, "ple_prep")))
      return rc;
  }
  for (int l = 0; l < Lc; ++l) {
    const Layer& ly = c->L[l];
    // 1. qkv GEMV; its prologue finishes the previous layer (last residual,
    //    layer scalar) and applies this layer's input norm
    GemvOut oq = {c->qkv, nullptr, nullptr, 0};
    const Q40Mat Wqkv = q40_view(ly.qkv, c->qkv_rows, H);
    if (l == 0) {
      if (PD) {
        rc = launch_q40(Wqkv, (const uint32_t*)c->xn, nullptr, EPI_F32, oq, 1, st);
      } else {
        const ProArgs p = pro(nullptr, nullptr, nullptr, ly.attn_norm, 1.0f);
        rc = launch_q40(Wqkv, nullptr, nullptr, EPI_F32, oq, 1, st, &p);
      }
    } else {
      const Layer& pv = c->L[l - 1];
      ProArgs p = PD ? pro(hnext, c->pp, pv.post_norm, ly.attn_norm, pv.scale)
                     : pro(hnext, c->dn, pv.post_ffw, ly.attn_norm, pv.scale);
      if (PD) p.na = PD / 32;  // the PLE branch leaves PD/32 partial projections
      if (c->lh) p.hsnap = c->lh + (size_t)(l - 1) * H;  // E4B_FLAG_LAYER_HIDDEN: the stream after layer l - 1
      rc = launch_q40(Wqkv, nullptr, nullptr, EPI_F32, oq, 1, st, &p);
      swap_h();
    }
    if (rc || (rc = tick(c, "qkv"))) return rc;
    // 2. attention (head prep, KV write, split-K); the combine is the o
    //    projection's prologue when the projection has 2048 columns and the
    //    layer's live span fits the prologue's 64 chunks per head (global
    //    layers of contexts beyond 4096 positions use the combine launch)
    const int chunk_l = ly.global ? c->chunk : c->chunk_sw;
    const int gch_layer = attn_chunks(ly.global ? ly.slots : k.window, chunk_l);
    const bool fuse_combine = QH * HD == kProAttnH && gch_layer <= kProAttnMaxChunks;
    AttnLaunch a;
    a.qkv = c->qkv;
    a.qw = ly.q_norm;
    a.kw = ly.k_norm;
    a.inv_freq = ly.global ? c->inv_global : c->inv_local;
    a.rope = c->rope + (ly.global ? HD / 2 : 0);
    a.kc = ly.kc;
    a.vc = ly.vc;
    a.params = c->params;
    a.pos = 0;
    a.part_o = c->part_o;
    a.part_ml = c->part_ml;
    a.out = c->attn;
    a.qh = QH;
    a.kvh = KVH;
    a.hd = HD;
    a.angles = k.rope_angles;
    a.slots = ly.slots;
    a.window = ly.global ? 0 : k.window;
    a.chunk = chunk_l;
    a.vslices = ly.global ? c->vs_gl : c->vs_sw;
    a.combine = !fuse_combine;
    a.eps = k.eps;
    a.kv_idx = 4;  // full layers: params[4] = the token's slot
    a.raw = ly.score ? c->raw : nullptr;
    if ((rc = launch_attn(a, st)) || (rc = tick(c, ly.global ? "attn_global" : "attn_sliding"))) return rc;
    if (ly.score && ((rc = launch_attn_score(c->part_ml, c->raw, c->params, 4, QH, ly.slots, c->chunk, ly.score, st)) ||
                     (rc = tick(c, "attn_score"))))
      return rc;
    // 3. o projection
    GemvOut oo = {c->o, nullptr, nullptr, 0};
    const Q40Mat Wo = q40_view(ly.o, H, (int64_t)QH * HD);
    if (fuse_combine) {
      ProArgs pa{};
      pa.part_o = c->part_o;
      pa.part_ml = c->part_ml;
      pa.params = c->params;
      pa.kv_idx = 4;
      pa.window = a.window;
      pa.chunk_shift = chunk_l == 64 ? 6 : 5;
      pa.gch = gch_layer;
      rc = launch_q40(Wo, nullptr, nullptr, EPI_F32, oo, E4B_TUNE_OKS, st, &pa);
    } else {
      rc = launch_q40(Wo, (const uint32_t*)c->attn, nullptr, EPI_F32, oo, 1, st);
    }
    if (rc || (rc = tick(c, "o_proj"))) return rc;
    // 4. gate/up + GeGLU; prologue: post-attention residual + FFN input norm
    {
      ProArgs p = pro(hnext, c->o, ly.post_attn, ly.ffn_norm, 1.0f);
      if (fuse_combine) p.na = E4B_TUNE_OKS;  // the o projection's column slices
      GemvOut og = {nullptr, c->gg, nullptr, FF};
      if ((rc = launch_q40(q40_view(ly.gu, 2 * (int64_t)FF, H), nullptr, nullptr, EPI_GEGLU, og, 1, st, &p)) ||
          (rc = tick(c, "gate_up_geglu")))
        return rc;
      swap_h();
    }
    // 5. down projection; with the PLE branch as its consumer the columns
    //    are split in two slices (dn[0..H) + dn[H..2H)), which halves the
    //    GeGLU-vector reads per workgroup; the PLE prologue adds the slices
    GemvOut od = {c->dn, nullptr, nullptr, 0};
    const int dks = (PD && (FF / 32) % 8 == 0) ? 2 : 1;
    if ((rc = launch_q40(q40_view(ly.down, H, FF), (const uint32_t*)c->gg, nullptr, EPI_F32, od, dks, st)) ||
        (rc = tick(c, "down")))
      return rc;
    if (PD) {
      // 6. PLE branch in one launch: post-FFN residual prologue, gate x GELU x
      //    per-layer input, projection partials (summed by the next consumer)
      ProArgs p = pro(hnext, c->dn, ly.post_ffw, nullptr, 1.0f);
      p.na = dks;
      const size_t nbp = (size_t)H * (PD / 32);
      PleLaunch pl;
      pl.gate = q40_view(ly.pg, PD, H);
      pl.proj_nib = (const uint4*)ly.pp;
      pl.proj_sc = (const uint16_t*)(ly.pp + E4B_ALIGN256(nbp * 16));
      pl.ple = c->ple + (int64_t)l * PD;
      pl.part = c->pp;
      pl.H = H;
      pl.PD = PD;
      if ((rc = launch_ple(pl, p, st)) || (rc = tick(c, "ple"))) return rc;
      swap_h();
    }
  }
  // last residual + final norm (f32, hi/lo split) -> lm-head -> argmax/feedback
  const Layer& last = c->L[Lc - 1];
  if (PD)
    rc = launch_tail(hcur, c->pp, PD / 32, last.post_norm, last.scale, c->out_norm, c->xo_hl, H, k.eps, st);
  else
    rc = launch_tail(hcur, c->dn, 1, last.post_ffw, last.scale, c->out_norm, c->xo_hl, H, k.eps, st);
  if (rc || (rc = tick(c, "final_norm"))) return rc;
  c->h_final = hcur;
  if ((rc = launch_q6k_gemv_argmax(E, (const uint32_t*)c->xo_hl, (const uint32_t*)(c->xo_hl + H), k.softcap,
                                   c->logits, nullptr, c->amax_part, st)) ||
      (rc = tick(c, "lm_head")))
    return rc;
  if ((rc = launch_feedback(c->amax_part, c->amax_parts, c->amax, c->params, c->tok_ring, c->ring_cap, st)))
    return rc;
  return tick(c, "argmax_feedback");
}

// One prefill chunk of the A4B recipe (src/engine-a4b.js:465-549
// encodeLayerPre, 550-584 prefill): tokens pf_ids[0..M) at positions p0 ..
// p0 + M - 1 (= the full layers' slots: a prefill starts from an empty
// cache), per layer the q|k(|v) GEMM, head prep of every token with the K/V
// rows into the caches, causal attention per (KV group, token), the o GEMM,
// the attention residual, the MoE half over the M tokens (k_moe_prefill.hip:
// router, top-8, expert-grouped gate/up and down, dense branch, tail).  The
// per-token arithmetic is the decode step's.  Leaves the final-norm input of
// every token in pf_xhl as an f16 hi/lo pair.
int prefill_chunk_a4b(e4b_ctx* c, uint32_t p0, int M) {
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, Lc = k.layers;
  const int64_t MH = (int64_t)M * H;
  hipStream_t st = c->st;
  int rc;
  auto gemm = [&](const Q40Mat& W, const uint16_t* X, int ldx, float* Y, int ks_want = 1) {
    GemmArgs g{};
    g.W = W;
    g.X = X;
    g.M = M;
    g.ldx = ldx;
    g.epi = GEMM_F32;
    g.Y = Y;
    g.ks = q40_gemm_kslices(W.nb, ks_want);
    return launch_q40_gemm(g, st);
  };
  // the o projection's K slices (its 2816 output rows alone give too few
  // workgroups): what q40_gemm_kslices makes of kPfA4bOKs for the layer
  auto ok_slices = [&](const Layer& ly) { return q40_gemm_kslices(QH * ly.hd / 32, kPfA4bOKs); };
  const Q6Mat E = q6_view(c->embd, k.vocab, H);
  if ((rc = launch_embed_rows(E, c->pf_ids, M, sqrtf((float)H), c->pf_h, c->pf_xhl, st)) ||
      (rc = tick(c, "embed_rows")))
    return rc;
  for (int l = 0; l < Lc; ++l) {
    const Layer& ly = c->L[l];
    const int window = ly.global ? 0 : k.window;
    if ((rc = launch_rownorm(c->pf_h, nullptr, nullptr, nullptr, 1.f, ly.attn_norm, c->pf_xn, nullptr, H, k.eps, st,
                             M)) ||
        (rc = tick(c, "norm_rows")) ||
        (rc = gemm(q40_view(ly.qkv, ly.qkv_rows, H), c->pf_xn, H, c->pf_qkv, kPfA4bQkvKs)) ||
        (rc = tick(c, "gemm_qkv")))
      return rc;
    HeadRowsGen hr{};
    hr.qkv = c->pf_qkv;
    hr.ld = ly.qkv_rows;
    hr.qw = ly.q_norm;
    hr.kw = ly.k_norm;
    hr.inv_freq = ly.global ? c->inv_global : c->inv_local;
    hr.kc = ly.kc;
    hr.vc = ly.vc;
    hr.q = c->pf_q;
    hr.qh = QH;
    hr.kvh = ly.kvh;
    hr.hd = ly.hd;
    hr.angles = ly.angles;
    hr.slots = ly.slots;
    hr.window = window;
    hr.keqv = ly.keqv;
    hr.p0 = p0;
    hr.eps = k.eps;
    hr.ks = q40_gemm_kslices(H / 32, kPfA4bQkvKs);
    hr.slice = (int64_t)M * ly.qkv_rows;
    // the matrix-core attention of the prefill (split keys + combine); other
    // head shapes: one workgroup per (KV group, token)
    PrefillAttnArgs pa{};
    pa.q = c->pf_q;
    pa.kc = ly.kc;
    pa.vc = ly.vc;
    pa.out = c->pf_attn;
    pa.M = M;
    pa.qh = QH;
    pa.kvh = ly.kvh;
    pa.slots = ly.slots;
    pa.hd = ly.hd;
    pa.window = window;
    pa.p0 = p0;
    pa.part = c->pf_apart;
    pa.part_bytes = c->pf_apart_bytes;
    const bool mfma_attn = a4b_pf_mfma_attn(ly, QH);
    AttnRowsGen ar{};
    ar.q = c->pf_q;
    ar.kc = ly.kc;
    ar.vc = ly.vc;
    ar.out = c->pf_attn;
    ar.qh = QH;
    ar.kvh = ly.kvh;
    ar.hd = ly.hd;
    ar.slots = ly.slots;
    ar.window = window;
    ar.p0 = p0;
    if ((rc = launch_headprep_rows_gen(hr, M, st)) || (rc = tick(c, "headprep_rows")) ||
        (rc = mfma_attn ? launch_attn_prefill(pa, st) : launch_attn_rows_gen(ar, M, st)) ||
        (rc = tick(c, "attn_rows")) ||
        (rc = gemm(q40_view(ly.o, H, (int64_t)QH * ly.hd), c->pf_attn, QH * ly.hd, c->pf_y, kPfA4bOKs)) ||
        (rc = tick(c, "gemm_o")) ||
        // h1 = h + rms(o) post_attn, in place (o: the sum of the K slices)
        (rc = launch_rownorm(c->pf_h, c->pf_h, c->pf_y, ly.post_attn, 1.f, nullptr, nullptr, nullptr, H, k.eps, st,
                             M, ok_slices(ly), MH)) ||
        (rc = tick(c, "attn_residual_rows")))
      return rc;
    MoeArgs a = c->moe;
    a.h = c->pf_h;
    a.h_out = c->pf_h;  // the tail reads each row before it writes it
    a.attn_o = nullptr;
    a.ffn_norm = ly.ffn_norm;
    a.router_scale = ly.router_scale;
    a.router_mult = 1.0f / sqrtf((float)H);
    a.pre_ffw2 = ly.pre_ffw2;
    a.router_w = ly.router_w;
    a.pes = ly.pes;
    a.dense_gu = q40_view(ly.gu, 2 * (int64_t)k.ffn, H);
    a.exp_gu = q40_view(ly.exp_gu, (int64_t)k.n_experts * 2 * k.expert_ffn, H);
    a.dense_down = q40_view(ly.down, H, k.ffn);
    a.exp_down = q40_view(ly.exp_down, (int64_t)k.n_experts * H, k.expert_ffn);
    a.post_ffw1 = ly.post_ffw1;
    a.post_ffw2 = ly.post_ffw2;
    a.post_ffw = ly.post_ffw;
    a.layer_scale = ly.scale;
    a.eps = k.eps;
    a.H = H;
    a.E = k.n_experts;
    a.FF = k.expert_ffn;
    a.FF2 = k.ffn;
    if ((rc = launch_moe_prefill(a, M, c->pf_mb, st)) || (rc = tick(c, "moe_prefill"))) return rc;
  }
  // final norm as the f16 hi/lo pair of the lm-head input
  if ((rc = launch_rownorm(c->pf_h, nullptr, nullptr, nullptr, 1.f, c->out_norm, c->pf_xhl, c->pf_xhl + MH, H, k.eps,
                           st, M)) ||
      (rc = tick(c, "final_norm_rows")))
    return rc;
  return E4B_OK;
}

// One prefill chunk: tokens pf_ids[0..M) at positions p0 .. p0 + M - 1,
// every layer as batched GEMMs on the matrix cores plus per-token kernels
// (src/engine-a4b.js:465-563 encodeLayerPre / prefill, with the E4B layer
// recipe of record_step).  Leaves the K/V rows of the chunk in the caches and,
// in pf_xhl, the final-norm input of every token as an f16 hi/lo pair.
int prefill_chunk(e4b_ctx* c, uint32_t p0, int M) {
  if (c->cfg.recipe == E4B_RECIPE_A4B) return prefill_chunk_a4b(c, p0, M);
  const e4b_config& k = c->cfg;
  const int H = k.hidden, QH = k.q_heads, KVH = k.kv_heads, HD = k.head_dim, FF = k.ffn, PD = k.ple_dim;
  const int Lc = k.layers;
  const int64_t NP = (int64_t)Lc * PD;
  const int64_t MH = (int64_t)M * H;
  hipStream_t st = c->st;
  int rc;
  auto gemm = [&](const Q40Mat& W, const uint16_t* X, int ldx, int epi, float* Y, uint16_t* Yh, int64_t ff,
                  const float* mul, int64_t mul_ld, int ks) {
    GemmArgs g{};
    g.W = W;
    g.X = X;
    g.M = M;
    g.ldx = ldx;
    g.epi = epi;
    g.Y = Y;
    g.Yh = Yh;
    g.ff = ff;
    g.mul = mul;
    g.mul_ld = mul_ld;
    g.ks = ks;
    return launch_q40_gemm(g, st);
  };
  const Q6Mat E = q6_view(c->embd, k.vocab, H);
  if ((rc = launch_embed_rows(E, c->pf_ids, M, sqrtf((float)H), c->pf_h, c->pf_xhl, st)) ||
      (rc = tick(c, "embed_rows")))
    return rc;
  if (PD) {
    // PLE model projection of the f32 embedding as two f16 GEMMs (hi, lo)
    const Q40Mat Wpm = q40_view(c->ple_proj, NP, H);
    const int64_t slice = (int64_t)M * NP;
    if ((rc = gemm(Wpm, c->pf_xhl, H, GEMM_F32, c->pf_proj, nullptr, 0, nullptr, 0, 1)) ||
        (rc = tick(c, "gemm_ple_model_proj")) ||
        (rc = gemm(Wpm, c->pf_xhl + MH, H, GEMM_F32, c->pf_proj + slice, nullptr, 0, nullptr, 0, 1)) ||
        (rc = tick(c, "gemm_ple_model_proj")) ||
        (rc = launch_ple_prep_rows(c->pf_proj, slice, c->ple_tab, c->ple_norm, c->pf_ids, M, Lc,
                                   1.0f / sqrtf((float)H), c->pf_ple, k.eps, st)) ||
        (rc = tick(c, "ple_prep_rows")))
      return rc;
  }
  // layer 0 input norm
  if ((rc = launch_resnorm_rows(M, c->pf_h, nullptr, 0, 0, nullptr, 1.0f, c->L[0].attn_norm, c->pf_xn, nullptr, H,
                                k.eps, st)) ||
      (rc = tick(c, "resnorm_rows")))
    return rc;
  const int ks_o = q40_gemm_kslices(QH * HD / 32, kPfKsO), ks_d = q40_gemm_kslices(FF / 32, kPfKs);
  const int ks_qkv = q40_gemm_kslices(H / 32, kPfKsQkv), ks_pg = q40_gemm_kslices(H / 32, kPfKsPle);
  for (int l = 0; l < Lc; ++l) {
    const Layer& ly = c->L[l];
    // attention block
    if ((rc = gemm(q40_view(ly.qkv, c->qkv_rows, H), c->pf_xn, H, GEMM_F32, c->pf_qkv, nullptr, 0, nullptr, 0, ks_qkv)) ||
        (rc = tick(c, "gemm_qkv")))
      return rc;
    if ((rc = launch_headprep_rows(c->pf_qkv, ks_qkv, (int64_t)M * c->qkv_rows, ly.q_norm, ly.k_norm, ly.global ? c->inv_global : c->inv_local,
                                   k.rope_angles, ly.kc, ly.vc, ly.slots, !ly.global, p0, M, c->pf_q, QH, KVH, k.eps,
                                   st)) ||
        (rc = tick(c, "headprep_rows")))
      return rc;
    PrefillAttnArgs pa;
    pa.q = c->pf_q;
    pa.kc = ly.kc;
    pa.vc = ly.vc;
    pa.out = c->pf_attn;
    pa.M = M;
    pa.qh = QH;
    pa.kvh = KVH;
    pa.slots = ly.slots;
    pa.window = ly.global ? 0 : k.window;
    pa.p0 = p0;
    pa.part = c->pf_apart;
    pa.part_bytes = c->pf_apart_bytes;
    if ((rc = launch_attn_prefill(pa, st)) || (rc = tick(c, "attn_prefill"))) return rc;
    if ((rc = gemm(q40_view(ly.o, H, (int64_t)QH * HD), c->pf_attn, QH * HD, GEMM_F32, c->pf_y, nullptr, 0, nullptr,
                   0, ks_o)) ||
        (rc = tick(c, "gemm_o")))
      return rc;
    // post-attention residual + FFN norm; gate/up + GeGLU; down
    if ((rc = launch_resnorm_rows(M, c->pf_h, c->pf_y, ks_o, MH, ly.post_attn, 1.0f, ly.ffn_norm, c->pf_xn, nullptr,
                                  H, k.eps, st)) ||
        (rc = tick(c, "resnorm_rows")) ||
        (rc = gemm(q40_view(ly.gu, 2 * (int64_t)FF, H), c->pf_xn, H, GEMM_GLU, nullptr, c->pf_gg, FF, nullptr, 0, 1)) ||
        (rc = tick(c, "gemm_gate_up_geglu")) ||
        (rc = gemm(q40_view(ly.down, H, FF), c->pf_gg, FF, GEMM_F32, c->pf_y, nullptr, 0, nullptr, 0, ks_d)) ||
        (rc = tick(c, "gemm_down")))
      return rc;
    // the last residual of the layer is followed by the next layer's input
    // norm, or after the last layer by the final norm (as an f16 hi/lo
    // split for the lm-head)
    const bool lastl = l + 1 == Lc;
    const float* w_next = lastl ? c->out_norm : c->L[l + 1].attn_norm;
    uint16_t* x_next = lastl ? c->pf_xhl : c->pf_xn;
    uint16_t* xlo_next = lastl ? c->pf_xhl + MH : nullptr;
    if (PD) {
      // post-FFN residual (x = f16(h)); PLE gate * GELU * per-layer input;
      // projection; post-PLE residual and layer scalar
      if ((rc = launch_resnorm_rows(M, c->pf_h, c->pf_y, ks_d, MH, ly.post_ffw, 1.0f, nullptr, c->pf_xn, nullptr, H,
                                    k.eps, st)) ||
          (rc = tick(c, "resnorm_rows")) ||
          (rc = gemm(q40_view(ly.pg, PD, H), c->pf_xn, H, GEMM_F32, c->pf_y, nullptr, 0, nullptr, 0, ks_pg)) ||
          (rc = tick(c, "gemm_ple_gate")) ||
          (rc = launch_gelu_mul_rows(c->pf_y, ks_pg, (int64_t)M * PD, M, PD, c->pf_ple + (int64_t)l * PD, NP, c->pf_gp,
                                     st)) ||
          (rc = tick(c, "gelu_mul_rows")) ||
          (rc = gemm(q40_view(ly.pp_rm, H, PD), c->pf_gp, PD, GEMM_F32, c->pf_y, nullptr, 0, nullptr, 0, 1)) ||
          (rc = tick(c, "gemm_ple_proj")) ||
          (rc = launch_resnorm_rows(M, c->pf_h, c->pf_y, 1, 0, ly.post_norm, ly.scale, w_next, x_next, xlo_next, H,
                                    k.eps, st)) ||
          (rc = tick(c, "resnorm_rows")))
        return rc;
    } else {
      if ((rc = launch_resnorm_rows(M, c->pf_h, c->pf_y, ks_d, MH, ly.post_ffw, ly.scale, w_next, x_next, xlo_next, H,
                                    k.eps, st)) ||
          (rc = tick(c, "resnorm_rows")))
        return rc;
    }
  }
  return E4B_OK;
}

int put_params(e4b_ctx* c, const uint32_t* v, int first, int count);

// batched prefill of ids[0..n) from position 0 in chunks of pf_cap tokens;
// then the lm-head + argmax of the last token, fed back as the next decode
// input exactly as the step's feedback does (params[0] = n, params[1] = token)
int prefill_batched(e4b_ctx* c, const uint32_t* ids, uint32_t n) {
  const e4b_config& k = c->cfg;
  const int H = k.hidden;
  int rc;
  int M = 0;
  for (uint32_t off = 0; off < n; off += (uint32_t)M) {
    M = (int)((n - off) < (uint32_t)c->pf_cap ? (n - off) : (uint32_t)c->pf_cap);
    E4B_HIP(hipMemcpyAsync(c->pf_ids, ids + off, (size_t)M * 4, hipMemcpyHostToDevice, c->st));
    if ((rc = prefill_chunk(c, off, M))) return rc;
  }
  const int64_t MH = (int64_t)M * H, last = (int64_t)(M - 1) * H;
  const Q6Mat E = q6_view(c->embd, k.vocab, H);
  if ((rc = launch_q6k_gemv_argmax(E, (const uint32_t*)(c->pf_xhl + last), (const uint32_t*)(c->pf_xhl + MH + last),
                                   k.softcap, c->logits, nullptr, c->amax_part, c->st)))
    return rc;
  // the feedback advances params[0] and params[4] to n: decode continues at
  // position n, full-layer slot n
  const uint32_t p[5] = {n - 1, 0u, 0u, 0u, n - 1};
  if ((rc = put_params(c, p, 0, 5))) return rc;
  if ((rc = launch_feedback(c->amax_part, c->amax_parts, c->amax, c->params, c->tok_ring, c->ring_cap, c->st)))
    return rc;
  float* hdst = c->h_final ? c->h_final : c->h;
  E4B_HIP(hipMemcpyAsync(hdst, c->pf_h + last, (size_t)H * 4, hipMemcpyDeviceToDevice, c->st));
  return E4B_OK;
}

int ready(e4b_ctx* c, const char* fn) {
  if (!c) return e4b_fail(E4B_EINVAL, "%s: null context", fn);
  if (!c->finalized) return e4b_fail(E4B_ESTATE, "%s before e4b_finalize", fn);
  return E4B_OK;
}

int check_status(e4b_ctx* c) {
  uint32_t s = 0;
  E4B_HIP(hipMemcpyAsync(&s, c->status, 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  if (s) {
    uint32_t z = 0;
    E4B_HIP(hipMemcpy(c->status, &z, 4, hipMemcpyHostToDevice));
    return e4b_fail(E4B_ERANGE, "token id out of range [0, %d)", c->cfg.vocab);
  }
  return E4B_OK;
}

// one token: replay the captured graph, or launch the kernels directly
int launch_token(e4b_ctx* c) {
  if (c->exec) {
    E4B_HIP(hipGraphLaunch(c->exec, c->st));
    return E4B_OK;
  }
  return record_step(c);
}

int put_params(e4b_ctx* c, const uint32_t* v, int first, int count) {
  E4B_HIP(hipMemcpyAsync(c->params + first, v, (size_t)count * 4, hipMemcpyHostToDevice, c->st));
  return E4B_OK;
}

int zero_scores(e4b_ctx* c) {
  for (const Layer& ly : c->L)
    if (ly.score) E4B_HIP(hipMemsetAsync(ly.score, 0, (size_t)c->cfg.q_heads * ly.slots * 4, c->st));
  return E4B_OK;
}

}  // namespace

extern "C" int e4b_step(e4b_ctx* c, uint32_t token, uint32_t pos, float* logits, uint32_t* argmax_out) {
  int rc = ready(c, "e4b_step");
  if (rc) return rc;
  if (token >= (uint32_t)c->cfg.vocab) return e4b_fail(E4B_ERANGE, "e4b_step: token %u >= vocab %d", token, c->cfg.vocab);
  // positions only rotate q/k and index the sliding rings (modulo); the full
  // layers' limit is their entry count
  if (pos >= 0x7fffffffu) return e4b_fail(E4B_ERANGE, "e4b_step: pos %u >= 2^31 - 1", pos);
  const uint32_t kv = pos == 0 ? 0u : c->kv_count;  // src/engine-a4b.js:695-699
  if (kv >= (uint32_t)c->cfg.max_seq)
    return e4b_fail(E4B_ERANGE, "e4b_step: %u full-layer entries fill max_seq %d (compact first)", kv, c->cfg.max_seq);
  const uint32_t p[5] = {pos, token, 0u, 0u, kv};
  if ((rc = put_params(c, p, 0, 5)) || (rc = launch_token(c))) return rc;
  c->kv_count = kv + 1;
  uint32_t am[2] = {0, 0};
  E4B_HIP(hipMemcpyAsync(am, c->amax, 8, hipMemcpyDeviceToHost, c->st));
  if (logits) E4B_HIP(hipMemcpyAsync(logits, c->logits, (size_t)c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->st));
  if ((rc = check_status(c))) return rc;
  if (argmax_out) *argmax_out = am[0];
  return E4B_OK;
}

static int prefill_common(e4b_ctx* c, const char* fn, const uint32_t* ids, uint32_t n, uint32_t* argmax_out,
                          bool steps) {
  int rc = ready(c, fn);
  if (rc) return rc;
  if (!ids || n == 0) return e4b_fail(E4B_EINVAL, "%s: empty prompt", fn);
  if (n > (uint32_t)c->max_prompt || n > (uint32_t)c->cfg.max_seq)
    return e4b_fail(E4B_ERANGE, "%s: %u tokens exceeds the prompt capacity %d", fn, n, c->max_prompt);
  for (uint32_t i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)c->cfg.vocab) return e4b_fail(E4B_ERANGE, "%s: ids[%u] = %u >= vocab", fn, i, ids[i]);
  if (steps) {
    E4B_HIP(hipMemcpyAsync(c->prompt, ids, (size_t)n * 4, hipMemcpyHostToDevice, c->st));
    const uint32_t p[5] = {0u, 0u, 0u, n, 0u};
    if ((rc = put_params(c, p, 0, 5))) return rc;
    for (uint32_t i = 0; i < n; ++i)
      if ((rc = launch_token(c))) return rc;
  } else if ((rc = prefill_batched(c, ids, n))) {
    return rc;
  }
  // the full layers hold the n prompt entries; the prefill leaves no mass
  // (src/engine-a4b.js:555-563: scores zeroed, batched attention unscored)
  c->kv_count = n;
  if ((rc = zero_scores(c))) return rc;
  uint32_t am[2] = {0, 0};
  E4B_HIP(hipMemcpyAsync(am, c->amax, 8, hipMemcpyDeviceToHost, c->st));
  if ((rc = check_status(c))) return rc;
  if (argmax_out) *argmax_out = am[0];
  return E4B_OK;
}

extern "C" int e4b_prefill(e4b_ctx* c, const uint32_t* ids, uint32_t n, uint32_t* argmax_out) {
  return prefill_common(c, "e4b_prefill", ids, n, argmax_out,
                        c && ((c->cfg.flags & E4B_FLAG_STEP_PREFILL) != 0 || c->pf_cap <= 0));
}

extern "C" int e4b_prefill_steps(e4b_ctx* c, const uint32_t* ids, uint32_t n, uint32_t* argmax_out) {
  return prefill_common(c, "e4b_prefill_steps", ids, n, argmax_out, true);
}

static int decode_launch(e4b_ctx* c, uint32_t start_pos, uint32_t count) {
  if ((uint64_t)start_pos + count >= 0x7fffffffu)
    return e4b_fail(E4B_ERANGE, "decode: positions [%u, %u) reach 2^31 - 1", start_pos, start_pos + count);
  if (count > (uint32_t)c->ring_cap) return e4b_fail(E4B_ERANGE, "decode: %u tokens exceed the token ring", count);
  if ((uint64_t)c->kv_count + count > (uint64_t)c->cfg.max_seq)
    return e4b_fail(E4B_ERANGE, "decode: %u full-layer entries + %u exceed max_seq %d (compact first)", c->kv_count,
                    count, c->cfg.max_seq);
  // the entry count continues from the last step (decodeChunk,
  // src/engine-a4b.js:786-795); the feedback advances it with the position
  const uint32_t p0 = start_pos, z[3] = {0u, 0u, c->kv_count};
  int rc;
  if ((rc = put_params(c, &p0, 0, 1)) || (rc = put_params(c, z, 2, 3))) return rc;
  for (uint32_t i = 0; i < count; ++i)
    if ((rc = launch_token(c))) return rc;
  c->kv_count += count;
  return E4B_OK;
}

extern "C" int e4b_decode(e4b_ctx* c, uint32_t start_pos, uint32_t count, uint32_t* tokens_out) {
  int rc = ready(c, "e4b_decode");
  if (rc) return rc;
  if (count == 0) return E4B_OK;
  if (!tokens_out) return e4b_fail(E4B_EINVAL, "e4b_decode: null tokens_out");
  if ((rc = decode_launch(c, start_pos, count))) return rc;
  E4B_HIP(hipMemcpyAsync(tokens_out, c->tok_ring, (size_t)count * 4, hipMemcpyDeviceToHost, c->st));
  return check_status(c);
}

extern "C" int e4b_time_decode(e4b_ctx* c, uint32_t start_pos, uint32_t count, float* ms_out) {
  int rc = ready(c, "e4b_time_decode");
  if (rc) return rc;
  if (!ms_out) return e4b_fail(E4B_EINVAL, "e4b_time_decode: null ms_out");
  hipEvent_t a, b;
  E4B_HIP(hipEventCreate(&a));
  E4B_HIP(hipEventCreate(&b));
  E4B_HIP(hipEventRecord(a, c->st));
  rc = decode_launch(c, start_pos, count);
  if (rc == E4B_OK) {
    E4B_HIP(hipEventRecord(b, c->st));
    E4B_HIP(hipEventSynchronize(b));
    E4B_HIP(hipEventElapsedTime(ms_out, a, b));
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return rc ? rc : check_status(c);
}

// ---- per-dispatch profiles (profileStep / profilePrefill) -----------------------
namespace {

// run `body` with a mark before it and after each of its launches, then sum
// the times between consecutive marks per label, labels in order of first use
template <typename F>
int profile_run(e4b_ctx* c, e4b_prof_entry* out, int cap, F body) {
  if (cap < 0 || (cap > 0 && !out)) return e4b_fail(E4B_EINVAL, "profile: bad output array");
  E4B_HIP(hipStreamSynchronize(c->st));
  c->prof_label.clear();
  c->prof_on = true;
  int rc = tick(c, nullptr);
  if (rc == E4B_OK) rc = body();
  c->prof_on = false;
  if (rc) return rc;
  E4B_HIP(hipStreamSynchronize(c->st));
  std::vector<std::string> names;
  std::vector<double> us;
  std::vector<int> cnt;
  for (size_t i = 1; i < c->prof_label.size(); ++i) {
    float ms = 0.f;
    E4B_HIP(hipEventElapsedTime(&ms, c->prof_ev[i - 1], c->prof_ev[i]));
    const std::string nm(c->prof_label[i]);
    size_t j = 0;
    while (j < names.size() && names[j] != nm) ++j;
    if (j == names.size()) {
      names.push_back(nm);
      us.push_back(0.0);
      cnt.push_back(0);
    }
    us[j] += 1000.0 * ms;
    cnt[j] += 1;
  }
  for (size_t j = 0; j < names.size() && (int)j < cap; ++j) {
    memset(out[j].name, 0, sizeof(out[j].name));
    strncpy(out[j].name, names[j].c_str(), sizeof(out[j].name) - 1);
    out[j].us = (float)us[j];
    out[j].n = cnt[j];
  }
  return (int)names.size();
}

}  // namespace

extern "C" int e4b_profile_step(e4b_ctx* c, uint32_t token, uint32_t pos, e4b_prof_entry* out, int cap) {
  int rc = ready(c, "e4b_profile_step");
  if (rc) return rc;
  if (token >= (uint32_t)c->cfg.vocab)
    return e4b_fail(E4B_ERANGE, "e4b_profile_step: token %u >= vocab %d", token, c->cfg.vocab);
  if (pos >= 0x7fffffffu) return e4b_fail(E4B_ERANGE, "e4b_profile_step: pos %u >= 2^31 - 1", pos);
  const uint32_t kv = pos == 0 ? 0u : c->kv_count;
  if (kv >= (uint32_t)c->cfg.max_seq)
    return e4b_fail(E4B_ERANGE, "e4b_profile_step: %u full-layer entries fill max_seq %d", kv, c->cfg.max_seq);
  const uint32_t p[5] = {pos, token, 0u, 0u, kv};
  if ((rc = put_params(c, p, 0, 5))) return rc;
  int n = profile_run(c, out, cap, [&]() { return record_step(c); });
  if (n < 0) return n;
  c->kv_count = kv + 1;
  if ((rc = check_status(c))) return rc;
  return n;
}

extern "C" int e4b_profile_prefill(e4b_ctx* c, const uint32_t* ids, uint32_t n, e4b_prof_entry* out, int cap) {
  int rc = ready(c, "e4b_profile_prefill");
  if (rc) return rc;
  if (!ids || n == 0) return e4b_fail(E4B_EINVAL, "e4b_profile_prefill: empty prompt");
  if (c->pf_cap <= 0)
    return e4b_fail(E4B_ESTATE, "e4b_profile_prefill: no batched prefill buffers (max_prompt, max_seq or the ring "
                                "leave no chunk); profile the step with e4b_profile_step");
  const int M = (int)(n < (uint32_t)c->pf_cap ? n : (uint32_t)c->pf_cap);
  for (int i = 0; i < M; ++i)
    if (ids[i] >= (uint32_t)c->cfg.vocab)
      return e4b_fail(E4B_ERANGE, "e4b_profile_prefill: ids[%d] = %u >= vocab", i, ids[i]);
  E4B_HIP(hipMemcpyAsync(c->pf_ids, ids, (size_t)M * 4, hipMemcpyHostToDevice, c->st));
  const int cnt = profile_run(c, out, cap, [&]() { return prefill_chunk(c, 0, M); });
  if (cnt < 0) return cnt;
  c->kv_count = (uint32_t)M;
  return cnt;
}

extern "C" int e4b_argmax(e4b_ctx* c, uint32_t* token_out) {
  int rc = ready(c, "e4b_argmax");
  if (rc) return rc;
  if (!token_out) return e4b_fail(E4B_EINVAL, "e4b_argmax: null");
  uint32_t am[2];
  E4B_HIP(hipMemcpyAsync(am, c->amax, 8, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  *token_out = am[0];
  return E4B_OK;
}

extern "C" int e4b_read_hidden(e4b_ctx* c, float* out) {
  int rc = ready(c, "e4b_read_hidden");
  if (rc) return rc;
  E4B_HIP(hipMemcpyAsync(out, c->h_final ? c->h_final : c->h, (size_t)c->cfg.hidden * 4, hipMemcpyDeviceToHost,
                         c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_read_layer_hidden(e4b_ctx* c, int layer, float* out) {
  int rc = ready(c, "e4b_read_layer_hidden");
  if (rc) return rc;
  if (!out) return e4b_fail(E4B_EINVAL, "e4b_read_layer_hidden: null output");
  if (layer < 0 || layer >= c->cfg.layers)
    return e4b_fail(E4B_ERANGE, "e4b_read_layer_hidden: layer %d of %d", layer, c->cfg.layers);
  if (!c->lh && layer < c->cfg.layers - 1)
    return e4b_fail(E4B_ESTATE, "e4b_read_layer_hidden: the engine was created without E4B_FLAG_LAYER_HIDDEN");
  const float* src = layer == c->cfg.layers - 1 ? (c->h_final ? c->h_final : c->h) : c->lh + (size_t)layer * c->cfg.hidden;
  E4B_HIP(hipMemcpyAsync(out, src, (size_t)c->cfg.hidden * 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_read_topk(e4b_ctx* c, int layer, uint32_t* idx, float* w) {
  int rc = ready(c, "e4b_read_topk");
  if (rc) return rc;
  if (c->cfg.recipe != E4B_RECIPE_A4B) return e4b_fail(E4B_EINVAL, "e4b_read_topk: the E4B recipe has no experts");
  if (!idx || !w) return e4b_fail(E4B_EINVAL, "e4b_read_topk: null output");
  if (layer < 0 || layer >= c->cfg.layers)
    return e4b_fail(E4B_ERANGE, "e4b_read_topk: layer %d of %d", layer, c->cfg.layers);
  E4B_HIP(hipMemcpyAsync(idx, c->moe.topk_idx + (size_t)kMoeTopK * layer, kMoeTopK * 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipMemcpyAsync(w, c->moe.topk_w + (size_t)kMoeTopK * layer, kMoeTopK * 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_read_logits(e4b_ctx* c, float* out) {
  int rc = ready(c, "e4b_read_logits");
  if (rc) return rc;
  E4B_HIP(hipMemcpyAsync(out, c->logits, (size_t)c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_kv_slots(e4b_ctx* c, int layer) {
  int rc = ready(c, "e4b_kv_slots");
  if (rc) return rc;
  if (layer < 0 || layer >= c->cfg.layers) return e4b_fail(E4B_EINVAL, "layer %d", layer);
  return c->L[layer].slots;
}

extern "C" int e4b_read_kv(e4b_ctx* c, int layer, uint16_t* k_out, uint16_t* v_out) {
  int rc = ready(c, "e4b_read_kv");
  if (rc) return rc;
  if (layer < 0 || layer >= c->cfg.layers) return e4b_fail(E4B_EINVAL, "layer %d", layer);
  const Layer& ly = c->L[layer];
  const size_t n = (size_t)ly.kvh * ly.slots * ly.hd * 2;
  if (k_out) E4B_HIP(hipMemcpyAsync(k_out, ly.kc, n, hipMemcpyDeviceToHost, c->st));
  if (v_out) E4B_HIP(hipMemcpyAsync(v_out, ly.vc, n, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_reset(e4b_ctx* c) {
  int rc = ready(c, "e4b_reset");
  if (rc) return rc;
  for (const Layer& ly : c->L) {
    const size_t n = (size_t)ly.kvh * ly.slots * ly.hd * 2;
    E4B_HIP(hipMemsetAsync(ly.kc, 0, n, c->st));
    E4B_HIP(hipMemsetAsync(ly.vc, 0, n, c->st));
  }
  E4B_HIP(hipMemsetAsync(c->params, 0, 16 * 4, c->st));
  E4B_HIP(hipMemsetAsync(c->status, 0, 4 * 4, c->st));
  E4B_HIP(hipMemsetAsync(c->amax, 0, 4 * 4, c->st));
  if ((rc = zero_scores(c))) return rc;
  c->kv_count = 0;
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_kv_count(e4b_ctx* c) {
  int rc = ready(c, "e4b_kv_count");
  if (rc) return rc;
  return (int)c->kv_count;
}

extern "C" int e4b_read_scores(e4b_ctx* c, int layer, float* out) {
  int rc = ready(c, "e4b_read_scores");
  if (rc) return rc;
  if (layer < 0 || layer >= c->cfg.layers) return e4b_fail(E4B_EINVAL, "e4b_read_scores: layer %d", layer);
  const Layer& ly = c->L[layer];
  if (!ly.score)
    return e4b_fail(E4B_ESTATE, "e4b_read_scores: layer %d keeps no scores (a full layer with E4B_FLAG_KV_SCORE)",
                    layer);
  if (!out) return e4b_fail(E4B_EINVAL, "e4b_read_scores: null output");
  E4B_HIP(hipMemcpyAsync(out, ly.score, (size_t)c->cfg.q_heads * ly.slots * 4, hipMemcpyDeviceToHost, c->st));
  E4B_HIP(hipStreamSynchronize(c->st));
  return E4B_OK;
}

extern "C" int e4b_kv_compact(e4b_ctx* c, int budget, int protect) {
  int rc = ready(c, "e4b_kv_compact");
  if (rc) return rc;
  if (!(c->cfg.flags & E4B_FLAG_KV_SCORE))
    return e4b_fail(E4B_ESTATE, "e4b_kv_compact: the context was created without E4B_FLAG_KV_SCORE");
  if (budget < 0 || protect < 0) return e4b_fail(E4B_EINVAL, "e4b_kv_compact: budget %d, protect %d", budget, protect);
  const int QH = c->cfg.q_heads;
  const int64_t n = c->kv_count;
  std::vector<float> sc;
  std::vector<uint32_t> keep((size_t)std::max<int64_t>(n, 1));
  E4B_HIP(hipStreamSynchronize(c->st));
  for (Layer& ly : c->L) {
    if (!ly.global) continue;
    sc.resize((size_t)QH * ly.slots);
    E4B_HIP(hipMemcpy(sc.data(), ly.score, sc.size() * 4, hipMemcpyDeviceToHost));
    const int64_t sel = e4b_kv_select(sc.data(), QH, ly.slots, n, budget, protect, keep.data());
    if (sel < 0) return (int)sel;
    const int cnt = (int)sel;
    if (cnt > 0) {
      E4B_HIP(hipMemcpyAsync(c->keep, keep.data(), (size_t)cnt * 4, hipMemcpyHostToDevice, c->st));
      const int KVH = ly.kvh, HD = ly.hd;
      if ((rc = HD == 256 ? launch_kv_gather(c->keep, cnt, ly.kc, ly.vc, KVH, ly.slots, c->kv_sk, c->kv_sv, ly.slots,
                                             c->st)
                          : launch_kv_gather_gen(c->keep, cnt, ly.kc, ly.vc, KVH, ly.slots, HD, c->kv_sk, c->kv_sv,
                                                 ly.slots, c->st)))
        return rc;
      // rows [0, cnt) of every head back into the cache
      for (int g = 0; g < KVH; ++g) {
        const size_t off = (size_t)g * ly.slots * HD, bytes = (size_t)cnt * HD * 2;
        E4B_HIP(hipMemcpyAsync(ly.kc + off, c->kv_sk + off, bytes, hipMemcpyDeviceToDevice, c->st));
        E4B_HIP(hipMemcpyAsync(ly.vc + off, c->kv_sv + off, bytes, hipMemcpyDeviceToDevice, c->st));
      }
    }
    E4B_HIP(hipMemsetAsync(ly.score, 0, sc.size() * 4, c->st));
    // keep is the host vector the copies read: finish before its next use
    E4B_HIP(hipStreamSynchronize(c->st));
    c->kv_count = (uint32_t)cnt;
  }
  return (int)c->kv_count;
}

extern "C" void e4b_destroy(e4b_ctx* c) {
  if (!c) return;
  if (c->st) (void)hipStreamSynchronize(c->st);
  if (c->exec) (void)hipGraphExecDestroy(c->exec);
  if (c->graph) (void)hipGraphDestroy(c->graph);
  for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
  for (void* p : c->allocs) (void)hipFree(p);
  if (c->st) (void)hipStreamDestroy(c->st);
  delete c;
}
