// e4b_napi.cc -- N-API addon: the JS host's binding of libe4b.so's engine ABI
// (include/e4b.h).  It replaces the WebGPU calls the reference's engine object
// makes (src/gpu.js:4-113 initDevice / upload / readback, driven by
// src/engine-a4b.js) with calls into the HIP library; engine.js builds the
// reference's engine surface (step, argmaxFast, decodeChunk, generateFast,
// prefill, readHidden) on top of it.
//
// Every function throws a JS Error carrying e4b_last_error() when the library
// returns a negative status, as the reference's engine throws on a missing
// tensor or a capacity overflow (src/gguf.js:76, src/engine-a4b.js:560).
// Contexts are external values; their finalizer destroys the context.
#define NAPI_VERSION 4
#include <node_api.h>

#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/e4b.h"

namespace {

#define CHECK_NAPI(call)                                   \
  do {                                                     \
    if ((call) != napi_ok) {                               \
      napi_throw_error(env, nullptr, "N-API call failed"); \
      return nullptr;                                      \
    }                                                      \
  } while (0)

napi_value throw_lib(napi_env env, const char* where, int rc) {
  std::string msg = std::string(where) + ": error " + std::to_string(rc) + ": " + e4b_last_error();
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

napi_value throw_msg(napi_env env, const char* msg) {
  napi_throw_type_error(env, nullptr, msg);
  return nullptr;
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return true;
}

bool get_i64(napi_env env, napi_value v, int64_t* out) { return napi_get_value_int64(env, v, out) == napi_ok; }
bool get_f64(napi_env env, napi_value v, double* out) { return napi_get_value_double(env, v, out) == napi_ok; }

// bytes of a TypedArray, DataView, Buffer or ArrayBuffer
bool get_bytes(napi_env env, napi_value v, const void** data, size_t* len) {
  bool is = false;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type t;
    size_t n = 0, off = 0;
    napi_value ab;
    void* d = nullptr;
    if (napi_get_typedarray_info(env, v, &t, &n, &d, &ab, &off) != napi_ok) return false;
    size_t es = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: es = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
      default: es = 1;
    }
    *data = d;
    *len = n * es;
    return true;
  }
  if (napi_is_dataview(env, v, &is) == napi_ok && is) {
    void* d = nullptr;
    napi_value ab;
    size_t off = 0;
    if (napi_get_dataview_info(env, v, len, &d, &ab, &off) != napi_ok) return false;
    *data = d;
    return true;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) {
    void* d = nullptr;
    if (napi_get_arraybuffer_info(env, v, &d, len) != napi_ok) return false;
    *data = d;
    return true;
  }
  return false;
}

napi_value make_typed(napi_env env, napi_typedarray_type t, size_t count, size_t es, void** data) {
  napi_value ab, arr;
  if (napi_create_arraybuffer(env, count * es, data, &ab) != napi_ok) return nullptr;
  if (napi_create_typedarray(env, t, count, ab, 0, &arr) != napi_ok) return nullptr;
  return arr;
}

struct Ctx {
  e4b_ctx* c;
  int32_t vocab, hidden, q_heads, max_seq;
};

void finalize_ctx(napi_env, void* data, void*) {
  Ctx* x = static_cast<Ctx*>(data);
  if (x->c) e4b_destroy(x->c);
  delete x;
}

Ctx* ctx_of(napi_env env, napi_value v) {
  void* p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) return nullptr;
  Ctx* x = static_cast<Ctx*>(p);
  return x->c ? x : nullptr;
}

// ---- library ------------------------------------------------------------------
napi_value version(napi_env env, napi_callback_info) {
  napi_value s;
  CHECK_NAPI(napi_create_string_utf8(env, e4b_version(), NAPI_AUTO_LENGTH, &s));
  return s;
}

napi_value last_error(napi_env env, napi_callback_info) {
  napi_value s;
  CHECK_NAPI(napi_create_string_utf8(env, e4b_last_error(), NAPI_AUTO_LENGTH, &s));
  return s;
}

napi_value device_count(napi_env env, napi_callback_info) {
  int n = 0;
  const int rc = e4b_device_count(&n);
  if (rc) return throw_lib(env, "deviceCount", rc);
  napi_value v;
  CHECK_NAPI(napi_create_int32(env, n, &v));
  return v;
}

// ---- engine -------------------------------------------------------------------
// create({hidden, layers, ..., layerGlobal: [0/1...]}) -> ctx
napi_value create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return throw_msg(env, "create(config)");
  e4b_config cfg;
  memset(&cfg, 0, sizeof(cfg));
  struct IntField {
    const char* name;
    int32_t* dst;
  } ints[] = {{"hidden", &cfg.hidden}, {"layers", &cfg.layers}, {"qHeads", &cfg.q_heads},
              {"kvHeads", &cfg.kv_heads}, {"headDim", &cfg.head_dim}, {"ffn", &cfg.ffn},
              {"pleDim", &cfg.ple_dim}, {"vocab", &cfg.vocab}, {"window", &cfg.window},
              {"ring", &cfg.ring}, {"maxSeq", &cfg.max_seq}, {"ropeAngles", &cfg.rope_angles},
              {"attnChunk", &cfg.attn_chunk}, {"maxPrompt", &cfg.max_prompt}, {"recipe", &cfg.recipe},
              {"headDimFull", &cfg.head_dim_full}, {"ropeAnglesFull", &cfg.rope_angles_full},
              {"nExperts", &cfg.n_experts}, {"expertFfn", &cfg.expert_ffn}};
  for (const IntField& f : ints) {
    napi_value v;
    bool has = false;
    CHECK_NAPI(napi_has_named_property(env, argv[0], f.name, &has));
    if (!has) continue;
    CHECK_NAPI(napi_get_named_property(env, argv[0], f.name, &v));
    int64_t x = 0;
    if (!get_i64(env, v, &x)) return throw_msg(env, "create: integer config field expected");
    *f.dst = (int32_t)x;
  }
  struct FloatField {
    const char* name;
    float* dst;
  } flts[] = {{"thetaLocal", &cfg.theta_local}, {"thetaGlobal", &cfg.theta_global}, {"eps", &cfg.eps},
              {"softcap", &cfg.softcap}};
  for (const FloatField& f : flts) {
    napi_value v;
    bool has = false;
    CHECK_NAPI(napi_has_named_property(env, argv[0], f.name, &has));
    if (!has) continue;
    CHECK_NAPI(napi_get_named_property(env, argv[0], f.name, &v));
    double x = 0;
    if (!get_f64(env, v, &x)) return throw_msg(env, "create: numeric config field expected");
    *f.dst = (float)x;
  }
  {
    napi_value v;
    bool has = false;
    CHECK_NAPI(napi_has_named_property(env, argv[0], "flags", &has));
    if (has) {
      CHECK_NAPI(napi_get_named_property(env, argv[0], "flags", &v));
      int64_t x = 0;
      if (!get_i64(env, v, &x)) return throw_msg(env, "create: flags must be an integer");
      cfg.flags = (uint32_t)x;
    }
  }
  std::vector<uint8_t> lg;
  {
    bool has = false;
    CHECK_NAPI(napi_has_named_property(env, argv[0], "layerGlobal", &has));
    if (has) {
      napi_value arr;
      CHECK_NAPI(napi_get_named_property(env, argv[0], "layerGlobal", &arr));
      uint32_t n = 0;
      if (napi_get_array_length(env, arr, &n) != napi_ok) return throw_msg(env, "create: layerGlobal must be an array");
      lg.resize(n);
      for (uint32_t i = 0; i < n; ++i) {
        napi_value e;
        CHECK_NAPI(napi_get_element(env, arr, i, &e));
        int64_t x = 0;
        if (!get_i64(env, e, &x)) return throw_msg(env, "create: layerGlobal entries must be 0/1");
        lg[i] = x ? 1 : 0;
      }
      if ((int32_t)n != cfg.layers) return throw_msg(env, "create: layerGlobal length must equal layers");
      cfg.layer_global = lg.data();
    }
  }
  std::vector<int32_t> kvh;  // KV heads per layer (the A4B recipe)
  {
    bool has = false;
    CHECK_NAPI(napi_has_named_property(env, argv[0], "layerKvHeads", &has));
    if (has) {
      napi_value arr;
      CHECK_NAPI(napi_get_named_property(env, argv[0], "layerKvHeads", &arr));
      uint32_t n = 0;
      if (napi_get_array_length(env, arr, &n) != napi_ok) return throw_msg(env, "create: layerKvHeads must be an array");
      kvh.resize(n);
      for (uint32_t i = 0; i < n; ++i) {
        napi_value e;
        CHECK_NAPI(napi_get_element(env, arr, i, &e));
        int64_t x = 0;
        if (!get_i64(env, e, &x)) return throw_msg(env, "create: layerKvHeads entries must be integers");
        kvh[i] = (int32_t)x;
      }
      if ((int32_t)n != cfg.layers) return throw_msg(env, "create: layerKvHeads length must equal layers");
      cfg.layer_kv_heads = kvh.data();
    }
  }
  e4b_ctx* c = e4b_create(&cfg);  // copies the config (and the per-layer arrays)
  if (!c) return throw_lib(env, "create", -1);
  Ctx* x = new Ctx{c, cfg.vocab, cfg.hidden, cfg.q_heads, cfg.max_seq};
  napi_value ext;
  if (napi_create_external(env, x, finalize_ctx, nullptr, &ext) != napi_ok) {
    e4b_destroy(c);
    delete x;
    return throw_msg(env, "create: napi_create_external failed");
  }
  return ext;
}

// setTensor(ctx, name, ggmlType, dims[], bytes)
napi_value set_tensor(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return throw_msg(env, "setTensor(ctx, name, type, dims, bytes)");
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "setTensor: not an engine context");
  char name[256];
  size_t nl = 0;
  if (napi_get_value_string_utf8(env, argv[1], name, sizeof(name), &nl) != napi_ok)
    return throw_msg(env, "setTensor: name must be a string");
  int64_t type = 0;
  if (!get_i64(env, argv[2], &type)) return throw_msg(env, "setTensor: type must be an integer");
  uint32_t nd = 0;
  if (napi_get_array_length(env, argv[3], &nd) != napi_ok || nd > 4) return throw_msg(env, "setTensor: dims array");
  int64_t dims[4] = {0, 0, 0, 0};
  for (uint32_t i = 0; i < nd; ++i) {
    napi_value e;
    CHECK_NAPI(napi_get_element(env, argv[3], i, &e));
    double d = 0;
    if (!get_f64(env, e, &d)) return throw_msg(env, "setTensor: dims must be numbers");
    dims[i] = (int64_t)d;
  }
  const void* data = nullptr;
  size_t len = 0;
  if (!get_bytes(env, argv[4], &data, &len)) return throw_msg(env, "setTensor: bytes must be a TypedArray or ArrayBuffer");
  const int rc = e4b_set_tensor(x->c, name, (int)type, dims, (int)nd, data, len);
  if (rc) return throw_lib(env, "setTensor", rc);
  return nullptr;
}

napi_value finalize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "finalize: not an engine context");
  const int rc = e4b_finalize(x->c);
  if (rc) return throw_lib(env, "finalize", rc);
  return nullptr;
}

// step(ctx, token, pos, wantLogits) -> {argmax, logits?}
napi_value step(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  get_args(env, info, 4, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "step: not an engine context");
  int64_t tok = 0, pos = 0;
  if (!get_i64(env, argv[1], &tok) || !get_i64(env, argv[2], &pos) || tok < 0 || pos < 0)
    return throw_msg(env, "step(ctx, token, pos, wantLogits)");
  bool want = false;
  napi_get_value_bool(env, argv[3], &want);
  void* lg = nullptr;
  napi_value logits = nullptr;
  if (want) {
    logits = make_typed(env, napi_float32_array, (size_t)x->vocab, 4, &lg);
    if (!logits) return throw_msg(env, "step: cannot allocate logits");
  }
  uint32_t am = 0;
  const int rc = e4b_step(x->c, (uint32_t)tok, (uint32_t)pos, (float*)lg, &am);
  if (rc) return throw_lib(env, "step", rc);
  napi_value out, a;
  CHECK_NAPI(napi_create_object(env, &out));
  CHECK_NAPI(napi_create_uint32(env, am, &a));
  CHECK_NAPI(napi_set_named_property(env, out, "argmax", a));
  if (logits) CHECK_NAPI(napi_set_named_property(env, out, "logits", logits));
  return out;
}

// a Uint32Array argument as (data, length)
bool get_u32s(napi_env env, napi_value v, const uint32_t** data, size_t* n) {
  napi_typedarray_type t;
  size_t off = 0;
  void* d = nullptr;
  napi_value ab;
  bool is = false;
  if (napi_is_typedarray(env, v, &is) != napi_ok || !is ||
      napi_get_typedarray_info(env, v, &t, n, &d, &ab, &off) != napi_ok || t != napi_uint32_array)
    return false;
  *data = (const uint32_t*)d;
  return true;
}

// prefill(ctx, Uint32Array ids) -> argmax: the batched prefill;
// prefillSteps(ctx, Uint32Array ids) -> argmax: token by token through the step
napi_value prefill_impl(napi_env env, napi_callback_info info, bool steps) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "prefill: not an engine context");
  const uint32_t* d = nullptr;
  size_t n = 0;
  if (!get_u32s(env, argv[1], &d, &n)) return throw_msg(env, "prefill(ctx, Uint32Array ids)");
  uint32_t am = 0;
  const int rc = steps ? e4b_prefill_steps(x->c, d, (uint32_t)n, &am) : e4b_prefill(x->c, d, (uint32_t)n, &am);
  if (rc) return throw_lib(env, steps ? "prefillSteps" : "prefill", rc);
  napi_value v;
  CHECK_NAPI(napi_create_uint32(env, am, &v));
  return v;
}
napi_value prefill(napi_env env, napi_callback_info info) { return prefill_impl(env, info, false); }
napi_value prefill_steps(napi_env env, napi_callback_info info) { return prefill_impl(env, info, true); }

// the library's per-role profile entries as [{name, us, n}, ...]
napi_value prof_array(napi_env env, const e4b_prof_entry* e, int n) {
  napi_value arr;
  CHECK_NAPI(napi_create_array_with_length(env, (size_t)n, &arr));
  for (int i = 0; i < n; ++i) {
    napi_value o, nm, us, cnt;
    CHECK_NAPI(napi_create_object(env, &o));
    CHECK_NAPI(napi_create_string_utf8(env, e[i].name, NAPI_AUTO_LENGTH, &nm));
    CHECK_NAPI(napi_create_double(env, (double)e[i].us, &us));
    CHECK_NAPI(napi_create_int32(env, e[i].n, &cnt));
    CHECK_NAPI(napi_set_named_property(env, o, "name", nm));
    CHECK_NAPI(napi_set_named_property(env, o, "us", us));
    CHECK_NAPI(napi_set_named_property(env, o, "n", cnt));
    CHECK_NAPI(napi_set_element(env, arr, (uint32_t)i, o));
  }
  return arr;
}

// profileStep(ctx, token, pos) -> [{name, us, n}]
napi_value profile_step(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  get_args(env, info, 3, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "profileStep: not an engine context");
  int64_t tok = 0, pos = 0;
  if (!get_i64(env, argv[1], &tok) || !get_i64(env, argv[2], &pos) || tok < 0 || pos < 0)
    return throw_msg(env, "profileStep(ctx, token, pos)");
  e4b_prof_entry e[64];
  const int n = e4b_profile_step(x->c, (uint32_t)tok, (uint32_t)pos, e, 64);
  if (n < 0) return throw_lib(env, "profileStep", n);
  return prof_array(env, e, n < 64 ? n : 64);
}

// profilePrefill(ctx, Uint32Array ids) -> [{name, us, n}]
napi_value profile_prefill(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "profilePrefill: not an engine context");
  const uint32_t* d = nullptr;
  size_t len = 0;
  if (!get_u32s(env, argv[1], &d, &len)) return throw_msg(env, "profilePrefill(ctx, Uint32Array ids)");
  e4b_prof_entry e[64];
  const int n = e4b_profile_prefill(x->c, d, (uint32_t)len, e, 64);
  if (n < 0) return throw_lib(env, "profilePrefill", n);
  return prof_array(env, e, n < 64 ? n : 64);
}

// decode(ctx, startPos, count) -> Uint32Array tokens
napi_value decode(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  get_args(env, info, 3, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "decode: not an engine context");
  int64_t start = 0, count = 0;
  if (!get_i64(env, argv[1], &start) || !get_i64(env, argv[2], &count) || start < 0 || count < 0 || count > (1 << 24))
    return throw_msg(env, "decode(ctx, startPos, count)");
  void* d = nullptr;
  napi_value arr = make_typed(env, napi_uint32_array, (size_t)count, 4, &d);
  if (!arr) return throw_msg(env, "decode: cannot allocate the token array");
  if (count) {
    const int rc = e4b_decode(x->c, (uint32_t)start, (uint32_t)count, (uint32_t*)d);
    if (rc) return throw_lib(env, "decode", rc);
  }
  return arr;
}

napi_value argmax(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "argmax: not an engine context");
  uint32_t am = 0;
  const int rc = e4b_argmax(x->c, &am);
  if (rc) return throw_lib(env, "argmax", rc);
  napi_value v;
  CHECK_NAPI(napi_create_uint32(env, am, &v));
  return v;
}

napi_value read_f32(napi_env env, napi_callback_info info, bool hidden) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "read: not an engine context");
  const size_t n = hidden ? (size_t)x->hidden : (size_t)x->vocab;
  void* d = nullptr;
  napi_value arr = make_typed(env, napi_float32_array, n, 4, &d);
  if (!arr) return throw_msg(env, "read: cannot allocate");
  const int rc = hidden ? e4b_read_hidden(x->c, (float*)d) : e4b_read_logits(x->c, (float*)d);
  if (rc) return throw_lib(env, hidden ? "readHidden" : "readLogits", rc);
  return arr;
}
napi_value read_hidden(napi_env env, napi_callback_info info) { return read_f32(env, info, true); }

// readLayerHidden(ctx, layer) -> Float32Array [hidden]: the residual stream
// after `layer` in the last decode step (the engine needs
// FLAG_LAYER_HIDDEN for the layers before the last)
napi_value read_layer_hidden(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "readLayerHidden: not an engine context");
  int32_t layer = 0;
  if (napi_get_value_int32(env, argv[1], &layer) != napi_ok) return throw_msg(env, "readLayerHidden(ctx, layer)");
  void* d = nullptr;
  napi_value arr = make_typed(env, napi_float32_array, (size_t)x->hidden, 4, &d);
  if (!arr) return throw_msg(env, "readLayerHidden: cannot allocate");
  const int rc = e4b_read_layer_hidden(x->c, layer, (float*)d);
  if (rc) return throw_lib(env, "readLayerHidden", rc);
  return arr;
}
napi_value read_logits(napi_env env, napi_callback_info info) { return read_f32(env, info, false); }

// full-layer KV budget (src/engine-a4b.js:587-617): kvCount(ctx) -> entries;
// readScores(ctx, layer) -> Float32Array [qHeads * maxSeq];
// kvCompact(ctx, budget, protect) -> entries after compactAll
napi_value kv_count(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "kvCount: not an engine context");
  const int n = e4b_kv_count(x->c);
  if (n < 0) return throw_lib(env, "kvCount", n);
  napi_value v;
  CHECK_NAPI(napi_create_int32(env, n, &v));
  return v;
}

napi_value read_scores(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "readScores: not an engine context");
  int64_t layer = 0;
  if (!get_i64(env, argv[1], &layer)) return throw_msg(env, "readScores(ctx, layer)");
  void* d = nullptr;
  napi_value arr = make_typed(env, napi_float32_array, (size_t)x->q_heads * (size_t)x->max_seq, 4, &d);
  if (!arr) return throw_msg(env, "readScores: cannot allocate");
  const int rc = e4b_read_scores(x->c, (int)layer, (float*)d);
  if (rc) return throw_lib(env, "readScores", rc);
  return arr;
}

napi_value kv_compact(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  get_args(env, info, 3, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "kvCompact: not an engine context");
  int64_t budget = 0, protect = 0;
  if (!get_i64(env, argv[1], &budget) || !get_i64(env, argv[2], &protect) || budget < 0 || protect < 0 ||
      budget > INT32_MAX || protect > INT32_MAX)
    return throw_msg(env, "kvCompact(ctx, budget, protect)");
  const int n = e4b_kv_compact(x->c, (int)budget, (int)protect);
  if (n < 0) return throw_lib(env, "kvCompact", n);
  napi_value v;
  CHECK_NAPI(napi_create_int32(env, n, &v));
  return v;
}

napi_value reset(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  Ctx* x = ctx_of(env, argv[0]);
  if (!x) return throw_msg(env, "reset: not an engine context");
  const int rc = e4b_reset(x->c);
  if (rc) return throw_lib(env, "reset", rc);
  return nullptr;
}

// destroy(ctx): releases the device memory now (the finalizer then does nothing)
napi_value destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  void* p = nullptr;
  if (napi_get_value_external(env, argv[0], &p) != napi_ok || !p) return throw_msg(env, "destroy: not a context");
  Ctx* x = static_cast<Ctx*>(p);
  if (x->c) e4b_destroy(x->c);
  x->c = nullptr;
  return nullptr;
}

// enumerable, like the functions of a JS module object
constexpr napi_property_attributes kMethod =
    static_cast<napi_property_attributes>(napi_writable | napi_enumerable | napi_configurable);

napi_value init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"version", nullptr, version, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"lastError", nullptr, last_error, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"deviceCount", nullptr, device_count, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"create", nullptr, create, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"setTensor", nullptr, set_tensor, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"finalize", nullptr, finalize, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"step", nullptr, step, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"prefill", nullptr, prefill, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"prefillSteps", nullptr, prefill_steps, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"profileStep", nullptr, profile_step, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"profilePrefill", nullptr, profile_prefill, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"decode", nullptr, decode, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"argmax", nullptr, argmax, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"readHidden", nullptr, read_hidden, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"readLayerHidden", nullptr, read_layer_hidden, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"readLogits", nullptr, read_logits, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"kvCount", nullptr, kv_count, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"readScores", nullptr, read_scores, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"kvCompact", nullptr, kv_compact, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"reset", nullptr, reset, nullptr, nullptr, nullptr, kMethod, nullptr},
      {"destroy", nullptr, destroy, nullptr, nullptr, nullptr, kMethod, nullptr},
  };
  if (napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props) != napi_ok) return nullptr;
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
