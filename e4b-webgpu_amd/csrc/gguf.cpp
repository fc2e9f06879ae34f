// gguf.cpp -- GGUF v2/v3 loader on the C ABI: the file is memory-mapped, the
// header, key/value metadata and tensor table are parsed once (the format and
// rules of openGGUF, src/gguf.js:17-83: tokenizer.* values skipped, data start
// aligned to general.alignment, default 32), the engine configuration is read
// from the metadata, and every tensor's bytes go to e4b_set_tensor straight
// from the mapping (the library repacks them as it uploads).
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "../../include/e4b.h"
#include "util.h"

namespace {

struct TensorInfo {
  std::string name;
  int64_t dims[4];
  int nd;
  uint32_t type;
  uint64_t offset;
};

struct Value {
  int type = -1;              // GGUF value type of a scalar, 8 = string, 9 = array
  double num = 0;             // numeric scalars
  std::string str;
  std::vector<double> arr;    // numeric / bool arrays
};

struct File {
  int fd = -1;
  const uint8_t* base = nullptr;
  size_t size = 0;
  std::vector<std::pair<std::string, Value>> kv;
  std::vector<TensorInfo> tensors;
  uint64_t data_start = 0;
  ~File() {
    if (base) munmap(const_cast<uint8_t*>(base), size);
    if (fd >= 0) close(fd);
  }
  const Value* find(const std::string& k) const {
    for (const auto& p : kv)
      if (p.first == k) return &p.second;
    return nullptr;
  }
};

struct Reader {
  const uint8_t* p;
  size_t n, off = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || off + k > n || off + k < off) return ok = false;
    return true;
  }
  uint64_t u(int bytes) {
    if (!need((size_t)bytes)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < bytes; ++i) v |= (uint64_t)p[off + i] << (8 * i);
    off += (size_t)bytes;
    return v;
  }
  std::string s() {
    const uint64_t len = u(8);
    if (!need((size_t)len)) return std::string();
    std::string r((const char*)p + off, (size_t)len);
    off += (size_t)len;
    return r;
  }
};

// scalar of GGUF type t as a double (ints exactly up to 2^53)
bool scalar(Reader& r, uint32_t t, double* out) {
  switch (t) {
    case 0: *out = (double)(uint8_t)r.u(1); return r.ok;
    case 1: *out = (double)(int8_t)r.u(1); return r.ok;
    case 2: *out = (double)(uint16_t)r.u(2); return r.ok;
    case 3: *out = (double)(int16_t)r.u(2); return r.ok;
    case 4: *out = (double)(uint32_t)r.u(4); return r.ok;
    case 5: *out = (double)(int32_t)r.u(4); return r.ok;
    case 6: {
      const uint32_t b = (uint32_t)r.u(4);
      float f;
      memcpy(&f, &b, 4);
      *out = f;
      return r.ok;
    }
    case 7: *out = r.u(1) ? 1.0 : 0.0; return r.ok;
    case 10: *out = (double)r.u(8); return r.ok;
    case 11: *out = (double)(int64_t)r.u(8); return r.ok;
    case 12: {
      const uint64_t b = r.u(8);
      double d;
      memcpy(&d, &b, 8);
      *out = d;
      return r.ok;
    }
  }
  return false;
}

bool value(Reader& r, uint32_t t, Value* v, bool keep) {
  v->type = (int)t;
  if (t == 8) {
    v->str = r.s();
    if (!keep) v->str.clear();
    return r.ok;
  }
  if (t == 9) {
    const uint32_t et = (uint32_t)r.u(4);
    const uint64_t n = r.u(8);
    if (!r.ok || n > r.n) return false;
    for (uint64_t i = 0; i < n; ++i) {
      if (et == 8) {
        r.s();
      } else if (et == 9) {
        Value sub;
        if (!value(r, et, &sub, false)) return false;
      } else {
        double d;
        if (!scalar(r, et, &d)) return false;
        if (keep) v->arr.push_back(d);
      }
      if (!r.ok) return false;
    }
    return true;
  }
  return scalar(r, t, &v->num);
}

int tensor_bytes(uint32_t type, const int64_t* dims, int nd, uint64_t* out) {
  uint64_t bb, be;
  switch (type) {
    case E4B_GGML_F32: bb = 4; be = 1; break;
    case E4B_GGML_F16: bb = 2; be = 1; break;
    case E4B_GGML_Q4_0: bb = 18; be = 32; break;
    case E4B_GGML_Q6_K: bb = 210; be = 256; break;
    default: return e4b_fail(E4B_EINVAL, "GGUF: ggml type %u is not used by this engine", type);
  }
  uint64_t n = 1;
  for (int i = 0; i < nd; ++i) n *= (uint64_t)dims[i];
  if (n % be) return e4b_fail(E4B_EINVAL, "GGUF: %llu elements are not whole blocks", (unsigned long long)n);
  *out = n / be * bb;
  return E4B_OK;
}

int open_file(const char* path, File* f) {
  if (!path) return e4b_fail(E4B_EINVAL, "GGUF: null path");
  f->fd = open(path, O_RDONLY);
  if (f->fd < 0) return e4b_fail(E4B_EINVAL, "GGUF: cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(f->fd, &st) != 0 || st.st_size < 24) return e4b_fail(E4B_EINVAL, "GGUF: %s is too short", path);
  f->size = (size_t)st.st_size;
  void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
  if (m == MAP_FAILED) return e4b_fail(E4B_EINVAL, "GGUF: mmap of %s failed: %s", path, strerror(errno));
  f->base = (const uint8_t*)m;
  Reader r{f->base, f->size};
  if (memcmp(f->base, "GGUF", 4) != 0) return e4b_fail(E4B_EINVAL, "GGUF: %s is not GGUF", path);
  r.off = 4;
  const uint32_t version = (uint32_t)r.u(4);
  if (version != 2 && version != 3) return e4b_fail(E4B_EINVAL, "GGUF: unsupported version %u", version);
  const uint64_t nt = r.u(8), nkv = r.u(8);
  if (!r.ok || nt > f->size || nkv > f->size) return e4b_fail(E4B_EINVAL, "GGUF: corrupt header");
  for (uint64_t i = 0; i < nkv; ++i) {
    std::string k = r.s();
    const uint32_t t = (uint32_t)r.u(4);
    Value v;
    const bool keep = k.compare(0, 10, "tokenizer.") != 0;
    if (!r.ok || !value(r, t, &v, keep)) return e4b_fail(E4B_EINVAL, "GGUF: truncated metadata (%s)", k.c_str());
    if (keep) f->kv.emplace_back(std::move(k), std::move(v));
  }
  uint64_t align = 32;
  if (const Value* a = f->find("general.alignment")) align = (uint64_t)a->num;
  if (align == 0 || (align & (align - 1))) return e4b_fail(E4B_EINVAL, "GGUF: alignment %llu", (unsigned long long)align);
  for (uint64_t i = 0; i < nt; ++i) {
    TensorInfo ti;
    ti.name = r.s();
    ti.nd = (int)r.u(4);
    if (!r.ok || ti.nd < 1 || ti.nd > 4) return e4b_fail(E4B_EINVAL, "GGUF: tensor %s has %d dims", ti.name.c_str(), ti.nd);
    for (int d = 0; d < 4; ++d) ti.dims[d] = d < ti.nd ? (int64_t)r.u(8) : 1;
    ti.type = (uint32_t)r.u(4);
    ti.offset = r.u(8);
    if (!r.ok) return e4b_fail(E4B_EINVAL, "GGUF: truncated tensor table");
    f->tensors.push_back(ti);
  }
  f->data_start = (r.off + align - 1) / align * align;
  return E4B_OK;
}

double num_or(const File& f, const std::string& k, double dflt, bool* found = nullptr) {
  const Value* v = f.find(k);
  if (found) *found = v && v->type != 8 && v->type != 9;
  return (v && v->type != 8 && v->type != 9) ? v->num : dflt;
}

// the A4B recipe of a gemma4 MoE file, read as loadEngineA4B reads it
// (src/engine-a4b.js:100-116, 150-156, 330-334): sliding layers of head dim
// key_length_swa rotating every pair with theta 1e4, full layers of head dim
// key_length rotating floor(0.25 * key_length / 2) pairs with theta 1e6 and
// V = K, KV heads per layer, a MoE half of expert_count experts (top 8) of
// expert_feed_forward_length beside the dense feed_forward_length branch,
// the ring window + 512 slots; theta 1e4 / 1e6 as the recipe fixes them
// (src/engine-a4b.js:329)
int gguf_config_a4b(const File& f, const std::string& p, e4b_config* cfg, int32_t* layer_kv_heads, int cap) {
  cfg->recipe = E4B_RECIPE_A4B;
  cfg->ple_dim = 0;
  const int used = (int)num_or(f, p + "expert_used_count", 8);
  if (used != 8) return e4b_fail(E4B_EINVAL, "GGUF: expert_used_count %d (the MoE kernels select 8)", used);
  cfg->n_experts = (int32_t)num_or(f, p + "expert_count", cfg->n_experts);
  cfg->expert_ffn = (int32_t)num_or(f, p + "expert_feed_forward_length", cfg->expert_ffn);
  cfg->head_dim_full = (int32_t)num_or(f, p + "attention.key_length", cfg->head_dim_full);
  cfg->head_dim = (int32_t)num_or(f, p + "attention.key_length_swa", cfg->head_dim);
  cfg->rope_angles = cfg->head_dim / 2;
  cfg->rope_angles_full = (int32_t)(0.25 * cfg->head_dim_full / 2);
  cfg->theta_local = 10000.0f;  // fixed by the recipe, not read from the file
  cfg->theta_global = 1000000.0f;
  if (cfg->ring < cfg->window + 512) cfg->ring = cfg->window + 512;
  if (const Value* kvh = f.find(p + "attention.head_count_kv")) {
    if (kvh->type == 9) {
      if ((int)kvh->arr.size() != cfg->layers)
        return e4b_fail(E4B_EINVAL, "GGUF: attention.head_count_kv lists %zu layers, not %d", kvh->arr.size(),
                        cfg->layers);
      if (!layer_kv_heads || cap < cfg->layers)
        return e4b_fail(E4B_EINVAL, "e4b_gguf_config: layer_kv_heads needs room for %d layers", cfg->layers);
      for (int i = 0; i < cfg->layers; ++i) layer_kv_heads[i] = (int32_t)kvh->arr[(size_t)i];
      cfg->layer_kv_heads = layer_kv_heads;
      cfg->kv_heads = layer_kv_heads[0];
    }
  }
  return E4B_OK;
}

}  // namespace

extern "C" int e4b_gguf_config(const char* path, e4b_config* cfg, uint8_t* layer_global, int32_t* layer_kv_heads,
                               int cap) {
  if (!cfg) return e4b_fail(E4B_EINVAL, "e4b_gguf_config: null config");
  File f;
  int rc = open_file(path, &f);
  if (rc) return rc;
  std::string arch = "e4b";
  if (const Value* a = f.find("general.architecture"))
    if (a->type == 8) arch = a->str;
  const std::string p = arch + ".";
  struct IntKey {
    const char* key;
    int32_t* dst;
  } ints[] = {{"embedding_length", &cfg->hidden}, {"block_count", &cfg->layers},
              {"attention.head_count", &cfg->q_heads}, {"attention.head_count_kv", &cfg->kv_heads},
              {"attention.key_length", &cfg->head_dim}, {"feed_forward_length", &cfg->ffn},
              {"embedding_length_per_layer_input", &cfg->ple_dim}, {"vocab_size", &cfg->vocab},
              {"attention.sliding_window", &cfg->window}, {"rope.dimension_count_half", &cfg->rope_angles}};
  for (const IntKey& k : ints) *k.dst = (int32_t)num_or(f, p + k.key, *k.dst);
  struct FloatKey {
    const char* key;
    float* dst;
  } flts[] = {{"rope.freq_base_swa", &cfg->theta_local}, {"rope.freq_base", &cfg->theta_global},
              {"attention.layer_norm_rms_epsilon", &cfg->eps}, {"final_logit_softcapping", &cfg->softcap}};
  for (const FloatKey& k : flts) *k.dst = (float)num_or(f, p + k.key, *k.dst);
  // the vocabulary of a file without vocab_size: the embedding's row count
  if (!f.find(p + "vocab_size"))
    for (const TensorInfo& t : f.tensors)
      if (t.name == "token_embd.weight" && t.nd >= 2) cfg->vocab = (int32_t)t.dims[1];
  if (f.find(p + "expert_count") && (rc = gguf_config_a4b(f, p, cfg, layer_kv_heads, cap))) return rc;
  if (const Value* pat = f.find(p + "attention.sliding_window_pattern")) {
    if (pat->type != 9 || (int)pat->arr.size() != cfg->layers)
      return e4b_fail(E4B_EINVAL, "GGUF: sliding_window_pattern must list %d layers", cfg->layers);
    if (!layer_global || cap < cfg->layers)
      return e4b_fail(E4B_EINVAL, "e4b_gguf_config: layer_global needs room for %d layers", cfg->layers);
    for (int i = 0; i < cfg->layers; ++i) layer_global[i] = pat->arr[(size_t)i] != 0.0 ? 0 : 1;
    cfg->layer_global = layer_global;
  }
  return E4B_OK;
}

extern "C" int e4b_load_gguf(e4b_ctx* ctx, const char* path) {
  if (!ctx) return e4b_fail(E4B_EINVAL, "e4b_load_gguf: null context");
  File f;
  int rc = open_file(path, &f);
  if (rc) return rc;
  for (const TensorInfo& t : f.tensors) {
    uint64_t n = 0;
    if ((rc = tensor_bytes(t.type, t.dims, t.nd, &n))) return rc;
    const uint64_t start = f.data_start + t.offset;
    if (start > f.size || n > f.size - start)
      return e4b_fail(E4B_EINVAL, "GGUF: tensor %s extends past the end of the file", t.name.c_str());
    if ((rc = e4b_set_tensor(ctx, t.name.c_str(), (int)t.type, t.dims, t.nd, f.base + start, (size_t)n))) return rc;
  }
  return E4B_OK;
}

extern "C" e4b_ctx* e4b_open_gguf(const char* path, const e4b_config* base) {
  e4b_config cfg;
  if (base) {
    cfg = *base;
  } else {
    memset(&cfg, 0, sizeof(cfg));
    cfg.ring = 1024;
    cfg.max_seq = 4096;
  }
  std::vector<uint8_t> lg(4096);
  std::vector<int32_t> kvh(4096);
  if (e4b_gguf_config(path, &cfg, lg.data(), kvh.data(), (int)lg.size())) return nullptr;
  e4b_ctx* c = e4b_create(&cfg);
  if (!c) return nullptr;
  if (e4b_load_gguf(c, path) || e4b_finalize(c)) {
    const std::string msg = e4b_last_error();
    e4b_destroy(c);
    e4b_fail(E4B_EINVAL, "%s", msg.c_str());
    return nullptr;
  }
  return c;
}
