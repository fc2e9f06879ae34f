// lib.hip -- C-ABI plumbing (errors, device memory, workspace) and the
// kernel-level entry points of libe4b.
#include <algorithm>
#include <mutex>
#include <vector>
#include <string.h>

#include "../../include/e4b.h"
#include "kernels.h"
#include "moe.h"
#include "step.h"
#include "util.h"

static thread_local char g_last_error[1024] = "";

int e4b_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* e4b_version(void) { return "e4b-mi355x 0.1 (gfx950)"; }
extern "C" const char* e4b_last_error(void) { return g_last_error; }

extern "C" int e4b_device_count(int* n) {
  if (!n) return e4b_fail(E4B_EINVAL, "e4b_device_count: null");
  E4B_HIP(hipGetDeviceCount(n));
  return E4B_OK;
}
extern "C" int e4b_set_device(int device) {
  E4B_HIP(hipSetDevice(device));
  return E4B_OK;
}
extern "C" void* e4b_dev_alloc(size_t bytes) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    e4b_fail(E4B_ENOMEM, "hipMalloc(%zu) -> %s", bytes, hipGetErrorString(e));
    return nullptr;
  }
  return p;
}
extern "C" int e4b_dev_free(void* p) {
  if (p) E4B_HIP(hipFree(p));
  return E4B_OK;
}
extern "C" int e4b_memcpy_h2d(void* dst, const void* src, size_t n) {
  E4B_HIP(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
  return E4B_OK;
}
extern "C" int e4b_memcpy_d2h(void* dst, const void* src, size_t n) {
  E4B_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
  return E4B_OK;
}
extern "C" int e4b_memset_dev(void* dst, int value, size_t n) {
  E4B_HIP(hipMemset(dst, value, n));
  return E4B_OK;
}
extern "C" int e4b_sync(void) {
  E4B_HIP(hipDeviceSynchronize());
  return E4B_OK;
}
extern "C" int e4b_stream_sync(void* stream) {
  E4B_HIP(hipStreamSynchronize((hipStream_t)stream));
  return E4B_OK;
}

extern "C" void* e4b_event_create(void) {
  hipEvent_t e = nullptr;
  hipError_t rc = hipEventCreate(&e);
  if (rc != hipSuccess) {
    e4b_fail(E4B_EHIP, "hipEventCreate -> %s", hipGetErrorString(rc));
    return nullptr;
  }
  return (void*)e;
}
extern "C" int e4b_event_record(void* ev, void* stream) {
  E4B_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
  return E4B_OK;
}
extern "C" int e4b_event_elapsed_ms(void* a, void* b, float* ms) {
  if (!ms) return e4b_fail(E4B_EINVAL, "e4b_event_elapsed_ms: null");
  E4B_HIP(hipEventSynchronize((hipEvent_t)b));
  E4B_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
  return E4B_OK;
}
extern "C" int e4b_event_destroy(void* ev) {
  if (ev) E4B_HIP(hipEventDestroy((hipEvent_t)ev));
  return E4B_OK;
}

// ---- per-device workspace ---------------------------------------------------
// One grow-only scratch buffer per device.  Calls that use it on one device
// must not overlap (one stream at a time).  A buffer outgrown by a later call
// is retired, not freed: a graph captured earlier, or work still queued on
// another stream, may hold its address.
namespace {
struct DevWs {
  uint8_t* buf = nullptr;
  size_t cap = 0;
  std::vector<uint8_t*> retired;
};
std::mutex g_ws_mu;
DevWs g_ws[64];
}  // namespace

int e4b_workspace(size_t bytes, Workspace* out, hipStream_t st) {
  int dev = 0;
  E4B_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return e4b_fail(E4B_EINVAL, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_ws_mu);
  DevWs& w = g_ws[dev];
  if (bytes > w.cap) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    E4B_HIP(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return e4b_fail(E4B_EINVAL,
                      "the call needs %zu bytes of library workspace (%zu held), which would allocate inside a "
                      "stream capture: make the same call once before capturing",
                      bytes, w.cap);
    const size_t cap = E4B_ALIGN256(bytes < (1u << 20) ? (1u << 20) : bytes);
    uint8_t* nb = nullptr;
    E4B_HIP(hipMalloc(&nb, cap));
    if (w.buf) w.retired.push_back(w.buf);
    w.buf = nb;
    w.cap = cap;
  }
  out->buf = w.buf;
  out->cap = w.cap;
  return E4B_OK;
}

// ---- kernel-level entry points -----------------------------------------------
static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int e4b_k_q40_gemv(const void* w_packed, int64_t rows, int64_t cols, const void* x, int x_dtype,
                              float* y, void* stream) {
  if (!w_packed || !x || !y || rows <= 0 || cols <= 0 || cols % 32)
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemv: bad arguments (rows=%lld cols=%lld)", (long long)rows,
                    (long long)cols);
  if (!aligned16(w_packed) || !aligned16(x))
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemv: weight and x must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const Q40Mat W = q40_view(w_packed, rows, cols);
  if (x_dtype == E4B_DT_F16) return launch_q40_gemv(W, (const uint32_t*)x, nullptr, y, st);
  if (x_dtype == E4B_DT_F32_HL)
    return launch_q40_gemv(W, (const uint32_t*)x, (const uint32_t*)((const uint16_t*)x + cols), y, st);
  if (x_dtype != E4B_DT_F32) return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemv: x_dtype %d", x_dtype);
  Workspace ws;
  const size_t half = E4B_ALIGN256((size_t)cols * 2);
  int rc = e4b_workspace(2 * half, &ws, st);
  if (rc) return rc;
  uint16_t* hi = (uint16_t*)ws.buf;
  uint16_t* lo = (uint16_t*)(ws.buf + half);
  if ((rc = launch_split_f32((const float*)x, cols, hi, lo, st))) return rc;
  return launch_q40_gemv(W, (const uint32_t*)hi, (const uint32_t*)lo, y, st);
}

extern "C" int e4b_k_q40_gemv_geglu(const void* w_packed, int64_t ff, int64_t cols, const void* x, void* out,
                                    void* stream) {
  if (!w_packed || !x || !out || ff <= 0 || cols <= 0 || cols % 32)
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemv_geglu: bad arguments (ff=%lld cols=%lld)", (long long)ff,
                    (long long)cols);
  if (!aligned16(w_packed) || !aligned16(x))
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemv_geglu: weight and x must be 16-byte aligned");
  GemvOut o = {nullptr, (uint16_t*)out, nullptr, ff};
  return launch_q40(q40_view(w_packed, 2 * ff, cols), (const uint32_t*)x, nullptr, EPI_GEGLU, o, 1,
                    (hipStream_t)stream);
}

extern "C" int e4b_k_q40_gemm(const void* w_packed, int64_t rows, int64_t cols, const void* x, int m, float* y,
                              void* stream) {
  if (!w_packed || !x || !y || rows <= 0 || cols <= 0 || cols % 32 || m <= 0)
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemm: bad arguments (rows=%lld cols=%lld m=%d)", (long long)rows,
                    (long long)cols, m);
  if (!aligned16(w_packed) || !aligned16(x))
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemm: weight and x must be 16-byte aligned");
  return launch_q40_gemm(q40_view(w_packed, rows, cols), (const uint16_t*)x, m, y, nullptr, 0, (hipStream_t)stream);
}

extern "C" int e4b_k_q40_gemm_geglu(const void* w_packed, int64_t ff, int64_t cols, const void* x, int m, void* out,
                                    void* stream) {
  if (!w_packed || !x || !out || ff <= 0 || cols <= 0 || cols % 32 || m <= 0)
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemm_geglu: bad arguments (ff=%lld cols=%lld m=%d)", (long long)ff,
                    (long long)cols, m);
  if (!aligned16(w_packed) || !aligned16(x))
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_gemm_geglu: weight and x must be 16-byte aligned");
  return launch_q40_gemm(q40_view(w_packed, 2 * ff, cols), (const uint16_t*)x, m, nullptr, (uint16_t*)out, ff,
                         (hipStream_t)stream);
}

extern "C" int e4b_k_q40_geglu_prenorm(const void* w_packed, int64_t ff, int64_t cols, const float* h_in,
                                       const float* resid, const float* w_resid, const float* w_in, float scale,
                                       float eps, float* h_out, void* out_f16, void* stream) {
  if (!w_packed || !h_in || !w_in || !out_f16 || (resid && !w_resid) || ff <= 0 || !q40_prologue_supported((int)cols))
    return e4b_fail(E4B_EINVAL, "e4b_k_q40_geglu_prenorm: bad arguments (ff=%lld cols=%lld; cols 256/512/1024/2048)",
                    (long long)ff, (long long)cols);
  if (!aligned16(w_packed)) return e4b_fail(E4B_EINVAL, "e4b_k_q40_geglu_prenorm: weight must be 16-byte aligned");
  GemvOut o = {nullptr, (uint16_t*)out_f16, nullptr, ff};
  ProArgs p{};
  p.hin = h_in;
  p.hout = h_out;
  p.a = resid;
  p.w1 = w_resid;
  p.w2 = w_in;
  p.scale = scale;
  p.H = (int)cols;
  p.eps = eps;
  return launch_q40(q40_view(w_packed, 2 * ff, cols), nullptr, nullptr, EPI_GEGLU, o, 1, (hipStream_t)stream, &p);
}

extern "C" int e4b_memcpy_d2d(void* dst, const void* src, size_t n, void* stream) {
  E4B_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return E4B_OK;
}

extern "C" int e4b_split_f32(const float* x, int64_t n, void* hl, void* stream) {
  if (!x || !hl || n <= 0) return e4b_fail(E4B_EINVAL, "e4b_split_f32: bad arguments");
  return launch_split_f32(x, n, (uint16_t*)hl, (uint16_t*)hl + n, (hipStream_t)stream);
}

extern "C" int e4b_k_q6k_gemv_argmax(const void* w_packed, int64_t rows, int64_t cols, const float* x,
                                     float softcap, float* logits, uint32_t* amax, void* stream) {
  if (!w_packed || !x || !amax || rows <= 0 || rows > 0xffffffffLL || cols <= 0 || cols % 256)
    return e4b_fail(E4B_EINVAL, "e4b_k_q6k_gemv_argmax: bad arguments (rows=%lld cols=%lld)", (long long)rows,
                    (long long)cols);
  if (!aligned16(w_packed)) return e4b_fail(E4B_EINVAL, "e4b_k_q6k_gemv_argmax: weight must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  Workspace ws;
  const size_t half = E4B_ALIGN256((size_t)cols * 2);
  const size_t partb = 2048 * sizeof(uint2);
  int rc = e4b_workspace(2 * half + partb, &ws, st);
  if (rc) return rc;
  uint16_t* hi = (uint16_t*)ws.buf;
  uint16_t* lo = (uint16_t*)(ws.buf + half);
  uint2* part = (uint2*)(ws.buf + 2 * half);
  if ((rc = launch_split_f32(x, cols, hi, lo, st))) return rc;
  return launch_q6k_gemv_argmax(q6_view(w_packed, rows, cols), (const uint32_t*)hi, (const uint32_t*)lo, softcap,
                                logits, amax, part, st);
}

// ---- allocation-free lm-head --------------------------------------------------
// e4b_k_q6k_gemv_argmax_noalloc keeps its scratch in a file-scope device array
// instead of the workspace: the f16 hi and lo halves of x (cols <= 4096) and
// the argmax partials of at most 2048 workgroups.  Each device holds its own
// copy; host code addresses it only through the pointer hipGetSymbolAddress
// returns for the current device.
constexpr size_t kNoAllocHalf = 4096 * sizeof(uint16_t);
constexpr size_t kNoAllocPart = 2048 * sizeof(uint2);
constexpr size_t kNoAllocBytes = 2 * kNoAllocHalf + kNoAllocPart;  // 32 KiB
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {
std::mutex g_scratch_mu;
uint8_t* g_scratch_dev[64];  // per device: the device address of `scratch`
}  // namespace

// The device address of `scratch` on the current device, looked up once per
// device (no allocation).
static int scratch_address(uint8_t** out) {
  int dev = 0;
  E4B_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return e4b_fail(E4B_EINVAL, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return e4b_fail(E4B_EHIP, "hipGetSymbolAddress(scratch) on device %d -> %s", dev, hipGetErrorString(e));
    g_scratch_dev[dev] = (uint8_t*)ptr;
  }
  *out = g_scratch_dev[dev];
  return E4B_OK;
}

extern "C" int e4b_k_q6k_gemv_argmax_noalloc(const void* w_packed, int64_t rows, int64_t cols, const float* x,
                                             float softcap, float* logits, uint32_t* amax, void* stream) {
  if (!w_packed || !x || !amax || rows <= 0 || rows > 0xffffffffLL || cols <= 0 || cols % 256)
    return e4b_fail(E4B_EINVAL, "e4b_k_q6k_gemv_argmax_noalloc: bad arguments (rows=%lld cols=%lld)",
                    (long long)rows, (long long)cols);
  if ((size_t)cols * sizeof(uint16_t) > kNoAllocHalf)
    return e4b_fail(E4B_ERANGE,
                    "e4b_k_q6k_gemv_argmax_noalloc: %lld columns exceed the %zu-column maximum of its %zu-byte "
                    "scratch",
                    (long long)cols, kNoAllocHalf / sizeof(uint16_t), kNoAllocBytes);
  if ((size_t)q6k_gemv_grid(rows, (int)(cols / 32)) * sizeof(uint2) > kNoAllocPart)
    return e4b_fail(E4B_ERANGE, "e4b_k_q6k_gemv_argmax_noalloc: %d argmax partials exceed the scratch",
                    q6k_gemv_grid(rows, (int)(cols / 32)));
  if (!aligned16(w_packed))
    return e4b_fail(E4B_EINVAL, "e4b_k_q6k_gemv_argmax_noalloc: weight must be 16-byte aligned");
  uint8_t* sp = nullptr;
  int rc = scratch_address(&sp);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  // every byte read below is written earlier in the same call: the split
  // writes hi/lo[0, cols), each GEMV workgroup writes its own partial and
  // the fold reads only the partials of this launch's workgroups
  uint16_t* hi = (uint16_t*)sp;
  uint16_t* lo = (uint16_t*)(sp + kNoAllocHalf);
  uint2* part = (uint2*)(sp + 2 * kNoAllocHalf);
  if ((rc = launch_split_f32(x, cols, hi, lo, st))) return rc;
  return launch_q6k_gemv_argmax(q6_view(w_packed, rows, cols), (const uint32_t*)hi, (const uint32_t*)lo, softcap,
                                logits, amax, part, st);
}

extern "C" int e4b_k_q6k_row(const void* w_packed, int64_t rows, int64_t cols, int64_t row, float mult, float* out,
                             void* stream) {
  if (!w_packed || !out || rows <= 0 || cols <= 0 || cols % 256 || row < 0 || row >= rows)
    return e4b_fail(E4B_EINVAL, "e4b_k_q6k_row: bad arguments (rows=%lld cols=%lld row=%lld)", (long long)rows,
                    (long long)cols, (long long)row);
  return launch_q6k_row(q6_view(w_packed, rows, cols), row, nullptr, mult, out, (hipStream_t)stream);
}

extern "C" int e4b_k_argmax(const float* x, int64_t n, uint32_t* amax, void* stream) {
  if (!x || !amax || n <= 0 || n > 0xffffffffLL) return e4b_fail(E4B_EINVAL, "e4b_k_argmax: bad arguments");
  Workspace ws;
  int rc = e4b_workspace(1024 * sizeof(uint2), &ws, (hipStream_t)stream);
  if (rc) return rc;
  return launch_argmax(x, n, amax, (uint2*)ws.buf, (hipStream_t)stream);
}

extern "C" int e4b_rope_inv_freq(float theta, int head_dim, int angles, float* out) {
  if (!out || head_dim <= 0 || head_dim % 2 || angles < 0 || angles > head_dim / 2 || !(theta > 0.f))
    return e4b_fail(E4B_EINVAL, "e4b_rope_inv_freq: bad arguments (theta=%g head_dim=%d angles=%d)", (double)theta,
                    head_dim, angles);
  rope_inv_freq(theta, head_dim, angles, out);
  return E4B_OK;
}

extern "C" int e4b_k_attn_prefill(const float* q, const void* kc, const void* vc, void* out, int m, int q_heads,
                                  int kv_heads, int slots, int window, uint32_t p0, void* stream) {
  if (!q || !kc || !vc || !out || m <= 0 || q_heads <= 0 || kv_heads <= 0 || slots <= 0 || window < 0)
    return e4b_fail(E4B_EINVAL, "e4b_k_attn_prefill: bad arguments");
  if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(out))
    return e4b_fail(E4B_EINVAL, "e4b_k_attn_prefill: buffers must be 16-byte aligned");
  PrefillAttnArgs a;
  a.q = q;
  a.kc = (const uint16_t*)kc;
  a.vc = (const uint16_t*)vc;
  a.out = (uint16_t*)out;
  a.M = m;
  a.qh = q_heads;
  a.kvh = kv_heads;
  a.slots = slots;
  a.window = window;
  a.p0 = p0;
  Workspace ws;
  int rc = e4b_workspace(attn_prefill_part_bytes(m, kv_heads, q_heads / kv_heads), &ws, (hipStream_t)stream);
  if (rc) return rc;
  a.part = (float*)ws.buf;
  a.part_bytes = ws.cap;
  return launch_attn_prefill(a, (hipStream_t)stream);
}

// Argument checks and launch description shared by the two decode-attention
// entry points; *part_bytes receives the size of the split-K partials
// ([q_heads][chunks][head_dim] f32 outputs at offset 0, then the
// [q_heads][chunks][2] (max, sum) pairs at *ml_off).
static int attn_decode_prepare(const char* fn, const float* qkv, const float* q_norm, const float* k_norm,
                               const float* inv_freq, int rope_angles, void* k_cache, void* v_cache, int q_heads,
                               int kv_heads, int head_dim, int slots, int window, uint32_t pos, float eps, int chunk,
                               void* out_f16, AttnLaunch* a, size_t* part_bytes, size_t* ml_off) {
  if (!qkv || !q_norm || !k_norm || (rope_angles > 0 && !inv_freq) || !k_cache || !v_cache || !out_f16 ||
      q_heads <= 0 || kv_heads <= 0 || slots <= 0 || window < 0 || rope_angles < 0 || rope_angles > head_dim / 2)
    return e4b_fail(E4B_EINVAL, "%s: bad arguments", fn);
  if (window == 0 && pos >= (uint32_t)slots)
    return e4b_fail(E4B_ERANGE, "%s: position %u beyond the %d-position global cache", fn, pos, slots);
  if (chunk == 0) chunk = 64;
  if (chunk != 32 && chunk != 64) return e4b_fail(E4B_EINVAL, "%s: chunk %d is not 32 or 64", fn, chunk);
  const int span = window > 0 ? window : slots;
  const int nch = attn_chunks(span, chunk);
  *ml_off = E4B_ALIGN256((size_t)q_heads * nch * head_dim * sizeof(float));
  *part_bytes = *ml_off + (size_t)q_heads * nch * 2 * sizeof(float);
  a->qkv = qkv;
  a->qw = q_norm;
  a->kw = k_norm;
  a->inv_freq = inv_freq;
  a->rope = nullptr;
  a->kc = (uint16_t*)k_cache;
  a->vc = (uint16_t*)v_cache;
  a->params = nullptr;
  a->pos = pos;
  a->part_o = nullptr;
  a->part_ml = nullptr;
  a->out = (uint16_t*)out_f16;
  a->qh = q_heads;
  a->kvh = kv_heads;
  a->hd = head_dim;
  a->angles = rope_angles;
  a->slots = slots;
  a->window = window;
  a->chunk = chunk;
  // V slices per chunk: 4 (more blocks) while few chunks are live, 2 (each
  // chunk's K rows read by half as many blocks) from 32 live chunks on
  // (measured on MI355X for c2: global layer at 4096 positions 9.9 us with
  // 2 slices against 11.9 with 4)
  {
    const uint32_t live = window > 0 ? std::min(pos + 1, (uint32_t)window) : pos + 1;
    a->vslices = attn_chunks((int)live, chunk) >= 32 ? 2 : 4;
  }
  a->combine = true;
  a->eps = eps;
  return E4B_OK;
}

extern "C" int e4b_k_attn_decode(const float* qkv, const float* q_norm, const float* k_norm, const float* inv_freq,
                                 int rope_angles, void* k_cache, void* v_cache, int q_heads, int kv_heads,
                                 int head_dim, int slots, int window, uint32_t pos, float eps, int chunk,
                                 void* out_f16, void* stream) {
  AttnLaunch a;
  size_t need = 0, ml_off = 0;
  int rc = attn_decode_prepare("e4b_k_attn_decode", qkv, q_norm, k_norm, inv_freq, rope_angles, k_cache, v_cache,
                               q_heads, kv_heads, head_dim, slots, window, pos, eps, chunk, out_f16, &a, &need,
                               &ml_off);
  if (rc) return rc;
  Workspace ws;
  if ((rc = e4b_workspace(need, &ws, (hipStream_t)stream))) return rc;
  a.part_o = (float*)ws.buf;
  a.part_ml = (float*)(ws.buf + ml_off);
  return launch_attn(a, (hipStream_t)stream);
}

// ---- MoE half-layer ----------------------------------------------------------
static int moe_setup(const e4b_moe_weights* w, const float* h, MoeArgs* A, Workspace* ws, hipStream_t st) {
  if (!w || !h || !w->ffn_norm || !w->router_scale || !w->pre_ffw2 || !w->router_w || !w->pes || !w->dense_gate_up ||
      !w->exp_gate_up || !w->dense_down || !w->exp_down || !w->post_ffw1 || !w->post_ffw2 || !w->post_ffw)
    return e4b_fail(E4B_EINVAL, "MoE layer: null pointer argument");
  const int H = w->hidden, E = w->n_experts, FF = w->expert_ffn, FF2 = w->dense_ffn;
  if (H <= 0 || H % 256 || E < kMoeTopK || E > 256 || FF <= 0 || FF % 32 || FF2 <= 0 || FF2 % 32)
    return e4b_fail(E4B_EINVAL, "MoE layer: bad shape (hidden %d, experts %d, expert_ffn %d, dense_ffn %d)", H, E, FF,
                    FF2);
  if (!aligned16(w->dense_gate_up) || !aligned16(w->exp_gate_up) || !aligned16(w->dense_down) ||
      !aligned16(w->exp_down) || !aligned16(h) || !aligned16(w->router_w) || !aligned16(w->router_scale))
    return e4b_fail(E4B_EINVAL, "MoE layer: weights and h must be 16-byte aligned");
  // scratch: scores, xd, xm, topk, g_dense, g_slots, dense_out, moe_out
  size_t off[8], cur = 0;
  const size_t sz[8] = {(size_t)E * 4, (size_t)H * 2, (size_t)H * 2, 64, (size_t)FF2 * 2,
                        (size_t)kMoeTopK * FF * 2, (size_t)H * 4, (size_t)H * 4};
  for (int i = 0; i < 8; ++i) {
    off[i] = cur;
    cur += E4B_ALIGN256(sz[i]);
  }
  int rc = e4b_workspace(cur, ws, st);
  if (rc) return rc;
  MoeArgs& a = *A;
  a = MoeArgs{};
  a.h = h;
  a.ffn_norm = w->ffn_norm;
  a.router_scale = w->router_scale;
  a.router_mult = 1.0f / sqrtf((float)H);
  a.pre_ffw2 = w->pre_ffw2;
  a.router_w = w->router_w;
  a.pes = w->pes;
  a.dense_gu = q40_view(w->dense_gate_up, 2 * (int64_t)FF2, H);
  a.exp_gu = q40_view(w->exp_gate_up, (int64_t)E * 2 * FF, H);
  a.dense_down = q40_view(w->dense_down, H, FF2);
  a.exp_down = q40_view(w->exp_down, (int64_t)E * H, FF);
  a.post_ffw1 = w->post_ffw1;
  a.post_ffw2 = w->post_ffw2;
  a.post_ffw = w->post_ffw;
  a.layer_scale = w->layer_scale;
  a.eps = w->eps;
  a.H = H;
  a.E = E;
  a.FF = FF;
  a.FF2 = FF2;
  uint8_t* b = ws->buf;
  a.scores = (float*)(b + off[0]);
  a.xd = (uint16_t*)(b + off[1]);
  a.xm = (uint16_t*)(b + off[2]);
  a.topk_idx = (uint32_t*)(b + off[3]);
  a.topk_w = (float*)(b + off[3] + 32);
  a.g_dense = (uint16_t*)(b + off[4]);
  a.g_slots = (uint16_t*)(b + off[5]);
  a.dense_out = (float*)(b + off[6]);
  a.moe_out = (float*)(b + off[7]);
  return E4B_OK;
}

extern "C" int e4b_k_router_top8(const e4b_moe_weights* w, const float* h, uint32_t* topk_idx, float* topk_w,
                                 void* stream) {
  if (!topk_idx || !topk_w) return e4b_fail(E4B_EINVAL, "e4b_k_router_top8: null output");
  MoeArgs a;
  Workspace ws;
  int rc = moe_setup(w, h, &a, &ws, (hipStream_t)stream);
  if (rc) return rc;
  a.topk_idx = topk_idx;
  a.topk_w = topk_w;
  return launch_moe_topk(a, (hipStream_t)stream);
}

extern "C" int e4b_k_moe_prefill(const e4b_moe_weights* w, const float* h, int m, float* h_out, uint32_t* topk_idx,
                                 float* topk_w, float* dense_out, float* moe_out, void* stream) {
  if (!h_out || m < 1 || m > 1024) return e4b_fail(E4B_EINVAL, "e4b_k_moe_prefill: null h_out or m=%d outside 1..1024", m);
  MoeArgs a;
  Workspace ws;
  int rc = moe_setup(w, h, &a, &ws, (hipStream_t)stream);  // validates the weights (its scratch is not used)
  if (rc) return rc;
  const size_t bytes = moe_prefill_scratch(a, m, nullptr, nullptr);
  if ((rc = e4b_workspace(bytes, &ws, (hipStream_t)stream))) return rc;
  MoePrefillBufs b;
  moe_prefill_scratch(a, m, &b, ws.buf);
  a.h_out = h_out;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_moe_prefill(a, m, b, st))) return rc;
  const size_t P = (size_t)m * kMoeTopK * 4, HB = (size_t)m * a.H * 4;
  if (topk_idx) E4B_HIP(hipMemcpyAsync(topk_idx, b.topk_idx, P, hipMemcpyDeviceToDevice, st));
  if (topk_w) E4B_HIP(hipMemcpyAsync(topk_w, b.topk_w, P, hipMemcpyDeviceToDevice, st));
  if (dense_out) E4B_HIP(hipMemcpyAsync(dense_out, b.dense_out, HB, hipMemcpyDeviceToDevice, st));
  if (moe_out) E4B_HIP(hipMemcpyAsync(moe_out, b.moe_out, HB, hipMemcpyDeviceToDevice, st));
  return E4B_OK;
}

extern "C" int e4b_k_moe_layer(const e4b_moe_weights* w, const float* h, float* h_out, uint32_t* topk_idx,
                               float* topk_w, float* dense_out, float* moe_out, void* stream) {
  if (!h_out) return e4b_fail(E4B_EINVAL, "e4b_k_moe_layer: null h_out");
  MoeArgs a;
  Workspace ws;
  int rc = moe_setup(w, h, &a, &ws, (hipStream_t)stream);
  if (rc) return rc;
  a.h_out = h_out;
  if (topk_idx) a.topk_idx = topk_idx;
  if (topk_w) a.topk_w = topk_w;
  if (dense_out) a.dense_out = dense_out;
  if (moe_out) a.moe_out = moe_out;
  return launch_moe_ffn(a, (hipStream_t)stream);
}

// ---- device-side timeline (E4B_TRACE builds) -------------------------------------
#include "trace.h"

static std::vector<TraceBinder>& trace_binders() {
  static std::vector<TraceBinder> v;
  return v;
}
bool trace_register(TraceBinder b) {
  trace_binders().push_back(b);
  return true;
}
static_assert(sizeof(TraceRec) == sizeof(e4b_trace_rec), "trace record layout");
static TraceRec* g_tr_host_buf = nullptr;
static unsigned* g_tr_host_cnt = nullptr;
static size_t g_tr_host_cap = 0;

static int trace_bind_all(TraceRec* buf, unsigned* cnt, unsigned cap) {
  for (TraceBinder b : trace_binders())
    if (b(buf, cnt, cap)) return e4b_fail(E4B_EHIP, "trace: binding a unit's trace buffer failed");
  return E4B_OK;
}

extern "C" int e4b_trace_start(size_t cap) {
#ifndef E4B_TRACE
  (void)cap;
  return e4b_fail(E4B_EINVAL, "e4b_trace_start: this library was built without E4B_TRACE (use libe4b_trace.so)");
#else
  if (cap < kTraceXcds || cap > (1u << 26)) return e4b_fail(E4B_EINVAL, "e4b_trace_start: capacity %zu", cap);
  int rc = e4b_trace_stop();
  if (rc) return rc;
  // one segment of cap / 8 records per XCD, one counter per segment
  E4B_HIP(hipMalloc(&g_tr_host_buf, cap * sizeof(TraceRec)));
  E4B_HIP(hipMalloc(&g_tr_host_cnt, kTraceXcds * kTraceCntStride * sizeof(unsigned)));
  E4B_HIP(hipMemset(g_tr_host_cnt, 0, kTraceXcds * kTraceCntStride * sizeof(unsigned)));
  g_tr_host_cap = cap / kTraceXcds;
  E4B_HIP(hipDeviceSynchronize());
  return trace_bind_all(g_tr_host_buf, g_tr_host_cnt, (unsigned)g_tr_host_cap);
#endif
}

extern "C" int e4b_trace_read(e4b_trace_rec* out, size_t cap, size_t* recorded) {
  if (!g_tr_host_buf) return e4b_fail(E4B_ESTATE, "e4b_trace_read: no trace running");
  if (!recorded || (cap && !out)) return e4b_fail(E4B_EINVAL, "e4b_trace_read: null output");
  E4B_HIP(hipDeviceSynchronize());
  unsigned n[kTraceXcds * kTraceCntStride];
  E4B_HIP(hipMemcpy(n, g_tr_host_cnt, sizeof(n), hipMemcpyDeviceToHost));
  size_t total = 0, put = 0;
  for (int x = 0; x < kTraceXcds; ++x) {
    const size_t nx = n[x * kTraceCntStride];
    total += nx;
    const size_t m = std::min(std::min(nx, g_tr_host_cap), cap - put);
    if (m) E4B_HIP(hipMemcpy(out + put, g_tr_host_buf + x * g_tr_host_cap, m * sizeof(TraceRec), hipMemcpyDeviceToHost));
    put += m;
  }
  *recorded = total;
  return E4B_OK;
}

extern "C" int e4b_trace_stop(void) {
  if (!g_tr_host_buf) return E4B_OK;
  E4B_HIP(hipDeviceSynchronize());
  int rc = trace_bind_all(nullptr, nullptr, 0);
  (void)hipFree(g_tr_host_buf);
  (void)hipFree(g_tr_host_cnt);
  g_tr_host_buf = nullptr;
  g_tr_host_cnt = nullptr;
  g_tr_host_cap = 0;
  return rc;
}

extern "C" int e4b_trace_clock_khz(int* khz) {
  if (!khz) return e4b_fail(E4B_EINVAL, "e4b_trace_clock_khz: null");
  int dev = 0;
  E4B_HIP(hipGetDevice(&dev));
  E4B_HIP(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev));
  return E4B_OK;
}
