// trace.h -- opt-in device-side timeline of the decode kernels.
//
// A library built with -DE4B_TRACE (the `trace` make target: libe4b_trace.so)
// records, for every workgroup of every instrumented kernel, the real-time
// counter (s_memrealtime, a chip-wide constant-rate clock) at the kernel's
// first instruction and at wave 0's exit, a tag naming the kernel variant,
// and where it ran (hardware ids: XCD, shader engine, CU).  The records land
// in one device buffer, so they survive hipGraph replay: the timeline of a
// graph-replayed step, which kernel-trace profilers do not follow here, is
// read back as is.  A workgroup takes its record slot with one atomic on its
// XCD's own counter at phase mark 0 (after the kernel has requested its
// loads, so no wait for those loads also waits for the atomic's return) or,
// in kernels without mark 0, at exit, and writes the record at exit.  In
// the product build every E4B_TRACE_SCOPE compiles to nothing.
#pragma once
#include <stdint.h>

struct TraceRec {
  uint64_t t0, t1;   // real-time counter at entry and at wave 0's exit
  uint32_t tag;      // kernel family << 16 | variant
  uint32_t blk;      // linear workgroup index
  uint32_t hw_id;    // wave 0's HW_ID register (CU, shader array, shader engine)
  uint32_t xcc;      // wave 0's XCC_ID register (the XCD)
  uint32_t mark[4];  // wave 0's phase marks (E4B_TRACE_MARK), ticks after t0; 0 = not reached
  uint32_t pad[4];
};
constexpr int kTraceMarks = 4;
constexpr int kTraceXcds = 8;         // record segments, one per XCD
constexpr int kTraceCntStride = 64;   // counters 256 bytes apart

// kernel families (the high half of a tag)
enum TraceFamily : uint32_t {
  TR_Q40 = 1,       // variant: PROK + 8 | EPI << 5 | log2(R) << 8 | (KW == 4) << 12 | (ks > 1) << 13
  TR_ATTN = 2,      // variant: 1 global / 0 sliding
  TR_PLE = 3,
  TR_EMBED = 4,
  TR_PLE_PREP = 5,
  TR_TAIL = 6,
  TR_LMHEAD = 7,
  TR_FEEDBACK = 8,
  TR_ATTN_GEN = 9,  // A4B attention (variant: head dim)
  TR_ATTN_MERGE = 10,
  TR_MOE_ROUTER = 11,
  TR_MOE_GU = 12,
  TR_MOE_DOWN = 13,
  TR_MOE_TAIL = 14,
  TR_ROWNORM = 15,
};

// host side (lib.hip): every translation unit that holds instrumented kernels
// registers a binder that points its device-side globals at the buffer
typedef int (*TraceBinder)(TraceRec* buf, unsigned* cnt, unsigned cap);
bool trace_register(TraceBinder b);

#if defined(E4B_TRACE) && defined(__HIPCC__)
#include <hip/hip_runtime.h>

namespace {
__constant__ TraceRec* g_trace_buf;  // constant space: scalar loads, no wait on the vector memory counter
__constant__ unsigned* g_trace_cnt;
__constant__ unsigned g_trace_cap;  // records per XCD segment

struct TraceScope {
  uint64_t t0;
  uint32_t tag, slot, xcc;
  uint32_t mark[kTraceMarks] = {0, 0, 0, 0};
  __device__ __forceinline__ explicit TraceScope(uint32_t t) : t0(__builtin_amdgcn_s_memrealtime()), tag(t), slot(~0u), xcc(0) {
    xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // HW_REG_XCC_ID
  }
  __device__ __forceinline__ void take_slot() {
    if (threadIdx.x == 0 && slot == ~0u && g_trace_buf)
      slot = atomicAdd(g_trace_cnt + (xcc % kTraceXcds) * kTraceCntStride, 1u);
  }
  __device__ __forceinline__ ~TraceScope() {
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    take_slot();
    if (threadIdx.x == 0 && slot < g_trace_cap) {
      const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID
      const uint32_t blk = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
      uint4* d = reinterpret_cast<uint4*>(g_trace_buf + (size_t)(xcc % kTraceXcds) * g_trace_cap + slot);
      d[0] = make_uint4((uint32_t)t0, (uint32_t)(t0 >> 32), (uint32_t)t1, (uint32_t)(t1 >> 32));
      d[1] = make_uint4(tag, blk, hw, xcc);
      d[2] = make_uint4(mark[0], mark[1], mark[2], mark[3]);
    }
  }
  // phase mark i of wave 0 (the time since entry), e.g. "the prologue's
  // inputs are in", "the dot products are done"
  __device__ __forceinline__ void stamp(int i) {
    if (threadIdx.x < 64) mark[i] = (uint32_t)(__builtin_amdgcn_s_memrealtime() - t0);
    if (i == 0) take_slot();
  }
};

int trace_bind_unit(TraceRec* buf, unsigned* cnt, unsigned cap) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace_buf), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_trace_cnt), &cnt, sizeof(cnt)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_trace_cap), &cap, sizeof(cap)) != hipSuccess)
    return -1;
  return 0;
}
const bool g_trace_registered = trace_register(&trace_bind_unit);
}  // namespace

#define E4B_TRACE_SCOPE(tag) TraceScope e4b_trace_scope_((uint32_t)(tag))
#define E4B_TRACE_MARK(i)                 \
  do {                                    \
    __builtin_amdgcn_sched_barrier(0);    \
    e4b_trace_scope_.stamp(i);            \
    __builtin_amdgcn_sched_barrier(0);    \
  } while (0)
#else
#define E4B_TRACE_SCOPE(tag) ((void)0)
#define E4B_TRACE_MARK(i) ((void)0)
#endif

constexpr uint32_t trace_tag(uint32_t family, uint32_t variant) { return family << 16 | (variant & 0xffffu); }
