// util.h -- error reporting shared by every translation unit of libe4b.
#pragma once
#include <stdarg.h>
#include <stdio.h>

// Records a formatted message as the calling thread's last error and returns
// `code`, so call sites read `return e4b_fail(E4B_EINVAL, "...")`.
int e4b_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// RoPE inverse frequencies theta^(-2p/head_dim) for p < angles, rounded once
// to f32 from a double pow (host.cpp)
void rope_inv_freq(float theta, int head_dim, int angles, float* out);

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define E4B_HIP(call)                                                                      \
  do {                                                                                     \
    hipError_t e4b_err_ = (call);                                                          \
    if (e4b_err_ != hipSuccess)                                                            \
      return e4b_fail(E4B_EHIP, "%s:%d %s -> %s", __FILE__, __LINE__, #call,               \
                      hipGetErrorString(e4b_err_));                                        \
  } while (0)
#endif
