// lt_internal.h -- shared declarations of the libllamatov_hip.so translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

#include "../../include/llamatov_hip.h"
#include "lt_numerics.h"

struct lt_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool capturing = false;
  int num_cus = 0;
  // the device address of lt_attn.hip's scratch array on this context's device (bound at
  // lt_init by lt_attn_scratch_bind), or null with the lookup's error in attn_scratch_err
  void* attn_scratch = nullptr;
  size_t attn_scratch_bytes = 0;
  hipError_t attn_scratch_err = hipSuccess;
};

// Binds ctx->attn_scratch to the device copy of the attention scratch array (the device
// must be current).  Never fails the caller: a failed lookup is kept in attn_scratch_err and
// reported by the entry point that needs the scratch.
void lt_attn_scratch_bind(lt_ctx* ctx);
// Gives the scratch back when ctx owns it (lt_free_ctx).
void lt_attn_scratch_release(lt_ctx* ctx);

int lt_fail(int code, const char* fmt, ...);
int lt_fail_hip(hipError_t e, const char* what, const char* file, int line);
int lt_check_launch(const char* kernel);

#define LT_CHECK(call)                                              \
  do {                                                              \
    hipError_t e_ = (call);                                         \
    if (e_ != hipSuccess) return lt_fail_hip(e_, #call, __FILE__, __LINE__); \
  } while (0)

#define LT_REQUIRE(cond, ...)                                       \
  do {                                                              \
    if (!(cond)) return lt_fail(LT_EINVAL, __VA_ARGS__);            \
  } while (0)

static inline bool lt_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Split-K attention workspace for `rows` = batch * nh query heads and nsplit splits:
// per-split maxima m[rows][nsplit], sums z[rows][nsplit], outputs o[rows][nsplit][hd]
// (16-byte aligned).
struct AttnWs {
  float* m;
  float* z;
  float* o;
};

static inline size_t lt_attn_ws_bytes(int rows, int hd, int nsplit) {
  const size_t nrow = (size_t)rows * nsplit;
  return nrow * (size_t)(2 + hd) * sizeof(float) + 256;
}

static inline AttnWs lt_attn_ws_layout(void* ws, int rows, int hd, int nsplit) {
  const size_t nrow = (size_t)rows * nsplit;
  AttnWs w;
  w.m = (float*)ws;
  w.z = w.m + nrow;
  w.o = (float*)(((uintptr_t)(w.z + nrow) + 15) & ~(uintptr_t)15);
  return w;
}

// Device helpers shared by the kernel translation units.
__device__ __forceinline__ float lt_h2f(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
