// lt_runtime.hip -- context, memory, error reporting and HIP-graph capture for
// libllamatov_hip.so.  Replaces the reference's ctypes binding of the CUDA driver API
// (bpd/lib/fact_dispatch.py:36-72) and GraphRunner's capture/replay calls
// (bpd/lib/dev_residency.py:1732-1818).
#include "lt_internal.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>

static thread_local char g_err[1024] = "";

int lt_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int lt_fail_hip(hipError_t e, const char* what, const char* file, int line) {
  snprintf(g_err, sizeof(g_err), "%s failed: %s (%d) at %s:%d", what, hipGetErrorString(e), (int)e,
           file, line);
  return (int)e;
}

int lt_check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return lt_fail_hip(e, kernel, __FILE__, __LINE__);
  return LT_OK;
}

extern "C" {

int lt_version(void) { return 1; }

int lt_last_error(char* buf, size_t n) {
  if (!buf || n == 0) return LT_EINVAL;
  snprintf(buf, n, "%s", g_err);
  return LT_OK;
}

int lt_device_count(int* n) {
  if (!n) return lt_fail(LT_EINVAL, "lt_device_count: null out");
  LT_CHECK(hipGetDeviceCount(n));
  return LT_OK;
}

int lt_init(int device, lt_ctx** out) {
  if (!out) return lt_fail(LT_EINVAL, "lt_init: null out");
  *out = nullptr;
  int n = 0;
  LT_CHECK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return lt_fail(LT_EINVAL, "lt_init: device %d of %d", device, n);
  LT_CHECK(hipSetDevice(device));
  lt_ctx* c = new lt_ctx();
  c->device = device;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return lt_fail_hip(e, "hipStreamCreateWithFlags", __FILE__, __LINE__);
  }
  hipDeviceProp_t prop;
  LT_CHECK(hipGetDeviceProperties(&prop, device));
  c->num_cus = prop.multiProcessorCount;
  lt_attn_scratch_bind(c);
  *out = c;
  return LT_OK;
}

int lt_free_ctx(lt_ctx* ctx) {
  if (!ctx) return LT_OK;
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_free_ctx: capture in progress");
  LT_CHECK(hipSetDevice(ctx->device));
  LT_CHECK(hipStreamSynchronize(ctx->stream));
  LT_CHECK(hipStreamDestroy(ctx->stream));
  lt_attn_scratch_release(ctx);
  delete ctx;
  return LT_OK;
}

int lt_malloc(lt_ctx* ctx, void** ptr, size_t nbytes) {
  if (!ctx || !ptr) return lt_fail(LT_EINVAL, "lt_malloc: null argument");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_malloc: not allowed during graph capture");
  *ptr = nullptr;
  LT_CHECK(hipSetDevice(ctx->device));
  LT_CHECK(hipMalloc(ptr, nbytes ? nbytes : 1));
  return LT_OK;
}

int lt_free(lt_ctx* ctx, void* ptr) {
  if (!ctx) return lt_fail(LT_EINVAL, "lt_free: null ctx");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_free: not allowed during graph capture");
  if (!ptr) return LT_OK;
  LT_CHECK(hipSetDevice(ctx->device));
  LT_CHECK(hipFree(ptr));
  return LT_OK;
}

int lt_memcpy_h2d(lt_ctx* ctx, void* dst, const void* src, size_t nbytes) {
  if (!ctx || (nbytes && (!dst || !src))) return lt_fail(LT_EINVAL, "lt_memcpy_h2d: null argument");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_memcpy_h2d: host copies cannot be captured");
  if (!nbytes) return LT_OK;
  LT_CHECK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, ctx->stream));
  LT_CHECK(hipStreamSynchronize(ctx->stream));
  return LT_OK;
}

int lt_memcpy_d2h(lt_ctx* ctx, void* dst, const void* src, size_t nbytes) {
  if (!ctx || (nbytes && (!dst || !src))) return lt_fail(LT_EINVAL, "lt_memcpy_d2h: null argument");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_memcpy_d2h: host copies cannot be captured");
  if (!nbytes) return LT_OK;
  LT_CHECK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, ctx->stream));
  LT_CHECK(hipStreamSynchronize(ctx->stream));
  return LT_OK;
}

int lt_memcpy_d2d(lt_ctx* ctx, void* dst, const void* src, size_t nbytes) {
  if (!ctx || (nbytes && (!dst || !src))) return lt_fail(LT_EINVAL, "lt_memcpy_d2d: null argument");
  if (!nbytes) return LT_OK;
  LT_CHECK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, ctx->stream));
  return LT_OK;
}

int lt_sync(lt_ctx* ctx) {
  if (!ctx) return lt_fail(LT_EINVAL, "lt_sync: null ctx");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_sync: not allowed during graph capture");
  LT_CHECK(hipStreamSynchronize(ctx->stream));
  return LT_OK;
}

struct lt_graph {
  hipGraph_t graph;
  hipGraphExec_t exec;
  int device;
};

int lt_graph_begin(lt_ctx* ctx) {
  if (!ctx) return lt_fail(LT_EINVAL, "lt_graph_begin: null ctx");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_graph_begin: capture already in progress");
  LT_CHECK(hipSetDevice(ctx->device));
  LT_CHECK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  return LT_OK;
}

int lt_graph_end(lt_ctx* ctx, lt_graph** out) {
  if (!ctx || !out) return lt_fail(LT_EINVAL, "lt_graph_end: null argument");
  if (!ctx->capturing) return lt_fail(LT_ESTATE, "lt_graph_end: no capture in progress");
  *out = nullptr;
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  LT_CHECK(hipStreamEndCapture(ctx->stream, &g));
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g);
    return lt_fail_hip(e, "hipGraphInstantiate", __FILE__, __LINE__);
  }
  lt_graph* lg = new lt_graph{g, ex, ctx->device};
  *out = lg;
  return LT_OK;
}

int lt_graph_launch(lt_ctx* ctx, lt_graph* g) {
  if (!ctx || !g) return lt_fail(LT_EINVAL, "lt_graph_launch: null argument");
  if (ctx->capturing) return lt_fail(LT_ESTATE, "lt_graph_launch: capture in progress");
  LT_CHECK(hipGraphLaunch(g->exec, ctx->stream));
  return LT_OK;
}

int lt_event_create(lt_ctx* ctx, void** ev) {
  if (!ctx || !ev) return lt_fail(LT_EINVAL, "lt_event_create: null argument");
  hipEvent_t e = nullptr;
  LT_CHECK(hipSetDevice(ctx->device));
  LT_CHECK(hipEventCreate(&e));
  *ev = (void*)e;
  return LT_OK;
}

int lt_event_record(lt_ctx* ctx, void* ev) {
  if (!ctx || !ev) return lt_fail(LT_EINVAL, "lt_event_record: null argument");
  LT_CHECK(hipEventRecord((hipEvent_t)ev, ctx->stream));
  return LT_OK;
}

int lt_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!start || !stop || !ms) return lt_fail(LT_EINVAL, "lt_event_elapsed_ms: null argument");
  LT_CHECK(hipEventSynchronize((hipEvent_t)stop));
  LT_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return LT_OK;
}

int lt_event_destroy(void* ev) {
  if (!ev) return LT_OK;
  LT_CHECK(hipEventDestroy((hipEvent_t)ev));
  return LT_OK;
}

int lt_graph_free(lt_graph* g) {
  if (!g) return LT_OK;
  LT_CHECK(hipSetDevice(g->device));
  LT_CHECK(hipGraphExecDestroy(g->exec));
  LT_CHECK(hipGraphDestroy(g->graph));
  delete g;
  return LT_OK;
}

}  // extern "C"
