// C-ABI plumbing: device selection, errors, streams, events, memory, and the
// small data-movement kernels (fill, embedding gather, KV-cache append).
#include <atomic>
#include <cstring>
#include <mutex>

#include "common.h"

namespace cdml {

static thread_local char g_err[512] = "";
static std::atomic<int> g_device{-1};
static std::mutex g_init_mu;

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static int hip_fail(hipError_t e, const char *what) {
  return fail(CDML_E_HIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

int ensure_device() {
  int dev = g_device.load(std::memory_order_acquire);
  if (dev < 0) {
    int rc = cdml_init(0);
    if (rc != CDML_OK) return rc;
    dev = g_device.load(std::memory_order_acquire);
  }
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != dev) {
    hipError_t e = hipSetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  }
  return CDML_OK;
}

int num_cus() {
  static std::atomic<int> cus{0};
  int n = cus.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus.store(n, std::memory_order_relaxed);
  }
  return n;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return CDML_OK;
}

// ---- small kernels -------------------------------------------------------

__global__ void fill_zero_kernel(float *__restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0.0f;
}

// One workgroup row-copies table[ids[i]] into out[i] (float4 when aligned).
__global__ void embed_kernel(const int *__restrict__ ids, int count,
                             const float *__restrict__ table, int vocab, int dim,
                             float *__restrict__ out, int *__restrict__ bad, int vec4) {
  int i = blockIdx.x;
  if (i >= count) return;
  int t = ids[i];
  bool ok = (unsigned)t < (unsigned)vocab;
  if (!ok && bad && threadIdx.x == 0) atomicAdd(bad, 1);
  float *dst = out + (size_t)i * dim;
  const float *src = table + (size_t)(ok ? t : 0) * dim;
  if (vec4) {
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
    float4 *d4 = reinterpret_cast<float4 *>(dst);
    for (int c = threadIdx.x; c < dim / 4; c += blockDim.x)
      d4[c] = ok ? s4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    for (int c = threadIdx.x; c < dim; c += blockDim.x) dst[c] = ok ? src[c] : 0.0f;
  }
}

__global__ void fill_i32_kernel(int *__restrict__ p, size_t n, int value) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

// One wave per row: lane-strided scan keeping (max, lowest index), then a
// butterfly reduction that prefers the larger value and, on ties, the lower
// index.  NaN never compares greater, so it never wins.
__global__ void __launch_bounds__(256) argmax_rows_kernel(const float *__restrict__ x, int rows,
                                                          int cols, int ld, int *__restrict__ out,
                                                          int out_stride) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + (size_t)row * ld;
  float best = -INFINITY;
  int idx = cols;  // sentinel: no finite candidate seen yet
  for (int c = lane; c < cols; c += 64) {
    const float v = xr[c];
    if (v > best || (v == best && c < idx)) {
      best = v;
      idx = c;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(idx, off);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  if (lane == 0) out[(size_t)row * out_stride] = idx < cols ? idx : 0;
}

__global__ void kv_append_kernel(const float *__restrict__ k_new, const float *__restrict__ v_new,
                                 float *__restrict__ kc, float *__restrict__ vc,
                                 const int *__restrict__ pos, int t_max, int dim) {
  int b = blockIdx.x;
  int p = pos[b];
  if (p < 0 || p >= t_max) return;
  size_t dst = ((size_t)b * t_max + p) * dim;
  for (int c = threadIdx.x; c < dim; c += blockDim.x) {
    kc[dst + c] = k_new[(size_t)b * dim + c];
    vc[dst + c] = v_new[(size_t)b * dim + c];
  }
}

}  // namespace cdml

using namespace cdml;

extern "C" {

const char *cdml_last_error(void) { return g_err; }

const char *cdml_version(void) { return "cdml-hip 0.1 (gfx950)"; }

int cdml_device_count(int *count) {
  if (!count) return fail(CDML_E_INVALID, "cdml_device_count: count is NULL");
  *count = 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice || (e == hipSuccess && n == 0)) {
    (void)hipGetLastError();
    return CDML_OK;
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return hip_fail(e, "hipGetDeviceCount");
  }
  *count = n;
  return CDML_OK;
}

int cdml_init(int device) {
  std::lock_guard<std::mutex> lock(g_init_mu);
  int n = 0;
  int rc = cdml_device_count(&n);
  if (rc != CDML_OK) return rc;
  if (n == 0) return fail(CDML_E_NODEVICE, "cdml_init: no HIP device is visible");
  if (device < 0 || device >= n)
    return fail(CDML_E_INVALID, "cdml_init: device %d out of range [0, %d)", device, n);
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  // A failure here leaves the library usable and the last error untouched;
  // the no-allocation entry point reports it when it is called.
  char msg[256];
  (void)noalloc_scratch_setup(device, msg, sizeof(msg));
  g_device.store(device, std::memory_order_release);
  return CDML_OK;
}

int cdml_device_info_get(int device, cdml_device_info *info) {
  if (!info) return fail(CDML_E_INVALID, "cdml_device_info_get: info is NULL");
  int n = 0;
  int rc = cdml_device_count(&n);
  if (rc != CDML_OK) return rc;
  if (n == 0) return fail(CDML_E_NODEVICE, "no HIP device is visible");
  if (device < 0 || device >= n) return fail(CDML_E_INVALID, "device %d out of range", device);
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  memset(info, 0, sizeof(*info));
  snprintf(info->name, sizeof(info->name), "%s", p.name);
  snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
  info->compute_units = p.multiProcessorCount;
  info->max_clock_mhz = p.clockRate / 1000;
  info->memory_clock_mhz = p.memoryClockRate / 1000;
  info->memory_bus_bits = p.memoryBusWidth;
  info->total_memory = p.totalGlobalMem;
  info->lds_per_workgroup = p.sharedMemPerBlock;
  return CDML_OK;
}

int cdml_stream_create(cdml_stream *stream) {
  if (!stream) return fail(CDML_E_INVALID, "cdml_stream_create: stream is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t s;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
  *stream = reinterpret_cast<cdml_stream>(s);
  return CDML_OK;
}

struct cdml_graph_s {
  hipGraphExec_t exec;
};

int cdml_graph_capture_begin(cdml_stream stream) {
  if (!stream) return fail(CDML_E_INVALID, "cdml_graph_capture_begin: recording needs a created stream");
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipStreamBeginCapture(as_hip(stream), hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
  return CDML_OK;
}

int cdml_graph_capture_end(cdml_stream stream, cdml_graph *graph) {
  if (!graph) return fail(CDML_E_INVALID, "cdml_graph_capture_end: graph is NULL");
  *graph = nullptr;
  if (!stream) return fail(CDML_E_INVALID, "cdml_graph_capture_end: recording needs a created stream");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(as_hip(stream), &g);
  (void)hipGetLastError();  // a failed recording also leaves the error state set
  if (e != hipSuccess || !g) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(e != hipSuccess ? e : hipErrorStreamCaptureInvalidated, "hipStreamEndCapture");
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph = new cdml_graph_s{exec};
  return CDML_OK;
}

int cdml_graph_launch(cdml_graph graph, cdml_stream stream) {
  if (!graph) return fail(CDML_E_INVALID, "cdml_graph_launch: graph is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipGraphLaunch(graph->exec, as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
  return CDML_OK;
}

int cdml_graph_destroy(cdml_graph graph) {
  if (!graph) return CDML_OK;
  hipError_t e = hipGraphExecDestroy(graph->exec);
  delete graph;
  if (e != hipSuccess) return hip_fail(e, "hipGraphExecDestroy");
  return CDML_OK;
}

int cdml_stream_destroy(cdml_stream stream) {
  if (!stream) return CDML_OK;
  hipError_t e = hipStreamDestroy(as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, "hipStreamDestroy");
  return CDML_OK;
}

int cdml_stream_synchronize(cdml_stream stream) {
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipStreamSynchronize(as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return CDML_OK;
}

int cdml_stream_wait_event(cdml_stream stream, cdml_event event) {
  if (!event) return fail(CDML_E_INVALID, "cdml_stream_wait_event: event is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipStreamWaitEvent(as_hip(stream), reinterpret_cast<hipEvent_t>(event), 0);
  if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
  return CDML_OK;
}

int cdml_event_create(cdml_event *event) {
  if (!event) return fail(CDML_E_INVALID, "cdml_event_create: event is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  hipEvent_t ev;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  *event = reinterpret_cast<cdml_event>(ev);
  return CDML_OK;
}

int cdml_event_destroy(cdml_event event) {
  if (!event) return CDML_OK;
  hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(event));
  if (e != hipSuccess) return hip_fail(e, "hipEventDestroy");
  return CDML_OK;
}

int cdml_event_record(cdml_event event, cdml_stream stream) {
  if (!event) return fail(CDML_E_INVALID, "cdml_event_record: event is NULL");
  hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  return CDML_OK;
}

int cdml_event_create_sync_only(cdml_event *event) {
  if (!event) return fail(CDML_E_INVALID, "cdml_event_create_sync_only: event is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  hipEvent_t ev;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags");
  *event = reinterpret_cast<cdml_event>(ev);
  return CDML_OK;
}

int cdml_event_synchronize(cdml_event event) {
  if (!event) return fail(CDML_E_INVALID, "cdml_event_synchronize: event is NULL");
  hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(event));
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  return CDML_OK;
}

int cdml_event_elapsed_ms(cdml_event start, cdml_event stop, float *ms) {
  if (!start || !stop || !ms) return fail(CDML_E_INVALID, "cdml_event_elapsed_ms: NULL argument");
  hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  return CDML_OK;
}

int cdml_malloc(void **ptr, size_t bytes) {
  if (!ptr) return fail(CDML_E_INVALID, "cdml_malloc: ptr is NULL");
  *ptr = nullptr;
  int rc = ensure_device();
  if (rc) return rc;
  if (bytes == 0) return CDML_OK;
  hipError_t e = hipMalloc(ptr, bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  return CDML_OK;
}

int cdml_free(void *ptr) {
  if (!ptr) return CDML_OK;
  hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return CDML_OK;
}

int cdml_host_alloc_pinned(void **ptr, size_t bytes) {
  if (!ptr) return fail(CDML_E_INVALID, "cdml_host_alloc_pinned: ptr is NULL");
  *ptr = nullptr;
  int rc = ensure_device();
  if (rc) return rc;
  if (bytes == 0) return CDML_OK;
  hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
  if (e != hipSuccess) return hip_fail(e, "hipHostMalloc");
  return CDML_OK;
}

int cdml_host_free_pinned(void *ptr) {
  if (!ptr) return CDML_OK;
  hipError_t e = hipHostFree(ptr);
  if (e != hipSuccess) return hip_fail(e, "hipHostFree");
  return CDML_OK;
}

static int copy_async(void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                      cdml_stream stream, const char *what) {
  if (bytes == 0) return CDML_OK;
  if (!dst || !src) return fail(CDML_E_INVALID, "%s: NULL pointer", what);
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, what);
  return CDML_OK;
}

int cdml_memcpy_h2d_async(void *dst, const void *src, size_t bytes, cdml_stream stream) {
  return copy_async(dst, src, bytes, hipMemcpyHostToDevice, stream, "cdml_memcpy_h2d_async");
}

int cdml_memcpy_d2h_async(void *dst, const void *src, size_t bytes, cdml_stream stream) {
  return copy_async(dst, src, bytes, hipMemcpyDeviceToHost, stream, "cdml_memcpy_d2h_async");
}

int cdml_memcpy_d2d_async(void *dst, const void *src, size_t bytes, cdml_stream stream) {
  return copy_async(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "cdml_memcpy_d2d_async");
}

int cdml_zero_f32_async(float *dst, size_t count, cdml_stream stream) {
  if (count == 0) return CDML_OK;
  if (!dst) return fail(CDML_E_INVALID, "cdml_zero_f32_async: dst is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  size_t blocks = (count + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  fill_zero_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(dst, count);
  return check_launch("fill_zero_kernel");
}

int cdml_fill_i32_async(int *dst, size_t count, int value, cdml_stream stream) {
  if (count == 0) return CDML_OK;
  if (!dst) return fail(CDML_E_INVALID, "cdml_fill_i32_async: dst is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  size_t blocks = (count + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  fill_i32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(dst, count, value);
  return check_launch("fill_i32_kernel");
}

int cdml_memcpy2d_d2d_async(void *dst, size_t dpitch, const void *src, size_t spitch,
                            size_t width_bytes, size_t height, cdml_stream stream) {
  if (width_bytes == 0 || height == 0) return CDML_OK;
  if (!dst || !src) return fail(CDML_E_INVALID, "cdml_memcpy2d_d2d_async: NULL pointer");
  if (dpitch < width_bytes || spitch < width_bytes)
    return fail(CDML_E_INVALID, "cdml_memcpy2d_d2d_async: pitch smaller than the row");
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = hipMemcpy2DAsync(dst, dpitch, src, spitch, width_bytes, height,
                                  hipMemcpyDeviceToDevice, as_hip(stream));
  if (e != hipSuccess) return hip_fail(e, "cdml_memcpy2d_d2d_async");
  return CDML_OK;
}

int cdml_argmax_rows(const float *x, int rows, int cols, int ld, int *out, int out_stride,
                     cdml_stream stream) {
  if (rows < 0 || cols <= 0 || ld < cols || out_stride < 1)
    return fail(CDML_E_INVALID, "cdml_argmax_rows: bad size (rows %d, cols %d, ld %d, stride %d)",
                rows, cols, ld, out_stride);
  if (rows == 0) return CDML_OK;
  if (!x || !out) return fail(CDML_E_INVALID, "cdml_argmax_rows: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  argmax_rows_kernel<<<dim3((rows + 3) / 4), dim3(256), 0, as_hip(stream)>>>(x, rows, cols, ld, out,
                                                                            out_stride);
  return check_launch("argmax_rows_kernel");
}

int cdml_embed_tokens(const int *ids, int count, const float *table, int vocab, int dim,
                      float *out, int *bad_count, cdml_stream stream) {
  if (count < 0 || vocab < 0 || dim < 0)
    return fail(CDML_E_INVALID, "cdml_embed_tokens: negative size");
  if (count == 0 || dim == 0) return CDML_OK;
  if (!ids || !table || !out) return fail(CDML_E_INVALID, "cdml_embed_tokens: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  int vec4 = (dim % 4 == 0) && aligned16(table) && aligned16(out);
  embed_kernel<<<dim3(count), dim3(64), 0, as_hip(stream)>>>(ids, count, table, vocab, dim, out,
                                                           bad_count, vec4);
  return check_launch("embed_kernel");
}

int cdml_kv_cache_append(const float *k_new, const float *v_new, float *kcache, float *vcache,
                         const int *positions, int batch, int t_max, int dim, cdml_stream stream) {
  if (batch < 0 || t_max <= 0 || dim <= 0)
    return fail(CDML_E_INVALID, "cdml_kv_cache_append: bad size");
  if (batch == 0) return CDML_OK;
  if (!k_new || !v_new || !kcache || !vcache || !positions)
    return fail(CDML_E_INVALID, "cdml_kv_cache_append: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  kv_append_kernel<<<dim3(batch), dim3(256), 0, as_hip(stream)>>>(k_new, v_new, kcache, vcache,
                                                                 positions, t_max, dim);
  return check_launch("kv_append_kernel");
}

}  // extern "C"
