// nlg_runtime.hip -- device bring-up, memory, streams, events, graphs.
//
// Replaces the Vulkan plumbing of host/vkserver.c: init_vulkan (:213-245),
// make_buffer_ex (:126-149), staged_write (:169-205), write_buffer
// (:207-211) and the compiled command buffers (:511-615).  One HIP stream
// replaces the single queue + fence; every buffer is device memory in HBM.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "nlg_internal.h"

static thread_local char g_err[1024];
static int g_inited = 0;
static int g_device = 0;
static int g_num_cu = 0;
static hipStream_t g_stream = nullptr;
static char g_arch[64];

// pinned staging for file uploads: two halves, double-buffered
static const size_t kStageBytes = 64u << 20;
static char *g_stage = nullptr;
static hipEvent_t g_stage_ev[2];

// Scratch of the allocation-free entry points: one fixed array per GPU (the
// code object's device globals exist once per device), reached through the
// device address looked up for each device at init.  Host code never uses
// the array's own name, which on the host is only a stand-in symbol.
static __device__ __align__(256) uint8_t scratch[NLG_NOALLOC_SCRATCH_BYTES];
#define NLG_MAX_DEVICES 64
static void *g_noalloc_scratch[NLG_MAX_DEVICES];

extern "C" const char *nlg_last_error(void) { return g_err; }

int nlg_fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return NLG_ERR;
}

extern "C" int nlg_init(int device) {
  if (g_inited) return NLG_OK;
  if (device < 0) {
    const char *e = getenv("NELISP_GPU_DEVICE");
    device = e ? atoi(e) : 0;
  }
  int n = 0;
  NLG_HIP(hipGetDeviceCount(&n));
  if (n <= 0) return nlg_fail("no GPU device visible");
  if (device < 0 || device >= n) device = 0;  // vkcompute.c:100's fallback
  NLG_HIP(hipSetDevice(device));
  if (device < NLG_MAX_DEVICES && !g_noalloc_scratch[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return nlg_fail("init: no device address for the fixed scratch array (%s)", hipGetErrorString(e));
    g_noalloc_scratch[device] = p;
  }
  hipDeviceProp_t prop;
  NLG_HIP(hipGetDeviceProperties(&prop, device));
  g_num_cu = prop.multiProcessorCount;
  snprintf(g_arch, sizeof g_arch, "%s", prop.gcnArchName);
  // The stream is blocking with respect to the null stream, so the
  // synchronous copies below are ordered after every kernel on it.
  NLG_HIP(hipStreamCreate(&g_stream));
  g_device = device;
  g_inited = 1;
  return NLG_OK;
}

int nlg_ensure_init(void) { return g_inited ? NLG_OK : nlg_init(-1); }

void *nlg_noalloc_scratch(void) {
  if (!g_inited || g_device >= NLG_MAX_DEVICES || !g_noalloc_scratch[g_device]) {
    nlg_fail("fixed scratch: device %d has none (library not initialised?)", g_device);
    return nullptr;
  }
  return g_noalloc_scratch[g_device];
}
int nlg_num_cu(void) { return g_num_cu; }

hipStream_t nlg_stream(void *s) { return s ? (hipStream_t)s : g_stream; }

// Library scratch for the batched linears' int8 activations, one per stream
// (calls on different streams may run concurrently; calls on one stream run
// in order, so they can share).  Grown by allocating a larger buffer; older
// ones stay allocated (a captured graph may still use them) until
// nlg_shutdown.
struct StreamScratch {
  std::vector<void *> bufs;
  size_t bytes = 0;
};
static std::map<std::pair<hipStream_t, int>, StreamScratch> g_scratch;
static std::mutex g_scratch_mu;

// Slot 0: the batched linears' int8 activations.  Slot 1: the column-split
// GEMM's partial sums and arrival counters, zero-filled when allocated (the
// GEMM leaves its counters at zero).
static void *scratch_get(size_t bytes, hipStream_t st, int slot, bool quiet) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  StreamScratch &e = g_scratch[{st, slot}];
  if (bytes <= e.bytes) return e.bufs.back();
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
    if (!quiet)
      nlg_fail("batched linear: its %zu-byte scratch must be reserved on this stream before graph capture "
               "(run the call once on it outside the capture first)", bytes);
    return nullptr;
  }
  size_t want = e.bytes ? e.bytes : (1u << 20);
  while (want < bytes) want *= 2;
  void *p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) {
    if (!quiet) nlg_fail("scratch: hipMalloc(%zu) failed", want);
    return nullptr;
  }
  if (slot == 1 && hipMemsetAsync(p, 0, want, st) != hipSuccess) {
    (void)hipFree(p);
    if (!quiet) nlg_fail("scratch: zero fill failed");
    return nullptr;
  }
  e.bufs.push_back(p);
  e.bytes = want;
  return p;
}

void *nlg_scratch(size_t bytes, hipStream_t st) { return scratch_get(bytes, st, 0, false); }
void *nlg_scratch_try(size_t bytes, hipStream_t st, int slot) { return scratch_get(bytes, st, slot, true); }

extern "C" int nlg_shutdown(void) {
  if (!g_inited) return NLG_OK;
  (void)hipDeviceSynchronize();
  nlg_tiled_release_all();
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    for (auto &kv : g_scratch)
      for (void *p : kv.second.bufs) (void)hipFree(p);
    g_scratch.clear();
  }
  if (g_stage) {
    (void)hipEventDestroy(g_stage_ev[0]);
    (void)hipEventDestroy(g_stage_ev[1]);
    (void)hipHostFree(g_stage);
    g_stage = nullptr;
  }
  (void)hipStreamDestroy(g_stream);
  g_stream = nullptr;
  g_inited = 0;
  return NLG_OK;
}

extern "C" int nlg_device_name(char *buf, size_t len) {
  if (nlg_ensure_init()) return NLG_ERR;
  char name[256] = {0};
  if (hipDeviceGetName(name, sizeof name, g_device) != hipSuccess || !name[0]) {
    hipDeviceProp_t prop;
    NLG_HIP(hipGetDeviceProperties(&prop, g_device));
    snprintf(name, sizeof name, "%s", prop.name[0] ? prop.name : prop.gcnArchName);
  }
  snprintf(buf, len, "%s", name);
  return NLG_OK;
}

extern "C" int nlg_device_info(int *num_cu, char *arch, size_t arch_len) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (num_cu) *num_cu = g_num_cu;
  if (arch && arch_len) snprintf(arch, arch_len, "%s", g_arch);
  return NLG_OK;
}

__global__ void k_zero(uint4 *p, uint64_t n16, uint8_t *tail, uint32_t ntail) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n16; i += stride) p[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

extern "C" int nlg_zero(void *dev, size_t bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!bytes) return NLG_OK;
  void *const dst0 = dev;
  const size_t bytes0 = bytes;
  // fast path needs 16-byte alignment; hipMalloc gives 256
  uintptr_t a = (uintptr_t)dev;
  if (a & 15) {
    size_t head = 16 - (a & 15);
    if (head > bytes) head = bytes;
    hipLaunchKernelGGL(k_zero, dim3(1), dim3(64), 0, nlg_stream(stream), (uint4 *)nullptr,
                       (uint64_t)0, (uint8_t *)dev, (uint32_t)head);
    NLG_LAUNCHED("zero");
    dev = (char *)dev + head;
    bytes -= head;
  }
  uint64_t n16 = bytes / 16;
  uint32_t tail = (uint32_t)(bytes % 16);
  uint32_t grid = nlg_blocks(n16, 256 * 8);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(k_zero, dim3(grid), dim3(256), 0, nlg_stream(stream), (uint4 *)dev, n16,
                     (uint8_t *)dev + n16 * 16, tail);
  NLG_LAUNCHED("zero");
  nlg_tiled_refresh_range(dst0, bytes0, nlg_stream(stream));
  NLG_LAUNCHED("tiled-copy refresh");
  return NLG_OK;
}

extern "C" void *nlg_malloc(size_t bytes) {
  if (nlg_ensure_init()) return nullptr;
  void *p = nullptr;
  size_t sz = bytes ? bytes : 4;  // the reference's zero-size buffers are 4 bytes (vkserver.c:128)
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) {
    nlg_fail("hipMalloc(%zu) failed: %s", sz, hipGetErrorString(e));
    return nullptr;
  }
  if (nlg_zero(p, sz, nullptr) || hipStreamSynchronize(g_stream) != hipSuccess) {
    (void)hipFree(p);
    return nullptr;
  }
  return p;
}

extern "C" int nlg_free(void *dev) {
  if (!dev) return NLG_OK;
  // registrations of tiled weight copies inside this allocation go with it
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)dev) == hipSuccess && base)
    nlg_tiled_drop_range((const void *)base, size);
  else
    nlg_tiled_drop_range(dev, 1);
  NLG_HIP(hipFree(dev));
  return NLG_OK;
}

extern "C" int nlg_upload(void *dst, const void *src, size_t bytes) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!bytes) return NLG_OK;
  NLG_HIP(hipStreamSynchronize(g_stream));
  NLG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  nlg_tiled_refresh_range(dst, bytes, g_stream);
  NLG_LAUNCHED("tiled-copy refresh");
  return NLG_OK;
}

extern "C" int nlg_download(void *dst, const void *src, size_t bytes) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!bytes) return NLG_OK;
  NLG_HIP(hipStreamSynchronize(g_stream));
  NLG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return NLG_OK;
}

extern "C" int nlg_copy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  if (!bytes) return NLG_OK;
  NLG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, nlg_stream(stream)));
  nlg_tiled_refresh_range(dst, bytes, nlg_stream(stream));
  NLG_LAUNCHED("tiled-copy refresh");
  return NLG_OK;
}

extern "C" int nlg_upload_file(void *dst, const char *path, uint64_t offset, size_t bytes,
                               size_t *missing) {
  if (missing) *missing = 0;
  if (nlg_ensure_init()) return NLG_ERR;
  FILE *f = fopen(path, "rb");
  if (!f) return nlg_fail("cannot open %s", path);
  if (fseeko(f, (off_t)offset, SEEK_SET) != 0) {
    fclose(f);
    return nlg_fail("cannot seek %s to %llu", path, (unsigned long long)offset);
  }
  if (!g_stage) {
    hipError_t e = hipHostMalloc((void **)&g_stage, 2 * kStageBytes, hipHostMallocDefault);
    if (e != hipSuccess) {
      g_stage = nullptr;
      fclose(f);
      return nlg_fail("hipHostMalloc staging failed: %s", hipGetErrorString(e));
    }
    (void)hipEventCreateWithFlags(&g_stage_ev[0], hipEventDisableTiming);
    (void)hipEventCreateWithFlags(&g_stage_ev[1], hipEventDisableTiming);
    (void)hipEventRecord(g_stage_ev[0], g_stream);
    (void)hipEventRecord(g_stage_ev[1], g_stream);
  }
  size_t done = 0, short_by = 0;
  int half = 0;
  while (done < bytes) {
    size_t n = bytes - done;
    if (n > kStageBytes) n = kStageBytes;
    char *buf = g_stage + (size_t)half * kStageBytes;
    // the copy that last used this half must be finished before refilling it
    NLG_HIP(hipEventSynchronize(g_stage_ev[half]));
    size_t got = fread(buf, 1, n, f);
    if (got < n) {
      memset(buf + got, 0, n - got);
      short_by = bytes - done - got;
    }
    NLG_HIP(hipMemcpyAsync((char *)dst + done, buf, n, hipMemcpyHostToDevice, g_stream));
    NLG_HIP(hipEventRecord(g_stage_ev[half], g_stream));
    done += n;
    half ^= 1;
    if (short_by) break;
  }
  fclose(f);
  if (short_by && done < bytes) {
    // the rest of the destination stays as nlg_malloc left it (zero)
  }
  nlg_tiled_refresh_range(dst, done, g_stream);
  NLG_LAUNCHED("tiled-copy refresh");
  NLG_HIP(hipStreamSynchronize(g_stream));
  if (missing) *missing = short_by;
  return NLG_OK;
}

extern "C" void *nlg_stream_create(void) {
  if (nlg_ensure_init()) return nullptr;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreate(&s);  // default priority (no priority streams)
  if (e != hipSuccess) {
    nlg_fail("hipStreamCreate failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  return (void *)s;
}
// Destroying a stream releases the batched-linear scratch the library keeps
// for it (after the stream's work is done); a graph captured on the stream
// must not be launched afterwards.
extern "C" int nlg_stream_destroy(void *s) {
  if (!s) return NLG_OK;
  NLG_HIP(hipStreamSynchronize((hipStream_t)s));
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    for (auto it = g_scratch.begin(); it != g_scratch.end();) {
      if (it->first.first == (hipStream_t)s) {
        for (void *p : it->second.bufs) (void)hipFree(p);
        it = g_scratch.erase(it);
      } else {
        ++it;
      }
    }
  }
  NLG_HIP(hipStreamDestroy((hipStream_t)s));
  return NLG_OK;
}
extern "C" int nlg_stream_sync(void *s) {
  if (nlg_ensure_init()) return NLG_ERR;
  NLG_HIP(hipStreamSynchronize(nlg_stream(s)));
  return NLG_OK;
}
extern "C" void *nlg_default_stream(void) {
  if (nlg_ensure_init()) return nullptr;
  return (void *)g_stream;
}

extern "C" void *nlg_event_create(void) {
  if (nlg_ensure_init()) return nullptr;
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) {
    nlg_fail("hipEventCreate failed");
    return nullptr;
  }
  return (void *)e;
}
extern "C" int nlg_event_destroy(void *ev) {
  if (ev) NLG_HIP(hipEventDestroy((hipEvent_t)ev));
  return NLG_OK;
}
extern "C" int nlg_event_record(void *ev, void *stream) {
  NLG_HIP(hipEventRecord((hipEvent_t)ev, nlg_stream(stream)));
  return NLG_OK;
}
extern "C" int nlg_event_elapsed_ms(void *a, void *b, float *ms) {
  NLG_HIP(hipEventSynchronize((hipEvent_t)b));
  NLG_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
  return NLG_OK;
}

extern "C" int nlg_graph_begin(void *stream) {
  if (nlg_ensure_init()) return NLG_ERR;
  NLG_HIP(hipStreamBeginCapture(nlg_stream(stream), hipStreamCaptureModeThreadLocal));
  return NLG_OK;
}
extern "C" int nlg_graph_end(void *stream, void **graph_exec) {
  hipGraph_t g = nullptr;
  NLG_HIP(hipStreamEndCapture(nlg_stream(stream), &g));
  hipGraphExec_t ge = nullptr;
  hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return nlg_fail("hipGraphInstantiate failed: %s", hipGetErrorString(e));
  *graph_exec = (void *)ge;
  return NLG_OK;
}
extern "C" int nlg_graph_launch(void *graph_exec, void *stream) {
  NLG_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, nlg_stream(stream)));
  return NLG_OK;
}
extern "C" int nlg_graph_destroy(void *graph_exec) {
  if (graph_exec) NLG_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  return NLG_OK;
}
