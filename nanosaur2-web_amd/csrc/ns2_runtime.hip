// Runtime half of the C ABI: device selection, errors, stream, buffer pool, workspace,
// copies and timing events. Replaces the WebGPU runtime of app/gpu/device.js.
#include <math.h>
#include <stdarg.h>
#include <string.h>

#include <map>
#include <string>
#include <mutex>
#include <vector>

#include "ns2_common.h"

namespace ns2 {

static thread_local char g_error[1024] = "";
static bool g_init = false;
static int g_device = 0;
static hipStream_t g_stream = nullptr;
static hipStream_t g_own_stream = nullptr;  // the library's stream when the caller sets none

// ---- graph capture state ------------------------------------------------------------------
// While a capture is open or a recorded graph is alive, device memory that a graph may address
// is never freed: workspace buffers that grow are retired (freed when the last graph goes) and
// the pool keeps its cached buffers.
static bool g_capturing = false;
static int g_graphs = 0;
static std::vector<void*> g_retired;

// ---- staging of small host-to-device copies ------------------------------------------------
// Pinned slots (allocated on first use, held until the process ends), each with the event of the
// last copy that read it.
constexpr size_t kStageBytes = 64 << 10;
constexpr int kStageSlots = 16;
struct Stage {
  std::mutex mu;
  void* base = nullptr;
  hipEvent_t done[kStageSlots] = {};
  bool used[kStageSlots] = {};
  int next = 0;
};
static Stage g_stage;

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = 0; }
hipStream_t stream() { return g_stream; }
bool initialised() { return g_init; }

// ---- buffer pool: size buckets of app/gpu/device.js:33-39 ------------------------------
struct Pool {
  std::mutex mu;
  std::map<size_t, std::vector<void*>> free_lists;
  size_t allocated = 0;
  size_t peak = 0;
};
static Pool g_pool;

// ---- workspace ----------------------------------------------------------------------------
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
static Workspace g_ws[kWorkspaceSlots];

void* workspace(int slot, size_t bytes) {
  if (slot < 0 || slot >= kWorkspaceSlots) return nullptr;
  Workspace& w = g_ws[slot];
  if (w.bytes >= bytes && w.ptr) return w.ptr;
  if (w.ptr) {
    if (g_capturing || g_graphs > 0) {
      // a graph (recorded or being recorded) may address the old buffer
      g_retired.push_back(w.ptr);
    } else {
      // the old buffer may still be read by queued kernels: wait before freeing it
      if (hipStreamSynchronize(g_stream) != hipSuccess) return nullptr;
      if (hipFree(w.ptr) != hipSuccess) return nullptr;
    }
    w.ptr = nullptr;
    w.bytes = 0;
  }
  size_t want = bytes + bytes / 4 + 4096;
  if (hipMalloc(&w.ptr, want) != hipSuccess) {
    w.ptr = nullptr;
    return nullptr;
  }
  w.bytes = want;
  return w.ptr;
}

// ---- fixed scratch of the allocation-free entry points ------------------------------------
// A file-scope device array: every GPU the library runs on holds its own copy, at its own
// address, until the process ends. Its name is only a host-side stand-in for the symbol: host
// code uses the address that ns2_init resolves per device with hipGetSymbolAddress, never the
// name itself.
static __device__ __align__(256) unsigned char scratch[NS2_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];

void* noalloc_scratch() { return g_init && g_device < kMaxDevices ? g_scratch[g_device] : nullptr; }

// ---- kernel profiler -----------------------------------------------------------------------
struct ProfPending {
  const char* name;
  hipEvent_t a, b;
};
struct ProfStat {
  long long count = 0;
  double ms = 0;
};
static bool g_prof_on = false;
static std::vector<ProfPending> g_prof_pending;
static std::vector<hipEvent_t> g_prof_spare;
static std::map<std::string, ProfStat> g_prof_stats;

static hipEvent_t prof_event() {
  if (!g_prof_spare.empty()) {
    hipEvent_t e = g_prof_spare.back();
    g_prof_spare.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void prof_begin(const char* name) {
  if (!g_prof_on) return;
  hipEvent_t a = prof_event();
  if (!a) return;
  (void)hipEventRecord(a, g_stream);
  g_prof_pending.push_back({name, a, nullptr});
}

void prof_end() {
  if (!g_prof_on || g_prof_pending.empty() || g_prof_pending.back().b) return;
  hipEvent_t b = prof_event();
  if (!b) return;
  (void)hipEventRecord(b, g_stream);
  g_prof_pending.back().b = b;
}

static int prof_collect() {
  for (auto& p : g_prof_pending) {
    if (p.b) {
      float ms = 0;
      NS2_HIP(hipEventSynchronize(p.b));
      NS2_HIP(hipEventElapsedTime(&ms, p.a, p.b));
      ProfStat& s = g_prof_stats[p.name];
      s.count++;
      s.ms += ms;
      g_prof_spare.push_back(p.b);
    }
    g_prof_spare.push_back(p.a);
  }
  g_prof_pending.clear();
  return NS2_OK;
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t value, size_t count) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) p[i] = value;
}

}  // namespace ns2

using namespace ns2;

extern "C" {

const char* ns2_last_error(void) { return g_error; }

int ns2_init(int device) {
  clear_error();
  int n = 0;
  NS2_HIP(hipGetDeviceCount(&n));
  NS2_REQUIRE(device >= 0 && device < n, "ns2_init: device %d out of range (%d devices)", device, n);
  NS2_REQUIRE(device < kMaxDevices, "ns2_init: device %d beyond the %d this library tracks", device, kMaxDevices);
  NS2_HIP(hipSetDevice(device));
  g_device = device;
  // this device's copy of the allocation-free entry points' scratch array (once per device,
  // with the device current)
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    NS2_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch[device] = ptr;
  }
  // launches go to a stream of the library's own (default priority) unless the caller sets
  // one: the legacy null stream cannot be captured into a graph
  if (!g_own_stream) NS2_HIP(hipStreamCreate(&g_own_stream));
  if (!g_stream) g_stream = g_own_stream;
  g_init = true;
  return NS2_OK;
}

int ns2_device_info(char* name, size_t cap, int* compute_units, size_t* hbm_bytes) {
  NS2_READY();
  hipDeviceProp_t p;
  NS2_HIP(hipGetDeviceProperties(&p, g_device));
  if (name && cap) {
    snprintf(name, cap, "%s (%s)", p.name, p.gcnArchName);
  }
  if (compute_units) *compute_units = p.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
  return NS2_OK;
}

int ns2_set_stream(void* hip_stream) {
  g_stream = (hipStream_t)hip_stream;
  return NS2_OK;
}

void* ns2_get_stream(void) { return (void*)g_stream; }

int ns2_malloc(void** ptr, size_t bytes) {
  NS2_READY();
  NS2_REQUIRE(ptr != nullptr, "ns2_malloc: null out-pointer");
  // padded to 16 bytes like app/gpu/device.js:135 (vector-loadable tails)
  size_t size = bytes < 16 ? 16 : (bytes + 15) / 16 * 16;
  if (hipMalloc(ptr, size) != hipSuccess) {
    *ptr = nullptr;
    (void)hipGetLastError();
    return set_error(NS2_ERR_OOM, "ns2_malloc: out of device memory for %zu bytes", size);
  }
  return NS2_OK;
}

int ns2_free(void* ptr) {
  if (!ptr) return NS2_OK;
  NS2_READY();
  // a kernel still queued may read the buffer
  NS2_HIP(hipStreamSynchronize(g_stream));
  NS2_HIP(hipFree(ptr));
  return NS2_OK;
}

size_t ns2_pool_round(size_t bytes) {
  size_t b = bytes < 256 ? 256 : bytes;
  size_t p = 1;
  while (p <= b / 2) p <<= 1;  // largest power of two <= b
  size_t step = p / 8 < 256 ? 256 : p / 8;
  return (b + step - 1) / step * step;
}

int ns2_pool_get(size_t bytes, void** ptr, size_t* rounded) {
  NS2_READY();
  NS2_REQUIRE(ptr != nullptr, "ns2_pool_get: null out-pointer");
  size_t size = ns2_pool_round(bytes);
  if (rounded) *rounded = size;
  {
    std::lock_guard<std::mutex> lk(g_pool.mu);
    auto it = g_pool.free_lists.find(size);
    if (it != g_pool.free_lists.end() && !it->second.empty()) {
      *ptr = it->second.back();
      it->second.pop_back();
      return NS2_OK;
    }
  }
  if (hipMalloc(ptr, size) != hipSuccess) {
    *ptr = nullptr;
    (void)hipGetLastError();
    return set_error(NS2_ERR_OOM, "ns2_pool_get: out of device memory for %zu bytes", size);
  }
  std::lock_guard<std::mutex> lk(g_pool.mu);
  g_pool.allocated += size;
  if (g_pool.allocated > g_pool.peak) g_pool.peak = g_pool.allocated;
  return NS2_OK;
}

int ns2_pool_put(void* ptr, size_t rounded) {
  if (!ptr) return NS2_OK;
  NS2_REQUIRE(rounded == ns2_pool_round(rounded), "ns2_pool_put: %zu is not a bucket size", rounded);
  std::lock_guard<std::mutex> lk(g_pool.mu);
  g_pool.free_lists[rounded].push_back(ptr);
  return NS2_OK;
}

int ns2_pool_trim(void) {
  NS2_READY();
  if (g_capturing || g_graphs > 0) return NS2_OK;  // recorded graphs may address cached buffers
  NS2_HIP(hipStreamSynchronize(g_stream));
  std::lock_guard<std::mutex> lk(g_pool.mu);
  for (auto& kv : g_pool.free_lists) {
    for (void* p : kv.second) {
      NS2_HIP(hipFree(p));
      g_pool.allocated -= kv.first;
    }
  }
  g_pool.free_lists.clear();
  return NS2_OK;
}

int ns2_pool_stats(size_t* allocated, size_t* peak) {
  std::lock_guard<std::mutex> lk(g_pool.mu);
  if (allocated) *allocated = g_pool.allocated;
  if (peak) *peak = g_pool.peak;
  return NS2_OK;
}

int ns2_h2d(void* dst, const void* src, size_t bytes) {
  NS2_READY();
  if (!bytes) return NS2_OK;
  NS2_REQUIRE(dst && src, "ns2_h2d: null pointer");
  NS2_REQUIRE(!g_capturing, "ns2_h2d: no uploads inside a graph capture");
  if (bytes <= kStageBytes) {
    // small copies (the per-pass timestep embedding): through a ring of pinned staging slots,
    // queued on the stream without waiting for the work before it; a slot is reused once the
    // copy that last read it has run
    std::lock_guard<std::mutex> lock(g_stage.mu);
    if (!g_stage.base) {
      NS2_HIP(hipHostMalloc(&g_stage.base, kStageBytes * kStageSlots, hipHostMallocDefault));
      for (int i = 0; i < kStageSlots; ++i) NS2_HIP(hipEventCreateWithFlags(&g_stage.done[i], hipEventDisableTiming));
    }
    const int i = g_stage.next;
    g_stage.next = (i + 1) % kStageSlots;
    if (g_stage.used[i]) NS2_HIP(hipEventSynchronize(g_stage.done[i]));
    char* slot = static_cast<char*>(g_stage.base) + (size_t)i * kStageBytes;
    memcpy(slot, src, bytes);
    NS2_HIP(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, g_stream));
    NS2_HIP(hipEventRecord(g_stage.done[i], g_stream));
    g_stage.used[i] = true;
    return NS2_OK;
  }
  // pageable source: the copy has completed reading src when this returns
  NS2_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  NS2_HIP(hipStreamSynchronize(g_stream));
  return NS2_OK;
}

int ns2_d2h(void* dst, const void* src, size_t bytes) {
  NS2_READY();
  if (!bytes) return NS2_OK;
  NS2_REQUIRE(dst && src, "ns2_d2h: null pointer");
  NS2_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  NS2_HIP(hipStreamSynchronize(g_stream));
  return NS2_OK;
}

int ns2_sync(void) {
  NS2_READY();
  NS2_HIP(hipStreamSynchronize(g_stream));
  NS2_HIP(hipGetLastError());
  return NS2_OK;
}

int ns2_fill_u32(void* dst, uint32_t value, size_t count) {
  NS2_READY();
  if (!count) return NS2_OK;
  NS2_REQUIRE(dst != nullptr, "ns2_fill_u32: null pointer");
  size_t blocks = (count + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  fill_u32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, g_stream>>>((uint32_t*)dst, value, count);
  NS2_LAUNCHED("fill_u32");
  return NS2_OK;
}

int ns2_event_create(void** ev) {
  NS2_READY();
  NS2_REQUIRE(ev != nullptr, "ns2_event_create: null out-pointer");
  hipEvent_t e;
  NS2_HIP(hipEventCreate(&e));
  *ev = (void*)e;
  return NS2_OK;
}

int ns2_event_record(void* ev) {
  NS2_READY();
  NS2_REQUIRE(ev != nullptr, "ns2_event_record: null event");
  NS2_HIP(hipEventRecord((hipEvent_t)ev, g_stream));
  return NS2_OK;
}

int ns2_event_elapsed(void* start, void* end, float* ms) {
  NS2_READY();
  NS2_REQUIRE(start && end && ms, "ns2_event_elapsed: null argument");
  NS2_HIP(hipEventSynchronize((hipEvent_t)end));
  NS2_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return NS2_OK;
}

int ns2_event_destroy(void* ev) {
  if (!ev) return NS2_OK;
  NS2_HIP(hipEventDestroy((hipEvent_t)ev));
  return NS2_OK;
}

int ns2_profile_enable(int on) {
  NS2_READY();
  NS2_REQUIRE(!(on && g_capturing), "ns2_profile_enable: a graph capture is open");
  if (!on) {
    int rc = prof_collect();
    if (rc) return rc;
  }
  g_prof_on = on != 0;
  return NS2_OK;
}

int ns2_profile_reset(void) {
  NS2_READY();
  int rc = prof_collect();
  if (rc) return rc;
  g_prof_stats.clear();
  return NS2_OK;
}

int ns2_profile_report(char* buf, size_t cap) {
  NS2_READY();
  NS2_REQUIRE(buf && cap > 2, "ns2_profile_report: null or tiny buffer");
  int rc = prof_collect();
  if (rc) return rc;
  std::string s = "{";
  bool first = true;
  for (const auto& kv : g_prof_stats) {
    char line[256];
    snprintf(line, sizeof(line), "%s\"%s\": {\"count\": %lld, \"ms\": %.6f}", first ? "" : ", ",
             kv.first.c_str(), kv.second.count, kv.second.ms);
    s += line;
    first = false;
  }
  s += "}";
  NS2_REQUIRE(s.size() < cap, "ns2_profile_report: buffer of %zu bytes too small (%zu needed)", cap, s.size() + 1);
  memcpy(buf, s.c_str(), s.size() + 1);
  return NS2_OK;
}


// ---- HIP graphs ------------------------------------------------------------------------------
// The recorded analogue of the reference's command-buffer batching (app/gpu/device.js:196-215):
// every launch issued between ns2_graph_begin and ns2_graph_end is recorded (not run) and
// ns2_graph_launch replays the whole sequence with one call.

int ns2_graph_begin(void) {
  NS2_READY();
  NS2_REQUIRE(!g_capturing, "ns2_graph_begin: a capture is already open");
  NS2_REQUIRE(!g_prof_on, "ns2_graph_begin: disable the kernel profiler before capturing");
  NS2_REQUIRE(g_stream != nullptr, "ns2_graph_begin: the null stream cannot be captured (ns2_set_stream)");
  NS2_HIP(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed));
  g_capturing = true;
  return NS2_OK;
}

int ns2_graph_end(void** graph) {
  NS2_READY();
  NS2_REQUIRE(g_capturing, "ns2_graph_end: no capture is open");
  g_capturing = false;
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(g_stream, &g);
  if (e != hipSuccess || !g) {
    (void)hipGetLastError();
    if (g) (void)hipGraphDestroy(g);
    return set_error(NS2_ERR_HIP, "ns2_graph_end: the capture failed (%s); calls that wait for the stream "
                     "(reads, writes, sync) cannot be recorded", hipGetErrorString(e));
  }
  hipGraphExec_t x = nullptr;
  const hipError_t e2 = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e2 != hipSuccess) {
    (void)hipGetLastError();
    return set_error(NS2_ERR_HIP, "ns2_graph_end: hipGraphInstantiate: %s", hipGetErrorString(e2));
  }
  if (!graph) {
    (void)hipGraphExecDestroy(x);
    return set_error(NS2_ERR_INVALID, "ns2_graph_end: null out-pointer (the graph was discarded)");
  }
  g_graphs++;
  *graph = (void*)x;
  return NS2_OK;
}

int ns2_graph_launch(void* graph) {
  NS2_READY();
  NS2_REQUIRE(graph != nullptr, "ns2_graph_launch: null graph");
  NS2_REQUIRE(!g_capturing, "ns2_graph_launch: a capture is open");
  NS2_HIP(hipGraphLaunch((hipGraphExec_t)graph, g_stream));
  return NS2_OK;
}

int ns2_graph_destroy(void* graph) {
  NS2_READY();
  if (!graph) return NS2_OK;
  NS2_REQUIRE(g_graphs > 0, "ns2_graph_destroy: no live graph");
  NS2_HIP(hipStreamSynchronize(g_stream));
  NS2_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
  if (--g_graphs == 0 && !g_capturing) {
    for (void* p : g_retired) NS2_HIP(hipFree(p));
    g_retired.clear();
  }
  return NS2_OK;
}

}  // extern "C"
