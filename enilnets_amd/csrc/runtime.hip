// Library lifecycle, errors, device memory, copies and event timing.
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace enq {

namespace {

thread_local std::string g_error;

struct DeviceState {
  bool ready = false;
  int device = -1;
  int cu_count = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t user_stream = nullptr;  // enq_set_stream
  void* workspace[2] = {nullptr, nullptr};
  size_t workspace_bytes[2] = {0, 0};
};

DeviceState g_state;
std::mutex g_mutex;
// captured graphs alive (enq_graph_end .. enq_graph_destroy): their kernels
// hold workspace addresses, so the workspace may not move meanwhile
int g_live_graphs = 0;

// The allocation-free entry point's scratch.  Host code never uses this name
// as an address (on the host it is only a stand-in for the symbol): enq_init
// asks the runtime for the array's address on each device it sets up, and
// noalloc_scratch hands out that address.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
void* g_scratch_addr[kMaxDevices] = {};

// Caching device allocator behind enq_malloc / enq_free.  Every kernel and
// copy of the library runs in order on one stream, so a freed block can be
// handed out again at once: whatever is enqueued on it next runs after the
// work that used it before.  Freeing therefore neither synchronises nor
// calls hipFree; blocks are kept per size class until enq_release_cached_memory
// (or an allocation that fails) returns them to the device.  Switching the
// stream (enq_set_stream) first synchronises the old one, which keeps that
// ordering argument true for the cached blocks.
struct BlockCache {
  std::mutex mu;
  std::unordered_map<void*, size_t> live;                  // block -> size class
  std::unordered_map<size_t, std::vector<void*>> idle;    // size class -> blocks
};
BlockCache g_blocks;

// 256 B .. 1 MiB in powers of two, then multiples of 2 MiB.
size_t size_class(size_t bytes) {
  if (bytes <= (size_t(1) << 20)) {
    size_t c = 256;
    while (c < bytes) c <<= 1;
    return c;
  }
  const size_t g = size_t(2) << 20;
  return (bytes + g - 1) / g * g;
}

// Returns every idle block to the device; the caller holds g_blocks.mu.
void release_idle_locked() {
  bool any = false;
  for (auto& kv : g_blocks.idle) any = any || !kv.second.empty();
  if (!any) return;
  ENQ_HIP(hipStreamSynchronize(stream()));
  for (auto& kv : g_blocks.idle)
    for (void* p : kv.second) ENQ_HIP(hipFree(p));
  g_blocks.idle.clear();
}

}  // namespace

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

const char* last_error() { return g_error.c_str(); }

void fail(int status, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  throw Failure{status};
}

void require_init() {
  if (!g_state.ready)
    fail(ENQ_ERR_NO_DEVICE, "enilnets_amd is not initialised: call enq_init(device) first");
  int cur = -1;
  ENQ_HIP(hipGetDevice(&cur));
  if (cur != g_state.device) ENQ_HIP(hipSetDevice(g_state.device));
}

hipStream_t stream() {
  return g_state.user_stream ? g_state.user_stream : g_state.own_stream;
}

int device_cu_count() { return g_state.cu_count; }

void* workspace(size_t bytes, int slot) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (slot != kKernelSlot && slot != kLayerSlot) fail(ENQ_ERR_RUNTIME, "bad workspace slot");
  if (bytes <= g_state.workspace_bytes[slot]) return g_state.workspace[slot];
  if (g_live_graphs > 0)
    fail(ENQ_ERR_INVALID,
         "this call needs %zu bytes of workspace, more than the %zu held while a captured "
         "graph is alive; destroy the graph first, or run this call once before capturing",
         bytes, g_state.workspace_bytes[slot]);
  // Round up so repeated small growth does not reallocate every call.
  size_t want = 1u << 20;
  while (want < bytes) want <<= 1;
  if (g_state.workspace[slot]) {
    // Earlier work on the stream may still read the old buffer.
    ENQ_HIP(hipStreamSynchronize(stream()));
    ENQ_HIP(hipFree(g_state.workspace[slot]));
    g_state.workspace[slot] = nullptr;
    g_state.workspace_bytes[slot] = 0;
  }
  ENQ_HIP(hipMalloc(&g_state.workspace[slot], want));
  g_state.workspace_bytes[slot] = want;
  return g_state.workspace[slot];
}

void* noalloc_scratch(size_t bytes) {
  ENQ_REQUIRE(bytes <= kNoAllocScratchBytes,
              "needs %zu bytes of scratch; the allocation-free entry point has %zu (64 MiB)",
              bytes, kNoAllocScratchBytes);
  void* p = g_scratch_addr[g_state.device];
  if (p == nullptr) fail(ENQ_ERR_RUNTIME, "scratch of device %d not set up", g_state.device);
  return p;
}

void check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    fail(ENQ_ERR_RUNTIME, "launch of %s failed: %s", what, hipGetErrorString(err));
}

}  // namespace enq

using namespace enq;

extern "C" {

int enq_abi_version(void) { return ENQ_ABI_VERSION; }

const char* enq_last_error(void) { return last_error(); }

int enq_init(int device) {
  return guarded([&] {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_state.ready && g_state.device == device) return;
    int count = 0;
    hipError_t err = hipGetDeviceCount(&count);
    if (err != hipSuccess || count == 0)
      fail(ENQ_ERR_NO_DEVICE, "no HIP device visible (%s)",
           err == hipSuccess ? "device count is 0" : hipGetErrorString(err));
    if (device < 0 || device >= count)
      fail(ENQ_ERR_INVALID, "device %d out of range [0, %d)", device, count);
    hipDeviceProp_t prop;
    ENQ_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      fail(ENQ_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only",
           device, prop.gcnArchName);
    if (g_state.ready) {
      ENQ_HIP(hipStreamSynchronize(g_state.own_stream));
      ENQ_HIP(hipStreamDestroy(g_state.own_stream));
      for (void* w : g_state.workspace)
        if (w) ENQ_HIP(hipFree(w));
      g_state = DeviceState{};
    }
    if (device >= kMaxDevices)
      fail(ENQ_ERR_INVALID, "device %d beyond the %d this library tracks", device, kMaxDevices);
    ENQ_HIP(hipSetDevice(device));
    if (g_scratch_addr[device] == nullptr) {
      // once per device, with that device current: its own copy of the array
      void* p = nullptr;
      ENQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      g_scratch_addr[device] = p;
    }
    hipStream_t s = nullptr;
    // Default priority on purpose: streams of mixed priority are avoided.
    ENQ_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    g_state.device = device;
    g_state.cu_count = prop.multiProcessorCount;
    g_state.own_stream = s;
    g_state.ready = true;
  });
}

int enq_get_device_info(enq_device_info* out) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(out != nullptr, "out is NULL");
    hipDeviceProp_t prop;
    ENQ_HIP(hipGetDeviceProperties(&prop, g_state.device));
    std::memset(out, 0, sizeof(*out));
    std::strncpy(out->name, prop.name, sizeof(out->name) - 1);
    std::strncpy(out->arch, prop.gcnArchName, sizeof(out->arch) - 1);
    out->device = g_state.device;
    out->compute_units = prop.multiProcessorCount;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width = prop.memoryBusWidth;
    out->l2_bytes = prop.l2CacheSize;
    out->lds_bytes_per_block = static_cast<int>(prop.sharedMemPerBlock);
    out->wavefront_size = prop.warpSize;
    out->global_memory_bytes = static_cast<long long>(prop.totalGlobalMem);
  });
}

int enq_synchronize(void) {
  return guarded([&] {
    require_init();
    ENQ_HIP(hipStreamSynchronize(stream()));
  });
}

int enq_get_stream(void** s) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(s != nullptr, "stream out-pointer is NULL");
    *s = stream();
  });
}

int enq_set_stream(void* s) {
  return guarded([&] {
    require_init();
    // cached blocks were last used on the old stream
    ENQ_HIP(hipStreamSynchronize(stream()));
    g_state.user_stream = static_cast<hipStream_t>(s);
  });
}

int enq_graph_begin(void) {
  return guarded([&] {
    require_init();
    ENQ_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeGlobal));
  });
}

int enq_graph_end(void** graph) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(graph != nullptr, "graph out-pointer is NULL");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    // ends the capture even when a captured call failed (then with an error)
    ENQ_HIP(hipStreamEndCapture(stream(), &g));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    ENQ_HIP(hipGraphDestroy(g));
    ENQ_HIP(err);
    std::lock_guard<std::mutex> lock(g_mutex);
    ++g_live_graphs;
    *graph = exec;
  });
}

int enq_graph_launch(void* graph) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(graph != nullptr, "graph is NULL");
    ENQ_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), stream()));
  });
}

int enq_graph_destroy(void* graph) {
  return guarded([&] {
    require_init();
    if (graph == nullptr) return;
    // replays still queued read the graph's buffers and code
    ENQ_HIP(hipStreamSynchronize(stream()));
    ENQ_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
    std::lock_guard<std::mutex> lock(g_mutex);
    --g_live_graphs;
  });
}

int enq_malloc(void** dptr, size_t bytes) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(dptr != nullptr, "dptr is NULL");
    *dptr = nullptr;
    if (bytes == 0) return;
    const size_t c = size_class(bytes);
    std::lock_guard<std::mutex> lock(g_blocks.mu);
    auto it = g_blocks.idle.find(c);
    void* p = nullptr;
    if (it != g_blocks.idle.end() && !it->second.empty()) {
      p = it->second.back();
      it->second.pop_back();
    } else if (hipMalloc(&p, c) != hipSuccess) {
      (void)hipGetLastError();
      release_idle_locked();  // give the cached blocks back and try once more
      ENQ_HIP(hipMalloc(&p, c));
    }
    g_blocks.live[p] = c;
    *dptr = p;
  });
}

int enq_free(void* dptr) {
  return guarded([&] {
    require_init();
    if (dptr == nullptr) return;
    std::lock_guard<std::mutex> lock(g_blocks.mu);
    auto it = g_blocks.live.find(dptr);
    ENQ_REQUIRE(it != g_blocks.live.end(), "enq_free: %p was not allocated by enq_malloc",
                dptr);
    g_blocks.idle[it->second].push_back(dptr);
    g_blocks.live.erase(it);
  });
}

int enq_release_cached_memory(void) {
  return guarded([&] {
    require_init();
    std::lock_guard<std::mutex> lock(g_blocks.mu);
    release_idle_locked();
  });
}

int enq_copy_to_device(void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    require_init();
    if (bytes == 0) return;
    ENQ_REQUIRE(dst && src, "NULL pointer in copy");
    ENQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()));
    ENQ_HIP(hipStreamSynchronize(stream()));
  });
}

int enq_copy_to_host(void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    require_init();
    if (bytes == 0) return;
    ENQ_REQUIRE(dst && src, "NULL pointer in copy");
    ENQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream()));
    ENQ_HIP(hipStreamSynchronize(stream()));
  });
}

int enq_copy_on_device(void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    require_init();
    if (bytes == 0) return;
    ENQ_REQUIRE(dst && src, "NULL pointer in copy");
    ENQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()));
    ENQ_HIP(hipStreamSynchronize(stream()));
  });
}

int enq_event_create(void** event) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(event != nullptr, "event out-pointer is NULL");
    hipEvent_t e;
    ENQ_HIP(hipEventCreate(&e));
    *event = e;
  });
}

int enq_event_destroy(void* event) {
  return guarded([&] {
    require_init();
    if (event) ENQ_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  });
}

int enq_event_record(void* event) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(event != nullptr, "event is NULL");
    ENQ_HIP(hipEventRecord(static_cast<hipEvent_t>(event), stream()));
  });
}

int enq_event_elapsed_ms(void* start, void* end, float* ms) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(start && end && ms, "NULL argument");
    ENQ_HIP(hipEventSynchronize(static_cast<hipEvent_t>(end)));
    ENQ_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                static_cast<hipEvent_t>(end)));
  });
}

}  // extern "C"
