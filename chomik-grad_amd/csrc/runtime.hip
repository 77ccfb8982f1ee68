// libchomik_hip runtime: device bring-up, caching allocator, staged uploads,
// plan executor (hipGraph with per-node re-pointing), sampling, timing.
#include "chip.h"
#include "chomik_hip.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace chip {

namespace {

std::string g_error = "no error";
int g_device = -1;
hipStream_t g_stream = nullptr;
int* g_err_dev = nullptr;      // device error word
int* g_err_host = nullptr;     // pinned mirror for reads
int g_err_latched = 0;
int64_t* g_argmax_dev = nullptr;
int64_t* g_argmax_host = nullptr;
int64_t g_argmax_cap = 0;
bool g_debug = false;
bool g_use_graph = true;

int fail(int code, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_error = buffer;
  return code;
}

#define HIP_TRY(expr)                                                            \
  do {                                                                           \
    hipError_t status_ = (expr);                                                 \
    if (status_ != hipSuccess)                                                   \
      return fail(CHIP_EHIP, "%s failed: %s", #expr, hipGetErrorString(status_)); \
  } while (0)

#define NEED_INIT()                                                       \
  do {                                                                    \
    if (g_device < 0) return fail(CHIP_ENODEV, "chip_init was not called"); \
  } while (0)

// ------------------------------------------------------------ kind registry
std::vector<Planner>& registry() {
  static std::vector<Planner> table(64, nullptr);
  return table;
}

// ------------------------------------------------------------ allocator
// Size-binned caching pool.  Requests are rounded (512 B below 1 MiB, 2 MiB
// above) and a cached block is reused when it is at most 25% larger.
struct Pool {
  std::multimap<size_t, void*> free_blocks;
  std::unordered_map<void*, size_t> live;
  size_t in_use = 0, peak = 0, cached = 0;

  static size_t round(size_t n) {
    if (n == 0) n = 1;
    if (n < (1u << 20)) return (n + 511) & ~size_t(511);
    const size_t two_mib = size_t(2) << 20;
    return (n + two_mib - 1) / two_mib * two_mib;
  }

  int release_cached() {
    if (free_blocks.empty()) return CHIP_OK;
    HIP_TRY(hipStreamSynchronize(g_stream));
    for (auto& entry : free_blocks) HIP_TRY(hipFree(entry.second));
    free_blocks.clear();
    cached = 0;
    return CHIP_OK;
  }

  int allocate(size_t n, void** out) {
    const size_t size = round(n);
    auto it = free_blocks.lower_bound(size);
    if (it != free_blocks.end() && it->first <= size + size / 4) {
      *out = it->second;
      live[it->second] = it->first;
      in_use += it->first;
      cached -= it->first;
      free_blocks.erase(it);
    } else {
      void* ptr = nullptr;
      hipError_t status = hipMalloc(&ptr, size);
      if (status != hipSuccess) {
        (void)hipGetLastError();
        int rc = release_cached();
        if (rc) return rc;
        status = hipMalloc(&ptr, size);
        if (status != hipSuccess) {
          (void)hipGetLastError();
          return fail(CHIP_ENOMEM, "hipMalloc of %zu bytes failed: %s", size,
                      hipGetErrorString(status));
        }
      }
      live[ptr] = size;
      in_use += size;
      *out = ptr;
    }
    if (in_use > peak) peak = in_use;
    return CHIP_OK;
  }

  int release(void* ptr) {
    auto it = live.find(ptr);
    if (it == live.end()) return fail(CHIP_EINVAL, "chip_free of a pointer not from chip_malloc");
    free_blocks.emplace(it->second, ptr);
    in_use -= it->second;
    cached += it->second;
    live.erase(it);
    return CHIP_OK;
  }
};
Pool g_pool;

// ------------------------------------------------------------ staged upload
// Pinned ring for small asynchronous uploads; each region remembers the event
// of the copy that last read it.
struct Staging {
  static constexpr size_t kBytes = size_t(8) << 20;
  static constexpr int kRegions = 16;
  char* base = nullptr;
  size_t head = 0;
  struct Region { size_t begin, end; hipEvent_t done; bool busy; };
  std::vector<Region> regions;
  int next_region = 0;

  int init() {
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&base), kBytes, hipHostMallocDefault));
    regions.resize(kRegions);
    for (auto& r : regions) {
      r.busy = false;
      HIP_TRY(hipEventCreateWithFlags(&r.done, hipEventDisableTiming));
    }
    return CHIP_OK;
  }

  static bool overlaps(size_t a0, size_t a1, size_t b0, size_t b1) { return a0 < b1 && b0 < a1; }

  int upload(void* dst, const void* src, size_t n) {
    if (head + n > kBytes) head = 0;
    const size_t begin = head, end = head + n;
    for (auto& r : regions) {  // wait for earlier copies still reading this range
      if (r.busy && overlaps(begin, end, r.begin, r.end)) {
        HIP_TRY(hipEventSynchronize(r.done));
        r.busy = false;
      }
    }
    Region& slot = regions[next_region];
    next_region = (next_region + 1) % kRegions;
    if (slot.busy) {
      HIP_TRY(hipEventSynchronize(slot.done));
      slot.busy = false;
    }
    std::memcpy(base + begin, src, n);
    HIP_TRY(hipMemcpyAsync(dst, base + begin, n, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipEventRecord(slot.done, g_stream));
    slot.begin = begin;
    slot.end = end;
    slot.busy = true;
    head = (end + 255) & ~size_t(255);
    return CHIP_OK;
  }
};
Staging g_staging;

__global__ void k_fill_bytes(KArgs a) {
  // p[0] dst (uint8), n[0] bytes, n[1] byte value
  unsigned char* dst = static_cast<unsigned char*>(a.p[0]);
  const int64_t n = a.n[0];
  const unsigned char v = static_cast<unsigned char>(a.n[1]);
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = v;
}

__global__ void k_zero_word(int* word) { *word = 0; }

int check_errors_now() {
  HIP_TRY(hipStreamSynchronize(g_stream));
  HIP_TRY(hipMemcpy(g_err_host, g_err_dev, sizeof(int), hipMemcpyDeviceToHost));
  if (*g_err_host) {
    g_err_latched |= *g_err_host;
    const int bits = *g_err_host;
    hipLaunchKernelGGL(k_zero_word, dim3(1), dim3(1), 0, g_stream, g_err_dev);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipStreamSynchronize(g_stream));
    return fail(CHIP_EKERNEL, "kernel error bits 0x%x (%s%s%s)", bits,
                (bits & ERR_GATHER_INDEX) ? "gather index out of range " : "",
                (bits & ERR_POSITION) ? "position out of range " : "",
                (bits & ERR_SHAPE) ? "shape check failed" : "");
  }
  return CHIP_OK;
}

}  // namespace

void register_kind(int kind, Planner planner) {
  if (kind > 0 && kind < static_cast<int>(registry().size())) registry()[kind] = planner;
}
Planner planner_for(int kind) {
  if (kind <= 0 || kind >= static_cast<int>(registry().size())) return nullptr;
  return registry()[kind];
}
int* device_error_word() { return g_err_dev; }
hipStream_t library_stream() { return g_stream; }

// Argmax kernels live in k_llama.hip.
int launch_argmax(const void* src, int dtype, int64_t rows, int64_t cols, int64_t* out_dev,
                  hipStream_t stream);
int launch_greedy_advance(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                          void* tokens_out, void* history, int64_t step, void* position,
                          void* attention_mask, int64_t mask_row, void* write_mask,
                          int64_t write_row, int mask_dtype, int64_t cache_length,
                          hipStream_t stream);
int noalloc_setup(int device, hipStream_t stream);
int launch_greedy_advance_noalloc(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                                  void* tokens_out, void* history, int64_t step, void* position,
                                  void* attention_mask, int64_t mask_row, void* write_mask,
                                  int64_t write_row, int mask_dtype, int64_t cache_length,
                                  int device, hipStream_t stream);

// ------------------------------------------------------------ plans
struct Fixup {
  int index;      // which p[] entry
  int64_t slot;   // -1 = null
  int64_t offset; // bytes
};

struct Step {
  int kind = 0;
  KArgs args{};
  std::vector<Fixup> fixups;
  Launch launch;
  void* params[1] = {nullptr};
  hipGraphNode_t node = nullptr;
  bool dirty = true;
};

}  // namespace chip

struct chip_plan {
  std::vector<chip::Step> steps;
  std::vector<void*> slots;
  std::vector<std::vector<int>> users;  // slot -> steps using it
  std::vector<char> slot_dirty;
  int64_t arena_bytes = 0;
  void* arena = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

using namespace chip;

extern "C" {

const char* chip_last_error(void) { return g_error.c_str(); }

int chip_init(int device) {
  if (g_device == device) return CHIP_OK;
  if (g_device >= 0) return fail(CHIP_EINVAL, "library already bound to device %d", g_device);
  int count = 0;
  hipError_t status = hipGetDeviceCount(&count);
  if (status != hipSuccess || count <= 0)
    return fail(CHIP_ENODEV, "no HIP device available (%s)", hipGetErrorString(status));
  if (device < 0 || device >= count) return fail(CHIP_ENODEV, "device %d not present", device);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(CHIP_ENODEV, "device %d is %s; this library is built for gfx950", device,
                prop.gcnArchName);
  HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  HIP_TRY(hipMalloc(reinterpret_cast<void**>(&g_err_dev), 256));
  HIP_TRY(hipMemset(g_err_dev, 0, 256));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&g_err_host), 256, hipHostMallocDefault));
  int rc = g_staging.init();
  if (rc) return rc;
  rc = noalloc_setup(device, g_stream);  // the allocation-free entry points' static scratch
  if (rc) return rc;
  const char* debug = std::getenv("CHOMIK_HIP_DEBUG");
  g_debug = debug && debug[0] && debug[0] != '0';
  const char* graph = std::getenv("CHOMIK_HIP_GRAPH");
  g_use_graph = !(graph && graph[0] == '0') && !g_debug;
  HIP_TRY(hipDeviceSynchronize());
  g_device = device;
  return CHIP_OK;
}

int chip_device_info(chip_info* out) {
  NEED_INIT();
  if (!out) return fail(CHIP_EINVAL, "null info pointer");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, g_device));
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->wavefront_size = prop.warpSize;
  out->total_memory = prop.totalGlobalMem;
  out->lds_per_block = prop.sharedMemPerBlock;
  out->clock_khz = prop.clockRate;
  out->memory_clock_khz = prop.memoryClockRate;
  out->memory_bus_width = prop.memoryBusWidth;
  return CHIP_OK;
}

int chip_malloc(size_t nbytes, void** out) {
  NEED_INIT();
  if (!out) return fail(CHIP_EINVAL, "null output pointer");
  return g_pool.allocate(nbytes, out);
}

int chip_free(void* ptr) {
  NEED_INIT();
  if (!ptr) return CHIP_OK;
  return g_pool.release(ptr);
}

int chip_empty_cache(void) {
  NEED_INIT();
  return g_pool.release_cached();
}

int chip_memcpy_h2d(void* dst, const void* src, size_t nbytes, int async) {
  NEED_INIT();
  if (nbytes == 0) return CHIP_OK;
  if (!dst || !src) return fail(CHIP_EINVAL, "null pointer in chip_memcpy_h2d");
  if (async && nbytes <= Staging::kBytes / 4) return g_staging.upload(dst, src, nbytes);
  HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  return CHIP_OK;
}

int chip_memcpy_d2h(void* dst, const void* src, size_t nbytes) {
  NEED_INIT();
  if (nbytes == 0) return CHIP_OK;
  if (!dst || !src) return fail(CHIP_EINVAL, "null pointer in chip_memcpy_d2h");
  HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  return CHIP_OK;
}

int chip_memcpy_d2d(void* dst, const void* src, size_t nbytes) {
  NEED_INIT();
  if (nbytes == 0) return CHIP_OK;
  HIP_TRY(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, g_stream));
  return CHIP_OK;
}

int chip_memset(void* dst, int value, size_t nbytes) {
  NEED_INIT();
  if (nbytes == 0) return CHIP_OK;
  KArgs a{};
  a.p[0] = dst;
  a.n[0] = static_cast<int64_t>(nbytes);
  a.n[1] = value & 0xff;
  int64_t blocks = (static_cast<int64_t>(nbytes) + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_fill_bytes, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, g_stream, a);
  HIP_TRY(hipGetLastError());
  return CHIP_OK;
}

int chip_synchronize(void) {
  NEED_INIT();
  return check_errors_now();
}

int chip_errors(int* bits_out) {
  NEED_INIT();
  if (bits_out) *bits_out = g_err_latched;
  g_err_latched = 0;
  return CHIP_OK;
}

int chip_plan_create(const int64_t* tape, size_t n_words, chip_plan** out) {
  NEED_INIT();
  if (!tape || !out) return fail(CHIP_EINVAL, "null tape or output");
  size_t at = 0;
  auto take = [&](int64_t& value) -> bool {
    if (at >= n_words) return false;
    value = tape[at++];
    return true;
  };
  int64_t magic = 0, version = 0, n_slots = 0, n_steps = 0, arena = 0;
  if (!take(magic) || !take(version) || !take(n_slots) || !take(n_steps) || !take(arena))
    return fail(CHIP_EINVAL, "plan tape header truncated");
  if (magic != 0x43484950 || version != 1) return fail(CHIP_EINVAL, "bad plan tape magic/version");
  if (n_slots < 1 || n_slots > (1 << 20) || n_steps < 0 || n_steps > (1 << 20) || arena < 0)
    return fail(CHIP_EINVAL, "plan tape header out of range");

  auto plan = new chip_plan();
  plan->slots.assign(static_cast<size_t>(n_slots), nullptr);
  plan->users.resize(static_cast<size_t>(n_slots));
  plan->slot_dirty.assign(static_cast<size_t>(n_slots), 1);
  plan->arena_bytes = arena;
  plan->steps.resize(static_cast<size_t>(n_steps));
  auto bail = [&](int code) {
    delete plan;
    return code;
  };
  for (int64_t s = 0; s < n_steps; ++s) {
    Step& step = plan->steps[static_cast<size_t>(s)];
    int64_t kind = 0, n_ptr = 0, n_int = 0, n_float = 0;
    if (!take(kind) || !take(n_ptr) || !take(n_int) || !take(n_float))
      return bail(fail(CHIP_EINVAL, "step %lld header truncated", (long long)s));
    if (n_ptr < 0 || n_ptr > kMaxPtr || n_int < 0 || n_int > kMaxInt || n_float < 0 ||
        n_float > kMaxFloat)
      return bail(fail(CHIP_EINVAL, "step %lld has too many parameters", (long long)s));
    step.kind = static_cast<int>(kind);
    for (int64_t i = 0; i < n_ptr; ++i) {
      int64_t slot = 0, offset = 0;
      if (!take(slot) || !take(offset))
        return bail(fail(CHIP_EINVAL, "step %lld pointers truncated", (long long)s));
      if (slot < -1 || slot >= n_slots || offset < 0)
        return bail(fail(CHIP_EINVAL, "step %lld pointer %lld: bad slot %lld", (long long)s,
                         (long long)i, (long long)slot));
      step.fixups.push_back({static_cast<int>(i), slot, offset});
      if (slot >= 0) plan->users[static_cast<size_t>(slot)].push_back(static_cast<int>(s));
    }
    for (int64_t i = 0; i < n_int; ++i)
      if (!take(step.args.n[i])) return bail(fail(CHIP_EINVAL, "step ints truncated"));
    for (int64_t i = 0; i < n_float; ++i) {
      int64_t bits = 0;
      if (!take(bits)) return bail(fail(CHIP_EINVAL, "step floats truncated"));
      uint32_t word = static_cast<uint32_t>(bits);
      std::memcpy(&step.args.f[i], &word, sizeof(float));
    }
    Planner planner = planner_for(step.kind);
    if (!planner) return bail(fail(CHIP_EINVAL, "step %lld: unknown kind %d", (long long)s, step.kind));
    const char* problem = planner(step.args, step.launch);
    if (problem)
      return bail(fail(CHIP_EINVAL, "step %lld (kind %d): %s", (long long)s, step.kind, problem));
    if (!step.launch.func) return bail(fail(CHIP_EINVAL, "step %lld: planner chose no kernel", (long long)s));
    step.params[0] = &step.args;
  }
  if (at != n_words) return bail(fail(CHIP_EINVAL, "plan tape has trailing words"));
  if (arena > 0) {
    int rc = g_pool.allocate(static_cast<size_t>(arena), &plan->arena);
    if (rc) return bail(rc);
    plan->slots[0] = plan->arena;
  }
  *out = plan;
  return CHIP_OK;
}

int chip_plan_bind(chip_plan* plan, uint32_t slot, void* ptr) {
  if (!plan || slot == 0 || slot >= plan->slots.size())
    return fail(CHIP_EINVAL, "bad plan slot %u", slot);
  if (plan->slots[slot] != ptr) {
    plan->slots[slot] = ptr;
    plan->slot_dirty[slot] = 1;
  }
  return CHIP_OK;
}

int chip_plan_bind_many(chip_plan* plan, uint32_t n, const uint32_t* slots, void* const* ptrs) {
  for (uint32_t i = 0; i < n; ++i) {
    int rc = chip_plan_bind(plan, slots[i], ptrs[i]);
    if (rc) return rc;
  }
  return CHIP_OK;
}

static int resolve(chip_plan* plan, Step& step) {
  for (const Fixup& f : step.fixups) {
    if (f.slot < 0) {
      step.args.p[f.index] = nullptr;
      continue;
    }
    char* base = static_cast<char*>(plan->slots[static_cast<size_t>(f.slot)]);
    if (!base) return fail(CHIP_EINVAL, "plan slot %lld is unbound", (long long)f.slot);
    step.args.p[f.index] = base + f.offset;
  }
  return CHIP_OK;
}

static hipKernelNodeParams node_params(Step& step) {
  hipKernelNodeParams p{};
  p.func = const_cast<void*>(step.launch.func);
  p.gridDim = step.launch.grid;
  p.blockDim = step.launch.block;
  p.sharedMemBytes = static_cast<unsigned>(step.launch.shmem);
  p.kernelParams = step.params;
  p.extra = nullptr;
  return p;
}

int chip_plan_run(chip_plan* plan) {
  NEED_INIT();
  if (!plan) return fail(CHIP_EINVAL, "null plan");
  for (size_t s = 0; s < plan->slots.size(); ++s) {
    if (!plan->slot_dirty[s]) continue;
    for (int user : plan->users[s]) plan->steps[static_cast<size_t>(user)].dirty = true;
    plan->slot_dirty[s] = 0;
  }
  for (Step& step : plan->steps) {
    if (!step.dirty) continue;
    int rc = resolve(plan, step);
    if (rc) return rc;
  }
  if (!g_use_graph) {
    for (size_t s = 0; s < plan->steps.size(); ++s) {
      Step& step = plan->steps[s];
      step.dirty = false;
      HIP_TRY(hipLaunchKernel(step.launch.func, step.launch.grid, step.launch.block, step.params,
                              step.launch.shmem, g_stream));
      if (g_debug) {
        hipError_t status = hipStreamSynchronize(g_stream);
        if (status != hipSuccess)
          return fail(CHIP_EHIP, "step %zu (kind %d) failed: %s", s, step.kind,
                      hipGetErrorString(status));
        int rc = check_errors_now();
        if (rc) return fail(rc, "step %zu (kind %d): %s", s, step.kind, g_error.c_str());
      }
    }
    return CHIP_OK;
  }
  if (!plan->exec) {
    HIP_TRY(hipGraphCreate(&plan->graph, 0));
    hipGraphNode_t previous = nullptr;
    for (Step& step : plan->steps) {
      hipKernelNodeParams p = node_params(step);
      HIP_TRY(hipGraphAddKernelNode(&step.node, plan->graph, previous ? &previous : nullptr,
                                    previous ? 1 : 0, &p));
      previous = step.node;
      step.dirty = false;
    }
    HIP_TRY(hipGraphInstantiate(&plan->exec, plan->graph, nullptr, nullptr, 0));
  } else {
    for (Step& step : plan->steps) {
      if (!step.dirty) continue;
      hipKernelNodeParams p = node_params(step);
      HIP_TRY(hipGraphExecKernelNodeSetParams(plan->exec, step.node, &p));
      step.dirty = false;
    }
  }
  HIP_TRY(hipGraphLaunch(plan->exec, g_stream));
  return CHIP_OK;
}

int chip_plan_info(chip_plan* plan, int64_t* n_steps, int64_t* arena_bytes) {
  if (!plan) return fail(CHIP_EINVAL, "null plan");
  if (n_steps) *n_steps = static_cast<int64_t>(plan->steps.size());
  if (arena_bytes) *arena_bytes = plan->arena_bytes;
  return CHIP_OK;
}

int chip_plan_time_steps(chip_plan* plan, float* ms_out, int64_t capacity) {
  NEED_INIT();
  if (!plan || !ms_out) return fail(CHIP_EINVAL, "null plan or output");
  for (size_t s = 0; s < plan->slots.size(); ++s) {
    if (!plan->slot_dirty[s]) continue;
    for (int user : plan->users[s]) plan->steps[static_cast<size_t>(user)].dirty = true;
    plan->slot_dirty[s] = 0;
  }
  for (Step& step : plan->steps) {
    if (!step.dirty) continue;
    int rc = resolve(plan, step);
    if (rc) return rc;
    // the graph (if any) must still be re-pointed before its next launch
  }
  const size_t n = plan->steps.size();
  std::vector<hipEvent_t> events(2 * n);
  for (auto& e : events) HIP_TRY(hipEventCreate(&e));
  for (size_t s = 0; s < n; ++s) {
    Step& step = plan->steps[s];
    HIP_TRY(hipEventRecord(events[2 * s], g_stream));
    HIP_TRY(hipLaunchKernel(step.launch.func, step.launch.grid, step.launch.block, step.params,
                            step.launch.shmem, g_stream));
    HIP_TRY(hipEventRecord(events[2 * s + 1], g_stream));
  }
  HIP_TRY(hipStreamSynchronize(g_stream));
  for (size_t s = 0; s < n && static_cast<int64_t>(s) < capacity; ++s)
    HIP_TRY(hipEventElapsedTime(&ms_out[s], events[2 * s], events[2 * s + 1]));
  for (auto& e : events) (void)hipEventDestroy(e);
  return check_errors_now();
}

int chip_plan_time_repeat(chip_plan* plan, const int64_t* steps, int64_t n, int64_t rounds, float* ms_out) {
  NEED_INIT();
  if (!plan || !steps || !ms_out || n <= 0 || rounds <= 0) return fail(CHIP_EINVAL, "bad timing arguments");
  for (int64_t i = 0; i < n; ++i)
    if (steps[i] < 0 || steps[i] >= static_cast<int64_t>(plan->steps.size()))
      return fail(CHIP_EINVAL, "step index %lld out of range", static_cast<long long>(steps[i]));
  for (size_t s = 0; s < plan->slots.size(); ++s) {
    if (!plan->slot_dirty[s]) continue;
    for (int user : plan->users[s]) plan->steps[static_cast<size_t>(user)].dirty = true;
    plan->slot_dirty[s] = 0;
  }
  for (Step& step : plan->steps) {
    if (!step.dirty) continue;
    int rc = resolve(plan, step);
    if (rc) return rc;
  }
  hipEvent_t start, stop;
  HIP_TRY(hipEventCreate(&start));
  HIP_TRY(hipEventCreate(&stop));
  HIP_TRY(hipEventRecord(start, g_stream));
  for (int64_t r = 0; r < rounds; ++r)
    for (int64_t i = 0; i < n; ++i) {
      Step& step = plan->steps[static_cast<size_t>(steps[i])];
      HIP_TRY(hipLaunchKernel(step.launch.func, step.launch.grid, step.launch.block, step.params,
                              step.launch.shmem, g_stream));
    }
  HIP_TRY(hipEventRecord(stop, g_stream));
  HIP_TRY(hipEventSynchronize(stop));
  float ms = 0.f;
  HIP_TRY(hipEventElapsedTime(&ms, start, stop));
  *ms_out = ms / static_cast<float>(n * rounds);
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  return check_errors_now();
}

int chip_plan_destroy(chip_plan* plan) {
  if (!plan) return CHIP_OK;
  if (g_device >= 0) (void)hipStreamSynchronize(g_stream);
  if (plan->exec) (void)hipGraphExecDestroy(plan->exec);
  if (plan->graph) (void)hipGraphDestroy(plan->graph);
  if (plan->arena) (void)g_pool.release(plan->arena);
  delete plan;
  return CHIP_OK;
}

int chip_argmax(const void* src, int dtype, int64_t rows, int64_t cols, int64_t* out_host) {
  NEED_INIT();
  if (!src || !out_host || rows <= 0 || cols <= 0) return fail(CHIP_EINVAL, "bad argmax arguments");
  if (rows > g_argmax_cap) {
    if (g_argmax_dev) {
      HIP_TRY(hipStreamSynchronize(g_stream));
      HIP_TRY(hipFree(g_argmax_dev));
      HIP_TRY(hipHostFree(g_argmax_host));
    }
    const int64_t cap = rows < 1024 ? 1024 : rows;
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&g_argmax_dev), cap * sizeof(int64_t)));
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&g_argmax_host), cap * sizeof(int64_t),
                          hipHostMallocDefault));
    g_argmax_cap = cap;
  }
  int rc = launch_argmax(src, dtype, rows, cols, g_argmax_dev, g_stream);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(g_argmax_host, g_argmax_dev, rows * sizeof(int64_t),
                         hipMemcpyDeviceToHost, g_stream));
  rc = check_errors_now();
  if (rc) return rc;
  std::memcpy(out_host, g_argmax_host, rows * sizeof(int64_t));
  return CHIP_OK;
}

int chip_greedy_advance(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                        void* tokens_out, void* history, int64_t step, void* position,
                        void* attention_mask, int64_t mask_row, void* write_mask,
                        int64_t write_row, int mask_dtype, int64_t cache_length) {
  NEED_INIT();
  if (!logits || !tokens_out || rows <= 0 || cols <= 0)
    return fail(CHIP_EINVAL, "bad greedy-advance arguments");
  return launch_greedy_advance(logits, logits_dtype, rows, cols, tokens_out, history, step,
                               position, attention_mask, mask_row, write_mask, write_row,
                               mask_dtype, cache_length, g_stream);
}

int chip_greedy_advance_noalloc(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                                void* tokens_out, void* history, int64_t step, void* position,
                                void* attention_mask, int64_t mask_row, void* write_mask,
                                int64_t write_row, int mask_dtype, int64_t cache_length) {
  NEED_INIT();
  if (!logits || !tokens_out || rows <= 0 || cols <= 0)
    return fail(CHIP_EINVAL, "bad greedy-advance arguments");
  return launch_greedy_advance_noalloc(logits, logits_dtype, rows, cols, tokens_out, history, step,
                                       position, attention_mask, mask_row, write_mask, write_row,
                                       mask_dtype, cache_length, g_device, g_stream);
}

int chip_peak_memory(size_t* out) {
  if (out) *out = g_pool.peak;
  return CHIP_OK;
}

int chip_reset_peak_memory(void) {
  g_pool.peak = g_pool.in_use;
  return CHIP_OK;
}

int chip_event_create(void** out) {
  NEED_INIT();
  hipEvent_t event;
  HIP_TRY(hipEventCreate(&event));
  *out = event;
  return CHIP_OK;
}

int chip_event_record(void* event) {
  NEED_INIT();
  HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), g_stream));
  return CHIP_OK;
}

int chip_event_elapsed_ms(void* start, void* stop, float* ms) {
  NEED_INIT();
  HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return CHIP_OK;
}

int chip_event_destroy(void* event) {
  if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
  return CHIP_OK;
}

}  // extern "C"

namespace chip {
// Launch helpers used by other translation units for errors.
int set_error(int code, const char* message) { return fail(code, "%s", message); }
}  // namespace chip
