// runtime.cpp - TInferCuda of the reference (src/infer/mormot.ai.infer.cuda.pas
// :179-771) for HIP: device, a non-blocking stream, the gfx950 code objects
// embedded in this library and loaded with hipModuleLoadData, buffers,
// copies, events and stream capture into graphs.
#include <cstdio>
#include <cstring>

#include "internal.h"

// hip_ext.h's launch with per-dispatch timing events (the header itself needs
// the HIP compiler; the library is built by the host one)
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz,
                                               uint32_t lx, uint32_t ly, uint32_t lz, size_t shmem,
                                               hipStream_t stream, void** params, void** extra,
                                               hipEvent_t start, hipEvent_t stop, uint32_t flags);

// the code objects, linked in by embed.S (.incbin of the built .hsaco
// files): ihip_co_count pairs of (begin, end)
extern "C" const char* const ihip_co_table[];
extern "C" const int ihip_co_count;

namespace ihip {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg)
{
  g_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what)
{
  g_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return (int)e;
}

hipFunction_t kernel(ihip_ctx* c, const char* name)
{
  auto it = c->kernels.find(name);
  if (it != c->kernels.end()) return it->second;
  for (auto& m : c->modules) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, m.mod, name) == hipSuccess && f) {
      c->kernels.emplace(name, f);
      return f;
    }
  }
  (void)hipGetLastError();
  return nullptr;
}

int resident_blocks(ihip_ctx* c, const char* name, int block, size_t shmem)
{
  const std::string key = std::string(name) + ":" + std::to_string(block) + ":" + std::to_string(shmem);
  auto it = c->resident.find(key);
  if (it != c->resident.end()) return it->second;
  int n = 1;
  hipFunction_t f = kernel(c, name);
  if (!f || hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, block, shmem) != hipSuccess ||
      n < 1) {
    (void)hipGetLastError();
    n = 1;
  }
  c->resident.emplace(key, n);
  return n;
}

int launch(ihip_ctx* c, const char* name, dim3 grid, dim3 block, void* args, size_t shmem)
{
  hipFunction_t f = kernel(c, name);
  if (!f) return fail(IHIP_E_UNSUPPORTED, std::string("no kernel ") + name);
  if (grid.x == 0 || grid.y == 0 || grid.z == 0)
    return fail(IHIP_E_ARG, std::string("empty grid for ") + name);
  void* params[] = {args};
  hipError_t e;
  // a timing build: this launch's stamps into its own buffer
  const bool traced = !c->trace_prefix.empty() && !c->capturing &&
                      c->trace_used + 1 < c->trace_ptrs.size() &&
                      strncmp(name, c->trace_prefix.c_str(), c->trace_prefix.size()) == 0;
  if (traced)
    for (uint64_t g : c->trace_globals) {
      e = hipMemcpyHtoDAsync((hipDeviceptr_t)g, &c->trace_ptrs[c->trace_used], 8, c->stream);
      if (e != hipSuccess) return hip_fail(e, "trace");
    }
  if (!c->timer_prefix.empty() && !c->capturing && c->timer_used * 2 < c->timer_events.size() &&
      (c->timer_prefix == "*" || strncmp(name, c->timer_prefix.c_str(), c->timer_prefix.size()) == 0)) {
    // the dispatch's own start and end (the times a profiler reports)
    c->timer_names[c->timer_used] = name;
    hipEvent_t* ev = &c->timer_events[2 * c->timer_used++];
    e = hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x,
                                 block.y, block.z, shmem, c->stream, params, nullptr, ev[0], ev[1], 0);
  } else {
    e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)shmem,
                              c->stream, params, nullptr);
  }
  if (e != hipSuccess) return hip_fail(e, name);
  if (traced) {
    c->trace_used++;
    for (uint64_t g : c->trace_globals) {
      e = hipMemcpyHtoDAsync((hipDeviceptr_t)g, &c->trace_ptrs.back(), 8, c->stream);
      if (e != hipSuccess) return hip_fail(e, "trace");
    }
  }
  return 0;
}

int scratch(ihip_ctx* c, uint64_t& buf, uint64_t& cap, uint64_t bytes)
{
  if (buf && cap >= bytes) return 0;
  if (c->capturing) return fail(IHIP_E_CAPTURE, "scratch growth while capturing");
  if (buf) {
    IHIP_CHECK(hipStreamSynchronize(c->stream));
    IHIP_CHECK(hipFree((void*)buf));
    buf = 0;
    cap = 0;
  }
  uint64_t n = bytes + bytes / 4 + 256;
  void* p = nullptr;
  IHIP_CHECK(hipMalloc(&p, n));
  buf = (uint64_t)p;
  cap = n;
  return 0;
}

}  // namespace ihip

using namespace ihip;

extern "C" {

const char* ihip_last_error(void) { return g_error.c_str(); }

int ihip_available(void)
{
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int usable = 0;
  for (int i = 0; i < n; i++) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0)
      usable++;
  }
  return usable;
}

int ihip_create(int device, ihip_ctx** out)
{
  if (!out) return fail(IHIP_E_ARG, "ihip_create: no out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
    (void)hipGetLastError();
    return fail(IHIP_E_NODEVICE, "ihip_create: no HIP device " + std::to_string(device));
  }
  hipDeviceProp_t p;
  IHIP_CHECK(hipGetDeviceProperties(&p, device));
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return fail(IHIP_E_NODEVICE, std::string("ihip_create: device is ") + p.gcnArchName +
                                     ", the code objects are for gfx950");
  IHIP_CHECK(hipSetDevice(device));
  ihip_ctx* c = new ihip_ctx();
  c->device = device;
  c->cus = p.multiProcessorCount;
  if (const char* v = getenv("IHIP_GEMV_BLOCKS_PER_CU")) c->gemv_blocks_per_cu = std::max(1, atoi(v));
  if (const char* v = getenv("IHIP_GEMM")) c->use_gemm = atoi(v) != 0;
  if (const char* v = getenv("IHIP_GEMM_MIN_ROWS")) c->gemm_min_rows = std::max(GEMM_TILE_ROWS, atoi(v));
  if (const char* v = getenv("IHIP_GEMM_MIN_ROWS_FLOAT"))
    c->gemm_min_rows_float = std::max(GEMM_TILE_ROWS, atoi(v));
  if (const char* v = getenv("IHIP_GEMV_HOLD")) c->gemv_hold = std::max(1, atoi(v));
  if (const char* v = getenv("IHIP_ATTN_MFMA")) c->attn_mfma = atoi(v) != 0;
  if (const char* v = getenv("IHIP_GEMM8")) c->use_gemm8 = atoi(v) != 0;
  if (const char* v = getenv("IHIP_GEMM_SPLIT")) c->gemm_split = atoi(v) != 0;
  if (const char* v = getenv("IHIP_GEMM_F8")) c->gemm_f8 = atoi(v) != 0;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  for (int i = 0; i < ihip_co_count; i++) {
    Module m;
    e = hipModuleLoadData(&m.mod, ihip_co_table[2 * i]);
    if (e != hipSuccess) {
      ihip_destroy(c);
      return hip_fail(e, "hipModuleLoadData");
    }
    c->modules.push_back(m);
  }
  for (auto& ev : c->events) {
    if (hipEventCreate(&ev) != hipSuccess) {
      ihip_destroy(c);
      return fail(IHIP_E_NODEVICE, "hipEventCreate");
    }
  }
  void* bad = nullptr;
  if (hipMalloc(&bad, 256) != hipSuccess) {
    ihip_destroy(c);
    return fail(IHIP_E_NOMEM, "hipMalloc");
  }
  c->scratch_bad = (uint64_t)bad;
  void* am = nullptr;
  if (hipMalloc(&am, ARGMAX_PARTS * 8) != hipSuccess) {
    ihip_destroy(c);
    return fail(IHIP_E_NOMEM, "hipMalloc");
  }
  c->scratch_argmax = (uint64_t)am;
  if (int rc = static_scratch_init(c)) {
    ihip_destroy(c);
    return rc;
  }
  *out = c;
  return 0;
}

void ihip_destroy(ihip_ctx* c)
{
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  static_scratch_release(c);
  for (int i = 0; i < 16; i++) {
    if (c->execs[i]) (void)hipGraphExecDestroy(c->execs[i]);
    if (c->graphs[i]) (void)hipGraphDestroy(c->graphs[i]);
  }
  for (auto& w : c->weights) (void)hipFree((void*)w.dev);
  for (auto a : c->allocations) (void)hipFree((void*)a);
  for (uint64_t b : {c->scratch_x, c->scratch_y, c->scratch_q, c->scratch_bad, c->scratch_attn,
                     c->scratch_argmax, c->scratch_split, c->scratch_planes})
    if (b) (void)hipFree((void*)b);
  for (auto ev : c->events)
    if (ev) (void)hipEventDestroy(ev);
  for (auto ev : c->timer_events) (void)hipEventDestroy(ev);
  for (auto& m : c->modules)
    if (m.mod) (void)hipModuleUnload(m.mod);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

int ihip_device_info(ihip_ctx* c, char* name, int name_len, uint64_t* total_mem, int* cus)
{
  if (!c) return fail(IHIP_E_ARG, "no context");
  hipDeviceProp_t p;
  IHIP_CHECK(hipGetDeviceProperties(&p, c->device));
  if (name && name_len > 0) {
    snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
  }
  if (total_mem) *total_mem = p.totalGlobalMem;
  if (cus) *cus = p.multiProcessorCount;
  return 0;
}

int ihip_alloc(ihip_ctx* c, uint64_t bytes, uint64_t* dev)
{
  if (!c || !dev) return fail(IHIP_E_ARG, "ihip_alloc: no context");
  if (c->capturing) return fail(IHIP_E_CAPTURE, "ihip_alloc while capturing");
  void* p = nullptr;
  IHIP_CHECK(hipSetDevice(c->device));
  IHIP_CHECK(hipMalloc(&p, bytes ? bytes : 4));
  c->allocations.push_back((uint64_t)p);
  *dev = (uint64_t)p;
  return 0;
}

int ihip_free(ihip_ctx* c, uint64_t dev)
{
  if (!c) return fail(IHIP_E_ARG, "ihip_free: no context");
  for (size_t i = 0; i < c->allocations.size(); i++)
    if (c->allocations[i] == dev) {
      IHIP_CHECK(hipStreamSynchronize(c->stream));
      IHIP_CHECK(hipFree((void*)dev));
      c->allocations.erase(c->allocations.begin() + i);
      return 0;
    }
  return fail(IHIP_E_ARG, "ihip_free: not a buffer of this context");
}

int ihip_upload(ihip_ctx* c, uint64_t dev, const void* host, uint64_t bytes)
{
  if (!c || (!host && bytes)) return fail(IHIP_E_ARG, "ihip_upload");
  if (c->capturing) return fail(IHIP_E_CAPTURE, "ihip_upload while capturing");
  if (!bytes) return 0;
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)dev, (void*)host, bytes, c->stream));
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  return 0;
}

int ihip_download(ihip_ctx* c, void* host, uint64_t dev, uint64_t bytes)
{
  if (!c || (!host && bytes)) return fail(IHIP_E_ARG, "ihip_download");
  if (c->capturing) return fail(IHIP_E_CAPTURE, "ihip_download while capturing");
  if (!bytes) return 0;
  IHIP_CHECK(hipMemcpyDtoHAsync(host, (hipDeviceptr_t)dev, bytes, c->stream));
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  return 0;
}

int ihip_upload_async(ihip_ctx* c, uint64_t dev, const void* host, uint64_t bytes)
{
  if (!c || (!host && bytes)) return fail(IHIP_E_ARG, "ihip_upload_async");
  if (!bytes) return 0;
  IHIP_CHECK(hipMemcpyHtoDAsync((hipDeviceptr_t)dev, (void*)host, bytes, c->stream));
  return 0;
}

int ihip_copy_async(ihip_ctx* c, uint64_t dst, uint64_t src, uint64_t bytes)
{
  if (!c) return fail(IHIP_E_ARG, "ihip_copy_async");
  if (!bytes) return 0;
  IHIP_CHECK(hipMemcpyDtoDAsync((hipDeviceptr_t)dst, (hipDeviceptr_t)src, bytes, c->stream));
  return 0;
}

int ihip_synchronize(ihip_ctx* c)
{
  if (!c) return fail(IHIP_E_ARG, "ihip_synchronize");
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  return 0;
}

int ihip_capture_begin(ihip_ctx* c)
{
  if (!c || c->capturing) return fail(IHIP_E_CAPTURE, "ihip_capture_begin: already capturing");
  IHIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  c->capturing = true;
  return 0;
}

int ihip_capture_end(ihip_ctx* c, int slot)
{
  if (!c || !c->capturing) return fail(IHIP_E_CAPTURE, "ihip_capture_end: not capturing");
  if (slot < 0 || slot >= 16) return fail(IHIP_E_ARG, "ihip_capture_end: slot");
  c->capturing = false;
  hipGraph_t g = nullptr;
  IHIP_CHECK(hipStreamEndCapture(c->stream, &g));
  // TInferCuda.CaptureEnd (cuda.pas:692-720): update the executable graph of
  // the slot in place when the topology allows, else instantiate anew
  if (c->execs[slot]) {
    hipGraphExecUpdateResult res;
    hipGraphNode_t err_node = nullptr;
    if (hipGraphExecUpdate(c->execs[slot], g, &err_node, &res) == hipSuccess &&
        res == hipGraphExecUpdateSuccess) {
      if (c->graphs[slot]) (void)hipGraphDestroy(c->graphs[slot]);
      c->graphs[slot] = g;
      return 0;
    }
    (void)hipGetLastError();
    (void)hipGraphExecDestroy(c->execs[slot]);
    c->execs[slot] = nullptr;
  }
  if (c->graphs[slot]) (void)hipGraphDestroy(c->graphs[slot]);
  c->graphs[slot] = g;
  IHIP_CHECK(hipGraphInstantiate(&c->execs[slot], g, nullptr, nullptr, 0));
  return 0;
}

int ihip_graph_launch(ihip_ctx* c, int slot)
{
  if (!c || slot < 0 || slot >= 16 || !c->execs[slot])
    return fail(IHIP_E_ARG, "ihip_graph_launch: no graph in slot");
  IHIP_CHECK(hipGraphLaunch(c->execs[slot], c->stream));
  return 0;
}

int ihip_event_record(ihip_ctx* c, int i)
{
  if (!c || i < 0 || i >= 64) return fail(IHIP_E_ARG, "ihip_event_record");
  IHIP_CHECK(hipEventRecord(c->events[i], c->stream));
  return 0;
}

// the kernel timer: every later direct launch (not under capture) of a
// kernel whose name starts with prefix is timed by its own dispatch's start
// and end; NULL or "" stops it. At most `capacity` launches are timed
// between two reads.
int ihip_kernel_timer(ihip_ctx* c, const char* prefix, int64_t capacity)
{
  if (!c || capacity < 0 || capacity > 65536) return fail(IHIP_E_ARG, "ihip_kernel_timer");
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  c->timer_used = 0;
  c->timer_prefix = prefix ? prefix : "";
  while ((int64_t)c->timer_events.size() < 2 * capacity) {
    hipEvent_t ev = nullptr;
    IHIP_CHECK(hipEventCreate(&ev));
    c->timer_events.push_back(ev);
  }
  c->timer_names.resize(c->timer_events.size() / 2);
  return 0;
}

// a timing build's stamp buffers (IHIP_STAMP): launch k of a kernel named
// prefix* records into dev + k * stride, for k < count (the module's
// ihip_trace pointer is set before the launch and cleared after it); an
// ordinary build has no ihip_trace and ignores the call
int ihip_trace_buffer(ihip_ctx* c, uint64_t dev, uint64_t stride, int64_t count, const char* prefix)
{
  if (!c || count < 0) return fail(IHIP_E_ARG, "ihip_trace_buffer");
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  c->trace_ptrs.clear();
  c->trace_globals.clear();
  c->trace_prefix = (dev && prefix) ? prefix : "";
  c->trace_used = 0;
  if (c->trace_prefix.empty()) return 0;
  for (auto& m : c->modules) {
    hipDeviceptr_t p = nullptr;
    size_t bytes = 0;
    if (hipModuleGetGlobal(&p, &bytes, m.mod, "ihip_trace") != hipSuccess) {
      (void)hipGetLastError();
      continue;
    }
    c->trace_globals.push_back((uint64_t)p);
  }
  // the pointer values the copies read: k = 0..count-1, then the null
  c->trace_ptrs.resize((size_t)count + 1);
  for (int64_t k = 0; k < count; k++) c->trace_ptrs[k] = dev + (uint64_t)k * stride;
  c->trace_ptrs[count] = 0;
  return 0;
}

int ihip_kernel_timer_report(ihip_ctx* c, char* text, int64_t len)
{
  if (!c || !text || len < 1) return fail(IHIP_E_ARG, "ihip_kernel_timer_report");
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  std::vector<std::string> order;
  std::unordered_map<std::string, std::pair<int64_t, double>> agg;
  for (size_t i = 0; i < c->timer_used; i++) {
    float ms = 0;
    IHIP_CHECK(hipEventElapsedTime(&ms, c->timer_events[2 * i], c->timer_events[2 * i + 1]));
    auto it = agg.find(c->timer_names[i]);
    if (it == agg.end()) {
      order.push_back(c->timer_names[i]);
      it = agg.emplace(c->timer_names[i], std::make_pair((int64_t)0, 0.0)).first;
    }
    it->second.first++;
    it->second.second += ms;
  }
  std::string out;
  char line[160];
  for (auto& n : order) {
    snprintf(line, sizeof line, "%s %lld %.6f\n", n.c_str(), (long long)agg[n].first, agg[n].second);
    out += line;
  }
  snprintf(text, (size_t)len, "%s", out.c_str());
  c->timer_used = 0;
  return 0;
}

int ihip_kernel_timer_read(ihip_ctx* c, int64_t* launches, double* total_ms)
{
  if (!c || !launches || !total_ms) return fail(IHIP_E_ARG, "ihip_kernel_timer_read");
  IHIP_CHECK(hipStreamSynchronize(c->stream));
  double t = 0;
  for (size_t i = 0; i < c->timer_used; i++) {
    float ms = 0;
    IHIP_CHECK(hipEventElapsedTime(&ms, c->timer_events[2 * i], c->timer_events[2 * i + 1]));
    t += ms;
  }
  *launches = (int64_t)c->timer_used;
  *total_ms = t;
  c->timer_used = 0;
  return 0;
}

int ihip_event_elapsed(ihip_ctx* c, int from, int to, float* ms)
{
  if (!c || from < 0 || from >= 64 || to < 0 || to >= 64 || !ms)
    return fail(IHIP_E_ARG, "ihip_event_elapsed");
  IHIP_CHECK(hipEventSynchronize(c->events[to]));
  IHIP_CHECK(hipEventElapsedTime(ms, c->events[from], c->events[to]));
  return 0;
}

}  // extern "C"
