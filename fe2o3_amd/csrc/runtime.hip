// runtime.hip -- the runtime seam of the C-ABI: device discovery, the
// 312-byte property record, streams, events and memory.  Mirrors the
// capability set of crates/fe2o3-hip-sys/src/lib.rs:92-165 and the C shim
// crates/fe2o3-hip-sys/native/device_properties.c:63-101.
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "common.hpp"
#include "internal.hpp"
#include "status_track.hpp"

static_assert(sizeof(Fe2o3HipDeviceProperties) == 312, "property record is 312 bytes");
static_assert(offsetof(Fe2o3HipDeviceProperties, warp_size) == 256, "warp_size offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, max_threads_per_block) == 260, "offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, max_block_dim) == 264, "offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, max_grid_dim) == 276, "offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, shared_mem_per_block) == 288, "offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, shared_mem_per_block_optin) == 296, "offset");
static_assert(offsetof(Fe2o3HipDeviceProperties, architecture_features) == 304, "offset");

namespace fe2o3_host {

bool fault_point(const char* entry) {
  const char* env = getenv("FE2O3_FAULT_POINT");
  return env != nullptr && strcmp(env, entry) == 0;
}

// Registered kernels, filled by the static tables of every source file when
// the library loads (a function-local static, so registration order across
// files does not matter).
// A table that would overflow is recorded (`dropped`) and every query then
// fails with FE2O3_ERR_OVERFLOW rather than answer from a partial table.
static constexpr int kMaxKernels = 512;
struct Registry {
  KernelInfo k[kMaxKernels];
  int n = 0;
  int dropped = 0;
};
static Registry& registry() {
  static Registry r;
  return r;
}
KernelRegistrar::KernelRegistrar(const KernelInfo& k) {
  Registry& r = registry();
  if (r.n < kMaxKernels)
    r.k[r.n++] = k;
  else
    ++r.dropped;
}

// One non-finite rejection counter per device.  The reference's kernels
// trap on a non-finite input and the fault surfaces when the host
// synchronizes; here the kernel adds 1 to this counter instead, writes its
// documented sentinel outputs and exits normally, and the next
// fe2o3_rt_stream_synchronize or fe2o3_rt_device_synchronize on the device
// that reads a count it has not reported yet returns FE2O3_ERR_NONFINITE
// (the bookkeeping is StatusTracker, status_track.hpp).  Neither the kernels
// nor the host ever clear the counter.
static __device__ __align__(256) uint32_t status_word_dev;

static constexpr int kMaxDevices = 64;
static std::mutex status_mu;
static uint32_t* status_ptrs[kMaxDevices];
static StatusTracker status_seen[kMaxDevices];

uint32_t* status_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(status_mu);
  if (status_ptrs[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(status_word_dev)) != hipSuccess) return nullptr;
    status_ptrs[dev] = (uint32_t*)p;
  }
  return status_ptrs[dev];
}

// Reads the current device's counter after a successful synchronize and
// reports whether it moved since the device's last report.  The counter is
// per device: a rejection by a kernel that finished on another stream of the
// device is reported here too, once.
static int32_t take_status(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return (int32_t)hipErrorInvalidDevice;
  uint32_t* p = status_word();
  if (p == nullptr) return (int32_t)hipErrorInvalidSymbol;
  uint32_t v = 0;
  hipError_t e = hipMemcpyAsync(&v, p, sizeof v, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return (int32_t)e;
  std::lock_guard<std::mutex> lock(status_mu);
  return status_seen[dev].report(v) ? FE2O3_ERR_NONFINITE : FE2O3_OK;
}

// CU and XCD counts per device, queried on first use.  A packed word per
// device (cus << 8 | xcds; 0 = not yet queried), so concurrent first calls
// may both query but every reader sees a whole value.
static std::atomic<uint64_t> topology_word[kMaxDevices];

int32_t device_topology(tile_plan::Topology* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int32_t)e;
  if (dev < 0 || dev >= kMaxDevices) return (int32_t)hipErrorInvalidDevice;
  uint64_t w = topology_word[dev].load(std::memory_order_acquire);
  if (w == 0) {
    int cus = 0, xcds = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int32_t)e;
    if (cus <= 0) return (int32_t)hipErrorInvalidDevice;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) {
      (void)hipGetLastError();  // the failed query must not surface as a launch error
      xcds = 1;
    }
    if (xcds <= 0 || xcds > 255) xcds = 1;
    w = (uint64_t)cus << 8 | (uint64_t)xcds;
    topology_word[dev].store(w, std::memory_order_release);
  }
  out->cus = (uint32_t)(w >> 8);
  out->xcds = (uint32_t)(w & 0xffu);
  return 0;
}

// Stream-ordered scratch: one library-owned memory pool per device, its
// release threshold at the maximum so blocks freed at the end of one call
// stay in the pool for the next (a pool of the device's own would hand them
// back at every synchronize).  Allocation and free are ordered on the
// caller's stream, so concurrent calls on different streams get different
// blocks and a call never frees memory its kernels still use.
static hipMemPool_t scratch_pools[kMaxDevices];
static std::mutex scratch_mu;

static int32_t scratch_pool(hipMemPool_t* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int32_t)e;
  if (dev < 0 || dev >= kMaxDevices) return (int32_t)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_pools[dev] == nullptr) {
    hipMemPoolProps props;
    memset(&props, 0, sizeof props);
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    e = hipMemPoolCreate(&pool, &props);
    if (e != hipSuccess) return (int32_t)e;
    uint64_t keep = ~0ull;
    e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
    if (e != hipSuccess) {
      (void)hipMemPoolDestroy(pool);
      return (int32_t)e;
    }
    scratch_pools[dev] = pool;
  }
  *out = scratch_pools[dev];
  return 0;
}

int32_t scratch_alloc(void** p, size_t bytes, hipStream_t s) {
  *p = nullptr;
  hipMemPool_t pool = nullptr;
  const int32_t rc = scratch_pool(&pool);
  if (rc != 0) return rc;
  return (int32_t)hipMallocFromPoolAsync(p, bytes == 0 ? 16 : bytes, pool, s);
}

int32_t scratch_free(void* p, hipStream_t s) {
  return p == nullptr ? 0 : (int32_t)hipFreeAsync(p, s);
}

}  // namespace fe2o3_host

static_assert(sizeof(Fe2o3KernelResources) == 120, "resource record is 120 bytes");

extern "C" {

const char* fe2o3_status_string(int32_t status) {
  switch (status) {
    case FE2O3_OK: return "success";
    case FE2O3_ERR_LENGTH: return "slice length does not match the shape";
    case FE2O3_ERR_SHAPE: return "unsupported shape or profile";
    case FE2O3_ERR_STRIDE: return "stride smaller than the row extent";
    case FE2O3_ERR_NONFINITE: return "non-finite input rejected by the contract";
    case FE2O3_ERR_WEIGHTS: return "route weight pair violates the policy";
    case FE2O3_ERR_OVERFLOW: return "extent arithmetic overflows";
    case FE2O3_ERR_NULL: return "required pointer is NULL";
    case FE2O3_ERR_DEVICE: return "current device is not gfx950";
    case FE2O3_ERR_ALIGNMENT: return "pointer misaligned for this entry point";
    case FE2O3_ERR_WORKSPACE: return "workspace too small";
    case FE2O3_ERR_INJECTED: return "failure injected by FE2O3_FAULT_POINT";
    case FE2O3_ERR_M_TAIL: return "M is not a multiple of the 16-row tile";
    case FE2O3_ERR_N_TAIL: return "N is not a multiple of the 16-column tile";
    case FE2O3_ERR_K_TAIL: return "K is not a multiple of the 16-deep reduction tile";
    case FE2O3_ERR_JOIN: return "code object and host request do not reconcile";
    case FE2O3_ERR_LOAD: return "lifecycle load rejected";
    case FE2O3_ERR_DISPATCH: return "lifecycle dispatch rejected";
    case FE2O3_ERR_STATE: return "lifecycle call out of order";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown fe2o3 status";
}

// device_properties.c:63-101: zero the record, then fill the stable subset;
// on failure the record stays zeroed.
int32_t fe2o3HipGetDeviceProperties(int32_t device_id, Fe2o3HipDeviceProperties* properties) {
  if (properties == nullptr) return (int32_t)hipErrorInvalidValue;
  memset(properties, 0, sizeof(*properties));
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device_id);
  if (e != hipSuccess) return (int32_t)e;
  strncpy(properties->gcn_arch_name, p.gcnArchName, sizeof(properties->gcn_arch_name) - 1);
  properties->warp_size = p.warpSize;
  properties->max_threads_per_block = p.maxThreadsPerBlock;
  for (int i = 0; i < 3; ++i) {
    properties->max_block_dim[i] = p.maxThreadsDim[i];
    properties->max_grid_dim[i] = p.maxGridSize[i];
  }
  properties->shared_mem_per_block = (uint64_t)p.sharedMemPerBlock;
  properties->shared_mem_per_block_optin = (uint64_t)p.sharedMemPerBlockOptin;
  uint64_t f = 0;
  if (p.arch.hasGlobalInt32Atomics) f |= FE2O3_HIP_DEVICE_ARCH_HAS_GLOBAL_INT32_ATOMICS;
  if (p.arch.hasSharedInt32Atomics) f |= FE2O3_HIP_DEVICE_ARCH_HAS_SHARED_INT32_ATOMICS;
  if (p.arch.hasGlobalInt64Atomics) f |= FE2O3_HIP_DEVICE_ARCH_HAS_GLOBAL_INT64_ATOMICS;
  if (p.arch.hasSharedInt64Atomics) f |= FE2O3_HIP_DEVICE_ARCH_HAS_SHARED_INT64_ATOMICS;
  if (p.arch.hasWarpVote) f |= FE2O3_HIP_DEVICE_ARCH_HAS_WARP_VOTE;
  if (p.arch.hasWarpBallot) f |= FE2O3_HIP_DEVICE_ARCH_HAS_WARP_BALLOT;
  if (p.arch.hasWarpShuffle) f |= FE2O3_HIP_DEVICE_ARCH_HAS_WARP_SHUFFLE;
  properties->architecture_features = f;
  return FE2O3_OK;
}

int32_t fe2o3_rt_init(uint32_t flags) { return (int32_t)hipInit(flags); }

int32_t fe2o3_rt_get_device_count(int32_t* count) {
  if (count == nullptr) return FE2O3_ERR_NULL;
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  *count = e == hipSuccess ? c : 0;
  return (int32_t)e;
}

int32_t fe2o3_rt_set_device(int32_t device_id) { return (int32_t)hipSetDevice(device_id); }

int32_t fe2o3_rt_get_device(int32_t* device_id) {
  if (device_id == nullptr) return FE2O3_ERR_NULL;
  int d = 0;
  hipError_t e = hipGetDevice(&d);
  *device_id = d;
  return (int32_t)e;
}

int32_t fe2o3_rt_device_rates(int32_t device_id, int32_t* compute_units, int32_t* clock_khz,
                              int32_t* memory_clock_khz, int32_t* memory_bus_bits) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device_id);
  if (e != hipSuccess) return (int32_t)e;
  if (compute_units) *compute_units = p.multiProcessorCount;
  if (clock_khz) *clock_khz = p.clockRate;
  if (memory_clock_khz) *memory_clock_khz = p.memoryClockRate;
  if (memory_bus_bits) *memory_bus_bits = p.memoryBusWidth;
  return FE2O3_OK;
}

int32_t fe2o3_rt_require_gfx950(int32_t device_id) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device_id);
  if (e != hipSuccess) return (int32_t)e;
  return strncmp(p.gcnArchName, "gfx950", 6) == 0 ? FE2O3_OK : FE2O3_ERR_DEVICE;
}

int32_t fe2o3_rt_device_synchronize(void) {
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return (int32_t)e;
  return fe2o3_host::take_status(nullptr);
}

int32_t fe2o3_rt_stream_create(void** stream) {
  if (stream == nullptr) return FE2O3_ERR_NULL;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreate(&s);  // default priority, as every stream here
  *stream = (void*)s;
  return (int32_t)e;
}

int32_t fe2o3_rt_stream_destroy(void* stream) {
  return (int32_t)hipStreamDestroy((hipStream_t)stream);
}

int32_t fe2o3_rt_stream_synchronize(void* stream) {
  const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return (int32_t)e;
  return fe2o3_host::take_status((hipStream_t)stream);
}

int32_t fe2o3_rt_event_create(void** event, uint32_t flags) {
  if (event == nullptr) return FE2O3_ERR_NULL;
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, flags);
  *event = (void*)ev;
  return (int32_t)e;
}

int32_t fe2o3_rt_event_destroy(void* event) { return (int32_t)hipEventDestroy((hipEvent_t)event); }

int32_t fe2o3_rt_event_record(void* event, void* stream) {
  return (int32_t)hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
}

int32_t fe2o3_rt_event_synchronize(void* event) {
  return (int32_t)hipEventSynchronize((hipEvent_t)event);
}

int32_t fe2o3_rt_event_query(void* event) { return (int32_t)hipEventQuery((hipEvent_t)event); }

int32_t fe2o3_rt_event_elapsed_ms(float* milliseconds, void* start, void* stop) {
  if (milliseconds == nullptr) return FE2O3_ERR_NULL;
  return (int32_t)hipEventElapsedTime(milliseconds, (hipEvent_t)start, (hipEvent_t)stop);
}

int32_t fe2o3_rt_malloc(void** ptr, size_t bytes) {
  if (ptr == nullptr) return FE2O3_ERR_NULL;
  *ptr = nullptr;
  return (int32_t)hipMalloc(ptr, bytes);
}

int32_t fe2o3_rt_free(void* ptr) { return (int32_t)hipFree(ptr); }

int32_t fe2o3_rt_host_malloc(void** ptr, size_t bytes) {
  if (ptr == nullptr) return FE2O3_ERR_NULL;
  *ptr = nullptr;
  return (int32_t)hipHostMalloc(ptr, bytes, 0);
}

int32_t fe2o3_rt_host_free(void* ptr) { return (int32_t)hipHostFree(ptr); }

int32_t fe2o3_rt_memcpy_async(void* dst, const void* src, size_t bytes, uint32_t kind,
                              void* stream) {
  if (kind > 4) return (int32_t)hipErrorInvalidMemcpyDirection;
  return (int32_t)hipMemcpyAsync(dst, src, bytes, (hipMemcpyKind)kind, (hipStream_t)stream);
}

int32_t fe2o3_rt_memcpy(void* dst, const void* src, size_t bytes, uint32_t kind) {
  if (kind > 4) return (int32_t)hipErrorInvalidMemcpyDirection;
  return (int32_t)hipMemcpy(dst, src, bytes, (hipMemcpyKind)kind);
}

int32_t fe2o3_rt_memset_async(void* dst, int32_t value, size_t bytes, void* stream) {
  return (int32_t)hipMemsetAsync(dst, value, bytes, (hipStream_t)stream);
}

// lib.rs:144-165: the module subset.  Handles are HIP's, passed through as
// opaque pointers; null out-pointers and names are refused before any HIP
// call.
int32_t fe2o3_rt_module_load(void** module, const char* file_name) {
  if (module == nullptr || file_name == nullptr) return FE2O3_ERR_NULL;
  *module = nullptr;
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoad(&m, file_name);
  if (e == hipSuccess) *module = (void*)m;
  return (int32_t)e;
}

int32_t fe2o3_rt_module_load_data(void** module, const void* image) {
  if (module == nullptr || image == nullptr) return FE2O3_ERR_NULL;
  *module = nullptr;
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoadData(&m, image);
  if (e == hipSuccess) *module = (void*)m;
  return (int32_t)e;
}

int32_t fe2o3_rt_module_unload(void* module) {
  if (module == nullptr) return FE2O3_ERR_NULL;
  return (int32_t)hipModuleUnload((hipModule_t)module);
}

int32_t fe2o3_rt_module_get_function(void** function, void* module, const char* kernel_name) {
  if (function == nullptr || module == nullptr || kernel_name == nullptr) return FE2O3_ERR_NULL;
  *function = nullptr;
  hipFunction_t f = nullptr;
  const hipError_t e = hipModuleGetFunction(&f, (hipModule_t)module, kernel_name);
  if (e == hipSuccess) *function = (void*)f;
  return (int32_t)e;
}

int32_t fe2o3_rt_module_launch_kernel(void* function, uint32_t grid_dim_x, uint32_t grid_dim_y,
                                      uint32_t grid_dim_z, uint32_t block_dim_x,
                                      uint32_t block_dim_y, uint32_t block_dim_z,
                                      uint32_t shared_mem_bytes, void* stream,
                                      void** kernel_params, void** extra) {
  if (function == nullptr) return FE2O3_ERR_NULL;
  return (int32_t)hipModuleLaunchKernel((hipFunction_t)function, grid_dim_x, grid_dim_y,
                                        grid_dim_z, block_dim_x, block_dim_y, block_dim_z,
                                        shared_mem_bytes, (hipStream_t)stream, kernel_params,
                                        extra);
}

int32_t fe2o3_kernel_resources(const char* entry, uint32_t index, Fe2o3KernelResources* out,
                               uint32_t* count) {
  if (!entry || !count) return FE2O3_ERR_NULL;
  const fe2o3_host::Registry& r = fe2o3_host::registry();
  if (r.dropped != 0) {
    *count = 0;
    return FE2O3_ERR_OVERFLOW;
  }
  const fe2o3_host::KernelInfo* hit = nullptr;
  uint32_t n = 0;
  for (int i = 0; i < r.n; ++i)
    if (strcmp(r.k[i].entry, entry) == 0) {
      if (n == index) hit = &r.k[i];
      ++n;
    }
  *count = n;
  if (!hit) return FE2O3_ERR_LENGTH;
  if (!out) return FE2O3_ERR_NULL;
  hipFuncAttributes attr;
  const hipError_t e = hipFuncGetAttributes(&attr, hit->fn);
  if (e != hipSuccess) return (int32_t)e;
  memset(out, 0, sizeof *out);
  strncpy(out->kernel, hit->kernel, sizeof out->kernel - 1);
  out->workgroup_size = hit->threads;
  out->static_lds_bytes = (uint32_t)attr.sharedSizeBytes;
  out->dynamic_lds_bytes = hit->dynamic_lds;
  out->private_segment_bytes = (uint32_t)attr.localSizeBytes;
  out->vgprs = (uint32_t)attr.numRegs;
  out->max_threads_per_workgroup = (uint32_t)attr.maxThreadsPerBlock;
  return FE2O3_OK;
}

}  // extern "C"
