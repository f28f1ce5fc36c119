// internal.hpp -- host-side helpers shared by the entry points (not exported).
#pragma once

#include <stdint.h>

#include <initializer_list>

#include <hip/hip_runtime.h>

#include "tile_plan.hpp"

namespace fe2o3_host {

// True when the environment variable FE2O3_FAULT_POINT names `entry`: the
// entry point then fails with FE2O3_ERR_INJECTED before any launch.  This is
// the host-forced failure path used by the failure-handling tests.
bool fault_point(const char* entry);

// Raises the dynamic-LDS limit of each kernel in `fns` to `bytes` and returns
// 0 or the first hipError_t.  Call sites keep the result in a function-local
// static, so this runs once per process, thread-safely.
inline int32_t set_dynamic_lds(std::initializer_list<const void*> fns, int bytes) {
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return (int32_t)e;
  }
  return 0;
}

// The current device's non-finite counter: a device address that kernels
// admitting only finite inputs receive as an argument and add 1 to
// (mark_nonfinite) when they find a NaN or an infinity.  Each device has its
// own counter (a file-scope __device__ variable of runtime.hip, located once
// per device with hipGetSymbolAddress); nothing clears it, and a
// synchronize reports a count it has not reported before as
// FE2O3_ERR_NONFINITE (status_track.hpp).  nullptr on failure.
uint32_t* status_word();

// The current device's CU and XCD counts as the runtime reports them
// (hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeNumberOfXccs),
// queried once per device and cached.  0, or the hipError_t of the query.
// An XCD count the runtime does not report is taken as 1 (the tile orders
// then stay in id order, which is correct on any part).
int32_t device_topology(tile_plan::Topology* out);

// Stream-ordered device scratch for entry points that stage operands (a
// library-owned pool per device; runtime.hip): scratch_alloc enqueues the
// allocation on stream s, scratch_free its release after the work enqueued
// before it.  0, or a hipError_t.
int32_t scratch_alloc(void** p, size_t bytes, hipStream_t s);
int32_t scratch_free(void* p, hipStream_t s);

// `rows` rows of `cols` bf16 elements, `ld` apart from src (any 2-byte
// alignment), copied on stream s into rows of dst_cols elements (a multiple
// of 8; zeros from cols on) at dst (16-byte aligned).  0, or a hipError_t.
int32_t repack_bf16_rows(const uint16_t* src, uint32_t rows, uint32_t cols, uint32_t ld,
                         uint16_t* dst, uint32_t dst_cols, hipStream_t s);

// Enqueue status: 0, or the hipError_t of the launch just made.
inline int32_t after_launch() {
  hipError_t e = hipGetLastError();
  return (int32_t)e;
}

// One kernel launched by a C-ABI entry point, with the launch facts the
// runtime cannot report (workgroup size, dynamic LDS requested).  Each
// source file registers its kernels with a static table of KernelRegistrar;
// fe2o3_kernel_resources adds what HIP reports for the loaded code object.
struct KernelInfo {
  const char* entry;     // C-ABI entry point
  const char* kernel;    // kernel name
  const void* fn;        // host launch stub
  uint32_t threads;      // workgroup size of its launch
  uint32_t dynamic_lds;  // dynamic LDS bytes of its launch (largest)
};
struct KernelRegistrar {
  explicit KernelRegistrar(const KernelInfo& k);
};

}  // namespace fe2o3_host

// First statement of every C-ABI entry point that launches kernels:
//  - FE2O3_FAULT_POINT naming `entry` fails it with FE2O3_ERR_INJECTED
//    before anything else;
//  - the calling thread's last HIP error is cleared, so after_launch()
//    reports the entry's own launches only.  HIP keeps the last failed call
//    of any API in thread-local state until it is read (a failed
//    hipModuleGetFunction, say, or the caller's own failed launch), and
//    successful calls do not reset it.
#define FE2O3_ENTRY(entry)                                             \
  do {                                                                \
    if (fe2o3_host::fault_point(entry)) return FE2O3_ERR_INJECTED;     \
    (void)hipGetLastError();                                          \
  } while (0)
