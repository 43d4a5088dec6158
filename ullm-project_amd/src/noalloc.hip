// noalloc.hip -- the allocation-free forward entry point.
//
// ullm_linear_forward_noalloc runs exactly what ullm_linear_forward runs, but
// takes every byte of scratch (split-K counters and fp32 partials of the
// decode GEMV, per-token quantized activations of the prefill GEMM) from a
// fixed file-scope device array instead of a caller workspace or a
// library-owned hipMalloc buffer, so it never allocates: for callers under
// HIP graph capture, in tight serving loops, or in harnesses that forbid
// allocation.  Calls that would need more than the array holds are refused.
//
// The array exists once per device (each device that loads the library holds
// kScratchBytes until the process ends).  Host code reaches it only through
// the device address hipGetSymbolAddress returns for the current device; the
// array's name in host code is not a device address.  All calls on one
// device share the array: calls that overlap in time on one device (two
// streams, two threads) race and must be ordered by the caller.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "abi_common.hpp"
#include "kernels.hpp"
#include "ullm/linear.h"

namespace {

constexpr uint64_t kScratchBytes = uint64_t(32) << 20;  // 32 MiB per device
constexpr uint64_t kCounterBytes = uint64_t(64) << 10;  // first 64 KiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void zero_words(uint32_t *p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    p[i] = 0u;
  }
}

struct DeviceScratch {
  char *ptr = nullptr;     // device address of `scratch` on this device
  bool counters_zeroed = false;
};

std::mutex g_mu;
DeviceScratch g_dev[kMaxDevices];

// Resolves the array's address on `device` (current) once, and queues the
// clearing of its counter region on the first call's stream (a fill kernel,
// so a first call under stream capture records it like any other kernel).
ullm_status_t fixed_scratch(int device, hipStream_t stream,
                            ullm::FixedScratch *out, ullm_error_sink_t *sink) {
  if (device < 0 || device >= kMaxDevices) {
    return ullm::write_error(sink, ULLM_STATUS_UNSUPPORTED,
                             "device ordinal beyond the fixed-scratch table");
  }
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceScratch &d = g_dev[device];
  if (d.ptr == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return ullm::write_errorf(
          sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
          std::string("hipGetSymbolAddress (fixed scratch): ") +
              hipGetErrorName(e));
    }
    d.ptr = static_cast<char *>(p);
  }
  if (!d.counters_zeroed) {
    const uint32_t words = uint32_t(kCounterBytes / 4);
    hipLaunchKernelGGL(zero_words, dim3((words + 255) / 256), dim3(256), 0,
                       stream, reinterpret_cast<uint32_t *>(d.ptr), words);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      return ullm::write_errorf(sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                                std::string("fixed scratch clear: ") +
                                    hipGetErrorName(e));
    }
    d.counters_zeroed = true;
  }
  out->counters = d.ptr;
  out->counter_bytes = kCounterBytes;
  out->base = d.ptr + kCounterBytes;
  out->bytes = kScratchBytes - kCounterBytes;
  return ULLM_STATUS_OK;
}

}  // namespace

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_forward_noalloc(
    const ullm_linear_forward_desc_t *desc, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "linear forward (no allocation)", {
    return ullm::forward_dispatch(desc, error_sink, fixed_scratch);
  });
}
