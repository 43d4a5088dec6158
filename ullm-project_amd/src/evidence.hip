// evidence.hip -- the model-free HIP evidence ABI on gfx950.
//
// Behaviour contract: reference native/hip/src/evidence_abi.h:10-60 and the
// runtime it declares (native/hip/src/hip_evidence_runtime.hip.cpp:539-789):
// submit copies the caller's bytes and queues two device allocations, two
// host<->device copies and one XOR-0x5a dispatch; wait and destroy consume
// the handle; at most two completions are outstanding.  Argument validation
// and its diagnostics are the reference's, so a caller sees the same status
// and message for the same malformed call (checked against the reference's
// own stub in the CPU tests).
//
// Design on this part:
//   * A fixed table of two slots, one per outstanding completion, each with
//     its completion event and pinned host staging (grown on demand, reused).
//     Handles are integers that are never reissued, mapped to slots.
//   * All submissions share one library stream (non-blocking, default
//     priority).  Device buffers come from the stream-ordered allocator
//     (hipMallocAsync / hipFreeAsync), so they are released in stream order
//     right after the result is copied out: no cleanup thread and no
//     blocking free.  Where the device has no memory pools, hipMalloc is used
//     and the buffers are freed once the slot's event has completed.
//   * A consumed slot whose work may still run is "retired"; any later call
//     reclaims retired slots whose event reports completion, without ever
//     blocking.  A slot whose event reports an error is never reused (its
//     staging may still be in use), which closes one of the two slots for the
//     rest of the process, as the reference's circuit breaker does.
//   * The kernel moves 16 bytes per lane in a grid-stride loop; the tail
//     (fewer than 16 bytes) is handled by the first lanes.  One dispatch.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <thread>

#include "abi_common.hpp"
#include "ullm/hip_evidence.h"

namespace {

using ullm::write_error;
using ullm::write_errorf;

constexpr int kSlots = 2;

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void evidence_xor_kernel(
    const uint8_t *__restrict__ in, uint8_t *__restrict__ out, uint64_t n,
    bool vec) {
  const uint64_t tid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  const uint64_t body = vec ? n / 16 : 0;
  const u32x4v key = {0x5a5a5a5au, 0x5a5a5a5au, 0x5a5a5a5au, 0x5a5a5a5au};
  for (uint64_t i = tid; i < body; i += stride) {
    reinterpret_cast<u32x4v *>(out)[i] =
        reinterpret_cast<const u32x4v *>(in)[i] ^ key;
  }
  for (uint64_t i = body * 16 + tid; i < n; i += stride) {
    out[i] = static_cast<uint8_t>(in[i] ^ ULLM_HIP_EVIDENCE_TRANSFORM_XOR);
  }
}

enum class SlotState { kFree, kLive, kWaiting, kRetired, kBroken };

struct Slot {
  SlotState state = SlotState::kFree;
  uint64_t handle = 0;
  hipEvent_t done = nullptr;
  uint8_t *host_in = nullptr;  // pinned staging, reused across submissions
  uint8_t *host_out = nullptr;
  uint64_t host_cap = 0;
  uint64_t size = 0;
  // Device buffers of the hipMalloc path (null with memory pools: those are
  // returned to the pool in stream order by the submission itself).
  uint8_t *dev_in = nullptr;
  uint8_t *dev_out = nullptr;
  uint64_t allocations = 0, copies = 0, dispatches = 0;
};

struct Runtime {
  std::mutex mu;
  Slot slots[kSlots];
  hipStream_t stream = nullptr;
  bool pools = false;
  bool device_ok = false;
  uint64_t next_handle = 1;
};

Runtime &runtime() {
  // Never destroyed: process exit must not wait on device work or free
  // memory a wedged device may still use.
  static Runtime *const r = new Runtime();
  return *r;
}

ullm_hip_evidence_completion_t *to_opaque(uint64_t h) {
  return reinterpret_cast<ullm_hip_evidence_completion_t *>(uintptr_t(h));
}
uint64_t from_opaque(const ullm_hip_evidence_completion_t *c) {
  return uint64_t(reinterpret_cast<uintptr_t>(c));
}

// Releases the hipMalloc-path buffers of a slot whose work has completed.
void free_device_buffers(Slot &s) {
  if (s.dev_in != nullptr) {
    (void)hipFree(s.dev_in);
    s.dev_in = nullptr;
  }
  if (s.dev_out != nullptr) {
    (void)hipFree(s.dev_out);
    s.dev_out = nullptr;
  }
}

// Retired slots whose event has completed become free; never blocks.
// Caller holds the runtime mutex.
void reclaim(Runtime &r) {
  for (Slot &s : r.slots) {
    if (s.state != SlotState::kRetired) {
      continue;
    }
    const hipError_t q = hipEventQuery(s.done);
    if (q == hipSuccess) {
      free_device_buffers(s);
      s.state = SlotState::kFree;
    } else if (q != hipErrorNotReady) {
      s.state = SlotState::kBroken;
    }
  }
}

Slot *find_live(Runtime &r, uint64_t handle) {
  if (handle == 0) {
    return nullptr;
  }
  for (Slot &s : r.slots) {
    if (s.state == SlotState::kLive && s.handle == handle) {
      return &s;
    }
  }
  return nullptr;
}

ullm_status_t hip_error(ullm_error_sink_t *sink, const char *what,
                        hipError_t e) {
  return write_errorf(sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                      std::string(what) + " failed: " + hipGetErrorString(e));
}

// The reference's request checks, in its order and with its diagnostics
// (hip_evidence_runtime.hip.cpp:399-432).
ullm_status_t validate_request(const ullm_hip_evidence_request_t *req,
                               ullm_error_sink_t *sink) {
  if (req == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence request is null");
  }
  if (req->struct_size < sizeof(*req)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence request struct_size is too small");
  }
  if (req->abi_version != ULLM_HIP_EVIDENCE_ABI_VERSION) {
    return write_error(sink, ULLM_STATUS_INVALID_ABI_VERSION,
                       "unsupported evidence ABI version");
  }
  if (!ullm::all_zero(req->reserved)) {
    return write_error(sink, ULLM_STATUS_RESERVED_NONZERO,
                       "evidence request reserved field is non-zero");
  }
  if (req->input == nullptr || req->input_size == 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence input must be non-null and non-empty");
  }
  if (req->input_size > uint64_t(std::numeric_limits<size_t>::max())) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence input is too large");
  }
  return ULLM_STATUS_OK;
}

ullm_status_t validate_result(const ullm_hip_evidence_result_t *res,
                              ullm_error_sink_t *sink) {
  if (res == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence result is null");
  }
  if (res->struct_size < sizeof(*res)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "evidence result struct_size is too small");
  }
  if (res->abi_version != ULLM_HIP_EVIDENCE_ABI_VERSION) {
    return write_error(sink, ULLM_STATUS_INVALID_ABI_VERSION,
                       "unsupported evidence result ABI version");
  }
  if (!ullm::all_zero(res->reserved)) {
    return write_error(sink, ULLM_STATUS_RESERVED_NONZERO,
                       "evidence result reserved field is non-zero");
  }
  return ULLM_STATUS_OK;
}

// One-time device set-up: exactly one visible device, a gfx950 one (the
// reference pins one device too, hip_evidence_runtime.hip.cpp:449-485; the
// architecture name may carry feature suffixes such as
// "gfx950:sramecc+:xnack-"), the library stream, the slots' events.
ullm_status_t ensure_device(Runtime &r, ullm_error_sink_t *sink) {
  if (r.device_ok) {
    return hipSetDevice(0) == hipSuccess
               ? ULLM_STATUS_OK
               : write_error(sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                             "hipSetDevice failed");
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) {
    return hip_error(sink, "hipGetDeviceCount", e);
  }
  if (count != 1) {
    return write_error(sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                       "HIP evidence requires exactly one visible device");
  }
  hipDeviceProp_t prop{};
  e = hipGetDeviceProperties(&prop, 0);
  if (e != hipSuccess) {
    return hip_error(sink, "hipGetDeviceProperties", e);
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0 ||
      (prop.gcnArchName[6] != '\0' && prop.gcnArchName[6] != ':')) {
    return write_errorf(sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                        std::string("HIP gcnArchName '") + prop.gcnArchName +
                            "' is not the gfx950 this library was built for");
  }
  e = hipSetDevice(0);
  if (e != hipSuccess) {
    return hip_error(sink, "hipSetDevice", e);
  }
  int pools = 0;
  if (hipDeviceGetAttribute(&pools, hipDeviceAttributeMemoryPoolsSupported, 0) !=
      hipSuccess) {
    pools = 0;
  }
  if (r.stream == nullptr) {
    e = hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      r.stream = nullptr;
      return hip_error(sink, "hipStreamCreateWithFlags", e);
    }
  }
  for (Slot &s : r.slots) {
    if (s.done == nullptr) {
      e = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
      if (e != hipSuccess) {
        s.done = nullptr;
        return hip_error(sink, "hipEventCreateWithFlags", e);
      }
    }
  }
  r.pools = pools != 0;
  r.device_ok = true;
  return ULLM_STATUS_OK;
}

// Grows a free slot's pinned staging to `bytes` (its previous buffers are
// idle: the slot is free).
hipError_t ensure_staging(Slot &s, uint64_t bytes) {
  if (s.host_cap >= bytes) {
    return hipSuccess;
  }
  if (s.host_in != nullptr) {
    (void)hipHostFree(s.host_in);
    s.host_in = nullptr;
  }
  if (s.host_out != nullptr) {
    (void)hipHostFree(s.host_out);
    s.host_out = nullptr;
  }
  s.host_cap = 0;
  hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&s.host_in), bytes,
                               hipHostMallocDefault);
  if (e == hipSuccess) {
    e = hipHostMalloc(reinterpret_cast<void **>(&s.host_out), bytes,
                      hipHostMallocDefault);
  }
  if (e != hipSuccess) {
    if (s.host_in != nullptr) {
      (void)hipHostFree(s.host_in);
      s.host_in = nullptr;
    }
    return e;
  }
  s.host_cap = bytes;
  return hipSuccess;
}

// Queues the slot's work on the library stream.  Returns the first failing
// call; whatever was queued before it stays ordered before the slot's event,
// which is recorded whenever anything was queued.
hipError_t enqueue(Runtime &r, Slot &s, bool *queued) {
  const hipStream_t st = r.stream;
  uint8_t *din = nullptr, *dout = nullptr;
  hipError_t e;
  if (r.pools) {
    e = hipMallocAsync(reinterpret_cast<void **>(&din), s.size, st);
    *queued = true;
    if (e != hipSuccess) return e;
    ++s.allocations;
    e = hipMallocAsync(reinterpret_cast<void **>(&dout), s.size, st);
  } else {
    e = hipMalloc(reinterpret_cast<void **>(&din), s.size);
    if (e != hipSuccess) return e;
    s.dev_in = din;
    ++s.allocations;
    e = hipMalloc(reinterpret_cast<void **>(&dout), s.size);
    if (e == hipSuccess) s.dev_out = dout;
  }
  auto release = [&]() {
    if (r.pools) {
      if (din != nullptr) (void)hipFreeAsync(din, st);
      if (dout != nullptr) (void)hipFreeAsync(dout, st);
    }
  };
  if (e != hipSuccess) {
    release();
    return e;
  }
  ++s.allocations;
  *queued = true;
  e = hipMemcpyAsync(din, s.host_in, s.size, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) {
    ++s.copies;
    const bool vec = reinterpret_cast<uintptr_t>(din) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(dout) % 16 == 0;
    const uint64_t lanes = vec ? (s.size + 15) / 16 : s.size;
    const uint64_t blocks = (lanes + 255) / 256;
    const uint32_t grid = uint32_t(blocks < 2048 ? (blocks ? blocks : 1) : 2048);
    hipLaunchKernelGGL(evidence_xor_kernel, dim3(grid), dim3(256), 0, st, din,
                       dout, s.size, vec);
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    ++s.dispatches;
    e = hipMemcpyAsync(s.host_out, dout, s.size, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) ++s.copies;
  }
  release();
  return e;
}

}  // namespace

extern "C" ULLM_HIP_API ullm_status_t ullm_hip_evidence_submit(
    const ullm_hip_evidence_request_t *request,
    ullm_hip_evidence_completion_t **completion,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "evidence submit", {
    ullm_status_t st = validate_request(request, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (completion == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "completion output is null");
    }
    *completion = nullptr;
    Runtime &r = runtime();
    std::lock_guard<std::mutex> lock(r.mu);
    st = ensure_device(r, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    reclaim(r);
    Slot *slot = nullptr;
    for (Slot &s : r.slots) {
      if (s.state == SlotState::kFree) {
        slot = &s;
        break;
      }
    }
    if (slot == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INTERNAL_ERROR,
                         "HIP evidence has two completions outstanding (or a "
                         "failed one holds a slot); wait on or destroy one first");
    }
    Slot &s = *slot;
    const hipError_t se = ensure_staging(s, request->input_size);
    if (se != hipSuccess) {
      return hip_error(error_sink, "hipHostMalloc (evidence staging)", se);
    }
    // The caller's bytes are copied now; its pointer is not kept.
    std::memcpy(s.host_in, request->input, size_t(request->input_size));
    s.size = request->input_size;
    s.allocations = s.copies = s.dispatches = 0;
    bool queued = false;
    const hipError_t e = enqueue(r, s, &queued);
    if (queued) {
      const hipError_t re = hipEventRecord(s.done, r.stream);
      // Without a recorded event the slot's completion can never be shown:
      // the slot is closed.
      s.state = re == hipSuccess ? SlotState::kRetired : SlotState::kBroken;
    } else {
      free_device_buffers(s);
    }
    if (e != hipSuccess) {
      return hip_error(error_sink, "HIP evidence submit", e);
    }
    if (s.state != SlotState::kRetired) {
      return write_error(error_sink, ULLM_STATUS_HIP_RUNTIME_ERROR,
                         "HIP evidence submit failed: hipEventRecord");
    }
    s.state = SlotState::kLive;
    s.handle = r.next_handle++;
    *completion = to_opaque(s.handle);
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_hip_evidence_wait(
    ullm_hip_evidence_completion_t *completion, uint32_t timeout_ms,
    uint8_t *output, uint64_t output_capacity,
    ullm_hip_evidence_result_t *result, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "evidence wait", {
    Runtime &r = runtime();
    Slot *slot = nullptr;
    {
      std::lock_guard<std::mutex> lock(r.mu);
      slot = find_live(r, from_opaque(completion));
      if (slot == nullptr) {
        return write_error(error_sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                           "evidence completion handle is not live");
      }
      // The handle is consumed whatever follows.
      slot->state = SlotState::kRetired;
      ullm_status_t st = validate_result(result, error_sink);
      if (st != ULLM_STATUS_OK) {
        return st;
      }
      if (output == nullptr || output_capacity < slot->size) {
        return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "evidence output is null or too small");
      }
      // Owned by this call while it polls: reclaim() leaves it alone.
      slot->state = SlotState::kWaiting;
    }
    Slot &s = *slot;
    // Poll the event (never a blocking synchronize) until the deadline.
    const auto deadline = std::chrono::steady_clock::now() +
                          std::chrono::milliseconds(timeout_ms);
    hipError_t q;
    for (;;) {
      q = hipEventQuery(s.done);
      if (q != hipErrorNotReady) {
        break;
      }
      const auto now = std::chrono::steady_clock::now();
      if (timeout_ms == 0 || now >= deadline) {
        break;
      }
      const auto left = deadline - now;
      const auto nap = std::chrono::microseconds(50);
      std::this_thread::sleep_for(left < nap ? left : nap);
    }
    std::lock_guard<std::mutex> lock(r.mu);
    if (q == hipErrorNotReady) {
      s.state = SlotState::kRetired;
      return write_error(error_sink, ULLM_STATUS_HIP_TIMEOUT,
                         "evidence completion timed out");
    }
    if (q != hipSuccess) {
      s.state = SlotState::kBroken;
      return hip_error(error_sink, "hipEventQuery", q);
    }
    free_device_buffers(s);
    s.state = SlotState::kFree;
    if (s.allocations != 2 || s.copies != 2 || s.dispatches > 1) {
      return write_error(error_sink, ULLM_STATUS_HIP_DISPATCH_CONTRACT,
                         "HIP evidence requires exactly two allocations, two "
                         "copies, and one dispatch");
    }
    if (s.dispatches == 0) {
      return write_error(error_sink, ULLM_STATUS_HIP_ZERO_DISPATCH,
                         "HIP evidence completed with zero kernel dispatches");
    }
    std::memcpy(output, s.host_out, size_t(s.size));
    result->output_size = s.size;
    result->allocation_count = s.allocations;
    result->copy_count = s.copies;
    result->dispatch_count = s.dispatches;
    result->selected_backend = ULLM_BACKEND_HIP;
    result->fallback_used = 0;
    result->terminal = 1;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_hip_evidence_destroy(
    ullm_hip_evidence_completion_t **completion, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "evidence destroy", {
    if (completion == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "completion pointer is null");
    }
    Runtime &r = runtime();
    std::lock_guard<std::mutex> lock(r.mu);
    Slot *slot = find_live(r, from_opaque(*completion));
    if (slot == nullptr) {
      return write_error(error_sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                         "evidence completion handle is not live");
    }
    slot->state = SlotState::kRetired;  // reclaimed once its work completes
    *completion = nullptr;
    reclaim(r);
    return ULLM_STATUS_OK;
  });
}
