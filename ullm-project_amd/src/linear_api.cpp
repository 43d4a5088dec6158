// linear_api.cpp -- C entry points of the quantized linear layer.
//
// Validation order per entry: sink, descriptor header (size, version),
// reserved words, handles, enums, sizes, pointers; only then is the device
// touched.  HIP failures map to ULLM_STATUS_HIP_RUNTIME_ERROR (allocation
// failures to ULLM_STATUS_OUT_OF_MEMORY) with the HIP error name in the sink.
// Weight handles are registered in a mutex-guarded table so that stale or
// foreign pointers are rejected with ULLM_STATUS_HIP_INVALID_HANDLE, the
// identity check the reference applies to its evidence handles
// (native/hip/src/hip_evidence_runtime.hip.cpp:276-303).
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "abi_common.hpp"
#include "kernels.hpp"
#include "layout.hpp"
#include "ullm/linear.h"

#include "weight.hpp"

namespace ullm {
hipError_t launch_fp8_gemm(const uint8_t *xq, const float *xs, uint64_t ldxq,
                           const ullm_linear_weight_t *w, uint32_t m,
                           void *y, uint64_t ldy, bool y_f32, float alpha,
                           const Epilogue &epi, const GemmPlan &p, uint32_t *cnt,
                           float *part, hipStream_t s);
}  // namespace ullm

namespace {

using ullm::write_error;
using ullm::write_errorf;

constexpr uint64_t kMaxDim = (uint64_t(1) << 31) - 1;

std::mutex g_registry_mutex;
std::unordered_set<const ullm_linear_weight_t *> g_registry;

bool registered(const ullm_linear_weight_t *w) {
  std::lock_guard<std::mutex> lock(g_registry_mutex);
  return g_registry.count(w) != 0;
}

// Library-owned workspaces, one per (device, stream, kind) and grown on
// demand: the prefill path's quantized activations, and the decode path's
// split-K scratch (its counter words are zero on allocation and every launch
// leaves them zero).  Calls on one stream are ordered, so they may share a
// buffer; calls on different streams get different buffers.  A buffer that
// is outgrown is retired, not freed: a HIP graph captured earlier may still
// hold its address, and stays valid.
struct Workspace {
  void *ptr = nullptr;
  uint64_t bytes = 0;
};
struct WorkspaceKey {
  int device;
  const void *stream;
  bool split;
  bool operator==(const WorkspaceKey &o) const {
    return device == o.device && stream == o.stream && split == o.split;
  }
};
struct WorkspaceKeyHash {
  size_t operator()(const WorkspaceKey &k) const {
    return std::hash<const void *>()(k.stream) ^ (size_t(k.device) << 1) ^
           size_t(k.split);
  }
};
std::mutex g_ws_mutex;
std::unordered_map<WorkspaceKey, Workspace, WorkspaceKeyHash> g_ws;
std::vector<std::pair<int, void *>> g_ws_retired;  // (device, buffer)


// Makes `device` current for the scope and restores the caller's device.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) {
      prev_ = -1;
    }
    err_ = hipSetDevice(device);
  }
  ~DeviceScope() {
    if (prev_ >= 0) {
      (void)hipSetDevice(prev_);
    }
  }
  hipError_t error() const { return err_; }

 private:
  int prev_ = -1;
  hipError_t err_ = hipSuccess;
};

ullm_status_t hip_fail(ullm_error_sink_t *sink, const char *what,
                       hipError_t err) {
  const ullm_status_t st = err == hipErrorOutOfMemory
                               ? ULLM_STATUS_OUT_OF_MEMORY
                               : ULLM_STATUS_HIP_RUNTIME_ERROR;
  return write_errorf(sink, st,
                      std::string(what) + ": " + hipGetErrorName(err));
}

#define HIP_TRY(sink, what, expr)              \
  do {                                         \
    const hipError_t e_ = (expr);              \
    if (e_ != hipSuccess) {                    \
      return hip_fail(sink, what, e_);         \
    }                                          \
  } while (0)

// The library-owned workspace of at least `need` bytes for this call
// (zeroed when first allocated, for the split-K counters).  Allocates, so a
// call that needs a larger buffer is refused under stream capture.  The
// zeroing is queued on the call's own stream, so the kernel that follows is
// ordered after it even on a non-blocking stream.
ullm_status_t library_workspace(int device, const void *stream, bool split,
                                uint64_t need, void **out,
                                ullm_error_sink_t *error_sink) {
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace &cache = g_ws[WorkspaceKey{device, stream, split}];
  if (cache.bytes < need) {
    const hipStream_t s = static_cast<hipStream_t>(const_cast<void *>(stream));
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(error_sink, "hipStreamIsCapturing", hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "the library-owned workspace must grow, which allocates: "
                         "make this call once outside stream capture, or pass a workspace");
    }
    void *p = nullptr;
    HIP_TRY(error_sink, "hipMalloc (workspace)", hipMalloc(&p, need));
    if (split) {
      const hipError_t e = hipMemsetAsync(p, 0, need, s);
      if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(error_sink, "hipMemsetAsync (workspace)", e);
      }
    }
    if (cache.ptr != nullptr) {
      g_ws_retired.emplace_back(device, cache.ptr);
    }
    cache.ptr = p;
    cache.bytes = need;
  }
  *out = cache.ptr;
  return ULLM_STATUS_OK;
}

ullm_status_t check_device(int device, ullm_error_sink_t *sink) {
  int count = 0;
  const hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess || count == 0) {
    return write_error(sink, ULLM_STATUS_HIP_UNAVAILABLE,
                       "no HIP device is visible");
  }
  if (device < 0 || device >= count) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "device ordinal is out of range");
  }
  hipDeviceProp_t prop;
  HIP_TRY(sink, "hipGetDeviceProperties", hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return write_errorf(sink, ULLM_STATUS_UNSUPPORTED,
                        std::string("device architecture ") + prop.gcnArchName +
                            " is not gfx950");
  }
  return ULLM_STATUS_OK;
}

// Owns device allocations until released (exception/early-return safe).
struct DevBuf {
  void *p = nullptr;
  ~DevBuf() {
    if (p != nullptr) {
      (void)hipFree(p);
    }
  }
  void *release() {
    void *r = p;
    p = nullptr;
    return r;
  }
};

// Bring `bytes` of caller data to the device: device memory is used in place,
// host memory is copied into `staging`.
ullm_status_t stage_source(const void *src, uint64_t bytes, uint32_t memory,
                           DevBuf &staging, const void **out,
                           ullm_error_sink_t *sink) {
  if (memory == ULLM_MEMORY_DEVICE) {
    *out = src;
    return ULLM_STATUS_OK;
  }
  HIP_TRY(sink, "hipMalloc (staging)", hipMalloc(&staging.p, bytes));
  HIP_TRY(sink, "hipMemcpy (host to device)",
          hipMemcpy(staging.p, src, bytes, hipMemcpyHostToDevice));
  *out = staging.p;
  return ULLM_STATUS_OK;
}

ullm_status_t validate_weight_desc(const ullm_linear_weight_desc_t *d,
                                   ullm_error_sink_t *sink) {
  ullm_status_t st = ullm::validate_header(d, sink, "weight descriptor is null");
  if (st != ULLM_STATUS_OK) {
    return st;
  }
  if (!ullm::all_zero(d->reserved) || d->reserved0 != 0) {
    return write_error(sink, ULLM_STATUS_RESERVED_NONZERO,
                       "weight descriptor reserved fields must be zero");
  }
  if (d->layout != ULLM_LINEAR_LAYOUT_PLAIN &&
      d->layout != ULLM_LINEAR_LAYOUT_GATED_PAIRS) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "unknown weight layout");
  }
  if (d->encoding != ULLM_LINEAR_ENCODING_FP8_E4M3_ROW &&
      d->encoding != ULLM_LINEAR_ENCODING_AQ4_G128) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED, "unknown weight encoding");
  }
  if (d->source != ULLM_LINEAR_SOURCE_F32 &&
      d->source != ULLM_LINEAR_SOURCE_ENCODED) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "unknown weight source kind");
  }
  if (d->memory != ULLM_MEMORY_HOST && d->memory != ULLM_MEMORY_DEVICE) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "unknown memory kind");
  }
  if (d->n == 0 || d->k == 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "weight dimensions must be at least 1");
  }
  if (d->n > kMaxDim || d->k > kMaxDim) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                       "weight dimension exceeds 2^31 - 1");
  }
  if (d->layout == ULLM_LINEAR_LAYOUT_GATED_PAIRS && d->n % 2 != 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "a gated-pair weight needs an even N (gate rows, then up rows)");
  }
  if (d->encoding == ULLM_LINEAR_ENCODING_AQ4_G128 && d->k % 128 != 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "AQ4 g128 requires K to be a multiple of 128");
  }
  if (d->values == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "weight values pointer is null");
  }
  if (d->source == ULLM_LINEAR_SOURCE_ENCODED) {
    if (d->scales == nullptr) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "encoded weight scales pointer is null");
    }
    if (d->encoding == ULLM_LINEAR_ENCODING_AQ4_G128 && d->zeros == nullptr) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "encoded AQ4 zeros pointer is null");
    }
  }
  return ULLM_STATUS_OK;
}

ullm_status_t lookup_weight(const ullm_linear_weight_t *w,
                            ullm_error_sink_t *sink) {
  if (w == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "weight handle is null");
  }
  if (!registered(w)) {
    return write_error(sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                       "weight handle is not live");
  }
  return ULLM_STATUS_OK;
}

ullm_status_t create_weight(const ullm_linear_weight_desc_t *d,
                            ullm_linear_weight_t **out,
                            ullm_error_sink_t *sink) {
  auto w = new ullm_linear_weight_t();
  struct Owner {
    ullm_linear_weight_t *w;
    ~Owner() {
      if (w != nullptr) {
        (void)hipFree(w->tiles);
        (void)hipFree(w->aux);
        delete w;
      }
    }
  } owner{w};
  w->encoding = d->encoding;
  w->device = d->device;
  w->n = d->n;
  w->k = d->k;
  w->gate = d->layout == ULLM_LINEAR_LAYOUT_GATED_PAIRS ? d->n / 2 : 0;
  const hipStream_t stream = static_cast<hipStream_t>(d->stream);
  const bool fp8 = d->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
  if (fp8) {
    w->fp8 = ullm::make_fp8_layout(d->n, d->k, w->gate);
    w->tile_bytes = w->fp8.bytes();
    w->aux_bytes = w->fp8.n16 * sizeof(float);
  } else {
    w->aq4 = ullm::make_aq4_layout(d->n, d->k, w->gate);
    w->tile_bytes = w->aq4.words() * sizeof(uint32_t);
    w->aux_bytes = w->aq4.sz_words() * sizeof(uint32_t);
  }
  HIP_TRY(sink, "hipMalloc (weight tiles)", hipMalloc(&w->tiles, w->tile_bytes));
  HIP_TRY(sink, "hipMalloc (weight scales)", hipMalloc(&w->aux, w->aux_bytes));
  HIP_TRY(sink, "hipMemsetAsync", hipMemsetAsync(w->tiles, 0, w->tile_bytes, stream));
  HIP_TRY(sink, "hipMemsetAsync", hipMemsetAsync(w->aux, 0, w->aux_bytes, stream));

  DevBuf sv, ss, sz;
  const void *values = nullptr, *scales = nullptr, *zeros = nullptr;
  ullm_status_t st;
  if (d->source == ULLM_LINEAR_SOURCE_F32) {
    st = stage_source(d->values, d->n * d->k * sizeof(float), d->memory, sv,
                      &values, sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (fp8) {
      HIP_TRY(sink, "fp8 quantize kernel",
              ullm::launch_fp8_quantize(static_cast<const float *>(values), w->fp8,
                                        static_cast<uint8_t *>(w->tiles),
                                        static_cast<float *>(w->aux), stream));
    } else {
      HIP_TRY(sink, "aq4 quantize kernel",
              ullm::launch_aq4_quantize(static_cast<const float *>(values), w->aq4,
                                        static_cast<uint32_t *>(w->tiles),
                                        static_cast<uint32_t *>(w->aux), stream));
    }
  } else if (fp8) {
    st = stage_source(d->values, d->n * d->k, d->memory, sv, &values, sink);
    if (st == ULLM_STATUS_OK) {
      st = stage_source(d->scales, d->n * sizeof(float), d->memory, ss, &scales,
                        sink);
    }
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    HIP_TRY(sink, "fp8 pack kernel",
            ullm::launch_fp8_pack(static_cast<const uint8_t *>(values),
                                  static_cast<const float *>(scales), w->fp8,
                                  static_cast<uint8_t *>(w->tiles),
                                  static_cast<float *>(w->aux), stream));
  } else {
    const uint64_t gbytes = d->n * (d->k / 128) * sizeof(uint16_t);
    st = stage_source(d->values, d->n * (d->k / 8) * sizeof(uint32_t), d->memory,
                      sv, &values, sink);
    if (st == ULLM_STATUS_OK) {
      st = stage_source(d->scales, gbytes, d->memory, ss, &scales, sink);
    }
    if (st == ULLM_STATUS_OK) {
      st = stage_source(d->zeros, gbytes, d->memory, sz, &zeros, sink);
    }
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    HIP_TRY(sink, "aq4 pack kernel",
            ullm::launch_aq4_pack(static_cast<const uint32_t *>(values),
                                  static_cast<const uint16_t *>(scales),
                                  static_cast<const uint16_t *>(zeros), w->aq4,
                                  static_cast<uint32_t *>(w->tiles),
                                  static_cast<uint32_t *>(w->aux), stream));
  }
  HIP_TRY(sink, "hipStreamSynchronize", hipStreamSynchronize(stream));
  {
    std::lock_guard<std::mutex> lock(g_registry_mutex);
    g_registry.insert(w);
  }
  *out = w;
  owner.w = nullptr;
  return ULLM_STATUS_OK;
}

ullm_status_t validate_forward(const ullm_linear_forward_desc_t *d,
                               ullm_error_sink_t *sink) {
  ullm_status_t st = ullm::validate_header(d, sink, "forward descriptor is null");
  if (st != ULLM_STATUS_OK) {
    return st;
  }
  if (!ullm::all_zero(d->reserved)) {
    return write_error(sink, ULLM_STATUS_RESERVED_NONZERO,
                       "forward descriptor reserved fields must be zero");
  }
  st = lookup_weight(d->weight, sink);
  if (st != ULLM_STATUS_OK) {
    return st;
  }
  const ullm_linear_weight_t *w = d->weight;
  if (d->x_dtype != ULLM_LINEAR_DTYPE_BF16 &&
      d->x_dtype != ULLM_LINEAR_DTYPE_F8E4M3FN) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                       "activation dtype must be bf16 or f8e4m3fn");
  }
  if (d->y_dtype != ULLM_LINEAR_DTYPE_BF16 && d->y_dtype != ULLM_LINEAR_DTYPE_F32) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                       "output dtype must be bf16 or f32");
  }
  if (d->activation_mode != ULLM_LINEAR_ACT_EXACT &&
      d->activation_mode != ULLM_LINEAR_ACT_FP8_PER_TOKEN) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "unknown activation mode");
  }
  const bool fp8_acts = d->x_dtype == ULLM_LINEAR_DTYPE_F8E4M3FN ||
                        d->activation_mode == ULLM_LINEAR_ACT_FP8_PER_TOKEN;
  if (fp8_acts && w->encoding != ULLM_LINEAR_ENCODING_FP8_E4M3_ROW) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                       "FP8 activations require an FP8 weight");
  }
  if (d->x_dtype == ULLM_LINEAR_DTYPE_F8E4M3FN && d->x_scales == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "f8e4m3fn activations need x_scales");
  }
  if (d->x_row_stride != 0 && d->x_row_stride < w->k) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "x_row_stride is smaller than K");
  }
  if (d->epilogue != ULLM_LINEAR_EPILOGUE_NONE &&
      d->epilogue != ULLM_LINEAR_EPILOGUE_SILU_MUL &&
      d->epilogue != ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "unknown epilogue");
  }
  const bool gated = w->gate != 0;
  if (gated != (d->epilogue == ULLM_LINEAR_EPILOGUE_SILU_MUL)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       gated ? "a gated-pair weight needs the SILU_MUL epilogue"
                             : "SILU_MUL needs a gated-pair weight");
  }
  const uint64_t n_out = gated ? w->gate : w->n;
  if (d->y_row_stride != 0 && d->y_row_stride < n_out) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "y_row_stride is smaller than the output width");
  }
  if (d->epilogue == ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD) {
    if (d->residual_dtype != ULLM_LINEAR_DTYPE_BF16 &&
        d->residual_dtype != ULLM_LINEAR_DTYPE_F32) {
      return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                         "residual dtype must be bf16 or f32");
    }
    if (d->residual_row_stride != 0 && d->residual_row_stride < w->n) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "residual_row_stride is smaller than N");
    }
    if (d->m != 0 && d->residual == nullptr) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "residual pointer is null");
    }
    const uint64_t ldr = d->residual_row_stride ? d->residual_row_stride : w->n;
    const uint64_t ldy = d->y_row_stride ? d->y_row_stride : w->n;
    if (d->residual == d->y && (d->residual_dtype != d->y_dtype || ldr != ldy)) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "an in-place residual must match y's dtype and row stride");
    }
  } else if (d->residual != nullptr || d->residual_dtype != 0 ||
             d->residual_row_stride != 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "residual fields are set without the RESIDUAL_ADD epilogue");
  }
  if (d->m > 65535ULL * 32ULL) {
    return write_error(sink, ULLM_STATUS_UNSUPPORTED,
                       "M exceeds 2097120 rows per call");
  }
  if (d->m != 0 && (d->x == nullptr || d->y == nullptr)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "x or y pointer is null");
  }
  return ULLM_STATUS_OK;
}

// Prefill scratch: the split-K counter region (zero; prefill calls that do
// not split leave it alone), the split-K partial sums, then (for bf16
// activations) the quantized activations and their scales.
uint64_t prefill_split_bytes(const ullm::GemmPlan &p) {
  const uint64_t split = ullm::gemm_split_bytes(p);
  return split != 0 ? split : ullm::kGemmCounterBytes;
}
uint64_t prefill_workspace_bytes(uint64_t m, uint64_t k, const ullm::GemmPlan &p) {
  return prefill_split_bytes(p) + ullm::round_up(m * k, 256) +
         ullm::round_up(m * sizeof(float), 256);
}
// The GEMM plan of a prefill call; quantized activations in the workspace
// sit at a 256-byte multiple past its start.
ullm::GemmPlan prefill_plan(const ullm_linear_forward_desc_t *desc) {
  const ullm_linear_weight_t *w = desc->weight;
  const uint64_t ldx = desc->x_row_stride ? desc->x_row_stride : w->k;
  const bool prequant = desc->x_dtype == ULLM_LINEAR_DTYPE_F8E4M3FN;
  const void *xq = prequant ? desc->x : desc->workspace;  // null: library-owned
  return ullm::plan_fp8_gemm_call(xq, prequant ? ldx : w->k, w,
                                  static_cast<uint32_t>(desc->m));
}

}  // namespace

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_create(
    const ullm_linear_weight_desc_t *desc, ullm_linear_weight_t **weight,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight create", {
    ullm_status_t st = validate_weight_desc(desc, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (weight == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "weight output pointer is null");
    }
    *weight = nullptr;
    st = check_device(desc->device, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    DeviceScope scope(desc->device);
    HIP_TRY(error_sink, "hipSetDevice", scope.error());
    return create_weight(desc, weight, error_sink);
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_destroy(
    ullm_linear_weight_t **weight, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight destroy", {
    if (weight == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "weight handle pointer is null");
    }
    ullm_linear_weight_t *w = *weight;
    if (w == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "weight handle is null");
    }
    {
      std::lock_guard<std::mutex> lock(g_registry_mutex);
      if (g_registry.erase(w) == 0) {
        return write_error(error_sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                           "weight handle is not live");
      }
    }
    *weight = nullptr;
    DeviceScope scope(w->device);
    // hipFree synchronizes with outstanding work on the device.
    const hipError_t e1 = hipFree(w->tiles);
    const hipError_t e2 = hipFree(w->aux);
    delete w;
    if (e1 != hipSuccess) {
      return hip_fail(error_sink, "hipFree", e1);
    }
    if (e2 != hipSuccess) {
      return hip_fail(error_sink, "hipFree", e2);
    }
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_query(
    const ullm_linear_weight_t *weight, ullm_linear_weight_info_t *info,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight query", {
    ullm_status_t st = lookup_weight(weight, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    st = ullm::validate_header(info, error_sink, "weight info output is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(info->reserved) || info->reserved0 != 0) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "weight info reserved fields must be zero");
    }
    info->encoding = weight->encoding;
    info->device = weight->device;
    info->n = weight->n;
    info->k = weight->k;
    info->device_bytes = weight->tile_bytes + weight->aux_bytes;
    info->layout = weight->gate != 0 ? ULLM_LINEAR_LAYOUT_GATED_PAIRS
                                     : ULLM_LINEAR_LAYOUT_PLAIN;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_export(
    const ullm_linear_weight_t *weight,
    const ullm_linear_weight_export_desc_t *desc,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight export", {
    ullm_status_t st = lookup_weight(weight, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    st = ullm::validate_header(desc, error_sink, "export descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved) || desc->reserved0 != 0) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "export descriptor reserved fields must be zero");
    }
    if (desc->memory != ULLM_MEMORY_HOST && desc->memory != ULLM_MEMORY_DEVICE) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "unknown memory kind");
    }
    const bool fp8 = weight->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
    if (desc->values == nullptr || desc->scales == nullptr ||
        (!fp8 && desc->zeros == nullptr)) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "export destination pointer is null");
    }
    DeviceScope scope(weight->device);
    HIP_TRY(error_sink, "hipSetDevice", scope.error());
    const hipStream_t stream = static_cast<hipStream_t>(desc->stream);
    const uint64_t n = weight->n, k = weight->k;
    const uint64_t vbytes = fp8 ? n * k : n * (k / 8) * 4;
    const uint64_t sbytes = fp8 ? n * 4 : n * (k / 128) * 2;
    const bool host = desc->memory == ULLM_MEMORY_HOST;
    DevBuf bv, bs, bz;
    void *dv = desc->values, *ds = desc->scales, *dz = desc->zeros;
    if (host) {
      HIP_TRY(error_sink, "hipMalloc (staging)", hipMalloc(&bv.p, vbytes));
      HIP_TRY(error_sink, "hipMalloc (staging)", hipMalloc(&bs.p, sbytes));
      dv = bv.p;
      ds = bs.p;
      if (!fp8) {
        HIP_TRY(error_sink, "hipMalloc (staging)", hipMalloc(&bz.p, sbytes));
        dz = bz.p;
      }
    }
    if (fp8) {
      HIP_TRY(error_sink, "fp8 export kernel",
              ullm::launch_fp8_export(static_cast<const uint8_t *>(weight->tiles),
                                      static_cast<const float *>(weight->aux),
                                      weight->fp8, static_cast<uint8_t *>(dv),
                                      static_cast<float *>(ds), stream));
    } else {
      HIP_TRY(error_sink, "aq4 export kernel",
              ullm::launch_aq4_export(static_cast<const uint32_t *>(weight->tiles),
                                      static_cast<const uint32_t *>(weight->aux),
                                      weight->aq4, static_cast<uint32_t *>(dv),
                                      static_cast<uint16_t *>(ds),
                                      static_cast<uint16_t *>(dz), stream));
    }
    if (host) {
      HIP_TRY(error_sink, "hipStreamSynchronize", hipStreamSynchronize(stream));
      HIP_TRY(error_sink, "hipMemcpy",
              hipMemcpy(desc->values, dv, vbytes, hipMemcpyDeviceToHost));
      HIP_TRY(error_sink, "hipMemcpy",
              hipMemcpy(desc->scales, ds, sbytes, hipMemcpyDeviceToHost));
      if (!fp8) {
        HIP_TRY(error_sink, "hipMemcpy",
                hipMemcpy(desc->zeros, dz, sbytes, hipMemcpyDeviceToHost));
      }
    }
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_dequantize(
    const ullm_linear_weight_t *weight, float *out, void *stream,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight dequantize", {
    const ullm_status_t st = lookup_weight(weight, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (out == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "dequantize output pointer is null");
    }
    DeviceScope scope(weight->device);
    HIP_TRY(error_sink, "hipSetDevice", scope.error());
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (weight->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW) {
      HIP_TRY(error_sink, "fp8 dequantize kernel",
              ullm::launch_fp8_dequant(static_cast<const uint8_t *>(weight->tiles),
                                       static_cast<const float *>(weight->aux),
                                       weight->fp8, out, s));
    } else {
      HIP_TRY(error_sink, "aq4 dequantize kernel",
              ullm::launch_aq4_dequant(static_cast<const uint32_t *>(weight->tiles),
                                       static_cast<const uint32_t *>(weight->aux),
                                       weight->aq4, out, s));
    }
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_workspace_size(
    const ullm_linear_forward_desc_t *desc, uint64_t *bytes,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "workspace size", {
    const ullm_status_t st = validate_forward(desc, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (bytes == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "bytes output pointer is null");
    }
    const bool quantize = desc->x_dtype == ULLM_LINEAR_DTYPE_BF16 &&
                          desc->activation_mode == ULLM_LINEAR_ACT_FP8_PER_TOKEN;
    const ullm_linear_weight_t *w = desc->weight;
    if (quantize) {
      *bytes = desc->m == 0 ? 0 : prefill_workspace_bytes(desc->m, w->k, prefill_plan(desc));
    } else if (desc->x_dtype == ULLM_LINEAR_DTYPE_F8E4M3FN && desc->m != 0) {
      *bytes = ullm::gemm_split_bytes(prefill_plan(desc));
    } else if (desc->x_dtype == ULLM_LINEAR_DTYPE_BF16 && desc->m != 0) {
      // Decode: split-K scratch when the launch would split K.
      const bool fp8w = w->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
      ullm::GemvArgs a{};
      a.x = static_cast<const uint16_t *>(desc->x);
      a.ldx = desc->x_row_stride ? desc->x_row_stride : w->k;
      a.m = static_cast<uint32_t>(desc->m);
      a.n = static_cast<uint32_t>(w->n);
      a.k = static_cast<uint32_t>(w->k);
      a.n16 = static_cast<uint32_t>(fp8w ? w->fp8.n16 : w->aq4.n16);
      a.units = static_cast<uint32_t>(fp8w ? w->fp8.blocks_per_stripe() : w->aq4.groups);
      *bytes = ullm::gemv_scratch_bytes(a, !fp8w);
    } else {
      *bytes = 0;
    }
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_forward_plan(
    const ullm_linear_forward_desc_t *desc, ullm_linear_plan_t *plan,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "forward plan", {
    ullm_status_t st = validate_forward(desc, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    st = ullm::validate_header(plan, error_sink, "plan output is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(plan->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "plan reserved fields must be zero");
    }
    plan->kernel = 0;
    plan->block_m = plan->block_n = plan->tiles = plan->grid = 0;
    plan->split_k = 1;
    plan->gemv_variant = plan->gemv_waves = plan->gemv_stripes = 0;
    plan->gemv_row_classes = 0;
    if (desc->m == 0) {
      return ULLM_STATUS_OK;
    }
    const ullm_linear_weight_t *w = desc->weight;
    DeviceScope scope(w->device);
    HIP_TRY(error_sink, "hipSetDevice", scope.error());
    const uint64_t ldx = desc->x_row_stride ? desc->x_row_stride : w->k;
    const bool fp8w = w->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
    if (desc->x_dtype == ULLM_LINEAR_DTYPE_BF16 &&
        desc->activation_mode == ULLM_LINEAR_ACT_EXACT) {
      ullm::GemvArgs a{};
      a.x = static_cast<const uint16_t *>(desc->x);
      a.ldx = ldx;
      a.m = static_cast<uint32_t>(desc->m);
      a.n = static_cast<uint32_t>(w->n);
      a.k = static_cast<uint32_t>(w->k);
      a.n16 = static_cast<uint32_t>(fp8w ? w->fp8.n16 : w->aq4.n16);
      a.units = static_cast<uint32_t>(fp8w ? w->fp8.blocks_per_stripe() : w->aq4.groups);
      const ullm::GemvChoice c = ullm::gemv_choice(a, !fp8w, true);
      plan->kernel = ULLM_LINEAR_KERNEL_GEMV;
      plan->split_k = c.ks;
      plan->gemv_variant = c.variant;
      plan->gemv_waves = c.waves;
      plan->gemv_stripes = c.stripes;
      plan->gemv_row_classes = c.classes;
      return ULLM_STATUS_OK;
    }
    // The prefill path quantizes into the workspace (256-byte aligned past
    // its start); pre-quantized activations keep the caller's pointer and
    // stride.
    const ullm::GemmPlan p = prefill_plan(desc);
    plan->kernel = p.kind == ullm::kGemmDirect ? ULLM_LINEAR_KERNEL_GEMM_DIRECT
                                               : ULLM_LINEAR_KERNEL_GEMM_LDS;
    plan->block_m = p.block_m;
    plan->block_n = p.block_n;
    plan->tiles = p.tiles;
    plan->grid = p.grid;
    plan->split_k = p.ksplit;
    return ULLM_STATUS_OK;
  });
}

namespace ullm {

// One forward call: validation, then the decode GEMV or the prefill GEMM.
// Scratch (split-K counters and partials, quantized activations) comes from
// the caller's workspace or the library-owned buffers, or, when `fixed` is
// given, from the fixed scratch it returns for the weight's device (the
// allocation-free entry point); then nothing is allocated.
ullm_status_t forward_dispatch(const ullm_linear_forward_desc_t *desc,
                               ullm_error_sink_t *error_sink,
                               FixedScratchFn fixed) {
  const ullm_status_t st = validate_forward(desc, error_sink);
  if (st != ULLM_STATUS_OK) {
    return st;
  }
  if (fixed != nullptr && desc->workspace != nullptr) {
    return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "the allocation-free forward uses the library's fixed "
                       "scratch: workspace must be null");
  }
  if (desc->m == 0) {
    return ULLM_STATUS_OK;
  }
  const ullm_linear_weight_t *w = desc->weight;
  DeviceScope scope(w->device);
  HIP_TRY(error_sink, "hipSetDevice", scope.error());
  const hipStream_t s = static_cast<hipStream_t>(desc->stream);
  FixedScratch fs{};
  if (fixed != nullptr) {
    const ullm_status_t fst = fixed(w->device, s, &fs, error_sink);
    if (fst != ULLM_STATUS_OK) {
      return fst;
    }
  }
  const uint64_t ldx = desc->x_row_stride ? desc->x_row_stride : w->k;
  const uint64_t n_out = w->gate != 0 ? w->gate : w->n;
  const uint64_t ldy = desc->y_row_stride ? desc->y_row_stride : n_out;
  const bool y_f32 = desc->y_dtype == ULLM_LINEAR_DTYPE_F32;
  const bool fp8w = w->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
  ullm::Epilogue epi{};
  epi.kind = desc->epilogue == ULLM_LINEAR_EPILOGUE_SILU_MUL ? ullm::kEpiSiluMul
             : desc->epilogue == ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD
                 ? ullm::kEpiResidual
                 : ullm::kEpiNone;
  epi.n_out = static_cast<uint32_t>(n_out);
  epi.res = desc->residual;
  epi.ldr = desc->residual_row_stride ? desc->residual_row_stride : w->n;
  epi.res_f32 = desc->residual_dtype == ULLM_LINEAR_DTYPE_F32;

  if (desc->x_dtype == ULLM_LINEAR_DTYPE_BF16 &&
      desc->activation_mode == ULLM_LINEAR_ACT_EXACT) {
    ullm::GemvArgs a{};
    a.tiles = w->tiles;
    a.aux = w->aux;
    a.x = static_cast<const uint16_t *>(desc->x);
    a.y = desc->y;
    a.ldx = ldx;
    a.ldy = ldy;
    a.m = static_cast<uint32_t>(desc->m);
    a.n = static_cast<uint32_t>(w->n);
    a.k = static_cast<uint32_t>(w->k);
    a.alpha = desc->alpha;
    a.y_f32 = y_f32;
    a.epi = epi;
    a.n16 = static_cast<uint32_t>(fp8w ? w->fp8.n16 : w->aq4.n16);
    a.units = static_cast<uint32_t>(fp8w ? w->fp8.blocks_per_stripe() : w->aq4.groups);
    const uint64_t need = ullm::gemv_scratch_bytes(a, !fp8w);
    if (need != 0) {
      const uint64_t cnt_bytes = ullm::gemv_scratch_part_offset(a);
      if (fixed != nullptr) {
        // Counters in the fixed scratch's zeroed counter region (every
        // launch leaves them zero), partials past it.
        if (cnt_bytes > fs.counter_bytes || need - cnt_bytes > fs.bytes) {
          return write_errorf(error_sink, ULLM_STATUS_UNSUPPORTED,
                              "this call needs " + std::to_string(need) +
                                  " bytes of split-K scratch; the fixed scratch holds " +
                                  std::to_string(fs.bytes));
        }
        a.cnt = reinterpret_cast<uint32_t *>(fs.counters);
        a.part = reinterpret_cast<float *>(fs.base);
      } else {
        void *ws = desc->workspace;
        if (ws != nullptr) {
          if (desc->workspace_size < need) {
            return write_errorf(error_sink, ULLM_STATUS_BUFFER_TOO_SMALL,
                                "workspace needs " + std::to_string(need) + " bytes");
          }
        } else {
          const ullm_status_t st =
              library_workspace(w->device, desc->stream, true, need, &ws, error_sink);
          if (st != ULLM_STATUS_OK) {
            return st;
          }
        }
        a.cnt = static_cast<uint32_t *>(ws);
        a.part = reinterpret_cast<float *>(static_cast<char *>(ws) + cnt_bytes);
      }
    }
    if (fp8w) {
      a.n16 = static_cast<uint32_t>(w->fp8.n16);
      a.units = static_cast<uint32_t>(w->fp8.blocks_per_stripe());
      HIP_TRY(error_sink, "fp8 gemv kernel", ullm::launch_fp8_gemv(a, s));
    } else {
      a.n16 = static_cast<uint32_t>(w->aq4.n16);
      a.units = static_cast<uint32_t>(w->aq4.groups);
      HIP_TRY(error_sink, "aq4 gemv kernel", ullm::launch_aq4_gemv(a, s));
    }
    return ULLM_STATUS_OK;
  }

  // FP8 activations on the FP8 matrix cores.  Scratch layout: split-K
  // counters (zero on entry, left zero), split-K partial sums, then the
  // quantized activations and their scales when x is bf16.
  const bool prequant = desc->x_dtype == ULLM_LINEAR_DTYPE_F8E4M3FN;
  const ullm::GemmPlan plan = prefill_plan(desc);
  const uint64_t split = ullm::gemm_split_bytes(plan);
  const uint64_t head = prequant ? split : prefill_split_bytes(plan);
  const uint64_t need = prequant ? split : prefill_workspace_bytes(desc->m, w->k, plan);
  char *ws = nullptr;       // the scratch past the counter region
  void *counters = nullptr;  // the counter region
  if (need != 0) {
    if (fixed != nullptr) {
      if (need - ullm::kGemmCounterBytes > fs.bytes ||
          ullm::kGemmCounterBytes > fs.counter_bytes) {
        return write_errorf(error_sink, ULLM_STATUS_UNSUPPORTED,
                            "this call needs " + std::to_string(need) +
                                " bytes of prefill scratch; the fixed scratch holds " +
                                std::to_string(fs.bytes));
      }
      counters = fs.counters;
      ws = fs.base;
    } else {
      void *buf = desc->workspace;
      if (buf != nullptr) {
        if (desc->workspace_size < need) {
          return write_errorf(error_sink, ULLM_STATUS_BUFFER_TOO_SMALL,
                              "workspace needs " + std::to_string(need) + " bytes");
        }
      } else {
        const ullm_status_t st =
            library_workspace(w->device, desc->stream, true, need, &buf, error_sink);
        if (st != ULLM_STATUS_OK) {
          return st;
        }
      }
      counters = buf;
      ws = static_cast<char *>(buf) + ullm::kGemmCounterBytes;
    }
  }
  const uint8_t *xq = nullptr;
  const float *xs = nullptr;
  uint64_t ldxq = ldx;
  if (prequant) {
    xq = static_cast<const uint8_t *>(desc->x);
    xs = desc->x_scales;
  } else {
    uint8_t *wq = reinterpret_cast<uint8_t *>(ws) + (head - ullm::kGemmCounterBytes);
    float *wsc = reinterpret_cast<float *>(wq + ullm::round_up(desc->m * w->k, 256));
    HIP_TRY(error_sink, "activation quantize kernel",
            ullm::launch_act_quant(static_cast<const uint16_t *>(desc->x), ldx,
                                   desc->m, w->k, wq, wsc, s));
    xq = wq;
    xs = wsc;
    ldxq = w->k;
  }
  HIP_TRY(error_sink, "fp8 gemm kernel",
          ullm::launch_fp8_gemm(xq, xs, ldxq, w, static_cast<uint32_t>(desc->m),
                                desc->y, ldy, y_f32, desc->alpha, epi, plan,
                                static_cast<uint32_t *>(counters),
                                reinterpret_cast<float *>(ws), s));
  return ULLM_STATUS_OK;
}

}  // namespace ullm

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_forward(
    const ullm_linear_forward_desc_t *desc, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "linear forward", {
    return ullm::forward_dispatch(desc, error_sink, nullptr);
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_quantize_activations(
    const ullm_linear_act_quant_desc_t *desc, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "activation quantize", {
    const ullm_status_t st =
        ullm::validate_header(desc, error_sink, "activation descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "activation descriptor reserved fields must be zero");
    }
    if (desc->k == 0 || desc->k > kMaxDim || desc->m > kMaxDim) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "activation dimensions out of range");
    }
    if (desc->x_row_stride != 0 && desc->x_row_stride < desc->k) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "x_row_stride is smaller than K");
    }
    if (desc->m == 0) {
      return ULLM_STATUS_OK;
    }
    if (desc->x == nullptr || desc->xq == nullptr || desc->x_scales == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "activation pointer is null");
    }
    const uint64_t ldx = desc->x_row_stride ? desc->x_row_stride : desc->k;
    HIP_TRY(error_sink, "activation quantize kernel",
            ullm::launch_act_quant(static_cast<const uint16_t *>(desc->x), ldx,
                                   desc->m, desc->k,
                                   static_cast<uint8_t *>(desc->xq),
                                   desc->x_scales,
                                   static_cast<hipStream_t>(desc->stream)));
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_add_quantize_activations(
    const ullm_linear_add_act_quant_desc_t *desc, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "add and quantize activations", {
    const ullm_status_t st =
        ullm::validate_header(desc, error_sink, "activation descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "activation descriptor reserved fields must be zero");
    }
    if (desc->k == 0 || desc->k > kMaxDim || desc->m > kMaxDim) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "activation dimensions out of range");
    }
    for (const uint64_t ld : {desc->a_row_stride, desc->b_row_stride, desc->sum_row_stride}) {
      if (ld != 0 && ld < desc->k) {
        return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "a row stride is smaller than K");
      }
    }
    if (desc->m == 0) {
      return ULLM_STATUS_OK;
    }
    if (desc->a == nullptr || desc->b == nullptr || desc->xq == nullptr ||
        desc->x_scales == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "activation pointer is null");
    }
    const uint64_t lda = desc->a_row_stride ? desc->a_row_stride : desc->k;
    const uint64_t ldb = desc->b_row_stride ? desc->b_row_stride : desc->k;
    const uint64_t lds = desc->sum_row_stride ? desc->sum_row_stride : desc->k;
    if (desc->sum != nullptr &&
        ((desc->sum == desc->a && lds != lda) || (desc->sum == desc->b && lds != ldb))) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "an in-place sum needs the row stride of the input it replaces");
    }
    HIP_TRY(error_sink, "add and activation quantize kernel",
            ullm::launch_add_act_quant(
                static_cast<const uint16_t *>(desc->a), lda,
                static_cast<const uint16_t *>(desc->b), ldb,
                static_cast<uint16_t *>(desc->sum), lds, desc->m, desc->k,
                static_cast<uint8_t *>(desc->xq), desc->x_scales,
                static_cast<hipStream_t>(desc->stream)));
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_release_workspaces(
    int32_t device, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "release workspaces", {
    const ullm_status_t st = check_device(device, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    DeviceScope scope(device);
    HIP_TRY(error_sink, "hipSetDevice", scope.error());
    // Every stream of the device may still use a buffer.
    HIP_TRY(error_sink, "hipDeviceSynchronize", hipDeviceSynchronize());
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    hipError_t first = hipSuccess;
    for (auto it = g_ws.begin(); it != g_ws.end();) {
      if (it->first.device == device) {
        const hipError_t e = hipFree(it->second.ptr);
        first = first == hipSuccess ? e : first;
        it = g_ws.erase(it);
      } else {
        ++it;
      }
    }
    for (auto it = g_ws_retired.begin(); it != g_ws_retired.end();) {
      if (it->first == device) {
        const hipError_t e = hipFree(it->second);
        first = first == hipSuccess ? e : first;
        it = g_ws_retired.erase(it);
      } else {
        ++it;
      }
    }
    HIP_TRY(error_sink, "hipFree (workspace)", first);
    return ULLM_STATUS_OK;
  });
}
