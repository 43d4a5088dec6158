// abi_v1.cpp -- the reference's four ABI v1 functions, now backed by a real
// HIP runtime.  Argument validation and sink behaviour are those of the
// reference host stub (native/hip/src/hip_stub.cpp:120-219); the probes report
// a usable backend when a gfx950 device is visible instead of the stub's
// unconditional "unavailable".
#include <hip/hip_runtime_api.h>

#include <string>

#include "abi_common.hpp"
#include "ullm/hip.h"

namespace {

struct DeviceScan {
  bool runtime_present = false;
  int devices = 0;
  int gfx950 = 0;
  std::string detail;
};

DeviceScan scan_devices() {
  DeviceScan d;
  int count = 0;
  const hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess) {
    d.runtime_present = true;  // the runtime library answered
    d.detail = std::string("no HIP device visible (") + hipGetErrorName(err) + ")";
    return d;
  }
  d.runtime_present = true;
  d.devices = count;
  for (int i = 0; i < count; ++i) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, i) == hipSuccess &&
        std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) {
      ++d.gfx950;
    }
  }
  if (d.gfx950 == 0) {
    d.detail = "no gfx950 device among " + std::to_string(count) + " visible";
  }
  return d;
}

}  // namespace

extern "C" ULLM_HIP_API ullm_status_t
ullm_get_abi_version(uint32_t *abi_version, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "ABI version query", {
    if (abi_version == nullptr) {
      return ullm::write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                               "abi_version output is null");
    }
    *abi_version = ULLM_HIP_ABI_VERSION;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t
ullm_query_version(ullm_version_info_t *version, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "version query", {
    const ullm_status_t st =
        ullm::validate_header(version, error_sink, "version output is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(version->reserved)) {
      return ullm::write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                               "version reserved fields must be zero");
    }
    version->major = ULLM_HIP_LIBRARY_VERSION_MAJOR;
    version->minor = ULLM_HIP_LIBRARY_VERSION_MINOR;
    version->patch = ULLM_HIP_LIBRARY_VERSION_PATCH;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t
ullm_backend_probe(uint32_t backend, ullm_backend_probe_result_t *result,
                   ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "backend probe", {
    const ullm_status_t st =
        ullm::validate_header(result, error_sink, "probe result is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(result->reserved)) {
      return ullm::write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                               "probe result reserved fields must be zero");
    }
    if (backend != ULLM_BACKEND_HIP) {
      return ullm::write_error(error_sink, ULLM_STATUS_UNSUPPORTED,
                               "unknown backend identifier");
    }
    const DeviceScan d = scan_devices();
    result->backend = backend;
    result->hip_runtime_present = d.runtime_present ? 1U : 0U;
    result->available = d.gfx950 > 0 ? 1U : 0U;
    if (d.gfx950 == 0) {
      return ullm::write_errorf(error_sink, ULLM_STATUS_HIP_UNAVAILABLE,
                                "HIP backend is unavailable: " + d.detail);
    }
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t
ullm_context_probe(const ullm_context_t *context,
                   ullm_context_probe_result_t *result,
                   ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "context probe", {
    const ullm_status_t st = ullm::validate_header(
        result, error_sink, "context probe result is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(result->reserved)) {
      return ullm::write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                               "context probe reserved fields must be zero");
    }
    const DeviceScan d = scan_devices();
    result->context_present = context == nullptr ? 0U : 1U;
    result->hip_available = d.gfx950 > 0 ? 1U : 0U;
    if (d.gfx950 == 0) {
      return ullm::write_errorf(error_sink, ULLM_STATUS_HIP_UNAVAILABLE,
                                "HIP context is unavailable: " + d.detail);
    }
    return ULLM_STATUS_OK;
  });
}
