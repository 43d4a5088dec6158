// abi_common.hpp -- error-sink and struct-header handling shared by every C
// entry point.  Semantics follow the reference's ABI v1 exactly
// (native/hip/src/hip_stub.cpp:10-83):
//   * a null sink is allowed and leaves the primary status unchanged;
//   * a sink with struct_size < 48, a wrong abi_version, non-zero reserved
//     words, or capacity without a buffer is rejected before anything else;
//   * messages are NUL-terminated and truncated to capacity - 1 bytes,
//     message_length always receives the full length, and truncation turns
//     the status into ULLM_STATUS_BUFFER_TOO_SMALL.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>

#include "ullm/linear.h"

namespace ullm {

inline ullm_status_t write_error(ullm_error_sink_t *sink, ullm_status_t status,
                                 const char *message) noexcept {
  if (sink == nullptr) {
    return status;
  }
  const std::size_t len = message == nullptr ? 0U : std::strlen(message);
  sink->message_length = static_cast<uint64_t>(len);
  if (sink->message_capacity == 0U) {
    return ULLM_STATUS_BUFFER_TOO_SMALL;
  }
  if (sink->message == nullptr) {
    return ULLM_STATUS_INVALID_ARGUMENT;
  }
  const std::size_t room = static_cast<std::size_t>(sink->message_capacity) - 1U;
  const std::size_t n = len < room ? len : room;
  if (n != 0U) {
    std::memcpy(sink->message, message, n);
  }
  sink->message[n] = '\0';
  return len <= room ? status : ULLM_STATUS_BUFFER_TOO_SMALL;
}

inline ullm_status_t write_errorf(ullm_error_sink_t *sink, ullm_status_t status,
                                  const std::string &message) noexcept {
  return write_error(sink, status, message.c_str());
}

inline ullm_status_t validate_sink(ullm_error_sink_t *sink) noexcept {
  if (sink == nullptr) {
    return ULLM_STATUS_OK;
  }
  if (sink->struct_size < sizeof(ullm_error_sink_t)) {
    return ULLM_STATUS_INVALID_ARGUMENT;
  }
  if (sink->abi_version != ULLM_HIP_ABI_VERSION) {
    return ULLM_STATUS_INVALID_ABI_VERSION;
  }
  if (sink->reserved[0] != 0U || sink->reserved[1] != 0U) {
    return ULLM_STATUS_RESERVED_NONZERO;
  }
  if (sink->message_capacity >
      static_cast<uint64_t>(std::numeric_limits<std::size_t>::max())) {
    return ULLM_STATUS_INVALID_ARGUMENT;
  }
  if (sink->message_capacity != 0U && sink->message == nullptr) {
    return ULLM_STATUS_INVALID_ARGUMENT;
  }
  sink->message_length = 0U;
  if (sink->message != nullptr && sink->message_capacity != 0U) {
    sink->message[0] = '\0';
  }
  return ULLM_STATUS_OK;
}

// Null pointer, short struct_size and ABI version checks for any struct that
// begins with {struct_size, abi_version}.
template <typename S>
ullm_status_t validate_header(const S *value, ullm_error_sink_t *sink,
                              const char *null_message) noexcept {
  if (value == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, null_message);
  }
  if (value->struct_size < sizeof(S)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "struct_size is smaller than the ABI v1 struct");
  }
  if (value->abi_version != ULLM_HIP_ABI_VERSION) {
    return write_error(sink, ULLM_STATUS_INVALID_ABI_VERSION,
                       "unsupported ABI version");
  }
  return ULLM_STATUS_OK;
}

template <typename T, std::size_t N>
bool all_zero(const T (&words)[N]) noexcept {
  for (std::size_t i = 0; i < N; ++i) {
    if (words[i] != 0) {
      return false;
    }
  }
  return true;
}

}  // namespace ullm

// Wraps an entry point body so that no C++ exception crosses the ABI
// (reference hip_stub.cpp:123,134): the sink is validated first, then the
// body runs; any exception becomes ULLM_STATUS_INTERNAL_ERROR.
#define ULLM_ENTRY(sink, what, ...)                                           \
  do {                                                                        \
    try {                                                                     \
      const ullm_status_t sink_status_ = ::ullm::validate_sink(sink);         \
      if (sink_status_ != ULLM_STATUS_OK) {                                   \
        return sink_status_;                                                  \
      }                                                                       \
      __VA_ARGS__                                                             \
    } catch (...) {                                                           \
      return ::ullm::write_error(sink, ULLM_STATUS_INTERNAL_ERROR,            \
                                 "unexpected exception in " what);            \
    }                                                                         \
  } while (0)
