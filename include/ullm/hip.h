/*
 * ullm/hip.h -- versioned C ABI v1 of the uLLM HIP backend (gfx950 build).
 *
 * The v1 surface (statuses, error sink, probe structs and the four probe
 * functions) must stay binary-identical to the reference's public header so
 * that crates/ullm-hip-sys/src/bindings.rs:1-119 binds this library
 * unchanged.  Each declaration cites the reference interface it replaces:
 *   reference include/ullm/hip.h:16-19   ABI / library version macros
 *   reference include/ullm/hip.h:21-30   status codes 0..7
 *   reference include/ullm/hip.h:32-38   backend id and access modes
 *   reference include/ullm/hip.h:40-46   opaque handles
 *   reference include/ullm/hip.h:48-73   error sink and its initializer
 *   reference include/ullm/hip.h:75-100  probe structs
 *   reference include/ullm/hip.h:106-121 probe functions
 * The linear-layer extension lives in ullm/linear.h.
 */
#ifndef ULLM_HIP_H
#define ULLM_HIP_H

#include <stdint.h>

/* Export control (reference include/ullm/hip.h:6-13).  A Windows DLL build
 * defines ULLM_HIP_SHARED (and ULLM_HIP_BUILD while compiling the library);
 * ELF builds compile with -fvisibility=hidden, so the public entry points
 * carry default visibility explicitly, in the shared library and in the
 * static archive alike. */
#if defined(_WIN32) && defined(ULLM_HIP_SHARED)
#if defined(ULLM_HIP_BUILD)
#define ULLM_HIP_API __declspec(dllexport)
#else
#define ULLM_HIP_API __declspec(dllimport)
#endif
#elif defined(__GNUC__)
#define ULLM_HIP_API __attribute__((visibility("default")))
#else
#define ULLM_HIP_API
#endif

#define ULLM_HIP_ABI_VERSION UINT32_C(1)
#define ULLM_HIP_LIBRARY_VERSION_MAJOR UINT32_C(0)
#define ULLM_HIP_LIBRARY_VERSION_MINOR UINT32_C(2)
#define ULLM_HIP_LIBRARY_VERSION_PATCH UINT32_C(0)

typedef uint32_t ullm_status_t;

/* Public statuses (reference hip.h:23-30). */
#define ULLM_STATUS_OK UINT32_C(0)
#define ULLM_STATUS_INVALID_ARGUMENT UINT32_C(1)
#define ULLM_STATUS_BUFFER_TOO_SMALL UINT32_C(2)
#define ULLM_STATUS_UNSUPPORTED UINT32_C(3)
#define ULLM_STATUS_HIP_UNAVAILABLE UINT32_C(4)
#define ULLM_STATUS_INVALID_ABI_VERSION UINT32_C(5)
#define ULLM_STATUS_RESERVED_NONZERO UINT32_C(6)
#define ULLM_STATUS_INTERNAL_ERROR UINT32_C(7)

#define ULLM_BACKEND_HIP UINT32_C(1)

typedef uint32_t ullm_access_mode_t;

#define ULLM_ACCESS_READ UINT32_C(1)
#define ULLM_ACCESS_WRITE UINT32_C(2)
#define ULLM_ACCESS_READ_WRITE UINT32_C(3)

/* Opaque handles: callers never dereference them. */
typedef struct ullm_context_t ullm_context_t;
typedef struct ullm_queue_t ullm_queue_t;
typedef struct ullm_buffer_t ullm_buffer_t;
typedef struct ullm_event_t ullm_event_t;
typedef struct ullm_completion_t ullm_completion_t;

/* Caller-owned diagnostic sink, 48 bytes on LP64.
 * message_capacity counts the terminating NUL.  On a diagnostic error
 * message_length receives the full message length (without NUL) even when the
 * copy is truncated; a truncated copy returns ULLM_STATUS_BUFFER_TOO_SMALL.
 * A null sink leaves the primary status unchanged. */
typedef struct ullm_error_sink_t {
  uint32_t struct_size;
  uint32_t abi_version;
  char *message;
  uint64_t message_capacity;
  uint64_t message_length;
  uint64_t reserved[2];
} ullm_error_sink_t;

/* Initializer for a sink over a character array (not a pointer). */
#define ULLM_ERROR_SINK_INIT(buffer)                                           \
  {sizeof(ullm_error_sink_t), ULLM_HIP_ABI_VERSION, (buffer), sizeof(buffer), \
   0, {0, 0}}

typedef struct ullm_version_info_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t major;
  uint32_t minor;
  uint32_t patch;
  uint32_t reserved[3];
} ullm_version_info_t;

typedef struct ullm_backend_probe_result_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t backend;
  uint32_t available;
  uint32_t hip_runtime_present;
  uint32_t reserved[3];
} ullm_backend_probe_result_t;

typedef struct ullm_context_probe_result_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t context_present;
  uint32_t hip_available;
  uint32_t reserved[4];
} ullm_context_probe_result_t;

#ifdef __cplusplus
extern "C" {
#endif

/* reference hip.h:106-107 */
ULLM_HIP_API ullm_status_t ullm_get_abi_version(uint32_t *abi_version,
                                                ullm_error_sink_t *error_sink);

/* reference hip.h:109-110 */
ULLM_HIP_API ullm_status_t ullm_query_version(ullm_version_info_t *version,
                                              ullm_error_sink_t *error_sink);

/* reference hip.h:112-115.  Reports available=1 and ULLM_STATUS_OK when a
 * gfx950 device is visible; otherwise ULLM_STATUS_HIP_UNAVAILABLE with a
 * diagnostic naming what is missing. */
ULLM_HIP_API ullm_status_t
ullm_backend_probe(uint32_t backend, ullm_backend_probe_result_t *result,
                   ullm_error_sink_t *error_sink);

/* reference hip.h:117-121.  The handle is never dereferenced. */
ULLM_HIP_API ullm_status_t ullm_context_probe(
    const ullm_context_t *context, ullm_context_probe_result_t *result,
    ullm_error_sink_t *error_sink);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* ULLM_HIP_H */
