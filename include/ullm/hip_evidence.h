/*
 * ullm/hip_evidence.h -- the model-free HIP evidence ABI (gfx950 build).
 *
 * Declarations follow the reference's private evidence header
 * (native/hip/src/evidence_abi.h:10-60) byte for byte, so that the Rust
 * bindings (crates/ullm-hip-sys/src/evidence_bindings.rs:1-74) link against
 * this library unchanged and ullm-hip's submit_evidence / wait / Drop
 * (crates/ullm-hip/src/lib.rs:293-441) keep their behaviour:
 *
 *   submit  copies the caller's bytes at once (the caller's pointer is never
 *           kept), and queues on the device exactly two device allocations,
 *           two host<->device copies and one kernel dispatch that writes
 *           input[i] ^ 0x5a;
 *   wait    consumes the handle whatever it returns; polls for completion up
 *           to timeout_ms (0 = one poll), then ULLM_STATUS_HIP_TIMEOUT;
 *   destroy consumes a live handle and nulls *completion;
 *   a handle that is not live (consumed, destroyed, never issued) is
 *   ULLM_STATUS_HIP_INVALID_HANDLE.
 *
 * At most two completions are outstanding at once (live handles plus
 * consumed ones whose device work has not finished), as in the reference
 * (hip_evidence_runtime.hip.cpp:35); a further submit is
 * ULLM_STATUS_INTERNAL_ERROR.  It needs exactly one visible gfx950 device.
 */
#ifndef ULLM_HIP_EVIDENCE_H
#define ULLM_HIP_EVIDENCE_H

#include <stdint.h>

#include "ullm/hip.h"

#define ULLM_HIP_EVIDENCE_ABI_VERSION UINT32_C(1)
#define ULLM_HIP_EVIDENCE_TRANSFORM_XOR UINT8_C(0x5a)

/* Status values 8..12 (evidence_abi.h:13-17). */
#ifndef ULLM_STATUS_HIP_TIMEOUT
#define ULLM_STATUS_HIP_TIMEOUT UINT32_C(8)
#define ULLM_STATUS_HIP_INVALID_HANDLE UINT32_C(9)
#define ULLM_STATUS_HIP_ZERO_DISPATCH UINT32_C(10)
#define ULLM_STATUS_HIP_RUNTIME_ERROR UINT32_C(11)
#define ULLM_STATUS_HIP_DISPATCH_CONTRACT UINT32_C(12)
#endif

/* 40 bytes (evidence_abi.h:19-25). */
typedef struct ullm_hip_evidence_request_t {
  uint32_t struct_size;
  uint32_t abi_version; /* ULLM_HIP_EVIDENCE_ABI_VERSION */
  const uint8_t *input; /* host bytes, non-null */
  uint64_t input_size;  /* >= 1 */
  uint32_t reserved[4];
} ullm_hip_evidence_request_t;

/* 72 bytes (evidence_abi.h:27-40). */
typedef struct ullm_hip_evidence_result_t {
  uint32_t struct_size;
  uint32_t abi_version; /* ULLM_HIP_EVIDENCE_ABI_VERSION */
  uint64_t output_size;
  /* Successful device allocations; excludes pinned host staging. */
  uint64_t allocation_count;
  /* Successful host<->device transfers; excludes CPU memcpy. */
  uint64_t copy_count;
  uint64_t dispatch_count;
  uint32_t selected_backend; /* ULLM_BACKEND_HIP */
  uint32_t fallback_used;    /* always 0: there is no CPU path */
  uint32_t terminal;         /* 1: the handle is consumed */
  uint32_t reserved[4];
} ullm_hip_evidence_result_t;

typedef struct ullm_hip_evidence_completion_t ullm_hip_evidence_completion_t;

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces ullm_hip_evidence_submit (evidence_abi.h:48-50). */
ULLM_HIP_API ullm_status_t ullm_hip_evidence_submit(
    const ullm_hip_evidence_request_t *request,
    ullm_hip_evidence_completion_t **completion,
    struct ullm_error_sink_t *error_sink);

/* Replaces ullm_hip_evidence_wait (evidence_abi.h:52-56).  output must hold
 * input_size bytes. */
ULLM_HIP_API ullm_status_t ullm_hip_evidence_wait(
    ullm_hip_evidence_completion_t *completion, uint32_t timeout_ms,
    uint8_t *output, uint64_t output_capacity,
    ullm_hip_evidence_result_t *result, struct ullm_error_sink_t *error_sink);

/* Replaces ullm_hip_evidence_destroy (evidence_abi.h:58-59). */
ULLM_HIP_API ullm_status_t ullm_hip_evidence_destroy(
    ullm_hip_evidence_completion_t **completion,
    struct ullm_error_sink_t *error_sink);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* ULLM_HIP_EVIDENCE_H */
