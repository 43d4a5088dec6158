//! What `HipBackend::supports` reports once the gfx950 library is linked
//! (reference crates/ullm-hip/src/lib.rs:496-505), for crates/ullm-hip.
//! Not compiled in this build's container (no Rust toolchain).
//!
//! Wiring (rust/patches/ullm-hip.patch): `mod backend_support;` in
//! crates/ullm-hip/src/lib.rs, and in
//! `impl Backend for HipBackend`:
//!
//! ```ignore
//! fn capabilities(&self) -> BackendCapabilities {
//!     BackendCapabilities { metadata_only: false, numerical_execution: true,
//!                           max_materialization_bytes: None }
//! }
//! fn supports(&self, operation: &SemanticOp) -> BackendSupport {
//!     backend_support::quantized_matmul_support(operation)
//! }
//! ```
//!
//! `execute` stays `BackendUnavailable` for `SemanticOp`s: the reference's
//! descriptors carry tensor metadata only (crates/ullm-core/src/tensor.rs:
//! 7-14), no device buffers, so there is nothing to run on.  Callers that
//! own device buffers run a supported Matmul through `linear::LinearWeight::
//! forward` (rust/ullm-hip/src/linear.rs), which is what the Python mirror
//! and every GPU test of this library call.

use ullm_core::{is_quantized_matmul, BackendSupport, SemanticOp, SemanticOpKind};

pub fn quantized_matmul_support(operation: &SemanticOp) -> BackendSupport {
    if operation.kind() != SemanticOpKind::Matmul {
        return BackendSupport::Unsupported {
            reason: "the HIP backend executes quantized Matmul only",
        };
    }
    let (inputs, outputs) = (operation.inputs(), operation.outputs());
    if inputs.len() == 2
        && outputs.len() == 1
        && is_quantized_matmul(&inputs[0], &inputs[1], &outputs[0])
    {
        BackendSupport::Supported
    } else {
        BackendSupport::Unsupported {
            reason: "Matmul needs bf16 activations and an FP8 row-scaled or AQ4 weight",
        }
    }
}
