// Bindings of the gfx950 library's linear-layer ABI (include/ullm/linear.h)
// and weight-file ABI (include/ullm/weights_io.h), for
// crates/ullm-hip-sys.  Not compiled in this build's container (no Rust
// toolchain).  tests/test_rust_bindings.py checks every constant, struct
// layout and function signature here against the C headers, and
// abi_layout_probe.rs prints the layouts for the patched build.rs's
// comparison with the C++ probe (reference crates/ullm-hip-sys/build.rs:330-408).
//
// Wiring (rust/patches/ullm-hip-sys.patch): `pub mod linear {
// include!("linear_bindings.rs"); }` in
// crates/ullm-hip-sys/src/lib.rs, next to the `evidence` module
// (reference crates/ullm-hip-sys/src/lib.rs:8-13).  The evidence functions
// keep their existing bindings (evidence_bindings.rs) unchanged; this
// library exports them.

use core::ffi::{c_char, c_void};

use crate::{ullm_error_sink_t, ullm_status_t};

pub const ULLM_STATUS_OUT_OF_MEMORY: ullm_status_t = 13;

pub const ULLM_LINEAR_ENCODING_FP8_E4M3_ROW: u32 = 1;
pub const ULLM_LINEAR_ENCODING_AQ4_G128: u32 = 2;
pub const ULLM_LINEAR_LAYOUT_PLAIN: u32 = 0;
pub const ULLM_LINEAR_LAYOUT_GATED_PAIRS: u32 = 1;
pub const ULLM_LINEAR_EPILOGUE_NONE: u32 = 0;
pub const ULLM_LINEAR_EPILOGUE_SILU_MUL: u32 = 1;
pub const ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD: u32 = 2;
pub const ULLM_LINEAR_SOURCE_F32: u32 = 1;
pub const ULLM_LINEAR_SOURCE_ENCODED: u32 = 2;
pub const ULLM_MEMORY_HOST: u32 = 1;
pub const ULLM_MEMORY_DEVICE: u32 = 2;
pub const ULLM_LINEAR_DTYPE_BF16: u32 = 1;
pub const ULLM_LINEAR_DTYPE_F32: u32 = 2;
pub const ULLM_LINEAR_DTYPE_F8E4M3FN: u32 = 3;
pub const ULLM_LINEAR_ACT_EXACT: u32 = 0;
pub const ULLM_LINEAR_ACT_FP8_PER_TOKEN: u32 = 1;
pub const ULLM_LINEAR_KERNEL_GEMV: u32 = 1;
pub const ULLM_LINEAR_KERNEL_GEMM_DIRECT: u32 = 2;
pub const ULLM_LINEAR_KERNEL_GEMM_LDS: u32 = 3;
pub const ULLM_LINEAR_GEMV_SINGLE: u32 = 1;
pub const ULLM_LINEAR_GEMV_SINGLE_LDS: u32 = 2;
pub const ULLM_LINEAR_GEMV_MULTI_STRIPE: u32 = 3;
pub const ULLM_LINEAR_GEMV_REGISTER_STAGED: u32 = 4;
pub const ULLM_LINEAR_GEMV_SPLIT_K: u32 = 5;

#[repr(C)]
pub struct ullm_linear_weight_t {
    _private: [u8; 0],
}

/// 104 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_weight_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub encoding: u32,
    pub source: u32,
    pub n: u64,
    pub k: u64,
    pub memory: u32,
    pub device: i32,
    pub values: *const c_void,
    pub scales: *const c_void,
    pub zeros: *const c_void,
    pub stream: *mut c_void,
    pub layout: u32,
    pub reserved0: u32,
    pub reserved: [u64; 3],
}

/// 72 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_weight_info_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub encoding: u32,
    pub device: i32,
    pub n: u64,
    pub k: u64,
    pub device_bytes: u64,
    pub layout: u32,
    pub reserved0: u32,
    pub reserved: [u64; 3],
}

/// 136 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_forward_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub weight: *const ullm_linear_weight_t,
    pub m: u64,
    pub x: *const c_void,
    pub x_row_stride: u64,
    pub x_scales: *const f32,
    pub y: *mut c_void,
    pub y_row_stride: u64,
    pub x_dtype: u32,
    pub y_dtype: u32,
    pub activation_mode: u32,
    pub alpha: f32,
    pub stream: *mut c_void,
    pub workspace: *mut c_void,
    pub workspace_size: u64,
    pub epilogue: u32,
    pub residual_dtype: u32,
    pub residual: *const c_void,
    pub residual_row_stride: u64,
    pub reserved: [u64; 1],
}

/// 64 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_plan_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub kernel: u32,
    pub block_m: u32,
    pub block_n: u32,
    pub tiles: u32,
    pub grid: u32,
    pub split_k: u32,
    pub gemv_variant: u32,
    pub gemv_waves: u32,
    pub gemv_stripes: u32,
    pub gemv_row_classes: u32,
    pub reserved: [u64; 2],
}

/// 96 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_act_quant_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub m: u64,
    pub k: u64,
    pub x: *const c_void,
    pub x_row_stride: u64,
    pub xq: *mut c_void,
    pub x_scales: *mut f32,
    pub stream: *mut c_void,
    pub reserved: [u64; 4],
}

/// 128 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_add_act_quant_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub m: u64,
    pub k: u64,
    pub a: *const c_void,
    pub a_row_stride: u64,
    pub b: *const c_void,
    pub b_row_stride: u64,
    pub sum: *mut c_void,
    pub sum_row_stride: u64,
    pub xq: *mut c_void,
    pub x_scales: *mut f32,
    pub stream: *mut c_void,
    pub reserved: [u64; 4],
}

/// 80 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_weight_export_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub memory: u32,
    pub reserved0: u32,
    pub values: *mut c_void,
    pub scales: *mut c_void,
    pub zeros: *mut c_void,
    pub stream: *mut c_void,
    pub reserved: [u64; 4],
}

pub const ULLM_ST_DTYPE_BOOL: u32 = 1;
pub const ULLM_ST_DTYPE_U8: u32 = 2;
pub const ULLM_ST_DTYPE_I8: u32 = 3;
pub const ULLM_ST_DTYPE_F8_E4M3: u32 = 4;
pub const ULLM_ST_DTYPE_F8_E5M2: u32 = 5;
pub const ULLM_ST_DTYPE_U16: u32 = 6;
pub const ULLM_ST_DTYPE_I16: u32 = 7;
pub const ULLM_ST_DTYPE_F16: u32 = 8;
pub const ULLM_ST_DTYPE_BF16: u32 = 9;
pub const ULLM_ST_DTYPE_U32: u32 = 10;
pub const ULLM_ST_DTYPE_I32: u32 = 11;
pub const ULLM_ST_DTYPE_F32: u32 = 12;
pub const ULLM_ST_DTYPE_U64: u32 = 13;
pub const ULLM_ST_DTYPE_I64: u32 = 14;
pub const ULLM_ST_DTYPE_F64: u32 = 15;
pub const ULLM_ST_MAX_RANK: u32 = 8;

#[repr(C)]
pub struct ullm_safetensors_t {
    _private: [u8; 0],
}

/// 64 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_safetensors_open_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub path: *const c_char,
    pub expected_sha256: *const u8,
    pub expected_size: u64,
    pub reserved: [u64; 4],
}

/// 128 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_safetensors_tensor_info_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub dtype: u32,
    pub rank: u32,
    pub shape: [u64; 8],
    pub offset: u64,
    pub bytes: u64,
    pub reserved: [u64; 4],
}

/// 96 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_weight_load_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub file: *const ullm_safetensors_t,
    pub encoding: u32,
    pub layout: u32,
    pub values: *const *const c_char,
    pub value_parts: u32,
    pub device: i32,
    pub scales: *const c_char,
    pub zeros: *const c_char,
    pub stream: *mut c_void,
    pub reserved: [u64; 4],
}

/// 96 bytes.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ullm_linear_weights_save_desc_t {
    pub struct_size: u32,
    pub abi_version: u32,
    pub path: *const c_char,
    pub names: *const *const c_char,
    pub weights: *const *const ullm_linear_weight_t,
    pub count: u64,
    pub metadata_keys: *const *const c_char,
    pub metadata_values: *const *const c_char,
    pub metadata_count: u64,
    pub reserved: [u64; 4],
}

unsafe extern "C" {
    pub fn ullm_linear_weight_create(
        desc: *const ullm_linear_weight_desc_t,
        weight: *mut *mut ullm_linear_weight_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weight_destroy(
        weight: *mut *mut ullm_linear_weight_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weight_query(
        weight: *const ullm_linear_weight_t,
        info: *mut ullm_linear_weight_info_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weight_export(
        weight: *const ullm_linear_weight_t,
        desc: *const ullm_linear_weight_export_desc_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weight_dequantize(
        weight: *const ullm_linear_weight_t,
        out: *mut f32,
        stream: *mut c_void,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_forward(
        desc: *const ullm_linear_forward_desc_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_forward_noalloc(
        desc: *const ullm_linear_forward_desc_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_forward_plan(
        desc: *const ullm_linear_forward_desc_t,
        plan: *mut ullm_linear_plan_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_workspace_size(
        desc: *const ullm_linear_forward_desc_t,
        bytes: *mut u64,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_release_workspaces(
        device: i32,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_quantize_activations(
        desc: *const ullm_linear_act_quant_desc_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_add_quantize_activations(
        desc: *const ullm_linear_add_act_quant_desc_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;

    pub fn ullm_safetensors_open(
        desc: *const ullm_safetensors_open_desc_t,
        file: *mut *mut ullm_safetensors_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_close(
        file: *mut *mut ullm_safetensors_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_tensor_count(
        file: *const ullm_safetensors_t,
        count: *mut u64,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_tensor_name(
        file: *const ullm_safetensors_t,
        index: u64,
        name: *mut c_char,
        capacity: u64,
        length: *mut u64,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_tensor_info(
        file: *const ullm_safetensors_t,
        name: *const c_char,
        info: *mut ullm_safetensors_tensor_info_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_metadata(
        file: *const ullm_safetensors_t,
        key: *const c_char,
        value: *mut c_char,
        capacity: u64,
        length: *mut u64,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_safetensors_file_sha256(
        file: *const ullm_safetensors_t,
        sha256: *mut u8,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weight_load(
        desc: *const ullm_linear_weight_load_desc_t,
        weight: *mut *mut ullm_linear_weight_t,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
    pub fn ullm_linear_weights_save(
        desc: *const ullm_linear_weights_save_desc_t,
        sha256: *mut u8,
        error_sink: *mut ullm_error_sink_t,
    ) -> ullm_status_t;
}
