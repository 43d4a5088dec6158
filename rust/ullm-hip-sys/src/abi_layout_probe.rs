//! ABI layout probe of the checked-in Rust bindings: the counterpart of
//! native/hip/src/abi_layout_probe.cpp, printing the same lines from the
//! Rust declarations.  The patched crates/ullm-hip-sys/build.rs compiles it
//! with rustc (as the reference build.rs:393-404 compiles its generated
//! probe) and requires its output to equal the C++ probe's, once without
//! arguments (hip.h, bindings.rs) and once with `--extensions` (linear.h and
//! weights_io.h, linear_bindings.rs).
#![allow(non_camel_case_types, non_upper_case_globals, dead_code)]

#[path = "bindings.rs"]
mod bindings;
pub use bindings::*;

#[path = "evidence_bindings.rs"]
pub mod evidence;

pub mod linear {
    include!("linear_bindings.rs");
}

use evidence::*;
use linear::*;
use std::mem::{align_of, offset_of, size_of};

macro_rules! consts {
    ($($name:ident),* $(,)?) => {
        $(println!("const {}={}", stringify!($name), $name);)*
    };
}

macro_rules! layout {
    ($ty:ident { $($field:ident),* $(,)? }) => {{
        print!("layout {} size={} align={}", stringify!($ty), size_of::<$ty>(), align_of::<$ty>());
        $(print!(" {}={}", stringify!($field), offset_of!($ty, $field));)*
        println!();
    }};
}

fn print_v1() {
    consts!(
        ULLM_HIP_ABI_VERSION,
        ULLM_HIP_LIBRARY_VERSION_MAJOR,
        ULLM_HIP_LIBRARY_VERSION_MINOR,
        ULLM_HIP_LIBRARY_VERSION_PATCH,
        ULLM_STATUS_OK,
        ULLM_STATUS_INVALID_ARGUMENT,
        ULLM_STATUS_BUFFER_TOO_SMALL,
        ULLM_STATUS_UNSUPPORTED,
        ULLM_STATUS_HIP_UNAVAILABLE,
        ULLM_STATUS_INVALID_ABI_VERSION,
        ULLM_STATUS_RESERVED_NONZERO,
        ULLM_STATUS_INTERNAL_ERROR,
        ULLM_BACKEND_HIP,
        ULLM_ACCESS_READ,
        ULLM_ACCESS_WRITE,
        ULLM_ACCESS_READ_WRITE,
    );
    layout!(ullm_error_sink_t {
        struct_size, abi_version, message, message_capacity, message_length, reserved,
    });
    layout!(ullm_version_info_t {
        struct_size, abi_version, major, minor, patch, reserved,
    });
    layout!(ullm_backend_probe_result_t {
        struct_size, abi_version, backend, available, hip_runtime_present, reserved,
    });
    layout!(ullm_context_probe_result_t {
        struct_size, abi_version, context_present, hip_available, reserved,
    });
}

fn print_extensions() {
    consts!(
        ULLM_STATUS_HIP_TIMEOUT,
        ULLM_STATUS_HIP_INVALID_HANDLE,
        ULLM_STATUS_HIP_ZERO_DISPATCH,
        ULLM_STATUS_HIP_RUNTIME_ERROR,
        ULLM_STATUS_HIP_DISPATCH_CONTRACT,
        ULLM_STATUS_OUT_OF_MEMORY,
        ULLM_LINEAR_ENCODING_FP8_E4M3_ROW,
        ULLM_LINEAR_ENCODING_AQ4_G128,
        ULLM_LINEAR_LAYOUT_PLAIN,
        ULLM_LINEAR_LAYOUT_GATED_PAIRS,
        ULLM_LINEAR_EPILOGUE_NONE,
        ULLM_LINEAR_EPILOGUE_SILU_MUL,
        ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD,
        ULLM_LINEAR_SOURCE_F32,
        ULLM_LINEAR_SOURCE_ENCODED,
        ULLM_MEMORY_HOST,
        ULLM_MEMORY_DEVICE,
        ULLM_LINEAR_DTYPE_BF16,
        ULLM_LINEAR_DTYPE_F32,
        ULLM_LINEAR_DTYPE_F8E4M3FN,
        ULLM_LINEAR_ACT_EXACT,
        ULLM_LINEAR_ACT_FP8_PER_TOKEN,
        ULLM_LINEAR_KERNEL_GEMV,
        ULLM_LINEAR_KERNEL_GEMM_DIRECT,
        ULLM_LINEAR_KERNEL_GEMM_LDS,
        ULLM_LINEAR_GEMV_SINGLE,
        ULLM_LINEAR_GEMV_SINGLE_LDS,
        ULLM_LINEAR_GEMV_MULTI_STRIPE,
        ULLM_LINEAR_GEMV_REGISTER_STAGED,
        ULLM_LINEAR_GEMV_SPLIT_K,
    );
    layout!(ullm_linear_weight_desc_t {
        struct_size, abi_version, encoding, source, n, k, memory, device, values,
        scales, zeros, stream, layout, reserved0, reserved,
    });
    layout!(ullm_linear_weight_info_t {
        struct_size, abi_version, encoding, device, n, k, device_bytes, layout,
        reserved0, reserved,
    });
    layout!(ullm_linear_forward_desc_t {
        struct_size, abi_version, weight, m, x, x_row_stride, x_scales, y, y_row_stride,
        x_dtype, y_dtype, activation_mode, alpha, stream, workspace, workspace_size,
        epilogue, residual_dtype, residual, residual_row_stride, reserved,
    });
    layout!(ullm_linear_act_quant_desc_t {
        struct_size, abi_version, m, k, x, x_row_stride, xq, x_scales, stream, reserved,
    });
    layout!(ullm_linear_add_act_quant_desc_t {
        struct_size, abi_version, m, k, a, a_row_stride, b, b_row_stride, sum,
        sum_row_stride, xq, x_scales, stream, reserved,
    });
    layout!(ullm_linear_weight_export_desc_t {
        struct_size, abi_version, memory, reserved0, values, scales, zeros, stream,
        reserved,
    });
    layout!(ullm_linear_plan_t {
        struct_size, abi_version, kernel, block_m, block_n, tiles, grid, split_k,
        gemv_variant, gemv_waves, gemv_stripes, gemv_row_classes, reserved,
    });
    consts!(
        ULLM_ST_DTYPE_BOOL,
        ULLM_ST_DTYPE_U8,
        ULLM_ST_DTYPE_I8,
        ULLM_ST_DTYPE_F8_E4M3,
        ULLM_ST_DTYPE_F8_E5M2,
        ULLM_ST_DTYPE_U16,
        ULLM_ST_DTYPE_I16,
        ULLM_ST_DTYPE_F16,
        ULLM_ST_DTYPE_BF16,
        ULLM_ST_DTYPE_U32,
        ULLM_ST_DTYPE_I32,
        ULLM_ST_DTYPE_F32,
        ULLM_ST_DTYPE_U64,
        ULLM_ST_DTYPE_I64,
        ULLM_ST_DTYPE_F64,
        ULLM_ST_MAX_RANK,
    );
    layout!(ullm_safetensors_open_desc_t {
        struct_size, abi_version, path, expected_sha256, expected_size, reserved,
    });
    layout!(ullm_safetensors_tensor_info_t {
        struct_size, abi_version, dtype, rank, shape, offset, bytes, reserved,
    });
    layout!(ullm_linear_weight_load_desc_t {
        struct_size, abi_version, file, encoding, layout, values, value_parts, device,
        scales, zeros, stream, reserved,
    });
    layout!(ullm_linear_weights_save_desc_t {
        struct_size, abi_version, path, names, weights, count, metadata_keys,
        metadata_values, metadata_count, reserved,
    });
}

fn main() {
    let args: Vec<String> = std::env::args().skip(1).collect();
    match args.as_slice() {
        [] => print_v1(),
        [flag] if flag == "--extensions" => print_extensions(),
        _ => {
            eprintln!("usage: abi_layout_probe [--extensions]");
            std::process::exit(2);
        }
    }
}
