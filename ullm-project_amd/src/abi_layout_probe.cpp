// ABI layout probe: prints constants and struct layouts (size, alignment,
// field offsets in declaration order) of the public headers.
//
// Without arguments it prints exactly the lines of the reference's probe
// (native/hip/src/abi_layout_probe.cpp, hip.h only), which
// crates/ullm-hip-sys/build.rs:330-408 compares with the same figures printed
// from the checked-in Rust bindings; build.rs runs it that way.  With
// `--extensions` it prints the same kind of lines for linear.h and
// weights_io.h, for the comparison with the Rust probe of the extension
// bindings (crates/ullm-hip-sys/src/abi_layout_probe.rs).
// Host-only: it includes the headers, not the HIP runtime.
#include "ullm/linear.h"
#include "ullm/weights_io.h"

#include <cstddef>
#include <cstring>
#include <iostream>

#define ULLM_PRINT_CONSTANT(name) std::cout << "const " #name "=" << (name) << '\n'

#define ULLM_LAYOUT_BEGIN(type)                                                \
  {                                                                            \
    using probe_t = type;                                                      \
    std::cout << "layout " #type " size=" << sizeof(probe_t)                   \
              << " align=" << alignof(probe_t);
#define ULLM_FIELD(field) std::cout << " " #field "=" << offsetof(probe_t, field);
#define ULLM_LAYOUT_END                                                        \
  std::cout << '\n';                                                           \
  }

static void print_v1() {
  // hip.h (the reference probe's lines, in its order)
  ULLM_PRINT_CONSTANT(ULLM_HIP_ABI_VERSION);
  ULLM_PRINT_CONSTANT(ULLM_HIP_LIBRARY_VERSION_MAJOR);
  ULLM_PRINT_CONSTANT(ULLM_HIP_LIBRARY_VERSION_MINOR);
  ULLM_PRINT_CONSTANT(ULLM_HIP_LIBRARY_VERSION_PATCH);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_OK);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_INVALID_ARGUMENT);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_BUFFER_TOO_SMALL);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_UNSUPPORTED);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_UNAVAILABLE);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_INVALID_ABI_VERSION);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_RESERVED_NONZERO);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_INTERNAL_ERROR);
  ULLM_PRINT_CONSTANT(ULLM_BACKEND_HIP);
  ULLM_PRINT_CONSTANT(ULLM_ACCESS_READ);
  ULLM_PRINT_CONSTANT(ULLM_ACCESS_WRITE);
  ULLM_PRINT_CONSTANT(ULLM_ACCESS_READ_WRITE);

  ULLM_LAYOUT_BEGIN(ullm_error_sink_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(message)
  ULLM_FIELD(message_capacity) ULLM_FIELD(message_length) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_version_info_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(major)
  ULLM_FIELD(minor) ULLM_FIELD(patch) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_backend_probe_result_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(backend)
  ULLM_FIELD(available) ULLM_FIELD(hip_runtime_present) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_context_probe_result_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(context_present)
  ULLM_FIELD(hip_available) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
}

static void print_extensions() {
  // linear.h
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_TIMEOUT);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_INVALID_HANDLE);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_ZERO_DISPATCH);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_RUNTIME_ERROR);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_HIP_DISPATCH_CONTRACT);
  ULLM_PRINT_CONSTANT(ULLM_STATUS_OUT_OF_MEMORY);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_ENCODING_FP8_E4M3_ROW);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_ENCODING_AQ4_G128);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_LAYOUT_PLAIN);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_LAYOUT_GATED_PAIRS);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_EPILOGUE_NONE);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_EPILOGUE_SILU_MUL);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_SOURCE_F32);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_SOURCE_ENCODED);
  ULLM_PRINT_CONSTANT(ULLM_MEMORY_HOST);
  ULLM_PRINT_CONSTANT(ULLM_MEMORY_DEVICE);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_DTYPE_BF16);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_DTYPE_F32);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_DTYPE_F8E4M3FN);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_ACT_EXACT);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_ACT_FP8_PER_TOKEN);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_KERNEL_GEMV);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_KERNEL_GEMM_DIRECT);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_KERNEL_GEMM_LDS);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_GEMV_SINGLE);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_GEMV_SINGLE_LDS);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_GEMV_MULTI_STRIPE);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_GEMV_REGISTER_STAGED);
  ULLM_PRINT_CONSTANT(ULLM_LINEAR_GEMV_SPLIT_K);

  ULLM_LAYOUT_BEGIN(ullm_linear_weight_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(encoding)
  ULLM_FIELD(source) ULLM_FIELD(n) ULLM_FIELD(k) ULLM_FIELD(memory)
  ULLM_FIELD(device) ULLM_FIELD(values) ULLM_FIELD(scales) ULLM_FIELD(zeros)
  ULLM_FIELD(stream) ULLM_FIELD(layout) ULLM_FIELD(reserved0)
  ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_weight_info_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(encoding)
  ULLM_FIELD(device) ULLM_FIELD(n) ULLM_FIELD(k) ULLM_FIELD(device_bytes)
  ULLM_FIELD(layout) ULLM_FIELD(reserved0) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_forward_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(weight)
  ULLM_FIELD(m) ULLM_FIELD(x) ULLM_FIELD(x_row_stride) ULLM_FIELD(x_scales)
  ULLM_FIELD(y) ULLM_FIELD(y_row_stride) ULLM_FIELD(x_dtype)
  ULLM_FIELD(y_dtype) ULLM_FIELD(activation_mode) ULLM_FIELD(alpha)
  ULLM_FIELD(stream) ULLM_FIELD(workspace) ULLM_FIELD(workspace_size)
  ULLM_FIELD(epilogue) ULLM_FIELD(residual_dtype) ULLM_FIELD(residual)
  ULLM_FIELD(residual_row_stride) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_act_quant_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(m) ULLM_FIELD(k)
  ULLM_FIELD(x) ULLM_FIELD(x_row_stride) ULLM_FIELD(xq) ULLM_FIELD(x_scales)
  ULLM_FIELD(stream) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_add_act_quant_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(m) ULLM_FIELD(k)
  ULLM_FIELD(a) ULLM_FIELD(a_row_stride) ULLM_FIELD(b) ULLM_FIELD(b_row_stride)
  ULLM_FIELD(sum) ULLM_FIELD(sum_row_stride) ULLM_FIELD(xq)
  ULLM_FIELD(x_scales) ULLM_FIELD(stream) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_weight_export_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(memory)
  ULLM_FIELD(reserved0) ULLM_FIELD(values) ULLM_FIELD(scales)
  ULLM_FIELD(zeros) ULLM_FIELD(stream) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_plan_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(kernel)
  ULLM_FIELD(block_m) ULLM_FIELD(block_n) ULLM_FIELD(tiles) ULLM_FIELD(grid)
  ULLM_FIELD(split_k) ULLM_FIELD(gemv_variant) ULLM_FIELD(gemv_waves)
  ULLM_FIELD(gemv_stripes) ULLM_FIELD(gemv_row_classes) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END

  // weights_io.h
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_BOOL);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_U8);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_I8);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_F8_E4M3);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_F8_E5M2);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_U16);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_I16);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_F16);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_BF16);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_U32);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_I32);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_F32);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_U64);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_I64);
  ULLM_PRINT_CONSTANT(ULLM_ST_DTYPE_F64);
  ULLM_PRINT_CONSTANT(ULLM_ST_MAX_RANK);

  ULLM_LAYOUT_BEGIN(ullm_safetensors_open_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(path)
  ULLM_FIELD(expected_sha256) ULLM_FIELD(expected_size) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_safetensors_tensor_info_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(dtype)
  ULLM_FIELD(rank) ULLM_FIELD(shape) ULLM_FIELD(offset) ULLM_FIELD(bytes)
  ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_weight_load_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(file)
  ULLM_FIELD(encoding) ULLM_FIELD(layout) ULLM_FIELD(values)
  ULLM_FIELD(value_parts) ULLM_FIELD(device) ULLM_FIELD(scales)
  ULLM_FIELD(zeros) ULLM_FIELD(stream) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
  ULLM_LAYOUT_BEGIN(ullm_linear_weights_save_desc_t)
  ULLM_FIELD(struct_size) ULLM_FIELD(abi_version) ULLM_FIELD(path)
  ULLM_FIELD(names) ULLM_FIELD(weights) ULLM_FIELD(count)
  ULLM_FIELD(metadata_keys) ULLM_FIELD(metadata_values)
  ULLM_FIELD(metadata_count) ULLM_FIELD(reserved)
  ULLM_LAYOUT_END
}

int main(int argc, char **argv) {
  if (argc == 1) {
    print_v1();
    return 0;
  }
  if (argc == 2 && std::strcmp(argv[1], "--extensions") == 0) {
    print_extensions();
    return 0;
  }
  std::cerr << "usage: abi_layout_probe [--extensions]\n";
  return 2;
}
