//! Weight encodings of the gfx950 quantized linear layer, for
//! crates/ullm-core.  Not compiled in this build's container (no Rust
//! toolchain); the byte counts below are the ones tests/test_gpu_linear.py and
//! bench.py use (FP8: N*K + 4N; AQ4: N*K/2 + 4*N*K/128).
//!
//! Wiring, as rust/patches/ullm-core.patch applies it (reference
//! crates/ullm-core/src/dtype.rs:55-122, op.rs:97-113):
//!
//! 1. `mod quant; pub use quant::*;` in crates/ullm-core/src/lib.rs.
//! 2. Two `Encoding` variants next to `Nvfp4`:
//!    `Fp8RowScaled { row_len: usize, scale_dtype: DType }` and
//!    `Aq4 { group_size: usize, scale_dtype: DType, zero_dtype: DType }`.
//!    `row_len` is K, so that `storage_bytes(dtype, elements)` can count the
//!    per-row scales from the element count alone.
//! 3. Their arms in `offset_alignment` (1: packed bytes), `validate`
//!    (`validate_fp8_row_scaled` / `validate_aq4` below) and `storage_bytes`
//!    (`fp8_row_scaled_bytes` / `aq4_bytes` below).
//! 4. In `SemanticOpDescriptor::validate`'s Matmul arm, accept
//!    `is_quantized_matmul(left, right, output)` besides the existing
//!    same-dtype rule.

use crate::{DType, Encoding, EncodingError, TensorView};

/// Group size of the AQ4 encoding: one scale and zero per 128 k.
pub const AQ4_GROUP: usize = 128;

/// FP8 row-scaled storage: u8 E4M3FN codes, one f32 scale per row of
/// `row_len` codes.
pub fn validate_fp8_row_scaled(
    dtype: DType,
    row_len: usize,
    scale_dtype: DType,
) -> Result<(), EncodingError> {
    if row_len == 0 {
        return Err(EncodingError::ZeroBlockSize);
    }
    if dtype != DType::F8E4M3Fn {
        return Err(EncodingError::PackedStorageMustBeU8 { dtype });
    }
    if scale_dtype != DType::F32 {
        return Err(EncodingError::InvalidScaleDType { dtype: scale_dtype });
    }
    Ok(())
}

/// AQ4 storage: u8 bytes of packed nibbles (eight per u32 word, low nibble
/// first), an f16 scale and an f16 zero per group of 128 along each row.
pub fn validate_aq4(
    dtype: DType,
    group_size: usize,
    scale_dtype: DType,
    zero_dtype: DType,
) -> Result<(), EncodingError> {
    if group_size != AQ4_GROUP {
        return Err(EncodingError::ZeroBlockSize);
    }
    if dtype != DType::U8 {
        return Err(EncodingError::PackedStorageMustBeU8 { dtype });
    }
    if scale_dtype != DType::F16 {
        return Err(EncodingError::InvalidScaleDType { dtype: scale_dtype });
    }
    if zero_dtype != DType::F16 {
        return Err(EncodingError::InvalidScaleDType { dtype: zero_dtype });
    }
    Ok(())
}

/// Bytes of `elements` FP8 codes plus one f32 scale per row of `row_len`.
pub fn fp8_row_scaled_bytes(elements: u64, row_len: usize) -> Result<u64, EncodingError> {
    let row_len = u64::try_from(row_len).map_err(|_| EncodingError::SizeOverflow)?;
    if row_len == 0 {
        return Err(EncodingError::ZeroBlockSize);
    }
    let rows = elements / row_len + u64::from(elements % row_len != 0);
    rows.checked_mul(4)
        .and_then(|scales| scales.checked_add(elements))
        .ok_or(EncodingError::SizeOverflow)
}

/// Bytes of `elements` AQ4 codes: half a byte each (whole u32 words), and
/// 4 bytes (f16 scale + f16 zero) per group of 128.
pub fn aq4_bytes(elements: u64) -> Result<u64, EncodingError> {
    let group = AQ4_GROUP as u64;
    let words = elements / 8 + u64::from(elements % 8 != 0);
    let groups = elements / group + u64::from(elements % group != 0);
    let packed = words.checked_mul(4).ok_or(EncodingError::SizeOverflow)?;
    groups
        .checked_mul(4)
        .and_then(|sz| sz.checked_add(packed))
        .ok_or(EncodingError::SizeOverflow)
}

/// Whether `encoding` is one the quantized linear layer executes.
pub fn is_linear_weight_encoding(encoding: Encoding) -> bool {
    matches!(
        encoding,
        Encoding::Fp8RowScaled { .. } | Encoding::Aq4 { .. }
    )
}

/// A Matmul the quantized linear layer accepts: bf16 activations
/// `left` [M, K] (unquantized), a weight `right` of logical shape [K, N]
/// in an FP8 row-scaled or AQ4 encoding (stored one row of K per output
/// feature, with `row_len == K`), and a bf16 or f32 `output` [M, N].
pub fn is_quantized_matmul(left: &TensorView, right: &TensorView, output: &TensorView) -> bool {
    let (l, r, o) = (left.shape(), right.shape(), output.shape());
    if l.len() != 2 || r.len() != 2 || o.len() != 2 || l[1] != r[0] || o != [l[0], r[1]] {
        return false;
    }
    if left.dtype() != DType::Bf16 || left.encoding() != Encoding::Unquantized {
        return false;
    }
    if !matches!(output.dtype(), DType::Bf16 | DType::F32)
        || output.encoding() != Encoding::Unquantized
    {
        return false;
    }
    match right.encoding() {
        Encoding::Fp8RowScaled { row_len, .. } => row_len == r[0],
        Encoding::Aq4 { .. } => r[0] % AQ4_GROUP == 0,
        _ => false,
    }
}
