//! Rust bindings to `libmlxq.so` (`include/mlxq.h`): the MI355X quantized
//! matmul library that stands in for MLX's `quantized_matmul`, `gather_qmm`,
//! `dequantize`, `quantize`, `quantized_linear_forward` and the fused decode
//! MoE kernels behind mlxcel's `cxx` bridge.
//!
//! `sys` holds the raw `extern "C"` declarations, one per symbol of the
//! header.  The safe layer mirrors the reference's bridge functions
//! (`src/lib/mlxcel-core/src/lib.rs:1374-1416` `gather_qmm` /
//! `quantized_matmul` / `dequantize`, `:697-707` `quantized_linear_forward`,
//! `:2336-2380` `fused_moe_expert_kernel` / `fused_moe_geglu_kernel`,
//! `:2666` `clear_memory_cache`, `:2720` `get_cache_memory`, `:2925-2940`
//! `quantized_matmul_matches_dense_gemm`): same argument order and meaning,
//! nullable arrays as `Option`, and a `Result` whose error carries the
//! library's status and message (the reference's `std::invalid_argument`
//! text for argument errors).  The library is eager: callers pass device
//! views of already-allocated arrays and a HIP stream; the output shape and
//! dtype come from the `*_shape` queries.

#![allow(clippy::too_many_arguments)]

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::c_void;

/// Raw declarations of `include/mlxq.h`.
pub mod sys {
    #![allow(non_camel_case_types)]
    use std::os::raw::{c_char, c_void};

    pub const MLXQ_MAX_DIMS: usize = 8;

    pub const MLXQ_OK: i32 = 0;
    pub const MLXQ_EINVAL: i32 = 1;
    pub const MLXQ_EUNSUPPORTED: i32 = 2;
    pub const MLXQ_EHIP: i32 = 3;
    pub const MLXQ_ENOMEM: i32 = 4;

    /// A strided view of device memory (strides in elements).
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct mlxq_array {
        pub data: *mut c_void,
        pub dtype: i32,
        pub ndim: i32,
        pub shape: [i64; MLXQ_MAX_DIMS],
        pub strides: [i64; MLXQ_MAX_DIMS],
    }

    extern "C" {
        pub fn mlxq_last_error() -> *const c_char;
        pub fn mlxq_version() -> *const c_char;
        pub fn mlxq_workspace_reserve(bytes: usize, stream: *mut c_void) -> i32;
        pub fn mlxq_get_cache_memory() -> usize;
        pub fn mlxq_clear_cache() -> i32;
        pub fn mlxq_reload_options();

        pub fn mlxq_quantized_matmul(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            transpose: bool, group_size: i32, bits: i32, mode: *const c_char, out: *mut mlxq_array,
            stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_quantized_matmul_noalloc(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            transpose: bool, group_size: i32, bits: i32, mode: *const c_char, out: *mut mlxq_array,
            stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_quantized_linear(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            linear_bias: *const mlxq_array, group_size: i32, bits: i32, mode: *const c_char,
            out: *mut mlxq_array, stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_quantized_matmul_matches_dense_gemm(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            group_size: i32, bits: i32,
        ) -> i32;
        pub fn mlxq_quantized_matmul_multi(
            x: *const mlxq_array, n: i32, w: *const *const mlxq_array, scales: *const *const mlxq_array,
            biases: *const *const mlxq_array, group_size: i32, bits: i32, mode: *const c_char,
            out: *const *mut mlxq_array, stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_quantized_matmul_shape(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            transpose: bool, group_size: i32, bits: i32, mode: *const c_char, out_ndim: *mut i32,
            out_shape: *mut i64, out_dtype: *mut i32,
        ) -> i32;
        pub fn mlxq_gather_qmm(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            lhs_indices: *const mlxq_array, rhs_indices: *const mlxq_array, transpose: bool, group_size: i32,
            bits: i32, sorted_indices: bool, mode: *const c_char, global_scale: *const mlxq_array,
            out: *mut mlxq_array, stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_gather_qmm_shape(
            x: *const mlxq_array, w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array,
            lhs_indices: *const mlxq_array, rhs_indices: *const mlxq_array, transpose: bool, group_size: i32,
            bits: i32, mode: *const c_char, out_ndim: *mut i32, out_shape: *mut i64, out_dtype: *mut i32,
        ) -> i32;
        pub fn mlxq_dequantize(
            w: *const mlxq_array, scales: *const mlxq_array, biases: *const mlxq_array, group_size: i32,
            bits: i32, mode: *const c_char, dtype: i32, out: *mut mlxq_array, stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_quantize(
            w: *const mlxq_array, group_size: i32, bits: i32, mode: *const c_char, wq_out: *mut mlxq_array,
            scales_out: *mut mlxq_array, biases_out: *mut mlxq_array, stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_fused_moe_expert(
            x: *const mlxq_array, indices: *const mlxq_array, gate_w: *const mlxq_array,
            gate_s: *const mlxq_array, gate_b: *const mlxq_array, up_w: *const mlxq_array,
            up_s: *const mlxq_array, up_b: *const mlxq_array, down_w: *const mlxq_array,
            down_s: *const mlxq_array, down_b: *const mlxq_array, scores: *const mlxq_array, din: i32,
            dff: i32, k: i32, gu_bits: i32, d_bits: i32, group_size: i32, out: *mut mlxq_array,
            stream: *mut c_void,
        ) -> i32;
        pub fn mlxq_fused_moe_geglu(
            x: *const mlxq_array, indices: *const mlxq_array, gate_w: *const mlxq_array,
            gate_s: *const mlxq_array, gate_b: *const mlxq_array, up_w: *const mlxq_array,
            up_s: *const mlxq_array, up_b: *const mlxq_array, down_w: *const mlxq_array,
            down_s: *const mlxq_array, down_b: *const mlxq_array, scores: *const mlxq_array, din: i32,
            dff: i32, k: i32, gu_bits: i32, d_bits: i32, group_size: i32, out: *mut mlxq_array,
            stream: *mut c_void,
        ) -> i32;
    }
}

pub use sys::MLXQ_MAX_DIMS;

/// Element types, numbered as `mlx::core::Dtype::Val` (`include/mlxq.h`).
#[repr(i32)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Dtype {
    Bool = 0,
    Uint8 = 1,
    Uint16 = 2,
    Uint32 = 3,
    Uint64 = 4,
    Int8 = 5,
    Int16 = 6,
    Int32 = 7,
    Int64 = 8,
    Float16 = 9,
    Float32 = 10,
    Float64 = 11,
    Bfloat16 = 12,
    Complex64 = 13,
}

impl Dtype {
    pub fn from_code(code: i32) -> Option<Dtype> {
        use Dtype::*;
        Some(match code {
            0 => Bool,
            1 => Uint8,
            2 => Uint16,
            3 => Uint32,
            4 => Uint64,
            5 => Int8,
            6 => Int16,
            7 => Int32,
            8 => Int64,
            9 => Float16,
            10 => Float32,
            11 => Float64,
            12 => Bfloat16,
            13 => Complex64,
            _ => return None,
        })
    }
}

/// What a failing call returned.  `Invalid` carries the reference's
/// exception text (rethrow it as MLX would); `Unsupported` means "fall back
/// to MLX"; `Hip` and `NoMem` are execution failures.
#[derive(Clone, Debug, PartialEq, Eq)]
pub enum Error {
    Invalid(String),
    Unsupported(String),
    Hip(String),
    NoMem(String),
    Other(i32, String),
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            Error::Invalid(m) | Error::Unsupported(m) | Error::Hip(m) | Error::NoMem(m) => f.write_str(m),
            Error::Other(code, m) => write!(f, "mlxq status {code}: {m}"),
        }
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

fn last_error() -> String {
    // SAFETY: the library returns a NUL-terminated, thread-local string.
    unsafe {
        let p = sys::mlxq_last_error();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// Maps a status code to `Ok(())` or the error with the thread's message.
pub fn check(status: i32) -> Result<()> {
    match status {
        sys::MLXQ_OK => Ok(()),
        sys::MLXQ_EINVAL => Err(Error::Invalid(last_error())),
        sys::MLXQ_EUNSUPPORTED => Err(Error::Unsupported(last_error())),
        sys::MLXQ_EHIP => Err(Error::Hip(last_error())),
        sys::MLXQ_ENOMEM => Err(Error::NoMem(last_error())),
        code => Err(Error::Other(code, last_error())),
    }
}

/// A strided view of device memory: what mlxcel's bridge builds from an
/// evaluated `mlx::core::array` (its data pointer, dtype, shape and strides
/// in elements).
#[derive(Clone, Copy, Debug)]
pub struct ArrayView {
    raw: sys::mlxq_array,
}

impl ArrayView {
    /// Row-contiguous view of `shape`.
    ///
    /// # Safety
    /// `data` must be a device pointer of the current HIP device holding the
    /// whole view, alive until the stream has run the calls that use it.
    pub unsafe fn contiguous(data: *mut c_void, dtype: Dtype, shape: &[i64]) -> ArrayView {
        let mut strides = vec![0i64; shape.len()];
        let mut st = 1i64;
        for i in (0..shape.len()).rev() {
            strides[i] = st;
            st *= shape[i];
        }
        ArrayView::strided(data, dtype, shape, &strides)
    }

    /// View with explicit strides (in elements).
    ///
    /// # Safety
    /// As `contiguous`; every element the strides reach must lie inside the
    /// allocation.
    pub unsafe fn strided(data: *mut c_void, dtype: Dtype, shape: &[i64], strides: &[i64]) -> ArrayView {
        assert!(shape.len() <= MLXQ_MAX_DIMS && strides.len() == shape.len(), "at most 8 dimensions");
        let mut raw = sys::mlxq_array {
            data,
            dtype: dtype as i32,
            ndim: shape.len() as i32,
            shape: [0; MLXQ_MAX_DIMS],
            strides: [0; MLXQ_MAX_DIMS],
        };
        raw.shape[..shape.len()].copy_from_slice(shape);
        raw.strides[..strides.len()].copy_from_slice(strides);
        ArrayView { raw }
    }

    pub fn shape(&self) -> &[i64] {
        &self.raw.shape[..self.raw.ndim as usize]
    }

    pub fn dtype(&self) -> Option<Dtype> {
        Dtype::from_code(self.raw.dtype)
    }

    pub fn as_raw(&self) -> *const sys::mlxq_array {
        &self.raw
    }

    fn as_raw_mut(&mut self) -> *mut sys::mlxq_array {
        &mut self.raw
    }
}

fn opt(a: Option<&ArrayView>) -> *const sys::mlxq_array {
    a.map_or(std::ptr::null(), |v| v.as_raw())
}

fn cmode(mode: &str) -> CString {
    // a mode with an interior NUL cannot name a valid mode; the library
    // rejects the empty string with the reference's message
    CString::new(mode).unwrap_or_default()
}

/// Output shape and dtype of a call, from a `*_shape` query.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct OutSpec {
    pub shape: Vec<i64>,
    pub dtype: Dtype,
}

fn out_spec(ndim: i32, shape: &[i64; MLXQ_MAX_DIMS], dtype: i32) -> Result<OutSpec> {
    let dtype = Dtype::from_code(dtype).ok_or_else(|| Error::Other(-1, format!("unknown dtype code {dtype}")))?;
    Ok(OutSpec { shape: shape[..ndim as usize].to_vec(), dtype })
}

/// The library's version string.
pub fn version() -> String {
    // SAFETY: a static NUL-terminated string.
    unsafe { CStr::from_ptr(sys::mlxq_version()).to_string_lossy().into_owned() }
}

/// Shape and dtype `quantized_matmul` would produce (the reference's
/// validation and messages, no device work).
pub fn quantized_matmul_shape(
    x: &ArrayView, w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>, transpose: bool,
    group_size: i32, bits: i32, mode: &str,
) -> Result<OutSpec> {
    let m = cmode(mode);
    let (mut nd, mut sh, mut dt) = (0i32, [0i64; MLXQ_MAX_DIMS], 0i32);
    // SAFETY: the views are plain structs; no device memory is touched.
    check(unsafe {
        sys::mlxq_quantized_matmul_shape(
            x.as_raw(), w.as_raw(), scales.as_raw(), opt(biases), transpose, group_size, bits, m.as_ptr(),
            &mut nd, sh.as_mut_ptr(), &mut dt,
        )
    })?;
    out_spec(nd, &sh, dt)
}

/// `y = x @ dequantize(w, scales, biases)^T` (transpose) or without the
/// transpose, as the reference's `ffi::quantized_matmul`, into `out`.
///
/// # Safety
/// Every view must describe live device memory of the current device;
/// `stream` is a `hipStream_t` (null: the default stream).
pub unsafe fn quantized_matmul(
    x: &ArrayView, w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>, transpose: bool,
    group_size: i32, bits: i32, mode: &str, out: &mut ArrayView, stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    check(sys::mlxq_quantized_matmul(
        x.as_raw(), w.as_raw(), scales.as_raw(), opt(biases), transpose, group_size, bits, m.as_ptr(),
        out.as_raw_mut(), stream,
    ))
}

/// `quantized_matmul` with its scratch in the library's fixed per-GPU array:
/// for callers that cannot allocate (HIP-graph capture, serving loops).
/// Calls that overlap on one GPU race on that array.
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn quantized_matmul_noalloc(
    x: &ArrayView, w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>, transpose: bool,
    group_size: i32, bits: i32, mode: &str, out: &mut ArrayView, stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    check(sys::mlxq_quantized_matmul_noalloc(
        x.as_raw(), w.as_raw(), scales.as_raw(), opt(biases), transpose, group_size, bits, m.as_ptr(),
        out.as_raw_mut(), stream,
    ))
}

/// The reference's `quantized_linear_forward`: `x @ W^T + linear_bias`.
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn quantized_linear_forward(
    x: &ArrayView, weight: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>,
    linear_bias: Option<&ArrayView>, group_size: i32, bits: i32, mode: &str, out: &mut ArrayView,
    stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    check(sys::mlxq_quantized_linear(
        x.as_raw(), weight.as_raw(), scales.as_raw(), opt(biases), opt(linear_bias), group_size, bits,
        m.as_ptr(), out.as_raw_mut(), stream,
    ))
}

/// The reference's `quantized_matmul_matches_dense_gemm`: false here for
/// every input (no call returns the bytes of dequantize + a dense GEMM).
pub fn quantized_matmul_matches_dense_gemm(
    x: &ArrayView, weight: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>, group_size: i32,
    bits: i32,
) -> bool {
    // SAFETY: host-only predicate.
    unsafe {
        sys::mlxq_quantized_matmul_matches_dense_gemm(
            x.as_raw(), weight.as_raw(), scales.as_raw(), opt(biases), group_size, bits,
        ) != 0
    }
}

/// Several projections of one activation (q/k/v, gate/up): bit for bit the
/// separate `quantized_matmul` calls, one launch at decode row counts.
///
/// # Safety
/// As `quantized_matmul`; the slices have equal lengths (1 to 4).
pub unsafe fn quantized_matmul_multi(
    x: &ArrayView, w: &[&ArrayView], scales: &[&ArrayView], biases: Option<&[&ArrayView]>, group_size: i32,
    bits: i32, mode: &str, out: &mut [&mut ArrayView], stream: *mut c_void,
) -> Result<()> {
    let n = w.len();
    assert!(scales.len() == n && out.len() == n && biases.map_or(true, |b| b.len() == n));
    let m = cmode(mode);
    let wp: Vec<*const sys::mlxq_array> = w.iter().map(|v| v.as_raw()).collect();
    let sp: Vec<*const sys::mlxq_array> = scales.iter().map(|v| v.as_raw()).collect();
    let bp: Option<Vec<*const sys::mlxq_array>> = biases.map(|b| b.iter().map(|v| v.as_raw()).collect());
    let op: Vec<*mut sys::mlxq_array> = out.iter_mut().map(|v| v.as_raw_mut()).collect();
    check(sys::mlxq_quantized_matmul_multi(
        x.as_raw(), n as i32, wp.as_ptr(), sp.as_ptr(), bp.as_ref().map_or(std::ptr::null(), |b| b.as_ptr()),
        group_size, bits, m.as_ptr(), op.as_ptr(), stream,
    ))
}

/// Shape and dtype `gather_qmm` would produce.
pub fn gather_qmm_shape(
    x: &ArrayView, w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>,
    lhs_indices: Option<&ArrayView>, rhs_indices: Option<&ArrayView>, transpose: bool, group_size: i32,
    bits: i32, mode: &str,
) -> Result<OutSpec> {
    let m = cmode(mode);
    let (mut nd, mut sh, mut dt) = (0i32, [0i64; MLXQ_MAX_DIMS], 0i32);
    // SAFETY: host-only query.
    check(unsafe {
        sys::mlxq_gather_qmm_shape(
            x.as_raw(), w.as_raw(), scales.as_raw(), opt(biases), opt(lhs_indices), opt(rhs_indices), transpose,
            group_size, bits, m.as_ptr(), &mut nd, sh.as_mut_ptr(), &mut dt,
        )
    })?;
    out_spec(nd, &sh, dt)
}

/// The reference's `ffi::gather_qmm`, into `out`.
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn gather_qmm(
    x: &ArrayView, w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>,
    lhs_indices: Option<&ArrayView>, rhs_indices: Option<&ArrayView>, transpose: bool, group_size: i32,
    bits: i32, sorted_indices: bool, mode: &str, global_scale: Option<&ArrayView>, out: &mut ArrayView,
    stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    check(sys::mlxq_gather_qmm(
        x.as_raw(), w.as_raw(), scales.as_raw(), opt(biases), opt(lhs_indices), opt(rhs_indices), transpose,
        group_size, bits, sorted_indices, m.as_ptr(), opt(global_scale), out.as_raw_mut(), stream,
    ))
}

/// The reference's `ffi::dequantize` (`dtype`: None = the reference
/// default), into `out`.
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn dequantize(
    w: &ArrayView, scales: &ArrayView, biases: Option<&ArrayView>, group_size: i32, bits: i32, mode: &str,
    dtype: Option<Dtype>, out: &mut ArrayView, stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    check(sys::mlxq_dequantize(
        w.as_raw(), scales.as_raw(), opt(biases), group_size, bits, m.as_ptr(), dtype.map_or(-1, |d| d as i32),
        out.as_raw_mut(), stream,
    ))
}

/// `mlx::core::quantize` into caller-allocated outputs (`biases_out` for
/// affine only).
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn quantize(
    w: &ArrayView, group_size: i32, bits: i32, mode: &str, wq_out: &mut ArrayView, scales_out: &mut ArrayView,
    biases_out: Option<&mut ArrayView>, stream: *mut c_void,
) -> Result<()> {
    let m = cmode(mode);
    let b = biases_out.map_or(std::ptr::null_mut(), |v| v.as_raw_mut());
    check(sys::mlxq_quantize(
        w.as_raw(), group_size, bits, m.as_ptr(), wq_out.as_raw_mut(), scales_out.as_raw_mut(), b, stream,
    ))
}

/// The twelve arrays of one fused decode-MoE call, in the reference's order.
pub struct MoeArrays<'a> {
    pub x: &'a ArrayView,
    pub indices: &'a ArrayView,
    pub gate_w: &'a ArrayView,
    pub gate_s: &'a ArrayView,
    pub gate_b: &'a ArrayView,
    pub up_w: &'a ArrayView,
    pub up_s: &'a ArrayView,
    pub up_b: &'a ArrayView,
    pub down_w: &'a ArrayView,
    pub down_s: &'a ArrayView,
    pub down_b: &'a ArrayView,
    pub scores: &'a ArrayView,
}

/// The reference's `fused_moe_expert_kernel` (SwiGLU experts).  `Err(
/// Unsupported)` for configurations without a kernel: the caller takes its
/// `gather_qmm` route, as it does for the reference's `Err`.
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn fused_moe_expert_kernel(
    a: &MoeArrays, din: i32, dff: i32, k: i32, gu_bits: i32, d_bits: i32, group_size: i32, out: &mut ArrayView,
    stream: *mut c_void,
) -> Result<()> {
    check(sys::mlxq_fused_moe_expert(
        a.x.as_raw(), a.indices.as_raw(), a.gate_w.as_raw(), a.gate_s.as_raw(), a.gate_b.as_raw(),
        a.up_w.as_raw(), a.up_s.as_raw(), a.up_b.as_raw(), a.down_w.as_raw(), a.down_s.as_raw(),
        a.down_b.as_raw(), a.scores.as_raw(), din, dff, k, gu_bits, d_bits, group_size, out.as_raw_mut(), stream,
    ))
}

/// The reference's `fused_moe_geglu_kernel` (GeGLU experts).
///
/// # Safety
/// As `quantized_matmul`.
pub unsafe fn fused_moe_geglu_kernel(
    a: &MoeArrays, din: i32, dff: i32, k: i32, gu_bits: i32, d_bits: i32, group_size: i32, out: &mut ArrayView,
    stream: *mut c_void,
) -> Result<()> {
    check(sys::mlxq_fused_moe_geglu(
        a.x.as_raw(), a.indices.as_raw(), a.gate_w.as_raw(), a.gate_s.as_raw(), a.gate_b.as_raw(),
        a.up_w.as_raw(), a.up_s.as_raw(), a.up_b.as_raw(), a.down_w.as_raw(), a.down_s.as_raw(),
        a.down_b.as_raw(), a.scores.as_raw(), din, dff, k, gu_bits, d_bits, group_size, out.as_raw_mut(), stream,
    ))
}

/// Grows `stream`'s workspace (so later calls, e.g. under graph capture,
/// need not allocate).
pub fn workspace_reserve(bytes: usize, stream: *mut c_void) -> Result<()> {
    // SAFETY: allocates on the current device; `stream` is a hipStream_t.
    check(unsafe { sys::mlxq_workspace_reserve(bytes, stream) })
}

/// The reference's `get_cache_memory`: bytes the library's workspaces hold.
pub fn get_cache_memory() -> usize {
    // SAFETY: reads the library's bookkeeping only.
    unsafe { sys::mlxq_get_cache_memory() }
}

/// The reference's `clear_memory_cache`: synchronizes and frees every
/// workspace (graphs captured earlier must not be replayed afterwards).
pub fn clear_memory_cache() -> Result<()> {
    // SAFETY: synchronizes the devices that hold a workspace first.
    check(unsafe { sys::mlxq_clear_cache() })
}

/// Re-reads the `MLXQ_*` environment switches (A/B measurement only).
pub fn reload_options() {
    // SAFETY: swaps an immutable snapshot.
    unsafe { sys::mlxq_reload_options() }
}

#[cfg(test)]
mod tests {
    use super::*;

    fn view(dtype: Dtype, shape: &[i64]) -> ArrayView {
        // shape queries never dereference the data pointer
        unsafe { ArrayView::contiguous(std::ptr::null_mut(), dtype, shape) }
    }

    #[test]
    fn version_names_the_target() {
        assert!(version().contains("gfx950"));
    }

    #[test]
    fn shape_query_follows_the_reference() {
        let x = view(Dtype::Bfloat16, &[3, 4096]);
        let w = view(Dtype::Uint32, &[14336, 512]);
        let s = view(Dtype::Bfloat16, &[14336, 64]);
        let spec = quantized_matmul_shape(&x, &w, &s, Some(&s), true, 64, 4, "affine").unwrap();
        assert_eq!(spec, OutSpec { shape: vec![3, 14336], dtype: Dtype::Bfloat16 });
    }

    #[test]
    fn argument_errors_carry_the_reference_text() {
        let x = view(Dtype::Bfloat16, &[3, 4096]);
        let w = view(Dtype::Uint32, &[14336, 512]);
        let s = view(Dtype::Bfloat16, &[14336, 64]);
        match quantized_matmul_shape(&x, &w, &s, None, true, 64, 4, "affine") {
            Err(Error::Invalid(m)) => assert!(m.contains("Biases must be provided")),
            other => panic!("{other:?}"),
        }
    }

    #[test]
    fn strides_default_to_row_major() {
        let v = view(Dtype::Float16, &[2, 3, 4]);
        assert_eq!(v.raw.strides[..3], [12, 4, 1]);
        assert_eq!(v.shape(), &[2, 3, 4]);
        assert_eq!(v.dtype(), Some(Dtype::Float16));
    }
}
