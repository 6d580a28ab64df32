//! gfx950 weight-only quantized GEMM for `crates/nebula-hydrogen` (Linux / ROCm): the Rust
//! host side over libnebula_hq.so's C ABI (include/hq_qgemm.h), replacing
//! hydrogen::MarlinGemmEngine (hydrogen/include/marlin_gemm.hpp:59-172) and the weight loading
//! of hydrogen::ModelLoader (hydrogen/include/tensor_loader.hpp:14-53) for this path.
//!
//! Conventions follow the crate (crates/nebula-hydrogen/src/ipc.rs): `#[repr(C)]` mirrors with
//! size asserts, `thiserror` errors, `unsafe` only inside `// SAFETY:` blocks. Every entry
//! point of the header is declared below, with the same names, arity and types
//! (tests/test_rust_binding.py checks them against the header). Device pointers and streams
//! (`hipStream_t`) are raw pointers: the crate does not own HIP memory.
#![allow(dead_code)]

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::ptr;

/// hq_status (0 = ok); see [`QgemmError`].
pub type Status = i32;
/// A hipStream_t (null: the null stream).
pub type Stream = *mut c_void;

#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Dtype {
    F16 = 1,
    Bf16 = 2,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Format {
    Int4 = 1,
    Ternary2 = 2,
}

/// hq_segment: one projection of a fused call.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Segment {
    pub wp: *const u32,
    pub scales: *const u16,
    pub bias: *const f32,
    pub y: *mut c_void,
    pub ldy: i64,
    pub n: u32,
}
const _: () = assert!(std::mem::size_of::<Segment>() == 48);

/// hq_gguf: an open GGUF file (opaque).
#[repr(C)]
pub struct Gguf {
    _private: [u8; 0],
}

/// hq_gguf_header_info.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct GgufHeaderInfo {
    pub version: u32,
    pub tensor_count: u64,
    pub kv_count: u64,
    pub alignment: u64,
    pub header_bytes: u64,
    pub tensor_data_offset: u64,
    pub total_tensor_bytes: u64,
    pub file_bytes: u64,
}
const _: () = assert!(std::mem::size_of::<GgufHeaderInfo>() == 64);

/// hq_gguf_tensor_info.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct GgufTensorInfo {
    pub name: *const c_char,
    pub n_dims: u32,
    pub shape: [u64; 4],
    pub r#type: u32,
    pub offset: u64,
    pub absolute_offset: u64,
    pub size_bytes: u64,
    pub data: *const c_void,
}
const _: () = assert!(std::mem::size_of::<GgufTensorInfo>() == 88);

pub const MAX_SEGMENTS: usize = 8;
pub const NOALLOC_SCRATCH_BYTES: usize = 16 << 20;

#[link(name = "nebula_hq")]
extern "C" {
    pub fn hq_version() -> *const c_char;
    pub fn hq_last_error() -> *const c_char;
    pub fn hq_status_string(s: Status) -> *const c_char;
    pub fn hq_linear_words(fmt: Format, k: u32, n: u32) -> usize;
    pub fn hq_packed_words(fmt: Format, k: u32, n: u32) -> usize;
    pub fn hq_workspace_bytes(fmt: Format, m: u32, k: u32, n: u32, group: u32, bytes: *mut usize) -> Status;
    pub fn hq_workspace_bytes_fused(fmt: Format, m: u32, k: u32, group: u32, ns: *const u32, nseg: u32,
                                    with_bias: c_int, bytes: *mut usize) -> Status;
    pub fn hq_describe_gemm(fmt: Format, dtype: Dtype, m: u32, k: u32, n: u32, group: u32, with_bias: c_int,
                            buf: *mut c_char, buf_len: usize) -> Status;
    pub fn hq_device_status(stream: Stream) -> Status;
    pub fn hq_repack_int4_ref(src_linear: *const u32, dst: *mut u32, k: u32, n: u32) -> Status;
    pub fn hq_repack_int4(src_linear: *const u32, dst_packed: *mut u32, k: u32, n: u32) -> Status;
    pub fn hq_repack_ternary2(src_linear: *const u32, dst_packed: *mut u32, k: u32, n: u32) -> Status;
    pub fn hq_unpack_int4(packed: *const u32, dst_linear: *mut u32, k: u32, n: u32) -> Status;
    pub fn hq_unpack_ternary2(packed: *const u32, dst_linear: *mut u32, k: u32, n: u32) -> Status;
    pub fn hq_repack_int4_device(d_src_linear: *const u32, d_dst_packed: *mut u32, k: u32, n: u32,
                                 stream: Stream) -> Status;
    pub fn hq_repack_ternary2_device(d_src_linear: *const u32, d_dst_packed: *mut u32, k: u32, n: u32,
                                     d_bad_flag: *mut u32, stream: Stream) -> Status;
    pub fn hq_tq1_0_bytes(k: u32, n: u32) -> usize;
    pub fn hq_convert_tq1_0(blocks: *const c_void, k: u32, n: u32, codes_linear: *mut u32,
                            scales: *mut u16) -> Status;
    pub fn hq_repack_tq1_0_device(d_blocks: *const c_void, k: u32, n: u32, d_packed: *mut u32,
                                  d_scales: *mut u16, stream: Stream) -> Status;
    pub fn hq_gguf_open(path: *const c_char, out: *mut *mut Gguf) -> Status;
    pub fn hq_gguf_parse(data: *const c_void, bytes: usize, out: *mut *mut Gguf) -> Status;
    pub fn hq_gguf_close(g: *mut Gguf);
    pub fn hq_gguf_header(g: *const Gguf, out: *mut GgufHeaderInfo) -> Status;
    pub fn hq_gguf_tensor_at(g: *const Gguf, index: u64, out: *mut GgufTensorInfo) -> Status;
    pub fn hq_gguf_find_tensor(g: *const Gguf, name: *const c_char, out: *mut GgufTensorInfo) -> Status;
    pub fn hq_gguf_get_int(g: *const Gguf, key: *const c_char, out: *mut i64) -> Status;
    pub fn hq_gguf_get_float(g: *const Gguf, key: *const c_char, out: *mut f64) -> Status;
    pub fn hq_gguf_get_string(g: *const Gguf, key: *const c_char, buf: *mut c_char, buf_len: usize,
                              len: *mut usize) -> Status;
    pub fn hq_gguf_get_array(g: *const Gguf, key: *const c_char, elem_type: *mut u32, count: *mut u64) -> Status;
    pub fn hq_gguf_load_tq1_0(g: *const Gguf, name: *const c_char, d_staging: *mut c_void, staging_bytes: usize,
                              d_packed: *mut u32, d_scales: *mut u16, k: *mut u32, n: *mut u32,
                              stream: Stream) -> Status;
    pub fn hq_convert_q4_k(blocks: *const c_void, k: u32, n: u32, codes_linear: *mut u32, scales: *mut u16,
                           bias: *mut f32) -> Status;
    pub fn hq_gguf_convert_q4_k(g: *const Gguf, name: *const c_char, codes_linear: *mut u32, scales: *mut u16,
                                bias: *mut f32, k: *mut u32, n: *mut u32) -> Status;
    pub fn hq_gemm_w4a16(x: *const c_void, dtype: Dtype, ldx: i64, wp: *const u32, scales: *const u16,
                         bias: *const f32, y: *mut c_void, ldy: i64, m: u32, k: u32, n: u32, group: u32,
                         workspace: *mut c_void, workspace_bytes: usize, stream: Stream) -> Status;
    pub fn hq_gemm_w2a16(x: *const c_void, dtype: Dtype, ldx: i64, wp: *const u32, scales: *const u16,
                         y: *mut c_void, ldy: i64, m: u32, k: u32, n: u32, group: u32, workspace: *mut c_void,
                         workspace_bytes: usize, stream: Stream) -> Status;
    pub fn hq_gemm_fused(x: *const c_void, dtype: Dtype, ldx: i64, fmt: Format, segs: *const Segment,
                         nseg: u32, m: u32, k: u32, group: u32, workspace: *mut c_void, workspace_bytes: usize,
                         stream: Stream) -> Status;
    pub fn hq_gemm_fused_noalloc(x: *const c_void, dtype: Dtype, ldx: i64, fmt: Format, segs: *const Segment,
                                 nseg: u32, m: u32, k: u32, group: u32, stream: Stream) -> Status;

    // The int8 path (forward_cutlass_int8, hydrogen/src/model/marlin_gemm.cu:603-617).
    pub fn hq_int8_packed_bytes(k: u32, n: u32) -> usize;
    pub fn hq_repack_int8(w_kn: *const i8, k: u32, n: u32, packed: *mut i8) -> Status;
    pub fn hq_unpack_int8(packed: *const i8, k: u32, n: u32, w_kn: *mut i8) -> Status;
    pub fn hq_workspace_bytes_w8a8(m: u32, k: u32, n: u32, bytes: *mut usize) -> Status;
    pub fn hq_gemm_w8a8(x: *const f32, ldx: i64, wp: *const i8, scales: *const f32, y: *mut f32, ldy: i64,
                        m: u32, k: u32, n: u32, workspace: *mut c_void, workspace_bytes: usize,
                        stream: Stream) -> Status;
}

/// A failed call: the status and hq_last_error's message (the reference throws
/// std::runtime_error from CUDA_CHECK instead, hydrogen/src/model/marlin_gemm.cu:19-27).
#[derive(Debug, thiserror::Error)]
#[error("qgemm status {status}: {message}")]
pub struct QgemmError {
    pub status: Status,
    pub message: String,
}

fn check(status: Status) -> Result<(), QgemmError> {
    if status == 0 {
        return Ok(());
    }
    // SAFETY: hq_last_error returns a NUL-terminated thread-local string that stays valid until
    // the next call on this thread; it is copied out at once.
    let message = unsafe { CStr::from_ptr(hq_last_error()) }.to_string_lossy().into_owned();
    Err(QgemmError { status, message })
}

/// The library's version string.
pub fn version() -> String {
    // SAFETY: a static NUL-terminated string.
    unsafe { CStr::from_ptr(hq_version()) }.to_string_lossy().into_owned()
}

/// Host repack of reference-linear weights ([K/8][N] int4 or [K/16][N] ternary words) into the
/// gfx950 tile layout (replaces MarlinGemmEngine::repack_q4k_to_marlin, marlin_gemm.hpp:78-83).
pub fn repack(fmt: Format, linear: &[u32], k: u32, n: u32) -> Result<Vec<u32>, QgemmError> {
    // SAFETY: pure size queries.
    let (need, words) = unsafe { (hq_linear_words(fmt, k, n), hq_packed_words(fmt, k, n)) };
    if need == 0 || words == 0 || linear.len() != need {
        return Err(QgemmError { status: 2, message: format!("linear weight of {} words, K={k} N={n} needs {need}", linear.len()) });
    }
    let mut out = vec![0u32; words];
    // SAFETY: `linear` holds `need` words and `out` holds `words`: the sizes the library reads and writes.
    check(unsafe {
        match fmt {
            Format::Int4 => hq_repack_int4(linear.as_ptr(), out.as_mut_ptr(), k, n),
            Format::Ternary2 => hq_repack_ternary2(linear.as_ptr(), out.as_mut_ptr(), k, n),
        }
    })?;
    Ok(out)
}

/// Workspace bytes of one call (0: none); see hq_workspace_bytes / hq_workspace_bytes_fused.
pub fn workspace_bytes_fused(fmt: Format, m: u32, k: u32, group: u32, ns: &[u32], with_bias: bool)
                             -> Result<usize, QgemmError> {
    let mut bytes = 0usize;
    // SAFETY: `ns` holds `ns.len()` widths; `bytes` is a valid out pointer.
    check(unsafe { hq_workspace_bytes_fused(fmt, m, k, group, ns.as_ptr(), ns.len() as u32, with_bias as c_int,
                                            &mut bytes) })?;
    Ok(bytes)
}

/// Device buffers of one int4 GEMM (replaces forward_marlin_int4, marlin_gemm.hpp:100-107).
/// `bias`: null, or the reference's fp32 [K/group][N] biases. `workspace`: null/0, or a buffer of
/// at least workspace_bytes (zero-filled once before its first use).
/// # Safety
/// The device buffers must have the sizes M, K, N, group, ldx and ldy imply and stay alive until
/// `stream` has executed the call.
pub unsafe fn gemm_w4a16(x: *const c_void, dtype: Dtype, ldx: i64, wp: *const u32, scales: *const u16,
                         bias: *const f32, y: *mut c_void, ldy: i64, m: u32, k: u32, n: u32, group: u32,
                         workspace: *mut c_void, workspace_bytes: usize, stream: Stream) -> Result<(), QgemmError> {
    check(hq_gemm_w4a16(x, dtype, ldx, wp, scales, bias, y, ldy, m, k, n, group, workspace, workspace_bytes, stream))
}

/// Fused projections over one activation read (QKV, gate||up).
/// # Safety
/// As [`gemm_w4a16`], for every segment.
pub unsafe fn gemm_fused(x: *const c_void, dtype: Dtype, ldx: i64, fmt: Format, segs: &[Segment], m: u32, k: u32,
                         group: u32, workspace: *mut c_void, workspace_bytes: usize, stream: Stream)
                         -> Result<(), QgemmError> {
    check(hq_gemm_fused(x, dtype, ldx, fmt, segs.as_ptr(), segs.len() as u32, m, k, group, workspace,
                        workspace_bytes, stream))
}

/// The same without any allocation (callers under stream capture): the library's static scratch.
/// # Safety
/// As [`gemm_w4a16`]; calls on one GPU must not overlap in time.
pub unsafe fn gemm_fused_noalloc(x: *const c_void, dtype: Dtype, ldx: i64, fmt: Format, segs: &[Segment], m: u32,
                                 k: u32, group: u32, stream: Stream) -> Result<(), QgemmError> {
    check(hq_gemm_fused_noalloc(x, dtype, ldx, fmt, segs.as_ptr(), segs.len() as u32, m, k, group, stream))
}

/// Host repack of int8 weights [K][N] (the reference's forward_cutlass_int8 operand,
/// marlin_gemm.hpp:112-118) into the gfx950 i8 tile layout.
pub fn repack_int8(w_kn: &[i8], k: u32, n: u32) -> Result<Vec<i8>, QgemmError> {
    // SAFETY: a pure size query.
    let bytes = unsafe { hq_int8_packed_bytes(k, n) };
    if bytes == 0 || w_kn.len() != k as usize * n as usize {
        return Err(QgemmError { status: 2, message: format!("int8 weight of {} bytes, K={k} N={n}", w_kn.len()) });
    }
    let mut out = vec![0i8; bytes];
    // SAFETY: `w_kn` holds K * N bytes and `out` the packed size the library writes.
    check(unsafe { hq_repack_int8(w_kn.as_ptr(), k, n, out.as_mut_ptr()) })?;
    Ok(out)
}

/// Workspace bytes of one int8 call (the quantised activations and K-piece partial sums).
pub fn workspace_bytes_w8a8(m: u32, k: u32, n: u32) -> Result<usize, QgemmError> {
    let mut bytes = 0usize;
    // SAFETY: `bytes` is a valid out pointer.
    check(unsafe { hq_workspace_bytes_w8a8(m, k, n, &mut bytes) })?;
    Ok(bytes)
}

/// The int8 forward (replaces forward_cutlass_int8, marlin_gemm.cu:603-617): fp32 activations
/// quantised to int8, exact int32 sums, y = scale * sum / 127. `workspace`: null/0 (the library
/// allocates on first use) or at least workspace_bytes_w8a8 bytes (zero-filled once).
/// # Safety
/// The device buffers must have the sizes M, K, N, ldx and ldy imply and stay alive until
/// `stream` has executed the call.
pub unsafe fn gemm_w8a8(x: *const f32, ldx: i64, wp: *const i8, scales: *const f32, y: *mut f32, ldy: i64, m: u32,
                        k: u32, n: u32, workspace: *mut c_void, workspace_bytes: usize, stream: Stream)
                        -> Result<(), QgemmError> {
    check(hq_gemm_w8a8(x, ldx, wp, scales, y, ldy, m, k, n, workspace, workspace_bytes, stream))
}

/// An open GGUF file (replaces hydrogen::ModelLoader for the weights of this path).
pub struct GgufFile {
    g: *mut Gguf,
}

impl GgufFile {
    pub fn open(path: &str) -> Result<Self, QgemmError> {
        let c = CString::new(path).map_err(|e| QgemmError { status: 1, message: e.to_string() })?;
        let mut g = ptr::null_mut();
        // SAFETY: `c` is NUL-terminated; `g` receives an owned handle on success.
        check(unsafe { hq_gguf_open(c.as_ptr(), &mut g) })?;
        Ok(Self { g })
    }

    pub fn header(&self) -> Result<GgufHeaderInfo, QgemmError> {
        let mut h = GgufHeaderInfo::default();
        // SAFETY: `self.g` is a live handle; `h` is a valid out pointer.
        check(unsafe { hq_gguf_header(self.g, &mut h) })?;
        Ok(h)
    }

    pub fn get_int(&self, key: &str) -> Result<i64, QgemmError> {
        let c = CString::new(key).map_err(|e| QgemmError { status: 1, message: e.to_string() })?;
        let mut v = 0i64;
        // SAFETY: live handle, NUL-terminated key, valid out pointer.
        check(unsafe { hq_gguf_get_int(self.g, c.as_ptr(), &mut v) })?;
        Ok(v)
    }

    /// A TQ1_0 projection onto the device (staging >= the tensor's bytes); returns (K, N).
    /// # Safety
    /// The device buffers must hold the sizes hq_gguf_load_tq1_0 documents; keep `self` alive
    /// until `stream` has passed the copy.
    pub unsafe fn load_tq1_0(&self, name: &str, d_staging: *mut c_void, staging_bytes: usize, d_packed: *mut u32,
                             d_scales: *mut u16, stream: Stream) -> Result<(u32, u32), QgemmError> {
        let c = CString::new(name).map_err(|e| QgemmError { status: 1, message: e.to_string() })?;
        let (mut k, mut n) = (0u32, 0u32);
        check(hq_gguf_load_tq1_0(self.g, c.as_ptr(), d_staging, staging_bytes, d_packed, d_scales, &mut k, &mut n,
                                 stream))?;
        Ok((k, n))
    }
}

impl Drop for GgufFile {
    fn drop(&mut self) {
        // SAFETY: `self.g` came from hq_gguf_open and is closed once.
        unsafe { hq_gguf_close(self.g) }
    }
}
