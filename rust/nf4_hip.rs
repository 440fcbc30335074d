//! `extern "C"` binding of libnf4stream.so (include/nf4stream.h) for the
//! AethelStream crates, compiled under a `hip` feature.
//!
//! A maintainer drops this file into `shard_engine/src/nf4_hip.rs` (and
//! `doublepass` uses it through `shard_engine`), following the crates'
//! existing Rust->native convention (galore/src/kernels/mod.rs:6-96):
//! `extern "C"` functions returning an `i32` status (0 = ok), device buffers
//! and the stream as raw pointers, a status mapped to the crate's error type.
//! Every declaration here matches the C header one for one
//! (tests/test_rust_binding.py checks names, argument types and the struct
//! layouts); nothing in this repository compiles it, as the image has no
//! Rust toolchain.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_void};

pub const NF4S_ABI_VERSION: i32 = 3;

pub const NF4S_OK: i32 = 0;
pub const NF4S_ERR_INVALID_ARGUMENT: i32 = 1;
pub const NF4S_ERR_ABSMAX_TOO_SMALL: i32 = 2;
pub const NF4S_ERR_PACKED_TOO_SMALL: i32 = 3;
pub const NF4S_ERR_MISALIGNED: i32 = 4;
pub const NF4S_ERR_UNSUPPORTED_SHAPE: i32 = 5;
pub const NF4S_ERR_HIP: i32 = 6;
pub const NF4S_ERR_IO: i32 = 7;
pub const NF4S_ERR_JSON: i32 = 8;
pub const NF4S_ERR_LAYER_NOT_FOUND: i32 = 9;
pub const NF4S_ERR_PARAM_NOT_FOUND: i32 = 10;
pub const NF4S_ERR_MALFORMED_INDEX: i32 = 11;
pub const NF4S_ERR_PREFETCH_MISS: i32 = 12;

/// `enum nf4s_precision`: flowcast/src/config.rs:16-27 Precision, plus NF4.
pub const NF4S_PRECISION_FP32: i32 = 0;
pub const NF4S_PRECISION_FP16: i32 = 1;
pub const NF4S_PRECISION_BF16: i32 = 2;
pub const NF4S_PRECISION_INT8: i32 = 3;
pub const NF4S_PRECISION_INT4: i32 = 4;
pub const NF4S_PRECISION_NF4: i32 = 5;

/// `struct nf4s_tensor`: one NF4 tensor resident in device memory.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Nf4sTensor {
    pub packed: *const u8,
    pub packed_len: i64,
    pub absmax: *const f32,
    pub absmax_q: *const u8,
    pub absmax_scale: *const f32,
    pub absmax_len: i64,
    pub scale_len: i64,
    pub block_size: i32,
    pub dq_group: i32,
}

/// `struct nf4s_param_info`: IndexStore::tensor_info as a plain struct.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Nf4sParamInfo {
    pub shape: [i64; 8],
    pub ndim: i32,
    pub precision: i32,
    pub numel: i64,
    pub byte_length: i64,
    pub absmax_len: i64,
    pub scale_len: i64,
    pub block_size: i32,
    pub dq_group: i32,
    pub out_elems: i64,
    pub precision_str: [c_char; 16],
    pub dtype_str: [c_char; 16],
}

/// `struct nf4s_ready_layer`: FlowCast's ReadyLayer (flowcast/src/ready.rs:20-52).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Nf4sReadyLayer {
    pub layer_idx: u32,
    pub slab_device_ptr: *mut c_void,
    pub bytes: i64,
    pub copy_event: *mut c_void,
    pub precision: i32,
    pub needs_decode: i32,
}

/// `struct nf4s_blob_entry`: one parameter's parts inside a layer blob.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Nf4sBlobEntry {
    pub packed_off: i64,
    pub packed_len: i64,
    pub absmax_off: i64,
    pub absmax_len: i64,
    pub scale_off: i64,
    pub scale_len: i64,
    pub block_size: i32,
    pub dq_group: i32,
}

/// Opaque `nf4s_dbuf` (VRAM double buffer).
#[repr(C)]
pub struct Nf4sDbuf {
    _private: [u8; 0],
}

/// Opaque `nf4s_residency` (the prefetch state machine's ready map).
#[repr(C)]
pub struct Nf4sResidency {
    _private: [u8; 0],
}

/// Opaque `nf4s_loader` (shard loader).
#[repr(C)]
pub struct Nf4sLoader {
    _private: [u8; 0],
}

#[link(name = "nf4stream")]
extern "C" {
    pub fn nf4s_abi_version() -> i32;
    pub fn nf4s_strerror(status: i32) -> *const c_char;
    pub fn nf4s_last_error_message() -> *const c_char;

    pub fn nf4s_quantize(x: *const f32, n: i64, block_size: i32, packed: *mut u8,
                         absmax: *mut f32, stream: *mut c_void) -> i32;
    pub fn nf4s_dq_encode(absmax: *const f32, nblocks: i64, group: i32, q: *mut u8,
                          scale: *mut f32, stream: *mut c_void) -> i32;
    pub fn nf4s_quantize_bf16(x: *const u16, n: i64, block_size: i32, packed: *mut u8,
                              absmax: *mut f32, stream: *mut c_void) -> i32;
    pub fn nf4s_quantize_dq(x: *const f32, n: i64, block_size: i32, group: i32,
                            packed: *mut u8, absmax_q: *mut u8, absmax_scale: *mut f32,
                            stream: *mut c_void) -> i32;
    pub fn nf4s_quantize_dq_bf16(x: *const u16, n: i64, block_size: i32, group: i32,
                                 packed: *mut u8, absmax_q: *mut u8, absmax_scale: *mut f32,
                                 stream: *mut c_void) -> i32;

    pub fn nf4s_dequant_f16(t: *const Nf4sTensor, n: i64, out: *mut u16,
                            stream: *mut c_void) -> i32;
    pub fn nf4s_dequant_bf16(t: *const Nf4sTensor, n: i64, out: *mut u16,
                             stream: *mut c_void) -> i32;
    pub fn nf4s_dequant_batch_bf16(ts: *const Nf4sTensor, ns: *const i64, outs: *const *mut u16,
                                   count: i32, stream: *mut c_void) -> i32;

    pub fn nf4s_gemm_fwd(x: *const u16, w: *const Nf4sTensor, m: i64, n: i64, k: i64,
                         y: *mut u16, stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_dgrad(dy: *const u16, w: *const Nf4sTensor, m: i64, n: i64, k: i64,
                           dx: *mut u16, stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_fwd_grouped(x: *const u16, ws: *const Nf4sTensor, ns: *const i64,
                                 ys: *const *mut u16, count: i32, m: i64, k: i64,
                                 stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_fwd_swiglu(x: *const u16, w_gate: *const Nf4sTensor,
                                w_up: *const Nf4sTensor, m: i64, ff: i64, k: i64,
                                hidden: *mut u16, stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_dgrad_sum(dys: *const *const u16, ws: *const Nf4sTensor, ns: *const i64,
                               count: i32, m: i64, k: i64, dx: *mut u16,
                               stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_dgrad_sum_ws(dys: *const *const u16, ws: *const Nf4sTensor, ns: *const i64,
                                  count: i32, m: i64, k: i64, dx: *mut u16,
                                  workspace: *mut c_void, workspace_bytes: i64,
                                  stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_dgrad_workspace_size(ns: *const i64, count: i32, m: i64, k: i64,
                                          bytes: *mut i64) -> i32;
    pub fn nf4s_gemm_fwd_grouped_ws(x: *const u16, ws: *const Nf4sTensor, ns: *const i64,
                                    ys: *const *mut u16, count: i32, m: i64, k: i64,
                                    workspace: *mut c_void, workspace_bytes: i64,
                                    stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_fwd_workspace_size(ns: *const i64, count: i32, m: i64, k: i64,
                                        bytes: *mut i64) -> i32;
    pub fn nf4s_gemm_fwd_grouped_noalloc(x: *const u16, ws: *const Nf4sTensor, ns: *const i64,
                                         ys: *const *mut u16, count: i32, m: i64, k: i64,
                                         stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_wgrad(dy: *const c_void, x: *const c_void, m: i64, n: i64, k: i64,
                           dw: *mut f32, accumulate: i32, stream: *mut c_void) -> i32;
    pub fn nf4s_gemm_wgrad_grouped(dys: *const *const c_void, ns: *const i64,
                                   dws: *const *mut f32, count: i32, x: *const c_void, m: i64,
                                   k: i64, accumulate: i32, stream: *mut c_void) -> i32;
    pub fn nf4s_rmsnorm_fwd(x: *const f32, w: *const f32, m: i64, d: i64, eps: f32, y: *mut u16,
                            rms: *mut f32, stream: *mut c_void) -> i32;

    pub fn nf4s_host_alloc(bytes: i64, out: *mut *mut c_void) -> i32;
    pub fn nf4s_host_free(p: *mut c_void) -> i32;
    pub fn nf4s_dbuf_create(slot_bytes: i64, out: *mut *mut Nf4sDbuf) -> i32;
    pub fn nf4s_dbuf_destroy(d: *mut Nf4sDbuf) -> i32;
    pub fn nf4s_dbuf_capacity(d: *const Nf4sDbuf) -> i64;
    pub fn nf4s_dbuf_advance(d: *mut Nf4sDbuf, layer_idx: u32, src: *const c_void, len: i64,
                             dev_ptr: *mut *mut c_void, ready_event: *mut *mut c_void) -> i32;
    pub fn nf4s_dbuf_release(d: *mut Nf4sDbuf, dev_ptr: *const c_void,
                             compute_stream: *mut c_void) -> i32;
    pub fn nf4s_take_ready(d: *mut Nf4sDbuf, layer_idx: u32, pinned: *const c_void, len: i64,
                           out: *mut Nf4sReadyLayer) -> i32;
    pub fn nf4s_residency_create(num_layers: u32, out: *mut *mut Nf4sResidency) -> i32;
    pub fn nf4s_residency_destroy(r: *mut Nf4sResidency) -> i32;
    pub fn nf4s_residency_publish(r: *mut Nf4sResidency, layer_idx: u32, pinned: *const c_void,
                                  bytes: i64, precision: i32) -> i32;
    pub fn nf4s_residency_wait(r: *mut Nf4sResidency, layer_idx: u32, timeout_us: i64,
                               pinned: *mut *const c_void, bytes: *mut i64,
                               precision: *mut i32) -> i32;
    pub fn nf4s_take_ready_wait(d: *mut Nf4sDbuf, r: *mut Nf4sResidency, layer_idx: u32,
                                timeout_us: i64, out: *mut Nf4sReadyLayer) -> i32;
    pub fn nf4s_retire_layer(d: *mut Nf4sDbuf, layer: *const Nf4sReadyLayer,
                             compute_stream: *mut c_void) -> i32;
    pub fn nf4s_stream_wait_event(stream: *mut c_void, event: *mut c_void) -> i32;

    pub fn nf4s_loader_open(model_dir: *const c_char, out: *mut *mut Nf4sLoader) -> i32;
    pub fn nf4s_loader_close(l: *mut Nf4sLoader) -> i32;
    pub fn nf4s_loader_param_info(l: *mut Nf4sLoader, name: *const c_char,
                                  out: *mut Nf4sParamInfo) -> i32;
    pub fn nf4s_loader_load_layer(l: *mut Nf4sLoader, layer: u32, data: *mut *const u8,
                                  len: *mut i64) -> i32;
    pub fn nf4s_loader_staging_size(l: *mut Nf4sLoader, name: *const c_char,
                                    bytes: *mut i64) -> i32;
    pub fn nf4s_loader_load_param_f16(l: *mut Nf4sLoader, name: *const c_char, out: *mut u16,
                                      out_len: i64, staging: *mut c_void, staging_bytes: i64,
                                      stream: *mut c_void) -> i32;
    pub fn nf4s_loader_load_param_nf4(l: *mut Nf4sLoader, name: *const c_char, packed: *mut u8,
                                      packed_bytes: i64, absmax_or_q: *mut c_void,
                                      absmax_bytes: i64, scale: *mut f32, scale_bytes: i64,
                                      stream: *mut c_void) -> i32;
    pub fn nf4s_loader_pack_layer(l: *mut Nf4sLoader, names: *const *const c_char, count: i32,
                                  dst: *mut c_void, dst_bytes: i64, entries: *mut Nf4sBlobEntry,
                                  bytes: *mut i64) -> i32;
    pub fn nf4s_blob_tensor(e: *const Nf4sBlobEntry, base: *const c_void,
                            out: *mut Nf4sTensor) -> i32;
}

/// The message of the last call on this thread ("" after a success).
pub fn last_error() -> String {
    // SAFETY: the library returns a NUL-terminated thread-local buffer.
    unsafe { std::ffi::CStr::from_ptr(nf4s_last_error_message()) }
        .to_string_lossy()
        .into_owned()
}

/// Maps a status to the reference's error type (shard_engine/src/error.rs:5-28):
/// the two dequant checks keep their MalformedIndex field names
/// (nf4.rs:46-57), an I/O failure is Io, anything else MalformedIndex with
/// the library's message.
pub fn check(status: i32) -> crate::error::Result<()> {
    use crate::error::ShardEngineError as E;
    if status == NF4S_OK {
        return Ok(());
    }
    let msg = last_error();
    Err(match status {
        NF4S_ERR_ABSMAX_TOO_SMALL => E::MalformedIndex("nf4_absmax".to_owned(), msg),
        NF4S_ERR_PACKED_TOO_SMALL => E::MalformedIndex("nf4_packed".to_owned(), msg),
        NF4S_ERR_IO => E::Io(std::io::Error::new(std::io::ErrorKind::Other, msg)),
        _ => E::MalformedIndex("nf4_hip".to_owned(), msg),
    })
}
