//! Raw FFI of `libmi355x_attn.so`, the gfx950 attention hot path of the MI355X build.
//!
//! The declarations mirror `include/mi355x_attn.h` one for one (a CPU test of the
//! repository checks every name and parameter type against the header). Every compute
//! entry takes raw device pointers, element strides, a dtype code (0 bf16, 1 fp16, as the
//! reference's native launchers) and a `hipStream_t` as `*mut c_void`, and returns NULL on
//! success or a thread-local error string (valid until the next failing call on the thread).
//! `current_stream` gives the ATen current stream of a device, the stream every call of the
//! reference's bridges runs on.
#![allow(clippy::too_many_arguments)]

use std::ffi::{CStr, c_char, c_int, c_void};

#[link(name = "mi355x_attn")]
unsafe extern "C" {
    pub fn mi355x_attn_error() -> *const c_char;
    pub fn mi355x_store_kv(k: *const c_void, v: *const c_void, kc: *mut c_void, vc: *mut c_void,
        loc: *const c_void, tokens: i64, heads: i64, width: i64, capacity: i64,
        kt: i64, kh: i64, vt: i64, vh: i64, reserved: i64, index64: bool,
        error_count: *mut i32, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_rms_norm(x: *const c_void, w: *const c_void, out: *mut c_void, tokens: i64,
        heads: i64, width: i64, token_stride: i64, head_stride: i64, eps: f64, dtype: c_int,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_add_rms_norm(x: *mut c_void, residual: *mut c_void, w: *const c_void,
        tokens: i64, width: i64, x_stride: i64, residual_stride: i64, eps: f64, dtype: c_int,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_qk_norm(q: *mut c_void, k: *mut c_void, qw: *const c_void, kw: *const c_void,
        tokens: i64, q_heads: i64, k_heads: i64, width: i64, q_ts: i64, q_hs: i64,
        k_ts: i64, k_hs: i64, eps: f64, dtype: c_int, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_decode_prepare(existing: *mut c_void, block_table: *const i32, batch: i64,
        columns: i64, table_stride: i64, seq_lens: *const i32, num_q_heads: i64,
        num_kv_heads: i64, head_dim: i64, page_size: i64, dtype: i64, graph: bool,
        host_lengths: *const i32, host_rows: i64, stream: *mut c_void) -> *mut c_void;
    pub fn mi355x_decode_run(plan: *const c_void, q: *const c_void, q_sn: i64, q_sh: i64,
        k_cache: *const c_void, v_cache: *const c_void, out: *mut c_void, o_sn: i64, o_sh: i64,
        batch: i64, num_q_heads: i64, num_kv_heads: i64, page_size: i64, dtype: i64,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_decode_plan_drop(plan: *mut c_void);
    pub fn mi355x_decode_workspace_allocations(plan: *const c_void) -> u64;
    pub fn mi355x_prefill_prepare(existing: *mut c_void, q_indptr: *const i32,
        block_table: *const i32, batch: i64, columns: i64, table_stride: i64,
        q_host: *const i32, prefix_host: *const i32, num_q_heads: i64, num_kv_heads: i64,
        page_size: i64, dtype: i64, stream: *mut c_void) -> *mut c_void;
    pub fn mi355x_prefill_run(plan: *const c_void, q: *const c_void, q_sn: i64, q_sh: i64,
        k: *const c_void, k_sn: i64, k_sh: i64, v: *const c_void, v_sn: i64, v_sh: i64,
        out: *mut c_void, o_sn: i64, o_sh: i64, total_q: i64, num_q_heads: i64,
        num_kv_heads: i64, page_size: i64, dtype: i64, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_prefill_plan_drop(plan: *mut c_void);
    pub fn mi355x_rope(q: *mut c_void, k: *mut c_void, positions: *const i64, cos: *const f32,
        sin: *const f32, tokens: i64, q_heads: i64, k_heads: i64, width: i64, q_ts: i64,
        q_hs: i64, k_ts: i64, k_hs: i64, max_positions: i64, dtype: c_int,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_qk_norm_rope_store(q: *mut c_void, k: *mut c_void, v: *const c_void,
        q_weight: *const c_void, k_weight: *const c_void, positions: *const i64,
        cos: *const f32, sin: *const f32, max_positions: i64, k_cache: *mut c_void,
        v_cache: *mut c_void, loc: *const c_void, index64: bool, capacity: i64, reserved: i64,
        error_count: *mut i32, tokens: i64, q_heads: i64, k_heads: i64, width: i64,
        q_ts: i64, q_hs: i64, k_ts: i64, k_hs: i64, v_ts: i64, v_hs: i64, eps: f64,
        dtype: c_int, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_silu_mul(gate_up: *const c_void, out: *mut c_void, tokens: i64, width: i64,
        dtype: c_int, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_linear_qk_norm_rope_store(x: *const c_void, ldx: i64, w: *const c_void,
        ldw: i64, qkv: *mut c_void, ldo: i64, m: i64, k: i64, q_heads: i64, k_heads: i64,
        workspace: *mut c_void, workspace_bytes: i64, cus: i32, q_weight: *const c_void,
        k_weight: *const c_void, positions: *const i64, cos: *const f32, sin: *const f32,
        max_positions: i64, k_cache: *mut c_void, v_cache: *mut c_void, loc: *const c_void,
        index64: bool, capacity: i64, reserved: i64, error_count: *mut i32, eps: f64,
        dtype: c_int, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_linear(x: *const c_void, ldx: i64, w: *const c_void, ldw: i64,
        out: *mut c_void, ldo: i64, m: i64, n: i64, k: i64, workspace: *mut c_void,
        workspace_bytes: i64, cus: i32, config: i32, splits: i32, dtype: i64,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_linear_add_rms_norm(x: *const c_void, ldx: i64, w: *const c_void, ldw: i64,
        residual: *mut c_void, ldr: i64, norm_weight: *const c_void, eps: f64,
        out: *mut c_void, ldo: i64, m: i64, n: i64, k: i64, workspace: *mut c_void,
        workspace_bytes: i64, cus: i32, dtype: i64, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_linear_silu_mul(x: *const c_void, ldx: i64, w: *const c_void, ldw: i64,
        out: *mut c_void, ldo: i64, m: i64, width: i64, k: i64, cus: i32, config: i32,
        dtype: i64, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_linear_workspace_bytes(m: i64, n: i64, k: i64, cus: i32, config: i32,
        splits: i32) -> i64;
    pub fn mi355x_linear_noalloc(x: *const c_void, ldx: i64, w: *const c_void, ldw: i64,
        out: *mut c_void, ldo: i64, m: i64, n: i64, k: i64, cus: i32, config: i32,
        splits: i32, dtype: i64, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_sample(logits: *const c_void, rows: i64, vocab: i64, row_stride: i64,
        dtype: c_int, temperature: *const f32, top_k: *const i32, top_p: *const f32,
        seed: u64, offset: u64, out: *mut i64, stream: *mut c_void) -> *const c_char;
}

/// Introspection and host-side planning entries (ported tests, diagnostics); the serving
/// path does not need them.
#[link(name = "mi355x_attn")]
unsafe extern "C" {
    pub fn mi355x_attn_abi_version() -> c_int;
    pub fn mi355x_decode_plan_info(plan: *const c_void, out6: *mut i64) -> *const c_char;
    pub fn mi355x_decode_plan_read(plan: *const c_void, indptr: *mut i32, indices: *mut i32,
        last_len: *mut i32, work: *mut i32, merge: *mut i32,
        stream: *mut c_void) -> *const c_char;
    pub fn mi355x_decode_schedule(lengths: *const i32, batch: i64, cus: i64, num_kv_heads: i64,
        work: *mut i32, work_capacity: i64, merge: *mut i32, chunk_tokens: *mut i64) -> i64;
    pub fn mi355x_decode_items_capacity(rows: i64, cus: i64, num_kv_heads: i64) -> i64;
    pub fn mi355x_prefill_plan_info(plan: *const c_void, out6: *mut i64) -> *const c_char;
    pub fn mi355x_prefill_plan_read(plan: *const c_void, kv_indptr: *mut i32,
        indices: *mut i32, last_len: *mut i32, stream: *mut c_void) -> *const c_char;
    pub fn mi355x_prefill_schedule(q_host: *const i32, prefix_host: *const i32, batch: i64,
        num_q_heads: i64, num_kv_heads: i64, work: *mut i32, capacity: i64) -> i64;
    pub fn mi355x_prefill_workspace_allocations(plan: *const c_void) -> u64;
}

#[cfg(has_mi355x_stream_shim)]
unsafe extern "C" {
    /// `c10::hip::getCurrentHIPStream(device).stream()` (shim/current_stream.cpp).
    fn mi355x_sys_current_stream(device: c_int) -> *mut c_void;
}

/// The ATen current stream of `device` (the stream the reference's bridges launch on), or
/// the null (default) stream when the shim was not built.
pub fn current_stream(device: i64) -> *mut c_void {
    #[cfg(has_mi355x_stream_shim)]
    {
        unsafe { mi355x_sys_current_stream(device as c_int) }
    }
    #[cfg(not(has_mi355x_stream_shim))]
    {
        let _ = device;
        std::ptr::null_mut()
    }
}

/// Turns an entry's returned error string into `Err(message)`.
pub fn check(status: *const c_char) -> Result<(), String> {
    if status.is_null() {
        Ok(())
    } else {
        Err(unsafe { CStr::from_ptr(status) }.to_string_lossy().into_owned())
    }
}

/// The message of the last failed call on this thread (for entries that return a handle).
pub fn last_error() -> String {
    let message = unsafe { mi355x_attn_error() };
    if message.is_null() {
        String::new()
    } else {
        unsafe { CStr::from_ptr(message) }.to_string_lossy().into_owned()
    }
}
