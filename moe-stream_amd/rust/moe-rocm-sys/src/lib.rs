//! Raw declarations of include/moe_rocm.h, one per header item, in header order.
//!
//! The safe layer is the `rocm` module of moe-stream-core (the `#[cfg(feature = "rocm")]`
//! sibling of `#[cfg(feature = "metal")] pub mod metal;`, moe-stream-core/src/lib.rs:7-8).
//! Every function returns MR_OK (0) or a negative MR_E_* code; mr_last_error(ctx) holds the
//! message of the context's last failing call. Device pointers are `*const f32` / `*mut f32`
//! addresses in the context device's memory.
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};

// ---- status codes
pub const MR_OK: c_int = 0;
pub const MR_E_INVAL: c_int = -1;
pub const MR_E_NOMEM: c_int = -2;
pub const MR_E_NODEV: c_int = -3;
pub const MR_E_LAUNCH: c_int = -4;
pub const MR_E_UNSUPPORTED: c_int = -5;

// ---- GGML block types (reader.rs:34-128)
pub const MR_GGML_Q4_K: c_int = 12;
pub const MR_GGML_MXFP4: c_int = 39;

// ---- routing flags (top_k_routing, layer.rs:2346-2403)
pub const MR_ROUTE_SOFTMAX_AFTER_TOPK: u32 = 1;
pub const MR_ROUTE_NORM_TOPK: u32 = 2;

// ---- activations (ops/activation.rs:13-38)
pub const MR_ACT_SILU: u32 = 0;
pub const MR_ACT_SWIGLU_OAI: u32 = 1;

pub const MR_DEVICE_NONE: c_int = -1;

// ---- context options
pub const MR_OPT_DECODE_KERNEL: c_int = 1;
pub const MR_DECODE_AUTO: c_int = 0;
pub const MR_DECODE_VALU: c_int = 1;
pub const MR_DECODE_FUSED: c_int = 2;
pub const MR_OPT_PROFILE: c_int = 2;
pub const MR_OPT_WAIT_LIMIT_US: c_int = 3;

pub const MR_STATIC_SCRATCH_BYTES: u64 = 64 << 20;

// ---- opaque handles
#[repr(C)]
pub struct mr_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct mr_pack {
    _p: [u8; 0],
}
#[repr(C)]
pub struct mr_layer {
    _p: [u8; 0],
}
#[repr(C)]
pub struct mr_graph {
    _p: [u8; 0],
}
#[repr(C)]
pub struct mr_gguf {
    _p: [u8; 0],
}

/// What run_moe reads for one layer (cache.rs:319-398; metal/mod.rs:1202-1216, 1440-1485).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct mr_layer_desc {
    pub gate: *const mr_pack,
    pub up: *const mr_pack,
    pub down: *const mr_pack,
    pub gate_bias: *const f32,
    pub up_bias: *const f32,
    pub down_bias: *const f32,
    pub router_w: *const f32,
    pub router_b: *const f32,
    pub dummy_mask: *const f32,
    pub sh_gate: *const mr_pack,
    pub sh_up: *const mr_pack,
    pub sh_down: *const mr_pack,
    pub sh_gate_inp: *const f32,
    pub top_k: u32,
    pub route_flags: u32,
    pub act: u32,
    pub alpha: f32,
    pub limit: f32,
}

/// One tensor's TensorInfo (reader.rs:131-154).
#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct mr_gguf_tensor {
    pub ggml_type: u32,
    pub n_dims: u32,
    pub dims: [u64; 4],
    pub data_offset: u64,
    pub nbytes: u64,
}

/// Options of mr_gguf_layer_create (0 / -1: taken from the file's metadata).
#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct mr_gguf_layer_opts {
    pub top_k: u32,
    pub route_flags: i32,
    pub act: i32,
    pub alpha: f32,
    pub limit: f32,
}

#[link(name = "moe_rocm")]
extern "C" {
    // ---- context, errors, streams
    pub fn mr_ctx_create(device: c_int, out: *mut *mut mr_ctx) -> c_int;
    pub fn mr_ctx_destroy(ctx: *mut mr_ctx);
    pub fn mr_last_error(ctx: *const mr_ctx) -> *const c_char;
    pub fn mr_status_string(status: c_int) -> *const c_char;
    pub fn mr_ctx_device(ctx: *const mr_ctx) -> c_int;
    pub fn mr_ctx_set_stream(ctx: *mut mr_ctx, hip_stream: *mut c_void) -> c_int;
    pub fn mr_ctx_stream(ctx: *const mr_ctx) -> *mut c_void;
    pub fn mr_ctx_set_option(ctx: *mut mr_ctx, option: c_int, value: c_int) -> c_int;
    pub fn mr_sync(ctx: *mut mr_ctx) -> c_int;

    // ---- device memory
    pub fn mr_dev_alloc(ctx: *mut mr_ctx, nbytes: u64, out_dptr: *mut *mut c_void) -> c_int;
    pub fn mr_dev_free(ctx: *mut mr_ctx, dptr: *mut c_void) -> c_int;
    pub fn mr_upload(ctx: *mut mr_ctx, dst: *mut c_void, host_src: *const c_void, nbytes: u64) -> c_int;
    pub fn mr_download(ctx: *mut mr_ctx, host_dst: *mut c_void, src: *const c_void, nbytes: u64) -> c_int;
    pub fn mr_dev_zero(ctx: *mut mr_ctx, dst: *mut c_void, nbytes: u64) -> c_int;

    // ---- expert weights in native GGUF layout
    pub fn mr_pack_upload(
        ctx: *mut mr_ctx,
        ggml_type: c_int,
        host_bytes: *const c_void,
        nbytes: u64,
        n_experts: u32,
        out_features: u32,
        in_features: u32,
        host_offsets: *const u64,
        out: *mut *mut mr_pack,
    ) -> c_int;
    pub fn mr_pack_wrap(
        ctx: *mut mr_ctx,
        ggml_type: c_int,
        dev_bytes: *const c_void,
        nbytes: u64,
        n_experts: u32,
        out_features: u32,
        in_features: u32,
        host_offsets: *const u64,
        out: *mut *mut mr_pack,
    ) -> c_int;
    pub fn mr_pack_destroy(pack: *mut mr_pack);
    pub fn mr_matrix_bytes(ggml_type: c_int, rows: u64, cols: u64) -> u64;
    pub fn mr_dequant(ctx: *mut mr_ctx, pack: *const mr_pack, expert: u32, out: *mut f32) -> c_int;

    // ---- one MoE layer
    pub fn mr_layer_create(ctx: *mut mr_ctx, desc: *const mr_layer_desc, out: *mut *mut mr_layer) -> c_int;
    pub fn mr_layer_destroy(layer: *mut mr_layer);
    pub fn mr_layer_set_next(layer: *mut mr_layer, next: *const mr_layer) -> c_int;
    pub fn mr_layer_set_norm(layer: *mut mr_layer, norm_w: *const f32) -> c_int;
    pub fn mr_layer_set_logits_out(layer: *mut mr_layer, logits: *mut f32, max_tokens: u32) -> c_int;
    pub fn mr_reserve(ctx: *mut mr_ctx, layer: *const mr_layer, max_tokens: u32) -> c_int;

    // ---- hot path
    pub fn mr_router_topk(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        x: *const f32,
        n_tokens: u32,
        idx: *mut i32,
        w: *mut f32,
        logits: *mut f32,
    ) -> c_int;
    pub fn mr_topk(
        ctx: *mut mr_ctx,
        logits: *const f32,
        n_tokens: u32,
        n_experts: u32,
        top_k: u32,
        route_flags: u32,
        idx: *mut i32,
        w: *mut f32,
    ) -> c_int;
    pub fn mr_moe_experts(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        x: *const f32,
        n_tokens: u32,
        idx: *const i32,
        w: *const f32,
        y: *mut f32,
    ) -> c_int;
    pub fn mr_moe_forward(ctx: *mut mr_ctx, layer: *const mr_layer, x: *const f32, y: *mut f32) -> c_int;
    pub fn mr_moe_forward_residual(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        h: *const f32,
        norm_w: *const f32,
        eps: f32,
        h_out: *mut f32,
    ) -> c_int;
    pub fn mr_moe_forward_batched(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        x: *const f32,
        n_tokens: u32,
        y: *mut f32,
    ) -> c_int;
    pub fn mr_moe_forward_batched_residual(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        h: *const f32,
        n_tokens: u32,
        norm_w: *const f32,
        eps: f32,
        h_out: *mut f32,
    ) -> c_int;
    pub fn mr_moe_forward_batched_noalloc(
        ctx: *mut mr_ctx,
        layer: *const mr_layer,
        x: *const f32,
        n_tokens: u32,
        y: *mut f32,
    ) -> c_int;

    // ---- GGUF files
    pub fn mr_gguf_open(path: *const c_char, out: *mut *mut mr_gguf) -> c_int;
    pub fn mr_gguf_close(g: *mut mr_gguf);
    pub fn mr_gguf_n_tensors(g: *const mr_gguf) -> u64;
    pub fn mr_gguf_tensor_name(g: *const mr_gguf, i: u64) -> *const c_char;
    pub fn mr_gguf_tensor_info(g: *const mr_gguf, name: *const c_char, out: *mut mr_gguf_tensor) -> c_int;
    pub fn mr_gguf_tensor_data(
        g: *const mr_gguf,
        name: *const c_char,
        data: *mut *const c_void,
        nbytes: *mut u64,
    ) -> c_int;
    pub fn mr_gguf_meta_u32(g: *const mr_gguf, key: *const c_char, out: *mut u32) -> c_int;
    pub fn mr_gguf_meta_f32(g: *const mr_gguf, key: *const c_char, out: *mut f32) -> c_int;
    pub fn mr_gguf_meta_str(g: *const mr_gguf, key: *const c_char, str_: *mut *const c_char, len: *mut u64) -> c_int;
    pub fn mr_gguf_meta_u32_array(
        g: *const mr_gguf,
        key: *const c_char,
        out: *mut u32,
        cap: u64,
        n: *mut u64,
    ) -> c_int;
    pub fn mr_gguf_upload_experts(
        ctx: *mut mr_ctx,
        g: *const mr_gguf,
        name: *const c_char,
        out: *mut *mut mr_pack,
    ) -> c_int;
    pub fn mr_gguf_layer_create(
        ctx: *mut mr_ctx,
        g: *const mr_gguf,
        layer: u32,
        opts: *const mr_gguf_layer_opts,
        out: *mut *mut mr_layer,
        norm_w: *mut *const f32,
        eps: *mut f32,
    ) -> c_int;

    // ---- graph capture of a sequence of calls
    pub fn mr_graph_begin(ctx: *mut mr_ctx) -> c_int;
    pub fn mr_graph_end(ctx: *mut mr_ctx, out: *mut *mut mr_graph) -> c_int;
    pub fn mr_graph_launch(ctx: *mut mr_ctx, graph: *const mr_graph) -> c_int;
    pub fn mr_graph_destroy(graph: *mut mr_graph);

    // ---- timing on the context stream
    pub fn mr_timer_start(ctx: *mut mr_ctx) -> c_int;
    pub fn mr_timer_stop(ctx: *mut mr_ctx, out_ms: *mut f32) -> c_int;
    pub fn mr_profile_read(ctx: *mut mr_ctx, kernel: *const c_char, out_count: *mut u64, out_total_ms: *mut f64)
        -> c_int;
    pub fn mr_profile_reset(ctx: *mut mr_ctx) -> c_int;

}
