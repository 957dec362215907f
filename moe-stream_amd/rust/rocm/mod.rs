//! `moe-stream-core/src/rocm/mod.rs`: the MI355X expert-FFN path, compiled with
//! `--features rocm` beside `#[cfg(feature = "metal")] pub mod metal;` (lib.rs:7-8).
//!
//! Enabling it in moe-stream-core:
//!   Cargo.toml  [features]     rocm = ["dep:moe-rocm-sys"]
//!               [dependencies] moe-rocm-sys = { path = "<this repo>/moe-stream_amd/rust/moe-rocm-sys", optional = true }
//!   src/lib.rs  #[cfg(feature = "rocm")] pub mod rocm;
//!
//! Safe owners around the raw handles of moe-rocm-sys, errors in the reference's style
//! (`candle_core::Error::Msg`, as metal/mod.rs:1308-1318 reports Metal failures). Hidden
//! states are device pointers (`*const f32` / `*mut f32` of [n_tokens, hidden] f32) in the
//! context device's memory, allocated with `DeviceBuffer`.
use candle_core::{Error, Result};
use moe_rocm_sys as sys;
use std::ffi::{CStr, CString};
use std::os::raw::c_void;
use std::path::Path;

fn last_error(ctx: *const sys::mr_ctx) -> String {
    let p = unsafe { sys::mr_last_error(ctx) };
    if p.is_null() {
        return String::from("unknown error");
    }
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

fn check(ctx: *const sys::mr_ctx, rc: i32, what: &str) -> Result<()> {
    if rc == sys::MR_OK {
        return Ok(());
    }
    Err(Error::Msg(format!("moe-rocm {what}: {}", last_error(ctx))))
}

/// One HIP device and its stream (replaces `Device::new_metal(0)`, engine.rs:278-298).
pub struct RocmContext {
    raw: *mut sys::mr_ctx,
}

impl RocmContext {
    pub fn new(device: i32) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(std::ptr::null(), unsafe { sys::mr_ctx_create(device, &mut raw) }, "mr_ctx_create")?;
        Ok(Self { raw })
    }
    pub fn raw(&self) -> *mut sys::mr_ctx {
        self.raw
    }
    /// Waits for the enqueued work; also reports a fused launch whose bounded wait ran out.
    pub fn sync(&self) -> Result<()> {
        check(self.raw, unsafe { sys::mr_sync(self.raw) }, "mr_sync")
    }
    pub fn alloc(&self, n_floats: usize) -> Result<DeviceBuffer<'_>> {
        let mut p: *mut c_void = std::ptr::null_mut();
        check(self.raw, unsafe { sys::mr_dev_alloc(self.raw, (n_floats * 4) as u64, &mut p) }, "mr_dev_alloc")?;
        Ok(DeviceBuffer { ctx: self, ptr: p as *mut f32, len: n_floats })
    }
}

impl Drop for RocmContext {
    fn drop(&mut self) {
        unsafe { sys::mr_ctx_destroy(self.raw) };
    }
}

/// Device f32 array owned by a context.
pub struct DeviceBuffer<'a> {
    ctx: &'a RocmContext,
    pub ptr: *mut f32,
    pub len: usize,
}

impl DeviceBuffer<'_> {
    pub fn upload(&self, host: &[f32]) -> Result<()> {
        assert!(host.len() <= self.len);
        let rc = unsafe { sys::mr_upload(self.ctx.raw, self.ptr as *mut c_void, host.as_ptr() as *const c_void, (host.len() * 4) as u64) };
        check(self.ctx.raw, rc, "mr_upload")
    }
    /// Stream-ordered: returns after the copy (the reference's `to_vec1` sync, layer.rs:938).
    pub fn download(&self, host: &mut [f32]) -> Result<()> {
        assert!(host.len() <= self.len);
        let rc = unsafe { sys::mr_download(self.ctx.raw, host.as_mut_ptr() as *mut c_void, self.ptr as *const c_void, (host.len() * 4) as u64) };
        check(self.ctx.raw, rc, "mr_download")
    }
}

impl Drop for DeviceBuffer<'_> {
    fn drop(&mut self) {
        unsafe { sys::mr_dev_free(self.ctx.raw, self.ptr as *mut c_void) };
    }
}

/// A memory-mapped GGUF file (GgufReader::open, reader.rs:259-358).
pub struct RocmGguf {
    raw: *mut sys::mr_gguf,
}

impl RocmGguf {
    pub fn open(path: &Path) -> Result<Self> {
        let c = CString::new(path.to_string_lossy().as_bytes()).map_err(|e| Error::Msg(e.to_string()))?;
        let mut raw = std::ptr::null_mut();
        check(std::ptr::null(), unsafe { sys::mr_gguf_open(c.as_ptr(), &mut raw) }, "mr_gguf_open")?;
        Ok(Self { raw })
    }
}

impl Drop for RocmGguf {
    fn drop(&mut self) {
        unsafe { sys::mr_gguf_close(self.raw) };
    }
}

/// One MoE layer resident on the device, with its post-attention norm (what
/// `preload_experts_gpu` + `preload_gates` keep per layer, engine.rs:606-652, 1079-1255).
pub struct RocmLayer {
    raw: *mut sys::mr_layer,
    pub post_norm_w: *const f32,
    pub eps: f32,
}

impl RocmLayer {
    /// Experts uploaded in their native GGUF bytes; routing mode, activation and top-k from
    /// the file's metadata unless `opts` overrides them.
    pub fn from_gguf(ctx: &RocmContext, g: &RocmGguf, layer: u32, opts: Option<&sys::mr_gguf_layer_opts>) -> Result<Self> {
        let (mut raw, mut norm_w, mut eps) = (std::ptr::null_mut(), std::ptr::null(), 0f32);
        let o = opts.map_or(std::ptr::null(), |o| o as *const _);
        let rc = unsafe { sys::mr_gguf_layer_create(ctx.raw, g.raw, layer, o, &mut raw, &mut norm_w, &mut eps) };
        check(ctx.raw, rc, "mr_gguf_layer_create")?;
        Ok(Self { raw, post_norm_w: norm_w, eps })
    }
    /// Scratch for up to max_tokens tokens (BatchedMoeBuffers::new, metal/mod.rs:1240); call
    /// before capturing graphs.
    pub fn reserve(&self, ctx: &RocmContext, max_tokens: u32) -> Result<()> {
        check(ctx.raw, unsafe { sys::mr_reserve(ctx.raw, self.raw, max_tokens) }, "mr_reserve")
    }
}

impl Drop for RocmLayer {
    fn drop(&mut self) {
        unsafe { sys::mr_layer_destroy(self.raw) };
    }
}

/// Links each layer to the next in decode order (the last to the first): each layer's kernel
/// then reads the next layer's router rows into the caches. Results do not change.
pub fn set_decode_order(layers: &mut [RocmLayer]) -> Result<()> {
    let n = layers.len();
    for i in 0..n {
        let next = layers[(i + 1) % n].raw as *const sys::mr_layer;
        check(std::ptr::null(), unsafe { sys::mr_layer_set_next(layers[i].raw, next) }, "mr_layer_set_next")?;
    }
    Ok(())
}

/// One decode token through a layer: router, top-k, experts and combine on the GPU with no
/// host sync (gpu_routed_moe_forward_metal, metal/mod.rs:1512-1677). x, y: [1, hidden].
pub fn gpu_routed_moe_forward_rocm(ctx: &RocmContext, layer: &RocmLayer, x: *const f32, y: *mut f32) -> Result<()> {
    check(ctx.raw, unsafe { sys::mr_moe_forward(ctx.raw, layer.raw, x, y) }, "mr_moe_forward")
}

/// The MoE half of DecoderLayer::forward (layer.rs:462-473) on the resident hidden state:
/// h <- h + moe(rms_norm(h, post_norm_w, eps)), in place.
pub fn moe_block_rocm(ctx: &RocmContext, layer: &RocmLayer, h: *mut f32) -> Result<()> {
    if layer.post_norm_w.is_null() {
        return Err(Error::Msg("moe-rocm: layer has no post_attention_norm weight".into()));
    }
    let rc = unsafe { sys::mr_moe_forward_residual(ctx.raw, layer.raw, h, layer.post_norm_w, layer.eps, h) };
    check(ctx.raw, rc, "mr_moe_forward_residual")
}

/// n_tokens tokens (prefill): tokens grouped by expert, each expert's weights read once
/// (layer.rs:1449-1514, 2148-2183). x, y: [n_tokens, hidden].
pub fn batched_moe_forward_rocm(ctx: &RocmContext, layer: &RocmLayer, x: *const f32, n_tokens: u32, y: *mut f32) -> Result<()> {
    check(ctx.raw, unsafe { sys::mr_moe_forward_batched(ctx.raw, layer.raw, x, n_tokens, y) }, "mr_moe_forward_batched")
}
