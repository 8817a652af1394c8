//! Raw bindings to `include/iq_qgemm.h` (libiq_qgemm.so) and thin safe
//! wrappers with the signatures inferq's `qgemm` / `QuantizedMatrix` /
//! `QuantizedMoeLayer` call sites use.  Every entry returns 0 or a negative
//! status; `check` turns a status into an `anyhow` error carrying the
//! library's message (the reference reports errors the same way).
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr, CString};

pub const IQ_Q8_0: c_int = 8;
pub const IQ_Q4_K: c_int = 12;
pub const IQ_Q5_K: c_int = 13;
pub const IQ_Q6_K: c_int = 14;
/// Unquantised matrices (the reference's F32 / BF16 QuantizedMatrix).
pub const IQ_F32: c_int = 0;
pub const IQ_BF16: c_int = 30;

pub const IQ_OK: c_int = 0;
pub const IQ_ERR_INVALID: c_int = -1;
pub const IQ_ERR_SHAPE: c_int = -2;
pub const IQ_ERR_DTYPE: c_int = -3;
pub const IQ_ERR_OOM: c_int = -4;
pub const IQ_ERR_HIP: c_int = -5;
pub const IQ_ERR_RANGE: c_int = -6;

/// enum iq_path (the reference's MultiRowPath, src/gguf.rs:43-62).
pub const IQ_PATH_AUTO: c_int = 0;
pub const IQ_PATH_LANES: c_int = 1;
pub const IQ_PATH_GEMV: c_int = 2;
pub const IQ_PATH_LANE_MFMA: c_int = 3;
pub const IQ_PATH_PREFILL_TILES: c_int = 4;

#[repr(C)]
pub struct iq_weight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct iq_moe {
    _p: [u8; 0],
}
#[repr(C)]
pub struct iq_gguf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct iq_experts {
    _p: [u8; 0],
}
pub type iq_weight_t = *mut iq_weight;
pub type iq_moe_t = *mut iq_moe;
pub type iq_gguf_t = *mut iq_gguf;
pub type iq_experts_t = *mut iq_experts;
/// hipStream_t (null: the default stream).
pub type iq_stream_t = *mut c_void;

/// iq_moe_desc: one MoE sublayer over device-resident GGUF expert tensors.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct iq_moe_desc {
    pub hidden: i64,
    pub inter: i64,
    pub n_experts: i64,
    pub top_k: i64,
    pub normalize: c_int,
    pub gate_dtype: c_int,
    pub down_dtype: c_int,
    pub gate: *const c_void,
    pub up: *const c_void,
    pub down: *const c_void,
    pub gate_bytes: usize,
    pub up_bytes: usize,
    pub down_bytes: usize,
    pub shared_gate_dtype: c_int,
    pub shared_down_dtype: c_int,
    pub shared_gate: *const c_void,
    pub shared_up: *const c_void,
    pub shared_down: *const c_void,
    pub selector: *const f32,
    pub router: *const f32,
}

extern "C" {
    pub fn iq_version() -> *const c_char;
    pub fn iq_last_error() -> *const c_char;
    pub fn iq_init(device: c_int) -> c_int;

    pub fn iq_weights_upload(host: *const c_void, n: usize, dtype: c_int, rows: i64, cols: i64,
                             out: *mut iq_weight_t) -> c_int;
    pub fn iq_weights_view(dev: *const c_void, n: usize, dtype: c_int, rows: i64, cols: i64,
                           out: *mut iq_weight_t) -> c_int;
    pub fn iq_weights_free(w: iq_weight_t) -> c_int;
    pub fn iq_weights_info(w: iq_weight_t, dtype: *mut c_int, rows: *mut i64, cols: *mut i64, nbytes: *mut usize,
                           dev: *mut *const c_void) -> c_int;
    pub fn iq_weights_concat_rows(a: iq_weight_t, b: iq_weight_t, out: *mut iq_weight_t) -> c_int;
    pub fn iq_weights_leading_rows(a: iq_weight_t, rows: i64, out: *mut iq_weight_t) -> c_int;

    pub fn iq_matmul(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, stream: iq_stream_t) -> c_int;
    pub fn iq_matmul_via(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, path: c_int, stream: iq_stream_t)
        -> c_int;
    pub fn iq_matmul_noalloc(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, stream: iq_stream_t) -> c_int;
    pub fn iq_matmul_noalloc_max_bytes() -> usize;
    pub fn iq_matmul_workspace_size(w: iq_weight_t, m: i64) -> usize;
    pub fn iq_matmul_reserve(w: iq_weight_t, m: i64, stream: iq_stream_t) -> c_int;
    pub fn iq_workspace_release(stream: iq_stream_t) -> c_int;
    pub fn iq_matmul_ws(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, ws: *mut c_void, ws_bytes: usize,
                        stream: iq_stream_t) -> c_int;
    pub fn iq_matmul_host(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32) -> c_int;

    pub fn iq_q4k_q8k_row(weight: *const c_void, weight_blocks: usize, inputs: *const c_void, input_blocks: usize,
                          rows: usize, out: *mut f32, out_len: usize) -> c_int;
    pub fn iq_q6k_q8k_row(weight: *const c_void, weight_blocks: usize, inputs: *const c_void, input_blocks: usize,
                          rows: usize, out: *mut f32, out_len: usize) -> c_int;
    pub fn iq_q80_q80_row(weight: *const c_void, weight_blocks: usize, inputs: *const c_void, input_blocks: usize,
                          rows: usize, out: *mut f32, out_len: usize) -> c_int;

    pub fn iq_argmax_rows(y: *const f32, m: i64, n: i64, idx: *mut i32, val: *mut f32, stream: iq_stream_t) -> c_int;
    pub fn iq_matmul_argmax(w: iq_weight_t, x: *const f32, m: i64, idx: *mut i32, val: *mut f32,
                            stream: iq_stream_t) -> c_int;

    pub fn iq_quantize_q8k(x: *const f32, m: i64, k: i64, out: *mut c_void, stream: iq_stream_t) -> c_int;
    pub fn iq_quantize_q80(x: *const f32, m: i64, k: i64, out: *mut c_void, stream: iq_stream_t) -> c_int;
    pub fn iq_block_sums(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, isum: *mut i32, msum: *mut i32,
                         stream: iq_stream_t) -> c_int;
    pub fn iq_prefill_block_sums(w: iq_weight_t, x: *const f32, m: i64, y: *mut f32, isum: *mut i32,
                                 msum: *mut i32, stream: iq_stream_t) -> c_int;

    pub fn iq_moe_create(d: *const iq_moe_desc, out: *mut iq_moe_t) -> c_int;
    pub fn iq_moe_destroy(l: iq_moe_t) -> c_int;
    pub fn iq_moe_reserve(l: iq_moe_t, max_tokens: i64, stream: iq_stream_t) -> c_int;
    pub fn iq_moe_slice_tokens(l: iq_moe_t) -> i64;
    pub fn iq_moe_set_path(l: iq_moe_t, path: c_int) -> c_int;
    pub fn iq_moe_forward(l: iq_moe_t, x: *const f32, logits: *const f32, m: i64, out: *mut f32,
                          experts: *mut i32, weights: *mut f32, stream: iq_stream_t) -> c_int;
    pub fn iq_moe_forward_x(l: iq_moe_t, x: *const f32, m: i64, residual: *const f32, out: *mut f32,
                            experts: *mut i32, weights: *mut f32, stream: iq_stream_t) -> c_int;
    pub fn iq_moe_forward_timed(l: iq_moe_t, x: *const f32, logits: *const f32, m: i64, out: *mut f32,
                                experts: *mut i32, weights: *mut f32, events: *const *mut c_void,
                                stream: iq_stream_t) -> c_int;
    pub fn iq_moe_forward_stage(l: iq_moe_t, stage: c_int, stream: iq_stream_t) -> c_int;

    pub fn iq_gguf_open(path: *const c_char, out: *mut iq_gguf_t) -> c_int;
    pub fn iq_gguf_close(g: iq_gguf_t) -> c_int;
    pub fn iq_gguf_tensor_count(g: iq_gguf_t) -> i64;
    pub fn iq_gguf_tensor_name(g: iq_gguf_t, index: i64) -> *const c_char;
    pub fn iq_gguf_tensor_info(g: iq_gguf_t, name: *const c_char, dtype: *mut c_int, n_dims: *mut c_int,
                               dims: *mut i64, file_offset: *mut u64, nbytes: *mut u64) -> c_int;
    pub fn iq_gguf_meta_int(g: iq_gguf_t, key: *const c_char, value: *mut i64) -> c_int;
    pub fn iq_gguf_meta_str(g: iq_gguf_t, key: *const c_char) -> *const c_char;
    pub fn iq_gguf_load_matrix(g: iq_gguf_t, name: *const c_char, out: *mut iq_weight_t) -> c_int;
    pub fn iq_gguf_upload_tensor(g: iq_gguf_t, name: *const c_char, dst: *mut c_void, capacity: usize,
                                 stream: iq_stream_t) -> c_int;
    pub fn iq_gguf_load_experts(g: iq_gguf_t, n_layers: i64, out: *mut iq_experts_t) -> c_int;
    pub fn iq_experts_free(r: iq_experts_t) -> c_int;
    pub fn iq_experts_bytes(r: iq_experts_t) -> usize;
    pub fn iq_experts_layer(r: iq_experts_t, layer: i64, desc: *mut iq_moe_desc) -> c_int;
}

/// A status as an `anyhow` error with the library's message.
pub fn check(status: c_int) -> anyhow::Result<()> {
    if status == IQ_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(iq_last_error()) }.to_string_lossy().into_owned();
    anyhow::bail!("{msg} (status {status})")
}

/// The GGUF blocks of the reference's `qgemm` mirrors (src/qgemm.rs:46-65):
/// plain bytes with the reference's sizes, so a `&[Q4KBlock]` slice of the
/// reference can be passed as-is.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q4KBlock(pub [u8; 144]);
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q6KBlock(pub [u8; 210]);
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q80Block(pub [u8; 34]);
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q8KBlock(pub [u8; 292]);

/// `q4k_q8k_row` with the reference's signature (src/qgemm.rs:447-468):
/// one weight row against `rows` block-major inputs; the debug asserts
/// become errors.
pub fn q4k_q8k_row(weight: &[Q4KBlock], inputs: &[Q8KBlock], rows: usize, out: &mut [f32]) -> anyhow::Result<()> {
    check(unsafe {
        iq_q4k_q8k_row(weight.as_ptr().cast(), weight.len(), inputs.as_ptr().cast(), inputs.len(), rows,
                       out.as_mut_ptr(), out.len())
    })
}

pub fn q6k_q8k_row(weight: &[Q6KBlock], inputs: &[Q8KBlock], rows: usize, out: &mut [f32]) -> anyhow::Result<()> {
    check(unsafe {
        iq_q6k_q8k_row(weight.as_ptr().cast(), weight.len(), inputs.as_ptr().cast(), inputs.len(), rows,
                       out.as_mut_ptr(), out.len())
    })
}

pub fn q80_q80_row(weight: &[Q80Block], inputs: &[Q80Block], rows: usize, out: &mut [f32]) -> anyhow::Result<()> {
    check(unsafe {
        iq_q80_q80_row(weight.as_ptr().cast(), weight.len(), inputs.as_ptr().cast(), inputs.len(), rows,
                       out.as_mut_ptr(), out.len())
    })
}

/// An HBM-resident GGUF matrix (the GPU side of QuantizedMatrix); freed on drop.
pub struct GpuMatrix(pub iq_weight_t);

unsafe impl Send for GpuMatrix {}
unsafe impl Sync for GpuMatrix {}

impl GpuMatrix {
    /// QuantizedMatrix::new (src/gguf.rs:297-320) for the executable dtypes.
    pub fn upload(bytes: &[u8], dtype: c_int, rows: usize, cols: usize) -> anyhow::Result<Self> {
        let mut h: iq_weight_t = std::ptr::null_mut();
        check(unsafe { iq_weights_upload(bytes.as_ptr().cast(), bytes.len(), dtype, rows as i64, cols as i64, &mut h) })?;
        Ok(Self(h))
    }

    /// forward_rows (src/gguf.rs:433-456): host rows in, host rows out.
    pub fn forward_rows(&self, values: &[f32], rows: usize, cols: usize, out_rows: usize) -> anyhow::Result<Vec<f32>> {
        anyhow::ensure!(values.len() == rows * cols, "expected {} input values, got {}", rows * cols, values.len());
        let mut out = vec![0f32; rows * out_rows];
        check(unsafe { iq_matmul_host(self.0, values.as_ptr(), rows as i64, out.as_mut_ptr()) })?;
        Ok(out)
    }

    /// multi_row_forward / fused_forward on device rows (src/gguf.rs:558-690).
    ///
    /// # Safety
    /// `x` and `y` are device pointers of `m * cols` and `m * rows` f32.
    pub unsafe fn forward_device(&self, x: *const f32, m: usize, y: *mut f32, stream: iq_stream_t) -> anyhow::Result<()> {
        check(iq_matmul(self.0, x, m as i64, y, stream))
    }

    /// Size the library workspace of `stream` for up to `m` input rows of
    /// this matrix, so that a graph can capture such calls without an eager
    /// call first.
    pub fn reserve(&self, m: usize, stream: iq_stream_t) -> anyhow::Result<()> {
        check(unsafe { iq_matmul_reserve(self.0, m as i64, stream) })
    }

    /// concatenate_rows (src/gguf.rs:379-404).
    pub fn concatenate_rows(&self, other: &GpuMatrix) -> anyhow::Result<Self> {
        let mut h: iq_weight_t = std::ptr::null_mut();
        check(unsafe { iq_weights_concat_rows(self.0, other.0, &mut h) })?;
        Ok(Self(h))
    }

    /// leading_rows (src/gguf.rs:352-377).
    pub fn leading_rows(&self, rows: usize) -> anyhow::Result<Self> {
        let mut h: iq_weight_t = std::ptr::null_mut();
        check(unsafe { iq_weights_leading_rows(self.0, rows as i64, &mut h) })?;
        Ok(Self(h))
    }
}

impl Drop for GpuMatrix {
    fn drop(&mut self) {
        unsafe {
            iq_weights_free(self.0);
        }
    }
}

/// A GGUF checkpoint parsed by the library (GgufCheckpoint, src/gguf.rs:790-1460).
pub struct Gguf(pub iq_gguf_t);

impl Gguf {
    pub fn open(path: &str) -> anyhow::Result<Self> {
        let c = CString::new(path)?;
        let mut h: iq_gguf_t = std::ptr::null_mut();
        check(unsafe { iq_gguf_open(c.as_ptr(), &mut h) })?;
        Ok(Self(h))
    }

    /// load_matrix (src/gguf.rs:1234).
    pub fn load_matrix(&self, name: &str) -> anyhow::Result<GpuMatrix> {
        let c = CString::new(name)?;
        let mut h: iq_weight_t = std::ptr::null_mut();
        check(unsafe { iq_gguf_load_matrix(self.0, c.as_ptr(), &mut h) })?;
        Ok(GpuMatrix(h))
    }

    /// warm_all_experts with a pinned cache (src/residency.rs:39-131).
    pub fn warm_all_experts(&self, n_layers: usize) -> anyhow::Result<Experts> {
        let mut h: iq_experts_t = std::ptr::null_mut();
        check(unsafe { iq_gguf_load_experts(self.0, n_layers as i64, &mut h) })?;
        Ok(Experts(h))
    }
}

impl Drop for Gguf {
    fn drop(&mut self) {
        unsafe {
            iq_gguf_close(self.0);
        }
    }
}

/// Resident expert tensors of a checkpoint.
pub struct Experts(pub iq_experts_t);

impl Experts {
    /// The routed-expert fields of a layer's descriptor.
    pub fn layer_desc(&self, layer: usize) -> anyhow::Result<iq_moe_desc> {
        let mut d: iq_moe_desc = unsafe { std::mem::zeroed() };
        check(unsafe { iq_experts_layer(self.0, layer as i64, &mut d) })?;
        Ok(d)
    }
}

impl Drop for Experts {
    fn drop(&mut self) {
        unsafe {
            iq_experts_free(self.0);
        }
    }
}

/// One MoE sublayer (QuantizedMoeLayer, src/qwen/quantized_moe.rs:105-460).
pub struct Moe(pub iq_moe_t);

unsafe impl Send for Moe {}

impl Moe {
    pub fn create(desc: &iq_moe_desc) -> anyhow::Result<Self> {
        let mut h: iq_moe_t = std::ptr::null_mut();
        check(unsafe { iq_moe_create(desc, &mut h) })?;
        Ok(Self(h))
    }

    /// Size the workspace for calls of up to `max_tokens` tokens, so that a
    /// graph can capture them without an eager call first.
    pub fn reserve(&self, max_tokens: usize, stream: iq_stream_t) -> anyhow::Result<()> {
        check(unsafe { iq_moe_reserve(self.0, max_tokens as i64, stream) })
    }

    /// Down products of grouped calls in tile order (`IQ_PATH_PREFILL_TILES`,
    /// within 1e-4, not bitwise) or the reference's order (`IQ_PATH_AUTO`).
    pub fn set_path(&self, path: c_int) -> anyhow::Result<()> {
        check(unsafe { iq_moe_set_path(self.0, path) })
    }

    /// forward (src/qwen/quantized_moe.rs:227-281) with the router on the GPU
    /// and the decoder layer's residual add (src/qwen/quantized_layer.rs:212).
    ///
    /// # Safety
    /// Device pointers: `x`, `residual` (or null), `out` of `m * hidden` f32;
    /// `experts` / `weights` of `m * top_k` (or null).
    pub unsafe fn forward_x(&self, x: *const f32, m: usize, residual: *const f32, out: *mut f32, experts: *mut i32,
                            weights: *mut f32, stream: iq_stream_t) -> anyhow::Result<()> {
        check(iq_moe_forward_x(self.0, x, m as i64, residual, out, experts, weights, stream))
    }
}

impl Drop for Moe {
    fn drop(&mut self) {
        unsafe {
            iq_moe_destroy(self.0);
        }
    }
}

/// The library version string.
pub fn version() -> String {
    unsafe { CStr::from_ptr(iq_version()) }.to_string_lossy().into_owned()
}

/// Select and check the device (require_exact_kernels, src/gguf.rs:1043-1053).
pub fn init(device: i32) -> anyhow::Result<()> {
    check(unsafe { iq_init(device) })
}
