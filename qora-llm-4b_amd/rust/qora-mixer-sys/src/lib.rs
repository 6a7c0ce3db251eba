//! qora-mixer-sys: the Rust side of the MI355X token-mixer library.
//!
//! `raw` declares every entry point of `include/qora_mixer.h` as it is; the
//! rest is a thin safe layer (a context that is destroyed on drop, device
//! buffers, status codes as `Result`) for the reference's GPU layer-forwards
//! (`gpu_inference.rs:125-130`, `:247-254`, `:436-441`, `:670-677`), which keep
//! their signatures and call the mixer between their projections.  A non-zero
//! status becomes `Err(MixerError)`; the reference's GPU thread turns a panic
//! into `Err(String)` and falls back to the CPU (`gpu_inference.rs:950-975`,
//! `main.rs:141-144`), so a caller may `panic!` on it to keep that path.
//!
//! The build script compiles the gfx950 code objects and `libqora_mixer.so`
//! into `OUT_DIR`; `qm_create` loads the code objects from the library's own
//! directory.
#![allow(non_camel_case_types)]

use std::ffi::CStr;
use std::os::raw::{c_char, c_void};
use std::ptr;

pub mod raw {
    use std::os::raw::{c_char, c_void};

    #[repr(C)]
    pub struct qm_context {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct qm_graph {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct qm_event {
        _p: [u8; 0],
    }
    /// hipStream_t; null is the context's own stream.
    pub type qm_stream = *mut c_void;

    pub const QM_OK: i32 = 0;
    pub const QM_ERR_NO_DEVICE: i32 = 1;
    pub const QM_ERR_CODE_OBJECT: i32 = 2;
    pub const QM_ERR_INVALID_ARG: i32 = 3;
    pub const QM_ERR_SHAPE: i32 = 4;
    pub const QM_ERR_ROPE_RANGE: i32 = 5;
    pub const QM_ERR_CAPACITY: i32 = 6;
    pub const QM_ERR_HIP: i32 = 7;
    pub const QM_ERR_OUT_OF_MEMORY: i32 = 8;
    pub const QM_ERR_WORKSPACE: i32 = 9;

    pub const QM_OPT_DN_DECODE_THREADS: i32 = 1;
    pub const QM_OPT_GQA_DECODE_CHUNK: i32 = 2;
    pub const QM_OPT_GQA_PREFILL_ORDER: i32 = 3;
    pub const QM_F32: i32 = 0;
    pub const QM_F16: i32 = 1;
    pub const QM_BF16: i32 = 2;
    pub const QM_DN_POSTACT: i32 = 0;
    pub const QM_DN_PREACT: i32 = 1;
    pub const QM_SAMPLE_WGPU: i32 = 1;

    /// Qor4bConfig's mixer fields (config.rs:4-32).
    #[repr(C)]
    #[derive(Clone, Copy, Debug, PartialEq, Eq)]
    pub struct qm_config {
        pub num_qk_heads: i32,
        pub num_v_heads: i32,
        pub dn_head_dim: i32,
        pub conv_kernel: i32,
        pub num_heads: i32,
        pub num_kv_heads: i32,
        pub attn_head_dim: i32,
        pub rope_dim: i32,
    }

    /// One output of a multi-weight Q4 GEMV launch.
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct qm_q4_out {
        pub n: i32,
        pub codes_dev: *const u8,
        pub gscales_dev: *const u16,
        pub y_dev: *mut f32,
        pub residual_dev: *const f32,
    }

    /// GenerateParams' sampling settings (generate.rs:9-21) and the decode
    /// loop's per-step choices (generate.rs:185-198).
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct qm_sample_params {
        pub temperature: f32,
        pub top_p: f32,
        pub top_k: i32,
        pub repetition_penalty: f32,
        pub presence_penalty: f32,
        pub banned_id: i32,
        pub flags: i32,
    }

    #[link(name = "qora_mixer")]
    extern "C" {
        // ---- context
        pub fn qm_default_config(cfg: *mut qm_config);
        pub fn qm_create(ctx: *mut *mut qm_context, cfg: *const qm_config, code_object_dir: *const c_char,
                         device: i32) -> i32;
        pub fn qm_destroy(ctx: *mut qm_context) -> i32;
        pub fn qm_status_string(status: i32) -> *const c_char;
        pub fn qm_last_error(ctx: *const qm_context) -> *const c_char;
        pub fn qm_device_count(count: *mut i32) -> i32;
        pub fn qm_reserve(ctx: *mut qm_context, max_batch: i32, max_kv_len: i32, max_prefill_tokens: i32) -> i32;
        pub fn qm_set_option(ctx: *mut qm_context, option: i32, value: i64) -> i32;

        // ---- device memory, streams, events, graphs
        pub fn qm_alloc(ctx: *mut qm_context, bytes: u64, dev: *mut *mut c_void) -> i32;
        pub fn qm_free(ctx: *mut qm_context, dev: *mut c_void) -> i32;
        pub fn qm_memcpy_h2d(ctx: *mut qm_context, dst_dev: *mut c_void, src_host: *const c_void, bytes: u64,
                             stream: qm_stream) -> i32;
        pub fn qm_memcpy_d2h(ctx: *mut qm_context, dst_host: *mut c_void, src_dev: *const c_void, bytes: u64,
                             stream: qm_stream) -> i32;
        pub fn qm_memcpy_d2d(ctx: *mut qm_context, dst_dev: *mut c_void, src_dev: *const c_void, bytes: u64,
                             stream: qm_stream) -> i32;
        pub fn qm_memset(ctx: *mut qm_context, dst_dev: *mut c_void, byte_value: i32, bytes: u64,
                         stream: qm_stream) -> i32;
        pub fn qm_stream_create(ctx: *mut qm_context, stream: *mut qm_stream) -> i32;
        pub fn qm_stream_destroy(ctx: *mut qm_context, stream: qm_stream) -> i32;
        pub fn qm_sync(ctx: *mut qm_context, stream: qm_stream) -> i32;
        pub fn qm_event_create(ctx: *mut qm_context, ev: *mut *mut qm_event) -> i32;
        pub fn qm_event_destroy(ctx: *mut qm_context, ev: *mut qm_event) -> i32;
        pub fn qm_event_record(ctx: *mut qm_context, ev: *mut qm_event, stream: qm_stream) -> i32;
        pub fn qm_event_elapsed_ms(ctx: *mut qm_context, start: *mut qm_event, stop: *mut qm_event,
                                   ms: *mut f32) -> i32;
        pub fn qm_graph_begin(ctx: *mut qm_context, stream: qm_stream) -> i32;
        pub fn qm_graph_end(ctx: *mut qm_context, stream: qm_stream, graph: *mut *mut qm_graph) -> i32;
        pub fn qm_graph_launch(ctx: *mut qm_context, graph: *mut qm_graph, stream: qm_stream) -> i32;
        pub fn qm_graph_destroy(ctx: *mut qm_context, graph: *mut qm_graph) -> i32;

        // ---- host helpers
        pub fn qm_rope_table(theta: f64, rope_dim: i32, max_pos: i32, cos_host: *mut f32,
                             sin_host: *mut f32) -> i32;
        pub fn qm_fill_normal(ctx: *mut qm_context, dst_dev: *mut c_void, dtype: i32, count: u64, mean: f32,
                              std: f32, seed: u64, stream: qm_stream) -> i32;

        // ---- the mixer
        pub fn qm_deltanet_decode(ctx: *mut qm_context, stream: qm_stream, batch: i32, flags: i32,
                                  qkv_dev: *const f32, conv_buf_dev: *mut f32, conv_w_dev: *const f32,
                                  a_dev: *const f32, b_dev: *const f32, a_log_dev: *const f32,
                                  dt_bias_dev: *const f32, z_dev: *const f32, norm_w_dev: *const u16,
                                  state_dev: *mut f32, state_stride: i64, out_dev: *mut f32) -> i32;
        pub fn qm_deltanet_prefill(ctx: *mut qm_context, stream: qm_stream, seq_len: i32, qkv_dev: *const u16,
                                   conv_buf_dev: *mut f32, conv_w_dev: *const f32, a_dev: *const f32,
                                   b_dev: *const f32, a_log_dev: *const f32, dt_bias_dev: *const f32,
                                   z_dev: *const u16, norm_w_dev: *const u16, state_dev: *mut f32,
                                   out_dev: *mut u16) -> i32;
        pub fn qm_gqa_decode(ctx: *mut qm_context, stream: qm_stream, batch: i32, q_gate_dev: *const f32,
                             k_new_dev: *const f32, v_new_dev: *const f32, q_norm_dev: *const u16,
                             k_norm_dev: *const u16, rope_cos_dev: *const f32, rope_sin_dev: *const f32,
                             rope_len: i32, pos_dev: *const i32, max_pos: i32, k_cache_dev: *mut u16,
                             v_cache_dev: *mut u16, cache_capacity: i64, out_dev: *mut f32) -> i32;
        pub fn qm_gqa_decode_noalloc(ctx: *mut qm_context, stream: qm_stream, batch: i32, q_gate_dev: *const f32,
                                     k_new_dev: *const f32, v_new_dev: *const f32, q_norm_dev: *const u16,
                                     k_norm_dev: *const u16, rope_cos_dev: *const f32, rope_sin_dev: *const f32,
                                     rope_len: i32, pos_dev: *const i32, max_pos: i32, k_cache_dev: *mut u16,
                                     v_cache_dev: *mut u16, cache_capacity: i64, out_dev: *mut f32) -> i32;
        pub fn qm_gqa_prefill(ctx: *mut qm_context, stream: qm_stream, seq_len: i32, q_gate_dev: *const u16,
                              k_dev: *const u16, v_dev: *const u16, q_norm_dev: *const u16, k_norm_dev: *const u16,
                              rope_cos_dev: *const f32, rope_sin_dev: *const f32, rope_len: i32,
                              k_cache_dev: *mut u16, v_cache_dev: *mut u16, cache_capacity: i64,
                              out_dev: *mut u16) -> i32;

        // ---- Q4 projections
        pub fn qm_q4_repack(ctx: *mut qm_context, stream: qm_stream, k: i32, n: i32, packed_dev: *const u8,
                            scales_dev: *const u16, codes_dev: *mut u8, gscales_dev: *mut u16) -> i32;
        pub fn qm_q4_gemv(ctx: *mut qm_context, stream: qm_stream, k: i32, n: i32, x_dev: *const f32,
                          codes_dev: *const u8, gscales_dev: *const u16, y_dev: *mut f32) -> i32;
        pub fn qm_q4_gemv_multi(ctx: *mut qm_context, stream: qm_stream, k: i32, x_dev: *const f32,
                                norm_w_dev: *const u16, count: i32, outs: *const qm_q4_out) -> i32;
        pub fn qm_q4_gemv_multi_conv(ctx: *mut qm_context, stream: qm_stream, k: i32, x_dev: *const f32,
                                     norm_w_dev: *const u16, count: i32, outs: *const qm_q4_out,
                                     conv_buf_dev: *mut f32, conv_w_dev: *const f32) -> i32;
        pub fn qm_q4_gate_up(ctx: *mut qm_context, stream: qm_stream, k: i32, n: i32, x_dev: *const f32,
                             norm_w_dev: *const u16, gate_codes_dev: *const u8, gate_gscales_dev: *const u16,
                             up_codes_dev: *const u8, up_gscales_dev: *const u16, out_dev: *mut f32) -> i32;
        pub fn qm_rms_norm_f16(ctx: *mut qm_context, stream: qm_stream, m: i32, k: i32, x_dev: *const f32,
                               norm_w_dev: *const u16, out_dev: *mut u16) -> i32;
        pub fn qm_q4_gemm(ctx: *mut qm_context, stream: qm_stream, m: i32, k: i32, n: i32, x_dev: *const u16,
                          x_dtype: i32, codes_dev: *const u8, gscales_dev: *const u16, residual_dev: *const f32,
                          y_dev: *mut f32, y_bf16_dev: *mut u16) -> i32;
        pub fn qm_q4_gemm_gate_up(ctx: *mut qm_context, stream: qm_stream, m: i32, k: i32, n: i32,
                                  x_dev: *const u16, x_dtype: i32, gate_codes_dev: *const u8,
                                  gate_gscales_dev: *const u16, up_codes_dev: *const u8,
                                  up_gscales_dev: *const u16, out_dev: *mut u16) -> i32;

        // ---- vocabulary side and sampling
        pub fn qm_q4_lm_head(ctx: *mut qm_context, stream: qm_stream, vocab: i32, hidden: i32, x_dev: *const f32,
                             norm_w_dev: *const u16, packed_dev: *const u8, scales_dev: *const u16,
                             logits_dev: *mut f32) -> i32;
        pub fn qm_q4_embed(ctx: *mut qm_context, stream: qm_stream, count: i32, vocab: i32, hidden: i32,
                           ids_dev: *const i32, packed_dev: *const u8, scales_dev: *const u16,
                           out_dev: *mut f32) -> i32;
        pub fn qm_sample(ctx: *mut qm_context, stream: qm_stream, vocab: i32, logits_dev: *mut f32,
                         generated_dev: *const i32, n_generated: i32, params: *const qm_sample_params,
                         rng_state_dev: *mut u64, token_out_dev: *mut i32, top_ids_dev: *mut i32,
                         top_probs_dev: *mut f32) -> i32;
    }
}

pub use raw::{qm_config, qm_q4_out, qm_sample_params, qm_stream};

/// A non-zero status of the library, with its detail message.
#[derive(Debug, Clone)]
pub struct MixerError {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for MixerError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        let name = unsafe { CStr::from_ptr(raw::qm_status_string(self.code)) };
        write!(f, "{}: {}", name.to_string_lossy(), self.message)
    }
}

impl std::error::Error for MixerError {}

pub type Result<T> = std::result::Result<T, MixerError>;

fn message(p: *const c_char) -> String {
    if p.is_null() {
        String::new()
    } else {
        unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
    }
}

/// One mixer context on one device: the loaded code objects, a stream and
/// the workspace.  Not `Sync`: one context per host thread, as the
/// reference calls its layer-forwards from one thread
/// (`gpu_inference.rs:946-948`).
pub struct Context {
    raw: *mut raw::qm_context,
}

impl Context {
    /// `qm_create` with the 4B mixer config, code objects from the
    /// library's directory.
    pub fn new(device: i32) -> Result<Context> {
        let mut h: *mut raw::qm_context = ptr::null_mut();
        let st = unsafe { raw::qm_create(&mut h, ptr::null(), ptr::null(), device) };
        if st != raw::QM_OK {
            return Err(MixerError { code: st, message: message(unsafe { raw::qm_last_error(ptr::null()) }) });
        }
        Ok(Context { raw: h })
    }

    pub fn as_raw(&self) -> *mut raw::qm_context {
        self.raw
    }

    /// Maps a status of a call on this context to `Result`.
    pub fn check(&self, status: i32) -> Result<()> {
        if status == raw::QM_OK {
            Ok(())
        } else {
            Err(MixerError { code: status, message: message(unsafe { raw::qm_last_error(self.raw) }) })
        }
    }

    /// `qm_reserve`: size the workspace once so that no later mixer call
    /// allocates (required before capturing calls into a graph).
    pub fn reserve(&self, max_batch: i32, max_kv_len: i32, max_prefill_tokens: i32) -> Result<()> {
        self.check(unsafe { raw::qm_reserve(self.raw, max_batch, max_kv_len, max_prefill_tokens) })
    }

    pub fn sync(&self, stream: qm_stream) -> Result<()> {
        self.check(unsafe { raw::qm_sync(self.raw, stream) })
    }

    pub fn alloc(&self, bytes: usize) -> Result<DeviceBuffer<'_>> {
        let mut p: *mut c_void = ptr::null_mut();
        self.check(unsafe { raw::qm_alloc(self.raw, bytes as u64, &mut p) })?;
        Ok(DeviceBuffer { ctx: self, ptr: p, bytes })
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe {
            raw::qm_destroy(self.raw);
        }
    }
}

/// A device allocation owned by a context (freed on drop).
pub struct DeviceBuffer<'a> {
    ctx: &'a Context,
    ptr: *mut c_void,
    bytes: usize,
}

impl<'a> DeviceBuffer<'a> {
    pub fn as_ptr<T>(&self) -> *const T {
        self.ptr as *const T
    }
    pub fn as_mut_ptr<T>(&mut self) -> *mut T {
        self.ptr as *mut T
    }
    pub fn len_bytes(&self) -> usize {
        self.bytes
    }
    /// Synchronous host -> device copy of `src` to the start of the buffer.
    pub fn upload<T: Copy>(&mut self, src: &[T]) -> Result<()> {
        let n = std::mem::size_of_val(src);
        assert!(n <= self.bytes, "upload of {} bytes into a {}-byte buffer", n, self.bytes);
        self.ctx.check(unsafe {
            raw::qm_memcpy_h2d(self.ctx.raw, self.ptr, src.as_ptr() as *const c_void, n as u64, ptr::null_mut())
        })
    }
    /// Synchronous device -> host copy of the start of the buffer.
    pub fn download<T: Copy>(&self, dst: &mut [T]) -> Result<()> {
        let n = std::mem::size_of_val(dst);
        assert!(n <= self.bytes, "download of {} bytes from a {}-byte buffer", n, self.bytes);
        self.ctx.check(unsafe {
            raw::qm_memcpy_d2h(self.ctx.raw, dst.as_mut_ptr() as *mut c_void, self.ptr, n as u64, ptr::null_mut())
        })
    }
}

impl<'a> Drop for DeviceBuffer<'a> {
    fn drop(&mut self) {
        unsafe {
            raw::qm_free(self.ctx.raw, self.ptr);
        }
    }
}

/// GpuDeltaNetState (`gpu_inference.rs:30-36`) as device pointers in the
/// reference's layouts: `s` f32 [32][128 v][128 k], `conv_buf` f32 [8192][3].
pub struct DeltaNetStateDev {
    pub s: *mut f32,
    pub conv_buf: *mut f32,
    pub conv_pos: usize,
}

/// GpuKvCacheEntry (`gpu_inference.rs:38-42`) as device pointers: f16
/// [4 kv heads][capacity][256] K and V, `seq_len` positions filled.
pub struct KvCacheDev {
    pub k: *mut u16,
    pub v: *mut u16,
    pub seq_len: usize,
    pub capacity: usize,
}

/// The mixer parameters of a DeltaNet layer (`gpu_loader.rs:37-52`), on the
/// device: conv1d f32 [8192][4], A_log / dt_bias f32 [32], norm f16 [128].
pub struct DeltaNetMixerDev {
    pub conv1d_weight: *const f32,
    pub a_log: *const f32,
    pub dt_bias: *const f32,
    pub attn_norm_weight: *const u16,
}

/// The mixer parameters of an attention layer (`gpu_loader.rs:54-66`): the
/// q / k RMSNorm weights, f16 [256], (1 + gamma).
pub struct AttnMixerDev {
    pub q_norm: *const u16,
    pub k_norm: *const u16,
}

/// A length or position that does not fit the C ABI's 32-bit integers
/// becomes an error instead of wrapping.
fn to_i32(what: &str, v: usize) -> Result<i32> {
    i32::try_from(v).map_err(|_| MixerError {
        code: raw::QM_ERR_INVALID_ARG,
        message: format!("{} = {} does not fit in a 32-bit signed integer", what, v),
    })
}

fn to_i64(what: &str, v: usize) -> Result<i64> {
    i64::try_from(v).map_err(|_| MixerError {
        code: raw::QM_ERR_INVALID_ARG,
        message: format!("{} = {} does not fit in a 64-bit signed integer", what, v),
    })
}

/// Mixer slice of `forward_deltanet_decode_gpu` (`gpu_inference.rs:149-227`):
/// `qkv` is the raw in_proj_qkv output (conv1d + SiLU run here and the conv
/// buffer shifts), `a`, `b`, `z` the other input projections; `out` [4096]
/// receives the gated output, the out_proj input.  One sequence.
///
/// # Safety
/// Every pointer (the arguments and the fields of `layer` and `state`) must
/// be a device address of this context's GPU, 16-byte aligned, valid for the
/// whole launch and sized as stated: `qkv` f32 [8192], `a` / `b` f32 [32],
/// `z` f32 [4096], `out` f32 [4096], `state.s` f32 [32][128][128],
/// `state.conv_buf` f32 [8192][3], and the layer parameters as
/// `DeltaNetMixerDev` documents.  The kernels read and write through them
/// without further checks; the library only rejects null and misaligned
/// pointers.
pub unsafe fn deltanet_decode(ctx: &Context, stream: qm_stream, qkv: *const f32, a: *const f32, b: *const f32,
                              z: *const f32, layer: &DeltaNetMixerDev, state: &mut DeltaNetStateDev,
                              out: *mut f32) -> Result<()> {
    ctx.check(raw::qm_deltanet_decode(ctx.raw, stream, 1, raw::QM_DN_PREACT, qkv, state.conv_buf,
                                      layer.conv1d_weight, a, b, layer.a_log, layer.dt_bias, z,
                                      layer.attn_norm_weight, state.s, 32 * 128 * 128, out))?;
    state.conv_pos += 1;
    Ok(())
}

/// Mixer slice of `forward_attn_decode_gpu` (`gpu_inference.rs:271-349`):
/// q/gate interleaved per head [16][512], k and v [4][256] of the new
/// token; appends at `kv.seq_len` and advances it (`gemv.rs:952-956`).
///
/// # Safety
/// Every pointer must be a device address of this context's GPU, 16-byte
/// aligned and valid for the launch: `q_gate` f32 [16][512], `k_new` /
/// `v_new` f32 [4][256], `out` f32 [16][256], `rope_cos` / `rope_sin` f32
/// [rope_len][32], `layer`'s norms f16 [256], and `kv.k` / `kv.v` f16
/// [4][kv.capacity][256].  The library checks `kv.seq_len < kv.capacity`
/// and `kv.seq_len < rope_len`, not the sizes behind the pointers.
pub unsafe fn attn_decode(ctx: &Context, stream: qm_stream, q_gate: *const f32, k_new: *const f32,
                          v_new: *const f32, layer: &AttnMixerDev, kv: &mut KvCacheDev, rope_cos: *const f32,
                          rope_sin: *const f32, rope_len: usize, out: *mut f32) -> Result<()> {
    let pos = to_i32("kv.seq_len", kv.seq_len)?;
    let cap = to_i64("kv.capacity", kv.capacity)?;
    let rl = to_i32("rope_len", rope_len)?;
    ctx.check(raw::qm_gqa_decode(ctx.raw, stream, 1, q_gate, k_new, v_new, layer.q_norm, layer.k_norm, rope_cos,
                                 rope_sin, rl, ptr::null(), pos, kv.k, kv.v, cap, out))?;
    kv.seq_len += 1;
    Ok(())
}

/// Mixer slice of `prefill_deltanet_layer_gpu` (`gpu_inference.rs:465-603`):
/// `seq_len` tokens of bf16 in_proj_qkv / in_proj_z outputs, f32 a / b, in
/// chunks of 64; the state and conv buffer continue from where they are;
/// `out` bf16 [seq_len][4096].
///
/// # Safety
/// Every pointer must be a device address of this context's GPU, 16-byte
/// aligned and valid for the launch: `qkv_bf16` [seq_len][8192], `a` / `b`
/// f32 [seq_len][32], `z_bf16` [seq_len][4096], `out_bf16` [seq_len][4096],
/// and `state` / `layer` as for `deltanet_decode`.
pub unsafe fn deltanet_prefill(ctx: &Context, stream: qm_stream, seq_len: usize, qkv_bf16: *const u16,
                               a: *const f32, b: *const f32, z_bf16: *const u16, layer: &DeltaNetMixerDev,
                               state: &mut DeltaNetStateDev, out_bf16: *mut u16) -> Result<()> {
    let t = to_i32("seq_len", seq_len)?;
    ctx.check(raw::qm_deltanet_prefill(ctx.raw, stream, t, qkv_bf16, state.conv_buf, layer.conv1d_weight, a, b,
                                       layer.a_log, layer.dt_bias, z_bf16, layer.attn_norm_weight, state.s,
                                       out_bf16))?;
    state.conv_pos += seq_len;
    Ok(())
}

/// Mixer slice of `prefill_attn_layer_gpu` (`gpu_inference.rs:679-766`): the
/// cache is replaced by positions 0 .. seq_len-1 (`gemv.rs:1397-1400`).
///
/// # Safety
/// Every pointer must be a device address of this context's GPU, 16-byte
/// aligned and valid for the launch: `q_gate_bf16` [seq_len][16][512],
/// `k_bf16` / `v_bf16` [seq_len][4][256], `out_bf16` [seq_len][16][256],
/// `rope_cos` / `rope_sin` f32 [rope_len][32], `layer`'s norms f16 [256],
/// and `kv.k` / `kv.v` f16 [4][kv.capacity][256].  The library checks
/// `seq_len <= kv.capacity` and `seq_len <= rope_len`, not the sizes behind
/// the pointers.
pub unsafe fn attn_prefill(ctx: &Context, stream: qm_stream, seq_len: usize, q_gate_bf16: *const u16,
                           k_bf16: *const u16, v_bf16: *const u16, layer: &AttnMixerDev, kv: &mut KvCacheDev,
                           rope_cos: *const f32, rope_sin: *const f32, rope_len: usize, out_bf16: *mut u16)
                           -> Result<()> {
    let t = to_i32("seq_len", seq_len)?;
    let cap = to_i64("kv.capacity", kv.capacity)?;
    let rl = to_i32("rope_len", rope_len)?;
    ctx.check(raw::qm_gqa_prefill(ctx.raw, stream, t, q_gate_bf16, k_bf16, v_bf16, layer.q_norm, layer.k_norm,
                                  rope_cos, rope_sin, rl, kv.k, kv.v, cap, out_bf16))?;
    kv.seq_len = seq_len;
    Ok(())
}

/// RoPE tables [max_pos][32] with the formula of `convert.rs:161-176`.
pub fn rope_table(max_pos: usize) -> Result<(Vec<f32>, Vec<f32>)> {
    let n = to_i32("max_pos", max_pos)?;
    let mut cos = vec![0.0f32; max_pos * 32];
    let mut sin = vec![0.0f32; max_pos * 32];
    let st = unsafe { raw::qm_rope_table(1.0e7, 64, n, cos.as_mut_ptr(), sin.as_mut_ptr()) };
    if st != raw::QM_OK {
        return Err(MixerError { code: st, message: "qm_rope_table".to_string() });
    }
    Ok((cos, sin))
}
