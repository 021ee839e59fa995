//! Raw bindings of `libscratchtape_hip.so`, the MI355X (gfx950) library behind scratchtape's
//! matrix-multiplication path. Every struct and function mirrors `include/scratchtape_hip.h` field
//! for field and argument for argument.
//!
//! The entry points replace these reference interfaces, whose Rust signatures stay unchanged and
//! forward here (the wrappers in [`safe`] keep their argument meaning):
//! - `src/gpu_step/matmul.rs:86-106` (`matmul`, `matmul_f32`, `matmul_with`, `MatRef`, `Epilogue`),
//!   and the Linear backward's two independent GEMMs (`src/gpu_step/tape.rs:324-347`) as one
//!   grouped call;
//! - `src/tensor.rs:241` (`NdArray::matmul`);
//! - `src/gpu_step/knn/ivf.rs:466` (`KnnStore::search_ivf`: probe selection and the IVF scan) and
//!   `src/gpu_step/knn.rs:292-299` (`search_tagged` / `search_tail`);
//! - `src/gpu_step/rows.rs:65, 90` (`layer_norm`, `layer_norm_backward`) and the device tape's
//!   softmax and attention.
//!
//! Every call is asynchronous on the given stream (`hipStream_t`, null for the default stream)
//! except `st_ndarray_matmul`, which is synchronous; a status other than `ST_OK` leaves a message
//! for `st_last_error`.
#![allow(non_camel_case_types)]
#![allow(clippy::too_many_arguments)]

use std::ffi::{c_char, c_void, CStr};

pub mod safe;

pub type st_status = i32;
pub const ST_OK: st_status = 0;
/// Bad shape or argument (the reference's assert).
pub const ST_ERR_INVALID: st_status = -1;
/// A HIP runtime call failed.
pub const ST_ERR_HIP: st_status = -2;
/// The scratch arena could not grow.
pub const ST_ERR_OOM: st_status = -3;
/// No gfx950 device visible.
pub const ST_ERR_NO_DEVICE: st_status = -4;

/// Size of the fixed device scratch of `st_matmul_grouped_noalloc`.
pub const ST_NOALLOC_SCRATCH_BYTES: u32 = 64 << 20;

/// `hipStream_t`; null is the default stream.
pub type st_stream = *mut c_void;

/// A matrix inside a device buffer (`MatRef`, `src/gpu_step/matmul.rs:33`): matrix z starts at
/// `off + (z / group) * stride + (z % group) * inner` elements of `p`, its stored rows are `ld`
/// apart (0: packed), and `trans` says it is stored transposed.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct st_matref {
    pub p: *mut f32,
    pub off: i64,
    pub stride: i64,
    pub trans: i32,
    pub reserved: i32,
    pub ld: i64,
    pub group: i64,
    pub inner: i64,
}

/// The GEMM epilogue (`Epilogue`, `src/gpu_step/matmul.rs:63`); null pointers and zero flags are
/// "no epilogue".
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct st_epilogue {
    pub bias: *const f32,
    pub bias_off: i64,
    pub bias_stride: i64,
    pub mask: *const f32,
    pub mask_off: i64,
    pub residual: *const f32,
    pub residual_off: i64,
    pub relu: i32,
    pub accumulate: i32,
    pub has_col_sum: i32,
    pub reserved: i32,
    pub col_sum_off: i64,
    pub col_sum_stride: i64,
}

impl st_epilogue {
    /// The all-zero epilogue: out = a @ b.
    pub const NONE: Self = Self {
        bias: std::ptr::null(),
        bias_off: 0,
        bias_stride: 0,
        mask: std::ptr::null(),
        mask_off: 0,
        residual: std::ptr::null(),
        residual_off: 0,
        relu: 0,
        accumulate: 0,
        has_col_sum: 0,
        reserved: 0,
        col_sum_off: 0,
        col_sum_stride: 0,
    };
}

/// One GEMM of `st_matmul_grouped`: the arguments of `st_matmul_with`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct st_gemm {
    pub a: st_matref,
    pub b: st_matref,
    pub out: st_matref,
    pub epi: st_epilogue,
    pub batch: i64,
    pub m: i64,
    pub k: i64,
    pub n: i64,
    pub use_f16: i32,
    pub reserved: i32,
}

extern "C" {
    /// `matmul` (`src/gpu_step/matmul.rs:86`): out[z] (+)= epilogue(a[z] @ b[z]), the f16 route when
    /// `st_f16_enabled()`.
    pub fn st_matmul(
        a: *const st_matref,
        b: *const st_matref,
        out: *const st_matref,
        batch: i64,
        m: i64,
        k: i64,
        n: i64,
        epi: *const st_epilogue,
        stream: st_stream,
    ) -> st_status;
    /// `matmul_f32` (`src/gpu_step/matmul.rs:93`): always f32.
    pub fn st_matmul_f32(
        a: *const st_matref,
        b: *const st_matref,
        out: *const st_matref,
        batch: i64,
        m: i64,
        k: i64,
        n: i64,
        epi: *const st_epilogue,
        stream: st_stream,
    ) -> st_status;
    /// `matmul_with` (`src/gpu_step/matmul.rs:106`): the f16 route chosen by the caller.
    pub fn st_matmul_with(
        a: *const st_matref,
        b: *const st_matref,
        out: *const st_matref,
        batch: i64,
        m: i64,
        k: i64,
        n: i64,
        epi: *const st_epilogue,
        use_f16: i32,
        stream: st_stream,
    ) -> st_status;
    /// Independent GEMMs the reference issues back to back (`src/gpu_step/tape.rs:324-347`) as one
    /// submission; no GEMM may read or write memory another one writes.
    pub fn st_matmul_grouped(gemms: *const st_gemm, count: i64, stream: st_stream) -> st_status;
    /// `st_matmul_grouped` with its split-k partials in a fixed per-device array of
    /// `ST_NOALLOC_SCRATCH_BYTES`: no device allocation (no reference counterpart; for callers that
    /// cannot allocate, such as code under graph capture).
    pub fn st_matmul_grouped_noalloc(gemms: *const st_gemm, count: i64, stream: st_stream) -> st_status;
    /// `f16_enabled` (`src/gpu_step/matmul.rs:99`): 0 when `TRAIN_F16=0`.
    pub fn st_f16_enabled() -> i32;
    /// `NdArray::matmul` (`src/tensor.rs:241`): host arrays in and out, synchronous.
    pub fn st_ndarray_matmul(a: *const f32, b: *const f32, out: *mut f32, m: i64, k: i64, n: i64) -> st_status;
    pub fn st_softmax(
        x: *const f32,
        y: *mut f32,
        rows: i64,
        n: i64,
        t: i64,
        scale: f32,
        causal: i32,
        one: i32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_softmax_backward(
        dy: *const f32,
        y: *const f32,
        dx: *mut f32,
        rows: i64,
        n: i64,
        scale: f32,
        stream: st_stream,
    ) -> st_status;
    /// `layer_norm` (`src/gpu_step/rows.rs:65`).
    pub fn st_layer_norm(
        x: *const f32,
        rows: i64,
        d: i64,
        params: *const f32,
        off: i64,
        eps: f32,
        models: i64,
        model_stride: i64,
        y: *mut f32,
        mean: *mut f32,
        rstd: *mut f32,
        stream: st_stream,
    ) -> st_status;
    /// `layer_norm_backward` (`src/gpu_step/rows.rs:90`).
    pub fn st_layer_norm_backward(
        dy: *const f32,
        x: *const f32,
        mean: *const f32,
        rstd: *const f32,
        rows: i64,
        d: i64,
        params: *const f32,
        grads: *mut f32,
        off: i64,
        dx: *mut f32,
        accumulate: i32,
        models: i64,
        model_stride: i64,
        stream: st_stream,
    ) -> st_status;
    pub fn st_attention_fused_fwd(
        qkv: *const f32,
        ctx: *mut f32,
        lse: *mut f32,
        b: i64,
        h: i64,
        t: i64,
        hd: i64,
        scale: f32,
        one: i32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_attention_fused_bwd(
        qkv: *const f32,
        ctx: *const f32,
        dctx: *const f32,
        lse: *const f32,
        dqkv: *mut f32,
        b: i64,
        h: i64,
        t: i64,
        hd: i64,
        scale: f32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_knn_quantize_2bit(
        keys: *const f32,
        n: i64,
        d: i64,
        codes: *mut u8,
        scales: *mut f32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_knn_key_norms_2bit(
        codes: *const u8,
        scales: *const f32,
        n: i64,
        d: i64,
        norms: *mut f32,
        stream: st_stream,
    ) -> st_status;
    /// The scored part of `search_ivf` (`src/gpu_step/knn/ivf.rs:466`): every probed cell of every
    /// query, top-k nearest first.
    pub fn st_knn_search_ivf_2bit(
        codes: *const u8,
        scales: *const f32,
        cell_start: *const i64,
        ncells: i64,
        max_cell: i64,
        queries: *const f32,
        probes: *const i32,
        nq: i64,
        nprobe: i64,
        d: i64,
        k: i64,
        out_idx: *mut i64,
        out_dist: *mut f32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_knn_centroid_digit_bytes(nlist: i64, d: i64) -> i64;
    pub fn st_knn_centroids_prep(
        centroids: *const f32,
        nlist: i64,
        d: i64,
        digits: *mut i8,
        cexp: *mut i32,
        cnorm: *mut f64,
        stream: st_stream,
    ) -> st_status;
    /// The probe stage of `search_ivf` (`src/gpu_step/knn/ivf.rs:473-489`).
    pub fn st_knn_probe(
        digits: *const i8,
        cexp: *const i32,
        cnorm: *const f64,
        nlist: i64,
        queries: *const f32,
        nq: i64,
        d: i64,
        nprobe: i64,
        probes: *mut i32,
        stream: st_stream,
    ) -> st_status;
    /// `search_tagged` / `search_tail` (`src/gpu_step/knn.rs:292-331`) over the quantised store.
    pub fn st_knn_set_scan_order(order: i32) -> st_status;
    pub fn st_knn_search_masked_2bit(
        codes: *const u8,
        scales: *const f32,
        nkeys: i64,
        queries: *const f32,
        lohi: *const i64,
        always: i64,
        nq: i64,
        d: i64,
        k: i64,
        out_idx: *mut i64,
        out_dist: *mut f32,
        stream: st_stream,
    ) -> st_status;
    /// Synthetic stores of the reference's seeded generator (benchmark and test support).
    pub fn st_knn_synth_store_2bit(
        seed: u64,
        row0: i64,
        n: i64,
        d: i64,
        codes: *mut u8,
        scales: *mut f32,
        stream: st_stream,
    ) -> st_status;
    pub fn st_knn_synth_keys_f32(seed: u64, row0: i64, n: i64, d: i64, keys: *mut f32, stream: st_stream)
        -> st_status;
    // Device ceilings (benchmark support; no reference counterpart).
    pub fn st_device_info(cus: *mut i32, clock_khz: *mut i32, mem_clock_khz: *mut i32, mem_bus_bits: *mut i32)
        -> st_status;
    pub fn st_peak_mfma(kind: i32, iters: i64, blocks: i32, sink: *mut f32, stream: st_stream) -> st_status;
    pub fn st_peak_read(src: *const c_void, bytes: i64, blocks: i32, sink: *mut f32, stream: st_stream)
        -> st_status;
    pub fn st_lane_selftest(out: *mut u32, stream: st_stream) -> st_status;
    /// The message of the calling thread's last failed call.
    pub fn st_last_error() -> *const c_char;
    /// Synchronises and frees the split-k scratch arena, current and superseded buffers.
    pub fn st_scratch_release() -> st_status;
    pub fn st_sync(stream: st_stream) -> st_status;
    pub fn st_set_wait_limit(polls: i64) -> st_status;
    pub fn st_version() -> *const c_char;
}

/// The reference panics on bad arguments; the library returns a status and keeps the reference's
/// message text, which this raises unchanged.
pub fn check(s: st_status) {
    if s != ST_OK {
        let msg = unsafe { CStr::from_ptr(st_last_error()) }.to_string_lossy().into_owned();
        panic!("{msg}");
    }
}

/// The library's version string.
pub fn version() -> String {
    unsafe { CStr::from_ptr(st_version()) }.to_string_lossy().into_owned()
}
