//! Wrappers with the reference's argument meaning, for the bodies of the reference's unchanged
//! signatures (`src/gpu_step/matmul.rs:86-106`, `src/tensor.rs:241`, `src/gpu_step/rows.rs:65, 90`,
//! `src/gpu_step/knn/ivf.rs:466`).
//!
//! - Device buffers name their address and byte length through [`DeviceBuffer`], an `unsafe`
//!   trait: an implementor promises that the range is device memory that stays valid while the
//!   work enqueued on it runs. The runtime's buffer handle implements it (the role of
//!   `cubecl::server::Handle` in `src/gpu_step/mod.rs:139-151`); [`DevicePtr`] wraps a bare
//!   address and length, and building one is `unsafe` for the same reason.
//! - Every safe wrapper checks, before the call, that each buffer holds every element the call
//!   reads or writes for the shapes given (and panics, as the reference's asserts do, if one does
//!   not), so a safe call never reaches outside its buffers. Calls whose extents depend on data in
//!   device memory (the cell table of [`knn_search_ivf_2bit`]), or that free or share memory
//!   behind the caller's back ([`scratch_release`], [`matmul_grouped_noalloc`]), are `unsafe fn`.
//! - Every call goes on the calling thread's stream, [`stream`] (the default stream unless
//!   [`set_stream`] chose another), as the reference puts every launch on its one queue.
//! - A failed status panics with the library's message, as the reference's asserts do.
use std::cell::Cell;
use std::ffi::c_void;

pub use crate::check;
use crate as sys;
use crate::st_stream;

/// Device memory that can name its device address and length.
///
/// # Safety
/// `device_ptr() .. device_ptr() + byte_len()` must be device memory of the current device that
/// stays allocated, and is not used by anything else the call does not know of, until the work
/// enqueued on it has finished.
pub unsafe trait DeviceBuffer {
    fn device_ptr(&self) -> *mut c_void;
    fn byte_len(&self) -> usize;
}

/// A bare device range (a `hipMalloc` result, or a torch tensor's `data_ptr()` and byte size).
#[derive(Clone, Copy, Debug)]
pub struct DevicePtr {
    ptr: *mut c_void,
    bytes: usize,
}

impl DevicePtr {
    /// # Safety
    /// `ptr .. ptr + bytes` must be device memory meeting [`DeviceBuffer`]'s contract.
    pub unsafe fn new(ptr: *mut c_void, bytes: usize) -> Self {
        Self { ptr, bytes }
    }
}

unsafe impl DeviceBuffer for DevicePtr {
    fn device_ptr(&self) -> *mut c_void {
        self.ptr
    }
    fn byte_len(&self) -> usize {
        self.bytes
    }
}

/// The device address of a buffer.
pub fn handle_ptr<H: DeviceBuffer + ?Sized>(h: &H) -> *mut c_void {
    h.device_ptr()
}

/// A buffer's device address as a mutable element pointer.
pub fn dptr<T, H: DeviceBuffer + ?Sized>(h: &H) -> *mut T {
    h.device_ptr() as *mut T
}

/// A buffer's device address as a read-only element pointer.
pub fn ptr<T, H: DeviceBuffer + ?Sized>(h: &H) -> *const T {
    h.device_ptr() as *const T
}

/// Panics unless `h` holds `count` elements of `T` (`count` counts from the buffer's start).
fn need<T, H: DeviceBuffer + ?Sized>(h: &H, count: usize, what: &str) {
    let bytes = count.checked_mul(std::mem::size_of::<T>());
    match bytes {
        Some(b) if b <= h.byte_len() => {}
        _ => panic!("{}: the buffer holds {} bytes, the call reaches {} elements of {} bytes", what,
                    h.byte_len(), count, std::mem::size_of::<T>()),
    }
}

fn mul(a: usize, b: usize) -> usize {
    a.checked_mul(b).expect("extent overflows usize")
}

fn add(a: usize, b: usize) -> usize {
    a.checked_add(b).expect("extent overflows usize")
}

thread_local! {
    static STREAM: Cell<st_stream> = Cell::new(std::ptr::null_mut());
}

/// Puts the calling thread's later calls on `s` (a `hipStream_t`; null for the default stream).
pub fn set_stream(s: st_stream) {
    STREAM.with(|c| c.set(s));
}

/// The calling thread's stream.
pub fn stream() -> st_stream {
    STREAM.with(|c| c.get())
}

/// `MatRef` (`src/gpu_step/matmul.rs:33-43`): matrix z of a batch starts at element
/// off + (z / group)·stride + (z % group)·inner of `h`, its stored rows are `ld` apart (0: packed),
/// and `trans` says it is stored transposed.
pub struct MatRef<'a, H: DeviceBuffer + ?Sized> {
    pub h: &'a H,
    pub off: usize,
    pub stride: usize,
    pub trans: bool,
    pub ld: usize,
    pub group: usize,
    pub inner: usize,
}

impl<'a, H: DeviceBuffer + ?Sized> Clone for MatRef<'a, H> {
    fn clone(&self) -> Self {
        *self
    }
}

impl<'a, H: DeviceBuffer + ?Sized> Copy for MatRef<'a, H> {}

impl<'a, H: DeviceBuffer + ?Sized> MatRef<'a, H> {
    /// The whole buffer from 0, one batch, not transposed (`MatRef::new`, `matmul.rs:45-48`).
    pub fn new(h: &'a H) -> Self {
        Self { h, off: 0, stride: 0, trans: false, ld: 0, group: 1, inner: 0 }
    }

    /// Attention heads in place (`MatRef::heads`, `matmul.rs:50-56`): matrix z = b·heads + h is rows
    /// b·t .. b·t + t, columns col0 + h·width .. + width, of a row-major [B·t, cols] buffer.
    pub fn heads(h: &'a H, col0: usize, cols: usize, t: usize, heads: usize, width: usize) -> Self {
        Self { off: col0, stride: t * cols, ld: cols, group: heads, inner: width, ..Self::new(h) }
    }

    /// One past the last element of `h` that `batch` logical [rows, cols] matrices reach.
    pub fn end(&self, batch: usize, rows: usize, cols: usize) -> usize {
        if batch == 0 || rows == 0 || cols == 0 {
            return self.off;
        }
        let (sr, sc) = if self.trans { (cols, rows) } else { (rows, cols) };
        let ld = if self.ld == 0 { sc } else { self.ld };
        let group = self.group.max(1);
        let mut zmax = 0usize;
        for z in 0..batch {
            zmax = zmax.max(add(mul(z / group, self.stride), mul(z % group, self.inner)));
        }
        add(add(self.off, zmax), add(mul(sr - 1, ld), sc))
    }

    pub fn raw(&self) -> sys::st_matref {
        sys::st_matref {
            p: dptr::<f32, H>(self.h),
            off: self.off as i64,
            stride: self.stride as i64,
            trans: self.trans as i32,
            reserved: 0,
            ld: self.ld as i64,
            group: self.group as i64,
            inner: self.inner as i64,
        }
    }
}

/// `Epilogue` (`src/gpu_step/matmul.rs:58-80`), applied in this order: + bias[col] (matrix z's bias
/// `bias_stride`·z further on), ReLU, zero where `mask` is not positive, + residual, + the value
/// already in out; `col_sum` = Some((off, stride)) also adds the column sums of b[z] into out's
/// buffer at off + z·stride + j.
pub struct Epilogue<'a, H: DeviceBuffer + ?Sized> {
    pub bias: Option<(&'a H, usize)>,
    pub bias_stride: usize,
    pub relu: bool,
    pub mask: Option<(&'a H, usize)>,
    pub residual: Option<(&'a H, usize)>,
    pub accumulate: bool,
    pub col_sum: Option<(usize, usize)>,
}

impl<'a, H: DeviceBuffer + ?Sized> Clone for Epilogue<'a, H> {
    fn clone(&self) -> Self {
        *self
    }
}

impl<'a, H: DeviceBuffer + ?Sized> Copy for Epilogue<'a, H> {}

impl<'a, H: DeviceBuffer + ?Sized> Default for Epilogue<'a, H> {
    fn default() -> Self {
        Self { bias: None, bias_stride: 0, relu: false, mask: None, residual: None, accumulate: false, col_sum: None }
    }
}

fn operand<H: DeviceBuffer + ?Sized>(o: Option<(&H, usize)>) -> (*const f32, i64) {
    match o {
        Some((h, off)) => (ptr::<f32, H>(h), off as i64),
        None => (std::ptr::null(), 0),
    }
}

impl<'a, H: DeviceBuffer + ?Sized> Epilogue<'a, H> {
    pub fn raw(&self) -> sys::st_epilogue {
        let (bias, bias_off) = operand(self.bias);
        let (mask, mask_off) = operand(self.mask);
        let (residual, residual_off) = operand(self.residual);
        let (has_col_sum, col_sum_off, col_sum_stride) = match self.col_sum {
            Some((off, stride)) => (1, off as i64, stride as i64),
            None => (0, 0, 0),
        };
        sys::st_epilogue {
            bias,
            bias_off,
            bias_stride: self.bias_stride as i64,
            mask,
            mask_off,
            residual,
            residual_off,
            relu: self.relu as i32,
            accumulate: self.accumulate as i32,
            has_col_sum,
            reserved: 0,
            col_sum_off,
            col_sum_stride,
        }
    }
}

/// Panics unless every buffer of a GEMM holds what the call reads and writes: a [m, k], b [k, n]
/// and out [m, n] per batch matrix through their `MatRef`s, bias `bias_stride`·z + n per matrix,
/// mask and residual laid out as out, and the column sums at off + z·stride + n of out's buffer.
fn check_gemm<H: DeviceBuffer + ?Sized>(
    a: &MatRef<'_, H>,
    b: &MatRef<'_, H>,
    out: &MatRef<'_, H>,
    batch: usize,
    m: usize,
    k: usize,
    n: usize,
    epi: &Epilogue<'_, H>,
) {
    if batch == 0 || m == 0 || n == 0 {
        return;
    }
    need::<f32, H>(a.h, a.end(batch, m, k), "matmul a");
    need::<f32, H>(b.h, b.end(batch, k, n), "matmul b");
    let out_end = out.end(batch, m, n);
    need::<f32, H>(out.h, out_end, "matmul out");
    if let Some((h, off)) = epi.bias {
        need::<f32, H>(h, add(off, add(mul(batch - 1, epi.bias_stride), n)), "matmul bias");
    }
    for (o, what) in [(epi.mask, "matmul mask"), (epi.residual, "matmul residual")] {
        if let Some((h, off)) = o {
            need::<f32, H>(h, add(off, out_end - out.off), what);
        }
    }
    if let Some((off, stride)) = epi.col_sum {
        need::<f32, H>(out.h, add(off, add(mul(batch - 1, stride), n)), "matmul col_sum");
    }
}

/// `matmul` (`src/gpu_step/matmul.rs:86`): out[z] (+)= epilogue(a[z] @ b[z]) for z in 0..batch, a[z]
/// logically [m, k], b[z] [k, n], out[z] row-major [m, n]; the f16 route when [`f16_enabled`].
pub fn matmul<H: DeviceBuffer + ?Sized>(
    a: MatRef<'_, H>,
    b: MatRef<'_, H>,
    out: MatRef<'_, H>,
    batch: usize,
    m: usize,
    k: usize,
    n: usize,
    epi: Epilogue<'_, H>,
) {
    check_gemm(&a, &b, &out, batch, m, k, n, &epi);
    let (a, b, o, e) = (a.raw(), b.raw(), out.raw(), epi.raw());
    check(unsafe { sys::st_matmul(&a, &b, &o, batch as i64, m as i64, k as i64, n as i64, &e, stream()) });
}

/// `matmul_f32` (`src/gpu_step/matmul.rs:93`): `matmul` always in f32.
pub fn matmul_f32<H: DeviceBuffer + ?Sized>(
    a: MatRef<'_, H>,
    b: MatRef<'_, H>,
    out: MatRef<'_, H>,
    batch: usize,
    m: usize,
    k: usize,
    n: usize,
    epi: Epilogue<'_, H>,
) {
    check_gemm(&a, &b, &out, batch, m, k, n, &epi);
    let (a, b, o, e) = (a.raw(), b.raw(), out.raw(), epi.raw());
    check(unsafe { sys::st_matmul_f32(&a, &b, &o, batch as i64, m as i64, k as i64, n as i64, &e, stream()) });
}

/// `matmul_with` (`src/gpu_step/matmul.rs:106`): the f16 route chosen by the caller (shapes it
/// cannot tile still run in f32).
pub fn matmul_with<H: DeviceBuffer + ?Sized>(
    a: MatRef<'_, H>,
    b: MatRef<'_, H>,
    out: MatRef<'_, H>,
    batch: usize,
    m: usize,
    k: usize,
    n: usize,
    epi: Epilogue<'_, H>,
    use_f16: bool,
) {
    check_gemm(&a, &b, &out, batch, m, k, n, &epi);
    let (a, b, o, e) = (a.raw(), b.raw(), out.raw(), epi.raw());
    check(unsafe {
        sys::st_matmul_with(&a, &b, &o, batch as i64, m as i64, k as i64, n as i64, &e, use_f16 as i32, stream())
    });
}

/// `f16_enabled` (`src/gpu_step/matmul.rs:99`): false when `TRAIN_F16=0`.
pub fn f16_enabled() -> bool {
    unsafe { sys::st_f16_enabled() != 0 }
}

/// One GEMM of [`matmul_grouped`]: the arguments of [`matmul_with`].
pub struct Gemm<'a, H: DeviceBuffer + ?Sized> {
    pub a: MatRef<'a, H>,
    pub b: MatRef<'a, H>,
    pub out: MatRef<'a, H>,
    pub batch: usize,
    pub m: usize,
    pub k: usize,
    pub n: usize,
    pub epi: Epilogue<'a, H>,
    pub use_f16: bool,
}

impl<'a, H: DeviceBuffer + ?Sized> Gemm<'a, H> {
    pub fn raw(&self) -> sys::st_gemm {
        sys::st_gemm {
            a: self.a.raw(),
            b: self.b.raw(),
            out: self.out.raw(),
            epi: self.epi.raw(),
            batch: self.batch as i64,
            m: self.m as i64,
            k: self.k as i64,
            n: self.n as i64,
            use_f16: self.use_f16 as i32,
            reserved: 0,
        }
    }
}

/// GEMMs the reference issues back to back that do not depend on each other (a Linear backward's
/// dW and dx, `src/gpu_step/tape.rs:324-347`) as one submission. No GEMM of the group may read or
/// write memory that another one writes.
pub fn matmul_grouped<H: DeviceBuffer + ?Sized>(gemms: &[Gemm<'_, H>]) {
    for g in gemms {
        check_gemm(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n, &g.epi);
    }
    let raw: Vec<sys::st_gemm> = gemms.iter().map(|g| g.raw()).collect();
    check(unsafe { sys::st_matmul_grouped(raw.as_ptr(), raw.len() as i64, stream()) });
}

/// [`matmul_grouped`] without device allocation: split-k partials live in the library's fixed
/// per-device array (`ST_NOALLOC_SCRATCH_BYTES`); a group needing more panics before anything is
/// launched.
///
/// # Safety
/// Every call on a device shares that device's array: no other call of this function may run on
/// the same device (on another stream or thread) until this one's work has finished.
pub unsafe fn matmul_grouped_noalloc<H: DeviceBuffer + ?Sized>(gemms: &[Gemm<'_, H>]) {
    for g in gemms {
        check_gemm(&g.a, &g.b, &g.out, g.batch, g.m, g.k, g.n, &g.epi);
    }
    let raw: Vec<sys::st_gemm> = gemms.iter().map(|g| g.raw()).collect();
    check(unsafe { sys::st_matmul_grouped_noalloc(raw.as_ptr(), raw.len() as i64, stream()) });
}

/// The body of `NdArray::matmul` (`src/tensor.rs:241-253`): row-major host arrays `a` [m, k] and
/// `b` [k, n] given with their shapes, the product [m, n] returned. Synchronous.
pub fn ndarray_matmul(a: &[f32], a_shape: &[usize], b: &[f32], b_shape: &[usize]) -> Vec<f32> {
    assert_eq!(a_shape.len(), 2, "matmul lhs must be 2D, got {:?}", a_shape);
    assert_eq!(b_shape.len(), 2, "matmul rhs must be 2D, got {:?}", b_shape);
    let (m, k) = (a_shape[0], a_shape[1]);
    let (k2, n) = (b_shape[0], b_shape[1]);
    assert_eq!(k, k2, "matmul inner dims must match: {:?} vs {:?}", a_shape, b_shape);
    assert_eq!(a.len(), m * k, "lhs data does not match its shape {:?}", a_shape);
    assert_eq!(b.len(), k * n, "rhs data does not match its shape {:?}", b_shape);
    let mut out = vec![0.0f32; m * n];
    check(unsafe { sys::st_ndarray_matmul(a.as_ptr(), b.as_ptr(), out.as_mut_ptr(), m as i64, k as i64, n as i64) });
    out
}

/// `Models` (`src/gpu_step/mod.rs:119-126`): `k` models whose parameters sit `stride` apart.
#[derive(Clone, Copy, Debug)]
pub struct Models {
    pub k: usize,
    pub stride: usize,
}

impl Models {
    pub const ONE: Self = Self { k: 1, stride: 0 };
}

/// `LnOut` (`src/gpu_step/rows.rs:54-58`): the forward's y [rows, d], mean and rstd [rows], in
/// buffers the caller owns.
pub struct LnOut<'a, H: DeviceBuffer + ?Sized> {
    pub y: &'a H,
    pub mean: &'a H,
    pub rstd: &'a H,
}

/// `layer_norm` (`src/gpu_step/rows.rs:65`): y = (x - mean) / sqrt(var + eps) · gamma + beta per
/// row of x [rows, d], gamma and beta at `params[off..]` of each model.
pub fn layer_norm<H: DeviceBuffer + ?Sized>(
    x: &H,
    rows: usize,
    d: usize,
    params: &H,
    off: usize,
    eps: f32,
    m: Models,
    out: &LnOut<'_, H>,
) {
    let params_end = add(add(off, mul(m.k.max(1) - 1, m.stride)), mul(2, d));
    need::<f32, H>(x, mul(rows, d), "layer_norm x");
    need::<f32, H>(params, params_end, "layer_norm params");
    need::<f32, H>(out.y, mul(rows, d), "layer_norm y");
    need::<f32, H>(out.mean, rows, "layer_norm mean");
    need::<f32, H>(out.rstd, rows, "layer_norm rstd");
    check(unsafe {
        sys::st_layer_norm(
            ptr(x),
            rows as i64,
            d as i64,
            ptr(params),
            off as i64,
            eps,
            m.k as i64,
            m.stride as i64,
            dptr(out.y),
            dptr(out.mean),
            dptr(out.rstd),
            stream(),
        )
    });
}

/// `layer_norm_backward` (`src/gpu_step/rows.rs:90`): dx (+)= the input gradient, and the gamma
/// and beta gradients added into `grads[off..]` of each model.
pub fn layer_norm_backward<H: DeviceBuffer + ?Sized>(
    dy: &H,
    x: &H,
    fwd: &LnOut<'_, H>,
    rows: usize,
    d: usize,
    params: &H,
    grads: &H,
    off: usize,
    dx: &H,
    accumulate: bool,
    m: Models,
) {
    let params_end = add(add(off, mul(m.k.max(1) - 1, m.stride)), mul(2, d));
    for (h, what) in [(dy, "layer_norm_backward dy"), (x, "layer_norm_backward x"), (dx, "layer_norm_backward dx")] {
        need::<f32, H>(h, mul(rows, d), what);
    }
    need::<f32, H>(fwd.mean, rows, "layer_norm_backward mean");
    need::<f32, H>(fwd.rstd, rows, "layer_norm_backward rstd");
    need::<f32, H>(params, params_end, "layer_norm_backward params");
    need::<f32, H>(grads, params_end, "layer_norm_backward grads");
    check(unsafe {
        sys::st_layer_norm_backward(
            ptr(dy),
            ptr(x),
            ptr(fwd.mean),
            ptr(fwd.rstd),
            rows as i64,
            d as i64,
            ptr(params),
            dptr(grads),
            off as i64,
            dptr(dx),
            accumulate as i32,
            m.k as i64,
            m.stride as i64,
            stream(),
        )
    });
}

/// `softmax` (`src/gpu_step/rows.rs:101-112`): y = softmax(scale · x) per row of x [rows, n]; with
/// `causal`, row r sees columns 0..=r % t and the rest are 0; `one` is softmax1 (a phantom logit 0).
pub fn softmax<H: DeviceBuffer + ?Sized>(x: &H, y: &H, rows: usize, n: usize, t: usize, scale: f32, causal: bool, one: bool) {
    need::<f32, H>(x, mul(rows, n), "softmax x");
    need::<f32, H>(y, mul(rows, n), "softmax y");
    check(unsafe {
        sys::st_softmax(ptr(x), dptr(y), rows as i64, n as i64, t as i64, scale, causal as i32, one as i32, stream())
    });
}

/// `softmax_backward` (`src/gpu_step/rows.rs:114-123`): dx = scale · y · (dy - sum(dy · y)).
pub fn softmax_backward<H: DeviceBuffer + ?Sized>(dy: &H, y: &H, dx: &H, rows: usize, n: usize, scale: f32) {
    for (h, what) in [(dy, "softmax_backward dy"), (y, "softmax_backward y"), (dx, "softmax_backward dx")] {
        need::<f32, H>(h, mul(rows, n), what);
    }
    check(unsafe { sys::st_softmax_backward(ptr(dy), ptr(y), dptr(dx), rows as i64, n as i64, scale, stream()) });
}

/// Fused causal attention forward over a packed [B·T, 3·H·hd] QKV buffer: ctx [B·T, H·hd] and the
/// row log-sum-exp lse [B·H·T] the backward needs.
pub fn attention_fused_fwd<H: DeviceBuffer + ?Sized>(
    qkv: &H,
    ctx: &H,
    lse: &H,
    b: usize,
    h: usize,
    t: usize,
    hd: usize,
    scale: f32,
    one: bool,
) {
    let ctx_len = mul(mul(mul(b, t), h), hd);
    need::<f32, H>(qkv, mul(3, ctx_len), "attention qkv");
    need::<f32, H>(ctx, ctx_len, "attention ctx");
    need::<f32, H>(lse, mul(mul(b, h), t), "attention lse");
    check(unsafe {
        sys::st_attention_fused_fwd(
            ptr(qkv),
            dptr(ctx),
            dptr(lse),
            b as i64,
            h as i64,
            t as i64,
            hd as i64,
            scale,
            one as i32,
            stream(),
        )
    });
}

/// Fused causal attention backward: dqkv from qkv, ctx, dctx and the forward's lse.
pub fn attention_fused_bwd<H: DeviceBuffer + ?Sized>(
    qkv: &H,
    ctx: &H,
    dctx: &H,
    lse: &H,
    dqkv: &H,
    b: usize,
    h: usize,
    t: usize,
    hd: usize,
    scale: f32,
) {
    let ctx_len = mul(mul(mul(b, t), h), hd);
    need::<f32, H>(qkv, mul(3, ctx_len), "attention qkv");
    need::<f32, H>(dqkv, mul(3, ctx_len), "attention dqkv");
    need::<f32, H>(ctx, ctx_len, "attention ctx");
    need::<f32, H>(dctx, ctx_len, "attention dctx");
    need::<f32, H>(lse, mul(mul(b, h), t), "attention lse");
    check(unsafe {
        sys::st_attention_fused_bwd(
            ptr(qkv),
            ptr(ctx),
            ptr(dctx),
            ptr(lse),
            dptr(dqkv),
            b as i64,
            h as i64,
            t as i64,
            hd as i64,
            scale,
            stream(),
        )
    });
}

/// Quantises f32 keys [n, d] to the store's 2-bit codes and per-key scales.
pub fn knn_quantize_2bit<H: DeviceBuffer + ?Sized>(keys: &H, n: usize, d: usize, codes: &H, scales: &H) {
    need::<f32, H>(keys, mul(n, d), "knn_quantize_2bit keys");
    need::<u8, H>(codes, mul(n, d) / 4, "knn_quantize_2bit codes");
    need::<f32, H>(scales, n, "knn_quantize_2bit scales");
    check(unsafe { sys::st_knn_quantize_2bit(ptr(keys), n as i64, d as i64, dptr(codes), dptr(scales), stream()) });
}

/// Per-key squared norms of the dequantised 2-bit keys (what the store file keeps per tile).
pub fn knn_key_norms_2bit<H: DeviceBuffer + ?Sized>(codes: &H, scales: &H, n: usize, d: usize, norms: &H) {
    need::<u8, H>(codes, mul(n, d) / 4, "knn_key_norms_2bit codes");
    need::<f32, H>(scales, n, "knn_key_norms_2bit scales");
    need::<f32, H>(norms, n, "knn_key_norms_2bit norms");
    check(unsafe { sys::st_knn_key_norms_2bit(ptr(codes), ptr(scales), n as i64, d as i64, dptr(norms), stream()) });
}

/// Bytes of the centroid digit blocks [`knn_centroids_prep`] writes; panics, as the reference's
/// assert does, for a dimension probe selection is not built for.
pub fn knn_centroid_digit_bytes(nlist: usize, d: usize) -> usize {
    let n = unsafe { sys::st_knn_centroid_digit_bytes(nlist as i64, d as i64) };
    assert!(n > 0, "probe selection is built for d == 256");
    n as usize
}

/// The centroid store of probe selection, built once per index (`Cent::new`,
/// `src/gpu_step/knn/ivf.rs:62-69`): digit blocks, exponents and norms.
pub fn knn_centroids_prep<H: DeviceBuffer + ?Sized>(centroids: &H, nlist: usize, d: usize, digits: &H, cexp: &H, cnorm: &H) {
    need::<f32, H>(centroids, mul(nlist, d), "knn_centroids_prep centroids");
    need::<u8, H>(digits, knn_centroid_digit_bytes(nlist, d), "knn_centroids_prep digits");
    need::<i32, H>(cexp, nlist, "knn_centroids_prep cexp");
    need::<f64, H>(cnorm, nlist, "knn_centroids_prep cnorm");
    check(unsafe {
        sys::st_knn_centroids_prep(ptr(centroids), nlist as i64, d as i64, dptr(digits), dptr(cexp), dptr(cnorm), stream())
    });
}

/// Each query's `nprobe` nearest cells, nearest first (`search_ivf`'s probe stage,
/// `src/gpu_step/knn/ivf.rs:473-489`); probes [nq, nprobe] stay on the device.
pub fn knn_probe<H: DeviceBuffer + ?Sized>(
    digits: &H,
    cexp: &H,
    cnorm: &H,
    nlist: usize,
    queries: &H,
    nq: usize,
    d: usize,
    nprobe: usize,
    probes: &H,
) {
    need::<u8, H>(digits, knn_centroid_digit_bytes(nlist, d), "knn_probe digits");
    need::<i32, H>(cexp, nlist, "knn_probe cexp");
    need::<f64, H>(cnorm, nlist, "knn_probe cnorm");
    need::<f32, H>(queries, mul(nq, d), "knn_probe queries");
    need::<i32, H>(probes, mul(nq, nprobe), "knn_probe probes");
    check(unsafe {
        sys::st_knn_probe(
            ptr(digits),
            ptr(cexp),
            ptr(cnorm),
            nlist as i64,
            ptr(queries),
            nq as i64,
            d as i64,
            nprobe as i64,
            dptr(probes),
            stream(),
        )
    });
}

/// The scored part of `search_ivf` (`src/gpu_step/knn/ivf.rs:466`): each query's top-k keys over
/// its probed cells, nearest first, as key indices [nq, k] and distances [nq, k].
///
/// # Safety
/// The kernel reads the rows `cell_start` names, which live in device memory and cannot be
/// checked here: `cell_start` must be non-decreasing, and `codes` and `scales` must hold
/// `cell_start[ncells]` keys (`d / 4` bytes and one f32 each). The other buffers are checked.
pub unsafe fn knn_search_ivf_2bit<H: DeviceBuffer + ?Sized>(
    codes: &H,
    scales: &H,
    cell_start: &H,
    ncells: usize,
    max_cell: usize,
    queries: &H,
    probes: &H,
    nq: usize,
    nprobe: usize,
    d: usize,
    k: usize,
    out_idx: &H,
    out_dist: &H,
) {
    need::<i64, H>(cell_start, add(ncells, 1), "knn_search_ivf_2bit cell_start");
    need::<f32, H>(queries, mul(nq, d), "knn_search_ivf_2bit queries");
    need::<i32, H>(probes, mul(nq, nprobe), "knn_search_ivf_2bit probes");
    need::<i64, H>(out_idx, mul(nq, k), "knn_search_ivf_2bit out_idx");
    need::<f32, H>(out_dist, mul(nq, k), "knn_search_ivf_2bit out_dist");
    check(unsafe {
        sys::st_knn_search_ivf_2bit(
            ptr(codes),
            ptr(scales),
            ptr(cell_start),
            ncells as i64,
            max_cell as i64,
            ptr(queries),
            ptr(probes),
            nq as i64,
            nprobe as i64,
            d as i64,
            k as i64,
            dptr(out_idx),
            dptr(out_dist),
            stream(),
        )
    });
}

/// `search_tagged` / `search_tail` (`src/gpu_step/knn.rs:292-331`) over the quantised store: each
/// query's top-k among keys [lo, hi) of its row of `lohi` [nq, 2] plus the first `always` keys.
pub fn knn_search_masked_2bit<H: DeviceBuffer + ?Sized>(
    codes: &H,
    scales: &H,
    nkeys: usize,
    queries: &H,
    lohi: &H,
    always: usize,
    nq: usize,
    d: usize,
    k: usize,
    out_idx: &H,
    out_dist: &H,
) {
    need::<u8, H>(codes, mul(nkeys, d) / 4, "knn_search_masked_2bit codes");
    need::<f32, H>(scales, nkeys, "knn_search_masked_2bit scales");
    need::<f32, H>(queries, mul(nq, d), "knn_search_masked_2bit queries");
    need::<i64, H>(lohi, mul(nq, 2), "knn_search_masked_2bit lohi");
    need::<i64, H>(out_idx, mul(nq, k), "knn_search_masked_2bit out_idx");
    need::<f32, H>(out_dist, mul(nq, k), "knn_search_masked_2bit out_dist");
    check(unsafe {
        sys::st_knn_search_masked_2bit(
            ptr(codes),
            ptr(scales),
            nkeys as i64,
            ptr(queries),
            ptr(lohi),
            always as i64,
            nq as i64,
            d as i64,
            k as i64,
            dptr(out_idx),
            dptr(out_dist),
            stream(),
        )
    });
}

/// Waits for the calling thread's stream.
pub fn sync() {
    check(unsafe { sys::st_sync(stream()) });
}

/// Synchronises and frees the library's scratch arenas.
///
/// # Safety
/// No graph that captured a library call may be replayed afterwards (it would use freed memory),
/// and no other library call may run at the same time (on any thread).
pub unsafe fn scratch_release() {
    check(unsafe { sys::st_scratch_release() });
}
