//! MI355X drop-in for `cf_core::ops::attention` (crates/core/src/ops/attention.rs:18-262):
//! the same items with the same signatures and panics, computed by the gfx950 kernels of
//! `libcfattn.so` (include/cfattn.h).
//!
//! Two layers:
//! - the top-level functions (`attention_forward`, `attention_backward` and their `_blocked`
//!   forms) take host slices, as the reference does; every call stages its operands through
//!   pinned memory to the GPU and its results back (PCIe-inclusive);
//! - [`device`] binds the entry points on device buffers (`cfattn_fwd`, `cfattn_bwd`,
//!   `cfattn_fused_fwd`, `cfattn_fused_bwd`, ...) for a caller whose tensors already live in HBM
//!   (a device-resident `Layer`, crates/model/src/layer.rs:104-121, 183-206); those calls queue
//!   on a HIP stream and return at once.
//!
//! Switching cpuforge over is a feature flag in crates/core/src/ops/attention.rs:
//! ```ignore
//! #[cfg(feature = "mi355x")]
//! pub use cf_attn_hip::{attention_backward, attention_backward_blocked, attention_forward,
//!                       attention_forward_blocked, AttnShape, DEFAULT_Q_BLOCK};
//! ```
use std::ffi::CStr;
use std::os::raw::{c_char, c_int, c_void};
use std::sync::Mutex;

/// Raw C ABI of libcfattn.so (include/cfattn.h).
pub mod ffi {
    use std::os::raw::{c_char, c_int, c_void};

    pub const CFATTN_OK: c_int = 0;
    pub const CFATTN_F32: c_int = 0;
    pub const CFATTN_BF16: c_int = 1;

    #[repr(C)]
    #[derive(Clone, Copy, Debug, PartialEq, Eq)]
    pub struct Shape {
        pub seq: usize,
        pub n_heads: usize,
        pub n_kv: usize,
        pub head_dim: usize,
    }

    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct Llama3Scaling {
        pub factor: f64,
        pub low_freq_factor: f64,
        pub high_freq_factor: f64,
        pub original_max_position: f64,
    }

    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct Prologue {
        pub cos: *const f32,
        pub sin: *const f32,
        pub max_pos: usize,
        pub pos0: usize,
        pub q_norm: *const f32,
        pub k_norm: *const f32,
        pub eps: f32,
    }

    #[repr(C)]
    pub struct Ctx {
        _private: [u8; 0],
    }

    extern "C" {
        pub fn cfattn_create(device: c_int, out: *mut *mut Ctx) -> c_int;
        pub fn cfattn_destroy(ctx: *mut Ctx) -> c_int;
        pub fn cfattn_last_error(ctx: *const Ctx) -> *const c_char;
        pub fn cfattn_set_mode(ctx: *mut Ctx, dtype: c_int) -> c_int;
        pub fn cfattn_get_mode(ctx: *const Ctx) -> c_int;
        pub fn cfattn_synchronize(ctx: *mut Ctx) -> c_int;

        pub fn cfattn_attention_forward_blocked(
            ctx: *mut Ctx, q: *const f32, q_len: usize, k: *const f32, k_len: usize, v: *const f32,
            v_len: usize, o: *mut f32, o_len: usize, lse: *mut f32, lse_len: usize, s: Shape, q_block: usize,
        ) -> c_int;
        pub fn cfattn_attention_backward_blocked(
            ctx: *mut Ctx, d_o: *const f32, d_o_len: usize, q: *const f32, q_len: usize, k: *const f32,
            k_len: usize, v: *const f32, v_len: usize, o: *const f32, o_len: usize, lse: *const f32,
            lse_len: usize, dq: *mut f32, dq_len: usize, dk: *mut f32, dk_len: usize, dv: *mut f32,
            dv_len: usize, s: Shape, q_block: usize,
        ) -> c_int;

        pub fn cfattn_fwd(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, q: *const c_void, k: *const c_void,
            v: *const c_void, o: *mut f32, lse: *mut f32, stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_bwd(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, d_o: *const c_void, q: *const c_void,
            k: *const c_void, v: *const c_void, o: *const f32, lse: *const f32, dq: *mut f32, dk: *mut f32,
            dv: *mut f32, stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_bwd_noalloc(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, d_o: *const c_void, q: *const c_void,
            k: *const c_void, v: *const c_void, o: *const f32, lse: *const f32, dq: *mut f32, dk: *mut f32,
            dv: *mut f32, stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_prologue_fwd(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, pr: *const Prologue, q_pre: *const f32,
            k_pre: *const f32, q_out: *mut c_void, k_out: *mut c_void, q_rstd: *mut f32, k_rstd: *mut f32,
            stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_prologue_bwd(
            ctx: *mut Ctx, s: Shape, batch: usize, pr: *const Prologue, dq: *const f32, dk: *const f32,
            q_pre: *const f32, k_pre: *const f32, q_rstd: *const f32, k_rstd: *const f32, dq_pre: *mut f32,
            dk_pre: *mut f32, dq_norm: *mut f32, dk_norm: *mut f32, stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_fused_fwd(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, pr: *const Prologue, q_pre: *const f32,
            k_pre: *const f32, v: *const c_void, q_out: *mut c_void, k_out: *mut c_void, q_rstd: *mut f32,
            k_rstd: *mut f32, o: *mut f32, lse: *mut f32, stream: *mut c_void,
        ) -> c_int;
        pub fn cfattn_fused_bwd(
            ctx: *mut Ctx, s: Shape, batch: usize, dtype: c_int, pr: *const Prologue, d_o: *const c_void,
            q_pre: *const f32, k_pre: *const f32, q: *const c_void, k: *const c_void, v: *const c_void,
            o: *const f32, lse: *const f32, q_rstd: *const f32, k_rstd: *const f32, dq_pre: *mut f32,
            dk_pre: *mut f32, dv: *mut f32, dq_norm: *mut f32, dk_norm: *mut f32, stream: *mut c_void,
        ) -> c_int;

        pub fn cfattn_rope_table(
            head_dim: usize, max_pos: usize, theta: f64, scaling: *const Llama3Scaling, cos_out: *mut f32,
            sin_out: *mut f32,
        ) -> c_int;
        pub fn cfattn_llama3_scale(scaling: *const Llama3Scaling, inv_freq: f64) -> f64;
        pub fn cfattn_set_ds_limit(ctx: *mut Ctx, bytes: usize) -> c_int;
    }
}

/// Query rows per block of the reference's blocked attention (attention.rs:18-26).
pub const DEFAULT_Q_BLOCK: usize = 128;

/// `cf_core::ops::attention::AttnShape`.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct AttnShape {
    pub seq: usize,
    pub n_heads: usize,
    pub n_kv: usize,
    pub head_dim: usize,
}

impl AttnShape {
    fn c(self) -> ffi::Shape {
        ffi::Shape { seq: self.seq, n_heads: self.n_heads, n_kv: self.n_kv, head_dim: self.head_dim }
    }
}

fn last_error(ctx: *mut ffi::Ctx) -> String {
    unsafe { CStr::from_ptr(ffi::cfattn_last_error(ctx) as *const c_char) }.to_string_lossy().into_owned()
}

struct Handle(*mut ffi::Ctx);
unsafe impl Send for Handle {}

// One context per process (device 0) for the host-slice functions; the calls are
// synchronous, as the reference op is.  CPUFORGE_ATTN_BF16 selects the bf16 mode
// (bf16 inputs, fp32 accumulation); the default is fp32, the reference's precision.
static CTX: Mutex<Option<Handle>> = Mutex::new(None);

/// Runs one library call on the process's context and panics, as the reference's
/// asserts do, when it fails.  The panic comes after the context lock is released,
/// so a caught panic (a failed shape check, say) leaves the context usable.
fn call(f: impl FnOnce(*mut ffi::Ctx) -> c_int) {
    let err = {
        // A lock poisoned by a panic elsewhere still guards a consistent context.
        let mut g = CTX.lock().unwrap_or_else(|e| e.into_inner());
        let mut err: Option<String> = None;
        if g.is_none() {
            let mut p = std::ptr::null_mut();
            let rc = unsafe { ffi::cfattn_create(0, &mut p) };
            if rc != ffi::CFATTN_OK {
                err = Some(format!("cfattn_create failed ({rc}): no usable MI355X"));
            } else {
                if std::env::var("CPUFORGE_ATTN_BF16").is_ok() {
                    unsafe { ffi::cfattn_set_mode(p, ffi::CFATTN_BF16) };
                }
                *g = Some(Handle(p));
            }
        }
        if let Some(h) = g.as_ref() {
            let c = h.0;
            // The library words its shape errors after the reference's assert_eq!.
            if f(c) != ffi::CFATTN_OK {
                err = Some(last_error(c));
            }
        }
        err
    };
    if let Some(msg) = err {
        panic!("{msg}");
    }
}

/// `attention_forward` (attention.rs:42-46): o = softmax(q k^T / sqrt(d), causal) v, lse per row.
pub fn attention_forward(q: &[f32], k: &[f32], v: &[f32], o: &mut [f32], lse: &mut [f32], s: AttnShape) {
    attention_forward_blocked(q, k, v, o, lse, s, DEFAULT_Q_BLOCK)
}

/// `attention_forward_blocked` (attention.rs:48-122).  `q_block` only sets the reference's
/// blocking; the result does not depend on it.
pub fn attention_forward_blocked(
    q: &[f32], k: &[f32], v: &[f32], o: &mut [f32], lse: &mut [f32], s: AttnShape, q_block: usize,
) {
    call(|c| unsafe {
        ffi::cfattn_attention_forward_blocked(
            c, q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(), v.len(), o.as_mut_ptr(), o.len(),
            lse.as_mut_ptr(), lse.len(), s.c(), q_block,
        )
    })
}

/// `attention_backward` (attention.rs:126-140): accumulates into dq, dk, dv.
#[allow(clippy::too_many_arguments)]
pub fn attention_backward(
    d_o: &[f32], q: &[f32], k: &[f32], v: &[f32], o: &[f32], lse: &[f32], dq: &mut [f32], dk: &mut [f32],
    dv: &mut [f32], s: AttnShape,
) {
    attention_backward_blocked(d_o, q, k, v, o, lse, dq, dk, dv, s, DEFAULT_Q_BLOCK)
}

/// `attention_backward_blocked` (attention.rs:142-262).
#[allow(clippy::too_many_arguments)]
pub fn attention_backward_blocked(
    d_o: &[f32], q: &[f32], k: &[f32], v: &[f32], o: &[f32], lse: &[f32], dq: &mut [f32], dk: &mut [f32],
    dv: &mut [f32], s: AttnShape, q_block: usize,
) {
    call(|c| unsafe {
        ffi::cfattn_attention_backward_blocked(
            c, d_o.as_ptr(), d_o.len(), q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(), v.len(),
            o.as_ptr(), o.len(), lse.as_ptr(), lse.len(), dq.as_mut_ptr(), dq.len(), dk.as_mut_ptr(), dk.len(),
            dv.as_mut_ptr(), dv.len(), s.c(), q_block,
        )
    })
}

/// The entry points on device buffers (hipMalloc'd, or any HBM pointer of the context's device).
///
/// Every function queues its kernels on `stream` (a `hipStream_t`; null is the device's null
/// stream) and returns at once.  The pointers are raw: the caller keeps the buffers alive and
/// sized as include/cfattn.h states until the stream has passed the call.
pub mod device {
    use super::{ffi, last_error, AttnShape};
    use std::os::raw::{c_int, c_void};

    /// Element type of q, k, v and dO (o, lse and every gradient are f32).
    #[derive(Clone, Copy, Debug, PartialEq, Eq)]
    pub enum Dtype {
        F32,
        Bf16,
    }

    impl Dtype {
        fn c(self) -> c_int {
            match self {
                Dtype::F32 => ffi::CFATTN_F32,
                Dtype::Bf16 => ffi::CFATTN_BF16,
            }
        }
    }

    /// A library error: the return code and the context's message.
    #[derive(Debug, Clone)]
    pub struct Error {
        pub code: i32,
        pub message: String,
    }

    impl std::fmt::Display for Error {
        fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
            write!(f, "cfattn error {}: {}", self.code, self.message)
        }
    }

    impl std::error::Error for Error {}

    /// A `hipStream_t`.
    #[derive(Clone, Copy, Debug)]
    pub struct Stream(pub *mut c_void);

    impl Stream {
        /// The device's null (default) stream.
        pub const NULL: Stream = Stream(std::ptr::null_mut());
    }

    /// The q/k prologue of `Layer::forward` (layer.rs:104-116) on device tables: RoPE
    /// cos/sin [max_pos][head_dim/2] (see [`rope_table`]) and optional Qwen3 norm gains.
    #[derive(Clone, Copy, Debug)]
    pub struct Prologue {
        pub cos: *const f32,
        pub sin: *const f32,
        pub max_pos: usize,
        pub pos0: usize,
        pub q_norm: Option<*const f32>,
        pub k_norm: Option<*const f32>,
        pub eps: f32,
    }

    impl Prologue {
        fn c(&self) -> ffi::Prologue {
            ffi::Prologue {
                cos: self.cos,
                sin: self.sin,
                max_pos: self.max_pos,
                pos0: self.pos0,
                q_norm: self.q_norm.unwrap_or(std::ptr::null()),
                k_norm: self.k_norm.unwrap_or(std::ptr::null()),
                eps: self.eps,
            }
        }
    }

    /// `RopeCache::with_scaling` (rope.rs:46-63): cos/sin tables into host buffers of
    /// max_pos * head_dim / 2 floats each, to be copied to the device by the caller.
    pub fn rope_table(
        head_dim: usize, max_pos: usize, theta: f64, scaling: Option<ffi::Llama3Scaling>, cos: &mut [f32],
        sin: &mut [f32],
    ) -> Result<(), Error> {
        assert_eq!(cos.len(), max_pos * head_dim / 2);
        assert_eq!(sin.len(), cos.len());
        let sc = scaling.as_ref().map_or(std::ptr::null(), |s| s as *const _);
        let rc = unsafe { ffi::cfattn_rope_table(head_dim, max_pos, theta, sc, cos.as_mut_ptr(), sin.as_mut_ptr()) };
        if rc == ffi::CFATTN_OK {
            Ok(())
        } else {
            Err(Error { code: rc, message: format!("cfattn_rope_table({head_dim}, {max_pos}, {theta})") })
        }
    }

    /// A library context on one device: its scratch pool and settings.  Calls on one context
    /// must not overlap on different streams (they share scratch).
    pub struct Context {
        raw: *mut ffi::Ctx,
    }

    unsafe impl Send for Context {}

    impl Context {
        pub fn new(device: i32) -> Result<Context, Error> {
            let mut p = std::ptr::null_mut();
            let rc = unsafe { ffi::cfattn_create(device, &mut p) };
            if rc != ffi::CFATTN_OK {
                return Err(Error { code: rc, message: format!("cfattn_create({device})") });
            }
            Ok(Context { raw: p })
        }

        fn check(&self, rc: c_int) -> Result<(), Error> {
            if rc == ffi::CFATTN_OK {
                Ok(())
            } else {
                Err(Error { code: rc, message: last_error(self.raw) })
            }
        }

        /// Waits for the context's own stream.
        pub fn synchronize(&self) -> Result<(), Error> {
            self.check(unsafe { ffi::cfattn_synchronize(self.raw) })
        }

        /// Bytes of device scratch the bf16 backward may use to store dS for its dQ pass.
        pub fn set_ds_limit(&self, bytes: usize) -> Result<(), Error> {
            self.check(unsafe { ffi::cfattn_set_ds_limit(self.raw, bytes) })
        }

        /// Forward: q [batch][seq][n_heads][D], k, v [batch][seq][n_kv][D] in `dt`; writes
        /// o (f32, q's layout) and lse (f32, [batch][n_heads][seq]).
        #[allow(clippy::too_many_arguments)]
        pub unsafe fn fwd(
            &self, s: AttnShape, batch: usize, dt: Dtype, q: *const c_void, k: *const c_void, v: *const c_void,
            o: *mut f32, lse: *mut f32, stream: Stream,
        ) -> Result<(), Error> {
            self.check(ffi::cfattn_fwd(self.raw, s.c(), batch, dt.c(), q, k, v, o, lse, stream.0))
        }

        /// Backward: accumulates into the f32 dq, dk, dv.
        #[allow(clippy::too_many_arguments)]
        pub unsafe fn bwd(
            &self, s: AttnShape, batch: usize, dt: Dtype, d_o: *const c_void, q: *const c_void, k: *const c_void,
            v: *const c_void, o: *const f32, lse: *const f32, dq: *mut f32, dk: *mut f32, dv: *mut f32,
            stream: Stream,
        ) -> Result<(), Error> {
            self.check(ffi::cfattn_bwd(self.raw, s.c(), batch, dt.c(), d_o, q, k, v, o, lse, dq, dk, dv, stream.0))
        }

        /// `bwd` with no allocation (fixed per-device scratch; batch * n_heads * seq <= 2^21).
        #[allow(clippy::too_many_arguments)]
        pub unsafe fn bwd_noalloc(
            &self, s: AttnShape, batch: usize, dt: Dtype, d_o: *const c_void, q: *const c_void, k: *const c_void,
            v: *const c_void, o: *const f32, lse: *const f32, dq: *mut f32, dk: *mut f32, dv: *mut f32,
            stream: Stream,
        ) -> Result<(), Error> {
            self.check(ffi::cfattn_bwd_noalloc(self.raw, s.c(), batch, dt.c(), d_o, q, k, v, o, lse, dq, dk, dv, stream.0))
        }

        /// `Layer::forward`'s attention part (layer.rs:104-121): f32 q_pre/k_pre -> [norm] ->
        /// RoPE -> q_out/k_out in `dt` (kept for the backward, LayerCache.q/k) -> o, lse.
        /// q_rstd/k_rstd ([batch*seq*heads]) are written with the norm and may be null without.
        #[allow(clippy::too_many_arguments)]
        pub unsafe fn fused_fwd(
            &self, s: AttnShape, batch: usize, dt: Dtype, pr: &Prologue, q_pre: *const f32, k_pre: *const f32,
            v: *const c_void, q_out: *mut c_void, k_out: *mut c_void, q_rstd: *mut f32, k_rstd: *mut f32,
            o: *mut f32, lse: *mut f32, stream: Stream,
        ) -> Result<(), Error> {
            let p = pr.c();
            self.check(ffi::cfattn_fused_fwd(
                self.raw, s.c(), batch, dt.c(), &p, q_pre, k_pre, v, q_out, k_out, q_rstd, k_rstd, o, lse, stream.0,
            ))
        }

        /// `Layer::backward`'s attention part (layer.rs:183-206): d_attn_o -> dq_pre, dk_pre, dv
        /// and, with the norm, the gain gradients dq_norm/dk_norm ([head_dim]).  Accumulates.
        #[allow(clippy::too_many_arguments)]
        pub unsafe fn fused_bwd(
            &self, s: AttnShape, batch: usize, dt: Dtype, pr: &Prologue, d_o: *const c_void, q_pre: *const f32,
            k_pre: *const f32, q: *const c_void, k: *const c_void, v: *const c_void, o: *const f32,
            lse: *const f32, q_rstd: *const f32, k_rstd: *const f32, dq_pre: *mut f32, dk_pre: *mut f32,
            dv: *mut f32, dq_norm: *mut f32, dk_norm: *mut f32, stream: Stream,
        ) -> Result<(), Error> {
            let p = pr.c();
            self.check(ffi::cfattn_fused_bwd(
                self.raw, s.c(), batch, dt.c(), &p, d_o, q_pre, k_pre, q, k, v, o, lse, q_rstd, k_rstd, dq_pre,
                dk_pre, dv, dq_norm, dk_norm, stream.0,
            ))
        }
    }

    impl Drop for Context {
        fn drop(&mut self) {
            unsafe { ffi::cfattn_destroy(self.raw) };
        }
    }
}

#[cfg(test)]
mod tests {
    //! The reference's own checks (attention.rs:264-394 restate them on the CPU op) need a GPU
    //! here: run with `cargo test -- --ignored` on an MI355X host.
    use super::*;

    fn naive(q: &[f32], k: &[f32], v: &[f32], s: AttnShape) -> Vec<f32> {
        let (t, h, kv, d) = (s.seq, s.n_heads, s.n_kv, s.head_dim);
        let g = h / kv;
        let scale = 1.0 / (d as f32).sqrt();
        let mut o = vec![0.0f32; t * h * d];
        for hh in 0..h {
            for i in 0..t {
                let qi = &q[(i * h + hh) * d..(i * h + hh + 1) * d];
                let mut sc: Vec<f32> = (0..=i)
                    .map(|j| {
                        let kj = &k[(j * kv + hh / g) * d..(j * kv + hh / g + 1) * d];
                        qi.iter().zip(kj).map(|(a, b)| a * b).sum::<f32>() * scale
                    })
                    .collect();
                let m = sc.iter().cloned().fold(f32::NEG_INFINITY, f32::max);
                let mut z = 0.0;
                for x in sc.iter_mut() {
                    *x = (*x - m).exp();
                    z += *x;
                }
                for (j, p) in sc.iter().enumerate() {
                    let vj = &v[(j * kv + hh / g) * d..(j * kv + hh / g + 1) * d];
                    for c in 0..d {
                        o[(i * h + hh) * d + c] += p / z * vj[c];
                    }
                }
            }
        }
        o
    }

    #[test]
    #[ignore]
    fn forward_matches_naive_softmax_attention() {
        let s = AttnShape { seq: 37, n_heads: 4, n_kv: 2, head_dim: 16 };
        let n = |x: usize| (0..x).map(|i| ((i * 7919 % 1000) as f32 / 1000.0 - 0.5)).collect::<Vec<f32>>();
        let (q, k, v) = (n(s.seq * s.n_heads * s.head_dim), n(s.seq * s.n_kv * s.head_dim), n(s.seq * s.n_kv * s.head_dim));
        let mut o = vec![0.0; q.len()];
        let mut lse = vec![0.0; s.seq * s.n_heads];
        attention_forward(&q, &k, &v, &mut o, &mut lse, s);
        let r = naive(&q, &k, &v, s);
        let e = o.iter().zip(&r).map(|(a, b)| (a - b).abs()).fold(0.0f32, f32::max);
        assert!(e <= 1e-4, "max abs error {e}");
    }

    /// A wrong q length panics, as the reference's `assert_eq!(q, seq * q_stride)` does
    /// (attention.rs:37).  The text is the library's: it starts as Rust's assert_eq!
    /// message does ("assertion `left == right` failed") but names the operand and
    /// both lengths on one line where Rust prints `left:` and `right:` lines.
    #[test]
    #[ignore]
    #[should_panic(expected = "assertion `left == right` failed: q.len() = 3, expected 64")]
    fn wrong_q_length_panics() {
        let s = AttnShape { seq: 4, n_heads: 2, n_kv: 1, head_dim: 8 };
        let q = vec![0.0f32; 3];
        let kv = vec![0.0f32; 4 * 8];
        let mut o = vec![0.0f32; 3];
        let mut lse = vec![0.0f32; 8];
        attention_forward(&q, &kv, &kv, &mut o, &mut lse, s);
    }

    /// A caught shape panic leaves the process's context usable: the next call runs.
    #[test]
    #[ignore]
    fn a_call_after_a_caught_shape_panic_still_runs() {
        let s = AttnShape { seq: 4, n_heads: 2, n_kv: 1, head_dim: 8 };
        let bad = std::panic::catch_unwind(|| {
            let (q, kv) = (vec![0.0f32; 3], vec![0.0f32; 4 * 8]);
            let (mut o, mut lse) = (vec![0.0f32; 3], vec![0.0f32; 8]);
            attention_forward(&q, &kv, &kv, &mut o, &mut lse, s);
        });
        assert!(bad.is_err());
        let (q, kv) = (vec![0.25f32; 4 * 2 * 8], vec![0.5f32; 4 * 8]);
        let (mut o, mut lse) = (vec![0.0f32; 4 * 2 * 8], vec![0.0f32; 8]);
        attention_forward(&q, &kv, &kv, &mut o, &mut lse, s);
        // All keys equal: every output row is v's row.
        assert!(o.iter().all(|&x| (x - 0.5).abs() <= 1e-6), "{o:?}");
    }

    #[test]
    fn shape_layout_matches_the_c_struct() {
        assert_eq!(std::mem::size_of::<ffi::Shape>(), 4 * std::mem::size_of::<usize>());
        let _ = c_void_ptr_is_pointer_sized();
    }

    fn c_void_ptr_is_pointer_sized() -> bool {
        std::mem::size_of::<*mut c_void>() == std::mem::size_of::<usize>()
    }
}
