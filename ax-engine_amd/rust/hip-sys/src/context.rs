//! Safe wrapper of one sampler context (`axs_context`): device workspace for
//! up to `max_batch` rows of `max_vocab` ids on one GPU.
use std::ptr::{NonNull, null_mut};

use crate::error::{HipSamplerError, check};
use crate::ffi;

/// Per-row parameters, the C `axs_sampling_params` (64 bytes).
pub type RowParams = ffi::axs_sampling_params;

/// One step's host inputs for [`HipSamplerContext::sample_host`].
pub struct HostBatch<'a> {
    /// `[batch * vocab]` f32 logits, row-major.
    pub logits: &'a [f32],
    pub batch: usize,
    pub vocab: usize,
    /// `[batch]` row parameters.
    pub params: &'a [RowParams],
    /// Token history in CSR form (oldest first per row); `history_offsets`
    /// empty = no history.
    pub history: &'a [u32],
    pub history_offsets: &'a [i64],
    /// One uniform per row, or `None` for the device's Philox(seed, row, step).
    pub uniforms: Option<&'a [f32]>,
}

/// Per-row outputs: token ids, logprobs (when asked for) and `AXS_FLAG_*` bits.
#[derive(Clone, Debug, Default, PartialEq)]
pub struct HostRowOutputs {
    pub token_ids: Vec<u32>,
    pub logprobs: Vec<f32>,
    pub flags: Vec<u32>,
}

#[derive(Debug)]
pub struct HipSamplerContext {
    raw: NonNull<ffi::axs_context>,
    device: i32,
}

// The library serialises the calls made on one context (a lock around each
// call, and an event between calls on different streams).
unsafe impl Send for HipSamplerContext {}
unsafe impl Sync for HipSamplerContext {}

impl HipSamplerContext {
    pub fn new(device: i32, max_batch: i32, max_vocab: i32) -> Result<Self, HipSamplerError> {
        crate::error::install_recoverable_error_handler();
        let mut raw: *mut ffi::axs_context = null_mut();
        check(unsafe { ffi::axs_context_create(device, max_batch, max_vocab, &mut raw) })?;
        let raw = NonNull::new(raw).ok_or_else(|| HipSamplerError {
            status: ffi::AXS_E_HIP as i32,
            message: String::from("axs_context_create returned no context"),
        })?;
        Ok(Self { raw, device })
    }

    pub fn device(&self) -> i32 {
        self.device
    }

    /// One batched sampling step over host data (`axs_sample_batch_host`):
    /// synchronous; the library copies the inputs to the GPU, samples and
    /// copies the outputs back.
    pub fn sample_host(
        &self,
        b: &HostBatch<'_>,
        want_logprobs: bool,
    ) -> Result<HostRowOutputs, HipSamplerError> {
        assert_eq!(b.logits.len(), b.batch * b.vocab, "logits must be [batch * vocab]");
        assert_eq!(b.params.len(), b.batch, "params must have one entry per row");
        let mut desc: ffi::axs_batch_desc = unsafe { std::mem::zeroed() };
        desc.logits = b.logits.as_ptr().cast();
        desc.dtype = ffi::AXS_DTYPE_F32 as i32;
        desc.batch = i32::try_from(b.batch).expect("batch fits in i32");
        desc.vocab = i32::try_from(b.vocab).expect("vocab fits in i32");
        desc.row_stride = b.vocab as i64;
        desc.params = b.params.as_ptr();
        if !b.history_offsets.is_empty() {
            assert_eq!(b.history_offsets.len(), b.batch + 1, "history_offsets must be [batch + 1]");
            desc.history = b.history.as_ptr();
            desc.history_offsets = b.history_offsets.as_ptr();
            desc.history_len = b.history.len() as i64;
        }
        if let Some(u) = b.uniforms {
            assert_eq!(u.len(), b.batch, "uniforms must have one entry per row");
            desc.uniforms = u.as_ptr();
        }
        let mut out = HostRowOutputs {
            token_ids: vec![0; b.batch],
            logprobs: if want_logprobs { vec![0.0; b.batch] } else { Vec::new() },
            flags: vec![0; b.batch],
        };
        let mut o: ffi::axs_outputs = unsafe { std::mem::zeroed() };
        o.token_ids = out.token_ids.as_mut_ptr();
        o.logprobs = if want_logprobs { out.logprobs.as_mut_ptr() } else { null_mut() };
        o.flags = out.flags.as_mut_ptr();
        check(unsafe { ffi::axs_sample_batch_host(self.raw.as_ptr(), &desc, &o) })?;
        Ok(out)
    }
}

impl Drop for HipSamplerContext {
    fn drop(&mut self) {
        unsafe {
            ffi::axs_context_destroy(self.raw.as_ptr());
        }
    }
}
