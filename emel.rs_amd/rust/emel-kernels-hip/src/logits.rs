//! emel-logits' native sampler and candidate validator over device buffers
//! (crates/emel-logits/src/sampler/sm.rs, validator/sm.rs).

use emel_logits::validator::{BuildResult, ValidatorError};

use crate::ffi;
use crate::kernel::{HipEvent, HipKernel};
use crate::view::{DeviceSlice, DeviceSliceMut};

/// The sampler's failures (sampler/sm.rs:40-52).  The reference's
/// `SamplerError` sits in a crate-private module, so this enum repeats the
/// two variants a native temperature/top-k request can produce.
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub enum SamplerError {
    /// The request guard (guard_temperature_valid, sm.rs:729-747) failed.
    InvalidRequest,
    /// The device library failed (a runtime error, a call refused while its
    /// stream is captured, an argument the reference's types cannot express).
    Internal,
}

/// `SampleTemperatureTopK::new` (sampler/sm.rs:148-195) over device
/// buffers: scale, soft_max in place, rank the `top_k` best and race them
/// with Park-Miller draws.  `random_state` stays on the host and advances by
/// `top_k` draws when the event is dispatched.
#[derive(Debug)]
pub struct SampleTemperatureTopK<'a> {
    card: usize,
    temperature: f32,
    top_k: usize,
    logits: DeviceSliceMut<'a>,
    sorted_indices: DeviceSliceMut<'a, i32>,
    top_probabilities: DeviceSliceMut<'a>,
    top_indices: DeviceSliceMut<'a, i32>,
    random_state: &'a mut u32,
    selected_token_out: DeviceSliceMut<'a, i32>,
    selected_score_out: DeviceSliceMut<'a>,
}

impl<'a> SampleTemperatureTopK<'a> {
    /// Creates the request; the guard runs when it is dispatched.
    #[must_use]
    #[allow(clippy::too_many_arguments)]
    pub const fn new(
        card: usize,
        temperature: f32,
        top_k: usize,
        logits: DeviceSliceMut<'a>,
        sorted_indices: DeviceSliceMut<'a, i32>,
        top_probabilities: DeviceSliceMut<'a>,
        top_indices: DeviceSliceMut<'a, i32>,
        random_state: &'a mut u32,
        selected_token_out: DeviceSliceMut<'a, i32>,
        selected_score_out: DeviceSliceMut<'a>,
    ) -> Self {
        Self {
            card,
            temperature,
            top_k,
            logits,
            sorted_indices,
            top_probabilities,
            top_indices,
            random_state,
            selected_token_out,
            selected_score_out,
        }
    }
}

impl HipEvent for SampleTemperatureTopK<'_> {
    type Output = Result<(), SamplerError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        if self.selected_token_out.is_empty() || self.selected_score_out.is_empty() {
            return Err(SamplerError::InvalidRequest);
        }
        let request = ffi::EmelSampleTemperatureTopKRequest {
            card: self.card as u64,
            temperature: self.temperature,
            reserved: 0,
            top_k: self.top_k as u64,
            logits: self.logits.ptr(),
            logits_len: self.logits.len() as u64,
            sorted_indices: self.sorted_indices.ptr(),
            sorted_indices_len: self.sorted_indices.len() as u64,
            top_probabilities: self.top_probabilities.ptr(),
            top_probabilities_len: self.top_probabilities.len() as u64,
            top_indices: self.top_indices.ptr(),
            top_indices_len: self.top_indices.len() as u64,
            random_state: core::ptr::from_mut(self.random_state),
            selected_token_out: self.selected_token_out.ptr(),
            selected_score_out: self.selected_score_out.ptr(),
            status_out: core::ptr::null_mut(),
        };
        // SAFETY: every buffer is live device memory of the stated length and
        // random_state a live host u32; the library checks the guard first.
        let status = kernel.call(|s| unsafe { ffi::emel_sample_temperature_top_k(&raw const request, s) });
        match status {
            ffi::EMEL_OK => Ok(()),
            ffi::EMEL_ERR_INVALID_REQUEST => Err(SamplerError::InvalidRequest),
            _ => Err(SamplerError::Internal),
        }
    }
}

/// `rows` independent temperature/top-k requests in one launch: row `r`
/// reads `logits[r * logits_stride ..]`, ranks into `sorted_indices[r *
/// sorted_stride ..]` and `top_*[r * top_stride ..]`, draws from
/// `random_states[r]` and writes `selected_*_out[r]`; `status_out[r]` gets
/// that row's result guard (sampler/sm.rs:849-858).
#[derive(Debug)]
pub struct SampleTemperatureTopKRows<'a> {
    request: SampleTemperatureTopK<'a>,
    rows: ffi::EmelSampleRows,
    random_states: &'a mut [u32],
    status_out: DeviceSliceMut<'a, i32>,
}

impl<'a> SampleTemperatureTopKRows<'a> {
    /// `request` carries the whole buffers (its `random_state` is unused;
    /// `random_states` holds one state per row).
    #[must_use]
    pub const fn new(
        request: SampleTemperatureTopK<'a>,
        rows: usize,
        strides: [usize; 3],
        random_states: &'a mut [u32],
        status_out: DeviceSliceMut<'a, i32>,
    ) -> Self {
        let rows = ffi::EmelSampleRows {
            rows: rows as u64,
            logits_stride: strides[0] as u64,
            sorted_stride: strides[1] as u64,
            top_stride: strides[2] as u64,
        };
        Self { request, rows, random_states, status_out }
    }
}

impl HipEvent for SampleTemperatureTopKRows<'_> {
    type Output = Result<(), SamplerError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let n = usize::try_from(self.rows.rows).unwrap_or(usize::MAX);
        let r = &self.request;
        if self.random_states.len() < n
            || self.status_out.len() < n
            || r.selected_token_out.len() < n
            || r.selected_score_out.len() < n
        {
            return Err(SamplerError::InvalidRequest);
        }
        let request = ffi::EmelSampleTemperatureTopKRequest {
            card: r.card as u64,
            temperature: r.temperature,
            reserved: 0,
            top_k: r.top_k as u64,
            logits: r.logits.ptr(),
            logits_len: r.logits.len() as u64,
            sorted_indices: r.sorted_indices.ptr(),
            sorted_indices_len: r.sorted_indices.len() as u64,
            top_probabilities: r.top_probabilities.ptr(),
            top_probabilities_len: r.top_probabilities.len() as u64,
            top_indices: r.top_indices.ptr(),
            top_indices_len: r.top_indices.len() as u64,
            random_state: self.random_states.as_mut_ptr(),
            selected_token_out: r.selected_token_out.ptr(),
            selected_score_out: r.selected_score_out.ptr(),
            status_out: self.status_out.ptr(),
        };
        let rows = self.rows;
        // SAFETY: as for SampleTemperatureTopK, with `rows` rows of each
        // buffer checked by the library against the whole lengths.
        let status = kernel.call(|s| unsafe {
            ffi::emel_sample_temperature_top_k_rows(&raw const request, &raw const rows, s)
        });
        match status {
            ffi::EMEL_OK => Ok(()),
            ffi::EMEL_ERR_INVALID_REQUEST => Err(SamplerError::InvalidRequest),
            _ => Err(SamplerError::Internal),
        }
    }
}

/// `SamplePreselected::new(vocab_size, selected_token)` (sampler/sm.rs:
/// 129-146): a host-only check that the upstream token lies in the
/// vocabulary; returns it.
///
/// # Errors
/// `SamplerError::InvalidRequest` when the guard (sm.rs:685-695) fails.
pub fn sample_preselected(vocab_size: usize, selected_token: i32) -> Result<i32, SamplerError> {
    let mut token = -1_i32;
    // SAFETY: host-only call; `token` is a valid out pointer.
    let status = unsafe { ffi::emel_sample_preselected(vocab_size as u64, selected_token, &raw mut token) };
    match status {
        ffi::EMEL_OK => Ok(token),
        ffi::EMEL_ERR_INVALID_REQUEST => Err(SamplerError::InvalidRequest),
        _ => Err(SamplerError::Internal),
    }
}

/// `validator::Build::new` (validator/sm.rs:33-66) over device buffers:
/// `candidate_ids[i] = i`, `candidate_scores[i] = logits[i] - max`.
#[derive(Debug)]
pub struct Build<'a> {
    logits: DeviceSlice<'a>,
    vocab_size: i32,
    candidate_ids: DeviceSliceMut<'a, i32>,
    candidate_scores: DeviceSliceMut<'a>,
    candidate_capacity: i32,
}

impl<'a> Build<'a> {
    /// Creates the request; the guard runs when it is dispatched.  The
    /// candidate count and error come back in the result instead of the
    /// reference's out-references.
    #[must_use]
    pub const fn new(
        logits: DeviceSlice<'a>,
        vocab_size: i32,
        candidate_ids: DeviceSliceMut<'a, i32>,
        candidate_scores: DeviceSliceMut<'a>,
        candidate_capacity: i32,
    ) -> Self {
        Self { logits, vocab_size, candidate_ids, candidate_scores, candidate_capacity }
    }
}

impl HipEvent for Build<'_> {
    type Output = Result<BuildResult, ValidatorError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let mut count = 0_i32;
        let mut error = ffi::EMEL_VALIDATOR_NONE as i32;
        let (l, nl) = (self.logits.ptr(), self.logits.len() as u64);
        let (ids, nids) = (self.candidate_ids.ptr(), self.candidate_ids.len() as u64);
        let (sc, nsc) = (self.candidate_scores.ptr(), self.candidate_scores.len() as u64);
        let (vocab, capacity) = (self.vocab_size, self.candidate_capacity);
        // SAFETY: live device buffers of the stated lengths; count and error
        // are host scalars written before the call returns.
        let status = kernel.call(|s| unsafe {
            ffi::emel_logits_validator_build(
                l, nl, vocab, ids, nids, sc, nsc, capacity, &raw mut count, &raw mut error, s,
            )
        });
        if status == ffi::EMEL_OK {
            return Ok(BuildResult { candidate_count: count });
        }
        Err(match u32::try_from(error).unwrap_or(u32::MAX) {
            ffi::EMEL_VALIDATOR_INVALID_REQUEST => ValidatorError::InvalidRequest,
            ffi::EMEL_VALIDATOR_INTERNAL_ERROR => ValidatorError::InternalError,
            ffi::EMEL_VALIDATOR_UNTRACKED => ValidatorError::Untracked,
            _ => ValidatorError::BackendError,
        })
    }
}
