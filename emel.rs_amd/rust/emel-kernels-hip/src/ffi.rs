//! Raw bindings to `libemel_hip`: a one-to-one mirror of `include/emel_hip.h`
//! at ABI version 2.
//!
//! Every struct keeps the header's field order and widths under `#[repr(C)]`,
//! every enum constant keeps its header value, and every `extern "C"`
//! declaration keeps the header's argument order and types.  Pointers inside
//! views are device addresses unless the header marks them HOST.  The safe
//! layer in this crate is the only intended caller.

#![allow(non_upper_case_globals)]
#![allow(missing_docs)] // documented in include/emel_hip.h, item for item

use core::ffi::{c_char, c_void};

/// `EMEL_HIP_ABI_VERSION`: `emel_abi_version()` returns this value.
pub const EMEL_HIP_ABI_VERSION: u32 = 2;
/// `EMEL_GET_ROWS_INLINE_INDICES`: host index spans up to this length are
/// passed inline in the kernel arguments.
pub const EMEL_GET_ROWS_INLINE_INDICES: u32 = 512;

// ---- emel_copy_shape (emel_stream_copy, a measurement reference) ----
pub const EMEL_COPY_FLAT: u32 = 0;
pub const EMEL_COPY_WAVE4: u32 = 1;
pub const EMEL_COPY_WAVE8: u32 = 2;
pub const EMEL_COPY_WALK: u32 = 3;

/// `emel_status`.
pub type Status = i32;
/// `emel_stream`: a `hipStream_t`; null is the default stream.
pub type Stream = *mut c_void;

// ---- emel_status ----
pub const EMEL_OK: Status = 0;
pub const EMEL_ERR_INVALID_VIEW: Status = 1;
pub const EMEL_ERR_SHAPE_MISMATCH: Status = 2;
pub const EMEL_ERR_INVALID_PARAMETERS: Status = 3;
pub const EMEL_ERR_UNEXPECTED_EVENT: Status = 4;
pub const EMEL_ERR_INTERNAL: Status = 5;
pub const EMEL_ERR_KERNEL_UNAVAILABLE: Status = 6;
pub const EMEL_ERR_DEVICE: Status = 7;
pub const EMEL_ERR_INVALID_ARGUMENT: Status = 8;
pub const EMEL_ERR_INVALID_SHAPE: Status = 9;
pub const EMEL_ERR_UNSUPPORTED_OPERATION: Status = 10;
pub const EMEL_ERR_INDEX_OUT_OF_BOUNDS: Status = 11;
pub const EMEL_ERR_UNSUPPORTED_SOURCE_STRIDE: Status = 12;
pub const EMEL_ERR_INVALID_REQUEST: Status = 13;
pub const EMEL_ERR_STREAM_CAPTURE: Status = 14;
pub const EMEL_ERR_INVALID_OFFSET: Status = 15;
pub const EMEL_ERR_ZERO_NORM: Status = 16;

// ---- emel_dtype ----
pub const EMEL_DTYPE_F32: u32 = 0;
pub const EMEL_DTYPE_F16: u32 = 1;
pub const EMEL_DTYPE_Q4_0: u32 = 2;
pub const EMEL_DTYPE_Q8_0: u32 = 8;
pub const EMEL_DTYPE_Q4_K: u32 = 12;
pub const EMEL_DTYPE_I32: u32 = 26;
pub const EMEL_DTYPE_BF16: u32 = 30;

// ---- emel_unary_subop ----
pub const EMEL_UNARY_ABS: u32 = 0;
pub const EMEL_UNARY_SGN: u32 = 1;
pub const EMEL_UNARY_NEG: u32 = 2;
pub const EMEL_UNARY_STEP: u32 = 3;
pub const EMEL_UNARY_TANH: u32 = 4;
pub const EMEL_UNARY_ELU: u32 = 5;
pub const EMEL_UNARY_RELU: u32 = 6;
pub const EMEL_UNARY_SIGMOID: u32 = 7;
pub const EMEL_UNARY_GELU: u32 = 8;
pub const EMEL_UNARY_GELU_QUICK: u32 = 9;
pub const EMEL_UNARY_SILU: u32 = 10;
pub const EMEL_UNARY_HARDSWISH: u32 = 11;
pub const EMEL_UNARY_HARDSIGMOID: u32 = 12;
pub const EMEL_UNARY_EXP: u32 = 13;
pub const EMEL_UNARY_EXPM1: u32 = 14;
pub const EMEL_UNARY_SOFTPLUS: u32 = 15;
pub const EMEL_UNARY_GELU_ERF: u32 = 16;
pub const EMEL_UNARY_XIELU: u32 = 17;
pub const EMEL_UNARY_FLOOR: u32 = 18;
pub const EMEL_UNARY_CEIL: u32 = 19;
pub const EMEL_UNARY_ROUND: u32 = 20;
pub const EMEL_UNARY_TRUNC: u32 = 21;

// ---- emel_glu_subop ----
pub const EMEL_GLU_REGLU: u32 = 0;
pub const EMEL_GLU_GEGLU: u32 = 1;
pub const EMEL_GLU_SWIGLU: u32 = 2;
pub const EMEL_GLU_SWIGLU_OAI: u32 = 3;
pub const EMEL_GLU_GEGLU_ERF: u32 = 4;
pub const EMEL_GLU_GEGLU_QUICK: u32 = 5;

// ---- emel_binary_op ----
pub const EMEL_BINARY_ADD: u32 = 0;
pub const EMEL_BINARY_SUB: u32 = 1;
pub const EMEL_BINARY_MUL: u32 = 2;
pub const EMEL_BINARY_DIV: u32 = 3;

// ---- emel_generic_op ----
pub const EMEL_GENERIC_DUP: u32 = 0;
pub const EMEL_GENERIC_ADD: u32 = 1;
pub const EMEL_GENERIC_ADD_ID: u32 = 2;
pub const EMEL_GENERIC_ADD1: u32 = 3;
pub const EMEL_GENERIC_ACC: u32 = 4;
pub const EMEL_GENERIC_SUB: u32 = 5;
pub const EMEL_GENERIC_MUL: u32 = 6;
pub const EMEL_GENERIC_DIV: u32 = 7;
pub const EMEL_GENERIC_SQR: u32 = 8;
pub const EMEL_GENERIC_SQRT: u32 = 9;
pub const EMEL_GENERIC_LOG: u32 = 10;
pub const EMEL_GENERIC_SIN: u32 = 11;
pub const EMEL_GENERIC_COS: u32 = 12;
pub const EMEL_GENERIC_SUM: u32 = 13;
pub const EMEL_GENERIC_SUM_ROWS: u32 = 14;
pub const EMEL_GENERIC_CUMSUM: u32 = 15;
pub const EMEL_GENERIC_MEAN: u32 = 16;
pub const EMEL_GENERIC_ARGMAX: u32 = 17;
pub const EMEL_GENERIC_COUNT_EQUAL: u32 = 18;
pub const EMEL_GENERIC_REPEAT: u32 = 19;
pub const EMEL_GENERIC_REPEAT_BACK: u32 = 20;
pub const EMEL_GENERIC_CONCAT: u32 = 21;
pub const EMEL_GENERIC_SILU_BACK: u32 = 22;
pub const EMEL_GENERIC_NORM: u32 = 23;
pub const EMEL_GENERIC_RMS_NORM: u32 = 24;
pub const EMEL_GENERIC_RMS_NORM_BACK: u32 = 25;
pub const EMEL_GENERIC_GROUP_NORM: u32 = 26;
pub const EMEL_GENERIC_L2_NORM: u32 = 27;
pub const EMEL_GENERIC_MUL_MAT: u32 = 28;
pub const EMEL_GENERIC_MUL_MAT_ARGMAX: u32 = 29;
pub const EMEL_GENERIC_MUL_MAT_ID: u32 = 30;
pub const EMEL_GENERIC_OUT_PROD: u32 = 31;
pub const EMEL_GENERIC_SCALE: u32 = 32;
pub const EMEL_GENERIC_SET: u32 = 33;
pub const EMEL_GENERIC_CPY: u32 = 34;
pub const EMEL_GENERIC_CONT: u32 = 35;
pub const EMEL_GENERIC_RESHAPE: u32 = 36;
pub const EMEL_GENERIC_VIEW: u32 = 37;
pub const EMEL_GENERIC_PERMUTE: u32 = 38;
pub const EMEL_GENERIC_TRANSPOSE: u32 = 39;
pub const EMEL_GENERIC_GET_ROWS: u32 = 40;
pub const EMEL_GENERIC_GET_ROWS_BACK: u32 = 41;
pub const EMEL_GENERIC_SET_ROWS: u32 = 42;
pub const EMEL_GENERIC_DIAG: u32 = 43;
pub const EMEL_GENERIC_DIAG_MASK_INF: u32 = 44;
pub const EMEL_GENERIC_DIAG_MASK_ZERO: u32 = 45;
pub const EMEL_GENERIC_SOFT_MAX: u32 = 46;
pub const EMEL_GENERIC_SOFT_MAX_BACK: u32 = 47;
pub const EMEL_GENERIC_ROPE: u32 = 48;
pub const EMEL_GENERIC_ROPE_BACK: u32 = 49;
pub const EMEL_GENERIC_CLAMP: u32 = 50;
pub const EMEL_GENERIC_CONV_TRANSPOSE_1D: u32 = 51;
pub const EMEL_GENERIC_IM2COL: u32 = 52;
pub const EMEL_GENERIC_IM2COL_BACK: u32 = 53;
pub const EMEL_GENERIC_IM2COL_3D: u32 = 54;
pub const EMEL_GENERIC_CONV_2D: u32 = 55;
pub const EMEL_GENERIC_CONV_3D: u32 = 56;
pub const EMEL_GENERIC_CONV_2D_DW: u32 = 57;
pub const EMEL_GENERIC_CONV_TRANSPOSE_2D: u32 = 58;
pub const EMEL_GENERIC_POOL_1D: u32 = 59;
pub const EMEL_GENERIC_POOL_2D: u32 = 60;
pub const EMEL_GENERIC_POOL_2D_BACK: u32 = 61;
pub const EMEL_GENERIC_UPSCALE: u32 = 62;
pub const EMEL_GENERIC_PAD: u32 = 63;
pub const EMEL_GENERIC_PAD_REFLECT_1D: u32 = 64;
pub const EMEL_GENERIC_ROLL: u32 = 65;
pub const EMEL_GENERIC_ARANGE: u32 = 66;
pub const EMEL_GENERIC_TIMESTEP_EMBEDDING: u32 = 67;
pub const EMEL_GENERIC_ARGSORT: u32 = 68;
pub const EMEL_GENERIC_TOP_K: u32 = 69;
pub const EMEL_GENERIC_LEAKY_RELU: u32 = 70;
pub const EMEL_GENERIC_TRI: u32 = 71;
pub const EMEL_GENERIC_FILL: u32 = 72;
pub const EMEL_GENERIC_FLASH_ATTN_EXT: u32 = 73;
pub const EMEL_GENERIC_FLASH_ATTN_BACK: u32 = 74;
pub const EMEL_GENERIC_SSM_CONV: u32 = 75;
pub const EMEL_GENERIC_SSM_SCAN: u32 = 76;
pub const EMEL_GENERIC_WIN_PART: u32 = 77;
pub const EMEL_GENERIC_WIN_UNPART: u32 = 78;
pub const EMEL_GENERIC_GET_REL_POS: u32 = 79;
pub const EMEL_GENERIC_ADD_REL_POS: u32 = 80;
pub const EMEL_GENERIC_RWKV_WKV6: u32 = 81;
pub const EMEL_GENERIC_GATED_LINEAR_ATTN: u32 = 82;
pub const EMEL_GENERIC_RWKV_WKV7: u32 = 83;
pub const EMEL_GENERIC_SOLVE_TRI: u32 = 84;
pub const EMEL_GENERIC_UNARY: u32 = 85;
pub const EMEL_GENERIC_MAP_CUSTOM1: u32 = 86;
pub const EMEL_GENERIC_MAP_CUSTOM2: u32 = 87;
pub const EMEL_GENERIC_MAP_CUSTOM3: u32 = 88;
pub const EMEL_GENERIC_CUSTOM: u32 = 89;
pub const EMEL_GENERIC_CROSS_ENTROPY_LOSS: u32 = 90;
pub const EMEL_GENERIC_CROSS_ENTROPY_LOSS_BACK: u32 = 91;
pub const EMEL_GENERIC_OPT_STEP_ADAMW: u32 = 92;
pub const EMEL_GENERIC_OPT_STEP_SGD: u32 = 93;
pub const EMEL_GENERIC_GLU: u32 = 94;
pub const EMEL_GENERIC_OPERATION_COUNT: u32 = 95;

// ---- emel_validator_error ----
pub const EMEL_VALIDATOR_NONE: u32 = 0;
pub const EMEL_VALIDATOR_INVALID_REQUEST: u32 = 1;
pub const EMEL_VALIDATOR_BACKEND_ERROR: u32 = 2;
pub const EMEL_VALIDATOR_INTERNAL_ERROR: u32 = 3;
pub const EMEL_VALIDATOR_UNTRACKED: u32 = 4;

/// `emel_tensor_view`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelTensorView {
    pub data: *const c_void,
    pub dtype: u32,
    pub reserved: u32,
    pub ne: [u64; 4],
    pub nb: [u64; 4],
    pub data_bytes: u64,
}

/// `emel_tensor_view_mut`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelTensorViewMut {
    pub data: *mut c_void,
    pub dtype: u32,
    pub reserved: u32,
    pub ne: [u64; 4],
    pub nb: [u64; 4],
    pub data_bytes: u64,
}

/// `emel_index_view`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelIndexView {
    pub data: *const i32,
    pub len: u64,
    pub ne: [u64; 3],
    pub nb: [u64; 3],
    pub explicit_strides: u32,
    pub on_host: u32,
}

/// `emel_generic_request`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelGenericRequest {
    pub operation: u32,
    pub unary_subop: u32,
    pub glu_subop: u32,
    pub pool_subop: u32,
    pub src0: *const EmelTensorView,
    pub src1: *const EmelTensorView,
    pub src2: *const EmelTensorView,
    pub dst: *const EmelTensorViewMut,
    pub op_params: [u8; 64],
    pub op_params_size: u32,
    pub reserved: u32,
    pub index_out: *mut i32,
}

/// `emel_sample_temperature_top_k_request`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelSampleTemperatureTopKRequest {
    pub card: u64,
    pub temperature: f32,
    pub reserved: u32,
    pub top_k: u64,
    pub logits: *mut f32,
    pub logits_len: u64,
    pub sorted_indices: *mut i32,
    pub sorted_indices_len: u64,
    pub top_probabilities: *mut f32,
    pub top_probabilities_len: u64,
    pub top_indices: *mut i32,
    pub top_indices_len: u64,
    pub random_state: *mut u32,
    pub selected_token_out: *mut i32,
    pub selected_score_out: *mut f32,
    pub status_out: *mut i32,
}

/// `emel_sample_rows`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct EmelSampleRows {
    pub rows: u64,
    pub logits_stride: u64,
    pub sorted_stride: u64,
    pub top_stride: u64,
}

// Linked by build.rs (`cargo:rustc-link-lib=dylib=emel_hip`).
unsafe extern "C" {
    pub fn emel_abi_version() -> u32;
    pub fn emel_status_string(status: Status) -> *const c_char;
    pub fn emel_last_error() -> *const c_char;
    pub fn emel_device_count(count: *mut i32) -> Status;
    pub fn emel_set_device(device: i32) -> Status;
    pub fn emel_malloc(ptr: *mut *mut c_void, bytes: u64) -> Status;
    pub fn emel_free(ptr: *mut c_void) -> Status;
    pub fn emel_memcpy_htod(dst: *mut c_void, src: *const c_void, bytes: u64, stream: Stream) -> Status;
    pub fn emel_memcpy_dtoh(dst: *mut c_void, src: *const c_void, bytes: u64, stream: Stream) -> Status;
    pub fn emel_stream_create(stream: *mut Stream) -> Status;
    pub fn emel_stream_destroy(stream: Stream) -> Status;
    pub fn emel_stream_synchronize(stream: Stream) -> Status;
    pub fn emel_release_workspaces() -> Status;
    pub fn emel_stream_reserve(stream: Stream, work_bytes: u64, counter_bytes: u64) -> Status;
    pub fn emel_stream_workspace(stream: Stream, work_bytes: *mut u64, counter_bytes: *mut u64) -> Status;
    pub fn emel_device_prepare(stream: Stream) -> Status;
    pub fn emel_stream_copy(src: *const c_void, dst: *mut c_void, bytes: u64, shape: u32, stream: Stream) -> Status;
    pub fn emel_validate_view(view: *const EmelTensorView, allow_singleton_zero_stride: i32) -> Status;
    pub fn emel_validate_normalization_view(view: *const EmelTensorView) -> Status;
    pub fn emel_op_add(lhs: *const EmelTensorView, rhs: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_sub(lhs: *const EmelTensorView, rhs: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_mul(lhs: *const EmelTensorView, rhs: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_div(lhs: *const EmelTensorView, rhs: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_add_broadcast_row(src0: *const EmelTensorView, src1: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_mul_broadcast_row(src0: *const EmelTensorView, src1: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_binary_broadcast(op: u32, src0: *const EmelTensorView, src1: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_unary(subop: u32, in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_silu(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_gelu(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_unary_event(event: u32, in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_log(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_sin(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_cos(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_swiglu(gate: *const EmelTensorView, up: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_slice_dup(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_add(lhs: *const f32, lhs_len: u64, rhs: *const f32, rhs_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_sub(lhs: *const f32, lhs_len: u64, rhs: *const f32, rhs_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_mul(lhs: *const f32, lhs_len: u64, rhs: *const f32, rhs_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_div(lhs: *const f32, lhs_len: u64, rhs: *const f32, rhs_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_sqr(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_slice_sqrt(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_op_sqr(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_sqrt(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_glu(subop: u32, input: *const f32, input_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_op_scale(in_: *const EmelTensorView, out: *const EmelTensorViewMut, scale: f32, stream: Stream) -> Status;
    pub fn emel_op_rms_norm(in_: *const EmelTensorView, out: *const EmelTensorViewMut, epsilon: f32, stream: Stream) -> Status;
    pub fn emel_op_rms_norm_mul(in_: *const EmelTensorView, weight: *const EmelTensorView, out: *const EmelTensorViewMut, epsilon: f32, stream: Stream) -> Status;
    pub fn emel_op_norm(in_: *const EmelTensorView, out: *const EmelTensorViewMut, epsilon: f32, stream: Stream) -> Status;
    pub fn emel_op_soft_max(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_soft_max_ext(src: *const EmelTensorView, mask: *const EmelTensorView, scale: f32, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_sum_rows(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_sum(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_mean(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_argmax(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_argmax_rows(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_clamp(in_: *const EmelTensorView, out: *const EmelTensorViewMut, min: f32, max: f32, stream: Stream) -> Status;
    pub fn emel_op_leaky_relu(in_: *const EmelTensorView, out: *const EmelTensorViewMut, negative_slope: f32, stream: Stream) -> Status;
    pub fn emel_op_silu_back(in_: *const EmelTensorView, gradient: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_add1(src: *const EmelTensorView, scalar: f32, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_acc(base: *const EmelTensorView, update: *const EmelTensorView, dst: *const EmelTensorViewMut, offset: u64, stream: Stream) -> Status;
    pub fn emel_op_diag(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, stream: Stream) -> Status;
    pub fn emel_op_diag_mask_inf(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, n_past: i32, stream: Stream) -> Status;
    pub fn emel_op_diag_mask_zero(input: *const f32, input_len: u64, output: *mut f32, output_len: u64, n_past: i32, stream: Stream) -> Status;
    pub fn emel_op_group_norm(in_: *const EmelTensorView, out: *const EmelTensorViewMut, groups: u64, epsilon: f32, stream: Stream) -> Status;
    pub fn emel_op_l2_norm(in_: *const EmelTensorView, out: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_argmax_rows_no_alloc(src: *const EmelTensorView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_f32_bytes(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_f16(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_bf16(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_q4_0(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_q8_0(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_op_get_rows_q4_k(src: *const EmelTensorView, indices: *const EmelIndexView, dst: *const EmelTensorViewMut, stream: Stream) -> Status;
    pub fn emel_generic_dispatch(request: *const EmelGenericRequest, stream: Stream) -> Status;
    pub fn emel_sample_temperature_top_k(request: *const EmelSampleTemperatureTopKRequest, stream: Stream) -> Status;
    pub fn emel_sample_temperature_top_k_rows(request: *const EmelSampleTemperatureTopKRequest, rows: *const EmelSampleRows, stream: Stream) -> Status;
    pub fn emel_sample_preselected(vocab_size: u64, selected_token: i32, token_out: *mut i32) -> Status;
    pub fn emel_logits_validator_build(logits: *const f32, logits_len: u64, vocab_size: i32, candidate_ids: *mut i32, candidate_ids_len: u64, candidate_scores: *mut f32, candidate_scores_len: u64, candidate_capacity: i32, candidate_count_out: *mut i32, error_out: *mut i32, stream: Stream) -> Status;
}
