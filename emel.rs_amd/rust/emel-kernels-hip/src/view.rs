//! Views over device memory: the reference's `TensorView` / `TensorViewMut`
//! (crates/emel-kernels/src/any/tensor_view.rs), `IndexView`
//! (get_rows.rs:35-160) and the dense `&[f32]` / `&mut [f32]` operands of
//! the slice events, with device addresses in place of host slices.
//!
//! A view records the bytes its allocation holds from the view's start
//! (`data_bytes`); the library checks every reachable element against it,
//! as the reference checks against the slice length.

use core::ffi::c_void;
use core::marker::PhantomData;

use emel_kernels::any::tensor_view::{DType, Layout};

use crate::device::DeviceBuffer;
use crate::ffi;

/// An immutable device tensor: pointer, bytes available, dtype, extents and
/// byte strides (`nb[0] == 0` selects the reference's implicit contiguous
/// strides, as in `Layout`).
#[derive(Clone, Copy, Debug)]
pub struct DeviceView<'a> {
    raw: ffi::EmelTensorView,
    _data: PhantomData<&'a [u8]>,
}

impl<'a> DeviceView<'a> {
    /// A view of `layout` over the whole of `buffer`.
    #[must_use]
    pub fn new<T: Copy>(buffer: &'a DeviceBuffer<T>, layout: Layout) -> Self {
        // SAFETY: the buffer holds byte_len() bytes and outlives 'a.
        unsafe { Self::from_raw(buffer.as_ptr().cast(), buffer.byte_len() as u64, layout) }
    }

    /// A view of `layout` starting `byte_offset` bytes into `buffer`, or
    /// `None` when the offset lies past its end.
    #[must_use]
    pub fn at<T: Copy>(buffer: &'a DeviceBuffer<T>, byte_offset: usize, layout: Layout) -> Option<Self> {
        let rest = buffer.byte_len().checked_sub(byte_offset)?;
        // SAFETY: the offset stays inside the allocation, which holds `rest`
        // bytes from there and outlives 'a.
        Some(unsafe { Self::from_raw(buffer.as_ptr().cast::<u8>().add(byte_offset).cast(), rest as u64, layout) })
    }

    /// A view over memory this crate did not allocate.
    ///
    /// # Safety
    /// `data` must be a device address of the current device with at least
    /// `data_bytes` readable bytes that stay valid for 'a.
    #[must_use]
    pub unsafe fn from_raw(data: *const c_void, data_bytes: u64, layout: Layout) -> Self {
        Self {
            raw: ffi::EmelTensorView {
                data,
                dtype: u32::from(layout.dtype().code()),
                reserved: 0,
                ne: layout.ne(),
                nb: layout.nb(),
                data_bytes,
            },
            _data: PhantomData,
        }
    }

    /// The view's layout.
    #[must_use]
    pub fn layout(&self) -> Layout {
        Layout::new(dtype_of(self.raw.dtype), self.raw.ne, self.raw.nb)
    }

    /// The C-ABI form.
    #[must_use]
    pub const fn as_ffi(&self) -> &ffi::EmelTensorView {
        &self.raw
    }

    /// `Layout::validate` (tensor_view.rs:365-447) of this view against its
    /// own `data_bytes`, on the host; `allow_singleton_zero_stride` admits a
    /// zero stride over an extent of one.
    #[must_use]
    pub fn is_valid(&self, allow_singleton_zero_stride: bool) -> bool {
        // SAFETY: reads the view only; no device access.
        unsafe { ffi::emel_validate_view(&raw const self.raw, i32::from(allow_singleton_zero_stride)) == ffi::EMEL_OK }
    }

    /// The normalisation events' view check (normalization.rs:364-386).
    #[must_use]
    pub fn is_valid_for_normalization(&self) -> bool {
        // SAFETY: reads the view only; no device access.
        unsafe { ffi::emel_validate_normalization_view(&raw const self.raw) == ffi::EMEL_OK }
    }
}

/// A writable device tensor (the reference's `TensorViewMut`).
#[derive(Debug)]
pub struct DeviceViewMut<'a> {
    raw: ffi::EmelTensorViewMut,
    _data: PhantomData<&'a mut [u8]>,
}

impl<'a> DeviceViewMut<'a> {
    /// A view of `layout` over the whole of `buffer`.
    #[must_use]
    pub fn new<T: Copy>(buffer: &'a mut DeviceBuffer<T>, layout: Layout) -> Self {
        let bytes = buffer.byte_len() as u64;
        // SAFETY: the buffer holds `bytes` bytes and is borrowed mutably for 'a.
        unsafe { Self::from_raw(buffer.as_mut_ptr().cast(), bytes, layout) }
    }

    /// A view of `layout` starting `byte_offset` bytes into `buffer`, or
    /// `None` when the offset lies past its end.
    #[must_use]
    pub fn at<T: Copy>(buffer: &'a mut DeviceBuffer<T>, byte_offset: usize, layout: Layout) -> Option<Self> {
        let rest = buffer.byte_len().checked_sub(byte_offset)?;
        // SAFETY: as for DeviceView::at, with the buffer borrowed mutably.
        Some(unsafe { Self::from_raw(buffer.as_mut_ptr().cast::<u8>().add(byte_offset).cast(), rest as u64, layout) })
    }

    /// A writable view over memory this crate did not allocate.
    ///
    /// # Safety
    /// `data` must be a device address of the current device with at least
    /// `data_bytes` writable bytes, valid and not otherwise accessed for 'a.
    #[must_use]
    pub unsafe fn from_raw(data: *mut c_void, data_bytes: u64, layout: Layout) -> Self {
        Self {
            raw: ffi::EmelTensorViewMut {
                data,
                dtype: u32::from(layout.dtype().code()),
                reserved: 0,
                ne: layout.ne(),
                nb: layout.nb(),
                data_bytes,
            },
            _data: PhantomData,
        }
    }

    /// The view's layout.
    #[must_use]
    pub fn layout(&self) -> Layout {
        Layout::new(dtype_of(self.raw.dtype), self.raw.ne, self.raw.nb)
    }

    /// The C-ABI form.
    #[must_use]
    pub const fn as_ffi(&self) -> &ffi::EmelTensorViewMut {
        &self.raw
    }
}

fn dtype_of(code: u32) -> DType {
    // Codes come from DType::code(), a u8.
    DType::from_code(u8::try_from(code).unwrap_or(u8::MAX))
}

/// A dense run of values in device memory (the reference's `&[f32]`, or
/// `&[i32]` with `T = i32`).
#[derive(Clone, Copy, Debug)]
pub struct DeviceSlice<'a, T: Copy = f32> {
    ptr: *const T,
    len: usize,
    _data: PhantomData<&'a [T]>,
}

impl<'a, T: Copy> DeviceSlice<'a, T> {
    /// The whole buffer.
    #[must_use]
    pub const fn new(buffer: &'a DeviceBuffer<T>) -> Self {
        Self { ptr: buffer.as_ptr(), len: buffer.len(), _data: PhantomData }
    }

    /// `len` values from `start`, or `None` past the end.
    #[must_use]
    pub fn sub(self, start: usize, len: usize) -> Option<Self> {
        let end = start.checked_add(len)?;
        if end > self.len {
            return None;
        }
        // SAFETY: start + len <= self.len, inside the allocation.
        Some(Self { ptr: unsafe { self.ptr.add(start) }, len, _data: PhantomData })
    }

    /// Number of values.
    #[must_use]
    pub const fn len(&self) -> usize {
        self.len
    }

    /// Whether the slice is empty.
    #[must_use]
    pub const fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub(crate) const fn ptr(&self) -> *const T {
        self.ptr
    }
}

/// A dense writable run of values (the reference's `&mut [f32]`, or
/// `&mut [i32]` with `T = i32`).
#[derive(Debug)]
pub struct DeviceSliceMut<'a, T: Copy = f32> {
    ptr: *mut T,
    len: usize,
    _data: PhantomData<&'a mut [T]>,
}

impl<'a, T: Copy> DeviceSliceMut<'a, T> {
    /// The whole buffer.
    #[must_use]
    pub const fn new(buffer: &'a mut DeviceBuffer<T>) -> Self {
        let len = buffer.len();
        Self { ptr: buffer.as_mut_ptr(), len, _data: PhantomData }
    }

    /// `len` values from `start`, or `None` past the end.
    #[must_use]
    pub fn sub(self, start: usize, len: usize) -> Option<Self> {
        let end = start.checked_add(len)?;
        if end > self.len {
            return None;
        }
        // SAFETY: start + len <= self.len, inside the allocation.
        Some(Self { ptr: unsafe { self.ptr.add(start) }, len, _data: PhantomData })
    }

    /// Number of values.
    #[must_use]
    pub const fn len(&self) -> usize {
        self.len
    }

    /// Whether the slice is empty.
    #[must_use]
    pub const fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub(crate) const fn ptr(&self) -> *mut T {
        self.ptr
    }
}

/// Where the index values of a [`DeviceIndexView`] live.
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub enum IndexMemory<'a> {
    /// Host memory: up to `EMEL_GET_ROWS_INLINE_INDICES` values travel in the
    /// kernel arguments, more are uploaded by the call.
    Host(&'a [i32]),
    /// Device memory: the call copies the span to the host to check it.
    Device(*const i32, usize),
}

/// The reference's `IndexView` (get_rows.rs:35-160): I32 row indices with
/// three extents and, optionally, explicit byte strides.
#[derive(Clone, Copy, Debug)]
pub struct DeviceIndexView<'a> {
    raw: ffi::EmelIndexView,
    _data: PhantomData<&'a [i32]>,
}

impl<'a> DeviceIndexView<'a> {
    /// Row-major indices (`IndexView::new`).
    #[must_use]
    pub fn new(data: IndexMemory<'a>, ne: [u64; 3]) -> Self {
        Self::build(data, ne, [0; 3], false)
    }

    /// Indices with explicit byte strides (`IndexView::with_strides`;
    /// `byte_strides[0] == 0` selects the contiguous form).
    #[must_use]
    pub fn with_strides(data: IndexMemory<'a>, ne: [u64; 3], byte_strides: [u64; 3]) -> Self {
        Self::build(data, ne, byte_strides, true)
    }

    /// Indices resident in device memory.
    ///
    /// # Safety
    /// `data` must address `len` readable i32 values on the current device,
    /// valid for 'a.
    #[must_use]
    pub const unsafe fn device(data: *const i32, len: usize) -> IndexMemory<'a> {
        IndexMemory::Device(data, len)
    }

    fn build(data: IndexMemory<'a>, ne: [u64; 3], nb: [u64; 3], explicit: bool) -> Self {
        let (ptr, len, on_host) = match data {
            IndexMemory::Host(values) => (values.as_ptr(), values.len(), 1),
            IndexMemory::Device(ptr, len) => (ptr, len, 0),
        };
        Self {
            raw: ffi::EmelIndexView {
                data: ptr,
                len: len as u64,
                ne,
                nb,
                explicit_strides: u32::from(explicit),
                on_host,
            },
            _data: PhantomData,
        }
    }

    /// The C-ABI form.
    #[must_use]
    pub const fn as_ffi(&self) -> &ffi::EmelIndexView {
        &self.raw
    }
}
