// api.cpp -- the C ABI declared in include/emel_hip.h.
//
// Every entry point follows the reference actor's order: the guards run on
// the host first (view validity, then shape, then parameters, classified
// into the same error variants the Rust actors return), and only an
// accepted request reaches the device.  A rejected request enqueues nothing
// and never writes dst.  There is no CPU fallback.
#include "emel_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "launch.hpp"

namespace {

using u128 = unsigned __int128;
using emel::Operand;

thread_local std::string g_last_error;

emel_status fail(emel_status s, const std::string &why)
{
    g_last_error = why;
    return s;
}

emel_status hip_fail(hipError_t e, const char *what)
{
    return fail(EMEL_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// ---- view rules (tensor_view.rs) ------------------------------------------

template <class V>
bool element_count(const V &v, uint64_t &count)
{
    u128 c = 1;
    for (int d = 0; d < 4; ++d) {
        if (v.ne[d] == 0) return false;
        c *= v.ne[d];
        if (c > static_cast<u128>(UINT64_MAX)) return false;
    }
    count = static_cast<uint64_t>(c);
    return true;
}

template <class V>
uint64_t count_or_zero(const V &v)
{
    uint64_t c = 0;
    return element_count(v, c) ? c : 0;
}

// Layout::effective_f32_strides (tensor_view.rs:262-277): nb[0] == 0 means
// row-major; defined for F32 only.
template <class V>
bool effective_f32_strides(const V &v, uint64_t st[4])
{
    if (v.dtype != EMEL_DTYPE_F32) return false;
    if (v.nb[0] != 0) {
        for (int d = 0; d < 4; ++d) st[d] = v.nb[d];
        return true;
    }
    u128 s = 4;
    st[0] = 4;
    for (int d = 1; d < 4; ++d) {
        s *= v.ne[d - 1];
        if (s > static_cast<u128>(UINT64_MAX)) return false;
        st[d] = static_cast<uint64_t>(s);
    }
    return true;
}

template <class V>
bool span_fits(const V &v, const uint64_t st[4], uint64_t elem)
{
    u128 max_offset = 0;
    for (int d = 0; d < 4; ++d) max_offset += static_cast<u128>(v.ne[d] - 1) * st[d];
    return max_offset + elem <= static_cast<u128>(v.data_bytes);
}

// Layout::validate_element_storage (tensor_view.rs:397-447) for F32 views;
// allow_zero selects validate_binary's singleton-zero-stride allowance.
template <class V>
bool valid_f32(const V &v, bool allow_zero)
{
    uint64_t count, st[4];
    if (v.dtype != EMEL_DTYPE_F32 || v.reserved != 0) return false;
    if (!element_count(v, count)) return false;
    if (!effective_f32_strides(v, st)) return false;
    for (int d = 0; d < 4; ++d) {
        const bool singleton_zero = allow_zero && v.ne[d] == 1 && st[d] == 0;
        if (!singleton_zero && (st[d] < 4 || st[d] % 4 != 0)) return false;
    }
    return span_fits(v, st, 4);
}

// Layout::validate_i32 (tensor_view.rs:384-395): strides as given.
template <class V>
bool valid_i32(const V &v)
{
    uint64_t count;
    if (v.dtype != EMEL_DTYPE_I32 || v.reserved != 0) return false;
    if (!element_count(v, count)) return false;
    for (int d = 0; d < 4; ++d)
        if (v.nb[d] < 4 || v.nb[d] % 4 != 0) return false;
    return span_fits(v, v.nb, 4);
}

// normalization_view_valid (normalization.rs:237-287).
template <class V>
bool valid_normalization(const V &v)
{
    if (v.dtype != EMEL_DTYPE_F32 || v.reserved != 0 || v.ne[0] == 0) return false;
    if (v.nb[0] != 0) {
        if (v.nb[0] < 4 || v.nb[0] % 4 != 0) return false;
        for (int d = 0; d < 4; ++d)
            if (v.ne[d] > 1 && v.nb[d] == 0) return false;
    }
    for (int d = 0; d < 4; ++d)
        if (v.ne[d] == 0) return false;
    uint64_t st[4];
    if (!effective_f32_strides(v, st)) return false;
    for (int d = 0; d < 4; ++d)
        if (st[d] < 4 || st[d] % 4 != 0) return false;
    return span_fits(v, st, 4);
}

// soft_max_dense_layout (reductions.rs:488-495).
template <class V>
bool soft_max_dense_layout(const V &v)
{
    uint64_t st[4];
    if (v.nb[0] == 0) return effective_f32_strides(v, st);
    if (v.dtype != EMEL_DTYPE_F32) return false;
    u128 expect = 4;
    for (int d = 0; d < 4; ++d) {
        if (v.nb[d] != expect) return false;
        expect *= v.ne[d];
        if (expect > static_cast<u128>(UINT64_MAX)) return false;
    }
    return true;
}

template <class A, class B>
bool same_ne(const A &a, const B &b)
{
    for (int d = 0; d < 4; ++d)
        if (a.ne[d] != b.ne[d]) return false;
    return true;
}

// Byte range [lo, hi) a validated view touches.
template <class V>
std::pair<uintptr_t, uintptr_t> byte_range(const V &v, uint64_t elem)
{
    uint64_t st[4];
    if (!effective_f32_strides(v, st)) std::memcpy(st, v.nb, sizeof st);
    u128 max_offset = 0;
    for (int d = 0; d < 4; ++d) max_offset += static_cast<u128>(v.ne[d] - 1) * st[d];
    const uintptr_t lo = reinterpret_cast<uintptr_t>(v.data);
    return {lo, lo + static_cast<uintptr_t>(max_offset) + elem};
}

// dst may be exactly a source (same address and layout); any other overlap
// with a source would make the result depend on thread order.
template <class S>
bool overlap_ok(const emel_tensor_view_mut &dst, uint64_t delem, const S &src, uint64_t selem)
{
    const auto d = byte_range(dst, delem);
    const auto s = byte_range(src, selem);
    if (d.second <= s.first || s.second <= d.first) return true;
    return dst.data == src.data && delem == selem && same_ne(dst, src) &&
           std::memcmp(dst.nb, src.nb, sizeof dst.nb) == 0;
}

// Whether no two elements of a validated view share a byte, by the
// sufficient rule: with the dims of extent > 1 sorted by stride, each stride
// is at least the span of the dims below it.  The reference's sequential
// loops accept any layout and keep the last write to a shared element; the
// device writes in parallel, so a view that fails this rule is refused
// rather than written in an unspecified order.
template <class V>
bool elements_disjoint(const V &v, uint64_t elem)
{
    uint64_t st[4];
    if (!effective_f32_strides(v, st)) std::memcpy(st, v.nb, sizeof st);
    int dims[4];
    int n = 0;
    for (int d = 0; d < 4; ++d)
        if (v.ne[d] > 1) dims[n++] = d;
    for (int i = 1; i < n; ++i)
        for (int j = i; j > 0 && st[dims[j]] < st[dims[j - 1]]; --j) std::swap(dims[j], dims[j - 1]);
    u128 span = elem;
    for (int i = 0; i < n; ++i) {
        const int d = dims[i];
        if (static_cast<u128>(st[d]) < span) return false;
        span += static_cast<u128>(v.ne[d] - 1) * st[d];
    }
    return true;
}

template <class V>
Operand operand(const V &v, uint64_t elem)
{
    Operand o{};
    o.data = const_cast<void *>(static_cast<const void *>(v.data));
    uint64_t st[4];
    if (!effective_f32_strides(v, st)) std::memcpy(st, v.nb, sizeof st);
    for (int d = 0; d < 4; ++d) {
        o.ne[d] = v.ne[d];
        o.st[d] = static_cast<int64_t>(st[d] / elem);
    }
    return o;
}

// ---- device ------------------------------------------------------------------

std::mutex g_mutex;
std::map<int, bool> g_device_ok; // device -> is gfx950

emel_status ensure_device()
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(EMEL_ERR_KERNEL_UNAVAILABLE, std::string("no HIP device: ") + hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_device_ok.find(dev);
    if (it == g_device_ok.end()) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        const bool ok = e == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
        it = g_device_ok.emplace(dev, ok).first;
    }
    if (!it->second) return fail(EMEL_ERR_KERNEL_UNAVAILABLE, "the current HIP device is not gfx950");
    return EMEL_OK;
}

// ---- per-(device, stream) scratch ------------------------------------------
//
// Calls on one stream run in order on the device, so they share one set of
// scratch buffers per (device, stream).  A call holds the stream's lock from
// its first use of that scratch until its last launch is enqueued, so calls
// from several host threads on one stream never interleave their launch
// sequences or their index checks.
//   - `work`: general scratch (reduction partials, sampler state, uploaded
//     indices); each call fully writes what it later reads.
//   - `counters`: the reductions' per-row arrival counters.  They are zeroed
//     when the buffer is allocated and every launch leaves them zero, so the
//     buffer holds nothing else.
//   - `staging`: pinned host memory for index copies back to the host.
// A buffer that must grow is replaced, and the old one is kept until
// emel_release_workspaces or emel_stream_destroy: a graph captured earlier
// may still reference it.  Growth allocates and zeroes memory, which a stream
// under capture must not do, so a call that needs it during a capture is
// refused with EMEL_ERR_STREAM_CAPTURE before anything is enqueued.
struct Buffer {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

struct StreamState {
    std::mutex lock;
    Buffer work, counters, staging;
    std::vector<void *> retired_dev, retired_host;
};

std::map<std::pair<int, hipStream_t>, std::unique_ptr<StreamState>> g_streams; // guarded by g_mutex

emel_status not_capturing(hipStream_t stream, const char *what)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
        return fail(EMEL_ERR_STREAM_CAPTURE, std::string(what) + " cannot run while the stream is being captured");
    return EMEL_OK;
}

class StreamLease {
public:
    emel_status acquire(hipStream_t stream)
    {
        int dev = 0;
        const hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
        {
            std::lock_guard<std::mutex> g(g_mutex);
            auto &slot = g_streams[{dev, stream}];
            if (!slot) slot.reset(new StreamState);
            st_ = slot.get();
        }
        hold_ = std::unique_lock<std::mutex>(st_->lock);
        stream_ = stream;
        return EMEL_OK;
    }

    emel_status work(uint64_t bytes, void **out) { return device(st_->work, bytes, false, out); }
    emel_status counters(uint64_t bytes, void **out) { return device(st_->counters, bytes, true, out); }

    emel_status staging(uint64_t bytes, void **out)
    {
        *out = nullptr;
        Buffer &b = st_->staging;
        if (b.bytes < bytes) {
            emel_status s = not_capturing(stream_, "growing the pinned index staging buffer");
            if (s != EMEL_OK) return s;
            void *p = nullptr;
            const uint64_t size = grown(b.bytes, bytes, uint64_t{1} << 16);
            const hipError_t e = hipHostMalloc(&p, size, hipHostMallocDefault);
            if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(staging)");
            if (b.ptr) st_->retired_host.push_back(b.ptr);
            b.ptr = p;
            b.bytes = size;
        }
        *out = b.ptr;
        return EMEL_OK;
    }

private:
    static uint64_t grown(uint64_t have, uint64_t need, uint64_t floor)
    {
        uint64_t size = have * 2 > need ? have * 2 : need;
        return size < floor ? floor : size;
    }

    emel_status device(Buffer &b, uint64_t bytes, bool zeroed, void **out)
    {
        *out = nullptr;
        if (bytes == 0) return EMEL_OK;
        if (b.bytes < bytes) {
            emel_status s = not_capturing(stream_, "growing the stream's device scratch");
            if (s != EMEL_OK) return s;
            void *p = nullptr;
            const uint64_t size = grown(b.bytes, bytes, uint64_t{1} << 20);
            hipError_t e = hipMalloc(&p, size);
            if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch)");
            if (zeroed) {
                e = hipMemsetAsync(p, 0, size, stream_); // ordered before this call's launches
                if (e != hipSuccess) {
                    (void)hipFree(p);
                    return hip_fail(e, "hipMemsetAsync(scratch)");
                }
            }
            if (b.ptr) st_->retired_dev.push_back(b.ptr);
            b.ptr = p;
            b.bytes = size;
        }
        *out = b.ptr;
        return EMEL_OK;
    }

    StreamState *st_ = nullptr;
    std::unique_lock<std::mutex> hold_;
    hipStream_t stream_ = nullptr;
};

// Frees every buffer of `st` (the caller has synchronised the device or the
// stream).
void free_state(StreamState &st)
{
    for (Buffer *b : {&st.work, &st.counters}) {
        if (b->ptr) (void)hipFree(b->ptr);
        *b = Buffer{};
    }
    if (st.staging.ptr) (void)hipHostFree(st.staging.ptr);
    st.staging = Buffer{};
    for (void *p : st.retired_dev) (void)hipFree(p);
    for (void *p : st.retired_host) (void)hipHostFree(p);
    st.retired_dev.clear();
    st.retired_host.clear();
}

emel_status launched(hipError_t e)
{
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(EMEL_ERR_STREAM_CAPTURE, "a step the call needs is not permitted while the stream is being "
                                             "captured (the first GELU on a device builds its table and waits)");
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    g_last_error.clear();
    return EMEL_OK;
}

hipStream_t as_stream(emel_stream s) { return static_cast<hipStream_t>(s); }

// ---- op plumbing ---------------------------------------------------------------

emel_status elementwise(emel::Ew op, const emel_tensor_view *a, emel::Addr aa, const emel_tensor_view *b,
                        emel::Addr ba, const emel_tensor_view_mut *o, float scale, emel_stream stream,
                        float scale2 = 0.0f)
{
    if (!overlap_ok(*o, 4, *a, 4) || (b && !overlap_ok(*o, 4, *b, 4)))
        return fail(EMEL_ERR_INVALID_VIEW, "dst partially overlaps a source");
    if (!elements_disjoint(*o, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst elements overlap one another");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::EwArgs args{};
    args.op = op;
    args.scale = scale;
    args.scale2 = scale2;
    args.a = operand(*a, 4);
    if (b) args.b = operand(*b, 4);
    args.o = operand(*o, 4);
    args.a_addr = aa;
    args.b_addr = ba;
    args.count = count_or_zero(*o);
    return launched(emel::launch_elementwise(args, as_stream(stream)));
}

emel::Addr pair_addr(const emel_tensor_view &src, const emel_tensor_view_mut &dst)
{
    return same_ne(src, dst) ? emel::Addr::SameCoords : emel::Addr::Ordinal;
}

// binary.rs:320-340: views_valid (validate_binary) then equal counts.
emel_status binary(emel::Ew op, const emel_tensor_view *lhs, const emel_tensor_view *rhs,
                   const emel_tensor_view_mut *out, emel_stream stream)
{
    if (!lhs || !rhs || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*lhs, true) || !valid_f32(*rhs, true) || !valid_f32(*out, true))
        return fail(EMEL_ERR_INVALID_VIEW, "binary view failed validation");
    const uint64_t n = count_or_zero(*out);
    if (count_or_zero(*lhs) != count_or_zero(*rhs) || count_or_zero(*lhs) != n)
        return fail(EMEL_ERR_SHAPE_MISMATCH, "binary element counts differ");
    return elementwise(op, lhs, pair_addr(*lhs, *out), rhs, pair_addr(*rhs, *out), out, 1.0f, stream);
}

// broadcast.rs:321-350.
template <class O>
emel_status broadcast_row_guard(const emel_tensor_view &src0, const emel_tensor_view &src1, const O &dst)
{
    if (!valid_f32(src0, true) || !valid_f32(src1, true) || !valid_f32(dst, true))
        return fail(EMEL_ERR_INVALID_VIEW, "broadcast view failed validation");
    const uint64_t *d = dst.ne, *r = src1.ne;
    if (!(same_ne(src0, dst) && d[0] > 0 && r[0] == d[0] && r[1] == 1 && r[2] == 1 && r[3] == 1 && d[1] > 0 &&
          count_or_zero(dst) > count_or_zero(src1)))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "broadcast shapes do not match the row contract");
    return EMEL_OK;
}

emel_status broadcast_row(emel::Ew op, const emel_tensor_view *src0, const emel_tensor_view *src1,
                          const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src0 || !src1 || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    emel_status s = broadcast_row_guard(*src0, *src1, *dst);
    if (s != EMEL_OK) return s;
    return elementwise(op, src0, emel::Addr::SameCoords, src1, emel::Addr::Broadcast, dst, 1.0f, stream);
}

bool unary_accepted(emel_unary_subop s)
{
    return s == EMEL_UNARY_ABS || s == EMEL_UNARY_NEG || s == EMEL_UNARY_TANH || s == EMEL_UNARY_ELU ||
           s == EMEL_UNARY_RELU || s == EMEL_UNARY_GELU || s == EMEL_UNARY_SILU || s == EMEL_UNARY_EXP;
}

emel::Ew unary_fn(emel_unary_subop s)
{
    switch (s) {
    case EMEL_UNARY_ABS: return emel::Ew::Abs;
    case EMEL_UNARY_NEG: return emel::Ew::Neg;
    case EMEL_UNARY_TANH: return emel::Ew::Tanh;
    case EMEL_UNARY_ELU: return emel::Ew::Elu;
    case EMEL_UNARY_RELU: return emel::Ew::Relu;
    case EMEL_UNARY_SIGMOID: return emel::Ew::Sigmoid;
    case EMEL_UNARY_GELU: return emel::Ew::Gelu;
    case EMEL_UNARY_SILU: return emel::Ew::Silu;
    default: return emel::Ew::Exp;
    }
}

// Dedicated unary events (impl_unary_context, unary.rs:702-728).
emel_status unary_event(emel::Ew fn, const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*in, false) || !valid_f32(*out, false))
        return fail(EMEL_ERR_INVALID_VIEW, "unary view failed validation");
    if (count_or_zero(*in) != count_or_zero(*out))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "unary element counts differ");
    return elementwise(fn, in, pair_addr(*in, *out), nullptr, emel::Addr::SameCoords, out, 1.0f, stream);
}

emel_status rows(const emel::RowArgs &args, const emel_tensor_view &in, const emel_tensor_view_mut &out,
                 const emel_tensor_view *extra, emel_stream stream)
{
    if (!overlap_ok(out, 4, in, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst partially overlaps the source");
    if (extra && !overlap_ok(out, 4, *extra, extra->dtype == EMEL_DTYPE_F16 ? 2 : 4))
        return fail(EMEL_ERR_INVALID_VIEW, "dst overlaps an operand");
    if (!elements_disjoint(out, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst elements overlap one another");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    return launched(emel::launch_rows(args, as_stream(stream)));
}

emel_status reduce(emel::RedOp op, const emel_tensor_view &src, const emel_tensor_view_mut &dst, emel_stream stream,
                   bool static_scratch = false)
{
    if (!overlap_ok(dst, 4, src, 4) || dst.data == src.data)
        return fail(EMEL_ERR_INVALID_VIEW, "dst overlaps the source");
    if (!elements_disjoint(dst, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst elements overlap one another");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::RedArgs args{};
    args.op = op;
    args.x = operand(src, 4);
    args.dst = dst.data;
    args.dst_view = operand(dst, 4);
    if (dst.dtype == EMEL_DTYPE_I32)
        for (int d = 0; d < 4; ++d) args.dst_view.st[d] = static_cast<int64_t>(dst.nb[d] / 4);
    args.scratch = emel::reduce_scratch_bytes(args);
    StreamLease lease;
    if (static_scratch) {
        const hipError_t e = emel::reduce_static_scratch(args, as_stream(stream));
        if (e == hipErrorOutOfMemory)
            return fail(EMEL_ERR_INVALID_PARAMETERS, "the reduction needs more scratch than the allocation-free "
                                                     "entry point's static 64 KiB partials / 64 KiB counters");
        if (e != hipSuccess) return hip_fail(e, "setting up the static reduction scratch");
    } else if (args.scratch.partials) {
        s = lease.acquire(as_stream(stream));
        if (s == EMEL_OK) s = lease.work(args.scratch.partials, &args.partials);
        if (s == EMEL_OK) s = lease.counters(args.scratch.counters, &args.counters);
        if (s != EMEL_OK) return s;
    }
    const hipError_t e = emel::launch_reduce(args, as_stream(stream));
    if (e == hipErrorInvalidValue) return fail(EMEL_ERR_INTERNAL, "reduction size outside the supported range");
    return launched(e);
}

bool scalar_dst(const emel_tensor_view_mut &d) { return d.ne[0] == 1 && d.ne[1] == 1 && d.ne[2] == 1 && d.ne[3] == 1; }

template <class S, class D>
bool rows_dst(const S &s, const D &d)
{
    return d.ne[0] == 1 && d.ne[1] == s.ne[1] && d.ne[2] == s.ne[2] && d.ne[3] == s.ne[3];
}

emel_status norm_guard(const emel_tensor_view *in, const emel_tensor_view_mut *out, float eps)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_normalization(*in) || !valid_normalization(*out))
        return fail(EMEL_ERR_INVALID_VIEW, "normalization view failed validation");
    if (!same_ne(*in, *out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "normalization shapes differ");
    if (!(std::isfinite(eps) && eps >= 0.0f))
        return fail(EMEL_ERR_INVALID_PARAMETERS, "epsilon must be finite and non-negative");
    return EMEL_OK;
}

emel_status norm_op(emel::RowOp op, const emel_tensor_view *in, const emel_tensor_view *w,
                    const emel_tensor_view_mut *out, float eps, emel_stream stream)
{
    emel_status s = norm_guard(in, out, eps);
    if (s != EMEL_OK) return s;
    emel::RowArgs args{};
    args.op = op;
    args.x = operand(*in, 4);
    args.y = operand(*out, 4);
    args.eps = eps;
    if (op == emel::RowOp::RmsNormMul) {
        if (!w) return fail(EMEL_ERR_INVALID_ARGUMENT, "null weight view");
        s = broadcast_row_guard(*reinterpret_cast<const emel_tensor_view *>(out), *w, *out);
        if (s != EMEL_OK) return s;
        const Operand wo = operand(*w, 4);
        args.w = static_cast<const float *>(wo.data);
        args.w_st0 = wo.st[0];
    }
    return rows(args, *in, *out, w, stream);
}

} // namespace

// The entry points below take C language linkage from their declarations in
// emel_hip.h; the helper namespaces between them stay internal.

uint32_t emel_abi_version(void) { return EMEL_HIP_ABI_VERSION; }

const char *emel_status_string(emel_status s)
{
    switch (s) {
    case EMEL_OK: return "ok";
    case EMEL_ERR_INVALID_VIEW: return "invalid tensor view";
    case EMEL_ERR_SHAPE_MISMATCH: return "tensor shapes differ";
    case EMEL_ERR_INVALID_PARAMETERS: return "invalid parameters";
    case EMEL_ERR_UNEXPECTED_EVENT: return "unexpected event";
    case EMEL_ERR_INTERNAL: return "internal dispatch error";
    case EMEL_ERR_KERNEL_UNAVAILABLE: return "kernel unavailable (no gfx950 device)";
    case EMEL_ERR_DEVICE: return "HIP runtime error";
    case EMEL_ERR_INVALID_ARGUMENT: return "invalid argument";
    case EMEL_ERR_INVALID_SHAPE: return "invalid kernel shape";
    case EMEL_ERR_UNSUPPORTED_OPERATION: return "unsupported operation";
    case EMEL_ERR_INDEX_OUT_OF_BOUNDS: return "index out of bounds";
    case EMEL_ERR_UNSUPPORTED_SOURCE_STRIDE: return "unsupported source stride";
    case EMEL_ERR_INVALID_REQUEST: return "invalid request";
    case EMEL_ERR_STREAM_CAPTURE: return "not capturable: the stream is being captured";
    case EMEL_ERR_INVALID_OFFSET: return "invalid offset";
    case EMEL_ERR_ZERO_NORM: return "zero norm";
    }
    return "unknown status";
}

const char *emel_last_error(void) { return g_last_error.c_str(); }

emel_status emel_device_count(int32_t *count)
{
    if (!count) return fail(EMEL_ERR_INVALID_ARGUMENT, "null count");
    *count = 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return EMEL_OK;
    int32_t ok = 0;
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++ok;
    }
    *count = ok;
    return EMEL_OK;
}

emel_status emel_set_device(int32_t device)
{
    const hipError_t e = hipSetDevice(device);
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipSetDevice");
}

emel_status emel_malloc(void **ptr, uint64_t bytes)
{
    if (!ptr) return fail(EMEL_ERR_INVALID_ARGUMENT, "null pointer");
    const hipError_t e = hipMalloc(ptr, bytes);
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipMalloc");
}

emel_status emel_free(void *ptr)
{
    const hipError_t e = hipFree(ptr);
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipFree");
}

emel_status emel_memcpy_htod(void *dst, const void *src, uint64_t bytes, emel_stream stream)
{
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipMemcpyAsync(HtoD)");
}

emel_status emel_memcpy_dtoh(void *dst, const void *src, uint64_t bytes, emel_stream stream)
{
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipMemcpyAsync(DtoH)");
}

emel_status emel_stream_create(emel_stream *stream)
{
    if (!stream) return fail(EMEL_ERR_INVALID_ARGUMENT, "null stream pointer");
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
    *stream = s;
    return EMEL_OK;
}

emel_status emel_stream_destroy(emel_stream stream)
{
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        for (auto it = g_streams.begin(); it != g_streams.end();) {
            if (it->first.second == as_stream(stream)) {
                (void)hipStreamSynchronize(as_stream(stream));
                free_state(*it->second);
                it = g_streams.erase(it);
            } else {
                ++it;
            }
        }
    }
    const hipError_t e = hipStreamDestroy(as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipStreamDestroy");
}

emel_status emel_stream_synchronize(emel_stream stream)
{
    const hipError_t e = hipStreamSynchronize(as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipStreamSynchronize");
}

emel_status emel_release_workspaces(void)
{
    std::lock_guard<std::mutex> lock(g_mutex);
    hipError_t e = hipDeviceSynchronize();
    for (auto &kv : g_streams) free_state(*kv.second);
    g_streams.clear();
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipDeviceSynchronize");
}

emel_status emel_stream_reserve(emel_stream stream, uint64_t work_bytes, uint64_t counter_bytes)
{
    const emel_status d = ensure_device();
    if (d != EMEL_OK) return d;
    emel_status s = not_capturing(as_stream(stream), "reserving a stream's scratch");
    if (s != EMEL_OK) return s;
    StreamLease lease;
    s = lease.acquire(as_stream(stream));
    if (s != EMEL_OK) return s;
    void *p = nullptr;
    s = lease.work(work_bytes, &p);
    if (s != EMEL_OK) return s;
    return lease.counters(counter_bytes, &p);
}

emel_status emel_stream_workspace(emel_stream stream, uint64_t *work_bytes, uint64_t *counter_bytes)
{
    if (!work_bytes || !counter_bytes) return fail(EMEL_ERR_INVALID_ARGUMENT, "null size pointer");
    *work_bytes = 0;
    *counter_bytes = 0;
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    // g_mutex, then the stream's lock: no thread takes them in the other
    // order, and holding g_mutex keeps the state from being released
    std::lock_guard<std::mutex> g(g_mutex);
    const auto it = g_streams.find({dev, as_stream(stream)});
    if (it == g_streams.end()) return EMEL_OK;
    std::lock_guard<std::mutex> hold(it->second->lock);
    *work_bytes = it->second->work.bytes;
    *counter_bytes = it->second->counters.bytes;
    return EMEL_OK;
}

emel_status emel_device_prepare(emel_stream stream)
{
    const emel_status d = ensure_device();
    if (d != EMEL_OK) return d;
    const emel_status s = not_capturing(as_stream(stream), "building the device's tables");
    if (s != EMEL_OK) return s;
    const hipError_t e = emel::prepare_device_tables(as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "building the device's tables");
}

emel_status emel_stream_copy(const void *src, void *dst, uint64_t bytes, uint32_t shape, emel_stream stream)
{
    if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15u) != 0)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "stream copy: bytes and both pointers must be multiples of 16");
    if (bytes != 0 && (!src || !dst)) return fail(EMEL_ERR_INVALID_ARGUMENT, "stream copy: null pointer");
    if (shape > EMEL_COPY_WALK) return fail(EMEL_ERR_INVALID_ARGUMENT, "stream copy: unknown shape");
    const emel_status d = ensure_device();
    if (d != EMEL_OK) return d;
    const hipError_t e = emel::launch_stream_copy(src, dst, bytes, static_cast<emel::CopyShape>(shape), as_stream(stream));
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "stream copy launch");
}

emel_status emel_validate_view(const emel_tensor_view *view, int32_t allow_singleton_zero_stride)
{
    if (!view) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    return valid_f32(*view, allow_singleton_zero_stride != 0) ? EMEL_OK : EMEL_ERR_INVALID_VIEW;
}

emel_status emel_validate_normalization_view(const emel_tensor_view *view)
{
    if (!view) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    return valid_normalization(*view) ? EMEL_OK : EMEL_ERR_INVALID_VIEW;
}

emel_status emel_op_add(const emel_tensor_view *l, const emel_tensor_view *r, const emel_tensor_view_mut *o, emel_stream s)
{
    return binary(emel::Ew::Add, l, r, o, s);
}
emel_status emel_op_sub(const emel_tensor_view *l, const emel_tensor_view *r, const emel_tensor_view_mut *o, emel_stream s)
{
    return binary(emel::Ew::Sub, l, r, o, s);
}
emel_status emel_op_mul(const emel_tensor_view *l, const emel_tensor_view *r, const emel_tensor_view_mut *o, emel_stream s)
{
    return binary(emel::Ew::Mul, l, r, o, s);
}
emel_status emel_op_div(const emel_tensor_view *l, const emel_tensor_view *r, const emel_tensor_view_mut *o, emel_stream s)
{
    return binary(emel::Ew::Div, l, r, o, s);
}

emel_status emel_op_add_broadcast_row(const emel_tensor_view *a, const emel_tensor_view *b,
                                      const emel_tensor_view_mut *d, emel_stream s)
{
    return broadcast_row(emel::Ew::Add, a, b, d, s);
}

emel_status emel_op_mul_broadcast_row(const emel_tensor_view *a, const emel_tensor_view *b,
                                      const emel_tensor_view_mut *d, emel_stream s)
{
    return broadcast_row(emel::Ew::Mul, a, b, d, s);
}

emel_status emel_op_binary_broadcast(emel_binary_op op, const emel_tensor_view *src0, const emel_tensor_view *src1,
                                     const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src0 || !src1 || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (op < EMEL_BINARY_ADD || op > EMEL_BINARY_DIV) return fail(EMEL_ERR_UNEXPECTED_EVENT, "unknown binary op");
    // OpRepeat's source contract (f32_valid, generic.rs:471-476) and the
    // binary op's contract for src0 and dst.
    if (!valid_f32(*src0, true) || !valid_f32(*src1, false) || !valid_f32(*dst, true))
        return fail(EMEL_ERR_INVALID_VIEW, "broadcast view failed validation");
    if (!same_ne(*src0, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "src0 and dst shapes differ");
    for (int d = 0; d < 4; ++d)
        if (dst->ne[d] % src1->ne[d] != 0)
            return fail(EMEL_ERR_SHAPE_MISMATCH, "src1 extents do not divide dst extents");
    static const emel::Ew fns[4] = {emel::Ew::Add, emel::Ew::Sub, emel::Ew::Mul, emel::Ew::Div};
    return elementwise(fns[op], src0, emel::Addr::SameCoords, src1, emel::Addr::Broadcast, dst, 1.0f, stream);
}

emel_status emel_op_unary(emel_unary_subop subop, const emel_tensor_view *in, const emel_tensor_view_mut *out,
                          emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // OpUnary reports every failed guard as UnexpectedEvent (unary.rs:1014-1027).
    if (!unary_accepted(subop) || !valid_f32(*in, false) || !valid_f32(*out, false) ||
        count_or_zero(*in) != count_or_zero(*out))
        return fail(EMEL_ERR_UNEXPECTED_EVENT, "op_unary request rejected");
    return elementwise(unary_fn(subop), in, pair_addr(*in, *out), nullptr, emel::Addr::SameCoords, out, 1.0f, stream);
}

emel_status emel_op_silu(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream s)
{
    return unary_event(emel::Ew::Silu, in, out, s);
}

emel_status emel_op_gelu(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream s)
{
    return unary_event(emel::Ew::Gelu, in, out, s);
}

// The 21 typed unary events, keyed by the UnarySubOp wire code of the
// formula each applies (unary.rs:72-92, formulas :472-610).  Xielu (17) has
// no typed event.
emel_status emel_op_unary_event(uint32_t event, const emel_tensor_view *in, const emel_tensor_view_mut *out,
                                emel_stream s)
{
    emel::Ew fn;
    switch (event) {
    case EMEL_UNARY_ABS: fn = emel::Ew::Abs; break;
    case EMEL_UNARY_SGN: fn = emel::Ew::Sgn; break;
    case EMEL_UNARY_NEG: fn = emel::Ew::Neg; break;
    case EMEL_UNARY_STEP: fn = emel::Ew::Step; break;
    case EMEL_UNARY_TANH: fn = emel::Ew::Tanh; break;
    case EMEL_UNARY_ELU: fn = emel::Ew::Elu; break;
    case EMEL_UNARY_RELU: fn = emel::Ew::Relu; break;
    case EMEL_UNARY_SIGMOID: fn = emel::Ew::Sigmoid; break;
    case EMEL_UNARY_GELU: fn = emel::Ew::Gelu; break;
    case EMEL_UNARY_GELU_QUICK: fn = emel::Ew::GeluQuick; break;
    case EMEL_UNARY_SILU: fn = emel::Ew::Silu; break;
    case EMEL_UNARY_HARDSWISH: fn = emel::Ew::Hardswish; break;
    case EMEL_UNARY_HARDSIGMOID: fn = emel::Ew::Hardsigmoid; break;
    case EMEL_UNARY_EXP: fn = emel::Ew::Exp; break;
    case EMEL_UNARY_EXPM1: fn = emel::Ew::Expm1; break;
    case EMEL_UNARY_SOFTPLUS: fn = emel::Ew::Softplus; break;
    case EMEL_UNARY_GELU_ERF: fn = emel::Ew::GeluErf; break;
    case EMEL_UNARY_FLOOR: fn = emel::Ew::Floor; break;
    case EMEL_UNARY_CEIL: fn = emel::Ew::Ceil; break;
    case EMEL_UNARY_ROUND: fn = emel::Ew::Round; break;
    case EMEL_UNARY_TRUNC: fn = emel::Ew::Trunc; break;
    default: return fail(EMEL_ERR_UNEXPECTED_EVENT, "no typed unary event has this code");
    }
    return unary_event(fn, in, out, s);
}

// reductions::OpLog / OpSin / OpCos (reductions.rs:45-90, guards :508-517,
// effects :640-668): views valid, equal element counts, elementwise by
// ordinal; ReductionError's InvalidView / ShapeMismatch.
emel_status emel_op_log(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream s)
{
    return unary_event(emel::Ew::Log, in, out, s);
}

emel_status emel_op_sin(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream s)
{
    return unary_event(emel::Ew::Sin, in, out, s);
}

emel_status emel_op_cos(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream s)
{
    return unary_event(emel::Ew::Cos, in, out, s);
}

emel_status emel_op_swiglu(const emel_tensor_view *gate, const emel_tensor_view *up, const emel_tensor_view_mut *out,
                           emel_stream stream)
{
    if (!gate || !up || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // OpSilu's contract for gate, then OpMul's for up and out.
    if (!valid_f32(*gate, false) || !valid_f32(*up, true) || !valid_f32(*out, true))
        return fail(EMEL_ERR_INVALID_VIEW, "swiglu view failed validation");
    const uint64_t n = count_or_zero(*out);
    if (count_or_zero(*gate) != n || count_or_zero(*up) != n)
        return fail(EMEL_ERR_SHAPE_MISMATCH, "swiglu element counts differ");
    return elementwise(emel::Ew::Swiglu, gate, pair_addr(*gate, *out), up, pair_addr(*up, *out), out, 1.0f, stream);
}

namespace {

// A caller slice of `len` floats as a contiguous [len, 1, 1, 1] view.
emel_tensor_view slice_view(const void *p, uint64_t len)
{
    emel_tensor_view v{};
    v.data = p;
    v.data_bytes = len * 4;
    v.dtype = EMEL_DTYPE_F32;
    v.ne[0] = len;
    v.ne[1] = v.ne[2] = v.ne[3] = 1;
    return v;
}

emel_tensor_view_mut slice_view_mut(void *p, uint64_t len)
{
    emel_tensor_view_mut v{};
    v.data = p;
    v.data_bytes = len * 4;
    v.dtype = EMEL_DTYPE_F32;
    v.ne[0] = len;
    v.ne[1] = v.ne[2] = v.ne[3] = 1;
    return v;
}

// Output and input slices either are the same range or do not overlap.
bool slices_disjoint_or_same(const float *out, uint64_t out_len, const float *in, uint64_t in_len)
{
    if (out == in && out_len == in_len) return true;
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(out), o1 = o0 + out_len * 4;
    const uintptr_t i0 = reinterpret_cast<uintptr_t>(in), i1 = i0 + in_len * 4;
    return o1 <= i0 || i1 <= o0;
}

} // namespace

emel_status emel_op_glu(emel_glu_subop subop, const float *input, uint64_t input_len, float *output,
                        uint64_t output_len, emel_stream stream)
{
    static constexpr emel::Ew kOps[6] = {emel::Ew::GluRe, emel::Ew::GluGe, emel::Ew::GluSwi,
                                         emel::Ew::GluSwiOai, emel::Ew::GluGeErf, emel::Ew::GluGeQuick};
    const uint32_t code = static_cast<uint32_t>(subop);
    if (code >= 6) return fail(EMEL_ERR_UNEXPECTED_EVENT, "unknown glu subop");
    if (!input || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    // split_len (glu.rs:85-91)
    if (input_len == 0 || input_len % 2 != 0 || output_len != input_len / 2)
        return fail(EMEL_ERR_SHAPE_MISMATCH, "glu input must split into two halves the size of the output");
    const uint64_t n = output_len;
    if (n > (UINT64_MAX / 8)) return fail(EMEL_ERR_SHAPE_MISMATCH, "glu length overflows");
    const uintptr_t i0 = reinterpret_cast<uintptr_t>(input), i1 = i0 + input_len * 4;
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(output), o1 = o0 + n * 4;
    if (o0 < i1 && i0 < o1) return fail(EMEL_ERR_INVALID_ARGUMENT, "glu output overlaps its input");
    const emel_tensor_view values = slice_view(input, n), gates = slice_view(input + n, n);
    const emel_tensor_view_mut out = slice_view_mut(output, n);
    return elementwise(kOps[code], &values, emel::Addr::SameCoords, &gates, emel::Addr::SameCoords, &out, 1.0f,
                       stream);
}

// ---- dense-slice root events (event.rs:133-259, :523-568) -----------------

emel_status emel_slice_dup(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                           emel_stream stream)
{
    // guard_dup_valid (actor.rs:2498-2501)
    if (input_len == 0 || input_len != output_len) return fail(EMEL_ERR_INVALID_SHAPE, "dup lengths");
    if (!input || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    if (!slices_disjoint_or_same(output, output_len, input, input_len))
        return fail(EMEL_ERR_INVALID_ARGUMENT, "output partially overlaps the input");
    const emel_tensor_view in = slice_view(input, input_len);
    const emel_tensor_view_mut out = slice_view_mut(output, output_len);
    return elementwise(emel::Ew::Copy, &in, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, &out, 1.0f,
                       stream);
}

namespace {

// guard_{add,sub,mul,div}_valid (actor.rs:2522-2560): lhs non-empty, all
// three lengths equal; the effect zips the slices.
emel_status slice_binary(emel::Ew op, const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len,
                         float *output, uint64_t output_len, emel_stream stream)
{
    if (lhs_len == 0 || lhs_len != rhs_len || lhs_len != output_len)
        return fail(EMEL_ERR_INVALID_SHAPE, "binary slice lengths");
    if (!lhs || !rhs || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    if (!slices_disjoint_or_same(output, output_len, lhs, lhs_len) ||
        !slices_disjoint_or_same(output, output_len, rhs, rhs_len))
        return fail(EMEL_ERR_INVALID_ARGUMENT, "output partially overlaps an input");
    const emel_tensor_view a = slice_view(lhs, lhs_len), b = slice_view(rhs, rhs_len);
    const emel_tensor_view_mut out = slice_view_mut(output, output_len);
    return elementwise(op, &a, emel::Addr::SameCoords, &b, emel::Addr::SameCoords, &out, 1.0f, stream);
}

// op_sqr / op_sqrt (actor.rs:1521-1555): both slices become contiguous
// [len, 1, 1, 1] views; an empty slice or unequal counts (PowerError
// InvalidView / ShapeMismatch) map to the root InvalidShape.
emel_status slice_power(emel::Ew op, const float *input, uint64_t input_len, float *output, uint64_t output_len,
                        emel_stream stream)
{
    if (input_len == 0 || output_len == 0 || input_len != output_len)
        return fail(EMEL_ERR_INVALID_SHAPE, "power slice lengths");
    if (!input || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    if (!slices_disjoint_or_same(output, output_len, input, input_len))
        return fail(EMEL_ERR_INVALID_ARGUMENT, "output partially overlaps the input");
    const emel_tensor_view in = slice_view(input, input_len);
    const emel_tensor_view_mut out = slice_view_mut(output, output_len);
    return elementwise(op, &in, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, &out, 1.0f, stream);
}

// power.rs:266-273: validate both views, then equal logical counts.
emel_status view_power(emel::Ew op, const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*in, false) || !valid_f32(*out, false))
        return fail(EMEL_ERR_INVALID_VIEW, "power view failed validation");
    if (count_or_zero(*in) != count_or_zero(*out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "power counts differ");
    return elementwise(op, in, pair_addr(*in, *out), nullptr, emel::Addr::SameCoords, out, 1.0f, stream);
}

} // namespace

emel_status emel_slice_add(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream)
{
    return slice_binary(emel::Ew::Add, lhs, lhs_len, rhs, rhs_len, output, output_len, stream);
}

emel_status emel_slice_sub(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream)
{
    return slice_binary(emel::Ew::Sub, lhs, lhs_len, rhs, rhs_len, output, output_len, stream);
}

emel_status emel_slice_mul(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream)
{
    return slice_binary(emel::Ew::Mul, lhs, lhs_len, rhs, rhs_len, output, output_len, stream);
}

emel_status emel_slice_div(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream)
{
    return slice_binary(emel::Ew::Div, lhs, lhs_len, rhs, rhs_len, output, output_len, stream);
}

emel_status emel_slice_sqr(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                           emel_stream stream)
{
    return slice_power(emel::Ew::Sqr, input, input_len, output, output_len, stream);
}

emel_status emel_slice_sqrt(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                            emel_stream stream)
{
    return slice_power(emel::Ew::Sqrt, input, input_len, output, output_len, stream);
}

emel_status emel_op_sqr(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream)
{
    return view_power(emel::Ew::Sqr, in, out, stream);
}

emel_status emel_op_sqrt(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream)
{
    return view_power(emel::Ew::Sqrt, in, out, stream);
}

emel_status emel_op_scale(const emel_tensor_view *in, const emel_tensor_view_mut *out, float scale, emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*in, false) || !valid_f32(*out, false))
        return fail(EMEL_ERR_INVALID_VIEW, "scale view failed validation");
    if (!same_ne(*in, *out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "scale shapes differ");
    return elementwise(emel::Ew::Scale, in, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, out, scale,
                       stream);
}

emel_status emel_op_rms_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, float eps, emel_stream s)
{
    return norm_op(emel::RowOp::RmsNorm, in, nullptr, out, eps, s);
}

emel_status emel_op_rms_norm_mul(const emel_tensor_view *in, const emel_tensor_view *weight,
                                 const emel_tensor_view_mut *out, float eps, emel_stream s)
{
    return norm_op(emel::RowOp::RmsNormMul, in, weight, out, eps, s);
}

emel_status emel_op_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, float eps, emel_stream s)
{
    return norm_op(emel::RowOp::Norm, in, nullptr, out, eps, s);
}

emel_status emel_op_soft_max(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_f32(*dst, false))
        return fail(EMEL_ERR_INVALID_VIEW, "soft_max view failed validation");
    const uint64_t width = src->ne[0], n = count_or_zero(*src);
    if (!(width > 0 && n > 0 && n % width == 0 && n == count_or_zero(*dst)))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "soft_max element counts differ");
    emel::RowArgs args{};
    args.op = emel::RowOp::SoftMax;
    args.x = operand(*src, 4);
    args.y = operand(*dst, 4);
    args.dense_sum = soft_max_dense_layout(*src) && soft_max_dense_layout(*dst);
    return rows(args, *src, *dst, nullptr, stream);
}

emel_status emel_op_soft_max_ext(const emel_tensor_view *src, const emel_tensor_view *mask, float scale,
                                 const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_f32(*dst, false))
        return fail(EMEL_ERR_INVALID_VIEW, "soft_max view failed validation");
    if (mask) {
        // dense f16 [ne0, ne1, m2, m3]
        const uint64_t *m = mask->ne;
        uint64_t cnt;
        if (mask->dtype != EMEL_DTYPE_F16 || mask->reserved != 0 || !element_count(*mask, cnt))
            return fail(EMEL_ERR_INVALID_VIEW, "mask must be a non-empty f16 view");
        if (!(mask->nb[0] == 2 && mask->nb[1] == 2 * m[0] && mask->nb[2] == mask->nb[1] * m[1] &&
              mask->nb[3] == mask->nb[2] * m[2]) ||
            static_cast<u128>(cnt) * 2 > mask->data_bytes)
            return fail(EMEL_ERR_INVALID_VIEW, "mask must be dense and inside its allocation");
    }
    if (!same_ne(*src, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "soft_max shapes differ");
    if (mask && (mask->ne[0] != src->ne[0] || mask->ne[1] != src->ne[1] || src->ne[2] % mask->ne[2] != 0 ||
                 src->ne[3] % mask->ne[3] != 0))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "mask does not broadcast to the scores");
    emel::RowArgs args{};
    args.op = emel::RowOp::SoftMaxExt;
    args.x = operand(*src, 4);
    args.y = operand(*dst, 4);
    args.scale = scale;
    args.dense_sum = true;
    if (mask) {
        args.mask = static_cast<const uint16_t *>(mask->data);
        args.mask_ne2 = mask->ne[2];
        args.mask_ne3 = mask->ne[3];
    }
    return rows(args, *src, *dst, mask, stream);
}

emel_status emel_op_sum_rows(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_f32(*dst, false))
        return fail(EMEL_ERR_INVALID_VIEW, "sum_rows view failed validation");
    if (!rows_dst(*src, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "sum_rows dst must be [1, ne1, ne2, ne3]");
    return reduce(emel::RedOp::SumRows, *src, *dst, stream);
}

static emel_status scalar_reduce(emel::RedOp op, const emel_tensor_view *src, const emel_tensor_view_mut *dst,
                                 emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_f32(*dst, false))
        return fail(EMEL_ERR_INVALID_VIEW, "reduction view failed validation");
    if (!scalar_dst(*dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "reduction dst must be [1, 1, 1, 1]");
    return reduce(op, *src, *dst, stream);
}

emel_status emel_op_sum(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream s)
{
    return scalar_reduce(emel::RedOp::Sum, src, dst, s);
}

emel_status emel_op_mean(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream s)
{
    return scalar_reduce(emel::RedOp::Mean, src, dst, s);
}

emel_status emel_op_argmax(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream s)
{
    return scalar_reduce(emel::RedOp::Argmax, src, dst, s);
}

emel_status emel_op_argmax_rows(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_i32(*dst))
        return fail(EMEL_ERR_INVALID_VIEW, "argmax_rows view failed validation");
    if (!rows_dst(*src, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "argmax_rows dst must be [1, ne1, ne2, ne3]");
    return reduce(emel::RedOp::ArgmaxRows, *src, *dst, stream);
}

// The same op with its partials and arrival counters in the device's static
// scratch (reduce.hip): no allocation, no synchronisation, no host state.
emel_status emel_op_argmax_rows_no_alloc(const emel_tensor_view *src, const emel_tensor_view_mut *dst,
                                         emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*src, false) || !valid_i32(*dst))
        return fail(EMEL_ERR_INVALID_VIEW, "argmax_rows view failed validation");
    if (!rows_dst(*src, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "argmax_rows dst must be [1, ne1, ne2, ne3]");
    return reduce(emel::RedOp::ArgmaxRows, *src, *dst, stream, true);
}

// ---- row gather (get_rows.rs) -------------------------------------------------

namespace {

// IndexView::new / with_strides (get_rows.rs:54-136): metadata, count and
// the byte span its reads cover.
struct IndexInfo {
    bool valid = false; // metadata_valid && span_valid (:154-157)
    uint64_t count = 0;
    uint64_t st[3] = {0, 0, 0}; // byte strides read through
    uint64_t span = 0;          // bytes from data to the end of the last index
};

IndexInfo index_info(const emel_index_view &v)
{
    IndexInfo out;
    bool inferred = true;
    bool allow_implicit = false;
    if (v.explicit_strides == 0 || v.nb[0] == 0) {
        allow_implicit = v.explicit_strides != 0;
        out.st[0] = 4;
        for (int d = 1; d < 3; ++d) {
            const u128 s = static_cast<u128>(out.st[d - 1]) * v.ne[d - 1];
            if (s > static_cast<u128>(UINT64_MAX)) {
                inferred = false;
                out.st[d] = 0;
            } else {
                out.st[d] = static_cast<uint64_t>(s);
            }
        }
    } else {
        for (int d = 0; d < 3; ++d) out.st[d] = v.nb[d];
    }
    uint64_t count = 1;
    bool zero = false, shape_ok = true, strides_ok = inferred;
    for (int d = 0; d < 3; ++d) {
        const uint64_t extent = v.ne[d], stride = out.st[d];
        if (extent > 1 && stride == 0 && !allow_implicit) strides_ok = false;
        if (stride != 0 && (stride < 4 || stride % 4 != 0)) strides_ok = false;
        if (extent == 0) {
            zero = true;
        } else if (!zero) {
            const u128 c = static_cast<u128>(count) * extent;
            if (c > static_cast<u128>(UINT64_MAX)) {
                shape_ok = false;
                count = 0;
            } else {
                count = static_cast<uint64_t>(c);
            }
        }
    }
    if (zero) count = 0;
    bool span_ok = false;
    if (strides_ok && shape_ok) {
        if (zero) {
            span_ok = true;
        } else {
            u128 max_offset = 0;
            span_ok = true;
            for (int d = 0; d < 3 && span_ok; ++d) {
                const u128 c = static_cast<u128>(v.ne[d] - 1) * out.st[d];
                if (max_offset > ~static_cast<u128>(0) - c) span_ok = false;
                else max_offset += c;
            }
            if (span_ok) {
                const u128 cap = static_cast<u128>(v.len) * 4;
                span_ok = max_offset + 4 <= cap;
                out.span = static_cast<uint64_t>(max_offset + 4);
            }
        }
    }
    out.valid = strides_ok && shape_ok && span_ok;
    out.count = out.valid ? count : 0;
    return out;
}

// Layout::is_dense_contiguous_for (tensor_view.rs:297-314): the given nb.
template <class V>
bool dense_for(const V &v, uint32_t dtype, uint64_t elem)
{
    if (v.dtype != dtype) return false;
    u128 expect = elem;
    for (int d = 0; d < 4; ++d) {
        if (v.nb[d] != expect) return false;
        expect *= v.ne[d];
        if (expect > static_cast<u128>(UINT64_MAX)) return false;
    }
    return true;
}

// The F32 metadata a no-op (empty index) route checks (get_rows.rs:920-943,
// :883-904); elem 2 for BF16 (:1076-1097).
bool empty_source_valid(const emel_tensor_view &s, uint32_t dtype, uint64_t elem, bool f32_bytes)
{
    if (s.dtype != dtype || s.ne[0] == 0 || s.ne[1] == 0) return false;
    if (f32_bytes) {
        if (s.nb[0] != 0 && (s.nb[0] < 4 || s.nb[0] % 4 != 0)) return false;
    } else if (s.nb[0] != 0 && s.nb[0] != elem) {
        return false;
    }
    if (s.nb[0] != 0)
        for (int d = 0; d < 4; ++d)
            if (s.ne[d] > 1 && s.nb[d] == 0) return false;
    return true;
}

// ByteTensorView::validate (tensor_view.rs:588-645).
bool byte_view_valid(const emel_tensor_view &s)
{
    uint64_t count;
    if (s.dtype != EMEL_DTYPE_F32 || !element_count(s, count)) return false;
    if (s.nb[0] != 0) {
        if (s.nb[0] < 4 || s.nb[0] % 4 != 0) return false;
        for (int d = 0; d < 4; ++d)
            if (s.ne[d] > 1 && s.nb[d] == 0) return false;
    }
    uint64_t st[4];
    if (!effective_f32_strides(s, st)) return false;
    u128 max_offset = 0;
    for (int d = 1; d < 4; ++d) max_offset += static_cast<u128>(s.ne[d] - 1) * st[d];
    return max_offset + static_cast<u128>(s.ne[0]) * 4 <= static_cast<u128>(s.data_bytes);
}

// Effective strides of a 2-byte source (nb[0] == 0: row-major).
bool half_strides(const emel_tensor_view &s, uint64_t st[4])
{
    if (s.nb[0] != 0) {
        for (int d = 0; d < 4; ++d) st[d] = s.nb[d];
        return true;
    }
    u128 x = 2;
    st[0] = 2;
    for (int d = 1; d < 4; ++d) {
        x *= s.ne[d - 1];
        if (x > static_cast<u128>(UINT64_MAX)) return false;
        st[d] = static_cast<uint64_t>(x);
    }
    return true;
}

bool half_span_ok(const emel_tensor_view &s, const uint64_t st[4])
{
    u128 max_offset = 0;
    for (int d = 0; d < 4; ++d) {
        const u128 c = static_cast<u128>(s.ne[d] - 1) * st[d];
        if (max_offset > ~static_cast<u128>(0) - c) return false;
        max_offset += c;
    }
    return max_offset + 2 <= static_cast<u128>(s.data_bytes / 2) * 2;
}

// F16View::validate (f16_matmul.rs:49-90).
bool f16_view_valid(const emel_tensor_view &s)
{
    uint64_t st[4], count;
    if (!half_strides(s, st) || s.dtype != EMEL_DTYPE_F16 || !element_count(s, count)) return false;
    for (int d = 0; d < 4; ++d)
        if (s.ne[d] > 1 && (st[d] < 2 || st[d] % 2 != 0)) return false;
    return half_span_ok(s, st);
}

// Bf16View::validate (get_rows.rs:302-343).
bool bf16_view_valid(const emel_tensor_view &s)
{
    uint64_t st[4], count;
    if (s.dtype != EMEL_DTYPE_BF16 || !element_count(s, count) || !half_strides(s, st)) return false;
    if (s.nb[0] != 0)
        for (int d = 0; d < 4; ++d)
            if ((s.ne[d] > 1 && s.nb[d] == 0) || (s.nb[d] != 0 && (s.nb[d] < 2 || s.nb[d] % 2 != 0))) return false;
    return half_span_ok(s, st);
}

// PackedRowView::validate (tensor_view.rs:487-532).
bool packed_view_valid(const emel_tensor_view &s, uint32_t code, uint64_t block_values, uint64_t block_bytes)
{
    if (s.dtype != code) return false;
    for (int d = 0; d < 4; ++d)
        if (s.ne[d] == 0) return false;
    if (s.ne[0] % block_values != 0 || s.nb[0] != 1) return false;
    const u128 row = static_cast<u128>(s.ne[0] / block_values) * block_bytes;
    const u128 rs2 = row * s.ne[1];
    const u128 rs3 = rs2 * s.ne[2];
    if (rs3 > static_cast<u128>(UINT64_MAX) || row == 0) return false;
    if (s.nb[1] != row || s.nb[2] != rs2 || s.nb[3] != rs3) return false;
    u128 max_offset = 0;
    for (int d = 1; d < 4; ++d) max_offset += static_cast<u128>(s.ne[d] - 1) * s.nb[d];
    return max_offset + row <= static_cast<u128>(s.data_bytes);
}

enum class GrKind { F32, F32Bytes, F16, Bf16, Q4_0, Q8_0, Q4K };

emel_status get_rows(GrKind kind, const emel_tensor_view *src, const emel_index_view *idx,
                     const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !idx || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (idx->on_host > 1 || src->reserved != 0 || dst->reserved != 0)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "on_host must be 0 or 1 and reserved fields 0");
    // Pointers no Rust slice of the element type can hold.
    const uintptr_t sp = reinterpret_cast<uintptr_t>(src->data);
    if ((reinterpret_cast<uintptr_t>(idx->data) & 3u) || (reinterpret_cast<uintptr_t>(dst->data) & 3u) ||
        (kind == GrKind::F32 && (sp & 3u)) || ((kind == GrKind::F16 || kind == GrKind::Bf16) && (sp & 1u)))
        return fail(EMEL_ERR_INVALID_ARGUMENT, "data pointer not aligned to its element type");

    const IndexInfo ix = index_info(*idx);
    const uint64_t n = ix.count;
    const emel_tensor_view &s = *src;
    // views_valid* (get_rows.rs:855-1091)
    bool dst_ok;
    if (n == 0) dst_ok = dense_for(*dst, EMEL_DTYPE_F32, 4);
    else dst_ok = valid_f32(*dst, false) && dense_for(*dst, EMEL_DTYPE_F32, 4);
    bool src_ok = false;
    switch (kind) {
    case GrKind::F32: src_ok = n == 0 ? empty_source_valid(s, EMEL_DTYPE_F32, 4, false) : valid_f32(s, true); break;
    case GrKind::F32Bytes: src_ok = n == 0 ? empty_source_valid(s, EMEL_DTYPE_F32, 4, true) : byte_view_valid(s); break;
    case GrKind::F16: src_ok = f16_view_valid(s); if (n == 0) dst_ok = valid_f32(*dst, false) && dense_for(*dst, EMEL_DTYPE_F32, 4); break;
    case GrKind::Bf16: src_ok = n == 0 ? empty_source_valid(s, EMEL_DTYPE_BF16, 2, false) : bf16_view_valid(s); break;
    case GrKind::Q4_0: src_ok = packed_view_valid(s, EMEL_DTYPE_Q4_0, 32, 18); break;
    case GrKind::Q8_0: src_ok = packed_view_valid(s, EMEL_DTYPE_Q8_0, 32, 34); break;
    case GrKind::Q4K: src_ok = packed_view_valid(s, EMEL_DTYPE_Q4_K, 256, 144); break;
    }
    if (!ix.valid || !src_ok || !dst_ok) return fail(EMEL_ERR_INVALID_VIEW, "get_rows view failed validation");
    // shape_valid (get_rows.rs:966-975)
    if (!(s.ne[0] > 0 && s.ne[1] > 0 && dst->ne[0] == s.ne[0] && dst->ne[1] == idx->ne[0] &&
          dst->ne[2] == idx->ne[1] && dst->ne[3] == idx->ne[2] && s.ne[2] == idx->ne[1] && s.ne[3] == idx->ne[2]))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "get_rows shapes differ");
    // source_stride_valid (get_rows.rs:961-964), the F32 route only
    if (kind == GrKind::F32 && !(s.nb[0] == 0 || (s.nb[0] >= 4 && s.nb[0] % 4 == 0)))
        return fail(EMEL_ERR_UNSUPPORTED_SOURCE_STRIDE, "get_rows source element stride");
    // dst must not overlap what the gather reads (impossible for Rust's borrows)
    if (n > 0) {
        const auto d = byte_range(*dst, 4);
        auto hit = [&](uintptr_t lo, uint64_t bytes) { return lo < d.second && d.first < lo + bytes; };
        if (hit(sp, s.data_bytes) || (!idx->on_host && hit(reinterpret_cast<uintptr_t>(idx->data), ix.span)))
            return fail(EMEL_ERR_INVALID_VIEW, "dst overlaps the source or the indices");
    }
    emel_status st = ensure_device();
    if (st != EMEL_OK) return st;
    if (n == 0) {
        g_last_error.clear();
        return EMEL_OK; // the reference's loops run zero times
    }
    // indices_valid (get_rows.rs:1239-1250): every index in [0, src.ne1),
    // read from host memory (on_host) or from a host copy of the index span.
    const hipStream_t hs = as_stream(stream);
    const int32_t *hp = idx->data;
    // Held through the index check and the launch: another host thread on
    // this stream cannot refill the staging copy or the uploaded indices.
    StreamLease lease;
    if (!idx->on_host) {
        st = not_capturing(hs, "get_rows with device-resident indices (copied back and checked on the host)");
        if (st == EMEL_OK) st = lease.acquire(hs);
        if (st != EMEL_OK) return st;
        void *stage = nullptr;
        st = lease.staging(ix.span, &stage);
        if (st != EMEL_OK) return st;
        hipError_t e = hipMemcpyAsync(stage, idx->data, ix.span, hipMemcpyDeviceToHost, hs);
        if (e == hipSuccess) e = hipStreamSynchronize(hs);
        if (e != hipSuccess) return hip_fail(e, "copying the indices to the host");
        hp = static_cast<const int32_t *>(stage);
    }
    const uint64_t es[3] = {ix.st[0] / 4, ix.st[1] / 4, ix.st[2] / 4};
    std::vector<int32_t> compact;
    if (idx->on_host) compact.resize(n);
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t i0 = k % idx->ne[0], rem = k / idx->ne[0];
        const uint64_t i1 = rem % idx->ne[1], i2 = rem / idx->ne[1];
        const int32_t row = hp[i0 * es[0] + i1 * es[1] + i2 * es[2]];
        if (row < 0 || static_cast<uint64_t>(row) >= s.ne[1])
            return fail(EMEL_ERR_INDEX_OUT_OF_BOUNDS, "get_rows index " + std::to_string(row) + " at ordinal " +
                                                          std::to_string(k) + " is outside the source rows");
        if (idx->on_host) compact[k] = row;
    }
    emel::GetRowsArgs a{};
    switch (kind) {
    case GrKind::F32: a.kind = emel::RowSrc::F32; break;
    case GrKind::F32Bytes: a.kind = emel::RowSrc::F32Bytes; break;
    case GrKind::F16: a.kind = emel::RowSrc::F16; break;
    case GrKind::Bf16: a.kind = emel::RowSrc::Bf16; break;
    case GrKind::Q4_0: a.kind = emel::RowSrc::Q4_0; break;
    case GrKind::Q8_0: a.kind = emel::RowSrc::Q8_0; break;
    case GrKind::Q4K: a.kind = emel::RowSrc::Q4K; break;
    }
    a.src = s.data;
    uint64_t stv[4] = {s.nb[0], s.nb[1], s.nb[2], s.nb[3]};
    if (kind == GrKind::F32 || kind == GrKind::F32Bytes) effective_f32_strides(s, stv);
    else if (kind == GrKind::F16 || kind == GrKind::Bf16) half_strides(s, stv);
    for (int d = 0; d < 4; ++d) {
        a.src_ne[d] = s.ne[d];
        a.src_st[d] = static_cast<int64_t>(s.ne[d] > 1 ? stv[d] : 0); // a singleton's stride never moves
    }
    for (int d = 0; d < 3; ++d) a.idx_ne[d] = idx->ne[d];
    a.dst = static_cast<float *>(dst->data);
    a.rows = n;
    a.cols = s.ne[0];
    if (!idx->on_host) {
        a.idx = idx->data;
        for (int d = 0; d < 3; ++d) a.idx_st[d] = static_cast<int64_t>(idx->ne[d] > 1 ? es[d] : 0);
        return launched(emel::launch_get_rows(a, nullptr, hs));
    }
    if (n <= emel::kInlineIndices && emel::get_rows_row_kernels(a)) {
        emel::IdxInline ii{};
        std::memcpy(ii.v, compact.data(), n * sizeof(int32_t));
        return launched(emel::launch_get_rows(a, &ii, hs));
    }
    // More indices than the arguments carry: upload the checked values in
    // ordinal order and read them row-major.
    st = not_capturing(hs, "get_rows with more host indices than the launch arguments carry (uploaded and awaited)");
    if (st == EMEL_OK) st = lease.acquire(hs);
    if (st != EMEL_OK) return st;
    void *ws = nullptr;
    st = lease.work(n * sizeof(int32_t), &ws);
    if (st != EMEL_OK) return st;
    hipError_t e = hipMemcpyAsync(ws, compact.data(), n * sizeof(int32_t), hipMemcpyHostToDevice, hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs); // the host vector goes away on return
    if (e != hipSuccess) return hip_fail(e, "uploading the indices");
    a.idx = static_cast<const int32_t *>(ws);
    a.idx_st[0] = 1;
    a.idx_st[1] = static_cast<int64_t>(idx->ne[0]);
    a.idx_st[2] = static_cast<int64_t>(idx->ne[0] * idx->ne[1]);
    return launched(emel::launch_get_rows(a, nullptr, hs));
}

} // namespace

emel_status emel_op_get_rows(const emel_tensor_view *src, const emel_index_view *indices,
                             const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::F32, src, indices, dst, stream);
}

emel_status emel_op_get_rows_f32_bytes(const emel_tensor_view *src, const emel_index_view *indices,
                                       const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::F32Bytes, src, indices, dst, stream);
}

emel_status emel_op_get_rows_f16(const emel_tensor_view *src, const emel_index_view *indices,
                                 const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::F16, src, indices, dst, stream);
}

emel_status emel_op_get_rows_bf16(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::Bf16, src, indices, dst, stream);
}

emel_status emel_op_get_rows_q4_0(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::Q4_0, src, indices, dst, stream);
}

emel_status emel_op_get_rows_q8_0(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::Q8_0, src, indices, dst, stream);
}

emel_status emel_op_get_rows_q4_k(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream)
{
    return get_rows(GrKind::Q4K, src, indices, dst, stream);
}

// ---- generic wire envelope (generic.rs, guards actor.rs:2448-2983) ----------

namespace {

enum GenOpCode : uint32_t {
    kDup = 0, kAdd = 1, kAdd1 = 3, kSub = 5, kMul = 6, kDiv = 7, kSqr = 8, kSqrt = 9, kLog = 10, kSin = 11,
    kCos = 12, kSum = 13, kCumsum = 15, kMean = 16, kArgmax = 17, kCountEqual = 18, kRepeat = 19,
    kRepeatBack = 20, kConcat = 21, kSiluBack = 22, kNorm = 23, kRmsNorm = 24, kRmsNormBack = 25, kL2Norm = 27,
    kMulMat = 28, kMulMatArgmax = 29, kScale = 32, kDiag = 43, kDiagMaskInf = 44, kDiagMaskZero = 45,
    kSoftMax = 46, kSoftMaxBack = 47, kClamp = 50, kArange = 66, kLeakyRelu = 70, kFill = 72, kUnary = 85,
    kGenericOps = 95
};

using GView = emel_tensor_view; // the sources; dst is read through the same fields

struct GenReq {
    const emel_generic_request &r;
    const GView *s0, *s1, *s2, *d;

    explicit GenReq(const emel_generic_request &req)
        : r(req), s0(req.src0), s1(req.src1), s2(req.src2),
          d(reinterpret_cast<const GView *>(req.dst)) {}

    bool param_bytes(uint32_t slot, uint8_t out[4]) const
    {
        if (r.op_params_size < 4 * (slot + 1)) return false;
        std::memcpy(out, r.op_params + 4 * slot, 4);
        return true;
    }
    bool param_f32(uint32_t slot, float &v) const
    {
        uint8_t b[4];
        if (!param_bytes(slot, b)) return false;
        std::memcpy(&v, b, 4);
        return true;
    }
    bool param_i32(uint32_t slot, int32_t &v) const
    {
        uint8_t b[4];
        if (!param_bytes(slot, b)) return false;
        std::memcpy(&v, b, 4);
        return true;
    }
};

// The strides validate_span and byte_offset use: effective F32 strides for
// F32, the given nb otherwise (generic.rs:850-857, :911-917).
bool gen_strides(const GView &v, uint64_t st[4])
{
    if (v.dtype == EMEL_DTYPE_F32) return effective_f32_strides(v, st);
    std::memcpy(st, v.nb, sizeof v.nb);
    return true;
}

// validate_span (generic.rs:849-894): non-zero extents with a usize count,
// no zero stride on an extent > 1, and the last element's first byte inside
// the slice.
bool gen_span(const GView &v)
{
    uint64_t st[4];
    if (!gen_strides(v, st)) return false;
    u128 count = 1;
    for (int d = 0; d < 4; ++d) {
        if (v.ne[d] == 0) return false;
        count *= v.ne[d];
        if (count > static_cast<u128>(UINT64_MAX)) return false;
        if (v.ne[d] > 1 && st[d] == 0) return false;
    }
    u128 max_offset = 0;
    for (int d = 0; d < 4; ++d) {
        const u128 c = static_cast<u128>(v.ne[d] - 1) * st[d];
        if (max_offset > ~static_cast<u128>(0) - c) return false;
        max_offset += c;
    }
    return max_offset + 1 <= static_cast<u128>(v.data_bytes);
}

// RawTensorView::f32_valid (generic.rs:471-476).
bool gen_f32(const GView *v)
{
    if (!v || v->dtype != EMEL_DTYPE_F32) return false;
    uint64_t st[4];
    if (!effective_f32_strides(*v, st) || !gen_span(*v)) return false;
    for (int d = 0; d < 4; ++d)
        if (st[d] < 4) return false;
    return true;
}

// RawTensorView::f16_valid (generic.rs:489-493) with is_dense_contiguous_f16
// (tensor_view.rs:293-314).
bool gen_f16(const GView *v)
{
    if (!v || v->dtype != EMEL_DTYPE_F16 || !gen_span(*v)) return false;
    u128 expect = 2;
    for (int d = 0; d < 4; ++d) {
        if (v->nb[d] != expect) return false;
        expect *= v->ne[d];
        if (expect > static_cast<u128>(UINT64_MAX)) return false;
    }
    return true;
}

uint64_t gen_count(const GView *v) { return count_or_zero(*v); }

bool ne_eq(const GView *a, const GView *b) { return same_ne(*a, *b); }

bool ne_is(const GView *v, uint64_t a, uint64_t b, uint64_t c, uint64_t e)
{
    return v->ne[0] == a && v->ne[1] == b && v->ne[2] == c && v->ne[3] == e;
}

// GenericRequest::validate (generic.rs:769-789).
bool gen_request_valid(const GenReq &q)
{
    for (const GView *v : {q.s0, q.s1, q.s2, q.d})
        if (v && !gen_span(*v)) return false;
    return !(q.r.operation == kMulMatArgmax && !q.r.index_out);
}

// ---- the maintained predicates (generic.rs:935-1262) ----

bool pair_valid(const GenReq &q)
{
    return gen_f32(q.s0) && gen_f32(q.d) && gen_count(q.s0) == gen_count(q.d);
}

bool triplet_valid(const GenReq &q)
{
    return gen_f32(q.s0) && gen_f32(q.s1) && gen_f32(q.d) && ne_eq(q.s0, q.s1) && ne_eq(q.s0, q.d);
}

bool scalar_valid(const GenReq &q)
{
    float p;
    return pair_valid(q) && q.param_f32(0, p) && std::isfinite(p);
}

bool clamp_valid(const GenReq &q)
{
    float lo, hi;
    return pair_valid(q) && q.param_f32(0, lo) && q.param_f32(1, hi) && std::isfinite(lo) && std::isfinite(hi) &&
           lo <= hi;
}

bool cumsum_valid(const GenReq &q) { return gen_f32(q.s0) && gen_f32(q.d) && ne_eq(q.s0, q.d); }

bool repeat_shape(const GView *src, const GView *dst)
{
    for (int d = 0; d < 4; ++d)
        if (src->ne[d] == 0 || dst->ne[d] == 0 || dst->ne[d] % src->ne[d] != 0) return false;
    return true;
}

bool repeat_valid(const GenReq &q) { return gen_f32(q.s0) && gen_f32(q.d) && repeat_shape(q.s0, q.d); }
bool repeat_back_valid(const GenReq &q) { return gen_f32(q.s0) && gen_f32(q.d) && repeat_shape(q.d, q.s0); }

bool concat_valid(const GenReq &q, int axis)
{
    int32_t p;
    if (!gen_f32(q.s0) || !gen_f32(q.s1) || !gen_f32(q.d) || !q.param_i32(0, p) || p != axis) return false;
    for (int d = 0; d < 4; ++d) {
        if (d == axis) {
            const u128 sum = static_cast<u128>(q.s0->ne[d]) + q.s1->ne[d];
            if (sum != q.d->ne[d]) return false;
        } else if (q.s0->ne[d] != q.s1->ne[d] || q.s0->ne[d] != q.d->ne[d]) {
            return false;
        }
    }
    return true;
}

bool fill_valid(const GenReq &q)
{
    float v;
    return !q.s0 && gen_f32(q.d) && q.param_f32(0, v) && std::isfinite(v);
}

bool arange_valid(const GenReq &q)
{
    float a, b;
    return !q.s0 && gen_f32(q.d) && q.param_f32(0, a) && std::isfinite(a) && q.param_f32(1, b) && std::isfinite(b);
}

bool diag_valid(const GenReq &q)
{
    if (!q.s0 || !q.d) return false;
    const uint64_t n = q.s0->ne[0];
    const u128 side = static_cast<u128>(n) * n;
    if (side > static_cast<u128>(UINT64_MAX)) return false;
    return gen_f32(q.s0) && gen_f32(q.d) && q.s0->ne[1] == 1 && q.s0->ne[2] == 1 && q.s0->ne[3] == 1 &&
           ne_is(q.d, n, n, 1, 1) && gen_count(q.d) == static_cast<uint64_t>(side);
}

bool mask_valid(const GenReq &q)
{
    int32_t n_past;
    if (!q.s0 || !q.d || !q.param_i32(0, n_past)) return false;
    const GView *s = q.s0;
    return n_past >= 0 && gen_f32(q.s0) && gen_f32(q.d) && ne_eq(q.s0, q.d) && s->ne[0] > 0 && s->ne[1] == s->ne[0] &&
           s->ne[2] == 1 && s->ne[3] == 1;
}

bool l2_valid(const GenReq &q) { return gen_f32(q.s0) && gen_f32(q.d) && ne_eq(q.s0, q.d) && gen_count(q.s0) > 0; }

bool softmax_back_valid(const GenReq &q)
{
    int32_t row;
    if (!triplet_valid(q) || !q.param_i32(0, row)) return false;
    return row > 0 && gen_count(q.s0) % static_cast<uint64_t>(row) == 0;
}

bool rms_norm_back_valid(const GenReq &q)
{
    float eps;
    if (!triplet_valid(q) || !q.param_f32(0, eps)) return false;
    return std::isfinite(eps) && eps >= 0.0f && q.s0->ne[0] > 0;
}

bool count_equal_valid(const GenReq &q)
{
    return gen_f32(q.s0) && gen_f32(q.s1) && gen_f32(q.d) && gen_count(q.s0) == gen_count(q.s1) &&
           gen_count(q.d) == 1;
}

bool binary_valid(const GenReq &q)
{
    return gen_f32(q.s0) && gen_f32(q.s1) && gen_f32(q.d) && gen_count(q.s0) == gen_count(q.s1) &&
           gen_count(q.s0) == gen_count(q.d);
}

bool reduce_valid(const GenReq &q) { return gen_f32(q.s0) && gen_f32(q.d) && gen_count(q.d) == 1; }

bool norm_valid(const GenReq &q)
{
    float eps;
    return gen_f32(q.s0) && gen_f32(q.d) && ne_eq(q.s0, q.d) && q.param_f32(0, eps) && std::isfinite(eps) &&
           eps >= 0.0f;
}

bool matmul_f32_valid(const GenReq &q)
{
    if (!gen_f32(q.s0) || !gen_f32(q.s1) || !gen_f32(q.d)) return false;
    const uint64_t *l = q.s0->ne, *r = q.s1->ne, *o = q.d->ne;
    return l[0] > 0 && l[1] > 0 && r[0] > 0 && r[1] == l[0] && o[0] == r[0] && o[1] == l[1] && l[2] == 1 &&
           l[3] == 1 && r[2] == 1 && r[3] == 1 && o[2] == 1 && o[3] == 1;
}

bool matmul_argmax_valid(const GenReq &q)
{
    if (!q.r.index_out || !gen_f32(q.s0) || !gen_f32(q.s1) || !gen_f32(q.d)) return false;
    const uint64_t *l = q.s0->ne;
    return l[0] > 0 && l[1] > 0 && ne_is(q.s1, l[0], 1, 1, 1) && ne_is(q.d, 1, 1, 1, 1) && l[2] == 1 && l[3] == 1;
}

bool matmul_f16_valid(const GenReq &q)
{
    if (!gen_f16(q.s0) || !gen_f16(q.s1) || !gen_f32(q.d)) return false;
    const uint64_t *l = q.s0->ne, *r = q.s1->ne, *o = q.d->ne;
    return l[0] > 0 && l[1] > 0 && r[0] == l[0] && r[1] > 0 && o[0] == l[1] && o[1] == r[1] && l[2] == 1 &&
           l[3] == 1 && r[2] == 1 && r[3] == 1 && o[2] == 1 && o[3] == 1;
}

// The eight unary subops the generic lane executes (actor.rs:2875-2905).
bool unary_subop_routed(uint32_t s)
{
    return s == EMEL_UNARY_ABS || s == EMEL_UNARY_NEG || s == EMEL_UNARY_TANH || s == EMEL_UNARY_ELU ||
           s == EMEL_UNARY_RELU || s == EMEL_UNARY_GELU || s == EMEL_UNARY_SILU || s == EMEL_UNARY_EXP;
}

enum class Route {
    None, Dup, Binary, Scalar, Clamp, SiluBack, Cumsum, Repeat, RepeatBack, Concat, Diag, DiagMask, SoftMaxBack,
    RmsNormBack, L2Norm, CountEqual, Fill, Arange, MulMatF32, MulMatF16, MulMatArgmax, Power, Math, Reduce,
    SoftMax, Norm, Unary
};

// The guarded transitions of sm.rs:322-413, each `operation == X && route
// predicate`; at most one can hold for a request.
Route gen_route(const GenReq &q, int &concat_axis)
{
    switch (q.r.operation) {
    case kDup: return pair_valid(q) ? Route::Dup : Route::None;
    case kAdd: case kSub: case kMul: case kDiv: return binary_valid(q) ? Route::Binary : Route::None;
    case kAdd1: case kScale: case kLeakyRelu: return scalar_valid(q) ? Route::Scalar : Route::None;
    case kClamp: return clamp_valid(q) ? Route::Clamp : Route::None;
    case kSiluBack: return triplet_valid(q) ? Route::SiluBack : Route::None;
    case kCumsum: return cumsum_valid(q) ? Route::Cumsum : Route::None;
    case kRepeat: return repeat_valid(q) ? Route::Repeat : Route::None;
    case kRepeatBack: return repeat_back_valid(q) ? Route::RepeatBack : Route::None;
    case kConcat:
        for (int a = 0; a < 4; ++a)
            if (concat_valid(q, a)) {
                concat_axis = a;
                return Route::Concat;
            }
        return Route::None;
    case kDiag: return diag_valid(q) ? Route::Diag : Route::None;
    case kDiagMaskInf: case kDiagMaskZero: return mask_valid(q) ? Route::DiagMask : Route::None;
    case kSoftMaxBack: return softmax_back_valid(q) ? Route::SoftMaxBack : Route::None;
    case kRmsNormBack: return rms_norm_back_valid(q) ? Route::RmsNormBack : Route::None;
    case kL2Norm: return l2_valid(q) ? Route::L2Norm : Route::None;
    case kCountEqual: return count_equal_valid(q) ? Route::CountEqual : Route::None;
    case kFill: return fill_valid(q) ? Route::Fill : Route::None;
    case kArange: return arange_valid(q) ? Route::Arange : Route::None;
    case kMulMat:
        if (matmul_f32_valid(q)) return Route::MulMatF32;
        return matmul_f16_valid(q) ? Route::MulMatF16 : Route::None;
    case kMulMatArgmax: return matmul_argmax_valid(q) ? Route::MulMatArgmax : Route::None;
    case kSqr: case kSqrt: return pair_valid(q) ? Route::Power : Route::None;
    case kLog: case kSin: case kCos: return pair_valid(q) ? Route::Math : Route::None;
    case kSum: case kMean: case kArgmax: return reduce_valid(q) ? Route::Reduce : Route::None;
    case kSoftMax: return pair_valid(q) ? Route::SoftMax : Route::None;
    case kNorm: case kRmsNorm: return norm_valid(q) ? Route::Norm : Route::None;
    case kUnary: return unary_subop_routed(q.r.unary_subop) && pair_valid(q) ? Route::Unary : Route::None;
    default: return Route::None;
    }
}

// guard_generic_known_invalid (actor.rs:2907-2983): the maintained
// operations whose predicate failed (gen_route gave None).
bool gen_maintained(uint32_t op)
{
    switch (op) {
    case kDup: case kAdd: case kSub: case kMul: case kDiv: case kAdd1: case kScale: case kLeakyRelu: case kClamp:
    case kSiluBack: case kCumsum: case kRepeat: case kRepeatBack: case kConcat: case kDiag: case kDiagMaskInf:
    case kDiagMaskZero: case kSoftMaxBack: case kRmsNormBack: case kL2Norm: case kCountEqual: case kFill:
    case kArange: case kMulMat: case kMulMatArgmax: case kSqr: case kSqrt: case kLog: case kSin: case kCos:
    case kSum: case kMean: case kArgmax: case kSoftMax: case kNorm: case kRmsNorm: case kUnary:
        return true;
    default:
        return false;
    }
}

// Routes where each lane reads a source element (or row) before writing the
// same-ordinal destination element (or row), so dst may be the source view.
bool alias_ok(Route r)
{
    switch (r) {
    case Route::Dup: case Route::Binary: case Route::Scalar: case Route::Clamp: case Route::SiluBack:
    case Route::Cumsum: case Route::Repeat: case Route::RepeatBack: case Route::DiagMask: case Route::SoftMaxBack:
    case Route::RmsNormBack: case Route::L2Norm: case Route::Power: case Route::Math: case Route::SoftMax:
    case Route::Norm: case Route::Unary:
        return true;
    default:
        return false;
    }
}

bool same_view(const GView &a, const GView &b)
{
    if (a.data != b.data || !same_ne(a, b)) return false;
    uint64_t sa[4], sb[4];
    if (!gen_strides(a, sa) || !gen_strides(b, sb)) return false;
    for (int d = 0; d < 4; ++d)
        if (a.ne[d] > 1 && sa[d] != sb[d]) return false;
    return true;
}

uint64_t elem_bytes(const GView &v) { return v.dtype == EMEL_DTYPE_F16 ? 2 : 4; }

// The element-aligned addressing the device kernels use.
bool gen_aligned(const GView &v)
{
    const uint64_t e = elem_bytes(v);
    if (reinterpret_cast<uintptr_t>(v.data) % e != 0) return false;
    uint64_t st[4];
    if (!gen_strides(v, st)) return false;
    for (int d = 0; d < 4; ++d)
        if (v.ne[d] > 1 && st[d] % e != 0) return false;
    return true;
}

// The whole last element inside data_bytes (validate_span checks its first
// byte only).
bool gen_whole(const GView &v)
{
    uint64_t st[4];
    if (!gen_strides(v, st)) return false;
    return span_fits(v, st, elem_bytes(v));
}

emel::GView gview(const GView &v)
{
    emel::GView g{};
    g.data = const_cast<void *>(v.data);
    uint64_t st[4];
    gen_strides(v, st);
    const uint64_t e = elem_bytes(v);
    for (int d = 0; d < 4; ++d) {
        g.ne[d] = v.ne[d];
        g.st[d] = static_cast<int64_t>(st[d] / e);
    }
    return g;
}

emel::Ew unary_generic_fn(uint32_t s)
{
    switch (s) {
    case EMEL_UNARY_ABS: return emel::Ew::Abs;
    case EMEL_UNARY_NEG: return emel::Ew::Neg;
    case EMEL_UNARY_TANH: return emel::Ew::Tanh;
    case EMEL_UNARY_ELU: return emel::Ew::Elu;
    case EMEL_UNARY_RELU: return emel::Ew::Relu;
    case EMEL_UNARY_GELU: return emel::Ew::GeluGeneric;
    case EMEL_UNARY_SILU: return emel::Ew::Silu;
    default: return emel::Ew::Exp;
    }
}

emel_status gen_execute(const GenReq &q, Route route, int concat_axis, emel_stream stream)
{
    const uint32_t op = q.r.operation;
    const GView &dst = *q.d;
    const emel_tensor_view_mut &dmut = *q.r.dst;
    const GView *used[3] = {nullptr, nullptr, nullptr};
    int n_used = 0;
    switch (route) {
    case Route::Fill: case Route::Arange: break;
    case Route::Binary: case Route::SiluBack: case Route::Concat: case Route::SoftMaxBack: case Route::RmsNormBack:
    case Route::CountEqual: case Route::MulMatF32: case Route::MulMatF16: case Route::MulMatArgmax:
        used[n_used++] = q.s0;
        used[n_used++] = q.s1;
        break;
    default: used[n_used++] = q.s0; break;
    }

    // Divergences from the reference, refused before anything is enqueued.
    for (int i = 0; i < n_used; ++i)
        if (!gen_aligned(*used[i])) return fail(EMEL_ERR_UNSUPPORTED_OPERATION, "source view is not element-aligned");
    if (!gen_aligned(dst)) return fail(EMEL_ERR_UNSUPPORTED_OPERATION, "dst view is not element-aligned");
    for (int i = 0; i < n_used; ++i)
        if (!gen_whole(*used[i]))
            return fail(EMEL_ERR_INVALID_SHAPE, "a source's last element extends past data_bytes");
    if (!gen_whole(dst)) return fail(EMEL_ERR_INVALID_SHAPE, "dst's last element extends past data_bytes");
    if (!elements_disjoint(dst, 4))
        return fail(EMEL_ERR_UNSUPPORTED_OPERATION, "dst elements overlap one another");
    for (int i = 0; i < n_used; ++i) {
        const GView &s = *used[i];
        const auto a = byte_range(dst, 4);
        const auto b = byte_range(s, elem_bytes(s));
        const bool disjoint = a.second <= b.first || b.second <= a.first;
        if (!disjoint && !(alias_ok(route) && same_view(dst, s)))
            return fail(EMEL_ERR_INVALID_ARGUMENT, "dst overlaps a source");
    }
    if (route == Route::MulMatArgmax && q.s0->ne[1] > static_cast<uint64_t>(INT32_MAX))
        return fail(EMEL_ERR_INVALID_SHAPE, "mul_mat_argmax row index does not fit i32");

    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    const hipStream_t hs = as_stream(stream);
    float p0 = 0.0f, p1 = 0.0f;
    q.param_f32(0, p0);
    q.param_f32(1, p1);

    switch (route) {
    case Route::Dup:
        return elementwise(emel::Ew::Copy, q.s0, pair_addr(*q.s0, dmut), nullptr, emel::Addr::SameCoords, &dmut, 0.0f,
                           stream);
    case Route::Binary: {
        const emel::Ew fn = op == kAdd ? emel::Ew::Add : op == kSub ? emel::Ew::Sub : op == kMul ? emel::Ew::Mul
                                                                                                 : emel::Ew::Div;
        return elementwise(fn, q.s0, pair_addr(*q.s0, dmut), q.s1, pair_addr(*q.s1, dmut), &dmut, 0.0f, stream);
    }
    case Route::Scalar: {
        const emel::Ew fn = op == kAdd1 ? emel::Ew::Add1 : op == kScale ? emel::Ew::Scale : emel::Ew::LeakyRelu;
        return elementwise(fn, q.s0, pair_addr(*q.s0, dmut), nullptr, emel::Addr::SameCoords, &dmut, p0, stream);
    }
    case Route::Clamp:
        return elementwise(emel::Ew::Clamp, q.s0, pair_addr(*q.s0, dmut), nullptr, emel::Addr::SameCoords, &dmut, p0,
                           stream, p1);
    case Route::SiluBack:
        return elementwise(emel::Ew::SiluBack, q.s0, emel::Addr::SameCoords, q.s1, emel::Addr::SameCoords, &dmut,
                           0.0f, stream);
    case Route::Power:
        return elementwise(op == kSqr ? emel::Ew::Sqr : emel::Ew::Sqrt, q.s0, pair_addr(*q.s0, dmut), nullptr,
                           emel::Addr::SameCoords, &dmut, 0.0f, stream);
    case Route::Math: // f32::ln / sin / cos (generic.rs), the glibc replicas
        return elementwise(op == kLog ? emel::Ew::Log : op == kSin ? emel::Ew::Sin : emel::Ew::Cos, q.s0,
                           pair_addr(*q.s0, dmut), nullptr, emel::Addr::SameCoords, &dmut, 0.0f, stream);
    case Route::Unary:
        return elementwise(unary_generic_fn(q.r.unary_subop), q.s0, pair_addr(*q.s0, dmut), nullptr,
                           emel::Addr::SameCoords, &dmut, 0.0f, stream);
    case Route::Repeat:
        return elementwise(emel::Ew::Copy, q.s0, emel::Addr::Broadcast, nullptr, emel::Addr::SameCoords, &dmut, 0.0f,
                           stream);
    case Route::Reduce: {
        const emel::RedOp rop = op == kSum ? emel::RedOp::Sum : op == kMean ? emel::RedOp::Mean : emel::RedOp::Argmax;
        return reduce(rop, *q.s0, dmut, stream);
    }
    case Route::Cumsum: case Route::SoftMax: case Route::Norm: case Route::SoftMaxBack: case Route::RmsNormBack: {
        emel::GenRowArgs a{};
        a.x = gview(*q.s0);
        a.y = gview(dst);
        const uint64_t count = gen_count(q.s0);
        a.width = q.s0->ne[0];
        if (route == Route::Cumsum) a.op = emel::GenRow::Cumsum;
        else if (route == Route::SoftMax) a.op = emel::GenRow::SoftMax;
        else if (route == Route::Norm) a.op = op == kNorm ? emel::GenRow::Norm : emel::GenRow::RmsNorm;
        else if (route == Route::SoftMaxBack) a.op = emel::GenRow::SoftMaxBack;
        else a.op = emel::GenRow::RmsNormBack;
        if (route == Route::SoftMaxBack) {
            int32_t row = 1;
            q.param_i32(0, row);
            a.width = static_cast<uint64_t>(row);
        }
        if (route == Route::SoftMaxBack || route == Route::RmsNormBack) a.g = gview(*q.s1);
        a.eps = p0;
        a.rows = count / a.width;
        return launched(emel::launch_generic_rows(a, hs));
    }
    case Route::RepeatBack: case Route::Concat: case Route::Diag: case Route::DiagMask: case Route::Fill:
    case Route::Arange: {
        emel::GenOrdArgs a{};
        a.y = gview(dst);
        if (q.s0) a.a = gview(*q.s0);
        if (route == Route::Concat) a.b = gview(*q.s1);
        a.p0 = p0;
        a.p1 = p1;
        a.axis = static_cast<uint32_t>(concat_axis);
        int32_t n_past = 0;
        if (route == Route::DiagMask) q.param_i32(0, n_past);
        a.n_past = static_cast<uint64_t>(n_past);
        switch (route) {
        case Route::RepeatBack: a.op = emel::GenOrd::RepeatBack; break;
        case Route::Concat: a.op = emel::GenOrd::Concat; break;
        case Route::Diag: a.op = emel::GenOrd::Diag; break;
        case Route::DiagMask: a.op = op == kDiagMaskInf ? emel::GenOrd::DiagMaskInf : emel::GenOrd::DiagMaskZero; break;
        case Route::Fill: a.op = emel::GenOrd::Fill; break;
        default: a.op = emel::GenOrd::Arange; break;
        }
        return launched(emel::launch_generic_ordinal(a, hs));
    }
    case Route::L2Norm: {
        void *ws = nullptr;
        StreamLease lease;
        s = lease.acquire(hs);
        if (s == EMEL_OK) s = lease.work(emel::generic_workspace_bytes(emel::GenWork::L2Norm), &ws);
        if (s != EMEL_OK) return s;
        return launched(emel::launch_generic_l2_norm(gview(*q.s0), gview(dst), ws, hs));
    }
    case Route::CountEqual: {
        void *ws = nullptr;
        StreamLease lease;
        s = lease.acquire(hs);
        if (s == EMEL_OK) s = lease.work(emel::generic_workspace_bytes(emel::GenWork::CountEqual), &ws);
        if (s != EMEL_OK) return s;
        return launched(emel::launch_generic_count_equal(gview(*q.s0), gview(*q.s1), static_cast<float *>(dmut.data),
                                                         ws, hs));
    }
    case Route::MulMatF32: case Route::MulMatF16: case Route::MulMatArgmax: {
        emel::GenMatArgs a{};
        a.lhs = gview(*q.s0);
        a.rhs = gview(*q.s1);
        a.y = gview(dst);
        a.k = q.s0->ne[0];
        a.m = q.s0->ne[1];
        a.n = route == Route::MulMatF32 ? q.s1->ne[0] : q.s1->ne[1];
        a.f16 = route == Route::MulMatF16;
        a.argmax = route == Route::MulMatArgmax;
        a.index_out = q.r.index_out;
        StreamLease lease;
        if (a.argmax) {
            s = lease.acquire(hs);
            if (s == EMEL_OK) s = lease.work(emel::generic_workspace_bytes(emel::GenWork::MulMatArgmax), &a.workspace);
            if (s != EMEL_OK) return s;
        }
        return launched(emel::launch_generic_mul_mat(a, hs));
    }
    default:
        return fail(EMEL_ERR_INTERNAL, "unrouted generic request");
    }
}

} // namespace

emel_status emel_generic_dispatch(const emel_generic_request *request, emel_stream stream)
{
    if (!request) return fail(EMEL_ERR_INVALID_ARGUMENT, "null request");
    const emel_generic_request &r = *request;
    // Values no Rust GenericRequest can hold.
    if (r.operation >= kGenericOps) return fail(EMEL_ERR_INVALID_ARGUMENT, "operation code outside 0..94");
    if (r.unary_subop > 21 || r.glu_subop > 5 || r.pool_subop > 1)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "subop code outside its wire range");
    if (r.op_params_size > 64 || r.reserved != 0) return fail(EMEL_ERR_INVALID_ARGUMENT, "op_params_size > 64");
    for (const emel_tensor_view *v : {r.src0, r.src1, r.src2, reinterpret_cast<const emel_tensor_view *>(r.dst)})
        if (v && (v->dtype > 255 || v->reserved != 0))
            return fail(EMEL_ERR_INVALID_ARGUMENT, "view dtype outside the wire range");
    const GenReq q(r);
    int concat_axis = 0;
    const Route route = gen_route(q, concat_axis);
    if (route != Route::None) return gen_execute(q, route, concat_axis, stream);
    const bool valid = gen_request_valid(q);
    if (valid && gen_maintained(r.operation))
        return fail(EMEL_ERR_INVALID_SHAPE, "the operation's maintained route rejects the request");
    if (valid) return fail(EMEL_ERR_UNSUPPORTED_OPERATION, "no maintained route for this operation");
    return fail(EMEL_ERR_INVALID_SHAPE, "the request failed validation");
}

// ---- emel-logits: native sampler and candidate validator --------------------------

namespace {

constexpr uint64_t kParkMillerModulus = 2147483647u; // sampler/sm.rs:22
constexpr uint64_t kParkMillerMultiplier = 16807u;   // sampler/sm.rs:23

// state * 16807^steps mod (2^31 - 1): the state after `steps` draws.
uint32_t park_miller_advance(uint32_t state, uint64_t steps)
{
    uint64_t r = state % kParkMillerModulus, b = kParkMillerMultiplier;
    while (steps) {
        if (steps & 1) r = r * b % kParkMillerModulus;
        b = b * b % kParkMillerModulus;
        steps >>= 1;
    }
    return static_cast<uint32_t>(r);
}

struct ByteRange {
    uintptr_t lo, hi;
};
ByteRange span_of(const void *p, uint64_t rows, uint64_t stride, uint64_t width, uint64_t elem)
{
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    return ByteRange{lo, lo + ((rows - 1) * stride + width) * elem};
}
bool pairwise_disjoint(const ByteRange *r, int n)
{
    for (int i = 0; i < n; ++i)
        for (int j = i + 1; j < n; ++j)
            if (r[i].lo < r[j].hi && r[j].lo < r[i].hi) return false;
    return true;
}

// rows of `width` elements, `stride` apart, inside a buffer of `len` elements
bool rows_fit(uint64_t rows, uint64_t stride, uint64_t width, uint64_t len)
{
    if (rows > 1 && stride < width) return false; // rows of one call never share elements
    const u128 need = static_cast<u128>(rows - 1) * stride + width;
    return need <= len;
}

} // namespace

emel_status emel_sample_temperature_top_k_rows(const emel_sample_temperature_top_k_request *req,
                                               const emel_sample_rows *rows, emel_stream stream)
{
    if (!req || !rows) return fail(EMEL_ERR_INVALID_ARGUMENT, "null request");
    if (req->reserved != 0) return fail(EMEL_ERR_INVALID_ARGUMENT, "reserved must be 0");
    const uint64_t nrows = rows->rows;
    if (nrows == 0 || nrows > 0xffffffffull) return fail(EMEL_ERR_INVALID_ARGUMENT, "row count outside [1, 2^32)");
    if (!req->random_state) return fail(EMEL_ERR_INVALID_ARGUMENT, "null random_state");
    const uint64_t card = req->card, top_k = req->top_k;
    const float temperature = req->temperature;
    // guard_temperature_valid (sampler/sm.rs:729-747), for every row
    bool valid = card > 0 && top_k > 0 && top_k <= card && std::isfinite(temperature) && temperature > 0.0f &&
                 rows_fit(nrows, rows->logits_stride, card, req->logits_len) &&
                 rows_fit(nrows, rows->sorted_stride, card, req->sorted_indices_len) &&
                 rows_fit(nrows, rows->top_stride, top_k, req->top_probabilities_len) &&
                 rows_fit(nrows, rows->top_stride, top_k, req->top_indices_len);
    for (uint64_t r = 0; valid && r < nrows; ++r) valid = req->random_state[r] % kParkMillerModulus != 0;
    if (!valid) return fail(EMEL_ERR_INVALID_REQUEST, "sampler request failed its guard");
    if (!req->logits || !req->sorted_indices || !req->top_probabilities || !req->top_indices ||
        !req->selected_token_out || !req->selected_score_out)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "null buffer");
    // limits of this implementation (indices are i32 in the reference's outputs)
    if (card > 0x7fffffffull) return fail(EMEL_ERR_INVALID_ARGUMENT, "card beyond i32 indices");
    const ByteRange spans[7] = {
        span_of(req->logits, nrows, rows->logits_stride, card, 4),
        span_of(req->sorted_indices, nrows, rows->sorted_stride, card, 4),
        span_of(req->top_probabilities, nrows, rows->top_stride, top_k, 4),
        span_of(req->top_indices, nrows, rows->top_stride, top_k, 4),
        span_of(req->selected_token_out, nrows, 1, 1, 4),
        span_of(req->selected_score_out, nrows, 1, 1, 4),
        req->status_out ? span_of(req->status_out, nrows, 1, 1, 4) : ByteRange{0, 0},
    };
    if (!pairwise_disjoint(spans, req->status_out ? 7 : 6))
        return fail(EMEL_ERR_INVALID_ARGUMENT, "sampler buffers overlap");
    const uintptr_t misaligned = reinterpret_cast<uintptr_t>(req->logits) | reinterpret_cast<uintptr_t>(req->sorted_indices) |
                                 reinterpret_cast<uintptr_t>(req->top_probabilities) |
                                 reinterpret_cast<uintptr_t>(req->top_indices) |
                                 reinterpret_cast<uintptr_t>(req->selected_token_out) |
                                 reinterpret_cast<uintptr_t>(req->selected_score_out) |
                                 reinterpret_cast<uintptr_t>(req->status_out);
    if (misaligned & 3u) return fail(EMEL_ERR_INVALID_ARGUMENT, "sampler buffers must be 4-byte aligned");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::SamplerArgs a{};
    a.rows = static_cast<uint32_t>(nrows);
    a.card = card;
    a.top_k = static_cast<uint32_t>(top_k);
    a.scale = 1.0f / temperature; // effect_scale_temperature (sm.rs:766), f32
    a.logits = req->logits;
    a.logits_ld = static_cast<int64_t>(rows->logits_stride);
    a.sorted = req->sorted_indices;
    a.sorted_ld = static_cast<int64_t>(rows->sorted_stride);
    a.top_p = req->top_probabilities;
    a.top_i = req->top_indices;
    a.top_ld = static_cast<int64_t>(rows->top_stride);
    a.selected = req->selected_token_out;
    a.score = req->selected_score_out;
    a.status = req->status_out;
    a.states = req->random_state;
    // The draws advance the host-resident random_state when the call is
    // enqueued; a replayed graph would redraw from the captured states.
    s = not_capturing(as_stream(stream), "the sampler (its random_state advances on the host)");
    StreamLease lease;
    if (s == EMEL_OK) s = lease.acquire(as_stream(stream));
    if (s == EMEL_OK) s = lease.work(emel::sampler_workspace_bytes(a.rows, card, a.top_k), &a.workspace);
    if (s != EMEL_OK) return s;
    const hipError_t e = emel::launch_sampler(a, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "sampler launch");
    // effect_select_top_k (sm.rs:821-847) leaves the state after top_k draws
    for (uint64_t r = 0; r < nrows; ++r) req->random_state[r] = park_miller_advance(req->random_state[r], top_k);
    return launched(hipSuccess);
}

emel_status emel_sample_temperature_top_k(const emel_sample_temperature_top_k_request *req, emel_stream stream)
{
    if (!req) return fail(EMEL_ERR_INVALID_ARGUMENT, "null request");
    const emel_sample_rows one{1, req->card, req->card, req->top_k};
    return emel_sample_temperature_top_k_rows(req, &one, stream);
}

emel_status emel_sample_preselected(uint64_t vocab_size, int32_t selected_token, int32_t *token_out)
{
    if (!token_out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null output");
    // guard_preselected_valid (sampler/sm.rs:685-695)
    if (!(vocab_size > 0 && selected_token >= 0 && static_cast<uint64_t>(selected_token) < vocab_size))
        return fail(EMEL_ERR_INVALID_REQUEST, "preselected token outside the vocabulary");
    *token_out = selected_token;
    g_last_error.clear();
    return EMEL_OK;
}

emel_status emel_logits_validator_build(const float *logits, uint64_t logits_len, int32_t vocab_size,
                                        int32_t *candidate_ids, uint64_t candidate_ids_len, float *candidate_scores,
                                        uint64_t candidate_scores_len, int32_t candidate_capacity,
                                        int32_t *candidate_count_out, int32_t *error_out, emel_stream stream)
{
    if (!candidate_count_out || !error_out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null output");
    // begin_build, then valid_request (validator/sm.rs)
    *candidate_count_out = 0;
    *error_out = EMEL_VALIDATOR_NONE;
    const auto fits = [&](uint64_t len) { return len <= 0x7fffffffull && static_cast<int64_t>(len) >= vocab_size; };
    if (!(vocab_size > 0 && candidate_capacity >= vocab_size && fits(logits_len) && fits(candidate_ids_len) &&
          fits(candidate_scores_len))) {
        *candidate_count_out = 0;
        *error_out = EMEL_VALIDATOR_INVALID_REQUEST;
        return fail(EMEL_ERR_INVALID_REQUEST, "validator request failed its guard");
    }
    if (!logits || !candidate_ids || !candidate_scores) return fail(EMEL_ERR_INVALID_ARGUMENT, "null buffer");
    const uint64_t n = static_cast<uint64_t>(vocab_size);
    const ByteRange spans[3] = {span_of(logits, 1, 0, n, 4), span_of(candidate_ids, 1, 0, n, 4),
                                span_of(candidate_scores, 1, 0, n, 4)};
    if (!pairwise_disjoint(spans, 3)) return fail(EMEL_ERR_INVALID_ARGUMENT, "validator buffers overlap");
    if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(candidate_ids) |
         reinterpret_cast<uintptr_t>(candidate_scores)) & 3u)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "validator buffers must be 4-byte aligned");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    void *ws = nullptr;
    StreamLease lease;
    s = lease.acquire(as_stream(stream));
    if (s == EMEL_OK) s = lease.work(emel::validator_workspace_bytes(n), &ws);
    if (s != EMEL_OK) return s;
    const hipError_t e = emel::launch_validator(logits, n, candidate_ids, candidate_scores, ws, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "validator launch");
    *candidate_count_out = vocab_size; // execute_build
    return launched(hipSuccess);
}

// ---- the remaining typed events of activation.rs, elementwise.rs, diag.rs and
// ---- group_norm.rs -------------------------------------------------------------

namespace {

// activation.rs views_valid + same_shape (:168-175): Layout::validate on both,
// then equal extents.
emel_status activation_guard(const emel_tensor_view *in, const emel_tensor_view_mut *out)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_f32(*in, false) || !valid_f32(*out, false))
        return fail(EMEL_ERR_INVALID_VIEW, "activation view failed validation");
    if (!same_ne(*in, *out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "activation shapes differ");
    return EMEL_OK;
}

// diag.rs square_side (:107-120).
bool square_side(uint64_t len, uint64_t &side)
{
    if (len == 0) return false;
    const uint64_t r = static_cast<uint64_t>(std::sqrt(static_cast<double>(len)));
    for (uint64_t s = r > 2 ? r - 2 : 0; s <= r + 2; ++s)
        if (static_cast<u128>(s) * s == len) {
            side = s;
            return true;
        }
    return false;
}

// A validated F32 view as the generic kernels' operand (element strides).
template <class V>
emel::GView gview_of(const V &v)
{
    const Operand o = operand(v, 4);
    emel::GView g{};
    g.data = o.data;
    for (int d = 0; d < 4; ++d) {
        g.ne[d] = o.ne[d];
        g.st[d] = o.st[d];
    }
    return g;
}

emel::GView dense_gview(const float *p, uint64_t n0, uint64_t n1)
{
    emel::GView v{};
    v.data = const_cast<float *>(p);
    v.ne[0] = n0;
    v.ne[1] = n1;
    v.ne[2] = v.ne[3] = 1;
    v.st[0] = 1;
    v.st[1] = static_cast<int64_t>(n0);
    v.st[2] = v.st[3] = static_cast<int64_t>(n0 * n1);
    return v;
}

// Exact aliasing (output == input) is allowed: every element is read before
// its own write.  Any other overlap is refused.
bool slices_ok(const float *in, uint64_t in_len, const float *out, uint64_t out_len)
{
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(in), a1 = a0 + in_len * 4;
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(out), b1 = b0 + out_len * 4;
    return a1 <= b0 || b1 <= a0 || (a0 == b0 && in_len == out_len);
}

emel_status diag_mask(emel::GenOrd which, const float *input, uint64_t input_len, float *output, uint64_t output_len,
                      int32_t n_past, emel_stream stream)
{
    uint64_t side = 0;
    // mask_valid (diag.rs:122-124)
    if (!(n_past >= 0 && input_len == output_len && square_side(input_len, side)))
        return fail(EMEL_ERR_INVALID_SHAPE, "diag mask needs a non-empty square slice and n_past >= 0");
    if (!input || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    if (!slices_ok(input, input_len, output, output_len)) return fail(EMEL_ERR_INVALID_ARGUMENT, "slices overlap");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::GenOrdArgs a{};
    a.op = which;
    a.a = dense_gview(input, side, side);
    a.y = dense_gview(output, side, side);
    a.n_past = static_cast<uint64_t>(n_past);
    return launched(emel::launch_generic_ordinal(a, as_stream(stream)));
}

} // namespace

emel_status emel_op_clamp(const emel_tensor_view *in, const emel_tensor_view_mut *out, float min, float max,
                          emel_stream stream)
{
    emel_status s = activation_guard(in, out);
    if (s != EMEL_OK) return s;
    return elementwise(emel::Ew::ClampStd, in, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, out, min,
                       stream, max);
}

emel_status emel_op_leaky_relu(const emel_tensor_view *in, const emel_tensor_view_mut *out, float negative_slope,
                               emel_stream stream)
{
    emel_status s = activation_guard(in, out);
    if (s != EMEL_OK) return s;
    return elementwise(emel::Ew::LeakyRelu, in, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, out,
                       negative_slope, stream);
}

emel_status emel_op_silu_back(const emel_tensor_view *in, const emel_tensor_view *gradient,
                              const emel_tensor_view_mut *out, emel_stream stream)
{
    if (!in || !gradient || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // three_views_valid / three_views_same_shape (activation.rs:176-190)
    if (!valid_f32(*in, false) || !valid_f32(*gradient, false) || !valid_f32(*out, false))
        return fail(EMEL_ERR_INVALID_VIEW, "silu_back view failed validation");
    if (!same_ne(*in, *gradient) || !same_ne(*in, *out))
        return fail(EMEL_ERR_SHAPE_MISMATCH, "silu_back shapes differ");
    return elementwise(emel::Ew::SiluBack, in, emel::Addr::SameCoords, gradient, emel::Addr::SameCoords, out, 0.0f,
                       stream);
}

emel_status emel_op_add1(const emel_tensor_view *src, float scalar, const emel_tensor_view_mut *dst, emel_stream stream)
{
    if (!src || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // valid_pair / same_shape (elementwise.rs:203-209)
    if (!valid_f32(*src, false) || !valid_f32(*dst, false))
        return fail(EMEL_ERR_INVALID_VIEW, "add1 view failed validation");
    if (!same_ne(*src, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "add1 shapes differ");
    return elementwise(emel::Ew::Add1, src, emel::Addr::SameCoords, nullptr, emel::Addr::SameCoords, dst, scalar,
                       stream);
}

emel_status emel_op_acc(const emel_tensor_view *base, const emel_tensor_view *update, const emel_tensor_view_mut *dst,
                        uint64_t offset, emel_stream stream)
{
    if (!base || !update || !dst) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // guard order of the machine (elementwise.rs:110-116, :227-243)
    const bool pair = valid_f32(*base, false) && valid_f32(*dst, false) && valid_f32(*update, false);
    if (pair && !same_ne(*base, *dst)) return fail(EMEL_ERR_SHAPE_MISMATCH, "acc base and dst shapes differ");
    const bool views = pair && dense_for(*base, EMEL_DTYPE_F32, 4) && dense_for(*update, EMEL_DTYPE_F32, 4) &&
                       dense_for(*dst, EMEL_DTYPE_F32, 4);
    if (!views) return fail(EMEL_ERR_INVALID_VIEW, "acc views must be valid dense F32");
    const uint64_t n = count_or_zero(*dst), nu = count_or_zero(*update);
    if (!(offset <= n && nu <= n - offset)) return fail(EMEL_ERR_INVALID_OFFSET, "acc update extends past dst");
    if (!overlap_ok(*dst, 4, *base, 4) || !overlap_ok(*dst, 4, *update, 4) || dst->data == update->data)
        return fail(EMEL_ERR_INVALID_VIEW, "dst overlaps the update or partially overlaps the base");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    return launched(emel::launch_acc(static_cast<const float *>(base->data), static_cast<const float *>(update->data),
                                     static_cast<float *>(dst->data), n, offset, nu, as_stream(stream)));
}

emel_status emel_op_diag(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                         emel_stream stream)
{
    // OpDiag::side (diag.rs:57-64)
    if (input_len == 0 || static_cast<u128>(input_len) * input_len != output_len)
        return fail(EMEL_ERR_INVALID_SHAPE, "diag needs a non-empty input and an n*n output");
    if (!input || !output) return fail(EMEL_ERR_INVALID_ARGUMENT, "null slice");
    if (!slices_ok(input, input_len, output, output_len) || input == output)
        return fail(EMEL_ERR_INVALID_ARGUMENT, "slices overlap");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::GenOrdArgs a{};
    a.op = emel::GenOrd::Diag;
    a.a = dense_gview(input, input_len, 1);
    a.y = dense_gview(output, input_len, input_len);
    return launched(emel::launch_generic_ordinal(a, as_stream(stream)));
}

emel_status emel_op_diag_mask_inf(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                                  int32_t n_past, emel_stream stream)
{
    return diag_mask(emel::GenOrd::DiagMaskInf, input, input_len, output, output_len, n_past, stream);
}

emel_status emel_op_diag_mask_zero(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                                   int32_t n_past, emel_stream stream)
{
    return diag_mask(emel::GenOrd::DiagMaskZero, input, input_len, output, output_len, n_past, stream);
}

emel_status emel_op_group_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, uint64_t groups,
                               float epsilon, emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    // the machine's guard order (group_norm.rs:179-196, :205-226)
    if (!valid_normalization(*in) || !valid_normalization(*out))
        return fail(EMEL_ERR_INVALID_VIEW, "group_norm view failed validation");
    if (!same_ne(*in, *out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "group_norm shapes differ");
    if (!(groups != 0 && in->ne[2] % groups == 0 && std::isfinite(epsilon) && epsilon >= 0.0f))
        return fail(EMEL_ERR_INVALID_PARAMETERS, "groups must divide the channels; epsilon finite and >= 0");
    if (!overlap_ok(*out, 4, *in, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst partially overlaps the source");
    if (!elements_disjoint(*out, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst elements overlap one another");
    if (groups > 0x7fffffffull) return fail(EMEL_ERR_INVALID_PARAMETERS, "too many groups");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    const hipError_t e = emel::launch_group_norm(operand(*in, 4), operand(*out, 4), static_cast<uint32_t>(groups),
                                                 epsilon, as_stream(stream));
    if (e == hipErrorInvalidValue) return fail(EMEL_ERR_INTERNAL, "group_norm group size outside the supported range");
    return launched(e);
}

emel_status emel_op_l2_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream)
{
    if (!in || !out) return fail(EMEL_ERR_INVALID_ARGUMENT, "null view");
    if (!valid_normalization(*in) || !valid_normalization(*out))
        return fail(EMEL_ERR_INVALID_VIEW, "l2_norm view failed validation");
    if (!same_ne(*in, *out)) return fail(EMEL_ERR_SHAPE_MISMATCH, "l2_norm shapes differ");
    if (!overlap_ok(*out, 4, *in, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst partially overlaps the source");
    if (!elements_disjoint(*out, 4)) return fail(EMEL_ERR_INVALID_VIEW, "dst elements overlap one another");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    // guard_l2_norm_valid needs the sum (group_norm.rs:252-260): it is formed on
    // the device, read back, and checked before anything is written.
    const hipStream_t hs = as_stream(stream);
    s = not_capturing(hs, "l2_norm (its ZeroNorm guard reads the sum back)");
    StreamLease lease;
    if (s == EMEL_OK) s = lease.acquire(hs);
    void *ws = nullptr, *stage = nullptr;
    if (s == EMEL_OK) s = lease.work(2 * sizeof(float), &ws);
    if (s == EMEL_OK) s = lease.staging(2 * sizeof(float), &stage);
    if (s != EMEL_OK) return s;
    const emel::GView x = gview_of(*in), y = gview_of(*out);
    hipError_t e = emel::launch_generic_l2_sum(x, ws, hs);
    if (e == hipSuccess) e = hipMemcpyAsync(stage, ws, 2 * sizeof(float), hipMemcpyDeviceToHost, hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e != hipSuccess) return hip_fail(e, "l2_norm sum");
    const float sum = static_cast<const float *>(stage)[1];
    if (!(sum > 0.0f)) return fail(EMEL_ERR_ZERO_NORM, "l2_norm: the sum of squares is not positive");
    return launched(emel::launch_generic_l2_apply(x, y, ws, hs));
}
