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
#include <mutex>
#include <string>
#include <utility>

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

// Per-(device, stream) scratch for the split-row reductions' partials.
// Calls on one stream run in order, so they can share one buffer; different
// streams get different buffers.
struct Workspace {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};
std::map<std::pair<int, hipStream_t>, Workspace> g_workspaces;

emel_status workspace_for(hipStream_t stream, uint64_t bytes, void **out)
{
    *out = nullptr;
    if (bytes == 0) return EMEL_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_mutex);
    Workspace &w = g_workspaces[{dev, stream}];
    if (w.bytes < bytes) {
        if (w.ptr) {
            e = hipStreamSynchronize(stream); // the old buffer may still be in use
            if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        const uint64_t size = bytes < (uint64_t{1} << 20) ? (uint64_t{1} << 20) : bytes;
        e = hipMalloc(&w.ptr, size);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
        w.bytes = size;
    }
    *out = w.ptr;
    return EMEL_OK;
}

emel_status launched(hipError_t e)
{
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    g_last_error.clear();
    return EMEL_OK;
}

hipStream_t as_stream(emel_stream s) { return static_cast<hipStream_t>(s); }

// ---- op plumbing ---------------------------------------------------------------

emel_status elementwise(emel::Ew op, const emel_tensor_view *a, emel::Addr aa, const emel_tensor_view *b,
                        emel::Addr ba, const emel_tensor_view_mut *o, float scale, emel_stream stream)
{
    if (!overlap_ok(*o, 4, *a, 4) || (b && !overlap_ok(*o, 4, *b, 4)))
        return fail(EMEL_ERR_INVALID_VIEW, "dst partially overlaps a source");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::EwArgs args{};
    args.op = op;
    args.scale = scale;
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
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    return launched(emel::launch_rows(args, as_stream(stream)));
}

emel_status reduce(emel::RedOp op, const emel_tensor_view &src, const emel_tensor_view_mut &dst, emel_stream stream)
{
    if (!overlap_ok(dst, 4, src, 4) || dst.data == src.data)
        return fail(EMEL_ERR_INVALID_VIEW, "dst overlaps the source");
    emel_status s = ensure_device();
    if (s != EMEL_OK) return s;
    emel::RedArgs args{};
    args.op = op;
    args.x = operand(src, 4);
    args.dst = dst.data;
    args.dst_view = operand(dst, 4);
    if (dst.dtype == EMEL_DTYPE_I32)
        for (int d = 0; d < 4; ++d) args.dst_view.st[d] = static_cast<int64_t>(dst.nb[d] / 4);
    const uint64_t bytes = emel::reduce_workspace_bytes(args);
    s = workspace_for(as_stream(stream), bytes, &args.workspace);
    if (s != EMEL_OK) return s;
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

extern "C" {

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
        for (auto it = g_workspaces.begin(); it != g_workspaces.end();) {
            if (it->first.second == as_stream(stream)) {
                (void)hipStreamSynchronize(as_stream(stream));
                (void)hipFree(it->second.ptr);
                it = g_workspaces.erase(it);
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
    for (auto &kv : g_workspaces) (void)hipFree(kv.second.ptr);
    g_workspaces.clear();
    return e == hipSuccess ? EMEL_OK : hip_fail(e, "hipDeviceSynchronize");
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

} // extern "C"
