// oxm_capi.cpp -- the C-ABI of the gfx950 GEMM backend (include/oxm.h).
//
// Host-side responsibilities: validate every argument (shapes, strides,
// dtypes, devices, and that each view lies inside its device allocation) and
// report failures as oxmera's typed errors; classify each operand's layout to
// pick a global loader; fill the kernel argument block and launch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/oxm.h"
#include "gemm_args.hpp"
#include "elementwise_launch.hpp"
#include "gemm_launch.hpp"
#include "glue_launch.hpp"

namespace {

thread_local std::string g_last_error;

oxm_status fail(oxm_status st, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

oxm_status ok() {
    g_last_error.clear();
    return OXM_OK;
}

// Debug-style rendering of a shape, "[2, 3]", as oxmera's Shape prints.
std::string shape_str(int n, const int64_t *d) {
    std::string s = "[";
    for (int i = 0; i < n; ++i) {
        if (i) s += ", ";
        s += std::to_string((long long)d[i]);
    }
    return s + "]";
}

const char *dtype_name(int dt) {
    switch (dt) {
    case OXM_F32: return "F32";
    case OXM_F64: return "F64";
    case OXM_I32: return "I32";
    case OXM_I64: return "I64";
    case OXM_U8: return "U8";
    case OXM_BOOL: return "Bool";
    case OXM_BF16: return "BF16";
    case OXM_F16: return "F16";
    default: return "?";
    }
}

int dtype_size(int dt) {
    switch (dt) {
    case OXM_F32: case OXM_I32: return 4;
    case OXM_F64: case OXM_I64: return 8;
    case OXM_U8: case OXM_BOOL: return 1;
    case OXM_BF16: case OXM_F16: return 2;
    default: return 0;
    }
}

std::string device_str(int d) { return d < 0 ? std::string("Cpu") : "Rocm { index: " + std::to_string(d) + " }"; }

bool is_gemm_dtype(int dt) { return dt == OXM_F32 || dt == OXM_BF16 || dt == OXM_F16; }

// Structural checks of a view: pointers, rank, non-negative extents and offset.
oxm_status check_view(const oxm_view *v, const char *what, const char *op) {
    if (!v) return fail(OXM_E_INVALID_ARGUMENT, "%s: %s view is NULL", op, what);
    if (v->ndim < 0 || v->ndim > OXM_MAX_DIMS)
        return fail(OXM_E_RANK_MISMATCH, "%s: %s has rank %d, supported 0..%d", op, what, v->ndim, OXM_MAX_DIMS);
    if (v->ndim > 0 && (!v->shape || !v->strides))
        return fail(OXM_E_INVALID_ARGUMENT, "%s: %s has NULL shape or strides", op, what);
    if (dtype_size(v->dtype) == 0) return fail(OXM_E_INVALID_ARGUMENT, "%s: %s has unknown dtype %d", op, what, v->dtype);
    for (int i = 0; i < v->ndim; ++i)
        if (v->shape[i] < 0) return fail(OXM_E_INVALID_ARGUMENT, "%s: %s has negative extent", op, what);
    if (v->offset < 0) return fail(OXM_E_INVALID_ARGUMENT, "%s: %s has negative offset", op, what);
    // every later element count (numel, M*N, batch products) must fit int64
    bool empty = false;
    for (int i = 0; i < v->ndim; ++i) empty = empty || v->shape[i] == 0;
    int64_t n = 1;
    for (int i = 0; i < v->ndim && !empty; ++i)
        if (__builtin_mul_overflow(n, v->shape[i], &n))
            return fail(OXM_E_INDEX_OUT_OF_BOUNDS, "%s: %s of shape %s has more elements than int64 can count", op,
                        what, shape_str(v->ndim, v->shape).c_str());
    return OXM_OK;
}

// Element count of a view that passed check_view (which rules out overflow).
int64_t numel(const oxm_view *v) {
    int64_t n = 1;
    for (int i = 0; i < v->ndim; ++i) n *= v->shape[i];
    return n;
}

// The bytes a non-empty view can address, relative to v->data: [lo, hi).
// Every product and sum is checked, so a view whose strides or offset would
// wrap int64 (e.g. stride 2^61 of an F32 view) is refused instead of
// producing a range that looks valid.
bool byte_range(const oxm_view *v, int64_t *lo_bytes, int64_t *hi_bytes) {
    const int64_t es = dtype_size(v->dtype);
    int64_t lo = v->offset, hi = v->offset;
    for (int i = 0; i < v->ndim; ++i) {
        int64_t span;
        if (__builtin_mul_overflow(v->shape[i] - 1, v->strides[i], &span)) return false;
        if (__builtin_add_overflow(span < 0 ? lo : hi, span, span < 0 ? &lo : &hi)) return false;
    }
    int64_t hi1;
    if (__builtin_add_overflow(hi, (int64_t)1, &hi1)) return false;
    return !__builtin_mul_overflow(lo, es, lo_bytes) && !__builtin_mul_overflow(hi1, es, hi_bytes);
}

// Absolute address range [lo, hi) of a non-empty view that passed
// check_view_memory (its byte range is known not to overflow).
struct Span {
    uintptr_t lo, hi;
};
Span span_of(const oxm_view *v) {
    int64_t lo = 0, hi = 0;
    if (numel(v) == 0 || !byte_range(v, &lo, &hi)) return {0, 0};
    return {(uintptr_t)v->data + (uintptr_t)lo, (uintptr_t)v->data + (uintptr_t)hi};
}
Span span_bytes(const void *p, int64_t bytes) { return {(uintptr_t)p, (uintptr_t)p + (uintptr_t)bytes}; }
bool overlaps(Span x, Span y) { return x.lo < x.hi && y.lo < y.hi && x.lo < y.hi && y.lo < x.hi; }

// An output must be fresh storage ("the output of every operation is a fresh
// contiguous tensor", crates/oxmera-ops/src/lib.rs:16-17): a kernel that
// writes tiles, transposes through LDS or splits a reduction would read
// values it has already overwritten.  Byte ranges are compared, so two
// interleaved views of one buffer (even and odd columns) are refused too.
oxm_status refuse_overlap(Span out, const char *out_name, Span in, const char *in_name, const char *op) {
    if (!overlaps(out, in)) return OXM_OK;
    return fail(OXM_E_INVALID_ARGUMENT, "%s: the %s overlaps the %s (an output must not share memory with an input)",
                op, out_name, in_name);
}

// An elementwise input may be the output itself -- same first element and,
// over the output's shape, the output's own strides -- since every element is
// read and written by the same thread; any other overlap is refused.
bool same_elements(const oxm_view *out, const void *in_first, const int64_t *in_strides) {
    const int es = dtype_size(out->dtype);
    if ((const char *)in_first != (const char *)out->data + out->offset * es) return false;
    for (int d = 0; d < out->ndim; ++d)
        if (out->shape[d] != 1 && in_strides[d] != out->strides[d]) return false;
    return true;
}

bool is_contiguous(const oxm_view *v) {
    int64_t expect = 1;
    for (int i = v->ndim - 1; i >= 0; --i) {
        if (v->shape[i] != 1 && v->strides[i] != expect) return false;
        expect *= v->shape[i];
    }
    return true;
}

// Allocations made through oxm_alloc: base -> (bytes, device).  Views over
// them are validated against this registry without any HIP query (the HIP
// pointer queries synchronise with the device, which would serialise
// asynchronous launches); other pointers fall back to the HIP queries.
struct AllocInfo {
    size_t bytes;
    int device;
};
std::mutex g_alloc_mu;
std::map<uintptr_t, AllocInfo> g_allocs;

// The registered allocation containing p, if any.
bool find_alloc(const void *p, uintptr_t *base, AllocInfo *info) {
    const uintptr_t a = (uintptr_t)p;
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_allocs.upper_bound(a);
    if (it == g_allocs.begin()) return false;
    --it;
    if (a >= it->first + it->second.bytes) return false;
    *base = it->first;
    *info = it->second;
    return true;
}

// The device allocation holding [p, p + bytes) must contain it entirely and
// live on `device`.  This is what keeps a malformed view from reaching the
// GPU as an out-of-bounds access.
oxm_status check_device_range(const void *p, int64_t lo_bytes, int64_t hi_bytes, int device, const char *what,
                              const char *op) {
    uintptr_t rbase;
    AllocInfo info;
    if (find_alloc(p, &rbase, &info)) {
        if (info.device != device)
            return fail(OXM_E_DEVICE_MISMATCH, "%s: %s lives on %s, expected %s", op, what,
                        device_str(info.device).c_str(), device_str(device).c_str());
        const int64_t rel = (int64_t)((uintptr_t)p - rbase);
        int64_t a0 = 0, a1 = 0;
        if (__builtin_add_overflow(rel, lo_bytes, &a0) || __builtin_add_overflow(rel, hi_bytes, &a1) || a0 < 0 ||
            a1 > (int64_t)info.bytes)
            return fail(OXM_E_INDEX_OUT_OF_BOUNDS,
                        "%s: %s addresses bytes [%lld, %lld) relative to its pointer, outside its %zu-byte allocation",
                        op, what, (long long)lo_bytes, (long long)hi_bytes, info.bytes);
        return OXM_OK;
    }
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof attr);
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(OXM_E_DEVICE_MISMATCH, "%s: %s (%p) is not HIP device memory", op, what, p);
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged)
        return fail(OXM_E_DEVICE_MISMATCH, "%s: %s (%p) is not device memory", op, what, p);
    if (attr.device != device)
        return fail(OXM_E_DEVICE_MISMATCH, "%s: %s lives on %s, expected %s", op, what, device_str(attr.device).c_str(),
                    device_str(device).c_str());
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(OXM_E_HIP, "%s: cannot query the allocation of %s", op, what);
    }
    const int64_t rel = (int64_t)((uintptr_t)p - (uintptr_t)base);
    int64_t a0 = 0, a1 = 0;
    if (__builtin_add_overflow(rel, lo_bytes, &a0) || __builtin_add_overflow(rel, hi_bytes, &a1) || a0 < 0 ||
        a1 > (int64_t)size)
        return fail(OXM_E_INDEX_OUT_OF_BOUNDS,
                    "%s: %s addresses bytes [%lld, %lld) relative to its pointer, outside its %zu-byte allocation", op,
                    what, (long long)lo_bytes, (long long)hi_bytes, size);
    return OXM_OK;
}

// Every byte a strided view can address must lie in its allocation
// (Tensor::from_storage's rule, crates/oxmera-tensor/src/tensor.rs:21-28).
oxm_status check_view_memory(const oxm_view *v, const char *what, const char *op) {
    if (numel(v) == 0) return OXM_OK;
    int64_t lo = 0, hi = 0;
    if (!byte_range(v, &lo, &hi))
        return fail(OXM_E_INDEX_OUT_OF_BOUNDS, "%s: the byte range of %s (shape %s) overflows int64", op, what,
                    shape_str(v->ndim, v->shape).c_str());
    return check_device_range(v->data, lo, hi, v->device, what, op);
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

oxm_status hip_fail(hipError_t e, const char *op) {
    return fail(OXM_E_HIP, "%s: HIP error %d (%s)", op, (int)e, hipGetErrorString(e));
}

oxm_status finish(hipStream_t s, const char *op) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, op);
    if (!s) {
        e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) return hip_fail(e, op);
    }
    return ok();
}

// Operand loader choice from the view's strides (see gemm_kernels.hpp).  The
// vector loaders read through a 32-bit buffer resource per tile, so they
// also need non-negative strides and a tile byte range below 2^31.
int classify(const char *ptr, int64_t s_mn, int64_t s_k, int64_t mn, int64_t k, const int64_t *bstr, int nbd,
             int es, int tile_rows) {
    const int64_t vec = 16 / es;
    const int64_t kMaxRec = 0x7FFFFF00LL;
    if (mn == 1) s_mn = 0;
    if (k == 1) s_k = 0;
    if (es == 4) {
        // f32: 16-byte loads need only dword alignment and the loaders
        // handle rows that end mid-chunk, so any non-negative unit-stride
        // layout qualifies.
        // A ragged row needs one whole chunk inside it: K >= 4 (Ld::K), and
        // for Ld::MN at least 4 elements in the last, partial tile.
        const bool al4 = ((uintptr_t)ptr % 4) == 0;
        const int64_t edge = mn % tile_rows;
        if (al4 && s_k == 1 && s_mn >= 0 && (k % vec == 0 || k >= vec) &&
            ((int64_t)tile_rows * s_mn + k) * es <= kMaxRec)
            return k % vec == 0 ? oxm::kLdK : oxm::kLdKR;
        if (al4 && s_mn == 1 && s_k >= 0 && (mn % vec == 0 || edge == 0 || edge >= vec) &&
            (k * s_k + tile_rows) * es <= kMaxRec)
            return mn % vec == 0 ? oxm::kLdMN : oxm::kLdMNR;
        return oxm::kLdG;
    }
    bool aligned = ((uintptr_t)ptr % 16) == 0;
    bool batch_ok = true;
    for (int d = 0; d < nbd; ++d) batch_ok = batch_ok && (bstr[d] % vec == 0);
    if (aligned && batch_ok && s_k == 1 && k % vec == 0 && s_mn % vec == 0 && s_mn >= 0 &&
        ((int64_t)tile_rows * s_mn + k) * es <= kMaxRec)
        return oxm::kLdK;
    if (aligned && batch_ok && s_mn == 1 && mn % vec == 0 && s_k % vec == 0 && s_k >= 0 &&
        (k * s_k + tile_rows) * es <= kMaxRec)
        return oxm::kLdMN;
    return oxm::kLdG;
}

// Tile size from a wave-count model of the 256-CU chip.  A 256x256 tile
// occupies a whole CU (128 KB of LDS), so n256 tiles take ceil(n256 / 256)
// rounds; 128x128 tiles run two per CU, a round of 512 of them taking 0.57
// of a 256x256 round (measured at 4096^3 f32 and 8192^3 bf16), and a part
// round costs its share.  E.g. 4096^3: 1 round vs 1.14 -> 256x256;
// 4097x4095 (272 big tiles): 2 rounds vs 1.18 -> 128x128; C4's 32 batches
// of 512x768: 1 round vs 0.86 -> 128x128.
bool prefer_256_tiles(int64_t M, int64_t N, int64_t batch) {
    const int64_t n256 = ((M + 255) / 256) * ((N + 255) / 256) * batch;
    const int64_t n128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
    const double rounds256 = (double)((n256 + 255) / 256);
    double rounds128 = (double)n128 / 512.0;
    if (rounds128 < 0.5) rounds128 = 0.5;
    return rounds256 < 0.57 * rounds128;
}

// f32 256x192 tiles (direct-to-LDS kernel only) when their rounds, at 0.75
// of a 256x256 round each, beat both other tilings by 5 %: C4's 32 batches
// of 512x768 are 256 such tiles, one round (0.75) against one round of 192
// 256x256 tiles (1.0) or 768 128x128 tiles (0.86); 4096^3 stays on 256x256
// tiles (352 of them would take two rounds).
bool prefer_256x192_tiles(int64_t M, int64_t N, int64_t batch) {
    const int64_t n256 = ((M + 255) / 256) * ((N + 255) / 256) * batch;
    const int64_t n192 = ((M + 255) / 256) * ((N + 191) / 192) * batch;
    const int64_t n128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
    const double t256 = (double)((n256 + 255) / 256), t192 = 0.75 * (double)((n192 + 255) / 256);
    double t128 = (double)n128 / 512.0;
    t128 = 0.57 * (t128 < 0.5 ? 0.5 : t128);
    return t192 < 0.95 * (t256 < t128 ? t256 : t128);
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

bool is_float_dtype(int dt) { return dt == OXM_F32 || dt == OXM_F64 || dt == OXM_BF16 || dt == OXM_F16; }
bool is_int_dtype(int dt) { return dt == OXM_I32 || dt == OXM_I64 || dt == OXM_U8 || dt == OXM_BOOL; }

// Which ops the integer and boolean dtypes carry (elementwise_int.hip): neg
// and abs, add / sub / mul / div / eq, sum and max; Bool has no neg, sub or
// div (NumPy refuses them too).  exp and ln are "float dtypes only"
// (crates/oxmera-ops/src/lib.rs:31-34); sign and dgelu serve the float tape.
bool int_unary_ok(int dt, int op) { return op == OXM_UN_ABS || (op == OXM_UN_NEG && dt != OXM_BOOL); }
bool int_binary_ok(int dt, int op) {
    if (op == OXM_BIN_ADD || op == OXM_BIN_MUL || op == OXM_BIN_EQ) return true;
    return (op == OXM_BIN_SUB || op == OXM_BIN_DIV) && dt != OXM_BOOL;
}

// Row-major iteration space over `shape` for up to three operands (0 = the
// output), dims of extent 1 dropped and neighbours merged where every
// operand walks them as one (st[d] == st[d+1] * shape[d+1]).
oxm::EwShape collapse(int nd, const int64_t *shape, const int64_t *const st[3], int nops) {
    oxm::EwShape s{};
    s.numel = 1;
    for (int d = 0; d < nd; ++d) s.numel *= shape[d];
    int n = 0;
    for (int d = 0; d < nd; ++d) {
        if (shape[d] == 1) continue;
        bool merge = n > 0;
        for (int o = 0; o < nops && merge; ++o) merge = s.st[o][n - 1] == st[o][d] * shape[d];
        if (merge) {
            s.shape[n - 1] *= shape[d];
            for (int o = 0; o < nops; ++o) s.st[o][n - 1] = st[o][d];
        } else {
            s.shape[n] = shape[d];
            for (int o = 0; o < nops; ++o) s.st[o][n] = st[o][d];
            ++n;
        }
    }
    if (n == 0) {  // every extent 1: one element
        s.shape[0] = 1;
        n = 1;
    }
    s.ndim = n;
    return s;
}

// 16-byte path: every operand walks the space as one unit-stride run from a
// 16-byte aligned address, and the run is a whole number of 16-byte chunks.
bool contig16(const oxm::EwShape &s, int nops, const void *const ptr[3], int es) {
    if (s.ndim != 1 || (s.numel * es) % 16 != 0) return false;
    for (int o = 0; o < nops; ++o)
        if (s.st[o][0] != 1 || ((uintptr_t)ptr[o] % 16) != 0) return false;
    return true;
}

// Rows of 16-byte vectors: every operand is contiguous (stride 1) or
// repeated (stride 0) along the innermost dim, the output contiguous; the
// innermost extent a multiple of the vector, and every stride-1 operand's
// vectors 16-byte aligned.  Covers broadcasts of rows and of columns.
bool inner16(const oxm::EwShape &s, int nops, const void *const ptr[3], int es) {
    if (es != 2 && es != 4) return false;
    const int L = s.ndim - 1, V = 16 / es;
    if (s.shape[L] % V != 0 || s.st[0][L] != 1) return false;
    for (int o = 0; o < nops; ++o) {
        if (s.st[o][L] == 0) continue;
        if (s.st[o][L] != 1 || ((uintptr_t)ptr[o] % 16) != 0) return false;
        for (int d = 0; d < L; ++d)
            if (s.st[o][d] % V != 0) return false;
    }
    return true;
}

// Vector path for an elementwise launch (oxm::EwVec).
int ew_vec(const oxm::EwShape &s, int nops, const void *const ptr[3], int es) {
    if (contig16(s, nops, ptr, es)) return oxm::kEwContig16;
    if (inner16(s, nops, ptr, es)) return oxm::kEwInner16;
    return oxm::kEwScalar;
}

const char *unary_name(int op) {
    static const char *n[] = {"neg", "exp", "ln", "abs", "sign"};
    return op >= 0 && op < 5 ? n[op] : "unary";
}
const char *binary_name(int op) {
    static const char *n[] = {"add", "sub", "mul", "div", "eq", "dgelu"};
    return op >= 0 && op < 6 ? n[op] : "binary";
}

// The checks every elementwise output needs: dtype, shape, contiguity,
// device, memory.
oxm_status check_out(const oxm_view *out, int dtype, int nd, const int64_t *shape, int device, const char *op) {
    if (out->dtype != dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in %s (out)", dtype_name(dtype),
                    dtype_name(out->dtype), op);
    if (out->ndim != nd || (nd && memcmp(out->shape, shape, 8 * nd)))
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in %s", shape_str(nd, shape).c_str(),
                    shape_str(out->ndim, out->shape).c_str(), op);
    if (!is_contiguous(out)) return fail(OXM_E_NOT_IMPLEMENTED, "%s is not implemented for a non-contiguous output", op);
    if (out->device != device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in %s", device_str(device).c_str(),
                    device_str(out->device).c_str(), op);
    return OXM_OK;
}

oxm_status reduce_impl(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes, const oxm_view *out,
                       void *stream, bool noalloc);

// Integer division with its typed refusal of a zero divisor (BinaryOps::div,
// crates/oxmera-ops/src/lib.rs:47-48): the kernel raises a device flag,
// which is read back after the stream has run it, so this call is
// synchronous on `s` whatever the stream (the error has to be known when the
// call returns).  The output holds 0 where a divisor was 0.
oxm_status int_div(const oxm::EwShape &sh, int dtype, void *po, const void *pa, const void *pb, hipStream_t s) {
    const char *op = "div";
    int *flag = nullptr;
    hipError_t e = hipMallocAsync((void **)&flag, sizeof(int), s);
    if (e != hipSuccess) return hip_fail(e, op);
    int host_flag = 0;
    e = oxm::launch_fill_zero((float *)flag, 1, s);  // a fill kernel, not a memset node (graph-safe)
    if (e == hipSuccess) e = oxm::launch_elementwise_int(dtype, 2, OXM_BIN_DIV, sh, po, pa, pb, flag, s);
    if (e == hipSuccess) e = hipMemcpyAsync(&host_flag, flag, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    hipError_t f = hipFreeAsync(flag, s);
    if (e == hipSuccess) e = f;
    if (e != hipSuccess) return hip_fail(e, op);
    if (host_flag)
        return fail(OXM_E_DIVISION_BY_ZERO, "integer division by zero in div (dtype %s)", dtype_name(dtype));
    return ok();
}

}  // namespace

extern "C" {

const char *oxm_version(void) { return "oxmera-mi355x 0.1.0 (gfx950)"; }

const char *oxm_last_error(void) { return g_last_error.c_str(); }

const char *oxm_backend_name(void) { return "hip-gfx950"; }

oxm_status oxm_device_count(int32_t *count) {
    if (!count) return fail(OXM_E_INVALID_ARGUMENT, "device_count: NULL out pointer");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        *count = 0;
        return fail(OXM_E_BACKEND_UNAVAILABLE, "no backend available for device Rocm { index: 0 }: no HIP device");
    }
    *count = n;
    return ok();
}

oxm_status oxm_view_byte_range(const oxm_view *v, int64_t *lo_bytes, int64_t *hi_bytes) {
    const char *op = "view_byte_range";
    oxm_status st;
    if ((st = check_view(v, "view", op)) != OXM_OK) return st;
    if (!lo_bytes || !hi_bytes) return fail(OXM_E_INVALID_ARGUMENT, "%s: NULL output pointer", op);
    *lo_bytes = *hi_bytes = 0;
    if (numel(v) == 0) return ok();
    int64_t lo = 0, hi = 0;
    if (!byte_range(v, &lo, &hi))
        return fail(OXM_E_INDEX_OUT_OF_BOUNDS, "%s: the byte range of a view of shape %s overflows int64", op,
                    shape_str(v->ndim, v->shape).c_str());
    *lo_bytes = lo;
    *hi_bytes = hi;
    return ok();
}

oxm_status oxm_broadcast_shapes(int32_t na, const int64_t *a, int32_t nb, const int64_t *b, int32_t *nout,
                                int64_t *out) {
    if (na < 0 || nb < 0 || na > OXM_MAX_DIMS || nb > OXM_MAX_DIMS || (na && !a) || (nb && !b) || !nout || !out)
        return fail(OXM_E_INVALID_ARGUMENT, "broadcast_shapes: malformed arguments");
    int n = na > nb ? na : nb;
    int64_t tmp[OXM_MAX_DIMS];
    for (int i = 0; i < n; ++i) {
        int ia = na - n + i, ib = nb - n + i;
        int64_t da = ia >= 0 ? a[ia] : 1, db = ib >= 0 ? b[ib] : 1;
        if (da == db || db == 1)
            tmp[i] = da;
        else if (da == 1)
            tmp[i] = db;
        else
            return fail(OXM_E_BROADCAST_INCOMPATIBLE, "cannot broadcast %s with %s", shape_str(na, a).c_str(),
                        shape_str(nb, b).c_str());
    }
    for (int i = 0; i < n; ++i) out[i] = tmp[i];
    *nout = n;
    return ok();
}

oxm_status oxm_gemm_infer(const oxm_view *a, const oxm_view *b, int32_t *out_ndim, int64_t *out_shape) {
    const char *op = "matmul";
    oxm_status st;
    if ((st = check_view(a, "lhs", op)) != OXM_OK) return st;
    if ((st = check_view(b, "rhs", op)) != OXM_OK) return st;
    if (!out_ndim || !out_shape) return fail(OXM_E_INVALID_ARGUMENT, "matmul: NULL output shape pointer");
    if (a->ndim < 2 || b->ndim < 2)
        return fail(OXM_E_RANK_MISMATCH, "rank mismatch in matmul: operands of rank %d and %d, both must be >= 2",
                    a->ndim, b->ndim);
    if (a->dtype != b->dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in matmul", dtype_name(a->dtype),
                    dtype_name(b->dtype));
    const int64_t k = a->shape[a->ndim - 1];
    if (b->shape[b->ndim - 2] != k) {
        int64_t exp[OXM_MAX_DIMS];
        for (int i = 0; i < b->ndim; ++i) exp[i] = b->shape[i];
        exp[b->ndim - 2] = k;
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in matmul",
                    shape_str(b->ndim, exp).c_str(), shape_str(b->ndim, b->shape).c_str());
    }
    int32_t nbd = 0;
    int64_t bshape[OXM_MAX_DIMS];
    st = oxm_broadcast_shapes(a->ndim - 2, a->shape, b->ndim - 2, b->shape, &nbd, bshape);
    if (st != OXM_OK) return st;
    for (int i = 0; i < nbd; ++i) out_shape[i] = bshape[i];
    out_shape[nbd] = a->shape[a->ndim - 2];
    out_shape[nbd + 1] = b->shape[b->ndim - 1];
    *out_ndim = nbd + 2;
    return ok();
}

oxm_status oxm_gemm(const oxm_view *a, const oxm_view *b, const oxm_view *c, const oxm_epilogue *ep, void *stream) {
    const char *op = "matmul";
    int32_t nd = 0;
    int64_t oshape[OXM_MAX_DIMS];
    oxm_status st = oxm_gemm_infer(a, b, &nd, oshape);
    if (st != OXM_OK) return st;
    if ((st = check_view(c, "out", op)) != OXM_OK) return st;
    if (!is_gemm_dtype(a->dtype))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by matmul", dtype_name(a->dtype));
    if (a->dtype == OXM_F32 ? c->dtype != OXM_F32 : !is_gemm_dtype(c->dtype))
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in matmul (output)",
                    a->dtype == OXM_F32 ? "F32" : "F32/BF16/F16", dtype_name(c->dtype));
    if (c->ndim != nd || memcmp(c->shape, oshape, sizeof(int64_t) * nd) != 0)
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in matmul (output)",
                    shape_str(nd, oshape).c_str(), shape_str(c->ndim, c->shape).c_str());
    if (!is_contiguous(c)) return fail(OXM_E_NOT_IMPLEMENTED, "matmul is not implemented for a non-contiguous output");
    if (a->device < 0 || b->device != a->device || c->device != a->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in matmul", device_str(a->device).c_str(),
                    device_str(a->device != b->device ? b->device : c->device).c_str());
    const int nbd = nd - 2;
    if (nbd > oxm::kMaxBatchDims)
        return fail(OXM_E_NOT_IMPLEMENTED, "matmul is not implemented for %d batch dims (max %d)", nbd,
                    oxm::kMaxBatchDims);
    oxm_epilogue none = {nullptr, OXM_F32, OXM_ACT_NONE, nullptr, nullptr};
    if (!ep) ep = &none;
    if (ep->act < OXM_ACT_NONE || ep->act > OXM_ACT_MUL_AUX)
        return fail(OXM_E_INVALID_ARGUMENT, "matmul: unknown epilogue activation %d", ep->act);
    if (ep->act == OXM_ACT_DGELU && !ep->aux)
        return fail(OXM_E_INVALID_ARGUMENT, "matmul: the DGELU epilogue needs the pre-activation (aux)");
    if (ep->act == OXM_ACT_MUL_AUX && !ep->aux)
        return fail(OXM_E_INVALID_ARGUMENT, "matmul: the MUL_AUX epilogue needs its factor (aux)");
    const bool aux_in = ep->act == OXM_ACT_DGELU || ep->act == OXM_ACT_MUL_AUX;
    if (ep->bias && !is_gemm_dtype(ep->bias_dtype))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by matmul (bias)", dtype_name(ep->bias_dtype));

    const int64_t M = oshape[nd - 2], N = oshape[nd - 1], K = a->shape[a->ndim - 1];
    int64_t batch = 1;
    for (int i = 0; i < nbd; ++i) batch *= oshape[i];
    if (N == 0) return ok();
    if (batch == 0 || M == 0) {
        if (!ep->colsum) return ok();
        // sums over no rows: the column sums are zero
        DeviceGuard guard(a->device);
        if ((st = check_device_range(ep->colsum, 0, N * 4, a->device, "colsum", op)) != OXM_OK) return st;
        hipStream_t s = (hipStream_t)stream;
        hipError_t e = oxm::launch_fill_zero(ep->colsum, N, s);
        if (e != hipSuccess) return hip_fail(e, op);
        return finish(s, op);
    }

    DeviceGuard guard(a->device);
    if ((st = check_view_memory(a, "lhs", op)) != OXM_OK) return st;
    if ((st = check_view_memory(b, "rhs", op)) != OXM_OK) return st;
    if ((st = check_view_memory(c, "out", op)) != OXM_OK) return st;
    const int oes = dtype_size(c->dtype);
    if (ep->bias && (st = check_device_range(ep->bias, 0, N * dtype_size(ep->bias_dtype), a->device, "bias", op)) !=
                        OXM_OK)
        return st;
    if (ep->aux && (st = check_device_range(ep->aux, 0, batch * M * N * oes, a->device, "aux", op)) != OXM_OK)
        return st;
    if (ep->colsum && (st = check_device_range(ep->colsum, 0, N * 4, a->device, "colsum", op)) != OXM_OK)
        return st;
    {
        const Span sa = span_of(a), sb = span_of(b), sc = span_of(c);
        const Span sbias = ep->bias ? span_bytes(ep->bias, N * dtype_size(ep->bias_dtype)) : Span{0, 0};
        const Span saux = ep->aux ? span_bytes(ep->aux, batch * M * N * oes) : Span{0, 0};
        const Span scs = ep->colsum ? span_bytes(ep->colsum, N * 4) : Span{0, 0};
        const struct {
            Span out;
            const char *name;
        } outs[3] = {{sc, "output"}, {aux_in ? Span{0, 0} : saux, "aux output"}, {scs, "colsum"}};
        const struct {
            Span in;
            const char *name;
        } ins[4] = {{sa, "lhs"}, {sb, "rhs"}, {sbias, "bias"}, {aux_in ? saux : Span{0, 0}, "aux"}};
        for (const auto &o : outs) {
            for (const auto &i : ins)
                if ((st = refuse_overlap(o.out, o.name, i.in, i.name, op)) != OXM_OK) return st;
        }
        if ((st = refuse_overlap(sc, "output", saux, "aux output", op)) != OXM_OK) return st;
        if ((st = refuse_overlap(sc, "output", scs, "colsum", op)) != OXM_OK) return st;
        if ((st = refuse_overlap(saux, "aux", scs, "colsum", op)) != OXM_OK) return st;
    }

    const int es = dtype_size(a->dtype);
    oxm::GemmArgs g;
    memset(&g, 0, sizeof g);
    g.a = (const char *)a->data + a->offset * es;
    g.b = (const char *)b->data + b->offset * es;
    g.c = (char *)c->data + c->offset * oes;
    g.bias = ep->bias;
    g.aux = ep->aux;
    g.M = M;
    g.N = N;
    g.K = K;
    g.sam = a->strides[a->ndim - 2];
    g.sak = a->strides[a->ndim - 1];
    g.sbk = b->strides[b->ndim - 2];
    g.sbn = b->strides[b->ndim - 1];
    g.nbd = nbd;
    g.batch = batch;
    for (int d = 0; d < nbd; ++d) {
        int da = a->ndim - 2 - nbd + d, db = b->ndim - 2 - nbd + d;
        g.bext[d] = oshape[d];
        g.bsa[d] = (da >= 0 && a->shape[da] != 1) ? a->strides[da] : 0;
        g.bsb[d] = (db >= 0 && b->shape[db] != 1) ? b->strides[db] : 0;
    }
    g.act = ep->act;
    g.out_dtype = c->dtype;
    g.bias_dtype = ep->bias_dtype;

    // Row strip: when the last M % 256 rows alone would cost one more round
    // of 256x256 tiles (4097 x 4095: 16 tile-rows fill the CUs once, the 17th
    // holds one row), the whole 256-row tiles run as usual and those rows run
    // on the strip kernel, which reads B once with plain FMAs (one batch, a
    // plain store epilogue).
    int64_t strip = 0;
    if (batch == 1 && ep->act == OXM_ACT_NONE && !ep->bias && !ep->colsum && M > 256) {
        const int64_t rem = M % 256, tn = (N + 255) / 256;
        const int64_t full = ((M + 255) / 256) * tn, bulk = (M / 256) * tn;
        if (rem <= oxm::kStripMaxRows && (full + 255) / 256 > (bulk + 255) / 256 && prefer_256_tiles(M - rem, N, 1))
            strip = rem;
    }
    const int64_t Mt = M - strip;  // rows on MFMA tiles
    g.M = Mt;

    int cfg;
    int cfg_plain = 0;  // f32: the configuration without 256x192 tiles
    bool forced = false;
    const bool big = prefer_256_tiles(Mt, N, batch);
    if (a->dtype == OXM_F32) {
        // f32 problems of at most 64 128x128 tiles (a quarter of the CUs)
        // take 64x64 tiles: 256^3 runs on 16 CUs instead of 4
        const int64_t n128 = ((Mt + 127) / 128) * ((N + 127) / 128) * batch;
        cfg = big ? oxm::kCfgF32_256 : (n128 <= 64 ? oxm::kCfgF32_64 : oxm::kCfgF32_128);
        cfg_plain = cfg;
        if (cfg != oxm::kCfgF32_64 && prefer_256x192_tiles(Mt, N, batch)) cfg = oxm::kCfgF32_256x192;
        cfg = env_int("OXM_GEMM_CFG_F32", cfg);
        if (cfg != oxm::kCfgF32_256 && cfg != oxm::kCfgF32_64 && cfg != oxm::kCfgF32_256x192)
            cfg = oxm::kCfgF32_128;
    } else {
        cfg = big ? oxm::kCfgH_256 : oxm::kCfgH_128;
        forced = env_int("OXM_GEMM_CFG", -1) >= 0;
        cfg = env_int("OXM_GEMM_CFG", cfg);
        if ((cfg < oxm::kCfgH_256 || cfg > oxm::kCfgH_256_NS) && cfg != oxm::kCfgH_256_1W &&
            cfg != oxm::kCfgH_256_1W16)
            cfg = oxm::kCfgH_128;
    }
    oxm::TileShape ts = oxm::tile_shape(cfg);
    if (strip && ts.bm != 256) {  // a forced 128x128 configuration: no strip
        strip = 0;
        g.M = M;
    }
    int ld_a = classify((const char *)g.a, g.sam, g.sak, g.M, K, g.bsa, nbd, es, ts.bm);
    int ld_b = classify((const char *)g.b, g.sbn, g.sbk, N, K, g.bsb, nbd, es, ts.bn);
    if (cfg == oxm::kCfgF32_256x192 && !oxm::use_f32_dma(g, ld_a, ld_b)) {
        // 256x192 tiles run on the direct-to-LDS kernel only: the choice without them
        cfg = cfg_plain;
        ts = oxm::tile_shape(cfg);
        ld_a = classify((const char *)g.a, g.sam, g.sak, g.M, K, g.bsa, nbd, es, ts.bm);
        ld_b = classify((const char *)g.b, g.sbn, g.sbk, N, K, g.bsb, nbd, es, ts.bn);
    }
    // The 16x16x32 one-wave kernel in the band where it measured faster than
    // (or level with) the 2x4-wave kernel: interleaved medians, K-major bf16
    // operands, both with the global-load DMA and its short hazard pad --
    // K of 4096 to 12288 and at least 512 256x256 tiles (8192^3: 0.742 vs
    // 0.790 ms; 576 to 4096 tiles at K 4096-12288: 1.1-5.5 % faster, one
    // 2048-tile K 4096 shape level); at K 16384, on 256 tiles and under a
    // GELU / GELU' or column-sum epilogue it measured level to 20 % slower.
    if (!forced && cfg == oxm::kCfgH_256 && ld_a == oxm::kLdK && ld_b == oxm::kLdK && ep->act == OXM_ACT_NONE &&
        !ep->colsum && K >= 4096 && K <= 12288) {
        const int64_t n256 = ((g.M + 255) / 256) * ((N + 255) / 256) * batch;
        if (n256 >= 512) cfg = oxm::kCfgH_256_1W16;
    }
    int64_t ntiles = ((g.M + ts.bm - 1) / ts.bm) * ((N + ts.bn - 1) / ts.bn) * batch;
    if (ntiles > 0x7fffffffLL) return fail(OXM_E_NOT_IMPLEMENTED, "matmul is not implemented for %lld tiles", (long long)ntiles);
    hipStream_t s = (hipStream_t)stream;
    if (ep->colsum) {
        g.colsum = ep->colsum;
        hipError_t ez = oxm::launch_fill_zero(ep->colsum, N, s);
        if (ez != hipSuccess) return hip_fail(ez, op);
    }
    hipError_t e = oxm::launch_gemm(g, a->dtype, ld_a, ld_b, cfg, s);
    if (e != hipSuccess) return hip_fail(e, op);
    if (strip) {
        oxm::GemmArgs gs = g;
        gs.M = strip;
        gs.a = (const char *)g.a + g.M * g.sam * es;
        gs.c = (char *)g.c + g.M * N * oes;
        e = oxm::launch_gemm_strip(gs, a->dtype, s);
        if (e != hipSuccess) return hip_fail(e, op);
    }
    return finish(s, op);
}

oxm_status oxm_sum_rows(const oxm_view *x, const oxm_view *out, void *stream) {
    const char *op = "sum";
    oxm_status st;
    if ((st = check_view(x, "input", op)) != OXM_OK) return st;
    if ((st = check_view(out, "out", op)) != OXM_OK) return st;
    if (x->ndim != 2) return fail(OXM_E_RANK_MISMATCH, "sum: input of rank %d, expected 2", x->ndim);
    if (!is_gemm_dtype(x->dtype)) return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by sum", dtype_name(x->dtype));
    if (out->dtype != OXM_F32) return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected F32, got %s in sum", dtype_name(out->dtype));
    if (out->ndim != 1 || out->shape[0] != x->shape[1])
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected [%lld], got %s in sum", (long long)x->shape[1],
                    shape_str(out->ndim, out->shape).c_str());
    if (!is_contiguous(x) || !is_contiguous(out))
        return fail(OXM_E_NOT_IMPLEMENTED, "sum is not implemented for non-contiguous views");
    if (x->device < 0 || out->device != x->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in sum", device_str(x->device).c_str(),
                    device_str(out->device).c_str());
    if (out->shape[0] == 0) return ok();
    DeviceGuard guard(x->device);
    if ((st = check_view_memory(x, "input", op)) != OXM_OK) return st;
    if ((st = check_view_memory(out, "out", op)) != OXM_OK) return st;
    if ((st = refuse_overlap(span_of(out), "output", span_of(x), "input", op)) != OXM_OK) return st;
    int es = dtype_size(x->dtype);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = oxm::launch_sum_rows((const char *)x->data + x->offset * es, x->dtype, x->shape[0], x->shape[1],
                                        (float *)out->data + out->offset, s);
    if (e != hipSuccess) return hip_fail(e, op);
    return finish(s, op);
}

oxm_status oxm_mse_loss_grad(const oxm_view *y, const oxm_view *t, const oxm_view *loss, const oxm_view *dy,
                             const oxm_view *dy_colsum, void *stream) {
    const char *op = "mse_loss";
    oxm_status st;
    if ((st = check_view(y, "y", op)) != OXM_OK) return st;
    if ((st = check_view(t, "target", op)) != OXM_OK) return st;
    if ((st = check_view(loss, "loss", op)) != OXM_OK) return st;
    if ((st = check_view(dy, "dy", op)) != OXM_OK) return st;
    if (dy_colsum && (st = check_view(dy_colsum, "dy_colsum", op)) != OXM_OK) return st;
    if (!is_gemm_dtype(y->dtype)) return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by mse_loss", dtype_name(y->dtype));
    if (t->dtype != y->dtype || dy->dtype != y->dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in mse_loss", dtype_name(y->dtype),
                    dtype_name(t->dtype != y->dtype ? t->dtype : dy->dtype));
    if (loss->dtype != OXM_F32 || numel(loss) != 1)
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: mse_loss needs a one-element F32 loss");
    if (t->ndim != y->ndim || dy->ndim != y->ndim || memcmp(t->shape, y->shape, 8 * y->ndim) ||
        memcmp(dy->shape, y->shape, 8 * y->ndim))
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in mse_loss", shape_str(y->ndim, y->shape).c_str(),
                    shape_str(t->ndim, t->shape).c_str());
    if (!is_contiguous(y) || !is_contiguous(t) || !is_contiguous(dy))
        return fail(OXM_E_NOT_IMPLEMENTED, "mse_loss is not implemented for non-contiguous views");
    if (y->device < 0 || t->device != y->device || dy->device != y->device || loss->device != y->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch in mse_loss");
    const int64_t n = numel(y);
    if (n == 0) return fail(OXM_E_SHAPE_MISMATCH, "mse_loss of an empty tensor has no mean");
    const int64_t C = y->ndim > 0 ? y->shape[y->ndim - 1] : 1, R = n / C;
    if (dy_colsum) {
        if (dy_colsum->dtype != OXM_F32)
            return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected F32, got %s for dy_colsum in mse_loss",
                        dtype_name(dy_colsum->dtype));
        if (dy_colsum->ndim != 1 || dy_colsum->shape[0] != C || !is_contiguous(dy_colsum))
            return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected [%lld], got %s for dy_colsum in mse_loss",
                        (long long)C, shape_str(dy_colsum->ndim, dy_colsum->shape).c_str());
        if (dy_colsum->device != y->device) return fail(OXM_E_DEVICE_MISMATCH, "device mismatch in mse_loss");
    }
    DeviceGuard guard(y->device);
    if ((st = check_view_memory(y, "y", op)) != OXM_OK) return st;
    if ((st = check_view_memory(t, "target", op)) != OXM_OK) return st;
    if ((st = check_view_memory(dy, "dy", op)) != OXM_OK) return st;
    if ((st = check_view_memory(loss, "loss", op)) != OXM_OK) return st;
    if (dy_colsum && (st = check_view_memory(dy_colsum, "dy_colsum", op)) != OXM_OK) return st;
    {
        const Span outs[3] = {span_of(dy), span_of(loss), dy_colsum ? span_of(dy_colsum) : Span{0, 0}};
        const char *onames[3] = {"dy", "loss", "dy_colsum"};
        const Span ins[2] = {span_of(y), span_of(t)};
        const char *inames[2] = {"y", "target"};
        for (int o = 0; o < 3; ++o) {
            for (int i = 0; i < 2; ++i)
                if ((st = refuse_overlap(outs[o], onames[o], ins[i], inames[i], op)) != OXM_OK) return st;
            for (int o2 = o + 1; o2 < 3; ++o2)
                if ((st = refuse_overlap(outs[o], onames[o], outs[o2], onames[o2], op)) != OXM_OK) return st;
        }
    }
    int es = dtype_size(y->dtype);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = oxm::launch_mse((const char *)y->data + y->offset * es, (const char *)t->data + t->offset * es,
                                   (char *)dy->data + dy->offset * es, y->dtype, R, C,
                                   (float *)loss->data + loss->offset,
                                   dy_colsum ? (float *)dy_colsum->data + dy_colsum->offset : nullptr, s);
    if (e != hipSuccess) return hip_fail(e, op);
    return finish(s, op);
}

oxm_status oxm_alloc(int32_t device, size_t bytes, void **out) {
    if (!out) return fail(OXM_E_INVALID_ARGUMENT, "alloc: NULL out pointer");
    *out = nullptr;
    if (device < 0) return fail(OXM_E_DEVICE_MISMATCH, "alloc: device %d is not a HIP device", device);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device >= n) {
        (void)hipGetLastError();
        return fail(OXM_E_BACKEND_UNAVAILABLE, "no backend available for device %s", device_str(device).c_str());
    }
    DeviceGuard guard(device);
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *out = nullptr;
        return hip_fail(e, "alloc");
    }
    {
        std::lock_guard<std::mutex> lock(g_alloc_mu);
        g_allocs[(uintptr_t)*out] = AllocInfo{bytes ? bytes : 1, device};
    }
    return ok();
}

oxm_status oxm_free(int32_t device, void *ptr) {
    if (!ptr) return ok();
    {
        std::lock_guard<std::mutex> lock(g_alloc_mu);
        g_allocs.erase((uintptr_t)ptr);
    }
    DeviceGuard guard(device < 0 ? 0 : device);
    hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return hip_fail(e, "free");
    return ok();
}

oxm_status oxm_copy(void *dst, int32_t dst_device, const void *src, int32_t src_device, size_t bytes, void *stream) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(OXM_E_INVALID_ARGUMENT, "copy: NULL pointer");
    if (dst_device < 0 && src_device < 0) {  // host to host needs no device
        memmove(dst, src, bytes);
        return ok();
    }
    hipMemcpyKind kind;
    if (dst_device < 0 && src_device < 0)
        kind = hipMemcpyHostToHost;
    else if (dst_device < 0)
        kind = hipMemcpyDeviceToHost;
    else if (src_device < 0)
        kind = hipMemcpyHostToDevice;
    else
        kind = hipMemcpyDeviceToDevice;
    if (dst_device >= 0) {
        oxm_status st = check_device_range(dst, 0, (int64_t)bytes, dst_device, "dst", "copy");
        if (st != OXM_OK) return st;
    }
    if (src_device >= 0) {
        oxm_status st = check_device_range(src, 0, (int64_t)bytes, src_device, "src", "copy");
        if (st != OXM_OK) return st;
    }
    if (dst_device >= 0 && src_device >= 0 &&
        overlaps(span_bytes(dst, (int64_t)bytes), span_bytes(src, (int64_t)bytes)))
        return fail(OXM_E_INVALID_ARGUMENT, "copy: the destination overlaps the source");
    DeviceGuard guard(dst_device >= 0 ? dst_device : (src_device >= 0 ? src_device : 0));
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (!s) {
        e = hipMemcpy(dst, src, bytes, kind);
    } else {
        // ordered after the work queued on the stream; a copy to or from host
        // memory also completes before the call returns (the host buffer may
        // be read or released right after)
        e = hipMemcpyAsync(dst, src, bytes, kind, s);
        if (e == hipSuccess && kind != hipMemcpyDeviceToDevice) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) return hip_fail(e, "copy");
    return ok();
}

oxm_status oxm_unary(int32_t op, const oxm_view *x, const oxm_view *out, void *stream) {
    if (op < OXM_UN_NEG || op > OXM_UN_SIGN) return fail(OXM_E_INVALID_ARGUMENT, "unary: unknown op %d", op);
    const char *name = unary_name(op);
    oxm_status st;
    if ((st = check_view(x, "input", name)) != OXM_OK) return st;
    if ((st = check_view(out, "out", name)) != OXM_OK) return st;
    if (!is_float_dtype(x->dtype) && !(is_int_dtype(x->dtype) && int_unary_ok(x->dtype, op)))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(x->dtype), name);
    if (x->device < 0) return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s is not a HIP device in %s",
                                   device_str(x->device).c_str(), name);
    if ((st = check_out(out, x->dtype, x->ndim, x->shape, x->device, name)) != OXM_OK) return st;
    if (numel(x) == 0) return ok();
    DeviceGuard guard(x->device);
    if ((st = check_view_memory(x, "input", name)) != OXM_OK) return st;
    if ((st = check_view_memory(out, "out", name)) != OXM_OK) return st;
    const int es = dtype_size(x->dtype);
    if (!same_elements(out, (const char *)x->data + x->offset * es, x->strides) &&
        (st = refuse_overlap(span_of(out), "output", span_of(x), "input", name)) != OXM_OK)
        return st;
    std::vector<int64_t> ost(x->ndim > 0 ? x->ndim : 1);
    int64_t acc = 1;
    for (int d = x->ndim - 1; d >= 0; --d) {
        ost[d] = acc;
        acc *= x->shape[d];
    }
    const int64_t *sts[3] = {ost.data(), x->strides, nullptr};
    oxm::EwShape sh = collapse(x->ndim, x->shape, sts, 2);
    void *po = (char *)out->data + out->offset * es;
    const void *px = (const char *)x->data + x->offset * es;
    const void *ptrs[3] = {po, px, nullptr};
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = is_int_dtype(x->dtype)
                       ? oxm::launch_elementwise_int(x->dtype, 1, op, sh, po, px, nullptr, nullptr, s)
                       : oxm::launch_elementwise(x->dtype, 1, op, sh, po, px, nullptr, ew_vec(sh, 2, ptrs, es), s);
    if (e != hipSuccess) return hip_fail(e, name);
    return finish(s, name);
}

oxm_status oxm_binary(int32_t op, const oxm_view *a, const oxm_view *b, const oxm_view *out, void *stream) {
    if (op < OXM_BIN_ADD || op > OXM_BIN_DGELU) return fail(OXM_E_INVALID_ARGUMENT, "binary: unknown op %d", op);
    const char *name = binary_name(op);
    oxm_status st;
    if ((st = check_view(a, "lhs", name)) != OXM_OK) return st;
    if ((st = check_view(b, "rhs", name)) != OXM_OK) return st;
    if ((st = check_view(out, "out", name)) != OXM_OK) return st;
    if (a->dtype != b->dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in %s", dtype_name(a->dtype),
                    dtype_name(b->dtype), name);
    if (!is_float_dtype(a->dtype) && !(is_int_dtype(a->dtype) && int_binary_ok(a->dtype, op)))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(a->dtype), name);
    if (a->device != b->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in %s", device_str(a->device).c_str(),
                    device_str(b->device).c_str(), name);
    if (a->device < 0) return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s is not a HIP device in %s",
                                   device_str(a->device).c_str(), name);
    int32_t nd = 0;
    int64_t shape[OXM_MAX_DIMS];
    if ((st = oxm_broadcast_shapes(a->ndim, a->shape, b->ndim, b->shape, &nd, shape)) != OXM_OK) return st;
    if ((st = check_out(out, a->dtype, nd, shape, a->device, name)) != OXM_OK) return st;
    int64_t n = 1;
    for (int d = 0; d < nd; ++d) n *= shape[d];
    if (n == 0) return ok();
    DeviceGuard guard(a->device);
    if ((st = check_view_memory(a, "lhs", name)) != OXM_OK) return st;
    if ((st = check_view_memory(b, "rhs", name)) != OXM_OK) return st;
    if ((st = check_view_memory(out, "out", name)) != OXM_OK) return st;
    // operand strides over the output dims: right-aligned, 0 where broadcast
    int64_t so[OXM_MAX_DIMS], sa[OXM_MAX_DIMS], sb[OXM_MAX_DIMS];
    int64_t acc = 1;
    for (int d = nd - 1; d >= 0; --d) {
        so[d] = acc;
        acc *= shape[d];
        const int da = d - (nd - a->ndim), db = d - (nd - b->ndim);
        sa[d] = (da >= 0 && a->shape[da] != 1) ? a->strides[da] : 0;
        sb[d] = (db >= 0 && b->shape[db] != 1) ? b->strides[db] : 0;
    }
    const int64_t *sts[3] = {so, sa, sb};
    const int es = dtype_size(a->dtype);
    if (!same_elements(out, (const char *)a->data + a->offset * es, sa) &&
        (st = refuse_overlap(span_of(out), "output", span_of(a), "lhs", name)) != OXM_OK)
        return st;
    if (!same_elements(out, (const char *)b->data + b->offset * es, sb) &&
        (st = refuse_overlap(span_of(out), "output", span_of(b), "rhs", name)) != OXM_OK)
        return st;
    oxm::EwShape sh = collapse(nd, shape, sts, 3);
    void *po = (char *)out->data + out->offset * es;
    const void *pa = (const char *)a->data + a->offset * es, *pb = (const char *)b->data + b->offset * es;
    const void *ptrs[3] = {po, pa, pb};
    hipStream_t s = (hipStream_t)stream;
    if (is_int_dtype(a->dtype)) {
        if (op != OXM_BIN_DIV) {
            hipError_t e = oxm::launch_elementwise_int(a->dtype, 2, op, sh, po, pa, pb, nullptr, s);
            if (e != hipSuccess) return hip_fail(e, name);
            return finish(s, name);
        }
        return int_div(sh, a->dtype, po, pa, pb, s);
    }
    hipError_t e = oxm::launch_elementwise(a->dtype, 2, op, sh, po, pa, pb, ew_vec(sh, 3, ptrs, es), s);
    if (e != hipSuccess) return hip_fail(e, name);
    return finish(s, name);
}

oxm_status oxm_reduce_infer(const oxm_view *x, const int32_t *axes, int32_t naxes, int32_t *out_ndim,
                            int64_t *out_shape) {
    const char *op = "reduce";
    oxm_status st;
    if ((st = check_view(x, "input", op)) != OXM_OK) return st;
    if (!out_ndim || !out_shape || (naxes > 0 && !axes))
        return fail(OXM_E_INVALID_ARGUMENT, "reduce: NULL axes or output pointer");
    if (naxes < 0) return fail(OXM_E_INVALID_ARGUMENT, "reduce: negative axis count");
    bool red[OXM_MAX_DIMS] = {};
    for (int i = 0; i < naxes; ++i) {
        if (axes[i] < 0 || axes[i] >= x->ndim)
            return fail(OXM_E_INDEX_OUT_OF_BOUNDS, "index out of bounds: axis %d of a rank-%d tensor in reduce", axes[i],
                        x->ndim);
        if (red[axes[i]]) return fail(OXM_E_INVALID_ARGUMENT, "reduce: axis %d listed twice", axes[i]);
        red[axes[i]] = true;
    }
    int n = 0;
    for (int d = 0; d < x->ndim; ++d)
        if (naxes > 0 && !red[d]) out_shape[n++] = x->shape[d];
    *out_ndim = n;
    return ok();
}

oxm_status oxm_reduce(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes, const oxm_view *out,
                      void *stream) {
    return reduce_impl(op, x, axes, naxes, out, stream, false);
}

oxm_status oxm_reduce_noalloc(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes, const oxm_view *out,
                              void *stream) {
    return reduce_impl(op, x, axes, naxes, out, stream, true);
}

}  // extern "C"

namespace {

// oxm_reduce, and with `noalloc` oxm_reduce_noalloc: the same validation and
// kernels; the split partials go to the library's static per-device scratch
// instead of a stream allocation.
oxm_status reduce_impl(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes, const oxm_view *out,
                       void *stream, bool noalloc) {
    if (op != OXM_RED_SUM && op != OXM_RED_MAX) return fail(OXM_E_INVALID_ARGUMENT, "reduce: unknown op %d", op);
    const char *name = op == OXM_RED_SUM ? "sum" : "max";
    oxm_status st;
    int32_t nd = 0;
    int64_t oshape[OXM_MAX_DIMS];
    if ((st = oxm_reduce_infer(x, axes, naxes, &nd, oshape)) != OXM_OK) return st;
    if ((st = check_view(out, "out", name)) != OXM_OK) return st;
    if (!is_float_dtype(x->dtype) && !is_int_dtype(x->dtype))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(x->dtype), name);
    if (x->device < 0) return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s is not a HIP device in %s",
                                   device_str(x->device).c_str(), name);
    if ((st = check_out(out, x->dtype, nd, oshape, x->device, name)) != OXM_OK) return st;
    bool red[OXM_MAX_DIMS] = {};
    for (int i = 0; i < naxes; ++i) red[axes[i]] = true;
    if (naxes == 0)
        for (int d = 0; d < x->ndim; ++d) red[d] = true;
    int64_t n_out = 1, n_red = 1;
    for (int d = 0; d < x->ndim; ++d) (red[d] ? n_red : n_out) *= x->shape[d];
    if (n_out == 0) return ok();
    if (n_red == 0 && op == OXM_RED_MAX)
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: max over an empty extent of %s has no identity",
                    shape_str(x->ndim, x->shape).c_str());
    DeviceGuard guard(x->device);
    if ((st = check_view_memory(x, "input", name)) != OXM_OK) return st;
    if ((st = check_view_memory(out, "out", name)) != OXM_OK) return st;
    if ((st = refuse_overlap(span_of(out), "output", span_of(x), "input", name)) != OXM_OK) return st;
    // kept and reduced dims, each collapsed where the input walks them as one
    int64_t ks[OXM_MAX_DIMS], kt[OXM_MAX_DIMS], rs[OXM_MAX_DIMS], rt[OXM_MAX_DIMS];
    int nk = 0, nr = 0;
    for (int d = 0; d < x->ndim; ++d) {
        if (red[d]) {
            rs[nr] = x->shape[d];
            rt[nr++] = x->strides[d];
        } else {
            ks[nk] = x->shape[d];
            kt[nk++] = x->strides[d];
        }
    }
    auto pack = [](int n, const int64_t *shape, const int64_t *stv, int64_t *oshape_, int64_t *ost) {
        const int64_t *sts[3] = {stv, nullptr, nullptr};
        oxm::EwShape c = collapse(n, shape, sts, 1);
        for (int d = 0; d < c.ndim; ++d) {
            oshape_[d] = c.shape[d];
            ost[d] = c.st[0][d];
        }
        return c.ndim;
    };
    oxm::RedGeom g{};
    g.n_out = n_out;
    g.n_red = n_red;
    g.nk = pack(nk, ks, kt, g.kshape, g.kst);
    g.nr = pack(nr, rs, rt, g.rshape, g.rst);
    if (n_red == 0) {  // sum over nothing: zeros
        g.nr = 1;
        g.rshape[0] = 0;
        g.rst[0] = 0;
    }
    const int es = dtype_size(x->dtype);
    hipStream_t s = (hipStream_t)stream;
    const char *px = (const char *)x->data + x->offset * es;
    char *po = (char *)out->data + out->offset * es;
    if (is_int_dtype(x->dtype)) {  // no workspace either way
        hipError_t e = oxm::launch_reduce_int(x->dtype, op, g, px, po, s);
        if (e != hipSuccess) return hip_fail(e, name);
        return finish(s, name);
    }
    void *ws = nullptr;
    if (noalloc) {
        const size_t need = oxm::reduce_workspace_bytes(x->dtype, g, px);
        if (need > oxm::kReduceScratchBytes)
            return fail(OXM_E_NOT_IMPLEMENTED,
                        "%s (no-allocation variant) is not implemented for a reduction whose split partials need "
                        "%zu bytes: the static scratch holds %zu",
                        name, need, oxm::kReduceScratchBytes);
        if (need > 0) {
            hipError_t e = oxm::reduce_scratch(&ws);
            if (e != hipSuccess) return hip_fail(e, name);
        }
    }
    hipError_t e = oxm::launch_reduce(x->dtype, op, g, px, po, s, ws);
    if (e != hipSuccess) return hip_fail(e, name);
    return finish(s, name);
}

}  // namespace

extern "C" {

oxm_status oxm_copy_view(const oxm_view *src, const oxm_view *dst, void *stream) {
    const char *op = "contiguous";
    oxm_status st;
    if ((st = check_view(src, "src", op)) != OXM_OK) return st;
    if ((st = check_view(dst, "dst", op)) != OXM_OK) return st;
    if (dst->dtype != src->dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s, got %s in %s", dtype_name(src->dtype),
                    dtype_name(dst->dtype), op);
    if (dst->ndim != src->ndim || (src->ndim && memcmp(dst->shape, src->shape, 8 * src->ndim)))
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in %s",
                    shape_str(src->ndim, src->shape).c_str(), shape_str(dst->ndim, dst->shape).c_str(), op);
    if (src->device < 0 || dst->device != src->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in %s", device_str(src->device).c_str(),
                    device_str(dst->device).c_str(), op);
    for (int d = 0; d < dst->ndim; ++d)
        if (dst->shape[d] > 1 && dst->strides[d] == 0)
            return fail(OXM_E_INVALID_ARGUMENT, "%s: the destination view repeats elements (stride 0)", op);
    if (numel(src) == 0) return ok();
    DeviceGuard guard(src->device);
    if ((st = check_view_memory(src, "src", op)) != OXM_OK) return st;
    if ((st = check_view_memory(dst, "dst", op)) != OXM_OK) return st;
    const int es = dtype_size(src->dtype);
    // dst == src element for element: nothing to move
    if (same_elements(dst, (const char *)src->data + src->offset * es, src->strides)) return ok();
    if ((st = refuse_overlap(span_of(dst), "destination", span_of(src), "source", op)) != OXM_OK) return st;
    const int64_t *sts[3] = {dst->strides, src->strides, nullptr};
    oxm::EwShape sh = collapse(src->ndim, src->shape, sts, 2);
    void *pd = (char *)dst->data + dst->offset * es;
    const void *ps = (const char *)src->data + src->offset * es;
    const void *ptrs[3] = {pd, ps, nullptr};
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = oxm::launch_copy(es, sh, pd, ps, contig16(sh, 2, ptrs, es), s);
    if (e != hipSuccess) return hip_fail(e, op);
    return finish(s, op);
}

oxm_status oxm_convert(const oxm_view *src, const oxm_view *dst, void *stream) {
    const char *op = "convert";
    oxm_status st;
    if ((st = check_view(src, "src", op)) != OXM_OK) return st;
    if ((st = check_view(dst, "dst", op)) != OXM_OK) return st;
    if (!is_float_dtype(src->dtype))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(src->dtype), op);
    if (!is_float_dtype(dst->dtype))
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(dst->dtype), op);
    if (dst->ndim != src->ndim || (src->ndim && memcmp(dst->shape, src->shape, 8 * src->ndim)))
        return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in %s",
                    shape_str(src->ndim, src->shape).c_str(), shape_str(dst->ndim, dst->shape).c_str(), op);
    if (src->device < 0 || dst->device != src->device)
        return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in %s", device_str(src->device).c_str(),
                    device_str(dst->device).c_str(), op);
    for (int d = 0; d < dst->ndim; ++d)
        if (dst->shape[d] > 1 && dst->strides[d] == 0)
            return fail(OXM_E_INVALID_ARGUMENT, "%s: the destination view repeats elements (stride 0)", op);
    if (numel(src) == 0) return ok();
    DeviceGuard guard(src->device);
    if ((st = check_view_memory(src, "src", op)) != OXM_OK) return st;
    if ((st = check_view_memory(dst, "dst", op)) != OXM_OK) return st;
    if ((st = refuse_overlap(span_of(dst), "destination", span_of(src), "source", op)) != OXM_OK) return st;
    const int64_t *sts[3] = {dst->strides, src->strides, nullptr};
    oxm::EwShape sh = collapse(src->ndim, src->shape, sts, 2);
    void *pd = (char *)dst->data + dst->offset * dtype_size(dst->dtype);
    const void *ps = (const char *)src->data + src->offset * dtype_size(src->dtype);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = oxm::launch_convert(src->dtype, dst->dtype, sh, pd, ps, s);
    if (e != hipSuccess) return hip_fail(e, op);
    return finish(s, op);
}

oxm_status oxm_sgd_step(const oxm_view *param, const oxm_view *grad, const oxm_view *velocity, float lr,
                        float momentum, float weight_decay, int32_t nesterov, void *stream) {
    const char *op = "sgd_step";
    oxm_status st;
    if ((st = check_view(param, "param", op)) != OXM_OK) return st;
    if ((st = check_view(grad, "grad", op)) != OXM_OK) return st;
    if (param->dtype != OXM_F32 && param->dtype != OXM_BF16 && param->dtype != OXM_F16)
        return fail(OXM_E_UNSUPPORTED_DTYPE, "dtype %s is not supported by %s", dtype_name(param->dtype), op);
    if (grad->dtype != OXM_F32 && grad->dtype != param->dtype)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected %s or F32, got %s in %s (grad)",
                    dtype_name(param->dtype), dtype_name(grad->dtype), op);
    if (!std::isfinite(lr) || !std::isfinite(momentum) || !std::isfinite(weight_decay))
        return fail(OXM_E_INVALID_ARGUMENT, "%s: lr, momentum and weight_decay must be finite", op);
    if (nesterov && momentum == 0.0f)
        return fail(OXM_E_INVALID_ARGUMENT, "%s: Nesterov momentum needs momentum != 0", op);
    if ((momentum != 0.0f) != (velocity != nullptr))
        return fail(OXM_E_INVALID_ARGUMENT, "%s: a velocity buffer is required exactly when momentum != 0", op);
    if (velocity && (st = check_view(velocity, "velocity", op)) != OXM_OK) return st;
    if (velocity && velocity->dtype != OXM_F32)
        return fail(OXM_E_DTYPE_MISMATCH, "dtype mismatch: expected F32, got %s in %s (velocity)",
                    dtype_name(velocity->dtype), op);
    const oxm_view *vs[3] = {param, grad, velocity};
    const char *names[3] = {"param", "grad", "velocity"};
    for (int i = 0; i < 3; ++i) {
        const oxm_view *v = vs[i];
        if (!v) continue;
        if (i > 0 && (v->ndim != param->ndim || (param->ndim && memcmp(v->shape, param->shape, 8 * param->ndim))))
            return fail(OXM_E_SHAPE_MISMATCH, "shape mismatch: expected %s, got %s in %s (%s)",
                        shape_str(param->ndim, param->shape).c_str(), shape_str(v->ndim, v->shape).c_str(), op,
                        names[i]);
        if (v->device < 0 || v->device != param->device)
            return fail(OXM_E_DEVICE_MISMATCH, "device mismatch: %s vs %s in %s (%s)",
                        device_str(param->device).c_str(), device_str(v->device).c_str(), op, names[i]);
        if (!is_contiguous(v))
            return fail(OXM_E_NOT_IMPLEMENTED, "%s is not implemented for a non-contiguous %s", op, names[i]);
    }
    const int64_t n = numel(param);
    if (n == 0) return ok();
    DeviceGuard guard(param->device);
    for (int i = 0; i < 3; ++i)
        if (vs[i] && (st = check_view_memory(vs[i], names[i], op)) != OXM_OK) return st;
    // param and velocity are updated in place; no two of the three may share memory
    for (int i = 0; i < 3; ++i)
        for (int j = i + 1; j < 3; ++j)
            if (vs[i] && vs[j] && (st = refuse_overlap(span_of(vs[i]), names[i], span_of(vs[j]), names[j], op)) != OXM_OK)
                return st;
    void *pp = (char *)param->data + param->offset * dtype_size(param->dtype);
    const void *pg = (const char *)grad->data + grad->offset * dtype_size(grad->dtype);
    float *pv = velocity ? (float *)velocity->data + velocity->offset : nullptr;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = oxm::launch_sgd(param->dtype, grad->dtype, n, pp, pg, pv, lr, momentum, weight_decay, nesterov != 0, s);
    if (e != hipSuccess) return hip_fail(e, op);
    return finish(s, op);
}

oxm_status oxm_synchronize(int32_t device) {
    if (device < 0) return ok();
    DeviceGuard guard(device);
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "synchronize");
    return ok();
}

}  // extern "C"
