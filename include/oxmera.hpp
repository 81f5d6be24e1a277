// oxmera.hpp -- C++17 host-side mirror of oxmera's core, tensor, ops and
// runtime interfaces over the C-ABI in oxm.h (header-only).
//
// This is the host layer a C++ caller uses, and the shape of what the Rust
// `oxmera-hip` crate implements: the same names, argument meaning and error
// behaviour as the reference --
//   DType / Shape / Strides / Layout / Device / Error   crates/oxmera-core/src/*.rs
//   Storage / Tensor (views never copy)                 crates/oxmera-tensor/src/*.rs
//   MatmulOps / ReduceOps / Backend                     crates/oxmera-ops/src/lib.rs:27-69,
//                                                       crates/oxmera-runtime/src/lib.rs:25-34
//   backend_for / register_backend                      crates/oxmera-runtime/src/lib.rs:36-53
// Fallible calls return Result<T> (a value or a typed Error), never throw.
#pragma once

#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <string>
#include <utility>
#include <vector>

#include "oxm.h"

namespace oxmera {

// ---- dtype (dtype.rs:9-34, + BF16 / F16) ------------------------------------

enum class DType : int32_t { F32 = 0, F64 = 1, I32 = 2, I64 = 3, U8 = 4, Bool = 5, BF16 = 6, F16 = 7 };

inline size_t size_in_bytes(DType d) {
    switch (d) {
    case DType::F32: case DType::I32: return 4;
    case DType::F64: case DType::I64: return 8;
    case DType::U8: case DType::Bool: return 1;
    case DType::BF16: case DType::F16: return 2;
    }
    return 0;
}
inline bool is_float(DType d) { return d == DType::F32 || d == DType::F64 || d == DType::BF16 || d == DType::F16; }

// ---- device (device.rs:10-31, + Rocm) ---------------------------------------

struct Device {
    enum class Kind { Cpu, Rocm } kind = Kind::Cpu;
    int index = 0;
    static Device cpu() { return {}; }
    static Device rocm(int i) { return {Kind::Rocm, i}; }
    const char *kind_name() const { return kind == Kind::Cpu ? "cpu" : "rocm"; }
    int abi_index() const { return kind == Kind::Cpu ? -1 : index; }
    bool operator==(const Device &o) const { return kind == o.kind && index == o.index; }
    bool operator<(const Device &o) const { return std::make_pair(kind, index) < std::make_pair(o.kind, o.index); }
};

// ---- shapes -------------------------------------------------------------------

using Shape = std::vector<int64_t>;
using Strides = std::vector<int64_t>;  // element strides, signed (layout.rs:6-10)

inline int64_t numel(const Shape &s) {
    return std::accumulate(s.begin(), s.end(), int64_t{1}, [](int64_t a, int64_t b) { return a * b; });
}

inline std::string shape_str(const std::vector<int64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// ---- errors (error.rs:14-105) -------------------------------------------------

struct Error {
    enum class Kind {
        ShapeMismatch = OXM_E_SHAPE_MISMATCH,
        BroadcastIncompatible = OXM_E_BROADCAST_INCOMPATIBLE,
        DTypeMismatch = OXM_E_DTYPE_MISMATCH,
        UnsupportedDType = OXM_E_UNSUPPORTED_DTYPE,
        DeviceMismatch = OXM_E_DEVICE_MISMATCH,
        IndexOutOfBounds = OXM_E_INDEX_OUT_OF_BOUNDS,
        RankMismatch = OXM_E_RANK_MISMATCH,
        BackendUnavailable = OXM_E_BACKEND_UNAVAILABLE,
        NotImplemented = OXM_E_NOT_IMPLEMENTED,
        Hip = OXM_E_HIP,
        InvalidArgument = OXM_E_INVALID_ARGUMENT,
    } kind;
    std::string message;
    Shape lhs, rhs;                       // BroadcastIncompatible operands
    std::vector<int64_t> index;           // IndexOutOfBounds
    Shape shape;                          // IndexOutOfBounds
    size_t index_rank = 0, shape_rank = 0;  // RankMismatch

    static Error from_status(oxm_status st) { return Error{Kind(st), oxm_last_error(), {}, {}, {}, {}, 0, 0}; }
    const std::string &what() const { return message; }
};

template <typename T>
class Result {
  public:
    Result(T v) : ok_(true), v_(std::move(v)) {}
    Result(Error e) : ok_(false), e_(std::move(e)) {}
    bool is_ok() const { return ok_; }
    bool is_err() const { return !ok_; }
    const T &value() const { return v_; }
    T &value() { return v_; }
    const Error &error() const { return e_; }

  private:
    bool ok_;
    T v_{};
    Error e_{Error::Kind::InvalidArgument, {}, {}, {}, {}, {}, 0, 0};
};

template <>
class Result<void> {
  public:
    Result() : ok_(true) {}
    Result(Error e) : ok_(false), e_(std::move(e)) {}
    bool is_ok() const { return ok_; }
    bool is_err() const { return !ok_; }
    const Error &error() const { return e_; }

  private:
    bool ok_;
    Error e_{Error::Kind::InvalidArgument, {}, {}, {}, {}, {}, 0, 0};
};

// broadcast_shapes (shape.rs:45-58), computed by the library's host layer.
inline Result<Shape> broadcast_shapes(const Shape &lhs, const Shape &rhs) {
    int32_t n = 0;
    int64_t out[OXM_MAX_DIMS];
    oxm_status st = oxm_broadcast_shapes((int32_t)lhs.size(), lhs.data(), (int32_t)rhs.size(), rhs.data(), &n, out);
    if (st != OXM_OK) {
        Error e = Error::from_status(st);
        e.lhs = lhs;
        e.rhs = rhs;
        return e;
    }
    return Shape(out, out + n);
}

inline Strides contiguous_strides(const Shape &shape) {
    Strides s(shape.size());
    int64_t acc = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        s[i] = acc;
        acc *= shape[i];
    }
    return s;
}

// ---- layout (layout.rs:24-62) ---------------------------------------------------

struct Layout {
    Shape shape;
    Strides strides;
    int64_t offset = 0;

    static Layout contiguous(const Shape &shape) { return {shape, contiguous_strides(shape), 0}; }

    Result<int64_t> offset_of(const std::vector<int64_t> &index) const {
        if (index.size() != shape.size()) {
            Error e{Error::Kind::RankMismatch,
                    "rank mismatch: index of rank " + std::to_string(index.size()) + " against shape of rank " +
                        std::to_string(shape.size()),
                    {}, {}, {}, {}, index.size(), shape.size()};
            return e;
        }
        int64_t off = offset;
        for (size_t d = 0; d < shape.size(); ++d) {
            if (index[d] < 0 || index[d] >= shape[d]) {
                Error e{Error::Kind::IndexOutOfBounds,
                        "index " + shape_str(index) + " out of bounds for shape " + shape_str(shape), {}, {}, index,
                        shape, 0, 0};
                return e;
            }
            off += index[d] * strides[d];
        }
        return off;
    }

    bool is_contiguous() const {
        if (numel(shape) == 0) return true;
        int64_t expect = 1;
        for (size_t i = shape.size(); i-- > 0;) {
            if (shape[i] != 1 && strides[i] != expect) return false;
            expect *= shape[i];
        }
        return true;
    }
};

// ---- storage and tensors (storage.rs:12-68, tensor.rs:15-100) ---------------------

class Storage {
  public:
    Storage(size_t bytes, DType dtype, Device device) : bytes_(bytes), dtype_(dtype), device_(device) {}
    static Result<std::shared_ptr<Storage>> allocate(size_t bytes, DType dtype, Device device) {
        auto s = std::make_shared<Storage>(bytes, dtype, device);
        if (device.kind == Device::Kind::Cpu) {
            s->host_.assign(bytes ? bytes : 1, 0);
        } else {
            oxm_status st = oxm_alloc(device.index, bytes, &s->dev_);
            if (st != OXM_OK) return Error::from_status(st);
        }
        return s;
    }
    ~Storage() {
        if (dev_) oxm_free(device_.index, dev_);
    }
    Storage(const Storage &) = delete;
    Storage &operator=(const Storage &) = delete;
    void *data() { return dev_ ? dev_ : (void *)host_.data(); }
    size_t bytes() const { return bytes_; }
    DType dtype() const { return dtype_; }
    Device device() const { return device_; }

  private:
    size_t bytes_;
    DType dtype_;
    Device device_;
    std::vector<uint8_t> host_;
    void *dev_ = nullptr;
};

class Tensor {
  public:
    Tensor() = default;
    Tensor(std::shared_ptr<Storage> s, Layout l) : storage_(std::move(s)), layout_(std::move(l)) {}

    // A contiguous F32 tensor holding `data` (tensor.rs:30-36) on `device`.
    static Result<Tensor> from_vec_f32(const std::vector<float> &data, const Shape &shape,
                                       Device device = Device::cpu()) {
        if ((int64_t)data.size() != numel(shape))
            return Error{Error::Kind::ShapeMismatch, "shape mismatch in from_vec_f32", {}, {}, {}, shape, 0, 0};
        auto st = Storage::allocate(data.size() * 4, DType::F32, device);
        if (st.is_err()) return st.error();
        Tensor t(st.value(), Layout::contiguous(shape));
        auto w = t.write_bytes(data.data(), data.size() * 4);
        if (w.is_err()) return w.error();
        return t;
    }
    static Result<Tensor> empty(const Shape &shape, DType dtype, Device device) {
        auto st = Storage::allocate((size_t)numel(shape) * size_in_bytes(dtype), dtype, device);
        if (st.is_err()) return st.error();
        return Tensor(st.value(), Layout::contiguous(shape));
    }

    const Shape &shape() const { return layout_.shape; }
    const Layout &layout() const { return layout_; }
    DType dtype() const { return storage_->dtype(); }
    Device device() const { return storage_->device(); }
    const std::shared_ptr<Storage> &storage() const { return storage_; }

    // Views (tensor.rs:63-84): never copy.
    Result<Tensor> permute(const std::vector<size_t> &perm) const {
        std::vector<bool> seen(perm.size(), false);
        bool ok = perm.size() == shape().size();
        for (size_t p : perm) ok = ok && p < perm.size() && !seen[p] && (seen[p] = true);
        if (!ok) return Error{Error::Kind::RankMismatch, "permute: not a permutation", {}, {}, {}, {}, perm.size(),
                              shape().size()};
        Layout l{{}, {}, layout_.offset};
        for (size_t p : perm) {
            l.shape.push_back(layout_.shape[p]);
            l.strides.push_back(layout_.strides[p]);
        }
        return Tensor(storage_, l);
    }
    Result<Tensor> narrow(size_t dim, int64_t start, int64_t len) const {
        if (dim >= shape().size())
            return Error{Error::Kind::RankMismatch, "narrow: missing dim", {}, {}, {}, {}, dim, shape().size()};
        if (start < 0 || len < 0 || start + len > shape()[dim])
            return Error{Error::Kind::IndexOutOfBounds, "narrow past the end", {}, {}, {start + len}, shape(), 0, 0};
        Layout l = layout_;
        l.shape[dim] = len;
        l.offset += start * l.strides[dim];
        return Tensor(storage_, l);
    }
    Result<Tensor> reshape(const Shape &shape) const {
        if (numel(shape) != numel(this->shape()))
            return Error{Error::Kind::ShapeMismatch, "shape mismatch: expected " + shape_str(this->shape()) +
                                                          ", got " + shape_str(shape) + " in reshape",
                         {}, {}, {}, shape, 0, 0};
        if (!layout_.is_contiguous())
            return Error{Error::Kind::NotImplemented, "reshape of a non-contiguous view (it never copies)", {}, {},
                         {}, {}, 0, 0};
        return Tensor(storage_, Layout{shape, contiguous_strides(shape), layout_.offset});
    }

    // The elements in logical order as float (F32 only; host copy).
    Result<std::vector<float>> to_vec_f32() const {
        if (dtype() != DType::F32)
            return Error{Error::Kind::UnsupportedDType, "to_vec_f32 of a non-F32 tensor", {}, {}, {}, {}, 0, 0};
        const int64_t n = numel(shape());
        std::vector<float> out((size_t)n);
        if (n == 0) return out;
        int64_t lo = layout_.offset, hi = layout_.offset;
        for (size_t d = 0; d < shape().size(); ++d) {
            int64_t span = (shape()[d] - 1) * layout_.strides[d];
            (span < 0 ? lo : hi) += span;
        }
        std::vector<float> buf((size_t)(hi - lo + 1));
        const char *src = (const char *)storage_->data() + lo * 4;
        oxm_status st = oxm_copy(buf.data(), -1, src, device().abi_index(), buf.size() * 4, nullptr);
        if (st != OXM_OK) return Error::from_status(st);
        std::vector<int64_t> idx(shape().size(), 0);
        for (int64_t i = 0; i < n; ++i) {
            int64_t off = layout_.offset - lo;
            for (size_t d = 0; d < idx.size(); ++d) off += idx[d] * layout_.strides[d];
            out[(size_t)i] = buf[(size_t)off];
            for (size_t d = idx.size(); d-- > 0;) {
                if (++idx[d] < shape()[d]) break;
                idx[d] = 0;
            }
        }
        return out;
    }
    Result<float> get_f32(const std::vector<int64_t> &index) const {
        auto off = layout_.offset_of(index);
        if (off.is_err()) return off.error();
        Tensor one(storage_, Layout{{}, {}, off.value()});
        auto v = one.to_vec_f32();
        if (v.is_err()) return v.error();
        return v.value()[0];
    }

    // The C-ABI view; the vectors it points into live in this tensor's layout.
    oxm_view abi_view() const {
        return oxm_view{storage_->data(), (int32_t)dtype(), (int32_t)shape().size(), layout_.shape.data(),
                        layout_.strides.data(), layout_.offset, device().abi_index()};
    }

  private:
    Result<void> write_bytes(const void *src, size_t n) {
        if (!n) return {};
        oxm_status st = oxm_copy(storage_->data(), device().abi_index(), src, -1, n, nullptr);
        if (st != OXM_OK) return Error::from_status(st);
        return {};
    }
    std::shared_ptr<Storage> storage_;
    Layout layout_;
};

// ---- op traits and the backend (ops/src/lib.rs:27-69, runtime/src/lib.rs:25-34) ------

struct MatmulOps {
    virtual ~MatmulOps() = default;
    virtual Result<Tensor> matmul(const Tensor &lhs, const Tensor &rhs) const = 0;
};
struct ReduceOps {
    virtual ~ReduceOps() = default;
    virtual Result<Tensor> sum(const Tensor &a, const std::vector<size_t> &axes) const = 0;
    virtual Result<Tensor> max(const Tensor &a, const std::vector<size_t> &axes) const = 0;
};
struct Backend : MatmulOps, ReduceOps {
    virtual Device device() const = 0;
    virtual const char *name() const = 0;
};

// The MI355X backend: matmul and row sums on gfx950 through the C-ABI.
class HipBackend final : public Backend {
  public:
    explicit HipBackend(int index) : index_(index) {}
    Device device() const override { return Device::rocm(index_); }
    const char *name() const override { return oxm_backend_name(); }

    Result<Tensor> matmul(const Tensor &lhs, const Tensor &rhs) const override {
        oxm_view a = lhs.abi_view(), b = rhs.abi_view();
        int32_t nd = 0;
        int64_t shape[OXM_MAX_DIMS];
        oxm_status st = oxm_gemm_infer(&a, &b, &nd, shape);
        if (st != OXM_OK) return Error::from_status(st);
        // "a fresh contiguous tensor on the operands' device" (ops/src/lib.rs:16-17)
        auto out = Tensor::empty(Shape(shape, shape + nd), DType::F32, lhs.device());
        if (out.is_err()) return out.error();
        oxm_view c = out.value().abi_view();
        st = oxm_gemm(&a, &b, &c, nullptr, nullptr);
        if (st != OXM_OK) return Error::from_status(st);
        return out;
    }
    Result<Tensor> sum(const Tensor &a, const std::vector<size_t> &axes) const override {
        if (a.shape().size() != 2 || axes != std::vector<size_t>{0})
            return Error{Error::Kind::NotImplemented, "sum is not implemented for this rank / axes (hip backend)",
                         {}, {}, {}, {}, 0, 0};
        auto out = Tensor::empty({a.shape()[1]}, DType::F32, a.device());
        if (out.is_err()) return out.error();
        oxm_view x = a.abi_view(), o = out.value().abi_view();
        oxm_status st = oxm_sum_rows(&x, &o, nullptr);
        if (st != OXM_OK) return Error::from_status(st);
        return out;
    }
    Result<Tensor> max(const Tensor &, const std::vector<size_t> &) const override {
        return Error{Error::Kind::NotImplemented, "max is not implemented for the hip backend", {}, {}, {}, {}, 0, 0};
    }

  private:
    int index_;
};

// ---- the registry (runtime/src/lib.rs:36-53) ---------------------------------------

inline std::map<Device, std::shared_ptr<Backend>> &registry_() {
    static std::map<Device, std::shared_ptr<Backend>> r;
    return r;
}
inline std::mutex &registry_mu_() {
    static std::mutex m;
    return m;
}

inline void register_backend(std::shared_ptr<Backend> b) {
    std::lock_guard<std::mutex> lock(registry_mu_());
    registry_()[b->device()] = std::move(b);
}

inline Result<std::shared_ptr<Backend>> backend_for(Device d) {
    std::lock_guard<std::mutex> lock(registry_mu_());
    auto it = registry_().find(d);
    if (it == registry_().end())
        return Error{Error::Kind::BackendUnavailable, std::string("no backend available for device ") + d.kind_name(),
                     {}, {}, {}, {}, 0, 0};
    return it->second;
}

// Register a HipBackend per visible device; returns how many.
inline int register_hip_backends() {
    int32_t n = 0;
    if (oxm_device_count(&n) != OXM_OK) return 0;
    for (int i = 0; i < n; ++i) register_backend(std::make_shared<HipBackend>(i));
    return n;
}

// TensorOps::matmul (runtime/src/lib.rs:68-69, 99-102): resolve and dispatch.
inline Result<Tensor> matmul(const Tensor &a, const Tensor &b) {
    auto be = backend_for(a.device());
    if (be.is_err()) return be.error();
    return be.value()->matmul(a, b);
}

}  // namespace oxmera
