// spec_tests.cpp -- the reference's spec ladder restated against the C++
// host mirror (include/oxmera.hpp) over the HIP backend's C-ABI.
//
//   A1 shape and strides     exercises/a1-shape-and-strides/tests/spec.rs
//   A2 broadcasting          exercises/a2-broadcasting/tests/spec.rs
//   A3 strided views         exercises/a3-strided-views/tests/spec.rs
//   A4 the reference matmul  exercises/a4-reference-matmul/tests/spec.rs   (--gpu)
//   A5 error taxonomy        exercises/a5-error-taxonomy/tests/spec.rs
//   runtime harness          crates/oxmera-runtime/tests/harness.rs
// Every expected value is the spec's hand-computed constant.  Without
// --gpu only host-side cases run (no device is touched).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>

#include "oxmera.hpp"

using namespace oxmera;

static int g_fail = 0, g_pass = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (cond) {                                                              \
            ++g_pass;                                                            \
        } else {                                                                 \
            ++g_fail;                                                            \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
        }                                                                        \
    } while (0)

static Tensor t(const std::vector<float> &d, const Shape &s, Device dev) { return Tensor::from_vec_f32(d, s, dev).value(); }

static bool tensor_eq(const Result<Tensor> &r, const std::vector<float> &want, const Shape &shape) {
    if (r.is_err()) return false;
    if (r.value().shape() != shape) return false;
    auto v = r.value().to_vec_f32();
    return v.is_ok() && v.value() == want;
}

// ---- A1 ---------------------------------------------------------------------
static void a1() {
    CHECK(size_in_bytes(DType::F32) == 4 && size_in_bytes(DType::F64) == 8 && size_in_bytes(DType::I32) == 4);
    CHECK(size_in_bytes(DType::I64) == 8 && size_in_bytes(DType::U8) == 1 && size_in_bytes(DType::Bool) == 1);
    CHECK(is_float(DType::F32) && is_float(DType::F64) && !is_float(DType::I32) && !is_float(DType::I64));
    CHECK(!is_float(DType::U8) && !is_float(DType::Bool));
    CHECK(numel({}) == 1 && numel({0}) == 0 && numel({2, 3}) == 6 && numel({2, 0, 3}) == 0 && numel({1, 1, 1}) == 1);
    CHECK(contiguous_strides({}).empty());
    CHECK((contiguous_strides({4}) == Strides{1}));
    CHECK((contiguous_strides({2, 3}) == Strides{3, 1}));
    CHECK((contiguous_strides({2, 1, 3}) == Strides{3, 3, 1}));
    CHECK((contiguous_strides({4, 2, 3}) == Strides{6, 3, 1}));
    Layout l = Layout::contiguous({2, 3});
    CHECK(l.offset_of({0, 0}).value() == 0 && l.offset_of({0, 2}).value() == 2);
    CHECK(l.offset_of({1, 0}).value() == 3 && l.offset_of({1, 2}).value() == 5);
    CHECK(Layout::contiguous({}).offset_of({}).value() == 0);
    CHECK(l.offset_of({0}).is_err() && l.offset_of({0}).error().kind == Error::Kind::RankMismatch);
    CHECK(l.offset_of({0, 0, 0}).error().kind == Error::Kind::RankMismatch);
    CHECK(l.offset_of({2, 0}).error().kind == Error::Kind::IndexOutOfBounds);
    CHECK(l.offset_of({0, 3}).error().kind == Error::Kind::IndexOutOfBounds);
    CHECK(Layout::contiguous({2, 3}).is_contiguous() && Layout::contiguous({}).is_contiguous());
    CHECK(Layout::contiguous({0, 3}).is_contiguous());
    CHECK(!(Layout{{2, 3}, {1, 2}, 0}.is_contiguous()));
    // bijection onto [0, numel) for contiguous layouts, last index unit stride
    for (Shape s : {Shape{2, 3}, Shape{3, 1, 2}, Shape{1, 2, 3}}) {
        Layout c = Layout::contiguous(s);
        std::vector<bool> seen((size_t)numel(s), false);
        std::vector<int64_t> idx(s.size(), 0);
        for (int64_t i = 0; i < numel(s); ++i) {
            int64_t o = c.offset_of(idx).value();
            CHECK(o >= 0 && o < numel(s) && !seen[(size_t)o]);
            seen[(size_t)o] = true;
            for (size_t d = idx.size(); d-- > 0;) {
                if (++idx[d] < s[d]) break;
                idx[d] = 0;
            }
        }
    }
}

// ---- A2 ---------------------------------------------------------------------
static void a2() {
    struct Case { Shape l, r, want; };
    for (auto &c : {Case{{2, 3}, {3}, {2, 3}}, Case{{3}, {2, 3}, {2, 3}}, Case{{2, 1}, {1, 3}, {2, 3}},
                    Case{{}, {2, 3}, {2, 3}}, Case{{2, 3}, {}, {2, 3}}, Case{{}, {}, {}}, Case{{4, 1, 5}, {3, 1}, {4, 3, 5}},
                    Case{{1}, {1}, {1}}, Case{{5}, {1}, {5}}, Case{{0}, {1}, {0}}, Case{{2, 0}, {1, 1}, {2, 0}}}) {
        auto r = broadcast_shapes(c.l, c.r);
        CHECK(r.is_ok() && r.value() == c.want);
    }
    for (auto &c : {std::make_pair(Shape{2}, Shape{3}), std::make_pair(Shape{2, 3}, Shape{2, 4}),
                    std::make_pair(Shape{4, 3}, Shape{2, 1, 2}), std::make_pair(Shape{0}, Shape{2})}) {
        auto r = broadcast_shapes(c.first, c.second);
        CHECK(r.is_err() && r.error().kind == Error::Kind::BroadcastIncompatible);
        CHECK(r.error().lhs == c.first && r.error().rhs == c.second);
    }
    std::mt19937 rng(7);
    for (int it = 0; it < 200; ++it) {
        Shape a(rng() % 4), b(rng() % 4);
        for (auto &x : a) x = rng() % 4;
        for (auto &x : b) x = rng() % 4;
        auto ab = broadcast_shapes(a, b), ba = broadcast_shapes(b, a);
        CHECK(ab.is_ok() == ba.is_ok());
        if (ab.is_ok()) CHECK(ab.value() == ba.value() && ab.value().size() == std::max(a.size(), b.size()));
        CHECK(broadcast_shapes(a, a).value() == a);
        CHECK(broadcast_shapes(a, {}).value() == a);
    }
}

// ---- A3 ---------------------------------------------------------------------
static void a3(Device dev) {
    Tensor x = t({1, 2, 3, 4, 5, 6}, {2, 3}, dev);
    auto tt = x.permute({1, 0});
    CHECK(tt.is_ok() && (tt.value().shape() == Shape{3, 2}));
    CHECK(tt.value().get_f32({0, 0}).value() == 1 && tt.value().get_f32({0, 1}).value() == 4);
    CHECK(tt.value().get_f32({1, 0}).value() == 2 && tt.value().get_f32({2, 1}).value() == 6);
    CHECK(tt.value().storage() == x.storage());
    auto n = x.narrow(1, 1, 2);
    CHECK(tensor_eq(n, {2, 3, 5, 6}, {2, 2}) && n.value().storage() == x.storage());
    auto r = x.reshape({3, 2});
    CHECK(tensor_eq(r, {1, 2, 3, 4, 5, 6}, {3, 2}) && r.value().storage() == x.storage());
    CHECK(!tt.value().layout().is_contiguous());
    CHECK(x.permute({0, 0}).is_err() && x.permute({0}).is_err());
    CHECK(x.narrow(1, 2, 2).is_err() && x.narrow(2, 0, 1).is_err());
    CHECK(x.reshape({4, 2}).error().kind == Error::Kind::ShapeMismatch);
    CHECK(Tensor::from_vec_f32({1, 1, 1, 1, 1}, {2, 3}).error().kind == Error::Kind::ShapeMismatch);
}

// ---- A5 and the runtime harness -------------------------------------------------
static void a5() {
    CHECK(std::string(Device::cpu().kind_name()) == "cpu" && std::string(Device::rocm(1).kind_name()) == "rocm");
    auto e = broadcast_shapes({2}, {3}).error();
    CHECK(e.message.find('2') != std::string::npos && e.message.find('3') != std::string::npos);
    auto ie = Layout::contiguous({2, 3}).offset_of({0, 3}).error();
    CHECK(ie.message.find("[0, 3]") != std::string::npos && (ie.index == std::vector<int64_t>{0, 3}));
    auto re = Layout::contiguous({2, 3}).offset_of({0}).error();
    CHECK(re.index_rank == 1 && re.shape_rank == 2);
    // an unregistered device is a typed error, never a crash (runtime/tests/harness.rs:9-17)
    auto b = backend_for(Device::rocm(7));
    CHECK(b.is_err() && b.error().kind == Error::Kind::BackendUnavailable);
    // matmul validation needs no device: host tensors are refused before any launch
    HipBackend hb(0);
    auto m = hb.matmul(t({1, 2, 3, 4}, {2, 2}, Device::cpu()), t({5, 6, 7, 8}, {2, 2}, Device::cpu()));
    CHECK(m.is_err() && m.error().kind == Error::Kind::DeviceMismatch);
    CHECK(m.error().message.find("matmul") != std::string::npos);
    auto bad = hb.matmul(t({1, 1, 1, 1, 1, 1}, {2, 3}, Device::cpu()), t({1, 1, 1, 1, 1, 1, 1, 1}, {4, 2}, Device::cpu()));
    CHECK(bad.is_err() && bad.error().kind == Error::Kind::ShapeMismatch);
}

// ---- A4 on the GPU -----------------------------------------------------------------
static void a4_gpu() {
    CHECK(register_hip_backends() >= 1);
    Device d = Device::rocm(0);
    auto be = backend_for(d).value();
    CHECK(std::string(be->name()) == "hip-gfx950");
    CHECK(tensor_eq(be->matmul(t({1, 2, 3, 4}, {2, 2}, d), t({5, 6, 7, 8}, {2, 2}, d)), {19, 22, 43, 50}, {2, 2}));
    CHECK(tensor_eq(be->matmul(t({1, 2, 3, 4, 5, 6}, {2, 3}, d), t({1, 10, 100}, {3, 1}, d)), {321, 654}, {2, 1}));
    CHECK(tensor_eq(be->matmul(t({1.5f, -2, 0.25f, 4}, {2, 2}, d), t({1, 0, 0, 1}, {2, 2}, d)), {1.5f, -2, 0.25f, 4},
                    {2, 2}));
    CHECK(tensor_eq(be->matmul(t({3, -1, 2, 7, 0.5f, -4}, {2, 3}, d), t({0, 0, 0, 0, 0, 0}, {3, 2}, d)), {0, 0, 0, 0},
                    {2, 2}));
    auto mm = be->matmul(t({1, 1, 1, 1, 1, 1}, {2, 3}, d), t({1, 1, 1, 1, 1, 1, 1, 1}, {4, 2}, d));
    CHECK(mm.is_err() && mm.error().kind == Error::Kind::ShapeMismatch);
    CHECK(be->matmul(t({1, 1, 1, 1, 1, 1}, {6}, d), t({1, 1, 1, 1, 1, 1}, {6}, d)).is_err());
    Tensor bt = t({5, 7, 6, 8}, {2, 2}, d).permute({1, 0}).value();  // B^T in memory, read as a view
    CHECK(tensor_eq(be->matmul(t({1, 2, 3, 4}, {2, 2}, d), bt), {19, 22, 43, 50}, {2, 2}));
    CHECK(tensor_eq(matmul(t({1, 2, 3, 4}, {2, 2}, d), t({5, 6, 7, 8}, {2, 2}, d)), {19, 22, 43, 50}, {2, 2}));
    // transpose law and column independence on U(-8, 8) entries (a4 spec.rs:101-130)
    std::mt19937 rng(3);
    std::uniform_real_distribution<float> u(-8, 8);
    for (int it = 0; it < 16; ++it) {
        std::vector<float> av(6), bv(6), cv(9);
        for (auto &v : av) v = u(rng);
        for (auto &v : bv) v = u(rng);
        for (auto &v : cv) v = u(rng);
        Tensor a = t(av, {2, 3}, d), b = t(bv, {3, 2}, d);
        auto x = be->matmul(a, b).value().permute({1, 0}).value().to_vec_f32().value();
        auto y = be->matmul(b.permute({1, 0}).value(), a.permute({1, 0}).value()).value().to_vec_f32().value();
        for (int i = 0; i < 4; ++i) CHECK(std::fabs(x[i] - y[i]) <= 1e-4f * (1 + std::max(std::fabs(x[i]), std::fabs(y[i]))));
        Tensor c = t(cv, {3, 3}, d);
        size_t j = it % 2;
        auto full = be->matmul(c, b).value().to_vec_f32().value();
        auto col = be->matmul(c, b.narrow(1, (int64_t)j, 1).value()).value().to_vec_f32().value();
        for (int i = 0; i < 3; ++i) {
            float f = full[i * 2 + j], g = col[i];
            CHECK(std::fabs(f - g) <= 1e-4f * (1 + std::max(std::fabs(f), std::fabs(g))));
        }
    }
    // bias gradient: ReduceOps::sum over axis 0 of a rank-2 tensor
    auto s = be->sum(t({1, 2, 3, 4, 5, 6}, {2, 3}, d), {0});
    CHECK(tensor_eq(s, {5, 7, 9}, {3}));
    CHECK(be->max(t({1}, {1}, d), {0}).error().kind == Error::Kind::NotImplemented);
    // A3 views on device storage
    a3(d);
}

int main(int argc, char **argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    a1();
    a2();
    a3(Device::cpu());
    a5();
    if (gpu) a4_gpu();
    std::printf("%s: %d passed, %d failed\n", gpu ? "host+gpu" : "host", g_pass, g_fail);
    return g_fail ? 1 : 0;
}
