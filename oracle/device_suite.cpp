// device_suite.cpp - TEST INFRASTRUCTURE ONLY (the checker, never the product).
//
// kael's device-behaviour checks, restated as a table of named cases over kael's public C++ API
// and run against whichever kael::device backend the library is linked with:
//   libkael_ref-*.so   the reference's host emulation of its device tasks (proves each case
//                      checks what it should, on the CPU)
//   libkael_oracle.so  the C oracle (kd_oracle.c)
//   libkael_hip.so     the MI355X backend (kael.cpp_amd/host/backend_hip.cpp over libkd.so)
// Each case follows one test of the reference's device suite (tests/test_cuda.cpp:133-623,
// cited per case): the same inputs and seeds, results on Device::CUDA compared with kael's CPU
// results (f64 within 1e-10, everything else within 1e-4 relative + 1e-4 absolute, NaN equal to
// NaN; tests/test_cuda.cpp:40-53), plus the behaviour checks (devices, errors, identity).
//
// C entry points (test use only): ref_suite_size, ref_suite_name(i), ref_suite_run(i) -> 0 pass,
// 1 fail, 2 skipped; the failure report or skip reason is in ref_suite_message().
#include <cmath>
#include <cstdint>
#include <functional>
#include <limits>
#include <memory>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

#include "kael/autograd/gradcheck.h"
#include "kael/kael.h"
#include "kael/nn/activation.h"
#include "kael/nn/embedding.h"
#include "kael/nn/layernorm.h"
#include "kael/nn/linear.h"
#include "kael/nn/loss.h"
#include "kael/nn/sequential.h"
#include "kael/nn/transformer.h"
#include "kael/optim/adam.h"
#include "kael/optim/clip.h"

namespace {

using kael::Device;
using kael::DType;
using kael::Tensor;

thread_local std::string g_suite_message;

struct Skip {
    std::string reason;
};

// Collects every failed expectation of one case (a case keeps going after a failure, so one
// run reports all of them).
class Expect {
public:
    void that(bool ok, const std::string& what) {
        if (!ok) fail(what);
    }

    void fail(const std::string& what) {
        if (failures_.size() < 40) failures_.push_back(what);
        ++count_;
    }

    // `on_device` must live on the device and match `on_cpu` in shape, dtype and values.
    void matches_cpu(const Tensor& on_device, const Tensor& on_cpu, const std::string& label) {
        if (on_device.device() != Device::CUDA) fail(label + ": result is not on the device");
        if (on_device.shape() != on_cpu.shape()) {
            fail(label + ": shape " + kael::to_string(on_device.shape()) + " vs cpu " + kael::to_string(on_cpu.shape()));
            return;
        }
        if (on_device.dtype() != on_cpu.dtype()) {
            fail(label + ": dtype differs from the cpu result");
            return;
        }
        const double tol = on_cpu.dtype() == DType::F64 ? 1e-10 : 1e-4;
        const std::string where = first_difference(on_device.cpu().contiguous(), on_cpu.contiguous(), tol, tol);
        if (!where.empty()) fail(label + ": " + where);
    }

    // Bitwise-equal values (kael::equal), shapes and dtypes.
    void equal(const Tensor& a, const Tensor& b, const std::string& label) {
        that(a.shape() == b.shape() && a.dtype() == b.dtype() && kael::equal(a, b), label + ": not equal");
    }

    template <typename E, typename F> void throws(F&& f, const std::string& label, const std::string& needle = "") {
        try {
            f();
        } catch (const E& error) {
            if (!needle.empty() && std::string(error.what()).find(needle) == std::string::npos)
                fail(label + ": message lacks '" + needle + "': " + error.what());
            return;
        } catch (const std::exception& other) {
            fail(label + ": threw the wrong error type: " + other.what());
            return;
        }
        fail(label + ": did not throw");
    }

    template <typename F> void no_throw(F&& f, const std::string& label) {
        try {
            f();
        } catch (const std::exception& error) {
            fail(label + ": threw " + error.what());
        }
    }

    bool passed() const { return count_ == 0; }

    std::string report() const {
        std::string out = std::to_string(count_) + " failed expectation(s)";
        for (const auto& f : failures_) out += "\n  " + f;
        return out;
    }

private:
    static bool close(double a, double e, double rtol, double atol) {
        if (std::isnan(a) || std::isnan(e)) return std::isnan(a) && std::isnan(e);
        if (std::isinf(a) || std::isinf(e)) return a == e;
        return std::abs(a - e) <= atol + rtol * std::abs(e);
    }

    static std::string first_difference(const Tensor& actual, const Tensor& expected, double rtol, double atol) {
        const int64_t n = actual.numel();
        for (int64_t i = 0; i < n; ++i) {
            double a = 0, e = 0;
            bool exact = false;
            switch (actual.dtype()) {
            case DType::F32:
                a = actual.data_ptr<float>()[i];
                e = expected.data_ptr<float>()[i];
                break;
            case DType::F64:
                a = actual.data_ptr<double>()[i];
                e = expected.data_ptr<double>()[i];
                break;
            case DType::I64: {
                const int64_t ai = actual.data_ptr<int64_t>()[i], ei = expected.data_ptr<int64_t>()[i];
                if (ai != ei) return "element " + std::to_string(i) + ": " + std::to_string(ai) + " vs " + std::to_string(ei);
                exact = true;
                break;
            }
            case DType::Bool: {
                const uint8_t ab = actual.data_ptr<uint8_t>()[i], eb = expected.data_ptr<uint8_t>()[i];
                if (ab != eb) return "element " + std::to_string(i) + ": bool differs";
                exact = true;
                break;
            }
            }
            if (!exact && !close(a, e, rtol, atol)) {
                std::ostringstream s;
                s.precision(17);
                s << "element " << i << ": " << a << " vs cpu " << e;
                return s.str();
            }
        }
        return "";
    }

    std::vector<std::string> failures_;
    int64_t count_ = 0;
};

using UnaryOps = std::vector<std::pair<const char*, std::function<Tensor(const Tensor&)>>>;
using BinaryOps = std::vector<std::pair<const char*, std::function<Tensor(const Tensor&, const Tensor&)>>>;

// The operations the reference's suite runs on every layout (tests/test_cuda.cpp:58-103): the
// element functions, casts, every reduction and the row operations. Arguments that would leave
// an op's domain are mapped into it (log of |x| + 1 and the like) as there.
const UnaryOps& unary_ops() {
    static const UnaryOps ops = {
        {"neg", [](const Tensor& x) { return kael::neg(x); }},
        {"abs", [](const Tensor& x) { return kael::abs(x); }},
        {"sign", [](const Tensor& x) { return kael::sign(x); }},
        {"exp", [](const Tensor& x) { return kael::exp(x); }},
        {"log", [](const Tensor& x) { return kael::log(kael::abs(x) + 1); }},
        {"log1p", [](const Tensor& x) { return kael::log1p(kael::abs(x)); }},
        {"expm1", [](const Tensor& x) { return kael::expm1(x); }},
        {"sqrt", [](const Tensor& x) { return kael::sqrt(kael::abs(x)); }},
        {"rsqrt", [](const Tensor& x) { return kael::rsqrt(kael::abs(x) + 1); }},
        {"sin", [](const Tensor& x) { return kael::sin(x); }},
        {"cos", [](const Tensor& x) { return kael::cos(x); }},
        {"tanh", [](const Tensor& x) { return kael::tanh(x); }},
        {"sigmoid", [](const Tensor& x) { return kael::sigmoid(x); }},
        {"relu", [](const Tensor& x) { return kael::relu(x); }},
        {"gelu", [](const Tensor& x) { return kael::gelu(x); }},
        {"gelu_tanh", [](const Tensor& x) { return kael::gelu(x, true); }},
        {"clamp", [](const Tensor& x) { return kael::clamp(x, -0.5, 0.5); }},
        {"clone", [](const Tensor& x) { return x.clone(); }},
        {"to_f64", [](const Tensor& x) { return x.to(DType::F64); }},
        {"to_i64", [](const Tensor& x) { return x.to(DType::I64); }},
        {"to_bool", [](const Tensor& x) { return x.to(DType::Bool); }},
        {"sum", [](const Tensor& x) { return kael::sum(x); }},
        {"sum_dim0", [](const Tensor& x) { return kael::sum(x, {0}); }},
        {"sum_last_keepdim", [](const Tensor& x) { return kael::sum(x, {-1}, true); }},
        {"mean", [](const Tensor& x) { return kael::mean(x); }},
        {"mean_dim1", [](const Tensor& x) { return kael::mean(x, {1}); }},
        {"prod_dim1", [](const Tensor& x) { return kael::prod(x, {1}); }},
        {"max", [](const Tensor& x) { return kael::max(x); }},
        {"max_dim0", [](const Tensor& x) { return kael::max(x, {0}); }},
        {"min_dim1_keepdim", [](const Tensor& x) { return kael::min(x, {1}, true); }},
        {"argmax_dim1", [](const Tensor& x) { return kael::argmax(x, 1); }},
        {"argmin", [](const Tensor& x) { return kael::argmin(x); }},
        {"var_dim1", [](const Tensor& x) { return kael::var(x, {1}); }},
        {"std", [](const Tensor& x) { return kael::std(x); }},
        {"norm_dim0", [](const Tensor& x) { return kael::norm(x, {0}); }},
        {"all_dim0", [](const Tensor& x) { return kael::all(x, {0}); }},
        {"any", [](const Tensor& x) { return kael::any(x); }},
        {"softmax_last", [](const Tensor& x) { return kael::softmax(x, -1); }},
        {"softmax_first", [](const Tensor& x) { return kael::softmax(x, 0); }},
        {"log_softmax", [](const Tensor& x) { return kael::log_softmax(x, -1); }},
        {"logsumexp_dim1", [](const Tensor& x) { return kael::logsumexp(x, 1); }},
        {"standardize", [](const Tensor& x) { return kael::standardize(x, 1, 1e-5); }},
        {"logical_not", [](const Tensor& x) { return kael::logical_not(x); }},
    };
    return ops;
}

// Binary operations with broadcasting (tests/test_cuda.cpp:105-128).
const BinaryOps& binary_ops() {
    static const BinaryOps ops = {
        {"add", [](const Tensor& a, const Tensor& b) { return a + b; }},
        {"sub", [](const Tensor& a, const Tensor& b) { return a - b; }},
        {"mul", [](const Tensor& a, const Tensor& b) { return a * b; }},
        {"div", [](const Tensor& a, const Tensor& b) { return a / (kael::abs(b) + 1); }},
        {"floor_divide", [](const Tensor& a, const Tensor& b) { return kael::floor_divide(a, kael::abs(b) + 1); }},
        {"pow", [](const Tensor& a, const Tensor& b) { return kael::pow(kael::abs(a), b); }},
        {"maximum", [](const Tensor& a, const Tensor& b) { return kael::maximum(a, b); }},
        {"minimum", [](const Tensor& a, const Tensor& b) { return kael::minimum(a, b); }},
        {"eq", [](const Tensor& a, const Tensor& b) { return a == b; }},
        {"ne", [](const Tensor& a, const Tensor& b) { return a != b; }},
        {"lt", [](const Tensor& a, const Tensor& b) { return a < b; }},
        {"le", [](const Tensor& a, const Tensor& b) { return a <= b; }},
        {"gt", [](const Tensor& a, const Tensor& b) { return a > b; }},
        {"ge", [](const Tensor& a, const Tensor& b) { return a >= b; }},
        {"logical_and", [](const Tensor& a, const Tensor& b) { return kael::logical_and(a, b); }},
        {"logical_or", [](const Tensor& a, const Tensor& b) { return kael::logical_or(a, b); }},
        {"logical_xor", [](const Tensor& a, const Tensor& b) { return kael::logical_xor(a, b); }},
        {"where", [](const Tensor& a, const Tensor& b) { return kael::where(a > 0, a, b); }},
        {"masked_fill", [](const Tensor& a, const Tensor& b) { return kael::masked_fill(a, b > 0, 7.0); }},
    };
    return ops;
}

void unary_on(Expect& x, const Tensor& device_input, const Tensor& cpu_input, const std::string& tag) {
    for (const auto& [name, op] : unary_ops()) x.matches_cpu(op(device_input), op(cpu_input), std::string(name) + "/" + tag);
}

struct Case {
    const char* name;
    std::function<void(Expect&)> body;
};

const std::vector<Case>& cases() {
    static const std::vector<Case> table = {
        // tests/test_cuda.cpp:133-144
        {"transfers_round_trip",
         [](Expect& x) {
             for (DType dtype : {DType::F32, DType::F64, DType::I64, DType::Bool}) {
                 const Tensor host = kael::randn({5, 4}).to(dtype);
                 const Tensor dev = host.cuda();
                 x.that(dev.device() == Device::CUDA && dev.dtype() == dtype, "device copy has the device and dtype");
                 x.that(!dev.shares_storage(host), "device copy owns new storage");
                 const Tensor back = dev.cpu();
                 x.that(back.device() == Device::CPU, "copy back lands on the cpu");
                 x.equal(back, host, "round trip");
             }
         }},
        // :146-151
        {"same_device_returns_the_same_tensor",
         [](Expect& x) {
             const Tensor dev = kael::ones({2}).cuda();
             x.that(dev.cuda().is_same(dev), "cuda() of a device tensor is itself");
             const Tensor host = kael::ones({2});
             x.that(host.cpu().is_same(host), "cpu() of a cpu tensor is itself");
         }},
        // :153-158
        {"non_contiguous_tensors_transfer",
         [](Expect& x) {
             const Tensor base = kael::randn({4, 6});
             const Tensor view = base.T().slice(0, 1, 6, 2);
             x.that(!view.is_contiguous(), "the view is strided");
             x.equal(view.cuda().cpu(), view.contiguous(), "strided view through the device");
         }},
        // :160-171
        {"factories_create_on_the_device",
         [](Expect& x) {
             const Tensor z = kael::zeros({3, 2}, DType::F64, Device::CUDA);
             x.that(z.device() == Device::CUDA, "zeros on the device");
             x.equal(z.cpu(), kael::zeros({3, 2}, DType::F64), "zeros");
             x.equal(kael::ones({2}, DType::I64, Device::CUDA).cpu(), kael::ones({2}, DType::I64), "ones i64");
             x.equal(kael::full({2}, 2.5, DType::F32, Device::CUDA).cpu(), kael::full({2}, 2.5, DType::F32), "full");
             x.that(kael::zeros_like(z).device() == Device::CUDA, "zeros_like follows the device");
             x.that(kael::ones_like(z).device() == Device::CUDA, "ones_like follows the device");
             x.that(kael::empty_like(z).device() == Device::CUDA, "empty_like follows the device");
         }},
        // :173-178
        {"host_only_access_fails_clearly",
         [](Expect& x) {
             Tensor dev = kael::ones({2}).cuda();
             x.throws<kael::Error>([&] { (void)dev.data_ptr<float>(); }, "data_ptr on the device");
             x.throws<kael::Error>([&] { (void)dev.at<float>({0}); }, "at() on the device");
             x.no_throw([&] { (void)dev.device_data(); }, "device_data");
         }},
        // :180-188
        {"reading_values_copies_to_host",
         [](Expect& x) {
             const Tensor dev = kael::full({1}, 3.5, DType::F64).cuda();
             x.that(dev.item<double>() == 3.5, "item<double>");
             x.that(dev.item() == 3.5, "item()");
             std::ostringstream text;
             text << kael::ones({2}).cuda();
             x.that(text.str().find("1.0000") != std::string::npos, "printed values: " + text.str());
             x.that(text.str().find("device=cuda") != std::string::npos, "printed device: " + text.str());
         }},
        // :190-203
        {"mixed_devices_are_rejected",
         [](Expect& x) {
             const Tensor dev = kael::ones({2}).cuda();
             const Tensor host = kael::ones({2});
             x.throws<kael::Error>([&] { (void)(dev + host); }, "add across devices", "same device");
             x.throws<kael::Error>([&] { (void)kael::matmul(kael::ones({2, 2}).cuda(), kael::ones({2, 2})); },
                                   "matmul across devices");
             x.throws<kael::Error>([&] { (void)kael::cat({dev, host}); }, "cat across devices");
             x.throws<kael::Error>([&] { (void)kael::gather(host, 0, kael::zeros({1}, DType::I64).cuda()); },
                                   "gather with device indices into a cpu tensor");
         }},
        // :205-212
        {"scalars_follow_the_tensor_device",
         [](Expect& x) {
             const Tensor dev = kael::full({2}, 2.0).cuda();
             x.matches_cpu(dev * 3.0, kael::full({2}, 6.0), "tensor * scalar");
             x.matches_cpu(3.0 - dev, kael::full({2}, 1.0), "scalar - tensor");
             Tensor y = dev.clone();
             y += 1;
             x.matches_cpu(y, kael::full({2}, 3.0), "in-place scalar add");
         }},
        // :214-222
        {"copy_between_devices_works",
         [](Expect& x) {
             Tensor target = kael::zeros({2, 2}).cuda();
             const Tensor source = kael::full({2, 2}, 4.0);
             target.copy_(source);
             x.matches_cpu(target, source, "cpu into device");
             Tensor host = kael::zeros({2, 2});
             host.copy_(target);
             x.equal(host, source, "device into cpu");
         }},
        // :224-243
        {"unary_ops_match_cpu_on_every_layout",
         [](Expect& x) {
             const Tensor base = kael::randn({6, 8});
             const Tensor transposed = base.T();
             const Tensor strided = base.slice(0, 0, 6, 2).slice(1, 1, 8, 2);
             unary_on(x, base.cuda(), base, "contiguous");
             unary_on(x, transposed.cuda(), transposed, "transposed");
             unary_on(x, base.cuda().T(), transposed, "device view");
             unary_on(x, strided.cuda(), strided, "strided");
         }},
        // :245-250
        {"double_precision_matches_cpu",
         [](Expect& x) {
             const Tensor v = kael::randn({6, 8}, DType::F64);
             unary_on(x, v.cuda(), v, "f64");
         }},
        // :252-265
        {"binary_ops_match_cpu_with_broadcast",
         [](Expect& x) {
             const Tensor a = kael::randn({6, 8});
             const std::vector<std::pair<const char*, Tensor>> others = {{"same", kael::randn({6, 8})},
                                                                         {"row", kael::randn({8})},
                                                                         {"column", kael::randn({6, 1})},
                                                                         {"zero_dim", kael::randn({})}};
             for (const auto& [shape, b] : others)
                 for (const auto& [name, op] : binary_ops())
                     x.matches_cpu(op(a.cuda(), b.cuda()), op(a, b), std::string(name) + "/" + shape);
         }},
        // :267-279
        {"integer_ops_match_cpu",
         [](Expect& x) {
             const Tensor a = kael::randint(-20, 20, {5, 5});
             const Tensor b = kael::randint(1, 9, {5, 5});
             const Tensor da = a.cuda(), db = b.cuda();
             x.matches_cpu(da + db, a + b, "add i64");
             x.matches_cpu(da * db, a * b, "mul i64");
             x.matches_cpu(kael::pow(da, db), kael::pow(a, b), "pow i64");
             x.matches_cpu(kael::floor_divide(da, db), kael::floor_divide(a, b), "floor_divide i64");
             x.matches_cpu(kael::sum(da), kael::sum(a), "sum i64");
             x.matches_cpu(kael::max(da, {0}), kael::max(a, {0}), "max i64");
             x.matches_cpu(kael::abs(da), kael::abs(a), "abs i64");
             x.matches_cpu(da / db, a / b, "div i64");
         }},
        // :281-285
        {"bool_reductions_match_cpu",
         [](Expect& x) {
             const Tensor flags = kael::randn({5, 5}) > 0;
             x.matches_cpu(kael::sum(flags.cuda()), kael::sum(flags), "sum bool");
             x.matches_cpu(kael::sum(flags.cuda(), {1}), kael::sum(flags, {1}), "sum dim bool");
         }},
        // :287-300
        {"non_finite_values_match_cpu",
         [](Expect& x) {
             const float inf = std::numeric_limits<float>::infinity();
             const float nan = std::numeric_limits<float>::quiet_NaN();
             const Tensor v = kael::from_vector<float>({1.0f, inf, 2.0f, -inf, 1.0f, 2.0f, nan, 1.0f, 2.0f}, {3, 3});
             const Tensor d = v.cuda();
             x.matches_cpu(kael::max(d, {1}), kael::max(v, {1}), "max");
             x.matches_cpu(kael::min(d, {1}), kael::min(v, {1}), "min");
             x.matches_cpu(kael::sum(d, {1}), kael::sum(v, {1}), "sum");
             x.matches_cpu(kael::softmax(d, -1), kael::softmax(v, -1), "softmax");
             x.matches_cpu(kael::maximum(d, v.T().cuda()), kael::maximum(v, v.T()), "maximum");
             x.matches_cpu(kael::clamp(d, 0.0, 1.0), kael::clamp(v, 0.0, 1.0), "clamp");
         }},
        // :302-311
        {"long_sums_match_cpu_and_are_deterministic",
         [](Expect& x) {
             const Tensor v = kael::randn({200000}, DType::F64);
             const Tensor first = kael::sum(v.cuda());
             const Tensor second = kael::sum(v.cuda());
             x.equal(first.cpu(), second.cpu(), "two device sums are bitwise equal");
             x.matches_cpu(first, kael::sum(v), "long sum");
             const Tensor wide = kael::randn({3, 100000});
             x.matches_cpu(kael::sum(wide.cuda(), {1}), kael::sum(wide, {1}), "wide rows sum");
             x.matches_cpu(kael::max(wide.cuda(), {1}), kael::max(wide, {1}), "wide rows max");
         }},
        // :313-320
        {"empty_tensors_work",
         [](Expect& x) {
             const Tensor empty = kael::zeros({0, 3});
             const Tensor d = empty.cuda();
             x.matches_cpu(d + d, empty + empty, "add");
             x.matches_cpu(kael::sum(d), kael::sum(empty), "sum");
             x.matches_cpu(kael::sum(d, {0}), kael::sum(empty, {0}), "sum dim");
             x.matches_cpu(kael::prod(d), kael::prod(empty), "prod");
             x.throws<kael::Error>([&] { (void)kael::max(d); }, "max of nothing");
         }},
        // :322-341 (the parameterised shapes, seed 77)
        {"matmul_shapes_match_cpu",
         [](Expect& x) {
             const int64_t shapes[][3] = {{1, 1, 1}, {4, 4, 4}, {5, 3, 9}, {8, 16, 7}, {33, 20, 65}, {64, 1, 64}, {1, 64, 1}};
             for (const auto& s : shapes) {
                 kael::manual_seed(77);
                 for (DType dtype : {DType::F32, DType::F64}) {
                     const Tensor a = kael::randn({s[0], s[1]}, dtype);
                     const Tensor b = kael::randn({s[1], s[2]}, dtype);
                     x.matches_cpu(kael::matmul(a.cuda(), b.cuda()), kael::matmul(a, b),
                                   "matmul " + std::to_string(s[0]) + "x" + std::to_string(s[1]) + "x" + std::to_string(s[2]));
                 }
             }
         }},
        // :343-355
        {"matmul_batches_vectors_and_integers_match_cpu",
         [](Expect& x) {
             const Tensor a = kael::randn({3, 1, 4, 5});
             const Tensor b = kael::randn({2, 5, 6});
             x.matches_cpu(kael::matmul(a.cuda(), b.cuda()), kael::matmul(a, b), "batched with broadcast");
             const Tensor v = kael::randn({5});
             x.matches_cpu(kael::matmul(a.cuda(), v.cuda()), kael::matmul(a, v), "matrix-vector");
             x.matches_cpu(kael::dot(v.cuda(), v.cuda()), kael::dot(v, v), "dot");
             x.matches_cpu(kael::outer(v.cuda(), v.cuda()), kael::outer(v, v), "outer");
             const Tensor i = kael::randint(-5, 5, {6, 6});
             x.matches_cpu(kael::matmul(i.cuda(), i.cuda()), kael::matmul(i, i), "i64");
             const Tensor t = kael::randn({5, 4});
             x.matches_cpu(kael::matmul(t.T().cuda(), t.cuda()), kael::matmul(t.T(), t), "transposed operand");
         }},
        // :357-384
        {"indexing_matches_cpu",
         [](Expect& x) {
             const Tensor v = kael::randn({6, 5});
             const Tensor rows = kael::from_vector<int64_t>({5, 0, 0, 2});
             const Tensor picks = kael::randint(0, 5, {6, 3});
             const Tensor d = v.cuda();
             x.matches_cpu(kael::index_select(d, 0, rows.cuda()), kael::index_select(v, 0, rows), "index_select");
             x.matches_cpu(kael::gather(d, 1, picks.cuda()), kael::gather(v, 1, picks), "gather");
             x.matches_cpu(kael::gather(d.T(), 0, picks.T().cuda()), kael::gather(v.T(), 0, picks.T()),
                           "gather transposed");
             x.matches_cpu(kael::cat({d, d}, 1), kael::cat({v, v}, 1), "cat");
             x.matches_cpu(kael::stack({d, d}), kael::stack({v, v}), "stack");
             Tensor grid = kael::zeros({6, 5});
             Tensor dgrid = grid.clone().cuda();
             const Tensor source = kael::randn({6, 3});
             grid.scatter_add_(1, picks, source);
             dgrid.scatter_add_(1, picks.cuda(), source.cuda());
             x.matches_cpu(dgrid, grid, "scatter_add_");
             Tensor added = kael::zeros({6, 5});
             Tensor dadded = added.clone().cuda();
             const Tensor row_source = kael::randn({4, 5});
             added.index_add_(0, rows, row_source);
             dadded.index_add_(0, rows.cuda(), row_source.cuda());
             x.matches_cpu(dadded, added, "index_add_");
         }},
        // :386-394
        {"out_of_range_indices_still_throw",
         [](Expect& x) {
             const Tensor d = kael::zeros({2, 2}).cuda();
             x.throws<kael::IndexError>([&] { (void)kael::index_select(d, 0, kael::full({1}, 9, DType::I64).cuda()); },
                                        "index_select past the end");
             x.throws<kael::IndexError>([&] { (void)kael::gather(d, 0, kael::full({1, 2}, 9, DType::I64).cuda()); },
                                        "gather past the end");
             x.throws<kael::IndexError>([&] { (void)kael::gather(d, 0, kael::full({1, 2}, -1, DType::I64).cuda()); },
                                        "gather below zero");
         }},
        // :396-408
        {"backward_matches_cpu_and_stays_on_the_device",
         [](Expect& x) {
             const Tensor cpu_x = kael::randn({4, 3}, DType::F64).requires_grad_();
             const Tensor dev_x = cpu_x.detach().clone().cuda().requires_grad_();
             const auto loss = [](const Tensor& t) {
                 const Tensor hidden = kael::tanh(kael::matmul(t, t.T()));
                 return kael::sum(kael::softmax(hidden, -1) * hidden) + kael::mean(kael::exp(t)) +
                        kael::sum(kael::gelu(t, true)) + kael::sum(kael::max(t, {1}));
             };
             loss(cpu_x).backward();
             loss(dev_x).backward();
             x.that(dev_x.grad()->device() == Device::CUDA, "gradient stays on the device");
             x.matches_cpu(*dev_x.grad(), *cpu_x.grad(), "gradient");
         }},
        // :410-420
        {"gradients_cross_devices_back_to_the_origin",
         [](Expect& x) {
             const Tensor host = kael::randn({3}, DType::F64).requires_grad_();
             const Tensor moved = host.cuda();
             kael::sum(moved * moved).backward();
             x.that(host.grad()->device() == Device::CPU, "gradient returns to the cpu leaf");
             const Tensor want = host.detach() * 2;
             const Tensor got = *host.grad();
             bool ok = got.shape() == want.shape();
             for (int64_t i = 0; ok && i < 3; ++i)
                 ok = std::abs(got.data_ptr<double>()[i] - want.data_ptr<double>()[i]) <=
                      1e-14 + 1e-12 * std::abs(want.data_ptr<double>()[i]);
             x.that(ok, "gradient of sum(x*x) is 2x");
             const Tensor dev = kael::randn({3}, DType::F64).cuda().requires_grad_();
             kael::sum(dev.cpu() * 3).backward();
             x.that(dev.grad()->device() == Device::CUDA, "gradient returns to the device leaf");
         }},
        // :422-436
        {"view_and_indexing_gradients_match_cpu",
         [](Expect& x) {
             const Tensor cpu_x = kael::randn({4, 5}, DType::F64).requires_grad_();
             const Tensor dev_x = cpu_x.detach().clone().cuda().requires_grad_();
             const Tensor rows = kael::from_vector<int64_t>({1, 1, 3});
             const auto loss = [](const Tensor& t, const Tensor& picked) {
                 const Tensor narrowed = t.slice(1, 1, 5, 2).select(0, 2);
                 const Tensor selected = kael::index_select(t, 0, picked);
                 const Tensor gathered = kael::gather(t, 1, kael::zeros_like(t).to(DType::I64));
                 return kael::sum(narrowed * narrowed) + kael::sum(selected * 2) + kael::sum(gathered) +
                        kael::sum(kael::cat({t, t}, 0).T()) + kael::sum(kael::log_softmax(t, 0));
             };
             loss(cpu_x, rows).backward();
             loss(dev_x, rows.cuda()).backward();
             x.matches_cpu(*dev_x.grad(), *cpu_x.grad(), "gradient");
         }},
        // :438-446
        {"gradcheck_runs_on_the_device",
         [](Expect& x) {
             const Tensor v = kael::randn({3, 2}, DType::F64).requires_grad_();
             const auto result = kael::autograd::gradcheck(
                 [](const std::vector<Tensor>& in) { return kael::sum(kael::tanh(in[0].cuda()) * in[0].cuda()).cpu(); },
                 {v});
             x.that(result.passed, "gradcheck: " + result.report);
         }},
        // :448-460
        {"module_to_keeps_parameter_identity_and_values",
         [](Expect& x) {
             kael::nn::Linear layer(3, 2);
             const Tensor weight = layer.weight();
             const Tensor before = weight.detach().clone();
             layer.to(Device::CUDA);
             x.that(layer.weight().is_same(weight), "the parameter object is kept");
             x.that(weight.device() == Device::CUDA, "the parameter moved");
             x.that(weight.requires_grad(), "still requires grad");
             x.equal(weight.detach().cpu(), before, "values kept on the device");
             layer.to(Device::CPU);
             x.that(weight.device() == Device::CPU, "moved back");
             x.equal(weight.detach(), before, "values kept on the way back");
         }},
        // :462-468
        {"module_to_moves_existing_gradients",
         [](Expect& x) {
             kael::nn::Linear layer(2, 1);
             kael::sum(layer(kael::ones({1, 2}))).backward();
             layer.to(Device::CUDA);
             const auto grad = layer.weight().grad();
             x.that(grad.has_value() && grad->device() == Device::CUDA, "the gradient moved with the parameter");
         }},
        // :470-480
        {"integer_clamp_and_masked_fill_keep_every_bit",
         [](Expect& x) {
             const int64_t large = (int64_t{1} << 53) + 1;
             const Tensor values = kael::from_vector(std::vector<int64_t>{0, large + 10}).to(Device::CUDA);
             const Tensor clamped = kael::clamp(values, large, large).cpu();
             x.that(clamped.data_ptr<int64_t>()[0] == large && clamped.data_ptr<int64_t>()[1] == large,
                    "clamp to 2^53+1 is exact");
             const Tensor mask = kael::from_vector({true, false}).to(Device::CUDA);
             const Tensor filled = kael::masked_fill(values, mask, large).cpu();
             x.that(filled.data_ptr<int64_t>()[0] == large, "masked_fill with 2^53+1 is exact");
         }},
        // :482-489
        {"integer_scatter_add_wraps_around",
         [](Expect& x) {
             constexpr int64_t kMax = std::numeric_limits<int64_t>::max();
             Tensor target = kael::from_vector(std::vector<int64_t>{kMax}).to(Device::CUDA);
             target.scatter_add_(0, kael::from_vector(std::vector<int64_t>{0}).to(Device::CUDA),
                                 kael::from_vector(std::vector<int64_t>{1}).to(Device::CUDA));
             x.that(target.cpu().data_ptr<int64_t>()[0] == std::numeric_limits<int64_t>::min(), "INT64_MAX + 1 wraps");
         }},
        // :491-500
        {"integer_sum_wraps_and_float_conversion_saturates",
         [](Expect& x) {
             constexpr int64_t kMax = std::numeric_limits<int64_t>::max();
             const Tensor longs = kael::from_vector(std::vector<int64_t>{kMax, 1}).to(Device::CUDA);
             x.that(kael::sum(longs).item<int64_t>() == std::numeric_limits<int64_t>::min(), "sum wraps");
             const Tensor floats = kael::from_vector(std::vector<double>{std::nan(""), 1e300}).to(Device::CUDA);
             const Tensor converted = floats.to(DType::I64).cpu();
             x.that(converted.data_ptr<int64_t>()[0] == 0, "NaN converts to 0");
             x.that(converted.data_ptr<int64_t>()[1] == kMax, "1e300 saturates to INT64_MAX");
         }},
        // :502-514
        {"layers_match_cpu",
         [](Expect& x) {
             kael::nn::LayerNorm norm({4}, 1e-5, DType::F64);
             const Tensor v = kael::randn({2, 3, 4}, DType::F64);
             const Tensor want = norm(v);
             norm.to(Device::CUDA);
             x.matches_cpu(norm(v.cuda()), want, "layer norm");
             kael::nn::Embedding embedding(10, 4);
             const Tensor tokens = kael::randint(0, 10, {2, 3});
             const Tensor embedded = embedding(tokens);
             embedding.to(Device::CUDA);
             x.matches_cpu(embedding(tokens.cuda()), embedded, "embedding");
         }},
        // :516-552
        {"training_matches_cpu_step_by_step",
         [](Expect& x) {
             const auto build = [] {
                 kael::manual_seed(5);
                 return kael::nn::Sequential{std::make_shared<kael::nn::Linear>(4, 8, true, DType::F64),
                                             std::make_shared<kael::nn::ReLU>(),
                                             std::make_shared<kael::nn::Linear>(8, 3, true, DType::F64)};
             };
             kael::nn::Sequential cpu_model = build();
             kael::nn::Sequential dev_model = build();
             dev_model.to(Device::CUDA);
             kael::optim::AdamW cpu_opt(cpu_model.parameters());
             kael::optim::AdamW dev_opt(dev_model.parameters());
             kael::manual_seed(6);
             const Tensor inputs = kael::randn({16, 4}, DType::F64);
             const Tensor targets = kael::randint(0, 3, {16});
             for (int step = 0; step < 20; ++step) {
                 cpu_opt.zero_grad();
                 const Tensor cpu_loss = kael::nn::cross_entropy(cpu_model(inputs), targets);
                 cpu_loss.backward();
                 kael::optim::clip_grad_norm_(cpu_model.parameters(), 1.0);
                 cpu_opt.step();
                 dev_opt.zero_grad();
                 const Tensor dev_loss = kael::nn::cross_entropy(dev_model(inputs.cuda()), targets.cuda());
                 dev_loss.backward();
                 kael::optim::clip_grad_norm_(dev_model.parameters(), 1.0);
                 dev_opt.step();
                 x.matches_cpu(dev_loss, cpu_loss, "loss at step " + std::to_string(step));
             }
             const auto cpu_params = cpu_model.parameters();
             const auto dev_params = dev_model.parameters();
             for (size_t i = 0; i < cpu_params.size(); ++i)
                 x.matches_cpu(dev_params[i].detach(), cpu_params[i].detach(), "parameter " + std::to_string(i));
         }},
        // :554-572
        {"device_blocks_are_cached",
         [](Expect& x) {
             if (!kael::caching_allocator_enabled()) throw Skip{"kael built without the caching allocator"};
             kael::empty_cache();
             { const Tensor warm = kael::zeros({1000}).cuda(); }
             const kael::AllocatorStats before = kael::allocator_stats(Device::CUDA);
             x.that(before.cached_bytes > 0, "a released block stays cached");
             { const Tensor again = kael::zeros({1000}).cuda(); }
             const kael::AllocatorStats after = kael::allocator_stats(Device::CUDA);
             x.that(after.hits == before.hits + 1, "the second block is a cache hit");
             x.that(after.misses == before.misses, "and no new device allocation");
             kael::empty_cache();
             x.that(kael::allocator_stats(Device::CUDA).cached_bytes == 0, "empty_cache releases every block");
         }},
        // :574-582
        {"sequence_ops_match_cpu",
         [](Expect& x) {
             const Tensor v = kael::randn({5, 6});
             const Tensor d = v.cuda();
             x.matches_cpu(kael::cumsum(d, 1), kael::cumsum(v, 1), "cumsum");
             x.matches_cpu(kael::sort(d, 1).values, kael::sort(v, 1).values, "sort");
             x.matches_cpu(kael::topk(d, 2).indices, kael::topk(v, 2).indices, "topk");
             x.matches_cpu(kael::tril(d), kael::tril(v), "tril");
             x.matches_cpu(kael::triu(d, 1), kael::triu(v, 1), "triu");
             x.that(kael::multinomial(kael::ones({3}).cuda(), 2, true).device() == Device::CUDA,
                    "multinomial samples land on the device");
         }},
        // :584-609
        {"gpt_matches_cpu_including_the_cache_and_generation",
         [](Expect& x) {
             kael::nn::GptConfig config;
             config.vocab_size = 11;
             config.max_positions = 16;
             config.layers = 2;
             config.heads = 2;
             config.dimension = 8;
             config.dtype = DType::F64;
             kael::manual_seed(31);
             kael::nn::GPT model(config);
             const Tensor tokens = kael::randint(0, 11, {2, 6});
             const Tensor logits = model(tokens);
             const Tensor generated = kael::nn::generate(model, tokens, {.max_new_tokens = 4, .temperature = 0.0});
             model.to(Device::CUDA);
             x.matches_cpu(model(tokens.cuda()), logits, "logits");
             x.matches_cpu(kael::nn::generate(model, tokens.cuda(), {.max_new_tokens = 4, .temperature = 0.0}), generated,
                           "greedy generation with the cache");
             x.matches_cpu(kael::nn::generate(model, tokens.cuda(),
                                              {.max_new_tokens = 4, .temperature = 0.0, .use_cache = false}),
                           generated, "greedy generation without the cache");
             kael::sum(model(tokens.cuda())).backward();
             x.that(model.parameters()[0].grad()->device() == Device::CUDA, "parameter gradients on the device");
         }},
        // :611-620
        {"stepped_indices_work_on_the_device",
         [](Expect& x) {
             const Tensor v = kael::randn({4, 2}, DType::F64);
             const Tensor dev = v.clone().cuda().requires_grad_();
             const Tensor every_other = kael::from_vector<int64_t>({3, 0, 1, 0}).slice(0, 0, 4, 2);
             const Tensor selected = kael::index_select(dev, 0, every_other.cuda());
             x.matches_cpu(selected.detach(), kael::index_select(v, 0, every_other), "forward");
             kael::sum(selected).backward();
             x.that(dev.grad()->device() == Device::CUDA, "gradient on the device");
         }},
    };
    return table;
}

} // namespace

extern "C" {

int ref_suite_size(void) { return static_cast<int>(cases().size()); }

const char* ref_suite_name(int i) {
    if (i < 0 || i >= ref_suite_size()) return "";
    return cases()[static_cast<size_t>(i)].name;
}

const char* ref_suite_message(void) { return g_suite_message.c_str(); }

// The comparison rules must reject what they exist to reject: returns the number of planted
// mismatches (value, NaN, infinity sign, shape, dtype, device, integer, exact equality) that went
// unnoticed, so 0 means every one was caught.
int ref_suite_self_check(void) {
    int missed = 0;
    const auto caught = [&](const std::function<void(Expect&)>& plant) {
        Expect e;
        plant(e);
        if (e.passed()) ++missed;
    };
    const Tensor ones = kael::ones({3});
    caught([&](Expect& e) { e.matches_cpu(ones.cuda(), kael::full({3}, 1.001), "value"); });
    caught([&](Expect& e) { e.matches_cpu(ones.cuda(), kael::full({3}, std::nan("")), "nan"); });
    caught([&](Expect& e) {
        const float inf = std::numeric_limits<float>::infinity();
        e.matches_cpu(kael::from_vector<float>({inf}).cuda(), kael::from_vector<float>({-inf}), "inf sign");
    });
    caught([&](Expect& e) { e.matches_cpu(ones.cuda(), kael::ones({3, 1}), "shape"); });
    caught([&](Expect& e) { e.matches_cpu(ones.cuda(), kael::ones({3}, DType::F64), "dtype"); });
    caught([&](Expect& e) { e.matches_cpu(ones, ones, "device"); });
    caught([&](Expect& e) {
        e.matches_cpu(kael::from_vector<int64_t>({(int64_t{1} << 53) + 1}).cuda(), kael::from_vector<int64_t>({int64_t{1} << 53}),
                      "integer");
    });
    caught([&](Expect& e) { e.equal(ones, kael::full({3}, 1.0000001), "equal"); });
    caught([&](Expect& e) { e.throws<kael::Error>([] {}, "throws"); });
    return missed;
}

// 0 = passed, 1 = failed (report in ref_suite_message), 2 = skipped (reason there), -1 = bad index.
int ref_suite_run(int i) {
    if (i < 0 || i >= ref_suite_size()) return -1;
    g_suite_message.clear();
    if (!kael::cuda_is_available()) {
        g_suite_message = "no device backend available";
        return 2;
    }
    kael::manual_seed(2024);
    Expect expect;
    try {
        cases()[static_cast<size_t>(i)].body(expect);
    } catch (const Skip& skip) {
        g_suite_message = skip.reason;
        return 2;
    } catch (const std::exception& error) {
        expect.fail(std::string("unexpected exception: ") + error.what());
    }
    if (expect.passed()) return 0;
    g_suite_message = expect.report();
    return 1;
}

} // extern "C"
