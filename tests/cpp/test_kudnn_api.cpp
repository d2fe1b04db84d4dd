// Tests of the KuDNN-compatible C++ API (libkudnn.so): the reference gtests' negative and copy/move cases
// (test/dnn/llt/gtest/src/linear_activation_gtest.cpp:217-460, linear_res_gtest.cpp:547-765,
// matmul_gtest.cpp:437-545), re-expressed with a minimal assert harness (googletest is not available).
//
//   test_kudnn_api            host-only cases (descriptors, validation, exceptions); no GPU needed
//   test_kudnn_api --gpu      also runs numeric cases with host buffers, the way the reference's own tests
//                             call Run, and checks them against the CPU oracle (liboracle.so)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "kudnn.hpp"

using namespace KuDNN;

static int g_failed = 0;
static int g_passed = 0;

#define CHECK(cond)                                                                  \
    do {                                                                             \
        if (!(cond)) {                                                               \
            std::printf("  FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);            \
            ++g_failed;                                                              \
        } else {                                                                     \
            ++g_passed;                                                              \
        }                                                                            \
    } while (0)

template <typename E>
static bool Throws(const std::function<void()> &f)
{
    try {
        f();
    } catch (const E &) {
        return true;
    } catch (const std::exception &e) {
        std::printf("  unexpected exception type: %s\n", e.what());
        return false;
    }
    return false;
}

static bool NoThrow(const std::function<void()> &f)
{
    try {
        f();
    } catch (const std::exception &e) {
        std::printf("  unexpected exception: %s\n", e.what());
        return false;
    }
    return true;
}

static const Element::TypeT F32 = Element::TypeT::F32;
static const Element::TypeT BF16 = Element::TypeT::BF16;

static TensorInfo T5(Shape s, Element::TypeT t = F32, Layout l = Layout::ABCDE) { return TensorInfo(s, t, l); }
static TensorInfo Ones5(Element::TypeT t = F32) { return T5(Shape{1, 1, 1, 1, 1}, t); }

// ---------------------------------------------------------------------------------------------------
// descriptors

static void TestTensorInfo()
{
    std::printf("TensorInfo\n");
    TensorInfo w({4096, 11008}, BF16, Layout::BA);
    CHECK(w.GetStrides()[0] == 1 && w.GetStrides()[1] == 4096);  // logical [K,N], physical [N][K]
    CHECK(w.IsDense());
    TensorInfo b({1, 11008}, F32, Layout::AB);
    CHECK(b.GetStrides()[0] == 0 && b.GetStrides()[1] == 1);  // size-1 dims broadcast with stride 0
    TensorInfo x3({8, 2048, 5120}, BF16, Layout::ABC);
    CHECK(x3.GetStrides()[0] == 2048u * 5120u && x3.GetStrides()[1] == 5120 && x3.GetStrides()[2] == 1);
    TensorInfo acb({2, 3, 4}, F32, Layout::ACB);
    CHECK(acb.GetStrides()[0] == 12 && acb.GetStrides()[1] == 1 && acb.GetStrides()[2] == 3);
    CHECK(acb.GetAxisNumAccordingToLayout(1) == 2);
    CHECK(acb.HasStrideOverFastestDim() == false);
    TensorInfo strided({4, 5}, F32, Layout::AB, Shape{8, 1});
    CHECK(!strided.IsDense());
    CHECK(Throws<Service::LogicError>([] { TensorInfo t({4, 5}, F32, Layout::AB, Shape{4, 1}); }));
    CHECK(Throws<Service::LogicError>([] { TensorInfo t({1, 1, 1, 1, 1}, F32, Layout::ABCD); }));
    CHECK(Throws<Service::LogicError>([] { TensorInfo t({4, 5}, Element::TypeT::UNDEFINED, Layout::AB); }));
    CHECK(Throws<Service::LogicError>([] { Shape s(1, 2, 3, 4, 5, 6); }));
    CHECK(Throws<Service::LogicError>([] { Shape s(65536, 65536); }));  // 2^32 elements * 4 B > 3 GiB
    CHECK(TensorInfo({2, 3}, F32, Layout::AB).GetStandardBXALayout() == Layout::BA);
    CHECK(Element::Type(BF16).GetSize() == 2);
    CHECK(Service::GetIdxForUserLayout(Layout::CAB, 0) == 2);
}

// ---------------------------------------------------------------------------------------------------
// LinearActivationLayerFWD (linear_activation_gtest.cpp:217-460)

static LinearActivationLayerFWD MakeLA(TensorInfo s, TensorInfo w, TensorInfo d, TensorInfo b,
                                       ActivationFunction k = ActivationFunction::RELU, int nt = 0)
{
    return LinearActivationLayerFWD(s, w, d, b, 1.0f, 0.0f, k, nt);
}

static void TestLinearActivationNegative()
{
    std::printf("LinearActivationLayerFWD negative cases\n");
    CHECK(NoThrow([] {
        auto l1 = MakeLA(Ones5(), Ones5(), Ones5(), Ones5());
        LinearActivationLayerFWD l2(l1);
        LinearActivationLayerFWD l3(std::move(l1));
        l2 = l3;
        l3 = std::move(l2);
    }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(T5(Shape(-1, 1, 1, 1, 1)), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(Ones5(), T5(Shape{1, 1, 2, 2, 1}), Ones5(), Ones5()); }));
    CHECK(Throws<Service::Unsupported>(
        [] { MakeLA(Ones5(), Ones5(), Ones5(Element::TypeT::S8), Ones5(), ActivationFunction::SWISH); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLA(TensorInfo({1, 1, 1, 1, 1}, F32, Layout::ABCD), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] {
        auto l = MakeLA(Ones5(), Ones5(), Ones5(), Ones5());
        l.Run(nullptr, nullptr, nullptr, nullptr, 0);
    }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(T5(Shape(1, -1, 1, 1, 1)), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(T5(Shape(1, 1, -1, 1, 1)), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(T5(Shape(1, 1, 1, -1, 1)), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] { MakeLA(Ones5(), T5(Shape(1, 1, 1, 1, -1)), Ones5(), Ones5()); }));
    CHECK(Throws<Service::Unsupported>(
        [] { MakeLA(Ones5(), Ones5(), Ones5(), Ones5(), ActivationFunction::UNIMPLEMENTED); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLA(Ones5(), Ones5(), Ones5(), Ones5(), ActivationFunction::UNIMPLEMENTED, -1); }));
    // every forward kind of KuDNN's eltwise table is a fused epilogue here; the backward-only kinds are refused
    CHECK(LinearActivationLayerFWD::ValidateInput(Ones5(), Ones5(), Ones5(), Ones5(), 1.0f, 0.0f,
                                                  ActivationFunction::TANH) == Status::SUCCESS);
    CHECK(!Throws<Service::Unsupported>([] { MakeLA(Ones5(), Ones5(), Ones5(), Ones5(), ActivationFunction::TANH); }));
    CHECK(Throws<Service::Unsupported>([] { MakeLA(Ones5(), Ones5(), Ones5(), Ones5(), ActivationFunction::EXP_DST); }));
    // bias pointer without a bias descriptor
    CHECK(Throws<Service::LogicError>([] {
        LinearActivationLayerFWD l(Ones5(), Ones5(), Ones5(), 1.0f, 0.0f, ActivationFunction::RELU);
        float x = 1.0f;
        l.Run(&x, &x, &x, &x, 0);
    }));
}

// ---------------------------------------------------------------------------------------------------
// LinearResFWD (linear_res_gtest.cpp:547-765)

static LinearResFWD MakeLR(TensorInfo s, TensorInfo w, TensorInfo d, TensorInfo b, TensorInfo r, TensorInfo lr,
                           ResOpsFunction k = ResOpsFunction::RES_MUL, int nt = 0)
{
    return LinearResFWD(s, w, d, b, r, lr, 1.0f, 0.0f, 2.0f, k, nt);
}

static void TestLinearResNegative()
{
    std::printf("LinearResFWD negative cases\n");
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(T5(Shape(-1, 1, 1, 1, 1)), Ones5(), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(Ones5(), T5(Shape{1, 1, 2, 2, 1}), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::Unsupported>(
        [] { MakeLR(Ones5(), Ones5(), Ones5(), Ones5(), Ones5(Element::TypeT::S32), Ones5()); }));
    CHECK(Throws<Service::LogicError>([] {
        MakeLR(TensorInfo({1, 1, 1, 1, 1}, F32, Layout::ABCD), Ones5(), Ones5(), Ones5(), Ones5(), Ones5());
    }));
    CHECK(Throws<Service::LogicError>([] {
        auto l = MakeLR(Ones5(), Ones5(), Ones5(), Ones5(), Ones5(), Ones5());
        l.Run(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 2.0f);
    }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(T5(Shape(1, -1, 1, 1, 1)), Ones5(), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(T5(Shape(1, 1, -1, 1, 1)), Ones5(), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(T5(Shape(1, 1, 1, -1, 1)), Ones5(), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(Ones5(), T5(Shape(1, 1, 1, 1, -1)), Ones5(), Ones5(), Ones5(), Ones5()); }));
    CHECK(Throws<Service::LogicError>(
        [] { MakeLR(Ones5(), Ones5(), Ones5(), Ones5(), Ones5(), Ones5(), ResOpsFunction::RES_MUL, -1); }));
    CHECK(NoThrow([] {
        auto l1 = MakeLR(Ones5(), Ones5(), Ones5(), Ones5(), Ones5(), Ones5(), ResOpsFunction::RES_EXT);
        LinearResFWD l2(l1);
        LinearResFWD l3(std::move(l1));
        l2 = l3;
    }));
}

// ---------------------------------------------------------------------------------------------------
// Gemm (matmul_gtest.cpp:437-545)

static void TestGemmNegative()
{
    std::printf("Gemm negative cases\n");
    const int max = Threading::GetMaxNumThreads();
    CHECK(max >= 1);
    CHECK(Throws<Service::LogicError>([] {
        Gemm g(TensorInfo({5, 5}, F32, Layout::AB), TensorInfo({5, 5}, F32, Layout::AB),
               TensorInfo({5, 5}, F32, Layout::AB), 10000000);
    }));
    CHECK(Throws<Service::LogicError>([] {
        Gemm g(TensorInfo({5, 5}, F32, Layout::AB), TensorInfo({5, 5}, F32, Layout::AB),
               TensorInfo({5, 5}, F32, Layout::AB), -20);
    }));
    // shapes whose element count overflows throw while the Shape is built (D1 = -1 with M = K = 5)
    CHECK(Throws<Service::LogicError>([] {
        Shape s(-1, 1, 1, 5, 5);
        (void)s;
    }));
    CHECK(Throws<Service::LogicError>([] {
        Gemm g(T5(Shape(1, 1, 1, 5, 5), BF16), T5(Shape(1, 1, 1, 5, -5), BF16), T5(Shape(1, 1, 1, 5, 5), BF16),
               T5(Shape(1, 1, 1, 5, 5)), 0);
    }));
    CHECK(Gemm::ValidateInput(TensorInfo({5, 6}, F32, Layout::AB), TensorInfo({6, 7}, F32, Layout::BA),
                              TensorInfo({5, 7}, F32, Layout::AB)) == Status::SUCCESS);
    CHECK(Gemm::ValidateInput(TensorInfo({5, 6}, F32, Layout::AB), TensorInfo({7, 7}, F32, Layout::BA),
                              TensorInfo({5, 7}, F32, Layout::AB)) == Status::BAD_ARGUMENTS);
    CHECK(Gemm::ValidateInput(TensorInfo({5, 6}, Element::TypeT::S32, Layout::AB), TensorInfo({6, 7}, F32, Layout::BA),
                              TensorInfo({5, 7}, F32, Layout::AB)) == Status::UNSUPPORTED);
    // non-dense destination
    CHECK(Gemm::ValidateInput(TensorInfo({5, 6}, F32, Layout::AB), TensorInfo({6, 7}, F32, Layout::BA),
                              TensorInfo({5, 7}, F32, Layout::AB, Shape{8, 1})) == Status::UNSUPPORTED);
    // bias must broadcast to [M, N]
    CHECK(Gemm::ValidateInput(TensorInfo({5, 6}, F32, Layout::AB), TensorInfo({6, 7}, F32, Layout::BA),
                              TensorInfo({5, 7}, F32, Layout::AB), TensorInfo({2, 7}, F32, Layout::AB)) ==
          Status::BAD_ARGUMENTS);
    CHECK(NoThrow([] {
        Gemm g1(TensorInfo({5, 6}, F32, Layout::AB), TensorInfo({6, 7}, F32, Layout::BA),
                TensorInfo({5, 7}, F32, Layout::AB));
        Gemm g2(g1);
        Gemm g3(std::move(g1));
        g2 = g3;
        g3 = std::move(g2);
    }));
    // threading API keeps KuDNN's contract: out-of-range requests are ignored and the old value returned
    const int old = Threading::SetMaxNumThreads(0);
    CHECK(old == Threading::GetMaxNumThreads());
    CHECK(Threading::SetMaxNumThreads(1 << 20) == old);
}

// ---------------------------------------------------------------------------------------------------
// numeric cases with host buffers (needs a GPU), checked against the CPU oracle

#include "oracle.h"

static otensor OT(const TensorInfo &t)
{
    otensor o;
    std::memset(&o, 0, sizeof(o));
    o.ndims = static_cast<int32_t>(t.GetNumDims());
    o.dtype = static_cast<int32_t>(static_cast<Element::TypeT>(t.GetType()));
    for (SizeType i = 0; i < t.GetNumDims(); ++i) {
        o.dims[i] = static_cast<int64_t>(t.GetDims()[i]);
        o.strides[i] = static_cast<int64_t>(t.GetStrides()[i]);
    }
    return o;
}

static float MaxNormErr(const std::vector<float> &got, const std::vector<float> &ref)
{
    float md = 0.0f, mr = 0.0f;
    for (size_t i = 0; i < got.size(); ++i) {
        md = std::fmax(md, std::fabs(got[i] - ref[i]));
        mr = std::fmax(mr, std::fabs(ref[i]));
    }
    return mr > 0.0f ? md / mr : md;
}

static void TestNumericHostBuffers()
{
    std::printf("numeric (host buffers through the GPU)\n");
    // FWD_LINEAR_RELU_2D_FP32 shape of the reference test (linear_activation_gtest.cpp:461-476)
    {
        TensorInfo s({110, 20}, F32, Layout::AB), w({20, 200}, F32, Layout::AB), d({110, 200}, F32, Layout::AB),
            b({110, 200}, F32, Layout::AB);
        std::vector<float> vs(110 * 20), vw(20 * 200), vb(110 * 200), vd(110 * 200), vr(110 * 200);
        oracle_fill(vs.data(), 1, vs.size(), 100, 0, -1.0, 1.0);
        oracle_fill(vw.data(), 1, vw.size(), 101, 0, -1.0, 1.0);
        oracle_fill(vb.data(), 1, vb.size(), 102, 0, -1.0, 1.0);
        LinearActivationLayerFWD l(s, w, d, b, 0.0f, 0.0f, ActivationFunction::RELU, 0);
        l.Run(vs.data(), vw.data(), vd.data(), vb.data(), 0);
        ogemm g;
        std::memset(&g, 0, sizeof(g));
        g.a = OT(s); g.b = OT(w); g.c = OT(d); g.bias = OT(b);
        g.pa = vs.data(); g.pb = vw.data(); g.pbias = vb.data(); g.pc = vr.data();
        g.alpha = 1.0f;
        oracle_linear_act(&g, 5, 0.0f);
        const float e = MaxNormErr(vd, vr);
        std::printf("  linear+relu 110x20x200 fp32: max-normalised error %.3e\n", e);
        CHECK(e <= 1e-5f);
    }
    // FWD_LINEAR_RES_EXT fp32 with a W stored [N][K] (Layout::BA)
    {
        TensorInfo s({64, 48}, F32, Layout::AB), w({48, 80}, F32, Layout::BA), d({64, 80}, F32, Layout::AB),
            b({1, 80}, F32, Layout::AB), r({64, 80}, F32, Layout::AB), lr({64, 80}, F32, Layout::AB);
        std::vector<float> vs(64 * 48), vw(48 * 80), vb(80), vr(64 * 80), vc(64 * 80), vl(64 * 80), rc(64 * 80),
            rl(64 * 80);
        oracle_fill(vs.data(), 1, vs.size(), 110, 0, -1.0, 1.0);
        oracle_fill(vw.data(), 1, vw.size(), 111, 0, -1.0, 1.0);
        oracle_fill(vb.data(), 1, vb.size(), 112, 0, -0.1, 0.1);
        oracle_fill(vr.data(), 1, vr.size(), 113, 0, -1.0, 1.0);
        LinearResFWD op(s, w, d, b, r, lr, 1.0f, 0.0f, 1.0f, ResOpsFunction::RES_EXT, 0);
        op.Run(vs.data(), vw.data(), vc.data(), vb.data(), vr.data(), vl.data(), 0.5f);
        ogemm g;
        std::memset(&g, 0, sizeof(g));
        g.a = OT(s); g.b = OT(w); g.c = OT(d); g.bias = OT(b);
        g.pa = vs.data(); g.pb = vw.data(); g.pbias = vb.data(); g.pc = rc.data();
        g.alpha = 1.0f;
        otensor ores = OT(r), olr = OT(lr);
        oracle_linear_res(&g, &ores, vr.data(), &olr, rl.data(), 0, 0.5f);
        const float e1 = MaxNormErr(vc, rc), e2 = MaxNormErr(vl, rl);
        std::printf("  linear+res_ext 64x48x80 fp32: C %.3e linearRes %.3e\n", e1, e2);
        CHECK(e1 <= 1e-5f && e2 <= 1e-5f);
    }
}

int main(int argc, char **argv)
{
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    // unbuffered: a crash (here or at process exit) still leaves every line printed before it in the captured output
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    TestTensorInfo();
    TestLinearActivationNegative();
    TestLinearResNegative();
    TestGemmNegative();
    if (gpu) {
        TestNumericHostBuffers();
    }
    std::printf("%d checks passed, %d failed\n", g_passed, g_failed);
    std::printf("exiting\n");
    return g_failed == 0 ? 0 : 1;
}
