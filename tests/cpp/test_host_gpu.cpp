// Device tests of the C++ host layer (run on the MI355X by
// tests/test_host_cpp.py).  Every result is checked against the float64
// oracle (oracle/soar_oracle.c) with the path's parity bar
// |d| <= 1e-4 * (1 + |truth|) (statistics 1e-5 relative).
#include <cmath>
#include <cstdio>
#include <vector>

#include "check.hpp"
#include "soar/autograd.hpp"
#include "soar/engine.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar/model.hpp"
#include "soar/nn.hpp"
#include "soar_oracle.h"

using namespace soar;

static const float kEps = 1e-5f;

static double max_err(const std::vector<float>& got, const std::vector<double>& truth) {
    CHECK(got.size() == truth.size());
    double m = 0.0;
    for (size_t i = 0; i < got.size(); ++i)
        m = std::max(m, std::fabs((double)got[i] - truth[i]) / (1.0 + std::fabs(truth[i])));
    return m;
}

struct Data {
    int64_t N, C, H, W, G;
    std::vector<float> x, gamma, beta, dy;
    int64_t n() const { return N * C * H * W; }
};

static Data make_data(int64_t N, int64_t C, int64_t H, int64_t W, int64_t G, uint64_t seed) {
    Data d{N, C, H, W, G, {}, {}, {}, {}};
    d.x.resize(d.n());
    d.dy.resize(d.n());
    d.gamma.resize(C);
    d.beta.resize(C);
    orc_fill_normal(d.x.data(), d.n(), seed, 1, 0.0, 1.0);
    orc_fill_uniform(d.gamma.data(), C, seed, 2, 0.5, 1.5);
    orc_fill_normal(d.beta.data(), C, seed, 3, 0.0, 0.1);
    orc_fill_normal(d.dy.data(), d.n(), seed, 4, 0.0, 1e-2);
    return d;
}

static void set_params(nn::GroupNorm& m, const std::vector<float>& g, const std::vector<float>& b) {
    for (size_t c = 0; c < g.size(); ++c) {
        m.weight()->data()[c] = g[c];
        m.bias()->data()[c] = b[c];
    }
    m.to_device();
}

struct Truth {
    std::vector<double> y, dx, dg, db, mean, rstd;
};

static Truth oracle_block(const std::vector<float>& x, const Data& d, const std::vector<float>& dy,
                          const float* gamma, const float* beta, int silu, int residual) {
    Truth t;
    const int64_t HW = d.H * d.W;
    t.y.resize(x.size());
    t.dx.resize(x.size());
    t.dg.resize(d.C);
    t.db.resize(d.C);
    t.mean.resize(d.N * d.G);
    t.rstd.resize(d.N * d.G);
    CHECK(orc_gn_silu_fwd_f64(x.data(), gamma, beta, d.N, d.C, HW, d.G, (double)kEps, silu,
                              residual, t.y.data(), t.mean.data(), t.rstd.data()) == 0);
    CHECK(orc_gn_silu_bwd_f64(dy.data(), x.data(), gamma, beta, t.mean.data(), t.rstd.data(), d.N,
                              d.C, HW, d.G, silu, residual, t.dx.data(), t.dg.data(),
                              t.db.data()) == 0);
    return t;
}

static void check_close(const char* what, const std::vector<float>& got,
                        const std::vector<double>& truth) {
    const double e = max_err(got, truth);
    if (!(e <= 1e-4)) {
        char buf[160];
        std::snprintf(buf, sizeof buf, "%s: max error %.3e above 1e-4", what, e);
        throw std::runtime_error(buf);
    }
}

// GroupNorm -> SiLU as two modules and as the fused GNSiLU, through the
// engine, against float64 truth.
static void test_fused_and_unfused_layers() {
    memory::DeviceArena arena(512u << 20);
    memory::ArenaScope scope(arena);
    const Data d = make_data(2, 16, 64, 64, 4, 101);
    const Truth t = oracle_block(d.x, d, d.dy, d.gamma.data(), d.beta.data(), 1, 0);
    const Shape shape{d.N, d.C, d.H, d.W};
    for (int fused = 0; fused < 2; ++fused) {
        std::unique_ptr<nn::GroupNorm> gn;
        if (fused)
            gn = std::make_unique<nn::GNSiLU>(d.G, d.C);
        else
            gn = std::make_unique<nn::GroupNorm>(d.G, d.C);
        set_params(*gn, d.gamma, d.beta);
        nn::SiLU act;
        auto x = Tensor::from_blob(d.x.data(), shape, true, true);
        auto y = fused ? gn->forward(x) : act.forward(gn->forward(x));
        CHECK(y->grad_fn() != nullptr);
        check_close(fused ? "fused y" : "unfused y", y->to_host(), t.y);
        y->backward(Tensor::from_blob(d.dy.data(), shape, false, true));
        check_close(fused ? "fused dx" : "unfused dx", x->grad()->to_host(), t.dx);
        check_close("dgamma", gn->weight()->grad()->to_host(), t.dg);
        check_close("dbeta", gn->bias()->grad()->to_host(), t.db);
    }
}

// The SOAR residual block x + silu(gn(x)), three in a row: fused
// (GNSiLU with residual) and unfused (GroupNorm, SiLU, add_tensors).
static void test_residual_chain() {
    memory::DeviceArena arena(512u << 20);
    memory::ArenaScope scope(arena);
    const int B = 3;
    Data d = make_data(1, 8, 32, 32, 2, 202);
    std::vector<std::vector<float>> gam(B), bet(B);
    for (int b = 0; b < B; ++b) {
        gam[b].resize(d.C);
        bet[b].resize(d.C);
        orc_fill_uniform(gam[b].data(), d.C, 300 + b, 2, 0.5, 1.5);
        orc_fill_normal(bet[b].data(), d.C, 300 + b, 3, 0.0, 0.1);
    }
    // float64 truth block by block, activations rounded to fp32 between
    // blocks as the device stores them
    std::vector<std::vector<float>> acts{d.x};
    for (int b = 0; b < B; ++b) {
        Truth t = oracle_block(acts.back(), d, d.dy, gam[b].data(), bet[b].data(), 1, 1);
        std::vector<float> nx(t.y.begin(), t.y.end());
        acts.push_back(nx);
    }
    std::vector<float> g = d.dy;
    std::vector<Truth> tb(B);
    for (int b = B - 1; b >= 0; --b) {
        tb[b] = oracle_block(acts[b], d, g, gam[b].data(), bet[b].data(), 1, 1);
        g.assign(tb[b].dx.begin(), tb[b].dx.end());
    }
    const Shape shape{d.C, d.H, d.W};  // the reference's [C,H,W] layout
    for (int fused = 0; fused < 2; ++fused) {
        std::vector<std::unique_ptr<nn::GroupNorm>> gns;
        nn::SiLU act;
        auto x0 = Tensor::from_blob(d.x.data(), shape, true, true);
        TensorPtr h = x0;
        for (int b = 0; b < B; ++b) {
            if (fused)
                gns.push_back(std::make_unique<nn::GNSiLU>(d.G, d.C, kEps, true, true));
            else
                gns.push_back(std::make_unique<nn::GroupNorm>(d.G, d.C));
            set_params(*gns.back(), gam[b], bet[b]);
            h = fused ? gns.back()->forward(h) : nn::add_tensors(h, act.forward(gns.back()->forward(h)));
        }
        std::vector<double> yt(acts.back().begin(), acts.back().end());
        check_close("chain y", h->to_host(), yt);
        h->backward(Tensor::from_blob(d.dy.data(), shape, false, true));
        std::vector<double> dxt(g.begin(), g.end());
        check_close(fused ? "fused chain dx" : "unfused chain dx", x0->grad()->to_host(), dxt);
        for (int b = 0; b < B; ++b) {
            check_close("chain dgamma", gns[b]->weight()->grad()->to_host(), tb[b].dg);
            check_close("chain dbeta", gns[b]->bias()->grad()->to_host(), tb[b].db);
        }
    }
}

// [N,C,H,W] in one call equals the reference's per-sample loop over
// [C,H,W] with parameter gradients accumulated across samples
// (src/engine/trainer.cpp:179-220), and gradients accumulate in place into
// a buffer that keeps its address.
static void test_batch_equals_per_sample_and_accumulates() {
    memory::DeviceArena arena(512u << 20);
    memory::ArenaScope scope(arena);
    const Data d = make_data(3, 8, 32, 48, 4, 303);
    const Truth t = oracle_block(d.x, d, d.dy, d.gamma.data(), d.beta.data(), 1, 0);
    nn::GNSiLU per_sample(d.G, d.C);
    set_params(per_sample, d.gamma, d.beta);
    const int64_t S = d.C * d.H * d.W;
    std::vector<float> dx_all;
    for (int64_t n = 0; n < d.N; ++n) {
        auto xn = Tensor::from_blob(d.x.data() + n * S, {d.C, d.H, d.W}, true, true);
        auto yn = per_sample.forward(xn);
        yn->backward(Tensor::from_blob(d.dy.data() + n * S, {d.C, d.H, d.W}, false, true));
        auto g = xn->grad()->to_host();
        dx_all.insert(dx_all.end(), g.begin(), g.end());
    }
    check_close("per-sample dx", dx_all, t.dx);
    check_close("per-sample dgamma", per_sample.weight()->grad()->to_host(), t.dg);
    check_close("per-sample dbeta", per_sample.bias()->grad()->to_host(), t.db);

    nn::GNSiLU batched(d.G, d.C);
    set_params(batched, d.gamma, d.beta);
    const Shape shape{d.N, d.C, d.H, d.W};
    auto dy = Tensor::from_blob(d.dy.data(), shape, false, true);
    auto x = Tensor::from_blob(d.x.data(), shape, true, true);
    batched.forward(x)->backward(dy);
    check_close("batched dgamma", batched.weight()->grad()->to_host(), t.dg);
    const float* buf = batched.weight()->grad()->cuda_data();
    auto x2 = Tensor::from_blob(d.x.data(), shape, true, true);
    batched.forward(x2)->backward(dy);
    CHECK(batched.weight()->grad()->cuda_data() == buf);
    std::vector<double> twice(t.dg.size());
    for (size_t i = 0; i < twice.size(); ++i) twice[i] = 2.0 * t.dg[i];
    check_close("accumulated dgamma", batched.weight()->grad()->to_host(), twice);
    batched.zero_grad();
    for (float v : batched.weight()->grad()->to_host()) CHECK(v == 0.0f);
}

// Parameters in the static region; per-step activations reuse identical
// offsets after reset_dynamic_allocations (device_slab.cpp:39-56).
static void test_arena_step_reuse() {
    memory::DeviceArena arena(64u << 20);
    memory::ArenaScope scope(arena);
    const Data d = make_data(1, 8, 16, 16, 2, 404);
    nn::GNSiLU m(d.G, d.C);
    set_params(m, d.gamma, d.beta);
    arena.freeze_static_parameters();
    const size_t sb = arena.slab().static_boundary();
    CHECK(sb > 0);
    const float* out_ptr[2] = {nullptr, nullptr};
    std::vector<float> outs[2];
    for (int step = 0; step < 2; ++step) {
        arena.reset_dynamic_allocations();
        CHECK(arena.slab().current_offset() == sb);
        auto x = Tensor::from_blob(d.x.data(), {d.C, d.H, d.W}, true, true);
        auto y = m.forward(x);
        out_ptr[step] = y->cuda_data();
        outs[step] = y->to_host();
    }
    CHECK(out_ptr[0] == out_ptr[1]);
    CHECK(outs[0] == outs[1]);  // bitwise reproducible
    {
        autograd::NoGradGuard ng;
        auto x = Tensor::from_blob(d.x.data(), {d.C, d.H, d.W}, true, true);
        CHECK(m.forward(x)->grad_fn() == nullptr);
    }
    CHECK_THROWS(arena.allocate(128u << 20), OutOfMemory);
}

// The reference-named operator API (cuda_kernels.hpp) on one sample.
static void test_reference_operator_api() {
    memory::DeviceArena arena(64u << 20);
    memory::ArenaScope scope(arena);
    CHECK(hip::kernels::is_cuda_available());
    const Data d = make_data(1, 16, 32, 32, 4, 505);
    const Truth t = oracle_block(d.x, d, d.dy, d.gamma.data(), d.beta.data(), 0, 0);
    const Shape shape{d.C, d.H * d.W};
    auto x = Tensor::from_blob(d.x.data(), shape, false, true);
    auto gm = Tensor::from_blob(d.gamma.data(), {d.C}, false, true);
    auto bt = Tensor::from_blob(d.beta.data(), {d.C}, false, true);
    auto out = Tensor::create(shape, false, true);
    auto mean = Tensor::create({d.G}, false, true), rstd = Tensor::create({d.G}, false, true);
    hip::kernels::group_norm_forward(x->cuda_data(), gm->cuda_data(), bt->cuda_data(),
                                     out->cuda_data(), mean->cuda_data(), rstd->cuda_data(),
                                     d.G, d.C, d.H * d.W, kEps);
    check_close("group_norm_forward", out->to_host(), t.y);
    auto dy = Tensor::from_blob(d.dy.data(), shape, false, true);
    auto gx = Tensor::zeros(shape, false, true);
    auto gw = Tensor::zeros({d.C}, false, true), gb = Tensor::zeros({d.C}, false, true);
    hip::kernels::group_norm_backward(dy->cuda_data(), x->cuda_data(), gm->cuda_data(),
                                      mean->cuda_data(), rstd->cuda_data(), gx->cuda_data(),
                                      gw->cuda_data(), gb->cuda_data(), d.G, d.C, d.H * d.W);
    check_close("group_norm_backward dx", gx->to_host(), t.dx);
    check_close("group_norm_backward dgamma", gw->to_host(), t.dg);
    check_close("group_norm_backward dbeta", gb->to_host(), t.db);
    CHECK_THROWS(hip::kernels::group_norm_forward(x->cuda_data(), nullptr, nullptr,
                                                  out->cuda_data(), mean->cuda_data(),
                                                  rstd->cuda_data(), 3, d.C, d.H * d.W, kEps),
                 InvalidArgument);
}

static std::vector<float> host_copy(const TensorPtr& t) {
    return std::vector<float>(t->data(), t->data() + t->numel());
}

static std::vector<float> to_float(const std::vector<double>& v) {
    return std::vector<float>(v.begin(), v.end());
}

// Conv2d on the device: pointwise (with bias, N = 2), depthwise (k7 and
// k3 stride 2) and general grouped, forward and backward through the
// engine, against float64 truth (layers.cpp:17-372 semantics: dx fresh,
// dW/db accumulated).
static void test_conv2d_layers() {
    memory::DeviceArena arena(256u << 20);
    memory::ArenaScope scope(arena);
    {  // pointwise 16 -> 24
        const int64_t N = 2, Ci = 16, Co = 24, H = 20, W = 30, HW = H * W;
        nn::Conv2d conv(Ci, Co, 1, 1, -1, 1, 1, true);
        CHECK(conv.pointwise() && conv.padding() == 0);
        std::vector<float> x(N * Ci * HW), dy(N * Co * HW), b(Co);
        orc_fill_normal(x.data(), (int64_t)x.size(), 601, 1, 0.0, 1.0);
        orc_fill_normal(dy.data(), (int64_t)dy.size(), 601, 4, 0.0, 1.0);
        orc_fill_uniform(b.data(), Co, 601, 3, -0.5, 0.5);
        for (int64_t c = 0; c < Co; ++c) conv.bias()->data()[c] = b[c];
        const std::vector<float> w = host_copy(conv.weight());
        auto xt = Tensor::from_blob(x.data(), {N, Ci, H, W}, true, true);
        auto y = conv.forward(xt);
        CHECK(y->shape() == (Shape{N, Co, H, W}));
        std::vector<double> yt(N * Co * HW), dxt(N * Ci * HW), dwt(Co * Ci), dbt(Co);
        CHECK(orc_conv1x1_fwd_f64(x.data(), w.data(), b.data(), N, Ci, Co, HW, yt.data()) == 0);
        check_close("pw conv y", y->to_host(), yt);
        y->backward(Tensor::from_blob(dy.data(), {N, Co, H, W}, false, true));
        CHECK(orc_conv1x1_bwd_f64(dy.data(), x.data(), w.data(), N, Ci, Co, HW, dxt.data(),
                                  dwt.data(), dbt.data()) == 0);
        check_close("pw conv dx", xt->grad()->to_host(), dxt);
        check_close("pw conv dW", conv.weight()->grad()->to_host(), dwt);
        check_close("pw conv db", conv.bias()->grad()->to_host(), dbt);
    }
    struct Dw {
        int64_t N, C, H, W, K, S;
    };
    for (const Dw& c : {Dw{1, 8, 40, 50, 7, 1}, Dw{2, 8, 33, 47, 3, 2}}) {
        nn::Conv2d conv(c.C, c.C, c.K, c.S, -1, 1, c.C, true);
        CHECK(conv.depthwise() && conv.padding() == (size_t)(c.K / 2));
        const int64_t pad = c.K / 2;
        const int64_t Ho = (c.H + 2 * pad - c.K) / c.S + 1, Wo = (c.W + 2 * pad - c.K) / c.S + 1;
        std::vector<float> x(c.N * c.C * c.H * c.W), dy(c.N * c.C * Ho * Wo), b(c.C);
        orc_fill_normal(x.data(), (int64_t)x.size(), 602, 1, 0.0, 1.0);
        orc_fill_normal(dy.data(), (int64_t)dy.size(), 602, 4, 0.0, 1.0);
        orc_fill_uniform(b.data(), c.C, 602, 3, -0.5, 0.5);
        for (int64_t i = 0; i < c.C; ++i) conv.bias()->data()[i] = b[i];
        const std::vector<float> w = host_copy(conv.weight());
        auto xt = Tensor::from_blob(x.data(), {c.N, c.C, c.H, c.W}, true, true);
        auto y = conv.forward(xt);
        CHECK(y->shape() == (Shape{c.N, c.C, Ho, Wo}));
        std::vector<double> yt(dy.size()), dxt(x.size()), dwt(c.C * c.K * c.K), dbt(c.C);
        CHECK(orc_dw_fwd_f64(x.data(), w.data(), b.data(), c.N, c.C, c.H, c.W, Ho, Wo, c.K, pad,
                             c.S, 1, yt.data()) == 0);
        check_close("dw conv y", y->to_host(), yt);
        y->backward(Tensor::from_blob(dy.data(), {c.N, c.C, Ho, Wo}, false, true));
        CHECK(orc_dw_bwd_f64(dy.data(), x.data(), w.data(), c.N, c.C, c.H, c.W, Ho, Wo, c.K, pad,
                             c.S, 1, dxt.data(), dwt.data(), dbt.data()) == 0);
        check_close("dw conv dx", xt->grad()->to_host(), dxt);
        check_close("dw conv dW", conv.weight()->grad()->to_host(), dwt);
        check_close("dw conv db", conv.bias()->grad()->to_host(), dbt);
    }
    // a general grouped convolution (groups 2, k3, stride 2, bias) against
    // a direct float64 loop of its definition and of its adjoint
    {
        const int64_t Ci = 4, Co = 6, G = 2, K = 3, S = 2, P = 1, Hh = 9, Ww = 11;
        const int64_t Ho = (Hh + 2 * P - K) / S + 1, Wo = (Ww + 2 * P - K) / S + 1;
        nn::Conv2d general((size_t)Ci, (size_t)Co, (size_t)K, (size_t)S, -1, 1, (size_t)G, true);
        std::vector<float> x(Ci * Hh * Ww), dy(Co * Ho * Wo), b(Co);
        orc_fill_normal(x.data(), x.size(), 31, 1, 0.0, 1.0);
        orc_fill_normal(dy.data(), dy.size(), 31, 2, 0.0, 1.0);
        orc_fill_normal(b.data(), b.size(), 31, 3, 0.0, 0.5);
        std::copy(b.begin(), b.end(), general.bias()->data());
        const std::vector<float> w = host_copy(general.weight());
        auto xt = Tensor::from_blob(x.data(), {Ci, Hh, Ww}, true, true);
        auto y = general.forward(xt);
        CHECK(y->shape() == (Shape{Co, Ho, Wo}));
        const int64_t cig = Ci / G, cog = Co / G;
        std::vector<double> yt(dy.size()), dxt(x.size(), 0.0), dwt(w.size(), 0.0), dbt(Co, 0.0);
        for (int64_t co = 0; co < Co; ++co)
            for (int64_t oy = 0; oy < Ho; ++oy)
                for (int64_t ox = 0; ox < Wo; ++ox) {
                    double acc = b[co];
                    const double g = dy[(co * Ho + oy) * Wo + ox];
                    dbt[co] += g;
                    for (int64_t q = 0; q < cig; ++q)
                        for (int64_t ky = 0; ky < K; ++ky)
                            for (int64_t kx = 0; kx < K; ++kx) {
                                const int64_t iy = oy * S - P + ky, ix = ox * S - P + kx;
                                if (iy < 0 || iy >= Hh || ix < 0 || ix >= Ww) continue;
                                const int64_t ci = (co / cog) * cig + q;
                                const int64_t wi = ((co * cig + q) * K + ky) * K + kx;
                                const int64_t xi = (ci * Hh + iy) * Ww + ix;
                                acc += (double)w[wi] * x[xi];
                                dxt[xi] += (double)w[wi] * g;
                                dwt[wi] += (double)x[xi] * g;
                            }
                    yt[(co * Ho + oy) * Wo + ox] = acc;
                }
        check_close("general conv y", y->to_host(), yt);
        y->backward(Tensor::from_blob(dy.data(), {Co, Ho, Wo}, false, true));
        check_close("general conv dx", xt->grad()->to_host(), dxt);
        check_close("general conv dW", general.weight()->grad()->to_host(), dwt);
        check_close("general conv db", general.bias()->grad()->to_host(), dbt);
    }
}

// CBA: pointwise (one fused call, GroupNorm statistics in the conv
// epilogue) with SiLU, and depthwise k7 without activation (LKR.dw),
// against float64 truth composed block by block (conv, rounded to fp32 as
// stored, then GroupNorm(+SiLU), then the conv backward on the fp32-rounded
// dz).
static void test_cba_blocks() {
    memory::DeviceArena arena(256u << 20);
    memory::ArenaScope scope(arena);
    struct Case {
        int64_t N, c1, c2, H, W, k, g;
        bool act;
    };
    for (const Case& c : {Case{2, 16, 32, 24, 40, 1, 1, true}, Case{1, 8, 8, 30, 36, 7, 8, false}}) {
        nn::CBA cba(c.c1, c.c2, c.k, 1, -1, 1, c.g, c.act);
        const auto names = cba.named_parameters();
        CHECK(names.size() == 3 && names[0].first == "conv.weight" &&
              names[1].first == "norm.bias" && names[2].first == "norm.weight");
        const int64_t G = nn::select_group_count((int)c.c2), HW = c.H * c.W;
        std::vector<float> x(c.N * c.c1 * HW), dy(c.N * c.c2 * HW), gam(c.c2), bet(c.c2);
        orc_fill_normal(x.data(), (int64_t)x.size(), 700 + c.k, 1, 0.0, 1.0);
        orc_fill_normal(dy.data(), (int64_t)dy.size(), 700 + c.k, 4, 0.0, 1e-2);
        orc_fill_uniform(gam.data(), c.c2, 700 + c.k, 2, 0.5, 1.5);
        orc_fill_normal(bet.data(), c.c2, 700 + c.k, 3, 0.0, 0.1);
        for (int64_t i = 0; i < c.c2; ++i) {
            cba.norm()->weight()->data()[i] = gam[i];
            cba.norm()->bias()->data()[i] = bet[i];
        }
        const std::vector<float> w = host_copy(cba.conv()->weight());
        const int64_t pad = c.k / 2;
        std::vector<double> z64(c.N * c.c2 * HW);
        if (c.k == 1)
            CHECK(orc_conv1x1_fwd_f64(x.data(), w.data(), nullptr, c.N, c.c1, c.c2, HW,
                                      z64.data()) == 0);
        else
            CHECK(orc_dw_fwd_f64(x.data(), w.data(), nullptr, c.N, c.c1, c.H, c.W, c.H, c.W, c.k,
                                 pad, 1, 1, z64.data()) == 0);
        const std::vector<float> zf = to_float(z64);
        std::vector<double> yt(zf.size()), mean(c.N * G), rstd(c.N * G), dz(zf.size()),
            dgt(c.c2), dbt(c.c2), dxt(x.size()), dwt(w.size());
        const int s = c.act ? 1 : 0;
        CHECK(orc_gn_silu_fwd_f64(zf.data(), gam.data(), bet.data(), c.N, c.c2, HW, G,
                                  (double)kEps, s, 0, yt.data(), mean.data(), rstd.data()) == 0);
        CHECK(orc_gn_silu_bwd_f64(dy.data(), zf.data(), gam.data(), bet.data(), mean.data(),
                                  rstd.data(), c.N, c.c2, HW, G, s, 0, dz.data(), dgt.data(),
                                  dbt.data()) == 0);
        const std::vector<float> dzf = to_float(dz);
        if (c.k == 1)
            CHECK(orc_conv1x1_bwd_f64(dzf.data(), x.data(), w.data(), c.N, c.c1, c.c2, HW,
                                      dxt.data(), dwt.data(), nullptr) == 0);
        else
            CHECK(orc_dw_bwd_f64(dzf.data(), x.data(), w.data(), c.N, c.c1, c.H, c.W, c.H, c.W,
                                 c.k, pad, 1, 1, dxt.data(), dwt.data(), nullptr) == 0);
        auto xt = Tensor::from_blob(x.data(), {c.N, c.c1, c.H, c.W}, true, true);
        auto y = cba.forward(xt);
        check_close(c.k == 1 ? "cba pw y" : "cba dw y", y->to_host(), yt);
        y->backward(Tensor::from_blob(dy.data(), {c.N, c.c2, c.H, c.W}, false, true));
        check_close("cba dx", xt->grad()->to_host(), dxt);
        check_close("cba conv dW", cba.conv()->weight()->grad()->to_host(), dwt);
        check_close("cba dgamma", cba.norm()->weight()->grad()->to_host(), dgt);
        check_close("cba dbeta", cba.norm()->bias()->grad()->to_host(), dbt);
    }
}

// Trainer::train_step semantics (trainer.cpp:110-245) on the Nano model at
// 32 x 32: a [2,1,H,W] batch, two forward_backward calls at scale 1/2
// followed by clip + AdamW + zero_grad, and two train_step calls with
// accumulate_grad_batches = 2 (the first one accumulating) run the same
// kernels in the same order, so the three models end bitwise equal.
static void test_trainer_batch_and_accumulation() {
    const int64_t H = 32, HW = H * H;
    std::vector<float> img(2 * HW), msk(2 * HW);
    orc_fill_normal(img.data(), 2 * HW, 91, 1, 0.5, 0.25);
    for (int64_t b = 0; b < 2; ++b)
        for (int64_t y = 0; y < H; ++y)
            for (int64_t x = 0; x < H; ++x) {
                const double dy = (double)y - H / 2.0, dx = (double)x - H / (3.0 + b);
                msk[b * HW + y * H + x] = dy * dy + dx * dx < (H / 3.0) * (H / 3.0) ? 1.0f : 0.0f;
            }
    struct Run {
        std::unique_ptr<memory::DeviceArena> params, acts;
        std::shared_ptr<nn::SOARModel> model;
        std::unique_ptr<engine::Trainer> trainer;
    };
    auto build = [](size_t accumulate) {
        Run r;
        r.params = std::make_unique<memory::DeviceArena>(size_t(96) << 20, 256);
        r.acts = std::make_unique<memory::DeviceArena>(size_t(256) << 20, 256);
        nn::set_init_seed(12345);
        r.model = std::make_shared<nn::SOARModel>(1, 1, nn::ModelVariant::Nano);
        memory::ArenaScope scope(*r.params);
        r.model->to_device();
        optim::AdamWOptions o;
        o.lr = 1e-3f;
        r.trainer = std::make_unique<engine::Trainer>(
            r.model, losses::CompositeLoss(0.5f, 0.5f),
            std::make_unique<optim::AdamW>(r.model->parameters(), o), accumulate);
        return r;
    };
    Run a = build(1), b = build(1), c = build(2);
    {
        memory::ArenaScope scope(*a.acts);
        a.trainer->train_step(Tensor::from_blob(img.data(), {2, 1, H, H}, false, true),
                              Tensor::from_blob(msk.data(), {2, 1, H, H}, false, true));
    }
    {
        memory::ArenaScope scope(*b.acts);
        for (int64_t s = 0; s < 2; ++s)
            b.trainer->forward_backward(
                Tensor::from_blob(img.data() + s * HW, {1, H, H}, false, true),
                Tensor::from_blob(msk.data() + s * HW, {1, H, H}, false, true), 0.5f);
        b.trainer->optimizer().clip_grad_norm(b.trainer->grad_clip());
        b.trainer->optimizer().step();
        b.trainer->optimizer().zero_grad();
    }
    {
        memory::ArenaScope scope(*c.acts);
        for (int64_t s = 0; s < 2; ++s)
            c.trainer->train_step(
                Tensor::from_blob(img.data() + s * HW, {1, 1, H, H}, false, true),
                Tensor::from_blob(msk.data() + s * HW, {1, 1, H, H}, false, true), s == 0);
    }
    const auto pa = a.model->named_parameters(), pb = b.model->named_parameters(),
               pc = c.model->named_parameters();
    CHECK(pa.size() == pb.size() && pa.size() == pc.size());
    for (size_t i = 0; i < pa.size(); ++i) {
        const auto va = pa[i].second->to_host(), vb = pb[i].second->to_host(),
                   vc = pc[i].second->to_host();
        CHECK(va == vb);
        CHECK(va == vc);
    }
    // the step moved the weights, and the gradients are zero again
    nn::set_init_seed(12345);
    nn::SOARModel fresh(1, 1, nn::ModelVariant::Nano);
    const auto pf = fresh.named_parameters();
    size_t moved = 0;
    for (size_t i = 0; i < pa.size(); ++i) {
        if (pa[i].second->to_host() != pf[i].second->to_host()) ++moved;
        for (float g : pa[i].second->grad()->to_host()) CHECK(g == 0.0f);
    }
    CHECK(moved > pa.size() / 2);
}

int main() {
    std::printf("=== host layer: device tests ===\n");
    int fails = 0;
    fails += run_test("fused_and_unfused_layers", test_fused_and_unfused_layers);
    fails += run_test("residual_chain", test_residual_chain);
    fails += run_test("batch_equals_per_sample_and_accumulates",
                      test_batch_equals_per_sample_and_accumulates);
    fails += run_test("arena_step_reuse", test_arena_step_reuse);
    fails += run_test("reference_operator_api", test_reference_operator_api);
    fails += run_test("conv2d_layers", test_conv2d_layers);
    fails += run_test("cba_blocks", test_cba_blocks);
    fails += run_test("trainer_batch_and_accumulation", test_trainer_batch_and_accumulation);
    std::printf("%s (%d failed)\n", fails ? "FAILED" : "ALL PASSED", fails);
    return fails ? 1 : 0;
}
