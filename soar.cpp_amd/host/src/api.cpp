// The model-level C-ABI of include/soar_api.h: a handle around SOARModel,
// Trainer and Predictor with two device arenas (parameters + optimizer
// state; per-call activations).  Mirrors src/api/c_api.cpp:11-154 of the
// reference: exceptions become -1 / NULL; the message is kept for
// soar_api_last_error().
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <tuple>

#include "soar/autograd.hpp"
#include "soar/engine.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar/model.hpp"
#include "soar_api.h"
#include "soar_gn.h"

namespace {

thread_local std::string g_api_err;

using soar::TensorPtr;
using soar::memory::ArenaScope;
using soar::memory::DeviceArena;

constexpr size_t kAlign = 256;
constexpr size_t kMinActivationBytes = size_t(64) << 20;

size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw soar::DeviceError(std::string(what) + ": " + hipGetErrorString(e));
    }
}

// A training step captured into a graph for one image shape; valid while
// the activation arena it allocated from keeps its base address.
struct StepGraph {
    hipGraphExec_t exec = nullptr;
    void* acts_base = nullptr;
};

struct SoarModelHandle {
    std::unique_ptr<DeviceArena> params;
    std::unique_ptr<DeviceArena> acts;
    size_t act_peak = 0;
    std::shared_ptr<soar::nn::SOARModel> model;
    std::unique_ptr<soar::engine::Trainer> trainer;
    soar::engine::StepMetrics last;
    std::vector<std::pair<std::string, TensorPtr>> named;
    // ---- soar_train_step on the device, captured and replayed -----------
    hipStream_t stream = nullptr;
    bool graph_mode = true;
    double* dev_sums = nullptr;     // loss sums (device, params arena)
    float* dev_scalars = nullptr;   // AdamW lr, step size, sqrt(bc2) (device)
    float* pin_scalars = nullptr;   // the same, pinned host staging
    double* pin_out = nullptr;      // read-back: 4 loss sums + the squared norm
    float* pin_img = nullptr;       // pinned staging of the image and mask
    float* pin_msk = nullptr;
    size_t pin_elems = 0;           // capacity of each, floats
    std::map<std::tuple<int, int, int>, StepGraph> graphs;
    std::map<std::tuple<int, int, int>, int> seen;  // eager steps run per shape
    // ---- soar_predict the same way: graphs per (C, H, W, threshold bits) --
    float* pin_probs = nullptr;     // pinned read-back of the probabilities
    uint8_t* pin_mask = nullptr;    // and of the mask
    size_t pin_out_elems = 0;
    std::map<std::tuple<int, int, int, uint32_t>, StepGraph> pgraphs;
    std::map<std::tuple<int, int, int, uint32_t>, int> pseen;

    ~SoarModelHandle() {
        for (auto& [k, g] : graphs)
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
        for (auto& [k, g] : pgraphs)
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
        for (void* p : {(void*)pin_scalars, (void*)pin_out, (void*)pin_img, (void*)pin_msk,
                        (void*)pin_probs, (void*)pin_mask})
            if (p) (void)hipHostFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

SoarModelHandle* H(void* h) { return static_cast<SoarModelHandle*>(h); }

// Activation bytes for one training step on an H x W image: about 2 KiB
// per input pixel covers the Nano..Large widths at the sizes tried; a
// step that needs more grows the arena and runs again.
size_t activation_estimate(int64_t h, int64_t w) {
    const size_t px = (size_t)std::max<int64_t>(h, 32) * (size_t)std::max<int64_t>(w, 32);
    return std::max(kMinActivationBytes, align_up(px * 2048));
}

void drop_graphs(SoarModelHandle* s) {
    for (auto& [k, g] : s->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    s->graphs.clear();
    for (auto& [k, g] : s->pgraphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    s->pgraphs.clear();
}

void ensure_acts(SoarModelHandle* s, size_t need) {
    if (s->acts && s->acts->slab().total_capacity() >= need) return;
    // the graphs point into the arena being replaced (the stream is idle
    // at every C-ABI entry: each call ends with a synchronisation)
    drop_graphs(s);
    s->acts.reset();
    s->acts = std::make_unique<DeviceArena>(need, kAlign);
}

// Runs fn() with the activation arena reset and current; on OutOfMemory
// the arena doubles and fn runs again (at most four times).  `undo` is
// called before a retry (e.g. to clear partially accumulated gradients).
template <typename F, typename U>
void with_acts(SoarModelHandle* s, int64_t h, int64_t w, F&& fn, U&& undo) {
    ensure_acts(s, activation_estimate(h, w));
    for (int attempt = 0;; ++attempt) {
        try {
            ArenaScope scope(*s->acts);
            s->acts->reset_dynamic_allocations();
            fn();
            s->act_peak = std::max(s->act_peak, s->acts->slab().current_offset());
            return;
        } catch (const soar::OutOfMemory&) {
            // weight-gradient finishes of the abandoned attempt read its
            // arena, freed below (run_backward drops them too)
            soar_weight_grad_discard();
            if (attempt >= 3) throw;
            undo();
            ensure_acts(s, s->acts->slab().total_capacity() * 2);
        }
    }
}

// The RLE string into the caller's buffer, truncated to max_len - 1
// characters and NUL-terminated (the bytes past the NUL are left as they
// were: a zero fill of the whole buffer cost milliseconds per image).
void copy_rle(const std::string& rle, char* out, size_t max_len) {
    const size_t k = std::min(rle.size(), max_len - 1);
    std::memcpy(out, rle.data(), k);
    out[k] = '\0';
}

void check_image(int c, int h, int w) {
    if (c <= 0 || h <= 0 || w <= 0)
        throw soar::InvalidArgument("image dimensions must be positive");
}

float* metrics_out(const soar::engine::StepMetrics& m, float* out) {
    if (out) {
        out[0] = m.loss;
        out[1] = m.bce_loss;
        out[2] = m.dice_loss;
        out[3] = m.dice_score;
        out[4] = m.iou_score;
        out[5] = m.lr;
        out[6] = m.grad_norm;
    }
    return out;
}

template <typename F>
int guarded(F&& fn) {
    try {
        fn();
        g_api_err.clear();
        return 0;
    } catch (const std::exception& e) {
        g_api_err = e.what();
        return -1;
    } catch (...) {
        g_api_err = "unknown error";
        return -1;
    }
}

void* create(int in_channels, int num_classes, int variant, bool seeded, uint64_t seed) {
    try {
        if (in_channels <= 0 || num_classes <= 0 || variant < 0 || variant > 4)
            throw soar::InvalidArgument("soar_create_model: invalid channels or variant");
        auto h = std::make_unique<SoarModelHandle>();
        if (seeded) soar::nn::set_init_seed(seed);
        h->model = std::make_shared<soar::nn::SOARModel>(
            (size_t)in_channels, (size_t)num_classes,
            static_cast<soar::nn::ModelVariant>(variant));
        h->named = h->model->named_parameters();
        // parameter, gradient, two moments per tensor, plus the optimizer's
        // tables and the norm workspace
        size_t bytes = size_t(1) << 20;
        for (auto& [n, p] : h->named) bytes += 4 * align_up(p->bytes()) ;
        bytes += align_up(5 * h->named.size() * sizeof(void*)) + (size_t(64) << 10);
        h->params = std::make_unique<DeviceArena>(bytes, kAlign);
        {
            ArenaScope scope(*h->params);
            h->model->to_device();
            soar::optim::AdamWOptions opts;
            opts.lr = 1e-3f;
            auto opt = std::make_unique<soar::optim::AdamW>(h->model->parameters(), opts);
            h->trainer = std::make_unique<soar::engine::Trainer>(
                h->model, soar::losses::CompositeLoss(0.5f, 0.5f), std::move(opt));
            // the 4 loss sums, then the squared gradient norm: one read-back
            h->dev_sums = static_cast<double*>(
                h->params->allocate(5 * sizeof(double), {}, "loss_sums"));
            h->trainer->optimizer().set_norm_sq_buffer(h->dev_sums + 4);
            h->dev_scalars = static_cast<float*>(
                h->params->allocate(4 * sizeof(float), {}, "adamw_scalars"));
        }
        hip_check(hipStreamCreate(&h->stream), "hipStreamCreate");
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&h->pin_scalars), 4 * sizeof(float)),
                  "hipHostMalloc");
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&h->pin_out), 8 * sizeof(double)),
                  "hipHostMalloc");
        if (const char* g = std::getenv("SOAR_TRAIN_GRAPH")) h->graph_mode = std::atoi(g) != 0;
        g_api_err.clear();
        return h.release();
    } catch (const std::exception& e) {
        g_api_err = e.what();
        return nullptr;
    } catch (...) {
        g_api_err = "unknown error";
        return nullptr;
    }
}

TensorPtr host_image(const float* data, int64_t c, int64_t h, int64_t w) {
    return soar::Tensor::from_blob(data, {c, h, w}, false, true);
}

// Pinned staging for the image and mask of a step.
void ensure_pinned(SoarModelHandle* s, size_t elems) {
    if (s->pin_elems >= elems) return;
    drop_graphs(s);  // their uploads read the old staging
    for (float** p : {&s->pin_img, &s->pin_msk}) {
        if (*p) hip_check(hipHostFree(*p), "hipHostFree");
        *p = nullptr;
    }
    s->pin_elems = 0;
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&s->pin_img), elems * sizeof(float)),
              "hipHostMalloc");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&s->pin_msk), elems * sizeof(float)),
              "hipHostMalloc");
    s->pin_elems = elems;
}

// Pinned read-back buffers of predict's probabilities and mask.
void ensure_pinned_out(SoarModelHandle* s, size_t elems) {
    if (s->pin_out_elems >= elems) return;
    drop_graphs(s);  // their copies write the old buffers
    if (s->pin_probs) hip_check(hipHostFree(s->pin_probs), "hipHostFree");
    if (s->pin_mask) hip_check(hipHostFree(s->pin_mask), "hipHostFree");
    s->pin_probs = nullptr;
    s->pin_mask = nullptr;
    s->pin_out_elems = 0;
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&s->pin_probs), elems * sizeof(float)),
              "hipHostMalloc");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&s->pin_mask), elems), "hipHostMalloc");
    s->pin_out_elems = elems;
}

// The device work of one training step from the pinned staging, on the
// handle's stream (recorded into a graph while that stream is capturing).
void device_step(SoarModelHandle* s, int64_t c, int64_t h, int64_t w) {
    TensorPtr img = soar::Tensor::create({c, h, w}, false, true);
    TensorPtr msk = soar::Tensor::create({1, h, w}, false, true);
    soar::hip::kernels::check(soar_memcpy_async(img->cuda_data(), s->pin_img,
                                                (size_t)(c * h * w) * sizeof(float), 0,
                                                s->stream),
                              "image upload");
    soar::hip::kernels::check(soar_memcpy_async(msk->cuda_data(), s->pin_msk,
                                                (size_t)(h * w) * sizeof(float), 0, s->stream),
                              "mask upload");
    s->trainer->train_step_device(img, msk, s->dev_sums, s->pin_scalars, s->dev_scalars);
}

// Runs `work` (one call's device work on the handle's stream) as a replay
// of the graph held for `key`, else directly, captured (and then launched)
// from the second call of a key on.  `before_replay` does the host part a
// replay still needs (the graph holds device work only); `rollback` undoes
// the host effects of a capture that is thrown away; `undo` is with_acts'
// reset before a retry with a larger arena.  A capture that fails is
// discarded and the call runs uncaptured; graphs stay off for the handle
// from then on.
template <typename K, typename W, typename B, typename R, typename U>
void run_graphed(SoarModelHandle* s, std::map<K, StepGraph>& graphs, std::map<K, int>& seen,
                 const K& key, int h, int w, W&& work, B&& before_replay, R&& rollback,
                 U&& undo) {
    auto it = graphs.find(key);
    if (s->graph_mode && it != graphs.end() && s->acts &&
        it->second.acts_base == s->acts->base()) {
        before_replay();
        hip_check(hipGraphLaunch(it->second.exec, s->stream), "hipGraphLaunch");
        return;
    }
    const bool capture = s->graph_mode && seen[key] > 0;
    with_acts(
        s, h, w,
        [&] {
            if (!capture) {
                work();
                return;
            }
            hip_check(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal),
                      "hipStreamBeginCapture");
            hipGraph_t graph = nullptr;
            auto uncaptured = [&] {
                (void)hipGetLastError();
                rollback();
                s->graph_mode = false;
                s->acts->reset_dynamic_allocations();
                work();
            };
            try {
                work();
            } catch (const soar::OutOfMemory&) {
                (void)hipStreamEndCapture(s->stream, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                rollback();
                throw;  // with_acts grows the arena and runs again
            } catch (...) {
                (void)hipStreamEndCapture(s->stream, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                uncaptured();
                return;
            }
            hipGraphExec_t exec = nullptr;
            hipError_t e = hipStreamEndCapture(s->stream, &graph);
            if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (graph) (void)hipGraphDestroy(graph);
            if (e != hipSuccess) {
                uncaptured();
                return;
            }
            hip_check(hipGraphLaunch(exec, s->stream), "hipGraphLaunch");
            StepGraph& g = graphs[key];
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            g.exec = exec;
            g.acts_base = s->acts->base();
        },
        undo);
    seen[key] += 1;
}

void run_train_step(SoarModelHandle* s, int c, int h, int w) {
    auto& opt = s->trainer->optimizer();
    const int64_t step0 = opt.step_count();
    run_graphed(
        s, s->graphs, s->seen, std::make_tuple(c, h, w), h, w,
        [&] { device_step(s, c, h, w); }, [&] { opt.next_scalars(s->pin_scalars); },
        [&] { opt.set_step_count(step0); }, [&] { opt.zero_grad(); });
}

// The device work of one prediction from the pinned image: probabilities
// and mask into arena buffers, then copied into the pinned read-back.
void device_predict(SoarModelHandle* s, int64_t c, int64_t h, int64_t w, float threshold) {
    TensorPtr img = soar::Tensor::create({c, h, w}, false, true);
    soar::hip::kernels::check(soar_memcpy_async(img->cuda_data(), s->pin_img,
                                                (size_t)(c * h * w) * sizeof(float), 0,
                                                s->stream),
                              "image upload");
    const size_t n = (size_t)(h * w);
    auto* probs = static_cast<float*>(s->acts->allocate(n * sizeof(float), {}, "probs"));
    auto* mask = static_cast<uint8_t*>(s->acts->allocate(n, {}, "mask"));
    soar::engine::Predictor p(s->model, threshold);
    const auto [H, W] = p.predict_device(img, probs, mask);
    if ((size_t)(H * W) != n) throw soar::ShapeError("predict: logits are not H x W");
    soar::hip::kernels::check(
        soar_memcpy_async(s->pin_probs, probs, n * sizeof(float), 1, s->stream),
        "probabilities read-back");
    soar::hip::kernels::check(soar_memcpy_async(s->pin_mask, mask, n, 1, s->stream),
                              "mask read-back");
}

void run_predict(SoarModelHandle* s, int c, int h, int w, float threshold) {
    uint32_t tb = 0;
    std::memcpy(&tb, &threshold, sizeof tb);
    run_graphed(
        s, s->pgraphs, s->pseen, std::make_tuple(c, h, w, tb), h, w,
        [&] { device_predict(s, c, h, w, threshold); }, [] {}, [] {}, [] {});
}

}  // namespace

extern "C" {

SOAR_API const char* soar_api_last_error(void) { return g_api_err.c_str(); }

SOAR_API void* soar_create_model(int in_channels, int num_classes, int variant) {
    return create(in_channels, num_classes, variant, false, 0);
}

SOAR_API void* soar_create_model_seeded(int in_channels, int num_classes, int variant,
                                        uint64_t seed) {
    return create(in_channels, num_classes, variant, true, seed);
}

SOAR_API void soar_destroy_model(void* handle) {
    if (!handle) return;
    auto* s = H(handle);
    // the model and optimizer first: their tensors point into the arenas
    s->trainer.reset();
    s->named.clear();
    s->model.reset();
    delete s;
}

SOAR_API size_t soar_get_parameter_count(void* handle) {
    return handle ? H(handle)->model->parameter_count() : 0;
}

SOAR_API int soar_save_weights(void* handle, const char* path) {
    if (!handle || !path) return -1;
    return guarded([&] { H(handle)->model->save_weights(path); });
}

SOAR_API int soar_load_weights(void* handle, const char* path) {
    if (!handle || !path) return -1;
    return guarded([&] { H(handle)->model->load_weights(path); });
}

SOAR_API int soar_train_step(void* handle, const float* image_data, const float* mask_data,
                             int channels, int height, int width, float learning_rate,
                             float* out_loss, float* out_dice, float* out_iou) {
    if (!handle || !image_data || !mask_data) return -1;
    auto* s = H(handle);
    return guarded([&] {
        check_image(channels, height, width);
        s->trainer->optimizer().set_lr(learning_rate);
        const size_t px = (size_t)height * (size_t)width;
        ensure_pinned(s, (size_t)channels * px);
        std::memcpy(s->pin_img, image_data, (size_t)channels * px * sizeof(float));
        std::memcpy(s->pin_msk, mask_data, px * sizeof(float));
        {
            soar::exec::StreamScope scope(s->stream);
            run_train_step(s, channels, height, width);
        }
        // the loss sums and the squared norm lie together (dev_sums[0..4])
        soar::hip::kernels::check(
            soar_memcpy_async(s->pin_out, s->dev_sums, 5 * sizeof(double), 1, s->stream),
            "loss and norm read-back");
        hip_check(hipStreamSynchronize(s->stream), "hipStreamSynchronize");
        s->last = s->trainer->device_step_metrics(s->pin_out, s->pin_out[4], px);
        if (out_loss) *out_loss = s->last.loss;
        if (out_dice) *out_dice = s->last.dice_score;
        if (out_iou) *out_iou = s->last.iou_score;
    });
}

SOAR_API int soar_predict(void* handle, const float* image_data, int channels, int height,
                          int width, float threshold, float* out_probs, uint8_t* out_mask,
                          char* out_rle, size_t max_rle_len) {
    if (!handle || !image_data) return -1;
    auto* s = H(handle);
    return guarded([&] {
        check_image(channels, height, width);
        const size_t n = (size_t)height * (size_t)width;
        ensure_pinned(s, (size_t)channels * n);
        ensure_pinned_out(s, n);
        std::memcpy(s->pin_img, image_data, (size_t)channels * n * sizeof(float));
        {
            soar::exec::StreamScope scope(s->stream);
            run_predict(s, channels, height, width, threshold);
        }
        hip_check(hipStreamSynchronize(s->stream), "hipStreamSynchronize");
        if (out_probs) std::memcpy(out_probs, s->pin_probs, n * sizeof(float));
        if (out_mask) std::memcpy(out_mask, s->pin_mask, n);
        if (out_rle && max_rle_len > 0)
            copy_rle(soar::engine::Predictor::encode_rle(s->pin_mask, (size_t)height,
                                                         (size_t)width),
                     out_rle, max_rle_len);
    });
}

SOAR_API int soar_encode_rle(const uint8_t* mask, size_t height, size_t width, char* out_rle,
                             size_t max_rle_len) {
    if (!mask || !out_rle || max_rle_len == 0) return -1;
    return guarded([&] {
        copy_rle(soar::engine::Predictor::encode_rle(mask, height, width), out_rle, max_rle_len);
    });
}

SOAR_API int soar_model_num_tensors(void* handle) {
    return handle ? (int)H(handle)->named.size() : -1;
}

SOAR_API int soar_model_tensor_info(void* handle, int index, char* name, size_t name_len,
                                    int* ndim, int64_t shape[4]) {
    if (!handle) return -1;
    auto* s = H(handle);
    if (index < 0 || (size_t)index >= s->named.size()) return -1;
    const auto& [n, p] = s->named[(size_t)index];
    if (name && name_len > 0) {
        std::strncpy(name, n.c_str(), name_len - 1);
        name[name_len - 1] = '\0';
    }
    if (ndim) *ndim = (int)p->ndim();
    if (shape)
        for (int d = 0; d < 4; ++d) shape[d] = d < p->ndim() ? p->dim(d) : 1;
    return 0;
}

SOAR_API int soar_model_read_tensor(void* handle, int index, int what, float* out) {
    if (!handle || !out || (what != 0 && what != 1)) return -1;
    auto* s = H(handle);
    if (index < 0 || (size_t)index >= s->named.size()) return -1;
    return guarded([&] {
        const TensorPtr& p = s->named[(size_t)index].second;
        const TensorPtr t = what == 0 ? p : p->grad();
        if (!t) throw soar::InvalidArgument("tensor has no gradient");
        const std::vector<float> v = t->to_host();
        std::memcpy(out, v.data(), v.size() * sizeof(float));
    });
}

SOAR_API int soar_model_forward_backward(void* handle, const float* image_data,
                                         const float* mask_data, int channels, int height,
                                         int width, float* out_metrics) {
    if (!handle || !image_data || !mask_data) return -1;
    auto* s = H(handle);
    return guarded([&] {
        check_image(channels, height, width);
        soar::engine::StepMetrics m;
        with_acts(
            s, height, width,
            [&] {
                s->trainer->optimizer().zero_grad();
                s->model->train(true);
                TensorPtr img = host_image(image_data, channels, height, width);
                TensorPtr msk = host_image(mask_data, 1, height, width);
                m = s->trainer->forward_backward(img, msk, 1.0f);
            },
            [&] { s->trainer->optimizer().zero_grad(); });
        metrics_out(m, out_metrics);
    });
}

SOAR_API int soar_model_set_graph_mode(void* handle, int on) {
    if (!handle) return -1;
    auto* s = H(handle);
    return guarded([&] {
        s->graph_mode = on != 0;
        if (!on) drop_graphs(s);
    });
}

SOAR_API int soar_model_graph_info(void* handle, int* graph_mode, int* graphs_held) {
    if (!handle) return -1;
    auto* s = H(handle);
    if (graph_mode) *graph_mode = s->graph_mode ? 1 : 0;
    if (graphs_held) *graphs_held = (int)(s->graphs.size() + s->pgraphs.size());
    return 0;
}

SOAR_API int soar_model_zero_grad(void* handle) {
    if (!handle) return -1;
    return guarded([&] { H(handle)->trainer->optimizer().zero_grad(); });
}

SOAR_API int soar_model_last_metrics(void* handle, float* out_metrics) {
    if (!handle || !out_metrics) return -1;
    metrics_out(H(handle)->last, out_metrics);
    return 0;
}

SOAR_API int soar_model_forward(void* handle, const float* image_data, int channels, int height,
                                int width, float* out_logits) {
    if (!handle || !image_data || !out_logits) return -1;
    auto* s = H(handle);
    return guarded([&] {
        check_image(channels, height, width);
        with_acts(
            s, height, width,
            [&] {
                soar::autograd::NoGradGuard guard;
                s->model->eval();
                TensorPtr out = s->model->forward(host_image(image_data, channels, height, width));
                const std::vector<float> v = out->to_host();
                std::memcpy(out_logits, v.data(), v.size() * sizeof(float));
            },
            [] {});
    });
}

SOAR_API int soar_model_memory_info(void* handle, size_t* param_bytes,
                                    size_t* activation_capacity, size_t* activation_peak) {
    if (!handle) return -1;
    auto* s = H(handle);
    if (param_bytes) *param_bytes = s->params->slab().current_offset();
    if (activation_capacity) *activation_capacity = s->acts ? s->acts->slab().total_capacity() : 0;
    if (activation_peak) *activation_peak = s->act_peak;
    return 0;
}

}  // extern "C"
