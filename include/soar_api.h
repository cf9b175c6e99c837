/*
 * soar_api.h - the model-level C-ABI (exported by libsoar_host.so): create
 * a SOAR segmentation model on the MI355X, train it one image at a time,
 * predict, save and load .soar weights.  Same functions, arguments and
 * return convention as the reference's include/soar/api/c_api.h:17-45
 * (src/api/c_api.cpp:11-154): 0 on success, -1 on any failure (NULL from
 * soar_create_model).  Image and mask pointers are HOST pointers: fp32
 * [C][H][W] images and [1][H][W] masks, copied to the device per call.
 *
 * A handle holds the model's parameters, gradients and AdamW moments in
 * one device arena and the activations of a step in a second arena that
 * is reset at the start of every call (and grown when a larger image needs
 * more).  One handle must not be used by two threads at once.
 *
 * Entry points marked "extension" have no counterpart in the reference:
 * they expose what its C++ API exposes (the parameters, the step's
 * metrics, the seed of the initialisation) to callers that only have the
 * C boundary.
 */
#ifndef SOAR_API_H
#define SOAR_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SOAR_API
#define SOAR_API __attribute__((visibility("default")))
#endif

/* variant: 0 Nano, 1 Small, 2 Medium, 3 Large, 4 XLarge.  CompositeLoss
 * (bce 0.5, dice 0.5, pos_weight 3) and AdamW (lr 1e-3, betas 0.9/0.999,
 * eps 1e-8, weight decay 1e-2), gradient clip 2.0, as c_api.cpp:19-36.
 * Replaces: soar_create_model (c_api.h:17). */
SOAR_API void* soar_create_model(int in_channels, int num_classes, int variant);
/* Extension: the same with the Conv2d initialisation sequence seeded, so
 * two models created with one seed start identical. */
SOAR_API void* soar_create_model_seeded(int in_channels, int num_classes,
                                        int variant, uint64_t seed);
/* Replaces: soar_destroy_model (c_api.h:18). */
SOAR_API void soar_destroy_model(void* handle);
/* Total number of parameter values.  Replaces: soar_get_parameter_count
 * (c_api.h:19). */
SOAR_API size_t soar_get_parameter_count(void* handle);

/* .soar files (magic "SOAR", version 1; see SOARModel::save_weights).
 * Replaces: soar_save_weights / soar_load_weights (c_api.h:21-22). */
SOAR_API int soar_save_weights(void* handle, const char* path);
SOAR_API int soar_load_weights(void* handle, const char* path);

/* One training step on one image: forward, Dice+BCE loss, backward, clip,
 * AdamW step with learning_rate, zero_grad.  out_* may be NULL.
 * The step runs on the handle's own stream with the loss sums, the clip
 * decision and AdamW's bias corrections on the device; from the second
 * step of an image shape on it is captured into a HIP graph and replayed
 * (one graph per shape; soar_model_set_graph_mode).  Results are the same
 * bits with or without the graph.
 * Replaces: soar_train_step (c_api.h:24-32). */
SOAR_API int soar_train_step(void* handle, const float* image_data,
                             const float* mask_data, int channels, int height,
                             int width, float learning_rate, float* out_loss,
                             float* out_dice, float* out_iou);

/* Inference on one image: out_probs [H*W] sigmoid probabilities, out_mask
 * [H*W] 0/1 (prob >= threshold), out_rle the column-major RLE string
 * (truncated to max_rle_len - 1 characters).  Any output may be NULL.
 * The device work runs on the handle's stream through pinned staging,
 * replayed as a HIP graph from the second call of an image shape and
 * threshold on (soar_model_set_graph_mode); results are the same bits.
 * Replaces: soar_predict (c_api.h:34-41). */
SOAR_API int soar_predict(void* handle, const float* image_data, int channels,
                          int height, int width, float threshold,
                          float* out_probs, uint8_t* out_mask, char* out_rle,
                          size_t max_rle_len);

/* Column-major, 1-indexed "start length" runs of the non-zero pixels of a
 * row-major mask.  Replaces: soar_encode_rle (c_api.h:42-45). */
SOAR_API int soar_encode_rle(const uint8_t* mask, size_t height, size_t width,
                             char* out_rle, size_t max_rle_len);

/* ---- extensions ---------------------------------------------------------- */

/* Message of the last failing call of this API on this thread ("" if
 * none). */
SOAR_API const char* soar_api_last_error(void);

/* Number of parameter tensors, and tensor i's name (NUL-terminated, at
 * most name_len - 1 chars), rank and shape, in named_parameters() order. */
SOAR_API int soar_model_num_tensors(void* handle);
SOAR_API int soar_model_tensor_info(void* handle, int index, char* name,
                                    size_t name_len, int* ndim,
                                    int64_t shape[4]);
/* Copies tensor i's values (what = 0) or its current gradient (what = 1)
 * to host memory (numel floats). */
SOAR_API int soar_model_read_tensor(void* handle, int index, int what,
                                    float* out);

/* Forward, loss and backward of one image with no optimizer step: the
 * gradients of the parameters become those of this image's loss (they
 * are zeroed first).  out_metrics (may be NULL) receives 7 floats: loss,
 * bce, dice loss, dice score, iou score, lr, 0. */
SOAR_API int soar_model_forward_backward(void* handle, const float* image_data,
                                         const float* mask_data, int channels,
                                         int height, int width,
                                         float* out_metrics);
/* Zeroes every parameter gradient (what the reference's Trainer does
 * after each optimizer step). */
SOAR_API int soar_model_zero_grad(void* handle);
/* on != 0 (the default, or SOAR_TRAIN_GRAPH=0 in the environment at
 * creation for off): soar_train_step captures and replays its device work
 * as a HIP graph per image shape, and soar_predict per image shape and
 * threshold.  Off drops the graphs held.  No counterpart in the reference
 * (its calls are eager). */
SOAR_API int soar_model_set_graph_mode(void* handle, int on);
/* Whether graph mode is on (it turns itself off when a capture fails) and
 * how many training-step and predict graphs the handle holds (either may
 * be NULL). */
SOAR_API int soar_model_graph_info(void* handle, int* graph_mode,
                                   int* graphs_held);
/* The 7 metrics of the last soar_train_step (the last entry is the global
 * gradient norm before clipping). */
SOAR_API int soar_model_last_metrics(void* handle, float* out_metrics);
/* Logits [num_classes][H][W] of one image (no-grad forward). */
SOAR_API int soar_model_forward(void* handle, const float* image_data,
                                int channels, int height, int width,
                                float* out_logits);
/* Device bytes of the parameter arena, the activation arena's capacity
 * and the most any call has used of it (any pointer may be NULL). */
SOAR_API int soar_model_memory_info(void* handle, size_t* param_bytes,
                                    size_t* activation_capacity,
                                    size_t* activation_peak);

#ifdef __cplusplus
}
#endif

#endif /* SOAR_API_H */
