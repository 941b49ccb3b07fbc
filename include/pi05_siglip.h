/*
 * pi05_siglip.h -- C ABI of the MI355X (gfx950) vision tower of pi0.5: SigLIP So400m/14 and
 * PaliGemma's multi-modal projector, i.e. `get_image_features` as `embed_image` calls it
 * (gemma_pytorch.py:106-107; pi0_pytorch.py:200-220), producing the image part of the prefix
 * embeddings the prefill (pi05_prefill.h) consumes.
 *
 * One context (`pi05_vision_ctx`) owns the packed tower weights, the activations of one image
 * count and its GEMM plans.  The plain GEMMs (patch embedding in fp32, q|k|v, out_proj, fc1, fc2,
 * projector with their biases) run on hipBLASLt; LayerNorm, the attention (16 heads of 72) and
 * GELU are hand-written gfx950 kernels.  Conventions are those of pi05_denoise.h.
 */
#ifndef PI05_SIGLIP_H
#define PI05_SIGLIP_H

#include <stddef.h>
#include <stdint.h>

#include "pi05_denoise.h"

#ifdef __cplusplus
extern "C" {
#endif

/* SigLIP So400m/14 as PaliGemma configures it (gemma_pytorch.py:58-61 on transformers'
 * SiglipVisionConfig defaults).  Geometry fields must equal the compiled one; depth and
 * n_images are free. */
typedef struct pi05_vision_dims {
  int32_t width;     /* 1152 */
  int32_t depth;     /* 27 encoder layers */
  int32_t num_heads; /* 16 (head_dim 72) */
  int32_t mlp_dim;   /* 4304 */
  int32_t patch;     /* 14 */
  int32_t image;     /* 224 (256 patches) */
  int32_t channels;  /* 3 */
  int32_t proj_dim;  /* 2048 (the prefix LM's width) */
  int32_t n_images;  /* images per call: batch x camera views (>= 1) */
  float ln_eps;      /* 1e-6 */
  float out_scale;   /* multiplier of the projector output: 1 (see the vision oracle's header) */
} pi05_vision_dims;

typedef struct pi05_vision_ctx pi05_vision_ctx;

void pi05_vision_default_dims(pi05_vision_dims* dims);  /* depth 27, 3 images, out_scale 1 */
int pi05_vision_check_dims(const pi05_vision_dims* dims);
size_t pi05_vision_device_bytes(const pi05_vision_dims* dims);
int pi05_vision_create(const pi05_vision_dims* dims, pi05_vision_ctx** out);
int pi05_vision_destroy(pi05_vision_ctx* ctx);
const char* pi05_vision_last_error(const pi05_vision_ctx* ctx);

/* Encoder layer `layer` (borrowed device pointers, bf16 as the reference holds them):
 * wq, wk, wv, wo [W, W] and bq, bk, bv, bo [W]; w1 [I, W], b1 [I]; w2 [W, I], b2 [W];
 * ln1_w, ln1_b, ln2_w, ln2_b [W] (vision_tower.vision_model.encoder.layers.{i}.*). */
int pi05_vision_bind_layer(pi05_vision_ctx* ctx, int layer, const void* wq, const void* bq, const void* wk, const void* bk,
                           const void* wv, const void* bv, const void* wo, const void* bo, const void* w1, const void* b1,
                           const void* w2, const void* b2, const void* ln1_w, const void* ln1_b, const void* ln2_w,
                           const void* ln2_b);

/* Embeddings, final norm and projector: patch_w [W, 3, 14, 14], patch_b [W], pos [256, W] fp32
 * (kept fp32 by gemma_pytorch.py:93-97); post_w, post_b [W], proj_w [P, W], proj_b [P] bf16. */
int pi05_vision_bind_heads(pi05_vision_ctx* ctx, const float* patch_w, const float* patch_b, const float* pos,
                           const void* post_w, const void* post_b, const void* proj_w, const void* proj_b);

/* Pack every bound weight (fused q|k|v, fp32 biases and norm parameters), in place. */
int pi05_vision_refresh_weights(pi05_vision_ctx* ctx, void* stream);

/* pixels [N, 3, 224, 224] fp32 in [-1, 1] -> out [N, 256, proj_dim] bf16 image embeddings.
 * Enqueues only. */
int pi05_vision_forward(pi05_vision_ctx* ctx, const float* pixels, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PI05_SIGLIP_H */
