/*
 * pi05_prefill.h -- C ABI of the MI355X (gfx950) prefix-LM prefill: the PaliGemma Gemma-2B
 * language model run over the prefix embeddings to build the KV cache that the denoise loop
 * consumes (pi05_denoise.h, pi05_prime_prefix).
 *
 * One context (`pi05_prefix_ctx`) owns the Gemma-2B layer weights (packed on refresh), the
 * activation buffers of one (batch, prefix_len) signature and its GEMM plans.  The plain GEMMs
 * (q|k|v, o_proj, gate|up, down_proj) run on hipBLASLt; norms, RoPE and the K/V write, the
 * masked attention and GeGLU are hand-written gfx950 kernels.
 *
 * Conventions are those of pi05_denoise.h: device pointers unless a name says `host`, bf16 as
 * raw bit patterns, 0 / negative PI05_E* codes with a message from pi05_prefix_last_error, every
 * argument validated before the first HIP call, one stream per call, not thread-safe per context.
 */
#ifndef PI05_PREFILL_H
#define PI05_PREFILL_H

#include <stddef.h>
#include <stdint.h>

#include "pi05_denoise.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry of the prefix LM (openpi gemma_2b: gemma_pytorch.py:44-54) and the signature.  The
 * geometry fields must equal the compiled one: width 2048, 8 query heads, 1 KV head, head_dim
 * 256, mlp_dim 16384; depth, batch and prefix_len are free. */
typedef struct pi05_prefix_dims {
  int32_t width;           /* 2048 */
  int32_t depth;           /* 18 */
  int32_t num_heads;       /* 8 */
  int32_t num_kv_heads;    /* 1 */
  int32_t head_dim;        /* 256 */
  int32_t mlp_dim;         /* 16384 */
  int32_t batch;           /* B >= 1 */
  int32_t prefix_len;      /* P >= 1 prefix tokens (images + language) */
  float rms_eps;           /* 1e-6 */
  float rope_theta;        /* 10000 */
  int32_t skip_last_layer; /* 1: the last layer computes only its K/V, which is all the cache
                              needs (patches/prefix_last_layer.py:84-112, on by default there) */
} pi05_prefix_dims;

typedef struct pi05_prefix_ctx pi05_prefix_ctx;

/* Fill `dims` with the reference geometry (depth 18, B=1, P=968, last layer K/V only). */
void pi05_prefix_default_dims(pi05_prefix_dims* dims);

/* Validate `dims` without touching a GPU (0 or PI05_E_INVALID + pi05_prefix_last_error(NULL)). */
int pi05_prefix_check_dims(const pi05_prefix_dims* dims);

/* Bytes of device memory a context with these dims allocates; 0 on invalid dims. */
size_t pi05_prefix_device_bytes(const pi05_prefix_dims* dims);

/* Create / destroy a context on the current HIP device (the prefix half of
 * OpenPi0Inference.__init__, engine.py:179-212). */
int pi05_prefix_create(const pi05_prefix_dims* dims, pi05_prefix_ctx** out);
int pi05_prefix_destroy(pi05_prefix_ctx* ctx);

/* Last error message of `ctx` (or of the calling thread's last failed global call). */
const char* pi05_prefix_last_error(const pi05_prefix_ctx* ctx);

/* Bind layer `layer`'s weights (borrowed device pointers, read only by refresh):
 * wq [H*D, W], wk [D, W], wv [D, W], wo [W, H*D], wgate [I, W], wup [I, W], wdown [W, I] bf16
 * row-major nn.Linear weights (modeling_gemma.py:131-133, 291-302); ln1_w / ln2_w [W] fp32
 * input_layernorm / post_attention_layernorm weights (modeling_gemma.py:78, 469-470; kept fp32
 * by gemma_pytorch.py:84-104). */
int pi05_prefix_bind_layer(pi05_prefix_ctx* ctx, int layer, const void* wq, const void* wk, const void* wv,
                           const void* wo, const void* wgate, const void* wup, const void* wdown,
                           const float* ln1_w, const float* ln2_w);

/* Copy every bound weight into the context's layout (fused q|k|v and gate|up blocks), in place.
 * Call after binding and after any in-place update (the prefix half of
 * invalidate_weight_derived_caches, engine.py:526-554). */
int pi05_prefix_refresh_weights(pi05_prefix_ctx* ctx, void* stream);

/* Language-token embedding of embed_prefix: out[i] = bf16(table[ids[i]] * sqrt(width)) for
 * n_tokens int32 ids (pi0_pytorch.py:225-228).  table [vocab, W] bf16, out [n_tokens, W] bf16.
 * Enqueues only.  Ids outside [0, vocab) are caught on the device: their rows are zero-filled
 * and the call's tag goes to a pinned host word; the error is reported as PI05_E_INVALID once,
 * by the next pi05_prefix_embed_tokens on the context (which then enqueues nothing) or by
 * pi05_prefix_status.  (The reference's embedding lookup fails asynchronously too, with a
 * device-side assert.) */
int pi05_prefix_embed_tokens(pi05_prefix_ctx* ctx, const int32_t* ids, int64_t n_tokens, const void* table,
                             int64_t vocab, void* out, void* stream);

/* Waits for `stream` and reports a token id outside [0, vocab) met by an earlier
 * pi05_prefix_embed_tokens call on this context that has not been reported yet (PI05_E_INVALID,
 * once).  No counterpart in the reference (its lookup asserts on the device); call it where the
 * embeddings must be known good. */
int pi05_prefix_status(pi05_prefix_ctx* ctx, void* stream);

/* The prefill: embeds [B, P, W] bf16 (SigLIP image embeddings followed by the scaled language
 * embeddings, embed_prefix, pi0_pytorch.py:190-255) and prefix_pad [B, P] uint8/bool (1 = valid)
 * -> per layer l the K (after RoPE) and V of every prefix position, written to k_layers[l] /
 * v_layers[l]: bf16 [B, 1, P, D] with `kv_batch_stride` elements between samples and
 * `kv_row_stride` between positions (D for contiguous) -- the DynamicCache of
 * _build_prefix_cache (engine.py:770-794), ready for pi05_prime_prefix.  `k_layers` /
 * `v_layers` are HOST arrays of `depth` device pointers.  Positions are cumsum(pad) - 1 and
 * every valid token attends to every valid token (pi0_pytorch.py:236-250, 56-85).  Padded
 * positions get finite K/V that no valid token ever attends to.  Enqueues only. */
int pi05_prefix_forward(pi05_prefix_ctx* ctx, const void* embeds, const uint8_t* prefix_pad,
                        void* const* k_layers, void* const* v_layers, int64_t kv_batch_stride,
                        int64_t kv_row_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PI05_PREFILL_H */
