/*
 * pi05_denoise.h -- C ABI of the MI355X (gfx950) pi0.5 action-expert denoise engine.
 *
 * One context (`pi05_ctx`) owns everything one shape signature needs: packed bf16 expert weights,
 * the adaRMS modulation table, the re-laid-out static KV cache and the activation buffers of the
 * whole num_steps Euler loop.  The signature is (batch, prefix_len, num_steps);
 * a different signature needs a different context (the reference captures its graph per
 * signature as well: engine.py:884-906).
 *
 * Conventions
 *  - Every buffer argument is a DEVICE pointer on the context's device unless the name says
 *    `host`.  bf16 tensors are passed as `const void*` holding IEEE bfloat16 bits.
 *  - Every entry point returns 0 on success and a negative PI05_E* code on failure; the message
 *    is available from pi05_last_error(ctx) (or pi05_last_error(NULL) for failures of
 *    pi05_ctx_create).  No C++ exception crosses this boundary.  Shapes, pointers and alignment
 *    are validated before any HIP call is made, so the validation paths can be exercised on a
 *    machine without a GPU.
 *  - A context is bound to one device and is not thread-safe; calls on one context must be
 *    serialised by the caller.  Work is enqueued on the stream passed to each call
 *    (a hipStream_t, NULL = the legacy default stream).
 *  - Bound weight pointers are borrowed: the context copies (packs) them into its own layout in
 *    pi05_refresh_weights() and never reads them afterwards.  Prefix KV pointers are likewise
 *    only read inside pi05_prime_prefix().
 *
 * The reference interfaces these entry points replace are cited per function
 * (paths relative to the pi05-infer repository).
 */
#ifndef PI05_DENOISE_H
#define PI05_DENOISE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PI05_ABI_VERSION 1

/* error codes */
#define PI05_OK 0
#define PI05_E_INVALID (-1)     /* bad argument / shape outside what the engine supports */
#define PI05_E_STATE (-2)       /* call order violated (e.g. denoise before weights are bound) */
#define PI05_E_HIP (-3)         /* a HIP runtime call failed */
#define PI05_E_NOMEM (-4)       /* device allocation failed */
#define PI05_E_NODEVICE (-5)    /* no usable gfx950 device */

/* Model geometry + shape signature.  Mirrors the reference's Gemma-300M expert config
 * (openpi_patched/gemma_pytorch.py:64-76) plus the per-predict shapes
 * (engine.py:884-892).  The expert geometry fields must equal the compiled geometry
 * (width 1024, 8 query heads, 1 KV head, head_dim 256, mlp_dim 4096, action_dim 32,
 * action_horizon 50); depth, batch, prefix_len and num_steps are free. */
typedef struct pi05_dims {
  int32_t width;          /* 1024 */
  int32_t depth;          /* number of decoder layers (18) */
  int32_t num_heads;      /* 8 */
  int32_t num_kv_heads;   /* 1 */
  int32_t head_dim;       /* 256 */
  int32_t mlp_dim;        /* 4096 */
  int32_t action_dim;     /* 32 */
  int32_t action_horizon; /* 50 */
  int32_t batch;          /* B >= 1 */
  int32_t prefix_len;     /* P >= 1 prefix tokens in the static KV cache */
  int32_t num_steps;      /* Euler steps (10) */
  float rms_eps;          /* 1e-6 (GemmaRMSNorm eps, modeling_gemma.py:66) */
  float rope_theta;       /* 10000 (transformers default rope) */
  double time_min_period; /* 4e-3 (pi0_pytorch.py:298; a Python float, hence double) */
  double time_max_period; /* 4.0 */
} pi05_dims;

typedef struct pi05_ctx pi05_ctx;

/* ABI version of the loaded library (compare with PI05_ABI_VERSION). */
int pi05_abi_version(void);

/* Fill `dims` with the reference pi0.5 expert geometry (depth 18, B=1, P=968, 10 steps). */
void pi05_default_dims(pi05_dims* dims);

/* Validate `dims` without touching a GPU.  Returns 0 or PI05_E_INVALID (+ pi05_last_error(NULL)). */
int pi05_check_dims(const pi05_dims* dims);

/* Bytes of device memory a context with these dims allocates (for capacity planning).
 * Returns 0 on invalid dims. */
size_t pi05_ctx_device_bytes(const pi05_dims* dims);

/* Create a context on the current HIP device.  Replaces the construction done by
 * OpenPi0Inference.__init__ / capture_cuda_graph (engine.py:179-212, 831-860). */
int pi05_ctx_create(const pi05_dims* dims, pi05_ctx** out);

/* Destroy a context and free its device memory (cuda_graph.py:252-268 destroy()). */
int pi05_ctx_destroy(pi05_ctx* ctx);

/* Last error message of `ctx` (or of the calling thread's last failed global call if ctx is
 * NULL).  Valid until the next call on the same context / thread. */
const char* pi05_last_error(const pi05_ctx* ctx);

/* Bind one decoder layer's weights (borrowed device pointers).
 * wq [H*D, W], wk [D, W], wv [D, W], wo [W, H*D], wgate [I, W], wup [I, W], wdown [W, I]: bf16
 * row-major nn.Linear weights (modeling_gemma.py:131-133, 291-302).
 * ln1_w / ln2_w [3W, W], ln1_b / ln2_b [3W]: fp32 adaRMS dense weight/bias of
 * input_layernorm / post_attention_layernorm (modeling_gemma.py:73-77, 469-470).
 * Replaces the reference's per-layer module parameters + build_qkv_fused (modeling_gemma.py:331-351). */
int pi05_bind_layer(pi05_ctx* ctx, int layer, const void* wq, const void* wk, const void* wv,
                    const void* wo, const void* wgate, const void* wup, const void* wdown,
                    const float* ln1_w, const float* ln1_b, const float* ln2_w, const float* ln2_b);

/* Bind the final norm's adaRMS dense (model.norm.dense, modeling_gemma.py:564), the action
 * in/out projections (pi0_pytorch.py:104-105) and the time MLP (pi0_pytorch.py:108-109).
 * All fp32: norm_w [3W, W], norm_b [3W], in_w [W, A], in_b [W], out_w [A, W], out_b [A],
 * tin_w/tout_w [W, W], tin_b/tout_b [W]. */
int pi05_bind_heads(pi05_ctx* ctx, const float* norm_w, const float* norm_b, const float* in_w,
                    const float* in_b, const float* out_w, const float* out_b, const float* tin_w,
                    const float* tin_b, const float* tout_w, const float* tout_b);

/* (Re)pack every bound weight into the context's layout and rebuild the adaRMS modulation table
 * on the device, in place (device addresses never change, so a captured graph stays valid).
 * Call after binding and after any in-place weight update.  Replaces
 * invalidate_weight_derived_caches / refresh_derived_weights / _compute_adarms_table
 * (engine.py:526-599, modeling_gemma.py:627-652). */
int pi05_refresh_weights(pi05_ctx* ctx, void* stream);

/* Copy the modulation table [num_steps][2*depth+1][3W] fp32 (device) that refresh built, for
 * inspection.  Mirrors reading OpenPi0Inference._adarms_table[:, 0] (engine.py:645-649). */
int pi05_get_adarms_table(pi05_ctx* ctx, float* table_out, void* stream);

/* Load this predict's prefix: k_layers[l] / v_layers[l] are device pointers to bf16
 * [B, 1, P, D] tensors (the DynamicCache of _build_prefix_cache, engine.py:770-794) with
 * row stride `kv_row_stride` elements between consecutive prefix positions (D for contiguous),
 * and prefix_pad is a device uint8/bool [B, P] key-padding mask (1 = valid).  Packs the KV into
 * the context's static cache and derives positions, RoPE tables and key masks.  Replaces
 * prime_kv_static + _build_step_invariants (modeling_gemma.py:312-329, 605-615;
 * engine.py:453-524). `k_layers` / `v_layers` are HOST arrays of `depth` device pointers, read
 * during the call only; the packing is enqueued on `stream` (the call does not block). */
int pi05_prime_prefix(pi05_ctx* ctx, const void* const* k_layers, const void* const* v_layers,
                      int64_t kv_batch_stride, int64_t kv_row_stride, const uint8_t* prefix_pad,
                      void* stream);

/* Copy the step invariants that pi05_prime_prefix derived out of the context, in the reference's
 * layout (a parity / debug read; it does not change the context).  Replaces reading the buffers
 * of _build_step_invariants (engine.py:453-524):
 *   positions_out   int64 [B, A]: sum(prefix_pad[b]) + t, the RoPE positions (engine.py:476-477);
 *   key_valid_out   uint8 [B, P + A]: 1 where action query rows may attend key j, keys in the
 *                   reference's order (P prefix keys, then the A action keys): prefix_pad over
 *                   the prefix, 1 over the action keys -- the zero entries of the additive mask
 *                   of engine.py:471-478 / pi0_pytorch.py:160-163 (the same for every query row);
 *   stray_valid_out int32 [1]: padding slots of the context's key table that are marked valid
 *                   (0 for a correct table).
 * Device pointers, each nullable (not all).  Requires a primed prefix; enqueued on `stream`. */
int pi05_get_step_invariants(pi05_ctx* ctx, int64_t* positions_out, uint8_t* key_valid_out,
                             int32_t* stray_valid_out, void* stream);

/* Run the full num_steps Euler denoise loop (one cooperative kernel, or a hipGraph replay in the
 * graph schedule): x_inout [B, A, a] fp32 holds the initial noise x_1 on entry and the actions
 * x_0 on exit.  v_trace (nullable) [num_steps, B, A, a] fp32 receives each step's velocity.
 * Both schedules only enqueue work on `stream`; nothing blocks the host.  Every wait inside the
 * persistent kernel is bounded: a launch whose wait gives up leaves its outputs invalid and is
 * reported asynchronously, as PI05_E_HIP from the next pi05_denoise on this context (which then
 * enqueues nothing) or from pi05_denoise_status.
 * Graph capture: in the persistent schedule the call may be captured into a hipGraph (e.g. inside
 * torch.cuda.graph) and the graph replayed any number of times -- the launch carries no
 * per-call state; the kernel takes its flag epoch from the context's device memory and advances
 * it itself.  A timed-out replay is reported by the next pi05_denoise or pi05_denoise_status on
 * the context.  In the graph schedule (itself a hipGraph) a call on a capturing stream returns
 * PI05_E_STATE.  Replays and calls of one context must not overlap (one stream).
 * Replaces sample_actions' denoise loop (engine.py:389-405) with sample_mean_var_val /
 * get_velocity / the expert forward (engine.py:629-768, modeling_gemma.py:662-794). */
int pi05_denoise(pi05_ctx* ctx, float* x_inout, float* v_trace, void* stream);

/* Wait for `stream` and report the timed-out persistent launches of this context that have not been
 * reported yet (PI05_E_HIP), once.  The reference surfaces device-side failures at the next
 * synchronising call in the same way (CUDA/torch asynchronous error semantics); this is that
 * synchronising call for callers that want it per predict. */
int pi05_denoise_status(pi05_ctx* ctx, void* stream);

/* Test hook: polls after which a wait of the persistent kernel gives up (0 restores the default of
 * 2^20).  A small value makes waits give up on purpose, so the timeout path can be exercised;
 * every workgroup still leaves the kernel normally.  No counterpart in the reference. */
int pi05_debug_set_spin_limit(pi05_ctx* ctx, int polls);

/* Test hook: every persistent launch checks that its workgroups were dealt round-robin over the
 * 8 XCDs (workgroup w on XCD (w + d) mod 8, one d per launch), which its intra-XCD hand-offs
 * assume, and a launch that finds otherwise is reported as PI05_E_HIP by the next pi05_denoise or
 * pi05_denoise_status.  A skew of 1..7 is added to the offset the odd workgroups compute (their
 * placement and the kernel's work are unchanged), so that the report can be exercised; 0 (the
 * default) restores the plain check.  No counterpart in the reference. */
int pi05_debug_skew_placement_check(pi05_ctx* ctx, int skew);

/* Test hook: set the epoch of the last finished persistent launch (the next launch runs as
 * epoch + 1; the launch that reaches 2^31 zeroes the flags and the next one runs as epoch 1), so
 * that the wrap-around can be exercised without 2^31 launches.  Synchronises the device;
 * persistent schedule only (PI05_E_STATE otherwise).  epoch must be below 2^31.  No counterpart
 * in the reference. */
int pi05_debug_set_epoch(pi05_ctx* ctx, uint32_t epoch);

/* Drop the captured graph (it is recaptured on the next pi05_denoise).  Mirrors
 * release_cuda_graph (_vendored/base_policy.py:96-102). */
int pi05_release_graph(pi05_ctx* ctx);

/* Execution schedules of pi05_denoise.
 *  PI05_SCHEDULE_PERSISTENT (default where the device supports cooperative launch): the whole
 *    Euler loop is ONE cooperative kernel, one workgroup per compute unit, whose phases hand
 *    activations to each other through device memory and per-phase flags.
 *  PI05_SCHEDULE_GRAPH: one hipGraph of 1 + depth * 5..6 kernels per Euler step.
 * Both compute the same function with the same rounding points.  The reference runs its loop
 * eagerly or replays one captured flow_ode step per Euler step as a CUDA graph
 * (engine.py:831-860, 908-960); PI05_SCHEDULE_GRAPH is the counterpart of that graph, the
 * persistent kernel has no counterpart in the reference. */
#define PI05_SCHEDULE_PERSISTENT 0
#define PI05_SCHEDULE_GRAPH 1

/* Switch a context's schedule.  Frees the previous schedule's activation buffers, so the prefix
 * must be primed again (pi05_prime_prefix) before the next pi05_denoise; weights stay bound and
 * packed.  Synchronises the device.  No counterpart in the reference (see above). */
int pi05_set_schedule(pi05_ctx* ctx, int schedule);

/* Current schedule of `ctx` (PI05_SCHEDULE_*), or PI05_E_INVALID for NULL. */
int pi05_get_schedule(const pi05_ctx* ctx);

/* Number of kernel launches in one denoise step (for profiling): 1 + depth * 5..6 in the graph
 * schedule, 0 in the persistent schedule (one launch per pi05_denoise). */
int pi05_launches_per_step(const pi05_ctx* ctx);

/* Profiling hook: enqueue `iters` back-to-back launches of one kernel of the denoise step with the
 * arguments the graph uses for Euler step 0 and decoder layer `layer`, on `stream`.  kernel_id:
 * 0 step boundary (final norm + action_out_proj + Euler + action_in_proj), 1 qkv_rope,
 * 2 attention, 3 o_proj, 4 gate_up, 5 down_proj.  Graph schedule only (PI05_E_STATE otherwise).
 * It overwrites the context's activations, so call pi05_denoise again afterwards for a
 * meaningful result.  No counterpart in the reference (its tools/ time kernels from nsys
 * traces); it lets a benchmark time one kernel with events. */
int pi05_bench_kernel(pi05_ctx* ctx, int kernel_id, int layer, int iters, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving or RL weight-sync loops): the adaRMS modulation table that
 * pi05_refresh_weights builds (and pi05_get_adarms_table returns), computed without a context
 * straight from caller-owned fp32 weights -- the time MLP tin_w [W, W], tin_b [W], tout_w [W, W],
 * tout_b [W] and the 2*depth+1 norm dense layers (host arrays dense_w / dense_b of device
 * pointers to [3W, W] / [3W], in the table's norm order: input_layernorm and
 * post_attention_layernorm of each layer, then the final norm) -- into table_out
 * [num_steps][2*depth+1][3W] fp32 (device).  It replaces no reference interface: it is the
 * table-building part of pi05_refresh_weights as a stand-alone call.
 * It allocates nothing: its scratch (time embedding + two time-MLP activations, 384 KiB) is a
 * static device array of the library, one per GPU, kept until the process ends; num_steps above
 * 32 is rejected with PI05_E_INVALID.  Every call on one GPU shares that GPU's scratch (each call
 * rewrites all of it before reading it): calls that overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller.  Enqueued on `stream`; dims supplies depth,
 * num_steps and the time periods. */
int pi05_adarms_table_noalloc(const pi05_dims* dims, const float* tin_w, const float* tin_b,
                              const float* tout_w, const float* tout_b,
                              const float* const* dense_w, const float* const* dense_b,
                              float* table_out, void* stream);

/* ---- host-only helpers (no GPU needed; what the context computes on the host) ---- */

/* Euler schedule linspace(1, 1/N, N) ++ [0] in fp32, evaluated as the reference's device
 * linspace does (engine.py:411-429).  ts_host has num_steps + 1 entries. */
int pi05_euler_schedule(int num_steps, float* ts_host);

/* Sinusoidal timestep embedding [width] fp32 of scalar t (float64 math, pi0_pytorch.py:29-46). */
int pi05_time_embedding(const pi05_dims* dims, float t, float* out_host);

/* RoPE inverse frequencies [head_dim / 2] fp32 (transformers default rope:
 * 1 / theta ** (arange(0, D, 2) / D)). */
int pi05_rope_inv_freq(const pi05_dims* dims, float* out_host);

#ifdef __cplusplus
}
#endif

#endif /* PI05_DENOISE_H */
