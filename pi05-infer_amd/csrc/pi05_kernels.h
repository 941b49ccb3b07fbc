// Kernel argument blocks and launchers of the gfx950 denoise engine (host <-> device contract).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pi05 {

typedef uint16_t u16;

constexpr int kMaxSteps = 32;  // Euler steps the modulation-table builder supports

constexpr int kMaxDepth = 64;  // layers a context may have (the per-layer pointers travel as kernel arguments)

struct PrimeKvArgs {
  const void* k_ptrs[kMaxDepth];  // per layer: bf16 [B, 1, P, D] bases (passed by value, no device table)
  const void* v_ptrs[kMaxDepth];
  int64_t batch_stride;  // elements between samples
  int64_t row_stride;    // elements between prefix positions
  u16* kcache;           // [depth][B] fragment-major blocks of s_pad * D
  u16* vcache;
  int batch, prefix_len, s_pad;
  int suffix_base;  // keys [suffix_base, suffix_base + A) belong to the action tokens: left untouched
};

struct PrimeTablesArgs {
  const uint8_t* prefix_pad;  // [B, P]
  const float* inv_freq;      // [D/2]
  int32_t* positions;         // [B, A]
  uint8_t* valid;             // [B, s_pad]
  u16* cos_tab;               // [B, A, D] bf16
  u16* sin_tab;
  int prefix_len, s_pad;  // s_pad: keys per batch row of the valid mask
  int suffix_base;        // first key of the action tokens in the mask
};

// The step invariants of a primed context in the reference's key order (a debug / parity copy).
struct ExportInvariantsArgs {
  const int32_t* positions;  // [B, A]
  const uint8_t* valid;      // [B, valid_ld] the context's key-valid table
  int64_t* pos_out;          // [B, A] (nullable)
  uint8_t* valid_out;        // [B, P + A] prefix keys, then the A action keys (nullable)
  int32_t* stray_out;        // [1] padding slots of the table marked valid (nullable)
  int batch, prefix_len, valid_ld;
  int suffix_base;           // first slot of the action keys in the table
};

struct GemvArgs {
  const float* W;     // [rows, K]
  const float* bias;  // [rows]
  const float* in;    // [S, K]
  float* out;         // out[s * out_ld + out_off + row]
  int rows, K, S, out_ld, out_off, silu;
};

struct StepIoArgs {
  float* rowss;            // [M][64] partial sums of squares of h rows (read, then rewritten)
  u16* h;                  // [M, W] bf16 residual stream
  float* x;                // [M, a] actions (in/out)
  float* trace;            // [M, a] velocity of the previous step (nullable)
  const float* final_mod;  // modulation row of the final norm for the previous step [3W]
  const float* out_w;      // [a, W]
  const float* out_b;      // [a]
  const float* in_w;       // [W, a]
  const float* in_b;       // [W]
  float eps, t, one_minus_t, x0_weight, x1_weight;
  int M, has_prev, has_next;
};

// One argument block for the GEMM family (fields unused by a mode are ignored).
struct GemmArgs {
  const u16* w;          // packed weight tiles (q|k|v, gate, o_proj or down)
  const u16* w2;         // packed up_proj tiles (gate_up)
  const u16* act;        // [M, K] bf16 A operand (residual mode)
  const u16* h;          // [M, W] residual stream read by the adaRMSNorm prologue
  u16* h_out;            // [M, W] residual stream updated by the residual epilogue
  float* rowss;          // [M][64] row sums of squares: read by the prologue, written by the residual epilogue
  const float* mod;      // modulation row [3W] of this norm and step: scale | shift | gate
  const u16* cos_tab;    // [M, D] bf16 RoPE tables
  const u16* sin_tab;
  u16* q;                // [M, H*D]
  u16* kcache;           // this layer's [B] fragment-major K blocks
  u16* vcache;
  u16* out;              // [M, I] GeGLU output
  float eps;
  int M, prefix_len, s_pad;
};

constexpr int kMaxAttnSplits = 16;
// Persistent attention at batches of at least kAttnGroupMinBatch: items of kAttnGroup two-token
// row blocks of one sample, one per wave, sharing each K/V block through LDS; the key splits
// then fill the 256 workgroups once (attn_group_splits).
constexpr int kAttnGroupMinBatch = 3;
// Batches from which the persistent kernel's gate_up items split rows over waves instead of K
// (each wave one sample over the whole K; kernel instance 2).
constexpr int kRowSplitMinBatch = 3;
constexpr int kAttnGroup = 4;
constexpr int kAttnGroupsPerSample = (50 / 2 + kAttnGroup - 1) / kAttnGroup;  // 7 groups of the 25 row blocks
inline int attn_group_splits(int batch, int nkb) {
  int n = 256 / (batch * kAttnGroupsPerSample);
  if (n > kMaxAttnSplits) n = kMaxAttnSplits;
  if (n > nkb) n = nkb;
  return n < 1 ? 1 : n;
}

struct AttnArgs {
  const u16* q;        // [rows, D] (rows = M * H)
  const u16* kcache;   // this layer's [B] K blocks
  const u16* vcache;
  const uint8_t* valid;  // [B, s_pad]
  u16* out;            // [rows, D]
  float* part;         // [nsplit, rows, D]
  float* part_m;       // [nsplit, rows]
  float* part_l;
  int rows, s_pad, nsplit;
};

// Every completion flag of the persistent kernel is kept in kFlagCopies replicas; workgroup w
// polls replica w mod kFlagCopies.  Workgroups are dispatched to the 8 XCDs round robin, so with
// 16 replicas each replica is polled by 16 workgroups of one XCD.  Measured on MI355X, ms per
// predict against 32 replicas (968-token prefix): one sample 4 replicas +0.3 %, 8 -0.5 %,
// 16 -0.4 %, 64 +1.8 %; eight samples 8 +0.7 %, 16 -0.1 %; two samples 8 +0.4 %.  Each publish
// stores every replica, so fewer replicas complete a publish sooner; fewer pollers per replica
// answer a poll sooner.  16 is the count that helps one sample and costs eight nothing.
constexpr int kFlagCopies = 16;

// The whole Euler loop as one cooperative kernel.  Activations live in per-(Euler step s,
// layer l) slices ("slw" = s * depth + l; h / ss slices are per (s, l') with l' in [0, depth],
// l' = depth being the last layer's output) that are written once per launch.  Rows are padded
// per sample: row r = b * 64 + t for action token t < 50 (rows t >= 50 stay zero), R = 64 * B
// rows.  Activation matrices are stored as MFMA A-operand fragments (pi05_device.h:
// afrag_offset), so one wave-wide 16-byte load reads 1 KiB of contiguous memory.
//
// adaRMSNorm is folded into the GEMM that consumes it: next to each residual-stream slice h the
// producer writes g = bf16(h * (1 + scale)) and per-16-column partial sums of squares ss of the
// rows; the consumer computes y = rstd * (g . W^T) + shift . W^T, with shift . W^T precomputed
// per (step, layer) in `bias`.
constexpr int kBiasCols = 2560 + 2 * 4096;  // 2560 q|k|v columns, then 4096 gate, then 4096 up

// Launch-control words of a context (one zero-filled 256-byte block, each word on its own 64-byte
// line): the error word, the epoch of the last launch that finished, the count of workgroups that
// have left the running launch, and the placement word (bit d set by every workgroup whose XCD is
// (workgroup index + d) mod 8).
constexpr int kCtlErr = 0;
constexpr int kCtlEpoch = 16;
constexpr int kCtlExit = 32;
constexpr int kCtlXcd = 48;
// The pinned host words of a context: launches whose waits timed out, launches whose workgroups
// were not placed round-robin over the XCDs.
constexpr int kHostTimeouts = 0;
constexpr int kHostPlacement = 1;
constexpr unsigned kEpochWrap = 1u << 31;  // a launch with this epoch zeroes the flags; the next runs as epoch 1

struct MegaArgs {
  unsigned epoch;      // this launch's flag value (1, 2, ...), read from ctl[kCtlEpoch] at kernel entry
  unsigned* err;       // the launch-control block; err[kCtlErr] = the epoch of a launch whose wait timed out
  int spin_limit;      // polls before a wait gives up (each poll >= ~1 us)
  unsigned* flags;     // per-item completion flags [(steps+1)][depth+1][7 phases][kFlagCopies][fstride]
  int fstride;         // flag words per phase instance and copy (multiple of 256)
  int depth, steps, batch, R, nbp, nsplit, nsplit_pad, nbp_pad, s_pre;
  float eps;
  const float* table;     // [steps][2*depth+1][3W] adaRMS modulation rows: scale | shift | gate
  const float* table_s1;  // the same rows with 1 + scale in place of scale
  const float* bias;      // [steps][depth][kBiasCols] shift . W^T of the norm each GEMM consumes
  const float* euler;     // [steps][4]: t, 1 - t, x0 weight, x1 weight
  const float* out_w;     // [a, W]
  const float* out_b;     // [a]
  const float* in_w;      // [W, a]
  const float* in_b;      // [W]
  const u16* wpack;       // [depth] packed layer weights
  const u16* cos_tab;     // [B*50, D] bf16 RoPE tables (compact rows b*50 + t)
  const u16* sin_tab;
  const u16* kpre;        // [depth][B] fragment-major prefix K of s_pre keys
  const u16* vpre;
  const uint8_t* valid;   // [B][s_pre + 64]
  u16* h;                 // [steps][depth+1] A fragments of [R, W]: residual stream into layer l'
  u16* g;                 // [steps][depth] A fragments of [R, W]: bf16(h * (1 + scale)) of norm 2l
  float* ss;              // [steps][depth+1] tile-major [64][R] partial sums of squares of h rows
  u16* hmid;              // [steps][depth] residual stream after attention, A fragments [R, W]
  u16* gmid;              // [steps][depth] bf16(hmid * (1 + scale)) of norm 2l+1
  float* ssmid;           // [steps][depth] tile-major [64][R]
  u16* q;                 // [steps][depth] fragments of [R*8 query rows (r*8 + head), D]
  u16* ksuf;              // [steps][depth][B] fragment-major K of the 64-key action block
  u16* vsuf;
  u16* o;                 // [steps][depth] A fragments of [R, H*D]
  u16* act;               // [steps][depth] A fragments of [R, I]
  float* apart;           // [steps][depth][nsplit][nbp][16][D] attention split partials
  float* apart_ml;        // [steps][depth][nsplit][nbp][2][16] running max | sum of the splits
  float* dpart;           // [steps][depth][4][64][R][16] down_proj K-quarter partials
  float* x;               // [steps][B*50, a] actions after step s (slot 0 unused)
  float* x_io;            // [B*50, a] caller's buffer: noise on entry, actions on exit
  float* trace;           // [steps][B*50, a] caller's velocity buffer (nullable)
  unsigned* host_err;     // pinned host words [kHostTimeouts], [kHostPlacement] (device-visible mapping)
  unsigned xcd_skew;      // test hook: added to the placement offset of odd workgroups (0 in normal runs)
  size_t flag_bytes;      // size of `flags` (zeroed by the launch that reaches kEpochWrap)
};

// bias[s][l][j] = sum_k shift_{s, norm(j)}[k] * W_l[j][k] from the packed weights, for the fused
// q|k|v columns (norm 2l) and the gate and up columns (norm 2l+1).
struct ShiftBiasArgs {
  const u16* wpack;    // [depth] packed layer weights
  const float* table;  // [steps][2*depth+1][3W]
  float* bias;         // [steps][depth][kBiasCols]
  int depth, steps;
};

hipError_t launch_shift_bias(const ShiftBiasArgs& a, hipStream_t st);
hipError_t launch_denoise_loop(const MegaArgs& a, int grid, hipStream_t st);
int denoise_loop_threads();
const void* denoise_loop_kernel_ptr(int batch);  // the instance launch_denoise_loop uses for `batch`

hipError_t launch_pack_weight(const void* src, u16* dst, int N, int K, hipStream_t st);
hipError_t launch_prime_kv(const PrimeKvArgs& a, int depth, hipStream_t st);
hipError_t launch_prime_tables(const PrimeTablesArgs& a, int batch, hipStream_t st);
hipError_t launch_export_invariants(const ExportInvariantsArgs& a, hipStream_t st);
hipError_t launch_gemv_rows(const GemvArgs& a, hipStream_t st);
// temb[s][0:W/2] = sin(2 pi t_s / period_i), temb[s][W/2:W] = cos(...) in float64, rounded to fp32,
// periods min_p * (max_p / min_p)^frac_i over the float64 device linspace(0, 1, W/2)
// (pi0_pytorch.py:29-46), t_s the Euler schedule of num_steps steps (engine.py:411-429) computed
// on the device with the host's fp32 operations (bit-identical to euler_schedule on the host).
hipError_t launch_time_embedding(int num_steps, float* temb, double min_p, double max_p, hipStream_t st);

// The adaRMS modulation table (engine.py:578-599) from the time MLP and the 2*depth+1 norm dense
// layers: temb -> cond1 = silu(W1 temb + b1) -> cond = silu(W2 cond1 + b2) -> table[s][n] =
// dense_n(cond[s]).  temb / cond1 / cond: caller-provided scratch of num_steps * W floats each.
struct AdarmsTableArgs {
  const float* tin_w;
  const float* tin_b;
  const float* tout_w;
  const float* tout_b;
  const float* const* dense_w;  // host array of n_norms device pointers [3W, W]
  const float* const* dense_b;  // host array of n_norms device pointers [3W]
  int n_norms, num_steps;
  double min_period, max_period;
  float* temb;
  float* cond1;
  float* cond;
  float* table;  // [num_steps][n_norms][3W]
};
hipError_t launch_adarms_table(const AdarmsTableArgs& a, hipStream_t st);
// out[r] = in[r] with 1 + scale in place of scale, for rows of [3W] modulation (scale | shift | gate)
hipError_t launch_scale_plus_one(const float* in, float* out, int rows, hipStream_t st);
hipError_t launch_step_io(const StepIoArgs& a, hipStream_t st);
hipError_t launch_qkv_rope(const GemmArgs& a, hipStream_t st);
hipError_t launch_gate_up(const GemmArgs& a, hipStream_t st);
hipError_t launch_o_proj(const GemmArgs& a, hipStream_t st);
hipError_t launch_down(const GemmArgs& a, hipStream_t st);
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);

}  // namespace pi05
