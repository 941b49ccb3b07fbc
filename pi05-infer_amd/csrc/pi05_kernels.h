// Kernel argument blocks and launchers of the gfx950 denoise engine (host <-> device contract).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pi05 {

typedef uint16_t u16;

constexpr int kMaxSteps = 32;  // Euler steps the modulation-table builder supports

struct PrimeKvArgs {
  const void* const* k_ptrs;  // device array [depth] of bf16 [B, 1, P, D] bases
  const void* const* v_ptrs;
  int64_t batch_stride;  // elements between samples
  int64_t row_stride;    // elements between prefix positions
  u16* kcache;           // [depth][B] fragment-major blocks of s_pad * D
  u16* vcache;
  int batch, prefix_len, s_pad;
};

struct PrimeTablesArgs {
  const uint8_t* prefix_pad;  // [B, P]
  const float* inv_freq;      // [D/2]
  int32_t* positions;         // [B, A]
  uint8_t* valid;             // [B, s_pad]
  u16* cos_tab;               // [B, A, D] bf16
  u16* sin_tab;
  int prefix_len, s_pad;
};

struct GemvArgs {
  const float* W;     // [rows, K]
  const float* bias;  // [rows]
  const float* in;    // [S, K]
  float* out;         // out[s * out_ld + out_off + row]
  int rows, K, S, out_ld, out_off, silu;
};

struct StepIoArgs {
  float* rowss;            // [64][M] partial sums of squares of h rows (read, then rewritten)
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

struct QkvArgs {
  const u16* w;          // packed q|k|v tiles of this layer
  const u16* h;          // [M, W]
  const float* rowss;    // [64][M]
  const float* mod;      // input_layernorm modulation row [3W] of this step
  const u16* cos_tab;    // [M, D]
  const u16* sin_tab;
  u16* q;                // [M, H*D]
  u16* kcache;           // this layer's [B] fragment-major K blocks
  u16* vcache;
  float eps;
  int M, prefix_len, s_pad;
};

struct ResidualArgs {
  const u16* w;         // packed [W/16 tiles][K/32] fragments
  const u16* act;       // [M, K] bf16 GEMM input
  const float* mod_gate;  // gate third of the modulation row [W]
  u16* h;               // [M, W] residual stream (updated in place)
  float* rowss;         // [64][M] partial sums of squares (written)
  int M;
};

struct GateUpArgs {
  const u16* wgate;
  const u16* wup;
  const u16* h;
  const float* rowss;
  const float* mod;     // post_attention_layernorm modulation row [3W]
  u16* act;             // [M, I]
  float eps;
  int M;
};

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

hipError_t launch_pack_weight(const void* src, u16* dst, int N, int K, hipStream_t st);
hipError_t launch_prime_kv(const PrimeKvArgs& a, int depth, hipStream_t st);
hipError_t launch_prime_tables(const PrimeTablesArgs& a, int batch, hipStream_t st);
hipError_t launch_gemv_rows(const GemvArgs& a, hipStream_t st);
hipError_t launch_step_io(const StepIoArgs& a, hipStream_t st);
hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t st);
hipError_t launch_o_proj(const ResidualArgs& a, hipStream_t st);
hipError_t launch_down(const ResidualArgs& a, hipStream_t st);
hipError_t launch_gate_up(const GateUpArgs& a, hipStream_t st);
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);

}  // namespace pi05
