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

constexpr int kMaxAttnSplits = 8;

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
hipError_t launch_qkv_rope(const GemmArgs& a, hipStream_t st);
hipError_t launch_gate_up(const GemmArgs& a, hipStream_t st);
hipError_t launch_o_proj(const GemmArgs& a, hipStream_t st);
hipError_t launch_down(const GemmArgs& a, hipStream_t st);
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);

}  // namespace pi05
