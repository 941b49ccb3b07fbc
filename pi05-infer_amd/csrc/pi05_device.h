// Device-side building blocks of the gfx950 denoise engine: types, bf16 rounding, the MFMA
// wrapper and the fragment-major layouts shared by the packing kernels and the compute kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pi05 {

// Compiled expert geometry (pi0.5 gemma_300m action expert).
constexpr int kWidth = 1024;       // hidden width W
constexpr int kHeads = 8;          // query heads
constexpr int kHeadDim = 256;      // D
constexpr int kHalfDim = 128;      // D / 2 (rotate-half split)
constexpr int kMlp = 4096;         // GeGLU intermediate I
constexpr int kHorizon = 50;       // action tokens A
constexpr int kActDim = 32;        // action dim a
constexpr int kQkvCols = (kHeads + 2) * kHeadDim;  // 2560 fused q|k|v output columns
constexpr int kModW = 3 * kWidth;  // adaRMS modulation row: scale | shift | gate
constexpr int kRowSlots = kWidth / 16;  // per-row sum-of-squares partials (one per 16-column tile)
constexpr int kQRowsPerTok = kHeads;    // attention query rows per token (MQA: 8 heads share K/V)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf2f(u16 b) { return __uint_as_float((uint32_t)b << 16); }

// float -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ u16 f2bf(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Uncontracted fp32 arithmetic: the reference evaluates these as separate tensor ops, each
// rounded, so the kernels must not fuse them into FMAs.
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float fsub(float a, float b) { return __fsub_rn(a, b); }

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ bf16x8 load_frag(const u16* p) {
  return as_bf16x8(*reinterpret_cast<const u16x8*>(p));
}

__device__ __forceinline__ bf16x8 zero_frag() {
  u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  return as_bf16x8(z);
}

// ---------------------------------------------------------------------------------------------
// Fragment-major layouts.
//
// MFMA 16x16x32 bf16 operand fragment: lane l holds 8 consecutive K-elements of row (l % 16),
// K offset (l / 16) * 8.  A "fragment" is 64 lanes x 8 bf16 = 1 KiB, stored lane-major so one
// wave-wide 16-byte load reads 1 KiB of contiguous memory.
//
// Weight W[N][K] (nn.Linear, row-major) used as the B operand (k x n): fragment (nt, ks) holds
// W[nt*16 + l%16][ks*32 + (l/16)*8 + j]; fragments are ordered n-tile major, so the K/32
// fragments of one 16-column tile are one contiguous 32*K-byte block.
// ---------------------------------------------------------------------------------------------
__host__ __device__ constexpr size_t wfrag_offset(int nt, int ks, int ksteps) {
  return ((size_t)nt * ksteps + ks) * 512;  // in bf16 elements
}

// Activation X[R][K] (row-major meaning) stored as MFMA A-operand fragments: fragment
// (m-tile mt, k-step ks) holds X[mt*16 + l%16][ks*32 + (l/16)*8 + j] for lane l, j < 8,
// fragments m-tile major.  afrag_offset gives the element offset of fragment (mt, ks) for
// K = 32 * ksteps; afrag_index the element (m, k).  Eight consecutive k of one row are 16
// contiguous bytes; one fragment is 1 KiB.
__host__ __device__ constexpr size_t afrag_offset(int mt, int ks, int ksteps) {
  return ((size_t)mt * ksteps + ks) * 512;
}
__host__ __device__ constexpr size_t afrag_index(int m, int k, int ksteps) {
  return afrag_offset(m >> 4, k >> 5, ksteps) + (size_t)((((k & 31) >> 3) << 4) + (m & 15)) * 8 + (k & 7);
}

// Per-layer packed weight block (bf16 elements): q|k|v rows as 160 tiles over K=1024, then o_proj
// (64 tiles over K=2048), gate (256 tiles over 1024), up (256 tiles over 1024), down (64 tiles over 4096).
constexpr size_t kQkvElems = (size_t)kQkvCols * kWidth;
constexpr size_t kOElems = (size_t)kWidth * kHeads * kHeadDim;
constexpr size_t kGateElems = (size_t)kMlp * kWidth;
constexpr size_t kDownElems = (size_t)kWidth * kMlp;
constexpr size_t kOffQkv = 0;
constexpr size_t kOffO = kOffQkv + kQkvElems;
constexpr size_t kOffGate = kOffO + kOElems;
constexpr size_t kOffUp = kOffGate + kGateElems;
constexpr size_t kOffDown = kOffUp + kGateElems;
constexpr size_t kLayerElems = kOffDown + kDownElems;

// ---------------------------------------------------------------------------------------------
// Static KV cache, per (layer, batch), over S_pad keys (multiple of 32):
//   K: key tile kt (16 keys) x d-step ds (32 dims): fragment [kt][ds] holds
//      K[kt*16 + l%16][ds*32 + (l/16)*8 + j]  -- the A operand of S^T = K Q^T.
//   V: key block kb (32 keys) x d-tile dt (16 dims): fragment [kb][dt] holds
//      V[vkey(kb, l/16, j)][dt*16 + l%16]      -- the A operand of O^T = V^T P^T,
//      with the key order permuted so the P^T operand is exactly the S^T accumulator each lane
//      already holds (keys kt*16 + (l/16)*4 + i of tiles 2kb and 2kb+1).
// ---------------------------------------------------------------------------------------------
__host__ __device__ constexpr int vkey(int kb, int g, int j) {
  return kb * 32 + (j < 4 ? g * 4 + j : 16 + g * 4 + (j - 4));
}

__host__ __device__ constexpr size_t kfrag_index(int key, int d) {
  // element index inside one (layer, batch) K block
  return ((size_t)(key >> 4) * 8 + (d >> 5)) * 512 + (size_t)(((d & 31) >> 3) * 16 + (key & 15)) * 8 + (d & 7);
}

__host__ __device__ constexpr size_t vfrag_index(int key, int d) {
  // inverse of vkey(): key -> (kb, g, j)
  int kb = key >> 5, r = key & 31;
  int g = (r & 15) >> 2;
  int j = (r < 16) ? (r & 3) : 4 + (r & 3);
  return ((size_t)kb * 16 + (d >> 4)) * 512 + (size_t)(g * 16 + (d & 15)) * 8 + j;
}

}  // namespace pi05
