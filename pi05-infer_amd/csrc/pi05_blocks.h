// Device building blocks shared by the denoise kernels: MFMA weight-fragment streaming, the
// cross-wave reduction, GeGLU, and one 32-key block of the MQA online-softmax attention.
#pragma once

#include "pi05_device.h"

namespace pi05 {

enum GemmMode { kModeQkv = 0, kModeGateUp = 1 };

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = kGemmWaves * 64;

template <int NT, int KSW>
__device__ __forceinline__ void load_weights(bf16x8 (&w)[NT][KSW], const u16* const (&tile)[NT], int ks0, int lane) {
#pragma unroll
  for (int s = 0; s < KSW; ++s)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u16x8* p = reinterpret_cast<const u16x8*>(tile[t] + (size_t)(ks0 + s) * 512 + lane * 8);
      w[t][s] = as_bf16x8(__builtin_nontemporal_load(p));
    }
}

template <int NT>
__device__ __forceinline__ void store_partials(float* red, const f32x4 (&acc)[4][NT], int wave, int lane) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<f32x4*>(red + ((((size_t)wave * 4 + mt) * NT + t) * 64 + lane) * 4) = acc[mt][t];
}

// Sum over the 8 waves, in wave order, of the D fragment (m-tile mt, lane) of tile t.
template <int NT>
__device__ __forceinline__ f32x4 reduce_waves(const float* red, int mt, int lane, int t) {
  f32x4 v = *reinterpret_cast<const f32x4*>(red + (((size_t)mt * NT + t) * 64 + lane) * 4);
#pragma unroll
  for (int w = 1; w < kGemmWaves; ++w) v += *reinterpret_cast<const f32x4*>(red + ((((size_t)w * 4 + mt) * NT + t) * 64 + lane) * 4);
  return v;
}

// tanh(u) = 1 - 2 / (e^{2u} + 1), with the hardware exp2 (v_exp_f32) behind __expf and the
// hardware reciprocal (v_rcp_f32, 1 ulp): no branches, saturates to +-1 as e^{2u} overflows to inf
// or underflows to 0.  Its absolute error (a few 1e-7 near u = 0, where the subtraction cancels)
// is what GELU sees, since GELU adds it to 1.
__device__ __forceinline__ float tanh_fast(float u) { return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * u) + 1.0f); }

__device__ __forceinline__ float gelu_tanh(float x) {
  // GELU tanh approximation in the fused reference kernel's op order (rlinf_fused_denoise.py:168-173)
  const float t3 = fmul(x, 0.5f);
  const float t5 = fmul(fmul(x, x), x);
  const float t8 = fadd(x, fmul(t5, 0.044715f));
  const float t11 = tanh_fast(fmul(t8, 0.7978845608028654f));
  return fmul(t3, fadd(t11, 1.0f));
}

// max / sum of x and its value in lane l ^ 16 (rows of 16 lanes swapped pairwise) or l ^ 32
// (wave halves swapped), on the gfx950 permlane swaps: VALU only, where a __shfl_xor is an LDS
// crossbar operation whose lgkmcnt wait would also wait for every LDS read in flight.  The swap
// of two copies of x leaves x in one result and the partner's value in the other (which one
// depends on the lane), so max and sum are order-free and equal to the shuffle's.
__device__ __forceinline__ float lane_max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float lane_sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One 32-key block of K/V fragments (prefetched as a unit) and its key-valid bytes.
struct KvBlock {
  bf16x8 k[16];
  bf16x8 v[16];
  uint32_t valid0, valid1;
};

// kc / vc: fragment-major K / V of the block's key range, kb: block index within it;
// valid: the 32 key-valid bytes of this block.
__device__ __forceinline__ void load_kv_block(KvBlock& blk, const u16* kc, const u16* vc, const uint8_t* valid, int kb, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) blk.k[t * 8 + ds] = load_frag(kc + ((size_t)(2 * kb + t) * 8 + ds) * 512 + lane * 8);
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) blk.v[dt] = load_frag(vc + ((size_t)kb * 16 + dt) * 512 + lane * 8);
  blk.valid0 = *reinterpret_cast<const uint32_t*>(valid + g * 4);
  blk.valid1 = *reinterpret_cast<const uint32_t*>(valid + 16 + g * 4);
}

// One 32-key block of the online-softmax MQA attention for a 16-row query m-tile (2 tokens x 8
// heads sharing the KV head).  S^T = K Q^T on MFMA (two 16-key tiles), scores bf16(q.k) * 1/16
// (exact in bf16) with masked keys at -inf (modeling_gemma.py:265-268), the running max / sum
// update, P rounded to bf16 before P.V, and O^T = V^T P^T accumulated per 16-dim tile; the V
// fragments' key order (vkey) makes P^T exactly the S^T accumulator each lane holds.  qfrag(ds)
// returns the query fragment of d-step ds (from registers or from LDS, as the caller keeps it).
template <class QF>
__device__ __forceinline__ void attend_block_q(const KvBlock& blk, QF qfrag, float& m_run, float& l_run, f32x4 (&oacc)[16]) {
  f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) {
    const bf16x8 qf = qfrag(ds);
#pragma unroll
    for (int t = 0; t < 2; ++t) sacc[t] = mfma16x16x32(blk.k[t * 8 + ds], qf, sacc[t]);
  }
  float s[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = ((blk.valid0 >> (8 * i)) & 0xff) ? round_bf(sacc[0][i]) * 0.0625f : -INFINITY;
    s[4 + i] = ((blk.valid1 >> (8 * i)) & 0xff) ? round_bf(sacc[1][i]) * 0.0625f : -INFINITY;
  }
  float bm = s[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) bm = fmaxf(bm, s[i]);
  bm = lane_max_xor32(lane_max_xor16(bm));
  const float m_new = fmaxf(m_run, bm);
  float alpha = 1.f;
  float e[8];
  if (m_new == -INFINITY) {
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = 0.f;
  } else {
    alpha = __expf(m_run - m_new);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = __expf(s[i] - m_new);
  }
  float esum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) esum += e[i];
  l_run = l_run * alpha + esum;
  m_run = m_new;
  u16x8 pf;
#pragma unroll
  for (int i = 0; i < 8; ++i) pf[i] = f2bf(e[i]);
  const bf16x8 pfrag = as_bf16x8(pf);
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) {
    oacc[dt] *= alpha;
    oacc[dt] = mfma16x16x32(blk.v[dt], pfrag, oacc[dt]);
  }
}

// The same with the query fragments in registers.
__device__ __forceinline__ void attend_block(const KvBlock& blk, const bf16x8 (&qf)[8], float& m_run, float& l_run, f32x4 (&oacc)[16]) {
  attend_block_q(blk, [&](int ds) { return qf[ds]; }, m_run, l_run, oacc);
}

}  // namespace pi05
