// The pi0.5 vision tower on gfx950: SigLIP So400m/14 + PaliGemma's projector (get_image_features,
// gemma_pytorch.py:106-107; the tower itself is transformers' SiglipVisionModel).  Per image:
//   patches (fp32 im2col) . Wpatch^T          hipBLASLt fp32 GEMM
//   h = bf16(conv + bpatch + pos)              embed_kernel
//   27 x [ n = LN1(h); q|k|v = n.W^T + b      hipBLASLt (bias epilogue)
//          attention, 16 heads of 72          vision_attn_kernel (MFMA, K/V staged in LDS)
//          h = bf16(h + o.Wo^T + bo); n = LN2 hipBLASLt (split-K when faster) + layernorm_kernel
//          a = gelu_tanh(n.W1^T + b1)          hipBLASLt + gelu_kernel
//          h = bf16(h + a.W2^T + b2) ]         hipBLASLt (split-K when faster) + layernorm_kernel
//                                              (the next LN1 / post_layernorm)
//   out = (n.Wproj^T + bproj) * out_scale     hipBLASLt (+ scale_kernel)
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "pi05_blocks.h"
#include "pi05_gemm.h"
#include "pi05_siglip.h"

namespace pi05 {
namespace {

constexpr int kVW = 1152, kVH = 16, kVD = 72, kVI = 4304, kVPatch = 14, kVImg = 224, kVC = 3, kVProj = 2048;
// the MLP's hidden dim padded to 4352 = 64 x 68 in the fc1 output and the fc2 weight rows (the pad
// columns stay zero: gelu(0) = 0 and zero products add exactly nothing), so fc2 splits into 4 or 8
// K slices of 16-byte-aligned width
constexpr int kVIp = 4352;
constexpr int kVGrid = kVImg / kVPatch, kVS = kVGrid * kVGrid;  // 16 x 16 = 256 patches
constexpr int kVPD = kVC * kVPatch * kVPatch;                   // 588 values per patch
constexpr int kVQkvN = 3 * kVW;                                 // 3456 fused q|k|v columns
// attention operands, per (image, head): head dim padded to 96 for Q.K^T (3 k-steps of 32) and to
// 80 for P.V (5 d-tiles of 16); the padding stays zero
constexpr int kVKs = 3, kVDt = 5;
// per-layer packed bf16 weights: [Wq; Wk; Wv] | Wo | W1 | W2; fp32 parameters: bqkv | bo | b1 | b2 |
// ln1w | ln1b | ln2w | ln2b
constexpr size_t kVOffQkv = 0, kVOffO = kVOffQkv + (size_t)kVQkvN * kVW, kVOff1 = kVOffO + (size_t)kVW * kVW,
                 kVOff2 = kVOff1 + (size_t)kVI * kVW, kVLayerElems = kVOff2 + (size_t)kVW * kVIp;
constexpr size_t kVPOffBqkv = 0, kVPOffBo = kVQkvN, kVPOffB1 = kVPOffBo + kVW, kVPOffB2 = kVPOffB1 + kVI,
                 kVPOffLn1w = kVPOffB2 + kVW, kVPOffLn1b = kVPOffLn1w + kVW, kVPOffLn2w = kVPOffLn1b + kVW,
                 kVPOffLn2b = kVPOffLn2w + kVW, kVLayerParams = kVPOffLn2b + kVW;
constexpr size_t kVWorkspace = 32ull << 20;
constexpr int kVMaxSplits = 8;  // split-K candidates: 4 and 8 K slices (out_proj, fc2); 2 and 3 (fc1)

thread_local std::string g_vision_err;

// Attention operands in LDS, per (image, head): K over 96 padded head dims as the A operand of
// S^T = K Q^T (fragment (key tile, d-step)), V over 80 padded dims as the A operand of
// O^T = V^T P^T (fragment (key block, d-tile)) with the 32-key permutation vkey, so the P^T operand
// is the S^T accumulator a lane already holds.  The padding dims are zero.
constexpr int kVKFrags = (kVS / 16) * kVKs, kVVFrags = (kVS / 32) * kVDt;
// V fragments in LDS carry 16 bytes of padding after each 16-lane group (a fragment = 4 groups of
// 272 bytes), so the transposing 2-byte stores of one wave spread over 32 banks
constexpr int kVVGroup = 136, kVVFrag = 4 * kVVGroup;  // in bf16 elements

// im2col: patches[(n, p)][c*196 + ky*14 + kx] = pixels[n][c][14 py + ky][14 px + kx], p = 16 py + px
__global__ __launch_bounds__(256) void im2col_kernel(const float* px, float* patches, int n_img) {
  const size_t total = (size_t)n_img * kVS * kVPD;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const size_t row = i / kVPD;
    const int col = (int)(i % kVPD), n = (int)(row / kVS), p = (int)(row % kVS);
    const int c = col / (kVPatch * kVPatch), ky = (col / kVPatch) % kVPatch, kx = col % kVPatch;
    const int y = (p / kVGrid) * kVPatch + ky, x = (p % kVGrid) * kVPatch + kx;
    patches[i] = px[(((size_t)n * kVC + c) * kVImg + y) * kVImg + x];
  }
}

// h = bf16(conv + patch bias + position embedding) (SiglipVisionEmbeddings, fp32 until here)
__global__ __launch_bounds__(256) void embed_kernel(const float* conv, const float* pb, const float* pos, u16* h, size_t total) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const int c = (int)(i % kVW), p = (int)((i / kVW) % kVS);
    h[i] = f2bf(conv[i] + pb[c] + pos[(size_t)p * kVW + c]);
  }
}

// h = bf16(x + y), n = bf16((h - mean) / sqrt(var + eps) * w + b) with fp32 statistics
// (nn.LayerNorm after the residual add).  y is the bf16 Linear output, or (ys != null) the Linear
// as nsplit fp32 split-K partials reduced here: y = bf16(sum + ybias); neither: h = x.  One wave
// per 1152-wide row (9 pairs of bf16 per lane), 4 rows per workgroup.
__global__ __launch_bounds__(256) void layernorm_kernel(const u16* x, const u16* y, const float* ys, int nsplit, size_t split_stride,
                                                       const float* ybias, const float* w, const float* b, u16* h_out, u16* n_out,
                                                       float eps, int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const size_t ro = (size_t)row * kVW;
  // every load of the row is issued before the first use, the norm's weight and bias included
  float2 wv[9], bv[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    wv[j] = *reinterpret_cast<const float2*>(w + 2 * (lane + 64 * j));
    bv[j] = *reinterpret_cast<const float2*>(b + 2 * (lane + 64 * j));
  }
  uint32_t xv[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) xv[j] = *reinterpret_cast<const uint32_t*>(x + ro + 2 * (lane + 64 * j));
  float h[18];
#pragma unroll
  for (int j = 0; j < 9; ++j) h[2 * j] = bf2f((u16)(xv[j] & 0xffff)), h[2 * j + 1] = bf2f((u16)(xv[j] >> 16));
  if (ys) {
    // every split's partial row is loaded before the first sum (the splits are summed in order, as
    // before): a loop that waited for each split's loads in turn paid one memory round trip per split
    float2 acc[9], a[kVMaxSplits - 1][9], yb[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      acc[j] = *reinterpret_cast<const float2*>(ys + ro + 2 * (lane + 64 * j));
      yb[j] = *reinterpret_cast<const float2*>(ybias + 2 * (lane + 64 * j));
    }
#pragma unroll
    for (int sp = 1; sp < kVMaxSplits; ++sp)
      if (sp < nsplit)
#pragma unroll
        for (int j = 0; j < 9; ++j) a[sp - 1][j] = *reinterpret_cast<const float2*>(ys + (size_t)sp * split_stride + ro + 2 * (lane + 64 * j));
#pragma unroll
    for (int sp = 1; sp < kVMaxSplits; ++sp)
      if (sp < nsplit)
#pragma unroll
        for (int j = 0; j < 9; ++j) acc[j].x += a[sp - 1][j].x, acc[j].y += a[sp - 1][j].y;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      h[2 * j] = round_bf(fadd(h[2 * j], round_bf(fadd(acc[j].x, yb[j].x))));
      h[2 * j + 1] = round_bf(fadd(h[2 * j + 1], round_bf(fadd(acc[j].y, yb[j].y))));
    }
  } else if (y) {
    uint32_t yv[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) yv[j] = *reinterpret_cast<const uint32_t*>(y + ro + 2 * (lane + 64 * j));
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      h[2 * j] = round_bf(fadd(h[2 * j], bf2f((u16)(yv[j] & 0xffff))));
      h[2 * j + 1] = round_bf(fadd(h[2 * j + 1], bf2f((u16)(yv[j] >> 16))));
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 18; ++i) s += h[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = s * (1.0f / kVW);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 18; ++i) q += (h[i] - mean) * (h[i] - mean);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
  const float rstd = 1.0f / sqrtf(q * (1.0f / kVW) + eps);
  const bool write_h = (y || ys) && h_out;
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    const int e = 2 * (lane + 64 * j);
    const u16 n0 = f2bf(fadd(fmul(fmul(fsub(h[2 * j], mean), rstd), wv[j].x), bv[j].x));
    const u16 n1 = f2bf(fadd(fmul(fmul(fsub(h[2 * j + 1], mean), rstd), wv[j].y), bv[j].y));
    *reinterpret_cast<uint32_t*>(n_out + ro + e) = (uint32_t)n0 | ((uint32_t)n1 << 16);
    if (write_h) *reinterpret_cast<uint32_t*>(h_out + ro + e) = (uint32_t)f2bf(h[2 * j]) | ((uint32_t)f2bf(h[2 * j + 1]) << 16);
  }
}

// MHA over one image's 256 patches, straight from the fused q|k|v GEMM output [M, 3456]:
// workgroup = (image, head, half of the queries), 8 waves (two per SIMD, so one wave's softmax
// overlaps the other's MFMAs).  The workgroup stages the head's K and V for all 256 keys into LDS
// in fragment order (16-byte global loads of 8 head dims of one key); wave w loads its query m-tile
// 8 half + w as B fragments straight from global memory and streams the
// 8 key blocks of 32 through the online-softmax update: fp32 scores scaled by 72^-0.5 (no bf16
// rounding of the scores: the reference runs SDPA's flash kernel), P rounded to bf16 for P.V.
constexpr int kVAttnWaves = 8, kVKPass = (kVS / 16) * kVKs / kVAttnWaves, kVVPass = (kVS / 32) * kVDt / kVAttnWaves;

__global__ __launch_bounds__(512) void vision_attn_kernel(const u16* qkv, u16* out) {
  __shared__ __align__(16) u16 s_k[kVKFrags * 512];
  __shared__ __align__(16) u16 s_v[kVVFrags * kVVFrag];
  const int half = blockIdx.x & 1, head = (blockIdx.x >> 1) % kVH, n = (blockIdx.x >> 1) / kVH;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, mt = half * kVAttnWaves + wave;
  const u16* base = qkv + (size_t)n * kVS * kVQkvN + head * kVD;  // row r of the image: q | k | v at +0 | +W | +2W
  const u16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  static_assert(kVKPass * kVAttnWaves == (kVS / 16) * kVKs && kVVPass * kVAttnWaves == (kVS / 32) * kVDt, "staging passes");
  // K: pass (wave, t) fills fragment f = 6 wave + t = (key tile f / 3, d-step f % 3) whole: lane l
  // loads dims 8 (4 (f % 3) + l / 16) .. +7 of key 16 (f / 3) + l % 16 (zero beyond dim 72) and
  // stores them at its own 16-byte slot, so each 16-lane store group covers all banks once.
  // V: pass (wave, t) = combo 5 wave + t = (key block combo / 5, chunk pair combo % 5): lanes 0-31
  // load the even chunk, lanes 32-63 the odd chunk of the block's 32 keys; element (key r, dim d)
  // goes to fragment (r / 32, d / 16), group g, lane d % 16, slot j (vkey's inverse).
  u16x8 kv[kVKPass], vv[kVVPass];  // every global load is issued before the first LDS store
#pragma unroll
  for (int t = 0; t < kVKPass; ++t) {
    const int f = wave * kVKPass + t, r = (f / 3) * 16 + (lane & 15), c = (f % 3) * 4 + (lane >> 4);
    kv[t] = c < 9 ? *reinterpret_cast<const u16x8*>(base + (size_t)r * kVQkvN + kVW + c * 8) : zero;
  }
#pragma unroll
  for (int t = 0; t < kVVPass; ++t) {
    const int combo = wave * kVVPass + t, r = (combo / 5) * 32 + (lane & 31), c = (combo % 5) * 2 + (lane >> 5);
    vv[t] = c < 9 ? *reinterpret_cast<const u16x8*>(base + (size_t)r * kVQkvN + 2 * kVW + c * 8) : zero;
  }
#pragma unroll
  for (int t = 0; t < kVKPass; ++t) *reinterpret_cast<u16x8*>(s_k + (wave * kVKPass + t) * 512 + lane * 8) = kv[t];
#pragma unroll
  for (int t = 0; t < kVVPass; ++t) {
    const int combo = wave * kVVPass + t, r = lane & 31, c = (combo % 5) * 2 + (lane >> 5);
    const int g = (r & 15) >> 2, j = r < 16 ? (r & 3) : 4 + (r & 3);
    u16* dst = s_v + ((combo / 5) * kVDt + (c >> 1)) * kVVFrag + g * kVVGroup + (c & 1) * 64 + j;
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e * 8] = vv[t][e];
  }
  bf16x8 q[kVKs];
  const u16* qrow = base + (size_t)(mt * 16 + (lane & 15)) * kVQkvN;
#pragma unroll
  for (int ds = 0; ds < kVKs; ++ds) {
    const int d = ds * 32 + (lane >> 4) * 8;
    q[ds] = d < kVD ? load_frag(qrow + d) : zero_frag();
  }
  __syncthreads();
  const float scale = 0.11785113019775793f;  // 72 ** -0.5
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[kVDt];
#pragma unroll
  for (int d = 0; d < kVDt; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int blk = 0; blk < kVS / 32; ++blk) {
    bf16x8 k[2 * kVKs], v[kVDt];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ds = 0; ds < kVKs; ++ds) k[t * kVKs + ds] = load_frag(s_k + ((2 * blk + t) * kVKs + ds) * 512 + lane * 8);
#pragma unroll
    for (int dt = 0; dt < kVDt; ++dt) v[dt] = load_frag(s_v + (blk * kVDt + dt) * kVVFrag + (lane >> 4) * kVVGroup + (lane & 15) * 8);
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ds = 0; ds < kVKs; ++ds)
#pragma unroll
      for (int t = 0; t < 2; ++t) sacc[t] = mfma16x16x32(k[t * kVKs + ds], q[ds], sacc[t]);
    float s[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = sacc[0][i] * scale;
      s[4 + i] = sacc[1][i] * scale;
    }
    float bm = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) bm = fmaxf(bm, s[i]);
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float m_new = fmaxf(m_run, bm);
    const float alpha = __expf(m_run - m_new);  // m_run = -inf on the first block: alpha = 0
    float e[8], esum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      e[i] = __expf(s[i] - m_new);
      esum += e[i];
    }
    l_run = l_run * alpha + esum;
    m_run = m_new;
    u16x8 pf;
#pragma unroll
    for (int i = 0; i < 8; ++i) pf[i] = f2bf(e[i]);
    const bf16x8 pfrag = as_bf16x8(pf);
#pragma unroll
    for (int dt = 0; dt < kVDt; ++dt) oacc[dt] = mfma16x16x32(v[dt], pfrag, oacc[dt] * alpha);
  }
  float l = l_run;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  const float inv = 1.0f / l;
  const int tok = mt * 16 + (lane & 15), g = lane >> 4;
  u16* orow = out + ((size_t)n * kVS + tok) * kVW + head * kVD;
#pragma unroll
  for (int dt = 0; dt < kVDt; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dt * 16 + g * 4 + i;
      if (d < kVD) orow[d] = f2bf(oacc[dt][i] * inv);
    }
}

// bf16(gelu_tanh(x)) in place (transformers' gelu_pytorch_tanh on the bf16 fc1 output)
// (8 elements per thread over the padded rows; chunks = elements / 8)
__global__ __launch_bounds__(256) void gelu_kernel(u16* x, size_t chunks) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (size_t)gridDim.x * 256) {
    u16x8 v = *reinterpret_cast<const u16x8*>(x + i * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f2bf(gelu_tanh(bf2f(v[e])));
    *reinterpret_cast<u16x8*>(x + i * 8) = v;
  }
}

// act = bf16(gelu_tanh(bf16(sum of nsplit fp32 fc1 partials + b1))): fc1 run as a split-K GEMM,
// reduced here with its bias and the one rounding a GEMM epilogue would apply; the pad columns of
// the 4352-wide rows are written as zeros.
__global__ __launch_bounds__(256) void gelu_split_kernel(const float* part, int nsplit, size_t split_stride, const float* bias, u16* act,
                                                        size_t chunks) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (size_t)gridDim.x * 256) {
    const int col = (int)((i * 8) % kVIp);
    u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (col < kVI) {
      float a[8];
      const float4 p0 = *reinterpret_cast<const float4*>(part + i * 8), p1 = *reinterpret_cast<const float4*>(part + i * 8 + 4);
      a[0] = p0.x, a[1] = p0.y, a[2] = p0.z, a[3] = p0.w, a[4] = p1.x, a[5] = p1.y, a[6] = p1.z, a[7] = p1.w;
      for (int sp = 1; sp < nsplit; ++sp) {
        const float* q = part + (size_t)sp * split_stride + i * 8;
        const float4 q0 = *reinterpret_cast<const float4*>(q), q1 = *reinterpret_cast<const float4*>(q + 4);
        a[0] += q0.x, a[1] += q0.y, a[2] += q0.z, a[3] += q0.w, a[4] += q1.x, a[5] += q1.y, a[6] += q1.z, a[7] += q1.w;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = f2bf(gelu_tanh(round_bf(fadd(a[e], bias[col + e]))));
    }
    *reinterpret_cast<u16x8*>(act + i * 8) = v;
  }
}

__global__ __launch_bounds__(256) void scale_kernel(u16* x, size_t total, float s) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) x[i] = f2bf(bf2f(x[i]) * s);
}

__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const u16* src, float* dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = bf2f(src[i]);
}

struct VLayerBind {
  const void* p[16] = {};  // wq bq wk bk wv bv wo bo w1 b1 w2 b2 ln1w ln1b ln2w ln2b
};

struct VisionPlan {
  int L = 0, N = 0, M = 0;
  size_t w, par, head, h, qkv, act, part, patches, conv, ws;
  size_t total() const { return w + par + head + 4 * h + qkv + act + part + patches + conv + ws + 16 * 256; }
};

size_t vrup(size_t x) { return (x + 255) / 256 * 256; }

VisionPlan vplan_of(const pi05_vision_dims& d) {
  VisionPlan p;
  p.L = d.depth, p.N = d.n_images, p.M = d.n_images * kVS;
  const size_t M = p.M;
  p.w = vrup((size_t)p.L * kVLayerElems * 2);
  p.par = vrup((size_t)p.L * kVLayerParams * 4);
  // heads: patch_w [W, 588] + patch_b + pos [256, W] + post w/b (fp32), proj_w bf16, proj_b fp32
  p.head = vrup(((size_t)kVW * kVPD + kVW + (size_t)kVS * kVW + 2 * kVW + kVProj) * 4 + (size_t)kVProj * kVW * 2);
  p.h = vrup(M * kVW * 2);
  p.qkv = vrup(M * kVQkvN * 2);
  p.part = vrup(std::max((size_t)kVMaxSplits * M * kVW, (size_t)3 * M * kVIp) * 4);
  p.act = vrup(M * kVIp * 2);
  p.patches = vrup(M * kVPD * 4);
  p.conv = vrup(M * kVW * 4);
  p.ws = kVWorkspace;
  return p;
}

bool check_vision_dims(const pi05_vision_dims* d, std::string* m) {
  if (!d) {
    *m = "dims is NULL";
    return false;
  }
  if (d->width != kVW || d->num_heads != kVH || d->mlp_dim != kVI || d->patch != kVPatch || d->image != kVImg || d->channels != kVC ||
      d->proj_dim != kVProj) {
    *m = "vision geometry must be width 1152, 16 heads, mlp_dim 4304, patch 14, image 224, 3 channels, proj_dim 2048";
    return false;
  }
  if (d->depth < 1 || d->depth > 64 || d->n_images < 1 || d->n_images > 64) {
    *m = "depth must be in [1, 64] and n_images in [1, 64]";
    return false;
  }
  if (!(d->ln_eps > 0.f) || !(d->out_scale > 0.f)) {
    *m = "ln_eps and out_scale must be > 0";
    return false;
  }
  return true;
}

GemmOpts split_opts(int nsplit, int ld_k) {
  GemmOpts o;
  o.batch = nsplit;
  o.ld_k = ld_k;
  return o;
}

unsigned grid_for(size_t total) {
  const size_t g = (total + 255) / 256;
  return (unsigned)(g < 8192 ? g : 8192);
}

}  // namespace
}  // namespace pi05

using namespace pi05;

struct pi05_vision_ctx {
  pi05_vision_dims d{};
  VisionPlan plan;
  std::string err;
  std::vector<VLayerBind> binds;
  const float *b_patch_w = nullptr, *b_patch_b = nullptr, *b_pos = nullptr;
  const void *b_post_w = nullptr, *b_post_b = nullptr, *b_proj_w = nullptr, *b_proj_b = nullptr;
  bool refreshed = false;
  char* base = nullptr;
  u16 *w = nullptr, *h = nullptr, *n = nullptr, *y = nullptr, *attn = nullptr, *qkv = nullptr, *act = nullptr, *proj_w = nullptr;
  float *par = nullptr, *patch_w = nullptr, *patch_b = nullptr, *pos = nullptr, *post_w = nullptr, *post_b = nullptr, *proj_b = nullptr,
        *part = nullptr, *patches = nullptr, *conv = nullptr;
  void* ws = nullptr;
  hipblasLtHandle_t lt = nullptr;
  GemmPlan g_patch, g_qkv, g_o, g_fc1, g_fc2, g_proj;
  // out_proj / fc2 as fp32 split-K GEMMs (4 or 8 K slices) reduced in the LayerNorm, when faster
  GemmPlan g_osk[2], g_fc2sk[2];
  GemmPlan g_fc1sk[2];  // fc1 as 2 or 3 fp32 split-K GEMMs reduced (+ bias, GELU) in gelu_split_kernel
  int o_split = 0, fc2_split = 0, fc1_split = 0;  // chosen slice count (0: the single bf16 GEMM with its bias)
};

namespace {

int vfail(pi05_vision_ctx* c, int code, const std::string& m) {
  if (c) c->err = m;
  else g_vision_err = m;
  return code;
}

int vgemm(pi05_vision_ctx* c, const GemmPlan& p, const void* W, const void* A, void* C, const float* bias, hipStream_t st) {
  const hipblasStatus_t s = run_plan(c->lt, p, p.algo, p.ws, W, A, C, bias, c->ws, st);
  if (!lt_ok(s)) return vfail(c, PI05_E_HIP, "hipblasLtMatmul failed (status " + std::to_string((int)s) + ")");
  return PI05_OK;
}

}  // namespace

extern "C" {

void pi05_vision_default_dims(pi05_vision_dims* d) {
  if (!d) return;
  *d = pi05_vision_dims{kVW, 27, kVH, kVI, kVPatch, kVImg, kVC, kVProj, 3, 1e-6f, 1.0f};
}

int pi05_vision_check_dims(const pi05_vision_dims* dims) {
  std::string m;
  if (!check_vision_dims(dims, &m)) return vfail(nullptr, PI05_E_INVALID, m);
  return PI05_OK;
}

size_t pi05_vision_device_bytes(const pi05_vision_dims* dims) {
  std::string m;
  if (!check_vision_dims(dims, &m)) return 0;
  return vplan_of(*dims).total();
}

const char* pi05_vision_last_error(const pi05_vision_ctx* ctx) { return ctx ? ctx->err.c_str() : g_vision_err.c_str(); }

int pi05_vision_create(const pi05_vision_dims* dims, pi05_vision_ctx** out) {
  if (!out) return vfail(nullptr, PI05_E_INVALID, "out is NULL");
  *out = nullptr;
  std::string m;
  if (!check_vision_dims(dims, &m)) return vfail(nullptr, PI05_E_INVALID, m);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return vfail(nullptr, PI05_E_NODEVICE, std::string("no HIP device: ") + hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return vfail(nullptr, PI05_E_NODEVICE, std::string("device is not gfx950 (MI355X): ") + (e == hipSuccess ? prop.gcnArchName : hipGetErrorString(e)));
  pi05_vision_ctx* c = new pi05_vision_ctx();
  c->d = *dims;
  c->plan = vplan_of(*dims);
  c->binds.resize(dims->depth);
  const VisionPlan& p = c->plan;
  e = hipMalloc(&c->base, p.total());
  if (e != hipSuccess) {
    delete c;
    return vfail(nullptr, PI05_E_NOMEM, std::string("vision context allocation failed: ") + hipGetErrorString(e));
  }
  char* q = c->base;
  auto take = [&](size_t bytes) {
    char* r = q;
    q += bytes;
    return r;
  };
  c->w = reinterpret_cast<u16*>(take(p.w));
  c->par = reinterpret_cast<float*>(take(p.par));
  char* hd = take(p.head);
  c->patch_w = reinterpret_cast<float*>(hd);
  c->patch_b = c->patch_w + (size_t)kVW * kVPD;
  c->pos = c->patch_b + kVW;
  c->post_w = c->pos + (size_t)kVS * kVW;
  c->post_b = c->post_w + kVW;
  c->proj_b = c->post_b + kVW;
  c->proj_w = reinterpret_cast<u16*>(c->proj_b + kVProj);
  c->h = reinterpret_cast<u16*>(take(p.h));
  c->n = reinterpret_cast<u16*>(take(p.h));
  c->y = reinterpret_cast<u16*>(take(p.h));
  c->attn = reinterpret_cast<u16*>(take(p.h));
  c->qkv = reinterpret_cast<u16*>(take(p.qkv));
  c->act = reinterpret_cast<u16*>(take(p.act));
  c->part = reinterpret_cast<float*>(take(p.part));
  c->patches = reinterpret_cast<float*>(take(p.patches));
  c->conv = reinterpret_cast<float*>(take(p.conv));
  c->ws = take(p.ws);
  // zeroed once: tuning reads defined data
  e = hipMemset(c->base, 0, p.total());
  if (e != hipSuccess) {
    hipFree(c->base);
    delete c;
    return vfail(nullptr, PI05_E_HIP, std::string("vision context initialisation failed: ") + hipGetErrorString(e));
  }
  std::string perr;
  const int M = p.M;
  GemmOpts f32;
  f32.ab = HIP_R_32F;
  f32.c = HIP_R_32F;
  GemmOpts bias;
  bias.bias = true;
  GemmOpts fc1o = bias;
  fc1o.ld_c = kVIp;
  GemmOpts fc2o = bias;
  fc2o.ld_k = kVIp;
  constexpr int splits[2] = {4, 8};
  static_assert(splits[0] <= kVMaxSplits && splits[1] <= kVMaxSplits, "layernorm_kernel reduces at most kVMaxSplits slices");
  bool ok = lt_ok(hipblasLtCreate(&c->lt)) && make_plan(c->lt, M, kVW, kVPD, kVWorkspace, &c->g_patch, &perr, f32) &&
            make_plan(c->lt, M, kVQkvN, kVW, kVWorkspace, &c->g_qkv, &perr, bias) && make_plan(c->lt, M, kVW, kVW, kVWorkspace, &c->g_o, &perr, bias) &&
            make_plan(c->lt, M, kVI, kVW, kVWorkspace, &c->g_fc1, &perr, fc1o) && make_plan(c->lt, M, kVW, kVIp, kVWorkspace, &c->g_fc2, &perr, fc2o) &&
            make_plan(c->lt, M, kVProj, kVW, kVWorkspace, &c->g_proj, &perr, bias);
  const int fc1_splits[2] = {2, 3};
  for (int i = 0; i < 2 && ok; ++i) {
    GemmOpts f1 = split_opts(fc1_splits[i], kVW);
    f1.ld_c = kVIp;
    ok = make_plan(c->lt, M, kVW, kVW / splits[i], kVWorkspace, &c->g_osk[i], &perr, split_opts(splits[i], kVW)) &&
         make_plan(c->lt, M, kVW, kVIp / splits[i], kVWorkspace, &c->g_fc2sk[i], &perr, split_opts(splits[i], kVIp)) &&
         make_plan(c->lt, M, kVI, kVW / fc1_splits[i], kVWorkspace, &c->g_fc1sk[i], &perr, f1);
  }
  if (ok) {
    const float* bz = c->par;  // any fp32 vector long enough (zeros) stands in for the biases while timing
    // (weights rotate over the layers' blocks while timing, as the layer loop streams them)
    const size_t ls = kVLayerElems * 2;
    const int nl = p.L;
    ok = tune_plan(c->lt, &c->g_patch, c->patch_w, c->patches, c->conv, c->ws, nullptr) &&
         tune_plan(c->lt, &c->g_qkv, c->w, c->n, c->qkv, c->ws, nullptr, bz, ls, nl) &&
         tune_plan(c->lt, &c->g_o, c->w, c->attn, c->y, c->ws, nullptr, bz, ls, nl) &&
         tune_plan(c->lt, &c->g_fc1, c->w, c->n, c->act, c->ws, nullptr, bz, ls, nl) &&
         tune_plan(c->lt, &c->g_fc2, c->w, c->act, c->y, c->ws, nullptr, bz, ls, nl) &&
         tune_plan(c->lt, &c->g_proj, c->proj_w, c->n, c->act, c->ws, nullptr, bz);
    for (int i = 0; i < 2 && ok; ++i)
      ok = tune_plan(c->lt, &c->g_osk[i], c->w, c->attn, c->part, c->ws, nullptr, nullptr, ls, nl) &&
           tune_plan(c->lt, &c->g_fc2sk[i], c->w, c->act, c->part, c->ws, nullptr, nullptr, ls, nl) &&
           tune_plan(c->lt, &c->g_fc1sk[i], c->w, c->n, c->part, c->ws, nullptr, nullptr, ls, nl);
    if (!ok && perr.empty()) perr = "GEMM algorithm tuning failed";
    // split-K when the split GEMM plus the partials' extra traffic through the LayerNorm
    // ((4 nsplit - 2) bytes per output element at ~4 TB/s) beats the single bf16 GEMM
    auto extra_ms = [&](int ns) { return (float)((double)(4 * ns - 2) * M * kVW / 4e12 * 1e3); };
    float best_o = c->g_o.ms, best_2 = c->g_fc2.ms, best_1 = c->g_fc1.ms;
    for (int i = 0; i < 2 && ok; ++i) {
      // fc1: the partials replace the bf16 output that the GELU reads anyway
      const float x1 = (float)((double)(4 * fc1_splits[i] - 2) * M * kVIp / 4e12 * 1e3);
      if (c->g_fc1sk[i].ms + x1 < best_1) best_1 = c->g_fc1sk[i].ms + x1, c->fc1_split = fc1_splits[i];
      if (c->g_osk[i].ms + extra_ms(splits[i]) < best_o) best_o = c->g_osk[i].ms + extra_ms(splits[i]), c->o_split = splits[i];
      if (c->g_fc2sk[i].ms + extra_ms(splits[i]) < best_2) best_2 = c->g_fc2sk[i].ms + extra_ms(splits[i]), c->fc2_split = splits[i];
    }
  }
  if (!ok) {
    if (perr.empty()) perr = "hipblasLtCreate failed";
    pi05_vision_destroy(c);
    return vfail(nullptr, PI05_E_HIP, perr);
  }
  *out = c;
  return PI05_OK;
}

int pi05_vision_destroy(pi05_vision_ctx* c) {
  if (!c) return PI05_OK;
  for (GemmPlan* g : {&c->g_patch, &c->g_qkv, &c->g_o, &c->g_fc1, &c->g_fc2, &c->g_proj, &c->g_osk[0], &c->g_osk[1], &c->g_fc2sk[0],
                      &c->g_fc2sk[1], &c->g_fc1sk[0], &c->g_fc1sk[1]})
    free_plan(g);
  if (c->lt) hipblasLtDestroy(c->lt);
  if (c->base) hipFree(c->base);
  delete c;
  return PI05_OK;
}

int pi05_vision_bind_layer(pi05_vision_ctx* c, int layer, const void* wq, const void* bq, const void* wk, const void* bk, const void* wv,
                           const void* bv, const void* wo, const void* bo, const void* w1, const void* b1, const void* w2, const void* b2,
                           const void* ln1_w, const void* ln1_b, const void* ln2_w, const void* ln2_b) {
  if (!c) return vfail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (layer < 0 || layer >= c->d.depth) return vfail(c, PI05_E_INVALID, "layer out of range");
  const void* ps[16] = {wq, bq, wk, bk, wv, bv, wo, bo, w1, b1, w2, b2, ln1_w, ln1_b, ln2_w, ln2_b};
  VLayerBind b;
  for (int i = 0; i < 16; ++i) {
    if (!ps[i]) return vfail(c, PI05_E_INVALID, "a weight pointer is NULL");
    if (reinterpret_cast<uintptr_t>(ps[i]) % 16) return vfail(c, PI05_E_INVALID, "weight pointers must be 16-byte aligned");
    b.p[i] = ps[i];
  }
  c->binds[layer] = b;
  c->refreshed = false;
  return PI05_OK;
}

int pi05_vision_bind_heads(pi05_vision_ctx* c, const float* patch_w, const float* patch_b, const float* pos, const void* post_w,
                           const void* post_b, const void* proj_w, const void* proj_b) {
  if (!c) return vfail(nullptr, PI05_E_INVALID, "ctx is NULL");
  const void* ps[7] = {patch_w, patch_b, pos, post_w, post_b, proj_w, proj_b};
  for (const void* x : ps) {
    if (!x) return vfail(c, PI05_E_INVALID, "a weight pointer is NULL");
    if (reinterpret_cast<uintptr_t>(x) % 16) return vfail(c, PI05_E_INVALID, "weight pointers must be 16-byte aligned");
  }
  c->b_patch_w = patch_w, c->b_patch_b = patch_b, c->b_pos = pos;
  c->b_post_w = post_w, c->b_post_b = post_b, c->b_proj_w = proj_w, c->b_proj_b = proj_b;
  c->refreshed = false;
  return PI05_OK;
}

int pi05_vision_refresh_weights(pi05_vision_ctx* c, void* stream) {
  if (!c) return vfail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (!c->b_patch_w) return vfail(c, PI05_E_STATE, "heads are not bound");
  for (int l = 0; l < c->d.depth; ++l)
    if (!c->binds[l].p[0]) return vfail(c, PI05_E_STATE, "layer " + std::to_string(l) + " is not bound");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipMemcpyKind k = hipMemcpyDeviceToDevice;
  hipError_t e = hipSuccess;
  auto to_f32 = [&](const void* src, float* dst, size_t n) {
    bf16_to_f32_kernel<<<grid_for(n), 256, 0, st>>>(static_cast<const u16*>(src), dst, n);
  };
  for (int l = 0; l < c->d.depth && e == hipSuccess; ++l) {
    const VLayerBind& b = c->binds[l];
    u16* w = c->w + (size_t)l * kVLayerElems;
    float* pr = c->par + (size_t)l * kVLayerParams;
    const size_t ww = (size_t)kVW * kVW * 2;
    e = hipMemcpyAsync(w + kVOffQkv, b.p[0], ww, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kVOffQkv + (size_t)kVW * kVW, b.p[2], ww, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kVOffQkv + (size_t)2 * kVW * kVW, b.p[4], ww, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kVOffO, b.p[6], ww, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kVOff1, b.p[8], (size_t)kVI * kVW * 2, k, st);
    if (e == hipSuccess) e = hipMemcpy2DAsync(w + kVOff2, (size_t)kVIp * 2, b.p[10], (size_t)kVI * 2, (size_t)kVI * 2, kVW, k, st);
    to_f32(b.p[1], pr + kVPOffBqkv, kVW);
    to_f32(b.p[3], pr + kVPOffBqkv + kVW, kVW);
    to_f32(b.p[5], pr + kVPOffBqkv + 2 * kVW, kVW);
    to_f32(b.p[7], pr + kVPOffBo, kVW);
    to_f32(b.p[9], pr + kVPOffB1, kVI);
    to_f32(b.p[11], pr + kVPOffB2, kVW);
    to_f32(b.p[12], pr + kVPOffLn1w, kVW);
    to_f32(b.p[13], pr + kVPOffLn1b, kVW);
    to_f32(b.p[14], pr + kVPOffLn2w, kVW);
    to_f32(b.p[15], pr + kVPOffLn2b, kVW);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(c->patch_w, c->b_patch_w, (size_t)kVW * kVPD * 4, k, st);
  if (e == hipSuccess) e = hipMemcpyAsync(c->patch_b, c->b_patch_b, kVW * 4, k, st);
  if (e == hipSuccess) e = hipMemcpyAsync(c->pos, c->b_pos, (size_t)kVS * kVW * 4, k, st);
  if (e == hipSuccess) e = hipMemcpyAsync(c->proj_w, c->b_proj_w, (size_t)kVProj * kVW * 2, k, st);
  if (e == hipSuccess) {
    to_f32(c->b_post_w, c->post_w, kVW);
    to_f32(c->b_post_b, c->post_b, kVW);
    to_f32(c->b_proj_b, c->proj_b, kVProj);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return vfail(c, PI05_E_HIP, std::string("weight packing: ") + hipGetErrorString(e));
  c->refreshed = true;
  return PI05_OK;
}

int pi05_vision_forward(pi05_vision_ctx* c, const float* pixels, void* out, void* stream) {
  if (!c) return vfail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (!pixels || !out) return vfail(c, PI05_E_INVALID, "pixels and out must be non-NULL");
  if (reinterpret_cast<uintptr_t>(out) % 16) return vfail(c, PI05_E_INVALID, "out must be 16-byte aligned");
  if (!c->refreshed) return vfail(c, PI05_E_STATE, "weights are not bound and refreshed");
  const VisionPlan& p = c->plan;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float eps = c->d.ln_eps;
  const size_t M = p.M;
  int rc;
  im2col_kernel<<<grid_for(M * kVPD), 256, 0, st>>>(pixels, c->patches, p.N);
  if ((rc = vgemm(c, c->g_patch, c->patch_w, c->patches, c->conv, nullptr, st)) != PI05_OK) return rc;
  embed_kernel<<<grid_for(M * kVW), 256, 0, st>>>(c->conv, c->patch_b, c->pos, c->h, M * kVW);
  const float* pr0 = c->par;
  const unsigned ln_grid = (unsigned)((M + 3) / 4);
  const size_t pstride = M * kVW;
  layernorm_kernel<<<ln_grid, 256, 0, st>>>(c->h, nullptr, nullptr, 0, 0, nullptr, pr0 + kVPOffLn1w, pr0 + kVPOffLn1b, nullptr, c->n, eps, (int)M);
  for (int l = 0; l < p.L; ++l) {
    const u16* w = c->w + (size_t)l * kVLayerElems;
    const float* pr = c->par + (size_t)l * kVLayerParams;
    if ((rc = vgemm(c, c->g_qkv, w + kVOffQkv, c->n, c->qkv, pr + kVPOffBqkv, st)) != PI05_OK) return rc;
    vision_attn_kernel<<<(unsigned)(p.N * kVH * 2), 512, 0, st>>>(c->qkv, c->attn);
    if (c->o_split) {
      if ((rc = vgemm(c, c->g_osk[c->o_split == 8], w + kVOffO, c->attn, c->part, nullptr, st)) != PI05_OK) return rc;
      layernorm_kernel<<<ln_grid, 256, 0, st>>>(c->h, nullptr, c->part, c->o_split, pstride, pr + kVPOffBo, pr + kVPOffLn2w,
                                                pr + kVPOffLn2b, c->h, c->n, eps, (int)M);
    } else {
      if ((rc = vgemm(c, c->g_o, w + kVOffO, c->attn, c->y, pr + kVPOffBo, st)) != PI05_OK) return rc;
      layernorm_kernel<<<ln_grid, 256, 0, st>>>(c->h, c->y, nullptr, 0, 0, nullptr, pr + kVPOffLn2w, pr + kVPOffLn2b, c->h, c->n, eps,
                                                (int)M);
    }
    if (c->fc1_split) {
      if ((rc = vgemm(c, c->g_fc1sk[c->fc1_split == 3], w + kVOff1, c->n, c->part, nullptr, st)) != PI05_OK) return rc;
      gelu_split_kernel<<<grid_for(M * kVIp / 8), 256, 0, st>>>(c->part, c->fc1_split, M * kVIp, pr + kVPOffB1, c->act, M * kVIp / 8);
    } else {
      if ((rc = vgemm(c, c->g_fc1, w + kVOff1, c->n, c->act, pr + kVPOffB1, st)) != PI05_OK) return rc;
      gelu_kernel<<<grid_for(M * kVIp / 8), 256, 0, st>>>(c->act, M * kVIp / 8);
    }
    const bool last = l + 1 == p.L;
    const float* nw = last ? c->post_w : c->par + (size_t)(l + 1) * kVLayerParams + kVPOffLn1w;
    const float* nb = last ? c->post_b : c->par + (size_t)(l + 1) * kVLayerParams + kVPOffLn1b;
    if (c->fc2_split) {
      if ((rc = vgemm(c, c->g_fc2sk[c->fc2_split == 8], w + kVOff2, c->act, c->part, nullptr, st)) != PI05_OK) return rc;
      layernorm_kernel<<<ln_grid, 256, 0, st>>>(c->h, nullptr, c->part, c->fc2_split, pstride, pr + kVPOffB2, nw, nb, c->h, c->n, eps,
                                                (int)M);
    } else {
      if ((rc = vgemm(c, c->g_fc2, w + kVOff2, c->act, c->y, pr + kVPOffB2, st)) != PI05_OK) return rc;
      layernorm_kernel<<<ln_grid, 256, 0, st>>>(c->h, c->y, nullptr, 0, 0, nullptr, nw, nb, c->h, c->n, eps, (int)M);
    }
  }
  if ((rc = vgemm(c, c->g_proj, c->proj_w, c->n, out, c->proj_b, st)) != PI05_OK) return rc;
  if (c->d.out_scale != 1.0f) scale_kernel<<<grid_for(M * kVProj), 256, 0, st>>>(static_cast<u16*>(out), M * kVProj, c->d.out_scale);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return vfail(c, PI05_E_HIP, std::string("vision launch: ") + hipGetErrorString(e));
  return PI05_OK;
}

}  // extern "C"
