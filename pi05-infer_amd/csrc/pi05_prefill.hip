// Prefix-LM prefill on gfx950: PaliGemma's Gemma-2B language model over the prefix embeddings,
// producing the per-layer K/V cache the denoise loop consumes (_build_prefix_cache,
// engine.py:770-794).  Layer l (modeling_gemma.py:460-517):
//   n  = RMSNorm(h)                          rmsnorm_kernel
//   qkv = n . [Wq; Wk; Wv]^T                 hipBLASLt (bf16 in/out, fp32 accumulation)
//   q, k <- RoPE; k, v -> cache              rope_kv_kernel
//   o  = softmax(q k^T / 16 + mask) v        prefix_attn_kernel (MFMA, K/V staged through LDS)
//   h += o . Wo^T; n = RMSNorm(h)            hipBLASLt + rmsnorm_kernel (residual fused)
//   gu = n . [Wg; Wu]^T                      hipBLASLt, N = 32768 in one GEMM
//   a  = gelu_tanh(g) * u                    geglu_kernel
//   h += a . Wd^T; n = RMSNorm(h)            hipBLASLt + rmsnorm_kernel
// The last layer computes only its K/V (patches/prefix_last_layer.py:84-112).  Every valid
// token attends to every valid token of its sample (pi0_pytorch.py:236-250); positions are
// cumsum(pad) - 1 (engine.py:776).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "pi05_blocks.h"
#include "pi05_gemm.h"
#include "pi05_prefill.h"

namespace pi05 {
namespace {

constexpr int kPW = 2048;                    // prefix-LM width
constexpr int kPI = 16384;                   // GeGLU intermediate
constexpr int kPHD = kHeads * kHeadDim;      // 2048 attention output columns
constexpr int kPQkvN = kPHD + 2 * kHeadDim;  // 2560 fused q|k|v columns
constexpr int kPKvN = 2 * kHeadDim;          // 512: k|v columns (the K/V-only last layer)
constexpr int kPGuN = 2 * kPI;               // 32768 fused gate|up columns
// per-layer packed weights (bf16 elements): [q; k; v] | o | [gate; up] | down, nn.Linear layout
constexpr size_t kPOffQkv = 0;
constexpr size_t kPOffO = kPOffQkv + (size_t)kPQkvN * kPW;
constexpr size_t kPOffGu = kPOffO + (size_t)kPW * kPHD;
constexpr size_t kPOffD = kPOffGu + (size_t)kPGuN * kPW;
constexpr size_t kPLayerElems = kPOffD + (size_t)kPW * kPI;
constexpr int kDownSplits = 4;  // down_proj / o_proj split-K candidates: 4 slices of K
constexpr int kAttnMtPerWg = 8;  // attention m-tiles (16 query rows: 2 tokens x 8 heads) per workgroup
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt not waited for (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14])
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);

thread_local std::string g_prefix_err;

// ---------------------------------------------------------------------------------------------
// positions cumsum(pad) - 1 and key-valid bytes of one sample (one workgroup per sample)
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void positions_kernel(const uint8_t* pad, int P, int s_pad, int* pos, uint8_t* valid) {
  const int b = blockIdx.x, t = threadIdx.x;
  __shared__ int s_cnt[256];
  const uint8_t* pb = pad + (size_t)b * P;
  const int per = (P + 255) / 256, p0 = t * per, p1 = p0 + per < P ? p0 + per : P;
  int cnt = 0;
  for (int p = p0; p < p1; ++p) cnt += pb[p] ? 1 : 0;
  s_cnt[t] = cnt;
  __syncthreads();
  // inclusive scan over the 256 chunk counts (Hillis-Steele)
  for (int off = 1; off < 256; off <<= 1) {
    const int v = t >= off ? s_cnt[t - off] : 0;
    __syncthreads();
    s_cnt[t] += v;
    __syncthreads();
  }
  int run = s_cnt[t] - cnt;  // valid tokens before this chunk
  for (int p = p0; p < p1; ++p) {
    run += pb[p] ? 1 : 0;
    pos[(size_t)b * s_pad + p] = run - 1;
  }
  for (int key = t; key < s_pad; key += 256) valid[(size_t)b * s_pad + key] = key < P && pb[key] ? 1 : 0;
}

// ---------------------------------------------------------------------------------------------
// h = bf16(x + y) (y optional), n = bf16(h * rsqrt(mean(h^2) + eps) * (1 + w))
// (modeling_gemma.py:82-99 regular branch; _gated_residual without gate, 231-249).  One
// workgroup per row of 2048: 8 contiguous elements per thread.  h_out may alias x.  With ys, y is
// the bf16 rounding of the sum of nsplit fp32 split-K partials ys[s * split_stride + ...], added
// in split order (the GEMM's own rounding of its full sum).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const u16* x, const u16* y, const float* w, u16* h_out, u16* n_out, float eps,
                                                      const float* ys = nullptr, int nsplit = 0, size_t split_stride = 0) {
  const size_t off = (size_t)blockIdx.x * kPW + threadIdx.x * 8;
  __shared__ float s_part[4];
  // every load is issued before the first use: the norm weight, the row and every split's
  // partial (a loop that waited for each split in turn paid one memory round trip per split)
  const float4 w0 = *reinterpret_cast<const float4*>(w + threadIdx.x * 8);
  const float4 w1 = *reinterpret_cast<const float4*>(w + threadIdx.x * 8 + 4);
  const u16x8 xv = *reinterpret_cast<const u16x8*>(x + off);
  float h[8];
  if (ys) {
    float4 a[kDownSplits][2];
#pragma unroll
    for (int sp = 0; sp < kDownSplits; ++sp)
      if (sp < nsplit) {
        const float* q = ys + (size_t)sp * split_stride + off;
        a[sp][0] = *reinterpret_cast<const float4*>(q), a[sp][1] = *reinterpret_cast<const float4*>(q + 4);
      }
    float acc[8] = {a[0][0].x, a[0][0].y, a[0][0].z, a[0][0].w, a[0][1].x, a[0][1].y, a[0][1].z, a[0][1].w};
#pragma unroll
    for (int sp = 1; sp < kDownSplits; ++sp)
      if (sp < nsplit) {
        acc[0] += a[sp][0].x, acc[1] += a[sp][0].y, acc[2] += a[sp][0].z, acc[3] += a[sp][0].w;
        acc[4] += a[sp][1].x, acc[5] += a[sp][1].y, acc[6] += a[sp][1].z, acc[7] += a[sp][1].w;
      }
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = round_bf(fadd(bf2f(xv[i]), round_bf(acc[i])));
  } else if (y) {
    const u16x8 yv = *reinterpret_cast<const u16x8*>(y + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = round_bf(fadd(bf2f(xv[i]), bf2f(yv[i])));
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = bf2f(xv[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += h[i] * h[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float var = ((s_part[0] + s_part[1]) + (s_part[2] + s_part[3])) * (1.0f / kPW);
  const float rs = 1.0f / sqrtf(var + eps);
  const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  u16x8 hv, nv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    hv[i] = f2bf(h[i]);
    nv[i] = f2bf(fmul(fmul(h[i], rs), fadd(1.0f, wv[i])));
  }
  if ((y || ys) && h_out) *reinterpret_cast<u16x8*>(h_out + off) = hv;
  *reinterpret_cast<u16x8*>(n_out + off) = nv;
}

// ---------------------------------------------------------------------------------------------
// RoPE and the K/V write.  One workgroup per token row (b, p).  qkv row: [q (8 heads x 256) | k |
// v] (ldq = 2560), or [k | v] (ldq = 512, kv_only).  RoPE in fp32 on the bf16 values with bf16
// cos/sin of freq = inv_freq[d mod 128] * pos, rounded once (modeling_gemma.py:169-216): q to the
// attention's A-fragment layout (row = token * 8 + head), k and v to the attention's packed K/V
// block and to the caller's cache [B, 1, P, D].  The cos/sin values depend on the position only
// (a position is in [-1, P): leading pad tokens sit at cumsum - 1 = -1), so rope_table_kernel
// evaluates them once per context into tab[pos + 1][cos 128 | sin 128] (bf16 bits), and the
// per-layer kernel only reads them.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(128) void rope_table_kernel(const float* inv_freq, int P, u16* tab) {
  const int row = blockIdx.x, d = threadIdx.x, pos = row - 1;
  if (row > P) return;
  const float freq = fmul(inv_freq[d], (float)pos);
  tab[(size_t)row * kHeadDim + d] = f2bf(cosf(freq));
  tab[(size_t)row * kHeadDim + kHalfDim + d] = f2bf(sinf(freq));
}

struct RopeKvArgs {
  const u16* qkv;
  int ldq, kv_only, P, s_pad;
  const int* pos;
  const u16* tab;  // [P + 1][cos 128 | sin 128] bf16 bits, row = position + 1
  u16 *qf, *kf, *vf;   // per sample: q fragments [s_pad*8 rows][256], K / V blocks [s_pad keys][256]
  u16 *kout, *vout;    // caller's cache of this layer
  int64_t kv_bs, kv_rs;
};

__device__ __forceinline__ void rope4(const u16* src, const u16* cs, int lo, u16 (&olo)[4], u16 (&ohi)[4]) {
  const u16x4 c4 = *reinterpret_cast<const u16x4*>(cs + lo), s4 = *reinterpret_cast<const u16x4*>(cs + kHalfDim + lo);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float c = bf2f(c4[i]), s = bf2f(s4[i]);
    const float xl = bf2f(src[lo + i]), xh = bf2f(src[kHalfDim + lo + i]);
    olo[i] = f2bf(fsub(fmul(xl, c), fmul(xh, s)));
    ohi[i] = f2bf(fadd(fmul(xh, c), fmul(xl, s)));
  }
}

__device__ __forceinline__ void store4(u16* dst, const u16 (&v)[4]) {
  *reinterpret_cast<u16x4*>(dst) = u16x4{v[0], v[1], v[2], v[3]};
}

__global__ __launch_bounds__(256) void rope_kv_kernel(RopeKvArgs a) {
  const int row = blockIdx.x, b = row / a.P, p = row % a.P, t = threadIdx.x;
  const u16* src = a.qkv + (size_t)row * a.ldq;
  const u16* cs = a.tab + (size_t)(a.pos[(size_t)b * a.s_pad + p] + 1) * kHeadDim;
  const u16* ksrc = src + (a.kv_only ? 0 : kPHD);
  const u16* vsrc = ksrc + kHeadDim;
  if (!a.kv_only) {
    // q: thread t -> head t/32, dims 4(t%32) .. +3 and their partners + 128
    const int head = t >> 5, lo = (t & 31) * 4;
    u16 olo[4], ohi[4];
    rope4(src + head * kHeadDim, cs, lo, olo, ohi);
    u16* qb = a.qf + (size_t)b * a.s_pad * kHeads * kHeadDim;
    const int qrow = p * kHeads + head;
    store4(qb + afrag_index(qrow, lo, kHeadDim / 32), olo);
    store4(qb + afrag_index(qrow, lo + kHalfDim, kHeadDim / 32), ohi);
  }
  const size_t cache = (size_t)b * a.kv_bs + (size_t)p * a.kv_rs;
  if (t < 32) {
    const int lo = t * 4;
    u16 olo[4], ohi[4];
    rope4(ksrc, cs, lo, olo, ohi);
    u16* kb = a.kf + (size_t)b * a.s_pad * kHeadDim;
    store4(kb + kfrag_index(p, lo), olo);
    store4(kb + kfrag_index(p, lo + kHalfDim), ohi);
    store4(a.kout + cache + lo, olo);
    store4(a.kout + cache + lo + kHalfDim, ohi);
  } else if (t >= 64 && t < 128) {
    const int d0 = (t - 64) * 4;
    u16 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = vsrc[d0 + i];
    u16* vb = a.vf + (size_t)b * a.s_pad * kHeadDim;
#pragma unroll
    for (int i = 0; i < 4; ++i) vb[vfrag_index(p, d0 + i)] = v[i];
    store4(a.vout + cache + d0, v);
  }
}

// ---------------------------------------------------------------------------------------------
// Masked MQA attention over the prefix (modeling_gemma.py:219-275): 8 query heads share the one
// K/V head, so a 16-row m-tile holds 2 tokens x 8 heads against the same keys.  Workgroup = 8
// m-tiles of one sample in 8 waves, wave w owns m-tile w (query fragments in registers; one m-tile
// per wave keeps a wave under 256 registers, so two waves share each SIMD and one wave's softmax
// overlaps the other's MFMAs).  Key blocks of 32 (16 KiB of K + 16 KiB of V fragments) are staged
// into LDS with direct-to-LDS loads two blocks at a time (one barrier per two blocks), double
// buffered, and every wave runs the online-softmax block update of the denoise attention
// (attend_block) on its m-tile.  Masked keys are skipped; a query row with no valid key (a padded
// token) is written as zeros.  With nsplit > 1 the key blocks are split over nsplit
// workgroups per m-tile group (so that short prefixes still fill the GPU), which store their
// unnormalised fp32 O and running (max, sum) per row for attn_merge_kernel.
// ---------------------------------------------------------------------------------------------
struct AttnArgs {
  const u16 *qf, *kf, *vf;
  const uint8_t* valid;
  u16* out;    // [B*P, 2048] (nsplit == 1)
  float* po;   // [nsplit][B][n_mt*16 rows][256] partial O (nsplit > 1); row = token * 8 + head
  float* pml;  // [nsplit][B][n_mt*16 rows][2] running max, sum
  int B, P, s_pad, n_mt, items, nsplit;
};

constexpr int kAttnMaxBlocks = 65536 / 32;
constexpr int kAttnMaxSplits = 8;  // the split count's cap (prefill_plan)  // key blocks of the longest prefix (batch * prefix_len <= 65536)

__global__ __launch_bounds__(512, 1) void prefix_attn_kernel(AttnArgs a) {
  __shared__ __align__(16) u16 s_kv[2][64][512];  // two stages of two 32-key blocks
  __shared__ uint32_t s_bits[kAttnMaxBlocks];  // bit j of word i: key 32 (kb_lo + i) + j is valid
  const int split = blockIdx.x % a.nsplit, bi = blockIdx.x / a.nsplit;
  const int b = bi / a.items, item = bi % a.items;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int mt = item * kAttnMtPerWg + wave;
  const u16* qb = a.qf + (size_t)b * a.s_pad * kHeads * kHeadDim;
  const u16* kb0 = a.kf + (size_t)b * a.s_pad * kHeadDim;
  const u16* vb0 = a.vf + (size_t)b * a.s_pad * kHeadDim;
  const uint8_t* valid = a.valid + (size_t)b * a.s_pad;
  const int nkb = a.s_pad / 32, kb_lo = split * nkb / a.nsplit, kb_hi = (split + 1) * nkb / a.nsplit;
  // the key-valid bytes of the workgroup's key range as one bit-mask word per block, so the block
  // loop issues no vector loads besides the staging copies (a wait for a mask load would also wait
  // for the next block's copies)
  for (int i = tid; i < kb_hi - kb_lo; i += 512) {
    const uint4 v0 = *reinterpret_cast<const uint4*>(valid + (size_t)(kb_lo + i) * 32);
    const uint4 v1 = *reinterpret_cast<const uint4*>(valid + (size_t)(kb_lo + i) * 32 + 16);
    const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) bits |= (((w[j >> 2] >> (8 * (j & 3))) & 0xff) ? 1u : 0u) << j;
    s_bits[i] = bits;
  }
  bf16x8 qf[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) qf[ds] = mt < a.n_mt ? load_frag(qb + afrag_offset(mt, ds, kHeadDim / 32) + lane * 8) : zero_frag();
  // stage j = blocks kb_lo + 2j and + 1; wave w copies fragments 4w .. 4w+3 of each (K fragments
  // 0..15, then V fragments): one barrier per two blocks
  auto stage = [&](int j, int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kb = kb_lo + 2 * j + h;
      if (kb < kb_hi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int f = wu * 4 + i;
          const u16* src = f < 16 ? kb0 + ((size_t)2 * kb * 8 + f) * 512 : vb0 + ((size_t)kb * 16 + (f - 16)) * 512;
          __builtin_amdgcn_global_load_lds(const_cast<u16*>(src) + lane * 8, &s_kv[buf][32 * h + f][0], 16, 0, 0);
        }
      }
    }
  };
  stage(0, 0);
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; kb_lo + 2 * j < kb_hi; ++j) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this wave's copies of stage j have landed
    __syncthreads();  // every wave's copies of stage j have landed; buffer (j+1)&1 is no longer read
    if (kb_lo + 2 * (j + 1) < kb_hi) stage(j + 1, (j + 1) & 1);
    const int buf = j & 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kb = kb_lo + 2 * j + h;
      if (kb >= kb_hi) break;
      KvBlock blk;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        blk.k[i] = *reinterpret_cast<const bf16x8*>(&s_kv[buf][32 * h + i][lane * 8]);
        blk.v[i] = *reinterpret_cast<const bf16x8*>(&s_kv[buf][32 * h + 16 + i][lane * 8]);
      }
      // attend_block's key-valid bytes: keys 4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3
      const uint32_t bits = s_bits[kb - kb_lo];
      const uint32_t lo = (bits >> (4 * g)) & 15u, hi = (bits >> (16 + 4 * g)) & 15u;
      blk.valid0 = (lo & 1u) | ((lo & 2u) << 7) | ((lo & 4u) << 14) | ((lo & 8u) << 21);
      blk.valid1 = (hi & 1u) | ((hi & 2u) << 7) | ((hi & 4u) << 14) | ((hi & 8u) << 21);
      if (mt < a.n_mt) attend_block(blk, qf, m_run, l_run, oacc);
    }
  }
  // O = acc / l: lane (row r16 = token 2 mt + r16/8, head r16 % 8) holds dims 16 dt + 4 g .. +3
  if (mt >= a.n_mt) return;  // after the last barrier
  float l = l_run;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  const int r16 = lane & 15, token = 2 * mt + (r16 >> 3), head = r16 & 7;
  if (token >= a.P) return;
  if (a.nsplit > 1) {
    const size_t row = ((size_t)split * a.B + b) * ((size_t)a.n_mt * 16) + (size_t)mt * 16 + r16;
    float* prow = a.po + row * kHeadDim + g * 4;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) *reinterpret_cast<f32x4*>(prow + dt * 16) = oacc[dt];
    if (g == 0) {
      a.pml[row * 2] = m_run;
      a.pml[row * 2 + 1] = l;
    }
    return;
  }
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  u16* orow = a.out + ((size_t)b * a.P + token) * kPHD + head * kHeadDim + g * 4;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) {
    const f32x4 o = oacc[dt];
    *reinterpret_cast<u16x4*>(orow + dt * 16) = u16x4{f2bf(o[0] * inv), f2bf(o[1] * inv), f2bf(o[2] * inv), f2bf(o[3] * inv)};
  }
}

// The key splits of one token row (b, token): out = sum_s O_s w_s / sum_s l_s w_s with
// w_s = exp(m_s - max_s m_s), splits in order; thread t: head t/32, dims 8(t%32) .. +7.
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* po, const float* pml, u16* out, int B, int P, int n_mt, int nsplit) {
  const int b = blockIdx.x / P, token = blockIdx.x % P, t = threadIdx.x;
  const int head = t >> 5, d0 = (t & 31) * 8;
  const size_t rows = (size_t)n_mt * 16, row = (size_t)token * kHeads + head;
  // every split's (max, sum) and partial row are loaded before the first use (a loop that waited
  // for each split's loads in turn paid one memory round trip per split); splits combined in order
  float2 ml[kAttnMaxSplits];
  float4 v0[kAttnMaxSplits], v1[kAttnMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kAttnMaxSplits; ++sp)
    if (sp < nsplit) {
      const size_t r = ((size_t)sp * B + b) * rows + row;
      ml[sp] = *reinterpret_cast<const float2*>(pml + r * 2);
      v0[sp] = *reinterpret_cast<const float4*>(po + r * kHeadDim + d0);
      v1[sp] = *reinterpret_cast<const float4*>(po + r * kHeadDim + d0 + 4);
    }
  float M = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kAttnMaxSplits; ++sp)
    if (sp < nsplit) M = fmaxf(M, ml[sp].x);
  float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < kAttnMaxSplits; ++sp)
    if (sp < nsplit) {
      const float ms = ml[sp].x;
      const float w = ms == -INFINITY ? 0.f : __expf(ms - M);
      L += ml[sp].y * w;
      o[0] += v0[sp].x * w, o[1] += v0[sp].y * w, o[2] += v0[sp].z * w, o[3] += v0[sp].w * w;
      o[4] += v1[sp].x * w, o[5] += v1[sp].y * w, o[6] += v1[sp].z * w, o[7] += v1[sp].w * w;
    }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  u16x8 r8;
#pragma unroll
  for (int i = 0; i < 8; ++i) r8[i] = f2bf(o[i] * inv);
  *reinterpret_cast<u16x8*>(out + ((size_t)b * P + token) * kPHD + head * kHeadDim + d0) = r8;
}

// ---------------------------------------------------------------------------------------------
// act = bf16(gelu_tanh(g) * u) over gu rows [g (16384) | u (16384)] (modeling_gemma.py:147 with
// the fused pointwise rounding: fp32 on the bf16 GEMM outputs, one rounding)
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void geglu_kernel(const u16* gu, u16* act, size_t chunks) {
  for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (size_t)gridDim.x * 256) {
    const size_t row = c / (kPI / 8), j = (c % (kPI / 8)) * 8;
    const u16x8 gv = *reinterpret_cast<const u16x8*>(gu + row * kPGuN + j);
    const u16x8 uv = *reinterpret_cast<const u16x8*>(gu + row * kPGuN + kPI + j);
    u16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f2bf(fmul(gelu_tanh(bf2f(gv[i])), bf2f(uv[i])));
    *reinterpret_cast<u16x8*>(act + row * kPI + j) = o;
  }
}

// out[i] = bf16(table[ids[i]] * sqrt(2048)); an id outside [0, vocab) zero-fills its row and
// sets *err.
// A row whose id is outside [0, vocab) is written as zeros and the call's tag goes to a pinned
// host word (system scope), which the host reads without synchronising.
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* ids, const u16* table, int64_t vocab, u16* out,
                                                    unsigned* host_bad, unsigned tag) {
  const int64_t i = blockIdx.x;
  const int32_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  if (!ok && threadIdx.x == 0) __hip_atomic_store(host_bad, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const size_t d = (size_t)threadIdx.x * 8;
  u16x8 o = {0, 0, 0, 0, 0, 0, 0, 0};
  if (ok) {
    const u16x8 v = *reinterpret_cast<const u16x8*>(table + (size_t)id * kPW + d);
    const float scale = 45.254833995939045f;  // sqrt(2048) as an fp32 scalar
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = f2bf(fmul(bf2f(v[k]), scale));
  }
  *reinterpret_cast<u16x8*>(out + i * kPW + d) = o;
}

struct LayerBind {
  const void *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
  const float *ln1 = nullptr, *ln2 = nullptr;
};

// Device layout of one context: sizes in bytes.
struct PrefixPlan {
  int L = 0, B = 0, P = 0, M = 0, s_pad = 0, n_mt = 0, items = 0, nsplit = 1;
  size_t w, ln, h, n, y, qkv, attn, gu, act, qf, kv, pos, valid, invf, rtab, ws, po, pml, dpart;
  size_t total() const {
    return w + ln + 3 * h + qkv + attn + gu + act + qf + 2 * kv + pos + valid + invf + rtab + ws + po + pml + dpart + 16 * 256;
  }
};
constexpr size_t kWorkspace = 64ull << 20;

size_t rup(size_t x) { return (x + 255) / 256 * 256; }

PrefixPlan plan_of(const pi05_prefix_dims& d) {
  PrefixPlan p;
  p.L = d.depth, p.B = d.batch, p.P = d.prefix_len, p.M = d.batch * d.prefix_len;
  p.s_pad = (d.prefix_len + 31) / 32 * 32;
  p.n_mt = (d.prefix_len + 1) / 2;
  p.items = (p.n_mt + kAttnMtPerWg - 1) / kAttnMtPerWg;
  // key splits: as many as keep every attention workgroup in one round on 256 CUs (one
  // workgroup per CU), at most 8 and at most one per key block
  const int nkb = p.s_pad / 32;
  p.nsplit = 256 / (p.B * p.items);
  if (p.nsplit > kAttnMaxSplits) p.nsplit = kAttnMaxSplits;
  if (p.nsplit > nkb) p.nsplit = nkb;
  if (p.nsplit < 1) p.nsplit = 1;
  const size_t M = p.M;
  p.w = rup((size_t)p.L * kPLayerElems * 2);
  p.ln = rup((size_t)p.L * 2 * kPW * 4);
  p.h = rup(M * kPW * 2);
  p.qkv = rup(M * kPQkvN * 2);
  p.attn = rup(M * kPHD * 2);
  p.gu = rup(M * kPGuN * 2);
  p.act = rup(M * kPI * 2);
  p.qf = rup((size_t)p.B * p.s_pad * kHeads * kHeadDim * 2);
  p.kv = rup((size_t)p.B * p.s_pad * kHeadDim * 2);
  p.pos = rup((size_t)p.B * p.s_pad * 4);
  p.valid = rup((size_t)p.B * p.s_pad);
  p.invf = rup(kHalfDim * 4);
  p.rtab = rup((size_t)(p.P + 1) * kHeadDim * 2);
  p.ws = kWorkspace;
  const size_t rows = (size_t)p.B * p.n_mt * 16;
  p.po = p.nsplit > 1 ? rup((size_t)p.nsplit * rows * kHeadDim * 4) : 0;
  p.pml = p.nsplit > 1 ? rup((size_t)p.nsplit * rows * 2 * 4) : 0;
  p.dpart = rup((size_t)kDownSplits * M * kPW * 4);
  return p;
}

bool check_prefix_dims(const pi05_prefix_dims* d, std::string* msg) {
  if (!d) {
    *msg = "dims is NULL";
    return false;
  }
  if (d->width != kPW || d->num_heads != kHeads || d->num_kv_heads != 1 || d->head_dim != kHeadDim || d->mlp_dim != kPI) {
    *msg = "prefix geometry must be width 2048, 8 heads, 1 KV head, head_dim 256, mlp_dim 16384";
    return false;
  }
  if (d->depth < 1 || d->depth > 64) {
    *msg = "depth must be in [1, 64]";
    return false;
  }
  if (d->batch < 1 || d->prefix_len < 1 || (int64_t)d->batch * d->prefix_len > (1 << 16)) {
    *msg = "batch and prefix_len must be >= 1 with batch * prefix_len <= 65536";
    return false;
  }
  if (!(d->rms_eps > 0.f) || !(d->rope_theta > 1.f) || (d->skip_last_layer != 0 && d->skip_last_layer != 1)) {
    *msg = "rms_eps must be > 0, rope_theta > 1, skip_last_layer 0 or 1";
    return false;
  }
  return true;
}

// 1 / (theta ** (arange(0, D, 2) / D)) in fp32, as transformers' default RoPE computes it.
void prefix_inv_freq(float theta, float* out) {
  for (int i = 0; i < kHalfDim; ++i) {
    const float ex = (float)(2 * i) / (float)kHeadDim;
    out[i] = 1.0f / (float)std::pow((double)theta, (double)ex);
  }
}

}  // namespace
}  // namespace pi05

using namespace pi05;

struct pi05_prefix_ctx {
  pi05_prefix_dims d{};
  PrefixPlan plan;
  int device = -1;
  std::string err;
  std::vector<LayerBind> binds;
  bool refreshed = false;
  char* base = nullptr;
  u16 *w = nullptr, *h = nullptr, *n = nullptr, *y = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr;
  u16 *qf = nullptr, *kf = nullptr, *vf = nullptr;
  float *ln = nullptr, *inv_freq = nullptr, *po = nullptr, *pml = nullptr, *dpart = nullptr;
  u16* rope_tab = nullptr;  // [P + 1][cos | sin] bf16, row = position + 1
  bool down_split = false;  // down_proj as kDownSplits fp32 split-K GEMMs reduced in the residual norm
  bool o_split = false;     // o_proj likewise
  int* pos = nullptr;
  uint8_t* valid = nullptr;
  unsigned* host_bad = nullptr;  // pinned host word: tag of the last embed call that met a bad token id
  unsigned embed_tag = 0, reported_tag = 0;
  void* ws = nullptr;
  hipblasLtHandle_t lt = nullptr;
  GemmPlan g_qkv, g_kv, g_o, g_gu, g_d, g_dsk, g_osk;
};

namespace {

int fail(pi05_prefix_ctx* c, int code, const std::string& m) {
  if (c) c->err = m;
  else g_prefix_err = m;
  return code;
}

int hip_fail(pi05_prefix_ctx* c, const char* what, hipError_t e) {
  return fail(c, PI05_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

GemmOpts split_opts(int ld_k) {
  GemmOpts o;
  o.batch = kDownSplits;
  o.ld_k = ld_k;
  return o;
}

int gemm(pi05_prefix_ctx* c, const GemmPlan& p, const u16* W, const u16* A, void* C, hipStream_t st) {
  const hipblasStatus_t s = run_plan(c->lt, p, p.algo, p.ws, W, A, C, nullptr, c->ws, st);
  if (!lt_ok(s)) return fail(c, PI05_E_HIP, "hipblasLtMatmul failed (status " + std::to_string((int)s) + ")");
  return PI05_OK;
}

}  // namespace

extern "C" {

void pi05_prefix_default_dims(pi05_prefix_dims* d) {
  if (!d) return;
  *d = pi05_prefix_dims{};
  d->width = kPW;
  d->depth = 18;
  d->num_heads = kHeads;
  d->num_kv_heads = 1;
  d->head_dim = kHeadDim;
  d->mlp_dim = kPI;
  d->batch = 1;
  d->prefix_len = 968;
  d->rms_eps = 1e-6f;
  d->rope_theta = 10000.0f;
  d->skip_last_layer = 1;
}

int pi05_prefix_check_dims(const pi05_prefix_dims* dims) {
  std::string m;
  if (!check_prefix_dims(dims, &m)) return fail(nullptr, PI05_E_INVALID, m);
  return PI05_OK;
}

size_t pi05_prefix_device_bytes(const pi05_prefix_dims* dims) {
  std::string m;
  if (!check_prefix_dims(dims, &m)) return 0;
  return plan_of(*dims).total();
}

const char* pi05_prefix_last_error(const pi05_prefix_ctx* ctx) { return ctx ? ctx->err.c_str() : g_prefix_err.c_str(); }

int pi05_prefix_create(const pi05_prefix_dims* dims, pi05_prefix_ctx** out) {
  if (!out) return fail(nullptr, PI05_E_INVALID, "out is NULL");
  *out = nullptr;
  std::string m;
  if (!check_prefix_dims(dims, &m)) return fail(nullptr, PI05_E_INVALID, m);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(nullptr, PI05_E_NODEVICE, std::string("no HIP device: ") + hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, PI05_E_NODEVICE, std::string("device is not gfx950 (MI355X): ") + (e == hipSuccess ? prop.gcnArchName : hipGetErrorString(e)));
  pi05_prefix_ctx* c = new pi05_prefix_ctx();
  c->d = *dims;
  c->device = dev;
  c->plan = plan_of(*dims);
  c->binds.resize(dims->depth);
  const PrefixPlan& p = c->plan;
  e = hipMalloc(&c->base, p.total());
  if (e != hipSuccess) {
    delete c;
    return fail(nullptr, PI05_E_NOMEM, std::string("prefix context allocation failed: ") + hipGetErrorString(e));
  }
  char* q = c->base;
  auto take = [&](size_t bytes) {
    char* r = q;
    q += bytes;
    return r;
  };
  c->w = reinterpret_cast<u16*>(take(p.w));
  c->ln = reinterpret_cast<float*>(take(p.ln));
  c->h = reinterpret_cast<u16*>(take(p.h));
  c->n = reinterpret_cast<u16*>(take(p.h));
  c->y = reinterpret_cast<u16*>(take(p.h));
  c->qkv = reinterpret_cast<u16*>(take(p.qkv));
  c->attn = reinterpret_cast<u16*>(take(p.attn));
  c->gu = reinterpret_cast<u16*>(take(p.gu));
  c->act = reinterpret_cast<u16*>(take(p.act));
  c->qf = reinterpret_cast<u16*>(take(p.qf));
  c->kf = reinterpret_cast<u16*>(take(p.kv));
  c->vf = reinterpret_cast<u16*>(take(p.kv));
  c->pos = reinterpret_cast<int*>(take(p.pos));
  c->valid = reinterpret_cast<uint8_t*>(take(p.valid));
  c->inv_freq = reinterpret_cast<float*>(take(p.invf));
  c->rope_tab = reinterpret_cast<u16*>(take(p.rtab));
  c->ws = take(p.ws);
  c->po = reinterpret_cast<float*>(take(p.po));
  c->pml = reinterpret_cast<float*>(take(p.pml));
  c->dpart = reinterpret_cast<float*>(take(p.dpart));
  // everything starts zeroed: query rows and keys past P stay zero (finite and masked) for the
  // life of the context, and the GEMM tuning below reads defined values
  e = hipMemset(c->base, 0, p.total());
  if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->host_bad), sizeof(unsigned), hipHostMallocMapped);
  if (e == hipSuccess) *c->host_bad = 0;
  float invf[kHalfDim];
  prefix_inv_freq(dims->rope_theta, invf);
  if (e == hipSuccess) e = hipMemcpy(c->inv_freq, invf, sizeof(invf), hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    rope_table_kernel<<<p.P + 1, kHalfDim>>>(c->inv_freq, p.P, c->rope_tab);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
  }
  if (e != hipSuccess) {
    if (c->host_bad) (void)hipHostFree(c->host_bad);
    hipFree(c->base);
    delete c;
    return fail(nullptr, PI05_E_HIP, std::string("prefix context initialisation failed: ") + hipGetErrorString(e));
  }
  std::string perr;
  const int M = p.M;
  if (!lt_ok(hipblasLtCreate(&c->lt)) || !make_plan(c->lt, M, kPQkvN, kPW, kWorkspace, &c->g_qkv, &perr) ||
      !make_plan(c->lt, M, kPKvN, kPW, kWorkspace, &c->g_kv, &perr) || !make_plan(c->lt, M, kPW, kPHD, kWorkspace, &c->g_o, &perr) ||
      !make_plan(c->lt, M, kPGuN, kPW, kWorkspace, &c->g_gu, &perr) || !make_plan(c->lt, M, kPW, kPI, kWorkspace, &c->g_d, &perr) ||
      !make_plan(c->lt, M, kPW, kPI / kDownSplits, kWorkspace, &c->g_dsk, &perr, split_opts(kPI)) ||
      !make_plan(c->lt, M, kPW, kPHD / kDownSplits, kWorkspace, &c->g_osk, &perr, split_opts(kPHD))) {
    if (perr.empty()) perr = "hipblasLtCreate failed";
    pi05_prefix_destroy(c);
    return fail(nullptr, PI05_E_HIP, perr);
  }
  // pick each GEMM's fastest algorithm on this device and shape
  // (weights rotate over the layers' blocks while timing, as the layer loop streams them)
  const size_t ls = kPLayerElems * 2;
  const int nl = dims->depth;
  const bool tuned = tune_plan(c->lt, &c->g_qkv, c->w, c->n, c->qkv, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_kv, c->w, c->n, c->qkv, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_o, c->w, c->attn, c->y, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_gu, c->w, c->n, c->gu, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_d, c->w, c->act, c->y, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_dsk, c->w, c->act, c->dpart, c->ws, nullptr, nullptr, ls, nl) &&
                     tune_plan(c->lt, &c->g_osk, c->w, c->attn, c->dpart, c->ws, nullptr, nullptr, ls, nl);
  if (!tuned) {
    pi05_prefix_destroy(c);
    return fail(nullptr, PI05_E_HIP, "GEMM algorithm tuning failed");
  }
  // split-K down_proj when its GEMM plus the extra partial traffic of the fused reduction
  // ((kDownSplits * 4 - 2) bytes per output element at ~4 TB/s) beats the single bf16 GEMM
  const float extra_ms = (float)((double)(kDownSplits * 4 - 2) * M * kPW / 4e12 * 1e3);
  c->down_split = c->g_dsk.ms + extra_ms < c->g_d.ms;
  c->o_split = c->g_osk.ms + extra_ms < c->g_o.ms;
  *out = c;
  return PI05_OK;
}

int pi05_prefix_destroy(pi05_prefix_ctx* c) {
  if (!c) return PI05_OK;  // like free(NULL)
  free_plan(&c->g_qkv);
  free_plan(&c->g_kv);
  free_plan(&c->g_o);
  free_plan(&c->g_gu);
  free_plan(&c->g_d);
  free_plan(&c->g_dsk);
  free_plan(&c->g_osk);
  if (c->lt) hipblasLtDestroy(c->lt);
  // an embed kernel still in flight may write the pinned word
  if (c->host_bad) {
    (void)hipDeviceSynchronize();
    (void)hipHostFree(c->host_bad);
  }
  if (c->base) hipFree(c->base);
  delete c;
  return PI05_OK;
}

int pi05_prefix_bind_layer(pi05_prefix_ctx* c, int layer, const void* wq, const void* wk, const void* wv, const void* wo,
                           const void* wgate, const void* wup, const void* wdown, const float* ln1_w, const float* ln2_w) {
  if (!c) return fail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (layer < 0 || layer >= c->d.depth) return fail(c, PI05_E_INVALID, "layer out of range");
  const void* ptrs[] = {wq, wk, wv, wo, wgate, wup, wdown, ln1_w, ln2_w};
  for (const void* p : ptrs) {
    if (!p) return fail(c, PI05_E_INVALID, "a weight pointer is NULL");
    if (reinterpret_cast<uintptr_t>(p) % 16) return fail(c, PI05_E_INVALID, "weight pointers must be 16-byte aligned");
  }
  c->binds[layer] = LayerBind{wq, wk, wv, wo, wgate, wup, wdown, ln1_w, ln2_w};
  c->refreshed = false;
  return PI05_OK;
}

int pi05_prefix_refresh_weights(pi05_prefix_ctx* c, void* stream) {
  if (!c) return fail(nullptr, PI05_E_INVALID, "ctx is NULL");
  for (int l = 0; l < c->d.depth; ++l)
    if (!c->binds[l].wq) return fail(c, PI05_E_STATE, "layer " + std::to_string(l) + " is not bound");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipMemcpyKind k = hipMemcpyDeviceToDevice;
  for (int l = 0; l < c->d.depth; ++l) {
    const LayerBind& b = c->binds[l];
    u16* w = c->w + (size_t)l * kPLayerElems;
    const size_t sq = (size_t)kPHD * kPW * 2, sk = (size_t)kHeadDim * kPW * 2, sg = (size_t)kPI * kPW * 2;
    hipError_t e = hipMemcpyAsync(w + kPOffQkv, b.wq, sq, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffQkv + (size_t)kPHD * kPW, b.wk, sk, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffQkv + (size_t)(kPHD + kHeadDim) * kPW, b.wv, sk, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffO, b.wo, (size_t)kPW * kPHD * 2, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffGu, b.wg, sg, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffGu + (size_t)kPI * kPW, b.wu, sg, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(w + kPOffD, b.wd, (size_t)kPW * kPI * 2, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(c->ln + (size_t)l * 2 * kPW, b.ln1, kPW * 4, k, st);
    if (e == hipSuccess) e = hipMemcpyAsync(c->ln + (size_t)l * 2 * kPW + kPW, b.ln2, kPW * 4, k, st);
    if (e != hipSuccess) return hip_fail(c, "weight packing", e);
  }
  c->refreshed = true;
  return PI05_OK;
}

// A bad token id of an earlier embed call that has not been reported yet: report it (once).
static int pending_bad_ids(pi05_prefix_ctx* c) {
  const unsigned seen = __atomic_load_n(c->host_bad, __ATOMIC_ACQUIRE);
  if (seen > c->reported_tag) {
    c->reported_tag = seen;
    return fail(c, PI05_E_INVALID, "a token id of an earlier pi05_prefix_embed_tokens call was outside [0, vocab) (its row was written as zeros)");
  }
  return PI05_OK;
}

int pi05_prefix_embed_tokens(pi05_prefix_ctx* c, const int32_t* ids, int64_t n_tokens, const void* table, int64_t vocab,
                             void* out, void* stream) {
  if (!c) return fail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (!ids || !table || !out) return fail(c, PI05_E_INVALID, "ids, table and out must be non-NULL");
  if (n_tokens < 1 || n_tokens > (1 << 24) || vocab < 1) return fail(c, PI05_E_INVALID, "n_tokens must be in [1, 2^24] and vocab >= 1");
  if (reinterpret_cast<uintptr_t>(table) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(c, PI05_E_INVALID, "table and out must be 16-byte aligned");
  const int rc = pending_bad_ids(c);
  if (rc != PI05_OK) return rc;  // enqueues nothing
  hipStream_t st = static_cast<hipStream_t>(stream);
  embed_kernel<<<(unsigned)n_tokens, 256, 0, st>>>(ids, static_cast<const u16*>(table), vocab, static_cast<u16*>(out), c->host_bad,
                                                   ++c->embed_tag);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(c, "embed", e);
  return PI05_OK;
}

int pi05_prefix_status(pi05_prefix_ctx* c, void* stream) {
  if (!c) return fail(nullptr, PI05_E_INVALID, "ctx is NULL");
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(c, "status", e);
  return pending_bad_ids(c);
}

int pi05_prefix_forward(pi05_prefix_ctx* c, const void* embeds, const uint8_t* prefix_pad, void* const* k_layers,
                        void* const* v_layers, int64_t kv_batch_stride, int64_t kv_row_stride, void* stream) {
  if (!c) return fail(nullptr, PI05_E_INVALID, "ctx is NULL");
  if (!embeds || !prefix_pad || !k_layers || !v_layers) return fail(c, PI05_E_INVALID, "embeds, prefix_pad, k_layers and v_layers must be non-NULL");
  const PrefixPlan& p = c->plan;
  if (reinterpret_cast<uintptr_t>(embeds) % 16) return fail(c, PI05_E_INVALID, "embeds must be 16-byte aligned");
  if (kv_row_stride < kHeadDim || kv_row_stride % 4) return fail(c, PI05_E_INVALID, "kv_row_stride must be >= head_dim and a multiple of 4");
  if (p.B > 1 && kv_batch_stride < (int64_t)p.P * kv_row_stride) return fail(c, PI05_E_INVALID, "kv_batch_stride must cover prefix_len rows");
  if (kv_batch_stride % 4) return fail(c, PI05_E_INVALID, "kv_batch_stride must be a multiple of 4");
  for (int l = 0; l < p.L; ++l) {
    if (!k_layers[l] || !v_layers[l]) return fail(c, PI05_E_INVALID, "a K/V layer pointer is NULL");
    if (reinterpret_cast<uintptr_t>(k_layers[l]) % 8 || reinterpret_cast<uintptr_t>(v_layers[l]) % 8)
      return fail(c, PI05_E_INVALID, "K/V layer pointers must be 8-byte aligned");
  }
  if (!c->refreshed) return fail(c, PI05_E_STATE, "weights are not bound and refreshed");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u16* emb = static_cast<const u16*>(embeds);
  const float eps = c->d.rms_eps;
  positions_kernel<<<p.B, 256, 0, st>>>(prefix_pad, p.P, p.s_pad, c->pos, c->valid);
  rmsnorm_kernel<<<p.M, 256, 0, st>>>(emb, nullptr, c->ln, nullptr, c->n, eps);
  for (int l = 0; l < p.L; ++l) {
    const u16* w = c->w + (size_t)l * kPLayerElems;
    const float* ln = c->ln + (size_t)l * 2 * kPW;
    const bool kv_only = c->d.skip_last_layer && l == p.L - 1;
    RopeKvArgs ra{c->qkv, kv_only ? kPKvN : kPQkvN, kv_only ? 1 : 0, p.P, p.s_pad, c->pos, c->rope_tab,
                  c->qf, c->kf, c->vf, static_cast<u16*>(k_layers[l]), static_cast<u16*>(v_layers[l]), kv_batch_stride, kv_row_stride};
    int rc = kv_only ? gemm(c, c->g_kv, w + kPOffQkv + (size_t)kPHD * kPW, c->n, c->qkv, st) : gemm(c, c->g_qkv, w + kPOffQkv, c->n, c->qkv, st);
    if (rc != PI05_OK) return rc;
    rope_kv_kernel<<<p.M, 256, 0, st>>>(ra);
    if (kv_only) break;
    AttnArgs aa{c->qf, c->kf, c->vf, c->valid, c->attn, c->po, c->pml, p.B, p.P, p.s_pad, p.n_mt, p.items, p.nsplit};
    prefix_attn_kernel<<<p.B * p.items * p.nsplit, 512, 0, st>>>(aa);
    if (p.nsplit > 1) attn_merge_kernel<<<p.M, 256, 0, st>>>(c->po, c->pml, c->attn, p.B, p.P, p.n_mt, p.nsplit);
    if (c->o_split) {
      if ((rc = gemm(c, c->g_osk, w + kPOffO, c->attn, c->dpart, st)) != PI05_OK) return rc;
      rmsnorm_kernel<<<p.M, 256, 0, st>>>(l == 0 ? emb : c->h, nullptr, ln + kPW, c->h, c->n, eps, c->dpart, kDownSplits, (size_t)p.M * kPW);
    } else {
      if ((rc = gemm(c, c->g_o, w + kPOffO, c->attn, c->y, st)) != PI05_OK) return rc;
      rmsnorm_kernel<<<p.M, 256, 0, st>>>(l == 0 ? emb : c->h, c->y, ln + kPW, c->h, c->n, eps);
    }
    if ((rc = gemm(c, c->g_gu, w + kPOffGu, c->n, c->gu, st)) != PI05_OK) return rc;
    const size_t chunks = (size_t)p.M * (kPI / 8);
    geglu_kernel<<<(unsigned)((chunks + 255) / 256 < 4096 ? (chunks + 255) / 256 : 4096), 256, 0, st>>>(c->gu, c->act, chunks);
    if (c->down_split) {
      if ((rc = gemm(c, c->g_dsk, w + kPOffD, c->act, c->dpart, st)) != PI05_OK) return rc;
      if (l + 1 < p.L)
        rmsnorm_kernel<<<p.M, 256, 0, st>>>(c->h, nullptr, c->ln + (size_t)(l + 1) * 2 * kPW, c->h, c->n, eps, c->dpart, kDownSplits,
                                            (size_t)p.M * kPW);
    } else {
      if ((rc = gemm(c, c->g_d, w + kPOffD, c->act, c->y, st)) != PI05_OK) return rc;
      if (l + 1 < p.L) rmsnorm_kernel<<<p.M, 256, 0, st>>>(c->h, c->y, c->ln + (size_t)(l + 1) * 2 * kPW, c->h, c->n, eps);
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(c, "prefill launch", e);
  return PI05_OK;
}

}  // extern "C"
