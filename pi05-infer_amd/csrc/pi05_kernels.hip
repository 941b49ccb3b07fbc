// gfx950 kernels of the pi0.5 action-expert denoise step.
//
// One denoise step = step_io (final norm + action_out_proj + Euler of the previous step, then
// action_in_proj of this step) followed, per decoder layer, by
//   qkv_rope   : adaRMSNorm(input_layernorm) prologue + fused q|k|v GEMM + RoPE epilogue,
//                q -> activation buffer, k/v -> the fragment-major static KV cache tail
//   attention  : MQA attention of the 8*50 query rows over prefix + suffix keys (split-KV)
//   attn_merge : combine the split-KV partials (only when the keys are split)
//   o_proj     : o_proj GEMM + gated-residual epilogue (gate of input_layernorm)
//   gate_up    : adaRMSNorm(post_attention_layernorm) prologue + gate|up GEMM + GeGLU epilogue
//   down       : down_proj GEMM + gated-residual epilogue (gate of post_attention_layernorm)
// The small-M (M = 50 per sample) GEMMs stream weights that were packed fragment-major, so each
// wave-wide 16-byte load reads 1 KiB of contiguous memory, and run on bf16 MFMA 16x16x32.
// Numerics follow the reference's rounding points (bf16 tensor boundaries, fp32 statistics).

#include "pi05_device.h"
#include "pi05_kernels.h"

namespace pi05 {

// =============================================================================================
// packing
// =============================================================================================

// W[N][K] row-major bf16 -> fragment-major (see pi05_device.h).  One thread copies 16 bytes.
__global__ void pack_weight_kernel(const u16* __restrict__ src, u16* __restrict__ dst, int N, int K) {
  const int ksteps = K >> 5;
  const size_t total = (size_t)(N >> 4) * ksteps * 64;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const size_t frag = idx >> 6;
    const int ks = (int)(frag % ksteps);
    const int nt = (int)(frag / ksteps);
    const u16* s = src + (size_t)(nt * 16 + (lane & 15)) * K + ks * 32 + (lane >> 4) * 8;
    *reinterpret_cast<u16x8*>(dst + frag * 512 + lane * 8) = *reinterpret_cast<const u16x8*>(s);
  }
}

// Prefix K/V [B, 1, P, D] (strided) -> fragment-major cache keys [0, P); keys [P+A, S_pad) are
// zeroed so padded lanes never carry NaN/Inf into the masked MFMA products.
__global__ void prime_kv_kernel(PrimeKvArgs a) {
  const int layer = blockIdx.z;
  const int b = blockIdx.y;
  const u16* ksrc = reinterpret_cast<const u16*>(a.k_ptrs[layer]) + (size_t)b * a.batch_stride;
  const u16* vsrc = reinterpret_cast<const u16*>(a.v_ptrs[layer]) + (size_t)b * a.batch_stride;
  u16* kdst = a.kcache + ((size_t)layer * a.batch + b) * a.s_pad * kHeadDim;
  u16* vdst = a.vcache + ((size_t)layer * a.batch + b) * a.s_pad * kHeadDim;
  // one thread handles 8 consecutive d of one key
  const int per_key = kHeadDim / 8;
  const int total = a.s_pad * per_key;
  for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
    const int key = idx / per_key;
    const int d0 = (idx % per_key) * 8;
    u16x8 kv8 = {0, 0, 0, 0, 0, 0, 0, 0};
    u16x8 vv8 = {0, 0, 0, 0, 0, 0, 0, 0};
    const bool is_prefix = key < a.prefix_len;
    if (is_prefix) {
      kv8 = *reinterpret_cast<const u16x8*>(ksrc + (size_t)key * a.row_stride + d0);
      vv8 = *reinterpret_cast<const u16x8*>(vsrc + (size_t)key * a.row_stride + d0);
    } else if (key < a.prefix_len + kHorizon) {
      continue;  // suffix rows are written by every step's qkv_rope
    }
    // K: 8 consecutive d of one key are 8 consecutive elements of one lane
    *reinterpret_cast<u16x8*>(kdst + kfrag_index(key, d0)) = kv8;
#pragma unroll
    for (int j = 0; j < 8; ++j) vdst[vfrag_index(key, d0 + j)] = vv8[j];
  }
}

// Per batch row: positions sum(pad) + t (engine.py:476-477), key-valid mask, bf16 RoPE tables.
__global__ void prime_tables_kernel(PrimeTablesArgs a) {
  const int b = blockIdx.x;
  __shared__ int s_cnt[256];
  const uint8_t* pad = a.prefix_pad + (size_t)b * a.prefix_len;
  int cnt = 0;
  for (int p = threadIdx.x; p < a.prefix_len; p += blockDim.x) cnt += pad[p] ? 1 : 0;
  s_cnt[threadIdx.x] = cnt;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) s_cnt[threadIdx.x] += s_cnt[threadIdx.x + w];
    __syncthreads();
  }
  const int base = s_cnt[0];
  uint8_t* valid = a.valid + (size_t)b * a.s_pad;
  for (int key = threadIdx.x; key < a.s_pad; key += blockDim.x) {
    uint8_t v = 0;
    if (key < a.prefix_len) v = pad[key] ? 1 : 0;
    else if (key < a.prefix_len + kHorizon) v = 1;
    valid[key] = v;
  }
  for (int idx = threadIdx.x; idx < kHorizon * kHeadDim; idx += blockDim.x) {
    const int t = idx / kHeadDim;
    const int d = idx % kHeadDim;
    const int pos = base + t;
    if (d == 0) a.positions[b * kHorizon + t] = pos;
    // emb = cat(freqs, freqs): dims d and d + D/2 share inv_freq[d % (D/2)]
    const float freq = fmul(a.inv_freq[d % kHalfDim], (float)pos);
    const size_t o = ((size_t)b * kHorizon + t) * kHeadDim + d;
    a.cos_tab[o] = f2bf(cosf(freq));
    a.sin_tab[o] = f2bf(sinf(freq));
  }
}

// =============================================================================================
// adaRMS modulation table (once per weight refresh)
// =============================================================================================

// out[s][r] = act(sum_k W[r][k] * in[s][k] + bias[r]), fp32.  One wave per output row; the
// row is read once and applied to all S inputs.
__global__ __launch_bounds__(256) void gemv_rows_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const float* wr = a.W + (size_t)row * a.K;
  float acc[kMaxSteps];
#pragma unroll
  for (int s = 0; s < kMaxSteps; ++s) acc[s] = 0.f;
  for (int k = lane * 4; k < a.K; k += 256) {
    const float4 w4 = *reinterpret_cast<const float4*>(wr + k);
#pragma unroll
    for (int s = 0; s < kMaxSteps; ++s) {
      if (s < a.S) {
        const float4 x4 = *reinterpret_cast<const float4*>(a.in + (size_t)s * a.K + k);
        acc[s] += w4.x * x4.x + w4.y * x4.y + w4.z * x4.z + w4.w * x4.w;
      }
    }
  }
#pragma unroll
  for (int s = 0; s < kMaxSteps; ++s) {
    if (s < a.S) {
      float v = acc[s];
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
      if (lane == 0) {
        v += a.bias[row];
        if (a.silu) v = v / (1.0f + expf(-v));
        a.out[(size_t)s * a.out_ld + a.out_off + row] = v;
      }
    }
  }
}

// =============================================================================================
// step boundary: final norm + action_out_proj + Euler (previous step), action_in_proj (this step)
// =============================================================================================

__global__ __launch_bounds__(256) void step_io_kernel(StepIoArgs a) {
  const int m = blockIdx.x;  // token row (b * A + t)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  __shared__ float s_n[kWidth];
  __shared__ float s_x[kActDim];
  __shared__ float s_ss;

  if (a.has_prev) {
    // final adaRMSNorm (model.norm, modeling_gemma.py:782-783) of h[m]
    if (tid < 64) {
      float v = a.rowss[(size_t)tid * a.M + m];
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
      if (tid == 0) s_ss = v;
    }
    __syncthreads();
    const float rstd = 1.0f / sqrtf(fadd(s_ss * (1.0f / kWidth), a.eps));
    const u16* hrow = a.h + (size_t)m * kWidth;
    for (int c = tid; c < kWidth; c += 256) {
      const float hv = bf2f(hrow[c]);
      const float sc = a.final_mod[c];
      const float sh = a.final_mod[kWidth + c];
      s_n[c] = round_bf(fadd(fmul(fmul(hv, rstd), fadd(1.0f, sc)), sh));
    }
    __syncthreads();
    // v = action_out_proj(n) fp32 (engine.py:767): 8 threads per output, 128 k each
    const int j = tid >> 3;
    const int part = tid & 7;
    const float* wr = a.out_w + (size_t)j * kWidth + part * 128;
    float acc = 0.f;
    for (int k = 0; k < 128; k += 4) {
      const float4 w4 = *reinterpret_cast<const float4*>(wr + k);
      acc += w4.x * s_n[part * 128 + k] + w4.y * s_n[part * 128 + k + 1] + w4.z * s_n[part * 128 + k + 2] +
             w4.w * s_n[part * 128 + k + 3];
    }
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 4);
    if (part == 0) {
      const float v = acc + a.out_b[j];
      const float x = a.x[(size_t)m * kActDim + j];
      // flow_ode mean, reference op order (engine.py:664-675)
      const float x0_pred = fsub(x, fmul(v, a.t));
      const float x1_pred = fadd(x, fmul(v, a.one_minus_t));
      const float xn = fadd(fmul(x0_pred, a.x0_weight), fmul(x1_pred, a.x1_weight));
      a.x[(size_t)m * kActDim + j] = xn;
      s_x[j] = xn;
      if (a.trace) a.trace[(size_t)m * kActDim + j] = v;
    }
  } else if (tid < kActDim) {
    s_x[tid] = a.x[(size_t)m * kActDim + tid];
  }
  __syncthreads();

  if (a.has_next) {
    // h = bf16(action_in_proj(x)) (pi0_pytorch.py:303-306; modeling_gemma.py:724-725)
    const int c0 = tid * 4;
    float ss = 0.f;
    u16 hv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float* wr = a.in_w + (size_t)(c0 + q) * kActDim;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kActDim; k += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(wr + k);
        acc += w4.x * s_x[k] + w4.y * s_x[k + 1] + w4.z * s_x[k + 2] + w4.w * s_x[k + 3];
      }
      hv[q] = f2bf(acc + a.in_b[c0 + q]);
      const float hf = bf2f(hv[q]);
      ss += hf * hf;
    }
    u16x4 h4 = {hv[0], hv[1], hv[2], hv[3]};
    *reinterpret_cast<u16x4*>(a.h + (size_t)m * kWidth + c0) = h4;
    // per-16-column partial sums of squares (4 threads per 16-column tile)
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    if ((lane & 3) == 0) a.rowss[(size_t)(c0 >> 4) * a.M + m] = ss;
  }
}

// =============================================================================================
// GEMM family (small M, weight streaming on MFMA)
// =============================================================================================

// Weight fragments of this wave: NT tiles x KSW k-steps, issued up front (nontemporal: the
// weights are read once per step and must not evict the activations from L2).
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

// adaRMSNorm applied while forming the MFMA A fragment: 8 consecutive k of row `row`
// (modeling_gemma.py:82-116): bf16((h * rstd) * (1 + scale) + shift).
__device__ __forceinline__ bf16x8 norm_frag(const u16* __restrict__ h, int row, int k, float rstd,
                                            const float* __restrict__ scale, const float* __restrict__ shift) {
  const u16x8 hv = *reinterpret_cast<const u16x8*>(h + (size_t)row * kWidth + k);
  const float4 s0 = *reinterpret_cast<const float4*>(scale + k);
  const float4 s1 = *reinterpret_cast<const float4*>(scale + k + 4);
  const float4 t0 = *reinterpret_cast<const float4*>(shift + k);
  const float4 t1 = *reinterpret_cast<const float4*>(shift + k + 4);
  const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const float sh[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
  u16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f2bf(fadd(fmul(fmul(bf2f(hv[j]), rstd), fadd(1.0f, sc[j])), sh[j]));
  return as_bf16x8(o);
}

// rstd of 64 rows starting at m0 from the per-tile sum-of-squares partials.
__device__ __forceinline__ void row_rstd(float* s_rstd, const float* __restrict__ rowss, int M, int m0, float eps) {
  const int t = threadIdx.x;
  if (t < 64) {
    const int m = m0 + t;
    float ss = 0.f;
    if (m < M) {
      for (int s = 0; s < kRowSlots; ++s) ss += rowss[(size_t)s * M + m];
    }
    s_rstd[t] = 1.0f / sqrtf(fadd(ss * (1.0f / kWidth), eps));
  }
}

// Cross-wave K reduction through LDS.  Wave w stores acc[mt][t] (lane-major f32x4), then each
// output (row r in 0..63, col c in 0..15) is summed over waves in fixed order.
template <int NW, int NT>
__device__ __forceinline__ void store_partials(float* red, const f32x4 (&acc)[4][NT], int wave, int lane) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<f32x4*>(red + ((((size_t)wave * 4 + mt) * NT + t) * 64 + lane) * 4) = acc[mt][t];
}

template <int NW, int NT>
__device__ __forceinline__ float reduced(const float* red, int r, int c, int t) {
  const int mt = r >> 4, g = (r & 15) >> 2, i = r & 3;
  const int lane = g * 16 + c;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) v += red[((((size_t)w * 4 + mt) * NT + t) * 64 + lane) * 4 + i];
  return v;
}

// ---------------------------------------------------------------------------------------------
// qkv_rope: 80 workgroups x 4 waves.  WG p < 72 owns a RoPE pair of 16-column tiles of one
// rotated head (8 q heads + the k head): dims [dt*16, +16) and [128 + dt*16, +16); WG p >= 72
// owns two v tiles.  Waves split K = 1024 four ways.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void qkv_rope_kernel(QkvArgs a) {
  constexpr int NW = 4, NT = 2, KSW = 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int p = blockIdx.x;
  int tiles[2];
  const bool rotated = p < 72;
  const int head = p >> 3, dt = p & 7;
  if (rotated) {
    tiles[0] = head * 16 + dt;
    tiles[1] = head * 16 + 8 + dt;
  } else {
    tiles[0] = 144 + 2 * (p - 72);
    tiles[1] = tiles[0] + 1;
  }
  const u16* tile_ptr[NT] = {a.w + wfrag_offset(tiles[0], 0, 32), a.w + wfrag_offset(tiles[1], 0, 32)};
  bf16x8 w[NT][KSW];
  load_weights<NT, KSW>(w, tile_ptr, wave * KSW, lane);

  __shared__ float s_rstd[64];
  __shared__ float red[NW * 4 * NT * 64 * 4];
  const float* scale = a.mod;
  const float* shift = a.mod + kWidth;

  for (int m0 = 0; m0 < a.M; m0 += 64) {
    row_rstd(s_rstd, a.rowss, a.M, m0, a.eps);
    __syncthreads();
    f32x4 acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const int k = (wave * KSW + s) * 32 + g * 8;
      bf16x8 af[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = m0 + mt * 16 + r16;
        af[mt] = row < a.M ? norm_frag(a.h, row, k, s_rstd[mt * 16 + r16], scale, shift) : zero_frag();
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = mfma16x16x32(af[mt], w[t][s], acc[mt][t]);
    }
    store_partials<NW, NT>(red, acc, wave, lane);
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 16; e += NW * 64) {
      const int r = e >> 4, c = e & 15;
      const int m = m0 + r;
      if (m >= a.M) continue;
      const float x_lo = round_bf(reduced<NW, NT>(red, r, c, 0));
      const float x_hi = round_bf(reduced<NW, NT>(red, r, c, 1));
      const int b = m / kHorizon, tok = m % kHorizon;
      u16* kc = a.kcache + (size_t)b * a.s_pad * kHeadDim;
      u16* vc = a.vcache + (size_t)b * a.s_pad * kHeadDim;
      const int key = a.prefix_len + tok;
      if (rotated) {
        const int d = dt * 16 + c;
        const u16* cs = a.cos_tab + (size_t)m * kHeadDim;
        const u16* sn = a.sin_tab + (size_t)m * kHeadDim;
        // (x*cos) + (rotate_half(x)*sin), rotate_half(x) = cat(-x_hi, x_lo)
        // (rlinf_fused_denoise.py:264-278; modeling_gemma.py:185-216)
        const float o_lo = fsub(fmul(x_lo, bf2f(cs[d])), fmul(x_hi, bf2f(sn[d])));
        const float o_hi = fadd(fmul(x_hi, bf2f(cs[d + kHalfDim])), fmul(x_lo, bf2f(sn[d + kHalfDim])));
        if (head < kHeads) {
          u16* qrow = a.q + (size_t)m * (kHeads * kHeadDim) + head * kHeadDim;
          qrow[d] = f2bf(o_lo);
          qrow[d + kHalfDim] = f2bf(o_hi);
        } else {
          kc[kfrag_index(key, d)] = f2bf(o_lo);
          kc[kfrag_index(key, d + kHalfDim)] = f2bf(o_hi);
        }
      } else {
        const int dv = (tiles[0] - 144) * 16 + c;
        vc[vfrag_index(key, dv)] = f2bf(x_lo);
        vc[vfrag_index(key, dv + 16)] = f2bf(x_hi);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Residual GEMM (o_proj, K = 2048 / down_proj, K = 4096): 64 workgroups, one 16-column tile
// each, 8 waves splitting K.  Epilogue: h = bf16(h + bf16(bf16(y) * gate)) and the per-tile
// row sums of squares that the next adaRMSNorm consumes (modeling_gemma.py:231-249, 503, 511).
// ---------------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(512, 1) void residual_gemm_kernel(ResidualArgs a) {
  constexpr int NW = 8, NT = 1, KSW = K / 32 / NW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int nt = blockIdx.x;
  const u16* tile_ptr[NT] = {a.w + wfrag_offset(nt, 0, K / 32)};
  bf16x8 w[NT][KSW];
  load_weights<NT, KSW>(w, tile_ptr, wave * KSW, lane);

  __shared__ float red[NW * 4 * NT * 64 * 4];

  for (int m0 = 0; m0 < a.M; m0 += 64) {
    f32x4 acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const int k = (wave * KSW + s) * 32 + g * 8;
      bf16x8 af[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = m0 + mt * 16 + r16;
        af[mt] = row < a.M ? load_frag(a.act + (size_t)row * K + k) : zero_frag();
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt][0] = mfma16x16x32(af[mt], w[0][s], acc[mt][0]);
    }
    store_partials<NW, NT>(red, acc, wave, lane);
    __syncthreads();
    // 1024 outputs, 2 per thread; the 16 columns of a row sit in 16 consecutive threads
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int e = threadIdx.x + it * 512;
      const int r = e >> 4, c = e & 15;
      const int m = m0 + r;
      const int col = nt * 16 + c;
      float hn = 0.f;
      if (m < a.M) {
        const float y = round_bf(reduced<NW, NT>(red, r, c, 0));
        const float gate = round_bf(a.mod_gate[col]);
        const float prod = round_bf(fmul(y, gate));
        u16* hp = a.h + (size_t)m * kWidth + col;
        const u16 hb = f2bf(fadd(bf2f(*hp), prod));
        *hp = hb;
        hn = bf2f(hb);
      }
      float ss = hn * hn;
      ss += __shfl_xor(ss, 1);
      ss += __shfl_xor(ss, 2);
      ss += __shfl_xor(ss, 4);
      ss += __shfl_xor(ss, 8);
      if (c == 0 && m < a.M) a.rowss[(size_t)nt * a.M + m] = ss;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// gate_up: 256 workgroups x 4 waves; WG j owns gate tile j and up tile j (16 columns each).
// Prologue adaRMSNorm(post_attention_layernorm); epilogue GeGLU as the fused reference kernel
// defines it: bf16(gelu_tanh(bf16(g)) * u) (rlinf_fused_denoise.py:166-173).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float gelu_tanh(float x) {
  const float t3 = fmul(x, 0.5f);
  const float t5 = fmul(fmul(x, x), x);
  const float t8 = fadd(x, fmul(t5, 0.044715f));
  const float t11 = tanhf(fmul(t8, 0.7978845608028654f));
  return fmul(t3, fadd(t11, 1.0f));
}

__global__ __launch_bounds__(256, 1) void gate_up_kernel(GateUpArgs a) {
  constexpr int NW = 4, NT = 2, KSW = 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int nt = blockIdx.x;
  const u16* tile_ptr[NT] = {a.wgate + wfrag_offset(nt, 0, 32), a.wup + wfrag_offset(nt, 0, 32)};
  bf16x8 w[NT][KSW];
  load_weights<NT, KSW>(w, tile_ptr, wave * KSW, lane);

  __shared__ float s_rstd[64];
  __shared__ float red[NW * 4 * NT * 64 * 4];
  const float* scale = a.mod;
  const float* shift = a.mod + kWidth;

  for (int m0 = 0; m0 < a.M; m0 += 64) {
    row_rstd(s_rstd, a.rowss, a.M, m0, a.eps);
    __syncthreads();
    f32x4 acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const int k = (wave * KSW + s) * 32 + g * 8;
      bf16x8 af[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = m0 + mt * 16 + r16;
        af[mt] = row < a.M ? norm_frag(a.h, row, k, s_rstd[mt * 16 + r16], scale, shift) : zero_frag();
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = mfma16x16x32(af[mt], w[t][s], acc[mt][t]);
    }
    store_partials<NW, NT>(red, acc, wave, lane);
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 16; e += NW * 64) {
      const int r = e >> 4, c = e & 15;
      const int m = m0 + r;
      if (m >= a.M) continue;
      const float gv = round_bf(reduced<NW, NT>(red, r, c, 0));
      const float uv = reduced<NW, NT>(red, r, c, 1);
      a.act[(size_t)m * kMlp + nt * 16 + c] = f2bf(fmul(gelu_tanh(gv), uv));
    }
    __syncthreads();
  }
}

// =============================================================================================
// attention
// =============================================================================================

// One workgroup = 16 query rows (2 tokens x 8 heads share the single KV head) x one key split;
// the 4 waves split the split's key blocks (32 keys each) further and merge through LDS.
// S^T = K Q^T and O^T = V^T P^T keep every lane on one query row (lane % 16), so the online
// softmax statistics and the P operand never leave the lane.
__global__ __launch_bounds__(256, 1) void attention_kernel(AttnArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int rb = blockIdx.x;            // row block over B * 400 rows
  const int split = blockIdx.y;
  const int rows_per_sample = kHorizon * kQRowsPerTok;  // 400
  const int b = (rb * 16) / rows_per_sample;
  const int qrow = rb * 16 + r16;  // global query row (b*400 + tok*8 + head)

  const u16* kc = a.kcache + (size_t)b * a.s_pad * kHeadDim;
  const u16* vc = a.vcache + (size_t)b * a.s_pad * kHeadDim;
  const uint8_t* valid = a.valid + (size_t)b * a.s_pad;

  bf16x8 qf[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) qf[ds] = load_frag(a.q + (size_t)qrow * kHeadDim + ds * 32 + g * 8);

  const int nkb = a.s_pad >> 5;
  const int kb_lo = split * nkb / a.nsplit, kb_hi = (split + 1) * nkb / a.nsplit;
  const int span = kb_hi - kb_lo;
  const int w_lo = kb_lo + wave * span / 4, w_hi = kb_lo + (wave + 1) * span / 4;

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = w_lo; kb < w_hi; ++kb) {
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ds = 0; ds < 8; ++ds)
        sacc[t] = mfma16x16x32(load_frag(kc + ((size_t)(2 * kb + t) * 8 + ds) * 512 + lane * 8), qf[ds], sacc[t]);
    // scores: bf16(q.k) * 1/16 (exact in bf16), masked keys -> -inf (modeling_gemma.py:265-268)
    float s[8];
    const uint32_t v0 = *reinterpret_cast<const uint32_t*>(valid + kb * 32 + g * 4);
    const uint32_t v1 = *reinterpret_cast<const uint32_t*>(valid + kb * 32 + 16 + g * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = ((v0 >> (8 * i)) & 0xff) ? round_bf(sacc[0][i]) * 0.0625f : -INFINITY;
      s[4 + i] = ((v1 >> (8 * i)) & 0xff) ? round_bf(sacc[1][i]) * 0.0625f : -INFINITY;
    }
    float bm = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) bm = fmaxf(bm, s[i]);
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
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
      oacc[dt] = mfma16x16x32(load_frag(vc + ((size_t)kb * 16 + dt) * 512 + lane * 8), pfrag, oacc[dt]);
    }
  }
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);

  // merge the 4 waves of this workgroup
  __shared__ float s_m[4][16], s_l[4][16];
  __shared__ float s_o[4][16][kHeadDim + 4];
  if (g == 0) {
    s_m[wave][r16] = m_run;
    s_l[wave][r16] = l_run;
  }
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_o[wave][r16][dt * 16 + g * 4 + i] = oacc[dt][i];
  __syncthreads();
  const int rr = threadIdx.x >> 4;        // row 0..15
  const int d0 = (threadIdx.x & 15) * 16;  // 16 dims per thread
  float mw[4], ww[4];
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = s_m[w][rr];
    M = fmaxf(M, mw[w]);
  }
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    ww[w] = (mw[w] == -INFINITY) ? 0.f : __expf(mw[w] - M);
    L += s_l[w][rr] * ww[w];
  }
  const int orow = rb * 16 + rr;
  if (a.nsplit == 1) {
    const float inv = 1.0f / L;
    u16* out = a.out + (size_t)orow * kHeadDim + d0;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) o += s_o[w][rr][d0 + d] * ww[w];
      out[d] = f2bf(o * inv);
    }
  } else {
    float* part = a.part + ((size_t)split * a.rows + orow) * kHeadDim + d0;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) o += s_o[w][rr][d0 + d] * ww[w];
      part[d] = o;
    }
    if ((threadIdx.x & 15) == 0) {
      a.part_m[(size_t)split * a.rows + orow] = M;
      a.part_l[(size_t)split * a.rows + orow] = L;
    }
  }
}

// Combine split-KV partials: O = sum_c O_c e^{m_c - m} / sum_c l_c e^{m_c - m}.
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int d0 = (threadIdx.x & 63) * 4;
  float M = -INFINITY;
  for (int c = 0; c < a.nsplit; ++c) M = fmaxf(M, a.part_m[(size_t)c * a.rows + row]);
  float L = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < a.nsplit; ++c) {
    const float mc = a.part_m[(size_t)c * a.rows + row];
    const float wc = (mc == -INFINITY) ? 0.f : __expf(mc - M);
    L += a.part_l[(size_t)c * a.rows + row] * wc;
    const float4 p4 = *reinterpret_cast<const float4*>(a.part + ((size_t)c * a.rows + row) * kHeadDim + d0);
    o[0] += p4.x * wc;
    o[1] += p4.y * wc;
    o[2] += p4.z * wc;
    o[3] += p4.w * wc;
  }
  const float inv = 1.0f / L;
  u16x4 r4 = {f2bf(o[0] * inv), f2bf(o[1] * inv), f2bf(o[2] * inv), f2bf(o[3] * inv)};
  *reinterpret_cast<u16x4*>(a.out + (size_t)row * kHeadDim + d0) = r4;
}

// =============================================================================================
// host-side launchers (declared in pi05_kernels.h)
// =============================================================================================

hipError_t launch_pack_weight(const void* src, u16* dst, int N, int K, hipStream_t st) {
  const size_t total = (size_t)(N / 16) * (K / 32) * 64;
  const int grid = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  pack_weight_kernel<<<grid, 256, 0, st>>>(reinterpret_cast<const u16*>(src), dst, N, K);
  return hipGetLastError();
}

hipError_t launch_prime_kv(const PrimeKvArgs& a, int depth, hipStream_t st) {
  dim3 grid(32, a.batch, depth);
  prime_kv_kernel<<<grid, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_prime_tables(const PrimeTablesArgs& a, int batch, hipStream_t st) {
  prime_tables_kernel<<<batch, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_gemv_rows(const GemvArgs& a, hipStream_t st) {
  gemv_rows_kernel<<<(a.rows + 3) / 4, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_step_io(const StepIoArgs& a, hipStream_t st) {
  step_io_kernel<<<a.M, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t st) {
  qkv_rope_kernel<<<80, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_o_proj(const ResidualArgs& a, hipStream_t st) {
  residual_gemm_kernel<kHeads * kHeadDim><<<kWidth / 16, 512, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_down(const ResidualArgs& a, hipStream_t st) {
  residual_gemm_kernel<kMlp><<<kWidth / 16, 512, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_gate_up(const GateUpArgs& a, hipStream_t st) {
  gate_up_kernel<<<kMlp / 16, 256, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
  dim3 grid(a.rows / 16, a.nsplit);
  attention_kernel<<<grid, 256, 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.nsplit == 1) return e;
  attn_merge_kernel<<<(a.rows + 3) / 4, 256, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace pi05
