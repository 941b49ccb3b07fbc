// The whole num_steps Euler loop of the pi0.5 action expert as ONE cooperative kernel.
//
// Every workgroup (one per CU, 4 waves) walks the same phase sequence
//   step boundary, then per decoder layer: qkv_rope -> attention -> o_proj -> gate_up -> down
// and takes the work items of each phase that map to it (item i -> workgroup i mod grid).
// Phases hand data to each other through buffers that are written once per launch (one slice
// per Euler step and layer), with write-through (agent-scope, sc1) stores; a producer publishes
// a flag word (the launch epoch) once its stores are complete, and a consumer first issues its
// own weight loads, then polls the flags of the phase it depends on, then reads the data with
// ordinary cached loads.  Because no buffer slice is read before it is written within a launch,
// no cache can hold a stale copy, so no cache flush or invalidate is ever needed.
//
// Attention splits the keys over several workgroups; the last split of a row block to arrive
// (device-scope counter) merges them.  down_proj splits K four ways the same way; the last
// arrival adds the partials in fixed order and applies the gated residual.  Partials are read
// back with coherent loads because their buffers are reused across layers.
//
// Every wait is bounded: on timeout the kernel records an error and all workgroups leave.

#include "pi05_blocks.h"
#include "pi05_kernels.h"

namespace pi05 {

constexpr int kThreads = 256;  // 4 waves: one per SIMD, up to 512 registers per lane
constexpr int kWaves = 4;
constexpr int kSpinLimit = 1 << 20;  // polls (each >= ~1 us): a legitimate wait spans a few phases

// ---- coherent (agent-scope, write-through) accesses -------------------------------------------
__device__ __forceinline__ void st_u16(u16* p, u16 v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_u32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f32(float* p, float v) { st_u32(p, __float_as_uint(v)); }
__device__ __forceinline__ void st_u64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f32x4(float* p, float4 v) {
  st_u64(p, (uint64_t)__float_as_uint(v.x) | ((uint64_t)__float_as_uint(v.y) << 32));
  st_u64(p + 2, (uint64_t)__float_as_uint(v.z) | ((uint64_t)__float_as_uint(v.w) << 32));
}
__device__ __forceinline__ uint32_t ld_u32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_f32(const float* p) { return __uint_as_float(ld_u32(p)); }
__device__ __forceinline__ float4 ld_f32x4(const float* p) {
  const uint64_t a = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return float4{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                __uint_as_float((uint32_t)(b >> 32))};
}

// ---- phase bookkeeping ------------------------------------------------------------------------
enum { kPhIo = 0, kPhQkv = 1, kPhAttn = 2, kPhO = 3, kPhGu = 4, kPhDown = 5, kNumPh = 6 };
constexpr int kQkvItems = 80;
constexpr int kOItems = kWidth / 16;  // 64
constexpr int kGuItems = kMlp / 16;   // 256
constexpr int kDownSplit = 4;

__device__ __forceinline__ unsigned* flags_of(const MegaArgs& a, int s, int l, int ph) {
  return a.flags + ((size_t)(s * (a.depth + 1) + l) * kNumPh + ph) * a.flag_stride;
}

// Wait until flags[0, n) all equal this launch's epoch.  Wave 0 polls; uniform result.
__device__ bool wait_flags(const MegaArgs& a, const unsigned* f, int n, int* s_flag) {
  if (threadIdx.x < 64) {
    int ok = 1;
    for (int spins = 0;; ++spins) {
      bool done = true;
      for (int i = threadIdx.x; i < n; i += 64) done &= (ld_u32(f + i) == a.epoch);
      if (__all(done)) break;
      if (spins > kSpinLimit || ld_u32(a.err) != 0) {
        if (threadIdx.x == 0) {
          st_u32(a.err, 1u);
          __hip_atomic_store(a.host_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) *s_flag = ok;
  }
  __syncthreads();
  const bool ok = *s_flag != 0;
  __syncthreads();
  return ok;
}

// All of this workgroup's coherent stores are complete -> publish flag `item`.
__device__ __forceinline__ void publish(const MegaArgs& a, unsigned* f, int item) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) st_u32(f + item, a.epoch);
}

// Last-arrival election on a device-scope counter that every launch advances by `n` per slot.
__device__ __forceinline__ bool last_arrival(const MegaArgs& a, unsigned* ctr, unsigned n, int* s_flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = old == a.epoch * n - 1u;
  }
  __syncthreads();
  const bool last = *s_flag != 0;
  __syncthreads();
  return last;
}

// =============================================================================================
// step boundary: final norm + action_out_proj + Euler of step s-1, action_in_proj of step s.
// Items: token rows.  x[s] = Euler(x[s-1], v_{s-1}); h[s][0] = bf16(action_in_proj(x[s])).
// =============================================================================================
__device__ bool phase_io(const MegaArgs& a, int s, float* smem, int* s_flag) {
  const int M = a.M, L = a.depth, NN = 2 * L + 1;
  const int tid = threadIdx.x;
  const int j = tid >> 3, part = tid & 7;
  const int c0 = tid * 4;
  float* s_n = smem;          // [W]
  float* s_x = smem + kWidth; // [a]
  float* s_rstd = s_x + kActDim;
  bool waited = false;
  for (int m = blockIdx.x; m < M; m += gridDim.x) {
    const bool has_prev = s > 0, has_next = s < a.steps;
    // ---- loads first
    float4 wo[32];
    float4 rs = {0.f, 0.f, 0.f, 0.f};
    u16x4 hv = {0, 0, 0, 0};
    float4 sc = {0.f, 0.f, 0.f, 0.f}, sh = {0.f, 0.f, 0.f, 0.f};
    float bo = 0.f;
    if (has_prev) {
#pragma unroll
      for (int q = 0; q < 32; ++q) wo[q] = *reinterpret_cast<const float4*>(a.out_w + (size_t)j * kWidth + part * 128 + q * 4);
      const float* fmod = a.table + ((size_t)(s - 1) * NN + (NN - 1)) * kModW;
      sc = *reinterpret_cast<const float4*>(fmod + c0);
      sh = *reinterpret_cast<const float4*>(fmod + kWidth + c0);
      bo = a.out_b[j];
    }
    float4 wi[4][8];
    float4 bi = {0.f, 0.f, 0.f, 0.f};
    if (has_next) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int k = 0; k < 8; ++k) wi[q][k] = *reinterpret_cast<const float4*>(a.in_w + (size_t)(c0 + q) * kActDim + k * 4);
      bi = *reinterpret_cast<const float4*>(a.in_b + c0);
    }
    if (has_prev && !waited) {
      if (!wait_flags(a, flags_of(a, s - 1, L - 1, kPhDown), kOItems, s_flag)) return false;
      waited = true;
    }
    float xj = 0.f;
    if (has_prev) {
      const size_t sl = (size_t)(s - 1) * (L + 1) + L;
      if (tid < 16) rs = *reinterpret_cast<const float4*>(a.rowss + (sl * M + m) * kRowSlots + tid * 4);
      hv = *reinterpret_cast<const u16x4*>(a.h + (sl * M + m) * kWidth + c0);
      if (part == 0) xj = (s == 1 ? a.x_io : a.x + (size_t)(s - 1) * M * kActDim)[(size_t)m * kActDim + j];
      // final adaRMSNorm (model.norm, modeling_gemma.py:782-783)
      if (tid < 16) {
        float v = (rs.x + rs.y) + (rs.z + rs.w);
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        v += __shfl_xor(v, 4);
        v += __shfl_xor(v, 8);
        if (tid == 0) *s_rstd = 1.0f / sqrtf(fadd(v * (1.0f / kWidth), a.eps));
      }
      __syncthreads();
      const float rstd = *s_rstd;
      const float scs[4] = {sc.x, sc.y, sc.z, sc.w};
      const float shs[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) s_n[c0 + q] = round_bf(fadd(fmul(fmul(bf2f(hv[q]), rstd), fadd(1.0f, scs[q])), shs[q]));
      __syncthreads();
      // v = action_out_proj(n), fp32 (engine.py:767)
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const float* n = s_n + part * 128 + q * 4;
        acc += wo[q].x * n[0] + wo[q].y * n[1] + wo[q].z * n[2] + wo[q].w * n[3];
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if (part == 0) {
        const float v = acc + bo;
        const float* e = a.euler + (size_t)(s - 1) * 4;  // t, 1 - t, x0_weight, x1_weight
        // flow_ode mean in the reference's op order (engine.py:664-675)
        const float x0_pred = fsub(xj, fmul(v, e[0]));
        const float x1_pred = fadd(xj, fmul(v, e[1]));
        const float xn = fadd(fmul(x0_pred, e[2]), fmul(x1_pred, e[3]));
        st_f32((s == a.steps ? a.x_io : a.x + (size_t)s * M * kActDim) + (size_t)m * kActDim + j, xn);
        s_x[j] = xn;
        if (a.trace) st_f32(a.trace + ((size_t)(s - 1) * M + m) * kActDim + j, v);
      }
    } else if (tid < kActDim) {
      s_x[tid] = a.x_io[(size_t)m * kActDim + tid];
    }
    __syncthreads();
    if (has_next) {
      // h = bf16(action_in_proj(x)) (pi0_pytorch.py:303-306; modeling_gemma.py:724-725)
      const size_t sl = (size_t)s * (L + 1);
      const float bis[4] = {bi.x, bi.y, bi.z, bi.w};
      float ss = 0.f;
      u16 h4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          acc += wi[q][k].x * s_x[4 * k] + wi[q][k].y * s_x[4 * k + 1] + wi[q][k].z * s_x[4 * k + 2] + wi[q][k].w * s_x[4 * k + 3];
        h4[q] = f2bf(acc + bis[q]);
        const float hf = bf2f(h4[q]);
        ss += hf * hf;
      }
      st_u64(a.h + (sl * M + m) * kWidth + c0,
             (uint64_t)h4[0] | ((uint64_t)h4[1] << 16) | ((uint64_t)h4[2] << 32) | ((uint64_t)h4[3] << 48));
      ss += __shfl_xor(ss, 1);
      ss += __shfl_xor(ss, 2);
      if ((tid & 3) == 0) st_f32(a.rowss + (sl * M + m) * kRowSlots + (c0 >> 4), ss);
    }
    publish(a, flags_of(a, s, 0, kPhIo), m);
  }
  return true;
}

// =============================================================================================
// adaRMSNorm-prologue GEMM tile (K = 1024, 4 waves x 8 k-steps): qkv_rope and gate_up.
// =============================================================================================
template <int MODE>
__device__ bool phase_norm_gemm(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  constexpr int NT = 2, KSW = 8, KSTEPS = kWidth / 32;
  const int M = a.M, L = a.depth, NN = 2 * L + 1;
  const int n_items = MODE == kModeQkv ? kQkvItems : kGuItems;
  const int p = blockIdx.x;
  if (p >= n_items) return true;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int ks0 = wave * KSW;
  const int emt = tid >> 6, eg = (tid & 63) >> 4, ec = tid & 15;
  const size_t slw = (size_t)s * L + l;  // (step, layer) slice of per-layer arenas
  const u16* wl = a.wpack + (size_t)l * kLayerElems;

  int tile0;
  bool rotated = false;
  int head = 0, dt = 0;
  const u16* tp[NT];
  const u16* hin;
  const float* rin;
  const float* mod;
  if constexpr (MODE == kModeQkv) {
    rotated = p < 72;
    head = p >> 3;
    dt = p & 7;
    tile0 = rotated ? head * 16 + dt : 144 + 2 * (p - 72);
    const int tile1 = rotated ? head * 16 + 8 + dt : tile0 + 1;
    tp[0] = wl + kOffQkv + (size_t)tile0 * KSTEPS * 512;
    tp[1] = wl + kOffQkv + (size_t)tile1 * KSTEPS * 512;
    const size_t sl = (size_t)s * (L + 1) + l;
    hin = a.h + sl * M * kWidth;
    rin = a.rowss + sl * M * kRowSlots;
    mod = a.table + ((size_t)s * NN + 2 * l) * kModW;
  } else {
    tile0 = p;
    tp[0] = wl + kOffGate + (size_t)p * KSTEPS * 512;
    tp[1] = wl + kOffUp + (size_t)p * KSTEPS * 512;
    hin = a.hmid + slw * M * kWidth;
    rin = a.rowss_mid + slw * M * kRowSlots;
    mod = a.table + ((size_t)s * NN + 2 * l + 1) * kModW;
  }
  // ---- weights first: they do not depend on the previous phase
  bf16x8 w[NT][KSW];
  load_weights<NT, KSW>(w, tp, ks0, lane);
  const float4 mod4a = *reinterpret_cast<const float4*>(mod + tid * 8);
  const float4 mod4b = *reinterpret_cast<const float4*>(mod + tid * 8 + 4);
  if constexpr (MODE == kModeQkv) {
    if (!wait_flags(a, l == 0 ? flags_of(a, s, 0, kPhIo) : flags_of(a, s, l - 1, kPhDown), l == 0 ? M : kOItems, s_flag))
      return false;
  } else {
    if (!wait_flags(a, flags_of(a, s, l, kPhO), kOItems, s_flag)) return false;
  }

  float* s_mod = smem;                    // 1 + scale | shift
  float* s_rstd = smem + 2 * kWidth;      // [64]
  float* red = s_rstd + 64;               // [4 waves][4][NT][64][4]
  {
    const float v[8] = {mod4a.x, mod4a.y, mod4a.z, mod4a.w, mod4b.x, mod4b.y, mod4b.z, mod4b.w};
    const bool is_scale = tid * 8 < kWidth;
#pragma unroll
    for (int q = 0; q < 8; ++q) s_mod[tid * 8 + q] = is_scale ? fadd(1.0f, v[q]) : v[q];
  }
  for (int m0 = 0; m0 < M; m0 += 64) {
    u16x8 hr[4][KSW];
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) {
      const int k = (ks0 + s2) * 32 + g * 8;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = m0 + mt * 16 + r16;
        const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        hr[mt][s2] = row < M ? *reinterpret_cast<const u16x8*>(hin + (size_t)row * kWidth + k) : z;
      }
    }
    float4 rs[4];  // row statistics: 4 threads per row, 16 partial sums each
    const int srow = tid >> 2, q4 = tid & 3;
    const bool rvalid = m0 + srow < M;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      rs[q] = rvalid ? *reinterpret_cast<const float4*>(rin + (size_t)(m0 + srow) * kRowSlots + q4 * 16 + q * 4) : float4{0.f, 0.f, 0.f, 0.f};
    float ep_cs[4][4];
    if constexpr (MODE == kModeQkv) {
      if (rotated) {
        const int d = dt * 16 + ec;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + emt * 16 + eg * 4 + i;
          if (m < M) {
            const u16* cs = a.cos_tab + (size_t)m * kHeadDim;
            const u16* sn = a.sin_tab + (size_t)m * kHeadDim;
            ep_cs[i][0] = bf2f(cs[d]);
            ep_cs[i][1] = bf2f(sn[d]);
            ep_cs[i][2] = bf2f(cs[d + kHalfDim]);
            ep_cs[i][3] = bf2f(sn[d + kHalfDim]);
          }
        }
      }
    }
    {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) v += (rs[q].x + rs[q].y) + (rs[q].z + rs[q].w);
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      if (q4 == 0) s_rstd[srow] = 1.0f / sqrtf(fadd(v * (1.0f / kWidth), a.eps));
    }
    __syncthreads();
    // adaRMSNorm (modeling_gemma.py:82-116): A = bf16((h * rstd) * (1 + scale) + shift)
    f32x4 acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float rstd[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) rstd[mt] = s_rstd[mt * 16 + r16];
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) {
      const int k = (ks0 + s2) * 32 + g * 8;
      const f32x4 sc0 = *reinterpret_cast<const f32x4*>(s_mod + k);
      const f32x4 sc1 = *reinterpret_cast<const f32x4*>(s_mod + k + 4);
      const f32x4 sh0 = *reinterpret_cast<const f32x4*>(s_mod + kWidth + k);
      const f32x4 sh1 = *reinterpret_cast<const f32x4*>(s_mod + kWidth + k + 4);
      const float scs[8] = {sc0[0], sc0[1], sc0[2], sc0[3], sc1[0], sc1[1], sc1[2], sc1[3]};
      const float shs[8] = {sh0[0], sh0[1], sh0[2], sh0[3], sh1[0], sh1[1], sh1[2], sh1[3]};
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        u16x8 o;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) o[jj] = f2bf(fadd(fmul(fmul(bf2f(hr[mt][s2][jj]), rstd[mt]), scs[jj]), shs[jj]));
        const bf16x8 af = as_bf16x8(o);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = mfma16x16x32(af, w[t][s2], acc[mt][t]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        *reinterpret_cast<f32x4*>(red + ((((size_t)wave * 4 + mt) * NT + t) * 64 + lane) * 4) = acc[mt][t];
    __syncthreads();
    f32x4 v0 = *reinterpret_cast<const f32x4*>(red + (((size_t)emt * NT + 0) * 64 + (tid & 63)) * 4);
    f32x4 v1 = *reinterpret_cast<const f32x4*>(red + (((size_t)emt * NT + 1) * 64 + (tid & 63)) * 4);
#pragma unroll
    for (int w2 = 1; w2 < kWaves; ++w2) {
      v0 += *reinterpret_cast<const f32x4*>(red + ((((size_t)w2 * 4 + emt) * NT + 0) * 64 + (tid & 63)) * 4);
      v1 += *reinterpret_cast<const f32x4*>(red + ((((size_t)w2 * 4 + emt) * NT + 1) * 64 + (tid & 63)) * 4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + emt * 16 + eg * 4 + i;
      if (m >= M) continue;
      if constexpr (MODE == kModeQkv) {
        const float x_lo = round_bf(v0[i]);
        const float x_hi = round_bf(v1[i]);
        const int b = m / kHorizon, tok = m % kHorizon;
        if (rotated) {
          // (x*cos) + (rotate_half(x)*sin), rotate_half(x) = cat(-x_hi, x_lo)
          // (rlinf_fused_denoise.py:264-278; modeling_gemma.py:185-216)
          const int d = dt * 16 + ec;
          const float o_lo = fsub(fmul(x_lo, ep_cs[i][0]), fmul(x_hi, ep_cs[i][1]));
          const float o_hi = fadd(fmul(x_hi, ep_cs[i][2]), fmul(x_lo, ep_cs[i][3]));
          if (head < kHeads) {
            u16* qrow = a.q + (slw * M + m) * (kHeads * kHeadDim) + head * kHeadDim;
            st_u16(qrow + d, f2bf(o_lo));
            st_u16(qrow + d + kHalfDim, f2bf(o_hi));
          } else {
            u16* kc = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
            st_u16(kc + kfrag_index(tok, d), f2bf(o_lo));
            st_u16(kc + kfrag_index(tok, d + kHalfDim), f2bf(o_hi));
          }
        } else {
          u16* vc = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
          const int dv = (tile0 - 144) * 16 + ec;
          st_u16(vc + vfrag_index(tok, dv), f2bf(x_lo));
          st_u16(vc + vfrag_index(tok, dv + 16), f2bf(x_hi));
        }
      } else {
        // GeGLU as the fused reference kernel defines it: bf16(gelu_tanh(bf16(g)) * u)
        // (rlinf_fused_denoise.py:166-173)
        st_u16(a.act + (slw * M + m) * kMlp + tile0 * 16 + ec, f2bf(fmul(gelu_tanh(round_bf(v0[i])), v1[i])));
      }
    }
    __syncthreads();
  }
  publish(a, flags_of(a, s, l, MODE == kModeQkv ? kPhQkv : kPhGu), p);
  return true;
}

// =============================================================================================
// attention: item = (row block of 16 query rows, key split); 4 waves x 32-key blocks.
// Keys [0, s_pre) come from the static prefix cache, keys [s_pre, s_pre + 64) from this step's
// suffix blocks (50 valid).
// =============================================================================================
__device__ bool phase_attn(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  const int M = a.M, L = a.depth;
  const int nrb = M * kQRowsPerTok / 16;
  const int n_items = nrb * a.nsplit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const size_t slw = (size_t)s * L + l;
  const int nkb_pre = a.s_pre >> 5;
  const int nkb = nkb_pre + 2;
  const int rows = M * kQRowsPerTok;
  bool waited = false;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int rb = item % nrb, split = item / nrb;
    const int b = (rb * 16) / (kHorizon * kQRowsPerTok);
    const int qrow = rb * 16 + r16;
    const u16* kpre = a.kpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* vpre = a.vpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* ksf = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
    const u16* vsf = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
    const uint8_t* valid = a.valid + (size_t)b * (a.s_pre + 64);
    const int kb_lo = split * nkb / a.nsplit, kb_hi = (split + 1) * nkb / a.nsplit;
    const int span = kb_hi - kb_lo;
    const int w_lo = kb_lo + wave * span / 4, w_hi = kb_lo + (wave + 1) * span / 4;
    const int n = w_hi - w_lo;
    // block kb of this item: prefix blocks from the static cache, the last two from this step
    auto load = [&](KvBlock& blk, int kb) {
      if (kb >= nkb_pre) load_kv_block(blk, ksf, vsf, valid + kb * 32, kb - nkb_pre, lane);
      else load_kv_block(blk, kpre, vpre, valid + kb * 32, kb, lane);
    };
    // One block in flight per wave (two would not fit the 256 VGPRs that MFMA operands live
    // in); the split count is chosen so that a wave normally owns a single block.
    KvBlock blk;
    // prefix blocks do not depend on this step: fetch the first one before waiting
    if (n > 0 && w_lo < nkb_pre) load(blk, w_lo);
    if (!waited) {
      if (!wait_flags(a, flags_of(a, s, l, kPhQkv), kQkvItems, s_flag)) return false;
      waited = true;
    }
    if (n > 0 && w_lo >= nkb_pre) load(blk, w_lo);
    bf16x8 qf[8];
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qf[ds] = load_frag(a.q + (slw * M) * (kHeads * kHeadDim) + (size_t)qrow * kHeadDim + ds * 32 + g * 8);
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 oacc[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < n; ++i) {
      if (i > 0) load(blk, w_lo + i);
      attend_block(blk, qf, m_run, l_run, oacc);
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);

    // ---- merge the 4 waves of this workgroup
    float* s_m = smem;            // [4][16]
    float* s_l = smem + 64;       // [4][16]
    float* s_o = smem + 128;      // [4][16][D + 4]
    constexpr int OSTR = kHeadDim + 4;
    if (g == 0) {
      s_m[wave * 16 + r16] = m_run;
      s_l[wave * 16 + r16] = l_run;
    }
#pragma unroll
    for (int d = 0; d < 16; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_o[(wave * 16 + r16) * OSTR + d * 16 + g * 4 + i] = oacc[d][i];
    __syncthreads();
    const int rr = tid >> 4, d0 = (tid & 15) * 16;
    float Mx = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) Mx = fmaxf(Mx, s_m[w2 * 16 + rr]);
    float ww[4], Lx = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      ww[w2] = (s_m[w2 * 16 + rr] == -INFINITY) ? 0.f : __expf(s_m[w2 * 16 + rr] - Mx);
      Lx += s_l[w2 * 16 + rr] * ww[w2];
    }
    float o[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) v += s_o[(w2 * 16 + rr) * OSTR + d0 + d] * ww[w2];
      o[d] = v;
    }
    __syncthreads();
    const int orow = rb * 16 + rr;
    bool finish = true;
    if (a.nsplit > 1) {
      float* part = a.apart + ((size_t)split * rows + orow) * kHeadDim + d0;
#pragma unroll
      for (int d = 0; d < 16; d += 4) st_f32x4(part + d, float4{o[d], o[d + 1], o[d + 2], o[d + 3]});
      if ((tid & 15) == 0) {
        st_f32(a.apart_m + (size_t)split * rows + orow, Mx);
        st_f32(a.apart_l + (size_t)split * rows + orow, Lx);
      }
      finish = last_arrival(a, a.counters + slw * nrb + rb, (unsigned)a.nsplit, s_flag);
      if (finish) {
        // combine the splits in fixed order: O = sum_c O_c e^{m_c - m} / sum_c l_c e^{m_c - m}
        float mc[kMaxAttnSplits];
#pragma unroll
        for (int c = 0; c < kMaxAttnSplits; ++c) mc[c] = c < a.nsplit ? ld_f32(a.apart_m + (size_t)c * rows + orow) : -INFINITY;
        Mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < kMaxAttnSplits; ++c) Mx = fmaxf(Mx, mc[c]);
        Lx = 0.f;
#pragma unroll
        for (int d = 0; d < 16; ++d) o[d] = 0.f;
        for (int c0 = 0; c0 < a.nsplit; c0 += 4) {
          float lc[4];
          float4 oc[4][4];
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            if (c0 + cc < a.nsplit) {
              lc[cc] = ld_f32(a.apart_l + (size_t)(c0 + cc) * rows + orow);
              const float* pp = a.apart + ((size_t)(c0 + cc) * rows + orow) * kHeadDim + d0;
#pragma unroll
              for (int q = 0; q < 4; ++q) oc[cc][q] = ld_f32x4(pp + 4 * q);
            }
          }
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            if (c0 + cc < a.nsplit) {
              float m_c = -INFINITY;
#pragma unroll
              for (int c = 0; c < kMaxAttnSplits; ++c) m_c = c == c0 + cc ? mc[c] : m_c;
              const float wc = (m_c == -INFINITY) ? 0.f : __expf(m_c - Mx);
              Lx += lc[cc] * wc;
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                o[4 * q] += oc[cc][q].x * wc;
                o[4 * q + 1] += oc[cc][q].y * wc;
                o[4 * q + 2] += oc[cc][q].z * wc;
                o[4 * q + 3] += oc[cc][q].w * wc;
              }
            }
          }
        }
      }
    }
    if (finish) {
      const float inv = 1.0f / Lx;
      u16* out = a.o + (slw * M) * (kHeads * kHeadDim) + (size_t)orow * kHeadDim + d0;
#pragma unroll
      for (int d = 0; d < 16; d += 4)
        st_u64(out + d, (uint64_t)f2bf(o[d] * inv) | ((uint64_t)f2bf(o[d + 1] * inv) << 16) |
                            ((uint64_t)f2bf(o[d + 2] * inv) << 32) | ((uint64_t)f2bf(o[d + 3] * inv) << 48));
      publish(a, flags_of(a, s, l, kPhAttn), rb);
    }
  }
  return true;
}

// =============================================================================================
// o_proj (K = 2048, 4 waves x 16 k-steps, item = 16-column tile) and down_proj (K = 4096 split
// four ways over workgroups, 4 waves x 8 k-steps, item = (tile, K quarter)).  Epilogue: the
// gated residual h = bf16(h + bf16(bf16(y) * gate)) (modeling_gemma.py:231-249, 503, 511) and
// the tile's row sums of squares for the next adaRMSNorm.
// =============================================================================================
// acc[mt] = A[m0 + mt*16 .. +16, k-steps kstep0 .. +KSW] x W-tile, for the 4 m-tiles of a
// 64-row group.  KSW <= 8: every A fragment is loaded up front; KSW = 16: one m-tile in flight
// while the previous one is multiplied (keeps the A operand within 128 VGPRs).
template <int KSW>
__device__ __forceinline__ void load_a_tile(bf16x8 (&af)[KSW], const u16* act, int K, int row, int M, int kstep0, int g) {
#pragma unroll
  for (int s2 = 0; s2 < KSW; ++s2) af[s2] = row < M ? load_frag(act + (size_t)row * K + (kstep0 + s2) * 32 + g * 8) : zero_frag();
}

template <int KSW>
__device__ __forceinline__ void residual_mma(f32x4 (&acc)[4], const bf16x8 (&w)[KSW], const u16* act, int K, int m0, int M,
                                             int kstep0, int lane) {
  const int g = lane >> 4, r16 = lane & 15;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (KSW <= 8) {
    bf16x8 af[4][KSW];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) load_a_tile<KSW>(af[mt], act, K, m0 + mt * 16 + r16, M, kstep0, g);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = mfma16x16x32(af[mt][s2], w[s2], acc[mt]);
  } else {
    bf16x8 a0[KSW], a1[KSW];
    load_a_tile<KSW>(a0, act, K, m0 + r16, M, kstep0, g);
    load_a_tile<KSW>(a1, act, K, m0 + 16 + r16, M, kstep0, g);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) acc[0] = mfma16x16x32(a0[s2], w[s2], acc[0]);
    load_a_tile<KSW>(a0, act, K, m0 + 32 + r16, M, kstep0, g);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) acc[1] = mfma16x16x32(a1[s2], w[s2], acc[1]);
    load_a_tile<KSW>(a1, act, K, m0 + 48 + r16, M, kstep0, g);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) acc[2] = mfma16x16x32(a0[s2], w[s2], acc[2]);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) acc[3] = mfma16x16x32(a1[s2], w[s2], acc[3]);
  }
}

// y (4 rows of column `col`, reduced over K) -> residual update of rows m0 + emt*16 + eg*4 + i.
__device__ __forceinline__ void residual_epilogue(const MegaArgs& a, const f32x4& y4, const u16* hres, u16* hout, float* rout,
                                                  float gate, int m0, int tile, int col) {
  const int tid = threadIdx.x, emt = tid >> 6, eg = (tid & 63) >> 4, ec = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + emt * 16 + eg * 4 + i;
    float hn = 0.f;
    if (m < a.M) {
      const float prod = round_bf(fmul(round_bf(y4[i]), gate));
      const u16 hb = f2bf(fadd(bf2f(hres[(size_t)m * kWidth + col]), prod));
      st_u16(hout + (size_t)m * kWidth + col, hb);
      hn = bf2f(hb);
    }
    float ss = hn * hn;  // the 16 columns of row m sit in 16 consecutive lanes
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 8);
    if (ec == 0 && m < a.M) st_f32(rout + (size_t)m * kRowSlots + tile, ss);
  }
}

__device__ bool phase_o(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  constexpr int K = kHeads * kHeadDim, KSW = K / 32 / kWaves;  // 16
  const int p = blockIdx.x;
  if (p >= kOItems) return true;
  const int M = a.M, L = a.depth, NN = 2 * L + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int emt = tid >> 6, ec = tid & 15;
  const size_t slw = (size_t)s * L + l;
  const u16* tp[1] = {a.wpack + (size_t)l * kLayerElems + kOffO + (size_t)p * (K / 32) * 512};
  bf16x8 w[1][KSW];
  load_weights<1, KSW>(w, tp, wave * KSW, lane);
  const float* mod = a.table + ((size_t)s * NN + 2 * l) * kModW;
  const int col = p * 16 + ec;
  const float gate = round_bf(mod[2 * kWidth + col]);
  if (!wait_flags(a, flags_of(a, s, l, kPhAttn), M * kQRowsPerTok / 16, s_flag)) return false;
  const u16* act = a.o + slw * M * K;
  const u16* hres = a.h + ((size_t)s * (L + 1) + l) * M * kWidth;
  u16* hout = a.hmid + slw * M * kWidth;
  float* rout = a.rowss_mid + slw * M * kRowSlots;
  float* red = smem;
  for (int m0 = 0; m0 < M; m0 += 64) {
    f32x4 acc[4];
    residual_mma<KSW>(acc, w[0], act, K, m0, M, wave * KSW, lane);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4*>(red + (((size_t)wave * 4 + mt) * 64 + lane) * 4) = acc[mt];
    __syncthreads();
    f32x4 y4 = *reinterpret_cast<const f32x4*>(red + ((size_t)emt * 64 + (tid & 63)) * 4);
#pragma unroll
    for (int w2 = 1; w2 < kWaves; ++w2) y4 += *reinterpret_cast<const f32x4*>(red + (((size_t)w2 * 4 + emt) * 64 + (tid & 63)) * 4);
    residual_epilogue(a, y4, hres, hout, rout, gate, m0, p, col);
    __syncthreads();
  }
  publish(a, flags_of(a, s, l, kPhO), p);
  return true;
}

__device__ bool phase_down(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  constexpr int K = kMlp, KSW = K / kDownSplit / 32 / kWaves;  // 8
  const int M = a.M, L = a.depth, NN = 2 * L + 1;
  const int n_items = kOItems * kDownSplit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int emt = tid >> 6, ec = tid & 15;
  const size_t slw = (size_t)s * L + l;
  bool waited = false;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int nt = item % kOItems, ksp = item / kOItems;
    const int kstep0 = ksp * (K / 32 / kDownSplit) + wave * KSW;
    const u16* tp[1] = {a.wpack + (size_t)l * kLayerElems + kOffDown + (size_t)nt * (K / 32) * 512};
    bf16x8 w[1][KSW];
    load_weights<1, KSW>(w, tp, kstep0, lane);
    const float* mod = a.table + ((size_t)s * NN + 2 * l + 1) * kModW;
    const int col = nt * 16 + ec;
    const float gate = round_bf(mod[2 * kWidth + col]);
    if (!waited) {
      if (!wait_flags(a, flags_of(a, s, l, kPhGu), kGuItems, s_flag)) return false;
      waited = true;
    }
    const u16* act = a.act + slw * M * K;
    float* red = smem;
    for (int m0 = 0; m0 < M; m0 += 64) {
      f32x4 acc[4];
      residual_mma<KSW>(acc, w[0], act, K, m0, M, kstep0, lane);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4*>(red + (((size_t)wave * 4 + mt) * 64 + lane) * 4) = acc[mt];
      __syncthreads();
      f32x4 y4 = *reinterpret_cast<const f32x4*>(red + ((size_t)emt * 64 + (tid & 63)) * 4);
#pragma unroll
      for (int w2 = 1; w2 < kWaves; ++w2) y4 += *reinterpret_cast<const f32x4*>(red + (((size_t)w2 * 4 + emt) * 64 + (tid & 63)) * 4);
      // partial [ksplit][tile][row][16] (rows = m0 + emt*16 + eg*4 + i)
      float* part = a.dpart + (((size_t)ksp * kOItems + nt) * a.mp + m0 + emt * 16 + ((tid & 63) >> 4) * 4) * 16 + ec;
#pragma unroll
      for (int i = 0; i < 4; ++i) st_f32(part + i * 16, y4[i]);
      __syncthreads();
    }
    if (last_arrival(a, a.counters + a.ctr_down_off + slw * kOItems + nt, (unsigned)kDownSplit, s_flag)) {
      const u16* hres = a.hmid + slw * M * kWidth;
      u16* hout = a.h + ((size_t)s * (L + 1) + l + 1) * M * kWidth;
      float* rout = a.rowss + ((size_t)s * (L + 1) + l + 1) * M * kRowSlots;
      for (int m0 = 0; m0 < M; m0 += 64) {
        f32x4 y4 = {0.f, 0.f, 0.f, 0.f};
        const int rbase = m0 + emt * 16 + ((tid & 63) >> 4) * 4;
        float pv[kDownSplit][4];
#pragma unroll
        for (int q = 0; q < kDownSplit; ++q)
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[q][i] = ld_f32(a.dpart + (((size_t)q * kOItems + nt) * a.mp + rbase + i) * 16 + ec);
#pragma unroll
        for (int q = 0; q < kDownSplit; ++q)
#pragma unroll
          for (int i = 0; i < 4; ++i) y4[i] += pv[q][i];
        residual_epilogue(a, y4, hres, hout, rout, gate, m0, nt, col);
      }
      publish(a, flags_of(a, s, l, kPhDown), nt);
    }
  }
  return true;
}

// =============================================================================================
// the kernel
// =============================================================================================
constexpr int kSmemFloats = 16768 + 128;  // max over phases (attention: 128 + 4*16*(D+4))

__global__ __launch_bounds__(kThreads, 1) void denoise_loop_kernel(MegaArgs a) {
  __shared__ __align__(16) float smem[kSmemFloats];
  __shared__ int s_flag;
  for (int s = 0; s <= a.steps; ++s) {
    if (!phase_io(a, s, smem, &s_flag)) return;
    if (s == a.steps) break;
    for (int l = 0; l < a.depth; ++l) {
      if (!phase_norm_gemm<kModeQkv>(a, s, l, smem, &s_flag)) return;
      if (!phase_attn(a, s, l, smem, &s_flag)) return;
      if (!phase_o(a, s, l, smem, &s_flag)) return;
      if (!phase_norm_gemm<kModeGateUp>(a, s, l, smem, &s_flag)) return;
      if (!phase_down(a, s, l, smem, &s_flag)) return;
    }
  }
}

hipError_t launch_denoise_loop(const MegaArgs& a, int grid, hipStream_t st) {
  void* args[] = {const_cast<MegaArgs*>(&a)};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(denoise_loop_kernel), dim3(grid), dim3(kThreads), args, 0, st);
}

int denoise_loop_threads() { return kThreads; }

const void* denoise_loop_kernel_ptr() { return reinterpret_cast<const void*>(denoise_loop_kernel); }

}  // namespace pi05
