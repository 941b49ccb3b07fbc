// The whole num_steps Euler loop of the pi0.5 action expert as ONE cooperative kernel.
//
// Every workgroup (one per CU, 4 waves) walks the same phase sequence
//   step boundary, then per decoder layer: qkv -> attention -> o_proj -> gate_up -> down
// and takes the work items of each phase that map to it (item i -> workgroup i mod grid).
// Phases hand data to each other through buffers that are written once per launch (one slice
// per Euler step and layer), with write-through (agent-scope, sc1) stores; a producer publishes
// completion by incrementing the phase's counter once its stores are complete, and a consumer
// first issues its own weight loads, then polls the counter of the phase it depends on, then
// reads the data with ordinary cached loads.  Because no buffer slice is read before it is written within a launch,
// no cache can hold a stale copy, so no cache flush or invalidate is ever needed.
//
// Activations are stored as MFMA A-operand fragments (afrag_offset), rows padded per sample to
// 64 (row r = b*64 + t, t < 50 action tokens; padded rows are never written and stay zero), so
// every operand fetch is a 1 KiB-contiguous wave load and every 64-row group is one sample.
// Epilogues transpose their output tile through LDS and write whole 16-byte row chunks.
//
// Attention splits the keys over several workgroups; the last split of a row block to arrive
// (device-scope counter) merges them.  o_proj and down_proj split K four ways the same way; the
// last arrival adds the partials in fixed order and applies the gated residual.  Partials are
// per-(step, layer) slices too, so the merges read them with plain loads.
//
// Every wait is bounded: on timeout the kernel records an error and all workgroups leave.

#include "pi05_blocks.h"
#include "pi05_kernels.h"

namespace pi05 {

// Phase timestamps for profiling builds (-DPI05_PHASE_TIMESTAMPS): thread 0 of every workgroup
// records s_memrealtime (100 MHz) at fixed points of every phase of Euler step 1, layers 0..3,
// into pi05_phase_ts[workgroup][layer*6 + phase][event].  Compiled out otherwise.
#ifdef PI05_PHASE_TIMESTAMPS
__device__ unsigned long long pi05_phase_ts[256 * 4 * 6 * 10];
#define PHASE_TS(s, l, ph, ev)                                                                  \
  do {                                                                                          \
    if ((s) == 1 && (l) < 4 && threadIdx.x == 0 && blockIdx.x < 256)                           \
      pi05_phase_ts[((size_t)blockIdx.x * 24 + (l) * 6 + (ph)) * 10 + (ev)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define PHASE_TS(s, l, ph, ev) \
  do {                         \
  } while (0)
#endif

constexpr int kThreads = 256;  // 4 waves: one per SIMD, up to 512 registers per lane
constexpr int kWaves = 4;
constexpr int kSpinLimit = 1 << 20;  // polls (each >= ~1 us): a legitimate wait spans a few phases
constexpr int kRowsPerSample = 64;   // padded rows per sample (50 action tokens)

// ---- coherent (agent-scope, write-through) accesses -------------------------------------------
__device__ __forceinline__ void st_u32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f32(float* p, float v) { st_u32(p, __float_as_uint(v)); }
__device__ __forceinline__ void st_u64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// One 16-byte write-through vector store (the agent-scope form of a 16-byte store: whole
// 16-byte chunks, so lines are assembled from full chunks, never from 2- or 4-byte pieces).
// Completion is tracked by vmcnt like any vector store; publish() waits for it.  A vector store
// of more than 8 bytes reads its data VGPRs after issue, so the next instruction must not be a
// VALU write to them: the compiler cannot see into the asm, hence the wait states after it.
__device__ __forceinline__ void st_wt16(void* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
// 8 bf16 (16 contiguous bytes, 16-byte aligned)
__device__ __forceinline__ void st_bf16x8(u16* p, const u16 (&v)[8]) {
  st_wt16(p, u32x4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                   (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)});
}
__device__ __forceinline__ void st_f32x4(float* p, float4 v) {
  st_wt16(p, u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)});
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

// Thread index as an opaque value: every phase derives its lane addresses from it afresh, so the
// compiler does not hoist them out of the step/layer loops and hold them live across all phases.
__device__ __forceinline__ int phase_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// ---- phase bookkeeping ------------------------------------------------------------------------
enum { kPhIo = 0, kPhQkv = 1, kPhAttn = 2, kPhO = 3, kPhGu = 4, kPhDown = 5, kNumPh = 6 };
constexpr int kQkvItems = 80;
constexpr int kTiles = kWidth / 16;  // 64 output tiles of o_proj / down_proj
constexpr int kGuItems = kMlp / 16;  // 256
constexpr int kKSplit = 4;           // K quarters of o_proj / down_proj
constexpr int kPairs = kHorizon / 2; // 25 two-token attention row blocks per sample
// direct-to-LDS copies per copying wave (waves 1..3) of the weight regions
constexpr int kCopiesA = 72 / 3;     // region A: 64 weight + 8 modulation fragments
constexpr int kCopiesBMin = 32 / 3;  // region B: 32 fragments, 10 or 11 per wave

// Phase completion: one counter per (step, layer, phase), replicated kCtrReplicas times, each
// replica on its own 128-byte line.  Every item of a phase adds 1 to every replica after its
// stores are complete (one atomic per lane of wave 0); a launch advances each counter by
// exactly the phase's item count, so "phase done in launch e" is counter == e * items.  A
// workgroup polls replica blockIdx % kCtrReplicas, so no line is polled by more than
// grid / kCtrReplicas workgroups.
constexpr int kCtrStride = 32;
constexpr int kCtrReplicas = 8;
__device__ __forceinline__ unsigned* done_ctr(const MegaArgs& a, int s, int l, int ph) {
  return a.flags + ((size_t)(s * (a.depth + 1) + l) * kNumPh + ph) * kCtrReplicas * kCtrStride;
}

// Wait until the phase counter reaches this launch's target.  One lane polls; uniform result.
// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for), N a compile-time constant < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until the phase counter reaches this launch's target.  One lane polls; uniform result.
// keep >= 0: waves 1..3 also wait until at most `keep` of their vector memory operations are
// outstanding (their weight copies for this phase landed in LDS; only the `keep` copies issued
// after them, for a later phase, may still be in flight).
__device__ bool wait_done(const MegaArgs& a, const unsigned* ctr, int n_items, int* s_flag, int keep = -1) {
  if (keep >= 0 && threadIdx.x >= 64) {
    if (keep == 0) wait_vmcnt<0>();
    else if (keep == kCopiesBMin) wait_vmcnt<kCopiesBMin>();
    else wait_vmcnt<kCopiesA>();
  }
  if (threadIdx.x == 0) {
    const unsigned target = a.epoch * (unsigned)n_items;
    const unsigned* rep = ctr + (blockIdx.x % kCtrReplicas) * kCtrStride;
    int ok = 1;
    for (int spins = 0; ld_u32(rep) != target; ++spins) {
      if (spins > kSpinLimit || ((spins & 63) == 63 && ld_u32(a.err) != 0)) {
        st_u32(a.err, 1u);
        __hip_atomic_store(a.host_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    *s_flag = ok;
  }
  __syncthreads();
  const bool ok = *s_flag != 0;
  __syncthreads();
  return ok;
}

// All of this workgroup's stores for one item are complete -> count the item done.
__device__ __forceinline__ void publish(unsigned* ctr) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < kCtrReplicas) __hip_atomic_fetch_add(ctr + threadIdx.x * kCtrStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Sum the 4 waves' D fragments (red[wave][mt][t][lane], f32x4) in wave order and scatter them
// row-major into the LDS tile T[64][TS] (column t*16 + n), which may alias red.  Thread tid owns
// m-tile tid/64, lane tid%64 of every tile t.
template <int NT, int TS>
__device__ __forceinline__ void reduce_to_tile(const float* red, float* T) {
  const int mt = threadIdx.x >> 6, ln = threadIdx.x & 63;
  f32x4 v[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    v[t] = *reinterpret_cast<const f32x4*>(red + (((size_t)(0 * 4 + mt) * NT + t) * 64 + ln) * 4);
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v[t] += *reinterpret_cast<const f32x4*>(red + (((size_t)(w * 4 + mt) * NT + t) * 64 + ln) * 4);
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) T[(mt * 16 + (ln >> 4) * 4 + i) * TS + t * 16 + (ln & 15)] = v[t][i];
}

// ---- LDS map (floats).  Weight fragments reach LDS by direct global->LDS copies (no registers
// held while in flight), issued one phase ahead of their use:
//   A: qkv or gate_up weights of this workgroup's item (64 KiB) + its modulation row 1+scale|shift
//      (qkv(l) copied when down_proj(l-1) starts, gate_up(l) when o_proj(l) starts)
//   B: down_proj weights (32 KiB, copied when gate_up(l) starts); during attention it stages the
//      first KV block of wave 0 instead
//   C: o_proj weights (16 KiB, copied when this workgroup is done with qkv(l))
// then the working area of the current phase.  Copies are issued by waves 1..3 only, so wave 0,
// which polls completion counters, never has copies ahead of its polls in its in-order memory
// counter; a consumer's waves 1..3 wait for their copies with vmcnt(N), N = the copies they
// issued after them (in issue order), so they never wait for the next phase's copies.
constexpr int kLdsA = 0;
constexpr int kLdsAMod = kLdsA + 16384;  // after 64 KiB of fragments
constexpr int kLdsB = kLdsAMod + 2 * kWidth;
constexpr int kLdsC = kLdsB + 8192;
constexpr int kLdsWork = kLdsC + 4096;
constexpr int kWorkFloats = 128 + 4 * 16 * (kHeadDim / 2 + 4);  // attention merge, the largest
constexpr int kLdsFloats = kLdsWork + kWorkFloats;
static_assert(kLdsFloats * 4 <= 160 * 1024, "LDS budget of a gfx950 workgroup");

// Direct-to-LDS copies of nfrag 1 KiB fragments: fragment f lands at dst + f KiB and comes from
// src(f) (1 KiB contiguous).  Issued by waves 1..3 only, so that wave 0, which polls completion
// counters, never has copies ahead of its polls in its in-order memory counter.
template <class F>
__device__ __forceinline__ void lds_copy(float* dst, int nfrag, F src) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave == 0) return;
  u16* d = reinterpret_cast<u16*>(dst);
  for (int f = wave - 1; f < nfrag; f += kWaves - 1)
    __builtin_amdgcn_global_load_lds(const_cast<u16*>(src(f)) + lane * 8, d + (size_t)f * 512, 16, 0, 0);
}

// qkv (MODE = kModeQkv) or gate_up weights + modulation row of item blockIdx.x -> region A.
template <int MODE>
__device__ void prefetch_norm_gemm(const MegaArgs& a, int s, int l, float* smem) {
  constexpr int KSTEPS = kWidth / 32;
  const int p = blockIdx.x, NN = 2 * a.depth + 1;
  if (p >= (MODE == kModeQkv ? kQkvItems : kGuItems) || s >= a.steps) return;
  const u16* wl = a.wpack + (size_t)l * kLayerElems;
  const u16 *t0, *t1;
  if constexpr (MODE == kModeQkv) {
    const bool rotated = p < 72;
    const int head = p >> 3, dt = p & 7;
    const int tile0 = rotated ? head * 16 + dt : 144 + 2 * (p - 72);
    const int tile1 = rotated ? head * 16 + 8 + dt : tile0 + 1;
    t0 = wl + kOffQkv + (size_t)tile0 * KSTEPS * 512;
    t1 = wl + kOffQkv + (size_t)tile1 * KSTEPS * 512;
  } else {
    t0 = wl + kOffGate + (size_t)p * KSTEPS * 512;
    t1 = wl + kOffUp + (size_t)p * KSTEPS * 512;
  }
  const u16* mrow = reinterpret_cast<const u16*>(a.table_s1 + ((size_t)s * NN + 2 * l + (MODE == kModeQkv ? 0 : 1)) * kModW);
  lds_copy(smem + kLdsA, 2 * KSTEPS + 8, [&](int f) -> const u16* {
    return f < KSTEPS ? t0 + (size_t)f * 512 : f < 2 * KSTEPS ? t1 + (size_t)(f - KSTEPS) * 512 : mrow + (size_t)(f - 2 * KSTEPS) * 512;
  });
}

// o_proj (KSTEPS = 64, region C) or down_proj (KSTEPS = 128, region B) weights of item
// blockIdx.x = (tile, K quarter).
template <int KSTEPS>
__device__ void prefetch_residual(const MegaArgs& a, int l, float* smem) {
  constexpr bool kDown = KSTEPS == kMlp / 32;
  constexpr int KQ = KSTEPS / kKSplit;
  const int item = blockIdx.x;
  if (item >= kTiles * kKSplit) return;
  const int nt = item % kTiles, ksp = item / kTiles;
  const u16* tile = a.wpack + (size_t)l * kLayerElems + (kDown ? kOffDown : kOffO) + (size_t)nt * KSTEPS * 512 + (size_t)ksp * KQ * 512;
  lds_copy(smem + (kDown ? kLdsB : kLdsC), KQ, [&](int f) -> const u16* { return tile + (size_t)f * 512; });
}

template <int NT>
__device__ __forceinline__ void store_wave_partials(float* red, const f32x4 (&acc)[4][NT], int wave, int lane) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>(red + (((size_t)(wave * 4 + mt) * NT + t) * 64 + lane) * 4) = acc[mt][t];
}

// =============================================================================================
// step boundary: final norm + action_out_proj + Euler of step s-1, action_in_proj of step s.
// Items: action-token rows (compact c = b*50 + t).  x[s] = Euler(x[s-1], v_{s-1});
// h[s][0] = bf16(action_in_proj(x[s])).
// =============================================================================================
__device__ bool phase_io(const MegaArgs& a, int s, float* smem, int* s_flag) {
  const int L = a.depth, NN = 2 * L + 1, R = a.R, NC = a.batch * kHorizon;
  const int tid = phase_tid();
  const int j = tid >> 3, part = tid & 7;   // action_out_proj: 8 threads per output, 128 k each
  const int c0 = tid * 4;                   // action_in_proj: 4 hidden columns per thread
  const int kc = (tid >> 2) * 32 + (tid & 3) * 8;  // final norm: 8 columns per thread (tid < 128)
  float* s_n = smem + kLdsWork;  // [W]
  float* s_x = s_n + kWidth;      // [a]
  float* s_rstd = s_x + kActDim;
  bool waited = false;
  for (int c = blockIdx.x; c < NC; c += gridDim.x) {
    const int b = c / kHorizon, t = c % kHorizon, r = b * kRowsPerSample + t;
    const bool has_prev = s > 0, has_next = s < a.steps;
    // ---- loads that do not depend on the previous phase
    float4 wo[32];
    float4 sc[2] = {}, sh[2] = {};
    float bo = 0.f;
    if (has_prev) {
#pragma unroll
      for (int q = 0; q < 32; ++q) wo[q] = *reinterpret_cast<const float4*>(a.out_w + (size_t)j * kWidth + part * 128 + q * 4);
      if (tid < 128) {
        const float* fmod = a.table + ((size_t)(s - 1) * NN + (NN - 1)) * kModW;
        sc[0] = *reinterpret_cast<const float4*>(fmod + kc);
        sc[1] = *reinterpret_cast<const float4*>(fmod + kc + 4);
        sh[0] = *reinterpret_cast<const float4*>(fmod + kWidth + kc);
        sh[1] = *reinterpret_cast<const float4*>(fmod + kWidth + kc + 4);
      }
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
      if (!wait_done(a, done_ctr(a, s - 1, L - 1, kPhDown), kTiles, s_flag)) return false;
      waited = true;
    }
    if (has_prev) {
      const size_t sl = (size_t)(s - 1) * (L + 1) + L;
      float rs = 0.f;
      u16x8 hv = {0, 0, 0, 0, 0, 0, 0, 0};
      float xj = 0.f;
      if (tid < kRowSlots) rs = a.rowss[(sl * kRowSlots + tid) * R + r];  // tile-major slot
      if (tid < 128) hv = *reinterpret_cast<const u16x8*>(a.h + sl * R * kWidth + afrag_index(r, kc, kWidth / 32));
      if (part == 0) xj = (s == 1 ? a.x_io : a.x + (size_t)(s - 1) * NC * kActDim)[(size_t)c * kActDim + j];
      // final adaRMSNorm (model.norm, modeling_gemma.py:782-783)
      if (tid < kRowSlots) {
        float v = rs;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
        if (tid == 0) *s_rstd = 1.0f / sqrtf(fadd(v * (1.0f / kWidth), a.eps));
      }
      __syncthreads();
      if (tid < 128) {
        const float rstd = *s_rstd;
        const float scs[8] = {sc[0].x, sc[0].y, sc[0].z, sc[0].w, sc[1].x, sc[1].y, sc[1].z, sc[1].w};
        const float shs[8] = {sh[0].x, sh[0].y, sh[0].z, sh[0].w, sh[1].x, sh[1].y, sh[1].z, sh[1].w};
#pragma unroll
        for (int q = 0; q < 8; ++q) s_n[kc + q] = round_bf(fadd(fmul(fmul(bf2f(hv[q]), rstd), fadd(1.0f, scs[q])), shs[q]));
      }
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
        const float* e = a.euler + (size_t)(s - 1) * 4;  // t, 1 - t, x0 weight, x1 weight
        // flow_ode mean in the reference's op order (engine.py:664-675)
        const float x0_pred = fsub(xj, fmul(v, e[0]));
        const float x1_pred = fadd(xj, fmul(v, e[1]));
        const float xn = fadd(fmul(x0_pred, e[2]), fmul(x1_pred, e[3]));
        st_f32((s == a.steps ? a.x_io : a.x + (size_t)s * NC * kActDim) + (size_t)c * kActDim + j, xn);
        s_x[j] = xn;
        if (a.trace) st_f32(a.trace + ((size_t)(s - 1) * NC + c) * kActDim + j, v);
      }
    } else if (tid < kActDim) {
      s_x[tid] = a.x_io[(size_t)c * kActDim + tid];
    }
    __syncthreads();
    if (has_next) {
      // h = bf16(action_in_proj(x)) (pi0_pytorch.py:303-306; modeling_gemma.py:724-725)
      const size_t sl = (size_t)s * (L + 1);
      const float bis[4] = {bi.x, bi.y, bi.z, bi.w};
      float ss = 0.f;
      u16 h8[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          acc += wi[q][k].x * s_x[4 * k] + wi[q][k].y * s_x[4 * k + 1] + wi[q][k].z * s_x[4 * k + 2] + wi[q][k].w * s_x[4 * k + 3];
        h8[q] = f2bf(acc + bis[q]);
        const float hf = bf2f(h8[q]);
        ss += hf * hf;
      }
      // even thread stores columns c0..c0+7 (its 4 and its odd neighbour's 4) as one chunk
      const uint32_t lo = (uint32_t)h8[0] | ((uint32_t)h8[1] << 16), hi = (uint32_t)h8[2] | ((uint32_t)h8[3] << 16);
      const uint32_t nlo = __shfl_xor(lo, 1), nhi = __shfl_xor(hi, 1);
      if ((tid & 1) == 0) {
        h8[4] = (u16)nlo;
        h8[5] = (u16)(nlo >> 16);
        h8[6] = (u16)nhi;
        h8[7] = (u16)(nhi >> 16);
        st_bf16x8(a.h + sl * R * kWidth + afrag_index(r, c0, kWidth / 32), h8);
      }
      ss += __shfl_xor(ss, 1);
      ss += __shfl_xor(ss, 2);
      float* s_ss = s_rstd + 1;  // [64]
      if ((tid & 3) == 0) s_ss[c0 >> 4] = ss;
      __syncthreads();
      // the statistics slot of layer 0 is row-major: this row's 64 sums are one 256-byte run
      if (tid < kRowSlots / 4)
        st_f32x4(a.rowss + (sl * R + r) * kRowSlots + tid * 4, float4{s_ss[tid * 4], s_ss[tid * 4 + 1], s_ss[tid * 4 + 2], s_ss[tid * 4 + 3]});
    }
    publish(done_ctr(a, s, 0, kPhIo));
  }
  return true;
}

// =============================================================================================
// adaRMSNorm-prologue GEMM tile (K = 1024, 4 waves x 8 k-steps): qkv and gate_up.
// One 64-row group (one sample) at a time: row statistics first, then the A fragments, so the
// norm starts while fragments stream in.
// =============================================================================================
template <int MODE>
__device__ bool phase_norm_gemm(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  constexpr int NT = 2, KSW = 8, KSTEPS = kWidth / 32, TS = 33;
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int n_items = MODE == kModeQkv ? kQkvItems : kGuItems;
  const int p = blockIdx.x;
  if (p >= n_items) {
    if constexpr (MODE == kModeQkv) {
      prefetch_residual<kHeads * kHeadDim / 32>(a, l, smem);  // o_proj weights -> C
    } else {
      prefetch_residual<kMlp / 32>(a, l, smem);  // down_proj weights -> B
    }
    return true;
  }
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int ks0 = wave * KSW;
  const size_t slw = (size_t)s * L + l;  // (step, layer) slice of per-layer buffers
  int tile0;
  bool rotated = false;
  int head = 0, dt = 0;
  const u16* hin;
  const float* rin;
  if constexpr (MODE == kModeQkv) {
    rotated = p < 72;
    head = p >> 3;
    dt = p & 7;
    tile0 = rotated ? head * 16 + dt : 144 + 2 * (p - 72);
    const size_t sl = (size_t)s * (L + 1) + l;
    hin = a.h + sl * R * kWidth;
    rin = a.rowss + sl * R * kRowSlots;
  } else {
    tile0 = p;
    hin = a.hmid + slw * R * kWidth;
    rin = a.rowss_mid + slw * R * kRowSlots;
  }
  constexpr int PH = MODE == kModeQkv ? kPhQkv : kPhGu;
  PHASE_TS(s, l, PH, 0);
  // Region A holds this item's weights and modulation row, copied one phase earlier (qkv: when
  // down_proj(l-1) started; the launch's first qkv copies them now; gate_up: when o_proj(l)
  // started).  gate_up starts the down_proj copies (region B) before waiting.
  if constexpr (MODE == kModeQkv) {
    if (s == 0 && l == 0) prefetch_norm_gemm<kModeQkv>(a, 0, 0, smem);
    if (!wait_done(a, l == 0 ? done_ctr(a, s, 0, kPhIo) : done_ctr(a, s, l - 1, kPhDown),
                   l == 0 ? a.batch * kHorizon : kTiles, s_flag, 0))
      return false;
  } else {
    prefetch_residual<kMlp / 32>(a, l, smem);
    if (!wait_done(a, done_ctr(a, s, l, kPhO), kTiles, s_flag, kCopiesBMin)) return false;
  }
  PHASE_TS(s, l, PH, 2);

  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);  // [tile t][k-step] fragments
  const float* s_mod = smem + kLdsAMod;                          // 1 + scale | shift
  float* s_rstd = smem + kLdsWork;                               // [64]
  float* red = s_rstd + 64;                                      // [4 waves][4 m-tiles][NT][64 lanes][4]
  float* T = red;                                                // [64][TS], reuses red
  const int erow = tid >> 1, ehalf = tid & 1;  // epilogue: 64 rows x 2 halves of 8 columns
  for (int b = 0; b < a.batch; ++b) {
    const int m0 = b * kRowsPerSample;
    // row statistics first: 4 threads per row, 16 partial sums each (layer 0's slot, written
    // per row by the step boundary, is row-major; the others, written per 16-column tile by the
    // residual epilogues, are tile-major)
    float4 rs[4];
    const int srow = tid >> 2, q4 = tid & 3;
    if (MODE == kModeQkv && l == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) rs[q] = *reinterpret_cast<const float4*>(rin + (size_t)(m0 + srow) * kRowSlots + q4 * 16 + q * 4);
    } else {
      const float* rc = rin + (size_t)q4 * 16 * R + m0 + srow;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        rs[q] = float4{rc[(4 * q) * R], rc[(4 * q + 1) * R], rc[(4 * q + 2) * R], rc[(4 * q + 3) * R]};
    }
    // A fragments in the order they are consumed
    u16x8 hr[4][KSW];
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)  // rows t >= 50 are zero: not loaded
        hr[mt][s2] = r16 < kHorizon - mt * 16 ? *reinterpret_cast<const u16x8*>(hin + afrag_offset(b * 4 + mt, ks0 + s2, KSTEPS) + lane * 8)
                                              : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    // RoPE tables of this thread's epilogue chunk (static: issued with the fragments)
    u16x8 cs_lo = {}, sn_lo = {}, cs_hi = {}, sn_hi = {};
    if constexpr (MODE == kModeQkv) {
      if (rotated && tid < 128 && erow < kHorizon) {
        const size_t cr = (size_t)(b * kHorizon + erow) * kHeadDim + dt * 16 + ehalf * 8;
        cs_lo = *reinterpret_cast<const u16x8*>(a.cos_tab + cr);
        sn_lo = *reinterpret_cast<const u16x8*>(a.sin_tab + cr);
        cs_hi = *reinterpret_cast<const u16x8*>(a.cos_tab + cr + kHalfDim);
        sn_hi = *reinterpret_cast<const u16x8*>(a.sin_tab + cr + kHalfDim);
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
    if (b == 0) PHASE_TS(s, l, PH, 3);
    // adaRMSNorm (modeling_gemma.py:82-116): A = bf16((h * rstd) * (1 + scale) + shift), the
    // last multiply-add fused
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
      bf16x8 wf[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) wf[t] = *reinterpret_cast<const bf16x8*>(lw + ((size_t)t * KSTEPS + ks0 + s2) * 512 + lane * 8);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        u16x8 o;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) o[jj] = f2bf(__builtin_fmaf(fmul(bf2f(hr[mt][s2][jj]), rstd[mt]), scs[jj], shs[jj]));
        const bf16x8 af = as_bf16x8(o);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = mfma16x16x32(af, wf[t], acc[mt][t]);
      }
    }
    if (b == 0) PHASE_TS(s, l, PH, 4);
    __syncthreads();  // T of the previous sample and s_rstd readers are done with the area
    store_wave_partials<NT>(red, acc, wave, lane);
    __syncthreads();
    reduce_to_tile<NT, TS>(red, T);
    __syncthreads();
    if constexpr (MODE == kModeQkv) {
      if (rotated) {
        if (tid < 128 && erow < kHorizon) {
          // (x*cos) + (rotate_half(x)*sin), rotate_half(x) = cat(-x_hi, x_lo), from the bf16
          // GEMM values (rlinf_fused_denoise.py:264-278; modeling_gemma.py:185-216)
          u16 olo[8], ohi[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float x_lo = round_bf(T[erow * TS + ehalf * 8 + q]);
            const float x_hi = round_bf(T[erow * TS + 16 + ehalf * 8 + q]);
            olo[q] = f2bf(fsub(fmul(x_lo, bf2f(cs_lo[q])), fmul(x_hi, bf2f(sn_lo[q]))));
            ohi[q] = f2bf(fadd(fmul(x_hi, bf2f(cs_hi[q])), fmul(x_lo, bf2f(sn_hi[q]))));
          }
          const int d = dt * 16 + ehalf * 8;
          if (head < kHeads) {
            u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
            const int qrow = (m0 + erow) * kQRowsPerTok + head;
            st_bf16x8(qs + afrag_index(qrow, d, kHeadDim / 32), olo);
            st_bf16x8(qs + afrag_index(qrow, d + kHalfDim, kHeadDim / 32), ohi);
          } else {
            u16* kc = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
            st_bf16x8(kc + kfrag_index(erow, d), olo);
            st_bf16x8(kc + kfrag_index(erow, d + kHalfDim), ohi);
          }
        }
      } else {
        // v: thread -> (dim dcol of the tile pair, key group (kb, g) of the permuted V fragment)
        const int dcol = tid & 31, kg = tid >> 5, kb = kg >> 2, gg = kg & 3;
        u16 v8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int key = vkey(kb, gg, q);
          v8[q] = key < kHorizon ? f2bf(T[key * TS + dcol]) : (u16)0;
        }
        const int dv = (tile0 - 144) * 16 + dcol;
        u16* vc = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
        st_bf16x8(vc + ((size_t)kb * 16 + (dv >> 4)) * 512 + (size_t)(gg * 16 + (dv & 15)) * 8, v8);
      }
    } else {
      if (tid < 128 && erow < kHorizon) {
        // GeGLU as the fused reference kernel defines it: bf16(gelu_tanh(bf16(g)) * u)
        // (rlinf_fused_denoise.py:166-173)
        u16 o8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          o8[q] = f2bf(fmul(gelu_tanh(round_bf(T[erow * TS + ehalf * 8 + q])), T[erow * TS + 16 + ehalf * 8 + q]));
        st_bf16x8(a.act + slw * (size_t)R * kMlp + afrag_index(m0 + erow, tile0 * 16 + ehalf * 8, kMlp / 32), o8);
      }
    }
    __syncthreads();
  }
  PHASE_TS(s, l, PH, 5);
  publish(done_ctr(a, s, l, MODE == kModeQkv ? kPhQkv : kPhGu));
  PHASE_TS(s, l, PH, 6);
  if constexpr (MODE == kModeQkv) prefetch_residual<kHeads * kHeadDim / 32>(a, l, smem);  // o_proj weights -> C
  return true;
}

// =============================================================================================
// attention: item = (row block of 2 tokens x 8 heads of one sample, key split); 4 waves, one
// 32-key block in flight per wave.  Keys [0, s_pre) come from the static prefix cache, keys
// [s_pre, s_pre + 64) from this step's action-key block (50 valid).
// =============================================================================================
__device__ bool phase_attn(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  const int L = a.depth, R = a.R, nbp = a.nbp;
  const int n_items = nbp * a.nsplit;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4;
  const size_t slw = (size_t)s * L + l;
  const int nkb_pre = a.s_pre >> 5;
  const int nkb = nkb_pre + 2;
  const int prow = nbp * 16;  // partial rows
  // this layer's split partials (written once per launch, so read with plain loads)
  float* apart = a.apart + slw * (size_t)a.nsplit * prow * kHeadDim;
  float* apart_m = a.apart_m + slw * (size_t)a.nsplit * prow;
  float* apart_l = a.apart_l + slw * (size_t)a.nsplit * prow;
  bool waited = false;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int bp = item % nbp, split = item / nbp;
    const int b = bp / kPairs, pair = bp % kPairs;
    const int rbq = b * (kRowsPerSample / 2) + pair;  // query-row m-tile (16 rows = 2 tokens x 8 heads)
    const u16* kpre = a.kpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* vpre = a.vpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* ksf = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
    const u16* vsf = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
    const uint8_t* valid = a.valid + (size_t)b * (a.s_pre + 64);
    const int kb_lo = split * nkb / a.nsplit, kb_hi = (split + 1) * nkb / a.nsplit;
    const int span = kb_hi - kb_lo;
    const int w_lo = kb_lo + wave * span / 4, w_hi = kb_lo + (wave + 1) * span / 4;
    const int n = w_hi - w_lo;
    auto load = [&](KvBlock& blk, int kb) {
      if (kb >= nkb_pre) load_kv_block(blk, ksf, vsf, valid + kb * 32, kb - nkb_pre, lane);
      else load_kv_block(blk, kpre, vpre, valid + kb * 32, kb, lane);
    };
    // One block in flight per wave (two would not fit the 256 VGPRs that MFMA operands live
    // in); the split count is chosen so that a wave normally owns a single block.
    KvBlock blk;
    if (!waited) PHASE_TS(s, l, kPhAttn, 0);
    // Prefix blocks do not depend on this step: fetch the first one before waiting.  Wave 0
    // polls, so its first block is staged in LDS region B by waves 1..3 instead of loaded into
    // its registers (which would put the load ahead of its polls).
    const int w0_lo = kb_lo, w0_n = kb_lo + span / 4 - kb_lo;
    const bool staged = !waited && w0_n > 0 && w0_lo < nkb_pre;
    if (staged) {
      const u16* kc = kpre;
      const u16* vc = vpre;
      lds_copy(smem + kLdsB, 32, [&](int f) -> const u16* {
        return f < 16 ? kc + ((size_t)(2 * w0_lo + (f >> 3)) * 8 + (f & 7)) * 512 : vc + ((size_t)w0_lo * 16 + (f - 16)) * 512;
      });
    }
    if (n > 0 && w_lo < nkb_pre && !(staged && wave == 0)) load(blk, w_lo);
    if (!waited) {
      PHASE_TS(s, l, kPhAttn, 1);
      if (!wait_done(a, done_ctr(a, s, l, kPhQkv), kQkvItems, s_flag, 0)) return false;
      waited = true;
      PHASE_TS(s, l, kPhAttn, 2);
    }
    if (staged && wave == 0) {
      // the staged block, in load_kv_block's register order
      const u16* st = reinterpret_cast<const u16*>(smem + kLdsB);
#pragma unroll
      for (int f = 0; f < 16; ++f) blk.k[f] = *reinterpret_cast<const bf16x8*>(st + (size_t)f * 512 + lane * 8);
#pragma unroll
      for (int f = 0; f < 16; ++f) blk.v[f] = *reinterpret_cast<const bf16x8*>(st + (size_t)(16 + f) * 512 + lane * 8);
      blk.valid0 = *reinterpret_cast<const uint32_t*>(valid + w0_lo * 32 + g * 4);
      blk.valid1 = *reinterpret_cast<const uint32_t*>(valid + w0_lo * 32 + 16 + g * 4);
    }
    if (n > 0 && w_lo >= nkb_pre) load(blk, w_lo);
    const u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
    bf16x8 qf[8];
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qf[ds] = load_frag(qs + afrag_offset(rbq, ds, kHeadDim / 32) + lane * 8);
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
    if (item == (int)blockIdx.x) PHASE_TS(s, l, kPhAttn, 4);

    // ---- merge the 4 waves: each wave puts (m, l) per row and its O rows in LDS, one half of the
    // head dim at a time, and wave w combines d-tiles {2w, 2w+1, 8+2w, 9+2w} of all four with
    // 16-byte LDS accesses.  Lane (r16, g) ends up with O[row r16][dtile(j)*16 + g*4 + i].
    float* s_m = smem + kLdsWork;  // [4][16]
    float* s_l = s_m + 64;         // [4][16]
    float* s_o = s_m + 128;        // [4 waves][16 rows][D/2 + 4]
    constexpr int OSTR = kHeadDim / 2 + 4;
    const int r16 = lane & 15;
    if (g == 0) {
      s_m[wave * 16 + r16] = m_run;
      s_l[wave * 16 + r16] = l_run;
    }
    f32x4 om[4];
    auto dtile = [&](int j) { return (j >> 1) * 8 + 2 * wave + (j & 1); };
    float Mx = -INFINITY, Lx = 0.f, ww[4];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int q = 0; q < 8; ++q) *reinterpret_cast<f32x4*>(s_o + (wave * 16 + r16) * OSTR + q * 16 + g * 4) = oacc[hh * 8 + q];
      __syncthreads();
      if (hh == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) Mx = fmaxf(Mx, s_m[v * 16 + r16]);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          ww[v] = (s_m[v * 16 + r16] == -INFINITY) ? 0.f : __expf(s_m[v * 16 + r16] - Mx);
          Lx += s_l[v * 16 + r16] * ww[v];
        }
      }
#pragma unroll
      for (int j = 2 * hh; j < 2 * hh + 2; ++j) {
        const int q = 2 * wave + (j & 1);
        om[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < 4; ++v) om[j] += *reinterpret_cast<const f32x4*>(s_o + (v * 16 + r16) * OSTR + q * 16 + g * 4) * ww[v];
      }
      __syncthreads();
    }
    if (item == (int)blockIdx.x) PHASE_TS(s, l, kPhAttn, 5);
    const int orow = bp * 16 + r16;  // partial row
    bool finish = true;
    if (a.nsplit > 1) {
      // partials as 1 KiB fragments [split][row block][wave][j][lane][4]: the finisher's wave w
      // reads exactly what wave w wrote, 1 KiB per wave load
      float* part = apart + (((size_t)split * nbp + bp) * 16 + wave * 4) * 256 + lane * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) st_f32x4(part + j * 256, float4{om[j][0], om[j][1], om[j][2], om[j][3]});
      if (wave == 0 && g == 0) {
        st_f32(apart_m + (size_t)split * prow + orow, Mx);
        st_f32(apart_l + (size_t)split * prow + orow, Lx);
      }
      finish = last_arrival(a, a.counters + slw * nbp + bp, (unsigned)a.nsplit, s_flag);
      if (finish) {
        PHASE_TS(s, l, kPhAttn, 7);
        // combine the splits in fixed order, online over batches of 8 (one load round each):
        // O = sum_c O_c e^{m_c - m} / sum_c l_c e^{m_c - m}
        Mx = -INFINITY;
        Lx = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) om[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int c0 = 0; c0 < a.nsplit; c0 += 8) {
          float mc[8], lc[8];
          f32x4 oc[8][4];
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {
            const int c = c0 + cc;
            mc[cc] = -INFINITY;
            lc[cc] = 0.f;
            if (c < a.nsplit) {
              mc[cc] = apart_m[(size_t)c * prow + orow];
              lc[cc] = apart_l[(size_t)c * prow + orow];
              const float* pp = apart + (((size_t)c * nbp + bp) * 16 + wave * 4) * 256 + lane * 4;
#pragma unroll
              for (int j = 0; j < 4; ++j) oc[cc][j] = *reinterpret_cast<const f32x4*>(pp + j * 256);
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j) oc[cc][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
          float Mb = Mx;
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) Mb = fmaxf(Mb, mc[cc]);
          const float rescale = (Mx == -INFINITY) ? 0.f : __expf(Mx - Mb);
          Lx *= rescale;
#pragma unroll
          for (int j = 0; j < 4; ++j) om[j] *= rescale;
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {
            const float wc = (mc[cc] == -INFINITY) ? 0.f : __expf(mc[cc] - Mb);
            Lx += lc[cc] * wc;
#pragma unroll
            for (int j = 0; j < 4; ++j) om[j] += oc[cc][j] * wc;
          }
          Mx = Mb;
        }
      }
    }
    if (finish) {
      PHASE_TS(s, l, kPhAttn, 8);
      // attention output row (token, head) -> o_proj A operand [R, H*D]; lanes g even store the
      // 8 consecutive dims they share with lane g + 1
      const float inv = 1.0f / Lx;
      const int r = b * kRowsPerSample + 2 * pair + (r16 >> 3), head = r16 & 7;
      u16* os = a.o + slw * (size_t)R * (kHeads * kHeadDim);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = (uint32_t)f2bf(om[j][0] * inv) | ((uint32_t)f2bf(om[j][1] * inv) << 16);
        const uint32_t hi = (uint32_t)f2bf(om[j][2] * inv) | ((uint32_t)f2bf(om[j][3] * inv) << 16);
        const uint32_t nlo = __shfl_xor(lo, 16), nhi = __shfl_xor(hi, 16);
        if ((g & 1) == 0) {
          const int col = head * kHeadDim + dtile(j) * 16 + g * 4;
          st_wt16(os + afrag_index(r, col, kHeads * kHeadDim / 32), u32x4{lo, hi, nlo, nhi});
        }
      }
      publish(done_ctr(a, s, l, kPhAttn));
      PHASE_TS(s, l, kPhAttn, 9);
    }
  }
  return true;
}

// =============================================================================================
// o_proj (K = 2048) and down_proj (K = 4096): item = (16-column tile, K quarter), 4 waves split
// the quarter.  The last quarter to arrive adds the four partials in order and applies the gated
// residual h = bf16(h + bf16(bf16(y) * gate)) (modeling_gemma.py:231-249, 503, 511), storing the
// new residual rows and their per-tile sums of squares for the next adaRMSNorm.
// =============================================================================================
template <int KSW>
__device__ __forceinline__ void residual_mma(f32x4 (&acc)[4], const bf16x8 (&w)[KSW], const u16* act, int ksteps, int mt0,
                                             int kstep0, int lane) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 af[4][KSW];
  const int r16 = lane & 15;
#pragma unroll
  for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)  // rows t >= 50 are zero: not loaded
      af[mt][s2] = r16 < kHorizon - mt * 16 ? load_frag(act + afrag_offset(mt0 + mt, kstep0 + s2, ksteps) + lane * 8) : zero_frag();
#pragma unroll
  for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = mfma16x16x32(af[mt][s2], w[s2], acc[mt]);
}

template <int KSTEPS>
__device__ bool phase_residual(const MegaArgs& a, int s, int l, float* smem, int* s_flag) {
  constexpr bool kDown = KSTEPS == kMlp / 32;
  constexpr int KQ = KSTEPS / kKSplit, KSW = KQ / kWaves, TS = 17;
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int n_items = kTiles * kKSplit;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int erow = tid >> 1, ehalf = tid & 1;
  const size_t slw = (size_t)s * L + l;
  bool waited = false;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int nt = item % kTiles, ksp = item / kTiles;
    const int kstep0 = ksp * KQ + wave * KSW;
    constexpr int PH = kDown ? kPhDown : kPhO;
    if (!waited) PHASE_TS(s, l, PH, 0);
    if (!waited) {
      PHASE_TS(s, l, PH, 1);
      // this item's weights were copied one phase earlier (o_proj: region C, after qkv; down_proj:
      // region B, when gate_up started).  Start the next weight copies now (o_proj: gate_up ->
      // A; down_proj: the next qkv -> A) and wait for this phase's.
      bool ok;
      if constexpr (kDown) {
        const bool next_qkv = (l + 1 < L || s + 1 < a.steps) && blockIdx.x < kQkvItems;
        if (l + 1 < L) prefetch_norm_gemm<kModeQkv>(a, s, l + 1, smem);
        else prefetch_norm_gemm<kModeQkv>(a, s + 1, 0, smem);
        ok = wait_done(a, done_ctr(a, s, l, kPhGu), kGuItems, s_flag, next_qkv ? kCopiesA : 0);
      } else {
        prefetch_norm_gemm<kModeGateUp>(a, s, l, smem);
        ok = wait_done(a, done_ctr(a, s, l, kPhAttn), a.nbp, s_flag, kCopiesA);
      }
      if (!ok) return false;
      waited = true;
      PHASE_TS(s, l, PH, 2);
    }
    const u16* lw = reinterpret_cast<const u16*>(smem + (kDown ? kLdsB : kLdsC));  // this item's K-quarter fragments
    bf16x8 w[KSW];
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) w[s2] = *reinterpret_cast<const bf16x8*>(lw + (size_t)(wave * KSW + s2) * 512 + lane * 8);
    // gate of this thread's 8 epilogue columns (used by the finisher)
    const float* gmod = a.table + ((size_t)s * NN + 2 * l + (kDown ? 1 : 0)) * kModW + 2 * kWidth + nt * 16 + ehalf * 8;
    float4 g4[2] = {};
    if (tid < 128) {
      g4[0] = *reinterpret_cast<const float4*>(gmod);
      g4[1] = *reinterpret_cast<const float4*>(gmod + 4);
    }
    const u16* act = kDown ? a.act + slw * (size_t)R * kMlp : a.o + slw * (size_t)R * (kHeads * kHeadDim);
    // this phase's K-quarter partials [quarter][tile][row][16] (written once per launch)
    float* dpart = a.dpart + (slw * 2 + (kDown ? 1 : 0)) * (size_t)kKSplit * kTiles * R * 16;
    float* red = smem + kLdsWork;
    float* T = red + kWaves * 4 * 256;
    for (int b = 0; b < a.batch; ++b) {
      f32x4 acc[4];
      residual_mma<KSW>(acc, w, act, KSTEPS, b * 4, kstep0, lane);
      if (b == 0) PHASE_TS(s, l, PH, 4);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4*>(red + (((size_t)wave * 4 + mt) * 64 + lane) * 4) = acc[mt];
      __syncthreads();
      reduce_to_tile<1, TS>(red, T);
      __syncthreads();
      if (tid < 128) {
        // partial [quarter][tile][row][16]
        float* part = dpart + (((size_t)ksp * kTiles + nt) * R + b * kRowsPerSample + erow) * 16 + ehalf * 8;
        const float* tr = T + erow * TS + ehalf * 8;
        st_f32x4(part, float4{tr[0], tr[1], tr[2], tr[3]});
        st_f32x4(part + 4, float4{tr[4], tr[5], tr[6], tr[7]});
      }
      __syncthreads();
    }
    const size_t ctr = (kDown ? a.ctr_down_off : a.ctr_o_off) + slw * kTiles + nt;
    PHASE_TS(s, l, PH, 5);
    const bool finisher = last_arrival(a, a.counters + ctr, (unsigned)kKSplit, s_flag);
    if (finisher) {
      PHASE_TS(s, l, PH, 7);
      const u16* hres;
      u16* hout;
      float* rout;
      if (kDown) {
        hres = a.hmid + slw * (size_t)R * kWidth;
        hout = a.h + ((size_t)s * (L + 1) + l + 1) * R * kWidth;
        rout = a.rowss + ((size_t)s * (L + 1) + l + 1) * R * kRowSlots;
      } else {
        hres = a.h + ((size_t)s * (L + 1) + l) * R * kWidth;
        hout = a.hmid + slw * (size_t)R * kWidth;
        rout = a.rowss_mid + slw * (size_t)R * kRowSlots;
      }
      float* s_ss = T + 64 * TS;  // [64] row sums of squares of this tile
      const float gate[8] = {round_bf(g4[0].x), round_bf(g4[0].y), round_bf(g4[0].z), round_bf(g4[0].w),
                             round_bf(g4[1].x), round_bf(g4[1].y), round_bf(g4[1].z), round_bf(g4[1].w)};
      const int col = nt * 16 + ehalf * 8;
      for (int b = 0; b < a.batch; ++b) {
        if (tid < 128 && erow < kHorizon) {
          const int r = b * kRowsPerSample + erow;
          float4 pv[kKSplit][2];
#pragma unroll
          for (int q = 0; q < kKSplit; ++q) {
            const float* pp = dpart + (((size_t)q * kTiles + nt) * R + r) * 16 + ehalf * 8;
            pv[q][0] = *reinterpret_cast<const float4*>(pp);
            pv[q][1] = *reinterpret_cast<const float4*>(pp + 4);
          }
          const u16x8 hold = *reinterpret_cast<const u16x8*>(hres + afrag_index(r, col, kWidth / 32));
          float y[8];
#pragma unroll
          for (int q = 0; q < kKSplit; ++q) {
            const float v[8] = {pv[q][0].x, pv[q][0].y, pv[q][0].z, pv[q][0].w, pv[q][1].x, pv[q][1].y, pv[q][1].z, pv[q][1].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = q == 0 ? v[i] : y[i] + v[i];
          }
          u16 hn[8];
          float ss = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float prod = round_bf(fmul(round_bf(y[i]), gate[i]));
            hn[i] = f2bf(fadd(bf2f(hold[i]), prod));
            const float hf = bf2f(hn[i]);
            ss += hf * hf;
          }
          st_bf16x8(hout + afrag_index(r, col, kWidth / 32), hn);
          ss += __shfl_xor(ss, 1);  // the other 8 columns of the tile (same row, adjacent lane)
          if (ehalf == 0) s_ss[erow] = ss;
        } else if (tid < 128 && ehalf == 0) {
          s_ss[erow] = 0.f;  // padded rows
        }
        __syncthreads();
        // tile-major statistics: this tile's sums of the sample's 64 rows are one 256-byte run
        if (tid < kRowsPerSample / 4) {
          const float* q = s_ss + tid * 4;
          st_f32x4(rout + (size_t)nt * R + b * kRowsPerSample + tid * 4, float4{q[0], q[1], q[2], q[3]});
        }
        __syncthreads();
      }
      PHASE_TS(s, l, PH, 8);
      publish(done_ctr(a, s, l, kDown ? kPhDown : kPhO));
      PHASE_TS(s, l, PH, 9);
    }
  }
  return true;
}

// =============================================================================================
// the kernel
// =============================================================================================
static_assert(64 + kWaves * 4 * 2 * 256 <= kWorkFloats, "norm GEMM working area");
static_assert(kWaves * 4 * 256 + 64 * 17 + 64 <= kWorkFloats, "residual working area");

__global__ __launch_bounds__(kThreads, 1) void denoise_loop_kernel(MegaArgs a) {
  __shared__ __align__(16) float smem[kLdsFloats];
  __shared__ int s_flag;
  for (int s = 0; s <= a.steps; ++s) {
    if (!phase_io(a, s, smem, &s_flag)) return;
    if (s == a.steps) break;
    for (int l = 0; l < a.depth; ++l) {
      if (!phase_norm_gemm<kModeQkv>(a, s, l, smem, &s_flag)) return;
      if (!phase_attn(a, s, l, smem, &s_flag)) return;
      if (!phase_residual<kHeads * kHeadDim / 32>(a, s, l, smem, &s_flag)) return;
      if (!phase_norm_gemm<kModeGateUp>(a, s, l, smem, &s_flag)) return;
      if (!phase_residual<kMlp / 32>(a, s, l, smem, &s_flag)) return;
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

#ifdef PI05_PHASE_TIMESTAMPS
// Copy the phase timestamps of the last launch to the host (profiling builds only).
extern "C" int pi05_debug_phase_timestamps(unsigned long long* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(pi05::pi05_phase_ts), sizeof(pi05::pi05_phase_ts), 0, hipMemcpyDeviceToHost);
}
#endif
