// The whole num_steps Euler loop of the pi0.5 action expert as ONE cooperative kernel.
//
// Workgroups: one per CU, four waves (one per SIMD, so each keeps the 512-register budget the
// MFMA operand blocks need).  Waves 0..2 compute and store; wave 0 also polls completion flags and
// publishes.  Wave 3 copies weight fragments from HBM into LDS (direct global->LDS loads) phases
// ahead of their use, in bursts of at most 32 one-KiB fragments so that it never has more than 63
// memory operations in flight (more would stall it at issue, and with it every workgroup barrier
// it has to reach).  A wave's vector memory operations complete in issue order, so keeping the
// bulk copies in a wave of their own means that neither the loads on the critical path (freshly
// produced activations) nor the store completions that gate a publish ever queue behind them.
//
// Every workgroup walks the same phase sequence
//   step boundary, then per decoder layer:
//   qkv -> attention (key splits, then merges) -> o_proj -> gate_up -> down_proj
// and takes the items of each phase that map to it (item i -> workgroup i mod grid).  Phases
// hand data over through buffers that are written once per launch (one slice per Euler step and
// layer) with write-through stores; a producer publishes each item with a flag word (the
// launch's epoch), a consumer polls the flags of exactly the items it depends on (four per lane
// in one 16-byte coherent load) and then reads the data with ordinary loads.  No slice is read
// before it is written within a launch, so no cache holds a stale copy and no cache maintenance
// is ever issued.
//
// adaRMSNorm is folded into the GEMM that consumes it: whoever produces a tile of the residual
// stream h also writes g = bf16(h * (1 + scale)) and the tile's per-row sums of squares; the
// consumer multiplies g by its weights on MFMA and applies rstd (per row) and shift . W^T (per
// column, precomputed per step and layer) in its epilogue.
//
// Every wait is bounded: on timeout the kernel records an error and all workgroups leave.

#include <type_traits>

#include "pi05_blocks.h"
#include "pi05_kernels.h"

// This file is compiled three times: as itself (instance 0: the one-sample kernel and the
// host-side entry points), through pi05_persistent_batched.hip (instance 1: the kernel for batches
// of 2) and through pi05_persistent_grouped.hip (instance 2: batches of kRowSplitMinBatch and more,
// with the row-split gate_up and, from kAttnGroupMinBatch on, the grouped attention), so that no
// kernel's code generation depends on another's paths.
#ifndef PI05_PERSISTENT_INSTANCE
#define PI05_PERSISTENT_INSTANCE 0
#endif
#define PI05_INSTANCE_GROUPED (PI05_PERSISTENT_INSTANCE == 2)

namespace pi05 {

// Phase timestamps for profiling builds (-DPI05_PHASE_TIMESTAMPS): thread 0 of every workgroup
// records s_memrealtime (100 MHz) at fixed points of every phase of Euler step 1, layers 0..3,
// into pi05_phase_ts[workgroup][layer*7 + phase][event].  The stamps go to LDS while the kernel
// runs (an LDS write completes in a few cycles, where a global store would hold back the next
// barrier's implicit vmcnt(0) by its write acknowledgement) and are copied out at kernel exit.
// Compiled out otherwise.
#ifdef PI05_PHASE_TIMESTAMPS
__device__ unsigned long long pi05_phase_ts[256 * 4 * 7 * 16];
__shared__ unsigned long long pi05_phase_ts_lds[4 * 7 * 16];
#define PHASE_TS(s, l, ph, ev)                                                                  \
  do {                                                                                          \
    if ((s) == 1 && (l) < 4 && threadIdx.x == 0 && blockIdx.x < 256)                           \
      pi05_phase_ts_lds[((l) * 7 + (ph)) * 16 + (ev)] = __builtin_amdgcn_s_memrealtime();      \
  } while (0)
// the same, recorded by the first lane of wave w
#define PHASE_TS_W(w, s, l, ph, ev)                                                             \
  do {                                                                                          \
    if ((s) == 1 && (l) < 4 && threadIdx.x == 64 * (w) && blockIdx.x < 256)                    \
      pi05_phase_ts_lds[((l) * 7 + (ph)) * 16 + (ev)] = __builtin_amdgcn_s_memrealtime();      \
  } while (0)
#define PHASE_TS_INIT()                                                                         \
  do {                                                                                          \
    for (int i_ = threadIdx.x; i_ < 4 * 7 * 16; i_ += blockDim.x) pi05_phase_ts_lds[i_] = 0;    \
    __syncthreads();                                                                            \
  } while (0)
#define PHASE_TS_FLUSH()                                                                        \
  do {                                                                                          \
    __syncthreads();                                                                            \
    if (blockIdx.x < 256)                                                                       \
      for (int i_ = threadIdx.x; i_ < 4 * 7 * 16; i_ += blockDim.x)                             \
        pi05_phase_ts[(size_t)blockIdx.x * 448 + i_] = pi05_phase_ts_lds[i_];                  \
  } while (0)
#else
#define PHASE_TS_INIT() \
  do {                  \
  } while (0)
#define PHASE_TS_FLUSH() \
  do {                   \
  } while (0)
#define PHASE_TS(s, l, ph, ev) \
  do {                         \
  } while (0)
#define PHASE_TS_W(w, s, l, ph, ev) \
  do {                              \
  } while (0)
#endif

// ---- scalar register pressure ------------------------------------------------------------------
// The kernel's phases run inside the Euler-step and layer loops, and the compiler hoists out of
// those loops everything a phase derives from loop-invariant values -- the kernel arguments, the
// workgroup index -- where it then stays live across every phase and is spilled (the phases
// together need far more scalar registers than the 102 a wave has).  So every phase reads them
// afresh: the workgroup index and grid size through an opaque copy, the kernel arguments through
// a pointer into the kernel-argument segment that the compiler cannot see through (kargs(); the
// fields are scalar loads, cached).
__device__ __forceinline__ int wg_id() {
  int w = (int)blockIdx.x;
  asm volatile("" : "+v"(w));
  return __builtin_amdgcn_readfirstlane(w);
}
__device__ __forceinline__ int wg_count() {
  int n = (int)gridDim.x;
  asm volatile("" : "+v"(n));
  return __builtin_amdgcn_readfirstlane(n);
}
typedef const __attribute__((address_space(4))) MegaArgs KArgs;
__device__ __forceinline__ KArgs& kargs() {
  KArgs* p = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *p;
}

constexpr int kCompWaves = 3;
constexpr int kCompThreads = kCompWaves * 64;
constexpr int kThreads = kCompThreads + 64;  // + the copy wave
constexpr int kRowsPerSample = 64;           // padded rows per sample (50 action tokens)

// ---- coherent (agent-scope, write-through) accesses -------------------------------------------
__device__ __forceinline__ void st_u32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Buffer resources: a load at a byte offset past the resource's size returns zeros without
// touching memory (the hardware range check).  Masking lanes (padded rows) and surplus k-steps
// this way keeps the load sequences free of branches, so the compiler can count the loads in
// flight and let each MFMA wait only for its own operands.
typedef __amdgpu_buffer_rsrc_t brsrc;
constexpr int kOob = 0x7fffff00;  // an offset past every resource
constexpr int kAuxNt = 2;         // buffer-instruction cache-policy bits: nt (non-temporal)
__device__ __forceinline__ brsrc make_rsrc(const void* base, size_t bytes) {
  // the size and flag words pass through empty asm statements so that the compiler builds them
  // where the resource is used: hoisted out of the step / layer loops as loop-invariant
  // constants, dozens of them would stay live across every phase and be spilled
  int nrec = (int)bytes, flags = 0x00020000;
  asm volatile("" : "+s"(nrec), "+s"(flags));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nrec, flags);
}
// A pointer every lane holds the same value of, moved to scalar registers.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}
// One 16-byte write-through (sc1) store at `off` bytes past `base` (the same in every lane):
// whole 16-byte chunks, so lines are assembled from full chunks.  A buffer store the compiler
// sees, so it schedules the loads feeding it freely; completion is tracked by vmcnt like any
// vector store, and publish() waits for it.
__device__ __forceinline__ void st_wt16(const void* base, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(uniform_ptr(base), 0x7fffffff), off, 0, 16);
}
// The same for 8 bytes (offset 8-byte aligned).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_wt8(const void* base, uint32_t off, uint32_t lo, uint32_t hi) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, make_rsrc(uniform_ptr(base), 0x7fffffff), off, 0, 16);
}
// The same as a plain (L2 write-back) store, for data whose reader runs on the same XCD: it is
// complete once the XCD's L2 holds it, and that reader's sc1 loads see the dirty line.
__device__ __forceinline__ void st_l2_16(const void* base, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(uniform_ptr(base), 0x7fffffff), off, 0, 0);
}
__device__ __forceinline__ void st_bf16x8(u16* base, size_t idx, const u16 (&v)[8]) {
  st_wt16(base, (uint32_t)(idx * 2), u32x4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                                            (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)});
}
__device__ __forceinline__ void st_f32x4(float* base, size_t idx, float4 v) {
  st_wt16(base, (uint32_t)(idx * 4), u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)});
}
__device__ __forceinline__ void st_f32(float* p, float v) { st_u32(p, __float_as_uint(v)); }
__device__ __forceinline__ uint32_t ld_u32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte coherent load of four flag words, completed before it returns.
__device__ __forceinline__ u32x4 ld_flags4(const unsigned* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// Thread index as an opaque value: every phase derives its lane addresses from it afresh, so the
// compiler does not hoist them out of the step/layer loops and hold them live across all phases.
__device__ __forceinline__ int phase_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Marks values loaded ahead of a poll as used, on a path that leaves the phase without using
// them: a wait that gave up, or a wave or row that has no use for them.  The compiler's wait
// counting is path-insensitive, so a load still pending on such a path counts as pending
// wherever the phases continue, and the next write of its registers then gets a wait -- a full
// vmcnt(0) once a store is in flight, which also waits for the flag stores of the last publish
// ahead of the next phase's polls.  Where it is placed (before a publish, which waits for every
// store, or on the failure path) the wait it asks for costs nothing.  Measured on MI355X, B=1:
// qkv's and down_proj's preloads consumed, 4.997 -> 4.915 ms per predict; the same for o_proj,
// gate_up or the attention splits measured slower (register assignment moves the waits).
template <class T>
__device__ __forceinline__ void consume(const T& v) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8 || sizeof(T) == 4, "one value of whole registers");
  if constexpr (sizeof(T) == 16) {
    const u32x4 r = __builtin_bit_cast(u32x4, v);
    asm volatile("" ::"v"(r));
  } else if constexpr (sizeof(T) == 8) {
    const u32x2 r = __builtin_bit_cast(u32x2, v);
    asm volatile("" ::"v"(r));
  } else {
    const uint32_t r = __builtin_bit_cast(uint32_t, v);
    asm volatile("" ::"v"(r));
  }
}
template <class T, int N>
__device__ __forceinline__ void consume(const T (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) consume(v[i]);
}
template <class T, class... Ts>
__device__ __forceinline__ void consume(const T& v, const Ts&... vs) {
  consume(v);
  if constexpr (sizeof...(Ts) > 0) consume(vs...);
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for), N a compile-time constant < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ bool copy_wave() { return phase_tid() >= kCompThreads; }

// s_waitcnt vmcnt(0) that is also a compiler barrier for memory operations: every store issued
// before it in program order stays before it, so its completion is what the wait observes.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that orders LDS only: each wave's LDS operations complete, then s_barrier; the
// empty asm statements keep the compiler from moving memory operations across it.  Unlike
// __syncthreads() it carries no workgroup-scope fence, whose release half makes every wave with a
// vector load in flight wait for it (vmcnt(0)) before the barrier -- and a wave's vector memory
// operations complete in issue order, so that wait also covers the copy wave's whole direct-to-LDS
// burst, the poller's second poll and its earlier flag stores.  Uses that need global memory or
// a direct-to-LDS copy complete wait for it explicitly before the barrier (publish, the phase
// tops that consume copied weights, the query fragments of the attention splits).
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited for
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Operand blocks are loaded with the compiler's own buffer loads (so it counts them) and fenced
// with a scheduling barrier after the last one: the scheduler may not sink a load next to its
// use, so a whole block is in flight at once and each MFMA waits only for its own fragments.
__device__ __forceinline__ void buf_frag(bf16x8& v, brsrc r, int off) {
  v = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void buf_f32(float& v, brsrc r, int off) { v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)); }
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// MFMA steps S2.. of an operand block af[4][KSW]: step s2 reads its NT weight fragments from
// LDS (wk(t, s2)) and accumulates the four m-tiles.  WT: the products are formed as W . A^T, so
// lane l ends with output columns 4 (l / 16) .. + 3 of row l % 16 (the A . W form: rows
// 4 (l / 16) .. + 3 of column l % 16).
template <int KSW, int NT, int S2, int MT, bool WT = false, class WK>
__device__ __forceinline__ void mfma_steps(f32x4 (&acc)[MT][NT], bf16x8 (&af)[MT][KSW], WK wk) {
  if constexpr (S2 < KSW) {
    bf16x8 wf[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) wf[t] = wk(t, S2);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[mt][t] = WT ? mfma16x16x32(wf[t], af[mt][S2], acc[mt][t]) : mfma16x16x32(af[mt][S2], wf[t], acc[mt][t]);
    mfma_steps<KSW, NT, S2 + 1, MT, WT>(acc, af, wk);
  }
}

// Four bf16 (8 bytes, write-through) at element idx of base (idx a multiple of 4).
__device__ __forceinline__ void st_bf16x4(u16* base, size_t idx, const u16 (&v)[4]) {
  st_wt8(base, (uint32_t)(idx * 2), (uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
}

// What every phase's waits and publishes need: this launch's epoch (read from the context's
// launch-control block at kernel entry, by every workgroup, before any flag of this launch can be
// published; kept in a scalar register) and the workgroup's LDS word through which wave 0 tells
// the others how a wait ended.
struct Sync {
  unsigned epoch;
  int* flag;
};

// ---- phases, items and flags ------------------------------------------------------------------
enum { kPhIo = 0, kPhQkv = 1, kPhSplit = 2, kPhMerge = 3, kPhO = 4, kPhGu = 5, kPhDown = 6, kNumPh = 7 };
constexpr int kQkvPairs = 80;        // 72 RoPE pairs of q/k tiles + 8 pairs of v tiles
constexpr int kQkvItems = 2 * kQkvPairs;  // B = 2: each pair in two items, rows 0..31 and rows 32..49
// B = 2: qkv item i runs on workgroup kQkvWg0 + i, not on workgroups 0..63, which finish the
// previous layer's down_proj tiles (the two items of a pair share an XCD: 80 is a multiple of 8)
constexpr int kQkvWg0 = 64;
__device__ __forceinline__ int qkv_item() { return wg_id() - kQkvWg0; }
constexpr int kTiles = kWidth / 16;  // 64 output tiles of o_proj / down_proj
constexpr int kGuItems = kMlp / 16;  // 256 (gate tile j, up tile j)
constexpr int kKSplit = 4;           // K quarters of down_proj
constexpr int kHeadPairs = kHeads / 2;  // attention merges: (row block, pair of heads)
constexpr int kPairs = kHorizon / 2; // 25 two-token attention row blocks per sample

// Flags of one phase instance: kFlagCopies replicas of a.fstride words, word i = item i
// (attention: split flags at bp * nsplit_pad + split, merge flags at 4 * bp + head_pair).
// A producer sets every replica; workgroup w polls replica w mod kFlagCopies.
// o_proj: words [0, 256) flag the items (m-tile mq, tile nt) at 64 mq + nt.  down_proj: words
// [0, 64) flag the finished tiles; words kPartFlags + 4*tile + q - 1 flag K quarter q = 1..3 of a
// tile for its finisher (quarter 0)
constexpr int kPartFlags = 256;
constexpr int kOItems = kTiles * (kRowsPerSample / 16);  // o_proj items: (m-tile of a sample, tile)
constexpr int kDownItems1 = kTiles * (kRowsPerSample / 16);  // one-sample down_proj items: (tile, m-tile)
// Batches of kAttnGroupMinBatch and more (in kernel instance 2): grouped attention items
// (attn_group_items), which stage K/V blocks in region B as well, so down(l)'s weights are copied
// to B before o_proj(l) instead of at qkv(l).  G: a batched instance.
template <bool G>
__device__ __forceinline__ bool attn_grouped(KArgs& a) {
  return G && PI05_INSTANCE_GROUPED && a.batch >= kAttnGroupMinBatch;
}
__device__ __forceinline__ unsigned* flag_base(KArgs& a, int s, int l, int ph) {
  return a.flags + ((size_t)(s * (a.depth + 1) + l) * kNumPh + ph) * kFlagCopies * a.fstride;
}

// A timed-out wait: the launch's epoch goes to the device error word, which every waiting
// workgroup of this launch checks, so all of them leave (leave_launch then counts the launch in
// the host's word).  Words of earlier launches hold older epochs, so nothing needs clearing
// between launches.
__device__ void record_error(KArgs& a, unsigned epoch) { st_u32(a.err + kCtlErr, epoch); }

// Every workgroup counts itself out of the launch.  The last one out -- every other workgroup has
// read this launch's epoch by then, at its entry -- makes this epoch the last finished one and
// resets the count, so the next launch on the stream (another call, or a replay of a captured
// graph of this one) runs with a fresh epoch; the host passes none.  A launch whose waits timed out
// is counted in the pinned host word (one writer: the last workgroup out of a launch).  The launch
// that reaches kEpochWrap zeroes the flags and the error word first and restarts the epochs at 1.
//
// Placement check.  In the batch instances the down_proj K quarters of a tile hand their partials
// and flags over through one XCD's L2 (st_l2_16, publish_local), which is correct only if
// workgroups w and w + 8k run on the same XCD (the one-sample kernel has no such hand-off; its
// launches are checked all the same).  The dispatcher deals workgroups to the 8 XCDs round-robin, starting where the
// previous dispatch stopped, so workgroup w runs on XCD (w + d) mod 8 with one offset d per launch.
// Before counting itself out, every workgroup sets bit (XCC_ID - w) mod 8 of the placement word
// (and waits for the or, so it is performed before the count); the last one out counts a launch
// with more than one bit set in the pinned host word, which the host reports as an error.
__device__ void leave_launch(KArgs& a, Sync sy) {
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const unsigned w = (unsigned)wg_id();
    const unsigned d = (xcc - w + (w & 1u) * a.xcd_skew) & 7u;
    const unsigned prev = __hip_atomic_fetch_or(a.err + kCtlXcd, 1u << d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(prev));  // the or has been performed
    *sy.flag = __hip_atomic_fetch_add(a.err + kCtlExit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)wg_count() - 1;
  }
  __syncthreads();
  if (!*sy.flag) return;
  unsigned last = sy.epoch;
  if (threadIdx.x == 0 && ld_u32(a.err + kCtlErr) == sy.epoch) {
    const unsigned n = __hip_atomic_load(a.host_err + kHostTimeouts, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(a.host_err + kHostTimeouts, n + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  if (threadIdx.x == 0) {
    if (__builtin_popcount(ld_u32(a.err + kCtlXcd)) != 1) {
      const unsigned n = __hip_atomic_load(a.host_err + kHostPlacement, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(a.host_err + kHostPlacement, n + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    st_u32(a.err + kCtlXcd, 0);
  }
  if (sy.epoch >= kEpochWrap) {
    uint4* f = reinterpret_cast<uint4*>(a.flags);
    for (size_t i = threadIdx.x; i < a.flag_bytes / 16; i += blockDim.x) f[i] = uint4{0, 0, 0, 0};
    if (threadIdx.x == 0) st_u32(a.err + kCtlErr, 0);
    wait_stores();
    __syncthreads();
    last = 0;
  }
  if (threadIdx.x == 0) {
    st_u32(a.err + kCtlExit, 0);
    st_u32(a.err + kCtlEpoch, last);
  }
}

// Wave 0 polls until flags f[0..n) all hold this launch's epoch (f 16-byte aligned; the 16-byte
// loads may read up to 3 words past n, which the allocation covers).  Ends with a workgroup
// barrier; returns false (uniformly) after a timeout or another workgroup's error.
__device__ bool wait_flags(KArgs& a, const unsigned* f, int n, Sync sy) {
  f += (size_t)((unsigned)wg_id() % kFlagCopies) * a.fstride;
  if (phase_tid() < 64) {
    const int lane = phase_tid();
    const unsigned ep = sy.epoch;
    int ok = 1;
    // one coherent (sc1) 16-byte poll in flight at a time: measured on MI355X, keeping a second
    // poll in flight (staggered by half a round trip) makes the whole predict ~4% slower -- poll
    // traffic on the flag lines delays the flag stores it waits for.  The compiler barrier keeps
    // every poll a fresh load.
    const brsrc rf = make_rsrc(f, (size_t)a.fstride * 4);
    for (int base = 0; base < n && ok; base += 256) {
      const int i0 = base + lane * 4;
      const int off = i0 < n ? i0 * 4 : kOob;
      auto done = [&](u32x4 v) {
        return i0 >= n || (v[0] == ep && (i0 + 1 >= n || v[1] == ep) && (i0 + 2 >= n || v[2] == ep) && (i0 + 3 >= n || v[3] == ep));
      };
      for (int spins = 0;; ++spins) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rf, off, 0, 16);
        if (__all(done(v))) break;
        if (spins > a.spin_limit || ((spins & 63) == 63 && __builtin_amdgcn_readfirstlane(ld_u32(a.err + kCtlErr)) == sy.epoch)) {
          if (lane == 0) record_error(a, sy.epoch);
          ok = 0;
          break;
        }
        asm volatile("" ::: "memory");
      }
    }
    if (lane == 0) *sy.flag = ok;
  }
  wg_barrier();
  const bool ok = *sy.flag != 0;
  wg_barrier();
  return ok;
}

// The same for cnt runs of n flags each, run r starting stride words after run r - 1 (f and the
// stride 16-byte aligned): one poll covers the runs of every sample an item serves, where a wait
// per sample would cost a memory round trip each.
__device__ bool wait_flag_runs(KArgs& a, const unsigned* f, int n, int stride, int cnt, Sync sy) {
  f += (size_t)((unsigned)wg_id() % kFlagCopies) * a.fstride;
  if (phase_tid() < 64) {
    const int lane = phase_tid();
    const unsigned ep = sy.epoch;
    const int cpr = (n + 3) >> 2, nch = cpr * cnt;  // 4-word chunks per run, in all
    int ok = 1;
    const brsrc rf = make_rsrc(f, (size_t)a.fstride * 4);
    for (int base = 0; base < nch && ok; base += 64) {
      const int c = base + lane, run = c / cpr, j = (c - run * cpr) * 4;
      const bool act = c < nch;
      const int off = act ? (run * stride + j) * 4 : kOob;
      auto done = [&](u32x4 v) {
        return !act || (v[0] == ep && (j + 1 >= n || v[1] == ep) && (j + 2 >= n || v[2] == ep) && (j + 3 >= n || v[3] == ep));
      };
      for (int spins = 0;; ++spins) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rf, off, 0, 16);
        if (__all(done(v))) break;
        if (spins > a.spin_limit || ((spins & 63) == 63 && __builtin_amdgcn_readfirstlane(ld_u32(a.err + kCtlErr)) == sy.epoch)) {
          if (lane == 0) record_error(a, sy.epoch);
          ok = 0;
          break;
        }
        asm volatile("" ::: "memory");
      }
    }
    if (lane == 0) *sy.flag = ok;
  }
  wg_barrier();
  const bool ok = *sy.flag != 0;
  wg_barrier();
  return ok;
}

// The stores of this item are complete (the compute waves', and the copy wave's when
// `copy_stores`: it waits only then, since its stores complete behind its direct-to-LDS copies)
// -> wave 0 sets the item's flag in every replica.  Every thread of the workgroup calls it (it
// holds a barrier).
__device__ __forceinline__ void publish(KArgs& a, unsigned* flag, unsigned epoch, bool copy_stores = false) {
  if (!copy_wave() || copy_stores) wait_stores();
  wg_barrier();
  const int t = phase_tid();
  if (t < kFlagCopies) st_u32(flag + (size_t)t * a.fstride, epoch);
}

// The same for a flag that only workgroups of this XCD poll, after data stored with st_l2_16:
// one replica (this workgroup's, which its XCD's consumer polls), stored plain into the XCD's L2
// (an intra-XCD hand-off: 0.69 us against ~1 us through the memory side, measured on MI355X).
__device__ __forceinline__ void publish_local(KArgs& a, unsigned* flag, unsigned epoch) {
  if (!copy_wave()) wait_stores();
  wg_barrier();
  if (phase_tid() == 0) {
    const brsrc r = make_rsrc(uniform_ptr(flag + (size_t)((unsigned)wg_id() % kFlagCopies) * a.fstride), 4);
    __builtin_amdgcn_raw_buffer_store_b32(epoch, r, 0, 0, 0);
  }
}

// ---- LDS map (floats) -------------------------------------------------------------------------
//   A: qkv or gate_up weight fragments of this workgroup's item: two 32-fragment tiles (64 KiB);
//      during attention its upper half holds the O fragments of waves 1 and 2
//   B: down_proj weight fragments (32 KiB)
//   then the working area of the current phase.  (o_proj holds its weights in registers.)
// Copy schedule (copy wave, per layer l).  A copy takes about 25 ns to issue and lands 2-3 us
// later, so every burst is issued just before a flag wait (the copy wave reaches the next barrier
// while the producers are still working) and never between two compute barriers, where it would
// hold up the compute waves:
//   qkv(l) wait      : all copies landed (qkv(l) weights); B > 1: down(l) -> B (32); one sample:
//                      gate_up(l) tile 0 -> A (32)
//   attention(l) wait: B > 1: gate_up(l) tile 0 fragments 0..15 -> A (16), after the copy wave's
//                      own KV block loads
//   merge(l) wait    : B > 1: gate_up(l) tile 0 fragments 16..31 (16); tile 1 (32) -> A
//   o_proj(l) wait   : one sample: qkv(l+1) tile 0 -> B (32)
//   gate_up(l) wait  : all copies landed (gate_up(l) weights)
//   down(l) wait     : qkv(l+1) tile 1 fragments 0..30 (31) -> A, B > 1: and tile 0 (32) (one
//                      sample: after the copy wave's own down(l) weight loads)
// so at most 63 copies are ever in flight and a burst never waits for the one before it.
constexpr int kLdsA = 0;
constexpr int kLdsB = kLdsA + 16384;
constexpr int kLdsWork = kLdsB + 8192;
constexpr int kWorkFloats = 8736;
constexpr int kLdsFloats = kLdsWork + kWorkFloats;
// the batched kernel instance's working area (its gate_up reduces four waves' partials)
constexpr int kWorkFloatsBatched = 10752;
constexpr int kLdsFloatsBatched = kLdsWork + kWorkFloatsBatched;
static_assert(kLdsFloats * 4 <= 160 * 1024 && kLdsFloatsBatched * 4 <= 160 * 1024, "LDS budget of a gfx950 workgroup");
constexpr int kLdsA1 = kLdsA + 8192;  // upper half of A (tile 1); during attention: wave O slots

// An LDS address as an address-space-3 pointer, from the low 32 bits of a generic pointer into
// LDS (which hold the LDS offset).  Direct-to-LDS loads take their destination in that form;
// converting a generic pointer with a cast costs a null check per load and keeps 64-bit generic
// addresses live in scalar registers across the phases.
typedef __attribute__((address_space(3))) u16 lds_u16;
__device__ __forceinline__ lds_u16* lds_addr(const void* p) {
  return (lds_u16*)(uintptr_t)(uint32_t)reinterpret_cast<uintptr_t>(p);
}

// A burst of N contiguous 1 KiB fragments (N <= 63, a compile-time count) from src to LDS dst by
// the copy wave: first make room (at most 63 - N copies in flight), then N buffer loads straight
// into LDS (fragment f of src lands at dst + f KiB).  One VGPR holds the lane offset and the
// fragment offset is a scalar, and the sequence is unrolled, so the compiler counts the copies
// exactly and waits for later loads of this wave precisely.  The loads are non-temporal (aux bit
// nt): each weight byte is read once per step, and streaming it through the caches that way
// keeps the activations and the prefix K/V, which are re-read, resident (measured: 1.7% faster
// per predict than with the default policy).
template <int N>
__device__ __forceinline__ void lds_burst(float* dst, const u16* src) {
  static_assert(N > 0 && N <= 63, "vmcnt range");
  if (!copy_wave()) return;
  wait_vmcnt<63 - N>();
  const brsrc r = make_rsrc(src, (size_t)N * 1024);
  const unsigned vo = (phase_tid() & 63) * 16;
  lds_u16* d = lds_addr(dst);
#pragma unroll
  for (int f = 0; f < N; ++f) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, d + f * 512, 16, vo, f * 1024, 0, kAuxNt);
}

// Fragments [F0, F0 + N) of tile `which` (0 or 1) of the qkv (MODE = kModeQkv) or gate_up
// weights of item (unsigned)wg_id() -> region A.  A qkv item's tile 1 is copied without its last
// fragment (k-step 31), which the wave owning that k-step loads into registers: both qkv tiles
// then fit one 63-copy burst.
// gate_up items.  B = 1: workgroup w computes tile pair w (gate tile w, up tile w) for the one
// sample.  B > 1: workgroup w computes tile pairs 2g and 2g + 1, g = w mod 128, for half of the
// samples (w / 128): each activation row it reads then serves four tiles instead of two, so an
// XCD's workgroups read half as many activation bytes (the phase is bound by that L2 traffic).
// Region A holds pair 2g; the compute waves hold pair 2g + 1 in registers.
// The qkv of kernel instance 2 (phase_qkv_msplit): item i = tile pair i mod 80 for sample half
// i / 80.
template <bool G>
__device__ __forceinline__ constexpr bool qkv_msplit() {
  return G && PI05_INSTANCE_GROUPED;
}
// phase_qkv_msplit's items: tile pair i mod 80 for sample third i / 80; phase_qkv1's (one
// sample): tile pair i mod 80 for row group i / 80 (m-tile 0, m-tile 1, m-tiles 2 and 3); either
// way on workgroups 16..255 (the three items of a pair share an XCD: 80 is a multiple of 8)
constexpr int kQkvItemsRS = 3 * kQkvPairs;
constexpr int kQkvWg0RS = 256 - kQkvItemsRS;
template <bool G>
__device__ __forceinline__ constexpr int n_qkv_items() {
  return qkv_msplit<G>() || !G ? kQkvItemsRS : kQkvItems;
}
template <bool G>
__device__ __forceinline__ int qkv_item_of() {
  return qkv_msplit<G>() || !G ? wg_id() - kQkvWg0RS : qkv_item();
}
// The gate_up of kernel instance 2 (phase_gateup_msplit, batches of kRowSplitMinBatch and more):
// item w = pair w.
template <bool G>
__device__ __forceinline__ bool gu_msplit(KArgs&) {
  return G && PI05_INSTANCE_GROUPED;
}
__device__ __forceinline__ int gu_pair0(KArgs&) {
  return 2 * (wg_id() % (kGuItems / 2));
}
// qkv items.  B = 1: item i = qkv_item_of() computes tile pair i mod 80 over row group i / 80 of
// the sample.  B = 2 (kernel instance 1): item i computes tile pairs 2 (i mod 40) and 2 (i mod 40) + 1
// over row half (i / 40) mod 2 for sample half i / 80, as gate_up's pair items do; region A holds
// the first pair.  Kernel instance 2: item i = tile pair i mod 80 for sample third i / 80.
template <bool G>
__device__ __forceinline__ int qkv_pair0(KArgs& a) {
  return G && a.batch > 1 && !qkv_msplit<G>() ? 2 * (qkv_item() % (kQkvPairs / 2)) : qkv_item_of<G>() % kQkvPairs;
}
template <int MODE, bool G = false>
__device__ __forceinline__ const u16* norm_w_tile(KArgs& a, int l, int which) {
  constexpr int KSTEPS = kWidth / 32;
  const int p = MODE == kModeQkv ? qkv_pair0<G>(a) : (gu_msplit<G>(a) ? wg_id() : gu_pair0(a));  // qkv: the tile pair
  const u16* wl = a.wpack + (size_t)l * kLayerElems;
  if constexpr (MODE == kModeQkv) {
    const bool rotated = p < 72;
    const int head = p >> 3, dt = p & 7;
    const int tile0 = rotated ? head * 16 + dt : 144 + 2 * (p - 72);
    const int tile = which == 0 ? tile0 : (rotated ? tile0 + 8 : tile0 + 1);
    return wl + kOffQkv + (size_t)tile * KSTEPS * 512;
  } else {
    return wl + (which == 0 ? kOffGate : kOffUp) + (size_t)p * KSTEPS * 512;
  }
}
template <int MODE, int F0, int N, bool G = false>
__device__ void copy_norm_w(KArgs& a, int l, int which, float* smem) {
  if (!copy_wave()) return;
  if (MODE == kModeQkv ? (unsigned)qkv_item_of<G>() >= (unsigned)n_qkv_items<G>() : (unsigned)wg_id() >= kGuItems) return;
  lds_burst<N>(smem + kLdsA + which * 8192 + F0 * 256, norm_w_tile<MODE, G>(a, l, which) + F0 * 512);
}
// One sample: qkv(l)'s first tile -> region B, which nothing else uses at one sample (the second
// tile goes to region A1 at down_proj(l - 1), after gate_up's last read of region A).
__device__ void copy_qkv_tile0(KArgs& a, int l, float* smem) {
  if (!copy_wave() || (unsigned)qkv_item_of<false>() >= (unsigned)n_qkv_items<false>()) return;
  lds_burst<32>(smem + kLdsB, norm_w_tile<kModeQkv, false>(a, l, 0));
}

// down_proj weights of workgroup (unsigned)wg_id(): (tile, K quarter) -> region B.
// down_proj items.  B = 1 (phase_down_rows): workgroup w = (tile w mod 64, m-tile w / 64) over
// the whole K; its copy wave multiplies K quarter w / 64, which region B holds.  B > 1: workgroup
// w = 64 q + 32 h + g computes tiles 2g and 2g + 1 over K quarter q for half h of the samples --
// half the activation bytes per XCD, as for gate_up; the quarters of a group run on one XCD (w mod
// 8 is the same for all four) and poll one flag replica (w mod kFlagCopies), and the finishers (quarter 0)
// are workgroups 0..63, which hold no qkv item.  Region B holds the first tile's quarter; the
// compute waves hold the second one in registers.
__device__ __forceinline__ void down_item(KArgs& a, int* nt0, int* ksp, int* half = nullptr) {
  const int w = wg_id();
  *ksp = w / kTiles;
  if (a.batch > 1) {
    *nt0 = 2 * (w % (kTiles / 2));
    if (half) *half = (w / (kTiles / 2)) % 2;
  } else {
    *nt0 = w % kTiles;
    if (half) *half = 0;
  }
}
template <int KSTEPS>
__device__ void copy_residual_w(KArgs& a, int l, float* smem) {
  constexpr int KQ = KSTEPS / kKSplit;
  const int item = (unsigned)wg_id();
  if (!copy_wave() || item >= kTiles * kKSplit) return;
  int nt, ksp;
  down_item(a, &nt, &ksp);
  const u16* tile = a.wpack + (size_t)l * kLayerElems + kOffDown + (size_t)nt * KSTEPS * 512 + (size_t)ksp * KQ * 512;
  lds_burst<KQ>(smem + kLdsB, tile);
}

// Kernel instance 2: down_proj's second tile (nt0 + 1) of the item's K quarter -> the working
// area's first kDownW1Floats floats (phase_down_msplit reads it after tile nt0's quarter in B).
constexpr int kDownW1Floats = 8192;
__device__ void copy_down_w1(KArgs& a, int l, float* smem) {
  constexpr int KSTEPS = kMlp / 32, KQ = KSTEPS / kKSplit;
  if (!copy_wave() || wg_id() >= kTiles * kKSplit) return;
  int nt, ksp;
  down_item(a, &nt, &ksp);
  lds_burst<KQ>(smem + kLdsWork, a.wpack + (size_t)l * kLayerElems + kOffDown + (size_t)(nt + 1) * KSTEPS * 512 + (size_t)ksp * KQ * 512);
}

// The layer after (s, l): (s, l + 1), or (s + 1, 0) after the last layer; false past the loop.
__device__ __forceinline__ bool next_layer(KArgs& a, int s, int l, int* ln) {
  if (l + 1 < a.depth) {
    *ln = l + 1;
    return true;
  }
  *ln = 0;
  return s + 1 < a.steps;
}

template <int MT, int NT>
__device__ __forceinline__ void store_wave_partials(float* red, const f32x4 (&acc)[MT][NT], int wave, int lane) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>(red + (((size_t)(wave * MT + mt) * NT + t) * 64 + lane) * 4) = acc[mt][t];
}

// Sum the compute waves' D fragments (red[wave][mt][t][lane], f32x4, MT m-tiles) in wave order
// and scatter them row-major into the LDS tile T[16 MT][TS] (column t*16 + n), which must not
// alias red.  Thread tid < 64 MT owns m-tile tid/64, lane tid%64 of every tile t (with MT = 4 the
// copy wave takes m-tile 3: LDS work only).
template <int MT, int NT, int TS>
__device__ __forceinline__ void reduce_to_tile(const float* red, float* T) {
  const int tid = phase_tid();
  const int mt = tid >> 6, ln = tid & 63;
  if (mt >= MT) return;
  f32x4 r[kCompWaves][NT];
#pragma unroll
  for (int w = 0; w < kCompWaves; ++w)
#pragma unroll
    for (int t = 0; t < NT; ++t) r[w][t] = *reinterpret_cast<const f32x4*>(red + (((size_t)(w * MT + mt) * NT + t) * 64 + ln) * 4);
  sched_fence();  // every read in flight before the first sum
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 v = r[0][t];
#pragma unroll
    for (int w = 1; w < kCompWaves; ++w) v += r[w][t];
#pragma unroll
    for (int i = 0; i < 4; ++i) T[(mt * 16 + (ln >> 4) * 4 + i) * TS + t * 16 + (ln & 15)] = v[i];
  }
}

// The same over NW waves' partials (red[wave][mt][t][lane], NW * MT * NT fragments).
template <int NW, int MT, int NT, int TS>
__device__ __forceinline__ void reduce_to_tile_n(const float* red, float* T) {
  const int tid = phase_tid();
  const int mt = tid >> 6, ln = tid & 63;
  if (mt >= MT) return;
  f32x4 r[NW][NT];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int t = 0; t < NT; ++t) r[w][t] = *reinterpret_cast<const f32x4*>(red + (((size_t)(w * MT + mt) * NT + t) * 64 + ln) * 4);
  sched_fence();
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 v = r[0][t];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += r[w][t];
#pragma unroll
    for (int i = 0; i < 4; ++i) T[(mt * 16 + (ln >> 4) * 4 + i) * TS + t * 16 + (ln & 15)] = v[i];
  }
}

// Row sums of squares, tiles [t0, t0 + 32), of the 64 rows of sample b (lane = row) from the
// tile-major partials ss[64][R]: 32 loads of 256 contiguous bytes each.
__device__ __forceinline__ void load_row_stats(float (&v)[32], const float* ss, int R, int b, int t0, int lane) {
#pragma unroll
  for (int t = 0; t < 32; ++t) v[t] = ss[(size_t)(t0 + t) * R + b * kRowsPerSample + lane];
}
__device__ __forceinline__ float sum32(const float (&v)[32]) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int t = 0; t < 32; t += 4) {
    a0 += v[t];
    a1 += v[t + 1];
    a2 += v[t + 2];
    a3 += v[t + 3];
  }
  return (a0 + a1) + (a2 + a3);
}

// =============================================================================================
// step boundary: final norm + action_out_proj + Euler of step s-1, action_in_proj of step s.
// Items: action-token rows (compact c = b*50 + t).  x[s] = Euler(x[s-1], v_{s-1});
// h[s][0] = bf16(action_in_proj(x[s])), g[s][0] = bf16(h * (1 + scale_0)) and its row statistics.
// The three compute waves work here: action_out_proj with 6 threads per output (k-runs of 172,
// 172, 172, 172, 172, 164), action_in_proj with 6 hidden columns per thread.
// =============================================================================================
constexpr int kOutParts = 6;
constexpr int kOutRun = 172;
template <bool G>
__device__ bool phase_io(KArgs& a, int s, float* smem, Sync sy) {
  const int L = a.depth, NN = 2 * L + 1, R = a.R, NC = a.batch * kHorizon;
  const int tid = phase_tid();
  const bool comp = tid < kCompThreads;
  const int j = tid / kOutParts, part = tid % kOutParts;   // action_out_proj output j, k-run part
  const int k0 = part * kOutRun;
  const int nq = part < kOutParts - 1 ? kOutRun / 4 : (kWidth - (kOutParts - 1) * kOutRun) / 4;
  const int c0 = tid * 6;                                  // action_in_proj: hidden columns c0..c0+5
  const int kc = ((tid >> 2) & 31) * 32 + (tid & 3) * 8;   // final norm: 8 columns per thread (tid < 128)
  float* s_n = smem + kLdsWork;       // [W] final-norm output
  float* s_x = s_n + kWidth;          // [a] actions of step s
  float* s_v = s_x + kActDim;         // [a] velocity of step s-1 (unused slot kept for layout)
  float* s_rstd = s_v + kActDim;      // [4]
  float* s_red = s_rstd + 4;          // [192] action_out_proj partials
  u16* s_h = reinterpret_cast<u16*>(s_red + kCompThreads);  // [W] bf16 h row, then [W] bf16 g row
  u16* s_g = s_h + kWidth;
  const bool has_prev = s > 0, has_next = s < a.steps;
  bool waited = false;
  for (int c = (unsigned)wg_id(); c < NC; c += (unsigned)wg_count()) {
    const int b = c / kHorizon, t = c % kHorizon, r = b * kRowsPerSample + t;
    // ---- loads that do not depend on the previous phase (waves 1 and 2 only: wave 0 polls, so
    // it issues nothing ahead of its polls and loads its share after the wait)
    float4 wo[kOutRun / 4];
    float4 sc[2] = {}, sh[2] = {};
    auto load_wo = [&]() {
#pragma unroll
      for (int q = 0; q < kOutRun / 4; ++q)
        if (q < nq) wo[q] = *reinterpret_cast<const float4*>(a.out_w + (size_t)j * kWidth + k0 + q * 4);
    };
    auto load_mod = [&]() {  // final norm: 1 + scale and shift of this thread's 8 columns
      const float* fmod = a.table + ((size_t)(s - 1) * NN + (NN - 1)) * kModW;
      sc[0] = *reinterpret_cast<const float4*>(fmod + kc);
      sc[1] = *reinterpret_cast<const float4*>(fmod + kc + 4);
      sh[0] = *reinterpret_cast<const float4*>(fmod + kWidth + kc);
      sh[1] = *reinterpret_cast<const float4*>(fmod + kWidth + kc + 4);
    };
    if (has_prev && comp && tid >= 64) {
      load_wo();
      if (tid < 128) load_mod();
    }
    if (has_prev && !waited) {
      if (!wait_flags(a, flag_base(a, s - 1, L - 1, kPhDown), kKSplit * kTiles, sy)) return false;  // every down_proj item (256 either way)
      waited = true;
    }
    if (has_prev && tid < 64) {
      load_wo();
      load_mod();
    }
    if (has_prev) {
      const size_t sl = (size_t)(s - 1) * (L + 1) + L;
      float rs = 0.f;
      u16x8 hv = {0, 0, 0, 0, 0, 0, 0, 0};
      if (tid < kTiles) rs = a.ss[(sl * kTiles + tid) * R + r];
      if (tid < 128) hv = *reinterpret_cast<const u16x8*>(a.h + sl * R * kWidth + afrag_index(r, kc, kWidth / 32));
      // final adaRMSNorm (model.norm, modeling_gemma.py:782-783)
      if (tid < kTiles) {
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
      // v = action_out_proj(n), fp32 (engine.py:767): partial dot products, then in order
      if (comp) {
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < kOutRun / 4; ++q) {
          if (q < nq) {
            const float* n = s_n + k0 + q * 4;
            acc += wo[q].x * n[0] + wo[q].y * n[1] + wo[q].z * n[2] + wo[q].w * n[3];
          }
        }
        s_red[tid] = acc;
      }
      __syncthreads();
      if (tid < kActDim) {
        float v = s_red[tid * kOutParts];
#pragma unroll
        for (int q = 1; q < kOutParts; ++q) v += s_red[tid * kOutParts + q];
        v += a.out_b[tid];
        const float xj = (s == 1 ? a.x_io : a.x + (size_t)(s - 1) * NC * kActDim)[(size_t)c * kActDim + tid];
        const float* e = a.euler + (size_t)(s - 1) * 4;  // t, 1 - t, x0 weight, x1 weight
        // flow_ode mean in the reference's op order (engine.py:664-675)
        const float x0_pred = fsub(xj, fmul(v, e[0]));
        const float x1_pred = fadd(xj, fmul(v, e[1]));
        const float xn = fadd(fmul(x0_pred, e[2]), fmul(x1_pred, e[3]));
        s_x[tid] = xn;
        st_f32((s == a.steps ? a.x_io : a.x + (size_t)s * NC * kActDim) + (size_t)c * kActDim + tid, xn);
        if (a.trace) st_f32(a.trace + ((size_t)(s - 1) * NC + c) * kActDim + tid, v);
      }
    } else if (tid < kActDim) {
      s_x[tid] = a.x_io[(size_t)c * kActDim + tid];
    }
    __syncthreads();
    if (has_next) {
      // h = bf16(action_in_proj(x)) (pi0_pytorch.py:303-306; modeling_gemma.py:724-725),
      // g = bf16(h * (1 + scale)) of layer 0's input norm at step s
      if (comp && c0 < kWidth) {
        const int nc = c0 + 6 <= kWidth ? 6 : kWidth - c0;
        float4 wi[6][8];
#pragma unroll
        for (int q = 0; q < 6; ++q)
          if (q < nc)
#pragma unroll
            for (int k = 0; k < 8; ++k) wi[q][k] = *reinterpret_cast<const float4*>(a.in_w + (size_t)(c0 + q) * kActDim + k * 4);
        const float* s1 = a.table_s1 + (size_t)s * NN * kModW;
#pragma unroll
        for (int q = 0; q < 6; ++q) {
          if (q < nc) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k)
              acc += wi[q][k].x * s_x[4 * k] + wi[q][k].y * s_x[4 * k + 1] + wi[q][k].z * s_x[4 * k + 2] + wi[q][k].w * s_x[4 * k + 3];
            const u16 hb = f2bf(acc + a.in_b[c0 + q]);
            s_h[c0 + q] = hb;
            s_g[c0 + q] = f2bf(fmul(bf2f(hb), s1[c0 + q]));
          }
        }
      }
      __syncthreads();
      if (tid < 128) {
        // one 16-byte chunk of the h row and of the g row per thread; the tile sums of squares
        const size_t sl = (size_t)s * (L + 1), slg = (size_t)s * L;
        const int k = tid * 8;
        u16 hv8[8], gv8[8];
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          hv8[q] = s_h[k + q];
          gv8[q] = s_g[k + q];
          const float hf = bf2f(hv8[q]);
          ss += hf * hf;
        }
        st_bf16x8(a.h + sl * R * kWidth, afrag_index(r, k, kWidth / 32), hv8);
        st_bf16x8(a.g + slg * R * kWidth, afrag_index(r, k, kWidth / 32), gv8);
        ss += __shfl_xor(ss, 1);  // the tile's other 8 columns
        if ((tid & 1) == 0) st_f32(a.ss + (sl * kTiles + (tid >> 1)) * R + r, ss);
      }
    }
    publish(a, flag_base(a, s, 0, kPhIo) + c, sy.epoch);
    __syncthreads();  // the LDS rows are reused by the next item
  }
  return true;
}

// =============================================================================================
// qkv at one sample: adaRMSNorm-folded GEMM tile (K = 1024, 3 compute waves x 11 | 11 | 10
// k-steps) of one tile pair over one row group (m-tile 0, m-tile 1, or m-tiles 2 and 3).  A
// operand g straight from the producer; rstd from the tile sums of squares; the epilogue computes
// y = bf16(rstd * acc + shift . W^T) and then RoPE (q, k) or the permuted V layout (v).
// =============================================================================================
template <bool G>
__device__ bool phase_qkv1(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int NT = 2, KSW = 11, KSTEPS = kWidth / 32;
  constexpr int MT = 2;  // m-tile slots per item (the second used by row group 2 only)
  constexpr int PH = kPhQkv;
  const int L = a.depth, R = a.R;
  const int item = qkv_item_of<G>();
  const bool has_item = item >= 0 && item < kQkvItemsRS;
  const int p = item % kQkvPairs;   // tile pair
  const int rg = item / kQkvPairs;  // row group: m-tile 0, m-tile 1, m-tiles 2 and 3
  const int mt0 = rg < 2 ? rg : 2;  // its first m-tile
  const int rb = 16 * mt0;          // its first row within the sample
  const int nrow = rg < 2 ? 16 : kHorizon - rb;  // its action-token rows (16, 16, 18)
  PHASE_TS(s, l, PH, 0);
  // copy wave: this phase's weights (region A) and everything issued before them have landed;
  // then the bursts of this phase start
  if (copy_wave()) {
    wait_vmcnt<0>();
    // gate_up(l)'s first tile -> region A's lower half, free at one sample (qkv's first tile is in
    // region B), so the attention phases' bursts carry only its second tile.  (down_proj's copy
    // wave loads its weights itself, at down_proj.)
    copy_norm_w<kModeGateUp, 0, 32>(a, l, 0, smem);
  }
  if (!has_item) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool comp = tid < kCompThreads;
  const int r16 = lane & 15;
  const int ks0 = wave * KSW;  // this wave's k-steps [ks0, ks0 + KSW) (wave 2: the last one past K)
  const size_t slw = (size_t)s * L + l;
  const float* bias = a.bias + slw * kBiasCols;
  const bool rotated = p < 72;
  const int head = p >> 3, dt = p & 7;
  const int tile0 = rotated ? head * 16 + dt : 144 + 2 * (p - 72);
  const u16* gin = a.g + slw * R * kWidth;
  const float* ssin = a.ss + ((size_t)s * (L + 1) + l) * kTiles * R;
  // the products: W . A^T for the RoPE pairs (a lane then holds 4 consecutive columns of one row:
  // RoPE, which pairs column d of the two tiles, is lane-local, and the stores are 8 bytes), A . W
  // for the v pairs (a lane holds 4 rows of one column in each m-tile: with the two m-tiles, the 8
  // keys of one 16-byte chunk of the permuted V layout)
  const bool wt = rotated;
  float* s_rstd = smem + kLdsWork;  // [64] (item rows)
  float* s_bias = s_rstd + 64;      // [32] shift . W^T of the item's two tiles
  float* s_rs = s_bias + 32;        // [3][64] row sums of squares over tiles 22w .. 22w+21
  float* red = s_rs + 192;          // [3 waves][MT m-tiles][NT][64 lanes][4]
  // epilogue threads: waves 1 and 2 (wave 0 polls, so it issues nothing ahead of its polls),
  // e = tid - 64: RoPE pairs m-tile e / 64, lane e % 64; v pairs tile e / 64, lane e % 64 (both
  // m-tiles)
  const int e = tid - 64;
  const bool ep_thread = e >= 0 && e < 128;
  const int emt = e >> 6, eln = e & 63;
  const int erow = 16 * emt + (eln & 15);   // W . A^T: the thread's row within the item
  const int ecol = 4 * (eln >> 4);          // W . A^T: its first column within each tile
  // static operands, loaded ahead of the polls by waves 1 and 2: wave 2's qkv tile-1 fragment of
  // k-step 31 (not in LDS), and the RoPE cos/sin of the epilogue thread's row and 4 columns
  bf16x8 w31 = {};
  uint32_t rcs[4][2] = {};
  const bool rope_thread = rotated && ep_thread && erow < nrow;
  auto load_rope = [&](int b) {
    const size_t cr = (size_t)(b * kHorizon + rb + erow) * kHeadDim + dt * 16 + ecol;
    const u16* src[4] = {a.cos_tab + cr, a.sin_tab + cr, a.cos_tab + cr + kHalfDim, a.sin_tab + cr + kHalfDim};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint2 v = *reinterpret_cast<const uint2*>(src[k]);
      rcs[k][0] = v.x;
      rcs[k][1] = v.y;
    }
  };
  if (wave == 2) w31 = as_bf16x8(*reinterpret_cast<const u16x8*>(norm_w_tile<kModeQkv>(a, l, 1) + 31 * 512 + lane * 8));
  if (rope_thread) load_rope(0);
  // the item's shift . W^T columns (static within the launch), by wave 1 ahead of the polls and
  // straight into LDS: the work area is free (every wave passed the previous phase's last
  // barrier) and the wait's barrier orders the stores before their readers
  if (tid >= 64 && tid < 96) {
    const int c = tid - 64;
    const int col = c < 16 ? tile0 * 16 + c : (rotated ? tile0 + 8 : tile0 + 1) * 16 + c - 16;
    s_bias[c] = bias[col];
  }
  PHASE_TS(s, l, PH, 1);
  {
    const unsigned* dep = l == 0 ? flag_base(a, s, 0, kPhIo) : flag_base(a, s, l - 1, kPhDown);
    const int ndep = l == 0 ? a.batch * kHorizon : kDownItems1;
    if (!wait_flags(a, dep, ndep, sy)) {
      consume(w31, rcs);
      return false;
    }
  }
  PHASE_TS(s, l, PH, 2);
  const u16* lw0 = reinterpret_cast<const u16*>(smem + kLdsB);   // tile 0: [k-step] fragments
  const u16* lw1 = reinterpret_cast<const u16*>(smem + kLdsA1);  // tile 1
  {
    constexpr int b = 0;  // one sample: the batch instances have their own qkv and gate_up
    const int m0 = b * kRowsPerSample;
    // the row statistics first (wave w: tiles 22w .. 22w+21, lane = item row), then the A
    // fragments (k-step 32 of wave 2 and the padded rows read as zeros), all without branches
    f32x4 acc[MT][NT];
    if (comp) {
      const brsrc rsrc_s = make_rsrc(ssin, (size_t)kTiles * R * 4);
      const brsrc rsrc_g = make_rsrc(gin, (size_t)R * kWidth * 2);
      float st[22];
#pragma unroll
      for (int t = 0; t < 22; ++t) {
        const int tile = 22 * wave + t;
        buf_f32(st[t], rsrc_s, tile < kTiles && lane < 16 * MT ? ((tile * R + m0 + rb + lane) * 4) : kOob);
      }
      bf16x8 hr[MT][KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bool ok = r16 < nrow - mt * 16 && ks0 + s2 < KSTEPS;
          buf_frag(hr[mt][s2], rsrc_g, ok ? (int)((afrag_offset(b * 4 + mt0 + mt, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
        }
      sched_fence();
      float v = 0.f;
#pragma unroll
      for (int t = 0; t < 22; ++t) v += st[t];
      s_rs[wave * 64 + lane] = v;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      // zero A for wave 2's surplus step: any finite weights (k-step 31's); qkv tile 1's k-step 31
      // fragment is wave 2's register copy
      auto wk = [&](int t, int s2) {
        const int ksc = ks0 + s2 < KSTEPS ? ks0 + s2 : KSTEPS - 1;
        if (t == 1 && s2 >= KSTEPS - 1 - 2 * KSW && wave == 2) return w31;
        return *reinterpret_cast<const bf16x8*>((t == 0 ? lw0 : lw1) + (size_t)ksc * 512 + lane * 8);
      };
      if (wt) mfma_steps<KSW, NT, 0, MT, true>(acc, hr, wk);
      else mfma_steps<KSW, NT, 0, MT, false>(acc, hr, wk);
    }
    if (b == 0) PHASE_TS(s, l, PH, 4);
    __syncthreads();  // every wave is done with region A; the row sums are in LDS
    if (b == 0) PHASE_TS(s, l, PH, 3);
    if (comp) store_wave_partials<MT, NT>(red, acc, wave, lane);
    if (tid < 16 * MT) s_rstd[tid] = 1.0f / sqrtf(fadd(((s_rs[tid] + s_rs[64 + tid]) + s_rs[128 + tid]) * (1.0f / kWidth), a.eps));
    __syncthreads();
    if (b == 0) PHASE_TS(s, l, PH, 7);
    // the three waves' partials of this thread's accumulator positions, added in wave order
    auto wave_sum = [&](int mt, int t) {
      f32x4 r[kCompWaves];
#pragma unroll
      for (int w = 0; w < kCompWaves; ++w) r[w] = *reinterpret_cast<const f32x4*>(red + (((size_t)(w * MT + mt) * NT + t) * 64 + eln) * 4);
      return (r[0] + r[1]) + r[2];
    };
    {
      if (rotated) {
        // (x*cos) + (rotate_half(x)*sin), rotate_half(x) = cat(-x_hi, x_lo), from the bf16
        // GEMM values (rlinf_fused_denoise.py:264-278; modeling_gemma.py:185-216): dims d .. d + 3
        // of tile 0 and their partners d + 128 .. of tile 1
        if (rope_thread) {
          const f32x4 ylo = wave_sum(emt, 0), yhi = wave_sum(emt, 1);
          const float rstd = s_rstd[erow];
          u16 olo[4], ohi[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const auto half16 = [&](int k) { return bf2f((u16)(rcs[k][q >> 1] >> (16 * (q & 1)))); };
            const float x_lo = round_bf(__builtin_fmaf(rstd, ylo[q], s_bias[ecol + q]));
            const float x_hi = round_bf(__builtin_fmaf(rstd, yhi[q], s_bias[16 + ecol + q]));
            olo[q] = f2bf(fsub(fmul(x_lo, half16(0)), fmul(x_hi, half16(1))));
            ohi[q] = f2bf(fadd(fmul(x_hi, half16(2)), fmul(x_lo, half16(3))));
          }
          const int d = dt * 16 + ecol, r = rb + erow;
          if (head < kHeads) {
            u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
            const int qrow = (m0 + r) * kQRowsPerTok + head;
            st_bf16x4(qs, afrag_index(qrow, d, kHeadDim / 32), olo);
            st_bf16x4(qs, afrag_index(qrow, d + kHalfDim, kHeadDim / 32), ohi);
          } else {
            u16* kc = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
            st_bf16x4(kc, kfrag_index(r, d), olo);
            st_bf16x4(kc, kfrag_index(r, d + kHalfDim), ohi);
          }
        }
      } else if (ep_thread) {
        // v (A . W): this thread = tile e / 64, lane e % 64 -> column dcol of the tile pair, rows
        // 4 g .. 4 g + 3 of each m-tile (g = lane / 16).  The permuted V fragment's chunk (kb, g)
        // holds, in its order (vkey), keys 4 g .. 4 g + 3 of m-tiles 2 kb and 2 kb + 1: row group 2
        // writes whole chunks of kb = 1 (keys past the 50 action tokens zero), row groups 0 and 1
        // the first and second halves of the chunks of kb = 0
        const int t = emt, g = eln >> 4, dcol = t * 16 + (eln & 15);
        const int dv = (tile0 - 144) * 16 + dcol;
        u16* vc = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
        const f32x4 y0 = wave_sum(0, t);
        if (rg == 2) {
          const f32x4 y1 = wave_sum(1, t);
          u16 v8[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int row = (q < 4 ? 0 : 16) + 4 * g + (q & 3);  // vkey(1, g, q) - rb
            const float y = q < 4 ? y0[q] : y1[q - 4];
            v8[q] = rb + row < kHorizon ? f2bf(__builtin_fmaf(s_rstd[row], y, s_bias[dcol])) : (u16)0;
          }
          st_bf16x8(vc, ((size_t)16 + (dv >> 4)) * 512 + (size_t)(g * 16 + (dv & 15)) * 8, v8);
        } else {
          u16 v4[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v4[q] = f2bf(__builtin_fmaf(s_rstd[4 * g + q], y0[q], s_bias[dcol]));  // vkey(0, g, 4 rg + q) - rb
          st_bf16x4(vc, (size_t)(dv >> 4) * 512 + (size_t)(g * 16 + (dv & 15)) * 8 + 4 * rg, v4);
        }
      }
    }
  }
  PHASE_TS(s, l, PH, 5);
  consume(w31, rcs);  // (used by wave 2's last k-step and by the RoPE rows only)
  publish(a, flag_base(a, s, l, PH) + item, sy.epoch);
  PHASE_TS(s, l, PH, 6);
  return true;
}

// =============================================================================================
// gate_up at one sample, split by rows: item w = tile pairs 2p and 2p + 1 (p = w mod 128) over row
// half w / 128 (m-tiles 0, 1 or 2, 3), so an item fetches half of gmid after its wait where a
// one-pair item over all rows fetched all of it.  Pair 2p's tiles come from region A (the copy
// wave's bursts); waves 1..3 (the copy wave is free in this phase) split K (11/11/10 k-steps) and
// load pair 2p + 1's fragments of their k-steps into registers ahead of the polls; wave 0 only
// polls.  Products as W . A^T, the three waves' partials added in LDS by the epilogue threads,
// GeGLU lane-local (thread t: m-tile (t / 64) mod 2 of pair t / 128).
// =============================================================================================
__device__ bool phase_gateup_rows(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int NT = 4, MT = 2, KSW = 11, KSTEPS = kWidth / 32;
  constexpr int PH = kPhGu;
  const int L = a.depth, R = kRowsPerSample;
  const int item = wg_id();
  PHASE_TS(s, l, PH, 0);
  if (copy_wave()) wait_vmcnt<0>();  // this phase's weights (region A) have landed
  if (item >= kGuItems) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool mw = wave >= 1;  // MFMA waves 1..3
  const int cw = wave - 1;    // their K share
  const int r16 = lane & 15;
  const int ks0 = cw * KSW;   // k-steps [ks0, ks0 + KSW) (wave 3: the last one past K)
  const size_t slw = (size_t)s * L + l;
  const int p0 = 2 * (item % (kGuItems / 2)), mh = item / (kGuItems / 2);
  const int rb = 32 * mh;                                   // the item's first row
  const int nrow = kHorizon - rb < 32 ? kHorizon - rb : 32;  // its action-token rows
  const u16* gin = a.gmid + slw * R * kWidth;
  const float* ssin = a.ssmid + slw * kTiles * R;
  float* s_rstd = smem + kLdsWork;  // [32] (item rows)
  float* s_bias = s_rstd + 64;      // [2 pairs][32]: shift . W^T of gate and up tiles
  float* s_rs = s_bias + 64;        // [3][64] row sums of squares over tiles 22 cw .. 22 cw + 21
  float* red = s_rs + 192;          // [3 waves][MT][NT][64 lanes][4]
  // pair p0 + 1 of this wave's k-steps (the surplus step: any finite weights, A reads zeros)
  bf16x8 w1[2][KSW];
  if (mw) {
    const u16* wl = a.wpack + (size_t)l * kLayerElems;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const brsrc rw = make_rsrc(wl + (t == 0 ? kOffGate : kOffUp) + (size_t)(p0 + 1) * KSTEPS * 512, (size_t)KSTEPS * 1024);
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) {
        const int ks = ks0 + s2 < KSTEPS ? ks0 + s2 : KSTEPS - 1;
        buf_frag(w1[t][s2], rw, (ks * 512 + lane * 8) * 2);
      }
    }
  }
  // the items' shift . W^T columns (static within the launch), by the copy wave ahead of the polls
  if (wave == 3) {
    const float* bias = a.bias + slw * kBiasCols;
    const int pr = lane >> 5, c = lane & 31;
    s_bias[lane] = bias[kQkvCols + (c < 16 ? 0 : kMlp) + (p0 + pr) * 16 + (c & 15)];
  }
  PHASE_TS(s, l, PH, 1);
  if (!wait_flags(a, flag_base(a, s, l, kPhO), kOItems, sy)) return false;
  PHASE_TS(s, l, PH, 2);
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);  // pair p0: [tile t][k-step] fragments
  f32x4 acc[MT][NT];
  if (mw) {
    const brsrc rsrc_s = make_rsrc(ssin, (size_t)kTiles * R * 4);
    const brsrc rsrc_g = make_rsrc(gin, (size_t)R * kWidth * 2);
    float st[22];
#pragma unroll
    for (int t = 0; t < 22; ++t) {
      const int tile = 22 * cw + t;
      buf_f32(st[t], rsrc_s, tile < kTiles && lane < 32 ? ((tile * R + rb + lane) * 4) : kOob);
    }
    bf16x8 hr[MT][KSW];
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bool ok = r16 < nrow - mt * 16 && ks0 + s2 < KSTEPS;
        buf_frag(hr[mt][s2], rsrc_g, ok ? (int)((afrag_offset(2 * mh + mt, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
      }
    sched_fence();
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < 22; ++t) v += st[t];
    s_rs[cw * 64 + lane] = v;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    mfma_steps<KSW, NT, 0, MT, true>(acc, hr, [&](int t, int s2) {
      if (t >= 2) return w1[t - 2][s2];
      const int ksc = ks0 + s2 < KSTEPS ? ks0 + s2 : KSTEPS - 1;
      return *reinterpret_cast<const bf16x8*>(lw + ((size_t)t * KSTEPS + ksc) * 512 + lane * 8);
    });
  }
  PHASE_TS(s, l, PH, 4);
  __syncthreads();  // every wave is done with region A; the row sums are in LDS
  PHASE_TS(s, l, PH, 3);
  if (mw) store_wave_partials<MT, NT>(red, acc, cw, lane);
  if (tid < 32) s_rstd[tid] = 1.0f / sqrtf(fadd(((s_rs[tid] + s_rs[64 + tid]) + s_rs[128 + tid]) * (1.0f / kWidth), a.eps));
  __syncthreads();
  PHASE_TS(s, l, PH, 7);
  {
    // GeGLU as the fused reference kernel defines it: bf16(gelu_tanh(bf16(g)) * u), u the fp32
    // accumulator (rlinf_fused_denoise.py:166-173): columns ecol .. ecol + 3 of the pair's gate and
    // up tiles, row erow
    const int mt = (tid >> 6) & 1, pr = tid >> 7, eln = lane;
    const int erow = 16 * mt + (eln & 15), ecol = 4 * (eln >> 4);
    if (erow < nrow) {
      auto wave_sum = [&](int t) {
        f32x4 r[kCompWaves];
#pragma unroll
        for (int w = 0; w < kCompWaves; ++w) r[w] = *reinterpret_cast<const f32x4*>(red + (((size_t)(w * MT + mt) * NT + t) * 64 + eln) * 4);
        return (r[0] + r[1]) + r[2];
      };
      const f32x4 yg = wave_sum(2 * pr), yu = wave_sum(2 * pr + 1);
      const float rstd = s_rstd[erow];
      u16 o4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float gt = round_bf(__builtin_fmaf(rstd, yg[q], s_bias[pr * 32 + ecol + q]));
        const float up = __builtin_fmaf(rstd, yu[q], s_bias[pr * 32 + 16 + ecol + q]);
        o4[q] = f2bf(fmul(gelu_tanh(gt), up));
      }
      st_bf16x4(a.act + slw * (size_t)R * kMlp, afrag_index(rb + erow, (p0 + pr) * 16 + ecol, kMlp / 32), o4);
    }
  }
  PHASE_TS(s, l, PH, 5);
  publish(a, flag_base(a, s, l, PH) + item, sy.epoch, true);  // every wave stored rows
  PHASE_TS(s, l, PH, 6);
  return true;
}
static_assert(64 + 64 + 192 + 3 * 2 * 4 * 256 <= kWorkFloats, "one-sample gate_up working area");

// =============================================================================================
// qkv at B = 2 (kernel instance 1): two tile pairs (p0 = 2g from region A, p1 = 2g + 1 from
// registers) over row half mh for the samples [b0, b1) of sample half sh (see qkv_pair0), as
// gate_up's pair items do; both pairs are RoPE pairs (g < 36) or both v pairs.  The epilogue per
// pair is phase_qkv1's: bf16(rstd * acc + shift . W^T), then RoPE into the query rows or the
// action-key block, or the permuted V fragments.
// =============================================================================================
__device__ bool phase_qkv_pairs(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int NT = 4, KSW = 11, KSTEPS = kWidth / 32, TS = 33, MT = 2;
  const int L = a.depth, R = a.R;
  const int item = qkv_item();
  PHASE_TS(s, l, kPhQkv, 0);
  // copy wave: this phase's weights (region A) and everything issued before them have landed;
  // down(l) -> B here unless grouped attention stages K/V there (then at gate_up)
  if (copy_wave()) {
    wait_vmcnt<0>();
    if (!attn_grouped<true>(a)) copy_residual_w<kMlp / 32>(a, l, smem);
  }
  if (item < 0 || item >= kQkvItems) return true;
  const int grp = item % (kQkvPairs / 2), mh = (item / (kQkvPairs / 2)) % 2, sh = item / kQkvPairs;
  const int p0 = 2 * grp;
  const bool rotated = p0 < 72;
  const int rb = 32 * mh, nrow = MT * 16 < kHorizon - rb ? MT * 16 : kHorizon - rb;
  const int bh = (a.batch + 1) / 2, b0 = sh * bh, b1 = b0 + bh < a.batch ? b0 + bh : a.batch;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool comp = tid < kCompThreads;
  const int r16 = lane & 15;
  const int ks0 = wave * KSW;
  const size_t slw = (size_t)s * L + l;
  const u16* gin = a.g + slw * R * kWidth;
  const float* ssin = a.ss + ((size_t)s * (L + 1) + l) * kTiles * R;
  const float* bias = a.bias + slw * kBiasCols;
  // the pair's two tiles: RoPE pairs (head, d-tile dt) -> tiles head*16 + dt and + 8; v pairs ->
  // consecutive v tiles
  auto tile_of = [&](int p, int which) {
    const int t0 = p < 72 ? (p >> 3) * 16 + (p & 7) : 144 + 2 * (p - 72);
    return which == 0 ? t0 : (p < 72 ? t0 + 8 : t0 + 1);
  };
  float* s_rstd = smem + kLdsWork;  // [32] (item rows)
  float* s_bias = s_rstd + 64;      // [64] shift . W^T: pair p0 (tile 0, tile 1), pair p1 (tile 0, tile 1)
  float* s_rs = s_bias + 64;        // [3][64]
  float* red = s_rs + 192;          // [3 waves][MT][2][64 lanes][4] (one pair at a time)
  float* T = red + kCompWaves * MT * 2 * 256;  // [32][TS]
  // pair p1's weight fragments of this wave's k-steps (both tiles): waves 1 and 2 ahead of the
  // polls, wave 0 after them; wave 2's fragment of p0's tile 1 at k-step 31 (not in LDS)
  const u16* wq = a.wpack + (size_t)l * kLayerElems + kOffQkv;
  bf16x8 w1[2][KSW];
  auto load_w1 = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) {
        const int ks = ks0 + s2 < KSTEPS ? ks0 + s2 : KSTEPS - 1;  // the surplus step multiplies zeros
        w1[t][s2] = *reinterpret_cast<const bf16x8*>(wq + ((size_t)tile_of(p0 + 1, t) * KSTEPS + ks) * 512 + lane * 8);
      }
  };
  bf16x8 w31 = {};
  if (wave == 1 || wave == 2) load_w1();
  if (wave == 2) w31 = as_bf16x8(*reinterpret_cast<const u16x8*>(wq + ((size_t)tile_of(p0, 1) * KSTEPS + 31) * 512 + lane * 8));
  if (tid >= 64 && tid < 128) {
    const int c = tid - 64, pr = c >> 5, t = (c >> 4) & 1, n = c & 15;
    s_bias[c] = bias[tile_of(p0 + pr, t) * 16 + n];
  }
  PHASE_TS(s, l, kPhQkv, 1);
  {
    const unsigned* dep = l == 0 ? flag_base(a, s, 0, kPhIo) : flag_base(a, s, l - 1, kPhDown);
    const int ndep = l == 0 ? a.batch * kHorizon : kKSplit * kTiles;  // down_proj_pairs: one flag per (group, quarter)
    if (!wait_flags(a, dep, ndep, sy)) return false;
  }
  PHASE_TS(s, l, kPhQkv, 2);
  if (wave == 0) load_w1();
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);  // pair p0: [tile t][k-step] fragments
  const int et = tid - 64;  // RoPE epilogue thread: item row et/2, half et%2
  const bool rope_thread = rotated && et >= 0 && et < 2 * nrow;
  for (int b = b0; b < b1; ++b) {
    const int m0 = b * kRowsPerSample;
    f32x4 acc[MT][NT];
    if (comp) {
      const brsrc rsrc_s = make_rsrc(ssin, (size_t)kTiles * R * 4);
      const brsrc rsrc_g = make_rsrc(gin, (size_t)R * kWidth * 2);
      float st[22];
#pragma unroll
      for (int t = 0; t < 22; ++t) {
        const int tile = 22 * wave + t;
        buf_f32(st[t], rsrc_s, tile < kTiles && lane < 16 * MT ? ((tile * R + m0 + rb + lane) * 4) : kOob);
      }
      bf16x8 hr[MT][KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bool ok = r16 < nrow - mt * 16 && ks0 + s2 < KSTEPS;
          buf_frag(hr[mt][s2], rsrc_g, ok ? (int)((afrag_offset(b * 4 + 2 * mh + mt, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
        }
      sched_fence();
      float v = 0.f;
#pragma unroll
      for (int t = 0; t < 22; ++t) v += st[t];
      s_rs[wave * 64 + lane] = v;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      mfma_steps<KSW, NT, 0, MT>(acc, hr, [&](int t, int s2) {
        if (t >= 2) return w1[t - 2][s2];
        const int ksc = ks0 + s2 < KSTEPS ? ks0 + s2 : KSTEPS - 1;
        if (t == 1 && s2 >= KSTEPS - 1 - 2 * KSW && wave == 2) return w31;
        return *reinterpret_cast<const bf16x8*>(lw + ((size_t)t * KSTEPS + ksc) * 512 + lane * 8);
      });
    }
    __syncthreads();  // the row sums are in LDS
    if (tid < 16 * MT) s_rstd[tid] = 1.0f / sqrtf(fadd(((s_rs[tid] + s_rs[64 + tid]) + s_rs[128 + tid]) * (1.0f / kWidth), a.eps));
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      if (comp) {
        f32x4 accp[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) accp[mt][0] = acc[mt][2 * pr], accp[mt][1] = acc[mt][2 * pr + 1];
        store_wave_partials<MT, 2>(red, accp, wave, lane);
      }
      __syncthreads();
      reduce_to_tile<MT, 2, TS>(red, T);
      __syncthreads();
      const int p = p0 + pr, tile0 = tile_of(p, 0);
      if (rotated) {
        // (x*cos) + (rotate_half(x)*sin) as phase_qkv1's RoPE epilogue (rlinf_fused_denoise.py:264-278)
        if (rope_thread) {
          const int head = p >> 3, dt = p & 7;
          const int row = et >> 1, half = et & 1;
          const size_t cr = (size_t)(b * kHorizon + rb + row) * kHeadDim + dt * 16 + half * 8;
          const u16x8 cs_lo = *reinterpret_cast<const u16x8*>(a.cos_tab + cr), sn_lo = *reinterpret_cast<const u16x8*>(a.sin_tab + cr);
          const u16x8 cs_hi = *reinterpret_cast<const u16x8*>(a.cos_tab + cr + kHalfDim), sn_hi = *reinterpret_cast<const u16x8*>(a.sin_tab + cr + kHalfDim);
          const float rstd = s_rstd[row];
          float tl[8], th[8], bl[8], bhh[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            tl[q] = T[row * TS + half * 8 + q];
            th[q] = T[row * TS + 16 + half * 8 + q];
            bl[q] = s_bias[32 * pr + half * 8 + q];
            bhh[q] = s_bias[32 * pr + 16 + half * 8 + q];
          }
          sched_fence();
          u16 olo[8], ohi[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float x_lo = round_bf(__builtin_fmaf(rstd, tl[q], bl[q]));
            const float x_hi = round_bf(__builtin_fmaf(rstd, th[q], bhh[q]));
            olo[q] = f2bf(fsub(fmul(x_lo, bf2f(cs_lo[q])), fmul(x_hi, bf2f(sn_lo[q]))));
            ohi[q] = f2bf(fadd(fmul(x_hi, bf2f(cs_hi[q])), fmul(x_lo, bf2f(sn_hi[q]))));
          }
          const int d = dt * 16 + half * 8;
          if (head < kHeads) {
            u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
            const int qrow = (m0 + rb + row) * kQRowsPerTok + head;
            st_bf16x8(qs, afrag_index(qrow, d, kHeadDim / 32), olo);
            st_bf16x8(qs, afrag_index(qrow, d + kHalfDim, kHeadDim / 32), ohi);
          } else {
            u16* kc = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
            st_bf16x8(kc, kfrag_index(rb + row, d), olo);
            st_bf16x8(kc, kfrag_index(rb + row, d + kHalfDim), ohi);
          }
        }
      } else if (comp) {
        // v: chunk -> (dim dcol of the tile pair, key group (kb, g) of the permuted V fragment);
        // this item's rows are the keys of 32-key block kb = mh
        for (int ci = tid; ci < 128; ci += kCompThreads) {
          const int dcol = ci & 31, kb = mh, gg = ci >> 5;
          u16 v8[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int key = vkey(kb, gg, q);
            v8[q] = key < kHorizon ? f2bf(__builtin_fmaf(s_rstd[key - rb], T[(key - rb) * TS + dcol], s_bias[32 * pr + dcol])) : (u16)0;
          }
          const int dv = (tile0 - 144) * 16 + dcol;
          u16* vc = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
          st_bf16x8(vc, ((size_t)kb * 16 + (dv >> 4)) * 512 + (size_t)(gg * 16 + (dv & 15)) * 8, v8);
        }
      }
      __syncthreads();  // red and T are reused
    }
  }
  PHASE_TS(s, l, kPhQkv, 5);
  publish(a, flag_base(a, s, l, kPhQkv) + item, sy.epoch);
  PHASE_TS(s, l, kPhQkv, 6);
  return true;
}

// Row-split GEMM phases (kernel instance 2): A chunks of kGuCk k-steps x 4 m-tiles.
constexpr int kGuCk = 4;                     // k-steps per A chunk
constexpr int kGuChunks = kWidth / 32 / kGuCk;  // 8 chunks per sample
// chunks in flight ahead of the MFMAs (ring of 4).  One: measured on MI355X, a second chunk in
// flight made every row-split phase slower (the vector-memory instruction stream of the CU, not
// the latency, is what these phases wait on)
constexpr int kGuAhead = 1;
static_assert(kGuAhead >= 1 && kGuAhead <= 3, "the ring holds the current chunk and kGuAhead more");
// Grouped attention (attn_group_items): 32-key K/V blocks staged this many ahead of the one
// being attended, in a ring of kAttnRing LDS buffers.
constexpr int kAttnAhead = 1;  // blocks staged ahead of the one being attended
constexpr int kAttnRing = kAttnAhead + 1;
static_assert(kAttnAhead == 1 || kAttnAhead == 2, "ring of two or three buffers");
// chunk c of sample b (4 m-tiles x kGuCk k-steps) -> A; padded rows and absent samples read zeros
// (NKS: k-steps of the activation rows; KS0: the first k-step of chunk 0.)  M-tiles 0..2 take one
// load per k-step; m-tile 3 holds 2 rows (48, 49), so one load brings the whole chunk's: lane
// 16 kc + 2 s2 + r gets row 48 + r, k-step s2, k-range kc -> A[3][0], which gu_mfma_chunk spreads
// to the fragment lanes (16 kc + r) with a row shift per k-step.  The fragments' other lanes of
// m-tile 3 then hold other rows' data: they are rows 50..63, whose products no phase stores.
static_assert(kHorizon == 3 * 16 + 2, "m-tile 3 holds rows 48 and 49");
template <int NKS = kWidth / 32>
__device__ __forceinline__ void gu_load_chunk(bf16x8 (&A)[4][kGuCk], brsrc rg, int b, bool ok_b, int c, int lane, int ks0 = 0) {
  const int r16 = lane & 15;
#pragma unroll
  for (int s2 = 0; s2 < kGuCk; ++s2)
#pragma unroll
    for (int mt = 0; mt < 3; ++mt) {
      const bool ok = ok_b && r16 < kHorizon - mt * 16;
      buf_frag(A[mt][s2], rg, ok ? (int)((afrag_offset(b * 4 + mt, ks0 + c * kGuCk + s2, NKS) + lane * 8) * 2) : kOob);
    }
  const int s2 = r16 >> 1, r = r16 & 1, kc = lane >> 4;
  const bool ok = ok_b && r16 < 2 * kGuCk;
  buf_frag(A[3][0], rg, ok ? (int)((afrag_offset(b * 4 + 3, ks0 + c * kGuCk + s2, NKS) + (16 * kc + r) * 8) * 2) : kOob);
}
// Row statistics of the row-split phases, 16-byte loads: lane (j = lane % 16, q = lane / 16)
// loads the tile sums of squares of rows 4j .. 4j+3 for tile 16 q + t (t = 0 .. 15, in order);
// row_rstd adds the four tile groups across lanes and returns lane r's row rstd.
__device__ __forceinline__ float4 row_stats4(brsrc rs, int R, int b, int t, int lane) {
  const int j = lane & 15, q = lane >> 4;
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((16 * q + t) * R + b * kRowsPerSample + 4 * j) * 4, 0, 0));
}
__device__ __forceinline__ float row_rstd(float4 s, int lane, float eps) {
  float r4[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) r4[i] = 1.0f / sqrtf(fadd(lane_sum_xor32(lane_sum_xor16(r4[i])) * (1.0f / kWidth), eps));
  // row `lane` is component lane % 4 of lane lane / 4
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = __shfl(r4[i], lane >> 2);
    r = (lane & 3) == i ? v : r;
  }
  return r;
}
// v moved up by N lanes within each row of 16 (DPP row_shl: lane i takes lane i + N of its row)
template <int N>
__device__ __forceinline__ bf16x8 frag_row_shl(bf16x8 v) {
  if constexpr (N == 0) {
    return v;
  } else {
    const u32x4 x = __builtin_bit_cast(u32x4, v);
    u32x4 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x[i], 0x100 + N, 0xf, 0xf, false);
    return __builtin_bit_cast(bf16x8, y);
  }
}
template <int S2>
__device__ __forceinline__ bf16x8 mtile3_frag(const bf16x8 (&A)[4][kGuCk]) {
  return frag_row_shl<2 * S2>(A[3][0]);
}
// the products of chunk c with the two weight tiles in region A (lw: tile 0, then tile 1, 32
// fragments each); LAST1: tile 1's last k-step comes from the register w1_last instead
template <bool LAST1 = false>
__device__ __forceinline__ void gu_mfma_chunk(f32x4 (&accg)[4], f32x4 (&accu)[4], const bf16x8 (&A)[4][kGuCk], const u16* lw, int c,
                                              int lane, bf16x8 w1_last = {}) {
  constexpr int KSTEPS = kWidth / 32;
#pragma unroll
  for (int s2 = 0; s2 < kGuCk; ++s2) {
    const int ks = c * kGuCk + s2;
    const bf16x8 wg = *reinterpret_cast<const bf16x8*>(lw + (size_t)ks * 512 + lane * 8);
    const bf16x8 wu = LAST1 && s2 == kGuCk - 1 && c == kGuChunks - 1
                          ? w1_last
                          : *reinterpret_cast<const bf16x8*>(lw + ((size_t)KSTEPS + ks) * 512 + lane * 8);
    const bf16x8 a3 = s2 == 0 ? mtile3_frag<0>(A) : s2 == 1 ? mtile3_frag<1>(A) : s2 == 2 ? mtile3_frag<2>(A) : mtile3_frag<3>(A);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const bf16x8 am = mt < 3 ? A[mt][s2] : a3;
      accg[mt] = mfma16x16x32(wg, am, accg[mt]);
      accu[mt] = mfma16x16x32(wu, am, accu[mt]);
    }
  }
}

// =============================================================================================
// qkv of kernel instance 2, split by rows as phase_gateup_msplit: item i = tile pair i mod 80 (a
// RoPE pair of q or k tiles, or two consecutive v tiles) for sample third i / 80 (240 items on
// workgroups 16..255); region A holds
// the pair's two tiles except the second one's last k-step (the 63-copy burst leaves it out),
// which every wave loads into a register.  Wave j takes sample j of the third (j + 4, ... past 12
// samples): all four m-tiles over the whole K, A streamed one chunk ahead.  As W.A^T, a lane
// ends with columns 4g .. 4g+3 of both tiles for one row, so the RoPE rotation (which pairs
// column d of the first tile with column d of the second) and the 8-byte q / k stores are
// lane-local; v rows go through a per-wave LDS tile into the permuted V fragment layout.
// =============================================================================================
__device__ bool phase_qkv_msplit(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kWidth / 32;
  const int L = a.depth, R = a.R;
  const int item = qkv_item_of<true>();
  PHASE_TS(s, l, kPhQkv, 0);
  // copy wave: this phase's weights (region A) and everything issued before them have landed;
  // down(l) -> B here unless grouped attention stages K/V there (a ring of three; then before
  // o_proj)
  if (copy_wave()) {
    wait_vmcnt<0>();
    if (kAttnRing < 3 || !attn_grouped<true>(a)) copy_residual_w<kMlp / 32>(a, l, smem);
  }
  if (item < 0 || item >= kQkvItemsRS) return true;
  const int p = item % kQkvPairs, sg = item / kQkvPairs;
  const bool rotated = p < 72;
  const int bt = (a.batch + 2) / 3, b0 = sg * bt, b1 = b0 + bt < a.batch ? b0 + bt : a.batch;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const size_t slw = (size_t)s * L + l;
  const int t0 = rotated ? (p >> 3) * 16 + (p & 7) : 144 + 2 * (p - 72);
  const int t1 = rotated ? t0 + 8 : t0 + 1;
  const u16* wq = a.wpack + (size_t)l * kLayerElems + kOffQkv;
  const bf16x8 w1_last = load_frag(wq + ((size_t)t1 * KSTEPS + KSTEPS - 1) * 512 + lane * 8);
  // shift . W^T of this lane's columns 4g .. 4g+3 of both tiles
  const float* bias = a.bias + slw * kBiasCols;
  float bv0[4], bv1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bv0[i] = bias[t0 * 16 + 4 * g + i];
    bv1[i] = bias[t1 * 16 + 4 * g + i];
  }
  PHASE_TS(s, l, kPhQkv, 1);
  {
    const unsigned* dep = l == 0 ? flag_base(a, s, 0, kPhIo) : flag_base(a, s, l - 1, kPhDown);
    const int ndep = l == 0 ? a.batch * kHorizon : kKSplit * kTiles;  // down_proj_pairs: one flag per (group, quarter)
    if (!wait_flags(a, dep, ndep, sy)) return false;
  }
  PHASE_TS(s, l, kPhQkv, 2);
  const brsrc rg = make_rsrc(a.g + slw * R * kWidth, (size_t)R * kWidth * 2);
  const brsrc rs = make_rsrc(a.ss + ((size_t)s * (L + 1) + l) * kTiles * R, (size_t)kTiles * R * 4);
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);
  u16* s_v = reinterpret_cast<u16*>(smem + kLdsWork) + wave * 64 * 32;  // v items: [64 keys][32 dims]
  const int rope_d = (p & 7) * 16 + 4 * g;  // RoPE items: the lane's first column of the low tile
  const brsrc rcos = make_rsrc(a.cos_tab, (size_t)a.batch * kHorizon * kHeadDim * 2);
  const brsrc rsin = make_rsrc(a.sin_tab, (size_t)a.batch * kHorizon * kHeadDim * 2);
  bf16x8 A[4][4][kGuCk];  // [ring slot = chunk mod 4][m-tile][k-step]
  const int bf = b0 + wave;
#pragma unroll
  for (int c = 0; c < kGuAhead; ++c) gu_load_chunk(A[c], rg, bf, bf < b1, c, lane);
  sched_fence();
  for (int b = bf; b < b1; b += 4) {
    const int bn = b + 4;
    const bool ok_n = bn < b1;
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc0[mt] = acc1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float4 st[4][4];
    float4 ss4 = {0.f, 0.f, 0.f, 0.f};
    u32x2 cst[4][4];  // RoPE: [m-tile][cos lo, sin lo, cos hi, sin hi] of the lane's row, columns d .. d+3
#pragma unroll
    for (int c = 0; c < kGuChunks; ++c) {
      if (c + kGuAhead < kGuChunks) gu_load_chunk(A[(c + kGuAhead) % 4], rg, b, true, c + kGuAhead, lane);
      else gu_load_chunk(A[(c + kGuAhead) % 4], rg, bn, ok_n, c + kGuAhead - kGuChunks, lane);
      if (c < 4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) st[c][t] = row_stats4(rs, R, b, 4 * c + t, lane);
      }
      if (c == 4 && rotated) {
        // the epilogue's cos / sin, loaded here so that their latency hides behind the MFMAs
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int row = mt * 16 + r16;
          const bool ok = row < kHorizon;
          const int lo = ok ? (int)(((size_t)(b * kHorizon + row) * kHeadDim + rope_d) * 2) : kOob;
          const int hi = ok ? lo + kHalfDim * 2 : kOob;
          cst[mt][0] = __builtin_amdgcn_raw_buffer_load_b64(rcos, lo, 0, 0);
          cst[mt][1] = __builtin_amdgcn_raw_buffer_load_b64(rsin, lo, 0, 0);
          cst[mt][2] = __builtin_amdgcn_raw_buffer_load_b64(rcos, hi, 0, 0);
          cst[mt][3] = __builtin_amdgcn_raw_buffer_load_b64(rsin, hi, 0, 0);
        }
      }
      sched_fence();
      gu_mfma_chunk<true>(acc0, acc1, A[c % 4], lw, c, lane, w1_last);
      if (c >= 1 && c <= 4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) ss4 += st[c - 1][t];
      }
    }
    const float rstd_lane = row_rstd(ss4, lane, a.eps);
    if (rotated) {
      // (x*cos) + (rotate_half(x)*sin) as phase_qkv1's RoPE epilogue (rlinf_fused_denoise.py:264-278)
      const int head = p >> 3, d = rope_d;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = mt * 16 + r16;
        const float rstd = __shfl(rstd_lane, row);
        if (row < kHorizon) {
          const u16x4 cs_lo = __builtin_bit_cast(u16x4, cst[mt][0]), sn_lo = __builtin_bit_cast(u16x4, cst[mt][1]);
          const u16x4 cs_hi = __builtin_bit_cast(u16x4, cst[mt][2]), sn_hi = __builtin_bit_cast(u16x4, cst[mt][3]);
          u16 olo[4], ohi[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x_lo = round_bf(__builtin_fmaf(rstd, acc0[mt][i], bv0[i]));
            const float x_hi = round_bf(__builtin_fmaf(rstd, acc1[mt][i], bv1[i]));
            olo[i] = f2bf(fsub(fmul(x_lo, bf2f(cs_lo[i])), fmul(x_hi, bf2f(sn_lo[i]))));
            ohi[i] = f2bf(fadd(fmul(x_hi, bf2f(cs_hi[i])), fmul(x_lo, bf2f(sn_hi[i]))));
          }
          const uint32_t lo0 = (uint32_t)olo[0] | ((uint32_t)olo[1] << 16), lo1 = (uint32_t)olo[2] | ((uint32_t)olo[3] << 16);
          const uint32_t hi0 = (uint32_t)ohi[0] | ((uint32_t)ohi[1] << 16), hi1 = (uint32_t)ohi[2] | ((uint32_t)ohi[3] << 16);
          if (head < kHeads) {
            u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
            const int qrow = (b * kRowsPerSample + row) * kQRowsPerTok + head;
            st_wt8(qs, (uint32_t)(afrag_index(qrow, d, kHeadDim / 32) * 2), lo0, lo1);
            st_wt8(qs, (uint32_t)(afrag_index(qrow, d + kHalfDim, kHeadDim / 32) * 2), hi0, hi1);
          } else {
            u16* kc = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
            st_wt8(kc, (uint32_t)(kfrag_index(row, d) * 2), lo0, lo1);
            st_wt8(kc, (uint32_t)(kfrag_index(row, d + kHalfDim) * 2), hi0, hi1);
          }
        }
      }
    } else {
      // v: the wave's rows into its LDS tile (keys past the horizon as zeros), then chunk ci of
      // the 256 (block kb, key group gg, dim dcol) -> 8 keys of one dim of the permuted fragment
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = mt * 16 + r16;
        const float rstd = __shfl(rstd_lane, row);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s_v[row * 32 + 4 * g + i] = row < kHorizon ? f2bf(__builtin_fmaf(rstd, acc0[mt][i], bv0[i])) : (u16)0;
          s_v[row * 32 + 16 + 4 * g + i] = row < kHorizon ? f2bf(__builtin_fmaf(rstd, acc1[mt][i], bv1[i])) : (u16)0;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS writes are done
      u16* vc = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ci = lane + 64 * k, dcol = ci & 31, kb = ci >> 7, gg = (ci >> 5) & 3;
        u16 v8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v8[q] = s_v[vkey(kb, gg, q) * 32 + dcol];
        const int dv = (t0 - 144) * 16 + dcol;
        st_bf16x8(vc, ((size_t)kb * 16 + (dv >> 4)) * 512 + (size_t)(gg * 16 + (dv & 15)) * 8, v8);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the tile's reads are done before the next sample's writes
    }
  }
  PHASE_TS(s, l, kPhQkv, 5);
  publish(a, flag_base(a, s, l, kPhQkv) + item, sy.epoch, true);  // every wave stored rows
  PHASE_TS(s, l, kPhQkv, 6);
  return true;
}

// =============================================================================================
// gate_up at B = 2 (kernel instance 1): item w computes gate/up tile pairs 2g and 2g + 1,
// g = w mod 128 (pair 2g from region A, 2g + 1 from registers), for sample half w / 128 (see
// gu_pair0), with the copy wave as a fourth compute wave (its down_proj copy is issued before
// o_proj instead): K splits 8 k-steps per wave, so a sample's 48 loads per wave stay under the 63
// a wave may have in flight and each wave runs 128 MFMAs per sample instead of 176 (three waves);
// the four partials are added in wave order.
// =============================================================================================
__device__ bool phase_gateup_pairs4(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int NW = 4, NT = 4, KSW = 8, KSTEPS = kWidth / 32, TS = 33, MT = 4, TPW = kTiles / NW;
  const int L = a.depth, R = a.R;
  const int item = wg_id();
  PHASE_TS(s, l, kPhGu, 0);
  // copy wave: pair p0's weights (region A) and everything issued before them have landed
  if (copy_wave()) wait_vmcnt<0>();
  const int half = item / (kGuItems / 2), p0 = gu_pair0(a), p1 = p0 + 1;
  const int bh = (a.batch + 1) / 2, b0 = half * bh, b1 = b0 + bh < a.batch ? b0 + bh : a.batch;
  if (item >= kGuItems) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15;
  const int ks0 = wave * KSW;
  const size_t slw = (size_t)s * L + l;
  const u16* gin = a.gmid + slw * R * kWidth;
  const float* ssin = a.ssmid + slw * kTiles * R;
  const float* bias = a.bias + slw * kBiasCols;
  float* s_rstd = smem + kLdsWork;  // [64] (sample rows)
  float* s_bias = s_rstd + 64;      // [64] shift . W^T: gate p0, up p0, gate p1, up p1 (16 each)
  float* s_rs = s_bias + 64;        // [4][64]
  float* red = s_rs + 256;          // [4 waves][4 m-tiles][2 tiles][64 lanes][4] (one pair at a time)
  float* T = red + NW * MT * 2 * 256;  // [64][TS]
  const u16* wl = a.wpack + (size_t)l * kLayerElems;
  bf16x8 w1[2][KSW];
  auto load_w1 = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2)
        w1[t][s2] = *reinterpret_cast<const bf16x8*>(wl + (t == 0 ? kOffGate : kOffUp) + ((size_t)p1 * KSTEPS + ks0 + s2) * 512 + lane * 8);
  };
  if (wave != 0) load_w1();
  if (tid >= 64 && tid < 128) {
    const int c = tid - 64, pr = c >> 5, gu = (c >> 4) & 1, n = c & 15;
    s_bias[c] = bias[kQkvCols + gu * kMlp + (p0 + pr) * 16 + n];
  }
  PHASE_TS(s, l, kPhGu, 1);
  if (!wait_flags(a, flag_base(a, s, l, kPhO), kOItems, sy)) return false;
  PHASE_TS(s, l, kPhGu, 2);
  if (wave == 0) load_w1();
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);  // pair p0: [tile t][k-step] fragments
  for (int b = b0; b < b1; ++b) {
    const int m0 = b * kRowsPerSample;
    f32x4 acc[MT][NT];
    {
      const brsrc rsrc_s = make_rsrc(ssin, (size_t)kTiles * R * 4);
      const brsrc rsrc_g = make_rsrc(gin, (size_t)R * kWidth * 2);
      float st[TPW];
#pragma unroll
      for (int t = 0; t < TPW; ++t) buf_f32(st[t], rsrc_s, ((TPW * wave + t) * R + m0 + lane) * 4);
      bf16x8 hr[MT][KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          buf_frag(hr[mt][s2], rsrc_g, r16 < kHorizon - mt * 16 ? (int)((afrag_offset(b * 4 + mt, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
      sched_fence();
      float v = 0.f;
#pragma unroll
      for (int t = 0; t < TPW; ++t) v += st[t];
      s_rs[wave * 64 + lane] = v;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      mfma_steps<KSW, NT, 0, MT>(acc, hr, [&](int t, int s2) {
        if (t >= 2) return w1[t - 2][s2];
        return *reinterpret_cast<const bf16x8*>(lw + ((size_t)t * KSTEPS + ks0 + s2) * 512 + lane * 8);
      });
    }
    __syncthreads();  // the row sums are in LDS
    if (tid < 64) s_rstd[tid] = 1.0f / sqrtf(fadd((((s_rs[tid] + s_rs[64 + tid]) + s_rs[128 + tid]) + s_rs[192 + tid]) * (1.0f / kWidth), a.eps));
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      f32x4 accp[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) accp[mt][0] = acc[mt][2 * pr], accp[mt][1] = acc[mt][2 * pr + 1];
      store_wave_partials<MT, 2>(red, accp, wave, lane);
      __syncthreads();
      reduce_to_tile_n<NW, MT, 2, TS>(red, T);
      __syncthreads();
      // GeGLU (rlinf_fused_denoise.py:166-173) of pair p0 + pr; chunk = (row, half of 16 columns)
      if (tid < 2 * kHorizon) {
        const int row = tid >> 1, hf = tid & 1;
        const float rstd = s_rstd[row];
        float tg[8], tu[8], bgv[8], buv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          tg[q] = T[row * TS + hf * 8 + q];
          tu[q] = T[row * TS + 16 + hf * 8 + q];
          bgv[q] = s_bias[32 * pr + hf * 8 + q];
          buv[q] = s_bias[32 * pr + 16 + hf * 8 + q];
        }
        sched_fence();
        u16 o8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float gt = round_bf(__builtin_fmaf(rstd, tg[q], bgv[q]));
          const float up = __builtin_fmaf(rstd, tu[q], buv[q]);
          o8[q] = f2bf(fmul(gelu_tanh(gt), up));
        }
        st_bf16x8(a.act + slw * (size_t)R * kMlp, afrag_index(m0 + row, (p0 + pr) * 16 + hf * 8, kMlp / 32), o8);
      }
      __syncthreads();  // red and T are reused
    }
  }
  PHASE_TS(s, l, kPhGu, 5);
  publish(a, flag_base(a, s, l, kPhGu) + item, sy.epoch);
  PHASE_TS(s, l, kPhGu, 6);
  return true;
}
static_assert(64 + 64 + 256 + 4 * 4 * 2 * 256 + 64 * 33 <= kWorkFloatsBatched, "batched gate_up working area");

// =============================================================================================
// gate_up of kernel instance 2 (B >= 3), split by rows: item w = gate|up tile pair w for every
// sample; region A holds its two tiles (gate, up: 32 k-steps each).  Wave j takes samples j,
// j + 4, ...: for each, all four m-tiles over the whole K, so no partial sum crosses waves and the
// waves never wait for each other.  The A fragments stream from L2 in chunks of 4 k-steps, two
// chunks ahead of the MFMAs (into the next sample's first chunks at the end of a sample); the
// products are formed as W.A^T, so a lane ends with 4 consecutive columns of one row and its
// GeGLU and 8-byte stores need nothing from other lanes.  Lane r (= row r of the sample) sums its
// row's 64 tile sums of squares in four groups of 16, loaded during the first four chunks.
// =============================================================================================
__device__ bool phase_gateup_msplit(KArgs& a, int s, int l, float* smem, Sync sy) {
  const int L = a.depth, R = a.R;
  const int item = wg_id();
  PHASE_TS(s, l, kPhGu, 0);
  // copy wave: the pair's weights (region A) and everything issued before them have landed; then
  // down_proj's second tile into the working area (free from here to down_proj)
  if (copy_wave()) wait_vmcnt<0>();
  copy_down_w1(a, l, smem);
  if (item >= kGuItems) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const size_t slw = (size_t)s * L + l;
  const float* bias = a.bias + slw * kBiasCols;
  // shift . W^T of this lane's columns 4g .. 4g+3 of the gate and up tiles
  float bgv[4], buv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bgv[i] = bias[kQkvCols + item * 16 + 4 * g + i];
    buv[i] = bias[kQkvCols + kMlp + item * 16 + 4 * g + i];
  }
  PHASE_TS(s, l, kPhGu, 1);
  if (!wait_flags(a, flag_base(a, s, l, kPhO), kOItems, sy)) return false;
  PHASE_TS(s, l, kPhGu, 2);
  const brsrc rg = make_rsrc(a.gmid + slw * R * kWidth, (size_t)R * kWidth * 2);
  const brsrc rs = make_rsrc(a.ssmid + slw * kTiles * R, (size_t)kTiles * R * 4);
  u16* act = a.act + slw * (size_t)R * kMlp;
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsA);
  bf16x8 A[4][4][kGuCk];  // [ring slot = chunk mod 4][m-tile][k-step]
#pragma unroll
  for (int c = 0; c < kGuAhead; ++c) gu_load_chunk(A[c], rg, wave, wave < a.batch, c, lane);
  sched_fence();
  for (int b = wave; b < a.batch; b += 4) {
    const int bn = b + 4;
    const bool ok_n = bn < a.batch;
    f32x4 accg[4], accu[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) accg[mt] = accu[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float4 st[4][4];
    float4 ss4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kGuChunks; ++c) {
      // kGuAhead chunks ahead: this sample's, then the next sample's first ones
      if (c + kGuAhead < kGuChunks) gu_load_chunk(A[(c + kGuAhead) % 4], rg, b, true, c + kGuAhead, lane);
      else gu_load_chunk(A[(c + kGuAhead) % 4], rg, bn, ok_n, c + kGuAhead - kGuChunks, lane);
      if (c < 4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) st[c][t] = row_stats4(rs, R, b, 4 * c + t, lane);
      }
      sched_fence();
      gu_mfma_chunk(accg, accu, A[c % 4], lw, c, lane);
      if (c >= 1 && c <= 4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) ss4 += st[c - 1][t];
      }
    }
    // lane r's row r: rstd of adaRMSNorm (the same grouping as the one-sample phases)
    const float rstd_lane = row_rstd(ss4, lane, a.eps);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = mt * 16 + r16;
      const float rstd = __shfl(rstd_lane, row);
      if (row < kHorizon) {
        u16 o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // GeGLU (rlinf_fused_denoise.py:166-173)
          const float gt = round_bf(__builtin_fmaf(rstd, accg[mt][i], bgv[i]));
          const float up = __builtin_fmaf(rstd, accu[mt][i], buv[i]);
          o4[i] = f2bf(fmul(gelu_tanh(gt), up));
        }
        st_wt8(act, (uint32_t)(afrag_index(b * kRowsPerSample + row, item * 16 + 4 * g, kMlp / 32) * 2),
               (uint32_t)o4[0] | ((uint32_t)o4[1] << 16), (uint32_t)o4[2] | ((uint32_t)o4[3] << 16));
      }
    }
  }
  PHASE_TS(s, l, kPhGu, 5);
  publish(a, flag_base(a, s, l, kPhGu) + item, sy.epoch, true);  // every wave stored rows
  PHASE_TS(s, l, kPhGu, 6);
  return true;
}

// =============================================================================================
// attention, two stages.
// Splits: item = (row block bp of 2 tokens x 8 heads of one sample, key split c); compute wave w
// attends 32-key blocks kb_lo + w, kb_lo + w + 3, ... (online softmax).  Each wave's first block,
// if from the static prefix, is loaded into its registers before the wait; wave 0's second block
// (kb_lo + 3) is staged in LDS by the copy wave.  The waves are merged in LDS and the compute
// waves store the split's partial (O unnormalised, running max, running sum).  Keys [0, s_pre)
// come from the static prefix cache, keys [s_pre, s_pre + 64) from this step's action-key block.
// Merges: role = (row block bp, head pair hp): the 4 rows of heads 2hp, 2hp+1 are merged over the
// splits in fixed order and stored as o_proj's A operand; o_proj's K quarter hp needs exactly
// these rows.
// =============================================================================================
// One 32-key block with the query fragments read from LDS (sq: 8 fragments, 1 KiB each).
__device__ __forceinline__ void attend_block_lds(const KvBlock& blk, const u16* sq, int lane, float& m_run, float& l_run,
                                                 f32x4 (&oacc)[16]) {
  attend_block_q(blk, [&](int ds) { return *reinterpret_cast<const bf16x8*>(sq + ds * 512 + lane * 8); }, m_run, l_run, oacc);
}


typedef uint32_t u32x4_lds __attribute__((ext_vector_type(4)));
// One 16-byte LDS read issued as inline asm (ds_read_b128 at byte address addr); the caller waits
// for it with lds_reads_done.  The grouped attention reads its staged K/V blocks this way because
// the compiler cannot tell the two stage buffers apart and would otherwise wait for the next
// block's direct-to-LDS loads (vmcnt(0)) before reading the current one.
__device__ __forceinline__ u32x4_lds lds_read16(uint32_t addr) {
  u32x4_lds r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
// s_waitcnt lgkmcnt(0), then the N fragments `f` as in/out operands, so nothing that uses them
// is scheduled before the wait.
template <int N>
__device__ __forceinline__ void lds_reads_done(u32x4_lds (&f)[N], uint32_t& w0, uint32_t& w1) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(f[i]));
  asm volatile("" : "+v"(w0), "+v"(w1));
}
__device__ __forceinline__ uint32_t lds_read4(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}

// Grouped split items (batches of kAttnGroupMinBatch and more): item n = (sample n mod B, group
// grp of kAttnGroup two-token row blocks, key split c); wave j (the copy wave included) attends row
// block kAttnGroup * grp + j over the split's whole key range.  Every 32-key K/V block is staged
// once in LDS for the four waves (direct-to-LDS loads, 8 of its 32 fragments per wave, and its 32
// key-valid bytes by wave 0) in a ring of kAttnRing buffers -- the upper half of region A (free
// during attention), the working area and, for a third, region B (down_proj's weights are then
// copied there at o_proj, else at qkv) -- kAttnAhead blocks ahead of the one being attended: one, measured on MI355X
// (a second block in flight made batches of 8 0.5 % and of 4, 5 1.1 % slower: the fewer vector-memory
// instructions in flight, the sooner the ones waited for complete).  An item thus reads each block from L2
// once for 64 query rows instead of once per 16 (at B = 8 the splits' K/V delivery drops from 200
// MiB to 56 MiB per layer).  Everything the block loop waits for is staged through LDS and read
// with inline ds_reads: a global load waited for there would, loads completing in order, also wait
// for the later blocks' copies.  Each wave stores its row block's partial exactly as a split item
// does after its wave merge, so the merges are unchanged.  With 256 workgroups, item n runs on
// workgroup n: sample n mod B on XCD n mod 8 (at B = 8 all of a sample's items share the XCD whose
// L2 holds that sample's K/V).
// This wave's share of one K/V block's staging (see attn_group_items): fragments 8 (wave & 1) .. +7
// of the block's K (waves 0, 1) or V (waves 2, 3) -> dst + wave * 8 KiB, and for wave 0 the
// block's 32 key-valid bytes -> vdst.
__device__ __forceinline__ void attn_stage(const u16* pre_src, const u16* suf_src, const uint8_t* valid, int nkb_pre, int kb,
                                           u16* dst, float* vdst, int wave, int lane) {
  const bool pre = kb < nkb_pre;
  const u16* src = (pre ? pre_src : suf_src) + (size_t)(pre ? kb : kb - nkb_pre) * 16 * 512 + (size_t)(wave & 1) * 8 * 512;
  const brsrc r = make_rsrc(uniform_ptr(src), 8 * 1024);
  lds_u16* d = lds_addr(dst + wave * 8 * 512);
#pragma unroll
  for (int f = 0; f < 8; ++f) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, d + f * 512, 16, lane * 16, f * 1024, 0, 0);
  if (wave == 0) {
    const brsrc rv = make_rsrc(uniform_ptr(valid + kb * 32), 32);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, lds_addr(vdst), 4, lane * 4, 0, 0, 0);
  }
}
constexpr int kVringFloats = 64;  // per ring slot: 32 valid bytes (+ the zeros of the out-of-range lanes)
static_assert(8192 + kAttnRing * kVringFloats <= kWorkFloats, "grouped attention: K/V buffer and valid ring in the working area");
__device__ bool attn_group_items(KArgs& a, int s, int l, float* smem, Sync sy) {
  const int L = a.depth, R = a.R, nbp = a.nbp, nsplit = a.nsplit, B = a.batch;
  const int n_items = B * kAttnGroupsPerSample * nsplit;
  const int tid = phase_tid(), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const size_t slw = (size_t)s * L + l;
  const int nkb_pre = a.s_pre >> 5, nkb = nkb_pre + 2;
  float* apart = a.apart + slw * (size_t)nsplit * nbp * 16 * kHeadDim;
  float* apart_ml = a.apart_ml + slw * (size_t)nsplit * nbp * 32;
  unsigned* fsplit = flag_base(a, s, l, kPhSplit);
  u16* const buf0 = reinterpret_cast<u16*>(smem + kLdsA1);
  u16* const buf1 = reinterpret_cast<u16*>(smem + kLdsWork);
  u16* const buf2 = reinterpret_cast<u16*>(smem + kLdsB);
  float* const vring = smem + kLdsWork + 8192;
  const u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
  for (int item = (unsigned)wg_id(); item < n_items; item += (unsigned)wg_count()) {
    const int b = item % B, rr = item / B, grp = rr % kAttnGroupsPerSample, split = rr / kAttnGroupsPerSample;
    const int pair = grp * kAttnGroup + wave;
    const bool has_rows = pair < kPairs;
    const int bp = b * kPairs + pair;
    const int kb_lo = split * nkb / nsplit, kb_hi = (split + 1) * nkb / nsplit;
    const u16* kpre = a.kpre + ((size_t)l * B + b) * a.s_pre * kHeadDim;
    const u16* vpre = a.vpre + ((size_t)l * B + b) * a.s_pre * kHeadDim;
    const u16* ksf = a.ksuf + (slw * B + b) * 64 * kHeadDim;
    const u16* vsf = a.vsuf + (slw * B + b) * 64 * kHeadDim;
    const uint8_t* valid = a.valid + (size_t)b * (a.s_pre + 64);
    // this wave's 8 of block kb's 32 fragments [K 0..15 | V 0..15] -> ring slot `slot` (waves 0, 1:
    // the K halves, waves 2, 3: the V halves); wave 0 also the block's 32 key-valid bytes
    const u16* ksrc = wave < 2 ? kpre : vpre;
    const u16* ssrc = wave < 2 ? ksf : vsf;
    // the row block's query fragments (registers), then the first blocks
    bf16x8 qf[8];
    const int rbq = b * (kRowsPerSample / 2) + (has_rows ? pair : 0);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qf[ds] = load_frag(qs + afrag_offset(rbq, ds, kHeadDim / 32) + lane * 8);
    attn_stage(ksrc, ssrc, valid, nkb_pre, kb_lo, buf0, vring, wave, lane);
    if (kAttnAhead == 2 && kb_lo + 1 < kb_hi) attn_stage(ksrc, ssrc, valid, nkb_pre, kb_lo + 1, buf1, vring + kVringFloats, wave, lane);
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 oacc[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 3);
    for (int kb = kb_lo; kb < kb_hi; ++kb) {
      const int slot = (kb - kb_lo) % kAttnRing;
      // this wave's loads of block kb have landed (with two blocks ahead, block kb + 1's may still
      // be in flight: 9 loads for wave 0, 8 for the others), then every wave's (the barrier), which
      // also means every wave has read block kb - 1's slot: block kb + kAttnAhead replaces it
      if (kAttnAhead == 2 && kb + 1 < kb_hi) {
        if (wave == 0) wait_vmcnt<9>();
        else wait_vmcnt<8>();
      } else {
        wait_vmcnt<0>();
      }
      wg_barrier();
      if (kb + kAttnAhead < kb_hi) {
        const int sn = (kb + kAttnAhead - kb_lo) % kAttnRing;
        attn_stage(ksrc, ssrc, valid, nkb_pre, kb + kAttnAhead, sn == 0 ? buf0 : sn == 1 ? buf1 : buf2, vring + sn * kVringFloats, wave, lane);
      }
      u32x4_lds fr[32];
      const uint32_t base = (uint32_t)reinterpret_cast<uintptr_t>(slot == 0 ? buf0 : slot == 1 ? buf1 : buf2) + (uint32_t)lane * 16;
#pragma unroll
      for (int f = 0; f < 32; ++f) fr[f] = lds_read16(base + f * 1024);
      const uint32_t vbase = (uint32_t)reinterpret_cast<uintptr_t>(vring + slot * kVringFloats) + (uint32_t)g * 4;
      uint32_t v0 = lds_read4(vbase), v1 = lds_read4(vbase + 16);
      lds_reads_done(fr, v0, v1);
      KvBlock blk;
#pragma unroll
      for (int f = 0; f < 16; ++f) {
        blk.k[f] = __builtin_bit_cast(bf16x8, fr[f]);
        blk.v[f] = __builtin_bit_cast(bf16x8, fr[16 + f]);
      }
      blk.valid0 = v0;
      blk.valid1 = v1;
      if (has_rows) attend_block_q(blk, [&](int ds) { return qf[ds]; }, m_run, l_run, oacc);
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 4);
    // this row block's partial: O (unnormalised, relative to m_run), running max and sum; fp32
    // [16 rows][D], row r16 = lane % 16 holding dims dt*16 + g*4 .. +3 of d-tile dt
    if (has_rows) {
      float* part = apart + ((size_t)split * nbp + bp) * 16 * kHeadDim;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) st_f32x4(part, (size_t)r16 * kHeadDim + g * 4 + dt * 16, float4{oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]});
      if (g == 0) {
        st_f32(apart_ml + ((size_t)split * nbp + bp) * 32 + r16, m_run);
        st_f32(apart_ml + ((size_t)split * nbp + bp) * 32 + 16 + r16, l_run);
      }
    }
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 5);
    // the item's flags (one per row block), every replica; every wave stored rows
    wait_stores();
    wg_barrier();
    if (tid < kAttnGroup * kFlagCopies) {
      const int j = tid / kFlagCopies, rep = tid % kFlagCopies, pj = grp * kAttnGroup + j;
      if (pj < kPairs) st_u32(fsplit + (size_t)(b * kPairs + pj) * a.nsplit_pad + split + (size_t)rep * a.fstride, sy.epoch);
    }
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 6);
  }
  return true;
}

// Merges after the grouped split items: one role per row block (all four head pairs), so the 200
// row blocks at B = 8 take one pass of the grid instead of the 800 (row block, head pair) roles'
// three.  Thread t combines row t / 16 of the row block (16 rows: 2 tokens x 8 heads), dims
// (t % 16) * 16 .. +15, over the splits in the same order and arithmetic as the merges below, and
// stores them straight into o_proj's A operand; then the row block's four merge flags.
__device__ bool attn_group_merges(KArgs& a, int s, int l, Sync sy) {
  const int L = a.depth, R = a.R, nbp = a.nbp, nsplit = a.nsplit;
  const size_t slw = (size_t)s * L + l;
  const float* apart = a.apart + slw * (size_t)nsplit * nbp * 16 * kHeadDim;
  const float* apart_ml = a.apart_ml + slw * (size_t)nsplit * nbp * 32;
  const unsigned* fsplit = flag_base(a, s, l, kPhSplit);
  unsigned* fmerge = flag_base(a, s, l, kPhMerge);
  u16* os = a.o + slw * (size_t)R * (kHeads * kHeadDim);
  const int tid = phase_tid(), rr = tid >> 4, d0 = (tid & 15) * 16;
  const brsrc rml = make_rsrc(apart_ml, (size_t)nsplit * nbp * 32 * 4);
  const brsrc rpo = make_rsrc(apart, (size_t)nsplit * nbp * 16 * kHeadDim * 4);
  for (int bp = (unsigned)wg_id(); bp < nbp; bp += (unsigned)wg_count()) {
    const int b = bp / kPairs, pair = bp % kPairs;
    PHASE_TS(s, l, kPhMerge, 1);
    if (!wait_flags(a, fsplit + bp * a.nsplit_pad, nsplit, sy)) return false;
    PHASE_TS(s, l, kPhMerge, 2);
    // only the splits there are: masked loads would still take an issue slot each
    float mc[kMaxAttnSplits], lc[kMaxAttnSplits];
#pragma unroll
    for (int c = 0; c < kMaxAttnSplits; ++c) {
      mc[c] = -INFINITY, lc[c] = 0.f;
      if (c < nsplit) {
        const int mo = (c * nbp + bp) * 32 + rr;
        buf_f32(mc[c], rml, mo * 4);
        buf_f32(lc[c], rml, (mo + 16) * 4);
      }
    }
    float Mb = -INFINITY;
#pragma unroll
    for (int c = 0; c < kMaxAttnSplits; ++c) Mb = fmaxf(Mb, c < nsplit ? mc[c] : -INFINITY);
    float Lb = 0.f;
    f32x4 ob[4] = {};
    for (int c0 = 0; c0 < nsplit; c0 += 4) {
      f32x4 oc[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool ok = c0 + c < nsplit;
          oc[c][q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rpo, ok ? (int)((((size_t)((c0 + c) * nbp + bp) * 16 + rr) * kHeadDim + d0 + 4 * q) * 4) : kOob, 0, 0));
        }
      sched_fence();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c0 + c >= nsplit) break;
        float m = mc[0], lcv = lc[0];
#pragma unroll
        for (int k = 1; k < kMaxAttnSplits; ++k)
          if (k == c0 + c) m = mc[k], lcv = lc[k];
        const float wc = m == -INFINITY ? 0.f : __expf(m - Mb);
        Lb += lcv * wc;
#pragma unroll
        for (int q = 0; q < 4; ++q) ob[q] += oc[c][q] * wc;
      }
    }
    const float inv = 1.0f / Lb;
    const int token = rr >> 3, head = rr & 7;
    const int r = b * kRowsPerSample + 2 * pair + token;
#pragma unroll
    for (int h8 = 0; h8 < 2; ++h8) {
      u16 v8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v8[i] = f2bf(ob[2 * h8 + i / 4][i % 4] * inv);
      st_bf16x8(os, afrag_index(r, head * kHeadDim + d0 + 8 * h8, kHeads * kHeadDim / 32), v8);
    }
    // the row block's four (row block, head pair) flags, every replica
    PHASE_TS(s, l, kPhMerge, 4);
    wait_stores();
    PHASE_TS(s, l, kPhMerge, 5);
    wg_barrier();
    if (tid < kHeadPairs * kFlagCopies) st_u32(fmerge + 4 * bp + tid / kFlagCopies + (size_t)(tid % kFlagCopies) * a.fstride, sy.epoch);
    PHASE_TS(s, l, kPhMerge, 6);
  }
  return true;
}

template <bool G>
__device__ bool phase_attn(KArgs& a, int s, int l, float* smem, Sync sy) {
  const int L = a.depth, R = a.R, nbp = a.nbp, nsplit = a.nsplit;
  const int n_items = nbp * nsplit;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool comp = tid < kCompThreads;
  const int g = lane >> 4, r16 = lane & 15;
  const size_t slw = (size_t)s * L + l;
  const int nkb_pre = a.s_pre >> 5;
  const int nkb = nkb_pre + 2;
  float* apart = a.apart + slw * (size_t)nsplit * nbp * 16 * kHeadDim;
  float* apart_ml = a.apart_ml + slw * (size_t)nsplit * nbp * 32;
  unsigned* fsplit = flag_base(a, s, l, kPhSplit);
  unsigned* fmerge = flag_base(a, s, l, kPhMerge);
  u16* s_q = reinterpret_cast<u16*>(smem + kLdsWork);  // [8 fragments][512] bf16 (2048 floats)
  // per wave, the 12 O d-tiles the other waves combine ([12][64 lanes][4] each): waves 1, 2 in the
  // upper half of A, waves 0, 3 behind s_q; then the running max and sum of every wave
  auto o_slot = [&](int w) -> float* {
    return w == 1 ? smem + kLdsA1 : w == 2 ? smem + kLdsA1 + 3072 : smem + kLdsWork + 2048 + (w == 0 ? 0 : 3072);
  };
  float* s_m = smem + kLdsWork + 2048 + 6144;  // [4][16]
  float* s_l = s_m + 64;                       // [4][16]
  PHASE_TS(s, l, kPhSplit, 0);
  bool waited = false, burst = false;
  if (attn_grouped<G>(a)) {
    // gate_up(l) tile 0, fragments 0..15 -> region A's lower half, ahead of the polls
    copy_norm_w<kModeGateUp, 0, 16, G>(a, l, 0, smem);
    burst = true;
    PHASE_TS(s, l, kPhSplit, 1);
    if (!wait_flags(a, flag_base(a, s, l, kPhQkv), n_qkv_items<G>(), sy)) return false;
    PHASE_TS(s, l, kPhSplit, 2);
    if (!attn_group_items(a, s, l, smem, sy)) return false;
  }
  // One sample with 9 key splits (prefixes of 961..1056 keys): split s < 8 of every row block runs
  // on workgroup 8 bp + s (XCD s, up to the dispatcher's rotation), split 8 of row block bp on
  // workgroup 8 (25 + bp / 8) + bp mod 8, so each XCD fetches two splits' prefix keys into its L2
  // instead of all nine (measured on MI355X: the same time per predict, ~1.1 GB less traffic)
  const bool xcd_splits = !G && nsplit == 9 && nbp == kPairs;
  for (int item = attn_grouped<G>(a) ? n_items : wg_id(); item < (xcd_splits ? 256 : n_items); item += (unsigned)wg_count()) {
    int bp = item % nbp, split = item / nbp;
    if (xcd_splits) {
      const int x = item & 7, j = item >> 3;
      split = j < kPairs ? x : 8;
      bp = j < kPairs ? j : 8 * (j - kPairs) + x;
      if (bp >= kPairs) continue;
    }
    const int b = bp / kPairs, pair = bp % kPairs;
    const int rbq = b * (kRowsPerSample / 2) + pair;  // query-row m-tile (16 rows = 2 tokens x 8 heads)
    const u16* kpre = a.kpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* vpre = a.vpre + ((size_t)l * a.batch + b) * a.s_pre * kHeadDim;
    const u16* ksf = a.ksuf + (slw * a.batch + b) * 64 * kHeadDim;
    const u16* vsf = a.vsuf + (slw * a.batch + b) * 64 * kHeadDim;
    const uint8_t* valid = a.valid + (size_t)b * (a.s_pre + 64);
    const int kb_lo = split * nkb / nsplit, kb_hi = (split + 1) * nkb / nsplit;
    auto load = [&](KvBlock& blk, int kb) {
      if (kb >= nkb_pre) load_kv_block(blk, ksf, vsf, valid + kb * 32, kb - nkb_pre, lane);
      else load_kv_block(blk, kpre, vpre, valid + kb * 32, kb, lane);
    };
    // Blocks: the copy wave attends the split's first block if it is from the static prefix (it
    // loads it before the polls and before its gate_up copies, so the copies never delay it);
    // compute wave w attends blocks first + o(w), + 3, ... with o = 2, 0, 1 for waves 0, 1, 2
    // (wave 0 gets the fourth, which a split most often lacks).  Every wave loads its first block
    // ahead of the polls when it is from the prefix (wave 0's polls then complete after it lands).
    const bool cw_block = kb_lo < kb_hi && kb_lo < nkb_pre;
    const int first = kb_lo + (cw_block ? 1 : 0);
    const int kb0 = copy_wave() ? kb_lo : first + (wave == 0 ? 2 : wave - 1);
    const bool has_block = copy_wave() ? cw_block : kb0 < kb_hi;
    // wave 0 polls: anything it loads before its polls completes first (a wave's vector memory
    // operations complete in issue order), so its block is loaded after the wait
    const bool pre = has_block && kb0 < nkb_pre && wave != 0;
    KvBlock blk;
    if (pre) load(blk, kb0);
    if (!burst) {
      if constexpr (G) copy_norm_w<kModeGateUp, 0, 16, G>(a, l, 0, smem);  // gate_up(l) tile 0, fragments 0..15 -> A
      burst = true;  // (one sample: the whole tile was copied at qkv)
    }
    PHASE_TS(s, l, kPhSplit, 1);
    if (!waited) {
      if (!wait_flags(a, flag_base(a, s, l, kPhQkv), n_qkv_items<G>(), sy)) return false;
      waited = true;
    }
    PHASE_TS(s, l, kPhSplit, 2);
    // the row block's query fragments -> LDS (direct-to-LDS, compute waves), then the blocks not
    // yet loaded
    const u16* qs = a.q + slw * (size_t)R * kQRowsPerTok * kHeadDim;
    if (comp) {
      const int wu = __builtin_amdgcn_readfirstlane(wave);  // LDS addresses of direct-to-LDS loads are wave-uniform
      for (int f = wu; f < 8; f += kCompWaves)
        __builtin_amdgcn_global_load_lds(const_cast<u16*>(qs + afrag_offset(rbq, f, kHeadDim / 32)) + lane * 8, lds_addr(s_q + (size_t)f * 512),
                                         16, 0, 0);
      if (has_block && !pre) load(blk, kb0);
      wait_vmcnt<0>();  // the query fragments have landed in LDS (and this wave's block)
    }
    __syncthreads();
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 oacc[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (copy_wave()) {
      if (has_block) attend_block_lds(blk, s_q, lane, m_run, l_run, oacc);
    } else {
      for (int kb = kb0; kb < kb_hi; kb += kCompWaves) {
        if (kb != kb0) load(blk, kb);
        attend_block_lds(blk, s_q, lane, m_run, l_run, oacc);
      }
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (item == wg_id()) {
      PHASE_TS(s, l, kPhSplit, 4);
      PHASE_TS_W(1, s, l, kPhSplit, 7);
      PHASE_TS_W(2, s, l, kPhSplit, 8);
      PHASE_TS_W(3, s, l, kPhSplit, 9);
    }
    // ---- merge the 4 waves: wave w combines d-tiles 4w .. 4w+3 of all four waves.  Every wave
    // puts the 12 d-tiles the others combine (slot index: d-tiles below its own four, then those
    // above) and its (max, sum) per row in LDS (no slot aliases s_q), then combines its four in
    // wave order and stores them: fp32 [16 rows][D], row r16 = lane % 16 holding dims
    // dt*16 + g*4 .. +3 of d-tile dt
    if (g == 0) {
      s_m[wave * 16 + r16] = m_run;
      s_l[wave * 16 + r16] = l_run;
    }
    {
      float* so = o_slot(wave);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) {
        if ((dt >> 2) == wave) continue;
        const int si = dt < 4 * wave ? dt : dt - 4;
        *reinterpret_cast<f32x4*>(so + ((size_t)si * 64 + lane) * 4) = oacc[dt];
      }
    }
    __syncthreads();
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 3);
    {
      float mw[4], Mx = -INFINITY, Lx = 0.f, ww[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        mw[v] = s_m[v * 16 + r16];
        Mx = fmaxf(Mx, mw[v]);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        ww[v] = (mw[v] == -INFINITY) ? 0.f : __expf(mw[v] - Mx);
        Lx += s_l[v * 16 + r16] * ww[v];
      }
      float* part = apart + ((size_t)split * nbp + bp) * 16 * kHeadDim;  // + row r16, dims g*4 + dt*16
      auto combine = [&](auto wc) {
        constexpr int W = decltype(wc)::value;
        f32x4 ov[4][4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int dt = 4 * W + j;
            if (v == W) ov[v][j] = oacc[dt];
            else ov[v][j] = *reinterpret_cast<const f32x4*>(o_slot(v) + ((size_t)(dt < 4 * v ? dt : dt - 4) * 64 + lane) * 4);
          }
        sched_fence();  // all twelve LDS reads in flight before the first use
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 o = ov[0][j] * ww[0] + ov[1][j] * ww[1] + ov[2][j] * ww[2] + ov[3][j] * ww[3];
          st_f32x4(part, (size_t)r16 * kHeadDim + g * 4 + (4 * W + j) * 16, float4{o[0], o[1], o[2], o[3]});
        }
      };
      switch (wave) {
        case 0: combine(std::integral_constant<int, 0>{}); break;
        case 1: combine(std::integral_constant<int, 1>{}); break;
        case 2: combine(std::integral_constant<int, 2>{}); break;
        default: combine(std::integral_constant<int, 3>{}); break;
      }
      if (wave == 0 && g == 0) {
        st_f32(apart_ml + ((size_t)split * nbp + bp) * 32 + r16, Mx);
        st_f32(apart_ml + ((size_t)split * nbp + bp) * 32 + 16 + r16, Lx);
      }
    }
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 5);
    publish(a, fsplit + bp * a.nsplit_pad + split, sy.epoch, true);  // the copy wave stored d-tiles 12..15
    if (item == wg_id()) PHASE_TS(s, l, kPhSplit, 6);
    __syncthreads();  // the LDS tiles are reused by the next item
  }
  // the rest of gate_up(l) -> region A, whose upper half the split items no longer use (the
  // workgroups without a split item: all of it), ahead of the merge polls
  if constexpr (G) {
    if (!burst) copy_norm_w<kModeGateUp, 0, 16, G>(a, l, 0, smem);
    copy_norm_w<kModeGateUp, 16, 16, G>(a, l, 0, smem);
  }
  copy_norm_w<kModeGateUp, 0, 32, G>(a, l, 1, smem);
  if (attn_grouped<G>(a)) return attn_group_merges(a, s, l, sy);
  // ---- merges.  Role = hp * nbp + bp runs on workgroup role mod grid, i.e. with the split
  // (bp, hp) when hp < nsplit.  Every split item was finished above, so no workgroup waits here
  // on work of its own.  All four waves merge (the copy wave has nothing in flight by now): thread
  // t owns row t/64 of the head pair (r16 = 2hp + (j&1) + 8*(j>>1)) and dims (t%64)*4 .. +3, and
  // loads every split's (max, sum, O) at once.
  bool first_merge = true;
  for (int role = (unsigned)wg_id(); role < kHeadPairs * nbp; role += (unsigned)wg_count()) {
    const int bp = role % nbp, hp = role / nbp;
    const int b = bp / kPairs, pair = bp % kPairs;
    if (first_merge) PHASE_TS(s, l, kPhMerge, 1);
    if (!wait_flags(a, fsplit + bp * a.nsplit_pad, nsplit, sy)) return false;
    if (first_merge) PHASE_TS(s, l, kPhMerge, 2);
    {
      const int jr = tid >> 6, rr = 2 * hp + (jr & 1) + 8 * (jr >> 1);
      const int d0 = (tid & 63) * 4;
      const brsrc rml = make_rsrc(apart_ml, (size_t)nsplit * nbp * 32 * 4);
      const brsrc rpo = make_rsrc(apart, (size_t)nsplit * nbp * 16 * kHeadDim * 4);
      float mc[kMaxAttnSplits], lc[kMaxAttnSplits];
      f32x4 oc[kMaxAttnSplits];
#pragma unroll
      for (int c = 0; c < kMaxAttnSplits; ++c) {
        const bool ok = c < nsplit;
        const int mo = (c * nbp + bp) * 32 + rr;
        buf_f32(mc[c], rml, ok ? mo * 4 : kOob);
        buf_f32(lc[c], rml, ok ? (mo + 16) * 4 : kOob);
        oc[c] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rpo, ok ? (int)((((size_t)(c * nbp + bp) * 16 + rr) * kHeadDim + d0) * 4) : kOob, 0, 0));
      }
      sched_fence();
      float Mb = -INFINITY;
#pragma unroll
      for (int c = 0; c < kMaxAttnSplits; ++c) Mb = fmaxf(Mb, c < nsplit ? mc[c] : -INFINITY);
      float Lb = 0.f;
      f32x4 ob = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kMaxAttnSplits; ++c) {
        const float wc = (c >= nsplit || mc[c] == -INFINITY) ? 0.f : __expf(mc[c] - Mb);
        Lb += lc[c] * wc;
        ob += oc[c] * wc;
      }
      // straight into o_proj's A operand [R, H*D] (no LDS round trip): the thread's 4 dims of row
      // (token, head) are 8 contiguous bytes of one fragment
      const float inv = 1.0f / Lb;
      u16 v4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v4[i] = f2bf(ob[i] * inv);
      u16* os = a.o + slw * (size_t)R * (kHeads * kHeadDim);
      const int r = b * kRowsPerSample + 2 * pair + (rr >> 3), head = rr & 7;
      st_bf16x4(os, afrag_index(r, head * kHeadDim + d0, kHeads * kHeadDim / 32), v4);
    }
    publish(a, fmerge + 4 * bp + hp, sy.epoch);
    if (first_merge) PHASE_TS(s, l, kPhMerge, 6);
    first_merge = false;
  }
  return true;
}

// =============================================================================================
// o_proj (K = 2048) and the gated residual after attention: item = (m-tile mq of every sample,
// 16-column tile nt), 256 items, no K split.  The three compute waves split K (22 k-steps each;
// wave 2's last two are surplus and read A as zeros) and load their weight fragments into
// registers ahead of the polls, so only the attention output is fetched after them.  Per sample:
// wait for the merges of the m-tile's row blocks (all four head pairs), MFMA in four independent
// chains, add the waves in LDS, then h = bf16(h + bf16(bf16(y) * gate)) (modeling_gemma.py:231-249,
// 503), g = bf16(h * (1 + scale)) of the pre-MLP norm and the tile's row sums of squares.
// =============================================================================================
__device__ bool phase_oproj(KArgs& a, int s, int l, float* smem, Sync sy) {
  // waves 1 and 2 hold the tile's weights (K halves) and do the MFMA; wave 0 only polls, so
  // nothing it issued before its polls (a wave's vector memory operations complete in issue
  // order) delays seeing the merges; wave 1 also runs the residual epilogue
  constexpr int KSTEPS = kHeads * kHeadDim / 32, KSW = KSTEPS / 2;
  constexpr int NCH = 4;  // independent accumulation chains per wave
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int item = (unsigned)wg_id();
  PHASE_TS(s, l, kPhO, 0);
  {
    // copy wave (idle here): the next layer's first qkv tile -> region B, half of the burst that
    // down_proj's polls would otherwise share the memory side with
    int ln;
    if (next_layer(a, s, l, &ln)) copy_qkv_tile0(a, ln, smem);
  }
  if (item >= kOItems) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool mw = wave == 1 || wave == 2;  // MFMA waves
  const int nt = item % kTiles, mq = item / kTiles;
  const int col = nt * 16, ks0 = (wave == 2 ? 1 : 0) * KSW, r16 = lane & 15;
  const int nrow = kHorizon - 16 * mq < 16 ? kHorizon - 16 * mq : 16;  // action rows of the m-tile
  const int np = (nrow + 1) / 2;                                         // its two-token row blocks
  const size_t slw = (size_t)s * L + l;
  // the wave's weight fragments, ahead of the polls
  bf16x8 wf[KSW];
  if (mw) {
    const brsrc rw = make_rsrc(a.wpack + (size_t)l * kLayerElems + kOffO + (size_t)nt * KSTEPS * 512, (size_t)KSTEPS * 1024);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) buf_frag(wf[s2], rw, ((ks0 + s2) * 512 + lane * 8) * 2);
  }
  // the products are formed as W . A^T, so lane l ends with columns ec = 4 (l / 16) .. + 3 of row
  // l % 16; the epilogue is wave 1's, lane-local: gate and 1 + scale of its 4 columns ahead of
  // the polls
  const bool ep_wave = wave == 1;
  const int erow = r16, ec = 4 * (lane >> 4);
  const u16* hres = a.h + ((size_t)s * (L + 1) + l) * R * kWidth;
  float4 g4 = {}, s14 = {};
  if (ep_wave) {
    g4 = *reinterpret_cast<const float4*>(a.table + ((size_t)s * NN + 2 * l) * kModW + 2 * kWidth + col + ec);
    s14 = *reinterpret_cast<const float4*>(a.table_s1 + ((size_t)s * NN + 2 * l + 1) * kModW + col + ec);
  }
  PHASE_TS(s, l, kPhO, 1);
  const u16* act = a.o + slw * (size_t)R * (KSTEPS * 32);
  u16* hout = a.hmid + slw * (size_t)R * kWidth;
  u16* gout = a.gmid + slw * (size_t)R * kWidth;
  float* rout = a.ssmid + slw * kTiles * R;
  const unsigned* fmerge = flag_base(a, s, l, kPhMerge);
  float* red = smem + kLdsWork;  // [2 MFMA waves][64 lanes][4]
  const float gate[4] = {round_bf(g4.x), round_bf(g4.y), round_bf(g4.z), round_bf(g4.w)};
  const float s1[4] = {s14.x, s14.y, s14.z, s14.w};
  {
    constexpr int b = 0;  // one sample: the batch instances run phase_oproj_pairs / phase_oproj_msplit
    const int m = 4 * b + mq;  // m-tile of the activations
    // merge flags 4 * bp + hp: the m-tile's row blocks bp = 25 b + 8 mq .. are one contiguous run
    if (!wait_flags(a, fmerge + 4 * (b * kPairs + 8 * mq), 4 * np, sy)) return false;
    if (b == 0) PHASE_TS(s, l, kPhO, 2);
    // the residual rows: the merges waited for imply every earlier phase of the layer, so the
    // previous layer's down_proj has written them (this workgroup may have had no qkv item)
    const int r = 16 * m + erow;
    uint2 hold = {0u, 0u};
    if (ep_wave && erow < nrow) hold = *reinterpret_cast<const uint2*>(hres + afrag_index(r, col + ec, kWidth / 32));
    if (mw) {
      const brsrc ra = make_rsrc(act, (size_t)R * KSTEPS * 64);
      bf16x8 af[KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) {
        const bool ok = r16 < nrow;
        buf_frag(af[s2], ra, ok ? (int)((afrag_offset(m, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
      }
      sched_fence();
      f32x4 acc[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) acc[s2 % NCH] = mfma16x16x32(wf[s2], af[s2], acc[s2 % NCH]);
      *reinterpret_cast<f32x4*>(red + ((size_t)(wave - 1) * 64 + lane) * 4) = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    if (b == 0) PHASE_TS(s, l, kPhO, 4);
    __syncthreads();
    if (ep_wave) {
      // the two K halves in order, then h = bf16(h + bf16(bf16(y) * gate)), g = bf16(h * (1 + scale))
      // and the row's sum of squares over the tile's 16 columns (the four lanes of the row)
      const f32x4 y = *reinterpret_cast<const f32x4*>(red + (size_t)lane * 4) + *reinterpret_cast<const f32x4*>(red + (size_t)(64 + lane) * 4);
      float ss = 0.f;
      if (erow < nrow) {
        u16 hn[4], gn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u16 hb = (u16)((i < 2 ? hold.x : hold.y) >> (16 * (i & 1)));
          const float prod = round_bf(fmul(round_bf(y[i]), gate[i]));
          hn[i] = f2bf(fadd(bf2f(hb), prod));
          const float hf = bf2f(hn[i]);
          gn[i] = f2bf(fmul(hf, s1[i]));
          ss += hf * hf;
        }
        st_bf16x4(hout, afrag_index(r, col + ec, kWidth / 32), hn);
        st_bf16x4(gout, afrag_index(r, col + ec, kWidth / 32), gn);
      }
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      // tile-major statistics: the tile's sums of the m-tile's 16 rows (padded rows: zero)
      if (lane < 16) st_f32(rout + (size_t)nt * R + 16 * m + lane, ss);
    }
  }
  PHASE_TS(s, l, kPhO, 5);
  publish(a, flag_base(a, s, l, kPhO) + item, sy.epoch);
  PHASE_TS(s, l, kPhO, 6);
  return true;
}

// =============================================================================================
// o_proj of both batch instances: one wait for every sample's merges (which finish in one pass of
// the grid), then two wave pairs, (1, 2) and (0, 3), each holding the tile's weights in K halves
// (wave 1 / 0: k-steps 0..31, wave 2 / 3: 32..63), take samples 2i and 2i + 1 of iteration i side
// by side.  Per sample the arithmetic is phase_oproj's (same accumulation chains, K halves added in
// order, same epilogue); epilogue threads: lanes 0..31 of wave 1 (pair 0) and of wave 0 (pair 1).
// With grouped attention the copy wave issues down(l)'s weights into region B after its own weight
// loads and before the polls.  Measured on MI355X against one sample at a time on waves 1 and 2
// with a wait per sample: B=8 17.9 -> 17.1 ms, B=3 11.5 -> 11.4, B=2 7.88 -> 7.79 per predict.
// =============================================================================================
__device__ bool phase_oproj_pairs(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kHeads * kHeadDim / 32, KSW = KSTEPS / 2, TS = 17;
  constexpr int NCH = 4;
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int item = (unsigned)wg_id();
  PHASE_TS(s, l, kPhO, 0);
  const bool grouped = attn_grouped<true>(a);
  if (item >= kOItems) {
    if (grouped) copy_residual_w<kMlp / 32>(a, l, smem);
    return true;
  }
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int pr = (wave == 1 || wave == 2) ? 0 : 1;  // wave pair
  const int kh = (wave == 2 || wave == 3) ? 1 : 0;  // K half
  const int nt = item % kTiles, mq = item / kTiles;
  const int col = nt * 16, ks0 = kh * KSW, r16 = lane & 15;
  const int nrow = kHorizon - 16 * mq < 16 ? kHorizon - 16 * mq : 16;
  const int np = (nrow + 1) / 2;
  const size_t slw = (size_t)s * L + l;
  bf16x8 wf[KSW];
  {
    const brsrc rw = make_rsrc(a.wpack + (size_t)l * kLayerElems + kOffO + (size_t)nt * KSTEPS * 512, (size_t)KSTEPS * 1024);
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) buf_frag(wf[s2], rw, ((ks0 + s2) * 512 + lane * 8) * 2);
  }
  if (grouped) copy_residual_w<kMlp / 32>(a, l, smem);  // copy wave: down(l) -> B (after attention's use of B)
  const bool ep_thread = (wave == 1 || wave == 0) && lane < 32;
  const int erow = lane >> 1, ec0 = (lane & 1) * 8;
  const u16* hres = a.h + ((size_t)s * (L + 1) + l) * R * kWidth;
  float4 g4[2] = {}, s14[2] = {};
  if (ep_thread) {
    const float* gmod = a.table + ((size_t)s * NN + 2 * l) * kModW + 2 * kWidth + col + ec0;
    const float* smod = a.table_s1 + ((size_t)s * NN + 2 * l + 1) * kModW + col + ec0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      g4[i] = *reinterpret_cast<const float4*>(gmod + 4 * i);
      s14[i] = *reinterpret_cast<const float4*>(smod + 4 * i);
    }
  }
  PHASE_TS(s, l, kPhO, 1);
  const u16* act = a.o + slw * (size_t)R * (KSTEPS * 32);
  u16* hout = a.hmid + slw * (size_t)R * kWidth;
  u16* gout = a.gmid + slw * (size_t)R * kWidth;
  float* rout = a.ssmid + slw * kTiles * R;
  float* red = smem + kLdsWork;     // [pair][K half][64 lanes][4]
  float* T = red + 4 * 256;         // [pair][16][TS]
  float* s_ss = T + 2 * 16 * TS;    // [pair][2 column halves][16 rows]
  float* Tp = T + pr * 16 * TS;
  const float gate[8] = {round_bf(g4[0].x), round_bf(g4[0].y), round_bf(g4[0].z), round_bf(g4[0].w),
                         round_bf(g4[1].x), round_bf(g4[1].y), round_bf(g4[1].z), round_bf(g4[1].w)};
  const float s1[8] = {s14[0].x, s14[0].y, s14[0].z, s14[0].w, s14[1].x, s14[1].y, s14[1].z, s14[1].w};
  // merge flags 4 * bp + hp: sample b's run for this m-tile starts at 4 (25 b + 8 mq)
  if (!wait_flag_runs(a, flag_base(a, s, l, kPhMerge) + 4 * 8 * mq, 4 * np, 4 * kPairs, a.batch, sy)) return false;
  PHASE_TS(s, l, kPhO, 2);
  for (int i = 0; 2 * i < a.batch; ++i) {
    const int b = 2 * i + pr;
    const bool has = b < a.batch;
    const int m = 4 * b + mq;  // m-tile of the activations
    const int r = 16 * m + erow;
    u16x8 hold = {};
    if (ep_thread && has && erow < nrow) hold = *reinterpret_cast<const u16x8*>(hres + afrag_index(r, col + ec0, kWidth / 32));
    {
      const brsrc ra = make_rsrc(act, (size_t)R * KSTEPS * 64);
      bf16x8 af[KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) {
        const bool ok = has && r16 < nrow;
        buf_frag(af[s2], ra, ok ? (int)((afrag_offset(m, ks0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
      }
      sched_fence();
      f32x4 acc[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) acc[s2 % NCH] = mfma16x16x32(af[s2], wf[s2], acc[s2 % NCH]);
      *reinterpret_cast<f32x4*>(red + (((size_t)pr * 2 + kh) * 64 + lane) * 4) = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    if (i == 0) PHASE_TS(s, l, kPhO, 4);
    wg_barrier();
    // each pair's two K halves in order, scattered row-major into its T (wave p: pair p)
    if (tid < 128) {
      const int pp = tid >> 6;
      const float* rp = red + (size_t)pp * 2 * 256;
      const f32x4 v = *reinterpret_cast<const f32x4*>(rp + (size_t)lane * 4) + *reinterpret_cast<const f32x4*>(rp + (size_t)(64 + lane) * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) T[(size_t)pp * 16 * TS + ((lane >> 4) * 4 + j) * TS + (lane & 15)] = v[j];
    }
    wg_barrier();
    float ss = 0.f;
    if (ep_thread && has && erow < nrow) {
      u16 hn[8], gn[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float prod = round_bf(fmul(round_bf(Tp[erow * TS + ec0 + j]), gate[j]));
        hn[j] = f2bf(fadd(bf2f(hold[j]), prod));
        const float hf = bf2f(hn[j]);
        gn[j] = f2bf(fmul(hf, s1[j]));
        ss += hf * hf;
      }
      st_bf16x8(hout, afrag_index(r, col + ec0, kWidth / 32), hn);
      st_bf16x8(gout, afrag_index(r, col + ec0, kWidth / 32), gn);
    }
    if (ep_thread) s_ss[pr * 32 + (lane & 1) * 16 + erow] = ss;
    wg_barrier();
    // tile-major statistics of both samples: the tile's sums of the m-tile's 16 rows (padded rows: zero)
    if (tid < 32) {
      const int pp = tid >> 4, rr = tid & 15, bb = 2 * i + pp;
      if (bb < a.batch) st_f32(rout + (size_t)nt * R + 16 * (4 * bb + mq) + rr, s_ss[pp * 32 + rr] + s_ss[pp * 32 + 16 + rr]);
    }
    wg_barrier();  // red, T and s_ss are reused by the next iteration
  }
  PHASE_TS(s, l, kPhO, 5);
  publish(a, flag_base(a, s, l, kPhO) + item, sy.epoch);
  PHASE_TS(s, l, kPhO, 6);
  return true;
}

// =============================================================================================
// o_proj of kernel instance 2, split by rows.  KS = 2 (batches above 4): item i = (16-column tile
// nt = i mod 64, sample pair j = i / 64), wave (p, h) = (wave & 1, wave >> 1) takes sample 2j + p
// over K half h and finishes m-tiles 2h, 2h + 1.  KS = 4 (batches up to 4, so that every
// workgroup has an item): item i = (nt, sample j), wave h takes K quarter h and finishes m-tile
// h.  Items past the grid loop.  A wave's weight fragments are in registers (loaded before the
// polls); all four m-tiles of its sample's attention output stream one chunk ahead as in
// phase_gateup_msplit.  The K parts of a sample meet in LDS and are added in K order; the gated
// residual after attention then runs lane-local on columns 4g .. 4g+3 of one row
// (modeling_gemma.py:231-249, 503): h = bf16(h + bf16(bf16(y) * gate)), g = bf16(h * (1 + scale))
// of the pre-MLP norm, and the tile's row sums of squares (the four column groups added across
// lanes; padded rows: zero).  An item waits only for its samples' merges.  Every workgroup
// publishes one flag, after its items.
// =============================================================================================
template <int KS>
__device__ bool phase_oproj_msplit(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kHeads * kHeadDim / 32, KSW = KSTEPS / KS, NCH = KSW / kGuCk;
  constexpr int SPI = 4 / KS, MPW = 4 / KS;  // samples per item, m-tiles finished per wave
  static_assert(KS == 2 || KS == 4, "K halves or quarters");
  static_assert(4 * 4 * 64 * 4 <= kWorkFloatsBatched, "row-split o_proj: K-part exchange in the working area");
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  PHASE_TS(s, l, kPhO, 0);
  // copy wave: down(l) -> B, when grouped attention's K/V ring used B (else copied at qkv)
  if (kAttnRing >= 3 && attn_grouped<true>(a)) copy_residual_w<kMlp / 32>(a, l, smem);
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int pr = KS == 2 ? (wave & 1) : 0, kh = KS == 2 ? (wave >> 1) : wave;
  const int n_items = kTiles * ((a.batch + SPI - 1) / SPI);
  const size_t slw = (size_t)s * L + l;
  const brsrc rg = make_rsrc(a.o + slw * (size_t)R * (KSTEPS * 32), (size_t)R * KSTEPS * 64);
  const u16* hres = a.h + ((size_t)s * (L + 1) + l) * R * kWidth;
  u16* hout = a.hmid + slw * (size_t)R * kWidth;
  u16* gout = a.gmid + slw * (size_t)R * kWidth;
  float* rout = a.ssmid + slw * kTiles * R;
  float* xch = smem + kLdsWork;  // [sample p][from K part h][m-tile][64 lanes][4]
  auto pick = [](const f32x4 (&v)[4], int mt) { return mt == 0 ? v[0] : mt == 1 ? v[1] : mt == 2 ? v[2] : v[3]; };
  for (int item = wg_id(); item < n_items; item += (unsigned)wg_count()) {
    const int nt = item % kTiles, j = item / kTiles;
    const int col = nt * 16, b = SPI * j + pr;
    const bool has = b < a.batch;
    bf16x8 wf[KSW];
    auto load_w = [&]() {
      const brsrc rw = make_rsrc(a.wpack + (size_t)l * kLayerElems + kOffO + (size_t)nt * KSTEPS * 512, (size_t)KSTEPS * 1024);
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2) buf_frag(wf[s2], rw, ((kh * KSW + s2) * 512 + lane * 8) * 2);
    };
    // the weight fragments: before the polls, except wave 0's (it polls; its polls would queue
    // behind the workgroup's 128 KiB of weight loads)
    if (wave != 0) load_w();
    // gate (rounded to bf16) and 1 + scale of columns col + 4g .. col + 4g + 3
    const float4 g4 = *reinterpret_cast<const float4*>(a.table + ((size_t)s * NN + 2 * l) * kModW + 2 * kWidth + col + 4 * g);
    const float4 s14 = *reinterpret_cast<const float4*>(a.table_s1 + ((size_t)s * NN + 2 * l + 1) * kModW + col + 4 * g);
    const float gate[4] = {round_bf(g4.x), round_bf(g4.y), round_bf(g4.z), round_bf(g4.w)};
    const float s1[4] = {s14.x, s14.y, s14.z, s14.w};
    PHASE_TS(s, l, kPhO, 1);
    // the merges of the item's row blocks: 4 flags per row block, kPairs row blocks per sample
    const int nb = a.batch - SPI * j < SPI ? a.batch - SPI * j : SPI;
    if (!wait_flags(a, flag_base(a, s, l, kPhMerge) + 4 * kPairs * SPI * j, 4 * kPairs * nb, sy)) return false;
    PHASE_TS(s, l, kPhO, 2);
    if (wave == 0) load_w();
    // residual rows of the m-tiles this wave finishes (rows 16 mt + r16, columns col + 4g ..)
    uint2 hold[MPW] = {};
#pragma unroll
    for (int q = 0; q < MPW; ++q) {
      const int row = 16 * (MPW * kh + q) + r16;
      if (has && row < kHorizon)
        hold[q] = *reinterpret_cast<const uint2*>(hres + afrag_index(b * kRowsPerSample + row, col + 4 * g, kWidth / 32));
    }
    bf16x8 A[4][4][kGuCk];
#pragma unroll
    for (int c = 0; c < kGuAhead; ++c) gu_load_chunk<KSTEPS>(A[c], rg, b, has, c, lane, kh * KSW);
    sched_fence();
    f32x4 acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c + kGuAhead < NCH) gu_load_chunk<KSTEPS>(A[(c + kGuAhead) % 4], rg, b, has, c + kGuAhead, lane, kh * KSW);
      sched_fence();
#pragma unroll
      for (int s2 = 0; s2 < kGuCk; ++s2) {
        const bf16x8 a3 = s2 == 0 ? mtile3_frag<0>(A[c % 4]) : s2 == 1 ? mtile3_frag<1>(A[c % 4]) : s2 == 2 ? mtile3_frag<2>(A[c % 4]) : mtile3_frag<3>(A[c % 4]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt] = mfma16x16x32(wf[c * kGuCk + s2], mt < 3 ? A[c % 4][mt][s2] : a3, acc[mt]);
      }
    }
    if (item == wg_id()) PHASE_TS(s, l, kPhO, 4);
    // the m-tiles other waves finish -> LDS
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt / MPW != kh) *reinterpret_cast<f32x4*>(xch + ((((size_t)pr * KS + kh) * 4 + mt) * 64 + lane) * 4) = acc[mt];
    wg_barrier();
#pragma unroll
    for (int q = 0; q < MPW; ++q) {
      const int mt = MPW * kh + q, row = 16 * mt + r16;
      const f32x4 own = pick(acc, mt);
      f32x4 y;
#pragma unroll
      for (int h = 0; h < KS; ++h) {
        const f32x4 v = h == kh ? own : *reinterpret_cast<const f32x4*>(xch + ((((size_t)pr * KS + h) * 4 + mt) * 64 + lane) * 4);
        y = h == 0 ? v : y + v;
      }
      const bool live = has && row < kHorizon;
      const uint32_t hw[2] = {hold[q].x, hold[q].y};
      u16 hn[4], gn[4];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u16 hb = (u16)(hw[i >> 1] >> (16 * (i & 1)));
        const float prod = round_bf(fmul(round_bf(y[i]), gate[i]));
        hn[i] = f2bf(fadd(bf2f(hb), prod));
        const float hf = bf2f(hn[i]);
        gn[i] = f2bf(fmul(hf, s1[i]));
        ss += hf * hf;
      }
      if (live) {
        const uint32_t off = (uint32_t)(afrag_index(b * kRowsPerSample + row, col + 4 * g, kWidth / 32) * 2);
        st_wt8(hout, off, (uint32_t)hn[0] | ((uint32_t)hn[1] << 16), (uint32_t)hn[2] | ((uint32_t)hn[3] << 16));
        st_wt8(gout, off, (uint32_t)gn[0] | ((uint32_t)gn[1] << 16), (uint32_t)gn[2] | ((uint32_t)gn[3] << 16));
      }
      ss = lane_sum_xor32(lane_sum_xor16(live ? ss : 0.f));
      if (has && g == 0) st_f32(rout + (size_t)nt * R + b * kRowsPerSample + row, ss);
    }
    wg_barrier();  // xch is reused by the next item
  }
  PHASE_TS(s, l, kPhO, 5);
  if (wg_id() < kOItems) publish(a, flag_base(a, s, l, kPhO) + (unsigned)wg_id(), sy.epoch, true);  // every wave stored rows
  PHASE_TS(s, l, kPhO, 6);
  return true;
}

// =============================================================================================
// down_proj at one sample without a K split: item = (16-column tile nt, m-tile mq), 256 items, so
// no partial sum leaves the workgroup and no finisher hand-off follows.  The four waves each take
// a K quarter (32 k-steps): the copy wave, waves 1 and 2 take quarters mq, mq + 2 and mq + 3
// (mod 4) with their weight fragments loaded into registers ahead of the polls (the copy wave's
// before its burst of the next layer's copies, so they land first); wave 0, the poller, takes
// quarter mq + 1 and loads its fragments after the polls.  The four m-tiles' items of a tile run
// on one XCD and read the tile's four quarters at about the same time, so each quarter comes
// from the memory side once.  (Measured on MI355X: with the copy wave's quarter copied to region
// B during qkv, 20 us earlier, every quarter was fetched twice, 1.4 GB more per predict.)  The products are formed as W . A^T (a lane ends with 4 consecutive columns of one row);
// the quarters are added in quarter order in LDS and wave 1 runs the finisher's epilogue:
// h = bf16(hmid + bf16(bf16(y) * gate)) (modeling_gemma.py:503), g = bf16(h * (1 + scale)) of the
// next layer's first norm, and the tile's row sums of squares of h.
// =============================================================================================
// The copy wave's burst at down_proj(l): the next layer's second qkv tile -> region A1 (its first
// tile went to region B at o_proj(l)).
__device__ __forceinline__ void down_next_qkv_copies(KArgs& a, int s, int l, float* smem) {
  int ln;
  if (next_layer(a, s, l, &ln)) copy_norm_w<kModeQkv, 0, 31>(a, ln, 1, smem);
}
__device__ bool phase_down_rows(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kMlp / 32, KQ = KSTEPS / kKSplit;
  constexpr int NCH = 4;  // independent accumulation chains per wave
  constexpr int PH = kPhDown;
  const int L = a.depth, NN = 2 * L + 1, R = kRowsPerSample;
  const int item = (unsigned)wg_id();
  PHASE_TS(s, l, PH, 0);
  if (item >= kDownItems1) {
    down_next_qkv_copies(a, s, l, smem);
    return true;
  }
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int nt = item % kTiles, mq = item / kTiles;
  const int kq = (mq + (wave + 1) % 4) & (kKSplit - 1);  // this wave's K quarter
  const int col = nt * 16, r16 = lane & 15, ec = 4 * (lane >> 4);
  const int nrow = kHorizon - 16 * mq < 16 ? kHorizon - 16 * mq : 16;  // action rows of the m-tile
  const size_t slw = (size_t)s * L + l;
  bf16x8 wf[KQ];
  const brsrc rw = make_rsrc(a.wpack + (size_t)l * kLayerElems + kOffDown + (size_t)nt * KSTEPS * 512, (size_t)KSTEPS * 1024);
  auto load_w = [&]() {
    // (the quarter goes into the per-lane offset: a resource built from it would not be uniform)
#pragma unroll
    for (int s2 = 0; s2 < KQ; ++s2) buf_frag(wf[s2], rw, ((kq * KQ + s2) * 512 + lane * 8) * 2);
  };
  if (wave != 0) load_w();
  // wave 1 (the epilogue's): the gate of norm 2l + 1 and 1 + scale of the next layer's first norm
  // for its 4 columns, ahead of the polls
  const bool ep_wave = wave == 1;
  const bool next_g = l + 1 < L;  // the last layer's output feeds the final norm only
  // (unset in the other waves, which never read them: a zero there would be a register write
  // that waits for o_proj's loads into the same registers and the flag stores behind them)
  f32x4 g4, s14;
  if (ep_wave) {
    g4 = *reinterpret_cast<const f32x4*>(a.table + ((size_t)s * NN + 2 * l + 1) * kModW + 2 * kWidth + col + ec);
    if (next_g) s14 = *reinterpret_cast<const f32x4*>(a.table_s1 + ((size_t)s * NN + 2 * l + 2) * kModW + col + ec);
  }
  // copy wave, ahead of the polls: the next layer's qkv tiles (this layer's gate_up MFMA is done)
  down_next_qkv_copies(a, s, l, smem);
  PHASE_TS(s, l, PH, 1);
  // every gate_up item: the m-tile's rows over the whole K
  if (!wait_flags(a, flag_base(a, s, l, kPhGu), kGuItems, sy)) {
    consume(wf, g4, s14);
    return false;
  }
  PHASE_TS(s, l, PH, 2);
  const int r = 16 * mq + r16;
  const u16* hres = a.hmid + slw * (size_t)R * kWidth;
  uint2 hold = {0u, 0u};
  if (ep_wave && r16 < nrow) hold = *reinterpret_cast<const uint2*>(hres + afrag_index(r, col + ec, kWidth / 32));
  float* red = smem + kLdsWork;  // [4 waves][64 lanes][4]
  {
    const brsrc ra = make_rsrc(a.act + slw * (size_t)R * kMlp, (size_t)R * kMlp * 2);
    bf16x8 af[KQ];
#pragma unroll
    for (int s2 = 0; s2 < KQ; ++s2)
      buf_frag(af[s2], ra, r16 < nrow ? (int)((afrag_offset(mq, kq * KQ + s2, KSTEPS) + lane * 8) * 2) : kOob);
    if (wave == 0) load_w();
    sched_fence();
    f32x4 acc[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < KQ; ++s2) acc[s2 % NCH] = mfma16x16x32(wf[s2], af[s2], acc[s2 % NCH]);
    *reinterpret_cast<f32x4*>(red + ((size_t)kq * 64 + lane) * 4) = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  PHASE_TS(s, l, PH, 4);
  __syncthreads();
  if (ep_wave) {
    // the quarters in order, then the finisher's epilogue on the lane's row and 4 columns
    const f32x4 y = ((*reinterpret_cast<const f32x4*>(red + (size_t)lane * 4) + *reinterpret_cast<const f32x4*>(red + (size_t)(64 + lane) * 4)) +
                     *reinterpret_cast<const f32x4*>(red + (size_t)(128 + lane) * 4)) +
                    *reinterpret_cast<const f32x4*>(red + (size_t)(192 + lane) * 4);
    const float gate[4] = {round_bf(g4[0]), round_bf(g4[1]), round_bf(g4[2]), round_bf(g4[3])};
    const float s1[4] = {s14[0], s14[1], s14[2], s14[3]};
    float ss = 0.f;
    if (r16 < nrow) {
      u16 hn[4], gn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u16 hb = (u16)((i < 2 ? hold.x : hold.y) >> (16 * (i & 1)));
        const float prod = round_bf(fmul(round_bf(y[i]), gate[i]));
        hn[i] = f2bf(fadd(bf2f(hb), prod));
        const float hf = bf2f(hn[i]);
        gn[i] = f2bf(fmul(hf, s1[i]));
        ss += hf * hf;
      }
      st_bf16x4(a.h + ((size_t)s * (L + 1) + l + 1) * R * kWidth, afrag_index(r, col + ec, kWidth / 32), hn);
      if (next_g) st_bf16x4(a.g + (slw + 1) * (size_t)R * kWidth, afrag_index(r, col + ec, kWidth / 32), gn);
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    // tile-major statistics: the tile's sums of the m-tile's 16 rows (padded rows: zero)
    if (lane < 16) st_f32(a.ss + ((size_t)s * (L + 1) + l + 1) * kTiles * R + (size_t)nt * R + 16 * mq + lane, ss);
  }
  consume(hold, g4, s14);  // (used only by the rows the m-tile has)
  PHASE_TS(s, l, PH, 8);
  publish(a, flag_base(a, s, l, PH) + item, sy.epoch);
  PHASE_TS(s, l, PH, 9);
  return true;
}

// The finishing of phase_down_msplit (the same steps as phase_down_pairs' own): quarter ksp of the
// group finishes samples b0 + ksp, b0 + ksp + 4, ... of the half: it adds the four quarters'
// partials in order and applies the gated residual to both tiles (h, g of the next layer's first
// norm, the tiles' row sums of squares).  s_ss: 256 floats of LDS.
// The finisher thread's static operands (gate, 1 + scale of its 8 columns) and the residual rows of
// its first sample, loaded before the quarter flags' wait (they depend on nothing this phase makes).
struct DownFinishPre {
  float gate[8], s1[8];
  u16x8 hold0;
};
__device__ __forceinline__ void down_finish_prefetch(KArgs& a, int s, int l, int nt0, int ksp, int b0, int b1, bool next_g, int NN,
                                                     DownFinishPre& pre) {
  const int L = a.depth, R = a.R;
  const int tid = phase_tid();
  const int ft = tid >> 7, frow = tid & 63, fc0 = ((tid >> 6) & 1) * 8;
  const int col = (nt0 + ft) * 16;
  const size_t slw = (size_t)s * L + l;
  const float* gmod = a.table + ((size_t)s * NN + 2 * l + 1) * kModW + 2 * kWidth + col + fc0;
  const float* smod = a.table_s1 + ((size_t)s * NN + 2 * l + 2) * kModW + col + fc0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pre.gate[i] = gmod[i];
    pre.s1[i] = next_g ? smod[i] : 0.f;
  }
  pre.hold0 = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
  const int b = b0 + ksp;
  if (b < b1 && frow < kHorizon)
    pre.hold0 = *reinterpret_cast<const u16x8*>(a.hmid + slw * (size_t)R * kWidth + afrag_index(b * kRowsPerSample + frow, col + fc0, kWidth / 32));
}
__device__ __forceinline__ void down_pairs_finish(KArgs& a, int s, int l, float* s_ss, int nt0, int ksp, int b0, int b1, bool next_g,
                                                  const DownFinishPre& pre) {
  const int L = a.depth, R = a.R;
  const int tid = phase_tid();
  const size_t slw = (size_t)s * L + l;
  const float* dpart = a.dpart + slw * (size_t)kKSplit * kTiles * R * 16;
  {
    const int ft = tid >> 7, frow = tid & 63, fc0 = ((tid >> 6) & 1) * 8;
    const int col = (nt0 + ft) * 16;
    const u16* hres = a.hmid + slw * (size_t)R * kWidth;
    u16* hout = a.h + ((size_t)s * (L + 1) + l + 1) * R * kWidth;
    u16* gout = a.g + (slw + 1) * (size_t)R * kWidth;  // slice (s, l + 1); unused after the last layer
    float* rout = a.ss + ((size_t)s * (L + 1) + l + 1) * kTiles * R;
    float gate[8], s1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gate[i] = round_bf(pre.gate[i]);
      s1[i] = pre.s1[i];
    }
    for (int b = b0 + ksp; b < b1; b += kKSplit) {
      const int r = b * kRowsPerSample + frow;
      float ss = 0.f;
      if (frow < kHorizon) {
        float pv[kKSplit][8];
#pragma unroll
        for (int q = 0; q < kKSplit; ++q) {
          const float* pp = dpart + (((size_t)q * kTiles + nt0 + ft) * R + r) * 16 + fc0;
          const float4 v0 = *reinterpret_cast<const float4*>(pp), v1 = *reinterpret_cast<const float4*>(pp + 4);
          pv[q][0] = v0.x, pv[q][1] = v0.y, pv[q][2] = v0.z, pv[q][3] = v0.w;
          pv[q][4] = v1.x, pv[q][5] = v1.y, pv[q][6] = v1.z, pv[q][7] = v1.w;
        }
        const u16x8 hold = b == b0 + ksp ? pre.hold0 : *reinterpret_cast<const u16x8*>(hres + afrag_index(r, col + fc0, kWidth / 32));
        u16 hn[8], gn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float y = ((pv[0][i] + pv[1][i]) + pv[2][i]) + pv[3][i];
          const float prod = round_bf(fmul(round_bf(y), gate[i]));
          hn[i] = f2bf(fadd(bf2f(hold[i]), prod));
          const float hf = bf2f(hn[i]);
          gn[i] = f2bf(fmul(hf, s1[i]));
          ss += hf * hf;
        }
        st_bf16x8(hout, afrag_index(r, col + fc0, kWidth / 32), hn);
        if (next_g) st_bf16x8(gout, afrag_index(r, col + fc0, kWidth / 32), gn);
      }
      s_ss[(ft * 2 + (fc0 >> 3)) * 64 + frow] = ss;
      __syncthreads();
      // tile-major statistics: each tile's sums of the sample's 64 rows (one 256-byte run per tile)
      if (tid < 128) {
        const int t = tid >> 6, rw = tid & 63;
        st_f32(rout + (size_t)(nt0 + t) * R + b * kRowsPerSample + rw, s_ss[(t * 2) * 64 + rw] + s_ss[(t * 2 + 1) * 64 + rw]);
      }
      __syncthreads();  // s_ss is reused by the next sample
    }
  }
}

// =============================================================================================
// down_proj at B > 1: two tiles (nt0 = 2g from region B, nt1 = 2g + 1 from registers) and one K
// quarter for the samples [b0, b1) of half h (workgroup 64 q + 32 h + g, see down_item).  Every
// quarter stores its partials of both tiles and flags them for the group (the four quarters run on
// one XCD); then quarter q finishes samples b0 + q, b0 + q + 4, ... of the half: it adds the four
// quarters in order and applies the gated residual (modeling_gemma.py:231-249, 511) to both tiles.  Its
// flag (index 4 (g + 32 h) + q) covers both tiles and those samples, so the next phase waits for
// 256 flags.
// =============================================================================================
template <bool G>
__device__ bool phase_down_pairs(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kMlp / 32;
  constexpr int KQ = KSTEPS / kKSplit, KSW = (KQ + kCompWaves - 1) / kCompWaves, TS = 33;
  constexpr int PH = kPhDown, NG = kTiles / 2;
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int item = wg_id();
  PHASE_TS(s, l, PH, 0);
  // copy wave: with grouped attention this layer's down_proj weights were copied to region B at
  // gate_up; they have landed (read after the polls' barrier)
  if (attn_grouped<G>(a) && copy_wave()) wait_vmcnt<0>();
  // copy wave, ahead of the polls: the next layer's qkv tiles (this layer's gate_up MFMA is done)
  {
    int ln;
    if (next_layer(a, s, l, &ln)) {
      copy_norm_w<kModeQkv, 0, 32, G>(a, ln, 0, smem);
      copy_norm_w<kModeQkv, 0, 31, G>(a, ln, 1, smem);
    }
  }
  if (item >= kTiles * kKSplit) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const bool comp = tid < kCompThreads;
  int nt0, ksp, half;
  down_item(a, &nt0, &ksp, &half);
  const int grp = nt0 / 2;
  const int bh = (a.batch + 1) / 2, b0 = half * bh, b1 = b0 + bh < a.batch ? b0 + bh : a.batch;
  const int kw0 = wave * KSW;  // this wave's k-steps in the quarter: [kw0, kw0 + KSW) clipped to KQ
  const size_t slw = (size_t)s * L + l;
  const bool next_g = l + 1 < L;  // the last layer's output feeds the final norm only
  // the second tile's quarter: waves 1 and 2 ahead of the polls, wave 0 after them
  const u16* wl = a.wpack + (size_t)l * kLayerElems + kOffDown;
  bf16x8 w1[KSW];
  auto load_w1 = [&]() {
#pragma unroll
    for (int s2 = 0; s2 < KSW; ++s2) {
      const int kc = kw0 + s2 < KQ ? kw0 + s2 : KQ - 1;  // the surplus step multiplies zeros
      w1[s2] = *reinterpret_cast<const bf16x8*>(wl + ((size_t)(nt0 + 1) * KSTEPS + ksp * KQ + kc) * 512 + lane * 8);
    }
  };
  if (wave == 1 || wave == 2) load_w1();
  PHASE_TS(s, l, PH, 1);
  // the gate_up items of this quarter's activation columns for this half's samples
  // (phase_gateup_msplit: item w computes pair w for every sample)
  if (!(gu_msplit<G>(a) ? wait_flags(a, flag_base(a, s, l, kPhGu) + ksp * 64, 64, sy)
          : wait_flags(a, flag_base(a, s, l, kPhGu) + half * (kGuItems / 2) + ksp * 32, 32, sy)))
    return false;
  PHASE_TS(s, l, PH, 2);
  if (wave == 0) load_w1();
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsB);  // the first tile's K-quarter fragments
  const u16* act = a.act + slw * (size_t)R * kMlp;
  float* dpart = a.dpart + slw * (size_t)kKSplit * kTiles * R * 16;  // [quarter][tile][row][16]
  float* red = smem + kLdsWork;
  float* T = red + kCompWaves * 4 * 2 * 256;  // [64][TS]: the two tiles side by side
  const int r16 = lane & 15;
  const brsrc rsrc_a = make_rsrc(act, (size_t)R * KSTEPS * 32 * 2);
  for (int b = b0; b < b1; ++b) {
    if (comp) {
      bf16x8 af[4][KSW];
#pragma unroll
      for (int s2 = 0; s2 < KSW; ++s2)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const bool ok = r16 < kHorizon - mt * 16 && kw0 + s2 < KQ;
          buf_frag(af[mt][s2], rsrc_a, ok ? (int)((afrag_offset(b * 4 + mt, ksp * KQ + kw0 + s2, KSTEPS) + lane * 8) * 2) : kOob);
        }
      sched_fence();
      f32x4 acc[4][2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      mfma_steps<KSW, 2, 0, 4>(acc, af, [&](int t, int s2) {
        if (t == 1) return w1[s2];
        const int kc = kw0 + s2 < KQ ? kw0 + s2 : KQ - 1;
        return *reinterpret_cast<const bf16x8*>(lw + (size_t)kc * 512 + lane * 8);
      });
      store_wave_partials<4, 2>(red, acc, wave, lane);
    }
    __syncthreads();
    reduce_to_tile<4, 2, TS>(red, T);
    __syncthreads();
    // partials [quarter][tile][row][16] of both tiles (every quarter's: the finishers reload them);
    // compute waves only, whose stores publish_local waits for
    for (int e = tid; comp && e < 512; e += kCompThreads) {
      const int t = e >> 8, row = (e >> 2) & 63, q4 = e & 3;
      const float* tr = T + row * TS + t * 16 + 4 * q4;
      st_l2_16(dpart, (uint32_t)(((((size_t)ksp * kTiles + nt0 + t) * R + b * kRowsPerSample + row) * 16 + 4 * q4) * 4),
               u32x4{__float_as_uint(tr[0]), __float_as_uint(tr[1]), __float_as_uint(tr[2]), __float_as_uint(tr[3])});
    }
    __syncthreads();  // T is reused by the next sample
  }
  PHASE_TS(s, l, PH, 5);
  unsigned* fl = flag_base(a, s, l, PH);
  unsigned* fpart = fl + kPartFlags + 4 * (grp + NG * half);
  // this quarter's partials are in this XCD's L2: flag them for the group (all four quarters run on
  // this XCD), then wait for the other three; quarter q finishes samples b0 + q, b0 + q + 4, ...
  publish_local(a, fpart + ksp, sy.epoch);
  if (!wait_flags(a, fpart, kKSplit, sy)) return false;
  PHASE_TS(s, l, PH, 7);
  {
    const int ft = tid >> 7, frow = tid & 63, fc0 = ((tid >> 6) & 1) * 8;
    const int col = (nt0 + ft) * 16;
    const u16* hres = a.hmid + slw * (size_t)R * kWidth;
    u16* hout = a.h + ((size_t)s * (L + 1) + l + 1) * R * kWidth;
    u16* gout = a.g + (slw + 1) * (size_t)R * kWidth;  // slice (s, l + 1); unused after the last layer
    float* rout = a.ss + ((size_t)s * (L + 1) + l + 1) * kTiles * R;
    const float* gmod = a.table + ((size_t)s * NN + 2 * l + 1) * kModW + 2 * kWidth + col + fc0;
    const float* smod = a.table_s1 + ((size_t)s * NN + 2 * l + 2) * kModW + col + fc0;
    float gate[8], s1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gate[i] = round_bf(gmod[i]);
      if (next_g) s1[i] = smod[i];
    }
    float* s_ss = T;  // [2 tiles][2 halves][64 rows]
    for (int b = b0 + ksp; b < b1; b += kKSplit) {
      const int r = b * kRowsPerSample + frow;
      float ss = 0.f;
      if (frow < kHorizon) {
        float pv[kKSplit][8];
#pragma unroll
        for (int q = 0; q < kKSplit; ++q) {
          const float* pp = dpart + (((size_t)q * kTiles + nt0 + ft) * R + r) * 16 + fc0;
          const float4 v0 = *reinterpret_cast<const float4*>(pp), v1 = *reinterpret_cast<const float4*>(pp + 4);
          pv[q][0] = v0.x, pv[q][1] = v0.y, pv[q][2] = v0.z, pv[q][3] = v0.w;
          pv[q][4] = v1.x, pv[q][5] = v1.y, pv[q][6] = v1.z, pv[q][7] = v1.w;
        }
        const u16x8 hold = *reinterpret_cast<const u16x8*>(hres + afrag_index(r, col + fc0, kWidth / 32));
        u16 hn[8], gn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float y = ((pv[0][i] + pv[1][i]) + pv[2][i]) + pv[3][i];
          const float prod = round_bf(fmul(round_bf(y), gate[i]));
          hn[i] = f2bf(fadd(bf2f(hold[i]), prod));
          const float hf = bf2f(hn[i]);
          gn[i] = f2bf(fmul(hf, s1[i]));
          ss += hf * hf;
        }
        st_bf16x8(hout, afrag_index(r, col + fc0, kWidth / 32), hn);
        if (next_g) st_bf16x8(gout, afrag_index(r, col + fc0, kWidth / 32), gn);
      }
      s_ss[(ft * 2 + (fc0 >> 3)) * 64 + frow] = ss;
      __syncthreads();
      // tile-major statistics: each tile's sums of the sample's 64 rows (one 256-byte run per tile)
      if (tid < 128) {
        const int t = tid >> 6, rw = tid & 63;
        st_f32(rout + (size_t)(nt0 + t) * R + b * kRowsPerSample + rw, s_ss[(t * 2) * 64 + rw] + s_ss[(t * 2 + 1) * 64 + rw]);
      }
      __syncthreads();  // s_ss is reused by the next sample
    }
  }
  PHASE_TS(s, l, PH, 8);
  publish(a, fl + (grp + NG * half) * kKSplit + ksp, sy.epoch, true);  // the copy wave stored rows too
  PHASE_TS(s, l, PH, 9);
  return true;
}

// =============================================================================================
// down_proj of kernel instance 2, split by rows: the items of phase_down_pairs (tiles nt0, nt0 + 1,
// K quarter q, sample half h); the first tile's quarter in region B, the second's in the working
// area (copied there at gate_up), so wave j takes sample j of the half over the quarter's whole K
// with both tiles, as phase_gateup_msplit, and stores its partials straight from the accumulators
// (a lane: columns 4g .. 4g+3 of one row).  The finishers are phase_down_pairs'.
// =============================================================================================
__device__ bool phase_down_msplit(KArgs& a, int s, int l, float* smem, Sync sy) {
  constexpr int KSTEPS = kMlp / 32, KQ = KSTEPS / kKSplit;
  constexpr int PH = kPhDown, NG = kTiles / 2;
  static_assert(KQ == kGuChunks * kGuCk, "a K quarter is one row-split pass");
  const int L = a.depth, NN = 2 * L + 1, R = a.R;
  const int item = wg_id();
  PHASE_TS(s, l, PH, 0);
  // copy wave: this layer's down_proj weights (region B, the working area) have landed (read after
  // the polls' barrier); then, ahead of the polls, the next layer's qkv tiles
  if (copy_wave()) wait_vmcnt<0>();
  {
    int ln;
    if (next_layer(a, s, l, &ln)) {
      copy_norm_w<kModeQkv, 0, 32, true>(a, ln, 0, smem);
      copy_norm_w<kModeQkv, 0, 31, true>(a, ln, 1, smem);
    }
  }
  if (item >= kTiles * kKSplit) return true;
  const int tid = phase_tid(), lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  int nt0, ksp, half;
  down_item(a, &nt0, &ksp, &half);
  const int grp = nt0 / 2;
  const int bh = (a.batch + 1) / 2, b0 = half * bh, b1 = b0 + bh < a.batch ? b0 + bh : a.batch;
  const size_t slw = (size_t)s * L + l;
  const bool next_g = l + 1 < L;  // the last layer's output feeds the final norm only
  PHASE_TS(s, l, PH, 1);
  if (!wait_flags(a, flag_base(a, s, l, kPhGu) + ksp * 64, 64, sy)) return false;  // gate_up items 64 q ..
  PHASE_TS(s, l, PH, 2);
  const u16* lw = reinterpret_cast<const u16*>(smem + kLdsB);  // tile nt0's quarter, then nt0 + 1's
  const brsrc rg = make_rsrc(a.act + slw * (size_t)R * kMlp, (size_t)R * kMlp * 2);
  // the finisher's operands (the residual rows are o_proj's, which the gate_up flags imply)
  DownFinishPre fpre;
  down_finish_prefetch(a, s, l, nt0, ksp, b0, b1, next_g, NN, fpre);
  float* dpart = a.dpart + slw * (size_t)kKSplit * kTiles * R * 16;  // [quarter][tile][row][16]
  bf16x8 A[4][4][kGuCk];
  const int bf = b0 + wave;
#pragma unroll
  for (int c = 0; c < kGuAhead; ++c) gu_load_chunk<KSTEPS>(A[c], rg, bf, bf < b1, c, lane, ksp * KQ);
  sched_fence();
  for (int b = bf; b < b1; b += 4) {
    const int bn = b + 4;
    const bool ok_n = bn < b1;
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc0[mt] = acc1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kGuChunks; ++c) {
      if (c + kGuAhead < kGuChunks) gu_load_chunk<KSTEPS>(A[(c + kGuAhead) % 4], rg, b, true, c + kGuAhead, lane, ksp * KQ);
      else gu_load_chunk<KSTEPS>(A[(c + kGuAhead) % 4], rg, bn, ok_n, c + kGuAhead - kGuChunks, lane, ksp * KQ);
      sched_fence();
      gu_mfma_chunk(acc0, acc1, A[c % 4], lw, c, lane);
    }
    // partials of both tiles (into this XCD's L2, where the group's finishers read them)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = mt * 16 + r16;
      if (row < kHorizon) {
        const size_t r = (size_t)b * kRowsPerSample + row;
        st_l2_16(dpart, (uint32_t)(((((size_t)ksp * kTiles + nt0) * R + r) * 16 + 4 * g) * 4),
                 u32x4{__float_as_uint(acc0[mt][0]), __float_as_uint(acc0[mt][1]), __float_as_uint(acc0[mt][2]), __float_as_uint(acc0[mt][3])});
        st_l2_16(dpart, (uint32_t)(((((size_t)ksp * kTiles + nt0 + 1) * R + r) * 16 + 4 * g) * 4),
                 u32x4{__float_as_uint(acc1[mt][0]), __float_as_uint(acc1[mt][1]), __float_as_uint(acc1[mt][2]), __float_as_uint(acc1[mt][3])});
      }
    }
  }
  PHASE_TS(s, l, PH, 5);
  unsigned* fl = flag_base(a, s, l, PH);
  unsigned* fpart = fl + kPartFlags + 4 * (grp + NG * half);
  if (copy_wave()) wait_stores();  // publish_local waits for the compute waves' stores only
  publish_local(a, fpart + ksp, sy.epoch);
  if (!wait_flags(a, fpart, kKSplit, sy)) return false;
  PHASE_TS(s, l, PH, 7);
  down_pairs_finish(a, s, l, smem + kLdsWork + kDownW1Floats, nt0, ksp, b0, b1, next_g, fpre);
  PHASE_TS(s, l, PH, 8);
  publish(a, fl + (grp + NG * half) * kKSplit + ksp, sy.epoch, true);  // every wave stored rows
  PHASE_TS(s, l, PH, 9);
  return true;
}

// =============================================================================================
// the kernel
// =============================================================================================
static_assert(64 + 32 + 192 + kCompWaves * 4 * 2 * 256 + 64 * 33 <= kWorkFloats, "norm GEMM working area");
static_assert(64 + 64 + 192 + kCompWaves * 4 * 2 * 256 + 64 * 33 <= kWorkFloats, "gate_up pairs working area");
static_assert(64 + 64 + 192 + kCompWaves * 2 * 2 * 256 + 32 * 33 <= kWorkFloats, "qkv pairs working area");
static_assert(kCompWaves * 4 * 256 + 64 * 17 + 128 <= kWorkFloats, "residual working area");
static_assert(kCompWaves * 4 * 2 * 256 + 64 * 33 <= kWorkFloats, "down_proj pairs working area");
static_assert(2048 + 2 * 3072 + 128 <= kWorkFloats, "attention working area");
static_assert(kWidth + 2 * kActDim + 4 + kCompThreads + kWidth <= kWorkFloats, "step boundary working area");
static_assert(kDownW1Floats + 256 <= kWorkFloatsBatched, "row-split down_proj: second tile + finisher sums");

// Three instances of the kernel: G = false for one sample, G = true for batches; I = the instance
// number (0, 1, 2), instance 2 (batches of kRowSplitMinBatch and more) alone containing the
// row-split qkv / gate_up / down_proj phases and the grouped attention.  Each is compiled in a
// translation unit of its own: inlined into one module, the batched code changed the one-sample
// kernel's register allocation (measured +2-3.5 % per one-sample predict), and the batch paths each
// other's (+1-1.5 %).
template <bool G, int I>
__global__ __launch_bounds__(kThreads, 1) void denoise_loop_kernel(MegaArgs args) {
  __shared__ __align__(16) float smem[G ? kLdsFloatsBatched : kLdsFloats];
  __shared__ int s_flag;
  // this launch's epoch: one past the last finished launch's
  const Sync sy{(unsigned)__builtin_amdgcn_readfirstlane(ld_u32(args.err + kCtlEpoch)) + 1u, &s_flag};
  PHASE_TS_INIT();
  // the copy wave: step 0, layer 0 qkv weights (one sample: the first tile in region B)
  if constexpr (G) copy_norm_w<kModeQkv, 0, 32, G>(kargs(), 0, 0, smem);
  else copy_qkv_tile0(kargs(), 0, smem);
  copy_norm_w<kModeQkv, 0, 31, G>(kargs(), 0, 1, smem);
  bool ok = true;
  for (int s = 0; s <= kargs().steps && ok; ++s) {
    ok = phase_io<G>(kargs(), s, smem, sy);
    if (!ok || s == kargs().steps) break;
    for (int l = 0; l < kargs().depth && ok; ++l) {
      ok = (qkv_msplit<G>() ? phase_qkv_msplit(kargs(), s, l, smem, sy)
            : G             ? phase_qkv_pairs(kargs(), s, l, smem, sy)
                            : phase_qkv1<G>(kargs(), s, l, smem, sy)) &&
           phase_attn<G>(kargs(), s, l, smem, sy) &&
           (G && PI05_INSTANCE_GROUPED ? (kargs().batch <= 4 ? phase_oproj_msplit<4>(kargs(), s, l, smem, sy)
                                                             : phase_oproj_msplit<2>(kargs(), s, l, smem, sy))
            : G                         ? phase_oproj_pairs(kargs(), s, l, smem, sy)
                                        : phase_oproj(kargs(), s, l, smem, sy)) &&
           (G ? (gu_msplit<G>(kargs()) ? phase_gateup_msplit(kargs(), s, l, smem, sy) : phase_gateup_pairs4(kargs(), s, l, smem, sy))
              : phase_gateup_rows(kargs(), s, l, smem, sy)) &&
           (G && PI05_INSTANCE_GROUPED ? phase_down_msplit(kargs(), s, l, smem, sy)
            : G                         ? phase_down_pairs<G>(kargs(), s, l, smem, sy)
                                        : phase_down_rows(kargs(), s, l, smem, sy));
    }
  }
  // no direct-to-LDS copy may still be in flight when the workgroup's LDS is released
  wait_vmcnt<0>();
  PHASE_TS_FLUSH();
  leave_launch(kargs(), sy);
}

#if PI05_PERSISTENT_INSTANCE == 1
const void* denoise_loop_kernel_batched() { return reinterpret_cast<const void*>(denoise_loop_kernel<true, 1>); }
#elif PI05_PERSISTENT_INSTANCE == 2
const void* denoise_loop_kernel_grouped() { return reinterpret_cast<const void*>(denoise_loop_kernel<true, 2>); }
#else
const void* denoise_loop_kernel_batched();  // instance 1
const void* denoise_loop_kernel_grouped();  // instance 2

const void* denoise_loop_kernel_ptr(int batch) {
  return batch >= kRowSplitMinBatch ? denoise_loop_kernel_grouped()
         : batch > 1                 ? denoise_loop_kernel_batched()
                                     : reinterpret_cast<const void*>(denoise_loop_kernel<false, 0>);
}

hipError_t launch_denoise_loop(const MegaArgs& a, int grid, hipStream_t st) {
  void* args[] = {const_cast<MegaArgs*>(&a)};
  return hipLaunchCooperativeKernel(denoise_loop_kernel_ptr(a.batch), dim3(grid), dim3(kThreads), args, 0, st);
}

int denoise_loop_threads() { return kThreads; }

// =============================================================================================
// shift . W^T table (built by pi05_refresh_weights): one wave per (layer, output column), lane
// k-range [16 lane, 16 lane + 16), all steps.
// =============================================================================================
__global__ __launch_bounds__(256) void shift_bias_kernel(ShiftBiasArgs a) {
  const int l = blockIdx.y;
  const int j = (unsigned)wg_id() * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (j >= kBiasCols) return;
  constexpr int KSTEPS = kWidth / 32;
  const u16* wl = a.wpack + (size_t)l * kLayerElems;
  const u16* tile;
  int norm;
  if (j < kQkvCols) {
    tile = wl + kOffQkv + (size_t)(j >> 4) * KSTEPS * 512;
    norm = 2 * l;
  } else if (j < kQkvCols + kMlp) {
    tile = wl + kOffGate + (size_t)((j - kQkvCols) >> 4) * KSTEPS * 512;
    norm = 2 * l + 1;
  } else {
    tile = wl + kOffUp + (size_t)((j - kQkvCols - kMlp) >> 4) * KSTEPS * 512;
    norm = 2 * l + 1;
  }
  const int n = j & 15;
  // k = 16 lane + e: fragment ks = lane / 2, lane group (k % 32) / 8 = 2 (lane % 2) + e / 8
  const int ks = lane >> 1, g0 = 2 * (lane & 1);
  const u16x8 w0 = *reinterpret_cast<const u16x8*>(tile + (size_t)ks * 512 + ((g0 * 16) + n) * 8);
  const u16x8 w1 = *reinterpret_cast<const u16x8*>(tile + (size_t)ks * 512 + (((g0 + 1) * 16) + n) * 8);
  float wf[16];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wf[e] = bf2f(w0[e]);
    wf[8 + e] = bf2f(w1[e]);
  }
  const int NN = 2 * a.depth + 1;
  for (int s = 0; s < a.steps; ++s) {
    const float* sh = a.table + ((size_t)s * NN + norm) * kModW + kWidth + lane * 16;
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(sh[e], wf[e], acc);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) a.bias[((size_t)s * a.depth + l) * kBiasCols + j] = acc;
  }
}

hipError_t launch_shift_bias(const ShiftBiasArgs& a, hipStream_t st) {
  shift_bias_kernel<<<dim3((kBiasCols + 3) / 4, a.depth), 256, 0, st>>>(a);
  return hipGetLastError();
}

#endif  // PI05_PERSISTENT_INSTANCE

}  // namespace pi05

#ifdef PI05_PHASE_TIMESTAMPS
// Phase timestamps of the last launch to the host / zeroed before the launch to be recorded
// (profiling builds only).  Each instance has its own array; the one that did not run holds zeros.
#if PI05_PERSISTENT_INSTANCE == 1
int pi05_phase_ts_copy_batched(unsigned long long* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(pi05::pi05_phase_ts), sizeof(pi05::pi05_phase_ts), 0, hipMemcpyDeviceToHost);
}
int pi05_phase_ts_clear_batched(const unsigned long long* zeros) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(pi05::pi05_phase_ts), zeros, sizeof(pi05::pi05_phase_ts), 0, hipMemcpyHostToDevice);
}
#elif PI05_PERSISTENT_INSTANCE == 2
int pi05_phase_ts_copy_grouped(unsigned long long* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(pi05::pi05_phase_ts), sizeof(pi05::pi05_phase_ts), 0, hipMemcpyDeviceToHost);
}
int pi05_phase_ts_clear_grouped(const unsigned long long* zeros) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(pi05::pi05_phase_ts), zeros, sizeof(pi05::pi05_phase_ts), 0, hipMemcpyHostToDevice);
}
#else
int pi05_phase_ts_copy_batched(unsigned long long* host);
int pi05_phase_ts_clear_batched(const unsigned long long* zeros);
int pi05_phase_ts_copy_grouped(unsigned long long* host);
int pi05_phase_ts_clear_grouped(const unsigned long long* zeros);
extern "C" int pi05_debug_phase_timestamps(unsigned long long* host) {
  constexpr size_t n = sizeof(pi05::pi05_phase_ts) / sizeof(unsigned long long);
  static unsigned long long other[n];
  int rc = (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(pi05::pi05_phase_ts), sizeof(pi05::pi05_phase_ts), 0, hipMemcpyDeviceToHost);
  for (int inst = 1; inst <= 2 && rc == 0; ++inst) {
    rc = inst == 1 ? pi05_phase_ts_copy_batched(other) : pi05_phase_ts_copy_grouped(other);
    for (size_t i = 0; rc == 0 && i < n; ++i) host[i] += other[i];
  }
  return rc;
}
extern "C" int pi05_debug_phase_timestamps_clear(void) {
  static unsigned long long zeros[sizeof(pi05::pi05_phase_ts) / sizeof(unsigned long long)];
  int rc = (int)hipMemcpyToSymbol(HIP_SYMBOL(pi05::pi05_phase_ts), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
  if (rc == 0) rc = pi05_phase_ts_clear_batched(zeros);
  return rc == 0 ? pi05_phase_ts_clear_grouped(zeros) : rc;
}
#endif
#endif
