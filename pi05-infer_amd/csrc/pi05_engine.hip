// Host side of the gfx950 denoise engine: the C ABI declared in include/pi05_denoise.h.
//
// A context owns every device buffer of one shape signature (B, P, num_steps) and replays the
// whole Euler loop as one hipGraph, so the graph's kernel arguments (all context-owned device
// addresses) never change between predicts.  All argument validation happens before the first
// HIP call of an entry point.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "pi05_denoise.h"
#include "pi05_device.h"
#include "pi05_kernels.h"

using namespace pi05;

namespace {

thread_local std::string g_last_error;

struct LayerBind {
  const void* wq = nullptr;
  const void* wk = nullptr;
  const void* wv = nullptr;
  const void* wo = nullptr;
  const void* wgate = nullptr;
  const void* wup = nullptr;
  const void* wdown = nullptr;
  const float* ln1_w = nullptr;
  const float* ln1_b = nullptr;
  const float* ln2_w = nullptr;
  const float* ln2_b = nullptr;
  bool set = false;
};

struct HeadBind {
  const float* norm_w = nullptr;
  const float* norm_b = nullptr;
  const float* in_w = nullptr;
  const float* in_b = nullptr;
  const float* out_w = nullptr;
  const float* out_b = nullptr;
  const float* tin_w = nullptr;
  const float* tin_b = nullptr;
  const float* tout_w = nullptr;
  const float* tout_b = nullptr;
  bool set = false;
};

// Device buffer plan of one signature (sizes in bytes).  "Common" buffers exist in both
// schedules; the graph schedule keeps one activation set that every kernel overwrites, the
// persistent schedule slices its activations per (Euler step, layer) so that no buffer is read
// before it is written within one launch.
struct Plan {
  int M = 0, S = 0, s_pad = 0, n_norms = 0, rows = 0, nsplit = 1, mgroups = 1;
  // common
  size_t wpack = 0, table = 0, temb = 0, cond = 0, heads = 0, rope = 0, pos = 0, invf = 0, bias = 0;
  // graph schedule
  size_t kv = 0, valid = 0, h = 0, rowss = 0, q = 0, o = 0, act = 0, part = 0, partml = 0, x = 0, trace = 0;
  // persistent schedule
  int s_pre = 0, nsplit_p = 1, nsplit_pad = 4, nbp = 0, nbp_pad = 4, R = 0, fstride = 256;
  size_t p_kv = 0, p_valid = 0, p_h = 0, p_g = 0, p_ss = 0, p_hmid = 0, p_ssmid = 0, p_q = 0, p_suf = 0, p_act = 0;
  size_t p_apart = 0, p_apartml = 0, p_dpart = 0, p_x = 0, p_flags = 0, p_euler = 0;
  size_t common() const { return wpack + 2 * table + temb + 2 * cond + heads + 2 * rope + pos + invf + bias; }
  size_t graph_bytes() const { return 2 * kv + valid + h + rowss + q + o + act + part + 2 * partml + x + trace; }
  size_t persistent_bytes() const {
    return 2 * p_kv + p_valid + p_h + p_g + p_ss + p_hmid + p_g + p_ssmid + 2 * p_q + 2 * p_suf + p_act + p_apart + p_apartml +
           p_dpart + p_x + p_flags + p_euler + 256;
  }
};

// Split-KV factor of the graph schedule: one 32-key block per wave (4 per workgroup), at most 8
// splits; longer prefixes give each wave several blocks instead.
int choose_nsplit(int s_pad) {
  const int nkb = s_pad / 32;
  int ns = (nkb + 3) / 4;
  if (ns < 1) ns = 1;
  if (ns > 8) ns = 8;
  return ns;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

Plan make_plan(const pi05_dims& d) {
  Plan p;
  const size_t L = d.depth, T = d.num_steps;
  p.M = d.batch * kHorizon;
  p.S = d.prefix_len + kHorizon;
  p.s_pad = (p.S + 31) / 32 * 32;
  p.n_norms = 2 * d.depth + 1;
  p.rows = p.M * kHeads;
  p.nsplit = choose_nsplit(p.s_pad);
  p.wpack = L * kLayerElems * 2;
  p.table = T * p.n_norms * kModW * 4;
  p.temb = T * kWidth * 4;
  p.cond = T * kWidth * 4;
  p.heads = ((size_t)kWidth * kActDim * 2 + kWidth + kActDim) * 4;
  p.rope = (size_t)p.M * kHeadDim * 2;
  p.pos = (size_t)p.M * 4;
  p.invf = (size_t)kHalfDim * 4;
  p.bias = T * L * kBiasCols * 4;

  p.kv = L * d.batch * p.s_pad * kHeadDim * 2;
  p.valid = (size_t)d.batch * p.s_pad;
  p.h = (size_t)p.M * kWidth * 2;
  p.rowss = (size_t)kRowSlots * p.M * 4;
  p.q = (size_t)p.M * kHeads * kHeadDim * 2;
  p.o = p.q;
  p.act = (size_t)p.M * kMlp * 2;
  p.part = p.nsplit > 1 ? (size_t)p.nsplit * p.rows * kHeadDim * 4 : 0;
  p.partml = p.nsplit > 1 ? (size_t)p.nsplit * p.rows * 4 : 0;
  p.mgroups = (p.M + 63) / 64;
  p.x = (size_t)p.M * kActDim * 4;
  p.trace = T * p.M * kActDim * 4;

  // persistent: prefix keys padded to a 32-key boundary, then one 64-key block of action keys;
  // split count such that every wave normally owns one 32-key block.  Activation rows are padded
  // to 64 per sample (R rows), attention works on nbp two-token row blocks.
  p.s_pre = (d.prefix_len + 31) / 32 * 32;
  const int nkb = p.s_pre / 32 + 2;
  p.nsplit_p = (nkb + 3) / 4;
  if (p.nsplit_p > kMaxAttnSplits) p.nsplit_p = kMaxAttnSplits;
  {
    // large batches: when the split items would take more than 4 passes of the 256 workgroups,
    // use just enough splits to fill them once -- each split item has a fixed cost (query load,
    // wave merge, partial store, publish) that more keys per item amortize (B = 8, P = 968:
    // 2 splits, 25.9 ms/predict against 27.1 with 9; at B <= 2 and at P = 3272 fewer splits are
    // slower, so the rule leaves them alone)
    const int nbp = d.batch * (kHorizon / 2), fill = (256 + nbp - 1) / nbp;
    if (nbp * p.nsplit_p > 4 * 256 && p.nsplit_p > fill) p.nsplit_p = fill;
    // batches of kAttnGroupMinBatch and more: grouped items (4 row blocks each), one pass of the grid
    if (d.batch >= kAttnGroupMinBatch) p.nsplit_p = attn_group_splits(d.batch, nkb);
  }
  p.nsplit_pad = (p.nsplit_p + 3) / 4 * 4;
  p.R = 64 * d.batch;
  p.nbp = d.batch * (kHorizon / 2);
  p.nbp_pad = (p.nbp + 3) / 4 * 4;
  const size_t R = p.R;
  // flag words per phase instance: the largest item count of any phase (io rows, attention split
  // and merge flags, 256 GEMM items), 16-byte aligned sub-ranges
  size_t fw = 256;
  fw = std::max(fw, (size_t)p.M);
  fw = std::max(fw, (size_t)p.nbp * p.nsplit_pad);
  fw = std::max(fw, (size_t)4 * p.nbp_pad);
  fw = std::max(fw, (size_t)256 + 4 * (kWidth / 16));  // o_proj / down_proj K-quarter flags
  p.fstride = (int)round_up(fw, 256);
  p.p_kv = L * d.batch * p.s_pre * kHeadDim * 2;
  p.p_valid = round_up((size_t)d.batch * (p.s_pre + 64), 256);
  p.p_h = T * (L + 1) * R * kWidth * 2;
  p.p_g = T * L * R * kWidth * 2;
  p.p_ss = T * (L + 1) * R * kRowSlots * 4;
  p.p_hmid = T * L * R * kWidth * 2;
  p.p_ssmid = T * L * R * kRowSlots * 4;
  p.p_q = T * L * R * kHeads * kHeadDim * 2;
  p.p_suf = T * L * d.batch * 64 * kHeadDim * 2;
  p.p_act = T * L * R * kMlp * 2;
  p.p_apart = T * L * p.nsplit_p * p.nbp * 16 * kHeadDim * 4;
  p.p_apartml = round_up(T * L * p.nsplit_p * p.nbp * 32 * 4, 256);
  p.p_dpart = T * L * 4 * (kWidth / 16) * R * 16 * 4;
  p.p_x = round_up(T * p.M * kActDim * 4, 256);
  // 7 phases per (step, layer), 8 replicas each; 1 KiB of slack for the 16-byte flag loads past
  // a range's end
  p.p_flags = (T + 1) * (L + 1) * 7 * kFlagCopies * (size_t)p.fstride * 4 + 1024;
  p.p_euler = round_up(T * 4 * 4, 256);
  return p;
}

// The persistent kernel addresses each per-(step, layer) slice through a buffer resource whose
// byte offset is a 32-bit VGPR (signed in its bounds arithmetic): the largest such window of a
// plan must stay below 2^31 bytes.  The windows, as the kernel builds them: the A operands of the
// norm GEMMs (g / gmid rows) and of down_proj (the GeGLU rows), the query and K/V-tail stores, the
// attention split partials and their (m, l) pairs, the down K-quarter partials, the row
// statistics, and one phase instance's replicated flags.
size_t max_offset_window(const Plan& p, const pi05_dims& d) {
  const size_t R = p.R;
  const size_t w[] = {
      R * kWidth * 2,                                         // g, gmid, h slices
      R * kMlp * 2,                                           // act slice
      R * kQRowsPerTok * kHeadDim * 2,                        // q slice
      (size_t)d.batch * 64 * kHeadDim * 2,                    // K/V tail slice
      (size_t)p.nsplit_p * p.nbp * 16 * kHeadDim * 4,         // attention split partials
      (size_t)p.nsplit_p * p.nbp * 32 * 4,                    // their (m, l) pairs
      (size_t)4 * (kWidth / 16) * R * 16 * 4,                 // down K-quarter partials
      (size_t)kRowSlots * R * 4,                              // row statistics slice
      (size_t)kFlagCopies * p.fstride * 4,                    // one phase instance's flags
  };
  size_t m = 0;
  for (size_t v : w) m = std::max(m, v);
  return m;
}

bool check_dims_msg(const pi05_dims* d, std::string* msg) {
  char buf[256];
  if (!d) {
    *msg = "dims is NULL";
    return false;
  }
#define REQ(cond, ...)                          \
  do {                                          \
    if (!(cond)) {                              \
      snprintf(buf, sizeof buf, __VA_ARGS__);   \
      *msg = buf;                               \
      return false;                             \
    }                                           \
  } while (0)
  REQ(d->width == kWidth, "width %d unsupported (engine is compiled for %d)", d->width, kWidth);
  REQ(d->num_heads == kHeads, "num_heads %d unsupported (compiled for %d)", d->num_heads, kHeads);
  REQ(d->num_kv_heads == 1, "num_kv_heads %d unsupported (compiled for 1)", d->num_kv_heads);
  REQ(d->head_dim == kHeadDim, "head_dim %d unsupported (compiled for %d)", d->head_dim, kHeadDim);
  REQ(d->mlp_dim == kMlp, "mlp_dim %d unsupported (compiled for %d)", d->mlp_dim, kMlp);
  REQ(d->action_dim == kActDim, "action_dim %d unsupported (compiled for %d)", d->action_dim, kActDim);
  REQ(d->action_horizon == kHorizon, "action_horizon %d unsupported (compiled for %d)", d->action_horizon, kHorizon);
  REQ(d->depth >= 1 && d->depth <= kMaxDepth, "depth %d out of range [1, %d]", d->depth, kMaxDepth);
  REQ(d->batch >= 1 && d->batch <= 64, "batch %d out of range [1, 64]", d->batch);
  REQ(d->prefix_len >= 1 && d->prefix_len <= 16384, "prefix_len %d out of range [1, 16384]", d->prefix_len);
  REQ(d->num_steps >= 1 && d->num_steps <= kMaxSteps, "num_steps %d out of range [1, %d]", d->num_steps, kMaxSteps);
  REQ(std::isfinite(d->rms_eps) && d->rms_eps > 0.f, "rms_eps must be a positive finite float");
  REQ(std::isfinite(d->rope_theta) && d->rope_theta > 1.f, "rope_theta must be > 1");
  REQ(std::isfinite(d->time_min_period) && d->time_min_period > 0.0 && std::isfinite(d->time_max_period) &&
          d->time_max_period > d->time_min_period,
      "time periods must satisfy 0 < min_period < max_period");
  {
    const size_t win = max_offset_window(make_plan(*d), *d);
    REQ(win < ((size_t)1 << 31), "batch %d x prefix_len %d needs a %zu-byte slice, beyond the kernel's 32-bit offsets", d->batch,
        d->prefix_len, win);
  }
#undef REQ
  return true;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Euler schedule linspace(1, 1/N, N) ++ [0] as the elementwise fp32 GPU linspace evaluates it
// (engine.py:425-426): step = (end - start) / (N - 1); i < N/2: start + step*i, else
// end - step*(N - 1 - i).
std::vector<float> euler_schedule(int n) {
  std::vector<float> ts(n + 1, 0.f);
  const float start = 1.0f;
  const float end = (float)(1.0 / n);
  if (n == 1) {
    ts[0] = start;
  } else {
    const float step = (end - start) / (float)(n - 1);
    const int half = n / 2;
    for (int i = 0; i < n; ++i) ts[i] = i < half ? start + step * (float)i : end - step * (float)(n - i - 1);
  }
  ts[n] = 0.f;
  return ts;
}

// Sinusoidal timestep embedding in float64, cast to fp32 (pi0_pytorch.py:29-46; the fraction is
// the f64 GPU linspace(0, 1, dim/2)).
void sinusoid(float t, int dim, double min_p, double max_p, float* out) {
  const int half = dim / 2;
  const double step = (1.0 - 0.0) / (double)(half - 1);
  for (int i = 0; i < half; ++i) {
    const double frac = i < half / 2 ? 0.0 + step * (double)i : 1.0 - step * (double)(half - i - 1);
    const double period = min_p * std::pow(max_p / min_p, frac);
    const double scaling = 1.0 / period * 2.0 * M_PI;
    const double arg = scaling * (double)t;
    out[i] = (float)std::sin(arg);
    out[half + i] = (float)std::cos(arg);
  }
}

// RoPE inverse frequencies as transformers computes them in fp32:
// 1 / (theta ** (arange(0, D, 2) / D)), the power rounded to fp32, then the fp32 reciprocal.
void rope_inv_freq(float theta, float* out) {
  for (int i = 0; i < kHalfDim; ++i) {
    const float ex = (float)(2 * i) / (float)kHeadDim;
    const float pw = (float)std::pow((double)theta, (double)ex);
    out[i] = 1.0f / pw;
  }
}

}  // namespace

// Polls before a wait of the persistent kernel gives up (each poll >= ~1 us; a legitimate wait
// spans a few phases, so this is a fault detector, not a performance knob).
constexpr int kDefaultSpinLimit = 1 << 20;

struct pi05_ctx {
  pi05_dims d{};
  Plan plan;
  int device = -1;
  int schedule = PI05_SCHEDULE_PERSISTENT;
  int grid = 0;  // persistent schedule: one workgroup per compute unit
  std::vector<LayerBind> layers;
  HeadBind heads;
  std::vector<float> ts;

  // common
  u16* wpack = nullptr;
  float* table = nullptr;
  float* table_s1 = nullptr;  // table with 1 + scale (persistent kernel's adaRMSNorm operand)
  float* bias = nullptr;      // shift . W^T per (step, layer) (persistent kernel's adaRMSNorm fold)
  float* temb = nullptr;
  float* cond1 = nullptr;
  float* cond = nullptr;
  float* heads_buf = nullptr;  // in_w [W,a] | out_w [a,W] | in_b [W] | out_b [a]
  u16* cos_tab = nullptr;
  u16* sin_tab = nullptr;
  int32_t* positions = nullptr;
  float* inv_freq = nullptr;

  // graph schedule
  u16* kcache = nullptr;
  u16* vcache = nullptr;
  uint8_t* valid = nullptr;
  u16* h = nullptr;
  float* rowss = nullptr;
  u16* q = nullptr;
  u16* o = nullptr;
  u16* act = nullptr;
  float* part = nullptr;
  float* part_m = nullptr;
  float* part_l = nullptr;
  float* x = nullptr;
  float* trace = nullptr;
  hipStream_t cap = nullptr;
  hipGraphExec_t exec[2] = {nullptr, nullptr};

  // persistent schedule
  char* pbase = nullptr;  // one allocation, carved by carve_persistent()
  MegaArgs mega{};
  unsigned* host_err = nullptr;  // pinned host words: launches whose waits timed out, launches misplaced over the XCDs
  unsigned reported = 0;         // the timeout count already reported to the caller
  unsigned reported_placement = 0;  // the placement count already reported
  unsigned xcd_skew = 0;         // test hook (pi05_debug_skew_placement_check)
  int spin_limit = kDefaultSpinLimit;

  bool weights_ready = false;
  bool primed = false;
  std::string err;

  int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    err = buf;
    return code;
  }
  int hip_fail(hipError_t e, const char* what) {
    return fail(PI05_E_HIP, "%s failed: %s", what, hipGetErrorString(e));
  }
};

#define HIPCHK(ctx, expr)                            \
  do {                                               \
    hipError_t e_ = (expr);                          \
    if (e_ != hipSuccess) return (ctx)->hip_fail(e_, #expr); \
  } while (0)

namespace {

float* heads_in_w(pi05_ctx* c) { return c->heads_buf; }
float* heads_out_w(pi05_ctx* c) { return c->heads_buf + (size_t)kWidth * kActDim; }
float* heads_in_b(pi05_ctx* c) { return c->heads_buf + (size_t)kWidth * kActDim * 2; }
float* heads_out_b(pi05_ctx* c) { return heads_in_b(c) + kWidth; }

void free_schedule(pi05_ctx* c) {
  for (auto& e : c->exec)
    if (e) {
      (void)hipGraphExecDestroy(e);
      e = nullptr;
    }
  void** bufs[] = {(void**)&c->kcache, (void**)&c->vcache, (void**)&c->valid, (void**)&c->h, (void**)&c->rowss,
                   (void**)&c->q, (void**)&c->o, (void**)&c->act, (void**)&c->part, (void**)&c->part_m,
                   (void**)&c->part_l, (void**)&c->x, (void**)&c->trace, (void**)&c->pbase};
  for (void** p : bufs)
    if (*p) {
      (void)hipFree(*p);
      *p = nullptr;
    }
  c->mega = MegaArgs{};
  c->primed = false;
}

void free_all(pi05_ctx* c) {
  free_schedule(c);
  void* bufs[] = {c->wpack, c->table, c->table_s1, c->bias, c->temb, c->cond1, c->cond, c->heads_buf, c->cos_tab, c->sin_tab,
                  c->positions, c->inv_freq};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  if (c->host_err) (void)hipHostFree(c->host_err);
  c->host_err = nullptr;
  if (c->cap) (void)hipStreamDestroy(c->cap);
  c->cap = nullptr;
}

template <typename T>
hipError_t dalloc(T** p, size_t bytes) {
  if (bytes == 0) {
    *p = nullptr;
    return hipSuccess;
  }
  void* v = nullptr;
  hipError_t e = hipMalloc(&v, bytes);
  if (e != hipSuccess) return e;
  e = hipMemset(v, 0, bytes);
  *p = reinterpret_cast<T*>(v);
  return e;
}

// Slice the persistent schedule's single allocation (every slice 256-byte aligned) and fill the
// launch-invariant part of the kernel arguments.
void carve_persistent(pi05_ctx* c) {
  const Plan& p = c->plan;
  const pi05_dims& d = c->d;
  char* cur = c->pbase;
  auto take = [&cur](size_t bytes) {
    char* r = cur;
    cur += round_up(bytes, 256);
    return r;
  };
  MegaArgs& a = c->mega;
  a = MegaArgs{};
  a.err = reinterpret_cast<unsigned*>(take(256));
  a.flags = reinterpret_cast<unsigned*>(take(p.p_flags));
  a.flag_bytes = p.p_flags;
  a.fstride = p.fstride;
  a.depth = d.depth;
  a.steps = d.num_steps;
  a.batch = d.batch;
  a.R = p.R;
  a.nbp = p.nbp;
  a.nbp_pad = p.nbp_pad;
  a.nsplit = p.nsplit_p;
  a.nsplit_pad = p.nsplit_pad;
  a.s_pre = p.s_pre;
  a.eps = d.rms_eps;
  a.table = c->table;
  a.table_s1 = c->table_s1;
  a.bias = c->bias;
  a.euler = reinterpret_cast<float*>(take(p.p_euler));
  a.in_w = heads_in_w(c);
  a.out_w = heads_out_w(c);
  a.in_b = heads_in_b(c);
  a.out_b = heads_out_b(c);
  a.wpack = c->wpack;
  a.cos_tab = c->cos_tab;
  a.sin_tab = c->sin_tab;
  a.kpre = reinterpret_cast<u16*>(take(p.p_kv));
  a.vpre = reinterpret_cast<u16*>(take(p.p_kv));
  a.valid = reinterpret_cast<uint8_t*>(take(p.p_valid));
  a.h = reinterpret_cast<u16*>(take(p.p_h));
  a.g = reinterpret_cast<u16*>(take(p.p_g));
  a.ss = reinterpret_cast<float*>(take(p.p_ss));
  a.hmid = reinterpret_cast<u16*>(take(p.p_hmid));
  a.gmid = reinterpret_cast<u16*>(take(p.p_g));
  a.ssmid = reinterpret_cast<float*>(take(p.p_ssmid));
  a.q = reinterpret_cast<u16*>(take(p.p_q));
  a.o = reinterpret_cast<u16*>(take(p.p_q));
  a.ksuf = reinterpret_cast<u16*>(take(p.p_suf));
  a.vsuf = reinterpret_cast<u16*>(take(p.p_suf));
  a.act = reinterpret_cast<u16*>(take(p.p_act));
  a.apart = reinterpret_cast<float*>(take(p.p_apart));
  a.apart_ml = reinterpret_cast<float*>(take(p.p_apartml));
  a.dpart = reinterpret_cast<float*>(take(p.p_dpart));
  a.x = reinterpret_cast<float*>(take(p.p_x));
}

// Allocate the buffers of c->schedule (the previous schedule's buffers must be freed).
hipError_t alloc_schedule(pi05_ctx* c) {
  const Plan& p = c->plan;
  hipError_t ae = hipSuccess;
#define ALLOC(field, bytes) \
  if (ae == hipSuccess) ae = dalloc(&c->field, bytes)
  if (c->schedule == PI05_SCHEDULE_GRAPH) {
    ALLOC(kcache, p.kv);
    ALLOC(vcache, p.kv);
    ALLOC(valid, p.valid);
    ALLOC(h, p.h);
    ALLOC(rowss, p.rowss);
    ALLOC(q, p.q);
    ALLOC(o, p.o);
    ALLOC(act, p.act);
    ALLOC(part, p.part);
    ALLOC(part_m, p.partml);
    ALLOC(part_l, p.partml);
    ALLOC(x, p.x);
    ALLOC(trace, p.trace);
  } else {
    // zero-filled: flags must start at 0 (epoch 0 never matches a launch), and the launch-control
    // words (last finished epoch, exit count, error word) too
    ALLOC(pbase, p.persistent_bytes() + 64 * 256);
    if (ae == hipSuccess) carve_persistent(c);
    if (ae == hipSuccess) {
      std::vector<float> eu((size_t)c->d.num_steps * 4);
      for (int s = 0; s < c->d.num_steps; ++s) {
        // flow_ode mean coefficients of step s (engine.py:664-675)
        const float t = c->ts[s];
        const float delta = c->ts[s] - c->ts[s + 1];
        const float x1w = t - delta;
        eu[4 * s + 0] = t;
        eu[4 * s + 1] = 1.0f - t;
        eu[4 * s + 2] = 1.0f - x1w;
        eu[4 * s + 3] = x1w;
      }
      ae = hipMemcpy(const_cast<float*>(c->mega.euler), eu.data(), eu.size() * 4, hipMemcpyHostToDevice);
    }
  }
#undef ALLOC
  return ae;
}

// Kernel ids of one denoise step (pi05_bench_kernel).
enum { kKStepIo = 0, kKQkv = 1, kKAttn = 2, kKOProj = 3, kKGateUp = 4, kKDown = 5, kKCount = 6 };

int enqueue_step_io(pi05_ctx* c, hipStream_t st, int s, bool with_trace) {
  const pi05_dims& d = c->d;
  const Plan& p = c->plan;
  StepIoArgs io{};
  io.rowss = c->rowss;
  io.h = c->h;
  io.x = c->x;
  io.in_w = heads_in_w(c);
  io.in_b = heads_in_b(c);
  io.out_w = heads_out_w(c);
  io.out_b = heads_out_b(c);
  io.eps = d.rms_eps;
  io.M = p.M;
  io.has_prev = s > 0;
  io.has_next = s < d.num_steps;
  if (s > 0) {
    const int ps = s - 1;
    const float t = c->ts[ps];
    const float delta = c->ts[ps] - c->ts[ps + 1];
    io.t = t;
    io.one_minus_t = 1.0f - t;
    io.x1_weight = t - delta;
    io.x0_weight = 1.0f - io.x1_weight;
    io.final_mod = c->table + ((size_t)ps * p.n_norms + (p.n_norms - 1)) * kModW;
    io.trace = with_trace ? c->trace + (size_t)ps * p.M * kActDim : nullptr;
  }
  HIPCHK(c, launch_step_io(io, st));
  return PI05_OK;
}

// Enqueue the kernels of decoder layer l at Euler step s whose bit is set in `mask`.
int enqueue_layer(pi05_ctx* c, hipStream_t st, int s, int l, unsigned mask) {
  const pi05_dims& d = c->d;
  const Plan& p = c->plan;
  const size_t kv_block = (size_t)d.batch * p.s_pad * kHeadDim;
  const float* mod_step = c->table + (size_t)s * p.n_norms * kModW;
  const u16* wl = c->wpack + (size_t)l * kLayerElems;
  const float* mod1 = mod_step + (size_t)(2 * l) * kModW;
  const float* mod2 = mod_step + (size_t)(2 * l + 1) * kModW;
  u16* kc_l = c->kcache + (size_t)l * kv_block;
  u16* vc_l = c->vcache + (size_t)l * kv_block;
  if (mask & (1u << kKQkv)) {
    GemmArgs qa{};
    qa.w = wl + kOffQkv;
    qa.h = c->h;
    qa.rowss = c->rowss;
    qa.mod = mod1;
    qa.cos_tab = c->cos_tab;
    qa.sin_tab = c->sin_tab;
    qa.q = c->q;
    qa.kcache = kc_l;
    qa.vcache = vc_l;
    qa.eps = d.rms_eps;
    qa.M = p.M;
    qa.prefix_len = d.prefix_len;
    qa.s_pad = p.s_pad;
    HIPCHK(c, launch_qkv_rope(qa, st));
  }
  if (mask & (1u << kKAttn)) {
    AttnArgs aa{};
    aa.q = c->q;
    aa.kcache = kc_l;
    aa.vcache = vc_l;
    aa.valid = c->valid;
    aa.out = c->o;
    aa.part = c->part;
    aa.part_m = c->part_m;
    aa.part_l = c->part_l;
    aa.rows = p.rows;
    aa.s_pad = p.s_pad;
    aa.nsplit = p.nsplit;
    HIPCHK(c, launch_attention(aa, st));
  }
  if (mask & (1u << kKOProj)) {
    GemmArgs oa{};
    oa.w = wl + kOffO;
    oa.act = c->o;
    oa.mod = mod1;
    oa.h_out = c->h;
    oa.rowss = c->rowss;
    oa.M = p.M;
    HIPCHK(c, launch_o_proj(oa, st));
  }
  if (mask & (1u << kKGateUp)) {
    GemmArgs ga{};
    ga.w = wl + kOffGate;
    ga.w2 = wl + kOffUp;
    ga.h = c->h;
    ga.rowss = c->rowss;
    ga.mod = mod2;
    ga.out = c->act;
    ga.eps = d.rms_eps;
    ga.M = p.M;
    HIPCHK(c, launch_gate_up(ga, st));
  }
  if (mask & (1u << kKDown)) {
    GemmArgs da{};
    da.w = wl + kOffDown;
    da.act = c->act;
    da.mod = mod2;
    da.h_out = c->h;
    da.rowss = c->rowss;
    da.M = p.M;
    HIPCHK(c, launch_down(da, st));
  }
  return PI05_OK;
}

// Enqueue the full num_steps loop (what the graph records).
int enqueue_loop(pi05_ctx* c, hipStream_t st, bool with_trace) {
  const pi05_dims& d = c->d;
  for (int s = 0; s <= d.num_steps; ++s) {
    int rc = enqueue_step_io(c, st, s, with_trace);
    if (rc != PI05_OK) return rc;
    if (s == d.num_steps) break;
    for (int l = 0; l < d.depth; ++l) {
      rc = enqueue_layer(c, st, s, l, 0xffffffffu);
      if (rc != PI05_OK) return rc;
    }
  }
  return PI05_OK;
}

int ensure_graph(pi05_ctx* c, bool with_trace) {
  hipGraphExec_t& ex = c->exec[with_trace ? 1 : 0];
  if (ex) return PI05_OK;
  HIPCHK(c, hipStreamBeginCapture(c->cap, hipStreamCaptureModeThreadLocal));
  int rc = enqueue_loop(c, c->cap, with_trace);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->cap, &g);
  if (rc != PI05_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return c->hip_fail(e, "hipStreamEndCapture");
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    ex = nullptr;
    return c->hip_fail(e, "hipGraphInstantiate");
  }
  return PI05_OK;
}

}  // namespace

// ---- scratch of pi05_adarms_table_noalloc -----------------------------------------------------
// The time embedding and the two time-MLP activations of up to kMaxSteps steps live in a
// file-scope device array (one copy per GPU, held until the process ends), so that entry point
// allocates nothing.  Host code never passes `scratch` itself to a kernel (in host code the name
// stands for a host-side shadow, not a device address): the device address is looked up once
// per device with hipGetSymbolAddress, with that device current, and kept in g_scratch_dev.
constexpr size_t kNoallocScratchFloats = 3 * (size_t)kMaxSteps * kWidth;  // temb | cond1 | cond: 384 KiB
static __device__ __align__(256) float scratch[kNoallocScratchFloats];
constexpr int kMaxNoallocDevices = 64;
float* g_scratch_dev[kMaxNoallocDevices] = {};
std::mutex g_scratch_mu;

// The device address of `scratch` on the current device (looked up on the first call per device).
hipError_t noalloc_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxNoallocDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return hipSuccess;
}

extern "C" {

int pi05_adarms_table_noalloc(const pi05_dims* dims, const float* tin_w, const float* tin_b, const float* tout_w,
                              const float* tout_b, const float* const* dense_w, const float* const* dense_b, float* table_out,
                              void* stream) {
  // the scratch bound first: it holds kMaxSteps steps of the time MLP, and a caller that sizes
  // its own tables may ask for more than the scratch was built for
  if (dims && dims->num_steps > kMaxSteps) {
    g_last_error = "num_steps " + std::to_string(dims->num_steps) + " exceeds the no-alloc scratch maximum of " +
                   std::to_string(kMaxSteps) + " steps";
    return PI05_E_INVALID;
  }
  std::string msg;
  if (!check_dims_msg(dims, &msg)) {
    g_last_error = msg;
    return PI05_E_INVALID;
  }
  if (!tin_w || !tin_b || !tout_w || !tout_b || !dense_w || !dense_b || !table_out) {
    g_last_error = "a pointer argument is NULL";
    return PI05_E_INVALID;
  }
  if (!aligned16(tin_w) || !aligned16(tout_w) || !aligned16(table_out)) {
    g_last_error = "tin_w / tout_w / table_out must be 16-byte aligned";
    return PI05_E_INVALID;
  }
  const int n_norms = 2 * dims->depth + 1;
  for (int n = 0; n < n_norms; ++n) {
    if (!dense_w[n] || !dense_b[n] || !aligned16(dense_w[n])) {
      g_last_error = "dense_w[n] / dense_b[n] must be non-NULL, dense_w[n] 16-byte aligned";
      return PI05_E_INVALID;
    }
  }
  float* sp = nullptr;
  hipError_t e = noalloc_scratch(&sp);
  if (e != hipSuccess) {
    g_last_error = std::string("no-alloc scratch lookup failed: ") + hipGetErrorString(e);
    return PI05_E_HIP;
  }
  const size_t per = (size_t)kMaxSteps * kWidth;
  const AdarmsTableArgs ta{tin_w, tin_b, tout_w, tout_b, dense_w, dense_b, n_norms, dims->num_steps, dims->time_min_period,
                           dims->time_max_period, sp, sp + per, sp + 2 * per, table_out};
  e = launch_adarms_table(ta, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    g_last_error = std::string("no-alloc table kernels: ") + hipGetErrorString(e);
    return PI05_E_HIP;
  }
  return PI05_OK;
}


int pi05_abi_version(void) { return PI05_ABI_VERSION; }

void pi05_default_dims(pi05_dims* d) {
  if (!d) return;
  d->width = kWidth;
  d->depth = 18;
  d->num_heads = kHeads;
  d->num_kv_heads = 1;
  d->head_dim = kHeadDim;
  d->mlp_dim = kMlp;
  d->action_dim = kActDim;
  d->action_horizon = kHorizon;
  d->batch = 1;
  d->prefix_len = 968;
  d->num_steps = 10;
  d->rms_eps = 1e-6f;
  d->rope_theta = 10000.0f;
  d->time_min_period = 4e-3;
  d->time_max_period = 4.0;
}

int pi05_check_dims(const pi05_dims* dims) {
  std::string msg;
  if (!check_dims_msg(dims, &msg)) {
    g_last_error = msg;
    return PI05_E_INVALID;
  }
  return PI05_OK;
}

size_t pi05_ctx_device_bytes(const pi05_dims* dims) {
  std::string msg;
  if (!check_dims_msg(dims, &msg)) return 0;
  const Plan p = make_plan(*dims);
  return p.common() + p.persistent_bytes();
}

const char* pi05_last_error(const pi05_ctx* ctx) { return ctx ? ctx->err.c_str() : g_last_error.c_str(); }

int pi05_ctx_create(const pi05_dims* dims, pi05_ctx** out) {
  if (!out) {
    g_last_error = "out is NULL";
    return PI05_E_INVALID;
  }
  *out = nullptr;
  std::string msg;
  if (!check_dims_msg(dims, &msg)) {
    g_last_error = msg;
    return PI05_E_INVALID;
  }
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    g_last_error = std::string("no HIP device: ") + hipGetErrorString(e);
    return PI05_E_NODEVICE;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    g_last_error = std::string("device is not gfx950 (MI355X): ") + (e == hipSuccess ? prop.gcnArchName : hipGetErrorString(e));
    return PI05_E_NODEVICE;
  }
  pi05_ctx* c = new pi05_ctx();
  c->d = *dims;
  c->device = dev;
  c->plan = make_plan(*dims);
  c->layers.resize(dims->depth);
  c->ts = euler_schedule(dims->num_steps);
  const Plan& p = c->plan;
  hipError_t ae = hipSuccess;
#define ALLOC(field, bytes) \
  if (ae == hipSuccess) ae = dalloc(&c->field, bytes)
  ALLOC(wpack, p.wpack);
  ALLOC(table, p.table);
  ALLOC(table_s1, p.table);
  ALLOC(bias, p.bias);
  ALLOC(temb, p.temb);
  ALLOC(cond1, p.cond);
  ALLOC(cond, p.cond);
  ALLOC(heads_buf, p.heads);
  ALLOC(cos_tab, p.rope);
  ALLOC(sin_tab, p.rope);
  ALLOC(positions, p.pos);
  ALLOC(inv_freq, p.invf);
#undef ALLOC
  if (ae == hipSuccess) {
    ae = hipHostMalloc(reinterpret_cast<void**>(&c->host_err), 2 * sizeof(unsigned), hipHostMallocMapped);
    if (ae == hipSuccess) c->host_err[kHostTimeouts] = c->host_err[kHostPlacement] = 0;
  }
  // the persistent schedule needs every workgroup of the grid resident at once
  int coop = 0, per_cu = 0;
  if (ae == hipSuccess) ae = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev);
  if (ae == hipSuccess)
    ae = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, denoise_loop_kernel_ptr(c->d.batch), denoise_loop_threads(), 0);
  // one workgroup per CU; the weight phases have 256 items, one per workgroup
  c->grid = prop.multiProcessorCount;
  c->schedule = (coop && per_cu >= 1 && c->grid >= 256) ? PI05_SCHEDULE_PERSISTENT : PI05_SCHEDULE_GRAPH;
  if (ae == hipSuccess) ae = alloc_schedule(c);
  if (ae == hipSuccess) ae = hipStreamCreateWithFlags(&c->cap, hipStreamNonBlocking);
  if (ae == hipSuccess) {
    std::vector<float> invf(kHalfDim);
    rope_inv_freq(dims->rope_theta, invf.data());
    ae = hipMemcpy(c->inv_freq, invf.data(), p.invf, hipMemcpyHostToDevice);
  }
  if (ae != hipSuccess) {
    g_last_error = std::string("context allocation failed: ") + hipGetErrorString(ae);
    const int code = (ae == hipErrorOutOfMemory) ? PI05_E_NOMEM : PI05_E_HIP;
    free_all(c);
    delete c;
    return code;
  }
  *out = c;
  return PI05_OK;
}

int pi05_ctx_destroy(pi05_ctx* ctx) {
  if (!ctx) return PI05_OK;
  (void)hipDeviceSynchronize();
  free_all(ctx);
  delete ctx;
  return PI05_OK;
}

int pi05_bind_layer(pi05_ctx* c, int layer, const void* wq, const void* wk, const void* wv, const void* wo,
                    const void* wgate, const void* wup, const void* wdown, const float* ln1_w, const float* ln1_b,
                    const float* ln2_w, const float* ln2_b) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (layer < 0 || layer >= c->d.depth) return c->fail(PI05_E_INVALID, "layer %d out of range [0, %d)", layer, c->d.depth);
  const void* ptrs[] = {wq, wk, wv, wo, wgate, wup, wdown, ln1_w, ln1_b, ln2_w, ln2_b};
  const char* names[] = {"wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "ln1_w", "ln1_b", "ln2_w", "ln2_b"};
  for (int i = 0; i < 11; ++i) {
    if (!ptrs[i]) return c->fail(PI05_E_INVALID, "layer %d: %s is NULL", layer, names[i]);
    if (!aligned16(ptrs[i])) return c->fail(PI05_E_INVALID, "layer %d: %s is not 16-byte aligned", layer, names[i]);
  }
  LayerBind& b = c->layers[layer];
  b.wq = wq;
  b.wk = wk;
  b.wv = wv;
  b.wo = wo;
  b.wgate = wgate;
  b.wup = wup;
  b.wdown = wdown;
  b.ln1_w = ln1_w;
  b.ln1_b = ln1_b;
  b.ln2_w = ln2_w;
  b.ln2_b = ln2_b;
  b.set = true;
  c->weights_ready = false;
  return PI05_OK;
}

int pi05_bind_heads(pi05_ctx* c, const float* norm_w, const float* norm_b, const float* in_w, const float* in_b,
                    const float* out_w, const float* out_b, const float* tin_w, const float* tin_b, const float* tout_w,
                    const float* tout_b) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  const void* ptrs[] = {norm_w, norm_b, in_w, in_b, out_w, out_b, tin_w, tin_b, tout_w, tout_b};
  const char* names[] = {"norm_w", "norm_b", "in_w", "in_b", "out_w", "out_b", "tin_w", "tin_b", "tout_w", "tout_b"};
  for (int i = 0; i < 10; ++i) {
    if (!ptrs[i]) return c->fail(PI05_E_INVALID, "heads: %s is NULL", names[i]);
    if (!aligned16(ptrs[i])) return c->fail(PI05_E_INVALID, "heads: %s is not 16-byte aligned", names[i]);
  }
  HeadBind& h = c->heads;
  h.norm_w = norm_w;
  h.norm_b = norm_b;
  h.in_w = in_w;
  h.in_b = in_b;
  h.out_w = out_w;
  h.out_b = out_b;
  h.tin_w = tin_w;
  h.tin_b = tin_b;
  h.tout_w = tout_w;
  h.tout_b = tout_b;
  h.set = true;
  c->weights_ready = false;
  return PI05_OK;
}

int pi05_refresh_weights(pi05_ctx* c, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  for (int l = 0; l < c->d.depth; ++l)
    if (!c->layers[l].set) return c->fail(PI05_E_STATE, "layer %d weights are not bound", l);
  if (!c->heads.set) return c->fail(PI05_E_STATE, "head weights (norm/action/time) are not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const Plan& p = c->plan;
  for (int l = 0; l < c->d.depth; ++l) {
    const LayerBind& b = c->layers[l];
    u16* wl = c->wpack + (size_t)l * kLayerElems;
    HIPCHK(c, launch_pack_weight(b.wq, wl + kOffQkv, kHeads * kHeadDim, kWidth, st));
    HIPCHK(c, launch_pack_weight(b.wk, wl + kOffQkv + wfrag_offset(128, 0, 32), kHeadDim, kWidth, st));
    HIPCHK(c, launch_pack_weight(b.wv, wl + kOffQkv + wfrag_offset(144, 0, 32), kHeadDim, kWidth, st));
    HIPCHK(c, launch_pack_weight(b.wo, wl + kOffO, kWidth, kHeads * kHeadDim, st));
    HIPCHK(c, launch_pack_weight(b.wgate, wl + kOffGate, kMlp, kWidth, st));
    HIPCHK(c, launch_pack_weight(b.wup, wl + kOffUp, kMlp, kWidth, st));
    HIPCHK(c, launch_pack_weight(b.wdown, wl + kOffDown, kWidth, kMlp, st));
  }
  const HeadBind& hb = c->heads;
  HIPCHK(c, hipMemcpyAsync(heads_in_w(c), hb.in_w, (size_t)kWidth * kActDim * 4, hipMemcpyDeviceToDevice, st));
  HIPCHK(c, hipMemcpyAsync(heads_out_w(c), hb.out_w, (size_t)kWidth * kActDim * 4, hipMemcpyDeviceToDevice, st));
  HIPCHK(c, hipMemcpyAsync(heads_in_b(c), hb.in_b, (size_t)kWidth * 4, hipMemcpyDeviceToDevice, st));
  HIPCHK(c, hipMemcpyAsync(heads_out_b(c), hb.out_b, (size_t)kActDim * 4, hipMemcpyDeviceToDevice, st));
  // adaRMS modulation table (engine.py:578-599): cond = silu(W2 silu(W1 temb + b1) + b2),
  // table[s][n] = dense_n(cond[s]); the same kernels as pi05_adarms_table_noalloc
  const int S = c->d.num_steps;
  std::vector<const float*> dw(p.n_norms), db(p.n_norms);
  for (int n = 0; n < p.n_norms; ++n) {
    if (n == p.n_norms - 1) {
      dw[n] = hb.norm_w;
      db[n] = hb.norm_b;
    } else {
      const LayerBind& lb = c->layers[n / 2];
      dw[n] = (n & 1) ? lb.ln2_w : lb.ln1_w;
      db[n] = (n & 1) ? lb.ln2_b : lb.ln1_b;
    }
  }
  const AdarmsTableArgs ta{hb.tin_w, hb.tin_b, hb.tout_w, hb.tout_b, dw.data(), db.data(), p.n_norms, S,
                           c->d.time_min_period, c->d.time_max_period, c->temb, c->cond1, c->cond, c->table};
  HIPCHK(c, launch_adarms_table(ta, st));
  HIPCHK(c, launch_scale_plus_one(c->table, c->table_s1, S * p.n_norms, st));
  ShiftBiasArgs sb{c->wpack, c->table, c->bias, c->d.depth, S};
  HIPCHK(c, launch_shift_bias(sb, st));
  c->weights_ready = true;
  return PI05_OK;
}

int pi05_get_adarms_table(pi05_ctx* c, float* table_out, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (!table_out) return c->fail(PI05_E_INVALID, "table_out is NULL");
  if (!c->weights_ready) return c->fail(PI05_E_STATE, "weights not refreshed");
  HIPCHK(c, hipMemcpyAsync(table_out, c->table, c->plan.table, hipMemcpyDeviceToDevice, reinterpret_cast<hipStream_t>(stream)));
  return PI05_OK;
}

int pi05_prime_prefix(pi05_ctx* c, const void* const* k_layers, const void* const* v_layers, int64_t kv_batch_stride,
                      int64_t kv_row_stride, const uint8_t* prefix_pad, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  const pi05_dims& d = c->d;
  if (!k_layers || !v_layers) return c->fail(PI05_E_INVALID, "k_layers / v_layers is NULL");
  if (!prefix_pad) return c->fail(PI05_E_INVALID, "prefix_pad is NULL");
  if (kv_row_stride < kHeadDim || kv_row_stride % 8) return c->fail(PI05_E_INVALID, "kv_row_stride %lld must be >= %d and a multiple of 8", (long long)kv_row_stride, kHeadDim);
  if (d.batch > 1 && (kv_batch_stride < (int64_t)d.prefix_len * kv_row_stride || kv_batch_stride % 8))
    return c->fail(PI05_E_INVALID, "kv_batch_stride %lld too small or not a multiple of 8", (long long)kv_batch_stride);
  // the per-layer pointers go to the kernel by value: nothing to copy, nothing to wait for
  PrimeKvArgs ka{};
  for (int l = 0; l < d.depth; ++l) {
    if (!k_layers[l] || !v_layers[l]) return c->fail(PI05_E_INVALID, "layer %d K/V pointer is NULL", l);
    if (!aligned16(k_layers[l]) || !aligned16(v_layers[l])) return c->fail(PI05_E_INVALID, "layer %d K/V pointer is not 16-byte aligned", l);
    ka.k_ptrs[l] = k_layers[l];
    ka.v_ptrs[l] = v_layers[l];
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool persistent = c->schedule == PI05_SCHEDULE_PERSISTENT;
  // graph schedule: one cache of s_pad keys, action keys at [P, P + A);
  // persistent: prefix keys padded to s_pre, action keys in a separate per-step block
  const int kv_keys = persistent ? c->plan.s_pre : c->plan.s_pad;
  ka.batch_stride = kv_batch_stride;
  ka.row_stride = kv_row_stride;
  ka.kcache = persistent ? const_cast<u16*>(c->mega.kpre) : c->kcache;
  ka.vcache = persistent ? const_cast<u16*>(c->mega.vpre) : c->vcache;
  ka.batch = d.batch;
  ka.prefix_len = d.prefix_len;
  ka.s_pad = kv_keys;
  ka.suffix_base = persistent ? kv_keys : d.prefix_len;
  HIPCHK(c, launch_prime_kv(ka, d.depth, st));
  PrimeTablesArgs ta{};
  ta.prefix_pad = prefix_pad;
  ta.inv_freq = c->inv_freq;
  ta.positions = c->positions;
  ta.valid = persistent ? const_cast<uint8_t*>(c->mega.valid) : c->valid;
  ta.cos_tab = c->cos_tab;
  ta.sin_tab = c->sin_tab;
  ta.prefix_len = d.prefix_len;
  ta.s_pad = persistent ? kv_keys + 64 : kv_keys;
  ta.suffix_base = persistent ? kv_keys : d.prefix_len;
  HIPCHK(c, launch_prime_tables(ta, d.batch, st));
  c->primed = true;
  return PI05_OK;
}

int pi05_get_step_invariants(pi05_ctx* c, int64_t* positions_out, uint8_t* key_valid_out, int32_t* stray_valid_out, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (!positions_out && !key_valid_out && !stray_valid_out) return c->fail(PI05_E_INVALID, "every output is NULL");
  if (!c->primed) return c->fail(PI05_E_STATE, "prefix not primed (call pi05_prime_prefix)");
  const bool persistent = c->schedule == PI05_SCHEDULE_PERSISTENT;
  ExportInvariantsArgs a{};
  a.positions = c->positions;
  a.valid = persistent ? c->mega.valid : c->valid;
  a.pos_out = positions_out;
  a.valid_out = key_valid_out;
  a.stray_out = stray_valid_out;
  a.batch = c->d.batch;
  a.prefix_len = c->d.prefix_len;
  // the layouts pi05_prime_prefix wrote: persistent [B][s_pre + 64] with the action keys at
  // s_pre; graph [B][s_pad] with the action keys at P
  a.valid_ld = persistent ? c->plan.s_pre + 64 : c->plan.s_pad;
  a.suffix_base = persistent ? c->plan.s_pre : c->d.prefix_len;
  HIPCHK(c, launch_export_invariants(a, reinterpret_cast<hipStream_t>(stream)));
  return PI05_OK;
}

namespace {

// Timeouts recorded by launches of this context that have not been reported yet: the pinned host
// word counts the launches whose waits timed out (read without waiting: a launch still running is
// seen by a later call or by pi05_denoise_status).
int take_pending_error(pi05_ctx* c) {
  if (!c->host_err) return PI05_OK;
  const unsigned np = __atomic_load_n(c->host_err + kHostPlacement, __ATOMIC_ACQUIRE);
  if (np != c->reported_placement) {
    const unsigned fresh = np - c->reported_placement;
    c->reported_placement = np;
    return c->fail(PI05_E_HIP, "%u denoise launch%s on this context ran with workgroups not dealt round-robin over the 8 XCDs "
                   "(workgroups w and w + 8 on different XCDs); the intra-XCD hand-offs may have read stale data, so %s "
                   "actions are invalid", fresh, fresh == 1 ? "" : "es", fresh == 1 ? "its" : "their");
  }
  const unsigned n = __atomic_load_n(c->host_err + kHostTimeouts, __ATOMIC_ACQUIRE);
  if (n == c->reported) return PI05_OK;
  const unsigned fresh = n - c->reported;
  c->reported = n;
  return c->fail(PI05_E_HIP, "%u denoise launch%s on this context timed out waiting for inputs; %s actions are invalid "
                 "(nothing was enqueued by the call reporting it)", fresh, fresh == 1 ? "" : "es", fresh == 1 ? "its" : "their");
}

bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// One cooperative launch of the whole loop.  Nothing launch-specific is baked into the arguments:
// the kernel takes its epoch from the context's launch-control block and advances it itself, so
// the launch may be captured into a graph and replayed any number of times.
int denoise_persistent(pi05_ctx* c, float* x_inout, float* v_trace, hipStream_t st) {
  const int pending = take_pending_error(c);
  if (pending != PI05_OK) return pending;
  MegaArgs a = c->mega;
  a.spin_limit = c->spin_limit;
  a.x_io = x_inout;
  a.trace = v_trace;
  unsigned* host_err_dev = nullptr;
  HIPCHK(c, hipHostGetDevicePointer(reinterpret_cast<void**>(&host_err_dev), c->host_err, 0));
  a.host_err = host_err_dev;
  a.xcd_skew = c->xcd_skew;
  // enqueue only: a timed-out wait is reported by the next call or by pi05_denoise_status
  HIPCHK(c, launch_denoise_loop(a, c->grid, st));
  return PI05_OK;
}

}  // namespace

int pi05_denoise(pi05_ctx* c, float* x_inout, float* v_trace, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (!x_inout) return c->fail(PI05_E_INVALID, "x_inout is NULL");
  if (!c->weights_ready) return c->fail(PI05_E_STATE, "weights not bound/refreshed (call pi05_refresh_weights)");
  if (!c->primed) return c->fail(PI05_E_STATE, "prefix not primed (call pi05_prime_prefix)");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (c->schedule == PI05_SCHEDULE_PERSISTENT) return denoise_persistent(c, x_inout, v_trace, st);
  if (stream_capturing(st))
    return c->fail(PI05_E_STATE, "the graph schedule runs its loop as a hipGraph of its own and cannot be captured; "
                   "capture the persistent schedule (the default)");
  const bool with_trace = v_trace != nullptr;
  int rc = ensure_graph(c, with_trace);
  if (rc != PI05_OK) return rc;
  HIPCHK(c, hipMemcpyAsync(c->x, x_inout, c->plan.x, hipMemcpyDeviceToDevice, st));
  HIPCHK(c, hipGraphLaunch(c->exec[with_trace ? 1 : 0], st));
  HIPCHK(c, hipMemcpyAsync(x_inout, c->x, c->plan.x, hipMemcpyDeviceToDevice, st));
  if (with_trace) HIPCHK(c, hipMemcpyAsync(v_trace, c->trace, c->plan.trace, hipMemcpyDeviceToDevice, st));
  return PI05_OK;
}

int pi05_denoise_status(pi05_ctx* c, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  HIPCHK(c, hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
  return take_pending_error(c);
}

int pi05_debug_set_spin_limit(pi05_ctx* c, int polls) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (polls < 0) return c->fail(PI05_E_INVALID, "polls %d < 0", polls);
  c->spin_limit = polls == 0 ? kDefaultSpinLimit : polls;
  return PI05_OK;
}

int pi05_debug_skew_placement_check(pi05_ctx* c, int skew) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (skew < 0 || skew > 7) return c->fail(PI05_E_INVALID, "skew %d outside 0..7", skew);
  c->xcd_skew = (unsigned)skew;
  return PI05_OK;
}

int pi05_debug_set_epoch(pi05_ctx* c, uint32_t epoch) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (epoch >= kEpochWrap) return c->fail(PI05_E_INVALID, "epoch %u must be below 2^31", epoch);
  if (c->schedule != PI05_SCHEDULE_PERSISTENT) return c->fail(PI05_E_STATE, "the epoch belongs to the persistent schedule");
  HIPCHK(c, hipDeviceSynchronize());
  HIPCHK(c, hipMemcpy(c->mega.err + kCtlEpoch, &epoch, sizeof epoch, hipMemcpyHostToDevice));
  return PI05_OK;
}

int pi05_set_schedule(pi05_ctx* c, int schedule) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (schedule != PI05_SCHEDULE_PERSISTENT && schedule != PI05_SCHEDULE_GRAPH)
    return c->fail(PI05_E_INVALID, "schedule %d is not PI05_SCHEDULE_PERSISTENT or PI05_SCHEDULE_GRAPH", schedule);
  if (schedule == c->schedule) return PI05_OK;
  if (schedule == PI05_SCHEDULE_PERSISTENT) {
    int coop = 0, per_cu = 0;
    HIPCHK(c, hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, c->device));
    HIPCHK(c, hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, denoise_loop_kernel_ptr(c->d.batch), denoise_loop_threads(), 0));
    if (!coop || per_cu < 1 || c->grid < 256)
      return c->fail(PI05_E_NODEVICE, "device cannot run the persistent schedule (cooperative launch of 256 workgroups)");
  }
  HIPCHK(c, hipDeviceSynchronize());
  free_schedule(c);
  c->schedule = schedule;
  const hipError_t e = alloc_schedule(c);
  if (e != hipSuccess) {
    free_schedule(c);
    return c->fail(e == hipErrorOutOfMemory ? PI05_E_NOMEM : PI05_E_HIP, "schedule buffers: %s", hipGetErrorString(e));
  }
  return PI05_OK;
}

int pi05_get_schedule(const pi05_ctx* c) { return c ? c->schedule : PI05_E_INVALID; }

int pi05_release_graph(pi05_ctx* c) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  for (auto& e : c->exec)
    if (e) {
      HIPCHK(c, hipGraphExecDestroy(e));
      e = nullptr;
    }
  return PI05_OK;
}

int pi05_launches_per_step(const pi05_ctx* c) {
  if (!c) return 0;
  if (c->schedule == PI05_SCHEDULE_PERSISTENT) return 0;
  return 1 + c->d.depth * (c->plan.nsplit > 1 ? 6 : 5);
}

int pi05_bench_kernel(pi05_ctx* c, int kernel_id, int layer, int iters, void* stream) {
  if (!c) {
    g_last_error = "ctx is NULL";
    return PI05_E_INVALID;
  }
  if (kernel_id < 0 || kernel_id >= kKCount) return c->fail(PI05_E_INVALID, "kernel_id %d out of range [0, %d)", kernel_id, kKCount);
  if (layer < 0 || layer >= c->d.depth) return c->fail(PI05_E_INVALID, "layer %d out of range", layer);
  if (iters < 1 || iters > 100000) return c->fail(PI05_E_INVALID, "iters %d out of range [1, 100000]", iters);
  if (!c->weights_ready || !c->primed) return c->fail(PI05_E_STATE, "weights and prefix must be ready");
  if (c->schedule != PI05_SCHEDULE_GRAPH) return c->fail(PI05_E_STATE, "per-kernel timing needs the graph schedule");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (int i = 0; i < iters; ++i) {
    const int rc = kernel_id == kKStepIo ? enqueue_step_io(c, st, 1, false) : enqueue_layer(c, st, 0, layer, 1u << kernel_id);
    if (rc != PI05_OK) return rc;
  }
  return PI05_OK;
}

int pi05_euler_schedule(int num_steps, float* ts_host) {
  if (num_steps < 1 || num_steps > kMaxSteps || !ts_host) {
    g_last_error = "num_steps out of range or ts_host is NULL";
    return PI05_E_INVALID;
  }
  const std::vector<float> ts = euler_schedule(num_steps);
  memcpy(ts_host, ts.data(), ts.size() * sizeof(float));
  return PI05_OK;
}

int pi05_time_embedding(const pi05_dims* dims, float t, float* out_host) {
  if (pi05_check_dims(dims) != PI05_OK) return PI05_E_INVALID;
  if (!out_host) {
    g_last_error = "out_host is NULL";
    return PI05_E_INVALID;
  }
  sinusoid(t, kWidth, dims->time_min_period, dims->time_max_period, out_host);
  return PI05_OK;
}

int pi05_rope_inv_freq(const pi05_dims* dims, float* out_host) {
  if (pi05_check_dims(dims) != PI05_OK) return PI05_E_INVALID;
  if (!out_host) {
    g_last_error = "out_host is NULL";
    return PI05_E_INVALID;
  }
  rope_inv_freq(dims->rope_theta, out_host);
  return PI05_OK;
}

}  // extern "C"
