// Stand-alone C-ABI benchmark of the denoise loop: what a C/C++ host does with
// libpi05_denoise.so, without Python.  Used for profiling (rocprofv3 traces a plain process
// cleanly) and as the integration example of the C ABI.
//
//   denoise_bench [--prefix P] [--batch B] [--predicts K] [--warmup W] [--schedule persistent|graph]
//   denoise_bench --copy-bytes N   (one plain N-byte device copy kernel: calibrates HBM byte
//                                   counters such as FETCH_SIZE / WRITE_SIZE against a known size)
//   denoise_bench ... --with-copy N (the predicts, then that copy kernel in the same process, so
//                                   one counter run measures both)
//
// Weights are random-init on the device (N(0, 0.02)-scaled uniform noise, seed fixed), prefix
// KV uniform in [-1.7, 1.7] bf16 (unit variance), all prefix keys valid, noise N(0,1)-scaled
// uniform.  Prints one line: ms/predict over K predicts timed with HIP events.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "pi05_denoise.h"

#define CK(x)                                                                         \
  do {                                                                                \
    hipError_t e_ = (x);                                                              \
    if (e_ != hipSuccess) {                                                           \
      fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      exit(2);                                                                        \
    }                                                                                 \
  } while (0)
#define PI(ctx, x)                                                            \
  do {                                                                        \
    int rc_ = (x);                                                            \
    if (rc_ != PI05_OK) {                                                     \
      fprintf(stderr, "%s failed (%d): %s\n", #x, rc_, pi05_last_error(ctx)); \
      exit(3);                                                                \
    }                                                                         \
  } while (0)

namespace {

__device__ __forceinline__ float hash_uniform(uint64_t i, uint32_t seed) {
  // splitmix64 finaliser -> uniform in [-1, 1)
  uint64_t z = i * 0x9E3779B97F4A7C15ull + seed * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (2.0f / 16777216.0f) - 1.0f;
}

// uniform [-1, 1) has standard deviation 1/sqrt(3)
__global__ void fill_bf16(uint16_t* p, size_t n, float stddev, uint32_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = hash_uniform(i, seed) * stddev * 1.7320508f;
    p[i] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
}

__global__ void fill_f32(float* p, size_t n, float stddev, uint32_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = hash_uniform(i, seed) * stddev * 1.7320508f;
}

__global__ void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dst[i] = src[i];
}

int copy_calibration(size_t bytes) {
  const size_t n = bytes / 16;
  uint4 *src = nullptr, *dst = nullptr;
  CK(hipMalloc(&src, n * 16));
  CK(hipMalloc(&dst, n * 16));
  CK(hipMemset(src, 1, n * 16));
  CK(hipDeviceSynchronize());
  copy_kernel<<<4096, 256>>>(src, dst, n);
  CK(hipGetLastError());
  CK(hipDeviceSynchronize());
  printf("denoise_bench: copied %zu bytes (read %zu, write %zu)\n", n * 16, n * 16, n * 16);
  fflush(stdout);
  CK(hipFree(src));
  CK(hipFree(dst));
  return 0;
}

uint32_t g_seed = 1;

void* dev_bf16(size_t n, float stddev) {
  void* p = nullptr;
  CK(hipMalloc(&p, n * 2));
  fill_bf16<<<1024, 256>>>(reinterpret_cast<uint16_t*>(p), n, stddev, g_seed++);
  CK(hipGetLastError());
  return p;
}

float* dev_f32(size_t n, float stddev) {
  float* p = nullptr;
  CK(hipMalloc(&p, n * 4));
  fill_f32<<<1024, 256>>>(p, n, stddev, g_seed++);
  CK(hipGetLastError());
  return p;
}

}  // namespace

int main(int argc, char** argv) {
  int prefix = 968, batch = 1, predicts = 20, warmup = 3;
  size_t copy_bytes = 0;
  std::string schedule = "persistent";
  for (int i = 1; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    if (k == "--copy-bytes") return copy_calibration(strtoull(argv[i + 1], nullptr, 10));
    if (k == "--prefix") prefix = atoi(argv[i + 1]);
    else if (k == "--batch") batch = atoi(argv[i + 1]);
    else if (k == "--predicts") predicts = atoi(argv[i + 1]);
    else if (k == "--warmup") warmup = atoi(argv[i + 1]);
    else if (k == "--schedule") schedule = argv[i + 1];
    else if (k == "--with-copy") copy_bytes = strtoull(argv[i + 1], nullptr, 10);
    else {
      fprintf(stderr, "unknown option %s\n", argv[i]);
      return 1;
    }
  }
  if (predicts < 1 || warmup < 0 || (schedule != "persistent" && schedule != "graph")) {
    fprintf(stderr, "bad arguments\n");
    return 1;
  }
  pi05_dims d;
  pi05_default_dims(&d);
  d.prefix_len = prefix;
  d.batch = batch;
  if (pi05_check_dims(&d) != PI05_OK) {
    fprintf(stderr, "dims: %s\n", pi05_last_error(nullptr));
    return 1;
  }
  pi05_ctx* ctx = nullptr;
  PI(nullptr, pi05_ctx_create(&d, &ctx));
  PI(ctx, pi05_set_schedule(ctx, schedule == "graph" ? PI05_SCHEDULE_GRAPH : PI05_SCHEDULE_PERSISTENT));

  const size_t W = d.width, H = d.num_heads, D = d.head_dim, I = d.mlp_dim, A = d.action_dim;
  std::vector<void*> owned;
  for (int l = 0; l < d.depth; ++l) {
    void* wq = dev_bf16(H * D * W, 0.02f);
    void* wk = dev_bf16(D * W, 0.02f);
    void* wv = dev_bf16(D * W, 0.02f);
    void* wo = dev_bf16(W * H * D, 0.02f);
    void* wg = dev_bf16(I * W, 0.02f);
    void* wu = dev_bf16(I * W, 0.02f);
    void* wd = dev_bf16(W * I, 0.02f);
    float* l1w = dev_f32(3 * W * W, 0.02f);
    float* l1b = dev_f32(3 * W, 0.02f);
    float* l2w = dev_f32(3 * W * W, 0.02f);
    float* l2b = dev_f32(3 * W, 0.02f);
    PI(ctx, pi05_bind_layer(ctx, l, wq, wk, wv, wo, wg, wu, wd, l1w, l1b, l2w, l2b));
    owned.insert(owned.end(), {wq, wk, wv, wo, wg, wu, wd, l1w, l1b, l2w, l2b});
  }
  float* heads[10] = {dev_f32(3 * W * W, 0.02f), dev_f32(3 * W, 0.02f), dev_f32(W * A, 0.02f), dev_f32(W, 0.02f),
                      dev_f32(A * W, 0.02f),     dev_f32(A, 0.02f),     dev_f32(W * W, 0.02f), dev_f32(W, 0.02f),
                      dev_f32(W * W, 0.02f),     dev_f32(W, 0.02f)};
  PI(ctx, pi05_bind_heads(ctx, heads[0], heads[1], heads[2], heads[3], heads[4], heads[5], heads[6], heads[7], heads[8],
                          heads[9]));
  PI(ctx, pi05_refresh_weights(ctx, nullptr));

  std::vector<const void*> ks(d.depth), vs(d.depth);
  for (int l = 0; l < d.depth; ++l) {
    ks[l] = dev_bf16((size_t)batch * prefix * D, 1.0f);
    vs[l] = dev_bf16((size_t)batch * prefix * D, 1.0f);
  }
  uint8_t* pad = nullptr;
  CK(hipMalloc(&pad, (size_t)batch * prefix));
  CK(hipMemset(pad, 1, (size_t)batch * prefix));
  PI(ctx, pi05_prime_prefix(ctx, ks.data(), vs.data(), (int64_t)prefix * D, (int64_t)D, pad, nullptr));

  const size_t xn = (size_t)batch * d.action_horizon * A;
  float* noise = dev_f32(xn, 1.0f);
  float* x = nullptr;
  CK(hipMalloc(&x, xn * 4));
  CK(hipDeviceSynchronize());

  for (int i = 0; i < warmup; ++i) {
    CK(hipMemcpy(x, noise, xn * 4, hipMemcpyDeviceToDevice));
    PI(ctx, pi05_denoise(ctx, x, nullptr, nullptr));
  }
  CK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  CK(hipEventRecord(e0, nullptr));
  for (int i = 0; i < predicts; ++i) PI(ctx, pi05_denoise(ctx, x, nullptr, nullptr));
  CK(hipEventRecord(e1, nullptr));
  CK(hipEventSynchronize(e1));
  PI(ctx, pi05_denoise_status(ctx, nullptr));  // no launch timed out or ran misplaced
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<float> hx(xn);
  CK(hipMemcpy(hx.data(), x, xn * 4, hipMemcpyDeviceToHost));
  double checksum = 0;
  for (float v : hx) checksum += v;
  printf("denoise_bench: schedule=%s B=%d P=%d steps=%d depth=%d: %.4f ms/predict over %d predicts (checksum %.6g)\n",
         schedule.c_str(), batch, prefix, d.num_steps, d.depth, ms / predicts, predicts, checksum);
  fflush(stdout);

  PI(ctx, pi05_ctx_destroy(ctx));
  for (void* p : owned) CK(hipFree(p));
  for (float* p : heads) CK(hipFree(p));
  for (int l = 0; l < d.depth; ++l) {
    CK(hipFree(const_cast<void*>(ks[l])));
    CK(hipFree(const_cast<void*>(vs[l])));
  }
  CK(hipFree(pad));
  CK(hipFree(noise));
  CK(hipFree(x));
  return copy_bytes ? copy_calibration(copy_bytes) : 0;
}
