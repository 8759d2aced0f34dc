// gs_bench -- benchmark driver for libgruscan through its C ABI.
//
//   gs_bench <items> [launches=30] [warmup=10]
//
// <items> is a comma-separated list of configs 0..4 and "copy", run in that
// order in one process (one JSON line each). A config run builds the
// synthetic inputs of one of the five benchmark configurations (shapes,
// kinds and hidden quant of gru_qat_amd/configs.py;
// values from a fixed-seed generator, not the same draws as configs.py),
// calls the config's gs_*_fwd entry point `warmup` times, then `launches`
// times with a HIP event pair around each call on one stream (a spin kernel
// keeps the queue ahead of the device, so host overhead is not counted), and
// prints one JSON line with the mean and median launch duration.
//
// The copy item launches a plain copy kernel (float4 loads and stores) of
// 256 MiB; it reads and writes exactly that many bytes per launch, which
// calibrates byte counters (FETCH_SIZE, WRITE_SIZE) under rocprofv3 --pmc.
//
// It is also the smallest complete example of calling the library from C++:
// inputs, workspace sizing and zeroing, launch, and the fault-word check.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/gruscan.h"

namespace {

#define CHECK(x)                                                                           \
  do {                                                                                     \
    hipError_t e_ = (x);                                                                   \
    if (e_ != hipSuccess) {                                                                \
      fprintf(stderr, "gs_bench: %s failed: %s\n", #x, hipGetErrorString(e_));             \
      exit(1);                                                                             \
    }                                                                                      \
  } while (0)

struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  float uniform() {  // [0, 1)
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((s >> 40) * (1.0 / 16777216.0));
  }
  float sym(float bound) { return (uniform() * 2.0f - 1.0f) * bound; }
};

float* upload(const std::vector<float>& h) {
  float* d = nullptr;
  CHECK(hipMalloc(&d, std::max<size_t>(h.size(), 1) * sizeof(float)));
  CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
  return d;
}

std::vector<float> filled(size_t n, Rng& g, float bound) {
  std::vector<float> v(n);
  for (auto& x : v) x = g.sym(bound);
  return v;
}

// Holds the queue ahead of the device: spins for about `cycles` shader clocks.
__global__ void spin(long long cycles) {
  const long long t0 = clock64();
  while (clock64() - t0 < cycles) __builtin_amdgcn_s_sleep(127);
}

__global__ void copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst, size_t n4) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

const char* kNames[5] = {"diagonal_fp32", "dense_fp32", "dense_int8_qat", "monarch_nb8_two_factor_int8",
                         "butterfly_fp32"};

void report(const char* what, int idx, const std::vector<float>& ms, long long T, long long B, long long H) {
  std::vector<float> s = ms;
  std::sort(s.begin(), s.end());
  double mean = 0;
  for (float x : ms) mean += x;
  mean /= ms.size();
  printf("{\"driver\": \"gs_bench\", \"what\": \"%s\", \"config\": %d, \"T\": %lld, \"B\": %lld, \"H\": %lld, "
         "\"launches\": %zu, \"kernel_ms\": %.5f, \"kernel_ms_median\": %.5f}\n",
         what, idx, T, B, H, ms.size(), mean, (double)s[s.size() / 2]);
  fflush(stdout);
}

template <typename F>
std::vector<float> time_launches(F&& launch, int launches, int warmup, hipStream_t st) {
  for (int i = 0; i < warmup; ++i) launch();
  CHECK(hipStreamSynchronize(st));
  std::vector<float> ms;
  int done = 0;
  while (done < launches) {
    const int n = std::min(50, launches - done);
    std::vector<hipEvent_t> a(n), b(n);
    for (int i = 0; i < n; ++i) {
      CHECK(hipEventCreate(&a[i]));
      CHECK(hipEventCreate(&b[i]));
    }
    hipLaunchKernelGGL(spin, dim3(1), dim3(64), 0, st, 20000000LL);
    CHECK(hipGetLastError());
    for (int i = 0; i < n; ++i) {
      CHECK(hipEventRecord(a[i], st));
      launch();
      CHECK(hipEventRecord(b[i], st));
    }
    CHECK(hipStreamSynchronize(st));
    for (int i = 0; i < n; ++i) {
      float x = 0;
      CHECK(hipEventElapsedTime(&x, a[i], b[i]));
      ms.push_back(x);
      CHECK(hipEventDestroy(a[i]));
      CHECK(hipEventDestroy(b[i]));
    }
    done += n;
  }
  return ms;
}

int run_copy(int mib, int launches) {
  const size_t n4 = (size_t)mib * (1 << 20) / 16;
  float4 *src, *dst;
  CHECK(hipMalloc(&src, n4 * 16));
  CHECK(hipMalloc(&dst, n4 * 16));
  CHECK(hipMemset(src, 0, n4 * 16));
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  auto launch = [&] {
    hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, st, src, dst, n4);
    CHECK(hipGetLastError());
  };
  auto ms = time_launches(launch, launches, 2, st);
  std::vector<float> s = ms;
  std::sort(s.begin(), s.end());
  printf("{\"driver\": \"gs_bench\", \"what\": \"copy\", \"bytes_read_per_launch\": %zu, "
         "\"bytes_written_per_launch\": %zu, \"launches\": %zu, \"kernel_ms_median\": %.5f}\n",
         n4 * 16, n4 * 16, ms.size(), (double)s[s.size() / 2]);
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  CHECK(hipStreamDestroy(st));
  return 0;
}

int run_config(int idx, int launches, int warmup) {
  const long long T = idx == 4 ? 512 : 64, B = idx == 4 ? 64 : 32, H = idx == 4 ? 1024 : 512;
  Rng g(idx + 1);
  const float k = 1.0f / std::sqrt((float)H);
  gs_args a;
  memset(&a, 0, sizeof a);
  std::vector<float*> owned;
  int kind = 0;
  if (idx == 0) {
    kind = GS_KIND_DIAGONAL;
    owned.push_back(upload(filled(3 * H, g, k)));
    a.w = owned.back();
  } else if (idx == 1 || idx == 2) {
    kind = GS_KIND_DENSE;
    owned.push_back(upload(filled(3 * H * H, g, k)));
    a.w = owned.back();
  } else if (idx == 3) {
    kind = GS_KIND_MONARCH;
    a.nblocks = 8;
    a.blksz = H / 8;
    owned.push_back(upload(filled(3 * H * a.blksz, g, 0.125f)));
    a.w = owned.back();
    owned.push_back(upload(filled(3 * H * a.blksz, g, 0.125f)));
    a.w2 = owned.back();
  } else {
    kind = GS_KIND_BUTTERFLY;
    a.log_n = 10;
    a.bfly_nblocks = 1;
    owned.push_back(upload(filled(3 * 10 * 512 * 4, g, 1.0f)));
    a.w = owned.back();
  }
  owned.push_back(upload(filled(3 * H, g, k)));
  a.bh = owned.back();
  owned.push_back(upload(filled((size_t)T * B * 3 * H, g, 1.7f)));
  a.gi = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)B * H, 0.0f)));
  a.h0 = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)T * B * H, 0.0f)));
  a.out = owned.back();
  a.T = T;
  a.B = B;
  a.H = H;
  a.sg_t = B * 3 * H;
  a.sg_b = 3 * H;
  a.sh0_b = H;
  a.so_t = B * H;
  a.so_b = H;
  if (idx == 2 || idx == 3) {
    const gs_quant q = {1, 1.0f / 127.0f, -127, 127};
    a.q_in = q;
    a.q_out = q;
  }
  const int64_t need = gs_workspace_bytes(kind, &a);
  if (need < 0) {
    fprintf(stderr, "gs_bench: gs_workspace_bytes: %s\n", gs_last_error());
    return 1;
  }
  void* ws = nullptr;
  CHECK(hipMalloc(&ws, need));
  CHECK(hipMemset(ws, 0, need));
  a.workspace = ws;
  a.workspace_bytes = need;
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  int rc = GS_OK;
  auto launch = [&] {
    switch (kind) {
      case GS_KIND_DIAGONAL: rc = gs_diagonal_fwd(&a, st); break;
      case GS_KIND_DENSE: rc = gs_dense_fwd(&a, st); break;
      case GS_KIND_MONARCH: rc = gs_monarch_fwd(&a, st); break;
      default: rc = gs_butterfly_fwd(&a, st); break;
    }
    if (rc != GS_OK) {
      fprintf(stderr, "gs_bench: launch failed (%d): %s\n", rc, gs_last_error());
      exit(1);
    }
  };
  auto ms = time_launches(launch, launches, warmup, st);
  rc = gs_workspace_status(ws, need, st);
  if (rc != GS_OK) {
    fprintf(stderr, "gs_bench: a poll timed out (workspace fault word set)\n");
    return 1;
  }
  report(kNames[idx], idx, ms, T, B, H);
  CHECK(hipFree(ws));
  for (float* p : owned) CHECK(hipFree(p));
  CHECK(hipStreamDestroy(st));
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: gs_bench <items: configs 0..4 and/or copy, comma-separated> [launches] [warmup]\n");
    return 2;
  }
  const int launches = argc > 2 ? atoi(argv[2]) : 30;
  const int warmup = argc > 3 ? atoi(argv[3]) : 10;
  if (launches < 1 || warmup < 0) return 2;
  char items[256];
  snprintf(items, sizeof items, "%s", argv[1]);
  char* save = nullptr;  // the HIP runtime may call strtok itself
  for (char* tok = strtok_r(items, ",", &save); tok; tok = strtok_r(nullptr, ",", &save)) {
    int rc;
    if (!strcmp(tok, "copy")) {
      rc = run_copy(256, launches);
    } else {
      char* end = nullptr;
      const long idx = strtol(tok, &end, 10);
      if (*tok == 0 || *end != 0 || idx < 0 || idx > 4) {
        fprintf(stderr, "gs_bench: unknown item '%s'\n", tok);
        return 2;
      }
      rc = run_config((int)idx, launches, warmup);
    }
    if (rc) return rc;
  }
  return 0;
}
