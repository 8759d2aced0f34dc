// gs_bench -- benchmark driver for libgruscan through its C ABI.
//
//   gs_bench <items> [launches=30] [warmup=10]
//
// <items> is a comma-separated list of configs 0..5 (5: the single-factor
// Monarch form of config 3, not a BASELINE configuration) and "copy", run in that
// order in one process (one JSON line each). A config run builds the
// synthetic inputs of one of the five benchmark configurations (shapes,
// kinds and hidden quant of gru_qat_amd/configs.py;
// values from a fixed-seed generator, not the same draws as configs.py),
// calls the config's gs_*_fwd entry point `warmup` times, then `launches`
// times with a HIP event pair around each call on one stream (a spin kernel
// keeps the queue ahead of the device, so host overhead is not counted), and
// prints one JSON line with the mean and median launch duration.
//
// Items b0..b4 time the backward entry point of a configuration instead
// (gs_*_bwd on the forward's own output and a random upstream gradient),
// items c0..c4 the calibration forward (gs_observe_scan with both hidden
// quantizers as int8 symmetric min_max observers), items t1, t2 the dense
// training forward (gs_dense_fwd also storing gh through gs_args.gh_save),
// items s1, s2 the dense backward given that saved gh (gs_bwd_args.gh_saved),
// t5 and s5 the same for the single-factor Monarch configuration, i2 the
// int8-QAT dense configuration with Wh fake-quantized per row and passed with
// its codes (gs_quantize_rows, gs_weight_codes, gs_dense_fwd_i8w), and
// "proj" times the input projection at the benchmark shape (x [2048, 512],
// Wi_cat [1536, 512], int8 x and per-row weight fake-quant) forward and
// backward.
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

const char* kNames[6] = {"diagonal_fp32", "dense_fp32", "dense_int8_qat", "monarch_nb8_two_factor_int8",
                         "butterfly_fp32", "monarch_nb8_single_int8"};

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

enum Mode { kForward, kBackward, kCalibrate, kTrainForward, kSavedBackward, kInt8Weights };

int run_config(int idx, int launches, int warmup, Mode mode) {
  const bool backward = mode == kBackward || mode == kSavedBackward;
  const bool save = mode == kTrainForward || mode == kSavedBackward;
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
  } else if (idx == 3 || idx == 5) {
    kind = GS_KIND_MONARCH;
    a.nblocks = 8;
    a.blksz = H / 8;
    owned.push_back(upload(filled(3 * H * a.blksz, g, 0.125f)));
    a.w = owned.back();
    if (idx == 3) {
      owned.push_back(upload(filled(3 * H * a.blksz, g, 0.125f)));
      a.w2 = owned.back();
    }
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
  if (idx == 2 || idx == 3 || idx == 5) {
    const gs_quant q = {1, 1.0f / 127.0f, -127, 127};
    a.q_in = q;
    a.q_out = q;
  }
  int8_t* wcodes = nullptr;
  float* wscale = nullptr;
  if (mode == kInt8Weights) {
    if (idx != 2) {
      fprintf(stderr, "gs_bench: i%d: int8 weight codes are an option of configuration 2 only\n", idx);
      return 2;
    }
    // Wh fake-quantized per row (int8, qmax 127), then its codes recovered from it
    float* wq = nullptr;
    int32_t* exact = nullptr;
    CHECK(hipMalloc(&wq, sizeof(float) * 3 * H * H));
    CHECK(hipMalloc(&wcodes, 3 * H * H));
    CHECK(hipMalloc(&wscale, sizeof(float) * 3 * H));
    CHECK(hipMalloc(&exact, sizeof(int32_t) * 3 * H));
    gs_rows_args r;
    memset(&r, 0, sizeof r);
    r.w = a.w;
    r.scale = wscale;
    r.w_q = wq;
    r.rows = 3 * H;
    r.cols = H;
    r.qmin = -127;
    r.qmax = 127;
    if (gs_quantize_rows(&r, nullptr) != GS_OK ||
        gs_weight_codes(wq, 3 * H, H, wcodes, wscale, exact, nullptr) != GS_OK) {
      fprintf(stderr, "gs_bench: weight codes: %s\n", gs_last_error());
      return 1;
    }
    std::vector<int32_t> ex(3 * H);
    CHECK(hipMemcpy(ex.data(), exact, sizeof(int32_t) * 3 * H, hipMemcpyDeviceToHost));
    if (std::count(ex.begin(), ex.end(), 1) != 3 * H) {
      fprintf(stderr, "gs_bench: a fake-quantized row was not recovered as int8 codes\n");
      return 1;
    }
    CHECK(hipFree(exact));
    owned.push_back(wq);
    a.w = wq;
  }
  int64_t need = gs_workspace_bytes(kind, &a);
  if (need < 0) {
    fprintf(stderr, "gs_bench: gs_workspace_bytes: %s\n", gs_last_error());
    return 1;
  }
  gs_bwd_args b;
  memset(&b, 0, sizeof b);
  if (backward) {
    b.gi = a.gi;
    b.h0 = a.h0;
    b.w = a.w;
    b.w2 = a.w2;
    b.bh = a.bh;
    b.out = a.out;
    owned.push_back(upload(filled((size_t)T * B * H, g, 1.0f)));
    b.dout = owned.back();
    owned.push_back(upload(std::vector<float>((size_t)T * B * 3 * H, 0.0f)));
    b.dgi = owned.back();
    owned.push_back(upload(std::vector<float>((size_t)B * H, 0.0f)));
    b.dh0 = owned.back();
    const size_t nw = kind == GS_KIND_DENSE ? (size_t)3 * H * H
                      : kind == GS_KIND_MONARCH ? (size_t)3 * H * a.blksz
                      : kind == GS_KIND_DIAGONAL ? (size_t)B * 3 * H
                                                 : (size_t)3 * 10 * 512 * 4;
    owned.push_back(upload(std::vector<float>(nw, 0.0f)));
    b.dw_part = owned.back();
    if (a.w2) {
      owned.push_back(upload(std::vector<float>(nw, 0.0f)));
      b.dw2_part = owned.back();
    }
    owned.push_back(upload(std::vector<float>((size_t)B * 3 * H, 0.0f)));
    b.dbh_part = owned.back();
    b.T = T;
    b.B = B;
    b.H = H;
    b.sg_t = a.sg_t;
    b.sg_b = a.sg_b;
    b.sh0_b = a.sh0_b;
    b.so_t = a.so_t;
    b.so_b = a.so_b;
    b.nblocks = a.nblocks;
    b.blksz = a.blksz;
    b.log_n = a.log_n;
    b.bfly_nblocks = a.bfly_nblocks;
    b.q_in = a.q_in;
    b.q_out = a.q_out;
    const int64_t nb = gs_bwd_workspace_bytes(kind, &b);
    const int64_t ns = gs_bwd_scratch_bytes(kind, &b);
    if (nb < 0 || ns < 0) {
      fprintf(stderr, "gs_bench: gs_bwd_workspace_bytes / gs_bwd_scratch_bytes: %s\n", gs_last_error());
      return 1;
    }
    need = std::max(need, nb);
    if (ns > 0) {
      CHECK(hipMalloc(&b.scratch, ns));
      b.scratch_bytes = ns;
    }
  }
  gs_observe_args o;
  memset(&o, 0, sizeof o);
  float* stats = nullptr;
  if (mode == kCalibrate) {
    o.kind = kind;
    o.gi = a.gi;
    o.h0 = a.h0;
    o.w = a.w;
    o.w2 = a.w2;
    o.bh = a.bh;
    o.out = a.out;
    o.T = T;
    o.B = B;
    o.H = H;
    o.sg_t = a.sg_t;
    o.sg_b = a.sg_b;
    o.sh0_b = a.sh0_b;
    o.so_t = a.so_t;
    o.so_b = a.so_b;
    o.nblocks = a.nblocks;
    o.blksz = a.blksz;
    o.log_n = a.log_n;
    o.bfly_nblocks = a.bfly_nblocks;
    CHECK(hipMalloc(&stats, 6 * sizeof(float)));
    CHECK(hipMemset(stats, 0, 6 * sizeof(float)));  // not yet initialized
    const gs_observer q = {GS_OBS_MIN_MAX, 1, -127, 127, 1.0f, 0.0f, nullptr};
    o.q_in = q;
    o.q_in.stats = stats;
    o.q_out = q;
    o.q_out.stats = stats + 3;
    const int64_t ns = gs_observe_scan_scratch_bytes(&o);
    if (ns < 0) {
      fprintf(stderr, "gs_bench: gs_observe_scan_scratch_bytes: %s\n", gs_last_error());
      return 1;
    }
    CHECK(hipMalloc(&o.scratch, ns));
    o.scratch_bytes = ns;
  }
  float* gh = nullptr;
  if (save) {
    if (kind != GS_KIND_DENSE && !(kind == GS_KIND_MONARCH && a.w2 == nullptr)) {
      fprintf(stderr, "gs_bench: saved gh is an option of the dense and single-factor Monarch configurations "
                      "(1, 2, 5), not of %d\n", idx);
      return 2;
    }
    CHECK(hipMalloc(&gh, (size_t)T * B * 3 * H * sizeof(float)));
    a.gh_save = gh;
    if (backward) b.gh_saved = gh;
  }
  void* ws = nullptr;
  CHECK(hipMalloc(&ws, need));
  CHECK(hipMemset(ws, 0, need));
  a.workspace = ws;
  a.workspace_bytes = need;
  b.workspace = ws;
  b.workspace_bytes = need;
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  int rc = GS_OK;
  auto forward = [&] {
    switch (kind) {
      case GS_KIND_DIAGONAL: rc = gs_diagonal_fwd(&a, st); break;
      case GS_KIND_DENSE: rc = wcodes ? gs_dense_fwd_i8w(&a, wcodes, wscale, st) : gs_dense_fwd(&a, st); break;
      case GS_KIND_MONARCH: rc = gs_monarch_fwd(&a, st); break;
      default: rc = gs_butterfly_fwd(&a, st); break;
    }
    if (rc != GS_OK) {
      fprintf(stderr, "gs_bench: launch failed (%d): %s\n", rc, gs_last_error());
      exit(1);
    }
  };
  auto launch = [&] {
    if (mode == kCalibrate) {
      rc = gs_observe_scan(&o, st);
      if (rc != GS_OK) {
        fprintf(stderr, "gs_bench: gs_observe_scan failed (%d): %s\n", rc, gs_last_error());
        exit(1);
      }
      return;
    }
    if (!backward) return forward();
    switch (kind) {
      case GS_KIND_DIAGONAL: rc = gs_diagonal_bwd(&b, st); break;
      case GS_KIND_DENSE: rc = gs_dense_bwd(&b, st); break;
      case GS_KIND_MONARCH: rc = gs_monarch_bwd(&b, st); break;
      default: rc = gs_butterfly_bwd(&b, st); break;
    }
    if (rc != GS_OK) {
      fprintf(stderr, "gs_bench: backward launch failed (%d): %s\n", rc, gs_last_error());
      exit(1);
    }
  };
  if (backward) forward();  // out for the backward
  auto ms = time_launches(launch, launches, warmup, st);
  rc = gs_workspace_status(ws, need, st);
  if (rc != GS_OK) {
    fprintf(stderr, "gs_bench: a poll timed out (workspace fault word set)\n");
    return 1;
  }
  if (mode != kForward) {
    char name[64];
    snprintf(name, sizeof name, "%s_%s", kNames[idx],
             mode == kBackward        ? "backward"
             : mode == kSavedBackward ? "backward_saved_gh"
             : mode == kTrainForward  ? "train_forward"
             : mode == kInt8Weights   ? "int8_weight_codes"
                                      : "calibration");
    report(name, idx, ms, T, B, H);
  } else {
    report(kNames[idx], idx, ms, T, B, H);
  }
  CHECK(hipFree(ws));
  if (gh) CHECK(hipFree(gh));
  if (wcodes) CHECK(hipFree(wcodes));
  if (wscale) CHECK(hipFree(wscale));
  if (b.scratch) CHECK(hipFree(b.scratch));
  if (o.scratch) CHECK(hipFree(o.scratch));
  if (stats) CHECK(hipFree(stats));
  for (float* p : owned) CHECK(hipFree(p));
  CHECK(hipStreamDestroy(st));
  return 0;
}

int run_proj(int launches, int warmup) {
  const int64_t M = 2048, N = 1536, I = 512;
  Rng g(11);
  std::vector<float*> owned;
  owned.push_back(upload(filled((size_t)M * I, g, 1.0f)));
  float* x = owned.back();
  owned.push_back(upload(filled((size_t)N * I, g, 0.044f)));
  float* w = owned.back();
  owned.push_back(upload(filled((size_t)N, g, 0.044f)));
  float* bias = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)M * N, 0.0f)));
  float* gi = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)N * I, 0.0f)));
  float* wq = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)M * I, 0.0f)));
  float* xq = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)N, 0.0f)));
  float* sc = owned.back();
  owned.push_back(upload(filled((size_t)M * N, g, 1.0f)));
  float* dgi = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)M * I, 0.0f)));
  float* dx = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)N * I, 0.0f)));
  float* dw = owned.back();
  owned.push_back(upload(std::vector<float>((size_t)N, 0.0f)));
  float* db = owned.back();
  gs_proj_args p;
  memset(&p, 0, sizeof p);
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.gi = gi;
  p.x_q = xq;
  p.w_q = wq;
  p.w_scale = sc;
  p.M = M;
  p.N = N;
  p.I = I;
  p.sx = I;
  p.sgi = N;
  p.q_x = gs_quant{1, 0.02f, -127, 127};
  p.q_w = gs_quant{1, 1.0f, -127, 127};
  // int8 scratch: x's levels and the weight's codes (the int8 product)
  int8_t* xc = nullptr;
  int8_t* wc = nullptr;
  CHECK(hipMalloc(&xc, (size_t)M * I));
  CHECK(hipMalloc(&wc, (size_t)N * I));
  p.x_codes = xc;
  p.w_codes = wc;
  gs_proj_bwd_args q;
  memset(&q, 0, sizeof q);
  q.x = x;
  q.w = wq;
  q.x_q = xq;
  q.dgi = dgi;
  q.dx = dx;
  q.dw = dw;
  q.dbias = db;
  q.M = M;
  q.N = N;
  q.I = I;
  q.sx = I;
  q.sdgi = N;
  q.sdx = I;
  q.q_x = p.q_x;
  const int64_t need = gs_input_proj_bwd_workspace_bytes(&q);
  void* ws = nullptr;
  CHECK(hipMalloc(&ws, need));
  q.workspace = ws;
  q.workspace_bytes = need;
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  auto fwd = [&] {
    if (gs_input_proj(&p, st) != GS_OK) {
      fprintf(stderr, "gs_bench: gs_input_proj: %s\n", gs_last_error());
      exit(1);
    }
  };
  auto bwd = [&] {
    if (gs_input_proj_bwd(&q, st) != GS_OK) {
      fprintf(stderr, "gs_bench: gs_input_proj_bwd: %s\n", gs_last_error());
      exit(1);
    }
  };
  report("input_projection", -1, time_launches(fwd, launches, warmup, st), 64, 32, 512);
  report("input_projection_backward", -1, time_launches(bwd, launches, warmup, st), 64, 32, 512);
  CHECK(hipFree(ws));
  CHECK(hipFree(xc));
  CHECK(hipFree(wc));
  for (float* o : owned) CHECK(hipFree(o));
  CHECK(hipStreamDestroy(st));
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: gs_bench <items: configs 0..5, b0..b5 (backward), c0..c5 (calibration), "
                    "t1, t2, t5 (training forward), s1, s2, s5 (backward on the saved gh), i2 (int8 weight "
                    "codes), proj, copy; "
                    "comma-separated> "
                    "[launches] [warmup]\n");
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
    } else if (!strcmp(tok, "proj")) {
      rc = run_proj(launches, warmup);
    } else {
      const Mode mode = tok[0] == 'b'   ? kBackward
                        : tok[0] == 'c' ? kCalibrate
                        : tok[0] == 't' ? kTrainForward
                        : tok[0] == 's' ? kSavedBackward
                        : tok[0] == 'i' ? kInt8Weights
                                        : kForward;
      const char* num = mode == kForward ? tok : tok + 1;
      char* end = nullptr;
      const long idx = strtol(num, &end, 10);
      if (*num == 0 || *end != 0 || idx < 0 || idx > 5) {
        fprintf(stderr, "gs_bench: unknown item '%s'\n", tok);
        return 2;
      }
      rc = run_config((int)idx, launches, warmup, mode);
    }
    if (rc) return rc;
  }
  return 0;
}
