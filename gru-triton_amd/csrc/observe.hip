// Observer path (gfx950): the GRU scan and a tensor quantizer with per-tensor
// fake-quants whose scale is computed on the device from the tensor itself,
// and whose running statistics are updated, as GRULayer.calibrate runs them.
//
// Reference: the per-step path GRULayer.forward takes with use_triton off
// (LarocheC/gru-triton src/gru_qat/gru_layer.py:205-223) over step_with_gi
// (gru_cell.py:437-464), with FakeQuantize.forward (quantizers.py:84-96) in
// the dynamic or min_max mode: _compute_scale_zp of FakeQuantizePerTensor
// (quantizers.py:176-181) through _scale_zp_from_min_max (:124-134), then
// _update_observer (:136-156) in min_max mode, then fake_quant_ste
// (ste.py:65-95). calibrate (calibration.py:31-126, gru_layer.py:308-336)
// switches the activation quantizers to min_max and runs such forwards.
//
// A quantizer's scale depends on the min and max of the whole tensor it sees,
// so every step has a grid-wide reduction between computing h_t and
// quantizing it. The steps therefore run as short launches on the stream, with
// all scales kept on the device:
//   once:      the map as a dense [3H, H] matrix (gs_hidden_map_dense) unless
//              the kind is dense or diagonal; q_in's statistics of h0; hq_0.
//   per step:  gh = hq W^T + bh (MFMA GEMM, K-split partials; the diagonal kind
//              folds w_g * hq into the next kernel), the gates with a (min,
//              max) partial per workgroup (pre-quant h_t goes to out[t]), one
//              workgroup that reduces the partials and updates the scales and
//              statistics, and an elementwise pass that applies q_out to out[t]
//              in place and q_in for the next step's hq.
// fq is monotone, so the min and max of q_out(h_t), which q_in sees at step
// t + 1, are q_out of the pre-quant min and max: one reduction per step covers
// both quantizers.
#include "gs_gemm.h"

namespace gs {

int validate_map(const gs_map_args* a, const char* who);
int64_t hidden_map_scratch(const gs_map_args* a);
int materialize_map(const gs_map_args* a, hipStream_t stream, const char* who);

namespace {

constexpr int kRedThreads = 256;
constexpr int kMaxParts = 512;  // (min, max) partials of one reduction
constexpr int kMaxSplit = 8;    // K splits of the per-step GEMM
// _update_observer's mixing weights as the fp32 values torch multiplies by.
constexpr float kKeep = (float)0.99;
constexpr float kMix = (float)(1.0 - 0.99);

struct Obs {
  int mode, sym;
  float qmin, qmax, scale, zp;
  float* stats;
};

struct ObsPair {
  Obs in, out;
};

Obs to_obs(const gs_observer& o) {
  return Obs{o.mode, o.symmetric, (float)o.qmin, (float)o.qmax, o.scale, o.zero_point, o.stats};
}

__host__ __device__ inline bool is_dynamic(const Obs& o) {
  return o.mode == GS_OBS_DYNAMIC || o.mode == GS_OBS_MIN_MAX;
}

// fake_quant_ste's forward: clamp(round(x / s + zp), qmin, qmax), then (q - zp) s.
__device__ __forceinline__ float fq(float x, float s, float zp, float qmin, float qmax) {
#pragma clang fp contract(off)
  float v = __builtin_rintf(x / s + zp);
  v = __builtin_fminf(__builtin_fmaxf(v, qmin), qmax);
  return (v - zp) * s;
}

__device__ __forceinline__ void scale_zp(const Obs& o, float mn, float mx, float* s, float* zp) {
#pragma clang fp contract(off)
  if (o.sym) {
    const float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(mx), __builtin_fabsf(mn)), 1e-8f);
    *s = a / o.qmax;
    *zp = 0.0f;
  } else {
    *s = __builtin_fmaxf(mx - mn, 1e-8f) / (o.qmax - o.qmin);
    *zp = __builtin_rintf(o.qmin - mn / *s);
  }
}

__device__ __forceinline__ void observe(const Obs& o, float mn, float mx) {
  if (o.mode != GS_OBS_MIN_MAX) return;
  float* st = o.stats;
  if (st[2] == 0.0f) {
    st[0] = mn;
    st[1] = mx;
    st[2] = 1.0f;
  } else {
#pragma clang fp contract(off)
    st[0] = kKeep * st[0] + kMix * mn;
    st[1] = kKeep * st[1] + kMix * mx;
  }
}

// (min, max) over the workgroup, written by thread 0 to *dst.
__device__ __forceinline__ void block_minmax(float mn, float mx, float2* dst) {
  __shared__ float red[2][kRedThreads / 64];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mn = __builtin_fminf(mn, __shfl_xor(mn, o));
    mx = __builtin_fmaxf(mx, __shfl_xor(mx, o));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = mn;
    red[1][wave] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kRedThreads / 64; ++w) {
      mn = __builtin_fminf(mn, red[0][w]);
      mx = __builtin_fmaxf(mx, red[1][w]);
    }
    *dst = float2{mn, mx};
  }
}

__global__ __launch_bounds__(kRedThreads) void minmax_partials(const float* x, int64_t rows, int cols, int64_t ld,
                                                               float2* part) {
  float mn = __builtin_inff(), mx = -__builtin_inff();
  const int64_t n = rows * cols;
  for (int64_t e = blockIdx.x * (int64_t)kRedThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kRedThreads) {
    const int64_t r = e / cols;
    const float v = x[r * ld + (e - r * cols)];
    mn = __builtin_fminf(mn, v);
    mx = __builtin_fmaxf(mx, v);
  }
  block_minmax(mn, mx, part + blockIdx.x);
}

// One quantizer pass. Every workgroup first reduces the np (min, max)
// partials (np = 0: no dynamic quantizer needs them) and derives the scales
// itself; workgroup 0 alone writes them back to st, the trace and the running
// statistics. phase 0: the partials are of what c.in sees (h0, or the tensor of
// gs_observe_tensor), and hq = q_in(x). phase 1: they are of step t's
// pre-quant h_t in x, which c.out sees; then y = q_out(x) goes to dst (when
// apply_out) and, for step t + 1, hq = q_in(y), with q_in's scale from the min
// and max of y (q_out of the pre-quant ones). A word of st is written in a
// phase-1 launch only when its quantizer is dynamic, and read then by
// workgroup 0 alone (for the trace).
__global__ __launch_bounds__(kRedThreads) void quant_step(const float2* part, int np, ObsPair c, float* st,
                                                          float* trace, int t, int T, int phase, const float* x,
                                                          int64_t ldx, float* dst, int64_t ldd, float* hq,
                                                          int64_t rows, int cols, int apply_out) {
  __shared__ float2 tot;
  __shared__ float sc[4];
  float mn = __builtin_inff(), mx = -__builtin_inff();
  if (np > 0) {
    for (int i = threadIdx.x; i < np; i += kRedThreads) {
      mn = __builtin_fminf(mn, part[i].x);
      mx = __builtin_fmaxf(mx, part[i].y);
    }
    block_minmax(mn, mx, &tot);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const bool writer = blockIdx.x == 0;
    const bool din = is_dynamic(c.in), dout = is_dynamic(c.out);
    if (np > 0) {
      mn = tot.x;
      mx = tot.y;
    }
    float s_in = 1.0f, zp_in = 0.0f, s_out = 1.0f, zp_out = 0.0f;
    if (!din && c.in.mode == GS_OBS_FROZEN) {
      s_in = c.in.scale;
      zp_in = c.in.zp;
    }
    if (!dout && c.out.mode == GS_OBS_FROZEN) {
      s_out = c.out.scale;
      zp_out = c.out.zp;
    }
    if (phase == 0) {
      if (din) scale_zp(c.in, mn, mx, &s_in, &zp_in);
      if (writer) {
        if (din) observe(c.in, mn, mx);
        st[0] = s_in;  // no workgroup reads st in phase 0
        st[1] = zp_in;
      }
    } else {
      if (dout) {
        scale_zp(c.out, mn, mx, &s_out, &zp_out);
        if (writer) observe(c.out, mn, mx);
      }
      if (writer && trace != nullptr) {
        float* tr = trace + (int64_t)t * 4;
        tr[0] = din ? st[0] : s_in;  // the q_in scale step t used
        tr[1] = din ? st[1] : zp_in;
        tr[2] = s_out;
        tr[3] = zp_out;
      }
      if (din && t + 1 < T) {
        float a = mn, b = mx;
        if (c.out.mode != GS_OBS_OFF) {
          a = fq(mn, s_out, zp_out, c.out.qmin, c.out.qmax);
          b = fq(mx, s_out, zp_out, c.out.qmin, c.out.qmax);
        }
        scale_zp(c.in, a, b, &s_in, &zp_in);
        if (writer) {
          observe(c.in, a, b);
          st[0] = s_in;
          st[1] = zp_in;
        }
      }
    }
    sc[0] = s_in;
    sc[1] = zp_in;
    sc[2] = s_out;
    sc[3] = zp_out;
  }
  __syncthreads();
  const float s_in = sc[0], zp_in = sc[1], s_out = sc[2], zp_out = sc[3];
  const int64_t n = rows * cols;
  for (int64_t e = blockIdx.x * (int64_t)kRedThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kRedThreads) {
    const int64_t r = e / cols;
    const int k = (int)(e - r * cols);
    float v = x[r * ldx + k];
    if (apply_out) v = fq(v, s_out, zp_out, c.out.qmin, c.out.qmax);
    if (dst != nullptr) dst[r * ldd + k] = v;
    if (hq != nullptr) hq[e] = fq(v, s_in, zp_in, c.in.qmin, c.in.qmax);
  }
}

// The gates of one step; writes the pre-quant h_t to out_t and a (min, max)
// partial per workgroup. gh comes from `nsplit` GEMM partials [B, 3H] (split 0
// holds the bias), or, for the diagonal kind (dw != null), is dw_g * hq + bh_g.
__global__ __launch_bounds__(kRedThreads) void gates_step(const float* gi_t, int64_t sg_b, const float* gh, int nsplit,
                                                          int64_t split_stride, const float* dw, const float* bh,
                                                          const float* hq, int64_t shq_b, const float* hprev,
                                                          int64_t shp_b, float* out_t, int64_t so_b, int B, int H,
                                                          float2* part) {
  float mn = __builtin_inff(), mx = -__builtin_inff();
  const int64_t n = (int64_t)B * H;
  for (int64_t e = blockIdx.x * (int64_t)kRedThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kRedThreads) {
    const int b = (int)(e / H), k = (int)(e - (int64_t)b * H);
    float g3[3];
    if (dw != nullptr) {
      const float h = hq[(int64_t)b * shq_b + k];
#pragma unroll
      for (int g = 0; g < 3; ++g) {
#pragma clang fp contract(off)
        g3[g] = dw[g * H + k] * h + bh[g * H + k];
      }
    } else {
      const float* p = gh + (int64_t)b * 3 * H + k;
      float v[kMaxSplit][3];
#pragma unroll
      for (int q = 0; q < kMaxSplit; ++q)
#pragma unroll
        for (int g = 0; g < 3; ++g) v[q][g] = q < nsplit ? p[q * split_stride + g * H] : 0.0f;
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        float sum = v[0][g];
#pragma unroll
        for (int q = 1; q < kMaxSplit; ++q)
          if (q < nsplit) sum += v[q][g];
        g3[g] = sum;
      }
    }
    const float* gr = gi_t + (int64_t)b * sg_b + k;
    const float v = gru_update(gr[0], gr[H], gr[2 * H], g3[0], g3[1], g3[2], hprev[(int64_t)b * shp_b + k]);
    out_t[(int64_t)b * so_b + k] = v;
    mn = __builtin_fminf(mn, v);
    mx = __builtin_fmaxf(mx, v);
  }
  block_minmax(mn, mx, part + blockIdx.x);
}

int validate_observer(const gs_observer& o, const char* name, const char* who) {
  if (o.mode < GS_OBS_OFF || o.mode > GS_OBS_MIN_MAX)
    return set_error(GS_ERR_INVALID, "%s: %s mode %d is not a GS_OBS_* value", who, name, o.mode);
  if (o.mode == GS_OBS_OFF) return GS_OK;
  if (o.qmin > o.qmax)
    return set_error(GS_ERR_INVALID, "%s: %s qmin (%d) must be <= qmax (%d)", who, name, o.qmin, o.qmax);
  if (o.symmetric && o.qmax <= 0)
    return set_error(GS_ERR_INVALID, "%s: symmetric %s needs qmax > 0; got %d", who, name, o.qmax);
  if (!o.symmetric && o.qmax == o.qmin)
    return set_error(GS_ERR_INVALID, "%s: affine %s needs qmax > qmin", who, name);
  if (o.mode == GS_OBS_FROZEN && !(std::isfinite(o.scale) && o.scale > 0.0f && std::isfinite(o.zero_point)))
    return set_error(GS_ERR_INVALID, "%s: frozen %s needs a finite scale > 0 and a finite zero point", who, name);
  if (o.mode == GS_OBS_MIN_MAX && o.stats == nullptr)
    return set_error(GS_ERR_INVALID, "%s: %s in min_max mode needs its stats buffer", who, name);
  return GS_OK;
}

int check_plain_scratch(void* p, int64_t have, int64_t need, const char* who) {
  if (need <= 0) return GS_OK;
  if (p == nullptr || have < need)
    return set_error(GS_ERR_INVALID, "%s: scratch of %lld bytes required; got %lld", who, (long long)need,
                     (long long)have);
  if ((reinterpret_cast<uintptr_t>(p) & 255u) != 0)
    return set_error(GS_ERR_INVALID, "%s: scratch must be 256-byte aligned", who);
  return GS_OK;
}

unsigned parts_for(int64_t n) { return (unsigned)std::min<int64_t>((n + kRedThreads - 1) / kRedThreads, kMaxParts); }

dim3 grid1d(int64_t n) { return dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)); }

// Scratch of gs_observe_scan, each region 256-byte aligned:
// scales [4] | partials [kMaxParts] | hq [B, H] | gh [split][B, 3H] |
// map [3H, H] (Monarch, butterfly) | map construction scratch.
struct OPlan {
  bool gemm, own_map;
  int split;
  int64_t st, part, hq, gh, map, map_tmp;
  int64_t total() const { return st + part + hq + gh + map + map_tmp; }
};

gs_map_args map_view(const gs_observe_args* a) {
  gs_map_args m{};
  m.kind = a->kind;
  m.w = a->w;
  m.w2 = a->w2;
  m.H = a->H;
  m.nblocks = a->nblocks;
  m.blksz = a->blksz;
  m.log_n = a->log_n;
  m.bfly_nblocks = a->bfly_nblocks;
  return m;
}

int plan_observe(const gs_observe_args* a, OPlan* p, const char* who) {
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  gs_args f{};
  f.gi = a->gi;
  f.h0 = a->h0;
  f.w = a->w;
  f.bh = a->bh;
  f.out = a->out;
  f.T = a->T;
  f.B = a->B;
  f.H = a->H;
  f.sg_t = a->sg_t;
  f.sg_b = a->sg_b;
  f.sh0_b = a->sh0_b;
  f.so_t = a->so_t;
  f.so_b = a->so_b;
  int rc = validate_common(&f, who);
  if (rc) return rc;
  const gs_map_args m = map_view(a);
  rc = validate_map(&m, who);
  if (rc) return rc;
  rc = validate_observer(a->q_in, "h_in observer", who);
  if (rc) return rc;
  rc = validate_observer(a->q_out, "h_out observer", who);
  if (rc) return rc;
  const int64_t B = a->B, H = a->H;
  if (B * 3 * H > INT32_MAX / 4)
    return set_error(GS_ERR_INVALID, "%s: B * 3H = %lld is too large", who, (long long)(B * 3 * H));
  p->gemm = a->kind != GS_KIND_DIAGONAL;
  p->own_map = a->kind == GS_KIND_MONARCH || a->kind == GS_KIND_BUTTERFLY || a->kind == GS_KIND_CIRCULANT;
  // gh has only B rows: split K in up to 8 parts of >= 64 terms so that the
  // product spreads over a few hundred workgroups (the gates kernel sums them).
  p->split = p->gemm ? (int)std::max<int64_t>(1, std::min<int64_t>(kMaxSplit, H / 64)) : 1;
  p->st = 256;
  p->part = align256((int64_t)kMaxParts * 8);
  p->hq = align256(B * H * 4);
  p->gh = p->gemm ? align256((int64_t)p->split * B * 3 * H * 4) : 0;
  p->map = p->own_map ? align256(3 * H * H * 4) : 0;
  p->map_tmp = p->own_map ? hidden_map_scratch(&m) : 0;
  return GS_OK;
}

int64_t tensor_scratch(const gs_observe_tensor_args*) { return 256 + align256((int64_t)kMaxParts * 8); }

}  // namespace
}  // namespace gs

extern "C" int64_t gs_observe_scan_scratch_bytes(const gs_observe_args* a) {
  using namespace gs;
  OPlan p;
  const int rc = plan_observe(a, &p, "gs_observe_scan_scratch_bytes");
  if (rc) return rc;
  return p.total();
}

extern "C" int gs_observe_scan(const gs_observe_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_observe_scan";
  OPlan p;
  int rc = plan_observe(a, &p, who);
  if (rc) return rc;
  rc = check_plain_scratch(a->scratch, a->scratch_bytes, p.total(), who);
  if (rc) return rc;
  char* cur = static_cast<char*>(a->scratch);
  auto take = [&](int64_t bytes) {
    char* r = cur;
    cur += bytes;
    return r;
  };
  float* st = reinterpret_cast<float*>(take(p.st));
  float2* part = reinterpret_cast<float2*>(take(p.part));
  float* hq = reinterpret_cast<float*>(take(p.hq));
  float* gh = reinterpret_cast<float*>(take(p.gh));
  float* map = reinterpret_cast<float*>(take(p.map));
  void* map_tmp = take(p.map_tmp);

  const int T = (int)a->T, B = (int)a->B, H = (int)a->H;
  const ObsPair c{to_obs(a->q_in), to_obs(a->q_out)};
  const bool in_on = a->q_in.mode != GS_OBS_OFF, out_on = a->q_out.mode != GS_OBS_OFF;
  const int64_t BH = (int64_t)B * H;

  const float* W = a->w;
  if (p.own_map) {
    gs_map_args m = map_view(a);
    m.m = map;
    m.scratch = map_tmp;
    m.scratch_bytes = p.map_tmp;
    rc = materialize_map(&m, stream, who);
    if (rc) return rc;
    W = map;
  }
  const unsigned np = parts_for(BH);
  if (is_dynamic(c.in)) {
    hipLaunchKernelGGL(minmax_partials, dim3(np), dim3(kRedThreads), 0, stream, a->h0, (int64_t)B, H, a->sh0_b, part);
    GS_CHECK_HIP(hipGetLastError());
  }
  if (in_on) {
    hipLaunchKernelGGL(quant_step, grid1d(BH), dim3(kRedThreads), 0, stream, part, is_dynamic(c.in) ? (int)np : 0, c,
                       st, a->trace, 0, T, 0, a->h0, a->sh0_b, nullptr, (int64_t)0, hq, (int64_t)B, H, 0);
    GS_CHECK_HIP(hipGetLastError());
  }

  for (int t = 0; t < T; ++t) {
    const float* hprev = t == 0 ? a->h0 : a->out + (int64_t)(t - 1) * a->so_t;
    const int64_t shp = t == 0 ? a->sh0_b : a->so_b;
    const float* hm = in_on ? hq : hprev;  // the matmul-side h
    const int64_t shm = in_on ? H : shp;
    float* out_t = a->out + (int64_t)t * a->so_t;
    if (p.gemm) {
      GemmArgs g;
      g.a = hm;
      g.lda = shm;
      g.b = W;  // B(k, n) = W[n][k]
      g.ldb = H;
      g.c = gh;
      g.ldc = 3 * H;
      g.split_stride = (int64_t)B * 3 * H;
      g.bias = a->bh;
      g.M = B;
      g.N = 3 * H;
      g.K = H;
      g.ksplit = p.split;
      g.layout = kGemmNT;
      rc = gemm_f32(g, stream, who);
      if (rc) return rc;
    }
    hipLaunchKernelGGL(gates_step, dim3(np), dim3(kRedThreads), 0, stream, a->gi + (int64_t)t * a->sg_t, a->sg_b,
                       gh, p.split, (int64_t)B * 3 * H, p.gemm ? nullptr : a->w, a->bh, hm, shm, hprev, shp, out_t,
                       a->so_b, B, H, part);
    GS_CHECK_HIP(hipGetLastError());
    // q_out's pass runs every step: it also writes the trace
    const bool any_dyn = is_dynamic(c.in) || is_dynamic(c.out);
    float* hq_next = (in_on && t + 1 < T) ? hq : nullptr;
    hipLaunchKernelGGL(quant_step, grid1d(BH), dim3(kRedThreads), 0, stream, part, any_dyn ? (int)np : 0, c, st,
                       a->trace, t, T, 1, out_t, a->so_b, out_on ? out_t : nullptr, a->so_b, hq_next, (int64_t)B, H,
                       out_on ? 1 : 0);
    GS_CHECK_HIP(hipGetLastError());
  }
  return GS_OK;
}

extern "C" int64_t gs_observe_tensor_scratch_bytes(const gs_observe_tensor_args* a) {
  if (a == nullptr) return gs::set_error(GS_ERR_INVALID, "gs_observe_tensor_scratch_bytes: args is NULL");
  return gs::tensor_scratch(a);
}

extern "C" int gs_observe_tensor(const gs_observe_tensor_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_observe_tensor";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  if (a->rows < 1 || a->cols < 1 || a->cols > INT32_MAX || a->rows > (int64_t(1) << 40))
    return set_error(GS_ERR_INVALID, "%s: rows and cols must be > 0; got %lld, %lld", who, (long long)a->rows,
                     (long long)a->cols);
  if (a->rows > 1 && a->ld < a->cols)
    return set_error(GS_ERR_INVALID, "%s: row stride ld=%lld < cols=%lld", who, (long long)a->ld, (long long)a->cols);
  if (!a->x || !a->y) return set_error(GS_ERR_INVALID, "%s: x and y must be non-NULL device pointers", who);
  int rc = validate_observer(a->q, "observer", who);
  if (rc) return rc;
  rc = check_plain_scratch(a->scratch, a->scratch_bytes, tensor_scratch(a), who);
  if (rc) return rc;
  float* st = static_cast<float*>(a->scratch);
  float2* part = reinterpret_cast<float2*>(static_cast<char*>(a->scratch) + 256);
  // The tensor's quantizer takes the "in" slot of the scale words.
  const ObsPair c{to_obs(a->q), Obs{GS_OBS_OFF, 1, 0.f, 0.f, 1.f, 0.f, nullptr}};
  const int64_t n = a->rows * a->cols;
  const unsigned np = parts_for(n);
  if (is_dynamic(c.in)) {
    hipLaunchKernelGGL(minmax_partials, dim3(np), dim3(kRedThreads), 0, stream, a->x, a->rows, (int)a->cols, a->ld,
                       part);
    GS_CHECK_HIP(hipGetLastError());
  }
  // identity (observer off): y = x through the dst path; otherwise y = q(x)
  const bool off = c.in.mode == GS_OBS_OFF;
  hipLaunchKernelGGL(quant_step, grid1d(n), dim3(kRedThreads), 0, stream, part, is_dynamic(c.in) ? (int)np : 0, c, st,
                     nullptr, 0, 1, 0, a->x, a->ld, off ? a->y : nullptr, a->cols, off ? nullptr : a->y, a->rows,
                     (int)a->cols, 0);
  GS_CHECK_HIP(hipGetLastError());
  if (a->used != nullptr) GS_CHECK_HIP(hipMemcpyAsync(a->used, st, 2 * sizeof(float), hipMemcpyDeviceToDevice, stream));
  return GS_OK;
}
