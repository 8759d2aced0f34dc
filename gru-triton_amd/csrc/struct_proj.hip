// Structured input projection (gfx950): the gate inputs of a cell whose input
// side is structured, and their straight-through backward.
//
// Reference: GRUCellQuant.structured_input_projection (LarocheC/gru-triton
// src/gru_qat/gru_cell.py:466-503; per gate g: gi_g = quant_struct_Wi_g(
// struct_Wi_g(quant_x(x))) + b_ig, concatenated r, z, n), taken by
// GRULayer._forward_fast_dispatch when the input side is structured
// (gru_layer.py:256); the per-gate maps are the hidden-side kinds
// (structure.py:150-217) and the output quantizers fake_quant_ste
// (ste.py:65-95) with a per-tensor frozen scale or the per-row dynamic scale
// of FakeQuantizePerChannel on axis 0 (quantizers.py:124-134, 188-199).
//
// Forward: q_x(x) once into x_q (quant_copy); the map
//   diagonal   y = w_g * x_q elementwise, all three gates from one read of x_q;
//   Monarch    one batched MFMA GEMM, product (g, n) = block n of gate g:
//              y[:, g H + n bs + o] = sum_i x_q[:, n bs + i] W[g][n][o][i];
//   butterfly  the three gates' stages applied to the identity (the dense
//              [3H, H] map, scan_struct_bwd.hip) and one NT GEMM;
// then one workgroup per row applies the output quantizers and the bias
// (without output quantizers the map writes gi with the bias directly).
// Backward: a workgroup per (row, gate) takes dgi back through the output
// quantizer (the dynamic scale's path included), then the map's transpose
// and its weight gradient: diagonal elementwise with a deterministic
// column reduction; Monarch two batched GEMMs (NN per gate, summed; TN with
// a K split); butterfly NN and TN GEMMs against the dense map, the dense
// gradient carried onto the twiddles stage by stage.
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {

int bfly_materialize_keep(const float* tw, int nch, int L, int H, float* acts, float* M, hipStream_t stream);
int bfly_materialize(const float* tw, int nch, int L, int H, float* buf, float* M, hipStream_t stream);
int bfly_project_grad(const float* tw, int nch, int L, int H, const float* acts, const float* dM, float* gbuf,
                      float* dtw, hipStream_t stream);

// One gate's output quantizer on the device.
struct OQ {
  int mode;  // GS_OQ_*
  Quant q;   // GS_OQ_FROZEN
  float qmin, qmax;
};
struct OQ3 {
  OQ g[3];
};

constexpr int kSpThreads = 256;

// Sum (or max) over the workgroup's 256 threads; every thread gets the result.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(v, o);
    v = MAX ? fmaxf(v, u) : v + u;
  }
  __syncthreads();  // red may still be read by a previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kSpThreads / 64; ++w) r = MAX ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

// Backward of one row of a per-row dynamic symmetric fake-quant
// out_j = clamp(rint(y_j / s)) s with s = max(max_j |y_j|, 1e-8) / qmax, as
// torch's autograd differentiates FakeQuantizePerChannel + fake_quant_ste:
// STERound passes g_j, STEClamp passes it where rint(y_j / s) lies in
// [qmin, qmax] (mask m_j; |y_j / s| <= qmax, so only a range with
// qmin > -qmax clips, on the negative side), and the scale is a function of
// the row, so dL/ds = sum_j g_j (q_j - m_j y_j / s) reaches the row's max
// through |max| (if |max| >= |min|) and its min through |min| (if
// |min| >= |max|), halved on a tie of the two (torch.maximum), shared evenly
// by equal maxima (amax) or minima (amin), zero when the 1e-8 floor holds
// (clamp). The direct term is m_j g_j. d may alias g.
__device__ __forceinline__ void rows_dynamic_bwd(const float* y, float s, const float* g, float* d, int cols,
                                                 float qmin, float qmax, float* red) {
  float mx = -__builtin_inff(), mn = __builtin_inff();
  for (int k = threadIdx.x; k < cols; k += kSpThreads) {
    mx = fmaxf(mx, y[k]);
    mn = fminf(mn, y[k]);
  }
  mx = block_reduce<true>(mx, red);
  mn = -block_reduce<true>(-mn, red);
  float nmx = 0.f, nmn = 0.f, gs = 0.f;
  for (int k = threadIdx.x; k < cols; k += kSpThreads) {
    const float v = y[k], gk = g[k];
    const float r = __builtin_rintf(v / s);
    const float q = __builtin_fminf(__builtin_fmaxf(r, qmin), qmax);
    const bool keep = r >= qmin && r <= qmax;
    nmx += v == mx ? 1.f : 0.f;
    nmn += v == mn ? 1.f : 0.f;
    {
#pragma clang fp contract(off)
      gs += keep ? gk * q - gk * v / s : gk * q;
    }
  }
  nmx = block_reduce<false>(nmx, red);
  nmn = block_reduce<false>(nmn, red);
  gs = block_reduce<false>(gs, red);
  const float amx = fabsf(mx), amn = fabsf(mn);
  const float absmax = fmaxf(amx, amn);
  const float dabs = absmax >= 1e-8f ? gs / qmax : 0.0f;
  const float wmx = amx > amn ? 1.0f : (amx == amn ? 0.5f : 0.0f);
  const float wmn = amn > amx ? 1.0f : (amx == amn ? 0.5f : 0.0f);
  const float sgnmx = mx > 0.f ? 1.f : (mx < 0.f ? -1.f : 0.f);
  const float sgnmn = mn > 0.f ? 1.f : (mn < 0.f ? -1.f : 0.f);
  const float cmx = dabs * wmx * sgnmx / nmx, cmn = dabs * wmn * sgnmn / nmn;
  for (int k = threadIdx.x; k < cols; k += kSpThreads) {
    const float v = y[k];
    const float r = __builtin_rintf(v / s);
    float dk = (r >= qmin && r <= qmax) ? g[k] : 0.0f;
    if (v == mx) dk += cmx;
    if (v == mn) dk += cmn;
    d[k] = dk;
  }
}

// Rows of per-row dynamic fake-quant backward on a [rows, cols] matrix: y with
// row stride ldy, scales s[row], g / d with row strides ldg / ldd (d may alias
// g). The input projection's per-row weight quantizer uses it on the weight.
__global__ __launch_bounds__(kSpThreads) void rows_dynamic_bwd_kernel(const float* y, int64_t ldy, const float* s,
                                                                      const float* g, int64_t ldg, float* d,
                                                                      int64_t ldd, int cols, float qmin, float qmax) {
  __shared__ float red[kSpThreads / 64];
  const int64_t r = blockIdx.x;
  rows_dynamic_bwd(y + r * ldy, s[r], g + r * ldg, d + r * ldd, cols, qmin, qmax, red);
}

int launch_rows_dynamic_bwd(const float* y, int64_t ldy, const float* s, const float* g, int64_t ldg, float* d,
                            int64_t ldd, int rows, int cols, int qmin, int qmax, hipStream_t stream) {
  hipLaunchKernelGGL(rows_dynamic_bwd_kernel, dim3((unsigned)rows), dim3(kSpThreads), 0, stream, y, ldy, s, g, ldg, d,
                     ldd, cols, (float)qmin, (float)qmax);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

namespace {

dim3 grid_elems(int64_t n) { return dim3((unsigned)std::min<int64_t>((n + 255) / 256, 16384)); }

OQ to_oq(const gs_oquant& o) {
  OQ r;
  r.mode = o.mode;
  gs_quant q{o.mode == GS_OQ_FROZEN ? 1 : 0, o.mode == GS_OQ_FROZEN ? o.scale : 1.0f, o.qmin, o.qmax};
  r.q = to_quant(q);
  r.qmin = (float)o.qmin;
  r.qmax = (float)o.qmax;
  return r;
}

OQ3 to_oq3(const gs_oquant (&o)[3]) {
  OQ3 r;
  for (int g = 0; g < 3; ++g) r.g[g] = to_oq(o[g]);
  return r;
}

// ---- forward kernels ------------------------------------------------------------------

// y[m][g H + i] = x_q[m][i] w[g][i] (+ bias[g H + i] when bias != null); the
// product and the sum round separately, as x * weight then + b_i in torch.
__global__ void diag_map_kernel(const float* xq, int64_t ldx, const float* w, const float* bias, float* y,
                                int64_t ldy, int64_t M, int H) {
  const int64_t n = M * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / H;
    const int i = (int)(e - m * H);
    const float xv = xq[m * ldx + i];
#pragma unroll
    for (int g = 0; g < 3; ++g) {
#pragma clang fp contract(off)
      float v = xv * w[g * H + i];
      if (bias != nullptr) v = v + bias[g * H + i];
      y[m * ldy + g * H + i] = v;
    }
  }
}

// One workgroup per row m: gate g's output quantizer on y[m][g H ..], then
// the bias; writes gi and, for dynamic per-row gates, the row's scale.
__global__ __launch_bounds__(kSpThreads) void oq_rows_fwd(const float* y, const float* bias, float* gi, int64_t sgi,
                                                          float* y_scale, int64_t M, int H, OQ3 oq) {
  __shared__ float red[kSpThreads / 64];
  const int64_t m = blockIdx.x;
  const float* yr = y + m * 3 * H;
  float* gr = gi + m * sgi;
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const OQ o = oq.g[g];
    float s = 1.0f;
    if (o.mode == GS_OQ_DYNAMIC_ROWS) {
      float a = 0.0f;
      for (int k = threadIdx.x; k < H; k += kSpThreads) a = fmaxf(a, fabsf(yr[g * H + k]));
      a = block_reduce<true>(a, red);
      s = fmaxf(a, 1e-8f) / o.qmax;
      if (threadIdx.x == 0) y_scale[g * M + m] = s;
    }
    for (int k = threadIdx.x; k < H; k += kSpThreads) {
      float v = yr[g * H + k];
      if (o.mode == GS_OQ_DYNAMIC_ROWS)
        v = __builtin_fminf(__builtin_fmaxf(__builtin_rintf(v / s), o.qmin), o.qmax) * s;
      else if (o.mode == GS_OQ_FROZEN)
        v = fake_quant(v, o.q);
      if (bias != nullptr) {
#pragma clang fp contract(off)
        v = v + bias[g * H + k];
      }
      gr[g * H + k] = v;
    }
  }
}

// ---- backward kernels -----------------------------------------------------------------

// One workgroup per (row m, gate g): dy = d oq_g / dy applied to dgi.
__global__ __launch_bounds__(kSpThreads) void oq_rows_bwd(const float* y, const float* y_scale, const float* dgi,
                                                          int64_t sdgi, float* dy, int64_t M, int H, OQ3 oq) {
  __shared__ float red[kSpThreads / 64];
  const int64_t m = blockIdx.x;
  const int g = blockIdx.y;
  const OQ o = oq.g[g];
  const float* yr = y + m * 3 * H + g * H;
  const float* gr = dgi + m * sdgi + g * H;
  float* dr = dy + m * 3 * H + g * H;
  if (o.mode == GS_OQ_DYNAMIC_ROWS) {
    rows_dynamic_bwd(yr, y_scale[g * M + m], gr, dr, H, o.qmin, o.qmax, red);
    return;
  }
  for (int k = threadIdx.x; k < H; k += kSpThreads) {
    const float gk = gr[k];
    dr[k] = (o.mode == GS_OQ_FROZEN && !quant_keeps(yr[k], o.q)) ? 0.0f : gk;
  }
}

// dx[m][i] = q_x's clipped-STE mask at x[m][i] times
// sum_{p < parts} src[p][m][i] (parts apart by pstride, rows ld_src), or for
// the diagonal kind (w != null) sum_g w[g][i] dy[m][g H + i].
__global__ void gather_dx(const float* src, int64_t ld_src, int64_t pstride, int parts, const float* w, float* dx,
                          int64_t sdx, const float* x, int64_t sx, int64_t M, int H, Quant qx) {
  const int64_t n = M * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / H;
    const int i = (int)(e - m * H);
    float v = 0.0f;
    if (w != nullptr) {
#pragma clang fp contract(off)
      v = w[i] * src[m * ld_src + i] + w[H + i] * src[m * ld_src + H + i] + w[2 * H + i] * src[m * ld_src + 2 * H + i];
    } else {
      for (int p = 0; p < parts; ++p) v += src[p * pstride + m * ld_src + i];
    }
    if (qx.on && !quant_keeps(x[m * sx + i], qx)) v = 0.0f;
    dx[m * sdx + i] = v;
  }
}

constexpr int kDiagRows = 256;  // rows per partial column sum

// part[c][j] = sum over rows m of chunk c of dy[m][j] x_q[m][j % H] (j < 3H).
__global__ void diag_dw_partial(const float* dy, int64_t ldy, const float* xq, int64_t ldx, float* part, int64_t M,
                                int H) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= 3 * H) return;
  const int i = j % H;
  const int64_t m0 = (int64_t)blockIdx.y * kDiagRows;
  const int64_t m1 = m0 + kDiagRows < M ? m0 + kDiagRows : M;
  float acc = 0.0f;
  for (int64_t m = m0; m < m1; ++m) acc += dy[m * ldy + j] * xq[m * ldx + i];
  part[(int64_t)blockIdx.y * 3 * H + j] = acc;
}

// ---- planning -------------------------------------------------------------------------

struct SPlan {
  int kind = 0, H = 0, M = 0, nb = 0, bs = 0, L = 0, N = 0, nch = 0;
  bool any_oq = false, any_rows = false;
  // scratch layout (bytes)
  int64_t map_b = 0, acts_b = 0, gbuf_b = 0, dy_b = 0, xq_b = 0, part_b = 0, colp_b = 0, dm_b = 0;
  int64_t pp_b = 0;  // forward: two stage planes of the butterfly materialization
  int split = 1;
};

int validate_oq(const gs_oquant& o, int g, const char* who) {
  static const char* names[3] = {"r", "z", "n"};
  switch (o.mode) {
    case GS_OQ_OFF:
      return GS_OK;
    case GS_OQ_FROZEN: {
      gs_quant q{1, o.scale, o.qmin, o.qmax};
      char nm[32];
      snprintf(nm, sizeof nm, "out_quant[%s]", names[g]);
      return validate_quant(q, nm, who);
    }
    case GS_OQ_DYNAMIC_ROWS:
      if (!(o.qmax > 0) || o.qmin > o.qmax)
        return set_error(GS_ERR_INVALID, "%s: dynamic per-row out_quant[%s] needs qmax > 0 and qmin <= qmax; got [%d, %d]",
                         who, names[g], o.qmin, o.qmax);
      return GS_OK;
    default:
      return set_error(GS_ERR_INVALID, "%s: out_quant[%s] has unknown mode %d", who, names[g], o.mode);
  }
}

int plan(int32_t kind, int64_t M, int64_t H, int64_t nblocks, int64_t blksz, int64_t log_n, int64_t nch,
         const gs_quant& qx, const gs_oquant (&oq)[3], bool bwd, SPlan* p, const char* who) {
  // M: one workgroup per row in the output-quantizer kernels (256 threads each, fewer than
  // 2^32 work-items) and one grid row per kDiagRows rows in diag_dw_partial (gridDim.y <= 65535)
  constexpr int64_t kMaxRows = int64_t(65535) * kDiagRows;
  if (M < 1 || H < 1 || M > kMaxRows || H > 4096)
    return set_error(GS_ERR_INVALID, "%s: need 1 <= M <= %lld and 1 <= H <= 4096; got M=%lld, H=%lld", who,
                     (long long)kMaxRows, (long long)M, (long long)H);
  int rc = validate_quant(qx, "x_quant", who);
  if (rc) return rc;
  for (int g = 0; g < 3; ++g) {
    rc = validate_oq(oq[g], g, who);
    if (rc) return rc;
    p->any_oq |= oq[g].mode != GS_OQ_OFF;
    p->any_rows |= oq[g].mode == GS_OQ_DYNAMIC_ROWS;
  }
  p->kind = kind;
  p->M = (int)M;
  p->H = (int)H;
  switch (kind) {
    case GS_KIND_DIAGONAL:
      break;
    case GS_KIND_MONARCH:
      if (nblocks < 1 || blksz < 1 || nblocks * blksz != H)
        return set_error(GS_ERR_INVALID, "%s: Wi_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                         (long long)nblocks, (long long)blksz, (long long)H);
      if (3 * nblocks > 65535)
        return set_error(GS_ERR_INVALID, "%s: at most 21845 Monarch blocks; got %lld", who, (long long)nblocks);
      p->nb = (int)nblocks;
      p->bs = (int)blksz;
      break;
    case GS_KIND_BUTTERFLY:
      if (log_n < 1 || log_n > 12 || nch < 1 || nch > 64)
        return set_error(GS_ERR_INVALID, "%s: butterfly needs 1 <= log_n <= 12 and 1 <= nblocks <= 64; got %lld, %lld",
                         who, (long long)log_n, (long long)nch);
      if ((int64_t(1) << log_n) < H)
        return set_error(GS_ERR_INVALID, "%s: H_PAD = 2^log_n = %lld must be >= H = %lld", who,
                         (long long)(int64_t(1) << log_n), (long long)H);
      p->L = (int)log_n;
      p->N = 1 << p->L;
      p->nch = (int)nch;
      p->map_b = align256((int64_t)3 * H * H * 4);
      p->acts_b = align256((int64_t)3 * (p->nch * p->L + 1) * p->N * H * 4);
      p->pp_b = align256((int64_t)2 * 3 * p->N * H * 4);
      break;
    default:
      return set_error(GS_ERR_INVALID, "%s: structured input kind must be diagonal, Monarch or butterfly; got %d", who,
                       kind);
  }
  if (!bwd) return GS_OK;
  p->dy_b = p->any_oq ? align256((int64_t)M * 3 * H * 4) : 0;
  p->xq_b = align256((int64_t)M * H * 4);  // q_x(x) when the forward's x_q is not given
  p->colp_b = align256(colsum_partial_floats((int)M, (int)(3 * H)) * 4);
  switch (kind) {
    case GS_KIND_DIAGONAL:
      p->part_b = align256((int64_t)((M + kDiagRows - 1) / kDiagRows) * 3 * H * 4);
      break;
    case GS_KIND_MONARCH:
      p->split = gemm_pick_split(p->bs, p->bs, (int)M);
      if ((int64_t)3 * p->nb * p->split > 65535) p->split = (int)(65535 / (3 * p->nb));
      // dx partials per gate, and the weight gradient's K-split partials
      p->part_b = align256((int64_t)3 * M * H * 4) +
                  (p->split > 1 ? align256((int64_t)p->split * 3 * H * p->bs * 4) : 0);
      break;
    default:
      p->split = gemm_pick_split((int)(3 * H), (int)H, (int)M);
      p->dm_b = align256((int64_t)3 * H * H * 4);
      p->gbuf_b = align256((int64_t)2 * 3 * p->N * H * 4);
      p->part_b = align256((int64_t)M * H * 4) + (p->split > 1 ? align256((int64_t)p->split * 3 * H * H * 4) : 0);
      break;
  }
  return GS_OK;
}

// The forward keeps no stage activations (the backward recomputes them).
int64_t fwd_scratch(const SPlan& p) { return p.map_b + p.pp_b; }
int64_t bwd_scratch(const SPlan& p) {
  return p.map_b + p.acts_b + p.dm_b + p.gbuf_b + p.dy_b + p.xq_b + p.part_b + p.colp_b;
}

int check_buf(void* ptr, int64_t have, int64_t need, const char* who) {
  if (need <= 0) return GS_OK;
  if (ptr == nullptr || have < need)
    return set_error(GS_ERR_INVALID, "%s: scratch of %lld bytes required; got %lld", who, (long long)need,
                     (long long)have);
  if ((reinterpret_cast<uintptr_t>(ptr) & 255u) != 0)
    return set_error(GS_ERR_INVALID, "%s: scratch must be 256-byte aligned", who);
  return GS_OK;
}

// The map's forward: y (row stride ldy) = map(x_q) (+ bias when non-null).
int map_forward(const SPlan& p, const float* xq, int64_t ldx, const float* w, const float* bias, float* y,
                int64_t ldy, char* scratch, hipStream_t stream, const char* who) {
  const int M = p.M, H = p.H;
  if (p.kind == GS_KIND_DIAGONAL) {
    hipLaunchKernelGGL(diag_map_kernel, grid_elems((int64_t)M * H), dim3(256), 0, stream, xq, ldx, w, bias, y, ldy,
                       (int64_t)M, H);
    GS_CHECK_HIP(hipGetLastError());
    return GS_OK;
  }
  GemmArgs g;
  g.layout = kGemmNT;
  g.a = xq;
  g.lda = ldx;
  g.c = y;
  g.ldc = ldy;
  g.M = M;
  if (p.kind == GS_KIND_MONARCH) {
    // product z = gate * nb + block: A = x_q[:, block bs ...], B(k, o) = W[gate][block][o][k]
    g.b = w;
    g.ldb = p.bs;
    g.N = p.bs;
    g.K = p.bs;
    g.batch = 3 * p.nb;
    g.a_mod = p.nb;
    g.a_bs = p.bs;
    g.b_mod = 3 * p.nb;
    g.b_bs = (int64_t)p.bs * p.bs;
    g.c_bs = p.bs;  // columns gate H + block bs = z bs
    g.bias = bias;
    g.bias_bs = p.bs;
    return gemm_f32(g, stream, who);
  }
  float* map = reinterpret_cast<float*>(scratch);
  float* planes = reinterpret_cast<float*>(scratch + p.map_b);
  int rc = bfly_materialize(w, p.nch, p.L, H, planes, map, stream);
  if (rc) return rc;
  g.b = map;  // B(k, j) = map[j][k]
  g.ldb = H;
  g.N = 3 * H;
  g.K = H;
  g.bias = bias;
  return gemm_f32(g, stream, who);
}

}  // namespace
}  // namespace gs

extern "C" int64_t gs_struct_input_proj_scratch_bytes(const gs_sproj_args* a) {
  using namespace gs;
  if (a == nullptr) return set_error(GS_ERR_INVALID, "gs_struct_input_proj_scratch_bytes: args is NULL");
  SPlan p;
  const int rc = plan(a->kind, a->M, a->H, a->nblocks, a->blksz, a->log_n, a->bfly_nblocks, a->q_x, a->q_out, false,
                      &p, "gs_struct_input_proj_scratch_bytes");
  if (rc) return rc;
  return fwd_scratch(p);
}

extern "C" int gs_struct_input_proj(const gs_sproj_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_struct_input_proj";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  SPlan p;
  int rc = plan(a->kind, a->M, a->H, a->nblocks, a->blksz, a->log_n, a->bfly_nblocks, a->q_x, a->q_out, false, &p, who);
  if (rc) return rc;
  if (!a->x || !a->w || !a->gi) return set_error(GS_ERR_INVALID, "%s: x, w and gi must be non-NULL device pointers", who);
  if (a->sx < a->H || a->sgi < 3 * a->H)
    return set_error(GS_ERR_INVALID, "%s: row strides (sx=%lld, sgi=%lld) shorter than the rows", who,
                     (long long)a->sx, (long long)a->sgi);
  if (p.any_oq && a->y == nullptr)
    return set_error(GS_ERR_INVALID, "%s: y must be non-NULL when an output quantizer is on", who);
  if (p.any_rows && a->y_scale == nullptr)
    return set_error(GS_ERR_INVALID, "%s: y_scale must be non-NULL for a dynamic per-row output quantizer", who);
  if (a->q_x.enabled && a->x_q == nullptr)
    return set_error(GS_ERR_INVALID, "%s: x_q must be non-NULL when the x quantizer is on", who);
  rc = check_buf(a->scratch, a->scratch_bytes, fwd_scratch(p), who);
  if (rc) return rc;
  const int M = p.M, H = p.H;
  const float* xq = a->x;
  int64_t ldx = a->sx;
  if (a->q_x.enabled) {
    rc = quant_copy(a->x_q, a->x, a->sx, M, H, to_quant(a->q_x), stream, who);
    if (rc) return rc;
    xq = a->x_q;
    ldx = H;
  }
  if (!p.any_oq)
    return map_forward(p, xq, ldx, a->w, a->bias, a->gi, a->sgi, static_cast<char*>(a->scratch), stream, who);
  rc = map_forward(p, xq, ldx, a->w, nullptr, a->y, 3 * (int64_t)H, static_cast<char*>(a->scratch), stream, who);
  if (rc) return rc;
  hipLaunchKernelGGL(oq_rows_fwd, dim3((unsigned)M), dim3(kSpThreads), 0, stream, a->y, a->bias, a->gi, a->sgi,
                     a->y_scale, (int64_t)M, H, to_oq3(a->q_out));
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

extern "C" int64_t gs_struct_input_proj_bwd_scratch_bytes(const gs_sproj_bwd_args* a) {
  using namespace gs;
  if (a == nullptr) return set_error(GS_ERR_INVALID, "gs_struct_input_proj_bwd_scratch_bytes: args is NULL");
  SPlan p;
  const int rc = plan(a->kind, a->M, a->H, a->nblocks, a->blksz, a->log_n, a->bfly_nblocks, a->q_x, a->q_out, true,
                      &p, "gs_struct_input_proj_bwd_scratch_bytes");
  if (rc) return rc;
  return bwd_scratch(p);
}

extern "C" int gs_struct_input_proj_bwd(const gs_sproj_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_struct_input_proj_bwd";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  SPlan p;
  int rc = plan(a->kind, a->M, a->H, a->nblocks, a->blksz, a->log_n, a->bfly_nblocks, a->q_x, a->q_out, true, &p, who);
  if (rc) return rc;
  if (!a->x || !a->w || !a->dgi || !a->dx || !a->dw)
    return set_error(GS_ERR_INVALID, "%s: x, w, dgi, dx and dw must be non-NULL device pointers", who);
  if (a->sx < a->H || a->sdgi < 3 * a->H || a->sdx < a->H)
    return set_error(GS_ERR_INVALID, "%s: row strides shorter than the rows", who);
  if (p.any_oq && a->y == nullptr)
    return set_error(GS_ERR_INVALID, "%s: y (the forward's map outputs) must be non-NULL when an output quantizer is on",
                     who);
  if (p.any_rows && a->y_scale == nullptr)
    return set_error(GS_ERR_INVALID, "%s: y_scale must be non-NULL for a dynamic per-row output quantizer", who);
  rc = check_buf(a->scratch, a->scratch_bytes, bwd_scratch(p), who);
  if (rc) return rc;
  const int M = p.M, H = p.H;
  char* sc = static_cast<char*>(a->scratch);
  char* s_map = sc;
  char* s_dm = s_map + p.map_b + p.acts_b;
  char* s_gbuf = s_dm + p.dm_b;
  char* s_dy = s_gbuf + p.gbuf_b;
  char* s_xq = s_dy + p.dy_b;
  char* s_part = s_xq + p.xq_b;
  char* s_colp = s_part + p.part_b;
  const Quant qx = to_quant(a->q_x);

  if (a->dbias) {
    rc = colsum(a->dbias, a->dgi, a->sdgi, M, 3 * H, reinterpret_cast<float*>(s_colp), stream, who);
    if (rc) return rc;
  }
  // gradient reaching the map's output
  const float* dy = a->dgi;
  int64_t ldy = a->sdgi;
  if (p.any_oq) {
    float* dyb = reinterpret_cast<float*>(s_dy);
    hipLaunchKernelGGL(oq_rows_bwd, dim3((unsigned)M, 3), dim3(kSpThreads), 0, stream, a->y, a->y_scale, a->dgi,
                       a->sdgi, dyb, (int64_t)M, H, to_oq3(a->q_out));
    GS_CHECK_HIP(hipGetLastError());
    dy = dyb;
    ldy = 3 * (int64_t)H;
  }
  // the map's input: q_x(x)
  const float* xq = a->x;
  int64_t ldx = a->sx;
  if (qx.on) {
    if (a->x_q != nullptr) {
      xq = a->x_q;
    } else {
      rc = quant_copy(reinterpret_cast<float*>(s_xq), a->x, a->sx, M, H, qx, stream, who);
      if (rc) return rc;
      xq = reinterpret_cast<const float*>(s_xq);
    }
    ldx = H;
  }
  float* part = reinterpret_cast<float*>(s_part);

  if (p.kind == GS_KIND_DIAGONAL) {
    hipLaunchKernelGGL(gather_dx, grid_elems((int64_t)M * H), dim3(256), 0, stream, dy, ldy, (int64_t)0, 0, a->w, a->dx,
                       a->sdx, a->x, a->sx, (int64_t)M, H, qx);
    GS_CHECK_HIP(hipGetLastError());
    const int chunks = (M + kDiagRows - 1) / kDiagRows;
    hipLaunchKernelGGL(diag_dw_partial, dim3((unsigned)((3 * H + 255) / 256), (unsigned)chunks), dim3(256), 0, stream,
                       dy, ldy, xq, ldx, part, (int64_t)M, H);
    GS_CHECK_HIP(hipGetLastError());
    return sum_partials(a->dw, part, 3 * (int64_t)H, chunks, 3 * (int64_t)H, stream, who);
  }

  if (p.kind == GS_KIND_MONARCH) {
    const int nb = p.nb, bs = p.bs;
    // dx_g[:, n bs + i] = sum_o dy[:, g H + n bs + o] W[g][n][o][i], one batched NN product per gate
    for (int g = 0; g < 3; ++g) {
      GemmArgs d;
      d.layout = kGemmNN;
      d.a = dy + (int64_t)g * H;
      d.lda = ldy;
      d.b = a->w + (int64_t)g * nb * bs * bs;
      d.ldb = bs;
      d.c = part + (int64_t)g * M * H;
      d.ldc = H;
      d.M = M;
      d.N = bs;
      d.K = bs;
      d.batch = nb;
      d.a_bs = bs;
      d.a_mod = nb;
      d.b_bs = (int64_t)bs * bs;
      d.b_mod = nb;
      d.c_bs = bs;
      rc = gemm_f32(d, stream, who);
      if (rc) return rc;
    }
    hipLaunchKernelGGL(gather_dx, grid_elems((int64_t)M * H), dim3(256), 0, stream, part, (int64_t)H, (int64_t)M * H, 3,
                       nullptr, a->dx, a->sdx, a->x, a->sx, (int64_t)M, H, qx);
    GS_CHECK_HIP(hipGetLastError());
    // dW[g][n][o][i] = sum_m dy[m][g H + n bs + o] x_q[m][n bs + i]: TN, product z = g nb + n
    float* wpart = reinterpret_cast<float*>(s_part + align256((int64_t)3 * M * H * 4));
    GemmArgs t;
    t.layout = kGemmTN;
    t.a = dy;
    t.lda = ldy;
    t.b = xq;
    t.ldb = ldx;
    t.c = p.split > 1 ? wpart : a->dw;
    t.ldc = bs;
    t.split_stride = (int64_t)3 * H * bs;
    t.M = bs;
    t.N = bs;
    t.K = M;
    t.ksplit = p.split;
    t.batch = 3 * nb;
    t.a_bs = bs;
    t.a_mod = 3 * nb;
    t.b_bs = bs;
    t.b_mod = nb;
    t.c_bs = (int64_t)bs * bs;
    rc = gemm_f32(t, stream, who);
    if (rc) return rc;
    if (p.split > 1) return sum_partials(a->dw, wpart, (int64_t)3 * H * bs, p.split, (int64_t)3 * H * bs, stream, who);
    return GS_OK;
  }

  // butterfly: dense map M [3H, H] (stage activations kept), then
  // dx = dy M (NN), dM = dy^T x_q (TN), dM carried onto the twiddles
  float* map = reinterpret_cast<float*>(s_map);
  float* acts = reinterpret_cast<float*>(s_map + p.map_b);
  rc = bfly_materialize_keep(a->w, p.nch, p.L, H, acts, map, stream);
  if (rc) return rc;
  GemmArgs d;
  d.layout = kGemmNN;
  d.a = dy;
  d.lda = ldy;
  d.b = map;
  d.ldb = H;
  d.c = part;
  d.ldc = H;
  d.M = M;
  d.N = H;
  d.K = 3 * H;
  rc = gemm_f32(d, stream, who);
  if (rc) return rc;
  hipLaunchKernelGGL(gather_dx, grid_elems((int64_t)M * H), dim3(256), 0, stream, part, (int64_t)H, (int64_t)0, 1,
                     nullptr, a->dx, a->sdx, a->x, a->sx, (int64_t)M, H, qx);
  GS_CHECK_HIP(hipGetLastError());
  float* dm = reinterpret_cast<float*>(s_dm);
  float* mpart = reinterpret_cast<float*>(s_part + align256((int64_t)M * H * 4));
  GemmArgs t;
  t.layout = kGemmTN;
  t.a = dy;
  t.lda = ldy;
  t.b = xq;
  t.ldb = ldx;
  t.c = p.split > 1 ? mpart : dm;
  t.ldc = H;
  t.split_stride = (int64_t)3 * H * H;
  t.M = 3 * H;
  t.N = H;
  t.K = M;
  t.ksplit = p.split;
  rc = gemm_f32(t, stream, who);
  if (rc) return rc;
  if (p.split > 1) {
    rc = sum_partials(dm, mpart, (int64_t)3 * H * H, p.split, (int64_t)3 * H * H, stream, who);
    if (rc) return rc;
  }
  return bfly_project_grad(a->w, p.nch, p.L, H, acts, dm, reinterpret_cast<float*>(s_gbuf), a->dw, stream);
}
