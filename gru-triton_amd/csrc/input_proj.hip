// Input projection that produces the scan's gate inputs (gfx950):
//   gi = q_x(x) W_q^T + bi,   W_q = per-row int8 fake-quant of Wi_cat
// and its backward.
//
// Reference: GRULayer._forward_fast_dispatch (LarocheC/gru-triton
// src/gru_qat/gru_layer.py:249-255: xq = quant_x(x); Wi_cat, bi_cat =
// cell.quantize_input_weights(); gi = F.linear(xq, Wi_cat, bi_cat)), the
// weight quantizer FakeQuantizePerChannel (quantizers.py:188-199) with its
// symmetric scale (quantizers.py:124-134: scale = max(|min|, |max|) clamped to
// 1e-8, over qmax), and fake_quant_ste (ste.py:65-95) for both quantizers.
//
// The forward is one NT GEMM (gemm.hip) whose epilogue adds bi. q_x is applied
// either by one elementwise pass into a caller buffer (x_q), which the
// backward reuses, or as the GEMM loads x (the fake-quant prologue; that
// repeats the quantization once per output tile and measured 25 % slower).
// The weight is fake-quantized once per call by a row kernel (a reduction for
// the row's absmax, then the codes), which also returns the per-row scales.
// The backward follows the straight-through estimator: dx = mask_x (dgi W_q) with q_x's clipped-STE
// mask, dW = dgi^T q_x(x) (the gradient reaching W_q; the per-row clamp never
// clips, since every |W / scale| <= qmax) plus, as the reference's autograd
// has it for a scale computed from the weight itself, each row scale's
// gradient carried to the row's max and min elements (launch_rows_dynamic_bwd,
// struct_proj.hip); dbi = column sums of dgi. x's frozen scale is a constant.
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kRowThreads = 256;

// One workgroup per row of w [rows, cols]: the row's scale, then wq = the
// fake-quantized row (when wq != null) and its integer codes (when codes != null).
__global__ __launch_bounds__(kRowThreads) void weight_quant_rows(const float* w, int cols, float qmin, float qmax,
                                                                 float* wq, float* scale_out, int8_t* codes) {
  __shared__ float red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const float* src = w + row * cols;
  float m = 0.0f;
  for (int k = threadIdx.x; k < cols; k += kRowThreads) m = fmaxf(m, fabsf(src[k]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float absmax = red[0];
  for (int i = 1; i < kRowThreads / 64; ++i) absmax = fmaxf(absmax, red[i]);
  const float scale = fmaxf(absmax, 1e-8f) / qmax;
  for (int k = threadIdx.x; k < cols; k += kRowThreads) {
    const float c = __builtin_fminf(__builtin_fmaxf(__builtin_rintf(src[k] / scale), qmin), qmax);
    if (wq != nullptr) wq[row * cols + k] = c * scale;  // fake_quant of src[k] at this scale
    if (codes != nullptr) codes[row * cols + k] = (int8_t)c;
  }
  if (threadIdx.x == 0) scale_out[row] = scale;
}

// One wave per row of an already fake-quantized weight w [rows, cols]: finds a
// scale s for which every element is fl(c * s) with an integer code |c| <= 127
// (the candidates are fl(max|w| / 127) and its neighbours up to two ulps away,
// the scales weight_quant_rows' rule can have produced), then writes s, the
// codes and exact[row] = 1; exact[row] = 0 (codes 0) when no candidate fits.
__global__ __launch_bounds__(64) void recover_codes_rows(const float* w, int cols, int8_t* codes, float* scale_out,
                                                         int32_t* exact) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* src = w + row * cols;
  float m = 0.0f;
  for (int k = lane; k < cols; k += 64) m = fmaxf(m, fabsf(src[k]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  bool found = m == 0.0f;  // an all-zero row: codes 0 at any scale
  float s = 1.0f;
  const float s0 = m / 127.0f;
  for (int d = 0; d < 5 && !found; ++d) {
    const int step = d == 0 ? 0 : (d & 1) ? (d + 1) / 2 : -(d / 2);  // 0, +1, -1, +2, -2 ulps
    const float sc = __int_as_float(__float_as_int(s0) + step);
    bool ok = sc > 0.0f && sc < __builtin_inff();
    for (int k = lane; k < cols && ok; k += 64) {
      const float c = __builtin_rintf(src[k] / sc);
      ok = fabsf(c) <= 127.0f && c * sc == src[k];
    }
    if (__all(ok)) {
      found = true;
      s = sc;
    }
  }
  for (int k = lane; k < cols; k += 64) codes[row * cols + k] = found ? (int8_t)__builtin_rintf(src[k] / s) : 0;
  if (lane == 0) {
    scale_out[row] = s;
    exact[row] = found ? 1 : 0;
  }
}

// dx[m][i] = 0 where q_x clipped x[m][i].
__global__ void mask_clipped(float* dx, int64_t sdx, const float* x, int64_t sx, int rows, int cols, Quant q) {
  const int64_t n = (int64_t)rows * cols;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / cols;
    const int i = (int)(e - m * cols);
    if (!quant_keeps(x[m * sx + i], q)) dx[m * sdx + i] = 0.0f;
  }
}

int validate_proj(int64_t M, int64_t N, int64_t I, const char* who) {
  if (M < 1 || N < 1 || I < 1)
    return set_error(GS_ERR_INVALID, "%s: M, N and I must be > 0; got M=%lld, N=%lld, I=%lld", who, (long long)M,
                     (long long)N, (long long)I);
  if (M > INT32_MAX / 4 || N > (1 << 20) || I > (1 << 20))
    return set_error(GS_ERR_INVALID, "%s: dims out of supported range (M=%lld, N=%lld, I=%lld)", who, (long long)M,
                     (long long)N, (long long)I);
  return GS_OK;
}

// K split of the dx product (dx contiguous only: the split sums run over
// whole planes). At the benchmark shape its 256 tiles fill the CUs once per
// split: 2 splits, 512 workgroups, instead of one workgroup per CU.
int dx_split(const gs_proj_bwd_args* a) {
  return a->sdx == a->I ? gemm_pick_split((int)a->M, (int)a->I, (int)a->N) : 1;
}

// workspace: colsum partials | dW split partials | dx split partials
int64_t proj_bwd_bytes(const gs_proj_bwd_args* a) {
  const int split = gemm_pick_split((int)a->N, (int)a->I, (int)a->M);
  const int dxs = dx_split(a);
  return align256(colsum_partial_floats((int)a->M, (int)a->N) * 4) +
         (split > 1 ? align256((int64_t)split * a->N * a->I * 4) : 0) +
         (dxs > 1 ? align256((int64_t)dxs * a->M * a->I * 4) : 0);
}

}  // namespace
}  // namespace gs

extern "C" int gs_input_proj(const gs_proj_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_input_proj";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  int rc = validate_proj(a->M, a->N, a->I, who);
  if (rc) return rc;
  if (!a->x || !a->w || !a->gi)
    return set_error(GS_ERR_INVALID, "%s: x, w and gi must be non-NULL device pointers", who);
  if (a->sx < a->I || a->sgi < a->N)
    return set_error(GS_ERR_INVALID, "%s: row strides (sx=%lld, sgi=%lld) shorter than the rows", who,
                     (long long)a->sx, (long long)a->sgi);
  rc = validate_quant(a->q_x, "x_quant", who);
  if (rc) return rc;
  const float* w = a->w;
  if (a->q_w.enabled) {
    if (!a->w_q || !a->w_scale)
      return set_error(GS_ERR_INVALID, "%s: w_q and w_scale must be non-NULL when the weight quant is on", who);
    if (!(a->q_w.qmax > 0) || a->q_w.qmin > a->q_w.qmax)
      return set_error(GS_ERR_INVALID, "%s: weight quant needs qmax > 0 and qmin <= qmax; got [%d, %d]", who,
                       a->q_w.qmin, a->q_w.qmax);
    // the codes too when the int8 product may run (int8 scratch given, byte range)
    int8_t* codes = a->w_codes != nullptr && a->q_w.qmin >= -128 && a->q_w.qmax <= 127 ? a->w_codes : nullptr;
    hipLaunchKernelGGL(weight_quant_rows, dim3((unsigned)a->N), dim3(kRowThreads), 0, stream, a->w, (int)a->I,
                       (float)a->q_w.qmin, (float)a->q_w.qmax, a->w_q, a->w_scale, codes);
    GS_CHECK_HIP(hipGetLastError());
    w = a->w_q;
  }
  // Both operands int8 (the int8 QAT layer: q_x and the per-row weight quant
  // with byte ranges) and the int8 scratch given: the pre-passes write x's
  // levels and the weight's codes, and the product runs on the int8 MFMA, exact
  // integer sums scaled once (gemm_i8_nt).
  const bool i8 = a->q_x.enabled && a->q_x.qmin >= -128 && a->q_x.qmax <= 127 && a->q_w.enabled &&
                  a->q_w.qmin >= -128 && a->q_w.qmax <= 127 && a->x_codes != nullptr && a->w_codes != nullptr;
  if (i8) {
    GemmI8Args h;
    h.a = a->x_codes;
    h.lda = a->I;
    h.sa = a->q_x.scale;
    h.b = a->w_codes;
    h.ldb = a->I;
    h.b_scale = a->w_scale;
    h.bias = a->bias;
    h.c = a->gi;
    h.ldc = a->sgi;
    h.M = (int)a->M;
    h.N = (int)a->N;
    h.K = (int)a->I;
    if (gemm_i8_applies(h)) {
      rc = quant_copy_codes(a->x_q, a->x_codes, a->x, a->sx, (int)a->M, (int)a->I, to_quant(a->q_x), stream, who);
      if (rc) return rc;
      return gemm_i8_nt(h, stream, who);
    }
  }
  GemmArgs g;
  g.a = a->x;
  g.lda = a->sx;
  g.qa = to_quant(a->q_x);
  if (a->q_x.enabled && a->x_q) {
    // one fake-quant pass instead of one per output tile of the GEMM
    rc = quant_copy(a->x_q, a->x, a->sx, (int)a->M, (int)a->I, g.qa, stream, who);
    if (rc) return rc;
    g.a = a->x_q;
    g.lda = a->I;
    g.qa.on = 0;
  }
  g.b = w;  // B(k, n) = W[n][k]
  g.ldb = a->I;
  g.c = a->gi;
  g.ldc = a->sgi;
  g.bias = a->bias;
  g.M = (int)a->M;
  g.N = (int)a->N;
  g.K = (int)a->I;
  g.layout = kGemmNT;
  return gemm_f32(g, stream, who);
}

extern "C" int64_t gs_input_proj_bwd_workspace_bytes(const gs_proj_bwd_args* a) {
  using namespace gs;
  if (a == nullptr) return set_error(GS_ERR_INVALID, "gs_input_proj_bwd_workspace_bytes: args is NULL");
  const int rc = validate_proj(a->M, a->N, a->I, "gs_input_proj_bwd_workspace_bytes");
  if (rc) return rc;
  return proj_bwd_bytes(a);
}

extern "C" int gs_input_proj_bwd(const gs_proj_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_input_proj_bwd";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  int rc = validate_proj(a->M, a->N, a->I, who);
  if (rc) return rc;
  if (!a->x || !a->w || !a->dgi || !a->dx || !a->dw)
    return set_error(GS_ERR_INVALID, "%s: x, w, dgi, dx and dw must be non-NULL device pointers", who);
  if (a->sx < a->I || a->sdgi < a->N || a->sdx < a->I)
    return set_error(GS_ERR_INVALID, "%s: row strides shorter than the rows", who);
  rc = validate_quant(a->q_x, "x_quant", who);
  if (rc) return rc;
  const int64_t need = proj_bwd_bytes(a);
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return set_error(GS_ERR_INVALID, "%s: workspace of %lld bytes required; got %lld", who, (long long)need,
                     (long long)a->workspace_bytes);
  const int M = (int)a->M, N = (int)a->N, I = (int)a->I;
  const Quant qx = to_quant(a->q_x);
  float* colp = static_cast<float*>(a->workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + align256(colsum_partial_floats(M, N) * 4));
  const int split = gemm_pick_split(N, I, M);
  const int dxs = dx_split(a);
  float* part_dx = reinterpret_cast<float*>(reinterpret_cast<char*>(part) +
                                            (split > 1 ? align256((int64_t)split * N * I * 4) : 0));

  // dx = dgi W  (NN: A(m, n) = dgi[m][n], B(n, i) = W[n][i]), then q_x's mask
  GemmArgs g;
  g.a = a->dgi;
  g.lda = a->sdgi;
  g.b = a->w;
  g.ldb = I;
  g.c = dxs > 1 ? part_dx : a->dx;
  g.ldc = dxs > 1 ? I : a->sdx;
  g.split_stride = (int64_t)M * I;
  g.M = M;
  g.N = I;
  g.K = N;
  g.ksplit = dxs;
  g.layout = kGemmNN;
  rc = gemm_f32(g, stream, who);
  if (rc) return rc;
  if (dxs > 1) {
    rc = sum_partials(a->dx, part_dx, (int64_t)M * I, dxs, (int64_t)M * I, stream, who);
    if (rc) return rc;
  }
  if (qx.on) {
    const int64_t n = (int64_t)M * I;
    hipLaunchKernelGGL(mask_clipped, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256), 0, stream,
                       a->dx, a->sdx, a->x, a->sx, M, I, qx);
    GS_CHECK_HIP(hipGetLastError());
  }

  // dW = dgi^T q_x(x)  (TN: A(n, m) = dgi[m][n], B(m, i) = q_x(x[m][i]))
  GemmArgs h;
  h.a = a->dgi;
  h.lda = a->sdgi;
  h.b = a->x_q ? a->x_q : a->x;
  h.ldb = a->x_q ? I : a->sx;
  h.c = split > 1 ? part : a->dw;
  h.ldc = I;
  h.split_stride = (int64_t)N * I;
  h.M = N;
  h.N = I;
  h.K = M;
  h.ksplit = split;
  h.layout = kGemmTN;
  if (!a->x_q) h.qb = qx;
  rc = gemm_f32(h, stream, who);
  if (rc) return rc;
  if (split > 1) {
    rc = sum_partials(a->dw, part, (int64_t)N * I, split, (int64_t)N * I, stream, who);
    if (rc) return rc;
  }
  if (a->q_w.enabled) {
    // the per-row weight scales depend on the weight: add their gradient path
    if (!a->w_raw || !a->w_scale)
      return set_error(GS_ERR_INVALID, "%s: w_raw and w_scale must be non-NULL when the weight quant is on", who);
    if (!(a->q_w.qmax > 0) || a->q_w.qmin > a->q_w.qmax)
      return set_error(GS_ERR_INVALID, "%s: weight quant needs qmax > 0 and qmin <= qmax; got [%d, %d]", who,
                       a->q_w.qmin, a->q_w.qmax);
    rc = launch_rows_dynamic_bwd(a->w_raw, I, a->w_scale, a->dw, I, a->dw, I, N, I, a->q_w.qmin, a->q_w.qmax, stream);
    if (rc) return rc;
  }
  if (a->dbias) return colsum(a->dbias, a->dgi, a->sdgi, M, N, colp, stream, who);
  return GS_OK;
}

extern "C" int gs_quantize_rows(const gs_rows_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_quantize_rows";
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  if (a->rows < 1 || a->cols < 1 || a->rows > INT32_MAX || a->cols > (1 << 24))
    return set_error(GS_ERR_INVALID, "%s: rows and cols must be in [1, 2^31) and [1, 2^24]; got %lld, %lld", who,
                     (long long)a->rows, (long long)a->cols);
  if (!a->w || !a->scale || (!a->w_q && !a->codes))
    return set_error(GS_ERR_INVALID, "%s: w, scale and at least one of w_q and codes must be non-NULL", who);
  if (!(a->qmax > 0) || a->qmin > a->qmax)
    return set_error(GS_ERR_INVALID, "%s: needs qmax > 0 and qmin <= qmax; got [%d, %d]", who, a->qmin, a->qmax);
  if (a->codes && (a->qmin < -128 || a->qmax > 127))
    return set_error(GS_ERR_INVALID, "%s: int8 codes need qmin >= -128 and qmax <= 127; got [%d, %d]", who, a->qmin,
                     a->qmax);
  hipLaunchKernelGGL(weight_quant_rows, dim3((unsigned)a->rows), dim3(kRowThreads), 0, stream, a->w, (int)a->cols,
                     (float)a->qmin, (float)a->qmax, a->w_q, a->scale, a->codes);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

extern "C" int gs_weight_codes(const float* w, int64_t rows, int64_t cols, int8_t* codes, float* scale,
                               int32_t* exact, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_weight_codes";
  if (rows < 1 || cols < 1 || rows > INT32_MAX || cols > (1 << 24))
    return set_error(GS_ERR_INVALID, "%s: rows and cols must be in [1, 2^31) and [1, 2^24]; got %lld, %lld", who,
                     (long long)rows, (long long)cols);
  if (!w || !codes || !scale || !exact)
    return set_error(GS_ERR_INVALID, "%s: w, codes, scale and exact must be non-NULL", who);
  hipLaunchKernelGGL(recover_codes_rows, dim3((unsigned)rows), dim3(64), 0, stream, w, (int)cols, codes, scale, exact);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}
