// fp32 GEMM on MFMA for the plain matrix products around the scans:
//   C[i, j] = sum_k qa(A(i, k)) qb(B(k, j)) (+ bias[j])
// in three layouts: NT, both operands contiguous along k
// (A(i, k) = a[i lda + k], B(k, j) = b[j ldb + k]); TN, both contiguous
// along their output dimension (A(i, k) = a[k lda + i], B(k, j) = b[k ldb + j]);
// NN, A along k and B along j (A(i, k) = a[i lda + k], B(k, j) = b[k ldb + j]).
// qa and qb are optional per-tensor fake-quants applied to A and B as they are
// loaded.
#pragma once

#include "gs_host.h"

namespace gs {

enum GemmLayout : int { kGemmNT = 0, kGemmTN = 1, kGemmNN = 2 };

struct GemmArgs {
  const float* a = nullptr;
  int64_t lda = 0;
  const float* b = nullptr;
  int64_t ldb = 0;
  float* c = nullptr;  // C[i * ldc + j]; split s of a K-split product writes c + s * split_stride
  int64_t ldc = 0;
  int64_t split_stride = 0;
  const float* bias = nullptr;  // [N] added once (by split 0), or null
  int M = 0, N = 0, K = 0, ksplit = 1;
  int layout = kGemmNT;                 // GemmLayout
  Quant qa{1.0f, 0.0f, 0.0f, 0, 1.0f};   // applied to A on load when qa.on
  Quant qb{1.0f, 0.0f, 0.0f, 0, 1.0f};   // applied to B on load when qb.on
  // Batched products: product z < batch uses a + (z % a_mod) a_bs,
  // b + (z % b_mod) b_bs, c + z c_bs and bias + z bias_bs (splits of
  // product z still step by split_stride from there).
  int batch = 1, a_mod = 1, b_mod = 1;
  int64_t a_bs = 0, b_bs = 0, c_bs = 0, bias_bs = 0;
};

// Launches the product on `stream`. Every element of C (of every split) is written.
int gemm_f32(const GemmArgs& g, hipStream_t stream, const char* who);

// NT product of int8 operands on the int8 MFMA:
//   C[i, j] = float(sum_k a[i lda + k] b[j ldb + k]) * (sa * b_scale[j]) (+ bias[j])
// with a the levels of a per-tensor fake-quant of scale sa and b per-row codes
// of scale b_scale[j] (int8, rows 16-byte aligned: K, lda and ldb multiples of
// 16). The integer sums are exact (K <= 65536: no int32 overflow), so C is
// within an fp32 rounding of each product of gemm_f32 on the fake-quantized
// operands.
struct GemmI8Args {
  const int8_t* a = nullptr;
  int64_t lda = 0;
  float sa = 1.0f;
  const int8_t* b = nullptr;
  int64_t ldb = 0;
  const float* b_scale = nullptr;
  const float* bias = nullptr;
  float* c = nullptr;
  int64_t ldc = 0;
  int M = 0, N = 0, K = 0;
};
bool gemm_i8_applies(const GemmI8Args& g);
int gemm_i8_nt(const GemmI8Args& g, hipStream_t stream, const char* who);

// dst_q[m][i] = fake_quant(src[m ld + i], q) (dst_q contiguous [rows, cols], or
// NULL) and codes[m][i] its level (int8, contiguous), for q's range in a byte.
int quant_copy_codes(float* dst_q, int8_t* codes, const float* src, int64_t ld, int rows, int cols, const Quant& q,
                     hipStream_t stream, const char* who);

// dst[e] = sum_{s < parts} src[s * stride + e] for e < n.
int sum_partials(float* dst, const float* src, int64_t n, int parts, int64_t stride, hipStream_t stream,
                 const char* who);

// One sum_partials job; sum_partials2 runs two of them in one launch (the
// jobs' destinations must not overlap each other's sources).
struct SumJob {
  float* dst;
  const float* src;
  int64_t n;
  int parts;
  int64_t stride;
};
int sum_partials2(const SumJob& a, const SumJob& b, hipStream_t stream, const char* who);

// dst[j] = sum_{i < rows} src[i * ld + j] for j < cols; `partials` holds
// colsum_partial_floats(rows, cols) floats of scratch.
int64_t colsum_partial_floats(int rows, int cols);
int colsum(float* dst, const float* src, int64_t ld, int rows, int cols, float* partials, hipStream_t stream,
           const char* who);

// Number of K splits that fills the device for an M x N output with K terms.
int gemm_pick_split(int M, int N, int K);

// dst[m][i] = fake_quant(src[m ld + i], q), dst contiguous [rows, cols].
int quant_copy(float* dst, const float* src, int64_t ld, int rows, int cols, const Quant& q, hipStream_t stream,
               const char* who);

// hq[m][k] = q(m < B ? h0[m sh0_b + k] : out[(m - B) so_b + k]) for m < T B,
// k < H: the previous-state matrix [h0; out[0..T-2]] (fake-quantized when
// q.on) as a contiguous [T B, H] block.
int build_prev_state(float* hq, const float* h0, int64_t sh0_b, const float* out, int64_t so_b, int T, int B, int H,
                     const Quant& q, hipStream_t stream, const char* who);

// Backward of a per-row dynamic symmetric fake-quant (scale = max(max |row|,
// 1e-8) / qmax) on rows x cols, with the scale's own gradient path, as
// torch's autograd gives it for a scale computed from the tensor: d = g plus
// the scale terms on each row's max and min elements (struct_proj.hip).
// y and g/d have row strides ldy and ldg/ldd, s[row] the row scales; d may alias g.
int launch_rows_dynamic_bwd(const float* y, int64_t ldy, const float* s, const float* g, int64_t ldg, float* d,
                            int64_t ldd, int rows, int cols, int qmin, int qmax, hipStream_t stream);

}  // namespace gs
