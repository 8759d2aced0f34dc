// fp32 GEMM on MFMA for the plain matrix products around the scans:
//   C[i, j] = sum_k A(i, k) B(k, j) (+ bias[j])
// Operands are strided 2-D views, optionally fake-quantized on load, and the
// rows of one operand may come from two tensors (the h0 rows followed by the
// out rows of the previous-state matrix [h0; out[0..T-2]]).
#pragma once

#include "gs_host.h"

namespace gs {

// Element (r, c) is p[r * sr + c * sc], or p0[r * s0r + c * sc] for r < rows0;
// with q.on, fake_quant(., q) is applied to every element loaded.
struct GemmOperand {
  const float* p;
  int64_t sr, sc;
  const float* p0;
  int64_t s0r;
  int rows0;
  Quant q;
};

struct GemmArgs {
  GemmOperand a;  // rows i < M, columns k < K
  GemmOperand b;  // rows k < K, columns j < N
  float* c;       // C[i * ldc + j]; split s of a K-split product writes c + s * split_stride
  int64_t ldc;
  int64_t split_stride;
  const float* bias;  // [N] added once (by split 0), or null
  int M, N, K, ksplit;
};

inline GemmOperand plain_operand(const float* p, int64_t sr, int64_t sc) {
  return GemmOperand{p, sr, sc, nullptr, 0, 0, Quant{1.0f, 0.0f, 0.0f, 0}};
}

// Launches the product on `stream`. Every element of C (of every split) is
// written. Requires one of each operand's strides to be 1.
int gemm_f32(const GemmArgs& g, hipStream_t stream, const char* who);

// dst[e] = sum_{s < parts} src[s * stride + e] for e < n.
int sum_partials(float* dst, const float* src, int64_t n, int parts, int64_t stride, hipStream_t stream,
                 const char* who);

// Number of K splits that fills the device for an M x N output with K terms.
int gemm_pick_split(int M, int N, int K);

}  // namespace gs
