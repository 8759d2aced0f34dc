// fp32 GEMM on v_mfma_f32_16x16x4f32 (gfx950) for the products around the
// scans: the backward's recomputation of the hidden projection for all steps
// at once, gh = q_in([h0; out[0..T-2]]) Wh^T + bh, and the weight gradient
// dWh = dgh^T q_in([h0; out[0..T-2]]) (the per-step products of the
// reference backward, src/gru_qat/triton_kernels/scan.py:388-421 and
// :576-619, batched over every step because neither depends on the reverse
// recurrence).
//
// Tiling: a workgroup of 4 waves computes a 64 x 64 tile of C; wave (wy, wx)
// owns the 32 x 32 quarter as 2 x 2 MFMA tiles of 16 x 16. K advances in
// slices of 32 staged through LDS as [k][i] and [k][j] (a column of 16
// consecutive i or j per MFMA operand read, conflict-free), double-buffered:
// the next slice's global loads are in flight while the current one feeds
// the MFMAs. Global loads run along each operand's unit-stride dimension.
//
// MFMA operand layout (16x16x4 f32): lane l supplies A[i = l % 16][k = l / 16]
// and B[k = l / 16][j = l % 16]; D VGPR v of lane l is C[4 (l / 16) + v][l % 16].
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, kGemmThreads = 256, kPad = 1;
constexpr int kPerThread = BM * BK / kGemmThreads;  // elements of each operand per thread per slice
static_assert(BM * BK == BK * BN, "both operands stage the same element count");

// Element (r, c) of an operand whose column stride is 1 (CUNIT) or whose row
// stride is 1 (!CUNIT).
template <bool CUNIT>
__device__ __forceinline__ float operand_at(const GemmOperand& o, int r, int c) {
  const float* src;
  if (r < o.rows0)
    src = o.p0 + (int64_t)r * o.s0r;
  else
    src = o.p + (CUNIT ? (int64_t)(r - o.rows0) * o.sr : (int64_t)(r - o.rows0));
  float v = src[CUNIT ? (int64_t)c : (int64_t)c * o.sc];
  if (o.q.on) v = fake_quant(v, o.q);
  return v;
}

// A_KFAST: A's column (k) stride is 1, else its row (i) stride is 1.
// B_NFAST: B's column (j) stride is 1, else its row (k) stride is 1.
template <bool A_KFAST, bool B_NFAST>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs g) {
  __shared__ float As[2][BK][BM + kPad];
  __shared__ float Bs[2][BK][BN + kPad];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wy = wave >> 1, wx = wave & 1;
  const int i0 = blockIdx.x * BM, j0 = blockIdx.y * BN;
  const int kper = ((g.K + g.ksplit - 1) / g.ksplit + BK - 1) / BK * BK;
  const int kbeg = blockIdx.z * kper;
  const int kend = min(g.K, kbeg + kper);

  float ra[kPerThread], rb[kPerThread];
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int idx = tid + kGemmThreads * e;
      const int ai = A_KFAST ? idx / BK : idx % BM, ak = A_KFAST ? idx % BK : idx / BM;
      const int i = i0 + ai, k = k0 + ak;
      ra[e] = (i < g.M && k < kend) ? operand_at<A_KFAST>(g.a, i, k) : 0.0f;
      const int bj = B_NFAST ? idx % BN : idx / BK, bk = B_NFAST ? idx / BN : idx % BK;
      const int j = j0 + bj, kb = k0 + bk;
      rb[e] = (j < g.N && kb < kend) ? operand_at<B_NFAST>(g.b, kb, j) : 0.0f;
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int idx = tid + kGemmThreads * e;
      const int ai = A_KFAST ? idx / BK : idx % BM, ak = A_KFAST ? idx % BK : idx / BM;
      As[buf][ak][ai] = ra[e];
      const int bj = B_NFAST ? idx % BN : idx / BK, bk = B_NFAST ? idx / BN : idx % BK;
      Bs[buf][bk][bj] = rb[e];
    }
  };

  f4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, kq = lane >> 4;
  int buf = 0;
  if (kbeg < kend) {
    load(kbeg);
    stage(0);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load(k0 + BK);
#pragma unroll
    for (int k4 = 0; k4 < BK; k4 += 4) {
      const float* ar = &As[buf][k4 + kq][32 * wy + r16];
      const float* br = &Bs[buf][k4 + kq][32 * wx + r16];
      const float a0 = ar[0], a1 = ar[16], b0 = br[0], b1 = br[16];
      acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  float* c = g.c + (int64_t)blockIdx.z * g.split_stride;
  const bool add_bias = g.bias != nullptr && blockIdx.z == 0;
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
      const int j = j0 + 32 * wx + 16 * tj + r16;
      if (j >= g.N) continue;
      const float bias = add_bias ? g.bias[j] : 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 32 * wy + 16 * ti + 4 * kq + v;
        if (i < g.M) c[(int64_t)i * g.ldc + j] = acc[ti][tj][v] + bias;
      }
    }
}

__global__ void sum_partials_kernel(float* dst, const float* src, int64_t n, int parts, int64_t stride) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    float s = src[e];
    for (int p = 1; p < parts; ++p) s += src[p * stride + e];
    dst[e] = s;
  }
}

typedef void (*GemmFn)(GemmArgs);

}  // namespace

int gemm_pick_split(int M, int N, int K) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int s = (512 + tiles - 1) / tiles;       // about two workgroups per CU
  const int smax = (K + 255) / 256;        // at least 256 terms per split
  if (s > smax) s = smax;
  return s < 1 ? 1 : s;
}

int gemm_f32(const GemmArgs& g, hipStream_t stream, const char* who) {
  if (g.M < 1 || g.N < 1 || g.K < 1 || g.ksplit < 1)
    return set_error(GS_ERR_INVALID, "%s: GEMM dims must be positive (M=%d, N=%d, K=%d, ksplit=%d)", who, g.M, g.N,
                     g.K, g.ksplit);
  const bool a_kfast = g.a.sc == 1, b_nfast = g.b.sc == 1;
  if ((!a_kfast && g.a.sr != 1) || (!b_nfast && g.b.sr != 1))
    return set_error(GS_ERR_INVALID, "%s: GEMM operands need a unit stride", who);
  GemmFn fn = a_kfast ? (b_nfast ? gemm_kernel<true, true> : gemm_kernel<true, false>)
                      : (b_nfast ? gemm_kernel<false, true> : gemm_kernel<false, false>);
  const dim3 grid((unsigned)((g.M + BM - 1) / BM), (unsigned)((g.N + BN - 1) / BN), (unsigned)g.ksplit);
  hipLaunchKernelGGL(fn, grid, dim3(kGemmThreads), 0, stream, g);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int sum_partials(float* dst, const float* src, int64_t n, int parts, int64_t stride, hipStream_t stream,
                 const char* who) {
  (void)who;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, stream, dst,
                     src, n, parts, stride);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace gs
