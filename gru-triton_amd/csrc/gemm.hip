// fp32 GEMM on v_mfma_f32_16x16x4f32 (gfx950) for the products around the
// scans: the backward's recomputation of the hidden projection for all steps
// at once, gh = q_in([h0; out[0..T-2]]) Wh^T + bh (NT), and the weight
// gradient dWh = dgh^T q_in([h0; out[0..T-2]]) (TN) -- the per-step products
// of the reference backward (src/gru_qat/triton_kernels/scan.py:388-421 and
// :576-619), batched over every step because neither depends on the reverse
// recurrence.
//
// Tiling: a workgroup of 4 waves computes a 64 x 64 tile of C; wave (wy, wx)
// owns a 32 x 32 quarter as 2 x 2 MFMA tiles of 16 x 16. K advances in slices
// of 32, staged through LDS and double-buffered: the next slice's global
// loads are in flight while the current one feeds the MFMAs. Global loads are
// float4 along each operand's contiguous dimension when the shapes allow it
// (scalar otherwise), and land in LDS without transposition:
//   k-contiguous operand: S[row][k], row stride 40;
//   row-contiguous operand: S[k][row], row stride 68 (NN) or 80 (TN).
// A k-contiguous operand is read as float4s: lane (row r, k-group q) reads
// k = 4 q and 4 q + 16, and MFMA s takes k = 4 q + 16 (s / 4) + s % 4.
// gfx950 serves a 16-byte LDS read in 16-lane passes that pair 8-lane groups
// {0, 3}, {1, 2}, {4, 7}, {5, 6}, i.e. rows r < 8 of one k-group with rows
// r >= 8 of the next; with stride 40 (10 four-bank groups) every row starts on
// an even group and the two k-groups of a pass sit one group apart, so a pass
// covers all 64 banks (the earlier k = 8 q + s with stride 36 put two lanes of
// every pass on one bank). A row-contiguous operand is read as single words
// (32 banks, 32-lane passes covering k-groups q and q + 1): under the NN
// mapping those rows are 4 k apart, 4 x 68 = 16 mod 32 words; under TN's
// k = q + 4 s they are 1 k apart, 80 = 16 mod 32. Any bijection between (MFMA
// step, k-group) and k is valid as long as A and B use the same one.
//
// MFMA operand layout (16x16x4 f32): lane l supplies A[i = l % 16][k-group
// l / 16] and B[k-group l / 16][j = l % 16]; D VGPR v of lane l is
// C[4 (l / 16) + v][l % 16].
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, kGemmThreads = 256;
constexpr int kKStride = BK + 8;  // floats per LDS row of a k-contiguous operand (one row of the tile, 32 k)
// floats per LDS row of a row-contiguous operand (one k, 64 rows of the tile)
constexpr int kRStrideNN = 64 + 4, kRStrideTN = 64 + 16;
constexpr int kStageFloats = (BM * kKStride > BK * kRStrideTN) ? BM * kKStride : BK * kRStrideTN;

typedef float f4v __attribute__((ext_vector_type(4)));

// Loads of one operand tile (64 rows of the output dimension x 32 k) into
// registers, then into LDS. KC: the operand is contiguous along k.
template <bool KC, bool VEC, bool QUANT, int RS>
struct TileLoader {
  // VEC: 2 float4 per thread; scalar: 8 floats per thread.
  static constexpr int N = VEC ? 2 : 8;
  float r[VEC ? 8 : 8];
  const float* base;
  int64_t ld;
  int lim_row, lim_k;  // rows < lim_row, k < lim_k (absolute)
  int row0;
  Quant q;

  __device__ __forceinline__ void init(const float* p, int64_t ld_, int row0_, int lim_row_, int lim_k_) {
    base = p;
    ld = ld_;
    row0 = row0_;
    lim_row = lim_row_;
    lim_k = lim_k_;
  }
  __device__ __forceinline__ void load(int k0) {
    const int tid = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int idx = tid + kGemmThreads * e;
        int row, k;
        if constexpr (KC) {
          row = idx >> 3;
          k = (idx & 7) * 4;
        } else {
          k = idx >> 4;
          row = (idx & 15) * 4;
        }
        const int R = row0 + row, Kk = k0 + k;
        f4v v = f4v{0.f, 0.f, 0.f, 0.f};
        // Shapes are multiples of 4 along the contiguous dimension, so a
        // float4 is either wholly inside or wholly outside.
        if (R < lim_row && Kk < lim_k)
          v = *reinterpret_cast<const f4v*>(KC ? base + (int64_t)R * ld + Kk : base + (int64_t)Kk * ld + R);
        if constexpr (QUANT) {
          // zero padding stays zero: fake_quant(0) == 0
          v[0] = fake_quant(v[0], q);
          v[1] = fake_quant(v[1], q);
          v[2] = fake_quant(v[2], q);
          v[3] = fake_quant(v[3], q);
        }
        r[4 * e + 0] = v[0];
        r[4 * e + 1] = v[1];
        r[4 * e + 2] = v[2];
        r[4 * e + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = tid + kGemmThreads * e;
        int row, k;
        if constexpr (KC) {
          row = idx >> 5;
          k = idx & 31;
        } else {
          k = idx >> 6;
          row = idx & 63;
        }
        const int R = row0 + row, Kk = k0 + k;
        float v = (R < lim_row && Kk < lim_k) ? (KC ? base[(int64_t)R * ld + Kk] : base[(int64_t)Kk * ld + R]) : 0.0f;
        if constexpr (QUANT) v = fake_quant(v, q);
        r[e] = v;
      }
    }
  }
  __device__ __forceinline__ void stage(float* s) const {
    const int tid = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int idx = tid + kGemmThreads * e;
        float* d;
        if constexpr (KC)
          d = s + (idx >> 3) * kKStride + (idx & 7) * 4;
        else
          d = s + (idx >> 4) * RS + (idx & 15) * 4;
        *reinterpret_cast<f4v*>(d) = f4v{r[4 * e], r[4 * e + 1], r[4 * e + 2], r[4 * e + 3]};
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = tid + kGemmThreads * e;
        if constexpr (KC)
          s[(idx >> 5) * kKStride + (idx & 31)] = r[e];
        else
          s[(idx >> 6) * RS + (idx & 63)] = r[e];
      }
    }
  }
};

template <int LAYOUT, bool VEC, bool QA, bool QB>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs g) {
  constexpr bool A_KC = LAYOUT != kGemmTN, B_KC = LAYOUT == kGemmNT;
  constexpr bool VEC_A = VEC, VEC_B = VEC;
  __shared__ __attribute__((aligned(16))) float As[2][kStageFloats];
  __shared__ __attribute__((aligned(16))) float Bs[2][kStageFloats];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wy = wave >> 1, wx = wave & 1;
  const int i0 = blockIdx.x * BM, j0 = blockIdx.y * BN;
  const int kper = ((g.K + g.ksplit - 1) / g.ksplit + BK - 1) / BK * BK;
  const int z = blockIdx.z / g.ksplit, split = blockIdx.z - z * g.ksplit;
  const int kbeg = split * kper;
  const int kend = min(g.K, kbeg + kper);

  constexpr int RS = LAYOUT == kGemmNN ? kRStrideNN : kRStrideTN;
  TileLoader<A_KC, VEC_A, QA, RS> la;
  TileLoader<B_KC, VEC_B, QB, RS> lb;
  la.init(g.a + (int64_t)(z % g.a_mod) * g.a_bs, g.lda, i0, g.M, kend);
  lb.init(g.b + (int64_t)(z % g.b_mod) * g.b_bs, g.ldb, j0, g.N, kend);
  la.q = g.qa;
  lb.q = g.qb;

  f4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, kq = lane >> 4;
  int buf = 0;
  if (kbeg < kend) {
    la.load(kbeg);
    lb.load(kbeg);
    la.stage(As[0]);
    lb.stage(Bs[0]);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) {
      la.load(k0 + BK);
      lb.load(k0 + BK);
    }
    const float* as = As[buf];
    const float* bs = Bs[buf];
    if constexpr (A_KC && B_KC) {
      // lane: rows 32 wy + 16 ti + r16 (A) and 32 wx + 16 tj + r16 (B), k = 4 kq + 16 h + e
      f4v a[2][2], b[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          a[t][h] = *reinterpret_cast<const f4v*>(as + (32 * wy + 16 * t + r16) * kKStride + 4 * kq + 16 * h);
          b[t][h] = *reinterpret_cast<const f4v*>(bs + (32 * wx + 16 * t + r16) * kKStride + 4 * kq + 16 * h);
        }
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
            acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ti][s >> 2][s & 3], b[tj][s >> 2][s & 3],
                                                               acc[ti][tj], 0, 0, 0);
    } else if constexpr (A_KC) {
      // NN: A as float4s (as NT), B single words of row k = 4 kq + 16 (s / 4) + s % 4
      f4v a[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          a[t][h] = *reinterpret_cast<const f4v*>(as + (32 * wy + 16 * t + r16) * kKStride + 4 * kq + 16 * h);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float* br = bs + (4 * kq + 16 * (s >> 2) + (s & 3)) * RS + 32 * wx + r16;
        const float b0 = br[0], b1 = br[16];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
          acc[ti][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ti][s >> 2][s & 3], b0, acc[ti][0], 0, 0, 0);
          acc[ti][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ti][s >> 2][s & 3], b1, acc[ti][1], 0, 0, 0);
        }
      }
    } else {
      // TN: k = kq + 4 s
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float* ar = as + (kq + 4 * s) * RS + 32 * wy + r16;
        const float a0 = ar[0], a1 = ar[16];
        const float* br = bs + (kq + 4 * s) * RS + 32 * wx + r16;
        const float b0 = br[0], b1 = br[16];
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
      }
    }
    if (more) {
      la.stage(As[buf ^ 1]);
      lb.stage(Bs[buf ^ 1]);
    }
    __syncthreads();
    buf ^= 1;
  }

  float* c = g.c + (int64_t)z * g.c_bs + (int64_t)split * g.split_stride;
  const float* biasp = g.bias ? g.bias + (int64_t)z * g.bias_bs : nullptr;
  const bool add_bias = biasp != nullptr && split == 0;
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
      const int j = j0 + 32 * wx + 16 * tj + r16;
      if (j >= g.N) continue;
      const float bias = add_bias ? biasp[j] : 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 32 * wy + 16 * ti + 4 * kq + v;
        if (i < g.M) c[(int64_t)i * g.ldc + j] = acc[ti][tj][v] + bias;
      }
    }
}

// ---- int8 NT product (gemm_i8_nt) -----------------------------------------------
// A 64 x 64 tile of C per workgroup of 4 waves, each wave 2 x 2 tiles of
// v_mfma_i32_16x16x64_i8; K advances by 64, double-buffered through LDS. Each
// thread loads 16 consecutive k (16 bytes) of one row of each operand and
// stores them with one 16-byte LDS write; a row holds 64 bytes in a stride of
// 20 words, so the 16 rows that a 16-lane pass of the operand reads start on
// distinct 4-bank groups (20 r mod 64) and the 16-byte reads are free of
// conflicts. MFMA operand layout: lane l supplies the 16 bytes of row l % 16
// at k-group l / 16 for A and for B alike, so whatever k the hardware assigns
// a byte, A's and B's bytes at one position are the same k; D VGPR v of lane
// l is C[4 (l / 16) + v][l % 16].
constexpr int kI8Tile = 64, kI8BK = 64, kI8RowWords = 20;
typedef int i4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kGemmThreads) void gemm_i8_nt_kernel(GemmI8Args g) {
  __shared__ __attribute__((aligned(16))) int As[2][kI8Tile * kI8RowWords];
  __shared__ __attribute__((aligned(16))) int Bs[2][kI8Tile * kI8RowWords];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wy = wave >> 1, wx = wave & 1;
  const int i0 = blockIdx.x * kI8Tile, j0 = blockIdx.y * kI8Tile;
  // loader: row lr of the tile, k = 16 lk .. 16 lk + 15 of the slice
  const int lr = threadIdx.x >> 2, lk = threadIdx.x & 3;
  const int ra = i0 + lr, rb = j0 + lr;
  const bool oka = ra < g.M, okb = rb < g.N;
  const int8_t* pa = g.a + (int64_t)(oka ? ra : 0) * g.lda + 16 * lk;
  const int8_t* pb = g.b + (int64_t)(okb ? rb : 0) * g.ldb + 16 * lk;
  i4v va, vb;
  auto load = [&](int k0) {
    const bool in = k0 + 16 * lk < g.K;  // K % 16 == 0: 16 bytes wholly inside or outside
    va = (oka && in) ? *reinterpret_cast<const i4v*>(pa + k0) : i4v{0, 0, 0, 0};
    vb = (okb && in) ? *reinterpret_cast<const i4v*>(pb + k0) : i4v{0, 0, 0, 0};
  };
  auto stage = [&](int buf) {
    *reinterpret_cast<i4v*>(&As[buf][lr * kI8RowWords + 4 * lk]) = va;
    *reinterpret_cast<i4v*>(&Bs[buf][lr * kI8RowWords + 4 * lk]) = vb;
  };
  i4v acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = i4v{0, 0, 0, 0};
  const int r16 = lane & 15, kg = lane >> 4;
  int buf = 0;
  load(0);
  stage(0);
  __syncthreads();
  for (int k0 = 0; k0 < g.K; k0 += kI8BK) {
    const bool more = k0 + kI8BK < g.K;
    if (more) load(k0 + kI8BK);
    i4v a[2], b[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      a[t] = *reinterpret_cast<const i4v*>(&As[buf][(32 * wy + 16 * t + r16) * kI8RowWords + 4 * kg]);
      b[t] = *reinterpret_cast<const i4v*>(&Bs[buf][(32 * wx + 16 * t + r16) * kI8RowWords + 4 * kg]);
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj) acc[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[ti], b[tj], acc[ti][tj], 0, 0, 0);
    if (more) stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int tj = 0; tj < 2; ++tj) {
    const int j = j0 + 32 * wx + 16 * tj + r16;
    if (j >= g.N) continue;
    const float sc = g.sa * g.b_scale[j];
    const float bias = g.bias ? g.bias[j] : 0.0f;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 32 * wy + 16 * ti + 4 * kg + v;
        if (i < g.M) g.c[(int64_t)i * g.ldc + j] = (float)acc[ti][tj][v] * sc + bias;
      }
  }
}

__global__ void quant_codes_kernel(float* dst_q, int8_t* codes, const float* src, int64_t ld, int rows, int cols,
                                   Quant q) {
  const int64_t n = (int64_t)rows * cols;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / cols;
    const int i = (int)(e - m * cols);
    const float lv = quant_level(src[m * ld + i], q);
    if (dst_q != nullptr) dst_q[e] = lv * q.scale;
    codes[e] = (int8_t)(int)lv;
  }
}

__global__ void sum_partials_kernel(float* dst, const float* src, int64_t n, int parts, int64_t stride) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    float s = src[e];
    for (int p = 1; p < parts; ++p) s += src[p * stride + e];
    dst[e] = s;
  }
}

// Two independent sums of partials in one launch: element e < a.n of job a,
// then the elements of job b.
__global__ void sum_partials2_kernel(SumJob a, SumJob b) {
  const int64_t n = a.n + b.n;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const bool first = e < a.n;
    const SumJob& j = first ? a : b;
    const int64_t i = first ? e : e - a.n;
    float s = j.src[i];
    for (int p = 1; p < j.parts; ++p) s += j.src[p * j.stride + i];
    j.dst[i] = s;
  }
}

// Column sums: a workgroup takes 64 columns x kColRows rows; its 256 threads
// are 64 columns x 4 row lanes, each lane summing every 4th row (8 loads in
// flight), and the 4 lanes are combined through LDS into partial[chunk][j].
constexpr int kColRows = 256;
__global__ __launch_bounds__(256) void colsum_kernel(const float* src, int64_t ld, int rows, int cols,
                                                     float* partial) {
  __shared__ float red[4][64];
  const int jl = threadIdx.x & 63, lane_r = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + jl;
  const int r0 = blockIdx.y * kColRows;
  const int r1 = min(rows, r0 + kColRows);
  float s = 0.0f;
  if (j < cols) {
    int r = r0 + lane_r;
    for (; r + 28 < r1; r += 32) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[(int64_t)(r + 4 * u) * ld + j];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; r < r1; r += 4) s += src[(int64_t)r * ld + j];
  }
  red[lane_r][jl] = s;
  __syncthreads();
  if (lane_r == 0 && j < cols)
    partial[(int64_t)blockIdx.y * cols + j] = ((red[0][jl] + red[1][jl]) + red[2][jl]) + red[3][jl];
}

__global__ void quant_copy_kernel(float* dst, const float* src, int64_t ld, int rows, int cols, Quant q) {
  const int64_t n = (int64_t)rows * cols;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / cols;
    const int i = (int)(e - m * cols);
    dst[e] = fake_quant(src[m * ld + i], q);
  }
}

__global__ void prev_state_kernel(float* hq, const float* h0, int64_t sh0_b, const float* out, int64_t so_b,
                                  int64_t rows, int B, int H, Quant q) {
  const int64_t n = rows * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / H;
    const int k = (int)(e - m * H);
    float v = m < B ? h0[m * sh0_b + k] : out[(m - B) * so_b + k];
    if (q.on) v = fake_quant(v, q);
    hq[e] = v;
  }
}

typedef void (*GemmFn)(GemmArgs);

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// K split of a product: at least two workgroups per CU of the MI355X (256
// CUs) where K allows it (at least 256 terms per split, at most 16 splits),
// and among those splits the one whose last round of workgroups fills the
// CUs best (smallest on ties). The dense backward's dWh at T=64, B=32,
// H=512 (192 tiles) then splits K in 4 (768 workgroups, 3 per CU) rather
// than 3 (576, a last round a quarter full): 51.5 -> 42.1 us.
int gemm_pick_split(int M, int N, int K) {
  constexpr int kCUs = 256;
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int smax = std::max(1, std::min(16, (K + 255) / 256));
  int best = 1;
  int64_t best_num = -1, best_den = 1;  // fill fraction best_num / best_den
  for (int s = 1; s <= smax; ++s) {
    const int64_t n = (int64_t)tiles * s;
    if (n < 2 * kCUs && s < smax) continue;
    const int64_t den = (int64_t)kCUs * ((n + kCUs - 1) / kCUs);
    if (n * best_den > best_num * den) {
      best = s;
      best_num = n;
      best_den = den;
    }
  }
  return best;
}

int gemm_f32(const GemmArgs& g, hipStream_t stream, const char* who) {
  if (g.M < 1 || g.N < 1 || g.K < 1 || g.ksplit < 1)
    return set_error(GS_ERR_INVALID, "%s: GEMM dims must be positive (M=%d, N=%d, K=%d, ksplit=%d)", who, g.M, g.N,
                     g.K, g.ksplit);
  if (g.batch < 1 || g.a_mod < 1 || g.b_mod < 1 || (int64_t)g.batch * g.ksplit > 65535)
    return set_error(GS_ERR_INVALID, "%s: bad GEMM batch (batch=%d, a_mod=%d, b_mod=%d, ksplit=%d)", who, g.batch,
                     g.a_mod, g.b_mod, g.ksplit);
  if (g.layout != kGemmNT && g.layout != kGemmTN && g.layout != kGemmNN)
    return set_error(GS_ERR_INVALID, "%s: unknown GEMM layout %d", who, g.layout);
  // float4 loads need 16-byte aligned bases, leading dimensions that keep
  // rows aligned, and contiguous extents that are multiples of 4.
  const bool a_kc = g.layout != kGemmTN, b_kc = g.layout == kGemmNT;
  const bool vec = aligned16(g.a) && aligned16(g.b) && g.lda % 4 == 0 && g.ldb % 4 == 0 && g.a_bs % 4 == 0 &&
                   g.b_bs % 4 == 0 &&
                   (a_kc ? g.K % 4 == 0 : g.M % 4 == 0) && (b_kc ? g.K % 4 == 0 : g.N % 4 == 0);
#define GS_GEMM_ROW(L, V) \
  {{gemm_kernel<L, V, false, false>, gemm_kernel<L, V, false, true>}, \
   {gemm_kernel<L, V, true, false>, gemm_kernel<L, V, true, true>}}
  static const GemmFn table[3][2][2][2] = {
      {GS_GEMM_ROW(kGemmNT, false), GS_GEMM_ROW(kGemmNT, true)},
      {GS_GEMM_ROW(kGemmTN, false), GS_GEMM_ROW(kGemmTN, true)},
      {GS_GEMM_ROW(kGemmNN, false), GS_GEMM_ROW(kGemmNN, true)},
  };
#undef GS_GEMM_ROW
  GemmFn fn = table[g.layout][vec ? 1 : 0][g.qa.on ? 1 : 0][g.qb.on ? 1 : 0];
  const dim3 grid((unsigned)((g.M + BM - 1) / BM), (unsigned)((g.N + BN - 1) / BN),
                  (unsigned)(g.batch * g.ksplit));
  hipLaunchKernelGGL(fn, grid, dim3(kGemmThreads), 0, stream, g);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

bool gemm_i8_applies(const GemmI8Args& g) {
  return g.K >= 1 && g.K <= 65536 && g.K % 16 == 0 && g.lda % 16 == 0 && g.ldb % 16 == 0 && aligned16(g.a) &&
         aligned16(g.b) && g.b_scale != nullptr;
}

int gemm_i8_nt(const GemmI8Args& g, hipStream_t stream, const char* who) {
  if (g.M < 1 || g.N < 1 || !gemm_i8_applies(g))
    return set_error(GS_ERR_INVALID, "%s: int8 GEMM operands out of its contract (M=%d, N=%d, K=%d)", who, g.M, g.N,
                     g.K);
  const dim3 grid((unsigned)((g.M + kI8Tile - 1) / kI8Tile), (unsigned)((g.N + kI8Tile - 1) / kI8Tile));
  hipLaunchKernelGGL(gemm_i8_nt_kernel, grid, dim3(kGemmThreads), 0, stream, g);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int quant_copy_codes(float* dst_q, int8_t* codes, const float* src, int64_t ld, int rows, int cols, const Quant& q,
                     hipStream_t stream, const char* who) {
  (void)who;
  const int64_t n = (int64_t)rows * cols;
  hipLaunchKernelGGL(quant_codes_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256), 0,
                     stream, dst_q, codes, src, ld, rows, cols, q);
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

int sum_partials2(const SumJob& a, const SumJob& b, hipStream_t stream, const char* who) {
  (void)who;
  const int64_t blocks = (a.n + b.n + 255) / 256;
  if (blocks == 0) return GS_OK;
  hipLaunchKernelGGL(sum_partials2_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, stream, a,
                     b);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int64_t colsum_partial_floats(int rows, int cols) { return (int64_t)((rows + kColRows - 1) / kColRows) * cols; }

int colsum(float* dst, const float* src, int64_t ld, int rows, int cols, float* partials, hipStream_t stream,
           const char* who) {
  const int chunks = (rows + kColRows - 1) / kColRows;
  hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)((cols + 63) / 64), (unsigned)chunks), dim3(256), 0, stream, src,
                     ld, rows, cols, partials);
  GS_CHECK_HIP(hipGetLastError());
  return sum_partials(dst, partials, cols, chunks, cols, stream, who);
}

int quant_copy(float* dst, const float* src, int64_t ld, int rows, int cols, const Quant& q, hipStream_t stream,
               const char* who) {
  (void)who;
  const int64_t n = (int64_t)rows * cols;
  hipLaunchKernelGGL(quant_copy_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256), 0, stream,
                     dst, src, ld, rows, cols, q);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int build_prev_state(float* hq, const float* h0, int64_t sh0_b, const float* out, int64_t so_b, int T, int B, int H,
                     const Quant& q, hipStream_t stream, const char* who) {
  (void)who;
  const int64_t n = (int64_t)T * B * H;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(prev_state_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream, hq, h0,
                     sh0_b, out, so_b, (int64_t)T * B, B, H, q);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace gs
