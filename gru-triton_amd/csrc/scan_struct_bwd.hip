// Monarch and butterfly GRU scan backward (gfx950) through the dense backward.
//
// References: the Monarch backward (LarocheC/gru-triton
// src/gru_qat/triton_kernels/scan_monarch.py:409-884, PyTorch form :955-1053)
// and the butterfly backward (scan_butterfly.py:462-1075). Both hidden maps
// are linear in q_in(h): gh_g = M_g q_in(h) + bh_g with an H x H matrix M_g
// fixed by the parameters. The backward of the scan only needs M_g (to carry
// the gradient through the map) and the map's dense gradient
// dM_g = sum_t dgh_g,t^T q_in(h_{t-1}); both are what the dense backward
// (scan_dense_bwd.hip) computes for a [3H, H] weight. So each entry point
//   1. materializes M = [M_r; M_z; M_n] into the scratch,
//   2. runs the dense backward core with it (dgi, dh0, dbh, dM), and
//   3. carries dM onto the structured parameters:
//      Monarch single factor   dW[g][n] = the n-th diagonal block of dM_g;
//      Monarch two factors     M_g = P^T BL_g P BR_g (BR, BL block-diagonal
//                              from w and w2, (P z)[c nb + a] = z[a bs + c]):
//                              dBL = P dM BR^T P^T and dBR = P^T BL^T P dM,
//                              each kept on its diagonal blocks;
//      butterfly               M_g = S_K ... S_1 (one sparse stage per
//                              twiddle layer, rows and columns cut to H):
//                              with A_j = S_j ... S_1 [I; 0] and
//                              G_j = S_{j+1}^T ... S_K^T [dM_g; 0], the
//                              twiddles of stage j get the row-wise dot
//                              products of G_j with A_{j-1} (own row for the
//                              diagonal twiddle, partner row for the other).
// Every projected entry is a sum over H (or over a block) computed by one
// thread or one workgroup, so results are deterministic.
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {

int64_t dense_bwd_core_bytes(const gs_bwd_args* a, const char* who, bool tiled = false);
int64_t dense_bwd_core_scratch(const gs_bwd_args* a, const char* who, bool tiled = false);
int dense_bwd_core(const gs_bwd_args* a, const float* w, float* dw, hipStream_t stream, const char* who,
                   bool tiled = false);

namespace {

dim3 grid_for(int64_t n) { return dim3((unsigned)std::min<int64_t>((n + 255) / 256, 16384)); }

// ---- Monarch -----------------------------------------------------------------------

// Single factor: M[g H + x][k] = W[g][x / bs][x % bs][k % bs] inside the
// diagonal blocks, 0 elsewhere.
__global__ void monarch1_materialize(const float* w, float* m, int H, int nb, int bs) {
  const int64_t n = (int64_t)3 * H * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(e / H), k = (int)(e - (int64_t)row * H);
    const int g = row / H, x = row - g * H;
    m[e] = (x / bs == k / bs) ? w[(((int64_t)g * nb + x / bs) * bs + x % bs) * bs + k % bs] : 0.0f;
  }
}

__global__ void monarch1_project(const float* dm, float* dw, int H, int nb, int bs) {
  const int64_t n = (int64_t)3 * H * bs;  // = 3 nb bs bs
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(e % bs);
    const int64_t r = e / bs;  // (g nb + blk) bs + o
    const int o = (int)(r % bs);
    const int64_t gb = r / bs;
    const int blk = (int)(gb % nb), g = (int)(gb / nb);
    dw[e] = dm[((int64_t)g * H + blk * bs + o) * H + blk * bs + i];
  }
}

// Two factors: with perm[q] = (q % nb) bs + q / nb and inv its inverse,
// M_g[perm[j]][k] = sum over q in j's block with q % nb == k / bs of
// L[g][j / bs][j % bs][q % bs] R[g][k / bs][q / nb][k % bs].
__device__ __forceinline__ int m2_perm(int q, int nb, int bs) { return (q % nb) * bs + q / nb; }
__device__ __forceinline__ int m2_inv(int x, int nb, int bs) { return (x % bs) * nb + x / bs; }

__global__ void monarch2_materialize(const float* R, const float* L, float* m, int H, int nb, int bs) {
  const int64_t n = (int64_t)3 * H * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(e / H), k = (int)(e - (int64_t)row * H);
    const int g = row / H, x = row - g * H;
    const int j = m2_inv(x, nb, bs), jb = j / bs, kb = k / bs;
    const float* Lr = L + (((int64_t)g * nb + jb) * bs + j % bs) * bs;
    const float* Rb = R + ((int64_t)g * nb + kb) * bs * bs + k % bs;
    float acc = 0.0f;
    for (int i = 0; i < bs; ++i) {
      const int q = jb * bs + i;
      if (q % nb == kb) acc += Lr[i] * Rb[(int64_t)(q / nb) * bs];
    }
    m[e] = acc;
  }
}

// dL[g][n][o][i] = sum_{k' < bs} dM_g[perm[n bs + o]][mb bs + k'] R[g][mb][m % bs][k'],
//   m = perm[n bs + i], mb = m / bs;
// dR[g][n][o][i] = sum_{q' in q's block} L[g][q / bs][q' % bs][q % bs] dM_g[perm[q']][n bs + i],
//   q = inv[n bs + o].
__global__ void monarch2_project(const float* dm, const float* R, const float* L, float* dR, float* dL, int H, int nb,
                                 int bs) {
  const int64_t n = (int64_t)3 * H * bs;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(e % bs);
    const int64_t r = e / bs;
    const int o = (int)(r % bs);
    const int64_t gb = r / bs;
    const int blk = (int)(gb % nb), g = (int)(gb / nb);
    const float* dmg = dm + (int64_t)g * H * H;
    {
      const int x = m2_perm(blk * bs + o, nb, bs);
      const int mm = m2_perm(blk * bs + i, nb, bs), mb = mm / bs;
      const float* dmr = dmg + (int64_t)x * H + mb * bs;
      const float* Rr = R + (((int64_t)g * nb + mb) * bs + mm % bs) * bs;
      float acc = 0.0f;
      for (int k = 0; k < bs; ++k) acc += dmr[k] * Rr[k];
      dL[e] = acc;
    }
    {
      const int q = m2_inv(blk * bs + o, nb, bs), qb = q / bs;
      const float* Lb = L + ((int64_t)g * nb + qb) * bs * bs + q % bs;
      float acc = 0.0f;
      for (int i2 = 0; i2 < bs; ++i2) {
        const int qq = qb * bs + i2;
        acc += Lb[(int64_t)i2 * bs] * dmg[(int64_t)m2_perm(qq, nb, bs) * H + blk * bs + i];
      }
      dR[e] = acc;
    }
  }
}

// ---- butterfly ---------------------------------------------------------------------

// Stage j of the chain: chain c = j / L, layer s = j % L; stride 2^ls with
// ls = s for even chains and L - 1 - s for odd ones. Row i pairs with
// i ^ stride; its twiddles sit at tw[g][c][s][pair][m][*],
// m = (i >> ls) & 1, pair = (i >> (ls + 1)) stride + (i & (stride - 1)).
struct Stage {
  int ls, stride;
  int64_t tw_off;  // offset of tw[g][c][s][0][0][0] without the gate term
};

__device__ __forceinline__ Stage stage_of(int j, int L, int N) {
  const int c = j / L, s = j - c * L;
  Stage st;
  st.ls = (c % 2 == 0) ? s : L - 1 - s;
  st.stride = 1 << st.ls;
  st.tw_off = ((int64_t)c * L + s) * (N / 2) * 4;
  return st;
}

__device__ __forceinline__ int64_t tw_index(const Stage& st, int i) {
  const int m = (i >> st.ls) & 1;
  const int pair = (i >> (st.ls + 1)) * st.stride + (i & (st.stride - 1));
  return st.tw_off + (int64_t)pair * 4 + m * 2;  // + m' for the column
}

// A_0 = [I_H; 0] for every gate: acts[g][0] is [N][H].
__global__ void bfly_identity(float* acts, int64_t gate_stride, int N, int H) {
  const int64_t n = (int64_t)3 * N * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int g = (int)(e / ((int64_t)N * H));
    const int64_t r = e - (int64_t)g * N * H;
    const int i = (int)(r / H), k = (int)(r - (int64_t)i * H);
    acts[g * gate_stride + r] = (i == k) ? 1.0f : 0.0f;
  }
}

// dst = A_{j+1} from src = A_j (each [N][H] per gate, gates gate_stride
// apart): A_{j+1}[i][k] = tw_ii A_j[i][k] + tw_ip A_j[i ^ stride][k]; the
// last stage also writes rows i < H into M (rows g H + i).
__global__ void bfly_stage_fwd(const float* tw, int64_t tw_gate, const float* src, float* dst, int64_t gate_stride,
                               int j, int L, int N, int H, float* m_out) {
  const int64_t n = (int64_t)3 * N * H;
  const Stage st = stage_of(j, L, N);
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int g = (int)(e / ((int64_t)N * H));
    const int64_t r = e - (int64_t)g * N * H;
    const int i = (int)(r / H), k = (int)(r - (int64_t)i * H);
    const float* a = src + g * gate_stride;
    const float* t = tw + g * tw_gate + tw_index(st, i);
    const int m = (i >> st.ls) & 1;
    float y;
    {
#pragma clang fp contract(off)
      y = t[m] * a[(int64_t)i * H + k] + t[1 - m] * a[(int64_t)(i ^ st.stride) * H + k];
    }
    dst[g * gate_stride + r] = y;
    if (m_out != nullptr && i < H) m_out[((int64_t)g * H + i) * H + k] = y;
  }
}

// Diagonal: M[g H + x][k] = (x == k) ? w[g][k] : 0.
__global__ void diagonal_materialize(const float* w, float* m, int H) {
  const int64_t n = (int64_t)3 * H * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(e / H), k = (int)(e - (int64_t)row * H);
    const int g = row / H, x = row - g * H;
    m[e] = x == k ? w[(int64_t)g * H + k] : 0.0f;
  }
}

// Circulant: M[g H + i][k] = col[g][(i - k) mod H].
__global__ void circulant_materialize(const float* col, float* m, int H) {
  const int64_t n = (int64_t)3 * H * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(e / H), k = (int)(e - (int64_t)row * H);
    const int g = row / H, i = row - g * H;
    int d = i - k;
    if (d < 0) d += H;
    m[e] = col[(int64_t)g * H + d];
  }
}

// dcol[g][d] = sum_i dM[g H + i][(i - d) mod H], one thread per (g, d), i ascending.
__global__ void circulant_project(const float* dm, float* dcol, int H) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 3 * H) return;
  const int g = e / H, d = e - g * H;
  const float* base = dm + (int64_t)g * H * H;
  float acc = 0.0f;
  for (int i = 0; i < H; ++i) {
    int k = i - d;
    if (k < 0) k += H;
    acc += base[(int64_t)i * H + k];
  }
  dcol[e] = acc;
}

// dw[g][k] = dM[g H + k][k].
__global__ void diagonal_project(const float* dm, float* dw, int H) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 3 * H) return;
  const int g = e / H, k = e - g * H;
  dw[e] = dm[((int64_t)g * H + k) * H + k];
}

// G_K = [dM_g; 0].
__global__ void bfly_grad_init(const float* dm, float* gbuf, int64_t gate_stride, int N, int H) {
  const int64_t n = (int64_t)3 * N * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int g = (int)(e / ((int64_t)N * H));
    const int64_t r = e - (int64_t)g * N * H;
    const int i = (int)(r / H), k = (int)(r - (int64_t)i * H);
    gbuf[g * gate_stride + r] = i < H ? dm[((int64_t)g * H + i) * H + k] : 0.0f;
  }
}

// One workgroup per (gate, row i) of stage j: the twiddle gradients of row i
// (dots of G_{j+1}[i] with A_j[i] and A_j[i ^ stride]) and row i of
// G_j = S_j^T G_{j+1}: G_j[i] = tw_ii G_{j+1}[i] + tw'_{pi} G_{j+1}[i ^ stride],
// where tw'_{pi} is the partner row's off-diagonal twiddle.
constexpr int kRowThreads = 256;
__global__ __launch_bounds__(kRowThreads) void bfly_stage_bwd(const float* tw, int64_t tw_gate, const float* acts,
                                                              int64_t act_gate, const float* gin, float* gout,
                                                              int64_t g_gate, float* dtw, int j, int L, int N, int H) {
  __shared__ float red[2][kRowThreads / 64];
  const int g = blockIdx.y, i = blockIdx.x;
  const Stage st = stage_of(j, L, N);
  const int p = i ^ st.stride;
  const int m = (i >> st.ls) & 1;
  const float* t = tw + g * tw_gate + tw_index(st, i);
  const float* tp = tw + g * tw_gate + tw_index(st, p);  // partner row: its own m is 1 - m
  const float t_ii = t[m], t_pi = tp[m];                 // tp[(1 - m_p) = m] is the partner's off-diagonal
  const float* Gi = gin + g * g_gate + (int64_t)i * H;
  const float* Gp = gin + g * g_gate + (int64_t)p * H;
  const float* Ai = acts + g * act_gate + (int64_t)j * N * H + (int64_t)i * H;
  const float* Ap = acts + g * act_gate + (int64_t)j * N * H + (int64_t)p * H;
  float* Go = gout + g * g_gate + (int64_t)i * H;
  float s_ii = 0.f, s_ip = 0.f;
  for (int k = threadIdx.x; k < H; k += kRowThreads) {
    const float gi = Gi[k];
    s_ii += gi * Ai[k];
    s_ip += gi * Ap[k];
    float y;
    {
#pragma clang fp contract(off)
      y = t_ii * gi + t_pi * Gp[k];
    }
    Go[k] = y;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    s_ii += __shfl_xor(s_ii, o);
    s_ip += __shfl_xor(s_ip, o);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = s_ii;
    red[1][wave] = s_ip;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = 0.f, b = 0.f;
    for (int w = 0; w < kRowThreads / 64; ++w) {
      a += red[0][w];
      b += red[1][w];
    }
    float* d = dtw + g * tw_gate + tw_index(st, i);
    d[m] = a;
    d[1 - m] = b;
  }
}

struct StructPlan {
  int64_t core, core_scratch, mat_bytes, act_bytes, g_bytes;
  int N = 0, L = 0, K = 0;
  int64_t total() const { return core; }  // tagged workspace: the dense core's
  int64_t scratch() const { return core_scratch + 2 * mat_bytes + act_bytes + g_bytes; }
};

int plan_struct(int kind, const gs_bwd_args* a, StructPlan* sp, const char* who) {
  const int64_t core = dense_bwd_core_bytes(a, who);
  if (core < 0) return (int)core;
  const int64_t core_scratch = dense_bwd_core_scratch(a, who);
  if (core_scratch < 0) return (int)core_scratch;
  sp->core = core;
  sp->core_scratch = core_scratch;
  const int64_t H = a->H;
  sp->mat_bytes = align256(3 * H * H * 4);
  sp->act_bytes = sp->g_bytes = 0;
  if (kind == GS_KIND_MONARCH) {
    if (a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != H)
      return set_error(GS_ERR_INVALID, "%s: Wh_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                       (long long)a->nblocks, (long long)a->blksz, (long long)H);
  } else {
    if (a->log_n < 1 || a->log_n > 12 || a->bfly_nblocks < 1 || a->bfly_nblocks > 64)
      return set_error(GS_ERR_INVALID, "%s: butterfly needs 1 <= log_n <= 12 and 1 <= nblocks <= 64; got %lld, %lld", who,
                       (long long)a->log_n, (long long)a->bfly_nblocks);
    sp->N = 1 << a->log_n;
    sp->L = (int)a->log_n;
    sp->K = (int)a->bfly_nblocks * sp->L;
    if (sp->N < H)
      return set_error(GS_ERR_INVALID, "%s: H_PAD = 2^log_n = %d must be >= H = %lld", who, sp->N, (long long)H);
    sp->act_bytes = align256((int64_t)3 * (sp->K + 1) * sp->N * H * 4);
    sp->g_bytes = align256((int64_t)2 * 3 * sp->N * H * 4);
  }
  return GS_OK;
}

}  // namespace

// The materialized-map backward of either kind (the butterfly entry point
// also falls back here for shapes its stage kernels cannot hold in LDS).
int run_struct(int kind, const gs_bwd_args* a, hipStream_t stream, const char* who) {
  clear_error();
  int rc = validate_bwd_common(a, who);
  if (rc) return rc;
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  if (kind == GS_KIND_MONARCH && a->w2 != nullptr && a->dw2_part == nullptr)
    return set_error(GS_ERR_INVALID, "%s: dw2_part must be non-NULL for a two-factor Monarch", who);
  if (kind == GS_KIND_BUTTERFLY && a->w2 != nullptr)
    return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the butterfly kind", who);
  StructPlan sp;
  rc = plan_struct(kind, a, &sp, who);
  if (rc) return rc;
  const gs_args f = fwd_view(*a);
  rc = check_workspace(&f, sp.total(), who);
  if (rc) return rc;
  rc = check_scratch(a, sp.scratch(), who);
  if (rc) return rc;

  const int H = (int)a->H;
  char* base = static_cast<char*>(a->scratch) + sp.core_scratch;
  float* M = reinterpret_cast<float*>(base);
  float* dM = reinterpret_cast<float*>(base + sp.mat_bytes);
  const int64_t nmat = (int64_t)3 * H * H;

  if (kind == GS_KIND_MONARCH) {
    const int nb = (int)a->nblocks, bs = (int)a->blksz;
    if (a->w2 == nullptr)
      hipLaunchKernelGGL(monarch1_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, M, H, nb, bs);
    else
      hipLaunchKernelGGL(monarch2_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, a->w2, M, H, nb, bs);
    GS_CHECK_HIP(hipGetLastError());
    rc = dense_bwd_core(a, M, dM, stream, who);
    if (rc) return rc;
    const int64_t np = (int64_t)3 * H * bs;
    if (a->w2 == nullptr)
      hipLaunchKernelGGL(monarch1_project, grid_for(np), dim3(256), 0, stream, dM, a->dw_part, H, nb, bs);
    else
      hipLaunchKernelGGL(monarch2_project, grid_for(np), dim3(256), 0, stream, dM, a->w, a->w2, a->dw_part,
                         a->dw2_part, H, nb, bs);
    GS_CHECK_HIP(hipGetLastError());
    return GS_OK;
  }

  // butterfly
  const int N = sp.N, L = sp.L, K = sp.K;
  float* acts = reinterpret_cast<float*>(base + 2 * sp.mat_bytes);
  float* gb = reinterpret_cast<float*>(base + 2 * sp.mat_bytes + sp.act_bytes);
  const int64_t act_gate = (int64_t)(K + 1) * N * H;
  const int64_t g_gate = (int64_t)N * H;
  const int64_t tw_gate = (int64_t)a->bfly_nblocks * L * (N / 2) * 4;
  const int64_t nstage = (int64_t)3 * N * H;
  hipLaunchKernelGGL(bfly_identity, grid_for(nstage), dim3(256), 0, stream, acts, act_gate, N, H);
  GS_CHECK_HIP(hipGetLastError());
  for (int j = 0; j < K; ++j) {
    hipLaunchKernelGGL(bfly_stage_fwd, grid_for(nstage), dim3(256), 0, stream, a->w, tw_gate,
                       acts + (int64_t)j * N * H, acts + (int64_t)(j + 1) * N * H, act_gate, j, L, N, H,
                       j == K - 1 ? M : nullptr);
    GS_CHECK_HIP(hipGetLastError());
  }
  rc = dense_bwd_core(a, M, dM, stream, who);
  if (rc) return rc;
  float* g0 = gb;
  float* g1 = gb + 3 * g_gate;
  hipLaunchKernelGGL(bfly_grad_init, grid_for(nstage), dim3(256), 0, stream, dM, g0, g_gate, N, H);
  GS_CHECK_HIP(hipGetLastError());
  for (int j = K - 1; j >= 0; --j) {
    hipLaunchKernelGGL(bfly_stage_bwd, dim3((unsigned)N, 3), dim3(kRowThreads), 0, stream, a->w, tw_gate, acts,
                       act_gate, g0, g1, g_gate, a->dw_part, j, L, N, H);
    GS_CHECK_HIP(hipGetLastError());
    std::swap(g0, g1);
  }
  return GS_OK;
}

int validate_map(const gs_map_args* a, const char* who) {
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  const int64_t H = a->H;
  if (H < 1 || H > 4096) return set_error(GS_ERR_INVALID, "%s: H must be in [1, 4096]; got %lld", who, (long long)H);
  switch (a->kind) {
    case GS_KIND_DENSE:
    case GS_KIND_DIAGONAL:
    case GS_KIND_CIRCULANT:
      if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for this kind", who);
      return GS_OK;
    case GS_KIND_MONARCH:
      if (a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != H)
        return set_error(GS_ERR_INVALID, "%s: Wh_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                         (long long)a->nblocks, (long long)a->blksz, (long long)H);
      return GS_OK;
    case GS_KIND_BUTTERFLY:
      if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the butterfly kind", who);
      if (a->log_n < 1 || a->log_n > 12 || a->bfly_nblocks < 1 || a->bfly_nblocks > 64)
        return set_error(GS_ERR_INVALID, "%s: butterfly needs 1 <= log_n <= 12 and 1 <= nblocks <= 64; got %lld, %lld",
                         who, (long long)a->log_n, (long long)a->bfly_nblocks);
      if ((int64_t(1) << a->log_n) < H)
        return set_error(GS_ERR_INVALID, "%s: H_PAD = 2^log_n = %lld must be >= H = %lld", who,
                         (long long)(int64_t(1) << a->log_n), (long long)H);
      return GS_OK;
    default:
      return set_error(GS_ERR_INVALID, "%s: unknown kind %d", who, a->kind);
  }
}

int64_t hidden_map_scratch(const gs_map_args* a) {
  if (a->kind != GS_KIND_BUTTERFLY) return 0;
  return 2 * align256((int64_t)3 * (int64_t(1) << a->log_n) * a->H * 4);
}

// Writes the hidden map of `a` as the dense [3H, H] matrix a->m
// (gh = hq m^T + bh).
int materialize_map(const gs_map_args* a, hipStream_t stream, const char* who) {
  const int H = (int)a->H;
  const int64_t nmat = (int64_t)3 * H * H;
  switch (a->kind) {
    case GS_KIND_DENSE:
      GS_CHECK_HIP(hipMemcpyAsync(a->m, a->w, nmat * 4, hipMemcpyDeviceToDevice, stream));
      return GS_OK;
    case GS_KIND_DIAGONAL:
      hipLaunchKernelGGL(diagonal_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, a->m, H);
      break;
    case GS_KIND_CIRCULANT:
      hipLaunchKernelGGL(circulant_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, a->m, H);
      break;
    case GS_KIND_MONARCH:
      if (a->w2 == nullptr)
        hipLaunchKernelGGL(monarch1_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, a->m, H, (int)a->nblocks,
                           (int)a->blksz);
      else
        hipLaunchKernelGGL(monarch2_materialize, grid_for(nmat), dim3(256), 0, stream, a->w, a->w2, a->m, H,
                           (int)a->nblocks, (int)a->blksz);
      break;
    default: {  // butterfly: A_0 = [I; 0], then the K stages ping-ponging through the scratch
      const int L = (int)a->log_n, N = 1 << L, K = (int)a->bfly_nblocks * L;
      const int64_t half = hidden_map_scratch(a) / 2;
      float* buf[2] = {static_cast<float*>(a->scratch),
                       reinterpret_cast<float*>(static_cast<char*>(a->scratch) + half)};
      const int64_t gate = (int64_t)N * H, nstage = 3 * gate;
      const int64_t tw_gate = (int64_t)a->bfly_nblocks * L * (N / 2) * 4;
      hipLaunchKernelGGL(bfly_identity, grid_for(nstage), dim3(256), 0, stream, buf[0], gate, N, H);
      GS_CHECK_HIP(hipGetLastError());
      for (int j = 0; j < K; ++j) {
        hipLaunchKernelGGL(bfly_stage_fwd, grid_for(nstage), dim3(256), 0, stream, a->w, tw_gate, buf[j & 1],
                           buf[(j + 1) & 1], gate, j, L, N, H, j == K - 1 ? a->m : nullptr);
        GS_CHECK_HIP(hipGetLastError());
      }
      return GS_OK;
    }
  }
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

// The butterfly map of all three gates as the dense M [3H, H], keeping every
// stage's activations A_j in acts ([3][K + 1][N][H] floats, K = nch L).
int bfly_materialize_keep(const float* tw, int nch, int L, int H, float* acts, float* M, hipStream_t stream) {
  const int N = 1 << L, K = nch * L;
  const int64_t act_gate = (int64_t)(K + 1) * N * H, nstage = (int64_t)3 * N * H;
  const int64_t tw_gate = (int64_t)nch * L * (N / 2) * 4;
  hipLaunchKernelGGL(bfly_identity, grid_for(nstage), dim3(256), 0, stream, acts, act_gate, N, H);
  GS_CHECK_HIP(hipGetLastError());
  for (int j = 0; j < K; ++j) {
    hipLaunchKernelGGL(bfly_stage_fwd, grid_for(nstage), dim3(256), 0, stream, tw, tw_gate,
                       acts + (int64_t)j * N * H, acts + (int64_t)(j + 1) * N * H, act_gate, j, L, N, H,
                       j == K - 1 ? M : nullptr);
    GS_CHECK_HIP(hipGetLastError());
  }
  return GS_OK;
}

// The same map without keeping the activations: the stages ping-pong between
// two planes of 3 N H floats in buf.
int bfly_materialize(const float* tw, int nch, int L, int H, float* buf, float* M, hipStream_t stream) {
  const int N = 1 << L, K = nch * L;
  const int64_t gate = (int64_t)N * H, nstage = 3 * gate;
  const int64_t tw_gate = (int64_t)nch * L * (N / 2) * 4;
  float* pp[2] = {buf, buf + nstage};
  hipLaunchKernelGGL(bfly_identity, grid_for(nstage), dim3(256), 0, stream, pp[0], gate, N, H);
  GS_CHECK_HIP(hipGetLastError());
  for (int j = 0; j < K; ++j) {
    hipLaunchKernelGGL(bfly_stage_fwd, grid_for(nstage), dim3(256), 0, stream, tw, tw_gate, pp[j & 1],
                       pp[(j + 1) & 1], gate, j, L, N, H, j == K - 1 ? M : nullptr);
    GS_CHECK_HIP(hipGetLastError());
  }
  return GS_OK;
}

// Carries a dense gradient dM [3H, H] of that map onto the twiddles dtw (the
// shape of tw), with the activations bfly_materialize_keep left in acts;
// gbuf holds 2 * 3 N H floats.
int bfly_project_grad(const float* tw, int nch, int L, int H, const float* acts, const float* dM, float* gbuf,
                      float* dtw, hipStream_t stream) {
  const int N = 1 << L, K = nch * L;
  const int64_t act_gate = (int64_t)(K + 1) * N * H, g_gate = (int64_t)N * H, nstage = 3 * g_gate;
  const int64_t tw_gate = (int64_t)nch * L * (N / 2) * 4;
  float* g0 = gbuf;
  float* g1 = gbuf + 3 * g_gate;
  hipLaunchKernelGGL(bfly_grad_init, grid_for(nstage), dim3(256), 0, stream, dM, g0, g_gate, N, H);
  GS_CHECK_HIP(hipGetLastError());
  for (int j = K - 1; j >= 0; --j) {
    hipLaunchKernelGGL(bfly_stage_bwd, dim3((unsigned)N, 3), dim3(kRowThreads), 0, stream, tw, tw_gate, acts, act_gate,
                       g0, g1, g_gate, dtw, j, L, N, H);
    GS_CHECK_HIP(hipGetLastError());
    std::swap(g0, g1);
  }
  return GS_OK;
}

int64_t struct_bwd_workspace_bytes(int kind, const gs_bwd_args* a) {
  StructPlan sp;
  const int rc = plan_struct(kind, a, &sp, "gs_bwd_workspace_bytes");
  if (rc) return rc;
  return sp.total();
}

int64_t struct_bwd_scratch_bytes(int kind, const gs_bwd_args* a) {
  StructPlan sp;
  const int rc = plan_struct(kind, a, &sp, "gs_bwd_scratch_bytes");
  if (rc) return rc;
  return sp.scratch();
}

}  // namespace gs

extern "C" int64_t gs_hidden_map_scratch_bytes(const gs_map_args* a) {
  using namespace gs;
  const int rc = validate_map(a, "gs_hidden_map_scratch_bytes");
  if (rc) return rc;
  return hidden_map_scratch(a);
}

extern "C" int gs_hidden_map_grad(const gs_map_args* a, const float* dm, float* dw, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_hidden_map_grad";
  int rc = validate_map(a, who);
  if (rc) return rc;
  if (!dm || !dw) return set_error(GS_ERR_INVALID, "%s: dm and dw must be non-NULL device pointers", who);
  const int H = (int)a->H;
  const unsigned blocks = (unsigned)((3 * H + 255) / 256);
  switch (a->kind) {
    case GS_KIND_DIAGONAL:
      hipLaunchKernelGGL(diagonal_project, dim3(blocks), dim3(256), 0, stream, dm, dw, H);
      break;
    case GS_KIND_CIRCULANT:
      hipLaunchKernelGGL(circulant_project, dim3(blocks), dim3(256), 0, stream, dm, dw, H);
      break;
    case GS_KIND_MONARCH:
      if (a->w2 != nullptr)
        return set_error(GS_ERR_INVALID, "%s: a two-factor Monarch gets its gradients from gs_monarch_bwd", who);
      hipLaunchKernelGGL(monarch1_project, grid_for((int64_t)3 * H * a->blksz), dim3(256), 0, stream, dm, dw, H,
                         (int)a->nblocks, (int)a->blksz);
      break;
    default:
      return set_error(GS_ERR_INVALID, "%s: kind %d has no dense-gradient fold here (use its backward entry point)",
                       who, a->kind);
  }
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

extern "C" int gs_hidden_map_dense(const gs_map_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_hidden_map_dense";
  int rc = validate_map(a, who);
  if (rc) return rc;
  if (!a->w || !a->m) return set_error(GS_ERR_INVALID, "%s: w and m must be non-NULL device pointers", who);
  const int64_t need = hidden_map_scratch(a);
  if (need > 0 && (a->scratch == nullptr || a->scratch_bytes < need))
    return set_error(GS_ERR_INVALID, "%s: scratch of %lld bytes required; got %lld", who, (long long)need,
                     (long long)a->scratch_bytes);
  return materialize_map(a, stream, who);
}

