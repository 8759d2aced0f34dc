// Single-factor Monarch GRU scan backward (gfx950) on the block structure.
//
// Reference: the Monarch backward (LarocheC/gru-triton
// src/gru_qat/triton_kernels/scan_monarch.py:409-884, PyTorch form :955-1053),
// with the linearized recurrence of the dense backward (scan_dense_bwd.hip):
//   D_{t-1} = dout[t-1] + Zm_t D_t + Mi_t (dgh_t M),   dgh_t = D_t (Cr, Cz, Chn)_t
// The map M is block-diagonal (gh[b, g, n, o] = sum_i hq[b, n bs + i]
// W[g, n, o, i] + bh), so every block n of every batch row is its own
// recurrence: D_{t-1} restricted to block n needs only block n of dgh_t. The
// launcher runs the dense backward's passes with block-batched products:
//   0. hq = q_in([h0; out[0..T-2]])                      (build_prev_state)
//   1. gh: one batched NT GEMM, 3 nb products [T B, bs] x [bs, bs]^T + bh
//   2. coef_kernel (scan_dense_bwd.hip)
//   3. monarch1_bwd_kernel: one workgroup per (block, batch rows) walks t
//      from T-1 to 0 with D in registers and dgh_t in LDS; no exchange
//      between workgroups
//   4. grad_kernel (dgi, dbh, and dgh = (dg_r, dg_z, dgh_n) over cg)
//   5. dW[g][n] = sum_m dgh[m, g, n, :]^T hq[m, n, :]: one batched TN GEMM
//      of 3 nb products with the T B terms split, then one sum.
// The dense path would spend 3H H per row-step on the map; this one spends
// 3 bs^2 per block (1/nb of it) and never leaves the workgroup per step.
// Shapes outside blksz in {16, 32, 64, 128}, and the two-factor form, take
// the materialized path (scan_struct_bwd.hip).
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {

int run_struct(int kind, const gs_bwd_args* a, hipStream_t stream, const char* who);
int64_t struct_bwd_workspace_bytes(int kind, const gs_bwd_args* a);
int64_t struct_bwd_scratch_bytes(int kind, const gs_bwd_args* a);
int launch_coef(const gs_bwd_args* a, float* cg, float* cgn, float* zm, float* mi, hipStream_t stream,
                float* hq = nullptr);
int grad_chunks(int64_t T);
int launch_grad(const gs_bwd_args* a, const float* dsum, const float* cg, const float* cgn, float* dghn,
                float* dgh, float* chunks, hipStream_t stream, const char* who, SumJob* dbh_sum = nullptr);

namespace {

constexpr int kDepth = 8;  // steps of per-unit inputs loaded ahead

// Lanes (adjacent) sharing one unit's dot product over 3 bs terms (8 for
// blksz 128 measured 4x slower: 1024-thread workgroups leave 128 VGPRs a lane).
template <int BS>
constexpr int split_k() {
  return 4;
}

struct M1Params {
  const float* w;     // [3, nb, bs, bs] (out, in)
  const float* dout;  // [T, B, H]
  const float* cg;    // [T, B, 3H] (Cr, Cz, Chn)
  const float* zm;    // [T, B, H]
  const float* mi;    // [T, B, H]
  float* dsum;        // [T, B, H] D_t
  float* dh0;         // [B, H]
  int T, B, H, nb;
};

template <int BS>
constexpr int rows_per_wg() {
  return split_k<BS>() * BS >= 256 ? 1 : 256 / (split_k<BS>() * BS);
}

template <int BS>
constexpr int m1_threads() {
  return split_k<BS>() * BS * rows_per_wg<BS>();
}

// Thread (row slot rs, unit u, part kq) of workgroup (block n, row group):
// holds W[g][n][j][u] for its part of the 3 bs terms kk = g bs + j in
// registers, sums dgh_t[kk] W over them, and the SK adjacent lanes of unit u
// combine the parts (DPP). Every one of them then has D_{t-1}[u]; lane
// kq < 3 writes dgh_{t-1}[kq][u] = D_{t-1} C_kq for the next step.
template <int BS>
__global__ __launch_bounds__(m1_threads<BS>()) void monarch1_bwd_kernel(M1Params p) {
  constexpr int SK = split_k<BS>();
  constexpr int TPR = SK * BS;  // threads per batch row
  constexpr int R = rows_per_wg<BS>();
  constexpr int KT = 3 * BS / SK;  // terms per thread
  static_assert(KT % 4 == 0, "terms per thread must be whole float4s");
  __shared__ __attribute__((aligned(16))) float dgh[2][R][3 * BS];

  const int n = blockIdx.x;
  const int rs = threadIdx.x / TPR, lt = threadIdx.x - rs * TPR;
  const int u = lt / SK, kq = lt % SK;
  const int b = blockIdx.y * R + rs;
  const bool live = b < p.B;
  const int H = p.H, T = p.T;
  const int col = n * BS + u;
  const int64_t BH = (int64_t)p.B * H;
  const int64_t e0 = (int64_t)(live ? b : 0) * H + col;                    // (b, col) in a [B, H] plane
  const int64_t c0 = (int64_t)(live ? b : 0) * 3 * H + (kq < 3 ? kq : 0) * H + col;  // gate kq in cg

  float wt[KT];
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    const int kk = kq * KT + i, g = kk / BS, j = kk - g * BS;
    wt[i] = p.w[(((int64_t)g * p.nb + n) * BS + j) * BS + u];
  }

  // Per-step inputs of the iteration that consumes D_t: Zm_t, Mi_t, dout[t-1],
  // C_kq[t-1]. Rows past B read row 0 and t is clamped to 0, so no load is
  // branched around; the values a step must not use (dead rows, t = 0, parts
  // kq = 3) are zeroed when the step reads them. Two register sets take turns
  // (one set's kDepth steps compute while the other's loads are in flight), so
  // the wait before a step counts only the loads issued before its own.
  auto load = [&](int t0, float* zm, float* mi, float* dn, float* cc) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const int t = max(t0 - i, 0), tp = max(t0 - i - 1, 0);
      zm[i] = p.zm[(int64_t)t * BH + e0];
      mi[i] = p.mi[(int64_t)t * BH + e0];
      dn[i] = p.dout[(int64_t)tp * BH + e0];
      cc[i] = p.cg[(int64_t)tp * 3 * BH + c0];
    }
  };

  // D_{T-1} = dout[T-1]
  float D = live ? p.dout[(int64_t)(T - 1) * BH + e0] : 0.0f;
  if (live && kq == 0) p.dsum[(int64_t)(T - 1) * BH + e0] = D;
  if (kq < 3) dgh[0][rs][kq * BS + u] = live ? D * p.cg[(int64_t)(T - 1) * 3 * BH + c0] : 0.0f;

  int buf = 0;
  // Runs steps t0 down to t0 - kDepth + 1; true once step 0 is done.
  auto run = [&](int t0, const float* czm, const float* cmi, const float* cdn, const float* ccc) -> bool {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const int t = t0 - i;
      if (t < 0) return true;
      const float* src = &dgh[buf][rs][kq * KT];
      f4 a4 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < KT; q += 4) {
        const f4 v = *reinterpret_cast<const f4*>(src + q);
#pragma unroll
        for (int c = 0; c < 4; ++c) a4[c] += v[c] * wt[q + c];
      }
      float acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
      acc += lane_xor_c<1>(acc);
      acc += lane_xor_c<2>(acc);
      const float zm = live ? czm[i] : 0.0f, mi = live ? cmi[i] : 0.0f;
      float carry;
      {
#pragma clang fp contract(off)
        carry = zm * D + mi * acc;
      }
      if (t == 0) {
        if (live && kq == 0) p.dh0[e0] = carry;
      } else {
        D = (live ? cdn[i] : 0.0f) + carry;
        if (kq < 3) dgh[buf ^ 1][rs][kq * BS + u] = D * (live ? ccc[i] : 0.0f);
        if (live && kq == 0) p.dsum[(int64_t)(t - 1) * BH + e0] = D;
      }
      // LDS-only barrier: the step's global stores need not complete here
      lds_barrier();
      buf ^= 1;
    }
    return t0 - kDepth < 0;
  };

  float azm[kDepth], ami[kDepth], adn[kDepth], acc_[kDepth];
  float xzm[kDepth], xmi[kDepth], xdn[kDepth], xcc[kDepth];
  load(T - 1, azm, ami, adn, acc_);
  __syncthreads();
  for (int t0 = T - 1;; t0 -= 2 * kDepth) {
    load(t0 - kDepth, xzm, xmi, xdn, xcc);
    if (run(t0, azm, ami, adn, acc_)) return;
    load(t0 - 2 * kDepth, azm, ami, adn, acc_);
    if (run(t0 - kDepth, xzm, xmi, xdn, xcc)) return;
  }
}

typedef void (*M1Fn)(M1Params);

M1Fn pick_m1(int bs, int* threads, int* rows) {
  switch (bs) {
    case 16: *rows = rows_per_wg<16>(); *threads = m1_threads<16>(); return monarch1_bwd_kernel<16>;
    case 32: *rows = rows_per_wg<32>(); *threads = m1_threads<32>(); return monarch1_bwd_kernel<32>;
    case 64: *rows = rows_per_wg<64>(); *threads = m1_threads<64>(); return monarch1_bwd_kernel<64>;
    case 128: *rows = rows_per_wg<128>(); *threads = m1_threads<128>(); return monarch1_bwd_kernel<128>;
    default: return nullptr;
  }
}

// Scratch (plain floats), each region 256-byte aligned: hq, cgn, zm, mi, dsum
// [T B, H] | cg [T B, 3H] | dbh chunks | dW split partials.
struct M1Plan {
  bool ok = false;
  int bs = 0, nb = 0, split = 1;
  int64_t plane = 0, cg = 0, chunks = 0, part = 0;
  int64_t scratch() const { return 5 * plane + cg + chunks + part; }
};

M1Plan plan_m1(const gs_bwd_args* a) {
  M1Plan pl;
  if (a->w2 != nullptr || a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != a->H) return pl;
  int th = 0, rows = 0;
  if (pick_m1((int)a->blksz, &th, &rows) == nullptr) return pl;
  const int64_t TB = a->T * a->B, H = a->H;
  if (TB > INT32_MAX / 4) return pl;
  pl.bs = (int)a->blksz;
  pl.nb = (int)a->nblocks;
  pl.split = gemm_pick_split(pl.bs, pl.bs, (int)TB);
  pl.plane = align256(TB * H * 4);
  pl.cg = align256(TB * 3 * H * 4);
  pl.chunks = align256((int64_t)grad_chunks(a->T) * a->B * 3 * H * 4);
  pl.part = pl.split > 1 ? align256((int64_t)pl.split * 3 * H * pl.bs * 4) : 0;
  pl.ok = true;
  return pl;
}

}  // namespace

int64_t monarch_bwd_workspace_bytes(const gs_bwd_args* a) {
  if (plan_m1(a).ok) return 0;
  return struct_bwd_workspace_bytes(GS_KIND_MONARCH, a);
}

int64_t monarch_bwd_scratch_bytes(const gs_bwd_args* a) {
  const M1Plan pl = plan_m1(a);
  if (pl.ok) return pl.scratch();
  return struct_bwd_scratch_bytes(GS_KIND_MONARCH, a);
}

}  // namespace gs

extern "C" int gs_monarch_bwd(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  const char* who = "gs_monarch_bwd";
  clear_error();
  // gh_saved: the block-local single-factor backward only
  int rc = validate_bwd_common(a, who, a != nullptr && plan_m1(a).ok);
  if (rc) return rc;
  const M1Plan pl = plan_m1(a);
  if (!pl.ok) return run_struct(GS_KIND_MONARCH, a, stream, who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  if (a->T > 1 && a->so_t != a->B * a->so_b)
    return set_error(GS_ERR_INVALID, "%s: out must hold its steps back to back (so_t == B * so_b); got so_t=%lld, so_b=%lld",
                     who, (long long)a->so_t, (long long)a->so_b);
  rc = check_scratch(a, pl.scratch(), who);
  if (rc) return rc;

  const int T = (int)a->T, B = (int)a->B, H = (int)a->H, TB = T * B;
  const int bs = pl.bs, nb = pl.nb;
  char* cur = static_cast<char*>(a->scratch);
  auto take = [&](int64_t bytes) {
    char* r = cur;
    cur += bytes;
    return reinterpret_cast<float*>(r);
  };
  float* hq = take(pl.plane);
  float* cgn = take(pl.plane);
  float* zm = take(pl.plane);
  float* mi = take(pl.plane);
  float* dsum = take(pl.plane);
  float* cg = take(pl.cg);
  float* chunks = take(pl.chunks);
  float* part = take(pl.part);

  // 0. hq = q_in([h0; out[0..T-2]]); with the saved gh the coefficient pass writes it instead
  if (a->gh_saved == nullptr) {
    rc = build_prev_state(hq, a->h0, a->sh0_b, a->out, a->so_b, T, B, H, to_quant(a->q_in), stream, who);
    if (rc) return rc;
  }

  // 1. gh: product z = g nb + n writes cg[:, z bs : (z + 1) bs] = hq[:, n bs : (n + 1) bs] W[g][n]^T + bh,
  //    unless the forward saved it (launch_coef then reads it and adds bh)
  if (a->gh_saved == nullptr) {
    GemmArgs g1;
    g1.a = hq;
    g1.lda = H;
    g1.a_bs = bs;
    g1.a_mod = nb;
    g1.b = a->w;  // B(k, j) = W[z][j][k]
    g1.ldb = bs;
    g1.b_bs = (int64_t)bs * bs;
    g1.b_mod = 3 * nb;
    g1.c = cg;
    g1.ldc = 3 * H;
    g1.c_bs = bs;
    g1.bias = a->bh;
    g1.bias_bs = bs;
    g1.M = TB;
    g1.N = bs;
    g1.K = bs;
    g1.batch = 3 * nb;
    g1.layout = kGemmNT;
    rc = gemm_f32(g1, stream, who);
    if (rc) return rc;
  }

  // 2. coefficient planes
  rc = launch_coef(a, cg, cgn, zm, mi, stream, a->gh_saved != nullptr ? hq : nullptr);
  if (rc) return rc;

  // 3. the block-local recurrence
  int threads = 0, rows = 0;
  M1Fn fn = pick_m1(bs, &threads, &rows);
  M1Params p;
  p.w = a->w;
  p.dout = a->dout;
  p.cg = cg;
  p.zm = zm;
  p.mi = mi;
  p.dsum = dsum;
  p.dh0 = a->dh0;
  p.T = T;
  p.B = B;
  p.H = H;
  p.nb = nb;
  hipLaunchKernelGGL(fn, dim3((unsigned)nb, (unsigned)((B + rows - 1) / rows)), dim3(threads), 0, stream, p);
  GS_CHECK_HIP(hipGetLastError());

  // 4. dgi, dbh, and dgh = (dg_r, dg_z, dgh_n) written over the coefficients in cg
  SumJob dbh_sum;  // run with the dW split sums below, in one launch
  rc = launch_grad(a, dsum, cg, cgn, nullptr, cg, chunks, stream, who, &dbh_sum);
  if (rc) return rc;

  // 5. dW[z][j][k] = sum_m dgh[m][z bs + j] hq[m][n bs + k], z = g nb + n: one
  //    batched product over the three gates (H = nb bs, so gate g block n sits
  //    at column z bs of dgh)
  const int64_t wsize = (int64_t)3 * nb * bs * bs;
  float* dst = pl.split > 1 ? part : a->dw_part;
  GemmArgs g3;
  g3.a = cg;  // A(j, m) = dgh[m][z bs + j]
  g3.lda = 3 * H;
  g3.a_bs = bs;
  g3.a_mod = 3 * nb;
  g3.b = hq;  // B(m, k) = hq[m][n bs + k]
  g3.ldb = H;
  g3.b_bs = bs;
  g3.b_mod = nb;
  g3.c = dst;
  g3.ldc = bs;
  g3.c_bs = (int64_t)bs * bs;
  g3.split_stride = wsize;
  g3.M = bs;
  g3.N = bs;
  g3.K = TB;
  g3.ksplit = pl.split;
  g3.batch = 3 * nb;
  g3.layout = kGemmTN;
  rc = gemm_f32(g3, stream, who);
  if (rc) return rc;
  if (pl.split > 1) return sum_partials2(dbh_sum, SumJob{a->dw_part, part, wsize, pl.split, wsize}, stream, who);
  return sum_partials(dbh_sum.dst, dbh_sum.src, dbh_sum.n, dbh_sum.parts, dbh_sum.stride, stream, who);
}
