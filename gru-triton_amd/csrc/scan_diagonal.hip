// Diagonal-hidden GRU scan forward (gfx950).
//
// Reference: LarocheC/gru-triton src/gru_qat/triton_kernels/scan_diagonal.py:127-223
// (kernel) and :226-282 (launcher); math of the PyTorch oracle :79-124.
//
// gh_g = w_g * q_in(h) + b_g is elementwise, so every (b, j) lane is an
// independent scalar GRU: one thread owns one lane for all T steps and keeps h
// in a register. There is no cross-thread traffic at all. The step chain is
// latency bound (a few dozen dependent VALU ops), so the kernel's job is to
// keep HBM latency off that chain: gi for the next kDepth steps is always in
// flight while the current kDepth steps compute, and out[t] stores are
// fire-and-forget. Loads of gi[t, b, g*H + j] for consecutive threads are
// consecutive floats, so each wave reads 256 contiguous bytes per gate.
#include "gs_host.h"

namespace gs {
namespace {

// Forward launch shape (measured at T=64, B=32, H=512: 64-thread workgroups
// put the B H lanes on every CU instead of a quarter of them, and 16 steps in
// flight hide the loads; 16.3 -> 13.6 us per launch against 256 x 8).
constexpr int kDepth = 16;   // steps of gi prefetched ahead
constexpr int kThreads = 64;
// Backward launch shape.
constexpr int kBwdDepth = 8;
constexpr int kBwdThreads = 64;

struct DiagParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* bh;
  float* out;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  Quant qin, qout;
};

// QIN: 0 no q_in, 1 q_in on h0 only (q_in == q_out, so the carried state is
// already on q_in's grid), 2 q_in every step. QOUT: q_out on. The modes are
// template arguments so that the step holds no branch and no per-step test.
// BUF: gi and out through raw buffer offsets (their extents fit 32 bits).
template <int QIN, bool QOUT, bool BUF>
__global__ __launch_bounds__(kThreads) void diagonal_fwd_kernel(DiagParams p) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= (int64_t)p.B * p.H) return;
  const int b = (int)(e / p.H);
  const int j = (int)(e - (int64_t)b * p.H);
  const int H = p.H;

  // Weights and biases pre-scaled for gru_update_l2: the r and z arguments are
  // fma(-log2e w, hq, -log2e (gi + b)), gh_n's is fma(2 log2e w_n, hq, 2 log2e b_n).
  constexpr float kR = -kLog2e, kN = 2.0f * kLog2e;
  const float wr = kR * p.w[j], wz = kR * p.w[H + j], wn = kN * p.w[2 * H + j];
  const float br = kR * p.bh[j], bz = kR * p.bh[H + j], bn = kN * p.bh[2 * H + j];
  float h = p.h0[(int64_t)b * p.sh0_b + j];
  float hq = QIN ? fake_quant(h, p.qin) : h;  // the matmul-side state of the next step

  const float* gib = p.gi + (int64_t)b * p.sg_b + j;
  float* outb = p.out + (int64_t)b * p.so_b + j;
  const auto grs = raw_rsrc(p.gi), ors = raw_rsrc(p.out);
  const uint32_t gl = (uint32_t)(((int64_t)b * p.sg_b + j) * 4), ol = (uint32_t)(((int64_t)b * p.so_b + j) * 4);
  const uint32_t gt4 = (uint32_t)(p.sg_t * 4), ot4 = (uint32_t)(p.so_t * 4);

  // Two register sets of gi take turns: while one set's kDepth steps compute,
  // the other set's loads are in flight. Loads past T are clamped to T - 1 and
  // never branched around, so the compiler's wait before step i counts only
  // the loads issued before that step's own (a conditional or copied prefetch
  // made it wait for the whole next chunk at the first step of each chunk).
  const int tl = p.T - 1;
  auto load = [&](int t0, float* r, float* z, float* c) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      if constexpr (BUF) {
        const uint32_t so = (uint32_t)min(t0 + i, tl) * gt4;
        r[i] = buf_ld(grs, gl, so);
        z[i] = buf_ld(grs, gl + 4u * H, so);
        c[i] = buf_ld(grs, gl + 8u * H, so);
      } else {
        const float* g = gib + (int64_t)min(t0 + i, tl) * p.sg_t;
        r[i] = g[0];
        z[i] = g[H];
        c[i] = g[2 * H];
      }
    }
  };
  // Runs steps t0 .. t0 + kDepth - 1; true once step T - 1 is done.
  auto run = [&](int t0, const float* r, const float* z, const float* c) -> bool {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const int t = t0 + i;
      if (t >= p.T) return true;
      const float ar = __builtin_fmaf(wr, hq, __builtin_fmaf(kR, r[i], br));
      const float az = __builtin_fmaf(wz, hq, __builtin_fmaf(kR, z[i], bz));
      const float gn2 = __builtin_fmaf(wn, hq, bn);
      float hn = gru_update_l2(ar, az, gn2, kN * c[i], h);
      if constexpr (QOUT) hn = fake_quant(hn, p.qout);
      if constexpr (BUF)
        buf_st(ors, ol, (uint32_t)t * ot4, hn);
      else
        outb[(int64_t)t * p.so_t] = hn;
      h = hn;
      hq = QIN == 2 ? fake_quant(hn, p.qin) : hn;
    }
    return t0 + kDepth >= p.T;
  };

  float ar[kDepth], az[kDepth], an[kDepth];
  float xr[kDepth], xz[kDepth], xn[kDepth];
  load(0, ar, az, an);
  for (int t0 = 0;; t0 += 2 * kDepth) {
    load(t0 + kDepth, xr, xz, xn);
    if (run(t0, ar, az, an)) return;
    load(t0 + 2 * kDepth, ar, az, an);
    if (run(t0 + kDepth, xr, xz, xn)) return;
  }
}

template <bool BUF>
void (*pick_fwd(int qin, bool qout))(DiagParams) {
  if (qout)
    return qin == 0 ? diagonal_fwd_kernel<0, true, BUF>
                    : qin == 1 ? diagonal_fwd_kernel<1, true, BUF> : diagonal_fwd_kernel<2, true, BUF>;
  return qin == 0 ? diagonal_fwd_kernel<0, false, BUF> : diagonal_fwd_kernel<2, false, BUF>;
}

// ---- backward ---------------------------------------------------------------------
// Reference: scan_diagonal.py:285-561 (Triton backward kernel and launcher) and
// its PyTorch restatement :564-647. Every (b, j) lane is again independent: one
// thread walks t from T-1 to 0 carrying dh in a register, recomputes the
// gates from h_{t-1} = out[t-1] (h0 at t = 0) with the forward's arithmetic,
// and accumulates its lane's contribution to dWh_diag and dbh in registers;
// the per-row partials go to dw_part / dbh_part at the end. gi, out[t-1] and
// dout[t] of the next kBwdDepth steps (in reverse) are in flight while the
// current kBwdDepth steps compute.
struct DiagBwdParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* bh;
  const float* out;
  const float* dout;
  float* dgi;
  float* dh0;
  float* dw_part;
  float* dbh_part;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  Quant qin, qout;
};

// QIN / QOUT: the quantizers are on (template arguments, so the step holds no
// branch on them). BUF: the per-step tensors through raw buffer offsets.
template <bool QIN, bool QOUT, bool BUF>
__global__ __launch_bounds__(kBwdThreads) void diagonal_bwd_kernel(DiagBwdParams p) {
  const int64_t e = (int64_t)blockIdx.x * kBwdThreads + threadIdx.x;
  if (e >= (int64_t)p.B * p.H) return;
  const int b = (int)(e / p.H);
  const int j = (int)(e - (int64_t)b * p.H);
  const int H = p.H;

  const float wr = p.w[j], wz = p.w[H + j], wn = p.w[2 * H + j];
  const float br = p.bh[j], bz = p.bh[H + j], bn = p.bh[2 * H + j];
  const float h0 = p.h0[(int64_t)b * p.sh0_b + j];

  const float* gib = p.gi + (int64_t)b * p.sg_b + j;
  const float* outb = p.out + (int64_t)b * p.so_b + j;
  const float* doutb = p.dout + ((int64_t)b * H + j);
  float* dgib = p.dgi + ((int64_t)b * 3 * H + j);
  const int64_t sd_t = (int64_t)p.B * H, sdg_t = (int64_t)p.B * 3 * H;
  const auto grs = raw_rsrc(p.gi), ors = raw_rsrc(p.out), drs = raw_rsrc(p.dout), dgrs = raw_rsrc(p.dgi);
  const uint32_t gl = (uint32_t)(((int64_t)b * p.sg_b + j) * 4), ol = (uint32_t)(((int64_t)b * p.so_b + j) * 4);
  const uint32_t dl = (uint32_t)(((int64_t)b * H + j) * 4), dgl = (uint32_t)(((int64_t)b * 3 * H + j) * 4);
  const uint32_t gt4 = (uint32_t)(p.sg_t * 4), ot4 = (uint32_t)(p.so_t * 4), dt4 = (uint32_t)(sd_t * 4),
                 dgt4 = (uint32_t)(sdg_t * 4);
  Quant qin = p.qin, qout = p.qout;
  qin.on = QIN;
  qout.on = QOUT;

  // Step i of a chunk is t = t0 - i; its loads are gi[t], out[t-1] and
  // dout[t], with t clamped to 0 (out[-1] is h0, selected at compute time). As
  // in the forward, two register sets take turns and no load is branched
  // around, so the wait before a step counts only the loads issued before its
  // own.
  auto load = [&](int t0, float* gr, float* gz, float* gn, float* hp, float* dd) {
#pragma unroll
    for (int i = 0; i < kBwdDepth; ++i) {
      const int t = max(t0 - i, 0);
      if constexpr (BUF) {
        const uint32_t so = (uint32_t)t * gt4;
        gr[i] = buf_ld(grs, gl, so);
        gz[i] = buf_ld(grs, gl + 4u * H, so);
        gn[i] = buf_ld(grs, gl + 8u * H, so);
        hp[i] = buf_ld(ors, ol, (uint32_t)max(t - 1, 0) * ot4);
        dd[i] = buf_ld(drs, dl, (uint32_t)t * dt4);
      } else {
        const float* g = gib + (int64_t)t * p.sg_t;
        gr[i] = g[0];
        gz[i] = g[H];
        gn[i] = g[2 * H];
        hp[i] = outb[(int64_t)max(t - 1, 0) * p.so_t];
        dd[i] = doutb[(int64_t)t * sd_t];
      }
    }
  };

  float dh = 0.0f;
  float dwr = 0.f, dwz = 0.f, dwn = 0.f, dbr = 0.f, dbz = 0.f, dbn = 0.f;
  // Runs steps t0 down to t0 - kBwdDepth + 1; true once step 0 is done.
  auto run = [&](int t0, const float* cr, const float* cz, const float* cn, const float* ch,
                 const float* cd) -> bool {
#pragma unroll
    for (int i = 0; i < kBwdDepth; ++i) {
      const int t = t0 - i;
      if (t < 0) return true;
      const float h_prev = t > 0 ? ch[i] : h0;
      float hq = h_prev;
      bool keep_in = true;
      if constexpr (QIN) {
        keep_in = quant_keeps(h_prev, qin);
        hq = fake_quant(h_prev, qin);
      }
      const float ghr = mul_add_nofma(wr, hq, br);
      const float ghz = mul_add_nofma(wz, hq, bz);
      const float ghn = mul_add_nofma(wn, hq, bn);
      const GateGrad gg = gru_backward(cr[i], cz[i], cn[i], ghr, ghz, ghn, h_prev, cd[i] + dh, qout);
      if constexpr (BUF) {
        const uint32_t so = (uint32_t)t * dgt4;
        buf_st(dgrs, dgl, so, gg.dgr);
        buf_st(dgrs, dgl + 4u * H, so, gg.dgz);
        buf_st(dgrs, dgl + 8u * H, so, gg.dgn);
      } else {
        float* dg = dgib + (int64_t)t * sdg_t;
        dg[0] = gg.dgr;
        dg[H] = gg.dgz;
        dg[2 * H] = gg.dgn;
      }
      {
#pragma clang fp contract(off)
        float via = gg.dgr * wr + gg.dgz * wz + gg.dghn * wn;
        if (!keep_in) via = 0.0f;
        dh = gg.dh_direct + via;
        dwr += gg.dgr * hq;
        dwz += gg.dgz * hq;
        dwn += gg.dghn * hq;
        dbr += gg.dgr;
        dbz += gg.dgz;
        dbn += gg.dghn;
      }
    }
    return t0 - kBwdDepth < 0;
  };

  float ar[kBwdDepth], az[kBwdDepth], an[kBwdDepth], ah[kBwdDepth], ad[kBwdDepth];
  float xr[kBwdDepth], xz[kBwdDepth], xn[kBwdDepth], xh[kBwdDepth], xd[kBwdDepth];
  load(p.T - 1, ar, az, an, ah, ad);
  for (int t0 = p.T - 1;; t0 -= 2 * kBwdDepth) {
    load(t0 - kBwdDepth, xr, xz, xn, xh, xd);
    if (run(t0, ar, az, an, ah, ad)) break;
    load(t0 - 2 * kBwdDepth, ar, az, an, ah, ad);
    if (run(t0 - kBwdDepth, xr, xz, xn, xh, xd)) break;
  }
  p.dh0[(int64_t)b * H + j] = dh;
  float* dwp = p.dw_part + (int64_t)b * 3 * H + j;
  dwp[0] = dwr;
  dwp[H] = dwz;
  dwp[2 * H] = dwn;
  float* dbp = p.dbh_part + (int64_t)b * 3 * H + j;
  dbp[0] = dbr;
  dbp[H] = dbz;
  dbp[2 * H] = dbn;
}

typedef void (*DiagBwdFn)(DiagBwdParams);

template <bool BUF>
DiagBwdFn pick_bwd_buf(bool qin, bool qout) {
  return qin ? (qout ? diagonal_bwd_kernel<true, true, BUF> : diagonal_bwd_kernel<true, false, BUF>)
             : (qout ? diagonal_bwd_kernel<false, true, BUF> : diagonal_bwd_kernel<false, false, BUF>);
}

DiagBwdFn pick_bwd(bool qin, bool qout, bool buf) {
  return buf ? pick_bwd_buf<true>(qin, qout) : pick_bwd_buf<false>(qin, qout);
}

}  // namespace
}  // namespace gs

extern "C" int gs_diagonal_bwd(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_diagonal_bwd";
  int rc = validate_bwd_common(a, who);
  if (rc) return rc;
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the diagonal kind", who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);

  DiagBwdParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.bh = a->bh;
  p.out = a->out;
  p.dout = a->dout;
  p.dgi = a->dgi;
  p.dh0 = a->dh0;
  p.dw_part = a->dw_part;
  p.dbh_part = a->dbh_part;
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);

  const int64_t n = a->B * a->H;
  const dim3 grid((unsigned)((n + kBwdThreads - 1) / kBwdThreads));
  // dout and dgi are dense [T, B, H] and [T, B, 3H]
  const bool buf = fits_buf32(a->T, a->sg_t, a->B, a->sg_b, 3 * a->H) &&
                   fits_buf32(a->T, a->so_t, a->B, a->so_b, a->H) && fits_buf32(a->T, a->B * a->H, a->B, a->H, a->H) &&
                   fits_buf32(a->T, a->B * 3 * a->H, a->B, 3 * a->H, 3 * a->H);
  hipLaunchKernelGGL(pick_bwd(a->q_in.enabled != 0, a->q_out.enabled != 0, buf), grid, dim3(kBwdThreads), 0, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

extern "C" int gs_diagonal_fwd(const gs_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_diagonal_fwd";
  int rc = validate_common(a, who);
  if (rc) return rc;
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the diagonal kind", who);

  DiagParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.bh = a->bh;
  p.out = a->out;
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);

  const int64_t n = a->B * a->H;
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
  const int qin = !a->q_in.enabled ? 0 : same_quant(a->q_in, a->q_out) ? 1 : 2;
  const bool buf = fits_buf32(a->T, a->sg_t, a->B, a->sg_b, 3 * a->H) && fits_buf32(a->T, a->so_t, a->B, a->so_b, a->H);
  void (*fn)(DiagParams) = buf ? pick_fwd<true>(qin, a->q_out.enabled != 0) : pick_fwd<false>(qin, a->q_out.enabled != 0);
  hipLaunchKernelGGL(fn, grid, dim3(kThreads), 0, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}
