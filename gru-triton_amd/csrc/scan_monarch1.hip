// Single-factor Monarch GRU scan forward for blksz in {16, 32, 64, 128} (gfx950).
//
// Reference: LarocheC/gru-triton src/gru_qat/triton_kernels/scan_monarch.py:130-291
// (kernel), :320-406 (launcher), math of the PyTorch form :74-127:
//   gh[b, g, n, o] = sum_i q_in(h)[b, n bs + i] W[g, n, o, i] + bh[g H + n bs + o]
// then the GRU gates (gru_cell.py:437-464).
//
// Blocks never mix (scan_monarch.py:204-208), so block n of batch row b is a
// recurrence of its own over bs units: one workgroup per (block, batch rows)
// runs it for all T steps with the state in LDS and no traffic between
// workgroups. Four adjacent lanes share unit u: each holds a quarter of row u
// of W[g][n] for the three gates in VGPRs, dots it with its quarter of
// q_in(h_{t-1}) (float4 LDS broadcasts), the quad sums the quarters with DPP,
// and every lane of the quad then runs the same gate epilogue; lane 0 stores
// out[t] and writes q_in(h_t) for the next step, and an LDS-only barrier ends
// the step. gi for the next kDepth steps is in flight while the current
// kDepth steps compute. Against the MFMA kernel of scan_dense.hip (one
// workgroup per block and 4 batch rows, gi loaded inside the step) this puts
// B nb workgroups on the device instead of B nb / 4, and keeps gi's load
// latency off the step.
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kSK = 4;     // lanes per unit
constexpr int kDepth = 8;  // steps of gi loaded ahead

template <int BS>
constexpr int rows_per_wg() {
  return kSK * BS >= 256 ? 1 : 256 / (kSK * BS);
}

template <int BS>
constexpr int m1f_threads() {
  return kSK * BS * rows_per_wg<BS>();
}

struct M1FParams {
  const float* gi;
  const float* h0;
  const float* w;   // [3, nb, bs, bs] (out, in)
  const float* bh;  // [3H]
  float* out;
  float* gh_save;  // SAVE instances: [T, B, 3H] q_in(h_{t-1}) W^T per block (no bias)
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H, nb;
  Quant qin, qout;
};

// QIN: 0 no q_in, 1 q_in on h0 only (q_in == q_out, so the carried state is
// already on q_in's grid), 2 q_in every step. QOUT: q_out on. Template
// arguments, so that the step holds no branch on them. SAVE: also store gh.
template <int BS, int QIN, bool QOUT, bool SAVE = false>
__global__ __launch_bounds__(m1f_threads<BS>()) void monarch1_fwd_kernel(M1FParams p) {
  constexpr int TPR = kSK * BS;
  constexpr int R = rows_per_wg<BS>();
  constexpr int KT = BS / kSK;  // terms per gate and thread
  static_assert(KT % 4 == 0, "terms per thread must be whole float4s");
  __shared__ __attribute__((aligned(16))) float hs[2][R][BS];  // q_in(h) of the step

  const int n = blockIdx.x;
  const int rs = threadIdx.x / TPR, lt = threadIdx.x - rs * TPR;
  const int u = lt / kSK, kq = lt % kSK;
  const int b = blockIdx.y * R + rs;
  const bool live = b < p.B;
  const int H = p.H, T = p.T;
  const int col = n * BS + u;

  float wr[3][KT];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const float* row = p.w + (((int64_t)g * p.nb + n) * BS + u) * BS + kq * KT;
#pragma unroll
    for (int i = 0; i < KT; ++i) wr[g][i] = row[i];
  }
  // Biases pre-scaled for gru_update_l2 (-log2e for r and z, 2 log2e for n).
  constexpr float kR = -kLog2e, kN = 2.0f * kLog2e;
  const float br = kR * p.bh[col], bz = kR * p.bh[H + col], bn = kN * p.bh[2 * H + col];
  float h = live ? p.h0[(int64_t)b * p.sh0_b + col] : 0.0f;
  if (kq == 0) hs[0][rs][u] = QIN ? fake_quant(h, p.qin) : h;

  // Rows past B read row 0 and never store; loads past T are clamped to
  // T - 1. Two register sets of gi take turns (one set's kDepth steps compute
  // while the other's loads are in flight) and no load is branched around, so
  // the wait before step i counts only the loads issued before its own.
  const float* gib = p.gi + (int64_t)(live ? b : 0) * p.sg_b + col;
  float* outb = p.out + (int64_t)(live ? b : 0) * p.so_b + col;
  const int tl = T - 1;
  auto load = [&](int t0, float* r, float* z, float* c) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const float* g = gib + (int64_t)min(t0 + i, tl) * p.sg_t;
      r[i] = g[0];
      z[i] = g[H];
      c[i] = g[2 * H];
    }
  };
  int buf = 0;
  // Runs steps t0 .. t0 + kDepth - 1; true once step T - 1 is done.
  auto run = [&](int t0, const float* cr, const float* cz, const float* cn) -> bool {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const int t = t0 + i;
      if (t >= T) return true;
      const float* src = &hs[buf][rs][kq * KT];
      f4 a[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) a[g] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < KT; q += 4) {
        const f4 v = *reinterpret_cast<const f4*>(src + q);
#pragma unroll
        for (int g = 0; g < 3; ++g)
#pragma unroll
          for (int c = 0; c < 4; ++c) a[g][c] += v[c] * wr[g][q + c];
      }
      float gh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        float s = (a[g][0] + a[g][1]) + (a[g][2] + a[g][3]);
        s += lane_xor_c<1>(s);
        s += lane_xor_c<2>(s);
        gh[g] = s;
      }
      const float ar = __builtin_fmaf(kR, gh[0], __builtin_fmaf(kR, cr[i], br));
      const float az = __builtin_fmaf(kR, gh[1], __builtin_fmaf(kR, cz[i], bz));
      const float gn2 = __builtin_fmaf(kN, gh[2], bn);
      float hn = gru_update_l2(ar, az, gn2, kN * cn[i], h);
      if constexpr (QOUT) hn = fake_quant(hn, p.qout);
      if (kq == 0) hs[buf ^ 1][rs][u] = QIN == 2 ? fake_quant(hn, p.qin) : hn;
      if (live && kq == 0) outb[(int64_t)t * p.so_t] = hn;
      if constexpr (SAVE) {
        // the unit's four lanes hold the same sums: lane kq < 3 stores gate kq; issued
        // after the LDS write, off the gates' critical path, and non-temporal (read once, by
        // the backward)
        if (live && kq < 3)
          __builtin_nontemporal_store(kq == 0 ? gh[0] : kq == 1 ? gh[1] : gh[2], &p.gh_save[((int64_t)t * p.B + b) * 3 * H + kq * H + col]);
      }
      h = hn;
      lds_barrier();  // LDS only: the out stores need not complete here
      buf ^= 1;
    }
    return t0 + kDepth >= T;
  };

  float ar[kDepth], az[kDepth], an[kDepth];
  float xr[kDepth], xz[kDepth], xn[kDepth];
  load(0, ar, az, an);
  __syncthreads();
  for (int t0 = 0;; t0 += 2 * kDepth) {
    load(t0 + kDepth, xr, xz, xn);
    if (run(t0, ar, az, an)) return;
    load(t0 + 2 * kDepth, ar, az, an);
    if (run(t0 + kDepth, xr, xz, xn)) return;
  }
}

typedef void (*M1FFn)(M1FParams);

template <int BS, bool SAVE>
M1FFn pick_modes(int qin, bool qout) {
  if (qout)
    return qin == 0   ? monarch1_fwd_kernel<BS, 0, true, SAVE>
           : qin == 1 ? monarch1_fwd_kernel<BS, 1, true, SAVE>
                      : monarch1_fwd_kernel<BS, 2, true, SAVE>;
  return qin == 0 ? monarch1_fwd_kernel<BS, 0, false, SAVE> : monarch1_fwd_kernel<BS, 2, false, SAVE>;
}

template <int BS>
M1FFn pick_save(int qin, bool qout, bool save) {
  return save ? pick_modes<BS, true>(qin, qout) : pick_modes<BS, false>(qin, qout);
}

// qin: 0 off, 1 on h0 only, 2 every step (see monarch1_fwd_kernel); save: the
// training instance that also stores gh
M1FFn pick(int bs, int qin, bool qout, int* threads, int* rows, bool save = false) {
  switch (bs) {
    case 16: *rows = rows_per_wg<16>(); *threads = m1f_threads<16>(); return pick_save<16>(qin, qout, save);
    case 32: *rows = rows_per_wg<32>(); *threads = m1f_threads<32>(); return pick_save<32>(qin, qout, save);
    case 64: *rows = rows_per_wg<64>(); *threads = m1f_threads<64>(); return pick_save<64>(qin, qout, save);
    case 128: *rows = rows_per_wg<128>(); *threads = m1f_threads<128>(); return pick_save<128>(qin, qout, save);
    default: return nullptr;
  }
}

}  // namespace

// True when the single-factor Monarch forward of `a` runs here (blksz 16, 32,
// 64 or 128 tiling H); it then needs no workspace.
bool monarch1_local_ok(const gs_args* a) {
  int th = 0, rows = 0;
  return a->w2 == nullptr && a->nblocks >= 1 && a->blksz >= 1 && a->nblocks * a->blksz == a->H &&
         pick((int)a->blksz, 0, false, &th, &rows) != nullptr && a->nblocks <= 65535 &&
         (a->B + rows - 1) / rows <= 65535;
}

int run_monarch1_local(const gs_args* a, hipStream_t stream) {
  int threads = 0, rows = 0;
  const int qin = !a->q_in.enabled ? 0 : same_quant(a->q_in, a->q_out) ? 1 : 2;
  M1FFn fn = pick((int)a->blksz, qin, a->q_out.enabled != 0, &threads, &rows, a->gh_save != nullptr);
  M1FParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.bh = a->bh;
  p.out = a->out;
  p.gh_save = a->gh_save;
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.nb = (int)a->nblocks;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  hipLaunchKernelGGL(fn, dim3((unsigned)p.nb, (unsigned)((p.B + rows - 1) / rows)), dim3(threads), 0, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace gs
