// Dense GRU scan backward (gfx950): a linear reverse recurrence on fp32 MFMA,
// framed by parallel passes and two GEMMs.
//
// Reference: gru_scan_backward_persistent and its kernel
// (LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py:646-752, :296-643),
// whose math is the PyTorch backward at scan.py:1460-1550. Per step t, walking
// t from T-1 to 0 with h_{t-1} = out[t-1] (h0 at t = 0), D_t = dout[t] + the
// carry from step t+1 is the gradient reaching h_t, and the step's gradients
// (gru_backward) are linear in D_t with coefficients fixed by the forward:
//   (dgr, dgz, dgn, dgh_n, dh_direct) = D_t * (Cr, Cz, Cgn, Chn, Zm)_t
// (q_out's clipped-STE mask is folded into the coefficients), dgh_t =
// (dgr, dgz, dgh_n), and
//   D_{t-1} = dout[t-1] + Zm_t D_t + Mi_t (dgh_t Wh),   Mi_t = q_in's mask on h_{t-1}
//   dh0 = Zm_0 D_0 + Mi_0 (dgh_0 Wh)
//   dWh = sum_t dgh_t^T q_in(h_{t-1}),  dbh = sum_t sum_b dgh_t
// Only D_t sits on the recurrence. The launcher runs
//   0. hq = q_in([h0; out[0..T-2]]) as one [T B, H] block;
//   1. gemm: gh = hq Wh^T + bh for every step at once;
//   2. coef_kernel: the coefficient planes from gi, gh and h_{t-1}
//      (Cr, Cz, Chn overwrite gh in place; Cgn, Zm, Mi in planes of their own);
//   3. dense_bwd_kernel: the recurrence, writing D_t for every t and dh0;
//   4. grad_kernel: dgi, dgh_n and per-row dbh sums from D and the planes;
//   5. gemm: dWh = dgh^T hq, K split over T B, then a sum.
//
// The recurrence kernel has the forward's shape (scan_dense.hip) with the
// reduction over 3H: the exchanged vector is D_t (H tagged words per batch
// row, as the forward exchanges h) and each compute wave owns a quad of units
// u of D_{t-1}, holding the Wh columns of those units over all 3H rows in
// VGPRs (wt[g][m] = Wh[g H + kmap(m)][u]). The poller waves poll D_t, scale
// it by the step's coefficients (prefetched while the compute waves work) and
// stage dgh_t = D_t (Cr, Cz, Chn) into LDS; a compute wave runs one MFMA chain
// over the three staged segments, reduces the K slices, and the 16 lanes of
// row 0 form D_{t-1} and publish it.
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

// Poller waves per batch row of the recurrence: two at KC 16 and 32 (each
// polls half of the row's D words), one otherwise.
__host__ __device__ constexpr int bwd_pollers_per_row(int KC) { return KC == 16 || KC == 32 ? 2 : 1; }
// Per-unit values staged for the iteration that consumes D_t: 0 Zm_t, 1 Mi_t, 2 dout[t-1]
constexpr int kNV = 3;

// ---- parallel passes ---------------------------------------------------------------

// For every (t, b, k): gradients of step t per unit D_t (gru_backward with
// dh = 1) from gh [T B, 3H] (plus bh [3H] when bh is non-NULL: gh then holds
// the bias-free product the forward saved); writes (Cr, Cz, Chn) to cg
// [T B, 3H], which may be gh itself (each thread reads its three gh values
// before it writes the same three positions). hq (NULL: not written): also
// writes q_in(h_{t-1}) [T B, H], as build_prev_state does, from the h_{t-1}
// the thread reads anyway.
__global__ void coef_kernel(const float* gi, int64_t sg_t, int64_t sg_b, const float* h0, int64_t sh0_b,
                            const float* out, int64_t so_t, int64_t so_b, const float* gh, const float* bh,
                            float* cg, float* cgn, float* zm, float* mi, float* hq, int T, int B, int H,
                            Quant qin, Quant qout) {
  const int64_t n = (int64_t)T * B * H;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / H;
    const int k = (int)(e - m * H);
    const int t = (int)(m / B), b = (int)(m - (int64_t)t * B);
    const float* g = gi + (int64_t)t * sg_t + (int64_t)b * sg_b + k;
    const float* h = gh + m * 3 * H + k;
    float* c = cg + m * 3 * H + k;
    const float hp = t > 0 ? out[(int64_t)(t - 1) * so_t + (int64_t)b * so_b + k] : h0[(int64_t)b * sh0_b + k];
    float ghr = h[0], ghz = h[H], ghn = h[2 * H];
    if (bh != nullptr) {
      ghr += bh[k];
      ghz += bh[H + k];
      ghn += bh[2 * H + k];
    }
    const GateGrad gg = gru_backward(g[0], g[H], g[2 * H], ghr, ghz, ghn, hp, 1.0f, qout);
    c[0] = gg.dgr;
    c[H] = gg.dgz;
    c[2 * H] = gg.dghn;
    cgn[e] = gg.dgn;
    zm[e] = gg.dh_direct;
    mi[e] = (qin.on && !quant_keeps(hp, qin)) ? 0.0f : 1.0f;
    if (hq != nullptr) hq[e] = qin.on ? fake_quant(hp, qin) : hp;
  }
}

// dgi, dgh_n and per-row partial dbh sums over chunks of kGradSteps steps:
// thread (chunk, b, k) walks the chunk's steps t. Optional outputs (NULL: not
// written): dghn [T B, H], and dgh [T B, 3H] = (dg_r, dg_z, dgh_n), the A
// operand of the one dWh product; dgh may be cg itself, since each thread
// reads its three coefficients before it writes the same three positions.
constexpr int kGradSteps = 8;
__global__ void grad_kernel(const float* dsum, const float* cg, const float* cgn, float* dgi, float* dghn,
                            float* dgh, float* dbh_chunks, int T, int B, int H) {
  const int64_t per_chunk = (int64_t)B * H;
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int nchunks = (T + kGradSteps - 1) / kGradSteps;
  if (e >= per_chunk * nchunks) return;
  const int chunk = (int)(e / per_chunk);
  const int64_t bk = e - chunk * per_chunk;
  const int b = (int)(bk / H), k = (int)(bk - (int64_t)b * H);
  float sr = 0.f, sz = 0.f, sn = 0.f;
  const int t1 = min(T, (chunk + 1) * kGradSteps);
  for (int t = chunk * kGradSteps; t < t1; ++t) {
    const int64_t m = (int64_t)t * B + b;
    const float D = dsum[m * H + k];
    const float* c = cg + m * 3 * H + k;
    float* d = dgi + m * 3 * H + k;
    const float gr = D * c[0], gz = D * c[H], ghn = D * c[2 * H];
    d[0] = gr;
    d[H] = gz;
    d[2 * H] = D * cgn[m * H + k];
    if (dghn != nullptr) dghn[m * H + k] = ghn;
    if (dgh != nullptr) {
      float* o = dgh + m * 3 * H + k;
      o[0] = gr;
      o[H] = gz;
      o[2 * H] = ghn;
    }
    sr += gr;
    sz += gz;
    sn += ghn;
  }
  float* o = dbh_chunks + ((int64_t)chunk * B + b) * 3 * H + k;
  o[0] = sr;
  o[H] = sz;
  o[2 * H] = sn;
}

// ---- the recurrence ----------------------------------------------------------------

struct BParams {
  const float* w;
  const float* dout;  // [T, B, H] contiguous
  const float* cg;    // [T, B, 3H] (Cr, Cz, Chn)
  const float* zm;    // [T, B, H]
  const float* mi;    // [T, B, H]
  float* dsum;        // [T, B, H] D_t
  float* dh0;         // [B, H] contiguous
  uint64_t* xh;       // [2][Bp][H] tagged D_t
  uint64_t* xw;       // [nwg] tagged XCD ids
  Ctrl ctrl;
  int T, B, H;
  int ngroups, RB, nrb, Bp, nwg, P, nwc, hsz;
};

template <int KC>
__device__ __forceinline__ void load_wt(const float* w, int H, int o0, int j, int kb4, bool ok_q,
                                        float (&wt)[3][KC]) {
  const int u = o0 + j;
  const bool ok = ok_q && u < H;
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int m = 0; m < KC; ++m) {
      const int k = kmap(m, kb4);
      wt[g][m] = (ok && k < H) ? w[(int64_t)(g * H + k) * H + u] : 0.0f;
    }
}

template <int KC, int NT>
__global__ __launch_bounds__(NT) void dense_bwd_kernel(BParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwc = p.nwc;
  const bool poller = wave >= nwc;
  const int j = lane & 3, kb4 = lane >> 2, s = (lane >> 2) & 3;
  const bool lead = lane < 16;
  const int H = p.H, T = p.T;

  const int gid = blockIdx.x % p.ngroups;
  const int pw = blockIdx.x / p.ngroups;
  const int o0 = 4 * (pw * nwc + wave);
  const bool quad_ok = !poller && o0 < H;
  const int U = 4 * nwc;
  const int ulo = 4 * pw * nwc;
  const int unit = ulo + 4 * wave + j;
  const bool unit_ok = quad_ok && o0 + j < H;

  const int rb_begin = gid * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);
  const int nrbm = rb_end - rb_begin;

  float* hst = lds;                   // [2][3][hsz] staged dgh_t (il_index per gate block)
  float* sti = hst + 6 * p.hsz;       // [2][4][kNV][U] staged per-unit values
  float* dd = sti + 2 * 4 * kNV * U;  // [RB][4][U] D_t of this workgroup's units
  int* flags = reinterpret_cast<int*>(dd + p.RB * 4 * U);  // [0] compute-wave iterations published,
                                                          // [1] bit 0: group on one XCD, bit 1: a
                                                          // wait of this workgroup gave up
  // The compute waves' Wh columns are loaded first, so that the latency of
  // these strided loads overlaps the LDS clear and the prologue (6 us less
  // per launch at T=64, B=32, H=512).
  float wt[3][KC];
  if (!poller) load_wt<KC>(p.w, H, o0, j, kb4, quad_ok, wt);
  const int lds_floats = 6 * p.hsz + 8 * kNV * U + p.RB * 4 * U + 4;
  for (int i = threadIdx.x; i < lds_floats; i += blockDim.x) lds[i] = 0.0f;

  const uint32_t base = __hip_atomic_load(ctrl_tag_base(p.ctrl), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const Ctrl ctrl = launch_ctrl(p.ctrl, base);
  if (threadIdx.x == 0) st_tagged(p.xw + blockIdx.x, __uint_as_float(xcc_id()), base + 1u);
  const int niter = T * nrbm;
  const int64_t BH = (int64_t)p.B * H;

  // Staged value v of unit k of `row` for the iteration consuming D_t.
  auto step_value = [&](int t, int row, int k, int v) -> float {
    const int64_t e = (int64_t)t * BH + (int64_t)row * H + k;
    if (v == 0) return p.zm[e];
    if (v == 1) return p.mi[e];
    return t > 0 ? p.dout[e - BH] : 0.0f;
  };
  // First iteration of row-block nx: D_{T-1} = dout[T-1] needs no exchange.
  auto stage_first = [&](int nx, int r, int k) {
    const int row = 4 * (rb_begin + nx) + r;
    if (row >= p.B) return;
    const int64_t e = (int64_t)(T - 1) * BH + (int64_t)row * H + k;
    const float D = p.dout[e];
    const float* c = p.cg + ((int64_t)(T - 1) * p.B + row) * 3 * H + k;
    float* hs = hst + (nx & 1) * 3 * p.hsz + il_index(r, k);
    hs[0] = D * c[0];
    hs[p.hsz] = D * c[H];
    hs[2 * p.hsz] = D * c[2 * H];
    const int u = k - ulo;
    if (u >= 0 && u < U) {
      dd[(nx * 4 + r) * U + u] = D;
      p.dsum[e] = D;
    }
  };

  // Prologue (all waves): iteration 0's inputs.
  lds_barrier();
  for (int w = threadIdx.x; w < 4 * H; w += blockDim.x) stage_first(0, w / H, w % H);
  for (int w = threadIdx.x; w < 4 * kNV * U; w += blockDim.x) {
    const int r = w / (kNV * U), rem = w - r * kNV * U, v = rem / U, u = rem - v * U;
    const int row = 4 * rb_begin + r;
    sti[w] = (row < p.B && ulo + u < H) ? step_value(T - 1, row, ulo + u, v) : 0.0f;
  }
  lds_barrier();

  if (!poller) {
    const int uo = 4 * wave + j;
    for (int it = 0; it < niter; ++it) {
      const int st = it / nrbm;
      const int rbl = it - st * nrbm;
      const int buf = it & 1;
      const int row = 4 * (rb_begin + rbl) + s;
      const int t = T - 1 - st;
      f4 acc0 = f4{0.f, 0.f, 0.f, 0.f}, acc1 = f4{0.f, 0.f, 0.f, 0.f};
      static_for<0, 3>([&](auto G) {
        float a[KC];
        lds_a_il<KC>(hst + (buf * 3 + G) * p.hsz, lane, a);
#pragma unroll
        for (int m = 0; m < KC; m += 2) {
          acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[m], wt[G][m], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[m + 1], wt[G][m + 1], acc1, 0, 0, 0);
        }
      });
      const float via_w = reduce16(acc0 + acc1, s);
      // after a give-up the workgroup's D_t and dh0 are NaN and it publishes nothing more
      const int fl = __builtin_amdgcn_readfirstlane(flags[1]);
      const bool xcd_local = (fl & 1) != 0;
      const bool dead = (fl & 2) != 0;
      if (lead && unit_ok && row < p.B) {
        const float* sv = sti + (buf * 4 + s) * kNV * U + uo;
        float* ddp = dd + (rbl * 4 + s) * U + uo;
        float carry;
        {
#pragma clang fp contract(off)
          carry = sv[0] * *ddp + sv[U] * via_w;
        }
        if (t == 0) {
          p.dh0[(int64_t)row * H + unit] = dead ? __builtin_nanf("") : carry;
        } else {
          const float dn = sv[2 * U] + carry;  // D_{t-1}
          uint64_t* dst = p.xh + ((int64_t)(st & 1) * p.Bp + row) * H + unit;
          if (!dead) {
            if (xcd_local)
              st_tagged_xcd(dst, dn, base + (uint32_t)st + 1u);
            else
              st_tagged(dst, dn, base + (uint32_t)st + 1u);
          }
          p.dsum[(int64_t)(t - 1) * BH + (int64_t)row * H + unit] = dead ? __builtin_nanf("") : dn;
          *ddp = dn;
        }
      }
      if (lane == 0) __hip_atomic_fetch_add(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
    }
  } else {
    // Poller wave pr stages row pr of iteration it + 1 while the compute
    // waves run iteration it: per-unit values and the row's coefficients are
    // loaded first (their latency overlaps the poll), then D_t is polled once
    // this workgroup's compute waves have published iteration it, and dgh_t
    // = D_t (Cr, Cz, Chn) goes to LDS.
    constexpr int NPR = bwd_pollers_per_row(KC);
    static_assert(NT / 64 >= 4 * NPR + 1, "launch bounds hold the poller waves");
    const int pq = wave - nwc;
    const int pr = pq / NPR, part = pq - pr * NPR;
    constexpr int KW = 16 * KC / NPR;  // this wave's share of a row's words: k in [part KW, part KW + KW)
    constexpr int MPW = KW / 64;       // polled words per lane
    const int k0 = part * KW;
    constexpr int NWC_MAX = NT / 64 - 4 * NPR;
    constexpr int NSV = (kNV * 4 * NWC_MAX + 63) / 64;  // staged values per lane (part 0)
    for (int it = 0; it < niter; ++it) {
      const int nx = it + 1;
      if (nx < niter) {
        const int st2 = nx / nrbm;
        const int rbl2 = nx - st2 * nrbm;
        const int row = 4 * (rb_begin + rbl2) + pr;
        const int t2 = T - 1 - st2;
        float sv[NSV];
#pragma unroll
        for (int i = 0; i < NSV; ++i) {
          const int w = lane + 64 * i;
          const int v = w / U, u = w - v * U;
          sv[i] = (part == 0 && w < kNV * U && row < p.B && ulo + u < H) ? step_value(t2, row, ulo + u, v) : 0.0f;
        }
        if (st2 == 0) {
          for (int k = k0 + lane; k < min(H, k0 + KW); k += 64) stage_first(nx, pr, k);
        } else if (row < p.B) {
          const float* crow = p.cg + ((int64_t)t2 * p.B + row) * 3 * H + k0 + lane;
          float cf[3][MPW];
#pragma unroll
          for (int m = 0; m < MPW; ++m) {
            const bool ok = k0 + lane + 64 * m < H;
#pragma unroll
            for (int g = 0; g < 3; ++g) cf[g][m] = ok ? crow[g * H + 64 * m] : 0.0f;
          }
          if (pq == 0 && nx == nrbm &&  // first exchange of the launch
              p.P <= 64 && group_on_one_xcd(ctrl, p.xw + gid, p.ngroups, p.P, base + 1u, &flags[1]))
            __hip_atomic_fetch_or(&flags[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          wait_lds_count(ctrl, &flags[0], nwc * (it + 1), &flags[1]);
          uint64_t v[MPW];
          uint32_t valid = 0;
          if (k0 < H)
            valid = poll_row_words<MPW>(ctrl, p.xh + ((int64_t)((st2 - 1) & 1) * p.Bp + row) * H + k0, H - k0,
                                        base + (uint32_t)st2, v, &flags[1]);
          float* hs = hst + (nx & 1) * 3 * p.hsz;
          static_for<0, MPW>([&](auto I) {
            if ((valid >> I) & 1u) {
              const float D = value_of(v[I]);
              const int li = il_index(pr, k0 + lane + 64 * I);
              hs[li] = D * cf[0][I];
              hs[p.hsz + li] = D * cf[1][I];
              hs[2 * p.hsz + li] = D * cf[2][I];
            }
          });
        }
        float* sd = sti + ((nx & 1) * 4 + pr) * kNV * U;
        if (part == 0) {
#pragma unroll
          for (int i = 0; i < NSV; ++i) {
            const int w = lane + 64 * i;
            if (w < kNV * U) sd[w] = sv[i];
          }
        }
      }
      lds_barrier();
    }
  }
  leave_grid(ctrl, (uint32_t)p.nwg, base, (uint32_t)T, &flags[1], 2);
}

typedef void (*BFn)(BParams);

BFn pick_bwd(int KC, int* nt) {
  switch (KC) {
    case 4: *nt = 1024; return dense_bwd_kernel<4, 1024>;
    case 8: *nt = 1024; return dense_bwd_kernel<8, 1024>;
    case 16: *nt = 768; return dense_bwd_kernel<16, 768>;
    case 32: *nt = 768; return dense_bwd_kernel<32, 768>;
    case 64: *nt = 512; return dense_bwd_kernel<64, 512>;
    default: return nullptr;
  }
}

// Workspace (tagged words only): control words | xh [2][Bp][H] tagged D |
// xw [nrb P]. Scratch (plain floats), each region 256-byte aligned:
// cg [T B, 3H] | hq, cgn, zm, mi, dsum [T B, H] each |
// dbh chunks [nchunks][B][3H] | dWh split partials.
struct BPlan {
  bool tiled;  // the recurrence runs on the batch-tiled kernel (scan_tiled.hip)
  int KC, nt, nwc, P, nrb, Bp, hsz, split, nchunks;
  int64_t xh_bytes, xw_bytes, cg_bytes, plane_bytes, chunk_bytes, part_bytes, wt_bytes;
  int64_t total() const { return tiled ? 0 : kCtrlBytes + xh_bytes + xw_bytes; }
  int64_t scratch() const { return cg_bytes + 5 * plane_bytes + chunk_bytes + part_bytes + wt_bytes; }
};

// tiled: run the recurrence on the batch-tiled kernel (it also does for H > 1024,
// beyond the persistent kernel's largest reduction).
int plan_bwd(const gs_bwd_args* a, BPlan* pl, const char* who, bool tiled) {
  const int H = (int)a->H;
  pl->tiled = tiled || a->H > kPersistentMaxH;
  pl->KC = pl->nt = pl->nwc = pl->P = pl->hsz = 0;
  pl->xh_bytes = pl->xw_bytes = pl->wt_bytes = 0;
  pl->nrb = (int)((a->B + 3) / 4);
  pl->Bp = 4 * pl->nrb;
  if (pl->tiled) {
    if (a->H > tiled_max_h())
      return set_error(GS_ERR_INVALID, "%s: hidden size %d exceeds the supported maximum of %lld", who, H,
                       (long long)tiled_max_h());
    pl->wt_bytes = tiled_bwd_wt_bytes(H);
  } else {
    pl->KC = choose_kc(H);
    if (pl->KC < 0)
      return set_error(GS_ERR_INVALID, "%s: hidden size %d exceeds the supported maximum of 1024", who, H);
    const int qpb = (H + 3) / 4;
    const int nwmax = pl->KC >= 16 ? 4 : 12;
    pl->nwc = qpb < nwmax ? qpb : nwmax;
    pl->P = (qpb + pl->nwc - 1) / pl->nwc;
    pick_bwd(pl->KC, &pl->nt);
    pl->hsz = 64 * pl->KC;
    // The pollers load 16 KC words per row from the row's start; the pad keeps
    // the reads past the last row inside the workspace.
    pl->xh_bytes = align256(2 * (int64_t)pl->Bp * H * 8 + 16 * pl->KC * 8);
    pl->xw_bytes = align256((int64_t)pl->nrb * pl->P * 8);
  }
  const int64_t TB = a->T * a->B;
  if (TB > INT32_MAX / 4) return set_error(GS_ERR_INVALID, "%s: T*B = %lld is too large", who, (long long)TB);
  pl->split = gemm_pick_split(3 * H, H, (int)TB);
  pl->nchunks = (int)((a->T + kGradSteps - 1) / kGradSteps);
  pl->cg_bytes = align256(TB * 3 * H * 4);
  pl->plane_bytes = align256(TB * H * 4);
  pl->chunk_bytes = align256((int64_t)pl->nchunks * a->B * 3 * H * 4);
  pl->part_bytes = pl->split > 1 ? align256((int64_t)pl->split * 3 * H * H * 4) : 0;
  return GS_OK;
}

}  // namespace

// coef_kernel from gh in cg, or from the forward's saved gh (a->gh_saved, bias added) when set;
// hq as in coef_kernel.
int launch_coef(const gs_bwd_args* a, float* cg, float* cgn, float* zm, float* mi, hipStream_t stream, float* hq) {
  const int64_t n = a->T * a->B * a->H;
  const float* gh = a->gh_saved != nullptr ? a->gh_saved : cg;
  const float* bh = a->gh_saved != nullptr ? a->bh : nullptr;
  hipLaunchKernelGGL(coef_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256), 0, stream,
                     a->gi, a->sg_t, a->sg_b, a->h0, a->sh0_b, a->out, a->so_t, a->so_b, gh, bh, cg, cgn, zm, mi, hq,
                     (int)a->T, (int)a->B, (int)a->H, to_quant(a->q_in), to_quant(a->q_out));
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int grad_chunks(int64_t T) { return (int)((T + kGradSteps - 1) / kGradSteps); }

// grad_kernel over every step, then the dbh row sums unless `dbh_sum` is given:
// then the sum is left to the caller, as *dbh_sum (to be run after the last
// reader of the chunks' producer has been launched, e.g. with sum_partials2).
// dghn and dgh as in grad_kernel (either may be NULL; dgh may be cg).
int launch_grad(const gs_bwd_args* a, const float* dsum, const float* cg, const float* cgn, float* dghn,
                float* dgh, float* chunks, hipStream_t stream, const char* who, SumJob* dbh_sum) {
  const int T = (int)a->T, B = (int)a->B, H = (int)a->H;
  const int nch = grad_chunks(T);
  const int64_t n = (int64_t)nch * B * H;
  hipLaunchKernelGGL(grad_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dsum, cg, cgn, a->dgi,
                     dghn, dgh, chunks, T, B, H);
  GS_CHECK_HIP(hipGetLastError());
  const SumJob job{a->dbh_part, chunks, (int64_t)B * 3 * H, nch, (int64_t)B * 3 * H};
  if (dbh_sum != nullptr) {
    *dbh_sum = job;
    return GS_OK;
  }
  return sum_partials(job.dst, job.src, job.n, job.parts, job.stride, stream, who);
}

int64_t dense_bwd_core_bytes(const gs_bwd_args* a, const char* who, bool tiled) {
  BPlan pl;
  const int rc = plan_bwd(a, &pl, who, tiled);
  if (rc) return rc;
  return pl.total();
}

int64_t dense_bwd_core_scratch(const gs_bwd_args* a, const char* who, bool tiled) {
  BPlan pl;
  const int rc = plan_bwd(a, &pl, who, tiled);
  if (rc) return rc;
  return pl.scratch();
}

int64_t dense_bwd_workspace_bytes(const gs_bwd_args* a, bool tiled) {
  return dense_bwd_core_bytes(a, "gs_bwd_workspace_bytes", tiled);
}
int64_t dense_bwd_scratch_bytes(const gs_bwd_args* a, bool tiled) {
  return dense_bwd_core_scratch(a, "gs_bwd_scratch_bytes", tiled);
}

namespace {
int launch_recurrence(const BPlan& pl, const float* w, const gs_bwd_args* a, const float* cg, const float* zm,
                      const float* mi, float* dsum, uint64_t* xh, uint64_t* xw, char* ws, hipStream_t stream,
                      const char* who);
}  // namespace

// The dense backward of a hidden map given as the matrix w [3H, H] (rows r,
// z, n); writes dgi, dh0 and dbh_part of `a` and the map's gradient dw
// [3H, H]. Uses the first dense_bwd_core_bytes(a) bytes of a->workspace and
// the first dense_bwd_core_scratch(a) bytes of a->scratch. tiled: the
// recurrence runs on the batch-tiled kernel, as it does anyway for H > 1024.
int dense_bwd_core(const gs_bwd_args* a, const float* w, float* dw, hipStream_t stream, const char* who, bool tiled) {
  if (a->T > 1 && a->so_t != a->B * a->so_b)
    return set_error(GS_ERR_INVALID, "%s: out must hold its steps back to back (so_t == B * so_b); got so_t=%lld, so_b=%lld",
                     who, (long long)a->so_t, (long long)a->so_b);
  BPlan pl;
  int rc = plan_bwd(a, &pl, who, tiled);
  if (rc) return rc;
  const gs_args f = fwd_view(*a);
  rc = check_workspace(&f, pl.total(), who);
  if (rc) return rc;
  rc = check_scratch(a, pl.scratch(), who);
  if (rc) return rc;

  const int T = (int)a->T, B = (int)a->B, H = (int)a->H, TB = T * B;
  char* ws = static_cast<char*>(a->workspace);
  uint64_t* xh = reinterpret_cast<uint64_t*>(ws + kCtrlBytes);
  uint64_t* xw = reinterpret_cast<uint64_t*>(ws + kCtrlBytes + pl.xh_bytes);
  char* cur = static_cast<char*>(a->scratch);
  auto take = [&](int64_t bytes) {
    char* r = cur;
    cur += bytes;
    return r;
  };
  float* cg = reinterpret_cast<float*>(take(pl.cg_bytes));
  float* hq = reinterpret_cast<float*>(take(pl.plane_bytes));
  float* cgn = reinterpret_cast<float*>(take(pl.plane_bytes));
  float* zm = reinterpret_cast<float*>(take(pl.plane_bytes));
  float* mi = reinterpret_cast<float*>(take(pl.plane_bytes));
  float* dsum = reinterpret_cast<float*>(take(pl.plane_bytes));
  float* chunks = reinterpret_cast<float*>(take(pl.chunk_bytes));
  float* part = reinterpret_cast<float*>(take(pl.part_bytes));
  const Quant qin = to_quant(a->q_in), qout = to_quant(a->q_out);
  const int64_t n_plane = (int64_t)TB * H;
  auto grid1d = [](int64_t n) { return dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)); };

  // 0. hq = q_in([h0; out[0..T-2]]): rows m = t B + b of a [T B, H] matrix; with the saved
  //    gh nothing reads it before the coefficient pass, which writes it then
  if (a->gh_saved == nullptr) {
    rc = build_prev_state(hq, a->h0, a->sh0_b, a->out, a->so_b, T, B, H, qin, stream, who);
    if (rc) return rc;
  }

  // 1. gh = hq Wh^T + bh  -> cg [T B, 3H], unless the forward saved it
  const float* gh = a->gh_saved != nullptr ? a->gh_saved : cg;
  if (a->gh_saved == nullptr) {
    GemmArgs g1;
    g1.a = hq;
    g1.lda = H;
    g1.b = w;  // B(k, n) = Wh[n][k]
    g1.ldb = H;
    g1.c = cg;
    g1.ldc = 3 * H;
    g1.split_stride = 0;
    g1.bias = a->bh;
    g1.M = TB;
    g1.N = 3 * H;
    g1.K = H;
    g1.ksplit = 1;
    g1.layout = kGemmNT;
    rc = gemm_f32(g1, stream, who);
    if (rc) return rc;
  }

  // 2. coefficient planes
  hipLaunchKernelGGL(coef_kernel, grid1d(n_plane), dim3(256), 0, stream, a->gi, a->sg_t, a->sg_b, a->h0, a->sh0_b,
                     a->out, a->so_t, a->so_b, gh, a->gh_saved != nullptr ? a->bh : nullptr, cg, cgn, zm, mi,
                     a->gh_saved != nullptr ? hq : nullptr, T,
                     B, H, qin, qout);
  GS_CHECK_HIP(hipGetLastError());

  // 3. the recurrence
  if (pl.tiled) {
    float* wt = reinterpret_cast<float*>(take(pl.wt_bytes));
    rc = run_tiled_bwd_recurrence(w, wt, a->dout, cg, zm, mi, dsum, a->dh0, T, B, H, stream, who);
    if (rc) return rc;
  } else {
    rc = launch_recurrence(pl, w, a, cg, zm, mi, dsum, xh, xw, ws, stream, who);
    if (rc) return rc;
  }

  // 4. dgi, per-row dbh, and dgh = (dg_r, dg_z, dgh_n) over the coefficients in cg
  const int64_t n_grad = (int64_t)pl.nchunks * B * H;
  hipLaunchKernelGGL(grad_kernel, dim3((unsigned)((n_grad + 255) / 256)), dim3(256), 0, stream, dsum, cg, cgn, a->dgi,
                     nullptr, cg, chunks, T, B, H);
  GS_CHECK_HIP(hipGetLastError());
  // the dbh row sums run with the dWh split sums below, in one launch
  const SumJob dbh_sum{a->dbh_part, chunks, (int64_t)B * 3 * H, pl.nchunks, (int64_t)B * 3 * H};

  // 5. dWh[n][k] = sum_m dgh[m][n] hq[m][k], one product over the 3H rows
  float* dst = pl.split > 1 ? part : dw;
  const int64_t split_stride = (int64_t)3 * H * H;
  GemmArgs g3;
  g3.a = cg;  // A(n, m) = dgh[m][n]
  g3.lda = 3 * H;
  g3.b = hq;  // B(m, k) = hq[m][k]
  g3.ldb = H;
  g3.c = dst;
  g3.ldc = H;
  g3.split_stride = split_stride;
  g3.bias = nullptr;
  g3.M = 3 * H;
  g3.N = H;
  g3.K = TB;
  g3.ksplit = pl.split;
  g3.layout = kGemmTN;
  rc = gemm_f32(g3, stream, who);
  if (rc) return rc;
  if (pl.split > 1) return sum_partials2(dbh_sum, SumJob{dw, part, split_stride, pl.split, split_stride}, stream, who);
  return sum_partials(dbh_sum.dst, dbh_sum.src, dbh_sum.n, dbh_sum.parts, dbh_sum.stride, stream, who);
}

namespace {

// Step 3 of dense_bwd_core on the persistent kernel (H <= 1024).
int launch_recurrence(const BPlan& pl, const float* w, const gs_bwd_args* a, const float* cg, const float* zm,
                      const float* mi, float* dsum, uint64_t* xh, uint64_t* xw, char* ws, hipStream_t stream,
                      const char* who) {
  const int T = (int)a->T, B = (int)a->B, H = (int)a->H;
  int rc = GS_OK;
  int nt = 0;
  BFn fn = pick_bwd(pl.KC, &nt);
  const int threads = 64 * (pl.nwc + 4 * bwd_pollers_per_row(pl.KC));
  int G = pl.nrb, RB = 1;
  size_t lds = 0;
  for (int pass = 0; pass < 2; ++pass) {
    RB = (pl.nrb + G - 1) / G;
    G = (pl.nrb + RB - 1) / RB;
    const int U = 4 * pl.nwc;
    lds = sizeof(float) * (size_t)(6 * pl.hsz + 8 * kNV * U + RB * 4 * U + 4);
    if (lds > 65536)
      GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int gfit = 0;
    rc = resident_groups((const void*)fn, threads, lds, pl.P, pl.nrb, &gfit, who);
    if (rc) return rc;
    if (gfit >= G) break;
    G = gfit;
  }
  BParams p;
  p.w = w;
  p.dout = a->dout;
  p.cg = cg;
  p.zm = zm;
  p.mi = mi;
  p.dsum = dsum;
  p.dh0 = a->dh0;
  p.xh = xh;
  p.xw = xw;
  p.ctrl = ctrl_of(ws, a->fault_mirror);
  p.T = T;
  p.B = B;
  p.H = H;
  p.ngroups = G;
  p.RB = RB;
  p.nrb = pl.nrb;
  p.Bp = pl.Bp;
  p.P = pl.P;
  p.nwg = G * pl.P;
  p.nwc = pl.nwc;
  p.hsz = pl.hsz;
  hipLaunchKernelGGL(fn, dim3(p.nwg), dim3(threads), lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace

}  // namespace gs

extern "C" int gs_dense_bwd(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_dense_bwd";
  int rc = validate_bwd_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  return dense_bwd_core(a, a->w, a->dw_part, stream, who, false);
}

// The barrier-free dense backward (reference gru_scan_backward_triton,
// scan.py:1355-1447, kernel gru_scan_bwd_kernel :916-1352): dense_bwd_core with
// the recurrence on the batch-tiled kernel at every H.
extern "C" int gs_dense_bwd_tiled(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_dense_bwd_tiled";
  int rc = validate_bwd_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  return dense_bwd_core(a, a->w, a->dw_part, stream, who, true);
}
