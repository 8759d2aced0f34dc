// Dense GRU scan backward (gfx950): the persistent reverse recurrence on fp32
// MFMA, framed by two GEMMs.
//
// Reference: gru_scan_backward_persistent and its kernel
// (LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py:646-752, :296-643),
// whose math is the PyTorch backward at scan.py:1460-1550. Per step t, walking
// t from T-1 to 0 with h_{t-1} = out[t-1] (h0 at t = 0):
//   gh_t    = q_in(h_{t-1}) Wh^T + bh                 (recomputed)
//   dh_t    = dout[t] + dh_carry, masked by q_out's clipped STE on h_t's raw value
//   dgi_t   = (dgr, dgz, dgn), dgh_t = (dgr, dgz, dgn * r)   (gru_backward)
//   dh_carry <- dh_t * z + mask_in(h_{t-1}) * (dgh_t Wh)
//   dWh += dgh_t^T q_in(h_{t-1}),  dbh += sum_b dgh_t
// Only the dgh_t Wh product sits on the recurrence. The launcher runs
//   1. gemm: gh for every step at once, into the workspace;
//   2. dense_bwd_kernel: the recurrence, writing dgi, dh0, dgh's n part
//      (dgi holds its r and z parts) and per-row dbh sums;
//   3. gemm: dWh = dgh^T q_in([h0; out[0..T-2]]), K split over T*B, then a sum.
//
// The recurrence kernel mirrors the forward's exchange (scan_dense.hip) with
// the roles of K and the output swapped: the exchanged vector is dgh_t
// (3H words per batch row) and each compute wave owns a quad of units u of
// dh_{t-1}, holding the Wh columns of those units over all 3H rows in VGPRs
// (wt[g][m] = Wh[g H + kmap(m)][u]). Per iteration a compute wave runs one
// MFMA chain over the three staged dgh segments, reduces the K slices, and
// the 16 lanes of row 0 finish the step: carry, gate gradients of step t-1,
// stores, and the tagged publish of dgh_{t-1}. Four poller waves per
// workgroup stage the next iteration's dgh row (polled) and the per-unit
// step inputs (gi, gh, dout, out, h0) into LDS. dgh_{T-1} needs no exchange:
// it depends only on inputs, so the stagers compute it for the whole row.
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kPollers = 4;
// Per-unit values staged for one iteration (consuming dgh_t):
//   0 h_{t-1} (q_in mask), 1 dout[t-1], 2..4 gi[t-1] (r, z, n),
//   5..7 gh[t-1] (r, z, n), 8 h_{t-2}
constexpr int kNV = 9;

struct BParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* out;
  const float* dout;  // [T, B, H] contiguous
  const float* gh;    // [T, B, 3H] contiguous, bias included
  float* dgi;         // [T, B, 3H] contiguous
  float* dghn;        // [T, B, H] contiguous
  float* dh0;         // [B, H] contiguous
  float* dbh_part;    // [B, 3H] contiguous
  uint64_t* xh;       // [2][Bp][3H] tagged dgh
  uint64_t* xw;       // [nwg] tagged XCD ids
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int ngroups, RB, nrb, Bp, nwg, P, nwc, hsz;
  Quant qin, qout;
};

// h_t of row `row` (t >= 0) or h0 (t == -1), unit k.
__device__ __forceinline__ float h_at(const BParams& p, int t, int row, int k) {
  return t >= 0 ? p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + k] : p.h0[(int64_t)row * p.sh0_b + k];
}

// Staged value v of unit k for the iteration that consumes dgh_t.
__device__ __forceinline__ float step_value(const BParams& p, int t, int row, int k, int v) {
  if (v == 0) return h_at(p, t - 1, row, k);
  if (t == 0) return 0.0f;
  const int tp = t - 1;
  if (v == 1) return p.dout[((int64_t)tp * p.B + row) * p.H + k];
  if (v <= 4) return p.gi[(int64_t)tp * p.sg_t + (int64_t)row * p.sg_b + (v - 2) * p.H + k];
  if (v <= 7) return p.gh[((int64_t)tp * p.B + row) * 3 * p.H + (v - 5) * p.H + k];
  return h_at(p, t - 2, row, k);
}

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

  float* hst = lds;                              // [2][3][hsz] staged dgh (il_index per gate block)
  float* sti = hst + 6 * p.hsz;                  // [2][4][kNV][U] staged per-unit step inputs
  float* dd = sti + 2 * 4 * kNV * U;             // [RB][4][U] dh_t * z_t carried to the next step
  float* dacc = dd + p.RB * 4 * U;               // [RB][4][3][U] running sums of dgh (dbh)
  int* flags = reinterpret_cast<int*>(dacc + p.RB * 12 * U);  // [0] compute-wave iterations published,
                                                               // [1] group on one XCD
  const int lds_floats = 6 * p.hsz + 8 * kNV * U + p.RB * 16 * U + 4;
  for (int i = threadIdx.x; i < lds_floats; i += blockDim.x) lds[i] = 0.0f;

  const uint32_t base = __hip_atomic_load(p.ctrl.tag_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) st_tagged(p.xw + blockIdx.x, __uint_as_float(xcc_id()), base + 1u);
  const int niter = T * nrbm;

  // dgh_{T-1} of unit k of local row r for iteration nx (< nrbm): computed
  // from inputs; the owner of unit k also stores its dgi / dgh_n, seeds the
  // dbh sums and keeps dh_{T-1} z_{T-1}.
  auto stage_first = [&](int nx, int r, int k) {
    const int row = 4 * (rb_begin + nx) + r;
    if (row >= p.B) return;
    const int t = T - 1;
    const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + k;
    const float* h = p.gh + ((int64_t)t * p.B + row) * 3 * H + k;
    const float dh = p.dout[((int64_t)t * p.B + row) * H + k];
    const GateGrad gg = gru_backward(g[0], g[H], g[2 * H], h[0], h[H], h[2 * H], h_at(p, t - 1, row, k), dh, p.qout);
    float* hs = hst + (nx & 1) * 3 * p.hsz + il_index(r, k);
    hs[0] = gg.dgr;
    hs[p.hsz] = gg.dgz;
    hs[2 * p.hsz] = gg.dghn;
    const int u = k - ulo;
    if (u >= 0 && u < U) {
      float* dgo = p.dgi + ((int64_t)t * p.B + row) * 3 * H + k;
      dgo[0] = gg.dgr;
      dgo[H] = gg.dgz;
      dgo[2 * H] = gg.dgn;
      p.dghn[((int64_t)t * p.B + row) * H + k] = gg.dghn;
      dd[(nx * 4 + r) * U + u] = gg.dh_direct;
      float* da = dacc + (nx * 4 + r) * 3 * U + u;
      da[0] = gg.dgr;
      da[U] = gg.dgz;
      da[2 * U] = gg.dghn;
    }
  };

  // Prologue (all waves): iteration 0's inputs.
  lds_barrier();
  for (int w = threadIdx.x; w < 4 * H; w += blockDim.x) stage_first(0, w / H, w % H);
  for (int w = threadIdx.x; w < 4 * kNV * U; w += blockDim.x) {
    const int r = w / (kNV * U), rem = w - r * kNV * U, v = rem / U, u = rem - v * U;
    const int row = 4 * rb_begin + r;
    sti[w] = (row < p.B && ulo + u < H) ? step_value(p, T - 1, row, ulo + u, v) : 0.0f;
  }
  lds_barrier();

  if (!poller) {
    float wt[3][KC];
    load_wt<KC>(p.w, H, o0, j, kb4, quad_ok, wt);
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
      float via_w = reduce16(acc0 + acc1, s);
      const bool xcd_local = st >= 1 && __builtin_amdgcn_readfirstlane(flags[1]) != 0;
      if (lead && unit_ok && row < p.B) {
        const float* sv = sti + (buf * 4 + s) * kNV * U + uo;
        float* ddp = dd + (rbl * 4 + s) * U + uo;
        if (p.qin.on && !quant_keeps(sv[0], p.qin)) via_w = 0.0f;
        const float carry = *ddp + via_w;
        if (t == 0) {
          p.dh0[(int64_t)row * H + unit] = carry;
        } else {
          const float dh = sv[U] + carry;
          const GateGrad gg = gru_backward(sv[2 * U], sv[3 * U], sv[4 * U], sv[5 * U], sv[6 * U], sv[7 * U],
                                           sv[8 * U], dh, p.qout);
          const int64_t rowt = (int64_t)(t - 1) * p.B + row;
          const uint32_t tag = base + (uint32_t)st + 1u;
          uint64_t* dst = p.xh + ((int64_t)(st & 1) * p.Bp + row) * 3 * H + unit;
          if (xcd_local) {
            st_tagged_xcd(dst, gg.dgr, tag);
            st_tagged_xcd(dst + H, gg.dgz, tag);
            st_tagged_xcd(dst + 2 * H, gg.dghn, tag);
          } else {
            st_tagged(dst, gg.dgr, tag);
            st_tagged(dst + H, gg.dgz, tag);
            st_tagged(dst + 2 * H, gg.dghn, tag);
          }
          float* dgo = p.dgi + rowt * 3 * H + unit;
          dgo[0] = gg.dgr;
          dgo[H] = gg.dgz;
          dgo[2 * H] = gg.dgn;
          p.dghn[rowt * H + unit] = gg.dghn;
          float* da = dacc + (rbl * 4 + s) * 3 * U + uo;
          da[0] += gg.dgr;
          da[U] += gg.dgz;
          da[2 * U] += gg.dghn;
          *ddp = gg.dh_direct;
        }
      }
      if (lane == 0) __hip_atomic_fetch_add(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
    }
  } else {
    // Poller wave pr stages row pr of iteration it + 1 while the compute
    // waves run iteration it: the per-unit step inputs first (their loads
    // overlap the poll), then the dgh row, polled once this workgroup's
    // compute waves have published iteration it.
    const int pr = wave - nwc;
    constexpr int NWC_MAX = NT / 64 - kPollers;
    constexpr int NSV = (kNV * 4 * NWC_MAX + 63) / 64;  // staged values per lane
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
          sv[i] = (w < kNV * U && row < p.B && ulo + u < H) ? step_value(p, t2, row, ulo + u, v) : 0.0f;
        }
        if (st2 == 0) {
          for (int k = lane; k < H; k += 64) stage_first(nx, pr, k);
        } else if (row < p.B) {
          if (pr == 0 && nx == nrbm)  // first exchange of the launch
            flags[1] = (p.P <= 64 && group_on_one_xcd(p.ctrl, p.xw + gid, p.ngroups, p.P, base + 1u)) ? 1 : 0;
          wait_lds_count(p.ctrl, &flags[0], nwc * (it + 1));
          const uint64_t* hb = p.xh + ((int64_t)((st2 - 1) & 1) * p.Bp + row) * 3 * H;
          poll_row_segs<KC / 4, 3>(p.ctrl, hb, H, hst + (nx & 1) * 3 * p.hsz, p.hsz, pr, H, base + (uint32_t)st2);
        } else if (pr == 0 && nx == nrbm) {
          flags[1] = (p.P <= 64 && group_on_one_xcd(p.ctrl, p.xw + gid, p.ngroups, p.P, base + 1u)) ? 1 : 0;
        }
        float* sd = sti + ((nx & 1) * 4 + pr) * kNV * U;
#pragma unroll
        for (int i = 0; i < NSV; ++i) {
          const int w = lane + 64 * i;
          if (w < kNV * U) sd[w] = sv[i];
        }
      }
      lds_barrier();
    }
  }

  // Per-row dbh sums of this workgroup's units.
  lds_barrier();
  for (int w = threadIdx.x; w < nrbm * 12 * U; w += blockDim.x) {
    const int rbl = w / (12 * U), rem = w - rbl * 12 * U, r = rem / (3 * U), rem2 = rem - r * 3 * U;
    const int g = rem2 / U, u = rem2 - g * U;
    const int row = 4 * (rb_begin + rbl) + r;
    if (row < p.B && ulo + u < H) p.dbh_part[(int64_t)row * 3 * H + g * H + ulo + u] = dacc[w];
  }
  leave_grid(p.ctrl, (uint32_t)p.nwg, base, (uint32_t)T);
}

typedef void (*BFn)(BParams);

BFn pick_bwd(int KC, int* nt) {
  switch (KC) {
    case 4: *nt = 1024; return dense_bwd_kernel<4, 1024>;
    case 8: *nt = 1024; return dense_bwd_kernel<8, 1024>;
    case 16: *nt = 512; return dense_bwd_kernel<16, 512>;
    case 32: *nt = 512; return dense_bwd_kernel<32, 512>;
    case 64: *nt = 512; return dense_bwd_kernel<64, 512>;
    default: return nullptr;
  }
}

struct BPlan {
  int KC, nt, nwc, P, nrb, Bp, hsz, split;
  int64_t xh_bytes, xw_bytes, gh_bytes, dghn_bytes, part_bytes;
  int64_t total() const { return kCtrlBytes + xh_bytes + xw_bytes + gh_bytes + dghn_bytes + part_bytes; }
};

int plan_bwd(const gs_bwd_args* a, BPlan* pl, const char* who) {
  const int H = (int)a->H;
  pl->KC = choose_kc(H);
  if (pl->KC < 0)
    return set_error(GS_ERR_INVALID, "%s: hidden size %d exceeds the supported maximum of 1024", who, H);
  const int qpb = (H + 3) / 4;
  const int nwmax = pl->KC >= 16 ? 4 : 12;
  pl->nwc = qpb < nwmax ? qpb : nwmax;
  pl->P = (qpb + pl->nwc - 1) / pl->nwc;
  pick_bwd(pl->KC, &pl->nt);
  pl->nrb = (int)((a->B + 3) / 4);
  pl->Bp = 4 * pl->nrb;
  pl->hsz = 64 * pl->KC;
  const int64_t TB = a->T * a->B;
  if (TB > INT32_MAX) return set_error(GS_ERR_INVALID, "%s: T*B = %lld exceeds 2^31 - 1", who, (long long)TB);
  pl->split = gemm_pick_split(3 * H, H, (int)TB);
  pl->xh_bytes = align256(2 * (int64_t)pl->Bp * 3 * H * 8 + 16 * pl->KC * 8);
  pl->xw_bytes = align256((int64_t)pl->nrb * pl->P * 8);
  pl->gh_bytes = align256(TB * 3 * H * 4);
  pl->dghn_bytes = align256(TB * H * 4);
  pl->part_bytes = pl->split > 1 ? align256((int64_t)pl->split * 3 * H * H * 4) : 0;
  return GS_OK;
}

}  // namespace

int64_t dense_bwd_workspace_bytes(const gs_bwd_args* a) {
  BPlan pl;
  const int rc = plan_bwd(a, &pl, "gs_bwd_workspace_bytes");
  if (rc) return rc;
  return pl.total();
}

}  // namespace gs

extern "C" int gs_dense_bwd(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  clear_error();
  const char* who = "gs_dense_bwd";
  int rc = validate_bwd_common(a, who);
  if (rc) return rc;
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  if (a->T > 1 && a->so_t != a->B * a->so_b)
    return set_error(GS_ERR_INVALID, "%s: out must hold its steps back to back (so_t == B * so_b); got so_t=%lld, so_b=%lld",
                     who, (long long)a->so_t, (long long)a->so_b);
  BPlan pl;
  rc = plan_bwd(a, &pl, who);
  if (rc) return rc;
  const gs_args f = fwd_view(*a);
  rc = check_workspace(&f, pl.total(), who);
  if (rc) return rc;

  const int T = (int)a->T, B = (int)a->B, H = (int)a->H, TB = T * B;
  char* ws = static_cast<char*>(a->workspace);
  uint64_t* xh = reinterpret_cast<uint64_t*>(ws + kCtrlBytes);
  uint64_t* xw = reinterpret_cast<uint64_t*>(ws + kCtrlBytes + pl.xh_bytes);
  float* gh = reinterpret_cast<float*>(ws + kCtrlBytes + pl.xh_bytes + pl.xw_bytes);
  float* dghn = reinterpret_cast<float*>(reinterpret_cast<char*>(gh) + pl.gh_bytes);
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(dghn) + pl.dghn_bytes);

  // q_in([h0; out[0..T-2]]) as rows m = t B + b of a [T B, H] matrix.
  GemmOperand hq{a->out, a->so_b, 1, a->h0, a->sh0_b, B, to_quant(a->q_in)};

  // 1. gh = hq Wh^T + bh  -> [T B, 3H]
  GemmArgs g1;
  g1.a = hq;
  g1.b = plain_operand(a->w, 1, H);  // B(k, n) = Wh[n][k]
  g1.c = gh;
  g1.ldc = 3 * H;
  g1.split_stride = 0;
  g1.bias = a->bh;
  g1.M = TB;
  g1.N = 3 * H;
  g1.K = H;
  g1.ksplit = 1;
  rc = gemm_f32(g1, stream, who);
  if (rc) return rc;

  // 2. the recurrence
  int nt = 0;
  BFn fn = pick_bwd(pl.KC, &nt);
  const int threads = 64 * (pl.nwc + kPollers);
  int G = pl.nrb, RB = 1;
  size_t lds = 0;
  for (int pass = 0; pass < 2; ++pass) {
    RB = (pl.nrb + G - 1) / G;
    G = (pl.nrb + RB - 1) / RB;
    const int U = 4 * pl.nwc;
    lds = sizeof(float) * (size_t)(6 * pl.hsz + 8 * kNV * U + RB * 16 * U + 4);
    if (lds > 65536)
      GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int gfit = 0;
    rc = resident_groups((const void*)fn, threads, lds, pl.P, pl.nrb, &gfit, who);
    if (rc) return rc;
    if (gfit >= G) break;
    G = gfit;
  }
  BParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.out = a->out;
  p.dout = a->dout;
  p.gh = gh;
  p.dgi = a->dgi;
  p.dghn = dghn;
  p.dh0 = a->dh0;
  p.dbh_part = a->dbh_part;
  p.xh = xh;
  p.xw = xw;
  p.ctrl = ctrl_of(ws);
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
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
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  hipLaunchKernelGGL(fn, dim3(p.nwg), dim3(threads), lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());

  // 3. dWh[n][k] = sum_m dgh[m][n] hq[m][k]: rows [0, 2H) from dgi's r and z
  //    parts, rows [2H, 3H) from dgh_n.
  float* dst = pl.split > 1 ? part : a->dw_part;
  const int64_t split_stride = (int64_t)3 * H * H;
  GemmArgs g3;
  g3.a = plain_operand(a->dgi, 1, 3 * H);  // A(n, m) = dgi[m][n]
  g3.b = hq;
  g3.c = dst;
  g3.ldc = H;
  g3.split_stride = split_stride;
  g3.bias = nullptr;
  g3.M = 2 * H;
  g3.N = H;
  g3.K = TB;
  g3.ksplit = pl.split;
  rc = gemm_f32(g3, stream, who);
  if (rc) return rc;
  g3.a = plain_operand(dghn, 1, H);
  g3.c = dst + (int64_t)2 * H * H;
  g3.M = H;
  rc = gemm_f32(g3, stream, who);
  if (rc) return rc;
  if (pl.split > 1) return sum_partials(a->dw_part, part, split_stride, pl.split, split_stride, stream, who);
  return GS_OK;
}
