// Butterfly GRU scan backward (gfx950), stage by stage.
//
// Reference: the butterfly backward kernel and launcher (LarocheC/gru-triton
// src/gru_qat/triton_kernels/scan_butterfly.py:462-1075) and the PyTorch
// backward it restates (scan.py:1460-1550 with the butterfly map). The map of
// gate g is a chain of K = nchains L sparse stages S_1 .. S_K on vectors
// zero-padded to N = 2^L (stage order, strides and twiddle selection as in the
// forward, scan_butterfly.hip), so gh_g = [S_K ... S_1 q_in(h)]_{:H} + bh_g.
//
// As in the dense backward (scan_dense_bwd.hip), every gradient of step t is
// D_t times a coefficient fixed by the forward, and the recurrence is
//   D_{t-1} = dout[t-1] + Zm_t D_t + Mi_t sum_g S_1^T ... S_K^T (D_t Cg_t)
// Batch rows never interact, so one workgroup owns one row for all T steps
// and applies the transposed stages in reverse order in LDS, with no
// exchange between workgroups. The launcher runs
//   1. bfly_apply_coef: for every (t, b) at once, hq = q_in(h_{t-1}) and gh
//      (the forward's stages on hq, kept in LDS), then the dense backward's
//      coefficient planes from gi, gh and h_{t-1}, and hq;
//   2. bfly_bwd_kernel: the recurrence, writing dh0 and the gradient planes
//      as it forms them (dgi, dgh_n) and the per-row dbh sums;
//   3. bfly_twiddle_grad: for every (t, b) and gate, the stages run forward on
//      hq (activations A_j kept in LDS) and dgh runs backward through them
//      (G_j); stage j's twiddles collect the dots of G_{j+1} with A_j (own
//      element for the diagonal twiddle, the partner for the other) in
//      per-workgroup LDS accumulators, summed over workgroups by
//      bfly_twiddle_sum.
// Shapes whose LDS needs exceed the device limit fall back to the
// materialized-map backward (scan_struct_bwd.hip).
#include <mutex>

#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {

int64_t struct_bwd_workspace_bytes(int kind, const gs_bwd_args* a);
int64_t struct_bwd_scratch_bytes(int kind, const gs_bwd_args* a);
int run_struct(int kind, const gs_bwd_args* a, hipStream_t stream, const char* who);

namespace {

// Twiddles of element i in layer s of a single chain (stride 2^s): the
// diagonal one (own element), the off-diagonal one (partner i ^ 2^s), and the
// partner row's off-diagonal one (S[partner][i]), which the transposed stage
// needs. tw_g is one gate's [L][N/2][2][2].
struct ElemTw {
  float t_ii, t_ip, t_pi;
};

__device__ __forceinline__ ElemTw elem_tw(const float* tw_g, int N, int s, int i) {
  const int m = (i >> s) & 1;
  const int pair = ((i >> (s + 1)) << s) | (i & ((1 << s) - 1));
  const float* t = tw_g + ((int64_t)s * (N / 2) + pair) * 4;
  ElemTw r;
  r.t_ii = t[3 * m];          // [m][m]
  r.t_ip = t[2 * m + 1 - m];  // [m][1 - m]
  r.t_pi = t[2 - m];          // [1 - m][m]
  return r;
}

// Lane layout of the forward's register kernel (scan_butterfly.hip): a gate
// vector of N = 256 WPG elements spreads over WPG waves; lane l of the gate's
// wave w holds elements i = l + 64 r + 256 w, r < 4. The partner of i in layer
// s (i ^ 2^s) comes from a DPP move (strides 1-8), an LDS permute (16, 32),
// another register of the same lane (64, 128) or an LDS exchange between the
// gate's waves (>= 256, the only case that needs a workgroup barrier).
template <int S, bool VX = false>
__device__ __forceinline__ void partner_of(const float (&x)[4], float (&y)[4], float* xch, const int (&idx)[4]) {
  if constexpr (S <= 3 || (VX && S < 6)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = lane_xor_c<1 << S>(x[r]);
  } else if constexpr (S < 6) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = lane_xor(x[r], 1 << S);
  } else if constexpr (S < 8) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = x[r ^ (1 << (S - 6))];
  } else {
    // lane-major exchange buffer: element r of lane l of wave w at 256 w + 4 l + r,
    // so a lane writes its four elements and reads its partners' (the same lane and
    // r of wave w ^ 2^(S-8)) with one 16-byte access each
    const int w = idx[0] >> 8, l = idx[0] & 63;
    *reinterpret_cast<f4*>(xch + 256 * w + 4 * l) = f4{x[0], x[1], x[2], x[3]};
    lds_barrier();
    const f4 v = *reinterpret_cast<const f4*>(xch + 256 * (w ^ (1 << (S - 8))) + 4 * l);
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = v[r];
  }
}

template <int LOGN>
struct Lay {
  static constexpr int N = 1 << LOGN;
  static constexpr int WPG = N / 256;  // waves per gate vector
};

// The planes that only these kernels read (hq and the coefficient planes)
// hold each row of N elements (zero past H) in lane order: element
// i = lane + 64 r + 256 w sits at 256 w + 4 lane + r, so a lane's four
// elements are one 16-byte load.
// (The four values stay one vector value from the load to their use, so the
// compiler keeps them in the load's registers.)
typedef float f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4 ld_lane4(const float* row, uint32_t off) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(raw_rsrc(row), (int)off, 0, 0));
}

struct CoefParams {
  const float* tw;
  const float* bh;
  const float* gi;   // [T, B, 3H], strides sg_t, sg_b
  const float* h0;   // [B, H], stride sh0_b
  const float* out;  // [T, B, H], steps back to back: row m = t B + b at out + m so_b
  float* hq;         // [T B, N] q_in(h_{t-1}), lane order
  float* cg;         // [T B, 3, N] (Cr, Cz, Chn), lane order
  float* cgn;        // [T B, N] lane order
  float* zm;         // [T B, N] lane order
  float* mi;         // [T B, N] lane order
  int64_t sg_t, sg_b, sh0_b, so_b, nvec;
  int B, H;
  Quant qin, qout;
};

// For every vector v = t B + b: h_{t-1} (h0 at t = 0) and hq = q_in(h_{t-1}),
// gh_g = [S_L ... S_1 hq]_{:H} + bh_g on 3 WPG waves (one gate per WPG of
// them), then the dense backward's coefficient planes of every element from
// gi, gh and h_{t-1} (coef_kernel in scan_dense_bwd.hip, the same arithmetic),
// and hq for the twiddle gradient. gh only passes through LDS. Element k's
// coefficients are formed by one of the three waves that hold it: slot r of
// wave w (elements lane + 64 r + 256 w) goes to gate (r + w) mod 3's wave, so
// a wave owns slot sa = (g - w) mod 3, and slot 3 as well when sa = 0. The
// coefficients go to LDS and from there to the lane-order planes, one
// 16-byte store per lane and row. Lanes past H read element H - 1's inputs
// (clamped loads and LDS reads) and stage zeros, so every iteration issues
// the same global memory operations on every path, and the waits for one
// register set never cover the stores or the other set's loads.
template <int LOGN>
__global__ __launch_bounds__(3 * (1 << LOGN) / 4) void bfly_apply_coef(CoefParams p) {
  constexpr int N = Lay<LOGN>::N, WPG = Lay<LOGN>::WPG, L = LOGN;
  __shared__ __attribute__((aligned(16))) float xch[2][3][N];
  __shared__ float ghs[2][3][N];
  __shared__ float stg[2][7][N];  // a vector's seven output rows, element order (two vectors in turn)
  // the wave index read into a scalar register, so that per-gate choices are scalar
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = wv / WPG,
            w = wv - g * WPG;
  const int H = p.H;
  int idx[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) idx[r] = lane + 64 * r + 256 * w;
  float tii[L][4], tip[L][4];
  const float* tw_g = p.tw + (int64_t)g * L * (N / 2) * 4;
#pragma unroll
  for (int s = 0; s < L; ++s)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const ElemTw e = elem_tw(tw_g, N, s, idx[r]);
      tii[s][r] = e.t_ii;
      tip[s][r] = e.t_ip;
    }
  // N = 1024: layers 8 and 9 (strides 256, 512) run as one exchange with
  // pre-multiplied coefficients, as the forward register kernel runs them
  // (scan_butterfly.hip), so gh rounds as the forward's does
  float c8[4][4];
  if constexpr (L == 10) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const ElemTw q = elem_tw(tw_g, N, 8, idx[r] ^ 512);
      c8[0][r] = tii[9][r] * tii[8][r];
      c8[1][r] = tii[9][r] * tip[8][r];
      c8[2][r] = tip[9][r] * q.t_ii;
      c8[3][r] = tip[9][r] * q.t_ip;
    }
  }
  float bias[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) bias[r] = idx[r] < H ? p.bh[g * H + idx[r]] : 0.0f;
  const int sa = (g - w % 3 + 3) % 3;
  const bool two = sa == 0;
  const int ka = lane + 64 * sa + 256 * w;
  const int kb = lane + 192 + 256 * w;  // slot 3, used when two
  const int kac = ka < H ? ka : H - 1, kbc = !two ? kac : kb < H ? kb : H - 1;
  // the slots' elements as staged (a slot past H stages zeros)
  const int kwa = ka, kwb = two ? kb : ka;
  const bool oka = ka < H, okb = two ? kb < H : oka;
  // The staged rows go out in lane order, one 16-byte store per lane and
  // row: the gate-r waves store Cr, Cz, Chn; the gate-z waves Cgn, Zm; the
  // gate-n waves Mi, hq; every wave issues three stores (the third of the
  // gate-z and gate-n waves goes to a zero-size resource and is dropped).
  const int srow[3] = {g == 0 ? 0 : g == 1 ? 3 : 5, g == 0 ? 1 : g == 1 ? 4 : 6, 2};
  const uint32_t loff = 16u * (64 * w + lane);
  // A vector's inputs (h_{t-1} at the lane's elements, gi at its coefficient
  // slots) sit in one of two register sets that take turns, each refilled for
  // the vector after next once used, at clamped addresses so that every
  // iteration issues the same loads (the wait for one set then never covers
  // the other's loads). Values are raw; lanes past H are masked at use.
  struct VecIn {
    float h[4], ga[3], gb[3];
  };
  const int64_t stride = gridDim.x;
  // Rows are addressed through buffer resources built per vector in scalar
  // registers, with 32-bit per-lane offsets that stay fixed across vectors.
  auto load_vec = [&](int64_t v, VecIn& in) {
    const int64_t vc = v < p.nvec ? v : p.nvec - 1;
    const auto hr = raw_rsrc(vc >= p.B ? p.out + (vc - p.B) * p.so_b : p.h0 + vc * p.sh0_b);
#pragma unroll
    for (int r = 0; r < 4; ++r) in.h[r] = buf_ld(hr, 4u * (idx[r] < H ? idx[r] : H - 1), 0);
    const uint32_t t = (uint32_t)vc / (uint32_t)p.B, b = (uint32_t)vc - t * (uint32_t)p.B;  // nvec < 2^31
    const auto gr = raw_rsrc(p.gi + t * p.sg_t + b * p.sg_b);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      in.ga[q] = buf_ld(gr, 4u * kac, 4u * q * H);
      in.gb[q] = buf_ld(gr, 4u * kbc, 4u * q * H);
    }
  };
  auto coef = [&](float(&st)[7][N], const float(&gs)[3][N], int k, int kw, bool ok, const float(&gv)[3],
                  float hp) {
    const GateGrad gg = gru_backward(gv[0], gv[1], gv[2], gs[0][k], gs[1][k], gs[2][k], hp, 1.0f, p.qout);
    st[0][kw] = ok ? gg.dgr : 0.0f;
    st[1][kw] = ok ? gg.dgz : 0.0f;
    st[2][kw] = ok ? gg.dghn : 0.0f;
    st[3][kw] = ok ? gg.dgn : 0.0f;
    st[4][kw] = ok ? gg.dh_direct : 0.0f;
    st[5][kw] = ok && !(p.qin.on && !quant_keeps(hp, p.qin)) ? 1.0f : 0.0f;
    st[6][kw] = !ok ? 0.0f : p.qin.on ? fake_quant(hp, p.qin) : hp;
  };
  // (live false: nothing to store yet; the stores go to zero-size resources.
  // The Mi row is stored only when q_in is on; the recurrence reads it only then.)
  auto store_rows = [&](const float(&st)[7][N], int64_t v, bool live) {
    float* const base[3] = {g == 0 ? p.cg + v * 3 * N : g == 1 ? p.cgn + v * N : p.mi + v * N,
                            g == 0 ? p.cg + (v * 3 + 1) * N : g == 1 ? p.zm + v * N : p.hq + v * N,
                            p.cg + (v * 3 + 2) * N};
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      typedef int i4 __attribute__((ext_vector_type(4)));
      const i4 q = {__float_as_int(st[srow[j]][idx[0]]), __float_as_int(st[srow[j]][idx[1]]),
                    __float_as_int(st[srow[j]][idx[2]]), __float_as_int(st[srow[j]][idx[3]])};
      const bool keep = j < 2 ? !(g == 2 && j == 0 && !p.qin.on) : g == 0;
      __builtin_amdgcn_raw_buffer_store_b128(q, bounded_rsrc(base[j], live && keep ? 4u * N : 0u), (int)loff, 0, 0);
    }
  };
  // A vector's rows are staged in stg[own] after the gather barrier and
  // stored by the next vector, after its gather barrier (which orders the
  // staging writes before those reads); the vector after next stages into
  // the same buffer only after its own gather barrier, which every thread
  // reaches after these reads. Two barriers per vector: layers 8-9 and the
  // gather.
  auto vec = [&](int64_t v, VecIn& in, float(&gs)[3][N], float(&st)[7][N], const float(&sp)[7][N], int64_t vp,
                 bool live_prev) {
    v = v < p.nvec ? v : p.nvec - 1;  // past the end: vector nvec - 1 again, the same bits to the same places
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float hp = idx[r] < H ? in.h[r] : 0.0f;
      x[r] = p.qin.on ? fake_quant(hp, p.qin) : hp;
    }
    static_for<0, L>([&](auto S) {
      constexpr int s = S;
      if constexpr (L == 10 && s >= 8) {
        if constexpr (s == 8) {
          // lane-major (partner_of): the partners at i ^ 256, ^ 512, ^ 768 are the
          // same lane and r of waves w ^ 1, ^ 2, ^ 3
          float* xs = xch[0][g];
          const int w = idx[0] >> 8, l = idx[0] & 63;
          *reinterpret_cast<f4*>(xs + 256 * w + 4 * l) = f4{x[0], x[1], x[2], x[3]};
          lds_barrier();
          const f4 p1 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 1) + 4 * l);
          const f4 p2 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 2) + 4 * l);
          const f4 p3 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 3) + 4 * l);
#pragma unroll
          for (int r = 0; r < 4; ++r) x[r] = c8[0][r] * x[r] + c8[1][r] * p1[r] + c8[2][r] * p2[r] + c8[3][r] * p3[r];
        }
        return;  // layer 9 is folded into layer 8's exchange
      }
      float y[4];
      partner_of<s>(x, y, xch[s & 1][g], idx);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = tii[s][r] * x[r] + tip[s][r] * y[r];
      }
    });
#pragma unroll
    for (int r = 0; r < 4; ++r) gs[g][idx[r]] = x[r] + bias[r];
    // gs of this vector is read below; its next writer (the vector after
    // next) first passes the next vector's barrier, which every thread
    // reaches after these reads. The barrier also orders xch's reuse.
    lds_barrier();
    store_rows(sp, vp, live_prev);
    const float hpa = sa == 0 ? in.h[0] : sa == 1 ? in.h[1] : in.h[2];
    coef(st, gs, kac, kwa, oka, in.ga, hpa);
    if (two) coef(st, gs, kbc, kwb, okb, in.gb, in.h[3]);  // LDS writes only: no memory count depends on it
    load_vec(v + 2 * stride, in);
  };
  VecIn in0, in1;
  load_vec(blockIdx.x, in0);
  load_vec(blockIdx.x + stride, in1);
  // both vectors of a pair unconditionally, so that no branch skips memory
  // operations (see the slots above)
  int64_t v = blockIdx.x;
  for (; v < p.nvec; v += 2 * stride) {
    const int64_t vp = v - stride < p.nvec ? v - stride : p.nvec - 1;
    vec(v, in0, ghs[0], stg[0], stg[1], vp, v != (int64_t)blockIdx.x);
    vec(v + stride, in1, ghs[1], stg[1], stg[0], v, true);
  }
  lds_barrier();
  store_rows(stg[1], v - stride < p.nvec ? v - stride : p.nvec - 1, v != (int64_t)blockIdx.x);
}

struct RecParams {
  const float* tw;
  const float* dout;  // [T, B, H]
  const float* cg;    // [T B, 3, N] (Cr, Cz, Chn), lane order
  const float* zm;    // [T B, N] lane order
  const float* mi;    // [T B, N] lane order
  float* dsum;        // [T B, N] D_t, lane order
  float* dbh_part;    // [B, 3H] sum over t of D_t (Cr, Cz, Chn)
  float* dh0;         // [B, H]
  float* dcar;        // [B, H] D_{t_lo - 1} handed from one span's launch to the next
  int T, B, H;
  int t_hi, t_lo;     // this launch's steps, t_hi down to t_lo (an even count)
  int first;          // t_hi is the first step (dbh starts at 0, D from dout[T-1])
};


// One workgroup per batch row b for all T steps, the forward's wave layout.
// Per step: the gate-r waves store D_t (the twiddle gradient forms the
// step's gradients from it); each gate's waves form v_g = D_t Cg_t on their
// elements and add it to the row's dbh sum, then run the transposed layers
// from L-1 down to 0; the three gates' results meet in LDS, where every wave
// forms the carry and D_{t-1} for its own elements.
// MI: q_in is on, so Mi (q_in's mask on h_{t-1}) is read; without q_in it is
// 1 everywhere (Mi·via = via exactly) and neither loaded nor stored.
template <int LOGN, bool MI>
__global__ __launch_bounds__(3 * (1 << LOGN) / 4) void bfly_bwd_kernel(RecParams p) {
  constexpr int N = Lay<LOGN>::N, WPG = Lay<LOGN>::WPG, L = LOGN;
  __shared__ __attribute__((aligned(16))) float xch[2][3][N];
  __shared__ float ghs[2][3][N];
  // the wave index read into a scalar register, so that per-gate choices are scalar
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = wv / WPG,
            w = wv - g * WPG;
  const int H = p.H, b = blockIdx.x;
  int idx[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) idx[r] = lane + 64 * r + 256 * w;
  float tii[L][4], tpi[L][4];
  const float* tw_g = p.tw + (int64_t)g * L * (N / 2) * 4;
#pragma unroll
  for (int s = 0; s < L; ++s)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const ElemTw e = elem_tw(tw_g, N, s, idx[r]);
      tii[s][r] = e.t_ii;
      tpi[s][r] = e.t_pi;
    }
  // N = 1024: the transposed layers 9 and 8 (strides 512, 256) both cross
  // waves; they run as one exchange. With x9[j] = tii9(j) x[j] + tpi9(j) x[j^512],
  //   x8[i] = tii8 tii9(i) x[i] + tii8 tpi9(i) x[i^512] + tpi8 tii9(i^256) x[i^256]
  //         + tpi8 tpi9(i^256) x[i^768],
  // the four products formed here once (as in the forward's register kernel).
  float c89[4][4];
  if constexpr (L == 10) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const ElemTw q = elem_tw(tw_g, N, 9, idx[r] ^ 256);
      c89[0][r] = tii[8][r] * tii[9][r];
      c89[1][r] = tii[8][r] * tpi[9][r];
      c89[2][r] = tpi[8][r] * q.t_ii;
      c89[3][r] = tpi[8][r] * q.t_pi;
    }
  }
  const int64_t BH = (int64_t)p.B * H;
  // Steps run in pairs, from t_hi down to t_lo, with no condition between
  // them (a skippable second step would leave the wait at the top of the
  // loop unable to count the other set's loads). An odd T starts at the step
  // T past the end with D_T = 0: its products are zero, its gradient stores
  // are dropped (a zero-size store resource), and it forms
  // D_{T-1} = dout[T-1] + 0 as the carry. A launch covers one span of steps;
  // the next span's launch continues from D_{t_lo - 1} in dcar and from the
  // dbh sums so far.
  const int t0 = p.t_hi;
  float d[4];  // D_t of this lane's elements
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float* src = p.first ? p.dout + (int64_t)(p.T - 1) * BH + (int64_t)b * H : p.dcar + (int64_t)b * H;
    d[r] = idx[r] < H && t0 < p.T ? src[idx[r]] : 0.0f;
  }
  // The step's inputs (Cg for every gate; Zm, Mi and dout[t-1] for gate r)
  // sit in two register sets that take turns: a set is refilled, for two
  // steps ahead, after the stores of the step that used it, so the wait for
  // one set never covers the other set's loads. (With one set, loaded one
  // step ahead at the top of the step, the wait before the step's first
  // product covered the loads just issued, and each step paid a full memory
  // latency.)
  struct StepIn {
    f4 c, z, m;
    float dp[4];
  };
  // Every wave issues the same memory operations every step, in the same
  // order: its Cg row, then Zm, Mi and dout[t-1] (which only the gate-r
  // waves use; the others' loads hit the same lines), and at the start of a
  // step one store of D_t (a zero-size resource for the waves other than
  // gate r's: those stores are dropped). The compiler's wait for one set then
  // counts exactly the operations issued after it, and never covers the
  // other set's loads. Loaded values are raw: a select after a load would
  // wait for it.
  // per-lane byte offsets: of the lane's four elements in the lane-order
  // planes, and of each element in the [.., H] rows (past the resource's end
  // for lanes past H: those loads read 0 and those stores are dropped)
  const uint32_t loff = 16u * (64 * w + lane);
  uint32_t goff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) goff[r] = idx[r] < H ? 4u * idx[r] : kOffNone;
  // (pin: keep the loads in this order; the loop's loads are issued in it,
  // and the prologue's must be too, since the wait at the top of the loop
  // counts from the entry's order as well)
  auto load_step = [&](int t, StepIn& in, auto pin) {
    const int tc = t < 0 ? 0 : t < p.T ? t : p.T - 1;
    const int64_t row = (int64_t)tc * p.B + b;
    const int64_t rowp = (int64_t)(t > 0 ? t - 1 : 0) * p.B + b;
    in.c = ld_lane4(p.cg + (row * 3 + g) * N, loff);
    if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
    in.z = ld_lane4(p.zm + row * N, loff);
    if constexpr (MI) in.m = ld_lane4(p.mi + row * N, loff);
    if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
    const auto dr = bounded_rsrc(p.dout + rowp * H, 4u * H);  // 0 past H
#pragma unroll
    for (int r = 0; r < 4; ++r) in.dp[r] = buf_ld(dr, goff[r], 0);
    if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
  };
  float dbh[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) dbh[r] = idx[r] < H && !p.first ? p.dbh_part[(int64_t)b * 3 * H + g * H + idx[r]] : 0.0f;
  auto step = [&](int t, StepIn& in, float(&gs)[3][N]) {
    const bool real = t < p.T;
    const int64_t row = (int64_t)(real ? t : p.T - 1) * p.B + b;
    {
      typedef int i4 __attribute__((ext_vector_type(4)));
      const i4 dq = {__float_as_int(d[0]), __float_as_int(d[1]), __float_as_int(d[2]), __float_as_int(d[3])};
      __builtin_amdgcn_raw_buffer_store_b128(dq, bounded_rsrc(p.dsum + row * N, real && g == 0 ? 4u * N : 0u),
                                             (int)loff, 0, 0);
    }
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = real ? d[r] * in.c[r] : 0.0f;  // Cg is 0 past H
      dbh[r] += x[r];
    }
    static_for<0, L>([&](auto S) {
      constexpr int s = L - 1 - S;
      if constexpr (L == 10 && s >= 8) {
        if constexpr (s == 9) {
          // lane-major, as in the coefficient pass
          float* xs = xch[0][g];
          const int w = idx[0] >> 8, l = idx[0] & 63;
          *reinterpret_cast<f4*>(xs + 256 * w + 4 * l) = f4{x[0], x[1], x[2], x[3]};
          lds_barrier();
          const f4 p1 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 1) + 4 * l);
          const f4 p2 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 2) + 4 * l);
          const f4 p3 = *reinterpret_cast<const f4*>(xs + 256 * (w ^ 3) + 4 * l);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            x[r] = ((c89[0][r] * x[r] + c89[1][r] * p2[r]) + c89[2][r] * p1[r]) + c89[3][r] * p3[r];
        }
        return;  // layer 8 is folded into layer 9's exchange
      }
      float y[4];
      partner_of<s>(x, y, xch[S & 1][g], idx);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = tii[s][r] * x[r] + tpi[s][r] * y[r];
      }
    });
    // Every wave gathers the three gates' results for its elements and forms
    // D_{t-1} = dout[t-1] + Zm D_t + Mi (sum of the gates) itself (all waves
    // hold Zm, Mi and dout[t-1]; the same inputs give the same bits), so one
    // barrier per step serves the gather. At t = 0 the carry is dh0, stored
    // after the loop. gs alternates between two buffers with the step's
    // parity: its next writer (two steps on) passes the next step's barrier
    // first, which every wave reaches after these reads.
#pragma unroll
    for (int r = 0; r < 4; ++r) gs[g][idx[r]] = x[r];
    lds_barrier();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float via, carry;
      {
#pragma clang fp contract(off)
        via = (gs[0][idx[r]] + gs[1][idx[r]]) + gs[2][idx[r]];
        carry = in.z[r] * d[r] + (MI ? in.m[r] * via : via);
      }
      const float dn = t > 0 ? in.dp[r] + carry : carry;
      d[r] = idx[r] < H ? dn : 0.0f;
    }
    load_step(t - 2, in, std::false_type{});  // unconditional; past step 0 it reloads step 0
  };
  StepIn in0, in1;
  load_step(t0, in0, std::true_type{});
  load_step(t0 - 1, in1, std::true_type{});
  for (int t = t0; t > p.t_lo; t -= 2) {  // t0 is odd (t_hi always is)
    step(t, in0, ghs[0]);
    step(t - 1, in1, ghs[1]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (idx[r] < H) {
      p.dbh_part[(int64_t)b * 3 * H + g * H + idx[r]] = dbh[r];
      if (g == 0 && p.t_lo > 0) p.dcar[(int64_t)b * H + idx[r]] = d[r];  // D_{t_lo - 1}
      if (g == 0 && p.t_lo == 0) p.dh0[(int64_t)b * H + idx[r]] = d[r];  // step 0's carry
    }
  }
}

struct TwParams {
  const float* tw;
  const float* hq;    // [TB, N] lane order
  const float* dsum;  // [TB, N] D, lane order
  const float* cg;    // [TB, 3, N] (Cr, Cz, Chn), lane order
  const float* cgn;   // [TB, N] lane order
  float* dgi;         // [TB, 3H] D (Cr, Cz, Cgn)
  float* part;        // [3][nchunk][L][N][2]
  int64_t v_lo, v_hi; // this launch's vectors
  int nchunk, H;
  int first;          // the first launch writes part; later ones add to it
};

// Workgroup (chunk, gate) of WPG waves, the forward's lane layout: for
// vectors v = chunk, chunk + nchunk, ... the gate's gradient dgh = D Cg is
// formed and its dgi part stored (dgi_r, dgi_z, and dgi_n = D Cgn for gate n;
// the dense backward's grad_kernel products), the layers run forward on hq, each
// lane keeping its elements' activations and their partners' (a, ap) in
// registers, then dgh runs backward through the transposed layers; each lane
// accumulates its elements' two twiddle gradients per layer in registers.
template <int LOGN>
__global__ __launch_bounds__((1 << LOGN) / 4) void bfly_twiddle_grad(TwParams p) {
  constexpr int N = Lay<LOGN>::N, L = LOGN;
  __shared__ __attribute__((aligned(16))) float xch[2][N];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int chunk = blockIdx.x, g = blockIdx.y, H = p.H;
  int idx[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) idx[r] = lane + 64 * r + 256 * w;
  float tii[L][4], tip[L][4], tpi[L][4], accd[L][4], acco[L][4];
  const float* tw_g = p.tw + (int64_t)g * L * (N / 2) * 4;
#pragma unroll
  for (int s = 0; s < L; ++s)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const ElemTw e = elem_tw(tw_g, N, s, idx[r]);
      tii[s][r] = e.t_ii;
      tip[s][r] = e.t_ip;
      tpi[s][r] = e.t_pi;
      accd[s][r] = acco[s][r] = 0.0f;
    }
  // A vector's inputs (its hq row and its gradient row) sit in two register
  // sets that take turns, each refilled for the vector after next once used,
  // at clamped addresses so that every iteration issues the same loads; the
  // wait for one set then never covers the other's loads. (Loaded at the top
  // of each vector's iteration, every vector paid a full memory latency.)
  struct VecIn {
    f4 h, d, c, n;
  };
  const uint32_t loff = 16u * (64 * w + lane);
  uint32_t goff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) goff[r] = idx[r] < H ? 4u * idx[r] : kOffNone;
  // (pin: keep the loads in this order, as the loop issues them; the wait at
  // the top of the loop counts from the entry's order as well)
  auto load_vec = [&](int64_t v, VecIn& in, auto pin) {
    const int64_t vc = v < p.v_hi ? v : p.v_hi - 1;
    in.h = ld_lane4(p.hq + vc * N, loff);  // lane-order planes: 0 past H
    if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
    in.d = ld_lane4(p.dsum + vc * N, loff);
    in.c = ld_lane4(p.cg + (vc * 3 + g) * N, loff);
    in.n = ld_lane4(p.cgn + vc * N, loff);  // used by gate n only
    if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
  };
  // A vector past the end of the span (the second of the last pair) repeats
  // the span's last vector: its dgi stores put the same bits in the same
  // places, and its gradient is zeroed, so it adds nothing to the sums. So
  // both vectors of a pair run unconditionally and no branch skips memory
  // operations.
  auto vec = [&](int64_t v, VecIn& in) {
    // (no instruction moves into another vector's code: the scheduler would
    // otherwise hoist the next vector's products above the wait for its set)
    __builtin_amdgcn_sched_barrier(0);
    const bool live = v < p.v_hi;
    v = live ? v : p.v_hi - 1;
    float a[L][4], ap[L][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a[0][r] = in.h[r];
    static_for<0, L>([&](auto S) {
      constexpr int s = S;
      partner_of<s>(a[s], ap[s], xch[s & 1], idx);
      if constexpr (s + 1 < L) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          a[s + 1][r] = tii[s][r] * a[s][r] + tip[s][r] * ap[s][r];
        }
      }
    });
    float gv[4];
    const auto gr = bounded_rsrc(p.dgi + v * 3 * H + g * H, 4u * H);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float dg = in.d[r] * in.c[r];
      buf_st(gr, goff[r], 0, g == 2 ? in.d[r] * in.n[r] : dg);
      gv[r] = live ? dg : 0.0f;
    }
    static_for<0, L>([&](auto S) {
      constexpr int s = L - 1 - S;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        accd[s][r] += gv[r] * a[s][r];
        acco[s][r] += gv[r] * ap[s][r];
      }
      if constexpr (s > 0) {
        // buffer (s + 1) & 1: never the one the last forward layer (L - 1)
        // used, whose reads no barrier separates from this write
        float y[4];
        partner_of<s>(gv, y, xch[(s + 1) & 1], idx);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          gv[r] = tii[s][r] * gv[r] + tpi[s][r] * y[r];
        }
      }
    });
    lds_barrier();  // the next vector's exchanges reuse xch
    load_vec(v + 2 * (int64_t)p.nchunk, in, std::false_type{});
  };
  VecIn in0, in1;
  load_vec(p.v_lo + chunk, in0, std::true_type{});
  load_vec(p.v_lo + chunk + p.nchunk, in1, std::true_type{});
  for (int64_t v = p.v_lo + chunk; v < p.v_hi; v += 2 * (int64_t)p.nchunk) {
    vec(v, in0);
    vec(v + p.nchunk, in1);
  }
  float2* out = reinterpret_cast<float2*>(p.part) + ((int64_t)g * p.nchunk + chunk) * L * N;
#pragma unroll
  for (int s = 0; s < L; ++s)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float2 o = make_float2(accd[s][r], acco[s][r]);
      if (!p.first) {
        const float2 q = out[(int64_t)s * N + idx[r]];
        o.x += q.x;
        o.y += q.y;
      }
      out[(int64_t)s * N + idx[r]] = o;
    }
}

// dtw[g][0][s][pair][m][*] from the chunk sums of element i = the element
// with that pair and m. A workgroup takes 64 consecutive elements of one
// gate's [L][N] (coalesced float2 loads); its four waves sum the chunks
// c = ph mod 4 in a fixed order and the four partial sums are added in a
// fixed order (deterministic; each thread used to walk all chunks alone,
// latency bound: 104 us at config 4).
constexpr int kTwSumPhases = 4;
__global__ __launch_bounds__(64 * kTwSumPhases) void bfly_twiddle_sum(const float* part, float* dtw, int nchunk,
                                                                    int N, int L) {
  __shared__ float2 red[kTwSumPhases][64];
  const int64_t per_gate = (int64_t)L * N;
  const int o = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t e = (int64_t)blockIdx.x * 64 + o;
  const bool ok = e < 3 * per_gate;
  const int g = ok ? (int)(e / per_gate) : 0;
  const int64_t r = ok ? e - g * per_gate : 0;
  float sd = 0.0f, so = 0.0f;
  if (ok) {
    const float2* src = reinterpret_cast<const float2*>(part) + ((int64_t)g * nchunk * per_gate + r);
    for (int c = ph; c < nchunk; c += kTwSumPhases) {
      const float2 v = src[(int64_t)c * per_gate];
      sd += v.x;
      so += v.y;
    }
  }
  red[ph][o] = make_float2(sd, so);
  __syncthreads();
  if (ph != 0 || !ok) return;
#pragma unroll
  for (int k = 1; k < kTwSumPhases; ++k) {
    sd += red[k][o].x;
    so += red[k][o].y;
  }
  const int s = (int)(r / N), i = (int)(r - (int64_t)s * N);
  const int m = (i >> s) & 1;
  const int pair = ((i >> (s + 1)) << s) | (i & ((1 << s) - 1));
  float* d = dtw + (int64_t)g * L * (N / 2) * 4 + ((int64_t)s * (N / 2) + pair) * 4 + 2 * m;
  d[m] = sd;
  d[1 - m] = so;
}

struct NativePlan {
  bool ok = false;
  int nchunk = 0;
  int64_t hq, cg, lplane, part, dcar;
  int64_t scratch() const { return hq + cg + 4 * lplane + part + dcar; }  // no tagged words
};

// Twiddle-gradient workgroups per gate. 3 x 64 = 192 one-per-CU workgroups
// leave 64 of the 256 CUs to the recurrence's one-per-CU row workgroups
// (B = 64 at the headline shape), so the two run side by side.
constexpr int kTwChunks = 64;
// The recurrence runs in up to kSpans launches of an even number of steps
// each; the twiddle gradient of a span runs on a second stream while the
// recurrence works on the next span.
constexpr int kSpans = 8;

NativePlan plan_native(const gs_bwd_args* a) {
  NativePlan pl;
  // The stage-wise kernels hold one chain's twiddles in registers: one chain,
  // N = 2^log_n in {256, 512, 1024} (the forward's register-kernel shapes).
  if (a->bfly_nblocks != 1 || a->log_n < 8 || a->log_n > 10) return pl;
  const int N = 1 << a->log_n;
  const int64_t H = a->H, TB = a->T * a->B;
  if (N < H || TB >= ((int64_t)1 << 31)) return pl;
  pl.nchunk = kTwChunks;
  pl.hq = align256(TB * N * 4);
  pl.cg = align256(TB * 3 * N * 4);
  pl.lplane = align256(TB * N * 4);
  pl.part = align256((int64_t)3 * pl.nchunk * 2 * a->log_n * N * 4);
  pl.dcar = align256(a->B * H * 4);
  pl.ok = true;
  return pl;
}

// A second stream per device for the twiddle gradient, and the events that
// order it after each span of the recurrence (created on first use with the
// device current; default priority). `mu` serializes the calls that use
// them. When they cannot be created, everything runs on the caller's stream.
struct Side {
  std::mutex mu;
  bool tried = false;
  hipStream_t s = nullptr;
  hipEvent_t ev[kSpans + 1] = {};
};
Side g_side[64];

Side* side_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  Side& sd = g_side[dev];
  std::lock_guard<std::mutex> lk(sd.mu);
  if (!sd.tried) {
    sd.tried = true;
    bool ok = hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) == hipSuccess;
    for (int k = 0; ok && k <= kSpans; ++k) ok = hipEventCreateWithFlags(&sd.ev[k], hipEventDisableTiming) == hipSuccess;
    if (!ok) sd.s = nullptr;
    (void)hipGetLastError();
  }
  return sd.s != nullptr ? &sd : nullptr;
}

template <int LOGN>
int launch_stages(const gs_bwd_args* a, const NativePlan& pl, float* hq, float* cg, float* cgn, float* zm, float* mi,
                  float* dsum, float* part, float* dcar, hipStream_t stream) {
  constexpr int NT3 = 3 * (1 << LOGN) / 4;
  const int T = (int)a->T, B = (int)a->B, H = (int)a->H;
  const int64_t TB = (int64_t)T * B;
  CoefParams cp;
  cp.tw = a->w;
  cp.bh = a->bh;
  cp.gi = a->gi;
  cp.h0 = a->h0;
  cp.out = a->out;
  cp.hq = hq;
  cp.cg = cg;
  cp.cgn = cgn;
  cp.zm = zm;
  cp.mi = mi;
  cp.sg_t = a->sg_t;
  cp.sg_b = a->sg_b;
  cp.sh0_b = a->sh0_b;
  cp.so_b = a->so_b;
  cp.nvec = TB;
  cp.B = B;
  cp.H = H;
  cp.qin = to_quant(a->q_in);
  cp.qout = to_quant(a->q_out);
  hipLaunchKernelGGL(bfly_apply_coef<LOGN>, dim3((unsigned)std::min<int64_t>(TB, 2048)), dim3(NT3), 0, stream, cp);
  GS_CHECK_HIP(hipGetLastError());
  RecParams rp;
  rp.tw = a->w;
  rp.dout = a->dout;
  rp.cg = cg;
  rp.zm = zm;
  rp.mi = mi;
  rp.dsum = dsum;
  rp.dbh_part = a->dbh_part;
  rp.dh0 = a->dh0;
  rp.dcar = dcar;
  rp.T = T;
  rp.B = B;
  rp.H = H;
  TwParams tp;
  tp.tw = a->w;
  tp.hq = hq;
  tp.dsum = dsum;
  tp.cg = cg;
  tp.cgn = cgn;
  tp.dgi = a->dgi;
  tp.part = part;
  tp.nchunk = pl.nchunk;
  tp.H = H;
  // Spans of the step range t0 .. 0 (t0 = T - 1, or T for an odd T: see the
  // recurrence), each an even number of steps, latest first.
  const int t0 = (T & 1) ? T : T - 1;
  const int nsteps = t0 + 1;
  const int span = (((nsteps + kSpans - 1) / kSpans) + 1) & ~1;
  Side* sd = side_for_current_device();
  std::unique_lock<std::mutex> lk;
  if (sd != nullptr) lk = std::unique_lock<std::mutex>(sd->mu);
  hipStream_t tws = sd != nullptr ? sd->s : stream;
  // Once the second stream has work of this call, the caller's stream waits
  // for all of it on every way out, an error return included, so that nothing
  // of this call runs after the caller may reuse its buffers.
  bool forked = false;
  struct Join {
    Side* sd;
    hipStream_t stream;
    const bool& forked;
    ~Join() {
      if (sd == nullptr || !forked) return;
      if (hipEventRecord(sd->ev[kSpans], sd->s) == hipSuccess) (void)hipStreamWaitEvent(stream, sd->ev[kSpans], 0);
    }
  } join{sd, stream, forked};
  int k = 0;
  for (int hi = t0; hi >= 0; hi -= span, ++k) {
    const int lo = std::max(hi - span + 1, 0);
    rp.t_hi = hi;
    rp.t_lo = lo;
    rp.first = hi == t0;
    if (cp.qin.on)
      hipLaunchKernelGGL((bfly_bwd_kernel<LOGN, true>), dim3((unsigned)B), dim3(NT3), 0, stream, rp);
    else
      hipLaunchKernelGGL((bfly_bwd_kernel<LOGN, false>), dim3((unsigned)B), dim3(NT3), 0, stream, rp);
    GS_CHECK_HIP(hipGetLastError());
    if (sd != nullptr) {
      GS_CHECK_HIP(hipEventRecord(sd->ev[k], stream));
      GS_CHECK_HIP(hipStreamWaitEvent(tws, sd->ev[k], 0));
      forked = true;
    }
    tp.v_lo = (int64_t)lo * B;
    tp.v_hi = (int64_t)(std::min(hi, T - 1) + 1) * B;
    tp.first = hi == t0;
    hipLaunchKernelGGL(bfly_twiddle_grad<LOGN>, dim3((unsigned)pl.nchunk, 3), dim3((1 << LOGN) / 4), 0, tws, tp);
    GS_CHECK_HIP(hipGetLastError());
  }
  if (sd != nullptr) {
    GS_CHECK_HIP(hipEventRecord(sd->ev[kSpans], tws));
    GS_CHECK_HIP(hipStreamWaitEvent(stream, sd->ev[kSpans], 0));
    forked = false;  // joined
  }
  const int64_t nsum = (int64_t)3 * LOGN * (1 << LOGN);
  hipLaunchKernelGGL(bfly_twiddle_sum, dim3((unsigned)((nsum + 63) / 64)), dim3(64 * kTwSumPhases), 0, stream, part,
                     a->dw_part, pl.nchunk, 1 << LOGN, LOGN);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace

int64_t butterfly_bwd_workspace_bytes(const gs_bwd_args* a) {
  const NativePlan pl = plan_native(a);
  if (pl.ok) return 0;
  return struct_bwd_workspace_bytes(GS_KIND_BUTTERFLY, a);
}

int64_t butterfly_bwd_scratch_bytes(const gs_bwd_args* a) {
  const NativePlan pl = plan_native(a);
  if (pl.ok) return pl.scratch();
  return struct_bwd_scratch_bytes(GS_KIND_BUTTERFLY, a);
}

}  // namespace gs

extern "C" int gs_butterfly_bwd(const gs_bwd_args* a, hipStream_t stream) {
  using namespace gs;
  const char* who = "gs_butterfly_bwd";
  clear_error();
  int rc = validate_bwd_common(a, who);
  if (rc) return rc;
  const NativePlan pl = plan_native(a);
  if (!pl.ok) return run_struct(GS_KIND_BUTTERFLY, a, stream, who);
  if (a->dw_part == nullptr) return set_error(GS_ERR_INVALID, "%s: dw_part must be a non-NULL device pointer", who);
  if (a->w2 != nullptr) return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the butterfly kind", who);
  if (a->T > 1 && a->so_t != a->B * a->so_b)
    return set_error(GS_ERR_INVALID, "%s: out must hold its steps back to back (so_t == B * so_b); got so_t=%lld, so_b=%lld",
                     who, (long long)a->so_t, (long long)a->so_b);
  rc = check_scratch(a, pl.scratch(), who);
  if (rc) return rc;

  char* cur = static_cast<char*>(a->scratch);
  auto take = [&](int64_t bytes) {
    char* r = cur;
    cur += bytes;
    return reinterpret_cast<float*>(r);
  };
  float* hq = take(pl.hq);
  float* cg = take(pl.cg);
  float* cgn = take(pl.lplane);
  float* zm = take(pl.lplane);
  float* mi = take(pl.lplane);
  float* dsum = take(pl.lplane);
  float* part = take(pl.part);
  float* dcar = take(pl.dcar);

  switch (a->log_n) {
    case 8: return launch_stages<8>(a, pl, hq, cg, cgn, zm, mi, dsum, part, dcar, stream);
    case 9: return launch_stages<9>(a, pl, hq, cg, cgn, zm, mi, dsum, part, dcar, stream);
    default: return launch_stages<10>(a, pl, hq, cg, cgn, zm, mi, dsum, part, dcar, stream);
  }
}
