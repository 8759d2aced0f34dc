// Barrier-free dense GRU scan (gfx950): one workgroup per tile of batch rows
// runs every step of its rows and reads Wh from memory each step, so no
// workgroup ever waits for another.
//
// References (LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py):
//   forward   gru_scan_fwd_kernel :755-913, launched by gru_scan_forward :1688-1765
//   backward  gru_scan_bwd_kernel :916-1352, launched by gru_scan_backward_triton :1355-1447
// Like those kernels the grid is 1-D over batch tiles and has no co-residency
// requirement, no workspace and no bound on H beyond what a workgroup's LDS
// holds. The persistent kernels (scan_dense.hip, scan_dense_bwd.hip) keep Wh
// resident and exchange the state between workgroups every step; they are the
// fast path up to H = 1024. These kernels serve gru_scan / gru_scan_forward by
// name, and every dense recurrence with H > 1024 (gs_dense_fwd, gs_dense_bwd and
// the materialized-map backwards of the structured kinds).
//
// Work split. A workgroup of 8 waves owns BT <= 4 batch rows. Per step each
// wave takes quads of 4 hidden units (quad q, q + 8, ...) and forms their 3
// gates' products with v_mfma_f32_4x4x1_16b_f32 chains exactly as the
// persistent kernels do (A = the 4 staged rows from LDS, B = 4 weight rows,
// the 16 MFMA blocks as 16 K slices, two accumulators alternating by
// instruction, reduce16), so the products, and the gate epilogue after them,
// are bit for bit those of the persistent kernels. The weights reach the MFMA
// through an LDS transpose (forward) or a copy in operand order (backward), so
// that every load instruction reads contiguous memory.
// Then an LDS barrier, a pass that stages the next step's operand rows from
// the new state, and a second barrier.
//
// Bound: each workgroup streams the whole of Wh (3 H^2 floats) from L2 or
// memory every step through one CU's texture addresser (about 64 bytes per
// clock for contiguous 16-byte lanes), so a step takes at least 3 H^2 4 / 64
// clocks whatever BT is (BT only sets how many CUs work).
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kTileWaves = 8;  // forward (its LDS weight staging takes 6.9 KiB per wave)
constexpr int kTileThreads = 64 * kTileWaves;
constexpr int kBwdWaves = 16;  // backward recurrence (measured 3.04 ms with 8 waves, 2.36 ms with 16)
constexpr int kBwdThreads = 64 * kBwdWaves;
// LDS a workgroup may take (gfx950: 160 KiB per CU).
constexpr int64_t kTileLdsMax = 160 * 1024;
// Backward: K chunks of 64 whose loads a wave issues together
constexpr int kUnroll = 4;

struct TFParams {
  const float* gi;
  const float* h0;
  const float* w;  // [3H, H]
  const float* bh;
  float* out;
  float* gh_save;  // SAVE: [T, B, 3H] q_in(h_{t-1}) Wh^T (no bias)
  const int8_t* wq;  // I8: int8 codes of Wh [3H, H], w == fl(code * wsc[row])
  const float* wsc;  // I8: the code scale of each of Wh's 3H rows
  float pscale;      // I8: q_in's scale (the staged state is q_in levels)
  int rsi;           // I8: LDS row stride of the staged levels, words (16 mod 64)
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int BT;   // batch rows per workgroup
  int nch;  // K chunks of 64
  int rs;   // LDS row stride of the staged rows: 64 nch + 16 (16 mod 64: conflict-free operand reads)
  int hr;   // LDS row stride of the raw state
  Quant qin, qout;
  int qin_after_first;
};

// Forward weight staging. The MFMA's B operand puts 4 different units (rows of
// Wh) on every 4 adjacent lanes, and loading it in place spans 4 rows per group
// of 4 lanes, which the texture addresser serves at about 14 bytes per clock.
// So a wave loads an item (KI = 128 consecutive k of the 12 rows of its quad:
// 3 gates x 4 units) with 32 lanes per row (512 contiguous bytes each half
// wave), writes it to a wave-private LDS buffer and reads the operands back in
// MFMA order; the next item's loads are in flight meanwhile. The buffer holds
// 12 rows of kItemK floats with a stride of 16 mod 64 floats: the 16-byte
// stores (8 lanes a pass, 128 contiguous bytes) and the operand reads (lanes
// 4 b + j at row j, 4 b, rows 16 banks apart) are free of bank conflicts.
constexpr int kItemK = 128;           // k per item: 2 chunks of 64
constexpr int kItemRS = kItemK + 16;  // LDS row stride of the staging buffer (floats)
constexpr int kItemFloats = 12 * kItemRS;
constexpr int kItemLoads = 6;         // 12 rows, 2 per load instruction
// items whose loads are in flight: 3 for 16-byte loads; the scalar path holds
// 4 addresses per float4 and spills at 3
template <bool VEC> constexpr int kFwdDepth = VEC ? 3 : 2;

// Int8 weights (I8): the products of gs_dense_fwd_i8w's persistent instance
// (scan_dense.hip) on the same item pipeline. The state is staged as q_in
// levels (word c of a row holds k = 4 c .. 4 c + 3, one byte each), an item is
// 512 k of the quad's 12 code rows (the same 6 KiB of 16-byte loads and the
// same staging buffer as 128 k of fp32), and each 64-k chunk is one
// v_mfma_i32_4x4x4_16b_i8 per gate. The integer sums are exact, reduced in
// integers, and gh = sum * (row scale * q_in scale): bit for bit the persistent
// instance's gh wherever it runs (K <= 1024, sums within 2^24).
template <bool VEC, bool SAVE, bool I8 = false>
__global__ __launch_bounds__(kTileThreads) void tiled_fwd_kernel(TFParams p) {
  static_assert(!I8 || (VEC && !SAVE), "int8 weights: 16-byte code loads, no saved gh");
  constexpr int IK = I8 ? 4 * kItemK : kItemK;  // k per item
  constexpr int ICH = IK / 64;                  // 64-k chunks per item
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = p.H, BT = p.BT, rs = p.rs, hr = p.hr;
  const int r = lane & 3, kb = lane >> 2;          // MFMA A row, K slice
  const int j = lane & 3, s = (lane >> 2) & 3;     // epilogue: unit of the quad, row (lanes < 16)
  const bool lead = lane < 16;
  const int row0 = blockIdx.x * BT;
  float* hq = lds;                   // [BT][rs] staged q_in(h_{t-1}), zero from H on
  float* hraw = hq + BT * rs;        // [BT][hr] raw h_{t-1}
  float* wbuf = hraw + BT * hr + wave * kItemFloats;  // this wave's weight staging buffer

  int* hqi = reinterpret_cast<int*>(hq);  // I8: [BT][rsi] staged q_in levels, zero from H on
  if constexpr (I8) {
    for (int i = threadIdx.x; i < BT * p.rsi; i += kTileThreads) {
      const int rr = i / p.rsi, c = i - rr * p.rsi, row = row0 + rr;
      uint32_t wd = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = 4 * c + e;
        if (k < H && row < p.B)
          wd |= ((uint32_t)(int)quant_level(p.h0[(int64_t)row * p.sh0_b + k], p.qin) & 0xffu) << (8 * e);
      }
      hqi[i] = (int)wd;
    }
  } else {
    for (int i = threadIdx.x; i < BT * rs; i += kTileThreads) {
      const int rr = i / rs, k = i - rr * rs, row = row0 + rr;
      float v = 0.0f;
      if (k < H && row < p.B) {
        v = p.h0[(int64_t)row * p.sh0_b + k];
        if (p.qin.on) v = fake_quant(v, p.qin);
      }
      hq[i] = v;
    }
  }
  for (int i = threadIdx.x; i < BT * hr; i += kTileThreads) {
    const int rr = i / hr, k = i - rr * hr, row = row0 + rr;
    hraw[i] = (k < H && row < p.B) ? p.h0[(int64_t)row * p.sh0_b + k] : 0.0f;
  }
  lds_barrier();

  constexpr float kR = -kLog2e, kN = 2.0f * kLog2e;
  const int nq = (H + 3) >> 2;
  const bool a_ok = r < BT;
  const float* arow = hq + (a_ok ? r : 0) * rs + 4 * kb;
  const int* arowi = hqi + (a_ok ? r : 0) * p.rsi + kb;  // I8: word 16 c of chunk c
  const int64_t HH = (int64_t)H * H;
  const int row = row0 + s;
  const bool row_ok = lead && s < BT && row < p.B;
  const int row_c = min(row0 + (s < BT ? s : 0), p.B - 1);  // gate-input row, clamped to a valid one
  // staging: load instruction i of an item covers rows 2 i + lane / 32 (row = 4 g + unit), 4 floats
  // of k at kl = 4 (lane mod 32); operand reads: row 4 g + j, k = 64 c + 4 kb
  const int kl = 4 * (lane & 31), rh = lane >> 5;
  float* wst = wbuf + rh * kItemRS + kl;        // + 2 i kItemRS for load instruction i
  const float* wop = wbuf + j * kItemRS + 4 * kb;  // + 4 g kItemRS + 64 c for gate g, chunk c
  const int* wopi = reinterpret_cast<const int*>(wbuf) + j * kItemRS + kb;  // I8: + 4 g kItemRS + 16 c
  const int myq = wave < nq ? (nq - 1 - wave) / kTileWaves + 1 : 0;
  const int nbat = (H + IK - 1) / IK;   // items per quad
  const int nit = myq * nbat;
  for (int t = 0; t < p.T; ++t) {
    const float* git = p.gi + (int64_t)t * p.sg_t + (int64_t)row_c * p.sg_b;
    // Item (q, b): k in [b IK, (b + 1) IK) of quad q's 12 rows, loaded
    // coalesced into registers; also the quad's gate inputs and biases (raw),
    // and for I8 the rows' code scales times q_in's scale.
    struct Item {
      f4 w[kItemLoads];
      float g[3], bb[3], sc[I8 ? 3 : 1];
    };
    auto load = [&](int q, int b, Item& it) {
#pragma unroll
      for (int i = 0; i < kItemLoads; ++i) {
        const int rr = 2 * i + rh, g = rr >> 2, u = 4 * q + (rr & 3);
        const int k = b * IK + (I8 ? 4 * kl : kl);  // I8: byte k, 16 codes a lane
        const bool ok = u < H && k < H;
        const int64_t off = g * HH + (int64_t)(u < H ? u : H - 1) * H + k;
        if constexpr (I8) {
          typedef int i4v __attribute__((ext_vector_type(4)));
          const i4v v = *reinterpret_cast<const i4v*>(p.wq + (ok ? off : 0));
          const f4 bits = __builtin_bit_cast(f4, v);  // staged as raw words
          it.w[i] = ok ? bits : f4{0.f, 0.f, 0.f, 0.f};
        } else if constexpr (VEC) {
          const f4 v = *reinterpret_cast<const f4*>(p.w + (ok ? off : 0));
          it.w[i] = ok ? v : f4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool in = u < H && k + e < H;
            const float x = p.w[in ? off + e : 0];
            it.w[i][e] = in ? x : 0.0f;
          }
        }
      }
      const int uc = min(4 * q + j, H - 1);
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        it.g[g] = git[g * H + uc];
        it.bb[g] = p.bh[g * H + uc];
        if constexpr (I8) it.sc[g] = p.wsc[g * H + uc] * p.pscale;
      }
    };
    f4 p0[3], p1[3];
    i4 n0[3], n1[3];  // I8 accumulators
    // one item: stage its weights, its MFMAs, and after a quad's last item the
    // reduction and the gate epilogue (the staging buffer is this wave's alone,
    // and a wave's LDS accesses complete in order, so no barrier is needed)
    auto run = [&](int q, int b, const Item& it) {
#pragma unroll
      for (int i = 0; i < kItemLoads; ++i) *reinterpret_cast<f4*>(wst + 2 * i * kItemRS) = it.w[i];
      if (b == 0) {
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          p0[g] = p1[g] = f4{0.f, 0.f, 0.f, 0.f};
          n0[g] = n1[g] = i4{0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int ci = 0; ci < ICH; ++ci) {
        const int c = b * ICH + ci;
        if (c >= p.nch) break;  // uniform
        if constexpr (I8) {
          const int a = a_ok ? arowi[16 * c] : 0;
#pragma unroll
          for (int g = 0; g < 3; ++g) {
            const int wv = wopi[4 * g * kItemRS + 16 * ci];
            if (ci & 1)
              n1[g] = __builtin_amdgcn_mfma_i32_4x4x4i8(a, wv, n1[g], 0, 0, 0);
            else
              n0[g] = __builtin_amdgcn_mfma_i32_4x4x4i8(a, wv, n0[g], 0, 0, 0);
          }
        } else {
          const f4 a = a_ok ? *reinterpret_cast<const f4*>(arow + 64 * c) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int g = 0; g < 3; ++g) {
            const f4 wv = *reinterpret_cast<const f4*>(wop + 4 * g * kItemRS + 64 * ci);
            p0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[0], wv[0], p0[g], 0, 0, 0);
            p1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[1], wv[1], p1[g], 0, 0, 0);
            p0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[2], wv[2], p0[g], 0, 0, 0);
            p1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[3], wv[3], p1[g], 0, 0, 0);
          }
        }
      }
      if (b != nbat - 1) return;
      float gh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        if constexpr (I8)
          gh[g] = (float)reduce16_i(n0[g] + n1[g], s) * it.sc[g];
        else
          gh[g] = reduce16(p0[g] + p1[g], s);
      }
      const int u = 4 * q + j;
      if (row_ok && u < H) {
        float* hp = hraw + s * hr + u;
        const float cr = __builtin_fmaf(kR, it.g[0], kR * it.bb[0]);
        const float cz = __builtin_fmaf(kR, it.g[1], kR * it.bb[1]), an2 = kN * it.g[2];
        float hn = gru_update_l2(__builtin_fmaf(kR, gh[0], cr), __builtin_fmaf(kR, gh[1], cz),
                                 __builtin_fmaf(kN, gh[2], kN * it.bb[2]), an2, *hp);
        if (p.qout.on) hn = fake_quant(hn, p.qout);
        *hp = hn;  // only this lane reads or writes this (row, unit) during the step
        p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + u] = hn;
        if constexpr (SAVE) {
          float* o = p.gh_save + ((int64_t)t * p.B + row) * 3 * H + u;
#pragma unroll
          for (int g = 0; g < 3; ++g) __builtin_nontemporal_store(gh[g], o + g * H);
        }
      }
    };
    // item m is quad wave + kTileWaves (m / nbat), part m mod nbat; kD items
    // are in flight, in register sets that rotate at compile time
    auto quad_of = [&](int m) { return wave + kTileWaves * (m / nbat); };
    constexpr int kD = kFwdDepth<VEC>;
    Item buf[kD];
    static_for<0, kD - 1>([&](auto I) {
      if (I < nit) load(quad_of(I), I % nbat, buf[I]);
    });
    for (int n = 0; n < nit; n += kD) {
      static_for<0, kD>([&](auto I) {
        const int m = n + I;
        if (m < nit) {
          const int ml = m + kD - 1;
          if (ml < nit) load(quad_of(ml), ml % nbat, buf[(I + kD - 1) % kD]);
          run(quad_of(m), m % nbat, buf[I]);
        }
      });
    }
    lds_barrier();
    if (t + 1 < p.T) {
      if constexpr (I8) {
        // q_in levels of the new state (of q_out's value when q_in repeats q_out: the same level)
        const int nw = H >> 2;
        for (int i = threadIdx.x; i < BT * nw; i += kTileThreads) {
          const int rr = i / nw, c = i - rr * nw;
          const float* hv = hraw + rr * hr + 4 * c;
          uint32_t wd = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) wd |= ((uint32_t)(int)quant_level(hv[e], p.qin) & 0xffu) << (8 * e);
          hqi[rr * p.rsi + c] = (int)wd;
        }
      } else {
        for (int i = threadIdx.x; i < BT * H; i += kTileThreads) {
          const int rr = i / H, k = i - rr * H;
          float v = hraw[rr * hr + k];
          if (p.qin_after_first) v = fake_quant(v, p.qin);
          hq[rr * rs + k] = v;
        }
      }
      lds_barrier();
    }
  }
}

// Backward recurrence (the dense backward's step 3, scan_dense_bwd.hip):
//   D_{t-1} = dout[t-1] + Zm_t D_t + Mi_t (dgh_t Wh),   dgh_t = D_t (Cr, Cz, Chn)_t,
//   dh0 = Zm_0 D_0 + Mi_0 (dgh_0 Wh),
// with Wh read from a copy in the MFMA operand order (wl, written once per call
// by lane_order_kernel): the float4 that lane l of a wave needs for quad q and
// reduction chunk cc (over the 3H rows, 64 per chunk) sits at
// wl[((q 3 nch + cc) 64 + l) 4], so every load instruction of a wave reads 1 KiB
// of contiguous memory. (Read in place, lanes 4 b + j hold 4 different columns
// of Wh: each group of 4 adjacent lanes spans 4 rows of the transposed matrix,
// which the texture addresser serves at about 14 bytes per clock, the kernel's
// bound when first measured: TA_TA_BUSY ~93 % of the kernel's cycles.)
struct TBParams {
  const float* wl;    // [nq][3 nch][64][4], zero past H
  const float* dout;  // [T, B, H] contiguous
  const float* cg;    // [T, B, 3H] (Cr, Cz, Chn)
  const float* zm;    // [T, B, H]
  const float* mi;    // [T, B, H]
  float* dsum;        // [T, B, H] D_t
  float* dh0;         // [B, H]
  int T, B, H, BT, nch, rs, hr;
};

__global__ __launch_bounds__(kBwdThreads) void tiled_bwd_kernel(TBParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = p.H, BT = p.BT, rs = p.rs, hr = p.hr, T = p.T;
  const int r = lane & 3, kb = lane >> 2;
  const int j = lane & 3, s = (lane >> 2) & 3;
  const bool lead = lane < 16;
  const int row0 = blockIdx.x * BT;
  const int64_t BH = (int64_t)p.B * H;
  float* dg = lds;                  // [3][BT][rs] staged dgh_t, zero from H on
  float* dd = dg + 3 * BT * rs;     // [BT][hr] D_t

  // D_{T-1} = dout[T-1]
  for (int i = threadIdx.x; i < 3 * BT * rs; i += kBwdThreads) dg[i] = 0.0f;
  for (int i = threadIdx.x; i < BT * hr; i += kBwdThreads) {
    const int rr = i / hr, k = i - rr * hr, row = row0 + rr;
    float D = 0.0f;
    if (k < H && row < p.B) {
      const int64_t e = (int64_t)(T - 1) * BH + (int64_t)row * H + k;
      D = p.dout[e];
      p.dsum[e] = D;
    }
    dd[i] = D;
  }
  lds_barrier();

  const int nq = (H + 3) >> 2;
  const bool a_ok = r < BT;
  const int row = row0 + s;
  const bool row_ok = lead && s < BT && row < p.B;
  const int H3 = 3 * H;
  const int nk = 3 * p.nch;
  for (int st = 0; st < T; ++st) {
    const int t = T - 1 - st;
    // stage dgh_t = D_t (Cr, Cz, Chn)_t
    for (int i = threadIdx.x; i < BT * H; i += kBwdThreads) {
      const int rr = i / H, k = i - rr * H, rw = row0 + rr;
      if (rw < p.B) {
        const float D = dd[rr * hr + k];
        const float* c = p.cg + ((int64_t)t * p.B + rw) * H3 + k;
        float* d = dg + rr * rs + k;
        d[0] = D * c[0];
        d[BT * rs] = D * c[H];
        d[2 * BT * rs] = D * c[2 * H];
      }
    }
    lds_barrier();
    for (int q = wave; q < nq; q += kBwdWaves) {
      const int u = 4 * q + j;
      const bool u_ok = u < H;
      const bool mine = row_ok && u_ok;
      float zm = 0.f, mi = 0.f, dprev = 0.f;
      if (mine) {
        const int64_t e = (int64_t)t * BH + (int64_t)row * H + u;
        zm = p.zm[e];
        mi = p.mi[e];
        if (t > 0) dprev = p.dout[e - BH];
      }
      const f4* wq = reinterpret_cast<const f4*>(p.wl) + (int64_t)q * nk * 64 + lane;  // chunk cc at + 64 cc
      f4 acc0 = f4{0.f, 0.f, 0.f, 0.f}, acc1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        const float* arow = dg + (g * BT + (a_ok ? r : 0)) * rs + 4 * kb;
        const f4* wg = wq + (int64_t)g * p.nch * 64;
        for (int c0 = 0; c0 < p.nch; c0 += 2 * kUnroll) {
          f4 a[2 * kUnroll], wv[2 * kUnroll];
#pragma unroll
          for (int i = 0; i < 2 * kUnroll; ++i) {
            const int c = c0 + i;
            const bool in = c < p.nch;  // uniform
            a[i] = (in && a_ok) ? *reinterpret_cast<const f4*>(arow + 64 * c) : f4{0.f, 0.f, 0.f, 0.f};
            wv[i] = in ? wg[64 * c] : f4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int i = 0; i < 2 * kUnroll; ++i) {
            if (c0 + i >= p.nch) break;  // uniform
            acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][0], wv[i][0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][1], wv[i][1], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][2], wv[i][2], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][3], wv[i][3], acc1, 0, 0, 0);
          }
        }
      }
      const float via_w = reduce16(acc0 + acc1, s);
      if (mine) {
        float* dp = dd + s * hr + u;
        float carry;
        {
#pragma clang fp contract(off)
          carry = zm * *dp + mi * via_w;
        }
        if (t == 0) {
          p.dh0[(int64_t)row * H + u] = carry;
        } else {
          const float dn = dprev + carry;  // D_{t-1}
          p.dsum[(int64_t)(t - 1) * BH + (int64_t)row * H + u] = dn;
          *dp = dn;  // only this lane reads or writes this (row, unit) during the step
        }
      }
    }
    lds_barrier();
  }
}

// wl[((q 3 nch + cc) 64 + l) 4 + e] = Wh[g H + k][u] with g = cc / nch,
// k = 64 (cc mod nch) + 4 (l / 4) + e, u = 4 q + l mod 4, and zero where k or u
// is past H. One thread per float4; lanes 4 b .. 4 b + 3 read 16 contiguous
// bytes of a row of Wh.
__global__ void lane_order_kernel(const float* __restrict__ w, float* __restrict__ wl, int H, int nch, int64_t n4) {
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= n4) return;
  const int l = (int)(idx & 63);
  const int64_t qc = idx >> 6;
  const int nk = 3 * nch;
  const int q = (int)(qc / nk), cc = (int)(qc - (int64_t)q * nk);
  const int g = cc / nch, c = cc - g * nch;
  const int u = 4 * q + (l & 3), k0 = 64 * c + 4 * (l >> 2);
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int k = k0 + e;
    v[e] = (u < H && k < H) ? w[(int64_t)(g * H + k) * H + u] : 0.0f;
  }
  reinterpret_cast<f4*>(wl)[idx] = v;
}

int64_t fwd_lds(int BT, int rs, int hr) { return 4 * ((int64_t)BT * (rs + hr) + (int64_t)kTileWaves * kItemFloats); }
int64_t bwd_lds(int BT, int rs, int hr) { return 4 * (int64_t)BT * (3 * rs + hr); }

// Rows per workgroup: 4 (one MFMA row block) unless the batch is smaller or the
// LDS of 4 rows does not fit, then 2 or 1.
int tile_rows(int64_t B, int rs, int hr, bool bwd) {
  int bt = B >= 4 ? 4 : (B >= 2 ? 2 : 1);
  while (bt > 1 && (bwd ? bwd_lds(bt, rs, hr) : fwd_lds(bt, rs, hr)) > kTileLdsMax) bt /= 2;
  return bt;
}

struct TilePlan {
  int nch, rs, hr, BT;
  int64_t lds;
};

int plan_tiled(int64_t H, int64_t B, bool bwd, TilePlan* tp, const char* who) {
  tp->nch = (int)((H + 63) / 64);
  tp->rs = 64 * tp->nch + 16;
  tp->hr = (int)(((H + 3) / 4) * 4 + 4);
  tp->BT = tile_rows(B, tp->rs, tp->hr, bwd);
  tp->lds = bwd ? bwd_lds(tp->BT, tp->rs, tp->hr) : fwd_lds(tp->BT, tp->rs, tp->hr);
  if (tp->lds > kTileLdsMax)
    return set_error(GS_ERR_INVALID, "%s: hidden size %lld exceeds what one workgroup's LDS holds (%lld bytes needed, %lld available)",
                     who, (long long)H, (long long)tp->lds, (long long)kTileLdsMax);
  return GS_OK;
}

}  // namespace

// Largest H the batch-tiled kernels take (the forward's single-row LDS bound
// is larger; the backward's three staged gate rows set the common limit).
int64_t tiled_max_h() { return 8192; }

// codes / scales: Wh's int8 codes and row scales (gs_dense_fwd_i8w,
// gs_dense_fwd_tiled_i8w), or NULL; used when the launch qualifies.
int run_tiled_fwd(const gs_args* a, hipStream_t stream, const char* who, const int8_t* codes,
                  const float* scales) {
  if (a->H > tiled_max_h())
    return set_error(GS_ERR_INVALID, "%s: hidden size %lld exceeds the supported maximum of %lld", who,
                     (long long)a->H, (long long)tiled_max_h());
  TilePlan tp;
  int rc = plan_tiled(a->H, a->B, false, &tp, who);
  if (rc) return rc;
  TFParams p;
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
  p.BT = tp.BT;
  p.nch = tp.nch;
  p.rs = tp.rs;
  p.hr = tp.hr;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.qin_after_first = a->q_in.enabled && !same_quant(a->q_in, a->q_out);
  // float4 weight loads: rows of a multiple of 4 floats from a 16-byte aligned base
  const bool vec = a->H % 4 == 0 && (reinterpret_cast<uintptr_t>(a->w) & 15u) == 0;
  const bool save = a->gh_save != nullptr;
  const bool i8 = codes != nullptr && dense_i8_applies(a) && (reinterpret_cast<uintptr_t>(codes) & 15u) == 0;
  p.wq = i8 ? codes : nullptr;
  p.wsc = i8 ? scales : nullptr;
  p.pscale = a->q_in.scale;
  p.rsi = 64 * ((tp.nch + 3) / 4) + 16;
  void (*fn)(TFParams) = i8    ? tiled_fwd_kernel<true, false, true>
                         : vec ? (save ? tiled_fwd_kernel<true, true> : tiled_fwd_kernel<true, false>)
                               : (save ? tiled_fwd_kernel<false, true> : tiled_fwd_kernel<false, false>);
  if (tp.lds > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)tp.lds));
  const int64_t nblk = (a->B + tp.BT - 1) / tp.BT;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(kTileThreads), (size_t)tp.lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int64_t tiled_bwd_wt_bytes(int64_t H) {
  const int64_t nq = (H + 3) / 4, nch = (H + 63) / 64;
  return align256(nq * 3 * nch * 64 * 16);
}

// Step 3 of the dense backward with the batch-tiled kernel: Wh in the MFMA
// operand order into wt (tiled_bwd_wt_bytes of scratch), then the recurrence.
int run_tiled_bwd_recurrence(const float* w, float* wt, const float* dout, const float* cg, const float* zm,
                             const float* mi, float* dsum, float* dh0, int64_t T, int64_t B, int64_t H,
                             hipStream_t stream, const char* who) {
  if (H > tiled_max_h())
    return set_error(GS_ERR_INVALID, "%s: hidden size %lld exceeds the supported maximum of %lld", who,
                     (long long)H, (long long)tiled_max_h());
  TilePlan tp;
  int rc = plan_tiled(H, B, true, &tp, who);
  if (rc) return rc;
  const int64_t n4 = ((H + 3) / 4) * 3 * tp.nch * 64;
  hipLaunchKernelGGL(lane_order_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, w, wt, (int)H,
                     tp.nch, n4);
  GS_CHECK_HIP(hipGetLastError());
  TBParams p;
  p.wl = wt;
  p.dout = dout;
  p.cg = cg;
  p.zm = zm;
  p.mi = mi;
  p.dsum = dsum;
  p.dh0 = dh0;
  p.T = (int)T;
  p.B = (int)B;
  p.H = (int)H;
  p.BT = tp.BT;
  p.nch = tp.nch;
  p.rs = tp.rs;
  p.hr = tp.hr;
  void (*fn)(TBParams) = tiled_bwd_kernel;
  if (tp.lds > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)tp.lds));
  const int64_t nblk = (B + tp.BT - 1) / tp.BT;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(kBwdThreads), (size_t)tp.lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace gs

extern "C" int gs_dense_fwd_tiled(const gs_args* a, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_dense_fwd_tiled";
  int rc = gs::validate_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  return gs::run_tiled_fwd(a, stream, who);
}

extern "C" int gs_dense_fwd_tiled_i8w(const gs_args* a, const int8_t* w_codes, const float* w_scale,
                                      hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_dense_fwd_tiled_i8w";
  int rc = gs::validate_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  rc = gs::check_codes(w_codes, w_scale, who);
  if (rc) return rc;
  return gs::run_tiled_fwd(a, stream, who, w_codes, w_scale);
}
