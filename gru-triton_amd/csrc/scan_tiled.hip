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
// Work split. A workgroup of 16 waves owns BT <= 4 batch rows. Per step each
// wave takes quads of 4 hidden units (quad q, q + 16, ...) and forms their 3
// gates' products with v_mfma_f32_4x4x1_16b_f32 chains exactly as the
// persistent kernels do (A = the 4 staged rows from LDS, B = 4 weight rows
// loaded as float4 from memory, the 16 MFMA blocks as 16 K slices, two
// accumulators alternating by instruction, reduce16), so the products, and the
// gate epilogue after them, are bit for bit those of the persistent kernels.
// Then an LDS barrier, a pass that stages the next step's operand rows from
// the new state, and a second barrier.
//
// Bound: each workgroup streams the whole of Wh (3 H^2 floats) from L2 or
// memory every step; a CU reads about 64 bytes per clock, so a step takes
// about 3 H^2 4 / 64 clocks whatever BT is (BT only sets how many CUs work).
#include "gs_gemm.h"
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kTileWaves = 16;
constexpr int kTileThreads = 64 * kTileWaves;
// LDS a workgroup may take (gfx950: 160 KiB per CU).
constexpr int64_t kTileLdsMax = 160 * 1024;
// K chunks of 64 whose loads a wave issues together (forward: 3 gates each)
constexpr int kUnroll = 4;

// A chunk of 4 consecutive weights of one row at k (from `row`, which already
// points at this lane's k offset), zero past `klim` elements. VEC: the row
// length is a multiple of 4, so a chunk is either whole or past the end and
// loads as one float4.
template <bool VEC>
__device__ __forceinline__ f4 ld_chunk(const float* row, int k, int klim, bool ok) {
  if constexpr (VEC) {
    return (ok && k < klim) ? *reinterpret_cast<const f4*>(row + k) : f4{0.f, 0.f, 0.f, 0.f};
  } else {
    f4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (ok && k + e < klim) ? row[k + e] : 0.0f;
    return v;
  }
}

struct TFParams {
  const float* gi;
  const float* h0;
  const float* w;  // [3H, H]
  const float* bh;
  float* out;
  float* gh_save;  // SAVE: [T, B, 3H] q_in(h_{t-1}) Wh^T (no bias)
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int BT;   // batch rows per workgroup
  int nch;  // K chunks of 64
  int rs;   // LDS row stride of the staged rows: 64 nch + 16 (16 mod 64: conflict-free operand reads)
  int hr;   // LDS row stride of the raw state
  Quant qin, qout;
  int qin_after_first;
};

template <bool VEC, bool SAVE>
__global__ __launch_bounds__(kTileThreads) void tiled_fwd_kernel(TFParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = p.H, BT = p.BT, rs = p.rs, hr = p.hr;
  const int r = lane & 3, kb = lane >> 2;          // MFMA A row, K slice
  const int j = lane & 3, s = (lane >> 2) & 3;     // epilogue: unit of the quad, row (lanes < 16)
  const bool lead = lane < 16;
  const int row0 = blockIdx.x * BT;
  float* hq = lds;              // [BT][rs] staged q_in(h_{t-1}), zero from H on
  float* hraw = hq + BT * rs;   // [BT][hr] raw h_{t-1}

  for (int i = threadIdx.x; i < BT * rs; i += kTileThreads) {
    const int rr = i / rs, k = i - rr * rs, row = row0 + rr;
    float v = 0.0f;
    if (k < H && row < p.B) {
      v = p.h0[(int64_t)row * p.sh0_b + k];
      if (p.qin.on) v = fake_quant(v, p.qin);
    }
    hq[i] = v;
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
  const int klim = H - 4 * kb;
  const int64_t HH = (int64_t)H * H;
  const int row = row0 + s;
  const bool row_ok = lead && s < BT && row < p.B;
  for (int t = 0; t < p.T; ++t) {
    for (int q = wave; q < nq; q += kTileWaves) {
      const int u = 4 * q + j;
      const bool u_ok = u < H;
      const bool mine = row_ok && u_ok;
      // epilogue inputs first: their latency overlaps the K loop
      float gir = 0.f, giz = 0.f, gin = 0.f, b0 = 0.f, b1 = 0.f, b2 = 0.f;
      if (mine) {
        const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + u;
        gir = g[0];
        giz = g[H];
        gin = g[2 * H];
        b0 = kR * p.bh[u];
        b1 = kR * p.bh[H + u];
        b2 = kN * p.bh[2 * H + u];
      }
      const float* w0 = p.w + (int64_t)u * H + 4 * kb;  // row u of gate r; gate g adds g H^2
      f4 p0[3], p1[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) p0[g] = p1[g] = f4{0.f, 0.f, 0.f, 0.f};
      // kUnroll chunks per iteration: their 3 kUnroll weight loads are in flight together
      for (int c0 = 0; c0 < p.nch; c0 += kUnroll) {
        f4 a[kUnroll], wv[kUnroll][3];
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) {
          const int c = c0 + i;
          const bool in = c < p.nch;  // uniform
          a[i] = (in && a_ok) ? *reinterpret_cast<const f4*>(arow + 64 * c) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int g = 0; g < 3; ++g) wv[i][g] = ld_chunk<VEC>(w0 + g * HH, 64 * c, klim, in && u_ok);
        }
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) {
          if (c0 + i >= p.nch) break;  // uniform: no MFMA past the last chunk
#pragma unroll
          for (int g = 0; g < 3; ++g) {
            p0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][0], wv[i][g][0], p0[g], 0, 0, 0);
            p1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][1], wv[i][g][1], p1[g], 0, 0, 0);
            p0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][2], wv[i][g][2], p0[g], 0, 0, 0);
            p1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i][3], wv[i][g][3], p1[g], 0, 0, 0);
          }
        }
      }
      float gh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) gh[g] = reduce16(p0[g] + p1[g], s);
      if (mine) {
        float* hp = hraw + s * hr + u;
        const float cr = __builtin_fmaf(kR, gir, b0), cz = __builtin_fmaf(kR, giz, b1), an2 = kN * gin;
        float hn = gru_update_l2(__builtin_fmaf(kR, gh[0], cr), __builtin_fmaf(kR, gh[1], cz),
                                 __builtin_fmaf(kN, gh[2], b2), an2, *hp);
        if (p.qout.on) hn = fake_quant(hn, p.qout);
        *hp = hn;  // only this lane reads or writes this (row, unit) during the step
        p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + u] = hn;
        if constexpr (SAVE) {
          float* o = p.gh_save + ((int64_t)t * p.B + row) * 3 * H + u;
#pragma unroll
          for (int g = 0; g < 3; ++g) __builtin_nontemporal_store(gh[g], o + g * H);
        }
      }
    }
    lds_barrier();
    if (t + 1 < p.T) {
      for (int i = threadIdx.x; i < BT * H; i += kTileThreads) {
        const int rr = i / H, k = i - rr * H;
        float v = hraw[rr * hr + k];
        if (p.qin_after_first) v = fake_quant(v, p.qin);
        hq[rr * rs + k] = v;
      }
      lds_barrier();
    }
  }
}

// Backward recurrence (the dense backward's step 3, scan_dense_bwd.hip):
//   D_{t-1} = dout[t-1] + Zm_t D_t + Mi_t (dgh_t Wh),   dgh_t = D_t (Cr, Cz, Chn)_t,
//   dh0 = Zm_0 D_0 + Mi_0 (dgh_0 Wh),
// with Wh read transposed (wt [H, 3H], wt[u][n] = Wh[n][u]) so that a unit's
// weights over the 3H reduction are one contiguous row.
struct TBParams {
  const float* wt;    // [H, 3H]
  const float* dout;  // [T, B, H] contiguous
  const float* cg;    // [T, B, 3H] (Cr, Cz, Chn)
  const float* zm;    // [T, B, H]
  const float* mi;    // [T, B, H]
  float* dsum;        // [T, B, H] D_t
  float* dh0;         // [B, H]
  int T, B, H, BT, nch, rs, hr;
};

template <bool VEC>
__global__ __launch_bounds__(kTileThreads) void tiled_bwd_kernel(TBParams p) {
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
  for (int i = threadIdx.x; i < 3 * BT * rs; i += kTileThreads) dg[i] = 0.0f;
  for (int i = threadIdx.x; i < BT * hr; i += kTileThreads) {
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
  const int klim = H - 4 * kb;
  const int row = row0 + s;
  const bool row_ok = lead && s < BT && row < p.B;
  const int H3 = 3 * H;
  for (int st = 0; st < T; ++st) {
    const int t = T - 1 - st;
    // stage dgh_t = D_t (Cr, Cz, Chn)_t
    for (int i = threadIdx.x; i < BT * H; i += kTileThreads) {
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
    for (int q = wave; q < nq; q += kTileWaves) {
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
      const float* w0 = p.wt + (int64_t)u * H3 + 4 * kb;
      f4 acc0 = f4{0.f, 0.f, 0.f, 0.f}, acc1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        const float* arow = dg + (g * BT + (a_ok ? r : 0)) * rs + 4 * kb;
        const float* wg = w0 + g * H;
        for (int c0 = 0; c0 < p.nch; c0 += 2 * kUnroll) {
          f4 a[2 * kUnroll], wv[2 * kUnroll];
#pragma unroll
          for (int i = 0; i < 2 * kUnroll; ++i) {
            const int c = c0 + i;
            const bool in = c < p.nch;  // uniform
            a[i] = (in && a_ok) ? *reinterpret_cast<const f4*>(arow + 64 * c) : f4{0.f, 0.f, 0.f, 0.f};
            wv[i] = ld_chunk<VEC>(wg, 64 * c, klim, in && u_ok);
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

__global__ void transpose_kernel(const float* __restrict__ src, float* __restrict__ dst, int rows, int cols) {
  // dst[c][r] = src[r][c], 32 x 32 tiles through LDS (padded against bank conflicts)
  __shared__ float tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: ty in [0, 8)
  for (int i = ty; i < 32; i += 8) {
    const int rr = r0 + i, cc = c0 + tx;
    tile[i][tx] = (rr < rows && cc < cols) ? src[(int64_t)rr * cols + cc] : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int cc = c0 + i, rr = r0 + tx;
    if (cc < cols && rr < rows) dst[(int64_t)cc * rows + rr] = tile[tx][i];
  }
}

int64_t fwd_lds(int BT, int rs, int hr) { return 4 * (int64_t)BT * (rs + hr); }
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

int run_tiled_fwd(const gs_args* a, hipStream_t stream, const char* who) {
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
  void (*fn)(TFParams) = vec ? (save ? tiled_fwd_kernel<true, true> : tiled_fwd_kernel<true, false>)
                             : (save ? tiled_fwd_kernel<false, true> : tiled_fwd_kernel<false, false>);
  if (tp.lds > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)tp.lds));
  const int64_t nblk = (a->B + tp.BT - 1) / tp.BT;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(kTileThreads), (size_t)tp.lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int64_t tiled_bwd_wt_bytes(int64_t H) { return align256(3 * H * H * 4); }

// Step 3 of the dense backward with the batch-tiled kernel: Wh transposed into
// wt (tiled_bwd_wt_bytes of scratch), then the recurrence.
int run_tiled_bwd_recurrence(const float* w, float* wt, const float* dout, const float* cg, const float* zm,
                             const float* mi, float* dsum, float* dh0, int64_t T, int64_t B, int64_t H,
                             hipStream_t stream, const char* who) {
  if (H > tiled_max_h())
    return set_error(GS_ERR_INVALID, "%s: hidden size %lld exceeds the supported maximum of %lld", who,
                     (long long)H, (long long)tiled_max_h());
  TilePlan tp;
  int rc = plan_tiled(H, B, true, &tp, who);
  if (rc) return rc;
  hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((H + 31) / 32), (unsigned)((3 * H + 31) / 32)), dim3(256), 0,
                     stream, w, wt, (int)(3 * H), (int)H);
  GS_CHECK_HIP(hipGetLastError());
  TBParams p;
  p.wt = wt;
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
  void (*fn)(TBParams) = (H % 4 == 0) ? tiled_bwd_kernel<true> : tiled_bwd_kernel<false>;
  if (tp.lds > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)tp.lds));
  const int64_t nblk = (B + tp.BT - 1) / tp.BT;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblk), dim3(kTileThreads), (size_t)tp.lds, stream, p);
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
