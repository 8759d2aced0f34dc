// Dense and Monarch GRU scan forward on fp32 MFMA (gfx950).
//
// References (LarocheC/gru-triton src/gru_qat/triton_kernels/):
//   dense    scan.py:76-210 (persistent kernel), scan.py:213-293 (launcher)
//   Monarch  scan_monarch.py:130-291 (kernel), :320-406 (launcher), math :74-127
//
// Decomposition. Hidden units are split into quads of 4 consecutive units; one
// wave owns one quad (all three gates: 12 rows of Wh) for the whole scan and
// keeps that slice of Wh in VGPRs, loaded once. A *group* is the set of
// workgroups that together produce every unit a batch row's next step needs
// (dense: all of H; single-factor Monarch: one block; two-factor Monarch: all
// of H). Each group owns RB row-blocks of 4 batch rows. Groups are
// interleaved in blockIdx (gid = blockIdx % ngroups), so under round-robin
// workgroup placement the members of a group share an XCD. All waves of a
// workgroup read the same K range (Monarch: the same block).
//
// Exchange. Every unit's matmul-side state q_in(h_t) is published as a
// tagged 64-bit word (gs_device.h); consumers poll exactly the words they
// need. Each workgroup stages the 4 x K slice of q_in(h_{t-1}) its waves read
// into LDS (double-buffered), so one workgroup-local barrier per step and
// phase is the only synchronisation; there is no grid barrier.
//
// Per step and row-block each wave computes gh[4 rows][4 units] for 3 gates
// with v_mfma_f32_4x4x1_16b_f32 chains: the instruction's 16 blocks are 16
// slices of K. A is q_in(h)[row = lane&3][k], B is Wh[unit = lane&3][k] and
// D block b holds slice b's partial dot products (row = vgpr index,
// unit = lane&3), with k(m, b) = 64*(m/4) + 4*b + m%4 so that each lane
// reads its A operand as float4s from LDS. The 16 partials are summed with
// two DPP row rotations and two permlane row swaps; lane l then holds
// gh[row = (l>>2)&3][unit = l&3] and the 16 lanes of row 0 run the gate
// epilogue, store out[t] and publish q_in(h_t).
//
// Two-factor Monarch runs two such phases per step: phase 1 publishes
// z_g = R_g q_in(h) (tagged, per gate), phase 2 stages the workgroup's block
// of P z_g, multiplies by L_g and lands the result on y = P^T v.
#include <mutex>

#include "gs_host.h"

namespace gs {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

enum : int { kDense = 0, kMonarch1 = 1, kMonarch2 = 2 };

struct MParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* w2;
  const float* bh;
  float* out;
  uint64_t* xh;  // [2][Bp][H] tagged q_in(h_t), Bp = 4 * nrb (padding rows hold finite filler)
  uint64_t* xz;  // two-factor Monarch: [2][3][Bp][H] tagged first-factor output
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int nb, bs;   // Monarch blocks (dense: nb = 1, bs = H)
  int qpb;      // quads per block = ceil(bs / 4)
  int ngroups;  // groups in the grid
  int G;        // row-block sets (ngroups = G, or G * nb for single-factor Monarch)
  int RB;       // row-blocks per set
  int nrb;      // row-blocks = ceil(B / 4)
  int Bp;       // 4 * nrb: rows of the exchange buffers
  int nwg;      // workgroups in the grid
  int rs;       // LDS row stride (floats) of the staging buffers
  Quant qin, qout;
  int qin_after_first;  // q_in must be applied to h_t before it is published
};

// k index of MFMA instruction m in k-slice b (see the header comment).
__device__ __forceinline__ int kmap(int m, int b) { return 64 * (m >> 2) + 4 * b + (m & 3); }

__device__ __forceinline__ float reduce16(f4 acc, int s) {
  // Sum the 4 k-slices that share this 16-lane row (lane bits 2..3) ...
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += row_ror<8>(acc[c]);
    acc[c] += row_ror<4>(acc[c]);
  }
  // ... keep the D row this lane will own (row index == lane bits 2..3) ...
  const float v = (s == 0) ? acc[0] : (s == 1) ? acc[1] : (s == 2) ? acc[2] : acc[3];
  // ... and add the other three 16-lane rows.
  return sum_across_rows(v);
}

// Loads Wh slice: w[((gate*nb + blk)*bs + o)*bs + k] for o = o0 + (lane&3),
// k = kmap(m, kb4); zero where o >= bs or k >= bs.
template <int KC>
__device__ __forceinline__ void load_w(const float* w, int nb, int bs, int blk, int o0, int j,
                                       int kb4, bool blk_ok, float (&wr)[3][KC]) {
  const int o = o0 + j;
  const bool ok = blk_ok && o < bs;
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const float* row = w + ((int64_t)(g * nb + blk) * bs + o) * bs;
#pragma unroll
    for (int m = 0; m < KC; ++m) {
      const int k = kmap(m, kb4);
      wr[g][m] = (ok && k < bs) ? row[k] : 0.0f;
    }
  }
}

// A operand from an LDS staging row: a[m] = row[kmap(m, kb4)].
template <int KC>
__device__ __forceinline__ void lds_a(const float* row, int kb4, float (&a)[KC]) {
#pragma unroll
  for (int q = 0; q < KC / 4; ++q) {
    const f4 v = *reinterpret_cast<const f4*>(row + 64 * q + 4 * kb4);
    a[4 * q + 0] = v[0];
    a[4 * q + 1] = v[1];
    a[4 * q + 2] = v[2];
    a[4 * q + 3] = v[3];
  }
}

// Three MFMA chains (one per gate), two accumulators each for issue overlap.
// With SHARED_A all gates multiply the same A operand (a[0]).
template <int KC, bool SHARED_A>
__device__ __forceinline__ void mfma3(const float (&a)[3][KC], const float (&wr)[3][KC], f4 (&acc)[3]) {
  f4 acc0[3], acc1[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    acc0[g] = f4{0.f, 0.f, 0.f, 0.f};
    acc1[g] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int m = 0; m < KC; m += 2) {
#pragma unroll
    for (int g = 0; g < 3; ++g)
      acc0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[SHARED_A ? 0 : g][m], wr[g][m], acc0[g], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 3; ++g)
      acc1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[SHARED_A ? 0 : g][m + 1], wr[g][m + 1], acc1[g], 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < 3; ++g) acc[g] = acc0[g] + acc1[g];
}

// Staging. Each thread owns MW words of a workgroup's per-step slice; its
// word offsets are computed once (StagePlan) and the per-step work is the
// poll. A slice larger than MW * threads (only for workgroups smaller than
// the instance's maximum) is staged in several passes with offsets computed
// on the fly.
template <int MW>
struct StagePlan {
  int src[MW];     // word offset from the row-block's slot base
  int dst[MW];     // LDS offset (floats)
  uint32_t valid;  // bit i: word i exists
  bool single;     // the whole slice fits one pass
};

// q_in(h) slice: rows r < 4, k < klen -> src r*H + klo + k, dst r*rs + k.
template <int MW>
__device__ __forceinline__ StagePlan<MW> plan_h(const MParams& p, int klo, int klen) {
  StagePlan<MW> pl;
  const int words = 4 * klen, tid = threadIdx.x, nth = blockDim.x;
  pl.valid = 0;
  pl.single = words <= MW * nth;
#pragma unroll
  for (int i = 0; i < MW; ++i) {
    const int w = tid + i * nth;
    const int r = w / klen, k = w - r * klen;
    const bool ok = w < words;
    pl.src[i] = ok ? r * p.H + klo + k : 0;
    pl.dst[i] = ok ? r * p.rs + k : 0;
    pl.valid |= (ok ? 1u : 0u) << i;
  }
  return pl;
}

// Two-factor Monarch: (P z_g)[blk*bs + k] for gates g, rows r < 4, k < bs
// -> src g*Bp*H + r*H + zpos, dst (g*4 + r)*rs + k.
__device__ __forceinline__ int zsrc(const MParams& p, int blk, int w) {
  const int gr = w / p.bs, k = w - gr * p.bs;
  const int idx = blk * p.bs + k;                      // position in P z
  const int zpos = (idx % p.nb) * p.bs + idx / p.nb;   // position in z
  return ((gr >> 2) * p.Bp + (gr & 3)) * p.H + zpos;
}

template <int MW>
__device__ __forceinline__ StagePlan<MW> plan_z(const MParams& p, int blk) {
  StagePlan<MW> pl;
  const int words = 12 * p.bs, tid = threadIdx.x, nth = blockDim.x;
  pl.valid = 0;
  pl.single = words <= MW * nth;
#pragma unroll
  for (int i = 0; i < MW; ++i) {
    const int w = tid + i * nth;
    const bool ok = w < words;
    const int gr = w / p.bs;
    pl.src[i] = ok ? zsrc(p, blk, w) : 0;
    pl.dst[i] = ok ? gr * p.rs + (w - gr * p.bs) : 0;
    pl.valid |= (ok ? 1u : 0u) << i;
  }
  return pl;
}

// Multi-pass staging with offsets computed per word (rare shapes only).
template <int MW, bool Z>
__device__ __forceinline__ void stage_general(const MParams& p, const uint64_t* base, int klo, int klen, int blk,
                                           float* dst, uint32_t tag) {
  const int words = Z ? 12 * p.bs : 4 * klen;
  const int tid = threadIdx.x, nth = blockDim.x;
  for (int c0 = 0; c0 < words; c0 += MW * nth) {
    int src[MW], off[MW];
    uint32_t valid = 0;
#pragma unroll
    for (int i = 0; i < MW; ++i) {
      const int w = c0 + tid + i * nth;
      const bool ok = w < words;
      if (Z) {
        const int gr = w / p.bs;
        src[i] = ok ? zsrc(p, blk, w) : 0;
        off[i] = ok ? gr * p.rs + (w - gr * p.bs) : 0;
      } else {
        const int r = w / klen, k = w - r * klen;
        src[i] = ok ? r * p.H + klo + k : 0;
        off[i] = ok ? r * p.rs + k : 0;
      }
      valid |= (ok ? 1u : 0u) << i;
    }
    poll_to_lds<MW>(p.ctrl, base, src, off, valid, tag, dst);
  }
}

// Step 0 input: q_in(h0) rows 4rb..4rb+3 (zeros past B), cols [klo, klo+klen).
__device__ __forceinline__ void stage_h0(const MParams& p, int rb, int klo, int klen, float* dst) {
  const int words = 4 * klen;
  for (int w = threadIdx.x; w < words; w += blockDim.x) {
    const int r = w / klen, k = w - r * klen;
    const int row = 4 * rb + r;
    float v = 0.0f;
    if (row < p.B) {
      v = p.h0[(int64_t)row * p.sh0_b + klo + k];
      if (p.qin.on) v = fake_quant(v, p.qin);
    }
    dst[r * p.rs + k] = v;
  }
}

template <int KIND, int KC, int NT>
__global__ __launch_bounds__(NT) void mfma_scan_kernel(MParams p) {
  extern __shared__ float lds[];
  constexpr int MWH = (4 * 16 * KC + NT - 1) / NT;   // staged h words per thread and pass
  constexpr int MWZ = (12 * 16 * KC + NT - 1) / NT;  // staged z words per thread and pass
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int j = lane & 3;         // unit within the quad (B and D column), A row
  const int kb4 = lane >> 2;      // k-slice (MFMA block)
  const int s = (lane >> 2) & 3;  // D row owned after the reduction
  const bool lead = lane < 16;    // lanes that store

  const int gid = blockIdx.x % p.ngroups;
  const int pw = blockIdx.x / p.ngroups;
  const int set = (KIND == kMonarch1) ? gid % p.G : gid;
  const int quad = pw * nw + wave;

  int blk, o0;
  if (KIND == kMonarch1) {
    blk = gid / p.G;
    o0 = 4 * quad;
  } else {
    blk = quad / p.qpb;
    o0 = 4 * (quad - blk * p.qpb);
  }
  const bool blk_ok = blk < p.nb && o0 < p.bs;
  // The K range every wave of this workgroup reads: [klo, klo + bs).
  const int wg_blk = (KIND == kDense) ? 0 : ((KIND == kMonarch1) ? blk : (pw * nw) / p.qpb);
  const bool wg_ok = wg_blk < p.nb;
  const int klo = wg_blk * p.bs;

  float* hst = lds;             // [2][4][rs]
  float* zst = lds + 8 * p.rs;  // two-factor Monarch: [2][12][rs]
  for (int i = threadIdx.x; i < (KIND == kMonarch2 ? 32 : 8) * p.rs; i += blockDim.x) lds[i] = 0.0f;
  __syncthreads();

  float wr[3][KC];
  load_w<KC>(p.w, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wr);
  float wl[3][KC];
  if (KIND == kMonarch2) load_w<KC>(p.w2, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wl);

  // Epilogue unit of this lane. Two-factor Monarch: the second factor's row
  // vi = blk*bs + o0 + j lands on y[(vi % nb) * bs + vi / nb] (P^T).
  const int vi = blk * p.bs + o0 + j;
  const bool unit_ok = blk_ok && (o0 + j) < p.bs;
  const int unit = (KIND == kMonarch2) ? (vi % p.nb) * p.bs + vi / p.nb : vi;
  float bias[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) bias[g] = unit_ok ? p.bh[g * p.H + unit] : 0.0f;

  const StagePlan<MWH> hplan = plan_h<MWH>(p, klo, p.bs);
  StagePlan<MWZ> zplan;
  if (KIND == kMonarch2) zplan = plan_z<MWZ>(p, wg_blk);

  const uint32_t base = __hip_atomic_load(p.ctrl.tag_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int rb_begin = set * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);
  int hbuf = 0, zbuf = 0;

  for (int t = 0; t < p.T; ++t) {
    const uint32_t tag = base + (uint32_t)t + 1u;
    const bool publish = t + 1 < p.T;
    for (int rb = rb_begin; rb < rb_end; ++rb) {
      const int row = 4 * rb + s;
      const bool mine = lead && row < p.B && unit_ok;
      const bool pub = lead && unit_ok;  // padding rows are published too (finite filler)
      // Epilogue operands first, so their latency overlaps the staging polls.
      float gir = 0.f, giz = 0.f, gin = 0.f, hprev = 0.f;
      if (mine) {
        const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + unit;
        gir = g[0];
        giz = g[p.H];
        gin = g[2 * p.H];
        hprev = (t == 0) ? p.h0[(int64_t)row * p.sh0_b + unit]
                         : p.out[(int64_t)(t - 1) * p.so_t + (int64_t)row * p.so_b + unit];
      }
      float* hs = hst + hbuf * 4 * p.rs;
      hbuf ^= 1;
      if (wg_ok) {
        if (t == 0) {
          stage_h0(p, rb, klo, p.bs, hs);
        } else {
          const uint64_t* hb = p.xh + ((int64_t)((t - 1) & 1) * p.Bp + 4 * rb) * p.H;
          if (hplan.single)
            poll_to_lds<MWH>(p.ctrl, hb, hplan.src, hplan.dst, hplan.valid, tag - 1u, hs);
          else
            stage_general<MWH, false>(p, hb, klo, p.bs, 0, hs, tag - 1u);
        }
      }
      __syncthreads();
      float a[3][KC];
      lds_a<KC>(hs + j * p.rs, kb4, a[0]);
      f4 acc[3];
      mfma3<KC, true>(a, wr, acc);
      float gh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);

      if (KIND == kMonarch2) {
        // Publish z_g = R_g q_in(h), then stage P z_g for this workgroup's block.
        if (pub) {
#pragma unroll
          for (int g = 0; g < 3; ++g)
            st_tagged(p.xz + ((int64_t)((t & 1) * 3 + g) * p.Bp + row) * p.H + vi, gh[g], tag);
        }
        float* zs = zst + zbuf * 12 * p.rs;
        zbuf ^= 1;
        if (wg_ok) {
          const uint64_t* zb = p.xz + (int64_t)(t & 1) * 3 * p.Bp * p.H + (int64_t)4 * rb * p.H;
          if (zplan.single)
            poll_to_lds<MWZ>(p.ctrl, zb, zplan.src, zplan.dst, zplan.valid, tag, zs);
          else
            stage_general<MWZ, true>(p, zb, 0, 0, wg_blk, zs, tag);
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < 3; ++g) lds_a<KC>(zs + (g * 4 + j) * p.rs, kb4, a[g]);
        mfma3<KC, false>(a, wl, acc);
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);
      }

      float hn = gru_update(gir, giz, gin, gh[0] + bias[0], gh[1] + bias[1], gh[2] + bias[2], hprev);
      if (p.qout.on) hn = fake_quant(hn, p.qout);
      if (mine) p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + unit] = hn;
      if (pub && publish) {
        const float hq = p.qin_after_first ? fake_quant(hn, p.qin) : hn;
        st_tagged(p.xh + ((int64_t)(t & 1) * p.Bp + row) * p.H + unit, hq, tag);
      }
    }
  }
  leave_grid(p.ctrl, (uint32_t)p.nwg, base, (uint32_t)p.T);
}

// ---- host side --------------------------------------------------------------------

struct DevInfo {
  int cus = 0;
  int coop = 0;
};

int device_info(DevInfo* out) {
  static std::mutex mu;
  static DevInfo cache[64];
  static bool have[64] = {};
  int dev = 0;
  GS_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return set_error(GS_ERR_HIP, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(mu);
  if (!have[dev]) {
    GS_CHECK_HIP(hipDeviceGetAttribute(&cache[dev].cus, hipDeviceAttributeMultiprocessorCount, dev));
    GS_CHECK_HIP(hipDeviceGetAttribute(&cache[dev].coop, hipDeviceAttributeCooperativeLaunch, dev));
    have[dev] = true;
  }
  *out = cache[dev];
  return GS_OK;
}

typedef void (*KernelFn)(MParams);

// Workgroup size bound per instance: small reduction lengths keep few
// registers per wave, so up to 16 waves share a workgroup; from KC = 16 on
// (8 for the two-factor form, which holds two weight slices) a wave needs
// more than 128 VGPRs and the workgroup is capped at 4 waves, one per SIMD.
template <int KIND>
KernelFn pick_kernel(int KC, int* nt) {
  switch (KC) {
    case 4: *nt = 1024; return mfma_scan_kernel<KIND, 4, 1024>;
    case 8:
      if constexpr (KIND == kMonarch2) {
        *nt = 256;
        return mfma_scan_kernel<KIND, 8, 256>;
      } else {
        *nt = 1024;
        return mfma_scan_kernel<KIND, 8, 1024>;
      }
    case 16: *nt = 256; return mfma_scan_kernel<KIND, 16, 256>;
    case 32: *nt = 256; return mfma_scan_kernel<KIND, 32, 256>;
    case 64: *nt = 256; return mfma_scan_kernel<KIND, 64, 256>;
    default: return nullptr;
  }
}

KernelFn pick(int kind, int KC, int* nt) {
  if (kind == kDense) return pick_kernel<kDense>(KC, nt);
  if (kind == kMonarch1) return pick_kernel<kMonarch1>(KC, nt);
  return pick_kernel<kMonarch2>(KC, nt);
}

int choose_kc(int klen) {
  const int need = (klen + 15) / 16;
  for (int kc : {4, 8, 16, 32, 64})
    if (kc >= need) return kc;
  return -1;
}

struct Plan {
  int kind, KC, nt, nw, P, G, RB, nrb, ngroups, nwg, nb, bs, qpb, rs;
  int64_t xh_bytes, xz_bytes;
  size_t lds_bytes;
};

// Static part of the plan (no device query): used for workspace sizing too.
int plan_static(int kind, const gs_args* a, Plan* pl, const char* who) {
  pl->kind = kind;
  if (kind == kDense) {
    pl->nb = 1;
    pl->bs = (int)a->H;
  } else {
    if (a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != a->H)
      return set_error(GS_ERR_INVALID,
                       "%s: Wh_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                       (long long)a->nblocks, (long long)a->blksz, (long long)a->H);
    pl->nb = (int)a->nblocks;
    pl->bs = (int)a->blksz;
  }
  pl->KC = choose_kc(pl->bs);
  if (pl->KC < 0)
    return set_error(GS_ERR_INVALID, "%s: reduction length %d exceeds the supported maximum of 1024", who, pl->bs);
  pl->qpb = (pl->bs + 3) / 4;
  if (!pick(kind, pl->KC, &pl->nt)) return set_error(GS_ERR_INVALID, "%s: no kernel for KC=%d", who, pl->KC);
  const int nwmax = pl->nt / 64;
  if (kind == kDense) {
    pl->nw = pl->qpb < nwmax ? pl->qpb : nwmax;
    pl->P = (pl->qpb + pl->nw - 1) / pl->nw;
  } else {
    // The waves of a workgroup must share one Monarch block, so the wave count
    // divides the quads per block.
    int nw = pl->qpb < nwmax ? pl->qpb : nwmax;
    while (pl->qpb % nw != 0) --nw;
    pl->nw = nw;
    pl->P = (kind == kMonarch1 ? pl->qpb : pl->nb * pl->qpb) / nw;
  }
  pl->nrb = (int)((a->B + 3) / 4);
  pl->rs = 16 * pl->KC + 4;  // one full MFMA K span per staged row (+4 floats of skew)
  pl->lds_bytes = (size_t)(kind == kMonarch2 ? 32 : 8) * pl->rs * sizeof(float);
  const int64_t Bp = 4 * (int64_t)pl->nrb;
  pl->xh_bytes = align256(2 * Bp * a->H * 8);
  pl->xz_bytes = (kind == kMonarch2) ? align256(6 * Bp * a->H * 8) : 0;
  return GS_OK;
}

int64_t workspace_bytes_for(int kind, const gs_args* a) {
  Plan pl;
  const int rc = plan_static(kind, a, &pl, "gs_workspace_bytes");
  if (rc) return rc;
  return kCtrlBytes + pl.xh_bytes + pl.xz_bytes;
}

int run(int kind, const gs_args* a, hipStream_t stream, const char* who) {
  clear_error();
  int rc = validate_common(a, who);
  if (rc) return rc;
  if (kind == kDense && a->w2 != nullptr)
    return set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  Plan pl;
  rc = plan_static(kind, a, &pl, who);
  if (rc) return rc;
  rc = check_workspace(a, kCtrlBytes + pl.xh_bytes + pl.xz_bytes, who);
  if (rc) return rc;

  KernelFn fn = pick(kind, pl.KC, &pl.nt);
  const int threads = pl.nw * 64;
  if (pl.lds_bytes > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)pl.lds_bytes));

  // Groups that span several workgroups wait on each other's published state,
  // so all of their workgroups must be resident at once (cooperative launch).
  const bool coop = pl.P > 1;
  const int per_set = pl.P * (kind == kMonarch1 ? pl.nb : 1);
  int G = pl.nrb;
  if (coop) {
    DevInfo di;
    rc = device_info(&di);
    if (rc) return rc;
    if (!di.coop) return set_error(GS_ERR_CAPACITY, "%s: device does not support cooperative launch", who);
    int occ = 0;
    GS_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)fn, threads, pl.lds_bytes));
    const int64_t resident = (int64_t)occ * di.cus;
    if (resident < per_set)
      return set_error(GS_ERR_CAPACITY,
                       "%s: persistent grid needs %d co-resident workgroups of %d threads per batch "
                       "group; the device holds %lld",
                       who, per_set, threads, (long long)resident);
    const int64_t gmax = resident / per_set;
    if (gmax < G) G = (int)gmax;
  }
  pl.RB = (pl.nrb + G - 1) / G;
  pl.G = (pl.nrb + pl.RB - 1) / pl.RB;
  pl.ngroups = pl.G * (kind == kMonarch1 ? pl.nb : 1);
  pl.nwg = pl.ngroups * pl.P;

  MParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.w2 = a->w2;
  p.bh = a->bh;
  p.out = a->out;
  char* ws = static_cast<char*>(a->workspace);
  p.ctrl = ctrl_of(ws);
  p.xh = reinterpret_cast<uint64_t*>(ws + kCtrlBytes);
  p.xz = pl.xz_bytes ? reinterpret_cast<uint64_t*>(ws + kCtrlBytes + pl.xh_bytes) : nullptr;
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.nb = pl.nb;
  p.bs = pl.bs;
  p.qpb = pl.qpb;
  p.ngroups = pl.ngroups;
  p.G = pl.G;
  p.RB = pl.RB;
  p.nrb = pl.nrb;
  p.Bp = 4 * pl.nrb;
  p.nwg = pl.nwg;
  p.rs = pl.rs;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.qin_after_first = a->q_in.enabled && !same_quant(a->q_in, a->q_out);

  if (coop) {
    void* kargs[] = {&p};
    GS_CHECK_HIP(hipLaunchCooperativeKernel((const void*)fn, dim3(pl.nwg), dim3(threads), kargs,
                                            (unsigned)pl.lds_bytes, stream));
  } else {
    hipLaunchKernelGGL(fn, dim3(pl.nwg), dim3(threads), pl.lds_bytes, stream, p);
    GS_CHECK_HIP(hipGetLastError());
  }
  return GS_OK;
}

}  // namespace

int64_t dense_workspace_bytes(const gs_args* a) { return workspace_bytes_for(kDense, a); }

int64_t monarch_workspace_bytes(const gs_args* a) {
  return workspace_bytes_for(a->w2 ? kMonarch2 : kMonarch1, a);
}

}  // namespace gs

extern "C" int gs_dense_fwd(const gs_args* a, hipStream_t stream) {
  return gs::run(gs::kDense, a, stream, "gs_dense_fwd");
}

extern "C" int gs_monarch_fwd(const gs_args* a, hipStream_t stream) {
  if (a == nullptr) return gs::set_error(GS_ERR_INVALID, "gs_monarch_fwd: args is NULL");
  return gs::run(a->w2 ? gs::kMonarch2 : gs::kMonarch1, a, stream, "gs_monarch_fwd");
}
