// Dense and Monarch GRU scan forward on fp32 MFMA (gfx950).
//
// References (LarocheC/gru-triton src/gru_qat/triton_kernels/):
//   dense    scan.py:76-210 (persistent kernel), scan.py:213-293 (launcher)
//   Monarch  scan_monarch.py:130-291 (kernel), :320-406 (launcher), math :74-127
//
// Decomposition. The hidden units are split into quads of 4 consecutive units;
// one wave owns one quad (all three gates, i.e. 12 rows of Wh) for the whole
// scan. Its slice of Wh lives in VGPRs, loaded once. A *group* is the set of
// workgroups that together cover every quad that a batch row depends on
// (dense: all of H; single-factor Monarch: one block; two-factor Monarch: all
// of H); each group handles its own row-blocks of 4 batch rows and
// synchronises only with itself, once per step (twice for two-factor
// Monarch). Groups are interleaved in blockIdx (gid = blockIdx % ngroups), so
// with round-robin workgroup placement the members of one group share an XCD.
//
// Per step and row-block, each wave computes gh[4 rows][4 units] for 3 gates
// as 3 chains of v_mfma_f32_4x4x1_16b_f32: the instruction's 16 blocks are 16
// interleaved slices of K (block b covers k = KC*b + m, m < KC), so KC
// instructions per gate cover K = 16*KC. A is q_in(h)[row = lane&3][k], B is
// Wh[unit = lane&3][k], D block b holds the partial dot products of slice b
// (row = vgpr index, unit = lane&3). The 16 partials are summed with two DPP
// row rotations and two cross-row swaps; afterwards lane l holds the full
// gh[row = (l>>2)&3][unit = l&3], and the 16 lanes of row 0 run the gate
// epilogue and store out[t].
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
  float* hqbuf;  // [2][B][H]: q_in(h_t) when the two quantizers differ
  float* zbuf;   // two-factor Monarch: [3][B][H] output of the first factor
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int nb, bs;     // Monarch blocks (dense: nb = 1, bs = H)
  int qpb;        // quads per block = ceil(bs / 4)
  int ngroups;    // groups in the grid
  int G;          // row-block sets (ngroups = G, or G * nb for single-factor Monarch)
  int RB;         // row-blocks per set
  int nrb;        // row-blocks = ceil(B / 4)
  int P;          // workgroups per group
  int nwg;        // workgroups in the grid
  Quant qin, qout;
  int hq_scratch;  // 1: matmul-side h of step t >= 1 comes from hqbuf, else from out
  int vec_ok;      // rows of out / hqbuf may be read as float4
  int coop;        // 1: groups span several workgroups (global barrier)
};

__device__ __forceinline__ float reduce16(f4 acc, int s) {
  // Sum the 4 k-slices that share this 16-lane row (lane bits 2..3) ...
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += row_ror<8>(acc[c]);
    acc[c] += row_ror<4>(acc[c]);
  }
  // ... keep the D row this lane will own (row index == lane bits 2..3) ...
  float v = (s == 0) ? acc[0] : (s == 1) ? acc[1] : (s == 2) ? acc[2] : acc[3];
  // ... and add the other three 16-lane rows.
  v += lane_xor(v, 16);
  v += lane_xor(v, 32);
  return v;
}

// Loads this lane's A operand: q_in(h)[row][kbase + KC*kb4 + m], m < KC, zero
// outside [0, klen) or for rows >= B.
template <int KC>
__device__ __forceinline__ void load_hq(const MParams& p, int t, int row, int kbase, int klen,
                                        int kb4, float (&a)[KC]) {
  const int k0 = KC * kb4;
  const bool row_ok = row < p.B;
  if (t == 0) {
    const float* src = p.h0 + (int64_t)row * p.sh0_b + kbase;
#pragma unroll
    for (int m = 0; m < KC; ++m) {
      float v = 0.0f;
      if (row_ok && k0 + m < klen) {
        v = src[k0 + m];
        if (p.qin.on) v = fake_quant(v, p.qin);
      }
      a[m] = v;
    }
    return;
  }
  const float* src = p.hq_scratch
                         ? p.hqbuf + (int64_t)((t - 1) & 1) * p.B * p.H + (int64_t)row * p.H + kbase
                         : p.out + (int64_t)(t - 1) * p.so_t + (int64_t)row * p.so_b + kbase;
  if (p.vec_ok && row_ok && k0 + KC <= klen) {
    const f4* v4 = reinterpret_cast<const f4*>(src + k0);
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const f4 v = v4[q];
      a[4 * q + 0] = v[0];
      a[4 * q + 1] = v[1];
      a[4 * q + 2] = v[2];
      a[4 * q + 3] = v[3];
    }
  } else {
#pragma unroll
    for (int m = 0; m < KC; ++m) a[m] = (row_ok && k0 + m < klen) ? src[k0 + m] : 0.0f;
  }
}

// Loads Wh slice: w[((gate*nb + blk)*bs + o)*bs + k] for o = o0 + (lane&3),
// k = KC*kb4 + m; zero where o >= bs or k >= bs.
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
      const int k = KC * kb4 + m;
      wr[g][m] = (ok && k < bs) ? row[k] : 0.0f;
    }
  }
}

template <int KC>
__device__ __forceinline__ void mfma3(const float (&a)[KC], const float (&wr)[3][KC], f4 (&acc)[3]) {
  f4 acc0[3], acc1[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    acc0[g] = f4{0.f, 0.f, 0.f, 0.f};
    acc1[g] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int m = 0; m < KC; m += 2) {
#pragma unroll
    for (int g = 0; g < 3; ++g) acc0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[m], wr[g][m], acc0[g], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 3; ++g)
      acc1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[m + 1], wr[g][m + 1], acc1[g], 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < 3; ++g) acc[g] = acc0[g] + acc1[g];
}

// Per-gate MFMA chain for the second Monarch factor (each gate has its own A).
template <int KC>
__device__ __forceinline__ void mfma3_sep(const float (&a)[3][KC], const float (&wr)[3][KC],
                                          f4 (&acc)[3]) {
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
      acc0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[g][m], wr[g][m], acc0[g], 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 3; ++g)
      acc1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[g][m + 1], wr[g][m + 1], acc1[g], 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < 3; ++g) acc[g] = acc0[g] + acc1[g];
}

// Gate epilogue for (row, unit): all lanes compute, lanes 0..15 store.
__device__ __forceinline__ void epilogue(const MParams& p, int t, int row, int unit, bool store,
                                         const float (&gh)[3], const float (&bias)[3], float gir,
                                         float giz, float gin, float hprev) {
  float hn = gru_update(gir, giz, gin, gh[0] + bias[0], gh[1] + bias[1], gh[2] + bias[2], hprev);
  if (p.qout.on) hn = fake_quant(hn, p.qout);
  if (store) {
    p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + unit] = hn;
    if (p.hq_scratch)
      p.hqbuf[(int64_t)(t & 1) * p.B * p.H + (int64_t)row * p.H + unit] = fake_quant(hn, p.qin);
  }
}

__device__ __forceinline__ void step_sync(const MParams& p, int gid, int t) {
  if (p.coop) {
    group_barrier(p.ctrl, gid, (uint32_t)p.P * (uint32_t)(t + 1));
  } else {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
}

template <int KIND, int KC, int NT>
__global__ __launch_bounds__(NT) void mfma_scan_kernel(MParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int j = lane & 3;          // unit within the quad (B and D column)
  const int kb4 = lane >> 2;       // k-slice (MFMA block)
  const int s = (lane >> 2) & 3;   // D row owned after the reduction
  const bool lead = lane < 16;     // lanes that store

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
  const int kbase = blk * p.bs;

  float wr[3][KC];
  load_w<KC>(p.w, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wr);
  float wl[3][KC];
  if (KIND == kMonarch2) load_w<KC>(p.w2, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wl);

  // Epilogue unit of this lane. Two-factor Monarch: the second factor's row
  // vi = blk*bs + o0 + j lands on y[(vi % nb) * bs + vi / nb] (P^T).
  const int vi = kbase + o0 + j;
  const bool unit_ok = blk_ok && (o0 + j) < p.bs;
  const int unit = (KIND == kMonarch2) ? (vi % p.nb) * p.bs + vi / p.nb : vi;
  float bias[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) bias[g] = unit_ok ? p.bh[g * p.H + unit] : 0.0f;

  const int rb_begin = set * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);

  for (int t = 0; t < p.T; ++t) {
    if (KIND != kMonarch2) {
      for (int rb = rb_begin; rb < rb_end; ++rb) {
        const int row = 4 * rb + s;
        const bool row_ok = row < p.B;
        const bool store = lead && row_ok && unit_ok;
        float gir = 0.f, giz = 0.f, gin = 0.f, hprev = 0.f;
        if (row_ok && unit_ok) {
          const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + unit;
          gir = g[0];
          giz = g[p.H];
          gin = g[2 * p.H];
          hprev = (t == 0) ? p.h0[(int64_t)row * p.sh0_b + unit]
                           : p.out[(int64_t)(t - 1) * p.so_t + (int64_t)row * p.so_b + unit];
        }
        float a[KC];
        load_hq<KC>(p, t, 4 * rb + j, kbase, p.bs, kb4, a);
        f4 acc[3];
        mfma3<KC>(a, wr, acc);
        float gh[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);
        epilogue(p, t, row, unit, store, gh, bias, gir, giz, gin, hprev);
      }
    } else {
      // Phase 1: z_g = R_g q_in(h), block-local.
      for (int rb = rb_begin; rb < rb_end; ++rb) {
        const int row = 4 * rb + s;
        float a[KC];
        load_hq<KC>(p, t, 4 * rb + j, kbase, p.bs, kb4, a);
        f4 acc[3];
        mfma3<KC>(a, wr, acc);
        float z[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) z[g] = reduce16(acc[g], s);
        if (lead && row < p.B && unit_ok) {
#pragma unroll
          for (int g = 0; g < 3; ++g)
            p.zbuf[((int64_t)g * p.B + row) * p.H + vi] = z[g];
        }
      }
      step_sync(p, gid, 2 * t);
      // Phase 2: v_g = L_g (P z_g); gh lands at y = P^T v.
      for (int rb = rb_begin; rb < rb_end; ++rb) {
        const int row = 4 * rb + s;
        const bool row_ok = row < p.B;
        const bool store = lead && row_ok && unit_ok;
        float gir = 0.f, giz = 0.f, gin = 0.f, hprev = 0.f;
        if (row_ok && unit_ok) {
          const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + unit;
          gir = g[0];
          giz = g[p.H];
          gin = g[2 * p.H];
          hprev = (t == 0) ? p.h0[(int64_t)row * p.sh0_b + unit]
                           : p.out[(int64_t)(t - 1) * p.so_t + (int64_t)row * p.so_b + unit];
        }
        const int arow = 4 * rb + j;
        float a[3][KC];
#pragma unroll
        for (int m = 0; m < KC; ++m) {
          const int k = KC * kb4 + m;
          const bool ok = arow < p.B && k < p.bs && blk_ok;
          const int idx = kbase + k;                       // position in P z
          const int src = (idx % p.nb) * p.bs + idx / p.nb;  // position in z
#pragma unroll
          for (int g = 0; g < 3; ++g)
            a[g][m] = ok ? p.zbuf[((int64_t)g * p.B + arow) * p.H + src] : 0.0f;
        }
        f4 acc[3];
        mfma3_sep<KC>(a, wl, acc);
        float gh[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);
        epilogue(p, t, row, unit, store, gh, bias, gir, giz, gin, hprev);
      }
    }
    if (t + 1 < p.T) step_sync(p, gid, KIND == kMonarch2 ? 2 * t + 1 : t);
  }
  if (p.coop) leave_grid(p.ctrl, p.ngroups, (uint32_t)p.nwg);
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

template <int KIND>
KernelFn pick_kernel(int KC, int* nt) {
  switch (KC) {
    case 4: *nt = 1024; return mfma_scan_kernel<KIND, 4, 1024>;
    case 8: *nt = 1024; return mfma_scan_kernel<KIND, 8, 1024>;
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
  int kind, KC, nt, nw, P, G, RB, nrb, ngroups, nwg, coop, nb, bs, qpb;
  int64_t counters_bytes, hq_bytes, z_bytes;
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
  const int quads = (kind == kMonarch1) ? pl->qpb : pl->nb * pl->qpb;
  const int nwmax = pl->KC >= 16 ? 4 : 16;
  pl->nw = quads < nwmax ? quads : nwmax;
  pl->P = (quads + pl->nw - 1) / pl->nw;
  pl->coop = pl->P > 1;
  pl->nrb = (int)((a->B + 3) / 4);
  const int64_t max_groups = (int64_t)pl->nrb * (kind == kMonarch1 ? pl->nb : 1);
  pl->counters_bytes = pl->coop ? align256(max_groups * kCounterBytes) : 0;
  const bool hq_scratch = a->q_in.enabled && !same_quant(a->q_in, a->q_out);
  pl->hq_bytes = hq_scratch ? align256(2 * a->B * a->H * 4) : 0;
  pl->z_bytes = (kind == kMonarch2) ? align256(3 * a->B * a->H * 4) : 0;
  return GS_OK;
}

int64_t workspace_bytes_for(int kind, const gs_args* a) {
  Plan pl;
  const int rc = plan_static(kind, a, &pl, "gs_workspace_bytes");
  if (rc) return rc;
  return kCtrlBytes + pl.counters_bytes + pl.hq_bytes + pl.z_bytes;
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
  const int64_t need = kCtrlBytes + pl.counters_bytes + pl.hq_bytes + pl.z_bytes;
  rc = check_workspace(a, need, who);
  if (rc) return rc;

  KernelFn fn = pick(kind, pl.KC, &pl.nt);
  if (!fn) return set_error(GS_ERR_INVALID, "%s: no kernel for KC=%d", who, pl.KC);
  const int threads = pl.nw * 64;

  const int per_set = pl.P * (kind == kMonarch1 ? pl.nb : 1);
  int G = pl.nrb;
  if (pl.coop) {
    DevInfo di;
    rc = device_info(&di);
    if (rc) return rc;
    if (!di.coop) return set_error(GS_ERR_CAPACITY, "%s: device does not support cooperative launch", who);
    int occ = 0;
    GS_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)fn, threads, 0));
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
  p.ctrl = ctrl_of(ws ? ws : nullptr);
  p.hqbuf = pl.hq_bytes ? reinterpret_cast<float*>(ws + kCtrlBytes + pl.counters_bytes) : nullptr;
  p.zbuf = pl.z_bytes ? reinterpret_cast<float*>(ws + kCtrlBytes + pl.counters_bytes + pl.hq_bytes)
                      : nullptr;
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
  p.P = pl.P;
  p.nwg = pl.nwg;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.hq_scratch = pl.hq_bytes != 0;
  const bool out_aligned = (reinterpret_cast<uintptr_t>(a->out) & 15u) == 0 && a->so_b % 4 == 0 &&
                           a->so_t % 4 == 0;
  p.vec_ok = (pl.bs % 4 == 0) && (a->H % 4 == 0) && (p.hq_scratch || out_aligned);
  p.coop = pl.coop;

  if (pl.coop) {
    void* kargs[] = {&p};
    GS_CHECK_HIP(hipLaunchCooperativeKernel((const void*)fn, dim3(pl.nwg), dim3(threads), kargs, 0, stream));
  } else {
    hipLaunchKernelGGL(fn, dim3(pl.nwg), dim3(threads), 0, stream, p);
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
