// Two-factor Monarch GRU scan forward on fp32 MFMA (gfx950).
//
// Hidden map (no reference counterpart; the single-factor form is
// LarocheC/gru-triton src/gru_qat/triton_kernels/scan_monarch.py:74-127):
//   gh_g = P^T L_g P R_g q_in(h) + bh_g,   (P z)[c * nb + a] = z[a * bs + c],
// with R_g = w[g], L_g = w2[g] block-diagonal ([nb, bs, bs] as (out, in)).
//
// monarch2_fused_kernel (bs <= 64, nb | bs, bs / nb a multiple of 4). One
// workgroup per block b of L and set of row-blocks. Block b of y = P z reads
// z[a * bs + c] for every first-factor block a and c in [b cpb, (b + 1) cpb),
// cpb = bs / nb, so the workgroup computes exactly those bs entries of z_g
// itself (phase 1, quads of 4 consecutive c under one a), stages them in LDS
// (quad order, below), multiplies by L_g[b] (phase 2) and runs the gate epilogue for
// the units y = P^T v places its outputs on. One exchange per step, of
// q_in(h_t), exactly as in the dense kernel: compute waves publish tagged
// words and eight poller waves, two per batch row, stage the next step's
// q_in(h) and gate inputs into LDS.
//
// monarch2_split_kernel (any nb, bs). A group covers all H units for its
// row-blocks. Phase 1: each wave's quad of R rows gives z_g = R_g q_in(h) for 4
// units, published as tagged words. Phase 2: each workgroup stages P z_g for
// its block (polling the z words), multiplies by L_g and lands the result on
// y = P^T v. Two exchanges per step.
#include "gs_mfma.h"

namespace gs {
namespace {

constexpr int kPollers = 8;  // fused kernel: poller waves per workgroup, two per row

struct M2FParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* w2;
  const float* bh;
  float* out;
  uint64_t* xh;  // [2][Bp][H] tagged q_in(h_t)
  uint64_t* xw;  // [nwg] tagged XCD ids
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int nb, bs, cpb, nq;  // nq = bs / 4 quads per phase
  int ngroups, RB, nrb, Bp, nwg;
  int nwc;       // compute waves per workgroup (quad groups, ceil(nq / 4))
  int hs, zs;    // LDS row strides of the staged q_in(h) and z (floats)
  int hpad;      // pad floats after every 256 units of a staged q_in(h) row (0 unless 256 % bs == 0)
  int ks, gs;    // LDS row strides of the raw h and of the staged gate inputs (floats)
  Quant qin, qout;
  int qin_after_first;
  float pscale;  // packed exchange: the scale of the published levels
  float pbias;   // -128 pscale (exact)
};

// Unit of H that output i of L-block b lands on: y = P^T v, v index m = b bs + i.
__device__ __forceinline__ int m2_unit(int m, int nb, int bs) { return (m % nb) * bs + m / nb; }

// LDS chunk of z quad qd: qd with bits 0 and 2 swapped when `swap` (an
// involution, so also the inverse map).
__device__ __forceinline__ int m2_zchunk(int qd, int swap) {
  return swap ? (qd & ~5) | ((qd & 1) << 2) | ((qd >> 2) & 1) : qd;
}

// Sum of a quad-group MFMA's four K slices, picked for the lane's row: the
// chain's D holds, in lane 16 qs + 4 sl + j, VGPR v = slice sl's partial for
// row v, unit j of quad qs. Two row rotations sum the slices (every lane of a
// quad column then holds all four rows), and the lane keeps row sl.
__device__ __forceinline__ float slice_sum(f4 acc, int sl) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += row_ror<8>(acc[c]);
    acc[c] += row_ror<4>(acc[c]);
  }
  const float lo = (sl & 1) ? acc[1] : acc[0];
  const float hi = (sl & 1) ? acc[3] : acc[2];
  return (sl & 2) ? hi : lo;
}

// Fused kernel. Quad-group MFMA layout: lane l = 16 qs + 4 sl + j supplies
// A[row j] and B[unit j] of K slice sl for quad qs, so one
// v_mfma_f32_4x4x1_16b_f32 covers 4 quads (16 outputs) x 4 rows x 4 K slices
// and a chain of SP instructions covers K = 4 SP (slice sl takes k in
// [sl SP, sl SP + SP)). The slice sum is two row rotations per accumulator
// row (slice_sum), and every lane ends with one (row, output): phase 2's
// gate epilogue runs on all 64 lanes. Compute wave w owns quads 4 w .. 4 w + 3
// of both phases; three gate chains, two accumulators each.
// EXACT: bs == 4 SP; otherwise phase-1 operands past the block are zeroed.
//
// LDS layout, for gfx950's banks as measured (4-byte accesses: 32 banks, 32
// lanes a pass; 16-byte reads: 64 banks, 16 lanes a pass, lane groups
// 8 i .. 8 i + 7 paired {0, 3}, {1, 2}, {4, 7}, {5, 6}). z sits in quad order:
// entry j of phase-1 quad qd at 4 m2_zchunk(qd) + j of each batch row, and
// phase 2's weights are gathered to match. A 32-lane pass of the z stores
// then covers two quads whose chunks lie 4 apart, times four rows 4 floats
// apart: 32 banks. Row strides of 4 mod 64 keep the 16-byte operand reads of
// both phases on 64 banks; the raw h and gate-input rows are 8 mod 32 apart,
// so the epilogue's 32-lane accesses (4 rows x 8 consecutive outputs) hit 32
// banks; and the pad after every 256 units of a staged q_in(h) row spreads the
// packed decode's stores (units 256 apart) across banks.
//
// PM > 0: packed exchange, for a published q_in(h) that is a fake-quant level
// in [-128, 127] times pscale (int8 hidden quant). A quad's four lanes of one
// row put their four levels, one byte each (level + 128 of output 4 qd + e in
// byte e), into one tagged word at row position b nq + qd, so a row has H / 4
// words instead of H, and each poller wave polls PM words per lane. The
// consumer's value fma(byte, pscale, -128 pscale) rounds (byte - 128) pscale
// once (-128 pscale is exact), so it is bit for bit the producer's fake_quant
// result. (Bytes are stored biased because this compiler folded a signed byte
// extract and an int-to-float conversion into an unsigned conversion of the
// sign-extended byte, which decodes negative levels wrongly.)
template <int SP, bool EXACT, int PM, int NT>
__global__ __launch_bounds__(NT) void monarch2_fused_kernel(M2FParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwc = p.nwc;
  const bool poller = wave >= nwc;
  const int j = lane & 3, sl = (lane >> 2) & 3, qs = lane >> 4;
  const int bs = p.bs, H = p.H, nb = p.nb;

  const int gid = blockIdx.x % p.ngroups;
  const int b = blockIdx.x / p.ngroups;  // block of L
  const int rb_begin = gid * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);
  const int nrbm = rb_end - rb_begin;
  const int U = bs;  // outputs per workgroup, in y order i = 0 .. bs-1
  const int HS = p.hs, ZS = p.zs, KS = p.ks, GS = p.gs;
  // LDS position of unit k in a staged q_in(h) row (hpad floats after every
  // 256; a block of bs units then never straddles a pad)
  const int hpad = p.hpad;
  auto hx = [hpad](int k) { return k + (k >> 8) * hpad; };

  float* hst = lds;                     // [2][4][HS]   staged q_in(h), row-major (hx)
  float* zst = hst + 8 * HS;            // [3][4][ZS]   z_g of block b in quad order, row-major
  float* hk = zst + 12 * ZS;            // [RB][4][KS]  raw h of this workgroup's units
  float* gst = hk + p.RB * 4 * KS;      // [2][4][GS]   staged gi, [3][U] per row
  int* flags = reinterpret_cast<int*>(gst + 8 * GS);  // [0] compute-wave iterations published,
                                                      // [1] bit 0: group on one XCD, bit 1: a
                                                      // wait of this workgroup gave up
  const int lds_floats = 8 * HS + 12 * ZS + p.RB * 4 * KS + 8 * GS + 4;
  for (int i = threadIdx.x; i < lds_floats; i += blockDim.x) lds[i] = 0.0f;

  const uint32_t base = __hip_atomic_load(ctrl_tag_base(p.ctrl), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const Ctrl ctrl = launch_ctrl(p.ctrl, base);
  if (threadIdx.x == 0) st_tagged(p.xw + blockIdx.x, __uint_as_float(xcc_id()), base + 1u);
  const int niter = p.T * nrbm;
  lds_barrier();

  // Prologue: q_in(h0) of the first row-block, raw h0 and step-0 gate inputs.
  {
    const int rb = rb_begin;
    for (int w = threadIdx.x; w < 4 * H; w += blockDim.x) {
      const int r = w / H, k = w - r * H;
      const int row = 4 * rb + r;
      float v = 0.0f;
      if (row < p.B) {
        v = p.h0[(int64_t)row * p.sh0_b + k];
        if (p.qin.on) v = fake_quant(v, p.qin);
      }
      hst[r * HS + hx(k)] = v;
    }
    for (int w = threadIdx.x; w < nrbm * 4 * U; w += blockDim.x) {
      const int rbl = w / (4 * U), rem = w - rbl * 4 * U, r = rem / U, i = rem - r * U;
      const int row = 4 * (rb_begin + rbl) + r;
      hk[(rbl * 4 + r) * KS + i] = row < p.B ? p.h0[(int64_t)row * p.sh0_b + m2_unit(b * bs + i, nb, bs)] : 0.0f;
    }
    for (int w = threadIdx.x; w < 12 * U; w += blockDim.x) {
      const int r = w / (3 * U), rem = w - r * 3 * U, g = rem / U, i = rem - g * U;
      const int row = 4 * rb + r;
      gst[r * GS + rem] = row < p.B ? p.gi[(int64_t)row * p.sg_b + g * H + m2_unit(b * bs + i, nb, bs)] : 0.0f;
    }
  }
  lds_barrier();

  if (!poller) {
    // Quad qd = 4 wave + qs. Phase 1: entries z[a bs + c0 + j] of first-factor
    // block a = qd / (cpb / 4), c0 = b cpb + 4 (qd - a cpb / 4). Phase 2: rows
    // 4 qd + j of L_g[b].
    const int qpa = p.cpb / 4;
    const int qd = 4 * wave + qs;
    const bool qok = qd < p.nq;
    const int a = qok ? qd / qpa : 0;
    const int c0 = b * p.cpb + 4 * (qd - a * qpa);
    // z quads are staged at swapped chunks exactly when nq = SP >= 8
    constexpr int QSW = EXACT && SP >= 8 ? 1 : 0;
    const int zpos = 4 * m2_zchunk(qd, QSW) + j;  // this lane's z entry (row sl)
    // Phase-2 K position k = 4 i + e holds entry e of quad m2_zchunk(i), whose
    // z index (a', c') is column c' nb + a' of L_g[b] (y order).
    int ycol[SP / 4];
#pragma unroll
    for (int i = 0; i < SP / 4; ++i) {
      const int qk = m2_zchunk(sl * (SP / 4) + i, QSW);
      const int ak = qk / qpa;
      ycol[i] = 4 * (qk - ak * qpa) * nb + ak;
    }
    float wr[3][SP], wl[3][SP];
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const float* r1 = p.w + ((int64_t)(g * nb + a) * bs + c0 + j) * bs;
      const float* r2 = p.w2 + ((int64_t)(g * nb + b) * bs + 4 * qd + j) * bs;
#pragma unroll
      for (int m = 0; m < SP; ++m) {
        const int k = sl * SP + m;
        const bool okk = qok && (EXACT || k < bs);
        wr[g][m] = okk ? r1[k] : 0.0f;
        wl[g][m] = okk ? r2[ycol[m >> 2] + (m & 3) * nb] : 0.0f;
      }
    }
    const int ie = 4 * qd + j;  // this lane's output in y order (row sl)
    const int unit = m2_unit(b * bs + ie, nb, bs);
    float bias[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) bias[g] = qok ? gate_scale(g) * p.bh[g * H + unit] : 0.0f;  // for gru_update_gb
    const int64_t lane_out = (int64_t)sl * p.so_b + unit;  // row = 4 rb + sl
    const int64_t lane_xh = (int64_t)sl * H + unit;
    // phase-1 A: row j of q_in(h), block a, slice sl (a block lies inside one
    // 256-run when hpad is on, so its reads stay contiguous)
    const int a1off = j * HS + hx(a * bs) + sl * SP;
    const int a2off = j * ZS + sl * SP;           // phase-2 A: row j of z_g, slice sl
    float* zw = zst + sl * ZS + zpos;             // phase-1 result of this lane (gate g at + 4 g ZS)

    // (t, rbl) = divmod(it, nrbm), stepped rather than divided
    for (int it = 0, t = 0, rbl = 0; it < niter; ++it, rbl = rbl + 1 == nrbm ? 0 : rbl + 1, t += rbl == 0) {
      const int rb = rb_begin + rbl;
      const int buf = it & 1;
      // phase 1: z_g entries of this wave's quads -> zst (y order)
      {
        float a1[3][SP];
        const float* src = hst + buf * 4 * HS + a1off;
#pragma unroll
        for (int q = 0; q < SP / 4; ++q) {
          const f4 v = *reinterpret_cast<const f4*>(src + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) a1[0][4 * q + e] = (EXACT || sl * SP + 4 * q + e < bs) ? v[e] : 0.0f;
        }
        f4 acc[3];
        mfma3<SP, true>(a1, wr, acc);
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          const float z = slice_sum(acc[g], sl);
          if (qok) zw[4 * g * ZS] = z;
        }
      }
      lds_barrier();
      // Epilogue inputs, read now so that their LDS latency overlaps phase 2
      // (lanes of quads past nq read a clamped address and discard it).
      const int iec = min(ie, U - 1);
      const float* gs_ = gst + buf * 4 * GS + sl * GS + iec;
      const float gir = gs_[0], giz = gs_[U], gin = gs_[2 * U];
      float* hkp = hk + (rbl * 4 + sl) * KS + iec;
      const float hprev = *hkp;
      // flags[1] as staged for this iteration, read as a vector value and made
      // uniform after phase 2: after a give-up the workgroup's outputs are NaN
      // and it publishes nothing more
      const int fl_v = flags[1];
      // the step's store addresses
      const int row = 4 * rb + sl;
      float* const outp = p.out + (int64_t)t * p.so_t + (int64_t)(4 * rb) * p.so_b + lane_out;
      uint64_t* const xdst = PM > 0 ? p.xh + ((int64_t)(t & 1) * p.Bp + 4 * rb + sl) * (H / 4) + b * p.nq + qd
                                    : p.xh + ((int64_t)(t & 1) * p.Bp + 4 * rb) * H + lane_xh;
      // keep these reads and addresses ahead of phase 2 (the scheduler would
      // sink them below its MFMAs, onto the step's chain)
      __builtin_amdgcn_sched_barrier(0);
      // phase 2: L_g[b] times the staged z_g
      float gh[3];
      {
        float a2[3][SP];
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          const float* src = zst + 4 * g * ZS + a2off;
#pragma unroll
          for (int q = 0; q < SP / 4; ++q) {
            const f4 v = *reinterpret_cast<const f4*>(src + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) a2[g][4 * q + e] = v[e];
          }
        }
        f4 acc[3];
        mfma3<SP, false>(a2, wl, acc);
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = slice_sum(acc[g], sl);
      }
      const int fl = __builtin_amdgcn_readfirstlane(fl_v);
      const bool dead = (fl & 2) != 0;
      if (qok) {
        float hn = gru_update_gb(gir, giz, gin, gh[0], gh[1], gh[2], bias[0], bias[1], bias[2], hprev);
        float lv = 0.0f;  // level of the published value (packed exchange)
        if (p.qout.on) {
          lv = quant_level(hn, p.qout);
          hn = lv * p.qout.scale;
        }
        *hkp = hn;
        if (t + 1 < p.T && !dead) {
          float hq = hn;
          if (p.qin_after_first) {
            lv = quant_level(hn, p.qin);
            hq = lv * p.qin.scale;
          }
          const uint32_t tag = base + (uint32_t)t + 1u;
          const bool xl = (fl & 1) != 0;
          if constexpr (PM > 0) {
            // the quad's four levels, byte e from lane j = e (a quad is all active or all idle)
            const int c = ((int)lv + 128) & 0xff;
            const int c0 = __builtin_amdgcn_mov_dpp(c, 0x00, 0xF, 0xF, true);
            const int c1 = __builtin_amdgcn_mov_dpp(c, 0x55, 0xF, 0xF, true);
            const int c2 = __builtin_amdgcn_mov_dpp(c, 0xAA, 0xF, 0xF, true);
            const int c3 = __builtin_amdgcn_mov_dpp(c, 0xFF, 0xF, 0xF, true);
            const uint32_t word = (uint32_t)c0 | ((uint32_t)c1 << 8) | ((uint32_t)c2 << 16) | ((uint32_t)c3 << 24);
            if (j == 0) {
              if (xl)
                st_tagged_xcd(xdst, __uint_as_float(word), tag);
              else
                st_tagged(xdst, __uint_as_float(word), tag);
            }
          } else {
            if (xl)
              st_tagged_xcd(xdst, hq, tag);
            else
              st_tagged(xdst, hq, tag);
          }
        }
        // the output store after the publish, off the exchange's chain
        if (row < p.B) *outp = dead ? __builtin_nanf("") : hn;
      }
      if (lane == 0) __hip_atomic_fetch_add(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
    }
  } else {
    // Poller waves 2 pr + part stage row pr of iteration it + 1 (see the dense
    // kernel), each half of the row's words.
    const int pq = wave - nwc;
    const int pr = pq >> 1, part = pq & 1;
    // first k of part 1: a multiple of 256 when q_in(h) rows are padded, so
    // that the 256-word poll chunks below stay contiguous in LDS
    const int kh = hpad ? (H / 2 + 255) / 256 * 256 : (H + 127) / 128 * 64;
    // Packed exchange: this wave polls words part 64 PM + lane + 64 m (m < PM)
    // of a row, word w carrying outputs 4 qd + e (e < 4) of workgroup b' =
    // w / nq, qd = w % nq, which land on units un[m][e].
    constexpr int PMX = PM > 0 ? PM : 1;
    int un[PMX][4];
    const int nwrow = H / 4;  // packed words per row
#pragma unroll
    for (int m = 0; m < PMX; ++m) {
      const int w = part * 64 * PM + lane + 64 * m;
      const int bw = w / p.nq, qw = w - bw * p.nq;
#pragma unroll
      for (int e = 0; e < 4; ++e) un[m][e] = PM > 0 && w < nwrow ? hx(m2_unit(bw * bs + 4 * qw + e, nb, bs)) : 0;
    }
    constexpr int NGI = (3 * 64 + 63) / 64;  // 3 U <= 192 gate inputs per row
    for (int it = 0; it < niter; ++it) {
      const int nx = it + 1;
      const bool more = nx < niter;
      const int t2 = nx / nrbm;
      const int rb2 = rb_begin + (nx - t2 * nrbm);
      const int row = 4 * rb2 + pr;
      float gv[NGI];
#pragma unroll
      for (int i = 0; i < NGI; ++i) {
        const int w = lane + 64 * i;
        const int g = w / U, ii = w - g * U;
        const bool okw = more && part == 0 && w < 3 * U && row < p.B;
        gv[i] = okw ? p.gi[(int64_t)t2 * p.sg_t + (int64_t)row * p.sg_b + g * H + m2_unit(b * bs + ii, nb, bs)] : 0.0f;
      }
      lds_barrier();  // the compute waves' phase-1/phase-2 barrier
      if (more) {
        float* hs = hst + (nx & 1) * 4 * HS + pr * HS;
        if (t2 == 0) {
          for (int k = lane + part * kh; k < (part ? H : min(H, kh)); k += 64) {
            float v = 0.0f;
            if (row < p.B) {
              v = p.h0[(int64_t)row * p.sh0_b + k];
              if (p.qin.on) v = fake_quant(v, p.qin);
            }
            hs[hx(k)] = v;
          }
        } else {
          if (pq == 0 && nx == nrbm &&  // first exchange of the launch
              nb <= 64 && group_on_one_xcd(ctrl, p.xw + gid, p.ngroups, nb, base + 1u, &flags[1]))
            __hip_atomic_fetch_or(&flags[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          wait_lds_count(ctrl, &flags[0], nwc * (it + 1), &flags[1]);
          const uint32_t tag = base + (uint32_t)t2;
          if constexpr (PM > 0) {
            // this wave's PM words per lane of row pr's H / 4 packed words
            const int w0 = part * 64 * PM;
            const uint64_t* hb = p.xh + ((int64_t)((t2 - 1) & 1) * p.Bp + row) * nwrow + w0;
            uint64_t v[PMX];
            uint32_t valid = 0;
            if (w0 < nwrow) valid = poll_row_words<PMX>(ctrl, hb, nwrow - w0, tag, v, &flags[1]);
#pragma unroll
            for (int m = 0; m < PMX; ++m) {
              if ((valid >> m) & 1u) {
                const uint32_t x = (uint32_t)v[m];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  hs[un[m][e]] = __builtin_fmaf((float)((x >> (8 * e)) & 0xffu), p.pscale, p.pbias);
              }
            }
          } else {
            const uint64_t* hb = p.xh + ((int64_t)((t2 - 1) & 1) * p.Bp + row) * H;
            // this wave's half of row pr's H words, in chunks of 256
            const int kend = part ? H : min(H, kh);
            for (int k0 = part * kh; k0 < kend; k0 += 256)
              poll_row_il<4, false>(ctrl, hb + k0, hs + hx(k0), pr, min(256, kend - k0), tag, &flags[1]);
          }
        }
        float* gs_ = gst + (nx & 1) * 4 * GS + pr * GS;
        if (part == 0) {
#pragma unroll
          for (int i = 0; i < NGI; ++i) {
            const int w = lane + 64 * i;
            if (w < 3 * U) gs_[w] = gv[i];
          }
        }
      }
      lds_barrier();
    }
  }
  leave_grid(ctrl, (uint32_t)p.nwg, base, (uint32_t)p.T, &flags[1], 2);
}

struct M2Params {
  const float* gi;
  const float* h0;
  const float* w;
  const float* w2;
  const float* bh;
  float* out;
  uint64_t* xh;  // [2][Bp][H] tagged q_in(h_t)
  uint64_t* xz;  // [2][3][Bp][H] tagged first-factor output
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int nb, bs, qpb;
  int nrb, Bp, RB, nwg, ngroups;
  int rs;  // LDS row stride (floats)
  Quant qin, qout;
  int qin_after_first;
};

// Polls `words` tagged words of one exchange slice into LDS, MW per thread and pass.
// Word w maps to (src offset, LDS offset) through addr(w, &src, &dst). `ok`
// turns false when a wait gave up; a thread whose `ok` is already false polls
// nothing.
template <int MW, typename Map>
__device__ __forceinline__ void stage_words(const Ctrl& c, const uint64_t* base, int words, uint32_t tag, float* lds,
                                            Map map, bool& ok, uint32_t forced_tag) {
  const int tid = threadIdx.x, nth = blockDim.x;
  for (int c0 = 0; c0 < words && ok; c0 += MW * nth) {
    int src[MW], dst[MW];
    uint32_t valid = 0;
#pragma unroll
    for (int i = 0; i < MW; ++i) {
      const int w = c0 + tid + i * nth;
      const bool ok = w < words;
      map(ok ? w : 0, src[i], dst[i]);
      valid |= (ok ? 1u : 0u) << i;
    }
    ok = poll_to_lds<MW>(c, base, src, dst, valid, tag, lds, tag == forced_tag);
  }
}

template <int KC, int NT>
__global__ __launch_bounds__(NT) void monarch2_split_kernel(M2Params p) {
  extern __shared__ float lds[];
  constexpr int MWH = (4 * 16 * KC + NT - 1) / NT;
  constexpr int MWZ = (12 * 16 * KC + NT - 1) / NT;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int j = lane & 3, kb4 = lane >> 2, s = (lane >> 2) & 3;
  const bool lead = lane < 16;

  const int gid = blockIdx.x % p.ngroups;
  const int pw = blockIdx.x / p.ngroups;
  const int quad = pw * nw + wave;
  const int blk = quad / p.qpb;
  const int o0 = 4 * (quad - blk * p.qpb);
  const bool blk_ok = blk < p.nb && o0 < p.bs;
  const int wg_blk = (pw * nw) / p.qpb;  // waves per workgroup divide quads per block
  const int klo = wg_blk * p.bs;

  float* hst = lds;             // [2][4][rs]
  float* zst = lds + 8 * p.rs;  // [2][12][rs]
  int* dead = reinterpret_cast<int*>(lds + 32 * p.rs);  // a wait of this workgroup gave up
  for (int i = threadIdx.x; i < 32 * p.rs + 1; i += blockDim.x) lds[i] = 0.0f;
  lds_barrier();

  float wr[3][KC], wl[3][KC];
  load_w<KC>(p.w, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wr);
  load_w<KC>(p.w2, p.nb, p.bs, blk, o0, j, kb4, blk_ok, wl);

  const int vi = blk * p.bs + o0 + j;
  const bool unit_ok = blk_ok && (o0 + j) < p.bs;
  const int unit = (vi % p.nb) * p.bs + vi / p.nb;
  float bias[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) bias[g] = unit_ok ? gate_scale(g) * p.bh[g * p.H + unit] : 0.0f;  // for gru_update_gb

  const uint32_t base = __hip_atomic_load(ctrl_tag_base(p.ctrl), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const Ctrl ctrl = launch_ctrl(p.ctrl, base);
  // tag of the exchange forced late (launch_ctrl; none: a tag no step uses)
  const uint32_t fstep = forced_step(ctrl);
  const uint32_t forced_tag = fstep != 0u ? base + fstep : base;
  bool alive = true;  // no wait of this thread has given up
  const int rb_begin = gid * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);
  int hbuf = 0, zbuf = 0;
  const int bs = p.bs, H = p.H, nb = p.nb, rs = p.rs, Bp = p.Bp;

  for (int t = 0; t < p.T; ++t) {
    const uint32_t tag = base + (uint32_t)t + 1u;
    for (int rb = rb_begin; rb < rb_end; ++rb) {
      const int row = 4 * rb + s;
      const bool mine = lead && row < p.B && unit_ok;
      const bool pub = lead && unit_ok;
      float gir = 0.f, giz = 0.f, gin = 0.f, hprev = 0.f;
      if (mine) {
        const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + unit;
        gir = g[0];
        giz = g[H];
        gin = g[2 * H];
        hprev = (t == 0) ? p.h0[(int64_t)row * p.sh0_b + unit]
                         : p.out[(int64_t)(t - 1) * p.so_t + (int64_t)row * p.so_b + unit];
      }
      // Phase 1 input: q_in(h_{t-1}) rows 4rb.., cols of this workgroup's block.
      float* hs = hst + hbuf * 4 * rs;
      hbuf ^= 1;
      if (t == 0) {
        for (int w = threadIdx.x; w < 4 * bs; w += blockDim.x) {
          const int r = w / bs, k = w - r * bs;
          const int row_r = 4 * rb + r;
          float v = 0.0f;
          if (row_r < p.B) {
            v = p.h0[(int64_t)row_r * p.sh0_b + klo + k];
            if (p.qin.on) v = fake_quant(v, p.qin);
          }
          hs[r * rs + k] = v;
        }
      } else {
        const uint64_t* hb = p.xh + ((int64_t)((t - 1) & 1) * Bp + 4 * rb) * H;
        stage_words<MWH>(ctrl, hb, 4 * bs, tag - 1u, hs, [&](int w, int& src, int& dst) {
          const int r = w / bs, k = w - r * bs;
          src = r * H + klo + k;
          dst = r * rs + k;
        }, alive, forced_tag);
        if (!alive) *dead = 1;
      }
      lds_barrier();
      // after a give-up the workgroup's outputs are NaN and it publishes nothing more
      const bool wg_dead = __builtin_amdgcn_readfirstlane(*dead) != 0;
      float a[3][KC];
      lds_a<KC>(hs + j * rs, kb4, a[0]);
      f4 acc[3];
      mfma3<KC, true>(a, wr, acc);
      float gh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);
      if (pub && !wg_dead) {
#pragma unroll
        for (int g = 0; g < 3; ++g) st_tagged(p.xz + ((int64_t)((t & 1) * 3 + g) * Bp + row) * H + vi, gh[g], tag);
      }
      // Phase 2 input: (P z_g)[wg_blk*bs + k], 3 gates x 4 rows.
      float* zs = zst + zbuf * 12 * rs;
      zbuf ^= 1;
      const uint64_t* zb = p.xz + (int64_t)(t & 1) * 3 * Bp * H + (int64_t)4 * rb * H;
      stage_words<MWZ>(ctrl, zb, 12 * bs, tag, zs, [&](int w, int& src, int& dst) {
        const int gr = w / bs, k = w - gr * bs;
        const int idx = wg_blk * bs + k;
        const int zpos = (idx % nb) * bs + idx / nb;
        src = ((gr >> 2) * Bp + (gr & 3)) * H + zpos;
        dst = gr * rs + k;
      }, alive, forced_tag);
      if (!alive) *dead = 1;
      lds_barrier();
      const bool wg_dead2 = __builtin_amdgcn_readfirstlane(*dead) != 0;
#pragma unroll
      for (int g = 0; g < 3; ++g) lds_a<KC>(zs + (g * 4 + j) * rs, kb4, a[g]);
      mfma3<KC, false>(a, wl, acc);
#pragma unroll
      for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);

      float hn = gru_update_gb(gir, giz, gin, gh[0], gh[1], gh[2], bias[0], bias[1], bias[2], hprev);
      if (p.qout.on) hn = fake_quant(hn, p.qout);
      if (mine) p.out[(int64_t)t * p.so_t + (int64_t)row * p.so_b + unit] = wg_dead2 ? __builtin_nanf("") : hn;
      if (pub && t + 1 < p.T && !wg_dead2) {
        const float hq = p.qin_after_first ? fake_quant(hn, p.qin) : hn;
        st_tagged(p.xh + ((int64_t)(t & 1) * Bp + row) * H + unit, hq, tag);
      }
    }
  }
  leave_grid(ctrl, (uint32_t)p.nwg, base, (uint32_t)p.T, dead, 1);
}

typedef void (*M2Fn)(M2Params);

M2Fn pick_split(int KC, int* nt) {
  switch (KC) {
    case 4: *nt = 1024; return monarch2_split_kernel<4, 1024>;
    case 8: *nt = 256; return monarch2_split_kernel<8, 256>;
    case 16: *nt = 256; return monarch2_split_kernel<16, 256>;
    case 32: *nt = 256; return monarch2_split_kernel<32, 256>;
    case 64: *nt = 256; return monarch2_split_kernel<64, 256>;
    default: return nullptr;
  }
}

struct M2Plan {
  int KC, nt, nw, P, nrb, Bp, rs;
  int64_t xh_bytes, xz_bytes;
  size_t lds;
};

int plan_m2(const gs_args* a, M2Plan* pl, const char* who) {
  if (a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != a->H)
    return set_error(GS_ERR_INVALID, "%s: Wh_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                     (long long)a->nblocks, (long long)a->blksz, (long long)a->H);
  const int bs = (int)a->blksz, nb = (int)a->nblocks;
  pl->KC = choose_kc(bs);
  if (pl->KC < 0) return set_error(GS_ERR_INVALID, "%s: block size %d exceeds the supported maximum of 1024", who, bs);
  if (!pick_split(pl->KC, &pl->nt)) return set_error(GS_ERR_INVALID, "%s: no kernel for KC=%d", who, pl->KC);
  const int qpb = (bs + 3) / 4;
  int nw = qpb < pl->nt / 64 ? qpb : pl->nt / 64;
  while (qpb % nw != 0) --nw;
  pl->nw = nw;
  pl->P = nb * qpb / nw;
  pl->nrb = (int)((a->B + 3) / 4);
  pl->Bp = 4 * pl->nrb;
  pl->rs = 16 * pl->KC + 4;
  pl->lds = (size_t)(32 * pl->rs + 1) * sizeof(float);
  pl->xh_bytes = align256(2 * (int64_t)pl->Bp * a->H * 8);
  pl->xz_bytes = align256(6 * (int64_t)pl->Bp * a->H * 8);
  return GS_OK;
}

// ---- fused kernel: host side ---------------------------------------------------

typedef void (*M2FFn)(M2FParams);

struct M2FPlan {
  int nwc, nrb, Bp, hs, zs, pm, hpad, ks, gs;
  float pscale;
  int64_t xh_bytes, xw_bytes;
  M2FFn fn;
};

// The fused kernel covers bs <= 64 with nb | bs and bs / nb a multiple of 4,
// for H <= 2048. A chain covers K = 4 SP with SP in {4, 8, 16}, the smallest
// with 4 SP >= bs.
bool plan_fused(const gs_args* a, M2FPlan* pl) {
  const int nb = (int)a->nblocks, bs = (int)a->blksz, H = (int)a->H;
  if (bs > 64 || bs % nb != 0 || (bs / nb) % 4 != 0 || H > 2048) return false;
  const int nq = bs / 4;
  pl->nwc = (nq + 3) / 4;
  const int SP = bs <= 16 ? 4 : bs <= 32 ? 8 : 16;
  const bool exact = bs == 4 * SP;
  // Packed exchange when the published value is a fake-quant level in
  // [-128, 127] (q_in after q_out, or q_out when q_in repeats it or is off):
  // PM words per lane for each of a row's two poller waves (H <= 16 * 64 for
  // this kernel, so at most 128 words per wave).
  const gs_quant& qp = (a->q_in.enabled && !same_quant(a->q_in, a->q_out)) ? a->q_in : a->q_out;
  const bool pack = qp.enabled && qp.qmin >= -128 && qp.qmax <= 127;
  const int half_words = (H / 4 + 1) / 2;
  if (pack && half_words > 128) return false;
  pl->pm = !pack ? 0 : half_words <= 64 ? 1 : 2;
  pl->pscale = pack ? qp.scale : 1.0f;
  switch (pl->pm * 8 + (SP == 4 ? 0 : SP == 8 ? 1 : 2) * 2 + (exact ? 1 : 0)) {
#define GS_M2F(PMV, SPI, SPV)                                                          \
  case PMV * 8 + SPI * 2 + 1: pl->fn = monarch2_fused_kernel<SPV, true, PMV, 768>; break; \
  case PMV * 8 + SPI * 2 + 0: pl->fn = monarch2_fused_kernel<SPV, false, PMV, 768>; break;
    GS_M2F(0, 0, 4) GS_M2F(0, 1, 8) GS_M2F(0, 2, 16)
    GS_M2F(1, 0, 4) GS_M2F(1, 1, 8) GS_M2F(1, 2, 16)
    GS_M2F(2, 0, 4) GS_M2F(2, 1, 8) GS_M2F(2, 2, 16)
#undef GS_M2F
    default: return false;
  }
  pl->nrb = (int)((a->B + 3) / 4);
  pl->Bp = 4 * pl->nrb;
  // LDS layout (the kernel's comment gives the bank reasoning). Phase-1 reads
  // of the last block run up to 4 SP - bs past H (masked when bs < 4 SP) and
  // stay inside the LDS allocation. The packed decode's 32-lane stores reach
  // H / 256 runs of 256 units (H = 512: 2, 1024: 4), so the pad is 32 / runs
  // banks.
  pl->hpad = 256 % bs != 0 ? 0 : H > 512 ? 8 : 16;
  const int hlen = H + ((H - 1) >> 8) * pl->hpad;  // padded row length
  pl->hs = (hlen + 63) / 64 * 64 + 4;
  pl->zs = 4 * SP + 4;
  pl->ks = (bs + 63) / 64 * 64 + 8;
  pl->gs = (3 * bs + 63) / 64 * 64 + 8;
  // pollers load up to 511 words past the last chunk start of a row
  pl->xh_bytes = align256(2 * (int64_t)pl->Bp * H * 8 + 512 * 8);
  pl->xw_bytes = align256((int64_t)pl->nrb * nb * 8);
  return true;
}

int run_fused(const gs_args* a, const M2FPlan& pl, hipStream_t stream, const char* who) {
  const int nb = (int)a->nblocks, bs = (int)a->blksz;
  const int threads = 64 * (pl.nwc + kPollers);
  int G = pl.nrb, RB = 1;
  size_t lds = 0;
  for (int pass = 0; pass < 2; ++pass) {
    RB = (pl.nrb + G - 1) / G;
    G = (pl.nrb + RB - 1) / RB;
    lds = sizeof(float) * (size_t)(8 * pl.hs + 12 * pl.zs + RB * 4 * pl.ks + 8 * pl.gs + 4);
    if (lds > 65536)
      GS_CHECK_HIP(hipFuncSetAttribute((const void*)pl.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int gfit = 0;
    const int rc = resident_groups((const void*)pl.fn, threads, lds, nb, pl.nrb, &gfit, who);
    if (rc) return rc;
    if (gfit >= G) break;
    G = gfit;
  }
  M2FParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.w2 = a->w2;
  p.bh = a->bh;
  p.out = a->out;
  char* ws = static_cast<char*>(a->workspace);
  p.ctrl = ctrl_of(ws, a->fault_mirror);
  p.xh = reinterpret_cast<uint64_t*>(ws + kCtrlBytes);
  p.xw = reinterpret_cast<uint64_t*>(ws + kCtrlBytes + pl.xh_bytes);
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.nb = nb;
  p.bs = bs;
  p.cpb = bs / nb;
  p.nq = bs / 4;
  p.ngroups = G;
  p.RB = RB;
  p.nrb = pl.nrb;
  p.Bp = pl.Bp;
  p.nwg = G * nb;
  p.nwc = pl.nwc;
  p.hs = pl.hs;
  p.hpad = pl.hpad;
  p.ks = pl.ks;
  p.gs = pl.gs;
  p.zs = pl.zs;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.qin_after_first = a->q_in.enabled && !same_quant(a->q_in, a->q_out);
  p.pscale = pl.pscale;
  p.pbias = -128.0f * pl.pscale;
  hipLaunchKernelGGL(pl.fn, dim3(p.nwg), dim3(threads), lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace

int64_t monarch2_workspace_bytes(const gs_args* a) {
  M2FPlan fp;
  if (a->nblocks >= 1 && a->blksz >= 1 && a->nblocks * a->blksz == a->H && plan_fused(a, &fp))
    return kCtrlBytes + fp.xh_bytes + fp.xw_bytes;
  M2Plan pl;
  const int rc = plan_m2(a, &pl, "gs_workspace_bytes");
  if (rc) return rc;
  return kCtrlBytes + pl.xh_bytes + pl.xz_bytes;
}

int run_monarch2(const gs_args* a, hipStream_t stream, const char* who) {
  M2Plan pl;
  int rc = plan_m2(a, &pl, who);
  if (rc) return rc;
  M2FPlan fp;
  if (plan_fused(a, &fp)) {
    rc = check_workspace(a, kCtrlBytes + fp.xh_bytes + fp.xw_bytes, who);
    if (rc) return rc;
    return run_fused(a, fp, stream, who);
  }
  rc = check_workspace(a, kCtrlBytes + pl.xh_bytes + pl.xz_bytes, who);
  if (rc) return rc;
  M2Fn fn = pick_split(pl.KC, &pl.nt);
  const int threads = pl.nw * 64;
  if (pl.lds > 65536)
    GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds));
  int G = pl.nrb;
  rc = resident_groups((const void*)fn, threads, pl.lds, pl.P, pl.nrb, &G, who);
  if (rc) return rc;
  const int RB = (pl.nrb + G - 1) / G;
  G = (pl.nrb + RB - 1) / RB;

  M2Params p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.w2 = a->w2;
  p.bh = a->bh;
  p.out = a->out;
  char* ws = static_cast<char*>(a->workspace);
  p.ctrl = ctrl_of(ws, a->fault_mirror);
  p.xh = reinterpret_cast<uint64_t*>(ws + kCtrlBytes);
  p.xz = reinterpret_cast<uint64_t*>(ws + kCtrlBytes + pl.xh_bytes);
  p.sg_t = a->sg_t;
  p.sg_b = a->sg_b;
  p.sh0_b = a->sh0_b;
  p.so_t = a->so_t;
  p.so_b = a->so_b;
  p.T = (int)a->T;
  p.B = (int)a->B;
  p.H = (int)a->H;
  p.nb = (int)a->nblocks;
  p.bs = (int)a->blksz;
  p.qpb = (p.bs + 3) / 4;
  p.nrb = pl.nrb;
  p.Bp = pl.Bp;
  p.RB = RB;
  p.nwg = G * pl.P;
  p.ngroups = G;
  p.rs = pl.rs;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.qin_after_first = a->q_in.enabled && !same_quant(a->q_in, a->q_out);
  hipLaunchKernelGGL(fn, dim3(p.nwg), dim3(threads), pl.lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

}  // namespace gs
