// Dense and single-factor Monarch GRU scan forward on fp32 MFMA (gfx950), and
// the dense forward on int8 MFMA when Wh comes as per-row int8 codes (I8).
//
// References (LarocheC/gru-triton src/gru_qat/triton_kernels/):
//   dense    scan.py:76-210 (persistent kernel), scan.py:213-293 (launcher)
//   Monarch  scan_monarch.py:130-291 (kernel), :320-406 (launcher), math :74-127
//
// Work split. Hidden units come in quads of 4; each compute wave owns one quad
// (3 gates x 4 units = 12 rows of Wh, K = H for dense or the block for Monarch)
// and keeps that weight slice in VGPRs for the whole scan. A *group* is the set
// of workgroups that produce every unit a batch row's next step reads (dense:
// all of H; Monarch: one block). Groups own RB row-blocks of 4 batch rows and
// are interleaved in blockIdx (gid = blockIdx % ngroups), which places a group
// on one XCD under round-robin workgroup dispatch.
//
// Per step and row-block a compute wave reads its A operand q_in(h)[4 rows][K]
// and the gate inputs from LDS, runs 3 chains of v_mfma_f32_4x4x1_16b_f32
// (gs_mfma.h), sums the 16 K-slice partials, and the 16 lanes of row 0 run the
// gate epilogue, store out[t] and pass q_in(h_t) on.
//
// Local mode (a group fits in one workgroup): compute waves write q_in(h_t)
// straight into the LDS staging buffer of the next step.
// Remote mode (a group spans workgroups): compute waves publish q_in(h_t) as
// tagged 64-bit words (gs_device.h) and never load from global memory inside
// the loop. Poller waves (one or two per batch row of the row-block) poll
// the words the next iteration needs and stage them, with the next gate
// inputs, into LDS while the compute waves work. The two roles meet
// at one LDS-only barrier per iteration, so no wave ever waits for its own
// stores to be acknowledged. During the first exchange the pollers check that
// their group runs on one XCD; if so, later steps publish with non-temporal
// stores that stay in that XCD's L2, which the group's agent-scope loads see
// sooner than stores written through to memory.
#include "gs_mfma.h"

namespace gs {
namespace {

// kCirculant: the dense scan of a circulant map, Wh_cat[g H + o][k] =
// col_g[(o - k) mod H], each compute wave forming its weight slice from the
// gate columns (Wh_circ [3, H]) instead of loading a materialized map: the
// same weights, so the same products as kDense on that map.
enum : int { kDense = 0, kMonarch1 = 1, kCirculant = 2 };

// The weight slice of a quad from circulant columns: as load_w on the
// materialized map, wr[g][m] = col[g H + (o - k) mod H] for o = o0 + j,
// k = kmap(m, kb4); zero where o >= H or k >= H.
template <int KC>
__device__ __forceinline__ void load_w_circ(const float* col, int H, int o0, int j, int kb4, bool ok_quad,
                                            float (&wr)[3][KC]) {
  const int o = o0 + j;
  const bool ok = ok_quad && o < H;
#pragma unroll
  for (int g = 0; g < 3; ++g) {
#pragma unroll
    for (int m = 0; m < KC; ++m) {
      const int k = kmap(m, kb4);
      const int d = o - k;
      wr[g][m] = (ok && k < H) ? col[g * H + (d < 0 ? d + H : d)] : 0.0f;
    }
  }
}
// Remote mode: poller waves per batch row. Two for KC = 16 and 32, each
// polling half of the row (measured 2 % faster than one at config 1: fewer
// words per lane shorten a poll round); one for KC <= 8, whose workgroups
// already hold up to 12 compute waves, and for KC = 64, whose 192 weight VGPRs
// need the register budget of two waves per SIMD.
constexpr int pollers_per_row(int KC) { return KC == 16 || KC == 32 ? 2 : 1; }

struct DParams {
  const float* gi;
  const float* h0;
  const float* w;
  const float* bh;
  float* out;
  float* gh_save;  // SAVE instances: [T, B, 3H] q_in(h_{t-1}) Wh^T as the step computed it (no bias)
  const int8_t* wq;  // I8 instances: int8 codes of Wh [3H, H], w == fl(code * wsc[row])
  const float* wsc;  // I8 instances: the code scale of each of Wh's 3H rows
  uint64_t* xh;  // remote mode: [2][Bp][H] tagged q_in(h_t)
  uint64_t* xw;  // remote mode: [nwg] tagged XCD ids
  Ctrl ctrl;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int T, B, H;
  int nb, bs, qpb;  // dense: nb = 1, bs = H
  int ngroups, G, RB, nrb, Bp, nwg, P;
  int nwc;  // compute waves per workgroup
  int hsz;  // floats per LDS staging block (4 rows x 16 KC, interleaved)
  int kr, gr;  // LDS row strides of the raw h (U units) and the staged gi (3 U), floats
  Quant qin, qout;
  int qin_after_first;
  float pscale, pbias;  // packed exchange: scale of the published levels, -128 pscale
};

// Packed exchange (PACK, dense remote mode, int8 hidden quant): a published
// q_in(h) that is a fake-quant level in [-128, 127] times pscale travels as
// one tagged word per quad of units and row (the four levels + 128, byte e
// for unit 4 w + e of word w = unit / 4), H / 4 words per row instead of H.
// A poller decodes a word into the four consecutive staged slots of its units
// with fma(byte, pscale, -128 pscale), bit for bit the producer's value (see
// the two-factor Monarch kernel, which packs the same way).
// Units per workgroup in dense remote mode (compute waves x 4).
__host__ __device__ constexpr int dense_remote_units(int KC) { return 4 * (KC >= 16 ? 4 : 12); }
// LDS row stride of a row of n floats that a wave reads as 4 rows x 4 units.
__host__ __device__ constexpr int row_stride_pad(int n) { return n % 16 == 0 ? n + 4 : n; }

// Int8 weights (I8, dense remote mode with the packed exchange, q_in on and
// the published levels in q_in's scale): Wh arrives as per-row int8 codes and
// scales, every A operand (q_in(h0) and each exchanged q_in(h_t)) is a level
// times that scale, so the step's products run on v_mfma_i32_4x4x4_16b_i8 over
// the levels and codes (exact integer sums, a quarter of the fp32 chain's
// instructions) and gh = sum * (code scale * level scale). The operand block
// is staged as int8 levels (i8_index) instead of floats.
template <int KIND, int KC, int NT, bool REMOTE, bool PACK = false, bool SAVE = false, bool I8 = false>
__global__ __launch_bounds__(NT) void scan_kernel(DParams p) {
  static_assert(!I8 || (KIND == kDense && REMOTE && PACK && !SAVE), "int8 weights: dense, remote, packed exchange");
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwc = p.nwc;
  const bool poller = REMOTE && wave >= nwc;
  const int j = lane & 3, kb4 = lane >> 2, s = (lane >> 2) & 3;
  const bool lead = lane < 16;

  const int gid = blockIdx.x % p.ngroups;
  const int pw = blockIdx.x / p.ngroups;
  const int set = (KIND == kMonarch1) ? gid % p.G : gid;
  const int blk_g = (KIND == kMonarch1) ? gid / p.G : 0;  // the group's block (dense: 0)
  const int klo = blk_g * p.bs;                           // K range [klo, klo + bs)
  const int quad = pw * nwc + wave;                       // within the group's K range
  const int o0 = 4 * quad;
  const bool quad_ok = !poller && o0 < p.bs;
  const int U = 4 * nwc;               // units per workgroup
  const int ulo = klo + 4 * pw * nwc;  // first unit of this workgroup
  const int unit = ulo + 4 * wave + j;
  const bool unit_ok = quad_ok && (o0 + j) < p.bs;

  const int rb_begin = set * p.RB;
  const int rb_end = min(rb_begin + p.RB, p.nrb);
  const int nrbm = rb_end - rb_begin;

  float* hst = lds;                  // [2][hsz]     staged q_in(h) of the K range (il_index)
  // The raw h and gi rows are read (and h written) by a wave as 4 rows x 4
  // consecutive units: row strides that are not multiples of 16 floats put
  // the four rows on different banks of each 32-lane pass. Dense remote mode
  // has U = 4 nwc fixed by KC (16 or 48), so its strides are constants.
  constexpr int UD = ((KIND == kDense || KIND == kCirculant) && REMOTE) ? dense_remote_units(KC) : 0;
  const int KR = UD ? row_stride_pad(UD) : p.kr, GR = UD ? row_stride_pad(3 * UD) : p.gr;
  float* hk = hst + 2 * p.hsz;       // [RB][4][KR]  raw h of this workgroup's units
  float* gst = hk + p.RB * 4 * KR;   // [2][4][GR]   staged gi, [3][U] per row (remote mode)
  int* flags = reinterpret_cast<int*>(gst + 8 * GR);  // remote mode: [0] compute-wave iterations
                                                      // published, [1] bit 0: group on one XCD,
                                                      // bit 1: a wait of this workgroup gave up
  // The compute waves' Wh slice is loaded first, so that its latency overlaps
  // the LDS clear and the prologue (T = 1 and 64: 0.6 and 1.8 us less).
  float wr[3][I8 ? 1 : KC];
  int wi[3][I8 ? KC / 4 : 1];
  if (!poller) {
    if constexpr (I8)
      load_wi<KC>(p.wq, p.H, o0, j, kb4, quad_ok, wi);
    else if constexpr (KIND == kCirculant)
      load_w_circ<KC>(p.w, p.H, o0, j, kb4, quad_ok, wr);
    else
      load_w<KC>(p.w, p.nb, p.bs, blk_g, o0, j, kb4, quad_ok, wr);
  }
  const int lds_floats = 2 * p.hsz + p.RB * 4 * KR + (REMOTE ? 8 * GR + 4 : 0);
  for (int i = threadIdx.x; i < lds_floats; i += blockDim.x) lds[i] = 0.0f;

  const uint32_t base = REMOTE ? __hip_atomic_load(ctrl_tag_base(p.ctrl), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
  const Ctrl ctrl = launch_ctrl(p.ctrl, base);
  if (REMOTE && threadIdx.x == 0) st_tagged(p.xw + blockIdx.x, __uint_as_float(xcc_id()), base + 1u);
  const int niter = p.T * nrbm;

  // Prologue (all waves): step-0 inputs of the first row-block, raw h0 of all.
  lds_barrier();
  {
    const int rb = rb_begin;
    for (int w = threadIdx.x; w < 4 * p.bs; w += blockDim.x) {
      const int r = w / p.bs, k = w - r * p.bs;
      const int row = 4 * rb + r;
      if constexpr (I8) {
        // the level of q_in(h0) (q_in is on in every I8 launch)
        const int lv = row < p.B ? (int)quant_level(p.h0[(int64_t)row * p.sh0_b + klo + k], p.qin) : 0;
        reinterpret_cast<int8_t*>(hst)[4 * i8_index(r, k >> 2) + (k & 3)] = (int8_t)lv;
      } else {
        float v = 0.0f;
        if (row < p.B) {
          v = p.h0[(int64_t)row * p.sh0_b + klo + k];
          if (p.qin.on) v = fake_quant(v, p.qin);
        }
        hst[il_index(r, k)] = v;
      }
    }
    for (int w = threadIdx.x; w < nrbm * 4 * U; w += blockDim.x) {
      const int rbl = w / (4 * U), rem = w - rbl * 4 * U, r = rem / U, u = rem - r * U;
      const int row = 4 * (rb_begin + rbl) + r;
      const bool ok = row < p.B && (ulo + u - klo) < p.bs;
      hk[(rbl * 4 + r) * KR + u] = ok ? p.h0[(int64_t)row * p.sh0_b + ulo + u] : 0.0f;
    }
    if (REMOTE) {
      for (int w = threadIdx.x; w < 12 * U; w += blockDim.x) {
        const int r = w / (3 * U), rem = w - r * 3 * U, g = rem / U, u = rem - g * U;
        const int row = 4 * rb + r;
        const bool ok = row < p.B && (ulo + u - klo) < p.bs;
        gst[r * GR + rem] = ok ? p.gi[(int64_t)row * p.sg_b + g * p.H + ulo + u] : 0.0f;
      }
    }
  }
  lds_barrier();

  // The compute waves and the poller waves run separate loops with the same
  // number of iterations and one barrier each, so each role's registers are
  // allocated only for its own live values.
  if (!poller) {
    // biases pre-scaled for gru_update_l2 (-log2e for r and z, 2 log2e for n)
    constexpr float kR = -kLog2e, kN = 2.0f * kLog2e;
    float bias[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) bias[g] = unit_ok ? (g == 2 ? kN : kR) * p.bh[g * p.H + unit] : 0.0f;
    // I8: gh = integer sum * (row's code scale * level scale)
    float gsc[3] = {0.0f, 0.0f, 0.0f};
    if constexpr (I8) {
#pragma unroll
      for (int g = 0; g < 3; ++g) gsc[g] = unit_ok ? p.wsc[g * p.H + unit] * p.pscale : 0.0f;
    }
    // lane parts of the out / exchange-word offsets (row = 4 rb + s)
    const int64_t lane_out = (int64_t)s * p.so_b + unit;
    const int64_t lane_xh = (int64_t)s * p.H + unit;
    // (t, rbl) = divmod(it, nrbm), stepped rather than divided
    for (int it = 0, t = 0, rbl = 0; it < niter; ++it, rbl = rbl + 1 == nrbm ? 0 : rbl + 1, t += rbl == 0) {
      const int rb = rb_begin + rbl;
      const int buf = it & 1;
      const int row = 4 * rb + s;
      const bool mine = lead && row < p.B && unit_ok;
      float gir = 0.f, giz = 0.f, gin = 0.f;
      if (REMOTE) {
        const float* gs_ = gst + buf * 4 * GR + s * GR + 4 * wave + j;
        gir = gs_[0];
        giz = gs_[U];
        gin = gs_[2 * U];
      } else if (mine) {
        const float* g = p.gi + (int64_t)t * p.sg_t + (int64_t)row * p.sg_b + unit;
        gir = g[0];
        giz = g[p.H];
        gin = g[2 * p.H];
      }
      // gate-input parts of the exp2 arguments, off the step's dependent chain
      const float cr = __builtin_fmaf(kR, gir, bias[0]), cz = __builtin_fmaf(kR, giz, bias[1]), an2 = kN * gin;
      float* hkp = hk + (rbl * 4 + s) * KR + 4 * wave + j;
      const float hprev = *hkp;
      // flags[1] as staged for this iteration (read as a vector value, made
      // uniform after the MFMAs): after a give-up the workgroup's outputs are
      // NaN and it publishes nothing more
      const int fl_v = REMOTE ? flags[1] : 0;
      // the step's store addresses
      float* const outp = p.out + (int64_t)t * p.so_t + (int64_t)(4 * rb) * p.so_b + lane_out;
      uint64_t* const xdst = !REMOTE ? nullptr
                             : PACK  ? p.xh + ((int64_t)(t & 1) * p.Bp + 4 * rb + s) * (p.H / 4) + (unit >> 2)
                                     : p.xh + ((int64_t)(t & 1) * p.Bp + 4 * rb) * p.H + lane_xh;
      // the epilogue's LDS reads and the store addresses are issued before the
      // MFMAs, so that none of them is on the chain after the last one
      __builtin_amdgcn_sched_barrier(0);
      float gh[3];
      if constexpr (I8) {
        int ai[KC / 4];
        lds_a_i8<KC>(reinterpret_cast<const int*>(hst + buf * p.hsz), lane, ai);
        i4 acc[3];
        mfma3_i8<KC>(ai, wi, acc);
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = reduce16(i4_to_f4(acc[g]), s) * gsc[g];
      } else {
        float a[3][KC];
        lds_a_il<KC>(hst + buf * p.hsz, lane, a[0]);
        f4 acc[3];
        mfma3<KC, true>(a, wr, acc);
#pragma unroll
        for (int g = 0; g < 3; ++g) gh[g] = reduce16(acc[g], s);
      }
      float hn = gru_update_l2(__builtin_fmaf(kR, gh[0], cr), __builtin_fmaf(kR, gh[1], cz),
                               __builtin_fmaf(kN, gh[2], bias[2]), an2, hprev);
      float lv = 0.0f;  // level of the published value (packed exchange)
      if (p.qout.on) {
        lv = quant_level(hn, p.qout);
        hn = lv * p.qout.scale;
      }
      const int fl = REMOTE ? __builtin_amdgcn_readfirstlane(fl_v) : 0;
      // bit 0: a poller of this workgroup has seen every workgroup of the group
      // on this XCD (first exchange), so a publish may stay in the XCD's L2
      const bool xcd_local = (fl & 1) != 0;
      const bool dead = (fl & 2) != 0;
      if (lead && unit_ok) {
        *hkp = hn;
        if (t + 1 < p.T && !dead) {
          float hq = hn;
          if (p.qin_after_first) {
            lv = quant_level(hn, p.qin);
            hq = lv * p.qin.scale;
          }
          if constexpr (PACK) {
            // lanes 4 s + j of one row hold the quad's four units (all valid or none)
            const int c = ((int)lv + 128) & 0xff;
            const int c0 = __builtin_amdgcn_mov_dpp(c, 0x00, 0xF, 0xF, true);
            const int c1 = __builtin_amdgcn_mov_dpp(c, 0x55, 0xF, 0xF, true);
            const int c2 = __builtin_amdgcn_mov_dpp(c, 0xAA, 0xF, 0xF, true);
            const int c3 = __builtin_amdgcn_mov_dpp(c, 0xFF, 0xF, 0xF, true);
            const uint32_t word = (uint32_t)c0 | ((uint32_t)c1 << 8) | ((uint32_t)c2 << 16) | ((uint32_t)c3 << 24);
            if (j == 0) {
              if (xcd_local)
                st_tagged_xcd(xdst, __uint_as_float(word), base + (uint32_t)t + 1u);
              else
                st_tagged(xdst, __uint_as_float(word), base + (uint32_t)t + 1u);
            }
          } else if (REMOTE) {
            if (xcd_local)
              st_tagged_xcd(xdst, hq, base + (uint32_t)t + 1u);
            else
              st_tagged(xdst, hq, base + (uint32_t)t + 1u);
          } else {
            hst[(buf ^ 1) * p.hsz + il_index(s, unit - klo)] = hq;  // local mode: RB == 1
          }
        }
      }
      // fp32 words: counted as published before the output store, so that the
      // pollers start one store earlier (config 1 0.1136 -> 0.1106 ms; the
      // packed instances measured 1 % slower that way and count after it)
      if (REMOTE && !PACK && lane == 0) __hip_atomic_fetch_add(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (mine) *outp = dead ? __builtin_nanf("") : hn;
      if constexpr (SAVE) {
        // after the publish, off the step's dependent chain; non-temporal (read once, by the
        // backward)
        if (mine) {
          float* o = p.gh_save + ((int64_t)t * p.B + row) * 3 * p.H + unit;
#pragma unroll
          for (int g = 0; g < 3; ++g) __builtin_nontemporal_store(gh[g], o + g * p.H);
        }
      }
      if (REMOTE && PACK && lane == 0) __hip_atomic_fetch_add(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      lds_barrier();
    }
  } else if (REMOTE) {
    // NPR poller waves per batch row stage row pr of iteration it + 1's inputs
    // while the compute waves run iteration it, each polling its share of the
    // row's words. The gate-input loads (by part 0) are issued first so that
    // their latency overlaps the polls, which start once this workgroup's
    // compute waves have published iteration it: the other workgroups publish
    // at about the same time, and polling earlier only loads the memory system
    // that carries their stores.
    constexpr int NPR = pollers_per_row(KC);
    static_assert(!REMOTE || NT / 64 >= 4 * NPR + 1, "launch bounds hold the poller waves");
    const int pq = wave - nwc;
    const int pr = pq / NPR, part = pq - pr * NPR;
    constexpr int NGI = NT / 64 > 4 * NPR ? (3 * 4 * (NT / 64 - 4 * NPR) + 63) / 64 : 1;  // gi words per lane
    for (int it = 0; it < niter; ++it) {
      const int nx = it + 1;
      // every wait of the launch is behind the barrier that ended iteration
      // niter - 2: the last poller wave counts the workgroup out while the
      // compute waves run the final step
      if (it == niter - 1 && wave == (int)(blockDim.x >> 6) - 1 && lane == 0)
        leave_grid_lane(ctrl, (uint32_t)p.nwg, base, (uint32_t)p.T, &flags[1], 2);
      if (nx < niter) {
        const int t2 = nx / nrbm;
        const int rb2 = rb_begin + (nx - t2 * nrbm);
        const int row = 4 * rb2 + pr;
        float gv[NGI];
#pragma unroll
        for (int i = 0; i < NGI; ++i) {
          const int w = lane + 64 * i;
          const int g = w / U, u = w - g * U;
          const bool ok = part == 0 && w < 3 * U && row < p.B && (ulo + u - klo) < p.bs;
          gv[i] = ok ? p.gi[(int64_t)t2 * p.sg_t + (int64_t)row * p.sg_b + g * p.H + ulo + u] : 0.0f;
        }
        float* hs = hst + (nx & 1) * p.hsz;
        if (t2 == 0) {
          for (int k = lane + 64 * part; k < p.bs; k += 64 * NPR) {
            if constexpr (I8) {
              const int lv = row < p.B ? (int)quant_level(p.h0[(int64_t)row * p.sh0_b + klo + k], p.qin) : 0;
              reinterpret_cast<int8_t*>(hs)[4 * i8_index(pr, k >> 2) + (k & 3)] = (int8_t)lv;
            } else {
              float v = 0.0f;
              if (row < p.B) {
                v = p.h0[(int64_t)row * p.sh0_b + klo + k];
                if (p.qin.on) v = fake_quant(v, p.qin);
              }
              hs[il_index(pr, k)] = v;
            }
          }
        } else {
          {
            if (pq == 0 && nx == nrbm &&  // first exchange of the launch
                p.P <= 64 && group_on_one_xcd(ctrl, p.xw + gid, p.ngroups, p.P, base + 1u, &flags[1]))
              __hip_atomic_fetch_or(&flags[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            wait_lds_count(ctrl, &flags[0], nwc * (it + 1), &flags[1]);
            // this wave's share of row pr's bs words: k in [part KW, part KW + KW)
            // (part KW is a multiple of 128, so the staged slots are those of il_index)
            constexpr int KW = 16 * KC / NPR;
            if constexpr (PACK) {
              // packed words w in [part KW / 4, part KW / 4 + KW / 4), PMW per lane
              constexpr int PMW = KW / 4 >= 64 ? KW / 4 / 64 : 1;
              const int nw = p.H / 4, w0 = part * (KW / 4);
              const uint64_t* hb = p.xh + ((int64_t)((t2 - 1) & 1) * p.Bp + row) * nw + w0;
              uint64_t v[PMW];
              uint32_t valid = 0;
              if (w0 < nw) valid = poll_row_words<PMW>(ctrl, hb, min(KW / 4, nw - w0), base + (uint32_t)t2, v, &flags[1]);
#pragma unroll
              for (int m = 0; m < PMW; ++m) {
                if ((valid >> m) & 1u) {
                  const uint32_t x = (uint32_t)v[m];
                  if constexpr (I8) {
                    // levels + 128 -> two's-complement int8 levels
                    reinterpret_cast<int*>(hs)[i8_index(pr, w0 + lane + 64 * m)] = (int)(x ^ 0x80808080u);
                  } else {
                    f4 q;
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[e] = __builtin_fmaf((float)((x >> (8 * e)) & 0xffu), p.pscale, p.pbias);
                    *reinterpret_cast<f4*>(hs + il_index(pr, 4 * (w0 + lane + 64 * m))) = q;
                  }
                }
              }
            } else {
              const uint64_t* hb = p.xh + ((int64_t)((t2 - 1) & 1) * p.Bp + row) * p.H + klo;
              if (part * KW < p.bs)
                poll_row_il<KC / 4 / NPR>(ctrl, hb + part * KW, hs + 4 * part * KW, pr, min(KW, p.bs - part * KW),
                                          base + (uint32_t)t2, &flags[1]);
            }
          }
        }
        float* gs_ = gst + (nx & 1) * 4 * GR + pr * GR;
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
}

typedef void (*DFn)(DParams);

template <int KIND, bool REMOTE, bool PACK = false, bool SAVE = false, bool I8 = false>
DFn pick_kernel(int KC, int* nt) {
  // Remote instances add 4 pollers_per_row(KC) poller waves to 4 compute
  // waves (KC >= 16) or to up to 12 (KC <= 8); local instances hold up to 16
  // compute waves.
  switch (KC) {
    case 4: *nt = 1024; return scan_kernel<KIND, 4, 1024, REMOTE, PACK, SAVE, I8>;
    case 8: *nt = 1024; return scan_kernel<KIND, 8, 1024, REMOTE, PACK, SAVE, I8>;
    case 16: *nt = REMOTE ? 768 : 256; return scan_kernel<KIND, 16, REMOTE ? 768 : 256, REMOTE, PACK, SAVE, I8>;
    case 32: *nt = REMOTE ? 768 : 256; return scan_kernel<KIND, 32, REMOTE ? 768 : 256, REMOTE, PACK, SAVE, I8>;
    case 64: *nt = REMOTE ? 512 : 256; return scan_kernel<KIND, 64, REMOTE ? 512 : 256, REMOTE, PACK, SAVE, I8>;
    default: return nullptr;
  }
}

// save: the dense instances that also write gh_t (the training forward);
// i8: the int8-weight instances (dense, remote, packed, no save)
DFn pick(int kind, bool remote, int KC, int* nt, bool pack = false, bool save = false, bool i8 = false) {
  if (i8) return pick_kernel<kDense, true, true, false, true>(KC, nt);
  if (kind == kDense && save) {
    if (remote && pack) return pick_kernel<kDense, true, true, true>(KC, nt);
    return remote ? pick_kernel<kDense, true, false, true>(KC, nt) : pick_kernel<kDense, false, false, true>(KC, nt);
  }
  if (kind == kCirculant) {
    if (remote && pack) return pick_kernel<kCirculant, true, true>(KC, nt);
    return remote ? pick_kernel<kCirculant, true>(KC, nt) : pick_kernel<kCirculant, false>(KC, nt);
  }
  if (kind == kDense && remote && pack) return pick_kernel<kDense, true, true>(KC, nt);
  if (kind == kDense) return remote ? pick_kernel<kDense, true>(KC, nt) : pick_kernel<kDense, false>(KC, nt);
  return remote ? pick_kernel<kMonarch1, true>(KC, nt) : pick_kernel<kMonarch1, false>(KC, nt);
}

struct DPlan {
  int KC, nt, nwc, P, nrb, Bp, hsz, nb, bs, qpb, kr, gr;
  bool remote;
  bool pack;     // packed int8 exchange (dense remote mode)
  float pscale;  // its level scale
  int64_t xh_bytes, xw_bytes;
};

int plan_dense(int kind, const gs_args* a, DPlan* pl, const char* who) {
  if (kind == kDense || kind == kCirculant) {
    pl->nb = 1;
    pl->bs = (int)a->H;
  } else {
    if (a->nblocks < 1 || a->blksz < 1 || a->nblocks * a->blksz != a->H)
      return set_error(GS_ERR_INVALID, "%s: Wh_struct block dims must tile H: nblocks=%lld, blksz=%lld, H=%lld", who,
                       (long long)a->nblocks, (long long)a->blksz, (long long)a->H);
    pl->nb = (int)a->nblocks;
    pl->bs = (int)a->blksz;
  }
  pl->KC = choose_kc(pl->bs);
  if (pl->KC < 0)
    return set_error(GS_ERR_INVALID, "%s: reduction length %d exceeds the supported maximum of 1024", who, pl->bs);
  pl->qpb = (pl->bs + 3) / 4;
  pl->remote = pl->qpb > 16;
  if (!pl->remote) {
    pl->nwc = pl->qpb;
    pl->P = 1;
  } else {
    const int nwmax = dense_remote_units(pl->KC) / 4;
    int nwc = pl->qpb < nwmax ? pl->qpb : nwmax;
    if (kind == kMonarch1)
      while (pl->qpb % nwc != 0) --nwc;
    pl->nwc = nwc;
    pl->P = (pl->qpb + nwc - 1) / nwc;
  }
  // Packed exchange when the published value is a fake-quant level in
  // [-128, 127] (q_in after q_out, or q_out when q_in repeats it or is off).
  const gs_quant& qp = (a->q_in.enabled && !same_quant(a->q_in, a->q_out)) ? a->q_in : a->q_out;
  pl->pack = (kind == kDense || kind == kCirculant) && pl->remote && a->H % 4 == 0 && qp.enabled &&
             qp.qmin >= -128 && qp.qmax <= 127;
  pl->pscale = pl->pack ? qp.scale : 1.0f;
  pick(kind, pl->remote, pl->KC, &pl->nt, pl->pack);
  pl->nrb = (int)((a->B + 3) / 4);
  pl->Bp = 4 * pl->nrb;
  pl->hsz = 64 * pl->KC;
  const int U = 4 * pl->nwc;
  if ((kind == kDense || kind == kCirculant) && pl->remote && U != dense_remote_units(pl->KC))
    return set_error(GS_ERR_INVALID, "%s: dense remote plan has %d units per workgroup, kernel assumes %d", who, U,
                     dense_remote_units(pl->KC));
  pl->kr = row_stride_pad(U);
  pl->gr = row_stride_pad(3 * U);
  // The pollers load 16 KC words per row from the row's first unit; the pad
  // keeps the reads past the last row inside the workspace.
  pl->xh_bytes = pl->remote ? align256(2 * (int64_t)pl->Bp * a->H * 8 + 16 * pl->KC * 8) : 0;
  // one XCD-id word per workgroup of the largest grid the launch can use
  pl->xw_bytes = pl->remote ? align256((int64_t)pl->nrb * pl->nb * pl->P * 8) : 0;
  return GS_OK;
}

// codes / scales: int8 codes of Wh and their row scales (gs_dense_fwd_i8w), or
// NULL; used when the launch qualifies for the int8-weight instances.
int run(int kind, const gs_args* a, hipStream_t stream, const char* who, const int8_t* codes = nullptr,
        const float* scales = nullptr) {
  DPlan pl;
  int rc = plan_dense(kind, a, &pl, who);
  if (rc) return rc;
  rc = check_workspace(a, kCtrlBytes + pl.xh_bytes + pl.xw_bytes, who);
  if (rc) return rc;
  // every A operand must be a q_in level in the published levels' scale (with q_in on,
  // the packed exchange publishes q_in's levels)
  const bool i8 = codes != nullptr && kind == kDense && dense_i8_applies(a) && pl.pack && a->q_in.scale == pl.pscale;
  DFn fn = pick(kind, pl.remote, pl.KC, &pl.nt, pl.pack, a->gh_save != nullptr, i8);
  const int threads = 64 * (pl.nwc + (pl.remote ? 4 * pollers_per_row(pl.KC) : 0));
  const int per_set = pl.P * (kind == kMonarch1 ? pl.nb : 1);

  int G = pl.nrb, RB = 1;
  size_t lds = 0;
  // Local mode keeps RB = 1 (a workgroup's LDS staging holds one row-block);
  // remote mode shrinks the group count until the grid is resident at once.
  for (int pass = 0; pass < 2; ++pass) {
    RB = (pl.nrb + G - 1) / G;
    G = (pl.nrb + RB - 1) / RB;
    lds = sizeof(float) * (size_t)(2 * pl.hsz + RB * 4 * pl.kr + (pl.remote ? 8 * pl.gr + 4 : 0));
    if (lds > 65536)
      GS_CHECK_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    if (!pl.remote) break;
    int gfit = 0;
    rc = resident_groups((const void*)fn, threads, lds, per_set, pl.nrb, &gfit, who);
    if (rc) return rc;
    if (gfit >= G) break;
    G = gfit;
  }

  DParams p;
  p.gi = a->gi;
  p.h0 = a->h0;
  p.w = a->w;
  p.bh = a->bh;
  p.out = a->out;
  p.gh_save = a->gh_save;
  p.wq = i8 ? codes : nullptr;
  p.wsc = i8 ? scales : nullptr;
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
  p.nb = pl.nb;
  p.bs = pl.bs;
  p.qpb = pl.qpb;
  p.G = G;
  p.RB = RB;
  p.nrb = pl.nrb;
  p.Bp = pl.Bp;
  p.ngroups = G * (kind == kMonarch1 ? pl.nb : 1);
  p.nwg = p.ngroups * pl.P;
  p.P = pl.P;
  p.nwc = pl.nwc;
  p.hsz = pl.hsz;
  p.kr = pl.kr;
  p.gr = pl.gr;
  p.qin = to_quant(a->q_in);
  p.qout = to_quant(a->q_out);
  p.qin_after_first = a->q_in.enabled && !same_quant(a->q_in, a->q_out);
  p.pscale = pl.pscale;
  p.pbias = -128.0f * pl.pscale;
  hipLaunchKernelGGL(fn, dim3(p.nwg), dim3(threads), lds, stream, p);
  GS_CHECK_HIP(hipGetLastError());
  return GS_OK;
}

int64_t ws_bytes(int kind, const gs_args* a) {
  if (kind == kDense && dense_uses_tiled(a)) return 0;  // the batch-tiled kernel exchanges nothing
  DPlan pl;
  const int rc = plan_dense(kind, a, &pl, "gs_workspace_bytes");
  if (rc) return rc;
  return kCtrlBytes + pl.xh_bytes + pl.xw_bytes;
}

}  // namespace

int64_t dense_workspace_bytes(const gs_args* a) { return ws_bytes(kDense, a); }

int64_t circulant_workspace_bytes(const gs_args* a) { return ws_bytes(kCirculant, a); }

int64_t monarch_workspace_bytes(const gs_args* a) {
  if (a->w2) return monarch2_workspace_bytes(a);
  return monarch1_local_ok(a) ? kCtrlBytes : ws_bytes(kMonarch1, a);
}

}  // namespace gs

extern "C" int gs_dense_fwd(const gs_args* a, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_dense_fwd";
  int rc = gs::validate_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  if (gs::dense_uses_tiled(a)) return gs::run_tiled_fwd(a, stream, who);
  return gs::run(gs::kDense, a, stream, who);
}

extern "C" int gs_dense_fwd_i8w(const gs_args* a, const int8_t* w_codes, const float* w_scale, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_dense_fwd_i8w";
  int rc = gs::validate_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  rc = gs::check_codes(w_codes, w_scale, who);
  if (rc) return rc;
  if (gs::dense_uses_tiled(a)) return gs::run_tiled_fwd(a, stream, who, w_codes, w_scale);
  return gs::run(gs::kDense, a, stream, who, w_codes, w_scale);
}

extern "C" int gs_circulant_fwd(const gs_args* a, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_circulant_fwd";
  int rc = gs::validate_common(a, who);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the circulant kind", who);
  if (gs::dense_uses_tiled(a))
    return gs::set_error(GS_ERR_INVALID,
                         "%s: H=%lld exceeds 1024; run gs_dense_fwd on the map gs_hidden_map_dense writes", who,
                         (long long)a->H);
  return gs::run(gs::kCirculant, a, stream, who);
}

extern "C" int gs_monarch_fwd(const gs_args* a, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_monarch_fwd";
  // gh_save: the single-factor forward on its block-local path only
  int rc = gs::validate_common(a, who, a != nullptr && a->w2 == nullptr && gs::monarch1_local_ok(a));
  if (rc) return rc;
  if (a->w2) return gs::run_monarch2(a, stream, who);
  if (gs::monarch1_local_ok(a)) return gs::run_monarch1_local(a, stream);
  return gs::run(gs::kMonarch1, a, stream, who);
}

// ---- dense forward without a caller workspace ----------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc): the dense forward's
// exchange workspace comes from this file-scope device array instead of the
// caller. Each GPU the library runs on holds its own copy until the process
// ends. Host code never uses the array's name as an address: its device
// address is looked up once per device with hipGetSymbolAddress.
namespace gs {
namespace {
constexpr int64_t kStaticScratchBytes = int64_t(4) << 20;
}  // namespace
}  // namespace gs

static __device__ __align__(256) unsigned char scratch[gs::kStaticScratchBytes];

namespace gs {
namespace {

__global__ void zero_scratch(uint4* p, int64_t n16) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

struct StaticScratch {
  void* ptr = nullptr;  // device address of `scratch` on this device
  uint64_t steps = 0;   // scan steps issued since the array was last cleared
  bool cleared = false;
};

std::mutex g_static_mu;
StaticScratch g_static[64];

// The device address of the stream's device's array (looked up on its first
// use, with that device current: a stream of another device is refused),
// cleared on first use and before a launch of `steps` steps could take the
// 32-bit step tags past their limit; the clear is a fill kernel queued on
// `stream`. The caller counts the launch's steps with count_static_steps once
// it has been queued.
int static_scratch(hipStream_t stream, int64_t steps, void** out, int* dev_out, const char* who) {
  int dev = 0;
  GS_CHECK_HIP(hipGetDevice(&dev));
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    GS_CHECK_HIP(hipStreamGetDevice(stream, &sdev));
    if (sdev != dev)
      return set_error(GS_ERR_INVALID, "%s: the stream belongs to device %d but device %d is current", who, (int)sdev,
                       dev);
  }
  if (dev < 0 || dev >= 64) return set_error(GS_ERR_HIP, "%s: device ordinal %d out of range", who, dev);
  *dev_out = dev;
  std::lock_guard<std::mutex> lk(g_static_mu);
  StaticScratch& s = g_static[dev];
  if (s.ptr == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(GS_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", who, hipGetErrorString(e));
    s.ptr = p;
  }
  constexpr uint64_t kTagLimit = (uint64_t(1) << 32) - (uint64_t(1) << 24);
  if (!s.cleared || s.steps + (uint64_t)steps + 1 >= kTagLimit) {
    hipLaunchKernelGGL(zero_scratch, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(s.ptr),
                       kStaticScratchBytes / 16);
    GS_CHECK_HIP(hipGetLastError());
    s.cleared = true;
    s.steps = 0;
  }
  *out = s.ptr;
  return GS_OK;
}

void count_static_steps(int dev, int64_t steps) {
  std::lock_guard<std::mutex> lk(g_static_mu);
  g_static[dev].steps += (uint64_t)steps;
}

}  // namespace
}  // namespace gs

extern "C" int gs_dense_fwd_noalloc(const gs_args* a, hipStream_t stream) {
  gs::clear_error();
  const char* who = "gs_dense_fwd_noalloc";
  int rc = gs::validate_common(a, who, true);
  if (rc) return rc;
  if (a->w2 != nullptr) return gs::set_error(GS_ERR_INVALID, "%s: w2 must be NULL for the dense kind", who);
  // the batch-tiled kernel of H > 1024 uses no scratch at all
  if (gs::dense_uses_tiled(a)) return gs::run_tiled_fwd(a, stream, who);
  gs::DPlan pl;
  rc = gs::plan_dense(gs::kDense, a, &pl, who);
  if (rc) return rc;
  const int64_t need = gs::kCtrlBytes + pl.xh_bytes + pl.xw_bytes;
  if (need > gs::kStaticScratchBytes)
    return gs::set_error(GS_ERR_INVALID,
                         "%s: this shape needs %lld bytes of exchange scratch; the static scratch holds %lld "
                         "(use gs_dense_fwd with a caller workspace)",
                         who, (long long)need, (long long)gs::kStaticScratchBytes);
  gs_args b = *a;
  int dev = 0;
  rc = gs::static_scratch(stream, a->T, &b.workspace, &dev, who);
  if (rc) return rc;
  b.workspace_bytes = gs::kStaticScratchBytes;
  rc = gs::run(gs::kDense, &b, stream, who);
  if (rc == GS_OK) gs::count_static_steps(dev, a->T);
  return rc;
}
