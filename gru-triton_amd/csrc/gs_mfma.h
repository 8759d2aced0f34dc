// Building blocks shared by the MFMA scan kernels (dense, single- and
// two-factor Monarch): the 4x4x1 MFMA chains over a wave's quad of hidden
// units (fp32, and int8 over int8 weight codes), the 16-way K-slice
// reduction, weight-slice loads and LDS operand reads, the workgroup barrier
// used between exchange stages, and host-side device queries.
//
// MFMA layout (v_mfma_f32_4x4x1_16b_f32, checked on the device): lane l
// supplies A[block l/4][row l%4] and B[block l/4][col l%4]; D block b, row v,
// col j is VGPR v of lane 4b + j. The kernels use the 16 blocks as 16 slices
// of K: instruction m of a chain covers k = kmap(m, b) for block b.
#pragma once

#include <mutex>

#include "gs_host.h"

namespace gs {

typedef float f4 __attribute__((ext_vector_type(4)));

// k index of MFMA instruction m in k-slice b: float4-contiguous per lane, so a
// lane reads its A operand from an LDS row with KC/4 ds_read_b128.
__device__ __forceinline__ int kmap(int m, int b) { return 64 * (m >> 2) + 4 * b + (m & 3); }

// Sums the 16 K-slice partials of one gate. Input: the chain's D (lane 4b+j,
// VGPR v = slice b's partial for row v, unit j). Output in lane l: the full
// sum for row s = (l >> 2) & 3, unit l & 3.
__device__ __forceinline__ float reduce16(f4 acc, int s) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += row_ror<8>(acc[c]);
    acc[c] += row_ror<4>(acc[c]);
  }
  // branch-free pick of acc[s] (lane-varying s)
  const float lo = (s & 1) ? acc[1] : acc[0];
  const float hi = (s & 1) ? acc[3] : acc[2];
  return sum_across_rows((s & 2) ? hi : lo);
}

// Wh slice of a quad: w[((gate*nb + blk)*bs + o)*bs + k] for o = o0 + j,
// k = kmap(m, kb4); zero where o >= bs or k >= bs.
template <int KC>
__device__ __forceinline__ void load_w(const float* w, int nb, int bs, int blk, int o0, int j, int kb4, bool ok_blk,
                                       float (&wr)[3][KC]) {
  const int o = o0 + j;
  const bool ok = ok_blk && o < bs;
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

// Interleaved staging layout of a 4-row operand block. K is cut into chunks
// of 4 (c = k / 4); chunk c holds the four rows' 4-float slices back to back,
// 16 floats, with row r in slot il_slot(r, c). The A operand of lane l for
// K-chunk q (k = 64 q + 4 (l / 4) + e, row l % 4) is then one float4 of chunk
// 16 q + l / 4, and a wave's 64 operand reads cover 1 KiB of contiguous LDS
// (each chunk's four slots read by its four lanes in some order), free of
// bank conflicts. The slot rotation makes the pollers' stores conflict-free
// too: a poller stores one row, lane l word k = l + 64 i at il_index(r, k);
// without rotation (slot = r) the 64 lanes would land on 16 banks, with
// slot = (r + c / 2 + c / 8) mod 4 they land on 64 distinct banks (and each
// half-wave on 32, so the layout is conflict-free with 32 or 64 banks). A
// block holding K values per row takes 4 K floats.
__device__ __forceinline__ int il_slot(int r, int c) { return (r + (c >> 1) + (c >> 3)) & 3; }
__device__ __forceinline__ int il_index(int r, int k) {
  const int c = k >> 2;
  return (c << 4) + (il_slot(r, c) << 2) + (k & 3);
}

// A operand of lane l from an interleaved block: a[m] = row (l % 4), k =
// kofs + kmap(m, l / 4). blk points at the block's chunk kofs / 4 (kofs a
// multiple of 4). Adding 16 to a chunk index adds 2 (mod 4) to its slot, so
// the reads alternate between two per-lane bases by the parity of q.
template <int KC>
__device__ __forceinline__ void lds_a_il(const float* blk, int lane, float (&a)[KC], int kofs = 0) {
  const int m = lane >> 2, x = (kofs >> 2) + m;
  const int s0 = ((lane & 3) + (x >> 1) + (x >> 3)) & 3;
  const float* p0 = blk + 16 * m + 4 * s0;
  const float* p1 = blk + 16 * m + 4 * (s0 ^ 2);
#pragma unroll
  for (int q = 0; q < KC / 4; ++q) {
    const f4 v = *reinterpret_cast<const f4*>(((q & 1) ? p1 : p0) + 256 * q);
    a[4 * q + 0] = v[0];
    a[4 * q + 1] = v[1];
    a[4 * q + 2] = v[2];
    a[4 * q + 3] = v[3];
  }
}

// Polls one row of tagged words: lane l waits for src[64 m + l] (m < MPR,
// 64 m + l < klen) to carry `tag` and returns the words in v[m]. Each load
// instruction reads 64 consecutive words (polling 4 rows x 16 words per
// instruction instead measured 25 % slower exchanges). Loads address up to
// src[64 MPR - 1], so the buffer must extend that far (words past klen are
// loaded but not waited for). Every round reloads all MPR words: a word that
// already carries the tag keeps it until this workgroup publishes its next
// step (the producer's next write to the same buffer half needs that step),
// and unconditional loads measured faster than reloading only the stale words
// under per-lane exec masks (one-way exchange latency of 512 words by one
// wave: 575 ns against 693 ns). Returns the mask of valid m; a wait that
// gives up marks the workgroup dead (mark_dead).
template <int MPR>
__device__ __forceinline__ uint32_t poll_row_words(const Ctrl& c, const uint64_t* src, int klen, uint32_t tag,
                                                   uint64_t (&v)[MPR], int* dead) {
  static_assert(MPR <= 32, "poll mask is 32 bits");
  const int lane = threadIdx.x & 63;
  const uint64_t* s0 = src + lane;
  uint32_t valid = 0;
#pragma unroll
  for (int m = 0; m < MPR; ++m) valid |= (lane + 64 * m < klen ? 1u : 0u) << m;
  static_for<0, MPR>([&](auto I) { v[I] = ld_tagged(s0 + 64 * I); });
  uint32_t polls = 0;
  while (true) {
    uint32_t pending = 0;
    static_for<0, MPR>([&](auto I) { pending |= (tag_of(v[I]) != tag ? 1u : 0u) << I; });
    pending &= valid;
    if (pending == 0u) break;
    if (++polls > c.limit) {
      raise_fault(c);
      mark_dead(dead);
      break;
    }
    if ((polls & 255u) == 0u && fault_raised(c)) {
      mark_dead(dead);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    static_for<0, MPR>([&](auto I) { v[I] = ld_tagged(s0 + 64 * I); });
  }
  return valid;
}

// Polls one row of tagged words into LDS: lane l takes k = 64 m + l (m < MPR)
// from src[k] and stores it for k < klen at dst[il_index(r, k)] (IL: the
// interleaved layout; a dst that starts k0 into a larger block keeps that
// block's slots when k0 is a multiple of 128) or at dst[k] (row-major), with
// the loads, waits and bounds of poll_row_words. (The wait loop is written out
// here rather than shared: the forward kernels' code around this inlined loop
// is tuned, and the shared form schedules differently.) A wait that gives up
// marks the workgroup dead (mark_dead).
template <int MPR, bool IL = true>
__device__ __forceinline__ void poll_row_il(const Ctrl& c, const uint64_t* src, float* dst, int r, int klen,
                                            uint32_t tag, int* dead) {
  static_assert(MPR <= 32, "poll mask is 32 bits");
  const int lane = threadIdx.x & 63;
  const uint64_t* s0 = src + lane;
  uint32_t valid = 0;
#pragma unroll
  for (int m = 0; m < MPR; ++m) valid |= (lane + 64 * m < klen ? 1u : 0u) << m;
  uint64_t v[MPR];
  static_for<0, MPR>([&](auto I) { v[I] = ld_tagged(s0 + 64 * I); });
  uint32_t polls = 0;
  while (true) {
    uint32_t pending = 0;
    static_for<0, MPR>([&](auto I) { pending |= (tag_of(v[I]) != tag ? 1u : 0u) << I; });
    pending &= valid;
    if (pending == 0u) break;
    if (++polls > c.limit) {
      raise_fault(c);
      mark_dead(dead);
      break;
    }
    if ((polls & 255u) == 0u && fault_raised(c)) {
      mark_dead(dead);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    static_for<0, MPR>([&](auto I) { v[I] = ld_tagged(s0 + 64 * I); });
  }
  static_for<0, MPR>([&](auto I) {
    if ((valid >> I) & 1u) dst[IL ? il_index(r, lane + 64 * I) : lane + 64 * I] = value_of(v[I]);
  });
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

// Three MFMA chains (one per gate), NA accumulators each for issue overlap
// (instruction m feeds accumulator m % NA; NA divides KC). SHARED_A: every
// gate multiplies a[0].
template <int KC, bool SHARED_A, int NA = 2>
__device__ __forceinline__ void mfma3(const float (&a)[3][KC], const float (&wr)[3][KC], f4 (&acc)[3]) {
  static_assert(NA == 2 || NA == 4, "accumulators per gate");
  static_assert(KC % NA == 0, "NA divides KC");
  f4 part[NA][3];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int g = 0; g < 3; ++g) part[i][g] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < KC; m += NA) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int g = 0; g < 3; ++g)
        part[i][g] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[SHARED_A ? 0 : g][m + i], wr[g][m + i], part[i][g], 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    acc[g] = part[0][g] + part[1][g];
    if constexpr (NA == 4) acc[g] += part[2][g] + part[3][g];
  }
}


// ---- int8 weight codes (v_mfma_i32_4x4x4_16b_i8) ------------------------------------
// Same lane layout as the fp32 chains, with 4 consecutive k per block packed
// as 4 bytes (byte e = k offset e): instruction q of a chain covers, in block
// b, k = 64 q + 4 b + e, which is what KC fp32 instructions m = 4 q + e cover
// (kmap), so the 16 block partials and reduce16 are those of the fp32 chains.

typedef int i4 __attribute__((ext_vector_type(4)));

// Int8 staging layout of a 4-row operand block: word c (k = 4 c .. 4 c + 3 of
// row r, one byte each) at 4 c + ((r + c / 16) mod 4). A lane's operand reads
// (row l % 4, word 16 q + l / 4) then cover 64 consecutive words per q, and a
// poller's stores of one row (lane l: word c = l + 64 i) 64 distinct banks.
__device__ __forceinline__ int i8_index(int r, int c) { return 4 * c + ((r + (c >> 4)) & 3); }

// A operand of lane l from an int8 staging block: a[q] = word 16 q + l / 4 of row l % 4.
template <int KC>
__device__ __forceinline__ void lds_a_i8(const int* blk, int lane, int (&a)[KC / 4]) {
  const int* b = blk + 4 * (lane >> 2);
#pragma unroll
  for (int q = 0; q < KC / 4; ++q) a[q] = b[64 * q + (((lane & 3) + q) & 3)];
}

// Int8 codes of a quad's 12 weight rows: wi[g][q] packs codes[(g H + o) H + k .. k + 3]
// for o = o0 + j, k = 64 q + 4 kb4; zero where o >= H or k >= H. H % 4 == 0 and
// codes 4-byte aligned, so each is one aligned 32-bit load.
template <int KC>
__device__ __forceinline__ void load_wi(const int8_t* codes, int H, int o0, int j, int kb4, bool ok_quad,
                                        int (&wi)[3][KC / 4]) {
  const int o = o0 + j;
  const bool ok = ok_quad && o < H;
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const int8_t* row = codes + ((int64_t)g * H + (ok ? o : 0)) * H;
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const int k = 64 * q + 4 * kb4;
      wi[g][q] = (ok && k < H) ? *reinterpret_cast<const int*>(row + k) : 0;
    }
  }
}

// Three int8 MFMA chains (one per gate) on a shared A operand, two accumulators
// each when the chain has two or more instructions. Sums are exact (|code| <= 128,
// K <= 1024: at most 2^24).
template <int KC>
__device__ __forceinline__ void mfma3_i8(const int (&a)[KC / 4], const int (&wi)[3][KC / 4], i4 (&acc)[3]) {
  constexpr int NQ = KC / 4;
  constexpr int NA = NQ >= 2 ? 2 : 1;
  i4 part[NA][3];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int g = 0; g < 3; ++g) part[i][g] = i4{0, 0, 0, 0};
#pragma unroll
  for (int q = 0; q < NQ; q += NA) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int g = 0; g < 3; ++g) part[i][g] = __builtin_amdgcn_mfma_i32_4x4x4i8(a[q + i], wi[g][q + i], part[i][g], 0, 0, 0);
  }
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    acc[g] = part[0][g];
    if constexpr (NA == 2) acc[g] += part[1][g];
  }
}

// The 16 block partials of an int8 chain as floats: exact, since every partial
// and every sum reduce16 forms is an integer of magnitude at most 2^24.
__device__ __forceinline__ f4 i4_to_f4(i4 v) { return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}; }

// reduce16 in integers, for chains whose sums may exceed 2^24 (K > 1024): the
// exact sum for row s = (l >> 2) & 3, unit l & 3, in lane l. Where every sum
// stays within 2^24 the float of it equals reduce16(i4_to_f4(acc), s).
__device__ __forceinline__ int reduce16_i(i4 acc, int s) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += __builtin_amdgcn_mov_dpp(acc[c], 0x128, 0xF, 0xF, true);  // row_ror:8
    acc[c] += __builtin_amdgcn_mov_dpp(acc[c], 0x124, 0xF, 0xF, true);  // row_ror:4
  }
  const int lo = (s & 1) ? acc[1] : acc[0];
  const int hi = (s & 1) ? acc[3] : acc[2];
  const int x = (s & 2) ? hi : lo;
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  const u2 a = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  const int y = (int)(a[0] + a[1]);
  const u2 b = __builtin_amdgcn_permlane32_swap((unsigned)y, (unsigned)y, false, false);
  return (int)(b[0] + b[1]);
}

// ---- host side --------------------------------------------------------------------

struct DevInfo {
  int cus = 0;
};

inline int device_info(DevInfo* out) {
  static std::mutex mu;
  static DevInfo cache[64];
  static bool have[64] = {};
  int dev = 0;
  GS_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return set_error(GS_ERR_HIP, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(mu);
  if (!have[dev]) {
    GS_CHECK_HIP(hipDeviceGetAttribute(&cache[dev].cus, hipDeviceAttributeMultiprocessorCount, dev));
    have[dev] = true;
  }
  *out = cache[dev];
  return GS_OK;
}

inline int choose_kc(int klen) {
  const int need = (klen + 15) / 16;
  for (int kc : {4, 8, 16, 32, 64})
    if (kc >= need) return kc;
  return -1;
}

// Persistent grids. Workgroups of one group wait for each other's exchange
// words, so a group's workgroups must run at the same time. The grid is sized
// to what the device holds at once (occupancy x CUs) and launched as an
// ordinary kernel: on an otherwise idle device every workgroup of such a grid
// is resident from the start. A kernel on another stream that holds CUs delays
// the rest of the grid until it ends; every wait in these kernels is bounded,
// so a delay beyond the poll bound ends the launch with the workspace fault
// word set instead of hanging. (hipLaunchCooperativeKernel would add about
// 16 us of dispatch overhead per call on this stack.)
//
// Largest number of groups the device holds at once: workgroups of
// `threads` threads and `lds` bytes, `per_group` workgroups per group.
inline int resident_groups(const void* fn, int threads, size_t lds, int per_group, int want, int* out,
                           const char* who) {
  DevInfo di;
  int rc = device_info(&di);
  if (rc) return rc;
  int occ = 0;
  GS_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, lds));
  const int64_t resident = (int64_t)occ * di.cus;
  if (resident < per_group)
    return set_error(GS_ERR_CAPACITY,
                     "%s: persistent grid needs %d co-resident workgroups of %d threads per batch group; "
                     "the device holds %lld",
                     who, per_group, threads, (long long)resident);
  const int64_t gmax = resident / per_group;
  *out = (int)(gmax < want ? gmax : want);
  return GS_OK;
}

// Dense hidden sizes above the persistent kernels' largest reduction (KC 64,
// 1024 units) run on the batch-tiled kernels of scan_tiled.hip.
constexpr int64_t kPersistentMaxH = 1024;
inline bool dense_uses_tiled(const gs_args* a) { return a->H > kPersistentMaxH; }
int64_t tiled_max_h();
int run_tiled_fwd(const gs_args* a, hipStream_t stream, const char* who, const int8_t* codes = nullptr,
                  const float* scales = nullptr);

// The dense forwards run their int8-weight instances (v_mfma_i32_4x4x4_16b_i8
// over q_in levels and Wh's int8 codes) when every A operand is a q_in level
// that fits a byte, rows of codes load as 16-byte words, the persistent kernel
// is in remote mode (H > 64) and no gh is saved. The rule is the same for the
// persistent and the batch-tiled kernel, so the two give the same outputs.
inline bool dense_i8_applies(const gs_args* a) {
  return a->q_in.enabled && a->q_in.qmin >= -128 && a->q_in.qmax <= 127 && a->H > 64 && a->H % 16 == 0 &&
         a->gh_save == nullptr;
}

// Arguments of the int8-weight entry points: both arrays given, the codes
// 16-byte aligned (the batch-tiled kernel loads 16 codes per lane).
inline int check_codes(const int8_t* codes, const float* scales, const char* who) {
  if (codes == nullptr || scales == nullptr)
    return set_error(GS_ERR_INVALID, "%s: w_codes and w_scale are required", who);
  if ((reinterpret_cast<uintptr_t>(codes) & 15u) != 0)
    return set_error(GS_ERR_INVALID, "%s: w_codes must be 16-byte aligned", who);
  return GS_OK;
}
int64_t tiled_bwd_wt_bytes(int64_t H);
int run_tiled_bwd_recurrence(const float* w, float* wt, const float* dout, const float* cg, const float* zm,
                             const float* mi, float* dsum, float* dh0, int64_t T, int64_t B, int64_t H,
                             hipStream_t stream, const char* who);

int64_t monarch2_workspace_bytes(const gs_args* a);
int run_monarch2(const gs_args* a, hipStream_t stream, const char* who);
// Single-factor Monarch forward with one workgroup per block and batch rows
// (scan_monarch1.hip): the shapes it takes, and its launch.
bool monarch1_local_ok(const gs_args* a);
int run_monarch1_local(const gs_args* a, hipStream_t stream);

}  // namespace gs
