// Device-side building blocks shared by the GRU scan kernels (gfx950 only).
//
// Numerics follow the reference PyTorch cell (LarocheC/gru-triton
// src/gru_qat/gru_cell.py:437-464): r = sigmoid(gi_r + gh_r),
// z = sigmoid(gi_z + gh_z), n = tanh(gi_n + r * gh_n), h' = (1 - z) * n + z * h.
// gru_update and gru_backward evaluate it in that order as separately rounded
// fp32 operations (FMA contraction off); the forward scans use gru_update_l2,
// the same math with the exp2 arguments fused into single fmas to shorten the
// step's dependent chain. sigmoid and tanh use the hardware
// base-2 exponential and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each);
// their deviation from torch's CPU functions is a few 1e-8 absolute, far inside
// the 1e-5 parity bar, and the fake-quant code is that of the IEEE quotient so
// integer codes depend only on the pre-quant value.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// Frozen per-tensor symmetric fake-quant (reference src/gru_qat/ste.py:65-95 with
// zero_point 0, and the in-kernel form at triton_kernels/scan.py:136-139):
// q = clamp(rint(x / s), qmin, qmax) * s, where x / s is the IEEE quotient and
// rint rounds half to even, so for a given fp32 x the integer code equals
// torch.round(x / s) exactly. `inv` is the fp32 rounding of 1 / s.
struct Quant {
  float scale;
  float qmin;
  float qmax;
  int on;
  float inv;
};

// rint(x / s) of the IEEE quotient, without the division sequence. With
// inv = fl(1 / s) (within half an ulp of 1 / s) and q0 = fl(x inv) (within one
// ulp of x / s), the residual r = x - q0 s is exact under an fma and
// fl(q0 + r inv) is the correctly rounded quotient (Markstein's final
// correction step, P. Markstein, IBM J. Res. Dev. 34(1), 1990). q0 is first
// clamped to [-2^24, 2^24], beyond which every code clamps to qmin or qmax
// anyway, so that infinite quotients leave no inf - inf. The host keeps s in
// [2^-126, 2^64] (inv stays normal and q0 s finite). The fake-quant result is
// then bit for bit that of clamp(rint(x / s)) s, NaN and infinities included;
// tests/test_quant_quotient.py checks the steps against the IEEE division on
// the CPU over sampled fp32 inputs, scales and code ranges.
__device__ __forceinline__ float quant_code(float x, const Quant& q) {
  float q0 = x * q.inv;
  q0 = __builtin_fminf(__builtin_fmaxf(q0, -0x1p24f), 0x1p24f);
  const float r = __builtin_fmaf(-q0, q.scale, x);
  return __builtin_rintf(__builtin_fmaf(r, q.inv, q0));
}

// The clamped integer level of fake_quant: fake_quant(x, q) == quant_level(x, q) * q.scale.
__device__ __forceinline__ float quant_level(float x, const Quant& q) {
  return __builtin_fminf(__builtin_fmaxf(quant_code(x, q), q.qmin), q.qmax);
}

__device__ __forceinline__ float fake_quant(float x, const Quant& q) { return quant_level(x, q) * q.scale; }

constexpr float kLog2e = 1.4426950408889634f;

// sigmoid(x) = 1 / (1 + e^-x) with e^y = 2^(y log2 e). Saturates correctly:
// x -> -inf gives rcp(inf) = 0, x -> +inf gives rcp(1) = 1.
__device__ __forceinline__ float sigmoid(float x) {
#pragma clang fp contract(off)
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -kLog2e));
}

// tanh(x) = 1 - 2 / (1 + e^2x). Absolute error stays at the fp32 rounding of
// values near 1 (a few 1e-8), including near 0 where the form cancels.
__device__ __forceinline__ float tanh_fast(float x) {
#pragma clang fp contract(off)
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * (2.0f * kLog2e)));
}

// One GRU gate epilogue. Inputs are the gate pre-activations' two halves; h is
// the raw (unquantized) previous state.
__device__ __forceinline__ float gru_update(float gir, float giz, float gin, float ghr, float ghz,
                                            float ghn, float h) {
#pragma clang fp contract(off)
  const float r = sigmoid(gir + ghr);
  const float z = sigmoid(giz + ghz);
  const float n = tanh_fast(gin + r * ghn);
  return (1.0f - z) * n + z * h;
}

// The same gate epilogue with every exp2 argument formed by one fma on the
// recurrence chain (11 dependent ops from h instead of 17). The caller passes
// the pre-activations already scaled by the base-2 exponent factors:
//   ar = -log2e (gi_r + gh_r),  az = -log2e (gi_z + gh_z),
//   gn2 = 2 log2e gh_n,  an2 = 2 log2e gi_n,
// and gets h' = n + z (h - n) with r = 1 / (1 + 2^ar), z = 1 / (1 + 2^az),
// n = 1 - 2 / (1 + 2^(r gn2 + an2)). The scalings and the fused products round
// differently from gru_update (a few 1e-8 absolute on r, z and n); both
// saturate the same way.
__device__ __forceinline__ float gru_update_l2(float ar, float az, float gn2, float an2, float h) {
  const float r = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(ar));
  const float z = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(az));
  const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(r, gn2, an2));
  const float n = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
  return __builtin_fmaf(z, h - n, n);
}

// Scale factors of gru_update_l2's arguments: -log2e for the r and z gates,
// 2 log2e for the n gate.
constexpr float kScaleRZ = -kLog2e;
constexpr float kScaleN = 2.0f * kLog2e;
__device__ __forceinline__ float gate_scale(int g) { return g == 2 ? kScaleN : kScaleRZ; }

// gru_update_l2 on the unscaled gate inputs gi*, hidden products gh* (bias not
// added) and the biases pre-scaled by gate_scale (bs*). The gi terms do not
// depend on the state, so only the three outer fmas sit on the step's chain.
__device__ __forceinline__ float gru_update_gb(float gir, float giz, float gin, float ghr, float ghz, float ghn,
                                               float bsr, float bsz, float bsn, float h) {
  return gru_update_l2(__builtin_fmaf(kScaleRZ, ghr, __builtin_fmaf(kScaleRZ, gir, bsr)),
                       __builtin_fmaf(kScaleRZ, ghz, __builtin_fmaf(kScaleRZ, giz, bsz)),
                       __builtin_fmaf(kScaleN, ghn, bsn), kScaleN * gin, h);
}

// Backward of one GRU step (reference src/gru_qat/triton_kernels/scan.py:1498-1540):
// recomputes r, z, n from the step's inputs with the forward's arithmetic,
// applies q_out's clipped-STE mask (round(h_raw / s) inside [qmin, qmax]) to
// the incoming gradient, and returns the gate-input gradients dg* (dgi), the
// n-gate hidden gradient dghn = dgn * r (dgh = (dgr, dgz, dghn)) and the
// direct carry dh * z.
struct GateGrad {
  float dgr, dgz, dgn, dghn, dh_direct;
};

__device__ __forceinline__ bool quant_keeps(float x, const Quant& q) {
  const float v = quant_code(x, q);
  return v >= q.qmin && v <= q.qmax;
}

__device__ __forceinline__ GateGrad gru_backward(float gir, float giz, float gin, float ghr, float ghz, float ghn,
                                                 float h_prev, float dh, const Quant& qout) {
#pragma clang fp contract(off)
  const float r = sigmoid(gir + ghr);
  const float z = sigmoid(giz + ghz);
  const float n = tanh_fast(gin + r * ghn);
  if (qout.on) {
    const float h_raw = (1.0f - z) * n + z * h_prev;
    if (!quant_keeps(h_raw, qout)) dh = 0.0f;
  }
  GateGrad gg;
  const float dn = dh * (1.0f - z);
  const float dz = dh * (h_prev - n);
  gg.dh_direct = dh * z;
  gg.dgn = dn * (1.0f - n * n);
  gg.dghn = gg.dgn * r;
  gg.dgz = dz * z * (1.0f - z);
  gg.dgr = gg.dgn * ghn * r * (1.0f - r);
  return gg;
}

// Diagonal hidden projection w * hq + b, rounded twice like torch's
// `w_hr * h + bh` (reference scan_diagonal.py:113-115).
__device__ __forceinline__ float mul_add_nofma(float w, float x, float b) {
#pragma clang fp contract(off)
  return w * x + b;
}

// ---- cross-lane helpers -----------------------------------------------------------
// DPP row rotation inside each 16-lane row: lane l reads lane ((l & ~15) | ((l + n) & 15)).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  static_assert(N >= 1 && N <= 15, "row_ror amount");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x120 + N, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_xor(float x, int m) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, __float_as_int(x)));
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// x[l ^ M] for M in {1, 2, 4, 8, 16, 32} with VALU lane moves instead of an
// LDS permute: quad permutes for 1 and 2; for 4, the half-row mirror
// (l -> l ^ 7 inside 8 lanes) followed by the quad reversal (l -> l ^ 3);
// for 8, a row rotation by 8 (either direction); for 16 and 32, the gfx950
// row swaps, whose two results hold the partner row in odd and even rows
// respectively (see sum_across_rows).
template <int M>
__device__ __forceinline__ float lane_xor_c(float x) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane_xor_c stride");
  if constexpr (M == 1) {
    return dpp_mov<0xB1>(x);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (M == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (M == 4) {
    return dpp_mov<0x1B>(dpp_mov<0x141>(x));  // row_half_mirror, then quad_perm [3, 2, 1, 0]
  } else if constexpr (M == 8) {
    return dpp_mov<0x128>(x);  // row_ror:8
  } else {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 a = (M == 16) ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((__lane_id() & M) ? a[0] : a[1]);
  }
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations, then s_barrier. Unlike __syncthreads it does not wait for the
// wave's global stores, whose acknowledgement (for coherent stores, a round
// trip to the device coherence point) would otherwise sit on the critical path.
// The asm memory clobber keeps the compiler from moving memory operations
// across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- raw buffer access --------------------------------------------------------------
// A buffer resource over the 4 GiB above `base`, addressed by a per-lane 32-bit
// byte offset (VGPR) plus a uniform 32-bit byte offset (SGPR). Against a
// global access this drops the per-access 64-bit address add from the VALU:
// the step loops of the latency-bound scans keep their per-lane offsets fixed
// and advance only the scalar offset (diagonal forward measured 133 -> 114 ns
// per step). Callers keep every offset sum below 2^32; the host checks the
// tensor extents and otherwise launches the global-address variant. dword3:
// DATA_FORMAT (bits 18:15) = 4, a 32-bit element; no other field set.
constexpr int kBufDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, kBufDword3);
}

// A buffer resource over `bytes` bytes at `base`: an access at a byte offset
// (per-lane offset; the uniform offset is kept 0) of `bytes` or more reads 0
// or is dropped by the hardware's range check, so a lane past the end of a
// row loads 0 and stores nothing without a branch around the access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bounded_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufDword3);
}
constexpr uint32_t kOffNone = 0x80000000u;  // a per-lane byte offset past every bounded_rsrc

__device__ __forceinline__ float buf_ld(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

__device__ __forceinline__ void buf_st(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, (int)soff, 0);
}

// x[l] + x[l ^ 16] + x[l ^ 32] + x[l ^ 48] in every lane, with gfx950's VALU
// row swaps: permlane16_swap(x, x) returns (x with odd rows replaced by the
// even rows below them, x with even rows replaced by the odd rows above
// them), so the sum of its two results is x[l] + x[l ^ 16] in every lane (the
// two operands are the same in both lanes of a pair, and fp32 addition
// commutes, so both lanes hold bitwise the same sum); permlane32_swap does
// the same for l ^ 32.
__device__ __forceinline__ float sum_across_rows(float x) {
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  const u2 a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const u2 b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ---- tagged exchange --------------------------------------------------------------
// Persistent kernels exchange hidden state between workgroups as 64-bit words
// {fp32 value (low half), 32-bit step tag (high half)}, written and read with
// relaxed agent-scope atomics. A consumer polls exactly the words it needs
// until each carries the tag of the step it wants; an aligned 8-byte atomic is
// single-copy atomic and coherent across the XCDs, so the value it returns is
// the one stored with that tag. No fence, counter or grid barrier is needed,
// and every wave proceeds as soon as its own inputs exist.
//
// Tags are tag_base + t + 1 for step t; tag_base lives in the workspace and
// advances by T at the end of every launch, so a word left over from an
// earlier launch (or a zeroed workspace, tag 0) never matches a tag the
// current launch waits for until the 32-bit tag space wraps, after 2^32
// steps on one workspace. Polls are bounded: after kSpinLimit polls the
// waiter raises the fault word and every waiter gives up, so a broken launch
// drains instead of hanging the device.
//
// The fault word is scoped to one launch: a waiter that gives up stores
// fval = tag_base + 1 of its launch, and waiters treat the word as raised only
// when it holds their own launch's fval. A fault left over from an earlier
// launch (a different tag_base) therefore never cuts a later launch's waits
// short. A workgroup whose wait gave up is dead for the rest of the launch:
// it stops publishing (so no other workgroup accepts words computed from
// stale inputs) and writes NaN into every output it would have written from
// then on. The last workgroup to leave copies a raised fault word into the
// optional host-visible `mirror` (hipHostMalloc memory), where the host can
// read it without synchronising.
constexpr uint32_t kSpinLimit = 1u << 22;

// One pointer addresses the workspace's control words (each on its own
// 64-byte line), so a kernel holds two scalar registers for them rather than
// eight: the persistent kernels run at the scalar-register limit, where every
// register held across the step loop can push a spill into it.
struct Ctrl {
  uint32_t* w;       // control words: ctrl_fault, ctrl_spin, ctrl_exit_count, ctrl_tag_base
  uint32_t* mirror;  // host-visible copy of a raised fault word, or NULL
  uint32_t fval;     // this launch's fault value, tag_base + 1 (set in the kernel)
  uint32_t limit;    // this launch's poll bound (set in the kernel)
};

// fval of the launch whose wait gave up (0: none yet)
__host__ __device__ __forceinline__ uint32_t* ctrl_fault(const Ctrl& c) { return c.w; }
// poll bound override: bits 0-23 the bound (0, as in a zeroed workspace: kSpinLimit),
// bits 24-31 a forced-late step (launch_ctrl)
__host__ __device__ __forceinline__ uint32_t* ctrl_spin(const Ctrl& c) { return c.w + 16; }
// workgroups that have finished this launch
__host__ __device__ __forceinline__ uint32_t* ctrl_exit_count(const Ctrl& c) { return c.w + 32; }
// tags of this launch are tag_base + t + 1
__host__ __device__ __forceinline__ uint32_t* ctrl_tag_base(const Ctrl& c) { return c.w + 48; }

// The poll-bound override word (ctrl_spin) holds the bound in bits 0-23 (0:
// kSpinLimit) and, in bits 24-31, a step F (0: none) whose exchange is forced
// late: the waits that check it (group_on_one_xcd, which every persistent
// kernel with XCD-local publishes runs on its first exchange, tag tag_base + 1,
// and the split two-factor kernel's waits, poll_to_lds) treat every word of
// tag tag_base + F as not yet arrived, so they run out at the bound and give
// up through the kernels' own fault path. Tests set it from the host to make a
// chosen exchange give up deterministically while every kernel still exits
// normally. The per-step word polls of the other kernels do not check it, so
// that their step loops carry nothing for it.
constexpr uint32_t kBoundMask = 0xffffffu;

// The kernel-side control block: the host's pointers plus this launch's fault
// value and poll bound (kSpinLimit unless the host wrote an override into the
// workspace).
__device__ __forceinline__ Ctrl launch_ctrl(const Ctrl& host, uint32_t base) {
  Ctrl c = host;
  c.fval = base + 1u;
  const uint32_t o = __hip_atomic_load(ctrl_spin(host), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kBoundMask;
  c.limit = o != 0u ? o : kSpinLimit;
  return c;
}

// The forced-late step F of this launch (0: none), read from the control word.
__device__ __forceinline__ uint32_t forced_step(const Ctrl& c) {
  return __hip_atomic_load(ctrl_spin(c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 24;
}

__device__ __forceinline__ void raise_fault(const Ctrl& c) {
  __hip_atomic_store(ctrl_fault(c), c.fval, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool fault_raised(const Ctrl& c) {
  return __hip_atomic_load(ctrl_fault(c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c.fval;
}

__device__ __forceinline__ uint64_t ld_tagged(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_tagged(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Non-temporal form of st_tagged: the word is written into the writer's XCD L2
// and not through to memory, which halves the time until an agent-scope load
// from the same XCD sees it. Only valid when every reader of the word runs
// on the writer's XCD (group_on_one_xcd); a reader elsewhere may not see the
// word until it is evicted.
__device__ __forceinline__ void st_tagged_xcd(uint64_t* p, float v, uint32_t tag) {
  __builtin_nontemporal_store(((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), p);
}

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return (uint32_t)(w >> 32); }
__device__ __forceinline__ float value_of(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Polls MW words base[src[i]] (those with bit i of `valid`) until each
// carries `tag`, then stores their values to dst_lds[dst[i]]. Offsets are
// precomputed by the caller, so the loop is loads, compares and a sleep.
// Returns false when the wait gave up (the staged values are then stale).
template <int MW>
__device__ __forceinline__ bool poll_to_lds(const Ctrl& c, const uint64_t* base, const int (&src)[MW],
                                            const int (&dst)[MW], uint32_t valid, uint32_t tag,
                                            float* dst_lds, bool forced = false) {
  uint64_t v[MW];
#pragma unroll
  for (int i = 0; i < MW; ++i) v[i] = ld_tagged(base + src[i]);
  uint32_t polls = 0;
  bool ok = true;
  while (true) {
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < MW; ++i) pending |= (tag_of(v[i]) != tag ? 1u : 0u) << i;
    pending &= valid;
    if (forced) pending = valid;  // forced late (launch_ctrl)
    if (pending == 0u) break;
    if (++polls > c.limit) {
      raise_fault(c);
      ok = false;
      break;
    }
    if ((polls & 255u) == 0u && fault_raised(c)) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < MW; ++i)
      if ((pending >> i) & 1u) v[i] = ld_tagged(base + src[i]);
  }
#pragma unroll
  for (int i = 0; i < MW; ++i)
    if ((valid >> i) & 1u) dst_lds[dst[i]] = value_of(v[i]);
  return ok;
}

// Calls f(integral_constant<int, I>) for I = 0 .. N-1 as straight-line code.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// A wait of this wave gave up: its workgroup is dead for the rest of the
// launch. `dead` is the workgroup's LDS flag word (bit 1), which the compute
// waves read every step and leave_grid reads at the end. Waits record this
// themselves rather than returning a status, so a poller loop carries no
// give-up state in registers: a loop-carried flag and the branches around
// each wait cost the dense forward 5.5 us and its backward 20 us per launch.
// A dead workgroup's later waits still run; with the fault word raised each
// ends within 256 polls.
__device__ __forceinline__ void mark_dead(int* dead) {
  __hip_atomic_fetch_or(dead, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits (bounded) until the LDS counter reaches target; marks the workgroup
// dead if it gave up.
__device__ __forceinline__ void wait_lds_count(const Ctrl& c, const int* cnt, int target, int* dead) {
  uint32_t polls = 0;
  while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    if (++polls > c.limit) {
      raise_fault(c);
      mark_dead(dead);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Whether the n workgroups whose XCD words sit at words[0], words[stride], ...
// all run on one XCD. Every workgroup stores its word (st_tagged of its
// xcc_id with `tag`) at launch; one wave of each workgroup calls this and all
// of them reach the same answer. n <= 64. A wait that gives up marks the
// workgroup dead (the answer is then false).
__device__ __forceinline__ bool group_on_one_xcd(const Ctrl& c, const uint64_t* words, int stride, int n,
                                                 uint32_t tag, int* dead) {
  const int lane = threadIdx.x & 63;
  const bool mine = lane < n;
  const uint64_t* src = words + (int64_t)(mine ? lane : 0) * stride;
  const uint32_t f = forced_step(c);
  const bool forced = f != 0u && tag == c.fval - 1u + f;  // forced late (launch_ctrl)
  uint64_t v = ld_tagged(src);
  uint32_t polls = 0;
  while (__ballot(mine && (forced || tag_of(v) != tag))) {
    if (++polls > c.limit) {
      raise_fault(c);
      mark_dead(dead);
      return false;
    }
    if ((polls & 255u) == 0u && fault_raised(c)) {
      mark_dead(dead);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
    if (mine && tag_of(v) != tag) v = ld_tagged(src);
  }
  const uint32_t x = (uint32_t)v;
  const uint32_t x0 = __builtin_amdgcn_readfirstlane(x);
  return __ballot(mine && x != x0) == 0;
}

// exit_count word: bits 0-15 count the workgroups that have left, bits 16-31
// those of them that were dead (a grid holds at most CUs x occupancy < 2^16
// workgroups, so neither field overflows).
constexpr uint32_t kExitDead = 1u << 16;

// Counts a workgroup out of the launch; called by one lane once every wait of
// the launch in this workgroup is over, so that its dead flag (the LDS word
// and bit mask that record whether a wait of this workgroup gave up) is
// final. A dead workgroup raises the fault word itself and adds 1 (plus
// kExitDead if dead) to exit_count. Every wait that raises the fault word, or
// gives up because it was raised, marks its workgroup dead, so the last
// workgroup to leave learns from the value its own increment returns whether
// this launch faulted: then it stores the fault value into the host mirror.
// It advances tag_base by the launch's step count (every workgroup read
// tag_base before it incremented exit_count) and rearms exit_count. All of
// this is one chain of read-modify-writes on one word, so relaxed atomics
// suffice; acquire / release ones would write back and invalidate the XCD's
// L2 once per workgroup (3.4 us per launch of the dense scan at 256
// workgroups). The next launch reads the words after the kernel boundary.
__device__ __forceinline__ void leave_grid_lane(const Ctrl& c, uint32_t nwg, uint32_t base, uint32_t steps,
                                                const int* dead_flag, int dead_mask) {
  const bool dead = (*dead_flag & dead_mask) != 0;
  if (dead) raise_fault(c);
  const uint32_t prev = __hip_atomic_fetch_add(ctrl_exit_count(c), dead ? 1u + kExitDead : 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
  if ((prev & (kExitDead - 1u)) == nwg - 1u) {
    if (c.mirror != nullptr && (dead || prev >= kExitDead))
      __hip_atomic_store(c.mirror, c.fval, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(ctrl_tag_base(c), base + steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctrl_exit_count(c), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// leave_grid_lane at the end of the kernel: called by every thread of every
// workgroup after its last exchange; the barrier makes the dead flag final.
__device__ __forceinline__ void leave_grid(const Ctrl& c, uint32_t nwg, uint32_t base, uint32_t steps,
                                           const int* dead_flag, int dead_mask) {
  __syncthreads();
  if (threadIdx.x == 0) leave_grid_lane(c, nwg, base, steps, dead_flag, dead_mask);
}

}  // namespace gs
