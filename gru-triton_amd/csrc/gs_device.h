// Device-side building blocks shared by the GRU scan kernels (gfx950 only).
//
// Numerics follow the reference PyTorch cell (LarocheC/gru-triton
// src/gru_qat/gru_cell.py:437-464): r = sigmoid(gi_r + gh_r),
// z = sigmoid(gi_z + gh_z), n = tanh(gi_n + r * gh_n), h' = (1 - z) * n + z * h,
// evaluated as separately rounded fp32 operations in that order (FMA
// contraction is switched off in the gate epilogue so each product rounds the
// way torch's elementwise kernels round it).
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// Frozen per-tensor symmetric fake-quant (reference src/gru_qat/ste.py:65-95 with
// zero_point 0, and the in-kernel form at triton_kernels/scan.py:136-139):
// q = clamp(rint(x / s), qmin, qmax) * s. The division is IEEE (HIP's default
// fp32 '/' is correctly rounded) and rint rounds half to even, so for a given
// fp32 x the integer code equals torch.round(x / s) exactly.
struct Quant {
  float scale;
  float qmin;
  float qmax;
  int on;
};

__device__ __forceinline__ float fake_quant(float x, const Quant& q) {
  float v = __builtin_rintf(x / q.scale);
  v = __builtin_fminf(__builtin_fmaxf(v, q.qmin), q.qmax);
  return v * q.scale;
}

// torch's CPU sigmoid is 1 / (1 + exp(-x)) with a 1-ulp exp and an exact
// division; this is the same expression on the ROCm device library's expf.
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// One GRU gate epilogue. Inputs are the gate pre-activations' two halves; h is
// the raw (unquantized) previous state.
__device__ __forceinline__ float gru_update(float gir, float giz, float gin, float ghr, float ghz,
                                            float ghn, float h) {
#pragma clang fp contract(off)
  const float r = sigmoid(gir + ghr);
  const float z = sigmoid(giz + ghz);
  const float n = tanhf(gin + r * ghn);
  return (1.0f - z) * n + z * h;
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
constexpr uint32_t kSpinLimit = 1u << 22;

struct Ctrl {
  uint32_t* fault;       // nonzero after a poll time-out
  uint32_t* exit_count;  // workgroups that have finished this launch
  uint32_t* tag_base;    // tags of this launch are tag_base + t + 1
};

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

// Polls N words until every valid one carries `tag`. addr(i) returns the
// word's address or nullptr for "no word" (value 0). Returns the values.
template <int N, typename Addr>
__device__ __forceinline__ void poll_tagged(const Ctrl& c, uint32_t tag, Addr addr, float (&out)[N]) {
  uint64_t v[N];
  const uint64_t ready_zero = (uint64_t)tag << 32;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint64_t* q = addr(i);
    v[i] = q ? ld_tagged(q) : ready_zero;
  }
  uint32_t polls = 0;
  while (true) {
    bool ready = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ready = ready && tag_of(v[i]) == tag;
    if (ready) break;
    if (++polls > kSpinLimit) {
      __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    if ((polls & 255u) == 0u && __hip_atomic_load(c.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (tag_of(v[i]) != tag) v[i] = ld_tagged(addr(i));
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = value_of(v[i]);
}

// Polls MW words base[src[i]] (those with bit i of `valid`) until each
// carries `tag`, then stores their values to dst_lds[dst[i]]. Offsets are
// precomputed by the caller, so the loop is loads, compares and a sleep.
template <int MW>
__device__ __forceinline__ void poll_to_lds(const Ctrl& c, const uint64_t* base, const int (&src)[MW],
                                            const int (&dst)[MW], uint32_t valid, uint32_t tag,
                                            float* dst_lds) {
  uint64_t v[MW];
#pragma unroll
  for (int i = 0; i < MW; ++i) v[i] = ld_tagged(base + src[i]);
  uint32_t polls = 0;
  while (true) {
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < MW; ++i) pending |= (tag_of(v[i]) != tag ? 1u : 0u) << i;
    pending &= valid;
    if (pending == 0u) break;
    if (++polls > kSpinLimit) {
      __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    if ((polls & 255u) == 0u && __hip_atomic_load(c.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < MW; ++i)
      if ((pending >> i) & 1u) v[i] = ld_tagged(base + src[i]);
  }
#pragma unroll
  for (int i = 0; i < MW; ++i)
    if ((valid >> i) & 1u) dst_lds[dst[i]] = value_of(v[i]);
}

// Calls f(integral_constant<int, I>) for I = 0 .. N-1 as straight-line code.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Polls R rows of tagged words into LDS: row r, word k = lane + 64 m
// (m < MPR) at src[r * src_stride + k], stored to dst[r * dst_stride + k] for
// k < klen. src and dst are wave-uniform; the loads address words up to
// k = 64 MPR - 1 of every row, so the buffer behind src must extend that far
// (words past klen are loaded but neither waited for nor stored). Only words
// whose tag is still stale are loaded again.
template <int R, int MPR>
__device__ __forceinline__ void poll_rows(const Ctrl& c, const uint64_t* src, int src_stride, float* dst,
                                          int dst_stride, int klen, uint32_t tag) {
  constexpr int MW = R * MPR;
  static_assert(MW <= 32, "poll mask is 32 bits");
  const int lane = threadIdx.x & 63;
  uint32_t valid = 0;
#pragma unroll
  for (int m = 0; m < MPR; ++m) {
    const bool ok = lane + 64 * m < klen;
#pragma unroll
    for (int r = 0; r < R; ++r) valid |= (ok ? 1u : 0u) << (r * MPR + m);
  }
  uint64_t v[MW];
  static_for<0, MW>([&](auto I) {
    constexpr int r = I / MPR, m = I % MPR;
    v[I] = ld_tagged(src + r * src_stride + lane + 64 * m);
  });
  uint32_t polls = 0;
  while (true) {
    uint32_t pending = 0;
    static_for<0, MW>([&](auto I) { pending |= (tag_of(v[I]) != tag ? 1u : 0u) << I; });
    pending &= valid;
    if (pending == 0u) break;
    if (++polls > kSpinLimit) {
      __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    if ((polls & 255u) == 0u && __hip_atomic_load(c.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      break;
    __builtin_amdgcn_s_sleep(1);
    static_for<0, MW>([&](auto I) {
      constexpr int r = I / MPR, m = I % MPR;
      if ((pending >> I) & 1u) v[I] = ld_tagged(src + r * src_stride + lane + 64 * m);
    });
  }
  static_for<0, MW>([&](auto I) {
    constexpr int r = I / MPR, m = I % MPR;
    if ((valid >> I) & 1u) dst[r * dst_stride + lane + 64 * m] = value_of(v[I]);
  });
}

// Waits (bounded) until the LDS counter reaches target.
__device__ __forceinline__ void wait_lds_count(const Ctrl& c, const int* cnt, int target) {
  uint32_t polls = 0;
  while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    if (++polls > kSpinLimit) {
      __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Whether the n workgroups whose XCD words sit at words[0], words[stride], ...
// all run on one XCD. Every workgroup stores its word (st_tagged of its
// xcc_id with `tag`) at launch; one wave of each workgroup calls this and all
// of them reach the same answer. n <= 64.
__device__ __forceinline__ bool group_on_one_xcd(const Ctrl& c, const uint64_t* words, int stride, int n,
                                                 uint32_t tag) {
  const int lane = threadIdx.x & 63;
  const bool mine = lane < n;
  const uint64_t* src = words + (int64_t)(mine ? lane : 0) * stride;
  uint64_t v = ld_tagged(src);
  uint32_t polls = 0;
  while (__ballot(mine && tag_of(v) != tag)) {
    if (++polls > kSpinLimit) {
      __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((polls & 255u) == 0u && __hip_atomic_load(c.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      return false;
    __builtin_amdgcn_s_sleep(1);
    if (mine && tag_of(v) != tag) v = ld_tagged(src);
  }
  const uint32_t x = (uint32_t)v;
  const uint32_t x0 = __builtin_amdgcn_readfirstlane(x);
  return __ballot(mine && x != x0) == 0;
}

// Called once by every workgroup after its last exchange. The last one to
// leave advances tag_base by the launch's step count (every workgroup read
// tag_base before it incremented exit_count) and rearms exit_count.
__device__ __forceinline__ void leave_grid(const Ctrl& c, uint32_t nwg, uint32_t base, uint32_t steps) {
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(c.exit_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == nwg - 1u) {
      __hip_atomic_store(c.tag_base, base + steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(c.exit_count, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace gs
