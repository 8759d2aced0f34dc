// Device-side building blocks shared by the GRU scan kernels (gfx950 only).
//
// Numerics follow the reference PyTorch cell (LarocheC/gru-triton
// src/gru_qat/gru_cell.py:437-464): r = sigmoid(gi_r + gh_r),
// z = sigmoid(gi_z + gh_z), n = tanh(gi_n + r * gh_n), h' = (1 - z) * n + z * h,
// evaluated as separately rounded fp32 operations in that order (FMA
// contraction is switched off in the gate epilogue so each product rounds the
// way torch's elementwise kernels round it).
#pragma once

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

// ---- group barrier ----------------------------------------------------------------
// All workgroups of one group share a monotonically increasing arrival counter;
// the barrier of step t waits for count >= nwg_in_group * (t + 1). Agent-scope
// release/acquire makes every store issued before the barrier (by any wave of
// any arriving workgroup) visible to every load issued after it, whichever XCD
// each workgroup runs on. The spin is bounded: if the counter has not moved for
// kSpinLimit polls, the workgroup raises the fault word and every other
// spinning workgroup leaves too, so a broken launch always drains instead of
// hanging the device.
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr int kCounterStride = 64;  // uint32 words between group counters (256 B)

struct Ctrl {
  uint32_t* fault;  // nonzero after a barrier time-out
  uint32_t* exit_count;
  uint32_t* counters;
};

__device__ __forceinline__ void group_barrier(const Ctrl& c, int group, uint32_t target) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* cnt = c.counters + (size_t)group * kCounterStride;
    __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t polls = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (__hip_atomic_load(c.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
      if (++polls > kSpinLimit) {
        __hip_atomic_store(c.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Called once by every workgroup of a cooperative launch after its last
// barrier. The last workgroup to leave zeroes the group counters and the exit
// count, so the workspace is ready for the next launch on the stream. By then
// every other workgroup has finished polling, so the reset cannot be observed
// by a waiter.
__device__ __forceinline__ void leave_grid(const Ctrl& c, int ngroups, uint32_t nwg) {
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(c.exit_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == nwg - 1u) {
      for (int g = 0; g < ngroups; ++g)
        __hip_atomic_store(c.counters + (size_t)g * kCounterStride, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(c.exit_count, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace gs
