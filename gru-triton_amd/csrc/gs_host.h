// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// argument validation and the workspace layout.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/gruscan.h"
#include "gs_device.h"

namespace gs {

int set_error(int code, const char* fmt, ...);
const char* last_error();
void clear_error();

#define GS_CHECK_HIP(expr)                                                                  \
  do {                                                                                      \
    hipError_t _e = (expr);                                                                 \
    if (_e != hipSuccess)                                                                   \
      return ::gs::set_error(GS_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));   \
  } while (0)

// Workspace layout (bytes from the start):
//   [0, 256)        control words: fault word (word 0; the fault value
//                   tag_base + 1 of the last launch whose wait gave up),
//                   poll bound override (word 16; bits 0-23 the bound, 0 = the
//                   default; bits 24-31 a forced-late step, gs_device.h),
//                   exit count (word 32), tag base (word 48); zero on first use
//   [256, ...)      tagged exchange words (uint64), 256-byte aligned regions
// Every launch leaves the exit count at zero and the tag base advanced, and
// only ever compares exchange words against tags newer than any word an
// earlier launch wrote, so regions of differently shaped launches may overlap.
constexpr int64_t kCtrlBytes = 256;

inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Host half of the control block; the kernel adds its launch's fault value.
inline Ctrl ctrl_of(void* ws, uint32_t* mirror) {
  return Ctrl{static_cast<uint32_t*>(ws), mirror, 0u, 0u};
}

inline Quant to_quant(const gs_quant& q) {
  return Quant{q.scale, (float)q.qmin, (float)q.qmax, q.enabled != 0, 1.0f / q.scale};
}

// The two quantizers are the same map when both are on with equal parameters.
// Then q_in(q_out(x)) == q_out(x) bit for bit: for |code| <= 2^22 the product
// code*s divided by s rounds back to the code, so the carried h can be read as
// the matmul-side h without applying q_in again.
inline bool same_quant(const gs_quant& a, const gs_quant& b) {
  return a.enabled && b.enabled && a.scale == b.scale && a.qmin == b.qmin && a.qmax == b.qmax &&
         std::fabs((double)a.qmin) <= 4194304.0 && std::fabs((double)a.qmax) <= 4194304.0;
}

// True when every byte offset of a [n2, n1, n0] view with element strides
// (s2, s1, 1) fits the 32-bit offsets of raw buffer access (gs_device.h).
inline bool fits_buf32(int64_t n2, int64_t s2, int64_t n1, int64_t s1, int64_t n0) {
  const int64_t last = (n2 - 1) * s2 + (n1 - 1) * s1 + n0;
  return n2 >= 1 && n1 >= 1 && s2 >= 0 && s1 >= 0 && last * 4 < (int64_t(1) << 32);
}

// gh_ok / gh_saved_ok: the entry point takes gs_args.gh_save / gs_bwd_args.gh_saved
// (dense only); elsewhere a non-NULL one is rejected.
int validate_common(const gs_args* a, const char* who, bool gh_ok = false);
// gs_args view of the forward fields of a backward call.
gs_args fwd_view(const gs_bwd_args& a);
// validate_common on the forward fields plus the gradient pointers.
int validate_bwd_common(const gs_bwd_args* a, const char* who, bool gh_saved_ok = false);
int validate_quant(const gs_quant& q, const char* name, const char* who);
int check_workspace(const gs_args* a, int64_t need, const char* who);
// The backward's plain scratch: non-NULL, large enough, 256-byte aligned.
int check_scratch(const gs_bwd_args* a, int64_t need, const char* who);

}  // namespace gs
