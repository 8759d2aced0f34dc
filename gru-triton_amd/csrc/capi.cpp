// C-ABI plumbing of libgruscan.so: error text, validation, workspace sizing and
// the workspace fault-word readback. The kernels and their launchers live in
// scan_*.hip.
#include <cstring>

#include "gs_host.h"

namespace gs {

static thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error.assign(buf);
  return code;
}

const char* last_error() { return g_error.c_str(); }
void clear_error() { g_error.clear(); }

int validate_quant(const gs_quant& q, const char* name, const char* who) {
  if (!q.enabled) return GS_OK;
  // [2^-126, 2^64]: the kernels' division-free quotient needs 1 / scale normal
  // and code * scale finite (gs_device.h quant_code)
  if (!(std::isfinite(q.scale) && q.scale >= 0x1p-126f && q.scale <= 0x1p64f))
    return set_error(GS_ERR_INVALID, "%s: %s scale must be in [2^-126, 2^64]; got %g", who, name,
                     (double)q.scale);
  if (q.qmin > q.qmax)
    return set_error(GS_ERR_INVALID, "%s: %s qmin (%d) must be <= qmax (%d)", who, name, q.qmin,
                     q.qmax);
  return GS_OK;
}

int validate_common(const gs_args* a, const char* who, bool gh_ok) {
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  if (a->gh_save != nullptr && !gh_ok)
    return set_error(GS_ERR_INVALID,
                     "%s: gh_save is only supported by the dense forward and the single-factor Monarch forward "
                     "with blksz 16, 32, 64 or 128; pass NULL",
                     who);
  if (a->T < 1) return set_error(GS_ERR_INVALID, "%s: seq length T must be > 0; got T=%lld", who, (long long)a->T);
  if (a->B < 1) return set_error(GS_ERR_INVALID, "%s: batch size B must be > 0; got B=%lld", who, (long long)a->B);
  if (a->H < 1) return set_error(GS_ERR_INVALID, "%s: hidden size H must be > 0; got H=%lld", who, (long long)a->H);
  if (a->T > (1ll << 30) || a->B > (1ll << 24) || a->H > (1ll << 20))
    return set_error(GS_ERR_INVALID, "%s: T/B/H out of supported range (T=%lld, B=%lld, H=%lld)", who,
                     (long long)a->T, (long long)a->B, (long long)a->H);
  if (!a->gi || !a->h0 || !a->w || !a->bh || !a->out)
    return set_error(GS_ERR_INVALID, "%s: gi, h0, w, bh and out must be non-NULL device pointers", who);
  // Rows of one step must not overlap, and steps must not overlap each other.
  if ((a->B > 1 && a->sg_b < 3 * a->H) || (a->T > 1 && a->sg_t < a->sg_b * (a->B - 1) + 3 * a->H))
    return set_error(GS_ERR_INVALID, "%s: gi strides (sg_t=%lld, sg_b=%lld) do not describe a [T, B, 3H] tensor", who,
                     (long long)a->sg_t, (long long)a->sg_b);
  if ((a->B > 1 && a->so_b < a->H) || (a->T > 1 && a->so_t < a->so_b * (a->B - 1) + a->H))
    return set_error(GS_ERR_INVALID, "%s: out strides (so_t=%lld, so_b=%lld) do not describe a [T, B, H] tensor", who,
                     (long long)a->so_t, (long long)a->so_b);
  if (a->sh0_b < a->H && a->B > 1)
    return set_error(GS_ERR_INVALID, "%s: h0 stride sh0_b=%lld < H=%lld", who, (long long)a->sh0_b, (long long)a->H);
  int rc = validate_quant(a->q_in, "h_in_quant", who);
  if (rc) return rc;
  return validate_quant(a->q_out, "h_out_quant", who);
}

gs_args fwd_view(const gs_bwd_args& a) {
  gs_args f;
  memset(&f, 0, sizeof f);
  f.gi = a.gi;
  f.h0 = a.h0;
  f.w = a.w;
  f.w2 = a.w2;
  f.bh = a.bh;
  f.out = const_cast<float*>(a.out);
  f.workspace = a.workspace;
  f.workspace_bytes = a.workspace_bytes;
  f.fault_mirror = a.fault_mirror;
  f.T = a.T;
  f.B = a.B;
  f.H = a.H;
  f.sg_t = a.sg_t;
  f.sg_b = a.sg_b;
  f.sh0_b = a.sh0_b;
  f.so_t = a.so_t;
  f.so_b = a.so_b;
  f.nblocks = a.nblocks;
  f.blksz = a.blksz;
  f.log_n = a.log_n;
  f.bfly_nblocks = a.bfly_nblocks;
  f.q_in = a.q_in;
  f.q_out = a.q_out;
  return f;
}

int validate_bwd_common(const gs_bwd_args* a, const char* who, bool gh_saved_ok) {
  if (a == nullptr) return set_error(GS_ERR_INVALID, "%s: args is NULL", who);
  if (a->gh_saved != nullptr && !gh_saved_ok)
    return set_error(GS_ERR_INVALID,
                     "%s: gh_saved is only supported by the dense backward and the single-factor Monarch backward "
                     "with blksz 16, 32, 64 or 128; pass NULL",
                     who);
  const gs_args f = fwd_view(*a);
  const int rc = validate_common(&f, who);
  if (rc) return rc;
  if (!a->dout || !a->dgi || !a->dh0 || !a->dbh_part)
    return set_error(GS_ERR_INVALID, "%s: dout, dgi, dh0 and dbh_part must be non-NULL device pointers", who);
  return GS_OK;
}

int check_workspace(const gs_args* a, int64_t need, const char* who) {
  if (need <= 0) return GS_OK;
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return set_error(GS_ERR_INVALID, "%s: workspace of %lld bytes required; got %lld at %p", who,
                     (long long)need, (long long)a->workspace_bytes, a->workspace);
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
    return set_error(GS_ERR_INVALID, "%s: workspace must be 256-byte aligned", who);
  return GS_OK;
}

int check_scratch(const gs_bwd_args* a, int64_t need, const char* who) {
  if (need <= 0) return GS_OK;
  if (a->scratch == nullptr || a->scratch_bytes < need)
    return set_error(GS_ERR_INVALID, "%s: scratch of %lld bytes required; got %lld at %p", who, (long long)need,
                     (long long)a->scratch_bytes, a->scratch);
  if ((reinterpret_cast<uintptr_t>(a->scratch) & 255u) != 0)
    return set_error(GS_ERR_INVALID, "%s: scratch must be 256-byte aligned", who);
  return GS_OK;
}

}  // namespace gs

// Defined in the kernel translation units.
namespace gs {
int64_t dense_workspace_bytes(const gs_args* a);
int64_t circulant_workspace_bytes(const gs_args* a);
int64_t monarch_workspace_bytes(const gs_args* a);
int64_t dense_bwd_workspace_bytes(const gs_bwd_args* a, bool tiled);
int64_t dense_bwd_scratch_bytes(const gs_bwd_args* a, bool tiled);
int64_t struct_bwd_workspace_bytes(int kind, const gs_bwd_args* a);
int64_t struct_bwd_scratch_bytes(int kind, const gs_bwd_args* a);
int64_t butterfly_bwd_workspace_bytes(const gs_bwd_args* a);
int64_t monarch_bwd_workspace_bytes(const gs_bwd_args* a);
int64_t monarch_bwd_scratch_bytes(const gs_bwd_args* a);
int64_t butterfly_bwd_scratch_bytes(const gs_bwd_args* a);
}  // namespace gs

extern "C" {

int64_t gs_workspace_bytes(int kind, const gs_args* a) {
  if (a == nullptr) return gs::set_error(GS_ERR_INVALID, "gs_workspace_bytes: args is NULL");
  switch (kind) {
    case GS_KIND_DENSE:
      return gs::dense_workspace_bytes(a);
    case GS_KIND_DENSE_TILED:
      return 0;
    case GS_KIND_MONARCH:
      return gs::monarch_workspace_bytes(a);
    case GS_KIND_CIRCULANT:
      return gs::circulant_workspace_bytes(a);
    case GS_KIND_DIAGONAL:
    case GS_KIND_BUTTERFLY:
      return gs::kCtrlBytes;
    default:
      return gs::set_error(GS_ERR_INVALID, "gs_workspace_bytes: unknown kind %d", kind);
  }
}

int64_t gs_bwd_workspace_bytes(int kind, const gs_bwd_args* a) {
  if (a == nullptr) return gs::set_error(GS_ERR_INVALID, "gs_bwd_workspace_bytes: args is NULL");
  switch (kind) {
    case GS_KIND_DENSE:
      return gs::dense_bwd_workspace_bytes(a, false);
    case GS_KIND_DENSE_TILED:
      return gs::dense_bwd_workspace_bytes(a, true);
    case GS_KIND_DIAGONAL:
      return 0;
    case GS_KIND_MONARCH:
      return gs::monarch_bwd_workspace_bytes(a);
    case GS_KIND_BUTTERFLY:
      return gs::butterfly_bwd_workspace_bytes(a);
    default:
      return gs::set_error(GS_ERR_INVALID, "gs_bwd_workspace_bytes: unknown kind %d", kind);
  }
}

int64_t gs_bwd_scratch_bytes(int kind, const gs_bwd_args* a) {
  if (a == nullptr) return gs::set_error(GS_ERR_INVALID, "gs_bwd_scratch_bytes: args is NULL");
  switch (kind) {
    case GS_KIND_DENSE:
      return gs::dense_bwd_scratch_bytes(a, false);
    case GS_KIND_DENSE_TILED:
      return gs::dense_bwd_scratch_bytes(a, true);
    case GS_KIND_DIAGONAL:
      return 0;
    case GS_KIND_MONARCH:
      return gs::monarch_bwd_scratch_bytes(a);
    case GS_KIND_BUTTERFLY:
      return gs::butterfly_bwd_scratch_bytes(a);
    default:
      return gs::set_error(GS_ERR_INVALID, "gs_bwd_scratch_bytes: unknown kind %d", kind);
  }
}

int gs_workspace_status(void* ws, int64_t bytes, hipStream_t stream) {
  if (ws == nullptr || bytes < gs::kCtrlBytes)
    return gs::set_error(GS_ERR_INVALID, "gs_workspace_status: workspace too small or NULL");
  GS_CHECK_HIP(hipStreamSynchronize(stream));
  uint32_t word = 0;
  GS_CHECK_HIP(hipMemcpy(&word, ws, sizeof(word), hipMemcpyDeviceToHost));
  if (word != 0) {
    const uint32_t zero = 0;
    GS_CHECK_HIP(hipMemcpy(ws, &zero, sizeof(zero), hipMemcpyHostToDevice));
  }
  return word != 0 ? 1 : 0;
}

const char* gs_last_error(void) { return gs::last_error(); }

int gs_abi_version(void) { return GS_ABI_VERSION; }

}  // extern "C"
