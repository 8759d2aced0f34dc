/*
 * gruscan.h -- C ABI of libgruscan.so, the MI355X (gfx950) persistent GRU scan.
 *
 * One entry point per hidden-weight kind. Each runs the whole T-step GRU
 * recurrence forward in one kernel launch on the given HIP stream:
 *
 *   hq_t   = q_in(h_{t-1})                     (optional frozen fake-quant)
 *   gh     = Wh(hq_t) + bh                     (dense / diagonal / Monarch / butterfly)
 *   r      = sigmoid(gi_r[t] + gh_r)
 *   z      = sigmoid(gi_z[t] + gh_z)
 *   n      = tanh(gi_n[t] + r * gh_n)
 *   h_t    = q_out((1 - z) * n + z * h_{t-1})   (raw h_{t-1} on the carry side)
 *   out[t] = h_t
 *
 * Gate order along the 3H axis is r, z, n. All tensors are fp32, device
 * resident, with unit stride along their last axis; the other strides are
 * given in elements. The library never allocates device memory: the caller
 * passes `out` and a scratch `workspace` of gs_workspace_bytes() bytes, zeroed
 * once when it is first allocated. The dense and Monarch kernels exchange the
 * hidden state between workgroups through words tagged with a step counter
 * that lives in the workspace and advances by T per call, so one workspace
 * serves any number of calls issued in order on one stream, up to 2^32 - 2^24
 * total scan steps, after which the caller zeroes it again; calls that overlap
 * in time (two streams) need distinct workspaces.
 *
 * Those kernels are persistent: the workgroups of a batch group wait for each
 * other's words every step. The grid is capped at what the device holds at
 * once (occupancy x CUs) and launched as an ordinary kernel. A kernel on
 * another stream that holds CUs delays part of the grid; every wait is
 * bounded, and a wait that runs out sets the workspace fault word (see
 * gs_workspace_status) instead of hanging. The fault is scoped to the launch
 * (a later launch's waits are not cut short by it) and never silent: every
 * output element the launch wrote after the failed wait is NaN, and, when
 * the caller passes fault_mirror, the launch's last workgroup stores the
 * nonzero fault value into that host-visible word as the launch ends, so the
 * host can check it without synchronising.
 *
 * Return codes: GS_OK, or a negative GS_ERR_* value; gs_last_error() then
 * returns a message for the calling thread.
 *
 * Reference interfaces replaced (LarocheC/gru-triton, src/gru_qat/triton_kernels/):
 *   gs_dense_fwd     <- scan.py:76-210 (gru_scan_fwd_persistent_kernel), launched by
 *                       gru_scan_forward_persistent scan.py:213-293
 *   gs_dense_fwd_tiled <- scan.py:755-913 (gru_scan_fwd_kernel, barrier-free), launched by
 *                       gru_scan_forward scan.py:1688-1765
 *   gs_diagonal_fwd  <- scan_diagonal.py:127-223, launched by scan_diagonal.py:226-282
 *   gs_monarch_fwd   <- scan_monarch.py:130-291, launched by scan_monarch.py:320-406
 *                       (w2 != NULL selects the two-factor form, which has no
 *                       reference counterpart; see gs_args.w2)
 *   gs_butterfly_fwd <- scan_butterfly.py:168-366, launched by scan_butterfly.py:369-459
 * The quant triple mirrors the (scale, qmin, qmax) tuples of those wrappers
 * (scan.py:269-270); the in-kernel fake-quant mirrors scan.py:136-139, 176-179.
 */
#ifndef GRUSCAN_H
#define GRUSCAN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_ABI_VERSION 5

#define GS_OK 0
#define GS_ERR_INVALID (-1)  /* bad pointer, shape, stride or quant parameter (Python: ValueError) */
#define GS_ERR_CAPACITY (-2) /* persistent grid does not fit co-resident on the device (RuntimeError) */
#define GS_ERR_HIP (-3)      /* HIP runtime error; message carries hipGetErrorString (RuntimeError) */

#define GS_KIND_DENSE 0
#define GS_KIND_DIAGONAL 1
#define GS_KIND_MONARCH 2
#define GS_KIND_BUTTERFLY 3
/* Circulant hidden weights (reference _CirculantLinear, src/gru_qat/structure.py:220-240:
 * y = irfft(rfft(col) * rfft(x)), i.e. y[i] = sum_j col[(i - j) mod H] x[j]): w is Wh_circ
 * [3, H], each gate's first column col. The reference runs this kind on its per-step loop
 * (gru_layer.py:109-113); here it is the dense scan on the circulant matrices:
 * gs_circulant_fwd (H <= 1024) forms them from col inside the persistent kernel; above
 * that, and for the backward, gs_hidden_map_dense(GS_KIND_CIRCULANT) writes them,
 * gs_dense_fwd / gs_dense_bwd run the scan, and gs_hidden_map_grad folds the dense
 * weight gradient back onto col. */
#define GS_KIND_CIRCULANT 4
/* Size queries only (gs_workspace_bytes, gs_bwd_workspace_bytes, gs_bwd_scratch_bytes): the
 * batch-tiled dense entry points gs_dense_fwd_tiled / gs_dense_bwd_tiled. */
#define GS_KIND_DENSE_TILED 5

/* Frozen per-tensor symmetric fake-quant: q = clamp(rint(x / scale), qmin, qmax) * scale,
 * with the IEEE quotient and round-half-to-even. enabled == 0 turns it off. When
 * enabled, scale must lie in [2^-126, 2^64] (GS_ERR_INVALID otherwise). */
typedef struct gs_quant {
  int32_t enabled;
  float scale;
  int32_t qmin;
  int32_t qmax;
} gs_quant;

typedef struct gs_args {
  const float* gi;  /* [T, B, 3H]; strides sg_t, sg_b, 1                                   */
  const float* h0;  /* [B, H];     strides sh0_b, 1                                         */
  const float* w;   /* dense: Wh_cat [3H, H] (rows r,z,n; gh = hq @ w^T), contiguous
                       diagonal: Wh_diag [3, H], contiguous
                       Monarch: Wh_struct [3, nblocks, blksz, blksz] as (out, in), contiguous
                       butterfly: twiddles [3, bfly_nblocks, log_n, 2^log_n / 2, 2, 2], contiguous */
  const float* w2;  /* Monarch only: second block-diagonal factor, same shape as w, or NULL.
                       With w2 the hidden map is gh_g = P^T L_g P R_g hq, where R_g = w[g],
                       L_g = w2[g] and P is the stride-nblocks permutation
                       (P z)[c * nblocks + a] = z[a * blksz + c]. w2 = identity blocks
                       gives back the single-factor map. Must be NULL for other kinds. */
  const float* bh;  /* [3H], contiguous                                                     */
  float* out;       /* [T, B, H];  strides so_t, so_b, 1                                    */
  void* workspace;  /* gs_workspace_bytes() bytes, 256-byte aligned, zero on first use     */
  int64_t workspace_bytes;
  uint32_t* fault_mirror; /* optional host-visible word (hipHostMalloc memory) or NULL: a
                             persistent launch whose wait gave up stores its nonzero fault
                             value there when it ends; the caller clears it                 */
  int64_t T, B, H;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int64_t nblocks, blksz;      /* Monarch: nblocks * blksz == H                             */
  int64_t log_n, bfly_nblocks; /* butterfly: 2^log_n >= H                                   */
  gs_quant q_in;  /* applied to the matmul-side h only                                      */
  gs_quant q_out; /* applied to h_t before it is stored and carried                         */
  float* gh_save; /* gs_dense_fwd, and gs_monarch_fwd for a single factor (w2 NULL) with blksz
                     16, 32, 64 or 128, nblocks <= 65535 and ceil(B / max(1, 64 / blksz))
                     <= 65535; optional (NULL: not written; other calls must pass NULL):
                     [T, B, 3H] contiguous, where the forward also stores q_in(h_{t-1}) Wh^T
                     (gh_t without the bias bh) of every step, so that a backward can take it as
                     gs_bwd_args.gh_saved instead of recomputing it. No counterpart in the
                     reference, whose backwards recompute gh (scan.py:388-421,
                     scan_monarch.py:409-884).                                                  */
} gs_args;

/* Dense forward. H <= 1024: the persistent kernel (Wh resident in registers, the state
 * exchanged between workgroups every step, a workspace of gs_workspace_bytes() bytes).
 * 1024 < H <= 8192: the batch-tiled kernel of gs_dense_fwd_tiled (same results,
 * no workspace: gs_workspace_bytes() returns 0). */
int gs_dense_fwd(const gs_args* args, hipStream_t stream);

/* Barrier-free dense forward (reference gru_scan_fwd_kernel, scan.py:755-913, launched
 * by gru_scan_forward, scan.py:1688-1765): a 1-D grid over tiles of up to 4 batch rows,
 * each workgroup running every step of its rows and reading Wh from memory each step,
 * so no workgroup waits for another: no co-residency requirement, no workspace
 * (workspace and fault_mirror are ignored), no poll bound. 1 <= H <= 8192.
 * Same products and gate arithmetic as gs_dense_fwd, so at H <= 1024 the two return
 * bit-identical outputs; gs_dense_fwd is the faster of the two there (each step here
 * streams all 3 H^2 weights through one CU). gh_save as for gs_dense_fwd. */
int gs_dense_fwd_tiled(const gs_args* args, hipStream_t stream);

/* Dense forward with Wh also given as per-row int8 codes: w_codes [3H, H] int8
 * (16-byte aligned) and w_scale [3H], such that args->w[i][k] is the fp32 product
 * w_codes[i][k] * w_scale[i] for every element (gs_weight_codes recovers them from a
 * fake-quantized Wh_cat). Same contract and results' tolerance as gs_dense_fwd, which
 * it replaces for the frozen-int8 configuration of gru_scan_persistent
 * (scan.py:1667-1685, the weight fake-quanted per row as in quantizers.py:188-199):
 * when every A operand is a q_in level in [-128, 127] (q_in on), H > 64 is a multiple
 * of 16 and gh_save is NULL, the step's products run on the int8 MFMA over the h
 * levels and the weight codes, whose integer sums are exact, and gh = sum *
 * (w_scale[i] * q_in scale): within an fp32 rounding of each product of gs_dense_fwd's
 * fp32 chains, which round every partial sum. Every other launch is gs_dense_fwd's,
 * codes unused. H > 1024 runs gs_dense_fwd_tiled_i8w's kernel. */
int gs_dense_fwd_i8w(const gs_args* args, const int8_t* w_codes, const float* w_scale, hipStream_t stream);

/* gs_dense_fwd_tiled with the int8 codes of gs_dense_fwd_i8w (reference gru_scan_forward,
 * scan.py:1688-1765, on frozen int8 weights): the batch-tiled kernel reads the codes
 * instead of the fp32 weights every step (a quarter of the bytes) and runs the same
 * int8 products under the same rule, so it returns gs_dense_fwd_i8w's outputs bit for
 * bit up to H = 1024. No counterpart in the reference beyond that entry point. */
int gs_dense_fwd_tiled_i8w(const gs_args* args, const int8_t* w_codes, const float* w_scale, hipStream_t stream);

int gs_diagonal_fwd(const gs_args* args, hipStream_t stream);
int gs_monarch_fwd(const gs_args* args, hipStream_t stream);

/* Circulant forward (GS_KIND_CIRCULANT; the reference's _CirculantLinear hidden map,
 * structure.py:220-240, which it scans on its per-step loop, gru_layer.py:109-113): w is
 * Wh_circ [3, H]. The persistent dense kernel with each compute wave forming its rows of
 * the circulant map from col, so its outputs equal gs_dense_fwd's on the map
 * gs_hidden_map_dense writes, bit for bit, without that map in memory. H <= 1024 (above,
 * run gs_dense_fwd on the written map); a workspace of gs_workspace_bytes(GS_KIND_CIRCULANT)
 * bytes; gh_save must be NULL. */
int gs_circulant_fwd(const gs_args* args, hipStream_t stream);
int gs_butterfly_fwd(const gs_args* args, hipStream_t stream);

/* Dense forward that allocates nothing and takes no workspace. No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same contract and kernels as gs_dense_fwd, except that
 * args->workspace and args->workspace_bytes are ignored: the exchange words
 * and control words live in a static 4 MiB device array inside the library
 * (one per GPU, held until the process ends), which serves shapes whose
 * gs_workspace_bytes(GS_KIND_DENSE, args) is at most 4 MiB (B * H up to about
 * 260,000); larger shapes return GS_ERR_INVALID. The array is cleared by a
 * fill kernel on the first call on each GPU and again before its step tags
 * could wrap, as counted on the host over this entry point's calls. Every
 * call on one GPU shares that GPU's array, so calls that overlap in time on
 * one GPU (two streams, two threads) race; issue them in order on one stream.
 * Under HIP graph capture the launch is recorded (make one call outside the
 * capture first, so that the first-use fill is not part of the graph); each
 * replay advances the array's device-side tag base by T without the host
 * counting it, so keep the steps of all replays plus those of the calls below
 * 2^32 - 2^24 (about 67 million replays of a T = 64 scan), after which tags
 * could repeat. fault_mirror is this entry point's only fault channel:
 * gs_workspace_status cannot reach the static array. Above H = 1024 the
 * batch-tiled kernel runs, which exchanges nothing and uses no array. */
int gs_dense_fwd_noalloc(const gs_args* args, hipStream_t stream);

/* Same contract as gs_butterfly_fwd, but always runs the general LDS kernel
 * (any 2^log_n <= 4096, any bfly_nblocks) instead of the register kernel that
 * gs_butterfly_fwd picks for one chain at 2^log_n in {256, 512, 1024}. No
 * reference counterpart: it lets tests cross-check the two implementations. */
int gs_butterfly_fwd_generic(const gs_args* args, hipStream_t stream);

/* Scratch bytes the kind needs for these arguments (control words, exchange
 * words). Pure host arithmetic; never touches the device. Negative on error. */
int64_t gs_workspace_bytes(int kind, const gs_args* args);

/* Reads and clears the device-side fault word of a workspace (nonzero means a
 * persistent kernel ran out of its bounded wait and its output is invalid; the
 * value is that launch's tag base + 1). Synchronises the stream. Returns 1 if
 * the word was set, 0 if not, or a negative GS_ERR_* value. */
int gs_workspace_status(void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---- backward ------------------------------------------------------------------
 * Gradients of the scan (reference: the recompute-based backward of
 * src/gru_qat/triton_kernels/scan.py:1460-1550 and its per-kind Triton kernels,
 * scan.py:296-752, scan_diagonal.py:285-561, scan_monarch.py:409-884,
 * scan_butterfly.py:462-1075). Walks t from T-1 to 0, recomputes the gates from
 * h_{t-1} = out[t-1] (h0 at t = 0) and pushes dout[t] plus the carried gradient
 * through q_out's clipped-STE mask, the gates and the hidden map; q_in's mask
 * gates the carry through the map. Bias gradients (and the diagonal kind's
 * weight gradient) are returned as per-batch-row partials (sum them over
 * rows), which keeps the kernels free of atomics and their results
 * deterministic, as the reference's partial buffers do (scan.py:1445-1446);
 * the dense kind's weight gradient comes out whole.
 */
typedef struct gs_bwd_args {
  const float* gi;    /* forward inputs and output as in gs_args                      */
  const float* h0;
  const float* w;
  const float* w2;
  const float* bh;
  const float* out;   /* [T, B, H] the forward's output                               */
  const float* dout;  /* [T, B, H] contiguous: upstream gradient of out               */
  float* dgi;         /* [T, B, 3H] contiguous: gradient of gi                        */
  float* dh0;         /* [B, H] contiguous: gradient of h0                            */
  float* dw_part;     /* diagonal: [B, 3, H] per-row partial gradient of Wh_diag;      *
                       * dense: [3H, H] gradient of Wh_cat; Monarch: [3, nb, bs, bs]   *
                       * gradient of w; butterfly: gradient of the twiddles           */
  float* dw2_part;    /* two-factor Monarch: [3, nb, bs, bs] gradient of w2, else NULL */
  float* dbh_part;    /* [B, 3H] per-row partial gradient of bh                       */
  void* workspace;     /* tagged exchange words: as the forward's workspace (zeroed    *
                        * once, may be shared with forward launches on one stream)   */
  int64_t workspace_bytes;
  uint32_t* fault_mirror; /* as gs_args.fault_mirror                                */
  void* scratch;       /* plain scratch (no initial contents required), 256-byte    *
                        * aligned; never shared with a workspace, whose tag words    *
                        * must not see arbitrary float data                          */
  int64_t scratch_bytes;
  int64_t T, B, H;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b; /* strides of gi, h0, out (elements)      */
  int64_t nblocks, blksz, log_n, bfly_nblocks;
  gs_quant q_in;
  gs_quant q_out;
  const float* gh_saved; /* gs_dense_bwd, and gs_monarch_bwd for a single factor with blksz 16,
                            32, 64 or 128 and T * B <= INT32_MAX / 4; optional (NULL: gh is
                            recomputed; other calls must pass NULL): [T, B, 3H] contiguous, the
                            gh the forward wrote through gs_args.gh_save with the same inputs */
} gs_bwd_args;

int gs_diagonal_bwd(const gs_bwd_args* args, hipStream_t stream);

/* Dense backward (reference gru_scan_backward_persistent, scan.py:646-752, and
 * its kernel, scan.py:296-643). `out` must hold its steps back to back
 * (so_t == B * so_b). Needs a workspace of gs_bwd_workspace_bytes(GS_KIND_DENSE,
 * args) bytes, 256-byte aligned, zeroed before its first use (like the
 * forward's, it may be shared with forward launches on the same stream), and
 * gs_bwd_scratch_bytes() bytes of scratch. H <= 1024: the reverse recurrence
 * runs on the persistent kernel; 1024 < H <= 8192: on the batch-tiled kernel of
 * gs_dense_bwd_tiled (no workspace; gs_bwd_workspace_bytes() returns 0). */
int gs_dense_bwd(const gs_bwd_args* args, hipStream_t stream);

/* Barrier-free dense backward (reference gru_scan_backward_triton, scan.py:1355-1447,
 * kernel gru_scan_bwd_kernel, scan.py:916-1352): the passes and products of
 * gs_dense_bwd with the reverse recurrence on a 1-D grid over tiles of batch rows
 * that never wait for each other (Wh transposed once into the scratch, then read
 * from memory every step). No workspace (gs_bwd_workspace_bytes(GS_KIND_DENSE_TILED)
 * is 0), gs_bwd_scratch_bytes(GS_KIND_DENSE_TILED, args) bytes of scratch,
 * 1 <= H <= 8192. Gradients bit-identical to gs_dense_bwd's at H <= 1024. */
int gs_dense_bwd_tiled(const gs_bwd_args* args, hipStream_t stream);

/* Monarch and butterfly backward (reference scan_monarch.py:409-884 and
 * scan_butterfly.py:462-1075). A single-factor Monarch with blksz 16, 32, 64 or
 * 128 and a butterfly with one chain at 2^log_n in {256, 512, 1024} run
 * block-local / stage-wise kernels. Otherwise the hidden map, linear in q_in(h),
 * is materialized as a [3H, H] matrix and run through the dense backward (its
 * recurrence persistent up to H = 1024, batch-tiled beyond), and its [3H, H]
 * gradient is carried onto the structured parameters (dw_part, and dw2_part for
 * a two-factor Monarch): H <= 8192 for Monarch, 2^log_n <= 4096 for butterfly.
 * The stage-wise butterfly backward runs its twiddle gradient on a stream the
 * library creates per device (non-blocking, default priority), ordered by
 * events in both directions: every write of the call is complete in `stream`'s
 * order, and under graph capture that stream forks from and joins `stream`. */
int gs_monarch_bwd(const gs_bwd_args* args, hipStream_t stream);
int gs_butterfly_bwd(const gs_bwd_args* args, hipStream_t stream);

/* Bytes of tagged workspace and of plain scratch a backward entry point needs
 * (0 when it uses none: the diagonal kind needs neither, the butterfly kind's
 * stage-wise path no workspace). Pure host arithmetic. Negative on error. */
int64_t gs_bwd_workspace_bytes(int kind, const gs_bwd_args* args);
int64_t gs_bwd_scratch_bytes(int kind, const gs_bwd_args* args);

/* ---- input projection ----------------------------------------------------------
 * The producer of gi (reference GRULayer._forward_fast_dispatch,
 * src/gru_qat/gru_layer.py:249-255: xq = quant_x(x); Wi_cat, bi_cat =
 * cell.quantize_input_weights(); gi = F.linear(xq, Wi_cat, bi_cat)):
 *   gi[m][n] = sum_i q_x(x[m][i]) W_q[n][i] + bias[n]
 * with q_x a frozen per-tensor fake-quant (ste.py:65-95) and W_q the per-row
 * symmetric fake-quant of w (FakeQuantizePerChannel, quantizers.py:188-199:
 * scale[n] = max(max_i |w[n][i]|, 1e-8) / qmax, quantizers.py:124-134), or w
 * itself when q_w is off. One fp32 MFMA GEMM with the x fake-quant applied as
 * the operand is loaded and the bias added in its epilogue. When both quants are
 * on with ranges in a byte (the int8 QAT layer), I is a multiple of 16 up to 65536
 * and the caller passes the int8 scratch x_codes and w_codes (16-byte aligned), the
 * pre-passes write q_x's levels and the weight's codes there and the product runs on
 * the int8 MFMA instead: exact integer sums, gi = sum * (q_x scale * scale[n]) +
 * bias[n], within an fp32 rounding of each product of the fp32 GEMM. No
 * counterpart in the reference for the two scratch fields (ABI version 5).
 */
typedef struct gs_proj_args {
  const float* x;     /* [M, I] rows (M = T B), row stride sx                        */
  const float* w;     /* [N, I] contiguous (Wi_cat, N = 3H)                          */
  const float* bias;  /* [N] or NULL                                                 */
  float* gi;          /* [M, N] output, row stride sgi                               */
  float* x_q;         /* [M, I] contiguous: q_x(x) is written here and fed to the GEMM *
                       * (q_x on); NULL fake-quantizes x as the GEMM loads it        */
  float* w_q;         /* [N, I] the fake-quantized weight (q_w on), else NULL        */
  float* w_scale;     /* [N] its per-row scales (q_w on), else NULL                  */
  int64_t M, N, I;
  int64_t sx, sgi;
  gs_quant q_x;       /* per-tensor fake-quant of x                                  */
  gs_quant q_w;       /* per-row weight fake-quant: enabled, qmin, qmax (scale unused) */
  int8_t* x_codes;    /* [M, I] int8 scratch for q_x's levels, or NULL (see above)    */
  int8_t* w_codes;    /* [N, I] int8 scratch for the weight's codes, or NULL          */
} gs_proj_args;

int gs_input_proj(const gs_proj_args* args, hipStream_t stream);

/* Backward of gs_input_proj with the straight-through estimator of
 * fake_quant_ste (ste.py:65-95): dx = mask_x (dgi w), with q_x's clipped-STE
 * mask (its frozen scale is a constant); dw = dgi^T q_x(x), the gradient
 * reaching the weight that was used, and, when the per-row weight quant was on
 * (q_w.enabled, with w_raw and w_scale), also the path through each row's
 * scale, which the reference's dynamic per-channel weight quantizer computes
 * from the weight without detaching it (quantizers.py:188-199): the row's
 * dL/ds = sum_i dw_q[n][i] (q[n][i] - w[n][i] / s[n]) carried to its max and
 * min elements (the per-row clamp never clips); dbias = the column sums of
 * dgi (skipped when NULL). No reference counterpart as one call: the
 * reference gets these from autograd through F.linear and fake_quant_ste. */
typedef struct gs_proj_bwd_args {
  const float* x;     /* [M, I], row stride sx                                       */
  const float* w;     /* [N, I] contiguous: the weight the forward used              */
  const float* x_q;   /* [M, I] contiguous q_x(x) from the forward, or NULL (then    *
                       * x is fake-quantized as it is loaded)                        */
  const float* dgi;   /* [M, N], row stride sdgi                                     */
  float* dx;          /* [M, I], row stride sdx                                      */
  float* dw;          /* [N, I] contiguous                                           */
  float* dbias;       /* [N] or NULL                                                 */
  void* workspace;    /* gs_input_proj_bwd_workspace_bytes(args) bytes               */
  int64_t workspace_bytes;
  int64_t M, N, I;
  int64_t sx, sdgi, sdx;
  gs_quant q_x;
  const float* w_raw;   /* [N, I] contiguous: the weight before its fake-quant (q_w on)  */
  const float* w_scale; /* [N] the forward's per-row scales (q_w on)                     */
  gs_quant q_w;         /* per-row weight fake-quant of the forward: enabled, qmin, qmax */
} gs_proj_bwd_args;

int64_t gs_input_proj_bwd_workspace_bytes(const gs_proj_bwd_args* args);
int gs_input_proj_bwd(const gs_proj_bwd_args* args, hipStream_t stream);

/* ---- structured input projection -------------------------------------------------
 * The producer of gi when the cell's input side is structured (reference
 * GRUCellQuant.structured_input_projection, src/gru_qat/gru_cell.py:466-503,
 * taken by GRULayer._forward_fast_dispatch at gru_layer.py:256): for gates
 * g = r, z, n,
 *   gi[m][g H + j] = oq_g(map_g(q_x(x[m])))[j] + bias[g H + j]
 * with map_g the gate's structured input weight (struct_Wi_g; input size ==
 * hidden size H), oq_g its output-side fake-quant (quant_struct_Wi_g, applied
 * to the map's output before the bias) and q_x a frozen per-tensor fake-quant.
 * Kinds: diagonal (w [3, H], y = w_g * x), Monarch single factor (w [3,
 * nblocks, blksz, blksz] as (out, in), one block-diagonal product) and
 * butterfly (twiddles [3, bfly_nblocks, log_n, 2^log_n / 2, 2, 2], the
 * stages of the hidden-side kind). Output quantizer modes: */
#define GS_OQ_OFF 0          /* identity                                                     */
#define GS_OQ_FROZEN 1       /* per tensor, the given scale (a frozen FakeQuantizePerTensor)  */
#define GS_OQ_DYNAMIC_ROWS 2 /* symmetric, one scale per row m of the gate's output:
                                max(max_j |y[m][j]|, 1e-8) / qmax -- FakeQuantizePerChannel on
                                axis 0 in dynamic mode (quantizers.py:124-134, 188-199), the
                                reference's default weight recipe (quantizers.py:292)         */

typedef struct gs_oquant {
  int32_t mode;  /* GS_OQ_*                                                              */
  float scale;   /* GS_OQ_FROZEN                                                         */
  int32_t qmin, qmax;
} gs_oquant;

typedef struct gs_sproj_args {
  int32_t kind;       /* GS_KIND_DIAGONAL, GS_KIND_MONARCH or GS_KIND_BUTTERFLY           */
  const float* x;     /* [M, H], row stride sx                                            */
  const float* w;     /* the three gates' input-side weights, layout of gs_args.w         */
  const float* bias;  /* [3H] (b_ir, b_iz, b_in) or NULL                                  */
  float* gi;          /* [M, 3H] output, row stride sgi                                   */
  float* y;           /* [M, 3H] contiguous: map outputs before the output fake-quant;
                         required when any gate's quantizer is on (the backward reads it) */
  float* y_scale;     /* [3, M]: per-row scales of GS_OQ_DYNAMIC_ROWS gates, else NULL    */
  float* x_q;         /* [M, H] contiguous q_x(x), required when q_x is on                */
  void* scratch;      /* gs_struct_input_proj_scratch_bytes() bytes, 256-byte aligned     */
  int64_t scratch_bytes;
  int64_t M, H, sx, sgi;
  int64_t nblocks, blksz, log_n, bfly_nblocks;
  gs_quant q_x;
  gs_oquant q_out[3];
} gs_sproj_args;

int64_t gs_struct_input_proj_scratch_bytes(const gs_sproj_args* args);
int gs_struct_input_proj(const gs_sproj_args* args, hipStream_t stream);

/* Backward with the straight-through estimator of fake_quant_ste (ste.py:65-95):
 * q_x and frozen output quantizers pass the gradient where they did not clip;
 * a dynamic per-row output quantizer also passes it through its scale, as the
 * reference's autograd does (the scale is computed from the tensor, not
 * detached): dL/ds = sum_j g_j (q_j - y_j / s), carried to the row's max and
 * min elements through max(|max|, |min|) / qmax (ties shared as torch's amax,
 * amin and maximum share them). dbias = column sums of dgi. No reference
 * counterpart as one call: the reference gets these from autograd. */
typedef struct gs_sproj_bwd_args {
  int32_t kind;
  const float* x;     /* [M, H], row stride sx                                            */
  const float* x_q;   /* the forward's x_q when q_x is on                                 */
  const float* w;
  const float* y;     /* the forward's y when any output quantizer is on                  */
  const float* y_scale; /* the forward's y_scale when a gate is GS_OQ_DYNAMIC_ROWS        */
  const float* dgi;   /* [M, 3H], row stride sdgi                                         */
  float* dx;          /* [M, H], row stride sdx                                           */
  float* dw;          /* gradient of w (same shape)                                       */
  float* dbias;       /* [3H] or NULL                                                     */
  void* scratch;      /* gs_struct_input_proj_bwd_scratch_bytes() bytes, 256-byte aligned */
  int64_t scratch_bytes;
  int64_t M, H, sx, sdgi, sdx;
  int64_t nblocks, blksz, log_n, bfly_nblocks;
  gs_quant q_x;
  gs_oquant q_out[3];
} gs_sproj_bwd_args;

int64_t gs_struct_input_proj_bwd_scratch_bytes(const gs_sproj_bwd_args* args);
int gs_struct_input_proj_bwd(const gs_sproj_bwd_args* args, hipStream_t stream);

/* ---- per-row weight codes (int8 export) -------------------------------------------
 * Per-row symmetric quantization of a weight w [rows, cols] with the rule of
 * FakeQuantizePerChannel (quantizers.py:188-199, 124-134): scale[r] =
 * max(max_c |w[r][c]|, 1e-8) / qmax, codes[r][c] = clamp(rint(w[r][c] / scale[r]),
 * qmin, qmax). Writes the scales, the int8 codes (codes != NULL, qmin >= -128,
 * qmax <= 127) and/or the fake-quantized weight w_q = codes * scale (bit-exact
 * with the input projection's weight fake-quant). This is the export the
 * reference leaves as a TODO (gru_cell.py:551-553: "export_int_weights()
 * returning a dict of int tensors, scales, and zero points"). */
typedef struct gs_rows_args {
  const float* w;   /* [rows, cols] contiguous                                   */
  float* scale;     /* [rows]                                                    */
  int8_t* codes;    /* [rows, cols] contiguous, or NULL                          */
  float* w_q;       /* [rows, cols] contiguous, or NULL                          */
  int64_t rows, cols;
  int32_t qmin, qmax;
} gs_rows_args;

int gs_quantize_rows(const gs_rows_args* args, hipStream_t stream);

/* The inverse for an already fake-quantized weight w [rows, cols] (contiguous): for
 * each row, a scale s among fl(max|w| / 127) and its neighbours within two ulps such
 * that every element is the fp32 product c * s of an integer code |c| <= 127 (what
 * gs_quantize_rows' w_q holds for qmax = 127). Writes scale[r], codes[r][:] and
 * exact[r] = 1, or exact[r] = 0 (codes 0) when no candidate reproduces the row.
 * No counterpart in the reference; it feeds gs_dense_fwd_i8w. */
int gs_weight_codes(const float* w, int64_t rows, int64_t cols, int8_t* codes, float* scale, int32_t* exact,
                    hipStream_t stream);

/* ---- dense form of a hidden map --------------------------------------------------
 * Writes the hidden map of any kind as the dense matrix m [3H, H] (rows r, z,
 * n) with gh = hq m^T + bh: the diagonal kind's diag(w_g) blocks, the Monarch
 * block-diagonal factor(s) composed, the butterfly's stages applied to the
 * identity and cut to H x H. The reference materializes these maps only in
 * its tests (e.g. tests/test_triton_monarch.py:81-101 against torch.block_diag);
 * here the materialized map feeds gs_observe_scan and the backward's
 * structured paths. */
typedef struct gs_map_args {
  int32_t kind;      /* GS_KIND_*                                                  */
  const float* w;    /* as gs_args.w                                               */
  const float* w2;   /* as gs_args.w2 (Monarch two-factor), else NULL              */
  float* m;          /* [3H, H] contiguous output                                  */
  void* scratch;     /* gs_hidden_map_scratch_bytes() bytes (butterfly), 256-byte aligned */
  int64_t scratch_bytes;
  int64_t H, nblocks, blksz, log_n, bfly_nblocks;
} gs_map_args;

int64_t gs_hidden_map_scratch_bytes(const gs_map_args* args);
int gs_hidden_map_dense(const gs_map_args* args, hipStream_t stream);

/* The reverse: carries a gradient dm [3H, H] of the dense form onto the map's
 * parameters, dw (the shape of args->w): diagonal dw[g][k] = dm[g H + k][k];
 * single-factor Monarch the diagonal blocks of each gate; circulant
 * dw[g][d] = sum_i dm[g H + i][(i - d) mod H]. Each entry is one thread's
 * fixed-order sum, so results are deterministic. Butterfly and two-factor
 * Monarch parameters get their gradients from gs_butterfly_bwd /
 * gs_monarch_bwd instead (GS_ERR_INVALID here). No reference counterpart:
 * the reference gets these from autograd. */
int gs_hidden_map_grad(const gs_map_args* args, const float* dm, float* dw, hipStream_t stream);

/* ---- observers (calibration) ----------------------------------------------------
 * The reference's per-step path with its quantizers firing: GRULayer.forward
 * with use_triton off (src/gru_qat/gru_layer.py:205-223) over the step
 * step_with_gi (gru_cell.py:437-464), which GRULayer.calibrate runs to gather
 * activation statistics (gru_layer.py:308-336, calibration.py:31-126). Every
 * quantizer call is a per-tensor FakeQuantize (quantizers.py:84-96) in one of
 * four modes:
 *   GS_OBS_OFF      no quantizer (identity)
 *   GS_OBS_FROZEN   the given scale and zero point (the fast-dispatch case)
 *   GS_OBS_DYNAMIC  scale and zero point from this tensor's min and max
 *                   (_scale_zp_from_min_max, quantizers.py:124-134)
 *   GS_OBS_MIN_MAX  as DYNAMIC, and the running statistics take the tensor's
 *                   min and max (_update_observer, quantizers.py:136-156: the
 *                   first call sets them, later ones mix with momentum 0.99)
 * The fake-quant is ste.py:65-95: q = clamp(rint(x / scale + zp), qmin, qmax),
 * y = (q - zp) * scale. Scales stay on the device; nothing synchronises. */
#define GS_OBS_OFF 0
#define GS_OBS_FROZEN 1
#define GS_OBS_DYNAMIC 2
#define GS_OBS_MIN_MAX 3

typedef struct gs_observer {
  int32_t mode;       /* GS_OBS_*                                                    */
  int32_t symmetric;  /* 1: scale = max(|min|, |max|, 1e-8) / qmax, zp = 0;          *
                       * 0: scale = max(max - min, 1e-8) / (qmax - qmin),           *
                       *    zp = rint(qmin - min / scale)                           */
  int32_t qmin, qmax;
  float scale, zero_point;  /* GS_OBS_FROZEN                                         */
  float* stats;       /* GS_OBS_MIN_MAX: device float[3] = running_min, running_max, *
                       * initialized (0 or 1); read and updated in place            */
} gs_observer;

/* One quantizer call on a [rows, cols] tensor (quant_x on the whole sequence,
 * gru_layer.py:249-250): observes x and writes y = fq(x). */
typedef struct gs_observe_tensor_args {
  const float* x;   /* [rows, cols], row stride ld                                  */
  float* y;         /* [rows, cols] contiguous output                               */
  float* used;      /* device float[2]: the scale and zero point applied, or NULL  */
  void* scratch;    /* gs_observe_tensor_scratch_bytes() bytes, 256-byte aligned     */
  int64_t scratch_bytes;
  int64_t rows, cols, ld;
  gs_observer q;
} gs_observe_tensor_args;

int64_t gs_observe_tensor_scratch_bytes(const gs_observe_tensor_args* args);
int gs_observe_tensor(const gs_observe_tensor_args* args, hipStream_t stream);

/* The T-step scan with quant_h_in and quant_h_out as observers: at step t,
 * q_in sees h_{t-1} (h0, then out[t-1]; T calls), q_out sees the pre-quant h_t
 * (T calls). Same tensors, strides and hidden-map fields as gs_args; the map
 * is materialized (gs_hidden_map_dense) into the scratch, the steps run as
 * short launches. Forward only. */
typedef struct gs_observe_args {
  int32_t kind;     /* GS_KIND_*                                                    */
  const float* gi;
  const float* h0;
  const float* w;
  const float* w2;
  const float* bh;
  float* out;
  float* trace;     /* device [T, 4]: (scale, zp) of q_in and of q_out used at step t, or NULL */
  void* scratch;    /* gs_observe_scan_scratch_bytes() bytes, 256-byte aligned       */
  int64_t scratch_bytes;
  int64_t T, B, H;
  int64_t sg_t, sg_b, sh0_b, so_t, so_b;
  int64_t nblocks, blksz, log_n, bfly_nblocks;
  gs_observer q_in;
  gs_observer q_out;
} gs_observe_args;

int64_t gs_observe_scan_scratch_bytes(const gs_observe_args* args);
int gs_observe_scan(const gs_observe_args* args, hipStream_t stream);

/* Message for the last failing call on this thread ("" if none). */
const char* gs_last_error(void);

int gs_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GRUSCAN_H */
