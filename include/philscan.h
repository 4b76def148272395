/*
 * philscan — C ABI of the MI355X (gfx950) linear-recurrence kernels.
 *
 * Every entry point computes, per batch row b and step t (row-major,
 * contiguous buffers, device pointers):
 *
 *     h[b,t] = A[b,t] h[b,t-1] + x[b,t],   h[b,-1] = zi[b]
 *
 * and writes the states after consuming x[b,t]: the exact output contract of
 * philtorch's `philtorch::*` operators (philtorch/csrc/host_recur2.cpp:162-171).
 * The `_bwd` entry points compute, in one fused reverse-time pass, the
 * gradients of that output for an upstream gradient `grad_y`:
 *
 *     lambda[t] = grad_y[t] + A[t+1]^H lambda[t+1],  lambda[T-1] = grad_y[T-1]
 *     grad_x[t] = lambda[t]
 *     grad_A[t] = lambda[t] conj(h[t-1])^T   (summed where A is shared)
 *     grad_zi   = A[0]^H lambda[0]
 *
 * which is what philtorch's registered backward closures compute
 * (philtorch/__init__.py:34-148).
 *
 * Conventions
 *   - `dtype` is a phs_dtype; all pointers of one call share it.
 *   - complex values are interleaved (re, im) pairs, as torch stores them.
 *   - every call is asynchronous on `stream` (a hipStream_t; NULL = the
 *     default stream), never synchronises and never allocates: the caller
 *     passes `workspace` of at least phs_workspace_size(...) bytes (a larger
 *     one is fine; pass its full size).  The workspace must be zero-filled
 *     once before its first use; every call leaves it ready for the next, so
 *     nothing is cleared per call.  Calls sharing one workspace must be
 *     ordered (same stream, or synchronised): concurrent calls on one
 *     workspace race.
 *   - nullable outputs of the `_bwd` calls are skipped when NULL.
 *   - return value: PHS_OK or a phs_status error code; inputs are never
 *     modified; a call with B == 0 or T == 0 does nothing.
 */
#ifndef PHILSCAN_H_
#define PHILSCAN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum phs_dtype { PHS_F32 = 0, PHS_F64 = 1, PHS_C64 = 2, PHS_C128 = 3, PHS_I64 = 4 };

enum phs_op {
  PHS_OP_RECUR = 0,
  PHS_OP_LTI_RECUR = 1,
  PHS_OP_RECUR2 = 2,
  PHS_OP_LTI_RECUR2 = 3,
  PHS_OP_RECURN = 4,    /* order-M ops, phs_workspace_size_n only */
  PHS_OP_LTI_RECURN = 5
};

enum phs_status {
  PHS_OK = 0,
  PHS_ERR_INVALID = 1,   /* bad size, null required pointer, unsupported combination */
  PHS_ERR_WORKSPACE = 2, /* workspace NULL or smaller than phs_workspace_size() */
  PHS_ERR_LAUNCH = 3,    /* the HIP runtime rejected a kernel launch */
  PHS_ERR_DTYPE = 4,     /* dtype not one of phs_dtype */
  PHS_ERR_TOO_LARGE = 5  /* beyond PHS_NOALLOC_SCRATCH_BYTES (phs_recur_fwd_noalloc only) */
};

/* Bytes of workspace that one call of `op` needs (backward != 0 for the
 * `_bwd` entry point).  `coef_shared` is the same flag the call receives. */
size_t phs_workspace_size(int op, int dtype, int64_t B, int64_t T, int coef_shared, int backward);

/* phs_workspace_size for an op of state order M.  PHS_OP_RECURN and
 * PHS_OP_LTI_RECURN take M = 1..4; the fixed-order ops accept only their own
 * order (1 for PHS_OP_RECUR / PHS_OP_LTI_RECUR, 2 for the *2 ops).  Returns 0
 * for an unsupported combination. */
size_t phs_workspace_size_n(int op, int dtype, int M, int64_t B, int64_t T, int coef_shared, int backward);

/* Human-readable text of a phs_status code (static storage). */
const char *phs_error_string(int status);

/* ABI version of this library (major*100 + minor). */
int phs_abi_version(void);

/* Testing hook, no counterpart in the reference.  Sets the number of
 * look-back polls a tile makes before it stops waiting for its predecessors
 * and computes its entry state from the inputs itself (0 restores the
 * default, about 0.1 s of waiting).  A tiny value forces that fallback path
 * so tests can check it; results are identical either way.  Process-wide;
 * takes effect for calls issued afterwards. */
void phs_debug_set_spin_limit(unsigned polls);

/* Testing hook, no counterpart in the reference.  With `on` != 0, every tile
 * after the first of its row publishes only its aggregate, never the state
 * leaving it, and no look-back polls early: each look-back then folds its
 * way back to the row's first tile, window after window of 64 aggregates,
 * which normal runs reach only when more than a window of predecessors are
 * still unresolved.  Every tile still publishes before it waits, so every
 * kernel completes; results are unchanged.  0 restores normal publishing.
 * Process-wide; takes effect for calls issued afterwards. */
void phs_debug_set_aggregates_only(int on);

/* Testing hook, no counterpart in the reference.  Forces the cascade
 * gradient backward's kept_step (phs_sosfilt_bwd and phs_biquad_bwd with
 * coefficient gradients): the sections whose forward input stays in LDS, so
 * that re-deriving a section's input runs from the nearest kept one (0: none
 * kept, every re-derivation runs from x).  step < 0 restores the automatic
 * choice, which this device's LDS and register counts decide; a forced
 * value whose kept inputs exceed the LDS left to the kernel makes the call
 * return PHS_ERR_INVALID.  Results are identical for every value.
 * Process-wide; takes effect for calls issued afterwards. */
void phs_debug_set_sos_kept_step(int step);

/* Measurement hook, no counterpart in the reference.  The next main-kernel
 * launch of this library (the scan, cascade, state-space or probe kernel of
 * the next call; not a follow-up reduction) records `start_event` and
 * `stop_event` (hipEvent_t, either may be NULL) around the kernel itself
 * through hipExtLaunchKernelGGL, so their elapsed time is that kernel's
 * duration from dispatch to completion, as a profiler's kernel trace
 * measures it, without the event packets' own overhead.  The hook is
 * consumed by that launch; NULL, NULL disarms it.  Process-wide. */
void phs_debug_time_next_launch(void *start_event, void *stop_event);

/* Measurement hook, no counterpart in the reference.  The next scan launch of
 * phs_{recur,lti_recur,recur2,lti_recur2}_{fwd,bwd} in fp32, fp64 (scalar
 * ops) or complex64 (scalar ops), and fp32 (2x2 ops) whose tile count is at
 * most `n_records` runs the tracing build of the scan kernel and writes one
 * record of 8 uint64 words per tile into `records` (device memory, tile id
 * order; tile id = position along the row * B + row, backward positions
 * counted from the row's end): s_memrealtime stamps (100 MHz) at the
 * workgroup's start, after its tile claim, when data wave 0 has loaded and
 * folded its segment, when the tile's look-back starts, when its entry state
 * is known and when data wave 0 has issued its last stores; then the
 * look-back's failed polls and the tile id.  Results are those of an
 * untraced launch.  The hook is consumed by the next scan launch, traced or
 * not (records untouched if it is not); NULL or 0 disarms it.
 * Process-wide. */
void phs_debug_trace_next_launch(void *records, size_t n_records);

/* LPV scalar scan.  A: [B,T] (coef_shared=0) or [T] shared by all rows
 * (coef_shared=1); zi: [B]; x, y: [B,T].
 * Replaces philtorch::recurN with 1x1 matrices, the only native time-varying
 * scalar scan of the reference: host_recurN.cpp:236-281 (CPU impl registered
 * at :285); the reference's lpv.linear_recurrence (lpv/recur.py:20-101) has
 * no native op of its own. */
int phs_recur_fwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                  const void *x, void *y, void *workspace, size_t workspace_bytes, void *stream);

/* phs_recur_fwd without a workspace argument: allocates nothing, takes no
 * workspace.  No counterpart in the reference; for callers that cannot
 * allocate or hand over device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Its workspace is a static
 * device array of PHS_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends (at most B * ceil(T / tile) tiles of 48 bytes for fp32/fp64 after a
 * 2 KiB header: about 716 M fp32 samples in 8192-step tiles); larger
 * problems return PHS_ERR_TOO_LARGE without launching anything.  The array
 * is cleared by a kernel on the first call on each device (and every 2^30
 * calls); every call on one GPU shares it and leaves it ready for the next,
 * so calls on one GPU must be ordered (one stream, or synchronised):
 * overlapping calls race.  Results are bit-identical to phs_recur_fwd's. */
#define PHS_NOALLOC_SCRATCH_BYTES (4u << 20)
int phs_recur_fwd_noalloc(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                          const void *x, void *y, void *stream);

/* Backward of phs_recur_fwd.  y: the forward output.  grad_A: [B,T], or [T]
 * when coef_shared (summed over rows).  grad_zi: [B].  grad_x: [B,T].
 * Replaces the recurN autograd closure philtorch/__init__.py:34-73. */
int phs_recur_bwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                  const void *y, const void *grad_y, void *grad_x, void *grad_A, void *grad_zi,
                  void *workspace, size_t workspace_bytes, void *stream);

/* LTI scalar scan.  a: [B] (coef_shared=0) or one value shared by all rows
 * (coef_shared=1); zi: [B]; x, y: [B,T].
 * Replaces lti_recur_cuda_impl, philtorch/csrc/lti_recur.cu:113-158
 * (registered at :160; CPU twin host_lti_recur.cpp:42-80). */
int phs_lti_recur_fwd(int dtype, int64_t B, int64_t T, const void *a, int coef_shared,
                      const void *zi, const void *x, void *y, void *workspace,
                      size_t workspace_bytes, void *stream);

/* Backward of phs_lti_recur_fwd.  grad_a: [B], or one value when
 * coef_shared: sum_t conj(h[t-1]) lambda[t], reduced deterministically.
 * Replaces _lti_recur_backward, philtorch/__init__.py:115-148. */
int phs_lti_recur_bwd(int dtype, int64_t B, int64_t T, const void *a, int coef_shared,
                      const void *zi, const void *y, const void *grad_y, void *grad_x,
                      void *grad_a, void *grad_zi, void *workspace, size_t workspace_bytes,
                      void *stream);

/* LPV 2x2 scan.  A: [B,T,2,2] (coef_shared=0) or [T,2,2] (coef_shared=1);
 * zi: [B,2]; x, y: [B,T,2].
 * Replaces mat_recur_second_order_cuda_impl, philtorch/csrc/recur2.cu:69-117
 * (registered at :119-122; CPU twin host_recurN.cpp:236-281). */
int phs_recur2_fwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                   const void *x, void *y, void *workspace, size_t workspace_bytes, void *stream);

/* Backward of phs_recur2_fwd.  grad_A: [B,T,2,2], or [T,2,2] when
 * coef_shared.  grad_zi: [B,2].  grad_x: [B,T,2].
 * Replaces the recur2 autograd closure philtorch/__init__.py:34-73. */
int phs_recur2_bwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared,
                   const void *zi, const void *y, const void *grad_y, void *grad_x, void *grad_A,
                   void *grad_zi, void *workspace, size_t workspace_bytes, void *stream);

/* LTI 2x2 scan.  A: [B,2,2] (coef_shared=0) or [2,2] (coef_shared=1);
 * zi: [B,2]; x, y: [B,T,2].
 * Replaces lti_mat_recur_second_order_cuda_impl,
 * philtorch/csrc/lti_recur2.cu:66-113 (registered at :115-118; CPU twin
 * host_lti_recurN.cpp:63-108). */
int phs_lti_recur2_fwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared,
                       const void *zi, const void *x, void *y, void *workspace,
                       size_t workspace_bytes, void *stream);

/* Backward of phs_lti_recur2_fwd.  grad_A: [B,2,2], or [2,2] when
 * coef_shared, sum_t lambda[t] conj(h[t-1])^T.
 * Replaces the lti_recur2 autograd closure philtorch/__init__.py:76-112. */
int phs_lti_recur2_bwd(int dtype, int64_t B, int64_t T, const void *A, int coef_shared,
                       const void *zi, const void *y, const void *grad_y, void *grad_x,
                       void *grad_A, void *grad_zi, void *workspace, size_t workspace_bytes,
                       void *stream);

/* LPV MxM scan of state order M = 1..4.  A: [B,T,M,M] (coef_shared=0) or
 * [T,M,M] (coef_shared=1), row-major matrices; zi: [B,M]; x, y: [B,T,M].
 * Replaces philtorch::recurN, whose only implementation in the reference is
 * the CPU one, host_recurN.cpp:236-281 (registered at :285).  M = 1 and 2 run
 * the kernels of phs_recur_fwd and phs_recur2_fwd. */
int phs_recurN_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                   const void *x, void *y, void *workspace, size_t workspace_bytes, void *stream);

/* Backward of phs_recurN_fwd.  grad_A: [B,T,M,M], or [T,M,M] when
 * coef_shared.  grad_zi: [B,M].  grad_x: [B,T,M].
 * Replaces the recurN autograd closure philtorch/__init__.py:34-73. */
int phs_recurN_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                   const void *y, const void *grad_y, void *grad_x, void *grad_A, void *grad_zi,
                   void *workspace, size_t workspace_bytes, void *stream);

/* LTI MxM scan of state order M = 1..4.  A: [B,M,M] (coef_shared=0) or
 * [M,M] (coef_shared=1); zi: [B,M]; x, y: [B,T,M].
 * Replaces philtorch::lti_recurN, CPU-only in the reference:
 * host_lti_recurN.cpp:63-108 (registered at :110-113).  M = 1 and 2 run the
 * kernels of phs_lti_recur_fwd and phs_lti_recur2_fwd. */
int phs_lti_recurN_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared,
                       const void *zi, const void *x, void *y, void *workspace, size_t workspace_bytes,
                       void *stream);

/* Backward of phs_lti_recurN_fwd.  grad_A: [B,M,M], or [M,M] when
 * coef_shared, sum_t lambda[t] conj(h[t-1])^T.
 * Replaces the lti_recurN autograd closure philtorch/__init__.py:76-112. */
int phs_lti_recurN_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared,
                       const void *zi, const void *y, const void *grad_y, void *grad_x, void *grad_A,
                       void *grad_zi, void *workspace, size_t workspace_bytes, void *stream);

/* ---- Cascade of second-order sections (biquads), fused.
 * No counterpart op in the reference: it replaces the caller pattern of one
 * philtorch lfilter(form="tdf2") per section (philtorch/lti/filtering.py:
 * 211-333, each section a philtorch::lti_recur2 with its Bx and C/D glue) by
 * one pass over all sections.  Semantics of scipy.signal.sosfilt: section s
 * of row b, sos[.., s, :] = (b0, b1, b2, a0 = 1, a1, a2), transposed direct
 * form II,
 *     y[t] = h[t-1].0 + b0 u[t],  h[t] = [[-a1, 1], [-a2, 0]] h[t-1] + (b1 - b0 a1, b2 - b0 a2) u[t],
 * h[-1] = zi[b, s], zf[b, s] = h[T-1]; section 0 reads x, section s+1 reads
 * section s's output, y is section S-1's output.  dtype PHS_F32 or PHS_F64;
 * S = 1..8 per call (a longer cascade is a chain of calls, each over its own
 * sections); sos: [B,S,6] (sos_shared=0) or [S,6] (sos_shared=1), the a0
 * entries are not read (callers normalise them to 1); x, y: [B,T];
 * zi, zf: [B,S,2]. */

/* Workspace bytes of phs_sosfilt_fwd (backward=0) or of either call
 * (backward!=0); 0 for unsupported arguments. */
size_t phs_sosfilt_workspace_size(int dtype, int64_t B, int64_t T, int S, int backward);

/* Bytes of the state checkpoints the forward writes for the backward's
 * coefficient gradients: the state entering every 32nd step (PHS_F32; every
 * 8th for PHS_F64) of every section, as fp64 pairs. */
size_t phs_sosfilt_ckpt_size(int dtype, int64_t B, int64_t T, int S);

/* Forward.  zi NULL = zero initial states; zf and ckpt are skipped when NULL.
 * ckpt (phs_sosfilt_ckpt_size bytes) is required later by the backward when
 * it computes grad_sos. */
int phs_sosfilt_fwd(int dtype, int64_t B, int64_t T, int S, const void *sos, int sos_shared, const void *zi,
                    const void *x, void *y, void *zf, void *ckpt, void *workspace, size_t workspace_bytes,
                    void *stream);

/* Backward: the adjoint cascade (sections in reverse order, time reversed).
 * grad_zf NULL = zero.  grad_x [B,T], grad_zi [B,S,2] are skipped when NULL.
 * grad_sos ([B,S,6], or [S,6] summed over rows when sos_shared; the a0 entries
 * are 0) needs x and the forward's ckpt; when NULL they are not read. */
int phs_sosfilt_bwd(int dtype, int64_t B, int64_t T, int S, const void *sos, int sos_shared, const void *x,
                    const void *ckpt, const void *grad_y, const void *grad_zf, void *grad_x, void *grad_sos,
                    void *grad_zi, void *workspace, size_t workspace_bytes, void *stream);

/* ---- One biquad given as lfilter's b and a where they lie (no sos array;
 * lfilter(b, a, x, form="tdf2"), philtorch/lti/filtering.py:211-333, for a
 * second-order filter: the forward is the state-space kernel's pass of the
 * TDF-II model, which also writes the checkpoints, the backward the cascade
 * kernel at S = 1): b [B, nb]
 * (nb = 1..3, missing taps zero) and a [B, 2] (after the leading 1), each
 * row at its own stride in elements (0 = one filter for all rows, inner
 * stride 1); zi, zf [B, 2]; ckpt as phs_sosfilt_fwd's at S = 1; workspace
 * phs_sosfilt_workspace_size at S = 1.  The backward writes grad_b [B|1, nb]
 * and grad_a [B|1, 2] (one row when both strides are 0; both NULL for no
 * coefficient gradient, then x and ckpt may be NULL). */
int phs_biquad_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                   int64_t a_row_stride, const void *zi, const void *x, void *y, void *zf, void *ckpt,
                   void *workspace, size_t workspace_bytes, void *stream);

int phs_biquad_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                   int64_t a_row_stride, const void *x, const void *ckpt, const void *grad_y, const void *grad_zf,
                   void *grad_x, void *grad_b, void *grad_a, void *grad_zi, void *workspace, size_t workspace_bytes,
                   void *stream);

/* phs_biquad_bwd for a biquad whose b and a are columns of coefficient
 * tables (the C4 caller pattern's b[:, s] of a [B, S, 3] table): the
 * gradient reduction writes the whole tables, grad_b_table [B|1, b_cols, nb]
 * with dL/db at column b_col and zeros in the other columns, grad_a_table
 * [B|1, a_cols, 2] likewise (contiguous; b_cols = a_cols = 1 and column 0
 * are phs_biquad_bwd's grad_b and grad_a).  No counterpart in the
 * reference: it replaces autograd's zero-filled table and column copy per
 * call of the caller pattern over philtorch/lti/filtering.py:211-333
 * (torch's select backward). */
int phs_biquad_bwd_cols(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                        int64_t a_row_stride, const void *x, const void *ckpt, const void *grad_y,
                        const void *grad_zf, void *grad_x, void *grad_b_table, int b_cols, int b_col,
                        void *grad_a_table, int a_cols, int a_col, void *grad_zi, void *workspace,
                        size_t workspace_bytes, void *stream);

/* ---- Zero-phase filtering with a filter of order 1..4 per row (its
 * gradients: phs_filtfilt_bwd below).  Replaces philtorch.lti.
 * filtering.filtfilt (philtorch/lti/filtering.py:413-484, with lfilter_zi
 * :107-142) for a filter b / a:
 *     ext = F.pad(x, (padlen, padlen), mode=padmode)
 *     y1  = lfilter(b, a, ext, zi = lfilter_zi(a, b) * ext[:, 0])
 *     y2  = lfilter(b, a, flip(y1), zi = lfilter_zi(a, b) * y1[:, -1])
 *     y   = flip(y2[:, padlen : padlen + T])
 * computed as two state-space launches (one per pass; the second runs in
 * reversed time) and no copies: the padded row, the flips and the trim are
 * never materialised, and each pass's entry state is derived inside the
 * kernel from the row's edge, with lfilter_zi in closed form (the
 * reference's linalg.solve synchronises with the host; a filter with a pole
 * at z = 1, 1 + sum(a) = 0, raises there and gives non-finite output here).
 * The output is the same for form "tdf2" and "df2": both start every pass
 * from the steady state of the same transfer function.  dtype PHS_F32 or
 * PHS_F64; b: [B,nb] (coef_shared=0) or [nb] (coef_shared=1), nb = 1..5;
 * a: [B,na] or [na], the denominator after its leading 1, na = 1..4 (as
 * philtorch's b and a; the order is max(nb - 1, na)); x, y: [B,T];
 * 0 <= padlen < T (T >= 1); padmode a phs_padmode code; padlen 0 means no
 * padding, whatever the mode. */
enum phs_padmode { PHS_PAD_CONSTANT = 0, PHS_PAD_REPLICATE = 1, PHS_PAD_REFLECT = 2, PHS_PAD_CIRCULAR = 3 };

/* Workspace bytes of phs_filtfilt_fwd (self-resetting, like every other
 * workspace here); 0 for unsupported arguments. */
size_t phs_filtfilt_workspace_size(int dtype, int64_t B, int64_t T);

/* Bytes of phs_filtfilt_fwd's scratch buffer `mid` (the first pass's output
 * and its [B,4] final states; any contents, 16-byte aligned). */
size_t phs_filtfilt_mid_size(int dtype, int64_t B, int64_t T);

int phs_filtfilt_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                     int coef_shared, int padmode, int64_t padlen, const void *x, void *y, void *mid, void *workspace,
                     size_t workspace_bytes, void *stream);

/* ---- Gradients of the zero-phase filter: grad_x = J^T grad_y of the
 * linear map x -> phs_filtfilt_fwd(x) (same b, a, padmode, padlen) and,
 * when grad_b and grad_a are given (both or neither), dL/db [nb] or [B,nb]
 * and dL/da [na] or [B,na] (shared filters: summed over the rows), for
 * L = <grad_y, y>.  Replaces the autograd of philtorch.lti.filtering.
 * filtfilt's composed graph (philtorch/lti/filtering.py:413-484: F.pad,
 * lfilter_zi * ext[:, :1] with its linalg.solve, two lfilter passes with
 * their flips, the trim).  Input only: two state-space launches of the
 * adjoint model (the DF-II form of b and a, each in the direction opposite
 * to its forward pass) and two one-thread-per-row kernels for the pad
 * pieces and the steady-state edge terms (padlen serial steps per row).
 * With coefficient gradients: both passes again keeping their states, the
 * adjoint launches also summing dL/dA, dL/dg, dL/db0 of the TDF-II model
 * over the interior, the pads' sums and dL/dz (z = lfilter_zi) in the
 * per-row kernels, the chain rule to b and a.  The padded, flipped and
 * trimmed signals are never materialised.  Arguments as phs_filtfilt_fwd;
 * x: [B,T], read only for coefficient gradients (may be NULL otherwise);
 * grad_y, grad_x: [B,T]; workspace as phs_filtfilt_workspace_size;
 * scratch: phs_filtfilt_bwd_scratch_size(dtype, M = max(nb - 1, na), B, T,
 * padlen, need_coef) bytes (any contents, 16-byte aligned). */
size_t phs_filtfilt_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T, int64_t padlen, int need_coef);

int phs_filtfilt_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                     int coef_shared, int padmode, int64_t padlen, const void *x, const void *grad_y, void *grad_x,
                     void *grad_b, void *grad_a, void *scratch, size_t scratch_bytes, void *workspace,
                     size_t workspace_bytes, void *stream);

/* ---- The filtfilt pair split for a caller that keeps the forward's states
 * (no counterpart in the reference, whose autograd saves the composed
 * route's tensors; philtorch/lti/filtering.py:107-142, 413-484).
 * phs_filtfilt_fwd_hs: phs_filtfilt_fwd whose two passes also write their
 * states, h1 and h2 [B,T,M] each (M = max(nb - 1, na)), beside pass 1's
 * output in `mid` (its y agrees with phs_filtfilt_fwd's to rounding: the
 * states-and-output mode scans other tile lengths).  phs_filtfilt_bwd_hs:
 * phs_filtfilt_bwd given that mid, h1 and h2 (all three, or none: then it
 * computes them again); with grad_b/grad_a it skips both passes' recompute,
 * with the same results bit for bit. */
int phs_filtfilt_fwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                        int coef_shared, int padmode, int64_t padlen, const void *x, void *y, void *mid, void *h1,
                        void *h2, void *workspace, size_t workspace_bytes, void *stream);

int phs_filtfilt_bwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                        int coef_shared, int padmode, int64_t padlen, const void *x, const void *mid, const void *h1,
                        const void *h2, const void *grad_y, void *grad_x, void *grad_b, void *grad_a, void *scratch,
                        size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream);

/* ---- Single-input, single-output LTI state space of order M = 1..4, fused
 * (forward).  Replaces philtorch.lti.state_space (philtorch/lti/ssm.py:
 * 386-510 with _ssm_C_D :513-589) for a 2D input x, B an M-vector (or
 * absent: the input enters state 0, as _ext_ss_recur pads it, :186-191), C
 * an M-vector or out_idx, D one value per row (or absent):
 *     h[0] = zi,  y[t] = c . h[t] + d x[t],  h[t+1] = A h[t] + b x[t],  zf = h[T]
 * in one pass, instead of the B x product, the scan, the shifted copy and
 * C h + D x (the route of lfilter in companion form, lti/filtering.py:
 * 273-333).  dtype PHS_F32 or PHS_F64; A: [B,M,M] or [M,M] (A_shared);
 * b, c: [B,M] or [M] (*_shared), b NULL = e0, c NULL = e_out_idx; d: [B] or
 * one value (d_shared), NULL = 0; zi [B,M] (NULL = zeros); x, y [B,T];
 * zf [B,M] (skipped when NULL). */

/* Workspace bytes of phs_lti_ss_fwd; 0 for unsupported arguments. */
size_t phs_lti_ss_workspace_size(int dtype, int M, int64_t B, int64_t T);

int phs_lti_ss_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream);

/* The same model run backwards in time (no counterpart in the reference,
 * which flips: it equals flipping x, running phs_lti_ss_fwd and flipping y):
 * h[T] = zi, y[t] = c . h[t+1] + d x[t], h[t] = A h[t+1] + b x[t],
 * zf = h[0].  The adjoint of the forward model is this one on (A^T, c, b, d)
 * from dL/dzf, so a gradient pass needs no flipped copies. */
int phs_lti_ss_rev(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream);

/* ---- lfilter of order M = max(nb - 1, na) = 1..4 in one pass (forward).
 * Replaces philtorch.lti.lfilter (philtorch/lti/filtering.py:211-333) in
 * the companion-form state space it builds (_ssm_lfilter :273-333) for forms
 * "tdf2" (A = companion(a)^T, B = b[1:] - b0 a, out_idx 0, D = b0) and "df2"
 * (A = companion(a), input into state 0, C = b[1:] - b0 a, D = b0), b and
 * a zero-padded to order M; the companion matrix and the B/C vectors are
 * built inside the kernel from b and a.  dtype PHS_F32 or PHS_F64; b [B,nb]
 * or [nb], a [B,na] or [na] (the denominator after its leading 1;
 * coef_shared for the 1D forms); form a phs_form code; zi [B,M] in the
 * form's state coordinates (NULL = zeros); x, y [B,T]; zf [B,M] (skipped
 * when NULL).  Workspace: phs_lti_ss_workspace_size(dtype, M, B, T). */
enum phs_form { PHS_FORM_TDF2 = 0, PHS_FORM_DF2 = 1 };

int phs_lfilter_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, void *y, void *zf, void *workspace,
                    size_t workspace_bytes, void *stream);

/* The same filter run backwards in time, as phs_lti_ss_rev (flip, filter,
 * flip without the copies; zi the state before x[T-1], zf the state after
 * x[0]).  The adjoint of a companion form is the other form run this way. */
int phs_lfilter_rev(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, void *y, void *zf, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ---- Gradients of phs_lti_ss_fwd (reverse = 0) or phs_lti_ss_rev
 * (reverse = 1) w.r.t. x, zi and every coefficient, in two passes and two
 * small reductions.  Replaces the autograd of the composed state space the
 * reference differentiates (philtorch/lti/ssm.py:386-589; B x, the scan, the
 * state shift, C h + D x):
 *     dL/dA = sum_t lambda[t+1] h[t]^T,  dL/db = sum_t lambda[t+1] x[t],
 *     dL/dc = sum_t g[t] h[t],           dL/dd = sum_t g[t] x[t],
 * with g = dL/dy, lambda[t] = dL/dh[t] = A^T lambda[t+1] + c g[t] from
 * lambda[T] = dL/dzf; dL/dx[t] = b . lambda[t+1] + d g[t], dL/dzi =
 * lambda[0].  The model's arguments are phs_lti_ss_fwd's (same shapes and
 * sharing); gy [B,T] = dL/dy; gzf [B,M] or NULL (zero); outputs gx [B,T],
 * gzi [B,M], gA, gb, gc, gd shaped like A, b, c, d (one for a shared
 * operand: summed over the rows), each nullable (gb, gc, gd must be NULL
 * when their operand is).  The first pass runs the model again and keeps
 * its states (B*T*M values) in `scratch` (phs_lti_ss_bwd_scratch_size
 * bytes, with the partial sums; any contents); `workspace` is
 * phs_lti_ss_workspace_size bytes, as for the forward. */
size_t phs_lti_ss_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T);

int phs_lti_ss_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, const void *gy, const void *gzf, void *gx, void *gzi, void *gA, void *gb, void *gc,
                   void *gd, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                   size_t workspace_bytes, void *stream);

/* Gradients of phs_lfilter_fwd / phs_lfilter_rev w.r.t. x, zi, b [.., nb]
 * and a [.., na] (gb, ga shaped like b and a, summed over the rows when
 * coef_shared), by the chain rule through the companion model (replaces the
 * autograd of philtorch/lti/filtering.py:273-333).  Scratch and workspace:
 * phs_lti_ss_bwd_scratch_size and phs_lti_ss_workspace_size at
 * M = max(nb - 1, na). */
int phs_lfilter_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, const void *gy, const void *gzf, void *gx, void *gzi,
                    void *gb, void *ga, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ---- The LTI pairs split for a caller that keeps the forward's states (no
 * counterpart in the reference, whose autograd saves the composed route's
 * tensors; philtorch/lti/ssm.py:386-589, philtorch/lti/filtering.py:273-333):
 * the forward (reverse = 0) or reversed pass that also writes hs [B,T,M],
 * the state before every step, in the same pass (its y may differ from the
 * plain pass's in the last bits: the states-and-output mode scans other tile
 * lengths), and the backward given those states, which runs the adjoint pass
 * only (hs NULL: recomputed, as phs_lti_ss_bwd / phs_lfilter_bwd; the
 * gradients equal theirs bit for bit). */
int phs_lti_ss_fwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b,
                      int b_shared, const void *c, int c_shared, int out_idx, const void *d, int d_shared,
                      const void *zi, const void *x, void *y, void *zf, void *hs, int reverse, void *workspace,
                      size_t workspace_bytes, void *stream);

int phs_lti_ss_bwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b,
                      int b_shared, const void *c, int c_shared, int out_idx, const void *d, int d_shared,
                      const void *zi, const void *x, const void *hs, const void *gy, const void *gzf, void *gx,
                      void *gzi, void *gA, void *gb, void *gc, void *gd, int reverse, void *scratch,
                      size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream);

int phs_lfilter_fwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                       int coef_shared, int form, const void *zi, const void *x, void *y, void *zf, void *hs,
                       int reverse, void *workspace, size_t workspace_bytes, void *stream);

int phs_lfilter_bwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                       int coef_shared, int form, const void *zi, const void *x, const void *hs, const void *gy,
                       const void *gzf, void *gx, void *gzi, void *gb, void *ga, int reverse, void *scratch,
                       size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream);

/* Flags of the A argument of phs_lpv_ss_fwd / phs_lpv_ss_rev (A_flags):
 * PHS_LPV_A_SHARED, A is [T,M,M] and shared by the rows; PHS_LPV_A_TRANSPOSED,
 * every step's matrix is read transposed, so the adjoint model's A[t]^T
 * needs no transposed copy of A. */
#define PHS_LPV_A_SHARED 1
#define PHS_LPV_A_TRANSPOSED 2

/* ---- Single-input, single-output LPV (time-varying) state space of order
 * M = 1..4, fused (forward).  Replaces philtorch.lpv.state_space
 * (philtorch/lpv/ssm.py:337-581, the glue :413-577) for a 2D input x:
 *     h[0] = zi,  y[t] = c[t] . h[t] + d[t] x[t],
 *     h[t+1] = A[t] h[t] + b[t] x[t],  zf = h[T]
 * in one pass: per step A[t], x[t] and the time-varying ones of b, c, d are
 * read and y[t] written.  dtype PHS_F32 or PHS_F64; A [B,T,M,M], or [T,M,M]
 * with PHS_LPV_A_SHARED in A_flags (PHS_LPV_A_TRANSPOSED: use A[t]^T); b, c element (row, t, i) at ptr + row * row_stride +
 * t * t_stride + i and d element (row, t) at ptr + row * row_stride +
 * t * t_stride (strides in elements, >= 0; 0 shares that axis); b NULL: the
 * input enters state 0; c NULL: y is state out_idx; d NULL: no feedthrough;
 * zi [B,M] (NULL = zeros); x, y [B,T]; zf [B,M] (skipped when NULL). */
size_t phs_lpv_ss_workspace_size(int dtype, int M, int64_t B, int64_t T);

int phs_lpv_ss_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream);

/* The same model run backwards in time (no counterpart in the reference,
 * which flips): h[T] = zi, y[t] = c[t] . h[t+1] + d[t] x[t],
 * h[t] = A[t] h[t+1] + b[t] x[t], zf = h[0].  The adjoint of the forward
 * model is this one on (A[t]^T, input vector c[t], output vector b[t], d[t])
 * from dL/dzf: y = grad_x, zf = grad_zi. */
int phs_lpv_ss_rev(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream);

/* ---- Gradients of phs_lpv_ss_fwd (reverse = 0) or phs_lpv_ss_rev
 * (reverse = 1) w.r.t. x, zi and every coefficient, in two passes (the
 * forward again keeping its states, then the adjoint model in the opposite
 * time direction).  Replaces the autograd of the composed LPV state space
 * (philtorch/lpv/ssm.py:337-581):
 *     dL/dA[t] = lambda[t+1] h[t]^T,  dL/db[t] = lambda[t+1] x[t],
 *     dL/dc[t] = g[t] h[t],           dL/dd[t] = g[t] x[t],
 * lambda[t] = A[t]^T lambda[t+1] + c[t] g[t] from lambda[T] = dL/dzf,
 * summed over the axes an operand shares.  The model's arguments are
 * phs_lpv_ss_fwd's; gy [B,T]; gzf [B,M] or NULL; outputs gx [B,T], gzi [B,M]
 * and gA, gb, gc, gd contiguous in their operand's shape (A [B|1,T,M,M]
 * without the row axis when shared; b, c [1|B, 1|T, M]; d [1|B, 1|T]; a
 * stride-0 axis of the operand has extent 1), each nullable (gb, gc, gd NULL
 * when their operand is).  `scratch`: phs_lpv_ss_bwd_scratch_size bytes for
 * the same step_shared, the PHS_LPV_GRAD_* bits of the operands that vary
 * along time and are shared by the rows (A with PHS_LPV_A_SHARED, b, c, d
 * with row stride 0 and time stride not 0), any contents; `workspace`:
 * phs_lpv_ss_workspace_size bytes. */
#define PHS_LPV_GRAD_A 1
#define PHS_LPV_GRAD_B 2
#define PHS_LPV_GRAD_C 4
#define PHS_LPV_GRAD_D 8

size_t phs_lpv_ss_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T, int step_shared);

int phs_lpv_ss_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, const void *gy, const void *gzf, void *gx, void *gzi, void *gA, void *gb, void *gc,
                   void *gd, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                   size_t workspace_bytes, void *stream);

/* ---- The same pair split for a caller that keeps the forward's states (no
 * counterpart in the reference, whose autograd saves the composed route's
 * tensors; philtorch/lpv/ssm.py:337-581).  phs_lpv_ss_fwd_hs: phs_lpv_ss_fwd
 * (reverse = 0) or phs_lpv_ss_rev (reverse = 1) that also writes hs [B,T,M],
 * the state before every step, in the same pass.  phs_lpv_ss_bwd_hs:
 * phs_lpv_ss_bwd given those states (the same model's, same reverse), so it
 * runs the adjoint pass only; hs NULL: it recomputes them, as
 * phs_lpv_ss_bwd.  Results equal phs_lpv_ss_bwd's bit for bit. */
int phs_lpv_ss_fwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                      int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride,
                      int64_t c_t_stride, int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride,
                      const void *zi, const void *x, void *y, void *zf, void *hs, int reverse, void *workspace,
                      size_t workspace_bytes, void *stream);

int phs_lpv_ss_bwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                      int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride,
                      int64_t c_t_stride, int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride,
                      const void *zi, const void *x, const void *hs, const void *gy, const void *gzf, void *gx,
                      void *gzi, void *gA, void *gb, void *gc, void *gd, int reverse, void *scratch,
                      size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream);

/* Bits of the `shared` argument of phs_mimo_ss_fwd / phs_mimo_ss_rev: an
 * operand with its bit set is one matrix for every row (else one per row). */
#define PHS_MIMO_A_SHARED 1
#define PHS_MIMO_B_SHARED 2
#define PHS_MIMO_C_SHARED 4
#define PHS_MIMO_D_SHARED 8
/* Bits of phs_mimo_ss_grad_sums' `shared` only: gA receives lam[t] h[t]^T
 * per step, [B,T,M,M], instead of its sum (the gradient of a time-varying
 * A[t], phs_lpv_mimo_ss); with PHS_MIMO_A_STEPS_T too, its transpose h[t]
 * lam[t]^T (the gradient of the A[t] a PHS_LPV_A_TRANSPOSED pass read).
 * Not with PHS_MIMO_A_SHARED. */
#define PHS_MIMO_A_STEPS 16
#define PHS_MIMO_A_STEPS_T 32

/* ---- Multi-input, multi-output LTI state space of order M = 1..4 with
 * F = 1..4 inputs and P = 1..4 outputs per step, fused (forward).  Replaces
 * philtorch.lti.state_space (philtorch/lti/ssm.py:386-589) for a 3D input
 * x (batch, time, features) or matrix-valued B, C, D: the composed route's
 * B x (:460-485), recurrence (_ext_ss_recur, :487-491), state shift
 * (:493-504) and _ssm_C_D (:506, :513-589) in one pass:
 *     h[0] = zi,  y[t] = C h[t] + D x[t],  h[t+1] = A h[t] + B x[t],  zf = h[T]
 * dtype PHS_F32 or PHS_F64; A [B,M,M], Bm [B,M,F], Cm [B,P,M], Dm [B,P,F]
 * (row-major; an operand with its PHS_MIMO_*_SHARED bit in `shared` is one
 * matrix, without the row axis); Dm NULL: no feedthrough; zi [B,M] (NULL =
 * zeros); x [B,T,F] and y [B,T,P], features innermost; zf [B,M] (skipped
 * when NULL; zi when T = 0).  `workspace`: phs_mimo_ss_workspace_size
 * bytes, under the conventions above. */
size_t phs_mimo_ss_workspace_size(int dtype, int M, int64_t B, int64_t T);

int phs_mimo_ss_fwd(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, const void *Bm,
                    const void *Cm, const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf,
                    void *workspace, size_t workspace_bytes, void *stream);

/* The same model run backwards in time (no counterpart in the reference,
 * which flips): h[T] = zi, y[t] = C h[t+1] + D x[t], h[t] = A h[t+1] +
 * B x[t], zf = h[0].  The adjoint of the forward model is this one on
 * (A^T, C^T, B^T, D^T) from dL/dzf: y = grad_x, zf = grad_zi; with C the
 * identity and no D, y[t] is the adjoint state dL/dh[t+1] that the
 * coefficient gradients sum against (dL/dA = sum lambda[t+1] h[t]^T,
 * dL/dB = sum lambda[t+1] x[t]^T). */
int phs_mimo_ss_rev(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, const void *Bm,
                    const void *Cm, const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf,
                    void *workspace, size_t workspace_bytes, void *stream);

/* ---- Multi-input, multi-output LPV (time-varying A) state space of order
 * M = 1..4 with F = 1..4 inputs and P = 1..4 outputs per step, fused.
 * Replaces philtorch.lpv.state_space (philtorch/lpv/ssm.py:337-581) for a
 * 3D x or matrix-valued B, C, D constant in time: the composed route's B x
 * (:413-454), the LPV scan (_ext_ss_recur), the state shift (:462-474) and
 * C h + D x (:480-577) in one pass:
 *     h[0] = zi,  y[t] = C h[t] + D x[t],  h[t+1] = A[t] h[t] + B x[t],  zf = h[T]
 * A [B,T,M,M], or [T,M,M] with PHS_LPV_A_SHARED in A_flags
 * (PHS_LPV_A_TRANSPOSED: use A[t]^T); Bm [B,M,F], Cm [B,P,M], Dm [B,P,F]
 * with their PHS_MIMO_{B,C,D}_SHARED bits in `shared` (one matrix, no row
 * axis); Dm NULL: no feedthrough; zi [B,M] (NULL = zeros); x [B,T,F], y
 * [B,T,P]; zf [B,M] (skipped when NULL; zi when T = 0).  reverse != 0 runs
 * the model backwards in time (no counterpart in the reference, which
 * flips): h[T] = zi, y[t] = C h[t+1] + D x[t], h[t] = A[t] h[t+1] + B x[t],
 * zf = h[0]; on the adjoint model (A[t]^T, C^T, B^T, D^T) from dL/dzf it
 * gives grad_x and grad_zi, and with C the identity the adjoint states.
 * `workspace`: phs_lpv_mimo_ss_workspace_size bytes, under the conventions
 * above. */
size_t phs_lpv_mimo_ss_workspace_size(int dtype, int M, int64_t B, int64_t T);

int phs_lpv_mimo_ss(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, int A_flags,
                    const void *Bm, const void *Cm, const void *Dm, int shared, const void *zi, const void *x,
                    void *y, void *zf, int reverse, void *workspace, size_t workspace_bytes, void *stream);

/* ---- phs_lpv_mimo_ss that also writes hs [B,T,M], the state before every
 * step, in the same pass (no counterpart in the reference, whose autograd
 * saves the composed route's tensors; philtorch/lpv/ssm.py:337-581): the
 * states the coefficient gradients read (phs_mimo_ss_grad_sums), so a
 * caller need not run the model again with C the identity.  Needs
 * P + M <= 4 (the states take output planes); y, zf as phs_lpv_mimo_ss's
 * bit for bit. */
int phs_lpv_mimo_ss_hs(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, int A_flags,
                       const void *Bm, const void *Cm, const void *Dm, int shared, const void *zi, const void *x,
                       void *y, void *zf, void *hs, int reverse, void *workspace, size_t workspace_bytes,
                       void *stream);

/* ---- The coefficient gradients of phs_mimo_ss_fwd summed over time in one
 * pass (no counterpart in the reference, whose autograd forms them as
 * matmuls over the composed route's tensors; philtorch/lti/ssm.py:460-589):
 *     gA = sum_t lam[t] h[t]^T (M x M),  gB = sum_t lam[t] x[t]^T (M x F),
 *     gC = sum_t g[t] h[t]^T (P x M),    gD = sum_t g[t] x[t]^T (P x F),
 * per row [B, ...], or with the operand's PHS_MIMO_*_SHARED bit in `shared`
 * summed over the rows too (no row axis).  lam [B,T,M] are the adjoint
 * states dL/dh[t+1] and h [B,T,M] the forward's states h[t] (both
 * phs_mimo_ss passes with C the identity), x [B,T,F] the input, g [B,T,P]
 * the upstream gradient; every output is nullable (not wanted), and an input
 * no wanted output reads may be NULL.  dtype PHS_F32 or PHS_F64, sums in
 * fp64.  PHS_MIMO_A_STEPS in `shared`: gA is the per-step product instead
 * (each element rounded once from the exact product, as an fp32 or fp64
 * multiply gives it).  gx (nullable) [B,T,F]: the input's gradient
 * gx[t] = Bm^T lam[t] + Dm^T g[t] per step, from the model's Bm [B,M,F] and
 * Dm [B,P,F] (NULL: no feedthrough), each one matrix with its
 * PHS_MIMO_{B,D}_SHARED bit, summed in fp64 and rounded once: the adjoint
 * pass that gives lam would give it with output matrix Bm^T, so one pass
 * serves both.  `scratch`: phs_mimo_ss_grad_sums_scratch_size bytes, any
 * contents. */
size_t phs_mimo_ss_grad_sums_scratch_size(int dtype, int64_t B, int64_t T);

int phs_mimo_ss_grad_sums(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *lam, const void *hs,
                          const void *x, const void *g, const void *Bm, const void *Dm, int shared, void *gA,
                          void *gB, void *gC, void *gD, void *gx, void *scratch, size_t scratch_bytes, void *stream);

/* ---- Measurement helper, no counterpart in the reference.  A streaming
 * kernel with no scan: out_j[i] = (j + 1) * sum_k in_k[i] over n fp32
 * elements, n_in = 1..3 input arrays and n_out = 1..2 output arrays (16-byte
 * aligned; n a multiple of 8192).  It moves the bytes of a scan launch with
 * nothing else to do, so its duration is the achievable floor for that
 * traffic (the forward scalar scan reads 2 arrays and writes 1, its
 * backward reads 3 and writes 2).  shape 0: the fp32 scalar scan's tile
 * geometry (8 waves, two rounds of 8 floats per lane and array, 8192
 * elements per workgroup); shape 1: one float4 per lane and array, 2048
 * elements per workgroup; shape 2: shape 0's grid with no memory access
 * (launch and drain only). */
int phs_stream_probe(int shape, int n_in, int n_out, int64_t n, const void *const *in, void *const *out,
                     void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PHILSCAN_H_ */
