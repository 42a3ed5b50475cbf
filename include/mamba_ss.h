/*
 * mamba_ss.h -- C ABI of the MI355X selective-scan library (libmamba_ss.so).
 *
 * Replaces the reference's native module `selective_scan`
 * (csrc/selective_scan/selective_scan.cpp:331-334, built by setup.py:10-16):
 *   selective_scan.forward(u, delta, A, B, C, D?, delta_bias?, softplus)
 *       -> [out, x]                          selective_scan.cpp:184-244
 *   selective_scan.backward(u, delta, A, B, C, D?, delta_bias?, dout, x?, softplus)
 *       -> [du, ddelta, dA, dB, dC, dD, ddelta_bias]   selective_scan.cpp:246-329
 *
 * Differences from the pybind boundary, all deliberate:
 *  - plain C: POD argument structs, raw device pointers, 64-bit sizes and
 *    element strides; no torch types and no C++ exceptions cross the ABI;
 *  - the library never allocates: the caller passes every output, the
 *    checkpoint buffer x and the gradient accumulators (dA, dB, dC, dD,
 *    ddelta_bias are accumulated into, or cleared first with zero_grads);
 *  - errors are returned as status codes, with a message in
 *    ss_last_error() (the reference has no argument checks at all);
 *  - an optional fused z gate (out = y * silu(z)) and bf16/fp16 I/O, which
 *    the reference kernels do not have (they are fp32-only).
 *
 * Layouts: u, delta, z, out, dout, du, ddelta, dz are (batch, dim, seqlen)
 * with unit stride along seqlen; A is (dim, dstate) fp32; variable B/C are
 * (batch, n_groups, dstate, seqlen) with unit stride along seqlen; constant
 * B/C are (dim, dstate) fp32; D and delta_bias are (dim) fp32 contiguous.
 * x is fp32 (batch, n_chunks, dim, dstate) contiguous: the state h at the
 * end of every chunk of ss_chunk_size() steps (the last chunk holds the
 * final state).  It plays the role of the reference's x
 * (selective_scan.cpp:207-212) and is consumed only by ss_bwd.
 *
 * All calls are asynchronous on `stream` (a hipStream_t, NULL = default
 * stream) and re-entrant: no global mutable state besides the thread-local
 * error message, except ss_bwd_noalloc, whose calls share one fixed scratch
 * buffer per GPU (see there).
 */
#ifndef MAMBA_SS_H
#define MAMBA_SS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_ABI_VERSION 16

/* element types of u / delta / z / out / dout / du / ddelta / dz / variable B, C */
enum ss_dtype { SS_F32 = 0, SS_BF16 = 1, SS_F16 = 2 };

/* status codes */
enum ss_status {
    SS_OK = 0,
    SS_ERR_INVALID = 1,     /* bad argument: shape, stride, null pointer, dtype */
    SS_ERR_UNSUPPORTED = 2, /* valid but outside what the kernels implement */
    SS_ERR_HIP = 3          /* a HIP runtime / launch error */
};

typedef struct ss_fwd_args {
    int64_t batch, dim, seqlen, dstate, n_groups;
    int32_t itype;           /* enum ss_dtype */
    int32_t is_var_B, is_var_C;
    int32_t has_D, has_delta_bias, has_z;
    int32_t delta_softplus;
    int64_t n_chunks;        /* must equal ceil(seqlen / ss_chunk_size()) */
    /* element strides (batch, dim) of the (batch, dim, seqlen) tensors */
    int64_t u_batch_stride, u_dim_stride;
    int64_t delta_batch_stride, delta_dim_stride;
    int64_t z_batch_stride, z_dim_stride;
    int64_t out_batch_stride, out_dim_stride;
    /* A (dim, dstate) */
    int64_t A_dim_stride, A_dstate_stride;
    /* variable B/C: (batch, group, dstate) strides; constant: (dim, dstate) in
       (*_group_stride := dim stride, *_dstate_stride) and *_batch_stride = 0 */
    int64_t B_batch_stride, B_group_stride, B_dstate_stride;
    int64_t C_batch_stride, C_group_stride, C_dstate_stride;
    const void* u;
    const void* delta;
    const float* A;
    const void* B;
    const void* C;
    const float* D;          /* may be NULL iff !has_D */
    const float* delta_bias; /* may be NULL iff !has_delta_bias */
    const void* z;           /* may be NULL iff !has_z */
    void* out;
    /* checkpoints for the backward.  Required by ss_bwd; ss_fwd may be given
       NULL (a forward that no backward follows): no checkpoints are written. */
    float* x;
    /* pre-gate output y = sum_n C h + D u, same layout as out.  Written by
       ss_fwd when has_z and y != NULL; required (read) by ss_bwd when has_z. */
    void* y;
    int64_t y_batch_stride, y_dim_stride;
    /* ss_fwd only, may be NULL: fp32 (batch, dim, dstate) contiguous, receives
       the state h after the last step (what decoding continues from). */
    float* last_state;
    /* ss_fwd only, optional device scratch of ss_fwd_workspace_bytes() bytes,
       16-byte aligned.  With it, a forward with too few (batch, channel)
       rows to fill the GPU (small batch, long sequence) scans segments of
       the sequence in parallel and joins them, and a dstate of 16 S (32,
       48, ..., 256; variable B and C) runs the dstate-16 fast kernels once
       per 16-state slice, carrying y from slice to slice in an fp32
       accumulator of batch x dim x seqlen floats (ABI v16); NULL (or less
       than that) gives the serial scan and, for dstate 16 S, the general
       kernels.  Results agree to rounding.  Calls that overlap must not
       share it. */
    void* workspace;
    int64_t workspace_bytes;
    /* 0, or at most 2^31: the byte span of x that one buffer resource of the
       fast kernels addresses (ABI v16).  The kernels address the checkpoints
       of a batch row through a resource based at a window of chunks whose
       offsets stay below this span, and rebase it when a chunk leaves the
       window; 0 means 2^31, where rows below 2^31 bytes of checkpoints
       (seqlen x dim below 2^25) use one window.  Results do not depend on
       it: a smaller span only rebases more often (at least one chunk, or one
       64-step super-chunk in the forward, per window).  For tests of the
       rebasing. */
    int64_t x_window_bytes;
} ss_fwd_args;

typedef struct ss_bwd_args {
    ss_fwd_args f;           /* inputs as for the forward; f.out is ignored, f.x is read */
    int64_t dout_batch_stride, dout_dim_stride;
    int64_t du_batch_stride, du_dim_stride;
    int64_t ddelta_batch_stride, ddelta_dim_stride;
    int64_t dz_batch_stride, dz_dim_stride;
    const void* dout;
    void* du;                /* overwritten, itype */
    void* ddelta;            /* overwritten, itype */
    void* dz;                /* overwritten, itype; may be NULL iff !has_z */
    float* dA;               /* accumulated into (see zero_grads), (dim, dstate) contiguous */
    float* dB;               /* accumulated into, fp32, shape of B, contiguous */
    float* dC;               /* accumulated into, fp32, shape of C, contiguous */
    float* dD;               /* accumulated into; may be NULL iff !has_D */
    float* ddelta_bias;      /* accumulated into; may be NULL iff !has_delta_bias */
    /* optional device scratch of at least ss_bwd_workspace_bytes() bytes,
       16-byte aligned, contents ignored (the call clears what it uses).  With
       it, the dB / dC sums over channels are spread over several copies and
       added up at the end, instead of every channel block adding into the
       same dB / dC addresses; for a dstate of 16 S (32, 48, ..., 256; variable
       B and C) it also holds two fp32 accumulators of
       batch x dim x seqlen floats, with which the backward runs the dstate-16
       fast kernel once per 16-state slice (ABI v16).  NULL (or less than
       ss_bwd_workspace_bytes()) gives the same results, more slowly when many
       channel blocks share a group, and on the general kernels for dstate
       16 S.  Calls that overlap in time must not share a workspace. */
    void* workspace;
    int64_t workspace_bytes;
    /* nonzero: dA, dB, dC, dD and ddelta_bias are cleared by the call before
       it accumulates (their contents on entry are ignored), as the
       reference's backward zero-initialises them (selective_scan.cpp:274-287);
       the clearing shares a launch with the workspace's.  0: accumulate into
       what the caller passes. */
    int32_t zero_grads;
    /* nonzero: deterministic sums (ABI v12).  dB and dC are summed over the
       channels, and dA, dD and ddelta_bias over batch rows and sequence
       segments, in a fixed order instead of by atomic adds, so repeated calls
       on the same inputs give the same bits.  Needs the fast kernels (dstate
       16, or 16 S as one pass per 16-state slice; variable B and C, dim and
       channels per group multiples of 16; SS_ERR_UNSUPPORTED otherwise) and
       a workspace of ss_bwd_workspace_bytes() bytes (one dB / dC partial per
       16-channel block: batch * dim / 8 * 16 * seqlen floats, seqlen rounded
       up to a multiple of 32, plus the accumulators of the 16 S passes).
       No counterpart in the reference, whose sums are
       atomic (backward_kernel.cu:472-475,553-578). */
    int32_t deterministic;
} ss_bwd_args;

/* ABI version (SS_ABI_VERSION of the built library). */
int ss_abi_version(void);

/* Steps per checkpoint chunk of x (the reference's chunk is 128,
   kernel_config.cuh:3-7). */
int64_t ss_chunk_size(void);

/* Largest dstate the kernels accept (the reference dispatches up to 256,
   static_switch.h:15-37). */
int64_t ss_max_dstate(void);

/* sizeof(ss_fwd_args) and sizeof(ss_bwd_args) of the built library, so a
   foreign-function binding can check its struct layout.  Either pointer may
   be NULL. */
void ss_struct_sizes(int64_t* fwd_args, int64_t* bwd_args);

/* Message for the last failing call on this thread ("" if none). */
const char* ss_last_error(void);

/* Argument checks only, no device work: SS_OK or an error code. */
int ss_fwd_check(const ss_fwd_args* a);
int ss_bwd_check(const ss_bwd_args* a);

/* Bytes of workspace ss_bwd can use for these arguments (0: none), or -1
   (with ss_last_error set) when the arguments fail the checks.  No device
   work.  The reference needs none: its backward adds every channel's dB / dC
   into the output directly (backward_kernel.cu:457-479). */
int64_t ss_bwd_workspace_bytes(const ss_bwd_args* a);

/* Bytes of workspace ss_fwd can use for these arguments (0: none), or -1
   (with ss_last_error set) when the arguments fail the checks.  No device
   work.  No counterpart in the reference, whose forward has one block per
   (batch, channel) row and no sequence parallelism. */
int64_t ss_fwd_workspace_bytes(const ss_fwd_args* a);

/* Base name of the kernel that ss_fwd / ss_bwd would launch for these
   arguments, given the workspace that ss_fwd_workspace_bytes /
   ss_bwd_workspace_bytes ask for ("ss_fwd_fast", "ss_fwd_kernel",
   "ss_bwd_fast", "ss_bwd_kernel"; for dstate 16 S the fast kernel runs once
   per 16-state slice), "" when there is no work, NULL (with ss_last_error
   set) when the arguments fail the checks.  No device work; for profiling
   and tests.  No counterpart in the reference, which has one kernel per
   direction. */
const char* ss_fwd_kernel_name(const ss_fwd_args* a);
const char* ss_bwd_kernel_name(const ss_bwd_args* a);

/* Forward scan: writes out and x.  Replaces selective_scan.forward /
   forward_kernel_launch (selective_scan.cpp:184-244, forward_kernel.cu:313-333). */
int ss_fwd(const ss_fwd_args* a, void* stream);

/* Backward scan: writes du, ddelta, dz; accumulates dA, dB, dC, dD,
   ddelta_bias (after clearing them when zero_grads is set).  Replaces selective_scan.backward / backward_kernel_launch
   (selective_scan.cpp:246-329, backward_kernel.cu:588-618). */
int ss_bwd(const ss_bwd_args* a, void* stream);

/* ss_bwd that allocates nothing and needs no workspace from the caller.  No
   counterpart in the reference: it is for callers that cannot allocate
   device memory (code under HIP graph capture, tight serving or training
   loops, harnesses that forbid hipMalloc).  Same arguments, kernels and
   results as ss_bwd; a->workspace and a->workspace_bytes are ignored.  The
   scratch that ss_bwd would take from a workspace (dB / dC slices, sequence
   segment carries, the accumulators of dstate 16 S) comes from a fixed
   device buffer of SS_NOALLOC_SCRATCH_BYTES bytes inside the library, one
   per GPU, held until the process ends.  A dstate of 16 S whose passes need
   more runs as one pass on the general kernel, as ss_bwd without a
   workspace; other arguments that need more (ss_bwd_workspace_bytes) are
   rejected with SS_ERR_UNSUPPORTED.  Every call on a GPU shares that GPU's
   buffer, and each call clears what it uses: calls that overlap in time on
   one GPU (several streams or threads) race and must be serialised by the
   caller. */
#define SS_NOALLOC_SCRATCH_BYTES (32ll << 20)
int ss_bwd_noalloc(const ss_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Causal depthwise conv1d (+ SiLU), the step before the scan in the Mamba
 * block.  Replaces nn.Conv1d(dim, dim, width, groups=dim, padding=width - 1)
 * cut to the first seqlen outputs, and the SiLU after it
 * (modules/mamba_simple.py:40-47,100-101):
 *   out[b, d, t] = act(bias[d] + sum_k weight[d, k] * x[b, d, t - (width - 1) + k])
 * with x = 0 before t = 0 and act = SiLU or identity.
 * x, out, dout, dx: (batch, dim, seqlen), seqlen stride 1, element type
 * itype; weight: fp32 (dim, width) with free strides; bias: fp32 (dim).
 * ------------------------------------------------------------------------ */
typedef struct ss_conv1d_args {
    int64_t batch, dim, seqlen, width;   /* width 1..4 */
    int32_t itype;                       /* enum ss_dtype */
    int32_t has_bias, silu;
    int32_t pad_;
    int64_t x_batch_stride, x_dim_stride;
    int64_t out_batch_stride, out_dim_stride;
    int64_t w_dim_stride, w_width_stride;
    const void* x;
    const float* weight;
    const float* bias;                   /* may be NULL iff !has_bias */
    void* out;                           /* ignored by ss_conv1d_bwd */
} ss_conv1d_args;

typedef struct ss_conv1d_bwd_args {
    ss_conv1d_args f;                    /* as for the forward (f.out ignored) */
    int64_t dout_batch_stride, dout_dim_stride;
    int64_t dx_batch_stride, dx_dim_stride;
    const void* dout;                    /* gradient of out (after the activation) */
    void* dx;                            /* overwritten, itype */
    float* dweight;                      /* accumulated into, fp32 (dim, width) contiguous */
    float* dbias;                        /* accumulated into, fp32 (dim); may be NULL iff !has_bias */
    /* ABI v15: with a workspace (NULL: none) of at least
     * ss_conv1d_bwd_workspace_bytes bytes, dweight / dbias are summed in a
     * fixed order (per-workgroup partials, then a second launch adds them per
     * channel in (batch, sequence tile) order): the same bits on every run.
     * Without it each workgroup adds its partial with fp32 atomics. */
    float* workspace;
    int64_t workspace_bytes;
} ss_conv1d_bwd_args;

/* Forward: writes out.  Backward: writes dx, accumulates dweight / dbias;
   recomputes the pre-activation from x, weight and bias. */
int ss_conv1d_fwd(const ss_conv1d_args* a, void* stream);
int ss_conv1d_bwd(const ss_conv1d_bwd_args* a, void* stream);
/* Workspace bytes of the fixed-order backward sums for these sizes (batch x
 * dim x sequence tiles x 5 floats); -1 on invalid sizes. */
int64_t ss_conv1d_bwd_workspace_bytes(const ss_conv1d_bwd_args* a);

/* ------------------------------------------------------------------------
 * RMSNorm with an optional residual add, on rows of dim elements.  Replaces
 * RMSNorm.forward (modules/rms_norm.py:19,29-31) and the residual add that
 * ends each block (models/causal_lm.py:31-35), fused:
 *   s    = x + residual, rounded to dtype        (s = x without residual)
 *   out  = s * rsqrt(mean(s^2) + eps) * (1 + weight), in fp32, rounded to dtype
 * x, residual, out, residual_out, dout, dresidual_out, dx: (rows, dim) with
 * unit column stride and free row strides, element type dtype; weight and
 * dweight: (dim) contiguous, w_dtype = dtype or SS_F32; rstd: fp32 (rows).
 * ------------------------------------------------------------------------ */
typedef struct ss_rmsnorm_args {
    int64_t rows, dim;
    int32_t dtype;                       /* enum ss_dtype */
    int32_t w_dtype;                     /* enum ss_dtype: dtype or SS_F32 */
    float eps;
    int32_t pad_;
    int64_t x_row_stride, residual_row_stride, out_row_stride, residual_out_row_stride;
    const void* x;
    const void* residual;                /* may be NULL: s = x */
    const void* weight;
    void* out;
    void* residual_out;                  /* s; may be NULL (not written); ignored without residual */
    float* rstd;                         /* may be NULL (not written); kept for the backward */
} ss_rmsnorm_args;

typedef struct ss_rmsnorm_bwd_args {
    int64_t rows, dim;
    int32_t dtype, w_dtype;
    int64_t s_row_stride, dout_row_stride, dresidual_out_row_stride, dx_row_stride;
    const void* s;                       /* the normalised rows: residual_out, or x without residual */
    const void* weight;
    const float* rstd;                   /* from the forward */
    const void* dout;
    const void* dresidual_out;           /* may be NULL: gradient arriving at residual_out */
    void* dx;                            /* written: gradient of s (= of x and of residual) */
    void* dweight;                       /* written (not accumulated), w_dtype */
    void* workspace;                     /* ss_rmsnorm_bwd_workspace_bytes(rows, dim) bytes */
    int64_t workspace_bytes;
} ss_rmsnorm_bwd_args;

/* Forward: writes out, residual_out and rstd.  Backward: writes dx and
   dweight; dweight is summed in a fixed order (the same bits every run). */
int ss_rmsnorm_fwd(const ss_rmsnorm_args* a, void* stream);
int ss_rmsnorm_bwd(const ss_rmsnorm_bwd_args* a, void* stream);
int64_t ss_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t dim);

/* ------------------------------------------------------------------------
 * Single-token decode.  The reference has no decode path (CausalLM.generate
 * is a stub, models/causal_lm.py:61-62); these advance, by one token, the
 * recurrences that ss_fwd (forward_kernel.cu:216-293) and the block's conv
 * (modules/mamba_simple.py:40-47,100-101) compute over a sequence, from a
 * state the caller keeps between tokens.
 *
 * ss_state_update, per (batch b, channel d), group g = d / (dim / n_groups):
 *   dt = delta[b, d] (+ delta_bias[d]), softplus if delta_softplus
 *   state[b, d, n] <- exp(dt * A[d, n]) * state[b, d, n] + dt * x[b, d] * B[b, g, n]
 *   out[b, d] = sum_n C[b, g, n] * state[b, d, n] (+ D[d] * x[b, d]) (* silu(z[b, d]))
 * state: fp32 (batch, dim, dstate), updated in place; x, delta, z, out:
 * (batch, dim); B, C: (batch, n_groups, dstate), element type itype; A:
 * fp32 (dim, dstate); D, delta_bias: fp32 (dim).  All strides free.
 * ------------------------------------------------------------------------ */
typedef struct ss_state_update_args {
    int64_t batch, dim, dstate, n_groups;
    int32_t itype;                       /* enum ss_dtype */
    int32_t has_D, has_z, has_delta_bias, delta_softplus;
    int32_t pad_;
    int64_t state_batch_stride, state_dim_stride, state_dstate_stride;
    int64_t x_batch_stride, x_dim_stride;
    int64_t delta_batch_stride, delta_dim_stride;
    int64_t z_batch_stride, z_dim_stride;
    int64_t out_batch_stride, out_dim_stride;
    int64_t A_dim_stride, A_dstate_stride;
    int64_t B_batch_stride, B_group_stride, B_dstate_stride;
    int64_t C_batch_stride, C_group_stride, C_dstate_stride;
    float* state;
    const void* x;
    const void* delta;
    const float* A;
    const void* B;
    const void* C;
    const float* D;                      /* may be NULL iff !has_D */
    const void* z;                       /* may be NULL iff !has_z */
    const float* delta_bias;             /* may be NULL iff !has_delta_bias */
    void* out;
    /* ABI v10: when delta_low is not NULL, delta is the low-rank product
     *   delta[b, d] = sum_r delta_low[b, r] * delta_weight[d, r]
     * (the block's delta projection, summed in fp32 inside the kernel and
     * rounded once to itype, as that projection's output is in the forward)
     * and the delta pointer and strides are ignored; delta_low (batch,
     * delta_rank) and delta_weight (dim, delta_rank) in itype. */
    int64_t delta_rank;
    int64_t delta_low_batch_stride, delta_low_rank_stride;
    int64_t delta_weight_dim_stride, delta_weight_rank_stride;
    const void* delta_low;
    const void* delta_weight;
} ss_state_update_args;

/* ss_conv1d_update, per (batch b, channel d), state = the last width inputs:
 *   conv_state[b, d, :] <- (conv_state[b, d, 1:], x[b, d])
 *   out[b, d] = act(bias[d] + sum_k weight[d, k] * conv_state[b, d, k])
 * x, out: (batch, dim); conv_state: (batch, dim, width), element type itype,
 * updated in place; weight fp32 (dim, width); bias fp32 (dim).  Strides free. */
typedef struct ss_conv1d_update_args {
    int64_t batch, dim, width;           /* width 1..4 */
    int32_t itype;                       /* enum ss_dtype */
    int32_t has_bias, silu;
    int32_t pad_;
    int64_t x_batch_stride, x_dim_stride;
    int64_t out_batch_stride, out_dim_stride;
    int64_t state_batch_stride, state_dim_stride, state_width_stride;
    int64_t w_dim_stride, w_width_stride;
    const void* x;
    void* conv_state;
    const float* weight;
    const float* bias;                   /* may be NULL iff !has_bias */
    void* out;
} ss_conv1d_update_args;

int ss_state_update(const ss_state_update_args* a, void* stream);
int ss_conv1d_update(const ss_conv1d_update_args* a, void* stream);

/* Decode-size linear layer on the matrix cores, nn.Linear's layout:
 *   y[b, n] = sum_k x[b, k] * weight[n, k] (+ bias[n])
 * for the few rows of a single-token step (the block's projections).  x, y:
 * (batch, n_out / k_in) rows; weight: (n_out, k_in) rows; unit column
 * strides, row strides multiples of 4 elements, 8-byte aligned bases; k_in a
 * multiple of 16; dtype bf16 or fp16; bias of that dtype or fp32.  No
 * counterpart in the reference (it has no decode path).
 *
 * ABI v13 adds two optional parts:
 * - workspace: with it the library may split K over several workgroups per
 *   16 x 16 output tile (a decode product streams the weight with only a few
 *   tiles, and each compute unit fetches a bounded number of cache lines at
 *   once); the last workgroup of a tile to finish sums the fp32 partial
 *   tiles in a fixed order, so results do not depend on timing.  Size from
 *   ss_decode_linear_workspace_bytes (0: no split for this shape, the
 *   workspace is not used).  The caller zeroes it once before its first
 *   use; every call leaves it ready for the next one (its tile counters back
 *   at zero), whatever the shape, so calls of different shapes can share
 *   one.  Calls that share a workspace must not run at the same time.
 * - conv: outputs n < conv->dim then pass through the causal conv1d update
 *   that ss_conv1d_update describes for x = the product (+ bias) rounded to
 *   dtype (conv->x and conv->out are ignored; the conv output is written to
 *   y[b, n], the conv state is advanced in place); outputs n >= conv->dim
 *   are written as they are.  This is the block's input projection followed
 *   by its conv step in one launch.  conv->itype must equal dtype,
 *   conv->batch equal batch, conv->dim <= n_out.
 *
 * ABI v14 adds norm: when it is not NULL the product's input rows are
 * norm's output, computed in the same launch as ss_rmsnorm_fwd computes it
 * (the same bits): x = rmsnorm(norm->x + norm->residual); norm->residual_out
 * and norm->rstd are written as ss_rmsnorm_fwd writes them, norm->out is
 * ignored, and the x / x_row_stride fields of this block are not used.  This
 * is the block's RMSNorm and input projection in one launch.  norm->rows
 * must equal batch, norm->dim equal k_in (at most 1024), norm->dtype equal
 * dtype; norm->x, residual and residual_out need 16-byte aligned rows
 * (bases and row strides), weight 16-byte alignment.  The K split is not
 * used with it.  Every output tile's workgroup reads norm->x and
 * norm->residual while the first one writes residual_out, so residual_out
 * must not overlap either (no in-place residual stream: SS_ERR_INVALID).
 * In every form, y must not overlap the input rows (x, or norm's x,
 * residual and residual_out): SS_ERR_INVALID. */
typedef struct ss_decode_linear_args {
    int64_t batch, n_out, k_in;
    int32_t dtype;                       /* SS_BF16 or SS_F16: x, weight, y */
    int32_t bias_dtype;                  /* dtype or SS_F32 (ignored without bias) */
    int64_t x_row_stride, w_row_stride, y_row_stride;
    const void* x;
    const void* weight;
    const void* bias;                    /* may be NULL */
    void* y;
    void* workspace;                     /* may be NULL (ABI v13) */
    int64_t workspace_bytes;
    const ss_conv1d_update_args* conv;   /* may be NULL (ABI v13) */
    const ss_rmsnorm_args* norm;         /* may be NULL (ABI v14) */
} ss_decode_linear_args;

/* Workspace bytes ss_decode_linear can use for this shape (0: none); -1 on
 * invalid sizes (see ss_last_error).  Depends on batch, n_out and k_in only. */
int64_t ss_decode_linear_workspace_bytes(const ss_decode_linear_args* a);
int ss_decode_linear(const ss_decode_linear_args* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_SS_H */
