// Kernel-side argument blocks and launcher declarations (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/mamba_ss.h"

namespace ss {

struct FwdParams {
    int64_t batch, dim, seqlen, dstate, dpg;  // dpg: channels per group
    int64_t n_chunks;
    int32_t var_B, var_C, has_z, softplus;
    int32_t vec_B, vec_C;                     // 16-byte aligned rows of variable B / C (general kernels)
    int32_t store_nt;                         // out / y rows all 16-byte aligned: non-temporal stores (fast forward)
    int64_t u_bs, u_ds, dl_bs, dl_ds, z_bs, z_ds, o_bs, o_ds, y_bs, y_ds;
    int64_t A_ds, A_ns;
    int64_t B_bs, B_gs, B_ns, C_bs, C_gs, C_ns;
    const void* u; const void* delta; const float* A; const void* B; const void* C;
    const float* D; const float* delta_bias; const void* z;
    void* out; float* x;
    void* y;                                  // pre-gate output (z gate only); may be null in forward
    float* last_state;                        // forward: h after the last step, (batch, dim, dstate); may be null
    // bytes from each array's base pointer to the end of its last element (0
    // for an absent array): the fast kernels' buffer resources end there, so
    // the hardware's range check drops any access past an array, and every
    // store to an absent optional output (x, y: a forward that no backward
    // follows writes neither)
    int64_t u_end, dl_end, z_end, o_end, y_end, B_end, C_end, x_end;
    // byte span of x one checkpoint resource of the fast kernels addresses
    // (at most 2^31, so the offsets inside it stay below 2^31)
    int64_t x_win;
    // states per channel of x and last_state (the call's dstate): the fast
    // kernels scan 16 states; for dstate 16 S they run once per 16-state
    // slice, with x, last_state, A, B and C based at the slice
    int64_t xN;
    // state slices (fast kernels, S > 1): the sums over states that the
    // slices share, accumulated in fp32 from pass to pass.  Forward: y
    // (batch, dim, seqlen); backward: sum_n g B, then sum_n A g a h (two such
    // arrays).  The extents are 0 where a pass does not read (the first) or
    // write (the last) them.
    float* acc;
    int64_t acc_in_end, acc_out_end;
    // sequence-parallel scan (fast paths): the sequence is cut into nseg
    // equal segments handled by separate workgroups; seg_h (batch, nseg,
    // dim, 16) holds each segment's end state (forward) or adjoint carry
    // (backward) from a zero start and seg_s (batch, nseg, dim) its sum of
    // delta' (nseg 1: the serial scan)
    int32_t nseg;
    float* seg_h;
    float* seg_s;
};
// segments the forward uses for p (1: serial), and the workspace they need
int fwd_segments(const FwdParams& p);
// the fast forward applies to p
bool fwd_fast_ok(const FwdParams& p);
inline int64_t fwd_seg_bytes(const FwdParams& p, int nseg) {
    return nseg > 1 ? p.batch * nseg * p.dim * 17 * int64_t(sizeof(float)) : 0;
}

struct BwdParams {
    FwdParams f;
    int64_t do_bs, do_ds, du_bs, du_ds, dd_bs, dd_ds, dz_bs, dz_ds;
    const void* dout; void* du; void* ddelta; void* dz;
    float* dA; float* dB; float* dC; float* dD; float* ddelta_bias;
    // dB / dC slices: when ws is set, the workgroups of channel block k add
    // into slice k % ws_slices of ws (2 * ws_slices arrays of ws_stride
    // floats: dB, dC of slice 0, then of slice 1, ...), summed into dB / dC
    // by a separate pass.  Fewer workgroups per address, less contention.
    float* ws;
    int32_t ws_slices;
    int64_t ws_stride;
    // byte extents of dout, du, ddelta, dz, dB, dC and the slices of ws (as
    // FwdParams' *_end)
    int64_t do_end, du_end, dd_end, dz_end, dB_end, dC_end, ws_end;
    // row length (floats) of the dB / dC rows the fast kernel adds into:
    // seqlen for dB / dC themselves; in the workspace the rows are padded to
    // whole chunk pairs (a multiple of 32 steps), so that every row starts on
    // a 128-byte boundary and the steps of the identity-padded tail chunks
    // have slots of their own
    int64_t bc_ld;
    // clear dA, dB, dC, dD, ddelta_bias before accumulating (element counts
    // of each; dB / dC are overwritten by the slice sum when ws is used)
    int32_t zero_grads;
    int64_t dA_n, dB_n, dC_n, dD_n;
    // deterministic sums (fast kernels only): every channel block writes its
    // dB / dC partials into a slice of ws of its own (one slice per channel
    // block of a group, plain stores), and every (batch row, segment)
    // workgroup its dA, dD and ddelta_bias partials into det_par
    // ((batch * nseg) rows of dim * dstate + 2 * dim floats); fixed-order
    // passes sum both, so the results are the same bits on every run
    int32_t det;
    float* det_par;
    // state slices: row length of dA (the call's dstate) and state rows per
    // (batch, group) of the dB / dC rows the fast kernel adds into (dstate for
    // dB / dC themselves, 16 in the workspace's slices)
    int64_t dA_N, bc_N;
};
// state slices the fast kernels run in for p (dstate 16 S: S; 1 where they
// do not apply or dstate is 16)
int state_slices(const FwdParams& p);

// dB / dC slices the fast backward uses for p (1: add into dB / dC directly;
// with p.det one per channel block of a group)
int bwd_ws_slices(const BwdParams& p);
// row length of the workspace's dB / dC rows: seqlen rounded up to 32
inline int64_t bwd_ws_ld(int64_t seqlen) { return (seqlen + 31) / 32 * 32; }
// the fast backward applies to p (deterministic sums need it)
bool bwd_fast_ok(const BwdParams& p);
// sequence segments the fast backward uses for p (1: serial); its pass A
// writes each segment's adjoint carry to f.seg_h and its sum of delta' to
// f.seg_s (the forward's layout and sizes, fwd_seg_bytes)
int bwd_segments(const BwdParams& p);
// arrays one clearing launch handles (workspace + five accumulators)
constexpr int kZeroSegs = 6;
// clears the accumulators of p (zero_grads) and nothing else: a call with
// no scan work (batch or seqlen 0) still returns zeroed gradients
hipError_t launch_bwd_zero_only(const BwdParams& p, hipStream_t stream);

// The fast kernels address a workgroup's rows as a uniform base plus a 32-bit
// per-thread byte offset of at most 16 rows x stride x 4 bytes; strides and
// seqlen below 2^26 elements keep every such offset below 2^32.
constexpr int64_t kMaxOffStride = int64_t(1) << 26;
inline bool small_strides(std::initializer_list<int64_t> strides) {
    for (int64_t s : strides)
        if (s >= kMaxOffStride) return false;
    return true;
}

// Return hipSuccess or the launch error.
hipError_t launch_fwd(const FwdParams& p, int itype, hipStream_t stream);
hipError_t launch_bwd(const BwdParams& p, int itype, hipStream_t stream);
// causal depthwise conv1d (+ SiLU); g == nullptr: forward, else backward
hipError_t conv1d_launch(const ss_conv1d_args* a, const ss_conv1d_bwd_args* g, hipStream_t stream);
// Sequence segments of the fast scans.  A launch of wgs workgroups (batch x
// channel blocks) doubles its segment count while it has fewer than
// kSegSlots workgroups (three per CU), up to kSegMax segments of at least
// min_units units each (super-chunks forward, chunk pairs backward); 1 when
// the batch already fills the GPU.  Segment s covers units [seg_begin(s),
// seg_begin(s + 1)), so any unit count splits (lengths differ by at most
// one unit).  (Counts that fit every segment into one round, such as 6 at
// 128 workgroups, measured the same as the doubled 8.)
constexpr int64_t kSegSlots = 768;
constexpr int kSegMax = 64;
inline int seg_count(int64_t wgs, int64_t units, int min_units) {
    int n = 1;
    while (wgs * n < kSegSlots && 2 * n <= kSegMax && units / (2 * n) >= min_units) n *= 2;
    return n;
}
__host__ __device__ inline int seg_begin(int s, int units, int nseg) { return int(int64_t(s) * units / nseg); }

// bytes of the backward's fixed-order partials (batch x dim x tiles x 5 floats)
int64_t conv1d_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen);
// single-token decode: selective-scan state update and conv1d state update
hipError_t state_update_launch(const ss_state_update_args* a, hipStream_t stream);
hipError_t conv_update_launch(const ss_conv1d_update_args* a, hipStream_t stream);
// decode-size linear layer (matrix cores); K split over ksplit workgroups
// per output tile (slices of kslice elements) when a workspace of
// workspace_bytes is given (ksplit 1, workspace_bytes 0: no split)
struct DecodeLinearSplit {
    int64_t ksplit, kslice, workspace_bytes;
};
// only shapes with fewer output tiles than this are split (measured: the
// split pays for 5 tiles and loses at 192), into at most kLinMaxSplit
// slices (5 tiles: 4 slices 5.25 us, 8 slices 5.5, 16 slices 5.8)
constexpr int64_t kLinSplitMaxTiles = 64;
constexpr int64_t kLinMaxSplit = 4;
// the workspace starts with one int counter per tile of the largest split
// shape
constexpr int64_t kLinCounterBytes = 256;
static_assert(kLinSplitMaxTiles * 4 <= kLinCounterBytes, "counter region");
DecodeLinearSplit decode_linear_split(int64_t batch, int64_t n_out, int64_t k_in);
hipError_t decode_linear_launch(const ss_decode_linear_args* a, hipStream_t stream);
// RMSNorm (+ residual); g == nullptr: forward, else backward (two kernels:
// per-workgroup dweight rows into g->workspace, then their fixed-order sum)
hipError_t rmsnorm_launch(const ss_rmsnorm_args* a, const ss_rmsnorm_bwd_args* g, hipStream_t stream);
// backward workgroups (= fp32 dweight rows of workspace) for `rows` rows
int64_t rmsnorm_bwd_parts(int64_t rows);
constexpr int64_t kRmsNormMaxParts = 512;
// the backward keeps one fp32 column sum per element of a row in LDS
constexpr int64_t kRmsNormMaxBwdDim = 16384;
// base name of the kernel template launch_fwd / launch_bwd picks for p
const char* fwd_kernel_name(const FwdParams& p);
const char* bwd_kernel_name(const BwdParams& p);

}  // namespace ss
