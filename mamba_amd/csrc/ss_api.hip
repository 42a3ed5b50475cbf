// extern "C" entry points of libmamba_ss.so: argument checks and dispatch.
//
// The reference binding (csrc/selective_scan/selective_scan.cpp:184-329)
// checks nothing; here every call is validated first and failures come back
// as status codes with a thread-local message, never as exceptions.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return SS_OK;
}

size_t elem_size(int itype) { return itype == SS_F32 ? 4 : 2; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Whether the byte ranges of two row arrays overlap: `rows` rows of p_cols
// (q_cols) elements of es bytes, row strides in elements.  An absent array
// overlaps nothing.
bool rows_overlap(const void* p, int64_t p_stride, int64_t p_cols, const void* q, int64_t q_stride, int64_t q_cols,
                  int64_t rows, size_t es) {
    if (!p || !q || rows <= 0 || p_cols <= 0 || q_cols <= 0) return false;
    const uintptr_t p0 = reinterpret_cast<uintptr_t>(p), q0 = reinterpret_cast<uintptr_t>(q);
    const uintptr_t p1 = p0 + uintptr_t(((rows - 1) * p_stride + p_cols) * int64_t(es));
    const uintptr_t q1 = q0 + uintptr_t(((rows - 1) * q_stride + q_cols) * int64_t(es));
    return p0 < q1 && q0 < p1;
}

int64_t n_chunks_for(int64_t L) { return (L + ss::kChunk - 1) / ss::kChunk; }

// Checks common to forward and backward.  `empty` is set when there is no
// work (batch, dim or seqlen is 0); pointers are then not inspected.
int check_fwd_common(const ss_fwd_args* a, bool* empty) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
        return fail(SS_ERR_INVALID, "negative size (batch=%lld dim=%lld seqlen=%lld)",
                    (long long)a->batch, (long long)a->dim, (long long)a->seqlen);
    if (a->dstate < 1 || a->dstate > 16 * ss::kMaxSPL)
        return fail(SS_ERR_UNSUPPORTED, "dstate=%lld outside [1, %d]", (long long)a->dstate, 16 * ss::kMaxSPL);
    if (a->itype != SS_F32 && a->itype != SS_BF16 && a->itype != SS_F16)
        return fail(SS_ERR_INVALID, "unknown itype %d", a->itype);
    if (a->is_var_B || a->is_var_C) {
        if (a->n_groups < 1) return fail(SS_ERR_INVALID, "n_groups=%lld < 1", (long long)a->n_groups);
        if (a->dim % a->n_groups != 0)
            return fail(SS_ERR_INVALID, "dim=%lld is not a multiple of n_groups=%lld",
                        (long long)a->dim, (long long)a->n_groups);
    }
    if (a->x_window_bytes < 0 || a->x_window_bytes > (int64_t(1) << 31))
        return fail(SS_ERR_INVALID, "x_window_bytes=%lld outside [0, 2^31]", (long long)a->x_window_bytes);
    if (a->n_chunks != n_chunks_for(a->seqlen))
        return fail(SS_ERR_INVALID, "n_chunks=%lld, expected ceil(seqlen / %d) = %lld",
                    (long long)a->n_chunks, ss::kChunk, (long long)n_chunks_for(a->seqlen));
    const int64_t nblk = (a->dim + ss::kChPerWG - 1) / ss::kChPerWG;
    if (a->batch > 0 && nblk > (int64_t(INT32_MAX) / a->batch))
        return fail(SS_ERR_UNSUPPORTED, "grid of %lld x %lld workgroups is too large",
                    (long long)nblk, (long long)a->batch);
    *empty = a->batch == 0 || a->dim == 0 || a->seqlen == 0;
    if (*empty) return SS_OK;
    const size_t es = elem_size(a->itype);
    struct P { const void* p; const char* name; bool need; size_t align; };
    const P ptrs[] = {
        {a->u, "u", true, es}, {a->delta, "delta", true, es}, {a->A, "A", true, 4},
        {a->B, "B", true, a->is_var_B ? es : 4}, {a->C, "C", true, a->is_var_C ? es : 4},
        {a->D, "D", a->has_D != 0, 4}, {a->delta_bias, "delta_bias", a->has_delta_bias != 0, 4},
        {a->z, "z", a->has_z != 0, es}, {a->x, "x", false, 4}, {a->last_state, "last_state", false, 4},
    };
    for (const P& q : ptrs) {
        if (q.need && !q.p) return fail(SS_ERR_INVALID, "%s is NULL", q.name);
        if (q.p && !aligned(q.p, q.align)) return fail(SS_ERR_INVALID, "%s is misaligned", q.name);
    }
    const int64_t strides[] = {a->u_batch_stride, a->u_dim_stride, a->delta_batch_stride, a->delta_dim_stride,
                               a->z_batch_stride, a->z_dim_stride, a->A_dim_stride, a->A_dstate_stride,
                               a->B_batch_stride, a->B_group_stride, a->B_dstate_stride,
                               a->C_batch_stride, a->C_group_stride, a->C_dstate_stride};
    for (int64_t s : strides)
        if (s < 0) return fail(SS_ERR_INVALID, "negative stride");
    return SS_OK;
}

bool vec_rows(const void* base, int64_t bs, int64_t gs, int64_t ns, int64_t L, size_t es) {
    // 16-byte loads need aligned row starts and a whole number of 16-byte
    // vectors per 16-step tile.
    const int64_t per16 = int64_t(16 / es);
    return aligned(base, 16) && bs % per16 == 0 && gs % per16 == 0 && ns % per16 == 0 && L >= 0;
}

// Bytes from a (batch, rows, seqlen) array's base to the end of its last
// element (strides in elements, non-negative); 0 for an absent array.
int64_t seq_end(const void* ptr, int64_t batch, int64_t rows, int64_t seqlen, int64_t bs, int64_t rs, size_t es) {
    if (!ptr || batch <= 0 || rows <= 0 || seqlen <= 0) return 0;
    return ((batch - 1) * bs + (rows - 1) * rs + seqlen) * int64_t(es);
}

ss::FwdParams make_fwd_params(const ss_fwd_args* a) {
    ss::FwdParams p{};
    const size_t es = elem_size(a->itype);
    p.batch = a->batch; p.dim = a->dim; p.seqlen = a->seqlen; p.dstate = a->dstate;
    p.dpg = (a->is_var_B || a->is_var_C) ? a->dim / a->n_groups : a->dim;
    if (p.dpg < 1) p.dpg = 1;
    p.n_chunks = a->n_chunks;
    p.var_B = a->is_var_B != 0; p.var_C = a->is_var_C != 0;
    p.has_z = a->has_z != 0; p.softplus = a->delta_softplus != 0;
    // 16-byte tile loads of B / C in the general kernels
    p.vec_B = p.var_B && vec_rows(a->B, a->B_batch_stride, a->B_group_stride, a->B_dstate_stride, a->seqlen, es);
    p.vec_C = p.var_C && vec_rows(a->C, a->C_batch_stride, a->C_group_stride, a->C_dstate_stride, a->seqlen, es);
    p.u_bs = a->u_batch_stride; p.u_ds = a->u_dim_stride;
    p.dl_bs = a->delta_batch_stride; p.dl_ds = a->delta_dim_stride;
    p.z_bs = a->z_batch_stride; p.z_ds = a->z_dim_stride;
    p.o_bs = a->out_batch_stride; p.o_ds = a->out_dim_stride;
    p.A_ds = a->A_dim_stride; p.A_ns = a->A_dstate_stride;
    p.B_bs = a->B_batch_stride; p.B_gs = a->B_group_stride; p.B_ns = a->B_dstate_stride;
    p.C_bs = a->C_batch_stride; p.C_gs = a->C_group_stride; p.C_ns = a->C_dstate_stride;
    p.u = a->u; p.delta = a->delta; p.A = a->A; p.B = a->B; p.C = a->C;
    p.D = a->has_D ? a->D : nullptr;
    p.delta_bias = a->has_delta_bias ? a->delta_bias : nullptr;
    p.z = a->has_z ? a->z : nullptr;
    p.out = a->out; p.x = a->x;
    p.y = a->has_z ? a->y : nullptr;
    p.last_state = a->last_state;
    p.nseg = 1;
    p.y_bs = a->y_batch_stride; p.y_ds = a->y_dim_stride;
    const int64_t B = a->batch, D = a->dim, L = a->seqlen, G = D / p.dpg, N = a->dstate;
    p.u_end = seq_end(p.u, B, D, L, p.u_bs, p.u_ds, es);
    p.dl_end = seq_end(p.delta, B, D, L, p.dl_bs, p.dl_ds, es);
    p.z_end = seq_end(p.z, B, D, L, p.z_bs, p.z_ds, es);
    p.o_end = seq_end(p.out, B, D, L, p.o_bs, p.o_ds, es);
    p.y_end = seq_end(p.y, B, D, L, p.y_bs, p.y_ds, es);
    // out / y with every row on a 16-byte boundary: the fast forward stores
    // them non-temporally (fp32 batch 8 x dim 1536 x seqlen 2048 forward
    // -2 %); on rows off that boundary the same stores cost +24 % (seqlen
    // 2047 184 -> 229 us), so those keep the default policy
    const int64_t per16 = int64_t(16 / es);
    p.store_nt = aligned(p.out, 16) && p.o_bs % per16 == 0 && p.o_ds % per16 == 0 &&
                 (!p.y || (aligned(p.y, 16) && p.y_bs % per16 == 0 && p.y_ds % per16 == 0));
    // variable B / C: (batch, groups, dstate, seqlen)
    p.B_end = p.var_B && N > 0 ? seq_end(p.B, B, G, L, p.B_bs, p.B_gs, es) + (N - 1) * p.B_ns * int64_t(es) : 0;
    p.C_end = p.var_C && N > 0 ? seq_end(p.C, B, G, L, p.C_bs, p.C_gs, es) + (N - 1) * p.C_ns * int64_t(es) : 0;
    p.x_end = p.x ? B * p.n_chunks * D * N * int64_t(sizeof(float)) : 0;
    p.x_win = a->x_window_bytes > 0 ? a->x_window_bytes : (int64_t(1) << 31);
    p.xN = N;
    p.acc = nullptr;
    p.acc_in_end = p.acc_out_end = 0;
    return p;
}

// ---- state slices: dstate 16 S on the dstate-16 fast kernels --------------
// A call with dstate 16 S (S from 2 to 16) runs the fast kernels S times,
// once per slice of 16 states: A, B, C, x and last_state (and dA, dB, dC)
// are based at the slice's first state, x and last_state keep the call's
// dstate as their row length (so every kernel, fast or general, reads and
// writes the same checkpoints), and the sums over states that the slices
// share (y forward; sum_n g B and sum_n A g a h backward) accumulate in fp32
// in the workspace from pass to pass.  The last pass adds D and produces the
// outputs.

// The forward parameters of slice s.
ss::FwdParams slice_fwd(const ss::FwdParams& p, int s, size_t es) {
    ss::FwdParams q = p;
    const int64_t n0 = int64_t(ss::kT) * s;
    q.dstate = ss::kT;
    q.A = p.A + n0 * p.A_ns;
    q.B = static_cast<const char*>(p.B) + n0 * p.B_ns * int64_t(es);
    q.C = static_cast<const char*>(p.C) + n0 * p.C_ns * int64_t(es);
    q.B_end = p.B_end - n0 * p.B_ns * int64_t(es);
    q.C_end = p.C_end - n0 * p.C_ns * int64_t(es);
    if (p.x) {
        q.x = p.x + n0;
        q.x_end = p.x_end - n0 * int64_t(sizeof(float));
    }
    if (p.last_state) q.last_state = p.last_state + n0;
    return q;
}

// Slices of the forward for p (1: dstate 16, or the fast kernels do not
// apply: the call runs as it is).
int fwd_slices(const ss::FwdParams& p) {
    if (p.dstate <= ss::kT || p.dstate % ss::kT != 0 || !p.var_B || !p.var_C) return 1;
    ss::FwdParams q = p;
    q.dstate = ss::kT;
    return ss::fwd_fast_ok(q) ? int(p.dstate / ss::kT) : 1;
}

// Bytes of the forward's y accumulator (batch, dim, seqlen) fp32.
int64_t fwd_acc_bytes(const ss::FwdParams& p) { return p.batch * p.dim * p.seqlen * int64_t(sizeof(float)); }

int check_fwd(const ss_fwd_args* a, bool* empty) {
    int rc = check_fwd_common(a, empty);
    if (rc != SS_OK || *empty) return rc;
    if (!a->out) return fail(SS_ERR_INVALID, "out is NULL");
    if (!aligned(a->out, elem_size(a->itype))) return fail(SS_ERR_INVALID, "out is misaligned");
    if (a->out_batch_stride < 0 || a->out_dim_stride < 0) return fail(SS_ERR_INVALID, "negative stride");
    if (a->has_z && a->y) {
        if (!aligned(a->y, elem_size(a->itype))) return fail(SS_ERR_INVALID, "y is misaligned");
        if (a->y_batch_stride < 0 || a->y_dim_stride < 0) return fail(SS_ERR_INVALID, "negative stride");
    }
    return SS_OK;
}

int check_bwd(const ss_bwd_args* a, bool* empty) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    int rc = check_fwd_common(&a->f, empty);
    if (rc != SS_OK || *empty) return rc;
    const size_t es = elem_size(a->f.itype);
    struct P { const void* p; const char* name; bool need; size_t align; };
    const P ptrs[] = {
        {a->dout, "dout", true, es}, {a->du, "du", true, es}, {a->ddelta, "ddelta", true, es},
        {a->dz, "dz", a->f.has_z != 0, es}, {a->dA, "dA", true, 4}, {a->dB, "dB", true, 4},
        {a->dC, "dC", true, 4}, {a->dD, "dD", a->f.has_D != 0, 4},
        {a->ddelta_bias, "ddelta_bias", a->f.has_delta_bias != 0, 4},
        {a->f.y, "y (saved pre-gate output)", a->f.has_z != 0, es},
        {a->f.x, "x", true, 4},
    };
    for (const P& q : ptrs) {
        if (q.need && !q.p) return fail(SS_ERR_INVALID, "%s is NULL", q.name);
        if (q.p && !aligned(q.p, q.align)) return fail(SS_ERR_INVALID, "%s is misaligned", q.name);
    }
    const int64_t strides[] = {a->dout_batch_stride, a->dout_dim_stride, a->du_batch_stride, a->du_dim_stride,
                               a->ddelta_batch_stride, a->ddelta_dim_stride, a->dz_batch_stride, a->dz_dim_stride,
                               a->f.y_batch_stride, a->f.y_dim_stride};
    for (int64_t s : strides)
        if (s < 0) return fail(SS_ERR_INVALID, "negative stride");
    return SS_OK;
}

ss::BwdParams make_bwd_params(const ss_bwd_args* a) {
    ss::BwdParams p{};
    p.f = make_fwd_params(&a->f);
    p.bc_ld = a->f.seqlen;
    {
        const size_t es = elem_size(a->f.itype);
        const int64_t B = a->f.batch, D = a->f.dim, L = a->f.seqlen;
        p.do_end = seq_end(a->dout, B, D, L, a->dout_batch_stride, a->dout_dim_stride, es);
        p.du_end = seq_end(a->du, B, D, L, a->du_batch_stride, a->du_dim_stride, es);
        p.dd_end = seq_end(a->ddelta, B, D, L, a->ddelta_batch_stride, a->ddelta_dim_stride, es);
        p.dz_end = a->f.has_z ? seq_end(a->dz, B, D, L, a->dz_batch_stride, a->dz_dim_stride, es) : 0;
        // dB / dC: contiguous fp32 of B's / C's shape
        const int64_t nbc = B * (D / p.f.dpg) * a->f.dstate * L * int64_t(sizeof(float));
        p.dB_end = a->dB ? nbc : 0;
        p.dC_end = a->dC ? nbc : 0;
    }
    p.do_bs = a->dout_batch_stride; p.do_ds = a->dout_dim_stride;
    p.du_bs = a->du_batch_stride; p.du_ds = a->du_dim_stride;
    p.dd_bs = a->ddelta_batch_stride; p.dd_ds = a->ddelta_dim_stride;
    p.dz_bs = a->dz_batch_stride; p.dz_ds = a->dz_dim_stride;
    p.dout = a->dout; p.du = a->du; p.ddelta = a->ddelta; p.dz = a->f.has_z ? a->dz : nullptr;
    p.dA = a->dA; p.dB = a->dB; p.dC = a->dC;
    p.dD = a->f.has_D ? a->dD : nullptr;
    p.ddelta_bias = a->f.has_delta_bias ? a->ddelta_bias : nullptr;
    p.ws = nullptr;
    p.ws_slices = 1;
    p.ws_stride = 0;
    p.zero_grads = a->zero_grads != 0;
    p.det = a->deterministic != 0;
    p.det_par = nullptr;
    const ss_fwd_args& f = a->f;
    const int64_t G = (f.is_var_B || f.is_var_C) ? f.n_groups : 1;
    p.dA_n = f.dim * f.dstate;
    p.dB_n = f.is_var_B ? f.batch * G * f.dstate * f.seqlen : f.dim * f.dstate;
    p.dC_n = f.is_var_C ? f.batch * G * f.dstate * f.seqlen : f.dim * f.dstate;
    p.dD_n = f.dim;
    p.dA_N = f.dstate;
    p.bc_N = f.dstate;
    return p;
}

// Slices of the backward for p (1 as for fwd_slices; the two accumulators
// below 2^31 bytes, addressed from one base).
int bwd_slices(const ss::BwdParams& p) {
    if (fwd_slices(p.f) <= 1) return 1;
    ss::BwdParams q = p;
    q.f.dstate = ss::kT;
    if (!ss::bwd_fast_ok(q) || p.f.batch * p.f.dim * p.f.seqlen >= (int64_t(1) << 29)) return 1;
    return int(p.f.dstate / ss::kT);
}

// Bytes of the backward's two accumulators (sum_n g B, sum_n A g a h).
int64_t bwd_acc_bytes(const ss::BwdParams& p) { return 2 * fwd_acc_bytes(p.f); }

// Workspace layout for p: slices and bytes (0 when the fast backward does
// not use one: other kernel, or one slice over 64-byte aligned dB / dC rows).
// Backward workspace: the dB / dC slices (when they apply), then the
// sequence-segment carries (when they apply).  *slice_bytes: the first part.
// The slices' rows are padded to ss::bwd_ws_ld(seqlen) floats.  They apply
// with more than 96 channel blocks per group, with deterministic sums (every
// channel block of a group has a slice of its own, even a lone one, and the
// dA / dD / ddelta_bias partials follow the carries: (batch * nseg) rows of
// dim * 18 floats), and with a seqlen that is not a multiple of 32: dB / dC
// rows that do not start on 64-byte boundaries (the 16-step adds of the
// kernel would straddle cache lines), or a last chunk wholly past the
// sequence (its zero adds would land on steps that other chunks add to).
// One slice with aligned, padded rows, summed into dB / dC afterwards,
// costs less.
int64_t ws_bytes_for(const ss::BwdParams& p, int* slices, int* nseg, int64_t* slice_bytes) {
    *slices = ss::bwd_ws_slices(p);
    *slice_bytes = 0;
    const bool fast = ss::bwd_fast_ok(p);
    const int64_t stride = p.f.batch * (p.f.dim / p.f.dpg) * p.f.dstate * ss::bwd_ws_ld(p.f.seqlen);
    // (dB / dC slices only with B and C both variable)
    if (fast && p.f.var_B && p.f.var_C && (p.det || *slices > 1 || p.f.seqlen % 32 != 0)) {
        *slice_bytes = int64_t(2) * *slices * stride * int64_t(sizeof(float));
    } else {
        *slices = 1;
    }
    *nseg = ss::bwd_segments(p);
    const int64_t par = p.det ? p.f.batch * *nseg * p.f.dim * (p.f.dstate + 2) * int64_t(sizeof(float)) : 0;
    return *slice_bytes + ss::fwd_seg_bytes(p.f, *nseg) + par;
}

// Deterministic sums need the fast kernels (dstate 16, or 16 S on them
// once per slice).
int check_det(const ss::BwdParams& p) {
    if (!p.det) return SS_OK;
    if (!ss::bwd_fast_ok(p) && bwd_slices(p) <= 1)
        return fail(SS_ERR_UNSUPPORTED,
                    "deterministic sums need the fast backward (dstate 16 or a multiple of 16, variable B and C, "
                    "dim and channels per group multiples of 16)");
    return SS_OK;
}

int check_conv(const ss_conv1d_args* a, bool* empty) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
        return fail(SS_ERR_INVALID, "negative size (batch=%lld dim=%lld seqlen=%lld)",
                    (long long)a->batch, (long long)a->dim, (long long)a->seqlen);
    if (a->width < 1 || a->width > 4) return fail(SS_ERR_UNSUPPORTED, "width=%lld outside [1, 4]", (long long)a->width);
    if (a->itype != SS_F32 && a->itype != SS_BF16 && a->itype != SS_F16)
        return fail(SS_ERR_INVALID, "unknown itype %d", a->itype);
    if (a->batch > 0 && a->dim > INT32_MAX / a->batch)
        return fail(SS_ERR_UNSUPPORTED, "batch * dim = %lld rows is too many", (long long)(a->batch * a->dim));
    if ((a->seqlen + 1023) / 1024 > 65535)
        return fail(SS_ERR_UNSUPPORTED, "seqlen=%lld is too long", (long long)a->seqlen);
    *empty = a->batch == 0 || a->dim == 0 || a->seqlen == 0;
    if (*empty) return SS_OK;
    const size_t es = elem_size(a->itype);
    if (!a->x) return fail(SS_ERR_INVALID, "x is NULL");
    if (!a->weight) return fail(SS_ERR_INVALID, "weight is NULL");
    if (a->has_bias && !a->bias) return fail(SS_ERR_INVALID, "bias is NULL");
    if (!aligned(a->x, es)) return fail(SS_ERR_INVALID, "x is misaligned");
    if (!aligned(a->weight, 4) || (a->bias && !aligned(a->bias, 4))) return fail(SS_ERR_INVALID, "weight / bias is misaligned");
    const int64_t st[] = {a->x_batch_stride, a->x_dim_stride, a->w_dim_stride, a->w_width_stride};
    for (int64_t v : st)
        if (v < 0) return fail(SS_ERR_INVALID, "negative stride");
    return SS_OK;
}

int check_norm_common(int64_t rows, int64_t dim, int dtype, int w_dtype, const void* weight) {
    if (rows < 0 || dim < 0)
        return fail(SS_ERR_INVALID, "negative size (rows=%lld dim=%lld)", (long long)rows, (long long)dim);
    if (dtype != SS_F32 && dtype != SS_BF16 && dtype != SS_F16) return fail(SS_ERR_INVALID, "unknown dtype %d", dtype);
    if (w_dtype != dtype && w_dtype != SS_F32)
        return fail(SS_ERR_UNSUPPORTED, "weight dtype %d must be the row dtype or fp32", w_dtype);
    if (dim == 0) return SS_OK;
    if (!weight) return fail(SS_ERR_INVALID, "weight is NULL");
    if (!aligned(weight, elem_size(w_dtype))) return fail(SS_ERR_INVALID, "weight is misaligned");
    return SS_OK;
}


// The backward of a call with no scan work (batch, dim or seqlen 0): only
// zero_grads has something to do, clearing the accumulators.
int bwd_empty(const ss_bwd_args* a, void* stream) {
    if (!a->zero_grads) return ok();
    ss::BwdParams p = make_bwd_params(a);
    struct G { const float* ptr; int64_t n; const char* name; };
    const G gs[] = {{a->dA, p.dA_n, "dA"}, {a->dB, p.dB_n, "dB"}, {a->dC, p.dC_n, "dC"},
                    {a->f.has_D ? a->dD : nullptr, a->f.has_D ? p.dD_n : 0, "dD"},
                    {a->f.has_delta_bias ? a->ddelta_bias : nullptr, a->f.has_delta_bias ? p.dD_n : 0,
                     "ddelta_bias"}};
    for (const G& g : gs) {
        if (g.n > 0 && !g.ptr) return fail(SS_ERR_INVALID, "%s is NULL", g.name);
        if (g.ptr && !aligned(g.ptr, 4)) return fail(SS_ERR_INVALID, "%s is misaligned", g.name);
    }
    hipError_t e = ss::launch_bwd_zero_only(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "backward launch failed: %s", hipGetErrorString(e));
    return ok();
}

// The backward of checked arguments with scratch ws of ws_bytes bytes (NULL:
// none; the kernels then run without dB / dC slices and sequence segments).
// The backward as S passes of the dstate-16 fast kernel, one per 16-state
// slice (see slice_fwd).  Workspace: what one pass needs (dB / dC slices,
// segment carries), then the two accumulators.  The gradients are cleared
// once up front (zero_grads); each pass then clears its workspace slices and
// adds its slice's dA / dB / dC; dD and ddelta_bias, and du / ddelta / dz,
// come from the last pass, which has the sums over all states.
int bwd_run_slices(const ss_bwd_args* a, ss::BwdParams p, int S, void* ws, int slices, int nseg,
                   int64_t slice_bytes, int64_t pass_bytes, hipStream_t st) {
    const size_t es = elem_size(a->f.itype);
    const int64_t L = p.f.seqlen;
    hipError_t e = hipSuccess;
    if (p.zero_grads) {
        e = ss::launch_bwd_zero_only(p, st);
        if (e != hipSuccess) return fail(SS_ERR_HIP, "backward launch failed: %s", hipGetErrorString(e));
    }
    float* acc = reinterpret_cast<float*>(static_cast<char*>(ws) + pass_bytes);
    for (int s = 0; s < S; ++s) {
        ss::BwdParams q = p;
        const int64_t n0 = int64_t(ss::kT) * s;
        q.f = slice_fwd(p.f, s, es);
        // (deterministic sums: each pass stores or adds its own rows of the
        // gradients in a fixed order; otherwise they were cleared up front)
        q.zero_grads = p.det ? p.zero_grads : 0;
        q.dA = p.dA + n0;
        // dB / dC rows of this slice: (batch, group) blocks of dstate rows of
        // seqlen floats, the slice's 16 from row n0
        q.dB = p.dB + n0 * L;
        q.dC = p.dC + n0 * L;
        q.dB_end = p.dB_end - n0 * L * int64_t(sizeof(float));
        q.dC_end = p.dC_end - n0 * L * int64_t(sizeof(float));
        if (slice_bytes > 0) {
            q.ws = static_cast<float*>(ws);
            q.ws_slices = slices;
            q.ws_stride = slice_bytes / int64_t(sizeof(float)) / (2 * slices);
            q.ws_end = slice_bytes;
            q.bc_ld = ss::bwd_ws_ld(L);
            q.bc_N = ss::kT;
        }
        if (nseg > 1) {
            q.f.nseg = nseg;
            q.f.seg_h = reinterpret_cast<float*>(static_cast<char*>(ws) + slice_bytes);
            q.f.seg_s = q.f.seg_h + q.f.batch * nseg * q.f.dim * 16;
        }
        if (p.det)
            q.det_par = reinterpret_cast<float*>(static_cast<char*>(ws) + slice_bytes + ss::fwd_seg_bytes(q.f, nseg));
        q.f.acc = acc;
        q.f.acc_in_end = s > 0 ? bwd_acc_bytes(p) : 0;
        q.f.acc_out_end = s < S - 1 ? bwd_acc_bytes(p) : 0;
        if (s < S - 1) {           // the per-step outputs, dD and ddelta_bias belong to the last pass
            q.du_end = q.dd_end = q.dz_end = 0;
            q.f.y_end = 0;
            q.dD = nullptr;
            q.ddelta_bias = nullptr;
        }
        e = ss::launch_bwd(q, a->f.itype, st);
        if (e != hipSuccess) return fail(SS_ERR_HIP, "backward launch failed: %s", hipGetErrorString(e));
    }
    return ok();
}

// Workspace bytes for the backward's fastest path for p: the state-sliced
// passes (what one pass needs, then the two accumulators) or one pass.
int64_t bwd_ws_need(const ss::BwdParams& p, int itype) {
    int slices = 1, nseg = 1;
    int64_t slice_bytes = 0;
    if (bwd_slices(p) > 1) {
        ss::BwdParams q0 = p;
        q0.f = slice_fwd(p.f, 0, elem_size(itype));
        return ws_bytes_for(q0, &slices, &nseg, &slice_bytes) + bwd_acc_bytes(p);
    }
    return ws_bytes_for(p, &slices, &nseg, &slice_bytes);
}

int bwd_run(const ss_bwd_args* a, void* ws, int64_t ws_bytes, void* stream) {
    ss::BwdParams p = make_bwd_params(a);
    int rc = check_det(p);
    if (rc != SS_OK) return rc;
    if (ws && !aligned(ws, 16)) return fail(SS_ERR_INVALID, "workspace is misaligned");
    const int S = bwd_slices(p);
    if (S > 1) {
        ss::BwdParams q0 = p;
        q0.f = slice_fwd(p.f, 0, elem_size(a->f.itype));
        int slices = 1, nseg = 1;
        int64_t slice_bytes = 0;
        const int64_t pass_bytes = ws_bytes_for(q0, &slices, &nseg, &slice_bytes);
        if (ws && ws_bytes >= pass_bytes + bwd_acc_bytes(p))
            return bwd_run_slices(a, p, S, ws, slices, nseg, slice_bytes, pass_bytes, static_cast<hipStream_t>(stream));
        if (p.det)
            return fail(SS_ERR_INVALID, "deterministic sums need a workspace of %lld bytes",
                        (long long)(pass_bytes + bwd_acc_bytes(p)));
        // without that much workspace: the general kernel, as below
    }
    int slices = 1, nseg = 1;
    int64_t slice_bytes = 0;
    const int64_t need = ws_bytes_for(p, &slices, &nseg, &slice_bytes);
    if (p.det && need > 0 && !ws)
        return fail(SS_ERR_INVALID, "deterministic sums need a workspace of %lld bytes", (long long)need);
    if (need > 0 && ws) {
        if (ws_bytes < need)
            return fail(SS_ERR_INVALID, "workspace of %lld bytes, %lld needed", (long long)ws_bytes,
                        (long long)need);
        if (!aligned(ws, 16)) return fail(SS_ERR_INVALID, "workspace is misaligned");
        if (slice_bytes > 0) {
            p.ws = static_cast<float*>(ws);
            p.ws_slices = slices;
            p.ws_stride = slice_bytes / int64_t(sizeof(float)) / (2 * slices);
            p.ws_end = slice_bytes;
            p.bc_ld = ss::bwd_ws_ld(p.f.seqlen);
        }
        const int64_t seg_bytes = ss::fwd_seg_bytes(p.f, nseg);
        if (nseg > 1) {
            p.f.nseg = nseg;
            p.f.seg_h = reinterpret_cast<float*>(static_cast<char*>(ws) + slice_bytes);
            p.f.seg_s = p.f.seg_h + p.f.batch * nseg * p.f.dim * 16;
        }
        if (p.det) p.det_par = reinterpret_cast<float*>(static_cast<char*>(ws) + slice_bytes + seg_bytes);
    }
    hipError_t e = ss::launch_bwd(p, a->f.itype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "backward launch failed: %s", hipGetErrorString(e));
    return ok();
}

// Fixed device scratch of ss_bwd_noalloc, for callers that cannot allocate.
// Each GPU the library runs on holds its own copy until the process ends.
// Host code never passes `scratch` itself to a kernel or a copy (on the host
// it names a stand-in, not device memory): it looks up the array's device
// address once per device with hipGetSymbolAddress and uses that.
constexpr int64_t kScratchBytes = SS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device, with that device current).
int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(SS_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(SS_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(SS_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return SS_OK;
}

}  // namespace

extern "C" {

int ss_abi_version(void) { return SS_ABI_VERSION; }

int64_t ss_chunk_size(void) { return ss::kChunk; }

int64_t ss_max_dstate(void) { return 16 * ss::kMaxSPL; }

void ss_struct_sizes(int64_t* fwd_args, int64_t* bwd_args) {
    if (fwd_args) *fwd_args = int64_t(sizeof(ss_fwd_args));
    if (bwd_args) *bwd_args = int64_t(sizeof(ss_bwd_args));
}

const char* ss_last_error(void) { return g_err.c_str(); }

int ss_fwd_check(const ss_fwd_args* a) {
    bool empty = false;
    int rc = check_fwd(a, &empty);
    return rc == SS_OK ? ok() : rc;
}

int ss_bwd_check(const ss_bwd_args* a) {
    bool empty = false;
    int rc = check_bwd(a, &empty);
    return rc == SS_OK ? ok() : rc;
}

int ss_fwd(const ss_fwd_args* a, void* stream) {
    bool empty = false;
    int rc = check_fwd(a, &empty);
    if (rc != SS_OK) return rc;
    if (empty) return ok();
    ss::FwdParams p = make_fwd_params(a);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (a->workspace && !aligned(a->workspace, 16)) return fail(SS_ERR_INVALID, "workspace is misaligned");
    const int slices = fwd_slices(p);
    const size_t es = elem_size(a->itype);
    // the sequence segments of each pass (the same for every slice), then,
    // for state slices, the y accumulator
    const ss::FwdParams q0 = slices > 1 ? slice_fwd(p, 0, es) : p;
    const int nseg = ss::fwd_segments(q0);
    const int64_t seg_bytes = nseg > 1 ? ss::fwd_seg_bytes(q0, nseg) : 0;
    const int64_t have = a->workspace ? a->workspace_bytes : 0;
    auto attach_segs = [&](ss::FwdParams& q) {
        if (nseg > 1 && have >= seg_bytes) {
            q.nseg = nseg;
            q.seg_h = static_cast<float*>(a->workspace);
            q.seg_s = q.seg_h + q.batch * nseg * q.dim * 16;
        }
    };
    if (slices > 1 && have >= seg_bytes + fwd_acc_bytes(p)) {
        float* acc = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + seg_bytes);
        for (int s = 0; s < slices; ++s) {
            ss::FwdParams q = slice_fwd(p, s, es);
            attach_segs(q);
            q.acc = acc;
            q.acc_in_end = s > 0 ? fwd_acc_bytes(p) : 0;
            q.acc_out_end = s < slices - 1 ? fwd_acc_bytes(p) : 0;
            if (s < slices - 1) {      // out, y and D belong to the last pass
                q.D = nullptr;
                q.o_end = 0;
                q.y_end = 0;
            }
            hipError_t e = ss::launch_fwd(q, a->itype, st);
            if (e != hipSuccess) return fail(SS_ERR_HIP, "forward launch failed: %s", hipGetErrorString(e));
        }
        return ok();
    }
    if (slices <= 1) attach_segs(p);
    hipError_t e = ss::launch_fwd(p, a->itype, st);
    if (e != hipSuccess) return fail(SS_ERR_HIP, "forward launch failed: %s", hipGetErrorString(e));
    return ok();
}

int64_t ss_fwd_workspace_bytes(const ss_fwd_args* a) {
    bool empty = false;
    if (check_fwd(a, &empty) != SS_OK) return -1;
    ok();
    if (empty) return 0;
    const ss::FwdParams p = make_fwd_params(a);
    const int slices = fwd_slices(p);
    const ss::FwdParams q0 = slices > 1 ? slice_fwd(p, 0, elem_size(a->itype)) : p;
    const int nseg = ss::fwd_segments(q0);
    return (nseg > 1 ? ss::fwd_seg_bytes(q0, nseg) : 0) + (slices > 1 ? fwd_acc_bytes(p) : 0);
}

int64_t ss_bwd_workspace_bytes(const ss_bwd_args* a) {
    bool empty = false;
    if (check_bwd(a, &empty) != SS_OK) return -1;
    if (empty) return ok(), 0;
    const ss::BwdParams p = make_bwd_params(a);
    if (check_det(p) != SS_OK) return -1;
    ok();
    return bwd_ws_need(p, a->f.itype);
}

const char* ss_fwd_kernel_name(const ss_fwd_args* a) {
    bool empty = false;
    if (check_fwd(a, &empty) != SS_OK) return nullptr;
    ok();
    if (empty) return "";
    const ss::FwdParams p = make_fwd_params(a);
    return fwd_slices(p) > 1 ? "ss_fwd_fast" : ss::fwd_kernel_name(p);
}

const char* ss_bwd_kernel_name(const ss_bwd_args* a) {
    bool empty = false;
    if (check_bwd(a, &empty) != SS_OK) return nullptr;
    ok();
    if (empty) return "";
    const ss::BwdParams p = make_bwd_params(a);
    return bwd_slices(p) > 1 ? "ss_bwd_fast" : ss::bwd_kernel_name(p);
}

int ss_bwd(const ss_bwd_args* a, void* stream) {
    bool empty = false;
    int rc = check_bwd(a, &empty);
    if (rc != SS_OK) return rc;
    if (empty) return bwd_empty(a, stream);
    return bwd_run(a, a->workspace, a->workspace ? a->workspace_bytes : 0, stream);
}

int ss_bwd_noalloc(const ss_bwd_args* a, void* stream) {
    bool empty = false;
    int rc = check_bwd(a, &empty);
    if (rc != SS_OK) return rc;
    if (empty) return bwd_empty(a, stream);
    const ss::BwdParams p = make_bwd_params(a);
    rc = check_det(p);
    if (rc != SS_OK) return rc;
    // the state-sliced passes when their workspace fits (deterministic sums
    // need it), else the one-pass backward
    int slices = 1, nseg = 1;
    int64_t slice_bytes = 0;
    int64_t need = bwd_ws_need(p, a->f.itype);
    if (need > kScratchBytes && !p.det && bwd_slices(p) > 1) need = ws_bytes_for(p, &slices, &nseg, &slice_bytes);
    if (need > kScratchBytes)
        return fail(SS_ERR_UNSUPPORTED,
                    "ss_bwd_noalloc: these arguments need %lld bytes of scratch, more than the %lld bytes "
                    "of its fixed device buffer; use ss_bwd with a workspace",
                    (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    if (need > 0) {
        rc = scratch_on_current_device(&ws);
        if (rc != SS_OK) return rc;
    }
    return bwd_run(a, ws, need, stream);
}

int ss_conv1d_fwd(const ss_conv1d_args* a, void* stream) {
    bool empty = false;
    int rc = check_conv(a, &empty);
    if (rc != SS_OK) return rc;
    if (empty) return ok();
    if (!a->out) return fail(SS_ERR_INVALID, "out is NULL");
    if (!aligned(a->out, elem_size(a->itype))) return fail(SS_ERR_INVALID, "out is misaligned");
    if (a->out_batch_stride < 0 || a->out_dim_stride < 0) return fail(SS_ERR_INVALID, "negative stride");
    hipError_t e = ss::conv1d_launch(a, nullptr, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "conv1d forward launch failed: %s", hipGetErrorString(e));
    return ok();
}

int ss_conv1d_bwd(const ss_conv1d_bwd_args* g, void* stream) {
    if (!g) return fail(SS_ERR_INVALID, "null argument block");
    bool empty = false;
    int rc = check_conv(&g->f, &empty);
    if (rc != SS_OK) return rc;
    if (empty) return ok();
    const size_t es = elem_size(g->f.itype);
    if (!g->dout || !g->dx) return fail(SS_ERR_INVALID, "%s is NULL", g->dout ? "dx" : "dout");
    if (!g->dweight) return fail(SS_ERR_INVALID, "dweight is NULL");
    if (g->f.has_bias && !g->dbias) return fail(SS_ERR_INVALID, "dbias is NULL");
    if (!aligned(g->dout, es) || !aligned(g->dx, es)) return fail(SS_ERR_INVALID, "dout / dx is misaligned");
    if (!aligned(g->dweight, 4) || (g->dbias && !aligned(g->dbias, 4)))
        return fail(SS_ERR_INVALID, "dweight / dbias is misaligned");
    if (g->dout_batch_stride < 0 || g->dout_dim_stride < 0 || g->dx_batch_stride < 0 || g->dx_dim_stride < 0)
        return fail(SS_ERR_INVALID, "negative stride");
    if (g->workspace) {
        if (!aligned(g->workspace, 4)) return fail(SS_ERR_INVALID, "workspace is misaligned");
        const int64_t need = ss::conv1d_bwd_workspace_bytes(g->f.batch, g->f.dim, g->f.seqlen);
        if (g->workspace_bytes < need)
            return fail(SS_ERR_INVALID, "workspace_bytes=%lld below the %lld the fixed-order sums need",
                        (long long)g->workspace_bytes, (long long)need);
    }
    hipError_t e = ss::conv1d_launch(&g->f, g, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "conv1d backward launch failed: %s", hipGetErrorString(e));
    return ok();
}

int ss_state_update(const ss_state_update_args* a, void* stream) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    if (a->batch < 0 || a->dim < 0 || a->dstate < 0 || a->n_groups < 1)
        return fail(SS_ERR_INVALID, "bad size (batch=%lld dim=%lld dstate=%lld n_groups=%lld)", (long long)a->batch,
                    (long long)a->dim, (long long)a->dstate, (long long)a->n_groups);
    if (a->itype != SS_F32 && a->itype != SS_BF16 && a->itype != SS_F16)
        return fail(SS_ERR_INVALID, "unknown itype %d", a->itype);
    if (a->dim % a->n_groups != 0)
        return fail(SS_ERR_INVALID, "dim=%lld is not a multiple of n_groups=%lld", (long long)a->dim,
                    (long long)a->n_groups);
    if (a->batch == 0 || a->dim == 0) return ok();
    if (a->batch > int64_t(UINT32_MAX) / 2 / (a->dim > 0 ? a->dim : 1))
        return fail(SS_ERR_UNSUPPORTED, "batch * dim is too large");
    const size_t es = elem_size(a->itype);
    const bool low = a->delta_low != nullptr;
    if (!a->state || !a->x || (!low && !a->delta) || !a->out || (a->dstate > 0 && (!a->A || !a->B || !a->C)))
        return fail(SS_ERR_INVALID, "state / x / delta / A / B / C / out is NULL");
    if (low && (!a->delta_weight || a->delta_rank < 1))
        return fail(SS_ERR_INVALID, "delta_low given without delta_weight or with delta_rank=%lld",
                    (long long)a->delta_rank);
    if (low && (!aligned(a->delta_low, elem_size(a->itype)) || !aligned(a->delta_weight, elem_size(a->itype))))
        return fail(SS_ERR_INVALID, "delta_low / delta_weight is misaligned");
    if (low && (a->delta_low_batch_stride < 0 || a->delta_low_rank_stride < 0 || a->delta_weight_dim_stride < 0 ||
                a->delta_weight_rank_stride < 0))
        return fail(SS_ERR_INVALID, "negative stride");
    if ((a->has_D && !a->D) || (a->has_z && !a->z) || (a->has_delta_bias && !a->delta_bias))
        return fail(SS_ERR_INVALID, "D / z / delta_bias is NULL but flagged present");
    const void* p2[] = {a->x, low ? nullptr : a->delta, a->B, a->C, a->has_z ? a->z : nullptr, a->out};
    for (const void* q : p2)
        if (q && !aligned(q, es)) return fail(SS_ERR_INVALID, "x / delta / B / C / z / out is misaligned");
    const void* p4[] = {a->state, a->A, a->has_D ? a->D : nullptr, a->has_delta_bias ? a->delta_bias : nullptr};
    for (const void* q : p4)
        if (q && !aligned(q, 4)) return fail(SS_ERR_INVALID, "state / A / D / delta_bias is misaligned");
    const int64_t st[] = {a->state_batch_stride, a->state_dim_stride, a->state_dstate_stride, a->x_batch_stride,
                          a->x_dim_stride, a->delta_batch_stride, a->delta_dim_stride, a->z_batch_stride,
                          a->z_dim_stride, a->out_batch_stride, a->out_dim_stride, a->A_dim_stride,
                          a->A_dstate_stride, a->B_batch_stride, a->B_group_stride, a->B_dstate_stride,
                          a->C_batch_stride, a->C_group_stride, a->C_dstate_stride};
    for (int64_t v : st)
        if (v < 0) return fail(SS_ERR_INVALID, "negative stride");
    hipError_t e = ss::state_update_launch(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "state update launch failed: %s", hipGetErrorString(e));
    return ok();
}

int ss_conv1d_update(const ss_conv1d_update_args* a, void* stream) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    if (a->batch < 0 || a->dim < 0)
        return fail(SS_ERR_INVALID, "negative size (batch=%lld dim=%lld)", (long long)a->batch, (long long)a->dim);
    if (a->width < 1 || a->width > 4) return fail(SS_ERR_UNSUPPORTED, "width=%lld outside [1, 4]", (long long)a->width);
    if (a->itype != SS_F32 && a->itype != SS_BF16 && a->itype != SS_F16)
        return fail(SS_ERR_INVALID, "unknown itype %d", a->itype);
    if (a->batch == 0 || a->dim == 0) return ok();
    if (a->batch > int64_t(UINT32_MAX) / 2 / a->dim) return fail(SS_ERR_UNSUPPORTED, "batch * dim is too large");
    const size_t es = elem_size(a->itype);
    if (!a->x || !a->conv_state || !a->weight || !a->out || (a->has_bias && !a->bias))
        return fail(SS_ERR_INVALID, "x / conv_state / weight / bias / out is NULL");
    if (!aligned(a->x, es) || !aligned(a->conv_state, es) || !aligned(a->out, es))
        return fail(SS_ERR_INVALID, "x / conv_state / out is misaligned");
    if (!aligned(a->weight, 4) || (a->has_bias && !aligned(a->bias, 4)))
        return fail(SS_ERR_INVALID, "weight / bias is misaligned");
    const int64_t st[] = {a->x_batch_stride, a->x_dim_stride, a->out_batch_stride, a->out_dim_stride,
                          a->state_batch_stride, a->state_dim_stride, a->state_width_stride,
                          a->w_dim_stride, a->w_width_stride};
    for (int64_t v : st)
        if (v < 0) return fail(SS_ERR_INVALID, "negative stride");
    hipError_t e = ss::conv_update_launch(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "conv1d update launch failed: %s", hipGetErrorString(e));
    return ok();
}

int ss_decode_linear(const ss_decode_linear_args* a, void* stream) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    if (a->batch < 0 || a->n_out < 0 || a->k_in < 0)
        return fail(SS_ERR_INVALID, "negative size (batch=%lld n_out=%lld k_in=%lld)", (long long)a->batch,
                    (long long)a->n_out, (long long)a->k_in);
    if (a->dtype != SS_BF16 && a->dtype != SS_F16)
        return fail(SS_ERR_UNSUPPORTED, "dtype %d: the matrix-core path takes bf16 or fp16", a->dtype);
    if (a->bias && a->bias_dtype != a->dtype && a->bias_dtype != SS_F32)
        return fail(SS_ERR_UNSUPPORTED, "bias dtype %d must be the row dtype or fp32", a->bias_dtype);
    if (a->k_in % 16 != 0) return fail(SS_ERR_UNSUPPORTED, "k_in=%lld is not a multiple of 16", (long long)a->k_in);
    if (a->workspace_bytes < 0) return fail(SS_ERR_INVALID, "negative workspace_bytes");
    if (a->workspace && !aligned(a->workspace, 16)) return fail(SS_ERR_INVALID, "workspace must be 16-byte aligned");
    if (const ss_conv1d_update_args* c = a->conv) {
        if (c->itype != a->dtype) return fail(SS_ERR_INVALID, "conv itype %d differs from dtype %d", c->itype, a->dtype);
        if (c->batch != a->batch)
            return fail(SS_ERR_INVALID, "conv batch=%lld differs from batch=%lld", (long long)c->batch, (long long)a->batch);
        if (c->dim < 0 || c->dim > a->n_out)
            return fail(SS_ERR_INVALID, "conv dim=%lld outside [0, n_out=%lld]", (long long)c->dim, (long long)a->n_out);
        if (c->width < 1 || c->width > 4) return fail(SS_ERR_UNSUPPORTED, "width=%lld outside [1, 4]", (long long)c->width);
        if (c->dim > 0 && a->batch > 0) {
            if (!c->conv_state || !c->weight || (c->has_bias && !c->bias))
                return fail(SS_ERR_INVALID, "conv_state / conv weight / conv bias is NULL");
            if (!aligned(c->conv_state, 2) || !aligned(c->weight, 4) || (c->has_bias && !aligned(c->bias, 4)))
                return fail(SS_ERR_INVALID, "conv_state / conv weight / conv bias is misaligned");
            const int64_t st[] = {c->state_batch_stride, c->state_dim_stride, c->state_width_stride, c->w_dim_stride,
                                  c->w_width_stride};
            for (int64_t v : st)
                if (v < 0) return fail(SS_ERR_INVALID, "negative conv stride");
        }
    }
    if (const ss_rmsnorm_args* n = a->norm) {
        if (n->rows != a->batch || n->dim != a->k_in)
            return fail(SS_ERR_INVALID, "norm rows=%lld dim=%lld must equal batch=%lld and k_in=%lld",
                        (long long)n->rows, (long long)n->dim, (long long)a->batch, (long long)a->k_in);
        if (n->dtype != a->dtype) return fail(SS_ERR_INVALID, "norm dtype %d differs from dtype %d", n->dtype, a->dtype);
        if (n->w_dtype != a->dtype && n->w_dtype != SS_F32)
            return fail(SS_ERR_UNSUPPORTED, "norm weight dtype %d must be the row dtype or fp32", n->w_dtype);
        if (a->k_in > 1024) return fail(SS_ERR_UNSUPPORTED, "the fused norm takes k_in <= 1024 (k_in=%lld)", (long long)a->k_in);
        if (!(n->eps >= 0.f)) return fail(SS_ERR_INVALID, "norm eps must be >= 0");
        if (a->batch > 0) {
            if (!n->x || !n->weight) return fail(SS_ERR_INVALID, "norm x / weight is NULL");
            const bool rows16 = aligned(n->x, 16) && n->x_row_stride % 8 == 0 && n->x_row_stride >= n->dim &&
                                (!n->residual || (aligned(n->residual, 16) && n->residual_row_stride % 8 == 0 &&
                                                  n->residual_row_stride >= n->dim)) &&
                                (!n->residual || !n->residual_out ||
                                 (aligned(n->residual_out, 16) && n->residual_out_row_stride % 8 == 0 &&
                                  n->residual_out_row_stride >= n->dim)) &&
                                aligned(n->weight, 16) && (!n->rstd || aligned(n->rstd, 4));
            if (!rows16) return fail(SS_ERR_INVALID, "the fused norm needs 16-byte aligned rows covering dim");
            // every output tile's workgroup reads x and residual, and only the
            // first writes residual_out: an in-place residual stream would let
            // the other tiles normalise rows already updated
            const size_t es = elem_size(n->dtype);
            const int64_t d = n->dim;
            if (n->residual &&
                (rows_overlap(n->residual_out, n->residual_out_row_stride, d, n->x, n->x_row_stride, d, n->rows, es) ||
                 rows_overlap(n->residual_out, n->residual_out_row_stride, d, n->residual, n->residual_row_stride, d,
                              n->rows, es)))
                return fail(SS_ERR_INVALID, "norm residual_out overlaps norm x or residual (no in-place residual)");
        }
    }
    if (a->batch == 0 || a->n_out == 0) return ok();
    if (a->k_in == 0) return fail(SS_ERR_UNSUPPORTED, "k_in=0");
    if ((a->n_out + 15) / 16 * ss::kLinMaxSplit > INT32_MAX || (a->batch + 15) / 16 > 65535)
        return fail(SS_ERR_UNSUPPORTED, "n_out or batch too large");
    if ((!a->norm && !a->x) || !a->weight || !a->y) return fail(SS_ERR_INVALID, "x / weight / y is NULL");
    if ((!a->norm && !aligned(a->x, 8)) || !aligned(a->weight, 8) || !aligned(a->y, 2))
        return fail(SS_ERR_INVALID, "x / weight must be 8-byte aligned, y 2-byte aligned");
    if (a->bias && !aligned(a->bias, a->bias_dtype == SS_F32 ? 4 : 2)) return fail(SS_ERR_INVALID, "bias is misaligned");
    {
        // y is written while other workgroups still read the input rows
        const size_t es = elem_size(a->dtype);
        const ss_rmsnorm_args* n = a->norm;
        const int64_t no = a->n_out, k = a->k_in, rows = a->batch;
        const bool ov =
            n ? (rows_overlap(a->y, a->y_row_stride, no, n->x, n->x_row_stride, k, rows, es) ||
                 (n->residual && (rows_overlap(a->y, a->y_row_stride, no, n->residual, n->residual_row_stride, k, rows, es) ||
                                  rows_overlap(a->y, a->y_row_stride, no, n->residual_out, n->residual_out_row_stride, k,
                                               rows, es))))
              : rows_overlap(a->y, a->y_row_stride, no, a->x, a->x_row_stride, k, rows, es);
        if (ov) return fail(SS_ERR_INVALID, "y overlaps the input rows (x, or the norm's x / residual / residual_out)");
    }
    if ((!a->norm && (a->x_row_stride < a->k_in || a->x_row_stride % 4)) || a->w_row_stride < a->k_in ||
        a->y_row_stride < a->n_out || a->w_row_stride % 4)
        return fail(SS_ERR_INVALID, "row strides must cover the rows, x / weight strides multiples of 4");
    hipError_t e = ss::decode_linear_launch(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "decode linear launch failed: %s", hipGetErrorString(e));
    return ok();
}

int64_t ss_decode_linear_workspace_bytes(const ss_decode_linear_args* a) {
    if (!a) {
        fail(SS_ERR_INVALID, "null argument block");
        return -1;
    }
    if (a->batch < 0 || a->n_out < 0 || a->k_in < 0 || a->k_in % 16 != 0) {
        fail(SS_ERR_INVALID, "invalid size (batch=%lld n_out=%lld k_in=%lld)", (long long)a->batch,
             (long long)a->n_out, (long long)a->k_in);
        return -1;
    }
    ok();
    return ss::decode_linear_split(a->batch, a->n_out, a->k_in).workspace_bytes;
}

int64_t ss_conv1d_bwd_workspace_bytes(const ss_conv1d_bwd_args* g) {
    if (!g) {
        fail(SS_ERR_INVALID, "null argument block");
        return -1;
    }
    if (g->f.batch < 0 || g->f.dim < 0 || g->f.seqlen < 0) {
        fail(SS_ERR_INVALID, "negative size (batch=%lld dim=%lld seqlen=%lld)", (long long)g->f.batch,
             (long long)g->f.dim, (long long)g->f.seqlen);
        return -1;
    }
    ok();
    return ss::conv1d_bwd_workspace_bytes(g->f.batch, g->f.dim, g->f.seqlen);
}

int64_t ss_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t dim) {
    if (rows < 0 || dim < 0) {
        fail(SS_ERR_INVALID, "negative size (rows=%lld dim=%lld)", (long long)rows, (long long)dim);
        return -1;
    }
    return ss::rmsnorm_bwd_parts(rows) * dim * int64_t(sizeof(float));
}

int ss_rmsnorm_fwd(const ss_rmsnorm_args* a, void* stream) {
    if (!a) return fail(SS_ERR_INVALID, "null argument block");
    int rc = check_norm_common(a->rows, a->dim, a->dtype, a->w_dtype, a->weight);
    if (rc != SS_OK) return rc;
    if (a->rows == 0 || a->dim == 0) return ok();
    if (!(a->eps >= 0.f)) return fail(SS_ERR_INVALID, "eps must be >= 0");
    const size_t es = elem_size(a->dtype);
    if (!a->x || !a->out) return fail(SS_ERR_INVALID, "%s is NULL", a->x ? "out" : "x");
    const void* ptrs[] = {a->x, a->residual, a->out, a->residual ? a->residual_out : nullptr};
    const int64_t rs[] = {a->x_row_stride, a->residual_row_stride, a->out_row_stride, a->residual_out_row_stride};
    for (int i = 0; i < 4; ++i) {
        if (!ptrs[i]) continue;
        if (!aligned(ptrs[i], es)) return fail(SS_ERR_INVALID, "x / residual / out / residual_out is misaligned");
        if (rs[i] < 0) return fail(SS_ERR_INVALID, "negative row stride");
    }
    if (a->rstd && !aligned(a->rstd, 4)) return fail(SS_ERR_INVALID, "rstd is misaligned");
    if (a->rows > int64_t(UINT32_MAX) * 4) return fail(SS_ERR_UNSUPPORTED, "too many rows");
    hipError_t e = ss::rmsnorm_launch(a, nullptr, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "rmsnorm forward launch failed: %s", hipGetErrorString(e));
    return ok();
}

int ss_rmsnorm_bwd(const ss_rmsnorm_bwd_args* g, void* stream) {
    if (!g) return fail(SS_ERR_INVALID, "null argument block");
    int rc = check_norm_common(g->rows, g->dim, g->dtype, g->w_dtype, g->weight);
    if (rc != SS_OK) return rc;
    if (g->dim == 0) return ok();
    if (g->dim > ss::kRmsNormMaxBwdDim)
        return fail(SS_ERR_UNSUPPORTED, "dim=%lld above %lld", (long long)g->dim, (long long)ss::kRmsNormMaxBwdDim);
    if (!g->dweight) return fail(SS_ERR_INVALID, "dweight is NULL");
    if (!aligned(g->dweight, g->w_dtype == SS_F32 ? 4 : 2)) return fail(SS_ERR_INVALID, "dweight is misaligned");
    const int64_t need = ss_rmsnorm_bwd_workspace_bytes(g->rows, g->dim);
    if (need > 0 && (!g->workspace || g->workspace_bytes < need))
        return fail(SS_ERR_INVALID, "workspace of %lld bytes needed (got %lld)", (long long)need,
                    (long long)(g->workspace ? g->workspace_bytes : 0));
    if (g->workspace && !aligned(g->workspace, 16)) return fail(SS_ERR_INVALID, "workspace is misaligned");
    if (g->rows > 0) {
        const size_t es = elem_size(g->dtype);
        if (!g->s || !g->dout || !g->dx || !g->rstd) return fail(SS_ERR_INVALID, "s / dout / dx / rstd is NULL");
        const void* ptrs[] = {g->s, g->dout, g->dresidual_out, g->dx};
        const int64_t rs[] = {g->s_row_stride, g->dout_row_stride, g->dresidual_out_row_stride, g->dx_row_stride};
        for (int i = 0; i < 4; ++i) {
            if (!ptrs[i]) continue;
            if (!aligned(ptrs[i], es)) return fail(SS_ERR_INVALID, "s / dout / dresidual_out / dx is misaligned");
            if (rs[i] < 0) return fail(SS_ERR_INVALID, "negative row stride");
        }
        if (!aligned(g->rstd, 4)) return fail(SS_ERR_INVALID, "rstd is misaligned");
    }
    hipError_t e = ss::rmsnorm_launch(nullptr, g, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(SS_ERR_HIP, "rmsnorm backward launch failed: %s", hipGetErrorString(e));
    return ok();
}

}  // extern "C"
