// Forward selective scan for gfx950.
//
// Semantics follow the reference forward kernel
// (csrc/selective_scan/forward_kernel.cu:174-310) plus the z gate applied by
// its caller (modules/mamba_simple.py:143-146):
//   delta' = softplus(delta + bias), a = exp2(delta' * A * log2 e),
//   h_t = a_t h_{t-1} + delta'_t u_t B_t,  y_t = sum_n C_t h_t + D u_t,
//   out = y * silu(z).
//
// Work decomposition (not the reference's one-block-per-(b, d) CUB scan): a
// lane owns one (channel, state) recurrence and walks time sequentially, so
// there is no cross-lane scan at all.  A 16-lane row is one channel; per
// 16-step tile, lane r loads the per-step inputs of step t0 + r and the
// other lanes read them with DPP row broadcasts folded into the arithmetic.
// The sum over states, y_t = sum_n C h, is an in-row transposed sum through
// LDS.  Every kChunk steps the state is checkpointed to x for the backward;
// with a z gate the pre-gate output y is also saved for the backward's dz.
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

// kVarBC: B and C are both variable (the common case, no runtime switches).
template <typename IT, int SPL, bool kVarBC>
__global__ __launch_bounds__(kThreads) void ss_fwd_kernel(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float tr_buf[kWaves * 2 * kTrWave];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int64_t nblk = (p.dim + kChPerWG - 1) / kChPerWG;
    const int64_t b = blockIdx.x / nblk;
    const int64_t c_raw = (blockIdx.x % nblk) * kChPerWG + w * kRows + j;
    const bool cval = c_raw < p.dim;
    const int64_t c = cval ? c_raw : p.dim - 1;
    const int64_t g = c / p.dpg;
    const int N = int(p.dstate);
    const int64_t L = p.seqlen;
    float* wbuf = tr_buf + w * 2 * kTrWave;

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    // without a z gate zp aliases u so that its (unused) load stays unconditional
    const IT* zp = p.has_z ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : u;
    IT* out = static_cast<IT*>(p.out) + b * p.o_bs + c * p.o_ds;
    IT* ysave = (p.has_z && p.y) ? static_cast<IT*>(p.y) + b * p.y_bs + c * p.y_ds : nullptr;
    const IT* Bv_base = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* Cv_base = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    const float* Bc_base = static_cast<const float*>(p.B) + c * p.B_gs;  // constant B: (dim, dstate)
    const float* Cc_base = static_cast<const float*>(p.C) + c * p.C_gs;
    float* xrow = p.x + (b * p.dim + c) * p.n_chunks * N;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;

    float A2[SPL], Bc[SPL], Cc[SPL], h[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        A2[s] = nv ? p.A[c * p.A_ds + n * p.A_ns] * kLog2e : 0.f;
        Bc[s] = (!p.var_B && nv) ? Bc_base[n * p.B_ns] : 0.f;
        Cc[s] = (!p.var_C && nv) ? Cc_base[n * p.C_ns] : 0.f;
        h[s] = 0.f;
    }

    // Inputs of one 16-step tile: the per-step values of step t0 + r owned by
    // this lane, and (single state group) the B / C rows of this lane's state.
    struct Tile {
        float u, dl, z;
        float B[kT], C[kT];
    };
    // Padding states (n >= dstate, only when dstate % 16 != 0) read a valid
    // row and get C = 0, so their h never reaches y or x.
    const bool pad_states = (N % 16) != 0;
    auto load_bc = [&](int64_t t0, int s, float (&Bo)[kT], float (&Co)[kT]) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        const int nn = nv ? n : N - 1;
        if (kVarBC || p.var_B) load_tile16<IT>(Bv_base + nn * p.B_ns, t0, L, p.vec_B != 0, Bo);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Bo[k] = Bc[s];
        }
        if (kVarBC || p.var_C) load_tile16<IT>(Cv_base + nn * p.C_ns, t0, L, p.vec_C != 0, Co);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = Cc[s];
        }
        if (pad_states && !nv) {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = 0.f;
        }
    };
    // Loads are unconditional (addresses clamped inside the sequence past its
    // end), so prefetches beyond the last tile are harmless.
    auto load_tile = [&](int64_t t0, Tile& T) {
        const int64_t t = t0 + r;
        if (t0 + kT <= L) {
            T.u = load_at(u, t);
            T.dl = load_at(dl, t);
            T.z = load_at(zp, t);
        } else {
            T.u = load_or0(u, t, L);
            T.dl = load_or0(dl, t, L);
            T.z = load_or0(zp, t, L);
        }
        if constexpr (SPL == 1) load_bc(t0, 0, T.B, T.C);
    };
    // The sum over states of a tile is written to LDS at the end of the tile
    // and read back in the middle of the next one, so its latency overlaps
    // that tile's arithmetic; two scratch slots alternate.  (The slot is
    // applied as an offset to the __shared__ array itself: a pointer picked
    // from an array of pointers would lose its LDS address space and turn
    // into slow flat loads.)
    int64_t pend_t = -1;          // step of the pending output (this lane), -1 if none
    float pend_u = 0.f, pend_z = 0.f;
    auto finish_pending = [&](int slot) {
        if (pend_t < 0) return;
        const float y = row_transpose_read(wbuf + slot * kTrWave, j, r);
        if (pend_t < L && cval) {
            float o = y + Dv * pend_u;
            if (p.has_z) {
                if (ysave) io<IT>::store(ysave + pend_t, o);
                o *= pend_z * sigmoidf_(pend_z);
            }
            io<IT>::store(out + pend_t, o);
        }
    };

    auto compute_tile = [&](int64_t t0, Tile& T, int slot) {
        float dt = T.dl + bias;
        if (p.softplus) dt = softplus20(dt);
        if (t0 + r >= L) dt = 0.f;               // identity step: a = 1, b = 0
        const float dtu = dt * T.u;

        float yp[kT];
#pragma unroll
        for (int k = 0; k < kT; ++k) yp[k] = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            float Bl[kT], Cl[kT];
            if constexpr (SPL > 1) load_bc(t0, s, Bl, Cl);
            const float (&Bt)[kT] = (SPL == 1) ? T.B : Bl;
            const float (&Ct)[kT] = (SPL == 1) ? T.C : Cl;
            const float a2 = A2[s];
            // decay factors and inputs of all 16 steps first: they do not
            // depend on h, so the exp latency is off the h chain
            float a[kT], bb[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                a[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
                bb[k] = row_bcast<k>(dtu) * Bt[k];
            });
            if (s == 0) finish_pending(slot ^ 1);
            float hs = h[s];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                hs = __builtin_fmaf(a[k], hs, bb[k]);
                yp[k] = __builtin_fmaf(Ct[k], hs, yp[k]);
            });
            h[s] = hs;
            const bool chunk_end = ((t0 + kT) % kChunk == 0) || (t0 + kT >= L);
            if (chunk_end && cval && n < N) xrow[(t0 / kChunk) * N + n] = hs;
        }
        row_transpose_write(wbuf + slot * kTrWave, yp, j, r);
        pend_t = t0 + r;
        pend_u = T.u;
        pend_z = T.z;
    };

    // two tile buffers, alternated by unrolling the time loop twice: the
    // loads of a tile are issued one tile before it is computed
    Tile T0, T1;
    load_tile(0, T0);
    int slot = 0;
    for (int64_t t0 = 0; t0 < L; t0 += 2 * kT) {
        load_tile(t0 + kT, T1);
        compute_tile(t0, T0, slot);
        slot ^= 1;
        load_tile(t0 + 2 * kT, T0);
        if (t0 + kT < L) { compute_tile(t0 + kT, T1, slot); slot ^= 1; }
    }
    finish_pending(slot ^ 1);
}

// Fast path: dstate 16, variable B and C with 16-byte aligned rows, seqlen a
// multiple of 32, dim a multiple of 16, z gate fixed at compile time.  Every
// step, state and channel is real, so the loop body has no branch around a
// memory access.  That matters on gfx950: loads and stores share one
// in-order counter (vmcnt), and after a branch that contains memory accesses
// the compiler waits for all of them (vmcnt(0)), which would also wait for
// the loads prefetched for the next tile.
template <typename IT, bool kZ>
__global__ __launch_bounds__(kThreads, 3) void ss_fwd_fast(const FwdParams p) {
    // 16-byte chunks per 16-step row of B / C: 4 for fp32, 2 for 16-bit types
    constexpr int CPR = (kT * int(sizeof(IT))) / 16;
    __shared__ __attribute__((aligned(16))) float tr_buf[kWaves * kTrWave];
    // per wave: one staged tile of B and C, 1 KB each
    __shared__ __attribute__((aligned(16))) float bc_buf[kWaves * 2 * 256];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int64_t nblk = p.dim / kChPerWG;
    const int64_t b = blockIdx.x / nblk;
    const int64_t c = (blockIdx.x % nblk) * kChPerWG + w * kRows + j;
    const int64_t g = c / p.dpg;
    const int64_t L = p.seqlen;
    float* wbuf = tr_buf + w * kTrWave;
    float* bcw = bc_buf + w * 2 * 256;

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    const IT* zp = kZ ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : u;
    IT* out = static_cast<IT*>(p.out) + b * p.o_bs + c * p.o_ds;
    IT* ysave = kZ ? static_cast<IT*>(p.y) + b * p.y_bs + c * p.y_ds : out;
    float* xrow = p.x + (b * p.dim + c) * p.n_chunks * kT;

    // B / C tiles are staged through LDS: every lane fetches the 16-byte chunk
    // of its LDS slot (see tile_slot) with a coalesced load, 4 lanes per
    // 64-byte state row segment; for 16-bit types lanes 0-31 fetch B and lanes
    // 32-63 fetch C.  Each lane then reads its own state row from LDS.
    const IT* Bbase = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* Cbase = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    const IT* stage_src_B;
    const IT* stage_src_C;
    {
        int n, i;
        if constexpr (CPR == 4) {
            tile_slot_inv<4>(lane, n, i);
            stage_src_B = Bbase + n * p.B_ns + 4 * i;
            stage_src_C = Cbase + n * p.C_ns + 4 * i;
        } else {
            tile_slot_inv<2>(lane & 31, n, i);
            stage_src_B = lane < 32 ? Bbase + n * p.B_ns + 8 * i : Cbase + n * p.C_ns + 8 * i;
            stage_src_C = stage_src_B;
        }
    }
    // coalesced fetch of this lane's 16-byte chunk of the tile (kept in
    // registers until the tile is computed), then a float4 write to its LDS slot
    struct Chunks { uint4 b, c; };
    auto fetch_bc = [&](int64_t t0, Chunks& F) {
        F.b = *reinterpret_cast<const uint4*>(stage_src_B + t0);
        if constexpr (CPR == 4) F.c = *reinterpret_cast<const uint4*>(stage_src_C + t0);
    };
    auto stage_bc = [&](const Chunks& F) {
        uint4* dst = reinterpret_cast<uint4*>(bcw);
        dst[lane] = F.b;
        if constexpr (CPR == 4) dst[64 + lane] = F.c;
    };
    // this lane's state row r of the staged tile, as float
    auto read_bc = [&](float (&Bo)[kT], float (&Co)[kT]) {
        const float* src = bcw;
        if constexpr (CPR == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 vb = *reinterpret_cast<const float4*>(src + 4 * tile_slot<4>(r, i));
                const float4 vc = *reinterpret_cast<const float4*>(src + 256 + 4 * tile_slot<4>(r, i));
                Bo[4 * i] = vb.x; Bo[4 * i + 1] = vb.y; Bo[4 * i + 2] = vb.z; Bo[4 * i + 3] = vb.w;
                Co[4 * i] = vc.x; Co[4 * i + 1] = vc.y; Co[4 * i + 2] = vc.z; Co[4 * i + 3] = vc.w;
            }
        } else {
            const IT* s16 = reinterpret_cast<const IT*>(src);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float tb[8], tc[8];
                load8_16(s16 + 8 * tile_slot<2>(r, i), tb);
                load8_16(s16 + 256 + 8 * tile_slot<2>(r, i), tc);
#pragma unroll
                for (int k = 0; k < 8; ++k) { Bo[8 * i + k] = tb[k]; Co[8 * i + k] = tc[k]; }
            }
        }
    };

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;
    const int64_t t_last = L - kT;

    struct Step {
        float u, dl, z;
        Chunks bc;
    };
    // the prefetch past the last tile re-reads the last tile
    auto load_step = [&](int64_t t0, Step& S) {
        const int64_t tc = t0 < t_last ? t0 : t_last;
        S.u = load_at(u, tc + r);
        S.dl = load_at(dl, tc + r);
        S.z = kZ ? load_at(zp, tc + r) : 0.f;
        fetch_bc(tc, S.bc);
    };
    float h = 0.f;
    auto compute_tile = [&](int64_t t0, const Step& S) {
        float Bt[kT], Ct[kT];
        stage_bc(S.bc);
        read_bc(Bt, Ct);
        const float pre = S.dl + bias;
        const float dt = softplus ? softplus20(pre) : pre;
        const float dtu = dt * S.u;
        // decay factors and inputs of all 16 steps first: they do not depend
        // on h, so the exp latency stays off the h chain
        float a[kT], bb[kT], yp[kT];
        static_for<kT>([&](auto K) {
            constexpr int k = decltype(K)::value;
            a[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
            bb[k] = row_bcast<k>(dtu) * Bt[k];
        });
        static_for<kT>([&](auto K) {
            constexpr int k = decltype(K)::value;
            h = __builtin_fmaf(a[k], h, bb[k]);
            yp[k] = Ct[k] * h;
        });
        xrow[(t0 / kT) * kT + r] = h;
        row_transpose_write(wbuf, yp, j, r);
        float y = row_transpose_read(wbuf, j, r) + Dv * S.u;
        if constexpr (kZ) {
            io<IT>::store(ysave + t0 + r, y);
            y *= S.z * sigmoidf_(S.z);
        }
        io<IT>::store(out + t0 + r, y);
    };

    Step S0, S1;
    load_step(0, S0);
    for (int64_t t0 = 0; t0 < L; t0 += 2 * kT) {
        load_step(t0 + kT, S1);
        compute_tile(t0, S0);
        load_step(t0 + 2 * kT, S0);
        compute_tile(t0 + kT, S1);
    }
}

bool fwd_fast_ok(const FwdParams& p) {
    return p.dstate == 16 && p.var_B && p.var_C && p.vec_B && p.vec_C && p.seqlen >= 32 &&
           p.seqlen % 32 == 0 && p.dim % kChPerWG == 0 && (!p.has_z || p.y != nullptr);
}

template <typename IT>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
    const int64_t nblk = (p.dim + kChPerWG - 1) / kChPerWG;
    const dim3 grid(unsigned(nblk * p.batch));
    const dim3 block(kThreads);
    const int spl = int((p.dstate + 15) / 16);
    const bool vbc = p.var_B && p.var_C;
    if (fwd_fast_ok(p)) {
        if (p.has_z) hipLaunchKernelGGL((ss_fwd_fast<IT, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((ss_fwd_fast<IT, false>), grid, block, 0, stream, p);
    } else if (spl <= 1) {
        if (vbc) hipLaunchKernelGGL((ss_fwd_kernel<IT, 1, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((ss_fwd_kernel<IT, 1, false>), grid, block, 0, stream, p);
    } else if (spl <= 2) hipLaunchKernelGGL((ss_fwd_kernel<IT, 2, false>), grid, block, 0, stream, p);
    else if (spl <= 4) hipLaunchKernelGGL((ss_fwd_kernel<IT, 4, false>), grid, block, 0, stream, p);
    else if (spl <= 8) hipLaunchKernelGGL((ss_fwd_kernel<IT, 8, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_fwd_kernel<IT, 16, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_fwd(const FwdParams& p, int itype, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_fwd_t<float>(p, stream);
        case SS_BF16: return launch_fwd_t<bf16_t>(p, stream);
        case SS_F16: return launch_fwd_t<_Float16>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
