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
    const int64_t blk = xcd_block_id();
    const int64_t b = blk / nblk;
    const int64_t c_raw = (blk % nblk) * kChPerWG + w * kRows + j;
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
    // x: (batch, chunk, dim, dstate)
    float* xrow = p.x + (b * p.n_chunks * p.dim + c) * N;
    const int64_t x_chunk_stride = p.dim * N;

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
            if (chunk_end && cval && n < N) xrow[(t0 / kChunk) * x_chunk_stride + n] = hs;
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

// Fast path: dstate 16, variable B and C, seqlen a multiple of 64, dim a
// multiple of 16, z gate fixed at compile time.  Every step, state and
// channel is real, so the loop body has no branch around a memory access
// (loads and stores share one in-order counter, vmcnt; after a branch that
// contains memory accesses the compiler waits for all of them, which would
// also wait for the prefetch of the next super-tile).
//
// Global traffic is workgroup-cooperative: per 64-step super-tile, each of
// the 256 threads moves one 16-byte piece of each of u, delta, z, B and C
// (16 rows x 256 contiguous bytes per array for fp32), prefetched one
// super-tile ahead in registers and staged in LDS; outputs go back the same
// way.  Lanes then read their per-step values and B / C rows from LDS.  A
// wave's checkpoint store is 4 channels x 16 states = 256 contiguous bytes.
constexpr int kS = 64;                       // steps per super-tile
constexpr int kSq = kS / kT;                 // 16-step sub-tiles per super-tile
constexpr int kStrm = kS + 16;               // LDS row stride of stream tiles (floats)
constexpr int kBCs = kS + 4;                 // LDS row stride of B / C tiles (floats)

template <typename IT>
struct Piece4 {                              // 4 consecutive elements of one row
    using raw = typename std::conditional<sizeof(IT) == 4, u32x4, u32x2>::type;
    raw v;
    __device__ __forceinline__ void load(const SS_GLOBAL IT* p) { v = *(const SS_GLOBAL raw*)p; }
    __device__ __forceinline__ float4 f() const {
        if constexpr (sizeof(IT) == 4) {
            return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
        } else if constexpr (__is_same(IT, bf16_t)) {
            return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                               __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
        } else {
            return make_float4(float(__builtin_bit_cast(_Float16, uint16_t(v.x & 0xffffu))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.x >> 16))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.y & 0xffffu))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.y >> 16))));
        }
    }
};

template <typename IT>
__device__ __forceinline__ void store4(SS_GLOBAL IT* p, float4 v) {
    if constexpr (sizeof(IT) == 4) {
        *(SS_GLOBAL f32x4*)p = f32x4{v.x, v.y, v.z, v.w};
    } else if constexpr (__is_same(IT, bf16_t)) {
        *(SS_GLOBAL u32x2*)p = u32x2{io<bf16_t>::pack2(v.x, v.y),
                                     io<bf16_t>::pack2(v.z, v.w)};
    } else {
        *(SS_GLOBAL u32x2*)p =
            u32x2{uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.x))) | (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.y))) << 16),
                  uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.z))) | (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.w))) << 16)};
    }
}

template <typename IT, bool kZ>
__global__ __launch_bounds__(kThreads, 3) void ss_fwd_fast(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float tr_buf[kWaves * kTrWave];
    // stream tiles [16 channels][64 steps] of u, delta, z; u and delta hold
    // the outputs (out, y) once every lane has read its inputs
    __shared__ __attribute__((aligned(16))) float s_u[kChPerWG * kStrm];
    __shared__ __attribute__((aligned(16))) float s_d[kChPerWG * kStrm];
    __shared__ __attribute__((aligned(16))) float s_z[kZ ? kChPerWG * kStrm : 4];
    // B / C tiles [16 states][64 steps]
    __shared__ __attribute__((aligned(16))) float s_B[16 * kBCs];
    __shared__ __attribute__((aligned(16))) float s_C[16 * kBCs];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;                 // this lane's channel row in the workgroup
    const int64_t nblk = p.dim / kChPerWG;
    const int64_t blk = xcd_block_id();
    const int64_t b = blk / nblk;
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    const int64_t L = p.seqlen;
    float* wbuf = tr_buf + w * kTrWave;

    // cooperative piece of this thread: row prow, steps 4 pc .. 4 pc + 3
    const int prow = tid >> 4, pc = tid & 15;
    // workgroup-uniform row bases plus per-thread byte offsets (below 2^32,
    // checked by fwd_fast_ok)
    const IT* gu = static_cast<const IT*>(p.u) + b * p.u_bs + c0 * p.u_ds;
    const IT* gd = static_cast<const IT*>(p.delta) + b * p.dl_bs + c0 * p.dl_ds;
    const IT* gz = kZ ? static_cast<const IT*>(p.z) + b * p.z_bs + c0 * p.z_ds : gu;
    const IT* gB = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* gC = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    IT* go = static_cast<IT*>(p.out) + b * p.o_bs + c0 * p.o_ds;
    IT* gy = kZ ? static_cast<IT*>(p.y) + b * p.y_bs + c0 * p.y_ds : go;
    constexpr uint32_t es = sizeof(IT);
    const uint32_t ou = uint32_t(prow * p.u_ds + 4 * pc) * es, od = uint32_t(prow * p.dl_ds + 4 * pc) * es;
    const uint32_t oz = kZ ? uint32_t(prow * p.z_ds + 4 * pc) * es : ou;
    const uint32_t oB = uint32_t(prow * p.B_ns + 4 * pc) * es, oC = uint32_t(prow * p.C_ns + 4 * pc) * es;
    const uint32_t oo = uint32_t(prow * p.o_ds + 4 * pc) * es;
    const uint32_t oy = kZ ? uint32_t(prow * p.y_ds + 4 * pc) * es : oo;
    const int spos = prow * kStrm + 4 * pc;        // this piece in a stream tile
    const int bpos = prow * kBCs + 4 * pc;         // this piece in a B / C tile
    // x: (batch, chunk, dim, dstate); a wave's 4 channels x 16 states are contiguous
    float* gx = p.x + (b * p.n_chunks * p.dim + c0) * kT;
    const uint32_t ox = uint32_t(row * kT + r) * 4u;
    const int64_t x_chunk_stride = p.dim * kT;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;

    struct Pieces { Piece4<IT> u, d, z, B, C; };
    auto fetch = [&](int64_t t0, Pieces& P) {   // t0 clamped by the caller
        P.u.load(goff(gbase(gu + t0), ou));
        P.d.load(goff(gbase(gd + t0), od));
        if constexpr (kZ) P.z.load(goff(gbase(gz + t0), oz));
        P.B.load(goff(gbase(gB + t0), oB));
        P.C.load(goff(gbase(gC + t0), oC));
    };
    auto stage = [&](const Pieces& P) {
        *reinterpret_cast<float4*>(s_u + spos) = P.u.f();
        *reinterpret_cast<float4*>(s_d + spos) = P.d.f();
        if constexpr (kZ) *reinterpret_cast<float4*>(s_z + spos) = P.z.f();
        *reinterpret_cast<float4*>(s_B + bpos) = P.B.f();
        *reinterpret_cast<float4*>(s_C + bpos) = P.C.f();
    };

    float h = 0.f;
    Pieces P;
    fetch(0, P);
    for (int64_t t0 = 0; t0 < L; t0 += kS) {
        lds_barrier();                 // previous super-tile's outputs have been stored
        stage(P);
        lds_barrier();
        fetch(t0 + kS < L ? t0 + kS : t0, P);      // prefetch (re-reads the last super-tile at the end)

        // per-step inputs of steps t0 + 16 q + r of this lane's channel
        float uq[kSq], dq[kSq], zq[kSq];
#pragma unroll
        for (int q = 0; q < kSq; ++q) {
            uq[q] = s_u[row * kStrm + kT * q + r];
            dq[q] = s_d[row * kStrm + kT * q + r];
            zq[q] = kZ ? s_z[row * kStrm + kT * q + r] : 0.f;
        }
        lds_barrier();                 // s_u / s_d are reused for the outputs below

#pragma unroll
        for (int q = 0; q < kSq; ++q) {
            float Bt[kT], Ct[kT];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 vb = *reinterpret_cast<const float4*>(s_B + r * kBCs + kT * q + 4 * i);
                const float4 vc = *reinterpret_cast<const float4*>(s_C + r * kBCs + kT * q + 4 * i);
                Bt[4 * i] = vb.x; Bt[4 * i + 1] = vb.y; Bt[4 * i + 2] = vb.z; Bt[4 * i + 3] = vb.w;
                Ct[4 * i] = vc.x; Ct[4 * i + 1] = vc.y; Ct[4 * i + 2] = vc.z; Ct[4 * i + 3] = vc.w;
            }
            const float pre = dq[q] + bias;
            const float dt = softplus ? softplus20(pre) : pre;
            const float dtu = dt * uq[q];
            // decay factors and inputs of all 16 steps first: they do not
            // depend on h, so the exp latency stays off the h chain
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
            *goff(gbase(gx + ((t0 + kT * q) / kT) * x_chunk_stride), ox) = h;
            row_transpose_write(wbuf, yp, j, r);
            float y = row_transpose_read(wbuf, j, r) + Dv * uq[q];
            if constexpr (kZ) {
                s_d[row * kStrm + kT * q + r] = y;
                y *= zq[q] * sigmoidf_(zq[q]);
            }
            s_u[row * kStrm + kT * q + r] = y;
        }
        lds_barrier();
        store4<IT>(goff(gbase(go + t0), oo), *reinterpret_cast<const float4*>(s_u + spos));
        if constexpr (kZ) store4<IT>(goff(gbase(gy + t0), oy), *reinterpret_cast<const float4*>(s_d + spos));
    }
}

bool fwd_fast_ok(const FwdParams& p) {
    return p.dstate == 16 && p.var_B && p.var_C && p.seqlen >= kS && p.seqlen % kS == 0 &&
           p.dim % kChPerWG == 0 && p.dpg % kChPerWG == 0 && p.stream_vec && (!p.has_z || p.y != nullptr) &&
           small_strides({p.seqlen, p.u_ds, p.dl_ds, p.z_ds, p.o_ds, p.y_ds, p.B_ns, p.C_ns});
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

const char* fwd_kernel_name(const FwdParams& p) { return fwd_fast_ok(p) ? "ss_fwd_fast" : "ss_fwd_kernel"; }

hipError_t launch_fwd(const FwdParams& p, int itype, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_fwd_t<float>(p, stream);
        case SS_BF16: return launch_fwd_t<bf16_t>(p, stream);
        case SS_F16: return launch_fwd_t<_Float16>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
