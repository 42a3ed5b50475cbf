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

template <typename IT, int SPL>
__global__ __launch_bounds__(kThreads) void ss_fwd_kernel(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float tr_buf[kWaves * kTrWave];

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
    float* wbuf = tr_buf + w * kTrWave;

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    const IT* zp = p.has_z ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : nullptr;
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

    for (int64_t t0 = 0; t0 < L; t0 += kT) {
        const int64_t t = t0 + r;
        const bool tv = t < L;
        const int nvalid = int(L - t0 < kT ? L - t0 : kT);
        const float uu = tv ? io<IT>::load(u + t) : 0.f;
        const float dr = tv ? io<IT>::load(dl + t) : 0.f;
        float dt = dr + bias;
        if (p.softplus) dt = softplus20(dt);
        if (!tv) dt = 0.f;                       // identity step: a = 1, b = 0
        const float dtu = dt * uu;

        float yp[kT];
#pragma unroll
        for (int k = 0; k < kT; ++k) yp[k] = 0.f;

#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            const bool nv = n < N;
            float Bt[kT], Ct[kT];
            if (p.var_B) {
                load16<IT>(Bv_base + n * p.B_ns + t0, nv ? nvalid : 0, p.vec_B != 0, Bt);
            } else {
#pragma unroll
                for (int k = 0; k < kT; ++k) Bt[k] = Bc[s];
            }
            if (p.var_C) {
                load16<IT>(Cv_base + n * p.C_ns + t0, nv ? nvalid : 0, p.vec_C != 0, Ct);
            } else {
#pragma unroll
                for (int k = 0; k < kT; ++k) Ct[k] = Cc[s];
            }
            float hs = h[s];
            const float a2 = A2[s];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                const float a = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
                hs = __builtin_fmaf(a, hs, row_bcast<k>(dtu) * Bt[k]);
                yp[k] = __builtin_fmaf(Ct[k], hs, yp[k]);
            });
            h[s] = hs;
            const bool chunk_end = ((t0 + kT) % kChunk == 0) || (t0 + kT >= L);
            if (chunk_end && cval && nv) xrow[(t0 / kChunk) * N + n] = hs;
        }

        const float y = row_transpose_sum(wbuf, yp, j, r);
        if (tv && cval) {
            float o = y + Dv * uu;
            if (p.has_z) {
                if (ysave) io<IT>::store(ysave + t, o);
                const float zz = io<IT>::load(zp + t);
                o *= zz * sigmoidf_(zz);
            }
            io<IT>::store(out + t, o);
        }
    }
}

template <typename IT>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
    const int64_t nblk = (p.dim + kChPerWG - 1) / kChPerWG;
    const dim3 grid(unsigned(nblk * p.batch));
    const dim3 block(kThreads);
    const int spl = int((p.dstate + 15) / 16);
    if (spl <= 1) hipLaunchKernelGGL((ss_fwd_kernel<IT, 1>), grid, block, 0, stream, p);
    else if (spl <= 2) hipLaunchKernelGGL((ss_fwd_kernel<IT, 2>), grid, block, 0, stream, p);
    else if (spl <= 4) hipLaunchKernelGGL((ss_fwd_kernel<IT, 4>), grid, block, 0, stream, p);
    else if (spl <= 8) hipLaunchKernelGGL((ss_fwd_kernel<IT, 8>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_fwd_kernel<IT, 16>), grid, block, 0, stream, p);
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
