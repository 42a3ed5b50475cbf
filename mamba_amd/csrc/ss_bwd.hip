// Backward selective scan for gfx950.
//
// Gradients follow the reference backward kernel
// (csrc/selective_scan/backward_kernel.cu:276-585), with g the adjoint of h:
//   g_t = a_{t+1} g_{t+1} + dy_t C_t              (reverse scan, :386-431)
//   du_t = D dy_t + delta'_t sum_n g B            (:334,437-438)
//   ddelta'_t = u_t sum_n g B + sum_n A g a_t h_{t-1}   (:439-440)
//   dA += delta' g a_t h_{t-1}   dB += g delta' u   dC += dy h_t   (:441-454)
//   dD += dy u; ddelta = ddelta' sigmoid(delta + bias) below 20; dbias += ddelta
// and, for the fused z gate, dy = dout silu(z), dz = dout y silu'(z) with the
// pre-gate output y saved by the forward.
//
// Same lane layout as the forward: a lane owns one (channel, state) chain.
// Chunks of kChunk steps are visited last to first.  For each chunk the lane
// restarts the forward recurrence from the checkpoint the forward stored in
// x, keeps a_t and h_t of the chunk in registers, then runs the adjoint
// backwards over the chunk.  Per-step partial values are streamed to LDS four
// steps at a time:
//  - sums over states (sum_n g B, sum_n A g a h) are in-row transposed sums;
//  - sums over channels (dB, dC) are first reduced over the wave's 4 rows,
//    then over the workgroup's 4 waves, then added to global memory once per
//    workgroup and (state, step).
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

constexpr int kTiles = kChunk / kT;
static_assert(kChunk % kT == 0, "chunk must be a whole number of tiles");

// Per-wave transposition buffer: [row j][lane r][step k], 256 floats per row,
// 16-step rows of a lane stored as four float4 with the float4 index XORed by
// (r >> 2), so the float4 writes of a row hit 64 distinct banks.
constexpr int kArr = kRows * kT * kT;   // 1024 floats

__device__ __forceinline__ int swz(int r, int chunk4) { return r * kT + 4 * (chunk4 ^ (r >> 2)); }

template <typename IT, int SPL>
__global__ __launch_bounds__(kThreads, 2) void ss_bwd_kernel(const BwdParams q) {
    // [wave][array: s1, s2, dB, dC][kArr]
    __shared__ __attribute__((aligned(16))) float trb[kWaves * 4 * kArr];
    // [array: dB, dC][wave][state n][16 steps] (swizzled like trb rows)
    __shared__ __attribute__((aligned(16))) float wgb[2 * kWaves * kT * kT];
    const FwdParams& p = q.f;

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

    float* tr_s1 = trb + (w * 4 + 0) * kArr;
    float* tr_s2 = trb + (w * 4 + 1) * kArr;
    float* tr_dB = trb + (w * 4 + 2) * kArr;
    float* tr_dC = trb + (w * 4 + 3) * kArr;
    // streaming write position of this lane (chunk4 added per group)
    const int wrow = j * kT * kT;
    // in-row transposed sum: element (lane r', step r) of row j lives at
    // wrow + r' * 16 + 4 * ((r >> 2) ^ (r' >> 2)) + (r & 3)
    int toff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) toff[m] = wrow + 4 * ((r >> 2) ^ m) + (r & 3);

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    const IT* zp = p.has_z ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : nullptr;
    const IT* yp = p.has_z ? static_cast<const IT*>(p.y) + b * p.y_bs + c * p.y_ds : nullptr;
    const IT* dop = static_cast<const IT*>(q.dout) + b * q.do_bs + c * q.do_ds;
    IT* dup = static_cast<IT*>(q.du) + b * q.du_bs + c * q.du_ds;
    IT* ddp = static_cast<IT*>(q.ddelta) + b * q.dd_bs + c * q.dd_ds;
    IT* dzp = p.has_z ? static_cast<IT*>(q.dz) + b * q.dz_bs + c * q.dz_ds : nullptr;
    const IT* Bv_base = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* Cv_base = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    const float* Bc_base = static_cast<const float*>(p.B) + c * p.B_gs;
    const float* Cc_base = static_cast<const float*>(p.C) + c * p.C_gs;
    const float* xrow = p.x + (b * p.dim + c) * p.n_chunks * N;
    // fp32 gradient rows of variable B / C for this (batch, group): (dstate, seqlen)
    const int64_t G = p.dim / p.dpg;
    float* dBrow = q.dB + (b * G + g) * int64_t(N) * L;
    float* dCrow = q.dC + (b * G + g) * int64_t(N) * L;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;

    float A2[SPL], Av[SPL], Bc[SPL], Cc[SPL];
    float gcar[SPL], acar[SPL], dA_acc[SPL], dBc_acc[SPL], dCc_acc[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        Av[s] = nv ? p.A[c * p.A_ds + n * p.A_ns] : 0.f;
        A2[s] = Av[s] * kLog2e;
        Bc[s] = (!p.var_B && nv) ? Bc_base[n * p.B_ns] : 0.f;
        Cc[s] = (!p.var_C && nv) ? Cc_base[n * p.C_ns] : 0.f;
        gcar[s] = 0.f;      // g_{t+1} entering the chunk from the right
        acar[s] = 1.f;      // a_{t+1} entering the chunk from the right
        dA_acc[s] = 0.f;
        dBc_acc[s] = 0.f;
        dCc_acc[s] = 0.f;
    }
    float dD_acc = 0.f, db_acc = 0.f;

    for (int64_t ck = p.n_chunks - 1; ck >= 0; --ck) {
        const int64_t tb = ck * kChunk;
        // per-step inputs of step tb + 16 qq + r, one per tile of the chunk
        float uu[kTiles], dt[kTiles], dtu[kTiles], dy[kTiles], pre[kTiles], dov[kTiles], zz[kTiles];
        bool tv[kTiles];
        int nval[kTiles];
#pragma unroll
        for (int qq = 0; qq < kTiles; ++qq) {
            const int64_t t = tb + kT * qq + r;
            tv[qq] = t < L;
            const int64_t rem = L - (tb + kT * qq);
            nval[qq] = int(rem <= 0 ? 0 : (rem < kT ? rem : kT));
            uu[qq] = tv[qq] ? io<IT>::load(u + t) : 0.f;
            pre[qq] = (tv[qq] ? io<IT>::load(dl + t) : 0.f) + bias;
            dt[qq] = p.softplus ? softplus20(pre[qq]) : pre[qq];
            if (!tv[qq]) dt[qq] = 0.f;
            dtu[qq] = dt[qq] * uu[qq];
            dov[qq] = tv[qq] ? io<IT>::load(dop + t) : 0.f;
            zz[qq] = (p.has_z && tv[qq]) ? io<IT>::load(zp + t) : 0.f;
            dy[qq] = p.has_z ? dov[qq] * zz[qq] * sigmoidf_(zz[qq]) : dov[qq];
            if (!cval) dy[qq] = 0.f;     // padding channels contribute nothing
        }
        float s1_red[kTiles], s2_red[kTiles];
#pragma unroll
        for (int qq = 0; qq < kTiles; ++qq) { s1_red[qq] = 0.f; s2_red[qq] = 0.f; }

#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            const bool nv = n < N;
            const float h0 = (ck > 0 && nv) ? xrow[(ck - 1) * N + n] : 0.f;

            // ---- recompute a_t and h_t of the chunk from the checkpoint
            float Bt[kChunk], as[kChunk], hs[kChunk];
            float hcur = h0;
            const float a2 = A2[s];
            static_for<kTiles>([&](auto QQ) {
                constexpr int qq = decltype(QQ)::value;
                float tmp[kT];
                if (p.var_B) {
                    load16<IT>(Bv_base + n * p.B_ns + tb + kT * qq, nv ? nval[qq] : 0, p.vec_B != 0, tmp);
                } else {
#pragma unroll
                    for (int k = 0; k < kT; ++k) tmp[k] = Bc[s];
                }
                static_for<kT>([&](auto K) {
                    constexpr int k = decltype(K)::value;
                    Bt[kT * qq + k] = tmp[k];
                    const float a = __builtin_amdgcn_exp2f(row_bcast<k>(dt[qq]) * a2);
                    hcur = __builtin_fmaf(a, hcur, row_bcast<k>(dtu[qq]) * tmp[k]);
                    as[kT * qq + k] = a;
                    hs[kT * qq + k] = hcur;
                });
            });

            // ---- adjoint, last step of the chunk first
            float gv = gcar[s];
            float anext = acar[s];
            const float av = Av[s];
            static_for<kTiles>([&](auto QQ) {
                constexpr int qq = kTiles - 1 - decltype(QQ)::value;
                const int64_t t0 = tb + kT * qq;
                float Ct[kT];
                if (p.var_C) {
                    load16<IT>(Cv_base + n * p.C_ns + t0, nv ? nval[qq] : 0, p.vec_C != 0, Ct);
                } else {
#pragma unroll
                    for (int k = 0; k < kT; ++k) Ct[k] = Cc[s];
                }
                float dAq = 0.f, dBq = 0.f, dCq = 0.f;
                static_for<4>([&](auto KG) {
                    constexpr int kg = 3 - decltype(KG)::value;
                    float s1p[4], s2p[4], dBp[4], dCp[4];
                    static_for<4>([&](auto KI) {
                        constexpr int ki = 3 - decltype(KI)::value;
                        constexpr int k = 4 * kg + ki;
                        constexpr int ii = kT * qq + k;
                        const float dyk = row_bcast<k>(dy[qq]);
                        gv = __builtin_fmaf(anext, gv, dyk * Ct[k]);
                        float hprev;
                        if constexpr (ii == 0) hprev = h0;
                        else hprev = hs[ii - 1];
                        const float gah = gv * (as[ii] * hprev);
                        dAq = __builtin_fmaf(row_bcast<k>(dt[qq]), gah, dAq);
                        s2p[ki] = av * gah;
                        s1p[ki] = gv * Bt[ii];
                        dBp[ki] = gv * row_bcast<k>(dtu[qq]);
                        dCp[ki] = dyk * hs[ii];
                        anext = as[ii];
                    });
                    const int o = wrow + swz(r, kg);
                    *reinterpret_cast<float4*>(tr_s1 + o) = make_float4(s1p[0], s1p[1], s1p[2], s1p[3]);
                    *reinterpret_cast<float4*>(tr_s2 + o) = make_float4(s2p[0], s2p[1], s2p[2], s2p[3]);
                    if (p.var_B) {
                        if (q.wg_reduce) {
                            *reinterpret_cast<float4*>(tr_dB + o) = make_float4(dBp[0], dBp[1], dBp[2], dBp[3]);
                        } else if (cval && nv) {
#pragma unroll
                            for (int ki = 0; ki < 4; ++ki)
                                if (4 * kg + ki < nval[qq]) atomicAdd(dBrow + n * L + t0 + 4 * kg + ki, dBp[ki]);
                        }
                    } else {
                        dBq += (dBp[0] + dBp[1]) + (dBp[2] + dBp[3]);
                    }
                    if (p.var_C) {
                        if (q.wg_reduce) {
                            *reinterpret_cast<float4*>(tr_dC + o) = make_float4(dCp[0], dCp[1], dCp[2], dCp[3]);
                        } else if (cval && nv) {
#pragma unroll
                            for (int ki = 0; ki < 4; ++ki)
                                if (4 * kg + ki < nval[qq]) atomicAdd(dCrow + n * L + t0 + 4 * kg + ki, dCp[ki]);
                        }
                    } else {
                        dCq += (dCp[0] + dCp[1]) + (dCp[2] + dCp[3]);
                    }
                });
                dA_acc[s] += dAq;
                dBc_acc[s] += dBq;
                dCc_acc[s] += dCq;

                // in-row transposed sums over states
                float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        a0 += tr_s1[toff[m] + (4 * m + i) * kT];
                        a1 += tr_s1[toff[m] + (4 * m + i + 1) * kT];
                        b0 += tr_s2[toff[m] + (4 * m + i) * kT];
                        b1 += tr_s2[toff[m] + (4 * m + i + 1) * kT];
                    }
                }
                s1_red[qq] += a0 + a1;
                s2_red[qq] += b0 + b1;

                // sums over channels: the wave's 4 rows, then the workgroup's waves
                if (q.wg_reduce && (p.var_B || p.var_C)) {
                    const int ro = swz(r, j);   // this lane sums steps 4j..4j+3 of state r
#pragma unroll
                    for (int arr = 0; arr < 2; ++arr) {
                        const bool use = arr == 0 ? p.var_B : p.var_C;
                        if (!use) continue;
                        const float* src = arr == 0 ? tr_dB : tr_dC;
                        float4 acc = *reinterpret_cast<const float4*>(src + ro);
#pragma unroll
                        for (int jj = 1; jj < kRows; ++jj) {
                            const float4 v = *reinterpret_cast<const float4*>(src + jj * kT * kT + ro);
                            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
                        }
                        *reinterpret_cast<float4*>(wgb + (arr * kWaves + w) * kT * kT + ro) = acc;
                    }
                    __syncthreads();
                    const int tid = threadIdx.x;
                    const int nl = tid >> 4, k = tid & 15;
                    const int ridx = nl * kT + 4 * ((k >> 2) ^ (nl >> 2)) + (k & 3);
                    const int ng = 16 * s + nl;
#pragma unroll
                    for (int arr = 0; arr < 2; ++arr) {
                        const bool use = arr == 0 ? p.var_B : p.var_C;
                        if (!use) continue;
                        float sum = 0.f;
#pragma unroll
                        for (int ww = 0; ww < kWaves; ++ww) sum += wgb[(arr * kWaves + ww) * kT * kT + ridx];
                        float* dst = arr == 0 ? dBrow : dCrow;
                        if (ng < N && k < nval[qq]) atomicAdd(dst + ng * L + t0 + k, sum);
                    }
                    __syncthreads();
                }
            });
            gcar[s] = gv;
            acar[s] = anext;
        }

        // ---- per-step outputs of steps tb + 16 qq + r
#pragma unroll
        for (int qq = 0; qq < kTiles; ++qq) {
            const int64_t t = tb + kT * qq + r;
            const float s1 = s1_red[qq], s2 = s2_red[qq];
            const float du = Dv * dy[qq] + dt[qq] * s1;
            const float ddt = uu[qq] * s1 + s2;
            const float dd = (p.softplus && pre[qq] <= 20.f) ? ddt * sigmoidf_(pre[qq]) : ddt;
            if (tv[qq] && cval) {
                io<IT>::store(dup + t, du);
                io<IT>::store(ddp + t, dd);
                if (p.has_z) {
                    const float sg = sigmoidf_(zz[qq]);
                    const float yv = io<IT>::load(yp + t);
                    io<IT>::store(dzp + t, dov[qq] * yv * sg * (1.f + zz[qq] * (1.f - sg)));
                }
                dD_acc += dy[qq] * uu[qq];
                db_acc += dd;
            }
        }
    }

    // ---- per-channel and per-(channel, state) sums over time and batch
    dD_acc = row_allsum(dD_acc);
    db_acc = row_allsum(db_acc);
    if (cval && r == 0) {
        if (q.dD) atomicAdd(q.dD + c, dD_acc);
        if (q.ddelta_bias) atomicAdd(q.ddelta_bias + c, db_acc);
    }
    if (cval) {
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            if (n < N) {
                atomicAdd(q.dA + c * N + n, dA_acc[s]);
                if (!p.var_B) atomicAdd(q.dB + c * N + n, dBc_acc[s]);
                if (!p.var_C) atomicAdd(q.dC + c * N + n, dCc_acc[s]);
            }
        }
    }
}

template <typename IT>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
    const int64_t nblk = (p.f.dim + kChPerWG - 1) / kChPerWG;
    const dim3 grid(unsigned(nblk * p.f.batch));
    const dim3 block(kThreads);
    const int spl = int((p.f.dstate + 15) / 16);
    if (spl <= 1) hipLaunchKernelGGL((ss_bwd_kernel<IT, 1>), grid, block, 0, stream, p);
    else if (spl <= 2) hipLaunchKernelGGL((ss_bwd_kernel<IT, 2>), grid, block, 0, stream, p);
    else if (spl <= 4) hipLaunchKernelGGL((ss_bwd_kernel<IT, 4>), grid, block, 0, stream, p);
    else if (spl <= 8) hipLaunchKernelGGL((ss_bwd_kernel<IT, 8>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_bwd_kernel<IT, 16>), grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd(const BwdParams& p, int itype, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_bwd_t<float>(p, stream);
        case SS_BF16: return launch_bwd_t<bf16_t>(p, stream);
        case SS_F16: return launch_bwd_t<_Float16>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
