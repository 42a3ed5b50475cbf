// Single-token decode on gfx950: the selective-scan state update and the
// causal conv1d state update.
//
// The reference has no decode path (CausalLM.generate is a stub,
// models/causal_lm.py:61-62); these kernels advance the recurrences that the
// scan (forward_kernel.cu:216-293) and the block's conv
// (modules/mamba_simple.py:40-47,100-101) compute over a whole sequence by
// one step, from a state kept between steps:
//
//   conv:  state <- (state[1:], x);  out = act(bias + sum_k w[k] * state[k])
//   scan:  delta' = softplus(delta + bias);  h[n] <- exp(delta' A[n]) h[n] + delta' x B[n]
//          y = sum_n C[n] h[n] + D x;  out = y * silu(z)
//
// One thread per (batch, channel): a decode step touches B * D * (N + a few)
// values, so the launch is small and latency-bound; the state row of a
// channel (N fp32) is read and written with 16-byte accesses when it is
// contiguous and aligned.  The exp is computed as exp2(delta' * A * log2 e)
// and the softplus with the threshold at 20, as in the scan kernels.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

// v rounded to IT and back to float (round to nearest even)
template <typename IT>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (sizeof(IT) == 4) return v;
    else if constexpr (__is_same(IT, bf16_t)) return __uint_as_float(uint32_t(io<bf16_t>::round(v)) << 16);
    else return float(_Float16(v));
}

namespace {

// threads per workgroup: a decode launch is bound by the cache lines each
// compute unit fetches (a unit has a limited number of misses in flight),
// so small workgroups spread a step's lines over more units
constexpr int kDT = 64;

// The 16 bytes of v as 16 / sizeof(IT) floats.
template <typename IT>
__device__ __forceinline__ void unpack16(const uint4 v, float (&o)[16 / sizeof(IT)]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(IT) == 4) {
            o[i] = __uint_as_float(w[i]);
        } else if constexpr (__is_same(IT, bf16_t)) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        } else {
            o[2 * i] = float(__builtin_bit_cast(_Float16, uint16_t(w[i] & 0xffffu)));
            o[2 * i + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[i] >> 16)));
        }
    }
}

// kN16: dstate 16 with contiguous, 16-byte aligned state and A rows (the
// host checks): the state, A, B and C of the channel are requested before
// the delta dot product, so the thread waits for memory twice instead of
// once per group of 4 states; the arithmetic and its order are those of the
// general path.
template <typename IT, bool kN16>
__global__ __launch_bounds__(kDT) void state_update_kernel(const ss_state_update_args a, bool vec, bool lowvec,
                                                          bool bcvec) {
    const int64_t i = int64_t(blockIdx.x) * kDT + threadIdx.x;
    if (i >= a.batch * a.dim) return;                   // no barrier in this kernel
    const int64_t b = i / a.dim, d = i % a.dim;
    const int64_t g = d / (a.dim / a.n_groups);
    const IT* Bp = static_cast<const IT*>(a.B) + b * a.B_batch_stride + g * a.B_group_stride;
    const IT* Cp = static_cast<const IT*>(a.C) + b * a.C_batch_stride + g * a.C_group_stride;
    const float* Ap = a.A + d * a.A_dim_stride;
    float* h = a.state + b * a.state_batch_stride + d * a.state_dim_stride;
    float hv[16], av[16], bv[16], cv[16];
    if constexpr (kN16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 h4 = *reinterpret_cast<const float4*>(h + 4 * q);
            const float4 a4 = *reinterpret_cast<const float4*>(Ap + 4 * q);
            hv[4 * q] = h4.x, hv[4 * q + 1] = h4.y, hv[4 * q + 2] = h4.z, hv[4 * q + 3] = h4.w;
            av[4 * q] = a4.x, av[4 * q + 1] = a4.y, av[4 * q + 2] = a4.z, av[4 * q + 3] = a4.w;
        }
        if (bcvec) {                                    // B, C rows contiguous and 16-byte aligned
            constexpr int E = 16 / int(sizeof(IT));
#pragma unroll
            for (int q = 0; q < 16 / E; ++q) {
                float bq[E], cq[E];
                unpack16<IT>(reinterpret_cast<const uint4*>(Bp)[q], bq);
                unpack16<IT>(reinterpret_cast<const uint4*>(Cp)[q], cq);
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    bv[q * E + e] = bq[e];
                    cv[q * E + e] = cq[e];
                }
            }
        } else {
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                bv[n] = io<IT>::load(Bp + n * a.B_dstate_stride);
                cv[n] = io<IT>::load(Cp + n * a.C_dstate_stride);
            }
        }
    }
    const IT* xs = static_cast<const IT*>(a.x);
    const IT* dts = static_cast<const IT*>(a.delta);
    const float x = io<IT>::load(xs + b * a.x_batch_stride + d * a.x_dim_stride);
    float dt;
    if (a.delta_low) {                                  // delta = delta_low[b, :] . delta_weight[d, :]
        const IT* lo = static_cast<const IT*>(a.delta_low) + b * a.delta_low_batch_stride;
        const IT* wr = static_cast<const IT*>(a.delta_weight) + d * a.delta_weight_dim_stride;
        float s0 = 0.f, s1 = 0.f;
        int64_t r = 0;
        if (lowvec) {                                   // both rows contiguous, 16-byte aligned, whole vectors
            constexpr int E = 16 / int(sizeof(IT));
            const uint4* lo4 = reinterpret_cast<const uint4*>(lo);
            const uint4* wr4 = reinterpret_cast<const uint4*>(wr);
            for (int64_t q = 0; q < a.delta_rank / E; ++q) {
                float lv[E], wv[E];
                unpack16<IT>(lo4[q], lv);
                unpack16<IT>(wr4[q], wv);
#pragma unroll
                for (int e = 0; e < E; e += 2) {
                    s0 = __builtin_fmaf(lv[e], wv[e], s0);
                    s1 = __builtin_fmaf(lv[e + 1], wv[e + 1], s1);
                }
            }
            r = a.delta_rank;
        }
        for (; r + 1 < a.delta_rank; r += 2) {
            s0 = __builtin_fmaf(io<IT>::load(lo + r * a.delta_low_rank_stride),
                                io<IT>::load(wr + r * a.delta_weight_rank_stride), s0);
            s1 = __builtin_fmaf(io<IT>::load(lo + (r + 1) * a.delta_low_rank_stride),
                                io<IT>::load(wr + (r + 1) * a.delta_weight_rank_stride), s1);
        }
        if (r < a.delta_rank)
            s0 = __builtin_fmaf(io<IT>::load(lo + r * a.delta_low_rank_stride),
                                io<IT>::load(wr + r * a.delta_weight_rank_stride), s0);
        // rounded to the element type, as the forward's delta is: there it is
        // the output of the block's delta projection, a GEMM in that type
        dt = round_to<IT>(s0 + s1);
    } else {
        dt = io<IT>::load(dts + b * a.delta_batch_stride + d * a.delta_dim_stride);
    }
    if (a.has_delta_bias) dt += a.delta_bias[d];
    if (a.delta_softplus) dt = softplus20(dt);
    const float dtx = dt * x;

    float y = 0.f;
    if constexpr (kN16) {
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            const float dA = __builtin_amdgcn_exp2f(dt * av[n] * kLog2e);
            hv[n] = __builtin_fmaf(dA, hv[n], dtx * bv[n]);
            y = __builtin_fmaf(cv[n], hv[n], y);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4*>(h + 4 * q) = make_float4(hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]);
    } else if (vec) {                                          // state, A rows contiguous and 16-byte aligned
        for (int64_t n = 0; n < a.dstate; n += 4) {
            float4 hv = *reinterpret_cast<const float4*>(h + n);
            const float4 av = *reinterpret_cast<const float4*>(Ap + n);
            float hn[4] = {hv.x, hv.y, hv.z, hv.w};
            const float an[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float dA = __builtin_amdgcn_exp2f(dt * an[k] * kLog2e);
                hn[k] = __builtin_fmaf(dA, hn[k], dtx * io<IT>::load(Bp + (n + k) * a.B_dstate_stride));
                y = __builtin_fmaf(io<IT>::load(Cp + (n + k) * a.C_dstate_stride), hn[k], y);
            }
            hv = make_float4(hn[0], hn[1], hn[2], hn[3]);
            *reinterpret_cast<float4*>(h + n) = hv;
        }
    } else {
        for (int64_t n = 0; n < a.dstate; ++n) {
            float* hp = h + n * a.state_dstate_stride;
            const float dA = __builtin_amdgcn_exp2f(dt * Ap[n * a.A_dstate_stride] * kLog2e);
            const float hn = __builtin_fmaf(dA, *hp, dtx * io<IT>::load(Bp + n * a.B_dstate_stride));
            *hp = hn;
            y = __builtin_fmaf(io<IT>::load(Cp + n * a.C_dstate_stride), hn, y);
        }
    }
    if (a.has_D) y = __builtin_fmaf(a.D[d], x, y);
    if (a.has_z) {
        const float z = io<IT>::load(static_cast<const IT*>(a.z) + b * a.z_batch_stride + d * a.z_dim_stride);
        y *= z * sigmoidf_(z);
    }
    io<IT>::store(static_cast<IT*>(a.out) + b * a.out_batch_stride + d * a.out_dim_stride, y);
}

template <typename IT>
__global__ __launch_bounds__(kDT) void conv_update_kernel(const ss_conv1d_update_args a) {
    const int64_t i = int64_t(blockIdx.x) * kDT + threadIdx.x;
    if (i >= a.batch * a.dim) return;                   // no barrier in this kernel
    const int64_t b = i / a.dim, d = i % a.dim;
    const int W = int(a.width);
    IT* st = static_cast<IT*>(a.conv_state) + b * a.state_batch_stride + d * a.state_dim_stride;
    float s[4];
    for (int k = 0; k < W - 1; ++k) s[k] = io<IT>::load(st + (k + 1) * a.state_width_stride);
    s[W - 1] = io<IT>::load(static_cast<const IT*>(a.x) + b * a.x_batch_stride + d * a.x_dim_stride);
    float acc = a.has_bias ? a.bias[d] : 0.f;
    for (int k = 0; k < W; ++k) {
        acc = __builtin_fmaf(a.weight[d * a.w_dim_stride + k * a.w_width_stride], s[k], acc);
        io<IT>::store(st + k * a.state_width_stride, s[k]);
    }
    if (a.silu) acc *= sigmoidf_(acc);
    io<IT>::store(static_cast<IT*>(a.out) + b * a.out_batch_stride + d * a.out_dim_stride, acc);
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

hipError_t state_update_launch(const ss_state_update_args* a, hipStream_t stream) {
    const bool vec = a->dstate % 4 == 0 && a->state_dstate_stride == 1 && a->A_dstate_stride == 1 &&
                     al16(a->state) && al16(a->A) && a->state_batch_stride % 4 == 0 &&
                     a->state_dim_stride % 4 == 0 && a->A_dim_stride % 4 == 0;
    const int64_t es = a->itype == SS_F32 ? 4 : 2;
    const bool lowvec = a->delta_low && a->delta_low_rank_stride == 1 && a->delta_weight_rank_stride == 1 &&
                        al16(a->delta_low) && al16(a->delta_weight) && (a->delta_low_batch_stride * es) % 16 == 0 &&
                        (a->delta_weight_dim_stride * es) % 16 == 0 && (a->delta_rank * es) % 16 == 0;
    const bool bcvec = a->B_dstate_stride == 1 && a->C_dstate_stride == 1 && al16(a->B) && al16(a->C) &&
                       (a->B_batch_stride * es) % 16 == 0 && (a->B_group_stride * es) % 16 == 0 &&
                       (a->C_batch_stride * es) % 16 == 0 && (a->C_group_stride * es) % 16 == 0;
    const dim3 grid{unsigned((a->batch * a->dim + kDT - 1) / kDT)};
    if (vec && a->dstate == 16) {
        switch (a->itype) {
            case SS_F32: hipLaunchKernelGGL((state_update_kernel<float, true>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
            case SS_BF16: hipLaunchKernelGGL((state_update_kernel<bf16_t, true>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
            case SS_F16: hipLaunchKernelGGL((state_update_kernel<_Float16, true>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (a->itype) {
        case SS_F32: hipLaunchKernelGGL((state_update_kernel<float, false>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
        case SS_BF16: hipLaunchKernelGGL((state_update_kernel<bf16_t, false>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
        case SS_F16: hipLaunchKernelGGL((state_update_kernel<_Float16, false>), grid, dim3(kDT), 0, stream, *a, vec, lowvec, bcvec); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t conv_update_launch(const ss_conv1d_update_args* a, hipStream_t stream) {
    const dim3 grid{unsigned((a->batch * a->dim + kDT - 1) / kDT)};
    switch (a->itype) {
        case SS_F32: hipLaunchKernelGGL((conv_update_kernel<float>), grid, dim3(kDT), 0, stream, *a); break;
        case SS_BF16: hipLaunchKernelGGL((conv_update_kernel<bf16_t>), grid, dim3(kDT), 0, stream, *a); break;
        case SS_F16: hipLaunchKernelGGL((conv_update_kernel<_Float16>), grid, dim3(kDT), 0, stream, *a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ss
